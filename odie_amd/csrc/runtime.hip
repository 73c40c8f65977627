// The native training-step runtime: the odie_* C ABI of the reference's Probe
// (odie/native/runtime.cu:163-331, bound by odie/native_backend.py:32-44), built on this
// library's kernels.  One handle owns every work buffer, the fp16 weight copies, the
// gradients and the Adam state, all allocated at create for batches of up to 65536 ids; a step
// allocates nothing and only launches work on the handle's stream, so it can be captured in a
// graph once a few eager steps have sized the library's workspace.
//
// The reference fixes the level count L (2..20), the row of raw features (RAW = sum of the
// levels' feature counts, padded to W = align16(RAW) with columns of 1) and G = align16(L) gate
// outputs at compile time (odie/native/runtime.cu:17-18, odie/build.py:26-30); here they come
// from the settings and the descriptors, and every buffer is sized from them at create.
//
// Step (odie/native/runtime.cu:246-312):
//   ids -> xy and packed RGB8 targets                       input_batch          (:30-38)
//   packed planes (active prefix, visibility) or hash grid  query / GridEncoding (:39-52,260)
//   router gate (when a gate is given)                      parallel_gate        (:64-76)
//   decoder forward, loss, backward                         (:270-273, :53-63)
//   gate backward -> grid upstream                          (:77-92, :99-103)
//   grid backward + Adam (hash grid: fused)                 (:281-305)
//   gate / decoder Adam                                     (:306-310)
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

#include "adam.h"
#include "grid.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kBatch = 65536;
constexpr int kMinLevels = 2, kMaxLevels = 20;   // odie/native/runtime.cu:18
constexpr int kMaxRow = 80;                       // align16(20 levels x 4 features)

int align16(int value) { return (value + 15) / 16 * 16; }
int64_t decoder_params(int row) { return int64_t{64} * row + 64 * 64 + 64 * 16; }      // odie/config.py:176
int64_t gate_params(int row, int levels) { return int64_t{32} * row + int64_t{32} * align16(levels); }

// ---------------------------------------------------------------------------------------------
// Settings: the flat JSON objects the reference's NativeOptimizer writes (numbers, booleans,
// strings, one nested object "hash_encoding").  Numbers keep their text so that 64-bit device
// addresses are read exactly.

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool flag = false;
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> fields;

    const Json* find(const std::string& key) const {
        for (const auto& f : fields)
            if (f.first == key) return &f.second;
        return nullptr;
    }
    const Json& at(const std::string& key) const {
        const Json* j = find(key);
        if (!j) throw std::runtime_error("missing setting: " + key);
        return *j;
    }
    double number() const {
        if (kind == Bool) return flag ? 1.0 : 0.0;
        if (kind != Number) throw std::runtime_error("expected a number");
        return std::strtod(text.c_str(), nullptr);
    }
    uint64_t u64() const {
        if (kind != Number) throw std::runtime_error("expected an integer");
        if (text.find_first_of(".eE") != std::string::npos) return static_cast<uint64_t>(number());
        return std::strtoull(text.c_str(), nullptr, 10);
    }
    int64_t i64() const {
        if (kind != Number) throw std::runtime_error("expected an integer");
        if (text.find_first_of(".eE") != std::string::npos) return static_cast<int64_t>(number());
        return std::strtoll(text.c_str(), nullptr, 10);
    }
};

struct Reader {
    const char* p;
    void space() {
        while (*p == ' ' || *p == '\n' || *p == '\t' || *p == '\r') ++p;
    }
    [[noreturn]] void error(const char* what) { throw std::runtime_error(std::string("settings JSON: ") + what); }
    std::string string() {
        if (*p != '"') error("expected a string");
        ++p;
        std::string out;
        while (*p && *p != '"') {
            if (*p == '\\') {
                ++p;
                if (!*p) error("unterminated escape");
                out.push_back(*p == 'n' ? '\n' : *p == 't' ? '\t' : *p);
                ++p;
            } else {
                out.push_back(*p++);
            }
        }
        if (*p != '"') error("unterminated string");
        ++p;
        return out;
    }
    Json value() {
        space();
        Json j;
        if (*p == '{') {
            j.kind = Json::Object;
            ++p;
            space();
            if (*p == '}') { ++p; return j; }
            while (true) {
                space();
                std::string key = string();
                space();
                if (*p != ':') error("expected ':'");
                ++p;
                j.fields.emplace_back(key, value());
                space();
                if (*p == ',') { ++p; continue; }
                if (*p == '}') { ++p; return j; }
                error("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            j.kind = Json::Array;
            ++p;
            space();
            if (*p == ']') { ++p; return j; }
            while (true) {
                j.items.push_back(value());
                space();
                if (*p == ',') { ++p; continue; }
                if (*p == ']') { ++p; return j; }
                error("expected ',' or ']'");
            }
        }
        if (*p == '"') { j.kind = Json::String; j.text = string(); return j; }
        if (!std::strncmp(p, "true", 4)) { j.kind = Json::Bool; j.flag = true; p += 4; return j; }
        if (!std::strncmp(p, "false", 5)) { j.kind = Json::Bool; p += 5; return j; }
        if (!std::strncmp(p, "null", 4)) { p += 4; return j; }
        const char* start = p;
        if (*p == '-' || *p == '+') ++p;
        while ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+') ++p;
        if (p == start) error("unexpected character");
        j.kind = Json::Number;
        j.text.assign(start, p);
        return j;
    }
};

Json parse(const char* text) {
    if (!text) throw std::runtime_error("settings JSON is null");
    Reader r{text};
    Json j = r.value();
    r.space();
    if (*r.p) r.error("trailing characters");
    if (j.kind != Json::Object) r.error("expected an object");
    return j;
}

template <class T> T* device_pointer(const Json& j, const char* key) { return reinterpret_cast<T*>(j.at(key).u64()); }

void hip(hipError_t status, const char* what) {
    if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

void call(int status) {
    if (status) throw std::runtime_error(error_slot());
}

// ---------------------------------------------------------------------------------------------

// ids -> xy and targets (odie/native/runtime.cu:30-38): x = fp32(id % W) * fp32(1/(W-1)), y
// likewise; an RGB8 image gives the pixel's bytes packed r | g << 8 | b << 16 (the decoder scales
// them by 1/255), an fp32 image its three values.  Ids past the image clamp to its last row, so
// every read stays inside the image and the planes (the reference reads past them).  The same
// launch clears `clear` [count] (the packed backward's gradient, which it then only adds into),
// so that the step takes no launch of its own for that.
__global__ __launch_bounds__(256) void batch_input_kernel(const int64_t* ids, int n, uint32_t width, uint32_t height,
                                                          float rx, float ry, const void* rgb, int rgb8, float* xy,
                                                          uint32_t* colors, float* target, float* clear, int64_t count) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int64_t threads = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t j = i; j < count / 4; j += threads) reinterpret_cast<float4*>(clear)[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t j = count / 4 * 4 + i; j < count; j += threads) clear[j] = 0.0f;
    if (i >= n) return;
    const uint32_t id = static_cast<uint32_t>(ids[i]);
    const uint32_t x = id % width, y = min(id / width, height - 1);
    xy[2 * i] = __fmul_rn(static_cast<float>(x), rx);
    xy[2 * i + 1] = __fmul_rn(static_cast<float>(y), ry);
    const uint64_t pixel_id = static_cast<uint64_t>(y) * width + x;
    if (rgb8) {
        const uint8_t* pixel = static_cast<const uint8_t*>(rgb) + 3 * pixel_id;
        colors[i] = pixel[0] | (uint32_t(pixel[1]) << 8) | (uint32_t(pixel[2]) << 16);
    } else {
        const float* pixel = static_cast<const float*>(rgb) + 3 * pixel_id;
        target[3 * i] = pixel[0];
        target[3 * i + 1] = pixel[1];
        target[3 * i + 2] = pixel[2];
    }
}

__global__ __launch_bounds__(256) void cast_half_kernel(const float* in, uint16_t* out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) out[i] = half_to_bits(__float2half_rn(in[i]));
}

// Columns [from, row) of every row of raw features set to fp16 1.0, the padding the decoder and
// gate read past the levels' features (odie/native/runtime.cu:51).
__global__ __launch_bounds__(256) void pad_columns_kernel(uint16_t* rows, int n, int row, int from) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int per = row - from;
    if (i < static_cast<int64_t>(n) * per) rows[(i / per) * row + from + i % per] = 0x3C00;
}

// Sets *flag when any word of [begin, end) of the three state arrays is nonzero.
__global__ __launch_bounds__(256) void any_state_kernel(const float* m, const float* v, const uint32_t* steps,
                                                        int64_t begin, int64_t end, int* flag) {
    for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < end;
         i += static_cast<int64_t>(gridDim.x) * 256)
        if (__float_as_uint(m[i]) | __float_as_uint(v[i]) | steps[i]) *flag = 1;
}

template <class T> struct DeviceBuffer {
    T* data = nullptr;
    size_t count = 0;
    void allocate(size_t n) {
        count = n;
        hip(hipMalloc(reinterpret_cast<void**>(&data), (n ? n : 1) * sizeof(T)), "hipMalloc");
    }
    void zero(hipStream_t s) { hip(hipMemsetAsync(data, 0, count * sizeof(T), s), "hipMemsetAsync"); }
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() {
        if (data) (void)hipFree(data);
    }
};

struct AdamState {
    DeviceBuffer<float> m, v;
    DeviceBuffer<uint32_t> steps;
    void allocate(size_t n, hipStream_t s) {
        m.allocate(n);
        v.allocate(n);
        steps.allocate(n);
        m.zero(s);
        v.zero(s);
        steps.zero(s);
    }
};

// An MLP head (gate or decoder): caller-owned fp32 master weights, the fp16 copy the kernels
// read, the weight gradient and tiny-cuda-nn Adam state (odie/native/runtime.cu:151-162).
struct Head {
    float* master = nullptr;
    int64_t count = 0;
    DeviceBuffer<uint16_t> half;
    DeviceBuffer<float> grad;
    AdamState adam;
    float lr = 0.0f;
    Head(float* weights, int64_t params, hipStream_t s) : master(weights), count(params) {
        if (!master || reinterpret_cast<uintptr_t>(master) % 16)
            throw std::runtime_error("head weights must be non-null and 16-byte aligned");
        half.allocate(count);
        grad.allocate(count);
        adam.allocate(count, s);
    }
};

constexpr float kBeta1 = 0.9f, kBeta2 = 0.999f, kEpsilon = 1e-15f;   // odie/native/runtime.cu:159,212

struct Runtime {
    hipStream_t stream;
    int64_t total;
    int width, height, mode;
    bool hash, rgb8 = true, half_grads, fused;
    const void* rgb;
    float* grid;                      // caller-owned fp32 master
    int levels = 0;                   // L
    int raw_width = 0, row = 0;       // RAW = sum of the levels' features, W = align16(RAW)
    std::vector<int32_t> features;    // F of each level (the descriptors' column 5)
    bool levels16x2 = false;          // 16 levels x 2 features in level order (the forward's fast path)
    bool pairs = false;               // 2 features per level but the last (1 or 2): rows of fp16 pairs
    int active = 0, coarse = 0, softplus = 0;
    float grid_lr = 0.0f;
    // packed planes (odie/model.py:100-101)
    const int32_t* desc = nullptr;
    const uint64_t* bits = nullptr;
    const int32_t* prefix = nullptr;
    const uint8_t* cells = nullptr;
    // hash grid
    std::vector<odie_grid_level> hash_levels;
    DeviceBuffer<uint16_t> grid_half;
    // work buffers, B = 65536 rows
    DeviceBuffer<float> xy, target, squares, sigmoid, grid_grad;
    DeviceBuffer<uint32_t> colors;
    DeviceBuffer<uint16_t> raw, weighted, dz, upstream, output;
    DeviceBuffer<uint8_t> vis;
    DeviceBuffer<int> flag;
    AdamState grid_adam;
    std::unique_ptr<Head> gate, decoder;

    explicit Runtime(const Json& j);
    void configure(const Json& j);
    void read_shape(const int32_t* descriptors);
    void sync_weights();
    void step(const int64_t* ids, int n, bool update);
    std::string pointers() const;
    std::string state(int64_t begin, int64_t end);
};

// HashGrid levels from the encoding settings, with the rounding points of odie/config.py:83-94.
std::vector<odie_grid_level> hash_grid_levels(const Json& e, int64_t& entries) {
    const int levels = static_cast<int>(e.at("n_levels").i64());
    const int features = static_cast<int>(e.at("n_features_per_level").i64());
    const int log2t = static_cast<int>(e.at("log2_hashmap_size").i64());
    const int base = static_cast<int>(e.at("base_resolution").i64());
    const float growth = static_cast<float>(e.at("per_level_scale").number());
    if (levels < kMinLevels || levels > kMaxLevels) throw std::runtime_error("HashGrid levels must be within 2..20");
    if (features != 1 && features != 2 && features != 4) throw std::runtime_error("HashGrid features per level must be 1, 2 or 4");
    if (log2t < 3 || log2t > 30 || base < 2 || !(growth > 1.0f) || !std::isfinite(growth))
        throw std::runtime_error("invalid hash_encoding");
    const float log_growth = static_cast<float>(std::log2(static_cast<double>(growth)));
    std::vector<odie_grid_level> rows(levels);
    entries = 0;
    for (int l = 0; l < levels; ++l) {
        const float exponent = static_cast<float>(static_cast<double>(l) * static_cast<double>(log_growth));
        const float power = static_cast<float>(std::pow(2.0, static_cast<double>(exponent)));
        const float product = power * static_cast<float>(base);   // rounded to fp32 before the subtraction
        const float scale = product - 1.0f;
        const uint32_t resolution = static_cast<uint32_t>(std::ceil(static_cast<double>(scale))) + 1;
        const uint64_t dense = (static_cast<uint64_t>(resolution) * resolution + 7) / 8 * 8;
        const uint64_t size = dense < (uint64_t{1} << log2t) ? dense : (uint64_t{1} << log2t);
        rows[l] = {scale, resolution, static_cast<uint32_t>(size), static_cast<uint32_t>(entries),
                   static_cast<uint32_t>(static_cast<uint64_t>(resolution) * resolution > size)};
        entries += static_cast<int64_t>(size);
    }
    return rows;
}

Runtime::Runtime(const Json& j)
    : stream(reinterpret_cast<hipStream_t>(j.at("stream").u64())),
      total(j.at("total").i64()),
      width(static_cast<int>(j.at("width").i64())),
      height(static_cast<int>(j.at("height").i64())),
      mode(static_cast<int>(j.at("mode").i64())),
      hash(j.find("hash_encoding") != nullptr),
      half_grads((mode & 4) != 0),
      fused((mode & 1) != 0),
      rgb(device_pointer<const void>(j, "rgb")),
      grid(device_pointer<float>(j, "grid")) {
    if (total <= 0 || total >= (int64_t{1} << 31) || width < 2 || height < 2 ||
        static_cast<int64_t>(width) * height > (int64_t{1} << 32))
        throw std::runtime_error("invalid total, width or height");
    if (!rgb || !grid) throw std::runtime_error("null rgb or grid");
    if (reinterpret_cast<uintptr_t>(grid) % 16) throw std::runtime_error("grid must be 16-byte aligned");
    // compile-time specializations of the reference library (odie/build.py:26-30), here settings:
    // levels (ODIE_LEVELS), raw_width (ODIE_RAW_WIDTH, checked against the levels' features),
    // rgb8, gate_coarse_levels, router_activation
    if (const Json* k = j.find("rgb8")) rgb8 = k->number() != 0.0;
    if (const Json* k = j.find("gate_coarse_levels")) coarse = static_cast<int>(k->i64());
    if (const Json* a = j.find("router_activation")) {
        if (a->text != "sigmoid" && a->text != "softplus")
            throw std::runtime_error("router_activation must be sigmoid or softplus");
        softplus = a->text == "softplus";
    }
    const bool router = j.find("gate") != nullptr;
    if (router && !(mode & 16)) throw std::runtime_error("the router gate is built as the parallel gate (mode bit 16)");
    if (router && fused && !hash)
        throw std::runtime_error("mode bit 1 with the router on packed planes is not built (NativeOptimizer uses 16 and 20)");
    if (hash) {
        if (!(mode & 4)) throw std::runtime_error("HashGrid requires native half gradients");
        const Json& e = j.at("hash_encoding");
        int64_t entries = 0;
        hash_levels = hash_grid_levels(e, entries);
        levels = static_cast<int>(hash_levels.size());
        if (const Json* k = j.find("levels"); k && k->i64() != levels)
            throw std::runtime_error("levels differs from the grid's level count");
        features.assign(levels, static_cast<int32_t>(e.at("n_features_per_level").i64()));
        if (entries * features[0] != total) throw std::runtime_error("HashGrid allocation differs from resolved layout");
        grid_half.allocate(total);
    } else {
        const Json* k = j.find("levels");
        if (!k) throw std::runtime_error("levels is required with packed planes (the reference fixes it at build time)");
        levels = static_cast<int>(k->i64());
        if (levels < kMinLevels || levels > kMaxLevels) throw std::runtime_error("levels must be within 2..20");
    }
    if (coarse < 0 || coarse > levels) throw std::runtime_error("gate_coarse_levels must be within 0..levels");
    if (const Json* k = j.find("raw_width"); k && (k->i64() < levels || k->i64() > kMaxRow))
        throw std::runtime_error("raw_width must be within levels..80");
    // settings are checked; the packed planes' feature row is read from the device descriptors
    if (!hash) read_shape(device_pointer<const int32_t>(j, "descriptors"));
    raw_width = 0;
    for (int32_t f : features) raw_width += f;
    if (const Json* k = j.find("raw_width"); k && k->i64() != raw_width)
        throw std::runtime_error("raw_width differs from the levels' features");
    row = align16(raw_width);
    if (row > kMaxRow) throw std::runtime_error("the levels' features exceed 80 columns");
    levels16x2 = levels == 16 && row == 32 && raw_width == 32;
    pairs = !features.empty() && (features.back() == 1 || features.back() == 2);
    for (size_t l = 0; l + 1 < features.size(); ++l) pairs = pairs && features[l] == 2;
    xy.allocate(2 * kBatch);
    if (!rgb8) target.allocate(3 * kBatch);
    colors.allocate(kBatch);
    squares.allocate(kBatch);
    raw.allocate(static_cast<size_t>(row) * kBatch);
    dz.allocate(static_cast<size_t>(row) * kBatch);
    output.allocate(16 * static_cast<size_t>(kBatch));
    vis.allocate(static_cast<size_t>(levels) * kBatch);
    flag.allocate(1);
    grid_grad.allocate(total);
    grid_grad.zero(stream);
    grid_adam.allocate(total, stream);
    decoder.reset(new Head(device_pointer<float>(j, "decoder"), decoder_params(row), stream));
    if (router) {
        gate.reset(new Head(device_pointer<float>(j, "gate"), gate_params(row, levels), stream));
        weighted.allocate(static_cast<size_t>(row) * kBatch);
        sigmoid.allocate(static_cast<size_t>(levels) * kBatch);
        upstream.allocate(static_cast<size_t>(row) * kBatch);
    }
    if (hash) hip(hipMemsetAsync(vis.data, 1, vis.count, stream), "hipMemsetAsync");
    configure(j);
    sync_weights();
    hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

// Per-level feature counts from the packed-plane descriptors (odie/model.py:100-101): F in
// {1, 2, 4}, output columns the running sum in level order (the gate and decoder read them so).
// The first call fixes the row layout; later descriptors (new supports) must keep it.
void Runtime::read_shape(const int32_t* d) {
    if (!d) throw std::runtime_error("null packed-plane pointer");
    std::vector<int32_t> host(8 * static_cast<size_t>(levels));
    hip(hipMemcpyAsync(host.data(), d, host.size() * 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    std::vector<int32_t> f(levels);
    int offset = 0;
    for (int l = 0; l < levels; ++l) {
        f[l] = host[8 * l + 5];
        if (f[l] != 1 && f[l] != 2 && f[l] != 4) throw std::runtime_error("plane features must be 1, 2 or 4");
        if (host[8 * l + 6] != offset) throw std::runtime_error("plane features must fill the row in level order");
        offset += f[l];
    }
    if (!features.empty() && f != features) throw std::runtime_error("the descriptors change the feature row");
    features = f;
}

void Runtime::configure(const Json& j) {
    const int a = static_cast<int>(j.at("active").i64());
    if (a < 2 || a > levels) throw std::runtime_error("Invalid active prefix");
    const float glr = static_cast<float>(j.at("grid_lr").number());
    const float dlr = static_cast<float>(j.at("decoder_lr").number());
    const float wlr = gate ? static_cast<float>(j.at("gate_lr").number()) : 0.0f;
    if (!hash) {
        const int32_t* d = device_pointer<const int32_t>(j, "descriptors");
        const uint64_t* b = device_pointer<const uint64_t>(j, "node_bitmap");
        const int32_t* p = device_pointer<const int32_t>(j, "node_prefix");
        const uint8_t* c = device_pointer<const uint8_t>(j, "bitmap");
        if (!d || !b || !p || !c) throw std::runtime_error("null packed-plane pointer");
        read_shape(d);
        desc = d;
        bits = b;
        prefix = p;
        cells = c;
    }
    active = a;
    grid_lr = glr;
    decoder->lr = dlr;
    if (gate) gate->lr = wlr;
}

void Runtime::sync_weights() {
    if (hash) cast_half_kernel<<<static_cast<uint32_t>((total + 255) / 256), 256, 0, stream>>>(grid, grid_half.data, total);
    for (Head* h : {gate.get(), decoder.get()})
        if (h) cast_half_kernel<<<static_cast<uint32_t>((h->count + 255) / 256), 256, 0, stream>>>(h->master, h->half.data, h->count);
    call(check_launch("odie_sync_weights"));
}

// One tiny-cuda-nn Adam step (variant 1: grid, zero gradients skipped; 2: heads) on gradients
// stored in fp16 as the reference's buffers hold them, divided by `divisor` in fp16 first.
AdamStep make_step(float* master, uint16_t* half_copy, AdamState& s, int variant, float lr, float loss_scale,
                   float divisor) {
    AdamStep a;
    call(make_adam_step("odie_step", master, half_copy, s.m.data, s.v.data, s.steps.data, variant, 1, lr, kBeta1,
                        kBeta2, kEpsilon, loss_scale, true, a));
    a.half_divisor = divisor;
    return a;
}

void Runtime::step(const int64_t* ids, int n, bool update) {
    if (n <= 0 || n > kBatch) throw std::runtime_error("Invalid native batch size");
    if (!ids) throw std::runtime_error("null ids");
    const uint64_t s = reinterpret_cast<uint64_t>(stream);
    const float rx = static_cast<float>(1.0 / static_cast<double>(width - 1));
    const float ry = static_cast<float>(1.0 / static_cast<double>(height - 1));
    // the packed backward adds into a gradient cleared here (its owner form writes every value)
    const bool clear = !hash;
    batch_input_kernel<<<(n + 255) / 256, 256, 0, stream>>>(ids, n, width, height, rx, ry, rgb, rgb8, xy.data,
                                                            colors.data, target.data, clear ? grid_grad.data : nullptr,
                                                            clear ? total : 0);
    call(check_launch("odie_step: batch input"));
    if (hash) {
        call(odie_grid_forward(xy.data, n, nullptr, 1, grid_half.data, total, ODIE_F16, hash_levels.data(), levels,
                               features[0], raw.data, row, s));
        if (raw_width < row) {
            const int64_t cells_to_pad = static_cast<int64_t>(n) * (row - raw_width);
            pad_columns_kernel<<<static_cast<uint32_t>((cells_to_pad + 255) / 256), 256, 0, stream>>>(raw.data, n, row,
                                                                                                      raw_width);
            call(check_launch("odie_step: padding columns"));
        }
    } else {
        call(packed_forward_internal(xy.data, n, grid, total, desc, levels, bits, prefix, cells, row, active, 0x3C00,
                                     raw.data, vis.data, stream, levels16x2, pairs));
    }
    const uint16_t* inputs = raw.data;
    if (gate) {
        call(odie_gate_forward(raw.data, n, row, levels, features.data(), gate->half.data, vis.data, coarse, softplus,
                               weighted.data, sigmoid.data, s));
        inputs = weighted.data;
    }
    call(odie_mlp_train(inputs, n, row, n, decoder->half.data, rgb8 ? colors.data : nullptr, nullptr, nullptr,
                        rgb8 ? nullptr : target.data, nullptr, output.data, nullptr, squares.data, dz.data,
                        decoder->grad.data, s));
    const uint16_t* up = dz.data;
    if (gate) {
        call(odie_gate_backward(raw.data, dz.data, n, row, levels, features.data(), gate->half.data, vis.data,
                                sigmoid.data, coarse, softplus, upstream.data, gate->grad.data, s));
        up = upstream.data;
    }
    // grid: fp16 gradients (mode bit 4) carrying the loss scale 128 (odie/native/runtime.cu:298,304-305)
    const float grid_divisor = half_grads ? 1.0f : 0.0f;
    AdamSet sets[kAdamSegments];   // the optimizer steps left for one launch at the end
    int pending = 0;
    if (hash && update) {
        const AdamStep a = make_step(grid, grid_half.data, grid_adam, 1, grid_lr, 128.0f, grid_divisor);
        call(grid_backward_adam_internal(xy.data, n, nullptr, 1, up, ODIE_F16, row, total, hash_levels.data(), levels,
                                         features[0], a, stream));
    } else if (hash) {
        call(odie_grid_backward(xy.data, n, nullptr, 1, up, ODIE_F16, row, total, hash_levels.data(), levels,
                                features[0], grid_grad.data, 1, s));
    } else {
        call(packed_backward_internal(xy.data, n, up, row, desc, levels, bits, prefix, cells, grid_grad.data, total,
                                      stream, clear));
        if (update)
            sets[pending++] = AdamSet{make_step(grid, nullptr, grid_adam, 1, grid_lr, 128.0f, grid_divisor),
                                      grid_grad.data, 0, total};
    }
    // heads: fp16 gradients carrying 16384, halved to 128 unless mode bit 1 (:300-303,306-309).  The
    // parameter sets are disjoint, so their updates share one launch.
    if (update) {
        for (Head* h : {gate.get(), decoder.get()})
            if (h)
                sets[pending++] = AdamSet{make_step(h->master, h->half.data, h->adam, 2, h->lr, fused ? 16384.0f : 128.0f,
                                                    fused ? 1.0f : 128.0f),
                                          h->grad.data, 0, h->count};
        call(launch_adam_sets(sets, pending, stream));
    }
}

std::string Runtime::pointers() const {
    auto field = [](const char* key, const void* p) {
        return std::string("\"") + key + "\": " + std::to_string(reinterpret_cast<uint64_t>(p));
    };
    return "{" + field("grid_grad", grid_grad.data) + ", " + field("half_grad", nullptr) + ", " +
           field("gate_grad", gate ? gate->grad.data : nullptr) + ", " + field("decoder_grad", decoder->grad.data) +
           ", " + field("output", output.data) + ", " + field("raw", raw.data) + ", " +
           field("squares", squares.data) + ", " + field("dirty_count", nullptr) + "}";
}

std::string Runtime::state(int64_t begin, int64_t end) {
    hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (begin >= 0) {
        if (end < begin || end > total) throw std::runtime_error("state range outside the grid");
        int found = 0;
        hip(hipMemsetAsync(flag.data, 0, sizeof(int), stream), "hipMemsetAsync");
        if (end > begin)
            any_state_kernel<<<static_cast<uint32_t>(std::min<int64_t>((end - begin + 255) / 256, 4096)), 256, 0,
                               stream>>>(grid_adam.m.data, grid_adam.v.data, grid_adam.steps.data, begin, end,
                                         flag.data);
        call(check_launch("odie_state"));
        hip(hipMemcpyAsync(&found, flag.data, sizeof(int), hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
        hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
        return found ? "{\"pristine\": false}" : "{\"pristine\": true}";
    }
    // FNV-1a 64 over the optimizer state: grid, gate, decoder, each m | v | ages
    uint64_t h = 14695981039346656037ull, bytes = 0;
    std::vector<unsigned char> host;
    auto feed = [&](const void* p, size_t n) {
        host.resize(n);
        hip(hipMemcpy(host.data(), p, n, hipMemcpyDeviceToHost), "hipMemcpy");
        for (unsigned char b : host) {
            h ^= b;
            h *= 1099511628211ull;
        }
        bytes += n;
    };
    std::vector<AdamState*> states{&grid_adam};
    if (gate) states.push_back(&gate->adam);
    states.push_back(&decoder->adam);
    for (AdamState* st : states) {
        feed(st->m.data, st->m.count * 4);
        feed(st->v.data, st->v.count * 4);
        feed(st->steps.data, st->steps.count * 4);
    }
    return "{\"hash_fnv1a64\": \"" + std::to_string(h) + "\", \"bytes\": " + std::to_string(bytes) + "}";
}

thread_local std::string reply;

template <class F> int guarded(F f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        return fail(e.what());
    }
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API void* odie_create(const char* settings) {
    try {
        return new Runtime(parse(settings));
    } catch (const std::exception& e) {
        fail(e.what());
        return nullptr;
    }
}

ODIE_API int odie_step(void* handle, uint64_t ids, int n, int update) {
    if (!handle) return fail("odie_step: null handle");
    return guarded([&] { static_cast<Runtime*>(handle)->step(reinterpret_cast<const int64_t*>(ids), n, update != 0); });
}

ODIE_API int odie_configure(void* handle, const char* settings) {
    if (!handle) return fail("odie_configure: null handle");
    return guarded([&] { static_cast<Runtime*>(handle)->configure(parse(settings)); });
}

ODIE_API const char* odie_pointers(void* handle) {
    if (!handle) {
        fail("odie_pointers: null handle");
        return nullptr;
    }
    reply = static_cast<Runtime*>(handle)->pointers();
    return reply.c_str();
}

ODIE_API const char* odie_state(void* handle, int begin, int end) {
    if (!handle) {
        fail("odie_state: null handle");
        return nullptr;
    }
    try {
        reply = static_cast<Runtime*>(handle)->state(begin, end);
        return reply.c_str();
    } catch (const std::exception& e) {
        fail(e.what());
        return nullptr;
    }
}

ODIE_API int odie_sync_weights(void* handle) {
    if (!handle) return fail("odie_sync_weights: null handle");
    return guarded([&] { static_cast<Runtime*>(handle)->sync_weights(); });
}

// No per-step context objects exist to keep alive for a captured graph: every buffer a step
// touches belongs to the handle.
ODIE_API void odie_pin_contexts(void*) {}
ODIE_API void odie_release_contexts(void*) {}

ODIE_API void odie_destroy(void* handle) {
    if (handle) {
        Runtime* r = static_cast<Runtime*>(handle);
        (void)hipStreamSynchronize(r->stream);
        delete r;
    }
}
