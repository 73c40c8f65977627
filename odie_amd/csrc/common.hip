// Thread-local error slot shared by every C-ABI entry point, plus odie_error/odie_copy.
#include <map>
#include <mutex>
#include <vector>

#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {

std::string& error_slot() {
    static thread_local std::string slot;
    return slot;
}

int fail(const std::string& message) {
    error_slot() = message;
    return -1;
}

int check_launch(const char* what) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return fail(std::string(what) + ": " + hipGetErrorString(status));
    return 0;
}

int fail_code(const std::string& message, hipError_t code) {
    error_slot() = message;
    return static_cast<int>(code);
}

int launch_code(const char* what) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return fail_code(std::string(what) + ": " + hipGetErrorString(status), status);
    return 0;
}

void* workspace(size_t bytes, hipStream_t stream) {
    static std::mutex lock;
    static std::map<int, std::pair<void*, size_t>> buffers;
    // Outgrown buffers stay allocated until the process ends: queued kernels and captured
    // graphs may still hold their addresses.
    static std::vector<void*> retired;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        fail("workspace: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(lock);
    auto& slot = buffers[device];
    if (slot.first && slot.second >= bytes) return slot.first;
    (void)stream;
    size_t size = slot.first ? (bytes > 2 * slot.second ? bytes : 2 * slot.second) : bytes + bytes / 4;
    size = (size + (size_t{2} << 20) - 1) / (size_t{2} << 20) * (size_t{2} << 20);
    void* pointer = nullptr;
    const hipError_t status = hipMalloc(&pointer, size);
    if (status != hipSuccess) {
        fail(std::string("workspace: hipMalloc failed: ") + hipGetErrorString(status));
        return nullptr;
    }
    if (slot.first) retired.push_back(slot.first);
    slot = {pointer, size};
    return pointer;
}

}  // namespace odie

ODIE_API const char* odie_error(void) { return odie::error_slot().c_str(); }

ODIE_API int odie_copy(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream) {
    if (bytes == 0) return 0;
    if (!dst || !src) return odie::fail("odie_copy: null pointer");
    const hipError_t status = hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), bytes,
                                             hipMemcpyDeviceToDevice, odie::as_stream(stream));
    if (status != hipSuccess) return odie::fail(std::string("odie_copy: ") + hipGetErrorString(status));
    return 0;
}
