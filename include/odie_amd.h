/*
 * odie_amd C-ABI: the MI355X (gfx950) implementation of ODIE's sparse grid-query hot path.
 *
 * Conventions (the reference's, odie/native/runtime.cu:318-331):
 *  - every pointer argument named *_device / passed as a buffer is device memory owned by
 *    the caller unless stated otherwise; host arrays are marked "host";
 *  - streams are hipStream_t values passed as uint64_t (0 = the null stream);
 *  - functions return 0 on success and -1 on failure, leaving a message that
 *    odie_error() returns (thread-local, valid until the next failing call on the thread);
 *    selection_init, selection_chunk and score_chunk, whose reference counterparts return the
 *    CUDA runtime's error code, return the HIP runtime's instead (hipErrorInvalidValue for a
 *    refused argument, the launch's code for a failed launch), with the message set as well;
 *  - arguments are validated before any device work is queued, so a call that fails has
 *    queued nothing;
 *  - fp16 data is IEEE binary16 (uint16_t bit patterns on the host side);
 *  - odie_grid_backward, odie_grid_backward_adam(_planes), odie_mlp_train(_planes),
 *    odie_gate_backward and odie_step use one library-owned scratch buffer per device.  It
 *    grows (hipMalloc) the first time a call needs more, and outgrown buffers are kept until
 *    the process ends, so queued work and captured graphs keep valid addresses.  These calls
 *    must not run concurrently on one device (queue them on one stream, or order the
 *    streams), and a call at a new, larger size should run once before a graph captures it.
 */
#ifndef ODIE_AMD_H
#define ODIE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread.  Replaces odie_error (odie/native/runtime.cu:320). */
const char* odie_error(void);

/* Device-to-device async copy.  Replaces odie_copy (odie/native/runtime.cu:329). */
int odie_copy(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Multiresolution hash grid encode (2D), the tiny-cuda-nn GridEncoding the reference's
 * HashGrid wraps (odie/hash_grid.py:27,54; odie/native/runtime.cu:186,260,287).
 * One level of the table: entries [offset, offset+size) of one expert's table, each of
 * `features` values.  scale/resolution/size follow odie/config.py:83-94.
 * --------------------------------------------------------------------------------------- */
typedef struct odie_grid_level {
    float scale;          /* fp32 grid scale 2^(l*log2 g)*base - 1 */
    uint32_t resolution;  /* ceil(scale) + 1 vertices per side */
    uint32_t size;        /* table entries of this level: min(align8(res^2), 2^log2T) */
    uint32_t offset;      /* first entry of this level inside one expert's table */
    uint32_t hashed;      /* 1 if res^2 > size (spatial hash), else dense x + y*res */
} odie_grid_level;

#define ODIE_MAX_LEVELS 32

/* dtype codes */
#define ODIE_F32 0
#define ODIE_F16 1

/* Forward encode of n coordinates in [0,1]^2 (coords fp32 [n,2]).
 * Experts: coordinates [offsets[e], offsets[e+1]) read the table at params + e*expert_params
 * (offsets: device int32 [experts+1], nondecreasing, offsets[0]=0, offsets[experts] <= n;
 * rows from offsets[experts] on belong to no expert: zero features, and no gradient in the
 * backward entry points); experts = 1 with offsets = NULL is a single grid.
 * param_dtype ODIE_F16: fp16 table, fp16 fused multiply-add chain, fp16 output;
 * ODIE_F32: fp32 table, fp32 chain, fp32 output.  levels: host array [n_levels].
 * Output row i: level l feature c at column l*features + c of out_width >= n_levels*features
 * columns; columns past n_levels*features are written as +0.
 * Replaces tcnn.Encoding.forward (odie/hash_grid.py:54) / GridEncoding fwd
 * (odie/native/runtime.cu:260). */
int odie_grid_forward(const float* coords, int64_t n, const int32_t* offsets, int experts,
                      const void* params, int64_t expert_params, int param_dtype,
                      const odie_grid_level* levels, int n_levels, int features,
                      void* out, int out_width, uint64_t stream);

/* Backward scatter: gradient[param] (fp32, experts*expert_params) receives
 * sum over coordinates and corners of w_k * upstream, skipping zero upstream values
 * (odie/packed_kernels.cu:66-88 semantics).  upstream: [n, up_width] of up_dtype.
 * zero_first = 1 clears the gradient first (the reference returns a fresh zeroed tensor,
 * odie/packed_kernels.cu:134); 0 accumulates.
 * Replaces GridEncoding bwd (odie/native/runtime.cu:287). */
int odie_grid_backward(const float* coords, int64_t n, const int32_t* offsets, int experts,
                       const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                       const odie_grid_level* levels, int n_levels, int features,
                       float* gradient, int zero_first, uint64_t stream);

/* odie_grid_backward for features = 2 with the fp16 upstream in the layout
 * odie_mlp_train_planes writes (planes uint32 [n_levels][n], blockmax fp32
 * [ceil(n/128)][2 n_levels]) instead of rows: the same gradient, bit for bit, without
 * transposing the upstream.  expert_params must equal the levels' table size.  No counterpart
 * in the reference (the backward of odie_grid_backward_adam_planes without the optimizer step). */
int odie_grid_backward_planes(const float* coords, int64_t n, const int32_t* offsets, int experts,
                              const uint32_t* planes, const float* blockmax, int64_t expert_params,
                              const odie_grid_level* levels, int n_levels, int features,
                              float* gradient, int zero_first, uint64_t stream);

/* Encode backward fused with the optimizer step: the gradient of every table value (as
 * odie_grid_backward with zero_first = 1 computes it) is applied to master / m / v / steps /
 * half_copy by the Adam update of odie_adam_step (variant, step, lr, betas, eps, loss_scale as
 * there) where it is formed, without writing it to memory.  Bit-identical to
 * odie_grid_backward followed by odie_adam_step.  expert_params must equal the levels' table
 * size.  Replaces the grid's GridEncoding bwd + optimizer step pair of the native step
 * (odie/native/runtime.cu:287,304-305). */
int odie_grid_backward_adam(const float* coords, int64_t n, const int32_t* offsets, int experts,
                            const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                            const odie_grid_level* levels, int n_levels, int features, float* master,
                            uint16_t* half_copy, float* m, float* v, uint32_t* steps, int variant, int64_t step,
                            float lr, float beta1, float beta2, float eps, float loss_scale, uint64_t stream);

/* odie_grid_backward_adam for features = 2 with the fp16 upstream given as odie_mlp_train_planes
 * writes it (planes uint32 [n_levels][n], blockmax fp32 [ceil(n/128)][2 n_levels]) instead of rows
 * [n, up_width]: the same update, bit for bit, without transposing the upstream.  No counterpart
 * in the reference (see odie_mlp_train_planes). */
int odie_grid_backward_adam_planes(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                   const uint32_t* planes, const float* blockmax, int64_t expert_params,
                                   const odie_grid_level* levels, int n_levels, int features, float* master,
                                   uint16_t* half_copy, float* m, float* v, uint32_t* steps, int variant,
                                   int64_t step, float lr, float beta1, float beta2, float eps, float loss_scale,
                                   uint64_t stream);

/* A handoff from the encode forward to the encode backward of the same batch.  No counterpart
 * in the reference: a split of this library's owner backward, for steps that run the encode
 * forward and then the backward on the same coordinates.  From its own plan for the batch the
 * backward would form, in passes over the coordinates, either the slice masks its unbanded hashed
 * slices walk by (a byte per coordinate and such level) or the band lists its banded passes walk
 * (the coordinates sorted into 2047 y-bands per expert).  The forward can form them instead: it
 * writes the masks as it forms every corner index, or builds the lists first and then walks the
 * coordinates in band order itself, reading the tables with locality (its rows still land at
 * their own indices).  Either way the backward skips that work.
 *
 * odie_grid_handoff_bytes: the handoff buffer's bytes for this batch and grid under the current
 * tuning (0 when the backward would take nothing; -1 on invalid arguments).
 * odie_grid_forward_handoff: odie_grid_forward that also fills the handoff (handoff_bytes at
 * least odie_grid_handoff_bytes; handoff may be null when that is 0).  Same features, bit for bit.
 * odie_grid_backward_handoff / odie_grid_backward_adam_planes_handoff: odie_grid_backward /
 * odie_grid_backward_adam_planes reading that handoff instead of forming it: the same gradient
 * or update, bit for bit, when it was filled by odie_grid_forward_handoff for the same coords,
 * n, offsets, experts and levels, with no odie_set_tuning call in between. */
int64_t odie_grid_handoff_bytes(int64_t n, int experts, int64_t expert_params, const odie_grid_level* levels,
                                int n_levels, int features);
int odie_grid_forward_handoff(const float* coords, int64_t n, const int32_t* offsets, int experts,
                              const void* params, int64_t expert_params, int param_dtype,
                              const odie_grid_level* levels, int n_levels, int features, void* out, int out_width,
                              void* handoff, int64_t handoff_bytes, uint64_t stream);
int odie_grid_backward_handoff(const float* coords, int64_t n, const int32_t* offsets, int experts,
                               const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                               const odie_grid_level* levels, int n_levels, int features, float* gradient,
                               int zero_first, const void* handoff, int64_t handoff_bytes, uint64_t stream);
int odie_grid_backward_adam_planes_handoff(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                           const uint32_t* planes, const float* blockmax, int64_t expert_params,
                                           const odie_grid_level* levels, int n_levels, int features,
                                           float* master, uint16_t* half_copy, float* m, float* v, uint32_t* steps,
                                           int variant, int64_t step, float lr, float beta1, float beta2, float eps,
                                           float loss_scale, const void* handoff, int64_t handoff_bytes,
                                           uint64_t stream);

/* Launch-shape knobs of the encode kernels, for measurement sweeps; no counterpart in the
 * reference.  Keys: "forward_chunk", "backward_chunk" (coordinates per block, multiples of
 * 256; forward_chunk 0 (default) = 1024 when at least half of the table fits the forward's
 * LDS staging, else 256), "lds_bytes" (LDS budget of the backward's coarse-level accumulator, <= 160 KiB),
 * "xcd_remap" (0/1: XCD-major block order), "backward_mode" (1: owner computes, 0: atomics),
 * "banded" (the owner's fine passes walk y-band lists of the coordinates: 0 never, 1 always,
 * 2 (default) when the lists cut the estimated visits at least four times),
 * "split_target" (banded: coordinate-level visits per owner work item, 0 = automatic),
 * "owner_lds_bytes", "paired_loads" (the forward's 16-byte corner-pair loads: 0 off, 1 on,
 * 2 (default) when one expert's fp16 table is larger than 1 MB), "forward_lds_bytes", "packed_owner" (1: the packed-plane
 * backward computes each slice of the gradient in one workgroup, 0 (default): global atomics),
 * "packed_splits" (0 = automatic), "route_part" (the routes' smallest sub-chunk of ids, a power
 * of two within 64..65536, default 512; size route workspaces after setting it),
 * "route_one_scan" (1, the default: the routes scan their counts in one launch when they have at
 * most 1024 segments of 1024 counts; 0: the reduce and apply launches).  Results do
 * not depend on them beyond fp32 summation order and the owner's fixed-point scale. */
int odie_set_tuning(const char* key, int value);

/* ---------------------------------------------------------------------------------------
 * Packed xy planes (the on-demand representation), replacing the torch extension ops
 * forward/backward (odie/packed_bindings.cpp:4-12, odie/packed_kernels.cu:107-145).
 * descriptors: device int32 [levels, 8] = R, points, plane offset, node-word offset,
 * cell-bitmap byte offset, F, output feature offset, direct (odie/model.py:100-101).
 * grid: fp32 master [parameter_count]; every read is rounded to fp16.
 * --------------------------------------------------------------------------------------- */
int odie_packed_forward(const float* coords, int64_t n, const float* grid, int64_t parameter_count,
                        const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                        const int32_t* node_prefix, const uint8_t* bitmap, int width,
                        uint16_t* features, uint8_t* visibility, uint64_t stream);

/* gradient (fp32 [parameter_count]) is written whole, not accumulated, with fp32 atomics as
 * the reference does (summation order free).  With the tuning key "packed_owner" = 1 each slice
 * of it is summed by one workgroup in 64-bit fixed point instead: deterministic, each
 * contribution the fp32 product w * u rounded to 2^-30 of the largest |u| of its levels; the
 * plane offsets must then ascend with the level (the layout's order). */
int odie_packed_backward(const float* coords, int64_t n, const uint16_t* upstream, int up_width,
                         const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                         const int32_t* node_prefix, const uint8_t* bitmap, float* gradient,
                         int64_t parameter_count, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Expert routing and compaction.  No counterpart in the reference (its "routing" is a soft
 * per-level gate); built from its pieces: pixel id -> (id % W, id / W) in 32-bit
 * arithmetic and the fp32 reciprocal-multiply coordinate convention of the batch kernel
 * (odie/native/runtime.cu:30-38), and the stable ascending tie order of its rankings
 * (odie/selection.py:116).
 *
 * The W x H image is cut into regions_x x regions_y tiles with bounds
 * x0[r] = ceil(r*W/regions_x), y0[r] = ceil(r*H/regions_y); pixel (x, y) belongs to expert
 * ry*regions_x + rx with x0[rx] <= x < x0[rx+1], y0[ry] <= y < y0[ry+1].  Its local
 * coordinate is u = fp32(x - x0[rx]) * fp32(1/(tile_width-1)), v likewise.
 * Outputs, in compacted order (grouped by expert, original order inside an expert):
 *   perm[j]   index of the input id placed at slot j           (int32 [n])
 *   coords[j] local (u, v) of that id                         (fp32 [n, 2])
 *   offsets   first slot of every expert, offsets[E] = n       (int32 [E+1])
 * expert (nullable) receives each input's expert id in input order (int32 [n]).
 * colors (nullable, uint32 [n]): with rgb, colors[j] = r | g << 8 | b << 16 of the pixel
 *   (y*W + x, with y clamped as above) of slot j, read from the RGB8 image rgb [H*W][3] --
 *   the training target of the slot, gathered in slot order so each tile's bytes are read
 *   through one L2; without rgb, colors[j] = y*W + x, the pixel index itself (odie_mlp_train
 *   gathers the target from it).  rgb without colors is refused.
 * workspace: caller-owned device scratch of odie_route_workspace(n, E) bytes (-1 for n outside
 *   [0, 2^31-1] or E outside [1, 4096]).
 * --------------------------------------------------------------------------------------- */
int64_t odie_route_workspace(int64_t n, int experts);

int odie_route(const int64_t* ids, int64_t n, int width, int height, int regions_x, int regions_y,
               int32_t* expert, int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb,
               uint32_t* colors, void* workspace, int64_t workspace_bytes, uint64_t stream);

/* odie_route on a stratified draw, with the draw fused in (odie/data.py:63-80, the id of slot i
 * as odie_stratified_ids computes it): uniforms fp32 [n][2] (torch.rand's draws) in place of
 * ids, n a square power of two.  The ids are never written; perm[j] is the stratified slot
 * placed at slot j.  Same outputs, bit for bit, as odie_route on odie_stratified_ids' ids. */
int odie_route_stratified(const float* uniforms, int64_t n, int width, int height, int regions_x, int regions_y,
                          int32_t* expert, int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb,
                          uint32_t* colors, void* workspace, int64_t workspace_bytes, uint64_t stream);

/* odie_route (ids) or odie_route_stratified (uniforms; exactly one of the two non-null) with
 * only some tiles owning an expert, as the gigapixel workload allocates experts to the tiles that
 * pass a predicate under a parameter budget (the analogue of the reference's supports,
 * odie/model.py:226-257, whose cells off the support read zero features).  slots: device int32
 * [regions_x*regions_y], tile -> expert in [0, experts); any other value: the tile has no
 * expert.  Ids are grouped by their tile's expert as odie_route groups them by tile, and the ids
 * of tiles without an expert follow every expert's, in input order: offsets int32 [experts + 1]
 * holds each expert's first slot and, at offsets[experts], the first of those (they run to n).
 * Their local coordinates and colours are formed as for any id; expert (nullable) reports -1 for
 * them.  odie_grid_forward gives rows from offsets[experts] on zero features, and the backward
 * gives them no gradient.  workspace: odie_route_workspace(n, experts + 1) bytes; experts within
 * 1..4095.  No counterpart in the reference. */
int odie_route_allocated(const int64_t* ids, const float* uniforms, int64_t n, int width, int height, int regions_x,
                         int regions_y, const int32_t* slots, int experts, int32_t* expert, int32_t* perm,
                         float* coords, int32_t* offsets, const uint8_t* rgb, uint32_t* colors, void* workspace,
                         int64_t workspace_bytes, uint64_t stream);

/* odie_route without the workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  It allocates nothing: its scratch is a static device array of
 * ODIE_ROUTE_NOALLOC_BYTES (4 MiB + 64 KiB) that every GPU the library runs on holds until the
 * process ends, resolved once per device.  Calls whose odie_route_workspace(n, E) exceeds it
 * fail (-1, nothing queued): up to 2^23 ids over 64 experts, 2^21 over 256, 2^19 over 1024 and
 * 2^17 over 4096 fit (exactly: n <= 8510976, 2127360, 531456 and 132608); 2^24 ids over 64
 * experts do not.  Every call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (different streams without ordering, or several host threads) race and give wrong results.
 * Same outputs as odie_route, bit for bit. */
#define ODIE_ROUTE_NOALLOC_BYTES ((int64_t)((4 << 20) + (64 << 10)))

int odie_route_noalloc(const int64_t* ids, int64_t n, int width, int height, int regions_x, int regions_y,
                       int32_t* expert, int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb,
                       uint32_t* colors, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Residual pass.  Same name, signature and meaning as the reference's score_chunk
 * (odie/residual_cuda.cu:45-52): pixels [begin, end) of a width-wide image in raster order;
 * prediction fp32 [end-begin, 3], target uint8 (rgb8) or fp32 [end-begin, 3]; the cells of rows
 * first_y.. (active_cells of them, row-major, `resolution` per row) with column/row bounds
 * xb[resolution+1], yb[resolution+1] (device int32); totals fp64 [resolution^2] are read and
 * updated: total += (fp64(d0^2) + fp64(d1^2) + fp64(d2^2)) / 3 per pixel, d = prediction - t,
 * t = byte/255 in fp32, summed sequentially in raster order within each cell.
 * --------------------------------------------------------------------------------------- */
int score_chunk(const float* prediction, const void* target, int64_t begin, int64_t end, int width,
                int resolution, int first_y, int active_cells, const int* xb, const int* yb,
                double* totals, bool rgb8, uint64_t stream);

/* Bounds of the residual's native geometry cells (the pixel -> cell map of odie/selection.py:44-55,
 * odie/gpu_residual.py:49-62): pixel column p has x = fp32(p) / fp32(width - 1) and the cell column
 * floor(fmaf(R - 1, x, 0.5)); xb[c] (device int32 [R+1]) is the first column of cell column c and
 * xb[R] = width; yb likewise over rows.  No counterpart entry point in the reference (its host
 * computes the fp32 thresholds of the same map). */
int odie_cell_bounds(int width, int height, int resolution, int32_t* xb, int32_t* yb, uint64_t stream);

/* Top-k cells by score: ids (device int32 [k]) of the k largest scores (fp64 [n], >= 0), ties to
 * the lower id, written in ascending id order.  Ranking rule of select_mean_rank
 * (odie/selection.py:103,116) with the sign-cleared FP64 key of the GPU selector
 * (odie/native/selection_cuda.cu:14-17).  No counterpart entry point in the reference. */
int odie_topk(const double* scores, int64_t n, int64_t k, int32_t* ids, uint64_t stream);

/* B1, the mean-rank admission of select_mean_rank (odie/selection.py:108-126), on the device:
 * the R^2 cells ranked by descending score (fp64 [R^2], finite and >= 0 -- the caller checks, as
 * the reference's _validate does), ties by ascending cell id (the sign-cleared FP64 key of
 * odie_topk), each admitted in rank order when the closure nodes it adds -- its corners
 * (cell + {0, 1, R, R+1}) mod align8(R^2) not yet taken, a corner listed twice counted twice --
 * keep the running count within cap (8-aligned, at most align8(R^2)).  Writes chosen uint8 [R^2],
 * nodes uint8 [align8(R^2)] (1: taken) and stats int64 [2] = {nodes counted against the cap,
 * cells walked = R^2}.  workspace: odie_select_mean_rank_workspace(R) bytes (-1 unless
 * 1 <= R^2 <= 2^24).  No counterpart entry point in the reference (its B1 runs in numpy). */
int64_t odie_select_mean_rank_workspace(int resolution);
int odie_select_mean_rank(const double* scores, int resolution, int cap, uint8_t* chosen, uint8_t* nodes,
                          int64_t* stats, void* workspace, int64_t workspace_bytes, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * B2 exact greedy support selection on the device (odie/selection.py:129-207): free cells
 * (no new closure node) are taken first, in ascending id; otherwise the cell with the best
 * score / new-node cost over costs 1..min(4, cap-used), ties to the lower id.
 * Same names, signatures and state buffers as the reference's selector
 * (odie/native/selection_cuda.cu:208-230, bound at odie/selection_cuda.py:46-49):
 *   scores fp64 [n] (n = resolution^2, >= 0), missing int32 [n], chosen uint8 [n],
 *   nodes uint8 [points] (points = align8(n)), tree int32 [odie_selection_tree_ints(n)],
 *   stats int64 [4] = {used nodes, iterations, done, invariant error}, trace int32 [n] or null
 *   (the chosen cells in order).
 * selection_init resets the state and builds the tournament trees; host_offsets/host_sizes/
 * levels may describe the caller's fan-32 tree allocation (then it is checked to be large
 * enough) or be null/0.  selection_chunk runs up to `chunk` costly choices, each followed by
 * the free cells it creates; call it until stats[2] (done) or stats[3] (error) is set.
 * offsets/sizes/levels of selection_chunk are accepted and ignored.
 * --------------------------------------------------------------------------------------- */
int64_t odie_selection_tree_ints(int n);

int selection_init(const double* scores, int n, int points, int* missing, uint8_t* chosen, uint8_t* nodes,
                   int* tree, int64_t* stats, const int* host_offsets, const int* host_sizes, int levels,
                   uint64_t stream);

int selection_chunk(const double* scores, int n, int points, int resolution, int cap, bool normalized,
                    int* missing, uint8_t* chosen, uint8_t* nodes, int* tree, const int* offsets,
                    const int* sizes, int levels, int chunk, int64_t* stats, int* trace, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Fused Adam over n parameters: master fp32 (updated), half_copy fp16 (nullable; receives
 * fp16(master) in the same pass), grad fp32 or fp16 carrying loss_scale, moments m, v fp32.
 * variant 0: torch.optim.Adam with global step `step` (odie/optimizer.py:33-44,77-84).
 * variant 1: per-parameter ages in steps (uint32 [n]); zero gradients skip the update and keep
 * the age (the grid optimizer of odie/native/runtime.cu:212-215, odie/train.py:121-124).
 * variant 2: per-parameter ages without the zero-gradient skip (the head optimizers of
 * odie/native/runtime.cu:159-160, whose weights are matrix parameters).
 * Replaces the TCNN optimizer step calls (odie/native/runtime.cu:304-310).
 * --------------------------------------------------------------------------------------- */
int odie_adam_step(float* master, uint16_t* half_copy, const void* grad, int grad_dtype, float* m, float* v,
                   uint32_t* steps, int64_t n, int variant, int64_t step, float lr, float beta1, float beta2,
                   float eps, float loss_scale, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Decoder MLP width -> 64 -> 64 -> 16 (ReLU hidden layers, no bias, no output activation), fp16
 * weights and activations, fp32 accumulation: the decoder head of the reference (TCNN
 * FullyFusedMLP with n_input_dims W = align16(sum of the grid's features), odie/hash_grid.py:32-34,
 * odie/native/runtime.cu:17,151-162,190; forward/backward at odie/native/runtime.cu:270,273).
 * width: 16, 32, 48, 64 or 80.  weights fp16 [64*width + 5120] = W1 [64][width] | W2 [64][64] |
 * W3 [16][64], row-major [out][in] (7168 at width 32).
 *
 * odie_mlp_forward: out fp16 [n][16] = decoder(x fp16 [n][width]).
 *
 * odie_mlp_train: forward, the step's loss (loss_grad, odie/native/runtime.cu:53-63) and
 * backward in one pass.  Tile row j reads x[j]; its input row is i = rows[j] (rows null:
 * i = j).  Target of tile row j, first given source wins: with colors and rgb,
 * rgb[3*colors[j] + c] * (1/255) (colors: uint32 [n] pixel indexes, as odie_route writes them
 * without rgb); with colors alone, byte c of colors[j] * (1/255) (colors packed as odie_route
 * writes them with rgb); rgb[3*ids[i] + c] * (1/255); target[3*i + c] (fp32).
 * dy_c = fp16(fp16(2*d_c/(3*real)*128)*128) for c < 3 (zero for i >= real), d = y - t.
 * Writes dz fp16 [n][width] = fp16(fp16(dL/dx * 16384) / 128) at row j (the grid's upstream,
 * half_unscale at odie/native/runtime.cu:282), dweights fp32 [64*width + 5120] = dL/dW * 16384
 * (overwritten; deterministic), and, where non-null, out fp16 [.][16] and squares fp32 [.] at
 * input row i (squares = sum_c d_c^2 / 3), hidden fp16 [n][128] = (h1 | h2) at row j.
 * x must be 16-byte aligned, dz and out 8-byte aligned; n * width < 2^31.
 * --------------------------------------------------------------------------------------- */
int odie_mlp_forward(const uint16_t* x, int64_t n, int width, const uint16_t* weights, uint16_t* out,
                     uint64_t stream);

int odie_mlp_train(const uint16_t* x, int64_t n, int width, int64_t real, const uint16_t* weights,
                   const uint32_t* colors, const uint8_t* rgb, const int64_t* ids, const float* target,
                   const int32_t* rows, uint16_t* out, uint16_t* hidden, float* squares, uint16_t* dz,
                   float* dweights, uint64_t stream);

/* odie_mlp_train at width 32 (16 levels x 2 features) with dz written in the layout
 * odie_grid_backward_adam_planes reads instead of rows: planes uint32 [16][n] (plane l, row j = the fp16 pair of columns 2l, 2l+1 of dz row j)
 * and blockmax fp32 [ceil(n/128)][32] (record r, column 2l + f = max |dz| of feature f of level l
 * over rows 128r..128r+127; NaN if any of them is NaN).  Same values as odie_mlp_train's
 * dz, bit for bit.  No counterpart in the reference: it saves the encode backward's transposition
 * of dz, a layout change of this implementation. */
int odie_mlp_train_planes(const uint16_t* x, int64_t n, int64_t real, const uint16_t* weights,
                          const uint32_t* colors, const uint8_t* rgb, const int64_t* ids, const float* target,
                          const int32_t* rows, uint16_t* out, uint16_t* hidden, float* squares, uint32_t* planes,
                          float* blockmax, float* dweights, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Router gate (router_enabled): gate MLP width -> 32 -> G (ReLU hidden layer, no bias, fp16;
 * G = align16(levels); weights fp16 [32*width + 32*G] = Wg1 [32][width] | Wg2 [G][32], row-major
 * [out][in], odie/config.py:176) on the raw features [n][width], then parallel_gate /
 * parallel_gate_back and hash_router_gradient of the native step (odie/native/runtime.cu:64-92,
 * 99-103).  Level l owns columns [o_l, o_l + F_l) of a row: features (host int32 [levels], each
 * 1, 2 or 4; null = 2 for every level) with o_l the running sum in level order, and
 * width = align16(sum F) (16..80); levels 1..32.
 * visible: uint8 [n][levels] or null (all visible).  Levels below `coarse` have s = 1 and no
 * gate gradient; softplus selects softplus (threshold 20) instead of the sigmoid.
 *
 * odie_gate_forward: weighted [n][width] = raw * fp16(s * visible) per level (columns past the
 *   levels' features: 1), s fp32 [n][levels].
 * odie_gate_backward: value = the decoder's input gradient / 128 ([n][width] fp16, as
 *   odie_mlp_train's dz); writes the grid's upstream [n][width] = fp16(direct + fp16(d_raw / 128))
 *   (direct = 0 in columns past the levels' features) and the gate's weight gradient fp32
 *   [32*width + 32*G] (overwritten, deterministic; loss scale 16384).
 * Rows are 16-byte aligned.
 * --------------------------------------------------------------------------------------- */
int odie_gate_forward(const uint16_t* raw, int64_t n, int width, int levels, const int32_t* features,
                      const uint16_t* weights, const uint8_t* visible, int coarse, int softplus, uint16_t* weighted,
                      float* sigmoid, uint64_t stream);

int odie_gate_backward(const uint16_t* raw, const uint16_t* value, int64_t n, int width, int levels,
                       const int32_t* features, const uint16_t* weights, const uint8_t* visible, const float* sigmoid,
                       int coarse, int softplus, uint16_t* upstream, float* dweights, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Stratified sampling, the device part of stratified_batches (odie/data.py:63-80): batch (a
 * square power of two, side = sqrt(batch)) slots, slot j in stratum (j % side, j / side);
 * uniforms fp32 [batch][2] (torch.rand's draws); ids int64 [batch] =
 * clamp(trunc((u/side + stratum/side) * W)) + W * clamp(trunc((v/side + stratum_y/side) * H)),
 * fp32 arithmetic as the reference's torch expression.
 * --------------------------------------------------------------------------------------- */
int odie_stratified_ids(const float* uniforms, int batch, int width, int height, int64_t* ids, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * Fused reconstruction: the streamed full-image inference of the residual pass
 * (odie/evaluation.py:12-36, odie/gpu_residual.py:130-179, scripts/reconstruct.py:9-48), for
 * the multi-expert hash-grid model.  Pixels [begin, begin+n) in raster order (id = y*W + x,
 * 32-bit); the pixel's tile and tile coordinate follow odie_route; the tile's table slot is
 * slots[tile] (device int32 [regions_x*regions_y]; < 0 or >= experts: no expert, features 0;
 * slots null: slot = tile); the 16-level x 2-feature fp16 encode of that slot's table
 * (table + slot*expert_params, the odie_grid_forward layout) feeds the decoder (weights as in
 * odie_mlp_forward) without leaving registers.  Writes, where non-null, prediction fp32 [n][3]
 * (the decoder's first three outputs), features fp16 [n][32] and output fp16 [n][16] at row
 * id - begin: the same bits as odie_route + odie_grid_forward + odie_mlp_forward.
 * --------------------------------------------------------------------------------------- */
int odie_reconstruct(int64_t begin, int64_t n, int width, int height, int regions_x, int regions_y,
                     const int32_t* slots, int experts, const uint16_t* table, int64_t expert_params,
                     const odie_grid_level* levels, int n_levels, const uint16_t* weights, float* prediction,
                     uint16_t* features, uint16_t* output, uint64_t stream);

/* Fused reconstruction + residual: every pixel of the image predicted as odie_reconstruct does,
 * scored into per-cell fp64 totals with score_chunk's rule and order (one cell at a time, its
 * pixels in raster order), with no prediction in memory.  target: RGB8 [H*W][3]; cells are
 * [xb[cx], xb[cx+1]) x [yb[cy], yb[cy+1]) for cx, cy < resolution (device int32 [R+1]);
 * totals fp64 [R*R] are read and updated (as successive score_chunk calls over the whole image
 * leave them); squares (fp64 [R*R], nullable) receive each cell's sum of (p - byte*(1/255))^2
 * over its pixels and channels in fp64 (the mse numerator of odie/evaluation.py:25, in a
 * different summation order); prediction (fp32 [H*W][3], nullable) receives the image. */
int odie_reconstruct_scores(int width, int height, int regions_x, int regions_y, const int32_t* slots, int experts,
                            const uint16_t* table, int64_t expert_params, const odie_grid_level* levels, int n_levels,
                            const uint16_t* weights, const uint8_t* target, int resolution, const int32_t* xb,
                            const int32_t* yb, double* totals, double* squares, float* prediction, uint64_t stream);

/* ---------------------------------------------------------------------------------------
 * The native training step: the reference's Probe handle (odie/native/runtime.cu:163-331),
 * bound by NativeOptimizer (odie/native_backend.py:32-44).  Same entry points, arguments and
 * 0 / -1 + odie_error convention; one step is ids -> xy and targets, the grid query (packed
 * planes with the active prefix, or the hash grid), the router gate when "gate" is given, the
 * decoder with the loss, the gate backward, the grid backward and the three Adam updates
 * (grid: per-parameter ages, zero gradients skipped, fp16 gradients at loss scale 128; heads:
 * fp16 gradients halved to 128 as the reference's half_unscale does unless mode bit 1).
 *
 * Settings (JSON object): the reference's keys stream, total, width, height, mode (bit 4: fp16
 * grid gradients, required for the hash grid; bit 16: parallel gate, required with a gate;
 * bit 8 accepted, no effect on results), rgb, grid, decoder, gate (optional), descriptors,
 * node_bitmap, node_prefix, bitmap (packed planes), hash_encoding (optional object),
 * active, grid_lr, gate_lr, decoder_lr; and, for what the reference fixes at compile time
 * (odie/build.py:26-30): levels (L, 2..20; required with packed planes, checked against
 * hash_encoding's n_levels), raw_width (RAW = the levels' features, checked), rgb8 (1: uint8
 * image, 0: fp32 image), gate_coarse_levels (K, default 0), router_activation ("sigmoid" |
 * "softplus").  Packed planes take each level's features (1, 2 or 4, columns in level order) from
 * the descriptors; the hash grid has n_features_per_level (1, 2 or 4) per level.  The decoder
 * reads rows of W = align16(RAW) <= 80 columns (columns past RAW are 1), its weights fp32
 * [64*W + 5120]; the gate's are fp32 [32*W + 32*align16(L)] (odie/native/runtime.cu:17-18,
 * odie/config.py:175-177).
 * Every buffer is allocated at create for batches of up to 65536 ids: odie_step allocates
 * nothing and only queues work on the settings' stream (graph-capturable).
 * --------------------------------------------------------------------------------------- */

/* Replaces odie_create (odie/native/runtime.cu:321); null on failure. */
void* odie_create(const char* settings);
/* Replaces odie_step (:322): ids device int64 [n], 1 <= n <= 65536; update = 0 computes the
 * gradients without the optimizer steps. */
int odie_step(void* handle, uint64_t ids, int n, int update);
/* Replaces odie_configure (:325): active, learning rates and (packed planes) the four pointers. */
int odie_configure(void* handle, const char* settings);
/* Replaces odie_pointers (:323): JSON of the handle's buffers (squares fp32 [65536] is the one
 * NativeOptimizer reads; grid_grad holds the fp32 grid gradient x128 of the last packed step or
 * hash step without update; half_grad and dirty_count are 0: no such buffers exist here). */
const char* odie_pointers(void* handle);
/* Replaces odie_state (:324): begin >= 0: {"pristine": bool} over grid parameters [begin, end);
 * begin < 0: {"hash_fnv1a64": "...", "bytes": N}, an FNV-1a digest of every Adam state array
 * (its value is this library's own; compare digests only with digests from this library). */
const char* odie_state(void* handle, int begin, int end);
/* Replaces odie_sync_weights (:327): fp16 copies of the fp32 master weights. */
int odie_sync_weights(void* handle);
/* Replace odie_pin_contexts / odie_release_contexts (:328,326): no per-step context objects
 * exist here (every buffer belongs to the handle), so both do nothing. */
void odie_pin_contexts(void* handle);
void odie_release_contexts(void* handle);
/* Replaces odie_destroy (:330): waits for the stream, frees the handle's buffers. */
void odie_destroy(void* handle);

#ifdef __cplusplus
}
#endif

#endif /* ODIE_AMD_H */
