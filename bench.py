"""Headline benchmark: one training step of the packed 64-expert hash-grid model on 2^22 coords.

Workload (the 64-expert configuration): a synthetic 2048x1365 RGB8 image (6 octaves of value
noise plus random axis-aligned edges, seed 0) cut into 8x8 tiles, one expert per tile; every
expert is a 16-level hash grid (2 fp16 features per level, 2^16-entry tables, base
resolution 16, per-level scale 1.38): 70,745,088 parameters in one packed table, fp32 master
+ fp16 copy.  Decoder 32->64->64->16 fp16 MLP.  2^22 pixel ids uniform over the image (seed 0),
resident in HBM.

One step = route + compact the ids to their experts, encode forward [2^22, 32] fp16, decoder
forward + loss + backward (MFMA), encode backward (fp32 gradient of all 70.7M parameters),
Adam on the grid (per-parameter ages, zero gradients skipped, writes the fp16 copy) and on
the decoder.  The metric counts the step's queries per second; the roofline line reports the
dominant kernel.  The CPU baseline times the oracle's port of the same step on a bounded
sample of the same ids, on the host's cores.

Prints one JSON line.
"""
import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'hash-grid fwd+bwd queries/s and achieved HBM GB/s (% peak), 64 experts, 2^22 coords'
HBM_PEAK_GBS = 8000.0
N_COORDS = 1 << 22
WIDTH, HEIGHT, REGIONS = 2048, 1365, 8
ENCODING = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=16, base_resolution=16,
                per_level_scale=1.38)
# Algorithmic HBM bytes per query of each stage (element-level accesses, no cache reuse):
#   route            read id 8, write perm 4 + local xy 8                                = 20
#   encode_forward   xy 8 + 16 levels*4 corners*2 feats*2 B gathers + 32*2 B features    = 328
#   decoder          features 64 + perm 4 + id 8 + rgb 3, write dz 64 + squared error 4  = 147
#   encode_backward  xy 8 + upstream 64 + 16*4*2*(4 B read + 4 B write) scatter          = 1096
# and per parameter per step:
#   adam             read master, m, v, grad, age (20), write master, m, v, age (16), fp16 copy (2) = 38
#   fused into the encode backward (the gradient stays in LDS): 38 - 8                   = 30
STAGE_BYTES = {'route': 20, 'encode_forward': 328, 'decoder': 147, 'encode_backward': 1096}
ADAM_BYTES, FUSED_ADAM_BYTES = 38, 30
KERNELS = {'route': 'route_count/scan/scatter/colors kernels', 'encode_forward': 'grid_forward_kernel',
           'decoder': 'mlp_train_kernel<true> (dz as level-major planes + 128-row maxima) + mlp_reduce_kernel',
           'encode_backward': 'owner_kernel (grid Adam fused into its flush; upstream planes from the decoder)',
           'grid_adam': 'adam_kernel',
           'decoder_adam': 'adam_kernel'}


def parse():
    parser = argparse.ArgumentParser()
    parser.add_argument('--gpus', type=int, default=1)
    parser.add_argument('--steps', type=int, default=20)
    parser.add_argument('--warmup', type=int, default=3)
    parser.add_argument('--cpu-seconds', type=float, default=24.0,
                        help='approximate budget of the CPU baseline sample')
    parser.add_argument('--no-cpu', action='store_true')
    parser.add_argument('--no-native', action='store_true', help='skip the 65536-id native step measurement')
    parser.add_argument('--no-single', action='store_true', help='skip the single-expert 2^19-table fwd+bwd line')
    parser.add_argument('--no-c1', action='store_true', help='skip the single-expert fp32 forward of 2^18 coords')
    parser.add_argument('--no-literal', action='store_true',
                        help='skip the encode fwd+bwd measurement without the optimizer step')
    parser.add_argument('--single-only', action='store_true',
                        help='print only the single-expert 2^19-table fwd+bwd line (for kernel traces of it)')
    parser.add_argument('--native-steps', type=int, default=200)
    parser.add_argument('--no-reconstruction', action='store_true', help='skip the 32768^2 residual pass')
    parser.add_argument('--reconstruction-batch', type=int, default=1 << 26)
    parser.add_argument('--no-gigapixel', action='store_true', help='skip the 1024-expert 2^24-id step')
    parser.add_argument('--gigapixel-steps', type=int, default=5)
    parser.add_argument('--tune', action='append', default=[], metavar='KEY=VALUE',
                        help='odie_set_tuning before the run (repeatable), e.g. owner_masks=0')
    parser.add_argument('--copy-probe', action='store_true',
                        help='only run a plain 256 MiB device copy (calibrates FETCH_SIZE/WRITE_SIZE)')
    return parser.parse_args()


def copy_probe():
    """A plain device-to-device copy of known size: its FETCH_SIZE/WRITE_SIZE readings give the
    factor between those counters and bytes moved."""
    import torch
    src = torch.ones(64 << 20, dtype=torch.float32, device='cuda')
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_probe_bytes_each_way': src.numel() * 4}))


def cpu_baseline(image, ids, table16, master, decoder16, levels, expert_params, budget):
    """Time the oracle's port of the step on a bounded sample of the same ids: routing, encode
    forward, decoder forward/loss/backward and encode backward per query; Adam over the whole
    table once per batch, measured on a slice and scaled to the table.  On all host cores, then on
    one thread (the reference pins its CPU work to one thread, odie/runtime_env.py:10,
    odie/train.py:72); each timing is the median of five runs."""
    import numpy as np
    import oracle
    rows = [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]
    cores = len(os.sched_getaffinity(0))
    total = table16.size
    rgb = image.reshape(-1, 3)

    def per_query(count, threads):
        sample = ids[:count]
        started = time.perf_counter()
        _, perm, local, offsets = oracle.route(sample, WIDTH, HEIGHT, REGIONS, REGIONS)
        raw = oracle.hash_forward(local, table16, rows, 2, offsets=offsets, expert_params=expert_params,
                                  threads=threads)
        dz, _ = oracle.mlp_step_f32(raw, decoder16, oracle.mlp_targets(perm, rgb=rgb, ids=sample), perm, count,
                                    threads=threads)
        oracle.hash_backward_f32(local, dz, rows, 2, total, offsets=offsets, expert_params=expert_params,
                                 threads=threads)
        return time.perf_counter() - started

    def adam(count):
        p = master[:count].astype(np.float64)
        g = np.where(np.arange(count) % 3 == 0, 0.0, 1e-3)
        m, v = np.zeros(count), np.zeros(count)
        steps = np.zeros(count, dtype=np.uint32)
        started = time.perf_counter()
        oracle.adam(1, p, g, m, v, steps, 1, 1e-2, scale=128.0)
        return time.perf_counter() - started

    def median(run, *args):
        return float(np.median([run(*args) for _ in range(5)]))

    def measure(threads, seconds):
        # per-query rate from two sample sizes (the difference removes once-per-batch costs such
        # as clearing the gradient), plus the once-per-batch part itself; Adam runs on the
        # OpenMP thread count the encode calls set
        probe = 1 << 12
        per_query(probe, threads)                      # warm-up (allocations, thread pools)
        rate = probe / per_query(probe, threads)
        small = int(min(len(ids) // 2, max(probe, rate * seconds * 0.5 / 15)))
        t_small = median(per_query, small, threads)
        t_large = median(per_query, 2 * small, threads)
        marginal = max(t_large - t_small, 1e-9) / small
        fixed = max(t_small - marginal * small, 0.0)
        slice_ = 1 << 20 if threads == 1 else 1 << 22
        per_query(probe, threads)
        adam_seconds = median(adam, slice_) * total / slice_
        step_seconds = marginal * N_COORDS + fixed + adam_seconds
        return step_seconds, small

    step_seconds, small = measure(cores, budget)
    one_seconds, one_small = measure(1, budget)
    return dict(value=N_COORDS / step_seconds, unit='queries/s', cores=cores, kind='port',
                sample='first %d and %d of the 2^22 ids through route+encode fwd+decoder+encode bwd (median of 5 '
                       'each; per-query rate from the difference; OpenMP %d threads for encode and Adam, torch-CPU '
                       'fp32 for the decoder), plus Adam over a 2^22-parameter slice scaled to the %d-parameter table, '
                       'once per 2^22-query batch' % (small, 2 * small, cores, total),
                seconds_per_step=step_seconds, one_thread={
                    'value': N_COORDS / one_seconds, 'seconds_per_step': one_seconds, 'cores': 1,
                    'sample': 'first %d and %d ids, median of 5; Adam over a 2^20-parameter slice' % (one_small,
                                                                                                    2 * one_small)},
                cpu=platform.processor() or platform.machine())


# The reference's own recorded runs the native-step lines reproduce (results/**/metrics.json, RTX
# 3060): the final packed layout of DIV2K image 0036 at 16, 8 and 20 levels (resolutions, node
# caps, feature dimensions, cells allowed per level, direct levels; 954,016 parameters each) and
# the Tokyo hash-grid ablation's encoding, with the run's throughput rgb_processed_pixels /
# optimization_loop_seconds.
DIV2K_SHAPE = (1536, 2040)          # results/div2k_50/0036/odie/metrics.json:129-132 (H, W)
DIV2K_RUNS = {
    'div2k_L16': dict(  # results/div2k_50/0036/odie/metrics.json:237,767
        resolutions=[8, 11, 15, 21, 29, 40, 56, 77, 106, 147, 203, 280, 387, 534, 738, 1020],
        caps=[64, 128, 232, 448, 848, 1600, 3136, 5936, 11240, 21616, 41216, 78400, 87936, 87936, 87936, 87968],
        allowed=[64, 121, 225, 441, 841, 1600, 3136, 5929, 11236, 21609, 41209, 78400, 87044, 84261, 74770, 63937],
        direct=12, reference_pixels_per_s=157286400 / 4.524877033662051),
    'div2k_L8': dict(   # results/expert_count/L8/0036/metrics.json:179,465
        resolutions=[8, 16, 32, 64, 128, 255, 510, 1020],
        caps=[64, 256, 1024, 4096, 16384, 65032, 257712, 257712],
        allowed=[64, 256, 1024, 4096, 16384, 65025, 257237, 244883], direct=6, reference_pixels_per_s=44.0e6),
    'div2k_L20': dict(  # results/expert_count/L20/0036/metrics.json:267,1009
        resolutions=[8, 10, 13, 17, 22, 29, 37, 48, 62, 80, 103, 132, 171, 221, 285, 368, 474, 612, 790, 1020],
        caps=[64, 104, 176, 296, 488, 848, 1376, 2304, 3848, 6400, 10616, 17424, 29248, 48848, 63560, 63560, 63560,
              63560, 63560, 63584],
        allowed=[64, 100, 169, 289, 484, 841, 1369, 2304, 3844, 6400, 10609, 17424, 29241, 48841, 62401, 62602, 59646,
                 54137, 48024, 43053], direct=14, reference_pixels_per_s=27.5e6),
}
TOKYO_SHAPE = (21450, 56718)        # results/tokyo_components/no_on_demand/metrics.json:137-140
TOKYO_HASH = dict(otype='HashGrid', n_levels=16, n_features_per_level=2, log2_hashmap_size=21, base_resolution=3,
                  per_level_scale=1.8409329652786255)
TOKYO_REFERENCE = 60830515200 / 3206.4612404829822   # no_on_demand/metrics.json:239,279


def _recorded_planes(run):
    """PackedPlanes with a recorded run's resolutions, caps and F2/F1 levels; each sparse level
    selects a row-major run of its recorded cell count, shortened if needed so the closure fits
    the cap (a run's own supports come from its image's residuals and are not recorded)."""
    import torch
    from odie_amd.model import PackedPlanes, plane_closure
    levels = len(run['resolutions'])
    supports = []
    for level, (r, cap, allowed) in enumerate(zip(run['resolutions'], run['caps'], run['allowed'])):
        support = torch.zeros(r * r, dtype=torch.bool)
        if level < run['direct']:
            support[:] = True
        else:
            count = allowed
            while True:
                support[:] = False
                support[:count] = True
                if plane_closure(support, r).numel() <= cap:
                    break
                count -= r
        supports.append(support)
    config = dict(resolutions=run['resolutions'], n_levels=levels, representation='xy_planes', coarse_levels=0,
                  gate_topology='shared', gate_position='feature', initial_active_prefix=run['direct'], seed=1729,
                  feature_init_std=1e-3)
    planes = PackedPlanes(config, supports, [2] * (levels - 1) + [1], run['caps'])
    planes.set_active_prefix(levels)
    return planes


def native_steps(steps):
    """The reference's own training step (NativeOptimizer over the odie_* runtime, router on,
    sigmoid gate) at its batch of 65536 ids, each step a stratified draw (odie_stratified_ids on
    torch.rand's uniforms) and a replay of the captured step, timed together: the recorded DIV2K
    0036 packed layouts at 16, 8 and 20 levels on a synthetic 2040x1536 image, and the Tokyo
    hash-grid ablation (16 levels x 2, 2^21-entry tables) on a synthetic 56718x21450 image.
    Reported beside the headline, with the reference's whole-run figure for the same
    configuration (its training loop also draws, evaluates and selects supports)."""
    import numpy as np
    import torch
    from odie_amd import synth
    from odie_amd.config import grid_levels
    from odie_amd.decoder import Decoder
    from odie_amd.gate import Gate
    from odie_amd.native_backend import NativeModel, NativeOptimizer, make_native_optimizer
    from odie_amd.sampling import stratified_ids

    out = {}
    stream = torch.cuda.Stream()
    generator = torch.Generator(device='cuda').manual_seed(1729)

    def run_steps(optimizer, shape):
        optimizer.prepare_epoch()
        draw = lambda: stratified_ids(torch.rand((65536, 2), device='cuda', generator=generator), shape)
        for _ in range(5):
            optimizer.train_batch(draw())
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            loss = optimizer.train_batch(draw())
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps, float(loss)

    with torch.cuda.stream(stream):
        image = torch.from_numpy(synth.image(0, DIV2K_SHAPE[1], DIV2K_SHAPE[0])).cuda().contiguous()
        for name, run in DIV2K_RUNS.items():
            levels = len(run['resolutions'])
            dims = [2] * (levels - 1) + [1]
            planes = _recorded_planes(run)
            width = (sum(dims) + 15) // 16 * 16
            model = NativeModel(Decoder(seed=0, width=width), Gate(seed=1, features=dims), planes=planes)
            config = dict(representation='xy_planes', n_levels=levels, plane_feature_dimensions=dims,
                          router_enabled=True, target_storage='uint8', gate_coarse_levels_K=0,
                          router_output_activation='sigmoid', grid_lr=1e-2, gate_lr=1e-3, decoder_lr=1e-3)
            optimizer, _ = make_native_optimizer(model, image, DIV2K_SHAPE, config)
            ms, loss = run_steps(optimizer, DIV2K_SHAPE)
            optimizer.close()
            params = model.grid.numel() + model.gate.params.numel() + model.decoder.params.numel()
            out[name] = {'ms_per_step': ms, 'pixels_per_s': 65536 / (ms / 1e3), 'params': params, 'levels': levels,
                         'row_width': width, 'loss': loss,
                         'reference_pixels_per_s': run['reference_pixels_per_s'],
                         'vs_reference': 65536 / (ms / 1e3) / run['reference_pixels_per_s']}
        del image
        tokyo = synth.image_device(2, TOKYO_SHAPE[1], TOKYO_SHAPE[0]).contiguous()
        levels, entries = grid_levels(TOKYO_HASH)
        grid = torch.from_numpy(synth.table(0, 2 * entries, name='native_hash')).cuda()
        model = NativeModel(Decoder(seed=0), Gate(seed=1), grid=grid)
        config = dict(representation='hash_grid', hash_encoding=TOKYO_HASH, n_levels=16, plane_feature_dimensions=[2] * 16,
                      router_enabled=True, target_storage='uint8', gate_coarse_levels_K=0,
                      router_output_activation='sigmoid', grid_lr=1e-2, gate_lr=1e-3, decoder_lr=1e-3)
        optimizer = NativeOptimizer(model, tokyo, TOKYO_SHAPE, config, [grid])
        ms, loss = run_steps(optimizer, TOKYO_SHAPE)
        optimizer.close()
        out['tokyo_hash_grid'] = {'ms_per_step': ms, 'pixels_per_s': 65536 / (ms / 1e3), 'params': grid.numel() + 1536 + 7168,
                                  'loss': loss, 'reference_pixels_per_s': TOKYO_REFERENCE,
                                  'vs_reference': 65536 / (ms / 1e3) / TOKYO_REFERENCE}
        del tokyo
    out['batch'] = 65536
    out['steps'] = steps
    out['note'] = ('same configurations as the reference runs named in the keys (recorded layouts, sampling, router, '
                   'batch); ours times a stratified draw plus a graph replay of the step per batch; the reference '
                   'figure is its whole training loop (rgb_processed_pixels / optimization_loop_seconds on an RTX '
                   '3060), which also evaluates and selects supports between stages')
    return out


C2_ENCODING = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=19, base_resolution=16, per_level_scale=1.38)
C2_BYTES = {'forward': 328, 'backward': 1096}   # per query: xy 8 + gathers 256 + features 64; xy 8 + upstream 64 + 1024


def profiled_traffic(stage):
    """HBM bytes per launch of a stage's kernels from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (calibrated against a plain copy), or None when that stage was not profiled."""
    traffic_file = ROOT / 'profiles' / 'traffic.json'
    if not traffic_file.exists():
        return None
    entry = json.loads(traffic_file.read_text()).get(stage)
    return entry['bytes'] if entry else None


def single_expert_steps(steps):
    """The single-expert workload: one 16-level x 2-feature fp16 hash grid (2^19-entry tables,
    base 16, scale 1.38, 5,487,024 parameters), 2^22 coordinates uniform in [0,1)^2 (seed 0), an
    upstream [2^22, 32] of N(0,1) rounded to fp16; forward encode and the backward scatter into
    a zeroed fp32 gradient, timed with events on the stream they run on.  The pair goes through
    the forward-to-backward handoff (odie_grid_forward_handoff / odie_grid_backward_handoff): the
    forward builds the owner's band lists and walks the coordinates in band order, and the
    backward reads the lists instead of building them."""
    import torch
    from odie_amd import synth
    from odie_amd.config import grid_levels
    from odie_amd.encoding import grid_backward, grid_forward, grid_handoff_bytes
    levels, entries = grid_levels(C2_ENCODING)
    n = N_COORDS
    table = torch.from_numpy(synth.table(0, 2 * entries)).cuda().half()
    xy = torch.from_numpy(synth.coordinates(0, n)).cuda()
    upstream = torch.from_numpy(synth.upstream(0, n, 32)).cuda()
    out = torch.empty((n, 32), dtype=torch.float16, device='cuda')
    gradient = torch.empty(2 * entries, dtype=torch.float32, device='cuda')
    size = grid_handoff_bytes(n, levels, 2, expert_params=2 * entries)
    handoff = torch.empty(max(size, 1), dtype=torch.uint8, device='cuda') if size > 0 else None
    stream = torch.cuda.current_stream()
    for _ in range(3):
        grid_forward(xy, table, levels, 2, out=out, handoff=handoff)
        grid_backward(xy, upstream, levels, 2, expert_params=2 * entries, gradient=gradient, handoff=handoff)
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b, c in marks:
        a.record(stream)
        grid_forward(xy, table, levels, 2, out=out, handoff=handoff)
        b.record(stream)
        grid_backward(xy, upstream, levels, 2, expert_params=2 * entries, gradient=gradient, handoff=handoff)
        c.record(stream)
    torch.cuda.synchronize()
    forward = sum(a.elapsed_time(b) for a, b, _ in marks) / steps
    backward = sum(b.elapsed_time(c) for _, b, c in marks) / steps
    total = forward + backward
    gbs = lambda per, ms: n * per / (ms / 1e3) / 1e9
    stage_gbs = {'forward': gbs(C2_BYTES['forward'], forward), 'backward': gbs(C2_BYTES['backward'], backward)}
    dominant = 'backward' if backward >= forward else 'forward'
    traffic = profiled_traffic('single_expert_' + dominant)
    return {'coords': n, 'params': 2 * entries, 'ms': {'forward': forward, 'backward': backward},
            'queries_per_s': n / (total / 1e3), 'GBps': gbs(sum(C2_BYTES.values()), total),
            'pct_hbm_peak': 100 * gbs(sum(C2_BYTES.values()), total) / HBM_PEAK_GBS,
            'roofline': {'bound': 'hbm', 'kernel': dominant, 'achieved': stage_gbs[dominant], 'peak': HBM_PEAK_GBS,
                         'unit': 'GB/s', 'frac': stage_gbs[dominant] / HBM_PEAK_GBS,
                         'algorithmic_bytes_per_launch': n * C2_BYTES[dominant],
                         'avg_ms': backward if dominant == 'backward' else forward, 'traffic': traffic,
                         'frac_physical': traffic / ((backward if dominant == 'backward' else forward) / 1e3)
                         / 1e9 / HBM_PEAK_GBS if traffic else None},
            'stage_GBps': stage_gbs}


def encode_literal(trainer, steps):
    """The headline metric's own definition, encode fwd+bwd with nothing else: on the step's
    routed batch (64 experts, 2^22 coordinates) and the decoder's upstream planes of the last
    timed step, the encode forward and the encode backward writing the fp32 gradient of all
    70.7 M parameters (the owner pass, no optimizer step), timed with events on their stream.
    1424 B per query (328 forward + 1096 backward)."""
    import torch
    n = N_COORDS
    view = trainer.routing
    coords, offsets = view.coords[:n], view.offsets
    planes = trainer.plane_buffer[:16 * n].view(16, n)
    blockmax = trainer.max_buffer[:32 * ((n + 127) // 128)].view(-1, 32)
    out = trainer.raw[:n]
    gradient = torch.empty(trainer.grid.table.numel(), dtype=torch.float32, device=coords.device)
    stream = torch.cuda.current_stream()
    for _ in range(3):
        trainer.grid.forward(coords, offsets, out=out)
        trainer.grid.backward_planes(coords, offsets, planes, blockmax, gradient=gradient)
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b, c in marks:
        a.record(stream)
        trainer.grid.forward(coords, offsets, out=out)
        b.record(stream)
        trainer.grid.backward_planes(coords, offsets, planes, blockmax, gradient=gradient)
        c.record(stream)
    torch.cuda.synchronize()
    forward = sum(a.elapsed_time(b) for a, b, _ in marks) / steps
    backward = sum(b.elapsed_time(c) for _, b, c in marks) / steps
    per = STAGE_BYTES['encode_forward'] + STAGE_BYTES['encode_backward']
    gbs = n * per / ((forward + backward) / 1e3) / 1e9
    return {'ms': {'forward': forward, 'backward': backward}, 'queries_per_s': n / ((forward + backward) / 1e3),
            'GBps': gbs, 'pct_hbm_peak': 100 * gbs / HBM_PEAK_GBS,
            'backward_GBps': n * STAGE_BYTES['encode_backward'] / (backward / 1e3) / 1e9,
            'kernels': 'grid_forward_kernel; owner_kernel writing the gradient (upstream planes from the decoder)'}


C1_ENCODING = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=19, base_resolution=16, per_level_scale=1.38)
C1_COORDS = 1 << 18
C1_BYTES = 648   # per query: xy 8 + 16 levels * 4 corners * 2 features * 4 B gathers + 32 * 4 B features


def c1_forward(steps, cpu):
    """The single-expert fp32 forward: 16 levels x 2 fp32 features, 2^19-entry tables, base 16,
    scale 1.38, tables U(-1e-4, 1e-4) (seed 0); the forward encode of 2^18 coordinates uniform in
    [0,1)^2 (seed 0) into fp32 [2^18, 32].  GPU: events around `steps` launches after a warm-up,
    the output compared with the oracle's bit for bit; CPU: the oracle's C forward on all host
    cores and on one thread, medians of five."""
    import numpy as np
    import torch
    import oracle
    from odie_amd import synth
    from odie_amd.config import grid_levels
    from odie_amd.encoding import grid_forward
    levels, entries = grid_levels(C1_ENCODING)
    rows = [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]
    table = synth.table(0, 2 * entries)
    xy = synth.coordinates(0, C1_COORDS)
    d_table, d_xy = torch.from_numpy(table).cuda(), torch.from_numpy(xy).cuda()
    out = torch.empty((C1_COORDS, 32), dtype=torch.float32, device='cuda')
    stream = torch.cuda.current_stream()
    for _ in range(5):
        grid_forward(d_xy, d_table, levels, 2, out=out)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        grid_forward(d_xy, d_table, levels, 2, out=out)
    stop.record(stream)
    torch.cuda.synchronize()
    gpu_ms = start.elapsed_time(stop) / steps
    result = {'coords': C1_COORDS, 'params': 2 * entries, 'dtype': 'f32', 'gpu_ms': gpu_ms,
              'queries_per_s': C1_COORDS / (gpu_ms / 1e3),
              'GBps': C1_COORDS * C1_BYTES / (gpu_ms / 1e3) / 1e9,
              'pct_hbm_peak': 100 * C1_COORDS * C1_BYTES / (gpu_ms / 1e3) / 1e9 / HBM_PEAK_GBS}
    if cpu:
        cores = len(os.sched_getaffinity(0))

        def median(threads):
            times = []
            for _ in range(5):
                started = time.perf_counter()
                expected = oracle.hash_forward(xy, table, rows, 2, threads=threads)
                times.append(time.perf_counter() - started)
            return float(np.median(times)), expected

        cpu_s, expected = median(cores)
        one_s, _ = median(1)
        result['matches_oracle'] = bool(np.array_equal(out.cpu().numpy().view(np.uint32), expected.view(np.uint32)))
        result['cpu_baseline'] = {'value': C1_COORDS / cpu_s, 'unit': 'queries/s', 'cores': cores, 'kind': 'port',
                                  'seconds': cpu_s, 'sample': 'the whole 2^18-coordinate forward, median of 5',
                                  'one_thread': {'value': C1_COORDS / one_s, 'seconds': one_s, 'cores': 1}}
        result['gpu_over_cpu'] = result['queries_per_s'] / result['cpu_baseline']['value']
        result['gpu_over_cpu_one_thread'] = result['queries_per_s'] / result['cpu_baseline']['one_thread']['value']
    return result


C5_SIDE, C5_TILES, C5_RESIDUAL_TILE, C5_TOP = 32768, 32, 256, 512
C4_BUDGET_PARAMS = 50 * 2 ** 20 // 2     # 50 MiB of fp16 parameters
C4_DECODER_PARAMS = 7168
C5_ENCODING = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=9, base_resolution=16,
                   per_level_scale=1.38)


def reconstruction_pass(batch, fused=True):
    """The residual + selection pass over the 32768x32768 synthetic image (seed 1): full
    reconstruction through a 1024-expert model (32x32 tiles of 1024^2, 16 levels x 2 fp16
    features, 2^9-entry tables: 16.25 M parameters, 31 MiB), fp64 per-tile residual over
    256x256 tiles (16384 tiles) in raster order, the mse, then the top 512 tiles by mean
    residual (ids ascending).  Reported beside the headline, not as it."""
    import numpy as np
    import torch
    from odie_amd import synth
    from odie_amd.decoder import Decoder
    from odie_amd.experts import ExpertGrid
    from odie_amd.reconstruction import score_image
    from odie_amd.selection import topk_tiles

    side = C5_SIDE
    target = synth.image_device(1, side, side).reshape(-1, 3)
    grid = ExpertGrid(C5_ENCODING, C5_TILES * C5_TILES)
    grid.table.copy_(torch.from_numpy(synth.table(1, grid.table.numel(), -1.0, 1.0, name='c5_table')).half())
    decoder = Decoder(seed=1)
    counts = None

    def run():
        metrics, scores = score_image(grid, decoder.half, target, (side, side), (C5_TILES, C5_TILES),
                                      tile=C5_RESIDUAL_TILE, batch=batch, fused=fused)
        means = scores.totals / torch.from_numpy(scores.counts).cuda()
        return metrics, topk_tiles(means, C5_TOP)

    run()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    metrics, ids = run()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop)
    pixels = side * side
    del target
    return {'pixels': pixels, 'ms': ms, 'pixels_per_s': pixels / (ms / 1e3), 'fused': fused,
            'batch': None if fused else batch,
            'experts': grid.experts, 'params': grid.table.numel(), 'mse': metrics['mse'],
            'top_ids_head': ids[:8].cpu().tolist(),
            'note': 'one odie_reconstruct_scores launch (a wave per residual tile: encode + decoder + fp64 residual '
                    'fold in registers) and odie_topk; random tables; the reference records 38 M px/s for '
                    'full-image inference + residual scoring on an RTX 3060'}


def gigapixel_steps(steps):
    """The gigapixel training step: the 32768x32768 synthetic image (seed 1), 1024 experts on
    its 32x32 tiles of 1024^2 (16 levels x 2 fp16 features, 2^9-entry tables: 16.25 M grid
    parameters + 7168 decoder parameters, 31 MiB in fp16, under the 50 MiB budget), 2^24 pixel
    ids per step; the same step as the headline.  Measured on stratified batches (one pixel per
    8x8 stratum, strata row by row: the reference's gigapixel configurations draw them so), then
    on ids uniform over the image.  The stratified draw is fused into the route
    (odie_route_stratified: torch.rand's uniforms in, the ids never written).  Experts go to the
    non-flat tiles (RGB8 range > 0) in tile order while their parameters fit the 50 MiB fp16
    budget less the decoder's (allocate_tiles); the route takes that tile -> expert map
    (odie_route_allocated), and the ids of tiles left without an expert read zero features.
    Reported beside the headline, not as it."""
    import torch
    from odie_amd import synth
    from odie_amd.config import grid_levels
    from odie_amd.experts import allocate_tiles
    from odie_amd.trainer import ExpertTrainer
    side, n = C5_SIDE, 1 << 24
    image = synth.image_device(1, side, side)
    expert_params = 2 * grid_levels(C5_ENCODING)[1]
    budget = C4_BUDGET_PARAMS - C4_DECODER_PARAMS
    slots, experts = allocate_tiles(image, C5_TILES, C5_TILES, expert_params, budget)
    trainer = ExpertTrainer(image, C5_ENCODING, C5_TILES, C5_TILES, n, grid_lr=1e-2, decoder_lr=1e-3, seed=1,
                            slots=slots, experts=experts)
    generator = torch.Generator(device='cuda').manual_seed(1)
    out = {'coords': n, 'experts': trainer.grid.experts, 'params': trainer.grid.table.numel(), 'steps': steps,
           'allocation': {'tiles': C5_TILES * C5_TILES, 'non_flat_tiles': int((slots >= 0).sum()),
                          'experts': experts, 'budget_params': budget, 'expert_params': expert_params,
                          'rule': 'non-flat tiles (largest per-channel RGB8 range > 0) in tile order, while '
                                  'experts * expert_params <= 26,214,400 (50 MiB fp16) - 7168 decoder params'}}
    stratified = [torch.rand((n, 2), device='cuda', generator=generator) for _ in range(2)]
    uniform = [torch.from_numpy(synth.integers(k, 'gigapixel_ids', n, side * side)).cuda() for k in range(2)]
    for name, batches, step in (('stratified', stratified, lambda b: trainer.step(None, uniforms=b)),
                                ('uniform_ids', uniform, trainer.step)):
        step(batches[0])
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for k in range(steps):
            step(batches[k % 2])
        stop.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(stop) / steps
        out[name] = {'ms_per_step': ms, 'queries_per_s': n / (ms / 1e3),
                     'loss': float(trainer.squares.double().mean())}
        del batches
    return out


def main():
    args = parse()
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1:
        print('bench.py measures one GPU: this build has no multi-GPU path (each GPU would run '
              'its own share of the experts); run with --gpus 1', file=sys.stderr)
        sys.exit(2)
    if args.tune:
        import torch
        torch.zeros(1, device='cuda')   # the runtime up before the library loads
        from odie_amd import _lib
        for item in args.tune:
            key, value = item.split('=')
            _lib.set_tuning(key, int(value))
    if args.single_only:
        print(json.dumps({'single_expert': single_expert_steps(args.steps)}))
        return
    import numpy as np
    import torch
    from odie_amd import synth
    from odie_amd.trainer import ExpertTrainer

    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    image = synth.image(0, WIDTH, HEIGHT)
    trainer = ExpertTrainer(image, ENCODING, REGIONS, REGIONS, N_COORDS, grid_lr=1e-2, decoder_lr=1e-3, seed=0,
                            device=device)
    ids_host = synth.integers(0, 'ids', N_COORDS, WIDTH * HEIGHT)
    ids = torch.from_numpy(ids_host).to(device)
    stream = torch.cuda.current_stream(device)
    table16 = trainer.grid.table.cpu().numpy() if not args.no_cpu else None
    master = trainer.master.cpu().numpy() if not args.no_cpu else None
    decoder16 = trainer.decoder.half.cpu().numpy()

    for _ in range(args.warmup):
        trainer.step(ids)
    torch.cuda.synchronize(device)
    # The K timed steps carry no event but the two around them (every event recorded between
    # kernels adds a few microseconds of stream time: an empty stage measures ~5 us); K more
    # steps, untimed for the headline, record an event after every stage for the breakdown.
    names = ['start', 'route', 'encode_forward', 'decoder', 'encode_backward', 'grid_adam', 'decoder_adam']
    marks = [{name: torch.cuda.Event(enable_timing=True) for name in names} for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    start.record(stream)
    for k in range(args.steps):
        trainer.step(ids)
    stop.record(stream)
    torch.cuda.synchronize(device)
    ms = start.elapsed_time(stop) / args.steps
    loss = float(trainer.squares.double().mean())
    for k in range(args.steps):
        marks[k]['start'].record(stream)
        trainer.step(ids, mark=lambda name, k=k: marks[k][name].record(stream))
    torch.cuda.synchronize(device)
    marked_ms = sum(m['start'].elapsed_time(m['decoder_adam']) for m in marks) / args.steps
    stage_ms = {names[i]: sum(m[names[i - 1]].elapsed_time(m[names[i]]) for m in marks) / args.steps
                for i in range(1, len(names))}
    params = trainer.grid.table.numel()
    stage_bytes = {name: per * N_COORDS for name, per in STAGE_BYTES.items()}
    # the grid's Adam runs inside the encode backward (its flush); its stage mark is empty
    stage_bytes['encode_backward'] += FUSED_ADAM_BYTES * params
    stage_bytes['grid_adam'] = 0
    stage_bytes['decoder_adam'] = ADAM_BYTES * trainer.decoder.params.numel()
    stage_gbs = {name: stage_bytes[name] / (stage_ms[name] / 1e3) / 1e9 if stage_bytes[name] else None
                 for name in stage_ms}
    qps = N_COORDS / (ms / 1e3)
    step_gbs = sum(stage_bytes.values()) / (ms / 1e3) / 1e9
    dominant = max(stage_ms, key=stage_ms.get)
    traffic = profiled_traffic(dominant)
    physical = traffic / (stage_ms[dominant] / 1e3) / 1e9 if traffic else None
    encode_ms = stage_ms['encode_forward'] + stage_ms['encode_backward']
    result = {
        'metric': METRIC, 'value': qps, 'unit': 'queries/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': ms, 'higher_is_better': True, 'scaling': 'weak',
        'vs_baseline': None, 'dtype': 'fp16 tables/features/MLP (fp32 accumulate), fp32 gradients and Adam',
        'data': 'synthetic (procedural 2048x1365 RGB8 image, uniform pixel ids, seed 0)',
        'config': {'workload': '64-expert packed hash grid (8x8 tiles of a 2048x1365 image), 16 levels x 2 fp16 '
                               'features, 2^16-entry tables; 2^22 ids per step: route + encode fwd + decoder '
                               '32-64-64-16 fwd/loss/bwd + encode bwd + Adam (grid and decoder)',
                   'experts': REGIONS * REGIONS, 'coords': N_COORDS, 'params': params,
                   'parallelism': 'single GPU'},
        'achieved_GBps_step': step_gbs, 'pct_hbm_peak_step': 100 * step_gbs / HBM_PEAK_GBS,
        'stage_ms': stage_ms, 'stage_GBps': stage_gbs, 'ms_per_step_with_stage_events': marked_ms,
        'encode_fwd_bwd_queries_per_s': N_COORDS / (encode_ms / 1e3),
        'encode_fwd_bwd_GBps': N_COORDS * (STAGE_BYTES['encode_forward'] + STAGE_BYTES['encode_backward'])
        / (encode_ms / 1e3) / 1e9,
        'roofline': {'bound': 'hbm', 'kernel': '%s (%s)' % (dominant, KERNELS[dominant]),
                     'achieved': stage_gbs[dominant], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': stage_gbs[dominant] / HBM_PEAK_GBS, 'traffic': traffic,
                     'physical_GBps': physical, 'frac_physical': physical / HBM_PEAK_GBS if physical else None,
                     'algorithmic_bytes_per_launch': stage_bytes[dominant], 'avg_ms': stage_ms[dominant]},
        'loss_after_timed_steps': loss,
    }
    if not args.no_literal:
        result['encode_fwd_bwd_literal'] = encode_literal(trainer, args.steps)
    if not args.no_c1:
        result['c1_forward'] = c1_forward(200, not args.no_cpu)
    if not args.no_single:
        result['single_expert'] = single_expert_steps(args.steps)
    if not args.no_native:
        result['native_step'] = native_steps(args.native_steps)
    if not args.no_reconstruction:
        result['reconstruction'] = reconstruction_pass(args.reconstruction_batch)
    if not args.no_gigapixel:
        result['gigapixel_step'] = gigapixel_steps(args.gigapixel_steps)
    if not args.no_cpu:
        result['cpu_baseline'] = cpu_baseline(image, ids_host, table16, master, decoder16, trainer.grid.levels,
                                              trainer.grid.expert_params, args.cpu_seconds)
        result['gpu_over_cpu'] = qps / result['cpu_baseline']['value']
        result['gpu_over_cpu_one_thread'] = qps / result['cpu_baseline']['one_thread']['value']
    print(json.dumps(result))


if __name__ == '__main__':
    main()
