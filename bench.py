"""Headline benchmark: packed 64-expert hash-grid encode forward+backward on 2^22 coords.

Workload: a 2048x1365 image cut into 8x8 tiles, one expert per tile; every expert is a
16-level hash grid (2 fp16 features per level, 2^16-entry tables, base resolution 16,
per-level scale 1.38), 70,745,088 parameters in one packed table.  2^22 pixel ids
(uniform, seed 0) are routed to their tile experts and compacted on the GPU once during
setup; the upstream gradient [2^22, 32] is fp16 N(0,1) (seed 0).

One step = encode forward (features [2^22,32] fp16) + encode backward (fp32 gradient of all
70.7M parameters, every value written), all resident in HBM.  The CPU baseline runs
the oracle's bit-exact port of the same fwd+bwd on the first coordinates of the same
batch, on the host's cores.

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
# Algorithmic bytes per query (fp16 table, fp32 gradient accumulators):
#   forward  8 (xy) + 16 levels*4 corners*2 feats*2 B (gathers) + 32*2 B (features)   = 328
#   backward 8 (xy) + 32*2 B (upstream) + 16*4*2*(4 B read + 4 B write) (scatter)     = 1096
FWD_BYTES, BWD_BYTES = 328, 1096


def parse():
    parser = argparse.ArgumentParser()
    parser.add_argument('--gpus', type=int, default=1)
    parser.add_argument('--steps', type=int, default=20)
    parser.add_argument('--warmup', type=int, default=3)
    parser.add_argument('--cpu-seconds', type=float, default=15.0,
                        help='approximate budget of the CPU baseline sample')
    parser.add_argument('--no-cpu', action='store_true')
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


def cpu_baseline(xy, offsets, table, upstream, levels, expert_params, budget):
    """Time the oracle's port of fwd+bwd on a bounded sample of the same routed batch."""
    import numpy as np
    import oracle
    rows = [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]
    cores = len(os.sched_getaffinity(0))
    experts = len(offsets) - 1
    # probe the rate on a small prefix, then size the sample to the budget
    def run(count):
        cut = np.minimum(offsets, count)
        started = time.perf_counter()
        oracle.hash_forward(xy[:count], table, rows, 2, offsets=cut, expert_params=expert_params, threads=cores)
        oracle.hash_backward_f32(xy[:count], upstream[:count], rows, 2, experts * expert_params, offsets=cut,
                                 expert_params=expert_params, threads=cores)
        return time.perf_counter() - started
    probe = 1 << 14
    rate = probe / run(probe)
    count = int(min(len(xy), max(probe, rate * budget / 3)))
    times = [run(count) for _ in range(3)]
    seconds = sorted(times)[1]
    return dict(value=count / seconds, unit='queries/s', cores=cores, kind='port',
                sample='first %d of the 2^22 routed coords (experts 0..%d), fwd+bwd, median of 3, '
                       'oracle C port with exact fp16 FMA emulation, OpenMP %d threads' % (
                           count, int(np.searchsorted(offsets, count, side='left')), cores),
                cpu=platform.processor() or platform.machine())


def main():
    args = parse()
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1:
        print('bench.py measures one GPU: this build has no multi-GPU path (each GPU would run '
              'its own share of the experts); run with --gpus 1', file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from odie_amd import synth
    from odie_amd.experts import ExpertGrid, route

    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    experts = REGIONS * REGIONS
    grid = ExpertGrid(ENCODING, experts, dtype=torch.float16, device=device)
    grid.table.copy_(torch.from_numpy(synth.table(0, grid.table.numel()).astype(np.float16)))
    ids = torch.from_numpy(synth.integers(0, 'ids', N_COORDS, WIDTH * HEIGHT)).to(device)
    routed = route(ids, WIDTH, HEIGHT, REGIONS, REGIONS)
    upstream = torch.from_numpy(synth.upstream(0, N_COORDS, grid.width)).to(device)
    features = torch.empty((N_COORDS, grid.width), dtype=torch.float16, device=device)
    gradient = torch.empty(grid.table.numel(), dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device)

    def step(events=None):
        # The backward writes every gradient value (it clears as part of the scatter), so the
        # step is exactly forward + backward.
        if events:
            events[0].record(stream)
        grid.forward(routed.coords, routed.offsets, out=features)
        if events:
            events[1].record(stream)
        grid.backward(routed.coords, routed.offsets, upstream, gradient=gradient, accumulate=False)
        if events:
            events[2].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(device)
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    start.record(stream)
    for k in range(args.steps):
        step(marks[k])
    stop.record(stream)
    torch.cuda.synchronize(device)
    ms = start.elapsed_time(stop) / args.steps
    fwd_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / args.steps
    bwd_ms = sum(m[1].elapsed_time(m[2]) for m in marks) / args.steps
    qps = N_COORDS / (ms / 1e3)
    step_gbs = N_COORDS * (FWD_BYTES + BWD_BYTES) / (ms / 1e3) / 1e9
    fwd_gbs = N_COORDS * FWD_BYTES / (fwd_ms / 1e3) / 1e9
    bwd_gbs = N_COORDS * BWD_BYTES / (bwd_ms / 1e3) / 1e9
    # The dominant launch is the backward: odie_grid_backward runs transpose_half2_kernel then
    # owner_kernel on the stream, timed together by the events around the call.
    dominant = ('grid_backward', bwd_ms, bwd_gbs, BWD_BYTES) if bwd_ms >= fwd_ms else \
        ('grid_forward', fwd_ms, fwd_gbs, FWD_BYTES)
    kernels = {'grid_backward': 'transpose_half2_kernel + owner_kernel', 'grid_forward': 'grid_forward_kernel'}
    traffic_file = ROOT / 'profiles' / 'traffic.json'
    traffic = None
    if traffic_file.exists():
        entry = json.loads(traffic_file.read_text()).get(dominant[0])
        traffic = entry['bytes'] if entry else None
    result = {
        'metric': METRIC, 'value': qps, 'unit': 'queries/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': ms, 'higher_is_better': True, 'scaling': 'weak',
        'vs_baseline': None, 'dtype': 'fp16 table/features, fp32 gradient', 'data': 'synthetic',
        'config': {'workload': '64-expert packed hash grid (8x8 tiles of a 2048x1365 image), 16 levels x 2 fp16 '
                               'features, 2^16-entry tables, 2^22 routed coords, encode fwd+bwd',
                   'experts': experts, 'coords': N_COORDS, 'params': grid.table.numel(),
                   'parallelism': 'single GPU'},
        'achieved_GBps_step': step_gbs, 'pct_hbm_peak_step': 100 * step_gbs / HBM_PEAK_GBS,
        'kernels_ms': {'forward': fwd_ms, 'backward': bwd_ms},
        'roofline': {'bound': 'hbm', 'kernel': '%s (%s)' % (dominant[0], kernels[dominant[0]]),
                     'achieved': dominant[2], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': dominant[2] / HBM_PEAK_GBS, 'traffic': traffic,
                     'algorithmic_bytes_per_launch': dominant[3] * N_COORDS, 'avg_ms': dominant[1]},
        'forward_GBps': fwd_gbs, 'backward_GBps': bwd_gbs,
    }
    if not args.no_cpu:
        order = routed.perm.long()
        xy = routed.coords.cpu().numpy()
        offsets = routed.offsets.cpu().numpy().astype(np.int64)
        result['cpu_baseline'] = cpu_baseline(xy, offsets, grid.table.cpu().numpy(), upstream.cpu().numpy(),
                                              grid.levels, grid.expert_params, args.cpu_seconds)
        result['gpu_over_cpu'] = qps / result['cpu_baseline']['value']
        del order
    print(json.dumps(result))


if __name__ == '__main__':
    main()
