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
    parser.add_argument('--cpu-seconds', type=float, default=15.0,
                        help='approximate budget of the CPU baseline sample')
    parser.add_argument('--no-cpu', action='store_true')
    parser.add_argument('--no-native', action='store_true', help='skip the 65536-id native step measurement')
    parser.add_argument('--native-steps', type=int, default=200)
    parser.add_argument('--no-reconstruction', action='store_true', help='skip the 32768^2 residual pass')
    parser.add_argument('--reconstruction-batch', type=int, default=1 << 26)
    parser.add_argument('--no-gigapixel', action='store_true', help='skip the 1024-expert 2^24-id step')
    parser.add_argument('--gigapixel-steps', type=int, default=5)
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
    """Time the oracle's port of the step on a bounded sample of the same ids: routing,
    encode forward, decoder forward/loss/backward and encode backward per query; Adam over the
    whole table once per batch, measured on a slice and scaled to the table."""
    import numpy as np
    import oracle
    rows = [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]
    cores = len(os.sched_getaffinity(0))
    experts = REGIONS * REGIONS
    total = table16.size
    rgb = image.reshape(-1, 3)

    def per_query(count):
        sample = ids[:count]
        started = time.perf_counter()
        _, perm, local, offsets = oracle.route(sample, WIDTH, HEIGHT, REGIONS, REGIONS)
        raw = oracle.hash_forward(local, table16, rows, 2, offsets=offsets, expert_params=expert_params,
                                  threads=cores)
        dz, _ = oracle.mlp_step_f32(raw, decoder16, oracle.mlp_targets(perm, rgb=rgb, ids=sample), perm, count,
                                    threads=cores)
        oracle.hash_backward_f32(local, dz, rows, 2, total, offsets=offsets, expert_params=expert_params,
                                 threads=cores)
        return time.perf_counter() - started

    def adam(count):
        p = master[:count].astype(np.float64)
        g = np.where(np.arange(count) % 3 == 0, 0.0, 1e-3)
        m, v = np.zeros(count), np.zeros(count)
        steps = np.zeros(count, dtype=np.uint32)
        started = time.perf_counter()
        oracle.adam(1, p, g, m, v, steps, 1, 1e-2, scale=128.0)
        return time.perf_counter() - started

    # per-query rate from two sample sizes (the difference removes once-per-batch costs such
    # as clearing the gradient), plus the once-per-batch part itself
    probe = 1 << 14
    rate = probe / per_query(probe)
    small = int(min(len(ids) // 2, max(probe, rate * budget * 0.5 / 9)))
    t_small = sorted(per_query(small) for _ in range(3))[1]
    t_large = sorted(per_query(2 * small) for _ in range(3))[1]
    marginal = max(t_large - t_small, 1e-9) / small
    fixed = max(t_small - marginal * small, 0.0)
    slice_ = 1 << 22
    adam_seconds = sorted(adam(slice_) for _ in range(3))[1] * total / slice_
    step_seconds = marginal * N_COORDS + fixed + adam_seconds
    count = 2 * small
    return dict(value=N_COORDS / step_seconds, unit='queries/s', cores=cores, kind='port',
                sample='first %d and %d of the 2^22 ids through route+encode fwd+decoder+encode bwd (median '
                       'of 3 each; per-query rate from the difference, OpenMP %d threads for encode and Adam, '
                       'torch-CPU fp32 for the decoder), plus Adam over a 2^22-parameter slice scaled to the %d-parameter '
                       'table, once per 2^22-query batch' % (count // 2, count, cores, total),
                seconds_per_step=step_seconds,
                cpu=platform.processor() or platform.machine())


NATIVE_RESOLUTIONS = [16, 23, 31, 43, 59, 81, 111, 153, 211, 291, 401, 554, 764, 1054, 1454, 2006]
NATIVE_HASH = dict(otype='HashGrid', n_levels=16, n_features_per_level=2, log2_hashmap_size=19, base_resolution=16,
                   per_level_scale=1.38)


def native_steps(image, steps):
    """The reference's own training step (NativeOptimizer over the odie_* runtime) at its batch of
    65536 ids, replayed from a captured graph: packed xy planes (16 full levels, R = 16..2006)
    and the hash grid (16 levels, 2^19-entry tables), both with the router gate.  Reported
    beside the headline, not as it."""
    import numpy as np
    import torch
    from odie_amd import synth
    from odie_amd.config import grid_levels
    from odie_amd.decoder import Decoder
    from odie_amd.gate import Gate
    from odie_amd.model import PackedPlanes
    from odie_amd.native_backend import NativeModel, NativeOptimizer, make_native_optimizer
    from odie_amd.sampling import stratified_batches

    target = torch.from_numpy(image).cuda().contiguous()
    shape = image.shape[:2]
    out = {}
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for kind in ('packed_planes', 'hash_grid'):
            config = dict(representation='xy_planes' if kind == 'packed_planes' else 'hash_grid',
                          hash_encoding=NATIVE_HASH, n_levels=16, plane_feature_dimensions=[2] * 16,
                          router_enabled=True, target_storage='uint8', gate_coarse_levels_K=0,
                          router_output_activation='sigmoid', grid_lr=1e-2, gate_lr=1e-3, decoder_lr=1e-3)
            if kind == 'packed_planes':
                supports = [torch.ones(r * r, dtype=torch.bool) for r in NATIVE_RESOLUTIONS]
                caps = [(r * r + 7) // 8 * 8 for r in NATIVE_RESOLUTIONS]
                planes = PackedPlanes(dict(resolutions=NATIVE_RESOLUTIONS, n_levels=16, representation='xy_planes',
                                           coarse_levels=0, gate_topology='shared', gate_position='feature',
                                           initial_active_prefix=16, seed=0, feature_init_std=1e-3),
                                      supports, [2] * 16, caps)
                model = NativeModel(Decoder(seed=0), Gate(seed=1), planes=planes)
                optimizer, _ = make_native_optimizer(model, target, shape, config)
            else:
                _, entries = grid_levels(NATIVE_HASH)
                grid = torch.from_numpy(synth.table(0, 2 * entries, name='native_hash')).cuda()
                model = NativeModel(Decoder(seed=0), Gate(seed=1), grid=grid)
                optimizer = NativeOptimizer(model, target, shape, config, [grid])
            optimizer.prepare_epoch()
            draw = stratified_batches(shape, 65536, torch.Generator(device='cuda').manual_seed(0))
            samplings = {'': [next(draw) for _ in range(4)],
                         '_uniform_ids': [torch.from_numpy(synth.integers(k, 'native_ids', 65536,
                                                                          shape[0] * shape[1])).cuda()
                                          for k in range(4)]}
            for suffix, batches in samplings.items():
                for k in range(5):
                    optimizer.train_batch(batches[k % 4])
                start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                start.record(stream)
                for k in range(steps):
                    optimizer.fixed.copy_(batches[k % 4])
                    optimizer.graph.replay()
                stop.record(stream)
                torch.cuda.synchronize()
                ms = start.elapsed_time(stop) / steps
                loss = float(optimizer.squares.double().mean())
                out[kind + suffix] = {'ms_per_step': ms, 'pixels_per_s': 65536 / (ms / 1e3),
                                      'params': model.grid.numel(), 'loss': loss}
            optimizer.close()
    out['batch'] = 65536
    out['steps'] = steps
    out['note'] = ('graph replays of odie_step (router on), ids resident, stratified batches as the '
                   "reference's configurations draw them (the *_uniform_ids lines: ids uniform over the "
                   'image); the reference records 34.8 M px/s (packed planes) and 19.0 M px/s (hash grid) '
                   'for this step on an RTX 3060')
    return out


C5_SIDE, C5_TILES, C5_RESIDUAL_TILE, C5_TOP = 32768, 32, 256, 512
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
    on ids uniform over the image.  Reported beside the headline, not as it."""
    import torch
    from odie_amd import synth
    from odie_amd.sampling import stratified_batches
    from odie_amd.trainer import ExpertTrainer
    side, n = C5_SIDE, 1 << 24
    image = synth.image_device(1, side, side)
    trainer = ExpertTrainer(image, C5_ENCODING, C5_TILES, C5_TILES, n, grid_lr=1e-2, decoder_lr=1e-3, seed=1)
    draw = stratified_batches((side, side), n, torch.Generator(device='cuda').manual_seed(1))
    out = {'coords': n, 'experts': trainer.grid.experts, 'params': trainer.grid.table.numel(), 'steps': steps}
    for name, batches in (('stratified', [next(draw) for _ in range(2)]),
                          ('uniform_ids', [torch.from_numpy(synth.integers(k, 'gigapixel_ids', n, side * side)).cuda()
                                           for k in range(2)])):
        trainer.step(batches[0])
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for k in range(steps):
            trainer.step(batches[k % 2])
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
    names = ['start', 'route', 'encode_forward', 'decoder', 'encode_backward', 'grid_adam', 'decoder_adam']
    marks = [{name: torch.cuda.Event(enable_timing=True) for name in names} for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    start.record(stream)
    for k in range(args.steps):
        marks[k]['start'].record(stream)
        trainer.step(ids, mark=lambda name, k=k: marks[k][name].record(stream))
    stop.record(stream)
    torch.cuda.synchronize(device)
    ms = start.elapsed_time(stop) / args.steps
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
    traffic_file = ROOT / 'profiles' / 'traffic.json'
    traffic = None
    if traffic_file.exists():
        entry = json.loads(traffic_file.read_text()).get(dominant)
        traffic = entry['bytes'] if entry else None
    encode_ms = stage_ms['encode_forward'] + stage_ms['encode_backward']
    loss = float(trainer.squares.double().mean())
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
        'stage_ms': stage_ms, 'stage_GBps': stage_gbs,
        'encode_fwd_bwd_queries_per_s': N_COORDS / (encode_ms / 1e3),
        'encode_fwd_bwd_GBps': N_COORDS * (STAGE_BYTES['encode_forward'] + STAGE_BYTES['encode_backward'])
        / (encode_ms / 1e3) / 1e9,
        'roofline': {'bound': 'hbm', 'kernel': '%s (%s)' % (dominant, KERNELS[dominant]),
                     'achieved': stage_gbs[dominant], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': stage_gbs[dominant] / HBM_PEAK_GBS, 'traffic': traffic,
                     'algorithmic_bytes_per_launch': stage_bytes[dominant], 'avg_ms': stage_ms[dominant]},
        'loss_after_timed_steps': loss,
    }
    if not args.no_native:
        result['native_step'] = native_steps(image, args.native_steps)
    if not args.no_reconstruction:
        result['reconstruction'] = reconstruction_pass(args.reconstruction_batch)
    if not args.no_gigapixel:
        result['gigapixel_step'] = gigapixel_steps(args.gigapixel_steps)
    if not args.no_cpu:
        result['cpu_baseline'] = cpu_baseline(image, ids_host, table16, master, decoder16, trainer.grid.levels,
                                              trainer.grid.expert_params, args.cpu_seconds)
        result['gpu_over_cpu'] = qps / result['cpu_baseline']['value']
    print(json.dumps(result))


if __name__ == '__main__':
    main()
