"""Grid geometry for the multiresolution hash grid.

hash_grid_layout restates odie/config.py:83-94: the per-level fp32 grid scale
2^(l*log2 g)*base - 1, resolution ceil(scale)+1 and table size min(align8(res^2), 2^log2T).
grid_levels turns an encoding description into the odie_grid_level table the native
encode consumes (a level is hashed when res^2 exceeds its table).
"""
import math

import numpy as np


def align(value, multiple=8):
    return (int(value) + multiple - 1) // multiple * multiple


def _integer(value, name, minimum, maximum=None):
    if type(value) is not int or value < minimum or (maximum is not None and value > maximum):
        raise ValueError(f'{name} must be an integer in [{minimum}, {maximum or "inf"}]')
    return value


def level_scales(n_levels, base_resolution, per_level_scale):
    """fp32 grid scales, rounded at the same points as odie/config.py:91-92."""
    growth = np.float32(per_level_scale)
    if not math.isfinite(float(growth)) or float(growth) <= 1:
        raise ValueError('HashGrid per_level_scale must be finite and greater than one')
    log_growth = np.float32(math.log2(float(growth)))
    scales = []
    for level in range(n_levels):
        exponent = np.float32(level * float(log_growth))
        power = np.float32(2.0 ** float(exponent))
        scales.append(np.float32(np.float32(power * np.float32(base_resolution)) - np.float32(1.0)))
    return scales


def hash_grid_layout(encoding):
    """Resolutions and per-level table sizes of a 2D HashGrid (odie/config.py:83-94)."""
    levels = _integer(encoding['n_levels'], 'HashGrid n_levels', 2, 20)
    base = _integer(encoding['base_resolution'], 'HashGrid base_resolution', 2)
    exponent = _integer(encoding['log2_hashmap_size'], 'log2_hashmap_size', 3, 30)
    scales = level_scales(levels, base, encoding['per_level_scale'])
    resolutions = [math.ceil(float(s)) + 1 for s in scales]
    return resolutions, [min(align(r * r), 1 << exponent) for r in resolutions]


def grid_levels(encoding, max_levels=32):
    """odie_grid_level rows for an encoding dict (n_levels, base_resolution,
    log2_hashmap_size, per_level_scale); the level count may exceed the reference's 20
    only up to the native limit of 32."""
    from ._lib import GridLevel
    levels = int(encoding['n_levels'])
    if not 1 <= levels <= max_levels:
        raise ValueError('n_levels must be within 1..%d' % max_levels)
    base = _integer(encoding['base_resolution'], 'base_resolution', 2)
    exponent = _integer(encoding['log2_hashmap_size'], 'log2_hashmap_size', 3, 30)
    scales = level_scales(levels, base, encoding['per_level_scale'])
    rows, offset = (GridLevel * levels)(), 0
    for level, scale in enumerate(scales):
        resolution = math.ceil(float(scale)) + 1
        size = min(align(resolution * resolution), 1 << exponent)
        rows[level] = GridLevel(float(scale), resolution, size, offset, int(resolution * resolution > size))
        offset += size
    return rows, offset


def describe_levels(rows):
    return [dict(scale=float(r.scale), resolution=r.resolution, size=r.size, offset=r.offset,
                 hashed=bool(r.hashed)) for r in rows]
