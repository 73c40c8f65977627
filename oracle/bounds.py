"""The checker's bar for encode gradients -- TEST INFRASTRUCTURE ONLY.

An entry of the gradient is within

    1e-4 * sum|c| + count * q / 2

of the oracle's sum, where sum|c| and count are the sum of the absolute values and the number
of its contributions c = fp32(w_k * u) (the oracle returns both), and q is the quantum of the
fixed-point sum that formed it.  The first term is the 1e-4 relative bar after summation (it
also covers the fp32 rounding of the final value, 2^-24 of it); the second is the rounding of
each contribution to the nearest multiple of q.  For fp32 atomic sums q is 0.

The owner backward forms every (level, feature) column of an expert's gradient at its own
scale: q = 2^-shift with shift = min(30 - ilogb(P), 61 - ilogb(4 * count * P)), capped at 120
(60 when P = 0), where P is the largest |u| of that column over the 128-row records that meet
the expert's coordinates and count the number of those coordinates -- one scale per column
whichever pass or split of the expert covers it.  The packed-plane owner takes P over all
coordinates and count = n.
"""
import numpy as np

RTOL = 1e-4
RECORD = 128   # rows per |upstream| maximum record


def fixed_point_quantum(peak, count):
    """q = 2^-shift for columns of largest |u| `peak` summed over `count` coordinates (arrays
    broadcast); inf where the peak is not finite (the backward writes NaN there)."""
    peak = np.asarray(peak, dtype=np.float64)
    count = np.asarray(count, dtype=np.float64)
    finite = np.isfinite(peak)
    safe = np.where(finite & (peak > 0), peak, 1.0)
    by_value = 30 - (np.frexp(safe)[1] - 1)                       # ilogb(x) = frexp exponent - 1
    by_sum = 61 - (np.frexp(4.0 * np.maximum(count, 1.0) * safe)[1] - 1)
    shift = np.where(peak > 0, np.minimum(by_value, by_sum), 60)
    shift = np.minimum(shift, 120)
    return np.where(finite, np.ldexp(1.0, -shift.astype(np.int64)), np.inf)


def _expert_ranges(offsets, n, experts):
    if offsets is None:
        return [(0, n)]
    offsets = np.asarray(offsets, dtype=np.int64)
    ranges = []
    for e in range(experts):
        base = min(max(int(offsets[e]), 0), n)
        stop = max(min(int(offsets[e + 1]), n), base)
        ranges.append((base, stop))
    return ranges


def hash_quantum(upstream, rows, features, total, *, offsets=None, expert_params=None):
    """Per-entry quantum bound [total] of the owner backward of a hash grid: rows are the
    levels' (scale, resolution, size, offset, hashed); upstream [n, width] as the backward read it."""
    u = np.abs(np.asarray(upstream).astype(np.float64))
    n = len(u)
    experts = 1 if offsets is None else len(offsets) - 1
    expert_params = expert_params or total // experts
    columns = len(rows) * features
    q = np.zeros(total, dtype=np.float64)
    for e, (base, stop) in enumerate(_expert_ranges(offsets, n, experts)):
        if stop <= base:
            continue
        r0, r1 = base // RECORD, (stop - 1) // RECORD
        peaks = u[RECORD * r0:min(n, RECORD * (r1 + 1)), :columns].max(axis=0)
        quanta = fixed_point_quantum(peaks, stop - base)
        for l, (_, _, size, offset, _) in enumerate(rows):
            for c in range(features):
                start = e * expert_params + offset * features + c
                q[start:start + size * features:features] = quanta[l * features + c]
    return q


def packed_quantum(upstream, layout, total):
    """Per-entry quantum bound [total] of the packed-plane owner backward (descriptor rows of
    the layout; upstream fp16 [n, width])."""
    u = np.abs(np.asarray(upstream).astype(np.float64))
    n, width = u.shape
    desc = np.asarray(layout['descriptors'], dtype=np.int64)
    q = np.zeros(total, dtype=np.float64)
    for l, d in enumerate(desc):
        end = int(desc[l + 1][2]) if l + 1 < len(desc) else total
        features = int(d[5])
        for c in range(features):
            column = int(d[6]) + c
            peak = u[:, column].max(initial=0.0) if column < width and n else 0.0
            q[int(d[2]) + c:end:features] = fixed_point_quantum(peak, n)
    return q


def gradient_bound(magnitude, counts, quantum):
    """The allowed |gpu - oracle| of every entry."""
    return RTOL * magnitude + counts * quantum * (0.5 + 2.0 ** -20)


def check_gradient(gpu, expected, magnitude, counts, quantum, label=''):
    """Raises AssertionError naming the first entries outside gradient_bound."""
    gpu = np.asarray(gpu, dtype=np.float64)
    bad = np.abs(gpu - expected) > gradient_bound(magnitude, counts, quantum)
    if bad.any():
        where = np.flatnonzero(bad)[:5]
        raise AssertionError('%s: %d/%d gradient entries out of tolerance, first %s: gpu %r oracle %r' % (
            label, bad.sum(), bad.size, where, gpu[where], expected[where]))
