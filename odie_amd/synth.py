"""Deterministic synthetic inputs, identical on every machine.

Random words come from a counter-based SplitMix64 (Steele, Lea & Flood 2014): word i of a
named stream is mix(key + (i+1)*0x9E3779B97F4A7C15), where key = mix(seed*phi + fnv1a(name)).
Each tensor draws from its own named stream, so adding a tensor never shifts another.
Derived values:
  uniform fp32 in [0,1): (word >> 40) * 2^-24
  uniform integer in [0, m): (word >> 32) * m >> 32
  normal: Box-Muller in fp64 on two words, u1 = ((w1>>11)+1)*2^-53, u2 = (w2>>11)*2^-53
"""
import numpy as np

PHI = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z):
    with np.errstate(over='ignore'):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _fnv1a(name):
    value = 14695981039346656037
    for byte in name.encode():
        value = ((value ^ byte) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return np.uint64(value)


def stream_key(seed, name):
    with np.errstate(over='ignore'):
        return _mix(np.asarray(np.uint64(seed) * PHI + _fnv1a(name), dtype=np.uint64))


def words(seed, name, count, start=0):
    key = stream_key(seed, name)
    counter = np.arange(start + 1, start + 1 + count, dtype=np.uint64)
    with np.errstate(over='ignore'):
        return _mix(key + counter * PHI)


def uniform(seed, name, count):
    """fp32 in [0, 1) with 24 random bits."""
    return ((words(seed, name, count) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24))


def integers(seed, name, count, modulus):
    """Uniform integers in [0, modulus) by 32-bit multiply-shift (modulus < 2^32)."""
    high = (words(seed, name, count) >> np.uint64(32))
    return ((high * np.uint64(modulus)) >> np.uint64(32)).astype(np.int64)


def normal(seed, name, count):
    w = words(seed, name, 2 * count)
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def coordinates(seed, count, name='coords'):
    """count x 2 fp32 coordinates uniform in [0, 1)^2."""
    return uniform(seed, name, 2 * count).reshape(count, 2)


def table(seed, count, low=-1e-4, high=1e-4, name='table'):
    """fp32 table values uniform in [low, high), computed in fp64 then rounded."""
    u = uniform(seed, name, count).astype(np.float64)
    return (low + (high - low) * u).astype(np.float32)


def upstream(seed, rows, columns, name='upstream'):
    """fp16 [rows, columns] standard normal upstream gradients."""
    return normal(seed, name, rows * columns).astype(np.float16).reshape(rows, columns)


def image(seed, width, height, octaves=6, edges=32):
    """uint8 [height, width, 3]: a sum of `octaves` octaves of band-limited value noise (a
    random lattice of 4*2^k cells per side, smoothstep-interpolated, amplitude 2^-k) plus
    `edges` random axis-aligned rectangles that add a random colour step, normalized to
    0..255."""
    xs = np.arange(width, dtype=np.float64) / (width - 1)
    ys = np.arange(height, dtype=np.float64) / (height - 1)
    rgb = np.zeros((height, width, 3))
    for k in range(octaves):
        cells = 4 << k
        lattice = uniform(seed, 'octave%d' % k, (cells + 1) * (cells + 1) * 3).astype(np.float64)
        lattice = lattice.reshape(cells + 1, cells + 1, 3)

        def axis(t):
            g = t * cells
            i = np.minimum(g.astype(np.int64), cells - 1)
            f = g - i
            return i, f * f * (3.0 - 2.0 * f)
        ix, fx = axis(xs)
        iy, fy = axis(ys)
        rows = lattice[:, ix] * (1 - fx)[None, :, None] + lattice[:, ix + 1] * fx[None, :, None]  # along x
        rgb += (rows[iy] * (1 - fy)[:, None, None] + rows[iy + 1] * fy[:, None, None]) * 0.5 ** k
    corners = integers(seed, 'edge_corners', edges * 4, 1 << 30)
    colours = uniform(seed, 'edge_colours', edges * 3).astype(np.float64).reshape(edges, 3) - 0.5
    for e in range(edges):
        x0, x1 = sorted(int(c) * width >> 30 for c in corners[4 * e:4 * e + 2])
        y0, y1 = sorted(int(c) * height >> 30 for c in corners[4 * e + 2:4 * e + 4])
        rgb[y0:y1 + 1, x0:x1 + 1] += colours[e]
    low, high = rgb.min(), rgb.max()
    return np.round((rgb - low) / (high - low) * 255.0).astype(np.uint8)


def image_device(seed, width, height, octaves=6, edges=32, device='cuda', rows=2048):
    """image() computed with torch on `device`, `rows` image rows at a time (for gigapixel
    sizes): the same fp64 operations in the same order, so the same bytes; uint8 [height,
    width, 3].  Divisions are tensor by tensor (torch turns division by a Python scalar into a
    reciprocal multiply)."""
    import torch

    def axis(size, cells):
        t = np.arange(size, dtype=np.float64) / (size - 1)
        g = t * cells
        i = np.minimum(g.astype(np.int64), cells - 1)
        f = g - i
        return torch.from_numpy(i).to(device), torch.from_numpy(f * f * (3.0 - 2.0 * f)).to(device)

    octave_rows, octave_y = [], []
    for k in range(octaves):
        cells = 4 << k
        lattice = torch.from_numpy(uniform(seed, 'octave%d' % k, (cells + 1) * (cells + 1) * 3).astype(np.float64)
                                   .reshape(cells + 1, cells + 1, 3)).to(device)
        ix, fx = axis(width, cells)
        octave_rows.append(lattice[:, ix] * (1 - fx)[None, :, None] + lattice[:, ix + 1] * fx[None, :, None])
        octave_y.append(axis(height, cells))
    corners = integers(seed, 'edge_corners', edges * 4, 1 << 30)
    colours = torch.from_numpy(uniform(seed, 'edge_colours', edges * 3).astype(np.float64).reshape(edges, 3) - 0.5)
    boxes = []
    for e in range(edges):
        x0, x1 = sorted(int(c) * width >> 30 for c in corners[4 * e:4 * e + 2])
        y0, y1 = sorted(int(c) * height >> 30 for c in corners[4 * e + 2:4 * e + 4])
        boxes.append((x0, x1, y0, y1, colours[e].to(device)))

    def block(r0, r1):
        rgb = torch.zeros((r1 - r0, width, 3), dtype=torch.float64, device=device)
        for k in range(octaves):
            iy, fy = octave_y[k]
            iy, fy = iy[r0:r1], fy[r0:r1]
            rows_ = octave_rows[k]
            rgb += (rows_[iy] * (1 - fy)[:, None, None] + rows_[iy + 1] * fy[:, None, None]) * 0.5 ** k
        for x0, x1, y0, y1, colour in boxes:
            a, b = max(y0, r0), min(y1 + 1, r1)
            if a < b:
                rgb[a - r0:b - r0, x0:x1 + 1] += colour
        return rgb

    low = high = None
    for r0 in range(0, height, rows):
        rgb = block(r0, min(r0 + rows, height))
        low = rgb.min() if low is None else torch.minimum(low, rgb.min())
        high = rgb.max() if high is None else torch.maximum(high, rgb.max())
    out = torch.empty((height, width, 3), dtype=torch.uint8, device=device)
    span = high - low
    for r0 in range(0, height, rows):
        r1 = min(r0 + rows, height)
        out[r0:r1] = torch.round((block(r0, r1) - low) / span * 255.0).to(torch.uint8)
    return out
