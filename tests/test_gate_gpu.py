"""Router gate on the GPU (odie_gate_forward / odie_gate_backward) against the oracle.

Forward: s within fp16-logit rounding of the oracle's, and the gated features bit-exact given
the GPU's s.  Backward: direct and the gate derivative bit-exact given the GPU's s (sigmoid),
the gate MLP's input gradient and the combined upstream within the fp16 tolerance of the
decoder tests, weight gradients within 2^-9 of their magnitude sums.  Inputs are drawn so that
no gate pre-activation lies within fp32-summation distance of zero (a flipped ReLU mask would
move a whole term)."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.gate import Gate

pytestmark = pytest.mark.gpu


# level rows of the reference's configurations (odie/config.py:129; DIV2K [2]*15+[1], the L8 / L12 /
# L20 ablations) and rows of mixed F1/F2/F4 levels whose columns straddle the 8-column lane groups
SHAPES = {
    '16x2': [2] * 16,
    'div2k': [2] * 15 + [1],
    'L8': [2] * 7 + [1],
    'L12': [2] * 11 + [1],
    'L20': [2] * 19 + [1],
    'mixed': [2, 2, 2, 4, 1, 4, 2, 1, 4, 2, 2, 1, 4, 2],
    '20x4': [4] * 20,
}


def _case(n, seed, features=None):
    features = [2] * 16 if features is None else features
    width = (sum(features) + 15) // 16 * 16
    for attempt in range(20):
        x = (synth.normal(seed + 100 * attempt, 'gate_x', n * width).reshape(n, width) * 0.5).astype(np.float16)
        gate = Gate(seed=seed + attempt, coarse=3, features=features)
        flat = gate.half.cpu().numpy()
        w1 = oracle.gate_weights(flat, len(features))[0].astype(np.float64)
        pre = x.astype(np.float64) @ w1.T
        margin = np.abs(pre) / (np.abs(x.astype(np.float64)) @ np.abs(w1).T + 1e-30)
        if margin.min() > 2.0 ** -18:     # fp32 sums in another order differ by < 2^-19 of it
            return x, gate, flat
    raise AssertionError('no input without near-zero pre-activations')


@pytest.mark.parametrize('n,with_visible,shape', [(4096, False, '16x2'), (1000, True, '16x2'), (3000, True, 'div2k'),
                                                  (2000, True, 'L8'), (2000, False, 'L12'), (2500, True, 'L20'),
                                                  (1500, True, 'mixed'), (1000, True, '20x4')])
def test_gate_forward_and_backward(n, with_visible, shape):
    features = SHAPES[shape]
    levels, width = len(features), (sum(features) + 15) // 16 * 16
    x, gate, flat = _case(n, 3, features)
    visible = synth.integers(5, 'vis', n * levels, 4).reshape(n, levels).astype(bool) if with_visible else None
    xd = torch.from_numpy(x).cuda()
    vd = torch.from_numpy(visible.astype(np.uint8)).cuda() if with_visible else None
    weighted, s = gate.forward(xd, visible=vd)
    s = s.cpu().numpy()
    assert s.shape == (n, levels)
    h, z, _ = oracle.gate_logits(x, flat, levels)
    ref_s = oracle.gate_values(z, 3)[:, :levels]
    z = z[:, :levels]
    # a one-ulp fp16 logit difference moves s by at most s(1-s) * 2^-10 * |z|
    assert np.all(np.abs(s - ref_s) <= ref_s * (1 - ref_s) * 2.0 ** -9 * (np.abs(z.astype(np.float64)) + 1) + 2.0 ** -22)
    assert np.array_equal(weighted.cpu().numpy().view(np.uint16),
                          oracle.gate_apply(x, s, visible, features).view(np.uint16))

    value = (synth.normal(7, 'gate_value', n * width).reshape(n, width) * 0.01).astype(np.float16)
    upstream = gate.backward(xd, torch.from_numpy(value).cuda(), torch.from_numpy(s).cuda(), visible=vd)
    direct, da = oracle.gate_back(x, value, s, 3, visible=visible, features=features)
    dr, dr_magnitude, dweights, magnitude = oracle.gate_mlp_backward(x, h, da, flat, levels)
    expected = oracle.gate_upstream(direct, dr)
    got = upstream.cpu().numpy().astype(np.float64)
    tolerance = 2.0 ** -10 * np.abs(expected.astype(np.float64)) + 2.0 ** -10 * dr_magnitude / 128 + 2.0 ** -24
    assert np.all(np.abs(got - expected) <= tolerance)
    bad = np.abs(gate.grad.cpu().numpy() - dweights) > 2.0 ** -9 * magnitude + 1e-6
    assert not bad.any(), np.flatnonzero(bad)[:8]


def test_gate_backward_is_deterministic_and_empty_batch():
    x, gate, flat = _case(3000, 9)
    xd = torch.from_numpy(x).cuda()
    _, s = gate.forward(xd)
    value = torch.from_numpy((synth.normal(8, 'v', 3000 * 32).reshape(3000, 32) * 0.01).astype(np.float16)).cuda()
    first = gate.backward(xd, value, s).cpu().numpy(), gate.grad.cpu().numpy()
    second = gate.backward(xd, value, s).cpu().numpy(), gate.grad.cpu().numpy()
    assert np.array_equal(first[0].view(np.uint16), second[0].view(np.uint16))
    assert np.array_equal(first[1].view(np.uint32), second[1].view(np.uint32))
    empty = torch.empty((0, 32), dtype=torch.float16, device='cuda')
    gate.backward(empty, empty, torch.empty((0, 16), device='cuda'))
    torch.cuda.synchronize()
    assert not gate.grad.any()
