"""Fused Adam against the oracle (fp64 closed form) and torch.optim.Adam."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.optimizer import FusedAdam

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('variant,grad_dtype,n', [('torch', torch.float32, 1000003), ('tcnn', torch.float16, 4099),
                                                  ('torch', torch.float16, 17), ('tcnn', torch.float32, 100000),
                                                  ('tcnn_dense', torch.float32, 7168)])
def test_adam_matches_oracle(variant, grad_dtype, n):
    start = synth.normal(5, 'params', n).astype(np.float32)
    master = torch.from_numpy(start).cuda()
    half = torch.empty(n, dtype=torch.float16, device='cuda')
    opt = FusedAdam(master, lr=1e-2, variant=variant, half_copy=half)
    p = start.astype(np.float64)
    m, v = np.zeros(n), np.zeros(n)
    steps = np.zeros(n, dtype=np.uint32)
    for t in range(1, 4):
        g = (synth.normal(5 + t, 'grad', n) * 128).astype(np.float32)
        g[::5] = 0.0
        grad = torch.from_numpy(g).to(grad_dtype)
        opt.step(grad.cuda(), loss_scale=128.0)
        p = oracle.adam({'torch': 0, 'tcnn': 1, 'tcnn_dense': 2}[variant], p, grad.float().numpy().astype(np.float64), m, v, steps, t,
                        1e-2, scale=128.0)
    got = master.cpu().numpy().astype(np.float64)
    assert np.allclose(got, p, rtol=1e-5, atol=1e-6), np.abs(got - p).max()
    assert np.array_equal(half.cpu().numpy().view(np.uint16), master.cpu().numpy().astype(np.float16).view(np.uint16))
    if variant != 'torch':
        assert np.array_equal(opt.steps.cpu().numpy().astype(np.uint32), steps)


def test_adam_matches_torch_optimizer():
    n = 5000
    start = synth.normal(9, 'params', n).astype(np.float32)
    reference = torch.nn.Parameter(torch.from_numpy(start.copy()))
    torch_opt = torch.optim.Adam([reference], lr=1e-3, betas=(.9, .999), eps=1e-15, foreach=False)
    master = torch.from_numpy(start.copy()).cuda()
    opt = FusedAdam(master, lr=1e-3)
    for t in range(5):
        g = torch.from_numpy(synth.normal(20 + t, 'grad', n).astype(np.float32))
        reference.grad = g / 128.0
        torch_opt.step()
        opt.step((g).cuda(), loss_scale=128.0)
    assert torch.allclose(master.cpu(), reference.detach(), rtol=1e-5, atol=1e-7)
