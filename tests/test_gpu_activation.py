"""The expert GEMMs' activation on the GPU against a float64 reference (run with -m gpu).

SiTU (kimi.py:194-196): 4 tanh(g/4) sigmoid(g) 25 tanh(u/25); SiLU (tasks/distributed.py:184):
g sigmoid(g) u. Both forms the kernels use are pinned: the library-function form (expf, tanhf;
the decode kernels) and the exponential-and-reciprocal form (the prefill GEMM's epilogue). The
inputs are bf16 values, as the kernels feed them (the activations of bf16-rounded gate and up
sums): every bf16 magnitude from 2^-30 to 128 at both signs against a spread of partners, plus
exact zeros. Bars: relative error to float64 (a floor of 2^-80 for values near underflow), and
for the fast form the fraction of bf16(h) equal to the library form's (h is rounded to bf16 next,
kimi.py:322).
"""

import numpy as np
import pytest
import torch

from k3moe import moe

pytestmark = pytest.mark.gpu


def bf16_grid():
    """Every bf16 value with |v| in [2^-30, 128], both signs, and zero."""
    bits = np.arange(0, 1 << 15, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    v = v[(v >= 2.0 ** -30) & (v <= 128.0)]
    return np.concatenate([v, -v, [0.0]]).astype(np.float32)


def reference(act, g, u):
    g, u = g.astype(np.float64), u.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g))
    if act == 'situ':
        return 4.0 * np.tanh(g / 4.0) * sig * 25.0 * np.tanh(u / 25.0)
    return g * sig * u


@pytest.mark.parametrize('act', ['situ', 'silu'])
def test_activation_forms_against_float64(gpu, act):
    grid = bf16_grid()
    rng = np.random.default_rng(7)
    g = np.concatenate([grid, rng.choice(grid, grid.size)])
    u = np.concatenate([rng.choice(grid, grid.size), grid])
    print(f'case: activation {act}, {g.size} pairs', flush=True)
    want = reference(act, g, u)
    gt, ut = torch.from_numpy(g).to(gpu), torch.from_numpy(u).to(gpu)
    lib = moe.activation(gt, ut, act, fast=False).cpu().numpy().astype(np.float64)
    fast = moe.activation(gt, ut, act, fast=True).cpu().numpy().astype(np.float64)
    scale = np.maximum(np.abs(want), 2.0 ** -80)   # (below it: sigmoids near the fp32 underflow)
    err_lib, err_fast = np.abs(lib - want) / scale, np.abs(fast - want) / scale
    print(f'   max rel error: library {err_lib.max():.3g}, fast {err_fast.max():.3g}', flush=True)
    assert err_lib.max() <= 2e-6        # a few fp32 ulps through the operation chain
    assert err_fast.max() <= 4e-6
    to_bf16 = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)
    same = float((to_bf16(fast) == to_bf16(lib)).double().mean())
    assert same >= 0.999, same
    assert np.all(np.isfinite(fast)) and np.all(fast[(g == 0) | (u == 0)] == 0)
