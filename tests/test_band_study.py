"""Band study: may the prefill step feed the scaled FP4 MFMA with 8-bit activations?

The f8f6f4 MFMA multiplies E2M1 weights (with their E8M0 block scales) by
8-bit operands, so its activations (the expert input rows for gate/up, h for
down) must be quantised. The reference allows other precisions when the
result stays in the band (megabench/integrations/make_kimi_workspace.py:55-56;
band of kimi.py:413-429: rel-L2(candidate, FP32 truth) <= 2 rel-L2(BF16
oracle, FP32 truth) + 0.002). This CPU study models the step with each
activation format in place of the BF16 operands, everything else as the BF16
oracle (fp32 accumulation, bf16 casts of kimi.py:322), on a prefill-shaped
layer (about 32 tokens per expert):

  mxfp8       one E4M3 value per element, one E8M0 scale per 32 (OCP MX:
              2^(floor(log2 amax) - 8), values clamped to 448), round to nearest;
  mxfp8-hilo  two terms: hi = E4M3 of x with scale 2^(floor(log2 amax) - 7),
              lo = E4M3 of the remainder x - hi with its own block scale; the
              MFMA runs twice (hi, lo) into one fp32 accumulator. A bf16 value
              has 8 significant bits and E4M3 4, so hi + lo is exact for every
              element within 2^9 of its block maximum (smaller ones lose only
              bits below 2^-17 of the block maximum).

Result (seed 0, B=128, E=16, top-4, h=2048, I=512; the printed table):
mxfp8 is far outside the band (rel-L2 5.5e-2, ratio 6.9); mxfp8-hilo gives
the BF16 oracle's own error (rel-L2 2.985e-3, ratio 0.375, the same as the
bf16 model to 4 digits), so the FP4 MFMA path uses the two-term split.
"""

import pytest
import torch

from k3moe import synthetic
from k3moe.configs import MoEConfig
from oracle import grading, moe_ref


def mx_e4m3(v: torch.Tensor, shift: int) -> torch.Tensor:
    """E4M3 values with one power-of-two scale 2^(floor(log2 amax) - shift) per block of 32,
    round to nearest even, clamped to +-448; returned dequantised (fp32)."""
    g = v.float().unflatten(-1, (-1, 32))
    amax = g.abs().amax(-1, keepdim=True)
    e = torch.where(amax > 0, torch.floor(torch.log2(amax)) - shift, torch.zeros_like(amax))
    q = torch.ldexp(g, -e.int()).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    return torch.ldexp(q, e.int()).flatten(-2)


def quantise(v: torch.Tensor, fmt: str) -> torch.Tensor:
    if fmt == 'bf16':
        return v.float()
    if fmt == 'mxfp8':
        return mx_e4m3(v, 8)
    if fmt == 'mxfp8-hilo':
        hi = mx_e4m3(v, 7)
        return hi + mx_e4m3(v.float() - hi, 7)
    raise ValueError(fmt)


def step_with(inputs, cfg, fmt):
    """The BF16 oracle's step (oracle/moe_ref.py) with the activation operands in `fmt`."""
    bf = torch.bfloat16
    r = moe_ref.route(inputs['x'], inputs['router'], inputs['router_bias'], cfg.topk, cfg.gating)
    idx, wts = r['indices'], r['weights']
    inp = inputs['x']
    out = torch.zeros(inp.shape, dtype=torch.float32)
    for e in idx.unique().tolist():
        rows, slots = (idx == e).nonzero(as_tuple=True)
        wg = moe_ref.unpack_mxfp4(inputs['gate_blocks'][e], inputs['gate_scales'][e])
        wu = moe_ref.unpack_mxfp4(inputs['up_blocks'][e], inputs['up_scales'][e])
        wd = moe_ref.unpack_mxfp4(inputs['down_blocks'][e], inputs['down_scales'][e])
        a = quantise(inp[rows], fmt)
        h = moe_ref.situ((a @ wg.T).to(bf), (a @ wu.T).to(bf)).to(bf)
        y = (quantise(h, fmt) @ wd.T).to(bf)
        out.index_add_(0, rows, y.float()*wts[rows, slots, None])
    return out, r['expert_ids']


@pytest.fixture(scope='module')
def study():
    cfg = MoEConfig('band-study', 16, 4, 2048, 512, 128)
    inputs = synthetic.moe_layer_inputs(cfg, 0)
    args = synthetic.step_args(inputs)
    kw = dict(topk=cfg.topk, gating=cfg.gating)
    oracle = moe_ref.moe_step(*args, **kw)
    truth = moe_ref.moe_step(*args, **kw, fp32=True)
    rows = {}
    for fmt in ('bf16', 'mxfp8', 'mxfp8-hilo'):
        got, ids = step_with(inputs, cfg, fmt)
        assert torch.equal(ids, oracle['expert_ids'])
        err = grading.rel_l2(got, truth['expert_sum'])
        limit = 2*grading.rel_l2(oracle['expert_sum'], truth['expert_sum']) + 0.002
        rows[fmt] = {'rel_l2': err, 'ratio': err/limit, 'vs_oracle': grading.rel_l2(got, oracle['expert_sum'])}
    print('\nformat       rel-L2 vs FP32   band ratio   rel-L2 vs BF16 oracle')
    for fmt, d in rows.items():
        print(f'{fmt:12s} {d["rel_l2"]:.3e}        {d["ratio"]:.3f}        {d["vs_oracle"]:.3e}')
    return rows, inputs


def test_bf16_model_is_the_oracle(study):
    rows, _ = study
    assert rows['bf16']['vs_oracle'] < 5e-4     # fp32 products rounded once vs torch's bf16 matmul: a few flips


def test_single_term_mxfp8_leaves_the_band(study):
    rows, _ = study
    assert rows['mxfp8']['ratio'] > 1.5


def test_two_term_mxfp8_stays_with_the_oracle(study):
    rows, _ = study
    assert rows['mxfp8-hilo']['ratio'] < 0.5
    assert abs(rows['mxfp8-hilo']['ratio'] - rows['bf16']['ratio']) < 0.01
    assert rows['mxfp8-hilo']['vs_oracle'] < 2e-3


def test_two_term_split_is_exact_on_bf16_values(study):
    _, inputs = study
    x = inputs['x'].float()
    hi = mx_e4m3(x, 7)
    lo = mx_e4m3(x - hi, 7)
    exact = (hi + lo) == x
    g = x.abs().unflatten(-1, (-1, 32))
    near = (g >= g.amax(-1, keepdim=True)*2.0**-8).flatten(-2)
    assert bool(exact[near].all())
    assert float(exact.float().mean()) > 0.99
