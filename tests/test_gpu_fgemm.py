"""GPU checks of the grouped GEMMs on the scaled FP4 MFMA (run with -m gpu).

The prefill-sized general path feeds v_mfma_scale_f32_16x16x128_f8f6f4 with the
MXFP4 weights as stored and the activations split into two E4M3 terms with
E8M0 block scales (tests/test_band_study.py: the split represents the bf16
values, one term alone leaves the band). Checks:
  * the split the step leaves in the workspace (the expert inputs) equals a
    torch model of its definition bit for bit: hi = E4M3(v / 2^eh), eh =
    floor(log2 max|v|) - 7 per block of 32, lo the same on v - hi 2^eh (torch's
    float8_e4m3fn conversion rounds to nearest even);
  * hi 2^eh + lo 2^el reproduces every input value within 2^8 of its block's
    maximum exactly, and the smaller ones to 2^-16 of the maximum;
  * the split h follows its definition on the h it represents (hi scale and
    the hi bytes of values within 2^8 of the block maximum), and that h equals the BF16 oracle's
    act(bf16(gate), bf16(up)) for at least 95 % of the sampled elements, the
    rest within two bf16 rounding steps (a flipped rounding of gate or up) or,
    for values far below their block's maximum, within the split's floor of
    2^-15 of that maximum;
  * end to end, the FP4-MFMA path and the bf16-MFMA grouped path agree with
    the oracle (expert sets, band, per-element) and with each other.
"""

import pytest
import torch

import k3moe
from k3moe import synthetic
from k3moe.configs import MoEConfig
from k3moe.moe import dims_for, workspace_bytes, workspace_layout
from oracle import moe_ref

pytestmark = pytest.mark.gpu

CASE = MoEConfig('fgemm-b512', 32, 4, 1024, 1024, 512, gating='softmax')   # ~64 tokens per expert


def say(*a):
    print(*a, flush=True)


def split_model(v: torch.Tensor):
    """Two-term E4M3 split of fp32 values [N, K] (bf16-exact), blocks of 32 along K."""
    g = v.float().unflatten(-1, (-1, 32))

    def term(x):
        amax = x.abs().amax(-1)
        be = (amax.view(torch.int32) >> 23) & 255
        s = torch.where(be > 7, be - 7, torch.zeros_like(be))
        q = (x*torch.ldexp(torch.ones_like(amax), 127 - s)[..., None]).to(torch.float8_e4m3fn)
        back = q.float()*torch.ldexp(torch.ones_like(amax), s - 127)[..., None]
        return q, s.to(torch.uint8), back

    hi, sh, bh = term(g)
    lo, sl, bl = term(g - bh)
    return hi.flatten(-2).view(torch.uint8), lo.flatten(-2).view(torch.uint8), sh, sl, bh + bl


def run_step(cfg, seed, dev, path):
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in synthetic.moe_layer_inputs(cfg, seed).items()}
    dims = dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating, cfg.activation,
                    None, path)
    ws = k3moe.new_workspace(workspace_bytes(dims), dev)
    got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, gating=cfg.gating, path=path, workspace=ws)
    torch.cuda.synchronize(dev)
    assert k3moe.workspace_status(ws) == 0
    return g, got, ws, workspace_layout(dims)


def test_input_split_matches_its_definition(gpu):
    cfg = CASE
    say(f'case: {cfg.name} seed=3 path=grouped, expert-input split from the workspace')
    g, got, ws, lay = run_step(cfg, 3, gpu, 'grouped')
    assert lay['input_split'] >= 0 and lay['h_split'] >= 0 and lay['pair_h'] == -1
    B, K = cfg.tokens, cfg.width
    raw = ws.cpu()
    o = lay['input_split']
    hi = raw[o:o + B*K].view(B, K)
    lo = raw[o + B*K:o + 2*B*K].view(B, K)
    sh = raw[o + 2*B*K:o + 2*B*K + B*K//32].view(B, K//32)
    sl = raw[o + 2*B*K + B*K//32:o + 2*B*K + 2*(B*K//32)].view(B, K//32)
    mh, ml, msh, msl, back = split_model(g['x'].cpu().float())
    assert torch.equal(sh, msh)
    assert torch.equal(sl, msl)
    assert torch.equal(hi, mh)
    assert torch.equal(lo, ml)
    # hi + lo is exact for every value within 2^8 of its block's maximum, and off by less than
    # 2^-16 of the maximum for the smaller ones
    x = g['x'].cpu().float().unflatten(-1, (-1, 32))
    amax = x.abs().amax(-1, keepdim=True)
    near = x.abs() >= amax*2.0**-8
    assert torch.equal(back[near], x[near])
    assert bool(((back - x).abs() <= amax*2.0**-16).all())


def test_h_split_is_the_oracle_activation(gpu):
    cfg = CASE
    say(f'case: {cfg.name} seed=4 path=grouped, h split against the oracle on 6 pairs')
    g, got, ws, lay = run_step(cfg, 4, gpu, 'grouped')
    P, I = cfg.tokens*cfg.topk, cfg.inter
    raw = ws.cpu()
    o = lay['h_split']
    hi = raw[o:o + P*I].view(P, I)
    lo = raw[o + P*I:o + 2*P*I].view(P, I)
    sh = raw[o + 2*P*I:o + 2*P*I + P*I//32].view(P, I//32)
    sl = raw[o + 2*P*I + P*I//32:o + 2*P*I + 2*(P*I//32)].view(P, I//32)
    scale = lambda s: torch.ldexp(torch.ones(s.shape), s.long() - 127).repeat_interleave(32, -1)   # noqa: E731
    h = hi.view(torch.float8_e4m3fn).float()*scale(sh) + lo.view(torch.float8_e4m3fn).float()*scale(sl)
    # h (SiTU outputs) has many values far below its block maximum; those within 2^8 of it are
    # represented exactly, so the block maximum is, and the hi scale and the hi bytes of those
    # values follow the definition
    blk = h.abs().unflatten(-1, (-1, 32))
    near = (blk >= blk.amax(-1, keepdim=True)*2.0**-8).flatten(-2)
    assert torch.equal(h[near].to(torch.bfloat16).float(), h[near])
    mh, _, msh, _, _ = split_model(h)
    assert torch.equal(msh, sh)
    assert torch.equal(mh[near], hi[near])
    # against the oracle's h of the same pairs: act(bf16(x wg), bf16(x wu)) in bf16
    ptok = raw[lay['pair_token']:lay['pair_token'] + 4*P].view(torch.int32).long()
    act = raw[lay['active']:lay['active'] + 4*cfg.experts].view(torch.int32).long()
    off = raw[lay['offsets']:lay['offsets'] + 4*cfg.experts].view(torch.int32).long()
    D = int(raw[lay['active_count']:lay['active_count'] + 4].view(torch.int32)[0])
    same = total = 0
    for d in (0, D//2, D - 1):
        e = int(act[d])
        wg = moe_ref.unpack_mxfp4(g['gate_blocks'][e].cpu(), g['gate_scales'][e].cpu()).to(torch.bfloat16)
        wu = moe_ref.unpack_mxfp4(g['up_blocks'][e].cpu(), g['up_scales'][e].cpu()).to(torch.bfloat16)
        for p in (int(off[d]), int(off[d]) + 1):
            xr = g['x'][ptok[p]].cpu()[None]
            ref = moe_ref.situ(xr @ wg.T, xr @ wu.T).to(torch.bfloat16).float()[0]
            diff = (h[p] - ref).abs()
            ulp = torch.ldexp(torch.ones(I), torch.frexp(ref)[1] - 8)
            floor = (h[p].abs().unflatten(-1, (-1, 32)).amax(-1, keepdim=True)*2.0**-15).expand(-1, 32).flatten()
            assert bool((diff <= 2*ulp*1.0001 + floor).all()), (d, p, float(diff.max()))
            same += int((diff == 0).sum())
            total += I
    assert same >= 0.95*total, same/total


@pytest.mark.parametrize('seed', [0, 5])
def test_fp4_and_bf16_grouped_gemms_agree(gpu, seed):
    """Same routing, same grouping: the two grouped-GEMM variants differ only in fp32 summation order."""
    cfg = CASE
    say(f'case: {cfg.name} seed={seed} grouped (FP4 MFMA) vs grouped_bf16')
    outs = {p: run_step(cfg, seed, gpu, p)[1] for p in ('grouped', 'grouped_bf16')}
    a, b = outs['grouped'], outs['grouped_bf16']
    assert torch.equal(a['expert_ids'], b['expert_ids'])
    assert torch.equal(a['route_weights'], b['route_weights'])
    assert bool(torch.isfinite(a['expert_sum']).all())
    assert moe_ref.rel_l2(a['expert_sum'].cpu(), b['expert_sum'].cpu()) < 2e-3
