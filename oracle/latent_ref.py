"""Torch-CPU restatement of the latent MoE block around the routed experts (test infrastructure).

This is the checker, not the product. Only tests, the smoke entry and the
benchmark's CPU-baseline leg import it.

The block of megabench/tasks/kimi.py:317-328 for one MoE layer, without the
TP all-reduces (``sum_value`` is the identity on one GPU, kimi.py:238):

    latent = project(latent_down, normalized)                          kimi.py:317
    expert_sum = routed experts of latent                               kimi.py:318-324 (moe_ref.moe_step)
    routed = project(latent_up, rms(cast(expert_sum), latent_norm, eps=1e-5))   kimi.py:325
    shared = project(shared_down, cast(situ(project(shared_gate, normalized),
                                            project(shared_up, normalized))))   kimi.py:326-327
    output = routed + cast(shared)                                      kimi.py:328

with project(W, x) = cast(x) @ cast(W).T (kimi.py:246-247), cast = .to(act)
(kimi.py:240), situ (kimi.py:194-196) and rms (common.py:13-21, neither the
Gemma offset nor an FP32 weight: the normalized value is cast to the
activation dtype before the weight multiply). fp32=False is the BF16 serving
oracle, fp32=True the FP32 truth (kimi.py:239-240).

Pin (tests/test_oracle.py): ``latent_in_f64`` and ``latent_out_f64``, float64
brute forces written per token and per output row with their own RMS and SiTU
formulas, chained with moe_ref.moe_step_f64 for the whole block; the RMS
epsilon against the closed form of a constant vector; planted mistakes (gate
and up swapped, the norm weight dropped, the mean taken over tokens) fail.
The BF16 mode against ``latent_in_bf16_f64`` and ``latent_out_bf16_f64``, the
same brute forces rounded to bf16 where the chain casts, chained with
moe_ref.moe_step_bf16_f64; planted moved or dropped casts (unrounded
projections, the norm weight applied in FP32, the expert sum not cast) fail.
"""

from __future__ import annotations

import numpy as np
import torch

from .moe_ref import moe_step, situ

RMS_EPS = 1e-5  # kimi.py:325


def project(weight: torch.Tensor, x: torch.Tensor, act: torch.dtype) -> torch.Tensor:
    """cast(x) @ cast(weight).T (kimi.py:246-247)."""
    return x.to(act) @ weight.to(act).T


def rms(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMS norm in FP32, cast to x's dtype, then times the weight in x's dtype (common.py:13-21)."""
    xf = x.float()
    normalized = xf*torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
    return normalized.to(x.dtype)*weight.to(x.dtype)


def latent_in(normalized, latent_down, shared_gate, shared_up, *, fp32: bool = False):
    """The block's projections of the layer input: (latent [B, lh], shared activation [B, S]) (kimi.py:317, 326)."""
    act = torch.float32 if fp32 else torch.bfloat16
    latent = project(latent_down, normalized, act)
    shared_h = situ(project(shared_gate, normalized, act), project(shared_up, normalized, act)).to(act)
    return latent, shared_h


def latent_out(expert_sum, latent_norm, latent_up, shared_h, shared_down, *, fp32: bool = False):
    """routed + cast(shared) [B, h] from the experts' sum and the shared activation (kimi.py:325-328)."""
    act = torch.float32 if fp32 else torch.bfloat16
    routed = project(latent_up, rms(expert_sum.to(act), latent_norm, RMS_EPS), act)
    shared = project(shared_down, shared_h, act)
    return routed + shared.to(act)


def latent_block(normalized, w: dict, *, topk: int, gating: str = 'sigmoid_bias', fp32: bool = False,
                 routes=None) -> dict:
    """The whole block: latent_in, the routed experts on the latent, latent_out.

    `w` holds latent_down, latent_up, latent_norm, shared_gate, shared_up, shared_down, router,
    router_bias and the {gate,up,down}_{blocks,scales} expert tensors (kimi.py:112-121 names
    without the layer prefix).
    """
    latent, shared_h = latent_in(normalized, w['latent_down'], w['shared_gate'], w['shared_up'], fp32=fp32)
    moe = moe_step(normalized, w['router'], w.get('router_bias'), w['gate_blocks'], w['gate_scales'],
                   w['up_blocks'], w['up_scales'], w['down_blocks'], w['down_scales'], topk=topk,
                   gating=gating, fp32=fp32, routes=routes, latent=latent)
    output = latent_out(moe['expert_sum'], w['latent_norm'], w['latent_up'], shared_h, w['shared_down'],
                        fp32=fp32)
    return {'output': output, 'latent': latent, 'shared_h': shared_h, **moe}


def latent_out_f64(expert_sum, latent_norm, latent_up, shared_h, shared_down) -> np.ndarray:
    """Float64 brute force of latent_out, per token and per output row (RMS and products in float64)."""
    e = expert_sum.double().numpy()
    wn = latent_norm.double().numpy()
    wu = latent_up.double().numpy()
    sh = shared_h.double().numpy()
    wd = shared_down.double().numpy()
    B, lh = e.shape
    out = np.zeros((B, wu.shape[0]))
    for t in range(B):
        r = 1.0/np.sqrt(sum(v*v for v in e[t])/lh + RMS_EPS)
        en = [e[t, k]*r*wn[k] for k in range(lh)]
        for row in range(wu.shape[0]):
            out[t, row] = sum(wu[row, k]*en[k] for k in range(lh)) + sum(wd[row, j]*sh[t, j] for j in range(len(sh[t])))
    return out


def latent_in_f64(normalized, latent_down, shared_gate, shared_up):
    """Float64 brute force of latent_in, per token and per row (its own SiTU formula)."""
    x = normalized.double().numpy()
    wl, wg, wu = (m.double().numpy() for m in (latent_down, shared_gate, shared_up))
    B = x.shape[0]
    lat = np.array([[float(np.dot(wl[r], x[t])) for r in range(wl.shape[0])] for t in range(B)])
    sh = np.zeros((B, wg.shape[0]))
    for t in range(B):
        for j in range(wg.shape[0]):
            g, u = float(np.dot(wg[j], x[t])), float(np.dot(wu[j], x[t]))
            sh[t, j] = 4.0*np.tanh(g/4.0)/(1.0 + np.exp(-g))*25.0*np.tanh(u/25.0)
    return lat, sh


def latent_in_bf16_f64(normalized, latent_down, shared_gate, shared_up):
    """Float64 brute force of latent_in's BF16 mode, per token, rounded to bf16 where kimi.py:317, 326 cast.

    latent = bf16(x . latent_down row); shared_h = bf16(situ(bf16(x . gate row), bf16(x . up row)))
    with its own SiTU formula (moe_ref.bf16_round_f64: nearest bf16, ties to even).
    """
    from .moe_ref import bf16_round_f64 as r16
    x = normalized.double().numpy()
    wl, wg, wu = (m.double().numpy() for m in (latent_down, shared_gate, shared_up))
    lat = np.stack([r16(wl @ x[t]) for t in range(x.shape[0])])
    sh = []
    for t in range(x.shape[0]):
        g, u = r16(wg @ x[t]), r16(wu @ x[t])
        sh.append(r16(4.0*np.tanh(g/4.0)/(1.0 + np.exp(-g))*25.0*np.tanh(u/25.0)))
    return lat, np.stack(sh)


def latent_out_bf16_f64(expert_sum, latent_norm, latent_up, shared_h, shared_down) -> np.ndarray:
    """Float64 brute force of latent_out's BF16 mode, per token (kimi.py:325-328, common.py:13-21).

    e = bf16(expert_sum); en = bf16(bf16(e / sqrt(mean(e^2) + 1e-5)) * w_norm);
    routed = bf16(latent_up . en); shared = bf16(shared_down . shared_h);
    out = bf16(routed + shared): each rounding is where the BF16 chain casts.
    """
    from .moe_ref import bf16_round_f64 as r16
    e = r16(expert_sum.double().numpy())
    wn = latent_norm.double().numpy()
    wu, wd = latent_up.double().numpy(), shared_down.double().numpy()
    sh = shared_h.double().numpy()
    out = []
    for t in range(e.shape[0]):
        inv = 1.0/np.sqrt(np.mean(e[t]*e[t]) + RMS_EPS)
        en = r16(r16(e[t]*inv)*wn)
        out.append(r16(r16(wu @ en) + r16(wd @ sh[t])))
    return np.stack(out)
