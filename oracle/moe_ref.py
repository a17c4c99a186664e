"""Torch-CPU restatement of the reference's MXFP4 MoE step (test infrastructure).

This is the checker, not the product. Only tests, the smoke entry and the
benchmark's CPU-baseline leg import it.

Each function names the reference lines it restates. The op chain, casts
and summation order follow the reference so that ``moe_step(..., fp32=False)``
is the BF16 serving oracle and ``moe_step(..., fp32=True)`` the FP32 truth
that the band grader measures against (megabench/tasks/kimi.py:239-240,
410-411).

Deliberate, documented choices where the reference leaves something open:
  * top-k ties: lowest expert index wins (stable descending sort). The
    reference calls ``torch.topk`` (kimi.py:310), whose tie order is
    unspecified; its softmax variant uses a stable argsort
    (distributed.py:175), which is this rule.
  * the SiLU variant is applied as an activation functor in FP32 followed
    by one cast, mirroring how ``situ`` is used (kimi.py:322); the Qwen
    oracle rounds ``F.silu`` and the product separately in BF16
    (distributed.py:184).

Independent pins (tests/test_oracle.py): the decode is checked bit for bit
against the C restatement in mxfp4_ref.c (bit construction from the OCP MX
E2M1/E8M0 definition) and against the closed form; the FP32 chain is checked
against ``moe_step_f64``, a float64 brute force written per token rather than
per expert, with a closed-form decode and its own activation formulas; the
BF16 chain against ``moe_step_bf16_f64``, the same brute force rounded to
bf16 (nearest, ties to even, ``bf16_round_f64``) exactly where kimi.py:322
casts, with planted dropped casts (through ``_expert_out``) that must fail it.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

# E2M1 code -> value (quantization.py:8-9). Codes 0-7 are positive, 8-15
# negative with the same magnitudes; code 8 is -0.0.
FP4_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)
MX_BLOCK = 32                                     # quantization.py:10

GATINGS = ('sigmoid_bias', 'softmax')
ACTIVATIONS = ('situ', 'silu')


def unpack_mxfp4(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """MXFP4 -> FP32, restating quantization.py:40-51.

    blocks u8 [..., K/32, 16], scales u8 [..., K/32] -> fp32 [..., K].
    Byte j of a block holds element 2j in its low nibble and 2j+1 in its high
    nibble (quantization.py:47). Value = FP4_VALUES[code] * 2**(scale-127)
    (quantization.py:48); scale byte 255 decodes every element of its block
    to NaN (quantization.py:50).
    """
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise ValueError("MXFP4 blocks and E8M0 scales must be uint8")
    if blocks.shape[:-1] != scales.shape or blocks.shape[-1] != MX_BLOCK // 2:
        raise ValueError("invalid MXFP4 block/scale geometry")
    lut = torch.tensor(FP4_VALUES, dtype=torch.float32)
    codes = torch.stack((blocks & 15, blocks >> 4), dim=-1).flatten(-2)
    decoded = torch.ldexp(lut[codes.long()], scales.int()[..., None] - 127)
    decoded = decoded.masked_fill(scales[..., None] == 255, torch.nan)
    return decoded.flatten(-2)


def situ(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """SiTU GLU activation in FP32 (kimi.py:194-196): 4 tanh(g/4) sigma(g) 25 tanh(u/25)."""
    gate, up = gate.float(), up.float()
    return 4*torch.tanh(gate/4)*gate.sigmoid()*(25*torch.tanh(up/25))


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """SiLU(g) * u in FP32 (the Qwen3-MoE variant, distributed.py:184)."""
    gate, up = gate.float(), up.float()
    return F.silu(gate)*up


def _activation(name: str):
    if name == 'situ':
        return situ
    if name == 'silu':
        return silu_mul
    raise ValueError(f"activation must be one of {ACTIVATIONS}, got {name!r}")


def _stable_topk_desc(values: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest per row, largest first, lowest index first on ties (NaN largest)."""
    return torch.sort(values, dim=-1, descending=True, stable=True).indices[..., :k]


def route(x: torch.Tensor, router: torch.Tensor, bias: torch.Tensor | None, topk: int,
          gating: str = 'sigmoid_bias', routes: torch.Tensor | None = None) -> dict:
    """Router logits, gating and top-k selection.

    sigmoid_bias restates kimi.py:308-316:
      scores = sigmoid(x.float() @ router.float().T); biased = scores + bias
      indices = top-k(biased); weights = scores[indices] / (sum + 1e-20)
      forced routes replace indices and report the shortfall (kimi.py:311-313).
    softmax restates distributed.py:174-176 batched over rows:
      logits = router.float() @ x.float(); selected = stable argsort desc [:k]
      weights = softmax(logits[selected]).
    Returns indices/weights in selection order (what the combine uses) plus
    expert_ids sorted ascending (kimi.py:316) and route_weights aligned to them.
    """
    if gating not in GATINGS:
        raise ValueError(f"gating must be one of {GATINGS}, got {gating!r}")
    logits = x.float() @ router.float().T                                   # kimi.py:308
    B, E = logits.shape
    out = {'logits': logits}
    if gating == 'sigmoid_bias':
        scores = logits.sigmoid()
        biased = scores + (bias.float() if bias is not None else 0.0)       # kimi.py:309
        best = _stable_topk_desc(biased, topk)                              # kimi.py:310
        indices = best
        if routes is not None:                                              # kimi.py:311-313
            indices = routes.to(dtype=torch.int64)
            kth = biased.gather(1, best)[:, -1]
            out['route_shortfall'] = (kth - biased.gather(1, indices).min(-1).values).clamp_min(0)
        weights = scores.gather(1, indices)                                 # kimi.py:314
        weights = weights/(weights.sum(-1, keepdim=True)+1e-20)             # kimi.py:315
        out['scores'], out['biased'] = scores, biased
    else:
        best = _stable_topk_desc(logits, topk)                              # distributed.py:175
        indices = best
        if routes is not None:
            indices = routes.to(dtype=torch.int64)
            kth = logits.gather(1, best)[:, -1]
            out['route_shortfall'] = (kth - logits.gather(1, indices).min(-1).values).clamp_min(0)
        weights = logits.gather(1, indices).softmax(-1)                     # distributed.py:176
    ids, order = indices.sort(-1)                                           # kimi.py:316
    out.update(indices=indices, weights=weights, expert_ids=ids,
               route_weights=weights.gather(1, order))
    return out


def moe_step(x, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
             down_blocks, down_scales, *, topk: int, gating: str = 'sigmoid_bias',
             activation: str = 'situ', fp32: bool = False, routes=None, latent=None,
             pair_out: bool = False) -> dict:
    """One MoE step on the CPU, restating kimi.py:307-324 (without the TP all-reduce).

    fp32=False is the BF16 serving oracle, fp32=True the FP32 truth
    (kimi.py:239-240). `latent` is the expert input when it differs from the
    router input (kimi.py:317); by default the experts read `x`.
    Returns expert_sum fp32 [B, K], expert_ids int64 [B, k] sorted,
    route_weights fp32 [B, k] aligned with expert_ids, and route_shortfall
    fp32 [B] when routes are forced; with pair_out, also 'pair_out' fp32
    [B, k, K]: each (token, expert) output (the down projection after its
    cast), in expert_ids order.
    """
    act = torch.float32 if fp32 else torch.bfloat16
    cast = lambda t: t.to(act)                                              # kimi.py:240
    fn = _activation(activation)
    r = route(x, router, router_bias, topk, gating, routes)
    indices, weights = r['indices'], r['weights']
    inp = cast(latent if latent is not None else x)
    B, K = inp.shape
    expert_sum = torch.zeros(B, K, dtype=torch.float32)                     # kimi.py:318
    pairs = torch.zeros(B, indices.shape[1], K, dtype=torch.float32) if pair_out else None
    for expert in indices.unique().tolist():                                # kimi.py:319
        rows, slots = (indices == expert).nonzero(as_tuple=True)            # kimi.py:320
        wg = unpack_mxfp4(gate_blocks[expert], gate_scales[expert]).to(act) # kimi.py:321
        wu = unpack_mxfp4(up_blocks[expert], up_scales[expert]).to(act)
        wd = unpack_mxfp4(down_blocks[expert], down_scales[expert]).to(act)
        out = _expert_out(inp[rows], wg, wu, wd, fn, cast)                  # kimi.py:322
        expert_sum.index_add_(0, rows, out.float()*weights[rows, slots, None])  # kimi.py:323
        if pairs is not None:
            pairs[rows, slots] = out.float()
    result = {'expert_sum': expert_sum, 'expert_ids': r['expert_ids'],
              'route_weights': r['route_weights']}
    if routes is not None:
        result['route_shortfall'] = r['route_shortfall']
    if pairs is not None:   # per (token, slot) expert output, aligned with expert_ids
        order = indices.sort(-1).indices
        result['pair_out'] = pairs.gather(1, order[..., None].expand(-1, -1, K))
    return result


def _expert_out(rows_inp, wg, wu, wd, fn, cast):
    """One expert's output rows, with the casts of kimi.py:322:
    cast(cast(act(inp @ wg.T, inp @ wu.T)) @ wd.T), where each matmul of
    activation-dtype operands returns the activation dtype."""
    hidden = cast(fn(rows_inp @ wg.T, rows_inp @ wu.T))
    return cast(hidden @ wd.T)


# ------------------------------------------------------------ float64 pin --

def _decode_f64(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Closed-form OCP MX decode in float64, independent of FP4_VALUES.

    E2M1: sign bit 3, exponent bits 2..1, mantissa bit 0; exponent 0 is
    subnormal (m * 0.5), else 2**(e-1) * (1 + m/2). E8M0: 2**(s-127), 255 = NaN.
    """
    lo, hi = blocks & 15, blocks >> 4
    codes = np.stack((lo, hi), axis=-1).reshape(*blocks.shape[:-1], MX_BLOCK).astype(np.int64)
    sign = np.where(codes & 8, -1.0, 1.0)
    e, m = (codes >> 1) & 3, codes & 1
    mag = np.where(e == 0, m*0.5, np.ldexp(1.0 + m/2.0, (e - 1).astype(np.int32)))
    scale = np.ldexp(1.0, scales.astype(np.int32) - 127)[..., None]
    value = sign*mag*scale
    value = np.where((scales == 255)[..., None], np.nan, value)
    return value.reshape(*blocks.shape[:-2], -1)


def moe_step_f64(x, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                 down_blocks, down_scales, *, routes, weights, activation='situ', latent=None):
    """Float64 brute force of the expert part for given routes and weights.

    Written per token (not per expert) with a closed-form decode, so that a
    dropped term, a sign, an index or a transposed operand in the restated
    chain shows up as a large distance. Returns expert_sum float64 [B, K].
    """
    inp = (latent if latent is not None else x).double().numpy()
    routes = routes.numpy()
    weights = weights.double().numpy()
    B, K = inp.shape
    out = np.zeros((B, K))
    cache = {}
    for b in range(B):
        for slot in range(routes.shape[1]):
            e = int(routes[b, slot])
            if e not in cache:
                cache[e] = tuple(_decode_f64(blk[e].numpy(), scl[e].numpy()) for blk, scl in
                                 ((gate_blocks, gate_scales), (up_blocks, up_scales), (down_blocks, down_scales)))
            wg, wu, wd = cache[e]
            g = wg @ inp[b]
            u = wu @ inp[b]
            if activation == 'situ':
                a = 4.0*np.tanh(g/4.0)*(1.0/(1.0 + np.exp(-g)))*25.0*np.tanh(u/25.0)
            else:
                a = g/(1.0 + np.exp(-g))*u
            out[b] += weights[b, slot]*(wd @ a)
    return out


def bf16_round_f64(v) -> np.ndarray:
    """Round float64 values to the nearest bfloat16 value, ties to even, returned as float64.

    bfloat16 keeps 8 significant bits: with v = m 2**e, 0.5 <= |m| < 1
    (frexp), the result is rint(m 2**8) 2**(e-8); numpy's rint rounds half to
    even. Valid for the normal bf16 range (|v| >= 2**-126), which the
    projections here stay in; zeros, infinities and NaN pass through.
    """
    v = np.asarray(v, dtype=np.float64)
    m, e = np.frexp(v)
    with np.errstate(invalid='ignore'):
        r = np.ldexp(np.rint(np.ldexp(m, 8)), e - 8)
    return np.where(np.isfinite(v), r, v)


def moe_step_bf16_f64(x, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                      down_blocks, down_scales, *, routes, weights, activation='situ', latent=None):
    """Float64 brute force of the BF16 serving chain for given routes and weights.

    Written per token like moe_step_f64, with a closed-form decode, and rounded
    to bf16 (bf16_round_f64) exactly where kimi.py:322 casts in BF16 mode:
    the gate and up projections, the activation, the down projection. The
    combine is a float64 sum of weight x bf16 output (kimi.py:323). It differs
    from the BF16 oracle only by FP32-versus-float64 arithmetic inside the dot
    products and the activation, which flips a bf16 rounding rarely; a dropped
    or added cast moves every value by about a rounding step.
    Returns expert_sum float64 [B, K].
    """
    inp = (latent if latent is not None else x).double().numpy()
    routes = routes.numpy()
    weights = weights.double().numpy()
    B, K = inp.shape
    out = np.zeros((B, K))
    cache = {}
    for b in range(B):
        for slot in range(routes.shape[1]):
            e = int(routes[b, slot])
            if e not in cache:
                cache[e] = tuple(_decode_f64(blk[e].numpy(), scl[e].numpy()) for blk, scl in
                                 ((gate_blocks, gate_scales), (up_blocks, up_scales), (down_blocks, down_scales)))
            wg, wu, wd = cache[e]
            g = bf16_round_f64(wg @ inp[b])
            u = bf16_round_f64(wu @ inp[b])
            if activation == 'situ':
                a = 4.0*np.tanh(g/4.0)*(1.0/(1.0 + np.exp(-g)))*25.0*np.tanh(u/25.0)
            else:
                a = g/(1.0 + np.exp(-g))*u
            y = bf16_round_f64(wd @ bf16_round_f64(a))
            out[b] += weights[b, slot]*y
    return out


def router_f64(x, router, bias, gating='sigmoid_bias') -> np.ndarray:
    """Float64 router scores used to certify top-k near-ties: biased sigmoid or raw logits."""
    logits = x.double().numpy() @ router.double().numpy().T
    if gating == 'softmax':
        return logits
    scores = 1.0/(1.0 + np.exp(-logits))
    return scores + (bias.double().numpy() if bias is not None else 0.0)


def rel_l2(a, b) -> float:
    """||a - b|| / ||b|| in float64 (the band's distance, kimi.py:420-424)."""
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    return math.sqrt(float((a - b).square().sum()) / max(float(b.square().sum()), 1e-30))
