"""CPU restatement of the reference's MXFP4 encoder (test infrastructure).

This is the checker, not the product: only tests and the benchmark's
CPU-baseline leg import it.

``pack_mxfp4`` restates megabench/tasks/quantization.py:13-37 with the same
torch CPU op chain (fp32 throughout):

    maximum  = |x|.amax over each block of 32                      (:24)
    exponent = ceil(log2(max(maximum / 6, 2^-126))), clamped to
               [-126, 127]                                         (:25-26)
    normal   = ldexp(x, -exponent)                                 (:27)
    code     = bucketize(|normal|, (0.25, 0.75, 1.25, 1.75, 2.5,
               3.5, 5.0)) + 1 at the ties 0.75, 1.75, 3.5, whose
               lower code is odd                                   (:28-34)
               | 8 when normal < 0                                 (:35)
    packed   = code[even] | code[odd] << 4, scale = exponent + 127 (:36-37)

Two properties of that chain the device encoder has to reproduce, and which
``pack_mxfp4_f64`` (an independent brute force) states explicitly:
  * torch's fp32 ``log2`` is rounded to the nearest fp32, so for a quotient a
    few ulps above a power of two 2^n the logarithm rounds to n itself and the
    ceiling keeps n (the exact ceiling would be n + 1);
  * a block holding a NaN has a NaN maximum, whose conversion to int32 on x86
    gives INT_MIN: the scale byte wraps to 127 and ldexp scales by 2^INT_MIN
    = 0, so NaN elements (and infinities) take code 7 and finite ones code 0.

Independent pins (tests/test_oracle_pack.py): ``pack_mxfp4_f64`` chooses the
nearest E2M1 magnitude by distance in float64 with ties to the even code,
and the exponent from a float64 log2 rounded once to fp32; hand-computed
codes at every rounding boundary and one float32 step either side; the
exponent at 2^n (1 + j 2^-23) for every n and j < 64; decode(encode(v)) == v
for every value the decoder produces.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle.moe_ref import FP4_VALUES, MX_BLOCK

BOUNDARIES = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)     # quantization.py:29-30


def pack_mxfp4(matrix: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Encode contiguous groups of 32 along the last axis (quantization.py:13-37).

    matrix [..., K] (any float dtype) -> packed u8 [..., K/32, 16], scales u8 [..., K/32].
    """
    if matrix.shape[-1] % MX_BLOCK:
        raise ValueError("MXFP4 block axis must be divisible by 32")
    groups = matrix.float().unflatten(-1, (-1, MX_BLOCK))
    maximum = groups.abs().amax(-1)
    exponent = torch.ceil(torch.log2((maximum/6.0).clamp_min(2.0**-126)))
    exponent = exponent.clamp(-126, 127).to(torch.int32)
    normalized = torch.ldexp(groups, -exponent[..., None])
    absolute = normalized.abs().contiguous()
    index = torch.bucketize(absolute, torch.tensor(BOUNDARIES))
    odd_tie = (absolute == 0.75) | (absolute == 1.75) | (absolute == 3.5)
    index = index + odd_tie.to(index.dtype)
    code = (index | ((normalized < 0).to(index.dtype) << 3)).to(torch.uint8)
    packed = code[..., 0::2] | (code[..., 1::2] << 4)
    return packed, (exponent + 127).to(torch.uint8)


def block_exponent_f64(maximum: np.ndarray) -> np.ndarray:
    """The encoder's block exponent from float32 block maxima, without torch.

    The quotient maximum / 6 is the IEEE float32 quotient (numpy float32
    division), floored at 2^-126; its base-2 logarithm is taken in float64 and
    rounded once to float32 (a correctly rounded fp32 log2), then the ceiling,
    clamped to [-126, 127]. Infinite maxima give 127. NaN maxima are the
    caller's (they have no exponent; see pack_mxfp4_f64).
    """
    m = np.asarray(maximum, dtype=np.float32)
    with np.errstate(over='ignore', invalid='ignore'):
        v = np.maximum(m/np.float32(6.0), np.float32(2.0**-126))
        lg = np.log2(v.astype(np.float64)).astype(np.float32)
    e = np.where(np.isinf(v), 127.0, np.ceil(lg.astype(np.float64)))
    return np.clip(np.nan_to_num(e, nan=0.0), -126, 127).astype(np.int64)


def pack_mxfp4_f64(matrix) -> tuple[np.ndarray, np.ndarray]:
    """Brute-force MXFP4 encoder: nearest E2M1 magnitude by distance, ties to the even code.

    Same contract as pack_mxfp4 (numpy in, numpy out). The block-normalised
    value is the float32 product x * 2^-e (subnormal results rounded, as the
    reference's ldexp rounds them); its code is the c in 0..7 minimising
    |a - FP4_VALUES[c]| computed in float64, the even c on an exact tie
    (magnitudes above 6 take code 7), plus 8 when the product is negative.
    NaN blocks follow the reference on x86 (module docstring).
    """
    x = np.asarray(matrix, dtype=np.float32)
    if x.shape[-1] % MX_BLOCK:
        raise ValueError("MXFP4 block axis must be divisible by 32")
    g = x.reshape(*x.shape[:-1], -1, MX_BLOCK)
    nan_block = np.isnan(g).any(-1)
    with np.errstate(invalid='ignore'):
        maximum = np.where(nan_block, np.float32(0), np.abs(g).max(-1, initial=np.float32(0)))
    e = block_exponent_f64(maximum)
    scale = np.where(nan_block, 127, e + 127).astype(np.uint8)
    step = np.ldexp(np.float32(1.0), (-e).astype(np.int32)).astype(np.float32)     # 2^-e, exact in float32
    step = np.where(nan_block, np.float32(0.0), step)
    with np.errstate(invalid='ignore', under='ignore', over='ignore'):
        normal = (g*step[..., None]).astype(np.float32)
    mags = np.array(FP4_VALUES[:8], dtype=np.float64)
    a = np.abs(normal.astype(np.float64))
    dist = np.abs(a[..., None] - mags)                   # [..., 32, 8]
    best = dist.min(-1, keepdims=True)
    tied = dist == best
    even_first = np.where(tied[..., 0::2].any(-1), np.argmax(tied[..., 0::2], -1)*2, np.argmax(tied, -1))
    code = np.where(np.isnan(a), 7, np.where(a > 6.0, 7, even_first)).astype(np.uint8)
    code = code | np.where(normal < 0, 8, 0).astype(np.uint8)
    packed = (code[..., 0::2] | (code[..., 1::2] << 4)).astype(np.uint8)
    return packed, scale
