"""Algorithmic bytes and FLOPs of one MoE step (the roofline's numerator).

Byte model after megabench/sol.py:23-24 (MXFP4 r x c = r c/2 + r c/32) and
sol.py:42-43 (expected distinct experts under uniform routing); the benchmark
uses the distinct count of the actual routing instead of the expectation.
"""

from __future__ import annotations

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E peak, GB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
MFMA_FP4_PEAK_TFLOPS = 10100.0  # MI355X dense MXFP4 MFMA


def mxfp4_bytes(rows: int, cols: int) -> int:
    """Packed MXFP4 bytes of a rows x cols matrix (sol.py:23-24)."""
    return rows*cols//2 + rows*cols//32


def expected_distinct(E: int, k: int, B: int) -> float:
    """E (1 - (1 - k/E)^B), the expected distinct experts of B uniform top-k draws (sol.py:42-43)."""
    return E*(1.0 - (1.0 - k/E)**B)


def expert_bytes(I: int, K: int) -> int:
    """Gate + up [I, K] and down [K, I] of one expert in MXFP4."""
    return 2*mxfp4_bytes(I, K) + mxfp4_bytes(K, I)


def step_bytes(*, B: int, E: int, k: int, h: int, I: int, distinct: int, K: int | None = None) -> int:
    """Router E h bf16 + bias E fp32 + x B h bf16 (+ latent B K bf16) + distinct experts
    + expert_sum B K fp32 + ids and weights B k (8 + 4)."""
    K = h if K is None else K
    latent = B*K*2 if K != h else 0
    return E*h*2 + E*4 + B*h*2 + latent + distinct*expert_bytes(I, K) + B*K*4 + B*k*(8 + 4)


def step_flops(*, B: int, E: int, k: int, h: int, I: int, K: int | None = None) -> int:
    """2 B E h (router) + 2 B k 3 I K (gate, up, down)."""
    K = h if K is None else K
    return 2*B*E*h + 2*B*k*3*I*K


def latent_in_bytes(*, B: int, h: int, lh: int, S: int) -> int:
    """latent_down lh h + shared gate/up 2 S h bf16 weights, x B h in, latent B lh and shared_h B S out."""
    return (lh + 2*S)*h*2 + B*h*2 + B*(lh + S)*2


def latent_out_bytes(*, B: int, h: int, lh: int, S: int) -> int:
    """latent_up h lh + shared_down h S bf16 weights + latent_norm lh, expert_sum B lh fp32 and
    shared_h B S in, output B h bf16 out."""
    return h*(lh + S)*2 + lh*2 + B*lh*4 + B*S*2 + B*h*2
