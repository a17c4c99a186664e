"""Seeded synthetic MoE-layer inputs in the reference's layouts.

Streams are keyed by ``seed_for(seed, name)`` = the little-endian blake2b-64
of "seed:name" (megabench/tasks/distributed.py:25-26), so every tensor of a
layer has an independent, reproducible stream.

Distributions (the MoE-layer configurations of the benchmark):
  router       bf16 N(0, 0.02)                      [E, h]
  router_bias  fp32 N(0, 0.01)   (kimi.py:138-139)  [E]
  x            bf16 N(0, 1)                         [B, h]
  *_blocks     uniform bytes, i.e. two uniform E2M1 codes per byte
  *_scales     E8M0 127 + U{-8..-4} (bytes 119..123), one per 32-block
The `kimi` scale mode instead restates the reference generator's exponents
(kimi.py:66-68): three consecutive values around round(-log2(2.93 sqrt(fan_in))).

Uint8 tensors come from numpy's PCG64 (fast, platform independent); normal
tensors from torch's CPU generator as in kimi.py:56-58. Everything is made on
the host CPU and copied, so the CPU oracle and the GPU see identical bytes.
For the largest layouts `device='cuda'` generation is available (different
streams, same distributions).
"""

from __future__ import annotations

import hashlib
import math

import numpy as np
import torch


def seed_for(seed: int, name: str) -> int:
    """blake2b-64 of f"{seed}:{name}", little endian (distributed.py:25-26)."""
    return int.from_bytes(hashlib.blake2b(f"{seed}:{name}".encode(), digest_size=8).digest(), "little")


def randn(seed: int, name: str, shape, scale: float, *, dtype=torch.bfloat16, device='cpu',
          shift: float = 0.0) -> torch.Tensor:
    """N(shift, scale) in float32 cast to dtype (kimi.py:56-58)."""
    if str(device).startswith('cuda'):
        g = torch.Generator(device=device).manual_seed(seed_for(seed, name) & ((1 << 63) - 1))
        return (torch.randn(shape, generator=g, device=device)*scale + shift).to(dtype)
    g = torch.Generator().manual_seed(seed_for(seed, name))
    return (torch.randn(shape, generator=g)*scale + shift).to(dtype).to(device)


def kimi_exponent(fan_in: int) -> int:
    """Centre E8M0 exponent of the reference generator (kimi.py:67)."""
    return round(-math.log2(2.93*fan_in**0.5))


def mxfp4(seed: int, name: str, lead: tuple, cols: int, *, scale_mode: str = 'uniform',
          exp_lo: int = -8, exp_hi: int = -4, fan_in: int | None = None, device='cpu'):
    """Random MXFP4 matrix [*lead, cols]: blocks u8 [*lead, cols/32, 16], scales u8 [*lead, cols/32].

    scale_mode 'uniform': exponent uniform in [exp_lo, exp_hi];
    'kimi': exponent in {c-1, c, c+1}, c = kimi_exponent(fan_in) (kimi.py:66-68).
    """
    if cols % 32:
        raise ValueError('MXFP4 block axis must be divisible by 32')
    if scale_mode == 'kimi':
        c = kimi_exponent(fan_in if fan_in is not None else cols)
        exp_lo, exp_hi = c - 1, c + 1
    elif scale_mode != 'uniform':
        raise ValueError(f'unknown scale_mode {scale_mode!r}')
    nb = cols // 32
    bshape, sshape = (*lead, nb, 16), (*lead, nb)
    if str(device).startswith('cuda'):
        g = torch.Generator(device=device).manual_seed(seed_for(seed, name) & ((1 << 63) - 1))
        blocks = torch.randint(0, 256, bshape, generator=g, device=device, dtype=torch.uint8)
        scales = (127 + exp_lo + torch.randint(0, exp_hi - exp_lo + 1, sshape, generator=g, device=device)
                  ).to(torch.uint8)
        return blocks, scales
    rng = np.random.Generator(np.random.PCG64(seed_for(seed, name)))
    blocks = np.frombuffer(rng.bytes(int(np.prod(bshape))), dtype=np.uint8).reshape(bshape)
    scales = rng.integers(127 + exp_lo, 127 + exp_hi + 1, size=sshape, dtype=np.uint8)
    return torch.from_numpy(blocks.copy()).to(device), torch.from_numpy(scales).to(device)


def moe_layer_inputs(cfg, seed: int, *, layer: int = 0, device='cpu', scale_mode: str = 'uniform',
                     with_bias: bool | None = None) -> dict:
    """Inputs of one MoE layer of `cfg` (a k3moe.configs.MoEConfig).

    Keys: x, router, router_bias (None for softmax gating unless with_bias),
    gate_blocks, gate_scales, up_blocks, up_scales, down_blocks, down_scales.
    Weight stream names carry the layer, l{layer}_<name>; x is shared by layers.
    """
    E, h, I, B = cfg.experts, cfg.hidden, cfg.inter, cfg.tokens
    K = cfg.latent or h
    p = f'l{layer}_'
    if with_bias is None:
        with_bias = cfg.gating == 'sigmoid_bias'
    out = {'x': randn(seed, 'x', (B, h), 1.0, device=device),
           'router': randn(seed, p + 'router', (E, h), 0.02, device=device),
           'router_bias': randn(seed, p + 'router_bias', (E,), 0.01, dtype=torch.float32, device=device)
           if with_bias else None}
    if cfg.latent:
        out['latent'] = randn(seed, 'latent', (B, K), 1.0, device=device)
    for name, lead, cols, fan in (('gate', (E, I), K, K), ('up', (E, I), K, K), ('down', (E, K), I, I)):
        out[name + '_blocks'], out[name + '_scales'] = mxfp4(seed, p + name, lead, cols, scale_mode=scale_mode,
                                                             fan_in=fan, device=device)
    return out


STEP_KEYS = ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks', 'up_scales',
             'down_blocks', 'down_scales')


def step_args(inputs: dict) -> tuple:
    """Positional arguments of k3moe.moe_step (and the oracle's moe_step) from an input dict."""
    return tuple(inputs[k] for k in STEP_KEYS)


def latent_block_inputs(cfg, seed: int, *, shared: int, shared_fan: int | None = None, layer: int = 0,
                        device='cpu', scale_mode: str = 'kimi') -> dict:
    """Inputs of one latent MoE block (kimi.py:112-121, 317-328) of `cfg` (cfg.latent set).

    The expert tensors and router of moe_layer_inputs, plus latent_down [lh, h],
    latent_up [h, lh], latent_norm [lh], shared_gate / shared_up [shared, h] and
    shared_down [h, shared], all bf16 with the reference generator's
    distributions (kimi.py:134-144): N(0, fan_in^-1/2), norm weights N(1, 0.1).
    shared_fan is shared_down's fan-in, the unsharded shared width for a TP
    shard (kimi.py:121: intermediate x shared_experts; 6144 for Kimi K3).
    `x` is the normalized layer input [B, h]; there is no separate `latent`.
    """
    if not cfg.latent:
        raise ValueError('latent_block_inputs needs a configuration with a latent width')
    out = moe_layer_inputs(cfg, seed, layer=layer, device=device, scale_mode=scale_mode)
    out.pop('latent')
    h, lh, p = cfg.hidden, cfg.latent, f'l{layer}_'
    for name, shape, fan in (('latent_down', (lh, h), h), ('latent_up', (h, lh), lh),
                             ('shared_gate', (shared, h), h), ('shared_up', (shared, h), h),
                             ('shared_down', (h, shared), shared_fan or shared)):
        out[name] = randn(seed, p + name, shape, fan**-0.5, device=device)
    out['latent_norm'] = randn(seed, p + 'latent_norm', (lh,), 0.1, shift=1.0, device=device)
    return out
