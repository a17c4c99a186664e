"""The latent MoE block of a Kimi K3 layer on MI355X (kimi.py:317-328, one TP rank).

    latent, shared_h = latent_in(normalized, latent_down, shared_gate, shared_up)     kimi.py:317, 326
    moe = moe_step(normalized, router, ..., latent=latent)                            kimi.py:318-324
    output = latent_out(moe['expert_sum'], latent_norm, latent_up, shared_h, shared_down)   kimi.py:325-328

`latent_block` runs the three on the current stream (three kernels, no host
sync) and returns the same dict as the CPU restatement's latent_block;
`latent_moe_layer` reads the weights from a reference-style value dict by the
keys of kimi.py:112-121. The TP all-reduces of kimi.py:324 and 326 are
identities on one rank and are not performed. Weights are bf16 and used in
place; the BF16 serving numerics are those of kimi.py:239-247 (fp32=True, the
FP32 truth mode, is the CPU oracle's).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from ._native import ACTIVATION, LatentDims, check
from .moe import _dev_ptr, _expect, cached_workspace, dims_for, prepare_step, workspace_bytes


def latent_dims(tokens: int, hidden: int, latent: int, shared: int, activation: str = 'situ') -> LatentDims:
    if activation not in ACTIVATION:
        raise ValueError(f'activation must be one of {sorted(ACTIVATION)}, got {activation!r}')
    return LatentDims(tokens=int(tokens), hidden=int(hidden), latent=int(latent), shared=int(shared),
                      activation=ACTIVATION[activation])


def latent_workspace_bytes(dims: LatentDims) -> int:
    n = ctypes.c_size_t(0)
    check(_native.load().k3moe_latent_workspace_bytes(ctypes.byref(dims), ctypes.byref(n)),
          'k3moe_latent_workspace_bytes')
    return int(n.value)


def _workspace(dims: LatentDims, device: torch.device, workspace: torch.Tensor | None) -> torch.Tensor:
    need = latent_workspace_bytes(dims)
    if workspace is None:
        return cached_workspace(need, device)
    if workspace.dtype != torch.uint8 or workspace.device != device or workspace.numel() < need:
        raise ValueError(f'workspace must be a uint8 tensor of at least {need} bytes on {device}')
    return workspace


def _device_of(x: torch.Tensor) -> torch.device:
    if not isinstance(x, torch.Tensor) or x.dim() != 2:
        raise ValueError('the activation must be a [B, width] tensor')
    if x.device.type != 'cuda':
        raise ValueError(f'input is on {x.device}; the latent block runs on a ROCm GPU')
    return x.device


def latent_in(normalized: torch.Tensor, latent_down: torch.Tensor, shared_gate: torch.Tensor,
              shared_up: torch.Tensor, *, activation: str = 'situ', out: dict | None = None,
              workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(latent [B, lh], shared_h [B, S]) bf16 from normalized [B, h] bf16 (kimi.py:317, 326-327).

    latent = bf16(normalized @ latent_down.T); shared_h = bf16(act(bf16(normalized @ shared_gate.T),
    bf16(normalized @ shared_up.T))) with FP32 accumulation. `out` may hold preallocated
    'latent' / 'shared_h' tensors.
    """
    device = _device_of(normalized)
    B, h = normalized.shape
    lh, S = latent_down.shape[0], shared_gate.shape[0]
    dims = latent_dims(B, h, lh, S, activation)
    _expect(normalized, 'normalized', torch.bfloat16, (B, h), device)
    _expect(latent_down, 'latent_down', torch.bfloat16, (lh, h), device)
    _expect(shared_gate, 'shared_gate', torch.bfloat16, (S, h), device)
    _expect(shared_up, 'shared_up', torch.bfloat16, (S, h), device)
    out = dict(out or {})
    with torch.cuda.device(device):
        lat = out.get('latent')
        if lat is None:
            lat = torch.empty(B, lh, dtype=torch.bfloat16, device=device)
        sh = out.get('shared_h')
        if sh is None:
            sh = torch.empty(B, S, dtype=torch.bfloat16, device=device)
        _expect(lat, 'latent', torch.bfloat16, (B, lh), device)
        _expect(sh, 'shared_h', torch.bfloat16, (B, S), device)
        ws = _workspace(dims, device, workspace)
        stream = torch.cuda.current_stream(device).cuda_stream
        check(_native.load().k3moe_latent_in(ctypes.byref(dims), _dev_ptr(normalized), _dev_ptr(latent_down),
                                             _dev_ptr(shared_gate), _dev_ptr(shared_up), _dev_ptr(lat),
                                             _dev_ptr(sh), _dev_ptr(ws), ctypes.c_size_t(ws.numel()),
                                             ctypes.c_void_p(stream)), 'k3moe_latent_in')
    return lat, sh


def latent_out(expert_sum: torch.Tensor, latent_norm: torch.Tensor, latent_up: torch.Tensor,
               shared_h: torch.Tensor, shared_down: torch.Tensor, *, out: torch.Tensor | None = None,
               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """routed + bf16(shared) [B, h] bf16 (kimi.py:325-328).

    routed = bf16(rms(bf16(expert_sum), latent_norm, eps=1e-5) @ latent_up.T) with rms as
    common.py:13-21; shared = bf16(shared_h @ shared_down.T).
    """
    device = _device_of(expert_sum)
    B, lh = expert_sum.shape
    h, S = latent_up.shape[0], shared_down.shape[1]
    dims = latent_dims(B, h, lh, S)
    _expect(expert_sum, 'expert_sum', torch.float32, (B, lh), device)
    _expect(latent_norm, 'latent_norm', torch.bfloat16, (lh,), device)
    _expect(latent_up, 'latent_up', torch.bfloat16, (h, lh), device)
    _expect(shared_h, 'shared_h', torch.bfloat16, (B, S), device)
    _expect(shared_down, 'shared_down', torch.bfloat16, (h, S), device)
    with torch.cuda.device(device):
        if out is None:
            out = torch.empty(B, h, dtype=torch.bfloat16, device=device)
        _expect(out, 'out', torch.bfloat16, (B, h), device)
        ws = _workspace(dims, device, workspace)
        stream = torch.cuda.current_stream(device).cuda_stream
        check(_native.load().k3moe_latent_out(ctypes.byref(dims), _dev_ptr(expert_sum), _dev_ptr(latent_norm),
                                              _dev_ptr(latent_up), _dev_ptr(shared_h), _dev_ptr(shared_down),
                                              _dev_ptr(out), _dev_ptr(ws), ctypes.c_size_t(ws.numel()),
                                              ctypes.c_void_p(stream)), 'k3moe_latent_out')
    return out


def latent_moe_step(normalized: torch.Tensor, w: dict, *, topk: int, gating: str = 'sigmoid_bias',
                    activation: str = 'situ', routes: torch.Tensor | None = None,
                    path: str = 'auto', out: dict | None = None) -> tuple[torch.Tensor, torch.Tensor, dict]:
    """latent_in and moe_step on its latent in one call (k3moe_latent_moe_step): one launch for a
    single token on the single-token kernel's geometry, else the two launches. Returns
    (latent, shared_h, moe_step's dict); `w` as latent_block's. `out` may hold preallocated
    'latent', 'shared_h' and moe_step output tensors."""
    out = dict(out or {})
    device = _device_of(normalized)
    B, h = normalized.shape
    lh, S = w['latent_down'].shape[0], w['shared_gate'].shape[0]
    _expect(normalized, 'normalized', torch.bfloat16, (B, h), device)
    _expect(w['latent_down'], 'latent_down', torch.bfloat16, (lh, h), device)
    _expect(w['shared_gate'], 'shared_gate', torch.bfloat16, (S, h), device)
    _expect(w['shared_up'], 'shared_up', torch.bfloat16, (S, h), device)
    with torch.cuda.device(device):
        latent = out.get('latent')
        if latent is None:
            latent = torch.empty(B, lh, dtype=torch.bfloat16, device=device)
        shared_h = out.get('shared_h')
        if shared_h is None:
            shared_h = torch.empty(B, S, dtype=torch.bfloat16, device=device)
    _expect(latent, 'latent', torch.bfloat16, (B, lh), device)
    _expect(shared_h, 'shared_h', torch.bfloat16, (B, S), device)
    # one workspace for both halves (the two-launch fallback runs latent_in on it too)
    mdims = dims_for(normalized, w['router'], w['gate_blocks'], w['down_blocks'], topk, gating, activation, latent,
                     path)
    ws = cached_workspace(max(workspace_bytes(mdims), latent_workspace_bytes(latent_dims(B, h, lh, S, activation))),
                          device)
    step = prepare_step(normalized, w['router'], w.get('router_bias'), w['gate_blocks'], w['gate_scales'],
                        w['up_blocks'], w['up_scales'], w['down_blocks'], w['down_scales'], topk=topk,
                        gating=gating, activation=activation, routes=routes, latent=latent, path=path, workspace=ws,
                        out=out)
    a = step._args  # (dims, x, latent, router .. shortfall, workspace, workspace bytes)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        check(_native.load().k3moe_latent_moe_step(
            a[0], ctypes.c_int32(S), a[1], _dev_ptr(w['latent_down']), _dev_ptr(w['shared_gate']),
            _dev_ptr(w['shared_up']), _dev_ptr(latent), _dev_ptr(shared_h), *a[3:16], _dev_ptr(ws),
            ctypes.c_size_t(ws.numel()), ctypes.c_void_p(stream)), 'k3moe_latent_moe_step')
    return latent, shared_h, step.result


def latent_block(normalized: torch.Tensor, w: dict, *, topk: int, gating: str = 'sigmoid_bias',
                 activation: str = 'situ', fp32: bool = False, routes: torch.Tensor | None = None,
                 path: str = 'auto', out: dict | None = None) -> dict:
    """The whole block: latent_in, the routed experts on the latent (moe_step), latent_out, in one
    call (k3moe_latent_block: one launch for one token on the single-token kernel's geometry, else
    latent_moe_step's one or two launches and latent_out's).

    `w` holds latent_down, latent_up, latent_norm, shared_gate, shared_up, shared_down, router,
    router_bias and {gate,up,down}_{blocks,scales} (kimi.py:112-121 names without the layer
    prefix). Returns {'output' bf16 [B, h], 'latent', 'shared_h', 'expert_sum', 'expert_ids',
    'route_weights', ['route_shortfall']}. `activation` is the routed and shared experts'
    (SiTU in kimi.py:322, 326). `out` may hold preallocated output tensors by those keys.
    """
    if fp32:
        raise NotImplementedError('fp32=True is the FP32 truth mode of the CPU oracle; '
                                  'the GPU block computes the BF16 serving path (fp32=False)')
    out = dict(out or {})
    device = _device_of(normalized)
    B, h = normalized.shape
    lh, S = w['latent_down'].shape[0], w['shared_gate'].shape[0]
    _expect(normalized, 'normalized', torch.bfloat16, (B, h), device)
    for name, shape in (('latent_down', (lh, h)), ('shared_gate', (S, h)), ('shared_up', (S, h)),
                        ('latent_norm', (lh,)), ('latent_up', (h, lh)), ('shared_down', (h, S))):
        _expect(w[name], name, torch.bfloat16, shape, device)
    with torch.cuda.device(device):
        for name, shape in (('latent', (B, lh)), ('shared_h', (B, S)), ('output', (B, h))):
            if out.get(name) is None:
                out[name] = torch.empty(*shape, dtype=torch.bfloat16, device=device)
            _expect(out[name], name, torch.bfloat16, shape, device)
    latent, shared_h, output = out['latent'], out['shared_h'], out['output']
    # one workspace for every launch of the block
    mdims = dims_for(normalized, w['router'], w['gate_blocks'], w['down_blocks'], topk, gating, activation, latent,
                     path)
    ws = cached_workspace(max(workspace_bytes(mdims), latent_workspace_bytes(latent_dims(B, h, lh, S, activation))),
                          device)
    step = prepare_step(normalized, w['router'], w.get('router_bias'), w['gate_blocks'], w['gate_scales'],
                        w['up_blocks'], w['up_scales'], w['down_blocks'], w['down_scales'], topk=topk,
                        gating=gating, activation=activation, routes=routes, latent=latent, path=path, workspace=ws,
                        out=out)
    a = step._args  # (dims, x, latent, router .. routes, expert_sum .. shortfall, workspace, workspace bytes)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        check(_native.load().k3moe_latent_block(
            a[0], ctypes.c_int32(S), a[1], _dev_ptr(w['latent_down']), _dev_ptr(w['shared_gate']),
            _dev_ptr(w['shared_up']), _dev_ptr(w['latent_norm']), _dev_ptr(w['latent_up']),
            _dev_ptr(w['shared_down']), *a[3:12], _dev_ptr(latent), _dev_ptr(shared_h), *a[12:16],
            _dev_ptr(output), _dev_ptr(ws), ctypes.c_size_t(ws.numel()), ctypes.c_void_p(stream)),
            'k3moe_latent_block')
    return {'output': output, 'latent': latent, 'shared_h': shared_h, **step.result}


BLOCK_KEYS = ('latent_down', 'latent_up', 'latent_norm', 'router', 'router_bias', 'gate_blocks', 'gate_scales',
              'up_blocks', 'up_scales', 'down_blocks', 'down_scales', 'shared_gate', 'shared_up', 'shared_down')


def latent_moe_layer(values: dict, layer: int, normalized: torch.Tensor, *, topk: int,
                     gating: str = 'sigmoid_bias', routes: torch.Tensor | None = None) -> dict:
    """latent_block on the weights of layer `layer` of a reference-style value dict.

    Reads l{layer}_<name> for the names of kimi.py:112-121 (read at kimi.py:308-327).
    `routes` may be the reference's [L, B, k] tensor, from which row `layer` is used.
    """
    p = f'l{layer}_'
    if routes is not None and routes.dim() == 3:
        routes = routes[layer]
    w = {k: values.get(p + k) for k in BLOCK_KEYS}
    return latent_block(normalized, w, topk=topk, gating=gating, routes=routes)
