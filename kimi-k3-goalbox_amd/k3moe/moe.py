"""Drop-in MoE step on MI355X: torch tensors in, torch tensors out.

`moe_step` takes the tensors the reference's MoE block reads
(megabench/tasks/kimi.py:308-323) in their stored layouts and dtypes and
returns the block's results; `moe_layer` reads them from a weight dict by the
reference's key names (kimi.py:114-119). The weights are never repacked or
copied: the kernels read the caller's uint8 MXFP4 blocks and E8M0 scales in
place. All work is enqueued on torch's current stream without a host sync
(except when forced routes are validated, see below).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from ._native import ACTIVATION, GATING, Dims, check

MX_BLOCK = 32
INIT_BYTES = 4096 + 65536 + 16384 + 2097152  # control block, zero area, latent-block counters and tag area (k3moe_workspace_init)


def _dev_ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _expect(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f'{name} must be a torch.Tensor, got {type(t).__name__}')
    if t.dtype != dtype:
        raise ValueError(f'{name} must be {dtype}, got {t.dtype}')
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f'{name} must have shape {tuple(shape)}, got {tuple(t.shape)}')
    if t.device != device:
        raise ValueError(f'{name} is on {t.device}, expected {device}')
    if not t.is_contiguous():
        raise ValueError(f'{name} must be contiguous')


def dims_for(x: torch.Tensor, router: torch.Tensor, gate_blocks: torch.Tensor, down_blocks: torch.Tensor,
             topk: int, gating: str, activation: str, latent: torch.Tensor | None = None,
             path: str = 'auto') -> Dims:
    if gating not in GATING:
        raise ValueError(f'gating must be one of {sorted(GATING)}, got {gating!r}')
    if activation not in ACTIVATION:
        raise ValueError(f'activation must be one of {sorted(ACTIVATION)}, got {activation!r}')
    if path not in _native.PATH:
        raise ValueError(f'path must be one of {sorted(_native.PATH)}, got {path!r}')
    if x.dim() != 2 or router.dim() != 2 or gate_blocks.dim() != 4 or down_blocks.dim() != 4:
        raise ValueError('invalid MXFP4 block/scale geometry')
    B, h = x.shape
    E, I = gate_blocks.shape[0], gate_blocks.shape[1]
    K = latent.shape[1] if latent is not None else h
    return Dims(tokens=B, experts=E, topk=int(topk), hidden=h, latent=K, inter=I,
                gating=GATING[gating], activation=ACTIVATION[activation], x_dtype=_native.DTYPE_BF16,
                path=_native.PATH[path])


def workspace_bytes(dims: Dims) -> int:
    lib = _native.load()
    n = ctypes.c_size_t(0)
    check(lib.k3moe_workspace_bytes(ctypes.byref(dims), ctypes.byref(n)), 'k3moe_workspace_bytes')
    return int(n.value)


_WORKSPACES: dict = {}


def get_workspace(dims: Dims, device: torch.device) -> torch.Tensor:
    """The cached step workspace of `device`, grown to fit `dims`.

    A new workspace is zero-initialised by k3moe_workspace_init (a kernel on
    the current stream, never a memset). Each launch takes its barrier targets
    from the counters' values at its start and the latent block's tile
    counters return to zero, so one workspace serves consecutive steps in
    stream order; steps that may run concurrently on other streams must pass
    their own workspace.
    """
    return cached_workspace(workspace_bytes(dims), device)


def cached_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """The device's cached workspace, grown to at least `nbytes` (shared by the MoE step and the latent block)."""
    need = max(int(nbytes), INIT_BYTES)
    key = (device.type, device.index)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = new_workspace(need, device)
        _WORKSPACES[key] = ws
    return ws


def new_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A fresh, initialised workspace of at least `nbytes` bytes."""
    ws = torch.empty(max(int(nbytes), INIT_BYTES), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        check(_native.load().k3moe_workspace_init(_dev_ptr(ws), ctypes.c_size_t(ws.numel()),
                                                   ctypes.c_void_p(stream)), 'k3moe_workspace_init')
    return ws


def workspace_layout(dims: Dims) -> dict:
    """Byte offsets of the general path's grouping lists in the workspace (k3moe_workspace_layout)."""
    lay = _native.Layout()
    check(_native.load().k3moe_workspace_layout(ctypes.byref(dims), ctypes.byref(lay)), 'k3moe_workspace_layout')
    return {n: int(getattr(lay, n)) for n, _ in _native.Layout._fields_}


def workspace_status(ws: torch.Tensor) -> int:
    """Sticky status word of a workspace: 0 = every step since its init completed normally, else
    bits STATUS_TIMEOUT (a wait timed out: that step's output holds NaN; re-initialise the
    workspace) and STATUS_ROUTES (a forced-route row was invalid and used its own top-k).
    Synchronises; the steps themselves never do."""
    st = ctypes.c_int32(-1)
    with torch.cuda.device(ws.device):
        stream = torch.cuda.current_stream(ws.device).cuda_stream
        check(_native.load().k3moe_workspace_status(_dev_ptr(ws), ctypes.byref(st), ctypes.c_void_p(stream)),
              'k3moe_workspace_status')
    return int(st.value)


def _validate_routes(routes: torch.Tensor, B: int, k: int, E: int, device) -> torch.Tensor:
    if not isinstance(routes, torch.Tensor) or routes.dim() != 2 or tuple(routes.shape) != (B, k):
        raise ValueError(f'routes must be a [{B}, {k}] tensor')
    if routes.dtype not in (torch.int64, torch.int32, torch.int16, torch.uint8):
        raise ValueError(f'routes must hold integer expert ids, got {routes.dtype}')
    r = routes.to(device=device, dtype=torch.int64).contiguous()
    # ids in range and distinct in each row (kimi.py:364-367); this check syncs
    ordered = r.sort(-1).values
    bad = ((r < 0) | (r >= E)).any() | (ordered[:, 1:] == ordered[:, :-1]).any()
    if bool(bad):
        raise ValueError('routes: ids out of range or repeated in a row')
    return r


class PreparedStep:
    """One MoE step's validated launch: the tensors, outputs, workspace and the C-ABI argument
    list are fixed when it is made (prepare_step), so a call only reads torch's current stream
    and calls k3moe_moe_step (a few microseconds on the host, where moe_step's checks take
    about 18). The tensors' contents may change between calls (new token rows in x, another
    step's forced routes): the kernels read them at each launch. Calling it returns the same
    output tensors each time, overwritten in stream order."""

    def __init__(self, device, args, result):
        self.device = device
        self.result = result
        self._args = args
        self._fn = _native.load().k3moe_moe_step

    def __call__(self) -> dict:
        dev = self.device
        if torch.cuda.current_device() != dev.index:
            with torch.cuda.device(dev):
                return self()
        rc = self._fn(*self._args, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        if rc:
            check(rc, 'k3moe_moe_step')
        return self.result


def prepare_step(x: torch.Tensor, router: torch.Tensor, router_bias: torch.Tensor | None,
                 gate_blocks: torch.Tensor, gate_scales: torch.Tensor,
                 up_blocks: torch.Tensor, up_scales: torch.Tensor,
                 down_blocks: torch.Tensor, down_scales: torch.Tensor, *,
                 topk: int, gating: str = 'sigmoid_bias', activation: str = 'situ',
                 fp32: bool = False, routes: torch.Tensor | None = None,
                 latent: torch.Tensor | None = None, out: dict | None = None,
                 workspace: torch.Tensor | None = None, path: str = 'auto') -> PreparedStep:
    """Validate a step's arguments once (moe_step's checks and errors) and return a
    PreparedStep that launches it; arguments as moe_step's."""
    if fp32:
        raise NotImplementedError('fp32=True is the FP32 truth mode of the CPU oracle; '
                                  'the GPU step computes the BF16 serving path (fp32=False)')
    if not isinstance(x, torch.Tensor) or x.dim() != 2:
        raise ValueError('x must be a [B, hidden] tensor')
    device = x.device
    if device.type != 'cuda':
        raise ValueError(f'x is on {device}; the k3moe step runs on a ROCm GPU')
    dims = dims_for(x, router, gate_blocks, down_blocks, topk, gating, activation, latent, path)
    B, h, E, k, K, I = dims.tokens, dims.hidden, dims.experts, dims.topk, dims.latent, dims.inter
    if not 1 <= k <= min(E, 32):
        raise ValueError(f'topk must be in [1, min(32, experts)], got {k}')
    if K % MX_BLOCK or I % MX_BLOCK:
        raise ValueError('MXFP4 block axis must be divisible by 32')
    _expect(x, 'x', torch.bfloat16, (B, h), device)
    _expect(router, 'router', torch.bfloat16, (E, h), device)
    if router_bias is not None:
        _expect(router_bias, 'router_bias', torch.float32, (E,), device)
    for name, t, shape in (('gate_blocks', gate_blocks, (E, I, K//32, 16)), ('gate_scales', gate_scales, (E, I, K//32)),
                           ('up_blocks', up_blocks, (E, I, K//32, 16)), ('up_scales', up_scales, (E, I, K//32)),
                           ('down_blocks', down_blocks, (E, K, I//32, 16)), ('down_scales', down_scales, (E, K, I//32))):
        if isinstance(t, torch.Tensor) and t.dtype != torch.uint8:
            raise ValueError('MXFP4 blocks and E8M0 scales must be uint8')
        _expect(t, name, torch.uint8, shape, device)
    if latent is not None:
        _expect(latent, 'latent', torch.bfloat16, (B, K), device)
    if routes is not None:
        routes = _validate_routes(routes, B, k, E, device)

    ws_bytes = workspace_bytes(dims)
    with torch.cuda.device(device):
        out = dict(out or {})
        expert_sum = out.get('expert_sum')
        if expert_sum is None:
            expert_sum = torch.empty(B, K, dtype=torch.float32, device=device)
        ids = out.get('expert_ids')
        if ids is None:
            ids = torch.empty(B, k, dtype=torch.int64, device=device)
        weights = out.get('route_weights')
        if weights is None:
            weights = torch.empty(B, k, dtype=torch.float32, device=device)
        shortfall = None
        if routes is not None:
            shortfall = out.get('route_shortfall')
            if shortfall is None:
                shortfall = torch.empty(B, dtype=torch.float32, device=device)
        _expect(expert_sum, 'expert_sum', torch.float32, (B, K), device)
        _expect(ids, 'expert_ids', torch.int64, (B, k), device)
        _expect(weights, 'route_weights', torch.float32, (B, k), device)
        if workspace is None:
            workspace = get_workspace(dims, device)
        elif workspace.dtype != torch.uint8 or workspace.device != device or workspace.numel() < ws_bytes:
            raise ValueError(f'workspace must be a uint8 tensor of at least {ws_bytes} bytes on {device}')
    args = (ctypes.byref(dims), _dev_ptr(x), _dev_ptr(latent), _dev_ptr(router), _dev_ptr(router_bias),
            _dev_ptr(gate_blocks), _dev_ptr(gate_scales), _dev_ptr(up_blocks), _dev_ptr(up_scales),
            _dev_ptr(down_blocks), _dev_ptr(down_scales), _dev_ptr(routes), _dev_ptr(expert_sum), _dev_ptr(ids),
            _dev_ptr(weights), _dev_ptr(shortfall), _dev_ptr(workspace), ctypes.c_size_t(workspace.numel()))
    result = {'expert_sum': expert_sum, 'expert_ids': ids, 'route_weights': weights}
    if routes is not None:
        result['route_shortfall'] = shortfall
    step = PreparedStep(device, args, result)
    # the tensors the argument list points at stay alive as long as the prepared step
    step._keep = (dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales, down_blocks,
                  down_scales, routes, workspace)
    return step


def moe_step(x: torch.Tensor, router: torch.Tensor, router_bias: torch.Tensor | None,
             gate_blocks: torch.Tensor, gate_scales: torch.Tensor,
             up_blocks: torch.Tensor, up_scales: torch.Tensor,
             down_blocks: torch.Tensor, down_scales: torch.Tensor, *,
             topk: int, gating: str = 'sigmoid_bias', activation: str = 'situ',
             fp32: bool = False, routes: torch.Tensor | None = None,
             latent: torch.Tensor | None = None, out: dict | None = None,
             workspace: torch.Tensor | None = None, path: str = 'auto') -> dict:
    """One MXFP4 MoE step (kimi.py:307-324 without the TP all-reduce) on the GPU.

    x [B, h] bf16 (the router input, kimi.py:308); router [E, h] bf16;
    router_bias [E] fp32 or None; gate/up blocks [E, I, K/32, 16] u8 and
    scales [E, I, K/32] u8; down blocks [E, K, I/32, 16] u8 and scales
    [E, K, I/32] u8 (kimi.py:114-119); latent [B, K] bf16 or None (the experts
    then read x, K = h). routes [B, k] forces the expert sets
    (kimi.py:311-313) and adds route_shortfall.

    Returns {'expert_sum': fp32 [B, K], 'expert_ids': int64 [B, k] ascending,
    'route_weights': fp32 [B, k] aligned with expert_ids,
    ['route_shortfall': fp32 [B]]}, all on x's device. Inputs are never
    written. `out` may supply preallocated output tensors by the same keys;
    `workspace` an initialised workspace (new_workspace), else the device's
    cached one is used. `path` forces an execution path ('auto', 'general',
    'decode', or the general path with 'grouped' GEMM or 'streamed' expert
    kernels); the default picks the persistent kernel for decode batches.
    prepare_step validates the same arguments once for repeated launches.
    """
    return prepare_step(x, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales, down_blocks,
                        down_scales, topk=topk, gating=gating, activation=activation, fp32=fp32, routes=routes,
                        latent=latent, out=out, workspace=workspace, path=path)()


def moe_layer(values: dict, layer: int, x: torch.Tensor, *, topk: int, gating: str = 'sigmoid_bias',
              activation: str = 'situ', fp32: bool = False, routes: torch.Tensor | None = None,
              latent: torch.Tensor | None = None) -> dict:
    """moe_step on the weights of MoE layer `layer` of a reference-style weight dict.

    Reads l{layer}_router, l{layer}_router_bias and l{layer}_{gate,up,down}_{blocks,scales}
    (kimi.py:114-119, read at kimi.py:308-321). `routes` may be the reference's
    [L, B, k] tensor, from which row `layer` is used (kimi.py:312).
    """
    p = f'l{layer}_'
    if routes is not None and routes.dim() == 3:
        routes = routes[layer]
    return moe_step(x, values[p + 'router'], values.get(p + 'router_bias'),
                    values[p + 'gate_blocks'], values[p + 'gate_scales'],
                    values[p + 'up_blocks'], values[p + 'up_scales'],
                    values[p + 'down_blocks'], values[p + 'down_scales'],
                    topk=topk, gating=gating, activation=activation, fp32=fp32, routes=routes, latent=latent)


def activation(g: torch.Tensor, u: torch.Tensor, activation: str = 'situ', fast: bool = False) -> torch.Tensor:
    """The expert GEMMs' activation act(g, u) on the GPU (debug entry point k3moe_activation):
    fast=False is the decode kernels' library-function form, fast=True the prefill GEMM's
    exponential-and-reciprocal form. g, u: fp32 tensors of one shape on one ROCm GPU."""
    if activation not in ('situ', 'silu'):
        raise ValueError(f"activation must be 'situ' or 'silu', got {activation!r}")
    if not isinstance(g, torch.Tensor) or not isinstance(u, torch.Tensor) or g.shape != u.shape:
        raise ValueError('g and u must be tensors of one shape')
    if g.dtype != torch.float32 or u.dtype != torch.float32:
        raise ValueError('g and u must be float32')
    if g.device.type != 'cuda' or u.device != g.device:
        raise ValueError('g and u must be on the same ROCm GPU')
    g, u = g.contiguous(), u.contiguous()
    out = torch.empty_like(g)
    with torch.cuda.device(g.device):
        stream = torch.cuda.current_stream(g.device).cuda_stream
        rc = _native.load().k3moe_activation(0 if activation == 'situ' else 1, 1 if fast else 0, _dev_ptr(g),
                                             _dev_ptr(u), _dev_ptr(out), g.numel(), ctypes.c_void_p(stream))
        check(rc, 'k3moe_activation')
    return out


def mxfp4_decode(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """unpack_mxfp4 (quantization.py:40-51) on the GPU, optionally with the bf16 cast of kimi.py:321.

    blocks u8 [..., n, 16], scales u8 [..., n] -> dtype [..., n*32], bit-exact.
    """
    if not isinstance(blocks, torch.Tensor) or not isinstance(scales, torch.Tensor):
        raise ValueError('blocks and scales must be tensors')
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise ValueError('MXFP4 blocks and E8M0 scales must be uint8')
    if blocks.shape[:-1] != scales.shape or blocks.shape[-1] != MX_BLOCK // 2:
        raise ValueError('invalid MXFP4 block/scale geometry')
    if blocks.device.type != 'cuda' or scales.device != blocks.device:
        raise ValueError('blocks and scales must be on the same ROCm GPU')
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f'dtype must be float32 or bfloat16, got {dtype}')
    blocks, scales = blocks.contiguous(), scales.contiguous()
    out = torch.empty(*scales.shape[:-1], scales.shape[-1]*MX_BLOCK if scales.dim() else 0,
                      dtype=dtype, device=blocks.device)
    code = _native.DTYPE_F32 if dtype == torch.float32 else _native.DTYPE_BF16
    with torch.cuda.device(blocks.device):
        stream = torch.cuda.current_stream(blocks.device).cuda_stream
        rc = _native.load().k3moe_mxfp4_decode(_dev_ptr(blocks), _dev_ptr(scales), scales.numel(), code,
                                               _dev_ptr(out), ctypes.c_void_p(stream))
        check(rc, 'k3moe_mxfp4_decode')
    return out


_ENCODE_DTYPES = {torch.float32: 'DTYPE_F32', torch.bfloat16: 'DTYPE_BF16', torch.float16: 'DTYPE_F16'}


def pack_mxfp4(matrix: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """pack_mxfp4 (quantization.py:13-37) on the GPU: groups of 32 along the last axis -> E2M1 + E8M0.

    matrix [..., K] on a ROCm GPU (float32, bfloat16 or float16 read as they are; any other dtype
    is first cast to float32, as the reference's ``matrix.float()``) -> packed u8 [..., K/32, 16]
    (low nibble = even element), scales u8 [..., K/32], bit for bit with the reference's torch CPU
    chain. Raises ValueError when K is not a multiple of 32, as the reference does.
    """
    if not isinstance(matrix, torch.Tensor):
        raise ValueError('matrix must be a tensor')
    if matrix.dim() == 0 or matrix.shape[-1] % MX_BLOCK:
        raise ValueError('MXFP4 block axis must be divisible by 32')
    if matrix.device.type != 'cuda':
        raise ValueError('matrix must be on a ROCm GPU')
    if matrix.dtype not in _ENCODE_DTYPES:
        matrix = matrix.float()
    src = matrix.contiguous()
    if src.data_ptr() % 16:  # a view starting inside a 16-byte word: the encoder reads 16-byte words
        src = src.clone()
    lead, n = tuple(matrix.shape[:-1]), matrix.shape[-1] // MX_BLOCK
    packed = torch.empty(*lead, n, MX_BLOCK // 2, dtype=torch.uint8, device=matrix.device)
    scales = torch.empty(*lead, n, dtype=torch.uint8, device=matrix.device)
    code = getattr(_native, _ENCODE_DTYPES[src.dtype])
    with torch.cuda.device(matrix.device):
        stream = torch.cuda.current_stream(matrix.device).cuda_stream
        rc = _native.load().k3moe_mxfp4_encode(_dev_ptr(src), code, scales.numel(), _dev_ptr(packed),
                                               _dev_ptr(scales), ctypes.c_void_p(stream))
        check(rc, 'k3moe_mxfp4_encode')
    return packed, scales
