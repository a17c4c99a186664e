"""ctypes binding of libk3moe.so, the HIP library behind the MoE step.

torch is imported first so that its HIP runtime (libamdhip64.so.7) is the one
the library binds to: one runtime per process, so torch's device pointers and
streams are valid inside the library. There is no CPU fallback: if the
library is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library links against)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libk3moe.so')

K3MOE_OK = 0
GATING = {'sigmoid_bias': 0, 'softmax': 1}
ACTIVATION = {'situ': 0, 'silu': 1}
DTYPE_BF16, DTYPE_F32, DTYPE_F16 = 0, 1, 2
PATH = {'auto': 0, 'general': 1, 'decode': 2, 'grouped': 3, 'streamed': 4, 'single': 5, 'grouped_bf16': 6}


class Dims(ctypes.Structure):
    """Mirror of k3moe_dims in include/k3moe.h."""
    _fields_ = [('tokens', ctypes.c_int32), ('experts', ctypes.c_int32), ('topk', ctypes.c_int32),
                ('hidden', ctypes.c_int32), ('latent', ctypes.c_int32), ('inter', ctypes.c_int32),
                ('gating', ctypes.c_int32), ('activation', ctypes.c_int32), ('x_dtype', ctypes.c_int32),
                ('path', ctypes.c_int32)]


class LatentDims(ctypes.Structure):
    """Mirror of k3moe_latent_dims in include/k3moe.h."""
    _fields_ = [('tokens', ctypes.c_int32), ('hidden', ctypes.c_int32), ('latent', ctypes.c_int32),
                ('shared', ctypes.c_int32), ('activation', ctypes.c_int32)]


class Layout(ctypes.Structure):
    """Mirror of k3moe_layout in include/k3moe.h (byte offsets of the grouping lists)."""
    _fields_ = [(n, ctypes.c_int64) for n in ('active_count', 'active', 'offsets', 'counts', 'pair_token',
                                               'pair_weight', 'pair_of', 'pair_h', 'pair_y', 'input_split',
                                               'h_split')]


# bits of the workspace status word (include/k3moe.h K3MOE_STATUS_*)
STATUS_TIMEOUT, STATUS_ROUTES = 1, 2

EXPORTS = ('k3moe_workspace_bytes', 'k3moe_workspace_init', 'k3moe_workspace_status', 'k3moe_moe_step',
           'k3moe_mxfp4_decode', 'k3moe_last_error', 'k3moe_version', 'k3moe_latent_workspace_bytes',
           'k3moe_latent_in', 'k3moe_latent_out', 'k3moe_latent_moe_step', 'k3moe_latent_block', 'k3moe_workspace_layout',
           'k3moe_moe_step_noalloc', 'k3moe_mxfp4_encode', 'k3moe_activation', 'k3moe_debug_stall')

_lib = None


class NativeError(RuntimeError):
    """A libk3moe call returned a non-zero status."""


def load(path: str | None = None):
    """Load libk3moe.so (once) and declare the C signatures. Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise ImportError(f'libk3moe.so not found at {path}; build it with '
                          f'`python -c "import __graft_entry__ as g; g.build()"`')
    lib = ctypes.CDLL(path)
    p, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    lib.k3moe_workspace_bytes.argtypes = [ctypes.POINTER(Dims), ctypes.POINTER(sz)]
    lib.k3moe_workspace_bytes.restype = ctypes.c_int
    lib.k3moe_workspace_init.argtypes = [p, sz, p]
    lib.k3moe_workspace_init.restype = ctypes.c_int
    lib.k3moe_workspace_status.argtypes = [p, ctypes.POINTER(i32), p]
    lib.k3moe_workspace_status.restype = ctypes.c_int
    lib.k3moe_moe_step.argtypes = [ctypes.POINTER(Dims)] + [p]*15 + [p, sz, p]
    lib.k3moe_moe_step.restype = ctypes.c_int
    lib.k3moe_moe_step_noalloc.argtypes = [ctypes.POINTER(Dims)] + [p]*15 + [p]
    lib.k3moe_moe_step_noalloc.restype = ctypes.c_int
    lib.k3moe_workspace_layout.argtypes = [ctypes.POINTER(Dims), ctypes.POINTER(Layout)]
    lib.k3moe_workspace_layout.restype = ctypes.c_int
    lib.k3moe_mxfp4_decode.argtypes = [p, p, i64, i32, p, p]
    lib.k3moe_mxfp4_decode.restype = ctypes.c_int
    lib.k3moe_mxfp4_encode.argtypes = [p, i32, i64, p, p, p]
    lib.k3moe_mxfp4_encode.restype = ctypes.c_int
    lib.k3moe_activation.argtypes = [i32, i32, p, p, p, i64, p]
    lib.k3moe_activation.restype = ctypes.c_int
    lib.k3moe_debug_stall.argtypes = [i32]
    lib.k3moe_debug_stall.restype = ctypes.c_int
    lib.k3moe_latent_workspace_bytes.argtypes = [ctypes.POINTER(LatentDims), ctypes.POINTER(sz)]
    lib.k3moe_latent_workspace_bytes.restype = ctypes.c_int
    lib.k3moe_latent_in.argtypes = [ctypes.POINTER(LatentDims)] + [p]*6 + [p, sz, p]
    lib.k3moe_latent_in.restype = ctypes.c_int
    lib.k3moe_latent_out.argtypes = [ctypes.POINTER(LatentDims)] + [p]*6 + [p, sz, p]
    lib.k3moe_latent_out.restype = ctypes.c_int
    lib.k3moe_latent_moe_step.argtypes = [ctypes.POINTER(Dims), i32] + [p]*6 + [p]*13 + [p, sz, p]
    lib.k3moe_latent_moe_step.restype = ctypes.c_int
    lib.k3moe_latent_block.argtypes = [ctypes.POINTER(Dims), i32] + [p]*23 + [p, sz, p]
    lib.k3moe_latent_block.restype = ctypes.c_int
    lib.k3moe_last_error.argtypes = []
    lib.k3moe_last_error.restype = ctypes.c_char_p
    lib.k3moe_version.argtypes = []
    lib.k3moe_version.restype = ctypes.c_char_p
    if path == LIB_PATH:
        _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != K3MOE_OK:
        msg = load().k3moe_last_error().decode(errors='replace')
        if rc == -1:
            raise ValueError(f'{what}: {msg}')
        raise NativeError(f'{what} failed ({rc}): {msg}')
