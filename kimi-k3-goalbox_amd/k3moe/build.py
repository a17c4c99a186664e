"""Compile libk3moe.so for gfx950 in-tree with hipcc (no torch C++ extension).

The library is plain `extern "C"` HIP code loaded with ctypes, so it does not
depend on torch's headers or ABI. Packed FP32 instructions are disabled for
the device code (-target-feature -packed-fp32-ops). Floating-point contraction
is off (-ffp-contract=off): every product and sum rounds where the source
writes it, as torch's separate operations do (the combine's w x bf16(y) is
rounded before it is added, kimi.py:323); HIP's default would fuse them into
one FMA with a single rounding (its __fmul_rn / __fadd_rn are plain operators).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
CSRC = os.path.join(PKG_ROOT, 'csrc')
REPO = os.path.dirname(PKG_ROOT)
OUT = os.path.join(HERE, 'libk3moe.so')
ARCH = os.environ.get('K3MOE_ARCH', 'gfx950')

SOURCES = ['k3moe.hip']
HEADERS = ['k3moe_device.hpp']


def hipcc() -> str:
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError('hipcc not found')


def command(out: str = OUT) -> list[str]:
    return [hipcc(), f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared', '-ffp-contract=off',
            '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
            '-Wno-unused-command-line-argument',
            '-I', os.path.join(REPO, 'include'),
            *[os.path.join(CSRC, s) for s in SOURCES], '-o', out]


def build(verbose: bool = False) -> str:
    """Compile every HIP source into libk3moe.so (always rebuilds) and return its path."""
    tmp = OUT + '.tmp'
    cmd = command(tmp)
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = [ln for ln in res.stderr.splitlines() if 'packed-fp32-ops' not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError('hipcc failed:\n' + res.stderr)
    if verbose and noise:
        print('\n'.join(noise), file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == '__main__':
    print(build(verbose=True))
