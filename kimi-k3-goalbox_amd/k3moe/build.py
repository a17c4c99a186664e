"""Compile libk3moe.so for gfx950 in-tree with hipcc (no torch C++ extension).

The library is plain `extern "C"` HIP code loaded with ctypes, so it does not
depend on torch's headers or ABI. Packed FP32 instructions are disabled for
the device code (-Xclang -target-feature -Xclang -packed-fp32-ops). hipcc hands
that option to both compiler passes and the host (x86) pass prints
"'-packed-fp32-ops' is not a recognized feature for this target"; the device
pass applies it. Every build then disassembles the gfx950 code object of the
new library and fails if a v_pk_add_f32, v_pk_mul_f32 or v_pk_fma_f32 is in it
(`check_no_packed_fp32`), so the guard does not rest on the option alone.

Floating-point contraction is off (-ffp-contract=off): every product and sum
rounds where the source writes it, as torch's separate operations do (the
combine's w x bf16(y) is rounded before it is added, kimi.py:323); HIP's
default would fuse them into one FMA with a single rounding (its __fmul_rn /
__fadd_rn are plain operators).
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


HOST_PASS_NOTE = "'-packed-fp32-ops' is not a recognized feature for this target"
PACKED_FP32 = ('v_pk_add_f32', 'v_pk_mul_f32', 'v_pk_fma_f32')


def llvm_tool(name: str) -> str:
    for root in (os.environ.get('ROCM_PATH', '/opt/rocm'), '/opt/rocm'):
        path = os.path.join(root, 'llvm', 'bin', name)
        if os.path.exists(path):
            return path
    raise RuntimeError(f'{name} not found under the ROCm llvm tools')


def device_disassembly(lib: str) -> str:
    """The gfx950 code object of `lib`, disassembled (llvm-objdump, in a scratch directory)."""
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        copy = os.path.join(tmp, 'lib.so')
        shutil.copyfile(lib, copy)
        subprocess.run([llvm_tool('llvm-objdump'), '--offloading', copy], cwd=tmp, check=True,
                       capture_output=True, text=True)
        objs = [f for f in os.listdir(tmp) if f.endswith(f'amdgcn-amd-amdhsa--{ARCH}')]
        if len(objs) != 1:
            raise RuntimeError(f'expected one {ARCH} code object in {lib}, found {objs}')
        res = subprocess.run([llvm_tool('llvm-objdump'), '-d', f'--mcpu={ARCH}', objs[0]], cwd=tmp,
                             check=True, capture_output=True, text=True)
        return res.stdout


def check_no_packed_fp32(lib: str = OUT) -> int:
    """Raise if the library's device code holds a packed-FP32 add, multiply or FMA;
    return the number of instructions checked."""
    text = device_disassembly(lib)
    found = sorted({op for op in PACKED_FP32 if op in text})
    if found:
        raise RuntimeError(f'{lib}: packed FP32 instructions in the device code: {found}')
    return sum(1 for ln in text.splitlines() if ln.startswith('\t'))


def build(verbose: bool = False) -> str:
    """Compile every HIP source into libk3moe.so (always rebuilds), check its
    device code for packed FP32 and return its path."""
    tmp = OUT + '.tmp'
    cmd = command(tmp)
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError('hipcc failed:\n' + res.stderr)
    lines = [ln for ln in res.stderr.splitlines() if ln.strip()]
    host_notes = [ln for ln in lines if HOST_PASS_NOTE in ln]
    other = [ln for ln in lines if HOST_PASS_NOTE not in ln]
    if verbose and host_notes:
        print(f'hipcc host pass: {HOST_PASS_NOTE} (x{len(host_notes)}; the device pass applies it)',
              file=sys.stderr)
    if verbose and other:
        print('\n'.join(other), file=sys.stderr)
    n = check_no_packed_fp32(tmp)
    if verbose:
        print(f'device code: {n} instructions, no packed FP32', flush=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == '__main__':
    print(build(verbose=True))
