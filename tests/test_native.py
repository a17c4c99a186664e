"""The C-ABI library loads and exports what include/k3moe.h declares (no GPU calls)."""

import ctypes
import os
import re

import pytest
import torch

from k3moe import _native, moe
from k3moe.configs import ALL as CONFIGS

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'include', 'k3moe.h')


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'^\s*(?:int|const char \*)\s*(k3moe_\w+)\s*\(', text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_functions()
    assert set(names) == set(_native.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.k3moe_version().decode().startswith('k3moe')


def test_debug_stall_takes_only_non_negative_polls():
    lib = _native.load()
    assert lib.k3moe_debug_stall(-1) == -1
    assert 'polls' in lib.k3moe_last_error().decode()
    assert lib.k3moe_debug_stall(0) == 0


def test_dims_struct_matches_header():
    text = open(HEADER).read()
    body = re.search(r'typedef struct k3moe_dims \{(.*?)\} k3moe_dims;', text, flags=re.S).group(1)
    fields = re.findall(r'int32_t\s+(\w+);', body)
    assert fields == [f for f, _ in _native.Dims._fields_]


@pytest.mark.parametrize('name', sorted(CONFIGS))
def test_workspace_bytes_for_every_config(name):
    c = CONFIGS[name]
    d = _native.Dims(tokens=c.tokens, experts=c.experts, topk=c.topk, hidden=c.hidden, latent=c.width,
                     inter=c.inter, gating=_native.GATING[c.gating], activation=_native.ACTIVATION[c.activation],
                     x_dtype=0, path=0)
    n = moe.workspace_bytes(d)
    assert n > 0 and n % 256 == 0
    # the activated intermediates alone need B k I bf16 values
    assert n >= c.tokens * c.topk * c.inter * 2


@pytest.mark.parametrize('field,value,msg', [
    ('experts', 0, 'experts'), ('experts', 2000, 'experts'), ('topk', 0, 'topk'), ('topk', 33, 'topk'),
    ('hidden', 100, 'hidden'), ('latent', 48, 'latent'), ('inter', 40, 'inter'), ('gating', 7, 'gating'),
    ('activation', 9, 'activation'), ('x_dtype', 1, 'x_dtype'), ('path', 7, 'path'), ('path', -1, 'path'),
    ('path', 3, 'grouped GEMM path needs latent'), ('tokens', 0, 'tokens')])
def test_invalid_dims_are_rejected_with_a_message(field, value, msg):
    d = _native.Dims(tokens=2, experts=16, topk=4, hidden=64, latent=64, inter=64, gating=0, activation=0,
                     x_dtype=0, path=0)
    setattr(d, field, value)
    with pytest.raises(ValueError, match=msg):
        moe.workspace_bytes(d)


def test_moe_step_rejects_host_tensors_and_bad_dtypes():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    r = torch.zeros(8, 64, dtype=torch.bfloat16)
    gb = torch.zeros(8, 64, 2, 16, dtype=torch.uint8)
    gs = torch.zeros(8, 64, 2, dtype=torch.uint8)
    db = torch.zeros(8, 64, 2, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match='ROCm GPU'):
        moe.moe_step(x, r, None, gb, gs, gb, gs, db, gs, topk=2)
    with pytest.raises(NotImplementedError):
        moe.moe_step(x, r, None, gb, gs, gb, gs, db, gs, topk=2, fp32=True)
    with pytest.raises(ValueError, match='uint8'):
        moe.mxfp4_decode(torch.zeros(2, 16, dtype=torch.int8), torch.zeros(2, dtype=torch.uint8))
    with pytest.raises(ValueError, match='geometry'):
        moe.mxfp4_decode(torch.zeros(2, 8, dtype=torch.uint8), torch.zeros(2, dtype=torch.uint8))


def test_product_package_does_not_import_the_oracle():
    pkg = os.path.dirname(os.path.abspath(moe.__file__))
    for root, _, files in os.walk(os.path.dirname(pkg)):
        for f in files:
            if f.endswith(('.py', '.hip', '.hpp', '.cpp', '.h')):
                text = open(os.path.join(root, f)).read()
                assert not re.search(r'^\s*(from|import)\s+oracle\b', text, flags=re.M), f
                assert 'liborc' not in text, f


def test_submission_build_validates_the_case():
    from k3moe import submission
    case = {'params': {'tokens': 2, 'experts': 16, 'topk': 4, 'hidden': 64, 'inter': 64}}
    assert callable(submission.build(case))
    with pytest.raises(ValueError, match='params'):
        submission.build({'params': {'tokens': 2}})
    with pytest.raises(ValueError, match='gating'):
        submission.build(dict(case, gating='top1'))
    with pytest.raises(ValueError, match='geometry'):
        submission.build({'params': dict(case['params'], hidden=48)})
    run = submission.build(case)
    with pytest.raises(ValueError, match='x must be'):
        run({'x': torch.zeros(3, 64, dtype=torch.bfloat16)})


def test_latent_dims_struct_matches_header():
    text = open(HEADER).read()
    body = re.search(r'typedef struct k3moe_latent_dims \{(.*?)\} k3moe_latent_dims;', text, flags=re.S).group(1)
    fields = re.findall(r'int32_t\s+(\w+);', body)
    assert fields == [f for f, _ in _native.LatentDims._fields_]


@pytest.mark.parametrize('B', [1, 8, 64, 200])
def test_latent_workspace_bytes_kimi_rank(B):
    from k3moe import latent
    n = latent.latent_workspace_bytes(latent.latent_dims(B, 7168, 3584, 768))
    # at least the counters' area and one split's fp32 partials of every output row
    assert n % 256 == 0 and n >= 4096 + 65536 + 16384 + min(B, 64)*7168*4
    if B > 64:   # launches of 64 token rows: the 64-row workspace serves them
        assert n == latent.latent_workspace_bytes(latent.latent_dims(64, 7168, 3584, 768))


@pytest.mark.parametrize('dims,msg', [
    ((0, 7168, 3584, 768), 'tokens'), ((-3, 7168, 3584, 768), 'tokens'), ((8, 7100, 3584, 768), 'multiples of 128'),
    ((8, 7168, 3500, 768), 'multiples of 128'), ((8, 7168, 3584, 0), 'multiples of 128'),
    ((64, 16384, 8192, 1024), 'does not fit')])
def test_latent_invalid_dims_are_rejected(dims, msg):
    from k3moe import latent
    with pytest.raises(ValueError, match=msg):
        latent.latent_workspace_bytes(latent.latent_dims(*dims))
    with pytest.raises(ValueError, match='activation'):
        latent.latent_dims(8, 7168, 3584, 768, activation='gelu')


def test_latent_rejects_host_tensors():
    from k3moe import latent
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    w = torch.zeros(128, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match='ROCm GPU'):
        latent.latent_in(x, w, w, w)
    with pytest.raises(NotImplementedError):
        latent.latent_block(x, {}, topk=2, fp32=True)


def test_integration_ctypes_snippet_matches_the_binding():
    """The ctypes declaration documented for other callers has the argument counts _native.py uses."""
    doc = open(os.path.join(os.path.dirname(HEADER), '..', 'INTEGRATION.md')).read()
    lib = _native.load()
    for name, want in (('k3moe_moe_step', lib.k3moe_moe_step.argtypes),
                       ('k3moe_latent_in', lib.k3moe_latent_in.argtypes)):
        m = re.search(rf'lib\.{name}\.argtypes = \[ctypes\.POINTER\(\w+\)\] \+ \[ctypes\.c_void_p\] \* (\d+) \+', doc)
        assert m, name
        assert 1 + int(m.group(1)) + 3 == len(want), name
    # and the header's pointer count for the step: 15 device pointers between dims and the workspace
    text = open(HEADER).read()
    decl = re.search(r'int k3moe_moe_step\((.*?)\);', text, flags=re.S).group(1)
    params = [p.strip() for p in decl.split(',')]
    assert len(params) == 1 + 15 + 3


def test_init_size_agrees_across_header_library_and_python():
    """k3moe_workspace_init's zeroed prefix: the library's size (from its size check, which fails
    before anything is launched), the header's documented number and moe.INIT_BYTES agree."""
    lib = _native.load()
    rc = lib.k3moe_workspace_init(ctypes.c_void_p(256), ctypes.c_size_t(16), None)
    assert rc == -2
    n = int(re.search(r'at least (\d+) bytes', lib.k3moe_last_error().decode()).group(1))
    assert n == moe.INIT_BYTES
    text = open(HEADER).read()
    assert int(re.search(r"Zero the workspace's first (\d+) bytes", text).group(1)) == n


@pytest.mark.parametrize('K,I,fp4', [(1024, 512, True), (512, 256, True), (7168, 2048, True), (768, 384, False),
                                     (1024, 384, False), (768, 512, False), (1024, 128, False)])
def test_fp4_grouped_gemms_only_for_whole_output_units(K, I, fp4):
    """The FP4-MFMA grouped GEMMs write 256 columns of I (gate/up) or 512 of the latent (down) per
    work unit, so the plan takes them only when both widths are whole multiples; other grouped
    shapes run the bf16-MFMA GEMMs (no activation split in the workspace, h kept in bf16)."""
    d = _native.Dims(tokens=512, experts=32, topk=4, hidden=K, latent=K, inter=I, gating=0, activation=0,
                     x_dtype=0, path=_native.PATH['grouped'])
    lay = moe.workspace_layout(d)
    assert (lay['input_split'] >= 0) == fp4
    assert (lay['h_split'] >= 0) == fp4
    assert (lay['pair_h'] == -1) == fp4


def test_device_code_has_no_packed_fp32():
    from k3moe import build
    assert build.check_no_packed_fp32(_native.LIB_PATH) > 100_000


PACKED_PROBE = r'''
#include <hip/hip_runtime.h>
extern "C" __global__ void probe(float2* a, const float2* b, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) { float2 x = a[i], y = b[i]; x.x = x.x * y.x + 1.0f; x.y = x.y * y.y + 1.0f; a[i] = x; }
}
'''


def test_packed_fp32_check_sees_what_the_option_removes(tmp_path):
    """A float2 kernel built without the option holds packed FP32 and fails the
    check; built with the library's options it passes."""
    import subprocess
    from k3moe import build
    src = tmp_path / 'probe.hip'
    src.write_text(PACKED_PROBE)
    flags = build.command(str(tmp_path / 'with.so'))
    cmd_with = [a if a != os.path.join(build.CSRC, 'k3moe.hip') else str(src) for a in flags]
    cmd_without = [a for a in cmd_with if a not in ('-Xclang', '-target-feature', '-packed-fp32-ops')]
    cmd_without[cmd_without.index(str(tmp_path / 'with.so'))] = str(tmp_path / 'without.so')
    subprocess.run(cmd_with, check=True, capture_output=True)
    subprocess.run(cmd_without, check=True, capture_output=True)
    build.check_no_packed_fp32(str(tmp_path / 'with.so'))
    with pytest.raises(RuntimeError, match='packed FP32'):
        build.check_no_packed_fp32(str(tmp_path / 'without.so'))
