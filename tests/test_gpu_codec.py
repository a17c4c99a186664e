"""GPU parity of the MXFP4 encoder k3moe.pack_mxfp4 (quantization.py:13-37) (run with -m gpu).

Bar: packed bytes and scale bytes bit-exact with the oracle (oracle/pack_ref.py,
the torch CPU chain, itself pinned in tests/test_oracle_pack.py) on seeded
inputs of every accepted dtype, the rounding boundaries, the block-exponent
grid, the special blocks and ragged shapes; at a TP8 rank's expert size the
size-independent properties (decode(encode(v)) == v for decoder outputs, and
encode(x) equal to the oracle on sampled rows); the input is not mutated.
Every test prints its case before touching the GPU.
"""

import numpy as np
import pytest
import torch

import k3moe
from oracle import moe_ref, pack_ref

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def gpu_pack(x: torch.Tensor, dev):
    xd = x.to(dev)
    before = xd.clone()
    p, s = k3moe.pack_mxfp4(xd)
    torch.cuda.synchronize(dev)
    assert torch.equal(xd.view(torch.uint8), before.view(torch.uint8))
    return p.cpu(), s.cpu()


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize('shape,scale', [((3, 64), 1.0), ((7, 5, 2048), 0.02), ((1, 7168), 300.0),
                                         ((333, 96), 1e-4)])
def test_encode_matches_oracle(gpu, dtype, shape, scale):
    say(f'case: encode {dtype} {shape} scale {scale}')
    g = torch.Generator().manual_seed(sum(shape) + 7*str(dtype).count('16'))
    x = (torch.randn(*shape, generator=g)*scale).to(dtype)
    flat = x.view(-1, shape[-1])
    flat[0, :32] = 0                                   # zero block
    if flat.shape[-1] >= 64:
        flat[0, 32:64] *= torch.logspace(-5, 0, 32).to(dtype)
    p, s = gpu_pack(x, gpu)
    q, t = pack_ref.pack_mxfp4(x)
    assert p.shape == q.shape and s.shape == t.shape
    assert torch.equal(s, t)
    assert torch.equal(p, q)


def test_encode_boundaries_and_specials(gpu):
    say('case: encode boundary table, exponent grid, special blocks')
    from test_oracle_pack import _boundary_table, exponent_grid
    rows = _boundary_table()
    base = np.array([v for v, _ in rows], np.float64)
    x = np.stack([(base*2.0**n).astype(np.float32) for n in range(-126, 126, 5)])
    x = np.concatenate([x, -x])
    _, _, m, _ = exponent_grid()
    grid = np.zeros((m.size, 32), np.float32)
    grid[:, 0] = m.reshape(-1)
    grid[:, 1] = -m.reshape(-1)/3
    spec = np.zeros((5, 32), np.float32)
    spec[0, 3], spec[0, 4], spec[0, 5] = np.nan, np.inf, -2.0
    spec[1, 7], spec[1, 8], spec[1, 9] = -np.inf, -1.0, 3.0e38
    spec[2, 0], spec[2, 1] = 1e-45, -1e-45
    spec[3, :] = -0.0
    spec[4, :] = np.float32(2.0**-140)*np.arange(-16, 16)     # subnormal block
    allx = torch.from_numpy(np.concatenate([x, grid, spec]))
    p, s = gpu_pack(allx, gpu)
    q, t = pack_ref.pack_mxfp4(allx)
    assert torch.equal(s, t)
    assert torch.equal(p, q)


def test_encode_empty_and_ragged(gpu):
    say('case: encode empty and ragged inputs')
    p, s = k3moe.pack_mxfp4(torch.zeros(0, 64, device=gpu))
    assert p.shape == (0, 2, 16) and s.shape == (0, 2)
    with pytest.raises(ValueError, match='divisible by 32'):
        k3moe.pack_mxfp4(torch.zeros(4, 48, device=gpu))
    # a non-contiguous view and an integer tensor (cast to float32 first, as matrix.float())
    x = torch.randn(64, 128, device=gpu).t()
    p, s = k3moe.pack_mxfp4(x)
    q, t = pack_ref.pack_mxfp4(x.cpu())
    assert torch.equal(p.cpu(), q) and torch.equal(s.cpu(), t)
    # a contiguous view that starts 8 bytes into its storage
    base = torch.randn(8 + 4*64, device=gpu).to(torch.bfloat16)
    xv = base[4:4 + 4*64].view(4, 64)
    p, s = k3moe.pack_mxfp4(xv)
    q, t = pack_ref.pack_mxfp4(xv.cpu())
    assert torch.equal(p.cpu(), q) and torch.equal(s.cpu(), t)
    xi = torch.randint(-40, 40, (4, 64), device=gpu, dtype=torch.int32)
    p, s = k3moe.pack_mxfp4(xi)
    q, t = pack_ref.pack_mxfp4(xi.cpu())
    assert torch.equal(p.cpu(), q) and torch.equal(s.cpu(), t)


def test_encode_tp8_rank_gate_round_trip(gpu):
    """A TP8 rank's gate weights (384 x 256 x 7168): decode -> encode -> decode is the identity
    (decoder outputs are exactly representable), and bf16 weights encode as the oracle does on
    sampled experts."""
    say('case: encode round trip at 384 x 256 x 7168')
    g = torch.Generator(device=gpu).manual_seed(5)
    blocks = torch.randint(0, 256, (384, 256, 224, 16), generator=g, device=gpu, dtype=torch.uint8)
    scales = torch.randint(119, 124, (384, 256, 224), generator=g, device=gpu, dtype=torch.uint8)
    v = k3moe.mxfp4_decode(blocks, scales, torch.bfloat16)
    p, s = k3moe.pack_mxfp4(v)
    back = k3moe.mxfp4_decode(p, s, torch.bfloat16)
    assert torch.equal(back.view(torch.int16) & 0x7FFF, v.view(torch.int16) & 0x7FFF)   # -0.0 -> +0.0
    assert bool(((back.view(torch.int16) == v.view(torch.int16)) | (v == 0)).all())
    del back
    w = (torch.randn(384, 256, 7168, generator=g, device=gpu)*0.02).to(torch.bfloat16)
    p, s = k3moe.pack_mxfp4(w)
    for e in (0, 191, 383):
        q, t = pack_ref.pack_mxfp4(w[e].cpu())
        assert torch.equal(p[e].cpu(), q) and torch.equal(s[e].cpu(), t), e
    ref_dec = moe_ref.unpack_mxfp4(p[7].cpu(), s[7].cpu())
    err = (ref_dec - w[7].float().cpu()).abs()
    assert float(err.max()) <= float(w[7].float().abs().amax().cpu())/3    # half a code step at most
