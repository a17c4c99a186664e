"""CPU pins of the oracle's MXFP4 encoder (oracle/pack_ref.py, quantization.py:13-37).

pack_mxfp4 (the torch restatement) is trusted only after:
  * agreement with pack_mxfp4_f64, a brute force that picks the nearest E2M1
    magnitude by float64 distance (ties to the even code) and takes the block
    exponent from a float64 log2 rounded once to fp32, on random data of
    several dtypes and magnitudes;
  * hand-computed codes at every rounding boundary and one float32 step to
    either side, at several block exponents;
  * the block exponent at 2^n (1 + j 2^-23) for every binade n and j < 64,
    including hand-checked cases where the rounded fp32 logarithm keeps n;
  * decode(encode(v)) == v for every value the decoder produces (all 16
    codes at every finite scale);
  * the NaN / infinity / zero / subnormal rules;
and planted mistakes in the oracle (a moved tie boundary, an exact
logarithm) fail these checks.
"""

import numpy as np
import pytest
import torch

from oracle import moe_ref, pack_ref


def both(x: torch.Tensor):
    p, s = pack_ref.pack_mxfp4(x)
    q, t = pack_ref.pack_mxfp4_f64(x.float().numpy())
    return p.numpy(), s.numpy(), q, t


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize('scale', [1.0, 1e-3, 37.0])
def test_encoder_matches_brute_force(dtype, scale):
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(24, 256, generator=g) * scale).to(dtype)
    x[0, :32] = 0.0                       # an all-zero block
    x[1, 5] = -0.0
    x[2, :32] *= torch.logspace(-6, 0, 32)  # mixed magnitudes inside a block
    p, s, q, t = both(x)
    assert p.shape == (24, 8, 16) and s.shape == (24, 8)
    assert np.array_equal(s, t)
    assert np.array_equal(p, q)


def codes_of(packed: np.ndarray) -> np.ndarray:
    """Codes of packed [..., n, 16] as [..., 32 n] (element order)."""
    return np.stack([packed & 15, packed >> 4], -1).reshape(*packed.shape[:-2], -1)


# (value, code) at a block exponent of 0 (block maximum 6): the rounding
# boundaries of quantization.py:29-34, ties to the even code, and one float32
# step to either side.
def _boundary_table():
    up = lambda v: float(np.nextafter(np.float32(v), np.float32(np.inf)))   # noqa: E731
    dn = lambda v: float(np.nextafter(np.float32(v), np.float32(0)))        # noqa: E731
    rows = [(0.0, 0), (0.25, 0), (up(0.25), 1), (0.5, 1), (dn(0.75), 1), (0.75, 2), (up(0.75), 2),
            (1.0, 2), (dn(1.25), 2), (1.25, 2), (up(1.25), 3), (1.5, 3), (dn(1.75), 3), (1.75, 4), (up(1.75), 4),
            (2.0, 4), (dn(2.5), 4), (2.5, 4), (up(2.5), 5), (3.0, 5), (dn(3.5), 5), (3.5, 6), (up(3.5), 6),
            (4.0, 6), (dn(5.0), 6), (5.0, 6), (up(5.0), 7), (5.9, 7)]
    assert len(rows) == 28
    return rows + [(6.0, 7), (-0.5, 9), (-0.75, 10), (-1.25, 10)]


@pytest.mark.parametrize('n', [0, -20, 7, 90])
def test_boundary_codes_by_hand(n):
    rows = _boundary_table()
    vals = np.array([v for v, _ in rows], np.float64) * 2.0**n
    want = np.array([c for _, c in rows], np.uint8)
    x = torch.from_numpy(vals.astype(np.float32)).reshape(1, 32)
    p, s, q, t = both(x)
    assert s[0, 0] == 127 + n and t[0, 0] == 127 + n
    assert np.array_equal(codes_of(p)[0], want)
    assert np.array_equal(codes_of(q)[0], want)


def exponent_grid():
    """Block maxima whose quotient by 6 is 2^n (1 + j 2^-23), n in [-126, 126], j in [0, 64)."""
    n = np.arange(-126, 127)
    j = np.arange(64)
    v = np.ldexp((1.0 + j[None, :] * 2.0**-23), n[:, None]).astype(np.float32)
    with np.errstate(over="ignore"):
        m = (v.astype(np.float64) * 6.0).astype(np.float32)
    keep = (m / np.float32(6.0)) == v          # maxima that give back exactly that quotient
    return n, j, m, keep


def test_block_exponent_every_binade():
    n, j, m, keep = exponent_grid()
    x = np.zeros((m.size, 32), np.float32)
    x[:, 0] = m.reshape(-1)
    p, s = pack_ref.pack_mxfp4(torch.from_numpy(x))
    e = s.numpy().astype(np.int64).reshape(m.shape) - 127
    assert np.array_equal(e, pack_ref.block_exponent_f64(m))
    assert keep.sum() > 0.9 * keep.size
    # hand-checked: the exact ceiling at j > 0 is n + 1, but one step above 2^-100 the rounded
    # fp32 log2 is exactly -100 (spacing 2^-17 there), while above 2^0 and 2^-1 it is not
    exact_ceiling = np.where(j[None, :] == 0, n[:, None], n[:, None] + 1)
    row = lambda nn: int(np.nonzero(n == nn)[0][0])   # noqa: E731
    assert keep[row(-100), 1] and e[row(-100), 1] == -100
    assert keep[row(0), 1] and e[row(0), 1] == 1
    assert keep[row(-1), 1] and e[row(-1), 1] == 0
    assert keep[row(5), 0] and e[row(5), 0] == 5
    differs = (e != exact_ceiling) & keep
    assert differs.any() and (j[None, :].repeat(n.size, 0)[differs] < 23).all()


def test_round_trip_every_code_and_scale():
    codes = np.arange(16, dtype=np.uint8)
    blocks = np.tile((codes[0::2] | (codes[1::2] << 4))[None, :], (252, 2))[:, :16]
    rng = np.random.default_rng(3)
    blocks = np.concatenate([blocks, rng.integers(0, 256, (252 * 4, 16), dtype=np.uint8)])
    scales = np.concatenate([np.arange(1, 253, dtype=np.uint8)] * 5)    # 253 and up overflow fp32 at code 7
    v = moe_ref.unpack_mxfp4(torch.from_numpy(blocks), torch.from_numpy(scales))
    p, s = pack_ref.pack_mxfp4(v)
    back = moe_ref.unpack_mxfp4(p, s)
    assert torch.equal(back, v)                           # -0.0 == 0.0; no NaN at scales < 255
    q, t = pack_ref.pack_mxfp4_f64(v.numpy())
    assert np.array_equal(q, p.numpy()) and np.array_equal(t, s.numpy())


def test_special_blocks():
    x = torch.zeros(4, 32)
    x[0, 3] = float('nan')
    x[0, 4] = float('inf')
    x[0, 5] = -2.0
    x[1, 7] = float('-inf')
    x[1, 8] = -1.0
    x[1, 9] = 3.0e38
    x[2, 0] = 1e-45                                       # subnormal input
    x[2, 1] = -1e-45
    x[3, :] = -0.0
    p, s, q, t = both(x)
    assert np.array_equal(p, q) and np.array_equal(s, t)
    c = codes_of(p)
    assert s[0, 0] == 127 and c[0, 3] == 7 and c[0, 4] == 7 and c[0, 5] == 0 and (c[0, 6:] == 0).all()
    assert s[1, 0] == 254 and c[1, 7] == 15
    assert c[1, 8] == 8                                   # -1 * 2^-127 stays a negative subnormal
    assert c[1, 9] == 4                                   # 3e38 * 2^-127 = 1.76 -> 2.0
    assert s[2, 0] == 1 and c[2, 0] == 0 and c[2, 1] == 8  # 2^-149 * 2^126: tiny but signed
    assert s[3, 0] == 1 and (c[3] == 0).all()             # -0.0 is not negative


def test_encoder_rejects_ragged_axis():
    with pytest.raises(ValueError, match='divisible by 32'):
        pack_ref.pack_mxfp4(torch.zeros(3, 48))
    with pytest.raises(ValueError, match='divisible by 32'):
        pack_ref.pack_mxfp4_f64(np.zeros((3, 48), np.float32))


def test_planted_mistakes_fail(monkeypatch):
    rows = _boundary_table()
    want = np.array([c for _, c in rows], np.uint8)
    x = torch.tensor([v for v, _ in rows], dtype=torch.float32).reshape(1, 32)
    # a tie boundary moved by one float32 step: 1.75 no longer rounds to the even code
    monkeypatch.setattr(pack_ref, 'BOUNDARIES', (0.25, 0.75, 1.25, float(np.nextafter(np.float32(1.75), 2)),
                                                 2.5, 3.5, 5.0))
    p, _ = pack_ref.pack_mxfp4(x)
    assert not np.array_equal(codes_of(p.numpy())[0], want)
    monkeypatch.undo()
    # an exact logarithm (float64) in place of torch's fp32 one
    monkeypatch.setattr(pack_ref.torch, 'log2', lambda t: torch.from_numpy(np.log2(t.double().numpy())))
    _, j, m, keep = exponent_grid()
    xx = np.zeros((m.size, 32), np.float32)
    xx[:, 0] = m.reshape(-1)
    _, s = pack_ref.pack_mxfp4(torch.from_numpy(xx))
    monkeypatch.undo()
    e = s.numpy().astype(np.int64).reshape(m.shape) - 127
    assert not np.array_equal(e, pack_ref.block_exponent_f64(m))
