"""CPU pins of the oracle (no GPU).

The oracle is trusted only after these checks:
  * decode: torch restatement == C bit construction == float64 closed form on
    every (byte, scale) pair, plus hand-computed special values and the
    committed code x scale table;
  * top-k / grouping: torch restatement == C restatement == brute force;
  * the FP32 expert chain == an independent float64 brute force (per token,
    closed-form decode) to FP32 rounding, on several seeds and both
    activations / gatings; a planted mistake fails it;
  * the BF16 expert chain (and the latent block's BF16 mode) == float64 brute
    forces rounded to bf16 at exactly the reference's casts, to ~1e-7; each
    planted dropped cast moves it by 5e-4 or more and fails;
  * band grader, shortfall and no-mutation rules behave as the reference's
    own unit tests require (megabench/tests/test_kimi.py:67-109).
"""

import os

import numpy as np
import pytest
import torch

from oracle import cdecode, grading, moe_ref

GOLDEN = os.path.join(os.path.dirname(__file__), 'golden')


def tiny_inputs(seed=0, E=8, k=2, h=64, I=64, B=3, gating='sigmoid_bias'):
    from k3moe import synthetic
    from k3moe.configs import MoEConfig
    cfg = MoEConfig('tiny', E, k, h, I, B, gating=gating)
    return cfg, synthetic.moe_layer_inputs(cfg, seed, scale_mode='kimi')


# ----------------------------------------------------------------- decode --

def all_pairs():
    blocks = np.tile(np.arange(256, dtype=np.uint8).reshape(1, 16, 16), (256, 1, 1))
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    return blocks, scales


def test_decode_three_restatements_agree_bitwise():
    blocks, scales = all_pairs()
    c = cdecode.mxfp4_decode_bits(blocks, scales)
    t = moe_ref.unpack_mxfp4(torch.from_numpy(blocks), torch.from_numpy(scales)).numpy().view(np.uint32)
    with np.errstate(over='ignore'):
        f = moe_ref._decode_f64(blocks, scales).astype(np.float32).view(np.uint32)
    assert c.shape == (256, 512)
    assert np.array_equal(c, t)
    assert np.array_equal(c, f)


def test_decode_special_values():
    def dec(byte, scale):
        return cdecode.mxfp4_decode_bits(np.full((1, 16), byte, np.uint8), np.array([scale], np.uint8))[:2]
    assert list(dec(0x21, 127).view(np.float32)) == [0.5, 1.0]           # low nibble is the even element
    assert list(dec(0x7F, 127).view(np.float32)) == [-6.0, 6.0]
    assert list(dec(0x88, 127)) == [0x80000000, 0x80000000]            # code 8 = -0.0
    assert list(dec(0x11, 0)) == [0x00200000, 0x00200000]              # 0.5 * 2^-127 = 2^-128, subnormal
    assert list(dec(0x33, 0)) == [0x00600000, 0x00600000]              # 1.5 * 2^-127
    assert list(dec(0x00, 255)) == [0x7FC00000, 0x7FC00000]            # scale 255 -> NaN, even for zero codes
    assert list(dec(0x37, 254)) == [0x7F800000, 0x7F400000]            # 6*2^127 = inf, 1.5*2^127 finite
    assert list(dec(0x44, 130).view(np.float32)) == [16.0, 16.0]       # 2 * 2^3


def test_decode_matches_committed_table():
    table = np.load(os.path.join(GOLDEN, 'mxfp4_code_scale_table.npy'))   # [scale][code] uint32
    assert table.shape == (256, 16) and table.dtype == np.uint32
    blocks = np.tile((np.arange(16, dtype=np.uint8) * 17).reshape(1, 1, 16), (256, 1, 1))  # byte = code | code<<4
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    bits = cdecode.mxfp4_decode_bits(blocks, scales)[:, 0:32:2]
    assert np.array_equal(bits, table)
    # closed form for every finite entry
    for s in range(255):
        for code in range(16):
            sign = -1.0 if code & 8 else 1.0
            e, m = (code >> 1) & 3, code & 1
            mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
            with np.errstate(over='ignore'):
                want = np.float32(sign * mag * 2.0 ** (s - 127))
            assert table[s, code] == want.view(np.uint32), (s, code)


def test_decode_rejects_bad_inputs():
    with pytest.raises(ValueError):
        moe_ref.unpack_mxfp4(torch.zeros(2, 16, dtype=torch.int8), torch.zeros(2, dtype=torch.uint8))
    with pytest.raises(ValueError):
        moe_ref.unpack_mxfp4(torch.zeros(2, 8, dtype=torch.uint8), torch.zeros(2, dtype=torch.uint8))


# ------------------------------------------------------- top-k / grouping --

def test_topk_restatements_agree():
    g = torch.Generator().manual_seed(7)
    v = torch.rand(50, 40, generator=g)
    v[3, 5] = v[3, 9] = v[3].max() + 1        # exact tie: lower index first
    v[4, 2] = float('nan')                     # NaN ranks first
    k = 6
    c = cdecode.topk_sorted(v.numpy(), k)
    t = moe_ref._stable_topk_desc(v, k).sort(-1).values.numpy()
    assert np.array_equal(c, t)
    assert 5 in c[3] and 9 in c[3]
    assert 2 in c[4]
    # brute force on tiny rows: enumerate all k-subsets
    import itertools
    small = torch.rand(5, 7, generator=g)
    for r in range(5):
        best = max(itertools.combinations(range(7), 3), key=lambda s: (sorted(small[r, list(s)].tolist())[0]))
        assert sorted(best) == list(cdecode.topk_sorted(small[r:r+1].numpy(), 3)[0])


def test_group_matches_nonzero_order():
    g = torch.Generator().manual_seed(3)
    B, E, k = 37, 20, 4
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(B)])
    counts, offsets, prow, pslot = cdecode.group(ids.numpy(), E)
    for e in range(E):
        rows, slots = (ids == e).nonzero(as_tuple=True)          # kimi.py:320
        lo, hi = offsets[e], offsets[e + 1]
        assert counts[e] == len(rows)
        assert list(prow[lo:hi]) == rows.tolist()
        assert list(pslot[lo:hi]) == slots.tolist()


# ------------------------------------------------------------ float chain --

@pytest.mark.parametrize('seed', [0, 1, 2])
@pytest.mark.parametrize('activation', ['situ', 'silu'])
def test_fp32_chain_matches_float64_brute_force(seed, activation):
    cfg, inp = tiny_inputs(seed)
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    r = moe_ref.moe_step(*args, topk=cfg.topk, activation=activation, fp32=True)
    ref = moe_ref.moe_step_f64(*args, routes=r['expert_ids'], weights=r['route_weights'], activation=activation)
    assert moe_ref.rel_l2(r['expert_sum'], ref) < 2e-6
    bf = moe_ref.moe_step(*args, topk=cfg.topk, activation=activation)
    err = moe_ref.rel_l2(bf['expert_sum'], ref)
    assert 1e-4 < err < 2e-2          # the BF16 oracle is visibly coarser than FP32, but close


BF16_CASES = [dict(), dict(E=16, k=4, h=256, I=128, B=5)]


@pytest.mark.parametrize('seed', [0, 1, 2])
@pytest.mark.parametrize('gating', ['sigmoid_bias', 'softmax'])
@pytest.mark.parametrize('activation', ['situ', 'silu'])
@pytest.mark.parametrize('shape', BF16_CASES, ids=['tiny', 'e16'])
def test_bf16_chain_matches_bf16_float64_brute_force(seed, gating, activation, shape):
    """The BF16 oracle equals a float64 brute force that rounds to bf16 at kimi.py:322's casts.

    They differ only by FP32 versus float64 arithmetic inside the sums, which
    flips a rounding rarely (measured 3-5e-8 rel-L2); a missing cast moves the
    result by 1.5e-3 or more (test_bf16_planted_dropped_casts_fail).
    """
    cfg, inp = tiny_inputs(seed, gating=gating, **shape)
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    r = moe_ref.moe_step(*args, topk=cfg.topk, gating=gating, activation=activation)
    ref = moe_ref.moe_step_bf16_f64(*args, routes=r['expert_ids'], weights=r['route_weights'],
                                    activation=activation)
    assert moe_ref.rel_l2(r['expert_sum'], ref) <= 1e-5


# plausible mistakes in the BF16 chain: one of kimi.py:322's casts dropped
BF16_PLANTS = {
    'gate/up not rounded': lambda x, wg, wu, wd, fn, cast: cast(cast(fn(x.float() @ wg.float().T,
                                                                        x.float() @ wu.float().T)) @ wd.T),
    'activation not rounded': lambda x, wg, wu, wd, fn, cast: cast(fn(x @ wg.T, x @ wu.T) @ wd.float().T),
    'down not rounded': lambda x, wg, wu, wd, fn, cast: cast(fn(x @ wg.T, x @ wu.T)).float() @ wd.float().T,
}


@pytest.mark.parametrize('plant', sorted(BF16_PLANTS))
@pytest.mark.parametrize('activation', ['situ', 'silu'])
def test_bf16_planted_dropped_casts_fail(monkeypatch, plant, activation):
    cfg, inp = tiny_inputs(1, E=16, k=4, h=256, I=128, B=5)
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    r = moe_ref.moe_step(*args, topk=cfg.topk, activation=activation)
    ref = moe_ref.moe_step_bf16_f64(*args, routes=r['expert_ids'], weights=r['route_weights'],
                                    activation=activation)
    monkeypatch.setattr(moe_ref, '_expert_out', BF16_PLANTS[plant])
    bad = moe_ref.moe_step(*args, topk=cfg.topk, activation=activation, routes=r['expert_ids'])
    assert moe_ref.rel_l2(bad['expert_sum'], ref) >= 1e-3


def test_bf16_round_f64_ties_and_torch():
    """Nearest bf16, ties to even, against hand values and torch's fp32 -> bf16 cast."""
    r = moe_ref.bf16_round_f64
    step = 2.0**-7                                                    # bf16 spacing in [1, 2)
    assert list(r(np.array([1 + step/2, 1 + 3*step/2, -(1 + step/2), 1 + step/2 + 2.0**-30]))) == \
        [1.0, 1 + 2*step, -1.0, 1 + step]
    assert list(r(np.array([0.0, -0.0, np.inf]))) == [0.0, 0.0, np.inf] and np.isnan(r(np.nan))
    g = torch.Generator().manual_seed(0)
    v = (torch.randn(20000, generator=g)*torch.exp(4*torch.randn(20000, generator=g))).float()
    assert np.array_equal(r(v.double().numpy()), v.bfloat16().double().numpy())


def test_pair_out_recombines_to_expert_sum():
    cfg, inp = tiny_inputs(4, E=16, k=4, h=128, I=64, B=6)
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    r = moe_ref.moe_step(*args, topk=cfg.topk, pair_out=True)
    assert r['pair_out'].shape == (6, 4, 128)
    # pair outputs are bf16 values; the weighted sum over ascending ids is the combine
    assert torch.equal(r['pair_out'], r['pair_out'].bfloat16().float())
    acc = torch.zeros(6, 128)
    for j in range(4):
        acc += r['pair_out'][:, j]*r['route_weights'][:, j, None]
    assert moe_ref.rel_l2(acc, r['expert_sum']) < 1e-6


def test_planted_mistake_fails_brute_force():
    cfg, inp = tiny_inputs(0)
    args = [inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                             'up_scales', 'down_blocks', 'down_scales')]
    r = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True)
    ref = moe_ref.moe_step_f64(*args, routes=r['expert_ids'], weights=r['route_weights'])
    # swap the gate and up operands: a plausible transposition mistake
    swapped = list(args)
    swapped[3], swapped[5] = args[5], args[3]
    swapped[4], swapped[6] = args[6], args[4]
    bad = moe_ref.moe_step(*swapped, topk=cfg.topk, fp32=True, routes=r['expert_ids'])
    assert moe_ref.rel_l2(bad['expert_sum'], ref) > 0.05


def test_routing_closed_form():
    cfg, inp = tiny_inputs(1, E=16, k=4, B=5)
    r = moe_ref.route(inp['x'], inp['router'], inp['router_bias'], 4)
    logits = inp['x'].double() @ inp['router'].double().T
    s = 1/(1 + torch.exp(-logits))
    biased = s + inp['router_bias'].double()
    for b in range(5):
        want = sorted(torch.argsort(biased[b], descending=True)[:4].tolist())
        assert r['expert_ids'][b].tolist() == want
        w = s[b, want] / s[b, want].sum()
        assert torch.allclose(r['route_weights'][b].double(), w, rtol=1e-6, atol=0)
    soft = moe_ref.route(inp['x'], inp['router'], None, 4, gating='softmax')
    for b in range(5):
        want = sorted(torch.argsort(logits[b], descending=True)[:4].tolist())
        assert soft['expert_ids'][b].tolist() == want
        p = torch.softmax(logits[b, want], 0)
        assert torch.allclose(soft['route_weights'][b].double(), p, rtol=1e-6, atol=0)


# ---------------------------------------------------------- grading rules --

def test_band_accepts_oracle_and_fp32_rejects_noise():
    cfg, inp = tiny_inputs(5)
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    bf = moe_ref.moe_step(*args, topk=cfg.topk)
    tr = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True, routes=bf['expert_ids'])
    grading.band_check(bf['expert_sum'], bf['expert_sum'], tr['expert_sum'], tr['expert_sum'])
    grading.band_check(tr['expert_sum'], bf['expert_sum'], tr['expert_sum'], tr['expert_sum'])
    g = torch.Generator().manual_seed(0)
    noisy = bf['expert_sum'] + 0.2*bf['expert_sum'].std()*torch.randn(bf['expert_sum'].shape, generator=g)
    with pytest.raises(AssertionError):
        grading.band_check(noisy, bf['expert_sum'], tr['expert_sum'], tr['expert_sum'])
    nan = bf['expert_sum'].clone()
    nan[0, 0] = float('nan')
    with pytest.raises(AssertionError):
        grading.band_check(nan, bf['expert_sum'], tr['expert_sum'], tr['expert_sum'])


def test_forced_routes_and_shortfall():
    cfg, inp = tiny_inputs(9)
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    own = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True)
    forced = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True, routes=own['expert_ids'])
    assert torch.equal(own['expert_sum'], forced['expert_sum'])
    assert float(forced['route_shortfall'].max()) == 0.0
    worst = torch.arange(cfg.experts - cfg.topk, cfg.experts).expand(cfg.tokens, -1)
    bad = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True, routes=worst)
    assert float(bad['route_shortfall'].max()) > grading.ROUTE_FLOOR
    assert grading.valid_routes(own['expert_ids'], cfg.experts)
    assert grading.valid_routes(own['expert_ids'].flip(-1), cfg.experts)
    rep = own['expert_ids'].clone()
    rep[:, 1] = rep[:, 0]
    assert not grading.valid_routes(rep, cfg.experts)


# Closed-form shortfall cases (kimi.py:311-313: kth-best biased score minus the
# lowest biased score among the forced routes, clamped at zero; the softmax
# variant's shortfall works on the raw logits). Token b's logits are the
# bf16-exact column b of the router, reached through a one-hot x row, so every
# score below is a textbook value: sigmoid(0) = 0.5, sigmoid(2) =
# 0.8807970779778823, sigmoid(-2) = 0.11920292202211755; biases are binary
# fractions. Each expected value is written out by hand.
SIG2, SIGM2 = 0.8807970779778823, 0.11920292202211755

SHORTFALL_CASES = [
    # (gating, k, per-token logits [E], bias [E], forced routes, expected shortfall)
    # the forced set takes the lowest biased expert: 1.125 - 0.5
    ('sigmoid_bias', 3, [0]*8, [0, .125, .25, .375, .5, .625, .75, .875], [0, 3, 7], 0.625),
    # the forced set is the top-k itself, in another order
    ('sigmoid_bias', 3, [0]*8, [0, .125, .25, .375, .5, .625, .75, .875], [6, 5, 7], 0.0),
    # a repeated forced id can sit above the kth best (1.25 > 1.125): the clamp gives 0
    # (the oracle accepts such a row as kimi.py does; the GPU path reports it as invalid)
    ('sigmoid_bias', 3, [0]*8, [0, .125, .25, .375, .5, .625, .75, .875], [7, 7, 6], 0.0),
    # one forced expert ties the kth best exactly (experts 1-3 all at 0.75)
    ('sigmoid_bias', 2, [0]*8, [0, .25, .25, .25, 0, 0, 0, 0], [1, 3], 0.0),
    # a known gap below a tie: kth best 0.75, forced min 0.5
    ('sigmoid_bias', 2, [0]*8, [0, .25, .25, .25, 0, 0, 0, 0], [0, 3], 0.25),
    # the bias reorders the sigmoid scores: biased = [s(2), .5, s(-2)+.5, .5, .5, .5, .5, .5]
    # top-2 = {0, 2}, kth = s(-2) + 0.5; forced {1, 3} have 0.5
    ('sigmoid_bias', 2, [2, 0, -2, 0, 0, 0, 0, 0], [0, 0, .5, 0, 0, 0, 0, 0], [1, 3], SIGM2),
    # forced onto the unbiased-best expert with a low biased score: kth = 0.5 + 0.25 (experts 4, 5),
    # forced {2, 4}: expert 2 has s(-2) + 0 -> shortfall 0.75 - s(-2)
    ('sigmoid_bias', 2, [2, 0, -2, 0, 0, 0, 0, 0], [-.5, 0, 0, 0, .25, .25, 0, 0], [2, 4], 0.75 - SIGM2),
    # the top score is forced with a much lower one: kth = s(2) - .5 vs. 0.5 + .375 ...
    # biased = [s(2) - .5, .5, s(-2), .875, .5, .5, .5, .5]: top-2 = {3, 1}; kth 0.5; forced {0, 3}
    ('sigmoid_bias', 2, [2, 0, -2, 0, 0, 0, 0, 0], [-.5, 0, 0, .375, 0, 0, 0, 0], [0, 3], 0.5 - (SIG2 - .5)),
    # softmax variant: shortfall on the logits; kth best 2, forced min -1
    ('softmax', 2, [3, 1, 2, -1, .5, 0, -2, .25], None, [1, 3], 3.0),
    ('softmax', 2, [3, 1, 2, -1, .5, 0, -2, .25], None, [2, 0], 0.0),
    ('softmax', 3, [3, 1, 2, -1, .5, 0, -2, .25], None, [0, 4, 2], 0.5),
]


def _shortfall_mismatches(route_fn):
    """Run every case through route_fn one token at a time and as one batch per
    (gating, k, bias); return the cases whose shortfall misses its hand value."""
    bad = []
    for i, (gating, k, logits, bias, forced, want) in enumerate(SHORTFALL_CASES):
        E = len(logits)
        router = torch.tensor(logits, dtype=torch.bfloat16)[:, None]          # [E, h=1]
        assert router.float().flatten().tolist() == [float(v) for v in logits]
        x = torch.ones(1, 1, dtype=torch.bfloat16)
        b = torch.tensor(bias, dtype=torch.float32) if bias is not None else None
        r = route_fn(x, router, b, k, gating, torch.tensor([forced]))
        got = float(r['route_shortfall'][0])
        if not abs(got - want) <= 1e-6:
            bad.append((i, got, want))
    # rows of one batch must not mix: token t reads column t of the router
    groups = {}
    for gating, k, logits, bias, forced, want in SHORTFALL_CASES:
        groups.setdefault((gating, k, tuple(bias) if bias else None), []).append((logits, forced, want))
    for (gating, k, bias), rows in groups.items():
        B = len(rows)
        router = torch.tensor([r[0] for r in rows], dtype=torch.bfloat16).T.contiguous()   # [E, B]
        x = torch.eye(B, dtype=torch.bfloat16)
        b = torch.tensor(bias, dtype=torch.float32) if bias is not None else None
        r = route_fn(x, router, b, k, gating, torch.tensor([r[1] for r in rows]))
        for t, (_, _, want) in enumerate(rows):
            got = float(r['route_shortfall'][t])
            if not abs(got - want) <= 1e-6:
                bad.append((gating, k, t, got, want))
    return bad


def _planted_route(old: str, new: str):
    """moe_ref.route with one source edit applied to its shortfall lines."""
    import inspect
    import textwrap
    src = textwrap.dedent(inspect.getsource(moe_ref.route))
    lines = [ln.replace(old, new) if ('route_shortfall' in ln or 'kth =' in ln) else ln
             for ln in src.splitlines()]
    mutated = '\n'.join(lines)
    assert mutated != src, f'planted edit {old!r} -> {new!r} changed nothing'
    ns = dict(vars(moe_ref))
    exec(compile(mutated, '<planted route>', 'exec'), ns)
    return ns['route']


def test_route_shortfall_closed_form():
    assert _shortfall_mismatches(moe_ref.route) == []


@pytest.mark.parametrize('old,new', [
    ('.min(-1)', '.max(-1)'),                      # the best forced score instead of the worst
    ('biased.gather', 'scores.gather'),            # unbiased sigmoid scores
    ('[:, -1]', '[:, 0]'),                         # the best score instead of the kth best
    ('.clamp_min(0)', ''),                         # no clamp at zero
])
def test_route_shortfall_planted_mistakes_fail(old, new):
    assert _shortfall_mismatches(_planted_route(old, new)) != []


def test_oracle_does_not_mutate_inputs():
    cfg, inp = tiny_inputs(17)
    before = grading.snapshot(inp)
    moe_ref.moe_step(*(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                        'up_scales', 'down_blocks', 'down_scales')), topk=cfg.topk)
    grading.check_unchanged(inp, before)
    inp['x'][0, 0] += 1
    with pytest.raises(AssertionError):
        grading.check_unchanged(inp, before)


def test_route_set_certification():
    cfg, inp = tiny_inputs(2, E=16, k=4, B=4)
    r = moe_ref.route(inp['x'], inp['router'], inp['router_bias'], 4)
    ok = grading.route_sets(r['expert_ids'], r['expert_ids'], inp['x'], inp['router'], inp['router_bias'], 4)
    assert ok['exact'] and ok['ok']
    other = r['expert_ids'].clone()
    b = r['biased'][0]
    order = torch.argsort(b, descending=True)
    other[0] = torch.cat([order[:3], order[4:5]]).sort().values     # swap the 4th and 5th best
    det = grading.route_sets(other, r['expert_ids'], inp['x'], inp['router'], inp['router_bias'], 4)
    assert det['differing'] == 1 and not det['ok']                   # gap is far above the tie threshold


def test_golden_tiny_case_regression():
    data = np.load(os.path.join(GOLDEN, 'tiny_moe_seed0.npz'))
    cfg, inp = tiny_inputs(0)
    for key in ('x', 'router', 'gate_blocks', 'down_scales'):
        t = inp[key]
        arr = t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()
        assert np.array_equal(arr, data['in_' + key]), key
    args = tuple(inp[k] for k in ('x', 'router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks',
                                  'up_scales', 'down_blocks', 'down_scales'))
    bf = moe_ref.moe_step(*args, topk=cfg.topk)
    fp = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True)
    assert np.array_equal(bf['expert_ids'].numpy(), data['expert_ids'])
    assert np.allclose(bf['route_weights'].numpy(), data['route_weights'], rtol=1e-6, atol=0)
    assert moe_ref.rel_l2(bf['expert_sum'], torch.from_numpy(data['expert_sum_bf16'])) < 1e-6
    assert moe_ref.rel_l2(fp['expert_sum'], torch.from_numpy(data['expert_sum_fp32'])) < 1e-6


# ----------------------------------------------------------- latent block --

def latent_case(seed=0, B=3, h=64, lh=32, S=16, E=8, k=2, I=64):
    from k3moe import synthetic
    from k3moe.configs import MoEConfig
    cfg = MoEConfig('tiny-latent', E, k, h, I, B, latent=lh)
    return cfg, synthetic.latent_block_inputs(cfg, seed, shared=S)


@pytest.mark.parametrize('seed', [0, 1])
def test_latent_in_matches_float64_brute_force(seed):
    from oracle import latent_ref
    _, w = latent_case(seed)
    args = (w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    lat64, sh64 = latent_ref.latent_in_f64(*args)
    lat, sh = latent_ref.latent_in(*args, fp32=True)
    assert lat.dtype == sh.dtype == torch.float32
    assert moe_ref.rel_l2(lat, lat64) < 2e-6 and moe_ref.rel_l2(sh, sh64) < 2e-6
    lat, sh = latent_ref.latent_in(*args)
    assert lat.dtype == sh.dtype == torch.bfloat16
    for got, want in ((lat, lat64), (sh, sh64)):
        assert 1e-4 < moe_ref.rel_l2(got, want) < 2e-2


@pytest.mark.parametrize('seed', [0, 1])
def test_latent_out_matches_float64_brute_force(seed):
    from oracle import latent_ref
    from k3moe import synthetic
    _, w = latent_case(seed)
    es = synthetic.randn(seed, 'expert_sum', (3, 32), 0.3, dtype=torch.float32)
    sh = synthetic.randn(seed, 'shared_h', (3, 16), 0.5, dtype=torch.float32)
    want = latent_ref.latent_out_f64(es, w['latent_norm'], w['latent_up'], sh, w['shared_down'])
    got = latent_ref.latent_out(es, w['latent_norm'], w['latent_up'], sh, w['shared_down'], fp32=True)
    assert got.dtype == torch.float32 and moe_ref.rel_l2(got, want) < 2e-6
    got = latent_ref.latent_out(es, w['latent_norm'], w['latent_up'], sh.bfloat16(), w['shared_down'])
    assert got.dtype == torch.bfloat16 and 1e-4 < moe_ref.rel_l2(got, want) < 2e-2


def test_latent_rms_epsilon_closed_form():
    """A constant row c has RMS |c|: the normalized value is c/sqrt(c^2 + 1e-5) (kimi.py:325)."""
    from oracle import latent_ref
    for c in (1e-3, 3e-3, 0.5):
        x = torch.full((2, 64), c)
        got = latent_ref.rms(x, torch.ones(64), latent_ref.RMS_EPS)
        assert torch.allclose(got, torch.full_like(got, c/(c*c + 1e-5)**0.5), rtol=1e-6, atol=0)
    # at c = 1e-3 the epsilon dominates: 0.3015 rather than 1
    assert abs(float(latent_ref.rms(torch.full((1, 8), 1e-3), torch.ones(8), latent_ref.RMS_EPS)[0, 0]) - 0.30151) < 1e-4


def test_latent_planted_mistakes_fail_brute_force(monkeypatch):
    from oracle import latent_ref
    from k3moe import synthetic
    _, w = latent_case(0)
    lat64, sh64 = latent_ref.latent_in_f64(w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    _, bad = latent_ref.latent_in(w['x'], w['latent_down'], w['shared_up'], w['shared_gate'], fp32=True)
    assert moe_ref.rel_l2(bad, sh64) > 0.05             # gate and up swapped
    es = synthetic.randn(0, 'expert_sum', (3, 32), 0.3, dtype=torch.float32)
    sh = torch.from_numpy(sh64).float()
    want = latent_ref.latent_out_f64(es, w['latent_norm'], w['latent_up'], sh, w['shared_down'])
    rms = latent_ref.rms
    plants = {
        'norm weight dropped': lambda x, weight, eps: rms(x, torch.ones_like(weight), eps),
        'mean over tokens': lambda x, weight, eps: (x.float()*torch.rsqrt(x.float().square().mean(0, keepdim=True)
                                                                         + eps)).to(x.dtype)*weight.to(x.dtype),
    }
    for name, fn in plants.items():
        monkeypatch.setattr(latent_ref, 'rms', fn)
        got = latent_ref.latent_out(es, w['latent_norm'], w['latent_up'], sh, w['shared_down'], fp32=True)
        assert moe_ref.rel_l2(got, want) > 0.02, name
    monkeypatch.setattr(latent_ref, 'rms', rms)


@pytest.mark.parametrize('seed', [0, 2])
def test_latent_block_chains_float64_pieces(seed):
    """The whole block in FP32 against latent_in_f64 -> moe_step_f64 on the latent -> latent_out_f64."""
    from oracle import latent_ref
    cfg, w = latent_case(seed)
    before = {k: v.clone() for k, v in w.items() if v is not None}
    r = latent_ref.latent_block(w['x'], w, topk=cfg.topk, fp32=True)
    assert all(torch.equal(before[k], w[k]) for k in before)
    lat64, sh64 = latent_ref.latent_in_f64(w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    es64 = moe_ref.moe_step_f64(w['x'], w['router'], w['router_bias'], w['gate_blocks'], w['gate_scales'],
                                w['up_blocks'], w['up_scales'], w['down_blocks'], w['down_scales'],
                                routes=r['expert_ids'], weights=r['route_weights'], latent=torch.from_numpy(lat64))
    out64 = latent_ref.latent_out_f64(torch.from_numpy(es64), w['latent_norm'], w['latent_up'],
                                      torch.from_numpy(sh64), w['shared_down'])
    assert moe_ref.rel_l2(r['output'], out64) < 1e-5
    bf = latent_ref.latent_block(w['x'], w, topk=cfg.topk, routes=r['expert_ids'])
    assert bf['output'].dtype == torch.bfloat16 and 1e-4 < moe_ref.rel_l2(bf['output'], out64) < 3e-2


@pytest.mark.parametrize('seed', [0, 1, 2])
@pytest.mark.parametrize('B,h,lh,S', [(3, 64, 32, 16), (5, 256, 128, 64)])
def test_latent_bf16_matches_bf16_float64_brute_force(seed, B, h, lh, S):
    """latent_in / latent_out in BF16 mode against float64 brute forces rounded at the chain's casts."""
    from oracle import latent_ref
    from k3moe import synthetic
    _, w = latent_case(seed, B=B, h=h, lh=lh, S=S)
    args = (w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    lat64, sh64 = latent_ref.latent_in_bf16_f64(*args)
    lat, sh = latent_ref.latent_in(*args)
    assert moe_ref.rel_l2(lat, lat64) <= 1e-5 and moe_ref.rel_l2(sh, sh64) <= 1e-5
    es = synthetic.randn(seed, 'expert_sum', (B, lh), 0.3, dtype=torch.float32)
    shb = synthetic.randn(seed, 'shared_h', (B, S), 0.5)
    want = latent_ref.latent_out_bf16_f64(es, w['latent_norm'], w['latent_up'], shb, w['shared_down'])
    got = latent_ref.latent_out(es, w['latent_norm'], w['latent_up'], shb, w['shared_down'])
    assert got.dtype == torch.bfloat16 and moe_ref.rel_l2(got, want) <= 1e-5


def test_latent_bf16_planted_mistakes_fail(monkeypatch):
    """Dropped or moved casts of the BF16 latent chain move it well away from the brute force."""
    from oracle import latent_ref
    from k3moe import synthetic
    _, w = latent_case(1, B=5, h=256, lh=128, S=64)
    args = (w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    lat64, sh64 = latent_ref.latent_in_bf16_f64(*args)
    es = synthetic.randn(1, 'expert_sum', (5, 128), 0.3, dtype=torch.float32)
    shb = synthetic.randn(1, 'shared_h', (5, 64), 0.5)
    want = latent_ref.latent_out_bf16_f64(es, w['latent_norm'], w['latent_up'], shb, w['shared_down'])
    out_args = (es, w['latent_norm'], w['latent_up'], shb, w['shared_down'])
    project, rms = latent_ref.project, latent_ref.rms
    # projections accumulate without rounding to bf16
    monkeypatch.setattr(latent_ref, 'project', lambda W, x, act: x.to(act).float() @ W.to(act).float().T)
    bl, bs = latent_ref.latent_in(*args)
    assert moe_ref.rel_l2(bl.float(), lat64) >= 5e-4 and moe_ref.rel_l2(bs.float(), sh64) >= 5e-4
    assert moe_ref.rel_l2(latent_ref.latent_out(*out_args).float(), want) >= 5e-4
    monkeypatch.setattr(latent_ref, 'project', project)
    plants = {
        # the norm weight applied in FP32 before the cast (the common.py weight_in_fp32 variant)
        'weight in fp32': lambda x, wt, eps: (x.float()*torch.rsqrt(x.float().square().mean(-1, keepdim=True) + eps)
                                              * wt.float()).to(x.dtype),
        # the expert sum normalised without its bf16 cast
        'sum not cast': lambda x, wt, eps: rms(es, wt, eps).to(x.dtype),
    }
    for name, fn in plants.items():
        monkeypatch.setattr(latent_ref, 'rms', fn)
        assert moe_ref.rel_l2(latent_ref.latent_out(*out_args), want) >= 5e-4, name
    monkeypatch.setattr(latent_ref, 'rms', rms)


@pytest.mark.parametrize('seed', [0, 2])
def test_latent_block_bf16_chains_bf16_pieces(seed):
    """The whole BF16 block against latent_in_bf16_f64 -> moe_step_bf16_f64 -> latent_out_bf16_f64."""
    from oracle import latent_ref
    cfg, w = latent_case(seed)
    r = latent_ref.latent_block(w['x'], w, topk=cfg.topk)
    lat64, sh64 = latent_ref.latent_in_bf16_f64(w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    es64 = moe_ref.moe_step_bf16_f64(w['x'], w['router'], w['router_bias'], w['gate_blocks'], w['gate_scales'],
                                     w['up_blocks'], w['up_scales'], w['down_blocks'], w['down_scales'],
                                     routes=r['expert_ids'], weights=r['route_weights'],
                                     latent=torch.from_numpy(lat64))
    out64 = latent_ref.latent_out_bf16_f64(torch.from_numpy(es64), w['latent_norm'], w['latent_up'],
                                           torch.from_numpy(sh64), w['shared_down'])
    assert moe_ref.rel_l2(r['output'], out64) <= 1e-5
