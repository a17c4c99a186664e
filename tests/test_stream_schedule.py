"""CPU checks of two kernels' load schedules (restated here from their sources).

k_fgemm (csrc/k3moe_fgemm.hpp): units stream back to back; a loader issues the
step two ahead at every barrier (the next unit's first two steps during the
last two of the current one), waits before the barrier of step g until only
the loads of step g + 1 may be outstanding, and puts weight-scale chunk c of a
unit (16 steps each) into buffer (unit's first chunk number + c) & 1. Checked:
the wait counts equal the loads issued after step g, and no chunk buffer is
overwritten while a step still reads its older content.

k_latent_sk (csrc/k3moe_latent.hpp): the (row tile, step) items are cut into G
equal runs; a tile must be whole in one run or cut once, every cut tile's two
segments must carry the parts they store, and the second to count in must sum
both into every step of the tile, each part exactly once.
"""
import pytest


def fgemm_stream(KS, nunits, kloads=11, ktiles=4, steps_per_chunk=16):
    nsc = (KS + steps_per_chunk - 1) // steps_per_chunk
    chunk_at = lambda s: s == 0 or (s >= 2 and (s - 2) % steps_per_chunk == 0
                                    and (s - 2) // steps_per_chunk + 1 < nsc)
    issued = []  # (global step, loads, (buffer, chunk number) or None)

    def issue(ks, g, cb0):
        chunk = None
        if chunk_at(ks):
            c = 0 if ks == 0 else (ks - 2) // steps_per_chunk + 1
            chunk = ((cb0 + c) & 1, cb0 + c)
        issued.append((g, kloads + (ktiles if chunk else 0), chunk))

    reads = {u * KS + ks: (((u * nsc + ks // steps_per_chunk) & 1), u * nsc + ks // steps_per_chunk)
             for u in range(nunits) for ks in range(KS)}
    issue(0, 0, 0)
    issue(1, 1, 0)
    for u in range(nunits):
        g0, cb0, have_next = u * KS, u * nsc, u + 1 < nunits
        for ks in range(KS):
            g = g0 + ks
            if ks + 1 < KS:
                allow = kloads + (ktiles if chunk_at(ks + 1) else 0)
            else:
                allow = kloads + ktiles if have_next else 0
            after = sum(n for gs, n, _ in issued if gs > g)
            assert after == allow, (KS, u, ks, after, allow)
            if ks + 2 < KS:
                issue(ks + 2, g + 2, cb0)
            elif have_next:
                issue(ks + 2 - KS, g + 2, cb0 + nsc)
            else:
                continue
            if issued[-1][2] is not None:
                buf, chunk = issued[-1][2]
                # the MFMA waves may still read step g (and later ones): none of them older content
                assert all(not (reads[gg][0] == buf and reads[gg][1] < chunk) for gg in range(g, nunits * KS))


@pytest.mark.parametrize('KS', [4, 8, 12, 16, 20, 24, 28, 32, 48, 56, 64])
@pytest.mark.parametrize('nunits', [1, 2, 3, 5])
def test_fgemm_stream_schedule(KS, nunits):
    fgemm_stream(KS, nunits)


def sk_order(lo, hi, KS):
    """k_latent_sk's processing order of a run's (tile, step) items: the last
    tile's head when that tile is cut, the first tile's tail when that one is,
    then the whole tiles between; (rt, ks, k0, k1) per item, k0 / k1 the
    tile's first step and end in the run."""
    rt_lo, ks_lo = lo // KS, lo % KS
    rt_hi, ks_end = (hi - 1) // KS, (hi - 1) % KS + 1
    cut_first, cut_last = ks_lo > 0, rt_hi != rt_lo and ks_end < KS
    entries = []
    if cut_last:
        entries.append((rt_hi, rt_hi, 0, ks_end))
    if cut_first:
        entries.append((rt_lo, rt_lo, ks_lo, KS))
    if rt_lo + cut_first <= rt_hi - cut_last:
        entries.append((rt_lo + cut_first, rt_hi - cut_last, 0, KS))
    items = []
    for r0, r1, k0, k1 in entries:
        for rt in range(r0, r1 + 1):
            a = k0 if rt == r0 else 0
            b = k1 if rt == r1 else KS
            items += [(rt, ks, a, b) for ks in range(a, b)]
    return items


def latent_sk_runs(RT, KS, KS0, G, out, second_first=False):
    NI = RT * KS
    has0 = lambda ka: (not out) or ka < KS0
    has1 = lambda kb: out and kb > KS0
    parts, result, count = {}, {}, {}
    counts = []
    for b in range(G):
        lo, hi = NI * b // G, NI * (b + 1) // G
        assert hi - lo >= KS
        items = sk_order(lo, hi, KS)
        assert sorted((rt * KS + ks) for rt, ks, _, _ in items) == list(range(lo, hi))
        acc0, acc1, cuts = set(), set(), []
        for rt, ks, ka, kb in items:
            (acc1 if out and ks >= KS0 else acc0).add((rt, ks))
            if ks + 1 == kb:
                if ka == 0 and kb == KS:
                    result[rt] = (frozenset(acc0), frozenset(acc1))
                else:
                    seg = 0 if ka == 0 else 1
                    if has0(ka):
                        parts[(rt, seg, 0)] = frozenset(acc0)
                    if has1(kb):
                        parts[(rt, seg, 1)] = frozenset(acc1)
                    cuts.append((rt, kb if ka == 0 else ka))
                acc0, acc1 = set(), set()
        assert len(cuts) <= 2  # the kernel keeps two
        counts += cuts
    # the counts arrive in any order; the second of a tile's two sums both
    # segments (after every partial is stored)
    for rt, kc in (reversed(counts) if second_first else counts):
        count[rt] = count.get(rt, 0) + 1
        if count[rt] == 1:
            continue
        s0 = parts[(rt, 0, 0)] | (parts[(rt, 1, 0)] if has0(kc) else frozenset())
        s1 = (parts[(rt, 0, 1)] if has1(kc) else frozenset()) | (parts[(rt, 1, 1)] if has1(KS) else frozenset())
        result[rt] = (s0, s1)
    assert all(c == 2 for c in count.values())
    for rt in range(RT):
        want0 = frozenset((rt, k) for k in range(KS) if (not out) or k < KS0)
        want1 = frozenset((rt, k) for k in range(KS0, KS)) if out else frozenset()
        assert result[rt] == (want0, want1), rt


@pytest.mark.parametrize('RT,KS,KS0,G,out', [
    (448, 34, 28, 256, True),    # latent_out of a Kimi K3 TP8 rank
    (320, 23, 20, 256, True),    # the test geometry with cut tiles
    (320, 56, 56, 256, False),
    (64, 12, 4, 64, True),
    (300, 7, 5, 256, True),
])
def test_latent_sk_segments(RT, KS, KS0, G, out):
    latent_sk_runs(RT, KS, KS0, G, out)
    latent_sk_runs(RT, KS, KS0, G, out, second_first=True)


def test_latent_sk_order_puts_cut_segments_first():
    # run [5, 5 + 20) of 8-step tiles: tile 0 steps 5-7, tile 1, tile 2, tile 3 steps 0-0
    items = sk_order(5, 25, 8)
    assert items[0] == (3, 0, 0, 1)
    assert [it[:2] for it in items[1:4]] == [(0, 5), (0, 6), (0, 7)]
    assert [it[:2] for it in items[4:]] == [(1, k) for k in range(8)] + [(2, k) for k in range(8)]
    assert sk_order(16, 24, 8) == [(2, k, 0, 8) for k in range(8)]
