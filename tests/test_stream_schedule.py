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


def latent_sk_runs(RT, KS, KS0, G, out):
    NI = RT * KS
    has0 = lambda ka: (not out) or ka < KS0
    has1 = lambda kb: out and kb > KS0
    parts, result, count = {}, {}, {}
    order = []
    for b in range(G):
        lo, hi = NI * b // G, NI * (b + 1) // G
        assert hi - lo >= KS
        seg_a, acc0, acc1 = lo % KS, set(), set()
        for s in range(hi - lo):
            it = lo + s
            rt, ks = it // KS, it % KS
            (acc1 if out and ks >= KS0 else acc0).add((rt, ks))
            if ks == KS - 1 or s == hi - lo - 1:
                ka, kb = seg_a, ks + 1
                if ka == 0 and kb == KS:
                    result[rt] = (frozenset(acc0), frozenset(acc1))
                else:
                    seg = 0 if ka == 0 else 1
                    if has0(ka):
                        parts[(rt, seg, 0)] = frozenset(acc0)
                    if has1(kb):
                        parts[(rt, seg, 1)] = frozenset(acc1)
                    order.append((rt, ka, kb))
                acc0, acc1, seg_a = set(), set(), 0
    for rt, ka, kb in order:
        count[rt] = count.get(rt, 0) + 1
        if count[rt] == 1:
            continue
        kc = kb if ka == 0 else ka
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
