"""GPU parity of the latent MoE block (kimi.py:317, 325-328) against the CPU restatement (run with -m gpu).

Bar: every float output within the oracle band rel-L2(gpu, truth) <= 2 rel-L2(bf16
oracle, truth) + 0.002 (truth = the FP32 mode on the same inputs), elementwise next
to the BF16 oracle (same rounding points: at most a rounding step apart), expert sets
exact (or certified FP64 near-ties) in the whole block, no input mutated, repeated
launches on one workspace bitwise identical. Each test prints its case first.
"""

import pytest
import torch

import k3moe
from k3moe import configs, synthetic
from k3moe.configs import MoEConfig
from oracle import grading, latent_ref, moe_ref

pytestmark = pytest.mark.gpu

# (B, h, lh, S): the Kimi K3 TP8 rank (h 7168, latent 3584, shared 768 = 3072 x 2 / 8) at the
# reference's batches, and small or ragged shapes (token tiles, splits and row tiles partly filled)
SHAPES = [(1, 7168, 3584, 768), (8, 7168, 3584, 768), (64, 7168, 3584, 768), (3, 256, 128, 128),
          (17, 512, 256, 128), (33, 1024, 512, 256), (40, 2048, 1024, 384), (1, 128, 128, 128),
          (100, 1024, 512, 256), (130, 512, 256, 128),   # more than 64 tokens: launches of 64 rows
          (40, 5120, 2560, 384)]  # latent_out streamed with cut row tiles (320 tiles of 23 steps, 256 runs)


def say(*a):
    print(*a, flush=True)


def block_weights(B, h, lh, S, seed):
    r = lambda name, shape, scale, **kw: synthetic.randn(seed, name, shape, scale, **kw)
    return {'x': r('x', (B, h), 1.0), 'latent_down': r('latent_down', (lh, h), h**-0.5),
            'shared_gate': r('shared_gate', (S, h), h**-0.5), 'shared_up': r('shared_up', (S, h), h**-0.5),
            'latent_up': r('latent_up', (h, lh), lh**-0.5), 'shared_down': r('shared_down', (h, S), S**-0.5),
            'latent_norm': r('latent_norm', (lh,), 0.1, shift=1.0),
            'expert_sum': r('expert_sum', (B, lh), 0.5, dtype=torch.float32)}


def near_oracle(got, oracle, steps=1, floor=2e-4):
    """bf16 values at most `steps` rounding steps (2^-7 relative) from the BF16 oracle, mostly equal.

    The absolute term (floor x the oracle's RMS) covers values that cancel to
    near zero, where the FP32 sums' different orders, or the roundings of
    addends, differ by more than the value's own rounding step.
    """
    g, o = got.float().cpu(), oracle.float()
    tol = o.abs()*(steps*2.0**-7) + floor*o.pow(2).mean().sqrt()
    bad = (g - o).abs() > tol
    if bool(bad.any()):
        i = int(((g - o).abs() - tol).flatten().argmax())
        raise AssertionError(f'{int(bad.sum())} values further than {steps} rounding steps from the oracle; '
                             f'worst at {i}: {float(g.flatten()[i])} vs {float(o.flatten()[i])}')
    same = float((g == o).float().mean())
    assert same >= 0.9, same


@pytest.mark.parametrize('B,h,lh,S', SHAPES)
def test_latent_in_matches_oracle(B, h, lh, S):
    say(f'latent_in B={B} h={h} lh={lh} S={S}')
    dev = torch.device('cuda:0')
    w = block_weights(B, h, lh, S, seed=B + h)
    g = {k: v.to(dev) for k, v in w.items()}
    before = grading.snapshot(g)
    lat, sh = k3moe.latent_in(g['x'], g['latent_down'], g['shared_gate'], g['shared_up'])
    torch.cuda.synchronize(dev)
    grading.check_unchanged(g, before)
    args = (w['x'], w['latent_down'], w['shared_gate'], w['shared_up'])
    o_lat, o_sh = latent_ref.latent_in(*args)
    t_lat, t_sh = latent_ref.latent_in(*args, fp32=True)
    # shared_h = bf16(act(bf16(g), bf16(u))): a flipped rounding of g or u moves the
    # activation by about one step before its own rounding
    for name, got, o, t, steps in (('latent', lat, o_lat, t_lat, 1), ('shared_h', sh, o_sh, t_sh, 2)):
        assert got.dtype == torch.bfloat16
        detail = grading.band_check(got.cpu(), o, t, t, name=name)
        say(f'  {name}: {detail}')
        near_oracle(got, o, steps)


@pytest.mark.parametrize('B,h,lh,S', SHAPES)
def test_latent_out_matches_oracle(B, h, lh, S):
    say(f'latent_out B={B} h={h} lh={lh} S={S}')
    dev = torch.device('cuda:0')
    w = block_weights(B, h, lh, S, seed=B + 2*h)
    w['shared_h'] = synthetic.randn(B + 2*h, 'shared_h', (B, S), 0.5)
    keys = ('expert_sum', 'latent_norm', 'latent_up', 'shared_h', 'shared_down')
    g = {k: w[k].to(dev) for k in keys}
    before = grading.snapshot(g)
    out = k3moe.latent_out(*(g[k] for k in keys))
    torch.cuda.synchronize(dev)
    grading.check_unchanged(g, before)
    o = latent_ref.latent_out(*(w[k] for k in keys))
    t = latent_ref.latent_out(*(w[k] for k in keys), fp32=True)
    assert out.dtype == torch.bfloat16
    detail = grading.band_check(out.cpu(), o, t, t, name='output')
    say(f'  output: {detail}')
    # the normalised row is rounded twice before the product, and the output is the
    # rounded sum of two rounded addends (routed + shared): a flipped rounding there
    # moves an output by a step of the addends, not of the (possibly cancelled) sum
    near_oracle(out, o, steps=2, floor=2.0**-7)


def test_latent_rms_small_expert_sum_uses_epsilon():
    """An expert sum near 1e-3 makes eps = 1e-5 dominate the RMS (kimi.py:325)."""
    B, h, lh, S = 2, 256, 128, 128
    say(f'latent_out tiny expert_sum B={B} h={h} lh={lh} S={S}')
    dev = torch.device('cuda:0')
    w = block_weights(B, h, lh, S, seed=5)
    w['expert_sum'] = w['expert_sum']*2e-3
    w['shared_h'] = torch.zeros(B, S, dtype=torch.bfloat16)
    keys = ('expert_sum', 'latent_norm', 'latent_up', 'shared_h', 'shared_down')
    out = k3moe.latent_out(*(w[k].to(dev) for k in keys)).cpu()
    o = latent_ref.latent_out(*(w[k] for k in keys))
    no_eps = latent_ref.latent_out(w['expert_sum']*1e3, *(w[k] for k in keys[1:]))
    assert moe_ref.rel_l2(out, o) < 0.01
    # without the epsilon the rows would be scale-free: visibly larger
    assert float(out.float().abs().mean()) < 0.7*float(no_eps.float().abs().mean())


def test_latent_repeated_launches_are_identical():
    B, h, lh, S = 8, 7168, 3584, 768
    say(f'latent repeat B={B} h={h} lh={lh} S={S}')
    dev = torch.device('cuda:0')
    w = {k: v.to(dev) for k, v in block_weights(B, h, lh, S, seed=3).items()}
    w['shared_h'] = synthetic.randn(3, 'shared_h', (B, S), 0.5, device=dev)
    ws = k3moe.new_workspace(32 << 20, dev)
    first = None
    for _ in range(4):
        lat, sh = k3moe.latent_in(w['x'], w['latent_down'], w['shared_gate'], w['shared_up'], workspace=ws)
        out = k3moe.latent_out(w['expert_sum'], w['latent_norm'], w['latent_up'], w['shared_h'], w['shared_down'],
                               workspace=ws)
        got = (lat.clone(), sh.clone(), out.clone())
        if first is None:
            first = got
        else:
            assert all(torch.equal(a, b) for a, b in zip(first, got))
    torch.cuda.synchronize(dev)
    assert k3moe.workspace_status(ws) == 0
    # each workgroup group's counter (64 bytes apart) grew by 1024 per launch: whole launches only
    cnt = ws[4096 + 65536:4096 + 65536 + 16384].view(torch.int32).view(-1, 16).cpu()
    assert int(cnt[:, 1:].abs().sum()) == 0
    used = cnt[:, 0][cnt[:, 0] != 0]
    assert used.numel() > 0 and bool((used == 8*1024).all()), used.unique()


def test_latent_out_streamed_counters_return_to_zero():
    """The streamed latent_in and latent_out (64 tokens, full grid): repeated launches agree bit for
    bit and leave every (row tile, token tile) counter at zero for the next launch."""
    B, h, lh, S = 64, 7168, 3584, 768
    say(f'latent_out streamed repeat B={B} h={h} lh={lh} S={S}')
    dev = torch.device('cuda:0')
    w = {k: v.to(dev) for k, v in block_weights(B, h, lh, S, seed=9).items()}
    w['shared_h'] = synthetic.randn(9, 'shared_h', (B, S), 0.5, device=dev)
    ws = k3moe.new_workspace(64 << 20, dev)
    outs = [k3moe.latent_out(w['expert_sum'], w['latent_norm'], w['latent_up'], w['shared_h'], w['shared_down'],
                             workspace=ws).clone() for _ in range(3)]
    ins = [torch.cat([t.flatten() for t in k3moe.latent_in(w['x'], w['latent_down'], w['shared_gate'],
                                                           w['shared_up'], workspace=ws)]) for _ in range(3)]
    torch.cuda.synchronize(dev)
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    assert all(torch.equal(ins[0], o) for o in ins[1:])
    assert k3moe.workspace_status(ws) == 0
    # the streamed kernels' counters: words 2048 .. 4095 of the latent counter area
    cnt = ws[4096 + 65536 + 2048 * 4:4096 + 65536 + 16384].view(torch.int32).cpu()
    assert int(cnt.abs().sum()) == 0


def block_case(cfg, seed, shared, shared_fan=None):
    return synthetic.latent_block_inputs(cfg, seed, shared=shared, shared_fan=shared_fan)


@pytest.mark.parametrize('cfg,shared,seed', [
    (MoEConfig('latent-small', 64, 8, 1024, 256, 5, latent=512), 256, 0),
    (MoEConfig('latent-b80', 64, 8, 1024, 256, 80, latent=512), 256, 3),   # general MoE path, two latent launches
    (MoEConfig('kimi-rank-e128-b8', 128, 16, 7168, 384, 8, latent=3584), 768, 1),
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768, 2),
])
def test_latent_block_matches_oracle(cfg, shared, seed):
    """latent_in -> moe_step on the latent -> latent_out against the restatement of kimi.py:317-328."""
    run_block(cfg, shared, seed)


def test_latent_block_kimi_rank_geometry():
    """The full Kimi K3 TP8 rank: 896 experts, top-16, I=384, latent 3584, shared 768, B=8."""
    run_block(configs.KIMI_K3_TP8, 768, 0, shared_fan=6144)


def test_latent_block_forced_routes():
    """Forced expert sets (kimi.py:311-313) through the whole block."""
    cfg = MoEConfig('latent-routes', 48, 6, 512, 128, 7, latent=256)
    w = block_case(cfg, 4, 128)
    g = torch.Generator().manual_seed(11)
    routes = torch.stack([torch.randperm(cfg.experts, generator=g)[:cfg.topk] for _ in range(cfg.tokens)])
    run_block(cfg, 128, 4, routes=routes, w=w)


def run_block(cfg, shared, seed, shared_fan=None, routes=None, w=None):
    say(f'latent_block {cfg.name} shared={shared} seed={seed} routes={routes is not None}')
    dev = torch.device('cuda:0')
    w = w if w is not None else block_case(cfg, seed, shared, shared_fan)
    g = {k: (v.to(dev) if v is not None else None) for k, v in w.items()}
    before = grading.snapshot({k: v for k, v in g.items() if v is not None})
    got = k3moe.latent_block(g['x'], g, topk=cfg.topk, routes=None if routes is None else routes.to(dev))
    torch.cuda.synchronize(dev)
    grading.check_unchanged({k: v for k, v in g.items() if v is not None}, before)
    got = {k: v.cpu() for k, v in got.items()}
    oracle = latent_ref.latent_block(w['x'], w, topk=cfg.topk, routes=routes)
    if routes is not None:
        assert torch.equal(got['expert_ids'], routes.sort(-1).values)
        assert torch.allclose(got['route_shortfall'], oracle['route_shortfall'], rtol=1e-5, atol=1e-6)
        sets = {'ok': True, 'exact': True}
    else:
        sets = grading.route_sets(got['expert_ids'], oracle['expert_ids'], w['x'], w['router'], w['router_bias'],
                                  cfg.topk)
    assert sets['ok'], sets
    truth_o = latent_ref.latent_block(w['x'], w, topk=cfg.topk, fp32=True, routes=oracle['expert_ids'])
    truth_c = truth_o if sets['exact'] else latent_ref.latent_block(w['x'], w, topk=cfg.topk, fp32=True,
                                                                    routes=got['expert_ids'])
    for name in ('latent', 'shared_h', 'expert_sum', 'output'):
        detail = grading.band_check(got[name], oracle[name], truth_o[name], truth_c[name], name=name)
        say(f'  {name}: {detail}')


@pytest.mark.parametrize('cfg,shared,forced', [
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768, False),   # one launch
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768, True),
    (MoEConfig('latent-one', 64, 8, 1024, 256, 1, latent=512), 256, False),             # one launch, small
    (MoEConfig('latent-wide-shared', 64, 8, 1024, 256, 1, latent=512), 6400, False),    # 52 rows: two launches
    (MoEConfig('latent-b3', 64, 8, 1024, 256, 3, latent=512), 256, False),              # decode kernel
    (MoEConfig('kimi-rank-e128-b8', 128, 16, 7168, 384, 8, latent=3584), 768, False),   # decode kernel
    (MoEConfig('kimi-rank-e128-b8', 128, 16, 7168, 384, 8, latent=3584), 768, True),
    (MoEConfig('latent-b40', 64, 8, 1024, 256, 40, latent=512), 256, False),            # two launches
])
def test_latent_moe_step_matches_separate_launches(cfg, shared, forced):
    """k3moe.latent_moe_step (one launch of the single-token or decode kernel where they take the
    projections, else latent_in then moe_step) against latent_in and moe_step called separately:
    the same expert sets, latent and
    shared_h within a rounding step (mostly equal: the one-launch sums run in another order), the
    expert sums within the step's band of the oracle."""
    say(f'latent_moe_step {cfg.name} shared={shared} forced={forced}')
    dev = torch.device('cuda:0')
    w = block_case(cfg, 5, shared)
    g = {k: (v.to(dev) if v is not None else None) for k, v in w.items()}
    routes = None
    if forced:
        gen = torch.Generator().manual_seed(3)
        routes = torch.stack([torch.randperm(cfg.experts, generator=gen)[:cfg.topk] for _ in range(cfg.tokens)])
    r_dev = None if routes is None else routes.to(dev)
    before = grading.snapshot({k: v for k, v in g.items() if v is not None})
    lat, sh, moe = k3moe.latent_moe_step(g['x'], g, topk=cfg.topk, routes=r_dev)
    lat2, sh2 = k3moe.latent_in(g['x'], g['latent_down'], g['shared_gate'], g['shared_up'])
    moe2 = k3moe.moe_step(g['x'], g['router'], g['router_bias'], g['gate_blocks'], g['gate_scales'], g['up_blocks'],
                          g['up_scales'], g['down_blocks'], g['down_scales'], topk=cfg.topk, latent=lat2, routes=r_dev)
    torch.cuda.synchronize(dev)
    grading.check_unchanged({k: v for k, v in g.items() if v is not None}, before)
    assert torch.equal(moe['expert_ids'].cpu(), moe2['expert_ids'].cpu())
    assert torch.equal(moe['route_weights'].cpu(), moe2['route_weights'].cpu())
    if forced:
        assert torch.equal(moe['route_shortfall'].cpu(), moe2['route_shortfall'].cpu())
    near_oracle(lat, lat2.cpu(), 1)
    near_oracle(sh, sh2.cpu(), 2)
    oracle = latent_ref.latent_block(w['x'], w, topk=cfg.topk, routes=routes)
    truth = latent_ref.latent_block(w['x'], w, topk=cfg.topk, fp32=True, routes=oracle['expert_ids'])
    for name, got in (('latent', lat), ('shared_h', sh), ('expert_sum', moe['expert_sum'])):
        detail = grading.band_check(got.cpu(), oracle[name], truth[name], truth[name], name=name)
        say(f'  {name}: {detail}')
    ws = k3moe.moe.get_workspace(k3moe.moe.dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'],
                                                    cfg.topk, 'sigmoid_bias', 'situ', lat), dev)
    assert k3moe.workspace_status(ws) == 0


@pytest.mark.parametrize('cfg,shared,forced', [
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768, False),   # one launch
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768, True),
    (MoEConfig('latent-one', 64, 8, 1024, 256, 1, latent=512), 256, False),             # one launch, small
    (MoEConfig('kimi-rank-e128-b8', 128, 16, 7168, 384, 8, latent=3584), 768, False),   # decode kernel
    (MoEConfig('latent-b3', 64, 8, 1024, 256, 3, latent=512), 256, True),
    (MoEConfig('latent-b6', 64, 8, 1024, 256, 6, latent=512), 256, False),
    (MoEConfig('latent-e8-b4', 8, 2, 1024, 256, 4, latent=512), 256, False),            # few active experts
    (MoEConfig('latent-b40', 64, 8, 1024, 256, 40, latent=512), 256, False),            # three launches
])
def test_latent_block_one_call_matches_separate_calls(cfg, shared, forced):
    """k3moe.latent_block (k3moe_latent_block: one launch for one token on the single-token
    kernel, the decode kernel with the projections and the output at 8 tokens) against
    latent_moe_step and latent_out called apart on the same workspace: the same expert sets and
    weights, the output within a rounding step of theirs (mostly equal: its rows are summed in
    another FP32 order) and in the oracle's band."""
    say(f'latent_block one call {cfg.name} shared={shared} forced={forced}')
    dev = torch.device('cuda:0')
    w = block_case(cfg, 6, shared)
    g = {k: (v.to(dev) if v is not None else None) for k, v in w.items()}
    routes = None
    if forced:
        gen = torch.Generator().manual_seed(4)
        routes = torch.stack([torch.randperm(cfg.experts, generator=gen)[:cfg.topk] for _ in range(cfg.tokens)])
    r_dev = None if routes is None else routes.to(dev)
    before = grading.snapshot({k: v for k, v in g.items() if v is not None})
    got = k3moe.latent_block(g['x'], g, topk=cfg.topk, routes=r_dev)
    lat, sh, moe = k3moe.latent_moe_step(g['x'], g, topk=cfg.topk, routes=r_dev)
    out2 = k3moe.latent_out(moe['expert_sum'], g['latent_norm'], g['latent_up'], sh, g['shared_down'])
    torch.cuda.synchronize(dev)
    grading.check_unchanged({k: v for k, v in g.items() if v is not None}, before)
    for key in ('expert_ids', 'route_weights', 'latent', 'shared_h', 'expert_sum'):
        ref = {'latent': lat, 'shared_h': sh}.get(key, moe.get(key))
        assert torch.equal(got[key].cpu(), ref.cpu()), key
    # out = bf16(bf16(routed) + bf16(shared)): where the two parts nearly cancel, one part's rounding
    # step (another summation order moves a part by one) is many of the result's own steps, so the
    # absolute floor is a part's step at a few times the output's RMS
    near_oracle(got['output'], out2.cpu(), 1, floor=0.03)
    oracle = latent_ref.latent_block(w['x'], w, topk=cfg.topk, routes=routes)
    truth = latent_ref.latent_block(w['x'], w, topk=cfg.topk, fp32=True, routes=oracle['expert_ids'])
    detail = grading.band_check(got['output'].cpu(), oracle['output'], truth['output'], truth['output'],
                                name='output')
    say(f'  output: {detail}')
    ws = k3moe.moe.get_workspace(k3moe.moe.dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'],
                                                    cfg.topk, 'sigmoid_bias', 'situ', got['latent']), dev)
    assert k3moe.workspace_status(ws) == 0


@pytest.mark.parametrize('cfg,shared', [
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768),   # single-token kernel
    (MoEConfig('kimi-rank-e128-b8', 128, 16, 7168, 384, 8, latent=3584), 768),   # decode kernel
], ids=['b1-single', 'b8-decode'])
def test_latent_block_across_the_tag_wrap(cfg, shared):
    """The one-launch latent block across the launch tag's wrap-around point: the launch counters
    preset as after 2**32 / G - 3 launches and the tag area holding slots with the first tag after
    the wrap (zero payloads), every call equals the first call on a fresh workspace. The cycle's
    last launch clears the tag area (at 8 tokens, after the workgroups that only arrived at the
    down phase's last barrier have waited for it)."""
    say(f'latent_block across the tag wrap {cfg.name} shared={shared}')
    dev = torch.device('cuda:0')
    w = block_case(cfg, 8, shared)
    g = {k: (v.to(dev) if v is not None else None) for k, v in w.items()}
    key = (dev.type, dev.index)
    saved = k3moe.moe._WORKSPACES.get(key)
    try:
        k3moe.moe._WORKSPACES.pop(key, None)      # a fresh workspace for this test alone
        ref = {k: v.clone() for k, v in k3moe.latent_block(g['x'], g, topk=cfg.topk).items()}
        torch.cuda.synchronize(dev)
        ws = k3moe.moe._WORKSPACES[key]
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        G = 1
        while G * 2 <= min(cus, 1024):
            G *= 2
        launches = (1 << 32) // G - 3
        ctl = ws[:4096].view(torch.int32)
        per = [0] * 16                           # launch counter c counts the workgroups b with b % 16 == c
        for b in range(G):
            per[b % 16] += 1
        for c in range(16):
            v = (per[c] * launches) & 0xFFFFFFFF
            ctl[640 + 16 * c] = v - (1 << 32) if v >= 1 << 31 else v
        tags = ws[k3moe.moe.INIT_BYTES - (2 << 20): k3moe.moe.INIT_BYTES].view(torch.int32).view(-1, 2)
        tags[:, 0] = 0
        tags[:, 1] = 1
        torch.cuda.synchronize(dev)
        for step in range(6):
            got = k3moe.latent_block(g['x'], g, topk=cfg.topk)
            torch.cuda.synchronize(dev)
            for k in ('output', 'latent', 'shared_h', 'expert_sum', 'expert_ids', 'route_weights'):
                assert torch.equal(got[k], ref[k]), (step, k)
        assert k3moe.workspace_status(ws) == 0
    finally:
        if saved is not None:
            k3moe.moe._WORKSPACES[key] = saved
        else:
            k3moe.moe._WORKSPACES.pop(key, None)


@pytest.mark.parametrize('cfg,shared', [
    (MoEConfig('kimi-rank-e128-b1', 128, 16, 7168, 384, 1, latent=3584), 768),   # single-token kernel
    (MoEConfig('kimi-rank-e128-b8', 128, 16, 7168, 384, 8, latent=3584), 768),   # decode kernel
], ids=['b1-single', 'b8-decode'])
def test_latent_block_wait_that_gives_up(cfg, shared):
    """The one-launch latent block's failure path, forced from the host (k3moe_debug_stall: the
    router-logit waits give up after 256 polls): every workgroup still ends, the block's output
    and the expert sum are NaN everywhere, the status word has the timeout bit, and after
    k3moe_workspace_init the workspace gives the first call's outputs again."""
    from k3moe import _native
    import ctypes
    say(f'latent_block failure path {cfg.name} shared={shared}')
    dev = torch.device('cuda:0')
    w = block_case(cfg, 10, shared)
    g = {k: (v.to(dev) if v is not None else None) for k, v in w.items()}
    key = (dev.type, dev.index)
    saved = k3moe.moe._WORKSPACES.get(key)
    try:
        k3moe.moe._WORKSPACES.pop(key, None)      # a fresh workspace for this test alone
        ref = {k: v.clone() for k, v in k3moe.latent_block(g['x'], g, topk=cfg.topk).items()}
        torch.cuda.synchronize(dev)
        ws = k3moe.moe._WORKSPACES[key]
        _native.check(_native.load().k3moe_debug_stall(256), 'k3moe_debug_stall')
        try:
            bad = k3moe.latent_block(g['x'], g, topk=cfg.topk)
            torch.cuda.synchronize(dev)
        finally:
            _native.check(_native.load().k3moe_debug_stall(0), 'k3moe_debug_stall')
        assert bool(torch.isnan(bad['output'].float()).all())
        assert bool(torch.isnan(bad['expert_sum']).all())
        assert k3moe.workspace_status(ws) & 1
        _native.check(_native.load().k3moe_workspace_init(
            ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()),
            ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)), 'k3moe_workspace_init')
        assert k3moe.workspace_status(ws) == 0
        for _ in range(2):
            got = k3moe.latent_block(g['x'], g, topk=cfg.topk)
            torch.cuda.synchronize(dev)
            for k in ('output', 'latent', 'shared_h', 'expert_sum', 'expert_ids', 'route_weights'):
                assert torch.equal(got[k], ref[k]), k
        assert k3moe.workspace_status(ws) == 0
    finally:
        if saved is not None:
            k3moe.moe._WORKSPACES[key] = saved
        else:
            k3moe.moe._WORKSPACES.pop(key, None)


def test_latent_moe_layer_reads_reference_keys():
    cfg = MoEConfig('latent-small', 64, 8, 1024, 256, 4, latent=512)
    say(f'latent_moe_layer {cfg.name}')
    dev = torch.device('cuda:0')
    w = synthetic.latent_block_inputs(cfg, 7, shared=256)
    x = w.pop('x')
    values = {f'l3_{k}': (v.to(dev) if v is not None else None) for k, v in w.items()}
    got = k3moe.latent_moe_layer(values, 3, x.to(dev), topk=cfg.topk)
    direct = k3moe.latent_block(x.to(dev), {k: values['l3_' + k] for k in w}, topk=cfg.topk)
    torch.cuda.synchronize(dev)
    for k in ('output', 'expert_ids', 'expert_sum'):
        assert torch.equal(got[k], direct[k]), k
