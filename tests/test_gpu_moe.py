"""GPU parity of the k3moe step against the CPU oracle (run with -m gpu).

Bar (from the task): expert sets bit-exact (a differing row must be an FP64
certified near-tie), MXFP4 decode bit-exact, expert_sum within the oracle
band rel-L2(gpu, truth_c) <= 2 rel-L2(bf16 oracle, truth_o) + 0.002, no input
mutated. Every test prints the case it runs before touching the GPU.
"""

import numpy as np
import pytest
import torch

import k3moe
from k3moe import configs, synthetic
from k3moe.configs import MoEConfig
from oracle import cdecode, grading, moe_ref

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def to_dev(inputs, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inputs.items()}


def decode_ok(cfg):
    return cfg.tokens <= 64 and cfg.tokens*cfg.topk <= 1024


def near_oracle_sum(got, oracle, steps=2, min_same=0.75):
    """expert_sum element by element next to the BF16 oracle.

    Both sum w * bf16(y) over a token's experts in ascending order in FP32 from
    zero, so an element differs only where the bf16 rounding of some pair
    output y flipped (FP32 sums in another order inside the dot products), or
    by the last bits of a route weight (the GPU's sigmoid and the CPU's differ
    by an ulp). The bound is `steps` rounding steps of each contribution:
    sum_j w_j steps ulp(y_j), plus 1e-6 of the row scale for outputs near
    zero. And the oracle's pair outputs recombined with the GPU's weights in
    that order must equal the GPU's sum bitwise for most elements (every
    element whose pair outputs all have the oracle's rounding; one flipped bf16
    rounding of an activation moves about a sixteenth of its expert's outputs by
    a step, and at one token every output sums every chosen expert); returns
    that fraction. The combine's own arithmetic is checked exactly by
    test_general_grouping_lists_match_oracle.
    """
    g, o = got['expert_sum'].double(), oracle['expert_sum'].double()
    y, w = oracle['pair_out'].double(), oracle['route_weights'].double()
    _, e = torch.frexp(y)
    ulp = torch.where(y != 0, torch.ldexp(torch.ones_like(y), e - 8), torch.zeros_like(y))
    scale = (w[..., None]*y.abs()).sum(1)
    tol = steps*(w[..., None]*ulp).sum(1) + 1e-6*scale.amax(-1, keepdim=True)
    bad = (g - o).abs() > tol
    if bool(bad.any()):
        i = int(((g - o).abs() - tol).flatten().argmax())
        raise AssertionError(f'{int(bad.sum())} expert_sum values further than {steps} rounding steps of their '
                             f'contributions from the oracle; worst at {i}: {float(g.flatten()[i])} vs '
                             f'{float(o.flatten()[i])} (tol {float(tol.flatten()[i])})')
    wg = got['route_weights'].float()
    re = torch.zeros_like(got['expert_sum'])
    for j in range(wg.shape[1]):       # FP32 products and adds, ascending expert order
        re = re + oracle['pair_out'][:, j]*wg[:, j, None]
    same = float((got['expert_sum'] == re).double().mean())
    assert same >= min_same, f'only {same:.3f} of expert_sum bitwise equal to the recombined oracle'
    return same


def run_and_check(cfg, inputs, dev, *, routes=None, rows=None, check_close_to_oracle=True, path='auto', host=None,
                  min_same=0.75):
    """GPU step vs oracle on `inputs` (CPU tensors, or device tensors with `host` their host_view).
    rows: optional subset of token rows for the oracle."""
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    g = to_dev(inputs, dev)
    before = grading.snapshot({k: v for k, v in g.items() if v is not None})
    ws = k3moe.new_workspace(1 << 20, dev) if path != 'auto' else None
    if ws is not None:
        from k3moe.moe import dims_for, workspace_bytes
        need = workspace_bytes(dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk,
                                        cfg.gating, cfg.activation, g.get('latent'), path))
        if need > ws.numel():
            ws = k3moe.new_workspace(need, dev)
    got = k3moe.moe_step(*synthetic.step_args(g), **kw, routes=None if routes is None else routes.to(dev),
                         latent=g.get('latent'), path=path, workspace=ws)
    torch.cuda.synchronize(dev)
    if ws is not None:
        assert k3moe.workspace_status(ws) == 0
    grading.check_unchanged({k: v for k, v in g.items() if v is not None}, before)
    got = {k: v.cpu() for k, v in got.items()}
    return check_outputs(cfg, got, inputs if host is None else host, routes=routes, rows=rows,
                         check_close_to_oracle=check_close_to_oracle, min_same=min_same)


class DeviceExperts:
    """An expert tensor left on the GPU, indexed by expert id on the host: the oracle reads
    only the routed experts, so each one's slice is copied to the CPU on first use."""

    def __init__(self, t):
        self.t, self.cache = t, {}

    def __getitem__(self, e):
        e = int(e)
        if e not in self.cache:
            self.cache[e] = self.t[e].cpu()
        return self.cache[e]


def host_view(g):
    """Oracle inputs for device-resident inputs g: small tensors copied, expert tensors lazy."""
    return {k: (DeviceExperts(v) if k.endswith(('_blocks', '_scales')) else
                v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in g.items()}


def check_outputs(cfg, got, inputs, *, routes=None, rows=None, check_close_to_oracle=True, min_same=0.75):
    """Oracle checks of a step's CPU outputs `got` on host inputs (or a host_view)."""
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    ref_in = dict(inputs)
    if rows is not None:
        ref_in['x'] = inputs['x'][rows]
        if inputs.get('latent') is not None:
            ref_in['latent'] = inputs['latent'][rows]
        got = {k: v[rows] for k, v in got.items()}
        if routes is not None:
            routes = routes[rows]
    args = synthetic.step_args(ref_in)
    lat = ref_in.get('latent')
    oracle = moe_ref.moe_step(*args, **kw, routes=routes, latent=lat, pair_out=True)
    sets = grading.route_sets(got['expert_ids'], oracle['expert_ids'], ref_in['x'], ref_in['router'],
                              ref_in['router_bias'], cfg.topk, cfg.gating)
    assert sets['ok'], f'expert sets differ beyond certified near-ties: {sets}'
    assert grading.valid_routes(got['expert_ids'], cfg.experts)
    assert torch.equal(got['expert_ids'], got['expert_ids'].sort(-1).values)
    o_routes = oracle['expert_ids'] if routes is None else routes
    truth_o = moe_ref.moe_step(*args, **kw, fp32=True, routes=o_routes, latent=lat)
    truth_c = truth_o if (sets['exact'] or routes is not None) else moe_ref.moe_step(
        *args, **kw, fp32=True, routes=got['expert_ids'], latent=lat)
    detail = grading.band_check(got['expert_sum'], oracle['expert_sum'], truth_o['expert_sum'],
                                truth_c['expert_sum'])
    if sets['exact']:
        w_err = (got['route_weights'] - oracle['route_weights']).abs().max().item()
        assert w_err <= 4e-7, w_err
    if check_close_to_oracle and sets['exact']:
        # same rounding points and combine order as the BF16 oracle: next to it element by element
        detail['bitwise_same'] = round(near_oracle_sum(got, oracle, min_same=min_same), 4)
    if routes is not None:
        assert torch.allclose(got['route_shortfall'], oracle['route_shortfall'], rtol=0, atol=1e-6)
    say('   ', cfg.name, 'sets', {k: sets[k] for k in ('rows', 'differing', 'certified')}, 'band', detail)
    return got, oracle


# ----------------------------------------------------------------- decode --

def test_decode_exhaustive_bit_exact(gpu):
    say('case: mxfp4_decode all 256 bytes x 256 scales, f32 and bf16')
    blocks = np.tile(np.arange(256, dtype=np.uint8).reshape(1, 16, 16), (256, 1, 1))
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    want = cdecode.mxfp4_decode_bits(blocks, scales)
    b, s = torch.from_numpy(blocks).to(gpu), torch.from_numpy(scales).to(gpu)
    f32 = k3moe.mxfp4_decode(b, s, torch.float32).cpu().numpy().view(np.uint32)
    assert np.array_equal(f32, want)
    bf = k3moe.mxfp4_decode(b, s, torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf.astype(np.uint32), want >> 16)
    # the bf16 values equal torch's own cast of the oracle's fp32 decode (kimi.py:321); the NaN
    # payload of that cast is platform-defined (torch-CPU gives 0xFFFF), so NaN compares as a class
    t = moe_ref.unpack_mxfp4(torch.from_numpy(blocks), torch.from_numpy(scales)).to(torch.bfloat16)
    tb = t.view(torch.int16).numpy().view(np.uint16)
    nan_t, nan_g = (tb & 0x7FFF) > 0x7F80, (bf & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_t, nan_g) and int(nan_g.sum()) == 16*32   # scale row 255
    assert np.array_equal(tb[~nan_t], bf[~nan_g])


def test_decode_random_layout(gpu):
    say('case: mxfp4_decode random [3, 40, 7, 16]')
    blk, scl = synthetic.mxfp4(4, 'dec', (3, 40), 7*32, device='cpu')
    got = k3moe.mxfp4_decode(blk.to(gpu), scl.to(gpu)).cpu()
    assert got.shape == (3, 40, 224)
    assert torch.equal(got.view(torch.int32), moe_ref.unpack_mxfp4(blk, scl).view(torch.int32))


# ------------------------------------------------------------- MoE parity --

TINY = [
    MoEConfig('tiny', 8, 2, 64, 64, 3),
    MoEConfig('tiny-softmax-silu', 8, 2, 64, 64, 3, gating='softmax', activation='silu'),
    MoEConfig('ragged', 40, 5, 160, 96, 19),
    MoEConfig('k1', 16, 1, 128, 64, 33),
    MoEConfig('k32', 48, 32, 96, 32, 5),
    MoEConfig('many-tokens', 24, 4, 256, 128, 70),
    # wide expert sets: the workgroup-cooperative selection (up to 1024 experts, top-32)
    MoEConfig('e1024-k32', 1024, 32, 64, 32, 2),
    MoEConfig('e600-k12', 600, 12, 96, 64, 7),
    MoEConfig('e896-k16', 896, 16, 128, 64, 9),
    # more than 32 active experts with I = 384 and 512: the expert-major down path's 3 and 4 k-steps
    MoEConfig('i384-wide', 96, 8, 128, 384, 7),
    MoEConfig('i512-wide', 64, 8, 128, 512, 9),
    # at most 8 active experts with up to 16 tokens each: the paired row-tile down path;
    # 9 to 12 active experts at small batches: the row-tile path's multi-expert waves
    MoEConfig('e8-b16', 8, 2, 512, 256, 16),
    MoEConfig('e16-k4', 16, 4, 256, 128, 3),
    MoEConfig('e12-k6', 12, 6, 384, 256, 2),
]


@pytest.mark.parametrize('cfg', TINY, ids=lambda c: c.name)
@pytest.mark.parametrize('seed', [0, 1])
@pytest.mark.parametrize('path', ['general', 'decode'])
def test_moe_small_geometries(gpu, cfg, seed, path):
    if path == 'decode' and not decode_ok(cfg):
        pytest.skip('shape is outside the persistent decode path')
    say(f'case: {cfg.name} seed={seed} path={path}')
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, seed, scale_mode='kimi'), gpu, path=path)


# one token on the single-token kernel: top-k <= 16 of <= 1024 experts, K a multiple of 512, I <= 512
SINGLE = [
    MoEConfig('single-e64-k8', 64, 8, 1024, 256, 1),
    MoEConfig('single-e896-k16-i384', 896, 16, 1024, 384, 1, latent=512),   # the Kimi rank's shape, narrower
    MoEConfig('single-e600-k12-i512', 600, 12, 512, 512, 1),
    MoEConfig('single-e1024-k9-i160', 1024, 9, 1536, 160, 1),
    MoEConfig('single-e40-k5-i96', 40, 5, 2048, 96, 1),
    MoEConfig('single-e512-softmax-silu', 512, 8, 1024, 128, 1, gating='softmax', activation='silu'),
    MoEConfig('single-k1', 16, 1, 1024, 64, 1),
    MoEConfig('single-k8192', 32, 4, 8192, 32, 1),
    MoEConfig('single-latent', 64, 8, 512, 256, 1, latent=1024),
]


@pytest.mark.parametrize('cfg', SINGLE, ids=lambda c: c.name)
@pytest.mark.parametrize('seed', [0, 1])
@pytest.mark.parametrize('path', ['single', 'decode'])
def test_moe_single_token_geometries(gpu, cfg, seed, path):
    say(f'case: {cfg.name} seed={seed} path={path}')
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, seed, scale_mode='kimi'), gpu, path=path)


def test_single_token_kimi_rank_geometry(gpu):
    """The reference's own Kimi K3 TP8 rank at one token (E=896, top-16, I=384, latent 3584, h 7168;
    megabench/cases.py:48-55) on the single-token kernel, against the oracle."""
    cfg = configs.KIMI_K3_TP8.with_tokens(1)
    say(f'case: {cfg.name} seed=5 path=single')
    g = synthetic.moe_layer_inputs(cfg, 5, device=gpu)
    run_and_check(cfg, g, gpu, path='single', host=host_view(g))


def test_single_and_decode_kernels_agree_tp8_b1(gpu):
    """The two kernels sum the router logits in different orders (whole rows per workgroup
    against k-splits on MFMA), both within FP32 rounding of the oracle: the same expert ids and
    weights to a few ulps; gate/up sums in another order, so expert_sum agrees to the oracle's
    rounding steps."""
    cfg = configs.TP8_B1
    say(f'case: {cfg.name} seed=11, single-token kernel vs general persistent kernel')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 11), gpu)
    outs = {}
    for path in ('single', 'decode'):
        outs[path] = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path)
        torch.cuda.synchronize(gpu)
    a, b = outs['single'], outs['decode']
    assert torch.equal(a['expert_ids'], b['expert_ids'])
    assert float((a['route_weights'] - b['route_weights']).abs().max()) <= 4e-7
    assert moe_ref.rel_l2(a['expert_sum'].cpu(), b['expert_sum'].cpu()) < 2e-3


def test_single_token_tags_across_launches(gpu):
    """Consecutive single-token launches on one workspace, alternating inputs and interleaved with
    a general persistent step (b8) and a latent-width change: each launch's outputs equal a fresh
    workspace's, so no launch reads another launch's tagged partials or intermediates."""
    from k3moe.moe import dims_for, workspace_bytes
    cfg = configs.TP8_B1
    say(f'case: {cfg.name} seeds 1-2 alternating on one workspace, with b8 and a wider step between')
    ins = [to_dev(synthetic.moe_layer_inputs(cfg, sd), gpu) for sd in (1, 2)]
    wide = MoEConfig('single-e64-k8', 64, 8, 1024, 256, 1)
    g_wide = to_dev(synthetic.moe_layer_inputs(wide, 3), gpu)
    g8 = to_dev(synthetic.moe_layer_inputs(configs.TP8_B8, 4), gpu)
    need = max(workspace_bytes(dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], c.topk, c.gating,
                                        c.activation)) for g, c in ((ins[0], cfg), (g8, configs.TP8_B8)))
    fresh = []
    for g, c in ((ins[0], cfg), (ins[1], cfg), (g_wide, wide), (g8, configs.TP8_B8)):
        fresh.append(k3moe.moe_step(*synthetic.step_args(g), topk=c.topk, workspace=k3moe.new_workspace(need, gpu)))
    ws = k3moe.new_workspace(need, gpu)
    order = [0, 1, 0, 2, 1, 3, 0, 1, 2, 0]
    plan = [(ins[0], cfg), (ins[1], cfg), (g_wide, wide), (g8, configs.TP8_B8)]
    for n, idx in enumerate(order):
        g, c = plan[idx]
        got = k3moe.moe_step(*synthetic.step_args(g), topk=c.topk, workspace=ws)
        torch.cuda.synchronize(gpu)
        for key in ('expert_sum', 'expert_ids', 'route_weights'):
            assert torch.equal(got[key], fresh[idx][key]), (n, idx, key)
    assert k3moe.workspace_status(ws) == 0


@pytest.mark.parametrize('stale', [False, True], ids=['zeroed', 'stale-slots'])
@pytest.mark.parametrize('cfg,path', [(configs.TP8_B1, 'single'), (configs.TP8_B1, 'decode'),
                                      (configs.TP8_B8, 'decode')], ids=['b1-single', 'b1-decode', 'b8-decode'])
def test_tags_from_a_large_launch_count(gpu, cfg, path, stale):
    """The tag of the single-token and decode kernels comes from the launch counters' sum: preset
    them to a large, consistent count (as after 2**32 / G - 3 launches) and run across the tag's
    wrap-around point. With stale slots: the tag area first holds slots carrying tag 1, the first
    tag after the wrap (as left by a launch a whole tag cycle earlier), with zero payloads (in-range
    ids and finite values); the cycle's last launch must clear them, so every step still equals a
    fresh workspace's."""
    from k3moe.moe import dims_for, workspace_bytes
    say(f'case: {cfg.name} seed=5 path={path}, launch counters preset near the 32-bit wrap')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 5), gpu)
    need = workspace_bytes(dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating,
                                    cfg.activation, None, path))
    ref = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=k3moe.new_workspace(need, gpu))
    ws = k3moe.new_workspace(need, gpu)
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    G = 1
    while G * 2 <= min(cus, 1024):
        G *= 2
    launches = (1 << 32) // G - 3
    ctl = ws[:4096].view(torch.int32)
    per = [0] * 16                                   # counter g gets the workgroups b with b % 16 == g
    for b in range(G):
        per[b % 16] += 1
    for gi in range(16):
        v = (per[gi] * launches) & 0xFFFFFFFF
        ctl[640 + 16 * gi] = v - (1 << 32) if v >= 1 << 31 else v
    if stale:   # the tag area is the last 2 MiB of the initialised prefix: 8-byte slots {payload, tag}
        tags = ws[k3moe.moe.INIT_BYTES - (2 << 20): k3moe.moe.INIT_BYTES].view(torch.int32).view(-1, 2)
        tags[:, 0] = 0
        tags[:, 1] = 1
    torch.cuda.synchronize(gpu)
    for step in range(6):
        got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=ws)
        torch.cuda.synchronize(gpu)
        for key in ('expert_sum', 'expert_ids', 'route_weights'):
            assert torch.equal(got[key], ref[key]), (step, key)
    assert k3moe.workspace_status(ws) == 0


def test_single_token_invalid_forced_routes(gpu):
    """Through the C ABI, one token's forced routes with a repeated id: its own top-k, status 2."""
    from k3moe.moe import dims_for, workspace_bytes
    cfg = MoEConfig('single-bad-routes', 64, 8, 1024, 256, 1)
    say(f'case: {cfg.name} seed=13 path=single, a repeated forced id through the C ABI')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 13, scale_mode='kimi'), gpu)
    free = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path='single')
    torch.cuda.synchronize(gpu)
    routes = free['expert_ids'].clone()
    routes[0, 5] = routes[0, 2]
    dims = dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating, cfg.activation,
                    None, 'single')
    ws = k3moe.new_workspace(workspace_bytes(dims), gpu)
    outs = {'expert_sum': torch.full((1, cfg.hidden), float('nan'), device=gpu),
            'expert_ids': torch.full((1, cfg.topk), -1, dtype=torch.int64, device=gpu),
            'route_weights': torch.zeros(1, cfg.topk, device=gpu), 'route_shortfall': torch.full((1,), -1.0, device=gpu)}
    raw_step(dims, g, routes.contiguous(), outs, ws)
    torch.cuda.synchronize(gpu)
    assert k3moe.workspace_status(ws) == 2
    for key in ('expert_sum', 'expert_ids', 'route_weights'):
        assert torch.equal(outs[key], free[key]), key


@pytest.mark.parametrize('seed', [0, 1, 2])
def test_moe_cpu_plumbing(gpu, seed):
    cfg = configs.CPU_PLUMBING
    say(f'case: {cfg.name} seed={seed}')
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, seed), gpu)


@pytest.mark.parametrize('cfg', [configs.TP8_B1, configs.TP8_B8], ids=lambda c: c.name)
@pytest.mark.parametrize('path', ['general', 'decode', 'single'])
def test_moe_tp8_rank(gpu, cfg, path):
    if path == 'single' and cfg.tokens != 1:
        pytest.skip('the single-token kernel takes one token')
    say(f'case: {cfg.name} seed=0 path={path}')
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 0), gpu, path=path)


def test_paths_agree_tp8_b8(gpu):
    cfg = configs.TP8_B8
    say(f'case: {cfg.name} seed=3, general vs persistent decode path')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 3), gpu)
    outs = {}
    for path in ('general', 'decode'):
        ws = k3moe.new_workspace(64 << 20, gpu)
        outs[path] = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=ws)
        torch.cuda.synchronize(gpu)
        assert k3moe.workspace_status(ws) == 0
    a, b = outs['general'], outs['decode']
    assert torch.equal(a['expert_ids'], b['expert_ids'])
    assert (a['route_weights'] - b['route_weights']).abs().max().item() <= 2e-7
    assert moe_ref.rel_l2(b['expert_sum'].cpu(), a['expert_sum'].cpu()) < 5e-3


@pytest.mark.parametrize('path', ['general', 'decode'])
def test_moe_tp8_b64_sampled_rows(gpu, path):
    cfg = configs.TP8_B64
    say(f'case: {cfg.name} seed=1 path={path} (oracle on 8 sampled rows)')
    rows = torch.tensor([0, 5, 17, 31, 32, 47, 58, 63])
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 1), gpu, rows=rows, path=path)


def test_moe_latent_input(gpu):
    cfg = MoEConfig('latent', 32, 4, 192, 64, 6, latent=96)
    say(f'case: {cfg.name}')
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 3, scale_mode='kimi'), gpu)


def test_forced_routes_and_shortfall(gpu):
    cfg = MoEConfig('forced', 32, 4, 128, 64, 9)
    say(f'case: {cfg.name} own routes, then the worst fixed set')
    inp = synthetic.moe_layer_inputs(cfg, 9, scale_mode='kimi')
    free, _ = run_and_check(cfg, inp, gpu)
    forced, _ = run_and_check(cfg, inp, gpu, routes=free['expert_ids'].flip(-1))
    assert torch.equal(forced['expert_sum'], free['expert_sum'])
    assert float(forced['route_shortfall'].max()) == 0.0
    worst = torch.arange(cfg.experts - cfg.topk, cfg.experts).expand(cfg.tokens, -1).contiguous()
    bad, _ = run_and_check(cfg, inp, gpu, routes=worst)
    assert float(bad['route_shortfall'].max()) > grading.ROUTE_FLOOR
    with pytest.raises(ValueError, match='repeated'):
        rep = worst.clone()
        rep[:, 1] = rep[:, 0]
        k3moe.moe_step(*synthetic.step_args(to_dev(inp, gpu)), topk=cfg.topk, routes=rep.to(gpu))


def test_edge_scale_bytes(gpu):
    """Scale bytes 0 and 1 (subnormal products), 2 and 200 (plain), 255 (NaN) inside the GEMMs."""
    cfg = MoEConfig('edge-scales', 16, 2, 128, 64, 8)
    say(f'case: {cfg.name}')
    inp = synthetic.moe_layer_inputs(cfg, 11, scale_mode='kimi')
    for key, val in (('gate_scales', 0), ('up_scales', 1), ('down_scales', 2), ('gate_scales', 200)):
        inp[key].view(-1)[::7] = val
    finite, _ = run_and_check(cfg, inp, gpu)
    assert torch.isfinite(finite['expert_sum']).all()
    nan_in = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    nan_in['gate_scales'][3, 5, 1] = 255        # expert 3 -> NaN for every token routed to it
    g = to_dev(nan_in, gpu)
    got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk)
    oracle = moe_ref.moe_step(*synthetic.step_args(nan_in), topk=cfg.topk)
    nan_rows = (oracle['expert_ids'] == 3).any(-1)
    assert torch.equal(torch.isnan(got['expert_sum'].cpu()).all(-1), nan_rows)
    assert torch.equal(torch.isnan(oracle['expert_sum']).all(-1), nan_rows)


def test_repeatable_bitwise(gpu):
    cfg = configs.TP8_B8
    say(f'case: {cfg.name} run twice, bitwise identical')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 2), gpu)
    a = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk)
    b = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk)
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_moe_layer_reads_reference_keys(gpu):
    cfg = MoEConfig('layer-dict', 16, 2, 64, 64, 4)
    say(f'case: {cfg.name}')
    inp = synthetic.moe_layer_inputs(cfg, 0, layer=3, scale_mode='kimi')
    values = {f'l3_{k}': v.to(gpu) for k, v in inp.items() if k != 'x' and v is not None}
    got = k3moe.moe_layer(values, 3, inp['x'].to(gpu), topk=cfg.topk)
    want = k3moe.moe_step(*synthetic.step_args(to_dev(inp, gpu)), topk=cfg.topk)
    for k in want:
        assert torch.equal(got[k], want[k]), k


@pytest.mark.gpu
def test_submission_build_run_matches_moe_step(gpu):
    from k3moe import submission
    cfg = MoEConfig('submission', 24, 4, 128, 64, 5)
    say(f'case: {cfg.name}')
    inp = to_dev(synthetic.moe_layer_inputs(cfg, 1), gpu)
    want = k3moe.moe_step(*synthetic.step_args(inp), topk=cfg.topk)
    params = {'tokens': cfg.tokens, 'experts': cfg.experts, 'topk': cfg.topk, 'hidden': cfg.hidden,
              'inter': cfg.inter}
    run = submission.build({'params': params})
    got = run({k: v for k, v in inp.items() if v is not None})
    assert set(got) == set(want)
    for k in want:
        assert torch.equal(got[k], want[k]), k
    run3 = submission.build({'params': params, 'layer': 3})
    got3 = run3({('x' if k == 'x' else f'l3_{k}'): v for k, v in inp.items() if v is not None})
    for k in want:
        assert torch.equal(got3[k], want[k]), k


@pytest.mark.parametrize('cfg', [configs.TP8_B8, configs.TP8_B64], ids=lambda c: c.name)
def test_decode_barrier_counters_wrap(gpu, cfg):
    """The persistent kernel's barrier counters are never reset; they grow by
    whole barriers and wrap at 2**32. Preset them (consistently) two barriers
    before the wrap and run steps across it (these batches run the expert-major
    down, one grid barrier before the combine): results equal a fresh
    workspace's and no barrier times out. A wrong target would only hit the
    barrier's bounded wait, which sets the status word."""
    say(f'case: {cfg.name} seed=5, barrier counters preset 2 barriers before the 32-bit wrap')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 5), gpu)
    from k3moe.moe import dims_for, workspace_bytes
    need = workspace_bytes(dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating,
                                    cfg.activation, g.get('latent'), 'decode'))
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    G = 1
    while G * 2 <= min(cus, 1024):
        G *= 2                                  # the persistent grid: largest power of two <= CUs
    groups = min(G, 16)
    members = G // groups
    fresh = k3moe.new_workspace(need, gpu)
    ref = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path='decode', workspace=fresh)
    ws = k3moe.new_workspace(need, gpu)
    ctl = ws[:4096].view(torch.int32)            # control block: top counter word 32, group g at 64 + 32 g
    ctl[32] = -2 * groups
    for gi in range(groups):
        ctl[64 + 32 * gi] = -2 * members
    torch.cuda.synchronize(gpu)
    for step in range(4):
        got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path='decode', workspace=ws)
        torch.cuda.synchronize(gpu)
        say(f'  step {step}: top counter {int(ctl[32].item()) & 0xFFFFFFFF:#x}')
        for key in ('expert_sum', 'expert_ids', 'route_weights'):
            assert torch.equal(got[key], ref[key]), key
    assert k3moe.workspace_status(ws) == 0
    assert k3moe.workspace_status(fresh) == 0
    assert int(ctl[32].item()) & 0xFFFFFFFF < 1 << 16, 'the top counter crossed the wrap'


# ---- the general path's grouped-GEMM expert kernels (many tokens per expert) ----

GROUPED_B512 = MoEConfig('grouped-b512', 32, 4, 1024, 1024, 512, gating='softmax')  # ~64 tokens per expert


@pytest.mark.parametrize('path', ['grouped', 'grouped_bf16', 'streamed'])
def test_general_expert_kernels_plumbing(gpu, path):
    """The expert-kernel variants of the general path on the small case (1-2 tokens per expert)."""
    cfg = configs.CPU_PLUMBING
    say(f'case: {cfg.name} seed=4 path={path}')
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 4), gpu, path=path)


@pytest.mark.parametrize('path', ['grouped', 'grouped_bf16'])
def test_grouped_gemm_b512_sampled_rows(gpu, path):
    cfg = GROUPED_B512
    say(f'case: {cfg.name} seed=2 path={path} (oracle on 8 sampled rows)')
    rows = torch.tensor([0, 1, 100, 255, 256, 300, 510, 511])
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 2), gpu, rows=rows, path=path)


def test_grouped_vs_streamed_b512(gpu):
    """Same routing kernels, so the expert sets are identical; the two expert-kernel
    variants differ only in FP32 summation order inside the dot products."""
    cfg = GROUPED_B512
    say(f'case: {cfg.name} seed=6, grouped vs streamed expert kernels')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 6), gpu)
    outs = {}
    for path in ('grouped', 'streamed'):
        outs[path] = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, gating=cfg.gating, path=path)
        torch.cuda.synchronize(gpu)
    a, b = outs['grouped'], outs['streamed']
    assert torch.equal(a['expert_ids'], b['expert_ids'])
    assert torch.equal(a['route_weights'], b['route_weights'])
    assert bool(torch.isfinite(a['expert_sum']).all())
    assert moe_ref.rel_l2(a['expert_sum'].cpu(), b['expert_sum'].cpu()) < 5e-3


@pytest.mark.parametrize('path', ['grouped', 'grouped_bf16'])
def test_grouped_gemm_experts_over_128_tokens(gpu, path):
    """Forced routes put all 512 tokens on experts 0-3: four 128-token tiles per expert."""
    cfg = GROUPED_B512
    say(f'case: {cfg.name} seed=7 path={path}, every token routed to experts 0-3')
    routes = torch.tensor([[0, 1, 2, 3], [3, 2, 1, 0]]).repeat(cfg.tokens // 2, 1).contiguous()
    rows = torch.tensor([0, 127, 128, 129, 255, 383, 384, 511])
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 7), gpu, routes=routes, rows=rows, path=path)


@pytest.mark.parametrize('width,inter', [(768, 384), (1536, 640)])
def test_grouped_gemm_widths_off_the_fp4_units(gpu, width, inter):
    """Grouped widths that are multiples of 128 but not of the FP4 GEMMs' output units (512 of the
    latent, 256 of inter) run the bf16-MFMA grouped GEMMs; every output column is checked."""
    cfg = MoEConfig(f'grouped-b512-{width}-{inter}', 32, 4, width, inter, 512, gating='softmax')
    say(f'case: {cfg.name} seed=8 path=grouped (oracle on 6 sampled rows)')
    rows = torch.tensor([0, 1, 200, 300, 510, 511])
    run_and_check(cfg, synthetic.moe_layer_inputs(cfg, 8), gpu, rows=rows, path='grouped')


# ---- the stacked-layer and prefill configurations at full size ----

def test_stacked_layers_tp8_b64(gpu):
    """8 stacked MoE layers of the TP8 shard at batch 64, fresh weights per layer (6.7 GB, made on
    the device), launched back to back on one workspace as the benchmark runs them; the oracle
    checks 4 sampled rows of every layer."""
    cfg = configs.TP8_B64_L8
    say(f'case: {cfg.name} seed=0, 8 layers back to back, oracle on 4 rows per layer')
    layers = [synthetic.moe_layer_inputs(cfg, 0, layer=n, device=gpu) for n in range(cfg.layers)]
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    outs = [k3moe.moe_step(*synthetic.step_args(g), **kw) for g in layers]
    torch.cuda.synchronize(gpu)
    ws = k3moe.moe.get_workspace(k3moe.moe.dims_for(layers[0]['x'], layers[0]['router'], layers[0]['gate_blocks'],
                                                    layers[0]['down_blocks'], cfg.topk, cfg.gating, cfg.activation),
                                 gpu)
    assert k3moe.workspace_status(ws) == 0
    for n, (g, o) in enumerate(zip(layers, outs)):
        rows = torch.tensor([n, 17 + n, 40 + n, 63 - n])
        say(f'  layer {n} rows {rows.tolist()}')
        check_outputs(cfg, {k: v.cpu() for k, v in o.items()}, host_view(g), rows=rows)


def test_prefill_b4096_sampled_rows(gpu):
    """The unsharded prefill chunk at full size: E=384, top-8, h=7168, I=2048, 4096 tokens (9 GB of
    MXFP4 experts made on the device), on the grouped-GEMM path AUTO picks; the oracle checks 7
    sampled rows (its routed experts copied to the host)."""
    cfg = configs.PREFILL
    say(f'case: {cfg.name} seed=0 path=auto (grouped GEMMs), oracle on 7 sampled rows')
    g = synthetic.moe_layer_inputs(cfg, 0, device=gpu)
    rows = torch.tensor([0, 1, 1000, 2047, 2048, 3001, 4095])
    # AUTO runs the FP4-MFMA GEMMs here. That MFMA sums each 32-element block of products in a
    # fixed-point register about 15 bits below the block's largest product, truncating the rest
    # (measured on gfx950), so more of the bf16 roundings of gate, up and y land on the other
    # side than with fp32 sums: about 6 % of the pair outputs instead of 0.3 %, with the same
    # band ratio (0.367). Every element stays within two rounding steps of the oracle.
    run_and_check(cfg, g, gpu, rows=rows, host=host_view(g), min_same=0.5)


# ---- status word, forced-route validation on the device, grouping lists ----

@pytest.mark.parametrize('path', ['decode', 'general', 'single'])
def test_old_status_does_not_shorten_waits(gpu, path):
    """A status word and abort counter left set by an earlier step must not let a later
    launch skip its waits: the outputs equal a clean workspace's, the status stays set."""
    cfg = configs.TP8_B1 if path == 'single' else configs.TP8_B8
    say(f'case: {cfg.name} seed=8 path={path}, status word 1 and abort counter 5 preset')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 8), gpu)
    from k3moe.moe import dims_for, workspace_bytes
    need = workspace_bytes(dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating,
                                    cfg.activation, None, path))
    clean = k3moe.new_workspace(need, gpu)
    ref = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=clean)
    ws = k3moe.new_workspace(need, gpu)
    ctl = ws[:4096].view(torch.int32)
    ctl[2] = 1                                   # status word: an old timeout
    ctl[3] = 5                                   # abort counter moved by earlier launches
    torch.cuda.synchronize(gpu)
    for _ in range(2):
        got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=ws)
        torch.cuda.synchronize(gpu)
        for key in ('expert_sum', 'expert_ids', 'route_weights'):
            assert torch.equal(got[key], ref[key]), key
    assert k3moe.workspace_status(ws) == 1
    assert k3moe.workspace_status(clean) == 0


def debug_stall(polls):
    """k3moe_debug_stall: with polls > 0 the router-logit waits give up after that many polls."""
    from k3moe import _native
    _native.check(_native.load().k3moe_debug_stall(polls), 'k3moe_debug_stall')


def reinit(ws):
    """k3moe_workspace_init on an existing workspace (on the current stream)."""
    import ctypes
    from k3moe import _native
    _native.check(_native.load().k3moe_workspace_init(
        ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()),
        ctypes.c_void_p(torch.cuda.current_stream(ws.device).cuda_stream)), 'k3moe_workspace_init')


@pytest.mark.parametrize('path', ['decode', 'single'])
def test_wait_that_gives_up_poisons_output_and_reinit_restores(gpu, path):
    """The failure path of the bounded waits, forced from the host: with k3moe_debug_stall(256)
    the router-logit waits never see their data and give up after 256 polls (a timeout). Every
    workgroup still ends (the others leave their own waits when the abort counter moves),
    expert_sum is NaN everywhere, the status word has the timeout bit; after
    k3moe_workspace_init the same workspace gives a clean workspace's outputs bit for bit."""
    cfg = configs.TP8_B1 if path == 'single' else configs.TP8_B8
    say(f'case: {cfg.name} seed=9 path={path}, router-logit waits forced to give up after 256 polls')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 9), gpu)
    from k3moe.moe import dims_for, workspace_bytes
    need = workspace_bytes(dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating,
                                    cfg.activation, None, path))
    clean = k3moe.new_workspace(need, gpu)
    ref = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=clean)
    ws = k3moe.new_workspace(need, gpu)
    debug_stall(256)
    try:
        bad = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=ws)
        torch.cuda.synchronize(gpu)
    finally:
        debug_stall(0)
    assert bool(torch.isnan(bad['expert_sum']).all())
    assert k3moe.workspace_status(ws) & 1
    reinit(ws)
    assert k3moe.workspace_status(ws) == 0
    for _ in range(2):
        got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, workspace=ws)
        torch.cuda.synchronize(gpu)
        for key in ('expert_sum', 'expert_ids', 'route_weights'):
            assert torch.equal(got[key], ref[key]), key
    assert k3moe.workspace_status(ws) == 0


def raw_step(dims, g, routes, outs, ws):
    """k3moe_moe_step through the C ABI, without the Python layer's checks of `routes`."""
    import ctypes
    from k3moe import _native
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    rc = _native.load().k3moe_moe_step(
        ctypes.byref(dims), p(g['x']), None, p(g['router']), p(g['router_bias']), p(g['gate_blocks']),
        p(g['gate_scales']), p(g['up_blocks']), p(g['up_scales']), p(g['down_blocks']), p(g['down_scales']),
        p(routes), p(outs['expert_sum']), p(outs['expert_ids']), p(outs['route_weights']),
        p(outs['route_shortfall']), p(ws), ctypes.c_size_t(ws.numel()),
        ctypes.c_void_p(torch.cuda.current_stream(ws.device).cuda_stream))
    _native.check(rc, 'k3moe_moe_step')


@pytest.mark.parametrize('path', ['decode', 'general'])
def test_invalid_forced_routes_use_own_topk(gpu, path):
    """Through the C ABI (no host-side check), rows of forced routes with an id out of range or a
    repeated id fall back to the row's own top-k and set status bit 2; valid rows are forced.
    Every id the kernels read is bounds-checked on the device before use."""
    from k3moe.moe import dims_for, workspace_bytes
    cfg = MoEConfig('bad-routes', 32, 4, 128, 64, 6)
    say(f'case: {cfg.name} seed=12 path={path}, forced routes with invalid rows through the C ABI')
    inp = synthetic.moe_layer_inputs(cfg, 12, scale_mode='kimi')
    g = to_dev(inp, gpu)
    free = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path)
    torch.cuda.synchronize(gpu)
    routes = free['expert_ids'].flip(-1).clone()           # valid rows: the own sets, other order
    routes[1, 2] = cfg.experts                              # out of range
    routes[2, 0] = -3                                       # negative
    routes[3, 3] = routes[3, 1]                             # repeated
    routes[4, 0] = 1 << 40                                  # far out of range
    dims = dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating,
                    cfg.activation, None, path)
    ws = k3moe.new_workspace(workspace_bytes(dims), gpu)
    B, k, K = cfg.tokens, cfg.topk, cfg.hidden
    outs = {'expert_sum': torch.full((B, K), float('nan'), device=gpu),
            'expert_ids': torch.full((B, k), -1, dtype=torch.int64, device=gpu),
            'route_weights': torch.zeros(B, k, device=gpu), 'route_shortfall': torch.full((B,), -1.0, device=gpu)}
    raw_step(dims, g, routes.contiguous(), outs, ws)
    torch.cuda.synchronize(gpu)
    assert k3moe.workspace_status(ws) == 2
    # invalid rows: their own top-k, as the free step computes it
    bad = torch.tensor([1, 2, 3, 4], device=gpu)
    for key in ('expert_sum', 'expert_ids', 'route_weights'):
        assert torch.equal(outs[key][bad], free[key][bad]), key
    # valid rows: forced, as a step whose every row is forced that way (the weights' renormalising
    # sum runs in route order, kimi.py:315, so a reordered set may move a weight by an ulp)
    valid = free['expert_ids'].flip(-1).contiguous()
    forced = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, path=path, routes=valid)
    torch.cuda.synchronize(gpu)
    good = torch.tensor([0, 5], device=gpu)
    for key in ('expert_sum', 'expert_ids', 'route_weights'):
        assert torch.equal(outs[key][good], forced[key][good]), key
    assert float(outs['route_shortfall'].abs().max()) == 0.0
    # a valid forced set on the same workspace: the status stays set (sticky) and routes apply
    worst = torch.arange(cfg.experts - k, cfg.experts, device=gpu).expand(B, -1).contiguous()
    raw_step(dims, g, worst, outs, ws)
    torch.cuda.synchronize(gpu)
    assert torch.equal(outs['expert_ids'].cpu(), worst.cpu())
    assert k3moe.workspace_status(ws) == 2


@pytest.mark.parametrize('cfg', [MoEConfig('group-b70', 40, 5, 160, 96, 70),
                                 MoEConfig('group-b300-e16', 16, 4, 128, 128, 300, gating='softmax'),
                                 configs.CPU_PLUMBING], ids=lambda c: c.name)
def test_general_grouping_lists_match_oracle(gpu, cfg):
    """The general path's grouping (kimi.py:319-320) read back from the workspace equals the C
    restatement's lists bit for bit: active experts ascending, per-expert offsets and counts,
    pair tokens (ascending inside an expert), pair weights and the (token, slot) -> pair map."""
    from k3moe.moe import dims_for, workspace_bytes, workspace_layout
    say(f'case: {cfg.name} seed=3 path=general, grouping lists from the workspace')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 3), gpu)
    dims = dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating,
                    cfg.activation, None, 'general')
    ws = k3moe.new_workspace(workspace_bytes(dims), gpu)
    got = k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, gating=cfg.gating, path='general', workspace=ws)
    torch.cuda.synchronize(gpu)
    lay = workspace_layout(dims)
    raw = ws.cpu().numpy()
    i32 = lambda off, n: raw[off:off + 4*n].view(np.int32)
    B, k, E = cfg.tokens, cfg.topk, cfg.experts
    P = B*k
    ids = got['expert_ids'].cpu().numpy()
    counts, offsets, prow, pslot = cdecode.group(ids, E)
    act = np.nonzero(counts)[0]
    D = int(i32(lay['active_count'], 1)[0])
    assert D == len(act)
    assert np.array_equal(i32(lay['active'], D), act)
    assert np.array_equal(i32(lay['offsets'], D), offsets[act])
    assert np.array_equal(i32(lay['counts'], D), counts[act])
    assert np.array_equal(i32(lay['pair_token'], P), prow)
    pof = np.empty(P, np.int32)
    pof[prow*k + pslot] = np.arange(P, dtype=np.int32)
    assert np.array_equal(i32(lay['pair_of'], P), pof)
    w = got['route_weights'].cpu().numpy()
    pw = raw[lay['pair_weight']:lay['pair_weight'] + 4*P].view(np.float32)
    assert np.array_equal(pw.view(np.uint32), w[prow, pslot].view(np.uint32))
    # the combine (kimi.py:318,323): the step's own pair outputs y times the weights, FP32 products
    # and sums from zero in ascending expert order, reproduce expert_sum bit for bit
    K = cfg.width
    y = torch.from_numpy(raw[lay['pair_y']:lay['pair_y'] + 2*P*K].copy()).view(torch.bfloat16).view(P, K).float()
    wt = got['route_weights'].cpu()
    re = torch.zeros(B, K)
    for j in range(k):
        p_of = torch.from_numpy(pof.reshape(B, k)[:, j].astype(np.int64))
        re = re + y[p_of]*wt[:, j, None]
    assert torch.equal(re, got['expert_sum'].cpu())


def test_prepared_step_matches_moe_step(gpu):
    """k3moe.prepare_step: validated once, then each call launches the step on the same tensors;
    a new token row written into x in place is read by the next call."""
    cfg = configs.TP8_B8
    say(f'case: {cfg.name} seeds 21-22 through a prepared step')
    g = to_dev(synthetic.moe_layer_inputs(cfg, 21), gpu)
    g2 = to_dev(synthetic.moe_layer_inputs(cfg, 22), gpu)
    rows = [g['x'].clone(), g2['x'].clone(), g['x'].clone()]
    step = k3moe.prepare_step(*synthetic.step_args(g), topk=cfg.topk)
    for xr in rows:
        g['x'].copy_(xr)
        got = {k: v.clone() for k, v in step().items()}
        want = k3moe.moe_step(*synthetic.step_args(dict(g, x=xr)), topk=cfg.topk)
        torch.cuda.synchronize(gpu)
        for key in want:
            assert torch.equal(got[key], want[key]), key
    with pytest.raises(ValueError, match='shape'):
        k3moe.prepare_step(g['x'][:, :64].contiguous(), *synthetic.step_args(g)[1:], topk=cfg.topk)
