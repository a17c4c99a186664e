"""The allocation-free entry point, k3moe_moe_step_noalloc, through the C ABI (run with -m gpu).

It runs the kernels of k3moe_moe_step on the library's own per-GPU scratch
array instead of a caller's workspace, so its outputs must equal that entry
point's bit for bit: on consecutive calls (the scratch keeps the previous
call's contents), the second with a smaller input, on the persistent decode
path and on the multi-kernel path. A step too large for the scratch is
rejected with a message before anything is launched.
"""

import ctypes

import pytest
import torch

import k3moe
from k3moe import _native, configs, synthetic
from k3moe.configs import MoEConfig
from k3moe.moe import dims_for, workspace_bytes

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def noalloc_step(cfg, g, routes=None):
    """k3moe_moe_step_noalloc on device inputs g; outputs allocated here by the caller."""
    dims = dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating, cfg.activation)
    B, k, K, dev = cfg.tokens, cfg.topk, cfg.width, g['x'].device
    out = {'expert_sum': torch.full((B, K), float('nan'), device=dev),
           'expert_ids': torch.full((B, k), -1, dtype=torch.int64, device=dev),
           'route_weights': torch.full((B, k), float('nan'), device=dev)}
    if routes is not None:
        out['route_shortfall'] = torch.full((B,), float('nan'), device=dev)
    rc = _native.load().k3moe_moe_step_noalloc(
        ctypes.byref(dims), ptr(g['x']), None, ptr(g['router']), ptr(g['router_bias']), ptr(g['gate_blocks']),
        ptr(g['gate_scales']), ptr(g['up_blocks']), ptr(g['up_scales']), ptr(g['down_blocks']),
        ptr(g['down_scales']), ptr(routes), ptr(out['expert_sum']), ptr(out['expert_ids']),
        ptr(out['route_weights']), ptr(out.get('route_shortfall')),
        ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _native.check(rc, 'k3moe_moe_step_noalloc')
    return out


def workspace_step(cfg, g, routes=None):
    """The same step through k3moe_moe_step with a fresh workspace of its own."""
    dims = dims_for(g['x'], g['router'], g['gate_blocks'], g['down_blocks'], cfg.topk, cfg.gating, cfg.activation)
    ws = k3moe.new_workspace(workspace_bytes(dims), g['x'].device)
    return k3moe.moe_step(*synthetic.step_args(g), topk=cfg.topk, gating=cfg.gating, activation=cfg.activation,
                          routes=routes, workspace=ws)


def test_noalloc_matches_workspace_entry_point(gpu):
    # consecutive calls on the shared scratch, each next one smaller: TP8 shard at b64, b8 and b1
    # (persistent decode path), then a small multi-kernel-path case and a forced-route call
    cases = [(configs.TP8_B64, 4, None), (configs.TP8_B8, 5, None), (configs.TP8_B1, 6, None),
             (MoEConfig('general-b70', 24, 4, 256, 128, 70), 7, None),
             (MoEConfig('forced-b9', 32, 4, 128, 64, 9), 8, 'own-reversed')]
    for cfg, seed, forced in cases:
        say(f'case: {cfg.name} seed={seed} routes={forced}, noalloc vs workspace entry point')
        g = synthetic.moe_layer_inputs(cfg, seed, device=gpu)
        routes = None
        if forced:
            routes = workspace_step(cfg, g)['expert_ids'].flip(-1).contiguous()
        want = workspace_step(cfg, g, routes)
        for call in range(2):              # the scratch keeps the previous call's contents
            got = noalloc_step(cfg, g, routes)
            torch.cuda.synchronize(gpu)
            for key in want:
                assert torch.equal(got[key], want[key]), (cfg.name, call, key)
        assert bool(torch.isfinite(got['expert_sum']).all())


def test_noalloc_rejects_a_step_larger_than_its_scratch(gpu):
    cfg = configs.PREFILL
    say(f'case: {cfg.name} dims only: the allocation-free entry point must refuse it')
    d = _native.Dims(tokens=cfg.tokens, experts=cfg.experts, topk=cfg.topk, hidden=cfg.hidden, latent=cfg.width,
                     inter=cfg.inter, gating=0, activation=0, x_dtype=0, path=0)
    lib = _native.load()
    rc = lib.k3moe_moe_step_noalloc(ctypes.byref(d), *([None]*15), ctypes.c_void_p(0))
    assert rc == -2
    msg = lib.k3moe_last_error().decode()
    assert 'allocation-free' in msg and 'workspace' in msg, msg


def scratch_status(dev):
    st = ctypes.c_int32(-1)
    rc = _native.load().k3moe_workspace_status(None, ctypes.byref(st),
                                              ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _native.check(rc, 'k3moe_workspace_status(NULL)')
    return st.value


def scratch_init(dev):
    rc = _native.load().k3moe_workspace_init(None, 0, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _native.check(rc, 'k3moe_workspace_init(NULL)')


def test_noalloc_status_is_readable_and_resettable(gpu):
    """workspace == NULL reads and resets the scratch's status word: a forced-route row with a repeated
    id sets K3MOE_STATUS_ROUTES (that row falls back to its own top-k, as the workspace entry point's
    does), the word stays set over a clean call, and k3moe_workspace_init(NULL) clears it; the next
    steps again equal the workspace entry point's bit for bit."""
    scratch_init(gpu)
    assert scratch_status(gpu) == 0
    cfg = MoEConfig('forced-b6', 32, 4, 128, 64, 6)
    say(f'case: {cfg.name} seed=13, a repeated forced id through the allocation-free entry point')
    g = synthetic.moe_layer_inputs(cfg, 13, device=gpu)
    own = workspace_step(cfg, g)['expert_ids']
    routes = own.flip(-1).clone()
    routes[2, 3] = routes[2, 1]                 # repeated: row 2 is invalid
    got = noalloc_step(cfg, g, routes.contiguous())
    torch.cuda.synchronize(gpu)
    assert scratch_status(gpu) == 2
    assert torch.equal(got['expert_ids'][2], own[2])
    clean = noalloc_step(cfg, g)
    torch.cuda.synchronize(gpu)
    assert scratch_status(gpu) == 2             # sticky until reset
    scratch_init(gpu)
    assert scratch_status(gpu) == 0
    for cfg2, seed in ((configs.TP8_B8, 14), (configs.TP8_B1, 15)):
        say(f'case: {cfg2.name} seed={seed} after the reset')
        g2 = synthetic.moe_layer_inputs(cfg2, seed, device=gpu)
        want = workspace_step(cfg2, g2)
        got2 = noalloc_step(cfg2, g2)
        torch.cuda.synchronize(gpu)
        for key in want:
            assert torch.equal(got2[key], want[key]), (cfg2.name, key)
    assert scratch_status(gpu) == 0
    assert torch.equal(clean['expert_ids'], own)
