"""The persistent kernels' top-k (threshold from group maxima, then exact ranks
among the candidates) on score patterns that stress it (run with -m gpu):
every key equal, blocks of exact ties, the k best all in one residue class of
the grouping (so that nearly every expert is a candidate), and both gatings.
Expert sets must equal the oracle's stable top-k (kimi.py:310, lowest index
first on ties, distributed.py:175) exactly, with no near-tie allowance.
"""

import pytest
import torch

import k3moe
from k3moe import synthetic
from k3moe.configs import MoEConfig
from oracle import moe_ref

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def with_pattern(cfg, seed, pattern):
    """Seeded inputs of cfg with the router and bias replaced to give the named score pattern."""
    inp = synthetic.moe_layer_inputs(cfg, seed, scale_mode='kimi')
    E, h = cfg.experts, cfg.hidden
    e = torch.arange(E)
    if pattern == 'all-equal':               # every logit 0: every score equal, no bias
        inp['router'] = torch.zeros(E, h, dtype=torch.bfloat16)
        inp['router_bias'] = None
    elif pattern == 'tie-blocks':            # logits 0, bias in five levels: blocks of exact ties
        inp['router'] = torch.zeros(E, h, dtype=torch.bfloat16)
        inp['router_bias'] = ((e * 7) % 5).float() * 0.0625
    elif pattern == 'one-residue':           # the best experts all in residue class 3 mod 32, the rest tied
        inp['router'] = torch.zeros(E, h, dtype=torch.bfloat16)
        inp['router_bias'] = torch.where(e % 32 == 3, 1.0, 0.0)
    elif pattern == 'descending':            # bias falling with the index, router small
        inp['router'] = (inp['router'].float() * 0.01).to(torch.bfloat16)
        inp['router_bias'] = -e.float() / E
    else:
        raise ValueError(pattern)
    return inp


CASES = [
    (MoEConfig('single-e384-k8', 384, 8, 1024, 256, 1), 'all-equal'),
    (MoEConfig('single-e384-k8', 384, 8, 1024, 256, 1), 'tie-blocks'),
    (MoEConfig('single-e384-k8', 384, 8, 1024, 256, 1), 'one-residue'),
    (MoEConfig('single-e384-k8', 384, 8, 1024, 256, 1), 'descending'),
    (MoEConfig('single-e512-k6-softmax', 512, 6, 512, 64, 1, gating='softmax'), 'all-equal'),
    (MoEConfig('decode-e384-k8-b5', 384, 8, 1024, 256, 5), 'tie-blocks'),
    (MoEConfig('decode-e384-k8-b5', 384, 8, 1024, 256, 5), 'one-residue'),
    (MoEConfig('decode-e896-k16-b3', 896, 16, 512, 128, 3), 'tie-blocks'),
    (MoEConfig('decode-e896-k16-b3', 896, 16, 512, 128, 3), 'one-residue'),
    (MoEConfig('decode-e1000-k32-b2', 1000, 32, 512, 64, 2), 'all-equal'),
    (MoEConfig('decode-e1000-k32-b2', 1000, 32, 512, 64, 2), 'descending'),
    (MoEConfig('decode-e64-k8-b8-softmax', 64, 8, 512, 64, 8, gating='softmax'), 'tie-blocks'),
]


@pytest.mark.parametrize('cfg,pattern', CASES, ids=[f'{c.name}-{p}' for c, p in CASES])
def test_topk_patterns_match_oracle_exactly(gpu, cfg, pattern):
    say(f'case: {cfg.name} pattern={pattern} seed=3')
    inp = with_pattern(cfg, 3, pattern)
    if cfg.gating == 'softmax' and pattern == 'tie-blocks':
        inp['router'] = torch.zeros_like(inp['router'])
        inp['router'][:, 0] = ((torch.arange(cfg.experts) * 7) % 5).to(torch.bfloat16)
        inp['x'][:, 0] = 1.0
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    g = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    got = k3moe.moe_step(*synthetic.step_args(g), **kw)
    torch.cuda.synchronize(gpu)
    want = moe_ref.route(inp['x'], inp['router'], inp['router_bias'], cfg.topk, cfg.gating)
    assert torch.equal(got['expert_ids'].cpu(), want['expert_ids']), (got['expert_ids'].cpu(), want['expert_ids'])
    assert float((got['route_weights'].cpu() - want['route_weights']).abs().max()) <= 4e-7
    if pattern == 'all-equal':
        assert torch.equal(want['expert_ids'][0], torch.arange(cfg.topk))
