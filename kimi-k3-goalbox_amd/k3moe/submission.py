"""The reference's plug-in interface for an MXFP4 MoE-layer case: build(case) -> run(inputs).

The reference loads a candidate module and calls ``build(case)`` once with ``Case.to_dict()``
(geometry in ``case['params']``), then ``run(inputs)`` per trial; outputs must match the
oracle's keys, shapes, dtypes and device (megabench/harness/runner.py:53-69,
megabench/tasks/kimi.py:385-394). For the MoE step the case parameters are

    params: tokens, experts, topk, hidden, inter [, latent]   (ints, as Case.params)
    gating: 'sigmoid_bias' (kimi.py:308-315) | 'softmax' (tasks/distributed.py:174-176)
    activation: 'situ' (kimi.py:194-196) | 'silu' (tasks/distributed.py:184)
    layer: optional int; then the weight tensors are read under the reference's
           per-layer names l{layer}_router, ... (kimi.py:114-119)

and ``run(inputs)`` takes x [tokens, hidden] bf16 (the router input, kimi.py:308), the
router / router_bias / {gate,up,down}_{blocks,scales} tensors, optionally ``latent``
[tokens, latent] bf16 (the expert input, kimi.py:317,322) and ``routes`` (forced expert
sets, kimi.py:311-313), and returns expert_sum, expert_ids, route_weights (and
route_shortfall with forced routes). Inputs are never written.
"""

from __future__ import annotations

import torch

from . import moe

REQUIRED = ('tokens', 'experts', 'topk', 'hidden', 'inter')
WEIGHTS = ('router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks', 'up_scales', 'down_blocks',
           'down_scales')


def build(case: dict):
    """Validate the case geometry and return run(inputs) -> outputs."""
    if not isinstance(case, dict) or not isinstance(case.get('params'), dict):
        raise ValueError('case must be a dict with a params dict (Case.to_dict())')
    params = case['params']
    missing = [k for k in REQUIRED if k not in params]
    if missing:
        raise ValueError(f'case params lack {missing}')
    B, E, k, h, I = (int(params[n]) for n in REQUIRED)
    K = int(params.get('latent', h))
    gating = case.get('gating', 'sigmoid_bias')
    activation = case.get('activation', 'situ')
    layer = case.get('layer')
    if gating not in ('sigmoid_bias', 'softmax'):
        raise ValueError(f"gating must be 'sigmoid_bias' or 'softmax', got {gating!r}")
    if activation not in ('situ', 'silu'):
        raise ValueError(f"activation must be 'situ' or 'silu', got {activation!r}")
    if min(B, E, k, h, I, K) < 1 or k > E or h % 32 or I % 32 or K % 32:
        raise ValueError(f'invalid MoE geometry {dict(params)}')
    prefix = f'l{int(layer)}_' if layer is not None else ''
    workspaces: dict = {}

    def run(inputs: dict) -> dict:
        x = inputs['x']
        if x.shape != (B, h):
            raise ValueError(f'x must be [{B}, {h}], got {tuple(x.shape)}')
        latent = inputs.get('latent')
        if K != h and latent is None:
            raise ValueError(f'the case has latent width {K}: inputs need latent [{B}, {K}]')
        w = {n: inputs.get(prefix + n) for n in WEIGHTS}
        absent = [prefix + n for n, t in w.items() if t is None and n != 'router_bias']
        if absent:
            raise ValueError(f'inputs lack {absent}')
        if w['router'].shape[0] != E or w['gate_blocks'].shape[1] != I:
            raise ValueError('weight shapes do not match the case geometry')
        dims = moe.dims_for(x, w['router'], w['gate_blocks'], w['down_blocks'], k, gating, activation,
                            latent=latent)
        nbytes = moe.workspace_bytes(dims)
        key = (x.device.index, nbytes)
        ws = workspaces.get(key)
        if ws is None:
            ws = workspaces[key] = moe.new_workspace(nbytes, x.device)
        routes = inputs.get('routes')
        if routes is not None and routes.dim() == 3:
            routes = routes[int(layer or 0)]
        with torch.inference_mode():
            return moe.moe_step(x, w['router'], w['router_bias'], w['gate_blocks'], w['gate_scales'],
                                w['up_blocks'], w['up_scales'], w['down_blocks'], w['down_scales'], topk=k,
                                gating=gating, activation=activation, routes=routes, latent=latent,
                                workspace=ws)

    return run
