#!/usr/bin/env python3
"""µs per MXFP4 MoE layer and achieved HBM bandwidth on one MI355X.

A step is one MoE layer (router top-k, MXFP4 gate/up, activation, down,
weighted combine) over one batch of seeded synthetic inputs resident in HBM.
Default workload: one TP8 rank's expert shard (E=384, top-8, h=7168, I=256)
at batch 1 (the headline line), with batches 8 and 64 reported beside it, and
(unless --no-extra) 8 stacked batch-64 layers of that shard with fresh weights
per layer, and the unsharded prefill chunk (I=2048, 4096 tokens), both with
inputs made on the device, and the MXFP4 encoder on a TP8 rank's gate weights
(the "codec" object), and the latent MoE block of the reference's own Kimi K3
TP8 rank at batches 1, 8 and 64 (see workload kimi-latent).

Self-check: the last timed run's outputs are checked against the CPU oracle
(expert sets exact or FP64-certified near-ties, the band ratio of kimi.py's
grader <= 1, finite values; all rows of the batches, sampled rows of the
stacked and prefill configurations), and the workspace status word is read
after each timed loop. A failure prints the JSON line, then exits with 3.

Timing: HIP events on the stream bracket each run of the step: by default the
step's kernel launch on the stream with its outputs and workspace allocated
beforehand (--launch stream), or a replay of the step captured in a HIP graph
(--launch graph; on this stack a one-kernel graph replay adds launch latency
of its own). Before every timed run a 1 GiB buffer is read (summed) so that L2
and the 256 MB MALL hold none of the step's weights (cold cache); a read
leaves no dirty lines whose write-back would land inside the timed region. W
untimed runs come first. The graph's outputs are checked bitwise against an
eager step either way.

Roofline: algorithmic bytes of the step (router + bias + x + the distinct
experts' MXFP4 gate/up/down + outputs, k3moe.traffic.step_bytes) over the
measured duration, against the 8 TB/s HBM peak.

CPU baseline: the CPU oracle's BF16 MoE step (oracle/moe_ref.py, the
restatement of megabench/tasks/kimi.py:307-323) on the same inputs on the host
cores, warmup 1, median of 3.

Workload kimi-latent: the whole latent MoE block of a Kimi K3 TP8 rank
(kimi.py:317-328: latent_down and the shared experts' gate/up, the MoE step on
the 3584-wide latent with 896 experts top-16 and I=384, then the RMS norm,
latent_up and shared_down; bf16 weights outside the experts), timed as one
k3moe.latent_block call (one launch at one and at 8 tokens; three launches at
64); CPU baseline: the restatement of the block (oracle/latent_ref.py).

Workload kimi-moe: the MoE step alone on that rank (its latent as the experts' input).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 2] [--workload tp8|tp8-l8|prefill|kimi-latent|kimi-moe]
                       [--no-extra] [--no-check] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(REPO, 'kimi-k3-goalbox_amd'), REPO]

METRIC = 'µs per MoE layer + achieved HBM GB/s (% of peak), b=1/8/64 on 1 MI355X'


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def percentile(vals, q):
    s = sorted(vals)
    at = (len(s) - 1)*q
    lo = int(at)
    return s[lo] + (s[min(lo + 1, len(s) - 1)] - s[lo])*(at - lo)


# HBM bytes per launch of the step kernel from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this
# script, calibrated on a device copy of known size (k3moe.rocpd writes the file).
TRAFFIC_FILE = 'profiles/hbm_traffic.json'


def measured_traffic() -> dict:
    path = os.path.join(REPO, TRAFFIC_FILE)
    if not os.path.exists(path):
        return {}
    with open(path) as fh:
        return json.load(fh).get('workloads', {})


PHASES = ('router', 'router_tail', 'topk', 'pairs_poll', 'group', 'gate_up', 'gate_up_done', 'down_combine')


def read_trace(cfg, device):
    """Per-phase timing of the last persistent step from its workspace trace area (K3MOE_TRACE=1)."""
    import torch
    import k3moe
    from k3moe import moe
    ws = moe._WORKSPACES.get((device.type, device.index))
    x = torch.empty(cfg.tokens, cfg.hidden, dtype=torch.bfloat16, device=device)
    g = torch.empty(cfg.experts, cfg.inter, cfg.width//32, 16, dtype=torch.uint8, device=device)
    d = torch.empty(cfg.experts, cfg.width, cfg.inter//32, 16, dtype=torch.uint8, device=device)
    r = torch.empty(cfg.experts, cfg.hidden, dtype=torch.bfloat16, device=device)
    lat = torch.empty(cfg.tokens, cfg.width, dtype=torch.bfloat16, device=device) if cfg.latent else None
    total = k3moe.workspace_bytes(moe.dims_for(x, r, g, d, cfg.topk, cfg.gating, cfg.activation, lat))
    full = ws[total - 1024*64*8: total].cpu().view(torch.int64).view(1024, 64).double()
    # rows of the persistent grid: the largest power of two <= the CU count
    # (rows past it hold other launches' stamps or never-written memory)
    G = 1
    while G*2 <= min(torch.cuda.get_device_properties(device).multi_processor_count, 1024):
        G *= 2
    full = full[:G]
    dump = os.environ.get('K3MOE_TRACE_DUMP')
    if dump:
        import numpy as np
        np.save(f'{dump}_{cfg.name}.npy', full.numpy())
    def bounds(out, t0, last):   # the workgroups' first instruction (slot 56) and end (slot 57)
        ent, ext = full[:, 56], full[:, 57]
        ok = (ent > 0) & (ext >= ent)
        if bool(ok.any()):
            out['workgroup_span_us'] = round(float((ext[ok].max() - ent[ok].min())*0.01), 2)
            out['entry_to_first_mark_med_us'] = round(float(((full[ok, 0] - ent[ok])*0.01).median()), 2)
            out['last_phase_to_end_us'] = round(float((ext[ok].max() - full[ok, last].max())*0.01), 2)
            out['first_entry_before_t0_us'] = round(float((t0 - ent[ok].min())*0.01), 2)
    if int(full[0, 55].item()) == 0x5349:   # the single-token kernel's rows
        names = ('router', 'poll_partials', 'gating', 'select', 'weights_ids', 'gate_up', 'poll_h', 'down_combine')
        t0 = full[:, 0].min()
        out = {'kernel': 'single', 'workgroups': G, 'start_spread_us': round(float((full[:, 0].max() - t0)*0.01), 2)}
        prev = full[:, 0]
        for n, name in enumerate(names):
            cur = full[:, n + 1]
            ok = cur > 0
            if not bool(ok.any()):
                continue
            out[name] = {'median_us': round(float(((cur[ok] - prev[ok])*0.01).median()), 2),
                         'grid_done_at_us': round(float((cur[ok].max() - t0)*0.01), 2),
                         'median_done_at_us': round(float((cur[ok].median() - t0)*0.01), 2)}
            prev = torch.where(ok, cur, prev)
        out['total_us'] = round(float((full[:, 8].max() - t0)*0.01), 2)

        def span(a, b):   # median over workgroups of slot b - slot a, where both were written in order
            x, y = full[:, a], full[:, b]
            ok = (x > 0) & (y >= x)
            return round(float(((y[ok] - x[ok])*0.01).median()), 2) if bool(ok.any()) else None
        out['sub_phases_med_us'] = {'poll_first_round_trip': span(1, 10), 'gu_issue': span(5, 9),
                                    'gu_data_and_mfma_wave0': span(9, 12), 'gu_reduce': span(12, 13),
                                    'gu_epilogue_store': span(13, 14), 'gu_tail': span(14, 6)}
        out['poll_rounds_median'] = float(full[:, 11].median())
        bounds(out, t0, 8)
        return out
    raw = full[:, :9]
    t0 = raw[:, 0].min()
    out = {'workgroups': G}
    for n, name in enumerate(PHASES):
        dur = (raw[:, n + 1] - raw[:, n])*0.01   # 100 MHz ticks -> us
        out[name] = {'median_us': round(float(dur.median()), 2), 'max_us': round(float(dur.max()), 2),
                     'grid_done_at_us': round(float((raw[:, n + 1].max() - t0)*0.01), 2)}
    out['total_us'] = round(float((raw[:, 8].max() - t0)*0.01), 2)
    gu = (raw[:, 6] - raw[:, 5])*0.01
    out['gate_up_by_wg_mod8'] = [round(float(gu[j::8].mean()), 1) for j in range(8)]
    out['gate_up_pct'] = [round(float(gu.quantile(q)), 1) for q in (0.0, 0.1, 0.5, 0.9, 1.0)]
    out['gate_up_slowest_wgs'] = [int(x) for x in gu.argsort(descending=True)[:8]]
    out['start_spread_us'] = round(float((raw[:, 0].max() - t0)*0.01), 2)
    bounds(out, t0, 8)
    if float(full[:, 9].max()) > 0:   # expert-major down: stream end, then barrier 4 and the combine
        out['down_stream_done_at_us'] = round(float((full[:, 9].max() - t0)*0.01), 2)
    sub = full[:, 10:12]   # inside top-k: logits gathered, selection done (workgroups that routed a token)
    ok = (sub[:, 0] >= raw[:, 2]) & (sub[:, 1] >= sub[:, 0]) & (sub[:, 1] <= raw[:, 3])
    if bool(ok.any()):
        out['topk_parts'] = {'logits_med_us': round(float(((sub[ok, 0] - raw[ok, 2])*0.01).median()), 2),
                             'select_med_us': round(float(((sub[ok, 1] - sub[ok, 0])*0.01).median()), 2),
                             'tail_med_us': round(float(((raw[ok, 3] - sub[ok, 1])*0.01).median()), 2)}
    def sub(a, b, name, rows=None):   # median of slot b - slot a over workgroups that wrote both in order
        x, y = full[:, a], full[:, b]
        ok = (x > 0) & (y >= x) & (x >= raw[:, 0])
        if bool(ok.any()):
            out.setdefault('sub_phases_med_us', {})[name] = round(float(((y[ok] - x[ok])*0.01).median()), 2)
    sub(0, 31, 'router_loads_mfma')
    sub(31, 1, 'router_reduce_store')
    sub(2, 44, 'topk_gather_loads')
    sub(44, 10, 'topk_gather_compute')
    sub(10, 30, 'topk_select_only')
    sub(30, 11, 'topk_weights_ids')
    sub(4, 28, 'group_count')
    sub(28, 29, 'group_scan')
    sub(29, 5, 'group_place')
    sub(5, 12, 'gu_entry')
    sub(12, 13, 'gu_pre_issue')
    sub(13, 45, 'gu_to_round_barrier')
    sub(35, 14, 'gu_cut_sums')
    sub(14, 15, 'gu_more_rounds')
    sub(15, 6, 'gu_exit')
    sub(5, 32, 'gu_round_table')
    sub(5, 45, 'gu_rt_to_first_barrier')
    sub(45, 46, 'gu_rt_lds_reads')
    sub(46, 47, 'gu_rt_table')
    sub(47, 32, 'gu_rt_second_barrier')
    sub(32, 33, 'gu_stage_x')
    sub(33, 34, 'gu_stream_wave0')
    sub(34, 35, 'gu_wait_all_waves')
    sub(35, 6, 'gu_reduce_finish')
    ends = full[:, 36:44]   # gate/up stream end of each wave, relative to the workgroup's staging barrier
    okw = (ends > 0).all(1) & (full[:, 33] > 0)
    if bool(okw.any()):
        rel = (ends[okw] - full[okw, 33:34])*0.01
        out['gu_stream_end_by_wave_med_us'] = [round(float(rel[:, j].median()), 1) for j in range(8)]
        out['gu_stream_spread_med_us'] = round(float((rel.max(1).values - rel.min(1).values).median()), 1)
    ends = full[:, 48:56]   # expert-major down: stream end of each wave, relative to barrier 3's exit
    okw = (ends > 0).all(1) & (ends.min(1).values >= raw[:, 7])
    if bool(okw.any()):
        rel = (ends[okw] - full[okw, 7:8])*0.01
        out['dn_stream_end_by_wave_med_us'] = [round(float(rel[:, j].median()), 1) for j in range(8)]
        out['dn_stream_end_max_us'] = round(float(rel.max()), 1)
    for n in (2, 3):   # inside grid barriers 3 (row-tile down) and 4 (before the combine): release+add, spin, acquire
        if float(full[:, 13 + 4*n].max()) <= 0:
            continue
        b = full[:, 12 + 4*n: 16 + 4*n]
        out[f'barrier{n + 1}_parts'] = {
            'release_add_med_us': round(float(((b[:, 1] - b[:, 0])*0.01).median()), 2),
            'release_add_max_us': round(float(((b[:, 1] - b[:, 0])*0.01).max()), 2),
            'last_arrival_at_us': round(float((b[:, 1].max() - t0)*0.01), 2),
            'first_release_seen_at_us': round(float((b[:, 2].min() - t0)*0.01), 2),
            'last_release_seen_at_us': round(float((b[:, 2].max() - t0)*0.01), 2),
            'acquire_max_us': round(float(((b[:, 3] - b[:, 2])*0.01).max()), 2)}
    return out


def gpu_inputs(cfg, seed, layers, device, host_gen):
    from k3moe import synthetic
    import torch
    out = []
    for layer in range(layers):
        if host_gen:
            inp = synthetic.moe_layer_inputs(cfg, seed, layer=layer)
            host = inp
            inp = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
        else:
            host = None
            inp = synthetic.moe_layer_inputs(cfg, seed, layer=layer, device=device)
        out.append((inp, host))
    return out


def measure(cfg, *, seed, steps, warmup, cold, device, layers=1, host_gen=True, launch='stream', host_timing=True):
    """Time `steps` runs of `layers` MoE layers; returns per-run ms and the routing stats.

    launch 'stream': each run is the layers' kernel launches on the stream (outputs and
    workspace preallocated); 'graph': each run replays a captured HIP graph of them. Either
    way HIP events on the stream bracket each run, and the graph's outputs are checked
    bitwise against an eager step."""
    import torch
    import k3moe
    from k3moe import synthetic, traffic

    data = gpu_inputs(cfg, seed, layers, device, host_gen)
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    distinct = []
    for inp, _ in data:
        o = k3moe.moe_step(*synthetic.step_args(inp), **kw, latent=inp.get('latent'))
        distinct.append(int(o['expert_ids'].unique().numel()))
    torch.cuda.synchronize(device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for inp, _ in data:   # warm the allocator outside the capture
            k3moe.moe_step(*synthetic.step_args(inp), **kw, latent=inp.get('latent'))
    torch.cuda.current_stream(device).wait_stream(stream)
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [k3moe.moe_step(*synthetic.step_args(inp), **kw, latent=inp.get('latent')) for inp, _ in data]
    flush = torch.ones(1 << 28, dtype=torch.float32, device=device) if cold else None
    sink = torch.zeros((), dtype=torch.float32, device=device)
    for i in range(warmup):
        if cold:
            torch.sum(flush, 0, out=sink)
        graph.replay()
    torch.cuda.synchronize(device)
    run = graph.replay
    host_us = []
    if launch == 'stream':
        calls = [(synthetic.step_args(inp), dict(kw, latent=inp.get('latent'), out=o)) for (inp, _), o in zip(data, outs)]

        def run():
            for a, k_ in calls:
                t = time.perf_counter()
                k3moe.moe_step(*a, **k_)
                host_us.append((time.perf_counter() - t)*1e6)
        for i in range(warmup):
            if cold:
                torch.sum(flush, 0, out=sink)
            run()
        torch.cuda.synchronize(device)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        if cold:
            torch.sum(flush, 0, out=sink)
        starts[i].record()
        run()
        ends[i].record()
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - t0
    ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    host_us = host_us[-steps*layers:]
    # the host side of one moe_step call alone (Python checks, the C ABI call and its launch),
    # back to back with no flush between calls: it bounds a drop-in loop of consecutive layers
    host_loop_us = host_prepared_us = None
    if launch == 'stream' and host_timing:
        t = time.perf_counter()
        for _ in range(50):
            run()
        host_loop_us = (time.perf_counter() - t)*1e6/(50*layers)
        torch.cuda.synchronize(device)
        # the same launches through prepared steps (validated once, k3moe.prepare_step)
        prepared = [k3moe.prepare_step(*a, **k_) for a, k_ in calls]
        t = time.perf_counter()
        for _ in range(50):
            for p in prepared:
                p()
        host_prepared_us = (time.perf_counter() - t)*1e6/(50*layers)
        torch.cuda.synchronize(device)
    # the last timed run's outputs, for the oracle checks
    timed = [{k: v.cpu() for k, v in o.items()} for o in outs]
    # the step's workspace status: 0 unless a wait timed out or a forced-route row was invalid
    inp0 = data[0][0]
    ws = k3moe.moe.get_workspace(k3moe.moe.dims_for(inp0['x'], inp0['router'], inp0['gate_blocks'],
                                                    inp0['down_blocks'], cfg.topk, cfg.gating, cfg.activation,
                                                    inp0.get('latent')), device)
    status = k3moe.workspace_status(ws)
    # the phase timestamps of the last timed (cold) step, before the eager step below overwrites them
    trace = read_trace(cfg, device) if os.environ.get('K3MOE_TRACE') == '1' and layers == 1 else None
    # the graph's outputs equal an eager step on the same inputs (bitwise)
    eager = k3moe.moe_step(*synthetic.step_args(inp0), **kw, latent=inp0.get('latent'))
    torch.cuda.synchronize(device)
    same = all(torch.equal(outs[0][k], eager[k]) for k in eager)
    nbytes = sum(traffic.step_bytes(B=cfg.tokens, E=cfg.experts, k=cfg.topk, h=cfg.hidden, I=cfg.inter,
                                    distinct=d, K=cfg.width) for d in distinct)
    flops = layers*traffic.step_flops(B=cfg.tokens, E=cfg.experts, k=cfg.topk, h=cfg.hidden, I=cfg.inter,
                                      K=cfg.width)
    del graph, outs, flush
    return {'ms': ms, 'wall_s': wall, 'distinct': distinct, 'bytes': nbytes, 'flops': flops,
            'host_us': host_us, 'host_loop_us': host_loop_us, 'host_prepared_us': host_prepared_us,
            'graph_matches_eager': same, 'host_inputs': [h for _, h in data], 'trace': trace,
            'timed': timed, 'status': status, 'device_inputs': [d for d, _ in data]}


KIMI_SHARED, KIMI_SHARED_FAN = 768, 6144  # shared-expert width of a TP8 rank (3072 x 2 / 8), unsharded fan-in
# token rows of the latent block the oracle check covers, per batch (every row up to 8 tokens)
LATENT_ROWS = {1: None, 8: None, 64: [0, 21, 42, 63]}


def measure_latent(cfg, *, seed, steps, warmup, cold, device):
    """Time the latent block (one k3moe.latent_block call) with events around it; returns the
    block's ms per run (as its one stage too)."""
    import torch
    import k3moe
    from k3moe import synthetic, traffic

    w = synthetic.latent_block_inputs(cfg, seed, shared=KIMI_SHARED, shared_fan=KIMI_SHARED_FAN, device=device)
    x = w['x']
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    r = k3moe.latent_block(x, w, **kw)
    torch.cuda.synchronize(device)
    distinct = int(r['expert_ids'].unique().numel())
    lat, sh, out = r['latent'], r['shared_h'], r['output']
    moe_out = {k: r[k] for k in ('expert_sum', 'expert_ids', 'route_weights')}
    # the whole block in one call (k3moe.latent_block: one launch at 1 and 8 tokens)
    outs = {'latent': lat, 'shared_h': sh, 'output': out, **moe_out}
    stages = [('latent_block', lambda: k3moe.latent_block(x, w, **kw, out=outs))]
    flush = torch.ones(1 << 28, dtype=torch.float32, device=device) if cold else None
    sink = torch.zeros((), dtype=torch.float32, device=device)
    for _ in range(warmup):
        if cold:
            torch.sum(flush, 0, out=sink)
        for _, f in stages:
            f()
    torch.cuda.synchronize(device)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(steps)]
    for i in range(steps):
        if cold:
            torch.sum(flush, 0, out=sink)
        ev[i][0].record()
        for j, (_, f) in enumerate(stages):
            f()
            ev[i][j + 1].record()
    torch.cuda.synchronize(device)
    block_ms = [e[0].elapsed_time(e[-1]) for e in ev]
    stage_ms = {name: [e[j].elapsed_time(e[j + 1]) for e in ev] for j, (name, _) in enumerate(stages)}
    timed = {'latent': lat.cpu(), 'shared_h': sh.cpu(), 'output': out.cpu(),
             **{k: v.cpu() for k, v in moe_out.items()}}
    same = torch.equal(out, k3moe.latent_block(x, w, **kw)['output'])
    B, h, lh, S = cfg.tokens, cfg.hidden, cfg.latent, KIMI_SHARED
    nbytes = {'latent_block': traffic.latent_in_bytes(B=B, h=h, lh=lh, S=S)
              + traffic.step_bytes(B=B, E=cfg.experts, k=cfg.topk, h=h, I=cfg.inter, distinct=distinct, K=lh)
              + traffic.latent_out_bytes(B=B, h=h, lh=lh, S=S)}
    host = host_view(w)
    del flush
    return {'ms': block_ms, 'stage_ms': stage_ms, 'distinct': distinct, 'bytes': sum(nbytes.values()),
            'stage_bytes': nbytes, 'repeat_matches': same, 'host': host, 'timed': timed}


def latent_check(cfg, got, host, rows=None) -> dict:
    """The latent block's timed outputs against its CPU restatement (oracle/latent_ref.py, the chain of
    kimi.py:317-328) on token rows `rows` (every row when None; each token's block is independent of
    the others): expert sets exact or FP64-certified, and the band ratio of the block output, the
    experts' latent input and expert_sum <= 1."""
    import torch
    from oracle import grading, latent_ref, moe_ref
    ref_in = dict(host)
    if rows is not None:
        rows = torch.as_tensor(rows)
        ref_in['x'] = host['x'][rows]
        got = {k: v[rows] for k, v in got.items()}
    bf = latent_ref.latent_block(ref_in['x'], ref_in, topk=cfg.topk, gating=cfg.gating)
    sets = grading.route_sets(got['expert_ids'], bf['expert_ids'], ref_in['x'], ref_in['router'],
                              ref_in['router_bias'], cfg.topk, cfg.gating)
    truth_o = latent_ref.latent_block(ref_in['x'], ref_in, topk=cfg.topk, gating=cfg.gating, fp32=True,
                                      routes=bf['expert_ids'])
    truth_c = truth_o if sets['exact'] else latent_ref.latent_block(
        ref_in['x'], ref_in, topk=cfg.topk, gating=cfg.gating, fp32=True, routes=got['expert_ids'])
    ratios = {}
    for name in ('latent', 'expert_sum', 'output'):
        cand = moe_ref.rel_l2(got[name], truth_c[name])
        orc = moe_ref.rel_l2(bf[name], truth_o[name])
        ratios[name] = round(cand/(grading.BAND*orc + grading.FLOOR), 4)
    finite = bool(torch.isfinite(got['output'].float()).all())
    return {'rows': 'all' if rows is None else [int(r) for r in rows], 'sets_exact': sets['exact'],
            'sets_certified': sets['certified'], 'band_ratio': ratios, 'finite': finite,
            'ok': bool(sets['ok'] and finite and max(ratios.values()) <= 1.0)}


def summarize_latent(cfg, m):
    ms_mean = statistics.fmean(m['ms'])
    gbps = m['bytes']/(ms_mean*1e-3)/1e9
    stages = {}
    for name, ms in m['stage_ms'].items():
        t = statistics.fmean(ms)
        g = m['stage_bytes'][name]/(t*1e-3)/1e9
        stages[name] = {'us': round(t*1000, 3), 'us_p50': round(statistics.median(ms)*1000, 3),
                        'algorithmic_bytes': m['stage_bytes'][name], 'hbm_GBps': round(g, 1),
                        'hbm_frac': round(g/8000.0, 4)}
    return {'tokens': cfg.tokens, 'layers': 1, 'us_per_layer': round(ms_mean*1000, 3),
            'us_per_layer_p50': round(statistics.median(m['ms'])*1000, 3),
            'us_per_layer_p95': round(percentile(m['ms'], 0.95)*1000, 3), 'distinct_experts': m['distinct'],
            'algorithmic_bytes': m['bytes'], 'hbm_GBps': round(gbps, 1), 'hbm_frac': round(gbps/8000.0, 4),
            'stages': stages, 'repeat_matches': m['repeat_matches']}


def cpu_baseline_latent(cfg, host, reps=3):
    """The CPU restatement of the latent block (BF16 mode) on the same inputs (warmup 1, median of reps)."""
    import torch
    from oracle import latent_ref
    cores = len(os.sched_getaffinity(0))
    share = os.environ.get('OMP_NUM_THREADS', '')
    if share.isdigit() and int(share) > 0:
        cores = min(cores, int(share))
    torch.set_num_threads(cores)
    latent_ref.latent_block(host['x'], host, topk=cfg.topk)
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        latent_ref.latent_block(host['x'], host, topk=cfg.topk)
        ts.append(time.perf_counter() - t)
    return {'us_per_layer': round(statistics.median(ts)*1e6, 1), 'cores': torch.get_num_threads(), 'reps': reps}


def summarize(cfg, m, layers):
    ms_mean = statistics.fmean(m['ms'])
    ms_p50 = statistics.median(m['ms'])
    us_layer = ms_mean*1000/layers
    gbps = m['bytes']/(ms_mean*1e-3)/1e9
    return {'tokens': cfg.tokens, 'layers': layers, 'us_per_layer': round(us_layer, 3),
            'us_per_layer_p50': round(ms_p50*1000/layers, 3),
            'us_per_layer_p95': round(percentile(m['ms'], 0.95)*1000/layers, 3),
            'distinct_experts': m['distinct'] if layers > 1 else m['distinct'][0],
            'algorithmic_bytes': m['bytes'], 'hbm_GBps': round(gbps, 1),
            'hbm_frac': round(gbps/8000.0, 4), 'tflops': round(m['flops']/(ms_mean*1e-3)/1e12, 3),
            'graph_matches_eager': m['graph_matches_eager'],
            **({'host_us_per_call': round(statistics.median(m['host_us']), 2)} if m['host_us'] else {}),
            **({'host_us_per_call_loop': round(m['host_loop_us'], 2),
                'host_us_per_call_prepared': round(m['host_prepared_us'], 2)} if m['host_loop_us'] else {}),
            **({'trace': m['trace']} if m['trace'] else {})}


def cpu_baseline(cfg, host_inputs, reps=3):
    """The CPU oracle's BF16 step on the same inputs (warmup 1, median of reps)."""
    import torch
    from oracle import moe_ref
    from k3moe import synthetic
    cores = len(os.sched_getaffinity(0))
    share = os.environ.get('OMP_NUM_THREADS', '')
    if share.isdigit() and int(share) > 0:   # the host share this process may use
        cores = min(cores, int(share))
    torch.set_num_threads(cores)
    args = synthetic.step_args(host_inputs)
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation, latent=host_inputs.get('latent'))
    result = moe_ref.moe_step(*args, **kw)
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        moe_ref.moe_step(*args, **kw)
        ts.append(time.perf_counter() - t)
    return {'us_per_layer': round(statistics.median(ts)*1e6, 1), 'cores': torch.get_num_threads(), 'reps': reps,
            'oracle': result}


class _DeviceExperts:
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
    """Oracle inputs for device-resident step inputs: small tensors copied, experts lazy."""
    import torch
    return {k: (_DeviceExperts(v) if k.endswith(('_blocks', '_scales')) else
                v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in g.items()}


def oracle_check(cfg, got, host, rows=None, oracle_bf16=None) -> dict:
    """The timed outputs against the CPU oracle (the grader of kimi.py:413-455): per-row expert
    sets (exact, or FP64-certified near-ties), route weights, and the band ratio
    rel-L2(got, FP32 truth) / (2 rel-L2(BF16 oracle, FP32 truth) + 0.002), which must be <= 1.
    `rows` restricts the oracle to sampled token rows (the large configurations)."""
    import torch
    from oracle import grading, moe_ref
    from k3moe import synthetic
    kw = dict(topk=cfg.topk, gating=cfg.gating, activation=cfg.activation)
    ref_in = dict(host)
    if rows is not None:
        rows = torch.as_tensor(rows)
        ref_in['x'] = host['x'][rows]
        if host.get('latent') is not None:
            ref_in['latent'] = host['latent'][rows]
        got = {k: v[rows] for k, v in got.items()}
    args = synthetic.step_args(ref_in)
    lat = ref_in.get('latent')
    bf = oracle_bf16 if oracle_bf16 is not None else moe_ref.moe_step(*args, **kw, latent=lat)
    sets = grading.route_sets(got['expert_ids'], bf['expert_ids'], ref_in['x'], ref_in['router'],
                              ref_in['router_bias'], cfg.topk, cfg.gating)
    truth_o = moe_ref.moe_step(*args, **kw, fp32=True, routes=bf['expert_ids'], latent=lat)
    truth_c = truth_o if sets['exact'] else moe_ref.moe_step(*args, **kw, fp32=True, routes=got['expert_ids'],
                                                             latent=lat)
    oracle_err = moe_ref.rel_l2(bf['expert_sum'], truth_o['expert_sum'])
    cand_err = moe_ref.rel_l2(got['expert_sum'], truth_c['expert_sum'])
    finite = bool(torch.isfinite(got['expert_sum']).all())
    ratio = cand_err/(grading.BAND*oracle_err + grading.FLOOR)
    out = {'rows': 'all' if rows is None else [int(r) for r in rows], 'sets_exact': sets['exact'],
           'sets_differing': sets['differing'], 'sets_certified': sets['certified'],
           'band_ratio': round(ratio, 4), 'candidate_rel_l2': cand_err, 'oracle_rel_l2': oracle_err,
           'finite': finite}
    if sets['exact']:
        out['route_weight_max_err'] = float((got['route_weights'] - bf['route_weights']).abs().max())
    out['ok'] = bool(sets['ok'] and finite and ratio <= 1.0)
    return out


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the platform's processor string."""
    try:
        with open('/proc/cpuinfo') as fh:
            for line in fh:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


# MI355X dense MFMA peaks. The prefill step's grouped GEMMs run the scaled FP4 MFMA
# (v_mfma_scale_f32_16x16x128_f8f6f4) at the FP8 rate, 5.0 PFLOP/s dense, twice per product (the
# activations are two E4M3 terms): 2.5 PFLOP/s of useful FLOPs, the bf16 MFMA peak.
MFMA_FP8_DENSE_TFLOPS = 5000.0
MFMA_USEFUL_TFLOPS = MFMA_FP8_DENSE_TFLOPS / 2


def measure_encode(device, steps, warmup, check):
    """MXFP4 encoder (k3moe.pack_mxfp4, quantization.py:13-37) on a TP8 rank's gate weights in bf16,
    [384, 256, 7168] made on the device: us per call (HIP events), algorithmic bytes (bf16 in, packed
    blocks and scales out) and GB/s; the first call's expert 0 and 383 are checked bit for bit against
    the oracle's encoder."""
    import torch
    import k3moe
    g = torch.Generator(device=device).manual_seed(11)
    w = (torch.randn(384, 256, 7168, generator=g, device=device)*0.02).to(torch.bfloat16)
    n = w.numel()
    nbytes = 2*n + n//2 + n//32
    out = k3moe.pack_mxfp4(w)
    ok = None
    if check:
        from oracle import pack_ref
        ok = all(torch.equal(out[0][e].cpu(), ref[0]) and torch.equal(out[1][e].cpu(), ref[1])
                 for e in (0, 383) for ref in [pack_ref.pack_mxfp4(w[e].cpu())])
    for _ in range(warmup):
        k3moe.pack_mxfp4(w)
    torch.cuda.synchronize(device)
    times = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        k3moe.pack_mxfp4(w)
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1)*1000.0)
    us = statistics.mean(times)
    del w, out
    return {'kernel': 'k3moe::k_encode', 'shape': [384, 256, 7168], 'dtype_in': 'bf16', 'us': round(us, 2),
            'us_p50': round(statistics.median(times), 2), 'algorithmic_bytes': nbytes,
            'hbm_GBps': round(nbytes/us/1e3, 1), 'hbm_frac': round(nbytes/us/1e3/8000.0, 4), 'oracle_exact': ok}


def roofline_entry(head, cfg, layers, measured, workload):
    """The roofline object of the JSON line: HBM for the decode-sized steps (one persistent kernel),
    MFMA for the prefill step (grouped GEMMs on the scaled FP4 MFMA; its HBM rate is given beside it)."""
    if workload == 'kimi-latent':
        return {'bound': 'hbm', 'kernel': 'k3moe::k_moe_single with the latent projections and output (the '
                                          'whole block, one launch at 1 token); 8 tokens: k_moe_decode with the '
                                          'projections and output (one launch); 64: k_latent_sk<0> + '
                                          'k_moe_decode + k_latent_sk<1>',
                'achieved': head['hbm_GBps'], 'peak': 8000.0, 'unit': 'GB/s', 'frac': head['hbm_frac'],
                'traffic': None}
    if workload == 'prefill':
        return {'bound': 'mfma', 'kernel': 'k3moe::k_fgemm<gate/up> + k3moe::k_fgemm<down> (grouped GEMMs on '
                                           'v_mfma_scale_f32_16x16x128_f8f6f4: MXFP4 weights, two-term E4M3 '
                                           'activations) with the router, top-k, grouping, split and combine kernels',
                'achieved': head['tflops'], 'peak': MFMA_USEFUL_TFLOPS, 'unit': 'TFLOP/s',
                'peak_note': 'useful FLOPs: FP8-rate MFMA (5.0 PFLOP/s dense) run twice per product',
                'frac': round(head['tflops'] / MFMA_USEFUL_TFLOPS, 4), 'traffic': None,
                'hbm': {'achieved': head['hbm_GBps'], 'peak': 8000.0, 'unit': 'GB/s', 'frac': head['hbm_frac']}}
    kernel = 'k3moe::k_moe_single' if cfg.tokens == 1 else 'k3moe::k_moe_decode'
    return {'bound': 'hbm', 'kernel': kernel + ' (the whole step, one launch)',
            'achieved': head['hbm_GBps'], 'peak': 8000.0, 'unit': 'GB/s', 'frac': head['hbm_frac'],
            'traffic': measured.get(cfg.name, {}).get('traffic_bytes') if layers == 1 else None,
            'traffic_source': TRAFFIC_FILE if measured else None}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--workload', default='tp8', choices=['tp8', 'tp8-l8', 'prefill', 'kimi-latent', 'kimi-moe'])
    ap.add_argument('--batches', default='1,8,64', help='batches of the tp8 workload; the first is the headline')
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--warm-cache', action='store_true', help='skip the L2/MALL flush before each replay')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--copy-probe', type=int, default=0, metavar='BYTES',
                    help='first copy BYTES between two device buffers three times (a kernel of known '
                         'traffic, to calibrate the FETCH_SIZE / WRITE_SIZE counters of a --pmc run)')
    ap.add_argument('--launch', default='stream', choices=['stream', 'graph'],
                    help='time stream-ordered launches (default) or HIP-graph replays')
    ap.add_argument('--trace', action='store_true', help='record per-phase timestamps of the persistent kernel '
                    '(sets K3MOE_TRACE=1; adds a few stores per phase)')
    ap.add_argument('--no-extra', action='store_true', help='tp8 workload: leave out the 8-stacked-layer and '
                    'prefill configurations (reported beside the batches by default)')
    ap.add_argument('--no-check', action='store_true', help='skip the oracle checks of the timed outputs')
    ap.add_argument('--no-host-timing', action='store_true', help='leave out the host-cost loops (50 back-to-back '
                    'moe_step calls and 50 prepared launches per workload, warm): for profiles of the timed launches')
    args = ap.parse_args()
    if args.trace:
        os.environ['K3MOE_TRACE'] = '1'
    if args.gpus != 1:
        print(f'bench.py measures one GPU (a TP rank\'s expert shard on one MI355X); --gpus {args.gpus} is not '
              'supported: the multi-GPU path (TP all-reduce of expert_sum) is not part of this build',
              file=sys.stderr)
        sys.exit(2)
    import torch
    from k3moe import configs
    device = torch.device('cuda:0')
    cold = not args.warm_cache

    # (config, layers, inputs made on the host, oracle rows: None = every row)
    if args.workload == 'tp8':
        batches = [int(b) for b in args.batches.split(',')]
        runs = [(configs.TP8_B1.with_tokens(b), 1, True, None) for b in batches]
        if not args.no_extra:
            runs += [(configs.TP8_B64_L8, 8, False, [0, 21, 42, 63]),
                     (configs.PREFILL, 1, False, [0, 1, 2047, 4095])]
            # the latent block of the reference's own Kimi K3 TP8 rank (896 experts, top-16, I=384)
            runs += [(configs.KIMI_K3_TP8.with_tokens(b), 1, False, LATENT_ROWS[b]) for b in (1, 8, 64)]
        workload = f'tp8-rank-b{batches[0]}'
    elif args.workload == 'tp8-l8':
        runs = [(configs.TP8_B64_L8, 8, False, [0, 21, 42, 63])]
        workload = 'tp8-rank-b64-8-stacked-layers'
    elif args.workload == 'kimi-moe':
        batches = [int(b) for b in args.batches.split(',')]
        runs = [(configs.KIMI_K3_TP8.with_tokens(b), 1, True, None) for b in batches]
        workload = f'kimi-k3-tp8-rank-moe-step-b{batches[0]}'
    elif args.workload == 'kimi-latent':
        batches = [int(b) for b in args.batches.split(',')]
        runs = [(configs.KIMI_K3_TP8.with_tokens(b), 1, False, LATENT_ROWS.get(b)) for b in batches]
        workload = f'kimi-k3-tp8-rank-latent-block-b{batches[0]}'
    else:
        runs = [(configs.PREFILL, 1, False, [0, 1, 2047, 4095])]
        workload = 'unsharded-prefill-b4096'

    if args.copy_probe:
        n = args.copy_probe // 16 * 16
        src = torch.ones(n // 4, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize(device)
        log(f'bench: copy probe of {n} bytes x 3 done')
        del src, dst

    results, host, timed, failures = {}, {}, {}, []
    for cfg, layers, host_gen, rows in runs:
        log(f'bench: {cfg.name} layers={layers} steps={args.steps} warmup={args.warmup} cold={cold}')
        if cfg.latent and args.workload != 'kimi-moe':
            m = measure_latent(cfg, seed=args.seed, steps=args.steps, warmup=args.warmup, cold=cold, device=device)
            results[cfg.name] = summarize_latent(cfg, m)
            host[cfg.name] = m['host']
            if not args.no_check:
                log(f'bench: oracle check of the latent block {cfg.name}, rows {rows}')
                results[cfg.name]['check'] = latent_check(cfg, m['timed'], m['host'], rows=rows)
            del m
        else:
            m = measure(cfg, seed=args.seed, steps=args.steps, warmup=args.warmup, cold=cold, device=device,
                        layers=layers, host_gen=host_gen, launch=args.launch, host_timing=not args.no_host_timing)
            results[cfg.name] = summarize(cfg, m, layers)
            results[cfg.name]['workspace_status'] = m['status']
            if m['status'] != 0:
                failures.append(f'{cfg.name}: workspace status {m["status"]} after the timed runs')
            host[cfg.name] = m['host_inputs'][0]
            timed[cfg.name] = m['timed']
            if not host_gen and not args.no_check:
                # inputs made on the device: the oracle on sampled rows of the last layer, now,
                # while the inputs are resident (its routed experts copied to the host)
                log(f'bench: oracle check of {cfg.name}, rows {rows}')
                chk = oracle_check(cfg, m['timed'][-1], host_view(m['device_inputs'][-1]), rows=rows)
                chk['layer'] = layers - 1
                results[cfg.name]['check'] = chk
            del m
        log(f'bench: {cfg.name} {results[cfg.name]}')
        torch.cuda.empty_cache()

    head_cfg, head_layers, _, _ = runs[0]
    head = results[head_cfg.name]
    measured = measured_traffic()
    for cfg, layers, _, _ in runs[1:]:
        if cfg.name == configs.PREFILL.name:   # its MFMA roofline beside the decode batches' HBM one
            results[cfg.name]['roofline'] = roofline_entry(results[cfg.name], cfg, layers, measured, 'prefill')
    for name, r in results.items():
        if name in measured and r['layers'] == 1:
            r['hbm_traffic_bytes'] = measured[name]['traffic_bytes']
    cpu, per = None, {}
    if not args.no_cpu_baseline and args.workload in ('tp8', 'kimi-latent', 'kimi-moe'):
        # the latent block's oracle decodes every routed expert (up to 896 at b64): head batch only;
        # the CPU baseline covers the configurations made on the host (the batches of one layer)
        for cfg, _, host_gen, _ in (runs[:1] if args.workload == 'kimi-latent' else runs):
            if args.workload == 'tp8' and (not host_gen or cfg.latent):
                results[cfg.name]['cpu_us_per_layer'] = None
                continue
            log(f'cpu baseline: {cfg.name}')
            per[cfg.name] = (cpu_baseline_latent if args.workload == 'kimi-latent' else cpu_baseline)(
                cfg, host[cfg.name])
            results[cfg.name]['cpu_us_per_layer'] = per[cfg.name]['us_per_layer']
        c0 = per[head_cfg.name]
        cpu = {'value': c0['us_per_layer'], 'unit': 'us/layer', 'cores': c0['cores'], 'kind': 'port',
               'sample': f'{head_cfg.name} seed {args.seed}: one full '
                         + ('latent MoE block' if args.workload == 'kimi-latent' else 'MoE layer')
                         + ' of the CPU oracle (BF16 mode), median of 3 after 1 warmup; batches '
                         + ', '.join(f'{k}: {v["us_per_layer"]} us' for k, v in per.items())
                         + ('' if args.workload == 'kimi-latent' else
                            '; not measured for the stacked-layer and prefill configurations (a stacked '
                            'layer is the b64 layer\'s work; the prefill oracle decodes every expert)'),
               'cpu': cpu_model()}
    if args.workload != 'kimi-latent' and not args.no_check:
        for cfg, layers, host_gen, rows in runs:
            if not host_gen or (cfg.latent and args.workload != 'kimi-moe'):
                continue
            log(f'bench: oracle check of {cfg.name}')
            orc = per[cfg.name]['oracle'] if cfg.name in per else None
            results[cfg.name]['check'] = oracle_check(cfg, timed[cfg.name][0], host[cfg.name], rows=rows,
                                                      oracle_bf16=orc)
    for name, r in results.items():
        if 'check' in r and not r['check']['ok']:
            failures.append(f'{name}: timed outputs fail the oracle check {r["check"]}')

    codec = None
    if args.workload == 'tp8' and not args.no_extra:
        log('bench: MXFP4 encoder')
        codec = measure_encode(device, args.steps, args.warmup, not args.no_check)
        log(f'bench: encoder {codec}')
        if codec['oracle_exact'] is False:
            failures.append(f'encoder output differs from the oracle {codec}')
        torch.cuda.empty_cache()
    ms_step = head['us_per_layer']*head_layers/1000.0
    line = {
        'metric': METRIC,
        'value': head['us_per_layer'],
        'unit': 'us/layer',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms_step, 6),
        'higher_is_better': False,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic',
        'config': {'workload': workload, 'experts': head_cfg.experts, 'topk': head_cfg.topk,
                   'hidden': head_cfg.hidden, 'inter': head_cfg.inter, 'tokens': head_cfg.tokens,
                   'layers': head_layers, 'weights': 'mxfp4 (e2m1 + e8m0/32), dequantized to bf16 in registers',
                   'accumulate': 'fp32', 'cache': 'cold (1 GiB read before each replay)' if cold else 'warm',
                   'timing': 'HIP events around ' + ('stream-ordered launches' if args.launch == 'stream'
                                                      else 'HIP-graph replays')},
        'hbm_GBps': head['hbm_GBps'],
        'hbm_frac': head['hbm_frac'],
        'checks_ok': None if args.no_check else not failures,
        'per_batch': results,
        'roofline': roofline_entry(head, head_cfg, head_layers, measured, args.workload),
        'cpu_baseline': cpu,
    }
    if codec is not None:
        line['codec'] = codec
    print(json.dumps(line), flush=True)
    if failures:
        for f in failures:
            log('bench: FAILED ' + f)
        sys.exit(3)


if __name__ == '__main__':
    main()
