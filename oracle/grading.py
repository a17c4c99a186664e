"""Grading rules restated from the reference (test infrastructure).

band_check       kimi.py:413-429 (rel-L2 band, whole tensor for non-logit outputs)
valid_routes     kimi.py:358-367 (in range, distinct per row)
route_sets       exact set equality with FP64 near-tie certification
snapshot / check_unchanged   megabench/harness/correctness.py:13-45
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .moe_ref import rel_l2, router_f64

BAND = 2.0          # kimi.py:38
FLOOR = 2e-3        # kimi.py:39
ROUTE_FLOOR = 1e-3  # kimi.py:40
TIE_GAP = 1e-5      # FP64 gap below which a differing top-k set counts as a certified near-tie


def band_check(candidate, oracle, truth_o, truth_c, *, name='expert_sum', band=BAND, floor=FLOOR) -> dict:
    """rel-L2(candidate, truth_c) <= band * rel-L2(oracle, truth_o) + floor (kimi.py:413-429).

    truth_o is the FP32 reference on the oracle's routes, truth_c on the
    candidate's routes (they are the same tensor when the routes agree).
    Raises AssertionError on failure or non-finite candidate values.
    """
    candidate = torch.as_tensor(candidate).float().cpu()
    oracle_err = rel_l2(oracle, truth_o)
    cand_err = rel_l2(candidate, truth_c)
    limit = band*oracle_err + floor
    detail = {'candidate_rel_l2': cand_err, 'oracle_rel_l2': oracle_err, 'limit': limit,
              'ratio': cand_err/limit}
    if not bool(torch.isfinite(candidate).all()):
        raise AssertionError(f'{name}: non-finite values {detail}')
    if not cand_err <= limit:
        raise AssertionError(f'{name}: outside the oracle band {detail}')
    return detail


def valid_routes(ids: torch.Tensor, experts: int) -> bool:
    """Ids in [0, experts) and distinct within each row (kimi.py:364-367)."""
    ids = ids.long()
    if bool(((ids < 0) | (ids >= experts)).any()):
        return False
    ordered = ids.sort(-1).values
    return not bool((ordered[..., 1:] == ordered[..., :-1]).any())


def route_sets(candidate_ids, oracle_ids, x, router, bias, topk, gating='sigmoid_bias') -> dict:
    """Exact comparison of per-row expert sets, with FP64 near-tie certification.

    A row whose set differs passes only when the FP64 score gap between the
    k-th and (k+1)-th best experts is at most TIE_GAP (a near-tie that the
    FP32 arithmetic of either side may legitimately resolve differently).
    """
    cand = candidate_ids.long().cpu().sort(-1).values
    orac = oracle_ids.long().cpu().sort(-1).values
    differ = (cand != orac).any(-1)
    rows = differ.nonzero().flatten().tolist()
    detail = {'rows': int(cand.shape[0]), 'differing': len(rows), 'certified': 0, 'gaps': []}
    if rows:
        scores = router_f64(x[rows], router, bias, gating)
        for i, r in enumerate(rows):
            s = np.sort(scores[i])[::-1]
            gap = float(s[topk - 1] - s[topk]) if s.shape[0] > topk else math.inf
            detail['gaps'].append(gap)
            if gap <= TIE_GAP:
                detail['certified'] += 1
    detail['exact'] = detail['differing'] == 0
    detail['ok'] = detail['differing'] == detail['certified']
    return detail


def snapshot(inputs: dict) -> dict:
    """Host copies (small tensors) or two 64-bit device checksums (large ones) of every input.

    Restates correctness.py:13-35: plain and position-weighted sums of the
    32-bit words, weights (i mod 65521) + 1, in chunks of 2**26 words.
    """
    result = {}
    for name, value in inputs.items():
        if not isinstance(value, torch.Tensor):
            continue
        value = value.detach()
        nbytes = value.numel()*value.element_size()
        if nbytes <= 1 << 26 or not value.is_contiguous() or nbytes % 4:
            result[name] = value.to('cpu', copy=True)
            continue
        words = value.reshape(-1).view(torch.uint8).view(torch.int32)
        total = torch.zeros(2, dtype=torch.int64, device=value.device)
        step = 1 << 26
        weight = (torch.arange(step, device=value.device, dtype=torch.int64) % 65521) + 1
        for start in range(0, words.numel(), step):
            chunk = words[start:start + step].to(torch.int64)
            total[0] += chunk.sum()
            total[1] += (chunk*weight[:chunk.numel()]).sum()
        result[name] = total.cpu()
    return result


def check_unchanged(inputs: dict, before: dict) -> None:
    """Raise AssertionError naming the first input whose snapshot changed (correctness.py:39-45)."""
    after = snapshot(inputs)
    for name in before:
        if not torch.equal(after[name], before[name]):
            raise AssertionError(f'candidate mutated input {name}')
