"""The converted-checkpoint layout and loader (k3moe.checkpoint; kimi_checkpoint.py:74-76,125-142,166-214).

CPU: synthetic Hugging Face-style expert tensors (weight_packed [rows, cols/2],
weight_scale [rows, cols/32] per expert) are converted for tp = 2 and 4,
written as tp<TP>/rank<R>/layer<NNN>.safetensors and read back. Pins:
  * each rank's shard is the expected row (gate/up) or column (down) slice of
    the stacked experts, byte for byte, and decodes (oracle unpack_mxfp4) to
    that slice of the full decoded matrices (low nibble = even column);
  * the reference's errors: missing directory or layer file, missing key,
    wrong shape, wrong dtype, a down shard that does not align to 32;
  * the TP split is the one the all-reduce undoes: in FP32 the sum over ranks
    of the oracle's per-rank expert_sum equals the unsplit experts' expert_sum
    (to float32 rounding), with the routing fixed.
GPU (-m gpu): every rank of a TP8 checkpoint loaded onto the GPU runs
k3moe.moe_layer; the sum over ranks is within the band of the FP32 truth on the
unsplit experts, next to the BF16 oracle's own per-rank sum; the latent block
runs from the loaded dict bit for bit as from the in-memory one.
"""

import numpy as np
import pytest
import torch

from k3moe import checkpoint as ck
from oracle import moe_ref


def small_geometry(tp):
    return ck.MoEGeometry(experts=16, hidden=256, latent_hidden=128, intermediate=256, shared_experts=2, tp=tp)


def hf_layer(g: ck.MoEGeometry, seed=0, layer=1):
    """A fake HF reader for one MoE layer of geometry g: name -> tensor."""
    gen = torch.Generator().manual_seed(seed)
    E, h, lh, I = g.experts, g.hidden, g.latent_hidden, g.intermediate
    S = I*g.shared_experts
    bf = lambda *s: (torch.randn(*s, generator=gen)*0.05).to(torch.bfloat16)   # noqa: E731
    m = f'language_model.model.layers.{layer}.block_sparse_moe.'
    t = {m + 'gate.weight': bf(E, h), m + 'gate.e_score_correction_bias': torch.randn(E, generator=gen)*0.01,
         m + 'routed_expert_down_proj.weight': bf(lh, h), m + 'routed_expert_up_proj.weight': bf(h, lh),
         m + 'routed_expert_norm.weight': (1 + 0.1*torch.randn(lh, generator=gen)).to(torch.bfloat16),
         m + 'shared_experts.gate_proj.weight': bf(S, h), m + 'shared_experts.up_proj.weight': bf(S, h),
         m + 'shared_experts.down_proj.weight': bf(h, S)}
    for w, rows, cols in (('w1', I, lh), ('w3', I, lh), ('w2', lh, I)):
        for e in range(E):
            t[f'{m}experts.{e}.{w}.weight_packed'] = torch.randint(0, 256, (rows, cols//2), generator=gen,
                                                                   dtype=torch.uint8)
            t[f'{m}experts.{e}.{w}.weight_scale'] = torch.randint(119, 124, (rows, cols//32), generator=gen,
                                                                  dtype=torch.uint8)
    return t


def write_checkpoint(tmp_path, g, layers=(1, 2), seed=0):
    tensors = {}
    for layer in layers:
        t = hf_layer(g, seed + layer, layer)
        tensors.update(t)
        ck.write_moe_layer(tmp_path, g.tp, layer, ck.convert_hf_moe_layer(t.__getitem__, layer, g))
    return tensors


@pytest.mark.parametrize('tp', [2, 4])
def test_shards_are_slices_of_the_stacked_experts(tmp_path, tp):
    g = small_geometry(tp)
    hf = write_checkpoint(tmp_path, g)
    m = 'language_model.model.layers.2.block_sparse_moe.'
    E = g.experts
    for r in range(tp):
        v = ck.load_moe_layers(tmp_path, g, r, [1, 2])
        assert len(v) == 2*len(ck.SPLIT)
        for key, w, dim in ck.EXPERT_WEIGHTS:
            packed = torch.stack([hf[f'{m}experts.{e}.{w}.weight_packed'] for e in range(E)])
            scales = torch.stack([hf[f'{m}experts.{e}.{w}.weight_scale'] for e in range(E)])
            if dim == 1:     # rows
                n = packed.shape[1]//tp
                want_b, want_s = packed[:, r*n:(r+1)*n], scales[:, r*n:(r+1)*n]
            else:            # columns: 16 packed bytes and one scale per block of 32
                nb = scales.shape[2]//tp
                want_b, want_s = packed[:, :, r*nb*16:(r+1)*nb*16], scales[:, :, r*nb:(r+1)*nb]
            got_b, got_s = v[f'l2_{key}_blocks'], v[f'l2_{key}_scales']
            assert torch.equal(got_b.reshape(want_b.shape), want_b)
            assert torch.equal(got_s, want_s)
            # decoded shard == the matching slice of the decoded full matrices
            full = moe_ref.unpack_mxfp4(packed.view(E, packed.shape[1], -1, 16), scales)
            dec = moe_ref.unpack_mxfp4(got_b, got_s)
            if dim == 1:
                assert torch.equal(dec, full[:, r*n:(r+1)*n])
            else:
                c = full.shape[2]//tp
                assert torch.equal(dec, full[:, :, r*c:(r+1)*c])
        S = g.intermediate*g.shared_experts//tp
        assert torch.equal(v['l2_shared_gate'], hf[m + 'shared_experts.gate_proj.weight'][r*S:(r+1)*S])
        assert torch.equal(v['l2_shared_down'], hf[m + 'shared_experts.down_proj.weight'][:, r*S:(r+1)*S])
        assert torch.equal(v['l2_router'], hf[m + 'gate.weight'])
        assert v['l2_router_bias'].dtype == torch.float32


def test_loader_errors(tmp_path):
    from safetensors.torch import load_file, save_file
    g = small_geometry(2)
    with pytest.raises(FileNotFoundError, match='no converted weights'):
        ck.load_moe_layers(tmp_path, g, 0, [1])
    write_checkpoint(tmp_path, g, layers=(1,))
    with pytest.raises(FileNotFoundError, match='layer 3'):
        ck.load_moe_layers(tmp_path, g, 0, [1, 3])
    path = ck.layer_path(tmp_path, 2, 1, 1)
    good = load_file(str(path))
    bad = dict(good)
    del bad['up_scales']
    save_file(bad, str(path))
    with pytest.raises(ValueError, match=r"missing \['l1_up_scales'\]"):
        ck.load_moe_layers(tmp_path, g, 1, [1])
    bad = dict(good, down_blocks=good['down_blocks'][:, :-1].contiguous())
    save_file(bad, str(path))
    with pytest.raises(ValueError, match=r'l1_down_blocks: converted \(16, 127, 4, 16\)'):
        ck.load_moe_layers(tmp_path, g, 1, [1])
    bad = dict(good, router=good['router'].float())
    save_file(bad, str(path))
    with pytest.raises(ValueError, match='l1_router: converted .* torch.float32, fixture .* torch.bfloat16'):
        ck.load_moe_layers(tmp_path, g, 1, [1])
    with pytest.raises(ValueError, match='groups of 32'):
        ck.moe_layer_shapes(ck.MoEGeometry(experts=4, hidden=64, latent_hidden=64, intermediate=96, tp=2))
    with pytest.raises(ValueError, match='MXFP4 blocks of 32'):
        ck.stack_expert_mxfp4([torch.zeros(4, 24, dtype=torch.uint8)], [torch.zeros(4, 1, dtype=torch.uint8)])


def test_tp_split_is_undone_by_the_sum_fp32(tmp_path):
    """Rank partials of the FP32 oracle sum to the unsplit experts' expert_sum (kimi.py:324)."""
    tp = 4
    g = small_geometry(tp)
    g1 = ck.MoEGeometry(g.experts, g.hidden, g.latent_hidden, g.intermediate, g.shared_experts, 1)
    hf = hf_layer(g, 3, 1)
    full = ck.convert_hf_moe_layer(hf.__getitem__, 1, g1)[0]
    ck.write_moe_layer(tmp_path, tp, 1, ck.convert_hf_moe_layer(hf.__getitem__, 1, g))
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(5, g.hidden, generator=gen).to(torch.bfloat16)
    lat = torch.randn(5, g.latent_hidden, generator=gen).to(torch.bfloat16)
    keys = ('router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks', 'up_scales', 'down_blocks',
            'down_scales')
    ref = moe_ref.moe_step(x, *[full[k] for k in keys], topk=4, fp32=True, latent=lat)
    total = torch.zeros_like(ref['expert_sum'])
    for r in range(tp):
        v = ck.load_moe_layers(tmp_path, g, r, [1])
        part = moe_ref.moe_step(x, *[v['l1_' + k] for k in keys], topk=4, fp32=True, latent=lat)
        assert torch.equal(part['expert_ids'], ref['expert_ids'])
        total += part['expert_sum']
    err = float((total - ref['expert_sum']).norm()/ref['expert_sum'].norm())
    assert err < 1e-6, err
    # a plausible mistake, every rank taking rank 0's down columns, is not undone by the sum
    wrong = torch.zeros_like(total)
    for r in range(tp):
        part = ck.shard_moe_layer(full, tp)[r]
        part['down_blocks'] = ck.tp_split(full['down_blocks'], 2, 0, tp)
        part['down_scales'] = ck.tp_split(full['down_scales'], 2, 0, tp)
        wrong += moe_ref.moe_step(x, *[part[k] for k in keys], topk=4, fp32=True, latent=lat)['expert_sum']
    assert float((wrong - ref['expert_sum']).norm()/ref['expert_sum'].norm()) > 0.1


@pytest.mark.gpu
def test_tp8_checkpoint_on_gpu_sums_to_the_unsplit_layer(gpu, tmp_path):
    """All 8 ranks of a converted TP8 layer, loaded onto the GPU, each run the MoE step; their sum
    (the all-reduce of kimi.py:324, on one GPU) is within the band of the FP32 truth on the unsplit
    experts, next to the BF16 oracle's sum over the same rank shards."""
    import k3moe
    from oracle import grading
    print('case: TP8 checkpoint E=64 h=1024 latent=512 I=2048 B=8 top-8', flush=True)
    tp = 8
    g = ck.MoEGeometry(experts=64, hidden=1024, latent_hidden=512, intermediate=2048, shared_experts=2, tp=tp)
    g1 = ck.MoEGeometry(g.experts, g.hidden, g.latent_hidden, g.intermediate, g.shared_experts, 1)
    hf = hf_layer(g, 5, 1)
    full = ck.convert_hf_moe_layer(hf.__getitem__, 1, g1)[0]
    ck.write_moe_layer(tmp_path, tp, 1, ck.convert_hf_moe_layer(hf.__getitem__, 1, g))
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(8, g.hidden, generator=gen).to(torch.bfloat16)
    lat = torch.randn(8, g.latent_hidden, generator=gen).to(torch.bfloat16)
    keys = ('router', 'router_bias', 'gate_blocks', 'gate_scales', 'up_blocks', 'up_scales', 'down_blocks',
            'down_scales')
    truth = moe_ref.moe_step(x, *[full[k] for k in keys], topk=8, fp32=True, latent=lat)
    cand = torch.zeros(8, g.latent_hidden, dtype=torch.float32, device=gpu)
    oracle = torch.zeros(8, g.latent_hidden)
    xd, ld = x.to(gpu), lat.to(gpu)
    for r in range(tp):
        v = ck.load_moe_layers(tmp_path, g, r, [1], device=gpu)
        assert all(t.device.type == 'cuda' for t in v.values())
        got = k3moe.moe_layer(v, 1, xd, topk=8, latent=ld)
        part = moe_ref.moe_step(x, *[v['l1_' + k].cpu() for k in keys], topk=8, latent=lat)
        assert torch.equal(got['expert_ids'].cpu(), part['expert_ids'])
        cand += got['expert_sum']
        oracle += part['expert_sum']
    torch.cuda.synchronize(gpu)
    detail = grading.band_check(cand.cpu(), oracle, truth['expert_sum'], truth['expert_sum'])
    print('band', detail, flush=True)
    # the latent block reads the loaded dict exactly as an in-memory one
    v = ck.load_moe_layers(tmp_path, g, 3, [1], device=gpu)
    mem = {k: t.to(gpu) for k, t in ck.shard_moe_layer(full, tp)[3].items()}
    mem = {f'l1_{k}': t for k, t in mem.items()}
    a = k3moe.latent_moe_layer(v, 1, xd, topk=8)
    b = k3moe.latent_moe_layer(mem, 1, xd, topk=8)
    torch.cuda.synchronize(gpu)
    for k in a:
        assert torch.equal(a[k], b[k]), k
