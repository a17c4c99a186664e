"""Write the committed fixtures under tests/golden/ (run from the repo root).

mxfp4_code_scale_table.npy  uint32 [256 scale bytes][16 E2M1 codes]: FP32 bits of
                            code x 2^(scale-127), NaN for scale 255, from the C
                            restatement (oracle/mxfp4_ref.c); the tests re-derive
                            every finite entry from the closed form.
tiny_moe_seed0.npz          a tiny MoE layer (E=8 k=2 h=64 I=64 B=3, seed 0,
                            kimi-style scales): some input tensors (to detect
                            generator drift) and the oracle's expert_ids,
                            route_weights and expert_sum in BF16 and FP32 modes.
The reference holds no vectors for this path, so these fixtures are
regression anchors of the build's own pinned oracle.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(REPO, 'kimi-k3-goalbox_amd'), REPO]

from k3moe import synthetic  # noqa: E402
from k3moe.configs import MoEConfig  # noqa: E402
from oracle import cdecode, moe_ref  # noqa: E402


def main():
    blocks = np.tile((np.arange(16, dtype=np.uint8) * 17).reshape(1, 1, 16), (256, 1, 1))
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    table = cdecode.mxfp4_decode_bits(blocks, scales)[:, 0:32:2].copy()
    np.save(os.path.join(HERE, 'mxfp4_code_scale_table.npy'), table)

    cfg = MoEConfig('tiny', 8, 2, 64, 64, 3)
    inp = synthetic.moe_layer_inputs(cfg, 0, scale_mode='kimi')
    args = synthetic.step_args(inp)
    bf = moe_ref.moe_step(*args, topk=cfg.topk)
    fp = moe_ref.moe_step(*args, topk=cfg.topk, fp32=True)
    arr = lambda t: t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()
    np.savez_compressed(os.path.join(HERE, 'tiny_moe_seed0.npz'),
                        **{'in_' + k: arr(inp[k]) for k in ('x', 'router', 'gate_blocks', 'down_scales')},
                        expert_ids=bf['expert_ids'].numpy(), route_weights=bf['route_weights'].numpy(),
                        expert_sum_bf16=bf['expert_sum'].numpy(), expert_sum_fp32=fp['expert_sum'].numpy())


if __name__ == '__main__':
    main()
