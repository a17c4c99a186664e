"""k3moe: the MXFP4 mixture-of-experts step of the Kimi K3 decode oracle on MI355X.

Public API
  moe_step(x, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
           down_blocks, down_scales, *, topk, gating, activation, fp32, routes, latent)
  prepare_step(...same arguments...)            validated once; calling it launches the step
  moe_layer(values, layer, x, *, topk, ...)     reads the reference's weight-dict keys
  mxfp4_decode(blocks, scales, dtype)           bit-exact unpack_mxfp4 on the GPU
  pack_mxfp4(matrix)                            bit-exact pack_mxfp4 (E2M1 + E8M0 encoder) on the GPU
  latent_in / latent_out / latent_block         the latent MoE block around the experts
  latent_moe_layer(values, layer, normalized, *, topk, ...)
  submission.build(case) -> run(inputs)         the reference's plug-in interface

The kernels live in libk3moe.so (hand-written HIP for gfx950, C ABI in
include/k3moe.h). There is no CPU fallback.
"""

from .moe import (moe_layer, moe_step, mxfp4_decode, new_workspace, pack_mxfp4, prepare_step,  # noqa: F401
                  workspace_bytes, workspace_layout, workspace_status)
from .configs import ALL as CONFIGS, MoEConfig  # noqa: F401
from .latent import latent_block, latent_in, latent_moe_layer, latent_moe_step, latent_out  # noqa: F401

__all__ = ['moe_step', 'prepare_step', 'moe_layer', 'mxfp4_decode', 'pack_mxfp4', 'workspace_bytes', 'latent_in', 'latent_out', 'latent_block',
           'latent_moe_layer', 'latent_moe_step', 'CONFIGS', 'MoEConfig']
