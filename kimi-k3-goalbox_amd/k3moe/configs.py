"""MoE-layer workloads: the geometries the step is tested and measured on.

  cpu-plumbing   E=64  k=8 h=2048 I=256  B=8     softmax top-k gating (the CPU-sized case)
  tp8-b1         E=384 k=8 h=7168 I=256  B=1     one TP8 rank's expert shard, decode
  tp8-b8         same shard, B=8
  tp8-b64        same shard, B=64
  tp8-b64-l8     8 stacked layers of the b64 shard, fresh weights per layer
  prefill-b4096  E=384 k=8 h=7168 I=2048 B=4096  unsharded experts, prefill chunk
  kimi-k3-tp8    E=896 k=16 h=7168 latent=3584 I=384  the real Kimi K3 TP8 rank geometry
                 (megabench/cases.py:48-55, kimi.py:111-121), B=8
All use sigmoid+bias gating (kimi.py:308-315) and SiTU (kimi.py:194-196)
unless stated.
"""

from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class MoEConfig:
    name: str
    experts: int
    topk: int
    hidden: int
    inter: int
    tokens: int
    gating: str = 'sigmoid_bias'
    activation: str = 'situ'
    layers: int = 1
    latent: int | None = None   # expert width when the experts read a separate latent input

    def with_tokens(self, tokens: int) -> 'MoEConfig':
        return replace(self, tokens=tokens, name=f'{self.name.rsplit("-b", 1)[0]}-b{tokens}')

    @property
    def width(self) -> int:
        return self.latent or self.hidden


CPU_PLUMBING = MoEConfig('cpu-plumbing', 64, 8, 2048, 256, 8, gating='softmax')
TP8_B1 = MoEConfig('tp8-b1', 384, 8, 7168, 256, 1)
TP8_B8 = MoEConfig('tp8-b8', 384, 8, 7168, 256, 8)
TP8_B64 = MoEConfig('tp8-b64', 384, 8, 7168, 256, 64)
TP8_B64_L8 = MoEConfig('tp8-b64-l8', 384, 8, 7168, 256, 64, layers=8)
PREFILL = MoEConfig('prefill-b4096', 384, 8, 7168, 2048, 4096)
KIMI_K3_TP8 = MoEConfig('kimi-k3-tp8-b8', 896, 16, 7168, 384, 8, latent=3584)

ALL = {c.name: c for c in (CPU_PLUMBING, TP8_B1, TP8_B8, TP8_B64, TP8_B64_L8, PREFILL, KIMI_K3_TP8)}
