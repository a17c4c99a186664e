"""Kimi K3 MoE-layer weights in the reference's converted per-rank layout.

Restates the MoE part of megabench/tasks/kimi_checkpoint.py:

  conversion (kimi_checkpoint.py:130-142, 74-76)
    Each routed expert of the Hugging Face checkpoint holds w1 (gate), w3 (up)
    and w2 (down) as ``weight_packed`` U8 [rows, cols/2] (E2M1 codes, element
    2j in the low nibble of byte j) and ``weight_scale`` U8 [rows, cols/32]
    (E8M0, bias 127). The experts are stacked to blocks [E, rows, cols/32, 16]
    and scales [E, rows, cols/32] (a view of the same bytes), then split across
    tensor-parallel ranks: gate and up by rows (dim 1), down by columns (the
    block axis, dim 2), the shared experts' gate/up by rows and down by
    columns; router, router_bias (as fp32), latent_down, latent_up and
    latent_norm are replicated (kimi_checkpoint.py:128-135).
  files (kimi_checkpoint.py:166-178)
    ``<root>/tp<TP>/rank<R>/layer<NNN>.safetensors`` holding the layer's
    tensors without the ``l<n>_`` prefix; written through a ``.tmp`` file that
    is then renamed.
  loading (kimi_checkpoint.py:189-214)
    The layer files of one rank become ``l<n>_<name>`` entries; a missing rank
    directory raises FileNotFoundError; the key set and every shape and dtype
    are checked against the per-rank MoE shapes of kimi.py:113-122, with the
    reference's ValueError messages.

Scope: only the MoE-layer tensors (the ones ``k3moe.moe_layer`` and
``k3moe.latent_moe_layer`` read); other keys a real converted file holds
(attention, norms) are left unread. On a GPU the tensors go through two pinned
staging buffers, so that reading the memory-mapped file overlaps the copies
to the device.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from pathlib import Path

import torch

# Per-rank tensor name -> TP split dimension (None: replicated), kimi_checkpoint.py:128-142.
SPLIT = {'router': None, 'router_bias': None, 'latent_down': None, 'latent_up': None, 'latent_norm': None,
         'shared_gate': 0, 'shared_up': 0, 'shared_down': 1,
         'gate_blocks': 1, 'gate_scales': 1, 'up_blocks': 1, 'up_scales': 1, 'down_blocks': 2, 'down_scales': 2}
EXPERT_WEIGHTS = (('gate', 'w1', 1), ('up', 'w3', 1), ('down', 'w2', 2))   # name, HF name, split dim + 1


@dataclass(frozen=True)
class MoEGeometry:
    """The case parameters a MoE layer's shapes depend on (megabench/cases.py:48-55 for Kimi K3)."""
    experts: int = 896
    hidden: int = 7168
    latent_hidden: int = 3584
    intermediate: int = 3072
    shared_experts: int = 2
    tp: int = 8


KIMI_K3 = MoEGeometry()


def moe_layer_shapes(g: MoEGeometry) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
    """Per-rank MoE tensors of one layer: name -> (shape, dtype), restating kimi.py:76-81,113-122."""
    if g.intermediate % g.tp:
        raise ValueError('Kimi attention heads, vocabulary and FFN intermediate must divide TP')
    if (g.intermediate//g.tp) % 32:
        raise ValueError('MXFP4 down-projection shards must align to groups of 32')
    E, h, lh, inter = g.experts, g.hidden, g.latent_hidden, g.intermediate//g.tp
    shared = g.intermediate*g.shared_experts//g.tp
    bf, f32, u8 = torch.bfloat16, torch.float32, torch.uint8
    return {'latent_down': ((lh, h), bf), 'latent_up': ((h, lh), bf), 'latent_norm': ((lh,), bf),
            'router': ((E, h), bf), 'router_bias': ((E,), f32),
            'gate_blocks': ((E, inter, lh//32, 16), u8), 'gate_scales': ((E, inter, lh//32), u8),
            'up_blocks': ((E, inter, lh//32, 16), u8), 'up_scales': ((E, inter, lh//32), u8),
            'down_blocks': ((E, lh, inter//32, 16), u8), 'down_scales': ((E, lh, inter//32), u8),
            'shared_gate': ((shared, h), bf), 'shared_up': ((shared, h), bf), 'shared_down': ((h, shared), bf)}


# ------------------------------------------------------------- conversion --

def stack_expert_mxfp4(packed: list[torch.Tensor], scales: list[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-expert weight_packed [rows, cols/2] and weight_scale [rows, cols/32] -> blocks
    [E, rows, cols/32, 16] and scales [E, rows, cols/32] (kimi_checkpoint.py:136-140)."""
    p, s = torch.stack(packed), torch.stack(scales)
    if p.dtype != torch.uint8 or s.dtype != torch.uint8:
        raise ValueError('MXFP4 blocks and E8M0 scales must be uint8')
    E, rows, half = p.shape
    if half % 16 or tuple(s.shape) != (E, rows, half//16):
        raise ValueError(f'weight_packed {tuple(p.shape)} and weight_scale {tuple(s.shape)} do not form '
                         'MXFP4 blocks of 32')
    return p.view(E, rows, half//16, 16), s


def tp_split(t: torch.Tensor, dim: int, rank: int, tp: int) -> torch.Tensor:
    """Rank `rank`'s contiguous 1/tp slice of `t` along `dim` (kimi_checkpoint.py:74-76)."""
    n = t.shape[dim]//tp
    return t.narrow(dim, rank*n, n).contiguous()


def shard_moe_layer(full: dict[str, torch.Tensor], tp: int) -> list[dict[str, torch.Tensor]]:
    """A layer's unsplit MoE tensors (SPLIT's names; experts already stacked) -> one dict per rank."""
    missing = sorted(set(SPLIT) - set(full))
    if missing:
        raise ValueError(f'MoE layer tensors missing: {missing}')
    out = [{} for _ in range(tp)]
    for name, dim in SPLIT.items():
        t = full[name].to(torch.float32) if name == 'router_bias' else full[name]
        for r in range(tp):
            out[r][name] = t.contiguous() if dim is None else tp_split(t, dim, r, tp)
    return out


def convert_hf_moe_layer(read, layer: int, g: MoEGeometry,
                         prefix: str = 'language_model.model.') -> list[dict[str, torch.Tensor]]:
    """One MoE layer of a Hugging Face Kimi K3 checkpoint -> per-rank tensors.

    `read(name)` returns a checkpoint tensor by its HF name (kimi_checkpoint.py:60-70's reader);
    the names are those of kimi_checkpoint.py:125-142.
    """
    m = f'{prefix}layers.{layer}.block_sparse_moe.'
    full = {'router': read(m + 'gate.weight'), 'router_bias': read(m + 'gate.e_score_correction_bias'),
            'latent_down': read(m + 'routed_expert_down_proj.weight'),
            'latent_up': read(m + 'routed_expert_up_proj.weight'),
            'latent_norm': read(m + 'routed_expert_norm.weight'),
            'shared_gate': read(m + 'shared_experts.gate_proj.weight'),
            'shared_up': read(m + 'shared_experts.up_proj.weight'),
            'shared_down': read(m + 'shared_experts.down_proj.weight')}
    for key, w, _ in EXPERT_WEIGHTS:
        full[key + '_blocks'], full[key + '_scales'] = stack_expert_mxfp4(
            [read(f'{m}experts.{e}.{w}.weight_packed') for e in range(g.experts)],
            [read(f'{m}experts.{e}.{w}.weight_scale') for e in range(g.experts)])
    return shard_moe_layer(full, g.tp)


def layer_path(root: str | os.PathLike, tp: int, rank: int, layer: int) -> Path:
    return Path(root)/f'tp{tp}'/f'rank{rank}'/f'layer{layer:03d}.safetensors'


def write_moe_layer(root: str | os.PathLike, tp: int, layer: int, shards: list[dict[str, torch.Tensor]]) -> None:
    """Write each rank's tensors to its layer file (kimi_checkpoint.py:166-178: .tmp, then rename)."""
    from safetensors.torch import save_file
    if len(shards) != tp:
        raise ValueError(f'{len(shards)} rank shards for tp={tp}')
    for r, tensors in enumerate(shards):
        path = layer_path(root, tp, r, layer)
        path.parent.mkdir(parents=True, exist_ok=True)
        tmp = path.with_name(path.name + '.tmp')
        save_file({k: v.contiguous().cpu() for k, v in tensors.items()}, str(tmp))
        os.replace(tmp, path)


# ---------------------------------------------------------------- loading --

class _Uploader:
    """Host -> GPU copies through two pinned staging buffers on the current stream: the
    memcpy of chunk i + 1 out of the memory-mapped file overlaps the DMA of chunk i."""

    def __init__(self, device: torch.device, chunk: int = 64 << 20):
        self.device, self.chunk = device, chunk
        self.bufs = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.done: list = [None, None]
        self.turn = 0

    def __call__(self, src: torch.Tensor) -> torch.Tensor:
        out = torch.empty(src.shape, dtype=src.dtype, device=self.device)
        if src.numel() == 0:
            return out
        flat = src.contiguous().reshape(-1).view(torch.uint8)
        dst = out.reshape(-1).view(torch.uint8)
        stream = torch.cuda.current_stream(self.device)
        for off in range(0, flat.numel(), self.chunk):
            b = self.turn
            self.turn ^= 1
            if self.done[b] is not None:
                self.done[b].synchronize()  # the DMA that last read this buffer has finished
            n = min(self.chunk, flat.numel() - off)
            self.bufs[b][:n].copy_(flat[off:off + n])
            dst[off:off + n].copy_(self.bufs[b][:n], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(stream)
            self.done[b] = ev
        return out

    def finish(self) -> None:
        for ev in self.done:
            if ev is not None:
                ev.synchronize()


def load_moe_layers(root: str | os.PathLike, g: MoEGeometry, rank: int, layers, device='cpu') -> dict:
    """Rank `rank`'s MoE tensors of `layers` as ``l<n>_<name>`` entries (kimi_checkpoint.py:189-214).

    Raises FileNotFoundError when the rank's directory or a layer file is missing, and ValueError
    (with the reference's messages) when a layer's MoE key set, a shape or a dtype differs from
    moe_layer_shapes(g).
    """
    from safetensors import safe_open
    directory = Path(root)/f'tp{g.tp}'/f'rank{rank}'
    if not directory.is_dir():
        raise FileNotFoundError(f'{directory}: no converted weights; run setup/convert_checkpoint.py --tp {g.tp}')
    expected = moe_layer_shapes(g)
    device = torch.device(device)
    upload = _Uploader(device) if device.type == 'cuda' else None
    values = {}
    for layer in layers:
        path = layer_path(root, g.tp, rank, layer)
        if not path.exists():
            raise FileNotFoundError(f'{path}: no converted weights for layer {layer}')
        with safe_open(str(path), framework='pt', device='cpu') as f:
            present = set(f.keys())
            missing = sorted(set(expected) - present)
            if missing:
                raise ValueError(f'converted weights do not match the fixture: missing '
                                 f'{[f"l{layer}_{k}" for k in missing][:5]}, extra []')
            for key, (shape, dtype) in expected.items():
                t = f.get_tensor(key)
                if tuple(t.shape) != shape or t.dtype != dtype:
                    raise ValueError(f'l{layer}_{key}: converted {tuple(t.shape)} {t.dtype}, fixture {shape} {dtype}')
                values[f'l{layer}_{key}'] = upload(t) if upload else t
    if upload:
        upload.finish()
    return values
