"""Qwen3-MoE FP8 expert layers from a local safetensors checkpoint (no hub access).

FP8 Qwen3-MoE checkpoints store every expert projection separately, with 128x128 block scales:

    model.layers.{L}.mlp.gate.weight                                bf16 [E, H]       (router)
    model.layers.{L}.mlp.experts.{e}.gate_proj.weight               float8_e4m3fn [I, H]
    model.layers.{L}.mlp.experts.{e}.gate_proj.weight_scale_inv     fp32 [I/128, H/128]
    model.layers.{L}.mlp.experts.{e}.up_proj.weight / ...scale_inv  the same shapes
    model.layers.{L}.mlp.experts.{e}.down_proj.weight               float8_e4m3fn [H, I]
    model.layers.{L}.mlp.experts.{e}.down_proj.weight_scale_inv     fp32 [H/128, I/128]

transformers fuses them on load into the ``FP8Experts`` parameters
(TF/integrations/finegrained_fp8.py:153-178, :662-680): the experts are stacked along a new
dim 0 and gate and up are concatenated along the output rows, gate first
(TF/conversion_mapping.py:893-906, ``MergeModulelist(dim=0)`` then ``Concatenate(dim=1)``).
The ``weight_scale_inv`` companions follow their weights (finegrained_fp8.py:925-940).
This module does the same stacking and concatenation without transformers, so the kernels can
take real weights from a local path.  A checkpoint that already holds the fused tensors
(``mlp.experts.gate_up_proj`` etc.) is read as it is.  bf16 / fp32 expert weights are accepted
too and quantised on the GPU with the 128x128 block quantiser.

Entry points: ``CheckpointIndex(path)``, ``load_moe_layer(path, layer)`` (a dict of tensors)
and ``load_moe_block(path, layer, top_k)`` (an ``MI355XSparseMoeBlock``).
"""

from __future__ import annotations

import glob
import json
import os
from dataclasses import dataclass

import torch

BLOCK = 128
_FP8 = torch.float8_e4m3fn
_FLOAT = (torch.bfloat16, torch.float16, torch.float32)


class CheckpointIndex:
    """Tensor name -> safetensors file of a local checkpoint directory (or a single file).

    Uses ``model.safetensors.index.json``'s ``weight_map`` when present, otherwise the key
    lists of every ``*.safetensors`` file in the directory.
    """

    def __init__(self, path: str):
        from safetensors import safe_open

        self._safe_open = safe_open
        self.root = path if os.path.isdir(path) else os.path.dirname(os.path.abspath(path))
        self.files: dict[str, str] = {}
        index = os.path.join(self.root, "model.safetensors.index.json")
        if os.path.isfile(path):
            with safe_open(path, framework="pt") as f:
                self.files = {k: path for k in f.keys()}
        elif os.path.isfile(index):
            with open(index) as fh:
                wm = json.load(fh)["weight_map"]
            self.files = {k: os.path.join(self.root, v) for k, v in wm.items()}
        else:
            shards = sorted(glob.glob(os.path.join(self.root, "*.safetensors")))
            if not shards:
                raise FileNotFoundError(f"no *.safetensors files under {path}")
            for shard in shards:
                with safe_open(shard, framework="pt") as f:
                    self.files.update({k: shard for k in f.keys()})
        self._handles: dict[str, object] = {}

    def __contains__(self, name: str) -> bool:
        return name in self.files

    def get(self, name: str) -> torch.Tensor:
        """The tensor on the CPU, in its stored dtype; KeyError names the missing tensor."""
        if name not in self.files:
            raise KeyError(f"tensor {name!r} not found in the checkpoint at {self.root}")
        fn = self.files[name]
        h = self._handles.get(fn)
        if h is None:
            h = self._safe_open(fn, framework="pt").__enter__()
            self._handles[fn] = h
        return h.get_tensor(name)

    def close(self) -> None:
        for h in self._handles.values():
            h.__exit__(None, None, None)
        self._handles.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


@dataclass
class MoeLayerWeights:
    """One layer's router and experts in the kernels' layout."""

    w_router: torch.Tensor            # bf16 [E, H]
    gate_up_proj: torch.Tensor        # e4m3fn [E, 2I, H] (or bf16/fp32 before quantisation)
    gate_up_proj_scale_inv: torch.Tensor | None  # fp32 [E, 2I/128, H/128]
    down_proj: torch.Tensor           # e4m3fn [E, H, I]
    down_proj_scale_inv: torch.Tensor | None     # fp32 [E, H/128, I/128]

    @property
    def fp8(self) -> bool:
        return self.gate_up_proj.dtype == _FP8


def _check_scale(name: str, w: torch.Tensor, s: torch.Tensor) -> None:
    if s.dtype != torch.float32:
        raise NotImplementedError(f"{name}: weight_scale_inv dtype {s.dtype} (only float32 block scales)")
    want = tuple(w.shape[:-2]) + (-(-w.shape[-2] // BLOCK), -(-w.shape[-1] // BLOCK))
    if tuple(s.shape) != want:
        raise ValueError(f"{name}: scale shape {tuple(s.shape)} does not match 128x128 blocks of "
                         f"weight {tuple(w.shape)} (expected {want})")


def _expert_count(idx: CheckpointIndex, prefix: str) -> int:
    n = 0
    while f"{prefix}.experts.{n}.down_proj.weight" in idx:
        n += 1
    return n


def load_moe_layer(path: str | CheckpointIndex, layer: int, device: str | torch.device = "cuda",
                   prefix: str = "model.layers") -> MoeLayerWeights:
    """Router and fused experts of decoder layer ``layer``, moved to ``device``."""
    idx = path if isinstance(path, CheckpointIndex) else CheckpointIndex(path)
    p = f"{prefix}.{layer}.mlp"
    w_router = idx.get(f"{p}.gate.weight")
    if w_router.dim() != 2:
        raise ValueError(f"{p}.gate.weight: expected [E, H], got {tuple(w_router.shape)}")
    E, H = w_router.shape
    if f"{p}.experts.gate_up_proj" in idx:  # already fused
        w13 = idx.get(f"{p}.experts.gate_up_proj")
        w2 = idx.get(f"{p}.experts.down_proj")
        s13 = idx.get(f"{p}.experts.gate_up_proj_scale_inv") if w13.dtype == _FP8 else None
        s2 = idx.get(f"{p}.experts.down_proj_scale_inv") if w2.dtype == _FP8 else None
    else:
        n = _expert_count(idx, p)
        if n != E:
            raise KeyError(f"{p}: router has {E} experts but the checkpoint holds {n} "
                           f"(missing {p}.experts.{n}.*)")
        gate = [idx.get(f"{p}.experts.{e}.gate_proj.weight") for e in range(E)]
        up = [idx.get(f"{p}.experts.{e}.up_proj.weight") for e in range(E)]
        down = [idx.get(f"{p}.experts.{e}.down_proj.weight") for e in range(E)]
        # MergeModulelist(dim=0) then Concatenate(dim=1): [E, I, H] gate rows, then up rows
        w13 = torch.cat([torch.stack(gate), torch.stack(up)], dim=1)
        w2 = torch.stack(down)
        s13 = s2 = None
        if w13.dtype == _FP8:
            sg = [idx.get(f"{p}.experts.{e}.gate_proj.weight_scale_inv") for e in range(E)]
            su = [idx.get(f"{p}.experts.{e}.up_proj.weight_scale_inv") for e in range(E)]
            s13 = torch.cat([torch.stack(sg), torch.stack(su)], dim=1)
        if w2.dtype == _FP8:
            s2 = torch.stack([idx.get(f"{p}.experts.{e}.down_proj.weight_scale_inv") for e in range(E)])
    if w13.dim() != 3 or w13.shape[0] != E or w13.shape[2] != H or w13.shape[1] % 2:
        raise ValueError(f"{p}: gate_up weights {tuple(w13.shape)} do not fit [E={E}, 2I, H={H}]")
    I = w13.shape[1] // 2
    if tuple(w2.shape) != (E, H, I):
        raise ValueError(f"{p}: down weights {tuple(w2.shape)}, expected {(E, H, I)}")
    if H % BLOCK or I % BLOCK:
        raise ValueError(f"{p}: hidden {H} and intermediate {I} must be multiples of {BLOCK}")
    for name, w, s in (("gate_up_proj", w13, s13), ("down_proj", w2, s2)):
        if w.dtype == _FP8:
            _check_scale(f"{p}.experts.{name}", w, s)
        elif w.dtype not in _FLOAT:
            raise NotImplementedError(f"{p}.experts.{name}: weight dtype {w.dtype}")
    if (w13.dtype == _FP8) != (w2.dtype == _FP8):
        raise ValueError(f"{p}: gate_up and down weights must both be FP8 or both be floating point")
    dev = torch.device(device)
    mv = lambda t: None if t is None else t.contiguous().to(dev)  # noqa: E731
    return MoeLayerWeights(mv(w_router.to(torch.bfloat16)), mv(w13), mv(s13), mv(w2), mv(s2))


def load_moe_block(path: str | CheckpointIndex, layer: int, top_k: int, norm_topk_prob: bool = True,
                   device: str | torch.device = "cuda", prefix: str = "model.layers"):
    """``MI355XSparseMoeBlock`` of decoder layer ``layer`` (FP8 weights copied, floating-point
    weights quantised on the GPU into 128x128 FP8 blocks)."""
    from .experts import MI355XFp8Experts, MI355XSparseMoeBlock

    lw = load_moe_layer(path, layer, device=device, prefix=prefix)
    E, H = lw.w_router.shape
    I = lw.down_proj.shape[2]
    block = MI355XSparseMoeBlock(E, H, I, top_k, norm_topk_prob, device=device)
    with torch.no_grad():
        block.gate.weight.copy_(lw.w_router)
        if lw.fp8:
            block.experts.gate_up_proj.copy_(lw.gate_up_proj)
            block.experts.gate_up_proj_scale_inv.copy_(lw.gate_up_proj_scale_inv)
            block.experts.down_proj.copy_(lw.down_proj)
            block.experts.down_proj_scale_inv.copy_(lw.down_proj_scale_inv)
        else:
            block.experts = MI355XFp8Experts.from_bf16(lw.gate_up_proj, lw.down_proj)
    return block
