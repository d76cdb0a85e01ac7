"""Checkpoint loading from ``*.safetensors`` (dyllm/utils/weight_loader.py:10-200).

Checkpoint names are first normalised by the model (``normalize_weight_name``, e.g. LLaDA's
``transformer.blocks.N.ff_proj`` -> ``model.layers.N.mlp.gate_proj``) and then routed to this
build's parameters:

* fused projections: ``k_proj``/``v_proj`` -> halves of ``kv_proj``, ``gate_proj``/``up_proj`` ->
  halves of ``gate_up_proj`` (the reference's ``packed_modules_mapping``);
* linear weights are stored as bare parameters (``...q_proj`` rather than ``...q_proj.weight``)
  and biases as ``q_bias`` / ``kv_bias``;
* MoE experts ``mlp.experts.E.{gate,up,down}_proj.weight`` -> slices of the stacked
  ``mlp.gate_up_proj[E]`` / ``mlp.down_proj[E]`` (lladamoe.py:318-348).

Only safetensors files are read (no pickle). Every parameter must be covered, except ``lm_head``
when the embeddings are tied.
"""
from __future__ import annotations

import glob
import os
from typing import Dict, Iterable, Iterator, Set, Tuple

import torch
from torch import nn

_PACKED = {"k_proj": ("kv_proj", 0), "v_proj": ("kv_proj", 1),
           "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1)}
_BIAS = {"q_proj": ("q_bias", None), "k_proj": ("kv_bias", 0), "v_proj": ("kv_bias", 1)}


def safetensor_files(path: str):
    if os.path.isfile(path) and path.endswith(".safetensors"):
        return [path]
    if os.path.isdir(path):
        return sorted(glob.glob(os.path.join(path, "**", "*.safetensors"), recursive=True))
    return []


def has_safetensors(path: str) -> bool:
    return bool(safetensor_files(path))


def safetensors_weights_iterator(path: str) -> Iterator[Tuple[str, torch.Tensor]]:
    from safetensors import safe_open

    files = safetensor_files(path)
    if not files:
        raise FileNotFoundError(f"no .safetensors under {path}")
    for f in files:
        with safe_open(f, framework="pt") as fh:
            for key in fh.keys():
                yield key, fh.get_tensor(key)


def _copy(dst: torch.Tensor, src: torch.Tensor, name: str) -> int:
    if tuple(dst.shape) != tuple(src.shape):
        raise RuntimeError(f"shape mismatch for {name}: parameter {tuple(dst.shape)} vs checkpoint {tuple(src.shape)}")
    dst.copy_(src.to(dtype=dst.dtype, device=dst.device))
    return dst.numel()


def _half(p: torch.Tensor, shard: int) -> torch.Tensor:
    n = p.shape[-2] // 2 if p.dim() == 3 else p.shape[0] // 2
    if p.dim() == 3:
        return p[:, shard * n:(shard + 1) * n]
    return p[shard * n:(shard + 1) * n]


@torch.no_grad()
def load_weights(model: nn.Module, weights: Iterable[Tuple[str, torch.Tensor]]) -> Set[str]:
    params: Dict[str, torch.Tensor] = {k: v.data for k, v in model.named_parameters()}
    written: Dict[str, int] = {}   # elements written per parameter (packed ones fill in parts)

    def put(tgt, dst, w, raw):
        written[tgt] = written.get(tgt, 0) + _copy(dst, w, raw)

    norm = getattr(model, "normalize_weight_name", lambda n: n)
    for raw, w in weights:
        name = norm(raw)
        if name in params:
            put(name, params[name], w, raw)
            continue
        base, _, kind = name.rpartition(".")
        if ".mlp.experts." in base and kind == "weight":
            head, tail = base.split(".mlp.experts.")
            eid, proj = tail.split(".", 1)
            eid = int(eid)
            if proj in ("gate_proj", "up_proj"):
                tgt = f"{head}.mlp.gate_up_proj"
                put(tgt, _half(params[tgt][eid:eid + 1], _PACKED[proj][1])[0], w, raw)
            elif proj == "down_proj":
                tgt = f"{head}.mlp.down_proj"
                put(tgt, params[tgt][eid], w, raw)
            else:
                raise KeyError(f"unexpected expert weight {raw}")
            continue
        if kind == "weight" and base in params:
            put(base, params[base], w, raw)
            continue
        prefix, _, last = base.rpartition(".")
        if kind == "weight" and last in _PACKED:
            tgt = f"{prefix}.{_PACKED[last][0]}"
            if tgt in params:
                put(tgt, _half(params[tgt], _PACKED[last][1]), w, raw)
                continue
        if kind == "bias" and last in _BIAS:
            tgt = f"{prefix}.{_BIAS[last][0]}"
            if tgt in params:
                shard = _BIAS[last][1]
                put(tgt, params[tgt] if shard is None else _half(params[tgt], shard), w, raw)
                continue
        raise KeyError(f"checkpoint tensor {raw!r} (normalised {name!r}) matches no parameter")
    missing = {n for n, p in params.items() if written.get(n, 0) < p.numel()}
    if getattr(getattr(model, "config", None), "tie_word_embeddings", False) and "lm_head" in missing:
        params["lm_head"].copy_(params["model.embed_tokens"])
        missing.discard("lm_head")
    # a checkpoint without attention biases leaves them at zero
    missing = {m for m in missing if not m.endswith("_bias")}
    if missing:
        raise RuntimeError(f"checkpoint leaves parameters unset: {sorted(missing)[:8]}")
    return set(written)


def load_model(model: nn.Module, path: str) -> Set[str]:
    return load_weights(model, safetensors_weights_iterator(path))
