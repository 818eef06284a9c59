"""Build-time NF4 staging straight from a local safetensors checkpoint.

``stream_load_and_quantize_module`` is the second call site of the quantizer
in the reference (``stratum/upload.py:671-904``): a module whose frozen
parameters are empty (meta device, or already freed) is filled from the
checkpoint one tensor at a time, and every NF4-eligible tensor is quantized as
it arrives -- here by the GPU kernel (``quantize_4bit`` on the current device),
with the payload copied back to pinned host memory -- so host memory holds the
payloads so far plus one source tensor. Version-1 cache files are used and
written exactly as ``prepare_nf4`` does.

Only local checkpoints are read: a ``*.safetensors`` file, or a directory with
``model.safetensors`` or ``model.safetensors.index.json`` (sharded). Mapping
pipeline parameter names to checkpoint keys beyond the plain name, resolving
hub model ids and reconstructing fused expert tensors belong to the caller
(``key_fn``).
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Callable, Optional

import torch

from . import upload as U

__all__ = ["stream_load_and_quantize_module"]


def _default_keys(name: str) -> list:
    """Checkpoint keys tried for a parameter name: the name without wrapper
    segments, then with / without a leading ``model.``."""
    canon = U._canonical_param_name(name)
    alt = canon[len("model."):] if canon.startswith("model.") else "model." + canon
    return [canon, alt]


def _shard_index(checkpoint: str | Path) -> Optional[dict]:
    """Checkpoint key -> shard file of a local checkpoint; None if there is none."""
    root = Path(checkpoint)
    if root.is_file() and root.suffix == ".safetensors":
        files = [root]
    elif (root / "model.safetensors.index.json").is_file():
        weight_map = json.loads((root / "model.safetensors.index.json").read_text())["weight_map"]
        return {key: root / shard for key, shard in weight_map.items()}
    elif (root / "model.safetensors").is_file():
        files = [root / "model.safetensors"]
    else:
        return None
    from safetensors import safe_open
    index = {}
    for f in files:
        with safe_open(str(f), framework="pt") as handle:
            index.update({key: f for key in handle.keys()})
    return index


@torch.no_grad()
def stream_load_and_quantize_module(module: torch.nn.Module, hf_model_name: str, *, min_numel: int = 4096,
                                    cache_dir: Optional[Path | str] = None, blocksize: int = 64,
                                    quant_type: str = "nf4", verbose: bool = False,
                                    key_fn: Optional[Callable[[str], list]] = None) -> Optional[U.NF4Stats]:
    """Fill the empty frozen parameters of *module* from the local checkpoint
    *hf_model_name*, NF4-staging the eligible ones as they are read.

    A cache hit attaches the cached payload without reading the checkpoint. A
    payload already attached is counted. Ineligible frozen parameters get their
    tensor (in the parameter's dtype). Returns the statistics, or None when the
    checkpoint or a key is missing (the reference's contract).
    """
    keys_of = key_fn or _default_keys
    cache_root = Path(cache_dir) if cache_dir else None
    stats = U.NF4Stats()
    todo = []
    for slot, p in U._plan(module).unique_params():
        payload = getattr(p, U.NF4_ATTR, None)
        if payload is not None:
            stats.count(payload)
            continue
        if p.requires_grad or not (p.device.type == "meta" or p.data.numel() == 0):
            continue
        if cache_root is not None and U._eligible(p, min_numel):
            payload = U._load_payload_from_cache(U._cache_path(cache_root, slot.qualname), p, blocksize=blocksize,
                                                 quant_type=quant_type)
            if payload is not None:
                U._attach(p, U.NF4_ATTR, payload, slot.owner, slot.name)
                stats.cache_hits += 1
                stats.count(payload)
                continue
        todo.append((slot, p))
    if todo:
        index = _shard_index(hf_model_name)
        if index is None:
            if verbose:
                print(f"  stream_nf4: no safetensors checkpoint at {hf_model_name}", flush=True)
            return None
        by_file: dict = {}
        for slot, p in todo:
            key = next((k for k in keys_of(slot.qualname) if k in index), None)
            if key is None:
                if verbose:
                    print(f"  stream_nf4: no checkpoint key for {slot.qualname}", flush=True)
                return None
            by_file.setdefault(index[key], []).append((slot, p, key))
        from safetensors import safe_open
        for path, items in by_file.items():  # each shard opened once
            with safe_open(str(path), framework="pt") as handle:
                for slot, p, key in items:
                    t = handle.get_tensor(key).to(dtype=p.dtype)
                    if tuple(t.shape) != tuple(p.shape):
                        raise ValueError(f"{key}: checkpoint shape {tuple(t.shape)} != parameter {tuple(p.shape)}")
                    if U._eligible(p, min_numel):
                        U.quantize_and_attach(slot.qualname, p, t, stats, cache_dir=cache_root, blocksize=blocksize,
                                              quant_type=quant_type, owner=slot.owner, pname=slot.name)
                    else:
                        U._replace_param_data(p, t, owner=slot.owner, pname=slot.name)
    if verbose:
        print(stats.summary("stream_nf4"), flush=True)
    return stats
