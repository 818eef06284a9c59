"""Build-time NF4 staging straight from a local safetensors checkpoint.

``stream_load_and_quantize_module`` is the second call site of the quantizer
in the reference (``stratum/upload.py:671-904``): a module whose frozen
parameters are empty (meta device, or already freed) is filled from the
checkpoint one tensor at a time, and every NF4-eligible tensor is quantized as
it arrives -- here by the GPU kernel (``quantize_4bit`` on the current device),
with the payload copied back to pinned host memory -- so host memory holds the
payloads so far plus one source tensor. Version-1 cache files are used and
written exactly as ``prepare_nf4`` does.

Checkpoints are read from local files only: a ``*.safetensors`` file, a
directory with ``model.safetensors`` or ``model.safetensors.index.json``
(sharded), or a hub model id whose files are already in the local Hugging Face
cache (looked up without any network access). Pipeline parameter names are
mapped to checkpoint keys as the reference maps them
(``stratum/upload.py:425-473``): stage wrappers that carry a layer index
(``idx``) and wrap a ``layer`` become ``model.layers.<idx>.``, PEFT's
``.base_layer.`` and the ``.inner.`` / ``.layer.`` wrapper segments are
dropped, a leading ``model.`` is optional, and a tied ``lm_head.weight`` falls
back to the input embedding. A fused 3-D expert bank
(``...feed_forward.experts.gate_up_proj`` / ``down_proj``) missing from the
checkpoint is stacked from its per-expert ``w1``/``w3`` / ``w2`` tensors
(``stratum/upload.py:477-531``). ``key_fn`` replaces the name mapping.
"""

from __future__ import annotations

import json
import re
from pathlib import Path
from typing import Callable, Optional

import torch

from . import upload as U

__all__ = ["stream_load_and_quantize_module", "checkpoint_key_fn"]


_LAYER_SEGMENT = re.compile(r"\.layer\.(?!layer)")


def _spellings(name: str) -> list:
    """Checkpoint spellings of one dotted name, in the order they are tried:
    with and without ``.inner.``; for each, as is and with ``.layer.``
    segments dropped; for each, with and without PEFT's ``.base_layer.``;
    then all of those again under a leading ``model.``."""
    bases = [name] + ([name.replace(".inner.", ".")] if ".inner." in name else [])
    out = []
    for b in bases:
        plain = [v for s in (b, _LAYER_SEGMENT.sub(".", b)) for v in (s, s.replace(".base_layer.", "."))]
        out += plain + ["model." + v for v in plain]
    return out


def checkpoint_key_fn(module: torch.nn.Module) -> Callable[[str], list]:
    """``name -> [checkpoint keys to try]`` for the parameters of *module*
    (the mapping of ``stratum/upload.py:425-473``, restated).

    Wrappers found in *module* that carry an integer ``idx`` and a ``layer``
    submodule are stage-local: a name under ``<wrapper>.layer.`` is also tried
    as ``model.layers.<idx>.<rest>``. ``lm_head.weight`` is also tried as the
    input embedding (tied heads store only that)."""
    globals_of = []
    for qual, sub in module.named_modules():
        idx = getattr(sub, "idx", None)
        if isinstance(idx, int) and not isinstance(idx, bool) and hasattr(sub, "layer"):
            globals_of.append((f"{qual}.layer." if qual else "layer.", f"model.layers.{idx}."))

    def keys(name: str) -> list:
        canon = U._canonical_param_name(name)
        names = [canon]
        if canon == "lm_head.weight":
            names += ["model.embed_tokens.weight", "embed_tokens.weight"]
        names += [g + canon[len(p):] for p, g in globals_of if canon.startswith(p)]
        return list(dict.fromkeys(k for n in names for k in _spellings(n)))

    return keys


_EXPERT_BANKS = {".feed_forward.experts.gate_up_proj": ("w1", "w3"), ".feed_forward.experts.down_proj": ("w2",)}


def _expert_bank_keys(name: str, p: torch.nn.Parameter, keys_of: Callable[[str], list], index: dict):
    """Per-expert keys of a fused expert bank parameter (3-D, ``[E, ...]``), as
    ``[[keys of expert 0], ...]`` with the tensors of one expert concatenated
    along dim 0 (gate_up = w1 ++ w3); None if *name* is no bank or the
    checkpoint lacks an expert."""
    if p.ndim != 3:
        return None
    canon = U._canonical_param_name(name)
    suffix = next((s for s in _EXPERT_BANKS if canon.endswith(s)), None)
    if suffix is None:
        return None
    for cand in keys_of(canon):
        if not cand.endswith(suffix):
            continue
        base = cand[: -len(suffix)] + ".feed_forward.experts"
        per = [[f"{base}.{e}.{w}.weight" for w in _EXPERT_BANKS[suffix]] for e in range(int(p.shape[0]))]
        if all(k in index for ks in per for k in ks):
            return per
    return None


def _resolve_checkpoint(source: str | Path) -> Optional[Path]:
    """A local path as given; a hub model id through the local Hugging Face
    cache only (the directory holding its cached index or single file)."""
    root = Path(source)
    if root.exists():
        return root
    try:
        from huggingface_hub import try_to_load_from_cache
    except ImportError:
        return None
    for fname in ("model.safetensors.index.json", "model.safetensors"):
        try:
            hit = try_to_load_from_cache(str(source), fname)
        except Exception:  # not a valid repo id
            return None
        if isinstance(hit, str) and Path(hit).is_file():
            return Path(hit).parent
    return None


def _shard_index(checkpoint: str | Path) -> Optional[dict]:
    """Checkpoint key -> shard file of a local checkpoint; None if there is none."""
    root = _resolve_checkpoint(checkpoint)
    if root is None:
        return None
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
    keys_of = key_fn or checkpoint_key_fn(module)
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
    if not todo:
        if verbose:
            print(stats.summary("stream_nf4"), flush=True)
        return stats
    index = _shard_index(hf_model_name)
    if index is None:
        if verbose:
            print(f"  stream_nf4: no safetensors checkpoint at {hf_model_name}", flush=True)
        return None
    by_file: dict = {}
    banks = []
    for slot, p in todo:
        key = next((k for k in keys_of(slot.qualname) if k in index), None)
        if key is not None:
            by_file.setdefault(index[key], []).append((slot, p, key))
            continue
        per_expert = _expert_bank_keys(slot.qualname, p, keys_of, index)
        if per_expert is None:
            if verbose:
                print(f"  stream_nf4: no checkpoint key for {slot.qualname}", flush=True)
            return None
        banks.append((slot, p, per_expert))

    def place(slot, p, t, key):
        t = t.to(dtype=p.dtype)
        if tuple(t.shape) != tuple(p.shape):
            raise ValueError(f"{key}: checkpoint shape {tuple(t.shape)} != parameter {tuple(p.shape)}")
        if U._eligible(p, min_numel):
            U.quantize_and_attach(slot.qualname, p, t, stats, cache_dir=cache_root, blocksize=blocksize,
                                  quant_type=quant_type, owner=slot.owner, pname=slot.name)
        else:
            U._replace_param_data(p, t, owner=slot.owner, pname=slot.name)

    from safetensors import safe_open
    for path, items in by_file.items():  # each shard opened once
        with safe_open(str(path), framework="pt") as handle:
            for slot, p, key in items:
                place(slot, p, handle.get_tensor(key), key)
    for slot, p, per_expert in banks:  # one bank in host memory at a time
        handles: dict = {}
        try:
            def get(k):
                f = index[k]
                if f not in handles:
                    handles[f] = safe_open(str(f), framework="pt")
                return handles[f].get_tensor(k)
            bank = torch.stack([torch.cat([get(k) for k in ks], dim=0) for ks in per_expert], dim=0)
        finally:
            handles.clear()
        place(slot, p, bank, slot.qualname)
        del bank
    if verbose:
        print(stats.summary("stream_nf4"), flush=True)
    return stats
