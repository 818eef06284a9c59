"""Build a staged module straight from a safetensors checkpoint.

Mirrors the checkpoint half of ``stratum/upload.py`` (425-904, 1325-1440): the
name mapping from pipeline parameter names to checkpoint keys, fused MoE
expert reconstruction, the FP16 loader, the single-pass load-and-quantize
build and the populate-from-cache path. Names, arguments, return values and
the meaning of ``min_numel`` / ``cache_dir`` / ``blocksize`` are the reference's,
so ``stratum/model/registry.py`` calls them unchanged.

The difference is where the quantization runs: each NF4-eligible tensor is read
from the checkpoint (safetensors maps the file; one tensor in host memory at a
time), quantized by the HIP kernel on the current GPU and its payload copied
back to pinned host memory -- instead of bitsandbytes' CPU quantizer, the
build's only hot loop (a 4096 x 14336 fp16 weight: ~32 us of kernel time).
Checkpoint files are found with transformers' ``cached_file``, which resolves a
local directory without any network access.
"""

from __future__ import annotations

import json
import re
from pathlib import Path
from typing import Callable, Optional

import torch

from . import upload as U

__all__ = [
    "_build_ckpt_key_fn",
    "_try_load_fused_experts",
    "load_module_fp16_from_checkpoint",
    "stream_load_and_quantize_module",
    "populate_from_hf_checkpoint",
]

_LAYER_WRAPPER = re.compile(r"\.layer\.(?!layer)")


def _build_ckpt_key_fn(module: torch.nn.Module) -> Callable[[str], list]:
    """``ckpt_keys(pname) -> [candidate checkpoint keys]`` for parameters of *module*
    (``stratum/upload.py:425-473``).

    A pipeline name may carry wrappers the checkpoint does not know: Stratum's
    ``.layer.`` (a decoder layer wrapped with its index), PEFT's
    ``.base_layer.``, ``.inner.``, and a missing ``model.`` prefix; tied
    ``lm_head.weight`` also maps to the embedding. Candidates are tried in order.
    """
    layer_prefixes = []
    for mod_name, sub in module.named_modules():
        idx = getattr(sub, "idx", None)
        if isinstance(idx, int) and hasattr(sub, "layer"):
            layer_prefixes.append((f"{mod_name}.layer." if mod_name else "layer.", f"model.layers.{idx}."))

    def no_base(name: str) -> str:
        return name.replace(".base_layer.", ".")

    def ckpt_keys(pname: str) -> list:
        pname = U._canonical_param_name(pname)
        out = []

        def add(name: str) -> None:
            variants = [name]
            if ".inner." in name:
                variants.append(name.replace(".inner.", "."))
            for v in variants:
                stripped = _LAYER_WRAPPER.sub(".", v)
                for cand in (v, stripped):
                    out.extend((cand, no_base(cand)))
                for cand in (v, stripped):
                    out.extend((f"model.{cand}", f"model.{no_base(cand)}"))

        add(pname)
        if pname == "lm_head.weight":
            add("model.embed_tokens.weight")
            add("embed_tokens.weight")
        for prefix, global_prefix in layer_prefixes:
            if pname.startswith(prefix):
                add(global_prefix + pname[len(prefix):])
        return list(dict.fromkeys(out))

    return ckpt_keys


_FUSED_SUFFIXES = (".feed_forward.experts.gate_up_proj", ".feed_forward.experts.down_proj")


def _try_load_fused_experts(handle, keys: set, pname: str, param: torch.nn.Parameter,
                            ckpt_key_fn) -> Optional[torch.Tensor]:
    """Stacked ``[E, ...]`` expert tensor from per-expert checkpoint keys
    (``stratum/upload.py:476-533``): ``gate_up_proj`` = cat(w1, w3) per expert,
    ``down_proj`` = w2 per expert. None when *pname* is not a fused expert
    parameter or the keys are absent."""
    pname = U._canonical_param_name(pname)
    suffix = next((s for s in _FUSED_SUFFIXES if pname.endswith(s)), None)
    if suffix is None or param.ndim != 3:
        return None
    n_exp = int(param.shape[0])
    for cand in ckpt_key_fn(pname):
        if not cand.endswith(suffix):
            continue
        base = cand[: -len(suffix)] + ".feed_forward.experts"
        if suffix.endswith("gate_up_proj"):
            need = [k for e in range(n_exp) for k in (f"{base}.{e}.w1.weight", f"{base}.{e}.w3.weight")]
            if not all(k in keys for k in need):
                continue
            return torch.stack([torch.cat([handle.get_tensor(f"{base}.{e}.w1.weight"),
                                           handle.get_tensor(f"{base}.{e}.w3.weight")], dim=0)
                                for e in range(n_exp)], dim=0)
        need = [f"{base}.{e}.w2.weight" for e in range(n_exp)]
        if not all(k in keys for k in need):
            continue
        return torch.stack([handle.get_tensor(k) for k in need], dim=0)
    return None


def _checkpoint_files(hf_model_name: str):
    """``("sharded", index_path)``, ``("single", file_path)`` or ``(None, None)``."""
    from transformers.utils.hub import cached_file

    def find(fname):
        try:
            p = cached_file(hf_model_name, fname, cache_dir=None)
        except (OSError, ValueError):
            return None
        return Path(p) if p is not None and Path(p).exists() else None

    idx = find("model.safetensors.index.json")
    if idx is not None:
        return "sharded", idx
    single = find("model.safetensors")
    if single is not None:
        return "single", single
    return None, None


def _set(param: torch.nn.Parameter, data: torch.Tensor, owner_map: dict) -> None:
    owner, pname = owner_map.get(id(param), (None, None))
    U._replace_param_data(param, data, owner=owner, pname=pname)


@torch.no_grad()
def load_module_fp16_from_checkpoint(module: torch.nn.Module, hf_model_name: str, *, verbose: bool = False) -> bool:
    """Fill the frozen meta-device parameters of *module* from the checkpoint,
    one tensor at a time (``stratum/upload.py:536-668``). True when every such
    parameter was found and set."""
    from safetensors import safe_open

    needed = [(n, p) for n, p in module.named_parameters() if p.device.type == "meta" and not p.requires_grad]
    if not needed:
        return True
    owner_map = U._build_param_owner_map(module)
    keys_of = _build_ckpt_key_fn(module)
    kind, path = _checkpoint_files(hf_model_name)
    if kind == "sharded":
        weight_map = json.loads(path.read_text())["weight_map"]
        per_shard: dict = {}
        for n, p in needed:
            ck = next((k for k in keys_of(n) if k in weight_map), None)
            if ck is None:
                if verbose:
                    print(f"  load_module: no checkpoint key for {n}", flush=True)
                return False
            per_shard.setdefault(weight_map[ck], []).append((ck, p))
        for shard, items in per_shard.items():
            sp = path.parent / shard
            if not sp.exists():
                return False
            with safe_open(str(sp), framework="pt") as f:
                for ck, p in items:
                    try:
                        _set(p, f.get_tensor(ck).to(device="cpu", dtype=p.dtype), owner_map)
                    except (RuntimeError, TypeError):
                        if verbose:
                            print(f"  load_module: can't set data for {ck}", flush=True)
                        return False
        return True
    if kind != "single":
        return False
    with safe_open(str(path), framework="pt") as f:
        keys = set(f.keys())
        for n, p in needed:
            ck = next((k for k in keys_of(n) if k in keys), None)
            t = f.get_tensor(ck) if ck is not None else _try_load_fused_experts(f, keys, n, p, keys_of)
            if t is None:
                if verbose:
                    print(f"  load_module: no checkpoint key for {n}", flush=True)
                return False
            try:
                _set(p, t.to(device="cpu", dtype=p.dtype), owner_map)
            except (RuntimeError, TypeError):
                if verbose:
                    print(f"  load_module: can't set data for {n}", flush=True)
                return False
    return True


@torch.no_grad()
def stream_load_and_quantize_module(module: torch.nn.Module, hf_model_name: str, *, min_numel: int = 4096,
                                    cache_dir: Optional[Path | str] = None, blocksize: int = 64,
                                    quant_type: str = "nf4", verbose: bool = False) -> Optional[U.NF4Stats]:
    """Load and NF4-quantize a meta-device module in one streaming pass
    (``stratum/upload.py:671-904``).

    Per frozen parameter: NF4-eligible with a cache hit -> attach the cached
    payload without reading the checkpoint; NF4-eligible without -> read the
    tensor, quantize it on the GPU, attach (and write the cache); otherwise ->
    read and keep it. Peak host memory is the payloads so far plus one tensor.
    Returns the stats, or None when a checkpoint key is missing.
    """
    from safetensors import safe_open

    cache_root = Path(cache_dir) if cache_dir else None
    owner_map = U._build_param_owner_map(module)
    keys_of = _build_ckpt_key_fn(module)

    def eligible(p: torch.nn.Parameter) -> bool:
        return p.ndim >= 2 and p.numel() >= min_numel and p.dtype in (torch.float16, torch.bfloat16, torch.float32)

    stats = U.NF4Stats()
    for _, p in module.named_parameters():  # payloads attached by an earlier pass count too
        if hasattr(p, U.NF4_ATTR):
            pl = getattr(p, U.NF4_ATTR)
            stats.tensors += 1
            stats.source_bytes += pl.source_bytes
            stats.payload_bytes += pl.payload_bytes
    needed = [(n, p) for n, p in module.named_parameters()
              if not p.requires_grad and not hasattr(p, U.NF4_ATTR)
              and (p.device.type == "meta" or p.data.numel() == 0)]
    if not needed:
        if verbose:
            print(f"  stream_nf4: {stats.tensors} tensors already processed", flush=True)
        return stats

    def from_cache(n: str, p: torch.nn.Parameter) -> bool:
        if cache_root is None:
            return False
        pl = U._load_payload_from_cache(U._cache_path(cache_root, n), p, blocksize=blocksize, quant_type=quant_type)
        if pl is None:
            return False
        setattr(p, U.NF4_ATTR, pl)
        _set(p, torch.empty(0, dtype=pl.dtype, device="cpu"), owner_map)
        stats.tensors += 1
        stats.source_bytes += pl.source_bytes
        stats.payload_bytes += pl.payload_bytes
        stats.cache_hits += 1
        return True

    def consume(n: str, p: torch.nn.Parameter, t: torch.Tensor) -> bool:
        if eligible(p):
            owner, pname = owner_map.get(id(p), (None, None))
            U.quantize_and_attach(n, p, t, stats, cache_dir=cache_root, blocksize=blocksize, quant_type=quant_type,
                                  owner=owner, pname=pname)
            return True
        try:
            _set(p, t, owner_map)
        except (RuntimeError, TypeError):
            if verbose:
                print(f"  stream_nf4: can't set data for {n}", flush=True)
            return False
        return True

    kind, path = _checkpoint_files(hf_model_name)
    if kind == "sharded":
        weight_map = json.loads(path.read_text())["weight_map"]
        todo = []
        for n, p in needed:  # phase 1: cache hits never touch the shards
            if eligible(p) and from_cache(n, p):
                continue
            ck = next((k for k in keys_of(n) if k in weight_map), None)
            if ck is None:
                if verbose:
                    print(f"  stream_nf4: no checkpoint key for {n}", flush=True)
                return None
            todo.append((n, p, ck))
        per_shard: dict = {}
        for item in todo:
            per_shard.setdefault(weight_map[item[2]], []).append(item)
        for shard, items in per_shard.items():  # phase 2: each shard opened once
            sp = path.parent / shard
            if not sp.exists():
                return None
            with safe_open(str(sp), framework="pt") as f:
                for n, p, ck in items:
                    if not consume(n, p, f.get_tensor(ck).to(device="cpu", dtype=p.dtype)):
                        return None
    elif kind == "single":
        with safe_open(str(path), framework="pt") as f:
            keys = set(f.keys())
            for n, p in needed:
                if eligible(p) and from_cache(n, p):
                    continue
                ck = next((k for k in keys_of(n) if k in keys), None)
                t = f.get_tensor(ck) if ck is not None else _try_load_fused_experts(f, keys, n, p, keys_of)
                if t is None:
                    if verbose:
                        print(f"  stream_nf4: no checkpoint key for {n}", flush=True)
                    return None
                if not consume(n, p, t.to(device="cpu", dtype=p.dtype)):
                    return None
    else:
        return None
    if verbose:
        print(f"  nf4 total: {stats.tensors} tensors, {stats.source_bytes / 1024**3:.2f} GiB -> "
              f"{stats.payload_bytes / 1024**3:.2f} GiB payload (cache hits={stats.cache_hits} "
              f"misses={stats.cache_misses} writes={stats.cache_writes})", flush=True)
    return stats


@torch.no_grad()
def populate_from_hf_checkpoint(model: torch.nn.Module, hf_model_name: str,
                                nf4_cache_dir: Optional[str | Path] = None, *, min_numel: int = 4096,
                                verbose: bool = True) -> bool:
    """Populate a meta-device model from the NF4 cache plus the checkpoint's
    small tensors (``stratum/upload.py:1325-1440``): NF4-eligible frozen
    parameters come from ``prepare_nf4_from_cache``; the rest of the frozen
    meta parameters (norms, biases) are read one tensor at a time under their
    own names. False when the cache misses or the checkpoint cannot be read.
    A meta parameter is replaced through its owner (``_replace_param_data``):
    assigning ``.data`` cannot move a meta tensor to the CPU."""
    from safetensors import safe_open

    owner_map = U._build_param_owner_map(model)
    small = {}
    for name, p in model.named_parameters():
        if p.requires_grad:
            continue
        if p.ndim >= 2 and p.numel() >= min_numel and p.dtype in (torch.float16, torch.bfloat16, torch.float32):
            continue
        if p.device.type != "meta":
            continue
        small[name] = p
    if nf4_cache_dir is not None:
        if U.prepare_nf4_from_cache(model, nf4_cache_dir, min_numel=min_numel, verbose=verbose) is None:
            if verbose:
                print("  populate: NF4 cache miss -- falling back to FP16 load", flush=True)
            return False
    if not small:
        return True
    if verbose:
        print(f"  populate: loading {len(small)} non-NF4 params from the checkpoint", flush=True)
    kind, path = _checkpoint_files(hf_model_name)
    if kind == "sharded":
        weight_map = json.loads(path.read_text())["weight_map"]
        per_shard: dict = {}
        for name in small:
            if name in weight_map:
                per_shard.setdefault(weight_map[name], []).append(name)
        for shard, names in per_shard.items():
            sp = path.parent / shard
            if not sp.exists():
                if verbose:
                    print(f"  populate: shard not found: {sp}", flush=True)
                return False
            with safe_open(str(sp), framework="pt") as f:
                for name in names:
                    _set(small[name], f.get_tensor(name).to("cpu"), owner_map)
        return True
    if kind == "single":
        with safe_open(str(path), framework="pt") as f:
            keys = set(f.keys())
            for name, p in small.items():
                if name not in keys:
                    if verbose:
                        print(f"  populate: key {name} not in checkpoint", flush=True)
                    return False
                _set(p, f.get_tensor(name).to("cpu"), owner_map)
        return True
    if verbose:
        print("  populate: no checkpoint files found", flush=True)
    return False
