"""NF4 weight staging: quantize frozen weights once, bring them to the GPU per step.

Host side of the NF4 frozen-weight path with the interface of the reference's
``stratum/upload.py`` (names, signatures, the ``NF4_ATTR`` / ``FP16_ATTR``
attributes, ``NF4Payload`` / ``FP16StagedPayload`` fields, the version-1 cache
files and the exception types), so ``DeviceStage`` / ``StratumPipeline`` /
``ModelArch.build`` call it unchanged. The arithmetic the reference delegates
to ``bitsandbytes.functional`` runs in the gfx950 HIP library
(``stratum_amd.functional``).

How this implementation is organised:

* A **staging plan** per module (``_plan``): every parameter and buffer slot of
  the module tree as (owner module, local name, qualified name), built once
  and cached. Slots are resolved through ``owner._parameters[name]`` on each
  call, so a parameter replaced by ``_replace_param_data`` (or by anyone) is
  seen; a structural change (a parameter or buffer added or removed, a child
  module added, removed or swapped) invalidates the plan. ``ensure_weights`` /
  ``free_weights`` / ``prefetch_weights`` therefore do not walk
  ``named_modules`` on every call.
* **One materialisation routine** (``_materialise``) for the three staged
  kinds: an NF4 payload is copied host-to-device (pinned memory, asynchronous)
  and dequantized by the GPU kernel; an FP16-staged payload is copied; a plain
  frozen parameter on the wrong device is moved. ``ensure_weights``,
  ``NF4Prefetch.finalize`` and ``upload_stream`` all go through it.
* **Consumer streams.** A tensor materialised on a side stream is read by
  other streams (the reference fences the default stream on an event,
  ``stratum/stage.py:99-121``). Every materialised tensor -- NF4 and FP16 --
  is ``record_stream``-ed on the consumer streams (by default the device's
  default stream), so the caching allocator cannot hand its block to the side
  stream again while queued consumer work still reads it (``free_weights``
  right after a layer's forward is then safe).
* Prefetch copies use one persistent copy stream per device; the ``code``
  table is not uploaded (the kernels carry the NF4 levels); cache files are
  read with ``torch.load(weights_only=True)``.
"""

from __future__ import annotations

import hashlib
import re
import time
import weakref
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, Iterator, Optional, Sequence

import torch

from .functional import DEFAULT_ROUNDING, QuantState, dequantize_4bit_many, get_4bit_type, quantize_4bit
from .utils import log_event

NF4_ATTR = "roundpipe_nf4_payload"
FP16_ATTR = "stratum_fp16_staged"

_STAGEABLE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


# ------------------------------------------------------------------ records
@dataclass
class NF4Stats:
    """Counters of one NF4 preparation pass (``stratum/upload.py:31-45``)."""
    tensors: int = 0
    source_bytes: int = 0
    payload_bytes: int = 0
    cache_hits: int = 0
    cache_misses: int = 0
    cache_writes: int = 0

    @property
    def compression(self) -> float:
        return self.source_bytes / self.payload_bytes if self.payload_bytes else 0.0

    def count(self, payload: "NF4Payload") -> None:
        self.tensors += 1
        self.source_bytes += payload.source_bytes
        self.payload_bytes += payload.payload_bytes

    def summary(self, what: str) -> str:
        return (f"  {what}: {self.tensors} tensors, {self.source_bytes / 2**30:.2f} GiB source -> "
                f"{self.payload_bytes / 2**30:.2f} GiB NF4 payload ({self.compression:.2f}x; "
                f"cache {self.cache_hits} hit / {self.cache_misses} miss / {self.cache_writes} written)")


@dataclass
class NF4Payload:
    """Packed NF4 weight kept in pinned host memory (``stratum/upload.py:70-95``).

    quantized: uint8 [(numel + 1) // 2, 1], two codes per byte (even element in the high nibble)
    absmax:    fp32 [ceil(numel / blocksize)]
    code:      fp32 [16], the NF4 levels
    shape:     original weight shape (3-D for stacked experts)
    dtype:     original weight dtype (the dequantize output dtype)
    """
    quantized: torch.Tensor
    absmax: torch.Tensor
    code: torch.Tensor
    shape: tuple
    dtype: torch.dtype
    blocksize: int
    quant_type: str
    source_numel: int
    source_bytes: int
    payload_bytes: int


@dataclass
class FP16StagedPayload:
    """Uncompressed frozen weight kept in pinned host memory (the ``--no-nf4`` path)."""
    data: torch.Tensor
    shape: tuple
    dtype: torch.dtype
    source_bytes: int


def _pin_cpu(t: torch.Tensor) -> torch.Tensor:
    """A page-locked host copy of *t* (so its host-to-device copy is asynchronous)."""
    host = t.detach().cpu().contiguous()
    if host.is_pinned():
        return host
    return host.pin_memory()


def _payload_bytes(*tensors: torch.Tensor) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).split(".", 1)[-1]


def _dtype_from_name(name: str) -> torch.dtype:
    dtype = getattr(torch, name.split(".", 1)[-1], None)
    if not isinstance(dtype, torch.dtype):
        raise ValueError(f"not a torch dtype: {name!r}")
    return dtype


def _eligible(param: torch.nn.Parameter, min_numel: int) -> bool:
    """A frozen floating-point weight of >= 2 dims and >= min_numel elements: the
    parameters both NF4 and FP16 staging take (``stratum/upload.py:111-160,305-398``)."""
    return (not param.requires_grad and param.ndim >= 2 and param.numel() >= min_numel
            and param.dtype in _STAGEABLE_DTYPES)


def _staged(param: torch.nn.Parameter):
    """The payload staged on *param* (NF4 first), or None."""
    payload = getattr(param, NF4_ATTR, None)
    return payload if payload is not None else getattr(param, FP16_ATTR, None)


# ----------------------------------------------------------- staging plan
class _Slot:
    """One named tensor slot of a module tree (the owner held weakly)."""
    __slots__ = ("_owner", "name", "qualname")

    def __init__(self, owner: torch.nn.Module, name: str, qualname: str):
        self._owner, self.name, self.qualname = weakref.ref(owner), name, qualname

    @property
    def owner(self) -> Optional[torch.nn.Module]:
        return self._owner()


class _StagePlan:
    """Parameter and buffer slots of a module tree, with a structural fingerprint:
    per owner, its parameter and buffer counts and the identity of its children
    (a child swapped for another module changes it). Owners are held weakly, so
    a cached plan never keeps a module alive."""

    def __init__(self, module: torch.nn.Module):
        owners = []
        self.params: list = []
        self.buffers: list = []
        for prefix, owner in module.named_modules(remove_duplicate=False):
            owners.append(owner)
            dot = prefix + "." if prefix else ""
            self.params += [_Slot(owner, n, dot + n) for n in owner._parameters]
            self.buffers += [_Slot(owner, n, dot + n) for n in owner._buffers]
        self.owners = [weakref.ref(o) for o in owners]
        self.fingerprint = self._fingerprint(owners)

    @staticmethod
    def _fingerprint(owners: list) -> tuple:
        return tuple((len(o._parameters), len(o._buffers), tuple(map(id, o._modules.values()))) for o in owners)

    def valid(self) -> bool:
        owners = [r() for r in self.owners]
        return all(o is not None for o in owners) and self._fingerprint(owners) == self.fingerprint

    def unique_params(self) -> Iterator:
        """(slot, parameter) of every distinct parameter, first slot wins (the
        order and de-duplication of ``named_parameters``)."""
        seen: set = set()
        for slot in self.params:
            p = slot.owner._parameters.get(slot.name)
            if p is None or id(p) in seen:
                continue
            seen.add(id(p))
            yield slot, p

    def unique_buffers(self) -> Iterator:
        seen: set = set()
        for slot in self.buffers:
            b = slot.owner._buffers.get(slot.name)
            if b is None or id(b) in seen:
                continue
            seen.add(id(b))
            yield slot, b


_plans: "weakref.WeakKeyDictionary[torch.nn.Module, _StagePlan]" = weakref.WeakKeyDictionary()


def _plan(module: torch.nn.Module) -> _StagePlan:
    """The cached staging plan of *module*, rebuilt when its structure changed."""
    plan = _plans.get(module)
    if plan is None or not plan.valid():
        plan = _StagePlan(module)
        _plans[module] = plan
    return plan


def _replace_param_data(param: torch.nn.Parameter, new_data: torch.Tensor, owner: Optional[torch.nn.Module] = None,
                        pname: Optional[str] = None) -> None:
    """Point *param* at *new_data*. Some Parameter subclasses refuse a ``.data``
    assignment; then a plain Parameter holding *new_data* (same ``requires_grad``,
    staged payloads carried over) is registered on *owner* under *pname* instead
    (``stratum/upload.py:1286-1310``). Without an owner the refusal is ignored."""
    try:
        param.data = new_data
        return
    except (RuntimeError, TypeError):
        if owner is None or pname is None:
            return
    replacement = torch.nn.Parameter(new_data, requires_grad=param.requires_grad)
    for attr in (NF4_ATTR, FP16_ATTR):
        payload = getattr(param, attr, None)
        if payload is not None:
            setattr(replacement, attr, payload)
    owner.register_parameter(pname, replacement)


def _build_param_owner_map(module: torch.nn.Module) -> dict:
    """id(param) -> (owner module, local name), from the cached plan."""
    return {id(p): (slot.owner, slot.name) for slot, p in _plan(module).unique_params()}


# ----------------------------------------------------------- cache (v1)
def _canonical_param_name(name: str) -> str:
    """Cache name of a parameter: wrapper ``.module.`` segments removed."""
    return name.replace(".module.", ".")


def _cache_path(cache_dir: Path, name: str) -> Path:
    """``<sha1(name)[:12]>-<name with unsafe characters as _, last 160>.pt``
    (the reference's file naming, ``stratum/upload.py:236-240``)."""
    canon = _canonical_param_name(name)
    tag = hashlib.sha1(canon.encode("utf-8")).hexdigest()[:12]
    return Path(cache_dir) / f"{tag}-{re.sub(r'[^A-Za-z0-9_.-]+', '_', canon)[-160:]}.pt"


def _cache_meta(shape: Sequence[int], dtype: torch.dtype, numel: int, nbytes: int, blocksize: int,
                quant_type: str) -> dict:
    """The metadata keys of a version-1 cache file (what a load must match)."""
    return {"version": 1, "shape": tuple(int(s) for s in shape), "dtype": _dtype_name(dtype),
            "blocksize": int(blocksize), "quant_type": str(quant_type), "source_numel": int(numel),
            "source_bytes": int(nbytes)}


def _load_payload_from_cache(path: Path, param: torch.nn.Parameter, *, blocksize: int,
                             quant_type: str) -> Optional[NF4Payload]:
    """A version-1 cache file whose metadata matches *param* exactly; None for a
    missing, unreadable or mismatched file (the caller re-quantizes)."""
    path = Path(path)
    if not path.is_file():
        return None
    want = _cache_meta(param.shape, param.dtype, param.numel(), param.numel() * param.element_size(), blocksize,
                       quant_type)
    try:
        obj = torch.load(path, map_location="cpu", weights_only=True)
        if not isinstance(obj, dict) or any(obj.get(k) != v for k, v in want.items()):
            return None
        tensors = [obj[k] for k in ("quantized", "absmax", "code")]
    except Exception:
        return None
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        return None
    quantized, absmax, code = (_pin_cpu(t) for t in tensors)
    return NF4Payload(quantized=quantized, absmax=absmax, code=code, shape=want["shape"], dtype=param.dtype,
                      blocksize=want["blocksize"], quant_type=want["quant_type"], source_numel=want["source_numel"],
                      source_bytes=want["source_bytes"], payload_bytes=_payload_bytes(*tensors))


def _save_payload_to_cache(path: Path, payload: NF4Payload) -> None:
    """Write a version-1 cache file atomically (``<name>.tmp`` then rename)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    record = _cache_meta(payload.shape, payload.dtype, payload.source_numel, payload.source_bytes,
                         payload.blocksize, payload.quant_type)
    for key in ("quantized", "absmax", "code"):
        record[key] = getattr(payload, key).detach().cpu().contiguous()
    tmp = path.with_name(path.name + ".tmp")
    torch.save(record, tmp)
    tmp.replace(path)


# ------------------------------------------------------------ preparation
def _make_payload(data: torch.Tensor, param: torch.nn.Parameter, *, blocksize: int, quant_type: str,
                  rounding: str) -> NF4Payload:
    """Quantize *data* (the weight of *param*) on the GPU into a pinned payload.
    Stacked expert weights [E, A, B] are quantized as their [-1, B] view and
    keep the original shape in the payload."""
    weight = data.detach()
    if weight.ndim > 2:
        weight = weight.reshape(-1, weight.shape[-1])
    packed, state = quantize_4bit(weight.contiguous(), blocksize=blocksize, compress_statistics=False,
                                  quant_type=quant_type, rounding=rounding)
    return NF4Payload(quantized=_pin_cpu(packed), absmax=_pin_cpu(state.absmax), code=_pin_cpu(state.code),
                      shape=tuple(data.shape), dtype=state.dtype, blocksize=int(state.blocksize),
                      quant_type=str(state.quant_type), source_numel=param.numel(),
                      source_bytes=param.numel() * param.element_size(),
                      payload_bytes=_payload_bytes(packed, state.absmax, state.code))


def _attach(param: torch.nn.Parameter, attr: str, payload, owner=None, pname=None) -> None:
    """Stage *payload* on *param* and drop its data (an empty tensor on the CPU
    when the parameter lived on the meta device)."""
    setattr(param, attr, payload)
    home = torch.device("cpu") if param.device.type == "meta" else param.device
    _replace_param_data(param, torch.empty(0, dtype=param.dtype, device=home), owner=owner, pname=pname)


@torch.no_grad()
def prepare_fp16_staged(module: torch.nn.Module, *, min_numel: int = 4096, verbose: bool = True) -> int:
    """Move every eligible frozen weight to pinned host memory for an uncompressed
    per-step upload (``stratum/upload.py:111-160``); returns how many were staged."""
    staged = 0
    for slot, p in _plan(module).unique_params():
        if not _eligible(p, min_numel) or _staged(p) is not None:
            continue
        payload = FP16StagedPayload(data=_pin_cpu(p.data), shape=tuple(p.shape), dtype=p.dtype,
                                    source_bytes=p.numel() * p.element_size())
        _attach(p, FP16_ATTR, payload, slot.owner, slot.name)
        staged += 1
    if verbose:
        total = sum(getattr(p, FP16_ATTR).source_bytes for _, p in _plan(module).unique_params()
                    if hasattr(p, FP16_ATTR))
        print(f"  fp16 staged: {staged} new tensors, {total / 2**30:.2f} GiB uploaded per step", flush=True)
    return staged


@torch.no_grad()
def prepare_nf4(module: torch.nn.Module, *, min_numel: int = 4096, cache_dir: Optional[Path | str] = None,
                verbose: bool = True, blocksize: int = 64, quant_type: str = "nf4",
                rounding: str = DEFAULT_ROUNDING) -> NF4Stats:
    """Quantize every eligible frozen weight to NF4 (GPU kernel), keep the payload in
    pinned host memory and empty the parameter (``stratum/upload.py:305-398``).
    A parameter that already carries a payload is counted, not re-quantized; with
    *cache_dir*, matching version-1 cache files are used and misses are written."""
    stats = NF4Stats()
    for slot, p in _plan(module).unique_params():
        if not _eligible(p, min_numel):
            continue
        payload = getattr(p, NF4_ATTR, None)
        if payload is None:
            path = _cache_path(Path(cache_dir), slot.qualname) if cache_dir else None
            payload = _load_payload_from_cache(path, p, blocksize=blocksize, quant_type=quant_type) if path else None
            if payload is not None:
                stats.cache_hits += 1
            else:
                payload = _make_payload(p.data, p, blocksize=blocksize, quant_type=quant_type, rounding=rounding)
                if path is not None:
                    stats.cache_misses += 1
                    _save_payload_to_cache(path, payload)
                    stats.cache_writes += 1
            _attach(p, NF4_ATTR, payload, slot.owner, slot.name)
        stats.count(payload)
    if verbose:
        print(stats.summary("nf4 prepared"), flush=True)
    return stats


@torch.no_grad()
def prepare_nf4_from_cache(module: torch.nn.Module, cache_dir: str | Path | None, *, min_numel: int = 4096,
                           blocksize: int = 64, quant_type: str = "nf4", verbose: bool = True) -> Optional[NF4Stats]:
    """Attach cached payloads to every eligible parameter (meta parameters too)
    without reading any weight; None as soon as one file is missing or stale, so
    the caller can fall back to a full load (``stratum/upload.py:1207-1283``)."""
    if cache_dir is None:
        return None
    stats = NF4Stats()
    pending = []
    for slot, p in _plan(module).unique_params():
        if not _eligible(p, min_numel):
            continue
        payload = getattr(p, NF4_ATTR, None)
        if payload is None:
            payload = _load_payload_from_cache(_cache_path(Path(cache_dir), slot.qualname), p, blocksize=blocksize,
                                               quant_type=quant_type)
            if payload is None:
                if verbose:
                    print(f"  nf4 cache: no usable file for {slot.qualname}", flush=True)
                return None
            stats.cache_hits += 1
            pending.append((slot, p, payload))
        stats.count(payload)
    for slot, p, payload in pending:  # attach only once every file was found
        _attach(p, NF4_ATTR, payload, slot.owner, slot.name)
    if verbose:
        print(stats.summary("nf4 from cache"), flush=True)
    return stats


@torch.no_grad()
def quantize_and_attach(name: str, param: torch.nn.Parameter, data: torch.Tensor, stats: NF4Stats, *,
                        cache_dir: Optional[Path | str] = None, blocksize: int = 64, quant_type: str = "nf4",
                        owner: Optional[torch.nn.Module] = None, pname: Optional[str] = None,
                        rounding: str = DEFAULT_ROUNDING) -> NF4Payload:
    """Quantize one freshly loaded tensor for *param* and stage it (the per-tensor
    step of a streaming build, ``stratum/upload.py:718-754``)."""
    payload = _make_payload(data, param, blocksize=blocksize, quant_type=quant_type, rounding=rounding)
    if cache_dir:
        stats.cache_misses += 1
        _save_payload_to_cache(_cache_path(Path(cache_dir), name), payload)
        stats.cache_writes += 1
    _attach(param, NF4_ATTR, payload, owner, pname)
    stats.count(payload)
    return payload


@torch.no_grad()
def estimate_module_upload_gib(module: torch.nn.Module) -> float:
    """Device footprint of *module* (GB, 10^9) with staged weights at their
    materialised size; a shared parameter counts once."""
    total = 0
    for _, p in _plan(module).unique_params():
        payload = _staged(p)
        total += payload.source_bytes if payload is not None else p.numel() * p.element_size()
        if p.grad is not None:
            total += p.grad.numel() * p.grad.element_size()
    total += sum(b.numel() * b.element_size() for _, b in _plan(module).unique_buffers())
    return total / 1e9


# -------------------------------------------------------- materialisation
def _cuda(device_id) -> torch.device:
    dev = torch.device("cuda", device_id) if isinstance(device_id, int) else torch.device(device_id)
    if dev.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(f"no GPU available to materialise staged weights on {dev}")
    return dev


def _consumers(device: torch.device, consumers: Optional[Iterable]) -> list:
    """Streams that will read tensors materialised now: the given ones, else the
    device's default stream; the current stream itself needs no record."""
    current = torch.cuda.current_stream(device)
    wanted = list(consumers) if consumers is not None else [torch.cuda.default_stream(device)]
    return [s for s in wanted if s != current]


def _hand_over(t: torch.Tensor, consumers: list) -> torch.Tensor:
    for s in consumers:
        t.record_stream(s)
    return t


def _upload_nf4(payload: NF4Payload, device: torch.device):
    """Packed codes and absmax of *payload* on *device* (asynchronous from pinned
    memory, on the current stream)."""
    return (payload.quantized.to(device, non_blocking=True), payload.absmax.to(device, non_blocking=True))


def _materialise_nf4(entries: list, device: torch.device, consumers: list) -> int:
    """Bring NF4 parameters to *device* on the current stream: H2D of each packed
    payload (or its prefetched copy), then one batched dequantize per
    (blocksize, dtype) group -- a layer's projections in one launch.
    *entries*: (slot, param, payload, prefetched (q, absmax) or None)."""
    if not entries:
        return 0
    groups: dict = {}
    with torch.cuda.device(device):
        for slot, p, payload, prefetched in entries:
            q_dev, a_dev = prefetched if prefetched is not None else _upload_nf4(payload, device)
            state = QuantState(absmax=a_dev, shape=payload.shape, code=payload.code, blocksize=payload.blocksize,
                               quant_type=payload.quant_type, dtype=payload.dtype)
            groups.setdefault((payload.blocksize, payload.dtype), []).append((slot, p, q_dev, state))
        for members in groups.values():
            weights = dequantize_4bit_many([(q, st) for _, _, q, st in members])
            for (slot, p, _, _), w in zip(members, weights):
                _replace_param_data(p, _hand_over(w, consumers), owner=slot.owner, pname=slot.name)
    return len(entries)


def _needs(p: torch.nn.Parameter, device: torch.device) -> bool:
    """A staged parameter has to be (re)materialised on *device*: it is empty, or
    materialised on another device (a weight shared by stages on two GPUs)."""
    return p.data.numel() == 0 or p.data.device != device


def _materialise(slot: _Slot, p: torch.nn.Parameter, device: torch.device, consumers: list) -> int:
    """Bring one non-NF4 parameter to *device* on the current stream; returns 1
    if a tensor was placed. FP16-staged: H2D copy; other frozen parameters are
    moved, trainable ones on another device are an error (Stratum never moves
    them). NF4 parameters go through ``_materialise_nf4``."""
    fp16 = getattr(p, FP16_ATTR, None)
    if fp16 is None:
        if p.data.numel() == 0 or p.data.device == device:
            return 0
        if p.requires_grad:
            raise RuntimeError(f"parameter {slot.qualname!r} is trainable and lives on {p.data.device}; "
                               f"a stage on {device} cannot take it over")
        p.data = p.data.to(device, non_blocking=True)
        return 1
    if not _needs(p, device):
        return 0
    w = torch.empty(fp16.shape, dtype=fp16.dtype, device=device)
    w.copy_(fp16.data, non_blocking=True)
    _replace_param_data(p, _hand_over(w, consumers), owner=slot.owner, pname=slot.name)
    return 1


def _materialise_buffers(plan: _StagePlan, device: torch.device) -> int:
    """Move buffers to *device*; a meta buffer becomes an (uninitialised) tensor
    allocated there directly, registered on its owner when ``.data`` is refused."""
    moved = 0
    for slot, b in plan.unique_buffers():
        if b.device == device:
            continue
        if b.device.type == "meta":
            fresh = torch.empty(b.shape, dtype=b.dtype, device=device)
            try:
                b.data = fresh
            except (RuntimeError, TypeError):
                persistent = slot.name not in slot.owner._non_persistent_buffers_set
                slot.owner.register_buffer(slot.name, fresh, persistent=persistent)
        else:
            b.data = b.data.to(device, non_blocking=True)
        moved += 1
    return moved


@torch.no_grad()
def ensure_weights(module: torch.nn.Module, device_id: int, *, consumers: Optional[Sequence] = None) -> int:
    """Materialise every staged parameter and every buffer of *module* on
    ``cuda:<device_id>`` (``stratum/upload.py:969-1069``); the opposite of
    ``free_weights``. GPU work is queued on the current stream; the tensors are
    handed over to *consumers* (default: the device's default stream, the
    stream the reference fences on the upload). Returns the number of tensors
    placed."""
    device = _cuda(device_id)
    plan = _plan(module)
    readers = _consumers(device, consumers)
    placed, nf4 = 0, []
    for slot, p in plan.unique_params():
        payload = getattr(p, NF4_ATTR, None)
        if payload is not None:
            if _needs(p, device):
                nf4.append((slot, p, payload, None))
        else:
            placed += _materialise(slot, p, device, readers)
    placed += _materialise_nf4(nf4, device, readers)
    return placed + _materialise_buffers(plan, device)


@torch.no_grad()
def free_weights(module: torch.nn.Module) -> int:
    """Drop the device data of every staged parameter of *module* (the payloads
    stay); returns how many were dropped (``stratum/upload.py:1144-1159``)."""
    dropped = 0
    for _, p in _plan(module).unique_params():
        if p.data.numel() and _staged(p) is not None:
            p.data = torch.empty(0, dtype=p.dtype, device=p.device)
            dropped += 1
    return dropped


@torch.no_grad()
def upload_stream(module: torch.nn.Module, device_id: int, *, verbose: bool = True) -> int:
    """Materialise *module* on ``cuda:<device_id>`` once and wait for it: staged
    weights through ``ensure_weights``' path, everything else moved
    (``stratum/upload.py:907-966``)."""
    t0 = time.time()
    device = _cuda(device_id)
    placed = ensure_weights(module, device_id)
    torch.cuda.current_stream(device).synchronize()
    seconds = time.time() - t0
    log_event("upload_stream", device=device_id, tensors=placed, seconds=round(seconds, 1))
    if verbose:
        print(f"  device {device_id}: {placed} tensors in {seconds:.1f}s", flush=True)
    return placed


# ----------------------------------------------------------------- prefetch
_copy_streams: dict = {}


def _copy_stream(device: torch.device) -> "torch.cuda.Stream":
    """The persistent host-to-device copy stream of *device* (default priority)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _copy_streams.get(index)
    if stream is None:
        stream = _copy_streams[index] = torch.cuda.Stream(device=index)
    return stream


@dataclass
class _PrefetchEntry:
    slot: _Slot
    param: torch.nn.Parameter
    payload: NF4Payload
    quantized: torch.Tensor  # device copy (copy stream)
    absmax: torch.Tensor


@dataclass
class NF4Prefetch:
    """Packed payloads of one module in flight to a device (``stratum/upload.py:174-228``).

    ``finalize()`` (alias ``wait()``) makes the current stream wait for the
    copies and dequantizes them into the parameters; an empty prefetch is a
    no-op that needs no GPU.
    """
    entries: list
    device: torch.device
    stream: Optional["torch.cuda.Stream"] = None
    event: Optional["torch.cuda.Event"] = None

    @torch.no_grad()
    def finalize(self, *, consumers: Optional[Sequence] = None) -> int:
        if not self.entries:
            return 0
        device = _cuda(self.device)
        current = torch.cuda.current_stream(device)
        if self.event is not None:
            current.wait_event(self.event)
        readers = _consumers(device, consumers)
        todo = []
        for e in self.entries:
            if not _needs(e.param, device):
                continue  # materialised meanwhile (e.g. by an ensure_weights)
            e.quantized.record_stream(current)  # allocated on the copy stream, read here
            e.absmax.record_stream(current)
            todo.append((e.slot, e.param, e.payload, (e.quantized, e.absmax)))
        self.entries = []
        return _materialise_nf4(todo, device, readers)

    def wait(self) -> int:
        return self.finalize()


@torch.no_grad()
def prefetch_weights(module: torch.nn.Module, device_id: int) -> NF4Prefetch:
    """Start the host-to-device copies of the packed payloads of *module*'s NF4
    parameters that are not materialised on ``cuda:<device_id>``, on the device's
    copy stream; parameters are not touched until ``finalize()``
    (``stratum/upload.py:1072-1125``)."""
    device = torch.device("cuda", device_id)
    todo = [(slot, p, getattr(p, NF4_ATTR)) for slot, p in _plan(module).unique_params()
            if hasattr(p, NF4_ATTR) and _needs(p, device)]
    if not todo:
        return NF4Prefetch([], device)
    device = _cuda(device)
    stream = _copy_stream(device)
    with torch.cuda.device(device), torch.cuda.stream(stream):
        entries = [_PrefetchEntry(slot, p, payload, *_upload_nf4(payload, device)) for slot, p, payload in todo]
        done = torch.cuda.Event()
        done.record(stream)
    return NF4Prefetch(entries, device=device, stream=stream, event=done)


@torch.no_grad()
def ensure_prefetched_weights(module: torch.nn.Module, device_id: int, prefetch: Optional[NF4Prefetch]) -> int:
    """Finalize *prefetch* (it must target ``cuda:<device_id>``), then run
    ``ensure_weights`` for what a prefetch does not carry (FP16-staged and plain
    parameters, buffers)."""
    if prefetch is None:
        return ensure_weights(module, device_id)
    if prefetch.device != torch.device("cuda", device_id):
        raise ValueError(f"prefetch targets {prefetch.device}, not cuda:{device_id}")
    return prefetch.finalize() + ensure_weights(module, device_id)


# ------------------------------------------------------- buffer snapshots
@torch.no_grad()
def snapshot_module_buffers(module: torch.nn.Module) -> dict:
    """Host clones of the non-empty buffers of *module*, by qualified name (taken
    before a forward whose recompute must see the same buffer state)."""
    return {name: b.detach().to("cpu", copy=True) for name, b in module.named_buffers() if b.numel()}


@torch.no_grad()
def restore_module_buffers(module: torch.nn.Module, snapshot: dict) -> int:
    """Copy a snapshot back into *module*'s buffers; returns how many were restored."""
    if not snapshot:
        return 0
    current = dict(module.named_buffers())
    restored = 0
    for name, saved in snapshot.items():
        b = current.get(name)
        if b is not None:
            b.copy_(saved.to(b.device))
            restored += 1
    return restored


def nf4_code_table(device=None) -> torch.Tensor:
    """The fp32 [16] NF4 level table kept in ``NF4Payload.code``."""
    return get_4bit_type("nf4", device=device)


# The checkpoint build (stream_load_and_quantize_module) lives in .checkpoint;
# imported last because it uses this module's helpers.
from .checkpoint import stream_load_and_quantize_module  # noqa: E402
