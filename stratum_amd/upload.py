"""NF4 weight staging: quantize frozen weights once, stream them to the GPU per step.

Host-side mirror of the reference's L3 module ``stratum/upload.py`` for the NF4
frozen-weight path, with the same names, signatures, attribute names, payload
fields, cache format (version 1) and error behaviour, so ``DeviceStage`` /
``StratumPipeline`` / ``ModelArch.build`` can call it unchanged. The arithmetic
that the reference delegates to ``bitsandbytes.functional`` runs in the gfx950
HIP library (``stratum_amd.functional``):

  prepare_nf4 / quantize_and_attach -> quantize_4bit on the GPU (payload returned to pinned host memory)
  ensure_weights / NF4Prefetch      -> async H2D of the packed payload + dequantize_4bit kernel

Differences from the reference, all on the device side of the same contract:
  * the 16-entry ``code`` table is not uploaded (the kernels carry the NF4 levels);
  * a dequantized weight produced on a side stream is ``record_stream``-ed on the
    device's default stream, the stream that consumes it (``stratum/stage.py:120-121``),
    so the caching allocator cannot hand its block to the side stream again while
    the compute that reads it is still queued;
  * prefetches reuse one copy stream per device instead of a new stream per call;
  * cache files are read with ``torch.load(weights_only=True)``.
"""

from __future__ import annotations

import hashlib
import re
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, cast

import torch

from .functional import DEFAULT_ROUNDING, QuantState, dequantize_4bit, get_4bit_type, quantize_4bit
from .layer_transfer import DEFAULT_CHUNK_UPLOAD_BYTES, copy_tensor_chunked
from .utils import log_event

NF4_ATTR = "roundpipe_nf4_payload"
FP16_ATTR = "stratum_fp16_staged"


@dataclass
class NF4Stats:
    """NF4 preparation statistics (``stratum/upload.py:31-45``)."""
    tensors: int = 0
    source_bytes: int = 0
    payload_bytes: int = 0
    cache_hits: int = 0
    cache_misses: int = 0
    cache_writes: int = 0

    @property
    def compression(self) -> float:
        if self.payload_bytes == 0:
            return 0.0
        return self.source_bytes / self.payload_bytes


def _pin_cpu(t: torch.Tensor) -> torch.Tensor:
    """Copy *t* to page-locked host memory (fast, asynchronous H2D)."""
    t = t.detach().contiguous().cpu()
    if t.is_pinned():
        return t
    pinned = torch.empty_like(t, device=torch.device("cpu"), pin_memory=True)
    pinned.copy_(t)
    return pinned


def _payload_bytes(*tensors: torch.Tensor) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix("torch.")


def _dtype_from_name(name: str) -> torch.dtype:
    return cast(torch.dtype, getattr(torch, name.removeprefix("torch.")))


@dataclass
class NF4Payload:
    """NF4 weight payload kept in pinned host memory between steps (``stratum/upload.py:70-95``).

    quantized: uint8 [(numel + 1) // 2, 1], two codes per byte (even element high nibble)
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
    """Uncompressed frozen weight kept in pinned host memory (``--no-nf4`` path)."""
    data: torch.Tensor
    shape: tuple
    dtype: torch.dtype
    source_bytes: int


@torch.no_grad()
def prepare_fp16_staged(module: torch.nn.Module, *, min_numel: int = 4096, verbose: bool = True) -> int:
    """Pin frozen >=2-D params for per-step uncompressed upload (``stratum/upload.py:111-160``)."""
    count = 0
    for name, param in module.named_parameters():
        if param.requires_grad:
            continue
        if param.numel() < min_numel:
            continue
        if param.ndim < 2:
            continue
        if hasattr(param, NF4_ATTR) or hasattr(param, FP16_ATTR):
            continue
        if param.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            continue
        payload = FP16StagedPayload(
            data=_pin_cpu(param.data),
            shape=tuple(param.shape),
            dtype=param.dtype,
            source_bytes=param.numel() * param.element_size(),
        )
        setattr(param, FP16_ATTR, payload)
        param.data = torch.empty(0, dtype=param.dtype, device=param.device)
        count += 1
    if verbose:
        total = sum(getattr(p, FP16_ATTR).source_bytes for p in module.parameters() if hasattr(p, FP16_ATTR))
        print(f"  fp16 staged: {count} tensors, {total / 1024**3:.2f} GiB to upload per step", flush=True)
    return count


@dataclass
class _PrefetchEntry:
    param: torch.nn.Parameter
    payload: NF4Payload
    quantized: torch.Tensor
    absmax: torch.Tensor
    code: torch.Tensor
    owner: Optional[torch.nn.Module] = None
    pname: Optional[str] = None


@dataclass
class NF4Prefetch:
    """Pending asynchronous payload upload for one module (``stratum/upload.py:174-228``).

    ``finalize()`` makes the current stream wait for the copy stream and
    dequantizes the prefetched payloads into the parameters' data.
    """
    entries: list
    device: torch.device
    stream: Optional["torch.cuda.Stream"] = None
    event: Optional["torch.cuda.Event"] = None

    def finalize(self) -> int:
        if not self.entries:
            return 0
        if self.device.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError(f"CUDA is not available for NF4 prefetch finalize on {self.device}")
        current = torch.cuda.current_stream(device=self.device)
        if self.event is not None:
            current.wait_event(self.event)
        tensors = 0
        with torch.cuda.device(self.device), torch.cuda.stream(current), torch.no_grad():
            for entry in self.entries:
                if entry.param.data.numel() > 0:
                    if entry.param.data.device == self.device:
                        continue
                    _replace_param_data(entry.param,
                                        torch.empty(0, dtype=entry.param.dtype, device=entry.param.device),
                                        owner=entry.owner, pname=entry.pname)
                # the uploads were made on the copy stream and are read here
                if self.stream is not None:
                    entry.quantized.record_stream(current)
                    entry.absmax.record_stream(current)
                _replace_param_data(entry.param, _dequantize_payload(entry.payload, entry.quantized, entry.absmax),
                                    owner=entry.owner, pname=entry.pname)
                tensors += 1
        return tensors

    def wait(self) -> int:
        return self.finalize()


def _dequantize_payload(payload: NF4Payload, q_dev: torch.Tensor, absmax_dev: torch.Tensor) -> torch.Tensor:
    state = QuantState(absmax=absmax_dev, shape=payload.shape, code=payload.code, blocksize=payload.blocksize,
                       quant_type=payload.quant_type, dtype=payload.dtype)
    out = dequantize_4bit(q_dev, state).contiguous()
    dev = out.device
    current = torch.cuda.current_stream(dev)
    default = torch.cuda.default_stream(dev)
    if current != default:
        out.record_stream(default)
    return out


def _canonical_param_name(name: str) -> str:
    """Checkpoint/cache name of a parameter inside transparent wrappers."""
    return name.replace(".module.", ".")


def _cache_path(cache_dir: Path, name: str) -> Path:
    """``<sha1(name)[:12]>-<sanitised name[-160:]>.pt`` (``stratum/upload.py:236-240``)."""
    name = _canonical_param_name(name)
    safe = re.sub(r"[^A-Za-z0-9_.-]+", "_", name)[-160:]
    digest = hashlib.sha1(name.encode("utf-8")).hexdigest()[:12]
    return cache_dir / f"{digest}-{safe}.pt"


def _load_payload_from_cache(path: Path, param: torch.nn.Parameter, *, blocksize: int,
                             quant_type: str) -> Optional[NF4Payload]:
    """Read a version-1 cache file; any mismatch or unreadable file returns None."""
    if not path.exists():
        return None
    try:
        obj = torch.load(path, map_location="cpu", weights_only=True)
    except Exception:
        return None
    if not isinstance(obj, dict):
        return None
    expected = {
        "version": 1,
        "shape": tuple(param.shape),
        "dtype": _dtype_name(param.dtype),
        "blocksize": int(blocksize),
        "quant_type": str(quant_type),
        "source_numel": int(param.numel()),
        "source_bytes": int(param.numel() * param.element_size()),
    }
    for key, value in expected.items():
        if obj.get(key) != value:
            return None
    try:
        quantized = cast(torch.Tensor, obj["quantized"])
        absmax = cast(torch.Tensor, obj["absmax"])
        code = cast(torch.Tensor, obj["code"])
    except KeyError:
        return None
    return NF4Payload(
        quantized=_pin_cpu(quantized),
        absmax=_pin_cpu(absmax),
        code=_pin_cpu(code),
        shape=tuple(obj["shape"]),
        dtype=_dtype_from_name(str(obj["dtype"])),
        blocksize=int(obj["blocksize"]),
        quant_type=str(obj["quant_type"]),
        source_numel=int(obj["source_numel"]),
        source_bytes=int(obj["source_bytes"]),
        payload_bytes=_payload_bytes(quantized, absmax, code),
    )


def _save_payload_to_cache(path: Path, payload: NF4Payload) -> None:
    """Atomic write (``.tmp`` + replace) of a version-1 cache file."""
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(f"{path.name}.tmp")
    torch.save({
        "version": 1,
        "shape": tuple(payload.shape),
        "dtype": _dtype_name(payload.dtype),
        "blocksize": int(payload.blocksize),
        "quant_type": str(payload.quant_type),
        "source_numel": int(payload.source_numel),
        "source_bytes": int(payload.source_bytes),
        "quantized": payload.quantized.detach().contiguous().cpu(),
        "absmax": payload.absmax.detach().contiguous().cpu(),
        "code": payload.code.detach().contiguous().cpu(),
    }, tmp)
    tmp.replace(path)


def _nf4_eligible(param: torch.nn.Parameter, min_numel: int) -> bool:
    return (not param.requires_grad and param.ndim >= 2 and param.numel() >= min_numel
            and param.dtype in (torch.float16, torch.bfloat16, torch.float32))


def _make_payload(data: torch.Tensor, param: torch.nn.Parameter, *, blocksize: int, quant_type: str,
                  rounding: str) -> NF4Payload:
    orig_shape = tuple(data.shape)
    weight = data.detach().contiguous()
    # quantize_4bit takes a 2-D tensor; stacked expert weights [E, A, B] are
    # flattened to [-1, B] and restored from payload.shape at dequant time
    if weight.ndim > 2:
        weight = weight.reshape(-1, weight.shape[-1])
    quantized, q_state = quantize_4bit(weight, blocksize=blocksize, compress_statistics=False,
                                       quant_type=quant_type, rounding=rounding)
    return NF4Payload(
        quantized=_pin_cpu(quantized),
        absmax=_pin_cpu(q_state.absmax),
        code=_pin_cpu(q_state.code),
        shape=orig_shape,
        dtype=q_state.dtype,
        blocksize=int(q_state.blocksize),
        quant_type=str(q_state.quant_type),
        source_numel=int(param.numel()),
        source_bytes=int(param.numel() * param.element_size()),
        payload_bytes=_payload_bytes(quantized, q_state.absmax, q_state.code),
    )


@torch.no_grad()
def prepare_nf4(module: torch.nn.Module, *, min_numel: int = 4096, cache_dir: Optional[Path | str] = None,
                verbose: bool = True, blocksize: int = 64, quant_type: str = "nf4",
                rounding: str = DEFAULT_ROUNDING) -> NF4Stats:
    """Quantize frozen >=2-D weights to NF4, attach the payload, drop the originals
    (``stratum/upload.py:305-398``). The weight is quantized by the GPU kernel and
    the payload comes back to pinned host memory; ``param.data`` becomes empty.
    """
    stats = NF4Stats()
    for name, param in module.named_parameters():
        if param.requires_grad:
            continue
        if param.ndim < 2:
            continue
        if param.numel() < min_numel:
            continue
        if param.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            continue
        if hasattr(param, NF4_ATTR):
            payload = cast(NF4Payload, getattr(param, NF4_ATTR))
            stats.tensors += 1
            stats.source_bytes += payload.source_bytes
            stats.payload_bytes += payload.payload_bytes
            continue

        cache_path = _cache_path(Path(cache_dir), name) if cache_dir else None
        payload = (_load_payload_from_cache(cache_path, param, blocksize=blocksize, quant_type=quant_type)
                   if cache_path is not None else None)
        if payload is not None:
            stats.cache_hits += 1
        if payload is None:
            if cache_path is not None:
                stats.cache_misses += 1
            payload = _make_payload(param.data, param, blocksize=blocksize, quant_type=quant_type, rounding=rounding)
            if cache_path:
                _save_payload_to_cache(cache_path, payload)
                stats.cache_writes += 1

        setattr(param, NF4_ATTR, payload)
        param.data = torch.empty(0, dtype=payload.dtype, device=param.device)
        stats.tensors += 1
        stats.source_bytes += payload.source_bytes
        stats.payload_bytes += payload.payload_bytes

    if verbose:
        print(f"  nf4 total: {stats.tensors} tensors, "
              f"{stats.source_bytes / 1024**3:.2f} GiB -> {stats.payload_bytes / 1024**3:.2f} GiB payload "
              f"(compression {stats.compression:.2f}x, "
              f"cache hits={stats.cache_hits} misses={stats.cache_misses} writes={stats.cache_writes})",
              flush=True)
    return stats


@torch.no_grad()
def quantize_and_attach(name: str, param: torch.nn.Parameter, data: torch.Tensor, stats: NF4Stats, *,
                        cache_dir: Optional[Path | str] = None, blocksize: int = 64, quant_type: str = "nf4",
                        owner: Optional[torch.nn.Module] = None, pname: Optional[str] = None,
                        rounding: str = DEFAULT_ROUNDING) -> NF4Payload:
    """Quantize one freshly loaded tensor and attach it to *param* -- the per-tensor
    step of the streaming low-RSS build (``stratum/upload.py:718-754``)."""
    payload = _make_payload(data, param, blocksize=blocksize, quant_type=quant_type, rounding=rounding)
    if cache_dir:
        _save_payload_to_cache(_cache_path(Path(cache_dir), name), payload)
        stats.cache_writes += 1
        stats.cache_misses += 1
    setattr(param, NF4_ATTR, payload)
    _replace_param_data(param, torch.empty(0, dtype=payload.dtype, device="cpu"), owner=owner, pname=pname)
    stats.tensors += 1
    stats.source_bytes += payload.source_bytes
    stats.payload_bytes += payload.payload_bytes
    return payload


@torch.no_grad()
def estimate_module_upload_gib(module: torch.nn.Module) -> float:
    """GPU footprint of a module with NF4 params counted at their dequantized size."""
    total = 0
    seen: set = set()
    for param in module.parameters():
        if id(param) in seen:
            continue
        seen.add(id(param))
        payload = getattr(param, NF4_ATTR, None)
        if payload is not None:
            total += payload.source_bytes
        else:
            total += param.numel() * param.element_size()
        if param.grad is not None:
            total += param.grad.numel() * param.grad.element_size()
    for buf in module.buffers():
        total += buf.numel() * buf.element_size()
    return total / 10**9


@torch.no_grad()
def upload_stream(module: torch.nn.Module, device_id: int, *, verbose: bool = True) -> int:
    """Upload every param/buffer of *module* once (synchronous copies); NF4 params
    are uploaded packed and dequantized on the GPU (``stratum/upload.py:907-966``)."""
    device = torch.device(f"cuda:{device_id}")
    tensors = 0
    t0 = time.time()
    for name, param in module.named_parameters():
        if param.data.device == device:
            continue
        payload = getattr(param, NF4_ATTR, None)
        if payload is not None:
            q_gpu = payload.quantized.to(device, non_blocking=False)
            a_gpu = payload.absmax.to(device, non_blocking=False)
            with torch.cuda.device(device):
                param.data = _dequantize_payload(payload, q_gpu, a_gpu)
            tensors += 1
            if verbose:
                mib = payload.quantized.numel() * payload.quantized.element_size() / 1024**2
                print(f"  stream {name}: nf4 {list(payload.shape)} -> {mib:.1f} MiB on GPU", flush=True)
        else:
            param.data = param.data.to(device, non_blocking=False)
            tensors += 1
    for buf in module.buffers():
        if buf.data.device == device:
            continue
        buf.data = buf.data.to(device, non_blocking=False)
    dt = time.time() - t0
    log_event("upload_stream", device=device_id, tensors=tensors, seconds=round(dt, 1))
    if verbose:
        print(f"  device {device_id}: {tensors} tensors in {dt:.1f}s", flush=True)
    return tensors


@torch.no_grad()
def ensure_weights(module: torch.nn.Module, device_id: int) -> int:
    """Materialise every staged parameter of *module* on ``cuda:<device_id>``
    (``stratum/upload.py:969-1069``): FP16-staged params are copied in chunks, NF4
    payloads are uploaded packed (asynchronously, from pinned memory) and
    dequantized by the GPU kernel, other params/buffers are moved if needed.
    Runs on the current stream. Returns the number of tensors touched.
    """
    device = torch.device(f"cuda:{device_id}")
    tensors = 0
    owner_map = _build_param_owner_map(module)
    for name, param in module.named_parameters():
        fp16_payload = getattr(param, FP16_ATTR, None)
        if fp16_payload is not None:
            if param.data.numel() > 0:
                if param.data.device == device:
                    continue
                # shared staged param reached from another device: re-upload here
                param.data = torch.empty(0, dtype=param.dtype, device=param.device)
            dst = torch.empty(fp16_payload.shape, dtype=fp16_payload.dtype, device=device)
            copy_tensor_chunked(fp16_payload.data, dst, chunk_bytes=DEFAULT_CHUNK_UPLOAD_BYTES, non_blocking=True)
            param.data = dst
            tensors += 1
            continue
        payload = getattr(param, NF4_ATTR, None)
        if payload is None:
            if param.data.numel() > 0 and param.data.device != device:
                if param.requires_grad:
                    raise RuntimeError(
                        f"trainable shared parameter {name!r} is on {param.data.device}, "
                        f"but module is running on {device}; Stratum cannot safely move "
                        "trainable parameters between stages")
                param.data = param.data.to(device, non_blocking=True)
                tensors += 1
            continue
        if param.data.numel() > 0:
            if param.data.device == device:
                continue  # already materialised on the target device
            # shared frozen weight used on another device: re-materialise from the payload
            target = "cpu" if param.device.type == "meta" else param.device
            owner, pname = owner_map.get(id(param), (None, None))
            _replace_param_data(param, torch.empty(0, dtype=param.dtype, device=target), owner=owner, pname=pname)
        q_gpu = payload.quantized.to(device, non_blocking=True)
        a_gpu = payload.absmax.to(device, non_blocking=True)
        owner, pname = owner_map.get(id(param), (None, None))
        with torch.cuda.device(device):
            weight = _dequantize_payload(payload, q_gpu, a_gpu)
        _replace_param_data(param, weight, owner=owner, pname=pname)
        tensors += 1
    for buf in module.buffers():
        replaced = False
        if buf.device.type == "meta":
            try:
                buf.data = torch.empty(buf.shape, dtype=buf.dtype, device="cpu")
            except (RuntimeError, TypeError):
                for _m_name, sub in module.named_modules():
                    for b_name, b in sub.named_buffers(recurse=False):
                        if b is buf:
                            new_b = torch.empty(buf.shape, dtype=buf.dtype, device="cpu")
                            sub.register_buffer(b_name, new_b)
                            buf = new_b
                            replaced = True
                            break
                    else:
                        continue
                    break
        if replaced:
            buf.data = buf.data.to(device, non_blocking=True)
            tensors += 1
        elif buf.data.device != device:
            buf.data = buf.data.to(device, non_blocking=True)
            tensors += 1
    return tensors


_copy_streams: dict = {}


def _copy_stream(device: torch.device) -> "torch.cuda.Stream":
    """One persistent H2D copy stream per device (default priority)."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    s = _copy_streams.get(key)
    if s is None:
        s = torch.cuda.Stream(device=device)
        _copy_streams[key] = s
    return s


@torch.no_grad()
def prefetch_weights(module: torch.nn.Module, device_id: int) -> NF4Prefetch:
    """Start the asynchronous H2D copies of the packed payloads of *module*'s empty
    NF4 params on the device's copy stream (``stratum/upload.py:1072-1125``).
    Parameter data is not touched until ``NF4Prefetch.finalize()``."""
    device = torch.device(f"cuda:{device_id}")
    owner_map = _build_param_owner_map(module)
    entries: list = []
    for name, param in module.named_parameters():
        payload = getattr(param, NF4_ATTR, None)
        if payload is None:
            continue
        if param.data.numel() > 0 and param.data.device == device:
            continue
        owner, pname = owner_map.get(id(param), (None, None))
        p = cast(NF4Payload, payload)
        entries.append(_PrefetchEntry(param=param, payload=p, quantized=p.quantized, absmax=p.absmax, code=p.code,
                                      owner=owner, pname=pname))
    if not entries:
        return NF4Prefetch([], device)
    if device.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(f"CUDA is not available for NF4 prefetch to {device}")
    stream = _copy_stream(device)
    prefetched: list = []
    with torch.cuda.device(device), torch.cuda.stream(stream):
        for e in entries:
            prefetched.append(_PrefetchEntry(
                param=e.param, payload=e.payload,
                quantized=e.quantized.to(device, non_blocking=True),
                absmax=e.absmax.to(device, non_blocking=True),
                code=e.code, owner=e.owner, pname=e.pname))
        event = torch.cuda.Event()
        stream.record_event(event)
    return NF4Prefetch(prefetched, device=device, stream=stream, event=event)


@torch.no_grad()
def ensure_prefetched_weights(module: torch.nn.Module, device_id: int, prefetch: Optional[NF4Prefetch]) -> int:
    """Finalize a matching prefetch, then run the regular ensure for the rest."""
    if prefetch is None:
        return ensure_weights(module, device_id)
    if prefetch.device != torch.device(f"cuda:{device_id}"):
        raise ValueError(f"prefetch device {prefetch.device} does not match cuda:{device_id}")
    return prefetch.finalize() + ensure_weights(module, device_id)


@torch.no_grad()
def free_weights(module: torch.nn.Module) -> int:
    """Drop the materialised data of staged params (payload kept). Returns the count."""
    tensors = 0
    for _name, param in module.named_parameters():
        if not hasattr(param, NF4_ATTR) and not hasattr(param, FP16_ATTR):
            continue
        if param.data.numel() == 0:
            continue
        param.data = torch.empty(0, dtype=param.dtype, device=param.device)
        tensors += 1
    return tensors


@torch.no_grad()
def snapshot_module_buffers(module: torch.nn.Module) -> dict:
    """CPU clones of all non-empty buffers, for restoring before a recompute."""
    snap: dict = {}
    for name, buf in module.named_buffers():
        if buf.numel() > 0:
            snap[name] = buf.detach().to("cpu", non_blocking=False).clone()
    return snap


@torch.no_grad()
def restore_module_buffers(module: torch.nn.Module, snapshot: dict) -> int:
    """Copy a snapshot back into the module's buffers. Returns the number restored."""
    if not snapshot:
        return 0
    buf_map = dict(module.named_buffers())
    restored = 0
    for name, cpu_clone in snapshot.items():
        buf = buf_map.get(name)
        if buf is None:
            continue
        buf.data.copy_(cpu_clone.to(buf.device, non_blocking=False))
        restored += 1
    return restored


@torch.no_grad()
def prepare_nf4_from_cache(module: torch.nn.Module, cache_dir: str | Path | None, *, min_numel: int = 4096,
                           blocksize: int = 64, quant_type: str = "nf4", verbose: bool = True) -> Optional[NF4Stats]:
    """Attach cached payloads to every eligible param (meta params allowed); None on
    the first miss so the caller can fall back (``stratum/upload.py:1207-1283``)."""
    if cache_dir is None:
        return None
    cache_root = Path(cache_dir)
    stats = NF4Stats()
    owner_map = _build_param_owner_map(module)
    for name, param in module.named_parameters():
        if param.requires_grad:
            continue
        if param.ndim < 2:
            continue
        if param.numel() < min_numel:
            continue
        if param.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            continue
        if hasattr(param, NF4_ATTR):
            payload = cast(NF4Payload, getattr(param, NF4_ATTR))
            stats.tensors += 1
            stats.source_bytes += payload.source_bytes
            stats.payload_bytes += payload.payload_bytes
            continue
        payload = _load_payload_from_cache(_cache_path(cache_root, name), param, blocksize=blocksize,
                                           quant_type=quant_type)
        if payload is None:
            if verbose:
                print(f"  nf4 cache miss: {name} -- requires FP16 load", flush=True)
            return None
        stats.cache_hits += 1
        setattr(param, NF4_ATTR, payload)
        owner, pname = owner_map.get(id(param), (None, None))
        _replace_param_data(param, torch.empty(0, dtype=payload.dtype, device="cpu"), owner=owner, pname=pname)
        stats.tensors += 1
        stats.source_bytes += payload.source_bytes
        stats.payload_bytes += payload.payload_bytes
    if verbose:
        print(f"  nf4 from cache: {stats.tensors} tensors, {stats.source_bytes / 1024**3:.2f} GiB source -> "
              f"{stats.payload_bytes / 1024**3:.2f} GiB payload (cache hits={stats.cache_hits})", flush=True)
    return stats


def _replace_param_data(param: torch.nn.Parameter, new_data: torch.Tensor, owner: Optional[torch.nn.Module] = None,
                        pname: Optional[str] = None) -> None:
    """``param.data = new_data``; when a Parameter subclass refuses, register a new
    Parameter (payload attributes carried over) on *owner* (``stratum/upload.py:1286-1310``)."""
    try:
        param.data = new_data
        return
    except (RuntimeError, TypeError):
        pass
    if owner is not None and pname is not None:
        new_param = torch.nn.Parameter(new_data, requires_grad=param.requires_grad)
        for attr in (NF4_ATTR, FP16_ATTR):
            if hasattr(param, attr):
                setattr(new_param, attr, getattr(param, attr))
        owner.register_parameter(pname, new_param)


def _build_param_owner_map(module: torch.nn.Module) -> dict:
    """id(param) -> (owner module, local name)."""
    pmap: dict = {}
    for _m_name, sub in module.named_modules():
        for p_name, p in sub.named_parameters(recurse=False):
            pmap[id(p)] = (sub, p_name)
    return pmap


def nf4_code_table(device=None) -> torch.Tensor:
    """The fp32 [16] NF4 level table stored in ``NF4Payload.code``."""
    return get_4bit_type("nf4", device=device)


# Checkpoint loaders (stratum/upload.py:425-904,1325-1440) live in .checkpoint;
# imported last because they use this module's helpers.
from .checkpoint import (_build_ckpt_key_fn, _try_load_fused_experts, load_module_fp16_from_checkpoint,  # noqa: E402
                         populate_from_hf_checkpoint, stream_load_and_quantize_module)
