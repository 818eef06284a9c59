"""NF4 operators on the gfx950 kernels, shaped like the ``bitsandbytes.functional``
API that the reference calls (``quantize_4bit``, ``dequantize_4bit``,
``QuantState``, ``get_4bit_type``), plus the fused frozen-base GEMMs.

Reference call sites this module replaces:
  quantize_4bit   stratum/upload.py:367-369, :725-727; scripts/doctor.py:80-85
  dequantize_4bit stratum/upload.py:221, :946, :1038; stratum/nf4_linear.py:46
  F.linear on the dequantized frozen weight, forward and input gradient:
                  stratum/nf4_linear.py:47, stratum/stage.py:135,
                  stratum/runtime.py:340-341, stratum/model/mlp_opt.py:181-183,206-212

Every operator runs the HIP library; there is no CPU implementation. A CPU
input to ``quantize_4bit`` is copied to the current GPU, quantized there and
copied back, so the result lands where bitsandbytes' would (on the input's
device).
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Optional, Sequence

import torch

from . import _lib

# NF4 levels (QLoRA, arXiv 2305.14314 App. E); the fp32 table bitsandbytes
# returns from get_4bit_type("nf4") and the reference stores in NF4Payload.code.
NF4_LEVELS = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)

ROUNDING_RULES = {"argmin": _lib.STM_NF4_ARGMIN, "threshold": _lib.STM_NF4_THRESHOLD}
# The reference quantizes CPU tensors (stratum/upload.py:360), i.e. with the
# torch/CPU backend of bitsandbytes, whose nearest-level rule is an fp32 argmin.
DEFAULT_ROUNDING = "argmin"


_CODE_ON_DEVICE: dict = {}


def get_4bit_type(typename: str = "nf4", device=None) -> torch.Tensor:
    """The 16 NF4 levels as an fp32 tensor on ``device``.

    On a GPU one tensor per device is created once and shared by every
    QuantState (a fresh host-to-device copy per quantize call would block the
    host); treat it as read-only.
    """
    if typename != "nf4":
        raise NotImplementedError(f"4-bit type {typename!r} is not supported (only 'nf4')")
    dev = torch.device(device) if device is not None else torch.device("cpu")
    if dev.type != "cuda":
        return torch.tensor(NF4_LEVELS, dtype=torch.float32, device=dev)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    code = _CODE_ON_DEVICE.get(dev)
    if code is None:
        code = _CODE_ON_DEVICE[dev] = torch.tensor(NF4_LEVELS, dtype=torch.float32, device=dev)
    return code


class QuantState:
    """Quantization metadata of one NF4 tensor (the fields bitsandbytes'
    QuantState carries on this path; ``stratum/upload.py:211-218,1031-1034``)."""

    def __init__(self, absmax: torch.Tensor, shape=None, code: Optional[torch.Tensor] = None,
                 blocksize: Optional[int] = None, quant_type: Optional[str] = None,
                 dtype: Optional[torch.dtype] = None, offset=None, state2=None):
        if offset is not None or state2 is not None:
            raise NotImplementedError("nested (compress_statistics=True) absmax is not supported")
        self.absmax = absmax
        self.shape = torch.Size(shape) if shape is not None else None
        self.code = code if code is not None else get_4bit_type("nf4", device=absmax.device)
        self.blocksize = int(blocksize) if blocksize is not None else 64
        self.quant_type = quant_type if quant_type is not None else "nf4"
        self.dtype = dtype
        self.offset = None
        self.state2 = None
        self.nested = False

    def to(self, device) -> "QuantState":
        self.absmax = self.absmax.to(device)
        self.code = self.code.to(device)
        return self

    def __repr__(self) -> str:
        return (f"QuantState(shape={tuple(self.shape) if self.shape is not None else None}, "
                f"dtype={self.dtype}, blocksize={self.blocksize}, quant_type={self.quant_type!r})")


def _check_nf4(quant_type: str, blocksize: int) -> None:
    if quant_type != "nf4":
        raise NotImplementedError(f"quant_type {quant_type!r} is not supported (only 'nf4')")
    if blocksize < 64 or blocksize > 4096 or blocksize & (blocksize - 1):
        raise ValueError(f"blocksize {blocksize} must be a power of two in [64, 4096]")


def _gpu_device(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("stratum_amd NF4 kernels need a GPU (HIP); none is available")
    return torch.device("cuda", torch.cuda.current_device())


def _aligned(t: torch.Tensor, a: int = 16) -> torch.Tensor:
    t = t.contiguous()
    if t.numel() and t.data_ptr() % a:
        t = t.clone()
    return t


def _gemm_workspace(M: int, N: int, K: int, backward: bool, device) -> Optional[torch.Tensor]:
    """fp32 split-reduction workspace for a fused GEMM of this size, from torch's
    caching allocator (None when the library does not split this problem)."""
    nbytes = int(_lib.lib().stm_nf4_gemm_workspace_bytes(M, N, K, int(backward)))
    if nbytes < 0:
        _lib.check(nbytes, "stm_nf4_gemm_workspace_bytes")
    if nbytes == 0:
        return None
    return torch.empty(nbytes // 4, dtype=torch.float32, device=device)


def _out_buffer(out: Optional[torch.Tensor], shape, dtype, device) -> torch.Tensor:
    """A fresh output tensor, or ``out`` viewed as ``shape`` after checking it can take the result."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    numel = 1
    for d in shape:
        numel *= int(d)
    if out.dtype != dtype or out.device != device or out.numel() != numel:
        raise ValueError(f"out must be a {dtype} tensor of {numel} elements on {device}")
    if not out.is_contiguous() or (numel and out.data_ptr() % 16):
        raise ValueError("out must be contiguous and 16-byte aligned")
    return out.view(shape)


@torch.no_grad()
def quantize_4bit(A: torch.Tensor, absmax: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                  blocksize: int = 64, compress_statistics: bool = False, quant_type: str = "nf4",
                  quant_storage: torch.dtype = torch.uint8, *, rounding: str = DEFAULT_ROUNDING):
    """Blockwise NF4 quantize + pack. Returns ``(packed uint8 [(n+1)//2, 1], QuantState)``.

    ``rounding`` picks the nearest-level rule: "argmin" (bitsandbytes' torch/CPU
    backend, the path the reference runs) or "threshold" (its CUDA kernel);
    the two differ only for values that sit exactly on an fp32 midpoint.
    """
    _check_nf4(quant_type, blocksize)
    if compress_statistics:
        raise NotImplementedError("compress_statistics=True is not supported (the reference passes False)")
    if quant_storage != torch.uint8:
        raise NotImplementedError("only uint8 quant_storage is supported")
    if rounding not in ROUNDING_RULES:
        raise ValueError(f"rounding must be one of {sorted(ROUNDING_RULES)}, got {rounding!r}")
    tag = _lib.dtype_tag(A.dtype)
    dev = _gpu_device(A)
    src = _aligned(A.detach().to(dev))
    n = src.numel()
    nblocks = -(-n // blocksize)
    packed = torch.empty(((n + 1) // 2, 1), dtype=torch.uint8, device=dev)
    am = torch.empty(nblocks, dtype=torch.float32, device=dev)
    L = _lib.lib()
    with torch.cuda.device(dev):
        rc = L.stm_nf4_quantize(src.data_ptr(), tag, n, blocksize, ROUNDING_RULES[rounding], packed.data_ptr(),
                                am.data_ptr(), _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_quantize")
    if not A.is_cuda:
        packed = packed.to(A.device)
        am = am.to(A.device)
    if out is not None:
        out.copy_(packed.view_as(out))
        packed = out
    if absmax is not None:
        absmax.copy_(am)
        am = absmax
    state = QuantState(absmax=am, shape=A.shape, code=get_4bit_type("nf4", device=am.device), blocksize=blocksize,
                       quant_type=quant_type, dtype=A.dtype)
    return packed, state


@torch.no_grad()
def dequantize_4bit(A: torch.Tensor, quant_state: Optional[QuantState] = None, absmax: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None, blocksize: int = 64, quant_type: str = "nf4",
                    *, dtype: Optional[torch.dtype] = None, shape: Optional[Sequence[int]] = None) -> torch.Tensor:
    """``out = dtype(code[q] * absmax)`` for every element, on A's device and the current stream.

    ``dtype`` overrides ``quant_state.dtype`` (e.g. an fp16-sourced payload
    dequantized to bf16 for bf16 compute).
    """
    if quant_state is not None:
        absmax = quant_state.absmax if absmax is None else absmax
        blocksize = quant_state.blocksize
        quant_type = quant_state.quant_type
        shape = quant_state.shape if shape is None else shape
        dtype = quant_state.dtype if dtype is None else dtype
    if absmax is None or shape is None:
        raise ValueError("dequantize_4bit needs a quant_state or absmax + shape")
    dtype = dtype or torch.float16
    _check_nf4(quant_type, blocksize)
    if not A.is_cuda:
        raise RuntimeError("dequantize_4bit runs on the GPU kernel; the packed tensor is on the CPU")
    dev = A.device
    n = 1
    for s in shape:
        n *= int(s)
    if A.numel() * 2 < n:
        raise ValueError(f"packed tensor holds {A.numel() * 2} codes, shape {tuple(shape)} needs {n}")
    if absmax.numel() < -(-n // blocksize):
        raise ValueError(f"absmax holds {absmax.numel()} blocks, need {-(-n // blocksize)}")
    q = _aligned(A, 4)
    am = _aligned(absmax.to(dev, torch.float32), 4)
    if out is None:
        out = torch.empty(tuple(shape), dtype=dtype, device=dev)
    elif not out.is_contiguous() or out.numel() != n or out.dtype != dtype or out.device != dev:
        raise ValueError("out must be a contiguous tensor of the quant_state shape and dtype, on the packed "
                         "tensor's device")
    with torch.cuda.device(dev):
        rc = _lib.lib().stm_nf4_dequantize(q.data_ptr(), am.data_ptr(), n, blocksize, out.data_ptr(),
                                           _lib.dtype_tag(dtype), _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_dequantize")
    return out


def _ptr_array(values, ctype=None):
    import ctypes
    ctype = ctype or ctypes.c_void_p
    return (ctype * max(1, len(values)))(*values)


@torch.no_grad()
def quantize_4bit_many(tensors: Sequence[torch.Tensor], blocksize: int = 64, *,
                       rounding: str = DEFAULT_ROUNDING) -> list:
    """``[quantize_4bit(t, blocksize=blocksize, rounding=rounding) for t in tensors]``
    with the whole blocks of up to 32 tensors in one launch (bit-identical
    results). All tensors must share a dtype; GPU tensors must share a device
    (CPU tensors are copied to it, and their results back)."""
    if rounding not in ROUNDING_RULES:
        raise ValueError(f"rounding must be one of {sorted(ROUNDING_RULES)}, got {rounding!r}")
    _check_nf4("nf4", blocksize)
    if not tensors:
        return []
    dtypes = {t.dtype for t in tensors}
    if len(dtypes) != 1:
        raise ValueError(f"quantize_4bit_many takes one dtype per call, got {sorted(map(str, dtypes))}")
    dtype = dtypes.pop()
    tag = _lib.dtype_tag(dtype)
    dev = _gpu_device(next((t for t in tensors if t.is_cuda), tensors[0]))
    if any(t.is_cuda and t.device != dev for t in tensors):
        raise ValueError("quantize_4bit_many takes the GPU tensors of one device per call")
    srcs = [_aligned(t.detach().to(dev)) for t in tensors]
    ns = [x.numel() for x in srcs]
    packed = [torch.empty(((n + 1) // 2, 1), dtype=torch.uint8, device=dev) for n in ns]
    ams = [torch.empty(-(-n // blocksize), dtype=torch.float32, device=dev) for n in ns]
    import ctypes
    with torch.cuda.device(dev):
        rc = _lib.lib().stm_nf4_quantize_many(
            len(srcs), _ptr_array([x.data_ptr() for x in srcs]), _ptr_array(ns, ctypes.c_int64), tag, blocksize,
            ROUNDING_RULES[rounding], _ptr_array([p.data_ptr() for p in packed]),
            _ptr_array([a.data_ptr() for a in ams]), _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_quantize_many")
    out = []
    for t, p, a in zip(tensors, packed, ams):
        if not t.is_cuda:
            p, a = p.to(t.device), a.to(t.device)
        out.append((p, QuantState(absmax=a, shape=t.shape, code=get_4bit_type("nf4", device=a.device),
                                  blocksize=blocksize, quant_type="nf4", dtype=t.dtype)))
    return out


@torch.no_grad()
def dequantize_4bit_many(items: Sequence[tuple], *, dtype: Optional[torch.dtype] = None,
                         out: Optional[Sequence[torch.Tensor]] = None) -> list:
    """``[dequantize_4bit(packed, state, dtype=dtype) for packed, state in items]``
    with the whole 8-element groups of up to 32 tensors in one launch
    (bit-identical results). All items must share blocksize, output dtype and
    GPU; ``out`` (optional) gives the output tensors."""
    if not items:
        return []
    states = [st for _, st in items]
    bss = {st.blocksize for st in states}
    dts = {dtype or st.dtype for st in states}
    if len(bss) != 1 or len(dts) != 1:
        raise ValueError("dequantize_4bit_many takes one blocksize and one output dtype per call")
    blocksize, odt = bss.pop(), dts.pop()
    _check_nf4("nf4", blocksize)
    for _, st in items:
        if st.quant_type != "nf4":
            raise ValueError(f"only nf4 is supported, got {st.quant_type!r}")
    dev = items[0][0].device
    if dev.type != "cuda" or any(q.device != dev for q, _ in items):
        raise RuntimeError("dequantize_4bit_many runs on the GPU kernel; every packed tensor must be on one GPU")
    ns = []
    for q, st in items:
        n = 1
        for d in st.shape:
            n *= int(d)
        if q.numel() * 2 < n:
            raise ValueError(f"packed tensor holds {q.numel() * 2} codes, shape {tuple(st.shape)} needs {n}")
        if st.absmax.numel() < -(-n // blocksize):
            raise ValueError(f"absmax holds {st.absmax.numel()} blocks, need {-(-n // blocksize)}")
        ns.append(n)
    qs = [_aligned(q, 4) for q, _ in items]
    ams = [_aligned(st.absmax.to(dev, torch.float32), 4) for st in states]
    if out is None:
        outs = [torch.empty(tuple(st.shape), dtype=odt, device=dev) for st in states]
    else:
        outs = list(out)
        if len(outs) != len(items) or any(not o.is_contiguous() or o.numel() != n or o.dtype != odt or o.device != dev
                                          for o, n in zip(outs, ns)):
            raise ValueError("out must hold one contiguous tensor of each item's shape and the output dtype")
    import ctypes
    with torch.cuda.device(dev):
        rc = _lib.lib().stm_nf4_dequantize_many(
            len(items), _ptr_array([q.data_ptr() for q in qs]), _ptr_array([a.data_ptr() for a in ams]),
            _ptr_array(ns, ctypes.c_int64), blocksize, _ptr_array([o.data_ptr() for o in outs]),
            _lib.dtype_tag(odt), _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_dequantize_many")
    return outs


@torch.no_grad()
def stack_nf4(items: Sequence[tuple]) -> tuple:
    """One NF4 weight ``[sum N_i, K]`` from weights ``[N_i, K]`` that share K and
    the blocksize: ``(packed, QuantState)`` with the packed bytes and absmax of
    the items back to back -- exactly what quantizing the row-stacked weight
    gives, since a block never straddles a row (K % blocksize == 0) and every
    row's bytes start on a byte (K even). A GEMM on the result computes the
    projections that read the same input (q/k/v, gate/up) as one launch, whose
    output columns are the items' outputs side by side."""
    if not items:
        raise ValueError("stack_nf4 needs at least one weight")
    states = [st for _, st in items]
    K = int(states[0].shape[-1])
    bs = states[0].blocksize
    for st in states:
        if len(st.shape) != 2 or int(st.shape[1]) != K or st.blocksize != bs or st.quant_type != "nf4":
            raise ValueError("stack_nf4 takes 2-D nf4 weights with one K and one blocksize")
    if K % bs or K % 2:
        raise ValueError(f"K = {K} must be a multiple of the blocksize {bs} (and even)")
    rows = [int(st.shape[0]) for st in states]
    packed = torch.cat([q.reshape(-1)[: n * K // 2] for (q, _), n in zip(items, rows)]).reshape(-1, 1)
    absmax = torch.cat([st.absmax.reshape(-1)[: n * K // bs] for st, n in zip(states, rows)])
    state = QuantState(absmax=absmax, shape=(sum(rows), K), code=states[0].code, blocksize=bs, quant_type="nf4",
                       dtype=states[0].dtype)
    return packed, state


# ------------------------------------------------------------ fused GEMMs
def _gemm_dtype(t: torch.Tensor) -> int:
    if t.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"fused NF4 GEMM computes in bf16 or fp16, got {t.dtype}")
    return _lib.dtype_tag(t.dtype)


def fused_supported(N: int, K: int, blocksize: int, backward: bool = False) -> bool:
    """Shapes the fused kernels take; other shapes go through dequantize + matmul."""
    if K % 64 or K % blocksize or N % 8:
        return False
    return not backward or N % 64 == 0


def _on_device(dev: torch.device, **tensors) -> None:
    """Every given tensor lives on *dev* (a pointer from another device or the
    host would be dereferenced by the kernel)."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, the kernel runs on {dev}")


def _check_weight(packed: torch.Tensor, absmax: torch.Tensor, N: int, K: int, blocksize: int, dev: torch.device,
                  experts: int = 1) -> None:
    """The packed codes and absmax hold ``experts`` weights of [N, K] on *dev*
    (checked before any launch: a short tensor would be read past its end)."""
    _check_nf4("nf4", blocksize)
    if packed.dtype != torch.uint8 or absmax.dtype != torch.float32:
        raise ValueError(f"packed must be uint8 and absmax float32, got {packed.dtype} and {absmax.dtype}")
    if packed.device != dev or absmax.device != dev:
        raise ValueError(f"packed ({packed.device}) and absmax ({absmax.device}) must be on {dev}")
    n = experts * N * K
    if packed.numel() * 2 < n:
        raise ValueError(f"packed holds {packed.numel() * 2} codes, {experts} weight(s) of [{N}, {K}] need {n}")
    if absmax.numel() * blocksize < n:
        raise ValueError(f"absmax holds {absmax.numel()} blocks, {-(-n // blocksize)} needed")


@torch.no_grad()
def nf4_gemm_fwd(x: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor, weight_shape: Sequence[int],
                 blocksize: int = 64, bias: Optional[torch.Tensor] = None, lora_t: Optional[torch.Tensor] = None,
                 lora_b: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x @ W.T (+ bias) (+ lora_t @ lora_b.T)`` with W [N, K] in NF4; output dtype = x.dtype.

    ``W`` is dequantized inside the kernel with the same rounding as
    ``dequantize_4bit(..., dtype=x.dtype)``. ``lora_t`` [M, R] and ``lora_b`` [N, R]
    (R a multiple of 16) add a rank-R term before the single output rounding.
    ``out``, if given, is a contiguous, 16-byte aligned tensor of the output's
    shape and dtype that receives the result.
    """
    N, K = int(weight_shape[0]), int(weight_shape[1])
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {K}")
    tag = _gemm_dtype(x)
    lead = x.shape[:-1]
    x2 = _aligned(x.reshape(-1, K))
    M = x2.shape[0]
    dev = x2.device
    _check_weight(packed, absmax, N, K, blocksize, dev)
    _on_device(dev, lora_t=lora_t, lora_b=lora_b)
    if bias is not None and (bias.numel() != N or bias.device != dev):
        raise ValueError(f"bias must hold {N} values on {dev}, got {bias.numel()} on {bias.device}")
    y = _out_buffer(out, (M, N), x.dtype, dev)
    b = _aligned(bias.to(x.dtype), 2) if bias is not None else None
    R = 0
    t = lb = None
    if lora_t is not None:
        t = _aligned(lora_t.reshape(M, -1).to(x.dtype))
        lb = _aligned(lora_b.to(x.dtype))
        R = t.shape[1]
        if lb.shape != (N, R):
            raise ValueError(f"lora_b shape {tuple(lb.shape)} != ({N}, {R})")
    with torch.cuda.device(dev):
        ws = _gemm_workspace(M, N, K, False, dev)
        rc = _lib.lib().stm_nf4_gemm_fwd(
            x2.data_ptr(), _aligned(packed).data_ptr(), _aligned(absmax, 4).data_ptr(),
            b.data_ptr() if b is not None else None,
            t.data_ptr() if t is not None else None, lb.data_ptr() if lb is not None else None, R,
            y.data_ptr(), M, N, K, blocksize, tag, ws.data_ptr() if ws is not None else None,
            4 * ws.numel() if ws is not None else 0, _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_gemm_fwd")
    return y.reshape(*lead, N)


@torch.no_grad()
def nf4_gemm_bwd_dx(dy: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor, weight_shape: Sequence[int],
                    blocksize: int = 64, lora_u: Optional[torch.Tensor] = None,
                    lora_at: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``dy @ W (+ lora_u @ lora_at.T)`` with W [N, K] in NF4; output dtype = dy.dtype
    (``out`` as for :func:`nf4_gemm_fwd`)."""
    N, K = int(weight_shape[0]), int(weight_shape[1])
    if dy.shape[-1] != N:
        raise ValueError(f"dy has {dy.shape[-1]} features, weight has {N} rows")
    tag = _gemm_dtype(dy)
    lead = dy.shape[:-1]
    d2 = _aligned(dy.reshape(-1, N))
    M = d2.shape[0]
    dev = d2.device
    _check_weight(packed, absmax, N, K, blocksize, dev)
    _on_device(dev, lora_u=lora_u, lora_at=lora_at)
    dx = _out_buffer(out, (M, K), dy.dtype, dev)
    R = 0
    u = at = None
    if lora_u is not None:
        u = _aligned(lora_u.reshape(M, -1).to(dy.dtype))
        at = _aligned(lora_at.to(dy.dtype))
        R = u.shape[1]
        if at.shape != (K, R):
            raise ValueError(f"lora_at shape {tuple(at.shape)} != ({K}, {R})")
    with torch.cuda.device(dev):
        ws = _gemm_workspace(M, N, K, True, dev)
        rc = _lib.lib().stm_nf4_gemm_bwd_dx(
            d2.data_ptr(), _aligned(packed).data_ptr(), _aligned(absmax, 4).data_ptr(),
            u.data_ptr() if u is not None else None, at.data_ptr() if at is not None else None, R,
            dx.data_ptr(), M, N, K, blocksize, tag, ws.data_ptr() if ws is not None else None,
            4 * ws.numel() if ws is not None else 0, _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_gemm_bwd_dx")
    return dx.reshape(*lead, K)


_OFFSETS_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
_OFFSETS_CACHE_SIZE = 8


def _device_offsets(host_off, dev: torch.device):
    """(pinned host int32 copy, device int32 copy) of validated offsets.

    The values go to the device from pinned memory without a host wait (the
    caching host allocator keeps the pinned block until the copy has run). The
    last few arrays are kept per device, so the projections of one MoE layer
    (gate/up, down, their input gradients) upload their shared offsets once; a
    hit from another stream waits on the upload's event first and hands the
    array over to that stream.
    """
    key = (dev.index, host_off.tobytes())
    hit = _OFFSETS_CACHE.get(key)
    stream = torch.cuda.current_stream(dev)
    if hit is not None:
        _OFFSETS_CACHE.move_to_end(key)
        staged, off, done, upload_stream = hit
        if upload_stream != stream:
            stream.wait_event(done)
            off.record_stream(stream)  # an eviction must not free it under this stream's kernels
        return staged, off
    staged = torch.empty(host_off.shape[0], dtype=torch.int32, pin_memory=True)
    staged.numpy()[:] = host_off
    with torch.cuda.device(dev):
        off = staged.to(dev, non_blocking=True)
        done = torch.cuda.Event()
        done.record(stream)
    _OFFSETS_CACHE[key] = (staged, off, done, stream)
    while len(_OFFSETS_CACHE) > _OFFSETS_CACHE_SIZE:
        _OFFSETS_CACHE.popitem(last=False)
    return staged, off


@torch.no_grad()
def nf4_grouped_gemm(x: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor, offsets: torch.Tensor,
                     expert_shape: Sequence[int], blocksize: int = 64, max_rows: Optional[int] = None,
                     backward: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-expert ``x[rows_e] @ W_e.T`` (or ``@ W_e`` when ``backward``) over a stacked
    NF4 payload of shape [E, N, K]; ``offsets`` int32 [E + 1] delimits each expert's rows.
    ``out`` (optional) is a contiguous [rows, N] (backward: [rows, K]) tensor of x's dtype.
    Offsets given as a CPU tensor are validated and uploaded without a device
    synchronisation.

    The offsets are checked on the host before any launch (one device-to-host
    copy, the synchronisation the grid size needs anyway): ``offsets[0] == 0``,
    non-decreasing, ``offsets[E] == x.shape[0]``; a given ``max_rows`` must cover
    the largest expert, and the payload must hold E * N * K codes. The kernels
    index X and Y with these values, so a bad array is a ValueError here rather
    than an out-of-bounds access on the GPU.
    """
    E = offsets.numel() - 1
    if E < 1:
        raise ValueError("offsets must hold at least two entries (one expert)")
    N, K = int(expert_shape[0]), int(expert_shape[1])
    tag = _gemm_dtype(x)
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [rows, features], got shape {tuple(x.shape)}")
    xin = _aligned(x)
    M_total = xin.shape[0]
    dev = xin.device
    host_off = offsets.detach().to("cpu", torch.int64).numpy()  # a device array: the one synchronisation
    counts = host_off[1:] - host_off[:-1]
    if host_off[0] != 0 or (counts < 0).any() or host_off[-1] != M_total:
        raise ValueError(f"offsets must start at 0, be non-decreasing and end at x.shape[0] = {M_total}; "
                         f"got {host_off.tolist()[:8]}{'...' if E > 7 else ''}")
    largest = int(counts.max())
    if max_rows is None:
        max_rows = largest
    elif int(max_rows) < largest:
        raise ValueError(f"max_rows = {max_rows} is below the largest expert's {largest} rows")
    _check_weight(packed, absmax, N, K, blocksize, dev, experts=E)
    if not xin.is_cuda:
        raise RuntimeError("nf4_grouped_gemm runs on the GPU kernels; x, packed and absmax must be on the GPU")
    staged, off = _device_offsets(host_off, dev)
    out_cols = K if backward else N
    in_cols = N if backward else K
    if xin.shape[1] != in_cols:
        raise ValueError(f"x has {xin.shape[1]} columns, expected {in_cols}")
    if out is None:
        y = torch.empty((M_total, out_cols), dtype=x.dtype, device=dev)
    else:
        if out.shape != (M_total, out_cols) or out.dtype != x.dtype or out.device != dev or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous [{M_total}, {out_cols}] {x.dtype} tensor on {dev}")
        y = out
    fn = _lib.lib().stm_nf4_grouped_gemm_bwd_dx if backward else _lib.lib().stm_nf4_grouped_gemm_fwd
    # the host copy of the offsets: validated by the library, and the forward's tile height
    lead = (xin.data_ptr(), _aligned(packed).data_ptr(), _aligned(absmax, 4).data_ptr(), off.data_ptr(),
            staged.data_ptr())
    with torch.cuda.device(dev):
        rc = fn(*lead, E, int(max_rows), y.data_ptr(), N, K, blocksize, tag, _lib.stream_handle(dev))
    _lib.check(rc, "stm_nf4_grouped_gemm_" + ("bwd_dx" if backward else "fwd"))
    return y


@torch.no_grad()
def swiglu_fwd(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``silu(gate) * up`` of a stacked projection output ``gate_up`` [..., 2 I] = [gate | up].

    fp32 arithmetic and one rounding to ``gate_up.dtype`` (bf16/fp16); the step
    ``act_fn(gate_proj(x)) * up_proj(x)`` of stratum/model/mlp_opt.py:178-180.
    """
    tag = _gemm_dtype(gate_up)
    two_i = gate_up.shape[-1]
    if two_i % 2:
        raise ValueError("gate_up must have an even last dimension [gate | up]")
    inter = two_i // 2
    gu = gate_up.reshape(-1, two_i).contiguous()
    rows = gu.shape[0]
    dev = gu.device
    h = _out_buffer(out, (rows, inter), gate_up.dtype, dev) if out is not None else \
        torch.empty((rows, inter), dtype=gate_up.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().stm_swiglu_fwd(gu.data_ptr(), h.data_ptr(), rows, inter, tag, _lib.stream_handle(dev))
    _lib.check(rc, "stm_swiglu_fwd")
    return h.reshape(*gate_up.shape[:-1], inter)


@torch.no_grad()
def swiglu_bwd(grad_out: torch.Tensor, gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gradient of :func:`swiglu_fwd` with respect to ``gate_up``: [..., 2 I] = [d gate | d up]."""
    tag = _gemm_dtype(gate_up)
    two_i = gate_up.shape[-1]
    inter = two_i // 2
    if grad_out.shape[-1] != inter or grad_out.dtype != gate_up.dtype:
        raise ValueError("grad_out must be [..., I] in gate_up's dtype")
    gu = gate_up.reshape(-1, two_i).contiguous()
    dh = grad_out.reshape(-1, inter).contiguous()
    rows = gu.shape[0]
    if dh.shape[0] != rows:
        raise ValueError("grad_out and gate_up have different row counts")
    dev = gu.device
    _on_device(dev, grad_out=dh)
    dgu = _out_buffer(out, (rows, two_i), gate_up.dtype, dev) if out is not None else \
        torch.empty((rows, two_i), dtype=gate_up.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().stm_swiglu_bwd(dh.data_ptr(), gu.data_ptr(), dgu.data_ptr(), rows, inter, tag,
                                       _lib.stream_handle(dev))
    _lib.check(rc, "stm_swiglu_bwd")
    return dgu.reshape(*gate_up.shape[:-1], two_i)


# ------------------------------------------------------------ LoRA side products
LORA_RANKS = (8, 16, 24, 32)


def lora_supported(rank: int, cols: int, rows: int = 0) -> bool:
    """Ranks, column counts (K or N of the frozen weight) and row counts the LoRA
    kernels take (a 256-row slice of the large operand and the fp32 partials of
    one 256-column block each within 2 GiB)."""
    return rank in LORA_RANKS and cols % 8 == 0 and cols * 512 <= 1 << 31 and rows * 128 <= 1 << 31


def _lora_workspace(rows: int, cols: int, rank: int, op: int, device) -> Optional[torch.Tensor]:
    nbytes = int(_lib.lib().stm_lora_workspace_bytes(rows, cols, rank, op))
    if nbytes < 0:
        _lib.check(nbytes, "stm_lora_workspace_bytes")
    if nbytes == 0:
        return None
    return torch.empty(nbytes // 4, dtype=torch.float32, device=device)


def _ptr(t: Optional[torch.Tensor]):
    return t.data_ptr() if t is not None and t.numel() else None


@torch.no_grad()
def lora_down(x: torch.Tensor, lora_a: torch.Tensor, scaling: float = 1.0) -> torch.Tensor:
    """``scaling * x @ lora_a.T`` as [rows, R] in x's dtype (the ``T`` the fused
    forward takes as ``lora_t``); one pass over x, fp32 accumulation, one rounding."""
    K = x.shape[-1]
    R = int(lora_a.shape[0])
    tag = _gemm_dtype(x)
    if tuple(lora_a.shape) != (R, K):
        raise ValueError(f"lora_a shape {tuple(lora_a.shape)} != ({R}, {K})")
    M = 1
    for d in x.shape[:-1]:
        M *= int(d)
    x2 = _aligned(x.reshape(M, K))
    dev = x2.device
    _on_device(dev, lora_a=lora_a)
    a = _aligned(lora_a.to(x.dtype))
    t = torch.empty((M, R), dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        ws = _lora_workspace(M, K, R, 0, dev)
        rc = _lib.lib().stm_lora_down(_ptr(x2), _ptr(a), _ptr(t), M, K, R, float(scaling), tag, _ptr(ws),
                                      4 * ws.numel() if ws is not None else 0, _lib.stream_handle(dev))
    _lib.check(rc, "stm_lora_down")
    return t


@torch.no_grad()
def lora_dy(dy: torch.Tensor, lora_b: torch.Tensor, t: Optional[torch.Tensor] = None, scaling: float = 1.0):
    """``(scaling * dy @ lora_b, dy.T @ t)`` -- the rank-R input of the LoRA term of
    dX and the gradient of ``lora_b`` -- from one pass over dy. The second is None
    when ``t`` is None. Results in dy's dtype."""
    N = dy.shape[-1]
    R = int(lora_b.shape[1])
    tag = _gemm_dtype(dy)
    if tuple(lora_b.shape) != (N, R):
        raise ValueError(f"lora_b shape {tuple(lora_b.shape)} != ({N}, {R})")
    d2 = _aligned(dy.reshape(-1, N))
    M = d2.shape[0]
    dev = d2.device
    _on_device(dev, lora_b=lora_b, t=t)
    b = _aligned(lora_b.to(dy.dtype))
    t2 = None
    if t is not None:
        t2 = _aligned(t.reshape(M, R).to(dy.dtype))
    u = torch.empty((M, R), dtype=dy.dtype, device=dev)
    db = torch.empty((N, R), dtype=dy.dtype, device=dev) if t is not None else None
    with torch.cuda.device(dev):
        ws = _lora_workspace(M, N, R, 1, dev)
        rc = _lib.lib().stm_lora_dy(_ptr(d2), _ptr(b), _ptr(t2), _ptr(u), _ptr(db), M, N, R, float(scaling), tag,
                                    _ptr(ws), 4 * ws.numel() if ws is not None else 0, _lib.stream_handle(dev))
    _lib.check(rc, "stm_lora_dy")
    return u, db


@torch.no_grad()
def lora_da(u: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """``u.T @ x`` ([R, K], x's dtype): the gradient of ``lora_a``; one pass over x."""
    K = x.shape[-1]
    x2 = _aligned(x.reshape(-1, K))
    M = x2.shape[0]
    R = int(u.shape[-1])
    tag = _gemm_dtype(x)
    dev = x2.device
    _on_device(dev, u=u)
    u2 = _aligned(u.reshape(M, R).to(x.dtype))
    da = torch.empty((R, K), dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        ws = _lora_workspace(M, K, R, 2, dev)
        rc = _lib.lib().stm_lora_da(_ptr(u2), _ptr(x2), _ptr(da), M, K, R, tag, _ptr(ws),
                                    4 * ws.numel() if ws is not None else 0, _lib.stream_handle(dev))
    _lib.check(rc, "stm_lora_da")
    return da
