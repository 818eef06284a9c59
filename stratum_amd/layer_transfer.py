"""Chunked tensor copy used by the FP16-staged branch of ``ensure_weights``
(``stratum/layer_transfer.py:18,59-89``)."""

from __future__ import annotations

import torch

DEFAULT_CHUNK_UPLOAD_BYTES = 256 * 1024 * 1024


def _chunk_numel(tensor: torch.Tensor, chunk_bytes: int) -> int:
    if chunk_bytes <= 0:
        raise ValueError(f"chunk_bytes must be positive, got {chunk_bytes}")
    return max(1, chunk_bytes // max(1, tensor.element_size()))


@torch.no_grad()
def copy_tensor_chunked(src: torch.Tensor, dst: torch.Tensor, *, chunk_bytes: int = DEFAULT_CHUNK_UPLOAD_BYTES,
                        non_blocking: bool = False) -> int:
    """Copy *src* into *dst* in flat chunks of at most *chunk_bytes*; returns the chunk count."""
    if src.shape != dst.shape:
        raise ValueError(f"shape mismatch: {tuple(src.shape)} != {tuple(dst.shape)}")
    if src.dtype != dst.dtype:
        raise ValueError(f"dtype mismatch: {src.dtype} != {dst.dtype}")
    if src.numel() == 0:
        return 0
    if not dst.is_contiguous():
        dst.copy_(src, non_blocking=non_blocking)
        return 1
    flat_src = src.detach().contiguous().view(-1)
    flat_dst = dst.view(-1)
    step = _chunk_numel(src, chunk_bytes)
    chunks = 0
    for start in range(0, src.numel(), step):
        end = min(start + step, src.numel())
        flat_dst[start:end].copy_(flat_src[start:end], non_blocking=non_blocking)
        chunks += 1
    return chunks
