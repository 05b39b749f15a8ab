"""Decode attention for the whole-model harness (model.py:104-153 at decode),
on the HIP kernel in csrc/attention.hip: one query token per (sequence,
head) against a contiguous KV cache, keys head_dim-major (B, heads,
head_dim, L) and values (B, heads, L, head_dim), positions past each
sequence's own masked.  Keys and values are each read once (the context is
split into 2048-position chunks whose partial softmax sums are merged by a
second launch); the arithmetic is fp32 up to the bf16 output.
"""

import torch

from . import _lib


def workspace(B, heads, head_dim, L, device):
    """The fp32 workspace decode_attention needs for these sizes (allocate
    once, outside graph capture)."""
    nbytes = _lib.lib().evo2_decode_attention_workspace_bytes(B, heads, head_dim, L)
    return torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=device)


def decode_attention(q, k_cache, v_cache, positions, scale, work=None):
    """q (B, heads, head_dim) bf16; k_cache (B, heads, head_dim, L) and v_cache
    (B, heads, L, head_dim) bf16 views; positions (B,) int64 (each sequence
    attends to cache positions 0..positions[b]).  Returns (B, heads,
    head_dim) bf16."""
    _lib.require_device(q, k_cache, v_cache, positions, work)
    B, heads, hd = q.shape
    L = k_cache.shape[-1]
    if k_cache.shape != (B, heads, hd, L) or v_cache.shape != (B, heads, L, hd):
        raise ValueError(f"cache shapes {tuple(k_cache.shape)}, {tuple(v_cache.shape)} do not "
                         f"match q {tuple(q.shape)}")
    if q.stride(2) != 1 or k_cache.stride(3) != 1 or v_cache.stride(3) != 1:
        raise ValueError("q rows, key positions and value dims must have unit stride")
    if positions.shape != (B,):
        raise ValueError(f"positions must be ({B},), got {tuple(positions.shape)}")
    positions = positions.to(torch.int64).contiguous()
    if work is None:
        work = workspace(B, heads, hd, L, q.device)
    out = torch.empty(B, heads, hd, dtype=torch.bfloat16, device=q.device)
    _lib.call("evo2_decode_attention",
              _lib.ptr(q), q.stride(0), q.stride(1),
              _lib.ptr(k_cache), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
              _lib.ptr(v_cache), v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
              _lib.ptr(positions), _lib.ptr(work), work.numel() * 4,
              _lib.ptr(out), out.stride(0), out.stride(1),
              B, heads, hd, L, float(scale), _lib.stream_of(q))
    return out


__all__ = ["decode_attention", "workspace"]
