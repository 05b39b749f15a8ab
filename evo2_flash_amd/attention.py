"""Attention for the whole-model harness (model.py:104-153).

Decode runs on the HIP kernel in csrc/attention.hip: one query token per
(sequence, head) against either a contiguous KV cache (keys head_dim-major
(B, heads, head_dim, L), values (B, heads, L, head_dim)) or a paged one of
16-position pages named by a per-sequence block table (key pages (pages,
heads, head_dim, 16), value pages (pages, heads, 16, head_dim)), positions
past each sequence's own masked.  Keys and values are each read once (the
context is split into 2048-position chunks whose partial softmax sums are
merged by a second launch); the arithmetic is fp32 up to the bf16 output.

Prefill attention (a prompt against itself, causal) runs on the HIP kernel
in csrc/attention_prefill.hip at head_dim 128 (the values transposed once
per call; fp32 scores and softmax, bf16 softmax weights in the value
product); other head dims on torch's fused attention kernels where the
platform has them for the inputs, else a chunked product with contiguous
operands and an fp32 softmax.
"""

import torch

from . import _lib

PAGE = 16  # positions per KV page


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


def paged_decode_attention(q, k_pages, v_pages, block_table, positions, scale, work=None,
                           shared_pages=0):
    """q (B, heads, head_dim) bf16; k_pages (pages, heads, head_dim, 16) and
    v_pages (pages, heads, 16, head_dim) bf16; block_table (>= B, max_pages)
    int32 (position l of sequence b is in page block_table[b, l // 16]);
    positions (B,) int64 (sequence b attends to 0..positions[b]).  Returns
    (B, heads, head_dim) bf16.  The kernel never reads through a table entry
    outside [0, pages): the positions of such an entry are left out of the
    softmax (check_block_table finds them on the host).  shared_pages: the
    first shared_pages entries of every row name the same pages (a prompt
    shared by all B sequences; shared_prefix_pages finds it on the host):
    those chunks read each page once for several sequences (head_dim 128: up
    to 32 on the matrix cores, the sums in another order, within a bf16
    rounding step of the undeclared result; 64: four, the same bits)."""
    _lib.require_device(q, k_pages, v_pages, block_table, positions, work)
    B, heads, hd = q.shape
    max_pages = block_table.shape[1]
    if (k_pages.shape[1:] != (heads, hd, PAGE) or v_pages.shape[1:] != (heads, PAGE, hd)
            or k_pages.shape[0] != v_pages.shape[0]):
        raise ValueError(f"page shapes {tuple(k_pages.shape)}, {tuple(v_pages.shape)} do not "
                         f"match q {tuple(q.shape)}")
    if q.stride(2) != 1 or k_pages.stride(3) != 1 or v_pages.stride(3) != 1:
        raise ValueError("q rows, key positions and value dims must have unit stride")
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1 or block_table.shape[0] < B:
        raise ValueError("block_table must be (>= B, max_pages) int32 with unit column stride")
    if positions.shape != (B,):
        raise ValueError(f"positions must be ({B},), got {tuple(positions.shape)}")
    positions = positions.to(torch.int64).contiguous()
    if work is None:
        work = workspace(B, heads, hd, max_pages * PAGE, q.device)
    out = torch.empty(B, heads, hd, dtype=torch.bfloat16, device=q.device)
    _lib.call("evo2_paged_decode_attention",
              _lib.ptr(q), q.stride(0), q.stride(1),
              _lib.ptr(k_pages), k_pages.stride(0), k_pages.stride(1), k_pages.stride(2),
              _lib.ptr(v_pages), v_pages.stride(0), v_pages.stride(1), v_pages.stride(2),
              k_pages.shape[0], _lib.ptr(block_table), block_table.stride(0), int(shared_pages),
              _lib.ptr(positions), _lib.ptr(work), work.numel() * 4,
              _lib.ptr(out), out.stride(0), out.stride(1),
              B, heads, hd, max_pages, float(scale), _lib.stream_of(q))
    return out


def shared_prefix_pages(block_table, B):
    """The number of leading entries that rows 0..B-1 of the block table
    share (the pages of a prompt behind all B sequences).  For tables built
    on the host; a device table is copied to the host first."""
    table = block_table.detach().cpu()[:B]
    if B <= 1:
        return 0
    same = (table == table[0:1]).all(dim=0)
    diff = (~same).nonzero()
    return int(diff[0, 0]) if diff.numel() else int(table.shape[1])


def check_block_table(block_table, lengths, num_pages, first_page=1):
    """Raise ValueError unless every page that sequence b's first lengths[b]
    positions use (block_table[b, :ceil(lengths[b] / 16)]) lies in
    [first_page, num_pages) (page 0 is the cache's null page).  For tables
    built on the host; a device table is copied to the host first."""
    table = block_table.detach().cpu()
    lengths = [int(n) for n in (lengths.detach().cpu().tolist()
                                if torch.is_tensor(lengths) else lengths)]
    if table.dim() != 2 or len(lengths) > table.shape[0]:
        raise ValueError(f"block_table {tuple(table.shape)} cannot serve {len(lengths)} sequences")
    for b, n in enumerate(lengths):
        npg = -(-n // PAGE)
        if npg > table.shape[1]:
            raise ValueError(f"sequence {b}: {n} positions need {npg} pages, the table has "
                             f"{table.shape[1]}")
        row = table[b, :npg]
        bad = (row < first_page) | (row >= num_pages)
        if bool(bad.any()):
            j = int(bad.nonzero()[0, 0])
            raise ValueError(f"sequence {b}: block_table[{b}, {j}] = {int(row[j])} is outside "
                             f"[{first_page}, {num_pages})")


class PagedKVCache:
    """One attention layer's KV pages: keys (pages, heads, head_dim, 16),
    values (pages, heads, 16, head_dim), bf16; page 0 is never handed out."""

    def __init__(self, num_pages, heads, head_dim, device):
        self.k = torch.zeros(num_pages, heads, head_dim, PAGE, dtype=torch.bfloat16,
                             device=device)
        self.v = torch.zeros(num_pages, heads, PAGE, head_dim, dtype=torch.bfloat16,
                             device=device)

    def append(self, k, v, block_table, positions):
        """k, v (B, heads, head_dim): the entries of sequence b at positions[b]."""
        B = k.shape[0]
        rows = torch.arange(B, device=k.device)
        page = block_table[rows, torch.div(positions, PAGE, rounding_mode="floor")].long()
        off = positions % PAGE
        self.k[page, :, :, off] = k
        self.v[page, :, off, :] = v

    def write_prompt(self, k, v, block_table):
        """k, v (B, heads, L, head_dim): positions 0..L-1 of sequences 0..B-1
        (the tail of the last page is zero)."""
        B, nh, L, hd = k.shape
        npg = -(-L // PAGE)
        if npg * PAGE != L:
            pad = npg * PAGE - L
            k = torch.nn.functional.pad(k, (0, 0, 0, pad))
            v = torch.nn.functional.pad(v, (0, 0, 0, pad))
        pages = block_table[:B, :npg].reshape(-1).long()
        self.k[pages] = k.reshape(B, nh, npg, PAGE, hd).permute(0, 2, 1, 4, 3).reshape(
            B * npg, nh, hd, PAGE)
        self.v[pages] = v.reshape(B, nh, npg, PAGE, hd).permute(0, 2, 1, 3, 4).reshape(
            B * npg, nh, PAGE, hd)

    def dense(self, block_table, B, L):
        """The first L positions of sequences 0..B-1 as contiguous caches
        (keys (B, heads, head_dim, L), values (B, heads, L, head_dim))."""
        npg = -(-L // PAGE)
        pages = block_table[:B, :npg].reshape(-1).long()
        nh, hd = self.k.shape[1], self.k.shape[2]
        kd = self.k[pages].reshape(B, npg, nh, hd, PAGE).permute(0, 2, 3, 1, 4).reshape(
            B, nh, hd, npg * PAGE)
        vd = self.v[pages].reshape(B, npg, nh, PAGE, hd).permute(0, 2, 1, 3, 4).reshape(
            B, nh, npg * PAGE, hd)
        return kd[..., :L], vd[:, :, :L]


_FUSED_SDPA = None  # whether torch's fused attention kernels take these inputs here


def _causal_chunked(q, k, v, scale, chunk=512):
    """softmax(scale q k^T + causal mask) v with every right operand
    contiguous, queries in chunks, the softmax in fp32."""
    N, nh, L, hd = q.shape
    qf = q.reshape(N * nh, L, hd)
    kt = k.reshape(N * nh, L, hd).transpose(1, 2).contiguous()    # (Nh, hd, L)
    vf = v.reshape(N * nh, L, hd)
    out = torch.empty_like(qf)
    for s0 in range(0, L, chunk):
        e = min(L, s0 + chunk)
        sc = torch.bmm(qf[:, s0:e].contiguous(), kt[:, :, :e].contiguous()).float() * scale
        i = torch.arange(s0, e, device=q.device)[:, None]
        j = torch.arange(e, device=q.device)[None, :]
        sc.masked_fill_(j > i, float("-inf"))
        p = torch.softmax(sc, dim=-1).to(q.dtype)
        out[:, s0:e] = torch.bmm(p, vf[:, :e].contiguous())
    return out.view(N, nh, L, hd)


def prefill_attention(q, k, v, scale):
    """Causal self-attention of prompts on this build's HIP kernel: q, k, v
    (N, heads, L, 128) bf16 with L a multiple of 8 -> (N, heads, L, 128)
    bf16.  The values are handed over transposed (one copy)."""
    _lib.require_device(q, k, v)
    N, nh, L, hd = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)} differ")
    if hd != 128 or L % 8:
        raise ValueError(f"prefill_attention takes head_dim 128 and L a multiple of 8, got {hd}, {L}")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("prefill_attention takes bf16 q, k, v")
    q = q.contiguous()
    k = k.contiguous()
    vt = v.transpose(-1, -2).contiguous()
    out = torch.empty_like(q)
    _lib.call("evo2_prefill_attention", _lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out),
              N, nh, L, hd, float(scale), _lib.stream_of(q))
    return out


def causal_prefill_attention(q, k, v, scale):
    """Causal self-attention of prompts: q, k, v (N, heads, L, head_dim) bf16
    -> (N, heads, L, head_dim).  head_dim 128 with L a multiple of 8 runs on
    prefill_attention (this build's kernel); other shapes on torch's fused
    kernels (flash or memory-efficient) where they accept the inputs, never
    its unfused math path, which multiplies by a transposed view."""
    if q.shape[-1] == 128 and q.shape[-2] % 8 == 0 and q.shape[-2] > 0 and q.is_cuda:
        return prefill_attention(q, k, v, scale)
    global _FUSED_SDPA
    if _FUSED_SDPA is not False:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                out = torch.nn.functional.scaled_dot_product_attention(
                    q, k, v, is_causal=True, scale=scale)
            _FUSED_SDPA = True
            return out
        except RuntimeError:
            _FUSED_SDPA = False
    return _causal_chunked(q, k, v, scale)


__all__ = ["decode_attention", "workspace", "paged_decode_attention", "check_block_table",
           "PagedKVCache", "causal_prefill_attention", "prefill_attention", "PAGE"]
