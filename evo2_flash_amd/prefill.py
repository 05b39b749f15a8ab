"""Varlen Hyena FIR prefill (HIP, gfx950).

`fir_prefill` and `fir_prefill_block_t` keep the signatures of
evo2_flash/triton_prefill.py:462-501; `hyena_fir_prefill` is the fused
prefill core of HyenaFIRMixer (mixers.py:1277-1305) between in_proj and
out_proj.  Kernels: csrc/prefill_fir.hip.
"""

import torch

from . import _lib

# Rows per tile.  A tile is swept in sub-tiles with the FIR history in LDS,
# so longer tiles amortise the (K-1)-row halo; shorter ones add parallelism
# when there are few tokens.  The fused K=128 core runs on the matrix cores
# once a tile holds a 256-row sub-tile, with four 16-channel workgroups per
# 64-channel block: at 7B/32k on one MI355X 466 us with 4096-row tiles,
# 477 with 2048, 494 with 1024, 564 with 512, 532 with 8192 (too few
# workgroups).
_MAX_BLOCK_T = {7: 1024, 128: 4096}
_MFMA_MIN_BLOCK_T = 256
_TARGET_WORKGROUPS = 2048
# Long filters: below 256 rows the 127-row halo is a third or more of a
# tile's reads, and on one MI355X 256-row tiles beat 64-row ones by 10-22%
# at 2048-8192 tokens (H = 1920 and 4096) once the launch has 128
# workgroups; with fewer (a few hundred tokens) parallelism wins again.
_LONG_FILTER_MIN_BLOCK_T = 256
_LONG_FILTER_MIN_WORKGROUPS = 128


# Single-pass form of the hcm and hcl cores (csrc/prefill_stripe.hip): a
# workgroup sweeps one whole segment for 16 channels, so a launch is
# segments x H/16 workgroups, each as long as its segment.  It is chosen
# while the longest segment is at most _STRIPE_BALANCE times the rows one of
# the _STRIPE_CUS compute units would sweep with the work spread evenly (at
# one 32k-token segment that is H >= 2731), and the launch passes a tile
# table of whole segments (block_t >= the step's rows).
_STRIPE_CUS = 256
_STRIPE_BALANCE = 1.5
_STRIPE_GROUP = 16


def stripe_block_t(num_tokens, hidden, max_segment=None):
    """block_t that selects the single-pass kernels for a step of
    `num_tokens` prefill rows whose longest segment has `max_segment` rows
    (default: one segment), or None when the tiled kernels fit better."""
    if num_tokens is None or hidden is None or int(num_tokens) <= 0:
        return None
    T, H = int(num_tokens), int(hidden)
    if H % _STRIPE_GROUP:
        return None
    longest = T if max_segment is None else max(1, int(max_segment))
    even = T * (H // _STRIPE_GROUP) / _STRIPE_CUS
    if longest > _STRIPE_BALANCE * even:
        return None
    return (T + 63) // 64 * 64


# The fused K=128 core on 32-channel stripes (H a multiple of 32): one
# workgroup per (tile, 32 channels), the tile swept with its FIR history in
# LDS after a 256-row lead-in.  Tiles are sized for about one workgroup per
# compute unit (a 32k-token segment at H=4096: two 16384-row tiles).
_STRIPE_FIR_GROUP = 32
_STRIPE_FIR_MIN = 256


def stripe_fir_block_t(num_tokens, hidden, max_segment=None):
    """block_t of the 32-channel K=128 kernel, or None when H does not fit it."""
    if num_tokens is None or hidden is None or int(num_tokens) <= 0:
        return None
    T, H = int(num_tokens), int(hidden)
    if H % _STRIPE_FIR_GROUP:
        return None
    tiles = max(1, _STRIPE_CUS // (H // _STRIPE_FIR_GROUP))
    bt = -(-T // tiles)
    if max_segment is not None:
        bt = min(bt, max(1, int(max_segment)))
    return max(_STRIPE_FIR_MIN, -(-bt // _STRIPE_FIR_MIN) * _STRIPE_FIR_MIN)


def fir_prefill_block_t(k, num_tokens=None, hidden=None, max_segment=None):
    """Rows per prefill tile for filter length k; the tile table is built for
    this value.  For k = 128 and H a multiple of 32 the tiles are sized for
    the 32-channel kernel (`stripe_fir_block_t`).  Otherwise, with
    `num_tokens` and `hidden` it shrinks (to a multiple of 64) until the
    launch has enough workgroups to fill the GPU (counting the fused K=128
    core's four 16-channel workgroups per 64-channel block at tiles of 256
    rows or more); for filters longer than 8 taps it stops at 256 rows once
    the launch has 128 workgroups."""
    if int(k) == 128:
        bt = stripe_fir_block_t(num_tokens, hidden, max_segment)
        if bt is not None:
            return bt
    bt = _MAX_BLOCK_T.get(int(k), 1024)
    if num_tokens is not None and hidden is not None:
        cblocks = max(1, (int(hidden) + 63) // 64)
        while bt > 64:
            groups = cblocks * (4 if int(k) > 8 and bt >= _MFMA_MIN_BLOCK_T else 1)
            nwg = ((int(num_tokens) + bt - 1) // bt) * groups
            if nwg >= _TARGET_WORKGROUPS:
                break
            if (int(k) > 8 and bt <= _LONG_FILTER_MIN_BLOCK_T
                    and nwg >= _LONG_FILTER_MIN_WORKGROUPS):
                break
            bt //= 2
    return bt


def _check_tables(seq_table, tile_table):
    for name, t, w in (("seq_table", seq_table, 3), ("tile_table", tile_table, 2)):
        if t.dtype != torch.int32 or t.dim() != 2 or t.shape[1] != w or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous (n, {w}) int32 tensor")


def fir_prefill(u, w, state, seq_table, blocks, tile_table, block_t):
    """Depthwise causal FIR over packed prefill rows, carrying per-sequence state.

    u: (T, H) bf16 packed rows.  w: (H, K) cross-correlation order (w[:, -1]
    pairs with the current sample).  state: (blocks, H, >=K-1) fp32, any
    strides.  seq_table: (n, 3) int32 [start, end, has_initial_state].
    blocks: (n,) state block per segment, any stride.  tile_table: (ntiles, 2)
    int32 [segment, first row] built for `block_t` (`fir_prefill_block_t`).

    Returns the filter output (T, H) bf16 and writes each segment's final
    (K-1)-input window into `state` (triton_prefill.py:462-496).
    """
    _lib.require_device(u, w, state, seq_table, blocks, tile_table)
    T, H = u.shape
    K = w.shape[1]
    if u.stride(1) != 1:
        raise ValueError("rows are addressed as t * stride(0) + channel")
    if u.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or state.dtype != torch.float32:
        raise ValueError("u and w must be bf16, state fp32")
    _check_tables(seq_table, tile_table)
    blocks = blocks if blocks.dtype == torch.int32 else blocks.to(torch.int32)
    w = w.contiguous()
    out = torch.empty(T, H, dtype=u.dtype, device=u.device)
    _lib.call(
        "evo2_fir_prefill",
        _lib.ptr(u), u.stride(0), _lib.ptr(w), w.stride(0), w.stride(1),
        K, _lib.ptr(state), *state.stride(),
        _lib.ptr(seq_table), seq_table.shape[0], _lib.ptr(blocks), blocks.stride(0),
        _lib.ptr(tile_table), tile_table.shape[0], int(block_t),
        _lib.ptr(out), out.stride(0), T, H, state.shape[0], _lib.stream_of(u))
    return out


def hyena_fir_prefill(z, short_w, conv_state, w, inner_state, D, seq_table, blocks,
                      tile_table, block_t):
    """g = x2 * (FIR(x1*v) [+ D*(x1*v)]) over packed prefill rows of z.

    z: (T, 3H) bf16 in_proj rows (interleaved x2, x1, v per channel).
    short_w: (3H, 3) bf16.  conv_state: (blocks, 3H, 2) bf16 view.  w: (H, K)
    bf16 inner taps (K = 7 or 128).  inner_state: (blocks, H, >=K-1) fp32
    view.  D: (H,) bf16 or None.  Tables as for `fir_prefill`.
    Returns g (T, H) bf16; both windows are rewritten for every segment.
    """
    _lib.require_device(z, short_w, conv_state, w, inner_state, seq_table, blocks, tile_table)
    T = z.shape[0]
    H, K = w.shape
    if z.shape[1] != 3 * H or z.stride(1) != 1 or z.dtype != torch.bfloat16:
        raise ValueError("z must be (T, 3H) bf16 with unit column stride")
    if short_w.shape != (3 * H, 3) or not short_w.is_contiguous():
        raise ValueError("short_w must be a contiguous (3H, 3) tensor")
    if conv_state.dtype != torch.bfloat16 or inner_state.dtype != torch.float32:
        raise ValueError("conv_state must be bf16 and inner_state fp32")
    _check_tables(seq_table, tile_table)
    if D is not None and (D.dtype != torch.bfloat16 or D.stride(0) != 1):
        D = D.to(torch.bfloat16).contiguous()
    blocks = blocks if blocks.dtype == torch.int32 else blocks.to(torch.int32)
    w = w.contiguous()
    out = torch.empty(T, H, dtype=z.dtype, device=z.device)
    _lib.call(
        "evo2_hyena_fir_prefill",
        _lib.ptr(z), z.stride(0), _lib.ptr(short_w),
        _lib.ptr(conv_state), *conv_state.stride(),
        _lib.ptr(w), w.stride(0), w.stride(1), K,
        _lib.ptr(inner_state), *inner_state.stride(),
        _lib.ptr(D),
        _lib.ptr(seq_table), seq_table.shape[0], _lib.ptr(blocks), blocks.stride(0),
        _lib.ptr(tile_table), tile_table.shape[0], int(block_t),
        _lib.ptr(out), out.stride(0), T, H, min(conv_state.shape[0], inner_state.shape[0]),
        _lib.stream_of(z))
    return out
