"""Hyena-LI (hcl) long convolution on gfx950: chunked 16-pole modal scan.

Keeps the reference's entry points:
  * `hcl_compute_filter(residues, log_poles, t, force_torch=False)`
    (evo2_flash/triton_hcl.py:88-123);
  * `iir_segment(seq, res, lp, s_prev, force_torch=False) -> (y, st)`
    (evo2_flash/mixers.py:144-210), now a scan instead of an FFT convolution;
plus `hyena_hcl_prefill`, the fused prefill core of HyenaIIRMixer
(mixers.py:1327-1401) between in_proj and out_proj.  Kernels:
csrc/prefill_hcl.hip.  `force_torch` is accepted for signature parity and
ignored: there is no torch path.
"""

import torch

from . import _lib
from .prefill import stripe_block_t

# Rows per tile of the chunked scan: shorter tiles add parallelism, longer
# ones amortise the carry pass.  Multiples of 16 (the LDS sub-tile).
_HCL_BLOCK_T = 1024
_TARGET_WORKGROUPS = 1024


def hcl_block_t(num_tokens=None, hidden=None, max_segment=None):
    """Rows per tile for the LI prefill tile table.  A step whose work spreads
    over the GPU in whole segments (`stripe_block_t`) takes the single-pass
    kernel (one tile per segment); otherwise tiles shrink until the tiled
    scan has ~1024 workgroups."""
    bt = stripe_block_t(num_tokens, hidden, max_segment)
    if bt is not None:
        return bt
    bt = _HCL_BLOCK_T
    if num_tokens is not None and hidden is not None:
        groups = max(1, (int(hidden) + 255) // 256)
        while bt > 64 and ((int(num_tokens) + bt - 1) // bt) * groups < _TARGET_WORKGROUPS:
            bt //= 2
    return bt


def _workspace(ntiles, H, device):
    nbytes = _lib.lib().evo2_hcl_workspace_bytes(ntiles, H)
    return torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=device), nbytes


def hcl_compute_filter(residues, log_poles, t, force_torch=False):
    """h[d, l] = sum_s residues[d, s] * exp(log_poles[d, s] * t[l]) -> (D, L) fp32."""
    if residues.dim() != 2 or log_poles.dim() != 2:
        raise ValueError(f"expected 2-D residues and log_poles, got {tuple(residues.shape)} "
                         f"and {tuple(log_poles.shape)}")
    if residues.shape != log_poles.shape:
        raise ValueError(f"residues {tuple(residues.shape)} and log_poles "
                         f"{tuple(log_poles.shape)} must match")
    if t.dim() != 1:
        raise ValueError(f"expected 1-D t, got {tuple(t.shape)}")
    _lib.require_device(residues, log_poles, t)
    D, S = residues.shape
    L = t.shape[0]
    residues = residues.float()
    log_poles = log_poles.float()
    t = t.float()
    h = torch.empty(D, L, dtype=torch.float32, device=residues.device)
    _lib.call("evo2_hcl_compute_filter",
              _lib.ptr(residues), *residues.stride(), _lib.ptr(log_poles), *log_poles.stride(),
              _lib.ptr(t), t.stride(0), _lib.ptr(h), *h.stride(), D, S, L,
              _lib.stream_of(residues))
    return h


def iir_segment(seq, res, lp, s_prev, force_torch=False, block_t=None):
    """One prefill segment of the diagonal LTI SSM s_t = p*s_{t-1} + x_t.

    seq: (H, L) fp32 inputs (any strides; the mixer passes a token-major
    view).  res, lp: (H, S=16).  s_prev: (H, S) state inherited from an
    earlier segment, or None.  Returns (y (H, L), s_last (H, S)) as
    mixers.py:144-210 does; y is a transposed view of a token-major buffer.
    """
    _lib.require_device(seq, res, lp, s_prev)
    H, L = seq.shape
    if res.shape != (H, 16) or lp.shape != (H, 16):
        raise ValueError("the LI scan takes 16 poles per channel")
    if seq.dtype != torch.float32:
        seq = seq.float()
    res = res.float()
    lp = lp.float()
    bt = int(block_t or hcl_block_t(L, H))
    ntiles = (L + bt - 1) // bt
    ybuf = torch.empty(L, H, dtype=torch.float32, device=seq.device)
    y = ybuf.t()
    st = torch.empty(H, 16, dtype=torch.float32, device=seq.device)
    work, nbytes = _workspace(ntiles, H, seq.device)
    sp = None if s_prev is None else s_prev.float()
    _lib.call("evo2_iir_segment",
              _lib.ptr(seq), *seq.stride(), _lib.ptr(res), *res.stride(),
              _lib.ptr(lp), *lp.stride(),
              _lib.ptr(sp), *(sp.stride() if sp is not None else (0, 0)),
              _lib.ptr(y), *y.stride(), _lib.ptr(st), _lib.ptr(work), nbytes,
              H, L, bt, _lib.stream_of(seq))
    return y, st


def iir_final_state(seq, lp, blk=None, block_t=None):
    """s[h, s] = sum_t seq[h, t] * p[h, s]^(L-1-t), p = exp(lp): the final
    state of one LI segment started from zero (triton_prefill.py:351-387).

    seq: (H, L) fp32, any strides (the mixer passes a token-major view).
    lp: (H, 16) log-poles.  `blk` (the reference's torch blocking of the state
    channels, which fixes torch's summation order) is accepted and unused:
    the state is the scan's, s_t = p*s_{t-1} + x_t in fp32, equal to the
    closed form within fp32 rounding rather than bit for bit.  Returns (H, 16)
    fp32, or None where the reference does too (a CPU or non-fp32 `seq`: the
    caller's torch path).
    """
    if not (seq.is_cuda and seq.dtype == torch.float32):
        return None
    _lib.require_device(lp)
    H, L = seq.shape
    if lp.shape != (H, 16):
        raise ValueError("the LI scan takes 16 poles per channel")
    lp = lp.float()
    bt = int(block_t or hcl_block_t(L, H))
    ntiles = (L + bt - 1) // bt
    st = torch.empty(H, 16, dtype=torch.float32, device=seq.device)
    work, nbytes = _workspace(ntiles, H, seq.device)
    _lib.call("evo2_iir_final_state",
              _lib.ptr(seq), *seq.stride(), _lib.ptr(lp), *lp.stride(), _lib.ptr(st),
              _lib.ptr(work), nbytes, H, L, bt, _lib.stream_of(seq))
    return st


def hyena_hcl_prefill(z, short_w, conv_state, residues, log_poles, ssm, D, seq_table, blocks,
                      tile_table, tile_start, block_t):
    """g = bf16(bf16(bf16(y) + bf16(u*D)) * x2) over packed prefill rows of z,
    with y the 16-pole LI response to u = x1*v (HyenaIIRMixer prefill,
    mixers.py:1327-1401).  Writes each segment's final state into `ssm` and
    its conv window into `conv_state`.

    z: (T, 3H) bf16.  short_w: (3H, 3) bf16.  conv_state: (blocks, 3H, 2)
    bf16 view.  residues, log_poles: (H, 16) fp32.  ssm: (blocks, H, 16) fp32
    view.  D: (H,).  seq_table (n, 3), tile_table (ntiles, 2) and tile_start
    (n + 1) int32, built for `block_t` (a multiple of 16).  Returns g (T, H) bf16.
    """
    _lib.require_device(z, short_w, conv_state, residues, log_poles, ssm, D, seq_table, blocks,
                        tile_table, tile_start)
    T = z.shape[0]
    H = residues.shape[0]
    if z.shape[1] != 3 * H or z.stride(1) != 1 or z.dtype != torch.bfloat16:
        raise ValueError("z must be (T, 3H) bf16 with unit column stride")
    if short_w.shape != (3 * H, 3) or not short_w.is_contiguous():
        raise ValueError("short_w must be a contiguous (3H, 3) tensor")
    if residues.shape != (H, 16) or log_poles.shape != (H, 16):
        raise ValueError("residues and log_poles must be (H, 16)")
    for name, t, w in (("seq_table", seq_table, 3), ("tile_table", tile_table, 2)):
        if t.dtype != torch.int32 or t.dim() != 2 or t.shape[1] != w or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous (n, {w}) int32 tensor")
    if tile_start.dtype != torch.int32 or tile_start.numel() != seq_table.shape[0] + 1:
        raise ValueError("tile_start must be (n + 1,) int32")
    tile_start = tile_start.contiguous()
    residues, log_poles = residues.float(), log_poles.float()
    D = D.to(torch.bfloat16).contiguous()
    blocks = blocks if blocks.dtype == torch.int32 else blocks.to(torch.int32)
    ntiles = tile_table.shape[0]
    work, nbytes = _workspace(ntiles, H, z.device)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=z.device)
    _lib.call("evo2_hyena_hcl_prefill",
              _lib.ptr(z), z.stride(0), _lib.ptr(short_w),
              _lib.ptr(conv_state), *conv_state.stride(),
              _lib.ptr(residues), *residues.stride(), _lib.ptr(log_poles), *log_poles.stride(),
              _lib.ptr(ssm), *ssm.stride(), _lib.ptr(D),
              _lib.ptr(seq_table), seq_table.shape[0], _lib.ptr(blocks), blocks.stride(0),
              _lib.ptr(tile_table), ntiles, _lib.ptr(tile_start), int(block_t),
              _lib.ptr(work), nbytes,
              _lib.ptr(out), out.stride(0), T, H, min(conv_state.shape[0], ssm.shape[0]),
              _lib.stream_of(z))
    return out
