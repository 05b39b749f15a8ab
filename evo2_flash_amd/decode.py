"""Fused single-token Hyena decode step (HIP, gfx950).

Drop-in for evo2_flash/triton_decode.py: `decode_supported` and
`hyena_decode` keep the reference's signatures, argument meaning and return
values (triton_decode.py:167-211).  The kernel is `hyena_decode_kernel` in
csrc/decode.hip, reached through `evo2_hyena_decode` in the C ABI.

Rounding points are the reference's: the short filter rounds each product
to bf16 and the sum to bf16, u = x1*v, D*u, y + D*u and x2*y are bf16 after
every op, the inner FIR sums in the reference's fixed order without FMA
contraction, and the LI state is s*exp(lp) + u in fp32.
"""

import torch

from . import _lib


def decode_supported(z, short_w, conv_state, inner, inner_state, D=None, log_poles=None):
    """Whether `hyena_decode` handles these tensors (triton_decode.py:167-182).

    Unlike the reference there is no torch-version gate: the HIP kernel fixes
    its own reduction order.  It does require ROCm tensors and the built library.
    """
    H = inner.shape[0]
    iir = log_poles is not None
    if not (z.is_cuda and z.dtype == torch.bfloat16 and z.dim() == 2 and z.stride(-1) == 1):
        return False
    if not (short_w.shape == (3 * H, 3) and short_w.is_contiguous()
            and short_w.dtype == torch.bfloat16):
        return False
    if not (conv_state.dtype == torch.bfloat16 and conv_state.dim() == 3
            and conv_state.shape[-1] == 2 and conv_state.shape[1] == 3 * H):
        return False
    if not (inner_state.dtype == torch.float32 and inner_state.dim() == 3
            and inner_state.shape[1] == H):
        return False
    if D is not None and D.dtype != torch.bfloat16:
        return False
    if iir:
        if not (inner.shape[1] == 16 and inner.dtype == torch.float32
                and log_poles.dtype == torch.float32 and log_poles.shape == (H, 16)
                and inner_state.shape[2] >= 16):
            return False
    elif not (inner.shape[1] in (7, 128) and inner.dtype == torch.bfloat16
              and inner_state.shape[2] >= inner.shape[1] - 1):
        return False
    try:
        _lib.lib()
    except (RuntimeError, OSError):
        return False
    return True


def channel_major_taps(w):
    """The FIR taps (H, K) as a view over channel-contiguous (K, H) storage.

    Same values and shape as `w`; only the memory order changes, so tap k of
    neighbouring channels is contiguous and the decode kernel reads each tap
    column as one coalesced sweep.  The mixers keep their decode taps in this
    layout (made once when the weights are loaded).
    """
    return w.t().contiguous().t()


def hyena_decode(z, short_w, conv_state, slots, inner, inner_state, D=None,
                 log_poles=None, null_block=0):
    """x2 * (inner(x1*v) + D*(x1*v)) for one decode token per row; states in place.

    z: (B, 3H) bf16 in_proj rows.  short_w: (3H, 3).  conv_state: (blocks, 3H, 2)
    bf16, any strides.  slots: (B,) block per row (a strided view is fine).
    inner: the FIR taps (H, 7 | 128), or the LI residues (H, 16) when
    `log_poles` (H, 16) is given.  inner_state: (blocks, H, K-1 | 16) fp32 view.
    D: (H,) or None.  Returns (B, H) bf16 (triton_decode.py:185-211).
    """
    B, H = z.shape[0], inner.shape[0]
    if slots.dim() != 1 or slots.shape[0] < B:
        raise ValueError(f"hyena_decode needs one state block per row: slots has shape "
                         f"{tuple(slots.shape)} for {B} rows")
    _lib.require_device(z, conv_state, inner, inner_state, slots)
    out = torch.empty(B, H, dtype=z.dtype, device=z.device)
    if not B:
        return out
    is_iir = log_poles is not None
    K = inner.shape[1]
    if slots.dtype != torch.int32:
        slots = slots.to(torch.int32)
    if D is not None and D.stride(0) != 1:
        D = D.contiguous()
    lp = log_poles if is_iir else None
    _lib.call(
        "evo2_hyena_decode",
        _lib.ptr(z), z.stride(0), _lib.ptr(short_w),
        _lib.ptr(conv_state), *conv_state.stride(),
        _lib.ptr(slots), slots.stride(0),
        _lib.ptr(inner), *inner.stride(),
        _lib.ptr(lp), *(lp.stride() if lp is not None else (0, 0)),
        _lib.ptr(inner_state), *inner_state.stride(),
        _lib.ptr(D), _lib.ptr(out), out.stride(0),
        B, H, K, int(is_iir), int(null_block), min(conv_state.shape[0], inner_state.shape[0]),
        _lib.stream_of(z),
    )
    return out
