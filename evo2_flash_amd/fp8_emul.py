"""Hopper fp8 fast-accumulation GEMM model on gfx950 (csrc/fp8_emul.hip).

The FP8-surgery projections of the released checkpoints (config.py:81-94:
`hyena_fp8_emulated_layers`, `hyena_fp8_emulated_channels`) run their fp8
in_proj through a software model of the sm_90 tensor-core accumulator, which
is not fp32 (fp8_emul.py:1-24).  These wrappers keep the reference's
signatures (fp8_emul_triton.py:142-191) and reproduce its arithmetic bit for
bit: groups of 32 k, alignment to the largest operand exponent sum (or the
accumulator's), 13 fraction bits, truncation toward zero.
"""

import torch

from . import _lib
from .fp8 import E4M3, quantize_input

GROUP = 32


def fast_accum_mm(a8, b_t, out=None):
    """The raw fp32 accumulator (N, M) of a8 (N, K) e4m3 times b_t (K, M), a
    bf16 tensor holding E4M3 values (K-major)."""
    _lib.require_device(a8, b_t)
    if a8.dtype != E4M3 or b_t.dtype != torch.bfloat16:
        raise ValueError("fast_accum_mm takes e4m3 activations and a bf16 (K, M) weight")
    N, K = a8.shape
    K2, M = b_t.shape
    if K != K2 or K % GROUP:
        raise ValueError(f"K mismatch or not a multiple of {GROUP}: {a8.shape} x {b_t.shape}")
    if a8.stride(1) != 1:
        a8 = a8.contiguous()
    if b_t.stride(1) != 1:
        b_t = b_t.contiguous()
    if out is None:
        out = torch.empty(N, M, dtype=torch.float32, device=a8.device)
    _lib.call("evo2_fp8_fast_accum_gemm", _lib.ptr(a8), a8.stride(0), _lib.ptr(b_t), b_t.stride(0),
              None, None, _lib.ptr(out), out.stride(0), 1, N, M, K, _lib.stream_of(a8))
    return out


def static_fp8_linear_emulated(x, w_t_e4m3_values, input_scale, weight_scale):
    """Emulated static W8A8 linear, (..., K) -> (..., M) in x's dtype
    (fp8_emul_triton.py:181-191): e4m3(clamp(x / input_scale)) times the
    E4M3-valued (K, M) weight through the fast-accumulation model, then
    (acc * input_scale) * weight_scale."""
    K = x.shape[-1]
    M = w_t_e4m3_values.shape[1]
    _lib.require_device(x, w_t_e4m3_values, input_scale, weight_scale)
    if x.dtype != torch.bfloat16:
        raise ValueError("the emulated fp8 linear takes bf16 activations (the mixers' dtype)")
    if w_t_e4m3_values.dtype != torch.bfloat16 or w_t_e4m3_values.shape[0] != K or K % GROUP:
        raise ValueError(f"expected a bf16 ({K}, M) weight with K a multiple of {GROUP}")
    b_t = w_t_e4m3_values if w_t_e4m3_values.stride(1) == 1 else w_t_e4m3_values.contiguous()
    x8 = quantize_input(x.reshape(-1, K), input_scale)
    sx = input_scale.to(torch.float32).reshape(1)
    sw = weight_scale.to(torch.float32).reshape(1)
    out = torch.empty(x8.shape[0], M, dtype=torch.bfloat16, device=x.device)
    _lib.call("evo2_fp8_fast_accum_gemm", _lib.ptr(x8), x8.stride(0), _lib.ptr(b_t),
              b_t.stride(0), _lib.ptr(sx), _lib.ptr(sw), _lib.ptr(out), out.stride(0), 0,
              x8.shape[0], M, K, _lib.stream_of(x))
    return out.reshape(*x.shape[:-1], M)


# The reference's name for the same entry point.
static_fp8_linear_emulated_triton = static_fp8_linear_emulated
