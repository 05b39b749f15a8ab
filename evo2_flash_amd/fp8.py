"""fp8 e4m3 projections on gfx950 MFMA (static per-tensor scales, fp32 accumulate).

The reference's in_proj is vLLM's static W8A8 `ReplicatedLinear` built from
`Fp8Config(is_checkpoint_fp8_serialized=True, activation_scheme="static")`
(mixers.py:741-757, 780-783): x is quantised as e4m3fn(clamp(x / input_scale,
+-448)) (fp8_emul.py:76-78), multiplied by the e4m3 weight with fp32
accumulation, and scaled by input_scale * weight_scale (dequantisation
convention, convert.py:195-201).  The checkpoint tensors are
`in_proj.weight` (3H, H) float8_e4m3fn, `in_proj.weight_scale` (1,) and
`in_proj.input_scale` (1,).  Kernels: csrc/fp8_gemm.hip.
"""

import torch
from torch import nn

from . import _lib

FP8_MAX = 448.0
E4M3 = torch.float8_e4m3fn


def quantize_input(x, input_scale):
    """e4m3fn(clamp(x / input_scale, -448, 448)) of a (..., K) bf16 tensor."""
    _lib.require_device(x, input_scale)
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16).contiguous()
    scale = input_scale.to(torch.float32).reshape(1)
    q = torch.empty(x2.shape, dtype=E4M3, device=x.device)
    _lib.call("evo2_fp8_quantize", _lib.ptr(x2), x2.stride(0), _lib.ptr(q), q.stride(0),
              _lib.ptr(scale), x2.shape[0], K, _lib.stream_of(x))
    return q.reshape(x.shape)


def fp8_gemm(x8, w8, x_scale, w_scale, bias=None, out=None):
    """bf16((x8 @ w8^T) * x_scale * w_scale [+ bias]) with x8 (M, K), w8 (N, K) e4m3."""
    _lib.require_device(x8, w8, x_scale, w_scale, bias)
    if x8.dtype != E4M3 or w8.dtype != E4M3:
        raise ValueError("fp8_gemm operands must be float8_e4m3fn")
    M, K = x8.shape
    N, K2 = w8.shape
    if K != K2:
        raise ValueError(f"K mismatch: {K} vs {K2}")
    if x8.stride(1) != 1:
        x8 = x8.contiguous()
    if w8.stride(1) != 1:
        w8 = w8.contiguous()
    xs = x_scale.to(torch.float32).reshape(1)
    ws = w_scale.to(torch.float32).reshape(1)
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=x8.device)
    elif (out.dtype != torch.bfloat16 or out.shape != (M, N) or out.stride(1) != 1
          or out.device != x8.device):
        raise ValueError(f"fp8_gemm: out must be ({M}, {N}) bf16 on {x8.device} with unit "
                         f"column stride, got {tuple(out.shape)} {out.dtype} stride {out.stride()}")
    _lib.call("evo2_fp8_gemm", _lib.ptr(x8), x8.stride(0), _lib.ptr(w8), w8.stride(0),
              _lib.ptr(xs), _lib.ptr(ws), _lib.ptr(bias), _lib.ptr(out), out.stride(0),
              M, N, K, _lib.stream_of(x8))
    return out


STREAM_MAX_WORK = 60000  # evo2_fp8_gemm streams the weight while ceil(M / 64) * N <= this


def streams_weight(M, N):
    """Whether evo2_fp8_gemm takes its weight-streaming kernel for M rows
    (always at M <= 64; over 64-row blocks while ceil(M / 64) * N is at most
    STREAM_MAX_WORK): the shapes where a packed weight copy is read instead."""
    return 0 < M and (M <= 64 or -(-M // 64) * N <= STREAM_MAX_WORK)


def packable(N, K):
    """Whether an (N, K) weight has a decode layout (fp8_pack_weight)."""
    return N % 16 == 0 and K % 128 == 0


def fp8_pack_weight(w8):
    """The decode layout of an (N, K) e4m3 weight (N a multiple of 16, K of
    128): each 16-row group's 128-byte K step as one contiguous 2 KB block,
    in the order the decode GEMM loads it.  Returned as an (N, K) e4m3
    tensor whose bytes are in that order (only fp8_gemm_packed reads it)."""
    _lib.require_device(w8)
    if w8.dtype != E4M3 or w8.dim() != 2:
        raise ValueError("fp8_pack_weight: w8 must be an (N, K) float8_e4m3fn tensor")
    N, K = w8.shape
    if not packable(N, K):
        raise ValueError(f"fp8_pack_weight: N={N} must be a multiple of 16 and K={K} of 128")
    if w8.stride(1) != 1 or w8.stride(0) % 16:
        w8 = w8.contiguous()
    wp = torch.empty(N, K, dtype=E4M3, device=w8.device)
    _lib.call("evo2_fp8_pack_weight", _lib.ptr(w8), w8.stride(0), _lib.ptr(wp), N, K,
              _lib.stream_of(w8))
    return wp


def fp8_gemm_packed(x8, wp, x_scale, w_scale, bias=None, out=None):
    """fp8_gemm with the weight in the decode layout (fp8_pack_weight); the
    same result bits.  Streams the weight once per 64-row block of x, so it
    is for the shapes streams_weight() accepts (decode and verify steps)."""
    _lib.require_device(x8, wp, x_scale, w_scale, bias)
    if x8.dtype != E4M3 or wp.dtype != E4M3:
        raise ValueError("fp8_gemm_packed operands must be float8_e4m3fn")
    M, K = x8.shape
    N, K2 = wp.shape
    if K != K2 or not wp.is_contiguous():
        raise ValueError(f"fp8_gemm_packed: wp must be a packed (N, {K}) weight")
    if x8.stride(1) != 1:
        x8 = x8.contiguous()
    xs = x_scale.to(torch.float32).reshape(1)
    ws = w_scale.to(torch.float32).reshape(1)
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=x8.device)
    elif (out.dtype != torch.bfloat16 or out.shape != (M, N) or out.stride(1) != 1
          or out.device != x8.device):
        raise ValueError(f"fp8_gemm_packed: out must be ({M}, {N}) bf16 on {x8.device} with "
                         f"unit column stride, got {tuple(out.shape)} {out.dtype}")
    _lib.call("evo2_fp8_gemm_packed", _lib.ptr(x8), x8.stride(0), _lib.ptr(wp),
              _lib.ptr(xs), _lib.ptr(ws), _lib.ptr(bias), _lib.ptr(out), out.stride(0),
              M, N, K, _lib.stream_of(x8))
    return out


def static_fp8_linear(x, weight, input_scale, weight_scale, bias=None, out=None, packed=None):
    """vLLM's static W8A8 linear: (..., K) bf16 -> (..., N) bf16; a 2-D x may
    write its result into `out` (M, N) bf16 with unit column stride.  With
    `packed` (fp8_pack_weight(weight)), inputs of at most 64 rows take the
    decode GEMM on it wherever the weight would be streamed (the same result
    bits)."""
    K = x.shape[-1]
    x8 = quantize_input(x.reshape(-1, K), input_scale)
    gemm = fp8_gemm
    w = weight
    if packed is not None and streams_weight(x8.shape[0], weight.shape[0]):
        gemm, w = fp8_gemm_packed, packed
    if out is not None:
        if x.dim() != 2 or out.shape != (x.shape[0], weight.shape[0]) or out.stride(1) != 1:
            raise ValueError("static_fp8_linear: out must be (M, N) with unit column stride")
        return gemm(x8, w, input_scale, weight_scale, bias, out=out)
    out = gemm(x8, w, input_scale, weight_scale, bias)
    return out.reshape(*x.shape[:-1], weight.shape[0])


class Fp8StaticLinear(nn.Module):
    """Replicated static-W8A8 linear with the checkpoint's tensor names.

    `forward(x) -> (y, None)` like vLLM's ReplicatedLinear, so mixer code and
    forward hooks see the projection output unchanged.
    """

    def __init__(self, in_features, out_features, bias=False, device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=E4M3,
                                               device=device), requires_grad=False)
        self.weight_scale = nn.Parameter(torch.ones(1, dtype=torch.float32, device=device),
                                         requires_grad=False)
        self.input_scale = nn.Parameter(torch.ones(1, dtype=torch.float32, device=device),
                                        requires_grad=False)
        self.bias = (nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16, device=device),
                                  requires_grad=False) if bias else None)
        # The engine's loader calls `param.weight_loader(param, tensor)` when a
        # parameter has one (a plain `param.data.copy_` would not be seen by
        # the decode copy below).
        self.weight.weight_loader = self._load_weight

    # The decode-layout copy costs N*K bytes per projection.  False keeps
    # every call on the row-major weight (the same result bits) and makes no
    # copy, for deployments that cannot spare the memory.
    decode_copies = True

    def process_weights_after_loading(self):
        """Make the decode copy now (or rewrite it in place), so that it exists
        before an engine measures free memory to size its pools."""
        self.decode_weight()

    def _load_weight(self, param, loaded):
        """Copy a checkpoint tensor into the weight and rewrite the decode copy
        in place (a HIP graph captured before the reload reads the new
        weight)."""
        param.data.copy_(loaded.to(param.dtype).view_as(param))
        self.refresh_decode_weight()

    def refresh_decode_weight(self):
        """Rewrite an existing decode copy from the current weight, in place;
        code that writes the weight other than through its weight_loader or
        in-place tensor ops (`.data`) calls this afterwards."""
        cached = getattr(self, "_decode_w", None)
        if cached is None:
            return
        w, wp = self.weight.detach(), cached[1]
        if w.shape != wp.shape or w.device != wp.device or not packable(*w.shape):
            self._decode_w = None
            return
        if w.stride(1) != 1 or w.stride(0) % 16:
            w = w.contiguous()
        _lib.call("evo2_fp8_pack_weight", _lib.ptr(w), w.stride(0), _lib.ptr(wp), w.shape[0],
                  w.shape[1], _lib.stream_of(w))
        self._decode_w = ((self.weight.data_ptr(), self.weight._version), wp)

    def decode_weight(self):
        """The weight in the decode layout (kept beside the checkpoint copy;
        not state).  Made once; after the weight changes in place it is
        rewritten into the same buffer, so a HIP graph captured on it reads
        the new weight once one eager call (or refresh_decode_weight()) has
        run.  None while a HIP graph is being captured and the copy is
        missing or stale, for shapes without a decode layout, and when
        decode_copies is off."""
        w = self.weight
        if not self.decode_copies or not packable(*w.shape) or not w.is_cuda:
            return None
        key = (w.data_ptr(), w._version)
        cached = getattr(self, "_decode_w", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        if torch.cuda.is_current_stream_capturing():
            return None
        if cached is not None:
            self.refresh_decode_weight()  # in place when shape and device match
            if self._decode_w is not None:
                return self._decode_w[1]
        wp = fp8_pack_weight(w.detach())
        self._decode_w = (key, wp)
        return wp

    def forward(self, x, out=None):
        rows = x.numel() // max(x.shape[-1], 1)
        packed = self.decode_weight() if streams_weight(rows, self.out_features) else None
        return static_fp8_linear(x, self.weight, self.input_scale, self.weight_scale,
                                 self.bias, out=out, packed=packed), None
