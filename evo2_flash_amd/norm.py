"""Evo2RMSNorm on gfx950 (csrc/norm.hip).

`rms_norm` keeps the signature of evo2_flash/triton_norm.py:125-156 and the
contract of Evo2RMSNorm (model.py:47-74): y = w * s / (||s||_2 * H^-1/2 + eps)
with eps outside the sqrt, s = x (+ residual), bf16 after every op.  With a
residual it returns (y, s).  `rms_norm_fp8` adds the activation quantisation
of the fp8 in_proj that consumes the pre-norm output, in the same pass.
"""

import torch

from . import _lib

E4M3 = torch.float8_e4m3fn


def _rows(t, H, name):
    if t.shape[-1] != H or t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit-stride rows of {H}")
    try:
        return t.view(-1, H)
    except RuntimeError as e:
        raise ValueError(f"{name} rows must share one stride") from e


def _norm(x, weight, eps, residual, input_scale, want_y):
    _lib.require_device(x, weight, residual, input_scale)
    H = x.shape[-1]
    if x.dtype != torch.bfloat16 or (residual is not None and residual.dtype != torch.bfloat16):
        raise ValueError("rms_norm takes bf16 rows")
    if residual is not None and residual.shape != x.shape:
        raise ValueError(f"residual {tuple(residual.shape)} must match x {tuple(x.shape)}")
    x2 = _rows(x, H, "x")
    r2 = None if residual is None else _rows(residual, H, "residual")
    w = weight.to(torch.bfloat16).contiguous()
    T = x2.shape[0]
    y = torch.empty(T, H, dtype=torch.bfloat16, device=x.device) if want_y else None
    s = torch.empty(T, H, dtype=torch.bfloat16, device=x.device) if r2 is not None else None
    q = qs = None
    if input_scale is not None:
        qs = input_scale.to(torch.float32).reshape(1)
        q = torch.empty(T, H, dtype=E4M3, device=x.device)
    _lib.call("evo2_rms_norm", _lib.ptr(x2), x2.stride(0),
              _lib.ptr(r2), r2.stride(0) if r2 is not None else 0,
              _lib.ptr(w), float(eps), _lib.ptr(y), H, _lib.ptr(s), H,
              _lib.ptr(qs), _lib.ptr(q), H, T, H, _lib.stream_of(x))
    shape = x.shape
    return (None if y is None else y.view(shape), None if s is None else s.view(shape),
            None if q is None else q.view(shape))


def rms_norm(x, weight, eps, residual=None):
    """weight * s / (||s||_2 * H^-1/2 + eps), s = x (+ residual); returns y,
    or (y, s) with a residual (triton_norm.py:125-156)."""
    y, s, _ = _norm(x, weight, eps, residual, None, True)
    return y if residual is None else (y, s)


def rms_norm_fp8(x, weight, eps, input_scale, residual=None, keep_y=False):
    """The norm and the static e4m3 quantisation of its output in one pass:
    returns q = e4m3(clamp(y / input_scale, +-448)), then y if `keep_y`, then
    s if a residual is given."""
    y, s, q = _norm(x, weight, eps, residual, input_scale, keep_y)
    out = (q,)
    if keep_y:
        out += (y,)
    if residual is not None:
        out += (s,)
    return out if len(out) > 1 else q


class Evo2RMSNorm(torch.nn.Module):
    """Drop-in for evo2_flash's Evo2RMSNorm (model.py:47-74): `weight` (H,),
    `eps`; forward(x, residual=None) -> y | (y, x + residual)."""

    def __init__(self, hidden_size, eps, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
        self.eps = eps
        self.hidden_size = hidden_size

    def forward(self, x, residual=None):
        return rms_norm(x, self.weight, self.eps, residual)
