"""Speculative verification of the inner Hyena operators (HIP, gfx950).

Drop-in for evo2_flash/triton_verifier.py: `fir_supported`, `fir_snapshots`,
`iir_supported`, `iir_snapshots`, `fir_one` and `iir_one` keep the
reference's signatures and argument meaning (triton_verifier.py:125-178).
`metadata` is the tuple `(ins, outs, starts, ends, accepted)` that
mixers.py's `_decode_tensors` builds: per request, the snapshot blocks of the
previous step, the blocks this step writes after each token, its packed token
range and the previous step's accepted count.  The kernels are in
csrc/verify.hip, reached through `evo2_fir_verify` / `evo2_iir_verify`.

Unlike the reference there is no torch-version gate: the kernels fix their
own reduction order (the reference kernel's, without FMA).
"""

import torch

from . import _lib


def _blocks(state):
    return state.shape[0]


def fir_supported(x, weight, state):
    """Whether `fir_snapshots` / `fir_one` take these tensors (triton_verifier.py:125-130)."""
    if not (x.is_cuda and x.dim() == 2 and x.dtype in (torch.float32, torch.bfloat16)):
        return False
    if not (weight.dim() == 2 and weight.shape[1] in (7, 128) and weight.dtype == torch.bfloat16
            and weight.shape[0] == x.shape[1]):
        return False
    if not (state.dim() == 3 and state.dtype == torch.float32 and state.stride(1) == 1
            and state.shape[1] == x.shape[1] and state.shape[2] >= weight.shape[1] - 1):
        return False
    try:
        _lib.lib()
    except (RuntimeError, OSError):
        return False
    return True


def iir_supported(x, poles, residues, state):
    """Whether `iir_snapshots` / `iir_one` take these tensors (triton_verifier.py:140-143)."""
    if not (x.is_cuda and x.dim() == 2 and x.dtype in (torch.float32, torch.bfloat16)):
        return False
    H = x.shape[1]
    for t in (poles, residues):
        if not (t.shape == (H, 16) and t.dtype == torch.float32 and t.stride(1) == 1
                and t.stride(0) % 4 == 0 and t.data_ptr() % 16 == 0):
            return False
    if not (state.dim() == 3 and state.dtype == torch.float32 and state.shape[1] == H
            and state.shape[2] >= 16 and state.stride(2) == 1):
        return False
    try:
        _lib.lib()
    except (RuntimeError, OSError):
        return False
    return True


def _i32(t):
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _i64(t):
    return (t if t.dtype == torch.int64 else t.to(torch.int64)).contiguous()


def _meta(metadata):
    ins, outs, starts, ends, accepted = metadata
    ins, outs = _i32(ins), _i32(outs)
    if ins.dim() == 1:
        ins = ins[:, None]
    if outs.dim() == 1:
        outs = outs[:, None]
    n = outs.shape[0]
    if ins.shape != outs.shape or not (starts.shape == ends.shape == accepted.shape == (n,)):
        raise ValueError(f"verify metadata shapes disagree: ins {tuple(ins.shape)}, outs "
                         f"{tuple(outs.shape)}, starts/ends/accepted {tuple(starts.shape)}/"
                         f"{tuple(ends.shape)}/{tuple(accepted.shape)}")
    return ins, outs, _i64(starts), _i64(ends), _i64(accepted)


def _fir(x, weight, state, ins, outs, starts, ends, accepted, y, nreq, null_block):
    _lib.call(
        "evo2_fir_verify",
        _lib.ptr(x), *x.stride(), int(x.dtype == torch.float32),
        _lib.ptr(weight), *weight.stride(), weight.shape[1],
        _lib.ptr(state), *state.stride(),
        _lib.ptr(ins), *ins.stride(),
        _lib.ptr(outs), *outs.stride(), outs.shape[1],
        _lib.ptr(starts), _lib.ptr(ends), _lib.ptr(accepted),
        _lib.ptr(y), y.stride(0), nreq, x.shape[0], x.shape[1], int(null_block), _blocks(state),
        _lib.stream_of(x),
    )
    return y


def _iir(x, poles, residues, state, ins, outs, starts, ends, accepted, y, nreq, null_block):
    _lib.call(
        "evo2_iir_verify",
        _lib.ptr(x), *x.stride(), int(x.dtype == torch.float32),
        _lib.ptr(poles), *poles.stride(),
        _lib.ptr(residues), *residues.stride(),
        _lib.ptr(state), *state.stride(),
        _lib.ptr(ins), *ins.stride(),
        _lib.ptr(outs), *outs.stride(), outs.shape[1],
        _lib.ptr(starts), _lib.ptr(ends), _lib.ptr(accepted),
        _lib.ptr(y), y.stride(0), nreq, x.shape[0], x.shape[1], int(null_block), _blocks(state),
        _lib.stream_of(x),
    )
    return y


def fir_snapshots(x, weight, state, metadata, null_block=0):
    """FIR over each request's draft tokens, one window snapshot per token.

    x: (T, H) packed decode tokens (bf16 or fp32).  weight: (H, K) bf16 taps,
    K = 7 or 128.  state: (blocks, H, K-1) fp32 view (unit channel stride),
    read at ins[r][accepted[r] - 1] and written at outs[r][pos].  Returns
    (T, H) in x's dtype, zero on rows no request covers
    (triton_verifier.py:125-135).
    """
    _lib.require_device(x, weight, state)
    ins, outs, starts, ends, accepted = _meta(metadata)
    _lib.require_device(ins, outs, starts, ends, accepted)
    y = torch.zeros(x.shape, dtype=x.dtype, device=x.device)
    return _fir(x, weight, state, ins, outs, starts, ends, accepted, y, ins.shape[0], null_block)


def iir_snapshots(x, poles, residues, state, metadata, null_block=0):
    """The LI recurrence over each request's draft tokens with a state
    snapshot after each (triton_verifier.py:146-155).  poles = exp(log_poles)
    and residues (H, 16) fp32; state (blocks, H, >= 16) fp32 view with unit
    state stride (the speculative layout's 17-column rows included)."""
    _lib.require_device(x, poles, residues, state)
    ins, outs, starts, ends, accepted = _meta(metadata)
    _lib.require_device(ins, outs, starts, ends, accepted)
    y = torch.zeros(x.shape, dtype=x.dtype, device=x.device)
    return _iir(x, poles, residues, state, ins, outs, starts, ends, accepted, y, ins.shape[0],
                null_block)


def fir_one(x, weight, state, slots, null_block=0):
    """One token per request: row r reads and rewrites block slots[r]
    (triton_verifier.py:157-167)."""
    _lib.require_device(x, weight, state, slots)
    s = _i32(slots)[:, None]
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    return _fir(x, weight, state, s, s, None, None, None, y, x.shape[0], null_block)


def iir_one(x, poles, residues, state, slots, null_block=0):
    """One LI update per request on block slots[r] (triton_verifier.py:170-178)."""
    _lib.require_device(x, poles, residues, state, slots)
    s = _i32(slots)[:, None]
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    return _iir(x, poles, residues, state, s, s, None, None, None, y, x.shape[0], null_block)
