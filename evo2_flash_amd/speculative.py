"""Host plumbing of speculative decode for the Hyena mixers.

A verify step packs each decode request's anchor token and drafts into
consecutive rows; request r owns rows query_start_loc_d[r] ..
query_start_loc_d[r+1]-1 and the slot row state_indices_tensor_d[r, :] of
1 + num_spec blocks.  The inner FIR and LI operators keep one full snapshot
per block: the step reads the snapshot in column accepted-1 (the state after
the previous step's last accepted token) and writes the state after its
token p into column p.  The short filter keeps vLLM's sliding window in
column 0 instead (`short_conv.causal_conv1d_update`, speculative form).

Which snapshot is live is resolved from position stamps, not from vLLM's
acceptance counts (mixers.py:17-28): every block carries in slice 2 row 0,
last column, the number of tokens its snapshot represents; a request that
has computed n' tokens finds its live snapshot at offset n' - stamp(column 0)
(mixers.py:960-999).  Each piece is one small launch (csrc/spec.hip) over
device tensors with no host synchronisation, so it can sit inside a
captured step: the accepted counts from the stamps, the step's verify plan
(snapshot blocks per position, packed row ranges, the engine's counts), the
stamps a step writes, and align-mode prefix caching's repair of resumed
prefill states.

Stamp mismatches (a request whose stamps do not match its computed-token
count) are counted in a device tensor the caller reads when it chooses
(`HyenaMixerBase.stamp_faults`), where the reference raises a device-side
assert: on ROCm such an assert aborts the whole process from inside a kernel.
"""

import ctypes
from typing import NamedTuple

import torch

from . import _lib


def _i32(t):
    """int32 and contiguous (a copy only when needed)."""
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def spec_accepted(stamps, slots, computed, num_spec, faults, counts=None):
    """(nreq,) int64 accepted counts of the previous step from the position
    stamps, one launch (mixers.py:960-999): request r finds offset =
    computed[r] - stamps[slots[r, 0]]; accepted = clamp(offset, 0,
    num_spec) + 1.  A request not on the null block whose offset is outside
    [0, num_spec] (or, with `counts`, disagrees with the engine's count) adds
    one to `faults`, an int64 device scalar; a slot outside the pool also
    counts.  `slots` None puts every request on the null block.

    stamps: (blocks,) fp32 view (any stride); slots (nreq, cols) or (nreq,)
    int32; computed (nreq,) tokens computed before the step."""
    _lib.require_device(stamps, slots, computed, faults, counts)
    nreq = computed.shape[0]
    if stamps.dim() != 1 or stamps.dtype != torch.float32:
        raise ValueError(f"stamps must be a (blocks,) fp32 view, got {tuple(stamps.shape)} "
                         f"{stamps.dtype}")
    if faults.dtype != torch.int64 or faults.numel() != 1:
        raise ValueError("faults must be one int64 element")
    if slots is not None:
        slots = slots if slots.dim() == 2 else slots[:, None]
        if slots.shape[0] < nreq:
            raise ValueError(f"slot rows={slots.shape[0]} < requests={nreq}")
        if slots.dtype != torch.int32:
            slots = slots.to(torch.int32)
    if counts is not None and counts.shape[0] < nreq:
        raise ValueError(f"counts holds {counts.shape[0]} entries for {nreq} requests")
    # converted copies stay bound until the launch is queued
    computed = _i32(computed[:nreq])
    counts = None if counts is None else _i32(counts[:nreq])
    acc = torch.empty(nreq, dtype=torch.int64, device=computed.device)
    _lib.call("evo2_spec_accepted", _lib.ptr(stamps), stamps.stride(0), stamps.shape[0],
              _lib.ptr(slots), 0 if slots is None else slots.stride(0), _lib.ptr(computed),
              _lib.ptr(counts), int(num_spec), nreq, _lib.ptr(acc), _lib.ptr(faults),
              _lib.stream_of(computed))
    return acc


def record_stamps(stamps, slots, qsl, computed, width, out_col=None, prefill_blocks=None,
                  seq_lens=None):
    """Stamp the snapshots a step wrote, one launch (mixers.py:1049-1074):
    decode request r (rows qsl[r] .. qsl[r+1]-1, computed n tokens) stamps
    block slots[r, out_col[r] + p] with n + p + 1 for p < min(width, its
    query length); prefill block prefill_blocks[j] gets seq_lens[j].  The
    null block, slots outside the pool and columns past the slot row are not
    written.  `slots` None (every decode request on the null block) writes
    no decode stamp."""
    _lib.require_device(stamps, slots, qsl, computed, out_col, prefill_blocks, seq_lens)
    if stamps.dim() != 1 or stamps.dtype != torch.float32:
        raise ValueError(f"stamps must be a (blocks,) fp32 view, got {tuple(stamps.shape)} "
                         f"{stamps.dtype}")
    nreq = 0 if qsl is None else qsl.shape[0] - 1
    if slots is not None:
        slots = slots if slots.dim() == 2 else slots[:, None]
        if slots.shape[0] < nreq:
            raise ValueError(f"slot rows={slots.shape[0]} < requests={nreq}")
        if slots.dtype != torch.int32:
            slots = slots.to(torch.int32)
    npf = 0 if prefill_blocks is None else prefill_blocks.shape[0]
    if npf and (seq_lens is None or seq_lens.shape[0] < npf):
        raise ValueError("prefill stamps need one sequence length per block")
    for t, what in ((computed, "computed"), (out_col, "out_col")):
        if nreq and t is not None and t.shape[0] < nreq:
            raise ValueError(f"{what} holds {t.shape[0]} entries for {nreq} requests")
    # converted copies stay bound until the launch is queued
    out_col = None if out_col is None or not nreq else _i32(out_col[:nreq])
    qsl = None if not nreq else _i32(qsl)
    computed = None if computed is None or not nreq else _i32(computed[:nreq])
    prefill_blocks = None if not npf else _i32(prefill_blocks)
    seq_lens = None if not npf else _i32(seq_lens[:npf])
    _lib.call("evo2_spec_record_stamps", _lib.ptr(stamps), stamps.stride(0), stamps.shape[0],
              _lib.ptr(slots), 0 if slots is None else slots.stride(0),
              0 if slots is None else slots.stride(1), 0 if slots is None else slots.shape[1],
              _lib.ptr(out_col), _lib.ptr(qsl), _lib.ptr(computed), nreq,
              int(width) if nreq else 0, _lib.ptr(prefill_blocks), _lib.ptr(seq_lens), npf,
              _lib.stream_of(stamps))


class VerifyPlan(NamedTuple):
    """What the snapshot operators need about a step's decode requests,
    besides the stamp-derived accepted counts: input and output snapshot
    blocks per verifier position, the packed row range of each request, and
    the engine's accepted counts (>= 1; ones when the step sends none)."""
    ins: torch.Tensor        # (nreq, width) int32
    outs: torch.Tensor       # (nreq, width) int32
    starts: torch.Tensor     # (nreq,) int64
    ends: torch.Tensor       # (nreq,) int64
    engine_accepted: torch.Tensor  # (nreq,) int64


def slot_matrix(m, nreq):
    """The decode requests' slot rows as a 2-D view (one column when the
    engine sends a vector)."""
    slots = m.state_indices_tensor_d
    if slots is None or slots.dim() not in (1, 2):
        raise ValueError("state_indices_tensor_d must be a vector or a matrix of slot rows")
    slots = slots[:, None] if slots.dim() == 1 else slots
    if slots.shape[0] < nreq:
        raise ValueError(f"{nreq} decode requests but {slots.shape[0]} slot rows")
    return slots


def pool_holds(named, pool_blocks):
    """False when a slot matrix naming `named` blocks is bigger than the
    pool: the engine's profiling pass sizes the pool for one block per
    request but sends one slot per verifier position, and every request then
    sits on the null block (mixers.py:527-541).  Shape-only, so fixed under
    capture."""
    return int(named) <= int(pool_blocks)


def packed_rows(m, nreq, device):
    """(nreq + 1,) packed row starts of the decode requests: the engine's
    query_start_loc_d, or one row per request when it sends none."""
    qsl = getattr(m, "query_start_loc_d", None)
    if qsl is not None:
        if qsl.numel() <= nreq:
            raise ValueError(f"query_start_loc_d has {qsl.numel()} entries for {nreq} requests")
        return qsl[:nreq + 1]
    if int(m.num_decode_tokens) != nreq:
        raise ValueError(f"{int(m.num_decode_tokens)} decode tokens in {nreq} requests need "
                         "query_start_loc_d")
    return torch.arange(nreq + 1, device=device, dtype=torch.int32)


def _block_pointers(m, nreq):
    """Prefix caching's block columns of the previous and this step's last
    scheduled token, both or neither."""
    prev = getattr(m, "block_idx_last_scheduled_token_prev_step", None)
    sched = getattr(m, "block_idx_last_scheduled_token", None)
    if prev is None or sched is None:
        return None, None
    return prev[:nreq], sched[:nreq]


_PLAN_ATTR = "_evo2_verify_plan"


def verify_plan(m, nreq, max_positions, pool_blocks):
    """The step's `VerifyPlan`, one launch (`evo2_spec_plan`).  Slot windows
    are the slot row itself, or with prefix caching's block pointers the
    `max_positions` columns from each pointer; a pool smaller than the slot
    matrix puts every request on the null block.  Kept on the metadata object
    for the step's other layers while its input tensors are unchanged (their
    version counters), and rebuilt on every call during graph capture so the
    launch is part of the graph."""
    slots = slot_matrix(m, nreq)
    device = slots.device
    rows = packed_rows(m, nreq, device)
    qsl = rows if getattr(m, "query_start_loc_d", None) is not None else None  # else r, r + 1
    prev, sched = _block_pointers(m, nreq)
    eng = getattr(m, "num_accepted_tokens", None)
    if eng is not None and eng.numel() < nreq:
        raise ValueError(f"num_accepted_tokens has {eng.numel()} entries for {nreq} requests")
    width = slots.shape[1] if prev is None else min(slots.shape[1], int(max_positions))
    holds = pool_holds(nreq * width, pool_blocks)
    # the engine's own tensors (views made here are new objects every call)
    inputs = tuple(getattr(m, f, None) for f in (
        "state_indices_tensor_d", "query_start_loc_d", "block_idx_last_scheduled_token_prev_step",
        "block_idx_last_scheduled_token", "num_accepted_tokens"))
    key = (nreq, width, holds) + tuple(None if t is None else (id(t), t._version) for t in inputs)
    capturing = torch.cuda.is_current_stream_capturing()
    memo = getattr(m, _PLAN_ATTR, None)
    if memo is not None and memo[0] == key and not capturing:
        return memo[2]
    _lib.require_device(slots, qsl, prev, sched, eng)
    qsl32, prev32, sched32, eng32 = (None if t is None else _i32(t[:nreq + 1] if t is qsl else t[:nreq])
                                     for t in (qsl, prev, sched, eng))
    slots32 = slots[:nreq] if slots.dtype == torch.int32 else slots[:nreq].to(torch.int32)
    ins = torch.empty(nreq, width, dtype=torch.int32, device=device)
    outs = torch.empty_like(ins)
    bounds = torch.empty(3, nreq, dtype=torch.int64, device=device)
    _lib.call("evo2_spec_plan", _lib.ptr(slots32), slots32.stride(0), slots32.stride(1),
              slots32.shape[1], _lib.ptr(qsl32), _lib.ptr(prev32), _lib.ptr(sched32),
              _lib.ptr(eng32), nreq, width, 0 if holds else 1, _lib.ptr(ins), _lib.ptr(outs),
              _lib.ptr(bounds[0]), _lib.ptr(bounds[1]), _lib.ptr(bounds[2]),
              _lib.stream_of(slots))
    plan = VerifyPlan(ins, outs, bounds[0], bounds[1], bounds[2])
    try:
        # the inputs stay referenced, so no other tensor can take their ids
        setattr(m, _PLAN_ATTR, (key, inputs, plan))
    except (AttributeError, TypeError):
        pass
    return plan


def repair_prefill_states(kv_cache, stamps, m, faults):
    """Align-mode prefix caching: a prefill row resuming from n computed
    tokens whose block is not stamped n, while the block of its last
    computed token is, takes that block's three slices (mixers.py:1001-1040).
    Two launches (decide, then copy only the rows that need it); a row whose
    repair would race another's counts in `faults` instead."""
    npf = int(m.num_prefills)
    need = getattr(m, "computed_before_p", None)
    src = getattr(m, "state_src_block_p", None)
    flags = getattr(m, "has_initial_states_p", None)
    if not npf or need is None or src is None or flags is None:
        return
    dst = m.state_indices_tensor_p
    _lib.require_device(stamps, dst, src, need, flags, faults)
    dst32, src32, need32 = (_i32(t[:npf]) for t in (dst, src, need))
    init8 = flags[:npf].to(torch.uint8).contiguous()
    take = torch.empty(npf, dtype=torch.int32, device=stamps.device)
    ptrs = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in kv_cache])
    strides = (ctypes.c_int64 * 9)(*[st for t in kv_cache for st in t.stride()])
    dims = (ctypes.c_int64 * 6)(*[d for t in kv_cache for d in t.shape[1:]])
    sizes = (ctypes.c_int32 * 3)(*[t.element_size() for t in kv_cache])
    for t in kv_cache:
        if t.dim() != 3:
            raise ValueError("state slices must be (blocks, d1, d2) views")
    _lib.call("evo2_spec_repair_prefill", _lib.ptr(stamps), stamps.stride(0), stamps.shape[0],
              _lib.ptr(dst32), _lib.ptr(src32), _lib.ptr(need32), _lib.ptr(init8), npf,
              _lib.ptr(take), _lib.ptr(faults), ptrs, strides, dims, sizes,
              _lib.stream_of(stamps))


__all__ = ["spec_accepted", "record_stamps", "VerifyPlan", "verify_plan", "slot_matrix",
           "pool_holds", "packed_rows", "repair_prefill_states"]
