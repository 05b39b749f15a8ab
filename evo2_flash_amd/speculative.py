"""Host plumbing of speculative decode for the Hyena mixers (torch, no kernels).

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
(mixers.py:960-999).  Everything here is small index arithmetic on device
tensors with no host synchronisation, so it can sit inside a captured step.

Stamp mismatches (a request whose stamps do not match its computed-token
count) are counted in a device tensor the caller reads when it chooses
(`HyenaMixerBase.stamp_faults`), where the reference raises a device-side
assert: on ROCm such an assert aborts the whole process from inside a kernel.
"""

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


def accepted_tokens(m, num_reqs, device):
    """vLLM's per-request accepted counts, >= 1; ones when absent
    (mixers.py:431-441)."""
    acc = getattr(m, "num_accepted_tokens", None)
    if acc is None:
        return torch.ones(num_reqs, device=device, dtype=torch.long)
    if acc.numel() < num_reqs:
        raise ValueError(f"num_accepted_tokens is too short: shape={tuple(acc.shape)}, "
                         f"num_decodes={num_reqs}")
    return acc[:num_reqs].to(dtype=torch.long).clamp_min(1)


def cache_all_decode_slots(m, slots, num_reqs, max_positions):
    """Input and output slot windows from prefix caching's block pointers, or
    the slot matrix itself for both (mixers.py:444-456)."""
    previous = getattr(m, "block_idx_last_scheduled_token_prev_step", None)
    scheduled = getattr(m, "block_idx_last_scheduled_token", None)
    if previous is None or scheduled is None:
        return slots, slots
    width = slots.shape[1] if max_positions is None else min(slots.shape[1], max_positions)
    offsets = torch.arange(width, device=slots.device, dtype=torch.long)
    ins = slots.gather(1, previous[:num_reqs, None].long() + offsets)
    outs = slots.gather(1, scheduled[:num_reqs, None].long() + offsets)
    return ins, outs


def decode_tensors(m, num_tokens, max_positions=None, accepted=None):
    """(ins, outs, starts, ends, accepted) of the packed decode requests, all
    on the device (mixers.py:459-524).  `accepted` defaults to vLLM's counts;
    the mixers pass the stamp-derived ones."""
    slots = m.state_indices_tensor_d
    if slots.dim() == 1:
        slots = slots[:, None]
    if slots.dim() != 2:
        raise ValueError(f"state_indices_tensor_d must be rank 1 or 2, got "
                         f"shape={tuple(slots.shape)}")
    num_reqs = int(m.num_decodes)
    if slots.shape[0] < num_reqs:
        raise ValueError(f"decode state rows={slots.shape[0]} smaller than "
                         f"num_decodes={num_reqs}")
    starts = getattr(m, "query_start_loc_d", None)
    if starts is None:
        if num_tokens != num_reqs:
            raise ValueError("packed multi-token decode requires query_start_loc_d: "
                             f"num_decode_tokens={num_tokens}, num_decodes={num_reqs}")
        starts = torch.arange(num_reqs + 1, device=slots.device, dtype=torch.int64)
    else:
        if starts.numel() < num_reqs + 1:
            raise ValueError(f"query_start_loc_d is too short: shape={tuple(starts.shape)}, "
                             f"num_decodes={num_reqs}")
    if accepted is None:
        accepted = accepted_tokens(m, num_reqs, slots.device)
    else:
        accepted = accepted[:num_reqs].to(dtype=torch.long)
    ins, outs = cache_all_decode_slots(m, slots[:num_reqs], num_reqs, max_positions)
    first, last = _row_bounds(m, starts, num_reqs)
    return ins, outs, first, last, accepted


def _row_bounds(m, qsl, num_reqs):
    """int64 (starts, ends) of the packed decode rows, computed once per
    step: every layer of a step sees the same metadata, so the pair is kept
    on it with the tensor it came from (held, so no other tensor can take
    its address) and that tensor's version counter (an in-place update
    recomputes)."""
    cache = getattr(m, "_evo2_row_bounds", None)
    if (cache is not None and cache[0] is qsl and cache[1] == qsl._version
            and cache[2] == num_reqs):
        return cache[3], cache[4]
    s = qsl[:num_reqs + 1].to(torch.int64)
    first, last = s[:-1], s[1:]
    try:
        m._evo2_row_bounds = (qsl, qsl._version, num_reqs, first, last)
    except AttributeError:   # a metadata object that takes no new attributes
        pass
    return first, last


def cache_safe_state_indices(indices, state):
    """The null block for every entry when a slot matrix names more blocks
    than the pool holds: the engine's profiling pass allocates one block per
    request but passes one index per verifier position (mixers.py:527-541).
    Shape-only, so constant under graph capture."""
    if indices.dim() == 2 and state.shape[0] < indices.numel():
        return torch.zeros_like(indices)
    return indices


def query_start_loc_d(m, num_reqs, device):
    """The decode rows' packed starts, or one row per request when the step
    carries none (the form `decode_tensors` accepts)."""
    qsl = getattr(m, "query_start_loc_d", None)
    if qsl is None:
        if int(m.num_decode_tokens) != num_reqs:
            raise ValueError("packed multi-token decode requires query_start_loc_d: "
                             f"num_decode_tokens={int(m.num_decode_tokens)}, "
                             f"num_decodes={num_reqs}")
        return torch.arange(num_reqs + 1, device=device, dtype=torch.int32)
    if qsl.numel() < num_reqs + 1:
        raise ValueError(f"query_start_loc_d is too short: shape={tuple(qsl.shape)}, "
                         f"num_decodes={num_reqs}")
    return qsl[:num_reqs + 1]


__all__ = ["spec_accepted", "record_stamps", "accepted_tokens", "cache_all_decode_slots",
           "decode_tensors", "cache_safe_state_indices", "query_start_loc_d"]
