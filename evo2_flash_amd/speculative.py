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
        starts = starts[:num_reqs + 1]
    if accepted is None:
        accepted = accepted_tokens(m, num_reqs, slots.device)
    else:
        accepted = accepted[:num_reqs].to(dtype=torch.long)
    ins, outs = cache_all_decode_slots(m, slots[:num_reqs], num_reqs, max_positions)
    return ins, outs, starts[:-1].long(), starts[1:].long(), accepted


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


__all__ = ["accepted_tokens", "cache_all_decode_slots", "decode_tensors",
           "cache_safe_state_indices", "query_start_loc_d"]
