"""vLLM's short causal depthwise convolution entry points on this build's kernels.

The reference's mixers run the K=3 short filter through two vLLM kernels
(evo2_flash/mixers.py:1121-1208):

    causal_conv1d_fn(z_p.T, w, None, activation=None, conv_states=conv_state,
                     has_initial_state=..., cache_indices=..., metadata=m,
                     query_start_loc=...)                       # prefill rows
    causal_conv1d_update(z_d, conv_state, w, None, activation=None,
                         conv_state_indices=...)                # decode rows

These functions take the same arguments and mutate the same window view
(blocks, dim, K-1) (the mixers' dim-first view of the (blocks, 2, 3H)
storage).  Outputs are rounded as the reference documents for vLLM's update
kernel (triton_decode.py:10-11): each product rounded to bf16, an fp32 sum
from the bias (or 0), oldest input first, bf16 out.  The mixers of this
build fuse the short filter into their own kernels and do not call these;
they are the drop-in for callers that bind the vLLM entry points.

The update also takes vLLM's speculative form (`num_accepted_tokens`,
`query_start_loc`, `max_query_len`, and the prefix-caching block pointers
`block_idx_last_scheduled_token` / `initial_state_idx`), which the
reference's mixers use for a verify step (mixers.py:1153-1193) with the
window convention mixers.py:222-240 states.  Not supported
(NotImplementedError): packed rows without `num_accepted_tokens`, and the
prefill's prefix-caching arguments.
"""

import torch

from . import _lib

PAD_SLOT_ID = -1

_UNSUPPORTED_FN = ("block_idx_first_scheduled_token", "block_idx_last_scheduled_token",
                   "initial_state_idx", "num_computed_tokens")


def _activation_code(activation):
    if activation in (None, False):
        return 0
    if activation in ("silu", "swish", True):
        return 1
    raise NotImplementedError(f"activation {activation!r} (None or 'silu' only)")


def _check_common(fn, x, weight, bias, conv_state):
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise NotImplementedError(f"{fn}: bf16 inputs and weights only")
    if weight.dim() != 2 or weight.shape[1] not in (2, 3, 4):
        raise ValueError(f"{fn}: weight must be (dim, K) with K in 2..4, got {tuple(weight.shape)}")
    dim, K = weight.shape
    if bias is not None and (bias.shape != (dim,) or bias.dtype != torch.bfloat16):
        raise ValueError(f"{fn}: bias must be ({dim},) bf16")
    if conv_state is not None:
        if conv_state.dtype != torch.bfloat16 or conv_state.dim() != 3:
            raise ValueError(f"{fn}: conv state must be a (blocks, dim, K-1) bf16 view")
        if conv_state.shape[1] != dim or conv_state.shape[2] < K - 1:
            raise ValueError(f"{fn}: conv state {tuple(conv_state.shape)} does not fit dim={dim}, K={K}")
    return dim, K


def _index_table(idx, n, fn, name):
    if idx is None:
        return None, 0
    if idx.dim() == 2:  # vLLM's (batch, max_query_len) slot matrix: column 0
        idx = idx[:, 0]
    if idx.dim() != 1 or idx.shape[0] < n:
        raise ValueError(f"{fn}: {name} must hold one slot per sequence")
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    return idx, idx.stride(0)


def _update_spec(x, conv_state, weight, bias, act, conv_state_indices, num_accepted_tokens,
                 query_start_loc, max_query_len, pad_slot_id, out_col, in_col):
    """The speculative varlen form (see `causal_conv1d_update`)."""
    fn = "causal_conv1d_update"
    if query_start_loc is None or x.dim() != 2:
        raise NotImplementedError(f"{fn}: the speculative form takes packed rows x (T, dim) "
                                  "with query_start_loc")
    if conv_state_indices is None:
        raise ValueError(f"{fn}: the speculative form needs conv_state_indices")
    _lib.require_device(x, conv_state, weight, bias, conv_state_indices, num_accepted_tokens,
                        query_start_loc, out_col, in_col)
    dim, K = _check_common(fn, x, weight, bias, conv_state)
    if x.shape[1] != dim:
        raise ValueError(f"{fn}: x must be (T, {dim})")
    idx = conv_state_indices if conv_state_indices.dim() == 2 else conv_state_indices[:, None]
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    nreq = query_start_loc.shape[0] - 1
    if nreq < 0 or idx.shape[0] < nreq or num_accepted_tokens.shape[0] < nreq:
        raise ValueError(f"{fn}: query_start_loc names {nreq} requests but conv_state_indices has "
                         f"{idx.shape[0]} rows and num_accepted_tokens {num_accepted_tokens.shape[0]}")
    if max_query_len is None or max_query_len < 1:
        max_query_len = idx.shape[1]
    state_len = conv_state.shape[2]
    if state_len < K - 2 + max_query_len:
        raise ValueError(f"{fn}: a conv state of {state_len} columns cannot hold a "
                         f"{max_query_len}-position verifier window for K={K}")
    qsl = query_start_loc.to(torch.int32).contiguous()
    acc = num_accepted_tokens[:nreq].to(torch.int64).contiguous()
    cols = []
    for c in (in_col, out_col):
        if c is not None:
            if c.shape[0] < nreq:
                raise ValueError(f"{fn}: block pointers must hold one entry per request")
            c = c[:nreq].to(torch.int32).contiguous()
        cols.append(c)
    T = x.shape[0]
    out = torch.zeros(T, dim, dtype=torch.bfloat16, device=x.device)
    _lib.call("evo2_causal_conv1d_update_spec",
              _lib.ptr(x), x.stride(0), x.stride(1),
              _lib.ptr(conv_state), *conv_state.stride(), state_len,
              _lib.ptr(weight), weight.stride(0), weight.stride(1), K,
              _lib.ptr(bias), act,
              _lib.ptr(idx), idx.stride(0), idx.stride(1), idx.shape[1],
              _lib.ptr(cols[0]), _lib.ptr(cols[1]), _lib.ptr(acc), _lib.ptr(qsl),
              int(max_query_len), int(pad_slot_id),
              _lib.ptr(out), out.stride(0), out.stride(1),
              nreq, T, dim, conv_state.shape[0], _lib.stream_of(x))
    return out


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None,
                         conv_state_indices=None, num_accepted_tokens=None, query_start_loc=None,
                         max_query_len=-1, pad_slot_id=PAD_SLOT_ID,
                         block_idx_last_scheduled_token=None, initial_state_idx=None,
                         validate_data=False):
    """One new row per sequence: x (B, dim) bf16 -> out (B, dim) bf16.

    conv_state (blocks, dim, >=K-1) bf16 view, updated in place for each row's
    slot conv_state_indices[b] (slot b when None); rows whose slot is
    pad_slot_id write no state and output zeros.  (B, dim, 1) inputs are
    accepted and returned in that shape.

    Speculative form (num_accepted_tokens given, as the reference's mixers
    call it for a verify step, mixers.py:1176-1193): x is (T, dim) packed
    rows, request r owning rows query_start_loc[r] .. query_start_loc[r+1]-1
    (at most max_query_len, default the slot matrix's width); its window
    starts at column num_accepted_tokens[r] - 1 of slot conv_state_indices[r,
    initial_state_idx[r]] and its new window goes to slot conv_state_indices[r,
    block_idx_last_scheduled_token[r]] (column 0 for either when None), laid
    out so that the next step's window starts at its accepted count - 1
    (mixers.py:222-240).  The conv state needs K-1 + max_query_len-1 columns.
    Rows no request covers are zero.
    """
    fn = "causal_conv1d_update"
    act = _activation_code(activation)
    if num_accepted_tokens is not None:
        return _update_spec(x, conv_state, weight, bias, act, conv_state_indices,
                            num_accepted_tokens, query_start_loc, max_query_len, pad_slot_id,
                            block_idx_last_scheduled_token, initial_state_idx)
    if query_start_loc is not None:
        raise NotImplementedError(f"{fn}: packed rows without num_accepted_tokens "
                                  "(non-speculative varlen) are not supported")
    if block_idx_last_scheduled_token is not None or initial_state_idx is not None:
        raise NotImplementedError(f"{fn}: prefix-caching block pointers are supported with "
                                  "the speculative form only")
    squeeze = x.dim() == 3
    if squeeze:
        if x.shape[2] != 1:
            raise NotImplementedError(f"{fn}: one token per sequence only (got seqlen {x.shape[2]})")
        x = x[..., 0]
    _lib.require_device(x, conv_state, weight, bias, conv_state_indices)
    dim, K = _check_common(fn, x, weight, bias, conv_state)
    if x.dim() != 2 or x.shape[1] != dim:
        raise ValueError(f"{fn}: x must be (B, {dim})")
    B = x.shape[0]
    idx, sidx = _index_table(conv_state_indices, B, fn, "conv_state_indices")
    out = torch.empty(B, dim, dtype=torch.bfloat16, device=x.device)
    _lib.call("evo2_causal_conv1d_update",
              _lib.ptr(x), x.stride(0), x.stride(1),
              _lib.ptr(conv_state), *conv_state.stride(),
              _lib.ptr(weight), weight.stride(0), weight.stride(1), K,
              _lib.ptr(bias), act,
              _lib.ptr(idx), sidx, int(pad_slot_id),
              _lib.ptr(out), out.stride(0), out.stride(1),
              B, dim, conv_state.shape[0], _lib.stream_of(x))
    return out.unsqueeze(-1) if squeeze else out


def causal_conv1d_fn(x, weight, bias=None, conv_states=None, query_start_loc=None,
                     cache_indices=None, has_initial_state=None, activation="silu",
                     pad_slot_id=PAD_SLOT_ID, metadata=None, validate_data=False, **prefix):
    """Packed prefill segments: x (dim, T) bf16 -> out (dim, T) bf16.

    Segment j is columns query_start_loc[j] .. query_start_loc[j+1] - 1 of x;
    its window is conv_states[cache_indices[j]] (slot j when None), read as
    left context when has_initial_state[j] and rewritten with the segment's
    last K-1 inputs.  `metadata` (vLLM's cached-buffer object) is accepted
    and unused.  The output is a transposed view of a token-major (T, dim)
    buffer, the orientation the mixers transpose back to.
    """
    fn = "causal_conv1d_fn"
    act = _activation_code(activation)
    for k in _UNSUPPORTED_FN:
        if prefix.pop(k, None) is not None:
            raise NotImplementedError(f"{fn}: prefix-caching argument {k!r} is not supported")
    prefix.pop("block_size_to_align", None)
    if prefix:
        raise TypeError(f"{fn}: unexpected arguments {sorted(prefix)}")
    if query_start_loc is None:
        raise NotImplementedError(f"{fn}: query_start_loc is required (packed segments)")
    if query_start_loc.dim() != 1 or query_start_loc.shape[0] < 1:
        raise ValueError(f"{fn}: query_start_loc must be (nseq + 1,) with nseq >= 0")
    _lib.require_device(x, weight, bias, conv_states, query_start_loc, cache_indices,
                        has_initial_state)
    dim, K = _check_common(fn, x, weight, bias, conv_states)
    if x.dim() != 2 or x.shape[0] != dim:
        raise ValueError(f"{fn}: x must be ({dim}, T)")
    T = x.shape[1]
    qsl = query_start_loc.to(torch.int32).contiguous()
    nseq = qsl.shape[0] - 1
    idx, sidx = _index_table(cache_indices, nseq, fn, "cache_indices")
    init = None
    if has_initial_state is not None:
        if has_initial_state.shape[0] < nseq:
            raise ValueError(f"{fn}: has_initial_state must hold one flag per sequence")
        init = has_initial_state.to(torch.uint8).contiguous()
    buf = torch.empty(T, dim, dtype=torch.bfloat16, device=x.device)
    out = buf.t()
    cs = conv_states
    _lib.call("evo2_causal_conv1d_fn",
              _lib.ptr(x), x.stride(0), x.stride(1),
              _lib.ptr(weight), weight.stride(0), weight.stride(1), K,
              _lib.ptr(bias), act,
              _lib.ptr(cs), *(cs.stride() if cs is not None else (0, 0, 0)),
              _lib.ptr(init), _lib.ptr(idx), sidx, int(pad_slot_id),
              _lib.ptr(qsl), nseq,
              _lib.ptr(out), out.stride(0), out.stride(1),
              T, dim, cs.shape[0] if cs is not None else 0, _lib.stream_of(x))
    return out


__all__ = ["causal_conv1d_fn", "causal_conv1d_update", "PAD_SLOT_ID"]
