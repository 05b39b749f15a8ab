"""Paged Hyena state: the unified three-slice spec and a block pool laid out
the way vLLM lays out a mamba layer's cache.

Every Hyena layer declares one spec (mixers.py:870-917, model.py:277-333):
  slice 0  conv state   native (blocks, K_short-1, 3H) bf16 -> view (blocks, 3H, 2)
  slice 1  inner FIR    native (blocks, K_max-1, H) fp32    -> view (blocks, H, 127)
  slice 2  LI state     (blocks, H, 16) fp32, not transposed
The three slices of a block share one padded page, so each slice's block
stride is the page size in that slice's element type, not its own size.
Views are oldest-first windows; block 0 is the null block.

With speculative decoding of `num_spec` draft tokens (mixers.py:887-900) the
conv window widens to K_short-1+num_spec columns and the LI slice gains a
17th column whose row 0 holds the block's position stamp: the number of
tokens the block's snapshot represents (mixers.py:952-958).
"""

from typing import NamedTuple

import torch

NULL_BLOCK = 0


class MambaCopySpec(NamedTuple):
    """A cached state to move between blocks: its first element's address
    and its element count (the engine copies them to the start of the
    destination block's state in the same slice)."""
    start_addr: int
    num_elements: int


def _conv_source(state, block_ids, cur_block_idx, num_accepted_tokens):
    # native (blocks, state_len, dim): after a verify step the block's window
    # is [older inputs, d_1 .. d_q]; the K-1 inputs before the next token
    # start num_accepted_tokens - 1 columns in
    return state[block_ids[cur_block_idx], num_accepted_tokens - 1:]


def _temporal_source(state, block_ids, cur_block_idx, num_accepted_tokens):
    # one whole snapshot per verifier position, in consecutive blocks
    return state[block_ids[cur_block_idx + num_accepted_tokens - 1]]


def get_conv_copy_spec(state, block_ids, cur_block_idx, num_accepted_tokens):
    """Copy rule of the sliding conv window (slice 0)."""
    src = _conv_source(state, block_ids, cur_block_idx, num_accepted_tokens)
    return MambaCopySpec(src.data_ptr(), src.numel())


def get_temporal_copy_spec(state, block_ids, cur_block_idx, num_accepted_tokens):
    """Copy rule of a temporal snapshot slice (slices 1 and 2)."""
    src = _temporal_source(state, block_ids, cur_block_idx, num_accepted_tokens)
    return MambaCopySpec(src.data_ptr(), src.numel())


def get_mamba_state_copy_func():
    """One copy rule per state slice (model.py:285-304): the sliding window
    for the conv slice, a whole snapshot for the inner-FIR and LI slices.
    vLLM's own rules when vLLM imports (its model runner consumes their spec
    type), else this module's, which follow the same arguments and layout."""
    try:
        from vllm.model_executor.layers.mamba.mamba_utils import (get_conv_copy_spec as conv,
                                                                  get_temporal_copy_spec as temp)
    except ImportError:
        conv, temp = get_conv_copy_spec, get_temporal_copy_spec
    return (conv, temp, temp)


def unified_state_shape(hidden, k_short=3, k_inner_max=128, state_size=16, num_spec=0):
    """Native shapes per block: ((K_short-1+num_spec, 3H), (K_max-1, H),
    (H, S + [num_spec > 0])) (mixers.py:892-900).

    The first two are vLLM's (state_len, dim) conv layout, normalised to
    (dim, state_len) by `conv_view` (mixers.py:858-868, 940-949).
    """
    return ((k_short - 1 + num_spec, 3 * hidden), (k_inner_max - 1, hidden),
            (hidden, state_size + (1 if num_spec else 0)))


def unified_state_dtype(model_dtype=torch.bfloat16):
    """(model dtype, fp32, fp32) (mixers.py:908-910)."""
    return (model_dtype, torch.float32, torch.float32)


def page_bytes(hidden, k_short=3, k_inner_max=128, state_size=16, align=256, num_spec=0):
    shapes = unified_state_shape(hidden, k_short, k_inner_max, state_size, num_spec)
    dtypes = unified_state_dtype()
    total = 0
    for shp, dt in zip(shapes, dtypes):
        n = 1
        for d in shp:
            n *= d
        total += n * torch.tensor([], dtype=dt).element_size()
    return (total + align - 1) // align * align


class HyenaStatePool:
    """One layer's state pool: a (blocks, page) byte buffer carved into three
    strided slices, like vLLM's mamba KV cache for a layer.

    `kv_cache` is the engine-facing 3-tuple of native-layout views;
    `conv_view`, `inner_view` and `ssm_view` are the normalised dim-first
    views the operators take.
    """

    def __init__(self, num_blocks, hidden, device, k_short=3, k_inner_max=128,
                 state_size=16, page_align=256, dtype=torch.bfloat16, num_spec=0):
        self.num_blocks = num_blocks
        self.hidden = hidden
        self.state_size = state_size
        self.num_spec = num_spec
        shapes = unified_state_shape(hidden, k_short, k_inner_max, state_size, num_spec)
        dtypes = unified_state_dtype(dtype)
        self.page = page_bytes(hidden, k_short, k_inner_max, state_size, page_align, num_spec)
        self.raw = torch.zeros(num_blocks, self.page, dtype=torch.uint8, device=device)
        views, off = [], 0
        for shp, dt in zip(shapes, dtypes):
            es = torch.tensor([], dtype=dt).element_size()
            assert off % es == 0 and self.page % es == 0
            flat = self.raw.view(-1).view(dt)
            inner_strides = []
            acc = 1
            for d in reversed(shp):
                inner_strides.insert(0, acc)
                acc *= d
            v = flat.as_strided((num_blocks, *shp), (self.page // es, *inner_strides), off // es)
            views.append(v)
            off += acc * es
        self.kv_cache = tuple(views)

    def conv_view(self):
        """(blocks, 3H, K_short-1) bf16, dim-first (mixers.py:940-949)."""
        return self.kv_cache[0].transpose(-1, -2)

    def inner_view(self, width=None):
        """(blocks, H, K_max-1) fp32, or its leading `width` columns."""
        v = self.kv_cache[1].transpose(-1, -2)
        return v if width is None else v[..., :width]

    def ssm_view(self):
        """(blocks, H, 16) fp32 (mixers.py:1334-1342): the recurrence part of
        slice 2, without the stamp column."""
        return self.kv_cache[2][..., :self.state_size]

    def stamps(self):
        """(blocks,) fp32 view of the position stamps (mixers.py:952-958);
        only with num_spec > 0."""
        if not self.num_spec:
            raise ValueError("position stamps exist only with speculative decoding (num_spec > 0)")
        return self.kv_cache[2][:, 0, -1]

    def copy_cached_state(self, block_ids, cur_block_idx, num_accepted_tokens, dst_block):
        """Apply the three copy rules to this pool, the way the engine does on
        its prefix-caching path: each slice's source (get_mamba_state_copy_func)
        goes to the start of `dst_block`'s state in that slice."""
        for state, src_of in zip(self.kv_cache, (_conv_source, _temporal_source, _temporal_source)):
            src = src_of(state, block_ids, cur_block_idx, num_accepted_tokens)
            n = src.numel()
            state[dst_block].reshape(-1)[:n].copy_(src.reshape(-1))
        return self

    def zero_(self):
        self.raw.zero_()
        return self
