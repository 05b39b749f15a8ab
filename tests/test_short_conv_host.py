"""Host-side behaviour of the short-convolution and final-state entry points
(no GPU): CPU tensors are refused (there is no CPU path) except where the
reference's own contract returns None for them (`iir_final_state`,
triton_prefill.py:360-361), and the forms this build does not implement
(packed rows without acceptance counts, the prefill's prefix-caching
arguments) raise NotImplementedError before any work.
"""

import pytest
import torch

from evo2_flash_amd.hcl import iir_final_state
from evo2_flash_amd.short_conv import causal_conv1d_fn, causal_conv1d_update

bf = torch.bfloat16


def test_iir_final_state_cpu_returns_none():
    assert iir_final_state(torch.zeros(4, 8), torch.zeros(4, 16)) is None
    assert iir_final_state(torch.zeros(4, 8, dtype=torch.float64), torch.zeros(4, 16)) is None


def test_short_conv_refuses_cpu_tensors():
    x = torch.zeros(2, 6, dtype=bf)
    st = torch.zeros(3, 6, 2, dtype=bf)
    w = torch.zeros(6, 3, dtype=bf)
    with pytest.raises(RuntimeError, match="GPU only"):
        causal_conv1d_update(x, st, w, None, activation=None)
    with pytest.raises(RuntimeError, match="GPU only"):
        causal_conv1d_fn(x.t(), w, None, conv_states=st,
                         query_start_loc=torch.tensor([0, 2], dtype=torch.int32))


def test_unsupported_forms_raise():
    x = torch.zeros(2, 6, dtype=bf)
    st = torch.zeros(3, 6, 2, dtype=bf)
    w = torch.zeros(6, 3, dtype=bf)
    with pytest.raises(NotImplementedError, match="non-speculative varlen"):
        causal_conv1d_update(x, st, w, None, query_start_loc=torch.tensor([0, 2]))
    with pytest.raises(NotImplementedError, match="query_start_loc"):
        causal_conv1d_update(x, st, w, None, num_accepted_tokens=torch.ones(2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU only"):
        causal_conv1d_update(x, st, w, None, conv_state_indices=torch.tensor([[1], [2]]),
                             num_accepted_tokens=torch.ones(2, dtype=torch.int32),
                             query_start_loc=torch.tensor([0, 1, 2], dtype=torch.int32))
    with pytest.raises(NotImplementedError, match="prefix-caching"):
        causal_conv1d_fn(x.t(), w, None, conv_states=st,
                         query_start_loc=torch.tensor([0, 2], dtype=torch.int32),
                         block_idx_first_scheduled_token=torch.zeros(1, dtype=torch.int32))
    with pytest.raises(NotImplementedError, match="activation"):
        causal_conv1d_update(x, st, w, None, activation="gelu")
    with pytest.raises(NotImplementedError, match="one token"):
        causal_conv1d_update(torch.zeros(2, 6, 3, dtype=bf), st, w)


def test_fn_rejects_empty_segment_table():
    x = torch.zeros(2, 6, dtype=bf)
    w = torch.zeros(6, 3, dtype=bf)
    with pytest.raises(ValueError, match="query_start_loc"):
        causal_conv1d_fn(x.t(), w, None, query_start_loc=torch.zeros(0, dtype=torch.int32))
