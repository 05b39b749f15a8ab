"""The vLLM short-convolution entry points (`causal_conv1d_update`,
`causal_conv1d_fn`, as mixers.py:1121-1208 calls them) and `iir_final_state`
(triton_prefill.py:351-387) on the GPU against the oracle.

Bar: outputs and windows bit-identical to the oracle's restatement (the
rounding the reference states for vLLM's update kernel) without activation;
SiLU within one bf16 ulp (the device and host `exp` may differ in the last
fp32 bit).  The final state is an fp32 scan: within 1e-4 of the float64
recurrence, and bit-identical to `iir_segment`'s state, which runs the same
two phases.  Cases: K = 2, 3, 4, bias, ragged segments (empty, one row,
shorter than the window, crossing row tiles), padding slots, strided views
shaped like the mixers' (z_p.T, the pool's dim-first conv view), and the
7B-shaped decode and prefill rows.
"""

import pytest
import torch

import oracle
from evo2_flash_amd.hcl import iir_final_state, iir_segment
from evo2_flash_amd.short_conv import causal_conv1d_fn, causal_conv1d_update
from evo2_flash_amd.state import HyenaStatePool

from _cases import bf16_ulp_diff

pytestmark = pytest.mark.gpu
DEV = "cuda"
bf = torch.bfloat16


def _qsl(lens):
    q = [0]
    for n in lens:
        q.append(q[-1] + n)
    return q


def _conv_state(nb, dim, K, g):
    """A dim-first (blocks, dim, K-1) view of (blocks, K-1, dim) storage, the
    pool's layout (mixers.py:940-949)."""
    raw = torch.randn(nb, K - 1, dim, generator=g).to(bf)
    return raw.transpose(1, 2)


@pytest.mark.parametrize("K,use_bias", [(2, False), (3, False), (3, True), (4, True)])
def test_update_bitwise(K, use_bias):
    g = torch.Generator().manual_seed(10 + K)
    dim, B, nb = 3 * 256 + 96, 9, 14
    wide = torch.randn(B, dim + 40, generator=g).to(bf)
    x = wide[:, 17:17 + dim]                       # strided rows
    w = (torch.randn(dim, K, generator=g) * 0.4).to(bf)
    bias = (torch.randn(dim, generator=g) * 0.5).to(bf) if use_bias else None
    st = _conv_state(nb, dim, K, g)
    slots = torch.tensor([5, 1, -1, 12, 3, 0, 9, 7, 13], dtype=torch.int32)
    st_ref = st.clone()
    ref = oracle.causal_conv1d_update_ref(x, st_ref, w, bias, None, slots.tolist())
    st_d = st.to(DEV)
    print(f"causal_conv1d_update K={K} bias={use_bias}", flush=True)
    out = causal_conv1d_update(x.to(DEV), st_d, w.to(DEV), None if bias is None else bias.to(DEV),
                               activation=None, conv_state_indices=slots.to(DEV))
    assert torch.equal(out.cpu().float(), ref)
    assert torch.equal(st_d.cpu(), st_ref)
    assert not out[2].any()                        # padding row


def test_update_silu_and_3d_input():
    g = torch.Generator().manual_seed(21)
    dim, B, nb = 512, 6, 8
    x = torch.randn(B, dim, generator=g).to(bf)
    w = (torch.randn(dim, 3, generator=g) * 0.4).to(bf)
    st = _conv_state(nb, dim, 3, g)
    slots = torch.tensor([1, 2, 3, 4, 5, 6], dtype=torch.int32)
    st_ref = st.clone()
    ref = oracle.causal_conv1d_update_ref(x, st_ref, w, None, "silu", slots.tolist())
    st_d = st.to(DEV)
    out = causal_conv1d_update(x.to(DEV).unsqueeze(-1), st_d, w.to(DEV), activation="silu",
                               conv_state_indices=slots.to(DEV))
    assert out.shape == (B, dim, 1)
    assert bf16_ulp_diff(out[..., 0].cpu(), ref.to(bf)).max() <= 1
    assert torch.equal(st_d.cpu(), st_ref)


def test_update_7b_decode_rows():
    """64 decode rows of the 7B in_proj output (3H = 12288) through the pool's
    conv view, slots from a permutation, as the mixers pass them."""
    H, B = 4096, 64
    g = torch.Generator().manual_seed(33)
    pool = HyenaStatePool(B + 1, H, "cpu")
    pool.kv_cache[0].copy_(torch.randn(pool.kv_cache[0].shape, generator=g).to(bf))
    w = (torch.randn(3 * H, 3, generator=g) * 0.3).to(bf)
    x = torch.randn(B, 3 * H, generator=g).to(bf)
    slots = (torch.randperm(B, generator=g) + 1).to(torch.int32)
    cv = pool.conv_view()
    ref_state = cv.clone()
    ref = oracle.causal_conv1d_update_ref(x, ref_state, w, None, None, slots.tolist())
    dpool = HyenaStatePool(B + 1, H, DEV)
    dpool.raw.copy_(pool.raw.to(DEV))
    print("causal_conv1d_update 7B rows", flush=True)
    out = causal_conv1d_update(x.to(DEV), dpool.conv_view(), w.to(DEV), None, activation=None,
                               conv_state_indices=slots.to(DEV))
    assert torch.equal(out.cpu().float(), ref)
    assert torch.equal(dpool.conv_view().cpu(), ref_state)


@pytest.mark.parametrize("K,use_bias,act", [(3, False, None), (2, True, None), (4, False, None),
                                            (3, True, "silu")])
def test_fn_ragged_segments(K, use_bias, act):
    """Segments of 5, 0, 1, 130, 2, 64 and 3 rows (one crossing two 64-row
    tiles, one shorter than the window), mixed has_initial_state, a padding
    slot; x is z_p.T of a token-major buffer with extra columns."""
    lens = [5, 0, 1, 130, 2, 64, 3]
    has_init = [1, 1, 0, 1, 1, 0, 1]
    slots = [4, 2, 9, -1, 7, 1, 11]
    dim = 2 * 256 + 72
    g = torch.Generator().manual_seed(40 + K)
    T = sum(lens)
    zp = torch.randn(T, dim + 24, generator=g).to(bf)[:, 8:8 + dim]
    w = (torch.randn(dim, K, generator=g) * 0.4).to(bf)
    bias = (torch.randn(dim, generator=g) * 0.5).to(bf) if use_bias else None
    st = _conv_state(12, dim, K, g)
    st_ref = st.clone()
    q = _qsl(lens)
    ref = oracle.causal_conv1d_ref(zp, w, bias, act, q, slots, has_init, st_ref)
    st_d = st.to(DEV)
    print(f"causal_conv1d_fn K={K} bias={use_bias} act={act}", flush=True)
    out = causal_conv1d_fn(zp.to(DEV).t(), w.to(DEV), None if bias is None else bias.to(DEV),
                           conv_states=st_d, query_start_loc=torch.tensor(q, dtype=torch.int32,
                                                                          device=DEV),
                           cache_indices=torch.tensor(slots, dtype=torch.int32, device=DEV),
                           has_initial_state=torch.tensor(has_init, dtype=torch.bool, device=DEV),
                           activation=act)
    assert out.shape == (dim, T)
    got = out.t().cpu()
    if act is None:
        assert torch.equal(got.float(), ref)
    else:
        assert bf16_ulp_diff(got, ref.to(bf)).max() <= 1
    assert torch.equal(st_d.cpu(), st_ref)


def test_fn_without_state_and_one_row_continuation():
    """conv_states=None reads and writes no window; a one-row segment that
    continues a window equals causal_conv1d_update on the same row."""
    g = torch.Generator().manual_seed(51)
    dim = 300
    x = torch.randn(70, dim, generator=g).to(bf)
    w = (torch.randn(dim, 3, generator=g) * 0.4).to(bf)
    ref = oracle.causal_conv1d_ref(x, w, None, None, [0, 70], None, None, None)
    out = causal_conv1d_fn(x.to(DEV).t(), w.to(DEV), None, query_start_loc=torch.tensor(
        [0, 70], dtype=torch.int32, device=DEV), activation=None)
    assert torch.equal(out.t().cpu().float(), ref)
    none = causal_conv1d_fn(x.to(DEV).t(), w.to(DEV), None, query_start_loc=torch.zeros(
        1, dtype=torch.int32, device=DEV), activation=None)   # no segment: rows are zero
    assert not none.any()

    st = _conv_state(4, dim, 3, g).to(DEV)
    st2 = st.clone()
    row = x[:3].to(DEV)
    slots = torch.tensor([3, 0, 2], dtype=torch.int32, device=DEV)
    a = causal_conv1d_fn(row.t(), w.to(DEV), None, conv_states=st,
                         query_start_loc=torch.tensor([0, 1, 2, 3], dtype=torch.int32, device=DEV),
                         cache_indices=slots, has_initial_state=torch.ones(3, dtype=torch.bool,
                                                                           device=DEV),
                         activation=None)
    b = causal_conv1d_update(row, st2, w.to(DEV), None, activation=None, conv_state_indices=slots)
    assert torch.equal(a.t(), b) and torch.equal(st, st2)


def test_fn_7b_prefill_rows():
    """8192 prefill rows of the 7B in_proj output (3H = 12288) in two
    segments, the second continuing its window, through the pool's conv view."""
    H, lens, has_init = 4096, [3000, 5192], [0, 1]
    g = torch.Generator().manual_seed(61)
    T = sum(lens)
    zp = torch.randn(T, 3 * H, generator=g).to(bf)
    w = (torch.randn(3 * H, 3, generator=g) * 0.3).to(bf)
    pool = HyenaStatePool(4, H, "cpu")
    pool.kv_cache[0].copy_(torch.randn(pool.kv_cache[0].shape, generator=g).to(bf))
    ref_state = pool.conv_view().clone()
    q = _qsl(lens)
    ref = oracle.causal_conv1d_ref(zp, w, None, None, q, [2, 3], has_init, ref_state)
    dpool = HyenaStatePool(4, H, DEV)
    dpool.raw.copy_(pool.raw.to(DEV))
    print("causal_conv1d_fn 7B rows", flush=True)
    out = causal_conv1d_fn(zp.to(DEV).t(), w.to(DEV), None, conv_states=dpool.conv_view(),
                           query_start_loc=torch.tensor(q, dtype=torch.int32, device=DEV),
                           cache_indices=torch.tensor([2, 3], dtype=torch.int32, device=DEV),
                           has_initial_state=torch.tensor(has_init, dtype=torch.bool, device=DEV),
                           activation=None)
    assert torch.equal(out.t().cpu().float(), ref)
    assert torch.equal(dpool.conv_view().cpu(), ref_state)


@pytest.mark.parametrize("H,L", [(300, 1), (256, 37), (1000, 1500), (4096, 4096)])
def test_iir_final_state(H, L):
    g = torch.Generator().manual_seed(L)
    base = torch.randn(L, H + 8, generator=g)
    seq = base[:, 3:3 + H].t()                     # token-major view, as the mixer passes it
    lp = torch.log(torch.rand(H, 16, generator=g) * 0.499 + 0.5)
    res = torch.randn(H, 16, generator=g) * 0.1
    rec = oracle.iir_final_state_recurrence(seq, lp)
    print(f"iir_final_state H={H} L={L}", flush=True)
    st = iir_final_state(seq.to(DEV), lp.to(DEV), blk=16)
    scale = rec.abs().max().item()
    assert (st.cpu().double() - rec).abs().max().item() <= 1e-4 * scale
    _, st2 = iir_segment(seq.to(DEV), res.to(DEV), lp.to(DEV), None)
    assert torch.equal(st, st2)
