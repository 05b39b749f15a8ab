"""Speculative decode plumbing without a GPU.

The oracle's widened short window (`causal_conv1d_update_spec_ref`) is pinned
by the special case that reduces it to the ordinary update, by the window
layout the reference states (mixers.py:222-240), and by the rollback
invariant the layout exists for: after any accepted prefix of a verify step,
the next step computes what one-token-at-a-time decoding of the accepted
tokens would.  The position-stamp rollback of the mixers (mixers.py:952-1074)
is small launches on the GPU; here the oracle's restatements of it are pinned
by hand-worked cases: stamps written per snapshot, accepted counts resolved
from them, mismatches counted, the step's verify plan, and the align-mode
repair of a resumed prefill.
"""

import pytest
import torch

import oracle
from evo2_flash_amd.config import HyenaConfig
from evo2_flash_amd.metadata import (HyenaMamba2Metadata, HyenaMamba2MetadataBuilder,
                                     Mamba2Metadata, build_metadata)
from evo2_flash_amd.mixers import make_mixer
from evo2_flash_amd.speculative import pool_holds
from evo2_flash_amd.state import HyenaStatePool, page_bytes, unified_state_shape
from evo2_flash_amd.synthetic import mixer_params


def _rand_window(nb, dim, width, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(nb, dim, width, generator=g) * 1.2).to(torch.bfloat16)


def test_spec_update_reduces_to_plain_update():
    """One verifier position, accepted 1, one row per request: the ordinary
    update, outputs and windows."""
    dim, K, nb = 24, 3, 6
    g = torch.Generator().manual_seed(1)
    w = torch.randn(dim, K, generator=g).to(torch.bfloat16)
    x = torch.randn(4, dim, generator=g).to(torch.bfloat16)
    st = _rand_window(nb, dim, K - 1, 2)
    st2 = st.clone()
    slots = torch.tensor([[3], [1], [5], [2]])
    ref = oracle.causal_conv1d_update_ref(x, st, w, slots=[3, 1, 5, 2])
    out = oracle.causal_conv1d_update_spec_ref(x, st2, w, slots, [1, 1, 1, 1],
                                               [0, 1, 2, 3, 4], 1)
    assert torch.equal(out, ref)
    assert torch.equal(st2, st)


def test_spec_update_window_layout():
    """Before [h1..hM], after a full verify step [h2..hM, d1..dq]
    (mixers.py:228-233, M = K-1, state K-1+q-1 columns)."""
    dim, K, q = 5, 3, 4
    st = _rand_window(2, dim, K - 1 + q - 1, 3)
    h = st[1].clone()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(q, dim, generator=g).to(torch.bfloat16)
    w = torch.randn(dim, K, generator=g).to(torch.bfloat16)
    oracle.causal_conv1d_update_spec_ref(x, st, w, torch.tensor([[1]]), [1], [0, q], q)
    assert torch.equal(st[1, :, :K - 2], h[:, 1:K - 1])
    assert torch.equal(st[1, :, K - 2:K - 2 + q], x.t())


@pytest.mark.parametrize("K", [2, 3, 4])
def test_spec_update_rollback_invariant(K):
    """Verify steps with ragged draft counts and random acceptance reproduce
    the one-token-at-a-time history of the accepted tokens."""
    dim, nspec = 16, 3
    Q = nspec + 1
    g = torch.Generator().manual_seed(10 + K)
    w = torch.randn(dim, K, generator=g).to(torch.bfloat16)
    width = K - 1 + nspec
    st = torch.zeros(2, dim, width, dtype=torch.bfloat16)
    start = (torch.randn(K - 1, dim, generator=g)).to(torch.bfloat16)
    st[1, :, :K - 1] = start.t()               # a prefill leaves the window in front
    hist = list(start)
    accepted = 1
    for step in range(12):
        q = int(torch.randint(1, Q + 1, (1,), generator=g))
        x = torch.randn(q, dim, generator=g).to(torch.bfloat16)
        out = oracle.causal_conv1d_update_spec_ref(x, st, w, torch.tensor([[1]]), [accepted],
                                                   [0, q], Q)
        # brute force: token t sees the last K-1 genuine inputs before it
        seen = list(hist)
        for t in range(q):
            window = torch.stack(seen[-(K - 1):] + [x[t]], dim=1).float()  # (dim, K)
            acc = torch.zeros(dim)
            for k in range(K):
                acc = acc + oracle.bf(window[:, k] * w[:, k].float())
            assert torch.equal(out[t], oracle.bf(acc)), (step, t)
            seen.append(x[t])
        accepted = int(torch.randint(1, q + 1, (1,), generator=g))
        hist = hist + list(x[:accepted])


def test_state_shape_with_spec():
    H = 64
    assert unified_state_shape(H, num_spec=3) == ((5, 3 * H), (127, H), (H, 17))
    assert unified_state_shape(H) == ((2, 3 * H), (127, H), (H, 16))
    assert page_bytes(H, align=1, num_spec=3) == 5 * 3 * H * 2 + 127 * H * 4 + H * 17 * 4
    pool = HyenaStatePool(3, H, "cpu", num_spec=3)
    assert pool.conv_view().shape == (3, 3 * H, 5)
    assert pool.ssm_view().shape == (3, H, 16)
    pool.stamps()[2] = 77.0
    assert pool.kv_cache[2][2, 0, 16] == 77.0 and pool.ssm_view()[2].abs().sum() == 0
    with pytest.raises(ValueError, match="stamps"):
        HyenaStatePool(2, H, "cpu").stamps()


_PFX = iter(range(10 ** 6))


def _mixer(kind, num_spec=3, H=32, blocks=12):
    idx = {"hcs": 0, "hcm": 1, "hcl": 2}[kind]
    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=3, hcs_layer_idxs=[0],
                      hcm_layer_idxs=[1], hcl_layer_idxs=[2])
    m = make_mixer(cfg, idx, prefix=f"host.specmix.{kind}.{next(_PFX)}", num_spec=num_spec)
    pool = HyenaStatePool(blocks, H, "cpu", num_spec=num_spec)
    m.kv_cache = pool.kv_cache
    assert m.get_state_shape() == unified_state_shape(H, num_spec=num_spec)
    return m, pool


def _spec_meta(slots, qlens, computed, prefill=None, seq_lens=None):
    """Decode requests with slot rows `slots` and query lengths `qlens`."""
    nd = len(qlens)
    qsl = [0]
    for n in qlens:
        qsl.append(qsl[-1] + n)
    m = HyenaMamba2Metadata(num_decodes=nd, num_decode_tokens=qsl[-1])
    m.state_indices_tensor_d = torch.tensor(slots, dtype=torch.int32)
    m.query_start_loc_d = torch.tensor(qsl, dtype=torch.int32)
    m.num_computed_tokens_d = torch.tensor(computed, dtype=torch.int32)
    if prefill:
        lens, pslots = prefill
        p = build_metadata(prefill_lens=lens, prefill_slots=pslots, has_init=[0] * len(lens),
                           device="cpu")
        m.num_prefills, m.num_prefill_tokens = p.num_prefills, p.num_prefill_tokens
        m.query_start_loc_p, m.has_initial_states_p = p.query_start_loc_p, p.has_initial_states_p
        m.state_indices_tensor_p = p.state_indices_tensor_p
    if seq_lens is not None:
        m.seq_lens = torch.tensor(seq_lens, dtype=torch.int32)
    return m


def test_stamps_record_and_resolve():
    """The oracle's stamp rules on a hand-checked step: a verify step from n
    tokens stamps column p with n + p + 1 (only the columns its rows reach)
    and prefill blocks with their lengths; the next step, having computed
    n + a tokens, resolves accepted = a (mixers.py:960-999, 1049-1074)."""
    st = [0.0] * 12
    slots = [[1, 2, 3, 4], [5, 6, 7, 8]]
    st[1], st[5] = 10, 30                       # live snapshots of the previous step
    acc, faults = oracle.spec_accepted_ref(st, slots, [10, 30], 3)
    assert acc == [1, 1] and faults == 0
    st = oracle.record_stamps_ref(st, slots, [0, 4, 6], [10, 30], 4,
                                  prefill_blocks=[9], seq_lens=[7])
    assert st[1:5] == [11, 12, 13, 14]
    assert st[5:7] == [31, 32] and st[7:9] == [0, 0]
    assert st[9] == 7
    # next step: request 0 accepted 3 of its 4 rows, request 1 both of its 2
    assert oracle.spec_accepted_ref(st, slots, [13, 32], 3) == ([3, 2], 0)
    # a window that starts at column 2 (prefix caching's block pointer)
    st2 = oracle.record_stamps_ref([0.0] * 12, [[1, 2, 3, 4, 5, 6]], [0, 3], [50], 4,
                                   out_col=[2])
    assert st2[3:6] == [51, 52, 53] and st2[1:3] == [0, 0] and st2[6] == 0
    # the null block, slots outside the pool and columns past the row are not written
    st3 = oracle.record_stamps_ref([5.0] * 4, [[0, 9, 2]], [0, 4], [1], 4, out_col=[0])
    assert st3 == [5.0, 5.0, 4.0, 5.0]


def test_stamp_mismatch_is_counted_and_clamped():
    st = [0.0] * 12
    st[1], st[5] = 10, 30
    acc, faults = oracle.spec_accepted_ref(st, [[1, 2, 3, 4], [5, 6, 7, 8]], [9, 40], 3)
    assert acc == [1, 4] and faults == 2        # -1 and +10: both bad
    # requests on the null block are exempt; a slot outside the pool is a fault
    assert oracle.spec_accepted_ref(st, [[0, 0, 0, 0]], [123], 3)[1] == 0
    assert oracle.spec_accepted_ref(st, [[12, 0, 0, 0]], [0], 3)[1] == 1
    assert oracle.spec_accepted_ref(st, None, [123], 3)[1] == 0
    # the engine's counts cross-check
    assert oracle.spec_accepted_ref(st, [[1, 2, 3, 4]], [12], 3, counts=[3]) == ([3], 0)
    assert oracle.spec_accepted_ref(st, [[1, 2, 3, 4]], [12], 3, counts=[2]) == ([3], 1)


@pytest.mark.parametrize("kind", ["hcs", "hcl"])
def test_stamp_kernels_refuse_cpu_tensors(kind):
    """The mixers resolve and record stamps with HIP kernels only."""
    mixer, pool = _mixer(kind)
    m = _spec_meta([[1, 2, 3, 4], [5, 6, 7, 8]], [4, 2], [10, 30], seq_lens=[14, 32])
    with pytest.raises(RuntimeError, match="GPU only"):
        mixer._resolve_accepted(m)
    with pytest.raises(RuntimeError, match="GPU only"):
        mixer._record_stamps(m)


def test_resolve_needs_computed_counts():
    mixer, _ = _mixer("hcs")
    m = _spec_meta([[1, 2, 3, 4]], [2], [5])
    m.num_computed_tokens_d = None
    with pytest.raises(RuntimeError, match="num_computed_tokens_d"):
        mixer._resolve_accepted(m)
    # without speculation configured nothing is resolved
    plain, _ = _mixer("hcs", num_spec=0)
    assert plain._resolve_accepted(m) is None


def test_repair_resumed_prefill_ref():
    """The oracle's align-mode repair (mixers.py:1001-1040), hand-worked: a
    prefill row resuming from n computed tokens whose block is not stamped n
    takes its state (all three slices) from the block of its last computed
    token when that one is stamped n; a row already right, and one with
    neither block stamped n, are untouched.  The GPU kernels are checked
    against this in test_speculative_gpu.py."""
    pool = HyenaStatePool(10, 128, "cpu", num_spec=3)
    g = torch.Generator().manual_seed(5)
    pool.raw.copy_(torch.randint(0, 255, pool.raw.shape, generator=g, dtype=torch.uint8))
    st = pool.stamps()
    st[2], st[3] = 5.0, 40.0     # row 0: dst 2 stale, src 3 good  -> repaired
    st[4], st[6] = 40.0, 40.0    # row 1: dst 4 already right      -> untouched
    st[7], st[8] = 1.0, 2.0      # row 2: neither matches          -> untouched
    slices = [t.contiguous().view(torch.uint8) if t.dtype != torch.uint8 else t
              for t in (pool.kv_cache[0].view(10, -1), pool.kv_cache[1].reshape(10, -1),
                        pool.kv_cache[2].reshape(10, -1))]
    new, rows = oracle.repair_prefill_ref(slices, st.tolist(), [2, 4, 7], [3, 6, 8],
                                          [40, 40, 40], [1, 1, 1])
    assert rows == [0]
    for old, upd in zip(slices, new):
        assert torch.equal(upd[2], old[3])
        keep = [b for b in range(10) if b != 2]
        assert torch.equal(upd[keep], old[keep])
    # a null destination or source, or a fresh row, is never repaired
    _, rows = oracle.repair_prefill_ref(slices, st.tolist(), [0, 2, 2], [3, 0, 3], [40] * 3,
                                        [1, 1, 0])
    assert rows == []


def test_metadata_builder():
    b = HyenaMamba2MetadataBuilder(max_num_seqs=8, block_size=16, device="cpu",
                                   mamba_cache_mode="align")
    base = Mamba2Metadata(num_decodes=2, num_decode_tokens=5, num_prefills=2,
                          num_prefill_tokens=9)
    table = torch.tensor([[1, 2, 3], [4, 5, 6], [7, 8, 9], [10, 11, 12]], dtype=torch.int32)
    m = b.build(base, torch.tensor([33, 7, 0, 17]), table)
    assert isinstance(m, HyenaMamba2Metadata) and m.num_prefill_tokens == 9
    assert m.num_computed_tokens_d.tolist() == [33, 7]
    assert m.num_computed_tokens_d.data_ptr() == b.decode_num_computed_tokens.data_ptr()
    assert m.computed_before_p.tolist() == [0, 17]
    # cp = 0 -> null block; cp = 17 -> the block holding token 16 (column 1)
    assert m.state_src_block_p.tolist() == [0, 11]
    m2 = b.build(base, torch.tensor([40, 8, 0, 1]), table)
    assert m2.num_computed_tokens_d.data_ptr() == m.num_computed_tokens_d.data_ptr()
    assert m.num_computed_tokens_d.tolist() == [40, 8]   # refreshed in place
    assert m2.state_src_block_p.tolist() == [0, 10]
    plain = HyenaMamba2MetadataBuilder(8, 16, "cpu").build(base, torch.tensor([1, 2, 3, 4]))
    assert plain.computed_before_p is None and plain.state_src_block_p is None


def test_verify_plan_ref_and_pool_rule():
    """The oracle's verify plan (mixers.py:431-541), hand-worked: without
    block pointers the slot row is both the input and the output window;
    with them, windows of `width` columns from each pointer; the engine's
    accepted counts are clamped to >= 1; a profiling-sized pool puts every
    request on the null block."""
    slots = [[1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12]]
    ins, outs, starts, ends, acc = oracle.verify_plan_ref(slots, 2, 6, qsl=[0, 2, 5])
    assert ins == outs == slots
    assert starts == [0, 2] and ends == [2, 5] and acc == [1, 1]
    assert oracle.verify_plan_ref(slots, 2, 6, eng_acc=[3, 0])[4] == [3, 1]
    ins, outs, starts, ends, _ = oracle.verify_plan_ref(slots, 2, 4, prev=[0, 2], sched=[1, 1])
    assert ins == [[1, 2, 3, 4], [9, 10, 11, 12]]
    assert outs == [[2, 3, 4, 5], [8, 9, 10, 11]]
    assert starts == [0, 1] and ends == [1, 2]
    # a window running past the row reads the null block
    assert oracle.verify_plan_ref(slots, 2, 4, prev=[4, 0], sched=[0, 0])[0][0] == [5, 6, 0, 0]
    assert oracle.verify_plan_ref(slots, 2, 6, null_all=True)[0] == [[0] * 6] * 2
    # the pool rule: a slot matrix naming more blocks than the pool holds
    assert pool_holds(8, 8) and not pool_holds(9, 8)


def _spec_pool(H, nb, nspec, seed):
    g = torch.Generator().manual_seed(seed)
    pool = HyenaStatePool(nb, H, "cpu", num_spec=nspec)
    pool.kv_cache[0].copy_(torch.randn(pool.kv_cache[0].shape, generator=g).to(torch.bfloat16))
    pool.kv_cache[1].copy_(torch.randn(pool.kv_cache[1].shape, generator=g)
                           .to(torch.bfloat16).float())
    pool.kv_cache[2].copy_(torch.randn(pool.kv_cache[2].shape, generator=g) * 5)
    return pool


def _clone(pool, nspec):
    p = HyenaStatePool(pool.num_blocks, pool.hidden, "cpu", num_spec=nspec)
    p.raw.copy_(pool.raw)
    return p


def _operator(kind, prm, H):
    """(inner, log_poles, poles, state view of a pool)"""
    if kind == "hcl":
        lp = prm["log_poles"][..., 0]
        return prm["residues"], lp, torch.exp(lp.float()), lambda p: p.ssm_view()
    K = prm["conv"].shape[-1]
    return prm["conv"].view(H, K), None, None, lambda p: p.inner_view()


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
@pytest.mark.parametrize("emulate", [True, False])
def test_speculative_composition_at_one_token(kind, emulate):
    """One token per request, previous step fully accepted (accepted = 1):
    the oracle's speculative composition (widened window, snapshot operator,
    D, gate) equals the plain decode composition bit for bit -- the kernel-
    order emulations (`hyena_decode_emulated`) or the reference's torch
    paths (`mixer_decode_unfused`) -- outputs and the written inner state."""
    H, nb, nspec = 64, 8, 3
    prm = mixer_params(kind, H, 3, in_proj_fp8=False)
    sw = prm["short_filter"].view(3 * H, 3)
    inner, lp, poles, view = _operator(kind, prm, H)
    pool = _spec_pool(H, nb, nspec, 1)
    g = torch.Generator().manual_seed(2)
    z = (torch.randn(3, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = torch.tensor([[2, 3, 4, 5], [6, 7, 1, 1], [1, 1, 1, 1]])
    p1, p2 = _clone(pool, nspec), _clone(pool, nspec)
    gs = oracle.mixer_decode_speculative(z, sw, p1.conv_view(), inner, view(p1), prm.get("D"),
                                         slots, [0, 1, 2, 3], [1, 1, 1], 1, poles=poles,
                                         emulate_kernels=emulate)
    window = p2.conv_view()[..., :2]
    if emulate:
        gd = oracle.hyena_decode_emulated(z, sw, window, slots[:, 0], inner, view(p2),
                                          prm.get("D"), lp)
    else:
        gd = oracle.mixer_decode_unfused(z, sw, window, slots[:, 0].tolist(), inner,
                                         view(p2), prm.get("D"), lp)
    assert torch.equal(gs.view(torch.int16), gd.view(torch.int16))
    for b in (2, 6):
        assert torch.equal(view(p1)[b], view(p2)[b])


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
@pytest.mark.parametrize("emulate", [True, False])
def test_fully_accepted_step_equals_chained_decodes(kind, emulate):
    """A verify step of Q tokens per request equals Q one-token decodes run in
    turn on the request's block, bit for bit: every output row, and the
    snapshot in the step's last column equals the state after the Q-th
    decode."""
    H, nb, nspec, Q = 64, 10, 3, 4
    prm = mixer_params(kind, H, 5, in_proj_fp8=False)
    sw = prm["short_filter"].view(3 * H, 3)
    inner, lp, poles, view = _operator(kind, prm, H)
    pool = _spec_pool(H, nb, nspec, 4)
    g = torch.Generator().manual_seed(6)
    slots = torch.tensor([[2, 3, 4, 5], [6, 7, 8, 9]])
    z = (torch.randn(2 * Q, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    p1 = _clone(pool, nspec)
    gs = oracle.mixer_decode_speculative(z, sw, p1.conv_view(), inner, view(p1), prm.get("D"),
                                         slots, [0, Q, 2 * Q], [1, 1], Q, poles=poles,
                                         emulate_kernels=emulate)
    width = inner.shape[1] - 1 if kind != "hcl" else 16
    for r in range(2):
        p2 = _clone(pool, nspec)
        blk = int(slots[r, 0])
        for p in range(Q):
            row = z[r * Q + p:r * Q + p + 1]
            window = p2.conv_view()[..., :2]
            if emulate:
                y = oracle.hyena_decode_emulated(row, sw, window, torch.tensor([blk]), inner,
                                                 view(p2), prm.get("D"), lp)
            else:
                y = oracle.mixer_decode_unfused(row, sw, window, [blk], inner, view(p2),
                                                prm.get("D"), lp)
            assert torch.equal(y.view(torch.int16), gs[r * Q + p:r * Q + p + 1].view(torch.int16)), (r, p)
        assert torch.equal(view(p2)[blk][:, :width], view(p1)[int(slots[r, Q - 1])][:, :width])


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
@pytest.mark.parametrize("accepted", [1, 2, 4])
def test_state_copy_rules_resume_after_partial_acceptance(kind, accepted):
    """The prefix-caching copy rules (model.py:285-304): after a verify step
    of Q tokens over blocks b_0 .. b_{Q-1}, copying each slice by its rule
    (sliding window from b_0 offset by accepted - 1, snapshot from
    b_{accepted-1}) into a fresh block and decoding the next token there
    gives, bit for bit, what decoding the accepted tokens and then that token
    one at a time gives.  A wrong window offset or snapshot block fails it."""
    from evo2_flash_amd.state import (MambaCopySpec, get_conv_copy_spec,
                                      get_mamba_state_copy_func, get_temporal_copy_spec)
    H, nb, nspec, Q = 64, 12, 3, 4
    prm = mixer_params(kind, H, 7, in_proj_fp8=False)
    sw = prm["short_filter"].view(3 * H, 3)
    inner, lp, poles, view = _operator(kind, prm, H)
    pool = _spec_pool(H, nb, nspec, 8)
    g = torch.Generator().manual_seed(9)
    blocks = [2, 3, 4, 5]
    z = (torch.randn(Q + 1, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    spec = _clone(pool, nspec)
    oracle.mixer_decode_speculative(z[:Q], sw, spec.conv_view(), inner, view(spec),
                                    prm.get("D"), torch.tensor([blocks]), [0, Q], [1], Q,
                                    poles=poles, emulate_kernels=True)
    rules = get_mamba_state_copy_func()
    assert rules == (get_conv_copy_spec, get_temporal_copy_spec, get_temporal_copy_spec)
    for state, rule in zip(spec.kv_cache, rules):
        cs = rule(state, blocks, 0, accepted)
        assert isinstance(cs, MambaCopySpec) and cs.num_elements > 0
    dst = 10
    spec.copy_cached_state(blocks, 0, accepted, dst)
    y_spec = oracle.hyena_decode_emulated(z[Q:Q + 1], sw, spec.conv_view()[..., :2],
                                          torch.tensor([dst]), inner, view(spec),
                                          prm.get("D"), lp)
    chain = _clone(pool, nspec)
    for p in list(range(accepted)) + [Q]:
        y = oracle.hyena_decode_emulated(z[p:p + 1], sw, chain.conv_view()[..., :2],
                                         torch.tensor([blocks[0]]), inner, view(chain),
                                         prm.get("D"), lp)
    assert torch.equal(y.view(torch.int16), y_spec.view(torch.int16))
    width = inner.shape[1] - 1 if kind != "hcl" else 16
    assert torch.equal(view(chain)[blocks[0]][:, :width], view(spec)[dst][:, :width])
    assert torch.equal(chain.conv_view()[blocks[0]][:, :2], spec.conv_view()[dst][:, :2])
