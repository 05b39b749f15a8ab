"""GPU parity of speculative decode (mixers.py:17-35, 578-660, 952-1074,
1153-1193) against the oracle.

* The speculative form of the short-conv update against
  `oracle.causal_conv1d_update_spec_ref`: bitwise outputs and windows, with
  ragged draft counts, random accepted offsets, in-place and moved blocks.
* The LI verify kernel on the stamped 17-column state rows: bitwise against
  the kernel-order emulation, the stamp column untouched.
* Each mixer kind through three steps on a speculative state pool: prefill;
  a mixed step (verify rows of 4 / 1 / 3 tokens from fresh prefills, then a
  new prefill); a second verify step after accepting 2 / 1 / 3 of those rows,
  whose live snapshots the mixer must find from the position stamps alone.
  Outputs within 1e-2 of the oracle's composition from the same projection
  rows; every snapshot and window of the verify rows bitwise; stamps exact.
* The stamp kernels against `oracle.spec_accepted_ref` /
  `oracle.record_stamps_ref` on random pools: accepted counts and fault
  totals (null-block rows, out-of-range offsets, a slot outside the pool,
  the engine-count cross-check) and every stamp after recording (ragged
  query lengths, shifted windows, prefill blocks), exact.
"""

import itertools

import pytest
import torch

import oracle
from evo2_flash_amd.config import HyenaConfig
from evo2_flash_amd.metadata import HyenaMamba2Metadata
from evo2_flash_amd.mixers import load_mixer_params, make_mixer, set_forward_context
from evo2_flash_amd.short_conv import causal_conv1d_update
from evo2_flash_amd.speculative import record_stamps, spec_accepted
from evo2_flash_amd.state import HyenaStatePool
from evo2_flash_amd.synthetic import mixer_params
from evo2_flash_amd.verify import iir_snapshots

from _cases import max_rel_err, verify_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
_ids = itertools.count()


def _bits(t):
    return t.contiguous().view(torch.uint8)


@pytest.mark.parametrize("K,nspec,moved", [(3, 3, False), (3, 3, True), (2, 5, False),
                                           (4, 2, True)])
def test_spec_short_conv_vs_oracle(K, nspec, moved):
    dim, nb, nreq = 768, 64, 9
    Q = nspec + 1
    g = torch.Generator().manual_seed(100 * K + nspec)
    lens = torch.randint(1, Q + 1, (nreq,), generator=g)
    lens[0], lens[3] = Q, 0                      # a full request and an empty one
    qsl = [0] + torch.cumsum(lens, 0).tolist()
    T = qsl[-1]
    x = (torch.randn(T + 3, dim, generator=g) * 1.5).to(torch.bfloat16)  # 3 uncovered rows
    w = torch.randn(dim, K, generator=g).to(torch.bfloat16)
    width = K - 1 + nspec
    st = (torch.randn(nb, dim, width, generator=g) * 1.5).to(torch.bfloat16)
    slots = (torch.randperm(nb - 1, generator=g)[: nreq * Q] + 1).view(nreq, Q).to(torch.int32)
    acc = torch.randint(1, Q + 1, (nreq,), generator=g)
    in_col = out_col = None
    if moved:  # prefix caching: read one column of the slot row, write another
        in_col = torch.randint(0, Q, (nreq,), generator=g).to(torch.int32)
        out_col = torch.randint(0, Q, (nreq,), generator=g).to(torch.int32)
    # the native (blocks, width, dim) storage seen dim-first, as the pool does
    gst = st.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    print(f"spec conv K={K} nspec={nspec} moved={moved} T={T}", flush=True)
    out = causal_conv1d_update(
        x.to(DEV), gst, w.to(DEV), None, conv_state_indices=slots.to(DEV),
        num_accepted_tokens=acc.to(DEV), query_start_loc=torch.tensor(qsl, device=DEV),
        max_query_len=Q,
        block_idx_last_scheduled_token=None if out_col is None else out_col.to(DEV),
        initial_state_idx=None if in_col is None else in_col.to(DEV)).cpu()
    ref = oracle.causal_conv1d_update_spec_ref(x, st, w, slots, acc.tolist(), qsl, Q,
                                               in_col, out_col)
    assert torch.equal(out.float(), ref)
    assert torch.equal(_bits(gst.cpu()), _bits(st))


@pytest.mark.parametrize("H,width", [(320, 17), (200, 17), (96, 20), (64, 40)])
def test_iir_verify_on_stamped_rows(H, width):
    """The speculative LI slice has 17 fp32 per channel (stride 17): the
    verify kernel's strided path (also at an H that leaves part of a
    workgroup empty and at wider rows), bitwise, leaving the columns past the
    16 states alone."""
    nreq, Q, nb = 6, 4, 64
    prm, x, state, meta = verify_case("hcl", H, nreq, Q, nb, seed=7)
    ins, outs, starts, ends, accepted = meta
    poles = torch.exp(prm["log_poles"][..., 0].float())
    res = prm["residues"].float()
    wide = torch.randn(nb, H, width, generator=torch.Generator().manual_seed(8))
    wide[..., :16] = state
    gwide = wide.to(DEV)
    gmeta = tuple(t.to(DEV) for t in meta)
    print(f"iir verify stamped rows H={H} width={width}", flush=True)
    y = iir_snapshots(x.to(DEV), poles.to(DEV), res.to(DEV), gwide[..., :16], gmeta).cpu()
    ref_state = wide.clone()
    ref = oracle.iir_verify_emulated(x, poles, res, ref_state[..., :16], ins, outs, starts, ends,
                                     accepted)
    assert torch.equal(_bits(y), _bits(ref))
    assert torch.equal(_bits(gwide.cpu()), _bits(ref_state))


# ---------------------------------------------------------------- mixer steps
H, NSPEC, NBLK = 256, 3, 20
Q = NSPEC + 1
SLOTS = [[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]]
LENS = [37, 20, 9]


def _meta(decode=None, prefill=None, seq_lens=()):
    """decode: (query lengths, computed tokens); prefill: (lengths, blocks)."""
    m = HyenaMamba2Metadata()
    if decode:
        qlens, computed = decode
        qsl = [0]
        for n in qlens:
            qsl.append(qsl[-1] + n)
        m.num_decodes, m.num_decode_tokens = len(qlens), qsl[-1]
        m.state_indices_tensor_d = torch.tensor(SLOTS[:len(qlens)], dtype=torch.int32,
                                                device=DEV)
        m.query_start_loc_d = torch.tensor(qsl, dtype=torch.int32, device=DEV)
        m.num_computed_tokens_d = torch.tensor(computed, dtype=torch.int32, device=DEV)
    if prefill:
        lens, blocks = prefill
        qsl = [0]
        for n in lens:
            qsl.append(qsl[-1] + n)
        m.num_prefills, m.num_prefill_tokens = len(lens), qsl[-1]
        m.query_start_loc_p = torch.tensor(qsl, dtype=torch.int32, device=DEV)
        m.has_initial_states_p = torch.zeros(len(lens), dtype=torch.bool, device=DEV)
        m.state_indices_tensor_p = torch.tensor(blocks, dtype=torch.int32, device=DEV)
    m.seq_lens = torch.tensor(list(seq_lens), dtype=torch.int32, device=DEV)
    return m


def _oracle_step(kind, prm, z, cpool, qlens, accepted, prefill, poles):
    """The oracle's composition of one step from the projection rows z."""
    sw = prm["short_filter"].view(3 * H, 3)
    D = prm.get("D")
    parts = []
    nd = sum(qlens)
    if qlens:
        qsl = [0]
        for n in qlens:
            qsl.append(qsl[-1] + n)
        slots = torch.tensor(SLOTS[:len(qlens)])
        if kind == "hcl":
            inner, st = prm["residues"], cpool.ssm_view()
        else:
            K = prm["conv"].shape[-1]
            inner, st = prm["conv"].view(H, K), cpool.inner_view(K - 1)
        parts.append(oracle.mixer_decode_speculative(
            z[:nd], sw, cpool.conv_view(), inner, st, D, slots, qsl, accepted, Q,
            poles=poles if kind == "hcl" else None))
    if prefill:
        lens, blocks = prefill
        qsl = [0]
        for n in lens:
            qsl.append(qsl[-1] + n)
        init = [0] * len(lens)
        if kind == "hcl":
            parts.append(oracle.iir_mixer_prefill(
                z[nd:], sw, cpool.conv_view(), prm["residues"], prm["log_poles"][..., 0],
                cpool.ssm_view(), D, qsl, blocks, init))
        else:
            K = prm["conv"].shape[-1]
            parts.append(oracle.fir_mixer_prefill(
                z[nd:], sw, cpool.conv_view(), prm["conv"].view(H, K), cpool.inner_view(K - 1),
                D, qsl, blocks, init))
    g = torch.cat(parts).float()
    return (g @ prm["out_proj.weight"].float().t() + prm["out_proj.bias"].float())


def _cpu_pool(gp):
    p = HyenaStatePool(NBLK, H, "cpu", num_spec=NSPEC)
    p.raw.copy_(gp.raw.cpu())
    return p


def _check_verify_blocks(kind, prm, gp, cpool, qlens, computed):
    """Bitwise snapshots and windows of the verify rows, and exact stamps."""
    for r, q in enumerate(qlens):
        conv_blk = SLOTS[r][0]
        assert torch.equal(_bits(gp.conv_view()[conv_blk].cpu()),
                           _bits(cpool.conv_view()[conv_blk])), (r, "window")
        for p in range(q):
            blk = SLOTS[r][p]
            if kind == "hcl":
                a, b = gp.ssm_view()[blk].cpu(), cpool.ssm_view()[blk]
            else:
                K = prm["conv"].shape[-1]
                a, b = gp.inner_view(K - 1)[blk].cpu(), cpool.inner_view(K - 1)[blk]
            assert torch.equal(_bits(a), _bits(b)), (r, p)
            assert gp.stamps()[blk].item() == computed[r] + p + 1


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_speculative_mixer_steps_vs_oracle(kind):
    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=3, hcs_layer_idxs=[0], hcm_layer_idxs=[1],
                      hcl_layer_idxs=[2])
    layer = {"hcs": 0, "hcm": 1, "hcl": 2}[kind]
    mixer = make_mixer(cfg, layer, prefix=f"spec{next(_ids)}.mixer", device=DEV,
                       num_spec=NSPEC)
    prm = mixer_params(kind, H, seed=80 + layer, in_proj_fp8=False)
    load_mixer_params(mixer, prm)
    gp = HyenaStatePool(NBLK, H, DEV, num_spec=NSPEC)
    assert tuple(gp.kv_cache[0].shape[1:]) == mixer.get_state_shape()[0]
    mixer.kv_cache = gp.kv_cache
    zs = []
    mixer.in_proj.register_forward_hook(lambda mod, inp, out: zs.append(out[0].detach().cpu()))
    gen = torch.Generator().manual_seed(90 + layer)
    poles = torch.exp(mixer.log_poles[..., 0]).cpu() if kind == "hcl" else None

    # step A: three prompts, one per request's column-0 block
    hs = torch.randn(sum(LENS), H, generator=gen).to(torch.bfloat16)
    m = _meta(prefill=(LENS, [s[0] for s in SLOTS]), seq_lens=LENS)
    print(f"spec mixer {kind}: prefill {LENS}", flush=True)
    with set_forward_context(m):
        mixer(hs.to(DEV))
    assert [gp.stamps()[s[0]].item() for s in SLOTS] == LENS

    # step B: verify rows 4 / 1 / 3 from the prefills, then a new 25-token prompt
    qlens, new = [4, 1, 3], ([25], [13])
    computed = list(LENS)
    before = _cpu_pool(gp)
    hs = torch.randn(sum(qlens) + 25 + 2, H, generator=gen).to(torch.bfloat16)  # 2 padding rows
    m = _meta(decode=(qlens, computed), prefill=new,
              seq_lens=[c + q for c, q in zip(computed, qlens)] + [25])
    print(f"spec mixer {kind}: mixed step {qlens} + prefill {new[0]}", flush=True)
    with set_forward_context(m):
        out = mixer(hs.to(DEV)).cpu()
    ref = _oracle_step(kind, prm, zs[-1], before, qlens, [1, 1, 1], new, poles)
    n = sum(qlens) + 25
    assert (out[n:].float() == 0).all()
    assert max_rel_err(out[:n], ref) <= 1e-2
    _check_verify_blocks(kind, prm, gp, before, qlens, computed)
    assert gp.stamps()[13].item() == 25
    assert mixer.stamp_faults() == 0

    # step C: 2 / 1 / 3 of those rows were accepted; the mixer finds the live
    # snapshots from the stamps alone
    accepted = [2, 1, 3]
    computed = [c + a for c, a in zip(computed, accepted)]
    qlens = [2, 4, 1]
    before = _cpu_pool(gp)
    hs = torch.randn(sum(qlens), H, generator=gen).to(torch.bfloat16)
    m = _meta(decode=(qlens, computed), seq_lens=[c + q for c, q in zip(computed, qlens)])
    print(f"spec mixer {kind}: verify step {qlens} after accepting {accepted}", flush=True)
    with set_forward_context(m):
        out = mixer(hs.to(DEV)).cpu()
    ref = _oracle_step(kind, prm, zs[-1], before, qlens, accepted, None, poles)
    assert max_rel_err(out, ref) <= 1e-2
    _check_verify_blocks(kind, prm, gp, before, qlens, computed)
    assert mixer.stamp_faults() == 0


@pytest.mark.parametrize("seed,with_counts,shifted", [(0, False, False), (1, True, False),
                                                      (2, False, True)])
def test_stamp_kernels_vs_oracle(seed, with_counts, shifted):
    g = torch.Generator().manual_seed(seed)
    nblk, nreq, ncols, nspec = 300, 37, 6 if shifted else 4, 3
    pool = HyenaStatePool(nblk, 64, DEV, num_spec=nspec)
    stamps = pool.stamps()
    base = torch.randint(0, 5000, (nblk,), generator=g).float()
    stamps.copy_(base.to(DEV))
    perm = (torch.randperm(nblk - 1, generator=g)[: nreq * ncols] + 1).view(nreq, ncols)
    slots = perm.to(torch.int32)
    slots[3] = 0                                   # a padded request on the null block
    slots[5, 0] = nblk + 7                         # a slot outside the pool
    first = slots[:, 0].long().clamp(0, nblk - 1)
    off = torch.randint(-2, nspec + 3, (nreq,), generator=g)   # some outside [0, nspec]
    computed = (base[first].long() + off).clamp_min(0).to(torch.int32)
    counts = None
    if with_counts:
        counts = (off.clamp(0, nspec) + 1).to(torch.int32)
        counts[::4] += 1                           # disagree on every fourth request
    faults = torch.zeros((), dtype=torch.int64, device=DEV)
    print(f"stamp kernels seed={seed} counts={with_counts} shifted={shifted}", flush=True)
    acc = spec_accepted(stamps, slots.to(DEV), computed.to(DEV), nspec, faults,
                        None if counts is None else counts.to(DEV))
    ref_acc, ref_faults = oracle.spec_accepted_ref(base.tolist(), slots.tolist(),
                                                   computed.tolist(), nspec,
                                                   None if counts is None else counts.tolist())
    assert acc.cpu().tolist() == ref_acc
    assert int(faults) == ref_faults and ref_faults > 0

    qlens = torch.randint(0, nspec + 3, (nreq,), generator=g)
    qsl = torch.cat([torch.zeros(1, dtype=torch.long), qlens.cumsum(0)]).to(torch.int32)
    out_col = torch.randint(0, ncols - nspec, (nreq,), generator=g).to(torch.int32) \
        if shifted else None
    width = 1 + nspec
    # prefill blocks are never decode slots of the same step
    free = sorted(set(range(1, nblk)) - set(slots.view(-1).tolist()))
    pf_blocks = torch.tensor([0, free[0], free[-1]], dtype=torch.int32)
    pf_lens = torch.tensor([11, 2222, 4096], dtype=torch.int32)
    before = stamps.cpu().tolist()
    record_stamps(stamps, slots.to(DEV), qsl.to(DEV), computed.to(DEV), width,
                  None if out_col is None else out_col.to(DEV), pf_blocks.to(DEV),
                  pf_lens.to(DEV))
    ref = oracle.record_stamps_ref(before, slots.tolist(), qsl.tolist(), computed.tolist(),
                                   width, None if out_col is None else out_col.tolist(),
                                   pf_blocks.tolist(), pf_lens.tolist())
    assert stamps.cpu().tolist() == ref


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("packed", [False, True])
def test_verify_plan_kernel_vs_oracle(seed, paged, packed):
    """The step's verify plan (one launch) against `oracle.verify_plan_ref`:
    slot windows with and without prefix caching's block pointers (some
    running past the slot row), packed or one-row requests, the engine's
    counts (zeros clamped to 1), and the profiling-pool rule; exact."""
    from evo2_flash_amd.speculative import verify_plan
    g = torch.Generator().manual_seed(seed)
    nreq, cols, width = 9, 6, 4
    slots = torch.randint(0, 50, (nreq, cols), generator=g, dtype=torch.int32)
    lens = torch.randint(1, width + 1, (nreq,), generator=g)
    qsl = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)]).to(torch.int32)
    prev = torch.randint(0, cols - 1, (nreq,), generator=g, dtype=torch.int32)
    sched = torch.randint(0, cols, (nreq,), generator=g, dtype=torch.int32)
    eng = torch.randint(0, 4, (nreq,), generator=g, dtype=torch.int32)
    for pool, eng_on in ((100, True), (40, False)):   # 40 < 9 x 4: the profiling pool
        m = HyenaMamba2Metadata(num_decodes=nreq, num_decode_tokens=int(qsl[-1]) if packed else nreq)
        m.state_indices_tensor_d = slots.to(DEV)
        m.query_start_loc_d = qsl.to(DEV) if packed else None
        if paged:
            m.block_idx_last_scheduled_token_prev_step = prev.to(DEV)
            m.block_idx_last_scheduled_token = sched.to(DEV)
        m.num_accepted_tokens = eng.to(DEV) if eng_on else None
        plan = verify_plan(m, nreq, width, pool)
        w = width if paged else cols
        ref = oracle.verify_plan_ref(slots.tolist(), nreq, w, qsl=qsl.tolist() if packed else None,
                                     prev=prev.tolist() if paged else None,
                                     sched=sched.tolist() if paged else None,
                                     eng_acc=eng.tolist() if eng_on else None,
                                     null_all=pool < nreq * w)
        got = (plan.ins.tolist(), plan.outs.tolist(), plan.starts.tolist(), plan.ends.tolist(),
               plan.engine_accepted.tolist())
        assert got == tuple(ref), (pool, eng_on)
        assert verify_plan(m, nreq, width, pool) is plan   # kept for the step's other layers
        m.state_indices_tensor_d.add_(0)                    # an in-place update rebuilds it
        assert verify_plan(m, nreq, width, pool) is not plan


@pytest.mark.parametrize("seed", [0, 1])
def test_repair_kernel_vs_oracle(seed):
    """Align-mode repair (two launches) against `oracle.repair_prefill_ref` on
    a random speculative pool: repaired rows take all three slices of their
    source bitwise, every other block is untouched; a row whose source is
    another repaired row's destination is left alone and counted as a fault."""
    from evo2_flash_amd.speculative import repair_prefill_states
    g = torch.Generator().manual_seed(seed)
    nb, H = 24, 128
    pool = HyenaStatePool(nb, H, "cpu", num_spec=3)
    pool.raw.copy_(torch.randint(0, 255, pool.raw.shape, generator=g, dtype=torch.uint8))
    st = pool.stamps()
    st.copy_(torch.randint(0, 6, (nb,), generator=g).float())
    # row: dst, src, need -- and what happens
    #  0: 2 <- 3, need 3, dst stale, src right      repaired
    #  1: 4 <- 6, need 5, dst already right         untouched
    #  2: 7 <- 8, need 99, neither block right      untouched
    #  3: 9 <- 10, need 2, dst stale, src right     repaired
    #  4: 11 <- 12, fresh prefill (no initial state) untouched
    #  5: null destination                          untouched
    #  6: null source                               untouched
    #  7: 15 <- 9, need 4: wants block 9, which row 3 repairs: refused, a fault
    dst = [2, 4, 7, 9, 11, 0, 13, 15]
    src = [3, 6, 8, 10, 12, 5, 0, 9]
    need = [3, 5, 99, 2, 1, 1, 1, 4]
    init = [1, 1, 1, 1, 0, 1, 1, 1]
    for b, v in ((2, 0), (3, 3), (4, 5), (6, 5), (9, 4), (10, 2), (15, 1), (12, 1), (11, 0)):
        st[b] = float(v)
    gp = HyenaStatePool(nb, H, DEV, num_spec=3)
    gp.raw.copy_(pool.raw)
    m = HyenaMamba2Metadata(num_prefills=len(dst))
    m.state_indices_tensor_p = torch.tensor(dst, dtype=torch.int32, device=DEV)
    m.state_src_block_p = torch.tensor(src, dtype=torch.int64, device=DEV)
    m.computed_before_p = torch.tensor(need, dtype=torch.int64, device=DEV)
    m.has_initial_states_p = torch.tensor(init, dtype=torch.bool, device=DEV)
    faults = torch.zeros((), dtype=torch.int64, device=DEV)
    repair_prefill_states(gp.kv_cache, gp.stamps(), m, faults)
    flat = [t.reshape(nb, -1) for t in pool.kv_cache]
    ref_slices, rows = oracle.repair_prefill_ref(flat, st.tolist(), dst, src, need, init)
    # the oracle's gather-then-scatter repairs the clashing row 7 as well;
    # the kernel refuses it and counts one fault
    assert rows == [0, 3, 7]
    expect = [t.clone() for t in ref_slices]
    for t_exp, t_old in zip(expect, flat):
        t_exp[dst[7]] = t_old[dst[7]]
    for k in range(3):
        assert torch.equal(_bits(gp.kv_cache[k].reshape(nb, -1).cpu()), _bits(expect[k])), k
    assert int(faults) == 1
