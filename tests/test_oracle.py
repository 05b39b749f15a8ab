"""Pins the CPU oracle (oracle/hyena_ref.py) against checks that do not share
its code: float64 brute force written from the mathematics, closed forms,
impulse responses, invariants and hand-computed known answers.  Each check is
chosen so that a plausible mistake in the oracle (a flipped tap order, a
dropped continuation term, eps inside the sqrt, a wrong window column) fails.

CPU only; runs in seconds.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from evo2_flash_amd.metadata import build_metadata, host_tables
from evo2_flash_amd.state import HyenaStatePool, page_bytes
from evo2_flash_amd.synthetic import mixer_params, random_slot_table

from _cases import bf16_ulp_diff, decode_case, max_rel_err, verify_case


def _qsl(lens):
    q = [0]
    for n in lens:
        q.append(q[-1] + n)
    return q


# ---------------------------------------------------------------- bf16
def test_bf_round_to_nearest_even():
    one = 1.0
    cases = {
        one + 2 ** -8: 1.0,              # tie -> even mantissa (1.0)
        one + 3 * 2 ** -8: 1.0 + 2 ** -6,  # tie -> even (up)
        one + 2 ** -8 + 2 ** -20: 1.0 + 2 ** -7,  # above the tie -> up
        -2.0 - 2 ** -7: -2.0,            # tie at exponent 1 -> even
    }
    for x, want in cases.items():
        assert oracle.bf(torch.tensor([x], dtype=torch.float32)).item() == want, x


# ---------------------------------------------------------------- depthwise FIR
def _fir_f64(seq, w, prev):
    """y_t = sum_k w[k] * x_{t-(K-1)+k} over cat(prev, seq), float64 loops."""
    dim, L = seq.shape
    K = w.shape[1]
    full = np.concatenate([prev, seq], axis=1)
    y = np.zeros((dim, L))
    for t in range(L):
        for k in range(K):
            y[:, t] += w[:, k] * full[:, t + k]
    return y


@pytest.mark.parametrize("K", [3, 7, 128])
def test_depthwise_prefill_vs_float64(K):
    dim, nblk = 6, 8
    lens, has_init = [40, 3, 0, 150, 1], [0, 1, 0, 1, 1]
    qsl = _qsl(lens)
    g = torch.Generator().manual_seed(K)
    x = torch.randn(qsl[-1], dim, generator=g).to(torch.bfloat16)
    w = (torch.randn(dim, K, generator=g) * 0.3).to(torch.bfloat16)
    slots = [3, 5, 6, 1, 2]
    state = torch.randn(nblk, dim, 127, generator=g)
    state0 = state.clone()
    y = oracle.depthwise_prefill(x, w, qsl, slots, has_init, state, K)
    wd = w.double().numpy()
    for j, (a, b) in enumerate(zip(qsl[:-1], qsl[1:])):
        blk = slots[j]
        if b == a:
            assert torch.equal(state[blk], state0[blk])  # empty segment: untouched
            continue
        prev = state0[blk, :, :K - 1].double().numpy() if has_init[j] else np.zeros((dim, K - 1))
        seq = x[a:b].double().numpy().T
        ref = torch.from_numpy(_fir_f64(seq, wd, prev).T).float().to(torch.bfloat16)
        assert bf16_ulp_diff(y[a:b], ref).max().item() <= 1, j
        # new window: last K-1 inputs of cat(prev, seq), oldest first, full even if short
        full = np.concatenate([prev, seq], axis=1)
        want = torch.from_numpy(full[:, -(K - 1):]).float()
        assert torch.equal(state[blk, :, :K - 1], want), j
        assert torch.equal(state[blk, :, K - 1:], state0[blk, :, K - 1:])


@pytest.mark.parametrize("K", [3, 7, 128])
def test_depthwise_impulse_pins_tap_order(K):
    """A unit impulse at t0 gives y[t0 + j] = w[K-1-j]: w[:, -1] pairs with
    the current sample (cross-correlation order)."""
    dim, L, t0 = 2, K + 10, 4
    x = torch.zeros(L, dim, dtype=torch.bfloat16)
    x[t0] = 1.0
    w = torch.arange(1, K + 1, dtype=torch.float32).repeat(dim, 1).to(torch.bfloat16)
    state = torch.zeros(2, dim, 127)
    y = oracle.depthwise_prefill(x, w, [0, L], [1], [0], state, K)
    for j in range(L - t0):
        want = float(w[0, K - 1 - j]) if j < K else 0.0
        assert y[t0 + j, 0].item() == want
    assert (y[:t0] == 0).all()


def test_depthwise_split_invariance():
    """prefill(L) == prefill(a) then a continued prefill(L - a), within 1 ulp."""
    dim, K, L = 5, 128, 300
    g = torch.Generator().manual_seed(2)
    x = torch.randn(L, dim, generator=g).to(torch.bfloat16)
    w = (torch.randn(dim, K, generator=g) * 0.1).to(torch.bfloat16)
    for a in (1, 50, 127, 200):
        s1 = torch.zeros(2, dim, 127)
        y1 = oracle.depthwise_prefill(x, w, [0, L], [1], [0], s1, K)
        s2 = torch.zeros(2, dim, 127)
        ya = oracle.depthwise_prefill(x[:a], w, [0, a], [1], [0], s2, K)
        yb = oracle.depthwise_prefill(x[a:], w, [0, L - a], [1], [1], s2, K)
        assert bf16_ulp_diff(y1, torch.cat([ya, yb])).max().item() <= 1
        assert torch.equal(s1, s2)


# ---------------------------------------------------------------- modal filter / LI
def test_hcl_filter_single_pole_closed_form():
    """S = 1: h[d, l] = r * p^t exactly as the geometric sequence."""
    r = torch.tensor([[0.5], [-2.0]])
    p = torch.tensor([[0.9], [0.5]])
    t = torch.arange(20, dtype=torch.float32)
    h = oracle.hcl_compute_filter(r, torch.log(p), t)
    want = r.double() * p.double() ** t.double()
    assert torch.allclose(h.double(), want, rtol=1e-5, atol=1e-7)


def _recurrence_f64(seq, res, lp, s0):
    p = np.exp(lp.astype(np.float64))
    H, L = seq.shape
    s = np.zeros(res.shape) if s0 is None else s0.astype(np.float64).copy()
    y = np.empty((H, L))
    for t in range(L):
        s = p * s + seq[:, t:t + 1]
        y[:, t] = (res * s).sum(1)
    return y, s


@pytest.mark.parametrize("with_prev", [False, True])
@pytest.mark.parametrize("L", [1, 17, 400])
def test_iir_segment_vs_sequential_recurrence(L, with_prev):
    """The FFT form with the closed-form final state (and the continuation
    terms) equals the sequential recurrence s_t = p s_{t-1} + x_t."""
    H, S = 8, 16
    g = torch.Generator().manual_seed(L)
    prm = mixer_params("hcl", H, seed=L, in_proj_fp8=False)
    res, lp = prm["residues"], prm["log_poles"][..., 0]
    seq = torch.randn(H, L, generator=g)
    s_prev = torch.randn(H, S, generator=g) * 3 if with_prev else None
    y, st = oracle.iir_segment(seq, res, lp, s_prev)
    yr, sr = _recurrence_f64(seq.double().numpy(), res.double().numpy(), lp.numpy(),
                             None if s_prev is None else s_prev.numpy())
    assert max_rel_err(y, torch.from_numpy(yr)) <= 1e-5
    assert max_rel_err(st, torch.from_numpy(sr)) <= 1e-5


def test_iir_segment_split_invariance():
    H, L, a = 4, 300, 123
    prm = mixer_params("hcl", H, seed=1, in_proj_fp8=False)
    res, lp = prm["residues"], prm["log_poles"][..., 0]
    seq = torch.randn(H, L, generator=torch.Generator().manual_seed(0))
    y, st = oracle.iir_segment(seq, res, lp, None)
    ya, sa = oracle.iir_segment(seq[:, :a], res, lp, None)
    yb, sb = oracle.iir_segment(seq[:, a:], res, lp, sa)
    assert max_rel_err(torch.cat([ya, yb], 1), y) <= 1e-5
    assert max_rel_err(sb, st) <= 1e-5


# ---------------------------------------------------------------- mixer prefill
def _short_f64(z, w, prev2):
    """K=3 short filter of one segment in float64, output rounded to bf16."""
    return torch.from_numpy(_fir_f64(z.double().numpy().T, w.double().numpy(),
                                     prev2).T).float().to(torch.bfloat16)


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_mixer_prefill_vs_float64(kind):
    """Composition of the mixer prefill (A.2): short filter, gate, inner
    operator, D, x2 -- recomputed here per segment in float64 from the
    definitions, with bf16 rounding only where a bf16 tensor is written."""
    H, nblk = 16, 6
    lens, has_init = [70, 0, 9, 130], [0, 0, 1, 1]
    qsl = _qsl(lens)
    prm = mixer_params(kind, H, seed=4, in_proj_fp8=False)
    g = torch.Generator().manual_seed(5)
    z = (torch.randn(qsl[-1], 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = [2, 3, 4, 5]
    pool = HyenaStatePool(nblk, H, "cpu")
    pool.kv_cache[0].copy_(torch.randn(pool.kv_cache[0].shape, generator=g).to(torch.bfloat16))
    pool.kv_cache[1].copy_(torch.randn(pool.kv_cache[1].shape, generator=g).to(torch.bfloat16).float())
    pool.kv_cache[2].copy_(torch.randn(pool.kv_cache[2].shape, generator=g))
    conv0 = pool.conv_view().clone()
    inner0 = pool.inner_view().clone()
    ssm0 = pool.ssm_view().clone()
    sw = prm["short_filter"].view(3 * H, 3)
    D = prm.get("D")
    if kind == "hcl":
        res, lp = prm["residues"], prm["log_poles"][..., 0]
        out = oracle.iir_mixer_prefill(z, sw, pool.conv_view(), res, lp, pool.ssm_view(), D,
                                       qsl, slots, has_init)
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        out = oracle.fir_mixer_prefill(z, sw, pool.conv_view(), w, pool.inner_view(K - 1), D,
                                       qsl, slots, has_init)
    for j, (a, b) in enumerate(zip(qsl[:-1], qsl[1:])):
        if b == a:
            continue
        blk = slots[j]
        prev2 = conv0[blk].double().numpy() if has_init[j] else np.zeros((3 * H, 2))
        zf = _short_f64(z[a:b], sw, prev2).float()
        x2, x1, v = zf[:, 0::3], zf[:, 1::3], zf[:, 2::3]
        u = oracle.bf(x1 * v)
        if kind == "hcl":
            s0 = ssm0[blk].numpy() if has_init[j] else None
            yv, sT = _recurrence_f64(u.double().numpy().T, res.double().numpy(), lp.numpy(), s0)
            y = oracle.bf(torch.from_numpy(yv.T).float())
            y = oracle.bf(y + oracle.bf(u * D.float()))
            assert max_rel_err(pool.ssm_view()[blk], torch.from_numpy(sT)) <= 1e-5
        else:
            prev = inner0[blk, :, :K - 1].double().numpy() if has_init[j] else np.zeros((H, K - 1))
            y = oracle.bf(torch.from_numpy(_fir_f64(u.double().numpy().T, w.double().numpy(),
                                                    prev).T).float())
            if D is not None:
                y = oracle.bf(y + oracle.bf(D.float() * u))
        ref = (x2 * y).to(torch.bfloat16)
        assert max_rel_err(out[a:b], ref) <= 1e-2, j
        # conv window: the last two z rows of cat(prev, segment), exactly
        full = torch.cat([torch.from_numpy(prev2).float(), z[a:b].float().t()], 1)
        assert torch.equal(pool.conv_view()[blk].float(), full[:, -2:]), j


# ---------------------------------------------------------------- decode
def _decode_f64(kind, prm, z, conv, inner_state, H):
    """One decode token per row from the definitions in float64 (no rounding
    inside the inner operator): returns (out, new conv window, new state)."""
    # The short tap's rounding points are part of the decode contract (A.1:
    # each product and the fp32 sum rounded to bf16); everything after the
    # gate is float64.
    sw = prm["short_filter"].view(3 * H, 3).float()
    c = conv.float()
    rb = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    short = rb((rb(c[:, 0] * sw[:, 0]) + rb(c[:, 1] * sw[:, 1])) + rb(z.float() * sw[:, 2]))
    short = short.double()
    x2, x1, v = short[0::3], short[1::3], short[2::3]
    u = (x1 * v).float().to(torch.bfloat16).double()
    if kind == "hcl":
        p = torch.exp(prm["log_poles"][..., 0].double())
        s = inner_state.double() * p + u[:, None]
        y = (s * prm["residues"].double()).sum(1)
        new_state = s
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K).double()
        win = inner_state[:, :K - 1].double()
        y = (win * w[:, :-1]).sum(1) + w[:, -1] * u
        new_state = torch.cat([win[:, 1:], u[:, None]], 1)
    if "D" in prm:
        y = y + prm["D"].double() * u
    return x2 * y, torch.stack([conv[:, 1].float(), z.float()], 1), new_state


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_decode_emulated_vs_float64(kind):
    H, B, nblk = 64, 6, 10
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=3, n_null=1)
    conv0 = pool.conv_view().clone()
    if kind == "hcl":
        st0 = pool.ssm_view().clone()
        inner, lp, st = prm["residues"], prm["log_poles"][..., 0], pool.ssm_view()
    else:
        K = prm["conv"].shape[-1]
        st0 = pool.inner_view().clone()
        inner, lp, st = prm["conv"].view(H, K), None, pool.inner_view(K - 1)
    raw0 = pool.raw.clone()
    out = oracle.hyena_decode_emulated(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(),
                                       slots, inner, st, prm.get("D"), lp)
    for b in range(B):
        blk = int(slots[b])
        if blk == 0:
            assert (out[b].float() == 0).all()
            continue
        ref, conv_new, st_new = _decode_f64(kind, prm, z[b], conv0[blk], st0[blk], H)
        assert max_rel_err(out[b], ref) <= 1e-2, b
        assert torch.equal(pool.conv_view()[blk].float(), conv_new)
        if kind == "hcl":
            assert max_rel_err(pool.ssm_view()[blk], st_new) <= 1e-6
        else:
            K = prm["conv"].shape[-1]
            assert torch.equal(pool.inner_view()[blk, :, :K - 1], st_new.float())
    # the null block's page and every block no row maps to are untouched
    used = {int(s) for s in slots} - {0}
    for blk in range(nblk):
        if blk not in used:
            assert torch.equal(pool.raw[blk], raw0[blk]), blk


@pytest.mark.parametrize("K", [7, 128])
def test_fir_decode_one_vs_float64(K):
    """The reference's unfused FIR decode (mixers.py:555-565): the output is
    the K-tap sum over the window and the new sample, taps in
    cross-correlation order (w[:, -1] multiplies the new sample), and the
    window shifts left by one with the sample appended; rows whose block is
    not named are untouched."""
    H, nblk = 16, 5
    g = torch.Generator().manual_seed(K)
    w = torch.randn(H, K, generator=g).to(torch.bfloat16)
    state = torch.randn(nblk, H, K - 1, generator=g)
    x = torch.randn(2, H, generator=g).to(torch.bfloat16)
    idx = torch.tensor([3, 1])
    st0 = state.clone()
    y = oracle.fir_decode_one(x, w, idx, state)
    for r, blk in enumerate(idx.tolist()):
        win = st0[blk].double()
        want = sum(win[:, k] * w[:, k].double() for k in range(K - 1)) \
            + w[:, K - 1].double() * x[r].double()
        assert max_rel_err(y[r], want) <= 1e-2
        assert torch.equal(state[blk, :, :K - 2], st0[blk, :, 1:])
        assert torch.equal(state[blk, :, K - 2], x[r].float())
    for blk in (0, 2, 4):
        assert torch.equal(state[blk], st0[blk])
    # an impulse window picks out one tap
    imp = torch.zeros(1, H, K - 1)
    imp[0, :, 0] = 1.0
    y1 = oracle.fir_decode_one(torch.zeros(1, H, dtype=torch.bfloat16), w, torch.tensor([0]), imp)
    assert torch.equal(y1[0], w[:, 0])


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_decode_emulated_vs_unfused(kind):
    """The rounding-point emulation and the unfused fp32 path agree to 1e-2
    and write the same windows."""
    H, B, nblk = 128, 8, 12
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=9)
    p2 = HyenaStatePool(nblk, H, "cpu")
    p2.raw.copy_(pool.raw)
    sw = prm["short_filter"].view(3 * H, 3)
    if kind == "hcl":
        args = (prm["residues"], pool.ssm_view(), prm["D"], prm["log_poles"][..., 0])
        args2 = (prm["residues"], p2.ssm_view(), prm["D"], prm["log_poles"][..., 0])
    else:
        K = prm["conv"].shape[-1]
        args = (prm["conv"].view(H, K), pool.inner_view(K - 1), prm.get("D"), None)
        args2 = (prm["conv"].view(H, K), p2.inner_view(), prm.get("D"), None)
    o1 = oracle.hyena_decode_emulated(z, sw, pool.conv_view(), slots, *args)
    o2 = oracle.mixer_decode_unfused(z, sw, p2.conv_view(), slots, *args2)
    assert max_rel_err(o1, o2) <= 1e-2
    assert torch.equal(pool.kv_cache[0], p2.kv_cache[0])
    if kind == "hcl":
        assert max_rel_err(pool.kv_cache[2], p2.kv_cache[2]) <= 1e-6
    else:
        assert torch.equal(pool.kv_cache[1], p2.kv_cache[1])


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_decode_after_prefill_matches_longer_prefill(kind):
    """prefill(L) then one decode token == the last row of prefill(L + 1)."""
    H, L = 32, 140
    prm = mixer_params(kind, H, seed=6, in_proj_fp8=False)
    z = (torch.randn(L + 1, 3 * H, generator=torch.Generator().manual_seed(1)) * 1.3
         ).to(torch.bfloat16)
    sw = prm["short_filter"].view(3 * H, 3)
    D = prm.get("D")
    outs, pools = [], []
    for n in (L + 1, L):
        pool = HyenaStatePool(3, H, "cpu")
        if kind == "hcl":
            o = oracle.iir_mixer_prefill(z[:n], sw, pool.conv_view(), prm["residues"],
                                         prm["log_poles"][..., 0], pool.ssm_view(), D,
                                         [0, n], [1], [0])
        else:
            K = prm["conv"].shape[-1]
            o = oracle.fir_mixer_prefill(z[:n], sw, pool.conv_view(), prm["conv"].view(H, K),
                                         pool.inner_view(K - 1), D, [0, n], [1], [0])
        outs.append(o)
        pools.append(pool)
    pool = pools[1]
    if kind == "hcl":
        last = oracle.mixer_decode_unfused(z[L:], sw, pool.conv_view(), [1], prm["residues"],
                                           pool.ssm_view(), D, prm["log_poles"][..., 0])
    else:
        K = prm["conv"].shape[-1]
        last = oracle.mixer_decode_unfused(z[L:], sw, pool.conv_view(), [1],
                                           prm["conv"].view(H, K), pool.inner_view(), D)
    assert max_rel_err(last, outs[0][L:]) <= 1e-2
    assert torch.equal(pool.kv_cache[0], pools[0].kv_cache[0])


# ---------------------------------------------------------------- norm
def test_rms_norm_known_answer():
    """x = 2 everywhere, H = 4: ||x|| = 4, * H^-1/2 = 2, + eps -> x / 2 = 1."""
    x = torch.full((1, 4), 2.0, dtype=torch.bfloat16)
    w = torch.tensor([1.0, -0.5, 3.0, 0.25], dtype=torch.bfloat16)
    y = oracle.rms_norm(x, w, 0.0)
    assert torch.equal(y.float(), w.float().view(1, 4))


def test_rms_norm_eps_outside_sqrt():
    """y = w x / (||x|| H^-1/2 + eps) -- with a large eps, eps inside the
    sqrt would give a clearly different value."""
    H, eps = 64, 0.5
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(3, H, generator=g) * 0.1).to(torch.bfloat16)
    w = torch.randn(H, generator=g).to(torch.bfloat16)
    y = oracle.rms_norm(x, w, eps)
    xd = x.double()
    den = xd.norm(dim=-1, keepdim=True) * H ** -0.5 + eps
    ref = w.double() * xd / den
    assert max_rel_err(y, ref) <= 1e-2
    wrong = w.double() * xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps)
    assert max_rel_err(y, wrong) > 0.1


def test_rms_norm_residual():
    H = 32
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, H, generator=g).to(torch.bfloat16)
    r = torch.randn(2, H, generator=g).to(torch.bfloat16)
    w = torch.ones(H, dtype=torch.bfloat16)
    y, s = oracle.rms_norm(x, w, 1e-6, r)
    assert torch.equal(s, (x.float() + r.float()).to(torch.bfloat16))
    assert torch.equal(y, oracle.rms_norm(s, w, 1e-6))


# ---------------------------------------------------------------- fp8
def _e4m3_values():
    """All finite non-negative OCP e4m3fn values from the format definition:
    1 sign, 4 exponent (bias 7), 3 mantissa bits; exponent field 15 with
    mantissa 7 is NaN, so the largest finite value is 448."""
    vals = []
    for code in range(0x7F):
        e, m = code >> 3, code & 7
        vals.append((m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7))
    return vals


def _e4m3_encode(x):
    """Round-to-nearest-even onto e4m3fn codes (ties to the even code), with
    saturation at 448 as the clamp in quantize_input makes it."""
    vals = _e4m3_values()
    mag = min(abs(x), 448.0)
    best = min(range(len(vals)), key=lambda c: (abs(vals[c] - mag), c & 1))
    return (0x80 if (x < 0 or (x == 0 and math.copysign(1, x) < 0)) else 0) | best


def test_quantize_input_matches_format_definition():
    g = torch.Generator().manual_seed(3)
    x = torch.cat([torch.randn(500, generator=g) * 4,
                   torch.tensor([0.0, -0.0, 448.0, 449.0, -1e4, 1e4, 0.0087890625, 2 ** -10,
                                 2 ** -9 * 1.5, 240.0, 248.0, 256.0, 464.0, -17.0])])
    x = x.to(torch.bfloat16)
    scale = torch.tensor([0.75])
    q = oracle.quantize_input(x, scale).view(torch.uint8)
    for xi, qi in zip(x.float().tolist(), q.tolist()):
        v = xi / 0.75
        assert qi == _e4m3_encode(float(np.float32(v))), (xi, qi)


def test_fp8_linear_known_answer():
    """Small-integer e4m3 operands: every product and sum is exact in fp32."""
    g = torch.Generator().manual_seed(4)
    x = torch.randint(-4, 5, (5, 32), generator=g).float().to(torch.bfloat16)
    w8 = torch.randint(-3, 4, (7, 32), generator=g).float().to(torch.float8_e4m3fn)
    out = oracle.fp8_linear_dequant(x, w8, torch.tensor([1.0]), torch.tensor([0.5]))
    want = (x.double() @ w8.double().t() * 0.5).float().to(torch.bfloat16)
    assert torch.equal(out, want)


# ---------------------------------------------------------------- tables, metadata, state
def test_prefill_tables_known():
    seq, tiles = oracle.prefill_tables([0, 100, 100, 164, 165], [0, 1, 1, 0], 64)
    assert seq.tolist() == [[0, 100, 0], [100, 100, 1], [100, 164, 1], [164, 165, 0]]
    assert tiles.tolist() == [[0, 0], [0, 64], [2, 100], [3, 164]]
    s2, t2, ts = host_tables([0, 100, 100, 164, 165], [0, 1, 1, 0], 64, with_tile_start=True)
    assert s2 == [tuple(r) for r in seq.tolist()]
    assert t2 == [tuple(r) for r in tiles.tolist()]
    assert ts == [0, 2, 2, 3, 4]


def test_host_tables_reject_negative_segment():
    with pytest.raises(ValueError):
        host_tables([0, 5, 3], [0, 0], 64)


def test_metadata_decode_indices_column0():
    m = build_metadata(decode_slots=[4, 7], device="cpu")
    from evo2_flash_amd.metadata import decode_state_indices
    assert decode_state_indices(m).tolist() == [4, 7]
    m.state_indices_tensor_d = torch.tensor([[4, 9], [7, 8]], dtype=torch.int32)
    assert decode_state_indices(m).tolist() == [4, 7]


def test_state_pool_layout_7b():
    """The unified spec at H=4096: 2,392,064 bytes of payload per block; the
    three slices alias one page, conv and FIR slices stored state-major."""
    H = 4096
    assert page_bytes(H, align=1) == 2 * 3 * H * 2 + 127 * H * 4 + H * 16 * 4 == 2392064
    pool = HyenaStatePool(3, H, "cpu")
    conv, inner, ssm = pool.kv_cache
    assert conv.shape == (3, 2, 3 * H) and inner.shape == (3, 127, H) and ssm.shape == (3, H, 16)
    page = pool.page
    assert conv.stride(0) * 2 == page and inner.stride(0) * 4 == page and ssm.stride(0) * 4 == page
    assert pool.conv_view().shape == (3, 3 * H, 2) and pool.conv_view().stride(1) == 1
    assert pool.inner_view(6).shape == (3, H, 6) and pool.inner_view().stride(1) == 1
    pool.inner_view()[1, 5, 0] = 7.0   # (block 1, channel 5, oldest column)
    flat = pool.raw[1].view(torch.float32)
    assert flat[(2 * 3 * H * 2) // 4 + 5].item() == 7.0


def test_random_slot_table_is_permutation_without_null():
    s = random_slot_table(64, 65, seed=3)
    assert sorted(s.tolist()) == list(range(1, 65))
    assert not torch.equal(s, torch.arange(1, 65, dtype=torch.int32))
    with pytest.raises(ValueError):
        random_slot_table(65, 65, seed=3)


# ---------------------------------------------------------------- speculative verify
def _verify_float64(kind, prm, x, state, meta):
    """Each request's tokens run one by one in float64 from its source
    snapshot: y per row, and the window / state after every token."""
    ins, outs, starts, ends, accepted = meta
    y = torch.zeros(x.shape, dtype=torch.float64)
    snaps = {}
    for r in range(ins.shape[0]):
        src = int(ins[r, int(accepted[r]) - 1])
        st = state[src].double().clone()
        for pos in range(int(ends[r] - starts[r])):
            t = int(starts[r]) + pos
            xt = x[t].double()
            if kind == "hcl":
                st = st * torch.exp(prm["log_poles"][..., 0].double()) + xt[:, None]
                y[t] = (prm["residues"].double() * st).sum(-1)
            else:
                K = prm["conv"].shape[-1]
                w = prm["conv"].view(-1, K).double()
                y[t] = (st * w[:, :-1]).sum(-1) + w[:, -1] * xt
                st = torch.cat([st[:, 1:], xt[:, None]], dim=1)
            snaps[(r, pos)] = st.clone()
    return y, snaps


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_verify_emulated_vs_float64(kind):
    """Snapshots after every token, outputs on every covered row, nothing
    written to the null block, to positions past a request's tokens or to
    the source blocks."""
    H, nreq, Q, nblk = 48, 5, 4, 60
    prm, x, state, meta = verify_case(kind, H, nreq, Q, nblk, seed=31, x_dtype=torch.float32)
    ins, outs, starts, ends, accepted = meta
    y64, snaps = _verify_float64(kind, prm, x, state, meta)
    st = state.clone()
    if kind == "hcl":
        poles = torch.exp(prm["log_poles"][..., 0].float())
        y = oracle.iir_verify_emulated(x, poles, prm["residues"], st, *meta)
        y2 = oracle.iir_decode_snapshots(x, poles, prm["residues"], state.clone(), *meta)
        tol = 1e-5
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        y = oracle.fir_verify_emulated(x, w, st, *meta)
        y2 = oracle.fir_decode_snapshots(x, w, state.clone(), *meta)
        tol = 1e-5
    assert ((y.double() - y64).abs().max() / y64.abs().max()).item() <= tol
    assert max_rel_err(y, y2) <= tol
    written = set()
    for (r, pos), s64 in snaps.items():
        d = int(outs[r, pos])
        if d == 0:
            continue
        written.add(d)
        if kind == "hcl":
            assert ((st[d].double() - s64).abs().max() / s64.abs().max()).item() <= 1e-5
        else:
            assert torch.equal(st[d].double(), s64)  # windows are copies of inputs
    for b in range(nblk):
        if b not in written:
            assert torch.equal(st[b], state[b]), b


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_verify_one_token_matches_decode_order(kind):
    """The one-token form rounds to the fused decode step's inner value bit
    for bit: both keep the same summation tree (triton_verifier.py:17-43,
    128-131 against triton_decode.py:81-143)."""
    from oracle import hyena_ref
    H, B, nblk = 64, 6, 20
    prm, x, state, _ = verify_case(kind, H, B, 1, nblk, seed=7)
    slots = torch.randperm(nblk - 1)[:B].to(torch.int32)[:, None] + 1
    st = state.clone()
    if kind == "hcl":
        poles = torch.exp(prm["log_poles"][..., 0].float())
        y = oracle.iir_verify_emulated(x, poles, prm["residues"], st, slots, slots, None, None,
                                       None)
        for b in range(B):
            s = state[int(slots[b])] * poles + x[b].float()[:, None]
            r = s * prm["residues"]
            r = r[:, :8] + r[:, 8:]
            r = r[:, :4] + r[:, 4:]
            r = r[:, :2] + r[:, 2:]
            assert torch.equal(y[b].float(), oracle.bf((r[:, 0] + r[:, 1]) + 0.0))
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        y = oracle.fir_verify_emulated(x, w, st, slots, slots, None, None, None)
        summ = hyena_ref._hcm_sum if K == 128 else hyena_ref._hcs_sum
        for b in range(B):
            ref = summ(state[int(slots[b])].float(), w.float(), x[b].float())
            assert torch.equal(y[b].float(), ref)


@pytest.mark.parametrize("kind", ["hcm", "hcl"])
def test_verify_equals_sequential_one_token_steps(kind):
    """Q draft tokens in one verify step == Q one-token steps chained through
    the snapshots (outputs and every snapshot, bit for bit)."""
    H, Q, nblk = 32, 4, 20
    prm, x, state, _ = verify_case(kind, H, 1, Q, nblk, seed=5, x_dtype=torch.float32)
    ins = torch.tensor([[3, 4, 5, 6]], dtype=torch.int32)
    outs = torch.tensor([[10, 11, 12, 13]], dtype=torch.int32)
    meta = (ins, outs, torch.tensor([0]), torch.tensor([Q]), torch.tensor([2]))
    s1, s2 = state.clone(), state.clone()
    s2[10] = s2[4]   # the one-token chain starts from the accepted snapshot in place
    if kind == "hcl":
        poles = torch.exp(prm["log_poles"][..., 0].float())
        y1 = oracle.iir_verify_emulated(x[:Q], poles, prm["residues"], s1, *meta)
        steps = [oracle.iir_verify_emulated(x[p:p + 1], poles, prm["residues"], s2,
                                            torch.tensor([[10 + max(p - 1, 0)]], dtype=torch.int32),
                                            torch.tensor([[10 + p]], dtype=torch.int32),
                                            None, None, None) for p in range(Q)]
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        y1 = oracle.fir_verify_emulated(x[:Q], w, s1, *meta)
        steps = []
        for p in range(Q):
            if p:
                s2[10 + p] = s2[10 + p - 1]
            steps.append(oracle.fir_verify_emulated(
                x[p:p + 1], w, s2, torch.tensor([[10 + p]], dtype=torch.int32),
                torch.tensor([[10 + p]], dtype=torch.int32), None, None, None))
    assert torch.equal(y1, torch.cat(steps))
    for p in range(Q):
        assert torch.equal(s1[10 + p], s2[10 + p]), p


# ---------------------------------------------------------------- Hopper fp8 model
def _fa(pairs, K=32):
    """fast_accum_mm of one output from (a, b) pairs placed at k = 0, 1, ..."""
    a = torch.zeros(1, K)
    b = torch.zeros(1, K)
    for k, (x, y) in enumerate(pairs):
        a[0, k], b[0, k] = x, y
    # the model takes E4M3 values: check the test's operands are representable
    assert torch.equal(a.to(torch.float8_e4m3fn).float(), a)
    assert torch.equal(b.to(torch.float8_e4m3fn).float(), b)
    return oracle.fast_accum_mm(a, b).item()


def test_fast_accum_known_answers():
    """Hand-worked cases of the fast-accumulation model (fp8_emul.py:8-20),
    each chosen so that plain fp32 accumulation gives a different answer."""
    # in-group alignment to the largest operand exponent sum (10): the 2^-8
    # product is below the 2^-3 ulp and is dropped (fp32: 1024.00390625)
    assert _fa([(32.0, 32.0), (2.0 ** -4, 2.0 ** -4)]) == 1024.0
    # the accumulator's exponent aligns the next group: 2^16, then 1 + ... in
    # the second group is below its 2^3 ulp (fp32: 65537)
    assert _fa([(256.0, 256.0)] + [(0.0, 0.0)] * 31 + [(1.0, 1.0)], K=64) == 65536.0
    # alignment comes from the operand exponents (0 + 0), not the product's
    # (2.25 has exponent 1): the third term 1.5 * 2^-13 keeps one 2^-13 ulp;
    # aligned at the product exponent it would vanish (answer 0.75)
    assert _fa([(1.5, 1.5), (-1.5, 1.0), (6 * 2.0 ** -9, 2.0 ** -6)]) == 0.75 + 2.0 ** -13
    # truncation toward zero: -1.5 ulp -> -1 ulp (round-to-nearest: 1 - 2^-12)
    assert _fa([(1.0, 1.0), (-4 * 2.0 ** -9, 1.5 * 2.0 ** -6)]) == 1.0 - 2.0 ** -13
    # renormalisation keeps 13 fraction bits of the sum's own exponent:
    # 1 + 2^-13 survives, 2 + 2^-13 becomes 2
    assert _fa([(1.0, 1.0), (1.0, 2.0 ** -9), (2.0 ** -4, 1.0 / 256)]) == 1.0 + 2.0 ** -9 + 2.0 ** -12
    assert _fa([(1.0, 1.0), (1.0, 1.0), (2.0 ** -7, 2.0 ** -6)]) == 2.0
    assert _fa([(1.0, 1.0), (2.0 ** -7, 2.0 ** -6)]) == 1.0 + 2.0 ** -13
    assert _fa([]) == 0.0


def test_fp8_linear_fast_accum_scales_known_answer():
    """The emulated static W8A8 linear's quantisation and scale epilogue
    (fp8_emul_triton.py:181-191), hand-worked with non-unit scales.
    x / s_in must be exact E4M3 values, the products exact, the sum below
    the fast-accumulation ulp, and the epilogue acc * s_in * s_w then rounds
    once to bf16:
      x = (1, 2, -0.5, 3, 0 ...), s_in = 0.5 -> (2, 4, -1, 6, 0 ...)
      row 0: w = (1, 0.5, 2, -1)      -> acc = 2 + 2 - 2 - 6 = -4
      row 1: w = (0.25, 0.125, 4, 1)  -> acc = 0.5 + 0.5 - 4 + 6 = 3
      s_w = 0.375 -> out = acc * 0.1875 = (-0.75, 0.5625), exact in bf16;
    and a saturating case: x = 300 with s_in = 0.5 clamps to 448, so the
    output is 448 * w * s_in * s_w, not 600 * w * s_in * s_w."""
    pad = lambda rows: torch.nn.functional.pad(torch.tensor(rows), (0, 28))  # K = 32
    x = pad([[1.0, 2.0, -0.5, 3.0]]).to(torch.bfloat16)
    w = pad([[1.0, 0.5, 2.0, -1.0], [0.25, 0.125, 4.0, 1.0]]).to(torch.float8_e4m3fn)
    out = oracle.fp8_linear_fast_accum(x, w, 0.5, 0.375)
    assert out.dtype == torch.bfloat16 and out.shape == (1, 2)
    assert out.float().tolist() == [[-0.75, 0.5625]]
    # the scales are not applied to each other first: a non-dyadic s_w rounds
    # only in the final bf16 cast: acc = 3, 3 * 0.5 * 0.1 = 0.15 -> bf16(0.15)
    out = oracle.fp8_linear_fast_accum(x, w[1:], 0.5, 0.1)
    assert out.float().item() == torch.tensor(3 * 0.5 * 0.1).to(torch.bfloat16).float().item()
    sat = oracle.fp8_linear_fast_accum(pad([[300.0, 0, 0, 0]]).to(torch.bfloat16), w[:1],
                                       0.5, 0.375)
    assert sat.float().item() == 448.0 * 1.0 * 0.5 * 0.375


def test_fast_accum_close_to_fp32_but_not_equal():
    g = torch.Generator().manual_seed(3)
    a = (torch.randn(16, 256, generator=g) * 4).to(torch.float8_e4m3fn).float()
    b = (torch.randn(24, 256, generator=g) * 0.05).to(torch.float8_e4m3fn).float()
    fa = oracle.fast_accum_mm(a, b)
    ref = a.double() @ b.double().t()
    # each group loses less than 33 ulps of 2^(e - 13): within 1e-2 of fp64
    assert ((fa.double() - ref).abs().max() / ref.abs().max()).item() < 1e-2
    assert not torch.equal(fa, (a @ b.t()).float())
    with pytest.raises(ValueError):
        oracle.fast_accum_mm(a[:, :40], b[:, :40])


# ------------------------------------------------------- short conv entry points
def test_conv1d_update_ref_known_answer():
    """Hand-worked: window (1, 2) / (0.5, -1), x = (3, 4), taps and bias exact
    in bf16, every product exact, so out = (7.5, 2.0); then a case where each
    product rounds: a = 1 + 2^-7, b = 1 - 2^-8, a*b = 1 + 2^-8 - 2^-15 -> bf16
    1.0, so three such products give 3.0 (exact products would give
    bf16(3.0116...) = 3.015625)."""
    st = torch.tensor([[[1.0, 2.0], [0.5, -1.0]]]).to(torch.bfloat16)
    w = torch.tensor([[0.5, 0.25, 2.0], [1.5, -0.75, 0.125]]).to(torch.bfloat16)
    x = torch.tensor([[3.0, 4.0]]).to(torch.bfloat16)
    out = oracle.causal_conv1d_update_ref(x, st, w, torch.tensor([0.5, 0.0]).to(torch.bfloat16))
    assert out.tolist() == [[7.5, 2.0]]
    assert st[0].float().tolist() == [[2.0, 3.0], [-1.0, 4.0]]
    a, b = 1 + 2 ** -7, 1 - 2 ** -8
    st = torch.full((1, 1, 2), a).to(torch.bfloat16)
    out = oracle.causal_conv1d_update_ref(torch.full((1, 1), a).to(torch.bfloat16), st,
                                          torch.full((1, 3), b).to(torch.bfloat16))
    assert out.item() == 3.0
    exact = (torch.tensor(a, dtype=torch.float64) * b * 3).to(torch.bfloat16).item()
    assert exact == 3.015625


def test_conv1d_update_ref_matches_decode_short_filter():
    """K=3 without bias is the fused decode's short filter, pinned by the
    decode tests: bitwise equal outputs and windows."""
    g = torch.Generator().manual_seed(3)
    dim, B, nb = 96, 5, 8
    w = (torch.randn(dim, 3, generator=g) * 0.3).to(torch.bfloat16)
    x = torch.randn(B, dim, generator=g).to(torch.bfloat16)
    st = torch.randn(nb, dim, 2, generator=g).to(torch.bfloat16)
    slots = [3, 1, 7, 2, 5]
    s1, s2 = st.clone(), st.clone()
    ref = oracle.short_conv_update(x, w, s1, slots)
    out = oracle.causal_conv1d_update_ref(x, s2, w, slots=slots)
    assert torch.equal(out, ref) and torch.equal(s1, s2)


def _conv_case(seed, lens, dim, K, nb=12):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    x = torch.randn(T, dim, generator=g).to(torch.bfloat16)
    w = (torch.randn(dim, K, generator=g) * 0.4).to(torch.bfloat16)
    st = torch.randn(nb, dim, K - 1, generator=g).to(torch.bfloat16)
    return x, w, st


@pytest.mark.parametrize("K", [2, 3, 4])
def test_conv1d_ref_vs_exact_products(K):
    """Against the reference's own torch form of the prefill short filter
    (`depthwise_prefill`, exact fp32 products): same outputs to bf16 rounding
    of the products, identical windows."""
    lens, has_init = [7, 0, 1, 40, 2], [1, 0, 1, 0, 1]
    slots = [4, 9, 2, 6, 11]
    x, w, st = _conv_case(5, lens, 64, K)
    s1, s2 = st.clone(), st.clone()
    q = _qsl(lens)
    ref = oracle.depthwise_prefill(x, w, q, slots, has_init, s1, K).float()
    out = oracle.causal_conv1d_ref(x, w, None, None, q, slots, has_init, s2)
    assert max_rel_err(out, ref) <= 2e-2
    assert torch.equal(s1, s2)


def test_conv1d_ref_impulse_pins_tap_order():
    K, L, t0 = 4, 12, 5
    x = torch.zeros(L, 3).to(torch.bfloat16)
    x[t0] = 1.0
    g = torch.Generator().manual_seed(1)
    w = torch.randn(3, K, generator=g).to(torch.bfloat16)
    out = oracle.causal_conv1d_ref(x, w, None, None, [0, L], [0], [0], None)
    for j in range(L - t0):
        want = w[:, K - 1 - j].float() if j < K else torch.zeros(3)
        assert torch.equal(out[t0 + j], want), j
    assert torch.equal(out[:t0], torch.zeros(t0, 3))


def test_conv1d_ref_one_row_continuation_equals_update():
    x, w, st = _conv_case(7, [1, 1, 1], 48, 3)
    bias = torch.linspace(-1, 1, 48).to(torch.bfloat16)
    s1, s2 = st.clone(), st.clone()
    slots = [2, 5, 8]
    a = oracle.causal_conv1d_ref(x, w, bias, None, [0, 1, 2, 3], slots, [1, 1, 1], s1)
    b = oracle.causal_conv1d_update_ref(x, s2, w, bias, None, slots)
    assert torch.equal(a, b) and torch.equal(s1, s2)


def test_conv1d_ref_split_invariance():
    L, cut = 23, 9
    x, w, st = _conv_case(9, [L], 32, 3)
    s1, s2 = st.clone(), st.clone()
    y = oracle.causal_conv1d_ref(x, w, None, None, [0, L], [3], [1], s1)
    ya = oracle.causal_conv1d_ref(x[:cut], w, None, None, [0, cut], [3], [1], s2)
    yb = oracle.causal_conv1d_ref(x[cut:], w, None, None, [0, L - cut], [3], [1], s2)
    assert torch.equal(y, torch.cat([ya, yb])) and torch.equal(s1, s2)


def test_conv1d_ref_silu_closed_form():
    st = torch.tensor([[[1.0, 2.0], [0.5, -1.0]]]).to(torch.bfloat16)
    w = torch.tensor([[0.5, 0.25, 2.0], [1.5, -0.75, 0.125]]).to(torch.bfloat16)
    x = torch.tensor([[3.0, 4.0]]).to(torch.bfloat16)
    out = oracle.causal_conv1d_update_ref(x, st, w, torch.tensor([0.5, 0.0]).to(torch.bfloat16),
                                          "silu")
    want = torch.nn.functional.silu(torch.tensor([7.5, 2.0])).to(torch.bfloat16).float()
    assert torch.equal(out[0], want)


def test_iir_final_state_recurrence_vs_closed_form():
    """The float64 recurrence against the reference's closed form
    sum_t x_t exp(lp (L-1-t)) (oracle.iir_segment, fp32)."""
    g = torch.Generator().manual_seed(4)
    H, L, S = 6, 57, 16
    seq = torch.randn(H, L, generator=g)
    lp = torch.log(torch.rand(H, S, generator=g) * 0.5 + 0.499)
    res = torch.randn(H, S, generator=g)
    _, st = oracle.iir_segment(seq, res, lp, None)
    rec = oracle.iir_final_state_recurrence(seq, lp)
    assert torch.allclose(st.double(), rec, rtol=1e-5, atol=1e-5)
