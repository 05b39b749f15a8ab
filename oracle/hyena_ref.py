"""CPU restatement of evo2_flash's Hyena mixer math (TEST INFRASTRUCTURE ONLY).

Citations are relative to the reference package `evo2_flash/`.  Tensors are
CPU torch tensors; bf16 values are carried as fp32 holding bf16-representable
numbers where the reference rounds, via `bf`.

State views follow the reference's normalised, dim-first orientation:
conv_state (blocks, 3H, 2) bf16, inner FIR state (blocks, H, K-1) fp32,
LI state (blocks, H, 16) fp32 (mixers.py:892-917, 940-949).
"""

import torch
import torch.nn.functional as F

__all__ = [
    "bf", "depthwise_prefill", "hcl_compute_filter", "iir_segment",
    "fir_mixer_prefill", "iir_mixer_prefill", "fir_decode_one", "iir_decode_one",
    "short_conv_update", "hyena_decode_emulated", "mixer_decode_unfused",
    "rms_norm", "quantize_input", "fp8_linear_dequant", "prefill_tables",
    "fir_decode_snapshots", "iir_decode_snapshots", "fir_verify_emulated",
    "iir_verify_emulated", "STATE_ACC_BUDGET", "fast_accum_mm", "fp8_linear_fast_accum",
    "causal_conv1d_update_ref", "causal_conv1d_ref", "iir_final_state_recurrence",
    "causal_conv1d_update_spec_ref", "mixer_decode_speculative",
    "spec_accepted_ref", "record_stamps_ref", "verify_plan_ref", "repair_prefill_ref",
]

# mixers.py:72-74: bound on the (H, blk, L) temporary of the LI final state.
STATE_ACC_BUDGET = 64 << 20


def bf(x):
    """Round fp32 to bf16 and back: the value a bf16 torch tensor holds."""
    return x.to(torch.bfloat16).to(torch.float32)


# ------------------------------------------------------------------ prefill
def depthwise_prefill(x_p, w, qsl, slots, has_init, state, k):
    """Per-segment depthwise causal conv over packed rows, carrying state.

    Follows `_depthwise_prefill_torch` (mixers.py:350-383), which is also the
    reference's torch form of the short filter's `causal_conv1d_fn`
    (`_short_fir_torch`, mixers.py:1210-1212).  `w` (dim, k) is in
    cross-correlation order: w[:, -1] multiplies the current sample.  The left
    context is the cached window (has_init) or zeros; the window written back
    is always the last k-1 inputs of cat(prev, seq), even for a segment
    shorter than k-1 (mixers.py:380-382).  Empty segments touch nothing.

    x_p: (T, dim); qsl: n+1 segment starts; slots: n state blocks;
    has_init: n flags; state: (blocks, dim, >=k-1) view, updated in place.
    Returns (T, dim) in x_p's dtype.
    """
    dim = x_p.shape[1]
    out = torch.empty_like(x_p)
    wt = w.float().unsqueeze(1)  # (dim, 1, k)
    for j in range(len(qsl) - 1):
        a, b = int(qsl[j]), int(qsl[j + 1])
        if b <= a:
            continue
        idx = int(slots[j])
        seq = x_p[a:b].transpose(0, 1).float()
        if has_init[j]:
            prev = state[idx, :, : k - 1].float()
        else:
            prev = torch.zeros(dim, k - 1, dtype=torch.float32)
        seq_in = torch.cat([prev, seq], dim=-1)
        y = F.conv1d(seq_in.unsqueeze(0), wt, padding=0, groups=dim)
        out[a:b] = y[0].transpose(0, 1).to(out.dtype)
        state[idx, :, : k - 1] = seq_in[..., -(k - 1):].to(state.dtype)
    return out


def hcl_compute_filter(residues, log_poles, t):
    """h[d, l] = sum_s residues[d, s] * exp(log_poles[d, s] * t[l]), fp32.

    The torch form `_compute_filter_torch` (triton_hcl.py:77-85): accumulate
    over state channels, never materialising (D, S, L).
    """
    D, S = residues.shape
    h = torch.zeros(D, t.shape[0], dtype=torch.float32)
    for s in range(S):
        h += residues[:, s:s + 1].float() * torch.exp(log_poles[:, s:s + 1].float() * t.float())
    return h


def iir_segment(seq, res, lp, s_prev):
    """One prefill segment of s_t = p*s_{t-1} + x_t (mixers.py:144-210).

    seq (H, L) fp32, res/lp (H, S), s_prev (H, S) or None.  Returns
    (y (H, L), s_last (H, S)).  y is the causal convolution with the modal
    filter, evaluated by FFT of length 2L (mixers.py:197-202); the final state
    is the closed form sum_t x_t p^(L-1-t), blocked over state channels to
    the reference's byte budget (mixers.py:181-195).  A continuation adds
    p^L s_prev to the state and sum_s res_s s_prev,s p_s^(t+1) to y
    (mixers.py:204-209).
    """
    H, L = seq.shape
    S = res.shape[1]
    t = torch.arange(L, dtype=torch.float32)
    h = hcl_compute_filter(res, lp, t)
    lag = t.flip(0)
    blk = min(S, max(1, int(STATE_ACC_BUDGET // max(H * L * 4, 1))))
    st = torch.empty(H, S, dtype=torch.float32)
    for s0 in range(0, S, blk):
        sl = slice(s0, min(s0 + blk, S))
        st[:, sl] = (seq.unsqueeze(1) * torch.exp(lp[:, sl].unsqueeze(-1) * lag)).sum(-1)
    n = 2 * L
    y = torch.fft.irfft(
        torch.fft.rfft(seq, n=n) * (torch.fft.rfft(h, n=n) / n), n=n, norm="forward"
    )[..., :L]
    if s_prev is not None:
        st = st + torch.exp(lp * L) * s_prev
        y = y + hcl_compute_filter(res * s_prev, lp, t + 1.0)
    return y, st


def _split(zf):
    """(x2, x1, v) from the interleaved projection (mixers.py:1206-1208)."""
    return zf[:, 0::3], zf[:, 1::3], zf[:, 2::3]


def fir_mixer_prefill(z_p, short_w, conv_state, w_inner, inner_state, D, qsl, slots,
                      has_init):
    """Prefill rows of HyenaFIRMixer between in_proj and out_proj.

    mixers.py:1277-1305 with the torch short filter (mixers.py:1121-1212) and
    the torch inner FIR (mixers.py:350-383): bf16 z -> short conv (bf16) ->
    u = x1*v (bf16) -> FIR (bf16) -> [+ D*u] -> g = x2*y, all bf16 ops.
    inner_state: (blocks, H, >= K-1) fp32 view.  Returns g (T, H) bf16.
    """
    k_short = short_w.shape[1]
    zf = depthwise_prefill(z_p, short_w, qsl, slots, has_init, conv_state, k_short)
    x2, x1, v = _split(zf)
    u = x1 * v
    K = w_inner.shape[1]
    y = depthwise_prefill(u, w_inner, qsl, slots, has_init, inner_state, K)
    if D is not None:
        y = y + D.to(y.dtype) * u
    return x2 * y


def iir_mixer_prefill(z_p, short_w, conv_state, res, lp, ssm, D, qsl, slots, has_init):
    """Prefill rows of HyenaIIRMixer between in_proj and out_proj.

    mixers.py:1327-1401: short conv, x1v = x1*v (bf16), per segment
    `iir_segment` on x1v as fp32 -> y (bf16), ssm[slot] <- final state, then
    g = (y + x1v*D) * x2 in bf16.  res, lp: (H, 16) fp32.  Returns g (T, H) bf16.
    """
    k_short = short_w.shape[1]
    zf = depthwise_prefill(z_p, short_w, qsl, slots, has_init, conv_state, k_short)
    x2, x1, v = _split(zf)
    x1v = x1 * v
    y = torch.empty_like(x1v)
    for j in range(len(qsl) - 1):
        a, b = int(qsl[j]), int(qsl[j + 1])
        if b <= a:
            continue
        seq = x1v[a:b].float().transpose(0, 1)
        idx = int(slots[j])
        s_prev = ssm[idx].float() if has_init[j] else None
        conv, st = iir_segment(seq, res, lp, s_prev)
        y[a:b] = conv.transpose(0, 1).to(y.dtype)
        ssm[idx] = st
    return (y + x1v * D.to(y.dtype)) * x2


# ------------------------------------------------------------------ decode
def fir_decode_one(x, weight, indices, state):
    """Unfused torch FIR decode (mixers.py:555-565), fp32 sums in torch's order."""
    st = state[indices].float()
    wf = weight.float()
    y = (st * wf[None, :, :-1]).sum(-1) + wf[None, :, -1] * x.float()
    state[indices] = torch.cat([st[..., 1:], x.float().unsqueeze(-1)], dim=-1).to(state.dtype)
    return y.to(x.dtype)


def iir_decode_one(x, poles, residues, indices, state):
    """Unfused torch LI decode (mixers.py:568-575)."""
    st = state[indices] * poles[None] + x[..., None]
    state[indices] = st
    return (residues[None] * st).sum(-1).to(x.dtype)


def short_conv_update(z, short_w, conv_state, slots):
    """The K=3 conv update as the fused decode rounds it (triton_decode.py:44-53).

    Per channel: bf16(((0 + bf16(c0 w0)) + bf16(c1 w1)) + bf16(x w2)), then
    window (c0, c1) <- (c1, x).  conv_state (blocks, 3H, 2) is updated in
    place for each row's slot.  Returns (B, 3H) fp32 holding bf16 values.
    """
    B, C = z.shape
    w = short_w.float()
    out = torch.empty(B, C, dtype=torch.float32)
    for b in range(B):
        blk = int(slots[b])
        c = conv_state[blk].float()
        x = z[b].float()
        acc = (0.0 + bf(c[:, 0] * w[:, 0])) + bf(c[:, 1] * w[:, 1])
        acc = acc + bf(x * w[:, 2])
        out[b] = bf(acc)
        conv_state[blk, :, 0] = conv_state[blk, :, 1]
        conv_state[blk, :, 1] = z[b].to(conv_state.dtype)
    return out


def _silu(acc):
    return acc / (1.0 + torch.exp(-acc))


def causal_conv1d_update_ref(x, conv_state, w, bias=None, activation=None, slots=None,
                             pad_slot_id=-1):
    """vLLM's causal_conv1d_update as the mixers call it (mixers.py:1194-1204),
    with the rounding the reference states for it (triton_decode.py:10-11):
    acc = bias (or 0), then + bf16(s_k w_k) over the window oldest first and
    + bf16(x w_{K-1}); optional SiLU; bf16 out.  The slot's window shifts in
    x.  A row whose slot is pad_slot_id (or outside the pool) outputs zeros
    and touches no state.  x (B, dim); w (dim, K); conv_state (blocks, dim,
    >=K-1) updated in place.  Returns (B, dim) fp32 holding bf16 values.
    """
    B, dim = x.shape
    K = w.shape[1]
    wf = w.float()
    b0 = bias.float() if bias is not None else torch.zeros(dim)
    out = torch.zeros(B, dim, dtype=torch.float32)
    for b in range(B):
        blk = int(slots[b]) if slots is not None else b
        if blk == pad_slot_id or not 0 <= blk < conv_state.shape[0]:
            continue
        s = conv_state[blk, :, : K - 1].float()
        xb = x[b].float()
        acc = b0.clone()
        for k in range(K - 1):
            acc = acc + bf(s[:, k] * wf[:, k])
        acc = acc + bf(xb * wf[:, K - 1])
        if activation:
            acc = _silu(acc)
        out[b] = bf(acc)
        new = torch.cat([s[:, 1:], xb.unsqueeze(1)], dim=1)
        conv_state[blk, :, : K - 1] = new.to(conv_state.dtype)
    return out


def causal_conv1d_update_spec_ref(x, conv_state, w, slots, accepted, qsl, max_query_len,
                                  in_col=None, out_col=None, pad_slot_id=-1):
    """vLLM's causal_conv1d_update in its speculative varlen form, as the
    mixers call it for a verify step (mixers.py:1176-1193), with the window
    convention mixers.py:222-240 states: before the step the window holds
    [h_1 .. h_M]; the step leaves [h_2 .. h_M, d_1 .. d_q]; after a later
    step accepts a of the q rows its live window starts at column a - 1.

    Request r owns rows qsl[r]..qsl[r+1]-1 of x (T, dim); its input block is
    slots[r, in_col[r]] and its output block slots[r, out_col[r]] (column 0
    when None).  The live (K-1)-window starts at column accepted[r] - 1; the
    output block's columns become [old cols accepted[r] .. accepted[r]+keep-1,
    the q inputs], keep = state_len - max_query_len, later columns unchanged.
    Rounding as `causal_conv1d_update_ref`.  Padding or out-of-range slots,
    q > max_query_len or accepted outside [1, max_query_len]: zero rows, no
    state.  conv_state (blocks, dim, state_len) updated in place.  Returns
    (T, dim) fp32 holding bf16 values, zero on rows no request covers.

    Parity unpinned against vLLM itself (its kernel is not in the reference);
    pinned by the special case q = accepted = 1, max_query_len = 1, which is
    `causal_conv1d_update_ref`, and by the rollback invariant the convention
    exists for (tests/test_oracle.py).
    """
    T, dim = x.shape
    K = w.shape[1]
    wf = w.float()
    state_len = conv_state.shape[2]
    keep = state_len - max_query_len
    out = torch.zeros(T, dim, dtype=torch.float32)
    for r in range(len(qsl) - 1):
        a, e = int(qsl[r]), int(qsl[r + 1])
        if e <= a:
            continue
        q = e - a
        ic = 0 if in_col is None else int(in_col[r])
        oc = 0 if out_col is None else int(out_col[r])
        src, dst, acc_n = int(slots[r, ic]), int(slots[r, oc]), int(accepted[r])
        nb = conv_state.shape[0]
        if (q > max_query_len or not 1 <= acc_n <= max_query_len
                or src == pad_slot_id or dst == pad_slot_id
                or not (0 <= src < nb and 0 <= dst < nb)):
            continue
        off = acc_n - 1
        old = conv_state[src].float().clone()             # (dim, state_len)
        s = old[:, off:off + K - 1].clone()
        for t in range(a, e):
            xt = x[t].float()
            acc = torch.zeros(dim)
            for k in range(K - 1):
                acc = acc + bf(s[:, k] * wf[:, k])
            acc = acc + bf(xt * wf[:, K - 1])
            out[t] = bf(acc)
            s = torch.cat([s[:, 1:], xt[:, None]], dim=1)
        new = conv_state[dst].float().clone()
        new[:, :keep] = old[:, off + 1:off + 1 + keep]
        new[:, keep:keep + q] = x[a:e].float().t()
        conv_state[dst] = new.to(conv_state.dtype)
    return out


def causal_conv1d_ref(x_p, w, bias, activation, qsl, slots, has_init, state, pad_slot_id=-1):
    """vLLM's causal_conv1d_fn over packed prefill segments as the mixers call
    it (mixers.py:1138-1150), with the update kernel's rounding (see
    `causal_conv1d_update_ref`): each output sums bf16-rounded products of its
    K inputs, oldest first, from the bias.  Segment j is rows qsl[j]..qsl[j+1]
    of x_p (T, dim); its left context is its slot's window when has_init[j]
    (zeros otherwise), and the window becomes the last K-1 inputs of
    cat(window or zeros, segment).  Empty segments and padding slots touch no
    state; rows outside every segment output zeros; state None skips every
    window.  Returns (T, dim) fp32 holding bf16 values.
    """
    T, dim = x_p.shape
    K = w.shape[1]
    wf = w.float()
    b0 = bias.float() if bias is not None else torch.zeros(dim)
    out = torch.zeros(T, dim, dtype=torch.float32)
    for j in range(len(qsl) - 1):
        a, e = int(qsl[j]), int(qsl[j + 1])
        if e <= a:
            continue
        blk = int(slots[j]) if slots is not None else j
        valid = state is not None and blk != pad_slot_id and 0 <= blk < state.shape[0]
        if valid and has_init is not None and bool(has_init[j]):
            prev = state[blk, :, : K - 1].float()
        else:
            prev = torch.zeros(dim, K - 1, dtype=torch.float32)
        seq = torch.cat([prev, x_p[a:e].transpose(0, 1).float()], dim=1)  # (dim, K-1+n)
        n = e - a
        acc = b0.unsqueeze(1).expand(dim, n).clone()
        for k in range(K):
            acc = acc + bf(seq[:, k:k + n] * wf[:, k:k + 1])
        if activation:
            acc = _silu(acc)
        out[a:e] = bf(acc).transpose(0, 1)
        if valid:
            state[blk, :, : K - 1] = seq[:, -(K - 1):].to(state.dtype)
    return out


def iir_final_state_recurrence(seq, lp):
    """Final state of s_t = exp(lp) * s_{t-1} + x_t from zero, in float64
    (the recurrence form of triton_prefill.py:351-387's closed form
    sum_t x_t p^(L-1-t)).  seq (H, L), lp (H, S).  Returns (H, S) float64."""
    p = torch.exp(lp.double())
    s = torch.zeros(lp.shape, dtype=torch.float64)
    x = seq.double()
    for t in range(x.shape[1]):
        s = p * s + x[:, t:t + 1]
    return s


def _hcm_sum(s, wf, u):
    """K=128 readout in the fused kernel's order (triton_decode.py:97-123)."""
    H = s.shape[0]
    acc = [[torch.zeros(H) for _ in range(4)] for _ in range(4)]
    for j in range(8):
        for m in range(4):
            for l in range(4):
                k = 16 * j + 4 * m + l
                if k < 127:
                    acc[m][l] = acc[m][l] + s[:, k] * wf[:, k]
                else:
                    acc[m][l] = acc[m][l] + 0.0
    p = [((acc[0][l] + acc[1][l]) + acc[2][l]) + acc[3][l] for l in range(4)]
    return bf(((p[0] + p[2]) + (p[1] + p[3])) + wf[:, 127] * u)


def _hcs_sum(s, wf, u):
    """K=7 readout in the fused kernel's order (triton_decode.py:125-143)."""
    a = (s[:, 0] * wf[:, 0] + 0.0) + s[:, 4] * wf[:, 4]
    b = (s[:, 1] * wf[:, 1] + 0.0) + s[:, 5] * wf[:, 5]
    c = s[:, 2] * wf[:, 2] + 0.0
    d = s[:, 3] * wf[:, 3] + 0.0
    return bf((((a + b) + c) + d) + wf[:, 6] * u)


def hyena_decode_emulated(z, short_w, conv_state, slots, inner, inner_state, D=None,
                          log_poles=None, null_block=0, poles=None):
    """The fused q=1 decode step with the reference kernel's rounding points.

    triton_decode.py:57-164 restated op by op in fp32 torch (no FMA on the
    CPU): rows whose slot is the null block output 0 and write no state; all
    three state slices are updated in place.  `poles` overrides exp(log_poles)
    so a caller can feed the exact fp32 poles a device computed.
    Returns (B, H) bf16.
    """
    B = z.shape[0]
    H = inner.shape[0]
    out = torch.zeros(B, H, dtype=torch.bfloat16)
    iir = log_poles is not None
    if iir and poles is None:
        poles = torch.exp(log_poles.float())
    for b in range(B):
        blk = int(slots[b])
        if blk == null_block:
            continue
        y3 = short_conv_update(z[b:b + 1], short_w, conv_state, [blk])[0].view(H, 3)
        x2, x1, v = y3[:, 0], y3[:, 1], y3[:, 2]
        u = bf(x1 * v)
        if iir:
            s = inner_state[blk].float() * poles + u[:, None]
            r = s * inner.float()
            r = r[:, :8] + r[:, 8:]
            r = r[:, :4] + r[:, 4:]
            r = r[:, :2] + r[:, 2:]
            y = bf((r[:, 0] + r[:, 1]) + 0.0)
            inner_state[blk] = s
        else:
            K = inner.shape[1]
            s = inner_state[blk, :, : K - 1].float()
            wf = inner.float()
            y = _hcm_sum(s, wf, u) if K == 128 else _hcs_sum(s, wf, u)
            inner_state[blk, :, : K - 1] = torch.cat([s[:, 1:], u[:, None]], dim=1)
        if D is not None:
            y = bf(y + bf(D.float() * u))
        out[b] = (x2 * y).to(torch.bfloat16)
    return out


def mixer_decode_unfused(z, short_w, conv_state, slots, inner, inner_state, D=None,
                         log_poles=None):
    """The reference's unfused decode (fp32 torch sums), for tolerance checks.

    FIR: mixers.py:1285-1305 with `_fir_decode_one`; LI: mixers.py:1355-1397
    with `_iir_decode_one`.  The short filter uses the fused rounding
    (`short_conv_update`), which is what vLLM's update kernel computes.
    """
    H = inner.shape[0]
    zf = bf(short_conv_update(z, short_w, conv_state, slots)).to(torch.bfloat16)
    x2, x1, v = _split(zf)
    u = x1 * v
    idx = torch.as_tensor([int(s) for s in slots], dtype=torch.long)
    if log_poles is not None:
        y = iir_decode_one(u.float(), torch.exp(log_poles.float()), inner.float(), idx,
                           inner_state).to(torch.bfloat16)
        y = (y + u * D.to(y.dtype)) * x2
        return y
    K = inner.shape[1]
    y = fir_decode_one(u, inner, idx, inner_state[..., : K - 1])
    if D is not None:
        y = y + D.to(y.dtype) * u
    return x2 * y


def mixer_decode_speculative(z, short_w, conv_state, inner, inner_state, D, slots, qsl,
                             accepted, max_query_len, poles=None, ins=None, outs=None,
                             in_col=None, out_col=None, emulate_kernels=True):
    """Decode rows of a speculative step between in_proj and out_proj
    (mixers.py:1277-1305 for the FIR, 1327-1401 for the LI, speculative
    branches): the widened short window (`causal_conv1d_update_spec_ref`),
    u = x1*v, the inner operator with one snapshot per verifier position
    (`fir_verify_emulated` / `iir_verify_emulated`, or with
    emulate_kernels=False the reference's torch paths
    `fir_decode_snapshots` / `iir_decode_snapshots`), then [+ D*u] and * x2
    in bf16.  `poles` (H, 16) selects the LI operator with `inner` the
    residues; else `inner` is the FIR taps (H, K).  Snapshot slots default to
    the slot matrix (ins = outs = slots).  States are updated in place.
    Returns g (T, H) bf16, zero on rows no request covers.
    """
    T = z.shape[0]
    zf = causal_conv1d_update_spec_ref(z, conv_state, short_w, slots, accepted, qsl,
                                       max_query_len, in_col, out_col).to(torch.bfloat16)
    x2, x1, v = _split(zf)
    u = x1 * v
    n = len(qsl) - 1
    starts = torch.as_tensor([int(qsl[r]) for r in range(n)], dtype=torch.long)
    ends = torch.as_tensor([int(qsl[r + 1]) for r in range(n)], dtype=torch.long)
    ins = slots if ins is None else ins
    outs = slots if outs is None else outs
    acc = torch.as_tensor([int(a) for a in accepted], dtype=torch.long)
    if poles is not None:
        fn = iir_verify_emulated if emulate_kernels else iir_decode_snapshots
        y = fn(u, poles.float(), inner.float(), inner_state, ins, outs, starts, ends, acc)
        return (y + u * D.to(y.dtype)) * x2
    K = inner.shape[1]
    fn = fir_verify_emulated if emulate_kernels else fir_decode_snapshots
    y = fn(u, inner, inner_state[..., : K - 1], ins, outs, starts, ends, acc)
    if D is not None:
        y = y + D.to(y.dtype) * u
    g = x2 * y
    covered = torch.zeros(T, dtype=torch.bool)
    for r in range(n):
        covered[int(qsl[r]):int(qsl[r + 1])] = True
    g[~covered] = 0
    return g


# ------------------------------------------------------------ position stamps
def spec_accepted_ref(stamps, slots, computed, num_spec, counts=None):
    """(accepted, faults) of a speculative decode step from the position
    stamps (mixers.py:960-999): request r on slot row slots[r] (a list; the
    first entry names its live-snapshot column 0 block) that has computed n
    tokens finds offset = n - stamps[slots[r][0]]; accepted = clamp(offset,
    0, num_spec) + 1.  A request not on the null block (0) whose offset lies
    outside [0, num_spec] -- or, with `counts`, whose count differs from
    offset + 1 -- is a fault (the reference asserts; here it is counted).
    `slots` None puts every request on the null block (mixers.py:527-541).
    A slot outside the pool is a fault and reads no stamp."""
    acc, faults = [], 0
    nb = len(stamps)
    for r in range(len(computed)):
        first = 0 if slots is None else int(slots[r][0])
        inside = 0 <= first < nb
        stamp = int(float(stamps[first])) if inside else 0
        off = int(computed[r]) - stamp
        bad = (not inside) or (first != 0 and (off < 0 or off > num_spec))
        if counts is not None and inside and first != 0 and int(counts[r]) != off + 1:
            bad = True
        faults += int(bad)
        acc.append(min(max(off, 0), num_spec) + 1)
    return acc, faults


def record_stamps_ref(stamps, slots, qsl, computed, width, out_col=None, prefill_blocks=(),
                      seq_lens=()):
    """Stamps after a step (mixers.py:1049-1074), as a new list: decode
    request r (query length qsl[r+1] - qsl[r], computed n tokens) stamps
    block slots[r][out_col[r] + p] with n + p + 1 for p < min(width, query
    length); prefill block j gets seq_lens[j].  The null block (0), slots
    outside the pool and columns past the slot row are left alone (the
    reference also writes the null block, whose stamp nothing reads).
    `slots` None writes no decode stamp (all requests on the null block)."""
    out = [float(v) for v in stamps]
    nb = len(out)

    def put(block, value):
        if 0 < block < nb:
            out[block] = float(value)

    if slots is not None:
        for r in range(len(qsl) - 1):
            qlen = int(qsl[r + 1]) - int(qsl[r])
            for p in range(min(width, qlen)):
                col = (0 if out_col is None else int(out_col[r])) + p
                if 0 <= col < len(slots[r]):
                    put(int(slots[r][col]), int(computed[r]) + p + 1)
    for b, n in zip(prefill_blocks, seq_lens):
        put(int(b), int(n))
    return out


def verify_plan_ref(slots, nreq, width, qsl=None, prev=None, sched=None, eng_acc=None,
                    null_all=False):
    """(ins, outs, starts, ends, acc) of a step's speculative decode requests
    as lists, following the reference's _decode_tensors and its helpers
    (mixers.py:431-541).  slots: rows of block ids.  Without both block
    pointers ins = outs = the slot row; with them, width columns from
    prev[r] and sched[r] (the reference's gather; a column outside the row
    is the null block here, where torch's gather would raise).  The packed
    rows are qsl[r] .. qsl[r+1], or r .. r+1 without qsl; acc =
    max(eng_acc[r], 1), or 1 without counts.  null_all: the profiling-pool
    rule, every block the null block (mixers.py:527-541)."""
    def window(r, base):
        row = slots[r]
        out = []
        for p in range(width):
            c = base + p
            out.append(0 if null_all or c < 0 or c >= len(row) else int(row[c]))
        return out
    paged = prev is not None and sched is not None
    ins = [window(r, int(prev[r]) if paged else 0) for r in range(nreq)]
    outs = [window(r, int(sched[r]) if paged else 0) for r in range(nreq)]
    starts = [int(qsl[r]) if qsl is not None else r for r in range(nreq)]
    ends = [int(qsl[r + 1]) if qsl is not None else r + 1 for r in range(nreq)]
    acc = [max(int(eng_acc[r]), 1) if eng_acc is not None else 1 for r in range(nreq)]
    return ins, outs, starts, ends, acc


def repair_prefill_ref(slices, stamps, dst, src, need, has_init):
    """Align-mode repair of resumed prefill states (mixers.py:1001-1037), on
    copies: row j (has_init) whose block dst[j] is not stamped need[j] while
    src[j] is takes src[j]'s contents in every slice; both blocks must be off
    the null block.  All sources are read before any destination is written
    (the reference's gather-then-scatter).  Returns (new slices, repaired
    rows).  `stamps` lists each block's stamp."""
    take = []
    for j in range(len(dst)):
        d, s_ = int(dst[j]), int(src[j])
        bad = (bool(has_init[j]) and d != 0 and s_ != 0 and float(stamps[d]) != float(need[j])
               and float(stamps[s_]) == float(need[j]))
        take.append(s_ if bad else d)
    out = [t.clone() for t in slices]
    for t_new, t_old in zip(out, slices):
        gathered = [t_old[b].clone() for b in take]
        for j, d in enumerate(dst):
            t_new[int(d)] = gathered[j]
    return out, [j for j in range(len(dst)) if take[j] != int(dst[j])]


# ------------------------------------------------------------ speculative verify
def _verify_rows(ins, outs, starts, ends, accepted, r):
    """(source block, first row, end row, destinations) of request r."""
    src = int(ins[r, int(accepted[r]) - 1])
    return src, int(starts[r]), int(ends[r]), [int(d) for d in outs[r]]


def fir_decode_snapshots(x, weight, state, ins, outs, starts, ends, accepted):
    """The reference's torch verify path for the FIR (mixers.py:578-624):
    each request starts from the snapshot ins[r, accepted-1], runs its tokens
    [starts[r], ends[r]) and writes the window after token pos to outs[r, pos]
    (block 0 is the null block: never written, as the fused kernel skips it).
    fp32 torch sums; returns (T, H) in x's dtype, zero outside every range.
    state: (blocks, H, K-1) fp32, modified in place."""
    K = weight.shape[1]
    wf = weight.float()
    y = torch.zeros(x.shape, dtype=torch.float32)
    for r in range(ins.shape[0]):
        src, a, e, dst = _verify_rows(ins, outs, starts, ends, accepted, r)
        st = state[src, :, : K - 1].float().clone()
        for pos in range(outs.shape[1]):
            if a + pos >= e:
                break
            xt = x[a + pos].float()
            y[a + pos] = (st * wf[:, :-1]).sum(-1) + wf[:, -1] * xt
            st = torch.cat([st[:, 1:], xt[:, None]], dim=1)
            if dst[pos] != 0:
                state[dst[pos], :, : K - 1] = st
    return y.to(x.dtype)


def iir_decode_snapshots(x, poles, residues, state, ins, outs, starts, ends, accepted):
    """The reference's torch verify path for the LI operator (mixers.py:627-658),
    with the same snapshot and null-block rules as `fir_decode_snapshots`."""
    y = torch.zeros(x.shape, dtype=torch.float32)
    for r in range(ins.shape[0]):
        src, a, e, dst = _verify_rows(ins, outs, starts, ends, accepted, r)
        st = state[src, :, :16].float().clone()
        for pos in range(outs.shape[1]):
            if a + pos >= e:
                break
            st = st * poles + x[a + pos].float()[:, None]
            if dst[pos] != 0:
                state[dst[pos], :, :16] = st
            y[a + pos] = (residues * st).sum(-1)
    return y.to(x.dtype)


def _fir_dot_kernel_order(s, wf):
    """sum_k s_k w_k, k < K-1, in the verify kernel's order
    (triton_verifier.py:17-43): for K=128 sixteen accumulators (m, l) over
    k = 16 j + 4 m + l, j in order, then ((m0 + m1) + m2) + m3, then
    (l0 + l2) + (l1 + l3); for K=7 ((p0 + p4) + (p1 + p5) + p2) + p3."""
    K = wf.shape[1]
    if K == 7:
        a = s[:, 0] * wf[:, 0] + s[:, 4] * wf[:, 4]
        b = s[:, 1] * wf[:, 1] + s[:, 5] * wf[:, 5]
        return ((a + b) + s[:, 2] * wf[:, 2]) + s[:, 3] * wf[:, 3]
    H = s.shape[0]
    acc = [[torch.zeros(H) for _ in range(4)] for _ in range(4)]
    for j in range(8):
        for m in range(4):
            for l in range(4):
                k = 16 * j + 4 * m + l
                if k < 127:
                    acc[m][l] = acc[m][l] + s[:, k] * wf[:, k]
    p = [((acc[0][l] + acc[1][l]) + acc[2][l]) + acc[3][l] for l in range(4)]
    return (p[0] + p[2]) + (p[1] + p[3])


def fir_verify_emulated(x, weight, state, ins, outs, starts, ends, accepted, null_block=0):
    """`fir_decode_snapshots` with the fused verify kernel's summation order
    (no FMA on the CPU), for bitwise comparison with a GPU kernel that keeps
    that order.  starts=None runs the one-token form (fir_one): row r reads
    and writes ins[r, 0] / outs[r, 0]."""
    K = weight.shape[1]
    wf = weight.float()
    y = torch.zeros(x.shape, dtype=torch.float32)
    one = starts is None
    for r in range(ins.shape[0]):
        if one:
            src, a, e, dst = int(ins[r, 0]), r, r + 1, [int(outs[r, 0])]
        else:
            src, a, e, dst = _verify_rows(ins, outs, starts, ends, accepted, r)
        st = state[src, :, : K - 1].float().clone()
        for pos in range(outs.shape[1]):
            if a + pos >= e:
                break
            xt = x[a + pos].float()
            y[a + pos] = _fir_dot_kernel_order(st, wf) + wf[:, K - 1] * xt
            st = torch.cat([st[:, 1:], xt[:, None]], dim=1)
            if dst[pos] != null_block:
                state[dst[pos], :, : K - 1] = st
    return y.to(x.dtype)


def iir_verify_emulated(x, poles, residues, state, ins, outs, starts, ends, accepted,
                        null_block=0):
    """`iir_decode_snapshots` with the fused kernel's halving-tree readout
    (triton_verifier.py:128-131): r[s] += r[s+8], += r[s+4], += r[s+2],
    += r[s+1], y = r[0]."""
    y = torch.zeros(x.shape, dtype=torch.float32)
    one = starts is None
    for r in range(ins.shape[0]):
        if one:
            src, a, e, dst = int(ins[r, 0]), r, r + 1, [int(outs[r, 0])]
        else:
            src, a, e, dst = _verify_rows(ins, outs, starts, ends, accepted, r)
        st = state[src, :, :16].float().clone()
        for pos in range(outs.shape[1]):
            if a + pos >= e:
                break
            st = st * poles + x[a + pos].float()[:, None]
            if dst[pos] != null_block:
                state[dst[pos], :, :16] = st
            q = st * residues
            q = q[:, :8] + q[:, 8:]
            q = q[:, :4] + q[:, 4:]
            q = q[:, :2] + q[:, 2:]
            y[a + pos] = q[:, 0] + q[:, 1]
    return y.to(x.dtype)


# ------------------------------------------------------------------ norm, fp8
def rms_norm(x, weight, eps, residual=None):
    """Evo2RMSNorm (model.py:47-74) with the rounding points of triton_norm.py:6-11.

    s = bf(x + r); n = bf(sqrt(sum s^2)) (fp32 sum); n = bf(n H^-1/2);
    n = bf(n + eps); y = bf(w * bf(s / n)).  eps sits outside the sqrt.
    Returns y, or (y, s) with a residual.  bf16 in and out.
    """
    H = x.shape[-1]
    s = x.float()
    if residual is not None:
        s = bf(s + residual.float())
    n = bf(torch.sqrt((s.double() * s.double()).sum(-1, keepdim=True)).float())
    n = bf(n * (H ** -0.5))
    n = bf(n + eps)
    y = bf(weight.float() * bf(s / n)).to(torch.bfloat16)
    if residual is None:
        return y
    return y, s.to(torch.bfloat16)


def quantize_input(x, input_scale):
    """Static per-tensor E4M3 activation quantisation (fp8_emul.py:76-78)."""
    return (x.float() / input_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def fp8_linear_dequant(x, w8, input_scale, weight_scale, bias=None):
    """bf16( (e4m3(x/s_in) @ W8^T) * s_in * s_w [+ b] ) in fp32 (convert.py:195-201)."""
    xq = quantize_input(x, input_scale).float()
    acc = xq @ w8.float().t()
    out = acc * float(input_scale) * float(weight_scale)
    if bias is not None:
        out = out + bias.float()
    return out.to(torch.bfloat16)


# ------------------------------------------------------------------ Hopper fp8 model
FAST_ACC_GROUP = 32
FAST_ACC_FRAC_BITS = 13


def _exp_floor(x):
    """floor(log2|x|) from the fp32 exponent field, as int64; -100000 for 0
    (fp8_emul_triton.py:28-33: the field minus 127, so a subnormal reads -127)."""
    bits = x.float().contiguous().view(torch.int32).to(torch.int64)
    e = ((bits >> 23) & 0xFF) - 127
    return torch.where(x == 0, torch.full_like(e, -100000), e)


def _pow2(e):
    """2^e as fp32 with e clamped to [-126, 127] (fp8_emul_triton.py:36-40)."""
    e = e.clamp(-126, 127)
    return ((e + 127) << 23).to(torch.int32).view(torch.float32)


def _trunc_mul(x, scale):
    """trunc(x * scale) as fp32: fp32 product, then round toward zero to an
    integer (the fp32 -> int32 -> fp32 conversion of the reference)."""
    return torch.trunc((x.float() * scale).float())


def fast_accum_mm(a, b_t):
    """Software model of Hopper's fp8 fast-accumulation GEMM, before the scale
    epilogue (fp8_emul.py:1-24, 45-73; the arithmetic of
    fp8_emul_triton.py:46-76).  a (N, K) and b_t (M, K) hold E4M3 values (any
    float dtype); returns the fp32 accumulator (N, M).

    For each group of 32 consecutive k, ascending:
      e   = max( max_k e(a_k) + e(b_k), e(acc) ),  e(x) = floor(log2|x|)
      s   = trunc(acc * 2^(13-e)) * 2^(e-13) + sum_k trunc(a_k b_k * 2^(13-e)) * 2^(e-13)
      acc = s truncated to 13 fraction bits of its own exponent (0 stays 0).
    Every step is exact in fp32 (products of E4M3 values are exact; the
    aligned terms are integers below 2^21 times the ulp)."""
    a = a.float()
    b = b_t.float()
    N, K = a.shape
    M = b.shape[0]
    if K % FAST_ACC_GROUP:
        raise ValueError(f"K={K} is not a multiple of {FAST_ACC_GROUP}")
    F = FAST_ACC_FRAC_BITS
    ea, eb = _exp_floor(a), _exp_floor(b)
    acc = torch.zeros(N, M, dtype=torch.float32)
    for k0 in range(0, K, FAST_ACC_GROUP):
        ks = slice(k0, k0 + FAST_ACC_GROUP)
        e = (ea[:, None, ks] + eb[None, :, ks]).amax(-1)              # (N, M)
        e = torch.maximum(e, _exp_floor(acc))
        ulp, inv = _pow2(e - F), _pow2(F - e)
        s = _trunc_mul(acc, inv) * ulp
        for k in range(k0, k0 + FAST_ACC_GROUP):
            p = a[:, k, None] * b[None, :, k]
            s = s + _trunc_mul(p, inv) * ulp
        es = _exp_floor(s)
        acc = torch.where(s == 0, s, _trunc_mul(s, _pow2(F - es)) * _pow2(es - F))
    return acc


def fp8_linear_fast_accum(x, w_e4m3, input_scale, weight_scale):
    """The reference's emulated static W8A8 linear
    (fp8_emul_triton.py:181-191): x quantised as in `quantize_input`, the
    fast-accumulation GEMM, then (acc * s_in * s_w) cast to x's dtype."""
    xq = quantize_input(x.reshape(-1, x.shape[-1]), input_scale)
    acc = fast_accum_mm(xq, w_e4m3)
    out = (acc * float(input_scale) * float(weight_scale)).to(x.dtype)
    return out.reshape(*x.shape[:-1], w_e4m3.shape[0])


# ------------------------------------------------------------------ tables
def prefill_tables(qsl, has_init, block_t):
    """(seq (n,3) [start, end, has_init], tiles (ntiles,2) [segment, row0]).

    `_prefill_tables` (mixers.py:386-415) on host lists.
    """
    seq, tiles = [], []
    for j in range(len(qsl) - 1):
        a, b = int(qsl[j]), int(qsl[j + 1])
        seq.append((a, b, int(bool(has_init[j]))))
        tiles.extend((j, t) for t in range(a, b, block_t))
    return (torch.tensor(seq, dtype=torch.int32).reshape(-1, 3),
            torch.tensor(tiles, dtype=torch.int32).reshape(-1, 2))
