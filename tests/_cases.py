"""Seeded test cases shared by the CPU and GPU tests."""

import torch

from evo2_flash_amd.state import HyenaStatePool
from evo2_flash_amd.synthetic import mixer_params, random_slot_table


def bf16_ulp_diff(a, b):
    """Per-element distance in bf16 units in the last place (same-sign values)."""
    ai = a.contiguous().view(torch.int16).to(torch.int32)
    bi = b.contiguous().view(torch.int16).to(torch.int32)
    # map sign-magnitude to a monotone integer line
    ai = torch.where(ai < 0, -32768 - ai, ai)
    bi = torch.where(bi < 0, -32768 - bi, bi)
    return (ai - bi).abs()


def max_rel_err(out, ref):
    """max|out - ref| / max|ref| in fp32 (the tolerance norm of the mixer tests)."""
    out = out.float()
    ref = ref.float()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def random_pool(num_blocks, H, seed, device="cpu"):
    """A state pool filled with seeded values of the right kind per slice:
    conv windows hold bf16 projections, FIR windows bf16-valued u's in fp32,
    LI states fp32 of magnitude ~10."""
    g = torch.Generator().manual_seed(seed)
    pool = HyenaStatePool(num_blocks, H, "cpu")
    conv = pool.kv_cache[0]
    conv.copy_(torch.randn(conv.shape, generator=g).to(conv.dtype))
    inner = pool.kv_cache[1]
    inner.copy_(torch.randn(inner.shape, generator=g).to(torch.bfloat16).float())
    ssm = pool.kv_cache[2]
    ssm.copy_(torch.randn(ssm.shape, generator=g) * 10.0)
    if device != "cpu":
        gp = HyenaStatePool(num_blocks, H, device)
        gp.raw.copy_(pool.raw)
        return pool, gp
    return pool


def clone_pool(pool, device):
    p = HyenaStatePool(pool.num_blocks, pool.hidden, device)
    p.raw.copy_(pool.raw)
    return p


def decode_case(kind, H, B, num_blocks, seed, n_null=0):
    """CPU tensors for one decode step: params, z, slots (some null rows), pool."""
    prm = mixer_params(kind, H, seed, in_proj_fp8=False)
    g = torch.Generator().manual_seed(seed + 1)
    z = (torch.randn(B, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = random_slot_table(B, num_blocks, seed + 2)
    if n_null:
        rows = torch.randperm(B, generator=g)[:n_null]
        slots[rows] = 0
    pool = random_pool(num_blocks, H, seed + 3)
    return prm, z, slots, pool


def verify_case(kind, H, nreq, Q, num_blocks, seed, x_dtype=torch.bfloat16, n_null_out=2):
    """CPU tensors for one speculative verify step of the inner operator.

    Requests carry 1..Q tokens (ragged, at least one full), start from the
    snapshot of their previous step's accepted count (1..Q) and write one
    snapshot per token.  ins and outs use disjoint blocks (block 0 is the
    null block); `n_null_out` destinations are the null block.
    Returns (params, x, state, (ins, outs, starts, ends, accepted)); state is
    (blocks, H, K-1 | 16) fp32.
    """
    g = torch.Generator().manual_seed(seed)
    prm = mixer_params(kind, H, seed, in_proj_fp8=False)
    lens = torch.randint(1, Q + 1, (nreq,), generator=g)
    lens[0] = Q
    T = int(lens.sum())
    x = (torch.randn(T, H, generator=g) * 1.3).to(x_dtype)
    ends = torch.cumsum(lens, 0)
    starts = ends - lens
    accepted = torch.randint(1, Q + 1, (nreq,), generator=g)
    perm = torch.randperm(num_blocks - 1, generator=g)[: 2 * nreq * Q] + 1
    if perm.numel() < 2 * nreq * Q:
        raise ValueError("state pool too small for disjoint snapshot blocks")
    ins = perm[: nreq * Q].view(nreq, Q).to(torch.int32)
    outs = perm[nreq * Q:].view(nreq, Q).clone().to(torch.int32)
    flat = outs.view(-1)
    flat[torch.randperm(flat.numel(), generator=g)[:n_null_out]] = 0
    if kind == "hcl":
        state = torch.randn(num_blocks, H, 16, generator=g) * 10.0
    else:
        K = prm["conv"].shape[-1]
        state = torch.randn(num_blocks, H, K - 1, generator=g).to(torch.bfloat16).float()
    return prm, x, state, (ins, outs, starts, ends, accepted)


def oracle_mixer_step(kind, prm, hs, pool, dec_slots, pre_lens, pre_slots, pre_init, H, z=None):
    """The oracle's composition of one mixer step (decode rows, then prefill
    segments, then zero padding rows): fp8 in_proj as the dequantised matmul,
    the mixer core, bf16 out_proj with bias."""
    import oracle

    nd, npt = len(dec_slots), sum(pre_lens)
    if z is None:  # else the caller's projection of hs[:nd + npt]
        z = oracle.fp8_linear_dequant(hs[:nd + npt], prm["in_proj.weight"],
                                      prm["in_proj.input_scale"], prm["in_proj.weight_scale"])
    sw = prm["short_filter"].view(3 * H, 3)
    D = prm.get("D")
    qsl = [0]
    for n in pre_lens:
        qsl.append(qsl[-1] + n)
    if kind == "hcl":
        res, lp = prm["residues"], prm["log_poles"][..., 0]
        gd = oracle.hyena_decode_emulated(z[:nd], sw, pool.conv_view(), dec_slots, res,
                                          pool.ssm_view(), D, lp)
        gp = oracle.iir_mixer_prefill(z[nd:], sw, pool.conv_view(), res, lp, pool.ssm_view(), D,
                                      qsl, pre_slots, pre_init)
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        gd = oracle.hyena_decode_emulated(z[:nd], sw, pool.conv_view(), dec_slots, w,
                                          pool.inner_view(K - 1), D)
        gp = oracle.fir_mixer_prefill(z[nd:], sw, pool.conv_view(), w, pool.inner_view(K - 1), D,
                                      qsl, pre_slots, pre_init)
    g = torch.cat([gd, gp]).float()
    out = (g @ prm["out_proj.weight"].float().t() + prm["out_proj.bias"].float()).to(torch.bfloat16)
    full = torch.zeros(hs.shape, dtype=torch.bfloat16)
    full[:nd + npt] = out
    return full
