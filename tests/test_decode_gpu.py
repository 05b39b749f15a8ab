"""GPU parity of the fused decode step (evo2_hyena_decode) against the oracle.

* bitwise: output and the whole state pool (every byte, so untouched blocks,
  the null block and page padding are covered) against the CPU emulation of
  the reference kernel's rounding points (triton_decode.py:57-164); the LI
  state is compared within fp32 rounding because exp() comes from different
  math libraries on the two sides;
* tolerance: output within 1e-2 max relative error of the reference's
  unfused fp32 torch path (mixers.py:555-575);
* slot mapping: null rows give zeros and write nothing; permuting rows and
  their slots permutes the outputs exactly.
"""

import pytest
import torch

import oracle
from evo2_flash_amd.decode import decode_supported, hyena_decode

from _cases import bf16_ulp_diff, clone_pool, decode_case, max_rel_err

pytestmark = pytest.mark.gpu

KINDS = ["hcs", "hcm", "hcl"]


def _args(kind, prm, pool, H):
    if kind == "hcl":
        inner = prm["residues"]
        lp = prm["log_poles"][..., 0]
        state = pool.ssm_view()
    else:
        K = prm["conv"].shape[-1]
        inner = prm["conv"].view(H, K)
        lp = None
        state = pool.inner_view(K - 1)
    D = prm.get("D")
    return inner, lp, state, D


def _run_gpu(kind, prm, z, slots, pool, H):
    dev = "cuda"
    gp = clone_pool(pool, dev)
    inner, lp, state_c, D = _args(kind, prm, pool, H)
    _, _, state_g, _ = _args(kind, prm, gp, H)
    args = (z.to(dev), prm["short_filter"].view(3 * H, 3).to(dev), gp.conv_view(),
            slots.to(dev), inner.to(dev), state_g,
            None if D is None else D.to(dev), None if lp is None else lp.to(dev))
    assert decode_supported(args[0], args[1], args[2], args[4], args[5], args[6], args[7])
    out = hyena_decode(*args[:6], D=args[6], log_poles=args[7])
    torch.cuda.synchronize()
    return out.cpu(), gp


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("H,B,nblk,n_null", [(256, 5, 9, 1), (4096, 64, 80, 3), (8192, 32, 40, 2),
                                             (1920, 24, 30, 2), (200, 7, 12, 1)])
def test_decode_bitwise_vs_emulation(kind, H, B, nblk, n_null):
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=11 + H, n_null=n_null)
    print(f"decode bitwise kind={kind} H={H} B={B}", flush=True)
    out_g, gp = _run_gpu(kind, prm, z, slots, pool, H)
    inner, lp, state, D = _args(kind, prm, pool, H)
    poles = None
    if lp is not None:
        poles = torch.exp(lp.cuda()).cpu()
    out_c = oracle.hyena_decode_emulated(z, prm["short_filter"].view(3 * H, 3),
                                         pool.conv_view(), slots, inner, state, D, lp,
                                         poles=poles)
    null_rows = slots == 0
    assert (out_g[null_rows].float() == 0).all()
    if kind == "hcl":
        assert bf16_ulp_diff(out_g, out_c).max().item() <= 1
        # slices 0 and 1 bitwise; the LI slice within fp32 rounding of exp
        assert torch.equal(gp.kv_cache[0].cpu(), pool.kv_cache[0])
        assert torch.equal(gp.kv_cache[1].cpu(), pool.kv_cache[1])
        torch.testing.assert_close(gp.kv_cache[2].cpu(), pool.kv_cache[2], rtol=2e-6, atol=1e-5)
    else:
        assert torch.equal(out_g.view(torch.int16), out_c.view(torch.int16))
        assert torch.equal(gp.raw.cpu(), pool.raw)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("H,B", [(4096, 64), (1920, 13)])
def test_decode_vs_unfused_fp32(kind, H, B):
    nblk = B + 6
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=5)
    out_g, _ = _run_gpu(kind, prm, z, slots, pool, H)
    inner, lp, state, D = _args(kind, prm, pool, H)
    ref = oracle.mixer_decode_unfused(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(),
                                      slots, inner, pool.ssm_view() if lp is not None
                                      else pool.inner_view(), D, lp)
    assert max_rel_err(out_g, ref) <= 1e-2


@pytest.mark.parametrize("kind", KINDS)
def test_decode_multi_step_and_permutation(kind):
    H, B, nblk = 512, 16, 40
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=21)
    dev = "cuda"
    gp = clone_pool(pool, dev)
    gp2 = clone_pool(pool, dev)
    inner, lp, _, D = _args(kind, prm, gp, H)
    _, _, st1, _ = _args(kind, prm, gp, H)
    _, _, st2, _ = _args(kind, prm, gp2, H)
    sw = prm["short_filter"].view(3 * H, 3).to(dev)
    inner, D = inner.to(dev), None if D is None else D.to(dev)
    lp = None if lp is None else lp.to(dev)
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(3))
    g = torch.Generator().manual_seed(8)
    for step in range(3):
        zs = (torch.randn(B, 3 * H, generator=g) * 1.3).to(torch.bfloat16).to(dev)
        o1 = hyena_decode(zs, sw, gp.conv_view(), slots.to(dev), inner, st1, D, lp)
        o2 = hyena_decode(zs[perm], sw, gp2.conv_view(), slots[perm].to(dev), inner, st2, D, lp)
        assert torch.equal(o1[perm].view(torch.int16), o2.view(torch.int16)), f"step {step}"
    torch.cuda.synchronize()
    assert torch.equal(gp.raw, gp2.raw)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("H", [1024, 255])
def test_decode_layouts_agree(kind, H):
    """Native pool views with (H, K) taps, channel-contiguous (K, H) taps, and
    dense dim-first state tensors (the generic strided kernel) give identical
    bits; odd H always takes the generic kernel."""
    B, nblk = 12, 20
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=31, n_null=2)
    dev = "cuda"
    sw = prm["short_filter"].view(3 * H, 3).to(dev)
    D = prm.get("D")
    D = None if D is None else D.to(dev)
    outs, states = [], []
    for layout in ("native", "taps_t", "dense"):
        gp = clone_pool(pool, dev)
        inner, lp, st, _ = _args(kind, prm, gp, H)
        inner = inner.to(dev)
        lp = None if lp is None else lp.to(dev)
        conv = gp.conv_view()
        if layout == "taps_t":
            inner = inner.t().contiguous().t()
        if layout == "dense":
            conv = conv.contiguous()
            st = st.contiguous()
        out = hyena_decode(z.to(dev), sw, conv, slots.to(dev), inner, st, D, lp)
        outs.append(out.cpu())
        states.append((conv.cpu().clone(), st.cpu().clone()))
    for o, (c, s) in zip(outs[1:], states[1:]):
        assert torch.equal(outs[0].view(torch.int16), o.view(torch.int16))
        assert torch.equal(states[0][0], c)
        assert torch.equal(states[0][1], s)


def test_decode_empty_batch():
    H = 256
    prm, z, slots, pool = decode_case("hcs", H, 1, 4, seed=1)
    out, _ = _run_gpu("hcs", prm, z[:0], slots[:0], pool, H)
    assert out.shape == (0, H)
