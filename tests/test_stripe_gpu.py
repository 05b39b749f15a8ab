"""GPU parity of the single-pass hcm / hcl prefill (one tile per segment,
csrc/prefill_stripe.hip) against the oracle.

* fused hcm and hcl mixer cores (mixers.py:1277-1305, 1327-1401) over varlen
  batches with empty, one-row, continued and multi-sub-tile segments, within
  1e-2 max relative error; conv windows bitwise, FIR windows within 1e-2, LI
  final states within 1e-3;
* H a multiple of 16 but not of 64 (a 64-channel block with fewer than four
  16-channel workgroups) and the 1B width H=1920;
* hcm on 32-channel stripes over tiles shorter than their segments (the
  FIR history rebuilt from the 256 rows before a tile);
* chunked prefill: prefill(L) against prefill(a) + continued prefill(L-a);
* decode after a single-pass prefill matches the last row of prefill(L+1);
* the 7B-shaped LI case (H=4096, one 32768-token segment) against a float64
  sequential recurrence of the reference's state update on 4 sampled
  channels, with the short filter and gate on the oracle's rounding path.
"""

import numpy as np
import pytest
import torch

import oracle
from evo2_flash_amd.decode import hyena_decode
from evo2_flash_amd.hcl import hcl_block_t, hyena_hcl_prefill
from evo2_flash_amd.metadata import host_tables
from evo2_flash_amd.prefill import fir_prefill_block_t, hyena_fir_prefill, stripe_block_t
from evo2_flash_amd.synthetic import mixer_params

from _cases import clone_pool, max_rel_err, random_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _whole(lens):
    """block_t of a tile table with one tile per segment."""
    return max(64, (sum(lens) + 63) // 64 * 64)


def _tables(lens, has_init, block_t):
    qsl = [0]
    for n in lens:
        qsl.append(qsl[-1] + n)
    seq, tiles, t0 = host_tables(qsl, has_init, block_t, with_tile_start=True)
    return (qsl, torch.tensor(seq, dtype=torch.int32).view(-1, 3).to(DEV),
            torch.tensor(tiles, dtype=torch.int32).view(-1, 2).to(DEV),
            torch.tensor(t0, dtype=torch.int32).to(DEV))


def _case(kind, H, lens, nblk, seed):
    prm = mixer_params(kind, H, seed, in_proj_fp8=False)
    g = torch.Generator().manual_seed(seed)
    z = (torch.randn(sum(lens), 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = torch.randperm(nblk - 1, generator=g)[:len(lens)].to(torch.int32) + 1
    pool = random_pool(nblk, H, seed=seed + 1)
    return prm, z, slots, pool


def _run(kind, prm, z, slots, gp, lens, has_init, H, bt=None):
    bt = bt or _whole(lens)
    _, seq_t, til_t, t0_t = _tables(lens, has_init, bt)
    sw = prm["short_filter"].view(3 * H, 3).to(DEV)
    if kind == "hcl":
        return hyena_hcl_prefill(z.to(DEV), sw, gp.conv_view(), prm["residues"].to(DEV),
                                 prm["log_poles"][..., 0].to(DEV), gp.ssm_view(),
                                 prm["D"].to(DEV), seq_t, slots.to(DEV), til_t, t0_t, bt)
    K = prm["conv"].shape[-1]
    D = prm.get("D")
    return hyena_fir_prefill(z.to(DEV), sw, gp.conv_view(), prm["conv"].view(H, K).to(DEV),
                             gp.inner_view(K - 1), None if D is None else D.to(DEV), seq_t,
                             slots.to(DEV), til_t, bt)


def _oracle(kind, prm, z, pool, lens, has_init, slots, H):
    qsl = [0]
    for n in lens:
        qsl.append(qsl[-1] + n)
    sw = prm["short_filter"].view(3 * H, 3)
    if kind == "hcl":
        return oracle.iir_mixer_prefill(z, sw, pool.conv_view(), prm["residues"],
                                        prm["log_poles"][..., 0], pool.ssm_view(), prm["D"],
                                        qsl, slots, has_init)
    K = prm["conv"].shape[-1]
    return oracle.fir_mixer_prefill(z, sw, pool.conv_view(), prm["conv"].view(H, K),
                                    pool.inner_view(K - 1), prm.get("D"), qsl, slots, has_init)


CASES = [
    (256, [300, 5, 0, 130, 1, 77], [0, 1, 0, 1, 1, 0]),
    (256, [64, 200], [1, 1]),
    (256, [700, 5, 0, 300, 1, 290], [0, 1, 0, 1, 1, 0]),
    (256, [1100, 130], [1, 0]),
    (320, [5000, 3, 4097, 129, 1, 2048], [0, 1, 1, 0, 1, 1]),
    (208, [513, 40], [1, 1]),
    (1920, [2048], [0]),
    (128, [256, 512, 257, 255], [1, 0, 1, 0]),
]


@pytest.mark.parametrize("kind", ["hcm", "hcl"])
@pytest.mark.parametrize("H,lens,has_init", CASES)
def test_single_pass_vs_oracle(kind, H, lens, has_init):
    nblk = len(lens) + 3
    prm, z, slots, pool = _case(kind, H, lens, nblk, seed=41 + H)
    gp = clone_pool(pool, DEV)
    print(f"single-pass {kind} H={H} lens={lens}", flush=True)
    out = _run(kind, prm, z, slots, gp, lens, has_init, H).cpu()
    ref = _oracle(kind, prm, z, pool, lens, has_init, slots, H)
    assert max_rel_err(out, ref) <= 1e-2
    assert torch.equal(gp.kv_cache[0].cpu(), pool.kv_cache[0])  # conv windows: copies of z
    if kind == "hcl":
        assert torch.equal(gp.kv_cache[1].cpu(), pool.kv_cache[1])  # FIR slice untouched
        for j in range(len(lens)):
            blk = int(slots[j])
            assert max_rel_err(gp.kv_cache[2][blk].cpu(), pool.kv_cache[2][blk]) <= 1e-3, j
    else:
        assert max_rel_err(gp.kv_cache[1].cpu(), pool.kv_cache[1]) <= 1e-2
        assert torch.equal(gp.kv_cache[2].cpu(), pool.kv_cache[2])  # LI slice untouched


@pytest.mark.parametrize("kind", ["hcm", "hcl"])
def test_single_pass_matches_tiled(kind):
    """The single-pass and tiled kernels on the same step agree to rounding."""
    H, lens, has_init = 256, [900, 17, 400], [1, 0, 1]
    prm, z, slots, pool = _case(kind, H, lens, 8, seed=5)
    gp1, gp2 = clone_pool(pool, DEV), clone_pool(pool, DEV)
    a = _run(kind, prm, z, slots, gp1, lens, has_init, H)
    b = _run(kind, prm, z, slots, gp2, lens, has_init, H, bt=256)
    assert max_rel_err(a.cpu(), b.cpu()) <= 1e-2
    assert torch.equal(gp1.kv_cache[0], gp2.kv_cache[0])
    for k in (1, 2):
        assert max_rel_err(gp1.kv_cache[k].cpu(), gp2.kv_cache[k].cpu()) <= 1e-3


@pytest.mark.parametrize("kind", ["hcm", "hcl"])
@pytest.mark.parametrize("split", [1, 200, 256, 513])
def test_single_pass_split(kind, split):
    """prefill(L) == prefill(split) + continued prefill(L - split): outputs
    within 1e-2, conv windows bitwise, FIR windows bitwise (copies of u), LI
    states within 1e-4."""
    H, L, nblk = 128, 1100, 4
    prm, z, slots, pool = _case(kind, H, [L], nblk, seed=19)
    slots = torch.tensor([2], dtype=torch.int32)
    gp1 = clone_pool(pool, DEV)
    full = _run(kind, prm, z, slots, gp1, [L], [0], H)
    gp2 = clone_pool(pool, DEV)
    ya = _run(kind, prm, z[:split], slots, gp2, [split], [0], H)
    yb = _run(kind, prm, z[split:], slots, gp2, [L - split], [1], H)
    torch.cuda.synchronize()
    assert max_rel_err(torch.cat([ya, yb]).cpu(), full.cpu()) <= 1e-2
    assert torch.equal(gp1.kv_cache[0], gp2.kv_cache[0])
    if kind == "hcl":
        assert max_rel_err(gp2.kv_cache[2][2].cpu(), gp1.kv_cache[2][2].cpu()) <= 1e-4
    else:
        assert torch.equal(gp1.kv_cache[1], gp2.kv_cache[1])


@pytest.mark.parametrize("kind", ["hcm", "hcl"])
def test_decode_after_single_pass(kind):
    H, L, nblk = 256, 700, 4
    prm, z, slots, pool = _case(kind, H, [L + 1], nblk, seed=23)
    gp1 = clone_pool(pool, DEV)
    full = _run(kind, prm, z, slots, gp1, [L + 1], [0], H)
    gp2 = clone_pool(pool, DEV)
    _run(kind, prm, z[:L], slots, gp2, [L], [0], H)
    sw = prm["short_filter"].view(3 * H, 3).to(DEV)
    if kind == "hcl":
        last = hyena_decode(z[L:].to(DEV), sw, gp2.conv_view(), slots.to(DEV),
                            prm["residues"].to(DEV), gp2.ssm_view(), prm["D"].to(DEV),
                            prm["log_poles"][..., 0].to(DEV))
    else:
        K = prm["conv"].shape[-1]
        last = hyena_decode(z[L:].to(DEV), sw, gp2.conv_view(), slots.to(DEV),
                            prm["conv"].view(H, K).to(DEV), gp2.inner_view(K - 1),
                            prm["D"].to(DEV))
    assert max_rel_err(last.cpu(), full[L:].cpu()) <= 1e-2


TILED_HCM = [
    (256, [700, 5, 0, 300, 1, 290], [0, 1, 0, 1, 1, 0], 256),
    (256, [1100, 130], [1, 0], 512),
    (128, [2000, 257, 513], [1, 0, 1], 768),
    (320, [5000, 3, 4097], [0, 1, 1], 1024),
]


@pytest.mark.parametrize("H,lens,has_init,block_t", TILED_HCM)
def test_hcm_tiles_vs_oracle(H, lens, has_init, block_t):
    """The 32-channel hcm kernel over tiles shorter than their segments: a
    tile after the first rebuilds its FIR history from the 256 rows before it."""
    nblk = len(lens) + 3
    prm, z, slots, pool = _case("hcm", H, lens, nblk, seed=61 + H)
    gp = clone_pool(pool, DEV)
    print(f"hcm tiles H={H} lens={lens} block_t={block_t}", flush=True)
    out = _run("hcm", prm, z, slots, gp, lens, has_init, H, bt=block_t).cpu()
    ref = _oracle("hcm", prm, z, pool, lens, has_init, slots, H)
    assert max_rel_err(out, ref) <= 1e-2
    assert torch.equal(gp.kv_cache[0].cpu(), pool.kv_cache[0])
    assert max_rel_err(gp.kv_cache[1].cpu(), pool.kv_cache[1]) <= 1e-2
    assert torch.equal(gp.kv_cache[2].cpu(), pool.kv_cache[2])


def test_block_t_choice():
    """The 7B shape takes the single-pass kernels (hcl: one tile per
    segment; hcm: two 16384-row tiles of 32-channel stripes), the 1B width
    at one long segment the tiled LI scan."""
    assert hcl_block_t(32768, 4096) >= 32768
    assert fir_prefill_block_t(128, 32768, 4096) == 16384
    assert fir_prefill_block_t(128, 131072, 8192) >= 131072
    assert fir_prefill_block_t(7, 32768, 4096) < 32768
    assert stripe_block_t(32768, 1920) is None
    assert stripe_block_t(32768, 1920, max_segment=8192) is not None
    assert stripe_block_t(4096, 1000) is None


def _featurize_channel(z, sw, ch):
    """u and x2 of one channel on the oracle's rounding path (fresh segment):
    short filter per sub-channel in fp32 rounded to bf16, u = bf16(x1 v)."""
    cols = [3 * ch, 3 * ch + 1, 3 * ch + 2]
    zz = torch.cat([torch.zeros(2, 3, dtype=torch.float32), z[:, cols].float()])
    w = sw[cols].float()
    y = (w[:, 0] * zz[:-2] + w[:, 1] * zz[1:-1]) + w[:, 2] * zz[2:]
    y = y.to(torch.bfloat16)
    return (y[:, 1] * y[:, 2]), y[:, 0]


def test_hcl_7b_segment_vs_float64_recurrence():
    """H=4096, one 32768-token segment through the mixer's default choice of
    kernel: g on 4 sampled channels against g built from a float64
    sequential recurrence s_t = p s_{t-1} + u_t, y_t = r . s_t with the
    reference's bf16 mixer tail; final states against the recurrence's."""
    H, L = 4096, 32768
    prm = mixer_params("hcl", H, 7, in_proj_fp8=False)
    g = torch.Generator().manual_seed(3)
    z = (torch.randn(L, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    pool = random_pool(3, H, seed=2)
    gp = clone_pool(pool, DEV)
    slots = torch.tensor([1], dtype=torch.int32)
    bt = hcl_block_t(L, H)
    assert bt >= L  # the single-pass kernel
    out = _run("hcl", prm, z, slots, gp, [L], [0], H, bt=bt).cpu()
    sw = prm["short_filter"].view(3 * H, 3)
    res, lp, D = prm["residues"], prm["log_poles"][..., 0], prm["D"]
    for ch in (0, 1234, 2777, 4095):
        u, x2 = _featurize_channel(z, sw, ch)
        p = np.exp(lp[ch].double().numpy())
        r = res[ch].double().numpy()
        s = np.zeros(16)
        y = np.empty(L)
        for t, x in enumerate(u.double().numpy()):
            s = p * s + x
            y[t] = r @ s
        yb = torch.from_numpy(y).float().to(torch.bfloat16)
        gref = (yb + u * D[ch].to(torch.bfloat16)) * x2
        err = max_rel_err(out[:, ch], gref)
        assert err <= 1e-2, (ch, err)
        st = gp.kv_cache[2][1][ch].cpu().double().numpy()
        assert np.abs(st - s).max() / np.abs(s).max() <= 1e-4, ch
