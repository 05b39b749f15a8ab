"""40B-shaped mixer layers on the GPU (H=8192, one 131072-token prefill, then
decode from that state), checked through properties that do not need the
oracle at full size:

* the fused prefill of each kind over the whole sequence, compared on four
  sampled channels with the oracle run on just those channels (every channel
  of the Hyena core is independent of the others);
* the final state of those channels (LI modal state, FIR window, conv window);
* decode after prefill(L) equals the last row of prefill(L+1), which also
  carries the LI scan across all 256 tiles of the segment.
"""

import pytest
import torch

import oracle
from evo2_flash_amd.decode import channel_major_taps, hyena_decode
from evo2_flash_amd.hcl import hcl_block_t, hyena_hcl_prefill
from evo2_flash_amd.metadata import host_tables
from evo2_flash_amd.prefill import fir_prefill_block_t, hyena_fir_prefill
from evo2_flash_amd.state import HyenaStatePool
from evo2_flash_amd.synthetic import mixer_params

from _cases import max_rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, L = 8192, 131072
CH = [0, 2049, 5000, 8191]  # sampled channels


def _tables(L, block_t, tile_start=False):
    out = host_tables([0, L], [0], block_t, with_tile_start=tile_start)
    seq = torch.tensor(out[0], dtype=torch.int32).view(-1, 3).to(DEV)
    tiles = torch.tensor(out[1], dtype=torch.int32).view(-1, 2).to(DEV)
    if tile_start:
        return seq, tiles, torch.tensor(out[2], dtype=torch.int32).to(DEV)
    return seq, tiles


def _prefill(kind, prm, z, pool, n):
    """Fused mixer prefill of the first n rows of z as one fresh segment on block 1."""
    sw = prm["short_filter"].view(3 * H, 3).to(DEV)
    slots = torch.ones(1, dtype=torch.int32, device=DEV)
    D = prm.get("D")
    D = None if D is None else D.to(DEV)
    if kind == "hcl":
        bt = hcl_block_t(n, H)
        seq, tiles, t0 = _tables(n, bt, tile_start=True)
        return hyena_hcl_prefill(z[:n], sw, pool.conv_view(), prm["residues"].to(DEV),
                                 prm["log_poles"][..., 0].to(DEV), pool.ssm_view(), D, seq, slots,
                                 tiles, t0, bt)
    K = prm["conv"].shape[-1]
    bt = fir_prefill_block_t(K, n, H)
    seq, tiles = _tables(n, bt)
    return hyena_fir_prefill(z[:n], sw, pool.conv_view(), prm["conv"].view(H, K).to(DEV),
                             pool.inner_view(K - 1), D, seq, slots, tiles, bt)


def _sub(prm, kind):
    """The parameters of the sampled channels only."""
    idx = torch.tensor(CH)
    tri = torch.stack([3 * idx, 3 * idx + 1, 3 * idx + 2], 1).reshape(-1)
    sub = {"short_filter": prm["short_filter"].view(3 * H, 3)[tri]}
    if "D" in prm:
        sub["D"] = prm["D"][idx]
    if kind == "hcl":
        sub["residues"] = prm["residues"][idx]
        sub["log_poles"] = prm["log_poles"][idx][..., 0]
    else:
        sub["conv"] = prm["conv"].view(H, -1)[idx]
    return sub, tri


@pytest.fixture(scope="module")
def z_full():
    g = torch.Generator(device=DEV).manual_seed(40)
    z = (torch.randn(L + 1, 3 * H, generator=g, device=DEV) * 1.3).to(torch.bfloat16)
    return z


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_prefill_131k_sampled_channels(kind, z_full):
    prm = mixer_params(kind, H, seed=41, in_proj_fp8=False)
    pool = HyenaStatePool(3, H, DEV)
    print(f"40B-shape prefill {kind} L={L} H={H}", flush=True)
    out = _prefill(kind, prm, z_full, pool, L)
    torch.cuda.synchronize()
    sub, tri = _sub(prm, kind)
    zs = z_full[:L, tri.to(DEV)].cpu()
    ref_pool = HyenaStatePool(3, len(CH), "cpu")
    slots = torch.ones(1, dtype=torch.int32)
    if kind == "hcl":
        ref = oracle.iir_mixer_prefill(zs, sub["short_filter"], ref_pool.conv_view(),
                                       sub["residues"], sub["log_poles"], ref_pool.ssm_view(),
                                       sub["D"], [0, L], slots, [0])
        st = pool.ssm_view()[1][torch.tensor(CH, device=DEV)].cpu()
        assert max_rel_err(st, ref_pool.ssm_view()[1]) <= 1e-3
    else:
        K = sub["conv"].shape[-1]
        ref = oracle.fir_mixer_prefill(zs, sub["short_filter"], ref_pool.conv_view(), sub["conv"],
                                       ref_pool.inner_view(K - 1), sub.get("D"), [0, L], slots,
                                       [0])
        win = pool.inner_view(K - 1)[1][torch.tensor(CH, device=DEV)].cpu()
        assert max_rel_err(win, ref_pool.inner_view(K - 1)[1]) <= 1e-2
    gout = out[:, torch.tensor(CH, device=DEV)].cpu()
    assert max_rel_err(gout, ref) <= 1e-2
    conv = pool.conv_view()[1][tri.to(DEV)].cpu()
    assert torch.equal(conv, ref_pool.conv_view()[1])  # the last two z rows, copied


@pytest.mark.parametrize("kind", ["hcm", "hcl"])
def test_decode_after_131k_prefill(kind, z_full):
    """prefill(L) + one decode step == the last row of prefill(L + 1)."""
    prm = mixer_params(kind, H, seed=43, in_proj_fp8=False)
    p1 = HyenaStatePool(3, H, DEV)
    full = _prefill(kind, prm, z_full, p1, L + 1)
    p2 = HyenaStatePool(3, H, DEV)
    _prefill(kind, prm, z_full, p2, L)
    sw = prm["short_filter"].view(3 * H, 3).to(DEV)
    slots = torch.ones(1, dtype=torch.int32, device=DEV)
    D = prm["D"].to(DEV)
    print(f"40B-shape decode after prefill {kind}", flush=True)
    if kind == "hcl":
        last = hyena_decode(z_full[L:L + 1], sw, p2.conv_view(), slots, prm["residues"].to(DEV),
                            p2.ssm_view(), D, prm["log_poles"][..., 0].to(DEV))
        assert max_rel_err(p2.ssm_view()[1].cpu(), p1.ssm_view()[1].cpu()) <= 1e-3
    else:
        taps = channel_major_taps(prm["conv"].view(H, -1).to(DEV))
        last = hyena_decode(z_full[L:L + 1], sw, p2.conv_view(), slots, taps, p2.inner_view(127), D)
        assert max_rel_err(p2.inner_view(127)[1].cpu(), p1.inner_view(127)[1].cpu()) <= 1e-2
    # Two paths with their own rounding orders (the decode step keeps the
    # reference's fused-kernel order, the prefill scan reads out in another),
    # each within 1e-2 of the fp32 reference, so within 2e-2 of each other:
    # one row of 8192 outputs holds a few elements that sit 1-2 bf16 ulps of
    # the row maximum apart after the x2 gate.
    assert max_rel_err(last.cpu(), full[L:].cpu()) <= 2e-2
    assert torch.equal(p2.conv_view()[1], p1.conv_view()[1])
