"""GPU parity of the varlen FIR prefill kernels against the oracle.

* fir_prefill (the reference's u -> FIR(u), triton_prefill.py:462-496) and the
  fused hcs/hcm mixer core (mixers.py:1277-1305) within 1e-2 max relative
  error of the fp32 torch path (mixers.py:350-383), over varlen batches with
  continuation segments, segments shorter than the window, empty segments and
  segments spanning many tiles;
* state windows: copies of inputs, so bit-exact where the inputs are given
  (conv window, fir_prefill window);
* chunked prefill: prefill(L) equals prefill(a) + prefill(L-a) continued,
  bit for bit (outputs and windows) on the VALU kernels; on the hcm
  matrix-core kernel outputs agree within 1e-2 (the MFMA's K-sum order
  depends on where a row's 16-row block starts) and windows bitwise;
* the hcm matrix-core kernel over multi-sub-tile, short, empty and
  continuing segments and a part-filled 16-channel group;
* decode after prefill(L) matches the last row of prefill(L+1).
"""

import pytest
import torch

import oracle
from evo2_flash_amd.decode import hyena_decode
from evo2_flash_amd.metadata import host_tables
from evo2_flash_amd.prefill import fir_prefill, fir_prefill_block_t, hyena_fir_prefill
from evo2_flash_amd.synthetic import mixer_params

from _cases import bf16_ulp_diff, clone_pool, max_rel_err, random_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tables(lens, has_init, block_t):
    qsl = [0]
    for n in lens:
        qsl.append(qsl[-1] + n)
    seq, tiles = host_tables(qsl, has_init, block_t)
    seq_t = torch.tensor(seq, dtype=torch.int32).reshape(-1, 3)
    tiles_t = torch.tensor(tiles, dtype=torch.int32).reshape(-1, 2)
    return qsl, seq_t.to(DEV), tiles_t.to(DEV)


VARLEN = [
    ([300, 5, 0, 130, 1, 77], [0, 1, 0, 1, 1, 0]),
    ([64, 200], [1, 1]),
]


@pytest.mark.parametrize("K", [7, 128])
@pytest.mark.parametrize("lens,has_init", VARLEN)
@pytest.mark.parametrize("block_t", [64, None])
def test_fir_prefill_vs_oracle(K, lens, has_init, block_t):
    H, nblk = 256, 12
    block_t = block_t or fir_prefill_block_t(K)
    g = torch.Generator().manual_seed(K + len(lens))
    T = sum(lens)
    u = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(H, K, generator=g) * 0.1).to(torch.bfloat16)
    slots = torch.randperm(nblk - 1, generator=g)[:len(lens)].to(torch.int32) + 1
    pool = random_pool(nblk, H, seed=K)
    gp = clone_pool(pool, DEV)
    qsl, seq_t, tiles_t = _tables(lens, has_init, block_t)
    print(f"fir_prefill K={K} lens={lens} block_t={block_t}", flush=True)
    y = fir_prefill(u.to(DEV), w.to(DEV), gp.inner_view(K - 1), seq_t, slots.to(DEV), tiles_t,
                    block_t).cpu()
    ref = oracle.depthwise_prefill(u, w, qsl, slots, has_init, pool.inner_view(K - 1), K)
    assert max_rel_err(y, ref) <= 1e-2
    assert bf16_ulp_diff(y, ref).max().item() <= 2
    assert torch.equal(gp.raw.cpu(), pool.raw)  # windows are copies: bit-exact


def _fused_case(kind, H, lens, has_init, nblk, seed):
    prm = mixer_params(kind, H, seed, in_proj_fp8=False)
    K = prm["conv"].shape[-1]
    g = torch.Generator().manual_seed(seed)
    z = (torch.randn(sum(lens), 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = torch.randperm(nblk - 1, generator=g)[:len(lens)].to(torch.int32) + 1
    pool = random_pool(nblk, H, seed=seed + 1)
    return prm, K, z, slots, pool


def _run_fused(prm, K, z, slots, gp, seq_t, tiles_t, block_t, H):
    D = prm.get("D")
    return hyena_fir_prefill(z.to(DEV), prm["short_filter"].view(3 * H, 3).to(DEV),
                             gp.conv_view(), prm["conv"].view(H, K).to(DEV), gp.inner_view(K - 1),
                             None if D is None else D.to(DEV), seq_t, slots.to(DEV), tiles_t,
                             block_t)


@pytest.mark.parametrize("kind", ["hcs", "hcm"])
@pytest.mark.parametrize("lens,has_init", VARLEN)
@pytest.mark.parametrize("block_t", [64, None])
def test_fused_fir_prefill_vs_oracle(kind, lens, has_init, block_t):
    H, nblk = 256, 12
    prm, K, z, slots, pool = _fused_case(kind, H, lens, has_init, nblk, seed=3)
    block_t = block_t or fir_prefill_block_t(K)
    gp = clone_pool(pool, DEV)
    qsl, seq_t, tiles_t = _tables(lens, has_init, block_t)
    print(f"fused {kind} lens={lens} block_t={block_t}", flush=True)
    gout = _run_fused(prm, K, z, slots, gp, seq_t, tiles_t, block_t, H).cpu()
    ref = oracle.fir_mixer_prefill(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(),
                                   prm["conv"].view(H, K), pool.inner_view(K - 1), prm.get("D"),
                                   qsl, slots, has_init)
    assert max_rel_err(gout, ref) <= 1e-2
    assert torch.equal(gp.kv_cache[0].cpu(), pool.kv_cache[0])       # conv windows: copies of z
    assert max_rel_err(gp.kv_cache[1].cpu(), pool.kv_cache[1]) <= 1e-2  # u windows
    assert torch.equal(gp.kv_cache[2].cpu(), pool.kv_cache[2])       # LI slice untouched


@pytest.mark.parametrize("kind", ["hcs", "hcm"])
def test_fused_config0_shape(kind):
    """One block at the CPU benchmark's shape: H=1920, one fresh 2048-token segment."""
    H, lens, has_init, nblk = 1920, [2048], [0], 3
    prm, K, z, slots, pool = _fused_case(kind, H, lens, has_init, nblk, seed=9)
    block_t = fir_prefill_block_t(K, sum(lens), H)
    gp = clone_pool(pool, DEV)
    qsl, seq_t, tiles_t = _tables(lens, has_init, block_t)
    gout = _run_fused(prm, K, z, slots, gp, seq_t, tiles_t, block_t, H).cpu()
    ref = oracle.fir_mixer_prefill(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(),
                                   prm["conv"].view(H, K), pool.inner_view(K - 1), prm.get("D"),
                                   qsl, slots, has_init)
    assert max_rel_err(gout, ref) <= 1e-2


@pytest.mark.parametrize("kind", ["hcs", "hcm"])
@pytest.mark.parametrize("split", [1, 63, 64, 100, 257])
def test_fused_split_invariance(kind, split):
    """Chunked prefill: one segment of L rows == split + continuation, bitwise."""
    H, L, nblk = 128, 400, 4
    prm, K, z, slots, pool = _fused_case(kind, H, [L], [0], nblk, seed=17)
    bt = 64
    gp1 = clone_pool(pool, DEV)
    _, seq1, til1 = _tables([L], [0], bt)
    y1 = _run_fused(prm, K, z, slots, gp1, seq1, til1, bt, H)
    gp2 = clone_pool(pool, DEV)
    _, seqa, tila = _tables([split], [0], bt)
    ya = _run_fused(prm, K, z[:split], slots, gp2, seqa, tila, bt, H)
    _, seqb, tilb = _tables([L - split], [1], bt)
    yb = _run_fused(prm, K, z[split:], slots, gp2, seqb, tilb, bt, H)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), torch.cat([ya, yb]).view(torch.int16))
    assert torch.equal(gp1.raw, gp2.raw)


# The hcm fused core on the matrix cores (tiles of >= 256 rows): segments of
# several 256-row sub-tiles, shorter than the 144-row history, empty, and
# continuing from a window; H = 200 leaves a last 16-channel group half full.
MFMA_CASES = [
    (256, [700, 5, 0, 300, 1, 290], [0, 1, 0, 1, 1, 0], 256),
    (256, [1100, 130], [1, 0], 512),
    (200, [513, 40], [1, 1], 256),
]


@pytest.mark.parametrize("H,lens,has_init,block_t", MFMA_CASES)
def test_fused_hcm_mfma_vs_oracle(H, lens, has_init, block_t):
    nblk = len(lens) + 3
    prm, K, z, slots, pool = _fused_case("hcm", H, lens, has_init, nblk, seed=31)
    gp = clone_pool(pool, DEV)
    qsl, seq_t, tiles_t = _tables(lens, has_init, block_t)
    print(f"fused hcm (matrix cores) H={H} lens={lens} block_t={block_t}", flush=True)
    gout = _run_fused(prm, K, z, slots, gp, seq_t, tiles_t, block_t, H).cpu()
    ref = oracle.fir_mixer_prefill(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(),
                                   prm["conv"].view(H, K), pool.inner_view(K - 1), prm.get("D"),
                                   qsl, slots, has_init)
    assert max_rel_err(gout, ref) <= 1e-2
    assert torch.equal(gp.kv_cache[0].cpu(), pool.kv_cache[0])
    assert max_rel_err(gp.kv_cache[1].cpu(), pool.kv_cache[1]) <= 1e-2
    assert torch.equal(gp.kv_cache[2].cpu(), pool.kv_cache[2])


@pytest.mark.parametrize("split", [1, 100, 257, 700])
def test_fused_hcm_mfma_split(split):
    """Chunked prefill on the matrix-core path: one 1100-row segment against
    split + continuation.  An output's products sit at other positions of
    the MFMA's K sum when its 16-row block starts elsewhere, so outputs agree
    to rounding (1e-2) rather than bitwise; the windows are copies of u and
    agree bitwise."""
    H, L, nblk, bt = 128, 1100, 4, 256
    prm, K, z, slots, pool = _fused_case("hcm", H, [L], [0], nblk, seed=19)
    gp1 = clone_pool(pool, DEV)
    _, seq1, til1 = _tables([L], [0], bt)
    y1 = _run_fused(prm, K, z, slots, gp1, seq1, til1, bt, H)
    gp2 = clone_pool(pool, DEV)
    _, seqa, tila = _tables([split], [0], bt)
    ya = _run_fused(prm, K, z[:split], slots, gp2, seqa, tila, bt, H)
    _, seqb, tilb = _tables([L - split], [1], bt)
    yb = _run_fused(prm, K, z[split:], slots, gp2, seqb, tilb, bt, H)
    torch.cuda.synchronize()
    assert max_rel_err(torch.cat([ya, yb]).cpu(), y1.cpu()) <= 1e-2
    assert torch.equal(gp1.raw, gp2.raw)


@pytest.mark.parametrize("kind", ["hcs", "hcm"])
def test_decode_after_prefill(kind):
    """prefill(L) then one decode step == last row of prefill(L+1) (within 1e-2)."""
    H, L, nblk = 256, 150, 4
    prm, K, z, slots, pool = _fused_case(kind, H, [L + 1], [0], nblk, seed=23)
    bt = 64
    gp1 = clone_pool(pool, DEV)
    _, s1, t1 = _tables([L + 1], [0], bt)
    full = _run_fused(prm, K, z, slots, gp1, s1, t1, bt, H)
    gp2 = clone_pool(pool, DEV)
    _, s2, t2 = _tables([L], [0], bt)
    _run_fused(prm, K, z[:L], slots, gp2, s2, t2, bt, H)
    D = prm.get("D")
    last = hyena_decode(z[L:].to(DEV), prm["short_filter"].view(3 * H, 3).to(DEV), gp2.conv_view(),
                        slots.to(DEV), prm["conv"].view(H, K).to(DEV), gp2.inner_view(K - 1),
                        None if D is None else D.to(DEV))
    assert max_rel_err(last.cpu(), full[L:].cpu()) <= 1e-2
    torch.testing.assert_close(gp2.kv_cache[1].float(), gp1.kv_cache[1].float(), rtol=1e-2, atol=1e-2)
    assert torch.equal(gp2.kv_cache[0], gp1.kv_cache[0])
