"""GPU parity of the LI (hcl) long convolution against the oracle.

* hcl_compute_filter against the torch modal filter (triton_hcl.py:77-85);
* iir_segment (scan) against the reference's FFT form (mixers.py:144-210),
  with and without an inherited state;
* the chunk carry: a 32768-token segment at H=4096 against a sequential
  float64 recurrence on 4 sampled channels;
* the fused mixer prefill (mixers.py:1327-1401) over varlen batches with
  continuation segments, within 1e-2 max relative error; final states and
  conv windows;
* chunked prefill (split + continuation) and decode after prefill.
"""

import numpy as np
import pytest
import torch

import oracle
from evo2_flash_amd.decode import hyena_decode
from evo2_flash_amd.hcl import hcl_block_t, hcl_compute_filter, hyena_hcl_prefill, iir_segment
from evo2_flash_amd.metadata import host_tables
from evo2_flash_amd.synthetic import mixer_params

from _cases import clone_pool, max_rel_err, random_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _poles(H, seed):
    prm = mixer_params("hcl", H, seed, in_proj_fp8=False)
    return prm, prm["residues"], prm["log_poles"][..., 0]


def _seq_recurrence(u, res, lp, s0=None):
    """float64 sequential s_t = p s_{t-1} + u_t, y_t = r.s_t for one channel."""
    p = np.exp(lp.astype(np.float64))
    s = np.zeros(16) if s0 is None else s0.astype(np.float64).copy()
    y = np.empty(len(u))
    for t, x in enumerate(u.astype(np.float64)):
        s = p * s + x
        y[t] = res.astype(np.float64) @ s
    return y, s


def test_filter_vs_torch():
    H, L = 64, 3000
    _, res, lp = _poles(H, 3)
    t = torch.arange(L, dtype=torch.float32) + 0.5
    h = hcl_compute_filter(res.to(DEV), lp.to(DEV), t.to(DEV)).cpu()
    ref = oracle.hcl_compute_filter(res, lp, t)
    torch.testing.assert_close(h, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("L,block_t", [(1, 16), (777, 64), (5000, None)])
@pytest.mark.parametrize("with_prev", [False, True])
def test_iir_segment_vs_fft(L, block_t, with_prev):
    H = 128
    _, res, lp = _poles(H, 5)
    g = torch.Generator().manual_seed(L)
    seq = torch.randn(H, L, generator=g)
    s_prev = torch.randn(H, 16, generator=g) * 10 if with_prev else None
    y, st = iir_segment(seq.to(DEV), res.to(DEV), lp.to(DEV),
                        None if s_prev is None else s_prev.to(DEV), block_t=block_t)
    yr, str_ = oracle.iir_segment(seq, res, lp, s_prev)
    assert max_rel_err(y.cpu(), yr) <= 1e-4
    assert max_rel_err(st.cpu(), str_) <= 1e-4


def test_chunk_carry_long_segment_sampled_channels():
    """32768 tokens, H=4096: GPU scan vs a sequential float64 recurrence on 4
    channels, including the final state (the carry crosses 32 tiles)."""
    H, L = 4096, 32768
    _, res, lp = _poles(H, 7)
    g = torch.Generator(device=DEV).manual_seed(1)
    seq_tok = torch.randn(L, H, generator=g, device=DEV)
    y, st = iir_segment(seq_tok.t(), res.to(DEV), lp.to(DEV), None)
    y, st = y.cpu(), st.cpu()
    for ch in (0, 1234, 2777, 4095):
        u = seq_tok[:, ch].cpu().numpy()
        yr, sr = _seq_recurrence(u, res[ch].numpy(), lp[ch].numpy())
        err = np.abs(y[ch].double().numpy() - yr).max() / np.abs(yr).max()
        assert err <= 1e-4, (ch, err)
        assert np.abs(st[ch].double().numpy() - sr).max() / np.abs(sr).max() <= 1e-4


def _tables(lens, has_init, block_t):
    qsl = [0]
    for n in lens:
        qsl.append(qsl[-1] + n)
    seq, tiles, t0 = host_tables(qsl, has_init, block_t, with_tile_start=True)
    return (qsl, torch.tensor(seq, dtype=torch.int32).view(-1, 3).to(DEV),
            torch.tensor(tiles, dtype=torch.int32).view(-1, 2).to(DEV),
            torch.tensor(t0, dtype=torch.int32).to(DEV))


def _fused(prm, z, slots, gp, seq_t, til_t, t0_t, bt, H):
    return hyena_hcl_prefill(z.to(DEV), prm["short_filter"].view(3 * H, 3).to(DEV), gp.conv_view(),
                             prm["residues"].to(DEV), prm["log_poles"][..., 0].to(DEV),
                             gp.ssm_view(), prm["D"].to(DEV), seq_t, slots.to(DEV), til_t, t0_t, bt)


VARLEN = [([300, 5, 0, 130, 1, 77], [0, 1, 0, 1, 1, 0]), ([64, 200], [1, 1])]


@pytest.mark.parametrize("lens,has_init", VARLEN)
@pytest.mark.parametrize("block_t", [16, 64, None])
def test_fused_hcl_prefill_vs_oracle(lens, has_init, block_t, H=256):
    _check_fused_hcl(lens, has_init, block_t, H)


def test_fused_hcl_prefill_long_segments():
    """Segments of many tiles, fresh and continued, between short ones: the
    carry scan crosses up to 80 tiles per segment and segments end in short
    tiles."""
    _check_fused_hcl([5000, 3, 4097, 129, 1, 2048], [0, 1, 1, 0, 1, 1], 64, 320)


@pytest.mark.parametrize("H", [1920, 1000, 200])
@pytest.mark.parametrize("block_t", [16, None])
def test_fused_hcl_prefill_partial_group(H, block_t):
    """H not a multiple of the 256-channel group: at 1920 the last group has
    two full waves (16-byte staging) and two with no channel; at 1000 and 200
    the last wave is partial (element staging)."""
    _check_fused_hcl(*VARLEN[0], block_t, H)


def test_fused_hcl_config0_shape():
    """One 1B-shaped block (H=1920) over one fresh 2048-token sequence, the
    CPU-benchmark shape, against the oracle's FFT form."""
    _check_fused_hcl([2048], [0], None, 1920)


def _check_fused_hcl(lens, has_init, block_t, H):
    nblk = 12
    prm, _, _ = _poles(H, 11)
    g = torch.Generator().manual_seed(4)
    z = (torch.randn(sum(lens), 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = torch.randperm(nblk - 1, generator=g)[:len(lens)].to(torch.int32) + 1
    pool = random_pool(nblk, H, seed=12)
    gp = clone_pool(pool, DEV)
    bt = block_t or hcl_block_t(sum(lens), H)
    qsl, seq_t, til_t, t0_t = _tables(lens, has_init, bt)
    print(f"hcl fused H={H} lens={lens} block_t={bt}", flush=True)
    out = _fused(prm, z, slots, gp, seq_t, til_t, t0_t, bt, H).cpu()
    ref = oracle.iir_mixer_prefill(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(),
                                   prm["residues"], prm["log_poles"][..., 0], pool.ssm_view(),
                                   prm["D"], qsl, slots, has_init)
    assert max_rel_err(out, ref) <= 1e-2
    assert torch.equal(gp.kv_cache[0].cpu(), pool.kv_cache[0])   # conv windows
    assert torch.equal(gp.kv_cache[1].cpu(), pool.kv_cache[1])   # FIR slice untouched
    for j, n in enumerate(lens):
        blk = int(slots[j])
        assert max_rel_err(gp.kv_cache[2][blk].cpu(), pool.kv_cache[2][blk]) <= 1e-3, j


@pytest.mark.parametrize("split", [1, 16, 100, 333])
def test_fused_hcl_split_and_decode(split):
    """prefill(L) == prefill(split) + continued prefill(L-split) (1e-2), and a
    decode step after prefill(L-1) matches the last row of prefill(L)."""
    H, L, nblk = 128, 400, 4
    prm, _, _ = _poles(H, 13)
    g = torch.Generator().manual_seed(9)
    z = (torch.randn(L, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = torch.tensor([2], dtype=torch.int32)
    pool = random_pool(nblk, H, seed=14)
    bt = 64
    gp1 = clone_pool(pool, DEV)
    _, s1, t1, o1 = _tables([L], [0], bt)
    full = _fused(prm, z, slots, gp1, s1, t1, o1, bt, H)
    gp2 = clone_pool(pool, DEV)
    _, sa, ta, oa = _tables([split], [0], bt)
    ya = _fused(prm, z[:split], slots, gp2, sa, ta, oa, bt, H)
    _, sb, tb, ob = _tables([L - split], [1], bt)
    yb = _fused(prm, z[split:], slots, gp2, sb, tb, ob, bt, H)
    assert max_rel_err(torch.cat([ya, yb]).cpu(), full.cpu()) <= 1e-2
    assert max_rel_err(gp2.kv_cache[2][2].cpu(), gp1.kv_cache[2][2].cpu()) <= 1e-4
    assert torch.equal(gp2.kv_cache[0], gp1.kv_cache[0])
    gp3 = clone_pool(pool, DEV)
    _, sc, tc, oc = _tables([L - 1], [0], bt)
    _fused(prm, z[:L - 1], slots, gp3, sc, tc, oc, bt, H)
    last = hyena_decode(z[L - 1:].to(DEV), prm["short_filter"].view(3 * H, 3).to(DEV),
                        gp3.conv_view(), slots.to(DEV), prm["residues"].to(DEV), gp3.ssm_view(),
                        prm["D"].to(DEV), prm["log_poles"][..., 0].to(DEV))
    assert max_rel_err(last.cpu(), full[L - 1:].cpu()) <= 1e-2
