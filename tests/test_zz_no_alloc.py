"""The allocation-free LI prefill entry point (evo2_hyena_hcl_prefill_noalloc)
against the entry point that takes a workspace, through the C ABI: same
kernels, so outputs, final states and conv windows must be identical bit for
bit.  Two calls in a row on one device, the second with fewer tiles (the
scratch keeps the first call's contents), and a request larger than the
scratch is refused before any device work."""

import ctypes

import pytest
import torch

from evo2_flash_amd import _lib
from evo2_flash_amd.hcl import hcl_block_t
from evo2_flash_amd.metadata import host_tables
from evo2_flash_amd.synthetic import mixer_params

from _cases import random_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(z, prm, pool, lens, has_init, slots, block_t, H):
    qsl = [0]
    for n in lens:
        qsl.append(qsl[-1] + n)
    seq, tiles, ts = host_tables(qsl, has_init, block_t, with_tile_start=True)
    seq_t = torch.tensor(seq, dtype=torch.int32, device=DEV).view(-1, 3)
    til_t = torch.tensor(tiles, dtype=torch.int32, device=DEV).view(-1, 2)
    ts_t = torch.tensor(ts, dtype=torch.int32, device=DEV)
    sw = prm["short_filter"].view(3 * H, 3).to(DEV)
    res = prm["residues"].to(DEV)
    lp = prm["log_poles"][..., 0].contiguous().to(DEV)
    D = prm["D"].to(DEV)
    conv, ssm = pool.conv_view(), pool.ssm_view()
    out = torch.empty(z.shape[0], H, dtype=torch.bfloat16, device=DEV)
    keep = (seq_t, til_t, ts_t, sw, res, lp, D, slots)
    P = _lib.ptr
    head = (P(z), z.stride(0), P(sw), P(conv), *conv.stride(), P(res), *res.stride(),
            P(lp), *lp.stride(), P(ssm), *ssm.stride(), P(D), P(seq_t), len(seq), P(slots),
            slots.stride(0), P(til_t), len(tiles), P(ts_t), block_t)
    tail = (P(out), out.stride(0), z.shape[0], H, min(conv.shape[0], ssm.shape[0]),
            _lib.stream_of(z))
    return head, tail, out, len(tiles), keep


def _run_both(z, prm, pool, lens, has_init, slots, block_t, H):
    """(out, pool) from the workspace entry and from the scratch entry."""
    from _cases import clone_pool

    gp1, gp2 = clone_pool(pool, DEV), clone_pool(pool, DEV)
    h1, t1, out1, ntiles, k1 = _args(z, prm, gp1, lens, has_init, slots, block_t, H)
    nbytes = _lib.lib().evo2_hcl_workspace_bytes(ntiles, H)
    work = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=DEV)
    _lib.call("evo2_hyena_hcl_prefill", *h1, _lib.ptr(work), nbytes, *t1)
    h2, t2, out2, _, k2 = _args(z, prm, gp2, lens, has_init, slots, block_t, H)
    _lib.call("evo2_hyena_hcl_prefill_noalloc", *h2, *t2)
    torch.cuda.synchronize()
    return (out1, gp1), (out2, gp2)


def test_noalloc_matches_workspace_entry_twice():
    H, nblk = 512, 10
    prm = mixer_params("hcl", H, seed=90, in_proj_fp8=False)
    pool = random_pool(nblk, H, seed=91)
    g = torch.Generator().manual_seed(92)
    cases = [([3000, 17, 700], [0, 1, 1], [2, 5, 7]),   # larger first
             ([40, 301], [1, 0], [3, 9])]               # then fewer tiles
    for lens, has_init, slot_list in cases:
        z = (torch.randn(sum(lens), 3 * H, generator=g) * 1.3).to(torch.bfloat16).to(DEV)
        slots = torch.tensor(slot_list, dtype=torch.int32, device=DEV)
        bt = hcl_block_t(sum(lens), H)
        print(f"noalloc H={H} lens={lens} block_t={bt}", flush=True)
        (o1, p1), (o2, p2) = _run_both(z, prm, pool, lens, has_init, slots, bt, H)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), lens
        assert torch.equal(p1.raw, p2.raw), lens


def test_noalloc_refuses_more_than_its_scratch():
    """ntiles * H * 64 bytes beyond 32 MiB: an error, before any launch."""
    lib = _lib.lib()
    n = None
    H, ntiles = 8192, 65
    assert lib.evo2_hcl_workspace_bytes(ntiles, H) > (32 << 20)
    rc = lib.evo2_hyena_hcl_prefill_noalloc(n, 0, n, n, 0, 0, 0, n, 0, 0, n, 0, 0, n, 0, 0, 0,
                                            n, n, 1, n, 1, n, ntiles, n, 1024, n, 0, 1, H, 2, n)
    assert rc == 2  # EVO2_ERR_UNSUPPORTED
    assert b"scratch" in lib.evo2_last_error()
