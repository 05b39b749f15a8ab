"""GPU parity of the Hopper fp8 fast-accumulation model (csrc/fp8_emul.hip)
against the oracle's restatement of fp8_emul.py, bit for bit: the raw
accumulator, the scaled linear, and the FP8-surgery mixers that use it
(a fully emulated layer and a hybrid layer, mixers.py:691-800, 1076-1092)."""

import itertools

import pytest
import torch

import oracle
from evo2_flash_amd.config import HyenaConfig
from evo2_flash_amd.fp8_emul import fast_accum_mm, static_fp8_linear_emulated
from evo2_flash_amd.metadata import build_metadata
from evo2_flash_amd.mixers import load_mixer_params, make_mixer, set_forward_context
from evo2_flash_amd.synthetic import mixer_params

from _cases import clone_pool, max_rel_err, oracle_mixer_step, random_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"
E4M3 = torch.float8_e4m3fn
_ids = itertools.count()


def _e4m3(shape, scale, seed, specials=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * scale).clamp(-448, 448).to(E4M3)
    if specials:  # zeros, subnormals, the largest magnitude, both signs
        flat = x.view(-1)
        idx = torch.randperm(flat.numel(), generator=g)[:8]
        vals = [0.0, -0.0, 2.0 ** -9, -3 * 2.0 ** -9, 448.0, -448.0, 2.0 ** -6, 0.0]
        flat[idx] = torch.tensor(vals).to(E4M3)
    return x


@pytest.mark.parametrize("N,M,K", [(5, 300, 64), (17, 520, 128), (64, 256, 1920), (1, 37, 32)])
def test_accumulator_bitwise(N, M, K):
    a8 = _e4m3((N, K), 3.0, seed=N + K)
    w8 = _e4m3((M, K), 0.05, seed=M + K)
    print(f"fast accum N={N} M={M} K={K}", flush=True)
    got = fast_accum_mm(a8.to(DEV), w8.float().t().contiguous().to(torch.bfloat16).to(DEV)).cpu()
    ref = oracle.fast_accum_mm(a8.float(), w8.float())
    assert torch.equal(got, ref)


def test_linear_bitwise_and_strided_weight():
    N, M, K = 33, 200, 256
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(3, 11, K, generator=g) * 2).to(torch.bfloat16)
    w8 = _e4m3((M, K), 0.05, seed=2)
    sx = torch.tensor([6.0 / 448])
    sw = torch.tensor([0.05 * 4 / 448])
    # the K-major weight as a column slice of a wider table
    wide = torch.zeros(K, 2 * M, dtype=torch.bfloat16)
    wide[:, 5:5 + M] = w8.float().t().to(torch.bfloat16)
    print("fast accum linear", flush=True)
    got = static_fp8_linear_emulated(x.to(DEV), wide.to(DEV)[:, 5:5 + M], sx.to(DEV),
                                     sw.to(DEV)).cpu()
    ref = oracle.fp8_linear_fast_accum(x, w8, sx, sw)
    assert got.shape == (3, 11, M)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    with pytest.raises(ValueError):
        static_fp8_linear_emulated(x.float().to(DEV), wide.to(DEV)[:, :M], sx.to(DEV), sw.to(DEV))


@pytest.mark.parametrize("mode", ["emulated", "hybrid"])
def test_surgery_mixer_vs_oracle(mode):
    """An hcm mixer whose in_proj is the emulated GEMM (whole, or 40 of its
    output channels over a bf16 projection), one decode + prefill step."""
    H, nblk = 256, 8
    kw = {"hyena_fp8_emulated_layers": [0]} if mode == "emulated" else \
        {"hyena_fp8_emulated_channels": {0: 40}}
    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=1, hcm_layer_idxs=[0],
                      fp8_surgery={"version": 1}, **kw).validate()
    mixer = make_mixer(cfg, 0, prefix=f"emul{next(_ids)}.mixer", device=DEV)
    base = mixer_params("hcm", H, seed=5, in_proj_fp8=True)
    w8, s_w = base.pop("in_proj.weight"), base.pop("in_proj.weight_scale")
    s_x = base.pop("in_proj.input_scale")
    scales = torch.cat([s_x, s_w]).float()
    prm = dict(base)
    if mode == "emulated":
        cols = torch.arange(3 * H)
        prm["in_proj_emul_weight_t"] = w8.float().t().contiguous().to(torch.bfloat16)
    else:
        g = torch.Generator().manual_seed(6)
        cols = torch.randperm(3 * H, generator=g)[:40].sort().values
        prm["in_proj.weight"] = (w8.float() * s_w).to(torch.bfloat16)
        prm["in_proj_emul_weight_t"] = w8.float()[cols].t().contiguous().to(torch.bfloat16)
        prm["in_proj_emul_cols"] = cols
    prm["in_proj_emul_scales"] = scales
    load_mixer_params(mixer, prm)
    pool = random_pool(nblk, H, seed=7)
    gp = clone_pool(pool, DEV)
    mixer.kv_cache = gp.kv_cache
    dec, lens, slots, init = [3, 0], [21, 40], [5, 2], [1, 0]
    nd, npt = len(dec), sum(lens)
    hs = torch.randn(nd + npt + 2, H, generator=torch.Generator().manual_seed(8))
    hs = hs.to(torch.bfloat16)
    m = build_metadata(decode_slots=dec, prefill_lens=lens, prefill_slots=slots, has_init=init,
                       device=DEV)
    print(f"surgery mixer {mode}", flush=True)
    with set_forward_context(m):
        got = mixer(hs.to(DEV)).cpu()
    emul = oracle.fp8_linear_fast_accum(hs[:nd + npt], w8[cols], s_x, s_w)
    if mode == "emulated":
        z = emul
    else:
        z = (hs[:nd + npt].float() @ prm["in_proj.weight"].float().t()).to(torch.bfloat16)
        z[:, cols] = emul
    ref = oracle_mixer_step("hcm", base, hs, pool, dec, lens, slots, init, H, z=z)
    assert max_rel_err(got, ref) <= 1e-2
    # the emulated projection itself is bit-exact: compare it directly
    zg, zh = mixer._project(hs[:nd + npt].to(DEV)).cpu(), z
    cmp = cols if mode == "hybrid" else slice(None)
    assert torch.equal(zg[:, cmp].view(torch.int16), zh[:, cmp].view(torch.int16))
