"""Converted checkpoints: the converter (vortex state dict -> directory,
convert.py:396-678) and the loader the mixers use (config.py:95-170 checks,
model.py:362-379 names), on a small synthetic vortex checkpoint.

The transformations are pinned by what they mean rather than by their
formulas: the Hyena-MR flip by an impulse through the oracle's FIR against
the source's true-convolution taps, the qkv permutation by building the
vortex layout from known Wq/Wk/Wv, the e4m3 export by its dequantisation
error bound and saturation.  The GPU test runs mixers loaded from the
directory against the oracle on the same tensors.
"""

import io
import itertools
import json
import os

import pytest
import torch

import oracle
from evo2_flash_amd import checkpoint, convert
from evo2_flash_amd.config import FP8_MARKER, HyenaConfig

from _cases import clone_pool, max_rel_err, oracle_mixer_step, random_pool

H, NH, VOCAB, MLP, S = 64, 4, 512, 96, 16
YML = {
    "hidden_size": H, "num_attention_heads": NH, "num_layers": 5, "vocab_size": VOCAB,
    "inner_mlp_size": MLP, "attn_layer_idxs": [3], "hcs_layer_idxs": [0, 4],
    "hcm_layer_idxs": [1], "hcl_layer_idxs": [2], "short_filter_length": 3,
    "hcs_filter_length": 7, "hcm_filter_length": 128, "state_size": S,
    "use_fp8_input_projections": True, "rotary_emb_base": 100000000, "tie_embeddings": True,
    "eps": 1e-6, "max_seqlen": 8192, "column_split": True, "interleave": True,
}
GROUPS = 16


def te_meta(scale_w, scale_x, seed):
    g = torch.Generator().manual_seed(seed)
    scale = torch.tensor([scale_x, scale_w, 1.0])
    return {"scale_fwd": scale, "scale_inv_fwd": 1.0 / scale,
            "amax_history_fwd": torch.rand(16, 3, generator=g),
            "extra_fp8_variables": {"fp8_checkpoint": True, "num_gemms": 1, "fp8_max_fwd": 448}}


def vortex_sd(seed=0, qkv=None):
    """A vortex-layout state dict for YML (fp8 Hyena projections with TE
    extra states, one as a serialised BytesIO as the real files hold them)."""
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    rn = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(bf)  # noqa: E731
    sd = {"embedding_layer.weight": rn(VOCAB, H, sc=1.0), "norm.scale": rn(H, sc=1.0)}
    sd["unembed.weight"] = sd["embedding_layer.weight"].clone()
    for i in range(YML["num_layers"]):
        p = f"blocks.{i}."
        sd[p + "pre_norm.scale"] = rn(H, sc=1.0)
        sd[p + "post_norm.scale"] = rn(H, sc=1.0)
        sd[p + "mlp.l1.weight"] = rn(MLP, H)
        sd[p + "mlp.l2.weight"] = rn(MLP, H)
        sd[p + "mlp.l3.weight"] = rn(H, MLP)
        if i in YML["attn_layer_idxs"]:
            sd[p + "inner_mha_cls.Wqkv.weight"] = qkv if qkv is not None else rn(3 * H, H)
            sd[p + "inner_mha_cls.out_proj.weight"] = rn(H, H)
            sd[p + "inner_mha_cls.out_proj.bias"] = rn(H)
            hd = H // NH
            # fp32 here: with this small head dim a bf16 inv_freq implies
            # 9980, not 10000, after the 3-significant-figure snap
            sd[p + "inner_mha_cls.rotary_emb.inv_freq"] = (
                1.0 / 10000.0 ** (torch.arange(0, hd, 2).float() / hd))
            continue
        w = torch.randn(3 * H, H, generator=g) * 0.02
        sd[p + "projections.weight"] = w.to(bf)
        meta = te_meta(scale_w=448.0 / w.abs().max().item(), scale_x=448.0 / 6.0, seed=seed + i)
        if i == 0:
            buf = io.BytesIO()
            torch.save(meta, buf)
            sd[p + "projections._extra_state"] = buf
        else:
            sd[p + "projections._extra_state"] = meta
        sd[p + "filter.short_filter_weight"] = rn(3 * H, 1, 3, sc=0.3)
        sd[p + "out_filter_dense.weight"] = rn(H, H)
        sd[p + "out_filter_dense.bias"] = rn(H)
        if i in YML["hcl_layer_idxs"]:
            lp = torch.log(0.5 + 0.49 * torch.rand(H, S, 1, generator=g))
            sd[p + "filter.log_poles"] = lp
            sd[p + "filter.residues"] = torch.randn(H, S, generator=g) * 0.1
            sd[p + "filter.D"] = rn(H, sc=1.0)
        else:
            K = YML["hcm_filter_length"] if i in YML["hcm_layer_idxs"] else YML["hcs_filter_length"]
            sd[p + "filter.h"] = rn(GROUPS, 1, K, sc=0.1)
            if K >= 128:
                sd[p + "filter.D"] = rn(H, sc=1.0)
    return sd


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("ckpt") / "evo2_tiny")
    sd = vortex_sd(seed=1)
    convert.convert_checkpoint(sd, dict(YML), out, log=lambda *a: None)
    return out, vortex_sd(seed=1)


def test_directory_layout_and_config(ckpt):
    out, _ = ckpt
    assert sorted(os.listdir(out)) == ["config.json", "metadata", "model.safetensors"]
    assert os.listdir(os.path.join(out, "metadata")) == ["hyena_in_proj_fp8_meta.safetensors"]
    raw = json.load(open(os.path.join(out, "config.json")))
    assert raw["hyena_in_proj_fp8"] == dict(FP8_MARKER, num_layers=4)
    assert raw["conv_kernels_pre_flipped"] is True
    # the stored inv_freq implies base 1e4, which wins over the yml's 1e8
    assert raw["rope_theta"] == 10000.0
    cfg = checkpoint.read_config(out)
    assert cfg.hyena_layers() == [0, 1, 2, 4] and cfg.layer_kind(2) == "hcl"


def test_hcm_taps_flipped_into_cross_correlation(ckpt):
    """An impulse through the oracle's cross-correlation FIR with the
    converted taps returns the source's true-convolution taps h[k] at lag k."""
    out, sd = ckpt
    prm = checkpoint.load_mixer_params(out, 1)
    w = prm["conv"].view(H, 128)
    src = sd["blocks.1.filter.h"].float()                          # (G, 1, K)
    L = 200
    x = torch.zeros(L, H)
    x[10] = 1.0
    st = torch.zeros(1, H, 127)
    y = oracle.depthwise_prefill(x, w, [0, L], [0], [0], st, 128)
    for c in (0, 5, H - 1):
        torch.testing.assert_close(y[10:138, c], src[c // (H // GROUPS), 0], rtol=0, atol=0)


def test_hcs_taps_expanded_not_flipped(ckpt):
    out, sd = ckpt
    w = checkpoint.load_mixer_params(out, 0)["conv"].view(H, 7)
    src = sd["blocks.0.filter.h"].float()
    x = torch.zeros(40, H)
    x[3] = 1.0
    y = oracle.depthwise_prefill(x, w, [0, 40], [0], [0], torch.zeros(1, H, 6), 7)
    # K < 128 sources are already cross-correlation: lag k multiplies w[K-1-k]
    for c in (0, 17, H - 1):
        torch.testing.assert_close(y[3:10, c], src[c // (H // GROUPS), 0].flip(0), rtol=0, atol=0)


def test_fp8_export(ckpt):
    out, sd = ckpt
    for i in (0, 1, 2, 4):
        prm = checkpoint.load_mixer_params(out, i)
        w8, sw, sx = prm["in_proj.weight"], prm["in_proj.weight_scale"], prm["in_proj.input_scale"]
        assert w8.dtype == torch.float8_e4m3fn
        w = sd[f"blocks.{i}.projections.weight"].float()
        # e4m3 keeps 3 mantissa bits: |deq - w| <= |w| / 16 in the normal range
        deq = w8.float() * sw
        normal = (w * (1.0 / sw)).abs() >= 2.0 ** -6
        assert ((deq - w).abs() <= w.abs() / 16 + 1e-12)[normal].all()
        assert sx.item() == pytest.approx(6.0 / 448.0, rel=1e-6)
    audit = checkpoint.load_fp8_audit(out)
    assert set(audit) == {0, 1, 2, 4}
    meta1 = sd["blocks.1.projections._extra_state"]
    torch.testing.assert_close(audit[1]["amax_history_fwd"], meta1["amax_history_fwd"])


def test_fp8_export_saturates():
    w = torch.tensor([[1.0, -1.0, 0.5, 1e4]])
    w8 = convert.quantize_te_weight(w, torch.tensor(300.0))
    # e4m3 spacing is 16 in [128, 256) and 32 in [256, 448]: 150 -> 144, 300 -> 288
    assert w8.float().tolist() == [[288.0, -288.0, 144.0, 448.0]]


def test_qkv_rows_become_q_k_v_blocks():
    """Build the vortex per-head interleaved Wqkv from known Wq, Wk, Wv; the
    converted qkv_proj must be [Wq; Wk; Wv]."""
    hd = H // NH
    g = torch.Generator().manual_seed(5)
    wq, wk, wv = (torch.randn(H, H, generator=g) for _ in range(3))
    # vortex: column j of the (H, 3H) transposed weight = (head, {q,k,v}, dim)
    cols = torch.stack([wq.t().reshape(H, NH, hd), wk.t().reshape(H, NH, hd),
                        wv.t().reshape(H, NH, hd)], dim=2)          # (H, NH, 3, hd)
    vortex = cols.reshape(H, 3 * H).t().contiguous()
    torch.testing.assert_close(convert.permute_qkv(vortex, H, NH), torch.cat([wq, wk, wv]))


def test_loaded_mixers_hold_checkpoint_tensors(ckpt):
    out, sd = ckpt
    mixers = checkpoint.load_hyena_mixers(out, device="cpu", name_prefix="cpu.")
    assert sorted(mixers) == [0, 1, 2, 4]
    m2 = mixers[2]
    torch.testing.assert_close(m2.log_poles, sd["blocks.2.filter.log_poles"], rtol=0, atol=0)
    torch.testing.assert_close(m2.residues, sd["blocks.2.filter.residues"], rtol=0, atol=0)
    assert m2.log_poles.dtype == torch.float32
    torch.testing.assert_close(mixers[4].short_filter, sd["blocks.4.filter.short_filter_weight"])
    torch.testing.assert_close(mixers[1].D, sd["blocks.1.filter.D"])
    torch.testing.assert_close(mixers[0].out_proj.bias, sd["blocks.0.out_filter_dense.bias"])


def _write_variant(src, dst, edit_cfg=None, edit_tensors=None, edit_audit=None):
    from safetensors.torch import load_file, save_file

    os.makedirs(os.path.join(dst, "metadata"), exist_ok=True)
    cfg = json.load(open(os.path.join(src, "config.json")))
    t = load_file(os.path.join(src, "model.safetensors"))
    a = load_file(os.path.join(src, "metadata", "hyena_in_proj_fp8_meta.safetensors"))
    if edit_cfg:
        edit_cfg(cfg)
    if edit_tensors:
        edit_tensors(t)
    if edit_audit:
        edit_audit(a)
    json.dump(cfg, open(os.path.join(dst, "config.json"), "w"))
    save_file(t, os.path.join(dst, "model.safetensors"))
    save_file(a, os.path.join(dst, "metadata", "hyena_in_proj_fp8_meta.safetensors"))
    return dst


_n = itertools.count()


@pytest.mark.parametrize("edit, err", [
    (lambda c: c["hyena_in_proj_fp8"].update(runtime="other"), ValueError),
    (lambda c: c["hyena_in_proj_fp8"].update(num_layers=3), ValueError),
    (lambda c: c.pop("hyena_in_proj_fp8"), ValueError),
    (lambda c: c.update(use_fp8_input_projections=False), ValueError),
    (lambda c: c.update(quantization_config={"quant_method": "fp8"}), ValueError),
    (lambda c: c.update(hyena_fp8_emulated_layers=[1]), ValueError),  # needs bf16 + surgery
    (lambda c: c.update(hyena_flip_x1x2=True), NotImplementedError),
    (lambda c: c.update(conv_kernels_pre_flipped=False), NotImplementedError),
    (lambda c: c.update(hcs_layer_idxs=[0, 4, 1]), ValueError),
])
def test_config_rejected(ckpt, tmp_path, edit, err):
    out, _ = ckpt
    bad = _write_variant(out, str(tmp_path / f"v{next(_n)}"), edit_cfg=edit)
    with pytest.raises(err):
        checkpoint.read_config(bad)


@pytest.mark.parametrize("edit", [
    lambda t: t.update({"model.layers.1.mixer.in_proj.weight":
                        t["model.layers.1.mixer.in_proj.weight"].to(torch.bfloat16)}),
    lambda t: t.pop("model.layers.2.mixer.residues"),
    lambda t: t.update({"model.layers.1.mixer.log_poles": torch.zeros(H, S, 1)}),
    lambda t: t.update({"model.layers.2.mixer.in_proj.weight_scale": torch.zeros(1)}),
    lambda t: t.update({"model.layers.4.mixer.conv.weight": torch.zeros(H, 1, 6,
                                                                       dtype=torch.bfloat16)}),
])
def test_tensors_rejected(ckpt, tmp_path, edit):
    out, _ = ckpt
    bad = _write_variant(out, str(tmp_path / f"t{next(_n)}"), edit_tensors=edit)
    cfg = checkpoint.read_config(bad)
    with pytest.raises(ValueError):
        for i in cfg.hyena_layers():
            checkpoint.load_mixer_params(bad, i, cfg)


def test_audit_mismatch_rejected(ckpt, tmp_path):
    out, _ = ckpt

    def tamper(t):
        t["model.layers.4.mixer.in_proj.input_scale"] = (
            t["model.layers.4.mixer.in_proj.input_scale"] * 1.001)

    bad = _write_variant(out, str(tmp_path / "audit"), edit_tensors=tamper)
    with pytest.raises(ValueError, match="scale_inv_fwd"):
        checkpoint.load_fp8_audit(bad)
    bad2 = _write_variant(out, str(tmp_path / "audit2"),
                          edit_audit=lambda a: a.pop("layers.2.amax_history_fwd"))
    with pytest.raises(ValueError, match="missing"):
        checkpoint.load_fp8_audit(bad2)


def test_te_extra_state_rejected():
    good = te_meta(2.0, 3.0, 0)
    convert.te_extra_state(good, "k")
    for edit in (lambda m: m.update(scale_inv_fwd=torch.ones(3)),
                 lambda m: m.update(scale_fwd=torch.tensor([1.0, -1.0, 1.0]),
                                    scale_inv_fwd=torch.tensor([1.0, -1.0, 1.0])),
                 lambda m: m.update(amax_history_fwd=torch.zeros(8, 3)),
                 lambda m: m["extra_fp8_variables"].update(num_gemms=2),
                 lambda m: m.pop("scale_fwd")):
        m = te_meta(2.0, 3.0, 0)
        edit(m)
        with pytest.raises(ValueError):
            convert.te_extra_state(m, "k")


def test_vortex_file_roundtrip(tmp_path):
    """A vortex .pt holding BytesIO extra states loads with the weights-only
    unpickler and converts to the same tensors as the in-memory dict."""
    sd = vortex_sd(seed=3)
    for k in [k for k in sd if k.endswith("_extra_state")]:
        if not isinstance(sd[k], io.BytesIO):
            buf = io.BytesIO()
            torch.save(sd[k], buf)
            sd[k] = buf
    path = str(tmp_path / "vortex.pt")
    torch.save({"module": sd}, path)
    a, _, _ = convert.convert_state_dict(convert.load_state_dict(path), dict(YML),
                                         log=lambda *x: None)
    b, _, _ = convert.convert_state_dict(vortex_sd(seed=3), dict(YML), log=lambda *x: None)
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k].view(torch.uint8) if a[k].dtype == torch.float8_e4m3fn else a[k],
                           b[k].view(torch.uint8) if b[k].dtype == torch.float8_e4m3fn else b[k]), k


def test_token_table_layer_projects_by_lookup():
    """FP8-surgery layer 0: the projection is the table row of each token."""
    from evo2_flash_amd.mixers import make_mixer

    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=2, vocab_size=VOCAB, hcs_layer_idxs=[0],
                      hcm_layer_idxs=[1], hyena_token_table_layers=[0],
                      fp8_surgery={"version": 1}).validate()
    m = make_mixer(cfg, 0, prefix="tt.mixer0")
    table = torch.randn(VOCAB, 3 * H).to(torch.bfloat16)
    m.in_proj_token_table.data.copy_(table)
    tok = torch.tensor([65, 67, 71, 84, 65])
    z = m._project(torch.zeros(5, H, dtype=torch.bfloat16), tok)
    assert torch.equal(z, table[tok])
    with pytest.raises(ValueError, match="input_ids"):
        m._project(torch.zeros(5, H, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        HyenaConfig(hidden_size=H, num_hidden_layers=2, hcs_layer_idxs=[0], hcm_layer_idxs=[1],
                    hyena_token_table_layers=[1], fp8_surgery={}).validate()


@pytest.mark.gpu
def test_mixers_from_checkpoint_vs_oracle(ckpt):
    """Mixers loaded from the converted directory onto the GPU, one mixed
    decode + prefill step each, against the oracle on the same tensors."""
    from evo2_flash_amd.metadata import build_metadata
    from evo2_flash_amd.mixers import set_forward_context

    out, _ = ckpt
    cfg = checkpoint.read_config(out)
    mixers = checkpoint.load_hyena_mixers(out, device="cuda", name_prefix="gpu.")
    for i, mixer in mixers.items():
        kind = cfg.layer_kind(i)
        prm = checkpoint.load_mixer_params(out, i, cfg)
        pool = random_pool(8, H, seed=50 + i)
        gp = clone_pool(pool, "cuda")
        mixer.kv_cache = gp.kv_cache
        dec, lens, slots, init = [2, 0], [33, 9], [5, 3], [1, 0]
        nd, npt = len(dec), sum(lens)
        hs = torch.randn(nd + npt + 3, H, generator=torch.Generator().manual_seed(i))
        hs = hs.to(torch.bfloat16)
        m = build_metadata(decode_slots=dec, prefill_lens=lens, prefill_slots=slots,
                           has_init=init, device="cuda")
        print(f"checkpoint mixer layer {i} ({kind})", flush=True)
        with set_forward_context(m):
            got = mixer(hs.to("cuda")).cpu()
        ref = oracle_mixer_step(kind, prm, hs, pool, dec, lens, slots, init, H)
        assert max_rel_err(got, ref) <= 1e-2, (i, kind)
        assert max_rel_err(gp.kv_cache[2].cpu(), pool.kv_cache[2]) <= 1e-3


def test_surgery_checkpoint_layers(tmp_path):
    """An FP8-surgery directory (config.py:73-94): token table on layer 0, a
    fully emulated layer and a hybrid layer load with their own tensors."""
    Hs, V = 64, 512
    cfg = {"hidden_size": Hs, "num_hidden_layers": 3, "vocab_size": V, "hcs_layer_idxs": [0],
           "hcm_layer_idxs": [1], "hcl_layer_idxs": [2], "use_fp8_input_projections": False,
           "hyena_token_table_layers": [0], "hyena_fp8_emulated_layers": [1],
           "hyena_fp8_emulated_channels": {"2": 12}, "fp8_surgery": {"version": 1}}
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    t = {}
    p = lambda i, n: f"model.layers.{i}.mixer.{n}"  # noqa: E731
    t[p(0, "in_proj_token_table")] = torch.randn(V, 3 * Hs, generator=g).to(bf)
    t[p(1, "in_proj_emul_weight_t")] = torch.randn(Hs, 3 * Hs, generator=g).to(bf)
    t[p(1, "in_proj_emul_scales")] = torch.tensor([0.01, 0.002])
    t[p(2, "in_proj.weight")] = torch.randn(3 * Hs, Hs, generator=g).to(bf)
    t[p(2, "in_proj_emul_weight_t")] = torch.randn(Hs, 12, generator=g).to(bf)
    t[p(2, "in_proj_emul_scales")] = torch.tensor([0.01, 0.002])
    t[p(2, "in_proj_emul_cols")] = torch.arange(12, dtype=torch.int64) * 5
    for i, K in ((0, 7), (1, 128)):
        t[p(i, "conv.weight")] = torch.randn(Hs, 1, K, generator=g).to(bf)
    t[p(1, "D")] = torch.randn(Hs).to(bf)
    t[p(2, "D")] = torch.randn(Hs).to(bf)
    t[p(2, "log_poles")] = -torch.rand(Hs, 16, 1)
    t[p(2, "residues")] = torch.randn(Hs, 16)
    for i in range(3):
        t[p(i, "short_filter.weight")] = torch.randn(3 * Hs, 1, 3, generator=g).to(bf)
        t[p(i, "out_proj.weight")] = torch.randn(Hs, Hs, generator=g).to(bf)
        t[p(i, "out_proj.bias")] = torch.randn(Hs, generator=g).to(bf)
    out = convert.write_checkpoint(str(tmp_path / "surgery"), t, cfg)
    rc = checkpoint.read_config(out)
    assert rc.hyena_fp8_emulated_channels == {2: 12}
    mixers = checkpoint.load_hyena_mixers(out, device="cpu", name_prefix="surgery.")
    assert mixers[0].in_proj_token_table is not None
    torch.testing.assert_close(mixers[1].in_proj_emul_weight_t, t[p(1, "in_proj_emul_weight_t")])
    assert torch.equal(mixers[2].in_proj_emul_cols, t[p(2, "in_proj_emul_cols")])
    assert mixers[2].in_proj.weight.dtype == torch.bfloat16
    bad = dict(t)
    bad.pop(p(2, "in_proj_emul_cols"))
    out2 = convert.write_checkpoint(str(tmp_path / "surgery2"), bad, cfg)
    with pytest.raises(ValueError, match="missing"):
        checkpoint.load_mixer_params(out2, 2)
    cfg_bad = dict(cfg, hyena_fp8_emulated_channels={"2": 3 * Hs})
    with pytest.raises(ValueError):
        HyenaConfig.from_dict(cfg_bad)
