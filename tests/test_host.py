"""Host-side logic without a GPU: the config layer maps, mixer construction
and parameter names (the checkpoint keys), the forward context, and that the
operators refuse to run on CPU tensors."""

import pytest
import torch

from evo2_flash_amd.config import HyenaConfig, evo2_1b, evo2_7b, evo2_40b
from evo2_flash_amd.mixers import (HyenaFIRMixer, HyenaIIRMixer, get_forward_context,
                                   load_mixer_params, make_mixer, set_forward_context,
                                   static_forward_context)
from evo2_flash_amd.metadata import build_metadata
from evo2_flash_amd.state import HyenaStatePool
from evo2_flash_amd.synthetic import mixer_params


def test_layer_maps():
    c7 = evo2_7b()
    kinds = [c7.layer_kind(i) for i in range(32)]
    assert kinds[:5] == ["hcs", "hcm", "hcl", "attn", "hcs"]
    assert kinds.count("attn") == 5 and len(c7.hyena_layers()) == 27
    assert c7.inner_filter_length(0) == 7 and c7.inner_filter_length(1) == 128
    with pytest.raises(KeyError):
        c7.inner_filter_length(2)
    c40 = evo2_40b()
    assert sum(c40.layer_kind(i) == "attn" for i in range(50)) == 8
    assert len(c40.hyena_layers()) == 42
    assert evo2_1b().layer_kind(24) == "attn"
    with pytest.raises(ValueError):
        HyenaConfig(num_hidden_layers=1).layer_kind(0)


def test_mixer_parameter_names_are_checkpoint_keys():
    cfg = HyenaConfig(hidden_size=128, num_hidden_layers=3, hcs_layer_idxs=[0],
                      hcm_layer_idxs=[1], hcl_layer_idxs=[2], use_fp8_input_projections=True)
    names = {}
    for i in range(3):
        m = make_mixer(cfg, i, prefix=f"host.names.{i}")
        names[cfg.layer_kind(i)] = dict(m.named_parameters())
    assert set(names["hcs"]) == {"in_proj.weight", "in_proj.weight_scale", "in_proj.input_scale",
                                 "out_proj.weight", "out_proj.bias", "short_filter", "conv"}
    assert set(names["hcm"]) == set(names["hcs"]) | {"D"}
    assert set(names["hcl"]) == (set(names["hcs"]) - {"conv"}) | {"D", "log_poles", "residues"}
    assert names["hcl"]["log_poles"].shape == (128, 16, 1)
    assert names["hcl"]["log_poles"].dtype == torch.float32
    assert names["hcm"]["in_proj.weight"].dtype == torch.float8_e4m3fn
    assert names["hcm"]["conv"].shape == (128, 1, 128)
    assert isinstance(make_mixer(cfg, 0, prefix="host.names.x"), HyenaFIRMixer)
    assert isinstance(make_mixer(cfg, 2, prefix="host.names.y"), HyenaIIRMixer)


def test_load_params_and_duplicate_prefix():
    cfg = HyenaConfig(hidden_size=128, num_hidden_layers=2, hcs_layer_idxs=[0],
                      hcm_layer_idxs=[1], use_fp8_input_projections=True)
    m = make_mixer(cfg, 1, prefix="host.load.1")
    prm = mixer_params("hcm", 128, seed=1, in_proj_fp8=True)
    load_mixer_params(m, prm)
    assert torch.equal(m.conv.detach(), prm["conv"])
    assert m._decode_taps.shape == (128, 128) and m._decode_taps.stride() == (1, 128)
    with pytest.raises(KeyError):
        load_mixer_params(m, {"nope": torch.zeros(1)})
    with pytest.raises(ValueError, match="Duplicate"):
        make_mixer(cfg, 1, prefix="host.load.1")
    assert static_forward_context["host.load.1"] is m


def test_forward_context_and_cpu_refusal():
    cfg = HyenaConfig(hidden_size=128, num_hidden_layers=1, hcs_layer_idxs=[0])
    mixer = make_mixer(cfg, 0, prefix="host.ctx.0")
    load_mixer_params(mixer, mixer_params("hcs", 128, seed=2, in_proj_fp8=False))
    m = build_metadata(decode_slots=[1], device="cpu")
    assert get_forward_context().attn_metadata is None
    with set_forward_context({"host.ctx.0": m}):
        assert mixer._meta() is m
        with pytest.raises(RuntimeError, match="not bound"):
            mixer(torch.zeros(1, 128, dtype=torch.bfloat16))
        mixer.kv_cache = HyenaStatePool(2, 128, "cpu").kv_cache
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            mixer(torch.zeros(1, 128, dtype=torch.bfloat16))
    assert get_forward_context().attn_metadata is None


def test_speculative_metadata_rejected():
    cfg = HyenaConfig(hidden_size=128, num_hidden_layers=1, hcs_layer_idxs=[0])
    mixer = make_mixer(cfg, 0, prefix="host.spec.0")
    m = build_metadata(decode_slots=[1], device="cpu")
    m.num_accepted_tokens = torch.ones(1, dtype=torch.int32)
    mixer.kv_cache = HyenaStatePool(2, 128, "cpu").kv_cache
    with pytest.raises(NotImplementedError):
        mixer._check_meta(m)
