"""The mixers under a vLLM-shaped engine, without vLLM: stub modules for
`vllm.forward_context`, `vllm.config` and `vllm.utils.torch_utils` stand in
for the engine, and the mixers must use them as the reference's do
(mixers.py:806-829, 852-856, 1407-1410): registration in the config's
static_forward_context plus the operator in splitting_ops, metadata from the
engine's forward context, and the operator's layer lookup through
no_compile_layers with the encoded layer name."""

import sys
import types

import pytest
import torch

from evo2_flash_amd import engine
from evo2_flash_amd.config import HyenaConfig
from evo2_flash_amd.metadata import build_metadata
from evo2_flash_amd.mixers import (HYENA_MIXER_OP, evo2_hyena_mixer, load_mixer_params,
                                   make_mixer, set_forward_context)
from evo2_flash_amd.synthetic import mixer_params


class _Comp:
    def __init__(self):
        self.static_forward_context = {}
        self.splitting_ops = ["vllm::unified_attention"]


class _Cfg:
    def __init__(self):
        self.compilation_config = _Comp()


class _Fwd:
    def __init__(self, attn_metadata, layers):
        self.attn_metadata = attn_metadata
        self.no_compile_layers = layers


@pytest.fixture
def stub_vllm(monkeypatch):
    cfg = _Cfg()
    state = {"ctx": None}

    def get_forward_context():
        assert state["ctx"] is not None, "Forward context is not set."
        return state["ctx"]

    fc = types.ModuleType("vllm.forward_context")
    fc.get_forward_context = get_forward_context
    vc = types.ModuleType("vllm.config")
    vc.get_current_vllm_config = lambda: cfg
    tu = types.ModuleType("vllm.utils.torch_utils")
    tu._encode_layer_name = lambda name: "enc:" + name
    tu._resolve_layer_name = lambda name: name[len("enc:"):] if name.startswith("enc:") else name
    root = types.ModuleType("vllm")
    utils = types.ModuleType("vllm.utils")
    for name, mod in (("vllm", root), ("vllm.forward_context", fc), ("vllm.config", vc),
                      ("vllm.utils", utils), ("vllm.utils.torch_utils", tu)):
        monkeypatch.setitem(sys.modules, name, mod)
    engine.reset_engine_binding()
    yield cfg, state
    engine.reset_engine_binding()


def _mixer(prefix):
    cfg = HyenaConfig(hidden_size=128, num_hidden_layers=1, hcs_layer_idxs=[0])
    mixer = make_mixer(cfg, 0, prefix=prefix)
    load_mixer_params(mixer, mixer_params("hcs", 128, seed=2, in_proj_fp8=False))
    return mixer


def test_registration_in_engine_config(stub_vllm):
    cfg, _ = stub_vllm
    mixer = _mixer("eng.reg.0")
    comp = cfg.compilation_config
    assert comp.static_forward_context["eng.reg.0"] is mixer
    assert comp.splitting_ops.count(HYENA_MIXER_OP) == 1
    _mixer("eng.reg.1")  # a second layer does not add the op twice
    assert comp.splitting_ops.count(HYENA_MIXER_OP) == 1
    with pytest.raises(ValueError, match="Duplicate"):
        _mixer("eng.reg.0")


def test_metadata_and_layer_from_engine_context(stub_vllm):
    cfg, state = stub_vllm
    mixer = _mixer("eng.ctx.0")
    m = build_metadata(decode_slots=[1], device="cpu")
    state["ctx"] = _Fwd(m, cfg.compilation_config.static_forward_context)
    assert mixer._meta() is m
    state["ctx"] = _Fwd({"eng.ctx.0": m, "other": None}, cfg.compilation_config.static_forward_context)
    assert mixer._meta() is m
    state["ctx"] = _Fwd(None, cfg.compilation_config.static_forward_context)
    assert mixer._meta() is None  # the engine's profiling pass
    # the operator receives the encoded name and resolves it through
    # no_compile_layers
    assert engine.layer_name("eng.ctx.0") == "enc:eng.ctx.0"
    assert engine.lookup_layer("enc:eng.ctx.0") is mixer
    # the operator itself: no metadata, so the profiling pass runs the
    # reference's torch form (out_proj(x2 * x1 * v)) into `output`
    hs = torch.randn(3, 128).to(torch.bfloat16)
    out = torch.empty_like(hs)
    evo2_hyena_mixer(hs, out, None, "enc:eng.ctx.0")
    assert torch.equal(out, mixer._profile_run(hs, None))


def test_local_context_takes_precedence(stub_vllm):
    cfg, state = stub_vllm
    mixer = _mixer("eng.local.0")
    m = build_metadata(decode_slots=[1], device="cpu")
    other = build_metadata(decode_slots=[2], device="cpu")
    state["ctx"] = _Fwd(other, {})
    with set_forward_context(m):
        assert mixer._meta() is m
        assert engine.lookup_layer("enc:eng.local.0") is mixer
    assert mixer._meta() is other


def test_without_engine_the_local_context_is_used(monkeypatch):
    monkeypatch.setitem(sys.modules, "vllm.forward_context", None)  # import fails
    engine.reset_engine_binding()
    try:
        assert engine.engine() is None
        mixer = _mixer("eng.none.0")
        assert engine.layer_name("eng.none.0") == "eng.none.0"
        assert mixer._meta() is None
        m = build_metadata(decode_slots=[1], device="cpu")
        with set_forward_context({"eng.none.0": m}):
            assert mixer._meta() is m
            assert engine.lookup_layer("eng.none.0") is mixer
    finally:
        engine.reset_engine_binding()
