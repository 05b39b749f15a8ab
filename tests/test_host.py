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


def _spec_mixer(prefix):
    cfg = HyenaConfig(hidden_size=128, num_hidden_layers=1, hcs_layer_idxs=[0])
    mixer = make_mixer(cfg, 0, prefix=prefix)
    mixer.kv_cache = HyenaStatePool(4, 128, "cpu").kv_cache
    return mixer


def test_speculative_predicate_is_the_reference_one():
    """Each of the reference's three conditions alone marks a step
    speculative (mixers.py:930-937), which sends its decode rows through the
    snapshot path."""
    mixer = _spec_mixer("host.spec.pred")
    plain = build_metadata(decode_slots=[1, 2], device="cpu")
    assert not mixer.is_speculative_decode(plain)
    mixer._check_meta(plain)
    # a speculative-capable runner's ordinary step: (nd, 2) slots, one token per row
    two_col = build_metadata(decode_slots=[1, 2], device="cpu")
    two_col.state_indices_tensor_d = torch.tensor([[1, 3], [2, 0]], dtype=torch.int32)
    assert two_col.num_decode_tokens == two_col.num_decodes
    assert mixer.is_speculative_decode(two_col)
    # more decode tokens than requests with a 1-D slot table
    packed = build_metadata(decode_slots=[1, 2], device="cpu")
    packed.num_decode_tokens = 4
    assert mixer.is_speculative_decode(packed)
    # acceptance counts alone
    counted = build_metadata(decode_slots=[1], device="cpu")
    counted.num_accepted_tokens = torch.ones(1, dtype=torch.int32)
    assert mixer.is_speculative_decode(counted)
    # a (nd, 1) column is not speculative
    one_col = build_metadata(decode_slots=[1, 2], device="cpu")
    one_col.state_indices_tensor_d = torch.tensor([[1], [2]], dtype=torch.int32)
    assert not mixer.is_speculative_decode(one_col)


def test_hyena_decode_refuses_short_slot_table():
    """Fewer slots than rows would make the kernel read past the slot table."""
    from evo2_flash_amd.decode import hyena_decode

    H = 128
    prm = mixer_params("hcs", H, seed=3, in_proj_fp8=False)
    pool = HyenaStatePool(4, H, "cpu")
    z = torch.zeros(3, 3 * H, dtype=torch.bfloat16)
    for slots in (torch.tensor([1, 2], dtype=torch.int32),
                  torch.tensor([[1, 2, 3]], dtype=torch.int32)):
        with pytest.raises(ValueError, match="one state block per row"):
            hyena_decode(z, prm["short_filter"].view(3 * H, 3), pool.conv_view(), slots,
                         prm["conv"].view(H, 7), pool.inner_view(6))


class _SlottedMetadata:
    """Metadata that refuses new attributes, like a class with __slots__."""
    __slots__ = ("num_prefills", "num_prefill_tokens", "num_decodes", "num_decode_tokens",
                 "query_start_loc_p", "has_initial_states_p", "state_indices_tensor_p",
                 "state_indices_tensor_d", "seq_lens")


def test_prefill_tables_on_engine_metadata_objects():
    """The tables are built from any object with vLLM's field names: memoised
    on it when it takes attributes, rebuilt per call when it does not
    (mixers.py:95-123, 386-415)."""
    import types

    from evo2_flash_amd.metadata import prefill_segments, prefill_tables

    qsl = torch.tensor([0, 5, 12], dtype=torch.int32)
    flags = torch.tensor([True, False])
    slots = torch.tensor([3, 1], dtype=torch.int32)
    want_seq = [[0, 5, 1], [5, 12, 0]]
    want_tiles = [[0, 0], [0, 4], [1, 5], [1, 9]]
    ns = types.SimpleNamespace(num_prefills=2, num_prefill_tokens=12, num_decodes=0,
                               num_decode_tokens=0, query_start_loc_p=qsl,
                               has_initial_states_p=flags, state_indices_tensor_p=slots)
    seq, tiles, ts = prefill_tables(ns, 4, "cpu")
    assert seq.tolist() == want_seq and tiles.tolist() == want_tiles and ts.tolist() == [0, 2, 4]
    assert prefill_tables(ns, 4, "cpu")[0] is seq  # memoised
    assert prefill_segments(ns) == ([0, 5, 12], [True, False])
    sl = _SlottedMetadata()
    sl.num_prefills, sl.num_prefill_tokens = 2, 12
    sl.query_start_loc_p, sl.has_initial_states_p, sl.state_indices_tensor_p = qsl, flags, slots
    seq2, tiles2, _ = prefill_tables(sl, 4, "cpu")
    assert seq2.tolist() == want_seq and tiles2.tolist() == want_tiles
    assert not hasattr(sl, "_evo2_prefill_tables")
    # no has_initial_states_p at all: every segment starts fresh
    bare = types.SimpleNamespace(num_prefills=1, num_prefill_tokens=5,
                                 query_start_loc_p=torch.tensor([0, 5]))
    assert prefill_tables(bare, 8, "cpu")[0].tolist() == [[0, 5, 0]]


def test_custom_op_registration_and_opcheck():
    """`vllm::evo2_hyena_mixer` is registered with `output` as its only
    mutated argument and a fake implementation; `forward` goes through it.
    Checked with torch.library.opcheck on the profiling path (no metadata),
    which runs on the CPU with bf16 projections."""
    schema = str(torch.ops.vllm.evo2_hyena_mixer.default._schema)
    assert schema == ("vllm::evo2_hyena_mixer(Tensor hidden_states, Tensor(a1!) output, "
                      "Tensor? token_ids, str layer_name) -> ()")
    H = 64
    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=1, hcm_layer_idxs=[0])
    mixer = make_mixer(cfg, 0, prefix="host.op.0")
    load_mixer_params(mixer, mixer_params("hcm", H, seed=5, in_proj_fp8=False))
    hs = torch.randn(6, H, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    out = torch.empty_like(hs)
    torch.library.opcheck(torch.ops.vllm.evo2_hyena_mixer.default,
                          (hs, out, None, "host.op.0"))
    got = mixer(hs)
    z = hs.float() @ mixer.in_proj.weight.float().t()
    z = z.to(torch.bfloat16)
    y = z[:, 0::3] * z[:, 1::3] * z[:, 2::3]
    want = torch.nn.functional.linear(y, mixer.out_proj.weight, mixer.out_proj.bias)
    assert torch.allclose(got.float(), want.float(), rtol=2e-2, atol=2e-2)
    # traced, the operator stays one opaque node
    gm = torch.fx.experimental.proxy_tensor.make_fx(
        lambda h, o: torch.ops.vllm.evo2_hyena_mixer(h, o, None, "host.op.0"),
        tracing_mode="fake")(hs, out)
    assert any("evo2_hyena_mixer" in str(n.target) for n in gm.graph.nodes)


def test_conv_reload_refreshes_decode_taps():
    """Loading `conv` through its weight_loader (the engine's load path,
    model.py:374-377) after the decode taps exist rewrites them in place."""
    H = 128
    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=2, hcs_layer_idxs=[0], hcm_layer_idxs=[1])
    mixer = make_mixer(cfg, 1, prefix="host.reload.1")
    load_mixer_params(mixer, mixer_params("hcm", H, seed=6, in_proj_fp8=False))
    taps = mixer._decode_taps
    assert torch.equal(taps, mixer.conv.detach().view(H, 128))
    new = mixer_params("hcm", H, seed=7, in_proj_fp8=False)["conv"]
    mixer.conv.weight_loader(mixer.conv, new)
    assert mixer._decode_taps is taps  # same storage: captured graphs stay valid
    assert torch.equal(taps, new.view(H, 128))


def test_packed_weight_rules():
    """Where the fp8 linear reads its packed decode copy: the shapes where
    evo2_fp8_gemm streams the weight (M <= 64, or ceil(M / 64) * N <= 60000,
    the constant the C dispatcher uses), for weights with a decode layout
    (N a multiple of 16, K of 128)."""
    import re
    from evo2_flash_amd.fp8 import STREAM_MAX_WORK, packable, streams_weight
    src = open(__file__.replace("tests/test_host.py",
                                "evo2_flash_amd/csrc/fp8_gemm.hip")).read()
    assert int(re.search(r"#define STREAM_MAX_WORK (\d+)", src).group(1)) == STREAM_MAX_WORK
    assert streams_weight(1, 10 ** 6) and streams_weight(64, 10 ** 6)
    assert not streams_weight(0, 12288)
    assert streams_weight(256, 12288)                 # verify-sized in_proj: 4 x 12288
    assert streams_weight(320, 12000) and not streams_weight(320, 12001)
    assert not streams_weight(8192, 12288)
    assert packable(12288, 4096) and packable(16, 128)
    assert not packable(12280, 4096) and not packable(4096, 4000)


def test_check_block_table():
    """The host check of a paged-attention block table: every page a
    sequence's positions use lies in [1, num_pages); pages past a sequence's
    length are not looked at."""
    from evo2_flash_amd.attention import check_block_table
    table = torch.tensor([[3, 1, 2, 0], [4, 5, 9, -1]], dtype=torch.int32)
    check_block_table(table, [48, 32], 6)          # 3 pages and 2 pages
    check_block_table(table, torch.tensor([1, 0]), 6)
    with pytest.raises(ValueError, match=r"block_table\[1, 2\] = 9 is outside \[1, 6\)"):
        check_block_table(table, [48, 48], 6)
    with pytest.raises(ValueError, match=r"block_table\[0, 3\] = 0"):
        check_block_table(table, [64, 16], 6)
    with pytest.raises(ValueError, match=r"block_table\[1, 3\] = -1"):
        check_block_table(table, [16, 64], 10)
    with pytest.raises(ValueError, match="need 5 pages"):
        check_block_table(table, [65, 16], 10)
    with pytest.raises(ValueError, match="cannot serve 3"):
        check_block_table(table, [16, 16, 16], 10)


def test_shared_prefix_pages():
    """The leading block-table entries that the first B rows share."""
    from evo2_flash_amd.attention import shared_prefix_pages
    table = torch.tensor([[7, 8, 9, 1, 2], [7, 8, 9, 3, 4], [7, 8, 5, 6, 0]], dtype=torch.int32)
    assert shared_prefix_pages(table, 2) == 3
    assert shared_prefix_pages(table, 3) == 2
    assert shared_prefix_pages(table, 1) == 0
    same = torch.tensor([[1, 2], [1, 2]], dtype=torch.int32)
    assert shared_prefix_pages(same, 2) == 2
    assert shared_prefix_pages(torch.tensor([[1, 2], [3, 2]], dtype=torch.int32), 2) == 0
