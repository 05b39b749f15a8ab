"""The Hyena fields of StripedHyena2Config (evo2_flash/config.py:6-205) that
the mixer path reads, the validation the reference applies to them when a
converted checkpoint's config.json is loaded (config.py:95-170), and the layer
maps of the released model sizes (evo2_flash/evo2_configs/
evo2-{1b-8k,7b-1m,40b-1m}.yml)."""

from dataclasses import dataclass, field, fields

# The selective fp8 marker a converted checkpoint carries when its Hyena
# in_proj weights are e4m3 (convert.py:631-642); config.py:137-147 accepts
# exactly these values.
FP8_RUNTIME = "vllm_fp8_static_w8a8_v1"
FP8_META_FILENAME = "metadata/hyena_in_proj_fp8_meta.safetensors"
FP8_MARKER = {
    "required": True,
    "runtime": FP8_RUNTIME,
    "format": "e4m3fn",
    "fp8_max": 448,
    "scale_scheme": "per_tensor_static",
    "scale_convention": "dequantization",
    "input_scale_source": "scale_inv_fwd[0]",
    "weight_scale_source": "scale_inv_fwd[1]",
    "metadata_file": FP8_META_FILENAME,
}


@dataclass
class HyenaConfig:
    hidden_size: int = 1920
    num_hidden_layers: int = 25
    num_attention_heads: int = 15
    intermediate_size: int = 5120
    vocab_size: int = 512
    attn_layer_idxs: list = field(default_factory=list)
    hcs_layer_idxs: list = field(default_factory=list)
    hcm_layer_idxs: list = field(default_factory=list)
    hcl_layer_idxs: list = field(default_factory=list)
    short_filter_length: int = 3
    hcs_filter_length: int = 7
    hcm_filter_length: int = 128
    state_size: int = 16
    rms_norm_eps: float = 1e-6
    use_fp8_input_projections: bool = False
    hyena_in_proj_fp8: dict = None
    # FP8 surgery output (config.py:73-112): layer 0's in_proj as a (vocab, 3H)
    # token table; layers whose whole in_proj, or a calibrated subset of its
    # output channels, runs the Hopper fast-accumulation fp8 model.
    hyena_token_table_layers: list = field(default_factory=list)
    hyena_fp8_emulated_layers: list = field(default_factory=list)
    hyena_fp8_emulated_channels: dict = field(default_factory=dict)
    fp8_surgery: dict = None
    # Layout conventions the converter records (convert.py:611-616); the mixer
    # kernels implement the released values only.
    conv_kernels_pre_flipped: bool = True
    interleave: bool = True
    column_split_hyena: bool = False
    hyena_flip_x1x2: bool = False
    tie_word_embeddings: bool = True

    @classmethod
    def from_dict(cls, d):
        """A config from a converted checkpoint's config.json contents, with
        the reference's checks (config.py:95-170) and this build's limits;
        raises ValueError (bad or inconsistent metadata, as the reference) or
        NotImplementedError (a valid layout this build does not run)."""
        names = {f.name for f in fields(cls)}
        kw = {k: v for k, v in d.items() if k in names}
        for k in ("attn_layer_idxs", "hcs_layer_idxs", "hcm_layer_idxs", "hcl_layer_idxs",
                  "hyena_token_table_layers", "hyena_fp8_emulated_layers"):
            kw[k] = [int(i) for i in (kw.get(k) or [])]
        kw["hyena_fp8_emulated_channels"] = {
            int(k): int(v) for k, v in (kw.get("hyena_fp8_emulated_channels") or {}).items()}
        cfg = cls(**kw)
        cfg.validate(quantization_config=d.get("quantization_config"))
        return cfg

    def validate(self, quantization_config=None):
        """Apply the acceptance rules of a converted checkpoint's config
        (config.py:73-170) in table order; the first rule a config breaks
        raises its error.  Returns self."""
        facts = _ConfigFacts(self, quantization_config)
        for rule in _RULES:
            if rule.applies(facts) and rule.broken(facts):
                raise rule.error(rule.message(facts))
        return self

    def layer_kind(self, i):
        """"attn" | "hcs" | "hcm" | "hcl" (config.py:190-199)."""
        if i in self.attn_layer_idxs:
            return "attn"
        if i in self.hcs_layer_idxs:
            return "hcs"
        if i in self.hcm_layer_idxs:
            return "hcm"
        if i in self.hcl_layer_idxs:
            return "hcl"
        raise ValueError(f"layer {i} is in no layer-type list")

    def inner_filter_length(self, i):
        """Inner FIR length of an hcs / hcm layer (config.py:201-205)."""
        return {"hcs": self.hcs_filter_length, "hcm": self.hcm_filter_length}[self.layer_kind(i)]

    def hyena_layers(self):
        return [i for i in range(self.num_hidden_layers) if self.layer_kind(i) != "attn"]


class _ConfigFacts:
    """What the acceptance rules read from one config: the config itself,
    the embedded quantization_config, and derived sets."""

    def __init__(self, cfg, quantization_config):
        self.cfg = cfg
        self.quant = quantization_config
        self.hyena = (set(cfg.hcs_layer_idxs) | set(cfg.hcm_layer_idxs)
                      | set(cfg.hcl_layer_idxs))
        self.kind_sets = [set(cfg.attn_layer_idxs), set(cfg.hcs_layer_idxs),
                          set(cfg.hcm_layer_idxs), set(cfg.hcl_layer_idxs)]
        marker = cfg.hyena_in_proj_fp8
        self.marker = marker if isinstance(marker, dict) else None
        self.surgery = isinstance(cfg.fp8_surgery, dict)

    def marker_mismatch(self):
        """Marker keys whose values differ from the converter's contract."""
        return {k: self.marker.get(k) for k, want in FP8_MARKER.items()
                if self.marker.get(k) != want}

    def bad_emulated_channels(self):
        c = self.cfg
        return {i: n for i, n in c.hyena_fp8_emulated_channels.items()
                if i not in self.hyena or i in c.hyena_fp8_emulated_layers
                or i in c.hyena_token_table_layers or not 0 < n < 3 * c.hidden_size}


@dataclass(frozen=True)
class _Rule:
    """One acceptance rule: where it applies, when it is broken, and the
    error it raises then."""
    applies: object
    broken: object
    error: type
    message: object


def _always(f):
    return True


def _partition_broken(f):
    covered = set().union(*f.kind_sets)
    return (sum(len(k) for k in f.kind_sets) != len(covered)
            or covered != set(range(f.cfg.num_hidden_layers)))


def _fp8(f):
    return f.cfg.use_fp8_input_projections


def _fp8_with_marker(f):
    return f.cfg.use_fp8_input_projections and f.marker is not None


def _token_table(f):
    return bool(f.cfg.hyena_token_table_layers)


def _emulated_layers(f):
    return bool(f.cfg.hyena_fp8_emulated_layers)


def _emulated_channels(f):
    return bool(f.cfg.hyena_fp8_emulated_channels)


def _surgery_needs_bf16(f):
    return f.cfg.use_fp8_input_projections or not f.surgery


# The checkpoint contract of config.py:73-170, plus the layouts this build's
# kernels implement (the released ones).  Messages are the reference's, so a
# user sees the same diagnosis from either implementation.
_RULES = (
    _Rule(_always, _partition_broken, ValueError,
          lambda f: "layer-type lists must partition range(num_hidden_layers)"),
    # fp8 in_proj: the converter's marker must be present, exact and consistent
    _Rule(_fp8, lambda f: f.marker is None, ValueError,
          lambda f: "use_fp8_input_projections=True requires converter-exported "
                    "hyena_in_proj_fp8 metadata; reconvert the source checkpoint"),
    _Rule(_fp8_with_marker, lambda f: f.marker_mismatch(), ValueError,
          lambda f: f"unsupported or incomplete hyena_in_proj_fp8 metadata: "
                    f"{f.marker_mismatch()}"),
    _Rule(_fp8_with_marker, lambda f: f.marker.get("num_layers") != len(f.hyena), ValueError,
          lambda f: "hyena_in_proj_fp8 num_layers does not match the layer map: "
                    f"{f.marker.get('num_layers')} != {len(f.hyena)}"),
    _Rule(_fp8, lambda f: f.quant is not None, ValueError,
          lambda f: "FP8 Hyena projections use the selective static-W8A8 runtime; "
                    "an embedded global quantization_config is unsupported"),
    _Rule(lambda f: not f.cfg.use_fp8_input_projections,
          lambda f: f.cfg.hyena_in_proj_fp8 is not None, ValueError,
          lambda f: "hyena_in_proj_fp8 metadata is present while "
                    "use_fp8_input_projections=False"),
    # FP8 surgery, layer 0 token table
    _Rule(_token_table, lambda f: f.cfg.hyena_token_table_layers != [0], ValueError,
          lambda f: "hyena_token_table_layers may only be [0]: only layer 0's projection "
                    f"input depends on the token alone, got {f.cfg.hyena_token_table_layers}"),
    _Rule(_token_table, lambda f: 0 in f.cfg.attn_layer_idxs, ValueError,
          lambda f: "layer 0 is attention; a token table needs Hyena"),
    _Rule(_token_table, _fp8, ValueError,
          lambda f: "hyena_token_table_layers is the output of FP8 surgery and cannot be "
                    "combined with use_fp8_input_projections=True"),
    _Rule(_token_table, lambda f: not f.surgery, ValueError,
          lambda f: "token-table checkpoints must carry fp8_surgery provenance"),
    # FP8 surgery, whole layers on the emulated GEMM
    _Rule(_emulated_layers,
          lambda f: (any(i not in f.hyena for i in f.cfg.hyena_fp8_emulated_layers)
                     or (0 in f.cfg.hyena_token_table_layers
                         and 0 in f.cfg.hyena_fp8_emulated_layers)),
          ValueError,
          lambda f: f"invalid hyena_fp8_emulated_layers {f.cfg.hyena_fp8_emulated_layers}"),
    _Rule(_emulated_layers, _surgery_needs_bf16, ValueError,
          lambda f: "hyena_fp8_emulated_layers is FP8-surgery output: needs "
                    "use_fp8_input_projections=False and fp8_surgery provenance"),
    # FP8 surgery, hybrid channels
    _Rule(_emulated_channels,
          lambda f: f.bad_emulated_channels() or _surgery_needs_bf16(f), ValueError,
          lambda f: f"invalid hyena_fp8_emulated_channels {f.bad_emulated_channels() or ''}: "
                    "needs FP8-surgery provenance, Hyena layers, 0 < n < 3H"),
    # layouts the kernels implement
    _Rule(_always, lambda f: not f.cfg.conv_kernels_pre_flipped, NotImplementedError,
          lambda f: "conv kernels must be in cross-correlation order "
                    "(conv_kernels_pre_flipped=True)"),
    _Rule(_always,
          lambda f: (not f.cfg.interleave or f.cfg.column_split_hyena
                     or f.cfg.hyena_flip_x1x2),
          NotImplementedError,
          lambda f: "only the interleaved (x2, x1, v) in_proj layout of the released "
                    "checkpoints is supported"),
)


def _with_marker(cfg):
    """Attach the fp8 marker the converter writes for an fp8 model (convert.py:631-642)."""
    if cfg.use_fp8_input_projections:
        cfg.hyena_in_proj_fp8 = dict(FP8_MARKER, num_layers=len(cfg.hyena_layers()))
    return cfg.validate()


def evo2_1b():
    """evo2-1b-8k.yml:4-17, 21, 30."""
    return _with_marker(HyenaConfig(
        hidden_size=1920, num_hidden_layers=25, num_attention_heads=15, intermediate_size=5120,
        attn_layer_idxs=[3, 10, 17, 24], hcl_layer_idxs=[2, 6, 9, 13, 16, 20, 23],
        hcm_layer_idxs=[1, 5, 8, 12, 15, 19, 22], hcs_layer_idxs=[0, 4, 7, 11, 14, 18, 21],
        use_fp8_input_projections=True))


def evo2_7b():
    """evo2-7b-1m.yml:4-17, 21, 32."""
    return _with_marker(HyenaConfig(
        hidden_size=4096, num_hidden_layers=32, num_attention_heads=32, intermediate_size=11264,
        attn_layer_idxs=[3, 10, 17, 24, 31], hcl_layer_idxs=[2, 6, 9, 13, 16, 20, 23, 27, 30],
        hcm_layer_idxs=[1, 5, 8, 12, 15, 19, 22, 26, 29],
        hcs_layer_idxs=[0, 4, 7, 11, 14, 18, 21, 25, 28], use_fp8_input_projections=True))


def evo2_40b():
    """evo2-40b-1m.yml:4-16, 20, 31 (attention at 3, 10, 17, 24, 31, 35, 42, 49)."""
    return _with_marker(HyenaConfig(
        hidden_size=8192, num_hidden_layers=50, num_attention_heads=64, intermediate_size=22528,
        attn_layer_idxs=[3, 10, 17, 24, 31, 35, 42, 49],
        hcl_layer_idxs=[2, 6, 9, 13, 16, 20, 23, 27, 30, 34, 38, 41, 45, 48],
        hcm_layer_idxs=[1, 5, 8, 12, 15, 19, 22, 26, 29, 33, 37, 40, 44, 47],
        hcs_layer_idxs=[0, 4, 7, 11, 14, 18, 21, 25, 28, 32, 36, 39, 43, 46],
        use_fp8_input_projections=True))
