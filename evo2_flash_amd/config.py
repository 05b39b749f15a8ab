"""The Hyena fields of StripedHyena2Config (evo2_flash/config.py:6-205) that
the mixer path reads, and the layer maps of the released model sizes
(evo2_flash/evo2_configs/evo2-{1b-8k,7b-1m,40b-1m}.yml)."""

from dataclasses import dataclass, field


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


def evo2_1b():
    """evo2-1b-8k.yml:4-17, 21, 30."""
    return HyenaConfig(
        hidden_size=1920, num_hidden_layers=25, num_attention_heads=15, intermediate_size=5120,
        attn_layer_idxs=[3, 10, 17, 24], hcl_layer_idxs=[2, 6, 9, 13, 16, 20, 23],
        hcm_layer_idxs=[1, 5, 8, 12, 15, 19, 22], hcs_layer_idxs=[0, 4, 7, 11, 14, 18, 21],
        use_fp8_input_projections=True)


def evo2_7b():
    """evo2-7b-1m.yml:4-17, 21, 32."""
    return HyenaConfig(
        hidden_size=4096, num_hidden_layers=32, num_attention_heads=32, intermediate_size=11264,
        attn_layer_idxs=[3, 10, 17, 24, 31], hcl_layer_idxs=[2, 6, 9, 13, 16, 20, 23, 27, 30],
        hcm_layer_idxs=[1, 5, 8, 12, 15, 19, 22, 26, 29],
        hcs_layer_idxs=[0, 4, 7, 11, 14, 18, 21, 25, 28], use_fp8_input_projections=True)


def evo2_40b():
    """evo2-40b-1m.yml:4-16, 20, 31 (attention at 3, 10, 17, 24, 31, 35, 42, 49)."""
    return HyenaConfig(
        hidden_size=8192, num_hidden_layers=50, num_attention_heads=64, intermediate_size=22528,
        attn_layer_idxs=[3, 10, 17, 24, 31, 35, 42, 49],
        hcl_layer_idxs=[2, 6, 9, 13, 16, 20, 23, 27, 30, 34, 38, 41, 45, 48],
        hcm_layer_idxs=[1, 5, 8, 12, 15, 19, 22, 26, 29, 33, 37, 40, 44, 47],
        hcs_layer_idxs=[0, 4, 7, 11, 14, 18, 21, 25, 28, 32, 36, 39, 43, 46],
        use_fp8_input_projections=True)
