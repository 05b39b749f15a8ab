"""Hyena mixers with evo2_flash's operator surface (mixers.py:711-1423).

`HyenaFIRMixer` (hcs K=7, hcm K=128) and `HyenaIIRMixer` (hcl) keep the
reference's constructor arguments, parameter names (which are the checkpoint
keys, convert.py:465-499), `kv_cache` 3-tuple and `forward(hidden_states,
token_ids=None)`.  A forward pass runs as the registered custom operator
`torch.ops.vllm.evo2_hyena_mixer(hidden_states, output, token_ids,
layer_name)` (schema `(Tensor hidden_states, Tensor(a!) output, Tensor?
token_ids, str layer_name) -> ()`, with a fake implementation), which looks
the layer up by name and writes into a preallocated `output`
(mixers.py:1404-1423): a compiler treats one mixer as one opaque node and
splits its graph there, so the metadata reads on the host stay out of traced
code.

Per step the metadata (a vLLM Mamba2 metadata object, or
`metadata.Mamba2Metadata`) comes from the forward context.  Decode rows come
first, then prefill rows (mixers.py:29-30); each group is one fused kernel
launch between in_proj and out_proj:

  decode rows   in_proj -> hyena_decode (short conv, gate, inner op, D, x2;
                paged state updated in place) -> out_proj
  prefill rows  in_proj -> hyena_fir_prefill | hyena_hcl_prefill -> out_proj

With no metadata (the engine's profiling pass) the mixer returns
out_proj(x2 * x1 * v) as the reference does (mixers.py:1230-1235).  There is
no CPU path and no speculative-decode path: the kernels run on ROCm devices
and a step whose metadata is speculative by the reference's predicate
(mixers.py:930-937) raises.
"""

import contextlib
from typing import Optional

import torch
from torch import nn

from .decode import channel_major_taps, hyena_decode
from .fp8 import Fp8StaticLinear
from .fp8_emul import static_fp8_linear_emulated
from .hcl import hcl_block_t, hyena_hcl_prefill
from .metadata import decode_state_indices, prefill_tables
from .prefill import fir_prefill_block_t, hyena_fir_prefill

# ---------------------------------------------------------------- forward context
# Layers register under their prefix here, as vLLM's
# compilation_config.static_forward_context does (mixers.py:806-810).
static_forward_context = {}


class ForwardContext:
    """What the mixers read from vLLM's forward context: `attn_metadata`,
    either one metadata object for every layer or a dict keyed by prefix."""

    def __init__(self):
        self.attn_metadata = None


_context = ForwardContext()


def get_forward_context():
    return _context


@contextlib.contextmanager
def set_forward_context(attn_metadata):
    """Run a model step with `attn_metadata` visible to every mixer."""
    prev = _context.attn_metadata
    _context.attn_metadata = attn_metadata
    try:
        yield _context
    finally:
        _context.attn_metadata = prev


# ---------------------------------------------------------------- projections
class Linear(nn.Module):
    """Replicated bf16 linear with vLLM's `forward(x) -> (y, None)`; the GEMM
    is the platform's library GEMM."""

    def __init__(self, in_features, out_features, bias=False, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(out_features, in_features, device=device,
                                               dtype=dtype), requires_grad=False)
        self.bias = (nn.Parameter(torch.zeros(out_features, device=device, dtype=dtype),
                                  requires_grad=False) if bias else None)

    def forward(self, x):
        return torch.nn.functional.linear(x, self.weight, self.bias), None


class ProjectionTap(nn.Module):
    """Parameter-free stand-in for in_proj when the projection is a token
    table (FP8-surgery layer 0, mixers.py:681-688): returns (z, None) like a
    linear, so a hook on `in_proj` still sees the projection output."""

    def forward(self, z):
        return z, None


# ---------------------------------------------------------------- mixers
class HyenaMixerBase(nn.Module):
    """Shared front half: in_proj, the stateful short filter, the paged state
    views and the operator entry (mixers.py:711-1235)."""

    def __init__(self, config, layer_idx, model_config=None, cache_config=None, prefix="",
                 quant_config=None, device=None):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.prefix = prefix or f"model.layers.{layer_idx}.mixer"
        h = config.hidden_size
        self.hidden = h
        self.k_short = config.short_filter_length
        # Only in_proj is fp8 in the released checkpoints (mixers.py:736-757);
        # out_proj follows the model-wide quantisation, bf16 by default.
        self.in_proj_token_table = None
        if layer_idx in getattr(config, "hyena_token_table_layers", ()):
            # FP8-surgery layer 0: the projection of each token, looked up
            # (mixers.py:761-767); its input depends on the token alone.
            self.in_proj = ProjectionTap()
            self.in_proj_token_table = nn.Parameter(
                torch.empty(config.vocab_size, 3 * h, device=device, dtype=torch.bfloat16),
                requires_grad=False)
        elif layer_idx in getattr(config, "hyena_fp8_emulated_layers", ()):
            # FP8 surgery: the whole projection through the Hopper
            # fast-accumulation model on E4M3 operands held in bf16, K-major
            # (mixers.py:768-777).
            self.in_proj = ProjectionTap()
            self.in_proj_emul_weight_t = nn.Parameter(
                torch.empty(h, 3 * h, device=device, dtype=torch.bfloat16), requires_grad=False)
            self.in_proj_emul_scales = nn.Parameter(
                torch.empty(2, device=device, dtype=torch.float32), requires_grad=False)
        elif config.use_fp8_input_projections:
            self.in_proj = Fp8StaticLinear(h, 3 * h, bias=False, device=device)
        else:
            self.in_proj = Linear(h, 3 * h, bias=False, device=device)
            n_emul = getattr(config, "hyena_fp8_emulated_channels", {}).get(layer_idx, 0)
            if n_emul:
                # FP8 surgery, hybrid: the calibrated worst output channels of
                # this bf16 projection are recomputed by the emulated fp8 GEMM
                # and written over the bf16 ones (mixers.py:691-702, 779-800).
                self.in_proj_emul_weight_t = nn.Parameter(
                    torch.empty(h, n_emul, device=device, dtype=torch.bfloat16),
                    requires_grad=False)
                self.in_proj_emul_scales = nn.Parameter(
                    torch.empty(2, device=device, dtype=torch.float32), requires_grad=False)
                self.in_proj_emul_cols = nn.Parameter(
                    torch.empty(n_emul, device=device, dtype=torch.int64), requires_grad=False)
        self.out_proj = (Fp8StaticLinear(h, h, bias=True, device=device)
                         if quant_config == "fp8" else Linear(h, h, bias=True, device=device))
        self.short_filter = nn.Parameter(torch.empty(3 * h, 1, self.k_short, device=device,
                                                     dtype=torch.bfloat16), requires_grad=False)
        if self.prefix in static_forward_context:
            raise ValueError(f"Duplicate layer name: {self.prefix}")
        static_forward_context[self.prefix] = self
        # bound by the engine: (conv, inner FIR, LI) native-layout slices
        self.kv_cache = (torch.tensor([]), torch.tensor([]))

    def forward(self, hidden_states, token_ids=None):
        output = torch.empty_like(hidden_states)
        torch.ops.vllm.evo2_hyena_mixer(hidden_states, output, token_ids, self.prefix)
        return output

    def _meta(self):
        raw = get_forward_context().attn_metadata
        if raw is None:
            return None
        return raw[self.prefix] if isinstance(raw, dict) else raw

    def _conv_state(self, i, width=None):
        """Dim-first view of state slice i (mixers.py:940-949): slices 0 and 1
        are stored state-major (blocks, K-1, dim) and viewed (blocks, dim, K-1)."""
        v = self.kv_cache[i].transpose(-1, -2)
        return v if width is None else v[..., :width]

    def _ssm_state(self):
        """Slice 2, (blocks, H, S) fp32, not transposed (mixers.py:1334-1342)."""
        return self.kv_cache[2]

    def _short_w(self):
        return self.short_filter.view(3 * self.hidden, self.k_short)

    def _project(self, hidden_states, token_ids=None):
        """in_proj, or for a token-table layer the table rows of the step's
        tokens (mixers.py:1076-1092)."""
        if self.in_proj_token_table is not None:
            if token_ids is None:
                raise ValueError(f"{self.prefix}: token-table projection needs input_ids "
                                 "(inputs_embeds are unsupported for FP8-surgery checkpoints)")
            z, _ = self.in_proj(self.in_proj_token_table[token_ids[: hidden_states.shape[0]]])
            return z
        emul_w = getattr(self, "in_proj_emul_weight_t", None)
        if isinstance(self.in_proj, ProjectionTap):  # fully emulated layer
            sc = self.in_proj_emul_scales
            z, _ = self.in_proj(static_fp8_linear_emulated(hidden_states, emul_w, sc[0], sc[1]))
            return z
        z, _ = self.in_proj(hidden_states)
        if emul_w is not None:  # hybrid: emulated channels over the bf16 ones
            sc = self.in_proj_emul_scales
            z = z.index_copy(-1, self.in_proj_emul_cols,
                             static_fp8_linear_emulated(hidden_states, emul_w, sc[0], sc[1]))
        return z

    @staticmethod
    def is_speculative_decode(m):
        """Whether the decode half of a step carries speculative snapshots
        (mixers.py:930-937): a slot matrix with more than one column, an
        accepted-token count, or a decode token count that differs from the
        number of decode requests.  A speculative-capable runner keeps the
        slot matrix even on an ordinary one-token step, which is therefore
        speculative too: the previous verify step may have accepted several
        tokens."""
        idx = m.state_indices_tensor_d
        return ((idx is not None and idx.dim() > 1 and idx.shape[1] > 1)
                or getattr(m, "num_accepted_tokens", None) is not None
                or int(m.num_decode_tokens) != int(m.num_decodes))

    def _check_meta(self, m):
        if len(self.kv_cache) != 3:
            raise RuntimeError(f"{self.prefix}: kv_cache is not bound (the engine binds the "
                               "layer's three state slices before a step)")
        if int(m.num_decodes) and self.is_speculative_decode(m):
            raise NotImplementedError(
                f"{self.prefix}: speculative decode metadata (a multi-column "
                "state_indices_tensor_d, num_accepted_tokens, or num_decode_tokens != "
                "num_decodes) is not supported by these mixers")

    @staticmethod
    def _unpad(out, hidden_states, n_actual):
        """Rows past the real ones (graph padding) are zero (mixers.py:1214-1228)."""
        if out.shape[0] == hidden_states.shape[0]:
            return out
        full = torch.zeros_like(hidden_states)
        full[:n_actual] = out
        return full

    def _profile_run(self, hidden_states, token_ids=None):
        z = self._project(hidden_states, token_ids)
        y = z[:, 0::3] * z[:, 1::3] * z[:, 2::3]
        out, _ = self.out_proj(y)
        return out

    def _finish(self, parts, hidden_states, n):
        g = torch.cat(parts, dim=0) if len(parts) > 1 else parts[0]
        out, _ = self.out_proj(g)
        return self._unpad(out, hidden_states, n)


class HyenaFIRMixer(HyenaMixerBase):
    """Hyena-SE (K=7) and Hyena-MR (K=128): explicit depthwise causal FIR
    (mixers.py:1238-1305).  `conv` (H, 1, K) in cross-correlation order; `D`
    only for K >= 128."""

    def __init__(self, config, layer_idx, model_config=None, cache_config=None, prefix="",
                 k_inner=None, quant_config=None, device=None):
        super().__init__(config, layer_idx, model_config, cache_config, prefix, quant_config,
                         device)
        h = config.hidden_size
        self.k_inner = k_inner or config.inner_filter_length(layer_idx)
        self.conv = nn.Parameter(torch.empty(h, 1, self.k_inner, device=device,
                                             dtype=torch.bfloat16), requires_grad=False)
        self.has_D = self.k_inner >= 128
        self.D = (nn.Parameter(torch.empty(h, device=device, dtype=torch.bfloat16),
                               requires_grad=False) if self.has_D else None)
        self._decode_taps = None
        # The engine's loader calls `param.weight_loader(param, tensor)` when a
        # parameter has one (model.py:374-377); loading `conv` through it also
        # refreshes the decode copy of the taps.
        self.conv.weight_loader = self._load_conv

    def _load_conv(self, param, loaded_weight):
        param.data.copy_(loaded_weight.to(param.dtype).view_as(param))
        if self._decode_taps is not None:
            self.process_weights_after_loading()

    def process_weights_after_loading(self):
        """Keep a channel-contiguous copy of the taps for the decode kernel,
        rewritten in place on a reload, so a HIP graph captured before it
        still reads the current taps.  `conv`'s weight_loader calls this on
        every load; code that writes `conv` by other means calls it after."""
        taps = channel_major_taps(self.conv.detach().view(self.hidden, self.k_inner))
        old = self._decode_taps
        if (old is not None and old.shape == taps.shape and old.stride() == taps.stride()
                and old.device == taps.device):
            old.copy_(taps)
        else:
            self._decode_taps = taps

    def _forward_impl(self, hidden_states, token_ids=None):
        m = self._meta()
        if m is None:
            return self._profile_run(hidden_states, token_ids)
        self._check_meta(m)
        if self._decode_taps is None or self._decode_taps.device != self.conv.device:
            self.process_weights_after_loading()
        nd, npt = int(m.num_decode_tokens), int(m.num_prefill_tokens)
        z = self._project(hidden_states[:nd + npt], token_ids)
        sw = self._short_w()
        conv_state = self._conv_state(0)
        inner_state = self._conv_state(1, self.k_inner - 1)
        parts = []
        if nd:
            parts.append(hyena_decode(z[:nd], sw, conv_state, decode_state_indices(m),
                                      self._decode_taps, inner_state, self.D))
        if npt:
            bt = fir_prefill_block_t(self.k_inner, npt, self.hidden)
            seq_t, til_t, _ = prefill_tables(m, bt, z.device)
            parts.append(hyena_fir_prefill(
                z[nd:nd + npt], sw, conv_state, self.conv.view(self.hidden, self.k_inner),
                inner_state, self.D, seq_t, m.state_indices_tensor_p, til_t, bt))
        return self._finish(parts, hidden_states, nd + npt)


class HyenaIIRMixer(HyenaMixerBase):
    """Hyena-LI: diagonal LTI SSM s_t = p*s_{t-1} + x_t over S real poles
    (mixers.py:1308-1401).  `log_poles` (H, S, 1) and `residues` (H, S) fp32."""

    def __init__(self, config, layer_idx, model_config=None, cache_config=None, prefix="",
                 quant_config=None, device=None):
        super().__init__(config, layer_idx, model_config, cache_config, prefix, quant_config,
                         device)
        h, s = config.hidden_size, config.state_size
        self.state_size = s
        self.log_poles = nn.Parameter(torch.empty(h, s, 1, device=device, dtype=torch.float32),
                                      requires_grad=False)
        self.residues = nn.Parameter(torch.empty(h, s, device=device, dtype=torch.float32),
                                     requires_grad=False)
        self.D = nn.Parameter(torch.empty(h, device=device, dtype=torch.bfloat16),
                              requires_grad=False)

    def process_weights_after_loading(self):
        pass

    def _forward_impl(self, hidden_states, token_ids=None):
        m = self._meta()
        if m is None:
            return self._profile_run(hidden_states, token_ids)
        self._check_meta(m)
        nd, npt = int(m.num_decode_tokens), int(m.num_prefill_tokens)
        z = self._project(hidden_states[:nd + npt], token_ids)
        sw = self._short_w()
        conv_state = self._conv_state(0)
        ssm = self._ssm_state()
        lp = self.log_poles[..., 0]
        res = self.residues
        parts = []
        if nd:
            parts.append(hyena_decode(z[:nd], sw, conv_state, decode_state_indices(m), res, ssm,
                                      self.D, log_poles=lp))
        if npt:
            bt = hcl_block_t(npt, self.hidden)
            seq_t, til_t, ts_t = prefill_tables(m, bt, z.device)
            parts.append(hyena_hcl_prefill(z[nd:nd + npt], sw, conv_state, res, lp, ssm, self.D,
                                           seq_t, m.state_indices_tensor_p, til_t, ts_t, bt))
        return self._finish(parts, hidden_states, nd + npt)


# ---------------------------------------------------------------- operator
HYENA_MIXER_OP = "vllm::evo2_hyena_mixer"


def evo2_hyena_mixer(hidden_states: torch.Tensor, output: torch.Tensor,
                     token_ids: Optional[torch.Tensor], layer_name: str) -> None:
    """The mixer as one opaque operator that writes `output` in place
    (mixers.py:1404-1410)."""
    layer = static_forward_context[layer_name]
    output.copy_(layer._forward_impl(hidden_states, token_ids))


def evo2_hyena_mixer_fake(hidden_states: torch.Tensor, output: torch.Tensor,
                          token_ids: Optional[torch.Tensor], layer_name: str) -> None:
    """Shape propagation for tracing: the operator only mutates `output`
    (mixers.py:1413-1415)."""
    return None


def _register_op():
    """Register `vllm::evo2_hyena_mixer` with `output` as its one mutated
    argument (mixers.py:1418-1423).  Registration is once per process; a
    second import of this module finds the operator already there."""
    try:
        return getattr(torch.ops.vllm, "evo2_hyena_mixer")
    except (AttributeError, RuntimeError):
        pass
    op = torch.library.custom_op(HYENA_MIXER_OP, evo2_hyena_mixer, mutates_args=("output",))
    op.register_fake(evo2_hyena_mixer_fake)
    return op


_register_op()


def make_mixer(config, layer_idx, prefix="", quant_config=None, device=None):
    """The mixer of a Hyena layer, as Evo2DecoderLayer builds it (model.py:163-182)."""
    kind = config.layer_kind(layer_idx)
    if kind == "hcl":
        return HyenaIIRMixer(config, layer_idx, prefix=prefix, quant_config=quant_config,
                             device=device)
    if kind in ("hcs", "hcm"):
        return HyenaFIRMixer(config, layer_idx, prefix=prefix,
                             k_inner=config.inner_filter_length(layer_idx),
                             quant_config=quant_config, device=device)
    raise ValueError(f"layer {layer_idx} is an attention layer")


def load_mixer_params(mixer, params):
    """Copy a {name: tensor} dict with checkpoint keys into a mixer (the
    subset of load_weights, model.py:362-379, a mixer owns) and prepare the
    decode layouts."""
    own = dict(mixer.named_parameters())
    for name, t in params.items():
        if name not in own:
            raise KeyError(f"{mixer.prefix}: unexpected parameter {name}")
        p = own[name]
        loader = getattr(p, "weight_loader", None)
        if loader is not None:
            loader(p, t)
        else:
            p.data.copy_(t.to(p.dtype).view_as(p))
    mixer.process_weights_after_loading()
    return mixer
