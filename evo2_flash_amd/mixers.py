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
no CPU path: the kernels run on ROCm devices.

Speculative decode (`num_spec` > 0 draft tokens, mixers.py:17-35, 952-1074):
a step whose metadata is speculative by the reference's predicate
(mixers.py:930-937) runs its decode rows as

  decode rows   in_proj -> causal_conv1d_update (speculative form: the
                widened window in column 0 of each request's slot row) ->
                u = x1*v -> fir_snapshots | iir_snapshots (one snapshot per
                verifier position) -> [+ D*u] -> x2*y -> out_proj

with the live snapshot of each request resolved from the position stamps in
slice 2 before any state is written, and every snapshot written in the step
stamped afterwards.  The state pool then carries the speculative layout
(`state.unified_state_shape(..., num_spec)`); prefill rows and ordinary
decode rows use the leading K_short-1 columns of the widened window.
"""

import os
from typing import Optional

import torch
from torch import nn

from . import engine
from .decode import channel_major_taps, hyena_decode
from .fp8 import Fp8StaticLinear
from .fp8_emul import static_fp8_linear_emulated
from .hcl import hcl_block_t, hyena_hcl_prefill
from .metadata import decode_state_indices, longest_prefill_segment, prefill_tables
from .prefill import fir_prefill_block_t, hyena_fir_prefill
from .short_conv import PAD_SLOT_ID, causal_conv1d_update
from .speculative import (packed_rows, pool_holds, record_stamps, repair_prefill_states,
                          slot_matrix, spec_accepted, verify_plan)
from .state import unified_state_dtype, unified_state_shape
from .verify import fir_snapshots, iir_snapshots

# Test-only cross-check (mixers.py:77, 989-998): where the engine does send
# acceptance counts, they must agree with the stamps.
_CHECK_VLLM_COUNTS = os.environ.get("EVO2_CHECK_VLLM_COUNTS") == "1"

# ---------------------------------------------------------------- forward context
# The engine binding (vLLM's forward context when vLLM imports, a local one
# otherwise) lives in engine.py; these names are re-exported for callers.
static_forward_context = engine.static_forward_context
get_forward_context = engine.get_forward_context
set_forward_context = engine.set_forward_context
ForwardContext = engine.ForwardContext


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

    def forward(self, x, out=None):
        """x (..., in) -> ((..., out), None); a 2-D x may write its result into
        `out` (the same GEMM F.linear runs: addmm with the bias)."""
        if out is None:
            return torch.nn.functional.linear(x, self.weight, self.bias), None
        if self.bias is not None:
            torch.addmm(self.bias, x, self.weight.t(), out=out)
        else:
            torch.mm(x, self.weight.t(), out=out)
        return out, None


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
                 quant_config=None, device=None, num_spec=0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.prefix = prefix or f"model.layers.{layer_idx}.mixer"
        h = config.hidden_size
        self.hidden = h
        self.k_short = config.short_filter_length
        # draft tokens per verify step: the engine's speculative config
        # (num_speculative_tokens, mixers.py:733-736), 0 without speculation
        self.num_spec = int(num_spec or 0)
        self._stamp_faults = None
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
        # the engine's static_forward_context and splitting_ops (mixers.py:806-820)
        engine.register_layer(self.prefix, self)
        # bound by the engine: (conv, inner FIR, LI) native-layout slices
        self.kv_cache = (torch.tensor([]), torch.tensor([]))

    def forward(self, hidden_states, token_ids=None):
        output = torch.empty_like(hidden_states)
        torch.ops.vllm.evo2_hyena_mixer(hidden_states, output, token_ids,
                                        engine.layer_name(self.prefix))
        return output

    def process_weights_after_loading(self):
        """Make the decode copies of the fp8 projections after loading, before
        an engine sizes its memory pools from what is free."""
        for proj in (self.in_proj, self.out_proj):
            if isinstance(proj, Fp8StaticLinear):
                proj.process_weights_after_loading()

    def _meta(self):
        """This layer's metadata from the forward context (mixers.py:852-856)."""
        return engine.step_metadata(self.prefix)

    def _conv_state(self, i, width=None):
        """Dim-first view of state slice i (mixers.py:940-949): slices 0 and 1
        are stored state-major (blocks, K-1, dim) and viewed (blocks, dim, K-1)."""
        v = self.kv_cache[i].transpose(-1, -2)
        return v if width is None else v[..., :width]

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

    def get_state_shape(self):
        """The one state spec every Hyena layer declares (mixers.py:892-913)."""
        cfg = self.config
        return unified_state_shape(cfg.hidden_size, cfg.short_filter_length,
                                   cfg.hcm_filter_length, cfg.state_size, self.num_spec)

    def get_state_dtype(self):
        return unified_state_dtype(self.short_filter.dtype)

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

    # ---- speculative rollback from position stamps (mixers.py:952-1074)
    def _position_stamps(self):
        """(blocks,) fp32 view of slice 2 row 0, last column: the tokens each
        block's snapshot represents (exact below 2**24)."""
        return self.kv_cache[2][:, 0, -1]

    def _fault_counter(self, device):
        if self._stamp_faults is None or self._stamp_faults.device != torch.device(device):
            self._stamp_faults = torch.zeros((), dtype=torch.int64, device=device)
        return self._stamp_faults

    def stamp_faults(self):
        """Decode requests so far whose stamps did not match their computed
        token count (or, with EVO2_CHECK_VLLM_COUNTS=1, the engine's counts);
        reading it synchronises.  The reference asserts on the device here
        (mixers.py:985-998); such a request is clamped to the nearest valid
        offset as there."""
        return 0 if self._stamp_faults is None else int(self._stamp_faults)

    def _verify_plan(self, m):
        """The step's verify plan (slot windows of 1 + num_spec positions,
        row ranges, the engine's counts), shared by the step's layers."""
        return verify_plan(m, int(m.num_decodes), 1 + self.num_spec, self.kv_cache[2].shape[0])

    def _spec_accepted(self, m):
        """Accepted count of the previous step per decode request, from the
        position stamps in one launch (mixers.py:960-999): the live snapshot
        sits at offset computed - stamp(column 0), accepted = offset + 1,
        clamped to [1, 1 + num_spec]; out-of-range offsets off the null block
        count as stamp faults."""
        n = int(m.num_decodes)
        done = getattr(m, "num_computed_tokens_d", None)
        if done is None:
            raise RuntimeError(f"{self.prefix}: a speculative step needs the computed-token "
                               "counts (num_computed_tokens_d), which "
                               "metadata.HyenaMamba2MetadataBuilder adds to the metadata")
        rows = slot_matrix(m, n)[:n]
        first = rows if pool_holds(rows.numel(), self.kv_cache[2].shape[0]) else None
        check = None
        if _CHECK_VLLM_COUNTS and getattr(m, "num_accepted_tokens", None) is not None:
            check = self._verify_plan(m).engine_accepted
        return spec_accepted(self._position_stamps(), first, done[:n], self.num_spec,
                             self._fault_counter(done.device), check)

    def _repair_resumed_prefill_state(self, m):
        """Align-mode prefix caching: resumed prefill rows whose block is not
        stamped with their computed count take the state of the block of
        their last computed token (mixers.py:1001-1040), in two launches."""
        if self.num_spec and int(m.num_prefills):
            repair_prefill_states(self.kv_cache, self._position_stamps(), m,
                                  self._fault_counter(self.kv_cache[2].device))

    def _resolve_accepted(self, m):
        """Stamp-derived accepted counts of a speculative step's decode rows,
        resolved before the layer writes any state (mixers.py:1039-1047); None
        for any other step."""
        speculative = self.num_spec > 0 and int(m.num_decodes) > 0 and self.is_speculative_decode(m)
        return self._spec_accepted(m) if speculative else None

    def _record_stamps(self, m):
        """Stamp every snapshot this step wrote, one launch: decode column p
        of a request that had computed n tokens holds n + p + 1, a prefill
        block its sequence length (mixers.py:1049-1074)."""
        if not self.num_spec:
            return
        stamps = self._position_stamps()
        nd, npf = int(m.num_decodes), int(m.num_prefills)
        slots = qsl = computed = out_col = None
        width = 0
        if nd and self.is_speculative_decode(m):
            slots = m.state_indices_tensor_d[:nd]
            if slots.dim() == 1:
                slots = slots[:, None]
            qsl = packed_rows(m, nd, stamps.device)
            computed = m.num_computed_tokens_d[:nd]
            # the written columns: prefix caching's window from the block of
            # the last scheduled token, else the slot row (mixers.py:444-456)
            width = slots.shape[1]
            if (getattr(m, "block_idx_last_scheduled_token_prev_step", None) is not None
                    and getattr(m, "block_idx_last_scheduled_token", None) is not None):
                width = min(width, 1 + self.num_spec)
                out_col = m.block_idx_last_scheduled_token[:nd]
            if self.kv_cache[2].shape[0] < nd * width:
                slots = None   # every request on the null block (mixers.py:527-541)
        if not npf and qsl is None:
            return
        record_stamps(stamps, slots, qsl, computed, width, out_col,
                      m.state_indices_tensor_p[:npf] if npf else None,
                      m.seq_lens[nd:nd + npf] if npf else None)

    def _spec_short_conv(self, z_d, m, accepted):
        """(x2, x1, v) of the decode rows of a speculative step through the
        widened short window (mixers.py:1153-1193)."""
        window = self._conv_state(0)
        n = int(m.num_decodes)
        engine_rows = m.state_indices_tensor_d
        rows = slot_matrix(m, n)
        if engine_rows.dim() == 2 and not pool_holds(engine_rows.numel(), window.shape[0]):
            rows = torch.zeros_like(rows)  # profiling-sized pool: the null block
        sched = getattr(m, "block_idx_last_scheduled_token", None)
        comp = getattr(m, "block_idx_last_computed_token", None)
        if accepted is None:
            accepted = self._verify_plan(m).engine_accepted
        zf = causal_conv1d_update(
            z_d, window, self._short_w(), None, activation=None,
            conv_state_indices=rows[:n],
            block_idx_last_scheduled_token=None if sched is None else sched[:n],
            initial_state_idx=None if comp is None else comp[:n],
            num_accepted_tokens=accepted, query_start_loc=packed_rows(m, n, z_d.device),
            max_query_len=rows.shape[1], pad_slot_id=PAD_SLOT_ID)
        return zf[:, 0::3], zf[:, 1::3], zf[:, 2::3]

    def _spec_tensors(self, m, num_tokens, state, accepted):
        """(ins, outs, starts, ends, accepted) for the inner operator's
        snapshots (mixers.py:578-598); `accepted` is the stamp-derived count,
        or the engine's when there is none."""
        plan = self._verify_plan(m)
        if state.shape[0] != self.kv_cache[2].shape[0]:
            raise ValueError(f"{self.prefix}: state slices of different pool sizes")
        acc = plan.engine_accepted if accepted is None else accepted[:int(m.num_decodes)]
        return plan.ins, plan.outs, plan.starts, plan.ends, acc

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

    def _finish(self, parts, hidden_states, n, output=None):
        """out_proj of the step's rows.  With `output` (the operator's buffer,
        contiguous, hidden_states' shape and dtype) the projection writes its
        rows there directly and the padding rows are zeroed, with no copy."""
        g = torch.cat(parts, dim=0) if len(parts) > 1 else parts[0]
        if (output is not None and output.dim() == 2 and output.shape == hidden_states.shape
                and output.dtype == hidden_states.dtype and output.is_contiguous()):
            self.out_proj(g, out=output[:n])
            if n < output.shape[0]:
                output[n:].zero_()
            return output
        out, _ = self.out_proj(g)
        return self._unpad(out, hidden_states, n)


class HyenaFIRMixer(HyenaMixerBase):
    """Hyena-SE (K=7) and Hyena-MR (K=128): explicit depthwise causal FIR
    (mixers.py:1238-1305).  `conv` (H, 1, K) in cross-correlation order; `D`
    only for K >= 128."""

    def __init__(self, config, layer_idx, model_config=None, cache_config=None, prefix="",
                 k_inner=None, quant_config=None, device=None, num_spec=0):
        super().__init__(config, layer_idx, model_config, cache_config, prefix, quant_config,
                         device, num_spec)
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
        super().process_weights_after_loading()
        taps = channel_major_taps(self.conv.detach().view(self.hidden, self.k_inner))
        old = self._decode_taps
        if (old is not None and old.shape == taps.shape and old.stride() == taps.stride()
                and old.device == taps.device):
            old.copy_(taps)
        else:
            self._decode_taps = taps

    def _spec_decode(self, z_d, m, accepted, inner_state):
        """g = x2 * (FIR(u) [+ D*u]) for the decode rows of a speculative step,
        one inner snapshot per verifier position (mixers.py:1264-1275, 1286-1298)."""
        x2, x1, v = self._spec_short_conv(z_d, m, accepted)
        u = x1 * v
        w = self.conv.view(self.hidden, self.k_inner)
        y = fir_snapshots(u, w, inner_state,
                          self._spec_tensors(m, u.shape[0], inner_state, accepted))
        if self.has_D:
            y = y + self.D.to(y.dtype) * u
        return x2 * y

    def _forward_impl(self, hidden_states, token_ids=None, output=None):
        m = self._meta()
        if m is None:
            return self._profile_run(hidden_states, token_ids)
        self._check_meta(m)
        self._repair_resumed_prefill_state(m)
        accepted = self._resolve_accepted(m)  # before any state is written
        if self._decode_taps is None or self._decode_taps.device != self.conv.device:
            self.process_weights_after_loading()
        nd, npt = int(m.num_decode_tokens), int(m.num_prefill_tokens)
        z = self._project(hidden_states[:nd + npt], token_ids)
        sw = self._short_w()
        window = self._conv_state(0, self.k_short - 1)
        inner_state = self._conv_state(1, self.k_inner - 1)
        parts = []
        if nd:
            if self.is_speculative_decode(m):
                parts.append(self._spec_decode(z[:nd], m, accepted, inner_state))
            else:
                parts.append(hyena_decode(z[:nd], sw, window, decode_state_indices(m),
                                          self._decode_taps, inner_state, self.D))
        if npt:
            bt = fir_prefill_block_t(self.k_inner, npt, self.hidden, longest_prefill_segment(m))
            seq_t, til_t, _ = prefill_tables(m, bt, z.device)
            parts.append(hyena_fir_prefill(
                z[nd:nd + npt], sw, window, self.conv.view(self.hidden, self.k_inner),
                inner_state, self.D, seq_t, m.state_indices_tensor_p, til_t, bt))
        self._record_stamps(m)
        return self._finish(parts, hidden_states, nd + npt, output)


class HyenaIIRMixer(HyenaMixerBase):
    """Hyena-LI: diagonal LTI SSM s_t = p*s_{t-1} + x_t over S real poles
    (mixers.py:1308-1401).  `log_poles` (H, S, 1) and `residues` (H, S) fp32."""

    def __init__(self, config, layer_idx, model_config=None, cache_config=None, prefix="",
                 quant_config=None, device=None, num_spec=0):
        super().__init__(config, layer_idx, model_config, cache_config, prefix, quant_config,
                         device, num_spec)
        h, s = config.hidden_size, config.state_size
        self.state_size = s
        self.log_poles = nn.Parameter(torch.empty(h, s, 1, device=device, dtype=torch.float32),
                                      requires_grad=False)
        self.residues = nn.Parameter(torch.empty(h, s, device=device, dtype=torch.float32),
                                     requires_grad=False)
        self.D = nn.Parameter(torch.empty(h, device=device, dtype=torch.bfloat16),
                              requires_grad=False)

    def _ssm_state(self):
        """Slice 2 without the speculative stamp column: (blocks, H, S) fp32,
        not transposed (mixers.py:666-678, 1334-1342)."""
        st = self.kv_cache[2]
        width = self.state_size + (1 if self.num_spec else 0)
        if st.shape[-2:] != (self.hidden, width):
            raise RuntimeError(f"{self.prefix}: temporal state cache has trailing shape "
                               f"{tuple(st.shape[-2:])}, expected {(self.hidden, width)}")
        return st[..., :self.state_size] if self.num_spec else st

    def _spec_decode(self, z_d, m, accepted, ssm, lp, res):
        """g = x2 * (LI(u) + u*D) for the decode rows of a speculative step, one
        state snapshot per verifier position (mixers.py:1366-1378, 1396)."""
        x2, x1, v = self._spec_short_conv(z_d, m, accepted)
        x1v = x1 * v
        y = iir_snapshots(x1v, torch.exp(lp), res, ssm,
                          self._spec_tensors(m, x1v.shape[0], ssm, accepted))
        return (y + x1v * self.D.to(y.dtype)) * x2

    def _forward_impl(self, hidden_states, token_ids=None, output=None):
        m = self._meta()
        if m is None:
            return self._profile_run(hidden_states, token_ids)
        self._check_meta(m)
        self._repair_resumed_prefill_state(m)
        accepted = self._resolve_accepted(m)  # before any state is written
        nd, npt = int(m.num_decode_tokens), int(m.num_prefill_tokens)
        z = self._project(hidden_states[:nd + npt], token_ids)
        sw = self._short_w()
        window = self._conv_state(0, self.k_short - 1)
        ssm = self._ssm_state()
        lp = self.log_poles[..., 0]
        res = self.residues
        parts = []
        if nd:
            if self.is_speculative_decode(m):
                parts.append(self._spec_decode(z[:nd], m, accepted, ssm, lp, res))
            else:
                parts.append(hyena_decode(z[:nd], sw, window, decode_state_indices(m), res, ssm,
                                          self.D, log_poles=lp))
        if npt:
            bt = hcl_block_t(npt, self.hidden, longest_prefill_segment(m))
            seq_t, til_t, ts_t = prefill_tables(m, bt, z.device)
            parts.append(hyena_hcl_prefill(z[nd:nd + npt], sw, window, res, lp, ssm, self.D,
                                           seq_t, m.state_indices_tensor_p, til_t, ts_t, bt))
        self._record_stamps(m)
        return self._finish(parts, hidden_states, nd + npt, output)


# ---------------------------------------------------------------- operator
HYENA_MIXER_OP = engine.HYENA_MIXER_OP


def evo2_hyena_mixer(hidden_states: torch.Tensor, output: torch.Tensor,
                     token_ids: Optional[torch.Tensor], layer_name: str) -> None:
    """The mixer as one opaque operator that writes `output` in place
    (mixers.py:1404-1410)."""
    layer = engine.lookup_layer(layer_name)
    res = layer._forward_impl(hidden_states, token_ids, output=output)
    if res is not output:
        output.copy_(res)


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


def make_mixer(config, layer_idx, prefix="", quant_config=None, device=None, num_spec=0):
    """The mixer of a Hyena layer, as Evo2DecoderLayer builds it (model.py:163-182);
    `num_spec` is the engine's speculative token count (0 without speculation)."""
    kind = config.layer_kind(layer_idx)
    if kind == "hcl":
        return HyenaIIRMixer(config, layer_idx, prefix=prefix, quant_config=quant_config,
                             device=device, num_spec=num_spec)
    if kind in ("hcs", "hcm"):
        return HyenaFIRMixer(config, layer_idx, prefix=prefix,
                             k_inner=config.inner_filter_length(layer_idx),
                             quant_config=quant_config, device=device, num_spec=num_spec)
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
