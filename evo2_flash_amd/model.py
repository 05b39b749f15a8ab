"""Evo 2 (StripedHyena2) decoder around this build's Hyena mixers, for
end-to-end decode (the reference's model.py:47-200, restated).

    x = embed(token)
    for each layer:  pre = RMSNorm(x)
                     m   = mixer(pre)            Hyena (hcs / hcm / hcl) or attention
                     post, x = RMSNorm(m + x), m + x
                     x   = MLP(post) + x          gated: l3(act(l1 post) * l2 post),
                                                  GELU on layer 0 only (model.py:77-101, 184)
    logits = RMSNorm(x) @ embed^T                 tied head (model.py:343-348)

The Hyena layers are this build's: RMSNorm kernel, fp8 in_proj on MFMA, the
fused decode step over the paged state pool, out_proj.  The attention layer
keeps a contiguous KV cache per layer (keys head_dim-major, values
position-major) rather than vLLM's paged cache, applies neox-style rotary
with the config's base and linear scaling (model.py:104-153), and attends
with this build's split-context decode attention kernel (attention.py),
which reads each cache once and masks positions past each sequence's; a
decode step has fixed shapes and captures into one HIP graph.  The
projections and MLPs are plain torch on ROCm (outside the mixer hot path).

Weights are random, seeded, in the benchmark's distributions; the Hyena
state pools and the KV cache are filled with random values that stand in for
a prefilled prompt.
"""

import torch
from torch import nn

from .attention import decode_attention, workspace as attention_workspace
from .metadata import build_metadata
from .mixers import Linear, load_mixer_params, make_mixer, set_forward_context
from .norm import Evo2RMSNorm
from .state import HyenaStatePool
from .synthetic import mixer_params


class Evo2MLP(nn.Module):
    """l3(act(l1 x) * l2 x), act = GELU on layer 0 only (model.py:77-101)."""

    def __init__(self, hidden, inter, use_act, device=None):
        super().__init__()
        self.l1 = Linear(hidden, inter, device=device)
        self.l2 = Linear(hidden, inter, device=device)
        self.l3 = Linear(inter, hidden, device=device)
        self.use_act = use_act

    def forward(self, x):
        z1, _ = self.l1(x)
        z2, _ = self.l2(x)
        if self.use_act:
            z1 = nn.functional.gelu(z1)
        out, _ = self.l3(z1 * z2)
        return out


def rotary_neox(x, positions, inv_freq, factor):
    """Neox rotary on (B, heads, head_dim): the two halves of each head rotate
    by angle (position / factor) * inv_freq (linear position scaling)."""
    ang = (positions.float() / factor)[:, None] * inv_freq[None, :]     # (B, hd/2)
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
    xf = x.float()
    half = xf.shape[-1] // 2
    x1, x2 = xf[..., :half], xf[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


class Evo2Attention(nn.Module):
    """Decode-time attention: qkv_proj, rotary, KV append, softmax attention
    over the cache, o_proj with bias (model.py:104-153)."""

    def __init__(self, config, max_batch, max_ctx, rope_theta=10000.0, rope_factor=1.0,
                 device=None):
        super().__init__()
        h = config.hidden_size
        self.heads = config.num_attention_heads
        self.hd = h // self.heads
        self.qkv_proj = Linear(h, 3 * h, device=device)
        self.o_proj = Linear(h, h, bias=True, device=device)
        self.rope_factor = float(rope_factor)
        self.register_buffer("inv_freq", 1.0 / rope_theta ** (
            torch.arange(0, self.hd, 2, device=device, dtype=torch.float32) / self.hd))
        # keys head_dim-major (B, nh, hd, L), values (B, nh, L, hd): both
        # products of a decode step then take a contiguous right operand,
        # (1 x hd)(hd x L) for the scores and (1 x L)(L x hd) for the output
        self.k_cache = torch.zeros(max_batch, self.heads, self.hd, max_ctx, dtype=torch.bfloat16,
                                   device=device)
        self.v_cache = torch.zeros(max_batch, self.heads, max_ctx, self.hd, dtype=torch.bfloat16,
                                   device=device)
        self._attn_ws = attention_workspace(max_batch, self.heads, self.hd, max_ctx, device)

    def forward_decode(self, x, positions):
        B = x.shape[0]
        qkv, _ = self.qkv_proj(x)
        q, k, v = qkv.view(B, 3, self.heads, self.hd).unbind(1)
        q = rotary_neox(q, positions, self.inv_freq, self.rope_factor)
        k = rotary_neox(k, positions, self.inv_freq, self.rope_factor)
        rows = torch.arange(B, device=x.device)
        self.k_cache[rows, :, :, positions] = k
        self.v_cache[rows, :, positions] = v.contiguous()
        out = decode_attention(q.contiguous(), self.k_cache[:B], self.v_cache[:B], positions,
                               self.hd ** -0.5, self._attn_ws)            # (B, nh, hd)
        o, _ = self.o_proj(out.reshape(B, self.heads * self.hd))
        return o


class Evo2DecoderLayer(nn.Module):
    """pre_norm -> mixer -> post_norm (+ residual) -> MLP (+ residual)
    (model.py:156-200)."""

    def __init__(self, config, i, mixer, device=None):
        super().__init__()
        h = config.hidden_size
        self.kind = config.layer_kind(i)
        self.pre_norm = Evo2RMSNorm(h, config.rms_norm_eps, device=device)
        self.post_norm = Evo2RMSNorm(h, config.rms_norm_eps, device=device)
        self.mixer = mixer
        self.mlp = Evo2MLP(h, config.intermediate_size, use_act=(i == 0), device=device)

    def forward(self, positions, x, token_ids):
        pre = self.pre_norm(x)
        if self.kind == "attn":
            m = self.mixer.forward_decode(pre, positions)
        else:
            m = self.mixer(pre, token_ids=token_ids)
        post, x = self.post_norm(m, x)
        return self.mlp(post) + x


class Evo2DecodeModel(nn.Module):
    """The whole model at decode for `max_batch` sequences with up to
    `max_ctx` positions each.  Each sequence b owns Hyena state block
    `slots[b]` in every Hyena layer's pool (block 0 is the null block)."""

    def __init__(self, config, max_batch, max_ctx, device, rope_theta=10000.0, rope_factor=1.0,
                 name="evo2"):
        super().__init__()
        self.config = config
        h = config.hidden_size
        self.embed = nn.Parameter(torch.empty(config.vocab_size, h, dtype=torch.bfloat16,
                                              device=device), requires_grad=False)
        layers, self.pools = [], {}
        for i in range(config.num_hidden_layers):
            if config.layer_kind(i) == "attn":
                mixer = Evo2Attention(config, max_batch, max_ctx, rope_theta, rope_factor, device)
            else:
                mixer = make_mixer(config, i, prefix=f"{name}.layers.{i}.mixer", device=device)
                pool = HyenaStatePool(max_batch + 1, h, device)
                mixer.kv_cache = pool.kv_cache
                self.pools[i] = pool
            layers.append(Evo2DecoderLayer(config, i, mixer, device))
        self.layers = nn.ModuleList(layers)
        self.norm = Evo2RMSNorm(h, config.rms_norm_eps, device=device)
        self.max_batch = max_batch
        self.slots = torch.arange(1, max_batch + 1, dtype=torch.int32, device=device)

    def init_random(self, seed, state_scale=1.0, kv_scale=1.0):
        """Seeded random weights (projections N(0, 0.02), norms 1, embedding
        N(0, 1), Hyena parameters as `synthetic.mixer_params`) and random
        Hyena states and KV entries standing in for a prefilled prompt."""
        dev = self.embed.device
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.embed.data.copy_(torch.randn(self.embed.shape, generator=g, device=dev))
        for i, layer in enumerate(self.layers):
            for mod in (layer.mlp.l1, layer.mlp.l2, layer.mlp.l3):
                mod.weight.data.copy_(torch.randn(mod.weight.shape, generator=g, device=dev) * 0.02)
            if layer.kind == "attn":
                a = layer.mixer
                for mod in (a.qkv_proj, a.o_proj):
                    mod.weight.data.copy_(torch.randn(mod.weight.shape, generator=g, device=dev) * 0.02)
                a.o_proj.bias.data.copy_(torch.randn(a.o_proj.bias.shape, generator=g, device=dev) * 0.02)
                a.k_cache.copy_(torch.randn(a.k_cache.shape, generator=g, device=dev) * kv_scale)
                a.v_cache.copy_(torch.randn(a.v_cache.shape, generator=g, device=dev) * kv_scale)
            else:
                prm = mixer_params(layer.kind, self.config.hidden_size, seed + 1000 + i, device=dev,
                                   in_proj_fp8=self.config.use_fp8_input_projections)
                load_mixer_params(layer.mixer, prm)
                pool = self.pools[i]
                pool.raw.zero_()
                pool.kv_cache[0].copy_(torch.randn(pool.kv_cache[0].shape, generator=g,
                                                   device=dev) * state_scale)
                pool.kv_cache[1].copy_(torch.randn(pool.kv_cache[1].shape, generator=g,
                                                   device=dev).to(torch.bfloat16).float()
                                       * state_scale)
                pool.kv_cache[2].copy_(torch.randn(pool.kv_cache[2].shape, generator=g,
                                                   device=dev) * state_scale)
        return self

    def decode_step(self, tokens, positions):
        """One token for each of the first B = len(tokens) sequences at the
        given positions: returns logits (B, vocab) and advances every layer's
        state (Hyena state blocks, KV cache)."""
        B = tokens.shape[0]
        m = getattr(self, "_meta", None)
        if m is None or m.num_decodes != B:
            m = self._meta = build_metadata(decode_slots=self.slots[:B].tolist(),
                                            device=tokens.device)
        x = self.embed[tokens]
        with set_forward_context(m):
            for layer in self.layers:
                x = layer(positions, x, tokens)
        h = self.norm(x)
        return torch.nn.functional.linear(h, self.embed)

    def hyena_params(self, i):
        """{parameter name: tensor} of Hyena layer i (checkpoint names)."""
        return {k: v for k, v in self.layers[i].mixer.named_parameters()}


def decode_flops_bytes(config, B, ctx):
    """Weight and KV bytes one decode step reads (for reporting): projections
    and MLPs once, the KV cache of every attention layer at `ctx` positions."""
    h, f = config.hidden_size, config.intermediate_size
    n_attn = len(config.attn_layer_idxs)
    n_hy = config.num_hidden_layers - n_attn
    w = config.num_hidden_layers * 3 * h * f * 2 + n_attn * 4 * h * h * 2
    w += n_hy * (3 * h * h * (1 if config.use_fp8_input_projections else 2) + h * h * 2)
    kv = n_attn * B * ctx * 2 * h * 2
    return w, kv


__all__ = ["Evo2MLP", "Evo2Attention", "Evo2DecoderLayer", "Evo2DecodeModel", "rotary_neox",
           "decode_flops_bytes"]
