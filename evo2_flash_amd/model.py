"""Evo 2 (StripedHyena2) decoder around this build's Hyena mixers, for
end-to-end prefill and decode (the reference's model.py:47-200, restated).

    x = embed(token)
    for each layer:  pre = RMSNorm(x)
                     m   = mixer(pre)            Hyena (hcs / hcm / hcl) or attention
                     post, x = RMSNorm(m + x), m + x
                     x   = MLP(post) + x          gated: l3(act(l1 post) * l2 post),
                                                  GELU on layer 0 only (model.py:77-101, 184)
    logits = RMSNorm(x) @ embed^T                 tied head (model.py:343-348)

The Hyena layers are this build's: RMSNorm kernel, fp8 in_proj on MFMA, the
fused prefill cores and decode step over the paged state pool, out_proj.
The attention layers keep their KV cache in 16-position pages named by a
block table that is a seeded random permutation of the pages (page 0 is
never handed out), apply neox-style rotary with the config's base and
linear scaling (model.py:104-153), and attend at decode with this build's
split-context paged decode attention kernel (attention.py), which reads each
page once and masks positions past each sequence's; a decode step has fixed
shapes and captures into one HIP graph.  Prefill runs prompts through the
same layers (the Hyena mixers on their prefill kernels, writing the states
the decode steps continue from) with causal attention in torch.  The
projections and MLPs are plain torch on ROCm (outside the mixer hot path).

Weights are random, seeded, in the benchmark's distributions.
"""

import torch
from torch import nn

from .attention import (PAGE, PagedKVCache, causal_prefill_attention, check_block_table,
                        paged_decode_attention, shared_prefix_pages,
                        workspace as attention_workspace)
from .metadata import build_metadata
from .mixers import Linear, load_mixer_params, make_mixer, set_forward_context
from .norm import Evo2RMSNorm
from .state import HyenaStatePool, get_mamba_state_copy_func
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
    """qkv_proj, rotary, KV written to the layer's pages, softmax attention
    over the sequence's positions, o_proj with bias (model.py:104-153)."""

    def __init__(self, config, num_pages, max_pages, max_batch, rope_theta=10000.0,
                 rope_factor=1.0, device=None):
        super().__init__()
        h = config.hidden_size
        self.heads = config.num_attention_heads
        self.hd = h // self.heads
        self.qkv_proj = Linear(h, 3 * h, device=device)
        self.o_proj = Linear(h, h, bias=True, device=device)
        self.rope_factor = float(rope_factor)
        self.register_buffer("inv_freq", 1.0 / rope_theta ** (
            torch.arange(0, self.hd, 2, device=device, dtype=torch.float32) / self.hd))
        self.cache = PagedKVCache(num_pages, self.heads, self.hd, device)
        self.shared_pages = 0  # leading block-table entries every sequence shares
        self._attn_ws = attention_workspace(max_batch, self.heads, self.hd, max_pages * PAGE,
                                            device)

    def _qkv(self, x, positions):
        n = x.shape[0]
        qkv, _ = self.qkv_proj(x)
        q, k, v = qkv.view(n, 3, self.heads, self.hd).unbind(1)
        return (rotary_neox(q, positions, self.inv_freq, self.rope_factor),
                rotary_neox(k, positions, self.inv_freq, self.rope_factor), v)

    def forward_decode(self, x, positions, block_table):
        """x (B, H): one token per sequence at `positions` (B,)."""
        B = x.shape[0]
        q, k, v = self._qkv(x, positions)
        self.cache.append(k, v.contiguous(), block_table, positions)
        out = paged_decode_attention(q.contiguous(), self.cache.k, self.cache.v, block_table,
                                     positions, self.hd ** -0.5, self._attn_ws,
                                     shared_pages=self.shared_pages)  # (B, nh, hd)
        o, _ = self.o_proj(out.reshape(B, self.heads * self.hd))
        return o

    def forward_prefill(self, x, nseq, L, block_table):
        """x (nseq * L, H): prompts of L tokens (positions 0..L-1) of sequences
        0..nseq-1 of `block_table`, packed in order."""
        pos = torch.arange(L, device=x.device).repeat(nseq)
        q, k, v = self._qkv(x, pos)
        shape = (nseq, L, self.heads, self.hd)
        q, k, v = (t.reshape(shape).transpose(1, 2).contiguous() for t in (q, k, v))
        self.cache.write_prompt(k, v, block_table)
        out = causal_prefill_attention(q, k, v, self.hd ** -0.5)       # (nseq, nh, L, hd)
        o, _ = self.o_proj(out.transpose(1, 2).reshape(nseq * L, self.heads * self.hd))
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

    def forward(self, positions, x, token_ids, block_table):
        """One decode token per sequence."""
        pre = self.pre_norm(x)
        if self.kind == "attn":
            m = self.mixer.forward_decode(pre, positions, block_table)
        else:
            m = self.mixer(pre, token_ids=token_ids)
        post, x = self.post_norm(m, x)
        return self.mlp(post) + x

    def forward_prefill(self, x, token_ids, nseq, L, block_table):
        """Prompts of L tokens of nseq sequences, packed (nseq * L, H); the
        Hyena mixer reads the step's prefill metadata from the forward
        context."""
        pre = self.pre_norm(x)
        if self.kind == "attn":
            m = self.mixer.forward_prefill(pre, nseq, L, block_table)
        else:
            m = self.mixer(pre, token_ids=token_ids)
        post, x = self.post_norm(m, x)
        return self.mlp(post) + x


class Evo2DecodeModel(nn.Module):
    """The whole model for `max_batch` sequences with up to `max_ctx`
    positions each.  Each sequence b owns Hyena state block `slots[b]` in
    every Hyena layer's pool (block 0 is the null block) and KV pages
    `block_table[b]` in every attention layer (a seeded random permutation
    of pages 1..; page 0 is never used)."""

    @classmethod
    def get_mamba_state_copy_func(cls):
        """The state slices' prefix-caching copy rules (model.py:285-304)."""
        return get_mamba_state_copy_func()

    def __init__(self, config, max_batch, max_ctx, device, rope_theta=10000.0, rope_factor=1.0,
                 name="evo2", page_seed=0, shared_prefix=0):
        super().__init__()
        self.config = config
        h = config.hidden_size
        self.embed = nn.Parameter(torch.empty(config.vocab_size, h, dtype=torch.bfloat16,
                                              device=device), requires_grad=False)
        self.max_pages = -(-max_ctx // PAGE)
        # With a shared prefix (a multiple of 16 positions) every sequence's
        # first pages are the same ones: one prompt, prefilled once, whose KV
        # all sequences read, each then writing its own pages.
        if shared_prefix % PAGE or shared_prefix > self.max_pages * PAGE:
            raise ValueError(f"shared_prefix {shared_prefix} must be a multiple of {PAGE} "
                             f"within max_ctx")
        sp = shared_prefix // PAGE
        own = self.max_pages - sp
        num_pages = sp + max_batch * own + 1
        g = torch.Generator().manual_seed(page_seed)
        perm = torch.randperm(num_pages - 1, generator=g) + 1
        table = torch.empty(max_batch, self.max_pages, dtype=torch.int32)
        table[:, :sp] = perm[:sp].to(torch.int32)
        table[:, sp:] = perm[sp:].to(torch.int32).view(max_batch, own)
        check_block_table(table, [self.max_pages * PAGE] * max_batch, num_pages)
        # the table's shared leading pages (the shared prompt's, whole pages of
        # it when max_batch > 1), declared to the decode attention
        shared_pages = min(sp, shared_prefix_pages(table, max_batch))
        self.block_table = table.to(device)
        self.shared_prefix = shared_prefix
        layers, self.pools = [], {}
        for i in range(config.num_hidden_layers):
            if config.layer_kind(i) == "attn":
                mixer = Evo2Attention(config, num_pages, self.max_pages, max_batch, rope_theta,
                                      rope_factor, device)
                mixer.shared_pages = shared_pages
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

    def init_random(self, seed, state_scale=1.0, kv_scale=1.0, embed_scale=1.0):
        """Seeded random weights (projections N(0, 0.02), norms 1, embedding
        N(0, embed_scale^2), which sets the residual stream's magnitude;
        Hyena parameters as `synthetic.mixer_params`); the Hyena states and
        KV pages random with the given scales (0 leaves them zero, as before
        a prefill)."""
        dev = self.embed.device
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.embed.data.copy_(torch.randn(self.embed.shape, generator=g, device=dev) * embed_scale)
        for i, layer in enumerate(self.layers):
            for mod in (layer.mlp.l1, layer.mlp.l2, layer.mlp.l3):
                mod.weight.data.copy_(torch.randn(mod.weight.shape, generator=g, device=dev) * 0.02)
            if layer.kind == "attn":
                a = layer.mixer
                for mod in (a.qkv_proj, a.o_proj):
                    mod.weight.data.copy_(torch.randn(mod.weight.shape, generator=g, device=dev) * 0.02)
                a.o_proj.bias.data.copy_(torch.randn(a.o_proj.bias.shape, generator=g, device=dev) * 0.02)
                if kv_scale:
                    a.cache.k.copy_(torch.randn(a.cache.k.shape, generator=g, device=dev) * kv_scale)
                    a.cache.v.copy_(torch.randn(a.cache.v.shape, generator=g, device=dev) * kv_scale)
                else:
                    a.cache.k.zero_()
                    a.cache.v.zero_()
            else:
                prm = mixer_params(layer.kind, self.config.hidden_size, seed + 1000 + i, device=dev,
                                   in_proj_fp8=self.config.use_fp8_input_projections)
                load_mixer_params(layer.mixer, prm)
                pool = self.pools[i]
                pool.raw.zero_()
                if state_scale:
                    pool.kv_cache[0].copy_(torch.randn(pool.kv_cache[0].shape, generator=g,
                                                       device=dev) * state_scale)
                    pool.kv_cache[1].copy_(torch.randn(pool.kv_cache[1].shape, generator=g,
                                                       device=dev).to(torch.bfloat16).float()
                                           * state_scale)
                    pool.kv_cache[2].copy_(torch.randn(pool.kv_cache[2].shape, generator=g,
                                                       device=dev) * state_scale)
        return self

    def prefill(self, tokens, chunk_seqs=8):
        """Prompts tokens (B, L) of sequences 0..B-1 through every layer, in
        groups of `chunk_seqs` sequences: fresh Hyena states (the prefill
        kernels write each sequence's final state and windows into its
        blocks) and KV pages for positions 0..L-1.  Returns the logits of the
        last position (B, vocab)."""
        B, L = tokens.shape
        if B > self.max_batch or L > self.max_pages * PAGE:
            raise ValueError(f"prompts ({B}, {L}) exceed the model's {self.max_batch} sequences "
                             f"of {self.max_pages * PAGE} positions")
        last = []
        for b0 in range(0, B, chunk_seqs):
            n = min(chunk_seqs, B - b0)
            tok = tokens[b0:b0 + n].reshape(-1)
            m = build_metadata(prefill_lens=[L] * n, prefill_slots=self.slots[b0:b0 + n].tolist(),
                               has_init=[0] * n, device=tokens.device)
            x = self.embed[tok]
            with set_forward_context(m):
                for layer in self.layers:
                    x = layer.forward_prefill(x, tok, n, L, self.block_table[b0:b0 + n])
            last.append(x.view(n, L, -1)[:, -1])
        h = self.norm(torch.cat(last))
        return torch.nn.functional.linear(h, self.embed)

    def prefill_shared(self, prompt):
        """Prefill one prompt (L,) with L = shared_prefix into sequence 0 and
        hand its state to every sequence: the KV pages are shared through the
        block table, the Hyena state blocks are copied.  Returns the logits
        of the last position (1, vocab)."""
        if prompt.shape[0] != self.shared_prefix:
            raise ValueError(f"the shared prompt has {self.shared_prefix} tokens, "
                             f"got {prompt.shape[0]}")
        logits = self.prefill(prompt[None], chunk_seqs=1)
        src = int(self.slots[0])
        for pool in self.pools.values():
            pool.raw[self.slots[1:].long()] = pool.raw[src].clone()
        return logits

    def decode_step(self, tokens, positions):
        """One token for each of the first B = len(tokens) sequences at the
        given positions: returns logits (B, vocab) and advances every layer's
        state (Hyena state blocks, KV pages)."""
        B = tokens.shape[0]
        m = getattr(self, "_meta", None)
        if m is None or m.num_decodes != B:
            m = self._meta = build_metadata(decode_slots=self.slots[:B].tolist(),
                                            device=tokens.device)
        x = self.embed[tokens]
        table = self.block_table[:B]
        with set_forward_context(m):
            for layer in self.layers:
                x = layer(positions, x, tokens, table)
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


def prefill_flops(config, L):
    """Multiply-add flop of one L-token prefill of one sequence: every
    projection and MLP over L rows, and causal attention (L^2 / 2 positions
    per head, two products)."""
    h, f = config.hidden_size, config.intermediate_size
    n_attn = len(config.attn_layer_idxs)
    n_hy = config.num_hidden_layers - n_attn
    per_tok = config.num_hidden_layers * 3 * h * f + n_attn * 4 * h * h + n_hy * 4 * h * h
    return 2 * L * per_tok + n_attn * 2 * 2 * h * L * L // 2


__all__ = ["Evo2MLP", "Evo2Attention", "Evo2DecoderLayer", "Evo2DecodeModel", "rotary_neox",
           "decode_flops_bytes", "prefill_flops"]
