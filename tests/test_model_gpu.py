"""The decoder harness (model.py:47-200 restated around this build's mixers)
against a CPU composition of the same weights: the oracle for RMSNorm and the
Hyena mixer steps, plain fp32 torch for the MLP and attention, bf16 at the
same op boundaries.  A five-layer model (hcs, hcm, hcl, attention, hcs) with
the KV cache in 16-position pages of a random block table:
* three decode steps of three sequences: logits within 2e-2 and the Hyena
  state pools within the mixer tolerance after every step;
* a prefill of two prompts: last-position logits within 2e-2, Hyena states
  and the KV pages of the prompt against the composition;
* both of the above also at the 7B model's layer shape (H=4096, 32 heads,
  MLP 11264, fp8 in_proj), where the stripe prefill kernels run;
* prefill(L) followed by one decode step equals prefill(L + 1) at the last
  position (logits and states), which ties the prefill and decode paths of
  every layer kind to each other;
* the whole decode step captured once as a HIP graph replays like eager steps."""

import pytest
import torch

import oracle
from evo2_flash_amd.config import HyenaConfig
from evo2_flash_amd.model import Evo2DecodeModel, rotary_neox
from evo2_flash_amd.state import HyenaStatePool

from _cases import max_rel_err, oracle_mixer_step

pytestmark = pytest.mark.gpu
DEV = "cuda"
bf = torch.bfloat16


def _lin(x, w, b=None):
    y = x.float() @ w.float().t()
    if b is not None:
        y = y + b.float()
    return y.to(bf)


def _attn_ref(a, x, pos, kc, vc):
    """fp32 decode attention of the harness's layer a, on CPU copies of its
    cache (updated in place)."""
    B, nh, hd = x.shape[0], a.heads, a.hd
    q, k, v = _lin(x, a.qkv_proj.weight.cpu()).view(B, 3, nh, hd).unbind(1)
    inv = a.inv_freq.cpu()
    q = rotary_neox(q, pos, inv, a.rope_factor)
    k = rotary_neox(k, pos, inv, a.rope_factor)
    for b in range(B):
        kc[b, :, :, pos[b]] = k[b]          # keys (B, nh, hd, L)
        vc[b, :, pos[b]] = v[b]             # values (B, nh, L, hd)
    out = torch.empty(B, nh, hd)
    for b in range(B):
        L = int(pos[b]) + 1
        s = (q[b].float().unsqueeze(1) @ kc[b, :, :, :L].float()).squeeze(1) * hd ** -0.5
        p = torch.softmax(s, dim=-1).to(bf).float()
        out[b] = p.unsqueeze(1).matmul(vc[b, :, :L].float()).squeeze(1)
    return _lin(out.to(bf).view(B, nh * hd), a.o_proj.weight.cpu(), a.o_proj.bias.cpu())


def _cfg5(H=256):
    return HyenaConfig(hidden_size=H, num_hidden_layers=5, num_attention_heads=4,
                       intermediate_size=384, vocab_size=512, hcs_layer_idxs=[0, 4],
                       hcm_layer_idxs=[1], hcl_layer_idxs=[2], attn_layer_idxs=[3],
                       use_fp8_input_projections=True)


def _mlp_ref(layer, post):
    z1 = _lin(post, layer.mlp.l1.weight.cpu())
    z2 = _lin(post, layer.mlp.l2.weight.cpu())
    if layer.mlp.use_act:
        z1 = torch.nn.functional.gelu(z1.float()).to(bf)
    return _lin((z1.float() * z2.float()).to(bf), layer.mlp.l3.weight.cpu())


def _decode_vs_composition(cfg, B, pos0, steps, name, seed=11, win_tol=2e-2, li_tol=1e-3):
    """`steps` decode steps of B sequences from positions pos0 against the
    CPU composition: logits within 2e-2 and the Hyena state pools within the
    mixer tolerances after every step: `win_tol` for the FIR windows (the
    step's new column is u = x1 v), `li_tol` for the LI states (one step adds
    u to p s, so a bf16 step of z from the fp8 in_proj moves every pole of a
    channel by the same du)."""
    H = cfg.hidden_size
    model = Evo2DecodeModel(cfg, max_batch=B, max_ctx=32, device=DEV, rope_theta=10000.0,
                            rope_factor=4.0, name=name)
    model.init_random(seed=seed, state_scale=0.5, kv_scale=0.5)
    # CPU copies of every state the step touches
    pools = {}
    for i, p in model.pools.items():
        c = HyenaStatePool(p.num_blocks, H, "cpu")
        c.raw.copy_(p.raw.cpu())
        pools[i] = c
    caches = {i: tuple(t.cpu() for t in layer.mixer.cache.dense(model.block_table, B, 32))
              for i, layer in enumerate(model.layers) if layer.kind == "attn"}
    emb = model.embed.detach().cpu()
    g = torch.Generator().manual_seed(3)
    pos = torch.tensor(pos0)
    slots = model.slots.cpu().tolist()
    for step in range(steps):
        tok = torch.randint(0, cfg.vocab_size, (B,), generator=g)
        print(f"{name}: decode step {step}", flush=True)
        logits = model.decode_step(tok.to(DEV), pos.to(DEV)).cpu()
        x = emb[tok]
        for i, layer in enumerate(model.layers):
            pre = oracle.rms_norm(x, layer.pre_norm.weight.cpu(), cfg.rms_norm_eps)
            if layer.kind == "attn":
                m = _attn_ref(layer.mixer, pre, pos, *caches[i])
            else:
                prm = {k: v.detach().cpu() for k, v in layer.mixer.named_parameters()}
                m = oracle_mixer_step(layer.kind, prm, pre, pools[i], slots, [], [], [], H)
            post, x = oracle.rms_norm(m, layer.post_norm.weight.cpu(), cfg.rms_norm_eps,
                                      residual=x)
            x = (_mlp_ref(layer, post).float() + x.float()).to(bf)
        ref = _lin(oracle.rms_norm(x, model.norm.weight.cpu(), cfg.rms_norm_eps), emb)
        assert max_rel_err(logits, ref) <= 2e-2, step
        for i, p in model.pools.items():
            assert max_rel_err(p.kv_cache[1].cpu(), pools[i].kv_cache[1]) <= win_tol, (step, i)
            assert max_rel_err(p.kv_cache[2].cpu(), pools[i].kv_cache[2]) <= li_tol, (step, i)
        pos = pos + 1


def test_decode_steps_vs_cpu_composition():
    _decode_vs_composition(_cfg5(256), 3, [10, 4, 17], 3, "harness_test")


def test_decode_steps_7b_layer_shape():
    """The same check at the 7B model's layer shape (H=4096, 32 heads of 128,
    MLP 11264, fp8 in_proj): one layer of each Hyena kind and an attention
    layer, two decode steps of three sequences."""
    cfg = HyenaConfig(hidden_size=4096, num_hidden_layers=5, num_attention_heads=32,
                      intermediate_size=11264, vocab_size=512, hcs_layer_idxs=[0, 4],
                      hcm_layer_idxs=[1], hcl_layer_idxs=[2], attn_layer_idxs=[3],
                      use_fp8_input_projections=True)
    # K = 4096 in_proj sums move a few z entries by a bf16 step or two against
    # the CPU's fp32 products, and u = x1 v carries that into the windows' new
    # column and every pole of an LI channel; the last layer's input also
    # carries the bf16 differences of four layers and their MLPs at H=4096.
    # States within 5e-2 here (a wrong slot, layer or window column is O(1);
    # the per-kernel tests pin the mixer cores tightly), logits within 2e-2.
    _decode_vs_composition(cfg, 3, [20, 5, 12], 2, "harness_7b_shape", seed=13, win_tol=5e-2,
                           li_tol=5e-2)


def test_decode_step_graph_replays():
    """The whole decode step captured once as a HIP graph: replays advance the
    states exactly as eager steps from the same starting state."""
    H, B = 256, 2
    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=4, num_attention_heads=4,
                      intermediate_size=256, vocab_size=512, hcs_layer_idxs=[0],
                      hcm_layer_idxs=[1], hcl_layer_idxs=[2], attn_layer_idxs=[3],
                      use_fp8_input_projections=True)

    def build(name):
        m = Evo2DecodeModel(cfg, max_batch=B, max_ctx=16, device=DEV, name=name)
        return m.init_random(seed=5, state_scale=0.5, kv_scale=0.5)

    eager, graphed = build("harness_eager"), build("harness_graph")
    tok = torch.tensor([65, 84], device=DEV)
    pos = torch.tensor([3, 7], device=DEV)
    static_pos = pos.clone()
    graphed.decode_step(tok, static_pos)        # warm-up outside capture (builds metadata)
    graphed.init_random(seed=5, state_scale=0.5, kv_scale=0.5)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            out = graphed.decode_step(tok, static_pos)
            static_pos.add_(1)
    torch.cuda.current_stream().wait_stream(s)
    # capture records without running: states and positions are still the
    # freshly initialised ones; reloading the weights in place keeps the
    # graph's buffers (the decode taps are rewritten, not reallocated)
    graphed.init_random(seed=5, state_scale=0.5, kv_scale=0.5)
    static_pos.copy_(pos)
    torch.cuda.synchronize()
    print("harness graph replays", flush=True)
    for step in range(3):
        graph.replay()
        torch.cuda.synchronize()
        ref = eager.decode_step(tok, pos + step)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), step
        for i in graphed.pools:
            assert torch.equal(graphed.pools[i].raw, eager.pools[i].raw), (step, i)


def _prefill_attn_ref(a, x, nseq, L):
    """fp32 causal attention of layer a over packed prompts x (nseq * L, H);
    returns the layer output and the rotated keys and values (nseq, nh, L, hd)."""
    nh, hd = a.heads, a.hd
    pos = torch.arange(L).repeat(nseq)
    q, k, v = _lin(x, a.qkv_proj.weight.cpu()).view(nseq * L, 3, nh, hd).unbind(1)
    inv = a.inv_freq.cpu()
    q = rotary_neox(q, pos, inv, a.rope_factor)
    k = rotary_neox(k, pos, inv, a.rope_factor)
    q, k, v = (t.reshape(nseq, L, nh, hd).transpose(1, 2) for t in (q, k, v))
    s = (q.float() @ k.float().transpose(-1, -2).contiguous()) * hd ** -0.5
    s = s.masked_fill(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
    o = torch.softmax(s, dim=-1) @ v.float()
    o = o.to(bf).transpose(1, 2).reshape(nseq * L, nh * hd)
    return _lin(o, a.o_proj.weight.cpu(), a.o_proj.bias.cpu()), k, v


def _prefill_vs_composition(cfg, B, L, name, seed=12, state_tol=2e-2):
    """Fresh L-token prompts of B sequences: last-position logits, the Hyena
    states written for each sequence (within `state_tol`) and every attention
    layer's KV pages against the CPU composition."""
    H = cfg.hidden_size
    model = Evo2DecodeModel(cfg, max_batch=B + 1, max_ctx=L + 32, device=DEV, rope_theta=10000.0,
                            rope_factor=4.0, name=name, page_seed=3)
    model.init_random(seed=seed, state_scale=0.0, kv_scale=0.0)
    g = torch.Generator().manual_seed(5)
    tok = torch.tensor([65, 67, 71, 84])[torch.randint(0, 4, (B, L), generator=g)]
    print(f"{name}: prefill {B} x {L}", flush=True)
    logits = model.prefill(tok.to(DEV), chunk_seqs=2).cpu()
    emb = model.embed.detach().cpu()
    pools = {i: HyenaStatePool(p.num_blocks, H, "cpu") for i, p in model.pools.items()}
    slots = model.slots.cpu()[:B].tolist()
    x = emb[tok.reshape(-1)]
    kv_ref = {}
    for i, layer in enumerate(model.layers):
        pre = oracle.rms_norm(x, layer.pre_norm.weight.cpu(), cfg.rms_norm_eps)
        if layer.kind == "attn":
            m, k_ref, v_ref = _prefill_attn_ref(layer.mixer, pre, B, L)
            kv_ref[i] = (k_ref, v_ref)
        else:
            prm = {k: v.detach().cpu() for k, v in layer.mixer.named_parameters()}
            m = oracle_mixer_step(layer.kind, prm, pre, pools[i], [], [L] * B, slots, [0] * B, H)
        post, x = oracle.rms_norm(m, layer.post_norm.weight.cpu(), cfg.rms_norm_eps, residual=x)
        x = (_mlp_ref(layer, post).float() + x.float()).to(bf)
    last = x.view(B, L, H)[:, -1]
    ref = _lin(oracle.rms_norm(last, model.norm.weight.cpu(), cfg.rms_norm_eps), emb)
    assert max_rel_err(logits, ref) <= 2e-2
    for i, p in model.pools.items():
        assert max_rel_err(p.kv_cache[1].cpu(), pools[i].kv_cache[1]) <= state_tol, i
        assert max_rel_err(p.kv_cache[2].cpu(), pools[i].kv_cache[2]) <= state_tol, i
    for i, (k_ref, v_ref) in kv_ref.items():
        kd, vd = model.layers[i].mixer.cache.dense(model.block_table, B, L)
        assert max_rel_err(kd.cpu(), k_ref.transpose(-1, -2)) <= 2e-2, i
        assert max_rel_err(vd.cpu(), v_ref) <= 2e-2, i


def test_prefill_vs_cpu_composition():
    """Two fresh 45-token prompts through the five-layer model."""
    _prefill_vs_composition(_cfg5(256), 2, 45, "harness_prefill")


def test_prefill_7b_layer_shape():
    """Two 300-token prompts at the 7B model's layer shape (the stripe
    prefill kernels take both Hyena cores at this size)."""
    cfg = HyenaConfig(hidden_size=4096, num_hidden_layers=5, num_attention_heads=32,
                      intermediate_size=11264, vocab_size=512, hcs_layer_idxs=[0, 4],
                      hcm_layer_idxs=[1], hcl_layer_idxs=[2], attn_layer_idxs=[3],
                      use_fp8_input_projections=True)
    # the last layer's states carry the bf16 differences of the four layers
    # before it at H=4096 (see test_decode_steps_7b_layer_shape)
    _prefill_vs_composition(cfg, 2, 300, "harness_prefill_7b_shape", seed=14, state_tol=5e-2)


def test_prefill_then_decode_matches_longer_prefill():
    """prefill(L) + one decode token == prefill(L + 1) at its last position:
    logits, Hyena states and the new KV entries, for prompts of 40 and 47
    tokens (the decode position in the middle of a page and at a page start)."""
    H, B = 256, 2
    cfg = _cfg5(H)
    for L in (40, 47):
        a = Evo2DecodeModel(cfg, max_batch=B, max_ctx=64, device=DEV, rope_theta=10000.0,
                            rope_factor=4.0, name=f"harness_pd_a{L}", page_seed=9)
        b = Evo2DecodeModel(cfg, max_batch=B, max_ctx=64, device=DEV, rope_theta=10000.0,
                            rope_factor=4.0, name=f"harness_pd_b{L}", page_seed=9)
        a.init_random(seed=21, state_scale=0.0, kv_scale=0.0)
        b.init_random(seed=21, state_scale=0.0, kv_scale=0.0)
        g = torch.Generator().manual_seed(L)
        tok = torch.tensor([65, 67, 71, 84])[torch.randint(0, 4, (B, L + 1), generator=g)].to(DEV)
        print(f"prefill({L}) + decode vs prefill({L + 1})", flush=True)
        full = a.prefill(tok)
        b.prefill(tok[:, :L])
        step = b.decode_step(tok[:, L].contiguous(), torch.full((B,), L, device=DEV))
        assert max_rel_err(step.cpu(), full.cpu()) <= 3e-2, L
        for i in a.pools:
            assert max_rel_err(b.pools[i].kv_cache[1].cpu(), a.pools[i].kv_cache[1].cpu()) <= 2e-2
            assert max_rel_err(b.pools[i].kv_cache[2].cpu(), a.pools[i].kv_cache[2].cpu()) <= 2e-2
            assert torch.equal(b.pools[i].kv_cache[0], a.pools[i].kv_cache[0]) or \
                max_rel_err(b.pools[i].kv_cache[0].cpu(), a.pools[i].kv_cache[0].cpu()) <= 2e-2
        ka, va = a.layers[3].mixer.cache.dense(a.block_table, B, L + 1)
        kb, vb = b.layers[3].mixer.cache.dense(b.block_table, B, L + 1)
        assert max_rel_err(kb.cpu(), ka.cpu()) <= 2e-2
        assert max_rel_err(vb.cpu(), va.cpu()) <= 2e-2
