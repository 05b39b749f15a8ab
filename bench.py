#!/usr/bin/env python3
"""Throughput of the Evo 2 Hyena mixer hot path on one MI355X.

Headline workload (`value`): 7B-shaped decode -- the 27 Hyena mixers of the
7B layer map (9 hcs, 9 hcm, 9 hcl; H=4096), batch 64, paged state in a
vLLM-layout pool with a seeded random slot table.  One step = one token for
all 64 sequences through every mixer core (the fused decode kernel).  Inputs
are resident in HBM before the timed region.

Also measured in the same run and reported in the same JSON line:
  * prefill: the 27 mixer cores over one 32768-token sequence (fused
    featurizer + FIR / modal scan + gate per layer), tokens/s;
  * fp8: the e4m3 projection GEMMs M=8192, K=4096 -> N=12288 and N=4096,
    TFLOP/s against the dense fp8 MFMA peak, and the decode-sized in_proj
    (M=64) against HBM;
  * verify: the inner operators of a speculative verify step (64 requests
    of 4 tokens, a state snapshot per token) against HBM;
  * model_decode: the whole 7B-shaped model at decode (the mixers and the
    paged decode attention on this build's kernels, projections and MLPs in
    torch), end-to-end tokens/s; model_prefill and model_40b the same
    harness at prefill and at the 40B shape;
  * attn_prefill: the harness's causal prefill attention kernel at the 7B
    prompt (and the 40B one with --only attn_prefill), with torch's fused
    attention on the same inputs as a reference;
  * config0_prefill: one mixer core of each kind at H=1920 over one fresh
    2048-token sequence, tokens/s per block on the GPU and for the oracle's
    restatement of the reference torch path on the host cores;
  * roofline of the dominant decode kernel (hcm) from HIP events on the
    stream it is launched on, and the CPU baseline: the oracle's restatement
    of the reference torch decode path timed on the host cores.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-prefill] [--no-gemm]
                    [--no-verify] [--no-model] [--no-model40b] [--model-steps N]
                    [--only decode|verify|prefill|gemm|copy|model|config0|model_prefill|model40b|
                            attn_prefill]
"""

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

H_7B = 4096
B_DECODE = 64
L_PREFILL = 32768
LAYER_MAP_7B = {  # evo2_configs/evo2-7b-1m.yml:7-9
    "hcs": [0, 4, 7, 11, 14, 18, 21, 25, 28],
    "hcm": [1, 5, 8, 12, 15, 19, 22, 26, 29],
    "hcl": [2, 6, 9, 13, 16, 20, 23, 27, 30],
}
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
METRIC = "decode tok/s (7B-shape, bs=64) + prefill tok/s at 32k; % HBM/MFMA roofline"


DECODE_ROOFLINE_KERNEL = "hcm_decode_split_kernel"
DECODE_PROFILE = os.path.join(ROOT, "profiles", "decode_7b_b64_kernels.md")


def profiled_traffic(kernel, path=DECODE_PROFILE):
    """HBM bytes per launch of `kernel` as measured by the FETCH_SIZE and
    WRITE_SIZE counter passes summarised in `path` (a line
    `traffic_bytes <kernel> <int>`, already scaled by the copy-kernel
    calibration); None when no such measurement is recorded."""
    try:
        with open(path) as f:
            for ln in f:
                m = re.match(r"\s*traffic_bytes\s+(\S+)\s+(\d+)", ln)
                if m and m.group(1) == kernel:
                    return int(m.group(2))
    except OSError:
        pass
    return None


def decode_bytes_per_launch(kind, B, H):
    """Algorithmic HBM bytes of one fused decode launch: every live state
    column the contract forces to be read and written, the z row in and the
    output row out per token, plus the parameters read once per launch."""
    conv = 2 * (3 * H) * 2 * 2                 # (c0, c1) bf16 read + write
    z_out = 3 * H * 2 + H * 2
    if kind == "hcs":
        inner, params = 6 * H * 4 * 2, 3 * H * 3 * 2 + H * 7 * 2
    elif kind == "hcm":
        inner, params = 127 * H * 4 * 2, 3 * H * 3 * 2 + H * 128 * 2 + H * 2
    else:
        inner, params = 16 * H * 4 * 2, 3 * H * 3 * 2 + 2 * H * 16 * 4 + H * 2
    return B * (conv + inner + z_out) + params


def prefill_bytes(T, H):
    """Fused minimum of one mixer-core prefill: read z (T, 3H) bf16 once and
    write g (T, H) bf16 once; state and parameter bytes are < 0.1% and left out."""
    return T * 3 * H * 2 + T * H * 2


def _timed(fn, reps, stream, batches=4):
    """Average duration (us) of one fn() call on `stream` (the stream the
    kernels run on): `batches` batches of reps/batches back-to-back calls,
    each batch bracketed by HIP events, so event overhead is amortised and
    the figure includes the launch gaps a real step has.  Returns (mean over
    all calls, median of the per-batch means)."""
    per = max(1, reps // batches)
    evs = []
    for _ in range(batches):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(per):
            fn()
        b.record(stream)
        evs.append((a, b))
    torch.cuda.synchronize()
    d = [a.elapsed_time(b) * 1e3 / per for a, b in evs]
    return statistics.mean(d), statistics.median(d)


def bench_copy(dev, nbytes=1 << 30, reps=8):
    """Plain device-to-device copy of nbytes (read + write): the achievable
    HBM bandwidth next to the 8 TB/s vendor peak."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    avg, _ = _timed(lambda: dst.copy_(src), reps, torch.cuda.current_stream())
    return {"bytes": 2 * nbytes, "avg_us": round(avg, 2),
            "GBs": round(2 * nbytes / (avg * 1e-6) / 1e9, 1)}


# ---------------------------------------------------------------- decode
class DecodeLayer:
    def __init__(self, kind, idx, H, B, dev, seed):
        from evo2_flash_amd.decode import channel_major_taps
        from evo2_flash_amd.state import HyenaStatePool
        from evo2_flash_amd.synthetic import mixer_params, random_slot_table

        self.kind = kind
        prm = mixer_params(kind, H, seed + idx, device=dev, in_proj_fp8=False)
        self.short_w = prm["short_filter"].view(3 * H, 3)
        self.D = prm.get("D")
        if kind == "hcl":
            self.inner = prm["residues"]
            self.lp = prm["log_poles"][..., 0]
        else:
            K = prm["conv"].shape[-1]
            # the decode taps as the mixers keep them: channel-contiguous
            self.inner = channel_major_taps(prm["conv"].view(H, K))
            self.lp = None
        self.pool = HyenaStatePool(B + 1, H, dev)
        g = torch.Generator(device=dev).manual_seed(seed + 1000 + idx)
        for s in self.pool.kv_cache:
            s.copy_(torch.randn(s.shape, generator=g, device=dev).to(s.dtype))
        self.state = (self.pool.ssm_view() if kind == "hcl"
                      else self.pool.inner_view(self.inner.shape[1] - 1))
        self.slots = random_slot_table(B, B + 1, seed + 2000 + idx, device=dev)
        self.z = (torch.randn(B, 3 * H, generator=g, device=dev) * 1.3).to(torch.bfloat16)

    def step(self):
        from evo2_flash_amd.decode import hyena_decode

        return hyena_decode(self.z, self.short_w, self.pool.conv_view(), self.slots,
                            self.inner, self.state, self.D, self.lp)


def _graph(fn, n):
    """A HIP graph of n back-to-back calls of fn (captured on a side stream,
    as torch requires); the decode step is replayed this way in serving."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(n):
                fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return g


def bench_decode(steps, warmup, dev, seed=1234):
    """27 fused decode launches per step, replayed from one HIP graph; per-kind
    launch durations from graphs of 36 launches of one kind (event-timed on
    the replay stream, so launch gaps are included)."""
    H, B = H_7B, B_DECODE
    order = sorted((i, k) for k, idxs in LAYER_MAP_7B.items() for i in idxs)
    layers = [DecodeLayer(k, i, H, B, dev, seed) for i, k in order]

    def step():
        for L in layers:
            L.step()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    g_step = _graph(step, 1)
    stream = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    g_step.replay()
    t0.record(stream)
    for _ in range(steps):
        g_step.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / steps
    per_kind = {}
    reps = 4
    for kind in LAYER_MAP_7B:
        Ls = [L for L in layers if L.kind == kind]
        g = _graph(lambda: [L.step() for L in Ls], reps)
        n = reps * len(Ls)
        avg, med = _timed(g.replay, max(4, steps // 4), stream)
        avg, med = avg / n, med / n
        nbytes = decode_bytes_per_launch(kind, B, H)
        per_kind[kind] = {"avg_us": round(avg, 3), "median_us": round(med, 3),
                          "bytes_per_launch": nbytes,
                          "achieved_GBs": round(nbytes / (avg * 1e-6) / 1e9, 1),
                          "frac": round(nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    ideal_us = 9 * sum(decode_bytes_per_launch(k, B, H) for k in LAYER_MAP_7B) / (HBM_PEAK_GBS * 1e3)
    kern_us = 9 * sum(v["avg_us"] for v in per_kind.values())
    return {"ms_per_step": ms_per_step, "tok_s": B / (ms_per_step * 1e-3), "per_kind": per_kind,
            "layers": len(layers), "kernel_us_per_step": round(kern_us, 2),
            "ideal_us_per_step": round(ideal_us, 2),
            "mixer_frac": round(ideal_us / kern_us, 4)}


# ---------------------------------------------------------------- whole model
CTX_7B = 8192 + 512   # prompt plus the decode steps of the 7B workload
PROMPT_7B = 8192
STEPS_7B = 512        # decode steps of the 7B workload
STEPS_40B = 8         # timed decode steps of the 40B workload (of its 256)
ACGT = (65, 67, 71, 84)


def _acgt(shape, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.tensor(ACGT, device=dev)[torch.randint(0, 4, shape, generator=g, device=dev)]


def _sync_time(fn):
    torch.cuda.synchronize()
    t = time.perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, time.perf_counter() - t


def _graph_decode(model, B, pos0, steps, dev, seed):
    """Replay one captured decode step `steps` times from position pos0 on;
    returns ms per step."""
    tok = _acgt((B,), dev, seed)
    pos = torch.full((B,), pos0, dtype=torch.int64, device=dev)
    model.decode_step(tok, pos)          # warm-up, builds the step's metadata
    pos.add_(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            model.decode_step(tok, pos)
            pos.add_(1)
    torch.cuda.current_stream().wait_stream(s)
    graph.replay()
    stream = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    del graph
    return t0.elapsed_time(t1) / steps


def bench_model(steps, dev, B=B_DECODE, seed=21):
    """Config 1 end to end: the whole 7B-shaped model (32 layers: 27 Hyena on
    this build's kernels, 5 attention layers on 16-position KV pages of a
    seeded random block table), B sequences each prefilled from an
    8192-token uniform-ACGT prompt (the mixers' prefill kernels write the
    states, attention writes the pages), then decode from position 8192 on,
    one HIP graph replay per step; rotary base 1e4 with linear scaling 128
    (evo2-7b-1m.yml:27-29).  Projections and MLPs are torch."""
    from evo2_flash_amd.config import evo2_7b
    from evo2_flash_amd.model import Evo2DecodeModel, decode_flops_bytes

    cfg = evo2_7b()
    # one page beyond the workload: _graph_decode runs two untimed steps first
    model = Evo2DecodeModel(cfg, max_batch=B, max_ctx=CTX_7B + 16, device=dev,
                            rope_theta=10000.0, rope_factor=128.0, name=f"bench_model_b{B}",
                            page_seed=seed)
    model.init_random(seed, state_scale=0.0, kv_scale=0.0)
    prompts = _acgt((B, PROMPT_7B), dev, seed + 1)
    _, t_pre = _sync_time(lambda: model.prefill(prompts, chunk_seqs=8))
    n = steps
    if PROMPT_7B + n + 2 > CTX_7B + 16:
        raise ValueError(f"{n} decode steps run past the cache")
    ms = _graph_decode(model, B, PROMPT_7B, n, dev, seed + 2)
    wbytes, kvbytes = decode_flops_bytes(cfg, B, PROMPT_7B + n)
    del model
    torch.cuda.empty_cache()
    return {"tok_s": round(B / (ms * 1e-3), 1), "ms_per_step": round(ms, 3), "batch": B,
            "context": f"{PROMPT_7B}..{PROMPT_7B + n + 1} (timed: the last {n} steps)",
            "steps": n, "layers": 32,
            "prefill": {"prompt_tokens": B * PROMPT_7B, "s": round(t_pre, 2),
                        "tok_s": round(B * PROMPT_7B / t_pre, 1)},
            "bytes_per_step": {"weights": wbytes, "kv_cache": kvbytes},
            "achieved_GBs": round((wbytes + kvbytes) / (ms * 1e-3) / 1e9, 1),
            "kv": "16-position pages, seeded random block table",
            "note": "states and KV pages from prefilling the prompts; Hyena mixers and decode "
                    "attention on this build's kernels; projections and MLP in torch"}


def _layer_timers(model):
    """Wrap each layer's mixer so a run records (kind, start, end) events
    around it, for the share of the mixers in a prefill."""
    recs = []
    for layer in model.layers:
        mixer = layer.mixer
        name = "forward_prefill" if layer.kind == "attn" else "forward"
        orig = getattr(mixer, name)

        def timed(*a, _orig=orig, _kind=layer.kind, **k):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            out = _orig(*a, **k)
            e1.record()
            recs.append((_kind, e0, e1))
            return out
        setattr(mixer, name, timed)
    return recs


def bench_model_prefill(dev, L=L_PREFILL, reps=3, seed=31):
    """Config 2 end to end: the whole 7B-shaped model over one L-token
    uniform-ACGT prompt (norms, fp8 in_proj, the mixer cores, out_proj, MLPs,
    causal attention), tokens/s; one instrumented run splits the time by
    layer kind (the Hyena layers' time is in_proj + core + out_proj)."""
    from evo2_flash_amd.config import evo2_7b
    from evo2_flash_amd.model import Evo2DecodeModel, prefill_flops

    cfg = evo2_7b()
    model = Evo2DecodeModel(cfg, max_batch=1, max_ctx=L, device=dev, rope_theta=10000.0,
                            rope_factor=128.0, name="bench_prefill_model", page_seed=seed)
    model.init_random(seed, state_scale=0.0, kv_scale=0.0)
    prompt = _acgt((1, L), dev, seed + 1)
    model.prefill(prompt, chunk_seqs=1)      # warm-up
    times = [_sync_time(lambda: model.prefill(prompt, chunk_seqs=1))[1] for _ in range(reps)]
    t = statistics.median(times)
    recs = _layer_timers(model)
    _, t_inst = _sync_time(lambda: model.prefill(prompt, chunk_seqs=1))
    per = {}
    for kind, e0, e1 in recs:
        per[kind] = per.get(kind, 0.0) + e0.elapsed_time(e1) * 1e3
    fl = prefill_flops(cfg, L)
    del model
    torch.cuda.empty_cache()
    return {"L": L, "ms": round(t * 1e3, 2), "tok_s": round(L / t, 1),
            "TFLOPs": round(fl / t / 1e12, 1), "flop": fl,
            "layer_us": {k: round(v, 1) for k, v in per.items()},
            "instrumented_ms": round(t_inst * 1e3, 2),
            "note": "whole 7B-shaped model, batch 1; Hyena layers = in_proj + mixer core + "
                    "out_proj and the causal attention on this build's kernels; attention "
                    "projections, MLP and norms' GEMMs in torch"}


def bench_attn_prefill(dev, shapes=((32, L_PREFILL),), reps=3, seed=51):
    """The harness's causal prefill attention (head_dim 128, one sequence) on
    this build's kernel, and torch's fused attention on the same inputs as a
    reference (not on any product path): ms per call and TFLOP/s of the
    causal half (4 L^2 d heads / 2)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from evo2_flash_amd.attention import prefill_attention

    out = {}
    for heads, L in shapes:
        g = torch.Generator(device=dev).manual_seed(seed)
        q, k, v = (torch.randn(1, heads, L, 128, generator=g, device=dev).to(torch.bfloat16)
                   for _ in range(3))
        scale = 128 ** -0.5
        flop = 4 * heads * L * L * 128 / 2

        def ref():
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                                        scale=scale)
        r = {}
        for name, fn in (("kernel", lambda: prefill_attention(q, k, v, scale)), ("torch", ref)):
            try:
                fn()
                times = [_sync_time(fn)[1] for _ in range(reps)]
                t = statistics.median(times)
                r[name + "_ms"] = round(t * 1e3, 3)
                r[name + "_TFLOPs"] = round(flop / t / 1e12, 1)
            except RuntimeError as e:  # torch's fused kernels may refuse the inputs
                r[name + "_error"] = str(e).splitlines()[0][:120]
        out[f"{heads}x{L}"] = r
        del q, k, v
        torch.cuda.empty_cache()
    out["note"] = ("kernel: csrc/attention_prefill.hip (values transposed once per call, "
                   "included); torch: scaled_dot_product_attention's fused kernels")
    return out


def bench_model40b(steps, dev, B=32, L=131072, seed=41):
    """Config 4 end to end: the 40B-shaped model (50 layers, H=8192, attention
    at 3, 10, 17, 24, 31, 35, 42, 49 as evo2-40b-1m.yml, fp8 in_proj),
    weights resident (~80 GB), the residual stream at ~1e6 (embedding rows
    scaled by 1e6), one L-token prompt prefilled once, its KV pages shared by
    all B sequences and its Hyena states copied to each, then B sequences
    decode from position L on (one HIP graph replay per step)."""
    from evo2_flash_amd.config import evo2_40b
    from evo2_flash_amd.model import Evo2DecodeModel, decode_flops_bytes, prefill_flops

    cfg = evo2_40b()
    model = Evo2DecodeModel(cfg, max_batch=B, max_ctx=L + 256, device=dev, rope_theta=10000.0,
                            rope_factor=128.0, name="bench_model_40b", page_seed=seed,
                            shared_prefix=L)
    model.init_random(seed, state_scale=0.0, kv_scale=0.0, embed_scale=1e6)
    prompt = _acgt((L,), dev, seed + 1)
    logits, t_pre = _sync_time(lambda: model.prefill_shared(prompt))
    finite = bool(torch.isfinite(logits).all())
    n = steps
    if n + 2 > 256:
        raise ValueError(f"{n} decode steps run past the cache")
    ms = _graph_decode(model, B, L, n, dev, seed + 2)
    wbytes, kvbytes = decode_flops_bytes(cfg, B, L + n)
    # the prompt's pages once, each sequence's own positions once: what the
    # step reads from distinct HBM addresses (the logical figure counts the
    # shared prompt once per sequence)
    _, kv_unique = decode_flops_bytes(cfg, 1, L + B * n)
    fl = prefill_flops(cfg, L)
    del model
    torch.cuda.empty_cache()
    return {"prefill": {"L": L, "s": round(t_pre, 2), "tok_s": round(L / t_pre, 1),
                        "TFLOPs": round(fl / t_pre / 1e12, 1), "logits_finite": finite},
            "decode": {"batch": B, "steps": n, "ms_per_step": round(ms, 3),
                       "tok_s": round(B / (ms * 1e-3), 1),
                       "bytes_per_step": {"weights": wbytes, "kv_cache_logical": kvbytes,
                                          "kv_cache_unique": kv_unique},
                       "logical_GBs": round((wbytes + kvbytes) / (ms * 1e-3) / 1e9, 1),
                       "unique_GBs": round((wbytes + kv_unique) / (ms * 1e-3) / 1e9, 1),
                       "steps_note": f"{n} of the workload's 256 steps: a step costs the same "
                                     f"at every position of 131072..131328 (the KV grows by "
                                     f"0.2%), and 256 steps would hold the GPU ~1 minute"},
            "kv": "one prompt's 16-position pages shared by all sequences through the block "
                  "table, then one page run per sequence",
            "residual_scale": 1e6}


# ---------------------------------------------------------------- speculative verify
def bench_verify(reps, dev, H=H_7B, B=B_DECODE, Q=4, seed=9):
    """The inner operators of a speculative verify step, 7B shape: B requests
    of Q = 4 tokens (3 drafts) each, every request reading its accepted
    snapshot and writing a snapshot per token (launch times from graph
    replays).  Bytes per launch: the source
    state and the Q snapshots (fp32), the token rows in and out (bf16 for
    the FIRs, fp32 for LI as the mixers pass them), the parameters once."""
    from evo2_flash_amd.synthetic import mixer_params
    from evo2_flash_amd.verify import fir_snapshots, iir_snapshots

    g = torch.Generator(device=dev).manual_seed(seed)
    nblk = 2 * B * Q + 1
    ins = (torch.randperm(B * Q, device=dev, generator=g) + 1).to(torch.int32).view(B, Q)
    outs = (torch.randperm(B * Q, device=dev, generator=g) + 1 + B * Q).to(torch.int32).view(B, Q)
    starts = torch.arange(B, device=dev, dtype=torch.int64) * Q
    meta = (ins, outs, starts, starts + Q, torch.full((B,), 2, device=dev, dtype=torch.int64))
    stream = torch.cuda.current_stream()
    res = {}
    for kind in ("hcs", "hcm", "hcl"):
        prm = mixer_params(kind, H, seed, in_proj_fp8=False)
        if kind == "hcl":
            x = torch.randn(B * Q, H, generator=g, device=dev)
            st = torch.randn(nblk, H, 16, generator=g, device=dev)
            poles = prm["log_poles"][..., 0].to(dev).exp()
            r = prm["residues"].to(dev)
            fn = lambda x=x, st=st, poles=poles, r=r: iir_snapshots(x, poles, r, st, meta)  # noqa: E731
            cols, xb, pbytes = 16, 4, 2 * H * 16 * 4
        else:
            K = prm["conv"].shape[-1]
            x = torch.randn(B * Q, H, generator=g, device=dev).to(torch.bfloat16)
            st = torch.randn(nblk, K - 1, H, generator=g, device=dev).transpose(1, 2)
            w = prm["conv"].view(H, K).to(dev)
            fn = lambda x=x, st=st, w=w: fir_snapshots(x, w, st, meta)  # noqa: E731
            cols, xb, pbytes = K - 1, 2, H * K * 2
        fn()
        torch.cuda.synchronize()
        # replayed from a graph of 8 calls, as a serving step runs them (eager
        # calls of the 10-20 us kernels would time the Python wrapper)
        g_k = _graph(fn, 8)
        avg, med = _timed(g_k.replay, max(4, reps // 4), stream)
        avg, med = avg / 8, med / 8
        nbytes = B * (1 + Q) * H * cols * 4 + 2 * B * Q * H * xb + pbytes
        res[kind] = {"avg_us": round(avg, 2), "median_us": round(med, 2), "bytes": nbytes,
                     "achieved_GBs": round(nbytes / (avg * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    steps = _bench_verify_mixers(reps, dev, H, B, Q, seed)
    for kind, v in steps.items():
        res[kind]["mixer_step"] = v
    return {"requests": B, "tokens_per_request": Q, "per_kind": res,
            "mixer_step_scope": "whole mixer forward of a verify step: fp8 in_proj, speculative "
                                "short window, snapshot verify, gate, bf16 out_proj, stamps "
                                "(plus one small stamp-reset launch per step), captured in one "
                                "HIP graph per step; eager launches timed beside it"}


def _bench_verify_mixers(reps, dev, H, B, Q, seed):
    """A whole speculative verify step through each mixer kind (num_spec =
    Q - 1): B requests of Q tokens, slot rows of Q distinct blocks, the
    previous step's accepted count resolved from the position stamps."""
    from evo2_flash_amd.config import HyenaConfig
    from evo2_flash_amd.metadata import HyenaMamba2Metadata
    from evo2_flash_amd.mixers import load_mixer_params, make_mixer, set_forward_context
    from evo2_flash_amd.state import HyenaStatePool
    from evo2_flash_amd.synthetic import mixer_params

    cfg = HyenaConfig(hidden_size=H, num_hidden_layers=3, hcs_layer_idxs=[0], hcm_layer_idxs=[1],
                      hcl_layer_idxs=[2], use_fp8_input_projections=True)
    nblk = B * Q + 1
    slots = (torch.arange(B * Q, device=dev, dtype=torch.int32) + 1).view(B, Q)
    computed = 8192
    m = HyenaMamba2Metadata()
    m.num_decodes, m.num_decode_tokens = B, B * Q
    m.state_indices_tensor_d = slots
    m.query_start_loc_d = torch.arange(B + 1, device=dev, dtype=torch.int32) * Q
    m.num_computed_tokens_d = torch.full((B,), computed, device=dev, dtype=torch.int32)
    m.seq_lens = torch.full((B,), computed + Q, device=dev, dtype=torch.int32)
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    hs = torch.randn(B * Q, H, generator=g, device=dev).to(torch.bfloat16)
    stream = torch.cuda.current_stream()
    out = {}
    for kind, layer in (("hcs", 0), ("hcm", 1), ("hcl", 2)):
        mixer = make_mixer(cfg, layer, prefix=f"bench.verify.{kind}", device=dev, num_spec=Q - 1)
        load_mixer_params(mixer, mixer_params(kind, H, seed + layer, in_proj_fp8=True))
        pool = HyenaStatePool(nblk, H, dev, num_spec=Q - 1)
        for t in pool.kv_cache:
            t.copy_(torch.randn(t.shape, generator=g, device=dev).to(t.dtype))
        mixer.kv_cache = pool.kv_cache

        live = slots[:, 0].long()

        def fn(mixer=mixer, pool=pool, live=live):
            # stamps of the live snapshots: the previous step accepted 2 tokens
            pool.stamps().index_fill_(0, live, float(computed - 1))
            with set_forward_context(m):
                return mixer(hs)

        start = [t.clone() for t in pool.kv_cache]

        def restore(pool=pool, start=start):
            for t, t0 in zip(pool.kv_cache, start):
                t.copy_(t0)

        ref = fn().clone()
        torch.cuda.synchronize()
        faults = mixer.stamp_faults()
        eager_avg, eager_med = _timed(fn, max(4, reps // 2), stream)
        # the same step captured once and replayed: each replay from the
        # restored pool must reproduce the eager output bit for bit
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            restore()
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            res_g = fn()
        exact = True
        for _ in range(3):
            restore()
            graph.replay()
            torch.cuda.synchronize()
            exact = exact and torch.equal(res_g.view(torch.int16), ref.view(torch.int16))
        avg, med = _timed(graph.replay, reps, stream)
        out[kind] = {"graph_avg_us": round(avg, 2), "graph_median_us": round(med, 2),
                     "tokens_per_s": round(B * Q / (avg * 1e-6), 1),
                     "eager_avg_us": round(eager_avg, 2), "eager_median_us": round(eager_med, 2),
                     "graph_matches_eager": exact, "stamp_faults": faults}
        del mixer, pool, graph, start
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- prefill
def bench_prefill(reps, dev, L=L_PREFILL, H=H_7B, seed=77, warmup=1):
    """One fresh L-token sequence through the 27 Hyena mixer cores of the 7B
    layer map, launched in layer order (9 each of hcs, hcm, hcl, interleaved
    as in the model).  `warmup` untimed passes, then `reps` passes timed as a
    whole (the step), then `reps` passes with an event between launches (the
    per-kind figures).  Timing each kind alone, back to back, measured the
    hcl core up to ~15% slower than inside the layer sequence: sustained
    back-to-back runs of it lower the clock."""
    from evo2_flash_amd.config import evo2_7b
    from evo2_flash_amd.hcl import hcl_block_t, hyena_hcl_prefill
    from evo2_flash_amd.metadata import build_metadata, prefill_tables
    from evo2_flash_amd.prefill import fir_prefill_block_t, hyena_fir_prefill
    from evo2_flash_amd.state import HyenaStatePool
    from evo2_flash_amd.synthetic import mixer_params

    g = torch.Generator(device=dev).manual_seed(seed)
    z = (torch.randn(L, 3 * H, generator=g, device=dev) * 1.3).to(torch.bfloat16)
    m = build_metadata(prefill_lens=[L], prefill_slots=[1], has_init=[0], device=dev)
    pool = HyenaStatePool(2, H, dev)
    stream = torch.cuda.current_stream()
    fns, block_t = {}, {}
    for kind in ("hcs", "hcm", "hcl"):
        prm = mixer_params(kind, H, seed, device=dev, in_proj_fp8=False)
        sw = prm["short_filter"].view(3 * H, 3)
        if kind == "hcl":
            bt = hcl_block_t(L, H)
            seq_t, til_t, ts_t = prefill_tables(m, bt, dev)

            def fn(prm=prm, sw=sw, bt=bt, seq_t=seq_t, til_t=til_t, ts_t=ts_t):
                return hyena_hcl_prefill(z, sw, pool.conv_view(), prm["residues"],
                                         prm["log_poles"][..., 0], pool.ssm_view(), prm["D"],
                                         seq_t, m.state_indices_tensor_p, til_t, ts_t, bt)
        else:
            K = prm["conv"].shape[-1]
            bt = fir_prefill_block_t(K, L, H)
            seq_t, til_t, _ = prefill_tables(m, bt, dev)
            w = prm["conv"].view(H, K)

            def fn(prm=prm, sw=sw, bt=bt, seq_t=seq_t, til_t=til_t, w=w, K=K):
                return hyena_fir_prefill(z, sw, pool.conv_view(), w, pool.inner_view(K - 1),
                                         prm.get("D"), seq_t, m.state_indices_tensor_p, til_t, bt)
        fns[kind], block_t[kind] = fn, bt
    cfg = evo2_7b()
    order = [cfg.layer_kind(i) for i in range(cfg.num_hidden_layers)]
    order = [k for k in order if k != "attn"]
    assert len(order) == 27 and all(order.count(k) == 9 for k in fns), order
    for _ in range(max(1, warmup)):
        for k in order:
            fns[k]()
    torch.cuda.synchronize()
    # the step: whole passes between two events
    steps = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for k in order:
            fns[k]()
        b.record(stream)
        steps.append((a, b))
    # per kind: an event after every launch
    passes = []
    for _ in range(reps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(order) + 1)]
        ev[0].record(stream)
        for j, k in enumerate(order):
            fns[k]()
            ev[j + 1].record(stream)
        passes.append(ev)
    torch.cuda.synchronize()
    step_us = statistics.mean(a.elapsed_time(b) * 1e3 for a, b in steps)
    per = {k: [] for k in fns}
    for ev in passes:
        for j, k in enumerate(order):
            per[k].append(ev[j].elapsed_time(ev[j + 1]) * 1e3)
    nbytes = prefill_bytes(L, H)
    res = {}
    for kind in ("hcs", "hcm", "hcl"):
        avg, med = statistics.mean(per[kind]), statistics.median(per[kind])
        res[kind] = {"avg_us": round(avg, 2), "median_us": round(med, 2), "block_t": block_t[kind],
                     "bytes": nbytes, "achieved_GBs": round(nbytes / (avg * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    ideal_us = 27 * nbytes / (HBM_PEAK_GBS * 1e3)
    del z
    return {"scope": "the 27 Hyena mixer cores of the 7B layer map, z -> g (short filter, "
                     "gate, inner FIR or modal scan, D, x2), launched in layer order; in_proj, "
                     "out_proj, norms, MLPs and attention are in model_prefill",
            "tok_s": round(L / (step_us * 1e-6), 1), "us_per_step": round(step_us, 1),
            "sum_of_kinds_us": round(9 * sum(v["avg_us"] for v in res.values()), 1),
            "L": L, "mixer_frac": round(ideal_us / step_us, 4), "per_kind": res}


# ---------------------------------------------------------------- 1B-shaped blocks
def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def bench_config0(reps, dev, H=1920, L=2048, seed=11, cpu=True):
    """One block of each Hyena kind at the reference's CPU-runnable shape
    (H=1920, one fresh 2048-token sequence): prefill tok/s per block of the
    mixer core (z -> g) on this build's kernels, and, when `cpu`, of the
    oracle's restatement of the reference torch path (the FIR mixer's prefill
    rows, mixers.py:1277-1305; the IIR mixer's, mixers.py:1327-1401) on the
    host cores, same inputs."""
    from evo2_flash_amd.hcl import hcl_block_t, hyena_hcl_prefill
    from evo2_flash_amd.metadata import build_metadata, prefill_tables
    from evo2_flash_amd.prefill import fir_prefill_block_t, hyena_fir_prefill
    from evo2_flash_amd.state import HyenaStatePool
    from evo2_flash_amd.synthetic import mixer_params

    g = torch.Generator().manual_seed(seed)
    z_cpu = (torch.randn(L, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    z = z_cpu.to(dev)
    m = build_metadata(prefill_lens=[L], prefill_slots=[1], has_init=[0], device=dev)
    pool = HyenaStatePool(2, H, dev)
    stream = torch.cuda.current_stream()
    n = len(os.sched_getaffinity(0))
    res = {}
    for kind in ("hcs", "hcm", "hcl"):
        prm = mixer_params(kind, H, seed, in_proj_fp8=False)
        pd = {k: v.to(dev) for k, v in prm.items()}
        sw = pd["short_filter"].view(3 * H, 3)
        if kind == "hcl":
            bt = hcl_block_t(L, H)
            seq_t, til_t, ts_t = prefill_tables(m, bt, dev)

            def fn(pd=pd, sw=sw, bt=bt, seq_t=seq_t, til_t=til_t, ts_t=ts_t):
                return hyena_hcl_prefill(z, sw, pool.conv_view(), pd["residues"],
                                         pd["log_poles"][..., 0], pool.ssm_view(), pd["D"],
                                         seq_t, m.state_indices_tensor_p, til_t, ts_t, bt)
        else:
            K = pd["conv"].shape[-1]
            bt = fir_prefill_block_t(K, L, H)
            seq_t, til_t, _ = prefill_tables(m, bt, dev)

            def fn(pd=pd, sw=sw, bt=bt, seq_t=seq_t, til_t=til_t, K=K):
                return hyena_fir_prefill(z, sw, pool.conv_view(), pd["conv"].view(H, K),
                                         pool.inner_view(K - 1), pd.get("D"), seq_t,
                                         m.state_indices_tensor_p, til_t, bt)
        fn()
        torch.cuda.synchronize()
        avg, med = _timed(fn, reps, stream)
        nbytes = prefill_bytes(L, H)
        entry = {"gpu_us": round(avg, 2), "gpu_tok_s": round(L / (avg * 1e-6), 1),
                 "bytes": nbytes, "achieved_GBs": round(nbytes / (avg * 1e-6) / 1e9, 1)}
        if cpu:
            import oracle
            torch.set_num_threads(n)
            cpool = HyenaStatePool(2, H, "cpu")
            sw_c = prm["short_filter"].view(3 * H, 3)
            times = []
            with torch.inference_mode():
                for _ in range(3):
                    t = time.perf_counter()
                    if kind == "hcl":
                        oracle.iir_mixer_prefill(z_cpu, sw_c, cpool.conv_view(), prm["residues"],
                                                 prm["log_poles"][..., 0], cpool.ssm_view(),
                                                 prm["D"], [0, L], [1], [0])
                    else:
                        K = prm["conv"].shape[-1]
                        oracle.fir_mixer_prefill(z_cpu, sw_c, cpool.conv_view(),
                                                 prm["conv"].view(H, K), cpool.inner_view(K - 1),
                                                 prm.get("D"), [0, L], [1], [0])
                    times.append(time.perf_counter() - t)
            cs = statistics.median(times[1:])
            entry.update({"cpu_s": round(cs, 4), "cpu_tok_s": round(L / cs, 1)})
        res[kind] = entry
    del z
    return {"scope": "one Hyena mixer core per kind, z -> g (short filter, gate, inner FIR or "
                     "modal scan, D, x2), the same on both legs; projections not included",
            "H": H, "L": L, "cores": n if cpu else None, "cpu_model": _cpu_model() if cpu else None,
            "cpu_kind": "oracle restatement of the reference torch path" if cpu else None,
            "per_block": res}


# ---------------------------------------------------------------- fp8 GEMMs
def bench_gemm(reps, dev, M=8192, K=4096, seed=5):
    from evo2_flash_amd.fp8 import fp8_gemm, fp8_gemm_packed, fp8_pack_weight, quantize_input
    from evo2_flash_amd.synthetic import quantize_weight_e4m3

    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    xs = (x.float().abs().max() / 448.0).reshape(1)
    x8 = quantize_input(x, xs)
    stream = torch.cuda.current_stream()
    out = {}
    for name, N in (("in_proj", 12288), ("out_proj", 4096)):
        w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=g, device=dev) * 0.02)
        o = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        fn = lambda: fp8_gemm(x8, w8, xs, ws, out=o)  # noqa: E731
        fn()
        torch.cuda.synchronize()
        avg, med = _timed(fn, reps, stream)
        flop = 2 * M * N * K
        tf = flop / (avg * 1e-6) / 1e12
        out[name] = {"M": M, "N": N, "K": K, "avg_us": round(avg, 2), "median_us": round(med, 2),
                     "TFLOPs": round(tf, 1), "frac": round(tf / FP8_PEAK_TFLOPS, 4)}
        # the platform library's fp8 GEMM on the same operands, for reference
        # (torch._scaled_mm -> hipBLASLt); not on any product path
        try:
            one = torch.ones((), device=dev)
            ref = lambda: torch._scaled_mm(x8, w8.t(), scale_a=one, scale_b=one,  # noqa: E731
                                           out_dtype=torch.bfloat16)
            ref()
            torch.cuda.synchronize()
            ravg, _ = _timed(ref, reps, stream)
            out[name]["library_us"] = round(ravg, 2)
            out[name]["library_TFLOPs"] = round(flop / (ravg * 1e-6) / 1e12, 1)
        except RuntimeError as e:  # the platform has no fp8 library GEMM for these inputs
            out[name]["library_us"] = None
            out[name]["library_error"] = str(e).splitlines()[0][:120]
    qavg, _ = _timed(lambda: quantize_input(x, xs), reps, stream)
    out["quantize"] = {"avg_us": round(qavg, 2), "bytes": M * K * 3,
                       "achieved_GBs": round(M * K * 3 / (qavg * 1e-6) / 1e9, 1)}
    # decode-sized in_proj (B=64 rows): bound by streaming the e4m3 weights.
    # Nine weights (450 MB, more than the 256 MB infinity cache holds) are
    # used in turn, as a decode step reads a different weight per layer.
    Md, N, nw = B_DECODE, 12288, 9
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=g, device=dev) * 0.02)
    wds = [w8] + [w8.clone() for _ in range(nw - 1)]
    xd8 = x8[:Md].contiguous()
    od = torch.empty(Md, N, dtype=torch.bfloat16, device=dev)
    turn = [0]

    def fn_rows():
        fp8_gemm(xd8, wds[turn[0] % nw], xs, ws, out=od)
        turn[0] += 1

    fn_rows()
    torch.cuda.synchronize()
    ravg, _ = _timed(fn_rows, max(reps, 36), stream)
    # the decode step's form: the weights in the decode layout (a packed copy
    # kept beside the checkpoint one), same result bits
    wps = [fp8_pack_weight(w) for w in wds]

    def fn():
        fp8_gemm_packed(xd8, wps[turn[0] % nw], xs, ws, out=od)
        turn[0] += 1

    fn()
    torch.cuda.synchronize()
    avg, med = _timed(fn, max(reps, 36), stream)
    nbytes = N * K + Md * K + Md * N * 2
    out["decode_in_proj"] = {"M": Md, "N": N, "K": K, "avg_us": round(avg, 2),
                             "median_us": round(med, 2), "bytes": nbytes,
                             "weights_in_turn": nw, "weight_layout": "decode (packed)",
                             "achieved_GBs": round(nbytes / (avg * 1e-6) / 1e9, 1),
                             "frac_hbm": round(nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             "row_major_avg_us": round(ravg, 2)}
    del wds, wps
    return out


# ---------------------------------------------------------------- CPU baseline
def _cpu_baseline_decode(budget_s=20.0):
    """The oracle's restatement of the reference torch decode path (unfused,
    mixers.py:555-575) for one layer of each kind at B=64, H=4096, timed on
    the host cores; the 27-layer step is 9x the sum of the three."""
    import oracle
    from evo2_flash_amd.state import HyenaStatePool
    from evo2_flash_amd.synthetic import mixer_params, random_slot_table

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    H, B = H_7B, B_DECODE
    per = {}
    t_start = time.perf_counter()
    for kind in ("hcs", "hcm", "hcl"):
        prm = mixer_params(kind, H, 99, in_proj_fp8=False)
        pool = HyenaStatePool(B + 1, H, "cpu")
        slots = random_slot_table(B, B + 1, 5)
        g = torch.Generator().manual_seed(4)
        z = (torch.randn(B, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
        sw = prm["short_filter"].view(3 * H, 3)
        if kind == "hcl":
            inner, lp, st = prm["residues"], prm["log_poles"][..., 0], pool.ssm_view()
        else:
            inner, lp, st = prm["conv"].view(H, -1), None, pool.inner_view()
        D = prm.get("D")
        times = []
        with torch.inference_mode():
            for _ in range(4):
                t = time.perf_counter()
                oracle.mixer_decode_unfused(z, sw, pool.conv_view(), slots, inner, st, D, lp)
                times.append(time.perf_counter() - t)
                if time.perf_counter() - t_start > budget_s:
                    break
        per[kind] = statistics.median(times[1:] if len(times) > 1 else times)
    step_s = 9 * sum(per.values())
    return {"value": round(B / step_s, 2), "unit": "tok/s", "cores": n, "kind": "port",
            "sample": ("oracle unfused torch decode (mixers.py:555-575 restated), one layer of "
                       "each kind at B=64 H=4096, median of 3 after 1 warm-up; 27-layer step "
                       "= 9 x (hcs + hcm + hcl); per-layer s: "
                       + ", ".join(f"{k}={v:.4f}" for k, v in per.items()))}


def _cpu_baseline_layers(L=4096, budget_s=30.0):
    """The oracle's restatement of the reference torch path for one layer of
    each Hyena kind at the other configs' shapes, on the host cores:
    config 2's prefill at H=4096 (L=4096 here, an eighth of the 32768-token
    prompt; the FIRs scale linearly in L, the FFT convolution as L log L) and
    config 4's decode step at B=32, H=8192.  Median of 2 after a warm-up."""
    import oracle
    from evo2_flash_amd.state import HyenaStatePool
    from evo2_flash_amd.synthetic import mixer_params, random_slot_table

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    t_start = time.perf_counter()
    out = {"cores": n, "cpu_model": _cpu_model(), "kind": "port"}
    pre, H = {}, H_7B
    g = torch.Generator().manual_seed(8)
    z = (torch.randn(L, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    for kind in ("hcs", "hcm", "hcl"):
        prm = mixer_params(kind, H, 77, in_proj_fp8=False)
        pool = HyenaStatePool(2, H, "cpu")
        sw = prm["short_filter"].view(3 * H, 3)

        def run(zz, prm=prm, pool=pool, sw=sw, kind=kind):
            if kind == "hcl":
                oracle.iir_mixer_prefill(zz, sw, pool.conv_view(), prm["residues"],
                                         prm["log_poles"][..., 0], pool.ssm_view(), prm["D"],
                                         [0, zz.shape[0]], [1], [0])
            else:
                K = prm["conv"].shape[-1]
                oracle.fir_mixer_prefill(zz, sw, pool.conv_view(), prm["conv"].view(H, K),
                                         pool.inner_view(K - 1), prm.get("D"),
                                         [0, zz.shape[0]], [1], [0])
        with torch.inference_mode():
            run(z[:512])
            ts = []
            for _ in range(2):
                t = time.perf_counter()
                run(z)
                ts.append(time.perf_counter() - t)
                if time.perf_counter() - t_start > budget_s:
                    break
        sec = statistics.median(ts)
        pre[kind] = {"s": round(sec, 4), "tok_s": round(L / sec, 1)}
    step = 9 * sum(v["s"] for v in pre.values())
    out["prefill_7b"] = {"H": H, "L": L, "per_layer": pre,
                         "mixer_cores_tok_s": round(L / step, 1),
                         "note": f"27 mixer cores = 9 x (hcs + hcm + hcl), same scope as the "
                                 f"GPU prefill leg; L={L} of config 2's {L_PREFILL}"}
    dec, H, B = {}, 8192, 32
    for kind in ("hcs", "hcm", "hcl"):
        prm = mixer_params(kind, H, 78, in_proj_fp8=False)
        pool = HyenaStatePool(B + 1, H, "cpu")
        slots = random_slot_table(B, B + 1, 6)
        zz = (torch.randn(B, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
        sw = prm["short_filter"].view(3 * H, 3)
        if kind == "hcl":
            inner, lp, st = prm["residues"], prm["log_poles"][..., 0], pool.ssm_view()
        else:
            inner, lp, st = prm["conv"].view(H, -1), None, pool.inner_view()
        ts = []
        with torch.inference_mode():
            for _ in range(3):
                t = time.perf_counter()
                oracle.mixer_decode_unfused(zz, sw, pool.conv_view(), slots, inner, st,
                                            prm.get("D"), lp)
                ts.append(time.perf_counter() - t)
        sec = statistics.median(ts[1:])
        dec[kind] = {"s": round(sec, 4)}
    step = 14 * sum(v["s"] for v in dec.values())
    out["decode_40b"] = {"H": H, "B": B, "per_layer": dec, "mixer_cores_tok_s": round(B / step, 1),
                         "note": "42 mixer cores = 14 x (hcs + hcm + hcl) of the 40B layer map"}
    out["s"] = round(time.perf_counter() - t_start, 1)
    return out


def _guarded(fn, *a, **k):
    """A whole-model leg whose failure (e.g. out of memory on a busy device)
    is reported in the JSON line rather than ending the run."""
    try:
        return fn(*a, **k)
    except (RuntimeError, torch.OutOfMemoryError) as e:
        torch.cuda.empty_cache()
        return {"error": f"{type(e).__name__}: {str(e)[:300]}"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the fp8 GEMM leg")
    ap.add_argument("--no-verify", action="store_true", help="skip the speculative verify leg")
    ap.add_argument("--no-model", action="store_true", help="skip the whole-model decode leg")
    ap.add_argument("--no-model40b", action="store_true",
                    help="skip the 40B-shaped whole model (131072-token prefill, then B=32 "
                         "decode; ~20 s, ~150 GB of HBM)")
    ap.add_argument("--model-steps", type=int, default=STEPS_7B,
                    help="decode steps of the 7B whole-model leg (the workload's 512 by default; "
                         "fewer for profiling)")
    ap.add_argument("--only", choices=["decode", "verify", "prefill", "gemm", "copy", "model",
                                       "config0", "model_prefill", "model40b", "attn_prefill"],
                    default=None,
                    help="run one leg only (for profiling); `copy` runs a plain 1 GiB "
                         "device copy, the reference dispatch for scaling HBM counters")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the mixer path has no multi-GPU form "
              "(it would shard over sequences and channels). Run with --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = "cuda:0"
    if args.only == "copy":
        print(json.dumps(bench_copy(dev, reps=max(3, args.steps))), flush=True)
        return 0
    run = lambda leg, flag: (args.only == leg) or (args.only is None and not flag)  # noqa: E731
    dec = bench_decode(args.steps, args.warmup, dev) if run("decode", False) else None
    ver = bench_verify(max(8, args.steps // 2), dev) if run("verify", args.no_verify) else None
    pre = (bench_prefill(max(3, args.steps // 8), dev, warmup=args.warmup)
           if run("prefill", args.no_prefill) else None)
    gem = bench_gemm(max(5, args.steps // 4), dev) if run("gemm", args.no_gemm) else None
    cf0 = (bench_config0(max(5, args.steps // 4), dev, cpu=not (args.no_cpu or args.only))
           if run("config0", False) else None)
    mod = _guarded(bench_model, args.model_steps, dev) if run("model", args.no_model) else None
    mpre = _guarded(bench_model_prefill, dev) if run("model_prefill", args.no_model) else None
    # the 40B shape (64 heads, 131072 positions: ~0.8 s of torch's kernel) only when asked
    apre = (_guarded(bench_attn_prefill, dev, **({"shapes": ((32, L_PREFILL), (64, 131072))}
                                               if args.only == "attn_prefill" else {}))
            if run("attn_prefill", args.no_model) else None)
    m40 = (_guarded(bench_model40b, STEPS_40B, dev) if run("model40b", args.no_model or args.no_model40b)
           else None)
    if mod and "error" not in mod:
        # the reference's one published whole-step figure: a plain decode step
        # of the 7B model at batch 8 under full CUDA graphs, 7.85 ms on
        # H100/H200, context length not stated (api.py:384-385)
        mod["batch8"] = _guarded(bench_model, args.model_steps, dev, B=8)
        mod["batch8"]["reference"] = {"ms_per_step": 7.85, "hardware": "H100/H200",
                                      "source": "api.py:384-385",
                                      "note": "plain decode, whole 7B model, batch 8; "
                                              "context length not stated"}
    cpu = None if (args.no_cpu or args.only) else _cpu_baseline_decode()
    if cpu is not None:
        cpu["configs"] = _cpu_baseline_layers()
    line = {
        "metric": METRIC,
        "value": round(dec["tok_s"], 1) if dec else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4) if dec else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 I/O, fp32 arithmetic",
        "data": "synthetic (seeded random states, z rows and weights)",
        "config": {"workload": "7B-shape Hyena decode: 27 mixer cores (9 hcs, 9 hcm, 9 hcl), "
                               "H=4096, B=64, paged state (page per block, random slot table), "
                               "one fused decode kernel per layer",
                   "global_batch": B_DECODE, "H": H_7B, "layers": 27,
                   "replay": "one HIP graph per step"},
    }
    if dec:
        hcm = dec["per_kind"]["hcm"]
        line["roofline"] = {"bound": "hbm", "kernel": DECODE_ROOFLINE_KERNEL,
                            "achieved": hcm["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": hcm["frac"],
                            "traffic": profiled_traffic(DECODE_ROOFLINE_KERNEL)}
        line["decode"] = dec
    if ver:
        line["verify"] = ver
    if pre:
        line["prefill"] = pre
    if gem:
        line["fp8_gemm"] = gem
    if mod:
        line["model_decode"] = mod
    if mpre:
        if pre and "error" not in mpre:  # the 27 mixer cores of this run's prefill leg, as a share
            mpre["mixer_core_us"] = pre["us_per_step"]
            mpre["mixer_core_share"] = round(pre["us_per_step"] / (mpre["ms"] * 1e3), 4)
        line["model_prefill"] = mpre
    if apre:
        line["attn_prefill"] = apre
    if m40:
        line["model_40b"] = m40
    if cf0:
        line["config0_prefill"] = cf0
    if not args.only:
        line["hbm_copy"] = bench_copy(dev)
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
