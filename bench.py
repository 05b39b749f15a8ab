#!/usr/bin/env python3
"""Throughput of the Evo 2 Hyena mixer hot path on one MI355X.

Workload (the headline): 7B-shaped decode, the 27 Hyena mixers of the 7B
layer map (9 hcs, 9 hcm, 9 hcl; H=4096), batch 64, paged state in a
vLLM-layout pool with a seeded random slot table.  One step = one token for
all 64 sequences through every mixer.  Inputs are resident in HBM before the
timed region.  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

H_7B = 4096
B_DECODE = 64
LAYER_MAP_7B = {  # evo2_configs/evo2-7b-1m.yml:7-10
    "hcs": [0, 4, 7, 11, 14, 18, 21, 25, 28],
    "hcm": [1, 5, 8, 12, 15, 19, 22, 26, 29],
    "hcl": [2, 6, 9, 13, 16, 20, 23, 27, 30],
}
HBM_PEAK_GBS = 8000.0


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


class DecodeLayer:
    def __init__(self, kind, idx, H, B, dev, seed):
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
            self.inner = prm["conv"].view(H, K)
            self.lp = None
        self.pool = HyenaStatePool(B + 1, H, dev)
        g = torch.Generator(device=dev).manual_seed(seed + 1000 + idx)
        self.pool.kv_cache[0].copy_(torch.randn(self.pool.kv_cache[0].shape, generator=g,
                                                device=dev).to(torch.bfloat16))
        self.pool.kv_cache[1].copy_(torch.randn(self.pool.kv_cache[1].shape, generator=g,
                                                device=dev))
        self.pool.kv_cache[2].copy_(torch.randn(self.pool.kv_cache[2].shape, generator=g,
                                                device=dev))
        self.state = (self.pool.ssm_view() if kind == "hcl"
                      else self.pool.inner_view(self.inner.shape[1] - 1))
        self.slots = random_slot_table(B, B + 1, seed + 2000 + idx, device=dev)
        self.z = (torch.randn(B, 3 * H, generator=g, device=dev) * 1.3).to(torch.bfloat16)

    def step(self):
        from evo2_flash_amd.decode import hyena_decode

        return hyena_decode(self.z, self.short_w, self.pool.conv_view(), self.slots,
                            self.inner, self.state, self.D, self.lp)


def bench_decode(steps, warmup, dev, seed=1234):
    H, B = H_7B, B_DECODE
    order = sorted((i, k) for k, idxs in LAYER_MAP_7B.items() for i in idxs)
    layers = [DecodeLayer(k, i, H, B, dev, seed) for i, k in order]
    for _ in range(warmup):
        for L in layers:
            L.step()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    ev = {k: [] for k in LAYER_MAP_7B}
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(steps):
        for L in layers:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            L.step()
            b.record(stream)
            ev[L.kind].append((a, b))
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    per_kind = {}
    for k, pairs in ev.items():
        durs = [a.elapsed_time(b) * 1e3 for a, b in pairs]  # us
        nbytes = decode_bytes_per_launch(k, B, H)
        avg = statistics.mean(durs)
        per_kind[k] = {"avg_us": round(avg, 3), "median_us": round(statistics.median(durs), 3),
                       "bytes_per_launch": nbytes,
                       "achieved_GBs": round(nbytes / (avg * 1e-6) / 1e9, 1)}
    ms_per_step = total_ms / steps
    return {"ms_per_step": ms_per_step, "tok_s": B / (ms_per_step * 1e-3), "per_kind": per_kind,
            "layers": len(layers)}


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
            for rep in range(4):
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


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the sharding design is described in DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = "cuda:0"
    dec = bench_decode(args.steps, args.warmup, dev)
    hcm = dec["per_kind"]["hcm"]
    cpu = None if args.no_cpu else _cpu_baseline_decode()
    line = {
        "metric": "decode tok/s (7B-shape, bs=64) + prefill tok/s at 32k; % HBM/MFMA roofline",
        "value": round(dec["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16/fp32",
        "data": "synthetic (seeded random states, z rows and weights)",
        "config": {"workload": "7B-shape Hyena decode: 27 mixer cores (9 hcs, 9 hcm, 9 hcl), "
                               "H=4096, B=64, paged state, fused decode kernel per layer",
                   "global_batch": B_DECODE, "H": H_7B, "layers": dec["layers"]},
        "roofline": {"bound": "hbm", "kernel": "hyena_decode_kernel<hcm>",
                     "achieved": hcm["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(hcm["achieved_GBs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "per_kind": dec["per_kind"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
