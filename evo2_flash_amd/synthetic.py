"""Seeded synthetic weights and inputs for the Hyena mixers.

Distributions follow the benchmark specification of this build:
  projections ~ N(0, 0.02); hcs taps (K=7) ~ N(0, 0.1); hcm taps (K=128)
  ~ N(0, 0.1) times a decay envelope largest at w[:, -1] (lag 0, the
  cross-correlation order of convert.py:486-494); hcl: 16 real poles per
  channel with p log-uniform in (0.5, 0.999), lp = log p in fp32, residues
  ~ N(0, 0.1); D ~ N(0, 1); short filter ~ N(0, 0.3).
  fp8 scales are per-tensor dequantisation scales amax/448 (convert.py:195-201).
Tokens are uniform over the bytes A, C, G, T.
"""

import math

import torch

FP8_MAX = 448.0
ACGT = torch.tensor([65, 67, 71, 84], dtype=torch.long)

# Static activation scale: in_proj inputs are RMS-normalised rows, |x| < ~6.
DEFAULT_INPUT_AMAX = 6.0


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def quantize_weight_e4m3(w):
    """(e4m3 weight, dequantisation scale) with a per-tensor amax scale."""
    amax = w.abs().max().float().clamp_min(1e-12)
    scale = (amax / FP8_MAX).reshape(1)
    w8 = (w.float() / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return w8, scale.to(torch.float32)


def mixer_params(kind, hidden, seed, device="cpu", k_hcs=7, k_hcm=128, state_size=16,
                 in_proj_fp8=True, input_amax=DEFAULT_INPUT_AMAX):
    """Parameters of one Hyena mixer under the reference's names (mixers.py:714-821,
    1241-1250, 1317-1325): in_proj.{weight,weight_scale,input_scale},
    short_filter (3H,1,3), conv (H,1,K) | log_poles (H,S,1) + residues (H,S),
    D (H,) for hcm/hcl, out_proj.{weight,bias}."""
    assert kind in ("hcs", "hcm", "hcl")
    H = hidden
    g = _gen(seed, device)
    bf16 = torch.bfloat16
    p = {}
    w_in = torch.randn(3 * H, H, generator=g, device=device) * 0.02
    if in_proj_fp8:
        w8, sw = quantize_weight_e4m3(w_in)
        p["in_proj.weight"] = w8
        p["in_proj.weight_scale"] = sw
        p["in_proj.input_scale"] = torch.full((1,), input_amax / FP8_MAX, device=device)
    else:
        p["in_proj.weight"] = w_in.to(bf16)
    del w_in
    p["short_filter"] = (torch.randn(3 * H, 1, 3, generator=g, device=device) * 0.3).to(bf16)
    if kind == "hcl":
        lo, hi = math.log(0.5), math.log(0.999)
        lp = lo + (hi - lo) * torch.rand(H, state_size, generator=g, device=device)
        p["log_poles"] = lp.float().unsqueeze(-1).contiguous()
        p["residues"] = (torch.randn(H, state_size, generator=g, device=device) * 0.1).float()
    else:
        K = k_hcs if kind == "hcs" else k_hcm
        w = torch.randn(H, 1, K, generator=g, device=device) * 0.1
        if kind == "hcm":
            lag = torch.arange(K - 1, -1, -1, device=device, dtype=torch.float32)
            w = w * torch.exp(-lag / 32.0)
        p["conv"] = w.to(bf16)
    if kind in ("hcm", "hcl"):
        p["D"] = torch.randn(H, generator=g, device=device).to(bf16)
    p["out_proj.weight"] = (torch.randn(H, H, generator=g, device=device) * 0.02).to(bf16)
    p["out_proj.bias"] = (torch.randn(H, generator=g, device=device) * 0.02).to(bf16)
    return p


def acgt_tokens(n, seed, device="cpu"):
    """n tokens uniform over {A, C, G, T} as byte ids."""
    g = _gen(seed, "cpu")
    idx = torch.randint(0, 4, (n,), generator=g)
    return ACGT[idx].to(device)


def random_slot_table(n_rows, num_blocks, seed, device="cpu"):
    """Distinct state blocks for n_rows rows: a seeded random permutation of
    blocks 1..num_blocks-1 (block 0 is the null block), as int32."""
    if n_rows > num_blocks - 1:
        raise ValueError(f"{n_rows} rows need more than {num_blocks - 1} usable blocks")
    g = _gen(seed, "cpu")
    perm = torch.randperm(num_blocks - 1, generator=g)[:n_rows] + 1
    return perm.to(torch.int32).to(device)
