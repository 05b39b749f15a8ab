"""Seeded test cases shared by the CPU and GPU tests."""

import torch

from evo2_flash_amd.state import HyenaStatePool
from evo2_flash_amd.synthetic import mixer_params, random_slot_table


def bf16_ulp_diff(a, b):
    """Per-element distance in bf16 units in the last place (same-sign values)."""
    ai = a.contiguous().view(torch.int16).to(torch.int32)
    bi = b.contiguous().view(torch.int16).to(torch.int32)
    # map sign-magnitude to a monotone integer line
    ai = torch.where(ai < 0, -32768 - ai, ai)
    bi = torch.where(bi < 0, -32768 - bi, bi)
    return (ai - bi).abs()


def max_rel_err(out, ref):
    """max|out - ref| / max|ref| in fp32 (the tolerance norm of the mixer tests)."""
    out = out.float()
    ref = ref.float()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def random_pool(num_blocks, H, seed, device="cpu"):
    """A state pool filled with seeded values of the right kind per slice:
    conv windows hold bf16 projections, FIR windows bf16-valued u's in fp32,
    LI states fp32 of magnitude ~10."""
    g = torch.Generator().manual_seed(seed)
    pool = HyenaStatePool(num_blocks, H, "cpu")
    conv = pool.kv_cache[0]
    conv.copy_(torch.randn(conv.shape, generator=g).to(conv.dtype))
    inner = pool.kv_cache[1]
    inner.copy_(torch.randn(inner.shape, generator=g).to(torch.bfloat16).float())
    ssm = pool.kv_cache[2]
    ssm.copy_(torch.randn(ssm.shape, generator=g) * 10.0)
    if device != "cpu":
        gp = HyenaStatePool(num_blocks, H, device)
        gp.raw.copy_(pool.raw)
        return pool, gp
    return pool


def clone_pool(pool, device):
    p = HyenaStatePool(pool.num_blocks, pool.hidden, device)
    p.raw.copy_(pool.raw)
    return p


def decode_case(kind, H, B, num_blocks, seed, n_null=0):
    """CPU tensors for one decode step: params, z, slots (some null rows), pool."""
    prm = mixer_params(kind, H, seed, in_proj_fp8=False)
    g = torch.Generator().manual_seed(seed + 1)
    z = (torch.randn(B, 3 * H, generator=g) * 1.3).to(torch.bfloat16)
    slots = random_slot_table(B, num_blocks, seed + 2)
    if n_null:
        rows = torch.randperm(B, generator=g)[:n_null]
        slots[rows] = 0
    pool = random_pool(num_blocks, H, seed + 3)
    return prm, z, slots, pool
