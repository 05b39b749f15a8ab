"""Decode attention of the whole-model harness (attention.py, csrc/attention.hip)
against plain fp32 attention on the CPU: out = softmax(scale q.k) v over cache
positions 0..positions[b].  Bar: max |out - ref| / max |ref| <= 1e-2 per case
(the kernel's output is bf16, ~4e-3 relative rounding).  Cases: head_dim 64 and
128; contexts of one and several 2048-position chunks; lengths ending inside a
chunk, at a chunk edge and at the cache end; a batch slice of a larger cache
(the harness's k_cache[:B]); the 7B attention shape (32 heads of 128) at the
benchmark's context; a prompt's pages shared by every sequence, with and
without the sharing declared (head_dim 64: bitwise the same; 128, the
matrix-core kernel: within a bf16 rounding step of the undeclared result,
nearly all elements the same bits), for one partial and two groups of 32
sequences.  Causal prefill attention (head_dim 128, the matrix-core kernel)
against fp32 attention on the CPU at several prompt lengths, and with
peaked scores.
"""

import pytest
import torch

from evo2_flash_amd.attention import (PAGE, PagedKVCache, decode_attention,
                                     paged_decode_attention, shared_prefix_pages, workspace)

from _cases import max_rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
bf = torch.bfloat16


def _ref(q, k, v, pos, scale):
    B, nh, hd = q.shape
    out = torch.empty(B, nh, hd)
    for b in range(B):
        n = int(pos[b]) + 1
        s = torch.einsum("hd,hdl->hl", q[b].float(), k[b, :, :, :n].float()) * scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.einsum("hl,hld->hd", p, v[b, :, :n].float())
    return out


@pytest.mark.parametrize("hd,L,pos", [(64, 16, [15, 0, 7]), (128, 4104, [4103, 5, 2047, 2048]),
                                      (64, 2056, [2055, 1000])])
def test_decode_attention_vs_fp32(hd, L, pos):
    g = torch.Generator().manual_seed(hd + L)
    B, nh, maxb = len(pos), 4, len(pos) + 2
    q = torch.randn(B, nh, hd, generator=g).to(bf)
    kc = torch.randn(maxb, nh, hd, L, generator=g).to(bf)      # head_dim-major keys
    vc = torch.randn(maxb, nh, L, hd, generator=g).to(bf)
    positions = torch.tensor(pos, dtype=torch.int64)
    scale = hd ** -0.5
    ref = _ref(q, kc[:B], vc[:B], positions, scale)
    kd, vd = kc.to(DEV), vc.to(DEV)
    ws = workspace(maxb, nh, hd, L, DEV)
    print(f"decode_attention hd={hd} L={L} pos={pos}", flush=True)
    out = decode_attention(q.to(DEV), kd[:B], vd[:B], positions.to(DEV), scale, ws)
    assert out.dtype == bf and out.shape == (B, nh, hd)
    assert max_rel_err(out.cpu(), ref) <= 1e-2


def test_decode_attention_7b_shape():
    """32 heads of 128 at the 7B benchmark's context (8192 prompt + 512 steps)."""
    g = torch.Generator().manual_seed(7)
    B, nh, hd, L = 3, 32, 128, 8704
    q = torch.randn(B, nh, hd, generator=g).to(bf)
    kc = (torch.randn(B, nh, hd, L, generator=g) * 0.5).to(bf)
    vc = (torch.randn(B, nh, L, hd, generator=g) * 0.5).to(bf)
    positions = torch.tensor([8192, 8703, 3000], dtype=torch.int64)
    ref = _ref(q, kc, vc, positions, hd ** -0.5)
    print("decode_attention 7B shape", flush=True)
    out = decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), positions.to(DEV), hd ** -0.5)
    assert max_rel_err(out.cpu(), ref) <= 1e-2


@pytest.mark.parametrize("hd,max_pages,pos", [(64, 3, [47, 0, 16, 15]),
                                              (128, 260, [4159, 2047, 2048, 100]),
                                              (128, 544, [8192, 8703, 17])])
def test_paged_decode_attention_vs_fp32(hd, max_pages, pos):
    """The cache in 16-position pages of a random block table (page 0 never
    used): the same attention as over the dense cache the pages hold."""
    g = torch.Generator().manual_seed(hd + max_pages)
    B, nh = len(pos), 4 if hd == 64 else 32
    num_pages = B * max_pages + 5
    table = (torch.randperm(num_pages - 1, generator=g)[:B * max_pages] + 1).to(torch.int32)
    table = table.view(B, max_pages)
    cache = PagedKVCache(num_pages, nh, hd, "cpu")
    cache.k.copy_((torch.randn(cache.k.shape, generator=g) * 0.5).to(bf))
    cache.v.copy_((torch.randn(cache.v.shape, generator=g) * 0.5).to(bf))
    q = torch.randn(B, nh, hd, generator=g).to(bf)
    positions = torch.tensor(pos, dtype=torch.int64)
    kd, vd = cache.dense(table, B, max_pages * PAGE)
    ref = _ref(q, kd, vd, positions, hd ** -0.5)
    print(f"paged decode_attention hd={hd} pages={max_pages} pos={pos}", flush=True)
    out = paged_decode_attention(q.to(DEV), cache.k.to(DEV), cache.v.to(DEV), table.to(DEV),
                                 positions.to(DEV), hd ** -0.5)
    assert out.shape == (B, nh, hd)
    assert max_rel_err(out.cpu(), ref) <= 1e-2


@pytest.mark.parametrize("hd", [64, 128])
def test_paged_decode_attention_masks_entries_outside_the_cache(hd):
    """Table entries outside [0, pages) (-1, pages, a large id) are never read
    through: their positions drop out of the softmax, and a sequence with no
    position left gets zeros (head_dim 64: the VALU kernel; 128: the
    matrix-core kernel)."""
    g = torch.Generator().manual_seed(3)
    nh, max_pages = 4, 140
    pos = [2239, 2239, 300, 40]
    B = len(pos)
    num_pages = B * max_pages + 1
    table = (torch.randperm(num_pages - 1, generator=g)[:B * max_pages] + 1).to(torch.int32)
    table = table.view(B, max_pages).clone()
    table[0, 5] = -1
    table[0, 130] = num_pages            # in the second 2048-position chunk
    table[1, :128] = 1 << 30             # the whole first chunk of sequence 1
    table[2, 3] = -7
    table[3, :3] = -1                    # every page sequence 3 uses
    cache = PagedKVCache(num_pages, nh, hd, "cpu")
    cache.k.copy_((torch.randn(cache.k.shape, generator=g) * 0.5).to(bf))
    cache.v.copy_((torch.randn(cache.v.shape, generator=g) * 0.5).to(bf))
    q = torch.randn(B, nh, hd, generator=g).to(bf)
    positions = torch.tensor(pos, dtype=torch.int64)
    ref = torch.zeros(B, nh, hd)
    for b in range(B):
        keep = [l for l in range(pos[b] + 1) if 0 <= int(table[b, l // PAGE]) < num_pages]
        if not keep:
            continue
        pg = table[b, [l // PAGE for l in keep]].long()
        off = torch.tensor([l % PAGE for l in keep])
        k = cache.k[pg, :, :, off].float()          # (n, heads, hd)
        v = cache.v[pg, :, off, :].float()          # (n, heads, hd)
        s = torch.einsum("hd,nhd->hn", q[b].float(), k) * hd ** -0.5
        ref[b] = torch.einsum("hn,nhd->hd", torch.softmax(s, dim=-1), v)
    print(f"paged decode_attention masked table entries hd={hd}", flush=True)
    out = paged_decode_attention(q.to(DEV), cache.k.to(DEV), cache.v.to(DEV), table.to(DEV),
                                 positions.to(DEV), hd ** -0.5).cpu()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out[3], torch.zeros(nh, hd, dtype=bf))
    assert max_rel_err(out[:3], ref[:3]) <= 1e-2


@pytest.mark.parametrize("B,hd", [(6, 128), (8, 128), (40, 128), (8, 64)])
def test_paged_decode_attention_shared_prompt(B, hd):
    """Rows sharing their first pages (one prompt behind every sequence), one
    shared entry masked, sequences shorter than the shared prompt.  With the
    sharing declared, the chunks inside the prompt read each page once for
    several sequences: at head_dim 64 four sequences per workgroup on the
    VALU, the same bits as without it; at 128 up to 32 per workgroup on the
    matrix cores (another order of the fp32 sums, the probabilities as bf16
    high and low parts), within a rounding step of the undeclared result.
    Both match fp32 attention over the pages."""
    g = torch.Generator().manual_seed(11 + B + hd)
    nh, sp, own = 4, 392, 24                   # 392 shared pages: three whole chunks and a part
    max_pages = sp + own
    num_pages = sp + B * own + 1
    perm = torch.randperm(num_pages - 1, generator=g) + 1
    table = torch.empty(B, max_pages, dtype=torch.int32)
    table[:, :sp] = perm[:sp].to(torch.int32)
    table[:, sp:] = perm[sp:].to(torch.int32).view(B, own)
    table[:, 70] = -1                           # masked for every sequence (inside chunk 0)
    pos = [sp * PAGE + 5, max_pages * PAGE - 1, 5000, sp * PAGE + 300, 4095, 2047, 6300, 6271]
    pos = (pos + torch.randint(0, max_pages * PAGE, (max(B - len(pos), 0),), generator=g).tolist())[:B]
    cache = PagedKVCache(num_pages, nh, hd, "cpu")
    cache.k.copy_((torch.randn(cache.k.shape, generator=g) * 0.5).to(bf))
    cache.v.copy_((torch.randn(cache.v.shape, generator=g) * 0.5).to(bf))
    q = torch.randn(B, nh, hd, generator=g).to(bf)
    positions = torch.tensor(pos, dtype=torch.int64)
    assert shared_prefix_pages(table, B) == sp
    ref = torch.zeros(B, nh, hd)
    for b in range(B):
        keep = [l for l in range(pos[b] + 1) if int(table[b, l // PAGE]) >= 0]
        pg = table[b, [l // PAGE for l in keep]].long()
        off = torch.tensor([l % PAGE for l in keep])
        k = cache.k[pg, :, :, off].float()
        v = cache.v[pg, :, off, :].float()
        s = torch.einsum("hd,nhd->hn", q[b].float(), k) * hd ** -0.5
        ref[b] = torch.einsum("hn,nhd->hd", torch.softmax(s, dim=-1), v)
    args = (q.to(DEV), cache.k.to(DEV), cache.v.to(DEV), table.to(DEV), positions.to(DEV), hd ** -0.5)
    print(f"paged decode_attention shared prompt B={B} hd={hd}", flush=True)
    plain = paged_decode_attention(*args).cpu()
    shared = paged_decode_attention(*args, shared_pages=sp).cpu()
    if hd == 64:
        assert torch.equal(plain.view(torch.int16), shared.view(torch.int16))
    else:
        pf, sf = plain.float(), shared.float()
        # one bf16 step is at most 2^-7 of the value
        assert ((sf - pf).abs() <= pf.abs() * 2.0 ** -7 + 1e-4 * pf.abs().max()).all()
        assert (plain.view(torch.int16) != shared.view(torch.int16)).float().mean() <= 0.01
    assert max_rel_err(shared, ref) <= 1e-2
    assert max_rel_err(plain, ref) <= 1e-2


def _causal_ref(q, k, v, scale):
    """fp32 causal attention on the CPU: (N, heads, L, hd)."""
    qf, kf, vf = q.float(), k.float(), v.float()
    L = q.shape[-2]
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    s.masked_fill_(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vf)


@pytest.mark.parametrize("N,nh,L", [(1, 2, 8), (2, 3, 200), (1, 2, 392), (1, 4, 1024), (1, 2, 4104),
                                    (1, 8, 1032), (2, 16, 520)])
def test_prefill_attention_vs_fp32(N, nh, L):
    """Causal prefill attention on the matrix-core kernel against fp32
    attention on the CPU: one partial 256-query block, several, prompts
    ending inside a key block, a prompt past 4096 (the last query block
    partly outside it), and head counts that split over the eight XCDs (the
    head-per-XCD grid), with two sequences.  Bar 1e-2 (bf16 output and bf16
    softmax weights)."""
    from evo2_flash_amd.attention import prefill_attention
    g = torch.Generator().manual_seed(L + nh)
    hd = 128
    q = torch.randn(N, nh, L, hd, generator=g).to(bf)
    k = torch.randn(N, nh, L, hd, generator=g).to(bf)
    v = torch.randn(N, nh, L, hd, generator=g).to(bf)
    ref = _causal_ref(q, k, v, hd ** -0.5)
    print(f"prefill_attention N={N} heads={nh} L={L}", flush=True)
    out = prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5).cpu()
    assert out.shape == q.shape and out.dtype == bf
    assert torch.isfinite(out.float()).all()
    assert max_rel_err(out, ref) <= 1e-2


def test_prefill_attention_peaked_scores():
    """Large scores (a softmax close to one-hot, and rows whose running max
    jumps late in the sweep): the online rescaling keeps the sums exact
    enough."""
    from evo2_flash_amd.attention import prefill_attention
    g = torch.Generator().manual_seed(5)
    N, nh, L, hd = 1, 2, 640, 128
    q = (torch.randn(N, nh, L, hd, generator=g) * 4).to(bf)
    k = (torch.randn(N, nh, L, hd, generator=g) * 4).to(bf)
    k[:, :, 600] *= 3                  # a late key that dominates the rows after it
    v = torch.randn(N, nh, L, hd, generator=g).to(bf)
    ref = _causal_ref(q, k, v, hd ** -0.5)
    print("prefill_attention peaked scores", flush=True)
    out = prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5).cpu()
    assert max_rel_err(out, ref) <= 1e-2
