"""GPU parity of the fp8 e4m3 projection kernels.

* activation quantisation bit-exact against torch's e4m3fn conversion of
  clamp(x / s, +-448) (fp8_emul.py:76-78), including saturation and ties;
* GEMM known answers: small-integer e4m3 operands whose fp32 sums are exact,
  so the bf16 output must equal the oracle bit for bit, on each kernel: the
  decode-sized one (also gridded over blocks of 64 rows), the 256x256 tile
  one and its persistent form (whole tiles, at least one per CU), in both tile orders
  of the latter (XCD
  blocks of 4 x 8 tiles, whole rounds and a part-filled last round, and
  row-major with some workgroups taking one tile more);
* GEMM within 2e-2 max relative error of the dequantised bf16 reference on
  random operands, at ragged shapes, at decode sizes (M <= 64, the 7B and
  40B in_proj) and at both config-3 shapes (M=8192, K=4096 -> N=12288 and
  N=4096).
"""

import pytest
import torch

import oracle
from evo2_flash_amd.fp8 import fp8_gemm, quantize_input, static_fp8_linear
from evo2_flash_amd.synthetic import quantize_weight_e4m3

from _cases import max_rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
E4M3 = torch.float8_e4m3fn


@pytest.mark.parametrize("rows,K,row_stride", [(4, 1027, None),    # 4-element kernel
                                              (4, 1024, None),    # 16-element kernel
                                              (3, 4096, 4104),    # strided rows, 16-element
                                              (3, 4096, 4100)])   # rows not 16-byte aligned
def test_quantize_bitexact(rows, K, row_stride):
    g = torch.Generator().manual_seed(0)
    n = rows * K
    special = torch.tensor([0.0, -0.0, 1e-9, 448.0, 449.0, -1e4, 1e4, 0.0087890625,
                            0.009765625, 240.0, 248.0, 256.0])
    x = torch.cat([torch.randn(n - special.numel(), generator=g) * 3, special])
    x = x[torch.randperm(n, generator=g)].to(torch.bfloat16).reshape(rows, K)
    scale = torch.tensor([0.75])
    xd = x.to(DEV)
    if row_stride is not None:
        wide = torch.zeros(rows, row_stride, dtype=torch.bfloat16, device=DEV)
        wide[:, :K] = xd
        xd = wide[:, :K]
    q = quantize_input(xd, scale.to(DEV)).cpu()
    ref = oracle.quantize_input(x, scale)
    assert torch.equal(q.view(torch.uint8), ref.view(torch.uint8))


def _small_int_e4m3(shape, g):
    return (torch.randint(-6, 7, shape, generator=g).float()).to(E4M3)


# With K a multiple of 128 the weight-streaming kernel takes M <= 64, and
# larger M over blocks of 64 rows while ceil(M / 64) x N <= 60000 (16 W rows
# per wave in registers, 16x16x128 MFMA, the blocks of one weight slice on
# one XCD); the others run the 256x256-tile kernel (K = 192 here, or too much
# work).
@pytest.mark.parametrize("M,N,K", [(64, 384, 256), (1, 64, 128), (5, 130, 1920),
                                   (64, 4096, 4096),                      # one row block
                                   (65, 200, 256), (130, 96, 384), (300, 512, 1920),
                                   (1000, 130, 640), (128, 12288, 256), (100, 10000, 384),
                                   (192, 12288, 256), (170, 12000, 256),
                                   (256, 12288, 512),                     # gridded over M
                                   (256, 256, 192), (1100, 6400, 640),
                                   (500, 12288, 256)])                    # 256x256 tiles
def test_gemm_known_answer(M, N, K):
    g = torch.Generator().manual_seed(M + N)
    x8 = _small_int_e4m3((M, K), g)
    w8 = _small_int_e4m3((N, K), g)
    xs, ws = torch.tensor([0.5]), torch.tensor([0.25])
    out = fp8_gemm(x8.to(DEV), w8.to(DEV), xs.to(DEV), ws.to(DEV)).cpu()
    acc = x8.float().double() @ w8.float().double().t()   # exact
    ref = (acc.float() * 0.5 * 0.25).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


# Persistent 256x256 form: (2048, 8192) has 8 x 32 tiles (the XCD-block
# order); (2048, 12288) has 8 x 48 = 384 tiles, twelve blocks of 4 x 8, so
# the XCD-block order's second round is half full and its last four blocks
# go out tile by tile; (3328, 5120) has 13 x 20 = 260 tiles over 256
# workgroups (row-major order, four workgroups take a second tile);
# (2048, 12288, 256) has tiles of one slice pair, the one that starts the
# accumulators.
@pytest.mark.parametrize("M,N,K", [(2048, 8192, 512), (2048, 12288, 512), (3328, 5120, 768),
                                   (2048, 12288, 256)])
def test_gemm_known_answer_persistent(M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    x8 = _small_int_e4m3((M, K), g)
    w8 = _small_int_e4m3((N, K), g)
    xs, ws = torch.tensor([0.5]), torch.tensor([0.25])
    print(f"persistent gemm M={M} N={N} K={K}", flush=True)
    out = fp8_gemm(x8.to(DEV), w8.to(DEV), xs.to(DEV), ws.to(DEV)).cpu()
    acc = x8.float() @ w8.float().t()   # exact: |sums| < 2^24
    ref = (acc * 0.5 * 0.25).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_static_linear_persistent_with_bias():
    M, N, K = 4096, 4096, 1024   # 16 x 16 tiles
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=g) * 0.02)
    xs = torch.tensor([6.0 / 448])
    bias = (torch.randn(N, generator=g) * 0.02).to(torch.bfloat16)
    out = static_fp8_linear(x.to(DEV), w8.to(DEV), xs.to(DEV), ws.to(DEV), bias.to(DEV)).cpu()
    ref = oracle.fp8_linear_dequant(x, w8, xs, ws, bias)
    assert max_rel_err(out, ref) <= 2e-2


@pytest.mark.parametrize("M,N,K", [(64, 12288, 4096), (333, 4096, 4096), (1000, 640, 1920),
                                   (1, 12288, 4096), (37, 200, 1920), (64, 16384, 8192),
                                   (48, 256, 192)])
def test_static_linear_vs_dequant(M, N, K):
    g = torch.Generator().manual_seed(K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=g) * 0.02)
    xs = torch.tensor([6.0 / 448])
    bias = (torch.randn(N, generator=g) * 0.02).to(torch.bfloat16)
    out = static_fp8_linear(x.to(DEV), w8.to(DEV), xs.to(DEV), ws.to(DEV), bias.to(DEV)).cpu()
    ref = oracle.fp8_linear_dequant(x, w8, xs, ws, bias)
    assert max_rel_err(out, ref) <= 2e-2


@pytest.mark.parametrize("N", [12288, 4096])
def test_config3_shapes(N):
    """M=8192 tokens ~N(0,1) quantised with a per-tensor amax scale, weights
    ~N(0,0.02); compared with the dequantised matmul in fp32 on the GPU."""
    M, K = 8192, 4096
    gen = torch.Generator(device=DEV).manual_seed(N)
    x = torch.randn(M, K, generator=gen, device=DEV).to(torch.bfloat16)
    xs = (x.float().abs().max() / 448.0).reshape(1)
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)
    x8 = quantize_input(x, xs)
    out = fp8_gemm(x8, w8, xs, ws)
    ref = (x8.float() @ w8.float().t()) * (xs * ws)
    assert max_rel_err(out, ref) <= 2e-2
    # the dequantised reference bf16((A8 s_a) @ (W8 s_w)^T), operands rounded to bf16 first
    ref_bf = ((x8.float() * xs).to(torch.bfloat16).float() @ (w8.float() * ws).to(torch.bfloat16).float().t())
    assert max_rel_err(out, ref_bf) <= 2e-2


@pytest.mark.parametrize("M,N,K", [(64, 12288, 4096), (1, 48, 128), (7, 4112, 256),
                                   (64, 4096, 4096), (100, 512, 384), (32, 24576, 8192),
                                   (256, 12288, 4096)])
def test_packed_weight_same_bits(M, N, K):
    """The decode weight layout (fp8_pack_weight) read by fp8_gemm_packed
    gives the unpacked GEMM's bits, at decode shapes, at N not a multiple of
    any workgroup's row count (the clamped last row group) and at M > 64
    (two row blocks); and its bytes are the documented permutation."""
    from evo2_flash_amd.fp8 import fp8_gemm_packed, fp8_pack_weight
    gen = torch.Generator(device=DEV).manual_seed(M + N)
    x8 = (torch.randn(M, K, generator=gen, device=DEV) * 2).to(E4M3)
    w8 = (torch.randn(N, K, generator=gen, device=DEV) * 0.5).to(E4M3)
    xs = torch.tensor([0.7], device=DEV)
    ws = torch.tensor([0.3], device=DEV)
    bias = (torch.randn(N, generator=gen, device=DEV) * 0.1).to(torch.bfloat16)
    wp = fp8_pack_weight(w8)
    perm = w8.view(torch.uint8).view(N // 16, 16, K // 128, 4, 2, 16).permute(0, 2, 4, 3, 1, 5)
    assert torch.equal(wp.view(torch.uint8).view(-1), perm.reshape(-1))
    for b in (None, bias):
        ref = fp8_gemm(x8, w8, xs, ws, b)
        out = fp8_gemm_packed(x8, wp, xs, ws, b)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_linear_module_decode_copy():
    """Fp8StaticLinear takes its packed copy where the GEMM streams the weight
    (decode and verify-sized inputs), the row-major weight above; same bits;
    the copy follows an in-place weight update."""
    from evo2_flash_amd.fp8 import Fp8StaticLinear
    N, K = 4096, 1024
    lin = Fp8StaticLinear(K, N, bias=True, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(5)
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)
    with torch.no_grad():
        lin.weight.copy_(w8)
        lin.weight_scale.copy_(ws)
        lin.input_scale.fill_(6.0 / 448)
        lin.bias.copy_((torch.randn(N, generator=gen, device=DEV) * 0.02).to(torch.bfloat16))
    for M in (1, 64, 65, 2000):
        x = torch.randn(M, K, generator=gen, device=DEV).to(torch.bfloat16)
        y, _ = lin(x)
        ref = static_fp8_linear(x, lin.weight, lin.input_scale, lin.weight_scale, lin.bias)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), M
    first = lin.decode_weight()
    assert first is not None and lin.decode_weight() is first
    w2, _ = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)
    with torch.no_grad():
        lin.weight.copy_(w2)
    x = torch.randn(8, K, generator=gen, device=DEV).to(torch.bfloat16)
    y, _ = lin(x)
    ref = static_fp8_linear(x, lin.weight, lin.input_scale, lin.weight_scale, lin.bias)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    assert lin.decode_weight() is first  # rewritten into the same buffer
    # the engine's loader path and a write through .data (which leaves the
    # version counter alone) followed by refresh_decode_weight()
    kept = lin.decode_weight()
    for load in ("loader", "data"):
        w3, _ = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)
        if load == "loader":
            lin.weight.weight_loader(lin.weight, w3)
        else:
            lin.weight.data.copy_(w3)
            lin.refresh_decode_weight()
        assert lin.decode_weight() is kept  # rewritten in place
        y, _ = lin(x)
        ref = static_fp8_linear(x, lin.weight, lin.input_scale, lin.weight_scale, lin.bias)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), load


def test_linear_decode_copy_in_graph():
    """A HIP graph captured on the packed decode GEMM replays the eager
    result, and after a reload through the weight's loader (which rewrites
    the copy in place) it computes with the new weight."""
    from evo2_flash_amd.fp8 import Fp8StaticLinear
    N, K, M = 2048, 1024, 16
    lin = Fp8StaticLinear(K, N, bias=False, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(11)
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)
    lin.weight.weight_loader(lin.weight, w8)
    with torch.no_grad():
        lin.weight_scale.copy_(ws)
        lin.input_scale.fill_(6.0 / 448)
    x = torch.randn(M, K, generator=gen, device=DEV).to(torch.bfloat16)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    lin(x, out=out)  # eager: makes the decode copy
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            lin(x, out=out)
    torch.cuda.current_stream().wait_stream(s)
    eager = torch.empty_like(out)
    for how in ("loader", "loader", "copy_"):
        w = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)[0]
        if how == "loader":
            lin.weight.weight_loader(lin.weight, w)
        else:
            # a plain in-place write: the next eager call rewrites the copy in
            # the buffer the graph holds
            with torch.no_grad():
                lin.weight.copy_(w)
            lin(x, out=eager)
        for _ in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            ref = static_fp8_linear(x, lin.weight, lin.input_scale, lin.weight_scale)
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), how


def test_linear_decode_copy_after_loading():
    """process_weights_after_loading makes the decode copy before any decode
    call (an engine sizes its pools after loading); with decode_copies off
    none is made and the row-major GEMM gives the same bits."""
    from evo2_flash_amd.fp8 import Fp8StaticLinear
    N, K = 1024, 512
    gen = torch.Generator(device=DEV).manual_seed(13)
    w8, ws = quantize_weight_e4m3(torch.randn(N, K, generator=gen, device=DEV) * 0.02)
    x = torch.randn(4, K, generator=gen, device=DEV).to(torch.bfloat16)
    outs = []
    for copies in (True, False):
        lin = Fp8StaticLinear(K, N, bias=False, device=DEV)
        lin.decode_copies = copies
        lin.weight.weight_loader(lin.weight, w8)
        with torch.no_grad():
            lin.weight_scale.copy_(ws)
            lin.input_scale.fill_(6.0 / 448)
        lin.process_weights_after_loading()
        made = getattr(lin, "_decode_w", None)
        assert (made is not None) == copies
        if copies:
            assert made[1].shape == (N, K) and lin.decode_weight() is made[1]
        outs.append(lin(x)[0])
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
