// Hopper fp8 "fast accumulation" GEMM, modelled exactly on gfx950 VALU.
//
// The released fp8 Evo 2 checkpoints were trained with Transformer Engine's
// forward fp8 GEMM on sm_90, whose tensor-core accumulator is not fp32.  Some
// layers of those checkpoints depend on its rounding (the FP8-surgery
// configs `hyena_fp8_emulated_layers` / `hyena_fp8_emulated_channels`,
// config.py:81-94), so the reference runs a software model of it
// (fp8_emul.py:1-24; arithmetic of fp8_emul_triton.py:46-76).  This file is
// that model as a HIP kernel.  For each group of 32 consecutive k, ascending:
//
//   e   = max( max_k e(a_k) + e(b_k), e(acc) ),   e(x) = floor(log2|x|)
//   s   = trunc(acc 2^(13-e)) 2^(e-13) + sum_k trunc(a_k b_k 2^(13-e)) 2^(e-13)
//   acc = s truncated to 13 fraction bits of its own exponent
//
// then out = bf16((acc * s_in) * s_w).  Every step is exact in fp32 (E4M3
// products are exact; aligned terms are integers below 2^21 times the ulp),
// so the kernel reproduces the reference bit for bit.
//
// Operands: a (N, K) e4m3 activation rows; b_t (K, M) bf16 holding E4M3
// values, K-major, the layout of the surgery checkpoints'
// `in_proj_emul_weight_t` (mixers.py:768-800).  A workgroup owns 8 rows and
// 256 columns (lane = column); each group's 8 x 32 activation values and
// exponents are decoded once into LDS and read as broadcasts.
#include "common.h"

#pragma clang fp contract(off)

namespace evo2 {

constexpr int FA_G = 32;    // accumulation group (k)
constexpr int FA_F = 13;    // fraction bits kept
constexpr int FA_BN = 8;    // rows per workgroup
constexpr int FA_BM = 256;  // columns per workgroup

struct FastAccArgs {
  const uint8_t *a; int64_t sa;    // (N, K) e4m3 rows, row stride (bytes)
  const bf16_t *b; int64_t sb;     // (K, M) bf16 E4M3 values, row stride (elements)
  const float *sx, *sw;            // (1,) dequantisation scales
  void *out; int64_t so;           // (N, M) bf16 (scaled) or fp32 (raw accumulator)
  int out_f32;
  int N, M, K;
};

// OCP e4m3fn byte -> fp32 (exact): bias 7, subnormals m * 2^-9, S.1111.111 NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t x) {
  const uint32_t s = (x >> 7) & 1, e = (x >> 3) & 15, m = x & 7;
  if (e == 15 && m == 7) return __uint_as_float(0x7fc00000u);
  float v;
  if (e == 0) v = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

// floor(log2|x|) from the exponent field; a very negative sentinel for 0
// (the reference's -100000; a subnormal reads -127 as there).
__device__ __forceinline__ int exp_floor(float x) {
  const int e = static_cast<int>((__float_as_uint(x) >> 23) & 0xFF) - 127;
  return x == 0.0f ? -100000 : e;
}

// 2^e with e clamped to [-126, 127], as the reference clamps.
__device__ __forceinline__ float pow2i(int e) {
  e = min(max(e, -126), 127);
  return __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
}

__global__ __launch_bounds__(FA_BM) void fast_accum_kernel(FastAccArgs p) {
  __shared__ float av[FA_BN][FA_G];
  __shared__ int ae[FA_BN][FA_G];
  const int tid = threadIdx.x;
  const int m = blockIdx.x * FA_BM + tid;
  const int n0 = blockIdx.y * FA_BN;
  const bool mok = m < p.M;
  const int mc = mok ? m : p.M - 1;
  float acc[FA_BN];
#pragma unroll
  for (int r = 0; r < FA_BN; ++r) acc[r] = 0.0f;

  for (int k0 = 0; k0 < p.K; k0 += FA_G) {
    // decode this group's activations: thread t -> row t / 32, k t % 32
    {
      const int r = tid >> 5, kk = tid & 31;
      const int n = n0 + r;
      const float v = n < p.N ? e4m3_to_f32(p.a[(int64_t)n * p.sa + k0 + kk]) : 0.0f;
      __syncthreads();  // every lane is done with the previous group
      av[r][kk] = v;
      ae[r][kk] = exp_floor(v);
      __syncthreads();
    }
    float bv[FA_G];
    int be[FA_G];
#pragma unroll
    for (int kk = 0; kk < FA_G; ++kk) {
      bv[kk] = mok ? bf2f(p.b[(int64_t)(k0 + kk) * p.sb + mc]) : 0.0f;
      be[kk] = exp_floor(bv[kk]);
    }
#pragma unroll
    for (int r = 0; r < FA_BN; ++r) {
      int e = exp_floor(acc[r]);
#pragma unroll
      for (int kk = 0; kk < FA_G; ++kk) e = max(e, ae[r][kk] + be[kk]);
      const float ulp = pow2i(e - FA_F), inv = pow2i(FA_F - e);
      float s = truncf(acc[r] * inv) * ulp;
#pragma unroll
      for (int kk = 0; kk < FA_G; ++kk) s = s + truncf((av[r][kk] * bv[kk]) * inv) * ulp;
      const int es = exp_floor(s);
      acc[r] = s == 0.0f ? s : truncf(s * pow2i(FA_F - es)) * pow2i(es - FA_F);
    }
  }
  if (!mok) return;
  const float sx = p.out_f32 ? 1.0f : p.sx[0], sw = p.out_f32 ? 1.0f : p.sw[0];
#pragma unroll
  for (int r = 0; r < FA_BN; ++r) {
    const int n = n0 + r;
    if (n >= p.N) break;
    if (p.out_f32) static_cast<float *>(p.out)[(int64_t)n * p.so + m] = acc[r];
    else static_cast<bf16_t *>(p.out)[(int64_t)n * p.so + m] = f2bf((acc[r] * sx) * sw);
  }
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_fp8_fast_accum_gemm(const void *a8, int64_t sa, const void *b_t, int64_t sb,
                                        const float *input_scale, const float *weight_scale,
                                        void *out, int64_t so, int32_t out_f32, int64_t N,
                                        int64_t M, int64_t K, void *stream) {
  if (N < 0 || M < 0 || K < 0 || N > (int64_t(1) << 31) - 1 || M > (int64_t(1) << 31) - 1 ||
      K > (int64_t(1) << 31) - 1)
    return fail(EVO2_ERR_INVALID, "fp8_fast_accum_gemm: bad sizes N=%lld M=%lld K=%lld",
                (long long)N, (long long)M, (long long)K);
  if (K % FA_G)
    return fail(EVO2_ERR_INVALID, "fp8_fast_accum_gemm: K=%lld is not a multiple of %d",
                (long long)K, FA_G);
  if (N == 0 || M == 0) return EVO2_OK;
  if (!a8 || !b_t || !out || (!out_f32 && (!input_scale || !weight_scale)))
    return fail(EVO2_ERR_INVALID, "fp8_fast_accum_gemm: null pointer argument");
  if (sa < K || sb < M || so < M)
    return fail(EVO2_ERR_INVALID, "fp8_fast_accum_gemm: row strides shorter than the rows");
  if (cdiv(N, FA_BN) > 65535)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_fast_accum_gemm: %lld rows exceed the grid",
                (long long)N);
  FastAccArgs a{static_cast<const uint8_t *>(a8), sa, static_cast<const bf16_t *>(b_t), sb,
                input_scale, weight_scale, out, so, out_f32, static_cast<int>(N),
                static_cast<int>(M), static_cast<int>(K)};
  dim3 grid(static_cast<unsigned>(cdiv(M, FA_BM)), static_cast<unsigned>(cdiv(N, FA_BN)));
  hipLaunchKernelGGL(fast_accum_kernel, grid, dim3(FA_BM), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("fp8_fast_accum_gemm");
}
