// fp8 e4m3 (OCP e4m3fn) projection GEMMs on gfx950 MFMA, with static
// per-tensor scales and fp32 accumulation:
//
//   out[m, n] = bf16( (sum_k X8[m, k] * W8[n, k]) * s_x * s_w  [+ bias[n]] )
//
// the vLLM static W8A8 linear of the reference's in_proj
// (mixers.py:741-757, 1076-1092; scales in the dequantisation convention,
// convert.py:195-201), and the same GEMM for out_proj when it is quantised.
//
// Kernel: a 256 x 256 output tile per workgroup (W rows x X rows), K in steps
// of 128 bytes.  Four waves each own a 128 x 128 quadrant as 4 x 4 tiles of
// v_mfma_f32_32x32x64_f8f6f4 (the weight is MFMA operand A, so each lane
// ends up with four consecutive output columns of one row, stored as one
// 8-byte write).  Tiles of W and X move HBM -> LDS with direct-to-LDS loads
// into a double buffer, the next K step in flight while the current one
// computes.  LDS rows are 128 bytes; the 16-byte chunk c of row r sits at
// c ^ (r & 7), so the b128 fragment reads of 8 consecutive rows hit 8
// different bank groups.
#include "common.h"

namespace evo2 {

typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;

constexpr int G_BM = 256;   // X rows per workgroup
constexpr int G_BN = 256;   // W rows per workgroup
constexpr int G_BK = 128;   // bytes of K per step

struct GemmArgs {
  const uint8_t *x; int64_t sx;   // (M, K) e4m3, row stride (bytes)
  const uint8_t *w; int64_t sw;   // (N, K) e4m3, row stride (bytes)
  const float *sx_scale;          // (1,)
  const float *sw_scale;          // (1,)
  const bf16_t *bias;             // (N,) or null
  bf16_t *out; int64_t so;        // (M, N) bf16, row stride
  int M, N, K;
};

__device__ __forceinline__ void vmcnt_wait_16() {
  // s_waitcnt vmcnt(16): vmcnt bits [3:0] and [15:14], expcnt/lgkmcnt maxed.
  __builtin_amdgcn_s_waitcnt((16 & 0xF) | ((16 >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__global__ __launch_bounds__(256) void fp8_gemm_kernel(GemmArgs p) {
  __shared__ __align__(16) uint8_t lw[2][G_BN * G_BK];
  __shared__ __align__(16) uint8_t lx[2][G_BM * G_BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * G_BN;
  const int m0 = blockIdx.y * G_BM;
  const int wn = (wave & 1) * 128;   // wave quadrant in W rows
  const int wm = (wave >> 1) * 128;  // wave quadrant in X rows

  // DMA: each wave instruction fills 1 KB = 8 rows of 128 bytes; lane i
  // writes LDS chunk i of that block, i.e. row i/8, physical chunk i%8,
  // which holds logical chunk (i%8) ^ (row & 7).
  auto issue = [&](int buf, int k0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int blk = wave * 8 + j;         // 32 blocks of 8 rows per tile
      const int row = blk * 8 + lane / 8;
      const int lchunk = (lane & 7) ^ (row & 7);
      const int wr = min(n0 + row, p.N - 1);
      const int xr = min(m0 + row, p.M - 1);
      __builtin_amdgcn_global_load_lds(p.w + (int64_t)wr * p.sw + k0 + lchunk * 16,
                                       (__attribute__((address_space(3))) void *)(&lw[buf][blk * 1024]),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(p.x + (int64_t)xr * p.sx + k0 + lchunk * 16,
                                       (__attribute__((address_space(3))) void *)(&lx[buf][blk * 1024]),
                                       16, 0, 0);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int KT = p.K / G_BK;
  issue(0, 0);
  const int g = lane >> 5;   // lane group: k bytes [32g, 32g + 32) of a 64-k step
  const int lr = lane & 31;  // row within a 32-row MFMA tile
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) {
      issue(buf ^ 1, (kt + 1) * G_BK);
      vmcnt_wait_16();  // this step's 16 loads have landed; the next 16 fly
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      i32x8 fa[4], fb[4];
      const int c0 = ks * 4 + 2 * g;  // logical chunks c0, c0+1
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int rw = wn + 32 * t + lr;
        const int rx = wm + 32 * t + lr;
        const uint4 a0 = *reinterpret_cast<const uint4 *>(&lw[buf][rw * G_BK + ((c0 ^ (rw & 7)) << 4)]);
        const uint4 a1 = *reinterpret_cast<const uint4 *>(&lw[buf][rw * G_BK + (((c0 + 1) ^ (rw & 7)) << 4)]);
        const uint4 b0 = *reinterpret_cast<const uint4 *>(&lx[buf][rx * G_BK + ((c0 ^ (rx & 7)) << 4)]);
        const uint4 b1 = *reinterpret_cast<const uint4 *>(&lx[buf][rx * G_BK + (((c0 + 1) ^ (rx & 7)) << 4)]);
        fa[t] = i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        fb[t] = i32x8{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      }
#pragma unroll
      for (int tn = 0; tn < 4; ++tn)
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
          acc[tn][tm] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[tn], fb[tm], acc[tn][tm],
                                                                         0, 0, 0, 0, 0, 0);
    }
    __syncthreads();  // everyone is done with `buf` before it is refilled
  }

  // Epilogue: lane holds, for X row m = m0 + wm + 32 tm + lr, the W rows
  // n = n0 + wn + 32 tn + 8 q + 4 g + i (i < 4) in acc[tn][tm][4 q + i].
  const float scale = p.sx_scale[0] * p.sw_scale[0];
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    const int m = m0 + wm + 32 * tm + lr;
    if (m >= p.M) continue;
    bf16_t *orow = p.out + (int64_t)m * p.so;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn + 32 * tn + 8 * q + 4 * g;
        if (n >= p.N) continue;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[tn][tm][4 * q + i] * scale;
          if (p.bias) v[i] += bf2f(p.bias[min(n + i, p.N - 1)]);
        }
        if (n + 4 <= p.N && ((reinterpret_cast<uintptr_t>(orow + n) & 7) == 0)) {
          uint2 st;
          st.x = pack_bf(v[0], v[1]);
          st.y = pack_bf(v[2], v[3]);
          *reinterpret_cast<uint2 *>(orow + n) = st;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n + i < p.N) orow[n + i] = f2bf(v[i]);
        }
      }
    }
  }
}

// x (rows, K) bf16 -> e4m3fn(clamp(x / s, -448, 448)) (fp8_emul.py:76-78),
// two values per v_cvt_pk_fp8_f32 (round to nearest even).
__global__ __launch_bounds__(256) void fp8_quantize_kernel(const bf16_t *x, int64_t sx, uint8_t *q,
                                                           int64_t sq, const float *scale, int rows,
                                                           int K) {
  const int r = blockIdx.y;
  const int k = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (r >= rows || k >= K) return;
  const float s = scale[0];
  const bf16_t *xr = x + (int64_t)r * sx;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float f = (k + i < K) ? bf2f(xr[k + i]) : 0.0f;
    v[i] = fminf(fmaxf(f / s, -448.0f), 448.0f);
  }
  int packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
  packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], packed, true);
  uint8_t *qr = q + (int64_t)r * sq;
  if (k + 4 <= K && ((reinterpret_cast<uintptr_t>(qr + k) & 3) == 0)) {
    *reinterpret_cast<int *>(qr + k) = packed;
  } else {
    for (int i = 0; i < 4 && k + i < K; ++i) qr[k + i] = static_cast<uint8_t>(packed >> (8 * i));
  }
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_fp8_quantize(const void *x, int64_t sx, void *q, int64_t sq,
                                 const float *scale, int64_t rows, int64_t K, void *stream) {
  if (rows < 0 || K < 0 || rows > 65535 * 64LL)
    return fail(EVO2_ERR_INVALID, "fp8_quantize: bad sizes rows=%lld K=%lld", (long long)rows,
                (long long)K);
  if (rows == 0 || K == 0) return EVO2_OK;
  if (!x || !q || !scale) return fail(EVO2_ERR_INVALID, "fp8_quantize: null pointer argument");
  if (rows > 65535) {
    // split the rows over several launches to respect the grid limit
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
      const int64_t n = rows - r0 < 65535 ? rows - r0 : 65535;
      int rc = evo2_fp8_quantize(static_cast<const bf16_t *>(x) + r0 * sx, sx,
                                 static_cast<uint8_t *>(q) + r0 * sq, sq, scale, n, K, stream);
      if (rc) return rc;
    }
    return EVO2_OK;
  }
  dim3 grid(static_cast<unsigned>(cdiv(K, 1024)), static_cast<unsigned>(rows));
  hipLaunchKernelGGL(fp8_quantize_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16_t *>(x), sx, static_cast<uint8_t *>(q), sq, scale,
                     static_cast<int>(rows), static_cast<int>(K));
  return check_launch("fp8_quantize");
}

extern "C" int evo2_fp8_gemm(const void *x8, int64_t sx, const void *w8, int64_t sw,
                             const float *x_scale, const float *w_scale, const void *bias,
                             void *out, int64_t so, int64_t M, int64_t N, int64_t K,
                             void *stream) {
  if (M < 0 || N <= 0 || K <= 0)
    return fail(EVO2_ERR_INVALID, "fp8_gemm: bad sizes M=%lld N=%lld K=%lld", (long long)M,
                (long long)N, (long long)K);
  if (M == 0) return EVO2_OK;
  if (!x8 || !w8 || !x_scale || !w_scale || !out)
    return fail(EVO2_ERR_INVALID, "fp8_gemm: null pointer argument");
  if (K % G_BK)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_gemm: K=%lld must be a multiple of %d", (long long)K, G_BK);
  if (sx % 16 || sw % 16 || reinterpret_cast<uintptr_t>(x8) % 16 ||
      reinterpret_cast<uintptr_t>(w8) % 16)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_gemm: operands must be 16-byte aligned rows");
  if (cdiv(M, G_BM) > 65535 || cdiv(N, G_BN) > 65535 || M > 0x7fffffff || N > 0x7fffffff)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_gemm: problem too large");
  GemmArgs a{static_cast<const uint8_t *>(x8), sx, static_cast<const uint8_t *>(w8), sw, x_scale,
             w_scale, static_cast<const bf16_t *>(bias), static_cast<bf16_t *>(out), so,
             static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)};
  dim3 grid(static_cast<unsigned>(cdiv(N, G_BN)), static_cast<unsigned>(cdiv(M, G_BM)));
  hipLaunchKernelGGL(fp8_gemm_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("fp8_gemm");
}
