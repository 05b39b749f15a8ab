// fp8 e4m3 (OCP e4m3fn) projection GEMMs on gfx950 MFMA, with static
// per-tensor scales and fp32 accumulation:
//
//   out[m, n] = bf16( (sum_k X8[m, k] * W8[n, k]) * s_x * s_w  [+ bias[n]] )
//
// the vLLM static W8A8 linear of the reference's in_proj
// (mixers.py:741-757, 1076-1092; scales in the dequantisation convention,
// convert.py:195-201), and the same GEMM for out_proj when it is quantised.
//
// Kernel: a 256 x 256 output tile per workgroup (W rows x X rows).  Four
// waves each own a 128 x 128 quadrant as 4 x 4 tiles of
// v_mfma_f32_32x32x64_f8f6f4 (the weight is MFMA operand A, so each lane
// ends up with four consecutive output columns of one row, stored as one
// 8-byte write).  K moves through a ring of five LDS stages of 64 bytes
// each (16 KB of W and 16 KB of X per stage), filled HBM -> LDS by
// direct-to-LDS loads four steps ahead of the MFMAs that consume them, so
// about three steps of MFMA work (~1.5 us) cover the load latency even when
// a load misses L2.  Each
// stage is its own __shared__ variable and the step loop is unrolled over
// the ring, so the compiler can see that reading one stage does not wait on
// the loads still landing in the others.  LDS rows are 64 bytes; the 16-byte
// chunk c of row r sits at c ^ ((r >> 2) & 3): a b128 read is served 16
// lanes (16 consecutive rows) at a time over 64 banks, and the swizzle puts
// those 16 rows' chunks in 16 different bank groups.
#include <type_traits>

#include "common.h"

namespace evo2 {

typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int G_BM = 256;       // X rows per workgroup
constexpr int G_BN = 256;       // W rows per workgroup
constexpr int G_BK = 64;        // bytes of K per stage (one MFMA k-step)
constexpr int G_STAGE = G_BN * G_BK;  // bytes per operand per stage

struct GemmArgs {
  const uint8_t *x; int64_t sx;   // (M, K) e4m3, row stride (bytes)
  const uint8_t *w; int64_t sw;   // (N, K) e4m3, row stride (bytes)
  const float *sx_scale;          // (1,)
  const float *sw_scale;          // (1,)
  const bf16_t *bias;             // (N,) or null
  bf16_t *out; int64_t so;        // (M, N) bf16, row stride
  int M, N, K;
};

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their maxima), without
// the workgroup memory fence __syncthreads adds.
template <int N>
__device__ __forceinline__ void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__global__ __launch_bounds__(256) void fp8_gemm_kernel(GemmArgs p) {
  __shared__ __align__(16) uint8_t w0[G_STAGE], w1[G_STAGE], w2[G_STAGE], w3[G_STAGE], w4[G_STAGE];
  __shared__ __align__(16) uint8_t x0[G_STAGE], x1[G_STAGE], x2[G_STAGE], x3[G_STAGE], x4[G_STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * G_BN;
  const int m0 = blockIdx.y * G_BM;
  const int wn = (wave & 1) * 128;   // wave quadrant in W rows
  const int wm = (wave >> 1) * 128;  // wave quadrant in X rows

  // DMA: one wave instruction fills 1 KB = 16 rows of 64 bytes; lane i
  // writes row i/4, physical chunk i%4, which holds logical chunk
  // (i%4) ^ ((row >> 2) & 3).  Each wave moves 4 such blocks of W and 4 of X
  // per stage; rows past M or N re-read the last row (never stored).
  const uint8_t *gw[4], *gx[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = (wave * 4 + j) * 16 + lane / 4;
    const int lchunk = (lane & 3) ^ ((row >> 2) & 3);
    gw[j] = p.w + (int64_t)min(n0 + row, p.N - 1) * p.sw + lchunk * 16;
    gx[j] = p.x + (int64_t)min(m0 + row, p.M - 1) * p.sx + lchunk * 16;
  }
  auto issue = [&](auto stage, int k0) __attribute__((always_inline)) {
    constexpr int S = decltype(stage)::value;
    uint8_t *lw = S == 0 ? w0 : S == 1 ? w1 : S == 2 ? w2 : S == 3 ? w3 : w4;
    uint8_t *lx = S == 0 ? x0 : S == 1 ? x1 : S == 2 ? x2 : S == 3 ? x3 : x4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = wave * 4 + j;
      __builtin_amdgcn_global_load_lds(gw[j] + k0, (lds_void *)(lw + blk * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(gx[j] + k0, (lds_void *)(lx + blk * 1024), 16, 0, 0);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int g = lane >> 5;   // lane group: k bytes [32g, 32g + 32) of the step
  const int lr = lane & 31;  // row within a 32-row MFMA tile
  // Byte offset of this lane's two 16-byte chunks in row r of a stage.
  auto frag_off = [&](int r) __attribute__((always_inline)) {
    const int sw = (r >> 2) & 3;
    return r * G_BK + (((2 * g) ^ sw) << 4);
  };
  auto frag_off1 = [&](int r) __attribute__((always_inline)) {
    const int sw = (r >> 2) & 3;
    return r * G_BK + (((2 * g + 1) ^ sw) << 4);
  };

  const int KT = p.K / G_BK;
  auto read_frags = [&](auto stage, i32x8 fa[4], i32x8 fb[4]) __attribute__((always_inline)) {
    constexpr int S = decltype(stage)::value;
    const uint8_t *lw = S == 0 ? w0 : S == 1 ? w1 : S == 2 ? w2 : S == 3 ? w3 : w4;
    const uint8_t *lx = S == 0 ? x0 : S == 1 ? x1 : S == 2 ? x2 : S == 3 ? x3 : x4;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int rw = wn + 32 * t + lr;
      const int rx = wm + 32 * t + lr;
      const uint4 a0 = *reinterpret_cast<const uint4 *>(lw + frag_off(rw));
      const uint4 a1 = *reinterpret_cast<const uint4 *>(lw + frag_off1(rw));
      const uint4 b0 = *reinterpret_cast<const uint4 *>(lx + frag_off(rx));
      const uint4 b1 = *reinterpret_cast<const uint4 *>(lx + frag_off1(rx));
      fa[t] = i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
      fb[t] = i32x8{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    }
  };
  auto mma = [&](const i32x8 fa[4], const i32x8 fb[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
        acc[tn][tm] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[tn], fb[tm], acc[tn][tm],
                                                                       0, 0, 0, 0, 0, 0);
  };

  // Step k runs the MFMAs of stage k from fragments read during step k - 1,
  // and meanwhile reads stage k + 1's fragments: it first waits for stage
  // k + 1's loads (stages k + 2 and k + 3 stay in flight) and a barrier
  // (every wave's loads for k + 1 have landed; every wave has consumed stage
  // k - 1, which is refilled with stage k + 4 right after).  Refills past the
  // end of K re-read the last slice, and the fragments read for the step
  // after the last are never used, so every step has the same shape.
  i32x8 fa[2][4], fb[2][4];
  auto step = [&](auto stage, auto fbuf, int k) __attribute__((always_inline)) {
    constexpr int S = decltype(stage)::value;
    constexpr int B = decltype(fbuf)::value;  // fragment buffer holding stage k
    vmcnt_wait<16>();
    __builtin_amdgcn_s_barrier();
    issue(std::integral_constant<int, (S + 4) % 5>{}, min(k + 4, KT - 1) * G_BK);
    read_frags(std::integral_constant<int, (S + 1) % 5>{}, fa[B ^ 1], fb[B ^ 1]);
    mma(fa[B], fb[B]);
    // Interleave: each MFMA is followed by one fragment read for the next
    // stage and (for the first eight) one refill load, so the LDS and memory
    // traffic hides under the matrix pipe instead of bunching up.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (i < 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  };
  // Ten steps cover every (stage, fragment buffer) pair once.
  auto ten_steps = [&](int k, bool guard) __attribute__((always_inline)) {
    using std::integral_constant;
    using I0 = integral_constant<int, 0>;
    using I1 = integral_constant<int, 1>;
    step(I0{}, I0{}, k);
    if (!guard || k + 1 < KT) step(I1{}, I1{}, k + 1);
    if (!guard || k + 2 < KT) step(integral_constant<int, 2>{}, I0{}, k + 2);
    if (!guard || k + 3 < KT) step(integral_constant<int, 3>{}, I1{}, k + 3);
    if (!guard || k + 4 < KT) step(integral_constant<int, 4>{}, I0{}, k + 4);
    if (!guard || k + 5 < KT) step(I0{}, I1{}, k + 5);
    if (!guard || k + 6 < KT) step(I1{}, I0{}, k + 6);
    if (!guard || k + 7 < KT) step(integral_constant<int, 2>{}, I1{}, k + 7);
    if (!guard || k + 8 < KT) step(integral_constant<int, 3>{}, I0{}, k + 8);
    if (!guard || k + 9 < KT) step(integral_constant<int, 4>{}, I1{}, k + 9);
  };

  using S0 = std::integral_constant<int, 0>;
  issue(S0{}, 0);
  issue(std::integral_constant<int, 1>{}, min(1, KT - 1) * G_BK);
  issue(std::integral_constant<int, 2>{}, min(2, KT - 1) * G_BK);
  issue(std::integral_constant<int, 3>{}, min(3, KT - 1) * G_BK);
  vmcnt_wait<24>();  // stage 0 (stages 1-3 in flight)
  __builtin_amdgcn_s_barrier();
  read_frags(S0{}, fa[0], fb[0]);
  int k = 0;
  for (; k + 10 <= KT; k += 10) ten_steps(k, false);
  if (k < KT) ten_steps(k, true);
  // No direct-to-LDS write may still be landing when the workgroup's LDS is
  // handed to the next one.
  vmcnt_wait<0>();

  // Epilogue: lane holds, for X row m = m0 + wm + 32 tm + lr, the W rows
  // n = n0 + wn + 32 tn + 8 q + 4 g + i (i < 4) in acc[tn][tm][4 q + i].
  const float scale = p.sx_scale[0] * p.sw_scale[0];
  const bool full = m0 + G_BM <= p.M && n0 + G_BN <= p.N && (p.so % 4) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.out) & 7) == 0;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    const int m = m0 + wm + 32 * tm + lr;
    if (!full && m >= p.M) continue;
    bf16_t *orow = p.out + (int64_t)m * p.so;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn + 32 * tn + 8 * q + 4 * g;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = acc[tn][tm][4 * q + i] * scale;
        if (p.bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += bf2f(p.bias[min(n + i, p.N - 1)]);
        }
        if (full || (n + 4 <= p.N && ((reinterpret_cast<uintptr_t>(orow + n) & 7) == 0))) {
          *reinterpret_cast<uint2 *>(orow + n) = make_uint2(pack_bf(v[0], v[1]), pack_bf(v[2], v[3]));
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
