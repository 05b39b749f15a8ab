// Evo2RMSNorm for gfx950 (model.py:47-74, triton_norm.py:125-156):
//
//   s = bf16(x + residual)            (residual optional; s is written back)
//   n = bf16(sqrt(sum s^2))           fp32 sum of squares
//   n = bf16(n * H^-1/2);  n = bf16(n + eps)      eps outside the sqrt
//   y = bf16(w * bf16(s / n))         correctly rounded division
//
// Many rows: one wavefront per row; each lane keeps its slice of the row in
// registers (packed bf16), so the row is read once and written once.  Few
// rows (decode batches): a workgroup per row, one 16-byte chunk per thread,
// so a row's 4096 correctly rounded divisions are spread over 512 lanes
// instead of 64.  Both sum the squares in one order: each 8-value chunk from
// zero, the chunks of lane l (l, l + 64, l + 128, ...) in turn, then a
// butterfly over the 64 lanes, so a row's result does not depend on how
// many rows the launch has.  Optionally the
// normalised row is also quantised for the fp8 in_proj that consumes it,
// q = e4m3fn(clamp(y / input_scale, +-448)) (fp8_emul.py:76-78), which saves
// the separate quantisation pass over y; y itself may then be skipped.
#include "common.h"

#pragma clang fp contract(off)

namespace evo2 {

struct NormArgs {
  const bf16_t *x; int64_t sx;
  const bf16_t *r; int64_t sr;     // residual or null
  const bf16_t *w;                 // (H,) bf16
  bf16_t *y; int64_t sy;           // normalised output or null
  bf16_t *s; int64_t ss;           // x + residual output (with residual)
  const float *qscale;             // (1,) dequantisation scale, or null
  uint8_t *q; int64_t sq;          // e4m3 output or null
  int64_t T;
  int H;
  float eps;
  float inv_sqrt_h;
};

// s = bf16(x + residual) for chunk j of a row, written to the s output.
__device__ __forceinline__ uint4 add_chunk(const NormArgs &p, int64_t row, int j, uint4 v) {
  const uint4 b = reinterpret_cast<const uint4 *>(p.r + row * p.sr)[j];
  const uint32_t av[4] = {v.x, v.y, v.z, v.w};
  const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack_bf(lo_bf(av[e]) + lo_bf(bv[e]), hi_bf(av[e]) + hi_bf(bv[e]));
  const uint4 s = make_uint4(o[0], o[1], o[2], o[3]);
  reinterpret_cast<uint4 *>(p.s + row * p.ss)[j] = s;
  return s;
}

// fp32 sum of the squares of a chunk's 8 values, in element order from zero.
__device__ __forceinline__ float chunk_sumsq(uint4 v) {
  const uint32_t av[4] = {v.x, v.y, v.z, v.w};
  float cs = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = lo_bf(av[e]), b = hi_bf(av[e]);
    cs = cs + a * a;
    cs = cs + b * b;
  }
  return cs;
}

__device__ __forceinline__ float lane_butterfly(float acc) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off);
  return acc;
}

// n = bf16(bf16(bf16(sqrt(sum)) * H^-1/2) + eps)
__device__ __forceinline__ float row_norm(float sumsq, const NormArgs &p) {
  float n = rbf(sqrtf(sumsq));
  n = rbf(n * p.inv_sqrt_h);
  return rbf(n + p.eps);
}

// y = bf16(w * bf16(s / n)) for chunk j (and its e4m3 quantisation).
template <bool QUANT>
__device__ __forceinline__ void norm_chunk(const NormArgs &p, int64_t row, int j, uint4 v, float n) {
  const uint4 wv = reinterpret_cast<const uint4 *>(p.w)[j];
  const uint32_t av[4] = {v.x, v.y, v.z, v.w};
  const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
  uint32_t o[4];
  float yv[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    yv[2 * e] = rbf(lo_bf(ww[e]) * rbf(lo_bf(av[e]) / n));
    yv[2 * e + 1] = rbf(hi_bf(ww[e]) * rbf(hi_bf(av[e]) / n));
    o[e] = pack_bf(yv[2 * e], yv[2 * e + 1]);
  }
  if (p.y) reinterpret_cast<uint4 *>(p.y + row * p.sy)[j] = make_uint4(o[0], o[1], o[2], o[3]);
  if constexpr (QUANT) {
    const float qs = p.qscale[0];
    int lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) yv[e] = fminf(fmaxf(yv[e] / qs, -448.0f), 448.0f);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(yv[0], yv[1], lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(yv[2], yv[3], lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(yv[4], yv[5], hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(yv[6], yv[7], hi, true);
    reinterpret_cast<uint2 *>(p.q + row * p.sq)[j] = make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi));
  }
}

// CH = 16-byte chunks (8 values) per lane; H = 512 * CH for the vector path.
template <int CH, bool ADD, bool QUANT>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(NormArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.T) return;  // wave-uniform
  uint4 v[CH];
  const uint4 *xr = reinterpret_cast<const uint4 *>(p.x + row * p.sx);
#pragma unroll
  for (int i = 0; i < CH; ++i) v[i] = xr[lane + 64 * i];
  if constexpr (ADD) {
#pragma unroll
    for (int i = 0; i < CH; ++i) v[i] = add_chunk(p, row, lane + 64 * i, v[i]);
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < CH; ++i) acc = acc + chunk_sumsq(v[i]);
  const float n = row_norm(lane_butterfly(acc), p);
#pragma unroll
  for (int i = 0; i < CH; ++i) norm_chunk<QUANT>(p, row, lane + 64 * i, v[i], n);
}

// Few rows: workgroup = one row of H = 512 CH, thread t holds chunk t (wave
// i, lane l: chunk l + 64 i, as lane l's i-th chunk in the per-row form).
// The chunk sums meet in LDS and wave 0 adds lane l's CH of them in order i.
template <int CH, bool ADD, bool QUANT>
__global__ __launch_bounds__(64 * CH) void rms_norm_row_kernel(NormArgs p) {
  __shared__ float part[CH][64];
  __shared__ float nrow;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  uint4 v = reinterpret_cast<const uint4 *>(p.x + row * p.sx)[t];
  if constexpr (ADD) v = add_chunk(p, row, t, v);
  part[wave][lane] = chunk_sumsq(v);
  __syncthreads();
  if (wave == 0) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < CH; ++i) acc = acc + part[i][lane];
    const float n = row_norm(lane_butterfly(acc), p);
    if (lane == 0) nrow = n;
  }
  __syncthreads();
  norm_chunk<QUANT>(p, row, t, v, nrow);
}

// Any H, any unit-stride rows: one wavefront per row, element by element.
template <bool ADD, bool QUANT>
__global__ __launch_bounds__(256) void rms_norm_scalar_kernel(NormArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.T) return;
  const bf16_t *xr = p.x + row * p.sx;
  float acc = 0.0f;
  for (int i = lane; i < p.H; i += 64) {
    float v = bf2f(xr[i]);
    if constexpr (ADD) {
      v = rbf(v + bf2f(p.r[row * p.sr + i]));
      p.s[row * p.ss + i] = f2bf(v);
    }
    acc = acc + v * v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off);
  float n = rbf(sqrtf(acc));
  n = rbf(n * p.inv_sqrt_h);
  n = rbf(n + p.eps);
  const float qs = QUANT ? p.qscale[0] : 1.0f;
  for (int i = lane; i < p.H; i += 64) {
    float v = bf2f(xr[i]);
    if constexpr (ADD) v = rbf(v + bf2f(p.r[row * p.sr + i]));
    const float y = rbf(bf2f(p.w[i]) * rbf(v / n));
    if (p.y) p.y[row * p.sy + i] = f2bf(y);
    if constexpr (QUANT) {
      const float c = fminf(fmaxf(y / qs, -448.0f), 448.0f);
      p.q[row * p.sq + i] = static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, 0.0f, 0, false));
    }
  }
}

// Up to this many rows a launch takes a workgroup per row (the per-row
// wavefront form leaves most of the chip idle and each wave's 8 H/512
// divisions serial).
#ifndef NORM_ROW_SPLIT_MAX
#define NORM_ROW_SPLIT_MAX 2048
#endif

template <int CH, bool ADD, bool QUANT>
static void launch_rows(const NormArgs &a, hipStream_t st) {
  hipLaunchKernelGGL((rms_norm_row_kernel<CH, ADD, QUANT>), dim3(static_cast<unsigned>(a.T)),
                     dim3(64 * CH), 0, st, a);
}

template <bool ADD, bool QUANT>
static void launch_norm(const NormArgs &a, bool vec, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(cdiv(a.T, 4)));
  if (vec && a.T <= NORM_ROW_SPLIT_MAX && (a.H == 1024 || a.H == 2048 || a.H == 4096 || a.H == 8192)) {
    if (a.H == 1024) launch_rows<2, ADD, QUANT>(a, st);
    else if (a.H == 2048) launch_rows<4, ADD, QUANT>(a, st);
    else if (a.H == 4096) launch_rows<8, ADD, QUANT>(a, st);
    else launch_rows<16, ADD, QUANT>(a, st);
  } else if (vec && a.H == 1024) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<2, ADD, QUANT>), grid, dim3(256), 0, st, a);
  } else if (vec && a.H == 2048) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<4, ADD, QUANT>), grid, dim3(256), 0, st, a);
  } else if (vec && a.H == 4096) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<8, ADD, QUANT>), grid, dim3(256), 0, st, a);
  } else if (vec && a.H == 8192) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<16, ADD, QUANT>), grid, dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((rms_norm_scalar_kernel<ADD, QUANT>), grid, dim3(256), 0, st, a);
  }
}

static bool al16(const void *p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_rms_norm(const void *x, int64_t sx, const void *residual, int64_t sr,
                             const void *weight, float eps, void *y, int64_t sy,
                             void *s_out, int64_t ss, const float *q_scale, void *q, int64_t sq,
                             int64_t T, int64_t H, void *stream) {
  if (T < 0 || H <= 0 || H > (1 << 24))
    return fail(EVO2_ERR_INVALID, "rms_norm: bad sizes T=%lld H=%lld", (long long)T, (long long)H);
  if (T == 0) return EVO2_OK;
  if (!x || !weight || (!y && !q))
    return fail(EVO2_ERR_INVALID, "rms_norm: null pointer argument");
  if (residual && !s_out)
    return fail(EVO2_ERR_INVALID, "rms_norm: a residual needs the s output");
  if (q && !q_scale) return fail(EVO2_ERR_INVALID, "rms_norm: fp8 output needs its scale");
  if (cdiv(T, 4) > 0x7fffffff) return fail(EVO2_ERR_UNSUPPORTED, "rms_norm: too many rows");
  NormArgs a{static_cast<const bf16_t *>(x), sx, static_cast<const bf16_t *>(residual), sr,
             static_cast<const bf16_t *>(weight), static_cast<bf16_t *>(y), sy,
             static_cast<bf16_t *>(s_out), ss, q_scale, static_cast<uint8_t *>(q), sq, T,
             static_cast<int>(H), eps, 1.0f / sqrtf(static_cast<float>(H))};
  // H^-1/2 as torch computes the Python float `hidden_size ** -0.5` and
  // multiplies a bf16 tensor by it (the scalar enters the fp32 op as float).
  a.inv_sqrt_h = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(H)));
  const bool vec = al16(x) && al16(residual) && al16(weight) && al16(y) && al16(s_out) &&
                   (q == nullptr || reinterpret_cast<uintptr_t>(q) % 8 == 0) &&
                   sx % 8 == 0 && (!residual || sr % 8 == 0) && (!y || sy % 8 == 0) &&
                   (!s_out || ss % 8 == 0) && (!q || sq % 8 == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (residual) q ? launch_norm<true, true>(a, vec, st) : launch_norm<true, false>(a, vec, st);
  else q ? launch_norm<false, true>(a, vec, st) : launch_norm<false, false>(a, vec, st);
  return check_launch("rms_norm");
}
