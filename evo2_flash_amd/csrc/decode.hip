// Fused single-token Hyena decode step for gfx950.
//
// One thread per (row b, channel h).  Lanes run along channels, so every
// state column, z triple and output row is read and written as one coalesced
// sweep across the wavefront; the hcm window shift is a column-by-column
// read / write-one-column-lower pass over the channel-contiguous native
// layout.  Each state element is read and written by exactly one thread, so
// the in-place update needs no barrier: within a thread, every load of a
// column precedes the store that overwrites it in program order.
//
// Rounding points follow evo2_flash/triton_decode.py:10-22, 44-53, 57-164:
// fp32 products are rounded separately from the sums (no FMA contraction in
// this file), reductions use the same association trees, and every value a
// bf16 torch tensor would hold is rounded to bf16.
#include "common.h"

#pragma clang fp contract(off)

namespace evo2 {

enum { KIND_HCS = 0, KIND_HCM = 1, KIND_HCL = 2 };

struct DecodeArgs {
  const bf16_t *z; int64_t sz;
  const bf16_t *ws;
  bf16_t *cs; int64_t cs0, cs1, cs2;
  const int32_t *slots; int64_t ssl;
  const void *inner; int64_t wi0, wi1;
  const float *lp; int64_t lp0, lp1;
  float *st; int64_t is0, is1, is2;
  const bf16_t *D;
  bf16_t *out; int64_t so;
  int H;
  int null_block;
  int64_t num_blocks;
  int rows;  // B
};

// vLLM's K=3 conv update for one channel (triton_decode.py:44-53):
// bf16(((0 + bf16(c0 w0)) + bf16(c1 w1)) + bf16(x w2)).
__device__ __forceinline__ float short_tap(float x, float c0, float c1, const bf16_t *w) {
  float acc = 0.0f + rbf(c0 * bf2f(w[0]));
  acc = acc + rbf(c1 * bf2f(w[1]));
  acc = acc + rbf(x * bf2f(w[2]));
  return rbf(acc);
}

template <int KIND, bool HAS_D, bool CONTIG_S>
__global__ __launch_bounds__(256) void hyena_decode_kernel(DecodeArgs a) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (h >= a.H) return;
  const int64_t blk = a.slots[b * a.ssl];
  bf16_t *o = a.out + b * a.so + h;
  // The null block (CUDA/HIP-graph padding rows) and any slot outside the
  // pool produce a zero row and touch no state.
  if (blk == a.null_block || blk < 0 || blk >= a.num_blocks) {
    *o = 0;
    return;
  }

  // ---- short filter on the interleaved triple (3h, 3h+1, 3h+2) = (x2, x1, v)
  const bf16_t *zr = a.z + b * a.sz + 3 * (int64_t)h;
  bf16_t *c = a.cs + blk * a.cs0 + 3 * (int64_t)h * a.cs1;
  bf16_t keep_c1[3], keep_x[3];
  float y3[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const bf16_t xb = zr[i];
    const bf16_t c0b = c[i * a.cs1];
    const bf16_t c1b = c[i * a.cs1 + a.cs2];
    y3[i] = short_tap(bf2f(xb), bf2f(c0b), bf2f(c1b), a.ws + (3 * (int64_t)h + i) * 3);
    keep_c1[i] = c1b;
    keep_x[i] = xb;
  }
  const float x2 = y3[0];
  const float u = rbf(y3[1] * y3[2]);
  float y;

  float *s = a.st + blk * a.is0 + (int64_t)h * a.is1;
  if constexpr (KIND == KIND_HCL) {
    // s <- s * exp(lp) + u; readout halving tree (triton_decode.py:81-96).
    const float *res = static_cast<const float *>(a.inner) + (int64_t)h * a.wi0;
    const float *lp = a.lp + (int64_t)h * a.lp0;
    float sv[16], r[16];
    if constexpr (CONTIG_S) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = reinterpret_cast<const float4 *>(s)[q];
        sv[4 * q] = v.x; sv[4 * q + 1] = v.y; sv[4 * q + 2] = v.z; sv[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) sv[i] = s[i * a.is2];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = expf(lp[i * a.lp1]);
      sv[i] = sv[i] * p + u;
      r[i] = sv[i] * res[i * a.wi1];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = r[i] + r[i + 8];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = r[i] + r[i + 4];
#pragma unroll
    for (int i = 0; i < 2; ++i) r[i] = r[i] + r[i + 2];
    y = rbf((r[0] + r[1]) + 0.0f);
    if constexpr (CONTIG_S) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<float4 *>(s)[q] =
            make_float4(sv[4 * q], sv[4 * q + 1], sv[4 * q + 2], sv[4 * q + 3]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i * a.is2] = sv[i];
    }
  } else if constexpr (KIND == KIND_HCM) {
    // Taps k = 16j + 4m + l: accumulator (m, l) sums j = 0..7 in order, then
    // ((m0 + m1) + m2) + m3 per l, then (l0 + l2) + (l1 + l3)
    // (triton_decode.py:97-124).  The window shifts down one column in place.
    const bf16_t *w = static_cast<const bf16_t *>(a.inner) + (int64_t)h * a.wi0;
    float acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int l = 0; l < 4; ++l) acc[m][l] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float sv[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int k = 16 * j + q;
        sv[q] = (k < 127) ? s[k * a.is2] : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int k = 16 * j + q;
        const float wk = (k < 127) ? bf2f(w[k * a.wi1]) : 0.0f;
        acc[q >> 2][q & 3] = acc[q >> 2][q & 3] + sv[q] * wk;
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int k = 16 * j + q;
        if (k >= 1 && k < 127) s[(k - 1) * a.is2] = sv[q];
      }
    }
    float p[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) p[l] = ((acc[0][l] + acc[1][l]) + acc[2][l]) + acc[3][l];
    const float last = bf2f(w[127 * a.wi1]);
    y = rbf(((p[0] + p[2]) + (p[1] + p[3])) + last * u);
    s[126 * a.is2] = u;
  } else {
    // K = 7: ((((s0w0 + s4w4) + (s1w1 + s5w5)) + s2w2) + s3w3) + w6 u
    // (triton_decode.py:125-150).
    const bf16_t *w = static_cast<const bf16_t *>(a.inner) + (int64_t)h * a.wi0;
    float sv[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) sv[k] = s[k * a.is2];
    const float aa = (sv[0] * bf2f(w[0]) + 0.0f) + sv[4] * bf2f(w[4 * a.wi1]);
    const float bb = (sv[1] * bf2f(w[a.wi1]) + 0.0f) + sv[5] * bf2f(w[5 * a.wi1]);
    const float cc = sv[2] * bf2f(w[2 * a.wi1]) + 0.0f;
    const float dd = sv[3] * bf2f(w[3 * a.wi1]) + 0.0f;
    const float last = bf2f(w[6 * a.wi1]);
    y = rbf((((aa + bb) + cc) + dd) + last * u);
#pragma unroll
    for (int k = 0; k < 5; ++k) s[k * a.is2] = sv[k + 1];
    s[5 * a.is2] = u;
  }

  // Short-filter window (c0, c1) <- (c1, x).
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    c[i * a.cs1] = keep_c1[i];
    c[i * a.cs1 + a.cs2] = keep_x[i];
  }

  if constexpr (HAS_D) y = rbf(y + rbf(bf2f(a.D[h]) * u));
  *o = f2bf(x2 * y);
}

template <int KIND, bool HAS_D, bool CONTIG_S>
static void launch(const DecodeArgs &a, int64_t B, hipStream_t stream) {
  constexpr int BH = 256;
  dim3 grid(static_cast<unsigned>(cdiv(a.H, BH)), static_cast<unsigned>(B));
  hipLaunchKernelGGL((hyena_decode_kernel<KIND, HAS_D, CONTIG_S>), grid, dim3(BH), 0, stream, a);
}

// ---------------------------------------------------------------------------
// Fast paths for the engine's native layouts.  A lane owns a channel pair
// (h0, h0+1), so every operand moves as 4/8/16-byte vectors: the z triple
// pair and both conv-state columns as three dwords each, FIR window columns
// as float2 (channel-contiguous native storage).  Arithmetic and rounding are
// exactly the generic kernel's.
//
// The fast kernels never return early on a null row: its loads go to block
// 0 (which always exists), its results are dropped and it writes a zero
// output.  With no branch in front of them, the loads that do not depend on
// the slot (z, taps, D) are issued while the slot lookup is in flight.
//
// WT: FIR taps in channel-contiguous (K, H) storage (wi0 == 1), one dword
// per tap for the pair; otherwise tap-contiguous (H, K) rows (wi1 == 1).

__device__ __forceinline__ void unpack3(const uint32_t *p, float f[6]) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const uint32_t v = p[i];
    f[2 * i] = lo_bf(v);
    f[2 * i + 1] = hi_bf(v);
  }
}

// Slot of decode row b: `blk` is the block to read (0 for a null row),
// the return value whether the row is live.
__device__ __forceinline__ bool row_slot(const DecodeArgs &a, int64_t b, int64_t &blk) {
  const int64_t sl = a.slots[b * a.ssl];
  // bitwise, not short-circuit: no branch may split the load sequence
  const bool live = (sl != a.null_block) & (sl >= 0) & (sl < a.num_blocks);
  blk = live ? sl : 0;
  return live;
}

// All ones for a live row, zero for a null one, as a value the optimizer
// cannot see through: the output is `result & mask`, so the row's loads and
// arithmetic are needed on both paths and stay in front of the slot lookup
// instead of being moved behind a branch on it.
__device__ __forceinline__ uint32_t live_mask(bool live) {
  uint32_t m = live ? 0xffffffffu : 0u;
  asm volatile("" : "+v"(m));
  return m;
}

// Short filter and gate for the six sub-channels of the pair h0, h0+1:
// x2 and u per channel (triton_decode.py:44-53, 72-78).
__device__ __forceinline__ void pair_featurize(const uint32_t zraw[3], const uint32_t c0raw[3],
                                               const uint32_t c1raw[3], const uint32_t wsraw[9],
                                               float x2[2], float u[2]) {
  float xf[6], c0f[6], c1f[6], wsf[18];
  unpack3(zraw, xf);
  unpack3(c0raw, c0f);
  unpack3(c1raw, c1f);
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    wsf[2 * i] = lo_bf(wsraw[i]);
    wsf[2 * i + 1] = hi_bf(wsraw[i]);
  }
  float y6[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    float acc = 0.0f + rbf(c0f[i] * wsf[3 * i]);
    acc = acc + rbf(c1f[i] * wsf[3 * i + 1]);
    acc = acc + rbf(xf[i] * wsf[3 * i + 2]);
    y6[i] = rbf(acc);
  }
  x2[0] = y6[0];
  x2[1] = y6[3];
  u[0] = rbf(y6[1] * y6[2]);
  u[1] = rbf(y6[4] * y6[5]);
}

// hcs (K=7): the 6-column window of the pair moves as six float2.
template <bool HAS_D, bool WT>
__global__ __launch_bounds__(128) void hcs_decode_pair_kernel(DecodeArgs a) {
  const int pair = blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = 2 * pair < a.H;
  const int h0 = active ? 2 * pair : 0;  // inactive lanes load channel pair 0, store nothing
  const int64_t b = blockIdx.y;

  const uint32_t *zr = reinterpret_cast<const uint32_t *>(a.z + b * a.sz + 3 * (int64_t)h0);
  const uint32_t *wsp = reinterpret_cast<const uint32_t *>(a.ws + 9 * (int64_t)h0);
  const bf16_t *w = static_cast<const bf16_t *>(a.inner);
  uint32_t zraw[3], wsraw[9];
#pragma unroll
  for (int i = 0; i < 3; ++i) zraw[i] = zr[i];
#pragma unroll
  for (int i = 0; i < 9; ++i) wsraw[i] = wsp[i];
  // taps kept as loaded (bf16 bits, tap k of channel h0+c) until after the
  // slot lookup has been issued
  bf16_t wb[2][7];
  if constexpr (WT) {
#pragma unroll
    for (int k = 0; k < 7; ++k) {
      const uint32_t v = *reinterpret_cast<const uint32_t *>(w + (int64_t)k * a.wi1 + h0);
      wb[0][k] = static_cast<bf16_t>(v);
      wb[1][k] = static_cast<bf16_t>(v >> 16);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int k = 0; k < 7; ++k) wb[c][k] = w[(int64_t)(h0 + c) * a.wi0 + k];
  }
  uint32_t dv = 0;
  if constexpr (HAS_D) dv = *reinterpret_cast<const uint32_t *>(a.D + h0);

  // the loads above go out before the slot lookup below is waited on
  __builtin_amdgcn_sched_barrier(0);
  int64_t blk;
  const bool live = row_slot(a, b, blk);  // uniform
  bf16_t *cbase = a.cs + blk * a.cs0 + 3 * (int64_t)h0;
  uint32_t *c0p = reinterpret_cast<uint32_t *>(cbase);
  uint32_t *c1p = reinterpret_cast<uint32_t *>(cbase + a.cs2);
  float *s = a.st + blk * a.is0 + h0;
  uint32_t c0raw[3], c1raw[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    c0raw[i] = c0p[i];
    c1raw[i] = c1p[i];
  }
  float2 sv[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) sv[k] = *reinterpret_cast<const float2 *>(s + k * a.is2);

  float x2[2], u[2], y[2];
  pair_featurize(zraw, c0raw, c1raw, wsraw, x2, u);
  float wf[2][7];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int k = 0; k < 7; ++k) wf[c][k] = bf2f(wb[c][k]);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float s6[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) s6[k] = c ? sv[k].y : sv[k].x;
    // triton_decode.py:126-143: ((((s0w0+s4w4)+(s1w1+s5w5))+s2w2)+s3w3)+w6u
    const float aa = (s6[0] * wf[c][0] + 0.0f) + s6[4] * wf[c][4];
    const float bb = (s6[1] * wf[c][1] + 0.0f) + s6[5] * wf[c][5];
    const float cc = s6[2] * wf[c][2] + 0.0f;
    const float dd = s6[3] * wf[c][3] + 0.0f;
    y[c] = rbf((((aa + bb) + cc) + dd) + wf[c][6] * u[c]);
  }
  if constexpr (HAS_D) {
    y[0] = rbf(y[0] + rbf(lo_bf(dv) * u[0]));
    y[1] = rbf(y[1] + rbf(hi_bf(dv) * u[1]));
  }
  if (!active) return;
  if (live) {
#pragma unroll
    for (int k = 0; k < 5; ++k) *reinterpret_cast<float2 *>(s + k * a.is2) = sv[k + 1];
    *reinterpret_cast<float2 *>(s + 5 * a.is2) = make_float2(u[0], u[1]);
    // Short-filter windows (c0, c1) <- (c1, x) for the 6 sub-channels.
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      c0p[i] = c1raw[i];
      c1p[i] = zraw[i];
    }
  }
  *reinterpret_cast<uint32_t *>(a.out + b * a.so + h0) =
      pack_bf(x2[0] * y[0], x2[1] * y[1]) & live_mask(live);
}

template <bool HAS_D, bool WT>
static void launch_hcs_pair(const DecodeArgs &a, int64_t B, hipStream_t stream) {
  constexpr int BT = 128;  // 256 channels per block
  dim3 grid(static_cast<unsigned>(cdiv(a.H / 2, BT)), static_cast<unsigned>(B));
  hipLaunchKernelGGL((hcs_decode_pair_kernel<HAS_D, WT>), grid, dim3(BT), 0, stream, a);
}

// ---------------------------------------------------------------------------
// hcm with the window split over four waves.  A workgroup owns one row and 64
// channel pairs; wave m holds window columns k = 16j + 4m + l (j < 8, l < 4),
// so its four accumulators are exactly the reference's acc[m][0..3] summed
// over j in order.  Waves 1-3 hand theirs to wave 0 through LDS, which
// combines them in the reference's order.  Every wave issues all its column
// loads at once (32 x 512 B in flight per wave, four times the pair kernel's
// per-channel share), and the shifted stores wait for a barrier: a wave
// writes column 16j + 4m - 1, which another wave loads.

template <bool HAS_D, bool WT>
__global__ __launch_bounds__(256) void hcm_decode_split_kernel(DecodeArgs a) {
  __shared__ float2 part[3][4][64];
  const int lane = threadIdx.x & 63;
  const int m = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;  // 256 threads
  const int h0 = 2 * (blockIdx.x * 64 + lane);
  const bool active = h0 < a.H;
  const int hc = active ? h0 : 0;
  const int64_t b = blockIdx.y;
  const bf16_t *w = static_cast<const bf16_t *>(a.inner);
  // Taps and window go through buffer descriptors: one lane offset in a
  // VGPR, the column offset in an SGPR, instead of a live 64-bit address per
  // access (which held the kernel at 192 VGPRs).  Record counts are the byte
  // extents, checked on the host to fit 32 bits.
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(w), 0,
      static_cast<int>(WT ? (126 * a.wi1 + a.H) * 2 : ((int64_t)(a.H - 1) * a.wi0 + 128) * 2),
      0x00020000);

  // Taps stay packed as loaded (bf16 pairs) and are widened at use (149
  // VGPRs: three waves per SIMD).  WT: tw[j][l] = (h0, h0+1) of
  // tap k; otherwise tw[j][2c], tw[j][2c+1] = taps (4m..4m+3) of channel h0+c.
  // They go out before the slot lookup, the window columns after it.
  uint32_t tw[8][4];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (WT) {
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const int k = 16 * j + 4 * m + l;
        tw[j][l] = k < 127 ? static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(
                                 wrs, 2 * hc, static_cast<int>(k * a.wi1 * 2), 0))
                           : 0u;
      }
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const auto t = __builtin_amdgcn_raw_buffer_load_b64(
            wrs, static_cast<int>((hc + c) * a.wi0 * 2), (16 * j + 4 * m) * 2, 0);
        tw[j][2 * c] = static_cast<uint32_t>(t[0]);
        tw[j][2 * c + 1] = (16 * j + 4 * m + 3 < 127) ? static_cast<uint32_t>(t[1])
                                                       : (static_cast<uint32_t>(t[1]) & 0xffffu);
      }
    }
  }
  // wave 0's epilogue operands that do not depend on the slot either (the
  // last tap and D) go out with the taps: fetched after the stores, they put
  // a memory round trip at the end of every workgroup
  uint32_t lastraw = 0u, draw = 0u;
  // and so do its short-filter inputs that do not depend on the slot
  uint32_t zraw[3], wsraw[9];
  if (m == 0) {
    if constexpr (WT) lastraw = *reinterpret_cast<const uint32_t *>(w + (int64_t)127 * a.wi1 + hc);
    else lastraw = pair_bf(w[(int64_t)hc * a.wi0 + 127], w[(int64_t)(hc + 1) * a.wi0 + 127]);
    if constexpr (HAS_D) draw = *reinterpret_cast<const uint32_t *>(a.D + hc);
    const uint32_t *zr = reinterpret_cast<const uint32_t *>(a.z + b * a.sz + 3 * (int64_t)hc);
    const uint32_t *wsp = reinterpret_cast<const uint32_t *>(a.ws + 9 * (int64_t)hc);
#pragma unroll
    for (int i = 0; i < 3; ++i) zraw[i] = zr[i];
#pragma unroll
    for (int i = 0; i < 9; ++i) wsraw[i] = wsp[i];
  }
  __builtin_amdgcn_sched_barrier(0);
  int64_t blk;
  const bool live = row_slot(a, b, blk);  // uniform
  float *s = a.st + blk * a.is0 + hc;  // is1 == 1: the pair is one float2
  // wave 0's conv window goes out before the window columns: the column
  // loads return in order, so a load issued after them would hold the short
  // filter until the whole window had arrived
  uint32_t c0raw[3], c1raw[3];
  uint32_t *c0p = nullptr, *c1p = nullptr;
  if (m == 0) {
    bf16_t *cbase = a.cs + blk * a.cs0 + 3 * (int64_t)hc;
    c0p = reinterpret_cast<uint32_t *>(cbase);
    c1p = reinterpret_cast<uint32_t *>(cbase + a.cs2);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      c0raw[i] = ld_nt(c0p + i);
      c1raw[i] = ld_nt(c1p + i);
    }
  }
  // The window moves through buffer loads and stores on a descriptor of this
  // block's window (records = its byte extent, checked on the host to fit 32
  // bits): one lane offset in a VGPR, the column offset in an SGPR, so no
  // per-column 64-bit address has to stay live from the loads to the
  // shifted stores after the barrier.
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      a.st + blk * a.is0, 0, static_cast<int>((126 * a.is2 + a.H) * 4), 0x00020000);
  // The window's loads and stores carry the non-temporal hint: read once and
  // rewritten once per step, its 2 MB per row are streamed rather than kept
  // in the caches.  Measured at 7B (64 rows, in graphs): 56.8 us plain, 49.2
  // with both loads and stores non-temporal, 56.5 with the loads alone; the
  // whole 27-core step 0.715 -> 0.614 ms, as the 276 MB stream no longer
  // evicts what the other kernels reuse.  The hcs and hcl kernels keep plain
  // accesses: the hint there made the step slower (0.617 ms).
  const int ls = 4 * hc;
  float2 v[8][4];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int k = 16 * j + 4 * m + l;
      if (k < 127) {
        const auto t = __builtin_amdgcn_raw_buffer_load_b64(srs, ls, static_cast<int>(k * a.is2 * 4), CPOL_NT);
        v[j][l] = make_float2(__int_as_float(t[0]), __int_as_float(t[1]));
      } else {
        v[j][l] = make_float2(0.f, 0.f);
      }
    }
  // bf16 tap l of channel c (0 = h0, 1 = h0 + 1) for column group j
  auto tap = [&](int j, int l, int c) -> float {
    if constexpr (WT) return c ? hi_bf(tw[j][l]) : lo_bf(tw[j][l]);
    const uint32_t t = tw[j][2 * c + (l >> 1)];
    return (l & 1) ? hi_bf(t) : lo_bf(t);
  };

  // Wave 0: the short filter on the 6 sub-channels of the pair and the gate,
  // while the window columns are still arriving.
  float x2[2] = {0.f, 0.f}, u[2] = {0.f, 0.f};
  if (m == 0) pair_featurize(zraw, c0raw, c1raw, wsraw, x2, u);

  float acc[2][4];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int l = 0; l < 4; ++l) acc[c][l] = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      acc[0][l] = acc[0][l] + v[j][l].x * tap(j, l, 0);
      acc[1][l] = acc[1][l] + v[j][l].y * tap(j, l, 1);
    }
  if (m > 0) {
#pragma unroll
    for (int l = 0; l < 4; ++l) part[m - 1][l][lane] = make_float2(acc[0][l], acc[1][l]);
  }
  __syncthreads();  // all window loads consumed; partial sums visible

  if (active && live) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const int k = 16 * j + 4 * m + l;
        if (k >= 1 && k < 127) {
          typedef __attribute__((ext_vector_type(2))) int i32x2;
          const i32x2 t = {__float_as_int(v[j][l].x), __float_as_int(v[j][l].y)};
          __builtin_amdgcn_raw_buffer_store_b64(t, srs, ls, static_cast<int>((k - 1) * a.is2 * 4), CPOL_NT);
        }
      }
  }
  if (m != 0 || !active) return;
  const float last[2] = {lo_bf(lastraw), hi_bf(lastraw)};
  float y[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float p[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const float2 p1 = part[0][l][lane], p2 = part[1][l][lane], p3 = part[2][l][lane];
      p[l] = ((acc[c][l] + (c ? p1.y : p1.x)) + (c ? p2.y : p2.x)) + (c ? p3.y : p3.x);
    }
    y[c] = rbf(((p[0] + p[2]) + (p[1] + p[3])) + last[c] * u[c]);
  }
  if (live) {
    st_nt(reinterpret_cast<float2 *>(s + 126 * a.is2), make_float2(u[0], u[1]));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      st_nt(c0p + i, c1raw[i]);
      st_nt(c1p + i, zraw[i]);
    }
  }
  if constexpr (HAS_D) {
    y[0] = rbf(y[0] + rbf(lo_bf(draw) * u[0]));
    y[1] = rbf(y[1] + rbf(hi_bf(draw) * u[1]));
  }
  *reinterpret_cast<uint32_t *>(a.out + b * a.so + h0) =
      pack_bf(x2[0] * y[0], x2[1] * y[1]) & live_mask(live);
}

template <bool HAS_D, bool WT>
static void launch_hcm_split(const DecodeArgs &a, int64_t B, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(cdiv(a.H / 2, 64)), static_cast<unsigned>(B));
  hipLaunchKernelGGL((hcm_decode_split_kernel<HAS_D, WT>), grid, dim3(256), 0, stream, a);
}

// ---------------------------------------------------------------------------
// hcl with four lanes per channel: lane q of a quad owns states 4q..4q+3, so
// the state, residue and log-pole rows move as one float4 per lane with the
// 64 lanes of a wave covering 1 KB contiguously.  Lanes 0-2 of the quad run
// the short filter for sub-channels x2, x1, v; the values are shared with
// quad DPP moves.  The readout keeps the reference's halving tree:
// r[i] += r[i+8] (lane q takes lane q+2), r[i] += r[i+4] (lane 0 takes lane
// 1), r[i] += r[i+2] in lane 0, y = r0 + r1 (triton_decode.py:81-96).
//
// A workgroup owns 64 channels of HCL_RB rows: the residues, log-poles and
// exp(log-poles) are fetched and computed once for those rows, and every
// row's slot, state, window and z loads are issued before any of them is
// used, so one memory round trip (after the slot lookup) covers all rows.
// Rows on the null block (or past the batch) read block 0, which always
// exists, and write nothing but a zero output.
constexpr int HCL_RB = 4;

template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <bool HAS_D>
__global__ __launch_bounds__(256) void hcl_decode_quad_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int q = lane & 3;
  const int h = blockIdx.x * 64 + (threadIdx.x >> 2);
  const bool active = h < a.H;
  const int hc = active ? h : a.H - 1;
  const int b0 = blockIdx.y * HCL_RB;
  const int i = q < 3 ? q : 2;  // short-filter sub-channel (lane 3 mirrors lane 2)
  const int64_t ch = 3 * (int64_t)hc + i;

  const float4 r4 = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.inner) +
                                                      (int64_t)hc * a.wi0 + 4 * q);
  const float4 l4 = *reinterpret_cast<const float4 *>(a.lp + (int64_t)hc * a.lp0 + 4 * q);
  const bf16_t w0b = a.ws[ch * 3], w1b = a.ws[ch * 3 + 1], w2b = a.ws[ch * 3 + 2];
  const bf16_t db = HAS_D ? a.D[hc] : bf16_t(0);
  bf16_t xb[HCL_RB];
#pragma unroll
  for (int r = 0; r < HCL_RB; ++r) xb[r] = a.z[(int64_t)min(b0 + r, a.rows - 1) * a.sz + ch];
  __builtin_amdgcn_sched_barrier(0);  // the loads above go out before the slot lookups
  int64_t blk[HCL_RB];
  bool live[HCL_RB];
  int32_t sl[HCL_RB];
#pragma unroll
  for (int r = 0; r < HCL_RB; ++r) sl[r] = a.slots[(int64_t)min(b0 + r, a.rows - 1) * a.ssl];
#pragma unroll
  for (int r = 0; r < HCL_RB; ++r) {
    live[r] = (b0 + r < a.rows) & (sl[r] != a.null_block) & (sl[r] >= 0) & (sl[r] < a.num_blocks);
    blk[r] = live[r] ? sl[r] : 0;
  }
  float4 s4[HCL_RB];
  bf16_t c0b[HCL_RB], c1b[HCL_RB];
#pragma unroll
  for (int r = 0; r < HCL_RB; ++r) {
    s4[r] = *reinterpret_cast<const float4 *>(a.st + blk[r] * a.is0 + (int64_t)hc * a.is1 + 4 * q);
    const bf16_t *cw = a.cs + blk[r] * a.cs0 + ch * a.cs1;
    c0b[r] = cw[0];
    c1b[r] = cw[a.cs2];
  }
  const float rv[4] = {r4.x, r4.y, r4.z, r4.w};
  const float pe[4] = {expf(l4.x), expf(l4.y), expf(l4.z), expf(l4.w)};
  const float w0 = bf2f(w0b), w1 = bf2f(w1b), w2 = bf2f(w2b), dval = bf2f(db);

#pragma unroll
  for (int r = 0; r < HCL_RB; ++r) {
    // bf16(((0 + bf16(c0 w0)) + bf16(c1 w1)) + bf16(x w2)) (triton_decode.py:44-53)
    float acc = 0.0f + rbf(bf2f(c0b[r]) * w0);
    acc = acc + rbf(bf2f(c1b[r]) * w1);
    acc = acc + rbf(bf2f(xb[r]) * w2);
    const float yi = rbf(acc);
    const float x2 = quad_perm<0x00>(yi);
    const float x1 = quad_perm<0x55>(yi);
    const float vv = quad_perm<0xAA>(yi);
    const float u = rbf(x1 * vv);
    float sv[4] = {s4[r].x, s4[r].y, s4[r].z, s4[r].w};
    float rr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sv[e] = sv[e] * pe[e] + u;
      rr[e] = sv[e] * rv[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) rr[e] = rr[e] + quad_perm<0xEE>(rr[e]);  // lane q += lane q+2
#pragma unroll
    for (int e = 0; e < 4; ++e) rr[e] = rr[e] + quad_perm<0xF5>(rr[e]);  // lane 0 += lane 1
    rr[0] = rr[0] + rr[2];
    rr[1] = rr[1] + rr[3];
    float y = rbf((rr[0] + rr[1]) + 0.0f);
    if constexpr (HAS_D) y = rbf(y + rbf(dval * u));

    if (live[r] && active) {  // live is uniform
      *reinterpret_cast<float4 *>(a.st + blk[r] * a.is0 + (int64_t)h * a.is1 + 4 * q) =
          make_float4(sv[0], sv[1], sv[2], sv[3]);
      if (q < 3) {
        bf16_t *cw = a.cs + blk[r] * a.cs0 + ch * a.cs1;
        cw[0] = c1b[r];
        cw[a.cs2] = xb[r];
      }
    }
    if (q == 0 && active && b0 + r < a.rows)
      a.out[(int64_t)(b0 + r) * a.so + h] = f2bf(x2 * y) & static_cast<bf16_t>(live_mask(live[r]));
  }
}

template <bool HAS_D>
static void launch_hcl_quad(const DecodeArgs &a, int64_t B, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(cdiv(a.H, 64)), static_cast<unsigned>(cdiv(B, HCL_RB)));
  hipLaunchKernelGGL((hcl_decode_quad_kernel<HAS_D>), grid, dim3(256), 0, stream, a);
}

static bool aligned(const void *p, uintptr_t n) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % n) == 0;
}

// Which fast-path variant applies: -1 none, 0 row-major taps, 1 transposed.
static int pair_variant(const DecodeArgs &a, int kind) {
  if (a.H % 2) return -1;
  if (a.sz % 2 || !aligned(a.z, 4)) return -1;
  if (a.cs1 != 1 || a.cs0 % 2 || a.cs2 % 2 || !aligned(a.cs, 4)) return -1;
  if (!aligned(a.ws, 4) || !aligned(a.D, 4)) return -1;
  if (a.so % 2 || !aligned(a.out, 4)) return -1;
  if (kind == KIND_HCL) {
    const bool ok = a.is2 == 1 && a.is1 % 4 == 0 && a.is0 % 4 == 0 && aligned(a.st, 16) &&
                    a.wi1 == 1 && a.wi0 % 4 == 0 && aligned(a.inner, 16) &&
                    a.lp1 == 1 && a.lp0 % 4 == 0 && aligned(a.lp, 16);
    return ok ? 0 : -1;
  }
  if (a.is1 != 1 || a.is0 % 2 || a.is2 % 2 || !aligned(a.st, 8)) return -1;
  // hcm addresses a block's window through a buffer descriptor: its byte
  // extent must fit the 32-bit record count
  if (kind == KIND_HCM && (a.is2 < 0 || (126 * a.is2 + a.H) * 4 >= (int64_t(1) << 31))) return -1;
  // and so do its taps' (either layout)
  if (kind == KIND_HCM && (a.wi0 < 0 || a.wi1 < 0 || (126 * a.wi1 + a.H) * 2 >= (int64_t(1) << 31) ||
                           ((a.H - 1) * a.wi0 + 128) * 2 >= (int64_t(1) << 31)))
    return -1;
  if (a.wi0 == 1 && a.wi1 % 2 == 0 && aligned(a.inner, 4)) return 1;
  if (a.wi1 == 1) {
    if (kind == KIND_HCS) return 0;
    if (a.wi0 % 8 == 0 && aligned(a.inner, 16)) return 0;
  }
  return -1;
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_hyena_decode(const void *z, int64_t sz, const void *short_w,
                                 void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                                 const int32_t *slots, int64_t ssl,
                                 const void *inner, int64_t wi0, int64_t wi1,
                                 const float *log_poles, int64_t lp0, int64_t lp1,
                                 float *inner_state, int64_t is0, int64_t is1, int64_t is2,
                                 const void *D, void *out, int64_t so,
                                 int64_t B, int64_t H, int32_t K, int32_t is_iir,
                                 int32_t null_block, int64_t num_blocks, void *stream) {
  if (B < 0 || H <= 0 || H > (1 << 30) || num_blocks <= 0)
    return fail(EVO2_ERR_INVALID, "hyena_decode: bad sizes B=%lld H=%lld blocks=%lld",
                (long long)B, (long long)H, (long long)num_blocks);
  if (B == 0) return EVO2_OK;
  if (B > 65535)
    return fail(EVO2_ERR_UNSUPPORTED, "hyena_decode: B=%lld exceeds 65535 rows", (long long)B);
  if (!z || !short_w || !conv_state || !slots || !inner || !inner_state || !out)
    return fail(EVO2_ERR_INVALID, "hyena_decode: null pointer argument");
  int kind;
  if (is_iir) {
    if (K != 16 || !log_poles)
      return fail(EVO2_ERR_INVALID, "hyena_decode: LI needs 16 poles and log_poles (K=%d)", K);
    kind = KIND_HCL;
  } else if (K == 7) {
    kind = KIND_HCS;
  } else if (K == 128) {
    kind = KIND_HCM;
  } else {
    return fail(EVO2_ERR_UNSUPPORTED, "hyena_decode: inner FIR length %d (7 or 128 only)", K);
  }
  DecodeArgs a{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
               static_cast<bf16_t *>(conv_state), cs0, cs1, cs2, slots, ssl,
               inner, wi0, wi1, log_poles, lp0, lp1, inner_state, is0, is1, is2,
               static_cast<const bf16_t *>(D), static_cast<bf16_t *>(out), so,
               static_cast<int>(H), null_block, num_blocks, static_cast<int>(B)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool hasD = D != nullptr;
  const int pv = pair_variant(a, kind);
  if (pv >= 0) {
    if (kind == KIND_HCL) {
      hasD ? launch_hcl_quad<true>(a, B, st) : launch_hcl_quad<false>(a, B, st);
    } else if (kind == KIND_HCM) {
      if (pv) hasD ? launch_hcm_split<true, true>(a, B, st) : launch_hcm_split<false, true>(a, B, st);
      else hasD ? launch_hcm_split<true, false>(a, B, st) : launch_hcm_split<false, false>(a, B, st);
    } else {
      if (pv) hasD ? launch_hcs_pair<true, true>(a, B, st) : launch_hcs_pair<false, true>(a, B, st);
      else hasD ? launch_hcs_pair<true, false>(a, B, st) : launch_hcs_pair<false, false>(a, B, st);
    }
    return check_launch("hyena_decode");
  }
  if (kind == KIND_HCL) {
    const bool contig = is2 == 1 && (is1 % 4) == 0 && (is0 % 4) == 0 &&
                        (reinterpret_cast<uintptr_t>(inner_state) % 16) == 0;
    if (hasD) {
      contig ? launch<KIND_HCL, true, true>(a, B, st) : launch<KIND_HCL, true, false>(a, B, st);
    } else {
      contig ? launch<KIND_HCL, false, true>(a, B, st) : launch<KIND_HCL, false, false>(a, B, st);
    }
  } else if (kind == KIND_HCM) {
    hasD ? launch<KIND_HCM, true, false>(a, B, st) : launch<KIND_HCM, false, false>(a, B, st);
  } else {
    hasD ? launch<KIND_HCS, true, false>(a, B, st) : launch<KIND_HCS, false, false>(a, B, st);
  }
  return check_launch("hyena_decode");
}
