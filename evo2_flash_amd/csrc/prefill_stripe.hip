// Single-pass prefill of the hcm (128-tap FIR) and hcl (16-pole modal LI)
// mixer cores for gfx950, z (T, 3H) -> g (T, H):
//   short K=3 filter -> u = x1 v -> inner filter y -> g = x2 bf16(bf16(y) [+ bf16(u D)])
// (mixers.py:1277-1305 for hcm, 1327-1401 for hcl; the rounding points are
// the fused VALU kernels' and the reference's).
//
// Work split.  A workgroup owns 16 channels of one whole segment (tile table
// with one tile per segment) and sweeps it in sub-tiles of 256 rows, so
//  * the LI state crosses sub-tiles inside the workgroup: z is read once and
//    there is no carry pass (the tiled LI form reads z twice);
//  * the FIR history stays in an LDS ring: no halo rows are re-read.
// The four 16-channel workgroups of a 64-channel block are workgroups b,
// b + 8, b + 16, b + 24: one XCD, dispatched together, so the 384-byte row
// slice of the block is fetched once into that XCD's L2.
//
// Waves.  Eight waves in two roles, one barrier per sub-tile:
//   featurizer waves 0-3: direct-to-LDS z loads two sub-tiles ahead into a
//     three-slot ring; thread (channel tid % 16, rows 16 (tid / 16) ..+15)
//     runs the short filter and the gate and writes u and x2 channel-major;
//   matrix waves 4-7: four channels each, the inner filter of the previous
//     sub-tile on the matrix cores, the epilogue, and the stores of the
//     sub-tile before that through a row-major LDS buffer.
//
// The inner filter on v_mfma_f32_16x16x32_bf16.  Rows of a sub-tile form 16
// chunks of 16; chunk n is column n of the B operand and output row i of
// chunk n is row 16 n + i.
//  * hcm: y[16n + i] = sum_j A[i][j] W_n[j] with the 160-row window
//    W_n[j] = u[16n - 144 + j] and A[i][j] = w[j - i - 17] (zero outside
//    0..127): five k-steps over an LDS ring of u with 144 rows of history.
//    Taps and u are bf16, so every product is exact; only the fp32
//    summation order differs from a per-tap loop.
//  * hcl: with p = exp(lp) per pole, h[m] = sum_s r_s p_s^m and the state
//    S_s(t) = p_s S_s(t-1) + u(t), per chunk n
//      y[16n + i] = sum_{j<=i} h[i-j] u[16n+j]          (intra-chunk Toeplitz)
//                 + sum_s r_s p_s^(i+1) S_s(16n - 1)      (state before the chunk)
//      X_s(n)     = sum_j p_s^(15-j) u[16n + j]           (chunk end state from 0)
//    X comes from one MFMA, the states before each chunk from a 16-lane scan
//    of X over the chunks (DPP row shifts, multipliers p^16, p^32, p^64,
//    p^128) plus p^(16n) times the state entering the sub-tile, and the
//    readout from two more MFMAs.  The fp32 coefficients (h, p^k, r p^k) and
//    the states are split into bf16 high and low parts, so the products keep
//    ~16 mantissa bits: the result agrees with the fp32 recurrence to
//    ~1e-5 relative, far inside the bf16 output rounding.
#include <type_traits>

#include "featurize.h"
#include "stripe.h"

namespace evo2 {
namespace stripe {
constexpr int CH = 16;                // channels per workgroup
constexpr int RS = 256;               // rows per sub-tile: 16 chunks of 16
constexpr int NF = 4;                 // featurizer waves
constexpr int NM = 4;                 // matrix waves
constexpr int NT = 64 * (NF + NM);
constexpr int CPW = CH / NM;          // channels per matrix wave
constexpr int ZW = 3 * CH;            // bf16 per staged z row (x2, x1, v triples)
constexpr int ZROWS = RS + 2;         // staged rows: the sub-tile and the short filter's 2-row halo
constexpr int ZCH = ZROWS * 6;        // 16-byte chunks of a slot's rows
constexpr int ZINS = (ZCH + 63) / 64; // wave loads per slot: wave w issues loads w, w + NF, ...
constexpr int SLOT = ZINS * 512;      // bf16 per slot (the last load's spare lanes land past row 257)
constexpr int UP = RS + 8;            // channel pitch (bf16) of the u and x2 buffers
constexpr int HIST = 144;             // hcm: ring rows before a sub-tile its windows reach
constexpr int RING = 768;             // hcm: ring rows per channel (>= HIST + 2 RS; pitch 776 keeps the bank spread)
constexpr int RP = RING + 8;          // hcm: ring pitch (bf16)
constexpr int KS = 5;                 // hcm: k-steps over the 160-row window
constexpr int TAPW = 176;             // hcm: zero-padded taps per channel for the A build
constexpr int ETAB = 17;              // hcl: p^m for m = 0..16 per pole
static_assert(HIST + 2 * RS <= RING && RING % 16 == 0, "ring: one sub-tile in flight each way, whole 16-row groups");
constexpr int NSLOT = 4;              // z staging slots: NSLOT - 1 sub-tiles in flight
static_assert((UP / 2) % 64 == 4 && (RP / 2) % 64 == 4, "pitches spread 16 channels over the banks");
static_assert(CH * TAPW <= SLOT, "the tap table borrows a staging slot");
// loads per slot of featurizer wave w; the sweep's waits assume waves 1..NF-1
// issue the same number and the prefetch loop bound covers them all
__host__ __device__ constexpr int zloads(int w) { return (ZINS - w + NF - 1) / NF; }
static_assert(zloads(1) == zloads(NF - 1) && NF * (NF + 3) >= ZINS, "featurizer wave load counts");
static_assert(CH * 16 * (ETAB + 2) * 4 <= SLOT * 2, "the LI tables borrow a staging slot");
}  // namespace stripe

typedef __attribute__((ext_vector_type(8))) __bf16 sbf16x8_t;
typedef __attribute__((ext_vector_type(4))) float sf32x4_t;
typedef __attribute__((ext_vector_type(4))) int si32x4_t;

// High and low bf16 parts of an fp32 value: v ~= hi + lo to ~16 bits.
__device__ __forceinline__ __bf16 bf_hi(float v) { return static_cast<__bf16>(v); }
__device__ __forceinline__ __bf16 bf_lo(float v) {
  return static_cast<__bf16>(v - static_cast<float>(static_cast<__bf16>(v)));
}

// Workgroup barrier for the sweep: this wave's LDS writes complete, then
// s_barrier.  __syncthreads() adds a release fence, which waits for every
// direct-to-LDS load still in flight (the next sub-tiles' z rows) as well;
// here each featurizer wave waits for exactly the loads the next step reads
// before it arrives.  The memory clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void sweep_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Lane l of each 16-lane row reads lane l - D of the same row (0 below D).
template <int D>
__device__ __forceinline__ float row_shr(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 | D, 0xf, 0xf, true));
}

template <int KIND, bool HAS_D, int NS>
__global__ __launch_bounds__(stripe::NT, 1) void stripe_kernel(StripeArgs p, int64_t units, int nblk64) {
  using namespace stripe;
  constexpr bool HCL = KIND == STRIPE_HCL;
  __shared__ __align__(16) bf16_t zs0[SLOT];
  __shared__ __align__(16) bf16_t zs1[SLOT];
  __shared__ __align__(16) bf16_t zs2[SLOT];
  __shared__ __align__(16) bf16_t zs3[NS > 3 ? SLOT : 8];
  static_assert(NS == 3 || NS == 4, "three or four staging slots");
  __shared__ __align__(16) bf16_t ubuf[HCL ? 2 * CH * UP : CH * RP];
  __shared__ __align__(16) bf16_t xbuf[2 * CH * UP];
  __shared__ __align__(16) bf16_t gbuf[2 * RS * CH];
  __shared__ float sfin[HCL ? CH * 16 : 1];                  // hcl: state before the last chunk

  // ---- workgroup -> (segment, 16-channel group)
  const int L = blockIdx.x;
  const int jslot = L >> 3;
  const int64_t unit = (static_cast<int64_t>(jslot >> 2) << 3) + (L & 7);
  if (unit >= units) return;  // uniform
  const int seg = static_cast<int>(unit / nblk64);
  const int c0 = static_cast<int>(unit % nblk64) * 64 + (jslot & 3) * CH;
  if (c0 >= p.H) return;  // uniform
  const int a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  if (e <= a) return;  // uniform
  const int64_t blk = p.blocks[seg * p.sblk];
  const bool blk_ok = blk >= 0 && blk < p.num_blocks;
  const bool init = p.seq[3 * seg + 2] != 0 && blk_ok;
  const int nsub = (e - a + RS - 1) / RS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool is_f = wave < NF;
  // featurizer role: channel fpc, rows 16 fprg .. 16 fprg + 15 of a sub-tile
  const int fpc = tid & (CH - 1);
  const int fprg = (tid >> 4) & 15;
  // matrix role: wave mw, lane (l16 = lane % 16, g = lane / 16)
  const int mw = wave - NF;
  const int l16 = lane & 15, g = lane >> 4;

  auto slot_ptr = [&](auto s) __attribute__((always_inline)) -> bf16_t * {
    constexpr int S = decltype(s)::value;
    return S == 0 ? zs0 : (S == 1 ? zs1 : (S == 2 ? zs2 : zs3));
  };

  // ---- z rows s0 - 2 .. s0 + 255 of sub-tile i (s0 = a + 256 i) into slot
  // rows 0 .. 257 by direct-to-LDS loads: chunk q = 64 (wave + NF j) + lane
  // is 16 bytes of slot row q / 6.  Rows past the segment end (and the spare
  // lanes of the last load) load the segment's last row again, never read;
  // rows before the segment start (sub-tile 0's halo) are not loaded: they
  // come from the conv window.
  auto prefetch = [&](auto s, int i) __attribute__((always_inline)) {
    bf16_t *dst = slot_ptr(s);
    const int s0 = a + RS * i - 2;
    const char *base = reinterpret_cast<const char *>(p.z + (int64_t)s0 * p.sz + 3 * c0);
    const int last = e - 1 - s0;
#pragma unroll
    for (int j = 0; j < NF + 3; ++j) {
      const int cw = wave + NF * j;
      if (cw < ZINS) {  // uniform
        const int q = 64 * cw + lane;
        const int row = q / 6;
        const int col = q - 6 * row;
        const uint32_t off = 2u * static_cast<uint32_t>(min(row, last) * static_cast<int>(p.sz) + 8 * col);
        if (i > 0 || row >= 2)  // sub-tile 0: lanes 0..11 of load 0 skip the halo rows
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(base + off),
                                           (__attribute__((address_space(3))) void *)(dst + 512 * cw),
                                           16, 0, 0);
      }
    }
  };
  // the short filter's left context of sub-tile 0, slot rows 0, 1 = rows
  // a - 2, a - 1: the conv window (column 0 = a - 2) when continuing, else
  // zero; written before any load targets the slot
  if (tid < 2 * ZW) {
    const int q = tid / ZW, k = tid - ZW * q;
    bf16_t v = 0;
    if (init) v = p.cs[blk * p.cs0 + (int64_t)(3 * c0 + k) * p.cs1 + q * p.cs2];
    zs0[tid] = v;
  }
  if (is_f) {
    prefetch(std::integral_constant<int, 0>{}, 0);
    if (nsub > 1) prefetch(std::integral_constant<int, 1>{}, 1);
    if constexpr (NS > 3) {
      if (nsub > 2) prefetch(std::integral_constant<int, 2>{}, 2);
    }
  }

  // ---- per-role constants
  ShortTaps wsp[3];
  if (is_f) {
#pragma unroll
    for (int i = 0; i < 3; ++i) wsp[i] = short_taps(p.ws, 3 * (int64_t)(c0 + fpc) + i);
  }
  float dv[CPW];
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc) dv[cc] = 0.f;
  if constexpr (HAS_D) {
    if (!is_f) {
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) dv[cc] = bf2f(p.D[c0 + CPW * mw + cc]);
    }
  }

  // hcm: A fragments (lane (i, kg), k-step s, element x holds
  // A[i][32 s + 8 kg + x] = w[32 s + 8 kg + x - i - 17]) and the ring's
  // history rows a - 144 .. a - 1 (the old window's columns, col 0 = a - 127)
  sbf16x8_t A[HCL ? 1 : CPW][HCL ? 1 : KS];
  // hcl: per channel the A fragments of the intra-chunk Toeplitz (AT), the
  // chunk end states (AB) and the readout (AC high, AC2 low parts), and per
  // lane (column n = l16, poles 4 g .. 4 g + 3): p^16, p^(16 n), the state
  // entering the sub-tile
  sbf16x8_t AT[HCL ? CPW : 1], AB[HCL ? CPW : 1], AC[HCL ? CPW : 1], AC2[HCL ? CPW : 1];
  float P16[HCL ? CPW : 1][4], carry[HCL ? CPW : 1][4];
  if constexpr (!HCL) {
    bf16_t *tp = slot_ptr(std::integral_constant<int, NS - 1>{});
    for (int i = tid; i < CH * TAPW; i += NT) {
      const int ch = i / TAPW, k = i - ch * TAPW - 32;
      bf16_t v = 0;
      if (k >= 0 && k < 128) v = p.w[(int64_t)(c0 + ch) * p.w0 + k];
      tp[i] = v;
    }
    for (int i = tid; i < CH * HIST; i += NT) {
      const int ch = i / HIST, r = i - HIST * ch;  // ring slot r holds row a - 144 + r
      const int col = r - (HIST - 127);
      float u = 0.f;
      if (init && col >= 0) u = p.st[blk * p.st0 + (int64_t)(c0 + ch) * p.st1 + (int64_t)col * p.st2];
      ubuf[ch * RP + r] = f2bf(u);
    }
    __syncthreads();
    if (!is_f) {
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc)
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int x = 0; x < 8; ++x)
            A[cc][s][x] = __builtin_bit_cast(__bf16, tp[(CPW * mw + cc) * TAPW + 32 * s + 8 * g + x - l16 + 15]);
    }
  } else {
    float *E = reinterpret_cast<float *>(slot_ptr(std::integral_constant<int, NS - 1>{}));  // [CH][16 poles][ETAB]: p^m
    float *R = E + CH * 16 * ETAB;              // [CH][16]: residues
    float *Hf = R + CH * 16;                    // [CH][16]: h[m], m < 16
    for (int i = tid; i < CH * 16 * ETAB; i += NT) {
      const int ch = i / (16 * ETAB), rem = i - ch * 16 * ETAB, q = rem / ETAB, m = rem - q * ETAB;
      E[i] = expf(p.lp[(int64_t)(c0 + ch) * p.l0 + q * p.l1] * static_cast<float>(m));
    }
    for (int i = tid; i < CH * 16; i += NT) R[i] = p.res[(int64_t)(c0 + (i >> 4)) * p.r0 + (i & 15) * p.r1];
    __syncthreads();
    for (int i = tid; i < CH * 16; i += NT) {
      const int ch = i >> 4, m = i & 15;
      float acc = 0.f;  // sum over poles in order (triton_hcl.py:77-85)
      for (int q = 0; q < 16; ++q) acc = fmaf(R[ch * 16 + q], E[(ch * 16 + q) * ETAB + m], acc);
      Hf[i] = acc;
    }
    __syncthreads();
    if (!is_f) {
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int ch = CPW * mw + cc;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          // K index 8 g + x: row 8 (g & 1) + x of the chunk, high part for g < 2
          const int j = 8 * (g & 1) + x;
          const float vt = j <= l16 ? Hf[ch * 16 + l16 - j] : 0.f;
          const float vb = E[(ch * 16 + l16) * ETAB + 15 - j];  // A row = pole l16
          AT[cc][x] = g < 2 ? bf_hi(vt) : bf_lo(vt);
          AB[cc][x] = g < 2 ? bf_hi(vb) : bf_lo(vb);
          // readout: K index 8 g + x pairs pole 4 g + x / 2 with the state's
          // high (x even) or low (x odd) part
          const int q = 4 * g + (x >> 1);
          const float vc = R[ch * 16 + q] * E[(ch * 16 + q) * ETAB + l16 + 1];
          AC[cc][x] = bf_hi(vc);
          AC2[cc][x] = bf_lo(vc);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int q = 4 * g + k;
          P16[cc][k] = E[(ch * 16 + q) * ETAB + 16];
          carry[cc][k] = init ? p.ssm[blk * p.m0 + (int64_t)(c0 + ch) * p.m1 + q * p.m2] : 0.f;
        }
      }
    }
  }

  // ---- featurizer: sub-tile i from its slot -> u, x2
  auto featurize = [&](auto s, int i) __attribute__((always_inline)) {
    const bf16_t *zs = slot_ptr(s);
    const int s0 = a + RS * i;
    const int r0 = 16 * fprg;
    auto zrow = [&](int lr) __attribute__((always_inline)) -> const bf16_t * { return zs + (lr + 2) * ZW; };
    uint32_t upk[8], xq[8];
    if (s0 + r0 + 16 <= e) {  // interior rows: pairs through v_dot2
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const int sb = r0 - 2 + 8 * g2;
        const bf16_t *rp[10];
#pragma unroll
        for (int k = 0; k < 10; ++k) rp[k] = zrow(sb + k);
        uint32_t P[9][3];
#pragma unroll
        for (int k = 0; k < 9; ++k)
#pragma unroll
          for (int j = 0; j < 3; ++j) P[k][j] = pair_bf(rp[k][3 * fpc + j], rp[k + 1][3 * fpc + j]);
#pragma unroll
        for (int r = 0; r < 8; r += 2) {
          float y0[3], y1[3];
          short_rows2(P[r], P[r + 1], P[r + 2], wsp, y0, y1);
          upk[4 * g2 + r / 2] = pack_bf(y0[1] * y0[2], y1[1] * y1[2]);
          xq[4 * g2 + r / 2] = pack_bf(y0[0], y1[0]);
        }
      }
    } else {  // rows reaching the segment end, one at a time; u = 0 past it
#pragma unroll
      for (int q = 0; q < 8; ++q) upk[q] = xq[q] = 0u;
#pragma unroll 1
      for (int r = 0; r < 16; ++r) {
        const int lr = r0 + r;
        if (s0 + lr >= e) break;
        const bf16_t *m2 = zrow(lr - 2), *m1 = zrow(lr - 1), *m0 = zrow(lr);
        float y3[3];
        for (int j = 0; j < 3; ++j)
          y3[j] = short_dot_rbf(pair_bf(m2[3 * fpc + j], m1[3 * fpc + j]),
                                pair_bf(m1[3 * fpc + j], m0[3 * fpc + j]), wsp[j]);
        const uint32_t ub = f2bf(rbf(y3[1] * y3[2])), xb = f2bf(y3[0]);
        const int sh = 16 * (r & 1);
        for (int q = 0; q < 8; ++q) {
          if (q == r / 2) {
            upk[q] |= ub << sh;
            xq[q] |= xb << sh;
          }
        }
      }
    }
    bf16_t *ud;
    if constexpr (HCL) ud = ubuf + (i & 1) * CH * UP + fpc * UP + r0;
    else ud = ubuf + fpc * RP + (s0 - a + r0 + HIST) % RING;
    bf16_t *xd = xbuf + (i & 1) * CH * UP + fpc * UP + r0;
    *reinterpret_cast<uint4 *>(ud) = make_uint4(upk[0], upk[1], upk[2], upk[3]);
    *reinterpret_cast<uint4 *>(ud + 8) = make_uint4(upk[4], upk[5], upk[6], upk[7]);
    *reinterpret_cast<uint4 *>(xd) = make_uint4(xq[0], xq[1], xq[2], xq[3]);
    *reinterpret_cast<uint4 *>(xd + 8) = make_uint4(xq[4], xq[5], xq[6], xq[7]);
  };

  // ---- matrix waves: inner filter and epilogue of sub-tile j into gbuf
  auto matrix = [&](int j) __attribute__((always_inline)) {
    const int s0 = a + RS * j;
    const int jb = j & 1;
    uint32_t gq[CPW][2];
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int ch = CPW * mw + cc;
      sf32x4_t Y;
      const bf16_t *up;  // u rows 16 n + 4 g .. + 3 of this channel (the epilogue's D term)
      if constexpr (HCL) {
        const bf16_t *uc = ubuf + jb * CH * UP + ch * UP;
        up = uc + 16 * l16 + 4 * g;
        const sbf16x8_t Bu = *reinterpret_cast<const sbf16x8_t *>(uc + 16 * l16 + 8 * (g & 1));
        Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AT[cc], Bu, sf32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        sf32x4_t X = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AB[cc], Bu, sf32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        // the state entering the sub-tile joins chunk 0's end state, then an
        // inclusive scan over the 16 chunks of each pole, X(n) += p^(16 d) X(n - d),
        // leaves the state at the end of every chunk
        float x[4], m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          m[k] = P16[cc][k];
          x[k] = fmaf(l16 == 0 ? m[k] : 0.f, carry[cc][k], X[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(m[k], row_shr<1>(x[k]), x[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] *= m[k];
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(m[k], row_shr<2>(x[k]), x[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] *= m[k];
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(m[k], row_shr<4>(x[k]), x[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] *= m[k];
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(m[k], row_shr<8>(x[k]), x[k]);
        // the state before chunk n (chunk 0: the entering state), and the
        // state leaving the sub-tile
        float sp[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sp[k] = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(carry[cc][k]), __float_as_int(x[k]),
                                                             0x111, 0xf, 0xf, false));
          carry[cc][k] = __shfl(x[k], (lane & 48) | 15);
        }
        if (j == nsub - 1 && l16 == ((e - s0 - 1) >> 4)) {
          // the state before the segment's last chunk, for the tail below
#pragma unroll
          for (int k = 0; k < 4; ++k) sfin[ch * 16 + 4 * g + k] = sp[k];
        }
        // B operand: K index 8 g + 2 k + h = (pole 4 g + k, high / low part)
        sbf16x8_t Bs;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          Bs[2 * k] = bf_hi(sp[k]);
          Bs[2 * k + 1] = bf_lo(sp[k]);
        }
        Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AC[cc], Bs, Y, 0, 0, 0);
        Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AC2[cc], Bs, Y, 0, 0, 0);
      } else {
        const bf16_t *rc = ubuf + ch * RP;
        // ring slot of row s0 - 144 (wave-uniform) plus the lane's offset,
        // wrapped once (offsets stay below 2 RING)
        const int base = __builtin_amdgcn_readfirstlane((s0 - a) % RING);
        auto wrap = [](int x) { return x >= RING ? x - RING : x; };
        up = rc + wrap(base + 16 * l16 + 4 * g + HIST);
        const int bpos = base + 16 * l16 + 8 * g;
        Y = sf32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const sbf16x8_t B = *reinterpret_cast<const sbf16x8_t *>(rc + wrap(bpos + 32 * s));
          Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[cc][s], B, Y, 0, 0, 0);
        }
      }
      // epilogue of rows 16 n + 4 g + k: bf16(y) [+ bf16(u D)], times x2
      const uint2 x4 = *reinterpret_cast<const uint2 *>(xbuf + jb * CH * UP + ch * UP + 16 * l16 + 4 * g);
      const float xx[4] = {lo_bf(x4.x), hi_bf(x4.x), lo_bf(x4.y), hi_bf(x4.y)};
      float gv[4];
      if constexpr (HAS_D) {
        const uint2 u4 = *reinterpret_cast<const uint2 *>(up);
        const float uu[4] = {lo_bf(u4.x), hi_bf(u4.x), lo_bf(u4.y), hi_bf(u4.y)};
#pragma unroll
        for (int k = 0; k < 4; ++k) gv[k] = xx[k] * rbf(rbf(Y[k]) + rbf(dv[cc] * uu[k]));
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) gv[k] = xx[k] * rbf(Y[k]);
      }
      gq[cc][0] = pack_bf(gv[0], gv[1]);
      gq[cc][1] = pack_bf(gv[2], gv[3]);
    }
    // gbuf row pr = 16 i + n holds sub-tile row 16 n + i (so the 16 lanes of
    // one output row index fall on distinct banks); this wave's four
    // channels are one 8-byte piece of it
    bf16_t *gb = gbuf + jb * RS * CH;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t b[CPW];
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) b[cc] = (gq[cc][k >> 1] >> (16 * (k & 1))) & 0xffffu;
      const int pr = 16 * (4 * g + k) + l16;
      *reinterpret_cast<uint2 *>(gb + pr * CH + CPW * mw) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
    }
  };

  // ---- matrix waves: sub-tile j's rows out of gbuf as 16-byte pieces
  // through a buffer descriptor ending at the segment's last row
  const __amdgpu_buffer_rsrc_t ores = __builtin_amdgcn_make_buffer_rsrc(
      p.out + (int64_t)a * p.so + c0, 0, static_cast<int>((int64_t)(e - a) * p.so * 2), 0x00020000);
  auto store = [&](int j) __attribute__((always_inline)) {
    const int s0 = a + RS * j;
    const bf16_t *gb = gbuf + (j & 1) * RS * CH;
    const int mt = tid - 64 * NF;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int q = mt + 256 * k, pr = q >> 1, half = q & 1;
      const uint4 v = *reinterpret_cast<const uint4 *>(gb + pr * CH + 8 * half);
      const int r = 16 * (pr & 15) + (pr >> 4);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(si32x4_t, v), ores,
                                             ((s0 - a + r) * static_cast<int>(p.so) + 8 * half) * 2, 0, 0);
    }
  };

  // ---- the sweep, one barrier per step: step i featurizes sub-tile i, runs
  // the matrix part of sub-tile i - 1 and stores sub-tile i - 2.  The two
  // roles run separate loops with the same barrier count, so the matrix
  // waves' per-channel constants are not live in the featurizer's code.
  // Before the barrier each featurizer wave waits for its own loads of
  // sub-tile i (those of i + 1 .. i + NS - 2 stay in flight); after it, slot
  // (i + NS - 1) % NS, last read for sub-tile i - 1, takes sub-tile i + NS - 1.
  if (is_f) {
    auto wait_slot = [&](int ahead) __attribute__((always_inline)) {
      // ahead = sub-tiles issued after sub-tile i (0 .. NS - 2)
      if (ahead <= 0) vmcnt_wait<0>();
      else if (ahead == 1) {
        if (wave == 0) vmcnt_wait<zloads(0)>();
        else vmcnt_wait<zloads(1)>();
      } else {
        if (wave == 0) vmcnt_wait<2 * zloads(0)>();
        else vmcnt_wait<2 * zloads(1)>();
      }
    };
    auto step = [&](auto s, int i) __attribute__((always_inline)) {
      constexpr int S = decltype(s)::value;
      if (i < nsub) wait_slot(min(NS - 2, nsub - 1 - i));
      sweep_barrier();
      if (i + NS - 1 < nsub) prefetch(std::integral_constant<int, (S + NS - 1) % NS>{}, i + NS - 1);
      if (i < nsub) featurize(s, i);
    };
    for (int i = 0; i <= nsub + 1; i += NS) {
      step(std::integral_constant<int, 0>{}, i);
      if (i + 1 <= nsub + 1) step(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 <= nsub + 1) step(std::integral_constant<int, 2>{}, i + 2);
      if constexpr (NS > 3) {
        if (i + 3 <= nsub + 1) step(std::integral_constant<int, 3 % NS>{}, i + 3);
      }
    }
  } else {
    for (int i = 0; i <= nsub + 1; ++i) {
      sweep_barrier();
      if (i >= 1 && i <= nsub) matrix(i - 1);
      if (i >= 2) store(i - 2);
    }
    if constexpr (HCL) {
      // the segment's last state: the recurrence over the rows of its last
      // chunk from the state before it, one (channel, pole) a thread; the
      // thread's channel is one of its own wave's, so the wave's sfin writes
      // precede these reads
      const int mt = tid - 64 * NF, ch = mt >> 4, q = mt & 15;
      const int s0 = a + RS * (nsub - 1);
      const int cf = (e - s0 - 1) >> 4, nr = e - s0 - 16 * cf;
      if (blk_ok) {
        const bf16_t *uc = ubuf + ((nsub - 1) & 1) * CH * UP + ch * UP + 16 * cf;
        const float pl = expf(p.lp[(int64_t)(c0 + ch) * p.l0 + q * p.l1]);
        float sf = sfin[ch * 16 + q];
        for (int r = 0; r < nr; ++r) sf = fmaf(pl, sf, bf2f(uc[r]));
        p.ssm[blk * p.m0 + (int64_t)(c0 + ch) * p.m1 + q * p.m2] = sf;
      }
    }
  }
}

bool stripe_supported(const StripeArgs &a, int64_t T, int64_t block_t) {
  using namespace stripe;
  if (block_t < T || a.H % CH) return false;
  if (a.sz % 8 || a.so % 8 || reinterpret_cast<uintptr_t>(a.z) % 16 ||
      reinterpret_cast<uintptr_t>(a.out) % 16)
    return false;
  if (a.sz * (RS + 16) * 2 >= (int64_t(1) << 31) || T * a.so * 2 >= (int64_t(1) << 31)) return false;
  if (cdiv(a.nseq * cdiv(a.H, 64), 8) * 32 > 0x7fffffff) return false;
  return true;
}

int launch_stripe(const StripeArgs &a, StripeKind kind, hipStream_t st) {
  using namespace stripe;
  const int nblk64 = static_cast<int>(cdiv(a.H, 64));
  const int64_t units = a.nseq * nblk64;
  if (units == 0) return EVO2_OK;
  const unsigned nwg = static_cast<unsigned>(cdiv(units, 8) * 32);
  if (kind == STRIPE_HCL)
    hipLaunchKernelGGL((stripe_kernel<STRIPE_HCL, true, NSLOT>), dim3(nwg), dim3(NT), 0, st, a, units, nblk64);
  else if (a.D)
    hipLaunchKernelGGL((stripe_kernel<STRIPE_HCM, true, NSLOT>), dim3(nwg), dim3(NT), 0, st, a, units, nblk64);
  else
    hipLaunchKernelGGL((stripe_kernel<STRIPE_HCM, false, NSLOT>), dim3(nwg), dim3(NT), 0, st, a, units, nblk64);
  return check_launch(kind == STRIPE_HCL ? "hcl stripe prefill" : "hcm stripe prefill");
}

}  // namespace evo2
