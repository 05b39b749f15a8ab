// Single-pass prefill of the hcm (128-tap FIR) and hcl (16-pole modal LI)
// mixer cores for gfx950, z (T, 3H) -> g (T, H):
//   short K=3 filter -> u = x1 v -> inner filter y -> g = x2 bf16(bf16(y) [+ bf16(u D)])
// (mixers.py:1277-1305 for hcm, 1327-1401 for hcl; the rounding points are
// the fused VALU kernels' and the reference's).
//
// Work split.  A workgroup owns CH channels and sweeps rows in steps:
//  * hcl: CH = 16, one whole segment per workgroup, steps of 256 rows.  The
//    LI state crosses steps inside the workgroup, so z is read once and there
//    is no carry pass (the tiled LI form reads z twice).  Splitting a segment
//    over workgroups would need a carry, so a single long segment has only
//    H / 16 workgroups and the 16-channel width.
//  * hcm: CH = 32, one tile of the tile table per workgroup, steps of 128
//    rows.  A tile after its segment's first starts its sweep 256 rows
//    early to rebuild the FIR history (the 128-tap window reaches 127 rows
//    back); the first tile starts from the cached window.
// The workgroups of one 64-channel block (four at CH = 16, two at CH = 32)
// are workgroups b, b + 8, ...: one XCD, dispatched together, so the
// 384-byte row slice of the block is fetched once into that XCD's L2.  The
// width matters for bandwidth: a workgroup's z row slice is 96 bytes at
// CH = 16, split over two 128-byte lines, and the load rate per CU follows
// the useful bytes per line request.  A load-and-store probe of this sweep
// on one MI355X moves 2.3 TB/s at 16 channels, 4.4 at 32 and 5.0 at 64;
// 64 channels do not fit the FIR's ring, x2 and output staging in LDS.
//
// Waves.  Featurizer waves 0-3 and CH / 4 matrix waves, one barrier per step:
//   featurizer: direct-to-LDS z loads two steps ahead into a three-slot ring;
//     thread (channel tid % CH, rows 16 (tid / CH) .. +15 of the step) runs
//     the short filter and the gate and writes u and x2 into channel-major
//     rings;
//   matrix: four channels a wave, the inner filter of each completed
//     256-row batch on the matrix cores, the epilogue into a row-major LDS
//     buffer, and the stores of that buffer one step later.
//
// The inner filter on v_mfma_f32_16x16x32_bf16.  Rows of a batch form 16
// chunks of 16; chunk n is column n of the B operand and output row i of
// chunk n is row 16 n + i.
//  * hcm: y[16n + i] = sum_j A[i][j] W_n[j] with the 160-row window
//    W_n[j] = u[16n - 144 + j] and A[i][j] = w[j - i - 17] (zero outside
//    0..127): five k-steps over the u ring, which keeps 144 rows of history.
//    Taps and u are bf16, so every product is exact; only the fp32
//    summation order differs from a per-tap loop.
//  * hcl: with p = exp(lp) per pole, h[m] = sum_s r_s p_s^m and the state
//    S_s(t) = p_s S_s(t-1) + u(t), per chunk n
//      y[16n + i] = sum_{j<=i} h[i-j] u[16n+j]          (intra-chunk Toeplitz)
//                 + sum_s r_s p_s^(i+1) S_s(16n - 1)      (state before the chunk)
//      X_s(n)     = sum_j p_s^(15-j) u[16n + j]           (chunk end state from 0)
//    X comes from one MFMA, the states before each chunk from a 16-lane scan
//    of X over the chunks (DPP row shifts, multipliers p^16, p^32, p^64,
//    p^128) with the state entering the batch folded into chunk 0, and the
//    readout from two more MFMAs.  The fp32 coefficients (h, p^k, r p^k) and
//    the states are split into bf16 high and low parts, so the products keep
//    ~16 mantissa bits: the result agrees with the fp32 recurrence to
//    ~1e-5 relative, far inside the bf16 output rounding.
#include <type_traits>

#include "featurize.h"
#include "stripe.h"

namespace evo2 {

// Geometry of the sweep for a channel width.
template <int CH_>
struct StripeGeo {
  static constexpr int CH = CH_;                 // channels per workgroup
  static constexpr int BATCH = 256;              // rows per MFMA batch: 16 chunks of 16
  static constexpr int STEP = CH == 16 ? 256 : 128;  // rows per step
  static constexpr int SPB = BATCH / STEP;       // steps per batch
  static constexpr int NF = 4;                   // featurizer waves
  static constexpr int NM = CH / 4;              // matrix waves (four channels each)
  static constexpr int NT = 64 * (NF + NM);
  static constexpr int FRG = STEP / 16;          // featurizer row groups per step
  static_assert(CH * FRG == 64 * NF, "one featurizer thread per (channel, 16-row group)");
  static constexpr int ZW = 3 * CH;              // bf16 per staged z row (x2, x1, v triples)
  static constexpr int ZROWS = STEP + 2;         // staged rows: the step and the short filter's halo
  static constexpr int ZCH = ZROWS * ZW / 8;     // 16-byte chunks of a slot's rows
  static constexpr int ZCPR = ZW / 8;            // chunks per staged row
  static constexpr int ZINS = (ZCH + 63) / 64;   // wave loads per slot: wave w issues w, w + NF, ...
  static constexpr int SLOT = ZINS * 512;        // bf16 per slot (spare lanes land past the rows)
  // loads per slot of featurizer wave w; the sweep's waits assume waves
  // 1..NF-1 issue the same number, and the prefetch loop bound covers all
  static constexpr int zloads(int w) { return (ZINS - w + NF - 1) / NF; }
  static_assert(zloads(1) == zloads(NF - 1) && NF * (NF + 3) >= ZINS, "featurizer wave load counts");
  static constexpr int HIST = 144;               // hcm: history rows a batch's windows reach
  // u ring rows: hcl keeps two batches; hcm the history, a batch being read
  // and the step being written meanwhile, rounded up to a multiple of 128
  // rows: a wrap then moves a read by whole 256-byte bank rows, which keeps
  // the matrix waves' 16-byte reads on distinct banks
  static constexpr int UR = CH == 16 ? 2 * BATCH : (HIST + BATCH + STEP + 127) / 128 * 128;
  static constexpr int UP = UR + 8;              // u ring pitch (bf16)
  static constexpr int XR = BATCH + STEP;        // x2 ring rows: a batch and the step after it
  static constexpr int XP = XR + 8;              // x2 ring pitch (bf16)
  // row pitches an odd multiple of 4 banks: the 16 channels of a b128 access
  // fall on distinct bank groups
  static_assert((UP / 2) % 8 == 4 && (XP / 2) % 8 == 4, "ring pitches spread channels over the banks");
  static_assert(UR % 16 == 0 && XR % 16 == 0, "16-row groups never wrap");
  static constexpr int NGB = SPB == 1 ? 2 : 1;   // output buffers (stores run one step after the epilogue)
  static constexpr int SIB = 64 / CH;            // workgroups per 64-channel block
  static constexpr int NSLOT = 3;                // z slots: two steps in flight (a
                                                 // fourth measured no faster for hcl)
  static constexpr int KS = 5;                   // hcm: k-steps over the 160-row window
  static constexpr int TAPW = 176;               // hcm: zero-padded taps per channel for the A build
  static constexpr int ETAB = 17;                // hcl: p^m for m = 0..16 per pole
  static_assert(CH * TAPW <= SLOT, "the tap table borrows a staging slot");
  static_assert(CH != 16 || CH * 16 * (ETAB + 2) * 4 <= SLOT * 2, "the LI tables borrow a staging slot");
};

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
// direct-to-LDS load still in flight (the next steps' z rows) as well; here
// each featurizer wave waits for exactly the loads the next step reads
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

template <int KIND, bool HAS_D, int CHW>
__global__ __launch_bounds__(StripeGeo<CHW>::NT, 1) void stripe_kernel(StripeArgs p, int64_t units, int nblk64) {
  using G = StripeGeo<CHW>;
  constexpr int CH = G::CH, STEP = G::STEP, SPB = G::SPB, NF = G::NF, ZW = G::ZW;
  constexpr int UR = G::UR, UP = G::UP, XR = G::XR, XP = G::XP, HIST = G::HIST, KS = G::KS;
  constexpr int TAPW = G::TAPW, ETAB = G::ETAB, SLOT = G::SLOT, ZINS = G::ZINS, ZCPR = G::ZCPR;
  constexpr bool HCL = KIND == STRIPE_HCL;
  static_assert(HCL ? CH == 16 : CH == 32, "hcl sweeps 16 channels, hcm 32");
  __shared__ __align__(16) bf16_t zs0[SLOT];
  __shared__ __align__(16) bf16_t zs1[SLOT];
  __shared__ __align__(16) bf16_t zs2[SLOT];
  __shared__ __align__(16) bf16_t ubuf[CH * UP];
  __shared__ __align__(16) bf16_t xbuf[CH * XP];
  __shared__ __align__(16) bf16_t gbuf[G::NGB * G::BATCH * CH];
  __shared__ float sfin[HCL ? CH * 16 : 1];                  // hcl: state before the last chunk
  // hcl: per channel the scan's multipliers p^16, p^32, p^64, p^128 of the 16
  // poles, [channel][j][pole] for p^(16 2^j)
  __shared__ __align__(16) float pmul[HCL ? CH * 4 * 16 : 1];

  // ---- workgroup -> (tile, CH-channel group)
  const int L = blockIdx.x;
  const int js = L >> 3;
  const int64_t unit = static_cast<int64_t>(js / G::SIB) * 8 + (L & 7);
  if (unit >= units) return;  // uniform
  const int c0 = static_cast<int>(unit % nblk64) * 64 + (js % G::SIB) * CH;
  if (c0 >= p.H) return;  // uniform
  const int tile = static_cast<int>(unit / nblk64);
  int seg, t0;
  if constexpr (HCL) {
    seg = tile;  // whole segments
    t0 = p.seq[3 * seg];
  } else {
    seg = p.tiles[2 * tile];
    t0 = p.tiles[2 * tile + 1];
  }
  const int a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  const int t_end = HCL ? e : min(t0 + p.block_t, e);
  if (t0 >= t_end) return;  // uniform
  const int64_t blk = p.blocks[seg * p.sblk];
  const bool blk_ok = blk >= 0 && blk < p.num_blocks;
  const bool init = p.seq[3 * seg + 2] != 0 && blk_ok;
  // hcm tiles after the first rebuild the history from a batch of z rows
  // before the tile (t0 - a >= 256: block_t >= 256)
  const int sb = (!HCL && t0 > a) ? t0 - G::BATCH : t0;  // first swept row
  const int skip = (t0 - sb) / G::BATCH;                  // batches without outputs (0 or 1)
  const int nstep = (t_end - sb + STEP - 1) / STEP;
  const int nbatch = (t_end - sb + G::BATCH - 1) / G::BATCH;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool is_f = wave < NF;
  // featurizer role: channel fpc, rows 16 fprg .. 16 fprg + 15 of a step
  const int fpc = tid % CH;
  const int fprg = (tid / CH) % G::FRG;
  // matrix role: wave mw (channels 4 mw .. 4 mw + 3), lane (l16 = lane % 16, g = lane / 16)
  const int mw = wave - NF;
  const int l16 = lane & 15, g = lane >> 4;

  auto slot_ptr = [&](auto s) __attribute__((always_inline)) -> bf16_t * {
    constexpr int S = decltype(s)::value;
    return S == 0 ? zs0 : (S == 1 ? zs1 : zs2);
  };

  // ---- z rows r0 - 2 .. r0 + STEP - 1 of step i (r0 = sb + STEP i) into slot
  // rows 0 .. STEP + 1 by direct-to-LDS loads: chunk q = 64 (wave + NF j) +
  // lane is 16 bytes of slot row q / ZCPR.  Rows past the tile end (and the
  // spare lanes of the last load) load the tile's last row again, never
  // read; rows before the segment start (step 0 of a first tile) are not
  // loaded: they come from the conv window.
  auto prefetch = [&](auto s, int i) __attribute__((always_inline)) {
    bf16_t *dst = slot_ptr(s);
    const int r0 = sb + STEP * i - 2;
    const char *base = reinterpret_cast<const char *>(p.z + (int64_t)r0 * p.sz + 3 * c0);
    const int last = t_end - 1 - r0;
    const int first = a - r0;  // slot rows below this precede the segment
#pragma unroll
    for (int j = 0; j < NF + 3; ++j) {
      const int cw = wave + NF * j;
      if (cw < ZINS) {  // uniform
        const int q = 64 * cw + lane;
        const int row = q / ZCPR;
        const int col = q - ZCPR * row;
        const uint32_t off = 2u * static_cast<uint32_t>(min(row, last) * static_cast<int>(p.sz) + 8 * col);
        if (row >= first)
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(base + off),
                                           (__attribute__((address_space(3))) void *)(dst + 512 * cw),
                                           16, 0, 0);
      }
    }
  };
  // the short filter's left context of step 0 when the sweep starts at the
  // segment start: slot rows 0, 1 = rows a - 2, a - 1 from the conv window
  // (column 0 = a - 2) when continuing, else zero; written before any load
  // targets the slot
  if (sb == a && tid < 2 * ZW) {
    const int q = tid / ZW, k = tid - ZW * q;
    bf16_t v = 0;
    if (init) v = p.cs[blk * p.cs0 + (int64_t)(3 * c0 + k) * p.cs1 + q * p.cs2];
    zs0[tid] = v;
  }
  if (is_f) {
    prefetch(std::integral_constant<int, 0>{}, 0);
    if (nstep > 1) prefetch(std::integral_constant<int, 1>{}, 1);
  }

  // ---- per-role constants
  ShortTaps wsp[3];
  if (is_f) {
#pragma unroll
    for (int i = 0; i < 3; ++i) wsp[i] = short_taps(p.ws, 3 * (int64_t)(c0 + fpc) + i);
  }
  float dv[4];
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) dv[cc] = 0.f;
  if constexpr (HAS_D) {
    if (!is_f) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) dv[cc] = bf2f(p.D[c0 + 4 * mw + cc]);
    }
  }

  // hcm: A fragments (lane (i, kg), k-step s, element x holds
  // A[i][32 s + 8 kg + x] = w[32 s + 8 kg + x - i - 17]) and the ring's
  // history rows a - 144 .. a - 1 of a first tile (the old window's columns,
  // col 0 = a - 127)
  sbf16x8_t A[HCL ? 1 : 4][HCL ? 1 : KS];
  // hcl: per channel the A fragments of the intra-chunk Toeplitz (AT), the
  // chunk end states (AB) and the readout (AC high, AC2 low parts), and per
  // lane (column n = l16, poles 4 g .. 4 g + 3): p^16 and the state entering
  // the batch
  sbf16x8_t AT[HCL ? 4 : 1], AB[HCL ? 4 : 1], AC[HCL ? 4 : 1], AC2[HCL ? 4 : 1];
  float P16[HCL ? 4 : 1][4], carry[HCL ? 4 : 1][4];
  if constexpr (!HCL) {
    bf16_t *tp = zs2;
    for (int i = tid; i < CH * TAPW; i += G::NT) {
      const int ch = i / TAPW, k = i - ch * TAPW - 32;
      bf16_t v = 0;
      if (k >= 0 && k < 128) v = p.w[(int64_t)(c0 + ch) * p.w0 + k];
      tp[i] = v;
    }
    for (int i = tid; i < CH * HIST; i += G::NT) {
      const int ch = i / HIST, r = i - HIST * ch;  // ring slot r holds row sb - 144 + r
      const int col = r - (HIST - 127);
      float u = 0.f;
      if (sb == a && init && col >= 0)
        u = p.st[blk * p.st0 + (int64_t)(c0 + ch) * p.st1 + (int64_t)col * p.st2];
      ubuf[ch * UP + r] = f2bf(u);
    }
    __syncthreads();
    if (!is_f) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int x = 0; x < 8; ++x)
            A[cc][s][x] = __builtin_bit_cast(__bf16, tp[(4 * mw + cc) * TAPW + 32 * s + 8 * g + x - l16 + 15]);
    }
  } else {
    float *E = reinterpret_cast<float *>(zs2);  // [CH][16 poles][ETAB]: p^m
    float *R = E + CH * 16 * ETAB;              // [CH][16]: residues
    float *Hf = R + CH * 16;                    // [CH][16]: h[m], m < 16
    for (int i = tid; i < CH * 16 * ETAB; i += G::NT) {
      const int ch = i / (16 * ETAB), rem = i - ch * 16 * ETAB, q = rem / ETAB, m = rem - q * ETAB;
      E[i] = expf(p.lp[(int64_t)(c0 + ch) * p.l0 + q * p.l1] * static_cast<float>(m));
    }
    for (int i = tid; i < CH * 16; i += G::NT) R[i] = p.res[(int64_t)(c0 + (i >> 4)) * p.r0 + (i & 15) * p.r1];
    __syncthreads();
    for (int i = tid; i < CH * 16; i += G::NT) {
      const int ch = i >> 4, m = i & 15;
      float acc = 0.f;  // sum over poles in order (triton_hcl.py:77-85)
      for (int q = 0; q < 16; ++q) acc = fmaf(R[ch * 16 + q], E[(ch * 16 + q) * ETAB + m], acc);
      Hf[i] = acc;
      // pole m's scan multipliers, squared in the order the scan applies them
      float pm = E[(ch * 16 + m) * ETAB + 16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pmul[(ch * 4 + j) * 16 + m] = pm;
        pm *= pm;
      }
    }
    __syncthreads();
    if (!is_f) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int ch = 4 * mw + cc;
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

  // ring positions: u row t at (t - sb [+ HIST]) mod UR, x2 row t at (t - sb) mod XR
  auto wrap_u = [](int x) __attribute__((always_inline)) { return x >= UR ? x - UR : x; };
  auto wrap_x = [](int x) __attribute__((always_inline)) { return x >= XR ? x - XR : x; };

  // ---- featurizer: step i from its slot -> u, x2
  auto featurize = [&](auto s, int i) __attribute__((always_inline)) {
    const bf16_t *zs = slot_ptr(s);
    const int r0 = 16 * fprg;       // first row of this thread in the step
    const int t = sb + STEP * i + r0;  // its absolute row
    auto zrow = [&](int lr) __attribute__((always_inline)) -> const bf16_t * { return zs + (lr + 2) * ZW; };
    uint32_t upk[8], xq[8];
    if (t + 16 <= t_end) {  // interior rows: pairs through v_dot2
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const int lb = r0 - 2 + 8 * g2;
        const bf16_t *rp[10];
#pragma unroll
        for (int k = 0; k < 10; ++k) rp[k] = zrow(lb + k);
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
    } else {  // rows reaching the tile end, one at a time; u = 0 past it
#pragma unroll
      for (int q = 0; q < 8; ++q) upk[q] = xq[q] = 0u;
#pragma unroll 1
      for (int r = 0; r < 16; ++r) {
        const int lr = r0 + r;
        if (t + r >= t_end) break;
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
    const int off = t - sb;  // < 2^31 / 2: positions by modulo, 16-row aligned
    bf16_t *ud = ubuf + fpc * UP + (HCL ? off % UR : (off + HIST) % UR);
    bf16_t *xd = xbuf + fpc * XP + off % XR;
    *reinterpret_cast<uint4 *>(ud) = make_uint4(upk[0], upk[1], upk[2], upk[3]);
    *reinterpret_cast<uint4 *>(ud + 8) = make_uint4(upk[4], upk[5], upk[6], upk[7]);
    *reinterpret_cast<uint4 *>(xd) = make_uint4(xq[0], xq[1], xq[2], xq[3]);
    *reinterpret_cast<uint4 *>(xd + 8) = make_uint4(xq[4], xq[5], xq[6], xq[7]);
  };

  // ---- matrix waves: inner filter and epilogue of batch m into gbuf.  gbuf
  // row pr = 16 i + n holds batch row 16 n + i; this wave's four channels
  // are 8-byte piece mw of it, placed at piece mw ^ (n >> SH) ^ NPC / 2 [i / 4
  // odd] so that the 32 lanes of one write (n < 16, i = 4 g + k for g = 0, 1:
  // rows 64 apart) fall on distinct banks
  constexpr int NPC = CH / 4;              // 8-byte pieces per gbuf row
  constexpr int SH = CH == 16 ? 3 : 2;     // n >> SH takes NPC / 2 ... values
  auto matrix = [&](int m) __attribute__((always_inline)) {
    const int ub0 = __builtin_amdgcn_readfirstlane((G::BATCH * m) % UR);  // ring slot of the batch's first row (no HIST)
    const int xb0 = __builtin_amdgcn_readfirstlane((G::BATCH * m) % XR);
    uint32_t gq[4][2];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int ch = 4 * mw + cc;
      const bf16_t *uc = ubuf + ch * UP;
      sf32x4_t Y;
      const bf16_t *up;  // u rows 16 n + 4 g .. + 3 of this channel (the epilogue's D term)
      if constexpr (HCL) {
        up = uc + ub0 + 16 * l16 + 4 * g;
        const sbf16x8_t Bu = *reinterpret_cast<const sbf16x8_t *>(uc + ub0 + 16 * l16 + 8 * (g & 1));
        Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AT[cc], Bu, sf32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        sf32x4_t X = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AB[cc], Bu, sf32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        // the state entering the batch joins chunk 0's end state, then an
        // inclusive scan over the 16 chunks of each pole, X(n) += p^(16 d) X(n - d),
        // leaves the state at the end of every chunk
        float x[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(l16 == 0 ? P16[cc][k] : 0.f, carry[cc][k], X[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(P16[cc][k], row_shr<1>(x[k]), x[k]);
        // p^32, p^64, p^128 of this lane's poles 4 g .. 4 g + 3 from the table
        const float *pmc = pmul + (4 * mw + cc) * 64 + 4 * g;
        const float4 m2 = *reinterpret_cast<const float4 *>(pmc + 16);
        const float4 m4 = *reinterpret_cast<const float4 *>(pmc + 32);
        const float4 m8 = *reinterpret_cast<const float4 *>(pmc + 48);
        const float mm2[4] = {m2.x, m2.y, m2.z, m2.w}, mm4[4] = {m4.x, m4.y, m4.z, m4.w};
        const float mm8[4] = {m8.x, m8.y, m8.z, m8.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(mm2[k], row_shr<2>(x[k]), x[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(mm4[k], row_shr<4>(x[k]), x[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fmaf(mm8[k], row_shr<8>(x[k]), x[k]);
        // the state before chunk n (chunk 0: the entering state), and the
        // state leaving the batch
        float sp[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sp[k] = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(carry[cc][k]), __float_as_int(x[k]),
                                                             0x111, 0xf, 0xf, false));
          carry[cc][k] = __shfl(x[k], (lane & 48) | 15);
        }
        if (m == nbatch - 1 && l16 == ((t_end - sb - G::BATCH * m - 1) >> 4)) {
          // the state before the segment's last chunk, for the tail below
#pragma unroll
          for (int k = 0; k < 4; ++k) sfin[ch * 16 + 4 * g + k] = sp[k];
        }
        // B operand: K index 8 g + 2 k + h = (pole 4 g + k, high / low part)
        // (hi = bf16(s) is exact in fp32, so packing (hi, s - hi) rounds only the
        // low part: the bits of bf_hi and bf_lo)
        si32x4_t bsw;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float hi = rbf_valu(sp[k]);  // sp: a DPP move, an ordinary VALU result
          bsw[k] = static_cast<int>(pack_bf(hi, sp[k] - hi));
        }
        const sbf16x8_t Bs = __builtin_bit_cast(sbf16x8_t, bsw);
        Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AC[cc], Bs, Y, 0, 0, 0);
        Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AC2[cc], Bs, Y, 0, 0, 0);
      } else {
        // window of chunk n at k-step s: rows 16 n - 144 + 32 s + 8 kg ..,
        // ring slots ub0 + 16 n + 8 kg + 32 s (HIST cancels), wrapped once
        up = uc + wrap_u(ub0 + 16 * l16 + 4 * g + HIST);
        const int bpos = ub0 + 16 * l16 + 8 * g;
        Y = sf32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const sbf16x8_t B = *reinterpret_cast<const sbf16x8_t *>(uc + wrap_u(bpos + 32 * s));
          Y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[cc][s], B, Y, 0, 0, 0);
        }
      }
      // epilogue of rows 16 n + 4 g + k: bf16(y) [+ bf16(u D)], times x2
      const uint2 x4 = *reinterpret_cast<const uint2 *>(xbuf + ch * XP + wrap_x(xb0 + 16 * l16 + 4 * g));
      const float xx[4] = {lo_bf(x4.x), hi_bf(x4.x), lo_bf(x4.y), hi_bf(x4.y)};
      float gv[4];
      if constexpr (HAS_D) {
        const uint2 u4 = *reinterpret_cast<const uint2 *>(up);
        const float uu[4] = {lo_bf(u4.x), hi_bf(u4.x), lo_bf(u4.y), hi_bf(u4.y)};
#pragma unroll
        for (int k = 0; k < 4; ++k) gv[k] = xx[k] * rbf_valu(rbf(Y[k]) + rbf_valu(dv[cc] * uu[k]));
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) gv[k] = xx[k] * rbf(Y[k]);
      }
      gq[cc][0] = pack_bf(gv[0], gv[1]);
      gq[cc][1] = pack_bf(gv[2], gv[3]);
    }
    bf16_t *gb = gbuf + (G::NGB == 2 ? (m & 1) : 0) * G::BATCH * CH;
    const int piece = mw ^ (l16 >> SH) ^ ((g & 1) * (NPC / 2));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t b[4];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) b[cc] = (gq[cc][k >> 1] >> (16 * (k & 1))) & 0xffffu;
      const int pr = 16 * (4 * g + k) + l16;
      *reinterpret_cast<uint2 *>(gb + pr * CH + 4 * piece) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
    }
  };

  // ---- matrix waves: batch m's rows out of gbuf as 16-byte pieces through
  // a buffer descriptor covering the tile's rows [t0, t_end)
  const __amdgpu_buffer_rsrc_t ores = __builtin_amdgcn_make_buffer_rsrc(
      p.out + (int64_t)t0 * p.so + c0, 0, static_cast<int>((int64_t)(t_end - t0) * p.so * 2), 0x00020000);
  auto store = [&](int m) __attribute__((always_inline)) {
    const bf16_t *gb = gbuf + (G::NGB == 2 ? (m & 1) : 0) * G::BATCH * CH;
    const int mt = tid - 64 * NF;
    constexpr int NCK = G::BATCH * CH / 8;   // 16-byte pieces of the batch
    constexpr int CPR = CH / 8;              // per row
#pragma unroll
    for (int k = 0; k < NCK / (64 * G::NM); ++k) {
      const int q = mt + 64 * G::NM * k, pr = q / CPR, ck = q % CPR;
      const int n = pr & 15;
      // pieces 2 ck, 2 ck + 1 of the row sit at (2 ck) ^ (n >> SH) ^ NPC / 2
      // [(pr >> 6) odd] and its neighbour, swapped when n >> SH is odd
      const int sw = n >> SH;
      const int hi = ((pr >> 6) & 1) * (NPC / 2);
      uint4 v = *reinterpret_cast<const uint4 *>(gb + pr * CH + 4 * ((2 * ck) ^ (sw & ~1) ^ hi));
      if (sw & 1) v = make_uint4(v.z, v.w, v.x, v.y);
      const int r = 16 * n + (pr >> 4);
      const int t = sb + G::BATCH * m + r;  // >= t0 for batches with outputs
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(si32x4_t, v), ores,
                                             ((t - t0) * static_cast<int>(p.so) + 8 * ck) * 2, 0, 0);
    }
  };

  // ---- the sweep, one barrier per step.  Step i featurizes rows of step i;
  // batch m (steps SPB m .. SPB m + SPB - 1) runs its matrix part at step
  // SPB (m + 1) and its stores one step later.  The two roles run separate
  // loops with the same barrier count, so the matrix waves' per-channel
  // constants are not live in the featurizer's code.  Before the barrier each
  // featurizer wave waits for its own loads of step i (those of i + 1 stay in
  // flight); after it, slot (i + 2) % 3, last read at step i - 1, takes
  // step i + 2.
  const int nsteps = SPB * nbatch + 2;
  if (is_f) {
    auto step = [&](auto s, int i) __attribute__((always_inline)) {
      constexpr int S = decltype(s)::value;
      if (i < nstep) {
        if (i + 1 >= nstep) vmcnt_wait<0>();
        else if (wave == 0) vmcnt_wait<G::zloads(0)>();
        else vmcnt_wait<G::zloads(1)>();
      }
      sweep_barrier();
      if (i + 2 < nstep) prefetch(std::integral_constant<int, (S + 2) % 3>{}, i + 2);
      if (i < nstep) featurize(s, i);
    };
    for (int i = 0; i < nsteps; i += 3) {
      step(std::integral_constant<int, 0>{}, i);
      if (i + 1 < nsteps) step(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < nsteps) step(std::integral_constant<int, 2>{}, i + 2);
    }
  } else {
    for (int i = 0; i < nsteps; ++i) {
      sweep_barrier();
      if (i >= SPB && i % SPB == 0) {
        const int m = i / SPB - 1;
        if (m >= skip && m < nbatch) matrix(m);
      }
      if (i > SPB && (i - 1) % SPB == 0) {
        const int m = (i - 1) / SPB - 1;
        if (m >= skip && m < nbatch) store(m);
      }
    }
    if constexpr (HCL) {
      // the segment's last state: the recurrence over the rows of its last
      // chunk from the state before it, one (channel, pole) a thread; the
      // thread's channel is one of its own wave's, so the wave's sfin writes
      // precede these reads
      const int mt = tid - 64 * NF, ch = mt >> 4, q = mt & 15;
      const int rb = G::BATCH * (nbatch - 1);  // last batch's first row, from sb
      const int cf = (t_end - sb - rb - 1) >> 4, nr = t_end - sb - rb - 16 * cf;
      if (blk_ok) {
        const bf16_t *uc = ubuf + ch * UP + rb % UR + 16 * cf;
        const float pl = expf(p.lp[(int64_t)(c0 + ch) * p.l0 + q * p.l1]);
        float sf = sfin[ch * 16 + q];
        for (int r = 0; r < nr; ++r) sf = fmaf(pl, sf, bf2f(uc[r]));
        p.ssm[blk * p.m0 + (int64_t)(c0 + ch) * p.m1 + q * p.m2] = sf;
      }
    }
  }
}

bool stripe_supported(const StripeArgs &a, StripeKind kind, int64_t T, int64_t block_t) {
  const int64_t ch = kind == STRIPE_HCL ? 16 : 32;
  if (a.H % ch) return false;
  if (kind == STRIPE_HCL && block_t < T) return false;  // whole segments
  if (kind == STRIPE_HCM && block_t < StripeGeo<32>::BATCH) return false;  // a tile holds a halo batch
  if (a.sz % 8 || a.so % 8 || reinterpret_cast<uintptr_t>(a.z) % 16 ||
      reinterpret_cast<uintptr_t>(a.out) % 16)
    return false;
  if (a.sz * (StripeGeo<16>::STEP + 16) * 2 >= (int64_t(1) << 31) || T * a.so * 2 >= (int64_t(1) << 31))
    return false;
  const int64_t tiles = kind == STRIPE_HCL ? a.nseq : a.ntiles;
  if (cdiv(tiles * cdiv(a.H, 64), 8) * 8 * (64 / ch) > 0x7fffffff) return false;
  return true;
}

int launch_stripe(const StripeArgs &a, StripeKind kind, hipStream_t st) {
  const int nblk64 = static_cast<int>(cdiv(a.H, 64));
  const int64_t units = (kind == STRIPE_HCL ? a.nseq : a.ntiles) * nblk64;
  if (units == 0) return EVO2_OK;
  if (kind == STRIPE_HCL) {
    using G = StripeGeo<16>;
    const unsigned nwg = static_cast<unsigned>(cdiv(units, 8) * 8 * G::SIB);
    hipLaunchKernelGGL((stripe_kernel<STRIPE_HCL, true, 16>), dim3(nwg), dim3(G::NT), 0, st, a, units, nblk64);
  } else {
    using G = StripeGeo<32>;
    const unsigned nwg = static_cast<unsigned>(cdiv(units, 8) * 8 * G::SIB);
    if (a.D)
      hipLaunchKernelGGL((stripe_kernel<STRIPE_HCM, true, 32>), dim3(nwg), dim3(G::NT), 0, st, a, units, nblk64);
    else
      hipLaunchKernelGGL((stripe_kernel<STRIPE_HCM, false, 32>), dim3(nwg), dim3(G::NT), 0, st, a, units, nblk64);
  }
  return check_launch(kind == STRIPE_HCL ? "hcl stripe prefill" : "hcm stripe prefill");
}

}  // namespace evo2
