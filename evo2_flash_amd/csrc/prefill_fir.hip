// Varlen Hyena FIR prefill for gfx950: hcs (K=7) and hcm (K=128).
//
// The fused hcm core over tiles of 256 rows or more runs on the matrix cores
// (fir128_mfma_kernel, below); everything else uses the VALU kernel here.
// Two forms share the VALU kernel template:
//  * FUSED: the mixer's whole prefill core between in_proj and out_proj:
//    z (T, 3H) -> short K=3 filter -> u = x1*v -> FIR(u) [+ D*u] -> g = x2*y.
//  * U_IN: the reference's `fir_prefill` (triton_prefill.py:462-496): the
//    FIR over given u rows, output bf16(y).
//
// Layout.  A workgroup owns 64 channels (lane = channel) and one tile of
// rows of one segment (tile table [segment, first row], as
// mixers.py:386-415 builds it).  It sweeps the tile in 64-row sub-tiles:
//   produce: each wave turns 16 rows into u and x2 for its 64 channels,
//            writes u into an LDS ring, u[channel][row mod RING], and keeps
//            x2 in registers for its own epilogue; the short filter runs as
//            v_dot2 over (z[t-1], z[t]) row pairs;
//   FIR:     each lane computes the same 16 outputs of its channel from
//            the ring as bf16 pairs with v_dot2c_f32_bf16 (u and the taps are
//            bf16, so every product is exact in fp32).  The ring's pairs start
//            at even rows; outputs whose window starts at an odd row use the
//            taps paired the other way, so no pair is ever re-aligned; the
//            channel's taps stay in VGPRs for the tile.
// For hcm this fits 168 VGPRs and 50 KB of LDS: three workgroups (three
// waves per SIMD) share a CU.
// The ring holds the K-1 rows of history the next sub-tile needs, so each
// z row is read from HBM once per tile plus a (K-1)-row halo per tile.
//
// Left context: rows before the segment start come from the cached windows
// when the segment continues a sequence (has_initial_state), else zero
// (mixers.py:126-141, 350-383).  The windows are rewritten by a second
// launch after every tile has read them (as triton_prefill.py:489-495).
#include <type_traits>

#include "featurize.h"
#include "stripe.h"

namespace evo2 {

struct FirArgs {
  const bf16_t *x; int64_t sx;              // z (FUSED) or u rows
  const bf16_t *ws;                         // (3H, 3) short taps (FUSED)
  const bf16_t *cs; int64_t cs0, cs1, cs2;  // conv window view (FUSED)
  const bf16_t *w; int64_t w0, w1;          // inner taps (H, K)
  float *st; int64_t st0, st1, st2;         // inner window view (blocks, H, >=K-1)
  const bf16_t *D;                          // (H,) or null
  bf16_t *out; int64_t so;
  const int32_t *seq;                       // (n, 3) [start, end, has_init]
  const int32_t *blocks; int64_t sblk;
  const int32_t *tiles;                     // (ntiles, 2) [segment, first row]
  int H;
  int block_t;
  int64_t num_blocks;
};

template <int K>
struct FirGeom {
  static constexpr int KP = (K + 1) & ~1;  // taps padded to even (zero tap first)
  static constexpr int NP = KP / 2;        // tap pairs
  // rows per sub-tile: 64 for hcm; 32 for hcs, whose time goes to memory,
  // not arithmetic (its two z staging buffers keep four workgroups on a CU)
  static constexpr int RS = K > 8 ? 64 : 32;
  static constexpr int NWAVE = 4;          // waves per workgroup
  static constexpr int NT = 64 * NWAVE;    // threads per workgroup
  // hcm: three waves per SIMD (<= 168 VGPRs; 50 KB of LDS lets three
  // workgroups share a CU)
  static constexpr int MIN_WAVES = K > 8 ? 3 : 1;
  static constexpr int RW = RS / NWAVE;    // rows per wave per sub-tile
  static_assert(RW % 8 == 0, "produce and the epilogue work in 8-row groups");
  // u ring rows per channel: exactly the KP + RS rows one sub-tile's FIR
  // reads for hcm (192; every b128 access starts at a multiple of 8 rows, so
  // none wraps), the next power of two for hcs.
  static constexpr int RING = K > 8 ? KP + RS : 64;
  // Row pitches are 36 dwords mod 64 banks, so the 16 lanes a b128 access
  // serves per cycle cover all banks once.
  static constexpr int PITCH = RING + 8;   // bf16 per channel row of the u ring
  static constexpr int ZROWS = RS + 2;     // staged z rows: sub-tile + 2-row short halo
  static constexpr int ZPITCH = 192;       // bf16 per staged z row (3 x 64 sub-channels)
  static_assert(KP + RS <= RING && RING % 8 == 0, "ring too small or misaligned");
  static_assert((PITCH / 2) % 64 == 36, "ring pitch bank pattern");
  // ring slot of a non-negative row offset
  static __device__ __forceinline__ int at(int x) {
    return (RING & (RING - 1)) == 0 ? (x & (RING - 1)) : static_cast<int>(static_cast<unsigned>(x) % RING);
  }
};

struct SegInfo {
  int a, e, t0, t_end;
  int64_t blk;
  bool init;
};

__device__ __forceinline__ SegInfo seg_of_tile(const FirArgs &p) {
  SegInfo s;
  const int seg = p.tiles[2 * blockIdx.x];
  s.t0 = p.tiles[2 * blockIdx.x + 1];
  s.a = p.seq[3 * seg];
  s.e = p.seq[3 * seg + 1];
  s.blk = p.blocks[seg * p.sblk];
  s.init = p.seq[3 * seg + 2] != 0 && s.blk >= 0 && s.blk < p.num_blocks;
  s.t_end = min(s.t0 + p.block_t, s.e);
  return s;
}



template <int K, bool HAS_D, bool FUSED>
__global__ __launch_bounds__(FirGeom<K>::NT, FirGeom<K>::MIN_WAVES) void fir_prefill_kernel(FirArgs p) {
  using G = FirGeom<K>;
  __shared__ __align__(16) bf16_t ring[64][G::PITCH];
  // z staging: two buffers for the fused 7-tap core (the next sub-tile's rows
  // load while this one computes, and the one after is issued as soon as a
  // buffer frees), one otherwise
  constexpr int NB = (FUSED && K <= 8) ? 2 : 1;
  __shared__ __align__(16) bf16_t zbuf[NB][FUSED ? G::ZROWS : 1][G::ZPITCH];
  bf16_t (*zst)[G::ZPITCH] = zbuf[0];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = blockIdx.y * 64;
  const int c = c0 + lane;
  const bool active = c < p.H;
  const int cl = active ? c : p.H - 1;  // clamped channel for loads
  // Output rows go out as channel pairs: even lanes store row r of (c, c+1),
  // odd lanes row r + 1 of (c - 1, c).
  const bool odd = lane & 1;
  const int cpair = c & ~1;
  bf16_t *const obase = p.out + (odd ? p.so : 0) + cpair;
  const SegInfo S = seg_of_tile(p);
  if (S.t0 >= S.t_end) return;  // uniform across the block

  // Taps as bf16 pairs, one zero tap in front when K is odd.  K=128 taps are
  // contiguous rows (the host guarantees it) and load as 16-byte vectors.
  uint32_t W[G::NP];
  if constexpr (K % 8 == 0) {
    const uint4 *wp = reinterpret_cast<const uint4 *>(p.w + (int64_t)cl * p.w0);
#pragma unroll
    for (int q = 0; q < G::NP / 4; ++q) {
      const uint4 v = wp[q];
      W[4 * q] = active ? v.x : 0u;
      W[4 * q + 1] = active ? v.y : 0u;
      W[4 * q + 2] = active ? v.z : 0u;
      W[4 * q + 3] = active ? v.w : 0u;
    }
  } else {
#pragma unroll
    for (int m = 0; m < G::NP; ++m) {
      const int k0 = 2 * m - (G::KP - K), k1 = k0 + 1;
      uint32_t lo = 0, hi = 0;
      if (active) {
        if (k0 >= 0) lo = p.w[(int64_t)c * p.w0 + (int64_t)k0 * p.w1];
        hi = p.w[(int64_t)c * p.w0 + (int64_t)k1 * p.w1];
      }
      W[m] = lo | (hi << 16);
    }
  }
  ShortTaps wsp[3];
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < 3; ++i) wsp[i] = short_taps(p.ws, 3 * (int64_t)cl + i);
  }
  const float *stc = S.init ? p.st + S.blk * p.st0 + (int64_t)cl * p.st1 : nullptr;
  const bool vec_z = FUSED && (c0 + 64 <= p.H) && (p.sx % 8 == 0) &&
                     ((reinterpret_cast<uintptr_t>(p.x) & 15) == 0) &&
                     p.sx * G::ZROWS < (int64_t(1) << 31);  // 32-bit lane offsets

  // ---- stage z rows [rs, rs + ZROWS) of this block's 192 sub-channels into
  // LDS with direct-to-LDS loads: chunk i = row*24 + col (16 bytes), and one
  // wave instruction moves 64 consecutive chunks (1 KB of the unpadded tile),
  // so the data never passes through VGPRs and the next sub-tile's loads fly
  // while the current one computes.  `prefetch` issues them; `fix` (after the
  // loads have landed) fills the rows the loads skip: the short filter's left
  // context (conv window rows a-2, a-1 when continuing, else zeros) and, when
  // z is not 16-byte addressable, every row element by element.  Rows at or
  // past the tile end keep stale (finite) values; only discarded rows read them.
  constexpr int ZCH = G::ZROWS * 24;             // 16-byte chunks per tile
  constexpr int ZW = (ZCH + 63) / 64;            // wave instructions per tile
  // Wave instruction j moves chunks i = (wave + NWAVE j) * 64 + lane, i.e.
  // row i / 24, column i % 24 of the (ZROWS x 192) tile, at element offset
  // (i / 24) * sx + 3 c0 + 8 (i % 24) from the tile's first row.  The offsets
  // are recomputed per sub-tile (a few VALU) rather than held in registers.
  // Interior sub-tiles (no row before the segment or past the tile end) skip
  // the row checks.
  constexpr int NJ = (ZW + G::NWAVE - 1) / G::NWAVE;
  auto prefetch = [&](int rs) {
    if (!vec_z) return;
    // uniform base plus a 32-bit per-lane byte offset (vec_z bounds it)
    const char *base = reinterpret_cast<const char *>(p.x + (int64_t)rs * p.sx + 3 * c0);
    const bool interior = rs >= S.a && rs + G::ZROWS <= S.t_end;  // uniform
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int cw = wave + G::NWAVE * j;  // wave-uniform
      if (cw >= ZW) break;
      const int i = cw * 64 + lane;
      const int row = i / 24;
      bool ok = i < ZCH;
      if (!interior) ok = ok && rs + row >= S.a && rs + row < S.t_end;
      const uint32_t off = 2u * static_cast<uint32_t>(row * static_cast<int>(p.sx) + 8 * (i - 24 * row));
      if (ok)
        __builtin_amdgcn_global_load_lds(
            reinterpret_cast<const uint4 *>(base + off),
            (__attribute__((address_space(3))) void *)(&zst[0][0] + cw * 512), 16, 0, 0);
    }
  };
  auto fix = [&](int rs) {
    const bf16_t *conv = S.init ? p.cs + S.blk * p.cs0 : nullptr;
    if (vec_z && rs >= S.a) return;  // uniform: nothing to patch
#pragma unroll 1
    for (int i = threadIdx.x; i < ZCH; i += G::NT) {
      const int row = i / 24, col = i - 24 * (i / 24);
      const int t = rs + row;
      const bool inside = t >= S.a && t < S.t_end;
      const bool left = t < S.a && t >= S.a - 2;
      if ((vec_z && inside) || !(inside || left)) continue;
#pragma unroll 1
      for (int e = 0; e < 8; ++e) {
        const int ch = 3 * c0 + 8 * col + e;
        bf16_t b = 0;
        if (ch < 3 * p.H) {
          if (inside) b = p.x[(int64_t)t * p.sx + ch];
          else if (conv) b = conv[ch * p.cs1 + (t - S.a + 2) * p.cs2];
        }
        zst[row][8 * col + e] = b;
      }
    }
  };
  auto land = [&]() { __builtin_amdgcn_s_waitcnt(0); };

  // ---- one row of u at a segment or tile boundary, lane = channel, written
  // to the ring; returns x2 (FUSED; zero otherwise).  Rows before the segment
  // start take u from the inner window (continuation) or zero; rows at or
  // past the tile end give zeros.
  auto produce_row = [&](int t, int rs) -> float {
    float u = 0.0f, x2 = 0.0f;
    if (t < S.a) {
      const int col = (K - 1) + (t - S.a);
      if (stc && col >= 0) u = stc[(int64_t)col * p.st2];
    } else if (t < S.t_end) {
      if constexpr (FUSED) {
        float y3[3];
        for (int i = 0; i < 3; ++i)
          y3[i] = short_dot_rbf(pair_bf(zst[t - 2 - rs][3 * lane + i], zst[t - 1 - rs][3 * lane + i]),
                                pair_bf(zst[t - 1 - rs][3 * lane + i], zst[t - rs][3 * lane + i]),
                                wsp[i]);
        x2 = y3[0];
        u = rbf(y3[1] * y3[2]);
      } else {
        u = active ? bf2f(p.x[(int64_t)t * p.sx + cl]) : 0.0f;
      }
    }
    ring[lane][G::at(t - S.t0 + G::KP)] = f2bf(u);
    return x2;
  };

  // ---- u for NR consecutive rows [r0, r0 + NR) of this wave, lane =
  // channel, written to the ring as packed row pairs with b128 stores; x2 of
  // the rows goes to xout[NR / 2] as packed row pairs when xout is given (the
  // wave that produces a row is the wave that finishes it, so x2 never
  // leaves registers).  FUSED reads z from the staged rows (stage row of t
  // is t - rs); U_IN loads u rows.  Groups touching a boundary go row by
  // row, x2 entering a 16-bit shift register so the row loop stays rolled.
  auto produce = [&](int r0, int rs, auto nr_tag, uint32_t *xout) {
    constexpr int NR = decltype(nr_tag)::value;
    static_assert(NR % 8 == 0, "rows are written as 8-row b128 groups");
    if (!(r0 >= S.a && r0 + NR <= S.t_end)) {  // wave-uniform
      uint32_t xf[NR / 2];
#pragma unroll
      for (int i = 0; i < NR / 2; ++i) xf[i] = 0u;
#pragma unroll 1
      for (int r = 0; r < NR; ++r) {
        const float x2 = produce_row(r0 + r, rs);
        if (xout) {
#pragma unroll
          for (int i = 0; i + 1 < NR / 2; ++i) xf[i] = __builtin_amdgcn_alignbit(xf[i + 1], xf[i], 16);
          xf[NR / 2 - 1] = (xf[NR / 2 - 1] >> 16) | (static_cast<uint32_t>(f2bf(x2)) << 16);
        }
      }
      if (xout) {
#pragma unroll
        for (int i = 0; i < NR / 2; ++i) xout[i] = xf[i];
      }
      return;
    }
    uint32_t upk[NR / 2], xpk[NR / 2];
    if constexpr (FUSED) {
      // Eight rows at a time from the row pairs (z[k], z[k+1]) of each
      // sub-channel: staged rows rb + 8g - 2 .. rb + 8g + 8.
      const int rb = r0 - rs;
#pragma unroll
      for (int g = 0; g < NR / 8; ++g) {
        uint32_t P[9][3];
#pragma unroll
        for (int k = 0; k < 9; ++k)
#pragma unroll
          for (int i = 0; i < 3; ++i)
            P[k][i] = pair_bf(zst[rb + 8 * g - 2 + k][3 * lane + i], zst[rb + 8 * g - 1 + k][3 * lane + i]);
#pragma unroll
        for (int r = 0; r < 8; r += 2) {
          float y0[3], y1[3];  // (x2, x1, v) of rows r and r + 1, rounded
          short_rows2(P[r], P[r + 1], P[r + 2], wsp, y0, y1);
          upk[4 * g + r / 2] = pack_bf(y0[1] * y0[2], y1[1] * y1[2]);
          xpk[4 * g + r / 2] = pack_bf(y0[0], y1[0]);
        }
      }
    } else {
      const bf16_t *xp = p.x + (int64_t)r0 * p.sx + cl;
#pragma unroll
      for (int r = 0; r < NR; r += 2) {
        const uint32_t v0 = xp[(int64_t)r * p.sx], v1 = xp[(int64_t)(r + 1) * p.sx];
        upk[r / 2] = active ? (v0 | (v1 << 16)) : 0u;
        xpk[r / 2] = 0;
      }
    }
    const int pos = r0 - S.t0 + G::KP;
#pragma unroll
    for (int g = 0; g < NR / 8; ++g)
      *reinterpret_cast<uint4 *>(&ring[lane][G::at(pos + 8 * g)]) =
          make_uint4(upk[4 * g], upk[4 * g + 1], upk[4 * g + 2], upk[4 * g + 3]);
    if (xout) {
#pragma unroll
      for (int i = 0; i < NR / 2; ++i) xout[i] = xpk[i];
    }
  };
  using RWC = std::integral_constant<int, G::RW>;
  using R8 = std::integral_constant<int, 8>;

  // ---- halo: rows t0-KP .. t0-1
  if constexpr (G::KP == 128) {
#pragma unroll 1
    for (int h = 0; h < G::KP / G::RS; ++h) {
      const int rbase = S.t0 - G::KP + G::RS * h;
      if constexpr (FUSED) {
        __syncthreads();
        prefetch(rbase - 2);
        land();
        fix(rbase - 2);
        __syncthreads();
      }
      produce(rbase + G::RW * wave, rbase - 2, RWC{}, nullptr);
    }
  } else {
    static_assert(G::KP == 8, "halo split assumes KP = 8 or 128");
    const int rbase = S.t0 - G::KP;
    if constexpr (FUSED) {
      prefetch(rbase - 2);
      land();
      fix(rbase - 2);
      __syncthreads();
    }
    if (wave == 0) produce(rbase, rbase - 2, R8{}, nullptr);
  }
  if constexpr (FUSED) {
    __syncthreads();
    prefetch(S.t0 - 2);
    land();
    fix(S.t0 - 2);
    __syncthreads();
    if constexpr (NB == 2) {
      if (S.t0 + G::RS < S.t_end) {
        zst = zbuf[1];
        prefetch(S.t0 + G::RS - 2);
      }
    }
  }

  int bi = 0;
  for (int s0 = S.t0; s0 < S.t_end; s0 += G::RS, bi ^= 1) {
    if constexpr (NB == 2) zst = zbuf[bi];
    uint32_t xq[G::RW / 2];  // x2 of this wave's rows, packed row pairs
    produce(s0 + wave * G::RW, s0 - 2, RWC{}, FUSED ? xq : nullptr);
    __syncthreads();  // ring complete; zst free
    const bool more = s0 + G::RS < S.t_end;
    // NB == 2: the prefetch of two sub-tiles ahead into the buffer just freed;
    // its loads and this sub-tile's output stores are the vector-memory ops
    // issued after the next sub-tile's loads (counted for the wait below
    // when both are whole)
    int after = -1;
    if constexpr (FUSED) {
      if constexpr (NB == 1) {
        if (more) prefetch(s0 + G::RS - 2);
      } else {
        const int rs2 = s0 + 2 * G::RS - 2;
        if (s0 + 2 * G::RS < S.t_end) {
          prefetch(rs2);
          if (vec_z && rs2 >= S.a && rs2 + G::ZROWS <= S.t_end)
            after = (ZW - wave + G::NWAVE - 1) / G::NWAVE;  // this wave's DMA instructions
        } else {
          after = 0;
        }
      }
    }

    // ---- FIR for rows s0 + 16*wave + r, r < 16
    const int pbase = (s0 - S.t0) + wave * G::RW;  // ring pos of row base
    // Tap pairs are consumed in order m = 0..NP-1.  At step m, odd row
    // r = 2j+1 reads window pair E[m + j + 1] against W[m], even row r = 2j
    // reads E[m + j] against V[m], and the even rows take one more step,
    // E[NP + j] against V[NP].  Even rows read the window pairs shifted by
    // one element against the odd rows, so they take the taps re-paired
    // the other way, V[m] = (w'[2m-1], w'[2m]) with w'[-1] = w'[KP] = 0, and
    // no window pair is ever re-aligned.  V[m] is formed at its step (one
    // v_alignbit for RW dot2) rather than held for the tile, which keeps
    // the tap registers to the NP pairs of W.
    // The window is loaded per 16-step quarter and the steps are fenced in
    // order, which keeps the live set to one quarter (otherwise the compiler
    // runs each accumulator's whole chain in turn and holds the whole
    // window).  Each fence also passes through the next step's tap pair, so
    // that step's V cannot be formed early (or hoisted out of the sweep).
    constexpr int MQ = G::NP >= 16 ? 16 : G::NP;  // tap pairs per quarter
    constexpr int EQ = MQ + G::RW / 2;            // window pairs per quarter
    static_assert(EQ % 4 == 0, "window quarters are whole b128 loads");
    float acc[G::RW];
#pragma unroll
    for (int r = 0; r < G::RW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int m0 = 0; m0 < G::NP; m0 += MQ) {
      uint32_t E[EQ];
#pragma unroll
      for (int q = 0; q < EQ / 4; ++q) {
        const uint4 v = *reinterpret_cast<const uint4 *>(&ring[lane][G::at(pbase + 2 * m0 + 8 * q)]);
        E[4 * q] = v.x; E[4 * q + 1] = v.y; E[4 * q + 2] = v.z; E[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        const int mm = m0 + m;
        const uint32_t wm = W[mm];
        const uint32_t vm = mm == 0 ? (W[0] << 16) : __builtin_amdgcn_alignbit(W[mm], W[mm - 1], 16);
#pragma unroll
        for (int j = 0; j < G::RW / 2; ++j) {
          acc[2 * j] = dot2(E[m + j], vm, acc[2 * j]);
          acc[2 * j + 1] = dot2(E[m + j + 1], wm, acc[2 * j + 1]);
        }
        // Empty volatile asm on every accumulator: volatile statements keep
        // their order, so step m+1 cannot start before step m is done.
#pragma unroll
        for (int r = 0; r < G::RW; ++r) asm volatile("" : "+v"(acc[r]));
        if (mm + 1 < G::NP) asm volatile("" : "+v"(W[mm + 1]));
      }
      if (m0 + MQ == G::NP) {
        const uint32_t vl = W[G::NP - 1] >> 16;
#pragma unroll
        for (int j = 0; j < G::RW / 2; ++j) acc[2 * j] = dot2(E[MQ + j], vl, acc[2 * j]);
      }
    }

    // hcm waits for the next sub-tile's rows (issued before its long FIR)
    // here, while no store is outstanding: stores count in vmcnt too, so a
    // wait after the epilogue also waits for the output rows to be
    // acknowledged.  hcs, whose FIR is short, measures faster waiting after
    // its stores.
    constexpr bool EARLY_LAND = K > 8;
    if constexpr (FUSED && EARLY_LAND) {
      if (more) {
        land();
        fix(s0 + G::RS - 2);
      }
    }

    // ---- epilogue on row pairs: bf16(y) [+ D*u] then * x2.
    uint32_t uq[G::RW / 2];
    if constexpr (HAS_D) {
#pragma unroll
      for (int q = 0; q < G::RW / 8; ++q) {
        const uint4 c4 = *reinterpret_cast<const uint4 *>(&ring[lane][G::at(pbase + G::KP + 8 * q)]);
        uq[4 * q] = c4.x; uq[4 * q + 1] = c4.y; uq[4 * q + 2] = c4.z; uq[4 * q + 3] = c4.w;
      }
    }
    float dval = 0.0f;
    if constexpr (HAS_D) dval = bf2f(p.D[cl]);
    const int trow = s0 + wave * G::RW;
    const bool full = trow + G::RW <= S.t_end && c0 + 64 <= p.H;  // uniform
    bf16_t *orow = obase + (int64_t)trow * p.so;
#pragma unroll
    for (int r = 0; r < G::RW; r += 2, orow += 2 * p.so) {
      uint32_t py;
      if constexpr (FUSED) {
        float y0 = rbf(acc[r]), y1 = rbf(acc[r + 1]);
        if constexpr (HAS_D) {
          const uint32_t pu = uq[r / 2];
          y0 = rbf_valu(y0 + rbf_valu(dval * lo_bf(pu)));
          y1 = rbf_valu(y1 + rbf_valu(dval * hi_bf(pu)));
        }
        const uint32_t px = xq[r / 2];
        py = pack_bf(lo_bf(px) * y0, hi_bf(px) * y1);
      } else {
        py = pack_bf(acc[r], acc[r + 1]);
      }
      // py = (row r, row r+1) of channel c
      const uint32_t nb = __shfl_xor(py, 1);
      const uint32_t dw = odd ? ((nb >> 16) | (py & 0xffff0000u)) : ((py & 0xffffu) | (nb << 16));
      if (full || (trow + r + (odd ? 1 : 0) < S.t_end && cpair < p.H))
        *reinterpret_cast<uint32_t *>(orow) = dw;
    }
    if constexpr (FUSED && !EARLY_LAND) {
      if (more) {
        if constexpr (NB == 2) {
          // wait for the next sub-tile's rows only: the ops issued after them
          // are this wave's prefetch and its RW / 2 row-pair stores
          const int n = full && after >= 0 ? after + G::RW / 2 : -1;  // uniform
          if (n == G::RW / 2 + 4) vmcnt_wait<G::RW / 2 + 4>();
          else if (n == G::RW / 2 + 3) vmcnt_wait<G::RW / 2 + 3>();
          else if (n == G::RW / 2) vmcnt_wait<G::RW / 2>();
          else land();
          zst = zbuf[bi ^ 1];
        } else {
          land();
        }
        fix(s0 + G::RS - 2);
      }
    }
    __syncthreads();  // next produce may overwrite the ring; zst committed
  }
}

// ---------------------------------------------------------------------------
// hcm (K = 128) fused prefill on the matrix cores.  Per channel the FIR is a
// Toeplitz product: for 16 output rows T + i (i < 16) and the 160-row window
// W[j] = u[T - 144 + j],
//
//   y[T + i] = sum_j A[i][j] W[j],   A[i][j] = w[j - i - 17] (0 outside 0..127),
//
// so 16 blocks of 16 rows, T = s0 + 16 n, are one v_mfma_f32_16x16x32_bf16
// chain of five k-steps: A (16 x 160, the channel's taps) times B (160 x 16,
// column n = the window of block n).  A depends on the channel only, so each
// wave builds the fragments of its four channels once per tile and keeps
// them in registers; the B fragments are aligned 8-row slices of the
// channel-major u ring.  u and the taps are bf16, so every product is exact
// and only the fp32 summation order differs from a per-tap loop.
//
// A workgroup owns 16 channels and one tile of rows, swept in 256-row
// sub-tiles:
//   produce:  thread (channel tid % 16, 16 rows) turns staged z rows into u
//             (to the ring) and x2 (kept in registers), as the dot2 kernel;
//   MFMA:     wave w runs the chains of channels 4w..4w+3 and writes bf16(y)
//             to a channel-major buffer;
//   epilogue: the thread that produced a row finishes it: [+ D*u] then * x2.
// The ring keeps 144 rows of history (the oldest row a window reaches).
// Workgroup order: the four 16-channel groups of a 64-channel block are
// workgroups b, b + 8, b + 16, b + 24, which run on one XCD back to back, so
// the 384-byte z row slice of the block is fetched into that XCD's L2 once.
namespace mfir {
constexpr int CH = 16;             // channels per workgroup
constexpr int NWAVE = 4;
constexpr int CPW = CH / NWAVE;    // channels per wave in the MFMA phase
constexpr int RS = 256;            // rows per sub-tile
constexpr int HIST = 144;          // history rows a sub-tile's windows reach
constexpr int RING = 512;          // ring rows per channel (power of two >= HIST + RS)
constexpr int KS = 5;              // MFMA k-steps (160-row window)
constexpr int ZW = 3 * CH;         // staged bf16 per z row
constexpr int ZROWS = RS + 2;      // staged z rows (sub-tile + short-filter halo)
constexpr int TAPW = 176;          // zero-padded taps per channel for the A build
static_assert(HIST + RS <= RING && HIST % 16 == 0, "ring geometry");
static_assert(CH * TAPW <= ZROWS * ZW, "the tap table borrows the z staging buffer");
}  // namespace mfir

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;

template <bool HAS_D>
__global__ __launch_bounds__(256, 2) void fir128_mfma_kernel(FirArgs p, int64_t ntiles, int64_t units) {
  using namespace mfir;
  // channel rows padded by 8 bf16 (16 bytes): consecutive channels start 4
  // banks apart, so the 16 channels a b128 access touches spread over all 64
  __shared__ __align__(16) bf16_t ring[CH][RING + 8];
  __shared__ __align__(16) bf16_t zst[ZROWS * ZW];
  __shared__ __align__(16) bf16_t ybuf[CH][RS + 8];

  // ---- workgroup -> (tile, 16-channel group)
  const int L = blockIdx.x;
  const int jslot = L >> 3;
  const int64_t unit = (static_cast<int64_t>(jslot >> 2) << 3) + (L & 7);
  if (unit >= units) return;  // uniform: padding of the grid to whole XCD rounds
  const int tile = static_cast<int>(unit % ntiles);
  const int c0 = static_cast<int>(unit / ntiles) * 64 + (jslot & 3) * CH;
  if (c0 >= p.H) return;  // uniform
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // produce / epilogue role: channel pc, rows 16 prg .. 16 prg + 15 of a sub-tile
  const int pc = tid & (CH - 1);
  const int prg = tid >> 4;
  const int c = c0 + pc;
  const bool active = c < p.H;
  const int cl = active ? c : p.H - 1;

  SegInfo S;
  {
    const int seg = p.tiles[2 * tile];
    S.t0 = p.tiles[2 * tile + 1];
    S.a = p.seq[3 * seg];
    S.e = p.seq[3 * seg + 1];
    S.blk = p.blocks[seg * p.sblk];
    S.init = p.seq[3 * seg + 2] != 0 && S.blk >= 0 && S.blk < p.num_blocks;
    S.t_end = min(S.t0 + p.block_t, S.e);
  }
  if (S.t0 >= S.t_end) return;  // uniform

  // ---- A fragments: lane (i = lane % 16, kg = lane / 16), k-step s, element
  // e holds A[i][32 s + 8 kg + e] = w[32 s + 8 kg + e - i - 17], read from a
  // zero-padded copy of the taps (tp[ch][x] = w[x - 32]) staged in zst.
  bf16x8_t A[CPW][KS];
  {
    bf16_t *tp = zst;
    for (int i = tid; i < CH * TAPW; i += 256) {
      const int ch = i / TAPW, k = i - ch * TAPW - 32;
      bf16_t v = 0;
      if (k >= 0 && k < 128 && c0 + ch < p.H) v = p.w[(int64_t)(c0 + ch) * p.w0 + k];
      tp[i] = v;
    }
    __syncthreads();
    const int ai = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc)
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          A[cc][s][e] = __builtin_bit_cast(__bf16, tp[(wave * CPW + cc) * TAPW + 32 * s + 8 * kg + e - ai + 15]);
    __syncthreads();  // zst is the z staging buffer from here on
  }

  ShortTaps wsp[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) wsp[i] = short_taps(p.ws, 3 * (int64_t)cl + i);
  const float *stc = S.init ? p.st + S.blk * p.st0 + (int64_t)cl * p.st1 : nullptr;
  float dval = 0.0f;
  if constexpr (HAS_D) dval = bf2f(p.D[cl]);
  const bool vec_z = (c0 + CH <= p.H) && (p.sx % 8 == 0) &&
                     ((reinterpret_cast<uintptr_t>(p.x) & 15) == 0) &&
                     p.sx * ZROWS < (int64_t(1) << 30);  // 32-bit lane byte offsets

  // ---- z rows [rs, rs + nrows) of the 48 sub-channels into zst (row pitch
  // 48 bf16 = 6 chunks of 16 bytes) with direct-to-LDS loads; rows outside
  // [a, t_end) are skipped.  `fix` (after the loads landed) writes the rows
  // a - 2 and a - 1 from the conv window (zero without one) and, when z is not
  // 16-byte addressable, every staged row element by element.
  auto prefetch = [&](int rs, int nrows) {
    if (!vec_z) return;
    const char *base = reinterpret_cast<const char *>(p.x + (int64_t)rs * p.sx + 3 * c0);
    const int nch = nrows * 6;
    const bool interior = rs >= S.a && rs + nrows <= S.t_end;  // uniform
    for (int j = 0;; ++j) {
      const int cw = wave + NWAVE * j;  // wave-uniform
      if (cw * 64 >= nch) break;
      const int i = cw * 64 + lane;
      const int row = i / 6;
      bool ok = i < nch;
      if (!interior) ok = ok && rs + row >= S.a && rs + row < S.t_end;
      const uint32_t off = 2u * static_cast<uint32_t>(row * static_cast<int>(p.sx) + 8 * (i - 6 * row));
      if (ok)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(base + off),
                                         (__attribute__((address_space(3))) void *)(zst + cw * 512),
                                         16, 0, 0);
    }
  };
  auto fix = [&](int rs, int nrows) {
    const bf16_t *conv = S.init ? p.cs + S.blk * p.cs0 : nullptr;
    if (vec_z && rs >= S.a) return;  // uniform: nothing to patch
    for (int i = tid; i < nrows * ZW; i += 256) {
      const int row = i / ZW, col = i - ZW * row;
      const int t = rs + row;
      const bool inside = t >= S.a && t < S.t_end;
      const bool left = t < S.a && t >= S.a - 2;
      if ((vec_z && inside) || !(inside || left)) continue;
      const int ch = 3 * c0 + col;
      bf16_t b = 0;
      if (ch < 3 * p.H) {
        if (inside) b = p.x[(int64_t)t * p.sx + ch];
        else if (conv) b = conv[ch * p.cs1 + (t - S.a + 2) * p.cs2];
      }
      zst[i] = b;
    }
  };
  auto land = [&]() { __builtin_amdgcn_s_waitcnt(0); };
  auto ring_pos = [&](int t) { return (t - S.t0 + HIST) & (RING - 1); };
  // output rows of this tile through a buffer descriptor that ends at the
  // tile's last row (16-byte stores of whole 16-channel groups)
  const bool vec_out = (c0 + CH <= p.H) && (p.so % 8 == 0) &&
                       ((reinterpret_cast<uintptr_t>(p.out) & 15) == 0) &&
                       (int64_t)(S.t_end - S.t0) * p.so * 2 < (int64_t(1) << 31);
  const __amdgpu_buffer_rsrc_t ores = __builtin_amdgcn_make_buffer_rsrc(
      p.out + (int64_t)S.t0 * p.so + c0, 0,
      vec_out ? static_cast<int>((int64_t)(S.t_end - S.t0) * p.so * 2) : 0, 0x00020000);

  // ---- u and x2 of this thread's 16 rows r0 .. r0 + 15 (z row t staged at
  // t - rs); u goes to the ring as two b128 stores, x2 to xq as row pairs.
  auto produce16 = [&](int r0, int rs, uint32_t (&xq)[8]) {
    uint32_t upk[8];
    if (r0 >= S.a && r0 + 16 <= S.t_end) {  // interior rows: pairs through v_dot2
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int sb = r0 - rs - 2 + 8 * g;  // staged row of z[r0 + 8 g - 2]
        uint32_t P[9][3];
#pragma unroll
        for (int k = 0; k < 9; ++k)
#pragma unroll
          for (int i = 0; i < 3; ++i)
            P[k][i] = pair_bf(zst[(sb + k) * ZW + 3 * pc + i], zst[(sb + k + 1) * ZW + 3 * pc + i]);
#pragma unroll
        for (int r = 0; r < 8; r += 2) {
          float y0[3], y1[3];
          short_rows2(P[r], P[r + 1], P[r + 2], wsp, y0, y1);
          upk[4 * g + r / 2] = pack_bf(y0[1] * y0[2], y1[1] * y1[2]);
          xq[4 * g + r / 2] = pack_bf(y0[0], y1[0]);
        }
      }
    } else {  // rows at a segment start or past the tile end, one at a time
#pragma unroll
      for (int q = 0; q < 8; ++q) upk[q] = xq[q] = 0u;
#pragma unroll 1
      for (int r = 0; r < 16; ++r) {
        const int t = r0 + r;
        float u = 0.0f, x2 = 0.0f;
        if (t < S.a) {
          const int col = 127 + (t - S.a);
          if (stc && col >= 0) u = stc[(int64_t)col * p.st2];
        } else if (t < S.t_end) {
          float y3[3];
          const int sr = t - rs;
          for (int i = 0; i < 3; ++i)
            y3[i] = short_dot_rbf(pair_bf(zst[(sr - 2) * ZW + 3 * pc + i], zst[(sr - 1) * ZW + 3 * pc + i]),
                                  pair_bf(zst[(sr - 1) * ZW + 3 * pc + i], zst[sr * ZW + 3 * pc + i]),
                                  wsp[i]);
          x2 = y3[0];
          u = rbf(y3[1] * y3[2]);
        }
        const uint32_t ub = f2bf(u), xb = f2bf(x2);
        // row r lands in the low (even r) or high (odd r) half of pair r / 2
        const int sh = 16 * (r & 1);
        for (int q = 0; q < 8; ++q) {
          if (q == r / 2) {
            upk[q] |= ub << sh;
            xq[q] |= xb << sh;
          }
        }
      }
    }
    const int pos = ring_pos(r0);
    *reinterpret_cast<uint4 *>(&ring[pc][pos]) = make_uint4(upk[0], upk[1], upk[2], upk[3]);
    *reinterpret_cast<uint4 *>(&ring[pc][pos + 8]) = make_uint4(upk[4], upk[5], upk[6], upk[7]);
  };

  // ---- halo: rows t0 - 144 .. t0 - 1 (nine row groups)
  {
    const int hs = S.t0 - HIST;
    prefetch(hs - 2, HIST + 2);
    land();
    fix(hs - 2, HIST + 2);
    __syncthreads();
    uint32_t xd[8];
    if (prg < HIST / 16) produce16(hs + 16 * prg, hs - 2, xd);
    __syncthreads();  // zst free
  }
  prefetch(S.t0 - 2, ZROWS);

  const int ai = lane & 15, kg = lane >> 4;
  for (int s0 = S.t0; s0 < S.t_end; s0 += RS) {
    const int nz = min(RS, S.t_end - s0) + 2;  // staged rows this sub-tile uses
    // this sub-tile's z rows: after the first sub-tile they were issued
    // before the previous epilogue's two buffer stores per wave, which may
    // stay in flight (loads and stores retire in order); the first sub-tile
    // and the element-wise store path wait for everything
    if (vec_out && s0 > S.t0) vmcnt_wait<2>();
    else land();
    fix(s0 - 2, nz);
    __syncthreads();  // staged rows visible
    uint32_t xq[8];
    produce16(s0 + 16 * prg, s0 - 2, xq);
    __syncthreads();  // ring complete; zst free
    if (s0 + RS < S.t_end) prefetch(s0 + RS - 2, min(RS, S.t_end - s0 - RS) + 2);

    // ---- MFMA: column block n = lane % 16 reads rows s0 + 16 n - 144 + 32 s
    // + 8 kg .. + 7, an aligned 8-row slice of the ring
    f32x4_t acc[CPW];
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) acc[cc] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int bpos = (s0 - S.t0) + 16 * ai + 8 * kg;  // ring position of the step-0 slice
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8_t B[CPW];
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc)
        B[cc] = *reinterpret_cast<const bf16x8_t *>(&ring[wave * CPW + cc][(bpos + 32 * s) & (RING - 1)]);
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc)
        acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[cc][s], B[cc], acc[cc], 0, 0, 0);
    }
    // lane holds y[s0 + 16 n + 4 kg + e], e < 4, of each channel
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const uint32_t lo = pack_bf(acc[cc][0], acc[cc][1]), hi = pack_bf(acc[cc][2], acc[cc][3]);
      *reinterpret_cast<uint2 *>(&ybuf[wave * CPW + cc][16 * ai + 4 * kg]) = make_uint2(lo, hi);
    }
    __syncthreads();  // ybuf complete

    // ---- epilogue: bf16(y) [+ D*u] then * x2 for rows s0 + 16 prg + r
    const int r0 = s0 + 16 * prg;
    const uint4 y4a = *reinterpret_cast<const uint4 *>(&ybuf[pc][16 * prg]);
    const uint4 y4b = *reinterpret_cast<const uint4 *>(&ybuf[pc][16 * prg + 8]);
    const uint32_t yq[8] = {y4a.x, y4a.y, y4a.z, y4a.w, y4b.x, y4b.y, y4b.z, y4b.w};
    uint32_t uq[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if constexpr (HAS_D) {
      const int pos = ring_pos(r0);
      const uint4 u4a = *reinterpret_cast<const uint4 *>(&ring[pc][pos]);
      const uint4 u4b = *reinterpret_cast<const uint4 *>(&ring[pc][pos + 8]);
      uq[0] = u4a.x; uq[1] = u4a.y; uq[2] = u4a.z; uq[3] = u4a.w;
      uq[4] = u4b.x; uq[5] = u4b.y; uq[6] = u4b.z; uq[7] = u4b.w;
    }
    uint32_t gq[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float y0 = lo_bf(yq[q]), y1 = hi_bf(yq[q]);
      if constexpr (HAS_D) {
        y0 = rbf_valu(y0 + rbf_valu(dval * lo_bf(uq[q])));
        y1 = rbf_valu(y1 + rbf_valu(dval * hi_bf(uq[q])));
      }
      gq[q] = pack_bf(lo_bf(xq[q]) * y0, hi_bf(xq[q]) * y1);
    }
    // g goes out through LDS as row-major 16-byte chunks (8 channels of a
    // row): gbuf (RS rows x CH channels) reuses ybuf once every thread has
    // read its y rows
    __syncthreads();
    bf16_t *gbuf = &ybuf[0][0];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      gbuf[(16 * prg + 2 * q) * CH + pc] = static_cast<bf16_t>(gq[q] & 0xffffu);
      gbuf[(16 * prg + 2 * q + 1) * CH + pc] = static_cast<bf16_t>(gq[q] >> 16);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int qi = tid + 256 * k, row = qi >> 1, half = qi & 1;
      const uint4 v = *reinterpret_cast<const uint4 *>(&gbuf[row * CH + 8 * half]);
      if (vec_out) {
        // rows past the tile end fall outside the descriptor and are dropped
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(i32x4_t, v), ores,
            ((s0 - S.t0 + row) * static_cast<int>(p.so) + 8 * half) * 2, 0, 0);
      } else {
        const int t = s0 + row;
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
        for (int e = 0; e < 8; ++e) {
          const int ce = c0 + 8 * half + e;
          if (t < S.t_end && ce < p.H)
            p.out[(int64_t)t * p.so + ce] = static_cast<bf16_t>(w4[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
    // the next produce overwrites ring rows this sub-tile's windows read
    // (all done: the barrier before the epilogue follows every wave's MFMAs)
    // and rows disjoint from those the epilogue reads; gbuf is read before
    // the next produce's barrier, after which the MFMAs rewrite it as ybuf
  }
}

// ---------------------------------------------------------------------------
// Window update after a prefill launch: per segment and channel, the new
// windows are the last inputs of cat(old window, segment) (mixers.py:380-382),
// oldest first.  The update is in place, and for a segment shorter than the
// window destination column q reads old column q + (e - a), so every value is
// gathered first and written after a workgroup barrier.  A workgroup owns 64
// channels of one segment (lane = channel for the gather: coalesced z rows);
// its waves park the values in LDS column by column, and after the barrier
// the block goes out in channel-major order, consecutive lanes on
// consecutive columns, so a window row is written as contiguous words rather
// than one word per channel.  The conv window (2 columns of the 3
// sub-channels) rides along with the first wave.  u near the segment start
// is recomputed through the short filter from z and the old conv window
// (FUSED), or read from u rows.
struct WinArgs {
  const bf16_t *x; int64_t sx;              // z (FUSED) or u rows
  const bf16_t *ws;
  bf16_t *cs; int64_t cs0, cs1, cs2;
  float *st; int64_t st0, st1, st2;
  const int32_t *seq;
  const int32_t *blocks; int64_t sblk;
  int H;
  bool fused;     // u from z through the short filter, else u = x
  bool conv;      // rewrite the conv window too
  int64_t num_blocks;
};

template <int W, int S>
__global__ __launch_bounds__(256) void window_update_kernel(WinArgs p) {
  constexpr int PER = (W + S - 1) / S;  // window columns per workgroup when split
  constexpr int CPW = (PER + 3) / 4;    // columns per wave per round
  constexpr int VP = 65;                // LDS floats per staged column (odd: no bank conflicts)
  __shared__ float vbuf[W][VP];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int cb = blockIdx.y * 64;
  const int c = cb + lane;
  const bool active = c < p.H;
  const int cl = active ? c : p.H - 1;
  const int seg = blockIdx.x;
  const int64_t a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  const int64_t blk = p.blocks[seg * p.sblk];
  if (e <= a || blk < 0 || blk >= p.num_blocks) return;  // uniform over the block
  // A segment of at least W + 2 rows reads no old window, so its columns are
  // split over the S workgroups of blockIdx.z; a shorter one is done whole
  // by the first, which reads every old value before it writes any.
  const bool split = e - a >= W + 2;
  if (!split && blockIdx.z != 0) return;
  const int r0 = split ? blockIdx.z : 0, r1 = split ? blockIdx.z + 1 : S;
  const bool init = p.seq[3 * seg + 2] != 0;
  const bf16_t *conv_old = init ? p.cs + blk * p.cs0 : nullptr;
  ShortCtx ctx{p.x, p.sx, conv_old, p.cs1, p.cs2, a, init};
  float *stb = p.st + blk * p.st0;
  float *st = stb + (int64_t)cl * p.st1;
  const int64_t last = e - 1;

  // ---- gather, one round per split.  Every load of a round is issued
  // before the first use: rows past the segment end (padding columns) are
  // clamped to its last row and their values discarded, and a window that
  // reaches before the segment start takes the slower per-row path.
  for (int round = r0; round < r1; ++round) {  // uniform
    const int q0 = round * PER + wave * CPW;
    const int qn = min(round * PER + PER, W);
    const int64_t src0 = e - W + q0;
    float v[CPW];
    if (p.fused) {
      float wsf[2][3], zz[CPW + 2][2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) wsf[i][j] = bf2f(p.ws[(3 * (int64_t)cl + 1 + i) * 3 + j]);
      if (src0 - 2 >= a) {  // uniform
#pragma unroll
        for (int r = 0; r < CPW + 2; ++r)
#pragma unroll
          for (int i = 0; i < 2; ++i)
            zz[r][i] = bf2f(p.x[min(src0 - 2 + r, last) * p.sx + 3 * (int64_t)cl + 1 + i]);
      } else {
#pragma unroll
        for (int r = 0; r < CPW + 2; ++r)
#pragma unroll
          for (int i = 0; i < 2; ++i)
            zz[r][i] = src0 - 2 + r <= last ? z_at(ctx, src0 - 2 + r, 3 * (int64_t)cl + 1 + i)
                                            : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < CPW; ++q)
        v[q] = rbf(short_out(zz[q][0], zz[q + 1][0], zz[q + 2][0], wsf[0]) *
                   short_out(zz[q][1], zz[q + 1][1], zz[q + 2][1], wsf[1]));
    } else {
#pragma unroll
      for (int q = 0; q < CPW; ++q) v[q] = bf2f(p.x[min(max(src0 + q, a), last) * p.sx + cl]);
    }
#pragma unroll
    for (int q = 0; q < CPW; ++q) {
      if (q0 + q >= qn) break;  // uniform
      if (src0 + q < a) v[q] = init ? st[(q0 + q + (e - a)) * p.st2] : 0.0f;
      vbuf[q0 + q][lane] = v[q];
    }
  }
  bf16_t cv[2][3];
  const bool do_conv = p.conv && wave == 0 && blockIdx.z == 0;
  bf16_t *cw = p.cs + blk * p.cs0;
  if (do_conv) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t src = e - 2 + q;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int64_t ch = 3 * (int64_t)cl + i;
        cv[q][i] = src >= a ? p.x[src * p.sx + ch]
                            : (init ? cw[ch * p.cs1 + (q + (e - a)) * p.cs2] : bf16_t(0));
      }
    }
  }
  __syncthreads();  // every old value is read before any write

  // ---- write columns [c0, c1) of the block's 64 channels
  const int c0 = r0 * PER, c1 = min(W, r1 * PER), ncol = c1 - c0;
  if (p.st2 == 1) {
    const int nch = min(64, p.H - cb);
    for (int f = threadIdx.x; f < nch * ncol; f += 256) {
      const int cc = f / ncol, q = c0 + f - cc * ncol;
      stb[(int64_t)(cb + cc) * p.st1 + q] = vbuf[q][cc];
    }
  } else if (active) {
    for (int q = c0; q < c1; ++q) st[q * p.st2] = vbuf[q][lane];
  }
  if (do_conv && active) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < 3; ++i) cw[(3 * (int64_t)c + i) * p.cs1 + q * p.cs2] = cv[q][i];
  }
}

template <int K, bool HAS_D, bool FUSED>
static void launch_fir(const FirArgs &a, int64_t ntiles, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(cdiv(a.H, 64)));
  hipLaunchKernelGGL((fir_prefill_kernel<K, HAS_D, FUSED>), grid, dim3(FirGeom<K>::NT), 0, st, a);
}

static int launch_window(const WinArgs &w, int K, int64_t nseq, hipStream_t st) {
  if (nseq == 0) return EVO2_OK;
  const unsigned gy = static_cast<unsigned>(cdiv(w.H, 64));
  if (K == 128)
    hipLaunchKernelGGL((window_update_kernel<127, 4>), dim3(static_cast<unsigned>(nseq), gy, 4),
                       dim3(256), 0, st, w);
  else
    hipLaunchKernelGGL((window_update_kernel<6, 1>), dim3(static_cast<unsigned>(nseq), gy, 1),
                       dim3(256), 0, st, w);
  return check_launch("prefill window update");
}

static int check_common(const char *fn, int64_t T, int64_t H, int32_t K, int64_t nseq,
                        int64_t ntiles, int32_t block_t, int64_t num_blocks) {
  if (T < 0 || H <= 0 || nseq < 0 || ntiles < 0 || num_blocks <= 0)
    return fail(EVO2_ERR_INVALID, "%s: bad sizes", fn);
  if (H % 2)
    return fail(EVO2_ERR_UNSUPPORTED, "%s: H=%lld must be even", fn, (long long)H);
  if (K != 7 && K != 128)
    return fail(EVO2_ERR_UNSUPPORTED, "%s: inner FIR length %d (7 or 128 only)", fn, K);
  if (block_t <= 0 || block_t % 64)
    return fail(EVO2_ERR_INVALID, "%s: block_t=%d must be a positive multiple of 64", fn, block_t);
  if (ntiles > 0x7fffffff || cdiv(H, 64) > 65535)
    return fail(EVO2_ERR_UNSUPPORTED, "%s: grid too large", fn);
  return EVO2_OK;
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_fir_prefill(const void *u, int64_t su, const void *w, int64_t w0, int64_t w1,
                                int32_t K, float *state, int64_t st0, int64_t st1, int64_t st2,
                                const int32_t *seq_table, int64_t nseq,
                                const int32_t *blocks, int64_t sblk,
                                const int32_t *tile_table, int64_t ntiles, int32_t block_t,
                                void *out, int64_t so, int64_t T, int64_t H,
                                int64_t num_blocks, void *stream) {
  int rc = check_common("fir_prefill", T, H, K, nseq, ntiles, block_t, num_blocks);
  if (rc) return rc;
  if (T == 0 || nseq == 0) return EVO2_OK;
  if (!u || !w || !state || !seq_table || !blocks || !out || (ntiles && !tile_table))
    return fail(EVO2_ERR_INVALID, "fir_prefill: null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  FirArgs a{static_cast<const bf16_t *>(u), su, nullptr, nullptr, 0, 0, 0,
            static_cast<const bf16_t *>(w), w0, w1, state, st0, st1, st2, nullptr,
            static_cast<bf16_t *>(out), so, seq_table, blocks, sblk, tile_table,
            static_cast<int>(H), block_t, num_blocks};
  if (K == 128 && (w1 != 1 || w0 % 8 || reinterpret_cast<uintptr_t>(w) % 16))
    return fail(EVO2_ERR_UNSUPPORTED, "fir_prefill: K=128 taps must be contiguous (H, 128) rows");
  if (ntiles) {
    if (K == 128) launch_fir<128, false, false>(a, ntiles, st);
    else launch_fir<7, false, false>(a, ntiles, st);
    rc = check_launch("fir_prefill");
    if (rc) return rc;
  }
  WinArgs wa{static_cast<const bf16_t *>(u), su, nullptr, nullptr, 0, 0, 0, state, st0, st1, st2,
             seq_table, blocks, sblk, static_cast<int>(H), false, false, num_blocks};
  return launch_window(wa, K, nseq, st);
}

extern "C" int evo2_hyena_fir_prefill(const void *z, int64_t sz, const void *short_w,
                                      void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                                      const void *w, int64_t w0, int64_t w1, int32_t K,
                                      float *inner_state, int64_t st0, int64_t st1, int64_t st2,
                                      const void *D,
                                      const int32_t *seq_table, int64_t nseq,
                                      const int32_t *blocks, int64_t sblk,
                                      const int32_t *tile_table, int64_t ntiles, int32_t block_t,
                                      void *out, int64_t so, int64_t T, int64_t H,
                                      int64_t num_blocks, void *stream) {
  int rc = check_common("hyena_fir_prefill", T, H, K, nseq, ntiles, block_t, num_blocks);
  if (rc) return rc;
  if (T == 0 || nseq == 0) return EVO2_OK;
  if (!z || !short_w || !conv_state || !w || !inner_state || !seq_table || !blocks || !out ||
      (ntiles && !tile_table))
    return fail(EVO2_ERR_INVALID, "hyena_fir_prefill: null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  FirArgs a{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
            static_cast<const bf16_t *>(conv_state), cs0, cs1, cs2,
            static_cast<const bf16_t *>(w), w0, w1, inner_state, st0, st1, st2,
            static_cast<const bf16_t *>(D), static_cast<bf16_t *>(out), so,
            seq_table, blocks, sblk, tile_table, static_cast<int>(H), block_t, num_blocks};
  if (K == 128 && (w1 != 1 || w0 % 8 || reinterpret_cast<uintptr_t>(w) % 16))
    return fail(EVO2_ERR_UNSUPPORTED, "hyena_fir_prefill: K=128 taps must be contiguous (H, 128) rows");
  StripeArgs sa{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
                static_cast<const bf16_t *>(conv_state), cs0, cs1, cs2,
                static_cast<const bf16_t *>(w), w0, inner_state, st0, st1, st2,
                nullptr, 0, 0, nullptr, 0, 0, nullptr, 0, 0, 0,
                static_cast<const bf16_t *>(D), static_cast<bf16_t *>(out), so, seq_table, nseq,
                blocks, sblk, tile_table, ntiles, block_t, static_cast<int>(H), num_blocks};
  if (ntiles && K == 128 && stripe_supported(sa, STRIPE_HCM, T, block_t)) {
    // 32-channel stripes over each tile (FIR history in LDS)
    rc = launch_stripe(sa, STRIPE_HCM, st);
    if (rc) return rc;
  } else if (ntiles) {
    const bool hasD = D != nullptr;
    if (K == 128 && block_t >= mfir::RS) {
      // the matrix-core kernel once a tile holds a whole 256-row sub-tile
      const int64_t units = ntiles * cdiv(H, 64);
      const int64_t nwg = 4 * cdiv(units, 8) * 8;
      if (nwg > 0x7fffffff) return fail(EVO2_ERR_UNSUPPORTED, "hyena_fir_prefill: grid too large");
      if (hasD)
        hipLaunchKernelGGL(fir128_mfma_kernel<true>, dim3(static_cast<unsigned>(nwg)), dim3(256), 0, st, a,
                           ntiles, units);
      else
        hipLaunchKernelGGL(fir128_mfma_kernel<false>, dim3(static_cast<unsigned>(nwg)), dim3(256), 0, st, a,
                           ntiles, units);
    } else if (K == 128) {
      hasD ? launch_fir<128, true, true>(a, ntiles, st) : launch_fir<128, false, true>(a, ntiles, st);
    } else {
      hasD ? launch_fir<7, true, true>(a, ntiles, st) : launch_fir<7, false, true>(a, ntiles, st);
    }
    rc = check_launch("hyena_fir_prefill");
    if (rc) return rc;
  }
  WinArgs wa{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
             static_cast<bf16_t *>(conv_state), cs0, cs1, cs2, inner_state, st0, st1, st2,
             seq_table, blocks, sblk, static_cast<int>(H), true, true, num_blocks};
  return launch_window(wa, K, nseq, st);
}
