// Varlen Hyena FIR prefill for gfx950: hcs (K=7) and hcm (K=128).
//
// Two forms share one kernel template:
//  * FUSED: the mixer's whole prefill core between in_proj and out_proj:
//    z (T, 3H) -> short K=3 filter -> u = x1*v -> FIR(u) [+ D*u] -> g = x2*y.
//  * U_IN: the reference's `fir_prefill` (triton_prefill.py:462-496): the
//    FIR over given u rows, output bf16(y).
//
// Layout.  A workgroup owns 64 channels (lane = channel) and one tile of
// rows of one segment (tile table [segment, first row], as
// mixers.py:386-415 builds it).  It sweeps the tile in 64-row sub-tiles:
//   produce: each wave turns 16 rows into u (and x2) for its 64 channels and
//            writes them into an LDS ring, u[channel][row mod RING];
//   FIR:     each lane computes 16 consecutive outputs of its channel from
//            the ring as bf16 pairs with v_dot2c_f32_bf16 (u and the taps are
//            bf16, so every product is exact in fp32).  Outputs at odd offsets
//            use pairs re-aligned by one element (one alignbit per tap pair
//            per 16 outputs); the channel's taps stay in VGPRs for the tile.
// The ring holds the K-1 rows of history the next sub-tile needs, so each
// z row is read from HBM once per tile plus a (K-1)-row halo per tile.
//
// Left context: rows before the segment start come from the cached windows
// when the segment continues a sequence (has_initial_state), else zero
// (mixers.py:126-141, 350-383).  The windows are rewritten by a second
// launch after every tile has read them (as triton_prefill.py:489-495).
#include "featurize.h"

namespace evo2 {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

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
  static constexpr int RS = 64;            // rows per sub-tile
  static constexpr int RW = 16;            // rows per wave in the FIR phase
  static constexpr int NE = NP + RW / 2;   // pairs in one wave's window
  static constexpr int RING = (KP + RS <= 128) ? 128 : 256;
  static constexpr int PITCH = RING + 8;   // bf16 per channel row (16-byte rows)
  static_assert(KP + RS <= RING, "ring too small");
};

struct SegInfo {
  int64_t a, e, t0, t_end, blk;
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
  s.t_end = min(s.t0 + (int64_t)p.block_t, s.e);
  return s;
}

template <int K, bool HAS_D, bool FUSED>
__global__ __launch_bounds__(256) void fir_prefill_kernel(FirArgs p) {
  using G = FirGeom<K>;
  __shared__ __align__(16) bf16_t ring[64][G::PITCH];
  __shared__ __align__(16) bf16_t x2s[64][G::RS + 8];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = blockIdx.y * 64 + lane;
  const bool active = c < p.H;
  const SegInfo S = seg_of_tile(p);
  if (S.t0 >= S.t_end) return;  // uniform across the block

  // Taps as bf16 pairs, one zero tap in front when K is odd.
  uint32_t W[G::NP];
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
  float wsf[3][3];
  ShortCtx ctx{};
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j)
        wsf[i][j] = active ? bf2f(p.ws[(3 * (int64_t)c + i) * 3 + j]) : 0.0f;
    ctx.z = p.x;
    ctx.sz = p.sx;
    ctx.conv = S.init ? p.cs + S.blk * p.cs0 : nullptr;
    ctx.cs1 = p.cs1;
    ctx.cs2 = p.cs2;
    ctx.a = S.a;
    ctx.init = S.init;
  }
  const float *stc = (S.init && active) ? p.st + S.blk * p.st0 + (int64_t)c * p.st1 : nullptr;

  // u (and x2) for rows [r0, r0 + n) by this wave, lane = channel.
  auto produce = [&](int64_t r0, int n, bool keep_x2) {
    float zm2[3] = {0.f, 0.f, 0.f}, zm1[3] = {0.f, 0.f, 0.f};
    if constexpr (FUSED) {
      if (active) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          zm2[i] = z_at(ctx, r0 - 2, 3 * (int64_t)c + i);
          zm1[i] = z_at(ctx, r0 - 1, 3 * (int64_t)c + i);
        }
      }
    }
    for (int r = 0; r < n; ++r) {
      const int64_t t = r0 + r;
      float u = 0.0f, x2 = 0.0f;
      if (active) {
        if (t < S.a) {
          const int64_t col = (K - 1) + (t - S.a);
          if (stc && col >= 0) u = stc[col * p.st2];
        } else if (t < S.t_end) {
          if constexpr (FUSED) {
            float z0[3], y3[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) {
              z0[i] = bf2f(p.x[t * p.sx + 3 * (int64_t)c + i]);
              y3[i] = short_out(zm2[i], zm1[i], z0[i], wsf[i]);
              zm2[i] = zm1[i];
              zm1[i] = z0[i];
            }
            x2 = y3[0];
            u = rbf(y3[1] * y3[2]);
          } else {
            u = bf2f(p.x[t * p.sx + c]);
          }
        }
        if constexpr (FUSED) {
          if (t < S.a) {
            // keep the short-filter window sliding through the left context
#pragma unroll
            for (int i = 0; i < 3; ++i) {
              zm2[i] = zm1[i];
              zm1[i] = z_at(ctx, t, 3 * (int64_t)c + i);
            }
          }
        }
      }
      const int pos = static_cast<int>((t - S.t0 + G::KP) & (G::RING - 1));
      ring[lane][pos] = f2bf(u);
      if (keep_x2) x2s[lane][(t - S.t0) & (G::RS - 1)] = f2bf(x2);
    }
  };

  // Halo: rows t0-KP .. t0-1, split over the four waves.
  {
    constexpr int per = G::KP / 4 > 0 ? G::KP / 4 : 1;
    if (wave * per < G::KP) produce(S.t0 - G::KP + wave * per, min(per, G::KP - wave * per), false);
  }

  for (int64_t s0 = S.t0; s0 < S.t_end; s0 += G::RS) {
    produce(s0 + wave * G::RW, G::RW, FUSED);
    __syncthreads();

    // ---- FIR for rows s0 + 16*wave + r, r < 16
    const int pbase = static_cast<int>(s0 - S.t0) + wave * G::RW;  // ring pos of row base
    uint32_t E[G::NE];
#pragma unroll
    for (int q = 0; q < G::NE / 4; ++q) {
      const uint4 v = *reinterpret_cast<const uint4 *>(&ring[lane][(pbase + 8 * q) & (G::RING - 1)]);
      E[4 * q] = v.x; E[4 * q + 1] = v.y; E[4 * q + 2] = v.z; E[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int i = (G::NE / 4) * 4; i < G::NE; ++i)
      E[i] = *reinterpret_cast<const uint32_t *>(&ring[lane][(pbase + 2 * i) & (G::RING - 1)]);
    float acc[G::RW];
#pragma unroll
    for (int r = 0; r < G::RW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int m = 0; m < G::NP; ++m) {
#pragma unroll
      for (int r = 0; r < G::RW; r += 2) {
        // row r (even) reads the odd-aligned pair starting at base+1+r+2m
        const uint32_t o = __builtin_amdgcn_alignbit(E[r / 2 + m + 1], E[r / 2 + m], 16);
        acc[r] = dot2(o, W[m], acc[r]);
        acc[r + 1] = dot2(E[r / 2 + m + 1], W[m], acc[r + 1]);
      }
    }

    // ---- epilogue: bf16(y) [+ D*u] then * x2; pair lanes to store dwords
    uint32_t vals[G::RW];
    float dval = 0.0f;
    if constexpr (HAS_D) dval = active ? bf2f(p.D[c]) : 0.0f;
#pragma unroll
    for (int r = 0; r < G::RW; ++r) {
      float y = rbf(acc[r]);
      if constexpr (FUSED) {
        const int pos = pbase + G::KP + r;  // ring position of row t
        const float u = bf2f(ring[lane][pos & (G::RING - 1)]);
        if constexpr (HAS_D) y = rbf(y + rbf(dval * u));
        y = bf2f(x2s[lane][(wave * G::RW + r) & (G::RS - 1)]) * y;
      }
      vals[r] = f2bf(y);
    }
    const bool odd = lane & 1;
#pragma unroll
    for (int r = 0; r < G::RW / 2; ++r) {
      // even lanes keep rows 0..7 of the pair (c, c+1); odd lanes rows 8..15.
      const uint32_t send = odd ? vals[r] : vals[r + G::RW / 2];
      const uint32_t recv = __shfl_xor(send, 1);
      const int rr = odd ? r + G::RW / 2 : r;
      const uint32_t mine = vals[rr];
      const uint32_t dw = odd ? (recv | (mine << 16)) : (mine | (recv << 16));
      const int64_t t = s0 + wave * G::RW + rr;
      const int cpair = c & ~1;
      if (t < S.t_end && cpair < p.H)
        *reinterpret_cast<uint32_t *>(p.out + t * p.so + cpair) = dw;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Window update after a prefill launch: per segment and channel, the new
// windows are the last inputs of cat(old window, segment) (mixers.py:380-382),
// written oldest first.  Destination column q reads source column q + (e-a)
// when it falls in the old window, so increasing q is safe in place.  The
// inner window is written before the conv window because recomputing u near
// the segment start reads the old conv window.
struct WinArgs {
  const bf16_t *x; int64_t sx;              // z (FUSED) or u rows
  const bf16_t *ws;
  bf16_t *cs; int64_t cs0, cs1, cs2;
  float *st; int64_t st0, st1, st2;
  const int32_t *seq;
  const int32_t *blocks; int64_t sblk;
  int H;
  int K;          // inner window K-1 columns; 0 for none
  bool fused;     // u from z through the short filter, else u = x
  bool conv;      // rewrite the conv window too
  int64_t num_blocks;
};

__global__ __launch_bounds__(64) void window_update_kernel(WinArgs p) {
  const int seg = blockIdx.x;
  const int c = blockIdx.y * 64 + threadIdx.x;
  if (c >= p.H) return;
  const int64_t a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  if (e <= a) return;
  const int64_t blk = p.blocks[seg * p.sblk];
  if (blk < 0 || blk >= p.num_blocks) return;
  const bool init = p.seq[3 * seg + 2] != 0;
  ShortCtx ctx{p.x, p.sx, init ? p.cs + blk * p.cs0 : nullptr, p.cs1, p.cs2, a, init};
  if (p.K > 1) {
    float *st = p.st + blk * p.st0 + (int64_t)c * p.st1;
    const int W = p.K - 1;
    float wsf[3][3];
    float zm2[3] = {0.f, 0.f, 0.f}, zm1[3] = {0.f, 0.f, 0.f};
    const int64_t src0 = e - W;
    if (p.fused) {
      for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j) wsf[i][j] = bf2f(p.ws[(3 * (int64_t)c + i) * 3 + j]);
        zm2[i] = z_at(ctx, src0 - 2, 3 * (int64_t)c + i);
        zm1[i] = z_at(ctx, src0 - 1, 3 * (int64_t)c + i);
      }
    }
    for (int q = 0; q < W; ++q) {
      const int64_t src = src0 + q;
      float v;
      if (p.fused) {
        float z0[3], y3[3];
        for (int i = 0; i < 3; ++i) {
          z0[i] = z_at(ctx, src, 3 * (int64_t)c + i);
          y3[i] = short_out(zm2[i], zm1[i], z0[i], wsf[i]);
          zm2[i] = zm1[i];
          zm1[i] = z0[i];
        }
        v = rbf(y3[1] * y3[2]);
      } else {
        v = (src >= a) ? bf2f(p.x[src * p.sx + c]) : 0.0f;
      }
      if (src < a) v = init ? st[(q + (e - a)) * p.st2] : 0.0f;
      st[q * p.st2] = v;
    }
  }
  if (p.conv) {
    bf16_t *cw = p.cs + blk * p.cs0;
    for (int q = 0; q < 2; ++q) {
      const int64_t src = e - 2 + q;
      for (int i = 0; i < 3; ++i) {
        const int64_t ch = 3 * (int64_t)c + i;
        bf16_t v;
        if (src >= a) v = p.x[src * p.sx + ch];
        else v = init ? cw[ch * p.cs1 + (q + (e - a)) * p.cs2] : bf16_t(0);
        cw[ch * p.cs1 + q * p.cs2] = v;
      }
    }
  }
}

template <int K, bool HAS_D, bool FUSED>
static void launch_fir(const FirArgs &a, int64_t ntiles, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(cdiv(a.H, 64)));
  hipLaunchKernelGGL((fir_prefill_kernel<K, HAS_D, FUSED>), grid, dim3(256), 0, st, a);
}

static int launch_window(const WinArgs &w, int64_t nseq, hipStream_t st) {
  if (nseq == 0) return EVO2_OK;
  dim3 grid(static_cast<unsigned>(nseq), static_cast<unsigned>(cdiv(w.H, 64)));
  hipLaunchKernelGGL(window_update_kernel, grid, dim3(64), 0, st, w);
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
  if (ntiles) {
    if (K == 128) launch_fir<128, false, false>(a, ntiles, st);
    else launch_fir<7, false, false>(a, ntiles, st);
    rc = check_launch("fir_prefill");
    if (rc) return rc;
  }
  WinArgs wa{static_cast<const bf16_t *>(u), su, nullptr, nullptr, 0, 0, 0, state, st0, st1, st2,
             seq_table, blocks, sblk, static_cast<int>(H), K, false, false, num_blocks};
  return launch_window(wa, nseq, st);
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
  if (ntiles) {
    const bool hasD = D != nullptr;
    if (K == 128) hasD ? launch_fir<128, true, true>(a, ntiles, st) : launch_fir<128, false, true>(a, ntiles, st);
    else hasD ? launch_fir<7, true, true>(a, ntiles, st) : launch_fir<7, false, true>(a, ntiles, st);
    rc = check_launch("hyena_fir_prefill");
    if (rc) return rc;
  }
  WinArgs wa{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
             static_cast<bf16_t *>(conv_state), cs0, cs1, cs2, inner_state, st0, st1, st2,
             seq_table, blocks, sblk, static_cast<int>(H), K, true, true, num_blocks};
  return launch_window(wa, nseq, st);
}
