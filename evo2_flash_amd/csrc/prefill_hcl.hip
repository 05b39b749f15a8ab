// Hyena-LI (hcl) prefill for gfx950: the long convolution as a chunked modal
// scan over 16 real poles per channel, replacing the reference's FFT
// convolution with the modal filter plus closed-form final state
// (mixers.py:144-210, triton_hcl.py:46-123, triton_prefill.py:351-387).
//
//   s_t = p (.) s_{t-1} + u_t,  y_t = sum_s r_s s_{t,s},  p = exp(lp)
//
// which equals the reference's y_t = (h * u)_t + sum_s r_s p_s^(t-a+1) s_{a-1,s}
// with h_n = sum_s r_s p_s^n (mixers.py:150-155), and whose last state is the
// reference's st = sum_t u_t p^(L-1-t) + p^L s_prev.
//
// Time is split into tiles of `block_t` rows (the same tile table as the FIR
// prefill) so that the launch has parallelism beyond H/256 workgroups:
//   phase 1  per tile, the end state of a scan started from zero;
//   phase 2  per segment, channel and pole, the carry into every tile
//            C_j = p^(L_{j-1}) C_{j-1} + E_{j-1}, C_0 = the cached state
//            (continuation) or 0, as one FMA chain over the tiles; the
//            segment's final state goes to the cache
//            (mixers.py:1391-1394);
//   phase 3  per tile, the scan again from its carry, the readout and the
//            mixer tail g = bf16(bf16(bf16(y) + bf16(u D)) x2) (mixers.py:1397).
// No workgroup waits on another, so the launch shape can never deadlock.
//
// Lanes run along channels (coalesced rows); a workgroup owns 256 channels
// (4 waves) and sweeps its tile in 8-row sub-tiles staged into LDS with
// direct-to-LDS loads, double-buffered so the next sub-tile lands while the
// current one computes.  Each wave stages, patches and reads only its own 64
// channels (a 384-byte slice of every z row), so the waves never wait for
// each other: the sweep has no barrier.
#include <mutex>
#include <type_traits>

#include "featurize.h"
#include "stripe.h"

namespace evo2 {

struct HclArgs {
  const bf16_t *z; int64_t sz;              // (T, 3H) in_proj rows
  const bf16_t *ws;                         // (3H, 3) short taps
  const bf16_t *cs; int64_t cs0, cs1, cs2;  // conv window view (blocks, 3H, 2)
  const float *res; int64_t r0, r1;         // residues (H, 16)
  const float *lp; int64_t l0, l1;          // log-poles (H, 16)
  float *ssm; int64_t m0, m1, m2;           // LI state view (blocks, H, 16)
  const bf16_t *D;                          // (H,)
  bf16_t *out; int64_t so;                  // g (T, H)
  const int32_t *seq;                       // (n, 3) [start, end, has_init]
  const int32_t *blocks; int64_t sblk;
  const int32_t *tiles;                     // (ntiles, 2) [segment, first row]
  const int32_t *tile_start;                // (n + 1) first tile of each segment
  float *work;                              // (ntiles, H, 16) tile end states / carries
  int H;
  int block_t;
  int64_t num_blocks;
};

constexpr int HCL_CH = 256;    // channels per workgroup (4 waves x 64 lanes)
constexpr int HCL_RS = 8;      // rows per sub-tile (8: three waves per SIMD in phase 3)
constexpr int HCL_TILE_ALIGN = 16;  // the documented block_t granularity
static_assert(HCL_TILE_ALIGN % HCL_RS == 0, "tiles are whole sub-tiles");
constexpr int HCL_ZROWS = HCL_RS + 2;
constexpr int HCL_WROW = 3 * 64;        // bf16 per staged row of one wave, unpadded
constexpr int HCL_WCH = HCL_ZROWS * HCL_WROW / 8;  // 16-byte chunks per wave stage (240)
constexpr int HCL_WINS = (HCL_WCH + 63) / 64;      // wave instructions per stage (4)
constexpr int HCL_WBUF = HCL_WINS * 512;           // bf16 per wave buffer (whole 1 KB loads)

template <int PHASE>
__global__ __launch_bounds__(256, PHASE == 3 ? 4 : 5) void hcl_scan_kernel(HclArgs p) {
  // Two staging buffers per wave (distinct variables, so reading one never
  // waits on the direct-to-LDS loads still landing in the other): sub-tile
  // i + 1 is loaded while sub-tile i computes.  Chunk i of a wave's stage
  // (16 bytes: row i / 24, column i % 24 of its slice) sits at bf16 offset
  // 8 i, so a staged row is 192 bf16 of (x2, x1, v) triples, lane-ordered.
  __shared__ __align__(16) bf16_t zs0[4][HCL_WBUF];
  __shared__ __align__(16) bf16_t zs1[4][HCL_WBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int c0 = blockIdx.y * HCL_CH;
  const int c = c0 + tid;  // lane = channel
  const bool active = c < p.H;
  const int cl = active ? c : p.H - 1;
  const int seg = p.tiles[2 * blockIdx.x];
  const int t0 = p.tiles[2 * blockIdx.x + 1];
  const int a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  const int64_t blk = p.blocks[seg * p.sblk];
  const bool init = p.seq[3 * seg + 2] != 0 && blk >= 0 && blk < p.num_blocks;
  const int t_end = min(t0 + p.block_t, e);
  if (t0 >= t_end) return;  // uniform
  // Waves are independent (own staging buffers, no barrier): one whose 64
  // channels all lie past H has nothing to do.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (c0 + 64 * wave >= p.H) return;

  ShortTaps wsp[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) wsp[i] = short_taps(p.ws, 3 * (int64_t)cl + i);
  float pole[16], res[16], s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    pole[i] = expf(p.lp[(int64_t)cl * p.l0 + i * p.l1]);
    res[i] = PHASE == 3 ? p.res[(int64_t)cl * p.r0 + i * p.r1] : 0.0f;
    s[i] = PHASE == 3 ? p.work[((int64_t)blockIdx.x * p.H + cl) * 16 + i] : 0.0f;
  }
  const float dval = PHASE == 3 ? bf2f(p.D[cl]) : 0.0f;
  // Per wave: the last group of an H that is not a multiple of 256 keeps its
  // whole waves on 16-byte staging.
  const bool vec_z = (c0 + 64 * wave + 64 <= p.H) && (p.sz % 8 == 0) &&
                     ((reinterpret_cast<uintptr_t>(p.z) & 15) == 0) &&
                     p.sz * HCL_ZROWS < (int64_t(1) << 30);  // 32-bit byte offsets
  const bf16_t *conv = init ? p.cs + blk * p.cs0 : nullptr;
  const int cw0 = 3 * (c0 + 64 * wave);  // first z column of this wave's slice
  // Rows [rs, rs + HCL_ZROWS) of the tile, this wave's slice: `prefetch`
  // issues direct-to-LDS loads for the interior rows; `fix` (after they land)
  // writes the rows the loads skip element by element: the short filter's
  // left context (conv window when continuing, else zero) and every row when
  // z is not 16-byte addressable.  Rows past the tile end are never read.
  // The per-lane offsets are recomputed at every prefetch from the lane id,
  // passed through an empty asm so that the compiler cannot hoist them: held
  // across the sweep they are the first values spilled, and reloading a
  // spill waits for the loads already in flight.
  auto prefetch = [&](auto buf, int rs) {
    bf16_t *zw = (decltype(buf)::value ? zs1 : zs0)[wave];
    if (!vec_z) return;
    const char *base = reinterpret_cast<const char *>(p.z + (int64_t)rs * p.sz + cw0);
    const bool interior = rs >= a && rs + HCL_ZROWS <= t_end;  // uniform
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int j = 0; j < HCL_WINS; ++j) {
      const int i = 64 * j + ln, row = i / 24;
      bool ok = i < HCL_WCH;
      if (!interior) ok = ok && rs + row >= a && rs + row < t_end;
      const uint32_t o = 2u * static_cast<uint32_t>(row * static_cast<int>(p.sz) + 8 * (i - 24 * row));
      if (ok)
        __builtin_amdgcn_global_load_lds(
            reinterpret_cast<const uint4 *>(base + o),
            (__attribute__((address_space(3))) void *)(zw + 512 * j), 16, 0, 0);
    }
  };
  auto fix = [&](auto buf, int rs) {
    bf16_t *zw = (decltype(buf)::value ? zs1 : zs0)[wave];
    if (vec_z && rs >= a) return;  // uniform: nothing to patch
#pragma unroll 1
    for (int i = lane; i < HCL_WCH; i += 64) {
      const int row = i / 24, col = i - 24 * row;
      const int t = rs + row;
      const bool inside = t >= a && t < t_end;
      if (vec_z && inside) continue;
#pragma unroll 1
      for (int q = 0; q < 8; ++q) {
        const int ch = cw0 + 8 * col + q;
        bf16_t b = 0;
        if (ch < 3 * p.H) {
          if (inside) b = p.z[(int64_t)t * p.sz + ch];
          else if (conv && t < a && t >= a - 2) b = conv[ch * p.cs1 + (t - a + 2) * p.cs2];
        }
        zw[8 * i + q] = b;
      }
    }
  };

  // One sub-tile from a staged buffer: short filter, gate, the scan
  // (and in phase 3 the readout and the mixer tail, stored as bf16 rows).
  // FULL: all HCL_RS rows are inside the tile, so no row is checked (a
  // per-row condition would make the compiler copy the 16 states around it).
  auto compute = [&](auto buf, auto full, int s0) {
    const bf16_t *zw = (decltype(buf)::value ? zs1 : zs0)[wave];
    constexpr bool FULL = decltype(full)::value;
    const int nr = FULL ? HCL_RS : min(HCL_RS, t_end - s0);
    // Row pairs (z[k], z[k+1]) of each sub-channel over the staged rows; rows
    // past the tile end hold stale values that only discarded rows read.
    uint32_t P[HCL_RS + 1][3];
#pragma unroll
    for (int k = 0; k <= HCL_RS; ++k)
#pragma unroll
      for (int i = PHASE == 3 ? 0 : 1; i < 3; ++i)
        P[k][i] = pair_bf(zw[HCL_WROW * k + 3 * lane + i], zw[HCL_WROW * (k + 1) + 3 * lane + i]);
    uint32_t gpk[HCL_RS / 2];
#pragma unroll
    for (int r = 0; r < HCL_RS; r += 2) {
      float ypair[2] = {0.f, 0.f}, upair[2], x2pair[2];
      if constexpr (PHASE == 3) {
        float y0[3], y1[3];  // (x2, x1, v) of rows r and r + 1, rounded
        short_rows2(P[r], P[r + 1], P[r + 2], wsp, y0, y1);
        x2pair[0] = y0[0];
        x2pair[1] = y1[0];
        upair[0] = rbf_valu(y0[1] * y0[2]);
        upair[1] = rbf_valu(y1[1] * y1[2]);
      } else {  // the end states need only u
        const uint32_t Pa[2] = {P[r][1], P[r][2]}, Pb[2] = {P[r + 1][1], P[r + 1][2]},
                       Pc[2] = {P[r + 2][1], P[r + 2][2]};
        const ShortTaps w12[2] = {wsp[1], wsp[2]};
        float y0[2], y1[2];  // (x1, v) of rows r and r + 1, rounded
        short_rows2(Pa, Pb, Pc, w12, y0, y1);
        upair[0] = rbf_valu(y0[0] * y0[1]);
        upair[1] = rbf_valu(y1[0] * y1[1]);
        x2pair[0] = x2pair[1] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (FULL || r + q < nr) {  // uniform
          float ya = 0.f, yb = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            s[i] = fmaf(pole[i], s[i], upair[q]);
            if constexpr (PHASE == 3) {
              if ((i & 1) == 0) ya = fmaf(res[i], s[i], ya);
              else yb = fmaf(res[i], s[i], yb);
            }
          }
          ypair[q] = ya + yb;
        }
      }
      if constexpr (PHASE == 3) {
        // g = bf16(bf16(bf16(y) + bf16(u D)) x2) for both rows
        const float s0r = rbf_valu(rbf_valu(ypair[0]) + rbf_valu(upair[0] * dval));
        const float s1r = rbf_valu(rbf_valu(ypair[1]) + rbf_valu(upair[1] * dval));
        gpk[r / 2] = pack_bf(x2pair[0] * s0r, x2pair[1] * s1r);
      }
    }
    if constexpr (PHASE == 3) {
      // gpk[r/2] = (row r, row r+1) of channel c; even lanes store row r of
      // the pair (c, c+1), odd lanes row r+1 of (c-1, c).
      const bool odd = lane & 1;
      const int cpair = c & ~1;
      bf16_t *orow = p.out + (int64_t)s0 * p.so + cpair;
#pragma unroll
      for (int r = 0; r < HCL_RS; r += 2) {
        const uint32_t py = gpk[r / 2];
        const uint32_t nb = __shfl_xor(py, 1);
        const uint32_t dw = odd ? ((nb >> 16) | (py & 0xffff0000u)) : ((py & 0xffffu) | (nb << 16));
        const int rr = r + (odd ? 1 : 0);
        if ((FULL || rr < nr) && cpair < p.H) *reinterpret_cast<uint32_t *>(orow + (int64_t)rr * p.so) = dw;
      }
    }
  };

  // Sub-tile i lives in buffer i & 1.  Per sub-tile: wait for its loads
  // (and, by the same count, for this wave's reads of the other buffer),
  // patch its boundary rows, issue the next sub-tile into the other buffer,
  // compute.  Every step touches only this wave's buffers.
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  auto sub = [&](auto buf, auto nbuf, int s0) {
    __builtin_amdgcn_s_waitcnt(0);
    fix(buf, s0 - 2);
    if (s0 + HCL_RS < t_end) prefetch(nbuf, s0 + HCL_RS - 2);
    if (s0 + HCL_RS <= t_end)  // uniform
      compute(buf, std::true_type{}, s0);
    else
      compute(buf, std::false_type{}, s0);
  };
  prefetch(B0{}, t0 - 2);
  for (int s0 = t0; s0 < t_end; s0 += 2 * HCL_RS) {
    sub(B0{}, B1{}, s0);
    if (s0 + HCL_RS < t_end) sub(B1{}, B0{}, s0 + HCL_RS);
  }
  if constexpr (PHASE == 1) {
    if (active) {
      float4 *w = reinterpret_cast<float4 *>(p.work + ((int64_t)blockIdx.x * p.H + c) * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) w[q] = make_float4(s[4 * q], s[4 * q + 1], s[4 * q + 2], s[4 * q + 3]);
    }
  }
}

// Phase 2: the carry across tiles.  Tile l of a segment maps its entering
// state s to p^len_l (.) s + E_l (E_l: its end state from a zero start), so
// the state entering tile l is C_l = p^len_{l-1} (.) C_{l-1} + E_{l-1}, with
// C_0 the segment's initial state.  One lane per (channel, pole): the chain
// is one FMA per tile, and consecutive lanes read consecutive floats of the
// tile end states, 16 tiles per batch of loads.  (A wavefront-per-channel
// form that composed the maps with a 6-step shuffle scan over 64 tiles ran
// the 7B/32k carry slower, ~23 us against ~17.)  The carries replace the end
// states in `work`; the state after the last tile is returned.
__device__ __forceinline__ float carry_chain(float *work, int64_t H, int c, int i, int j0, int n,
                                             int first_t0, int block_t, int e, float lpv,
                                             float S) {
  const float afull = expf(lpv * static_cast<float>(block_t));
  float *wp = work + ((int64_t)j0 * H + c) * 16 + i;
  const int64_t ts = H * 16;  // floats between tiles
  int t = first_t0;
  for (int b = 0; b < n; b += 16) {
    float E[16];
    const float *rp = wp;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      E[q] = b + q < n ? *rp : 0.0f;
      rp += ts;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (b + q < n) {  // uniform
        *wp = S;  // the carry into tile b + q
        wp += ts;
        const int len = min(t + block_t, e) - t;
        t += block_t;
        const float A = len == block_t ? afull : expf(lpv * static_cast<float>(len));
        S = fmaf(A, S, E[q]);
      }
    }
  }
  return S;
}

// One lane per (segment, channel, pole); writes the segment's final state
// to the cache (mixers.py:1391-1394).
__global__ __launch_bounds__(256) void hcl_carry_kernel(HclArgs p) {
  const int seg = blockIdx.x;
  const int gi = blockIdx.y * 256 + threadIdx.x;
  const int c = gi >> 4, i = gi & 15;
  if (c >= p.H) return;
  const int a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  if (e <= a) return;
  const int64_t blk = p.blocks[seg * p.sblk];
  if (blk < 0 || blk >= p.num_blocks) return;
  const bool init = p.seq[3 * seg + 2] != 0;
  float *st = p.ssm + blk * p.m0 + (int64_t)c * p.m1 + i * p.m2;
  float S = init ? *st : 0.0f;
  const float lpv = p.lp[(int64_t)c * p.l0 + i * p.l1];
  const int j0 = p.tile_start[seg], n = p.tile_start[seg + 1] - j0;
  if (n > 0) S = carry_chain(p.work, p.H, c, i, j0, n, p.tiles[2 * j0 + 1], p.block_t, e, lpv, S);
  *st = S;
}

// Conv window update for the LI prefill: same contract as the FIR window
// kernel, conv slice only.
__global__ __launch_bounds__(64) void hcl_conv_window_kernel(HclArgs p) {
  const int seg = blockIdx.x;
  const int c = blockIdx.y * 64 + threadIdx.x;
  if (c >= p.H) return;
  const int64_t a = p.seq[3 * seg], e = p.seq[3 * seg + 1];
  if (e <= a) return;
  const int64_t blk = p.blocks[seg * p.sblk];
  if (blk < 0 || blk >= p.num_blocks) return;
  const bool init = p.seq[3 * seg + 2] != 0;
  bf16_t *cw = const_cast<bf16_t *>(p.cs) + blk * p.cs0;
  for (int q = 0; q < 2; ++q) {
    const int64_t src = e - 2 + q;
    for (int i = 0; i < 3; ++i) {
      const int64_t ch = 3 * (int64_t)c + i;
      bf16_t v;
      if (src >= a) v = p.z[src * p.sz + ch];
      else v = init ? cw[ch * p.cs1 + (q + (e - a)) * p.cs2] : bf16_t(0);
      cw[ch * p.cs1 + q * p.cs2] = v;
    }
  }
}

}  // namespace evo2

using namespace evo2;

extern "C" int64_t evo2_hcl_workspace_bytes(int64_t ntiles, int64_t H) {
  return ntiles * H * 16 * static_cast<int64_t>(sizeof(float));
}

namespace evo2 {

// The fused LI prefill's checks and launches, shared by the entry point that
// takes a workspace and the one that uses the library's scratch.
static int hcl_prefill(const void *z, int64_t sz, const void *short_w,
                       void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                       const float *residues, int64_t r0, int64_t r1,
                       const float *log_poles, int64_t l0, int64_t l1,
                       float *ssm, int64_t m0, int64_t m1, int64_t m2, const void *D,
                       const int32_t *seq_table, int64_t nseq,
                       const int32_t *blocks, int64_t sblk,
                       const int32_t *tile_table, int64_t ntiles,
                       const int32_t *tile_start, int32_t block_t,
                       float *workspace, int64_t workspace_bytes,
                       void *out, int64_t so, int64_t T, int64_t H,
                       int64_t num_blocks, void *stream) {
  if (T < 0 || H <= 0 || nseq < 0 || ntiles < 0 || num_blocks <= 0)
    return fail(EVO2_ERR_INVALID, "hyena_hcl_prefill: bad sizes");
  if (H % 2) return fail(EVO2_ERR_UNSUPPORTED, "hyena_hcl_prefill: H must be even");
  if (block_t <= 0 || block_t % HCL_TILE_ALIGN)
    return fail(EVO2_ERR_INVALID, "hyena_hcl_prefill: block_t=%d must be a multiple of %d",
                block_t, HCL_TILE_ALIGN);
  if (T == 0 || nseq == 0) return EVO2_OK;
  if (!z || !short_w || !conv_state || !residues || !log_poles || !ssm || !D || !seq_table ||
      !blocks || !out || !tile_start || (ntiles && (!tile_table || !workspace)))
    return fail(EVO2_ERR_INVALID, "hyena_hcl_prefill: null pointer argument");
  if (workspace_bytes < evo2_hcl_workspace_bytes(ntiles, H))
    return fail(EVO2_ERR_INVALID, "hyena_hcl_prefill: workspace of %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)evo2_hcl_workspace_bytes(ntiles, H));
  if (ntiles > 0x7fffffff || cdiv(H, HCL_CH) > 65535)
    return fail(EVO2_ERR_UNSUPPORTED, "hyena_hcl_prefill: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  {
    // whole segments per tile: the single-pass kernel (no carry pass, z read once)
    StripeArgs sa{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
                  static_cast<const bf16_t *>(conv_state), cs0, cs1, cs2, nullptr, 0,
                  nullptr, 0, 0, 0, residues, r0, r1, log_poles, l0, l1, ssm, m0, m1, m2,
                  static_cast<const bf16_t *>(D), static_cast<bf16_t *>(out), so, seq_table, nseq,
                  blocks, sblk, tile_table, ntiles, block_t, static_cast<int>(H), num_blocks};
    if (stripe_supported(sa, STRIPE_HCL, T, block_t)) {
      int rc = launch_stripe(sa, STRIPE_HCL, st);
      if (rc) return rc;
      HclArgs wa{static_cast<const bf16_t *>(z), sz, nullptr, static_cast<const bf16_t *>(conv_state),
                 cs0, cs1, cs2, nullptr, 0, 0, nullptr, 0, 0, nullptr, 0, 0, 0, nullptr, nullptr, 0,
                 seq_table, blocks, sblk, nullptr, nullptr, nullptr, static_cast<int>(H), block_t,
                 num_blocks};
      hipLaunchKernelGGL(hcl_conv_window_kernel, dim3(static_cast<unsigned>(nseq),
                         static_cast<unsigned>(cdiv(H, 64))), dim3(64), 0, st, wa);
      return check_launch("hcl conv window");
    }
  }
  HclArgs a{static_cast<const bf16_t *>(z), sz, static_cast<const bf16_t *>(short_w),
            static_cast<const bf16_t *>(conv_state), cs0, cs1, cs2, residues, r0, r1,
            log_poles, l0, l1, ssm, m0, m1, m2, static_cast<const bf16_t *>(D),
            static_cast<bf16_t *>(out), so, seq_table, blocks, sblk, tile_table, tile_start,
            workspace, static_cast<int>(H), block_t, num_blocks};
  if (ntiles) {
    dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(cdiv(H, HCL_CH)));
    hipLaunchKernelGGL(hcl_scan_kernel<1>, grid, dim3(256), 0, st, a);
    int rc = check_launch("hcl phase 1");
    if (rc) return rc;
  }
  dim3 cgrid(static_cast<unsigned>(nseq), static_cast<unsigned>(cdiv(H, 16)));
  hipLaunchKernelGGL(hcl_carry_kernel, cgrid, dim3(256), 0, st, a);
  dim3 sgrid(static_cast<unsigned>(nseq), static_cast<unsigned>(cdiv(H, 64)));
  int rc = check_launch("hcl phase 2");
  if (rc) return rc;
  if (ntiles) {
    dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(cdiv(H, HCL_CH)));
    hipLaunchKernelGGL(hcl_scan_kernel<3>, grid, dim3(256), 0, st, a);
    rc = check_launch("hcl phase 3");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(hcl_conv_window_kernel, sgrid, dim3(64), 0, st, a);
  return check_launch("hcl conv window");
}

}  // namespace evo2

extern "C" int evo2_hyena_hcl_prefill(const void *z, int64_t sz, const void *short_w,
                                      void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                                      const float *residues, int64_t r0, int64_t r1,
                                      const float *log_poles, int64_t l0, int64_t l1,
                                      float *ssm, int64_t m0, int64_t m1, int64_t m2,
                                      const void *D,
                                      const int32_t *seq_table, int64_t nseq,
                                      const int32_t *blocks, int64_t sblk,
                                      const int32_t *tile_table, int64_t ntiles,
                                      const int32_t *tile_start, int32_t block_t,
                                      float *workspace, int64_t workspace_bytes,
                                      void *out, int64_t so, int64_t T, int64_t H,
                                      int64_t num_blocks, void *stream) {
  return hcl_prefill(z, sz, short_w, conv_state, cs0, cs1, cs2, residues, r0, r1, log_poles,
                     l0, l1, ssm, m0, m1, m2, D, seq_table, nseq, blocks, sblk, tile_table,
                     ntiles, tile_start, block_t, workspace, workspace_bytes, out, so, T, H,
                     num_blocks, stream);
}

// ---------------------------------------------------------------------------
// The LI prefill without a workspace argument, for callers that cannot
// allocate device memory.  Its tile end states and carries go to `scratch`,
// a file-scope device array every GPU that runs this library holds for the
// life of the process.  In host code `scratch` names a host-side stand-in,
// not device memory: the address a kernel may use is taken once per device
// with hipGetSymbolAddress, with that device current, and kept in
// g_scratch_dev.  Calls on one GPU share its array, so calls that overlap on
// one GPU (concurrent streams) race.  Nothing in it needs clearing between
// calls: phase 1 writes the end state of every tile before phase 2 reads
// any, and phase 2 writes every carry before phase 3 reads it.
namespace evo2 {

constexpr int64_t HCL_SCRATCH_BYTES = int64_t(32) << 20;
static __device__ __align__(256) float scratch[HCL_SCRATCH_BYTES / sizeof(float)];

constexpr int HCL_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static float *g_scratch_dev[HCL_MAX_DEVICES];

// This device's address of `scratch` (looked up on the first call made with
// the device current).  The kernels run on the stream's device, so a stream
// of another device than the current one is refused: its kernels would be
// handed the current device's address.
static int scratch_for_current_device(hipStream_t stream, float **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(EVO2_ERR_DEVICE, "hyena_hcl_prefill_noalloc: hipGetDevice failed: %s",
                hipGetErrorString(e));
  if (stream) {  // the null stream belongs to the current device
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess)
      return fail(EVO2_ERR_DEVICE, "hyena_hcl_prefill_noalloc: hipStreamGetDevice failed: %s",
                  hipGetErrorString(e));
    if (sdev != dev)
      return fail(EVO2_ERR_INVALID,
                  "hyena_hcl_prefill_noalloc: the stream is on device %d but device %d is "
                  "current; make the stream's device current first",
                  static_cast<int>(sdev), dev);
  }
  if (dev < 0 || dev >= HCL_MAX_DEVICES)
    return fail(EVO2_ERR_UNSUPPORTED, "hyena_hcl_prefill_noalloc: device %d beyond %d", dev,
                HCL_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(EVO2_ERR_DEVICE,
                  "hyena_hcl_prefill_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<float *>(ptr);
  }
  *out = g_scratch_dev[dev];
  return EVO2_OK;
}

}  // namespace evo2

extern "C" int evo2_hyena_hcl_prefill_noalloc(
    const void *z, int64_t sz, const void *short_w,
    void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
    const float *residues, int64_t r0, int64_t r1,
    const float *log_poles, int64_t l0, int64_t l1,
    float *ssm, int64_t m0, int64_t m1, int64_t m2, const void *D,
    const int32_t *seq_table, int64_t nseq, const int32_t *blocks, int64_t sblk,
    const int32_t *tile_table, int64_t ntiles, const int32_t *tile_start, int32_t block_t,
    void *out, int64_t so, int64_t T, int64_t H, int64_t num_blocks, void *stream) {
  if (ntiles < 0 || H <= 0)
    return fail(EVO2_ERR_INVALID, "hyena_hcl_prefill_noalloc: bad sizes");
  const int64_t need = evo2_hcl_workspace_bytes(ntiles, H);
  if (need > HCL_SCRATCH_BYTES)
    return fail(EVO2_ERR_UNSUPPORTED,
                "hyena_hcl_prefill_noalloc: %lld tiles at H=%lld need %lld bytes of scratch, "
                "more than its %lld (use evo2_hyena_hcl_prefill with a workspace, or fewer "
                "tiles)", (long long)ntiles, (long long)H, (long long)need,
                (long long)HCL_SCRATCH_BYTES);
  float *work = nullptr;
  int rc = scratch_for_current_device(static_cast<hipStream_t>(stream), &work);
  if (rc) return rc;
  return hcl_prefill(z, sz, short_w, conv_state, cs0, cs1, cs2, residues, r0, r1, log_poles,
                     l0, l1, ssm, m0, m1, m2, D, seq_table, nseq, blocks, sblk, tile_table,
                     ntiles, tile_start, block_t, work, HCL_SCRATCH_BYTES, out, so, T, H,
                     num_blocks, stream);
}

// ---------------------------------------------------------------------------
// iir_segment (mixers.py:144-210): one segment of the LI recurrence over an
// fp32 (H, L) input with any strides, from a cached state or zero.  Same
// three phases as the mixer prefill, lane = channel, rows sequential per tile.
namespace evo2 {

struct IirArgs {
  const float *x; int64_t xh, xl;           // seq (H, L)
  const float *res; int64_t r0, r1;
  const float *lp; int64_t l0, l1;
  const float *sp; int64_t sp0, sp1;        // s_prev (H, 16) or null
  float *y; int64_t yh, yl;                 // y (H, L)
  float *st;                                // (H, 16) contiguous final state
  float *work;                              // (ntiles, H, 16)
  int H, L, block_t, ntiles;
};

template <int PHASE>
__global__ __launch_bounds__(256) void iir_scan_kernel(IirArgs p) {
  const int c = blockIdx.y * 256 + threadIdx.x;
  if (c >= p.H) return;
  const int j = blockIdx.x;
  const int t0 = j * p.block_t, t1 = min(t0 + p.block_t, p.L);
  float pole[16], res[16], s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    pole[i] = expf(p.lp[(int64_t)c * p.l0 + i * p.l1]);
    res[i] = PHASE == 3 ? p.res[(int64_t)c * p.r0 + i * p.r1] : 0.0f;
    s[i] = PHASE == 3 ? p.work[((int64_t)j * p.H + c) * 16 + i] : 0.0f;
  }
  const float *xr = p.x + (int64_t)c * p.xh;
  float *yr = p.y + (int64_t)c * p.yh;
#pragma unroll 4
  for (int t = t0; t < t1; ++t) {
    const float u = xr[(int64_t)t * p.xl];
    float ya = 0.f, yb = 0.f, yc = 0.f, yd = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = fmaf(pole[i], s[i], u);
      if (PHASE == 3) {
        if ((i & 3) == 0) ya = fmaf(res[i], s[i], ya);
        if ((i & 3) == 1) yb = fmaf(res[i], s[i], yb);
        if ((i & 3) == 2) yc = fmaf(res[i], s[i], yc);
        if ((i & 3) == 3) yd = fmaf(res[i], s[i], yd);
      }
    }
    if (PHASE == 3) yr[(int64_t)t * p.yl] = (ya + yb) + (yc + yd);
  }
  if (PHASE == 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) p.work[((int64_t)j * p.H + c) * 16 + i] = s[i];
  }
}

__global__ __launch_bounds__(256) void iir_carry_kernel(IirArgs p) {
  const int gi = blockIdx.x * 256 + threadIdx.x;
  const int c = gi >> 4, i = gi & 15;  // one lane per (channel, pole)
  if (c >= p.H) return;
  float S = p.sp ? p.sp[(int64_t)c * p.sp0 + i * p.sp1] : 0.0f;
  const float lpv = p.lp[(int64_t)c * p.l0 + i * p.l1];
  if (p.ntiles > 0) S = carry_chain(p.work, p.H, c, i, 0, p.ntiles, 0, p.block_t, p.L, lpv, S);
  p.st[(int64_t)c * 16 + i] = S;
}

// h[d, l] = sum_s residues[d, s] * exp(log_poles[d, s] * t[l])  (triton_hcl.py:46-74)
__global__ __launch_bounds__(256) void hcl_filter_kernel(const float *res, int64_t r0, int64_t r1,
                                                         const float *lp, int64_t l0, int64_t l1,
                                                         const float *t, int64_t st,
                                                         float *h, int64_t h0, int64_t h1,
                                                         int D, int S, int L) {
  const int l = blockIdx.x * 256 + threadIdx.x;
  const int d = blockIdx.y;
  if (l >= L) return;
  const float tv = t[(int64_t)l * st];
  float acc = 0.0f;
  for (int s = 0; s < S; ++s)
    acc = fmaf(res[(int64_t)d * r0 + s * r1], expf(lp[(int64_t)d * l0 + s * l1] * tv), acc);
  h[(int64_t)d * h0 + (int64_t)l * h1] = acc;
}

}  // namespace evo2

extern "C" int evo2_iir_segment(const float *seq, int64_t xh, int64_t xl,
                                const float *residues, int64_t r0, int64_t r1,
                                const float *log_poles, int64_t l0, int64_t l1,
                                const float *s_prev, int64_t sp0, int64_t sp1,
                                float *y, int64_t yh, int64_t yl, float *st,
                                float *workspace, int64_t workspace_bytes,
                                int64_t H, int64_t L, int32_t block_t, void *stream) {
  if (H <= 0 || L < 0 || block_t <= 0)
    return fail(EVO2_ERR_INVALID, "iir_segment: bad sizes H=%lld L=%lld block_t=%d",
                (long long)H, (long long)L, block_t);
  const int64_t ntiles = cdiv(L, block_t);
  if (!seq || !residues || !log_poles || !y || !st || (ntiles && !workspace))
    return fail(EVO2_ERR_INVALID, "iir_segment: null pointer argument");
  if (workspace_bytes < evo2_hcl_workspace_bytes(ntiles, H))
    return fail(EVO2_ERR_INVALID, "iir_segment: workspace too small");
  if (ntiles > 65535 || L > 0x7fffffff)
    return fail(EVO2_ERR_UNSUPPORTED, "iir_segment: L=%lld too long for block_t=%d",
                (long long)L, block_t);
  hipStream_t strm = static_cast<hipStream_t>(stream);
  IirArgs a{seq, xh, xl, residues, r0, r1, log_poles, l0, l1, s_prev, sp0, sp1, y, yh, yl, st,
            workspace, static_cast<int>(H), static_cast<int>(L), block_t,
            static_cast<int>(ntiles)};
  dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(cdiv(H, 256)));
  if (ntiles) {
    hipLaunchKernelGGL(iir_scan_kernel<1>, grid, dim3(256), 0, strm, a);
    int rc = check_launch("iir_segment phase 1");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(iir_carry_kernel, dim3(static_cast<unsigned>(cdiv(H, 16))), dim3(256), 0, strm, a);
  int rc = check_launch("iir_segment phase 2");
  if (rc) return rc;
  if (ntiles) {
    hipLaunchKernelGGL(iir_scan_kernel<3>, grid, dim3(256), 0, strm, a);
    rc = check_launch("iir_segment phase 3");
  }
  return rc;
}

extern "C" int evo2_iir_final_state(const float *seq, int64_t xh, int64_t xl,
                                    const float *log_poles, int64_t l0, int64_t l1, float *st,
                                    float *workspace, int64_t workspace_bytes,
                                    int64_t H, int64_t L, int32_t block_t, void *stream) {
  if (H <= 0 || L < 0 || block_t <= 0)
    return fail(EVO2_ERR_INVALID, "iir_final_state: bad sizes H=%lld L=%lld block_t=%d",
                (long long)H, (long long)L, block_t);
  const int64_t ntiles = cdiv(L, block_t);
  if (!seq || !log_poles || !st || (ntiles && !workspace))
    return fail(EVO2_ERR_INVALID, "iir_final_state: null pointer argument");
  if (workspace_bytes < evo2_hcl_workspace_bytes(ntiles, H))
    return fail(EVO2_ERR_INVALID, "iir_final_state: workspace too small");
  if (ntiles > 65535 || L > 0x7fffffff)
    return fail(EVO2_ERR_UNSUPPORTED, "iir_final_state: L=%lld too long for block_t=%d",
                (long long)L, block_t);
  hipStream_t strm = static_cast<hipStream_t>(stream);
  // the scan's first two phases: tile end states, then the carry whose
  // value after the last tile is the final state (no residues, no y)
  IirArgs a{seq, xh, xl, nullptr, 0, 0, log_poles, l0, l1, nullptr, 0, 0, nullptr, 0, 0, st,
            workspace, static_cast<int>(H), static_cast<int>(L), block_t,
            static_cast<int>(ntiles)};
  if (ntiles) {
    dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(cdiv(H, 256)));
    hipLaunchKernelGGL(iir_scan_kernel<1>, grid, dim3(256), 0, strm, a);
    int rc = check_launch("iir_final_state phase 1");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(iir_carry_kernel, dim3(static_cast<unsigned>(cdiv(H, 16))), dim3(256), 0, strm, a);
  return check_launch("iir_final_state phase 2");
}

extern "C" int evo2_hcl_compute_filter(const float *residues, int64_t r0, int64_t r1,
                                       const float *log_poles, int64_t l0, int64_t l1,
                                       const float *t, int64_t st, float *h, int64_t h0, int64_t h1,
                                       int64_t D, int64_t S, int64_t L, void *stream) {
  if (D <= 0 || S <= 0 || L < 0 || D > 65535)
    return fail(EVO2_ERR_INVALID, "hcl_compute_filter: bad sizes D=%lld S=%lld L=%lld",
                (long long)D, (long long)S, (long long)L);
  if (L == 0) return EVO2_OK;
  if (!residues || !log_poles || !t || !h)
    return fail(EVO2_ERR_INVALID, "hcl_compute_filter: null pointer argument");
  dim3 grid(static_cast<unsigned>(cdiv(L, 256)), static_cast<unsigned>(D));
  hipLaunchKernelGGL(hcl_filter_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     residues, r0, r1, log_poles, l0, l1, t, st, h, h0, h1,
                     static_cast<int>(D), static_cast<int>(S), static_cast<int>(L));
  return check_launch("hcl_compute_filter");
}
