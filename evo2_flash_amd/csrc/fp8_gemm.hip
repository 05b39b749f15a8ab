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
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace evo2 {

typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(4))) int i32x4;
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
  // the scales first, as scalar loads whose latency the K loop hides
  const float scale = p.sx_scale[0] * p.sw_scale[0];

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

// ---------------------------------------------------------------------------
// Persistent form of the same tile.  One workgroup per CU walks the output
// tiles t = blockIdx.x, blockIdx.x + gridDim.x, ..., and its global -> LDS
// pipeline runs straight across tile boundaries: the first slice of the next
// tile is already loading while the current one finishes and writes its
// epilogue, so a tile's start-up latency is paid once per workgroup rather
// than once per tile.
//
// K moves in slices of 128 bytes: each row's slice is one whole 128-byte
// line, so a direct-to-LDS instruction (64 lanes x 16 bytes = 8 rows) asks
// for 8 full lines.  Two stages of 32 KB of W and 32 KB of X; slice k + 2 is
// loaded into the stage of slice k as soon as every wave has read slice k,
// and a slice takes two v_mfma_f32_32x32x64_f8f6f4 sub-steps (64 bytes of K
// each), so a load has a whole slice of matrix work (~1.1 us) to land and
// the workgroup meets at one barrier per slice.  LDS rows are 128 bytes;
// 16-byte chunk c of row r sits at c ^ ((r >> 1) & 7), which spreads the 16
// rows a b128 read serves per cycle over all 64 banks.
//
// Tile order: workgroup b runs on XCD b mod 8, so with a grid of 256 the 32
// tiles an XCD runs at once are made one block of 4 W tiles x 8 X tiles,
// whose operands that XCD's L2 then serves 8 and 4 times over.  A round of
// 256 tiles covers 8 such blocks; when the block count is not a multiple of
// 8, the blocks left after the last whole round are handed out tile by tile
// in block order.
// The lane's index in its wave, computed afresh (two VALU instructions) where
// code off the hot loop needs it, rather than kept live across the loop in
// a VGPR the compiler would spill: a spill reload waits for every operand
// load in flight.  In an asm statement, so it is not hoisted and shared.
__device__ __forceinline__ int lane_now() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

constexpr int Q_BK = 128;               // bytes of K per slice
constexpr int Q_STAGE = G_BN * Q_BK;    // bytes per operand per stage
constexpr int Q_KALIGN = 2 * Q_BK;      // K granularity: whole slice pairs per tile

// The grouped order needs a grid of 256 and whole 4 x 8 blocks.
__host__ __device__ inline bool persist_grouped(int ncu, int tiles_n, int tiles_m) {
  return ncu == 256 && tiles_n % 4 == 0 && tiles_m % 8 == 0;
}

// Output tile (bn, bm) of the t-th tile in the persistent order, for
// 0 <= t < tiles_n * tiles_m; a bijection onto the tile grid.
__host__ __device__ inline void persist_tile(int t, int tiles_n, int tiles_m, bool grouped, int &bn,
                                             int &bm) {
  if (grouped) {
    const int nbn = tiles_n >> 2;
    const int whole = ((nbn * (tiles_m >> 3)) >> 3) << 8;  // tiles in whole rounds
    int blk, i;
    if (t < whole) {
      blk = (t >> 8) * 8 + (t & 7);  // round, XCD
      i = (t >> 3) & 31;             // slot within the block
    } else {
      blk = (whole >> 5) + ((t - whole) >> 5);
      i = (t - whole) & 31;
    }
    bn = (blk % nbn) * 4 + (i & 3);
    bm = (blk / nbn) * 8 + (i >> 2);
  } else {
    bn = t % tiles_n;
    bm = t / tiles_n;
  }
}

__global__ __launch_bounds__(256) void fp8_gemm_persist_kernel(GemmArgs p, int tiles_n, int tiles_m,
                                                               int grouped) {
  __shared__ __align__(16) uint8_t w0[Q_STAGE], w1[Q_STAGE];
  __shared__ __align__(16) uint8_t x0[Q_STAGE], x1[Q_STAGE];
  // The bias of even and odd tiles, loaded direct-to-LDS a whole tile ahead
  // of the epilogue that adds it (64 lanes x 16 bytes: the tile's 256
  // columns and the next 256, unused).  Reading it then never waits on the
  // memory pipe, where a load would also wait for the next tile's operand
  // loads and the stores before it.
  __shared__ __align__(16) bf16_t bias0[512], bias1[512];
  constexpr int DB = Q_STAGE / 4 / 1024;  // 1 KB DMA blocks per operand, wave and slice (8)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = (wave & 1) * 128;   // wave's W rows
  const int wm = (wave >> 1) * 128;  // wave's X rows
  const int total = tiles_n * tiles_m;
  const int KT = p.K / Q_BK;  // slices per tile, even
  int grid = static_cast<int>(gridDim.x);
  asm volatile("" : "+s"(grid));  // kept in an SGPR, not reloaded from the dispatch packet
  const int ntile = (total - static_cast<int>(blockIdx.x) + grid - 1) / grid;
  const int nsteps = ntile * KT;

  // Operands through buffer descriptors over the whole matrices (their byte
  // extents fit 32 bits, checked on the host).
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.w), 0, static_cast<int>((int64_t)(p.N - 1) * p.sw + p.K), 0x00020000);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.x), 0, static_cast<int>((int64_t)(p.M - 1) * p.sx + p.K), 0x00020000);
  // bias reads past column N return zero
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(p.bias), 0, 2 * p.N, 0x00020000);

  // DMA: one wave instruction fills 1 KB = 8 rows of 128 bytes; lane i writes
  // row i / 8, physical chunk i % 8, which holds logical chunk
  // (i % 8) ^ ((row >> 1) & 7).  Block j of a wave covers rows
  // 8 (DB wave + j) + i / 8, whose swizzle is ((i / 16) + 4 (j & 1)) & 7: two
  // lane offsets per operand (even and odd blocks, row within the block and
  // chunk), the block's row offset and the K offset in SGPRs.
  int lw[2], lx[2];
  {
    const int r = lane >> 3;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int chunk = ((lane & 7) ^ (((lane >> 4) + 4 * par) & 7)) << 4;
      lw[par] = r * static_cast<int>(p.sw) + chunk;
      lx[par] = r * static_cast<int>(p.sx) + chunk;
    }
  }
  int tw = 0, tx = 0;  // byte offsets of the wave's first DMA row in the tile being loaded
  auto dma_tile = [&](int j) __attribute__((always_inline)) {
    int bn, bm;
    persist_tile(static_cast<int>(blockIdx.x) + j * grid, tiles_n, tiles_m, grouped != 0, bn, bm);
    tw = (bn * G_BN + DB * 8 * wave) * static_cast<int>(p.sw);
    tx = (bm * G_BM + DB * 8 * wave) * static_cast<int>(p.sx);
  };
  auto stage_w = [&](auto stage) __attribute__((always_inline)) -> uint8_t * {
    return decltype(stage)::value ? w1 : w0;
  };
  auto stage_x = [&](auto stage) __attribute__((always_inline)) -> uint8_t * {
    return decltype(stage)::value ? x1 : x0;
  };
  // Slice q of this workgroup's sequence (tile q / KT, K slice q % KT) into
  // a stage; slices past the end re-read the last one, so every step issues
  // the same loads and the wait counts stay exact.
  int dma_t = 0;  // tile whose offsets tw / tx hold
  auto issue = [&](auto stage, int q) __attribute__((always_inline)) {
    q = min(q, nsteps - 1);
    const int tq = q / KT;  // uniform
    if (tq != dma_t) {
      dma_t = tq;
      dma_tile(tq);
    }
    const int koff = (q - tq * KT) * Q_BK;
    uint8_t *lwp = stage_w(stage);
    uint8_t *lxp = stage_x(stage);
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      const int blk = wave * DB + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void *)(lwp + blk * 1024), 16, lw[j & 1],
                                               tw + 8 * j * static_cast<int>(p.sw) + koff, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void *)(lxp + blk * 1024), 16, lx[j & 1],
                                               tx + 8 * j * static_cast<int>(p.sx) + koff, 0, 0);
    }
  };

  const int g = lane >> 5;   // lane group: k bytes [32g, 32g + 32) of a sub-step
  const int lr = lane & 31;  // row within a 32-row MFMA tile
  const int sw = (lr >> 1) & 7;  // swizzle of every row this lane reads
  // Fragments of sub-step h of a stage: row r = base + 32 t + lr, logical
  // chunks 4h + 2g and 4h + 2g + 1.
  auto read_frags = [&](auto stage, auto sub, i32x8 fa[4], i32x8 fb[4]) __attribute__((always_inline)) {
    constexpr int H = decltype(sub)::value;
    const uint8_t *lwp = stage_w(stage);
    const uint8_t *lxp = stage_x(stage);
    const int c0 = ((4 * H + 2 * g) ^ sw) << 4, c1 = ((4 * H + 2 * g + 1) ^ sw) << 4;
    // in the order the MFMAs consume them (tn-major: every X fragment and W
    // fragment 0 first)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint8_t *row = lxp + (wm + 32 * t + lr) * Q_BK;
      const uint4 b0 = *reinterpret_cast<const uint4 *>(row + c0);
      const uint4 b1 = *reinterpret_cast<const uint4 *>(row + c1);
      fb[t] = i32x8{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint8_t *row = lwp + (wn + 32 * t + lr) * Q_BK;
      const uint4 a0 = *reinterpret_cast<const uint4 *>(row + c0);
      const uint4 a1 = *reinterpret_cast<const uint4 *>(row + c1);
      fa[t] = i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
    }
  };

  // The accumulators of a tile start at its first MFMAs, which take C = 0
  // (no clearing between tiles), so they are not live across tiles.
  f32x16 acc[4][4];
  const f32x16 zero16 = {};
  auto mma = [&](const i32x8 fa[4], const i32x8 fb[4], auto first) __attribute__((always_inline)) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
        acc[tn][tm] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            fa[tn], fb[tm], decltype(first)::value ? zero16 : acc[tn][tm], 0, 0, 0, 0, 0, 0);
  };
  const float scale = p.sx_scale[0] * p.sw_scale[0];
  // Wave 0 loads the bias of tile j into the buffer of its parity.
  auto load_bias = [&](auto par, int j) __attribute__((always_inline)) {
    if (!p.bias || wave != 0) return;  // uniform
    int bn, bm;
    persist_tile(static_cast<int>(blockIdx.x) + j * grid, tiles_n, tiles_m, grouped != 0, bn, bm);
    bf16_t *lb = decltype(par)::value ? bias1 : bias0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (lds_void *)lb, 16, 16 * lane_now(), 2 * bn * G_BN,
                                             0, 0);
  };
  // Epilogue of tile j: lane holds, for X row m = m0 + wm + 32 tm + lr, the
  // W rows n = n0 + wn + 32 tn + 8 q + 4 g + i (i < 4) in acc[tn][tm][4 q + i].
  // Every store address is one of four row pointers plus a constant; a lane
  // issues EPI_STORES 16-byte stores (4 tm x 4 tn x 2 pairs).
  constexpr int EPI_STORES = 4 * 4 * 2;
  auto epilogue = [&](auto par, int j) __attribute__((always_inline)) {
    int bn, bm;
    persist_tile(static_cast<int>(blockIdx.x) + j * grid, tiles_n, tiles_m, grouped != 0, bn, bm);
    // The order is a bijection onto the grid (checked on the host for every
    // grid up to 64 x 40 tiles); a tile outside it stores nothing rather than
    // past the output (the operand loads are bounded by their descriptors).
    if (bn < 0 || bn >= tiles_n || bm < 0 || bm >= tiles_m) return;  // wave-uniform
    // whole tiles only (the host checks M and N are multiples of 256 and the
    // output rows 16-byte aligned)
    // Lanes l and l + 32 hold the same row: for each pair of column groups
    // (q, q + 1) they swap halves (v_permlane32_swap) so that lane l ends up
    // with columns 16 p .. 16 p + 7 and lane l + 32 with 16 p + 8 .. 16 p + 15,
    // and each stores 16 contiguous bytes: half as many store requests.
    const int ln = lane_now();
    const int elr = ln & 31, eg = ln >> 5;
    bf16_t *obase = p.out + (int64_t)(bm * G_BM + wm + elr) * p.so + bn * G_BN + wn + 8 * eg;
    const bf16_t *lb = (decltype(par)::value ? bias1 : bias0) + wn + 4 * eg;
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      bf16_t *orow = obase + (int64_t)(32 * tm) * p.so;
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        uint32_t pk[4][2];  // column group q, packed pairs
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = acc[tn][tm][4 * q + i] * scale;
          if (has_bias) {
            const uint2 bb = *reinterpret_cast<const uint2 *>(lb + 32 * tn + 8 * q);
            v[0] += lo_bf(bb.x);
            v[1] += hi_bf(bb.x);
            v[2] += lo_bf(bb.y);
            v[3] += hi_bf(bb.y);
          }
          pk[q][0] = pack_bf(v[0], v[1]);
          pk[q][1] = pack_bf(v[2], v[3]);
        }
#pragma unroll
        for (int pq = 0; pq < 2; ++pq) {
          // swap(x, y): lanes < 32 keep x and get x of lane + 32; lanes >= 32
          // get y of lane - 32 and keep y
          const auto s0 = __builtin_amdgcn_permlane32_swap(pk[2 * pq][0], pk[2 * pq + 1][0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(pk[2 * pq][1], pk[2 * pq + 1][1], false, false);
          *reinterpret_cast<uint4 *>(orow + 32 * tn + 16 * pq) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
        }
      }
    }
  };

  // Step k (slice k in stage S = k % 2):
  //   sub-step 0: MFMAs of (k, 0) from fragments read during step k - 1,
  //     while reading (k, 1);
  //   then every wave waits for its loads of slice k + 1 and its reads of
  //     slice k, and meets the others at the barrier: slice k + 1 is in LDS
  //     and nobody reads stage S again, which is refilled with slice k + 2;
  //   sub-step 1: MFMAs of (k, 1) while reading (k + 1, 0) from the other
  //     stage.
  // The first step after an epilogue also has the epilogue's EPI_STORES
  // stores outstanding (and, in wave 0, the next bias load after them), all
  // issued after the loads of slice k + 1: loads and stores retire in order,
  // so waiting until at most EPI_STORES remain covers the loads.
  i32x8 fa[2][4], fb[2][4];
  auto interleave = [&](bool dma) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if (dma) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    }
  };
  using std::integral_constant;
  using I0 = integral_constant<int, 0>;
  using I1 = integral_constant<int, 1>;
  using F0 = integral_constant<bool, false>;
  using F1 = integral_constant<bool, true>;
  // first: slice 0 of a tile, whose sub-step 0 starts the accumulators
  auto step = [&](auto stage, int k, bool after_epilogue, auto first) __attribute__((always_inline)) {
    constexpr int S = decltype(stage)::value;
    read_frags(stage, I1{}, fa[1], fb[1]);
    mma(fa[0], fb[0], first);
    interleave(false);
    if (after_epilogue) vmcnt_wait<EPI_STORES>();
    else vmcnt_wait<0>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(stage, k + 2);
    read_frags(integral_constant<int, S ^ 1>{}, I0{}, fa[0], fb[0]);
    mma(fa[1], fb[1], F0{});
    interleave(true);
  };

  using P0 = integral_constant<int, 0>;
  using P1 = integral_constant<int, 1>;
  load_bias(P0{}, 0);
  dma_tile(0);
  issue(I0{}, 0);
  issue(I1{}, 1);
  vmcnt_wait<2 * DB>();  // slice 0 (slice 1 in flight; the bias before them)
  __builtin_amdgcn_s_barrier();
  read_frags(I0{}, I0{}, fa[0], fb[0]);
  int s = 0;
  // Tile j of parity P: first the bias of tile j + 1 into the other buffer
  // (its previous contents, tile j - 1's, were added before this tile
  // began), then the slices in pairs (KT is even, so every tile starts in
  // stage 0; the first pair starts the accumulators), then the epilogue
  // with this buffer.
  auto tile = [&](auto par, int j) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    if (j + 1 < ntile) load_bias(integral_constant<int, P ^ 1>{}, j + 1);
    step(I0{}, s, j > 0, F1{});
    step(I1{}, s + 1, false, F0{});
    s += 2;
    for (int k = 2; k < KT; k += 2, s += 2) {
      step(I0{}, s, false, F0{});
      step(I1{}, s + 1, false, F0{});
    }
    epilogue(par, j);
  };
  for (int j = 0; j < ntile; j += 2) {
    tile(P0{}, j);
    if (j + 1 < ntile) tile(P1{}, j + 1);
  }
  // No direct-to-LDS write may still be landing when the workgroup's LDS is
  // handed to the next one.
  vmcnt_wait<0>();
}

// ---------------------------------------------------------------------------
// Decode-sized GEMMs (M <= 64 rows, e.g. the in_proj of a 64-sequence decode
// step, and, over blocks of 64 rows, verify-sized ones): the weight stream is
// the whole cost (N x K bytes against 64 x K of activations), so the kernel
// is built to keep HBM busy rather than the matrix pipe.  A workgroup owns
// 16 W rows per wave (two to four waves) and one block of up to 64 rows;
// v_mfma_f32_16x16x128_f8f6f4 with the weight as operand A.  Each wave
// streams its 16 W rows straight into VGPRs, S_DEPTH K steps (128 bytes)
// ahead; the activation slice of every step (64 rows x 128 bytes) goes
// through a ring of S_DEPTH LDS stages filled by direct-to-LDS loads and is
// shared by the waves.  Steps past the end of K re-read the last slice with
// a zero weight fragment, so every step issues the same loads and the wait
// counts stay exact.  LDS rows are 128 bytes; 16-byte chunk c of row r sits
// at c ^ ((r >> 1) & 7), which spreads the 16 rows a b128 read serves per
// cycle over all 64 banks.
constexpr int S_BK = 128;                 // bytes of K per step
constexpr int S_ROWS = 64;                // activation rows (max M)
constexpr int S_DEPTH = 8;                // steps in flight
constexpr int S_STAGE = S_ROWS * S_BK;    // 8 KB of activations per step
typedef __attribute__((ext_vector_type(4))) float f32x4;

// Workgroup -> (weight slice x, activation block y) for the weight-streaming
// kernel, over a 1-D grid of 8 * gy * ceil(gx / 8) workgroups: workgroup b
// runs on XCD b mod 8, so the gy blocks that read weight slice x are
// workgroups 8 (gy (x / 8) + y) + x mod 8 -- one XCD, back to back -- and the
// slice comes from HBM once, the other reads hitting that XCD's L2.  Padding
// workgroups (x >= gx) return at once.
__device__ __forceinline__ bool stream_tile(int gx, int gy, int &x, int &y) {
  const int L = blockIdx.x;
  const int j = L >> 3;
  y = j % gy;
  x = (j / gy) * 8 + (L & 7);
  return x < gx;
}

static inline dim3 stream_grid(int64_t gx, int64_t gy) {
  return dim3(static_cast<unsigned>(8 * gy * cdiv(gx, 8)));
}

// PACKED: the weight in the decode layout written by fp8_pack_kernel (each
// wave's 16 rows x 128 bytes of a K step are one contiguous 2 KB block, in
// the order the fragments are loaded), so the weight stream is sequential.
template <int WPG, bool PACKED>  // waves per workgroup (2, 3 or 4): 16 W rows each
__global__ __launch_bounds__(256) void fp8_gemm_small_kernel(GemmArgs p) {
  // one variable per stage: the compiler then sees which stage each
  // direct-to-LDS load writes and waits only for that stage's loads
  __shared__ __align__(16) uint8_t s0[S_STAGE], s1[S_STAGE], s2[S_STAGE], s3[S_STAGE];
  __shared__ __align__(16) uint8_t s4[S_STAGE], s5[S_STAGE], s6[S_STAGE], s7[S_STAGE];
  auto stage_of = [&](auto slot) __attribute__((always_inline)) -> uint8_t * {
    constexpr int J = decltype(slot)::value;
    static_assert(S_DEPTH == 8, "eight stage variables");
    return J == 0 ? s0 : J == 1 ? s1 : J == 2 ? s2 : J == 3 ? s3
         : J == 4 ? s4 : J == 5 ? s5 : J == 6 ? s6 : s7;
  };
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int bx, by;
  if (!stream_tile((p.N + 16 * WPG - 1) / (16 * WPG), (p.M + S_ROWS - 1) / S_ROWS, bx, by))
    return;  // uniform: grid padding
  // the scales before any load that writes LDS: read here the compiler makes
  // them scalar loads, whose latency passes under the K loop (read after it,
  // they were vector loads the epilogue waited for)
  const float scale = p.sx_scale[0] * p.sw_scale[0];
  const int n0 = bx * 16 * WPG;
  const int m0 = by * S_ROWS;  // 64-row block of the activations
  const int mrows = p.M - m0;          // >= 1 (the grid covers M exactly)
  const uint8_t *xbase = p.x + (int64_t)m0 * p.sx;
  const int g = lane >> 4;   // K bytes [32g, 32g + 32) of a step
  const int lr = lane & 15;  // row within a 16-row tile
  const int KT = p.K / S_BK;

  // activation DMA: the 8 blocks of a stage (1 KB = 8 rows each) are split
  // over the waves, block wave + WPG j for j < XB; with three waves the
  // last wave's third block repeats block 7 (the same bytes to the same
  // place), so every wave issues XB loads and the wait counts stay uniform
  constexpr int XB = (8 + WPG - 1) / WPG;
  auto xblock = [&](int j) __attribute__((always_inline)) { return min(wave + WPG * j, 7); };
  int xoff[XB];
#pragma unroll
  for (int j = 0; j < XB; ++j) {
    const int row = xblock(j) * 8 + lane / 8;
    const int lchunk = (lane & 7) ^ ((row >> 1) & 7);
    xoff[j] = min(row, mrows - 1) * (int)p.sx + 16 * lchunk;
  }
  // weight rows of this wave, straight into registers
  const uint8_t *wrow =
      PACKED ? p.w + (int64_t)min((n0 >> 4) + wave, (p.N >> 4) - 1) * KT * 2048 + 16 * lane
             : p.w + (int64_t)min(n0 + 16 * wave + lr, p.N - 1) * p.sw + 32 * g;
  i32x8 wf[S_DEPTH];
  auto issue = [&](auto slot, int k) __attribute__((always_inline)) {
    constexpr int J = decltype(slot)::value;
    const int k0 = min(k, KT - 1) * S_BK;
    // (a uint4 source pointer: given a byte pointer inside this kernel
    // template, the host pass drops the template's launch stub)
#pragma unroll
    for (int j = 0; j < XB; ++j)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(xbase + k0 + xoff[j]),
                                       (lds_void *)(stage_of(slot) + xblock(j) * 1024), 16,
                                       0, 0);
    // packed: the step's block, halves 1 KB apart, with the non-temporal
    // hint (a sequential stream read once: 3-5% faster; on the row-major
    // weight the hint cost 12%); else bytes [32 g, 32 g + 32) of the row
    if constexpr (PACKED) {
      const int64_t wo = min(k, KT - 1) * 2048;
      const i32x4 a0 = ld_nt(reinterpret_cast<const i32x4 *>(wrow + wo));
      const i32x4 a1 = ld_nt(reinterpret_cast<const i32x4 *>(wrow + wo + 1024));
      wf[J] = i32x8{a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    } else {
      const uint4 a0 = *reinterpret_cast<const uint4 *>(wrow + k0);
      const uint4 a1 = *reinterpret_cast<const uint4 *>(wrow + k0 + 16);
      wf[J] = i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
    }
  };
  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // activation fragments of step k from its stage (rows 16 t + lr)
  auto read_x = [&](auto slot, i32x8 (&xf)[4]) __attribute__((always_inline)) {
    const uint8_t *xst = stage_of(slot);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = 16 * t + lr;
      const int sw = (r >> 1) & 7;
      const uint4 b0 = *reinterpret_cast<const uint4 *>(xst + r * S_BK + (((2 * g) ^ sw) << 4));
      const uint4 b1 = *reinterpret_cast<const uint4 *>(xst + r * S_BK + (((2 * g + 1) ^ sw) << 4));
      xf[t] = i32x8{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                    (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    }
  };
  // Step k runs its MFMAs on fragments read during step k - 1 and meanwhile
  // reads step k + 1's: it first waits until this wave's loads for steps k
  // and k + 1 have landed (the XB + 2 loads of each of the S_DEPTH - 3 later
  // steps may still fly), then a barrier makes every wave's share of stage
  // k + 1 visible.  Stage k - 1, refilled with step k + S_DEPTH - 1, was last
  // read during step k - 2, before the previous barrier.
  i32x8 xa[4], xb[4];
  auto step = [&](auto slot, i32x8 (&cur)[4], i32x8 (&nxt)[4], int k) __attribute__((always_inline)) {
    constexpr int J = decltype(slot)::value;
    vmcnt_wait<(XB + 2) * (S_DEPTH - 3)>();
    __builtin_amdgcn_s_barrier();
    // a step past the end of K multiplies a zero weight fragment (its loads
    // re-read the last slice), so every step has the same straight-line shape
    const bool live = k < KT;  // uniform
    i32x8 w = wf[J];
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = live ? w[e] : 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, cur[t], acc[t], 0, 0, 0, 0, 0,
                                                                 0);
      // the accumulators stay in fixed AGPRs (otherwise the unrolled loop
      // renames them at every step and copies them around)
      asm volatile("" : "+a"(acc[t]));
    }
    issue(std::integral_constant<int, (J + S_DEPTH - 1) % S_DEPTH>{}, k + S_DEPTH - 1);
    read_x(std::integral_constant<int, (J + 1) % S_DEPTH>{}, nxt);
  };
  using std::integral_constant;
  issue(integral_constant<int, 0>{}, 0);
  issue(integral_constant<int, 1>{}, 1);
  issue(integral_constant<int, 2>{}, 2);
  issue(integral_constant<int, 3>{}, 3);
  issue(integral_constant<int, 4>{}, 4);
  issue(integral_constant<int, 5>{}, 5);
  issue(integral_constant<int, 6>{}, 6);
  vmcnt_wait<(XB + 2) * (S_DEPTH - 2)>();  // step 0 landed
  __builtin_amdgcn_s_barrier();
  read_x(integral_constant<int, 0>{}, xa);
  for (int k = 0; k < KT; k += S_DEPTH) {
    step(integral_constant<int, 0>{}, xa, xb, k);
    step(integral_constant<int, 1>{}, xb, xa, k + 1);
    step(integral_constant<int, 2>{}, xa, xb, k + 2);
    step(integral_constant<int, 3>{}, xb, xa, k + 3);
    step(integral_constant<int, 4>{}, xa, xb, k + 4);
    step(integral_constant<int, 5>{}, xb, xa, k + 5);
    step(integral_constant<int, 6>{}, xa, xb, k + 6);
    step(integral_constant<int, 7>{}, xb, xa, k + 7);
  }
  vmcnt_wait<0>();  // no DMA may still target this workgroup's LDS

  // lane holds out[m0 + 16 t + lr][n = n0 + 16 wave + 4 g + i] in acc[t][i]
  const int n = n0 + 16 * wave + 4 * g;  // (n0 + 16 * wave: this wave's W rows)
  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.bias) {
#pragma unroll
    for (int i = 0; i < 4; ++i) bias[i] = bf2f(p.bias[min(n + i, p.N - 1)]);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int m = 16 * t + lr;
    if (m >= mrows) continue;
    bf16_t *o = p.out + (int64_t)(m0 + m) * p.so + n;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = acc[t][i] * scale + bias[i];
    if (n + 4 <= p.N && (reinterpret_cast<uintptr_t>(o) & 7) == 0) {
      *reinterpret_cast<uint2 *>(o) = make_uint2(pack_bf(v[0], v[1]), pack_bf(v[2], v[3]));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < p.N) o[i] = f2bf(v[i]);
    }
  }
}

template <int WPG, bool PACKED>
static void launch_small(const GemmArgs &a, hipStream_t stream) {
  const dim3 grid = stream_grid(cdiv(a.N, 16 * WPG), cdiv(a.M, S_ROWS));
  hipLaunchKernelGGL((fp8_gemm_small_kernel<WPG, PACKED>), grid, dim3(64 * WPG), 0, stream, a);
}

// Decode weight layout: 16-row group G, K step k (128 bytes), half h, lane
// l = r + 16 q holds W[16 G + r][128 k + 32 q + 16 h .. + 16) at byte
// ((G * K / 128 + k) * 2 + h) * 1024 + 16 l.  One thread per 16 bytes.
__global__ __launch_bounds__(256) void fp8_pack_kernel(const uint8_t *w, int64_t sw, uint8_t *wp,
                                                       int64_t chunks, int KT) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int l = static_cast<int>(i & 63);
  const int64_t blk = i >> 6;  // (G * KT + k) * 2 + h
  const int h = static_cast<int>(blk & 1);
  const int64_t gk = blk >> 1;
  const int k = static_cast<int>(gk % KT);
  const int64_t G = gk / KT;
  const uint8_t *src = w + (16 * G + (l & 15)) * sw + 128 * k + 32 * (l >> 4) + 16 * h;
  *reinterpret_cast<uint4 *>(wp + 16 * i) = *reinterpret_cast<const uint4 *>(src);
}

// The weight-streaming kernel reads the weight once per 64-row block, so its
// cost grows with ceil(M / 64) x N x K, while up to one round of 256 x 256
// tiles costs one tile's K loop.  Measured with the weights streaming from
// HBM (K = 4096, us, stream / tiles): M=256, N=12288 42 / 62; M=512 75 / 62;
// M=512, N=4096 25 / 41; M=1024 48 / 43; M=256, N=24576, K=8192 138 / 115.
// Streaming takes ceil(M / 64) x N up to this; M <= 64 always streams.
#ifndef STREAM_MAX_WORK
#define STREAM_MAX_WORK 60000
#endif

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

// The same for rows of whole 16-element chunks with 16-byte aligned rows:
// a thread converts 16 values (two 16-byte loads, one 16-byte store), the
// grid strides over the (rows x K / 16) chunks.
__global__ __launch_bounds__(256) void fp8_quantize16_kernel(const bf16_t *x, int64_t sx,
                                                             uint8_t *q, int64_t sq,
                                                             const float *scale, int64_t chunks,
                                                             int cpr) {
  const float s = scale[0];
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks;
       c += (int64_t)gridDim.x * 256) {
    const int64_t r = c / cpr;
    const int k = static_cast<int>(c - r * cpr) * 16;
    const uint4 *xp = reinterpret_cast<const uint4 *>(x + r * sx + k);
    const uint4 a = xp[0], b = xp[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    int out[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4] = {lo_bf(w[2 * j]), hi_bf(w[2 * j]), lo_bf(w[2 * j + 1]), hi_bf(w[2 * j + 1])};
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = fminf(fmaxf(v[i] / s, -448.0f), 448.0f);
      int packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
      out[j] = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], packed, true);
    }
    *reinterpret_cast<int4 *>(q + r * sq + k) = make_int4(out[0], out[1], out[2], out[3]);
  }
}

}  // namespace evo2

using namespace evo2;

// Compute units of the current device (0 if the query fails), cached per
// device ordinal.
static int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

// The weight-streaming kernel with the waves per workgroup (16 W rows each)
// whose workgroups fill the CUs most evenly (groups / (rounds x CUs)), the
// larger on a tie.  Measured with the weights streaming from HBM (9 rotating
// weights, more than the 256 MB infinity cache holds), K = 4096: the 7B
// decode in_proj (M=64, N=12288) 17.1 us with 3 waves against 18.9 with 4 and
// 21.8 with 2; at M = 128 / 192 / 256 / 512, N = 12288: 25.9 / 37.1 / 42.0 /
// 75.8 us, the fastest of this kernel and of workgroups covering 2-4 row
// blocks per weight load (which only won while the weights stayed
// cache-resident).
template <bool PACKED>
static void launch_stream(const GemmArgs &a, hipStream_t st) {
  const int ncu = cu_count() > 0 ? cu_count() : 256;
  const int64_t yblocks = cdiv(a.M, S_ROWS);
  int best_w = 4;
  double best_eff = -1.0;
  for (int w = 4; w >= 2; --w) {
    const int64_t groups = cdiv(a.N, 16 * w) * yblocks;
    const double eff = double(groups) / double(cdiv(groups, ncu) * ncu);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best_w = w;
    }
  }
  if (best_w == 4) launch_small<4, PACKED>(a, st);
  else if (best_w == 3) launch_small<3, PACKED>(a, st);
  else launch_small<2, PACKED>(a, st);
}

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
  if (K % 16 == 0 && sx % 8 == 0 && sq % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(q) % 16 == 0) {
    const int64_t chunks = rows * (K / 16);
    const int64_t blocks = std::min<int64_t>(cdiv(chunks, 256), 8192);
    hipLaunchKernelGGL(fp8_quantize16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const bf16_t *>(x), sx,
                       static_cast<uint8_t *>(q), sq, scale, chunks, static_cast<int>(K / 16));
    return check_launch("fp8_quantize");
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K % S_BK == 0 && sx * S_ROWS < (int64_t(1) << 31) &&
      (M <= S_ROWS || cdiv(M, S_ROWS) * N <= STREAM_MAX_WORK)) {
    // the weight-streaming kernel over ceil(M / 64) blocks of 64 rows
    launch_stream<false>(a, st);
    return check_launch("fp8_gemm");
  }
  const int64_t tiles_n = cdiv(N, G_BN), tiles_m = cdiv(M, G_BM);
  const int ncu = cu_count();
  // the persistent form once every CU has a tile; its ring needs K to be a
  // multiple of four K steps and the operands to fit 32-bit buffer offsets
  if (ncu > 0 && tiles_n * tiles_m >= ncu && K % Q_KALIGN == 0 &&
      M % G_BM == 0 && N % G_BN == 0 && so % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
      (!bias || reinterpret_cast<uintptr_t>(bias) % 8 == 0) &&
      (N - 1) * sw + K < (int64_t(1) << 31) && (M - 1) * sx + K < (int64_t(1) << 31)) {
    const int grouped = persist_grouped(ncu, static_cast<int>(tiles_n), static_cast<int>(tiles_m));
    hipLaunchKernelGGL(fp8_gemm_persist_kernel, dim3(static_cast<unsigned>(ncu)), dim3(256), 0, st, a,
                       static_cast<int>(tiles_n), static_cast<int>(tiles_m), grouped);
    return check_launch("fp8_gemm");
  }
  dim3 grid(static_cast<unsigned>(tiles_n), static_cast<unsigned>(tiles_m));
  hipLaunchKernelGGL(fp8_gemm_kernel, grid, dim3(256), 0, st, a);
  return check_launch("fp8_gemm");
}

extern "C" int evo2_fp8_pack_weight(const void *w8, int64_t sw, void *wp, int64_t N, int64_t K,
                                    void *stream) {
  if (N <= 0 || K <= 0 || N % 16 || K % S_BK)
    return fail(EVO2_ERR_UNSUPPORTED,
                "fp8_pack_weight: N=%lld must be a multiple of 16 and K=%lld of %d", (long long)N,
                (long long)K, S_BK);
  if (!w8 || !wp) return fail(EVO2_ERR_INVALID, "fp8_pack_weight: null pointer argument");
  if (sw < K || sw % 16 || reinterpret_cast<uintptr_t>(w8) % 16 ||
      reinterpret_cast<uintptr_t>(wp) % 16)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_pack_weight: rows must be 16-byte aligned");
  const int64_t chunks = N * K / 16;
  if (cdiv(chunks, 256) > 0x7fffffff) return fail(EVO2_ERR_UNSUPPORTED, "fp8_pack_weight: too large");
  hipLaunchKernelGGL(fp8_pack_kernel, dim3(static_cast<unsigned>(cdiv(chunks, 256))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t *>(w8), sw,
                     static_cast<uint8_t *>(wp), chunks, static_cast<int>(K / S_BK));
  return check_launch("fp8_pack_weight");
}

extern "C" int evo2_fp8_gemm_packed(const void *x8, int64_t sx, const void *wp,
                                    const float *x_scale, const float *w_scale, const void *bias,
                                    void *out, int64_t so, int64_t M, int64_t N, int64_t K,
                                    void *stream) {
  if (M < 0 || N <= 0 || K <= 0)
    return fail(EVO2_ERR_INVALID, "fp8_gemm_packed: bad sizes M=%lld N=%lld K=%lld", (long long)M,
                (long long)N, (long long)K);
  if (M == 0) return EVO2_OK;
  if (!x8 || !wp || !x_scale || !w_scale || !out)
    return fail(EVO2_ERR_INVALID, "fp8_gemm_packed: null pointer argument");
  if (N % 16 || K % S_BK)
    return fail(EVO2_ERR_UNSUPPORTED,
                "fp8_gemm_packed: N=%lld must be a multiple of 16 and K=%lld of %d", (long long)N,
                (long long)K, S_BK);
  if (sx % 16 || reinterpret_cast<uintptr_t>(x8) % 16 || reinterpret_cast<uintptr_t>(wp) % 16)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_gemm_packed: operands must be 16-byte aligned");
  if (sx * S_ROWS >= (int64_t(1) << 31) || cdiv(M, S_ROWS) * cdiv(N, 32) * 8 > 0x7fffffff ||
      N > 0x7fffffff)
    return fail(EVO2_ERR_UNSUPPORTED, "fp8_gemm_packed: problem too large");
  GemmArgs a{static_cast<const uint8_t *>(x8), sx, static_cast<const uint8_t *>(wp), K, x_scale,
             w_scale, static_cast<const bf16_t *>(bias), static_cast<bf16_t *>(out), so,
             static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)};
  launch_stream<true>(a, static_cast<hipStream_t>(stream));
  return check_launch("fp8_gemm_packed");
}

extern "C" int64_t evo2_fp8_gemm_persist_order(int64_t tiles_n, int64_t tiles_m, int ncu, int32_t *bn,
                                               int32_t *bm) {
  if (tiles_n <= 0 || tiles_m <= 0 || ncu <= 0 || tiles_n * tiles_m > 0x7fffffff) return -1;
  const int tn = static_cast<int>(tiles_n), tm = static_cast<int>(tiles_m);
  const bool grouped = persist_grouped(ncu, tn, tm);
  const int total = tn * tm;
  if (bn && bm) {
    for (int t = 0; t < total; ++t) {
      int n, m;
      persist_tile(t, tn, tm, grouped, n, m);
      bn[t] = n;
      bm[t] = m;
    }
  }
  return grouped ? 1 : 0;
}
