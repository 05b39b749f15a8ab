// Causal self-attention of prompts for the whole-model harness on the matrix
// cores (head_dim 128): out[i] = sum_{j <= i} softmax_j(scale q_i . k_j) v_j
// per (sequence, head), as Evo2Attention computes it at prefill
// (model.py:104-153; the reference leaves the kernel to vLLM's flash
// attention).  Inputs in the harness's layouts: q, k and out (N, heads, L,
// 128) and the values transposed, vt (N, heads, 128, L), so that both
// products read 16 contiguous bytes per lane and no operand is transposed in
// registers.
//
// A workgroup takes 256 queries of one (sequence, head): eight waves of 32
// (two 16-query tiles, two waves a SIMD; the workgroups of one XCD take whole
// heads when the heads split evenly over the eight), and sweeps the key
// blocks of 128 keys at or before its last query; each block's keys (128 x
// 256 B) and values (128 dims x 256 B) come through LDS by direct-to-LDS
// loads, double-buffered, one barrier per block.  A wave takes a block in two
// halves of 64 keys, on v_mfma_f32_16x16x32_bf16:
//  * scores S^T = K Q^T: four 16-key tiles, tile t row m = key 4 m + t of
//    the half; lane (m, g) reads 16 bytes of that key (dims 32 kk + 8 g ..
//    + 7), Q's B operand the same dims of its query.  Lane (n, g) then holds
//    the scores of keys 16 g .. 16 g + 15 of the half for queries n and
//    16 + n;
//  * o^T += V^T P^T: dim tile e row m = dim 8 m + e; lane (m, g) reads 16
//    bytes of value row 8 m + e (keys 16 g + 8 kp .. + 7 of the half); the B
//    operand is the lane's own probabilities of those keys as bf16.
// Online softmax in fp32 with exp2 of scores kept in log2 units; a row's
// reference max moves (and its sums are rescaled) only when a half's max
// exceeds it by more than AP_SLACK, so the probabilities stay below
// 2^AP_SLACK and most halves rescale nothing.  The probabilities enter the
// value product rounded to bf16, as in flash attention, and the row sums are
// the same bf16 probabilities summed by one more product (an all-ones
// operand), so numerator and denominator use the same values.  LDS rows are
// 256 bytes; 16-byte chunk c of key row r sits at c ^ ((r >> 2) & 15), of
// value row r at c ^ ((r >> 3) & 15), which puts the 16 rows a read serves
// on distinct bank groups.
#include "attn_common.h"

namespace evo2 {

constexpr int AP_HD = 128;                 // head dim
constexpr int AP_NW = 8;                   // waves per workgroup (two per SIMD)
constexpr int AP_NQT = 2;                  // 16-query tiles per wave
constexpr int AP_QW = 16 * AP_NQT;         // queries per wave
constexpr int AP_QB = AP_NW * AP_QW;       // queries per workgroup
constexpr int AP_KB = 128;                 // keys per block
constexpr int AP_TILE = AP_KB * AP_HD;     // bf16 per staged operand block (32 KB)
constexpr float AP_SLACK = 8.0f;           // log2 headroom of the reference max

struct PrefillArgs {
  const bf16_t *q, *k, *vt;
  bf16_t *out;
  int64_t plane;   // elements per (sequence, head) plane: L * 128
  int L;
  int heads;
  int nqb;         // query blocks per plane
  float c2;        // scale * log2(e)
  int xcd_heads;   // 1-D grid, whole heads per XCD (heads a multiple of 8)
};

__global__ __launch_bounds__(AP_NW * 64, 1) void attn_prefill_kernel(PrefillArgs p) {
  __shared__ __align__(16) bf16_t ks0[AP_TILE], ks1[AP_TILE];  // keys (key rows)
  __shared__ __align__(16) bf16_t vs0[AP_TILE], vs1[AP_TILE];  // values (dim rows)
  int qb, h;
  if (p.xcd_heads) {
    // workgroup w runs on XCD w % 8; XCD x takes heads x, x + 8, .. in
    // turn, each head's query blocks longest first, so the workgroups on
    // one XCD sweep the same keys and values together through its L2
    const int w = static_cast<int>(blockIdx.x), j = w >> 3;
    const int hh = j / p.nqb;
    qb = p.nqb - 1 - (j - hh * p.nqb);
    h = (w & 7) + 8 * hh;
  } else {
    qb = p.nqb - 1 - static_cast<int>(blockIdx.x);  // longest sweeps first
    h = static_cast<int>(blockIdx.y);
  }
  const int64_t pl = static_cast<int64_t>(blockIdx.z) * p.heads + h;
  const bf16_t *q = p.q + pl * p.plane, *k = p.k + pl * p.plane, *vt = p.vt + pl * p.plane;
  bf16_t *out = p.out + pl * p.plane;
  const int L = p.L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int q0 = qb * AP_QB;
  const int wq0 = q0 + AP_QW * wave;  // this wave's first query
  // key blocks the workgroup needs: up to its last query, inside the prompt
  const int nkb = (min(q0 + AP_QB, L) + AP_KB - 1) / AP_KB;

  // Block b into a stage: 32 KB of keys and 32 KB of values, 32 wave loads
  // of 1 KB each; wave w issues loads 4 w .. 4 w + 3 of both.  Lane i of
  // load j fills LDS row r = 4 j + i / 16, position i % 16, which holds chunk
  // (i % 16) ^ ((r >> 2) & 15) of key row kb0 + r (keys) or chunk
  // (i % 16) ^ ((r >> 3) & 15), keys kb0 + 8 c .., of dim row r (values).
  // Buffer loads over the (sequence, head) plane: a lane's offset within the
  // block is fixed, the block's in an SGPR; key rows past the prompt read
  // zeros (past the plane), value chunks past it the next row's first keys
  // or zeros, finite values whose probabilities are 0.
  const uint32_t pbytes = static_cast<uint32_t>(p.plane * 2);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(k), 0, pbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(vt), 0, pbytes, 0x00020000);
  uint32_t koff[32 / AP_NW], voff[32 / AP_NW];
#pragma unroll
  for (int jj = 0; jj < 32 / AP_NW; ++jj) {
    const int j = (32 / AP_NW) * wave + jj;
    const int r = 4 * j + (lane >> 4);
    // byte offsets below 256 L < 2^32 (checked on the host), in 32 bits unsigned
    koff[jj] = (static_cast<uint32_t>(r) * AP_HD + 8u * ((lane & 15) ^ ((r >> 2) & 15))) * 2u;
    voff[jj] =
        (static_cast<uint32_t>(r) * static_cast<uint32_t>(L) + 8u * ((lane & 15) ^ ((r >> 3) & 15))) * 2u;
  }
  auto issue = [&](int b) __attribute__((always_inline)) {
    const int kb0 = b * AP_KB;
    bf16_t *kd = b & 1 ? ks1 : ks0;
    bf16_t *vd = b & 1 ? vs1 : vs0;
#pragma unroll
    for (int jj = 0; jj < 32 / AP_NW; ++jj) {
      const int j = (32 / AP_NW) * wave + jj;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (alds_void *)(kd + 512 * j), 16, koff[jj],
                                               static_cast<int>(static_cast<uint32_t>(kb0) * (AP_HD * 2u)), 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (alds_void *)(vd + 512 * j), 16, voff[jj],
                                               static_cast<int>(static_cast<uint32_t>(kb0) * 2u), 0, 0);
    }
  };

  // Q as the B operand: k-slot (g, j) of k-step kk is dim 32 kk + 8 g + j
  abf16x8_t qop[AP_HD / 32][AP_NQT];
#pragma unroll
  for (int nt = 0; nt < AP_NQT; ++nt) {
    const bf16_t *qr = q + static_cast<int64_t>(min(wq0 + 16 * nt + n, L - 1)) * AP_HD + 8 * g;
#pragma unroll
    for (int kk = 0; kk < AP_HD / 32; ++kk)
      qop[kk][nt] = __builtin_bit_cast(abf16x8_t, *reinterpret_cast<const au32x4_t *>(qr + 32 * kk));
  }

  float mrun[AP_NQT];
  af32x4_t acc[8][AP_NQT];  // o^T: dim tile e (dims 32 g + 8 i + e in lane (n, g)), query tile nt
  af32x4_t lacc[AP_NQT];    // the probability sums of query tile nt (every element)
#pragma unroll
  for (int nt = 0; nt < AP_NQT; ++nt) {
    mrun[nt] = -INFINITY;
    lacc[nt] = af32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e][nt] = af32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // an all-ones A operand: ones x P^T sums each query's probabilities over
  // the k-step into every row of its column
  abf16x8_t ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = static_cast<__bf16>(1.0f);

  // Block b from its stage, in two halves of 64 keys; whole: every key of
  // the block lies at or before every query of this wave, inside the prompt.
  auto block = [&](int b, bool whole) __attribute__((always_inline)) {
    const int kb0 = b * AP_KB;
    const uint32_t kd = lds_addr(b & 1 ? ks1 : ks0), vd = lds_addr(b & 1 ? vs1 : vs0);
    static_for<2>([&](auto half) __attribute__((always_inline)) {
      constexpr int H = decltype(half)::value;
      // scores of keys kb0 + 64 H + 4 m + t (tile t, row m): lane (m, g)
      // reads key rows 64 H + 4 m .. + 3 (stride 256 bytes) at position
      // chunk ^ m
      af32x4_t s[4][AP_NQT];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int nt = 0; nt < AP_NQT; ++nt) s[t][nt] = af32x4_t{0.f, 0.f, 0.f, 0.f};
      static_for<AP_HD / 32>([&](auto kk) __attribute__((always_inline)) {
        au32x4_t kv[4];
        lds_read4<256>(kv, kd + 16384 * H + 1024 * n + 16 * ((4 * decltype(kk)::value + g) ^ n));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const abf16x8_t a = __builtin_bit_cast(abf16x8_t, kv[t]);
#pragma unroll
          for (int nt = 0; nt < AP_NQT; ++nt)
            s[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[kk][nt], s[t][nt], 0, 0, 0);
        }
      });
      // s[t][nt][i]: key kb0 + 64 H + 16 g + 4 i + t, query wq0 + 16 nt + n;
      // live while its offset 4 i + t in the lane's 16 keys is at most lim
      // (the query, or the prompt's last key, relative to the lane's first).
      // The max is taken on raw scores (c2 > 0), the probability is
      // exp2(c2 s - m) with m in log2 units.
#pragma unroll
      for (int nt = 0; nt < AP_NQT; ++nt) {
        float bm = -INFINITY;
        if (!whole) {  // wave-uniform
          const int lim = min(wq0 + 16 * nt + n, L - 1) - (kb0 + 64 * H + 16 * g);
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (4 * i + t > lim) s[t][nt][i] = -INFINITY;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) bm = fmaxf(bm, s[t][nt][i]);
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        bm *= p.c2;
        // the reference max moves only past the slack (from -inf: at the
        // first live score)
        const bool move = bm > mrun[nt] + AP_SLACK;
        const float mn = move ? bm : mrun[nt];
        const float msub = mn == -INFINITY ? 0.0f : mn;  // all masked so far: every exp2 is 0
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) s[t][nt][i] = __builtin_amdgcn_exp2f(fmaf(s[t][nt][i], p.c2, -msub));
        if (__any(move)) {  // wave-uniform
          const float alpha = move ? __builtin_amdgcn_exp2f(mrun[nt] - msub) : 1.0f;
          lacc[nt] *= alpha;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e][nt] *= alpha;
        }
        mrun[nt] = mn;
      }
      // the probabilities as bf16 B operands: k-step kp, k-slot (g, j) = key
      // kb0 + 64 H + 16 g + 8 kp + j = tile j % 4's element 2 kp + j / 4
      abf16x8_t ph[2][AP_NQT];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp)
#pragma unroll
        for (int nt = 0; nt < AP_NQT; ++nt) {
          au32x4_t u;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int j0 = 2 * jj, j1 = 2 * jj + 1;
            u[jj] = pack_bf(s[j0 & 3][nt][2 * kp + (j0 >> 2)], s[j1 & 3][nt][2 * kp + (j1 >> 2)]);
          }
          ph[kp][nt] = __builtin_bit_cast(abf16x8_t, u);
        }
      // o^T += V^T P^T: dim tile e, row m = dim 8 m + e; lane (m, g) reads
      // keys 64 H + 16 g + 8 kp .. + 7 of value row 8 m + e (chunk
      // 8 H + 2 g + kp at position chunk ^ m)
      static_for<2>([&](auto kp) __attribute__((always_inline)) {
        constexpr int KP = decltype(kp)::value;
        au32x4_t vv[8];
        lds_read8<256>(vv, vd + 2048 * n + 16 * ((8 * H + 2 * g + KP) ^ n));
#pragma unroll
        for (int nt = 0; nt < AP_NQT; ++nt)
          lacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, ph[KP][nt], lacc[nt], 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const abf16x8_t a = __builtin_bit_cast(abf16x8_t, vv[e]);
#pragma unroll
          for (int nt = 0; nt < AP_NQT; ++nt)
            acc[e][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph[KP][nt], acc[e][nt], 0, 0, 0);
        }
      });
    });
  };

  // One barrier per block: every wave's loads of block b have landed (each
  // waits for its own, the only ones in flight), and every wave is done with
  // block b - 1, whose stage then takes block b + 1.
  issue(0);
  for (int b = 0; b < nkb; ++b) {
    vmcnt_wait<0>();
    __builtin_amdgcn_s_barrier();
    if (b + 1 < nkb) issue(b + 1);
    const int kb0 = b * AP_KB;
    if (kb0 > wq0 + AP_QW - 1) continue;  // wave-uniform: keys after all of this wave's queries
    block(b, kb0 + AP_KB - 1 <= wq0 && kb0 + AP_KB <= L);
  }

  // out = o / sum, rows of this wave's queries inside the prompt
#pragma unroll
  for (int nt = 0; nt < AP_NQT; ++nt) {
    const float l = lacc[nt][0];
    const int qi = wq0 + 16 * nt + n;
    if (qi >= L) continue;
    const float inv = 1.0f / l;  // every query attends to itself: l >= 1
    bf16_t *orow = out + static_cast<int64_t>(qi) * AP_HD + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint4 w;
      w.x = pack_bf(acc[0][nt][i] * inv, acc[1][nt][i] * inv);
      w.y = pack_bf(acc[2][nt][i] * inv, acc[3][nt][i] * inv);
      w.z = pack_bf(acc[4][nt][i] * inv, acc[5][nt][i] * inv);
      w.w = pack_bf(acc[6][nt][i] * inv, acc[7][nt][i] * inv);
      *reinterpret_cast<uint4 *>(orow + 8 * i) = w;
    }
  }
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_prefill_attention(const void *q, const void *k, const void *vt, void *out, int64_t N,
                                      int64_t heads, int64_t L, int64_t head_dim, float scale,
                                      void *stream) {
  // a (sequence, head) plane of 256 L bytes is addressed by 32-bit buffer offsets
  if (N < 0 || heads <= 0 || L < 0 || N > 65535 || heads > 65535 || L * 256 > int64_t(0xffffffff))
    return fail(EVO2_ERR_INVALID, "prefill_attention: bad sizes N=%lld heads=%lld L=%lld", (long long)N,
                (long long)heads, (long long)L);
  if (head_dim != AP_HD)
    return fail(EVO2_ERR_UNSUPPORTED, "prefill_attention: head_dim %lld (128 only)", (long long)head_dim);
  if (!(scale > 0.0f))
    return fail(EVO2_ERR_INVALID, "prefill_attention: scale %g (must be positive)", (double)scale);
  if (N == 0 || L == 0) return EVO2_OK;
  if (!q || !k || !vt || !out) return fail(EVO2_ERR_INVALID, "prefill_attention: null pointer argument");
  // 16-byte loads of eight values along L in the transposed values
  if (L % 8 || reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(k) % 16 ||
      reinterpret_cast<uintptr_t>(vt) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail(EVO2_ERR_UNSUPPORTED, "prefill_attention: L %% 8 or 16-byte alignment not met (L=%lld)",
                (long long)L);
  PrefillArgs a{static_cast<const bf16_t *>(q), static_cast<const bf16_t *>(k), static_cast<const bf16_t *>(vt),
                static_cast<bf16_t *>(out), L * AP_HD, static_cast<int>(L), static_cast<int>(heads),
                static_cast<int>(cdiv(L, AP_QB)), scale * 1.4426950408889634f, 0};
  // whole heads per XCD where the heads split evenly over the eight (32
  // heads x 32768: 9.96 -> 8.34 ms, 8192: 1.05 -> 0.70 ms, the same bits)
  a.xcd_heads = heads % 8 == 0 && static_cast<int64_t>(a.nqb) * heads <= 0x7fffffff;
  if (a.xcd_heads)
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(static_cast<unsigned>(a.nqb * heads), 1, static_cast<unsigned>(N)),
                       dim3(AP_NW * 64), 0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(attn_prefill_kernel,
                       dim3(static_cast<unsigned>(a.nqb), static_cast<unsigned>(heads), static_cast<unsigned>(N)),
                       dim3(AP_NW * 64), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("prefill_attention");
}
