// Decode attention for the whole-model harness: one query token per
// (sequence, head) against that head's KV cache, as Evo2Attention computes it
// at decode (model.py:104-153), with the cache laid out for one-pass
// streaming, either contiguous per sequence
//
//   keys   (B, heads, head_dim, L)  head_dim-major: position is the unit stride
//   values (B, heads, L, head_dim)  position-major: dim is the unit stride
//
// or in 16-position pages named by a per-sequence block table (the paged
// cache of the serving engine), page = table[b, l / 16]:
//
//   key pages   (pages, heads, head_dim, 16)
//   value pages (pages, heads, 16, head_dim)
//
//   out[b, h] = sum_l softmax_l(scale * q . k_l) v_l  over l <= positions[b]
//
// A table entry outside [0, num_pages) is never dereferenced: the positions
// it would hold are left out of the softmax (a sequence with none left gets
// zeros), so a stale or garbage entry gives a wrong row, not a fault.
//
// Split over the context (flash decoding): a workgroup takes the 2048
// positions of one chunk c for head h and writes (o, max, sum) to a
// workspace; a second launch merges the chunks of each (sequence, head).
// Keys and values are each read once; everything is fp32 until the bf16
// output.  Two chunk kernels:
//  * the VALU kernel (contiguous cache, and paged at head_dim 64): workgroup
//    (c, h, b) computes its scores with 16-byte loads of eight consecutive
//    positions per lane (q in LDS), the chunk's max and exp-sum with a block
//    reduction, then sum_l p_l v_l with 16-byte loads of eight dims per lane
//    (6.2 TB/s at 64 sequences x 32 heads x 8704 positions, contiguous);
//  * the matrix-core kernel (paged, head_dim 128; below): one sequence per
//    workgroup, or 32 on chunks whose pages the caller declares shared by
//    every sequence (a prompt behind all of them), each key and value byte
//    then read once for all 32.
// The workgroups of one (chunk, head) pair are dispatched back to back on
// one XCD, so pages that several workgroups of a pair read stream from HBM
// once per pair and from L2 for the rest.  At head_dim 64 declared shared
// chunks take four sequences per VALU workgroup, each load serving all four
// (the same bits as one per workgroup).
#include "attn_common.h"

namespace evo2 {

constexpr int AT_T = 256;              // threads per workgroup
constexpr int AT_CHUNK = 8 * AT_T;     // positions per chunk (eight per lane)
constexpr int AT_PAGE = 16;            // positions per page of the paged cache

struct AttnArgs {
  const bf16_t *q; int64_t qb, qh;           // (B, heads, hd), dim stride 1
  const bf16_t *k; int64_t kb, kh, kd;       // (B, heads, hd, L) or (pages, heads, hd, 16);
                                             // position stride 1 (kb: sequence or page)
  const bf16_t *v; int64_t vb, vh, vl;       // (B, heads, L, hd) or (pages, heads, 16, hd);
                                             // dim stride 1 (vb: sequence or page)
  const int32_t *tbl; int64_t tbs;           // paged: (B, L / 16) block table, row stride
  int64_t num_pages;                         // paged: entries outside [0, num_pages) masked
  const int64_t *pos;                        // (B,) this step's position; length pos + 1
  float *part;                               // (B, heads, nchunk, hd + 2): o, max, sum
  bf16_t *out; int64_t ob, oh;               // (B, heads, hd), dim stride 1
  float scale;
  int heads, L, nchunk;
  int B;
  int pair_major;  // 1-D pair-major grid (below) or the (chunk, head, sequence) grid
};

__device__ __forceinline__ int valid_len(const AttnArgs &p, int b) {
  const int64_t n = p.pos[b] + 1;
  return static_cast<int>(n < 0 ? 0 : (n > p.L ? p.L : n));
}

// The (chunk c, head h, first sequence b0) of this workgroup, false for the
// padding of the pair-major grid.  Pair-major: (chunk, head) pair P and
// sequence group j % G; the G workgroups of a pair run back to back on one
// XCD (workgroup w runs on XCD w mod 8), so where sequences share pages (one
// prompt behind many sequences) the pair's keys and values come from HBM
// once and from that XCD's L2 for the rest.  Otherwise the grid is (chunk,
// head, sequence group).
__device__ __forceinline__ bool chunk_of(const AttnArgs &p, int nq, int c_first, int c_count, int &c,
                                         int &h, int &b0) {
  const int G = (p.B + nq - 1) / nq;  // sequence groups
  if (p.pair_major) {
    const int w = blockIdx.x;
    const int j = w >> 3;
    const int P = (j / G) * 8 + (w & 7);
    if (P >= c_count * p.heads) return false;
    b0 = (j % G) * nq;
    c = c_first + P % c_count;
    h = P / c_count;
  } else {
    c = c_first + blockIdx.x;
    h = blockIdx.y;
    b0 = blockIdx.z * nq;
  }
  return true;
}

// Chunks c_first .. c_first + c_count - 1 of NQ sequences b0 .. b0 + NQ - 1
// (those below B) and one head per workgroup.  With NQ > 1 (paged cache only)
// the sequences read the pages of row b0: the caller passes NQ > 1 only for
// chunks whose pages every sequence shares, and each key and value load then
// serves NQ queries.  Every query's arithmetic (score sums over d in order,
// the block reductions, the value sums over l in order) is the NQ = 1
// kernel's, so a chunk's partials do not depend on NQ.
template <int HD, bool PAGED, int NQ>
__global__ __launch_bounds__(AT_T) void attn_chunk_kernel(AttnArgs p, int c_first, int c_count) {
  static_assert(NQ == 1 || PAGED, "shared chunks are a paged-cache case");
  __shared__ float qs[NQ][HD];
  __shared__ float ps[NQ][AT_CHUNK];
  __shared__ float red[NQ][AT_T / 64];
  __shared__ float osum[NQ][AT_T / 64][HD];
  __shared__ int32_t pages[PAGED ? AT_CHUNK / AT_PAGE : 1];
  int c, h, b0;
  if (!chunk_of(p, NQ, c_first, c_count, c, h, b0)) return;  // uniform: padding
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l0 = c * AT_CHUNK;
  int l1[NQ];
  int l1max = l0;
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    l1[qi] = b0 + qi < p.B ? min(l0 + AT_CHUNK, valid_len(p, b0 + qi)) : l0;
    l1max = max(l1max, l1[qi]);
  }
  auto part_of = [&](int qi) -> float * {
    return p.part + (((int64_t)(b0 + qi) * p.heads + h) * p.nchunk + c) * (HD + 2);
  };
  if (l0 >= l1max) {  // uniform: an empty chunk contributes nothing
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      if (b0 + qi >= p.B) break;
      float *part = part_of(qi);
      if (t < HD) part[t] = 0.0f;
      if (t == 0) {
        part[HD] = -INFINITY;
        part[HD + 1] = 0.0f;
      }
    }
    return;
  }
  for (int i = t; i < NQ * HD; i += AT_T) {
    const int qi = i / HD, d = i - HD * qi;
    qs[qi][d] = b0 + qi < p.B ? bf2f(p.q[(int64_t)(b0 + qi) * p.qb + (int64_t)h * p.qh + d]) : 0.0f;
  }
  if constexpr (PAGED) {  // the chunk's pages that hold positions below l1max
    if (t < AT_CHUNK / AT_PAGE && l0 + AT_PAGE * t < l1max) {
      const int32_t pg = p.tbl[(int64_t)b0 * p.tbs + l0 / AT_PAGE + t];
      pages[t] = pg >= 0 && pg < p.num_pages ? pg : -1;  // -1: masked
    }
  }
  __syncthreads();

  // scores of positions l0 + 8t .. l0 + 8t + 7 (L % 8 == 0 keeps a group that
  // starts below l1 inside the cache; in the paged cache the eight lie in
  // one page)
  const int lb = l0 + 8 * t;
  const bool live = lb < l1max && (!PAGED || pages[(lb - l0) / AT_PAGE] >= 0);
  float s[NQ][8];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi)
#pragma unroll
    for (int e = 0; e < 8; ++e) s[qi][e] = 0.0f;
  if (live) {
    const bf16_t *kr =
        PAGED ? p.k + (int64_t)pages[(lb - l0) / AT_PAGE] * p.kb + (int64_t)h * p.kh + lb % AT_PAGE
              : p.k + (int64_t)b0 * p.kb + (int64_t)h * p.kh + lb;
#pragma unroll 8
    for (int d = 0; d < HD; ++d) {
      const uint4 kv = *reinterpret_cast<const uint4 *>(kr + (int64_t)d * p.kd);
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        const float qd = qs[qi][d];
        s[qi][0] += qd * lo_bf(kv.x); s[qi][1] += qd * hi_bf(kv.x);
        s[qi][2] += qd * lo_bf(kv.y); s[qi][3] += qd * hi_bf(kv.y);
        s[qi][4] += qd * lo_bf(kv.z); s[qi][5] += qd * hi_bf(kv.z);
        s[qi][6] += qd * lo_bf(kv.w); s[qi][7] += qd * hi_bf(kv.w);
      }
    }
  }
  float mx[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    mx[qi] = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[qi][e] = live && lb + e < l1[qi] ? s[qi][e] * p.scale : -INFINITY;
      mx[qi] = fmaxf(mx[qi], s[qi][e]);
    }
    for (int o = 32; o > 0; o >>= 1) mx[qi] = fmaxf(mx[qi], __shfl_xor(mx[qi], o));
    if (lane == 0) red[qi][wave] = mx[qi];
  }
  __syncthreads();
  float sum[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    mx[qi] = red[qi][0];
#pragma unroll
    for (int w = 1; w < AT_T / 64; ++w) mx[qi] = fmaxf(mx[qi], red[qi][w]);  // -inf only if all masked
    sum[qi] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pe = live && lb + e < l1[qi] ? expf(s[qi][e] - mx[qi]) : 0.0f;
      ps[qi][8 * t + e] = pe;
      sum[qi] += pe;
    }
    for (int o = 32; o > 0; o >>= 1) sum[qi] += __shfl_xor(sum[qi], o);
  }
  __syncthreads();  // ps complete; every wave has read red
  if (lane == 0) {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) red[qi][wave] = sum[qi];
  }

  // o[d] = sum_l p_l v[l][d]: 16-byte loads of eight dims; a wave covers
  // RW = 64 / (HD / 8) rows per instruction (lane = row group r, dim block
  // g), waves interleave their row blocks; lanes of one dim block are summed
  // with shuffles, then the waves through LDS.
  constexpr int GPR = HD / 8;         // lanes per row
  constexpr int RW = 64 / GPR;        // rows per wave instruction
  const int r = lane / GPR, g = lane % GPR;
  float o[NQ][8];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[qi][e] = 0.0f;
  {
    const bf16_t *vr = p.v + (PAGED ? 0 : (int64_t)b0 * p.vb) + (int64_t)h * p.vh + 8 * g;
    for (int l = l0 + wave * RW + r; l < l1max; l += (AT_T / 64) * RW) {
      const int pg = PAGED ? pages[(l - l0) / AT_PAGE] : 0;
      if (PAGED && pg < 0) continue;  // masked page: weight 0, never read
      const bf16_t *row = PAGED ? vr + (int64_t)pg * p.vb + (int64_t)(l % AT_PAGE) * p.vl
                                : vr + (int64_t)l * p.vl;
      const uint4 vv = *reinterpret_cast<const uint4 *>(row);
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        if (NQ > 1 && l >= l1[qi]) continue;  // past this query's positions
        const float pl = ps[qi][l - l0];
        o[qi][0] += pl * lo_bf(vv.x); o[qi][1] += pl * hi_bf(vv.x);
        o[qi][2] += pl * lo_bf(vv.y); o[qi][3] += pl * hi_bf(vv.y);
        o[qi][4] += pl * lo_bf(vv.z); o[qi][5] += pl * hi_bf(vv.z);
        o[qi][6] += pl * lo_bf(vv.w); o[qi][7] += pl * hi_bf(vv.w);
      }
    }
  }
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int sh = GPR; sh < 64; sh <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[qi][e] += __shfl_xor(o[qi][e], sh);
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) osum[qi][wave][8 * g + e] = o[qi][e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    if (b0 + qi >= p.B) break;
    float *part = part_of(qi);
    if (t < HD) {
      float ov = osum[qi][0][t];
#pragma unroll
      for (int w = 1; w < AT_T / 64; ++w) ov += osum[qi][w][t];
      part[t] = ov;
    }
    if (t == 0) {
      float tot = red[qi][0];
#pragma unroll
      for (int w = 1; w < AT_T / 64; ++w) tot += red[qi][w];
      part[HD] = mx[qi];
      part[HD + 1] = tot;
    }
  }
}

// Paged chunks on the matrix cores (head_dim 128): one workgroup per (chunk,
// head) and group of gq sequences whose pages are those of row b0: 32
// sequences in two 16-sequence tiles for chunks every sequence shares (the
// caller passes only such chunks), one sequence in one tile for the rest
// (fifteen idle query slots: the launch is bound by its loads, not by the
// matrix cores).  Each wave takes the 128-position blocks w, w + 4, .. of the
// chunk with a running max and sum (online softmax), on
// v_mfma_f32_16x16x32_bf16:
//  * scores S^T = K Q^T: eight 16-row tiles, tile t row m = position 8 m + t
//    of the block, so lane (m, g) loads 16 bytes (positions 8 m .. 8 m + 7)
//    of one key dim at a time; eight such loads (dims 32 kk + 4 j + g, j =
//    0..7: four neighbouring dims per page line) transposed in registers
//    give the A operands of all eight tiles for k-step kk, and Q's B operand
//    takes the same dims.  Lane (n, g) then holds the scores of positions
//    32 g .. 32 g + 31 for query slots n and 16 + n;
//  * o^T = V^T P^T: dim tile e row m = dim 8 m + e; lane (m, g) loads eight
//    16-byte value rows (positions 32 g + 8 kp + j, dims 8 m .. + 7) and
//    transposes them the same way; the B operand is the lane's own
//    probabilities of those positions, split into bf16 high and low parts
//    (~16 bits), so no lane exchanges data except for the max and sum.
// Products of bf16 are exact and sums fp32, as in the VALU kernel; the order
// of the sums differs, and the probabilities are exp2 of scores kept in log2
// units.  The four waves' (max, sum, o) meet in LDS for the chunk's partials.
// The key and value rows reach the lanes through a per-wave queue of
// direct-to-LDS loads (four 8 KB groups in flight, no registers held), read
// back with each lane's own 16 bytes, so the sweep streams while the matrix
// cores and the softmax work.  Blocks that every sequence attends to in full
// skip the masks.  Measured on one MI355X: the 40B shape's shared prompt (32
// sequences, 64 heads, 131072 positions: 4.3 GB of keys and values per layer)
// ~0.86 ms per launch (the four-sequence VALU kernel 5.4 ms); 64 sequences of
// 32 heads with 8700 positions of their own (8.6 GB) 1.36 ms against 1.66 ms
// on the VALU kernel (6.7 TB/s).  Pages that many sequences share without
// the caller declaring them stream from L2 once per sequence and cost the
// one-tile form its arithmetic: 32 sequences on one 131072-position prompt
// take 10.6 ms there against 7.9 ms on the VALU kernel.
constexpr int AS_NQ = 32;   // sequences per workgroup
constexpr int AS_BLK = 128; // positions per wave block

// Element t of the eight 16-byte rows r[0..7] (row j holds elements 0..7 in
// order) as one operand: (r[0][t], .., r[7][t]).
template <int T>
__device__ __forceinline__ abf16x8_t column8(const au32x4_t (&r)[8]) {
  au32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = r[2 * i][T / 2], b = r[2 * i + 1][T / 2];
    o[i] = T & 1 ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
  }
  return __builtin_bit_cast(abf16x8_t, o);
}

template <int CPOL, int NQT>
__global__ __launch_bounds__(AT_T, 1) void attn_mfma_kernel(AttnArgs p, int c_first, int c_count, int gq) {
  static_assert(NQT == 1 || NQT == 2, "one or two 16-sequence tiles");
  constexpr int HD = 128;
  constexpr int NW = AT_T / 64;
  __shared__ int32_t pages[AT_CHUNK / AT_PAGE];
  __shared__ float wm[NW][AS_NQ], wl[NW][AS_NQ];
  __shared__ int whole[AT_CHUNK / AS_BLK];  // block needs no masks
  // Per wave, four 8 KB slots of a load queue (one group of eight 1 KB
  // direct-to-LDS loads each); after the sweep slots 0 and 1 hold the
  // wave's o for sequences 0..15 and 16..31.  Separate arrays, so the
  // compiler's wait for a slot's loads counts only that slot's.
  __shared__ float ring0[NW][2048], ring1[NW][2048], ring2[NW][2048], ring3[NW][2048];
  int c, h, b0;
  if (!chunk_of(p, gq, c_first, c_count, c, h, b0)) return;  // uniform: padding
  // query slot qi holds sequence b0 + qi if qi < gq and b0 + qi < B
  auto live = [&](int qi) { return qi < gq && b0 + qi < p.B; };
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int l0 = c * AT_CHUNK;
  int l1max = l0;             // end of the positions any sequence of the group attends to
  int l1min = l0 + AT_CHUNK;  // end of those every sequence attends to
  for (int qi = 0; live(qi); ++qi) {
    const int e = min(l0 + AT_CHUNK, valid_len(p, b0 + qi));
    l1max = max(l1max, e);
    l1min = min(l1min, e);
  }
  int l1[NQT];     // this lane's query slots n and 16 + n
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) l1[nt] = live(16 * nt + n) ? min(l0 + AT_CHUNK, valid_len(p, b0 + 16 * nt + n)) : l0;
  float *const part0 = p.part + ((int64_t)b0 * p.heads + h) * p.nchunk * (HD + 2) + (int64_t)c * (HD + 2);
  const int64_t qstride = (int64_t)p.heads * p.nchunk * (HD + 2);  // between sequences
  if (l0 >= l1max) {  // uniform: an empty chunk contributes nothing
    for (int i = t; i < 16 * NQT * (HD + 2); i += AT_T) {
      const int qi = i / (HD + 2), d = i - qi * (HD + 2);
      if (live(qi)) part0[qi * qstride + d] = d == HD ? -INFINITY : 0.0f;
    }
    return;
  }
  if (t < AT_CHUNK / AT_PAGE) {  // the chunk's pages below l1max; -1: masked
    int32_t pg = -1;
    if (l0 + AT_PAGE * t < l1max) {
      pg = p.tbl[(int64_t)b0 * p.tbs + l0 / AT_PAGE + t];
      if (pg < 0 || pg >= p.num_pages) pg = -1;
    }
    pages[t] = pg;
    // a block whose pages are all in the cache and whose positions every
    // sequence attends to needs no masks
    const uint64_t bad = __ballot(pg < 0);
    if ((t & 7) == 0) whole[t / 8] = ((bad >> (t & 56)) & 0xff) == 0 && l0 + AS_BLK * (t / 8 + 1) <= l1min;
  }
  // Q as the B operand of the score products: k-slot (g, j) of k-step kk is
  // dim 32 kk + 4 j + g
  abf16x8_t qop[HD / 32][NQT];
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    const bool ok = live(16 * nt + n);
    const bf16_t *qr = p.q + (int64_t)(ok ? b0 + 16 * nt + n : b0) * p.qb + (int64_t)h * p.qh + g;
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        qop[kk][nt][j] = __builtin_bit_cast(__bf16, ok ? qr[32 * kk + 4 * j] : bf16_t(0));
  }
  __syncthreads();

  float mrun[NQT], lrun[NQT];
  af32x4_t acc[8][NQT];  // o^T: dim tile e (dims 32 g + 8 i + e in lane (n, g)), sequence tile nt
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    mrun[nt] = -INFINITY;
    lrun[nt] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int nt = 0; nt < NQT; ++nt) acc[e][nt] = af32x4_t{0.f, 0.f, 0.f, 0.f};

  // The wave's key and value rows pass through its slots: group kk of a
  // block (keys of k-step kk, then values of k-step kk) goes to slot kk, and
  // a group is requested as soon as the group before it in that slot has
  // been read, so four groups (32 KB) stay in flight.  Loads carry no
  // per-lane branch: a masked page's lanes read page 0 (its keys meet masked
  // scores only, its values are zeroed after the read).  Each page is read
  // once per launch, so the loads carry the non-temporal hint (5% faster).
  auto slot = [&](auto r) __attribute__((always_inline)) -> float * {
    constexpr int R = decltype(r)::value;
    return R == 0 ? ring0[wave] : R == 1 ? ring1[wave] : R == 2 ? ring2[wave] : ring3[wave];
  };
  // keys of k-step kk: lane (m, g) reads dims 32 kk + 4 j + g of positions
  // 8 m .. 8 m + 7 of the block
  auto kreq = [&](int blk, auto kk) __attribute__((always_inline)) {
    const int kpg = pages[(AS_BLK / AT_PAGE) * blk + (n >> 1)];
    const bf16_t *kr = p.k + (int64_t)max(kpg, 0) * p.kb + (int64_t)h * p.kh + 8 * (n & 1) +
                       (int64_t)(32 * kk + g) * p.kd;
    float *dst = slot(kk);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_amdgcn_global_load_lds(kr + (int64_t)(4 * j) * p.kd, (alds_void *)(dst + 256 * j), 16, 0, CPOL);
  };
  // values of k-step kp: lane (m, g) reads dims 8 m .. 8 m + 7 of positions
  // lb + 32 g + 8 kp + j (page pb + 2 g + kp / 2, row 8 (kp % 2) + j)
  auto vreq = [&](int blk, auto kp) __attribute__((always_inline)) {
    const int vpg = pages[(AS_BLK / AT_PAGE) * blk + 2 * g + kp / 2];
    const bf16_t *vr = p.v + (int64_t)max(vpg, 0) * p.vb + (int64_t)h * p.vh +
                       (int64_t)(8 * (kp & 1)) * p.vl + 8 * n;
    float *dst = slot(kp);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_amdgcn_global_load_lds(vr + (int64_t)j * p.vl, (alds_void *)(dst + 256 * j), 16, 0, CPOL);
  };
  // this lane's 16 bytes of each load of a slot's group, once no more than
  // `after` groups requested later are in flight; the slot is then free for
  // the next group (the reads have returned before it is requested)
  auto take = [&](au32x4_t(&r)[8], auto sl, auto after) __attribute__((always_inline)) {
    vmcnt_wait<8 * decltype(after)::value>();
    lds_read8<1024>(r, lds_addr(slot(sl) + 4 * lane));
  };
  using std::integral_constant;
  const int nblk = (l1max - l0 + AS_BLK - 1) / AS_BLK;  // blocks holding positions below l1max
  if (wave < nblk) static_for<HD / 32>([&](auto kk) __attribute__((always_inline)) { kreq(wave, kk); });
  // The running max is kept in log2 units of the scaled score, so each
  // probability is one FMA and one v_exp_f32 (exp2).
  const float c2 = p.scale * 1.4426950408889634f;
  // One block of the sweep; MASK: some position of the block is masked for
  // some sequence (a page outside the cache, or past a sequence's end).
  auto block = [&](int blk, auto mask_c) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_c)::value;
    const int lb = l0 + AS_BLK * blk;
    const int pb = (AS_BLK / AT_PAGE) * blk;  // the block's first page in the chunk
    int vpg[4];
    if constexpr (MASK) {
#pragma unroll
      for (int kp = 0; kp < 4; ++kp) vpg[kp] = pages[pb + 2 * g + kp / 2];
    }
    // scores
    af32x4_t s[8][NQT];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt)
#pragma unroll
      for (int nt = 0; nt < NQT; ++nt) s[tt][nt] = af32x4_t{0.f, 0.f, 0.f, 0.f};
    static_for<HD / 32>([&](auto kk) __attribute__((always_inline)) {
      au32x4_t kv[8];
      // after keys kk: keys kk + 1 .. 3 and values 0 .. kk - 1
      take(kv, kk, integral_constant<int, 3>{});
      vreq(blk, kk);
#define EVO2_SCORE_TILE(T)                                                                  \
  {                                                                                         \
    const abf16x8_t a = column8<T>(kv);                                                     \
    for (int nt = 0; nt < NQT; ++nt)                                                        \
      s[T][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[kk][nt], s[T][nt], 0, 0, 0); \
  }
      EVO2_SCORE_TILE(0) EVO2_SCORE_TILE(1) EVO2_SCORE_TILE(2) EVO2_SCORE_TILE(3)
      EVO2_SCORE_TILE(4) EVO2_SCORE_TILE(5) EVO2_SCORE_TILE(6) EVO2_SCORE_TILE(7)
#undef EVO2_SCORE_TILE
    });
    // s[tt][nt][i]: position lb + 32 g + 8 i + tt, sequence 16 nt + n; its
    // page pb + 2 g + i / 2.  Scores become scale log2(e) q.k (-inf where
    // masked), then probabilities exp2(score - running max).
#pragma unroll
    for (int nt = 0; nt < NQT; ++nt) {
      float bm = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = s[tt][nt][i] * c2;
          if constexpr (MASK) {
            const int l = lb + 32 * g + 8 * i + tt;
            v = vpg[i] >= 0 && l < l1[nt] ? v : -INFINITY;
          }
          s[tt][nt][i] = v;
          bm = fmaxf(bm, v);
        }
      bm = fmaxf(bm, __shfl_xor(bm, 16));
      bm = fmaxf(bm, __shfl_xor(bm, 32));
      const float mn = fmaxf(mrun[nt], bm);
      // while everything so far is masked, mn is -inf: subtract 0 instead
      // (every probability is then exp2(-inf) = 0)
      const float msub = mn == -INFINITY ? 0.0f : mn;
      const float alpha = __builtin_amdgcn_exp2f(mrun[nt] - msub);  // 0 while nothing came before
      float ls = 0.0f;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pe = __builtin_amdgcn_exp2f(s[tt][nt][i] - msub);
          s[tt][nt][i] = pe;
          ls += pe;
        }
      lrun[nt] = fmaf(lrun[nt], alpha, ls);  // this lane's positions only
      mrun[nt] = mn;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e][nt] *= alpha;
      }
    }
    // o^T += V^T P^T over k-steps kp: k-slot (g, j) is position lb + 32 g + 8 kp + j
    const bool more = blk + NW < nblk;  // uniform
    static_for<4>([&](auto kp) __attribute__((always_inline)) {
      constexpr int KP = decltype(kp)::value;
      au32x4_t vv[8];
      // after values kp: values kp + 1 .. 3 and, with a next block, its keys 0 .. kp - 1
      if (more) {
        take(vv, kp, integral_constant<int, 3>{});
        kreq(blk + NW, kp);
      } else {
        take(vv, kp, integral_constant<int, 3 - KP>{});
      }
      if constexpr (MASK) {
        const int lv = lb + 32 * g + 8 * KP;
#pragma unroll
        for (int j = 0; j < 8; ++j)  // masked pages and positions at or past l1max: zero
          if (vpg[KP] < 0 || lv + j >= l1max) vv[j] = au32x4_t{0u, 0u, 0u, 0u};
      }
      // probabilities as bf16 high and low parts (k-slot j = tile j's element KP)
      au32x4_t phu[NQT], plu[NQT];
#pragma unroll
      for (int nt = 0; nt < NQT; ++nt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float a = s[2 * jj][nt][KP], b = s[2 * jj + 1][nt][KP];
          const uint32_t hi = pack_bf(a, b);
          phu[nt][jj] = hi;
          plu[nt][jj] = pack_bf(a - lo_bf(hi), b - hi_bf(hi));
        }
      abf16x8_t ph[NQT], pl[NQT];
#pragma unroll
      for (int nt = 0; nt < NQT; ++nt) {
        ph[nt] = __builtin_bit_cast(abf16x8_t, phu[nt]);
        pl[nt] = __builtin_bit_cast(abf16x8_t, plu[nt]);
      }
#define EVO2_VALUE_TILE(E)                                                                  \
  {                                                                                         \
    const abf16x8_t a = column8<E>(vv);                                                     \
    for (int nt = 0; nt < NQT; ++nt) {                                                      \
      acc[E][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph[nt], acc[E][nt], 0, 0, 0); \
      acc[E][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pl[nt], acc[E][nt], 0, 0, 0); \
    }                                                                                       \
  }
      EVO2_VALUE_TILE(0) EVO2_VALUE_TILE(1) EVO2_VALUE_TILE(2) EVO2_VALUE_TILE(3)
      EVO2_VALUE_TILE(4) EVO2_VALUE_TILE(5) EVO2_VALUE_TILE(6) EVO2_VALUE_TILE(7)
#undef EVO2_VALUE_TILE
    });
  };
  for (int blk = wave; blk < nblk; blk += NW) {
    if (whole[blk]) block(blk, std::false_type{});  // uniform
    else block(blk, std::true_type{});
  }

  // the waves' partials into LDS (o in the wave's slots 0 and 1, whose
  // loads have all been read), then the chunk's (o, max, sum) per sequence
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    float l = lrun[nt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (g == 0) {
      wm[wave][16 * nt + n] = mrun[nt] * 0.6931471805599453f;  // log2 units -> natural
      wl[wave][16 * nt + n] = l;
    }
    float *wo = nt == 0 ? ring0[wave] : ring1[wave];  // (sequence n, dim) rows of HD
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i) wo[n * HD + 32 * g + 8 * i + e] = acc[e][nt][i];
  }
  __syncthreads();
  {
    constexpr int TPQ = AT_T / (16 * NQT);  // threads per sequence
    constexpr int DPT = HD / TPQ;      // dims per thread
    const int qi = t / TPQ, d0 = (t % TPQ) * DPT;
    if (live(qi)) {
      float M = wm[0][qi];
#pragma unroll
      for (int w = 1; w < NW; ++w) M = fmaxf(M, wm[w][qi]);
      float f[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) f[w] = wm[w][qi] == -INFINITY ? 0.0f : expf(wm[w][qi] - M);
      float *part = part0 + qi * qstride;
#pragma unroll
      for (int d = 0; d < DPT; ++d) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) o = fmaf(f[w], (qi < 16 ? ring0[w] : ring1[w])[(qi & 15) * HD + d0 + d], o);
        part[d0 + d] = o;
      }
      if (t % TPQ == 0) {
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) tot = fmaf(f[w], wl[w][qi], tot);
        part[HD] = M;
        part[HD + 1] = tot;
      }
    }
  }
}

// Merge the chunks of (sequence b, head h): lane d of HD.
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(AttnArgs p) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int n = valid_len(p, b);
  const int nc = (n + AT_CHUNK - 1) / AT_CHUNK;
  const float *part = p.part + ((int64_t)b * p.heads + h) * p.nchunk * (HD + 2);
  // unrolled so that several chunks' loads are in flight (the sums stay in
  // chunk order)
  float M = -INFINITY;
#pragma unroll 8
  for (int c = 0; c < nc; ++c) M = fmaxf(M, part[c * (HD + 2) + HD]);
  float tot = 0.0f, o = 0.0f;
#pragma unroll 8
  for (int c = 0; c < nc; ++c) {
    const float mc = part[c * (HD + 2) + HD];
    const float f = mc == -INFINITY ? 0.0f : expf(mc - M);  // a chunk of masked pages
    tot += f * part[c * (HD + 2) + HD + 1];
    o += f * part[c * (HD + 2) + d];
  }
  p.out[(int64_t)b * p.ob + (int64_t)h * p.oh + d] = f2bf(tot > 0.0f ? o / tot : 0.0f);
}

// Chunks [c_first, c_first + c_count) with NQ sequences per workgroup.
template <int HD, bool PAGED, int NQ>
static void launch_chunks(const AttnArgs &a, int c_first, int c_count, hipStream_t st) {
  const int64_t groups = cdiv(static_cast<int64_t>(a.B), NQ);
  const int64_t wgs = cdiv(static_cast<int64_t>(c_count) * a.heads, 8) * 8 * groups;
  AttnArgs b = a;
#ifdef ATTN_GRID3
  b.pair_major = 0;
#else
  b.pair_major = wgs <= 0x7fffffff;
#endif
  if (b.pair_major)
    hipLaunchKernelGGL((attn_chunk_kernel<HD, PAGED, NQ>), dim3(static_cast<unsigned>(wgs)), dim3(AT_T),
                       0, st, b, c_first, c_count);
  else
    hipLaunchKernelGGL((attn_chunk_kernel<HD, PAGED, NQ>),
                       dim3(static_cast<unsigned>(c_count), a.heads, static_cast<unsigned>(groups)),
                       dim3(AT_T), 0, st, b, c_first, c_count);
}

// Chunks [c_first, c_first + c_count) on the matrix-core kernel, gq sequences
// per workgroup.
template <int CPOL, int NQT>
static void launch_mfma(const AttnArgs &a, int c_first, int c_count, int gq, hipStream_t st) {
  const int64_t groups = cdiv(static_cast<int64_t>(a.B), gq);
  const int64_t wgs = cdiv(static_cast<int64_t>(c_count) * a.heads, 8) * 8 * groups;
  AttnArgs b = a;
  b.pair_major = wgs <= 0x7fffffff;
  if (b.pair_major)
    hipLaunchKernelGGL((attn_mfma_kernel<CPOL, NQT>), dim3(static_cast<unsigned>(wgs)), dim3(AT_T), 0, st, b, c_first, c_count,
                       gq);
  else
    hipLaunchKernelGGL((attn_mfma_kernel<CPOL, NQT>),
                       dim3(static_cast<unsigned>(c_count), a.heads, static_cast<unsigned>(groups)), dim3(AT_T),
                       0, st, b, c_first, c_count, gq);
}

// Sequences per workgroup of the one-load-many-queries VALU kernel on the
// chunks every sequence shares (head_dim 64; 128 takes the matrix cores).
constexpr int AT_SHARED_NQ = 4;

template <int HD, bool PAGED>
static int launch_attn(AttnArgs a, int64_t B, int shared_chunks, hipStream_t st) {
  a.B = static_cast<int>(B);
  if constexpr (PAGED) {
    if (shared_chunks > 0) {
      if constexpr (HD == 128) {
        launch_mfma<CPOL_NT, 2>(a, 0, shared_chunks, AS_NQ, st);
      } else {
        launch_chunks<HD, true, AT_SHARED_NQ>(a, 0, shared_chunks, st);
      }
      int rc = check_launch("decode_attention shared chunks");
      if (rc) return rc;
    }
  }
  if (shared_chunks < a.nchunk) {
    // The matrix-core kernel holds one workgroup per CU (its load queue fills
    // the LDS), which pays off when there are whole chunks to stream; a
    // region of own pages shorter than two chunks (a few positions per
    // sequence past a shared prompt) runs faster on the VALU kernel, many
    // workgroups per CU (40B shape, 32 x 64 heads, ~10 positions each: 17.6
    // against 56.4 us).
    bool mfma = false;
    if constexpr (PAGED && HD == 128) mfma = a.nchunk - shared_chunks >= 2;
    if (mfma)
      launch_mfma<CPOL_NT, 1>(a, shared_chunks, a.nchunk - shared_chunks, 1, st);
    else
      launch_chunks<HD, PAGED, 1>(a, shared_chunks, a.nchunk - shared_chunks, st);
    int rc = check_launch("decode_attention chunks");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(attn_merge_kernel<HD>, dim3(a.heads, static_cast<unsigned>(B)), dim3(HD), 0, st, a);
  return check_launch("decode_attention merge");
}

}  // namespace evo2

using namespace evo2;

extern "C" int64_t evo2_decode_attention_workspace_bytes(int64_t B, int64_t heads, int64_t head_dim,
                                                         int64_t L) {
  if (B <= 0 || heads <= 0 || head_dim <= 0 || L <= 0) return 0;
  return B * heads * cdiv(L, AT_CHUNK) * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int evo2_decode_attention(const void *q, int64_t qb, int64_t qh,
                                     const void *k, int64_t kb, int64_t kh, int64_t kd,
                                     const void *v, int64_t vb, int64_t vh, int64_t vl,
                                     const int64_t *positions, float *workspace,
                                     int64_t workspace_bytes, void *out, int64_t ob, int64_t oh,
                                     int64_t B, int64_t heads, int64_t head_dim, int64_t L,
                                     float scale, void *stream) {
  if (B < 0 || heads <= 0 || L <= 0 || B > 65535 || heads > 65535)
    return fail(EVO2_ERR_INVALID, "decode_attention: bad sizes B=%lld heads=%lld L=%lld",
                (long long)B, (long long)heads, (long long)L);
  if (head_dim != 64 && head_dim != 128)
    return fail(EVO2_ERR_UNSUPPORTED, "decode_attention: head_dim %lld (64 or 128)",
                (long long)head_dim);
  if (B == 0) return EVO2_OK;
  if (!q || !k || !v || !positions || !out || !workspace)
    return fail(EVO2_ERR_INVALID, "decode_attention: null pointer argument");
  if (workspace_bytes < evo2_decode_attention_workspace_bytes(B, heads, head_dim, L))
    return fail(EVO2_ERR_INVALID, "decode_attention: workspace too small");
  // 16-byte key loads of eight positions, 16-byte value loads of eight dims
  if (L % 8 || kd % 8 || kh % 8 || kb % 8 || reinterpret_cast<uintptr_t>(k) % 16 ||
      vl % 8 || vh % 8 || vb % 8 || reinterpret_cast<uintptr_t>(v) % 16 || L > 0x7fffffff)
    return fail(EVO2_ERR_UNSUPPORTED, "decode_attention: cache strides or alignment not supported");
  AttnArgs a{static_cast<const bf16_t *>(q), qb, qh, static_cast<const bf16_t *>(k), kb, kh, kd,
             static_cast<const bf16_t *>(v), vb, vh, vl, nullptr, 0, 0, positions, workspace,
             static_cast<bf16_t *>(out), ob, oh, scale, static_cast<int>(heads),
             static_cast<int>(L), static_cast<int>(cdiv(L, AT_CHUNK))};
  hipStream_t st = static_cast<hipStream_t>(stream);
  return head_dim == 64 ? launch_attn<64, false>(a, B, 0, st) : launch_attn<128, false>(a, B, 0, st);
}

extern "C" int evo2_paged_decode_attention(const void *q, int64_t qb, int64_t qh,
                                           const void *k_pages, int64_t kp, int64_t kh, int64_t kd,
                                           const void *v_pages, int64_t vp, int64_t vh, int64_t vl,
                                           int64_t num_pages, const int32_t *block_table,
                                           int64_t tbs, int64_t shared_pages,
                                           const int64_t *positions, float *workspace,
                                           int64_t workspace_bytes, void *out, int64_t ob,
                                           int64_t oh, int64_t B, int64_t heads,
                                           int64_t head_dim, int64_t max_pages, float scale,
                                           void *stream) {
  if (B < 0 || heads <= 0 || max_pages <= 0 || B > 65535 || heads > 65535 ||
      max_pages > (int64_t(1) << 26) || num_pages <= 0 || shared_pages < 0 ||
      shared_pages > max_pages)
    return fail(EVO2_ERR_INVALID,
                "paged_decode_attention: bad sizes B=%lld heads=%lld pages=%lld num_pages=%lld "
                "shared_pages=%lld",
                (long long)B, (long long)heads, (long long)max_pages, (long long)num_pages,
                (long long)shared_pages);
  if (head_dim != 64 && head_dim != 128)
    return fail(EVO2_ERR_UNSUPPORTED, "paged_decode_attention: head_dim %lld (64 or 128)",
                (long long)head_dim);
  if (B == 0) return EVO2_OK;
  if (!q || !k_pages || !v_pages || !block_table || !positions || !out || !workspace)
    return fail(EVO2_ERR_INVALID, "paged_decode_attention: null pointer argument");
  const int64_t L = max_pages * AT_PAGE;
  if (workspace_bytes < evo2_decode_attention_workspace_bytes(B, heads, head_dim, L))
    return fail(EVO2_ERR_INVALID, "paged_decode_attention: workspace too small");
  // 16-byte key loads of eight positions within a page, 16-byte value loads
  if (kd % 8 || kh % 8 || kp % 8 || reinterpret_cast<uintptr_t>(k_pages) % 16 || kd < AT_PAGE ||
      vl % 8 || vh % 8 || vp % 8 || reinterpret_cast<uintptr_t>(v_pages) % 16 || vl < head_dim)
    return fail(EVO2_ERR_UNSUPPORTED,
                "paged_decode_attention: page strides or alignment not supported");
  AttnArgs a{static_cast<const bf16_t *>(q), qb, qh, static_cast<const bf16_t *>(k_pages), kp,
             kh, kd, static_cast<const bf16_t *>(v_pages), vp, vh, vl, block_table, tbs,
             num_pages, positions, workspace, static_cast<bf16_t *>(out), ob, oh, scale,
             static_cast<int>(heads), static_cast<int>(L), static_cast<int>(cdiv(L, AT_CHUNK))};
  hipStream_t st = static_cast<hipStream_t>(stream);
  // chunks that lie wholly inside the shared prefix
  const int shared_chunks = static_cast<int>(shared_pages * AT_PAGE / AT_CHUNK);
  return head_dim == 64 ? launch_attn<64, true>(a, B, shared_chunks, st)
                        : launch_attn<128, true>(a, B, shared_chunks, st);
}
