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
// Split over the context (flash decoding): workgroup (c, h, b) takes the
// 2048 positions of chunk c, computes its scores with 16-byte loads of eight
// consecutive positions per lane (q in LDS), the chunk's max and exp-sum with
// a block reduction, then sum_l p_l v_l with 16-byte loads of eight dims per
// lane, and writes (o, max, sum) to a workspace; a second launch merges the
// chunks of each (sequence, head).  Keys and values are each read once
// (6.2 TB/s at 64 sequences x 32 heads x 8704 positions); everything is fp32
// until the bf16 output.  The workgroups of one (chunk, head) pair are
// dispatched back to back on one XCD: where the block table points many
// sequences at the same pages (a shared prompt), those pages stream from HBM
// once per pair and from L2 for the other sequences (32 sequences sharing a
// 131072-position prompt: 23.0 -> 8.0 ms per layer; 64 sequences with pages
// of their own: 1.70 -> 1.68 ms).  When the caller declares the shared
// leading pages, the chunks inside them take four sequences per workgroup,
// each key and value load serving all four (8.0 -> 5.4 ms per layer, the
// same bits).
#include "common.h"

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
  const int G = (p.B + NQ - 1) / NQ;  // sequence groups
  int c, h, b0;
  if (p.pair_major) {
    // (chunk, head) pair P and sequence group gi: the G workgroups of a pair
    // run back to back on one XCD (workgroup w runs on XCD w mod 8), so where
    // sequences share pages (one prompt behind many sequences) the pair's
    // keys and values come from HBM once and from that XCD's L2 for the rest
    const int w = blockIdx.x;
    const int j = w >> 3;
    const int P = (j / G) * 8 + (w & 7);
    if (P >= c_count * p.heads) return;  // uniform: padding
    b0 = (j % G) * NQ;
    c = c_first + P % c_count;
    h = P / c_count;
  } else {
    c = c_first + blockIdx.x;
    h = blockIdx.y;
    b0 = blockIdx.z * NQ;
  }
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

// Merge the chunks of (sequence b, head h): lane d of HD.
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(AttnArgs p) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int n = valid_len(p, b);
  const int nc = (n + AT_CHUNK - 1) / AT_CHUNK;
  const float *part = p.part + ((int64_t)b * p.heads + h) * p.nchunk * (HD + 2);
  float M = -INFINITY;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, part[c * (HD + 2) + HD]);
  float tot = 0.0f, o = 0.0f;
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

// Sequences per workgroup on the chunks every sequence shares.
constexpr int AT_SHARED_NQ = 4;

template <int HD, bool PAGED>
static int launch_attn(AttnArgs a, int64_t B, int shared_chunks, hipStream_t st) {
  a.B = static_cast<int>(B);
  if constexpr (PAGED) {
    if (shared_chunks > 0) {
      launch_chunks<HD, true, AT_SHARED_NQ>(a, 0, shared_chunks, st);
      int rc = check_launch("decode_attention shared chunks");
      if (rc) return rc;
    }
  }
  if (shared_chunks < a.nchunk) {
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
