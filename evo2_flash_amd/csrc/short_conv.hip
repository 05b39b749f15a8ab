// The short causal depthwise convolution as standalone operators, with the
// signatures of the vLLM kernels the reference's mixers call for the K=3
// short filter (mixers.py:1121-1208):
//
//   causal_conv1d_update  one new row per sequence (decode), the window of
//                         each sequence's state slot shifted in place;
//   causal_conv1d_fn      packed prefill segments (query_start_loc), the left
//                         context from the window when has_initial_state, the
//                         window rewritten with the segment's last K-1 inputs.
//
// Arithmetic, per output (the rounding the reference documents for vLLM's
// update kernel, triton_decode.py:10-11, 44-53): an fp32 accumulator that
// starts at the bias (or 0) and adds the K products x[t-K+1+k] * w[k], each
// rounded to bf16, oldest first; optional SiLU in fp32; bf16 out.  The
// prefill uses the same order, so a one-row prefill continuing a window
// equals an update bit for bit.  The fused mixer kernels do not call these
// operators; they exist for callers that bind the vLLM entry points.
//
// Lanes run along channels (rows are channel-contiguous for the reference's
// token-major z), one workgroup per 256 channels and row tile.
#include "common.h"

namespace evo2 {

constexpr int SC_CH = 256;   // channels per workgroup (lane = channel)
constexpr int SC_RT = 64;    // rows per prefill tile

struct ConvArgs {
  const bf16_t *x; int64_t xc, xt;          // input, channel / row strides
  const bf16_t *w; int64_t w0, w1;          // (dim, K)
  const bf16_t *bias;                       // (dim,) or null
  bf16_t *cs; int64_t cs0, cs1, cs2;        // window view (blocks, dim, >= K-1)
  const int32_t *idx; int64_t sidx;         // slot per sequence (null: sequence i uses slot i)
  const uint8_t *init;                      // prefill: has_initial_state per segment (null: none)
  const int32_t *qsl;                       // prefill: (nseq + 1) segment starts
  bf16_t *out; int64_t oc, ot;              // output, channel / row strides
  int dim, nrows, nseq;
  int64_t num_blocks;
  int pad_slot;
};

__device__ __forceinline__ bool slot_ok(const ConvArgs &p, int64_t s) {
  return s != p.pad_slot && s >= 0 && s < p.num_blocks;
}

template <bool SILU>
__device__ __forceinline__ float finish(float acc) {
  if constexpr (SILU) acc = acc / (1.0f + expf(-acc));
  return acc;
}

// One new row per sequence: out[b] from (window, x[b]); window <- (window[1:], x[b]).
template <int K, bool SILU>
__global__ __launch_bounds__(SC_CH) void conv_update_kernel(ConvArgs p) {
  const int c = blockIdx.x * SC_CH + threadIdx.x;
  const int b = blockIdx.y;
  if (c >= p.dim) return;
  const int64_t slot = p.idx ? p.idx[(int64_t)b * p.sidx] : b;
  bf16_t *orow = p.out + (int64_t)b * p.ot + (int64_t)c * p.oc;
  if (!slot_ok(p, slot)) {  // padding row: no state touched, zero output
    *orow = f2bf(0.0f);
    return;
  }
  bf16_t *win = p.cs + slot * p.cs0 + (int64_t)c * p.cs1;
  float s[K - 1];
#pragma unroll
  for (int k = 0; k < K - 1; ++k) s[k] = bf2f(win[k * p.cs2]);
  const float x = bf2f(p.x[(int64_t)b * p.xt + (int64_t)c * p.xc]);
  float acc = p.bias ? bf2f(p.bias[c]) : 0.0f;
#pragma unroll
  for (int k = 0; k < K - 1; ++k) acc += rbf(s[k] * bf2f(p.w[(int64_t)c * p.w0 + k * p.w1]));
  acc += rbf(x * bf2f(p.w[(int64_t)c * p.w0 + (K - 1) * p.w1]));
  *orow = f2bf(finish<SILU>(acc));
#pragma unroll
  for (int k = 0; k + 1 < K - 1; ++k) win[k * p.cs2] = f2bf(s[k + 1]);
  win[(K - 2) * p.cs2] = f2bf(x);
}

// Segment of packed row t (uniform): the last j with qsl[j] <= t.
__device__ __forceinline__ int segment_of(const ConvArgs &p, int t) {
  int lo = 0, hi = p.nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.qsl[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Rows [r0, r0 + SC_RT) of the packed input, lane = channel: a register
// window of the K-1 previous inputs, restarted at each segment start from the
// segment's window (has_initial_state) or zeros.  The windows are only read
// here; conv_window_kernel rewrites them after every tile has run.
template <int K, bool SILU>
__global__ __launch_bounds__(SC_CH) void conv_prefill_kernel(ConvArgs p) {
  const int c = blockIdx.y * SC_CH + threadIdx.x;
  const int r0 = blockIdx.x * SC_RT;
  if (c >= p.dim || r0 >= p.nrows) return;
  const int r1 = min(r0 + SC_RT, p.nrows);
  float wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) wk[k] = bf2f(p.w[(int64_t)c * p.w0 + k * p.w1]);
  const float bias = p.bias ? bf2f(p.bias[c]) : 0.0f;
  // rows [tb, te) of the tile lie in some segment; the others get zeros
  const int tb = max(r0, max(p.qsl[0], 0)), te = min(r1, p.qsl[p.nseq]);
  for (int t = r0; t < r1; ++t)
    if (t < tb || t >= te) p.out[(int64_t)t * p.ot + (int64_t)c * p.oc] = f2bf(0.0f);
  if (tb >= te) return;
  int j = segment_of(p, tb);  // qsl[j] <= tb < qsl[j + 1]
  int a = p.qsl[j], e = p.qsl[j + 1];
  float s[K - 1];
  // window entering row t of segment j: inputs t-K+1 .. t-1
  auto load_window = [&](int t) {
    const int64_t slot = p.idx ? p.idx[(int64_t)j * p.sidx] : j;
    const bool init = p.init && p.init[j] && slot_ok(p, slot);
    const bf16_t *win = init ? p.cs + slot * p.cs0 + (int64_t)c * p.cs1 : nullptr;
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
      const int tt = t - (K - 1) + k;
      float v = 0.0f;
      if (tt >= a && tt >= 0) v = bf2f(p.x[(int64_t)tt * p.xt + (int64_t)c * p.xc]);
      else if (win && tt < a) v = bf2f(win[(K - 1 + (tt - a)) * p.cs2]);
      s[k] = v;
    }
  };
  load_window(tb);
  for (int t = tb; t < te; ++t) {
    if (t >= e) {  // uniform: the next non-empty segment starts at t (t < qsl[nseq])
      while (t >= p.qsl[j + 1]) ++j;
      a = p.qsl[j];
      e = p.qsl[j + 1];
      load_window(t);
    }
    const float x = bf2f(p.x[(int64_t)t * p.xt + (int64_t)c * p.xc]);
    float acc = bias;
#pragma unroll
    for (int k = 0; k < K - 1; ++k) acc += rbf(s[k] * wk[k]);
    acc += rbf(x * wk[K - 1]);
    p.out[(int64_t)t * p.ot + (int64_t)c * p.oc] = f2bf(finish<SILU>(acc));
#pragma unroll
    for (int k = 0; k + 1 < K - 1; ++k) s[k] = s[k + 1];
    s[K - 2] = x;
  }
}

// Per segment and channel: the window <- the last K-1 inputs of cat(window
// or zeros, segment), oldest first, in place (every old value is read before
// any is written).  Empty segments and padding slots are left alone.
template <int K>
__global__ __launch_bounds__(SC_CH) void conv_window_kernel(ConvArgs p) {
  const int c = blockIdx.y * SC_CH + threadIdx.x;
  const int j = blockIdx.x;
  if (c >= p.dim) return;
  const int a = p.qsl[j], e = p.qsl[j + 1];
  const int64_t slot = p.idx ? p.idx[(int64_t)j * p.sidx] : j;
  if (e <= a || a < 0 || e > p.nrows || !slot_ok(p, slot)) return;  // rows must lie in x
  const bool init = p.init && p.init[j];
  bf16_t *win = p.cs + slot * p.cs0 + (int64_t)c * p.cs1;
  const int n = e - a;
  float v[K - 1];
#pragma unroll
  for (int k = 0; k < K - 1; ++k) {
    const int src = n + k;  // position in cat(window (K-1), segment (n))
    if (src >= K - 1) v[k] = bf2f(p.x[(int64_t)(a + src - (K - 1)) * p.xt + (int64_t)c * p.xc]);
    else v[k] = init ? bf2f(win[src * p.cs2]) : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < K - 1; ++k) win[k * p.cs2] = f2bf(v[k]);
}

// Speculative verification, packed varlen rows (vLLM's update convention under
// num_accepted_tokens + query_start_loc).  The state holds state_len columns,
// K-1 + (max_query_len - 1) for a verifier of max_query_len positions, and a
// request's live (K-1)-window starts at column accepted - 1.  A request of q
// tokens computes its outputs from that window and leaves in its output block
//   columns [0, keep)        <- old columns [accepted, accepted + keep)
//   columns [keep, keep + q) <- its q inputs
// with keep = state_len - max_query_len; later columns are left as they were.
// After a later step accepts a of these q tokens, the live window therefore
// starts at column a - 1 again: the last K-1 genuine inputs end at column
// keep + a - 1 = K - 2 + a - 1 when keep = K - 2.
struct SpecConvArgs {
  const bf16_t *x; int64_t xt, xc;          // (T, dim) packed rows
  const bf16_t *w; int64_t w0, w1;
  const bf16_t *bias;
  bf16_t *cs; int64_t cs0, cs1, cs2;        // (blocks, dim, state_len)
  const int32_t *idx; int64_t si0, si1;     // (nreq, ncols) slot matrix
  const int32_t *in_col, *out_col;          // per request (null: column 0)
  const int64_t *accepted;                  // per request, >= 1
  const int32_t *qsl;                       // (nreq + 1) packed row starts
  bf16_t *out; int64_t ot, oc;
  int dim, state_len, max_q, ncols;
  int64_t num_blocks;
  int pad_slot;
  int T;
};

template <int K, bool SILU>
__global__ __launch_bounds__(SC_CH) void conv_update_spec_kernel(SpecConvArgs p) {
  const int c = blockIdx.x * SC_CH + threadIdx.x;
  const int r = blockIdx.y;
  if (c >= p.dim) return;
  const int a = p.qsl[r], e = p.qsl[r + 1];
  if (e <= a || a < 0 || e > p.T) return;
  const int q = e - a;
  const int ic = p.in_col ? p.in_col[r] : 0, oc = p.out_col ? p.out_col[r] : 0;
  const int64_t in_slot = (ic >= 0 && ic < p.ncols) ? p.idx[(int64_t)r * p.si0 + (int64_t)ic * p.si1] : -1;
  const int64_t out_slot = (oc >= 0 && oc < p.ncols) ? p.idx[(int64_t)r * p.si0 + (int64_t)oc * p.si1] : -1;
  const int64_t acc_n = p.accepted[r];
  const int keep = p.state_len - p.max_q;
  // requests the convention cannot place: a padding or out-of-range slot,
  // more rows than the verifier has positions, or an accepted count past the
  // window; their rows are zero and no state is touched
  const bool ok = q <= p.max_q && acc_n >= 1 && acc_n <= p.max_q &&
                  in_slot != p.pad_slot && in_slot >= 0 && in_slot < p.num_blocks &&
                  out_slot != p.pad_slot && out_slot >= 0 && out_slot < p.num_blocks;
  if (!ok) {
    for (int t = a; t < e; ++t) p.out[(int64_t)t * p.ot + (int64_t)c * p.oc] = f2bf(0.0f);
    return;
  }
  const int off = static_cast<int>(acc_n) - 1;
  const bf16_t *src = p.cs + in_slot * p.cs0 + (int64_t)c * p.cs1;
  bf16_t *dst = p.cs + out_slot * p.cs0 + (int64_t)c * p.cs1;
  float s[K - 1];
#pragma unroll
  for (int k = 0; k < K - 1; ++k) s[k] = bf2f(src[(int64_t)(off + k) * p.cs2]);
  float wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) wk[k] = bf2f(p.w[(int64_t)c * p.w0 + k * p.w1]);
  const float bias = p.bias ? bf2f(p.bias[c]) : 0.0f;
  for (int t = a; t < e; ++t) {
    const float x = bf2f(p.x[(int64_t)t * p.xt + (int64_t)c * p.xc]);
    float acc = bias;
#pragma unroll
    for (int k = 0; k < K - 1; ++k) acc += rbf(s[k] * wk[k]);
    acc += rbf(x * wk[K - 1]);
    p.out[(int64_t)t * p.ot + (int64_t)c * p.oc] = f2bf(finish<SILU>(acc));
#pragma unroll
    for (int k = 0; k + 1 < K - 1; ++k) s[k] = s[k + 1];
    s[K - 2] = x;
  }
  // ascending copy: column i reads column off + 1 + i > i, so in place
  // (in_slot == out_slot) every old value is read before it is overwritten
  for (int i = 0; i < keep; ++i) dst[(int64_t)i * p.cs2] = src[(int64_t)(off + 1 + i) * p.cs2];
  for (int i = 0; i < q; ++i)
    dst[(int64_t)(keep + i) * p.cs2] = p.x[(int64_t)(a + i) * p.xt + (int64_t)c * p.xc];
}

template <int K>
static void launch_update(const ConvArgs &a, int64_t B, bool silu, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(cdiv(a.dim, SC_CH)), static_cast<unsigned>(B));
  if (silu) hipLaunchKernelGGL((conv_update_kernel<K, true>), grid, dim3(SC_CH), 0, st, a);
  else hipLaunchKernelGGL((conv_update_kernel<K, false>), grid, dim3(SC_CH), 0, st, a);
}

template <int K>
static int launch_prefill(const ConvArgs &a, bool silu, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(cdiv(a.nrows, SC_RT)), static_cast<unsigned>(cdiv(a.dim, SC_CH)));
  if (silu) hipLaunchKernelGGL((conv_prefill_kernel<K, true>), grid, dim3(SC_CH), 0, st, a);
  else hipLaunchKernelGGL((conv_prefill_kernel<K, false>), grid, dim3(SC_CH), 0, st, a);
  int rc = check_launch("causal_conv1d_fn");
  if (rc || !a.cs || a.nseq == 0) return rc;
  dim3 wgrid(static_cast<unsigned>(a.nseq), static_cast<unsigned>(cdiv(a.dim, SC_CH)));
  hipLaunchKernelGGL(conv_window_kernel<K>, wgrid, dim3(SC_CH), 0, st, a);
  return check_launch("causal_conv1d_fn window update");
}

static int check_conv(const char *fn, int64_t dim, int32_t K, int32_t activation) {
  if (dim <= 0 || dim > 0x7fffffff)
    return fail(EVO2_ERR_INVALID, "%s: bad dim %lld", fn, (long long)dim);
  if (K < 2 || K > 4)
    return fail(EVO2_ERR_UNSUPPORTED, "%s: width %d (2, 3 or 4 only)", fn, K);
  if (activation != 0 && activation != 1)
    return fail(EVO2_ERR_UNSUPPORTED, "%s: activation code %d (0 none, 1 silu)", fn, activation);
  if (cdiv(dim, SC_CH) > 65535)
    return fail(EVO2_ERR_UNSUPPORTED, "%s: dim %lld too large", fn, (long long)dim);
  return EVO2_OK;
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_causal_conv1d_update(const void *x, int64_t xb, int64_t xc,
                                         void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                                         const void *w, int64_t w0, int64_t w1, int32_t K,
                                         const void *bias, int32_t activation,
                                         const int32_t *indices, int64_t sidx, int32_t pad_slot_id,
                                         void *out, int64_t ob, int64_t oc,
                                         int64_t B, int64_t dim, int64_t num_blocks, void *stream) {
  int rc = check_conv("causal_conv1d_update", dim, K, activation);
  if (rc) return rc;
  if (B < 0 || B > 65535 || num_blocks <= 0)
    return fail(EVO2_ERR_INVALID, "causal_conv1d_update: bad sizes B=%lld num_blocks=%lld",
                (long long)B, (long long)num_blocks);
  if (B == 0) return EVO2_OK;
  if (!x || !conv_state || !w || !out)
    return fail(EVO2_ERR_INVALID, "causal_conv1d_update: null pointer argument");
  ConvArgs a{static_cast<const bf16_t *>(x), xc, xb, static_cast<const bf16_t *>(w), w0, w1,
             static_cast<const bf16_t *>(bias), static_cast<bf16_t *>(conv_state), cs0, cs1, cs2,
             indices, sidx, nullptr, nullptr, static_cast<bf16_t *>(out), oc, ob,
             static_cast<int>(dim), static_cast<int>(B), static_cast<int>(B), num_blocks, pad_slot_id};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool silu = activation == 1;
  if (K == 2) launch_update<2>(a, B, silu, st);
  else if (K == 3) launch_update<3>(a, B, silu, st);
  else launch_update<4>(a, B, silu, st);
  return check_launch("causal_conv1d_update");
}

extern "C" int evo2_causal_conv1d_fn(const void *x, int64_t xc, int64_t xt,
                                     const void *w, int64_t w0, int64_t w1, int32_t K,
                                     const void *bias, int32_t activation,
                                     void *conv_states, int64_t cs0, int64_t cs1, int64_t cs2,
                                     const uint8_t *has_initial_state,
                                     const int32_t *cache_indices, int64_t sidx, int32_t pad_slot_id,
                                     const int32_t *query_start_loc, int64_t nseq,
                                     void *out, int64_t oc, int64_t ot,
                                     int64_t T, int64_t dim, int64_t num_blocks, void *stream) {
  int rc = check_conv("causal_conv1d_fn", dim, K, activation);
  if (rc) return rc;
  if (T < 0 || T > 0x7fffffff || nseq < 0 || nseq > 0x7fffffff || (conv_states && num_blocks <= 0))
    return fail(EVO2_ERR_INVALID, "causal_conv1d_fn: bad sizes T=%lld nseq=%lld", (long long)T,
                (long long)nseq);
  if (T == 0) return EVO2_OK;
  if (!x || !w || !out || !query_start_loc)
    return fail(EVO2_ERR_INVALID, "causal_conv1d_fn: null pointer argument");
  if (cdiv(T, SC_RT) > 0x7fffffff || nseq > 0x7fffffff)
    return fail(EVO2_ERR_UNSUPPORTED, "causal_conv1d_fn: grid too large");
  ConvArgs a{static_cast<const bf16_t *>(x), xc, xt, static_cast<const bf16_t *>(w), w0, w1,
             static_cast<const bf16_t *>(bias), static_cast<bf16_t *>(conv_states), cs0, cs1, cs2,
             cache_indices, sidx, conv_states ? has_initial_state : nullptr, query_start_loc,
             static_cast<bf16_t *>(out), oc, ot, static_cast<int>(dim), static_cast<int>(T),
             static_cast<int>(nseq), conv_states ? num_blocks : 1, pad_slot_id};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool silu = activation == 1;
  if (K == 2) return launch_prefill<2>(a, silu, st);
  if (K == 3) return launch_prefill<3>(a, silu, st);
  return launch_prefill<4>(a, silu, st);
}

extern "C" int evo2_causal_conv1d_update_spec(
    const void *x, int64_t xt, int64_t xc,
    void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2, int32_t state_len,
    const void *w, int64_t w0, int64_t w1, int32_t K,
    const void *bias, int32_t activation,
    const int32_t *indices, int64_t si0, int64_t si1, int32_t ncols,
    const int32_t *in_col, const int32_t *out_col, const int64_t *num_accepted,
    const int32_t *query_start_loc, int32_t max_query_len, int32_t pad_slot_id,
    void *out, int64_t ot, int64_t oc,
    int64_t nreq, int64_t T, int64_t dim, int64_t num_blocks, void *stream) {
  const char *fn = "causal_conv1d_update (speculative)";
  int rc = check_conv(fn, dim, K, activation);
  if (rc) return rc;
  if (nreq < 0 || nreq > 65535 || T < 0 || T > 0x7fffffff || num_blocks <= 0 || ncols <= 0)
    return fail(EVO2_ERR_INVALID, "%s: bad sizes nreq=%lld T=%lld num_blocks=%lld ncols=%d", fn,
                (long long)nreq, (long long)T, (long long)num_blocks, ncols);
  if (max_query_len < 1 || state_len < K - 1 + max_query_len - 1)
    return fail(EVO2_ERR_INVALID,
                "%s: a state of %d columns cannot hold a %d-position verifier window (K=%d needs "
                "K-1 + max_query_len-1 columns)", fn, state_len, max_query_len, K);
  if (nreq == 0) return EVO2_OK;
  if (!x || !conv_state || !w || !out || !indices || !num_accepted || !query_start_loc)
    return fail(EVO2_ERR_INVALID, "%s: null pointer argument", fn);
  SpecConvArgs a{static_cast<const bf16_t *>(x), xt, xc, static_cast<const bf16_t *>(w), w0, w1,
                 static_cast<const bf16_t *>(bias), static_cast<bf16_t *>(conv_state), cs0, cs1, cs2,
                 indices, si0, si1, in_col, out_col, num_accepted, query_start_loc,
                 static_cast<bf16_t *>(out), ot, oc, static_cast<int>(dim), state_len, max_query_len,
                 ncols, num_blocks, pad_slot_id, static_cast<int>(T)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(cdiv(dim, SC_CH)), static_cast<unsigned>(nreq));
  const bool silu = activation == 1;
#define EVO2_SPEC_LAUNCH(KW)                                                                   \
  if (silu) hipLaunchKernelGGL((conv_update_spec_kernel<KW, true>), grid, dim3(SC_CH), 0, st, a); \
  else hipLaunchKernelGGL((conv_update_spec_kernel<KW, false>), grid, dim3(SC_CH), 0, st, a);
  if (K == 2) { EVO2_SPEC_LAUNCH(2) }
  else if (K == 3) { EVO2_SPEC_LAUNCH(3) }
  else { EVO2_SPEC_LAUNCH(4) }
#undef EVO2_SPEC_LAUNCH
  return check_launch(fn);
}
