// Speculative verification of the inner Hyena operators on gfx950: one
// request carries up to Q = 1 + num_spec tokens (packed rows
// [starts[r], ends[r])), starts from the snapshot its previous step
// accepted (ins[r][accepted[r] - 1]) and writes a complete state snapshot
// after every token (outs[r][pos]), so that the next step can resume from
// whichever prefix the sampler accepts.  Replaces triton_verifier.py
// (_fir_kernel / _iir_kernel, lines 46-137) and its wrappers fir_snapshots,
// iir_snapshots, fir_one, iir_one (lines 125-178); the plain torch form is
// mixers.py:578-660.
//
// Arithmetic follows the reference kernels exactly: separate multiply and
// add (no FMA in this file), the FIR sum over k = 16 j + 4 m + l kept as 16
// accumulators (m, l) over j in order, then ((m0 + m1) + m2) + m3 per l, then
// (l0 + l2) + (l1 + l3), plus last * x (triton_verifier.py:17-43, 73); the
// width-7 sum ((p0 + p4) + (p1 + p5) + p2) + p3; the LI readout as the
// halving tree r[s] += r[s + 8], r[s + 4], r[s + 2], r[s + 1] (lines 128-131).
// Outputs keep the input's dtype (bf16 or fp32); rows outside every
// request's range are not written (the wrappers zero them first).
//
// Layout: FIR windows are channel-contiguous native storage (blocks, K-1, H)
// seen as a (blocks, H, K-1) view with unit channel stride, so each column
// moves as one coalesced row per wave; LI states are (blocks, H, 16) with
// unit state stride.  The grid runs channel blocks fastest (blockIdx.x) and
// requests on blockIdx.y, so workgroups dispatched together write adjacent
// pieces of the same columns.  A destination equal to the null block, or outside the
// pool, is not written (the reference skips block 0, line 80); a source
// outside the pool reads as a zero state.
#include "common.h"

#pragma clang fp contract(off)

namespace evo2 {

struct VerifyArgs {
  const void *x; int64_t xs0, xs1;        // (T, H) bf16 or fp32 token inputs u
  int x_f32;
  const bf16_t *w; int64_t w0, w1;        // FIR taps (H, K) bf16
  const float *poles; int64_t p0, p1;     // LI poles exp(log_poles) (H, 16)
  const float *res; int64_t r0, r1;       // LI residues (H, 16)
  float *st; int64_t ss0, ss1, ss2;       // state view (blocks, H, K-1 | 16)
  const int32_t *ins; int64_t is0, is1;   // (nreq, Q) source snapshots
  const int32_t *outs; int64_t os0, os1;  // (nreq, Q) destination snapshots
  const int64_t *starts, *ends, *accepted;  // (nreq,) each; null: one token per request
  void *y; int64_t ys0;                   // (T, H) output, x's dtype
  int Q, H, null_block;
  int64_t num_blocks, T;
};

// Request r's token range, source block and whether it reads a real block.
struct Req {
  int64_t first, end, src;
  bool src_ok;
};

__device__ __forceinline__ Req request_of(const VerifyArgs &a, int64_t r) {
  Req q;
  int64_t col = 0;
  if (a.starts) {
    q.first = a.starts[r];
    q.end = a.ends[r];
    col = a.accepted[r] - 1;
  } else {
    q.first = r;
    q.end = r + 1;
  }
  // rows outside x are never touched, whatever the tables say
  q.end = min(q.end, a.T);
  if (q.first < 0) q.end = q.first;
  const bool col_ok = col >= 0 && col < a.Q;
  const int64_t s = col_ok ? a.ins[r * a.is0 + col * a.is1] : -1;
  q.src_ok = s >= 0 && s < a.num_blocks;
  q.src = q.src_ok ? s : 0;
  return q;
}

__device__ __forceinline__ int64_t dest_of(const VerifyArgs &a, int64_t r, int pos) {
  const int64_t d = a.outs[r * a.os0 + (int64_t)pos * a.os1];
  return (d == a.null_block || d < 0 || d >= a.num_blocks) ? -1 : d;
}

__device__ __forceinline__ float load_x(const VerifyArgs &a, int64_t t, int c) {
  const int64_t off = t * a.xs0 + (int64_t)c * a.xs1;
  return a.x_f32 ? static_cast<const float *>(a.x)[off] : bf2f(static_cast<const bf16_t *>(a.x)[off]);
}

__device__ __forceinline__ void store_y(const VerifyArgs &a, int64_t t, int c, float v) {
  const int64_t off = t * a.ys0 + c;
  if (a.x_f32) static_cast<float *>(a.y)[off] = v;
  else static_cast<bf16_t *>(a.y)[off] = f2bf(v);
}

// ---------------------------------------------------------------------------
// K = 128, requests of up to VQ tokens.  A workgroup owns one request and
// CPW channels.  Every output and snapshot of the step is a function of the
// source window and the step's tokens alone: with e = window ++ (x_0 ..
// x_{n-1}), snapshot p is e[p+1 .. p+127] and y_p sums e[p .. p+126] against
// the taps plus last * x_p.  So e is staged in LDS once; every wave then
// computes the outputs of its positions and issues its share of all snapshot
// stores back to back (no barrier between tokens, so the memory system sees
// every store of the step at once, and they drain while the next workgroup
// stages its window).
//  * copies: with CPW = 128 a lane moves a channel pair (8 bytes; 512 bytes
//    of a column per wave instruction), with CPW = 64 one channel (the form
//    for a state view whose channels are not unit-stride aligned pairs);
//  * waves: NW = 4 x (channels per lane); wave m stages and stores the
//    columns k = m (mod NW), so a block named by two positions ends with the
//    later one's contents (in position order per column, as the reference's
//    sequential writes leave it);
//  * sums: lane = channel; wave m takes the 64 channels of half m / 4 and the
//    positions p = m (mod 4), with the reference's 16 accumulators
//    (k = 16 j + 4 m' + l over j in order), combined as ((A0 + A1) + A2) + A3
//    per l, then (l0 + l2) + (l1 + l3), plus last * x.  Its taps are fetched
//    before the window, so their latency hides under the staging.
// 64 x 4 requests at 7B width (671 MB moved): 212 us with 64 channels and 4
// waves, 197 with channel pairs, 171 with 8 waves, 160 with the sums before
// the stores and the taps first (one process; all bitwise equal).
constexpr int VQ = 16;

template <int CPW>
__global__ __launch_bounds__(4 * CPW, 4) void fir128_verify_kernel(VerifyArgs a) {
  static_assert(CPW == 64 || CPW == 128, "one channel or one channel pair per lane");
  constexpr int CPL = CPW / 64;  // channels per lane in the copies
  constexpr int NW = 4 * CPL;    // waves per workgroup
  __shared__ float e[127 + VQ][CPW];
  const int lane = threadIdx.x & 63;
  const int m = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) % NW;
  const int64_t r = blockIdx.y;
  const int cbase = blockIdx.x * CPW;
  const Req q = request_of(a, r);
  const int n = static_cast<int>(max<int64_t>(0, min<int64_t>(a.Q, q.end - q.first)));

  // this wave's sums: channel cbase + 64 (m / 4) + lane, positions m % 4 + 4 i
  const int p0 = m & 3;
  const int c = cbase + 64 * (m >> 2) + lane;
  const bool active = c < a.H;
  const int cc = active ? c : 0;
  // the channel's taps as bf16 pairs (tap k = half k & 1 of W[k / 2])
  uint32_t W[64];
  const bf16_t *wrow = a.w + (int64_t)cc * a.w0;
  if (a.w1 == 1 && a.w0 % 8 == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint4 v = reinterpret_cast<const uint4 *>(wrow)[i];
      W[4 * i] = v.x; W[4 * i + 1] = v.y; W[4 * i + 2] = v.z; W[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; ++i) W[i] = pair_bf(wrow[(2 * i) * a.w1], wrow[(2 * i + 1) * a.w1]);
  }

  // the lane's channels in the copies: cbase + CPL lane + (0 .. CPL-1); with
  // CPL = 2, H is even, so a pair is wholly inside H or wholly past it
  const int cl = cbase + CPL * lane;
  const bool cact = cl < a.H;
  const int ccl = cact ? cl : 0;
  const float *src = a.st + q.src * a.ss0 + (int64_t)ccl * a.ss1;
  for (int k = m; k < 127; k += NW) {
    if constexpr (CPL == 2) {
      const float2 v = (q.src_ok && cact) ? *reinterpret_cast<const float2 *>(src + (int64_t)k * a.ss2)
                                          : make_float2(0.0f, 0.0f);
      *reinterpret_cast<float2 *>(&e[k][2 * lane]) = v;
    } else {
      e[k][lane] = (q.src_ok && cact) ? src[(int64_t)k * a.ss2] : 0.0f;
    }
  }
  for (int p = m; p < n; p += NW)
#pragma unroll
    for (int i = 0; i < CPL; ++i) e[127 + p][CPL * lane + i] = cact ? load_x(a, q.first + p, cl + i) : 0.0f;
  __syncthreads();

  if (p0 < n) {  // uniform
    const int hc = 64 * (m >> 2) + lane;  // the channel's LDS column
    const float last = hi_bf(W[63]);
    for (int p = p0; p < n; p += 4) {
      // the taps stay packed (64 VGPRs): an empty asm per position keeps the
      // compiler from hoisting 127 converted fp32 taps out of this loop
#pragma unroll
      for (int i = 0; i < 64; ++i) asm volatile("" : "+v"(W[i]));
      float acc[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int l = 0; l < 4; ++l) acc[i][l] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int l = 0; l < 4; ++l) {
            const int k = 16 * j + 4 * i + l;
            if (k < 127) {
              const float wk = (k & 1) ? hi_bf(W[k >> 1]) : lo_bf(W[k >> 1]);
              acc[i][l] = acc[i][l] + e[p + k][hc] * wk;
            }
          }
      }
      float pl[4];
#pragma unroll
      for (int l = 0; l < 4; ++l) pl[l] = ((acc[0][l] + acc[1][l]) + acc[2][l]) + acc[3][l];
      const float yv = ((pl[0] + pl[2]) + (pl[1] + pl[3])) + last * e[127 + p][hc];
      if (active) store_y(a, q.first + p, c, yv);
    }
  }

  for (int p = 0; p < n; ++p) {
    const int64_t d = dest_of(a, r, p);
    if (d >= 0 && cact) {
      float *dst = a.st + d * a.ss0 + (int64_t)cl * a.ss1;
#pragma unroll 8
      for (int k = m; k < 127; k += NW) {
        if constexpr (CPL == 2)
          *reinterpret_cast<float2 *>(dst + (int64_t)k * a.ss2) =
              *reinterpret_cast<const float2 *>(&e[p + 1 + k][2 * lane]);
        else
          dst[(int64_t)k * a.ss2] = e[p + 1 + k][lane];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K = 128, requests of more than VQ tokens (one token at a time).  A
// workgroup owns one request and 64 channels (lane = channel).
// The 127-column window lives in an LDS ring of 128 columns: at position p
// column k of the window is ring slot (p + k) mod 128, so appending the token
// overwrites the slot of the dropped column and nothing moves.  Wave m sums
// the columns k = 16 j + 4 m + l (its accumulators (m, l)); waves 1-3 hand
// their four partials to wave 0 through LDS, which combines them in the
// reference's order.  After each token every wave writes a quarter of the
// new window to the destination snapshot.
__global__ __launch_bounds__(256) void fir128_verify_serial_kernel(VerifyArgs a) {
  __shared__ float ring[128][64];
  __shared__ float part[3][4][64];
  const int lane = threadIdx.x & 63;
  const int m = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
  const int64_t r = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool active = c < a.H;
  const int cc = active ? c : 0;
  const Req q = request_of(a, r);

  // taps of this wave's columns, and the window from the source snapshot
  float wk[8][4];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int k = 16 * j + 4 * m + l;
      wk[j][l] = k < 127 ? bf2f(a.w[(int64_t)cc * a.w0 + (int64_t)k * a.w1]) : 0.0f;
    }
  const float last = bf2f(a.w[(int64_t)cc * a.w0 + 127 * a.w1]);
  const float *src = a.st + q.src * a.ss0 + (int64_t)cc * a.ss1;
  for (int k = m; k < 127; k += 4) ring[k][lane] = (q.src_ok && active) ? src[(int64_t)k * a.ss2] : 0.0f;
  __syncthreads();

  for (int pos = 0; pos < a.Q; ++pos) {
    if (q.first + pos >= q.end) break;  // uniform; positions are consecutive
    const int64_t t = q.first + pos;
    const float x = active ? load_x(a, t, c) : 0.0f;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const int k = 16 * j + 4 * m + l;
        const float s = k < 127 ? ring[(pos + k) & 127][lane] : 0.0f;
        acc[l] = acc[l] + s * wk[j][l];
      }
    if (m > 0) {
#pragma unroll
      for (int l = 0; l < 4; ++l) part[m - 1][l][lane] = acc[l];
    }
    __syncthreads();  // partials visible; every wave done reading this window
    if (m == 0) {
      float p[4];
#pragma unroll
      for (int l = 0; l < 4; ++l)
        p[l] = ((acc[l] + part[0][l][lane]) + part[1][l][lane]) + part[2][l][lane];
      const float yv = ((p[0] + p[2]) + (p[1] + p[3])) + last * x;
      if (active) store_y(a, t, c, yv);
      ring[(pos + 127) & 127][lane] = x;  // the dropped column's slot
    }
    __syncthreads();  // appended token visible; partials consumed
    const int64_t d = dest_of(a, r, pos);
    if (d >= 0 && active) {
      float *dst = a.st + d * a.ss0 + (int64_t)c * a.ss1;
      for (int k = m; k < 127; k += 4) dst[(int64_t)k * a.ss2] = ring[(pos + 1 + k) & 127][lane];
    }
  }
}

// ---------------------------------------------------------------------------
// K = 7: one channel per thread, the 6-column window in registers.
__global__ __launch_bounds__(256) void fir7_verify_kernel(VerifyArgs a) {
  const int64_t r = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.H) return;
  const Req q = request_of(a, r);
  float w[7], s[6];
#pragma unroll
  for (int k = 0; k < 7; ++k) w[k] = bf2f(a.w[(int64_t)c * a.w0 + (int64_t)k * a.w1]);
  const float *src = a.st + q.src * a.ss0 + (int64_t)c * a.ss1;
#pragma unroll
  for (int k = 0; k < 6; ++k) s[k] = q.src_ok ? src[(int64_t)k * a.ss2] : 0.0f;
  // the request's token inputs are loaded up front (up to VQ of them), so
  // their latencies overlap instead of one per token
  const int n = static_cast<int>(max<int64_t>(0, min<int64_t>(a.Q, q.end - q.first)));
  float xs[VQ];
#pragma unroll
  for (int i = 0; i < VQ; ++i) xs[i] = i < n ? load_x(a, q.first + i, c) : 0.0f;
  for (int pos = 0; pos < n; ++pos) {
    const int64_t t = q.first + pos;
    float x = 0.0f;
#pragma unroll
    for (int i = 0; i < VQ; ++i) x = i == pos ? xs[i] : x;
    if (pos >= VQ) x = load_x(a, t, c);
    // ((p0 + p4) + (p1 + p5) + p2) + p3 (triton_verifier.py:35-43)
    float pa = s[0] * w[0], pb = s[1] * w[1];
    const float pc = s[2] * w[2], pd = s[3] * w[3];
    pa = pa + s[4] * w[4];
    pb = pb + s[5] * w[5];
    const float yv = (((pa + pb) + pc) + pd) + w[6] * x;
    store_y(a, t, c, yv);
#pragma unroll
    for (int k = 0; k < 5; ++k) s[k] = s[k + 1];
    s[5] = x;
    const int64_t d = dest_of(a, r, pos);
    if (d >= 0) {
      float *dst = a.st + d * a.ss0 + (int64_t)c * a.ss1;
#pragma unroll
      for (int k = 0; k < 6; ++k) dst[(int64_t)k * a.ss2] = s[k];
    }
  }
}

// ---------------------------------------------------------------------------
// LI: four lanes per channel, lane q of a quad owns states 4q..4q+3 (one
// float4 of the state, residue and pole rows); the readout tree runs over
// quad DPP moves as in the fused decode step.
template <int CTRL>
__device__ __forceinline__ float quad_move(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// VEC: the state rows are 16 contiguous, 16-byte aligned fp32 (one float4 per
// lane); otherwise each lane moves its four states one by one (a row of the
// speculative layout is 17 fp32, its last column the position stamp).
template <bool VEC>
__global__ __launch_bounds__(256) void iir_verify_kernel(VerifyArgs a) {
  const int lane = threadIdx.x & 63;
  const int qd = lane & 3;
  const int64_t r = blockIdx.y;
  const int c = blockIdx.x * 64 + (threadIdx.x >> 2);
  const bool active = c < a.H;
  const int cc = active ? c : a.H - 1;
  const Req q = request_of(a, r);
  const float4 p4 = *reinterpret_cast<const float4 *>(a.poles + (int64_t)cc * a.p0 + 4 * qd);
  const float4 r4 = *reinterpret_cast<const float4 *>(a.res + (int64_t)cc * a.r0 + 4 * qd);
  const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
  const float rv[4] = {r4.x, r4.y, r4.z, r4.w};
  float sv[4] = {0.f, 0.f, 0.f, 0.f};
  if (q.src_ok) {
    const float *sp = a.st + q.src * a.ss0 + (int64_t)cc * a.ss1 + 4 * qd * a.ss2;
    if constexpr (VEC) {
      const float4 s4 = *reinterpret_cast<const float4 *>(sp);
      sv[0] = s4.x; sv[1] = s4.y; sv[2] = s4.z; sv[3] = s4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[e] = sp[e * a.ss2];
    }
  }
  // token inputs up front (up to VQ), so their latencies overlap
  const int n = static_cast<int>(max<int64_t>(0, min<int64_t>(a.Q, q.end - q.first)));
  float xs[VQ];
#pragma unroll
  for (int i = 0; i < VQ; ++i) xs[i] = i < n ? load_x(a, q.first + i, cc) : 0.0f;
  for (int pos = 0; pos < n; ++pos) {  // uniform
    const int64_t t = q.first + pos;
    float x = 0.0f;
#pragma unroll
    for (int i = 0; i < VQ; ++i) x = i == pos ? xs[i] : x;
    if (pos >= VQ) x = load_x(a, t, cc);
    float rr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sv[e] = sv[e] * pv[e] + x;
      rr[e] = sv[e] * rv[e];
    }
    const int64_t d = dest_of(a, r, pos);
    if (d >= 0 && active) {
      float *dp = a.st + d * a.ss0 + (int64_t)c * a.ss1 + 4 * qd * a.ss2;
      if constexpr (VEC) {
        *reinterpret_cast<float4 *>(dp) = make_float4(sv[0], sv[1], sv[2], sv[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dp[e * a.ss2] = sv[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) rr[e] = rr[e] + quad_move<0xEE>(rr[e]);  // += state + 8
#pragma unroll
    for (int e = 0; e < 4; ++e) rr[e] = rr[e] + quad_move<0xF5>(rr[e]);  // += state + 4
    rr[0] = rr[0] + rr[2];                                                   // += state + 2
    rr[1] = rr[1] + rr[3];
    const float yv = rr[0] + rr[1];                                          // += state + 1
    if (qd == 0 && active) store_y(a, t, c, yv);
  }
}

}  // namespace evo2

using namespace evo2;

static int verify_common(const char *who, const void *x, int64_t nreq, int64_t T, int64_t H,
                         int32_t Q,
                         const int32_t *ins, const int32_t *outs, const int64_t *starts,
                         const int64_t *ends, const int64_t *accepted, const void *y,
                         const float *state, int64_t num_blocks) {
  if (nreq < 0 || T < 0 || H <= 0 || H > (1 << 30) || Q <= 0 || num_blocks <= 0)
    return fail(EVO2_ERR_INVALID, "%s: bad sizes nreq=%lld H=%lld Q=%d blocks=%lld", who,
                (long long)nreq, (long long)H, Q, (long long)num_blocks);
  if (nreq > 65535) return fail(EVO2_ERR_UNSUPPORTED, "%s: %lld requests exceed 65535", who,
                                (long long)nreq);
  if (!x || !ins || !outs || !y || !state)
    return fail(EVO2_ERR_INVALID, "%s: null pointer argument", who);
  if ((starts == nullptr) != (ends == nullptr) || (starts == nullptr) != (accepted == nullptr))
    return fail(EVO2_ERR_INVALID, "%s: starts, ends and accepted go together", who);
  if (!starts && Q != 1) return fail(EVO2_ERR_INVALID, "%s: one-token form needs Q=1", who);
  return EVO2_OK;
}

extern "C" int evo2_fir_verify(const void *x, int64_t xs0, int64_t xs1, int32_t x_f32,
                               const void *w, int64_t w0, int64_t w1, int32_t K,
                               float *state, int64_t ss0, int64_t ss1, int64_t ss2,
                               const int32_t *ins, int64_t is0, int64_t is1,
                               const int32_t *outs, int64_t os0, int64_t os1, int32_t Q,
                               const int64_t *starts, const int64_t *ends,
                               const int64_t *accepted, void *y, int64_t ys0, int64_t nreq,
                               int64_t T, int64_t H, int32_t null_block, int64_t num_blocks,
                               void *stream) {
  int rc = verify_common("fir_verify", x, nreq, T, H, Q, ins, outs, starts, ends, accepted, y, state,
                         num_blocks);
  if (rc) return rc;
  if (K != 7 && K != 128)
    return fail(EVO2_ERR_UNSUPPORTED, "fir_verify: filter length %d (7 or 128 only)", K);
  if (!w) return fail(EVO2_ERR_INVALID, "fir_verify: null pointer argument");
  if (nreq == 0) return EVO2_OK;
  VerifyArgs a{x, xs0, xs1, x_f32, static_cast<const bf16_t *>(w), w0, w1, nullptr, 0, 0,
               nullptr, 0, 0, state, ss0, ss1, ss2, ins, is0, is1, outs, os0, os1,
               starts, ends, accepted, y, ys0, Q, static_cast<int>(H), null_block, num_blocks, T};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == 128) {
    // channel pairs move as 8-byte words when the state's channels are
    // unit-stride and every pair starts 8-byte aligned
    const bool pairs = ss1 == 1 && H % 2 == 0 && ss0 % 2 == 0 && ss2 % 2 == 0 &&
                       (reinterpret_cast<uintptr_t>(state) & 7) == 0;
    if (Q <= VQ && pairs) {
      dim3 grid(static_cast<unsigned>(cdiv(H, 128)), static_cast<unsigned>(nreq));
      hipLaunchKernelGGL(fir128_verify_kernel<128>, grid, dim3(512), 0, st, a);
    } else {
      dim3 grid(static_cast<unsigned>(cdiv(H, 64)), static_cast<unsigned>(nreq));
      if (Q <= VQ)
        hipLaunchKernelGGL(fir128_verify_kernel<64>, grid, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL(fir128_verify_serial_kernel, grid, dim3(256), 0, st, a);
    }
  } else {
    dim3 grid(static_cast<unsigned>(cdiv(H, 256)), static_cast<unsigned>(nreq));
    hipLaunchKernelGGL(fir7_verify_kernel, grid, dim3(256), 0, st, a);
  }
  return check_launch("fir_verify");
}

extern "C" int evo2_iir_verify(const void *x, int64_t xs0, int64_t xs1, int32_t x_f32,
                               const float *poles, int64_t p0, int64_t p1,
                               const float *residues, int64_t r0, int64_t r1,
                               float *state, int64_t ss0, int64_t ss1, int64_t ss2,
                               const int32_t *ins, int64_t is0, int64_t is1,
                               const int32_t *outs, int64_t os0, int64_t os1, int32_t Q,
                               const int64_t *starts, const int64_t *ends,
                               const int64_t *accepted, void *y, int64_t ys0, int64_t nreq,
                               int64_t T, int64_t H, int32_t null_block, int64_t num_blocks,
                               void *stream) {
  int rc = verify_common("iir_verify", x, nreq, T, H, Q, ins, outs, starts, ends, accepted, y, state,
                         num_blocks);
  if (rc) return rc;
  if (!poles || !residues) return fail(EVO2_ERR_INVALID, "iir_verify: null pointer argument");
  if (p1 != 1 || r1 != 1 || p0 % 4 || r0 % 4 ||
      reinterpret_cast<uintptr_t>(poles) % 16 || reinterpret_cast<uintptr_t>(residues) % 16)
    return fail(EVO2_ERR_UNSUPPORTED,
                "iir_verify: poles and residues need 16 contiguous, 16-byte aligned fp32 per "
                "channel");
  const bool vec = ss2 == 1 && ss1 % 4 == 0 && ss0 % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(state) % 16 == 0;
  if (nreq == 0) return EVO2_OK;
  VerifyArgs a{x, xs0, xs1, x_f32, nullptr, 0, 0, poles, p0, p1, residues, r0, r1,
               state, ss0, ss1, ss2, ins, is0, is1, outs, os0, os1,
               starts, ends, accepted, y, ys0, Q, static_cast<int>(H), null_block, num_blocks, T};
  dim3 grid(static_cast<unsigned>(cdiv(H, 64)), static_cast<unsigned>(nreq));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec) hipLaunchKernelGGL(iir_verify_kernel<true>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(iir_verify_kernel<false>, grid, dim3(256), 0, st, a);
  return check_launch("iir_verify");
}
