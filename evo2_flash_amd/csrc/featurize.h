// Featurizer pieces shared by the prefill kernels: the K=3 causal short
// filter over the interleaved (x2, x1, v) triple and the gate u = x1 * v.
//
// Prefill rounding: the short filter accumulates its three taps in fp32 and
// rounds the result to bf16 (the output dtype of vLLM's causal_conv1d_fn,
// mixers.py:1140-1150); u = bf16(x1 * v) (mixers.py:1293, 1356).
#pragma once

#include "common.h"

namespace evo2 {

// One segment's view of the packed rows for one channel, resolving the left
// context of the short filter: rows before the segment start `a` come from
// the conv window (oldest first, col 0 = row a-2, col 1 = row a-1) when the
// segment continues a sequence, else they are zero (mixers.py:126-141).
struct ShortCtx {
  const bf16_t *z;  // packed rows, token-major, unit column stride
  int64_t sz;       // row stride of z (elements)
  const bf16_t *conv;  // conv window of this segment's block, or nullptr
  int64_t cs1, cs2;    // strides of the conv window view (channel, column)
  int64_t a;           // segment start row
  bool init;           // has initial state
};

// z value of sub-channel ch (0..3H) at packed row t (t may precede a).
__device__ __forceinline__ float z_at(const ShortCtx &s, int64_t t, int64_t ch) {
  if (t >= s.a) return bf2f(s.z[t * s.sz + ch]);
  if (!s.init || t < s.a - 2) return 0.0f;
  return bf2f(s.conv[ch * s.cs1 + (t - s.a + 2) * s.cs2]);
}

// Short filter output for sub-channel ch at row t given its three inputs
// (oldest first) and taps w[ch*3 .. ch*3+2].
__device__ __forceinline__ float short_out(float zm2, float zm1, float z0, const float w[3]) {
  float acc = w[0] * zm2;
  acc = fmaf(w[1], zm1, acc);
  acc = fmaf(w[2], z0, acc);
  return rbf(acc);
}

}  // namespace evo2
