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

// The three taps of one sub-channel as bf16 pairs for v_dot2: (w0, w1) and
// (0, w2).
struct ShortTaps {
  uint32_t w01, w2;
};
__device__ __forceinline__ ShortTaps short_taps(const bf16_t *ws, int64_t ch) {
  return ShortTaps{pair_bf(ws[3 * ch], ws[3 * ch + 1]), pair_bf(0, ws[3 * ch + 2])};
}

// Short filter of two consecutive rows, rounded to bf16, for NS sub-channels
// (NS = 3: x2, x1, v; NS = 2: x1, v) from the row pairs Pa = (z0, z1),
// Pb = (z1, z2), Pc = (z2, z3) of each: y0 = bf16(w0 z0 + w1 z1 + w2 z2),
// y1 = bf16(w0 z1 + w1 z2 + w2 z3).  dot2(Pa, (w0, w1), 0) is
// round(w0 z0 + w1 z1) and dot2(Pb, (0, w2), that) adds the exact product
// w2 z2 with one more rounding: the same two roundings as
// fmaf(w2, z2, fmaf(w1, z1, w0 * z0)) in short_out.
//
// One asm block holds the DOTs and the roundings, so it carries its own
// hazard spacing: every DOT result is read at least three instructions after
// it is written (the other DOTs sit between), and what leaves the block comes
// from v_cvt_pk_bf16_f32 (an ordinary VALU op).  The three-operand VOP3P
// v_dot2_f32_bf16 takes the zero accumulator inline.
__device__ __forceinline__ void short_rows2(const uint32_t (&Pa)[3], const uint32_t (&Pb)[3],
                                            const uint32_t (&Pc)[3], const ShortTaps (&w)[3],
                                            float (&y0)[3], float (&y1)[3]) {
  asm("v_dot2_f32_bf16 %0, %6, %15, 0\n\t"
      "v_dot2_f32_bf16 %1, %7, %16, 0\n\t"
      "v_dot2_f32_bf16 %2, %8, %17, 0\n\t"
      "v_dot2_f32_bf16 %3, %9, %15, 0\n\t"
      "v_dot2_f32_bf16 %4, %10, %16, 0\n\t"
      "v_dot2_f32_bf16 %5, %11, %17, 0\n\t"
      "v_dot2_f32_bf16 %0, %9, %18, %0\n\t"
      "v_dot2_f32_bf16 %1, %10, %19, %1\n\t"
      "v_dot2_f32_bf16 %2, %11, %20, %2\n\t"
      "v_dot2_f32_bf16 %3, %12, %18, %3\n\t"
      "v_dot2_f32_bf16 %4, %13, %19, %4\n\t"
      "v_dot2_f32_bf16 %5, %14, %20, %5\n\t"
      "v_cvt_pk_bf16_f32 %0, 0, %0\n\t"
      "v_cvt_pk_bf16_f32 %1, 0, %1\n\t"
      "v_cvt_pk_bf16_f32 %2, 0, %2\n\t"
      "v_cvt_pk_bf16_f32 %3, 0, %3\n\t"
      "v_cvt_pk_bf16_f32 %4, 0, %4\n\t"
      "v_cvt_pk_bf16_f32 %5, 0, %5"
      : "=&v"(y0[0]), "=&v"(y0[1]), "=&v"(y0[2]), "=&v"(y1[0]), "=&v"(y1[1]), "=&v"(y1[2])
      : "v"(Pa[0]), "v"(Pa[1]), "v"(Pa[2]), "v"(Pb[0]), "v"(Pb[1]), "v"(Pb[2]),
        "v"(Pc[0]), "v"(Pc[1]), "v"(Pc[2]), "v"(w[0].w01), "v"(w[1].w01), "v"(w[2].w01),
        "v"(w[0].w2), "v"(w[1].w2), "v"(w[2].w2));
}

__device__ __forceinline__ void short_rows2(const uint32_t (&Pa)[2], const uint32_t (&Pb)[2],
                                            const uint32_t (&Pc)[2], const ShortTaps (&w)[2],
                                            float (&y0)[2], float (&y1)[2]) {
  asm("v_dot2_f32_bf16 %0, %4, %10, 0\n\t"
      "v_dot2_f32_bf16 %1, %5, %11, 0\n\t"
      "v_dot2_f32_bf16 %2, %6, %10, 0\n\t"
      "v_dot2_f32_bf16 %3, %7, %11, 0\n\t"
      "v_dot2_f32_bf16 %0, %6, %12, %0\n\t"
      "v_dot2_f32_bf16 %1, %7, %13, %1\n\t"
      "v_dot2_f32_bf16 %2, %8, %12, %2\n\t"
      "v_dot2_f32_bf16 %3, %9, %13, %3\n\t"
      "v_cvt_pk_bf16_f32 %0, 0, %0\n\t"
      "v_cvt_pk_bf16_f32 %1, 0, %1\n\t"
      "v_cvt_pk_bf16_f32 %2, 0, %2\n\t"
      "v_cvt_pk_bf16_f32 %3, 0, %3"
      : "=&v"(y0[0]), "=&v"(y0[1]), "=&v"(y1[0]), "=&v"(y1[1])
      : "v"(Pa[0]), "v"(Pa[1]), "v"(Pb[0]), "v"(Pb[1]), "v"(Pc[0]), "v"(Pc[1]),
        "v"(w[0].w01), "v"(w[1].w01), "v"(w[0].w2), "v"(w[1].w2));
}

// One rounded short-filter output from P0 = (z0, z1), P1 = (z1, z2), for the
// rows that are not handled in pairs (segment and tile boundaries).
__device__ __forceinline__ float short_dot_rbf(uint32_t P0, uint32_t P1, ShortTaps w) {
  return rbf(dot2(P1, w.w2, dot2(P0, w.w01, 0.0f)));
}

}  // namespace evo2
