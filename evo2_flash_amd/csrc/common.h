// Shared helpers for the gfx950 Hyena kernels: bf16 rounding, error reporting,
// launch checking.  Included by every .hip translation unit of the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/evo2_hyena.h"

namespace evo2 {

// ---------------------------------------------------------------- bf16 / fp32
typedef uint16_t bf16_t;  // raw bfloat16 bits in memory

__device__ __forceinline__ float bf2f(bf16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16 with round-to-nearest-even (hardware v_cvt_pk_bf16_f32), the
// rounding torch applies when an op writes a bf16 tensor.
__device__ __forceinline__ bf16_t f2bf(float x) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(x));
}

// Round fp32 to bf16 and back: the value a bf16 torch tensor would hold.
__device__ __forceinline__ float rbf(float x) { return bf2f(f2bf(x)); }

// The same rounding in one instruction: v_cvt_pk_bf16_f32 with the value in
// the high half and 0 in the low half is already that fp32 (the compiler's
// form is a cvt plus a shift or permute).  Inline asm is invisible to the
// compiler's hazard recognizer, so x must come from an ordinary VALU op (add,
// mul, fma, cvt, logic): a DOT, MFMA or transcendental result needs wait states
// before another instruction may read it, and none would be inserted here.
__device__ __forceinline__ float rbf_valu(float x) {
  float r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
  return r;
}

__device__ __forceinline__ float lo_bf(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float hi_bf(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}
// (bf16(lo), bf16(hi)) in one dword: a single v_cvt_pk_bf16_f32, the same
// rounding as two f2bf calls.
typedef __attribute__((ext_vector_type(2))) __bf16 bf16v2_t;
__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) {
  bf16v2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// a.lo * b.lo + a.hi * b.hi + c over bf16 pairs (v_dot2_f32_bf16): both
// products are exact in fp32.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16v2_t, a),
                                         __builtin_bit_cast(bf16v2_t, b), c, false);
}

// Two bf16 values (lo = older row) in one dword.
__device__ __forceinline__ uint32_t pair_bf(bf16_t lo, bf16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their maxima), without
// the workgroup memory fence __syncthreads adds.
template <int N>
__device__ __forceinline__ void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Cache-policy operand of the buffer intrinsics: bit 1 is the non-temporal
// hint on gfx950.  The hcm decode window, read and rewritten in place once
// per step, and the packed decode GEMM's sequential weight stream carry it
// (measured: not the snapshot stores of the verify kernel, the row-major
// decode GEMM weight, the prefill streams, the decode attention's KV pages or
// the hcs / hcl windows, where it was level or slower).
constexpr int CPOL_NT = 2;

// The same hint on plain pointer accesses (clang's non-temporal builtins take
// clang vector types, not HIP's float2 / float4 structs).
typedef float nt_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float2 ld_nt(const float2 *p) {
  const nt_f32x2 v = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x2 *>(p));
  return make_float2(v.x, v.y);
}
__device__ __forceinline__ void st_nt(float2 *p, float2 v) {
  __builtin_nontemporal_store(nt_f32x2{v.x, v.y}, reinterpret_cast<nt_f32x2 *>(p));
}
template <typename T>
__device__ __forceinline__ T ld_nt(const T *p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void st_nt(T *p, T v) { __builtin_nontemporal_store(v, p); }

// ---------------------------------------------------------------- host side
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);

// Checks the launch that was just enqueued; EVO2_ERR_LAUNCH with the runtime's
// message on failure.
int check_launch(const char *what);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace evo2
