// Pieces shared by the matrix-core attention kernels: operand vector types,
// a compile-time loop, and LDS reads that the compiler does not order after
// direct-to-LDS loads.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"

namespace evo2 {

typedef __attribute__((ext_vector_type(8))) __bf16 abf16x8_t;
typedef __attribute__((ext_vector_type(4))) float af32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int au32x4_t;
typedef __attribute__((address_space(3))) void alds_void;

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>): the
// index is a constant expression inside f.
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F &f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// Eight 16-byte LDS reads at byte address a + STRIDE j, then a wait for them.
// Inline assembly: the compiler would otherwise wait for every direct-to-LDS
// load in flight before any LDS read; the caller waits for the ones it reads.
template <int STRIDE>
__device__ __forceinline__ void lds_read8(au32x4_t (&r)[8], uint32_t a) {
  static_assert(STRIDE > 0 && 7 * STRIDE < 65536, "ds_read offsets are 16 bits");
  asm volatile(
      "ds_read_b128 %0, %8\n"
      "ds_read_b128 %1, %8 offset:%9\n"
      "ds_read_b128 %2, %8 offset:%10\n"
      "ds_read_b128 %3, %8 offset:%11\n"
      "ds_read_b128 %4, %8 offset:%12\n"
      "ds_read_b128 %5, %8 offset:%13\n"
      "ds_read_b128 %6, %8 offset:%14\n"
      "ds_read_b128 %7, %8 offset:%15\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),
        "=&v"(r[7])
      : "v"(a), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE), "i"(4 * STRIDE), "i"(5 * STRIDE),
        "i"(6 * STRIDE), "i"(7 * STRIDE)
      : "memory");
}

// Four 16-byte LDS reads at byte address a + STRIDE j, then a wait for them.
template <int STRIDE>
__device__ __forceinline__ void lds_read4(au32x4_t (&r)[4], uint32_t a) {
  static_assert(STRIDE > 0 && 3 * STRIDE < 65536, "ds_read offsets are 16 bits");
  asm volatile(
      "ds_read_b128 %0, %4\n"
      "ds_read_b128 %1, %4 offset:%5\n"
      "ds_read_b128 %2, %4 offset:%6\n"
      "ds_read_b128 %3, %4 offset:%7\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(a), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE)
      : "memory");
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

}  // namespace evo2
