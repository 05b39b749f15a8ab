/*
 * evo2_hyena.h -- C ABI of the MI355X (gfx950) Hyena mixer kernels.
 *
 * Every entry point takes plain device pointers, element strides (int64, in
 * elements of the pointed-to type) and sizes, plus the HIP stream to launch
 * on (`hipStream_t` passed as `void*`).  Nothing here allocates, frees or
 * synchronises unless its comment says so, so every call can be captured in a
 * HIP graph.  Return value: EVO2_OK (0) or one of the codes below; the host
 * wrapper raises on nonzero.  `evo2_last_error()` gives a message for the
 * calling thread's most recent failure.
 *
 * bf16 tensors are passed as `const void*` holding IEEE bfloat16 bit patterns;
 * fp8 tensors hold OCP float8_e4m3fn bytes.
 */
#ifndef EVO2_HYENA_H
#define EVO2_HYENA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  EVO2_OK = 0,
  EVO2_ERR_INVALID = 1,     /* bad shape, stride, size or null pointer      */
  EVO2_ERR_UNSUPPORTED = 2, /* valid request this library does not handle   */
  EVO2_ERR_LAUNCH = 3,      /* the HIP runtime rejected a launch            */
  EVO2_ERR_DEVICE = 4       /* device/runtime query failed                  */
};

/* Message for the calling thread's last nonzero return ("" if none). */
const char *evo2_last_error(void);

/* ABI version of this header; bumped on any signature change. */
int evo2_abi_version(void);

/*
 * Fused single-token (q=1) Hyena decode step: short K=3 conv on the
 * interleaved (x2, x1, v) triple, u = x1*v, the inner operator, + D*u, * x2.
 * All three state slices are updated in place.  Rows whose slot equals
 * `null_block` get a zero output and write no state.
 *
 * Replaces triton_decode.hyena_decode / _hyena_decode_kernel
 * (evo2_flash/triton_decode.py:57-164, 185-211), including its rounding points.
 *
 *   z           (B, 3H) bf16, row stride sz, unit column stride
 *   short_w     (3H, 3) bf16, contiguous
 *   conv_state  (blocks, 3H, 2) bf16 view, strides cs0, cs1, cs2
 *   slots       (B,) int32, stride ssl
 *   inner       FIR taps (H, K) bf16 (K = 7 or 128), or LI residues (H, 16)
 *               fp32 when is_iir; strides wi0, wi1
 *   log_poles   (H, 16) fp32, strides lp0, lp1 (is_iir only, else NULL)
 *   inner_state (blocks, H, K-1 | 16) fp32 view, strides is0, is1, is2
 *   D           (H,) bf16 or NULL
 *   out         (B, H) bf16, row stride so
 *   num_blocks  number of blocks in the state pool; a slot outside
 *               [0, num_blocks) is treated like the null block
 */
int evo2_hyena_decode(const void *z, int64_t sz, const void *short_w,
                      void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                      const int32_t *slots, int64_t ssl,
                      const void *inner, int64_t wi0, int64_t wi1,
                      const float *log_poles, int64_t lp0, int64_t lp1,
                      float *inner_state, int64_t is0, int64_t is1, int64_t is2,
                      const void *D, void *out, int64_t so,
                      int64_t B, int64_t H, int32_t K, int32_t is_iir,
                      int32_t null_block, int64_t num_blocks, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* EVO2_HYENA_H */
