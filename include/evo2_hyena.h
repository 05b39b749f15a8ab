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

/*
 * Varlen depthwise causal FIR over packed prefill rows, carrying per-segment
 * windows: y = FIR(u) (bf16 out), and each segment's last K-1 inputs of
 * cat(window, segment) written back into `state`.
 *
 * Replaces triton_prefill.fir_prefill (evo2_flash/triton_prefill.py:391-496).
 *
 *   u          (T, H) bf16, row stride su          w  (H, K) bf16, strides w0, w1
 *   state      (blocks, H, >=K-1) fp32 view, strides st0, st1, st2
 *   seq_table  (nseq, 3) int32 [start, end, has_initial_state], contiguous
 *   blocks     (nseq,) int32 state block per segment, stride sblk
 *   tile_table (ntiles, 2) int32 [segment, first row], rows step block_t
 *   out        (T, H) bf16, row stride so
 * K is 7 or 128; H must be even; block_t a positive multiple of 64.
 */
int evo2_fir_prefill(const void *u, int64_t su, const void *w, int64_t w0, int64_t w1,
                     int32_t K, float *state, int64_t st0, int64_t st1, int64_t st2,
                     const int32_t *seq_table, int64_t nseq,
                     const int32_t *blocks, int64_t sblk,
                     const int32_t *tile_table, int64_t ntiles, int32_t block_t,
                     void *out, int64_t so, int64_t T, int64_t H,
                     int64_t num_blocks, void *stream);

/*
 * Fused Hyena FIR mixer prefill (hcs K=7 / hcm K=128) between in_proj and
 * out_proj: z -> short K=3 filter (left context from conv_state) ->
 * u = x1*v -> FIR(u) (left context from inner_state) [+ D*u] -> g = x2*y.
 * Both windows are rewritten for every segment.
 *
 * Replaces the prefill rows of HyenaFIRMixer._forward_impl
 * (evo2_flash/mixers.py:1277-1305): vLLM causal_conv1d_fn (mixers.py:1140-1150),
 * the gate, _depthwise_prefill_triton (mixers.py:418-428) and the bf16 tail.
 *
 *   z          (T, 3H) bf16, row stride sz    short_w (3H, 3) bf16 contiguous
 *   conv_state (blocks, 3H, 2) bf16 view      D (H,) bf16 or NULL (hcs)
 *   other arguments as evo2_fir_prefill; out = g (T, H) bf16.
 */
int evo2_hyena_fir_prefill(const void *z, int64_t sz, const void *short_w,
                           void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                           const void *w, int64_t w0, int64_t w1, int32_t K,
                           float *inner_state, int64_t st0, int64_t st1, int64_t st2,
                           const void *D,
                           const int32_t *seq_table, int64_t nseq,
                           const int32_t *blocks, int64_t sblk,
                           const int32_t *tile_table, int64_t ntiles, int32_t block_t,
                           void *out, int64_t so, int64_t T, int64_t H,
                           int64_t num_blocks, void *stream);

/*
 * Bytes of workspace the LI prefill needs: one (H, 16) fp32 state per tile.
 */
int64_t evo2_hcl_workspace_bytes(int64_t ntiles, int64_t H);

/*
 * Fused Hyena LI (hcl) mixer prefill between in_proj and out_proj:
 * z -> short K=3 filter -> u = x1*v -> s_t = p*s_{t-1} + u_t over 16 real
 * poles p = exp(log_poles) (state from `ssm` when a segment continues) ->
 * y_t = sum_s r_s s_t -> g = bf16(bf16(bf16(y) + bf16(u*D)) * x2).  Writes
 * each segment's final state to `ssm` and its conv window.
 *
 * Replaces the prefill rows of HyenaIIRMixer._forward_impl
 * (evo2_flash/mixers.py:1327-1401): iir_segment's FFT convolution and
 * closed-form final state (mixers.py:144-210), hcl_compute_filter
 * (triton_hcl.py:88-123) and iir_final_state (triton_prefill.py:351-387).
 *
 *   residues, log_poles (H, 16) fp32      ssm (blocks, H, 16) fp32 view
 *   tile_start (nseq + 1) int32: index of each segment's first tile
 *   workspace  >= evo2_hcl_workspace_bytes(ntiles, H) bytes of device memory
 *   other arguments as evo2_hyena_fir_prefill; block_t a multiple of 16.
 */
int evo2_hyena_hcl_prefill(const void *z, int64_t sz, const void *short_w,
                           void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                           const float *residues, int64_t r0, int64_t r1,
                           const float *log_poles, int64_t l0, int64_t l1,
                           float *ssm, int64_t m0, int64_t m1, int64_t m2,
                           const void *D,
                           const int32_t *seq_table, int64_t nseq,
                           const int32_t *blocks, int64_t sblk,
                           const int32_t *tile_table, int64_t ntiles,
                           const int32_t *tile_start, int32_t block_t,
                           float *workspace, int64_t workspace_bytes,
                           void *out, int64_t so, int64_t T, int64_t H,
                           int64_t num_blocks, void *stream);

/*
 * evo2_hyena_hcl_prefill without the workspace argument: the same kernels,
 * with the tile states in the library's own device scratch (32 MiB per GPU,
 * held until the process ends).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc); it calls no hipMalloc,
 * hipFree or allocating library routine.  Returns EVO2_ERR_UNSUPPORTED when
 * evo2_hcl_workspace_bytes(ntiles, H) exceeds 32 MiB, i.e. when
 * ntiles * H > 524 288 (32 768 tokens at H=4096 with block_t >= 256, or
 * 65 536 at H=8192 with block_t 1024, fit).  Calls on one GPU share its
 * scratch: calls that overlap on one GPU (concurrent streams) race.
 */
int evo2_hyena_hcl_prefill_noalloc(const void *z, int64_t sz, const void *short_w,
                                   void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                                   const float *residues, int64_t r0, int64_t r1,
                                   const float *log_poles, int64_t l0, int64_t l1,
                                   float *ssm, int64_t m0, int64_t m1, int64_t m2,
                                   const void *D,
                                   const int32_t *seq_table, int64_t nseq,
                                   const int32_t *blocks, int64_t sblk,
                                   const int32_t *tile_table, int64_t ntiles,
                                   const int32_t *tile_start, int32_t block_t,
                                   void *out, int64_t so, int64_t T, int64_t H,
                                   int64_t num_blocks, void *stream);

/*
 * One prefill segment of the LI recurrence s_t = p*s_{t-1} + x_t:
 * y (H, L) fp32 and the final state st (H, 16) fp32 (contiguous), from
 * s_prev (H, 16) or zero (NULL).  seq is (H, L) fp32 with any strides.
 *
 * Replaces iir_segment (evo2_flash/mixers.py:144-210).
 */
int evo2_iir_segment(const float *seq, int64_t xh, int64_t xl,
                     const float *residues, int64_t r0, int64_t r1,
                     const float *log_poles, int64_t l0, int64_t l1,
                     const float *s_prev, int64_t sp0, int64_t sp1,
                     float *y, int64_t yh, int64_t yl, float *st,
                     float *workspace, int64_t workspace_bytes,
                     int64_t H, int64_t L, int32_t block_t, void *stream);

/*
 * Final state only of one LI prefill segment started from zero:
 * st[h, s] = sum_t seq[h, t] p[h, s]^(L-1-t), p = exp(log_poles), evaluated
 * as the recurrence s_t = p*s_{t-1} + x_t in fp32 (tile end states, then a
 * carry scan).  seq (H, L) fp32 with any strides; st (H, 16) contiguous;
 * workspace of evo2_hcl_workspace_bytes(cdiv(L, block_t), H) bytes.
 *
 * Replaces iir_final_state (evo2_flash/triton_prefill.py:351-387).
 */
int evo2_iir_final_state(const float *seq, int64_t xh, int64_t xl,
                         const float *log_poles, int64_t l0, int64_t l1, float *st,
                         float *workspace, int64_t workspace_bytes,
                         int64_t H, int64_t L, int32_t block_t, void *stream);

/*
 * Modal filter h[d, l] = sum_s residues[d, s] * exp(log_poles[d, s] * t[l]).
 *
 * Replaces hcl_compute_filter / _hcl_compute_filter_kernel
 * (evo2_flash/triton_hcl.py:46-123).
 */
int evo2_hcl_compute_filter(const float *residues, int64_t r0, int64_t r1,
                            const float *log_poles, int64_t l0, int64_t l1,
                            const float *t, int64_t st, float *h, int64_t h0, int64_t h1,
                            int64_t D, int64_t S, int64_t L, void *stream);

/*
 * Short causal depthwise convolution, one new row per sequence (decode):
 *   out[b, c] = bf16(act(((bias[c] + r(s0 w0)) + r(s1 w1)) + ... + r(x[b, c] w[K-1])))
 * with r() rounding a product to bf16, (s0 .. s_{K-2}) the window of slot
 * indices[b] (oldest first), which then becomes (s1 .. s_{K-2}, x[b, c]).
 *   x (B, dim) bf16 (strides xb, xc); conv_state (blocks, dim, >= K-1) bf16
 *   view; w (dim, K) bf16; bias (dim,) bf16 or NULL; activation 0 = none,
 *   1 = SiLU; indices (B,) int32 (stride sidx) or NULL for slot b; a row whose
 *   slot is pad_slot_id or outside [0, num_blocks) gets a zero output and
 *   touches no state.  K in {2, 3, 4}.
 *
 * Replaces vLLM's causal_conv1d_update as the reference's mixers call it for
 * the K=3 short filter (evo2_flash/mixers.py:1194-1204; rounding as
 * triton_decode.py:10-11, 44-53 states it).
 */
int evo2_causal_conv1d_update(const void *x, int64_t xb, int64_t xc,
                              void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                              const void *w, int64_t w0, int64_t w1, int32_t K,
                              const void *bias, int32_t activation,
                              const int32_t *indices, int64_t sidx, int32_t pad_slot_id,
                              void *out, int64_t ob, int64_t oc,
                              int64_t B, int64_t dim, int64_t num_blocks, void *stream);

/*
 * The same update for speculative verification: request r owns packed rows
 * [query_start_loc[r], query_start_loc[r + 1]) of x (T, dim) (at most
 * max_query_len of them) and the slot row indices[r, :] (ncols columns).
 * It reads the window of slot indices[r, in_col[r]] (column 0 when in_col is
 * NULL) at columns num_accepted[r]-1 .. num_accepted[r]+K-3, runs its rows
 * through it with the rounding above, and leaves in slot
 * indices[r, out_col[r]] (column 0 when NULL):
 *   columns [0, keep)        <- old columns [num_accepted[r], num_accepted[r] + keep)
 *   columns [keep, keep + q) <- its q inputs,   keep = state_len - max_query_len,
 * later columns untouched, so after a later step accepts a of the q rows the
 * live window starts at column a - 1.  The conv state is (blocks, dim,
 * state_len) with state_len >= K-1 + max_query_len-1.  A request with a
 * padding or out-of-range slot, more than max_query_len rows or num_accepted
 * outside [1, max_query_len] gets zero rows and touches no state; rows no
 * request covers are not written.  K in {2, 3, 4}.
 *
 * Replaces vLLM's causal_conv1d_update called with num_accepted_tokens,
 * query_start_loc and max_query_len (and, for prefix caching,
 * block_idx_last_scheduled_token / initial_state_idx as out_col / in_col),
 * as the reference's mixers call it for speculative decode
 * (evo2_flash/mixers.py:1153-1193; window convention mixers.py:222-240).
 */
int evo2_causal_conv1d_update_spec(const void *x, int64_t xt, int64_t xc,
                                   void *conv_state, int64_t cs0, int64_t cs1, int64_t cs2,
                                   int32_t state_len,
                                   const void *w, int64_t w0, int64_t w1, int32_t K,
                                   const void *bias, int32_t activation,
                                   const int32_t *indices, int64_t si0, int64_t si1, int32_t ncols,
                                   const int32_t *in_col, const int32_t *out_col,
                                   const int64_t *num_accepted, const int32_t *query_start_loc,
                                   int32_t max_query_len, int32_t pad_slot_id,
                                   void *out, int64_t ot, int64_t oc,
                                   int64_t nreq, int64_t T, int64_t dim, int64_t num_blocks,
                                   void *stream);

/*
 * Short causal depthwise convolution over packed prefill segments: segment j
 * is rows [query_start_loc[j], query_start_loc[j + 1]) of x, with slot
 * cache_indices[j] (or j when NULL).  Its left context is the slot's window
 * when has_initial_state[j] (else zeros); after the launch the window holds
 * the segment's last K-1 inputs of cat(window or zeros, segment).  Outputs
 * are rounded as in evo2_causal_conv1d_update; rows outside every segment
 * are zero.  x (dim, T) bf16 with strides (xc, xt); out likewise (oc, ot);
 * conv_states NULL skips every window read and write.  Empty segments and
 * padding slots touch no window.
 *
 * Replaces vLLM's causal_conv1d_fn as the reference's mixers call it for the
 * K=3 short filter (evo2_flash/mixers.py:1138-1150).
 */
int evo2_causal_conv1d_fn(const void *x, int64_t xc, int64_t xt,
                          const void *w, int64_t w0, int64_t w1, int32_t K,
                          const void *bias, int32_t activation,
                          void *conv_states, int64_t cs0, int64_t cs1, int64_t cs2,
                          const uint8_t *has_initial_state,
                          const int32_t *cache_indices, int64_t sidx, int32_t pad_slot_id,
                          const int32_t *query_start_loc, int64_t nseq,
                          void *out, int64_t oc, int64_t ot,
                          int64_t T, int64_t dim, int64_t num_blocks, void *stream);

/*
 * Decode attention of the whole-model harness: for each sequence b and head
 * h, out[b, h] = sum_l softmax_l(scale * q[b, h] . k[b, h, :, l]) v[b, h, l, :]
 * over l <= positions[b] (int64).  k is (B, heads, head_dim, L) with unit
 * position stride, v is (B, heads, L, head_dim) with unit dim stride, q and
 * out are (B, heads, head_dim) bf16 with unit dim stride.  head_dim 64 or
 * 128; L a multiple of 8; workspace of
 * evo2_decode_attention_workspace_bytes(B, heads, head_dim, L) bytes.
 *
 * Serves the attention layers of Evo2Attention at decode
 * (evo2_flash/model.py:104-153) over this build's contiguous KV cache (the
 * reference runs vLLM's paged attention there, outside the mixer path).
 */
int64_t evo2_decode_attention_workspace_bytes(int64_t B, int64_t heads, int64_t head_dim,
                                              int64_t L);
int evo2_decode_attention(const void *q, int64_t qb, int64_t qh,
                          const void *k, int64_t kb, int64_t kh, int64_t kd,
                          const void *v, int64_t vb, int64_t vh, int64_t vl,
                          const int64_t *positions, float *workspace, int64_t workspace_bytes,
                          void *out, int64_t ob, int64_t oh,
                          int64_t B, int64_t heads, int64_t head_dim, int64_t L,
                          float scale, void *stream);

/*
 * evo2_decode_attention over a paged KV cache of 16-position pages:
 * position l of sequence b lives in page block_table[b, l / 16] (row stride
 * tbs) at offset l % 16;
 *   key pages   (pages, heads, head_dim, 16): strides kp, kh, kd; position stride 1
 *   value pages (pages, heads, 16, head_dim): strides vp, vh, vl; dim stride 1
 * Sequence b attends to positions 0..positions[b] (< max_pages * 16); the
 * workspace is evo2_decode_attention_workspace_bytes(B, heads, head_dim,
 * max_pages * 16) bytes.  num_pages is the number of pages the cache holds:
 * a table entry outside [0, num_pages) is never read through; the positions
 * it names are left out of the softmax (zeros for a sequence left with none).
 * shared_pages (0 <= shared_pages <= max_pages) declares that the first
 * shared_pages entries of every row name the same pages (one prompt behind
 * all B sequences): the chunks of 2048 positions inside that prefix then
 * read each page once for up to 32 sequences (head_dim 128, on the matrix
 * cores: the sums in another order, within a bf16 rounding step of the
 * undeclared result) or four (head_dim 64, the same bits).  A wrong
 * declaration computes those chunks with row 0's pages for every sequence.
 *
 * Serves the attention layers of Evo2Attention at decode
 * (evo2_flash/model.py:104-153) over the paged cache layout the serving
 * engine keeps (vLLM's paged attention there, outside the mixer path).
 */
int evo2_paged_decode_attention(const void *q, int64_t qb, int64_t qh,
                                const void *k_pages, int64_t kp, int64_t kh, int64_t kd,
                                const void *v_pages, int64_t vp, int64_t vh, int64_t vl,
                                int64_t num_pages, const int32_t *block_table, int64_t tbs,
                                int64_t shared_pages,
                                const int64_t *positions, float *workspace,
                                int64_t workspace_bytes, void *out, int64_t ob, int64_t oh,
                                int64_t B, int64_t heads, int64_t head_dim, int64_t max_pages,
                                float scale, void *stream);

/*
 * Causal self-attention of prompts, the prefill form of the attention layers:
 *   out[n, h, i] = sum_{j <= i} softmax_j(scale q[n, h, i] . k[n, h, j]) v[n, h, j]
 *   q, k, out (N, heads, L, head_dim) bf16, contiguous;
 *   vt        (N, heads, head_dim, L) bf16, contiguous: the values transposed.
 * head_dim 128, L a multiple of 8 with 256 L < 2^32, 16-byte aligned
 * pointers, scale > 0.  Scores, the
 * softmax and the weighted sum are fp32, the softmax weights enter the value
 * product as bf16 (flash attention's rounding), the output is bf16.
 *
 * Serves the attention layers of Evo2Attention at prefill
 * (evo2_flash/model.py:104-153; vLLM's flash attention there, outside the
 * mixer path).
 */
int evo2_prefill_attention(const void *q, const void *k, const void *vt, void *out, int64_t N,
                           int64_t heads, int64_t L, int64_t head_dim, float scale, void *stream);

/*
 * Static per-tensor activation quantisation for the fp8 projections:
 * q = e4m3fn(clamp(x / scale[0], -448, 448)), round to nearest even.
 *   x (rows, K) bf16, row stride sx; q (rows, K) e4m3 bytes, row stride sq.
 *
 * Replaces the activation side of vLLM's static fp8 linear
 * (evo2_flash/fp8_emul.py:76-78 states the same contract).
 */
int evo2_fp8_quantize(const void *x, int64_t sx, void *q, int64_t sq,
                      const float *scale, int64_t rows, int64_t K, void *stream);

/*
 * fp8 e4m3 GEMM on MFMA with fp32 accumulation:
 * out[m, n] = bf16((sum_k x8[m, k] w8[n, k]) * x_scale[0] * w_scale[0] [+ bias[n]]).
 *   x8 (M, K), w8 (N, K) e4m3 bytes with 16-byte aligned rows (strides in
 *   bytes); bias (N,) bf16 or NULL; out (M, N) bf16, row stride so.
 *   K must be a multiple of 64.
 *
 * Replaces the in_proj GEMM of vLLM's static W8A8 ReplicatedLinear
 * (evo2_flash/mixers.py:741-757, 1076-1092) and, when quantised, out_proj
 * (mixers.py:801-803).
 */
int evo2_fp8_gemm(const void *x8, int64_t sx, const void *w8, int64_t sw,
                  const float *x_scale, const float *w_scale, const void *bias,
                  void *out, int64_t so, int64_t M, int64_t N, int64_t K, void *stream);

/*
 * The decode layout of an e4m3 weight for evo2_fp8_gemm_packed: w8 (N, K),
 * row stride sw bytes (16-byte aligned rows), into wp (N * K bytes, 16-byte
 * aligned).  With KT = K / 128, byte b of the 16-byte chunk
 * ((G * KT + k) * 2 + h) * 64 + r + 16 q of wp is w8[16 G + r][128 k + 32 q
 * + 16 h + b]: each 16-row group's 128-byte K step is one contiguous 2 KB
 * block, in the order the decode kernel's fragments load it.  N must be a
 * multiple of 16 and K of 128.  Asynchronous on `stream`.
 *
 * No counterpart in the reference (its weights stay in the checkpoint
 * layout): a one-time re-layout, kept beside the checkpoint copy, for
 * decode-sized GEMMs that stream the whole weight per step.
 */
int evo2_fp8_pack_weight(const void *w8, int64_t sw, void *wp, int64_t N, int64_t K,
                         void *stream);

/*
 * evo2_fp8_gemm with the weight in the decode layout written by
 * evo2_fp8_pack_weight (same x8, scales, bias, out and result bits as
 * evo2_fp8_gemm on the unpacked weight; N a multiple of 16, K of 128).  Runs
 * the weight-streaming kernel over ceil(M / 64) blocks of 64 rows, so it is
 * meant for the shapes where evo2_fp8_gemm streams too (M <= 64, or
 * ceil(M / 64) * N <= 60000: decode and verify steps).  The weight stream is
 * sequential per wave: the 7B decode in_proj (M=64, K=4096, N=12288) with the
 * weights streaming from HBM takes ~15.0 us against ~17.4 us unpacked.
 *
 * No counterpart in the reference: the decode-step form of the in_proj GEMM
 * (mixers.py:741-757, 1076-1092) for callers that keep a packed copy.
 */
int evo2_fp8_gemm_packed(const void *x8, int64_t sx, const void *wp,
                         const float *x_scale, const float *w_scale, const void *bias,
                         void *out, int64_t so, int64_t M, int64_t N, int64_t K, void *stream);

/*
 * The order in which evo2_fp8_gemm's persistent kernel (one workgroup per
 * compute unit, 256 x 256 output tiles) walks a grid of tiles_n x tiles_m
 * tiles on a device with ncu compute units: tile t, run by workgroup
 * t mod ncu, is output tile (bn[t], bm[t]).  Fills bn / bm (tiles_n * tiles_m
 * entries each, both may be NULL) and returns 1 for the XCD-grouped order,
 * 0 for row-major, -1 for bad sizes.  Host only, no GPU needed.
 *
 * No counterpart in the reference (its GEMM is a library call): a planning
 * query for callers and tests that check the tile order covers every tile.
 */
int64_t evo2_fp8_gemm_persist_order(int64_t tiles_n, int64_t tiles_m, int ncu,
                                    int32_t *bn, int32_t *bm);

/*
 * Software model of Hopper's fp8 "fast accumulation" GEMM (bit-exact):
 * per group of 32 consecutive k, e = max(max_k e(a_k) + e(b_k), e(acc)) with
 * e(x) = floor(log2|x|); the accumulator and every product are truncated
 * toward zero to 2^(e-13), summed, and the sum truncated to 13 fraction bits
 * of its own exponent.  out = bf16((acc * input_scale[0]) * weight_scale[0]),
 * or, with out_f32 != 0, the fp32 accumulator itself (scales unused).
 *   a8 (N, K) e4m3 bytes, row stride sa (bytes); b_t (K, M) bf16 holding E4M3
 *   values (K-major), row stride sb (elements); out (N, M), row stride so.
 *   K must be a multiple of 32.
 *
 * Replaces evo2_flash/fp8_emul_triton.py:44-77, 142-191
 * (fast_accum_mm_triton, static_fp8_linear_emulated_triton), which the
 * FP8-surgery projections call (mixers.py:691-708, 768-800, 1087-1089).
 */
int evo2_fp8_fast_accum_gemm(const void *a8, int64_t sa, const void *b_t, int64_t sb,
                             const float *input_scale, const float *weight_scale,
                             void *out, int64_t so, int32_t out_f32, int64_t N, int64_t M,
                             int64_t K, void *stream);

/*
 * Evo2RMSNorm, optionally with the residual add and an fp8 epilogue:
 *   s = bf16(x + residual)                     (when residual != NULL; written to s_out)
 *   y = bf16(w * bf16(s / bf16(bf16(bf16(||s||_2) * H^-1/2) + eps)))
 *   q = e4m3fn(clamp(y / q_scale[0], -448, 448))   (when q != NULL)
 * eps sits outside the sqrt.  y may be NULL when q is given (the row only
 * feeds the fp8 in_proj).  Rows have unit element stride.
 *
 *   x, residual, y, s_out  (T, H) bf16, row strides sx, sr, sy, ss
 *   weight (H,) bf16;  q (T, H) e4m3 bytes, row stride sq (bytes)
 *
 * Replaces triton_norm.rms_norm / _norm_kernel (evo2_flash/triton_norm.py:70-156)
 * behind Evo2RMSNorm.forward (evo2_flash/model.py:58-74), plus the activation
 * quantisation of the static fp8 in_proj (evo2_flash/fp8_emul.py:76-78).
 */
int evo2_rms_norm(const void *x, int64_t sx, const void *residual, int64_t sr,
                  const void *weight, float eps, void *y, int64_t sy,
                  void *s_out, int64_t ss, const float *q_scale, void *q, int64_t sq,
                  int64_t T, int64_t H, void *stream);

/*
 * Speculative verification of the inner FIR (K = 7 or 128): each request r
 * runs tokens [starts[r], ends[r]) of x (at most Q of them) from the snapshot
 * ins[r][accepted[r] - 1], writes y for those rows (x's dtype) and, after
 * each token pos, the whole window to block outs[r][pos] (skipped when that
 * is the null block or outside the pool).  With starts = ends = accepted =
 * NULL and Q = 1 it is the one-token step: request r is row r, reading
 * ins[r] and writing outs[r].  Summation order, rounding and the absence of
 * FMA follow the reference kernel.
 *
 * Replaces triton_verifier._fir_kernel, fir_snapshots and fir_one
 * (evo2_flash/triton_verifier.py:46-80, 125-135, 157-167).
 *
 *   x          (T, H) bf16 (x_f32 = 0) or fp32, strides xs0, xs1
 *   w          (H, K) bf16 taps, strides w0, w1
 *   state      (blocks, H, K-1) fp32 view, strides ss0, ss1, ss2
 *   ins, outs  (nreq, Q) int32 block ids, strides is0/is1, os0/os1 (the same
 *              Q columns in both)
 *   starts, ends, accepted  (nreq,) int64, or all NULL
 *   y          (T, H) output, x's dtype, row stride ys0, unit column stride
 *   Rows at or past T are never read or written, whatever the tables say.
 */
int evo2_fir_verify(const void *x, int64_t xs0, int64_t xs1, int32_t x_f32,
                    const void *w, int64_t w0, int64_t w1, int32_t K,
                    float *state, int64_t ss0, int64_t ss1, int64_t ss2,
                    const int32_t *ins, int64_t is0, int64_t is1,
                    const int32_t *outs, int64_t os0, int64_t os1, int32_t Q,
                    const int64_t *starts, const int64_t *ends, const int64_t *accepted,
                    void *y, int64_t ys0, int64_t nreq, int64_t T, int64_t H,
                    int32_t null_block, int64_t num_blocks, void *stream);

/*
 * The same for the LI operator: s = s * poles + x (separate multiply and
 * add), each token's 16-state snapshot written to outs[r][pos], y = the
 * halving-tree readout of residues * s.  poles = exp(log_poles).
 *
 * Replaces triton_verifier._iir_kernel, iir_snapshots and iir_one
 * (evo2_flash/triton_verifier.py:83-122, 146-155, 170-178).
 *
 *   poles, residues  (H, 16) fp32, strides p0/p1, r0/r1 (unit state stride,
 *                    16-byte aligned rows)
 *   state            (blocks, H, 16) fp32 view, any strides (16-byte aligned
 *                    contiguous rows take the vector path; the speculative
 *                    layout's 17-column rows, mixers.py:892-900, the other)
 *   other arguments as evo2_fir_verify.
 */
int evo2_iir_verify(const void *x, int64_t xs0, int64_t xs1, int32_t x_f32,
                    const float *poles, int64_t p0, int64_t p1,
                    const float *residues, int64_t r0, int64_t r1,
                    float *state, int64_t ss0, int64_t ss1, int64_t ss2,
                    const int32_t *ins, int64_t is0, int64_t is1,
                    const int32_t *outs, int64_t os0, int64_t os1, int32_t Q,
                    const int64_t *starts, const int64_t *ends, const int64_t *accepted,
                    void *y, int64_t ys0, int64_t nreq, int64_t T, int64_t H,
                    int32_t null_block, int64_t num_blocks, void *stream);

/*
 * Accepted counts of the previous speculative step from the position stamps
 * (slice 2 row 0 last column of every state block: the tokens its snapshot
 * represents).  For r < nreq: offset = computed[r] - stamps[slots[r * si0] * ss],
 * accepted[r] = clamp(offset, 0, num_spec) + 1.  A request whose block is
 * not the null block (0) with offset outside [0, num_spec], or with
 * counts[r] != offset + 1 when counts is not NULL, adds one to *faults
 * (int64), as does a block outside [0, num_blocks) (its stamp is not read).
 * slots NULL puts every request on the null block.
 *   stamps fp32, stride ss (elements); slots, computed, counts int32;
 *   accepted (nreq,) int64 out.
 *
 * Replaces the stamp lookup and check of the reference's speculative decode
 * (evo2_flash/mixers.py:960-999), whose device-side assert aborts the process
 * on ROCm; faults are counted instead.
 */
int evo2_spec_accepted(const float *stamps, int64_t ss, int64_t num_blocks,
                       const int32_t *slots, int64_t si0, const int32_t *computed,
                       const int32_t *counts, int num_spec, int64_t nreq,
                       int64_t *accepted, void *faults, void *stream);

/*
 * Stamps of the snapshots a step wrote.  Decode request r < nreq (query
 * length qsl[r+1] - qsl[r], computed[r] tokens before the step) stamps
 * block slots[r * si0 + (out_col[r] + p) * si1] with computed[r] + p + 1 for
 * p < min(width, query length) (out_col NULL: column p); prefill block
 * prefill_blocks[j] gets seq_lens[j], j < npf.  The null block, blocks
 * outside [0, num_blocks) and columns outside [0, ncols) are not written;
 * slots NULL writes no decode stamp.  All index arrays int32.
 *
 * Replaces the reference's stamp recording (evo2_flash/mixers.py:1049-1074).
 */
int evo2_spec_record_stamps(float *stamps, int64_t ss, int64_t num_blocks,
                            const int32_t *slots, int64_t si0, int64_t si1, int64_t ncols,
                            const int32_t *out_col, const int32_t *qsl,
                            const int32_t *computed, int64_t nreq, int64_t width,
                            const int32_t *prefill_blocks, const int32_t *seq_lens,
                            int64_t npf, void *stream);

/*
 * Per-step verify plan of nreq speculative decode requests, one launch:
 *   ins, outs  (nreq, width) int32: the input and output snapshot blocks of
 *              position p.  With both block pointers (prev, sched: prefix
 *              caching's block columns of the previous step's and this
 *              step's last scheduled token) slot-row columns prev[r] + p and
 *              sched[r] + p, else column p for both.  A column outside
 *              [0, ncols), and every entry when null_all != 0, is block 0.
 *   starts, ends (nreq,) int64: packed rows [qsl[r], qsl[r+1]) (qsl NULL:
 *              one row per request, [r, r + 1)).
 *   acc        (nreq,) int64: max(eng_acc[r], 1), or 1 with eng_acc NULL.
 * slots (nreq, ncols) int32 at element strides si0, si1; qsl (nreq + 1,),
 * prev, sched, eng_acc (nreq,) int32 or NULL (prev and sched together).
 *
 * Replaces the reference's decode-request plumbing (evo2_flash/mixers.py:
 * 431-541: accepted counts, cache-all slot windows, the packed row range and
 * the null-block rule for profiling-sized pools).
 */
int evo2_spec_plan(const int32_t *slots, int64_t si0, int64_t si1, int64_t ncols,
                   const int32_t *qsl, const int32_t *prev, const int32_t *sched,
                   const int32_t *eng_acc, int64_t nreq, int64_t width, int32_t null_all,
                   int32_t *ins, int32_t *outs, int64_t *starts, int64_t *ends, int64_t *acc,
                   void *stream);

/*
 * Align-mode repair of resumed prefill states, two launches.  Prefill row
 * j < npf (has_init[j] nonzero) continues from need[j] computed tokens in
 * block dst[j]; when dst[j]'s position stamp (stamps[b * ss]) is not need[j]
 * and block src[j]'s is, all three state slices of src[j] are copied over
 * dst[j].  Rows on the null block, blocks outside [0, num_blocks) and
 * dst == src are left alone.  A row whose source is another repaired row's
 * destination, or whose destination another repaired row also writes, is
 * not repaired and adds one to *faults (int64).  take (npf,) int32 is the
 * caller's workspace (the block each row copies from, -1 for none).
 * Slice k: slice_ptr[k] base of the (blocks, d1, d2) view, element strides
 * slice_strides[3k .. 3k+2], dims slice_dims[2k], slice_dims[2k+1], element
 * size slice_es[k] (2 or 4 bytes).  The pointer and size arrays are host
 * memory.
 *
 * Replaces the reference's _repair_resumed_prefill_state
 * (evo2_flash/mixers.py:1001-1037), which copies every prefill row's state
 * over itself or its source each step.
 */
int evo2_spec_repair_prefill(const float *stamps, int64_t ss, int64_t num_blocks,
                             const int32_t *dst, const int32_t *src, const int32_t *need,
                             const uint8_t *has_init, int64_t npf, int32_t *take,
                             void *faults, void *const *slice_ptr,
                             const int64_t *slice_strides, const int64_t *slice_dims,
                             const int32_t *slice_es, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* EVO2_HYENA_H */
