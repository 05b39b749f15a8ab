// Single-pass ("stripe") prefill of the hcm and hcl mixer cores: a workgroup
// sweeps a channel stripe row by row with its filter state in LDS and
// registers.  hcl: 16 channels of a whole segment, so the LI scan carries
// its state inside the workgroup (no carry pass, z read once).  hcm: 32
// channels of one tile, the 128-tap history rebuilt from the 256 rows
// before it.  Kernels: prefill_stripe.hip.  The entry points of
// prefill_fir.hip and prefill_hcl.hip take this path when the tile table
// and the layout allow it.
#pragma once

#include "common.h"

namespace evo2 {

struct StripeArgs {
  const bf16_t *z; int64_t sz;              // (T, 3H) in_proj rows, unit column stride
  const bf16_t *ws;                         // (3H, 3) short taps, contiguous
  const bf16_t *cs; int64_t cs0, cs1, cs2;  // conv window view (blocks, 3H, 2), read only
  const bf16_t *w; int64_t w0;              // hcm: inner taps (H, 128), unit tap stride
  const float *st; int64_t st0, st1, st2;   // hcm: inner window view (blocks, H, >=127), read only
  const float *res; int64_t r0, r1;         // hcl: residues (H, 16)
  const float *lp; int64_t l0, l1;          // hcl: log-poles (H, 16)
  float *ssm; int64_t m0, m1, m2;           // hcl: LI state view (blocks, H, 16), written
  const bf16_t *D;                          // (H,) or null (hcm only)
  bf16_t *out; int64_t so;                  // g (T, H)
  const int32_t *seq; int64_t nseq;         // (nseq, 3) [start, end, has_init]
  const int32_t *blocks; int64_t sblk;
  const int32_t *tiles; int64_t ntiles;     // hcm: (ntiles, 2) [segment, first row]
  int block_t;                              // hcm: rows per tile
  int H;
  int64_t num_blocks;
};

enum StripeKind { STRIPE_HCM = 0, STRIPE_HCL = 1 };

// True when the single-pass kernels can take this launch: hcl with every
// segment one tile (block_t >= T) and H a multiple of 16; hcm with tiles of
// at least 256 rows and H a multiple of 32; z and out 16-byte addressable
// with row strides that keep a step's byte offsets in 32 bits.
bool stripe_supported(const StripeArgs &a, StripeKind kind, int64_t T, int64_t block_t);

// Enqueues the single-pass kernel of `kind` (the conv and FIR windows are
// left to the callers' window kernels; hcl writes the final LI state).
int launch_stripe(const StripeArgs &a, StripeKind kind, hipStream_t st);

}  // namespace evo2
