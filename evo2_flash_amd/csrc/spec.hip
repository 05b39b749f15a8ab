// Position stamps of speculative decode: which state snapshot of a request
// is live, and the stamps of the snapshots a step writes.
//
// Every state block carries, in slice 2 row 0 last column, the number of
// tokens its snapshot represents (fp32, exact below 2^24).  A verify step
// reads the snapshot of the previous step's last accepted token, found as
// column computed - stamp(column 0) of the request's slot row (mixers.py:
// 960-999), and stamps every snapshot it writes: column p of a request that
// had computed n tokens holds n + p + 1, a prefill block its sequence length
// (mixers.py:1049-1074).  Both are a few hundred integers per step; each is
// one launch here instead of a chain of small tensor operations.
#include "common.h"

namespace evo2 {

struct SpecAcceptArgs {
  const float *stamps; int64_t ss; int64_t num_blocks;  // stamp of block b at stamps[b * ss]
  const int32_t *slots; int64_t si0;                    // column 0 of request r at slots[r * si0]
  const int32_t *computed;                              // (nreq,) tokens computed before the step
  const int32_t *counts;                                // (nreq,) engine's accepted counts, or null
  int64_t *accepted;                                    // (nreq,) out
  unsigned long long *faults;                           // (1,) incremented
  int num_spec; int nreq;
};

// accepted[r] = clamp(computed[r] - stamp(slots[r, 0]), 0, num_spec) + 1.
// A request not on the null block whose offset falls outside [0, num_spec]
// (or, with counts, disagrees with the engine's count) is a fault: counted,
// and clamped like the others.  A slot outside the pool counts as a fault
// and reads no stamp.  Faults are summed per workgroup, one atomic each.
__global__ __launch_bounds__(256) void spec_accepted_kernel(SpecAcceptArgs a) {
  __shared__ int nbad[4];
  const int r = blockIdx.x * 256 + threadIdx.x;
  int bad = 0;
  if (r < a.nreq) {
    const int64_t first = a.slots ? a.slots[r * a.si0] : 0;
    const bool inside = first >= 0 && first < a.num_blocks;
    const int64_t stamp = inside ? static_cast<int64_t>(a.stamps[first * a.ss]) : 0;
    const int64_t off = static_cast<int64_t>(a.computed[r]) - stamp;
    bad = !inside || (first != 0 && (off < 0 || off > a.num_spec));
    if (a.counts && inside && first != 0 && static_cast<int64_t>(a.counts[r]) != off + 1) bad = 1;
    a.accepted[r] = (off < 0 ? 0 : off > a.num_spec ? a.num_spec : off) + 1;
  }
  // workgroup sum of the fault flags: wave ballots, then one atomic
  const unsigned long long ballot = __ballot(bad);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) nbad[wave] = __popcll(ballot);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int n = nbad[0] + nbad[1] + nbad[2] + nbad[3];
    if (n) atomicAdd(a.faults, static_cast<unsigned long long>(n));
  }
}

struct SpecRecordArgs {
  float *stamps; int64_t ss; int64_t num_blocks;
  const int32_t *slots; int64_t si0, si1; int ncols;  // (nreq, ncols) slot rows, or null
  const int32_t *out_col;                             // (nreq,) first written column, or null (0)
  const int32_t *qsl;                                 // (nreq + 1,) packed row starts
  const int32_t *computed;                            // (nreq,)
  const int32_t *prefill_blocks;                      // (npf,)
  const int32_t *seq_lens;                            // (npf,) lengths of the prefill rows
  int nreq, width, npf;
};

// Thread i < nreq * width: request i / width, position p = i % width, active
// while p < its query length; it stamps block slots[r, out_col[r] + p] with
// computed[r] + p + 1.  Thread nreq * width + j stamps prefill block j with
// its length.  The null block (0), slots outside the pool and columns past
// the slot row are never written.
__global__ __launch_bounds__(256) void spec_record_kernel(SpecRecordArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t nd = static_cast<int64_t>(a.nreq) * a.width;
  int64_t dest = 0;
  float value = 0.f;
  if (i < nd) {
    if (!a.slots) return;
    const int r = static_cast<int>(i / a.width), p = static_cast<int>(i % a.width);
    if (p >= a.qsl[r + 1] - a.qsl[r]) return;
    const int col = (a.out_col ? a.out_col[r] : 0) + p;
    if (col < 0 || col >= a.ncols) return;
    dest = a.slots[r * a.si0 + col * a.si1];
    value = static_cast<float>(static_cast<int64_t>(a.computed[r]) + p + 1);
  } else if (i < nd + a.npf) {
    const int j = static_cast<int>(i - nd);
    dest = a.prefill_blocks[j];
    value = static_cast<float>(a.seq_lens[j]);
  } else {
    return;
  }
  if (dest <= 0 || dest >= a.num_blocks) return;
  a.stamps[dest * a.ss] = value;
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_spec_accepted(const float *stamps, int64_t ss, int64_t num_blocks,
                                  const int32_t *slots, int64_t si0, const int32_t *computed,
                                  const int32_t *counts, int num_spec, int64_t nreq,
                                  int64_t *accepted, void *faults, void *stream) {
  if (nreq < 0 || nreq > 0x7fffffff || num_spec < 0 || num_blocks < 0)
    return fail(EVO2_ERR_INVALID, "spec_accepted: bad sizes nreq=%lld num_spec=%d blocks=%lld",
                (long long)nreq, num_spec, (long long)num_blocks);
  if (nreq == 0) return EVO2_OK;
  if (!stamps || !computed || !accepted || !faults)
    return fail(EVO2_ERR_INVALID, "spec_accepted: null pointer argument");
  SpecAcceptArgs a{stamps, ss, num_blocks, slots, si0, computed, counts, accepted,
                   static_cast<unsigned long long *>(faults), num_spec, static_cast<int>(nreq)};
  hipLaunchKernelGGL(spec_accepted_kernel, dim3(static_cast<unsigned>(cdiv(nreq, 256))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("spec_accepted");
}

extern "C" int evo2_spec_record_stamps(float *stamps, int64_t ss, int64_t num_blocks,
                                       const int32_t *slots, int64_t si0, int64_t si1, int64_t ncols,
                                       const int32_t *out_col, const int32_t *qsl,
                                       const int32_t *computed, int64_t nreq, int64_t width,
                                       const int32_t *prefill_blocks, const int32_t *seq_lens,
                                       int64_t npf, void *stream) {
  if (nreq < 0 || width < 0 || npf < 0 || ncols < 0 || num_blocks < 0 ||
      nreq * width + npf > 0x7fffffffLL || ncols > 0x7fffffff)
    return fail(EVO2_ERR_INVALID, "spec_record_stamps: bad sizes nreq=%lld width=%lld npf=%lld",
                (long long)nreq, (long long)width, (long long)npf);
  const int64_t total = nreq * width + npf;
  if (total == 0) return EVO2_OK;
  if (!stamps || (nreq * width > 0 && (!qsl || !computed)) ||
      (npf > 0 && (!prefill_blocks || !seq_lens)))
    return fail(EVO2_ERR_INVALID, "spec_record_stamps: null pointer argument");
  SpecRecordArgs a{stamps, ss, num_blocks, slots, si0, si1, static_cast<int>(ncols), out_col, qsl,
                   computed, prefill_blocks, seq_lens, static_cast<int>(nreq),
                   static_cast<int>(width), static_cast<int>(npf)};
  hipLaunchKernelGGL(spec_record_kernel, dim3(static_cast<unsigned>(cdiv(total, 256))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("spec_record_stamps");
}
