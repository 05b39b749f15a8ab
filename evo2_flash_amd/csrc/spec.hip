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
#include <algorithm>

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

// ---------------------------------------------------------------------------
// Per-step verify plan of the decode requests: one launch produces everything
// the snapshot operators need besides the stamp-derived accepted counts.
// Thread (r, p), p < width: ins[r][p], outs[r][p] are the request's input and
// output snapshot blocks at position p: with prefix caching's block pointers
// (prev[r], sched[r]) the slot-row columns prev[r] + p and sched[r] + p, else
// column p of the slot row for both (mixers.py:444-456); a column outside the
// row, or every entry when `null_all` (a profiling-sized pool holding fewer
// blocks than the slot matrix names, mixers.py:527-541), is the null block.
// Thread (r, 0) also writes the request's packed row range [qsl[r], qsl[r+1])
// (one row per request without qsl) and the engine's accepted count,
// max(eng_acc[r], 1), or 1 without one (mixers.py:431-441).
struct SpecPlanArgs {
  const int32_t *slots; int64_t si0, si1; int ncols;
  const int32_t *qsl;       // (nreq + 1,) or null
  const int32_t *prev;      // (nreq,) or null
  const int32_t *sched;     // (nreq,) or null
  const int32_t *eng_acc;   // (nreq,) or null
  int32_t *ins, *outs;      // (nreq, width)
  int64_t *starts, *ends, *acc;  // (nreq,)
  int nreq, width;
  bool null_all;
};

__global__ __launch_bounds__(256) void spec_plan_kernel(SpecPlanArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(a.nreq) * a.width) return;
  const int r = static_cast<int>(i / a.width), p = static_cast<int>(i % a.width);
  const bool paged = a.prev && a.sched;
  auto column = [&](int base) -> int32_t {
    const int c = base + p;
    if (a.null_all || c < 0 || c >= a.ncols) return 0;
    return a.slots[r * a.si0 + static_cast<int64_t>(c) * a.si1];
  };
  a.ins[i] = column(paged ? a.prev[r] : 0);
  a.outs[i] = column(paged ? a.sched[r] : 0);
  if (p == 0) {
    a.starts[r] = a.qsl ? a.qsl[r] : r;
    a.ends[r] = a.qsl ? a.qsl[r + 1] : r + 1;
    a.acc[r] = a.eng_acc ? max(a.eng_acc[r], 1) : 1;
  }
}

// ---------------------------------------------------------------------------
// Align-mode repair of resumed prefill states (mixers.py:1001-1040).  Prefill
// row j continues from need[j] computed tokens in block dst[j]; when dst[j]'s
// stamp is not need[j] but block src[j]'s is, src[j]'s three slices replace
// dst[j]'s.  Decide: one thread per row writes take[j] (the block to copy
// from, or -1 for no copy).  Copies happen in a second launch, so no row's
// decision reads a stamp another row's copy already changed.  A row whose
// source is another repaired row's destination, or whose destination another
// repaired row also writes, is not repaired (the copy order would decide its
// result) and counts as a stamp fault.
struct SpecRepairArgs {
  const float *stamps; int64_t ss; int64_t num_blocks;
  const int32_t *dst, *src, *need;  // (npf,)
  const uint8_t *has_init;          // (npf,) bool
  int32_t *take;                    // (npf,) out
  unsigned long long *faults;
  int npf;
};

__device__ __forceinline__ bool repair_wanted(const SpecRepairArgs &a, int j) {
  const int64_t d = a.dst[j], s = a.src[j];
  if (!a.has_init[j] || d <= 0 || s <= 0 || d >= a.num_blocks || s >= a.num_blocks || d == s)
    return false;
  const float n = static_cast<float>(a.need[j]);
  return a.stamps[d * a.ss] != n && a.stamps[s * a.ss] == n;
}

__global__ __launch_bounds__(256) void spec_repair_plan_kernel(SpecRepairArgs a) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= a.npf) return;
  int32_t take = -1;
  if (repair_wanted(a, j)) {
    bool clash = false;
    for (int k = 0; k < a.npf && !clash; ++k) {
      if (k == j || !repair_wanted(a, k)) continue;
      clash = a.dst[k] == a.src[j] || a.dst[k] == a.dst[j];
    }
    if (clash) atomicAdd(a.faults, 1ull);
    else take = a.src[j];
  }
  a.take[j] = take;
}

// One slice of a block: (d1, d2) elements of `es` bytes at element strides
// (s0 between blocks, s1, s2).
struct StateSlice {
  char *base; int64_t s0, s1, s2; int d1, d2, es;
};
struct SpecCopyArgs {
  StateSlice sl[3];
  const int32_t *dst, *take;
  int npf;
};

// grid (element chunks, prefill row, slice): copy block take[j] over dst[j]
// where take[j] >= 0.
__global__ __launch_bounds__(256) void spec_repair_copy_kernel(SpecCopyArgs a) {
  const int j = blockIdx.y;
  const int32_t from = a.take[j];
  if (from < 0) return;
  const StateSlice &s = a.sl[blockIdx.z];
  const int64_t n = static_cast<int64_t>(s.d1) * s.d2;
  const int64_t to = a.dst[j];
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t i1 = e / s.d2, i2 = e - i1 * s.d2;
    const int64_t off = i1 * s.s1 + i2 * s.s2;
    char *d = s.base + (to * s.s0 + off) * s.es;
    const char *f = s.base + (static_cast<int64_t>(from) * s.s0 + off) * s.es;
    if (s.es == 4) *reinterpret_cast<uint32_t *>(d) = *reinterpret_cast<const uint32_t *>(f);
    else *reinterpret_cast<uint16_t *>(d) = *reinterpret_cast<const uint16_t *>(f);
  }
}

}  // namespace evo2

using namespace evo2;

extern "C" int evo2_spec_plan(const int32_t *slots, int64_t si0, int64_t si1, int64_t ncols,
                              const int32_t *qsl, const int32_t *prev, const int32_t *sched,
                              const int32_t *eng_acc, int64_t nreq, int64_t width,
                              int32_t null_all, int32_t *ins, int32_t *outs, int64_t *starts,
                              int64_t *ends, int64_t *acc, void *stream) {
  if (nreq < 0 || width < 1 || ncols < 1 || ncols > 0x7fffffff || nreq * width > 0x7fffffffLL)
    return fail(EVO2_ERR_INVALID, "spec_plan: bad sizes nreq=%lld width=%lld ncols=%lld",
                (long long)nreq, (long long)width, (long long)ncols);
  if (nreq == 0) return EVO2_OK;
  if (!slots || !ins || !outs || !starts || !ends || !acc)
    return fail(EVO2_ERR_INVALID, "spec_plan: null pointer argument");
  if ((prev == nullptr) != (sched == nullptr))
    return fail(EVO2_ERR_INVALID, "spec_plan: block pointers come in pairs (previous and scheduled)");
  SpecPlanArgs a{slots, si0, si1, static_cast<int>(ncols), qsl, prev, sched, eng_acc, ins, outs,
                 starts, ends, acc, static_cast<int>(nreq), static_cast<int>(width), null_all != 0};
  hipLaunchKernelGGL(spec_plan_kernel, dim3(static_cast<unsigned>(cdiv(nreq * width, 256))), dim3(256),
                     0, static_cast<hipStream_t>(stream), a);
  return check_launch("spec_plan");
}

extern "C" int evo2_spec_repair_prefill(const float *stamps, int64_t ss, int64_t num_blocks,
                                        const int32_t *dst, const int32_t *src,
                                        const int32_t *need, const uint8_t *has_init,
                                        int64_t npf, int32_t *take, void *faults,
                                        void *const *slice_ptr, const int64_t *slice_strides,
                                        const int64_t *slice_dims, const int32_t *slice_es,
                                        void *stream) {
  if (npf < 0 || npf > 65535 || num_blocks < 0)
    return fail(EVO2_ERR_INVALID, "spec_repair_prefill: bad sizes npf=%lld blocks=%lld",
                (long long)npf, (long long)num_blocks);
  if (npf == 0) return EVO2_OK;
  if (!stamps || !dst || !src || !need || !has_init || !take || !faults || !slice_ptr ||
      !slice_strides || !slice_dims || !slice_es)
    return fail(EVO2_ERR_INVALID, "spec_repair_prefill: null pointer argument");
  SpecCopyArgs c{};
  int64_t most = 0;
  for (int k = 0; k < 3; ++k) {
    const int es = slice_es[k];
    if (!slice_ptr[k] || (es != 2 && es != 4) || slice_dims[2 * k] < 1 || slice_dims[2 * k + 1] < 1 ||
        slice_dims[2 * k] > 0x7fffffff || slice_dims[2 * k + 1] > 0x7fffffff)
      return fail(EVO2_ERR_INVALID, "spec_repair_prefill: slice %d is not a (blocks, d1, d2) view of "
                  "2- or 4-byte elements", k);
    c.sl[k] = StateSlice{static_cast<char *>(slice_ptr[k]), slice_strides[3 * k], slice_strides[3 * k + 1],
                         slice_strides[3 * k + 2], static_cast<int>(slice_dims[2 * k]),
                         static_cast<int>(slice_dims[2 * k + 1]), es};
    most = std::max<int64_t>(most, slice_dims[2 * k] * slice_dims[2 * k + 1]);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  SpecRepairArgs a{stamps, ss, num_blocks, dst, src, need, has_init, take,
                   static_cast<unsigned long long *>(faults), static_cast<int>(npf)};
  hipLaunchKernelGGL(spec_repair_plan_kernel, dim3(static_cast<unsigned>(cdiv(npf, 256))), dim3(256), 0, st, a);
  int rc = check_launch("spec_repair_prefill (decide)");
  if (rc) return rc;
  c.dst = dst;
  c.take = take;
  c.npf = static_cast<int>(npf);
  const unsigned gx = static_cast<unsigned>(std::min<int64_t>(cdiv(most, 256), 1024));
  hipLaunchKernelGGL(spec_repair_copy_kernel, dim3(gx, static_cast<unsigned>(npf), 3), dim3(256), 0, st, c);
  return check_launch("spec_repair_prefill (copy)");
}

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
