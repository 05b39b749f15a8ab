"""ctypes binding of libevo2_hyena.so, the C ABI declared in include/evo2_hyena.h.

The library is loaded after torch so that its HIP runtime dependency
(soname libamdhip64.so.7) resolves to the runtime torch already mapped: a
`hipStream_t` taken from torch is then valid inside the library.  There is no
fallback: if the library is missing or fails to load, every operator raises.
"""

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load, see above)

from .build import LIB_PATH

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_p = ctypes.c_void_p
_c_f = ctypes.c_float

# name -> argtypes, in the order of include/evo2_hyena.h
SIGNATURES = {
    "evo2_last_error": [],
    "evo2_abi_version": [],
    "evo2_hyena_decode": [
        _c_p, _c_i64, _c_p,                       # z, sz, short_w
        _c_p, _c_i64, _c_i64, _c_i64,             # conv_state + strides
        _c_p, _c_i64,                             # slots, ssl
        _c_p, _c_i64, _c_i64,                     # inner + strides
        _c_p, _c_i64, _c_i64,                     # log_poles + strides
        _c_p, _c_i64, _c_i64, _c_i64,             # inner_state + strides
        _c_p, _c_p, _c_i64,                       # D, out, so
        _c_i64, _c_i64, _c_i32, _c_i32,           # B, H, K, is_iir
        _c_i32, _c_i64, _c_p,                     # null_block, num_blocks, stream
    ],
    "evo2_fir_prefill": [
        _c_p, _c_i64, _c_p, _c_i64, _c_i64,       # u, su, w, w0, w1
        _c_i32, _c_p, _c_i64, _c_i64, _c_i64,     # K, state + strides
        _c_p, _c_i64, _c_p, _c_i64,               # seq_table, nseq, blocks, sblk
        _c_p, _c_i64, _c_i32,                     # tile_table, ntiles, block_t
        _c_p, _c_i64, _c_i64, _c_i64,             # out, so, T, H
        _c_i64, _c_p,                             # num_blocks, stream
    ],
    "evo2_hyena_fir_prefill": [
        _c_p, _c_i64, _c_p,                       # z, sz, short_w
        _c_p, _c_i64, _c_i64, _c_i64,             # conv_state + strides
        _c_p, _c_i64, _c_i64, _c_i32,             # w, w0, w1, K
        _c_p, _c_i64, _c_i64, _c_i64,             # inner_state + strides
        _c_p,                                     # D
        _c_p, _c_i64, _c_p, _c_i64,               # seq_table, nseq, blocks, sblk
        _c_p, _c_i64, _c_i32,                     # tile_table, ntiles, block_t
        _c_p, _c_i64, _c_i64, _c_i64,             # out, so, T, H
        _c_i64, _c_p,                             # num_blocks, stream
    ],
    "evo2_hcl_workspace_bytes": [_c_i64, _c_i64],
    "evo2_hyena_hcl_prefill": [
        _c_p, _c_i64, _c_p,                       # z, sz, short_w
        _c_p, _c_i64, _c_i64, _c_i64,             # conv_state + strides
        _c_p, _c_i64, _c_i64,                     # residues + strides
        _c_p, _c_i64, _c_i64,                     # log_poles + strides
        _c_p, _c_i64, _c_i64, _c_i64,             # ssm + strides
        _c_p,                                     # D
        _c_p, _c_i64, _c_p, _c_i64,               # seq_table, nseq, blocks, sblk
        _c_p, _c_i64, _c_p, _c_i32,               # tile_table, ntiles, tile_start, block_t
        _c_p, _c_i64,                             # workspace, bytes
        _c_p, _c_i64, _c_i64, _c_i64,             # out, so, T, H
        _c_i64, _c_p,                             # num_blocks, stream
    ],
    "evo2_hyena_hcl_prefill_noalloc": [
        _c_p, _c_i64, _c_p,                       # z, sz, short_w
        _c_p, _c_i64, _c_i64, _c_i64,             # conv_state + strides
        _c_p, _c_i64, _c_i64,                     # residues + strides
        _c_p, _c_i64, _c_i64,                     # log_poles + strides
        _c_p, _c_i64, _c_i64, _c_i64,             # ssm + strides
        _c_p,                                     # D
        _c_p, _c_i64, _c_p, _c_i64,               # seq_table, nseq, blocks, sblk
        _c_p, _c_i64, _c_p, _c_i32,               # tile_table, ntiles, tile_start, block_t
        _c_p, _c_i64, _c_i64, _c_i64,             # out, so, T, H
        _c_i64, _c_p,                             # num_blocks, stream
    ],
    "evo2_iir_segment": [
        _c_p, _c_i64, _c_i64,                     # seq + strides
        _c_p, _c_i64, _c_i64,                     # residues + strides
        _c_p, _c_i64, _c_i64,                     # log_poles + strides
        _c_p, _c_i64, _c_i64,                     # s_prev + strides
        _c_p, _c_i64, _c_i64, _c_p,               # y + strides, st
        _c_p, _c_i64,                             # workspace, bytes
        _c_i64, _c_i64, _c_i32, _c_p,             # H, L, block_t, stream
    ],
    "evo2_iir_final_state": [
        _c_p, _c_i64, _c_i64,                     # seq + strides
        _c_p, _c_i64, _c_i64, _c_p,               # log_poles + strides, st
        _c_p, _c_i64,                             # workspace, bytes
        _c_i64, _c_i64, _c_i32, _c_p,             # H, L, block_t, stream
    ],
    "evo2_hcl_compute_filter": [
        _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64,  # residues, log_poles + strides
        _c_p, _c_i64, _c_p, _c_i64, _c_i64,           # t, st, h + strides
        _c_i64, _c_i64, _c_i64, _c_p,                 # D, S, L, stream
    ],
    "evo2_causal_conv1d_update": [
        _c_p, _c_i64, _c_i64,                     # x + strides (row, channel)
        _c_p, _c_i64, _c_i64, _c_i64,             # conv_state + strides
        _c_p, _c_i64, _c_i64, _c_i32,             # w + strides, K
        _c_p, _c_i32,                             # bias, activation
        _c_p, _c_i64, _c_i32,                     # indices, stride, pad_slot_id
        _c_p, _c_i64, _c_i64,                     # out + strides (row, channel)
        _c_i64, _c_i64, _c_i64, _c_p,             # B, dim, num_blocks, stream
    ],
    "evo2_causal_conv1d_update_spec": [
        _c_p, _c_i64, _c_i64,                     # x + strides (row, channel)
        _c_p, _c_i64, _c_i64, _c_i64, _c_i32,     # conv_state + strides, state_len
        _c_p, _c_i64, _c_i64, _c_i32,             # w + strides, K
        _c_p, _c_i32,                             # bias, activation
        _c_p, _c_i64, _c_i64, _c_i32,             # slot matrix + strides, columns
        _c_p, _c_p, _c_p, _c_p,                   # in_col, out_col, num_accepted, qsl
        _c_i32, _c_i32,                           # max_query_len, pad_slot_id
        _c_p, _c_i64, _c_i64,                     # out + strides (row, channel)
        _c_i64, _c_i64, _c_i64, _c_i64, _c_p,     # nreq, T, dim, num_blocks, stream
    ],
    "evo2_causal_conv1d_fn": [
        _c_p, _c_i64, _c_i64,                     # x + strides (channel, row)
        _c_p, _c_i64, _c_i64, _c_i32,             # w + strides, K
        _c_p, _c_i32,                             # bias, activation
        _c_p, _c_i64, _c_i64, _c_i64,             # conv_states + strides
        _c_p,                                     # has_initial_state
        _c_p, _c_i64, _c_i32,                     # cache_indices, stride, pad_slot_id
        _c_p, _c_i64,                             # query_start_loc, nseq
        _c_p, _c_i64, _c_i64,                     # out + strides (channel, row)
        _c_i64, _c_i64, _c_i64, _c_p,             # T, dim, num_blocks, stream
    ],
    "evo2_decode_attention_workspace_bytes": [_c_i64, _c_i64, _c_i64, _c_i64],
    "evo2_decode_attention": [
        _c_p, _c_i64, _c_i64,                     # q + strides (b, h)
        _c_p, _c_i64, _c_i64, _c_i64,             # k + strides (b, h, d)
        _c_p, _c_i64, _c_i64, _c_i64,             # v + strides (b, h, l)
        _c_p, _c_p, _c_i64,                       # positions, workspace, bytes
        _c_p, _c_i64, _c_i64,                     # out + strides (b, h)
        _c_i64, _c_i64, _c_i64, _c_i64, _c_f, _c_p,  # B, heads, head_dim, L, scale, stream
    ],
    "evo2_paged_decode_attention": [
        _c_p, _c_i64, _c_i64,                     # q + strides (b, h)
        _c_p, _c_i64, _c_i64, _c_i64,             # key pages + strides (page, h, d)
        _c_p, _c_i64, _c_i64, _c_i64,             # value pages + strides (page, h, l)
        _c_i64,                                   # num_pages
        _c_p, _c_i64,                             # block table, row stride
        _c_i64,                                   # shared_pages
        _c_p, _c_p, _c_i64,                       # positions, workspace, bytes
        _c_p, _c_i64, _c_i64,                     # out + strides (b, h)
        _c_i64, _c_i64, _c_i64, _c_i64, _c_f, _c_p,  # B, heads, head_dim, max_pages, scale, stream
    ],
    "evo2_prefill_attention": [
        _c_p, _c_p, _c_p, _c_p,                   # q, k, vt, out
        _c_i64, _c_i64, _c_i64, _c_i64, _c_f, _c_p,  # N, heads, L, head_dim, scale, stream
    ],
    "evo2_fp8_quantize": [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p],
    "evo2_rms_norm": [
        _c_p, _c_i64, _c_p, _c_i64,               # x, sx, residual, sr
        _c_p, _c_f, _c_p, _c_i64,                 # weight, eps, y, sy
        _c_p, _c_i64, _c_p, _c_p, _c_i64,         # s_out, ss, q_scale, q, sq
        _c_i64, _c_i64, _c_p,                     # T, H, stream
    ],
    "evo2_fp8_gemm": [
        _c_p, _c_i64, _c_p, _c_i64,               # x8, sx, w8, sw
        _c_p, _c_p, _c_p,                         # x_scale, w_scale, bias
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64,     # out, so, M, N, K
        _c_p,                                     # stream
    ],
    "evo2_fp8_pack_weight": [
        _c_p, _c_i64, _c_p, _c_i64, _c_i64,       # w8, sw, wp, N, K
        _c_p,                                     # stream
    ],
    "evo2_fp8_gemm_packed": [
        _c_p, _c_i64, _c_p,                       # x8, sx, wp
        _c_p, _c_p, _c_p,                         # x_scale, w_scale, bias
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64,     # out, so, M, N, K
        _c_p,                                     # stream
    ],
    "evo2_fp8_gemm_persist_order": [_c_i64, _c_i64, ctypes.c_int, _c_p, _c_p],
    "evo2_fp8_fast_accum_gemm": [
        _c_p, _c_i64, _c_p, _c_i64,               # a8, sa, b_t, sb
        _c_p, _c_p,                               # input_scale, weight_scale
        _c_p, _c_i64, _c_i32,                     # out, so, out_f32
        _c_i64, _c_i64, _c_i64, _c_p,             # N, M, K, stream
    ],
    "evo2_fir_verify": [
        _c_p, _c_i64, _c_i64, _c_i32,             # x, xs0, xs1, x_f32
        _c_p, _c_i64, _c_i64, _c_i32,             # w, w0, w1, K
        _c_p, _c_i64, _c_i64, _c_i64,             # state + strides
        _c_p, _c_i64, _c_i64,                     # ins + strides
        _c_p, _c_i64, _c_i64, _c_i32,             # outs + strides, Q
        _c_p, _c_p, _c_p,                         # starts, ends, accepted
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64,     # y, ys0, nreq, T, H
        _c_i32, _c_i64, _c_p,                     # null_block, num_blocks, stream
    ],
    "evo2_iir_verify": [
        _c_p, _c_i64, _c_i64, _c_i32,             # x, xs0, xs1, x_f32
        _c_p, _c_i64, _c_i64,                     # poles + strides
        _c_p, _c_i64, _c_i64,                     # residues + strides
        _c_p, _c_i64, _c_i64, _c_i64,             # state + strides
        _c_p, _c_i64, _c_i64,                     # ins + strides
        _c_p, _c_i64, _c_i64, _c_i32,             # outs + strides, Q
        _c_p, _c_p, _c_p,                         # starts, ends, accepted
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64,     # y, ys0, nreq, T, H
        _c_i32, _c_i64, _c_p,                     # null_block, num_blocks, stream
    ],
    "evo2_spec_accepted": [
        _c_p, _c_i64, _c_i64,                     # stamps, stride, num_blocks
        _c_p, _c_i64, _c_p, _c_p,                 # slots, si0, computed, counts
        _c_i32, _c_i64, _c_p, _c_p, _c_p,         # num_spec, nreq, accepted, faults, stream
    ],
    "evo2_spec_record_stamps": [
        _c_p, _c_i64, _c_i64,                     # stamps, stride, num_blocks
        _c_p, _c_i64, _c_i64, _c_i64,             # slots + strides, ncols
        _c_p, _c_p, _c_p, _c_i64, _c_i64,         # out_col, qsl, computed, nreq, width
        _c_p, _c_p, _c_i64, _c_p,                 # prefill_blocks, seq_lens, npf, stream
    ],
    "evo2_spec_plan": [
        _c_p, _c_i64, _c_i64, _c_i64,             # slots + strides, ncols
        _c_p, _c_p, _c_p, _c_p,                   # qsl, prev, sched, eng_acc
        _c_i64, _c_i64, _c_i32,                   # nreq, width, null_all
        _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,       # ins, outs, starts, ends, acc, stream
    ],
    "evo2_spec_repair_prefill": [
        _c_p, _c_i64, _c_i64,                     # stamps, stride, num_blocks
        _c_p, _c_p, _c_p, _c_p, _c_i64,           # dst, src, need, has_init, npf
        _c_p, _c_p,                               # take, faults
        _c_p, _c_p, _c_p, _c_p, _c_p,             # slice pointers, strides, dims, sizes, stream
    ],
}

RESTYPES = {"evo2_last_error": ctypes.c_char_p, "evo2_hcl_workspace_bytes": ctypes.c_int64,
            "evo2_decode_attention_workspace_bytes": ctypes.c_int64,
            "evo2_fp8_gemm_persist_order": ctypes.c_int64}

_lock = threading.Lock()
_lib = None


class Evo2Error(RuntimeError):
    """A nonzero status from the C ABI."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


def _hip_runtimes_mapped():
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line}
    except OSError:
        return set()


def lib():
    """The loaded library (loaded on first use).  Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m evo2_flash_amd.build` "
                "(or __graft_entry__.build()) first")
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise RuntimeError(f"more than one HIP runtime is mapped: {sorted(runtimes)}")
        _lib = handle
        return _lib


def call(name, *args):
    """Call a C-ABI entry point; raise Evo2Error on a nonzero status."""
    l = lib()
    rc = getattr(l, name)(*args)
    if rc != 0:
        msg = l.evo2_last_error().decode(errors="replace")
        raise Evo2Error(name, rc, msg)


def ptr(t):
    """Device pointer of a tensor (None for None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t=None):
    """The current torch stream on t's device, as a void* for the C ABI."""
    dev = t.device if t is not None else None
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def require_device(*tensors):
    """The HIP path runs on ROCm devices only: raise for CPU tensors."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "evo2_flash_amd operators run on the GPU only (got a CPU tensor); "
                "there is no CPU fallback")
