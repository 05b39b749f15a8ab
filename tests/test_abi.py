"""The C ABI without a GPU: the built library loads, exports every entry point
include/evo2_hyena.h declares (and the binding covers exactly those), and
argument validation that runs before any HIP call returns the documented
status codes.  The host wrappers refuse CPU tensors: there is no CPU path.
"""

import ctypes
import os
import re

import pytest
import torch

from evo2_flash_amd import _lib
from evo2_flash_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "evo2_hyena.h")

EVO2_OK, EVO2_ERR_INVALID, EVO2_ERR_UNSUPPORTED = 0, 1, 2


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(evo2_\w+)\s*\(", text))


def _codes():
    text = open(HEADER).read()
    return {k: int(v) for k, v in re.findall(r"\b(EVO2_\w+)\s*=\s*(\d+)", text)}


needs_lib = pytest.mark.skipif(not os.path.exists(LIB_PATH), reason="library not built")


def test_binding_covers_header():
    assert _declared() == set(_lib.SIGNATURES), (
        sorted(_declared() ^ set(_lib.SIGNATURES)))


def test_status_codes():
    c = _codes()
    assert (c["EVO2_OK"], c["EVO2_ERR_INVALID"], c["EVO2_ERR_UNSUPPORTED"]) == (0, 1, 2)


@needs_lib
def test_library_exports_every_symbol():
    handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
    for name in sorted(_declared()):
        assert hasattr(handle, name), name
    lib = _lib.lib()
    assert lib.evo2_abi_version() >= 1


@needs_lib
def test_workspace_bytes():
    lib = _lib.lib()
    assert lib.evo2_hcl_workspace_bytes(3, 4096) == 3 * 4096 * 16 * 4
    assert lib.evo2_hcl_workspace_bytes(0, 4096) == 0


@needs_lib
def test_validation_before_launch():
    """Calls rejected by argument checks never reach the HIP runtime."""
    lib = _lib.lib()
    n = None
    # the allocation-free LI prefill refuses more tiles than its 32 MiB scratch holds
    rc = lib.evo2_hyena_hcl_prefill_noalloc(n, 0, n, n, 0, 0, 0, n, 0, 0, n, 0, 0, n, 0, 0, 0,
                                            n, n, 1, n, 1, n, 65, n, 1024, n, 0, 1, 8192, 2, n)
    assert rc == EVO2_ERR_UNSUPPORTED
    rc = lib.evo2_hyena_decode(n, 0, n, n, 0, 0, 0, n, 0, n, 0, 0, n, 0, 0, n, 0, 0, 0, n, n, 0,
                               -1, 4096, 128, 0, 0, 2, n)
    assert rc == EVO2_ERR_INVALID
    assert b"bad sizes" in lib.evo2_last_error()
    rc = lib.evo2_hyena_decode(n, 0, n, n, 0, 0, 0, n, 0, n, 0, 0, n, 0, 0, n, 0, 0, 0, n, n, 0,
                               0, 4096, 128, 0, 0, 2, n)
    assert rc == EVO2_OK  # empty batch: nothing to do
    rc = lib.evo2_hyena_decode(n, 0, n, n, 0, 0, 0, n, 0, n, 0, 0, n, 0, 0, n, 0, 0, 0, n, n, 0,
                               4, 4096, 128, 0, 0, 2, n)
    assert rc == EVO2_ERR_INVALID  # null pointers
    rc = lib.evo2_fir_prefill(n, 0, n, 0, 0, 64, n, 0, 0, 0, n, 1, n, 0, n, 1, 64, n, 0, 10, 4096,
                              2, n)
    assert rc == EVO2_ERR_UNSUPPORTED and b"7 or 128" in lib.evo2_last_error()
    rc = lib.evo2_fir_prefill(n, 0, n, 0, 0, 7, n, 0, 0, 0, n, 1, n, 0, n, 1, 48, n, 0, 10, 4096,
                              2, n)
    assert rc == EVO2_ERR_INVALID and b"block_t" in lib.evo2_last_error()
    rc = lib.evo2_fp8_gemm(n, 16, n, 16, n, n, n, n, 0, 64, 4096, 4000, n)
    assert rc == EVO2_ERR_INVALID  # null pointers are checked before K
    rc = lib.evo2_fp8_pack_weight(n, 4096, n, 12280, 4096, n)
    assert rc == EVO2_ERR_UNSUPPORTED and b"multiple of 16" in lib.evo2_last_error()
    rc = lib.evo2_fp8_pack_weight(n, 4096, n, 12288, 4096, n)
    assert rc == EVO2_ERR_INVALID  # null pointers
    rc = lib.evo2_fp8_gemm_packed(n, 16, n, n, n, n, n, 0, 64, 4096, 4096, n)
    assert rc == EVO2_ERR_INVALID  # null pointers
    assert lib.evo2_fp8_gemm_packed(n, 16, n, n, n, n, n, 0, 0, 4096, 4096, n) == EVO2_OK
    rc = lib.evo2_hyena_hcl_prefill(n, 0, n, n, 0, 0, 0, n, 0, 0, n, 0, 0, n, 0, 0, 0, n, n, 1, n,
                                    0, n, 1, n, 40, n, 0, n, 0, 10, 4096, 2, n)
    assert rc == EVO2_ERR_INVALID and b"block_t" in lib.evo2_last_error()
    # prefill attention: a (sequence, head) plane of 256 L bytes must fit 32-bit offsets,
    # head_dim 128 only, L a multiple of 8, a positive scale
    rc = lib.evo2_prefill_attention(n, n, n, n, 1, 32, 1 << 24, 128, 0.088, n)
    assert rc == EVO2_ERR_INVALID and b"bad sizes" in lib.evo2_last_error()
    rc = lib.evo2_prefill_attention(n, n, n, n, 1, 32, 4096, 64, 0.125, n)
    assert rc == EVO2_ERR_UNSUPPORTED and b"128 only" in lib.evo2_last_error()
    rc = lib.evo2_prefill_attention(n, n, n, n, 1, 32, 4096, 128, -1.0, n)
    assert rc == EVO2_ERR_INVALID and b"positive" in lib.evo2_last_error()
    rc = lib.evo2_prefill_attention(n, n, n, n, 1, 32, 4100, 128, 0.088, n)
    assert rc == EVO2_ERR_INVALID  # null pointers, checked before L % 8
    assert lib.evo2_prefill_attention(n, n, n, n, 0, 32, 4096, 128, 0.088, n) == EVO2_OK


def test_wrappers_refuse_cpu_tensors():
    from evo2_flash_amd.decode import hyena_decode
    from evo2_flash_amd.fp8 import quantize_input
    from evo2_flash_amd.hcl import hcl_compute_filter

    H = 8
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        hyena_decode(torch.zeros(1, 3 * H, dtype=torch.bfloat16), torch.zeros(3 * H, 3),
                     torch.zeros(2, 3 * H, 2), torch.ones(1, dtype=torch.int32),
                     torch.zeros(H, 7), torch.zeros(2, H, 6))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        quantize_input(torch.zeros(2, 16, dtype=torch.bfloat16), torch.ones(1))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        hcl_compute_filter(torch.zeros(2, 16), torch.zeros(2, 16), torch.arange(4.0))


def test_decode_supported_false_on_cpu():
    from evo2_flash_amd.decode import decode_supported

    H = 8
    assert not decode_supported(torch.zeros(1, 3 * H, dtype=torch.bfloat16),
                                torch.zeros(3 * H, 3, dtype=torch.bfloat16),
                                torch.zeros(2, 3 * H, 2, dtype=torch.bfloat16),
                                torch.zeros(H, 7, dtype=torch.bfloat16), torch.zeros(2, H, 6))


def test_verify_validation_before_launch():
    """The verify entry points reject bad sizes, a missing table and an
    unsupported filter length before touching any pointer."""
    lib = _lib.lib()
    n = None
    args = lambda Q, K, starts, nreq: (n, 0, 0, 0, n, 0, 0, K, n, 0, 0, 0, n, 0, 0, n, 0, 0,  # noqa: E731
                                       Q, starts, n, n, n, 0, nreq, 4, 64, 0, 8, n)
    assert lib.evo2_fir_verify(*args(0, 128, n, 2)) == EVO2_ERR_INVALID      # Q = 0
    assert b"bad sizes" in lib.evo2_last_error()
    assert lib.evo2_fir_verify(*args(2, 128, n, 2)) == EVO2_ERR_INVALID      # null pointers
    ok = ctypes.c_void_p(8)  # never dereferenced: validation fails first
    full = (ok, 0, 0, 0, ok, 0, 0, 64, ok, 0, 0, 0, ok, 0, 0, ok, 0, 0, 1, n, n, n, ok, 0, 2, 4,
            64, 0, 8, n)
    assert lib.evo2_fir_verify(*full) == EVO2_ERR_UNSUPPORTED               # K = 64
    assert b"7 or 128" in lib.evo2_last_error()
    two = list(full)
    two[7], two[18] = 128, 2                                                # Q=2 without tables
    assert lib.evo2_fir_verify(*two) == EVO2_ERR_INVALID
    assert b"Q=1" in lib.evo2_last_error()
    iir = (ok, 0, 0, 1, ok, 16, 1, ok, 16, 1, ok, 0, 16, 1, ok, 0, 0, ok, 0, 0, 1, ok, n, n, ok,
           0, 2, 4, 64, 0, 8, n)
    assert lib.evo2_iir_verify(*iir) == EVO2_ERR_INVALID                     # starts without ends
    assert b"go together" in lib.evo2_last_error()


def test_verify_wrappers_check_metadata():
    from evo2_flash_amd.verify import fir_snapshots

    x = torch.zeros(3, 8)
    meta = (torch.zeros(2, 3, dtype=torch.int32), torch.zeros(2, 4, dtype=torch.int32),
            torch.zeros(2), torch.zeros(2), torch.ones(2))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fir_snapshots(x, torch.zeros(8, 7, dtype=torch.bfloat16), torch.zeros(4, 8, 6), meta)


@needs_lib
def test_fp8_persist_order_covers_every_tile():
    """The persistent GEMM's tile order is a bijection onto the tile grid for
    every grid shape, including block counts that leave the last round of the
    XCD-grouped order part-filled (48 x 8 tiles: 12 blocks of 4 x 8); while
    the rounds are whole, the 32 tiles one XCD runs at once form one block."""
    import numpy as np
    lib = _lib.lib()
    for ncu in (256, 80):
        for tn in range(1, 65, 3 if ncu == 256 else 7):
            for tm in range(1, 41, 1 if ncu == 256 else 5):
                total = tn * tm
                bn = np.full(total, -1, dtype=np.int32)
                bm = np.full(total, -1, dtype=np.int32)
                grouped = lib.evo2_fp8_gemm_persist_order(tn, tm, ncu, bn.ctypes.data,
                                                          bm.ctypes.data)
                assert grouped == (1 if ncu == 256 and tn % 4 == 0 and tm % 8 == 0 else 0)
                assert bn.min() >= 0 and bn.max() < tn and bm.min() >= 0 and bm.max() < tm, \
                    (ncu, tn, tm)
                assert len(np.unique(bm.astype(np.int64) * tn + bn)) == total, (ncu, tn, tm)
                if grouped:
                    whole = (tn // 4) * (tm // 8) // 8 * 256
                    t = np.arange(whole)
                    for key in np.unique((t >> 8) * 8 + (t & 7)):
                        sel = ((t >> 8) * 8 + (t & 7)) == key
                        assert len(np.unique(bn[:whole][sel] // 4)) == 1
                        assert len(np.unique(bm[:whole][sel] // 8)) == 1
    assert lib.evo2_fp8_gemm_persist_order(48, 8, 256, None, None) == 1
    assert lib.evo2_fp8_gemm_persist_order(0, 8, 256, None, None) == -1
