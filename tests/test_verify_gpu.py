"""GPU parity of the speculative verify kernels (triton_verifier.py) against
the oracle's emulation of the reference kernel's arithmetic.

* fir_snapshots / iir_snapshots over ragged requests (1..Q draft tokens each,
  accepted counts 1..Q, null destinations): outputs and the whole state pool
  bit for bit, bf16 and fp32 token inputs, strided block tables;
* fir_one / iir_one (one token per request, in place) bit for bit;
* the verify output within 1e-2 of the reference's plain torch form
  (mixers.py:578-660).
"""

import pytest
import torch

import oracle
from evo2_flash_amd.verify import (fir_one, fir_snapshots, fir_supported, iir_one, iir_snapshots,
                                   iir_supported)

from _cases import max_rel_err, verify_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _fir_state_dev(state):
    """(blocks, H, K-1) fp32 as a view over channel-contiguous (blocks, K-1, H)
    storage, the engine's native layout."""
    return state.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)


def _meta_dev(meta, strided):
    ins, outs, starts, ends, accepted = meta
    if strided:  # block tables as column slices of wider tables
        pad = torch.zeros(ins.shape[0], 2 * ins.shape[1], dtype=torch.int32)
        pad[:, ::2] = ins
        ins = pad.to(DEV)[:, ::2]
        pad = torch.zeros_like(pad)
        pad[:, ::2] = outs
        outs = pad.to(DEV)[:, ::2]
    else:
        ins, outs = ins.to(DEV), outs.to(DEV)
    return ins, outs, starts.to(DEV), ends.to(DEV), accepted.to(DEV)


@pytest.mark.parametrize("kind", ["hcs", "hcm"])
@pytest.mark.parametrize("H,x_dtype,strided", [(256, torch.bfloat16, False),
                                               (4096, torch.bfloat16, True),
                                               (192, torch.float32, True),
                                               (193, torch.bfloat16, False)])
def test_fir_snapshots_bitwise(kind, H, x_dtype, strided):
    """H = 192 leaves the channel-pair hcm kernel a part-filled last
    workgroup; an odd H takes the one-channel-per-lane form."""
    nreq, Q, nblk = 9, 4, 90
    prm, x, state, meta = verify_case(kind, H, nreq, Q, nblk, seed=H + Q, x_dtype=x_dtype)
    K = prm["conv"].shape[-1]
    w = prm["conv"].view(H, K)
    gst = _fir_state_dev(state)
    gx = x.to(DEV)
    assert fir_supported(gx, w.to(DEV), gst)
    print(f"fir verify {kind} H={H} {x_dtype} strided={strided}", flush=True)
    y = fir_snapshots(gx, w.to(DEV), gst, _meta_dev(meta, strided)).cpu()
    st = state.clone()
    ref = oracle.fir_verify_emulated(x, w, st, *meta)
    assert torch.equal(y.view(torch.int16) if x_dtype == torch.bfloat16 else y,
                       ref.view(torch.int16) if x_dtype == torch.bfloat16 else ref)
    assert torch.equal(gst.cpu(), st)
    plain = oracle.fir_decode_snapshots(x, w, state.clone(), *meta)
    assert max_rel_err(y, plain) <= 1e-2


@pytest.mark.parametrize("H,x_dtype,strided", [(256, torch.float32, False),
                                               (4096, torch.float32, True),
                                               (320, torch.bfloat16, False)])
def test_iir_snapshots_bitwise(H, x_dtype, strided):
    nreq, Q, nblk = 9, 4, 90
    prm, x, state, meta = verify_case("hcl", H, nreq, Q, nblk, seed=H + 1, x_dtype=x_dtype)
    poles = torch.exp(prm["log_poles"][..., 0].float())
    res = prm["residues"]
    gst = state.to(DEV)
    gx = x.to(DEV)
    assert iir_supported(gx, poles.to(DEV), res.to(DEV), gst)
    print(f"iir verify H={H} {x_dtype} strided={strided}", flush=True)
    y = iir_snapshots(gx, poles.to(DEV), res.to(DEV), gst, _meta_dev(meta, strided)).cpu()
    st = state.clone()
    ref = oracle.iir_verify_emulated(x, poles, res, st, *meta)
    assert torch.equal(y.float(), ref.float())
    assert torch.equal(gst.cpu(), st)
    plain = oracle.iir_decode_snapshots(x, poles, res, state.clone(), *meta)
    assert max_rel_err(y, plain) <= 1e-2


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_one_token_bitwise(kind):
    H, B, nblk = 512, 12, 30
    prm, x, state, _ = verify_case(kind, H, B, 1, nblk, seed=3,
                                   x_dtype=torch.float32 if kind == "hcl" else torch.bfloat16)
    slots = (torch.randperm(nblk - 1)[:B] + 1).to(torch.int32)
    slots[4] = 0   # a padding row on the null block: computed, never written
    st = state.clone()
    print(f"one-token verify {kind}", flush=True)
    if kind == "hcl":
        poles = torch.exp(prm["log_poles"][..., 0].float())
        gst = state.to(DEV)
        y = iir_one(x.to(DEV), poles.to(DEV), prm["residues"].to(DEV), gst, slots.to(DEV)).cpu()
        ref = oracle.iir_verify_emulated(x, poles, prm["residues"], st, slots[:, None],
                                         slots[:, None], None, None, None)
        assert torch.equal(y, ref)
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        gst = _fir_state_dev(state)
        y = fir_one(x.to(DEV), w.to(DEV), gst, slots.to(DEV)).cpu()
        ref = oracle.fir_verify_emulated(x, w, st, slots[:, None], slots[:, None], None, None,
                                         None)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(gst.cpu(), st)


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_long_requests_bitwise(kind):
    """More tokens per request (Q = 19) than the kernels stage at once (16):
    the one-token-at-a-time K=128 kernel and the per-token input loads past
    the staged ones, bit for bit against the emulation."""
    H, nreq, Q = 256, 3, 19
    nblk = 2 * nreq * Q + 2
    x_dtype = torch.float32 if kind == "hcl" else torch.bfloat16
    prm, x, state, meta = verify_case(kind, H, nreq, Q, nblk, seed=77, x_dtype=x_dtype)
    st = state.clone()
    print(f"long verify {kind} Q={Q}", flush=True)
    if kind == "hcl":
        poles = torch.exp(prm["log_poles"][..., 0].float())
        gst = state.to(DEV)
        y = iir_snapshots(x.to(DEV), poles.to(DEV), prm["residues"].to(DEV), gst,
                          _meta_dev(meta, False)).cpu()
        ref = oracle.iir_verify_emulated(x, poles, prm["residues"], st, *meta)
        assert torch.equal(y, ref)
    else:
        K = prm["conv"].shape[-1]
        w = prm["conv"].view(H, K)
        gst = _fir_state_dev(state)
        y = fir_snapshots(x.to(DEV), w.to(DEV), gst, _meta_dev(meta, False)).cpu()
        ref = oracle.fir_verify_emulated(x, w, st, *meta)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(gst.cpu(), st)
