"""The decode step captured in a HIP graph: every replay (with eager work and
synchronisation in between) matches the same step run eagerly on a twin
state pool, bit for bit, for outputs and the whole pool."""

import pytest
import torch

from evo2_flash_amd.decode import channel_major_taps, hyena_decode

from _cases import clone_pool, decode_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("kind", ["hcs", "hcm", "hcl"])
def test_decode_graph_replays_match_eager(kind):
    H, B, nblk = 512, 16, 24
    prm, z, slots, pool = decode_case(kind, H, B, nblk, seed=71, n_null=2)
    pa, pb = clone_pool(pool, DEV), clone_pool(pool, DEV)
    sw = prm["short_filter"].view(3 * H, 3).to(DEV)
    D = prm.get("D")
    D = None if D is None else D.to(DEV)
    if kind == "hcl":
        inner, lp = prm["residues"].to(DEV), prm["log_poles"][..., 0].to(DEV)
        sa, sb = pa.ssm_view(), pb.ssm_view()
    else:
        K = prm["conv"].shape[-1]
        inner, lp = channel_major_taps(prm["conv"].view(H, K).to(DEV)), None
        sa, sb = pa.inner_view(K - 1), pb.inner_view(K - 1)
    zs, sl = z.to(DEV), slots.to(DEV)

    def run(p, st):
        return hyena_decode(zs, sw, p.conv_view(), sl, inner, st, D, lp)

    run(pa, sa)
    run(pb, sb)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            out_graph = run(pa, sa)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        out_eager = run(pb, sb)
        torch.cuda.synchronize()
        assert torch.equal(out_graph.view(torch.int16), out_eager.view(torch.int16)), rep
        assert torch.equal(pa.raw, pb.raw), rep
