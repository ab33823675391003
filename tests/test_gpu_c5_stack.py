"""Config C5 as a tested configuration: 40 DeepSeek-V3-shaped MXFP4 layers
resident at once (240.5 GB of experts in one GPU's HBM), one token per
layer with independently seeded top-8 sigmoid routing, captured as ONE
hipGraph of 40 layer calls and replayed.  The reference pre-records one
command buffer per (layer, die) and replays it (moe-serv/src/moe_tp.h:646-701).

Checks: every replay equals the eager calls bit for bit, per layer, with
eager work between the replays; the first, middle and last layers against
the CPU oracle (only the 9 experts a layer's token touches are generated on
the host) with the two-stage check of parity.check_block.

The test has its own context and frees nothing it does not own; the other
GPU test modules release their layers when they end, and the caching
allocator's free blocks are returned first.
"""
import numpy as np
import pytest

import moe_block as mb
import workloads as wl
from parity import check_block, oracle_layer, say

pytestmark = pytest.mark.gpu

NL = 40
SEED = 5000


def test_c5_forty_layer_graph(oracle):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    dev = torch.device("cuda:0")
    sh = wl.V3
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info()
    say(f"C5: device memory free {free / 1e9:.1f} of {total / 1e9:.1f} GB; {NL} layers need "
        f"{NL * sh.layer_bytes / 1e9:.1f} GB")
    blk = mb.MoeBlock(0)
    try:
        for layer in range(NL):
            blk.generate_layer(layer, sh, seed=SEED + layer)
        torch.cuda.synchronize()
        say("C5: layers resident, budget used", NL * sh.layer_bytes)
        x, lg = wl.make_inputs(sh, NL, 77)  # row i: layer i's token and router logits
        ids, wts = oracle.route(lg, sh.n_used, sh.route_mode, norm=True)
        assert len({tuple(r) for r in ids.tolist()}) > NL // 2  # the layers route independently
        xd, idd, wd = (torch.from_numpy(a).to(dev) for a in (x, ids, wts))
        blk.reserve(sh, 1)
        eager = torch.empty((NL, sh.hidden), dtype=torch.float32, device=dev)
        for i in range(NL):
            blk.forward(i, xd[i:i + 1], idd[i:i + 1], wd[i:i + 1], eager[i:i + 1])
        torch.cuda.synchronize()
        eager_np = eager.cpu().numpy()
        out = torch.empty((NL, sh.hidden), dtype=torch.float32, device=dev)
        row = lambda t: [t[i:i + 1] for i in range(NL)]  # noqa: E731
        g = blk.graph_capture(list(range(NL)), row(xd), row(idd), row(wd), row(out))
        spare = torch.empty((1, sh.hidden), dtype=torch.float32, device=dev)
        for rep in range(3):
            out.fill_(float("nan"))
            g.launch()
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for i in range(NL):
                assert np.array_equal(got[i].view(np.uint32), eager_np[i].view(np.uint32)), f"replay {rep} layer {i}"
            say(f"C5 replay {rep}: {NL} layers bit-exact with eager")
            blk.forward(rep, xd[NL - 1:NL], idd[NL - 1:NL], wd[NL - 1:NL], spare)  # eager work between replays
        g.close()
        blk.set_taps(True)
        for i in (0, NL // 2, NL - 1):
            one = torch.empty((1, sh.hidden), dtype=torch.float32, device=dev)
            blk.forward(i, xd[i:i + 1], idd[i:i + 1], wd[i:i + 1], one)
            torch.cuda.synchronize()
            got = one.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), eager_np[i:i + 1].view(np.uint32))
            say(f"C5 layer {i}: ids {ids[i].tolist()}")
            L = oracle_layer(oracle, sh, SEED + i, i, ids[i:i + 1])
            check_block(oracle, L, blk, sh, x[i:i + 1], ids[i:i + 1], wts[i:i + 1], got, f"C5 layer {i}")
    finally:
        blk.close()
