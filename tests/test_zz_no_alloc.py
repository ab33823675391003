"""moe_forward_noalloc (the entry point that allocates nothing: its per-call
buffers live in the library's file-scope device scratch) against
moe_forward on the same inputs: bit for bit, on two calls in a row with the
second smaller than the first (the scratch keeps the first call's contents),
for the decode chain and the grouped chain.  A call too large for the
scratch is refused on the host.  Runs in its own context, alone or after
the other GPU tests."""
import numpy as np
import pytest

import moe_block as mb
import workloads as wl
from parity import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    b = mb.MoeBlock(0)
    b.generate_layer(0, wl.V3, seed=808)
    b.generate_layer(1, wl.C1, seed=809)
    yield torch, torch.device("cuda:0"), b
    b.close()


def _pair(ctx, oracle, layer, shape, T, seed, flags=0):
    torch, dev, b = ctx
    x, lg = wl.make_inputs(shape, T, seed, zipf=T > 1)
    ids, wts = oracle.route(lg, shape.n_used, shape.route_mode, norm=True)
    xd, idd, wd = (torch.from_numpy(a).to(dev) for a in (x, ids, wts))
    oshape = (T, shape.n_used, shape.hidden) if flags & mb.MOE_FWD_PER_SLOT else (T, shape.hidden)
    ref = torch.full(oshape, float("nan"), dtype=torch.float32, device=dev)
    got = torch.full(oshape, float("nan"), dtype=torch.float32, device=dev)
    b.forward(layer, xd, idd, wd, ref, flags)
    b.forward_noalloc(layer, xd, idd, wd, got, flags)
    torch.cuda.synchronize()
    return got.cpu().numpy(), ref.cpu().numpy()


@pytest.mark.parametrize("layer, Ts, flags", [
    (0, (64, 5), 0),                       # V3 grouped: octets, then pairs
    (0, (16, 1), 0),                       # V3 grouped, then decode (bal2 gate/up tickets)
    (0, (1, 1), mb.MOE_FWD_NO_SHARED),     # V3 decode without shared: every unit met by a ticket
    (1, (9, 2), mb.MOE_FWD_PER_SLOT),      # C1 grouped per-slot
    (1, (40, 20), 0),                      # C1 on the 16-row items (k_gate_up_ol, k_down_ol2)
    (1, (1, 1), 0),                        # C1 decode
])
def test_noalloc_equals_forward(ctx, oracle, layer, Ts, flags):
    shape = wl.V3 if layer == 0 else wl.C1
    for i, T in enumerate(Ts):
        say(f"noalloc layer {layer} T={T} flags={flags} (call {i + 1} of 2)")
        got, ref = _pair(ctx, oracle, layer, shape, T, 600 + 10 * layer + i, flags)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (layer, T, flags)


def test_noalloc_refuses_a_call_beyond_its_scratch(ctx):
    torch, dev, b = ctx
    T = 256  # a V3 grouped call of 256 tokens needs more than MOE_NOALLOC_SCRATCH_BYTES
    say("noalloc T=256 refused")
    x = torch.zeros((T, wl.V3.hidden), dtype=torch.float32, device=dev)
    ids = torch.zeros((T, 8), dtype=torch.int32, device=dev)
    wts = torch.zeros((T, 8), dtype=torch.float32, device=dev)
    out = torch.zeros((T, wl.V3.hidden), dtype=torch.float32, device=dev)
    with pytest.raises(mb.MoeError) as ei:
        b.forward_noalloc(0, x, ids, wts, out)
    assert ei.value.status == mb.MOE_ERR_INVALID_ARG and "scratch" in str(ei.value)
    torch.cuda.synchronize()
    assert float(out.abs().sum()) == 0.0
