"""GPU unit parity: the building blocks of the MoE block against the oracle.

Run on an MI355X through the C-ABI (libmoe_block.so).  Each test prints the
case it is about to run before touching the GPU.
"""
import numpy as np
import pytest

import moe_block as mb
import workloads as wl

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch, torch.device("cuda:0")


@pytest.fixture(scope="module")
def blk(torch_dev):
    b = mb.MoeBlock(0)
    yield b
    b.close()


def test_wave_sum_lane_layout(blk, torch_dev):
    torch, dev = torch_dev
    say("wave_sum 32 waves")
    rng = np.random.default_rng(0)
    x = rng.standard_normal(64 * 32).astype(np.float32)
    x[64:128] = np.arange(64, dtype=np.float32)  # exact: 2016 in every lane
    xd = torch.from_numpy(x).to(dev)
    out = torch.empty_like(xd)
    blk.debug_wave_sum(xd, out)
    got = out.cpu().numpy().reshape(32, 64)
    want = x.reshape(32, 64).astype(np.float64).sum(axis=1)
    assert np.all(got[1] == 2016.0)
    # every lane of a wave holds the same total
    assert np.all(got == got[:, :1])
    np.testing.assert_allclose(got[:, 0], want, rtol=1e-5, atol=1e-5)


def test_quantize_q8_0_bit_exact(blk, torch_dev, oracle):
    torch, dev = torch_dev
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((8, 7168)) * rng.uniform(1e-3, 30, (8, 1))).astype(np.float32)
    x[0, :32] = 0.0  # zero block
    x[1, :32] = np.float32(0.0)
    x[1, 0] = 127.0
    x[1, 1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]  # exact ties -> half to even
    say("quantize_q8_0", x.shape)
    xd = torch.from_numpy(x).to(dev)
    qs = torch.empty(x.shape, dtype=torch.int8, device=dev)
    d = torch.empty((8, 7168 // 32), dtype=torch.int16, device=dev)
    blk.debug_quantize_q8_0(xd, qs, d)
    torch.cuda.synchronize()
    oq, od = oracle.quantize_q8_0(x)
    np.testing.assert_array_equal(qs.cpu().numpy(), oq)
    np.testing.assert_array_equal(d.cpu().numpy().view(np.uint16), od)


def test_upload_repack_round_trip(blk, oracle):
    H, F, E = 256, 128, 4
    shape = wl.LayerShape(hidden=H, ffn=F, n_expert=E, n_used=2, has_shared=True, route_mode=1)
    rng = np.random.default_rng(2)
    gate = rng.integers(0, 256, (E, F, H // 32, 17), dtype=np.uint8)
    up = rng.integers(0, 256, (E, F, H // 32, 17), dtype=np.uint8)
    down = rng.integers(0, 256, (E, H, F // 32, 17), dtype=np.uint8)
    sh = (rng.integers(0, 256, (F, H // 32, 17), dtype=np.uint8),
          rng.integers(0, 256, (F, H // 32, 17), dtype=np.uint8),
          rng.integers(0, 256, (H, F // 32, 17), dtype=np.uint8))
    say("upload+read_blocks", H, F, E)
    blk.upload_layer(901, shape, gate, up, down, sh)
    try:
        for e in range(E):
            np.testing.assert_array_equal(blk.read_blocks(901, mb.T_GATE, e), gate[e])
            np.testing.assert_array_equal(blk.read_blocks(901, mb.T_UP, e), up[e])
            np.testing.assert_array_equal(blk.read_blocks(901, mb.T_DOWN, e), down[e])
        for t in range(3):
            np.testing.assert_array_equal(blk.read_blocks(901, t, E), sh[t])
        assert blk.layer_bytes(901) == shape.layer_bytes
    finally:
        blk.release_layer(901)


def test_device_generator_matches_oracle(blk, oracle):
    shape = wl.C1
    say("generate C1 layer")
    blk.generate_layer(902, shape, seed=77)
    try:
        for e in (0, 7, 31):
            np.testing.assert_array_equal(blk.read_blocks(902, mb.T_GATE, e),
                                          oracle.gen_mxfp4(77, 902, oracle.T_GATE, e, shape.ffn, shape.hidden))
            np.testing.assert_array_equal(blk.read_blocks(902, mb.T_DOWN, e),
                                          oracle.gen_mxfp4(77, 902, oracle.T_DOWN, e, shape.hidden, shape.ffn))
    finally:
        blk.release_layer(902)


@pytest.mark.parametrize("mode,E,k,T,bias", [(0, 32, 4, 5, False), (1, 256, 8, 33, False), (1, 256, 8, 16, True),
                                             (2, 256, 6, 9, True)])
def test_route_matches_oracle(blk, torch_dev, oracle, mode, E, k, T, bias):
    torch, dev = torch_dev
    rng = np.random.default_rng(3 + mode)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.1).astype(np.float32) if bias else None
    say("route", mode, E, k, T, bias)
    ids = torch.empty((T, k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, k), dtype=torch.float32, device=dev)
    blk.route(torch.from_numpy(lg).to(dev), k, mode, True, 1.0, ids, wts,
              bias=None if b is None else torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    oi, ow = oracle.route(lg, k, mode, norm=True, bias=b)
    np.testing.assert_array_equal(ids.cpu().numpy(), oi)
    np.testing.assert_allclose(wts.cpu().numpy(), ow, rtol=2e-6, atol=1e-7)


# P = 8800 (T = 1100): more than 8 steps of 64 pairs per wave, past the ids
# k_group keeps in registers
# P <= 128 takes the one-wave ballot grouping (k_group_few), one or two pairs per lane: P = 8, 12, 24,
# 32, 48, 64, 65, 80, 128, with E = 100 (not a multiple of 64) and E = 16, 32 (fewer experts than pairs:
# the per-expert loop runs on part of the wave); P = 250 and up take k_group; E = 1024 uses all 10 id bits
@pytest.mark.parametrize("T,k,E,zipf", [(1, 8, 256, False), (4, 8, 256, True), (8, 8, 256, True), (4, 6, 100, False),
                                        (13, 5, 100, True), (16, 8, 256, True), (8, 16, 1024, False), (25, 10, 1024, False),
                                        (12, 4, 16, True), (20, 4, 32, False),
                                        (16, 16, 1024, True), (32, 8, 256, True), (32, 8, 256, False),
                                        (64, 8, 256, True),
                                        (512, 8, 256, True), (512, 8, 256, False), (3, 4, 32, False),
                                        (1100, 8, 256, True), (1100, 8, 256, False)])
def test_group_bit_exact(blk, torch_dev, oracle, T, k, E, zipf):
    torch, dev = torch_dev
    shape = wl.LayerShape(hidden=64, ffn=64, n_expert=E, n_used=k, has_shared=False, route_mode=1)
    _, lg = wl.make_inputs(shape, T, seed=T * 7 + k, zipf=zipf)
    ids_np, _ = oracle.route(lg, k, 1)
    say("group", T, k, E, zipf)
    ids = torch.from_numpy(ids_np).to(dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    blk.group(ids, E, counts, offsets, perm, inv)
    torch.cuda.synchronize()
    g = oracle.group(ids_np, E)
    for name, t in (("counts", counts), ("offsets", offsets), ("perm", perm), ("inv", inv)):
        np.testing.assert_array_equal(t.cpu().numpy(), g[name], err_msg=name)


@pytest.mark.parametrize("T,k,E", [(300, 8, 256), (5, 4, 32), (6, 8, 100), (12, 8, 256), (8, 16, 1024),
                                   (20, 8, 256), (1100, 8, 256)])
def test_group_drops_out_of_range_ids(blk, torch_dev, T, k, E):
    """Out-of-range ids get no grouped row (inv = -1); the valid pairs keep
    ascending pair order within each expert (checked against a stable sort)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(T + E)
    ids_np = rng.integers(0, E, size=(T, k), dtype=np.int32)
    bad = rng.random((T, k)) < 0.1
    ids_np[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -1, E).astype(np.int32)
    say("group with dropped ids", T, k, E, int(bad.sum()))
    flat = ids_np.ravel()
    ok = (flat >= 0) & (flat < E)
    counts_ref = np.bincount(flat[ok], minlength=E).astype(np.int32)
    offsets_ref = np.concatenate([[0], np.cumsum(counts_ref)]).astype(np.int32)
    valid_pairs = np.nonzero(ok)[0]
    perm_ref = valid_pairs[np.argsort(flat[ok], kind="stable")].astype(np.int32)
    inv_ref = np.full(T * k, -1, np.int32)
    inv_ref[perm_ref] = np.arange(len(perm_ref), dtype=np.int32)
    ids = torch.from_numpy(ids_np).to(dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    perm = torch.full((T * k,), -7, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    blk.group(ids, E, counts, offsets, perm, inv)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(counts.cpu().numpy(), counts_ref)
    np.testing.assert_array_equal(offsets.cpu().numpy(), offsets_ref)
    np.testing.assert_array_equal(perm.cpu().numpy()[: len(perm_ref)], perm_ref)
    np.testing.assert_array_equal(inv.cpu().numpy(), inv_ref)
