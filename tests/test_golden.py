"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every committed fixture bit for bit, so a change
to the oracle cannot slip through.  GPU: the HIP library reproduces the
fixtures -- routing ids and grouping bit-exact, Q8_0 codes and scales
bit-exact, block outputs within max|diff| <= 1e-3 * RMS(fixture).
"""
import glob
import hashlib
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BLOCKS = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "block_*.npz")))


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def oracle_layer(oracle, g):
    return oracle.OracleLayer.generated(int(g["seed"]), int(g["layer"]), int(g["H"]), int(g["F"]), int(g["E"]),
                                        int(g["k"]), experts=range(int(g["E"])), shared=bool(g["shared"]),
                                        clamp=float(g["clamp"]), e_lo=int(g["e_lo"]), e_span=int(g["e_span"]))


def test_fixtures_present():
    assert len(BLOCKS) >= 5
    assert os.path.exists(os.path.join(HERE, "q8_0.npz"))


@pytest.mark.parametrize("name", BLOCKS)
def test_oracle_reproduces_fixture(oracle, name):
    g = load(name)
    bias = g.get("bias")
    ids, wts = oracle.route(g["logits"], int(g["k"]), int(g["mode"]), norm=True, bias=bias)
    np.testing.assert_array_equal(ids, g["ids"])
    np.testing.assert_array_equal(wts, g["wts"])
    L = oracle_layer(oracle, g)
    h = hashlib.sha256()
    for e in sorted(L.gate):
        for part in (L.gate[e], L.up[e], L.down[e]):
            h.update(part.tobytes())
    if L.shared is not None:
        for part in L.shared:
            h.update(part.tobytes())
    assert h.hexdigest() == str(g["weights_sha256"])
    res = L.forward(g["x"], ids, wts, per_slot=True, taps=True)
    np.testing.assert_array_equal(res["out"], g["out"])
    np.testing.assert_array_equal(res["per_slot"], g["per_slot"])
    np.testing.assert_array_equal(res["h"], g["h"])
    grp = oracle.group(ids, int(g["E"]))
    for key in ("counts", "offsets", "perm", "inv"):
        np.testing.assert_array_equal(grp[key], g[key], err_msg=key)


def test_oracle_reproduces_q8_fixture(oracle):
    g = load("q8_0")
    qs, d = oracle.quantize_q8_0(g["x"])
    np.testing.assert_array_equal(qs, g["qs"])
    np.testing.assert_array_equal(d, g["d"])


# ---- GPU ---------------------------------------------------------------------------------

def _rms_close(got, ref, tol=1e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    r = float(np.sqrt(np.mean(ref[fin] ** 2)))
    err = float(np.max(np.abs(got[fin] - ref[fin])))
    print(f"[gpu] rms={r:.4e} max|diff|={err:.3e} ratio={err / r:.3e}", flush=True)
    assert err <= tol * r


@pytest.fixture(scope="module")
def gpu():
    import torch

    import moe_block as mb
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    b = mb.MoeBlock(0)
    yield torch, b
    b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", BLOCKS)
def test_gpu_matches_fixture(gpu, name):
    import moe_block as mb
    import workloads as wl

    torch, blk = gpu
    g = load(name)
    print(f"[gpu] golden {name}", flush=True)
    dev = torch.device("cuda:0")
    shape = wl.LayerShape(hidden=int(g["H"]), ffn=int(g["F"]), n_expert=int(g["E"]), n_used=int(g["k"]),
                          has_shared=bool(g["shared"]), route_mode=int(g["mode"]), clamp=float(g["clamp"]))
    # the generator keys every tensor by (seed, layer id): the fixture's layer id regenerates its weights
    blk.generate_layer(int(g["layer"]), shape, seed=int(g["seed"]), e_lo=int(g["e_lo"]), e_span=int(g["e_span"]))
    try:
        T, k, E = int(g["T"]), int(g["k"]), int(g["E"])
        x = torch.from_numpy(g["x"]).to(dev)
        logits = torch.from_numpy(g["logits"]).to(dev)
        bias = torch.from_numpy(g["bias"]).to(dev) if "bias" in g else None
        ids = torch.empty((T, k), dtype=torch.int32, device=dev)
        wts = torch.empty((T, k), dtype=torch.float32, device=dev)
        blk.route(logits, k, int(g["mode"]), True, 1.0, ids, wts, bias=bias)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids.cpu().numpy(), g["ids"])
        np.testing.assert_allclose(wts.cpu().numpy(), g["wts"], rtol=2e-6, atol=1e-7)
        # block on the fixture's own ids / weights
        idf = torch.from_numpy(g["ids"]).to(dev)
        wtf = torch.from_numpy(g["wts"]).to(dev)
        out = torch.empty((T, int(g["H"])), dtype=torch.float32, device=dev)
        blk.forward(int(g["layer"]), x, idf, wtf, out)
        torch.cuda.synchronize()
        _rms_close(out.cpu().numpy(), g["out"])
        ps = torch.empty((T, k, int(g["H"])), dtype=torch.float32, device=dev)
        blk.forward(int(g["layer"]), x, idf, wtf, ps, flags=mb.MOE_FWD_PER_SLOT)
        torch.cuda.synchronize()
        _rms_close(ps.cpu().numpy(), g["per_slot"])
        # grouping
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        perm = torch.empty(T * k, dtype=torch.int32, device=dev)
        inv = torch.empty(T * k, dtype=torch.int32, device=dev)
        blk.group(idf, E, counts, offsets, perm, inv)
        torch.cuda.synchronize()
        for key, t in (("counts", counts), ("offsets", offsets), ("perm", perm), ("inv", inv)):
            np.testing.assert_array_equal(t.cpu().numpy(), g[key], err_msg=key)
    finally:
        blk.release_layer(int(g["layer"]))


@pytest.mark.gpu
def test_gpu_q8_fixture(gpu):
    torch, blk = gpu
    g = load("q8_0")
    print("[gpu] golden q8_0", flush=True)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(g["x"]).to(dev)
    qs = torch.empty(g["x"].shape, dtype=torch.int8, device=dev)
    d = torch.empty(g["d"].shape, dtype=torch.int16, device=dev)
    blk.debug_quantize_q8_0(x, qs, d)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(qs.cpu().numpy(), g["qs"])
    np.testing.assert_array_equal(d.cpu().numpy().view(np.uint16), g["d"])
