"""Pins the CPU oracle (oracle/moe_oracle.c) before anything is checked against it.

Each check compares the oracle with something it was not derived from: the
OCP MX format definitions (np_ref.py), numpy's / torch's own float
conversions, brute force, closed forms and invariants.  The reference ships
no golden vectors for this path (its gates need llama.cpp + GGUF models), so
these, plus the committed fixtures in tests/golden/, are what pin it.
"""
import math

import numpy as np
import pytest

import np_ref


# ---- number formats ------------------------------------------------------------

def test_e8m0_half_closed_form(oracle):
    # ggml's e8m0 "half" is 2^(e-128) for every byte, e<2 included (f32 denormals)
    for e in range(256):
        assert oracle.e8m0_half(e) == math.ldexp(1.0, e - 128), e


def test_dequant_matches_ocp_e2m1_definition(oracle):
    rng = np.random.default_rng(0)
    blocks = rng.integers(0, 256, size=(5, 4, 17), dtype=np.uint8)
    blocks[:, :, 0] = rng.integers(100, 150, size=(5, 4))
    got = oracle.dequant_mxfp4(blocks, 128).astype(np.float64)
    np.testing.assert_array_equal(got, np_ref.dequant_blocks(blocks))


def test_dequant_element_order(oracle):
    # byte j: low nibble -> element j, high nibble -> element j+16
    blk = np.zeros((1, 1, 17), np.uint8)
    blk[0, 0, 0] = 128  # scale 2^1
    for j in range(16):
        blk[0, 0, 1 + j] = (j & 0xF) | (((15 - j) & 0xF) << 4)
    v = oracle.dequant_mxfp4(blk, 32)[0]
    for j in range(16):
        assert v[j] == np_ref.e2m1_value(j) * 2.0
        assert v[j + 16] == np_ref.e2m1_value(15 - j) * 2.0


def test_fp16_conversion_vs_numpy(oracle):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 2000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  1.5e-8, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    for v in vals:
        with np.errstate(over="ignore"):  # values beyond fp16 round to inf, as intended
            want = np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]
        assert oracle.fp32_to_fp16_bits(float(v)) == want, v
        back = oracle.fp16_bits_to_fp32(int(want))
        assert back == float(np.array([want], np.uint16).view(np.float16)[0].astype(np.float32))


def test_bf16_conversion_vs_torch(oracle):
    import torch
    rng = np.random.default_rng(2)
    x = rng.standard_normal(5000).astype(np.float32) * 37.0
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.lib().mo_fp32_to_bf16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, want)


# ---- Q8_0 ------------------------------------------------------------------------

def test_q8_0_invariants(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 256)) * rng.uniform(1e-3, 50, (64, 1))).astype(np.float32)
    qs, d = oracle.quantize_q8_0(x)
    assert np.abs(qs.astype(np.int32)).max() <= 127
    xb = x.reshape(64, 8, 32).astype(np.float64)
    qb = qs.reshape(64, 8, 32).astype(np.int32)
    amax = np.abs(xb).max(axis=2)
    # every nonzero block reaches +-127 on its largest element
    assert np.all(np.abs(qb).max(axis=2) == 127)
    # d is fp16(amax/127)
    np.testing.assert_array_equal(d, (amax / 127.0).astype(np.float32).astype(np.float16).view(np.uint16))
    # each code is within half a step of x (step = amax/127, before fp16 rounding of d)
    step = amax / 127.0
    assert np.all(np.abs(qb * step[:, :, None] - xb) <= 0.5 * step[:, :, None] * (1 + 1e-5))


def test_q8_0_rounds_half_to_even(oracle):
    # amax = 127 -> id = 1: x * id is exact, so ties are real ties
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    qs, d = oracle.quantize_q8_0(x)
    assert qs[1:7].tolist() == [2, 4, -2, -4, 0, 0]  # roundf would give 3, 4, -3, -4, 1, -1
    assert np.array([d[0]], np.uint16).view(np.float16)[0] == np.float16(1.0)


def test_q8_0_zero_block(oracle):
    qs, d = oracle.quantize_q8_0(np.zeros(64, np.float32))
    assert not qs.any() and not d.any()


# ---- dots ------------------------------------------------------------------------

def test_block_isum_brute_force(oracle):
    rng = np.random.default_rng(4)
    kv2 = (np_ref.E2M1 * 2).astype(np.int64)  # doubled e2m1 = ggml's integer kvalues
    for _ in range(200):
        blk = rng.integers(0, 256, 17, dtype=np.uint8)
        q = rng.integers(-127, 128, 32).astype(np.int8)
        w = np.concatenate([kv2[blk[1:] & 0xF], kv2[blk[1:] >> 4]])
        assert oracle.block_isum(blk, q) == int(np.dot(w, q.astype(np.int64)))


def test_vec_dot_vs_float64(oracle):
    rng = np.random.default_rng(5)
    for K in (32, 256, 7168):
        row = rng.integers(0, 256, (1, K // 32, 17), dtype=np.uint8)
        row[0, :, 0] = rng.integers(120, 134, K // 32)
        x = rng.standard_normal(K).astype(np.float32)
        qs, d = oracle.quantize_q8_0(x)
        got = oracle.vec_dot(row, qs, d)
        terms = np_ref.dequant_blocks(row)[0] * np_ref.q8_dequant(qs, d)
        want = terms.sum()
        assert abs(got - want) <= 1e-6 * np.abs(terms).sum() + 1e-30, (K, got, want)


# ---- routing ---------------------------------------------------------------------

def test_route_sigmoid_closed_form(oracle):
    rng = np.random.default_rng(6)
    lg = rng.standard_normal((16, 256)).astype(np.float32)
    p = oracle.route_scores(lg, oracle.ROUTE_SIGMOID)
    np.testing.assert_allclose(p, 1.0 / (1.0 + np.exp(-lg.astype(np.float64))), rtol=3e-7)
    ids, w = oracle.route(lg, 8, oracle.ROUTE_SIGMOID)
    for t in range(16):
        assert ids[t].tolist() == np.argsort(-p[t], kind="stable")[:8].tolist()
        np.testing.assert_allclose(w[t], p[t, ids[t]] / p[t, ids[t]].astype(np.float64).sum(), rtol=1e-6)
        assert abs(w[t].astype(np.float64).sum() - 1.0) < 1e-6


def test_route_softmax_closed_form(oracle):
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((16, 32)).astype(np.float32)
    p = oracle.route_scores(lg, oracle.ROUTE_SOFTMAX)
    ex = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
    np.testing.assert_allclose(p, ex / ex.sum(axis=1, keepdims=True), rtol=1e-6)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, atol=1e-6)
    ids, w = oracle.route(lg, 4, oracle.ROUTE_SOFTMAX)
    for t in range(16):
        assert ids[t].tolist() == np.argsort(-lg[t], kind="stable")[:4].tolist()


def test_route_sqrt_softplus_closed_form(oracle):
    lg = np.linspace(-30, 30, 64, dtype=np.float32)[None, :]
    p = oracle.route_scores(lg, oracle.ROUTE_SQRT_SOFTPLUS)[0]
    want = np.sqrt(np.log1p(np.exp(lg[0].astype(np.float64))))
    np.testing.assert_allclose(p, want, rtol=2e-6)


def test_route_bias_selects_but_does_not_weigh(oracle):
    rng = np.random.default_rng(8)
    lg = rng.standard_normal((4, 64)).astype(np.float32)
    bias = np.zeros(64, np.float32)
    bias[[5, 9, 40]] = 10.0
    ids, w = oracle.route(lg, 6, oracle.ROUTE_SIGMOID, norm=False, bias=bias)
    p = oracle.route_scores(lg, oracle.ROUTE_SIGMOID)
    for t in range(4):
        assert set(ids[t, :3].tolist()) == {5, 9, 40}
        np.testing.assert_array_equal(w[t], p[t, ids[t]])


def test_route_norm_floor_and_scale(oracle):
    lg = np.full((1, 8), -40.0, np.float32)  # sigmoid ~ 4e-18: the 2^-14 floor binds
    lg[0, 3] = -39.0
    ids, w = oracle.route(lg, 2, oracle.ROUTE_SIGMOID, norm=True, scale=2.5)
    p = oracle.route_scores(lg, oracle.ROUTE_SIGMOID)[0]
    assert ids[0].tolist() == [3, 0]  # ties among the rest go to the lower id
    want = (p[ids[0]] / np.float32(6.103515625e-5)) * np.float32(2.5)
    np.testing.assert_array_equal(w[0], want.astype(np.float32))


def test_route_ties_lower_index_first(oracle):
    lg = np.zeros((1, 16), np.float32)
    ids, _ = oracle.route(lg, 5, oracle.ROUTE_SIGMOID)
    assert ids[0].tolist() == [0, 1, 2, 3, 4]


# ---- grouping ---------------------------------------------------------------------

@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (4, 8, 256), (64, 8, 256), (512, 8, 256), (7, 4, 32)])
def test_group_matches_stable_sort(oracle, T, k, E):
    rng = np.random.default_rng(T * 1000 + k)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    g = oracle.group(ids, E)
    flat = ids.ravel()
    np.testing.assert_array_equal(g["counts"], np.bincount(flat, minlength=E))
    np.testing.assert_array_equal(g["offsets"], np.concatenate([[0], np.cumsum(g["counts"])]))
    np.testing.assert_array_equal(g["perm"], np.argsort(flat, kind="stable"))
    np.testing.assert_array_equal(g["inv"][g["perm"]], np.arange(T * k))
    assert g["distinct"] == len(np.unique(flat))


# ---- the block ----------------------------------------------------------------------

def _tiny_layer(oracle, seed, H, F, E, k, shared, clamp, e_lo=124, e_span=7):
    return oracle.OracleLayer.generated(seed, 3, H, F, E, k, experts=range(E), shared=shared, clamp=clamp,
                                        e_lo=e_lo, e_span=e_span)


@pytest.mark.parametrize("shared,clamp", [(False, 0.0), (True, 0.0), (True, 3.0)])
def test_forward_vs_float64(oracle, shared, clamp):
    H, F, E, k, T = 128, 96, 6, 3, 4
    L = _tiny_layer(oracle, 11, H, F, E, k, shared, clamp, e_lo=120, e_span=4)
    rng = np.random.default_rng(12)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = rng.uniform(0.05, 0.6, (T, k)).astype(np.float32)
    res = L.forward(x, ids, wts, taps=True, per_slot=True)
    want, h = np_ref.moe_forward_f64(L, x, ids, wts, oracle.quantize_q8_0)
    rms = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(res["out"] - want)) <= 1e-4 * rms
    np.testing.assert_allclose(res["h"], h, rtol=1e-4, atol=1e-5 * np.abs(h).max())
    # per-slot rows sum (in slot order) to the routed part of out
    routed = res["per_slot"].astype(np.float64).sum(axis=1)
    if not shared:
        np.testing.assert_allclose(res["out"], routed, rtol=1e-5, atol=1e-6 * rms)
    if clamp:
        # the clamp really engaged: some pre-clamp |up| exceeded it
        assert np.abs(h).max() > 0


@pytest.mark.parametrize("shared,clamp", [(False, 0.0), (True, 0.0), (True, 0.75)])
def test_h_exact_vs_float64(oracle, shared, clamp):
    """The parity checker's yardstick: h with gate/up summed in float64 equals
    the numpy float64 restatement (dequantized matrices times the dequantized
    Q8_0 of x) to float64 rounding, routed and shared rows alike, with the
    clamp engaged (large exponents) or not; and the oracle's own f32 h sits
    within f32 summation error of it."""
    H, F, E, k, T = 256, 96, 6, 3, 4
    L = _tiny_layer(oracle, 41, H, F, E, k, shared, clamp, e_lo=128 if clamp else 120, e_span=4)
    rng = np.random.default_rng(42)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = np.ones((T, k), np.float32)
    h, hs = L.h_exact(x, ids, n_threads=3)
    _, want = np_ref.moe_forward_f64(L, x, ids, wts, oracle.quantize_q8_0)
    scale = np.abs(want).max()
    assert np.max(np.abs(h - want)) <= 1e-13 * scale
    if clamp:
        assert np.abs(want).max() <= clamp * clamp  # silu(g) <= g <= L and |u| <= L
    if shared:
        xq, xd = oracle.quantize_q8_0(x)
        xa = np_ref.q8_dequant(xq, xd)
        G, U = (np_ref.dequant_blocks(m) for m in L.shared[:2])
        want_s = np_ref.swiglu(xa @ G.T, xa @ U.T, clamp)
        assert np.max(np.abs(hs - want_s)) <= 1e-13 * np.abs(want_s).max()
    else:
        assert hs is None
    f32 = L.forward(x, ids, wts, taps=True)["h"]
    assert 0 < np.max(np.abs(f32 - h)) <= 1e-5 * scale


@pytest.mark.parametrize("clamp", [0.0, 2.0])
def test_h_bound_covers_other_orders_and_catches_a_dropped_term(oracle, clamp):
    """The checker's per-value f32 bound (h_bound) holds for f32 evaluations
    in orders other than the oracle's (the block terms summed in reverse, and
    pairwise, in numpy float32; the oracle's own h), and is tight enough that
    losing the largest block term of gate puts every value outside it whose
    h that loss moves by more than twice the bound -- most values, where no
    clamp hides it."""
    H, F, E, k, T = 1024, 64, 4, 2, 3
    L = _tiny_layer(oracle, 43, H, F, E, k, False, clamp, e_lo=126 if clamp else 122, e_span=4)
    rng = np.random.default_rng(44)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    h, _ = L.h_exact(x, ids)
    b, _ = L.h_bound(x, ids)
    f32 = L.forward(x, ids, np.ones((T, k), np.float32), taps=True)["h"]
    assert np.all(np.abs(f32.astype(np.float64) - h) <= b)
    xq, xd = oracle.quantize_q8_0(x)
    xa = np_ref.q8_dequant(xq, xd)  # [T, H] float64, exact
    nb = H // 32

    def act(g, u):  # clamp and SwiGLU in float32
        if clamp:
            u = np.clip(u, np.float32(-clamp), np.float32(clamp))
            g = np.minimum(g, np.float32(clamp))
        return (g / (np.float32(1) + np.exp(-g))) * u

    caught = total = 0
    for t in range(T):
        for s in range(k):
            G, U = (np_ref.dequant_blocks(m) for m in (L.gate[ids[t, s]], L.up[ids[t, s]]))
            tg = (G * xa[t]).reshape(F, nb, 32).sum(-1)  # [F, nb] exact block terms
            tu = (U * xa[t]).reshape(F, nb, 32).sum(-1)
            for order in ("reverse", "pairwise"):
                if order == "reverse":
                    g32 = np.zeros(F, np.float32)
                    u32 = np.zeros(F, np.float32)
                    for j in reversed(range(nb)):
                        g32 = g32 + tg[:, j].astype(np.float32)
                        u32 = u32 + tu[:, j].astype(np.float32)
                else:
                    g32, u32 = tg.astype(np.float32), tu.astype(np.float32)
                    while g32.shape[1] > 1:
                        g32 = g32[:, 0::2] + g32[:, 1::2]
                        u32 = u32[:, 0::2] + u32[:, 1::2]
                    g32, u32 = g32[:, 0], u32[:, 0]
                assert np.all(np.abs(act(g32, u32).astype(np.float64) - h[t, s]) <= b[t, s]), (t, s, order)
            # the largest term of gate lost: values where that changes h by
            # more than twice the bound in exact arithmetic (a clamp can hide
            # it) must all fall outside the bound in f32
            jg = np.argmax(np.abs(tg), axis=1)
            g_drop64 = tg.sum(1) - tg[np.arange(F), jg]
            err = np.abs(act(g_drop64.astype(np.float32), tu.sum(1).astype(np.float32)).astype(np.float64) - h[t, s])
            shift = np.abs(np_ref.swiglu(g_drop64, tu.sum(1), clamp) - h[t, s])
            visible = shift > 2 * b[t, s]
            caught += int(np.sum((err > b[t, s]) & visible))
            total += int(np.sum(visible))
            if not clamp:  # unclamped, most values show the lost term (not those where up is near 0)
                assert np.sum(visible) >= 0.7 * F, (t, s, int(np.sum(visible)))
    assert total > 0 and caught == total, (caught, total)


def test_forward_clamp_engages(oracle):
    # large weights make |g|, |u| far exceed a small limit: output must differ from unclamped
    H, F, E, k, T = 64, 64, 4, 2, 2
    L1 = _tiny_layer(oracle, 21, H, F, E, k, False, 0.0, e_lo=130, e_span=2)
    L2 = _tiny_layer(oracle, 21, H, F, E, k, False, 0.75, e_lo=130, e_span=2)
    rng = np.random.default_rng(22)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.array([[0, 1], [2, 3]], np.int32)
    wts = np.full((T, k), 0.5, np.float32)
    a = L1.forward(x, ids, wts, taps=True)
    b = L2.forward(x, ids, wts, taps=True)
    assert np.abs(a["h"]).max() > 5 * np.abs(b["h"]).max()
    want, _ = np_ref.moe_forward_f64(L2, x, ids, wts, oracle.quantize_q8_0)
    rms = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(b["out"] - want)) <= 1e-4 * rms


def test_forward_thread_count_invariant(oracle):
    H, F, E, k, T = 256, 128, 8, 4, 5
    L = _tiny_layer(oracle, 31, H, F, E, k, True, 0.0)
    rng = np.random.default_rng(32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = rng.uniform(0.1, 0.4, (T, k)).astype(np.float32)
    a = L.forward(x, ids, wts, n_threads=1)["out"]
    b = L.forward(x, ids, wts, n_threads=7)["out"]
    np.testing.assert_array_equal(a, b)


def test_vec_dot8_bit_exact_with_vec_dot(oracle):
    # the CPU baseline's eight-row dot against the scalar one, row by row:
    # random nibbles, codes at both ends of Q8_0's range, denormal and large
    # block scales, zero d
    rng = np.random.default_rng(41)
    for K in (32, 256, 7168):
        nb = K // 32
        for trial in range(4):
            rows = rng.integers(0, 256, (8, nb, 17), dtype=np.uint8)
            rows[:, :, 0] = rng.choice([0, 1, 2, 100, 127, 128, 140, 200], (8, nb))
            qs = rng.integers(-127, 128, K).astype(np.int8)
            qs[: min(K, 40)] = np.resize(np.array([127, -127], np.int8), min(K, 40))
            d = np.array([oracle.fp32_to_fp16_bits(float(v)) for v in rng.uniform(1e-4, 0.5, nb)], np.uint16)
            d[trial % nb] = 0
            got = oracle.vec_dot8(rows, qs, d)
            for r in range(8):
                want = np.float32(oracle.vec_dot(rows[r:r + 1], qs, d))
                assert got[r].view(np.uint32) == want.view(np.uint32), (K, trial, r, got[r], want)


@pytest.mark.parametrize("shared,clamp,threads", [(False, 0.0, 1), (True, 0.0, 3), (True, 0.75, 8)])
def test_forward_rows8_bit_exact_with_forward(oracle, shared, clamp, threads):
    H, F, E, k, T = 256, 128, 8, 4, 5
    L = _tiny_layer(oracle, 37, H, F, E, k, shared, clamp)
    rng = np.random.default_rng(38)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = rng.uniform(0.1, 0.4, (T, k)).astype(np.float32)
    a = L.forward(x, ids, wts, n_threads=1)["out"]
    b = L.forward_rows8(x, ids, wts, n_threads=threads)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- generator ----------------------------------------------------------------------

def test_mix64_known_answer(oracle):
    # SplitMix64 seeded with 0: first outputs as published with the algorithm
    assert oracle.lib().mo_mix64(0) == 0xE220A8397B1DCDAF
    assert oracle.lib().mo_mix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4


def test_generator_distribution(oracle):
    b = oracle.gen_mxfp4(99, 0, 0, 5, 512, 2048)
    e = b[:, :, 0].ravel()
    assert e.min() == 124 and e.max() == 130
    cnt_e = np.bincount(e - 124, minlength=7)
    assert np.all(np.abs(cnt_e / cnt_e.sum() - 1 / 7) < 0.01)
    nib = np.concatenate([(b[:, :, 1:] & 0xF).ravel(), (b[:, :, 1:] >> 4).ravel()])
    cnt = np.bincount(nib, minlength=16) / nib.size
    assert np.all(np.abs(cnt - 1 / 16) < 0.002)
    # different (layer, tensor, expert) keys give different bytes
    assert not np.array_equal(b, oracle.gen_mxfp4(99, 0, 0, 6, 512, 2048))
    assert not np.array_equal(b, oracle.gen_mxfp4(99, 0, 1, 5, 512, 2048))


def test_forward_from_h_reproduces_forward(oracle):
    """The oracle's down path from a given h, fed the oracle's own h, is the
    oracle's forward bit for bit (with and without the shared expert)."""
    for shared in (False, True):
        H, F, E, k, T = 256, 128, 8, 2, 3
        rng = np.random.default_rng(5)
        x = rng.standard_normal((T, H), dtype=np.float32)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        wts = rng.random((T, k), dtype=np.float32)
        L = oracle.OracleLayer.generated(9, 0, H, F, E, k, experts=list(range(E)), shared=shared)
        ref = L.forward(x, ids, wts, taps=True)
        got = L.forward_from_h(ids, wts, ref["h"], ref["h_shared"])
        np.testing.assert_array_equal(got, ref["out"])
