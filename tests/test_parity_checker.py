"""The GPU parity checker (tests/parity.py check_block) on the CPU: it accepts
an implementation whose h differs from the oracle's only by f32 summation
order, and rejects planted mistakes that the older fixed gate (max|dh| <=
2e-4 max|h| per row) let through.  The "device" here is the oracle itself,
with the mistakes planted in its h taps and outputs."""
import numpy as np
import pytest

import workloads as wl
from parity import Taps, check_block


def _case(oracle, T=6, clamp=0.0, e_lo=124, e_span=7):
    shape = wl.LayerShape(hidden=2048, ffn=512, n_expert=8, n_used=4, has_shared=True,
                          route_mode=wl.ROUTE_SIGMOID, clamp=clamp)
    x, lg = wl.make_inputs(shape, T, 5)
    ids, wts = oracle.route(lg, shape.n_used, shape.route_mode, norm=True)
    L = oracle.OracleLayer.generated(77, 0, shape.hidden, shape.ffn, shape.n_expert, shape.n_used,
                                     experts=range(shape.n_expert), shared=True, clamp=clamp, e_lo=e_lo,
                                     e_span=e_span)
    ref = L.forward(x, ids, wts, taps=True, n_threads=4)
    return shape, L, x, ids, wts, ref


def _reordered_h(L, x, ids):
    """An h whose only difference from the oracle's is the f32 summation
    order: the exact h rounded to f32 (every gate/up sum correctly rounded)."""
    h64, hs64 = L.h_exact(x, ids, n_threads=4)
    return h64.astype(np.float32), hs64.astype(np.float32)


@pytest.mark.parametrize("clamp", [0.0, 0.75])
def test_accepts_the_oracle_and_a_reordered_h(oracle, clamp):
    shape, L, x, ids, wts, ref = _case(oracle, clamp=clamp, e_lo=128 if clamp else 124, e_span=3 if clamp else 7)
    check_block(oracle, L, Taps(ref["h"], ref["h_shared"]), shape, x, ids, wts, ref["out"], "oracle", n_threads=4)
    h, hs = _reordered_h(L, x, ids)
    out = L.forward_from_h(ids, wts, h, hs, n_threads=4)
    check_block(oracle, L, Taps(h, hs), shape, x, ids, wts, out, "reordered", n_threads=4)


def test_rejects_a_uniform_h_error_under_the_old_gate(oracle):
    """h off by 1e-4 relative everywhere (below the old 2e-4 gate), with the
    outputs computed from that h, so that only the h check can see it."""
    shape, L, x, ids, wts, ref = _case(oracle)
    h, hs = ref["h"] * np.float32(1 + 1e-4), ref["h_shared"] * np.float32(1 + 1e-4)
    out = L.forward_from_h(ids, wts, h, hs, n_threads=4)
    with pytest.raises(AssertionError, match="oracle's own f32 error"):
        check_block(oracle, L, Taps(h, hs), shape, x, ids, wts, out, "planted 1e-4", n_threads=4)


def test_rejects_one_bad_row(oracle):
    """One h row of 320 (token 2, slot 1) with a shift of 4x that row's own
    RMS f32 error on a single 32-block: every value still within the f32
    error bound of some summation order and the shift diluted below the
    call-level gate, but caught by the per-row gate."""
    shape, L, x, ids, wts, ref = _case(oracle, T=64)
    h, hs = ref["h"].copy(), ref["h_shared"].copy()
    h64, _ = L.h_exact(x, ids, n_threads=4)
    e_row = float(np.sqrt(np.mean((ref["h"][2, 1].astype(np.float64) - h64[2, 1]) ** 2)))
    e_row = max(e_row, 2.0 ** -24 * float(np.sqrt(np.mean(h64[2, 1] ** 2))))
    row = h[2, 1]
    row[64:96] += np.float32(4 * e_row)  # 32 of 512 values
    out = L.forward_from_h(ids, wts, h, hs, n_threads=4)
    with pytest.raises(AssertionError, match="in row"):
        check_block(oracle, L, Taps(h, hs), shape, x, ids, wts, out, "planted row", n_threads=4)


def test_rejects_code_flips_beyond_f32_order(oracle):
    """Every h value nudged across its nearest Q8_0 rounding boundary would
    send every token to the GPU-h path; the flip bound refuses it even where
    the h gate is loosened to let the values through."""
    import parity
    shape, L, x, ids, wts, ref = _case(oracle, T=4)
    q, d = oracle.quantize_q8_0(ref["h"])
    dd = np.frombuffer(d.astype(np.uint16).tobytes(), np.float16).astype(np.float32).reshape(d.shape)
    step = np.repeat(dd, 32, axis=-1)
    # move each value halfway to the next code's center: a different code almost everywhere
    h = (ref["h"] + 0.6 * step * np.sign(ref["h"])).astype(np.float32)
    out = L.forward_from_h(ids, wts, h, ref["h_shared"], n_threads=4)
    saved = parity.H_VALUE_FACTOR, parity.H_CALL_FACTOR, parity.H_ROW_FACTOR
    parity.H_VALUE_FACTOR = parity.H_CALL_FACTOR = parity.H_ROW_FACTOR = 1e30
    try:
        with pytest.raises(AssertionError, match="code differences"):
            check_block(oracle, L, Taps(h, ref["h_shared"]), shape, x, ids, wts, out, "planted flips", n_threads=4)
    finally:
        parity.H_VALUE_FACTOR, parity.H_CALL_FACTOR, parity.H_ROW_FACTOR = saved
