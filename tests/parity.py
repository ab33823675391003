"""Parity checks shared by the GPU tests: the block's output against the CPU
oracle under the contract max|gpu - oracle| <= 1e-3 * RMS(oracle output),
with the activation quantization reproduced.

The reference's gates (hip-moe/src/moe_ggml_bench.cpp:308-321) normalise by
the reference RMS because near-zero outputs make a relative gate
meaningless; the build's contract tightens them to 1e-3 of the RMS.
"""
import numpy as np

import moe_block as mb

TOL = 1e-3  # max-abs error as a fraction of the oracle output's RMS


def say(*a):
    print("[gpu]", *a, flush=True)


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def assert_rms_close(got, ref, tol=TOL, what=""):
    """max|got - ref| <= tol * RMS(ref) over the finite outputs, and the same
    outputs non-finite on both sides.  The synthetic weights (E8M0 up to 2^2,
    codes up to 12) make |h| exceed 65504 * 127 for some tokens; Q8_0 stores
    d = amax/127 as fp16 (ggml's block_q8_0), so d becomes inf and the down
    rows of that slot inf/NaN, on the oracle exactly as in ggml-cpu."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin), f"{what}: non-finite outputs differ"
    if not fin.any():
        say(f"{what} all {ref.size} outputs non-finite on both sides")
        return
    r = rms(ref[fin])
    err = float(np.max(np.abs(got[fin] - ref[fin])))
    nf = int(ref.size - fin.sum())
    ratio = err / r if r > 0 else (0.0 if err == 0 else float("inf"))  # an all-zero reference row must be met exactly
    say(f"{what} rms(ref)={r:.4e} max|diff|={err:.3e} ratio={ratio:.3e}" + (f" non-finite={nf}" if nf else ""))
    assert err <= tol * r, f"{what}: max|diff| {err:.3e} > {tol} * rms {r:.3e}"


class Taps:
    """Stands in for the block in check_block when the h taps are at hand
    already, in the oracle's row order (routed [T, k, F], shared [T, F] or
    None): read back from another process, or planted by a CPU test."""

    def __init__(self, h, h_shared):
        self.h, self.h_shared = h, h_shared


def gpu_h(blk, oracle, shape, ids, shared=None):
    """The GPU's SwiGLU output (pre-quantization) of the last forward, in the
    oracle's row order: routed [T, k, F] (pair t*k+s) and shared [T, F] or
    None.  Decode (T == 1) keeps one row per slot; the grouped chain keeps
    grouped rows (pair p at row inv[p]) then the shared expert's T rows."""
    if isinstance(blk, Taps):
        return blk.h, blk.h_shared
    T, k = ids.shape
    F, P = shape.ffn, T * k
    has_sh = shape.has_shared if shared is None else shared
    n = P + (T if has_sh else 0)
    rows = blk.debug_last_h(n * F).reshape(n, F)
    inv = np.arange(P) if T == 1 else oracle.group(ids, shape.n_expert)["inv"]
    return rows[inv].reshape(T, k, F), (rows[P:P + T] if has_sh else None)


def _same_codes(oracle, a, b):
    qa, da = oracle.quantize_q8_0(a)
    qb, db = oracle.quantize_q8_0(b)
    return np.array_equal(qa, qb) and np.array_equal(da, db)


# Stage-1 gates on h: every value within the f32 error bound of any
# summation order (oracle.OracleLayer.h_bound), and the errors (against the
# exact float64 h of the same Q8_0(x), h_exact, each in units of its bound)
# of the oracle's own size.
H_VALUE_FACTOR = 1.0  # each value, in units of its f32 error bound
H_CALL_FACTOR = 2.0   # RMS over the call's h values
H_ROW_FACTOR = 4.0    # RMS over one h row, against the larger of its own and
                      # the call's pooled oracle error
# Stage-2 bound on Q8_0(h) codes that come out different on the two sides:
# at most FLIP_FACTOR x the number expected from errors of the oracle's size,
# plus FLIP_SLACK.
FLIP_FACTOR = 4.0
FLIP_SLACK = 4


def _rms_rows(a):
    return np.sqrt(np.mean(np.square(a), axis=-1))


def _h_gate(dev, ora, exact, bound, what):
    """dev, ora: f32 h rows [N, F]; exact, bound: float64 [N, F] (OracleLayer
    h_exact / h_bound).  Every value of both sides must lie within the bound
    of any f32 summation order (the oracle's own values check the bound
    itself); then, with each value's error in units of its bound (so that a
    value whose gate or up sum cancels, and whose bound is wide, weighs no
    more than a well-conditioned one), the device's error must be of the
    oracle's size: H_CALL_FACTOR over the call, H_ROW_FACTOR in any row."""
    dev, ora, exact, bound = (np.asarray(a, np.float64).reshape(-1, np.shape(a)[-1]) for a in (dev, ora, exact, bound))
    z_dev, z_ora = np.abs(dev - exact) / bound, np.abs(ora - exact) / bound
    r, c = np.unravel_index(int(np.argmax(z_ora)), z_ora.shape)
    assert z_ora.max() <= 1.0, f"{what}: the oracle's own h beyond its f32 error bound in row {r}, column {c}"
    r, c = np.unravel_index(int(np.argmax(z_dev)), z_dev.shape)
    assert z_dev.max() <= H_VALUE_FACTOR, (f"{what}: h value {z_dev.max():.2f}x the f32 error bound of any summation "
                                f"order in row {r}, column {c}")
    floor = 2.0 ** -24 * np.abs(exact) / bound  # one f32 rounding of h itself
    ora_call = max(float(np.sqrt(np.mean(np.square(z_ora)))), float(np.sqrt(np.mean(np.square(floor)))), 1e-30)
    call = float(np.sqrt(np.mean(np.square(z_dev)))) / ora_call
    # a row's yardstick: its own oracle error, or the call's pooled one,
    # whichever is larger (a row's own error can come from one or two values)
    rows = _rms_rows(z_dev) / np.maximum(np.maximum(_rms_rows(z_ora), ora_call), _rms_rows(floor) + 1e-30)
    say(f"{what}: rms(h err / bound) device/oracle = {call:.3f} over the call, rows max {rows.max():.3f} "
        f"median {float(np.median(rows)):.3f}, values max {z_dev.max():.3f} of the bound")
    assert call <= H_CALL_FACTOR, f"{what}: h error {call:.2f}x the oracle's own f32 error over the call"
    assert rows.max() <= H_ROW_FACTOR, (f"{what}: h error {rows.max():.2f}x the oracle's own f32 error in row "
                                        f"{int(np.argmax(rows))}")


def _code_flips(oracle, dev, ora, exact):
    """(observed, expected) code differences of Q8_0(h) between the device's
    and the oracle's h rows.  Observed: codes that differ in blocks whose d
    agrees, plus blocks whose d differs.  Expected, for two f32 orders with
    errors of the oracle's size: a code flips when a rounding boundary falls
    between the two values, with probability ~ their distance in code units
    (1.5 x the oracle's own distance from the exact h, for the difference of
    two such errors); a block's d (fp16 of amax/127) flips with probability ~
    amax's relative distance over fp16's 2^-11 step."""
    F = np.shape(dev)[-1]
    dev = np.ascontiguousarray(dev, np.float32).reshape(-1, F)
    ora = np.ascontiguousarray(ora, np.float32).reshape(-1, F)
    exact = np.asarray(exact, np.float64).reshape(-1, F)
    qa, da = oracle.quantize_q8_0(dev)
    qb, db = oracle.quantize_q8_0(ora)
    same_d = (da == db)[..., None]
    observed = int(((qa != qb).reshape(da.shape + (32,)) & same_d).sum() + (~same_d).sum())
    amax = np.abs(ora.reshape(da.shape + (32,))).max(axis=-1).astype(np.float64)
    step = 127.0 / np.maximum(amax, 1e-30)
    dist = np.abs(ora.astype(np.float64) - exact).reshape(da.shape + (32,))
    p_code = np.minimum(1.0, 1.5 * dist * step[..., None]).sum()
    a64 = np.abs(exact.reshape(da.shape + (32,))).max(axis=-1)
    p_d = np.minimum(1.0, 1.5 * np.abs(amax - a64) / np.maximum(amax, 1e-30) / 2.0 ** -11).sum()
    return observed, float(p_code + p_d)


def check_block(oracle, L, blk, shape, x, ids, wts, got, what, n_threads=16, per_slot=False, tol=TOL):
    """Parity of one forward, in two stages.

    1. gate/up + clamp + SwiGLU: the GPU's h and the oracle's (f32) h are
       both measured against the exact float64 h of the same Q8_0(x)
       (OracleLayer.h_exact).  The GPU's error may be at most H_CALL_FACTOR
       times the oracle's own f32 error in RMS over the call, and
       H_ROW_FACTOR times it in any one h row: only the f32 summation order
       may differ, so any error beyond that scale (a dropped or misscaled
       block term, a wrong clamp) fails here.
    2. The output, max|d| <= tol * RMS: against the oracle run end to end
       for every token (per_slot: every (token, slot) row) whose Q8_0(h)
       codes come out identical on both sides; where an h value sits so
       close to a Q8_0 rounding boundary that the two f32 orders round it to
       neighbouring codes, against the oracle's down path fed the GPU's h
       (the same Q8_0(h) codes: the activation quantization reproduced).
       The number of such code differences is bounded by what errors of
       the oracle's size explain (FLIP_FACTOR x expected + FLIP_SLACK).

    got: [T, H], or [T, k, H] with per_slot (the weighted per-slot rows, the
    shared expert not included)."""
    ref = L.forward(x, ids, wts, n_threads=n_threads, taps=True, per_slot=per_slot)
    h64, h64s = L.h_exact(x, ids, n_threads=n_threads)
    b64, b64s = L.h_bound(x, ids, n_threads=n_threads)
    hg, hgs = gpu_h(blk, oracle, shape, ids, shared=False if per_slot else None)
    F = hg.shape[-1]
    parts = [(hg, ref["h"], h64, b64)] + ([(hgs, ref["h_shared"], h64s, b64s)] if hgs is not None else [])
    _h_gate(*(np.concatenate([p[i].reshape(-1, F) for p in parts]) for i in range(4)), f"{what} h")
    observed, expected = 0, 0.0
    for a, b, c, _ in parts:
        o_, e_ = _code_flips(oracle, a, b, c)
        observed, expected = observed + o_, expected + e_
    say(f"{what}: {observed} Q8_0(h) code differences, {expected:.2f} expected from f32 order")
    assert observed <= FLIP_FACTOR * expected + FLIP_SLACK, (
        f"{what}: {observed} Q8_0(h) code differences, more than f32 summation order explains ({expected:.2f})")
    T, k = ids.shape
    flips = []
    for t in range(T):
        if per_slot:
            for s in range(k):
                if _same_codes(oracle, hg[t, s], ref["h"][t, s]):
                    assert_rms_close(got[t, s], ref["per_slot"][t, s], tol=tol, what=f"{what} t{t} s{s}")
                    continue
                flips.append((t, s))
                # the shared rows do not reach the per-slot output; the oracle's own stand in
                hs = None if ref["h_shared"] is None else ref["h_shared"][t:t + 1]
                _, ps = L.forward_from_h(ids[t:t + 1], wts[t:t + 1], hg[t:t + 1], hs, n_threads=n_threads,
                                         per_slot=True)
                assert_rms_close(got[t, s], ps[0, s], tol=tol, what=f"{what} t{t} s{s} (same Q8_0(h) codes)")
            continue
        codes_same = _same_codes(oracle, hg[t], ref["h"][t])
        if hgs is not None:
            codes_same = codes_same and _same_codes(oracle, hgs[t], ref["h_shared"][t])
        if codes_same:
            assert_rms_close(got[t], ref["out"][t], tol=tol, what=f"{what} t{t}")
        else:
            flips.append(t)
            same_q = L.forward_from_h(ids[t:t + 1], wts[t:t + 1], hg[t:t + 1],
                                      None if hgs is None else hgs[t:t + 1], n_threads=n_threads)
            assert_rms_close(got[t], same_q[0], tol=tol, what=f"{what} t{t} (same Q8_0(h) codes)")
    unit = "rows" if per_slot else "tokens"
    total = T * k if per_slot else T
    say(f"{what}: {len(flips)} of {total} {unit} with an h value on a Q8_0 rounding boundary", flips[:16])
    assert len(flips) <= observed
    return ref


def run_block(blk, torch_dev, layer, x, ids, wts, flags=0):
    torch, dev = torch_dev
    T = x.shape[0]
    d = blk.descs[layer]
    shape = (T, d.n_used, d.hidden) if flags & mb.MOE_FWD_PER_SLOT else (T, d.hidden)
    out = torch.empty(shape, dtype=torch.float32, device=dev)
    blk.forward(layer, torch.from_numpy(x).to(dev), torch.from_numpy(ids).to(dev),
                torch.from_numpy(wts).to(dev), out, flags)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_layer(oracle, shape, seed, layer, ids, clamp=None, e_lo=124, e_span=7, shared=None):
    return oracle.OracleLayer.generated(seed, layer, shape.hidden, shape.ffn, shape.n_expert, shape.n_used,
                                        experts=sorted(set(np.asarray(ids).ravel().tolist())),
                                        shared=shape.has_shared if shared is None else shared,
                                        clamp=shape.clamp if clamp is None else clamp, e_lo=e_lo, e_span=e_span)
