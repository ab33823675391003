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
    say(f"{what} rms(ref)={r:.4e} max|diff|={err:.3e} ratio={err / r:.3e}" + (f" non-finite={nf}" if nf else ""))
    assert err <= tol * r, f"{what}: max|diff| {err:.3e} > {tol} * rms {r:.3e}"


class Taps:
    """Stands in for the block in check_block when the h taps were already
    read (a subset of the tokens of a larger call)."""

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


def check_block(oracle, L, blk, shape, x, ids, wts, got, what, n_threads=16, per_slot=False, tol=TOL):
    """Parity of one forward, in two stages.

    1. gate/up + clamp + SwiGLU: the GPU's h against the oracle's h, max|dh|
       <= 2e-4 * max|h| per row (only the f32 summation order differs; the
       bound leaves room for cancellation in the gate/up sums, which is
       large when the clamp is active).
    2. The output, max|d| <= tol * RMS: against the oracle run end to end
       for every token (per_slot: every (token, slot) row) whose Q8_0(h)
       codes come out identical on both sides; where an h value sits so
       close to a Q8_0 rounding boundary that the two f32 orders round it to
       neighbouring codes, against the oracle's down path fed the GPU's h
       (the same Q8_0(h) codes: the activation quantization reproduced).
       The number of such tokens (rows) is reported.

    got: [T, H], or [T, k, H] with per_slot (the weighted per-slot rows, the
    shared expert not included)."""
    ref = L.forward(x, ids, wts, n_threads=n_threads, taps=True, per_slot=per_slot)
    hg, hgs = gpu_h(blk, oracle, shape, ids, shared=False if per_slot else None)
    pairs = [(hg, ref["h"], "h")] + ([(hgs, ref["h_shared"], "h shared")] if hgs is not None else [])
    for a, b, nm in pairs:
        a2 = a.reshape(-1, a.shape[-1]).astype(np.float64)
        b2 = b.reshape(-1, b.shape[-1]).astype(np.float64)
        scale = np.maximum(np.abs(b2).max(axis=1, keepdims=True), 1e-30)
        worst = float((np.abs(a2 - b2) / scale).max())
        say(f"{what} {nm}: max|dh|/max|h| = {worst:.3e}")
        assert worst <= 2e-4, f"{what} {nm}: max|dh|/max|h| = {worst:.3e}"
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
