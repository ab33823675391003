"""ctypes wrapper of the CPU oracle (oracle/libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker / the CPU baseline, never
as the thing measured.  The product (llama-sandbox_amd/) never imports this.

Every function follows moe_oracle.c, which cites the reference file:line it
restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "libmoe_oracle.so")

ROUTE_SOFTMAX, ROUTE_SIGMOID, ROUTE_SQRT_SOFTPLUS = 0, 1, 2
T_GATE, T_UP, T_DOWN, T_SH_GATE, T_SH_UP, T_SH_DOWN = range(6)

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


class _Layer(ctypes.Structure):
    _fields_ = [
        ("H", ctypes.c_int), ("F", ctypes.c_int), ("E", ctypes.c_int), ("k", ctypes.c_int),
        ("clamp", ctypes.c_float),
        ("gate", ctypes.POINTER(_u8p)), ("up", ctypes.POINTER(_u8p)), ("down", ctypes.POINTER(_u8p)),
        ("sh_gate", _u8p), ("sh_up", _u8p), ("sh_down", _u8p),
    ]


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    if force or not os.path.exists(_LIB):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        L.mo_e8m0_half.restype = ctypes.c_float
        L.mo_e8m0_half.argtypes = [ctypes.c_uint8]
        L.mo_fp32_to_fp16.restype = ctypes.c_uint16
        L.mo_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.mo_fp16_to_fp32.restype = ctypes.c_float
        L.mo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.mo_fp32_to_bf16.restype = ctypes.c_uint16
        L.mo_fp32_to_bf16.argtypes = [ctypes.c_float]
        L.mo_bf16_to_fp32.restype = ctypes.c_float
        L.mo_bf16_to_fp32.argtypes = [ctypes.c_uint16]
        L.mo_dequant_mxfp4_row.argtypes = [_u8p, ctypes.c_int, _f32p]
        L.mo_quantize_q8_0.argtypes = [_f32p, ctypes.c_int, _i8p, _u16p]
        L.mo_block_isum.restype = ctypes.c_int32
        L.mo_block_isum.argtypes = [_u8p, _i8p]
        L.mo_vec_dot_mxfp4_q8_0.restype = ctypes.c_float
        L.mo_vec_dot_mxfp4_q8_0.argtypes = [ctypes.c_int, _u8p, _i8p, _u16p]
        L.mo_route.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, ctypes.c_float, _i32p, _f32p]
        L.mo_route_scores.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.mo_group.restype = ctypes.c_int
        L.mo_group.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i32p, _i32p]
        L.mo_moe_forward_taps.restype = ctypes.c_int
        L.mo_moe_forward_taps.argtypes = [ctypes.POINTER(_Layer), ctypes.c_int, _f32p, _i32p, _f32p, _f32p,
                                          _f32p, _f32p, _f32p, ctypes.c_int]
        L.mo_moe_forward_from_h.restype = ctypes.c_int
        L.mo_moe_forward_from_h.argtypes = [ctypes.POINTER(_Layer), ctypes.c_int, _i32p, _f32p, _f32p, _f32p,
                                            _f32p, ctypes.c_int]
        L.mo_moe_forward_rows8.restype = ctypes.c_int
        L.mo_moe_forward_rows8.argtypes = [ctypes.POINTER(_Layer), ctypes.c_int, _f32p, _i32p, _f32p, _f32p,
                                           ctypes.c_int]
        L.mo_vec_dot8_mxfp4_q8_0.argtypes = [ctypes.c_int, _u8p, ctypes.c_size_t, _i8p, _u16p, _f32p]
        L.mo_simd_available.restype = ctypes.c_int
        L.mo_moe_h_exact.restype = ctypes.c_int
        L.mo_moe_h_exact.argtypes = [ctypes.POINTER(_Layer), ctypes.c_int, _f32p, _i32p, _f64p, _f64p,
                                     ctypes.c_int]
        L.mo_moe_h_bound.restype = ctypes.c_int
        L.mo_moe_h_bound.argtypes = [ctypes.POINTER(_Layer), ctypes.c_int, _f32p, _i32p, _f64p, _f64p,
                                     ctypes.c_int]
        L.mo_mix64.restype = ctypes.c_uint64
        L.mo_mix64.argtypes = [ctypes.c_uint64]
        L.mo_gen_key.restype = ctypes.c_uint64
        L.mo_gen_key.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.mo_gen_mxfp4.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, ctypes.c_int, _u8p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def vec_dot8(blocks: np.ndarray, qs: np.ndarray, d: np.ndarray) -> np.ndarray:
    """mo_vec_dot8_mxfp4_q8_0 over 8 rows of MXFP4 blocks [8, K/32, 17]
    against one Q8_0 vector (qs int8 [K], d fp16 bits [K/32])."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    qs = np.ascontiguousarray(qs, np.int8)
    d = np.ascontiguousarray(d, np.uint16)
    assert blocks.shape[0] == 8 and blocks.shape[2] == 17
    K = blocks.shape[1] * 32
    out = np.empty(8, np.float32)
    lib().mo_vec_dot8_mxfp4_q8_0(K, _p(blocks, _u8p), blocks.shape[1] * 17, _p(qs, _i8p), _p(d, _u16p),
                                 _p(out, _f32p))
    return out


def simd_available() -> bool:
    return bool(lib().mo_simd_available())


# ---- formats -----------------------------------------------------------------

def e8m0_half(e: int) -> float:
    return float(lib().mo_e8m0_half(e))


def fp32_to_fp16_bits(x: float) -> int:
    return int(lib().mo_fp32_to_fp16(x))


def fp16_bits_to_fp32(h: int) -> float:
    return float(lib().mo_fp16_to_fp32(h))


def dequant_mxfp4(blocks: np.ndarray, K: int) -> np.ndarray:
    """blocks: uint8 [rows, K/32, 17] (or flat) -> f32 [rows, K]."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, K // 32 * 17)
    out = np.empty((b.shape[0], K), np.float32)
    for r in range(b.shape[0]):
        lib().mo_dequant_mxfp4_row(_p(b[r], _u8p), K, _p(out[r], _f32p))
    return out


def quantize_q8_0(x: np.ndarray):
    """x: f32 [..., K] -> (qs int8 [..., K], d uint16 fp16 bits [..., K/32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    flat = x.reshape(-1, K)
    qs = np.empty(flat.shape, np.int8)
    d = np.empty((flat.shape[0], K // 32), np.uint16)
    for r in range(flat.shape[0]):
        lib().mo_quantize_q8_0(_p(flat[r], _f32p), K, _p(qs[r], _i8p), _p(d[r], _u16p))
    return qs.reshape(x.shape), d.reshape(x.shape[:-1] + (K // 32,))


def block_isum(wblock: np.ndarray, q: np.ndarray) -> int:
    wb = np.ascontiguousarray(wblock, dtype=np.uint8)
    qq = np.ascontiguousarray(q, dtype=np.int8)
    return int(lib().mo_block_isum(_p(wb, _u8p), _p(qq, _i8p)))


def vec_dot(wrow: np.ndarray, qs: np.ndarray, d: np.ndarray) -> float:
    wr = np.ascontiguousarray(wrow, dtype=np.uint8)
    q = np.ascontiguousarray(qs, dtype=np.int8)
    dd = np.ascontiguousarray(d, dtype=np.uint16)
    return float(lib().mo_vec_dot_mxfp4_q8_0(q.size, _p(wr, _u8p), _p(q, _i8p), _p(dd, _u16p)))


# ---- routing / grouping ---------------------------------------------------------

def route(logits: np.ndarray, k: int, mode: int, norm: bool = True, scale: float = 1.0,
          bias: np.ndarray | None = None):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    ids = np.empty((T, k), np.int32)
    wts = np.empty((T, k), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().mo_route(_p(lg, _f32p), None if b is None else _p(b, _f32p), T, E, k, mode, int(norm),
                   scale, _p(ids, _i32p), _p(wts, _f32p))
    return ids, wts


def route_scores(logits: np.ndarray, mode: int) -> np.ndarray:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    p = np.empty((T, E), np.float32)
    lib().mo_route_scores(_p(lg, _f32p), T, E, mode, _p(p, _f32p))
    return p


def group(ids: np.ndarray, E: int):
    """ids int32 [T, k] -> dict(counts, offsets, perm, inv, distinct)."""
    i = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = i.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    inv = np.empty(T * k, np.int32)
    n = lib().mo_group(_p(i, _i32p), T, k, E, _p(counts, _i32p), _p(offsets, _i32p), _p(perm, _i32p),
                       _p(inv, _i32p))
    return dict(counts=counts, offsets=offsets, perm=perm, inv=inv, distinct=int(n))


# ---- weights ----------------------------------------------------------------------

def gen_mxfp4(seed: int, layer: int, tensor: int, expert: int, rows: int, K: int,
              e_lo: int = 124, e_span: int = 7) -> np.ndarray:
    """Counter-based synthetic MXFP4 matrix, uint8 [rows, K/32, 17]."""
    out = np.empty((rows, K // 32, 17), np.uint8)
    lib().mo_gen_mxfp4(seed, layer, tensor, expert, rows, K, e_lo, e_span, _p(out, _u8p))
    return out


class OracleLayer:
    """Host MXFP4 tensors of one layer in ggml layout, keyed by expert.

    gate/up: {e: uint8 [F, H/32, 17]}, down: {e: uint8 [H, F/32, 17]}; only
    the experts a call touches need to be present.  shared: (gate, up, down)
    or None.
    """

    def __init__(self, H, F, E, k, gate, up, down, shared=None, clamp=0.0):
        self.H, self.F, self.E, self.k, self.clamp = H, F, E, k, float(clamp)
        self.gate = {int(e): np.ascontiguousarray(v, np.uint8) for e, v in gate.items()}
        self.up = {int(e): np.ascontiguousarray(v, np.uint8) for e, v in up.items()}
        self.down = {int(e): np.ascontiguousarray(v, np.uint8) for e, v in down.items()}
        self.shared = None if shared is None else tuple(np.ascontiguousarray(v, np.uint8) for v in shared)

    @classmethod
    def generated(cls, seed, layer, H, F, E, k, experts, shared=False, clamp=0.0, e_lo=124, e_span=7):
        g = {e: gen_mxfp4(seed, layer, T_GATE, e, F, H, e_lo, e_span) for e in experts}
        u = {e: gen_mxfp4(seed, layer, T_UP, e, F, H, e_lo, e_span) for e in experts}
        d = {e: gen_mxfp4(seed, layer, T_DOWN, e, H, F, e_lo, e_span) for e in experts}
        sh = None
        if shared:
            sh = (gen_mxfp4(seed, layer, T_SH_GATE, 0, F, H, e_lo, e_span),
                  gen_mxfp4(seed, layer, T_SH_UP, 0, F, H, e_lo, e_span),
                  gen_mxfp4(seed, layer, T_SH_DOWN, 0, H, F, e_lo, e_span))
        return cls(H, F, E, k, g, u, d, sh, clamp)

    def _struct(self):
        E = self.E
        arrs = []
        gp = (_u8p * E)()
        upp = (_u8p * E)()
        dp = (_u8p * E)()
        for e in range(E):
            for src, dst in ((self.gate, gp), (self.up, upp), (self.down, dp)):
                a = src.get(e)
                dst[e] = _p(a, _u8p) if a is not None else None
        s = _Layer(self.H, self.F, E, self.k, self.clamp, gp, upp, dp,
                   _p(self.shared[0], _u8p) if self.shared else None,
                   _p(self.shared[1], _u8p) if self.shared else None,
                   _p(self.shared[2], _u8p) if self.shared else None)
        arrs.extend([gp, upp, dp])
        return s, arrs

    def forward(self, x: np.ndarray, ids: np.ndarray, wts: np.ndarray, n_threads: int = 1,
                per_slot: bool = False, taps: bool = False):
        """x f32 [T, H], ids int32 [T, k], wts f32 [T, k] -> out f32 [T, H]
        (and per-slot rows [T, k, H], h taps if asked)."""
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        wts = np.ascontiguousarray(wts, np.float32)
        T = x.shape[0]
        out = np.empty((T, self.H), np.float32)
        ps = np.empty((T, self.k, self.H), np.float32) if per_slot else None
        hr = np.empty((T, self.k, self.F), np.float32) if taps else None
        hs = np.empty((T, self.F), np.float32) if (taps and self.shared) else None
        s, keep = self._struct()
        rc = lib().mo_moe_forward_taps(ctypes.byref(s), T, _p(x, _f32p), _p(ids, _i32p), _p(wts, _f32p),
                                       _p(out, _f32p), None if ps is None else _p(ps, _f32p),
                                       None if hr is None else _p(hr, _f32p),
                                       None if hs is None else _p(hs, _f32p), int(n_threads))
        del keep
        if rc != 0:
            raise ValueError("oracle forward rejected its arguments")
        res = {"out": out}
        if per_slot:
            res["per_slot"] = ps
        if taps:
            res["h"] = hr
            res["h_shared"] = hs
        return res

    def forward_rows8(self, x: np.ndarray, ids: np.ndarray, wts: np.ndarray, n_threads: int = 1) -> np.ndarray:
        """forward()'s out, bit for bit, with the dot products eight rows at
        a time (AVX2 where present): the CPU baseline's path."""
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        wts = np.ascontiguousarray(wts, np.float32)
        T = x.shape[0]
        out = np.empty((T, self.H), np.float32)
        s, keep = self._struct()
        rc = lib().mo_moe_forward_rows8(ctypes.byref(s), T, _p(x, _f32p), _p(ids, _i32p), _p(wts, _f32p),
                                        _p(out, _f32p), int(n_threads))
        del keep
        if rc != 0:
            raise ValueError("oracle forward rejected its arguments")
        return out

    def h_exact(self, x: np.ndarray, ids: np.ndarray, n_threads: int = 1):
        """The SwiGLU output with gate/up summed exactly in float64 (same
        Q8_0 of x as forward): (h [T, k, F] float64, shared [T, F] or None).
        The yardstick of the parity checker: the f32 error of forward's h and
        of the device's h are both measured against it."""
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        T = x.shape[0]
        hr = np.empty((T, self.k, self.F), np.float64)
        hs = np.empty((T, self.F), np.float64) if self.shared else None
        s, keep = self._struct()
        rc = lib().mo_moe_h_exact(ctypes.byref(s), T, _p(x, _f32p), _p(ids, _i32p), _p(hr, _f64p),
                                  None if hs is None else _p(hs, _f64p), int(n_threads))
        del keep
        if rc != 0:
            raise ValueError("oracle h_exact rejected its arguments")
        return hr, hs

    def h_bound(self, x: np.ndarray, ids: np.ndarray, n_threads: int = 1):
        """Per value of h_exact's h, a bound on the error of any f32
        evaluation that sums the gate/up block terms in any order (same
        layout as h_exact: [T, k, F], shared [T, F] or None)."""
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        T = x.shape[0]
        br = np.empty((T, self.k, self.F), np.float64)
        bs = np.empty((T, self.F), np.float64) if self.shared else None
        s, keep = self._struct()
        rc = lib().mo_moe_h_bound(ctypes.byref(s), T, _p(x, _f32p), _p(ids, _i32p), _p(br, _f64p),
                                  None if bs is None else _p(bs, _f64p), int(n_threads))
        del keep
        if rc != 0:
            raise ValueError("oracle h_bound rejected its arguments")
        return br, bs

    def forward_from_h(self, ids: np.ndarray, wts: np.ndarray, h: np.ndarray, h_shared=None,
                       n_threads: int = 1, per_slot: bool = False):
        """The block from a given SwiGLU output: h f32 [T, k, F] (and the
        shared expert's [T, F]) -> Q8_0(h) -> down x router weight ->
        combine -> out f32 [T, H] (per_slot: (out, the weighted per-slot rows
        [T, k, H])).  A test passes another implementation's h here to
        reproduce its activation quantization exactly."""
        ids = np.ascontiguousarray(ids, np.int32)
        wts = np.ascontiguousarray(wts, np.float32)
        T = ids.shape[0]
        rows = [np.asarray(h, np.float32).reshape(T * self.k, self.F)]
        if self.shared:
            rows.append(np.asarray(h_shared, np.float32).reshape(T, self.F))
        hh = np.ascontiguousarray(np.concatenate(rows, axis=0), np.float32)
        out = np.empty((T, self.H), np.float32)
        ps = np.empty((T, self.k, self.H), np.float32) if per_slot else None
        s, keep = self._struct()
        rc = lib().mo_moe_forward_from_h(ctypes.byref(s), T, _p(ids, _i32p), _p(wts, _f32p), _p(hh, _f32p),
                                         _p(out, _f32p), None if ps is None else _p(ps, _f32p), int(n_threads))
        del keep
        if rc != 0:
            raise ValueError("oracle forward_from_h rejected its arguments")
        return (out, ps) if per_slot else out
