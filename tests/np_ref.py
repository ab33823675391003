"""Independent float64 numpy restatement used to cross-check the C oracle.

Written from the OCP Microscaling (MX) v1.0 format definitions and the block
semantics the reference states (hip-moe/src/main.hip:44-95 for the block
layout, nano-glm/lib/models/deepseek4/moe_block.h:168-215 and
glm_dsa/moe_block.h:102-133 for the op order), not from the oracle's C:
  - E2M1: 1 sign bit, 2 exponent bits (bias 1), 1 mantissa bit; exponent 0
    is subnormal (0.5 * m).  E8M0 scale: 2^(e - 127).
  - values are decoded arithmetically here, never through a lookup table,
    and matmuls are float64 numpy products over whole dequantized matrices,
    so an index, sign or transposition mistake in either side shows up.
"""
from __future__ import annotations

import numpy as np


def e2m1_value(code: int) -> float:
    sign = -1.0 if code & 8 else 1.0
    exp = (code >> 1) & 3
    man = code & 1
    if exp == 0:
        mag = 0.5 * man
    else:
        mag = 2.0 ** (exp - 1) * (1.0 + 0.5 * man)
    return sign * mag


E2M1 = np.array([e2m1_value(c) for c in range(16)], dtype=np.float64)


def dequant_blocks(blocks: np.ndarray) -> np.ndarray:
    """uint8 [rows, KB, 17] -> float64 [rows, KB*32]."""
    b = np.asarray(blocks, np.uint8)
    rows, KB, _ = b.shape
    scale = np.ldexp(1.0, b[:, :, 0].astype(np.int64) - 127)  # [rows, KB]
    qs = b[:, :, 1:]
    lo = E2M1[qs & 0x0F]
    hi = E2M1[qs >> 4]
    vals = np.concatenate([lo, hi], axis=2) * scale[:, :, None]  # element j | j+16
    return vals.reshape(rows, KB * 32)


def fp16_bits_to_f64(d: np.ndarray) -> np.ndarray:
    return np.asarray(d, np.uint16).view(np.float16).astype(np.float64)


def q8_dequant(qs: np.ndarray, d: np.ndarray) -> np.ndarray:
    """int8 [..., K], fp16 bits [..., K/32] -> float64 [..., K]."""
    q = np.asarray(qs, np.int64).astype(np.float64)
    dd = fp16_bits_to_f64(d)
    K = q.shape[-1]
    return (q.reshape(q.shape[:-1] + (K // 32, 32)) * dd[..., None]).reshape(q.shape)


def swiglu(g: np.ndarray, u: np.ndarray, clamp: float) -> np.ndarray:
    if clamp > 1e-6:
        u = np.clip(u, -clamp, clamp)
        g = np.minimum(g, clamp)
    with np.errstate(over="ignore"):  # exp(-g) -> inf for very negative g gives silu(g) -> -0
        return g / (1.0 + np.exp(-g)) * u


def moe_forward_f64(layer, x, ids, wts, quantize):
    """float64 restatement of the block over the oracle's quantizer.

    layer: oracle.OracleLayer; quantize(f32 array) -> (qs, d) is the Q8_0
    under test (pinned separately).  Returns out [T, H] float64 and h
    [T, k, F] float64 (pre-quantization).
    """
    T = x.shape[0]
    k, H, F = layer.k, layer.H, layer.F
    xq, xd = quantize(np.asarray(x, np.float32))
    xa = q8_dequant(xq, xd)  # [T, H]
    out = np.zeros((T, H), np.float64)
    hs = np.zeros((T, k, F), np.float64)
    for t in range(T):
        for s in range(k):
            e = int(ids[t, s])
            G = dequant_blocks(layer.gate[e])
            U = dequant_blocks(layer.up[e])
            D = dequant_blocks(layer.down[e])
            h = swiglu(G @ xa[t], U @ xa[t], layer.clamp)
            hs[t, s] = h
            hq, hd = quantize(h.astype(np.float32)[None, :])
            out[t] += float(wts[t, s]) * (D @ q8_dequant(hq, hd)[0])
        if layer.shared is not None:
            G, U, D = (dequant_blocks(m) for m in layer.shared)
            h = swiglu(G @ xa[t], U @ xa[t], layer.clamp)
            hq, hd = quantize(h.astype(np.float32)[None, :])
            out[t] += D @ q8_dequant(hq, hd)[0]
    return out, hs
