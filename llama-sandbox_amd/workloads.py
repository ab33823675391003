"""Synthetic workloads of the MoE-block benchmark configurations.

Shapes and input distributions for the five configurations the block is
measured and parity-tested on.  Weights are never materialised here: they
are generated on the device by moe_layer_generate (counter-based, seeded by
(seed, layer, tensor, expert, block)), with nibbles uniform over all 16 codes
and E8M0 exponents uniform in [124, 130].

Inputs: activations N(0,1) (f32 for C1; rounded through bf16 for C2-C5),
router logits N(0,1) f32, optionally plus a per-expert Zipf(s=1.1) bias
ln p_{pi(e)} with p_r ~ (r+1)^-1.1 and pi a seeded permutation, which makes
the tokens-per-expert histogram skewed and ragged.
"""
from __future__ import annotations

import dataclasses

import numpy as np

ROUTE_SOFTMAX, ROUTE_SIGMOID, ROUTE_SQRT_SOFTPLUS = 0, 1, 2
E_LO, E_SPAN = 124, 7


@dataclasses.dataclass(frozen=True)
class LayerShape:
    hidden: int
    ffn: int
    n_expert: int
    n_used: int
    has_shared: bool
    route_mode: int
    norm: bool = True
    scale: float = 1.0
    clamp: float = 0.0
    bf16_act: bool = False

    @property
    def block_bytes_gu(self) -> int:
        """MXFP4 bytes of one gate (or up) matrix."""
        return self.ffn * (self.hidden // 32) * 17

    @property
    def block_bytes_down(self) -> int:
        return self.hidden * (self.ffn // 32) * 17

    @property
    def expert_bytes(self) -> int:
        return 2 * self.block_bytes_gu + self.block_bytes_down

    @property
    def layer_bytes(self) -> int:
        return (self.n_expert + int(self.has_shared)) * self.expert_bytes

    def touched_bytes(self, ids: np.ndarray) -> int:
        """Algorithmic HBM bytes of one call: every distinct routed expert in
        ids, plus the shared expert, read once."""
        return (len(np.unique(ids)) + int(self.has_shared)) * self.expert_bytes

    def flops(self, T: int) -> int:
        rows = T * self.n_used + (T if self.has_shared else 0)
        return 2 * rows * (2 * self.ffn * self.hidden + self.hidden * self.ffn)


# C1: CPU-runnable correctness case (softmax over 32, top-4 renormalised)
C1 = LayerShape(hidden=2048, ffn=768, n_expert=32, n_used=4, has_shared=False,
                route_mode=ROUTE_SOFTMAX)
# C2-C5: DeepSeek-V3-shaped layer (sigmoid over 256, top-8 renormalised over
# the selected 8, one shared expert of the same shape)
V3 = LayerShape(hidden=7168, ffn=2048, n_expert=256, n_used=8, has_shared=True,
                route_mode=ROUTE_SIGMOID, bf16_act=True)

# Shapes beyond the configurations, for the prefill kernels' other instances:
# the reference's DeepSeek-V4-Pro layer (hip-moe/README.md:280-286: 7168 -> 3072,
# 384 experts, top-6 sqrt(softplus) routing renormalised and scaled by 2.5,
# clamped SwiGLU, one shared expert), and the V3 layer with 1536-wide experts.
V4P = LayerShape(hidden=7168, ffn=3072, n_expert=384, n_used=6, has_shared=True,
                 route_mode=ROUTE_SQRT_SOFTPLUS, scale=2.5, clamp=10.0, bf16_act=True)
V3F1536 = LayerShape(hidden=7168, ffn=1536, n_expert=256, n_used=8, has_shared=True,
                     route_mode=ROUTE_SIGMOID, bf16_act=True)

CONFIGS = {
    "C1": dict(shape=C1, tokens=(1,), zipf=False),
    "C2": dict(shape=V3, tokens=(1,), zipf=False),
    "C3": dict(shape=V3, tokens=(4, 16, 64), zipf=True),
    "C4": dict(shape=V3, tokens=(512,), zipf=None),  # uniform and Zipf
    "C5": dict(shape=V3, tokens=(1,), zipf=False, layers=40),
    "V4P": dict(shape=V4P, tokens=(512,), zipf=None),
    "F1536": dict(shape=V3F1536, tokens=(512,), zipf=None),
}


def round_bf16(x: np.ndarray) -> np.ndarray:
    """f32 -> nearest bf16 (ties to even) -> f32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).reshape(np.shape(x))


def zipf_bias(E: int, seed: int, s: float = 1.1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    p = (np.arange(E, dtype=np.float64) + 1.0) ** (-s)
    p /= p.sum()
    perm = rng.permutation(E)
    return np.log(p[perm]).astype(np.float32)


def make_inputs(shape: LayerShape, T: int, seed: int, zipf: bool = False):
    """Activations x [T, H] f32 and router logits [T, E] f32."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, shape.hidden), dtype=np.float32)
    if shape.bf16_act:
        x = round_bf16(x)
    logits = rng.standard_normal((T, shape.n_expert), dtype=np.float32)
    if zipf:
        logits = (logits + zipf_bias(shape.n_expert, seed ^ 0x5EED)[None, :]).astype(np.float32)
    return x, logits
