"""Writer of small GGUF files for the reader's tests.

Layout (GGUF v3): "GGUF", u32 version, u64 tensor count, u64 key/value
count, the key/value pairs (u64-length string key, u32 value type, value),
the tensor infos (name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64
offset inside the data section), zero padding to the alignment, then the
tensor data, each tensor starting on an aligned offset.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
# ggml tensor types (not the key/value types above)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16, GGML_MXFP4 = 0, 1, 8, 30, 39


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        head = struct.pack("<IQ", et, len(items))
        if et == STR:
            return head + b"".join(_str(i) for i in items)
        return head + b"".join(struct.pack(_FMT[et], i) for i in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kvs, tensors, version: int = 3, alignment: int = 32) -> bytes:
    """kvs: [(key, type, value)]; tensors: [(name, ne, ggml type, data bytes)].
    The alignment is only used for the layout: a file with another alignment
    than 32 must also carry general.alignment among kvs."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for k, t, v in kvs:
        out += _str(k) + struct.pack("<I", t) + _value(t, v)
    off, placed = 0, []
    for name, ne, ty, data in tensors:
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", ty, off)
        placed.append((off, data))
        off = (off + len(data) + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    data = bytearray(off)
    for o, d in placed:
        data[o:o + len(d)] = d
    return bytes(out + data)


def moe_keys(arch: str, n_layer: int, H: int, F: int, E: int, k: int, gating=2, norm=True, scale=2.5,
             clamp=None, clamp_sh=None):
    """The <arch>.* keys of a MoE model (clamp / clamp_sh: per-layer lists or None)."""
    kv = [("general.architecture", STR, arch), (f"{arch}.block_count", U32, n_layer),
          (f"{arch}.embedding_length", U32, H), (f"{arch}.expert_count", U32, E),
          (f"{arch}.expert_used_count", U32, k), (f"{arch}.expert_feed_forward_length", U32, F),
          (f"{arch}.expert_weights_norm", BOOL, norm), (f"{arch}.expert_weights_scale", F32, scale)]
    if gating is not None:
        kv.append((f"{arch}.expert_gating_func", U32, gating))
    if clamp is not None:
        kv.append((f"{arch}.swiglu_clamp_exp", ARR, (F32, list(clamp))))
    if clamp_sh is not None:
        kv.append((f"{arch}.swiglu_clamp_shexp", ARR, (F32, list(clamp_sh))))
    return kv


def expert_tensors(layer: int, gate: np.ndarray, up: np.ndarray, down: np.ndarray, shared=None,
                   shared_type: int = GGML_MXFP4):
    """gate/up uint8 [E, F, H/32, 17], down [E, H, F/32, 17]; shared (gate, up,
    down) [F, H/32, 17], [F, H/32, 17], [H, F/32, 17] or None."""
    E, F, kbh, _ = gate.shape
    H = kbh * 32
    b = f"blk.{layer}."
    t = [(b + "ffn_gate_exps.weight", [H, F, E], GGML_MXFP4, gate.tobytes()),
         (b + "ffn_up_exps.weight", [H, F, E], GGML_MXFP4, up.tobytes()),
         (b + "ffn_down_exps.weight", [F, H, E], GGML_MXFP4, down.tobytes())]
    if shared is not None:
        sg, su, sd = shared
        t += [(b + "ffn_gate_shexp.weight", [H, F], shared_type, sg.tobytes()),
              (b + "ffn_up_shexp.weight", [H, F], shared_type, su.tobytes()),
              (b + "ffn_down_shexp.weight", [F, H], shared_type, sd.tobytes())]
    return t
