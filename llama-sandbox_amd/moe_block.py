"""Python binding of the gfx950 MoE block (ctypes over libmoe_block.so).

A thin host-side mirror of the C-ABI in include/moe_block.h.  Device
buffers are torch tensors on a ROCm device (torch is only the allocator and
stream owner here); every computation runs in the HIP library.  There is no
CPU fallback in this module: if the library is missing or a call fails, a
MoeError is raised and the caller decides (the reference's backend falls
back to ggml-cpu at that point, moe-serv/src/moe_backend.cpp:436-445).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoe_block.so")

MOE_OK = 0
MOE_ERR_INVALID_ARG = -1
MOE_ERR_HIP = -2
MOE_ERR_OUT_OF_BUDGET = -3
MOE_ERR_UNSUPPORTED = -4
MOE_ERR_NOT_RESIDENT = -5
MOE_ERR_NO_DEVICE = -6
MOE_ERR_INJECTED = -7
MOE_ERR_FORMAT = -8

MOE_FWD_PER_SLOT = 1
MOE_FWD_NO_SHARED = 2

ROUTE_SOFTMAX, ROUTE_SIGMOID, ROUTE_SQRT_SOFTPLUS = 0, 1, 2
T_GATE, T_UP, T_DOWN = 0, 1, 2

# every entry point include/moe_block.h declares
EXPORTS = (
    "moe_ctx_create", "moe_ctx_destroy", "moe_ctx_last_error", "moe_status_str", "moe_ctx_budget_left",
    "moe_device_memory",
    "moe_ctx_reserve", "moe_layer_upload", "moe_layer_generate", "moe_layer_read_blocks",
    "moe_layer_release", "moe_layer_bytes", "moe_route", "moe_group", "moe_forward", "moe_forward_noalloc",
    "moe_forward_host",
    "moe_route_forward", "moe_graph_capture", "moe_graph_launch", "moe_graph_destroy",
    "moe_prof_enable", "moe_prof_read", "moe_call_stats_read", "moe_debug_set_taps",
    "moe_debug_quantize_q8_0", "moe_debug_wave_sum", "moe_debug_last_h", "moe_debug_set_timeline",
    "moe_debug_read_timeline",
    "moe_gguf_read_layer", "moe_layer_upload_gguf",
    "moe_server_open", "moe_server_close", "moe_server_last_error", "moe_server_handle", "moe_server_listen",
    "moe_server_serve", "moe_router_logits", "moe_node_claimed", "moe_split_parse", "moe_split_compute",
)

# graph nodes of the ggml backend's split (include/moe_block.h, moe_node)
(NODE_NONE, NODE_RESHAPE, NODE_VIEW, NODE_PERMUTE, NODE_TRANSPOSE, NODE_MUL_MAT_ID, NODE_CLAMP, NODE_MUL, NODE_GLU,
 NODE_ADD, NODE_OTHER) = range(11)
GLU_SWIGLU = 2
GGML_F32, GGML_F16, GGML_BF16, GGML_I32, GGML_MXFP4 = 0, 1, 30, 26, 39

# nano-glm moe-server protocol v2 (include/moe_block.h, moe_wire_*)
WIRE_MAGIC, WIRE_VERSION = 0x454F4D4E, 2
WIRE_REQUEST, WIRE_RESPONSE, WIRE_HELLO = 1, 2, 3
WIRE_RET_COMBINED, WIRE_RET_PER_SLOT = 0, 1
WIRE_OK, WIRE_ERR_VERSION, WIRE_ERR_DIMS, WIRE_ERR_LAYER, WIRE_ERR_MODE, WIRE_ERR_INTERNAL = range(6)


class MoeError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


class LayerDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("ffn", ctypes.c_int32), ("n_expert", ctypes.c_int32),
                ("n_used", ctypes.c_int32), ("has_shared", ctypes.c_int32), ("clamp", ctypes.c_float)]

    @classmethod
    def of(cls, shape) -> "LayerDesc":
        return cls(shape.hidden, shape.ffn, shape.n_expert, shape.n_used, int(shape.has_shared),
                   float(shape.clamp))


class GgufLayer(ctypes.Structure):
    """moe_gguf_layer: one MoE layer of a GGUF model (shape and router keys)."""
    _fields_ = [("desc", LayerDesc), ("n_layer", ctypes.c_int32), ("route_mode", ctypes.c_int32),
                ("route_norm", ctypes.c_int32), ("route_scale", ctypes.c_float), ("shared_type", ctypes.c_int32),
                ("arch", ctypes.c_char * 32)]


class WireHelloRequest(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_uint32), ("version", ctypes.c_uint32), ("msg_type", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("payload_bytes", ctypes.c_uint64)]


class WireHelloResponse(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_uint32), ("version", ctypes.c_uint32), ("msg_type", ctypes.c_uint32),
                ("status", ctypes.c_uint32), ("arch", ctypes.c_char * 16), ("n_embd", ctypes.c_uint32),
                ("n_layer", ctypes.c_uint32), ("n_dense_lead", ctypes.c_uint32), ("n_expert", ctypes.c_uint32),
                ("n_expert_used", ctypes.c_uint32), ("n_ff_exp", ctypes.c_uint32), ("expert_scale", ctypes.c_float),
                ("expert_norm", ctypes.c_uint32), ("reserved", ctypes.c_uint32 * 2),
                ("payload_bytes", ctypes.c_uint64)]


class WireRequest(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("magic", "version", "msg_type", "layer", "n_embd", "n_tokens",
                                               "return_mode", "reserved")] + [("payload_bytes", ctypes.c_uint64)]


class WireResponse(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("magic", "version", "msg_type", "status", "n_embd", "n_tokens",
                                               "n_slots", "reserved", "t_parse_us", "t_route_us", "t_compute_us",
                                               "t_serialize_us")] + [("payload_bytes", ctypes.c_uint64)]


class MoeNode(ctypes.Structure):
    pass


MoeNode._fields_ = [("op", ctypes.c_int32), ("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                    ("contiguous", ctypes.c_int32), ("in_moe_buffer", ctypes.c_int32), ("glu_op", ctypes.c_int32),
                    ("glu_swapped", ctypes.c_int32), ("clamp_min", ctypes.c_float), ("clamp_max", ctypes.c_float),
                    ("src", ctypes.POINTER(MoeNode) * 3), ("view_src", ctypes.POINTER(MoeNode)),
                    ("data", ctypes.c_void_p), ("name", ctypes.c_char_p)]


class MoeSplit(ctypes.Structure):
    _fields_ = [(n, ctypes.POINTER(MoeNode)) for n in ("gate_w", "up_w", "down_w", "x", "ids", "wts", "out")] + \
               [(n, ctypes.c_float) for n in ("gate_min", "gate_max", "up_min", "up_max")] + \
               [(n, ctypes.c_int32) for n in ("layer", "n_slots", "n_tokens", "hidden", "ffn", "n_expert")]


class KernelStat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("launches", ctypes.c_uint64), ("total_us", ctypes.c_double)]


class CallStats(ctypes.Structure):
    """moe_call_stats: engagement and phase counters of the host-boundary calls."""
    _fields_ = [(n, ctypes.c_uint64) for n in ("calls", "refusals", "expert_loads", "timed_calls")] + \
               [(n, ctypes.c_double) for n in ("upload_us", "compute_us", "read_us", "total_us", "last_upload_us",
                                              "last_compute_us", "last_read_us", "last_total_us")] + \
               [(n, ctypes.c_uint32) for n in ("last_experts", "last_tokens", "last_timed")]


_vp = ctypes.c_void_p
_lib = None


def load_library(path: str | None = None):
    """Load libmoe_block.so; raises MoeError if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise MoeError(MOE_ERR_NO_DEVICE, f"{p} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(p)
    st = ctypes.c_int
    L.moe_ctx_create.restype = st
    L.moe_ctx_create.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.POINTER(_vp)]
    L.moe_ctx_destroy.restype = None
    L.moe_ctx_destroy.argtypes = [_vp]
    L.moe_ctx_last_error.restype = ctypes.c_char_p
    L.moe_ctx_last_error.argtypes = [_vp]
    L.moe_status_str.restype = ctypes.c_char_p
    L.moe_status_str.argtypes = [st]
    L.moe_ctx_budget_left.restype = ctypes.c_uint64
    L.moe_ctx_budget_left.argtypes = [_vp]
    L.moe_ctx_reserve.restype = st
    L.moe_ctx_reserve.argtypes = [_vp, ctypes.POINTER(LayerDesc), ctypes.c_int]
    L.moe_layer_upload.restype = st
    L.moe_layer_upload.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(LayerDesc)] + [_vp] * 6
    L.moe_layer_generate.restype = st
    L.moe_layer_generate.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(LayerDesc), ctypes.c_uint64,
                                     ctypes.c_int, ctypes.c_int]
    L.moe_layer_read_blocks.restype = st
    L.moe_layer_read_blocks.argtypes = [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp]
    L.moe_layer_release.restype = st
    L.moe_layer_release.argtypes = [_vp, ctypes.c_int]
    L.moe_layer_bytes.restype = st
    L.moe_layer_bytes.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)]
    L.moe_route.restype = st
    L.moe_route.argtypes = [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                            ctypes.c_int, ctypes.c_float, _vp, _vp, _vp]
    L.moe_group.restype = st
    L.moe_group.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp, _vp, _vp]
    L.moe_forward.restype = st
    L.moe_forward.argtypes = [_vp, ctypes.c_int, _vp, _vp, _vp, ctypes.c_int, _vp, ctypes.c_uint32, _vp]
    L.moe_forward_noalloc.restype = st
    L.moe_forward_noalloc.argtypes = [_vp, ctypes.c_int, _vp, _vp, _vp, ctypes.c_int, _vp, ctypes.c_uint32, _vp]
    L.moe_forward_host.restype = st
    L.moe_forward_host.argtypes = [_vp, ctypes.c_int, _vp, _vp, _vp, ctypes.c_int, _vp, ctypes.c_uint32]
    L.moe_route_forward.restype = st
    L.moe_route_forward.argtypes = [_vp, ctypes.c_int, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_float, _vp, _vp, _vp, ctypes.c_uint32, _vp]
    L.moe_graph_capture.restype = st
    L.moe_graph_capture.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_vp),
                                    ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                    ctypes.c_int, ctypes.c_uint32, ctypes.POINTER(_vp)]
    L.moe_graph_launch.restype = st
    L.moe_graph_launch.argtypes = [_vp, _vp]
    L.moe_graph_destroy.restype = None
    L.moe_graph_destroy.argtypes = [_vp]
    L.moe_prof_enable.restype = st
    L.moe_prof_enable.argtypes = [_vp, ctypes.c_int]
    L.moe_prof_read.restype = st
    L.moe_prof_read.argtypes = [_vp, ctypes.POINTER(KernelStat), ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                ctypes.c_int]
    L.moe_call_stats_read.restype = st
    L.moe_call_stats_read.argtypes = [_vp, ctypes.POINTER(CallStats), ctypes.c_int]
    L.moe_debug_set_taps.restype = st
    L.moe_debug_set_taps.argtypes = [_vp, ctypes.c_int]
    L.moe_debug_quantize_q8_0.restype = st
    L.moe_debug_quantize_q8_0.argtypes = [_vp, _vp, ctypes.c_int, _vp, _vp, _vp]
    L.moe_debug_wave_sum.restype = st
    L.moe_debug_wave_sum.argtypes = [_vp, _vp, ctypes.c_int, _vp, _vp]
    L.moe_debug_last_h.restype = st
    L.moe_debug_last_h.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    L.moe_debug_set_timeline.restype = st
    L.moe_debug_set_timeline.argtypes = [_vp, ctypes.c_int]
    L.moe_debug_read_timeline.restype = st
    L.moe_debug_read_timeline.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t),
                                          ctypes.POINTER(ctypes.c_size_t)]
    L.moe_gguf_read_layer.restype = st
    L.moe_gguf_read_layer.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(GgufLayer), ctypes.c_char_p,
                                      ctypes.c_size_t]
    L.moe_layer_upload_gguf.restype = st
    L.moe_layer_upload_gguf.argtypes = [_vp, ctypes.c_int, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(GgufLayer)]
    L.moe_server_open.restype = st
    L.moe_server_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_uint64, ctypes.POINTER(_vp),
                                  ctypes.c_char_p, ctypes.c_size_t]
    L.moe_server_close.restype = None
    L.moe_server_close.argtypes = [_vp]
    L.moe_server_last_error.restype = ctypes.c_char_p
    L.moe_server_last_error.argtypes = [_vp]
    L.moe_server_handle.restype = st
    L.moe_server_handle.argtypes = [_vp, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    L.moe_server_listen.restype = st
    L.moe_server_listen.argtypes = [_vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
    L.moe_server_serve.restype = st
    L.moe_server_serve.argtypes = [_vp, ctypes.c_int]
    L.moe_node_claimed.restype = ctypes.c_int
    L.moe_node_claimed.argtypes = [ctypes.POINTER(MoeNode)]
    L.moe_split_parse.restype = st
    L.moe_split_parse.argtypes = [ctypes.POINTER(ctypes.POINTER(MoeNode)), ctypes.c_int, ctypes.POINTER(MoeSplit),
                                  ctypes.c_char_p, ctypes.c_size_t]
    L.moe_split_compute.restype = st
    L.moe_split_compute.argtypes = [_vp, ctypes.POINTER(ctypes.POINTER(MoeNode)), ctypes.c_int]
    L.moe_router_logits.restype = st
    L.moe_router_logits.argtypes = [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp]
    if path is None:
        _lib = L
    return L


def node_list(nodes):
    """A C array of pointers to MoeNode structures (the caller keeps them alive)."""
    arr = (ctypes.POINTER(MoeNode) * len(nodes))()
    for i, nd in enumerate(nodes):
        arr[i] = ctypes.pointer(nd)
    return arr


def node_claimed(node: MoeNode) -> bool:
    return bool(load_library().moe_node_claimed(ctypes.byref(node)))


def split_parse(nodes) -> MoeSplit:
    """Parse the routed-expert split; raises MoeError (MOE_ERR_UNSUPPORTED with the reason)."""
    L = load_library()
    sp = MoeSplit()
    why = ctypes.create_string_buffer(256)
    st = L.moe_split_parse(node_list(nodes), len(nodes), ctypes.byref(sp), why, len(why))
    if st != MOE_OK:
        raise MoeError(st, f"moe_split_parse: {why.value.decode()}")
    return sp


def read_gguf_layer(path: str, layer: int) -> GgufLayer:
    """Shape and router keys of one MoE layer of a GGUF model (no device needed);
    raises MoeError (MOE_ERR_FORMAT for a file that cannot be read as one)."""
    L = load_library()
    info = GgufLayer()
    err = ctypes.create_string_buffer(512)
    st = L.moe_gguf_read_layer(os.fsencode(path), int(layer), ctypes.byref(info), err, len(err))
    if st != MOE_OK:
        raise MoeError(st, f"moe_gguf_read_layer: {err.value.decode(errors='replace')}")
    return info


def _ptr(t) -> int | None:
    """Device pointer of a torch tensor (or None)."""
    return None if t is None else int(t.data_ptr())


# ---- argument checks ---------------------------------------------------------------
# The C-ABI takes raw pointers and sizes: a tensor of the wrong dtype, shape or
# device would make the kernels read or write out of bounds.  Every wrapper
# below checks its tensors before the call and raises ValueError instead.
# The order (dtype, shape, contiguity, device) lets the CPU tests reach each
# refusal with host tensors.

NOALLOC_SCRATCH_BYTES = 64 << 20  # MOE_NOALLOC_SCRATCH_BYTES


def check_tensor(t, name: str, dtype: str, shape=None, device: bool = True):
    """t: a torch tensor of `dtype` ("float32", "int32", ...), `shape` (a
    tuple, None entries match anything), contiguous, on a GPU if `device`."""
    if t is None or not hasattr(t, "data_ptr"):
        raise ValueError(f"{name}: expected a torch tensor, got {type(t).__name__}")
    if str(t.dtype) != f"torch.{dtype}":
        raise ValueError(f"{name}: dtype {t.dtype}, expected torch.{dtype}")
    if shape is not None:
        if t.dim() != len(shape) or any(want is not None and got != want for got, want in zip(t.shape, shape)):
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: not contiguous")
    if device and t.device.type != "cuda":
        raise ValueError(f"{name}: on {t.device}, expected a ROCm device tensor")


def check_forward_args(desc, x, ids, wts, out, flags: int = 0):
    """moe_forward's tensors: x float32 [T, H]; ids int32 / wts float32
    [T, k]; out float32 [T, H], or [T, k, H] with MOE_FWD_PER_SLOT.  desc:
    the layer's LayerDesc (None: the layer is unknown here, the library
    answers MOE_ERR_NOT_RESIDENT; only dtypes and layout are checked)."""
    H = desc.hidden if desc is not None else None
    k = desc.n_used if desc is not None else None
    check_tensor(x, "x", "float32", (None, H), device=False)
    T = int(x.shape[0])
    if T <= 0:
        raise ValueError("x: no tokens")
    check_tensor(ids, "ids", "int32", (T, k), device=False)
    check_tensor(wts, "wts", "float32", (T, k), device=False)
    check_tensor(out, "out", "float32", (T, k, H) if flags & MOE_FWD_PER_SLOT else (T, H), device=False)
    for t, nm in ((x, "x"), (ids, "ids"), (wts, "wts"), (out, "out")):
        if t.device.type != "cuda":
            raise ValueError(f"{nm}: on {t.device}, expected a ROCm device tensor")
    return T


def check_host_forward_args(desc, x, ids, wts):
    """moe_forward_host's numpy arrays: x [T, H], ids / wts [T, k]."""
    if x.ndim != 2 or x.shape[1] != desc.hidden or x.shape[0] <= 0:
        raise ValueError(f"x: shape {x.shape}, expected (T, {desc.hidden})")
    T = x.shape[0]
    for a, nm in ((ids, "ids"), (wts, "wts")):
        if a.shape != (T, desc.n_used):
            raise ValueError(f"{nm}: shape {a.shape}, expected ({T}, {desc.n_used})")
    return T


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return int(torch.cuda.current_stream().cuda_stream)
    return int(stream)


class Graph:
    def __init__(self, ctx: "MoeBlock", handle: int, keep):
        self._ctx, self._h, self._keep = ctx, handle, keep

    def launch(self, stream=None):
        self._ctx._check(self._ctx.lib.moe_graph_launch(self._h, _stream(stream)), "moe_graph_launch")

    def close(self):
        if self._h:
            self._ctx.lib.moe_graph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeBlock:
    """One device context: resident layers plus per-call scratch."""

    def __init__(self, device: int = 0, budget_bytes: int = 2 ** 64 - 1, lib_path: str | None = None):
        self.lib = load_library(lib_path)
        h = _vp()
        st = self.lib.moe_ctx_create(device, budget_bytes, ctypes.byref(h))
        if st != MOE_OK:
            raise MoeError(st, f"moe_ctx_create: {self.lib.moe_status_str(st).decode()}")
        self.h = h.value
        self.descs: dict[int, LayerDesc] = {}

    # -- lifecycle --------------------------------------------------------
    def close(self):
        if getattr(self, "h", None):
            self.lib.moe_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int, what: str):
        if st != MOE_OK:
            msg = self.lib.moe_ctx_last_error(self.h).decode() if self.h else ""
            raise MoeError(st, f"{what}: {self.lib.moe_status_str(st).decode()}: {msg}")

    @property
    def budget_left(self) -> int:
        return int(self.lib.moe_ctx_budget_left(self.h))

    def reserve(self, shape, max_tokens: int):
        d = LayerDesc.of(shape)
        self._check(self.lib.moe_ctx_reserve(self.h, ctypes.byref(d), max_tokens), "moe_ctx_reserve")

    # -- residency ----------------------------------------------------------
    def upload_layer(self, layer: int, shape, gate: np.ndarray, up: np.ndarray, down: np.ndarray,
                     shared=None):
        d = LayerDesc.of(shape)
        arrs = [np.ascontiguousarray(a, np.uint8) for a in (gate, up, down)]
        sh = [np.ascontiguousarray(a, np.uint8) for a in shared] if shared is not None else [None] * 3
        ptrs = [a.ctypes.data if a is not None else None for a in arrs + sh]
        self._check(self.lib.moe_layer_upload(self.h, layer, ctypes.byref(d), *ptrs), "moe_layer_upload")
        self.descs[layer] = d

    def upload_layer_gguf(self, layer: int, path: str, file_layer: int) -> GgufLayer:
        """Make layer `file_layer` of a GGUF model resident as `layer`."""
        info = GgufLayer()
        self._check(self.lib.moe_layer_upload_gguf(self.h, int(layer), os.fsencode(path), int(file_layer),
                                                   ctypes.byref(info)), "moe_layer_upload_gguf")
        self.descs[layer] = info.desc
        return info

    def generate_layer(self, layer: int, shape, seed: int, e_lo: int = 124, e_span: int = 7):
        d = LayerDesc.of(shape)
        self._check(self.lib.moe_layer_generate(self.h, layer, ctypes.byref(d), seed, e_lo, e_span),
                    "moe_layer_generate")
        self.descs[layer] = d

    def read_blocks(self, layer: int, tensor: int, expert: int) -> np.ndarray:
        d = self.descs[layer]
        rows, K = (d.ffn, d.hidden) if tensor in (T_GATE, T_UP) else (d.hidden, d.ffn)
        out = np.empty((rows, K // 32, 17), np.uint8)
        self._check(self.lib.moe_layer_read_blocks(self.h, layer, tensor, expert, out.ctypes.data),
                    "moe_layer_read_blocks")
        return out

    def release_layer(self, layer: int):
        self._check(self.lib.moe_layer_release(self.h, layer), "moe_layer_release")
        self.descs.pop(layer, None)

    def layer_bytes(self, layer: int) -> int:
        v = ctypes.c_uint64()
        self._check(self.lib.moe_layer_bytes(self.h, layer, ctypes.byref(v)), "moe_layer_bytes")
        return int(v.value)

    # -- per call (torch device tensors) ---------------------------------------
    def route(self, logits, k: int, mode: int, norm: bool, scale: float, ids, wts, bias=None, stream=None):
        check_tensor(logits, "logits", "float32", (None, None))
        T, E = logits.shape
        check_tensor(ids, "ids", "int32", (T, k))
        check_tensor(wts, "wts", "float32", (T, k))
        if bias is not None:
            check_tensor(bias, "bias", "float32", (E,))
        self._check(self.lib.moe_route(self.h, _ptr(logits), _ptr(bias), T, E, k, mode, int(norm), scale,
                                       _ptr(ids), _ptr(wts), _stream(stream)), "moe_route")

    def router_logits(self, w, x, logits, w_type: int = 0, stream=None):
        """logits [T][E] = x [T][H] . w [E][H]^T (f32 device tensors); w_type:
        the ggml type w was widened from (GGML_F32 / GGML_F16 / GGML_BF16: x
        is rounded to it first, as ggml-cpu's mul_mat does)."""
        check_tensor(x, "x", "float32", (None, None))
        T, H = x.shape
        check_tensor(w, "w", "float32", (None, H))
        E = w.shape[0]
        check_tensor(logits, "logits", "float32", (T, E))
        self._check(self.lib.moe_router_logits(self.h, _ptr(w), _ptr(x), T, E, H, w_type, _ptr(logits),
                                               _stream(stream)),
                    "moe_router_logits")

    def group(self, ids, E: int, counts, offsets, perm, inv=None, stream=None):
        check_tensor(ids, "ids", "int32", (None, None))
        T, k = ids.shape
        check_tensor(counts, "counts", "int32", (E,))
        check_tensor(offsets, "offsets", "int32", (E + 1,))
        check_tensor(perm, "perm", "int32", (T * k,))
        if inv is not None:
            check_tensor(inv, "inv", "int32", (T * k,))
        self._check(self.lib.moe_group(self.h, _ptr(ids), T, k, E, _ptr(counts), _ptr(offsets), _ptr(perm),
                                       _ptr(inv), _stream(stream)), "moe_group")

    def forward(self, layer: int, x, ids, wts, out, flags: int = 0, stream=None):
        T = check_forward_args(self.descs.get(layer), x, ids, wts, out, flags)
        self._check(self.lib.moe_forward(self.h, layer, _ptr(x), _ptr(ids), _ptr(wts), T, _ptr(out), flags,
                                         _stream(stream)), "moe_forward")

    def forward_noalloc(self, layer: int, x, ids, wts, out, flags: int = 0, stream=None):
        """moe_forward_noalloc: the same block with the per-call buffers in the
        library's file-scope device scratch (no allocation)."""
        T = check_forward_args(self.descs.get(layer), x, ids, wts, out, flags)
        self._check(self.lib.moe_forward_noalloc(self.h, layer, _ptr(x), _ptr(ids), _ptr(wts), T, _ptr(out), flags,
                                                 _stream(stream)), "moe_forward_noalloc")

    def route_forward(self, layer: int, x, logits, ids, wts, out, mode: int, norm: bool = True,
                      scale: float = 1.0, bias=None, flags: int = 0, stream=None):
        d = self.descs.get(layer)
        T = check_forward_args(d, x, ids, wts, out, flags)
        check_tensor(logits, "logits", "float32", (T, d.n_expert if d is not None else None))
        if bias is not None:
            check_tensor(bias, "bias", "float32", (logits.shape[1],))
        self._check(self.lib.moe_route_forward(self.h, layer, _ptr(x), _ptr(logits), _ptr(bias), T, mode,
                                               int(norm), scale, _ptr(ids), _ptr(wts), _ptr(out), flags,
                                               _stream(stream)), "moe_route_forward")

    def split_compute(self, nodes):
        """Compute a parsed split (moe_split_compute) into its MUL node's host data."""
        self._check(self.lib.moe_split_compute(self.h, node_list(nodes), len(nodes)), "moe_split_compute")

    def forward_host(self, layer: int, x: np.ndarray, ids: np.ndarray, wts: np.ndarray,
                     flags: int = 0) -> np.ndarray:
        d = self.descs[layer]
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        wts = np.ascontiguousarray(wts, np.float32)
        T = check_host_forward_args(d, x, ids, wts)
        shape = (T, d.n_used, d.hidden) if flags & MOE_FWD_PER_SLOT else (T, d.hidden)
        out = np.empty(shape, np.float32)
        self._check(self.lib.moe_forward_host(self.h, layer, x.ctypes.data, ids.ctypes.data, wts.ctypes.data,
                                              T, out.ctypes.data, flags), "moe_forward_host")
        return out

    def graph_capture(self, layers, xs, ids, wts, outs, flags: int = 0) -> Graph:
        n = len(layers)
        if n == 0 or not (len(xs) == len(ids) == len(wts) == len(outs) == n):
            raise ValueError("graph_capture: one x/ids/wts/out per layer")
        T = xs[0].shape[0]
        for i in range(n):
            if check_forward_args(self.descs.get(layers[i]), xs[i], ids[i], wts[i], outs[i], flags) != T:
                raise ValueError(f"graph_capture: layer {i} has {xs[i].shape[0]} tokens, expected {T}")
        la = (ctypes.c_int * n)(*layers)
        mk = lambda ts: (_vp * n)(*[_ptr(t) for t in ts])  # noqa: E731
        px, pi, pw, po = mk(xs), mk(ids), mk(wts), mk(outs)
        g = _vp()
        self._check(self.lib.moe_graph_capture(self.h, n, la, px, pi, pw, po, T, flags, ctypes.byref(g)),
                    "moe_graph_capture")
        return Graph(self, g.value, (xs, ids, wts, outs))

    # -- profiling ----------------------------------------------------------------
    def prof_enable(self, on: bool = True):
        self._check(self.lib.moe_prof_enable(self.h, int(on)), "moe_prof_enable")

    def prof_read(self, reset: bool = True) -> dict:
        """{kernel class: (launches, total_us)} since the last reset."""
        cap = 16
        arr = (KernelStat * cap)()
        n = ctypes.c_int()
        self._check(self.lib.moe_prof_read(self.h, arr, cap, ctypes.byref(n), int(reset)), "moe_prof_read")
        return {arr[i].name.decode(): (int(arr[i].launches), float(arr[i].total_us)) for i in range(min(n.value, cap))}

    def call_stats(self, reset: bool = False) -> dict:
        """Engagement and phase counters of the host-boundary calls (moe_call_stats_read)."""
        cs = CallStats()
        self._check(self.lib.moe_call_stats_read(self.h, ctypes.byref(cs), int(reset)), "moe_call_stats_read")
        return {n: getattr(cs, n) for n, _ in CallStats._fields_}

    # -- test hooks -------------------------------------------------------------
    def set_taps(self, on: bool = True):
        self._check(self.lib.moe_debug_set_taps(self.h, int(on)), "moe_debug_set_taps")
    def debug_quantize_q8_0(self, x, qs, d, stream=None):
        check_tensor(x, "x", "float32")
        n = x.numel()
        check_tensor(qs, "qs", "int8", (n,) if qs.dim() == 1 else tuple(x.shape))
        if d.numel() != n // 32 or d.element_size() != 2:
            raise ValueError("d: expected n/32 16-bit scales")
        check_tensor(d, "d", str(d.dtype).replace("torch.", ""))
        self._check(self.lib.moe_debug_quantize_q8_0(self.h, _ptr(x), x.numel(), _ptr(qs), _ptr(d),
                                                     _stream(stream)), "moe_debug_quantize_q8_0")

    def debug_wave_sum(self, x, out, stream=None):
        check_tensor(x, "x", "float32")
        if x.numel() % 64 or out.numel() < x.numel() // 64:
            raise ValueError("debug_wave_sum: x of 64*n floats, out of n")
        check_tensor(out, "out", "float32")
        self._check(self.lib.moe_debug_wave_sum(self.h, _ptr(x), x.numel() // 64, _ptr(out), _stream(stream)),
                    "moe_debug_wave_sum")

    def debug_last_h(self, cap: int) -> np.ndarray:
        buf = np.empty(cap, np.float32)
        n = ctypes.c_size_t()
        self._check(self.lib.moe_debug_last_h(self.h, buf.ctypes.data, cap, ctypes.byref(n)), "moe_debug_last_h")
        return buf[: n.value]

    def set_timeline(self, on: bool = True):
        self._check(self.lib.moe_debug_set_timeline(self.h, int(on)), "moe_debug_set_timeline")

    def read_timeline(self):
        """The last eager decode call's per-wave stamps (100 MHz clock ticks):
        (gate_up [n, 3], down [n, 3]) uint64, columns entry / K-loop end / exit."""
        buf = np.empty(3 * 8192, np.uint64)
        ng, nd = ctypes.c_size_t(), ctypes.c_size_t()
        self._check(self.lib.moe_debug_read_timeline(self.h, buf.ctypes.data, buf.size, ctypes.byref(ng),
                                                     ctypes.byref(nd)), "moe_debug_read_timeline")
        st = buf[: 3 * (ng.value + nd.value)].reshape(-1, 3)
        return st[: ng.value].copy(), st[ng.value:].copy()


class MoeServer:
    """nano-glm moe-server protocol v2 served from the MoE block
    (moe_server_open / handle / listen / serve)."""

    def __init__(self, gguf_path: str, device: int = 0, budget_bytes: int = 2 ** 64 - 1,
                 lib_path: str | None = None):
        self.lib = load_library(lib_path)
        h = _vp()
        err = ctypes.create_string_buffer(512)
        st = self.lib.moe_server_open(os.fsencode(gguf_path), device, budget_bytes, ctypes.byref(h), err, len(err))
        if st != MOE_OK:
            raise MoeError(st, f"moe_server_open: {self.lib.moe_status_str(st).decode()}: "
                               f"{err.value.decode(errors='replace')}")
        self.h = h.value

    def close(self):
        if getattr(self, "h", None):
            self.lib.moe_server_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int, what: str):
        if st != MOE_OK:
            msg = self.lib.moe_server_last_error(self.h).decode() if self.h else ""
            raise MoeError(st, f"{what}: {self.lib.moe_status_str(st).decode()}: {msg}")

    def handle(self, msg: bytes) -> bytes:
        """One whole message in, the whole response out."""
        n = ctypes.c_size_t()
        cap = 1 << 16
        while True:
            buf = ctypes.create_string_buffer(cap)
            st = self.lib.moe_server_handle(self.h, msg, len(msg), buf, cap, ctypes.byref(n))
            if st == MOE_OK:
                return buf.raw[: n.value]
            if st == MOE_ERR_INVALID_ARG and n.value > cap:
                cap = n.value
                continue
            self._check(st, "moe_server_handle")

    def listen(self, host: str = "127.0.0.1", port: int = 0) -> int:
        """Bind; returns the port (port 0 = any free one)."""
        bound = ctypes.c_int()
        self._check(self.lib.moe_server_listen(self.h, host.encode(), port, ctypes.byref(bound)), "moe_server_listen")
        return bound.value

    def serve(self, max_connections: int = -1):
        """Serve connections one at a time (blocks; ctypes releases the GIL)."""
        self._check(self.lib.moe_server_serve(self.h, max_connections), "moe_server_serve")
