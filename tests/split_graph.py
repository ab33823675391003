"""The routed-expert block of one MoE layer as a graph of moe_node structures,
in the op order of llama.cpp's build_moe_ffn that nano-glm restates
(nano-glm/lib/models/glm_dsa/moe_block.h:104-133; deepseek4 adds the
SwiGLU clamps, deepseek4/moe_block.h:180-199):

    up    = mul_mat_id(ffn_up_exps,   x, ids)        x [H, 1, T], ids [k, T]
    gate  = mul_mat_id(ffn_gate_exps, x, ids)
    (gate = clamp(gate, -inf, L); up = clamp(up, -L, L))
    act   = glu(gate, up)  SwiGLU
    y     = mul_mat_id(ffn_down_exps, act, ids)      [H, k, T]
    y     = mul(y, weights)                          weights [1, k, T]
    out   = view(y, slot 0) + view(y, slot 1) + ...  (the trunk's ADD chain)
"""
import ctypes

import numpy as np

import moe_block as mb


class Graph:
    def __init__(self):
        self.keep = []
        self.nodes = []

    def node(self, op, ne=(1, 1, 1, 1), type_=mb.GGML_F32, src=(), data=None, name=None, ours=False,
             view_src=None, **kw):
        n = mb.MoeNode()
        n.op, n.type = op, type_
        ne = list(ne) + [1] * (4 - len(ne))
        for i in range(4):
            n.ne[i] = ne[i]
        n.contiguous = kw.get("contiguous", 1)
        n.in_moe_buffer = 1 if ours else 0
        n.glu_op = kw.get("glu_op", 0)
        n.glu_swapped = kw.get("glu_swapped", 0)
        n.clamp_min = kw.get("clamp_min", 0.0)
        n.clamp_max = kw.get("clamp_max", 0.0)
        for i, s in enumerate(src):
            n.src[i] = ctypes.pointer(s) if s is not None else None
        if view_src is not None:
            n.view_src = ctypes.pointer(view_src)
        if data is not None:
            self.keep.append(data)
            n.data = data.ctypes.data
        if name is not None:
            b = name.encode()
            self.keep.append(b)
            n.name = b
        self.keep.append(n)
        return n

    def add(self, n):
        self.nodes.append(n)
        return n


def block(H, F, E, k, T, layer, clamp=None, x=None, ids=None, wts=None, out=None, ours=True,
          weight_type=mb.GGML_MXFP4):
    """Returns (graph, named nodes).  x [T, H] f32, ids [T, k] i32, wts [T, k] f32,
    out [T, k, H] f32 (the MUL node's data); zeros when not given."""
    g = Graph()
    x = np.zeros((T, H), np.float32) if x is None else np.ascontiguousarray(x, np.float32)
    ids = np.zeros((T, k), np.int32) if ids is None else np.ascontiguousarray(ids, np.int32)
    wts = np.zeros((T, k), np.float32) if wts is None else np.ascontiguousarray(wts, np.float32)
    out = np.zeros((T, k, H), np.float32) if out is None else out
    b = f"blk.{layer}."
    w_gate = g.node(mb.NODE_NONE, (H, F, E), weight_type, name=b + "ffn_gate_exps.weight", ours=ours)
    w_up = g.node(mb.NODE_NONE, (H, F, E), weight_type, name=b + "ffn_up_exps.weight", ours=ours)
    w_down = g.node(mb.NODE_NONE, (F, H, E), weight_type, name=b + "ffn_down_exps.weight", ours=ours)
    xin = g.node(mb.NODE_NONE, (H, T), data=x, name="ffn_moe_input")
    xr = g.node(mb.NODE_RESHAPE, (H, 1, T), src=(xin,), data=x, view_src=xin)
    idn = g.node(mb.NODE_NONE, (k, T), mb.GGML_I32, data=ids, name="ffn_moe_topk")
    wn = g.node(mb.NODE_NONE, (1, k, T), data=wts, name="ffn_moe_weights")
    up = g.add(g.node(mb.NODE_MUL_MAT_ID, (F, k, T), src=(w_up, xr, idn)))
    gate = g.add(g.node(mb.NODE_MUL_MAT_ID, (F, k, T), src=(w_gate, xr, idn)))
    if clamp is not None:
        gate = g.add(g.node(mb.NODE_CLAMP, (F, k, T), src=(gate,), clamp_min=-np.inf, clamp_max=clamp))
        up = g.add(g.node(mb.NODE_CLAMP, (F, k, T), src=(up,), clamp_min=-clamp, clamp_max=clamp))
    act = g.add(g.node(mb.NODE_GLU, (F, k, T), src=(gate, up), glu_op=mb.GLU_SWIGLU))
    y = g.add(g.node(mb.NODE_MUL_MAT_ID, (H, k, T), src=(w_down, act, idn)))
    mul = g.add(g.node(mb.NODE_MUL, (H, k, T), src=(y, wn), data=out))
    views = [g.add(g.node(mb.NODE_VIEW, (H, T), src=(mul,), view_src=mul)) for _ in range(k)]
    s = views[0]
    adds = []
    for v in views[1:]:
        s = g.add(g.node(mb.NODE_ADD, (H, T), src=(s, v)))
        adds.append(s)
    named = dict(w_gate=w_gate, w_up=w_up, w_down=w_down, x=xr, ids=idn, wts=wn, up=up, gate=gate, act=act, y=y,
                 mul=mul, views=views, adds=adds, out=out)
    return g, named


def split_nodes(g, named):
    """The nodes the backend receives: the claimed run of the block (no ADDs)."""
    return [n for n in g.nodes if n.op != mb.NODE_ADD]
