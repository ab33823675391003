"""The ggml backend's claim set and split recognition on CPU
(moe_node_claimed, moe_split_parse), on the block graph of
tests/split_graph.py: what moe-serv claims (moe-serv/src/moe_backend.cpp:
262-345) and what its split parser accepts or refuses
(moe-serv/src/moe_tp.h:301-354, with more than one token allowed)."""
import os
import subprocess
import sys

import numpy as np
import pytest

import moe_block as mb
import split_graph as sg

H, F, E, K, T = 256, 128, 8, 2, 3


def claimed(n):
    return mb.node_claimed(n)


@pytest.mark.parametrize("clamp", [None, 7.0])
def test_claim_set_of_the_block(clamp):
    g, nd = sg.block(H, F, E, K, T, 3, clamp=clamp)
    for n in g.nodes:
        want = n.op != mb.NODE_ADD  # the expert block minus the expert sum
        assert claimed(n) == want, n.op


def test_weights_not_ours_claims_nothing_of_the_block():
    g, nd = sg.block(H, F, E, K, T, 3, clamp=7.0, ours=False)
    for n in g.nodes:
        assert claimed(n) == (n.op == mb.NODE_VIEW), n.op


def test_claim_rules_for_other_nodes():
    g, nd = sg.block(H, F, E, K, T, 3)
    attn = g.node(mb.NODE_NONE, (H, T), name="attn_out")
    assert not claimed(g.node(mb.NODE_MUL, (H, T), src=(attn, attn)))  # a mul of the trunk
    assert not claimed(g.node(mb.NODE_CLAMP, (H, T), src=(attn,)))
    assert claimed(g.node(mb.NODE_PERMUTE, (H, T), src=(attn,)))       # structural ops are free
    assert claimed(g.node(mb.NODE_TRANSPOSE, (H, T), src=(attn,)))
    assert not claimed(g.node(mb.NODE_OTHER, (H, T), src=(nd["mul"],)))
    # GLU other than SwiGLU: refused even over our weights
    assert not claimed(g.node(mb.NODE_GLU, (F, K, T), src=(nd["gate"], nd["up"]), glu_op=1))
    # the derivation walk stops after 4 links
    n = nd["y"]
    depth = []
    for _ in range(5):
        n = g.node(mb.NODE_MUL, (H, K, T), src=(n,))
        depth.append(claimed(n))
    assert depth == [True, True, True, False, False]
    # a weight that is a view of our buffer is ours
    wv = g.node(mb.NODE_VIEW, (H, F, E), mb.GGML_MXFP4, view_src=nd["w_gate"])
    assert claimed(g.node(mb.NODE_MUL_MAT_ID, (F, K, T), src=(wv, nd["x"], nd["ids"])))


def test_moeserv_disable_claims_nothing():
    code = ("import sys; sys.path[:0] = %r; import split_graph as sg, moe_block as mb\n"
            "g, nd = sg.block(64, 32, 4, 2, 1, 0)\n"
            "print(sum(mb.node_claimed(n) for n in g.nodes))\n") % (sys.path[:6],)
    env = dict(os.environ, MOESERV_DISABLE="1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "0"


@pytest.mark.parametrize("clamp", [None, 7.0])
def test_parse_the_split(clamp):
    g, nd = sg.block(H, F, E, K, T, 17, clamp=clamp)
    sp = mb.split_parse(sg.split_nodes(g, nd))
    assert (sp.layer, sp.n_slots, sp.n_tokens, sp.hidden, sp.ffn, sp.n_expert) == (17, K, T, H, F, E)
    if clamp is None:
        assert sp.gate_min == -np.inf and sp.gate_max == np.inf and sp.up_min == -np.inf and sp.up_max == np.inf
    else:
        assert (sp.gate_min, sp.gate_max, sp.up_min, sp.up_max) == (-np.inf, 7.0, -7.0, 7.0)
    assert sp.out.contents.data == nd["mul"].data and sp.x.contents.data == nd["x"].data


def _refuse(nodes, reason):
    with pytest.raises(mb.MoeError) as ei:
        mb.split_parse(nodes)
    assert ei.value.status == mb.MOE_ERR_UNSUPPORTED and reason in str(ei.value), str(ei.value)


def test_parse_refusals():
    def fresh(**kw):
        g, nd = sg.block(H, F, E, K, T, 5, clamp=7.0, **kw)
        return g, nd, sg.split_nodes(g, nd)

    g, nd, nodes = fresh()
    _refuse([n for n in nodes if n.op != mb.NODE_GLU], "no SwiGLU node")
    g, nd, nodes = fresh()
    nd["act"].glu_swapped = 1
    _refuse(nodes, "not an unswapped SwiGLU")
    g, nd, nodes = fresh()
    nd["act"].glu_op = 0
    _refuse(nodes, "not an unswapped SwiGLU")
    g, nd, nodes = fresh()
    other = g.node(mb.NODE_NONE, (H, K, T))
    nd["mul"].src[0] = mb.ctypes.pointer(other)
    _refuse(nodes, "does not take the down expert matmul")
    g, nd, nodes = fresh()
    nd["y"].src[1] = mb.ctypes.pointer(nd["gate"])
    _refuse(nodes, "does not read the SwiGLU output")
    g, nd, nodes = fresh()
    x2 = g.node(mb.NODE_NONE, (H, 1, T), data=np.zeros((T, H), np.float32))
    up_mm = nd["up"].src[0].contents  # the up clamp's source: the up mul_mat_id
    up_mm.src[1] = mb.ctypes.pointer(x2)
    _refuse(nodes, "same activations and expert ids")
    g, nd, nodes = fresh(weight_type=8)
    _refuse(nodes, "not MXFP4")
    g, nd, nodes = fresh()
    nd["ids"].type = mb.GGML_F32
    _refuse(nodes, "not f32, or the ids not i32")
    g, nd, nodes = fresh()
    nd["mul"].contiguous = 0
    _refuse(nodes, "not contiguous")
    g, nd, nodes = fresh()
    nd["w_down"].ne[0] = F + 32
    _refuse(nodes, "weight shapes do not agree")
    g, nd, nodes = fresh()
    nd["mul"].ne[1] = K + 1
    _refuse(nodes, "shapes do not match the weights")
    g, nd, nodes = fresh()
    nd["w_gate"].name = b"ffn_gate_exps.weight"
    _refuse(nodes, "does not start with blk.")
    g, nd, nodes = fresh()
    nd["mul"].data = None
    _refuse(nodes, "no host memory behind it")
