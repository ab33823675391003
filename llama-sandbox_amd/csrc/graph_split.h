// The ggml backend's claim set and split, over moe_node (host code, included
// by moe_block.hip after the C-ABI it calls).
//
// moe-serv's backend claims the routed-expert block of each MoE layer from
// llama.cpp's scheduler (moe-serv/src/moe_backend.cpp:262-345), receives it
// as one split, recognises its tensors (moe-serv/src/moe_tp.h:301-354) and
// computes it, falling back to the CPU backend on any failure
// (moe_backend.cpp:413-484).  The same three steps here work on moe_node, a
// plain description of a graph node that an adapter with ggml's headers
// fills from ggml_tensor; the computation is moe_forward_host.
#pragma once

#include <cmath>
#include <cstdlib>

static bool node_is_ours(const moe_node *t) {
  if (!t) return false;
  const moe_node *s = t->view_src ? t->view_src : t;
  return s->in_moe_buffer != 0;
}

// Does t descend, within `depth` links, from a MUL_MAT_ID over weights in
// the MoE buffer?  Depth 4 spans mul_mat_id -> clamp -> glu -> mul_mat_id ->
// mul, the longest chain of the block.
static bool node_derives_from_ours(const moe_node *t, int depth) {
  if (!t || depth <= 0) return false;
  if (t->op == MOE_NODE_MUL_MAT_ID && node_is_ours(t->src[0])) return true;
  for (int i = 0; i < 3; i++)
    if (node_derives_from_ours(t->src[i], depth - 1)) return true;
  return false;
}

extern "C" int moe_node_claimed(const moe_node *op) {
  if (!op) return 0;
  static const bool disabled = getenv("MOESERV_DISABLE") != nullptr;
  if (disabled) return 0;
  switch (op->op) {
    case MOE_NODE_NONE:
    case MOE_NODE_RESHAPE:
    case MOE_NODE_VIEW:
    case MOE_NODE_PERMUTE:
    case MOE_NODE_TRANSPOSE:
      return 1;
    case MOE_NODE_MUL_MAT_ID:
      return node_is_ours(op->src[0]) ? 1 : 0;
    case MOE_NODE_CLAMP:
    case MOE_NODE_MUL:
      return node_derives_from_ours(op, 4) ? 1 : 0;
    case MOE_NODE_GLU:
      return op->glu_op == MOE_GLU_SWIGLU && node_derives_from_ours(op, 4) ? 1 : 0;
    default:
      return 0;  // ADD included: it is also the residual add of the trunk
  }
}

static moe_status split_why(char *why, size_t len, const char *m) {
  if (why && len) snprintf(why, len, "%s", m);
  return MOE_ERR_UNSUPPORTED;
}

extern "C" moe_status moe_split_parse(const moe_node *const *nodes, int n, moe_split *c, char *why,
                                      size_t why_len) {
  if (why && why_len) why[0] = 0;
  if (!nodes || n <= 0 || !c) return MOE_ERR_INVALID_ARG;
  memset(c, 0, sizeof(*c));
  const moe_node *glu = nullptr, *mul = nullptr;
  for (int i = 0; i < n; i++) {
    const moe_node *t = nodes[i];
    if (!t) return MOE_ERR_INVALID_ARG;
    if (t->op == MOE_NODE_GLU) glu = t;
    if (t->op == MOE_NODE_MUL) mul = t;
  }
  if (!glu || !mul) return split_why(why, why_len, "the split has no SwiGLU node or no router-weight multiply");
  if (glu->glu_op != MOE_GLU_SWIGLU || glu->glu_swapped != 0) return split_why(why, why_len, "the activation is not an unswapped SwiGLU");
  // gate and up: a MUL_MAT_ID, each optionally behind a CLAMP
  const moe_node *gc = glu->src[0], *uc = glu->src[1];
  if (!gc || !uc) return split_why(why, why_len, "the SwiGLU node lacks a gate or an up input");
  c->gate_min = c->up_min = -INFINITY;
  c->gate_max = c->up_max = INFINITY;
  const moe_node *gmm = gc, *umm = uc;
  if (gc->op == MOE_NODE_CLAMP) {
    c->gate_min = gc->clamp_min;
    c->gate_max = gc->clamp_max;
    gmm = gc->src[0];
  }
  if (uc->op == MOE_NODE_CLAMP) {
    c->up_min = uc->clamp_min;
    c->up_max = uc->clamp_max;
    umm = uc->src[0];
  }
  if (!gmm || !umm || gmm->op != MOE_NODE_MUL_MAT_ID || umm->op != MOE_NODE_MUL_MAT_ID)
    return split_why(why, why_len, "gate or up is not an expert matmul (optionally clamped)");
  const moe_node *dmm = mul->src[0];
  if (!dmm || dmm->op != MOE_NODE_MUL_MAT_ID) return split_why(why, why_len, "the router-weight multiply does not take the down expert matmul");
  if (dmm->src[1] != glu) return split_why(why, why_len, "the down expert matmul does not read the SwiGLU output");
  c->gate_w = gmm->src[0];
  c->up_w = umm->src[0];
  c->down_w = dmm->src[0];
  c->x = gmm->src[1];
  c->ids = gmm->src[2];
  c->wts = mul->src[1];
  c->out = mul;
  if (!c->gate_w || !c->up_w || !c->down_w || !c->x || !c->ids || !c->wts)
    return split_why(why, why_len, "an expert matmul or the multiply lacks an operand");
  if (umm->src[1] != c->x || umm->src[2] != c->ids || dmm->src[2] != c->ids)
    return split_why(why, why_len, "gate, up and down do not read the same activations and expert ids");
  if (!c->x->data || !c->ids->data || !c->wts->data || !c->out->data) return split_why(why, why_len, "an input or the output has no host memory behind it");
  if (c->x->type != MOE_GGML_F32 || c->ids->type != MOE_GGML_I32 || c->wts->type != MOE_GGML_F32 ||
      c->out->type != MOE_GGML_F32)
    return split_why(why, why_len, "the activations, router weights or output are not f32, or the ids not i32");
  if (c->gate_w->type != MOE_GGML_MXFP4 || c->up_w->type != MOE_GGML_MXFP4 || c->down_w->type != MOE_GGML_MXFP4)
    return split_why(why, why_len, "an expert weight tensor is not MXFP4");
  if (!c->out->contiguous || !c->x->contiguous || !c->ids->contiguous || !c->wts->contiguous)
    return split_why(why, why_len, "an input or the output is not contiguous");
  // shapes: gate/up [H, F, E], down [F, H, E], x [H, 1, T], ids [k, T], wts [1, k, T], out [H, k, T]
  const int64_t H = c->gate_w->ne[0], F = c->gate_w->ne[1], E = c->gate_w->ne[2];
  const int64_t k = c->ids->ne[0], T = c->ids->ne[1];
  if (c->up_w->ne[0] != H || c->up_w->ne[1] != F || c->up_w->ne[2] != E || c->down_w->ne[0] != F ||
      c->down_w->ne[1] != H || c->down_w->ne[2] != E)
    return split_why(why, why_len, "the gate, up and down weight shapes do not agree");
  if (c->x->ne[0] != H || c->x->ne[1] != 1 || c->x->ne[2] != T || c->wts->ne[0] != 1 || c->wts->ne[1] != k ||
      c->wts->ne[2] != T || c->out->ne[0] != H || c->out->ne[1] != k || c->out->ne[2] != T)
    return split_why(why, why_len, "the activation, router-weight or output shapes do not match the weights");
  if (H <= 0 || F <= 0 || E <= 0 || k <= 0 || T <= 0 || H > INT32_MAX || F > INT32_MAX || E > INT32_MAX ||
      k > E || T > INT32_MAX)
    return split_why(why, why_len, "a dimension is empty, or the top-k exceeds the expert count");
  const char *name = c->gate_w->name;
  if (!name || strncmp(name, "blk.", 4) != 0 || name[4] < '0' || name[4] > '9')
    return split_why(why, why_len, "the gate weight name does not start with blk.<layer>.");
  c->layer = atoi(name + 4);
  c->n_slots = (int32_t)k;
  c->n_tokens = (int32_t)T;
  c->hidden = (int32_t)H;
  c->ffn = (int32_t)F;
  c->n_expert = (int32_t)E;
  return MOE_OK;
}

static moe_status split_compute_impl(moe_ctx *c, const moe_node *const *nodes, int n);

// A split the parse or the checks refuse counts as a refusal (the caller runs
// it on the CPU); one computed on the device is counted by moe_forward_host.
extern "C" moe_status moe_split_compute(moe_ctx *c, const moe_node *const *nodes, int n) {
  if (!c) return MOE_ERR_INVALID_ARG;
  const uint64_t before = c->calls.refusals;
  const moe_status st = split_compute_impl(c, nodes, n);
  if (st != MOE_OK && c->calls.refusals == before) c->calls.refusals++;
  return st;
}

static moe_status split_compute_impl(moe_ctx *c, const moe_node *const *nodes, int n) {
  moe_split sp;
  char why[128];
  const moe_status st = moe_split_parse(nodes, n, &sp, why, sizeof why);
  if (st != MOE_OK) return fail(c, st, "split: %s; CPU fallback", why[0] ? why : "bad arguments");
  auto it = c->layers.find(sp.layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident; CPU fallback", sp.layer);
  const moe_layer_desc &d = it->second.d;
  if (d.hidden != sp.hidden || d.ffn != sp.ffn || d.n_expert != sp.n_expert || d.n_used != sp.n_slots)
    return fail(c, MOE_ERR_UNSUPPORTED, "split: shape differs from resident layer %d; CPU fallback", sp.layer);
  // the kernels clamp gate <= L and up to [-L, L] with the layer's L, or not at all
  const float L = d.clamp > 1e-6f ? d.clamp : INFINITY;
  const bool clamp_ok = sp.gate_min == -INFINITY && sp.gate_max == L && sp.up_min == -L && sp.up_max == L;
  if (!clamp_ok)
    return fail(c, MOE_ERR_UNSUPPORTED, "split: clamps [%g, %g] / [%g, %g] are not the layer's (L = %g); CPU fallback",
                sp.gate_min, sp.gate_max, sp.up_min, sp.up_max, L);
  return moe_forward_host(c, sp.layer, static_cast<const float *>(sp.x->data),
                          static_cast<const int32_t *>(sp.ids->data), static_cast<const float *>(sp.wts->data),
                          sp.n_tokens, static_cast<float *>(sp.out->data), MOE_FWD_PER_SLOT);
}
