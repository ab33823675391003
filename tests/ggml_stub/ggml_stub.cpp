// TEST-ONLY: the few ggml functions the MoE backend adapter calls, for a
// host process (drive_backend.cpp) that loads the adapter the way llama.cpp
// does.  The CPU delegate is a fake: its graph_compute counts the call and
// fills the split's MUL node with a sentinel, so a test can tell which path
// produced a result; its set_n_threads records the count it was given.
#include "ggml_stub.h"

#include <cstdlib>
#include <cstring>

extern "C" {

const char *ggml_get_name(const ggml_tensor *t) { return t->name; }

size_t ggml_nbytes(const ggml_tensor *t) {
  int64_t n = 1;
  for (int i = 1; i < GGML_MAX_DIMS; i++) n *= t->ne[i];
  switch (t->type) {
    case GGML_TYPE_MXFP4: return (size_t)(t->ne[0] / 32 * 17 * n);
    case GGML_TYPE_F16:
    case GGML_TYPE_BF16: return (size_t)(t->ne[0] * 2 * n);
    default: return (size_t)(t->ne[0] * 4 * n);
  }
}

bool ggml_is_contiguous(const ggml_tensor *t) { return (t->flags & STUB_NOT_CONTIGUOUS) == 0; }

enum ggml_glu_op ggml_get_glu_op(const ggml_tensor *t) { return (enum ggml_glu_op)t->op_params[0]; }

const char *ggml_op_name(enum ggml_op op) {
  static const char *names[GGML_OP_COUNT] = {"NONE", "ADD", "MUL", "MUL_MAT", "MUL_MAT_ID", "RESHAPE",
                                             "VIEW", "PERMUTE", "TRANSPOSE", "CLAMP", "GLU", "SOFT_MAX"};
  return (int)op >= 0 && op < GGML_OP_COUNT ? names[op] : "?";
}

struct ggml_cgraph {
  int n_nodes;
  ggml_tensor **nodes;
};

int ggml_graph_n_nodes(ggml_cgraph *g) { return g->n_nodes; }
ggml_tensor *ggml_graph_node(ggml_cgraph *g, int i) { return g->nodes[i]; }

ggml_cgraph *stub_graph(ggml_tensor **nodes, int n) {
  auto *g = new ggml_cgraph;
  g->n_nodes = n;
  g->nodes = nodes;
  return g;
}

void stub_graph_free(ggml_cgraph *g) { delete g; }

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void *context, size_t size) {
  return new ggml_backend_buffer{iface, buft, context, size, GGML_BACKEND_BUFFER_USAGE_ANY};
}

bool ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer) {
  return buffer && buffer->buft && buffer->buft->iface.is_host && buffer->buft->iface.is_host(buffer->buft);
}

// ---- the fake CPU delegate ---------------------------------------------------

int stub_cpu_calls = 0;
int stub_cpu_threads = -1;

static void cpu_set_n_threads(ggml_backend_t backend, int n) {
  (void)backend;
  stub_cpu_threads = n;
}

static void *cpu_proc(ggml_backend_reg_t reg, const char *name) {
  (void)reg;
  return strcmp(name, "ggml_backend_set_n_threads") == 0 ? (void *)cpu_set_n_threads : nullptr;
}

static enum ggml_status cpu_compute(ggml_backend_t backend, ggml_cgraph *g) {
  (void)backend;
  stub_cpu_calls++;
  for (int i = 0; i < g->n_nodes; i++) {
    ggml_tensor *t = g->nodes[i];
    if (t->op == GGML_OP_MUL && t->data) {
      float *o = (float *)t->data;
      for (size_t j = 0; j < ggml_nbytes(t) / 4; j++) o[j] = STUB_CPU_SENTINEL;
    }
  }
  return GGML_STATUS_SUCCESS;
}

static ggml_backend_reg cpu_reg = {GGML_BACKEND_API_VERSION, {nullptr, nullptr, nullptr, cpu_proc}, nullptr};
static ggml_backend_device cpu_dev = {{}, &cpu_reg, nullptr};
static ggml_backend cpu_backend_obj;

ggml_backend_t ggml_backend_init_by_type(enum ggml_backend_dev_type type, const char *params) {
  (void)params;
  if (type != GGML_BACKEND_DEVICE_TYPE_CPU) return nullptr;
  cpu_backend_obj.iface.graph_compute = cpu_compute;
  cpu_backend_obj.device = &cpu_dev;
  return &cpu_backend_obj;
}

enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
  return backend->iface.graph_compute(backend, cgraph);
}

ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend) { return backend->device; }
ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t device) { return device->reg; }
void *ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char *name) {
  return reg->iface.get_proc_address ? reg->iface.get_proc_address(reg, name) : nullptr;
}

}  // extern "C"
