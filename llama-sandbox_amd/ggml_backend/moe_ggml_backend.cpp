// moe_ggml_backend.cpp -- the loadable ggml backend ("MoE") that puts
// llama.cpp's routed-expert blocks on the gfx950 MoE block.
//
// The reference's moe-serv backend (moe-serv/src/moe_backend.cpp) is a
// library that llama.cpp dlopens through GGML_BACKEND_PATH.  It exposes a
// buffer type named "MoE" (the `-ot ...exps=MoE` target), claims the expert
// half of each MoE layer from the scheduler, receives that half as one split
// and computes it, falling back to the CPU backend on anything it cannot do.
// This file is the same shell around this repository's C-ABI
// (include/moe_block.h): the claim set is moe_node_claimed, the split is
// moe_split_parse / moe_split_compute, residency is moe_layer_upload from
// the weights' host buffer.  ggml's own types are used unchanged; the only
// translation is ggml_tensor -> moe_node (node_map below).
//
// Build: against a ggml tree's headers (ggml.h, ggml-backend-impl.h) with
// GGML_BACKEND_DL, linked with libmoe_block.so; ggml's functions resolve
// from the host process that loads it, as for every dynamically loaded
// ggml backend.  In this repository it is compiled by the tests against
// test-only headers that declare the fields it uses.
//
// Environment (the reference's names, so that a drop-in keeps its scripts):
//   MOESERV_DISABLE        claim nothing (moe_node_claimed)
//   MOESERV_TP_BUDGET_MB   device bytes the expert layers may use (MB; 0 =
//                          every layer stays on the CPU); default: the
//                          device's free memory less MOESERV_RESERVE_MB
//   MOESERV_RESERVE_MB     device memory held back from the expert layers
//                          for the per-call scratch (default 1024)
//   MOESERV_PROFILE=<p>    per-split phase rows written to <p>-<pid>.csv at
//                          teardown, one row per split in the reference's 14
//                          columns (dev 0 = the GPU, -1 = the CPU delegate),
//                          and the per-device means on stderr
#include "ggml-backend-impl.h"
#include "ggml.h"
#include "moe_block.h"

#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#define MOE_GGML_NAME "MoE"

namespace {

// ---------------------------------------------------------------------------
// process-wide state (the backend is one set of singletons, driven by the
// scheduler thread one split at a time, as the reference's is)

// One MOESERV_PROFILE row, in the reference's columns (moe-serv/src/moe_prof.h:36-56).
// A device split is one pass over all its tokens, so chunk = n_tok and n_chunks = 1;
// build = graph_compute's own work before the device call (node conversion and the
// split parse); alloc = making the layer resident, on its first split only (the
// per-call scratch is reused, so there is no per-call allocation to time); free is 0.
struct split_row {
  uint64_t call;
  int dev;  // 0: the GPU, -1: the CPU delegate
  int n_nodes;
  int64_t n_tok, chunk, n_chunks, n_exp;
  double build_us, alloc_us, upload_us, compute_us, read_us, free_us, total_us;
};

struct backend_state {
  ggml_backend_buffer_t weights_buf = nullptr;  // the buffer that holds the model's expert weights
  moe_ctx *ctx = nullptr;
  bool ctx_tried = false;
  std::map<int, bool> layer_ok;  // layer -> resident (false: it fell back once and stays on the CPU)
  uint64_t n_device = 0, n_cpu = 0, n_calls = 0;
  int refusals_shown = 0;
  bool first_reported = false;
  ggml_backend_t cpu = nullptr;
  bool profile_checked = false;
  std::string profile_prefix;
  std::vector<split_row> rows;
};

backend_state g_state;

double now_us() {
  return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

ggml_backend_buffer_type_t moe_buffer_type();

// ---------------------------------------------------------------------------
// ggml_tensor -> moe_node

bool storage_is_ours(const ggml_tensor *t) {
  if (!t) return false;
  const ggml_tensor *s = t->view_src ? t->view_src : t;
  return s->buffer != nullptr && s->buffer->buft == moe_buffer_type();
}

int node_op(enum ggml_op op) {
  switch (op) {
    case GGML_OP_NONE: return MOE_NODE_NONE;
    case GGML_OP_RESHAPE: return MOE_NODE_RESHAPE;
    case GGML_OP_VIEW: return MOE_NODE_VIEW;
    case GGML_OP_PERMUTE: return MOE_NODE_PERMUTE;
    case GGML_OP_TRANSPOSE: return MOE_NODE_TRANSPOSE;
    case GGML_OP_MUL_MAT_ID: return MOE_NODE_MUL_MAT_ID;
    case GGML_OP_CLAMP: return MOE_NODE_CLAMP;
    case GGML_OP_MUL: return MOE_NODE_MUL;
    case GGML_OP_GLU: return MOE_NODE_GLU;
    case GGML_OP_ADD: return MOE_NODE_ADD;
    default: return MOE_NODE_OTHER;
  }
}

// The nodes of one question (one supports_op, one split), converted down to
// `depth` links from where they were asked for: the claim set looks 4 links
// up, the split parse 6, and neither needs the rest of the model's graph.
// std::unordered_map keeps its elements' addresses, so src pointers hold.
struct node_map {
  std::unordered_map<const ggml_tensor *, moe_node> nodes;
  std::unordered_map<const ggml_tensor *, int> depth;

  const moe_node *get(const ggml_tensor *t, int d) {
    if (!t) return nullptr;
    auto it = depth.find(t);
    if (it != depth.end() && it->second >= d) return &nodes[t];
    moe_node &n = nodes[t];
    depth[t] = d;
    n = moe_node{};
    n.op = node_op(t->op);
    n.type = (int32_t)t->type;
    for (int i = 0; i < 4; i++) n.ne[i] = t->ne[i];
    n.contiguous = ggml_is_contiguous(t) ? 1 : 0;
    n.in_moe_buffer = storage_is_ours(t) ? 1 : 0;
    if (t->op == GGML_OP_GLU) {
      n.glu_op = (int32_t)ggml_get_glu_op(t);
      memcpy(&n.glu_swapped, &t->op_params[1], sizeof(int32_t));
    }
    if (t->op == GGML_OP_CLAMP) {
      memcpy(&n.clamp_min, &t->op_params[0], sizeof(float));
      memcpy(&n.clamp_max, &t->op_params[1], sizeof(float));
    }
    n.data = t->data;
    n.name = ggml_get_name(t);
    if (d > 0) {
      for (int i = 0; i < 3; i++) n.src[i] = get(t->src[i], d - 1);
      n.view_src = get(t->view_src, d - 1);
    }
    return &nodes[t];
  }
};

// ---------------------------------------------------------------------------
// the CPU delegate: the host's own CPU backend, from its registry

ggml_backend_t cpu_backend() {
  if (!g_state.cpu) {
    g_state.cpu = ggml_backend_init_by_type(GGML_BACKEND_DEVICE_TYPE_CPU, nullptr);
    if (!g_state.cpu)
      fprintf(stderr, "%s: the host registry holds no CPU backend, so a split the device declines cannot run\n",
              MOE_GGML_NAME);
  }
  return g_state.cpu;
}

bool profiling() {
  if (!g_state.profile_checked) {
    g_state.profile_checked = true;
    if (const char *p = getenv("MOESERV_PROFILE")) g_state.profile_prefix = p;
  }
  return !g_state.profile_prefix.empty();
}

// The residency budget: MOESERV_TP_BUDGET_MB when set; otherwise the device's
// free memory less MOESERV_RESERVE_MB (default 1 GiB), held back for the
// per-call scratch so that a later, larger call (a prefill after decode) still
// finds room (the reference's placement holds the same reserve per device,
// moe-serv/src/moe_place.h:56-78).
uint64_t residency_budget() {
  if (const char *b = getenv("MOESERV_TP_BUDGET_MB")) return (uint64_t)strtoull(b, nullptr, 10) << 20;
  uint64_t reserve = 1024ull << 20;
  if (const char *r = getenv("MOESERV_RESERVE_MB")) reserve = (uint64_t)strtoull(r, nullptr, 10) << 20;
  uint64_t free_b = 0, total_b = 0;
  if (moe_device_memory(0, &free_b, &total_b) != MOE_OK) return UINT64_MAX;  // ctx creation reports it
  const uint64_t budget = free_b > reserve ? free_b - reserve : 0;
  fprintf(stderr, "%s-gfx950: residency budget %llu MB (%llu MB free, %llu MB held back)\n", MOE_GGML_NAME,
          (unsigned long long)(budget >> 20), (unsigned long long)(free_b >> 20), (unsigned long long)(reserve >> 20));
  return budget;
}

// Device context on first use: absent device, NO_DEVICE or a zero budget all
// leave ctx null and every split on the CPU.
moe_ctx *device_ctx() {
  if (!g_state.ctx_tried) {
    g_state.ctx_tried = true;
    const uint64_t budget = residency_budget();
    const moe_status st = moe_ctx_create(0, budget, &g_state.ctx);
    if (st != MOE_OK) {
      fprintf(stderr, "%s-gfx950: no device context (%s); every split runs on the CPU\n", MOE_GGML_NAME,
              moe_status_str(st));
      g_state.ctx = nullptr;
    } else if (profiling()) {
      (void)moe_prof_enable(g_state.ctx, 1);
    }
  }
  return g_state.ctx;
}

long long us(double v) { return (long long)llround(v); }

// <prefix>-<pid>.csv in the reference's columns (integer microseconds), then the
// per-device means on stderr (moe-serv/src/moe_prof.h:94-137).
void write_profile() {
  char path[1024];
  snprintf(path, sizeof path, "%s-%d.csv", g_state.profile_prefix.c_str(), (int)getpid());
  FILE *f = fopen(path, "wb");
  if (!f) {
    fprintf(stderr, "%s-gfx950: cannot write %s\n", MOE_GGML_NAME, path);
    return;
  }
  fprintf(f, "call,dev,n_nodes,n_tok,chunk,n_chunks,n_exp_loads,"
             "build_us,alloc_us,upload_us,compute_us,read_us,free_us,total_us\n");
  for (const split_row &r : g_state.rows)
    fprintf(f, "%llu,%d,%d,%lld,%lld,%lld,%lld,%lld,%lld,%lld,%lld,%lld,%lld,%lld\n", (unsigned long long)r.call,
            r.dev, r.n_nodes, (long long)r.n_tok, (long long)r.chunk, (long long)r.n_chunks, (long long)r.n_exp,
            us(r.build_us), us(r.alloc_us), us(r.upload_us), us(r.compute_us), us(r.read_us), us(r.free_us),
            us(r.total_us));
  fclose(f);
  fprintf(stderr, "%s-gfx950: profile -> %s (%zu rows)\n", MOE_GGML_NAME, path, g_state.rows.size());
  for (int dev = -1; dev <= 0; dev++) {
    double n = 0, sum[7] = {0, 0, 0, 0, 0, 0, 0};
    for (const split_row &r : g_state.rows) {
      if (r.dev != dev) continue;
      n++;
      const double v[7] = {r.build_us, r.alloc_us, r.upload_us, r.compute_us, r.read_us, r.free_us, r.total_us};
      for (int i = 0; i < 7; i++) sum[i] += v[i];
    }
    if (n == 0) continue;
    fprintf(stderr,
            "%s-gfx950:   %-8s n=%-6lld mean us: build %.1f alloc %.1f upload %.1f compute %.1f read %.1f free %.1f"
            " | total %.1f\n",
            MOE_GGML_NAME, dev < 0 ? "cpu" : "gfx950", (long long)n, sum[0] / n, sum[1] / n, sum[2] / n, sum[3] / n,
            sum[4] / n, sum[5] / n, sum[6] / n);
  }
}

void report_and_reset() {
  if (g_state.n_device || g_state.n_cpu)
    fprintf(stderr, "%s-gfx950: %llu splits on the device, %llu fell back\n", MOE_GGML_NAME,
            (unsigned long long)g_state.n_device, (unsigned long long)g_state.n_cpu);
  if (g_state.ctx) {
    moe_call_stats cs;
    if (moe_call_stats_read(g_state.ctx, &cs, 0) == MOE_OK && cs.timed_calls) {
      const double n = (double)cs.timed_calls;
      fprintf(stderr, "%s-gfx950: per call us: upload %.1f  compute %.1f  read %.1f  total %.1f  experts %.1f\n",
              MOE_GGML_NAME, cs.upload_us / n, cs.compute_us / n, cs.read_us / n, cs.total_us / (double)cs.calls,
              (double)cs.expert_loads / (double)cs.calls);
    }
  }
  if (profiling() && !g_state.rows.empty()) write_profile();
  if (g_state.ctx) moe_ctx_destroy(g_state.ctx);
  ggml_backend_t cpu = g_state.cpu;
  g_state = backend_state();
  g_state.cpu = cpu;  // the delegate belongs to the host's registry, not to the model
}

// ---------------------------------------------------------------------------
// buffer: plain host memory (is_host: unclaimed ops and the CPU delegate read
// the weights in place, moe-serv/src/moe_backend.cpp:40-50)

struct host_buffer {
  void *data = nullptr;
  size_t size = 0;
};

void buffer_free(ggml_backend_buffer_t buffer) {
  auto *hb = (host_buffer *)buffer->context;
  // only the weights buffer ends the model: zero-size probe buffers and the
  // scheduler's compute buffer are of this type too (moe_backend.cpp:64-85)
  if (buffer == g_state.weights_buf) report_and_reset();
  free(hb->data);
  delete hb;
}

void *buffer_get_base(ggml_backend_buffer_t buffer) { return ((host_buffer *)buffer->context)->data; }

// the one hook that sees a tensor's name before its data: a "blk.N." tensor
// marks this buffer as the one holding the model's expert weights
enum ggml_status buffer_init_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor) {
  const char *name = ggml_get_name(tensor);
  if (name && strncmp(name, "blk.", 4) == 0 && name[4] >= '0' && name[4] <= '9') g_state.weights_buf = buffer;
  return GGML_STATUS_SUCCESS;
}

void buffer_memset_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, uint8_t value, size_t offset,
                          size_t size) {
  GGML_UNUSED(buffer);
  memset((char *)tensor->data + offset, value, size);
}

void buffer_set_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, const void *data, size_t offset,
                       size_t size) {
  GGML_UNUSED(buffer);
  memcpy((char *)tensor->data + offset, data, size);
}

void buffer_get_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *tensor, void *data, size_t offset,
                       size_t size) {
  GGML_UNUSED(buffer);
  memcpy(data, (const char *)tensor->data + offset, size);
}

bool buffer_cpy_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *src, ggml_tensor *dst) {
  GGML_UNUSED(buffer);
  if (!src->buffer || !ggml_backend_buffer_is_host(src->buffer)) return false;  // ggml then stages the copy
  memcpy(dst->data, src->data, ggml_nbytes(src));
  return true;
}

void buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
  auto *hb = (host_buffer *)buffer->context;
  if (hb->data) memset(hb->data, value, hb->size);
}

const ggml_backend_buffer_i k_buffer_i = {
    /* .free_buffer   = */ buffer_free,
    /* .get_base      = */ buffer_get_base,
    /* .init_tensor   = */ buffer_init_tensor,
    /* .memset_tensor = */ buffer_memset_tensor,
    /* .set_tensor    = */ buffer_set_tensor,
    /* .get_tensor    = */ buffer_get_tensor,
    /* .set_tensor_2d = */ nullptr,
    /* .get_tensor_2d = */ nullptr,
    /* .cpy_tensor    = */ buffer_cpy_tensor,
    /* .clear         = */ buffer_clear,
    /* .reset         = */ nullptr,
};

// ---------------------------------------------------------------------------
// buffer type "MoE"

const char *buft_get_name(ggml_backend_buffer_type_t buft) {
  GGML_UNUSED(buft);
  return MOE_GGML_NAME;
}

ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
  auto *hb = new host_buffer;
  hb->size = size;
  hb->data = size ? malloc(size) : nullptr;  // ggml asks for zero-size buffers; malloc(0) may be null
  if (size && !hb->data) {
    fprintf(stderr, "%s: cannot allocate %zu bytes of host memory\n", MOE_GGML_NAME, size);
    delete hb;
    return nullptr;
  }
  return ggml_backend_buffer_init(buft, k_buffer_i, hb, size);
}

size_t buft_get_alignment(ggml_backend_buffer_type_t buft) {
  GGML_UNUSED(buft);
  return 64;
}

bool buft_is_host(ggml_backend_buffer_type_t buft) {
  GGML_UNUSED(buft);
  return true;
}

// ---------------------------------------------------------------------------
// device: ACCEL, so that -ngl never assigns it trunk layers (moe_backend.cpp:231-243)

const char *dev_get_name(ggml_backend_dev_t dev) {
  GGML_UNUSED(dev);
  return MOE_GGML_NAME;
}

const char *dev_get_description(ggml_backend_dev_t dev) {
  GGML_UNUSED(dev);
  return "routed-expert MoE block on MI355X (gfx950)";
}

void dev_get_memory(ggml_backend_dev_t dev, size_t *free_, size_t *total) {
  GGML_UNUSED(dev);
  *free_ = 0;  // host buffers only: no device memory to report to the scheduler
  *total = 0;
}

enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t dev) {
  GGML_UNUSED(dev);
  return GGML_BACKEND_DEVICE_TYPE_ACCEL;
}

void dev_get_props(ggml_backend_dev_t dev, ggml_backend_dev_props *props) {
  props->name = dev_get_name(dev);
  props->description = dev_get_description(dev);
  props->type = dev_get_type(dev);
  dev_get_memory(dev, &props->memory_free, &props->memory_total);
  props->caps.async = false;
  props->caps.host_buffer = false;
  props->caps.buffer_from_host_ptr = false;
  props->caps.events = false;
}

bool dev_supports_op(ggml_backend_dev_t dev, const ggml_tensor *op) {
  GGML_UNUSED(dev);
  node_map m;
  return moe_node_claimed(m.get(op, 5)) != 0;
}

bool dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft) {
  GGML_UNUSED(dev);
  return buft == moe_buffer_type();
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *params);

ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t dev) {
  GGML_UNUSED(dev);
  return moe_buffer_type();
}

const ggml_backend_device_i k_device_i = {
    /* .get_name             = */ dev_get_name,
    /* .get_description      = */ dev_get_description,
    /* .get_memory           = */ dev_get_memory,
    /* .get_type             = */ dev_get_type,
    /* .get_props            = */ dev_get_props,
    /* .init_backend         = */ dev_init_backend,
    /* .get_buffer_type      = */ dev_get_buffer_type,
    /* .get_host_buffer_type = */ nullptr,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    /* .offload_op           = */ nullptr,
    /* .event_new            = */ nullptr,
    /* .event_free           = */ nullptr,
    /* .event_synchronize    = */ nullptr,
};

// ---------------------------------------------------------------------------
// backend: graph_compute is the one entry point

const char *backend_get_name(ggml_backend_t backend) {
  GGML_UNUSED(backend);
  return MOE_GGML_NAME;
}

void backend_free(ggml_backend_t backend) { delete backend; }

// The n_tok of a split that did not parse: the first MUL_MAT_ID's ids tensor,
// as the reference counts its CPU rows (moe_backend.cpp:469-480).
int64_t tokens_of(ggml_cgraph *cgraph) {
  for (int i = 0; i < ggml_graph_n_nodes(cgraph); i++) {
    const ggml_tensor *t = ggml_graph_node(cgraph, i);
    if (t->op == GGML_OP_MUL_MAT_ID && t->src[2]) return t->src[2]->ne[1];
  }
  return 0;
}

enum ggml_status run_on_cpu(ggml_cgraph *cgraph, split_row &row, double t0) {
  g_state.n_cpu++;
  ggml_backend_t cpu = cpu_backend();
  if (!cpu) return GGML_STATUS_FAILED;
  const double tc = now_us();
  const enum ggml_status st = ggml_backend_graph_compute(cpu, cgraph);
  if (profiling()) {
    row.dev = -1;
    if (!row.n_tok) row.n_tok = tokens_of(cgraph);
    row.chunk = row.n_tok;
    row.n_chunks = 1;
    row.compute_us = now_us() - tc;
    row.total_us = now_us() - t0;
    g_state.rows.push_back(row);
  }
  return st;
}

void refusal(const char *why) {
  if (g_state.refusals_shown < 3) {  // at most three, as the reference logs its parse fallbacks
    g_state.refusals_shown++;
    fprintf(stderr, "%s-gfx950: CPU fallback: %s\n", MOE_GGML_NAME, why);
  }
}

// The device form of a split's clamps: none, or gate <= L and up in [-L, L]
// (the deepseek4 order the kernels apply); anything else stays on the CPU.
bool clamp_of(const moe_split &sp, float *L) {
  if (std::isinf(sp.gate_max) && std::isinf(sp.up_max) && std::isinf(sp.gate_min) && std::isinf(sp.up_min)) {
    *L = 0.0f;
    return true;
  }
  const float l = sp.up_max;
  if (l > 1e-6f && std::isfinite(l) && sp.up_min == -l && sp.gate_max == l && std::isinf(sp.gate_min) &&
      sp.gate_min < 0) {
    *L = l;
    return true;
  }
  return false;
}

enum ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
  GGML_UNUSED(backend);
  if (!cgraph) return GGML_STATUS_FAILED;
  const double t0 = now_us();
  const int n = ggml_graph_n_nodes(cgraph);
  if (!g_state.first_reported) {
    g_state.first_reported = true;
    int counts[GGML_OP_COUNT] = {0};
    for (int i = 0; i < n; i++) counts[ggml_graph_node(cgraph, i)->op]++;
    fprintf(stderr, "%s-gfx950: first split has %d nodes:", MOE_GGML_NAME, n);
    for (int o = 0; o < GGML_OP_COUNT; o++)
      if (counts[o]) fprintf(stderr, " %s x%d", ggml_op_name((enum ggml_op)o), counts[o]);
    fprintf(stderr, "\n");
  }
  split_row row = {};
  row.call = g_state.n_calls++;
  row.n_nodes = n;
  node_map m;
  std::vector<const moe_node *> nodes((size_t)n);
  for (int i = 0; i < n; i++) nodes[i] = m.get(ggml_graph_node(cgraph, i), 6);
  moe_split sp;
  char why[256];
  const bool parsed = moe_split_parse(nodes.data(), n, &sp, why, sizeof why) == MOE_OK;
  row.build_us = now_us() - t0;
  if (!parsed) {
    refusal(why);
    return run_on_cpu(cgraph, row, t0);
  }
  row.n_tok = sp.n_tokens;
  moe_ctx *ctx = device_ctx();
  if (!ctx) return run_on_cpu(cgraph, row, t0);
  auto it = g_state.layer_ok.find(sp.layer);
  if (it != g_state.layer_ok.end() && !it->second) return run_on_cpu(cgraph, row, t0);  // fell back once: stays
  if (it == g_state.layer_ok.end()) {
    // first split of this layer: make it resident from the weights' host data
    moe_layer_desc d = {};
    d.hidden = sp.hidden;
    d.ffn = sp.ffn;
    d.n_expert = sp.n_expert;
    d.n_used = sp.n_slots;
    d.has_shared = 0;  // the split carries the routed experts only; the trunk keeps the shared one
    float L = 0.0f;
    bool ok = clamp_of(sp, &L);
    if (!ok) {
      snprintf(why, sizeof why, "layer %d: clamps gate [%g, %g], up [%g, %g] have no device form", sp.layer,
               sp.gate_min, sp.gate_max, sp.up_min, sp.up_max);
      refusal(why);
    } else {
      d.clamp = L;
      const double ta = now_us();
      const moe_status st = moe_layer_upload(ctx, sp.layer, &d, sp.gate_w->data, sp.up_w->data, sp.down_w->data,
                                             nullptr, nullptr, nullptr);
      row.alloc_us = now_us() - ta;
      ok = st == MOE_OK;
      if (ok) {
        uint64_t bytes = 0;
        (void)moe_layer_bytes(ctx, sp.layer, &bytes);
        fprintf(stderr, "%s-gfx950: layer %d resident, %llu MB\n", MOE_GGML_NAME, sp.layer,
                (unsigned long long)(bytes >> 20));
      } else {
        snprintf(why, sizeof why, "layer %d: %s", sp.layer, moe_ctx_last_error(ctx));
        refusal(why);
      }
    }
    g_state.layer_ok[sp.layer] = ok;
    if (!ok) return run_on_cpu(cgraph, row, t0);
  }
  if (moe_split_compute(ctx, nodes.data(), n) != MOE_OK) {
    refusal(moe_ctx_last_error(ctx));
    return run_on_cpu(cgraph, row, t0);
  }
  if (g_state.n_device++ == 0)
    fprintf(stderr, "%s-gfx950: computed a split on the device (layer %d, %d slots, %d tokens)\n", MOE_GGML_NAME,
            sp.layer, sp.n_slots, sp.n_tokens);
  if (profiling()) {
    moe_call_stats cs;
    if (moe_call_stats_read(ctx, &cs, 0) == MOE_OK) {
      row.dev = 0;
      row.chunk = row.n_tok;
      row.n_chunks = 1;
      row.n_exp = cs.last_experts;
      row.upload_us = cs.last_upload_us;
      row.compute_us = cs.last_compute_us;
      row.read_us = cs.last_read_us;
      row.total_us = now_us() - t0;
      g_state.rows.push_back(row);
    }
  }
  return GGML_STATUS_SUCCESS;
}

const ggml_backend_i k_backend_i = {
    /* .get_name             = */ backend_get_name,
    /* .free                 = */ backend_free,
    /* .set_tensor_async     = */ nullptr,
    /* .get_tensor_async     = */ nullptr,
    /* .set_tensor_2d_async  = */ nullptr,
    /* .get_tensor_2d_async  = */ nullptr,
    /* .cpy_tensor_async     = */ nullptr,
    /* .synchronize          = */ nullptr,
    /* .graph_plan_create    = */ nullptr,
    /* .graph_plan_free      = */ nullptr,
    /* .graph_plan_update    = */ nullptr,
    /* .graph_plan_compute   = */ nullptr,
    /* .graph_compute        = */ backend_graph_compute,
    /* .event_record         = */ nullptr,
    /* .event_wait           = */ nullptr,
    /* .graph_optimize       = */ nullptr,
};

ggml_guid_t backend_guid() {
  static ggml_guid guid = {0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x2d, 0x6d,
                           0x6f, 0x65, 0x2d, 0x62, 0x6c, 0x6f, 0x63, 0x6b};  // "gfx950-moe-block"
  return &guid;
}

// ---------------------------------------------------------------------------
// reg: one device; get_proc_address hands llama.cpp our thread-count setter

const char *reg_get_name(ggml_backend_reg_t reg) {
  GGML_UNUSED(reg);
  return MOE_GGML_NAME;
}

size_t reg_get_device_count(ggml_backend_reg_t reg) {
  GGML_UNUSED(reg);
  return 1;
}

ggml_backend_reg_t moe_reg();

ggml_backend_dev_t reg_get_device(ggml_backend_reg_t reg, size_t index) {
  GGML_ASSERT(index == 0);
  static ggml_backend_device dev = {k_device_i, nullptr, nullptr};
  dev.reg = reg;
  return &dev;
}

// llama.cpp calls this with its own thread count; the CPU delegate must run
// with the same count, or its summation order (and so its bits) differs from
// a run without this backend (moe_backend.cpp:539-572).
void set_n_threads(ggml_backend_t backend, int n_threads) {
  GGML_UNUSED(backend);
  ggml_backend_t cpu = cpu_backend();
  if (!cpu) return;
  ggml_backend_dev_t dev = ggml_backend_get_device(cpu);
  ggml_backend_reg_t reg = dev ? ggml_backend_dev_backend_reg(dev) : nullptr;
  auto fn = reg ? (ggml_backend_set_n_threads_t)ggml_backend_reg_get_proc_address(reg, "ggml_backend_set_n_threads")
                : nullptr;
  static bool reported = false;
  if (!reported) {
    reported = true;
    fprintf(stderr, "%s-gfx950: CPU delegate threads %s %d\n", MOE_GGML_NAME,
            fn ? "set to" : "cannot be set (left at ggml's default); asked for", n_threads);
  }
  if (fn) fn(cpu, n_threads);
}

void *reg_get_proc_address(ggml_backend_reg_t reg, const char *name) {
  GGML_UNUSED(reg);
  if (name && strcmp(name, "ggml_backend_set_n_threads") == 0) return (void *)set_n_threads;
  return nullptr;
}

const ggml_backend_reg_i k_reg_i = {
    /* .get_name         = */ reg_get_name,
    /* .get_device_count = */ reg_get_device_count,
    /* .get_device       = */ reg_get_device,
    /* .get_proc_address = */ reg_get_proc_address,
};

ggml_backend_reg_t moe_reg() {
  static ggml_backend_reg reg = {GGML_BACKEND_API_VERSION, k_reg_i, nullptr};
  return &reg;
}

ggml_backend_buffer_type_t moe_buffer_type() {
  static ggml_backend_buffer_type buft = {
      {buft_get_name, buft_alloc_buffer, buft_get_alignment, nullptr, nullptr, buft_is_host}, nullptr, nullptr};
  buft.device = reg_get_device(moe_reg(), 0);
  return &buft;
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *params) {
  GGML_UNUSED(params);
  return new ggml_backend{backend_guid(), k_backend_i, dev, nullptr};
}

// Always loadable, as the reference's (moe_backend.cpp:625-631): without a
// usable gfx950 device every split goes to the CPU delegate, so a run with
// this library loaded computes what a run without it does.
int backend_score() { return 1; }

}  // namespace

GGML_BACKEND_DL_IMPL(moe_reg)
GGML_BACKEND_DL_SCORE_IMPL(backend_score)
