// moe_block.hip -- host side of the gfx950 MoE block behind include/moe_block.h.
//
// Owns: the device context, per-layer expert residency under a byte budget
// (moe-serv/src/moe_tp.h:551-707 and moe-serv/src/moe_mirror.h:68-119 are
// the reference's counterparts), per-call scratch sized once, dispatch of
// the decode / grouped kernel chains, and hipGraph capture of a stack of
// layers.  Everything here is plain C++ around hip* calls; no torch.
#include "../../include/moe_block.h"

#include "device_common.h"
#include "gguf_reader.h"
#include "kernels_decode.h"
#include "kernels_group.h"
#include "kernels_grouped.h"
#include "kernels_rows.h"
#include "kernels_stacked.h"

#include "kernels_weights.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

namespace {

enum { T_GATE = 0, T_UP = 1, T_DOWN = 2 };

// One tensor of a layer (gate, up or down) for all E' = E + has_shared
// experts, in the row-interleaved layout of kernels_weights.h.
struct dev_mat {
  uint8_t *w = nullptr;   // E' matrices of `stride` bytes (kernels_weights.h records)
  int rows = 0, kb = 0;
  uint64_t stride = 0;
};

struct dev_layer {
  moe_layer_desc d{};
  int n_mats = 0;      // E + has_shared (the shared expert is expert index E)
  dev_mat m[3];        // gate, up, down
  uint64_t bytes = 0;
  int graph_refs = 0;  // live graphs (moe_graph_capture) that read these weights
};

struct work_bufs {
  // sized for (T, H, F, E, k)
  int T = 0, H = 0, F = 0, E = 0, k = 0;
  uint32_t *hq = nullptr; float *hd = nullptr;     // staged h: [P+T][F/32][16] dwords, [P+T][F/32]
  float *htap = nullptr;                           // [P+T][F]
  float *y = nullptr;                              // [P+T][H]
  uint32_t *xq = nullptr; float *xd = nullptr;     // staged x of the grouped chain: [T][H/32][16] dwords, [T][H/32]
  // balanced decode gate/up: per-task row sums [16 slots][F/32][4][16] and
  // per-unit tickets (zeroed here once, left at zero by every launch)
  float *part = nullptr; int *tick = nullptr;
  int32_t *grp = nullptr;                          // grouping workspace
  size_t grp_words = 0;
  // host-boundary staging
  // one allocation for the three inputs, laid out as moe_forward_host's pinned
  // staging (ids at 0, wts at in_wts, x at in_x bytes) so one copy moves them
  int32_t *ids_in = nullptr; float *wts_in = nullptr; float *x_in = nullptr; float *out_buf = nullptr;
  size_t in_wts = 0, in_x = 0;
  size_t out_cap = 0;
  size_t h_rows = 0;     // rows written to htap by the last forward
  int last_F = 0;
  bool timed = true;     // kernels on these buffers are timed by the profiler (moe_prof_*)
};

}  // namespace

// Kernel classes timed by the profiler (moe_prof_*), in the order of
// kernel_names[].
enum { K_ROUTE = 0, K_GROUP, K_GU_DECODE, K_DOWN_DECODE, K_GU_GROUPED, K_DOWN_GROUPED,
       K_COMBINE, K_COUNT };
static const char *const kernel_names[K_COUNT] = {
    "route", "group", "gate_up_decode", "down_decode", "gate_up_grouped",
    "down_grouped", "combine"};

struct prof_state {
  bool on = false;
  struct rec { int kid; hipEvent_t a, b; };
  std::vector<hipEvent_t> pool;  // idle events
  std::vector<rec> pending;      // recorded, not yet read
  uint64_t launches[K_COUNT] = {};
  double total_us[K_COUNT] = {};
};

// Engagement and phase counters of the host-boundary calls (moe_forward_host,
// moe_split_compute), read with moe_call_stats_read.
struct call_state {
  uint64_t calls = 0, refusals = 0, expert_loads = 0, timed = 0;
  double upload_us = 0, compute_us = 0, read_us = 0, total_us = 0;
  moe_call_stats last{};
  hipEvent_t ev[4] = {};  // phase events, created at the first profiled call
};

struct moe_ctx {
  int device = 0;
  int n_cu = 256;
  uint64_t budget = 0, used = 0;
  std::map<int, dev_layer> layers;
  work_bufs sc;
  std::string err;
  int inject = 0;  // bit 0: forward fails, bit 1: budget forced to 0
  bool capturing = false;
  bool taps = false;  // keep the SwiGLU output h in sc.htap (moe_debug_set_taps)
  // per-wave timestamps of the last decode call's k_gate_up_bal2 and k_down_dec
  // (moe_debug_set_timeline): MOE_TL_RECORDS records of 3 stamps
  unsigned long long *tl = nullptr;
  size_t tl_gu = 0, tl_dn = 0;  // records written by the last decode call
  prof_state prof;
  // moe_forward_host's pinned staging (x, ids, wts in; out back), grown on demand
  uint8_t *pin = nullptr;
  size_t pin_bytes = 0;
  // Live graphs.  A graph holds raw device pointers to the scratch and to the
  // weights of the layers it captured, so while one is alive the scratch is
  // never reallocated and those layers are never released.
  std::set<moe_graph *> graphs;
  call_state calls;
  // this device's copy of the file-scope no-allocation scratch (null if its
  // set-up failed; noalloc_err says why)
  uint8_t *noalloc = nullptr;
  std::string noalloc_err;
};

// HIP-event pair around one kernel launch while profiling is on (never
// under graph capture: a captured launch is timed by its replays instead).
struct prof_scope {
  moe_ctx *c;
  int kid;
  hipStream_t st;
  hipEvent_t a = nullptr, b = nullptr;
  static hipEvent_t take(prof_state &p) {
    hipEvent_t e = nullptr;
    if (!p.pool.empty()) {
      e = p.pool.back();
      p.pool.pop_back();
    } else if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) {  // timing only: no cache flush
      e = nullptr;
    }
    return e;
  }
  prof_scope(moe_ctx *ctx, int k, hipStream_t s, bool timed) : c(ctx), kid(k), st(s) {
    if (!timed || !c->prof.on || c->capturing) return;
    a = take(c->prof);
    b = a ? take(c->prof) : nullptr;
    if (a && b && hipEventRecord(a, st) != hipSuccess) {
      c->prof.pool.push_back(a);
      c->prof.pool.push_back(b);
      a = b = nullptr;
    } else if (a && !b) {
      c->prof.pool.push_back(a);
      a = nullptr;
    }
  }
  ~prof_scope() {
    if (!a) return;
    if (hipEventRecord(b, st) == hipSuccess) {
      c->prof.pending.push_back({kid, a, b});
    } else {
      c->prof.pool.push_back(a);
      c->prof.pool.push_back(b);
    }
  }
};

struct moe_graph {
  moe_ctx *ctx = nullptr;      // null once the context is destroyed
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<int> layers;     // distinct layers the graph reads (one graph_refs count each)
};

// Drop a graph's executable and its holds on the context (its layers'
// graph_refs and its entry in ctx->graphs).
static void graph_detach(moe_graph *g) {
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  g->exec = nullptr;
  g->graph = nullptr;
  if (!g->ctx) return;
  for (int l : g->layers) {
    auto it = g->ctx->layers.find(l);
    if (it != g->ctx->layers.end() && it->second.graph_refs > 0) it->second.graph_refs--;
  }
  g->ctx->graphs.erase(g);
  g->ctx = nullptr;
}

// ---------------------------------------------------------------------------
static moe_status fail(moe_ctx *c, moe_status s, const char *fmt, ...) {
  if (c) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
  }
  return s;
}

#define HIPC(ctx, call)                                                                  \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess)                                                                \
      return fail((ctx), MOE_ERR_HIP, "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), \
                  __FILE__, __LINE__);                                                   \
  } while (0)

static int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// SplitMix64's output function, the host half of the weight generator's key
// derivation (the device half is mix64 in device_common.h).
static uint64_t host_mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static bool desc_ok(const moe_layer_desc *d) {
  // hidden and ffn are both a row count (multiple of 64 rows per lane group)
  // and a reduction length (multiple of 4 blocks of 32 per exponent dword)
  return d && d->hidden > 0 && d->ffn > 0 && d->n_expert > 0 && d->n_used > 0 &&
         d->hidden % 128 == 0 && d->ffn % 128 == 0 && d->n_used <= d->n_expert &&
         d->n_used <= 64 && d->n_expert <= MOE_ROUTE_MAX_E && (d->has_shared == 0 || d->has_shared == 1);
}

static uint64_t layer_bytes(const moe_layer_desc *d) {
  const uint64_t n = (uint64_t)d->n_expert + (uint64_t)d->has_shared;
  const uint64_t gu = (uint64_t)d->ffn * (d->hidden / 32) * 17u;
  const uint64_t dn = (uint64_t)d->hidden * (d->ffn / 32) * 17u;
  return n * (2 * gu + dn);
}

// ---------------------------------------------------------------------------
// scratch

#define MOE_TL_RECORDS 8192  // debug timeline: waves of one decode call's two launches

static void scratch_free(work_bufs &s) {
  void *ptrs[] = {s.hq, s.hd, s.htap, s.y, s.xq, s.xd, s.part, s.tick, s.grp, s.ids_in, s.out_buf};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  s = work_bufs();
}

static moe_status scratch_reserve(moe_ctx *c, int T, int H, int F, int E, int k) {
  work_bufs &s = c->sc;
  if (s.hq && T <= s.T && H <= s.H && F <= s.F && E <= s.E && k <= s.k) return MOE_OK;
  if (c->capturing) return fail(c, MOE_ERR_INVALID_ARG, "scratch too small under graph capture; call moe_ctx_reserve first");
  if (!c->graphs.empty())
    return fail(c, MOE_ERR_INVALID_ARG,
                "the per-call scratch would be reallocated while %zu captured graph(s) still point at it; destroy "
                "them first, or reserve for the largest call before capturing",
                c->graphs.size());
  T = T > s.T ? T : s.T;
  H = H > s.H ? H : s.H;
  F = F > s.F ? F : s.F;
  E = E > s.E ? E : s.E;
  k = k > s.k ? k : s.k;
  HIPC(c, hipDeviceSynchronize());
  scratch_free(s);
  const size_t P = (size_t)T * k, R = P + T;
  HIPC(c, hipMalloc(&s.hq, R * (F / 32) * 64));
  HIPC(c, hipMalloc(&s.hd, R * (F / 32) * 4));
  HIPC(c, hipMalloc(&s.htap, R * F * 4));
  HIPC(c, hipMalloc(&s.y, R * H * 4));
  HIPC(c, hipMalloc(&s.xq, (size_t)T * (H / 32) * 64));
  HIPC(c, hipMalloc(&s.xd, (size_t)T * (H / 32) * 4));
  HIPC(c, hipMalloc(&s.part, (size_t)16 * (F / 32) * 4 * 16 * 4));
  HIPC(c, hipMalloc(&s.tick, (size_t)16 * (F / 32) * 4));
  HIPC(c, hipMemset(s.tick, 0, (size_t)16 * (F / 32) * 4));
  s.grp_words = group_ws_words(T, k, E);
  HIPC(c, hipMalloc(&s.grp, s.grp_words * 4));
  s.in_wts = P * 4;
  s.in_x = (2 * P * 4 + 255) & ~(size_t)255;
  HIPC(c, hipMalloc(&s.ids_in, s.in_x + (size_t)T * H * 4));
  s.wts_in = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(s.ids_in) + s.in_wts);
  s.x_in = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(s.ids_in) + s.in_x);
  s.out_cap = P * H;
  HIPC(c, hipMalloc(&s.out_buf, s.out_cap * 4));
  HIPC(c, hipDeviceSynchronize());
  s.T = T; s.H = H; s.F = F; s.E = E; s.k = k;
  return MOE_OK;
}

// ---------------------------------------------------------------------------
// The no-allocation entry point's scratch (moe_forward_noalloc): one
// file-scope device array, so that a call allocates nothing.  Every GPU the
// library runs on holds its own copy (MOE_NOALLOC_SCRATCH_BYTES) until the
// process ends.  Host code never uses the array's name as a device address:
// hipGetSymbolAddress gives each device's address once, at the first
// moe_ctx_create on that device, and that pointer is what the kernels get.
// Layout for one call: [ticks: MOE_NOALLOC_TICK_BYTES][part][hq][hd][y][xq][xd]
// [grouping workspace], each 256-byte aligned.  The ticks must be zero when a
// gate/up launch starts; they are cleared once here, and every launch that
// counts on a tick returns it to zero.

#define MOE_NOALLOC_TICK_BYTES ((size_t)64 << 10)
#define MOE_MAX_DEVICES 64

static __device__ __align__(256) uint8_t scratch[MOE_NOALLOC_SCRATCH_BYTES];

static std::mutex g_noalloc_mu;
static uint8_t *g_noalloc_ptr[MOE_MAX_DEVICES];

__global__ void k_fill_zero(uint32_t *__restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

// Once per device, with that device current.
static void noalloc_setup(moe_ctx *c) {
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (c->device >= MOE_MAX_DEVICES) {
    c->noalloc_err = "device index beyond the no-allocation table";
    return;
  }
  if (!g_noalloc_ptr[c->device]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      c->noalloc_err = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
      return;
    }
    hipLaunchKernelGGL(k_fill_zero, dim3(64), dim3(256), 0, 0, (uint32_t *)p, MOE_NOALLOC_TICK_BYTES / 4);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      c->noalloc_err = std::string("clearing the no-allocation ticks failed: ") + hipGetErrorString(e);
      return;
    }
    g_noalloc_ptr[c->device] = (uint8_t *)p;
  }
  c->noalloc = g_noalloc_ptr[c->device];
}

// Carve one call's buffers out of the no-allocation scratch at base; returns
// the bytes they need (buffers are set only when that fits the array).
static size_t noalloc_layout(uint8_t *base, int T, int H, int F, int E, int k, work_bufs &s) {
  const size_t P = (size_t)T * k, R = P + T;
  size_t off = MOE_NOALLOC_TICK_BYTES;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = (off + bytes + 255) & ~(size_t)255;
    return base + at;
  };
  uint8_t *part = take((size_t)16 * (F / 32) * 4 * 16 * 4);
  uint8_t *hq = take(R * (F / 32) * 64);
  uint8_t *hd = take(R * (F / 32) * 4);
  uint8_t *y = take(R * H * 4);
  uint8_t *xq = take((size_t)T * (H / 32) * 64);
  uint8_t *xd = take((size_t)T * (H / 32) * 4);
  const size_t grp_words = group_ws_words(T, k, E);
  uint8_t *grp = take(grp_words * 4);
  const bool ticks_fit = (size_t)16 * (F / 32) * 4 <= MOE_NOALLOC_TICK_BYTES;
  if (off > MOE_NOALLOC_SCRATCH_BYTES || !ticks_fit) return ticks_fit ? off : SIZE_MAX;
  s = work_bufs();
  s.T = T; s.H = H; s.F = F; s.E = E; s.k = k;
  s.tick = reinterpret_cast<int *>(base);
  s.part = reinterpret_cast<float *>(part);
  s.hq = reinterpret_cast<uint32_t *>(hq);
  s.hd = reinterpret_cast<float *>(hd);
  s.y = reinterpret_cast<float *>(y);
  s.xq = reinterpret_cast<uint32_t *>(xq);
  s.xd = reinterpret_cast<float *>(xd);
  s.grp = reinterpret_cast<int32_t *>(grp);
  s.grp_words = grp_words;
  s.timed = false;  // the profiler's events would be created on demand: not here
  return off;
}

// ---------------------------------------------------------------------------
// context

extern "C" moe_status moe_ctx_create(int device, uint64_t budget_bytes, moe_ctx **out) {
  if (!out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  const char *inj = getenv("MOE_BLOCK_INJECT");
  int inject = 0;
  if (inj) {
    if (strstr(inj, "forward")) inject |= 1;
    if (strstr(inj, "budget")) inject |= 2;
    if (strstr(inj, "nodevice")) return MOE_ERR_NO_DEVICE;
  }
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return MOE_ERR_NO_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return MOE_ERR_NO_DEVICE;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return MOE_ERR_NO_DEVICE;
  if (hipSetDevice(device) != hipSuccess) return MOE_ERR_NO_DEVICE;
  moe_ctx *c = new moe_ctx;
  c->device = device;
  c->n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;

  c->budget = (inject & 2) ? 0 : budget_bytes;
  c->inject = inject;
  // the two-octet down kernels stage more than 64 KiB of LDS per workgroup
  const std::pair<const void *, int> big_lds[] = {{(const void *)k_down_ol2<6>, 6 * 4}};
  for (const auto &kb : big_lds)
    if (hipFuncSetAttribute(kb.first, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)(2 * octet_lds_bytes_z(kb.second))) != hipSuccess) {
      delete c;
      return MOE_ERR_NO_DEVICE;
    }
  // and the stacked-digit kernels (two 17 KiB chunk buffers, 34 KiB, and
  // down's router weights; set for uniformity)
  const std::pair<const void *, int> sk_kernels[] = {
      {(const void *)k_gate_up_sk<56>, MOE_SK_LDS_BYTES},   {(const void *)k_gate_up_sk<48>, MOE_SK_LDS_BYTES},
      {(const void *)k_gate_up_sk<32>, MOE_SK_LDS_BYTES},   {(const void *)k_gate_up_sk<16>, MOE_SK_LDS_BYTES},
      {(const void *)k_down_sk<24>, MOE_SK_DN_LDS_BYTES}, {(const void *)k_down_sk<16>, MOE_SK_DN_LDS_BYTES},
      {(const void *)k_down_sk<12>, MOE_SK_DN_LDS_BYTES}, {(const void *)k_down_sk<8>, MOE_SK_DN_LDS_BYTES}};
  for (const auto &kf : sk_kernels)
    if (hipFuncSetAttribute(kf.first, hipFuncAttributeMaxDynamicSharedMemorySize, kf.second) != hipSuccess) {
      delete c;
      return MOE_ERR_NO_DEVICE;
    }
  noalloc_setup(c);
  *out = c;
  return MOE_OK;
}

extern "C" void moe_ctx_destroy(moe_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  // graphs outlive the context only as empty handles: moe_graph_launch then
  // refuses them and moe_graph_destroy frees the handle
  while (!c->graphs.empty()) graph_detach(*c->graphs.begin());
  for (auto &kv : c->layers)
    for (dev_mat &m : kv.second.m)
      if (m.w) (void)hipFree(m.w);
  scratch_free(c->sc);
  if (c->pin) (void)hipHostFree(c->pin);
  if (c->tl) (void)hipFree(c->tl);
  for (auto &r : c->prof.pending) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (hipEvent_t e : c->prof.pool) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->calls.ev)
    if (e) (void)hipEventDestroy(e);
  delete c;
}

extern "C" const char *moe_ctx_last_error(const moe_ctx *c) { return c ? c->err.c_str() : ""; }

extern "C" const char *moe_status_str(moe_status s) {
  switch (s) {
    case MOE_OK: return "ok";
    case MOE_ERR_INVALID_ARG: return "invalid argument";
    case MOE_ERR_HIP: return "HIP runtime error";
    case MOE_ERR_OUT_OF_BUDGET: return "layer does not fit the residency budget";
    case MOE_ERR_UNSUPPORTED: return "unsupported shape";
    case MOE_ERR_NOT_RESIDENT: return "layer not resident";
    case MOE_ERR_NO_DEVICE: return "no usable gfx950 device";
    case MOE_ERR_INJECTED: return "injected failure";
    case MOE_ERR_FORMAT: return "model file unreadable or not an MXFP4 MoE layer";
  }
  return "unknown status";
}

extern "C" moe_status moe_device_memory(int device, uint64_t *free_bytes, uint64_t *total_bytes) {
  if (!free_bytes || !total_bytes) return MOE_ERR_INVALID_ARG;
  *free_bytes = *total_bytes = 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return MOE_ERR_NO_DEVICE;
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(device) != hipSuccess) return MOE_ERR_NO_DEVICE;
  size_t fr = 0, tot = 0;
  const hipError_t e = hipMemGetInfo(&fr, &tot);
  (void)hipSetDevice(prev);
  if (e != hipSuccess) return MOE_ERR_HIP;
  *free_bytes = fr;
  *total_bytes = tot;
  return MOE_OK;
}

extern "C" uint64_t moe_ctx_budget_left(const moe_ctx *c) {
  return c && c->budget > c->used ? c->budget - c->used : 0;
}

extern "C" moe_status moe_ctx_reserve(moe_ctx *c, const moe_layer_desc *d, int max_tokens) {
  if (!c || !desc_ok(d) || max_tokens <= 0) return fail(c, MOE_ERR_INVALID_ARG, "moe_ctx_reserve: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  return scratch_reserve(c, max_tokens, d->hidden, d->ffn, d->n_expert, d->n_used);
}

// ---------------------------------------------------------------------------
// residency

static moe_status layer_alloc(moe_ctx *c, int layer, const moe_layer_desc *d, dev_layer **out) {
  if (!desc_ok(d)) return fail(c, MOE_ERR_INVALID_ARG, "layer %d: bad descriptor", layer);
  if (c->layers.count(layer)) return fail(c, MOE_ERR_INVALID_ARG, "layer %d is already resident", layer);
  const uint64_t need = layer_bytes(d);
  if (c->used + need > c->budget || c->used + need < c->used)
    return fail(c, MOE_ERR_OUT_OF_BUDGET, "layer %d does not fit (%llu MB needed, %llu MB left); CPU fallback",
                layer, (unsigned long long)(need >> 20),
                (unsigned long long)((c->budget - c->used) >> 20));
  HIPC(c, hipSetDevice(c->device));
  dev_layer L;
  L.d = *d;
  L.n_mats = d->n_expert + d->has_shared;
  const int rows[3] = {d->ffn, d->ffn, d->hidden};
  const int kbs[3] = {d->hidden / 32, d->hidden / 32, d->ffn / 32};
  for (int t = 0; t < 3; t++) {
    L.m[t].rows = rows[t];
    L.m[t].kb = kbs[t];
    L.m[t].stride = mat_bytes(rows[t], kbs[t]);
    if (hipMalloc(&L.m[t].w, (size_t)L.n_mats * L.m[t].stride) != hipSuccess) {
      for (dev_mat &m : L.m)
        if (m.w) (void)hipFree(m.w);
      (void)hipGetLastError();
      return fail(c, MOE_ERR_OUT_OF_BUDGET, "layer %d: device allocation failed; CPU fallback", layer);
    }
  }
  L.bytes = need;
  c->used += need;
  auto it = c->layers.emplace(layer, L).first;
  *out = &it->second;
  return MOE_OK;
}

static void layer_drop(moe_ctx *c, int layer) {
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return;
  for (dev_mat &m : it->second.m)
    if (m.w) (void)hipFree(m.w);
  c->used -= it->second.bytes;
  c->layers.erase(it);
}

extern "C" moe_status moe_layer_upload(moe_ctx *c, int layer, const moe_layer_desc *d,
                                       const void *gate, const void *up, const void *down,
                                       const void *sh_gate, const void *sh_up, const void *sh_down) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!gate || !up || !down || (d && d->has_shared && (!sh_gate || !sh_up || !sh_down)))
    return fail(c, MOE_ERR_INVALID_ARG, "moe_layer_upload: missing tensor");
  dev_layer *L = nullptr;
  moe_status st = layer_alloc(c, layer, d, &L);
  if (st != MOE_OK) return st;
  // Stage whole expert matrices of 17-byte blocks through a bounded device
  // buffer (the layout interleaves the rows of an expert), repack on the device.
  size_t max_per_exp = 0;
  for (int t = 0; t < 3; t++) {
    const size_t pe = (size_t)L->m[t].rows * L->m[t].kb;
    max_per_exp = pe > max_per_exp ? pe : max_per_exp;
  }
  const size_t chunk_blocks = max_per_exp > ((size_t)1 << 22) ? max_per_exp : ((size_t)1 << 22);
  uint8_t *stage = nullptr;
  if (hipMalloc(&stage, chunk_blocks * 17) != hipSuccess) {
    layer_drop(c, layer);
    return fail(c, MOE_ERR_HIP, "moe_layer_upload: staging allocation failed");
  }
  const void *src[3][2] = {{gate, sh_gate}, {up, sh_up}, {down, sh_down}};
  for (int t = 0; t < 3 && st == MOE_OK; t++) {
    dev_mat &m = L->m[t];
    const size_t per_exp = (size_t)m.rows * m.kb;
    const size_t batch = chunk_blocks / per_exp;  // experts per staged copy (>= 1)
    for (int part = 0; part < 1 + d->has_shared && st == MOE_OK; part++) {
      const uint8_t *host = (const uint8_t *)src[t][part];
      const size_t n_exp = part == 0 ? (size_t)d->n_expert : 1;
      for (size_t e0 = 0; e0 < n_exp; e0 += batch) {
        const size_t ne = n_exp - e0 < batch ? n_exp - e0 : batch;
        const size_t n = ne * per_exp, off = e0 * per_exp;
        if (hipMemcpy(stage, host + off * 17, n * 17, hipMemcpyHostToDevice) != hipSuccess) {
          st = fail(c, MOE_ERR_HIP, "moe_layer_upload: host->device copy failed");
          break;
        }
        const size_t first = (part == 0 ? e0 : (size_t)d->n_expert);  // expert index of the batch's first matrix
        hipLaunchKernelGGL(k_repack_blocks, dim3(ceil_div((long)n, 256)), dim3(256), 0, 0, stage, (uint64_t)n,
                           (uint64_t)per_exp, m.stride, m.kb, m.w + first * m.stride);
      }
    }
  }
  if (st == MOE_OK && hipDeviceSynchronize() != hipSuccess) st = fail(c, MOE_ERR_HIP, "moe_layer_upload: repack failed");
  (void)hipFree(stage);
  if (st != MOE_OK) layer_drop(c, layer);
  return st;
}

// ---- GGUF ------------------------------------------------------------------

// Layer `layer` of an opened model: its shape and router keys into *info,
// pointers to the six expert tensors' bytes (the shared three NULL when the
// layer's shared expert is not one this library computes) into w[].
static moe_status gguf_layer(gguf::model &M, int layer, moe_gguf_layer *info, const uint8_t *w[6]) {
  memset(info, 0, sizeof(*info));
  for (int i = 0; i < 6; i++) w[i] = nullptr;
  std::string arch;
  if (!M.get_str("general.architecture", &arch) || arch.empty() || arch.size() >= sizeof(info->arch))
    return M.fail("general.architecture is missing"), MOE_ERR_FORMAT;
  memcpy(info->arch, arch.data(), arch.size());
  const std::string a = arch + ".";
  int64_t v;
  info->n_layer = M.get_int(a + "block_count", &v) && v >= 0 && v <= INT32_MAX ? (int32_t)v : -1;
  if (layer < 0 || (info->n_layer >= 0 && layer >= info->n_layer))
    return M.fail("layer " + std::to_string(layer) + " is out of range"), MOE_ERR_INVALID_ARG;
  const std::string blk = "blk." + std::to_string(layer) + ".";
  const char *names[6] = {"ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight",
                          "ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight"};
  const gguf::tensor *t[6];
  for (int i = 0; i < 6; i++) t[i] = M.find_tensor(blk + names[i]);
  for (int i = 0; i < 3; i++) {
    if (!t[i]) return M.fail("no tensor " + blk + names[i]), MOE_ERR_FORMAT;
    if (t[i]->type != gguf::GGML_TYPE_MXFP4 || t[i]->n_dims != 3)
      return M.fail(blk + names[i] + ": not a 3-d MXFP4 tensor (type " + std::to_string(t[i]->type) + ")"),
             MOE_ERR_FORMAT;
  }
  const uint64_t H = t[0]->ne[0], F = t[0]->ne[1], E = t[0]->ne[2];
  if (H == 0 || F == 0 || E == 0 || H % 32 || F % 32 || H > (1u << 20) || F > (1u << 20) || E > (1u << 16) ||
      t[1]->ne[0] != H || t[1]->ne[1] != F || t[1]->ne[2] != E || t[2]->ne[0] != F || t[2]->ne[1] != H ||
      t[2]->ne[2] != E)
    return M.fail(blk + "ffn_*_exps: dims do not form [H,F,E], [H,F,E], [F,H,E] with H, F multiples of 32"),
           MOE_ERR_FORMAT;
  if (!M.get_int(a + "expert_used_count", &v) || v < 1 || (uint64_t)v > E)
    return M.fail(a + "expert_used_count is missing or out of range"), MOE_ERR_FORMAT;
  const int64_t k = v;
  if (M.get_int(a + "expert_count", &v) && (uint64_t)v != E)
    return M.fail(a + "expert_count disagrees with the expert tensors"), MOE_ERR_FORMAT;
  if (M.get_int(a + "expert_feed_forward_length", &v) && (uint64_t)v != F)
    return M.fail(a + "expert_feed_forward_length disagrees with the expert tensors"), MOE_ERR_FORMAT;
  if (M.get_int(a + "embedding_length", &v) && (uint64_t)v != H)
    return M.fail(a + "embedding_length disagrees with the expert tensors"), MOE_ERR_FORMAT;
  float clamp = 0.0f;
  if (M.find(a + "swiglu_clamp_exp") && !M.get_f32_at(a + "swiglu_clamp_exp", (uint64_t)layer, &clamp))
    return M.fail(a + "swiglu_clamp_exp is not an f32 array covering the layer"), MOE_ERR_FORMAT;
  for (int i = 0; i < 3; i++)
    if (!(w[i] = M.data_of(*t[i]))) return MOE_ERR_FORMAT;
  // the shared expert, when it is one this library computes
  info->shared_type = t[3] ? (int32_t)t[3]->type : -1;
  float clamp_sh = 0.0f;
  const bool sh_clamp_ok = !M.find(a + "swiglu_clamp_shexp") ||
                           (M.get_f32_at(a + "swiglu_clamp_shexp", (uint64_t)layer, &clamp_sh));
  bool shared = t[3] && t[4] && t[5] && sh_clamp_ok && clamp_sh == clamp;
  for (int i = 3; i < 6 && shared; i++) {
    const uint64_t r0 = i == 5 ? F : H, r1 = i == 5 ? H : F;
    shared = t[i]->type == gguf::GGML_TYPE_MXFP4 && t[i]->n_dims == 2 && t[i]->ne[0] == r0 && t[i]->ne[1] == r1;
  }
  for (int i = 3; i < 6 && shared; i++)
    if (!(w[i] = M.data_of(*t[i]))) return MOE_ERR_FORMAT;
  if (!shared) w[3] = w[4] = w[5] = nullptr;
  info->desc.hidden = (int32_t)H;
  info->desc.ffn = (int32_t)F;
  info->desc.n_expert = (int32_t)E;
  info->desc.n_used = (int32_t)k;
  info->desc.has_shared = shared ? 1 : 0;
  info->desc.clamp = clamp;
  info->route_mode = -1;
  if (M.get_int(a + "expert_gating_func", &v))
    info->route_mode = v == 1 ? MOE_ROUTE_SOFTMAX : v == 2 ? MOE_ROUTE_SIGMOID : v == 4 ? MOE_ROUTE_SQRT_SOFTPLUS : -1;
  info->route_norm = M.get_int(a + "expert_weights_norm", &v) && v != 0 ? 1 : 0;
  info->route_scale = 1.0f;
  float sc;
  if (M.get_f32(a + "expert_weights_scale", &sc)) info->route_scale = sc;
  return MOE_OK;
}

extern "C" moe_status moe_gguf_read_layer(const char *path, int layer, moe_gguf_layer *info, char *err,
                                          size_t err_len) {
  if (err && err_len) err[0] = 0;
  if (!path || !info) return MOE_ERR_INVALID_ARG;
  gguf::model M;
  const uint8_t *w[6];
  const moe_status st = M.open(path) ? gguf_layer(M, layer, info, w) : MOE_ERR_FORMAT;
  if (st != MOE_OK && err && err_len) snprintf(err, err_len, "%s", M.err.c_str());
  return st;
}

extern "C" moe_status moe_layer_upload_gguf(moe_ctx *c, int layer, const char *path, int file_layer,
                                            moe_gguf_layer *info) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!path) return fail(c, MOE_ERR_INVALID_ARG, "moe_layer_upload_gguf: path is NULL");
  gguf::model M;
  moe_gguf_layer li;
  const uint8_t *w[6];
  const moe_status st = M.open(path) ? gguf_layer(M, file_layer, &li, w) : MOE_ERR_FORMAT;
  if (st != MOE_OK) return fail(c, st, "moe_layer_upload_gguf: %s", M.err.c_str());
  if (info) *info = li;
  return moe_layer_upload(c, layer, &li.desc, w[0], w[1], w[2], w[3], w[4], w[5]);
}

extern "C" moe_status moe_layer_generate(moe_ctx *c, int layer, const moe_layer_desc *d, uint64_t seed,
                                         int e_lo, int e_span) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (e_lo < 0 || e_span < 1 || e_lo + e_span > 256)
    return fail(c, MOE_ERR_INVALID_ARG, "moe_layer_generate: exponent range");
  dev_layer *L = nullptr;
  moe_status st = layer_alloc(c, layer, d, &L);
  if (st != MOE_OK) return st;
  for (int t = 0; t < 3; t++) {
    dev_mat &m = L->m[t];
    const size_t per_exp = (size_t)m.rows * m.kb;
    for (int e = 0; e < L->n_mats; e++) {
      const bool shared = e == d->n_expert;
      const int tensor = shared ? t + 3 : t;
      const int expert = shared ? 0 : e;
      const uint64_t id = ((uint64_t)(uint32_t)layer << 40) ^ ((uint64_t)(uint32_t)tensor << 32) ^
                          (uint64_t)(uint32_t)expert;
      const uint64_t key = host_mix64(seed ^ host_mix64(id));
      hipLaunchKernelGGL(k_generate_blocks, dim3(ceil_div((long)per_exp, 256)), dim3(256), 0, 0, key,
                         (uint64_t)per_exp, m.kb, (uint32_t)e_lo, (uint32_t)e_span, m.w + m.stride * e);
    }
  }
  if (hipDeviceSynchronize() != hipSuccess) {
    layer_drop(c, layer);
    return fail(c, MOE_ERR_HIP, "moe_layer_generate: kernel failed");
  }
  return MOE_OK;
}

extern "C" moe_status moe_layer_read_blocks(moe_ctx *c, int layer, int tensor, int expert, void *out) {
  if (!c || !out) return MOE_ERR_INVALID_ARG;
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident", layer);
  dev_layer &L = it->second;
  if (tensor < 0 || tensor > 2 || expert < 0 || expert >= L.n_mats)
    return fail(c, MOE_ERR_INVALID_ARG, "moe_layer_read_blocks: tensor/expert out of range");
  HIPC(c, hipSetDevice(c->device));
  dev_mat &m = L.m[tensor];
  const size_t nb = (size_t)m.rows * m.kb;
  uint8_t *tmp = nullptr;
  HIPC(c, hipMalloc(&tmp, nb * 17));
  hipLaunchKernelGGL(k_unpack_blocks, dim3(ceil_div((long)nb, 256)), dim3(256), 0, 0, m.w + m.stride * expert,
                     (uint64_t)nb, m.kb, tmp);
  hipError_t e = hipMemcpy(out, tmp, nb * 17, hipMemcpyDeviceToHost);
  (void)hipFree(tmp);
  if (e != hipSuccess) return fail(c, MOE_ERR_HIP, "moe_layer_read_blocks: copy failed");
  return MOE_OK;
}

extern "C" moe_status moe_layer_release(moe_ctx *c, int layer) {
  if (!c) return MOE_ERR_INVALID_ARG;
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident", layer);
  if (it->second.graph_refs > 0)
    return fail(c, MOE_ERR_INVALID_ARG, "layer %d is read by %d captured graph(s); destroy them before releasing it",
                layer, it->second.graph_refs);
  HIPC(c, hipSetDevice(c->device));
  HIPC(c, hipDeviceSynchronize());
  layer_drop(c, layer);
  return MOE_OK;
}

extern "C" moe_status moe_layer_bytes(const moe_ctx *c, int layer, uint64_t *bytes) {
  if (!c || !bytes) return MOE_ERR_INVALID_ARG;
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return MOE_ERR_NOT_RESIDENT;
  *bytes = it->second.bytes;
  return MOE_OK;
}

// ---------------------------------------------------------------------------
// per call

extern "C" moe_status moe_route(moe_ctx *c, const float *logits, const float *bias, int T, int E, int k,
                                int mode, int norm, float scale, int32_t *ids, float *wts, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!logits || !ids || !wts || T <= 0 || E <= 0 || E > MOE_ROUTE_MAX_E || k <= 0 || k > 64 || k > E ||
      mode < 0 || mode > 2)
    return fail(c, MOE_ERR_INVALID_ARG, "moe_route: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  {
    prof_scope ps(c, K_ROUTE, (hipStream_t)stream, true);
    hipLaunchKernelGGL(k_route, dim3(T), dim3(256), 0, (hipStream_t)stream, logits, bias, E, k, mode, norm,
                       scale, ids, wts);
  }
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

extern "C" moe_status moe_router_logits(moe_ctx *c, const float *w, const float *x, int T, int E, int H,
                                        int w_type, float *logits, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!w || !x || !logits || T <= 0 || E <= 0 || H <= 0 || H % 4 || ((uintptr_t)w | (uintptr_t)x) % 16 ||
      (w_type != MOE_GGML_F32 && w_type != MOE_GGML_F16 && w_type != MOE_GGML_BF16))
    return fail(c, MOE_ERR_INVALID_ARG, "moe_router_logits: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  const dim3 grid(ceil_div(E, 4), ceil_div(T, 4));
  if (w_type == MOE_GGML_F16)
    hipLaunchKernelGGL(k_router_logits<1>, grid, dim3(256), 0, (hipStream_t)stream, w, x, T, E, H, logits);
  else if (w_type == MOE_GGML_BF16)
    hipLaunchKernelGGL(k_router_logits<2>, grid, dim3(256), 0, (hipStream_t)stream, w, x, T, E, H, logits);
  else
    hipLaunchKernelGGL(k_router_logits<0>, grid, dim3(256), 0, (hipStream_t)stream, w, x, T, E, H, logits);
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

extern "C" moe_status moe_group(moe_ctx *c, const int32_t *ids, int T, int k, int E, int32_t *counts,
                                int32_t *offsets, int32_t *perm, int32_t *inv, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!ids || !counts || !offsets || !perm || T <= 0 || k <= 0 || E <= 0 || E > MOE_GROUP_MAX_E ||
      (long)T * k > MOE_GROUP_MAX_PAIRS)
    return fail(c, MOE_ERR_INVALID_ARG, "moe_group: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  {
    prof_scope ps(c, K_GROUP, (hipStream_t)stream, true);
    if ((long)T * k <= MOE_GF_PAIRS)
      hipLaunchKernelGGL(k_group_few, dim3(1), dim3(256), 0, (hipStream_t)stream, ids, T * k, E, T, 0, 1,
                         counts, offsets, perm, inv, (int32_t *)nullptr, (const float *)nullptr, 0,
                         (uint32_t *)nullptr, (float *)nullptr, 0, (int32_t *)nullptr);
    else
      hipLaunchKernelGGL(k_group, dim3(1), dim3(1024), 0, (hipStream_t)stream, ids, T * k, E, T, 0, 1, counts,
                         offsets, perm, inv, (int32_t *)nullptr, (const float *)nullptr, 0, (uint32_t *)nullptr,
                         (float *)nullptr, 0, (int32_t *)nullptr);
  }
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

// decode gate/up launch (k_gate_up with one token, columns = slots)
static void launch_gate_up_decode(dim3 g, hipStream_t st, const dev_layer &L, const float *x, const int32_t *ids,
                                  int shared, uint32_t *hq, float *hd, float *htap) {
  const moe_layer_desc &d = L.d;
  hipLaunchKernelGGL(k_gate_up<1>, g, dim3(64 * 2 * MOE_GU_KS), gate_up_lds_bytes(d.hidden, 1), st, L.m[T_GATE].w,
                     L.m[T_UP].w, x, 0, ids, (const int32_t *)nullptr, (const int32_t *)nullptr,
                     (const int32_t *)nullptr, d.n_used, d.n_expert, shared, 1, d.ffn, d.hidden, d.clamp, hq, hd,
                     htap);
}

static moe_status forward_grouped(moe_ctx *c, dev_layer &L, work_bufs &s, const float *x, const int32_t *ids,
                                  const float *wts, int T, float *out, uint32_t flags, hipStream_t st);

// The decode chain for T == 1, two launches: gate/up per (32-row unit, slot)
// with SwiGLU and Q8_0 of h, then down per 16-row tile of H with one wave per
// slot, the router weights and the slot-order combine.  s: the per-call
// buffers (the context's own, or the no-allocation entry point's).
static moe_status forward_decode(moe_ctx *c, dev_layer &L, work_bufs &s, const float *x, const int32_t *ids,
                                 const float *wts, float *out, uint32_t flags, hipStream_t st) {
  const moe_layer_desc &d = L.d;
  const int k = d.n_used, E = d.n_expert, H = d.hidden, F = d.ffn;
  const bool per_slot = flags & MOE_FWD_PER_SLOT;
  const int shared = (d.has_shared && !per_slot && !(flags & MOE_FWD_NO_SHARED)) ? 1 : 0;
  const int S = k + shared;
  float *htap = c->taps ? s.htap : nullptr;
  const size_t lds1 = gate_up_lds_bytes(H, 1), lds2 = down_dec_lds_bytes(F, S);
  if (S > 16 || lds1 > 65536 || lds2 > 65536)
    return forward_grouped(c, L, s, x, ids, wts, 1, out, flags, st);  // the grouped chain takes any shape
  // the debug timeline (eager calls only): gate/up's records, then down's
  const size_t n_dn = (size_t)(H / MOE_TILE) * S;
  unsigned long long *tl = c->tl && !c->capturing && n_dn <= MOE_TL_RECORDS ? c->tl : nullptr;
  c->tl_gu = 0;
  c->tl_dn = 0;
  {
    prof_scope pg(c, K_GU_DECODE, st, s.timed);
    // the balanced kernels run one workgroup per CU: for shapes too small to
    // fill half of the CUs that way (C1), the (unit, slot) grid spreads wider
    const long n_tasks = (long)S * (F / MOE_UNIT) * 4;
    const bool wide = n_tasks / MOE_BAL_WAVES >= c->n_cu / 2;
    if (!wide) {
      launch_gate_up_decode(dim3(F / MOE_UNIT, S), st, L, x, ids, shared, s.hq, s.hd, htap);
    } else if (n_tasks % MOE_BAL_WAVES == 0 && (n_tasks / MOE_BAL_WAVES) % 4 == 0 &&
               gate_up_bal2_lds_bytes(H) <= 65536) {
      const size_t n_gu = (size_t)n_tasks;  // 9 waves per workgroup, one task each
      unsigned long long *tg = tl && n_gu + n_dn <= MOE_TL_RECORDS ? tl : nullptr;
      hipLaunchKernelGGL(tg ? k_gate_up_bal2<true> : k_gate_up_bal2<false>, dim3(n_tasks / MOE_BAL_WAVES),
                         dim3(64 * MOE_BAL_WAVES), gate_up_bal2_lds_bytes(H), st, L.m[T_GATE].w, L.m[T_UP].w, x, ids, k,
                         E, S, F, H, d.clamp, s.part, s.tick, s.hq, s.hd, htap, tg);
      if (tg) c->tl_gu = n_gu;
    } else if (gate_up_bal_lds_bytes(H) <= 65536) {
      const int n_wg = ceil_div((long)S * (F / MOE_UNIT) * 4, MOE_BAL_WAVES);
      hipLaunchKernelGGL(k_gate_up_bal, dim3(n_wg), dim3(64 * MOE_BAL_WAVES), gate_up_bal_lds_bytes(H), st,
                         L.m[T_GATE].w, L.m[T_UP].w, x, ids, k, E, S, F, H, d.clamp, s.part, s.tick, s.hq, s.hd,
                         htap);
    } else {
      launch_gate_up_decode(dim3(F / MOE_UNIT, S), st, L, x, ids, shared, s.hq, s.hd, htap);
    }
  }
  s.h_rows = htap ? (size_t)S : 0;
  s.last_F = F;
  {
    prof_scope pd(c, K_DOWN_DECODE, st, s.timed);
    hipLaunchKernelGGL(tl ? k_down_dec<true> : k_down_dec<false>, dim3(H / MOE_TILE), dim3(64 * S), lds2, st,
                       L.m[T_DOWN].w, s.hq, s.hd, ids, wts, k, E, S, F, H, per_slot ? 1 : 0, out,
                       tl ? tl + 3 * c->tl_gu : nullptr);
    if (tl) c->tl_dn = n_dn;
  }
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

// The grouped chain runs token pairs on the 16x16x128 MFMA for T <= 4
// (items of at most 4 rows: NPMAX = 2 pairs), token octets on the 32x32x64
// MFMA above that (items of at most 8 rows).
static bool use_octets(int T) { return T > 4; }

static moe_status forward_grouped(moe_ctx *c, dev_layer &L, work_bufs &s, const float *x, const int32_t *ids,
                                  const float *wts, int T, float *out, uint32_t flags, hipStream_t st) {
  const moe_layer_desc &d = L.d;
  const int k = d.n_used, E = d.n_expert, P = T * k, H = d.hidden, F = d.ffn;
  const bool per_slot = flags & MOE_FWD_PER_SLOT;
  const int shared = (d.has_shared && !per_slot && !(flags & MOE_FWD_NO_SHARED)) ? 1 : 0;
  if (P > MOE_GROUP_MAX_PAIRS || E > MOE_GROUP_MAX_E)
    return fail(c, MOE_ERR_UNSUPPORTED, "grouped: more than %d pairs or %d experts", MOE_GROUP_MAX_PAIRS,
                MOE_GROUP_MAX_E);
  const bool oct = use_octets(T);
  const int BT = oct ? 8 : 4;
  // a few tokens (the pairs path): down per 16-row tile of H with the slot
  // combine in the same launch (k_down_few)
  const bool few = !oct && T <= MOE_DF_TMAX && k + 1 <= MOE_DF_SMAX && H % MOE_DF_ROWS == 0;
  int32_t *counts = s.grp, *offsets = counts + E, *perm = offsets + E + 1, *inv = perm + P, *items = inv + P;
  // where the shape has an instance and the batch averages 2 pairs per
  // expert or more, gate/up and down run on a second item list with B staged
  // in LDS: items of up to 32 rows on the stacked-digit kernels
  // (k_gate_up_sk, H = 128 * {16, 32, 48, 56}; k_down_sk, F = 128 * {8, 12,
  // 16, 24}), else items of up to 16 rows on the octet kernels (k_gate_up_ol /
  // k_down_ol2, H = 128 * {16, 32, 56}); below 2 pairs per expert most items
  // hold one octet and the 8-row list with B from global memory is used
  int32_t *items16 = items + group_list_words(T, k, E);
  const bool dense = oct && P >= 2 * E && (F / MOE_UNIT) % 4 == 0;
  const bool sk = dense && (H == 128 * 56 || H == 128 * 48 || H == 128 * 32 || H == 128 * 16) &&
                  (F == 128 * 8 || F == 128 * 12 || F == 128 * 16 || F == 128 * 24) && H % 256 == 0;
  const bool o2 = sk || (dense && (H == 128 * 56 || H == 128 * 32 || H == 128 * 16));
  const int BT2 = sk ? 32 : 16;
  float *htap = c->taps ? s.htap : nullptr;
  const int n_xblocks = T * (H / MOE_QK);
  {
    prof_scope pgr(c, K_GROUP, st, s.timed);
    // up to 128 pairs: the one-wave ballot grouping (no per-expert counts: nothing downstream reads them)
    if (P <= MOE_GF_PAIRS)
      hipLaunchKernelGGL(k_group_few, dim3(1 + ceil_div(n_xblocks, MOE_GF_QBLOCKS)), dim3(256), 0, st,
                         ids, P, E, T, shared, BT, (int32_t *)nullptr, (int32_t *)nullptr, perm, inv, items, x,
                         n_xblocks, s.xq, s.xd, BT2, (o2 || sk) ? items16 : (int32_t *)nullptr);
    else
      hipLaunchKernelGGL(k_group, dim3(1 + ceil_div(n_xblocks, MOE_GROUP_QBLOCKS)), dim3(1024), 0, st, ids, P, E, T,
                         shared, BT, counts, offsets, perm, inv, items, x, n_xblocks, s.xq, s.xd, BT2,
                         (o2 || sk) ? items16 : (int32_t *)nullptr);
  }
  const int cap = group_item_cap(T, k, E, BT);
  {
    prof_scope pg(c, K_GU_GROUPED, st, s.timed);
#define MOE_GU_ARGS L.m[T_GATE].w, L.m[T_UP].w, s.xq, s.xd, items, perm, k, T, F, H, d.clamp, s.hq, s.hd, htap
#define MOE_GU_ARGS16 L.m[T_GATE].w, L.m[T_UP].w, s.xq, s.xd, items16, perm, k, T, F, H, d.clamp, s.hq, s.hd, htap
    const dim3 g16(F / (4 * MOE_UNIT), group_item_cap(T, k, E, BT2));  // 4 units of F per workgroup
    if (sk && H == 128 * 56) hipLaunchKernelGGL(k_gate_up_sk<56>, g16, dim3(512), MOE_SK_LDS_BYTES, st, MOE_GU_ARGS16);
    else if (sk && H == 128 * 48) hipLaunchKernelGGL(k_gate_up_sk<48>, g16, dim3(512), MOE_SK_LDS_BYTES, st, MOE_GU_ARGS16);
    else if (sk && H == 128 * 32) hipLaunchKernelGGL(k_gate_up_sk<32>, g16, dim3(512), MOE_SK_LDS_BYTES, st, MOE_GU_ARGS16);
    else if (sk && H == 128 * 16) hipLaunchKernelGGL(k_gate_up_sk<16>, g16, dim3(512), MOE_SK_LDS_BYTES, st, MOE_GU_ARGS16);
    else if (o2 && H == 128 * 56) hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gate_up_ol<56, 4>), g16, dim3(512), 0, st, MOE_GU_ARGS16);
    else if (o2 && H == 128 * 32) hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gate_up_ol<32, 4>), g16, dim3(512), 0, st, MOE_GU_ARGS16);
    else if (o2 && H == 128 * 16) hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gate_up_ol<16, 4>), g16, dim3(512), 0, st, MOE_GU_ARGS16);
    else if (oct) hipLaunchKernelGGL(k_gate_up_o, dim3(F / (2 * MOE_UNIT), cap), dim3(256), 0, st, MOE_GU_ARGS);
    else hipLaunchKernelGGL(k_gate_up_g<2>, dim3(F / MOE_UNIT, cap), dim3(256), 0, st, MOE_GU_ARGS);
#undef MOE_GU_ARGS
#undef MOE_GU_ARGS16
  }
  s.h_rows = htap ? (size_t)P + (shared ? T : 0) : 0;
  s.last_F = F;
  {
    prof_scope pd(c, K_DOWN_GROUPED, st, s.timed);
#define MOE_DN_ARGS L.m[T_DOWN].w, s.hq, s.hd, P + T, items, perm, wts, F, H, s.y
    const dim3 gdo(H / 128, cap);
    const size_t lo = octet_lds_bytes(F / MOE_QK), lo2 = 2 * octet_lds_bytes_z(F / MOE_QK);
    // two octets per wave on the 16-row items where that list exists and two
    // workgroups' LDS (2 x 2 staged octets) fit a CU (F = 768; the stacked
    // kernels take F = 1024, 1536, 2048 and 3072)
    const dim3 gdo2(H / (32 * MOE_DOL2_WAVES), group_item_cap(T, k, E, BT2));
    const bool dn2 = o2 && !sk && H % (32 * MOE_DOL2_WAVES) == 0;
    const dim3 b2(64 * MOE_DOL2_WAVES);
#define MOE_DN_ARGS16 L.m[T_DOWN].w, s.hq, s.hd, P + T, items16, perm, wts, F, H, s.y
    if (sk && F == 128 * 16) hipLaunchKernelGGL(k_down_sk<16>, gdo2, b2, MOE_SK_DN_LDS_BYTES, st, MOE_DN_ARGS16);
    else if (sk && F == 128 * 24) hipLaunchKernelGGL(k_down_sk<24>, gdo2, b2, MOE_SK_DN_LDS_BYTES, st, MOE_DN_ARGS16);
    else if (sk && F == 128 * 12) hipLaunchKernelGGL(k_down_sk<12>, gdo2, b2, MOE_SK_DN_LDS_BYTES, st, MOE_DN_ARGS16);
    else if (sk && F == 128 * 8) hipLaunchKernelGGL(k_down_sk<8>, gdo2, b2, MOE_SK_DN_LDS_BYTES, st, MOE_DN_ARGS16);
    else if (dn2 && F == 128 * 6) hipLaunchKernelGGL(k_down_ol2<6>, gdo2, b2, lo2, st, MOE_DN_ARGS16);
    else if (oct && F == 128 * 16) hipLaunchKernelGGL(k_down_ol<16>, gdo, dim3(256), lo, st, MOE_DN_ARGS);
    else if (oct && F == 128 * 6) hipLaunchKernelGGL(k_down_ol<6>, gdo, dim3(256), lo, st, MOE_DN_ARGS);
    else if (oct && F == 128 * 8) hipLaunchKernelGGL(k_down_ol<8>, gdo, dim3(256), lo, st, MOE_DN_ARGS);
    else if (oct && F == 128 * 28) hipLaunchKernelGGL(k_down_ol<28>, gdo, dim3(256), lo, st, MOE_DN_ARGS);
    else if (oct) hipLaunchKernelGGL(k_down_o, gdo, dim3(256), 0, st, MOE_DN_ARGS);
    else if (few)
      hipLaunchKernelGGL(k_down_few<2>, dim3(H / MOE_DF_ROWS), dim3(64 * MOE_DF_WAVES), 0, st, L.m[T_DOWN].w, s.hq,
                         s.hd, P + T, items, perm, wts, T, k, F, H, shared, per_slot ? 1 : 0, out);
    else hipLaunchKernelGGL(k_down_g<2>, dim3(ceil_div(H / (2 * MOE_TILE), MOE_DG_WAVES), cap),
                            dim3(64 * MOE_DG_WAVES), 0, st, MOE_DN_ARGS);
#undef MOE_DN_ARGS
#undef MOE_DN_ARGS16
  }
  if (few) {  // k_down_few wrote out
    HIPC(c, hipGetLastError());
    return MOE_OK;
  }
  {
    prof_scope pc(c, K_COMBINE, st, s.timed);
    if ((reinterpret_cast<uintptr_t>(out) & 15) == 0)  // float4 stores
      hipLaunchKernelGGL(k_combine4, dim3(ceil_div((long)T * (H / 4), 256)), dim3(256), 0, st, s.y, inv, T, k, H,
                         shared, per_slot ? 1 : 0, out);
    else
      hipLaunchKernelGGL(k_combine, dim3(ceil_div((long)T * H, 256)), dim3(256), 0, st, s.y, inv, T, k, H, shared,
                         per_slot ? 1 : 0, out);
  }
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

extern "C" moe_status moe_forward(moe_ctx *c, int layer, const float *x, const int32_t *ids, const float *wts,
                                  int T, float *out, uint32_t flags, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (c->inject & 1) return fail(c, MOE_ERR_INJECTED, "forward failure injected by MOE_BLOCK_INJECT");
  if (!x || !ids || !wts || !out || T <= 0) return fail(c, MOE_ERR_INVALID_ARG, "moe_forward: bad arguments");
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident; CPU fallback", layer);
  dev_layer &L = it->second;
  if (!c->capturing) HIPC(c, hipSetDevice(c->device));
  moe_status st = scratch_reserve(c, T, L.d.hidden, L.d.ffn, L.d.n_expert, L.d.n_used);
  if (st != MOE_OK) return st;
  if (T == 1) return forward_decode(c, L, c->sc, x, ids, wts, out, flags, (hipStream_t)stream);
  return forward_grouped(c, L, c->sc, x, ids, wts, T, out, flags, (hipStream_t)stream);
}

extern "C" moe_status moe_forward_noalloc(moe_ctx *c, int layer, const float *x, const int32_t *ids,
                                          const float *wts, int T, float *out, uint32_t flags, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (c->inject & 1) return fail(c, MOE_ERR_INJECTED, "forward failure injected by MOE_BLOCK_INJECT");
  if (!x || !ids || !wts || !out || T <= 0) return fail(c, MOE_ERR_INVALID_ARG, "moe_forward_noalloc: bad arguments");
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident; CPU fallback", layer);
  if (!c->noalloc) return fail(c, MOE_ERR_HIP, "moe_forward_noalloc: %s", c->noalloc_err.c_str());
  dev_layer &L = it->second;
  const moe_layer_desc &d = L.d;
  if ((long)T * d.n_used > MOE_GROUP_MAX_PAIRS)
    return fail(c, MOE_ERR_INVALID_ARG, "moe_forward_noalloc: more than %d (token, slot) pairs", MOE_GROUP_MAX_PAIRS);
  work_bufs s;
  const size_t need = noalloc_layout(c->noalloc, T, d.hidden, d.ffn, d.n_expert, d.n_used, s);
  if (!s.hq)
    return fail(c, MOE_ERR_INVALID_ARG,
                "moe_forward_noalloc: T=%d on this layer needs %zu bytes of scratch, more than the %zu the "
                "library holds (MOE_NOALLOC_SCRATCH_BYTES); use moe_forward",
                T, need, (size_t)MOE_NOALLOC_SCRATCH_BYTES);
  if (!c->capturing) HIPC(c, hipSetDevice(c->device));
  if (T == 1) return forward_decode(c, L, s, x, ids, wts, out, flags, (hipStream_t)stream);
  return forward_grouped(c, L, s, x, ids, wts, T, out, flags, (hipStream_t)stream);
}

// Device phases of one host-boundary call, from events on the null stream
// (recorded only while moe_prof_enable is on).
struct host_phases {
  bool timed = false;
  float upload_ms = 0, compute_ms = 0, read_ms = 0;
};

static moe_status forward_host_impl(moe_ctx *c, int layer, const float *x, const int32_t *ids, const float *wts,
                                    int T, float *out, uint32_t flags, host_phases &ph);

extern "C" moe_status moe_forward_host(moe_ctx *c, int layer, const float *x, const int32_t *ids,
                                       const float *wts, int T, float *out, uint32_t flags) {
  if (!c) return MOE_ERR_INVALID_ARG;
  const auto t0 = std::chrono::steady_clock::now();
  host_phases ph;
  const moe_status st = forward_host_impl(c, layer, x, ids, wts, T, out, flags, ph);
  call_state &cs = c->calls;
  if (st != MOE_OK) {
    cs.refusals++;
    return st;
  }
  // distinct routed experts of the call: the expert matrices it read
  const int k = c->layers[layer].d.n_used, E = c->layers[layer].d.n_expert;
  std::vector<uint64_t> seen(((size_t)E + 63) / 64, 0);
  uint32_t distinct = 0;
  for (long i = 0; i < (long)T * k; i++) {
    const int e = ids[i];
    if (e < 0 || e >= E) continue;
    if (!(seen[e >> 6] >> (e & 63) & 1)) {
      seen[e >> 6] |= 1ull << (e & 63);
      distinct++;
    }
  }
  const double total = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
  cs.calls++;
  cs.expert_loads += distinct;
  cs.total_us += total;
  cs.last.last_total_us = total;
  cs.last.last_experts = distinct;
  cs.last.last_tokens = (uint32_t)T;
  cs.last.last_timed = ph.timed ? 1 : 0;
  cs.last.last_upload_us = ph.timed ? 1e3 * ph.upload_ms : 0.0;
  cs.last.last_compute_us = ph.timed ? 1e3 * ph.compute_ms : 0.0;
  cs.last.last_read_us = ph.timed ? 1e3 * ph.read_ms : 0.0;
  if (ph.timed) {
    cs.timed++;
    cs.upload_us += cs.last.last_upload_us;
    cs.compute_us += cs.last.last_compute_us;
    cs.read_us += cs.last.last_read_us;
  }
  return MOE_OK;
}

extern "C" moe_status moe_call_stats_read(moe_ctx *c, moe_call_stats *out, int reset) {
  if (!c || !out) return MOE_ERR_INVALID_ARG;
  call_state &cs = c->calls;
  *out = cs.last;
  out->calls = cs.calls;
  out->refusals = cs.refusals;
  out->expert_loads = cs.expert_loads;
  out->timed_calls = cs.timed;
  out->upload_us = cs.upload_us;
  out->compute_us = cs.compute_us;
  out->read_us = cs.read_us;
  out->total_us = cs.total_us;
  if (reset) {
    cs.calls = cs.refusals = cs.expert_loads = cs.timed = 0;
    cs.upload_us = cs.compute_us = cs.read_us = cs.total_us = 0;
  }
  return MOE_OK;
}

static moe_status forward_host_impl(moe_ctx *c, int layer, const float *x, const int32_t *ids, const float *wts,
                                    int T, float *out, uint32_t flags, host_phases &ph) {
  if (!x || !ids || !wts || !out || T <= 0) return fail(c, MOE_ERR_INVALID_ARG, "moe_forward_host: bad arguments");
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident; CPU fallback", layer);
  const moe_layer_desc &d = it->second.d;
  HIPC(c, hipSetDevice(c->device));
  moe_status st = scratch_reserve(c, T, d.hidden, d.ffn, d.n_expert, d.n_used);
  if (st != MOE_OK) return st;
  work_bufs &s = c->sc;
  const size_t P = (size_t)T * d.n_used;
  const size_t n_out = (flags & MOE_FWD_PER_SLOT) ? P * d.hidden : (size_t)T * d.hidden;
  // the caller's buffers are pageable: stage them through one pinned buffer in
  // the device layout of the inputs (host memcpy, then one asynchronous copy
  // in and one out), cheaper than a staged copy per array
  const size_t bx = (size_t)T * d.hidden * 4, bi = P * 4, bo = n_out * 4, bin = s.in_x + bx;
  const size_t need = ((bin + 255) & ~(size_t)255) + bo;
  if (c->pin_bytes < need) {
    if (c->pin) (void)hipHostFree(c->pin);
    c->pin = nullptr;
    c->pin_bytes = 0;
    HIPC(c, hipHostMalloc((void **)&c->pin, need, hipHostMallocDefault));
    c->pin_bytes = need;
  }
  uint8_t *pin_out = c->pin + ((bin + 255) & ~(size_t)255);
  memcpy(c->pin, ids, bi);
  memcpy(c->pin + s.in_wts, wts, bi);
  memcpy(c->pin + s.in_x, x, bx);
  hipEvent_t *ev = c->calls.ev;
  if (c->prof.on && !ev[0]) {
    for (int i = 0; i < 4; i++) HIPC(c, hipEventCreate(&ev[i]));
  }
  const bool timed = c->prof.on;
  if (timed) HIPC(c, hipEventRecord(ev[0], nullptr));
  HIPC(c, hipMemcpyAsync(s.ids_in, c->pin, bin, hipMemcpyHostToDevice, nullptr));
  if (timed) HIPC(c, hipEventRecord(ev[1], nullptr));
  st = moe_forward(c, layer, s.x_in, s.ids_in, s.wts_in, T, s.out_buf, flags, nullptr);
  if (st != MOE_OK) {
    (void)hipStreamSynchronize(nullptr);  // the staging copies finish before the next call reuses the buffer
    return st;
  }
  if (timed) HIPC(c, hipEventRecord(ev[2], nullptr));
  HIPC(c, hipMemcpyAsync(pin_out, s.out_buf, bo, hipMemcpyDeviceToHost, nullptr));
  if (timed) HIPC(c, hipEventRecord(ev[3], nullptr));
  HIPC(c, hipStreamSynchronize(nullptr));
  memcpy(out, pin_out, bo);
  if (timed) {
    HIPC(c, hipEventElapsedTime(&ph.upload_ms, ev[0], ev[1]));
    HIPC(c, hipEventElapsedTime(&ph.compute_ms, ev[1], ev[2]));
    HIPC(c, hipEventElapsedTime(&ph.read_ms, ev[2], ev[3]));
    ph.timed = true;
  }
  return MOE_OK;
}

extern "C" moe_status moe_route_forward(moe_ctx *c, int layer, const float *x, const float *logits,
                                        const float *bias, int T, int mode, int norm, float scale, int32_t *ids,
                                        float *wts, float *out, uint32_t flags, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident; CPU fallback", layer);
  const moe_layer_desc &d = it->second.d;
  moe_status st = moe_route(c, logits, bias, T, d.n_expert, d.n_used, mode, norm, scale, ids, wts, stream);
  if (st != MOE_OK) return st;
  return moe_forward(c, layer, x, ids, wts, T, out, flags, stream);
}

// ---------------------------------------------------------------------------
// graphs

extern "C" moe_status moe_graph_capture(moe_ctx *c, int n_layers, const int *layers, const float *const *x,
                                        const int32_t *const *ids, const float *const *wts, float *const *out,
                                        int T, uint32_t flags, moe_graph **g) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!g || n_layers <= 0 || !layers || !x || !ids || !wts || !out || T <= 0)
    return fail(c, MOE_ERR_INVALID_ARG, "moe_graph_capture: bad arguments");
  *g = nullptr;
  for (int i = 0; i < n_layers; i++) {
    auto it = c->layers.find(layers[i]);
    if (it == c->layers.end()) return fail(c, MOE_ERR_NOT_RESIDENT, "layer %d not resident", layers[i]);
    const moe_layer_desc &d = it->second.d;
    const work_bufs &s = c->sc;
    if (!s.hq || T > s.T || d.hidden > s.H || d.ffn > s.F || d.n_expert > s.E || d.n_used > s.k)
      return fail(c, MOE_ERR_INVALID_ARG, "moe_graph_capture: call moe_ctx_reserve for this shape first");
  }
  HIPC(c, hipSetDevice(c->device));
  HIPC(c, hipDeviceSynchronize());
  hipStream_t st;
  HIPC(c, hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  moe_status res = MOE_OK;
  if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    (void)hipStreamDestroy(st);
    return fail(c, MOE_ERR_HIP, "hipStreamBeginCapture failed");
  }
  c->capturing = true;
  for (int i = 0; i < n_layers && res == MOE_OK; i++)
    res = moe_forward(c, layers[i], x[i], ids[i], wts[i], T, out[i], flags, st);
  c->capturing = false;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(st, &graph);
  (void)hipStreamDestroy(st);
  if (res != MOE_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return res;
  }
  if (e != hipSuccess || !graph) return fail(c, MOE_ERR_HIP, "hipStreamEndCapture failed");
  hipGraphExec_t exec = nullptr;
  if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return fail(c, MOE_ERR_HIP, "hipGraphInstantiate failed");
  }
  moe_graph *mg = new moe_graph;
  mg->ctx = c;
  mg->graph = graph;
  mg->exec = exec;
  std::set<int> distinct(layers, layers + n_layers);
  mg->layers.assign(distinct.begin(), distinct.end());
  for (int l : mg->layers) c->layers[l].graph_refs++;
  c->graphs.insert(mg);
  *g = mg;
  return MOE_OK;
}

extern "C" moe_status moe_graph_launch(moe_graph *g, void *stream) {
  if (!g || !g->ctx || !g->exec) return MOE_ERR_INVALID_ARG;  // a graph whose context was destroyed
  HIPC(g->ctx, hipGraphLaunch(g->exec, (hipStream_t)stream));
  return MOE_OK;
}

extern "C" void moe_graph_destroy(moe_graph *g) {
  if (!g) return;
  graph_detach(g);
  delete g;
}

// ---------------------------------------------------------------------------
// profiling

extern "C" moe_status moe_prof_enable(moe_ctx *c, int on) {
  if (!c) return MOE_ERR_INVALID_ARG;
  c->prof.on = on != 0;
  return MOE_OK;
}

extern "C" moe_status moe_prof_read(moe_ctx *c, moe_kernel_stat *stats, int cap, int *n, int reset) {
  if (!c || !n || cap < 0 || (cap > 0 && !stats)) return fail(c, MOE_ERR_INVALID_ARG, "moe_prof_read: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  prof_state &p = c->prof;
  moe_status st = MOE_OK;
  for (auto &r : p.pending) {
    float ms = 0.0f;
    if (st == MOE_OK && (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess))
      st = fail(c, MOE_ERR_HIP, "moe_prof_read: event query failed");
    if (st == MOE_OK) {
      p.launches[r.kid] += 1;
      p.total_us[r.kid] += 1000.0 * (double)ms;
    }
    p.pool.push_back(r.a);
    p.pool.push_back(r.b);
  }
  p.pending.clear();
  int m = 0;
  for (int k = 0; k < K_COUNT; k++) {
    if (!p.launches[k]) continue;
    if (m < cap) {
      stats[m].name = kernel_names[k];
      stats[m].launches = p.launches[k];
      stats[m].total_us = p.total_us[k];
    }
    m++;
  }
  *n = m;
  if (reset) {
    for (int k = 0; k < K_COUNT; k++) {
      p.launches[k] = 0;
      p.total_us[k] = 0.0;
    }
  }
  return st;
}

// ---------------------------------------------------------------------------
// test hooks

extern "C" moe_status moe_debug_set_taps(moe_ctx *c, int on) {
  if (!c) return MOE_ERR_INVALID_ARG;
  c->taps = on != 0;
  return MOE_OK;
}

extern "C" moe_status moe_debug_set_timeline(moe_ctx *c, int on) {
  if (!c) return MOE_ERR_INVALID_ARG;
  HIPC(c, hipSetDevice(c->device));
  if (on && !c->tl) {
    HIPC(c, hipMalloc(&c->tl, (size_t)MOE_TL_RECORDS * 3 * 8));
  } else if (!on && c->tl) {
    HIPC(c, hipDeviceSynchronize());
    HIPC(c, hipFree(c->tl));
    c->tl = nullptr;
  }
  c->tl_gu = c->tl_dn = 0;
  return MOE_OK;
}

extern "C" moe_status moe_debug_read_timeline(moe_ctx *c, uint64_t *stamps, size_t cap, size_t *n_gate_up,
                                              size_t *n_down) {
  if (!c || !n_gate_up || !n_down || (cap && !stamps)) return MOE_ERR_INVALID_ARG;
  const size_t n = c->tl_gu + c->tl_dn;
  if (cap < 3 * n) return fail(c, MOE_ERR_INVALID_ARG, "moe_debug_read_timeline: %zu stamps do not fit %zu", 3 * n, cap);
  HIPC(c, hipDeviceSynchronize());
  if (n) HIPC(c, hipMemcpy(stamps, c->tl, n * 3 * 8, hipMemcpyDeviceToHost));
  *n_gate_up = c->tl_gu;
  *n_down = c->tl_dn;
  return MOE_OK;
}

extern "C" moe_status moe_debug_quantize_q8_0(moe_ctx *c, const float *x, int n, int8_t *qs, uint16_t *d,
                                              void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!x || !qs || !d || n <= 0 || n % 32) return fail(c, MOE_ERR_INVALID_ARG, "moe_debug_quantize_q8_0: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  const int nb = n / 32;
  hipLaunchKernelGGL(k_debug_quantize, dim3(ceil_div(nb, 32)), dim3(64), 0, (hipStream_t)stream, x, nb, qs, d);
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

extern "C" moe_status moe_debug_wave_sum(moe_ctx *c, const float *x, int n_waves, float *out, void *stream) {
  if (!c) return MOE_ERR_INVALID_ARG;
  if (!x || !out || n_waves <= 0) return fail(c, MOE_ERR_INVALID_ARG, "moe_debug_wave_sum: bad arguments");
  HIPC(c, hipSetDevice(c->device));
  hipLaunchKernelGGL(k_debug_wave_sum, dim3(n_waves), dim3(64), 0, (hipStream_t)stream, x, out);
  HIPC(c, hipGetLastError());
  return MOE_OK;
}

extern "C" moe_status moe_debug_last_h(moe_ctx *c, float *h, size_t cap, size_t *n) {
  if (!c || !h || !n) return MOE_ERR_INVALID_ARG;
  const size_t rows = c->sc.h_rows, F = (size_t)c->sc.last_F;
  const size_t cnt = rows * F < cap ? rows * F : cap;
  HIPC(c, hipDeviceSynchronize());
  if (cnt) HIPC(c, hipMemcpy(h, c->sc.htap, cnt * 4, hipMemcpyDeviceToHost));
  *n = cnt;
  return MOE_OK;
}

#include "moe_server.h"
#include "graph_split.h"
