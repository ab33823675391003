// TEST-ONLY driver of the MoE ggml backend adapter: dlopens the adapter
// (llama-sandbox_amd/ggml_backend/moe_ggml_backend.cpp built against the
// stand-in headers) and uses it the way llama.cpp's loader and scheduler do,
// then prints one JSON object of what it saw for tests/test_ggml_backend.py.
//
//   drive_backend <adapter.so> <gpu|cpu> [small|c1|v3] [dump_dir]
//
// Models (routed-expert layers in the backend's "MoE" host buffer):
//  small  H=1024, F=512, E=16, top-4, random MXFP4 bytes: layer 3 plain,
//         layer 4 with deepseek4's clamps (gate <= 7, up in [-7, 7]), layer 5
//         with a clamp the device has no form for (gate in [-7, 7]), layer 6
//         plain (set up to exceed MOESERV_TP_BUDGET_MB when the test sets it).
//  c1     the C1 shape (H=2048, F=768, E=32, top-4): layer 3 plain, layer 4
//         clamped at 0.75 with exponents that make the clamp bind (gpu only).
//  v3     the DeepSeek-V3 shape (H=7168, F=2048, E=256, top-8): layer 3 (gpu
//         only; 6 GB of host buffer).
// c1 and v3 weights come from the library's counter-based generator (seed
// 4242; moe_layer_generate on a second context, read back in ggml layout),
// so the test can rebuild them in the CPU oracle.  In gpu mode every split
// the backend computes is compared bit for bit with this library's own
// moe_forward_host(MOE_FWD_PER_SLOT) on that second context, and with a
// dump_dir each device split's x, ids, wts, MUL node and the second
// context's SwiGLU taps are written there for the oracle comparison.
#include "ggml_stub.h"
#include "moe_block.h"

#include <dlfcn.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

namespace {

const uint64_t kSeed = 4242;
const float kInf = INFINITY;

struct layer_spec {
  int id;
  float gmin, gmax, umin, umax;
  int e_lo, e_span;  // generated models only
};

struct run_spec {
  int li, T;
  const char *tag;
};

struct model_spec {
  const char *name;
  int H, F, E, K;
  bool generated;
  std::vector<layer_spec> layers;
  std::vector<run_spec> runs;
};

model_spec model_named(const std::string &n) {
  if (n == "c1")
    return {"c1", 2048, 768, 32, 4, true,
            {{3, -kInf, kInf, -kInf, kInf, 124, 7}, {4, -kInf, 0.75f, -0.75f, 0.75f, 128, 3}},
            {{0, 1, "c1_l3_t1"}, {0, 5, "c1_l3_t5"}, {1, 2, "c1_l4_t2"}, {1, 7, "c1_l4_t7"}}};
  if (n == "v3")
    return {"v3", 7168, 2048, 256, 8, true, {{3, -kInf, kInf, -kInf, kInf, 124, 7}}, {{0, 1, "v3_t1"}, {0, 4, "v3_t4"}}};
  return {"small", 1024, 512, 16, 4, false,
          {{3, -kInf, kInf, -kInf, kInf, 0, 0}, {4, -kInf, 7.0f, -7.0f, 7.0f, 0, 0},
           {5, -7.0f, 7.0f, -7.0f, 7.0f, 0, 0}, {6, -kInf, kInf, -kInf, kInf, 0, 0}},
          {{0, 1, "l3_t1"}, {0, 3, "l3_t3"}, {1, 2, "l4_clamp_t2"}, {2, 1, "l5_symclamp_a"}, {2, 1, "l5_symclamp_b"},
           {3, 1, "l6_a"}, {3, 2, "l6_b"}}};
}

float clamp_limit(const layer_spec &l) { return std::isfinite(l.umax) ? l.umax : 0.0f; }

struct layer_w {
  int id;
  ggml_tensor gate{}, up{}, down{};
  std::vector<uint8_t> bytes[3];  // host copies for the reference context (random models)
};

void set_name(ggml_tensor &t, const std::string &n) { snprintf(t.name, sizeof t.name, "%s", n.c_str()); }

ggml_tensor tensor(enum ggml_type type, std::initializer_list<int64_t> ne, enum ggml_op op = GGML_OP_NONE) {
  ggml_tensor t{};
  t.type = type;
  int i = 0;
  for (int64_t v : ne) t.ne[i++] = v;
  for (; i < GGML_MAX_DIMS; i++) t.ne[i] = 1;
  t.op = op;
  return t;
}

void random_mxfp4(std::vector<uint8_t> &b, size_t blocks, std::mt19937 &rng) {
  b.resize(blocks * 17);
  for (size_t i = 0; i < blocks; i++) {
    b[i * 17] = (uint8_t)(124 + rng() % 7);
    for (int j = 1; j < 17; j++) b[i * 17 + j] = (uint8_t)rng();
  }
}

// one layer's routed-expert block as the scheduler hands it over, plus the
// trunk's ADD chain (never claimed)
struct block_graph {
  ggml_tensor xin, x, ids, wts, up, gate, gclamp, uclamp, act, y, mul;
  std::vector<ggml_tensor> views, adds;
  std::vector<float> xv, wv, out;
  std::vector<int32_t> iv;
  std::vector<ggml_tensor *> split;
};

void build(block_graph &g, const model_spec &M, layer_w &L, int T, const layer_spec &ls, std::mt19937 &rng) {
  const int H = M.H, F = M.F, E = M.E, K = M.K;
  const float gmin = ls.gmin, gmax = ls.gmax, umin = ls.umin, umax = ls.umax;
  std::normal_distribution<float> nd;
  g.xv.resize((size_t)T * H);
  for (float &v : g.xv) v = nd(rng);
  g.iv.resize((size_t)T * K);
  g.wv.resize((size_t)T * K);
  for (int t = 0; t < T; t++) {
    std::vector<int> p(E);
    for (int e = 0; e < E; e++) p[e] = e;
    for (int j = 0; j < K; j++) {
      std::swap(p[j], p[j + rng() % (E - j)]);
      g.iv[t * K + j] = p[j];
      g.wv[t * K + j] = 0.1f + 0.05f * j;
    }
  }
  g.out.assign((size_t)T * K * H, 0.0f);
  g.xin = tensor(GGML_TYPE_F32, {H, T});
  g.xin.data = g.xv.data();
  set_name(g.xin, "ffn_moe_input");
  g.x = tensor(GGML_TYPE_F32, {H, 1, T}, GGML_OP_RESHAPE);
  g.x.src[0] = &g.xin;
  g.x.view_src = &g.xin;
  g.x.data = g.xv.data();
  g.ids = tensor(GGML_TYPE_I32, {K, T});
  g.ids.data = g.iv.data();
  g.wts = tensor(GGML_TYPE_F32, {1, K, T});
  g.wts.data = g.wv.data();
  g.up = tensor(GGML_TYPE_F32, {F, K, T}, GGML_OP_MUL_MAT_ID);
  g.up.src[0] = &L.up; g.up.src[1] = &g.x; g.up.src[2] = &g.ids;
  g.gate = tensor(GGML_TYPE_F32, {F, K, T}, GGML_OP_MUL_MAT_ID);
  g.gate.src[0] = &L.gate; g.gate.src[1] = &g.x; g.gate.src[2] = &g.ids;
  g.split = {&g.up, &g.gate};
  ggml_tensor *ga = &g.gate, *ua = &g.up;
  if (std::isfinite(gmax) || std::isfinite(gmin)) {
    g.gclamp = tensor(GGML_TYPE_F32, {F, K, T}, GGML_OP_CLAMP);
    g.gclamp.src[0] = &g.gate;
    memcpy(&g.gclamp.op_params[0], &gmin, 4);
    memcpy(&g.gclamp.op_params[1], &gmax, 4);
    g.uclamp = tensor(GGML_TYPE_F32, {F, K, T}, GGML_OP_CLAMP);
    g.uclamp.src[0] = &g.up;
    memcpy(&g.uclamp.op_params[0], &umin, 4);
    memcpy(&g.uclamp.op_params[1], &umax, 4);
    ga = &g.gclamp;
    ua = &g.uclamp;
    g.split.push_back(&g.gclamp);
    g.split.push_back(&g.uclamp);
  }
  g.act = tensor(GGML_TYPE_F32, {F, K, T}, GGML_OP_GLU);
  g.act.src[0] = ga; g.act.src[1] = ua;
  g.act.op_params[0] = GGML_GLU_OP_SWIGLU;
  g.y = tensor(GGML_TYPE_F32, {H, K, T}, GGML_OP_MUL_MAT_ID);
  g.y.src[0] = &L.down; g.y.src[1] = &g.act; g.y.src[2] = &g.ids;
  g.mul = tensor(GGML_TYPE_F32, {H, K, T}, GGML_OP_MUL);
  g.mul.src[0] = &g.y; g.mul.src[1] = &g.wts;
  g.mul.data = g.out.data();
  g.split.push_back(&g.act);
  g.split.push_back(&g.y);
  g.split.push_back(&g.mul);
  g.views.resize(K);
  g.adds.resize(K - 1);
  for (int j = 0; j < K; j++) {
    g.views[j] = tensor(GGML_TYPE_F32, {H, T}, GGML_OP_VIEW);
    g.views[j].src[0] = &g.mul;
    g.views[j].view_src = &g.mul;
  }
  for (int j = 0; j + 1 < K; j++) {
    g.adds[j] = tensor(GGML_TYPE_F32, {H, T}, GGML_OP_ADD);
    g.adds[j].src[0] = j ? &g.adds[j - 1] : &g.views[0];
    g.adds[j].src[1] = &g.views[j + 1];
  }
}

std::string facts;
void fact(const char *k, long long v) { facts += (facts.empty() ? "" : ", ") + std::string("\"") + k + "\": " + std::to_string(v); }
void fact_s(const char *k, const char *v) { facts += (facts.empty() ? "" : ", ") + std::string("\"") + k + "\": \"" + v + "\""; }

bool dump(const std::string &dir, const std::string &name, const void *p, size_t bytes) {
  const std::string path = dir + "/" + name;
  FILE *f = fopen(path.c_str(), "wb");
  if (!f) return false;
  const bool ok = fwrite(p, 1, bytes, f) == bytes;
  return fclose(f) == 0 && ok;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: drive_backend <adapter.so> <gpu|cpu> [small|c1|v3] [dump_dir]\n");
    return 2;
  }
  const bool gpu = strcmp(argv[2], "gpu") == 0;
  const model_spec M = model_named(argc > 3 ? argv[3] : "small");
  const std::string dump_dir = argc > 4 ? argv[4] : "";
  if (M.generated && !gpu) {
    fprintf(stderr, "driver: the %s model is generated on the device (gpu mode only)\n", M.name);
    return 2;
  }
  const int H = M.H, F = M.F, E = M.E, K = M.K;
  void *h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!h) {
    fprintf(stderr, "dlopen: %s\n", dlerror());
    return 1;
  }
  auto init = (ggml_backend_init_t)dlsym(h, "ggml_backend_init");
  auto score = (ggml_backend_score_t)dlsym(h, "ggml_backend_score");
  if (!init || !score) return 1;
  fact_s("model", M.name);
  fact("H", H);
  fact("F", F);
  fact("E", E);
  fact("K", K);
  fact("seed", (long long)kSeed);
  fact("score", score());
  ggml_backend_reg_t reg = init();
  fact("api_version", reg->api_version);
  fact_s("reg_name", reg->iface.get_name(reg));
  fact("device_count", (long long)reg->iface.get_device_count(reg));
  ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
  fact("device_type_accel", dev->iface.get_type(dev) == GGML_BACKEND_DEVICE_TYPE_ACCEL);
  ggml_backend_dev_props props{};
  dev->iface.get_props(dev, &props);
  fact("props_memory_total", (long long)props.memory_total);
  fact("props_async", props.caps.async);
  ggml_backend_buffer_type_t buft = dev->iface.get_buffer_type(dev);
  fact_s("buft_name", buft->iface.get_name(buft));
  fact("buft_is_host", buft->iface.is_host(buft));
  fact("buft_alignment", (long long)buft->iface.get_alignment(buft));
  fact("supports_own_buft", dev->iface.supports_buft(dev, buft));
  ggml_backend_buffer_type other{};
  fact("supports_other_buft", dev->iface.supports_buft(dev, &other));
  ggml_backend_t be = dev->iface.init_backend(dev, nullptr);
  auto set_nt = (ggml_backend_set_n_threads_t)reg->iface.get_proc_address(reg, "ggml_backend_set_n_threads");
  fact("has_set_n_threads", set_nt != nullptr);
  fact("unknown_proc_null", reg->iface.get_proc_address(reg, "ggml_backend_no_such_function") == nullptr);
  if (set_nt) set_nt(be, 7);
  fact("cpu_threads_forwarded", stub_cpu_threads);
  fact("async_slots_null", be->iface.synchronize == nullptr && be->iface.graph_plan_create == nullptr &&
                               be->iface.set_tensor_async == nullptr && be->iface.event_record == nullptr);

  // a zero-size probe buffer (llama.cpp's weight_buft_supported) comes and goes
  ggml_backend_buffer_t probe = buft->iface.alloc_buffer(buft, 0);
  fact("probe_buffer", probe != nullptr);
  probe->iface.free_buffer(probe);
  delete probe;

  // the second context: the bit-exact reference, and the generator of c1 / v3
  moe_ctx *ref = nullptr;
  if (gpu && moe_ctx_create(0, UINT64_MAX, &ref) != MOE_OK) {
    fprintf(stderr, "driver: no reference context\n");
    return 1;
  }
  if (ref && !dump_dir.empty()) (void)moe_debug_set_taps(ref, 1);

  // the weights buffer: the model's layers
  std::mt19937 rng(11);
  const size_t gu_blocks = (size_t)E * F * (H / 32), dn_blocks = (size_t)E * H * (F / 32);
  const size_t layer_bytes = (2 * gu_blocks + dn_blocks) * 17;
  std::vector<layer_w> layers(M.layers.size());
  ggml_backend_buffer_t wbuf = buft->iface.alloc_buffer(buft, layer_bytes * layers.size());
  if (!wbuf) return 1;
  uint8_t *base = (uint8_t *)wbuf->iface.get_base(wbuf);
  size_t off = 0;
  std::vector<bool> ref_up(layers.size(), false);
  for (size_t i = 0; i < layers.size(); i++) {
    layer_w &L = layers[i];
    const layer_spec &ls = M.layers[i];
    L.id = ls.id;
    if (M.generated) {
      const moe_layer_desc d = {H, F, E, K, 0, clamp_limit(ls)};
      if (moe_layer_generate(ref, L.id, &d, kSeed, ls.e_lo, ls.e_span) != MOE_OK) {
        fprintf(stderr, "driver: generate failed: %s\n", moe_ctx_last_error(ref));
        return 1;
      }
      ref_up[i] = true;
    }
    ggml_tensor *ts[3] = {&L.gate, &L.up, &L.down};
    const char *nm[3] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    for (int t = 0; t < 3; t++) {
      *ts[t] = t == 2 ? tensor(GGML_TYPE_MXFP4, {F, H, E}) : tensor(GGML_TYPE_MXFP4, {H, F, E});
      set_name(*ts[t], "blk." + std::to_string(L.id) + "." + nm[t] + ".weight");
      ts[t]->buffer = wbuf;
      ts[t]->data = base + off;
      wbuf->iface.init_tensor(wbuf, ts[t]);
      const size_t bytes = (t == 2 ? dn_blocks : gu_blocks) * 17;
      if (M.generated) {  // the generated layer read back in ggml layout, expert by expert
        const size_t per_expert = bytes / E;
        for (int e = 0; e < E; e++)
          if (moe_layer_read_blocks(ref, L.id, t, e, base + off + (size_t)e * per_expert) != MOE_OK) {
            fprintf(stderr, "driver: read-back failed: %s\n", moe_ctx_last_error(ref));
            return 1;
          }
      } else {
        random_mxfp4(L.bytes[t], t == 2 ? dn_blocks : gu_blocks, rng);
        wbuf->iface.set_tensor(wbuf, ts[t], L.bytes[t].data(), 0, L.bytes[t].size());
      }
      off += bytes;
    }
    char k[64];
    snprintf(k, sizeof k, "l%d_e_lo", L.id);
    fact(k, ls.e_lo);
    snprintf(k, sizeof k, "l%d_e_span", L.id);
    fact(k, ls.e_span);
    snprintf(k, sizeof k, "l%d_clamp_x1e6", L.id);
    fact(k, std::llround(clamp_limit(ls) * 1e6));
  }

  // the claim set over the first layer's block
  block_graph g0;
  build(g0, M, layers[0], 2, M.layers[0], rng);
  int claimed = 0, n_block = 0;
  for (ggml_tensor *t : {&g0.up, &g0.gate, &g0.act, &g0.y, &g0.mul, &g0.x}) {
    n_block++;
    claimed += dev->iface.supports_op(dev, t) ? 1 : 0;
  }
  for (auto &v : g0.views) { n_block++; claimed += dev->iface.supports_op(dev, &v) ? 1 : 0; }
  fact("block_nodes", n_block);
  fact("block_claimed", claimed);
  int adds = 0;
  for (auto &a : g0.adds) adds += dev->iface.supports_op(dev, &a) ? 1 : 0;
  fact("adds_claimed", adds);
  ggml_tensor attn_a = tensor(GGML_TYPE_F32, {H, 2}), attn_b = tensor(GGML_TYPE_F32, {H, 2});
  ggml_tensor attn_mul = tensor(GGML_TYPE_F32, {H, 2}, GGML_OP_MUL);
  attn_mul.src[0] = &attn_a; attn_mul.src[1] = &attn_b;
  fact("trunk_mul_claimed", dev->iface.supports_op(dev, &attn_mul));
  ggml_tensor geglu = g0.act;
  geglu.op_params[0] = GGML_GLU_OP_GEGLU;
  fact("geglu_claimed", dev->iface.supports_op(dev, &geglu));
  ggml_tensor cpu_w = tensor(GGML_TYPE_MXFP4, {H, F, E});
  ggml_tensor foreign = g0.up;
  foreign.src[0] = &cpu_w;
  fact("foreign_weights_claimed", dev->iface.supports_op(dev, &foreign));

  // the splits, one graph_compute each
  for (const run_spec &r : M.runs) {
    const layer_spec &ls = M.layers[r.li];
    layer_w &L = layers[r.li];
    block_graph g;
    build(g, M, L, r.T, ls, rng);
    ggml_cgraph *cg = stub_graph(g.split.data(), (int)g.split.size());
    const int before = stub_cpu_calls;
    const enum ggml_status st = be->iface.graph_compute(be, cg);
    stub_graph_free(cg);
    const bool on_cpu = stub_cpu_calls > before;
    const std::string k = r.tag;
    fact((k + "_status").c_str(), st);
    fact((k + "_cpu").c_str(), on_cpu);
    fact((k + "_sentinel").c_str(), g.out[0] == STUB_CPU_SENTINEL);
    fact((k + "_T").c_str(), r.T);
    fact((k + "_layer").c_str(), L.id);
    if (!gpu || on_cpu) continue;
    if (!ref_up[r.li]) {
      const moe_layer_desc d = {H, F, E, K, 0, clamp_limit(ls)};
      if (moe_layer_upload(ref, L.id, &d, L.bytes[0].data(), L.bytes[1].data(), L.bytes[2].data(), nullptr, nullptr,
                           nullptr) != MOE_OK) {
        fprintf(stderr, "driver: reference upload failed: %s\n", moe_ctx_last_error(ref));
        return 1;
      }
      ref_up[r.li] = true;
    }
    std::vector<float> want((size_t)r.T * K * H);
    if (moe_forward_host(ref, L.id, g.xv.data(), g.iv.data(), g.wv.data(), r.T, want.data(), MOE_FWD_PER_SLOT) !=
        MOE_OK)
      return 1;
    fact((k + "_bit_exact").c_str(), memcmp(want.data(), g.out.data(), want.size() * 4) == 0);
    double rms = 0;
    for (float v : want) rms += (double)v * v;
    fact((k + "_nonzero").c_str(), rms > 0);
    if (!dump_dir.empty()) {
      std::vector<float> hv((size_t)r.T * K * F);
      size_t nh = 0;
      bool ok = moe_debug_last_h(ref, hv.data(), hv.size(), &nh) == MOE_OK && nh == hv.size();
      ok = ok && dump(dump_dir, k + ".x.f32", g.xv.data(), g.xv.size() * 4);
      ok = ok && dump(dump_dir, k + ".ids.i32", g.iv.data(), g.iv.size() * 4);
      ok = ok && dump(dump_dir, k + ".wts.f32", g.wv.data(), g.wv.size() * 4);
      ok = ok && dump(dump_dir, k + ".out.f32", g.out.data(), g.out.size() * 4);
      ok = ok && dump(dump_dir, k + ".h.f32", hv.data(), hv.size() * 4);
      fact((k + "_dumped").c_str(), ok);
    }
  }
  if (ref) moe_ctx_destroy(ref);
  // teardown: the weights buffer ends the model (the adapter prints its report)
  wbuf->iface.free_buffer(wbuf);
  delete wbuf;
  fact("cpu_calls", stub_cpu_calls);
  printf("{%s}\n", facts.c_str());
  fflush(stdout);
  be->iface.free(be);
  return 0;
}
