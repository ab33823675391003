// nano-glm moe-server protocol v2 served from the MoE block (host code,
// included by moe_block.hip after the C-ABI it calls).
//
// Per request (nano-glm/apps/moe-server/main.cpp:606-741 does the same
// steps on ggml graphs): x to the device, router logits (k_router_logits),
// moe_route (score, bias for selection, top-k, renorm, scale), moe_forward
// of the routed experts with MOE_FWD_NO_SHARED (the shared expert stays with
// the trunk, glm_dsa/moe_block.h:99-100), the combined rows back.  One
// stream, one request at a time: the trunk is strictly sequential.
#pragma once

#include <arpa/inet.h>
#include <netinet/in.h>
#include <netinet/tcp.h>
#include <sys/socket.h>

#include <cerrno>
#include <chrono>

static_assert(sizeof(moe_wire_hello_request) == 24, "hello request layout");
static_assert(sizeof(moe_wire_hello_response) == 80, "hello response layout");
static_assert(sizeof(moe_wire_request) == 40, "request layout");
static_assert(sizeof(moe_wire_response) == 56, "response layout");

struct srv_layer {
  bool served = false;  // a MoE layer with MXFP4 experts and a learned router
  int route_mode = MOE_ROUTE_SIGMOID, route_norm = 0;
  float route_scale = 1.0f;
  float *w = nullptr;     // router [E][H] f32 (widened exactly from the file's f32 / f16 / bf16)
  int w_type = MOE_GGML_F32;  // the file's ggml type of the router (x is rounded to it)
  float *bias = nullptr;  // [E] f32 or null
};

struct moe_server {
  moe_ctx *ctx = nullptr;
  int device = 0;
  std::string path, arch, err;
  uint32_t n_embd = 0, n_layer = 0, n_dense_lead = 0, n_expert = 0, n_used = 0, n_ff = 0;
  float scale = 1.0f;
  uint32_t norm = 0;
  std::vector<srv_layer> layers;
  hipStream_t stream = nullptr;
  // per-request device buffers, grown on demand
  size_t cap_tokens = 0;
  float *x = nullptr, *logits = nullptr, *wts = nullptr, *out = nullptr;
  int32_t *ids = nullptr;
  float *pin_x = nullptr, *pin_out = nullptr;  // pinned host staging of x and the rows
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};  // request start, routed, evaluated
  int listen_fd = -1;
};

static void srv_free_buffers(moe_server *s) {
  for (void *p : {(void *)s->x, (void *)s->logits, (void *)s->wts, (void *)s->out, (void *)s->ids})
    if (p) (void)hipFree(p);
  for (void *p : {(void *)s->pin_x, (void *)s->pin_out})
    if (p) (void)hipHostFree(p);
  s->x = s->logits = s->wts = s->out = s->pin_x = s->pin_out = nullptr;
  s->ids = nullptr;
  s->cap_tokens = 0;
}

extern "C" void moe_server_close(moe_server *s) {
  if (!s) return;
  if (s->listen_fd >= 0) close(s->listen_fd);
  (void)hipSetDevice(s->device);
  (void)hipDeviceSynchronize();
  srv_free_buffers(s);
  for (srv_layer &l : s->layers) {
    if (l.w) (void)hipFree(l.w);
    if (l.bias) (void)hipFree(l.bias);
  }
  for (hipEvent_t e : s->ev)
    if (e) (void)hipEventDestroy(e);
  if (s->stream) (void)hipStreamDestroy(s->stream);
  if (s->ctx) moe_ctx_destroy(s->ctx);
  delete s;
}

extern "C" const char *moe_server_last_error(const moe_server *s) { return s ? s->err.c_str() : ""; }

static moe_status srv_fail(moe_server *s, moe_status st, const std::string &m) {
  s->err = m;
  return st;
}

static float *srv_upload(const std::vector<float> &v) {
  float *d = nullptr;
  if (hipMalloc(&d, v.size() * sizeof(float)) != hipSuccess) return nullptr;
  if (hipMemcpy(d, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(d);
    return nullptr;
  }
  return d;
}

static moe_status server_open(moe_server *s, const char *path, uint64_t budget);

extern "C" moe_status moe_server_open(const char *path, int device, uint64_t budget, moe_server **out, char *err,
                                      size_t err_len) {
  if (err && err_len) err[0] = 0;
  if (!path || !out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  moe_server *s = new moe_server;
  s->device = device;
  s->path = path;
  const moe_status st = server_open(s, path, budget);
  if (st != MOE_OK) {
    if (err && err_len) snprintf(err, err_len, "%s", s->err.c_str());
    moe_server_close(s);
    return st;
  }
  *out = s;
  return MOE_OK;
}

// The body of moe_server_open; on failure s->err says why and the caller
// closes s.
static moe_status server_open(moe_server *s, const char *path, uint64_t budget) {
  moe_status st = moe_ctx_create(s->device, budget, &s->ctx);
  if (st != MOE_OK) return srv_fail(s, st, moe_status_str(st));
  gguf::model M;
  if (!M.open(path)) {
    return srv_fail(s, MOE_ERR_FORMAT, M.err);
  }
  M.get_str("general.architecture", &s->arch);
  const std::string a = s->arch + ".";
  int64_t v = 0;
  if (s->arch.empty() || !M.get_int(a + "block_count", &v) || v < 1 || v > 100000) {
    return srv_fail(s, MOE_ERR_FORMAT, "general.architecture or <arch>.block_count is missing");
  }
  s->n_layer = (uint32_t)v;
  s->n_dense_lead = M.get_int(a + "leading_dense_block_count", &v) && v >= 0 ? (uint32_t)v : 0;
  const int64_t n_hash = M.get_int(a + "hash_layer_count", &v) && v > 0 ? v : 0;
  s->layers.resize(s->n_layer);
  if (hipSetDevice(s->device) != hipSuccess || hipStreamCreate(&s->stream) != hipSuccess ||
      hipEventCreate(&s->ev[0]) != hipSuccess || hipEventCreate(&s->ev[1]) != hipSuccess ||
      hipEventCreate(&s->ev[2]) != hipSuccess) {
    return srv_fail(s, MOE_ERR_HIP, "stream creation failed");
  }
  for (uint32_t il = s->n_dense_lead; il < s->n_layer; il++) {
    srv_layer &L = s->layers[il];
    if ((int64_t)il < n_hash) continue;  // routes by token id: not served
    if (!M.find_tensor("blk." + std::to_string(il) + ".ffn_gate_exps.weight")) continue;
    moe_gguf_layer info;
    st = moe_layer_upload_gguf(s->ctx, (int)il, path, (int)il, &info);
    if (st != MOE_OK) {
      return srv_fail(s, st, std::string("layer ") + std::to_string(il) + ": " + moe_ctx_last_error(s->ctx));
    }
    const uint32_t H = (uint32_t)info.desc.hidden, E = (uint32_t)info.desc.n_expert;
    if (s->n_embd == 0) {
      s->n_embd = H;
      s->n_expert = E;
      s->n_used = (uint32_t)info.desc.n_used;
      s->n_ff = (uint32_t)info.desc.ffn;
      s->scale = info.route_scale;
      s->norm = (uint32_t)info.route_norm;
    } else if (H != s->n_embd || E != s->n_expert || (uint32_t)info.desc.n_used != s->n_used) {
      return srv_fail(s, MOE_ERR_FORMAT, "layer " + std::to_string(il) + " differs in shape from the first MoE layer");
    }
    if (H % 4) {
      return srv_fail(s, MOE_ERR_UNSUPPORTED, "n_embd is not a multiple of 4");
    }
    const std::string b = "blk." + std::to_string(il) + ".";
    const gguf::tensor *tw = M.find_tensor(b + "ffn_gate_inp.weight");
    const gguf::tensor *tb = M.find_tensor(b + "exp_probs_b.bias");
    std::vector<float> w, bias;
    if (!tw || !M.read_f32(*tw, (uint64_t)H * E, w) || (tw->ne[0] != H) || (tb && !M.read_f32(*tb, E, bias))) {
      return srv_fail(s, MOE_ERR_FORMAT, b + "ffn_gate_inp.weight / exp_probs_b.bias: " +
                                           (M.err.empty() ? std::string("missing or not [n_embd, n_expert]") : M.err));
    }
    L.w = srv_upload(w);
    L.w_type = tw->type;
    if (tb) L.bias = srv_upload(bias);
    if (!L.w || (tb && !L.bias)) {
      return srv_fail(s, MOE_ERR_HIP, "router upload failed");
    }
    L.route_mode = info.route_mode >= 0 ? info.route_mode
                                        : (s->arch == "glm-dsa" ? MOE_ROUTE_SIGMOID : MOE_ROUTE_SOFTMAX);
    L.route_norm = info.route_norm;
    L.route_scale = info.route_scale;
    L.served = true;
  }
  if (s->n_embd == 0) return srv_fail(s, MOE_ERR_FORMAT, "the model has no MoE layer with MXFP4 experts");
  return MOE_OK;
}

using srv_clk = std::chrono::steady_clock;
static uint32_t srv_us(srv_clk::time_point t0) {
  const auto d = std::chrono::duration_cast<std::chrono::microseconds>(srv_clk::now() - t0).count();
  return (uint32_t)(d < 0 ? 0 : d);
}

static void srv_error(std::vector<uint8_t> &resp, uint32_t status, const char *msg) {
  moe_wire_response rh = {};
  rh.magic = MOE_WIRE_MAGIC;
  rh.version = MOE_WIRE_VERSION;
  rh.msg_type = MOE_WIRE_RESPONSE;
  rh.status = status;
  rh.payload_bytes = strlen(msg);
  resp.resize(sizeof(rh) + rh.payload_bytes);
  memcpy(resp.data(), &rh, sizeof(rh));
  memcpy(resp.data() + sizeof(rh), msg, rh.payload_bytes);
}

static moe_wire_hello_response srv_hello(const moe_server *s, uint32_t status, uint64_t payload) {
  moe_wire_hello_response rh = {};
  rh.magic = MOE_WIRE_MAGIC;
  rh.version = MOE_WIRE_VERSION;
  rh.msg_type = MOE_WIRE_HELLO;
  rh.status = status;
  snprintf(rh.arch, sizeof(rh.arch), "%s", s->arch.c_str());
  rh.n_embd = s->n_embd;
  rh.n_layer = s->n_layer;
  rh.n_dense_lead = s->n_dense_lead;
  rh.n_expert = s->n_expert;
  rh.n_expert_used = s->n_used;
  rh.n_ff_exp = s->n_ff;
  rh.expert_scale = s->scale;
  rh.expert_norm = s->norm;
  rh.payload_bytes = payload;
  return rh;
}

static std::string srv_fingerprint(const moe_server *s) {
  return "server=moe_block gfx950\nmodel=" + s->path + "\narch=" + s->arch + "\n";
}

// Hello exchange; false: the connection must close (a version error was answered).
static bool srv_hello_reply(const moe_server *s, const moe_wire_hello_request &rq, std::vector<uint8_t> &resp) {
  if (rq.magic != MOE_WIRE_MAGIC || rq.msg_type != MOE_WIRE_HELLO) {
    srv_error(resp, MOE_WIRE_ERR_VERSION, "expected MOE_MSG_HELLO as the first message");
    return false;
  }
  if (rq.version != MOE_WIRE_VERSION) {
    srv_error(resp, MOE_WIRE_ERR_VERSION, "protocol version mismatch");
    return false;
  }
  const std::string me = srv_fingerprint(s);
  const moe_wire_hello_response rh = srv_hello(s, MOE_WIRE_OK, me.size());
  resp.resize(sizeof(rh) + me.size());
  memcpy(resp.data(), &rh, sizeof(rh));
  memcpy(resp.data() + sizeof(rh), me.data(), me.size());
  return true;
}

// Header checks of a request, in moe-server's order; returns a wire status
// and sets *msg on error.
static uint32_t srv_check(const moe_server *s, const moe_wire_request &rq, const char **msg) {
  if (rq.magic != MOE_WIRE_MAGIC || rq.msg_type != MOE_WIRE_REQUEST)
    return *msg = "bad magic or message type", MOE_WIRE_ERR_VERSION;
  if (rq.version != MOE_WIRE_VERSION) return *msg = "protocol version mismatch", MOE_WIRE_ERR_VERSION;
  if (rq.n_embd != s->n_embd || rq.n_tokens == 0) return *msg = "n_embd mismatch or n_tokens == 0", MOE_WIRE_ERR_DIMS;
  if ((uint64_t)rq.n_tokens * s->n_used > MOE_GROUP_MAX_PAIRS)
    return *msg = "n_tokens * n_expert_used exceeds the grouped path's limit", MOE_WIRE_ERR_DIMS;
  if (rq.layer >= s->n_layer || rq.layer < s->n_dense_lead || !s->layers[rq.layer].served)
    return *msg = "layer out of range or not a MoE layer", MOE_WIRE_ERR_LAYER;
  if (rq.return_mode != MOE_WIRE_RET_COMBINED) return *msg = "only MOE_RET_COMBINED is implemented", MOE_WIRE_ERR_MODE;
  if (rq.payload_bytes != (uint64_t)rq.n_embd * rq.n_tokens * sizeof(float))
    return *msg = "payload_bytes does not match dims", MOE_WIRE_ERR_DIMS;
  return MOE_WIRE_OK;
}

static bool srv_reserve(moe_server *s, size_t T) {
  if (T <= s->cap_tokens) return true;
  (void)hipStreamSynchronize(s->stream);
  srv_free_buffers(s);
  const size_t H = s->n_embd, E = s->n_expert, k = s->n_used;
  if (hipMalloc(&s->x, T * H * 4) != hipSuccess || hipMalloc(&s->out, T * H * 4) != hipSuccess ||
      hipMalloc(&s->logits, T * E * 4) != hipSuccess || hipMalloc(&s->wts, T * k * 4) != hipSuccess ||
      hipMalloc(&s->ids, T * k * 4) != hipSuccess ||
      hipHostMalloc((void **)&s->pin_x, T * H * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void **)&s->pin_out, T * H * 4, hipHostMallocDefault) != hipSuccess) {
    srv_free_buffers(s);
    return false;
  }
  s->cap_tokens = T;
  return true;
}

// A checked request with its payload x (in s->pin_x already, or anywhere in
// host memory): route, evaluate, respond.  False: an error response was
// produced (the connection closes).
static bool srv_eval(moe_server *s, const moe_wire_request &rq, const void *x, uint32_t t_parse_us,
                     std::vector<uint8_t> &resp) {
  const srv_layer &L = s->layers[rq.layer];
  const int T = (int)rq.n_tokens, H = (int)s->n_embd, E = (int)s->n_expert, k = (int)s->n_used;
  const size_t n = (size_t)T * H;
  // route and evaluate back to back on the stream; the two phases are timed
  // with events (no host round trip between them)
  bool ok = hipSetDevice(s->device) == hipSuccess && srv_reserve(s, (size_t)T);
  if (ok && x != s->pin_x) memcpy(s->pin_x, x, n * 4);
  ok = ok && hipEventRecord(s->ev[0], s->stream) == hipSuccess &&
       hipMemcpyAsync(s->x, s->pin_x, n * 4, hipMemcpyHostToDevice, s->stream) == hipSuccess &&
       moe_router_logits(s->ctx, L.w, s->x, T, E, H, L.w_type, s->logits, s->stream) == MOE_OK &&
       moe_route(s->ctx, s->logits, L.bias, T, E, k, L.route_mode, L.route_norm, L.route_scale, s->ids, s->wts,
                 s->stream) == MOE_OK &&
       hipEventRecord(s->ev[1], s->stream) == hipSuccess &&
       moe_forward(s->ctx, (int)rq.layer, s->x, s->ids, s->wts, T, s->out, MOE_FWD_NO_SHARED, s->stream) == MOE_OK &&
       hipMemcpyAsync(s->pin_out, s->out, n * 4, hipMemcpyDeviceToHost, s->stream) == hipSuccess &&
       hipEventRecord(s->ev[2], s->stream) == hipSuccess && hipStreamSynchronize(s->stream) == hipSuccess;
  float ms_route = 0.0f, ms_compute = 0.0f;
  if (ok) {
    (void)hipEventElapsedTime(&ms_route, s->ev[0], s->ev[1]);
    (void)hipEventElapsedTime(&ms_compute, s->ev[1], s->ev[2]);
  }
  const uint32_t t_route_us = (uint32_t)(ms_route * 1e3f), t_compute_us = (uint32_t)(ms_compute * 1e3f);
  if (!ok) {
    s->err = moe_ctx_last_error(s->ctx);
    srv_error(resp, MOE_WIRE_ERR_INTERNAL, "evaluation failed");
    return false;
  }
  const auto t2 = srv_clk::now();
  moe_wire_response rh = {};
  rh.magic = MOE_WIRE_MAGIC;
  rh.version = MOE_WIRE_VERSION;
  rh.msg_type = MOE_WIRE_RESPONSE;
  rh.status = MOE_WIRE_OK;
  rh.n_embd = rq.n_embd;
  rh.n_tokens = rq.n_tokens;
  rh.n_slots = 0;
  rh.t_parse_us = t_parse_us;
  rh.t_route_us = t_route_us;
  rh.t_compute_us = t_compute_us;
  rh.payload_bytes = n * 4;
  resp.resize(sizeof(rh) + n * 4);
  memcpy(resp.data() + sizeof(rh), s->pin_out, n * 4);
  rh.t_serialize_us = srv_us(t2);
  memcpy(resp.data(), &rh, sizeof(rh));
  return true;
}

extern "C" moe_status moe_server_handle(moe_server *s, const void *msg, size_t len, void *resp, size_t cap,
                                        size_t *resp_len) {
  if (!s || !msg || !resp_len || (!resp && cap)) return MOE_ERR_INVALID_ARG;
  std::vector<uint8_t> r;
  const uint8_t *m = static_cast<const uint8_t *>(msg);
  uint32_t type = 0;
  if (len >= 12) memcpy(&type, m + 8, 4);
  if (type == MOE_WIRE_HELLO && len >= sizeof(moe_wire_hello_request)) {
    moe_wire_hello_request rq;
    memcpy(&rq, m, sizeof(rq));
    srv_hello_reply(s, rq, r);
  } else if (len < sizeof(moe_wire_request)) {
    srv_error(r, MOE_WIRE_ERR_VERSION, "message shorter than its header");
  } else {
    const auto t0 = srv_clk::now();
    moe_wire_request rq;
    memcpy(&rq, m, sizeof(rq));
    const char *why = nullptr;
    const uint32_t st = srv_check(s, rq, &why);
    if (st != MOE_WIRE_OK) {
      srv_error(r, st, why);
    } else if (len - sizeof(rq) != rq.payload_bytes) {
      srv_error(r, MOE_WIRE_ERR_DIMS, "payload_bytes does not match the message");
    } else {
      srv_eval(s, rq, m + sizeof(rq), srv_us(t0), r);
    }
  }
  *resp_len = r.size();
  if (r.size() > cap) return MOE_ERR_INVALID_ARG;
  memcpy(resp, r.data(), r.size());
  return MOE_OK;
}

// ---- TCP ---------------------------------------------------------------------

static bool srv_send_all(int fd, const void *p, size_t n) {
  const char *c = static_cast<const char *>(p);
  while (n > 0) {
    const ssize_t k = send(fd, c, n > (1u << 20) ? (1u << 20) : n, MSG_NOSIGNAL);
    if (k <= 0) {
      if (k < 0 && errno == EINTR) continue;
      return false;
    }
    c += k;
    n -= (size_t)k;
  }
  return true;
}

static bool srv_recv_all(int fd, void *p, size_t n) {
  char *c = static_cast<char *>(p);
  while (n > 0) {
    const ssize_t k = recv(fd, c, n > (1u << 20) ? (1u << 20) : n, 0);
    if (k <= 0) {
      if (k < 0 && errno == EINTR) continue;
      return false;  // 0: the peer closed
    }
    c += k;
    n -= (size_t)k;
  }
  return true;
}

extern "C" moe_status moe_server_listen(moe_server *s, const char *host, int port, int *bound_port) {
  if (!s || !host || port < 0 || port > 65535) return MOE_ERR_INVALID_ARG;
  if (s->listen_fd >= 0) close(s->listen_fd);
  s->listen_fd = socket(AF_INET, SOCK_STREAM | SOCK_CLOEXEC, 0);
  if (s->listen_fd < 0) return srv_fail(s, MOE_ERR_INVALID_ARG, std::string("socket: ") + strerror(errno));
  const int one = 1;
  setsockopt(s->listen_fd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof(one));
  sockaddr_in addr = {};
  addr.sin_family = AF_INET;
  addr.sin_port = htons((uint16_t)port);
  if (inet_pton(AF_INET, host, &addr.sin_addr) != 1 ||
      bind(s->listen_fd, reinterpret_cast<sockaddr *>(&addr), sizeof(addr)) != 0 || listen(s->listen_fd, 4) != 0) {
    const std::string e = strerror(errno);
    close(s->listen_fd);
    s->listen_fd = -1;
    return srv_fail(s, MOE_ERR_INVALID_ARG, "listen on " + std::string(host) + ": " + e);
  }
  socklen_t al = sizeof(addr);
  getsockname(s->listen_fd, reinterpret_cast<sockaddr *>(&addr), &al);
  if (bound_port) *bound_port = ntohs(addr.sin_port);
  return MOE_OK;
}

// One connection: hello, then requests until a disconnect or an error response.
static void srv_connection(moe_server *s, int fd) {
  std::vector<uint8_t> resp;
  moe_wire_hello_request hq;
  if (!srv_recv_all(fd, &hq, sizeof(hq))) return;
  const bool hello_ok = srv_hello_reply(s, hq, resp);
  if (hello_ok && hq.payload_bytes) {  // the client's fingerprint, read and dropped
    if (hq.payload_bytes > (1u << 20)) return;
    std::string peer(hq.payload_bytes, '\0');
    if (!srv_recv_all(fd, &peer[0], peer.size())) return;
  }
  if (!srv_send_all(fd, resp.data(), resp.size()) || !hello_ok) return;
  for (;;) {
    moe_wire_request rq;
    if (!srv_recv_all(fd, &rq, sizeof(rq))) return;
    const auto t0 = srv_clk::now();
    const char *why = nullptr;
    const uint32_t st = srv_check(s, rq, &why);
    if (st != MOE_WIRE_OK) {
      srv_error(resp, st, why);
      srv_send_all(fd, resp.data(), resp.size());
      return;  // the stream position is no longer trusted
    }
    const uint32_t t_parse_us = srv_us(t0);
    if (hipSetDevice(s->device) != hipSuccess || !srv_reserve(s, rq.n_tokens)) {
      srv_error(resp, MOE_WIRE_ERR_INTERNAL, "out of memory for the request");
      srv_send_all(fd, resp.data(), resp.size());
      return;
    }
    if (!srv_recv_all(fd, s->pin_x, rq.payload_bytes)) return;  // straight into the pinned staging
    const bool ok = srv_eval(s, rq, s->pin_x, t_parse_us, resp);
    if (!srv_send_all(fd, resp.data(), resp.size()) || !ok) return;
  }
}

extern "C" moe_status moe_server_serve(moe_server *s, int max_connections) {
  if (!s) return MOE_ERR_INVALID_ARG;
  if (s->listen_fd < 0) return srv_fail(s, MOE_ERR_INVALID_ARG, "moe_server_serve: not listening");
  if (hipSetDevice(s->device) != hipSuccess) return srv_fail(s, MOE_ERR_HIP, "hipSetDevice failed");
  for (int n = 0; max_connections < 0 || n < max_connections; n++) {
    const int fd = accept4(s->listen_fd, nullptr, nullptr, SOCK_CLOEXEC);
    if (fd < 0) {
      if (errno == EINTR || errno == ECONNABORTED) {
        n--;
        continue;
      }
      return srv_fail(s, MOE_ERR_INVALID_ARG, std::string("accept: ") + strerror(errno));
    }
    const int one = 1;
    setsockopt(fd, IPPROTO_TCP, TCP_NODELAY, &one, sizeof(one));  // latency, not throughput
    srv_connection(s, fd);
    close(fd);
  }
  return MOE_OK;
}
