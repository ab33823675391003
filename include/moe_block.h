/*
 * moe_block.h -- C-ABI of the MI355X (gfx950) routed-expert MoE block.
 *
 * This is the drop-in boundary for the reference's MoE-block hot path: the
 * work that moe-serv's ggml backend does behind GGML_OP_MUL_MAT_ID
 * (moe-serv/src/moe_backend.cpp:413-484 dispatching to
 * moe-serv/src/moe_tp.h:711-790).  A ggml-backend adapter, the nano-glm
 * moe-server, or a Python/ctypes caller sits on top of these entry points.
 *
 * Conventions
 *  - Every entry point returns a moe_status (0 = MOE_OK, negative = error);
 *    no C++ exception crosses this boundary.  On error the context keeps a
 *    message readable with moe_ctx_last_error().
 *  - A caller that gets an error other than MOE_ERR_INVALID_ARG runs the
 *    block on its CPU path instead: the reference's rule is "every fall-back
 *    is to the CPU, never a skip" (moe_backend.cpp:436-445, moe_tp.h:714-724).
 *  - Pointers named *_dev are device pointers (HBM); *_host are host memory.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *  - Weight bytes are ggml block_mxfp4: 17-byte blocks {uint8 e; uint8 qs[16]}
 *    along the reduction dimension; element j of a block is qs[j] & 0xF and
 *    element j+16 is qs[j] >> 4; value = kvalue(nibble) * 2^(e-128) with
 *    kvalues = {0,1,2,3,4,6,8,12,-0,-1,-2,-3,-4,-6,-8,-12}
 *    (moe-serv/src/moe_tp.h:229-233, hip-moe/src/main.hip:44-57).
 *  - One context owns one GPU.  Calls on one context are not thread-safe
 *    (the reference's backend state is process-global singletons,
 *    moe_backend.cpp:58-62, driven by one scheduler thread).
 */
#ifndef MOE_BLOCK_H
#define MOE_BLOCK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_BLOCK_ABI_VERSION 1

typedef struct moe_ctx moe_ctx;
typedef struct moe_graph moe_graph;

typedef enum {
  MOE_OK = 0,
  MOE_ERR_INVALID_ARG = -1,   /* caller bug: bad pointer, shape or id       */
  MOE_ERR_HIP = -2,           /* a HIP runtime call failed                  */
  MOE_ERR_OUT_OF_BUDGET = -3, /* layer does not fit the residency budget    */
  MOE_ERR_UNSUPPORTED = -4,   /* shape the kernels do not handle            */
  MOE_ERR_NOT_RESIDENT = -5,  /* layer id has no weights on the device      */
  MOE_ERR_NO_DEVICE = -6,     /* no usable gfx950 device                    */
  MOE_ERR_INJECTED = -7,      /* failure forced by MOE_BLOCK_INJECT         */
  MOE_ERR_FORMAT = -8         /* model file unreadable or not an MXFP4 MoE  */
} moe_status;

/* Router score functions (glm_dsa/moe_block.h:51-53 sigmoid;
 * deepseek4/moe_block.h:108 sqrt(softplus); softmax as llama.cpp). */
enum { MOE_ROUTE_SOFTMAX = 0, MOE_ROUTE_SIGMOID = 1, MOE_ROUTE_SQRT_SOFTPLUS = 2 };

/* moe_forward flags */
enum {
  /* out is [T][k][H]: the per-slot rows already multiplied by the router
   * weight (the MUL node of the reference's split, moe_tp.h:754-776); no
   * slot sum and no shared expert.  Default: out is [T][H], the slot rows
   * summed in slot order ((y0+y1)+y2)+... plus the shared expert. */
  MOE_FWD_PER_SLOT = 1u << 0,
  /* Skip the shared expert even if the layer has one. */
  MOE_FWD_NO_SHARED = 1u << 1
};

/* Shape of one MoE layer (moe_tp.h:494-545 reads the same numbers off the
 * ggml split: K = hidden, INTER = ffn, SLOTS = n_used). */
typedef struct {
  int32_t hidden;     /* H: reduction dim of gate/up, output rows of down */
  int32_t ffn;        /* F: expert FFN width                               */
  int32_t n_expert;   /* E: routed experts                                 */
  int32_t n_used;     /* k: experts per token                              */
  int32_t has_shared; /* 1: one always-on shared expert of the same shape  */
  float clamp;        /* SwiGLU limit L (> 1e-6 enables: up in [-L, L],
                         gate <= L, before SiLU; deepseek4/moe_block.h:183-190) */
} moe_layer_desc;

/* ---- context ------------------------------------------------------------- */

/* Open device `device`.  budget_bytes caps the expert bytes this context may
 * keep resident (0 = every upload fails with MOE_ERR_OUT_OF_BUDGET, the
 * analogue of MOESERV_TP_BUDGET_MB=0; UINT64_MAX = no cap).
 * Replaces moe_tp_init (moe-serv/src/moe_tp.h:392-491). */
moe_status moe_ctx_create(int device, uint64_t budget_bytes, moe_ctx **out);
void moe_ctx_destroy(moe_ctx *ctx);
const char *moe_ctx_last_error(const moe_ctx *ctx);
const char *moe_status_str(moe_status s);
uint64_t moe_ctx_budget_left(const moe_ctx *ctx);

/* Free and total device memory of `device` (hipMemGetInfo), without a
 * context: what a residency planner reads before choosing a budget.  The
 * reference's placement reads the same two numbers per device and holds
 * MOESERV_RESERVE_MB of the free memory back (ggml_backend_dev_memory in
 * moe_place_probe, moe-serv/src/moe_place.h:56-78).  MOE_ERR_NO_DEVICE
 * when the device does not exist. */
moe_status moe_device_memory(int device, uint64_t *free_bytes, uint64_t *total_bytes);

/* Pre-size the per-call scratch for up to max_tokens tokens per call on
 * layers of this shape, so that later moe_forward / graph capture calls do
 * no allocation (moe_tp_set_dims, moe_tp.h:494-545, fixes its scratch the
 * same way from the first call). */
moe_status moe_ctx_reserve(moe_ctx *ctx, const moe_layer_desc *desc, int max_tokens);

/* ---- residency ----------------------------------------------------------- */

/* Make a layer resident: copy the ggml MXFP4 tensors from host memory and
 * repack them on the device.  gate/up are [E][F][H/32] blocks, down is
 * [E][H][F/32] blocks, the shared expert's are [F][H/32], [F][H/32],
 * [H][F/32] (NULL when desc->has_shared == 0).  Replaces
 * moe_tp_setup_layer (moe_tp.h:551-707) and moe_mirror_upload
 * (moe-serv/src/moe_mirror.h:68-119). */
moe_status moe_layer_upload(moe_ctx *ctx, int layer, const moe_layer_desc *desc,
                            const void *gate_host, const void *up_host,
                            const void *down_host, const void *sh_gate_host,
                            const void *sh_up_host, const void *sh_down_host);

/* Make a layer resident with synthetic weights generated on the device by
 * the counter-based generator (seed, layer, tensor, expert, block) with
 * E8M0 exponents uniform in [e_lo, e_lo + e_span).  Tensor ids: 0 gate,
 * 1 up, 2 down, 3/4/5 shared gate/up/down.  No counterpart in the
 * reference (its probes quantize random floats on the host,
 * moe-serv/src/moe_probe_custom.cpp:679-696); it exists so that 40 layers
 * (240 GB) can be made resident without a host copy. */
moe_status moe_layer_generate(moe_ctx *ctx, int layer, const moe_layer_desc *desc,
                              uint64_t seed, int e_lo, int e_span);

/* Read one expert matrix back in ggml block layout (inverse of the device
 * repack), into host memory of rows*(K/32)*17 bytes.  expert = E selects
 * the shared expert.  For round-trip tests. */
moe_status moe_layer_read_blocks(moe_ctx *ctx, int layer, int tensor, int expert,
                                 void *out_host);

/* ---- GGUF models --------------------------------------------------------- */

/* One MoE layer of a GGUF model: its shape (H, F, E from the expert
 * tensors' dims; k = <arch>.expert_used_count; clamp =
 * <arch>.swiglu_clamp_exp[layer], 0 when absent), and the router settings
 * the caller passes to moe_route (<arch>.expert_gating_func 1/2/4 ->
 * MOE_ROUTE_SOFTMAX/SIGMOID/SQRT_SOFTPLUS, -1 when absent or another value;
 * expert_weights_norm, default 0; expert_weights_scale, default 1).  The
 * shared expert is part of the layer (desc.has_shared = 1) only when
 * blk.N.ffn_{gate,up,down}_shexp.weight are MXFP4 of the routed shape and
 * its clamp (swiglu_clamp_shexp[layer]) equals the routed one; otherwise
 * the trunk computes it, as in the reference, whose split claims only the
 * routed experts (moe-serv/src/moe_backend.cpp:289-296). */
typedef struct {
  moe_layer_desc desc;
  int32_t n_layer;     /* <arch>.block_count, -1 when absent            */
  int32_t route_mode;  /* MOE_ROUTE_*, or -1                            */
  int32_t route_norm;  /* 0 / 1                                         */
  float route_scale;   /* multiplier of the routing weights             */
  int32_t shared_type; /* ggml type of ffn_gate_shexp, -1 when absent   */
  char arch[32];       /* general.architecture, NUL-terminated          */
} moe_gguf_layer;

/* Read layer `layer` of the GGUF model at `path` (the first file of a
 * split model: <stem>-00001-of-000NN.gguf) without a device: the tensors
 * blk.N.ffn_{gate,up,down}_exps.weight (ggml type 39, MXFP4, dims
 * [H,F,E], [H,F,E], [F,H,E]) and the keys above.  err (may be NULL)
 * receives a message on failure: MOE_ERR_INVALID_ARG for a NULL
 * argument, MOE_ERR_FORMAT for a file that cannot be read, or a layer
 * without MXFP4 routed experts.  The names are the ones nano-glm binds
 * (nano-glm/lib/models/deepseek4/model.h:366-372). */
moe_status moe_gguf_read_layer(const char *path, int layer, moe_gguf_layer *info, char *err,
                               size_t err_len);

/* Make layer `gguf_layer` of a GGUF model resident as `layer`: the file is
 * mapped read-only and its expert tensors go through moe_layer_upload.
 * info (may be NULL) receives what moe_gguf_read_layer reads.  Replaces
 * the residency step that moe-serv takes from ggml's loaded tensors
 * (moe_tp_setup_layer, moe_tp.h:551-707, fed by llama.cpp's GGUF loader). */
moe_status moe_layer_upload_gguf(moe_ctx *ctx, int layer, const char *path, int gguf_layer,
                                 moe_gguf_layer *info);

/* ---- the ggml backend's claim set and split, without ggml ---------------- */

/* One graph node as the ggml backend sees it, filled from a ggml_tensor
 * field for field by the adapter (which has ggml's headers; this library
 * does not).  op: MOE_NODE_*; type: ggml's type number (0 f32, 26 i32,
 * 39 mxfp4); glu_op / glu_swapped: a GLU node's op_params[0] / [1]
 * (ggml's glu op numbering, SwiGLU = 2); clamp_min / clamp_max: a CLAMP
 * node's op_params as floats; in_moe_buffer: the storage of the node (of
 * its view_src when it is a view) is the MoE buffer type. */
enum {
  MOE_NODE_NONE = 0,
  MOE_NODE_RESHAPE,
  MOE_NODE_VIEW,
  MOE_NODE_PERMUTE,
  MOE_NODE_TRANSPOSE,
  MOE_NODE_MUL_MAT_ID,
  MOE_NODE_CLAMP,
  MOE_NODE_MUL,
  MOE_NODE_GLU,
  MOE_NODE_ADD,
  MOE_NODE_OTHER
};
#define MOE_GLU_SWIGLU 2
#define MOE_GGML_F32 0
#define MOE_GGML_F16 1
#define MOE_GGML_BF16 30
#define MOE_GGML_I32 26
#define MOE_GGML_MXFP4 39

typedef struct moe_node {
  int32_t op, type;
  int64_t ne[4];
  int32_t contiguous;
  int32_t in_moe_buffer;
  int32_t glu_op, glu_swapped;
  float clamp_min, clamp_max;
  const struct moe_node *src[3];
  const struct moe_node *view_src;
  void *data;
  const char *name;
} moe_node;

/* Does the backend claim this node?  Views and reshapes: yes (free);
 * MUL_MAT_ID: iff its weights (src[0]) are in the MoE buffer; CLAMP and
 * MUL: iff they descend within 4 links from such a MUL_MAT_ID; GLU: iff
 * SwiGLU and so descended; ADD and everything else: no (ADD is also the
 * trunk's residual add).  MOESERV_DISABLE set in the environment: claim
 * nothing.  Restates moeserv_device_supports_op / moeserv_is_ours /
 * moeserv_derives_from_ours (moe-serv/src/moe_backend.cpp:262-345). */
int moe_node_claimed(const moe_node *node);

/* The routed-expert split of one MoE layer, parsed from the nodes the
 * backend received: the MUL node (the router-weight multiply) whose src[0]
 * is the down MUL_MAT_ID, whose input is the GLU (SwiGLU, not swapped) of
 * the gate and up MUL_MAT_IDs, each optionally through a CLAMP; shared x
 * and ids; f32 x / wts / out, i32 ids, MXFP4 weights; the layer id from
 * the gate weight's name "blk.N.".  Clamps: gate [gate_min, gate_max], up
 * [up_min, up_max] (infinite when absent).  Restates moe_tp_parse
 * (moe-serv/src/moe_tp.h:301-354), with more than one token allowed. */
typedef struct {
  const moe_node *gate_w, *up_w, *down_w, *x, *ids, *wts, *out;
  float gate_min, gate_max, up_min, up_max;
  int32_t layer, n_slots, n_tokens, hidden, ffn, n_expert;
} moe_split;

/* MOE_OK, or MOE_ERR_UNSUPPORTED with the reason in why (may be NULL). */
moe_status moe_split_parse(const moe_node *const *nodes, int n_nodes, moe_split *split, char *why,
                           size_t why_len);

/* Compute a split on the device: parse, check it against resident layer
 * split.layer (shape; clamps of the form gate <= L, up in [-L, L] with the
 * layer's L), then moe_forward_host with MOE_FWD_PER_SLOT into out's host
 * data ([T][k][H], the MUL node).  Any failure is a status other than
 * MOE_OK and the caller runs the split on its CPU path, never skips it
 * (moeserv_backend_graph_compute, moe_backend.cpp:413-484). */
moe_status moe_split_compute(moe_ctx *ctx, const moe_node *const *nodes, int n_nodes);

/* ---- nano-glm moe-server protocol v2 ------------------------------------ */

/* The wire format of nano-glm/lib/moe_proto.h:45-157: little-endian, fixed
 * headers, payload_bytes following each header.  One request is one MoE
 * layer for one batch: x [n_tokens][n_embd] f32 in, the routed experts'
 * combined rows [n_tokens][n_embd] f32 out (MOE_RET_COMBINED; the shared
 * expert stays with the trunk).  A v2 connection starts with a hello. */
#define MOE_WIRE_MAGIC 0x454F4D4Eu /* "NMOE" */
#define MOE_WIRE_VERSION 2u
enum { MOE_WIRE_REQUEST = 1, MOE_WIRE_RESPONSE = 2, MOE_WIRE_HELLO = 3 };
enum { MOE_WIRE_RET_COMBINED = 0, MOE_WIRE_RET_PER_SLOT = 1 };
enum {
  MOE_WIRE_OK = 0,
  MOE_WIRE_ERR_VERSION = 1,
  MOE_WIRE_ERR_DIMS = 2,
  MOE_WIRE_ERR_LAYER = 3,
  MOE_WIRE_ERR_MODE = 4,
  MOE_WIRE_ERR_INTERNAL = 5
};

typedef struct { /* 24 bytes; payload: client fingerprint, key=value lines */
  uint32_t magic, version, msg_type, reserved;
  uint64_t payload_bytes;
} moe_wire_hello_request;

typedef struct { /* 80 bytes; payload: server fingerprint */
  uint32_t magic, version, msg_type, status;
  char arch[16];
  uint32_t n_embd, n_layer, n_dense_lead, n_expert, n_expert_used, n_ff_exp;
  float expert_scale;
  uint32_t expert_norm;
  uint32_t reserved[2];
  uint64_t payload_bytes;
} moe_wire_hello_response;

typedef struct { /* 40 bytes; payload: n_embd * n_tokens f32 */
  uint32_t magic, version, msg_type, layer, n_embd, n_tokens, return_mode, reserved;
  uint64_t payload_bytes;
} moe_wire_request;

typedef struct { /* 56 bytes; payload: rows, or an error string if status != 0 */
  uint32_t magic, version, msg_type, status, n_embd, n_tokens, n_slots, reserved;
  uint32_t t_parse_us, t_route_us, t_compute_us, t_serialize_us; /* server clock */
  uint64_t payload_bytes;
} moe_wire_response;

typedef struct moe_server moe_server;

/* Load a GGUF model's router (blk.N.ffn_gate_inp.weight [H,E] f32/f16/bf16,
 * blk.N.exp_probs_b.bias [E] when present) and routed experts for every MoE
 * layer (<arch>.leading_dense_block_count .. block_count - 1) onto `device`
 * under budget_bytes.  Layers without expert tensors, and deepseek4's
 * hash-routed layers (<arch>.hash_layer_count), are answered with
 * MOE_WIRE_ERR_LAYER.  Routing follows the layer's keys (moe_gguf_layer;
 * no expert_gating_func: sigmoid for glm-dsa, as nano-glm reads it,
 * glm_dsa/model.h:99-101, softmax otherwise).  Replaces moe-server's model
 * load (nano-glm/apps/moe-server/main.cpp:331-401).  err (may be NULL)
 * receives a message on failure. */
moe_status moe_server_open(const char *gguf_path, int device, uint64_t budget_bytes, moe_server **out,
                           char *err, size_t err_len);
void moe_server_close(moe_server *srv);
const char *moe_server_last_error(const moe_server *srv);

/* One exchange: msg holds one whole message (hello or request header plus
 * its payload); the whole response (header plus payload) is written to
 * resp (cap bytes) and its size to *resp_len.  Protocol errors give an
 * error response (MOE_WIRE_ERR_*, with a message payload) and MOE_OK; a
 * response that does not fit cap returns MOE_ERR_INVALID_ARG with
 * *resp_len = the size needed.  The checks and their order follow
 * serve_hello / serve_one (moe-server/main.cpp:762-880). */
moe_status moe_server_handle(moe_server *srv, const void *msg, size_t len, void *resp, size_t cap,
                             size_t *resp_len);

/* TCP (IPv4): bind host:port (port 0 = any free port, returned in
 * *bound_port), then serve connections one at a time: a hello, then
 * requests until the peer disconnects or sends a request that gets an
 * error response (the stream position is then no longer trusted, as in
 * moe-server).  TCP_NODELAY on every connection (moe_proto.h:206-213).
 * moe_server_serve returns after max_connections connections (< 0: never).
 * Replaces moe-server's accept loop (main.cpp:1129-1150). */
moe_status moe_server_listen(moe_server *srv, const char *host, int port, int *bound_port);
moe_status moe_server_serve(moe_server *srv, int max_connections);

/* Router logits on the device: logits [T][E] = x [T][H] . W [E][H]^T with
 * f32 accumulation (ggml_mul_mat(ffn_gate_inp, x),
 * nano-glm/lib/models/glm_dsa/moe_block.h:52), H % 4 == 0, pointers 16-byte
 * aligned.  W is f32 on the device; w_type is the ggml type it was widened
 * from (MOE_GGML_F32, MOE_GGML_F16 or MOE_GGML_BF16): for f16 and bf16, x is
 * rounded to that type before the products, as ggml-cpu's mul_mat converts
 * src1 to src0's vec_dot_type.  The router of moe_server_*; feeds moe_route
 * / moe_route_forward. */
moe_status moe_router_logits(moe_ctx *ctx, const float *w_dev, const float *x_dev, int T, int E, int H,
                             int w_type, float *logits_dev, void *stream);

/* Free a layer's device memory and return its bytes to the budget
 * (moe_tp_free, moe_tp.h:356-390). */
moe_status moe_layer_release(moe_ctx *ctx, int layer);

/* Device bytes held by a layer (weights only). */
moe_status moe_layer_bytes(const moe_ctx *ctx, int layer, uint64_t *bytes);

/* ---- per call ------------------------------------------------------------ */

/* Router: logits [T][E] f32 -> ids [T][k] i32, wts [T][k] f32.  Scores are
 * softmax / sigmoid / sqrt(softplus) of the logits; bias [E] (or NULL) is
 * added for selection only; top-k descending, ties to the lower expert id;
 * weights are the unbiased scores of the selected experts; if norm, divided
 * by max(sum, 2^-14); if scale is not 0 or 1, multiplied by it
 * (nano-glm/lib/models/glm_dsa/moe_block.h:48-91). */
moe_status moe_route(moe_ctx *ctx, const float *logits_dev, const float *bias_dev,
                     int T, int E, int k, int mode, int norm, float scale,
                     int32_t *ids_dev, float *wts_dev, void *stream);

/* Token-to-expert grouping of ggml's mul_mat_id: pairs p = t*k + s in
 * token-major, slot-minor order, stably grouped by expert.
 * counts[E], offsets[E+1] (exclusive prefix sum), perm[T*k] (grouped row ->
 * pair), inv[T*k] (pair -> grouped row; may be NULL).  Bit-exact with the
 * host restatements (nano-glm/apps/moe-server/main.cpp:403-466). */
moe_status moe_group(moe_ctx *ctx, const int32_t *ids_dev, int T, int k, int E,
                     int32_t *counts_dev, int32_t *offsets_dev, int32_t *perm_dev,
                     int32_t *inv_dev, void *stream);

/* The MoE block: x [T][H] f32, ids/wts [T][k] from the router.  Activations
 * are Q8_0-quantized per 32-block (x before gate/up and the shared expert,
 * the SwiGLU output before down), weights stay MXFP4; per-block integer
 * dots, f32 accumulation -- ggml-cpu's MXFP4 x Q8_0 mul_mat_id arithmetic.
 * Output per `flags` (see MOE_FWD_*).  Replaces moe_tp_compute
 * (moe_tp.h:711-790) and moe_vk_compute (moe-serv/src/moe_run_vk.h:132-434),
 * i.e. the device work behind moeserv_backend_graph_compute
 * (moe_backend.cpp:413-484). */
moe_status moe_forward(moe_ctx *ctx, int layer, const float *x_dev,
                       const int32_t *ids_dev, const float *wts_dev, int T,
                       float *out_dev, uint32_t flags, void *stream);

/* moe_forward that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory during a call (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as moe_forward; the
 * per-call buffers come from one file-scope device array of
 * MOE_NOALLOC_SCRATCH_BYTES per GPU, held from the first moe_ctx_create on
 * that GPU until the process ends, instead of the context's scratch.  A
 * call whose buffers do not fit (T > 213 tokens on a V3-shaped
 * layer) returns MOE_ERR_INVALID_ARG.  Every call on one GPU shares that
 * GPU's array, across contexts: calls that overlap in time on one GPU
 * (other streams, other threads) race and give wrong results.  No HIP
 * event profiling and no debug taps on this path. */
#define MOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
moe_status moe_forward_noalloc(moe_ctx *ctx, int layer, const float *x_dev,
                               const int32_t *ids_dev, const float *wts_dev, int T,
                               float *out_dev, uint32_t flags, void *stream);

/* moe_forward from host buffers, synchronous: the reference's per-call
 * boundary (stage x/ids/wts in, read the result back into the host MUL
 * node, moe_tp.h:726-777). */
moe_status moe_forward_host(moe_ctx *ctx, int layer, const float *x_host,
                            const int32_t *ids_host, const float *wts_host, int T,
                            float *out_host, uint32_t flags);

/* Router + block in one call: logits [T][E] -> ids/wts (written to the
 * given device buffers) -> out. */
moe_status moe_route_forward(moe_ctx *ctx, int layer, const float *x_dev,
                             const float *logits_dev, const float *bias_dev,
                             int T, int mode, int norm, float scale,
                             int32_t *ids_dev, float *wts_dev, float *out_dev,
                             uint32_t flags, void *stream);

/* ---- hipGraph of a decode step ------------------------------------------- */

/* Capture n_layers consecutive moe_forward calls (layer ids layers[i],
 * inputs x/ids/wts/out device pointers per layer) into one hipGraph.  The
 * reference pre-records one command buffer per (layer, die) and replays it
 * (moe_tp.h:646-701); this is the gfx950 counterpart, for a whole stack.
 * Needs moe_ctx_reserve for T beforehand (no allocation under capture).
 *
 * A graph replays raw device pointers: the context's per-call scratch and
 * the weights of the layers it captured.  While a graph is alive (captured
 * and not yet destroyed) the context therefore refuses, with
 * MOE_ERR_INVALID_ARG and nothing launched, every call that would move or
 * free them: a moe_forward / moe_forward_host / moe_split_compute /
 * moe_ctx_reserve that needs a larger scratch than the one reserved, and a
 * moe_layer_release of a captured layer.  Reserve for the largest call
 * first, and destroy the graphs before releasing their layers.  The
 * caller's x/ids/wts/out buffers stay the caller's to keep alive. */
moe_status moe_graph_capture(moe_ctx *ctx, int n_layers, const int *layers,
                             const float *const *x_dev, const int32_t *const *ids_dev,
                             const float *const *wts_dev, float *const *out_dev,
                             int T, uint32_t flags, moe_graph **out);
/* MOE_ERR_INVALID_ARG for a graph whose context was destroyed (the
 * graph's executable goes with the context; the handle stays valid for
 * moe_graph_destroy). */
moe_status moe_graph_launch(moe_graph *g, void *stream);
void moe_graph_destroy(moe_graph *g);

/* ---- profiling ----------------------------------------------------------- */

/* Per-kernel GPU time, from a HIP event pair recorded on the launch stream
 * around every kernel the context launches while profiling is on (not under
 * graph capture).  The reference keeps per-split phase timings the same way
 * (moe-serv/src/moe_prof.h:36-137, MOESERV_PROFILE) and GPU timestamps
 * around its dispatches (moe-serv/src/moe_probe_custom.cpp:411-475). */
typedef struct {
  const char *name;   /* kernel class, static string                        */
  uint64_t launches;  /* launches timed since the last reset               */
  double total_us;    /* summed event-to-event time                         */
} moe_kernel_stat;

moe_status moe_prof_enable(moe_ctx *ctx, int on);

/* Engagement and phase counters of the host-boundary calls (moe_forward_host
 * and moe_split_compute): how many ran on the device, how many were refused
 * (any error: the caller ran its CPU path), the distinct routed experts
 * they read, and their phases -- upload (inputs to the device), compute
 * (the block), read (rows back), from HIP events on the call's stream while
 * moe_prof_enable is on, and total host time always.  The last device call's
 * figures are kept separately, for a per-split phase record.  The
 * reference keeps the same figures: "N splits on the dies, M fell back",
 * per-call stage / submit / wait times (moe-serv/src/moe_tp.h:792-802) and
 * the per-split phase rows of MOESERV_PROFILE (moe-serv/src/moe_prof.h:36-137). */
typedef struct {
  uint64_t calls;        /* computed on the device                          */
  uint64_t refusals;     /* returned an error (the caller's CPU path ran)   */
  uint64_t expert_loads; /* distinct routed experts, summed over the calls  */
  uint64_t timed_calls;  /* calls whose phases were timed                   */
  double upload_us, compute_us, read_us; /* summed over the timed calls     */
  double total_us;       /* summed host time of the device calls            */
  double last_upload_us, last_compute_us, last_read_us, last_total_us;
  uint32_t last_experts, last_tokens, last_timed;
} moe_call_stats;

/* Copy the counters; reset != 0 clears the sums and counts (not the last
 * call's figures). */
moe_status moe_call_stats_read(moe_ctx *ctx, moe_call_stats *stats, int reset);
/* Wait for the recorded launches, add them up, and return one entry per
 * kernel class with launches > 0 (at most cap, *n = the number of classes).
 * reset != 0 clears the totals afterwards. */
moe_status moe_prof_read(moe_ctx *ctx, moe_kernel_stat *stats, int cap, int *n, int reset);

/* ---- test hooks ---------------------------------------------------------- */

/* Keep the SwiGLU output h of every forward for moe_debug_last_h (off by
 * default: it costs an extra f32 store per h value). */
moe_status moe_debug_set_taps(moe_ctx *ctx, int on);

/* Q8_0 of n floats (n % 32 == 0) with the kernels' own quantizer:
 * qs [n] int8, d [n/32] fp16 bits. */
moe_status moe_debug_quantize_q8_0(moe_ctx *ctx, const float *x_dev, int n,
                                   int8_t *qs_dev, uint16_t *d_dev, void *stream);

/* The kernels' 64-lane wave sum applied to 64*n floats (one wave per 64). */
moe_status moe_debug_wave_sum(moe_ctx *ctx, const float *x_dev, int n_waves,
                              float *out_dev, void *stream);

/* SwiGLU output of the last moe_forward with taps on (moe_debug_set_taps):
 * h [rows][F] f32 before Q8_0, rows = T*k routed pairs in pair order, then
 * T shared rows.  Copies at most `cap` floats; returns the count in *n. */
moe_status moe_debug_last_h(moe_ctx *ctx, float *h_host, size_t cap, size_t *n);

/* Per-wave timeline of the decode launches (no counterpart in the
 * reference; a profiling aid).  While on, every eager T == 1 moe_forward
 * that runs k_gate_up_bal2 and k_down_dec stamps, for each of their waves,
 * three readings of the device's constant 100 MHz clock: entry, end of the
 * wave's K loop, exit.  moe_debug_read_timeline copies the stamps of the
 * last such call: n_gate_up records of k_gate_up_bal2 (record = workgroup * 9 +
 * wave), then n_down of k_down_dec (record = 16-row tile * S + slot wave),
 * 3 uint64 each; cap counts uint64s.  Off by default; turning it on
 * allocates a device buffer of 8192 records. */
moe_status moe_debug_set_timeline(moe_ctx *ctx, int on);
moe_status moe_debug_read_timeline(moe_ctx *ctx, uint64_t *stamps_host, size_t cap, size_t *n_gate_up,
                                   size_t *n_down);

#ifdef __cplusplus
}
#endif
#endif /* MOE_BLOCK_H */
