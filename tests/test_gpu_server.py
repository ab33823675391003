"""nano-glm moe-server protocol v2 served from the MoE block, on the GPU.

A four-layer glm-dsa GGUF model (layer 0 dense; layers 1-3 MoE with f32,
bf16 and f16 routers, a selection bias on layer 1 and an MXFP4 shared
expert the server must leave to the trunk) is written from the generator's
blocks.  Every response is checked bit-exact against the same library
driven directly (moe_router_logits -> moe_route_forward with
MOE_FWD_NO_SHARED), and that against the CPU oracle: the oracle's routing
of the GPU's router logits gives the same ids, and the oracle's block on
those ids (routed experts only) matches the rows within 1e-3 of their RMS.
The router logits are checked against float64 numpy with x rounded to the
router's type first (ggml-cpu's mul_mat converts x to an f16 / bf16
weight's type; the products are then exact, so only the f32 summation
order can differ).  Error responses follow moe-server's checks
(nano-glm/apps/moe-server/main.cpp:815-852), over handle() and over TCP.
"""
import socket
import threading

import numpy as np
import pytest

import gguf_stub as gs
import moe_block as mb
import workloads as wl
from parity import check_block, oracle_layer

pytestmark = pytest.mark.gpu

H, F, E, K = 1024, 512, 16, 4
SEED = 91
SHAPE = wl.LayerShape(hidden=H, ffn=F, n_expert=E, n_used=K, has_shared=False, route_mode=wl.ROUTE_SIGMOID)


def say(*a):
    print("[gpu]", *a, flush=True)


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    u = a.astype(np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even


@pytest.fixture(scope="module")
def model(tmp_path_factory, oracle):
    rng = np.random.default_rng(SEED)
    kvs = gs.moe_keys("glm-dsa", 4, H, F, E, K, gating=2, norm=True, scale=2.5)
    kvs.append(("glm-dsa.leading_dense_block_count", gs.U32, 1))
    tensors = [("blk.0.ffn_gate.weight", [H, 4 * F], gs.GGML_F16, bytes(2 * H * 4 * F))]
    routers = {}
    for il in (1, 2, 3):
        g = [np.stack([oracle.gen_mxfp4(SEED, il, t, e, H if t == 2 else F, F if t == 2 else H) for e in range(E)])
             for t in range(3)]
        sh = tuple(oracle.gen_mxfp4(SEED, il, 3 + t, 0, H if t == 2 else F, F if t == 2 else H) for t in range(3))
        tensors += gs.expert_tensors(il, g[0], g[1], g[2], sh if il == 1 else None)
        w = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
        if il == 1:
            bias = (rng.standard_normal(E) * 0.02).astype(np.float32)
            tensors += [(f"blk.{il}.ffn_gate_inp.weight", [H, E], gs.GGML_F32, w.tobytes()),
                        (f"blk.{il}.exp_probs_b.bias", [E], gs.GGML_F32, bias.tobytes())]
        elif il == 2:
            bits = to_bf16_bits(w)
            w = (bits.astype(np.uint32) << 16).view(np.float32)  # what the server holds after the bf16 -> f32
            bias = None
            tensors.append((f"blk.{il}.ffn_gate_inp.weight", [H, E], gs.GGML_BF16, bits.tobytes()))
        else:
            w16 = w.astype(np.float16)
            w = w16.astype(np.float32)  # f16 -> f32 is exact
            bias = None
            tensors.append((f"blk.{il}.ffn_gate_inp.weight", [H, E], gs.GGML_F16, w16.tobytes()))
        routers[il] = (w, bias, {1: mb.GGML_F32, 2: mb.GGML_BF16, 3: mb.GGML_F16}[il])
    path = tmp_path_factory.mktemp("srv") / "glm-moe.gguf"
    path.write_bytes(gs.gguf_bytes(kvs, tensors))
    say("server model", path.stat().st_size, "bytes")
    return str(path), routers


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch, torch.device("cuda:0")


@pytest.fixture(scope="module")
def direct(model, torch_dev):
    """The same layers in a plain MoeBlock context (ids 101-103)."""
    path, _ = model
    b = mb.MoeBlock(0)
    b.set_taps(True)
    for il in (1, 2, 3):
        info = b.upload_layer_gguf(100 + il, path, il)
        assert info.desc.has_shared == (1 if il == 1 else 0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def server(model, torch_dev):
    s = mb.MoeServer(model[0], 0)
    yield s
    s.close()


def request(layer, x, n_embd=H, version=mb.WIRE_VERSION, mode=mb.WIRE_RET_COMBINED, magic=mb.WIRE_MAGIC,
            payload=None):
    body = np.ascontiguousarray(x, np.float32).tobytes() if payload is None else payload
    T = 0 if x is None else x.shape[0]
    hdr = mb.WireRequest(magic, version, mb.WIRE_REQUEST, layer, n_embd, T, mode, 0, len(body))
    return bytes(hdr) + body


def parse_response(r: bytes):
    h = mb.WireResponse.from_buffer_copy(r[:56])
    assert h.magic == mb.WIRE_MAGIC and h.msg_type == mb.WIRE_RESPONSE and len(r) == 56 + h.payload_bytes
    return h, r[56:]


def round_to(x: np.ndarray, w_type: int) -> np.ndarray:
    """x rounded to the router's ggml type (round to nearest even), as f32."""
    if w_type == mb.GGML_F16:
        return x.astype(np.float16).astype(np.float32)
    if w_type == mb.GGML_BF16:
        return (to_bf16_bits(x).astype(np.uint32) << 16).view(np.float32)
    return x


def reference(direct, torch_dev, routers, layer, x):
    """Router logits, ids, weights and combined routed rows through the
    library directly."""
    torch, dev = torch_dev
    w, bias, w_type = routers[layer]
    T = x.shape[0]
    xd = torch.from_numpy(x).to(dev)
    lg = torch.empty((T, E), dtype=torch.float32, device=dev)
    direct.router_logits(torch.from_numpy(w).to(dev), xd, lg, w_type=w_type)
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((T, K), dtype=torch.float32, device=dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)
    direct.route_forward(100 + layer, xd, lg, ids, wts, out, mb.ROUTE_SIGMOID, norm=True, scale=2.5,
                         bias=None if bias is None else torch.from_numpy(bias).to(dev), flags=mb.MOE_FWD_NO_SHARED)
    torch.cuda.synchronize()
    return lg.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy(), out.cpu().numpy()


def test_hello(server):
    hq = mb.WireHelloRequest(mb.WIRE_MAGIC, mb.WIRE_VERSION, mb.WIRE_HELLO, 0, 7)
    r = server.handle(bytes(hq) + b"k=v\nx=y")
    h = mb.WireHelloResponse.from_buffer_copy(r[:80])
    assert (h.status, h.arch, h.n_embd, h.n_layer, h.n_dense_lead) == (mb.WIRE_OK, b"glm-dsa", H, 4, 1)
    assert (h.n_expert, h.n_expert_used, h.n_ff_exp, h.expert_scale, h.expert_norm) == (E, K, F, 2.5, 1)
    assert b"server=" in r[80:] and len(r) == 80 + h.payload_bytes


@pytest.mark.parametrize("layer, T", [(1, 1), (1, 6), (2, 1), (2, 5), (3, 3)])
def test_request_matches_the_block(server, direct, model, torch_dev, layer, T):
    say("server request layer", layer, "T", T)
    x, _ = wl.make_inputs(SHAPE, T, 300 + 10 * layer + T)
    h, body = parse_response(server.handle(request(layer, x)))
    assert (h.status, h.n_embd, h.n_tokens, h.n_slots) == (mb.WIRE_OK, H, T, 0), body[:200]
    got = np.frombuffer(body, np.float32).reshape(T, H)
    lg, ids, wts, ref = reference(direct, torch_dev, model[1], layer, x)
    w, bias, w_type = model[1][layer]
    lg64 = round_to(x, w_type).astype(np.float64) @ w.astype(np.float64).T
    err = np.abs(lg - lg64).max() / np.abs(lg64).max()
    say(f"router logits (type {w_type}) max rel err {err:.2e}; timings parse/route/compute us", h.t_parse_us,
        h.t_route_us, h.t_compute_us)
    assert err < 1e-5  # without x rounded to bf16 / f16 the difference would be ~1e-3
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("layer, T", [(1, 1), (1, 6), (2, 5), (3, 3)])
def test_response_rows_match_the_oracle(server, direct, model, torch_dev, oracle, layer, T):
    """The server's rows against the CPU oracle: the oracle routes the GPU's
    router logits (sigmoid, selection bias, renorm, scale 2.5) to the same
    ids, and its block on those ids without the shared expert matches the
    rows at 1e-3 of their RMS (parity.check_block, the direct block's h
    taps: the rows are bit-exact with it)."""
    x, _ = wl.make_inputs(SHAPE, T, 700 + 10 * layer + T)
    h, body = parse_response(server.handle(request(layer, x)))
    assert h.status == mb.WIRE_OK, body[:200]
    got = np.frombuffer(body, np.float32).reshape(T, H)
    lg, ids, wts, ref = reference(direct, torch_dev, model[1], layer, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    w, bias, _ = model[1][layer]
    oi, ow = oracle.route(lg, K, mb.ROUTE_SIGMOID, norm=True, scale=2.5, bias=bias)
    np.testing.assert_array_equal(ids, oi)
    np.testing.assert_allclose(wts, ow, rtol=2e-6)  # the score's exp may differ by an ulp
    say(f"server layer {layer} T={T}: ids equal the oracle's routing of the logits", oi.tolist()[:2])
    L = oracle_layer(oracle, SHAPE, SEED, layer, oi)
    check_block(oracle, L, direct, SHAPE, x, oi, ow, got, f"server layer {layer} T{T}")


@pytest.mark.parametrize("case, status", [
    ("version", mb.WIRE_ERR_VERSION), ("magic", mb.WIRE_ERR_VERSION), ("n_embd", mb.WIRE_ERR_DIMS),
    ("n_tokens_0", mb.WIRE_ERR_DIMS), ("dense_layer", mb.WIRE_ERR_LAYER), ("layer_range", mb.WIRE_ERR_LAYER),
    ("per_slot", mb.WIRE_ERR_MODE), ("payload", mb.WIRE_ERR_DIMS), ("short", mb.WIRE_ERR_VERSION)])
def test_error_responses(server, case, status):
    x = np.zeros((2, H), np.float32)
    msg = {"version": lambda: request(1, x, version=1), "magic": lambda: request(1, x, magic=0x12345678),
           "n_embd": lambda: request(1, x[:, :512], n_embd=512), "n_tokens_0": lambda: request(1, x[:0]),
           "dense_layer": lambda: request(0, x), "layer_range": lambda: request(4, x),
           "per_slot": lambda: request(1, x, mode=mb.WIRE_RET_PER_SLOT),
           "payload": lambda: request(1, x, payload=b"\0" * 12), "short": lambda: b"NMOE\2\0\0\0"}[case]()
    h, body = parse_response(server.handle(msg))
    assert h.status == status and len(body) > 0, (case, h.status, body)


def _recv(sock, n):
    b = b""
    while len(b) < n:
        c = sock.recv(n - len(b))
        if not c:
            raise ConnectionError("closed")
        b += c
    return b


def test_tcp_connections(server, model):
    """Two connections on 127.0.0.1: hello + two requests (rows identical to
    handle()'s), then a client with the wrong version, which gets an error
    and a closed connection."""
    port = server.listen("127.0.0.1", 0)
    say("server listening on port", port)
    th = threading.Thread(target=server.serve, args=(2,), daemon=True)
    th.start()
    try:
        with socket.create_connection(("127.0.0.1", port), timeout=60) as c:
            c.sendall(bytes(mb.WireHelloRequest(mb.WIRE_MAGIC, mb.WIRE_VERSION, mb.WIRE_HELLO, 0, 4)) + b"a=b\n")
            hr = mb.WireHelloResponse.from_buffer_copy(_recv(c, 80))
            assert hr.status == mb.WIRE_OK and hr.n_embd == H
            _recv(c, hr.payload_bytes)
            for layer, T in ((1, 3), (2, 2)):
                x, _ = wl.make_inputs(SHAPE, T, 500 + layer)
                msg = request(layer, x)
                c.sendall(msg)
                rh = mb.WireResponse.from_buffer_copy(_recv(c, 56))
                body = _recv(c, rh.payload_bytes)
                assert rh.status == mb.WIRE_OK, body[:200]
                assert body == server.handle(msg)[56:]
        with socket.create_connection(("127.0.0.1", port), timeout=60) as c:
            c.sendall(bytes(mb.WireHelloRequest(mb.WIRE_MAGIC, 1, mb.WIRE_HELLO, 0, 0)))
            rh = mb.WireResponse.from_buffer_copy(_recv(c, 56))
            assert rh.status == mb.WIRE_ERR_VERSION
            assert b"version" in _recv(c, rh.payload_bytes)
            assert c.recv(1) == b""  # closed by the server
        th.join(timeout=60)
        assert not th.is_alive()
    finally:
        for _ in range(2):  # unblock a server still waiting in accept()
            if not th.is_alive():
                break
            try:
                socket.create_connection(("127.0.0.1", port), timeout=5).close()
            except OSError:
                pass
            th.join(timeout=10)


def test_deepseek4_model(tmp_path, oracle, torch_dev):
    """deepseek4 keys: sqrt-softplus gating (expert_gating_func 4), a per-layer
    SwiGLU clamp (swiglu_clamp_exp), hash-routed leading layers
    (hash_layer_count: answered with a LAYER error) and no dense lead."""
    torch, dev = torch_dev
    rng = np.random.default_rng(7)
    kvs = gs.moe_keys("deepseek4", 3, H, F, E, K, gating=4, norm=True, scale=1.5, clamp=[7.0, 7.0, 7.0],
                      clamp_sh=[7.0, 7.0, 7.0])
    kvs.append(("deepseek4.hash_layer_count", gs.U32, 2))
    tensors = []
    for il in (1, 2):
        g = [np.stack([oracle.gen_mxfp4(SEED, 10 + il, t, e, H if t == 2 else F, F if t == 2 else H)
                       for e in range(E)]) for t in range(3)]
        sh = tuple(oracle.gen_mxfp4(SEED, 10 + il, 3 + t, 0, H if t == 2 else F, F if t == 2 else H) for t in range(3))
        tensors += gs.expert_tensors(il, g[0], g[1], g[2], sh)
        w = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
        tensors.append((f"blk.{il}.ffn_gate_inp.weight", [H, E], gs.GGML_F32, w.tobytes()))
    path = tmp_path / "ds4.gguf"
    path.write_bytes(gs.gguf_bytes(kvs, tensors))
    srv = mb.MoeServer(str(path), 0)
    blk = mb.MoeBlock(0)
    try:
        hq = mb.WireHelloRequest(mb.WIRE_MAGIC, mb.WIRE_VERSION, mb.WIRE_HELLO, 0, 0)
        h = mb.WireHelloResponse.from_buffer_copy(srv.handle(bytes(hq))[:80])
        assert (h.arch, h.n_layer, h.n_dense_lead, h.expert_scale) == (b"deepseek4", 3, 0, 1.5)
        x, _ = wl.make_inputs(SHAPE, 4, 77)
        for layer in (0, 1):
            rh, body = parse_response(srv.handle(request(layer, x)))
            assert rh.status == mb.WIRE_ERR_LAYER, (layer, body)
        rh, body = parse_response(srv.handle(request(2, x)))
        assert rh.status == mb.WIRE_OK, body[:200]
        info = blk.upload_layer_gguf(202, str(path), 2)
        assert info.desc.clamp == 7.0 and info.route_mode == mb.ROUTE_SQRT_SOFTPLUS and info.desc.has_shared == 1
        w = np.frombuffer(tensors[-1][3], np.float32).reshape(E, H)
        xd = torch.from_numpy(x).to(dev)
        lg = torch.empty((4, E), dtype=torch.float32, device=dev)
        blk.router_logits(torch.from_numpy(w.copy()).to(dev), xd, lg, w_type=mb.GGML_F32)
        ids = torch.empty((4, K), dtype=torch.int32, device=dev)
        wts = torch.empty((4, K), dtype=torch.float32, device=dev)
        out = torch.empty((4, H), dtype=torch.float32, device=dev)
        blk.route_forward(202, xd, lg, ids, wts, out, mb.ROUTE_SQRT_SOFTPLUS, norm=True, scale=1.5,
                          flags=mb.MOE_FWD_NO_SHARED)
        torch.cuda.synchronize()
        ref = out.cpu().numpy()
        got = np.frombuffer(body, np.float32).reshape(4, H)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        blk.close()
        srv.close()
