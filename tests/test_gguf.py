"""The GGUF reader of the C-ABI (moe_gguf_read_layer) on CPU: shapes and
router keys of a MoE layer, the shared-expert rules, split models, and
errors for malformed files (every read of the file is bounds-checked, so
truncated or corrupted files must come back as MOE_ERR_FORMAT, never a
crash).  The files are written by tests/gguf_stub.py."""
import numpy as np
import pytest

import gguf_stub as gs
import moe_block as mb

H, F, E, K = 64, 32, 4, 2


def blocks(rng, *shape):
    return rng.integers(0, 256, size=shape + (17,), dtype=np.uint8)


def layer_arrays(seed=0, shared=True):
    rng = np.random.default_rng(seed)
    g, u = blocks(rng, E, F, H // 32), blocks(rng, E, F, H // 32)
    d = blocks(rng, E, H, F // 32)
    sh = (blocks(rng, F, H // 32), blocks(rng, F, H // 32), blocks(rng, H, F // 32)) if shared else None
    return g, u, d, sh


def write(tmp_path, kvs, tensors, name="m.gguf", **kw):
    p = tmp_path / name
    p.write_bytes(gs.gguf_bytes(kvs, tensors, **kw))
    return str(p)


def model(tmp_path, arch="deepseek2", clamp=None, clamp_sh=None, shared=True, shared_type=gs.GGML_MXFP4, gating=2,
          **kw):
    """Two layers: 0 dense (no expert tensors), 1 MoE."""
    g, u, d, sh = layer_arrays(shared=shared)
    if sh is not None and shared_type != gs.GGML_MXFP4:
        sh = tuple(np.zeros(a.size, np.uint8) for a in sh)  # stand-in bytes of another type
    kvs = gs.moe_keys(arch, 2, H, F, E, K, gating=gating, clamp=clamp, clamp_sh=clamp_sh)
    tensors = [("blk.0.ffn_gate.weight", [H, F], gs.GGML_F16, bytes(2 * H * F))]
    tensors += gs.expert_tensors(1, g, u, d, sh, shared_type)
    return write(tmp_path, kvs, tensors, **kw)


def read(path, layer=1):
    return mb.read_gguf_layer(path, layer)


def status_of(path, layer=1):
    with pytest.raises(mb.MoeError) as ei:
        read(path, layer)
    return ei.value.status, str(ei.value)


def test_layer_shape_and_router_keys(tmp_path):
    info = read(model(tmp_path, clamp=[0.0, 7.5], clamp_sh=[0.0, 7.5]))
    d = info.desc
    assert (d.hidden, d.ffn, d.n_expert, d.n_used, d.has_shared) == (H, F, E, K, 1)
    assert d.clamp == 7.5
    assert info.arch == b"deepseek2" and info.n_layer == 2
    assert (info.route_mode, info.route_norm, info.route_scale) == (mb.ROUTE_SIGMOID, 1, 2.5)
    assert info.shared_type == gs.GGML_MXFP4


@pytest.mark.parametrize("gating, mode", [(1, mb.ROUTE_SOFTMAX), (2, mb.ROUTE_SIGMOID),
                                          (4, mb.ROUTE_SQRT_SOFTPLUS), (3, -1), (None, -1)])
def test_gating_func_maps_to_route_mode(tmp_path, gating, mode):
    assert read(model(tmp_path, gating=gating)).route_mode == mode


def test_no_clamp_key_means_no_clamp(tmp_path):
    assert read(model(tmp_path)).desc.clamp == 0.0


def test_shared_expert_with_another_clamp_is_left_to_the_trunk(tmp_path):
    info = read(model(tmp_path, clamp=[0.0, 7.5], clamp_sh=[0.0, 10.0]))
    assert info.desc.has_shared == 0 and info.shared_type == gs.GGML_MXFP4


def test_shared_expert_of_another_type_is_left_to_the_trunk(tmp_path):
    info = read(model(tmp_path, shared_type=gs.GGML_Q8_0))
    assert info.desc.has_shared == 0 and info.shared_type == gs.GGML_Q8_0


def test_no_shared_expert(tmp_path):
    info = read(model(tmp_path, shared=False))
    assert info.desc.has_shared == 0 and info.shared_type == -1


def test_dense_layer_and_out_of_range_layer(tmp_path):
    p = model(tmp_path)
    st, msg = status_of(p, 0)
    assert st == mb.MOE_ERR_FORMAT and "blk.0.ffn_gate_exps.weight" in msg
    assert status_of(p, 2)[0] == mb.MOE_ERR_INVALID_ARG
    assert status_of(p, -1)[0] == mb.MOE_ERR_INVALID_ARG


def test_other_alignment_and_version_2(tmp_path):
    g, u, d, sh = layer_arrays()
    kvs = gs.moe_keys("glm-dsa", 1, H, F, E, K) + [("general.alignment", gs.U32, 64)]
    p = write(tmp_path, kvs, gs.expert_tensors(0, g, u, d, sh), alignment=64, version=2)
    assert read(p, 0).desc.n_expert == E


def test_split_model(tmp_path):
    """Metadata in the first file, the layer's tensors in the second."""
    g, u, d, sh = layer_arrays()
    kvs = gs.moe_keys("deepseek2", 2, H, F, E, K)
    write(tmp_path, kvs, [("blk.0.ffn_gate.weight", [H, F], gs.GGML_F16, bytes(2 * H * F))],
          name="m-00001-of-00002.gguf")
    first = str(tmp_path / "m-00001-of-00002.gguf")
    st, msg = status_of(first)
    assert st == mb.MOE_ERR_FORMAT and "m-00002-of-00002.gguf" in msg  # second file missing
    write(tmp_path, [("split.no", gs.U16, 1)], gs.expert_tensors(1, g, u, d, sh), name="m-00002-of-00002.gguf")
    info = read(first)
    assert (info.desc.hidden, info.desc.n_expert, info.desc.has_shared) == (H, E, 1)


@pytest.mark.parametrize("case", ["magic", "version", "routed_type", "dims", "used_missing", "used_range",
                                  "count", "ffn_len", "embd", "clamp_short", "clamp_type", "misaligned",
                                  "alignment", "array_of_arrays", "data_short", "ndims"])
def test_malformed_files(tmp_path, case):
    g, u, d, sh = layer_arrays()
    kvs = gs.moe_keys("deepseek2", 2, H, F, E, K)
    tensors = gs.expert_tensors(1, g, u, d, sh)
    kw = {}

    def set_key(key, t, v):
        nonlocal kvs
        kvs = [x for x in kvs if x[0] != key] + ([(key, t, v)] if t is not None else [])

    if case == "routed_type":
        tensors[0] = (tensors[0][0], tensors[0][1], gs.GGML_Q8_0, tensors[0][3])
    elif case == "dims":
        tensors[2] = (tensors[2][0], [H, F, E], gs.GGML_MXFP4, tensors[2][3])
    elif case == "ndims":
        tensors[1] = (tensors[1][0], [H, F * E], gs.GGML_MXFP4, tensors[1][3])
    elif case == "used_missing":
        set_key("deepseek2.expert_used_count", None, None)
    elif case == "used_range":
        set_key("deepseek2.expert_used_count", gs.U32, E + 1)
    elif case == "count":
        set_key("deepseek2.expert_count", gs.U32, E + 1)
    elif case == "ffn_len":
        set_key("deepseek2.expert_feed_forward_length", gs.U32, 2 * F)
    elif case == "embd":
        set_key("deepseek2.embedding_length", gs.U32, 2 * H)
    elif case == "clamp_short":
        set_key("deepseek2.swiglu_clamp_exp", gs.ARR, (gs.F32, [1.0]))
    elif case == "clamp_type":
        set_key("deepseek2.swiglu_clamp_exp", gs.ARR, (gs.I32, [1, 2]))
    elif case == "alignment":
        set_key("general.alignment", gs.U32, 48)
        kw["alignment"] = 48
    elif case == "array_of_arrays":
        set_key("x.nested", gs.ARR, (gs.ARR, []))
    elif case == "misaligned":
        kvs.append(("general.alignment", gs.U32, 64))  # tensors laid out at 32: the second starts at 32
        tensors.insert(0, ("blk.0.attn_norm.weight", [8], gs.GGML_F32, bytes(32)))
    raw = bytearray(gs.gguf_bytes(kvs, tensors, **kw))
    if case == "magic":
        raw[0:4] = b"GGML"
    elif case == "version":
        raw[4:8] = (1).to_bytes(4, "little")
    elif case == "data_short":
        raw = raw[:-100]
    p = tmp_path / "bad.gguf"
    p.write_bytes(bytes(raw))
    st, msg = status_of(str(p))
    assert st == mb.MOE_ERR_FORMAT, (case, st, msg)
    assert "moe_gguf_read_layer: " in msg and len(msg) > len("moe_gguf_read_layer: ") + 4


def test_missing_file(tmp_path):
    st, msg = status_of(str(tmp_path / "absent.gguf"))
    assert st == mb.MOE_ERR_FORMAT and "cannot open" in msg


def test_truncations_and_corruptions_never_crash(tmp_path):
    """Every prefix length up to the data section, and single-byte corruptions
    of the header and infos: each read returns a status (the process would die
    on an out-of-bounds read of the mapping)."""
    g, u, d, sh = layer_arrays()
    kvs = gs.moe_keys("deepseek2", 2, H, F, E, K, clamp=[0.0, 3.0], clamp_sh=[0.0, 3.0])
    raw = gs.gguf_bytes(kvs, gs.expert_tensors(1, g, u, d, sh))
    head = raw.index(b"blk.1.ffn_down_shexp.weight") + 64
    p = tmp_path / "t.gguf"
    for n in range(0, head):
        p.write_bytes(raw[:n])
        with pytest.raises(mb.MoeError):
            read(str(p))
    rng = np.random.default_rng(5)
    ok = 0
    for i in range(600):
        b = bytearray(raw)
        pos = int(rng.integers(0, head))
        b[pos] = int(rng.integers(0, 256))
        p.write_bytes(bytes(b))
        try:
            read(str(p))
            ok += 1
        except mb.MoeError as e:
            assert e.status in (mb.MOE_ERR_FORMAT, mb.MOE_ERR_INVALID_ARG)
    assert ok > 0  # corruptions that leave the layer readable still read
