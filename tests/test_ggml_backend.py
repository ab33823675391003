"""The ggml backend adapter (llama-sandbox_amd/ggml_backend/moe_ggml_backend.cpp)
as llama.cpp would load it: built against test-only stand-ins of ggml's
headers (tests/ggml_stub/include, the vtable field orders the reference's
backend initializes against ggml 0.18.1, moe-serv/src/moe_backend.cpp) and
dlopened by tests/ggml_stub/drive_backend.cpp, which plays the loader and the
scheduler with a fake CPU delegate.  What it checks, from the driver's JSON:

- the exports and the three tiers (moe_backend.cpp:633-642, :550-613,
  :231-350, :167-205, :486-503): score, reg "MoE" with one ACCEL device, the
  "MoE" host buffer type (alignment 64), only graph_compute in the backend,
  get_proc_address("ggml_backend_set_n_threads") forwarded to the delegate;
- the claim set over ggml tensors (the block yes, the trunk's ADDs, an
  attention MUL, GEGLU and foreign weights no; MOESERV_DISABLE: nothing);
- per split (CPU): every split falls back to the CPU delegate without a
  device, the engagement report at teardown of the weights buffer only;
- per split (GPU): a plain and a deepseek4-clamped layer computed on the
  device, bit-exact with moe_forward_host(MOE_FWD_PER_SLOT) of the same
  weights; a clamp form the kernels lack and a layer over the residency
  budget fall back to the CPU once and stay there (the memo), and the
  per-split phase CSV of MOESERV_PROFILE in the reference's 14 columns with
  the per-device means on stderr (moe-serv/src/moe_prof.h:36-56, 94-137);
- the adapter's MUL node against the CPU oracle (GPU): C1- and V3-shaped
  layers made from the generator, every device split's per-slot rows checked
  by parity.check_block at 1e-3 of their RMS -- the reference's control /
  treatment gate (moe-serv/gate.py:196-222) with the oracle as the control;
- the residency budget without MOESERV_TP_BUDGET_MB: the device's free
  memory less MOESERV_RESERVE_MB (moe-serv/src/moe_place.h:56-78).

ABI fidelity to ggml 0.18.1 itself stays unverified: no ggml headers are in
this image.
"""
import csv
import glob
import json
import os
import re
import subprocess

import numpy as np
import pytest

import workloads as wl
from parity import Taps, check_block

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STUB = os.path.join(REPO, "tests", "ggml_stub")
DRIVER = os.path.join(STUB, "_build", "drive_backend")
ADAPTER = os.path.join(STUB, "_build", "libggml-moe.so")


def build():
    subprocess.run(["make", "-s", "-C", STUB], check=True, capture_output=True, text=True)


# the reference's MOESERV_PROFILE header (moe-serv/src/moe_prof.h:105-106)
PROFILE_COLUMNS = ["call", "dev", "n_nodes", "n_tok", "chunk", "n_chunks", "n_exp_loads", "build_us", "alloc_us",
                   "upload_us", "compute_us", "read_us", "free_us", "total_us"]


def drive(mode, env_extra=None, timeout=300, model="small", dump_dir=None):
    env = dict(os.environ)
    for k in ("MOESERV_DISABLE", "MOESERV_TP_BUDGET_MB", "MOESERV_PROFILE", "MOESERV_RESERVE_MB"):
        env.pop(k, None)
    env.update(env_extra or {})
    args = [DRIVER, ADAPTER, mode, model] + ([str(dump_dir)] if dump_dir else [])
    r = subprocess.run(args, capture_output=True, text=True, env=env, timeout=timeout)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1]), r.stderr


def read_profile(tmp_path):
    with open(glob.glob(str(tmp_path / "prof-*.csv"))[0]) as f:
        rd = csv.DictReader(f)
        return list(rd), rd.fieldnames


class DumpedTaps:
    """The SwiGLU taps the driver dumped, read like the block's debug taps
    (parity.gpu_h reorders them into the oracle's rows)."""

    def __init__(self, h):
        self.h = h

    def debug_last_h(self, n):
        assert n <= self.h.size
        return self.h[:n]


def test_backend_shell_and_cpu_fallback(tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("the no-device fallback is exercised on CPU-only hosts")
    build()
    f, err = drive("cpu", {"MOESERV_PROFILE": str(tmp_path / "prof")})
    assert f["score"] == 1 and f["reg_name"] == "MoE" and f["device_count"] == 1 and f["device_type_accel"] == 1
    assert f["buft_name"] == "MoE" and f["buft_is_host"] == 1 and f["buft_alignment"] == 64
    assert f["supports_own_buft"] == 1 and f["supports_other_buft"] == 0 and f["props_memory_total"] == 0
    assert f["has_set_n_threads"] == 1 and f["unknown_proc_null"] == 1 and f["cpu_threads_forwarded"] == 7
    assert f["async_slots_null"] == 1 and f["probe_buffer"] == 1
    assert f["block_claimed"] == f["block_nodes"] == 10
    assert f["adds_claimed"] == 0 and f["trunk_mul_claimed"] == 0 and f["geglu_claimed"] == 0
    assert f["foreign_weights_claimed"] == 0
    runs = ["l3_t1", "l3_t3", "l4_clamp_t2", "l5_symclamp_a", "l5_symclamp_b", "l6_a", "l6_b"]
    for r in runs:  # no device: every split on the CPU delegate, none skipped
        assert f[r + "_status"] == 0 and f[r + "_cpu"] == 1 and f[r + "_sentinel"] == 1, r
    assert f["cpu_calls"] == len(runs)
    assert "no device context" in err and err.count("no device context") == 1
    assert "0 splits on the device, 7 fell back" in err
    assert "first split has 5 nodes: MUL x1 MUL_MAT_ID x3 GLU x1" in err
    rows, header = read_profile(tmp_path)
    assert header == PROFILE_COLUMNS
    assert len(rows) == len(runs) and all(r["dev"] == "-1" for r in rows)
    for r, T in zip(rows, (1, 3, 2, 1, 1, 1, 2)):  # CPU rows as the reference writes them
        assert int(r["n_tok"]) == int(r["chunk"]) == T and r["n_chunks"] == "1" and r["n_exp_loads"] == "0"
        assert 0 <= int(r["compute_us"]) <= int(r["total_us"])
    assert re.search(r"MoE-gfx950:   cpu +n=7 +mean us: build [0-9.]+ alloc 0\.0 upload 0\.0 compute [0-9.]+ "
                     r"read 0\.0 free 0\.0 \| total [0-9.]+", err), err


def test_backend_disable_claims_nothing():
    build()
    f, _ = drive("cpu", {"MOESERV_DISABLE": "1"})
    assert f["block_claimed"] == 0 and f["adds_claimed"] == 0


@pytest.mark.gpu
def test_backend_on_the_device(tmp_path):
    """Layers 3 (plain) and 4 (deepseek4 clamps, L = 7) on the device,
    bit-exact with moe_forward_host; layer 5's symmetric gate clamp and layer
    6 (beyond a 27 MB budget that holds two 13.4 MB layers) on the CPU, each
    refused once and then remembered."""
    assert os.path.exists(DRIVER), "tests/ggml_stub/_build is built by __graft_entry__.build()"
    print("[gpu] ggml backend adapter on the device", flush=True)
    f, err = drive("gpu", {"MOESERV_TP_BUDGET_MB": "27", "MOESERV_PROFILE": str(tmp_path / "prof")})
    print(err, flush=True)
    for r in ("l3_t1", "l3_t3", "l4_clamp_t2"):
        assert f[r + "_status"] == 0 and f[r + "_cpu"] == 0 and f[r + "_sentinel"] == 0, r
        assert f[r + "_bit_exact"] == 1 and f[r + "_nonzero"] == 1, r
    for r in ("l5_symclamp_a", "l5_symclamp_b", "l6_a", "l6_b"):
        assert f[r + "_status"] == 0 and f[r + "_cpu"] == 1 and f[r + "_sentinel"] == 1, r
    assert err.count("layer 5: clamps") == 1          # refused once, then the memo
    assert err.count("layer 6:") == 1 and "does not fit" in err
    assert err.count("resident,") == 2
    assert "3 splits on the device, 4 fell back" in err
    assert "computed a split on the device (layer 3, 4 slots, 1 tokens)" in err
    rows, header = read_profile(tmp_path)
    assert header == PROFILE_COLUMNS
    dev_rows = [r for r in rows if r["dev"] == "0"]
    assert len(rows) == 7 and len(dev_rows) == 3
    for r in dev_rows:
        assert int(r["compute_us"]) > 0 and int(r["upload_us"]) >= 0 and int(r["read_us"]) >= 0
        assert int(r["total_us"]) >= int(r["compute_us"]) and r["n_chunks"] == "1" and r["chunk"] == r["n_tok"]
        assert 1 <= int(r["n_exp_loads"]) <= 16
    # the first split of layers 3 and 4 made them resident (alloc), the second of layer 3 did not
    assert [int(r["alloc_us"]) > 0 for r in dev_rows] == [True, False, True]
    assert re.search(r"MoE-gfx950:   gfx950 +n=3 +mean us: build", err) and re.search(r"   cpu +n=4 +mean us", err)


@pytest.mark.gpu
@pytest.mark.parametrize("model", ["c1", "v3"])
def test_backend_matches_the_oracle(tmp_path, oracle, model):
    """The adapter's MUL node against the CPU oracle: the reference's gate runs
    the same split on the CPU delegate and on the device and compares them
    (moe-serv/gate.py:196-222); here the control is the oracle.  Layers of the
    C1 shape (one plain, one clamped at 0.75 so the clamp binds) and of the
    V3 shape (6 GB), with no budget set: the device's free memory less the
    default 1 GiB reserve holds them all.  Every device split's per-slot rows
    pass parity.check_block at 1e-3 of their RMS, and equal
    moe_forward_host's bit for bit."""
    assert os.path.exists(DRIVER), "tests/ggml_stub/_build is built by __graft_entry__.build()"
    print(f"[gpu] ggml backend adapter, {model} model, against the oracle", flush=True)
    f, err = drive("gpu", {"MOESERV_PROFILE": str(tmp_path / "prof")}, model=model, dump_dir=tmp_path, timeout=900)
    print(err, flush=True)
    m = re.search(r"residency budget (\d+) MB \((\d+) MB free, (\d+) MB held back\)", err)
    assert m and int(m.group(3)) == 1024 and int(m.group(1)) == int(m.group(2)) - 1024, err
    H, F, E, K = f["H"], f["F"], f["E"], f["K"]
    tags = [k[:-len("_T")] for k in f if k.endswith("_T")]
    assert len(tags) >= 2
    for tag in tags:
        assert f[tag + "_status"] == 0 and f[tag + "_cpu"] == 0 and f[tag + "_bit_exact"] == 1, tag
        assert f[tag + "_dumped"] == 1, tag
        T, lid = f[tag + "_T"], f[tag + "_layer"]
        clamp = f[f"l{lid}_clamp_x1e6"] / 1e6
        x = np.fromfile(tmp_path / f"{tag}.x.f32", np.float32).reshape(T, H)
        ids = np.fromfile(tmp_path / f"{tag}.ids.i32", np.int32).reshape(T, K)
        wts = np.fromfile(tmp_path / f"{tag}.wts.f32", np.float32).reshape(T, K)
        out = np.fromfile(tmp_path / f"{tag}.out.f32", np.float32).reshape(T, K, H)
        h = np.fromfile(tmp_path / f"{tag}.h.f32", np.float32)
        shape = wl.LayerShape(hidden=H, ffn=F, n_expert=E, n_used=K, has_shared=False, route_mode=wl.ROUTE_SIGMOID,
                              clamp=clamp)
        L = oracle.OracleLayer.generated(f["seed"], lid, H, F, E, K, experts=sorted(set(ids.ravel().tolist())),
                                         shared=False, clamp=clamp, e_lo=f[f"l{lid}_e_lo"],
                                         e_span=f[f"l{lid}_e_span"])
        if clamp:  # the clamp binds: the unclamped h is far larger
            free = oracle.OracleLayer.generated(f["seed"], lid, H, F, E, K, experts=sorted(set(ids.ravel().tolist())),
                                                shared=False, e_lo=f[f"l{lid}_e_lo"], e_span=f[f"l{lid}_e_span"])
            assert np.abs(free.forward(x, ids, wts, taps=True)["h"]).max() > 4 * np.abs(
                L.forward(x, ids, wts, taps=True)["h"]).max()
        check_block(oracle, L, DumpedTaps(h), shape, x, ids, wts, out, f"adapter {tag}", per_slot=True)
    assert f"{len(tags)} splits on the device, 0 fell back" in err
    rows, header = read_profile(tmp_path)
    assert header == PROFILE_COLUMNS and len(rows) == len(tags) and all(r["dev"] == "0" for r in rows)


@pytest.mark.gpu
def test_backend_reserve_above_free_memory_keeps_every_layer_on_the_cpu():
    """MOESERV_RESERVE_MB above the device's free memory leaves a budget of 0:
    every split runs on the CPU delegate (refused at residency, then
    remembered), none is skipped."""
    print("[gpu] ggml backend adapter, reserve above free memory", flush=True)
    f, err = drive("gpu", {"MOESERV_RESERVE_MB": str(1 << 30)})
    assert re.search(r"residency budget 0 MB \(\d+ MB free, 1073741824 MB held back\)", err), err
    for r in ("l3_t1", "l3_t3", "l4_clamp_t2", "l5_symclamp_a", "l5_symclamp_b", "l6_a", "l6_b"):
        assert f[r + "_status"] == 0 and f[r + "_cpu"] == 1 and f[r + "_sentinel"] == 1, r
    assert "0 splits on the device, 7 fell back" in err
