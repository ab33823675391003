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
  per-split phase CSV of MOESERV_PROFILE.

ABI fidelity to ggml 0.18.1 itself stays unverified: no ggml headers are in
this image.
"""
import csv
import glob
import json
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STUB = os.path.join(REPO, "tests", "ggml_stub")
DRIVER = os.path.join(STUB, "_build", "drive_backend")
ADAPTER = os.path.join(STUB, "_build", "libggml-moe.so")


def build():
    subprocess.run(["make", "-s", "-C", STUB], check=True, capture_output=True, text=True)


def drive(mode, env_extra=None, timeout=300):
    env = dict(os.environ)
    for k in ("MOESERV_DISABLE", "MOESERV_TP_BUDGET_MB", "MOESERV_PROFILE"):
        env.pop(k, None)
    env.update(env_extra or {})
    r = subprocess.run([DRIVER, ADAPTER, mode], capture_output=True, text=True, env=env, timeout=timeout)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1]), r.stderr


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
    rows = list(csv.DictReader(open(glob.glob(str(tmp_path / "prof-*.csv"))[0])))
    assert len(rows) == len(runs) and all(r["dev"] == "-1" for r in rows)


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
    rows = list(csv.DictReader(open(glob.glob(str(tmp_path / "prof-*.csv"))[0])))
    dev_rows = [r for r in rows if r["dev"] == "0"]
    assert len(rows) == 7 and len(dev_rows) == 3
    for r in dev_rows:
        assert float(r["compute_us"]) > 0 and float(r["upload_us"]) > 0 and float(r["read_us"]) > 0
        assert 1 <= int(r["n_exp_loads"]) <= 16
