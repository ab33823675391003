"""bench.py's command-line contract on CPU: one GPU only (--gpus N > 1 exits
with a message), and the workloads it accepts."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=REPO)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_workload_choices():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=300, cwd=REPO)
    assert r.returncode == 0
    for w in ("c1", "c2", "c3", "c4", "c5", "boundary", "server"):
        assert w in r.stdout


def test_trace_gaps_reads_a_kernel_trace(tmp_path):
    """--trace-gaps: the idle time between the replays' expert kernels per
    layer call, from a rocprofv3 kernel_trace.csv (synthetic here: 3 layer
    calls of gate/up 20 us + down 10 us with 1 us gaps, after an unrelated
    kernel and a long pause)."""
    import json
    head = ('"Kind","Agent_Id","Queue_Id","Stream_Id","Thread_Id","Dispatch_Id","Kernel_Id","Kernel_Name",'
            '"Correlation_Id","Start_Timestamp","End_Timestamp"\n')
    rows, t = [], 0
    rows.append(("k_generate_blocks(int)", 0, 5_000))
    rows.append(("k_gate_up_bal2(int)", 1_000_000, 1_020_000))  # eager, far from the replays
    t = 5_000_000
    for _ in range(3):
        rows.append(("k_gate_up_bal2(int)", t, t + 20_000))
        rows.append(("void k_down_span<16>(int)", t + 21_000, t + 31_000))  # a template instance's name
        t += 32_000
    p = tmp_path / "k.csv"
    p.write_text(head + "".join(f'"KERNEL_DISPATCH","Agent 1",1,0,1,{i},1,"{n}",{i},{a},{b}\n'
                                for i, (n, a, b) in enumerate(rows)))
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--trace-gaps", str(p)], capture_output=True,
                       text=True, timeout=300, cwd=REPO)
    assert r.returncode == 0, r.stderr
    line = json.loads(r.stdout)
    assert line["layer_calls"] == 3
    assert abs(line["value"] - 5.0 / 3) < 1e-3      # gaps: 1 us inside each call, 1 us between calls
    assert abs(line["kernel_us_per_layer"] - 30.0) < 1e-6


def test_host_cpus_reports_the_usable_count():
    sys.path.insert(0, REPO)
    import bench
    hc = bench.host_cpus()
    assert 1 <= hc["usable"] <= hc["affinity"] <= hc["visible"]
    assert isinstance(hc["model"], str)
