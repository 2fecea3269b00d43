"""CPU checks of bench.py's contract: the one-GPU refusal, the CPU-baseline
fields, and the dominant kernel's HBM traffic read from the committed
rocprofv3 summary (no GPU needed for any of them)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert r.stdout.strip() == "" or not r.stdout.lstrip().startswith("{"), "no JSON line for N > 1"


def test_cpu_baseline_fields():
    b = bench.cpu_baseline(0.2)
    assert set(b) >= {"value", "unit", "cores", "kind", "sample", "cpu"}
    assert b["kind"] == "port" and b["cores"] == 1 and b["unit"] == "GB/s"
    assert b["value"] > 0 and isinstance(b["cpu"], str) and b["cpu"]


def test_cpu_baseline_all_cores_bounded():
    b = bench.cpu_baseline_all_cores(0.2)
    assert 1 <= b["cores"] <= 16 and b["value"] > 0 and b["kind"] == "port"


def test_traffic_from_committed_profile():
    t = bench.read_traffic(bench.DOMINANT)
    assert t is not None, "profiles/swiglu_config1_pmc.txt missing or without traffic_bytes_per_launch"
    alg = bench.BYTES[bench.DOMINANT]
    assert abs(t / alg - 1) < 0.02, (t, alg)


def test_step_bytes_are_the_configs1_shapes():
    # gather: out 512 x 4096 fp32 + 512 Q8_0 rows of 4096 (128 blocks x 34 B) + 512 int32 ids
    assert bench.BYTES["gather"] == 512 * 4096 * 4 + 512 * 128 * 34 + 512 * 4
    # norm -> RoPE: x in + q out (512 x 4096 fp32), w, K in + out (512 x 1024)
    assert bench.BYTES["norm_rope"] == 2 * 512 * 4096 * 4 + 4096 * 4 + 2 * 512 * 1024 * 4
    assert bench.BYTES["swiglu"] == 3 * 512 * 14336 * 4
