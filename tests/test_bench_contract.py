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
    assert set(b) >= {"value", "unit", "cores", "kind", "sample", "cpu", "ops"}
    assert b["kind"] == "port" and b["cores"] == 1 and b["unit"] == "GB/s"
    assert b["value"] > 0 and b["cpu"]["model_name"]
    assert set(b["ops"]) == set(bench.BYTES) and all(v["GBps"] > 0 for v in b["ops"].values())
    assert "timed in C" in b["sample"] and "numpy" not in b["sample"]


def test_cpu_baseline_all_cores_bounded():
    b = bench.cpu_baseline_all_cores(0.2)
    assert 1 <= b["cores"] <= 16 and b["value"] > 0 and b["kind"] == "port"


def test_cpu_sample_is_an_eighth_of_each_op():
    # the sample sizes the value is scaled by: heads, rows and tokens divide evenly
    den = bench.CPU_SAMPLE_DEN
    assert bench.SM_HEADS % den == 0 and bench.T4 % den == 0


def test_traffic_from_committed_profile():
    t = bench.read_traffic()
    assert t is not None, "profiles/swiglu_config4_pmc.txt missing or without traffic_bytes_per_launch"
    alg = bench.BYTES[bench.DOMINANT]
    assert abs(t / alg - 1) < 0.02, (t, alg)


def test_step_bytes_are_the_configs4_shapes():
    # causal softmax: read keys 0..q of every query row, write all 2048 keys, 32 heads
    assert bench.BYTES["softmax"] == 32 * (2048 * 2049 // 2) * 4 + 32 * 2048 * 2048 * 4 == 805437440
    assert bench.BYTES["swiglu"] == 3 * 8192 * 14336 * 4 == 1409286144
    # interleaved RoPE in place on Q [8192 x 32 x 128] and K [8192 x 8 x 128]
    assert bench.BYTES["rope"] == 2 * 8192 * 40 * 128 * 4 == 335544320
    assert bench.STEP_BYTES == 805437440 + 1409286144 + 335544320


def test_attainable_is_cold_floor_plus_bytes_at_peak():
    """attainable_us = the op's own cold chain floor + its bytes at 8 TB/s;
    frac_of_attainable = attainable / measured."""
    res = [{"config": "floor", "key": "gather_one_id_cold", "us_mean": 4.0, "bytes": 16_000},
           {"config": "floor", "key": "swiglu_one_float4_cold", "us_mean": 3.5, "bytes": 48},
           {"config": 1, "key": "gather", "us_mean": 5.0, "bytes": 8_000_000},
           {"config": 1, "key": "swiglu", "us_mean": 14.0, "bytes": 88_000_000},
           {"config": 1, "key": "norm_rope", "us_mean": 6.0, "bytes": 21_000_000},  # its floor not measured
           {"config": 2, "key": "swiglu", "us_mean": 90.0, "bytes": 600_000_000}]
    bench.attainable(res)
    g = res[2]["attainable"]
    assert g["floor"] == "gather_one_id_cold" and g["attainable_us"] == 5.0 and g["frac_of_attainable"] == 1.0
    s = res[3]["attainable"]
    assert s["attainable_us"] == 3.5 + 11.0 and s["frac_of_attainable"] == round(14.5 / 14.0, 4)
    assert "attainable" not in res[4] and "attainable" not in res[5]


def test_softmax_mix_ceiling_moves_the_softmax_bytes():
    """The causal softmax's ceiling streams: in place over the unmasked scores
    (read + write), zeros over the masked ones (write) -- its own bytes."""
    n_rw, n_w = bench.causal_softmax_mix()
    assert 8 * n_rw + 4 * n_w == bench.BYTES["softmax"]
    assert n_rw % 4 == 0 and n_w % 4 == 0  # float4 streams, the second 16-byte aligned


def test_step_ceiling_is_the_harmonic_combination():
    assert bench.step_ceiling_gbps({op: 5000.0 for op in bench.BYTES}) == 5000.0
    rates = {"softmax": 6400.0, "swiglu": 6800.0, "rope": 6500.0}
    t = sum(bench.BYTES[op] / (r * 1e9) for op, r in rates.items())
    assert abs(bench.step_ceiling_gbps(rates) - bench.STEP_BYTES / t / 1e9) < 0.1
    assert min(rates.values()) < bench.step_ceiling_gbps(rates) < max(rates.values())
