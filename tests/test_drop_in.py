"""The C++ drop-in checks: tests/drop_in/decode_layer and decode_step call the
gfx950 kernels through the reference's launcher names (include/fence/ops.hpp)
in the order src/model/qwen3.cu does, and check each output against the linked
oracle.  decode_step runs a whole Qwen3-4B-shaped decode layer (Q6_K
projections, QK-norm, RoPE, KV store, attention, epilogues) plus the LM head
and argmax, and times whole decode steps."""
import json
import os
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "drop_in")
BIN = os.path.join(HERE, "decode_layer")
STEP = os.path.join(HERE, "decode_step")


def test_drop_in_binaries_are_built():
    for b in (BIN, STEP):
        assert os.path.exists(b), "build first: python -c 'import __graft_entry__ as g; g.build()'"


def run(args, timeout=300):
    print("running", " ".join(args), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
    return r.stdout


@pytest.mark.gpu
def test_drop_in_decode_layer():
    run([BIN])


@pytest.mark.gpu
def test_drop_in_decode_step_stages():
    out = run([STEP])
    assert "PASS argmax(logits)" in out
    assert "PASS argmax over many workgroups (fence_argmax_ws)" in out


@pytest.mark.gpu
def test_drop_in_decode_step_timing():
    """Two layers at position 300: the three launch sequences run and time."""
    line = run([STEP, "--time", "2", "300"]).strip().splitlines()[-1]
    rec = json.loads(line)
    assert rec["layers"] == 2 and rec["pos"] == 300
    for k in ("us_per_token_reference_sequence", "us_per_token_fused", "us_per_token_fused_graph"):
        assert rec[k] > 0


@pytest.mark.gpu
def test_drop_in_decode_step_fused_only_timing():
    """The profiler form: the fused sequence alone, two timed tokens."""
    line = run([STEP, "--time", "2", "300", "--no-graph", "--fused-only", "--tokens", "2"]).strip().splitlines()[-1]
    rec = json.loads(line)
    assert rec["us_per_token_fused"] > 0 and rec["us_per_token_reference_sequence"] == 0


def test_drop_in_decode_step_rejects_bad_options():
    """Argument errors end before any device call (runs without a GPU)."""
    import subprocess
    if not os.path.exists(STEP):
        pytest.skip("decode_step is not built")
    for args in (["--bogus"], ["--tokens", "0"], ["70"], ["2", "5000"]):
        r = subprocess.run([STEP, "--time"] + args, capture_output=True, text=True, timeout=60)
        assert r.returncode == 2 and "usage" in r.stderr, args
