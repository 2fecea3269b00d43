"""The C++ drop-in check: tests/drop_in/decode_layer calls the gfx950 kernels
through the reference's launcher names (include/fence/ops.hpp) in the order
src/model/qwen3.cu does, and checks each output against the linked oracle."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "drop_in", "decode_layer")


def test_drop_in_binary_is_built():
    assert os.path.exists(BIN), "build first: python -c 'import __graft_entry__ as g; g.build()'"


@pytest.mark.gpu
def test_drop_in_decode_layer():
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
