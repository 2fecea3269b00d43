"""GPU parity of greedy argmax against the oracle's restatement of the
reference's 256-thread block (src/kernels/ops.cuh:467-505), through the C ABI:
fence_argmax (one workgroup) and fence_argmax_ws (many workgroups, partials in
a caller workspace).  Index work: every result must equal the oracle's
exactly, ties included -- the reference's tree gives a tie to the thread
i mod 256 with the smallest 8-bit bit-reversal, then to the lowest index."""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod

pytestmark = pytest.mark.gpu

ENTRIES = ["one_workgroup", "workspace"]


def run_argmax(ptr, n, entry, ws_bytes=8192):
    torch = torch_mod()
    r = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    LIVE.append(r)
    if entry == "one_workgroup":
        F.argmax(ptr, r.data_ptr(), n, stream())
    else:
        ws = torch.full((max(1, ws_bytes // 8),), -1, dtype=torch.int64, device="cuda")
        LIVE.append(ws)
        F.argmax_ws(ptr, r.data_ptr(), n, ws.data_ptr(), ws_bytes, stream())
    return int(host(r)[0])


@pytest.mark.parametrize("entry", ENTRIES)
@pytest.mark.parametrize("n,off", [(151936, 0), (128256, 0), (1001, 1), (5, 0), (0, 0), (151937, 3)])
def test_argmax(oracle, entry, n, off):
    rng = np.random.default_rng(n + 3)
    x = rng.standard_normal(n + off + 1).astype(np.float32)
    if n > 10:
        x[off + n // 3] = x[off + n // 2] = 50.0  # a tie
        x[off + 1] = np.nan                       # NaN never wins
    assert run_argmax(dev(x).data_ptr() + 4 * off, n, entry) == oracle.argmax(x[off:off + n])


@pytest.mark.parametrize("entry", ENTRIES)
@pytest.mark.parametrize("idx,want", [((1, 256), 256), ((1, 2), 2), ((0, 255), 0), ((10, 700), 700),
                                      ((256, 512), 256), ((3, 259), 3), ((127, 129), 129),
                                      ((151935, 151679), 151679), ((9, 151936 - 247), 9)])
def test_argmax_reference_tie_rule(oracle, entry, idx, want):
    """Ties the reference's tree decides, worked out by hand: maxima at 1 and
    256 give 256 (thread 0 beats thread 1), at 1 and 2 give 2 (bit-reversals
    128 and 64), two indices of one thread give the first."""
    x = np.full(151936, -1.0, np.float32)
    x[list(idx)] = 9.0
    assert oracle.argmax(x) == want
    assert run_argmax(dev(x).data_ptr(), x.size, entry) == want


@pytest.mark.parametrize("entry", ENTRIES)
@pytest.mark.parametrize("n", [151936, 1027])
@pytest.mark.parametrize("pattern", ["equal", "spread_ties", "int_ties", "tail_max", "last", "neg_inf", "nan",
                                     "below_init", "zero_signs"])
def test_argmax_patterns(oracle, entry, n, pattern):
    """Orders the reduction must not change: ties spread over many threads,
    waves and workgroups, the maximum in the scalar tail or at the end, rows
    no value of which beats the initial -1e30 (index 0), and -0 against +0
    (equal, so the tie rule decides)."""
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    if pattern == "equal":
        x[:] = 1.5
    elif pattern == "spread_ties":
        x[rng.choice(n, 40, replace=False)] = 9.0
    elif pattern == "int_ties":
        x = rng.integers(-30, 4, n).astype(np.float32)
    elif pattern == "tail_max":
        x[n - 2] = 9.0   # n % 4 == 3 for 1027: a scalar-tail element
    elif pattern == "last":
        x[n - 1] = 9.0
    elif pattern == "neg_inf":
        x[:] = -np.inf
    elif pattern == "nan":
        x[:] = np.nan
    elif pattern == "below_init":
        x[:] = -1e35
    else:
        x[:] = -1.0
        x[rng.choice(n, 30, replace=False)] = -0.0
        x[rng.choice(n, 30, replace=False)] = 0.0
    assert run_argmax(dev(x).data_ptr(), n, entry) == oracle.argmax(x)


@pytest.mark.parametrize("ws_bytes", [8, 16, 24, 1000, 8192, 1 << 20])
@pytest.mark.parametrize("off", [0, 1])
def test_argmax_ws_any_partial_count(oracle, ws_bytes, off):
    """Any number of partials (1 .. 1024) gives the same index, on the float4
    and the scalar (unaligned) path."""
    rng = np.random.default_rng(ws_bytes + off)
    n = 151936
    x = rng.integers(-50, 6, n + off).astype(np.float32)
    want = oracle.argmax(x[off:])
    assert run_argmax(dev(x).data_ptr() + 4 * off, n, "workspace", ws_bytes) == want
    assert run_argmax(dev(x).data_ptr() + 4 * off, n, "one_workgroup") == want


def test_argmax_ws_many_seeds(oracle):
    """Fifty random tie-heavy vectors of random lengths, both entry points."""
    rng = np.random.default_rng(77)
    for trial in range(50):
        n = int(rng.integers(1, 300000))
        x = rng.integers(-9, int(rng.integers(1, 9)), n).astype(np.float32)
        want = oracle.argmax(x)
        xd = dev(x)
        for entry in ENTRIES:
            assert run_argmax(xd.data_ptr(), n, entry) == want, (trial, n, entry)
