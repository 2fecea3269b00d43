"""GPU parity of fence_gemv_q6k / fence_gemv_q6k_bias (every projection of a
decode step, src/model/qwen3.cu:281-337) against the oracle, through the C ABI.

Tolerance (fp32 dot products): per row
    |y - y_oracle| <= GEMV_TOL * sum_j |W_rj| |x_j|,   GEMV_TOL = 1e-5,
plus, with a bias, one fp32 rounding of the final add.  The reference's own
test vectors (tests/test_q6k_dot.cu TC1-TC6, tests/test_gemv_q6k.cu synthetic
64x256 and 128x512, committed in tests/golden/q6k_reference_tests.npz) must
also pass the reference's looser bars (atol 1e-2 / rtol 1e-3 for a block dot,
atol 0.5 / rtol 5e-3 per GEMV row).  Cases whose arithmetic is exact (a unit
vector picks a column; x -> 2x) are compared bit for bit.
"""
import os

import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod
from oracle_py import make_q6k_matrix, q6k_dequant_numpy

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def run_q6k(W, x16, M, K, bias=None):
    torch = torch_mod()
    y = torch.full((max(M, 1),), float("nan"), dtype=torch.float32, device="cuda")
    LIVE.append(y)
    Wd, xd = dev(W), dev(np.asarray(x16, np.uint16).view(np.int16))
    if bias is None:
        F.gemv_q6k(Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), M, K, stream())
    else:
        F.gemv_q6k_bias(Wd.data_ptr(), xd.data_ptr(), dev(bias).data_ptr(), y.data_ptr(), M, K, stream())
    return host(y)[:M]


def abs_scale(W, x16, K):
    ax = np.abs(np.asarray(x16, np.uint16).view(np.float16).astype(np.float64))
    out = np.empty(W.shape[0])
    for r0 in range(0, W.shape[0], 2048):
        out[r0:r0 + 2048] = np.abs(q6k_dequant_numpy(W[r0:r0 + 2048], K)) @ ax
    return out


def assert_close(got, ref, scale, what, slack=None):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{what}: NaN rows differ"
    fin = np.isfinite(ref)
    bound = GEMV_TOL * scale[fin] + (0 if slack is None else slack[fin])
    err = np.abs(got[fin] - ref[fin])
    assert np.all(err <= bound), (f"{what}: {int((err > bound).sum())} rows beyond the bar; worst "
                                  f"err/scale {np.max(err / np.maximum(scale[fin], 1e-300)):.3g}")


def rand_x(rng, K, std=1.0):
    return (std * rng.standard_normal(K)).astype(np.float16).view(np.uint16)


def test_reference_dot_vectors(oracle):
    """The reference's six Q6_K block tests, as 1 x 256 GEMVs."""
    fx = np.load(os.path.join(GOLDEN, "q6k_reference_tests.npz"))
    for t, (blk, x) in enumerate(zip(fx["dot_blocks"], fx["dot_x"])):
        got = run_q6k(blk.reshape(1, 210), x, 1, 256)[0]
        exp = fx["dot_expected"][t]
        err = abs(got - exp)
        assert err < 1e-2 or err / max(abs(exp), 1e-6) < 1e-3, f"TC{t + 1}: {got} vs {exp} (reference bar)"
        assert_close([got], [oracle.q6k_dot(blk, x)], abs_scale(blk.reshape(1, 210), x, 256), f"TC{t + 1}")
        closed = fx["dot_closed"][t]
        if not np.isnan(closed):
            assert got == np.float32(closed), f"TC{t + 1}: closed form {closed}, got {got}"


@pytest.mark.parametrize("name,K", [("small", 256), ("multi", 512)])
def test_reference_gemv_vectors(oracle, name, K):
    fx = np.load(os.path.join(GOLDEN, "q6k_reference_tests.npz"))
    W, x, exp = fx[f"{name}_W"], fx[f"{name}_x"], fx[f"{name}_expected"]
    got = run_q6k(W, x, W.shape[0], K)
    err = np.abs(got - exp)
    assert np.all((err <= 0.5) | (err / np.maximum(np.abs(exp), 1.0) <= 5e-3)), "reference GEMV bar"
    assert_close(got, oracle.gemv_q6k(W, x), abs_scale(W, x, K), f"reference {name}")


@pytest.mark.parametrize("M,K", [
    (4096, 2560),   # Qwen3-4B q projection (10 blocks per row)
    (1024, 2560),   # k / v
    (2560, 4096),   # o projection (16 blocks)
    (9728, 2560),   # gate / up
    (2560, 9728),   # down (38 blocks: four waves per row)
    (4096, 14336),  # Llama-3-8B down (56 blocks)
    (24, 5120),     # 20 blocks: two waves per row
])
def test_gemv_q6k_model_shapes(oracle, M, K):
    rng = np.random.default_rng(M + K)
    W = make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K)
    got = run_q6k(W, x, M, K)
    assert_close(got, oracle.gemv_q6k(W, x), abs_scale(W, x, K), f"q6k {M}x{K}")
    x2 = (np.asarray(x, np.uint16).view(np.float16) * np.float16(2)).view(np.uint16)
    assert np.array_equal(run_q6k(W, x2, M, K), 2 * got), "y(2x) != 2 y(x)"


@pytest.mark.parametrize("M,K", [(1, 256), (7, 2560), (13, 768), (3, 17920), (64, 256)])
def test_gemv_q6k_edge_shapes(oracle, M, K):
    """M * K/256 not a multiple of 8 (direct kernel), more than 64 blocks, one block."""
    rng = np.random.default_rng(7 * M + K)
    W = make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K)
    assert_close(run_q6k(W, x, M, K), oracle.gemv_q6k(W, x), abs_scale(W, x, K), f"q6k {M}x{K}")


@pytest.mark.parametrize("j", [0, 15, 16, 63, 64, 127, 128, 255, 256, 2559])
def test_gemv_q6k_unit_vector_selects_column(j):
    M, K = 40, 2560
    W = make_q6k_matrix(np.random.default_rng(90 + j), M, K)
    x = np.zeros(K, np.float16)
    x[j] = 1.0
    got = run_q6k(W, x.view(np.uint16), M, K)
    assert np.array_equal(got, q6k_dequant_numpy(W, K)[:, j].astype(np.float32)), "W e_j != column j"


def test_gemv_q6k_bias(oracle):
    M, K = 1024, 2560
    rng = np.random.default_rng(11)
    W = make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K)
    bias = rng.standard_normal(M).astype(np.float32)
    ref = oracle.gemv_q6k(W, x, bias)
    got = run_q6k(W, x, M, K, bias)
    assert_close(got, ref, abs_scale(W, x, K), "q6k bias", slack=2.0 ** -23 * np.abs(ref))


def test_gemv_q6k_unaligned_operands(oracle):
    """W only 2-byte aligned (direct kernel) and x 2-byte aligned."""
    torch = torch_mod()
    M, K = 16, 2560
    rng = np.random.default_rng(12)
    W = make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K)
    raw = torch.zeros(W.size + 16, dtype=torch.uint8, device="cuda")
    xbuf = torch.zeros(K + 8, dtype=torch.int16, device="cuda")
    y = torch.full((M,), float("nan"), device="cuda")
    LIVE.extend([raw, xbuf, y])
    raw[2:2 + W.size] = torch.from_numpy(W.reshape(-1)).to("cuda")
    xbuf[1:1 + K] = torch.from_numpy(x.view(np.int16)).to("cuda")
    F.gemv_q6k(raw.data_ptr() + 2, xbuf.data_ptr() + 2, y.data_ptr(), M, K, stream())
    assert_close(host(y), oracle.gemv_q6k(W, x), abs_scale(W, x, K), "q6k unaligned")
    # the same matrix 16-byte aligned but x only 2-byte aligned: staged kernel, scalar x loads
    y2 = torch.full((M,), float("nan"), device="cuda")
    LIVE.append(y2)
    F.gemv_q6k(dev(W).data_ptr(), xbuf.data_ptr() + 2, y2.data_ptr(), M, K, stream())
    assert_close(host(y2), oracle.gemv_q6k(W, x), abs_scale(W, x, K), "q6k x unaligned")


def test_gemv_q6k_nan_scale_row(oracle):
    M, K = 8, 512
    rng = np.random.default_rng(13)
    W = make_q6k_matrix(rng, M, K)
    W[3, 208:210] = np.array([0x00, 0x7E], np.uint8)  # block 0 of row 3: d = NaN
    x = rand_x(rng, K)
    got = run_q6k(W, x, M, K)
    ref = oracle.gemv_q6k(W, x)
    assert np.isnan(ref[3]) and np.isnan(got[3]) and np.isfinite(np.delete(got, 3)).all()
    assert_close(got, ref, np.nan_to_num(abs_scale(W, x, K), nan=0.0), "q6k NaN scale")
