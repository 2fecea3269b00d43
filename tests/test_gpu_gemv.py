"""GPU parity of fence_gemv_q8_0 (y = W x over a Q8_0 matrix, the tied LM
head of src/model/qwen3.cu:261) against the oracle, through the C ABI.

Tolerance (fp32 dot products): per row
    |y - y_oracle| <= GEMV_TOL * sum_j |W_rj| |x_j|,   GEMV_TOL = 1e-5,
the natural error scale of a K-term fp32 dot product (its forward error bound
is proportional to it; 1e-5 is about 84 ulp of fp32 at that scale).  NaN and
infinity positions and signs must match exactly.  Cases whose products and
sums are exact (a unit vector selects one column; scaling x by 2) are
compared bit for bit.
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, normal, stream, torch_mod
from oracle_checks import q8_0_kat_table
from oracle_py import make_q8_0_table, q8_0_dequant_numpy

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5


def abs_scale(table, x, K, chunk=4096):
    """Per row sum_j |W_rj| |x_j| in float64, from numpy's independent dequant."""
    ax = np.abs(np.asarray(x, np.float64))
    out = np.empty(table.shape[0], np.float64)
    for r0 in range(0, table.shape[0], chunk):
        ids = np.arange(r0, min(r0 + chunk, table.shape[0]))
        with np.errstate(invalid="ignore"):
            out[ids] = np.abs(q8_0_dequant_numpy(table, ids, K).astype(np.float64)) @ ax
    return out


def run_gemv(table, x, M, K, y_fill=np.nan):
    torch = torch_mod()
    W = dev(table)
    xd = dev(x)
    y = torch.full((max(M, 1),), y_fill, dtype=torch.float32, device="cuda")
    LIVE.append(y)
    F.gemv_q8_0(W.data_ptr(), xd.data_ptr(), y.data_ptr(), M, K, stream())
    return host(y)[:M]


def assert_gemv_close(got, ref, scale, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{what}: NaN rows differ"
    inf_g, inf_r = np.isinf(got), np.isinf(ref)
    assert np.array_equal(inf_g, inf_r), f"{what}: infinite rows differ"
    assert np.array_equal(np.sign(got[inf_g]), np.sign(ref[inf_r])), f"{what}: infinity signs differ"
    fin = np.isfinite(ref)
    err = np.abs(got[fin] - ref[fin])
    bound = GEMV_TOL * scale[fin]
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} rows beyond {GEMV_TOL:g} * sum|w x|; worst "
                           f"err/scale {np.max(err / np.maximum(scale[fin], 1e-300)):.3g}")
    return float(np.max(err / np.maximum(scale[fin], 1e-300))) if fin.any() else 0.0


@pytest.mark.parametrize("M,K,seed", [
    (151936, 2560, 1),   # Qwen3-4B tied LM head (configs[0] table shape)
    (128256, 4096, 2),   # Llama-3-8B LM head shape (configs[1] table shape)
])
def test_gemv_q8_0_lm_head_shapes(oracle, M, K, seed):
    rng = np.random.default_rng(seed)
    table = make_q8_0_table(rng, M, K)
    x = normal(rng, K)
    got = run_gemv(table, x, M, K)
    ref = oracle.gemv_q8_0(table, x)
    worst = assert_gemv_close(got, ref, abs_scale(table, x, K), f"gemv {M}x{K}")
    print(f"gemv {M}x{K}: worst err / sum|w x| = {worst:.3g}")
    # size-independent property at full size: scaling x by 2 scales y by 2 exactly
    got2 = run_gemv(table, 2 * x, M, K)
    assert np.array_equal(got2, 2 * got), f"gemv {M}x{K}: y(2x) != 2 y(x)"


@pytest.mark.parametrize("M,K", [
    (1, 32), (3, 64), (2, 96), (65, 480), (257, 512), (1000, 2560), (64, 4096),
    (33, 5120), (17, 8192),
    (9, 8224), (5, 16384),  # beyond 8192 columns: x re-read per row
])
def test_gemv_q8_0_shapes(oracle, M, K):
    rng = np.random.default_rng(1000 * M + K)
    table = make_q8_0_table(rng, M, K)
    x = normal(rng, K)
    got = run_gemv(table, x, M, K)
    assert_gemv_close(got, oracle.gemv_q8_0(table, x), abs_scale(table, x, K), f"gemv {M}x{K}")


@pytest.mark.parametrize("j", [0, 7, 8, 31, 32, 2559])
def test_gemv_q8_0_unit_vector_selects_column(j):
    """W e_j is column j of the dequantised matrix, exactly (one nonzero product)."""
    M, K = 300, 2560
    rng = np.random.default_rng(40 + j)
    table = make_q8_0_table(rng, M, K)
    x = np.zeros(K, np.float32)
    x[j] = 1.0
    got = run_gemv(table, x, M, K)
    col = q8_0_dequant_numpy(table, np.arange(M), K)[:, j]
    assert np.array_equal(got, col), "W e_j differs from the dequantised column"


def test_gemv_q8_0_special_scales(oracle):
    """Blocks with zero, subnormal, max-finite, infinite and NaN fp16 scales and
    int8 extremes (-128, 127): the non-finite rows follow d * block_sum."""
    table, K = q8_0_kat_table()
    M = table.shape[0]
    x = normal(np.random.default_rng(5), K)
    got = run_gemv(table, x, M, K)
    ref = oracle.gemv_q8_0(table, x)
    assert np.isnan(ref).any() and np.isinf(ref).any()
    assert_gemv_close(got, ref, abs_scale(table, x, K), "gemv special scales")


def test_gemv_q8_0_zero_columns_writes_zeros():
    torch = torch_mod()
    y = torch.full((7,), float("nan"), device="cuda")
    LIVE.append(y)
    dummy = dev(np.zeros(4, np.float32))
    F.gemv_q8_0(dummy.data_ptr(), dummy.data_ptr(), y.data_ptr(), 7, 0, stream())
    assert np.array_equal(host(y), np.zeros(7, np.float32))


def test_gemv_q8_0_unaligned_operands(oracle):
    """W only 2-byte aligned (block_q8_0's own alignment), x and y 4-byte aligned."""
    torch = torch_mod()
    M, K = 130, 2560
    rng = np.random.default_rng(77)
    table = make_q8_0_table(rng, M, K)
    x = normal(rng, K)
    raw = torch.zeros(table.size + 16, dtype=torch.uint8, device="cuda")
    xbuf = torch.zeros(K + 8, dtype=torch.float32, device="cuda")
    ybuf = torch.full((M + 8,), float("nan"), device="cuda")
    LIVE.extend([raw, xbuf, ybuf])
    raw[2:2 + table.size] = torch.from_numpy(table.reshape(-1)).to("cuda")
    xbuf[1:1 + K] = torch.from_numpy(x).to("cuda")
    F.gemv_q8_0(raw.data_ptr() + 2, xbuf.data_ptr() + 4, ybuf.data_ptr() + 12, M, K, stream())
    got = host(ybuf)[3:3 + M]
    assert_gemv_close(got, oracle.gemv_q8_0(table, x), abs_scale(table, x, K), "gemv unaligned")
    assert np.isnan(host(ybuf)[:3]).all() and np.isnan(host(ybuf)[3 + M:]).all(), "wrote outside y"
