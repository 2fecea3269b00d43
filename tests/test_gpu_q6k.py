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


@pytest.mark.parametrize("nb", [6, 10, 13, 14, 16, 17, 21, 24, 27, 32, 33, 40, 48, 49, 60, 64, 65, 70])
def test_direct_kernel_sums_in_the_staged_order(nb):
    """The direct kernel (weights only 2-byte aligned) must give every row the
    staged kernel's bits: rows of more than 16 blocks are summed per segment
    of 2 or 4 waves there, so the direct kernel sums in the same segments."""
    torch = torch_mod()
    K, M = 256 * nb, 64
    rng = np.random.default_rng(nb)
    W = make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K)
    staged = run_q6k(W, x, M, K)
    raw = torch.zeros(W.size + 16, dtype=torch.uint8, device="cuda")
    raw[2:2 + W.size] = dev(W.reshape(-1))
    y = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
    LIVE.extend([raw, y])
    F.gemv_q6k(raw.data_ptr() + 2, dev(x.view(np.int16)).data_ptr(), y.data_ptr(), M, K, stream())
    assert np.array_equal(host(y).view(np.uint32), staged.view(np.uint32)), "direct differs from staged"


# Multi launches of rows whose last pass holds two blocks (6, 10, 14), small
# and empty matrices among them, biases on some: each row must have the bits
# the direct kernel (2-byte aligned copies of the same matrices) gives it,
# its bias included, and only its own output may be written.
@pytest.mark.parametrize("shapes,nb", [((4, 12, 8), 10), ((8,), 10), ((4,), 6), ((12, 4), 14), ((4096, 1024, 1024), 10),
                                       ((1028, 4, 0, 8), 10)])
def test_multi_rows_equal_the_direct_kernel(oracle, shapes, nb):
    torch = torch_mod()
    K = 256 * nb
    rng = np.random.default_rng(sum(shapes) + nb)
    Ws = [make_q6k_matrix(rng, M, K) if M else np.zeros((0, nb * 210), np.uint8) for M in shapes]
    bs = [rng.standard_normal(M).astype(np.float32) if i % 2 == 0 else None for i, M in enumerate(shapes)]
    x = rand_x(rng, K)
    got = run_q6k_multi([W if W.size else None for W in Ws], x, list(shapes), K, bs)
    for i, (W, M) in enumerate(zip(Ws, shapes)):
        if M == 0:
            continue
        raw = torch.zeros(W.size + 16, dtype=torch.uint8, device="cuda")
        raw[2:2 + W.size] = dev(W.reshape(-1))
        y = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
        LIVE.extend([raw, y])
        F.gemv_q6k(raw.data_ptr() + 2, dev(x.view(np.int16)).data_ptr(), y.data_ptr(), M, K, stream())
        ref = host(y) + (bs[i] if bs[i] is not None else 0)
        assert np.array_equal(got[i].view(np.uint32), ref.astype(np.float32).view(np.uint32)), f"matrix {i}"
        assert_close(got[i] - (bs[i] if bs[i] is not None else 0), oracle.gemv_q6k(W, x), abs_scale(W, x, K),
                     f"two-row {i}")


@pytest.mark.parametrize("shapes,K", [((176, 73, 25, 103), 6912), ((248, 5), 5376), ((80, 139, 79), 9984),
                                      ((59, 43, 76, 99), 9728)])
def test_multi_with_a_matrix_that_cannot_be_staged(oracle, shapes, K):
    """One matrix of the launch has M * nb not a multiple of 8, so the whole
    launch runs the direct kernel while the others, alone, are staged: each
    must still equal its own launch bit for bit."""
    rng = np.random.default_rng(sum(shapes) + K)
    Ws = [make_q6k_matrix(rng, M, K) for M in shapes]
    x = rand_x(rng, K)
    got = run_q6k_multi(Ws, x, list(shapes), K)
    for i, (W, M) in enumerate(zip(Ws, shapes)):
        assert np.array_equal(got[i].view(np.uint32), run_q6k(W, x, M, K).view(np.uint32)), f"matrix {i}"
        assert_close(got[i], oracle.gemv_q6k(W, x), abs_scale(W, x, K), f"multi {i}")


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


# ------------------------------------------------- multi-matrix and gate/up + SwiGLU launches

def run_q6k_multi(Ws, x16, Ms, K, biases=None):
    torch = torch_mod()
    ys = [torch.full((max(M, 1),), float("nan"), dtype=torch.float32, device="cuda") for M in Ms]
    LIVE.extend(ys)
    xd = dev(np.asarray(x16, np.uint16).view(np.int16))
    wp = [dev(W).data_ptr() if W is not None else None for W in Ws]
    bp = None if biases is None else [None if b is None else dev(b).data_ptr() for b in biases]
    F.gemv_q6k_multi(wp, xd.data_ptr(), [y.data_ptr() for y in ys], Ms, K, bp, stream())
    return [host(y)[:M] for y, M in zip(ys, Ms)]


@pytest.mark.parametrize("shapes,K", [
    ((4096, 1024, 1024), 2560),        # Qwen3-4B q, k, v
    ((4096, 1024, 1024), 4096),        # Llama-3-8B q, k, v
    ((512, 256, 256, 8), 5120),        # four matrices, two waves per row
    ((7, 13, 3), 768),                 # row counts with M * nb % 8 != 0: direct kernel
    ((64, 0, 32), 2560),               # an empty matrix in the middle
])
def test_gemv_q6k_multi_equals_separate_launches(oracle, shapes, K):
    rng = np.random.default_rng(sum(shapes) + K)
    Ws = [make_q6k_matrix(rng, M, K) if M else np.zeros((0, K // 256 * 210), np.uint8) for M in shapes]
    x = rand_x(rng, K)
    got = run_q6k_multi([W if W.size else None for W in Ws], x, list(shapes), K)
    for i, (W, M) in enumerate(zip(Ws, shapes)):
        if M == 0:
            continue
        assert np.array_equal(got[i], run_q6k(W, x, M, K)), f"matrix {i}: differs from its own launch"
        assert_close(got[i], oracle.gemv_q6k(W, x), abs_scale(W, x, K), f"multi {i}")


BIG_ROWS = 8200  # more rows than the four-wave form takes (8192)


@pytest.mark.parametrize("K", [3328, 3584, 3840, 4096])
@pytest.mark.parametrize("M", [8, 256, 2560])
def test_few_long_rows_equal_the_one_wave_layout(oracle, K, M):
    """Launches of at most 8192 rows of 13-16 blocks run the one-wave layout
    spread over four waves per row; a multi launch with a second matrix of
    BIG_ROWS rows runs the one-wave layout itself.  Every row must agree bit
    for bit, biased or not, including x of mixed magnitudes and an all-zero
    x."""
    rng = np.random.default_rng(K + M)
    W = make_q6k_matrix(rng, M, K)
    big = make_q6k_matrix(rng, BIG_ROWS, K)
    b = rng.standard_normal(M).astype(np.float32)
    mag = np.exp(rng.uniform(-6, 6, K))
    xs = [rand_x(rng, K), (rng.standard_normal(K) * mag).astype(np.float16).view(np.uint16),
          np.zeros(K, np.uint16)]
    for i, x in enumerate(xs):
        few = run_q6k(W, x, M, K)
        many = run_q6k_multi([W, big], x, [M, BIG_ROWS], K)[0]
        if i == 0:
            assert_close(few, oracle.gemv_q6k(W, x), abs_scale(W, x, K), "few long rows")
        assert np.array_equal(few.view(np.uint32), many.view(np.uint32)), \
            f"{int((few.view(np.uint32) != many.view(np.uint32)).sum())} rows differ"
        fb = run_q6k(W, x, M, K, b)
        mb = run_q6k_multi([W, big], x, [M, BIG_ROWS], K, [b, None])[0]
        assert np.array_equal(fb.view(np.uint32), mb.view(np.uint32))


def test_four_wave_threshold_is_invisible():
    """8192 rows of 16 blocks take the four-wave form, 8200 rows the one-wave
    layout: the shared rows agree bit for bit across the threshold."""
    rng = np.random.default_rng(8192)
    K = 4096
    W = make_q6k_matrix(rng, BIG_ROWS, K)
    x = rand_x(rng, K)
    below = run_q6k(W[:8192], x, 8192, K)
    above = run_q6k(W, x, BIG_ROWS, K)
    assert np.array_equal(below.view(np.uint32), above[:8192].view(np.uint32))


def test_gemv_q6k_multi_biases(oracle):
    K = 2560
    rng = np.random.default_rng(21)
    Ms = (4096, 1024, 1024)
    Ws = [make_q6k_matrix(rng, M, K) for M in Ms]
    bs = [rng.standard_normal(M).astype(np.float32) for M in Ms]
    x = rand_x(rng, K)
    got = run_q6k_multi(Ws, x, list(Ms), K, [bs[0], None, bs[2]])
    assert np.array_equal(got[0], run_q6k(Ws[0], x, Ms[0], K, bs[0]))
    assert np.array_equal(got[1], run_q6k(Ws[1], x, Ms[1], K))
    assert np.array_equal(got[2], run_q6k(Ws[2], x, Ms[2], K, bs[2]))


def run_swiglu(Wg, Wu, x16, M, K, fp32=True):
    torch = torch_mod()
    o16 = torch.full((M,), -1, dtype=torch.int16, device="cuda")
    o32 = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda") if fp32 else None
    LIVE.extend([o16, o32])
    F.gemv_q6k_swiglu_f16(dev(Wg).data_ptr(), dev(Wu).data_ptr(), dev(np.asarray(x16, np.uint16).view(np.int16))
                          .data_ptr(), o16.data_ptr(), o32.data_ptr() if fp32 else None, M, K, stream())
    return host(o16).view(np.uint16), (host(o32) if fp32 else None)


def unfused_swiglu(Wg, Wu, x16, M, K):
    torch = torch_mod()
    g = torch.from_numpy(run_q6k(Wg, x16, M, K)).to("cuda")
    u = torch.from_numpy(run_q6k(Wu, x16, M, K)).to("cuda")
    o16 = torch.zeros((M,), dtype=torch.int16, device="cuda")
    o32 = torch.zeros((M,), dtype=torch.float32, device="cuda")
    LIVE.extend([g, u, o16, o32])
    F.swiglu_f16(o16.data_ptr(), o32.data_ptr(), g.data_ptr(), u.data_ptr(), M, stream())
    return host(o16).view(np.uint16), host(o32)


@pytest.mark.parametrize("M,K", [
    (9728, 2560),   # Qwen3-4B gate/up
    (14336, 4096),  # Llama-3-8B gate/up (16 blocks)
    (1000, 5120),   # 20 blocks: two waves per row
    (256, 9728),    # 38 blocks: more than a pair's staging holds -> direct kernel
    (13, 768),      # M * nb % 8 != 0 -> direct kernel
    (1, 256),
    # ~4 rows whose fp32 act rounds onto a binary16 tie: the conversion must
    # round the fp32 value (as the unfused chain does), not the exact product
    (65536, 256),
])
def test_gemv_q6k_swiglu_equals_unfused_sequence(oracle, M, K):
    rng = np.random.default_rng(M * 7 + K)
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K, std=0.5)
    got16, got32 = run_swiglu(Wg, Wu, x, M, K)
    ref16, ref32 = unfused_swiglu(Wg, Wu, x, M, K)
    assert np.array_equal(got32.view(np.uint32), ref32.view(np.uint32)), "fp32 act differs from the unfused chain"
    assert np.array_equal(got16, ref16), "binary16 act differs from the unfused chain"
    assert np.array_equal(run_swiglu(Wg, Wu, x, M, K, fp32=False)[0], ref16)
    # and against the oracle's chain: act = silu(g) * u with g, u within the GEMV bar
    g, u = oracle.gemv_q6k(Wg, x), oracle.gemv_q6k(Wu, x)
    sg, su = abs_scale(Wg, x, K), abs_scale(Wu, x, K)
    sig = 1 / (1 + np.exp(-g.astype(np.float64)))
    # d(act) <= |d silu/dg| |u| dg + |silu(g)| du, |d silu/dg| <= 1.1
    bound = 1.1 * np.abs(u) * GEMV_TOL * sg + np.abs(g * sig) * GEMV_TOL * su + 1e-6 * np.abs(oracle.silu_mul(g, u))
    assert np.all(np.abs(got32 - oracle.silu_mul(g, u)) <= bound + 1e-30)


# Gate/up pairs of rows of at most 16 blocks take the kernel with one wave per
# output row (8-wave workgroups, the next row prefetched): every pass count
# (1-4 passes of four blocks), masked block slots, a last pass of two blocks
# shared by gate and up (nb = 6, 10, 14), fewer rows than a
# workgroup's waves, exactly one workgroup's, and row counts either side of
# the resident grid's waves, each bit-equal to the two GEMV launches and the
# SwiGLU launch it replaces.  (M * nb % 8 == 0 keeps them on the staged path.)
@pytest.mark.parametrize("nb,M", [
    (1, 8), (1, 64), (2, 4), (3, 8), (4, 2), (5, 8), (8, 1), (8, 7), (8, 9),
    (9, 8), (12, 6), (13, 8), (16, 1), (16, 3), (16, 8), (10, 4092), (10, 4100), (10, 8196),
    (6, 8), (10, 4), (14, 4), (14, 1028),
])
def test_gemv_q6k_swiglu_one_wave_pair_edges(nb, M):
    K = 256 * nb
    assert (M * nb) % 8 == 0
    rng = np.random.default_rng(nb * 1009 + M)
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K, std=0.5)
    got16, got32 = run_swiglu(Wg, Wu, x, M, K)
    ref16, ref32 = unfused_swiglu(Wg, Wu, x, M, K)
    what = f"{M} rows of {nb} blocks"
    assert np.array_equal(got32.view(np.uint32), ref32.view(np.uint32)), what + ": fp32 act"
    assert np.array_equal(got16, ref16), what + ": binary16 act"


def test_gemv_q6k_swiglu_unaligned_weights():
    """W only 2-byte aligned: the direct pair kernel."""
    torch = torch_mod()
    M, K = 40, 2560
    rng = np.random.default_rng(33)
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    x = rand_x(rng, K)
    raw = torch.zeros(2 * Wg.size + 32, dtype=torch.uint8, device="cuda")
    o16 = torch.zeros(M, dtype=torch.int16, device="cuda")
    LIVE.extend([raw, o16])
    raw[2:2 + Wg.size] = torch.from_numpy(Wg.reshape(-1)).to("cuda")
    raw[18 + Wg.size:18 + 2 * Wg.size] = torch.from_numpy(Wu.reshape(-1)).to("cuda")
    F.gemv_q6k_swiglu_f16(raw.data_ptr() + 2, raw.data_ptr() + 18 + Wg.size, dev(x.view(np.int16)).data_ptr(),
                          o16.data_ptr(), None, M, K, stream())
    assert np.array_equal(host(o16).view(np.uint16), unfused_swiglu(Wg, Wu, x, M, K)[0])
