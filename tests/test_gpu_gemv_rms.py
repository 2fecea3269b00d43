"""GPU checks of the Q6_K GEMVs that compute their own input row
(fence_gemv_q6k_multi_rms, fence_gemv_q6k_swiglu_rms_f16): the layer-boundary
epilogue of src/model/qwen3.cu:267-278 and 310-325 (residual_add, rms_norm,
f32_to_f16) folded into the projection that reads it.

The bar is bit equality with the two launches it replaces:
fence_residual_rms_norm_f16 on a copy of hidden, then fence_gemv_q6k_multi /
fence_gemv_q6k_swiglu_f16 on its binary16 row -- each of which has its own
oracle parity tests.  Equality holds only if every workgroup sums the squares
in the norm kernel's order.  The rows here span e^-4..e^4 in magnitude, so the
fp32 sum depends on the order in its last bits, and across the ~130k elements
compared a one-ulp change of the scale would flip a binary16 rounding
somewhere (about one element in 8k).
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod
from oracle_py import make_q6k_matrix

pytestmark = pytest.mark.gpu

EPS = 1e-6


def row(rng, K, residual=True):
    mag = np.exp(rng.uniform(-4, 4, K))
    hid = (rng.standard_normal(K) * mag).astype(np.float32)
    res = (rng.standard_normal(K) * mag).astype(np.float32) if residual else None
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    return hid, res, w


def unfused_input(hid, res, w, K):
    """fence_residual_rms_norm_f16 on a copy of hidden: (h, x16)."""
    torch = torch_mod()
    h = dev(hid.copy())
    x16 = torch.full((K,), -1, dtype=torch.int16, device="cuda")
    LIVE.append(x16)
    F.residual_rms_norm_f16(h.data_ptr(), None if res is None else dev(res).data_ptr(), dev(w).data_ptr(), None,
                            x16.data_ptr(), 1, K, EPS, stream())
    return host(h), host(x16).view(np.uint16)


def run_q6k(W, x16, M, K):
    torch = torch_mod()
    y = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
    LIVE.append(y)
    F.gemv_q6k(dev(W).data_ptr(), dev(x16.view(np.int16)).data_ptr(), y.data_ptr(), M, K, stream())
    return host(y)


class Fused:
    """Device operands of one folded call; hid_off floats of offset misalign hidden."""

    def __init__(self, hid, res, w, K, hid_off=0):
        torch = torch_mod()
        self.raw = dev(np.concatenate([np.zeros(hid_off, np.float32), hid]))
        self.hid_ptr = self.raw.data_ptr() + 4 * hid_off
        self.res = None if res is None else dev(res)
        self.w = dev(w)
        self.hout = torch.full((K,), float("nan"), dtype=torch.float32, device="cuda")
        self.x16 = torch.full((K,), -1, dtype=torch.int16, device="cuda")
        LIVE.extend([self.hout, self.x16])
        self.rin = F.rms_input(self.hid_ptr, None if res is None else self.res.data_ptr(),
                               None if res is None else self.hout.data_ptr(), self.w.data_ptr(),
                               self.x16.data_ptr(), EPS)

    def outputs(self):
        return host(self.hout), host(self.x16).view(np.uint16)


def fused_multi(Ws, Ms, K, hid, res, w, hid_off=0):
    torch = torch_mod()
    op = Fused(hid, res, w, K, hid_off)
    ys = [torch.full((max(M, 1),), float("nan"), dtype=torch.float32, device="cuda") for M in Ms]
    LIVE.extend(ys)
    F.gemv_q6k_multi_rms([dev(W).data_ptr() if M else None for W, M in zip(Ws, Ms)], [y.data_ptr() for y in ys],
                         list(Ms), op.rin, K, stream=stream())
    return [host(y)[:M] for y, M in zip(ys, Ms)], *op.outputs()


def check_multi(Ws, Ms, K, hid, res, w, hid_off=0):
    ys, hout, x16 = fused_multi(Ws, Ms, K, hid, res, w, hid_off)
    ref_h, ref_x = unfused_input(hid, res, w, K)
    assert np.array_equal(x16, ref_x), f"x differs from the norm kernel's in {int((x16 != ref_x).sum())} elements"
    if res is not None:
        assert np.array_equal(hout.view(np.uint32), ref_h.view(np.uint32)), "hidden_out differs"
    else:
        assert np.all(np.isnan(hout)), "hidden_out written without a residual"
    for i, (W, M) in enumerate(zip(Ws, Ms)):
        if M:
            assert np.array_equal(ys[i].view(np.uint32), run_q6k(W, ref_x, M, K).view(np.uint32)), f"matrix {i}"


@pytest.mark.parametrize("Ms,K,residual", [
    ((4096, 1024, 1024), 2560, True),   # Qwen3-4B q, k, v: T 640, one float4 per lane
    ((4096, 1024, 1024), 2560, False),  # layer 0: the embedding row alone
    ((4096, 1024, 1024), 4096, True),   # Llama-3-8B shape: T 1024
    ((512, 256), 5120, True),           # two float4 per lane, two waves per row
    ((256,), 8192, True),               # the largest folded row
    ((64,), 256, True),                 # T 64: one wave's sum
    ((128, 0, 64), 1024, True),         # an empty matrix
    ((64,), 8448, True),                # 33 blocks: the two-launch path
    ((7, 13, 3), 768, True),            # M * nb % 8 != 0: norm kernel, then the direct GEMV
])
def test_multi_rms_equals_norm_then_gemv(Ms, K, residual):
    rng = np.random.default_rng(sum(Ms) + K + residual)
    Ws = [make_q6k_matrix(rng, M, K) if M else np.zeros((0, K // 256 * 210), np.uint8) for M in Ms]
    hid, res, w = row(rng, K, residual)
    check_multi(Ws, Ms, K, hid, res, w)


@pytest.mark.parametrize("K", [512, 768, 1024 + 256, 1536, 2048, 3072, 3584, 6144, 7936])
def test_multi_rms_row_lengths(K):
    """Row lengths of 2-31 blocks: every (PASSES, WPR) shape the prologue
    runs in, T from 128 to 1024 threads, one and two float4 per lane."""
    rng = np.random.default_rng(K)
    Ms = (96, 32)
    Ws = [make_q6k_matrix(rng, M, K) for M in Ms]
    hid, res, w = row(rng, K)
    check_multi(Ws, Ms, K, hid, res, w)


@pytest.mark.parametrize("K,rows", [(2560, 40), (5120, 12)])
def test_multi_rms_many_rows(K, rows):
    """Many rows through a small GEMV: the norm's order, element by element."""
    rng = np.random.default_rng(K + rows)
    Ws = [make_q6k_matrix(rng, 64, K)]
    for _ in range(rows):
        hid, res, w = row(rng, K)
        check_multi(Ws, (64,), K, hid, res, w)


def test_multi_rms_unaligned_hidden():
    """hidden only 4-byte aligned: the norm kernel's scalar form, then the GEMV."""
    K = 2560
    rng = np.random.default_rng(5)
    Ws = [make_q6k_matrix(rng, 256, K)]
    hid, res, w = row(rng, K)
    check_multi(Ws, (256,), K, hid, res, w, hid_off=1)


def run_pair(Wg, Wu, M, K, hid, res, w, fp32=True):
    torch = torch_mod()
    op = Fused(hid, res, w, K)
    o16 = torch.full((M,), -1, dtype=torch.int16, device="cuda")
    o32 = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda") if fp32 else None
    LIVE.extend([o16, o32])
    F.gemv_q6k_swiglu_rms_f16(dev(Wg).data_ptr(), dev(Wu).data_ptr(), op.rin, o16.data_ptr(),
                              o32.data_ptr() if fp32 else None, M, K, stream())
    return host(o16).view(np.uint16), (host(o32) if fp32 else None), *op.outputs()


@pytest.mark.parametrize("M,K", [
    (9728, 2560),   # Qwen3-4B gate/up
    (14336, 4096),  # Llama-3-8B gate/up
    (1000, 5120),   # two float4 per lane: a pair takes the two launches
    (40, 2560),
    (64, 9472),     # 37 blocks: the two-launch path
])
def test_swiglu_rms_equals_norm_then_pair(M, K):
    rng = np.random.default_rng(M + 3 * K)
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    hid, res, w = row(rng, K)
    got16, got32, hout, x16 = run_pair(Wg, Wu, M, K, hid, res, w)
    ref_h, ref_x = unfused_input(hid, res, w, K)
    assert np.array_equal(x16, ref_x) and np.array_equal(hout.view(np.uint32), ref_h.view(np.uint32))
    torch = torch_mod()
    r16 = torch.zeros(M, dtype=torch.int16, device="cuda")
    r32 = torch.zeros(M, dtype=torch.float32, device="cuda")
    LIVE.extend([r16, r32])
    F.gemv_q6k_swiglu_f16(dev(Wg).data_ptr(), dev(Wu).data_ptr(), dev(ref_x.view(np.int16)).data_ptr(),
                          r16.data_ptr(), r32.data_ptr(), M, K, stream())
    assert np.array_equal(got16, host(r16).view(np.uint16))
    assert np.array_equal(got32.view(np.uint32), host(r32).view(np.uint32))
    assert np.array_equal(run_pair(Wg, Wu, M, K, hid, res, w, fp32=False)[0], got16)


# The one-wave pair kernel with the norm prologue at its edges: fewer rows
# than a workgroup's waves, every pass count, no residual; bit for bit the
# norm launch followed by the pair launch on its binary16 row.
@pytest.mark.parametrize("nb,M,residual", [
    (1, 8, True), (3, 8, False), (4, 2, True), (8, 1, True), (9, 8, False), (13, 8, True),
    (16, 3, True), (10, 4100, False), (6, 8, True), (10, 4, True), (14, 4, False),
])
def test_swiglu_rms_one_wave_pair_edges(nb, M, residual):
    K = 256 * nb
    rng = np.random.default_rng(7 * M + nb)
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    hid, res, w = row(rng, K, residual)
    got16, got32, hout, x16 = run_pair(Wg, Wu, M, K, hid, res, w)
    ref_h, ref_x = unfused_input(hid, res, w, K)
    assert np.array_equal(x16, ref_x)
    if residual:
        assert np.array_equal(hout.view(np.uint32), ref_h.view(np.uint32))
    import test_gpu_q6k as q6
    ref16, ref32 = q6.run_swiglu(Wg, Wu, ref_x, M, K)
    assert np.array_equal(got16, ref16), f"{M} rows of {nb} blocks: binary16 act"
    assert np.array_equal(got32.view(np.uint32), ref32.view(np.uint32)), f"{M} rows of {nb} blocks: fp32 act"


def test_rms_input_rejects_overlap_and_missing_outputs():
    torch = torch_mod()
    K = 512
    rng = np.random.default_rng(9)
    W = dev(make_q6k_matrix(rng, 8, K))
    y = torch.zeros(8, dtype=torch.float32, device="cuda")
    buf = torch.zeros(4 * K, dtype=torch.float32, device="cuda")
    x16 = torch.zeros(K, dtype=torch.int16, device="cuda")
    LIVE.extend([y, buf, x16])
    b = buf.data_ptr()
    hid, res, hout, w = b, b + 4 * K, b + 8 * K, b + 12 * K
    L = F.lib()
    n1 = lambda v: (F.ctypes.c_void_p * 1)(v)  # noqa: E731
    M1 = (F.ctypes.c_int * 1)(8)

    def st(rin, k=K):
        return L.fence_gemv_q6k_multi_rms(1, n1(W.data_ptr()), n1(y.data_ptr()), None, M1, F.ctypes.byref(rin), k,
                                          stream())

    assert st(F.rms_input(hid, res, hout, w, x16.data_ptr(), EPS)) == 0
    assert st(F.rms_input(hid, res, hid, w, x16.data_ptr(), EPS)) == F.EINVAL       # in place
    assert st(F.rms_input(hid, res, res + 4, w, x16.data_ptr(), EPS)) == F.EINVAL   # overlaps residual
    assert st(F.rms_input(hid, res, None, w, x16.data_ptr(), EPS)) == F.EINVAL      # sum has nowhere to go
    assert st(F.rms_input(hid, res, hout, w, None, EPS)) == F.EINVAL                # no x
    assert st(F.rms_input(hid, res, hout, w, hid + 2 * K, EPS)) == F.EINVAL        # x inside hidden
    assert st(F.rms_input(hid, res, hout, w, x16.data_ptr(), EPS), k=0) == F.EINVAL
    assert st(F.rms_input(hid, None, None, w, x16.data_ptr(), EPS)) == 0           # no residual: no sum
    torch.cuda.synchronize()
