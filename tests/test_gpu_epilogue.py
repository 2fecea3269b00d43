"""GPU parity of the decode-step epilogue ops through the C ABI: residual add,
binary32 <-> binary16 conversion, the fused residual -> RMSNorm -> binary16
layer boundary, and SwiGLU -> binary16.

Bars: the residual sum and the conversions are exact (bit for bit against the
oracle / numpy; a NaN converts to some NaN).  Normalised and SwiGLU rows are
fp32 within 1e-5 per row of the oracle.  A binary16 output must be exactly
the round-to-nearest-even of the kernel's own fp32 result (checked when both
are written) and, against the oracle, within half a binary16 ulp of the
oracle's fp32 value plus that fp32 tolerance.
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, TOL, assert_bits_equal, assert_rows_close, dev, host, normal, stream, torch_mod
from oracle_checks import f32_patterns

pytestmark = pytest.mark.gpu


def empty(shape, dtype):
    torch = torch_mod()
    t = torch.full(shape, 0, dtype=dtype, device="cuda")
    LIVE.append(t)
    return t


def f16_vs_oracle(got16, ref32, row_len, what):
    """got16 (uint16 bits) against the oracle's fp32 values."""
    g = np.asarray(got16, np.uint16).view(np.float16).astype(np.float64).reshape(-1, row_len)
    r = np.asarray(ref32, np.float64).reshape(-1, row_len)
    bound = 2.0 ** -11 * np.abs(r) + TOL * np.max(np.abs(r), axis=1, keepdims=True) + 2.0 ** -25
    bad = np.abs(g - r) > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} binary16 values beyond half an ulp + {TOL:g}"


def test_f32_to_f16_bit_exact(oracle):
    torch = torch_mod()
    x = f32_patterns(np.random.default_rng(3)).view(np.float32)
    out = empty((x.size,), torch.int16)
    F.f32_to_f16(out.data_ptr(), dev(x).data_ptr(), x.size, stream())
    got = host(out).view(np.uint16)
    ref = oracle.f32_to_f16(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan]), "binary16 rounding differs from the oracle"
    assert np.all(np.isnan(got[nan].view(np.float16))), "NaN did not convert to NaN"


@pytest.mark.parametrize("n,off", [(2560, 0), (9728, 0), (1001, 0), (3, 0), (4096, 1)])
def test_f32_to_f16_shapes(oracle, n, off):
    """off: the output starts 2 bytes (one binary16) into its buffer."""
    torch = torch_mod()
    x = normal(np.random.default_rng(n), n, 0.0, 30.0)
    buf = empty((n + 4,), torch.int16)
    F.f32_to_f16(buf.data_ptr() + 2 * off, dev(x).data_ptr(), n, stream())
    got = host(buf).view(np.uint16)
    assert np.array_equal(got[off:off + n], oracle.f32_to_f16(x))
    assert not got[:off].any() and not got[off + n:].any(), "wrote outside the output"


def test_f16_to_f32_all_patterns():
    torch = torch_mod()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    out = empty((h.size,), torch.float32)
    F.f16_to_f32(out.data_ptr(), dev(h.view(np.int16)).data_ptr(), h.size, stream())
    assert_bits_equal(host(out), h.view(np.float16).astype(np.float32), "f16 -> f32")


@pytest.mark.parametrize("n,off", [(2560, 0), (4096, 0), (4097, 0), (4096, 1)])
def test_residual_add_bit_exact(n, off):
    rng = np.random.default_rng(n + off)
    x, r = normal(rng, n + 1), normal(rng, n + 1)
    xd = dev(x)
    F.residual_add(xd.data_ptr() + 4 * off, dev(r).data_ptr() + 4 * off, n, stream())
    want = x.copy()
    want[off:off + n] = x[off:off + n] + r[off:off + n]
    assert_bits_equal(host(xd), want, "residual_add")


@pytest.mark.parametrize("rows,n,eps,with_res", [
    (1, 2560, 1e-6, True),     # Qwen3-4B decode boundary
    (1, 4096, 1e-5, True),     # Llama-3-8B decode boundary
    (512, 4096, 1e-5, True),   # configs[1] prefill rows
    (64, 5120, 1e-6, False),   # first layer: no residual yet
    (3, 4097, 1e-6, True),     # ragged: scalar path
])
def test_residual_rms_norm_f16(oracle, rows, n, eps, with_res):
    torch = torch_mod()
    rng = np.random.default_rng(rows * n)
    h0 = normal(rng, (rows, n))
    res = normal(rng, (rows, n)) if with_res else None
    w = normal(rng, n, 1.0, 0.1)
    hd, wd = dev(h0), dev(w)
    rd = dev(res) if with_res else None
    normed = empty((rows, n), torch.float32)
    o16 = empty((rows, n), torch.int16)
    F.residual_rms_norm_f16(hd.data_ptr(), rd.data_ptr() if with_res else None, wd.data_ptr(),
                            normed.data_ptr(), o16.data_ptr(), rows, n, eps, stream())
    ref_h, ref_n, _ = oracle.residual_rms_norm_f16(h0, res, w, eps)
    assert_bits_equal(host(hd), ref_h, "hidden after the residual add")
    got_n = host(normed)
    assert_rows_close(got_n, ref_n, n, "normed")
    got16 = host(o16).view(np.uint16)
    assert np.array_equal(got16, got_n.astype(np.float16).view(np.uint16)), "f16 != RNE(own fp32)"
    f16_vs_oracle(got16, ref_n, n, "f16 vs oracle")
    # binary16 only (the production form): the same bits
    hd2 = dev(h0)
    o16b = empty((rows, n), torch.int16)
    F.residual_rms_norm_f16(hd2.data_ptr(), rd.data_ptr() if with_res else None, wd.data_ptr(), None,
                            o16b.data_ptr(), rows, n, eps, stream())
    assert np.array_equal(host(o16b).view(np.uint16), got16), "f16-only output differs"
    assert_bits_equal(host(hd2), ref_h, "hidden (f16-only form)")


@pytest.mark.parametrize("n", [9728, 14336, 512 * 14336, 1001])
def test_swiglu_f16(oracle, n):
    torch = torch_mod()
    rng = np.random.default_rng(n)
    g, u = normal(rng, n), normal(rng, n)
    gd, ud = dev(g), dev(u)
    out = empty((n,), torch.float32)
    o16 = empty((n,), torch.int16)
    F.swiglu_f16(o16.data_ptr(), out.data_ptr(), gd.data_ptr(), ud.data_ptr(), n, stream())
    ref, _ = oracle.swiglu_f16(g, u)
    got = host(out)
    row = n if n <= 14336 else 14336
    assert_rows_close(got, ref, row, "swiglu fp32")
    plain = empty((n,), torch.float32)
    F.swiglu(plain.data_ptr(), gd.data_ptr(), ud.data_ptr(), n, stream())
    assert_bits_equal(got, host(plain), "swiglu_f16 fp32 vs swiglu")
    got16 = host(o16).view(np.uint16)
    assert np.array_equal(got16, got.astype(np.float16).view(np.uint16)), "f16 != RNE(own fp32)"
    f16_vs_oracle(got16, ref, row, "swiglu f16 vs oracle")
    o16b = empty((n,), torch.int16)
    F.swiglu_f16(o16b.data_ptr(), None, gd.data_ptr(), ud.data_ptr(), n, stream())
    assert np.array_equal(host(o16b).view(np.uint16), got16), "f16-only output differs"


def test_swiglu_f16_unaligned_output(oracle):
    torch = torch_mod()
    n = 4096
    rng = np.random.default_rng(8)
    g, u = normal(rng, n), normal(rng, n)
    buf = empty((n + 2,), torch.int16)
    F.swiglu_f16(buf.data_ptr() + 2, None, dev(g).data_ptr(), dev(u).data_ptr(), n, stream())
    got16 = host(buf).view(np.uint16)
    ref, _ = oracle.swiglu_f16(g, u)
    f16_vs_oracle(got16[1:1 + n], ref, n, "unaligned swiglu f16")
    assert got16[0] == 0 and got16[n + 1] == 0, "wrote outside the output"
