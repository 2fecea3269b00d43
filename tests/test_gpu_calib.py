"""GPU check of the calibration streams the benchmark times beside each op
(fence_calib_stream, fence_calib_read): every mode writes what it says --
a + b, a (also in place), zeros, each wave's sum of what it read -- at every
launch shape, including a ragged last workgroup.
It has no counterpart in the reference; its numbers are only a ceiling, but a
ceiling that skipped work would not bound anything."""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod

pytestmark = pytest.mark.gpu

SHAPES = [(64, 1), (64, 2), (64, 4), (256, 1), (256, 2), (256, 4)]


@pytest.mark.parametrize("threads,vpt", SHAPES)
@pytest.mark.parametrize("n", [4, 4096, 4 * 1000 + 4 * 257])
def test_calib_stream_modes(threads, vpt, n):
    torch = torch_mod()
    rng = np.random.default_rng(n * 7 + threads + vpt)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    da, db = dev(a), dev(b)

    out = torch.full((n + 4,), 7.0, device="cuda")  # one float4 past n must stay untouched
    LIVE.append(out)
    F.calib_stream(out.data_ptr(), da.data_ptr(), db.data_ptr(), n, threads, vpt, stream())
    got = host(out)
    assert np.array_equal(got[:n], a + b)
    assert np.all(got[n:] == 7.0)

    F.calib_stream(out.data_ptr(), da.data_ptr(), None, n, threads, vpt, stream())
    assert np.array_equal(host(out)[:n], a)

    F.calib_stream(out.data_ptr(), None, None, n, threads, vpt, stream())
    got = host(out)
    assert np.all(got[:n] == 0.0) and np.all(got[n:] == 7.0)

    x = dev(a.copy())  # in place
    F.calib_stream(x.data_ptr(), x.data_ptr(), None, n, threads, vpt, stream())
    assert np.array_equal(host(x), a)


@pytest.mark.parametrize("threads,vpt", SHAPES)
@pytest.mark.parametrize("n", [4, 4096, 4 * 1000 + 4 * 257])
def test_calib_read_wave_sums(threads, vpt, n):
    """Small integers, so every wave's sum is exact in any order: each wave
    reports exactly the floats its lanes were given, and nothing past the
    last wave's slot is written."""
    torch = torch_mod()
    rng = np.random.default_rng(n * 11 + threads + vpt)
    a = rng.integers(-64, 64, n).astype(np.float32)
    n4 = n // 4
    per_wg = threads * vpt
    groups = -(-n4 // per_wg)
    waves = groups * threads // 64
    i = np.arange(n4)
    t = (i % per_wg) % threads
    wave = (i // per_wg) * (threads // 64) + t // 64
    want = np.bincount(wave, weights=a.reshape(n4, 4).sum(axis=1).astype(np.float64), minlength=waves)
    sums = torch.full((waves + 4,), 7.0, device="cuda")
    LIVE.append(sums)
    F.calib_read(sums.data_ptr(), dev(a).data_ptr(), n, threads, vpt, stream())
    got = host(sums)
    assert np.array_equal(got[:waves], want.astype(np.float32))
    assert np.all(got[waves:] == 7.0)
