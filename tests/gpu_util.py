"""Helpers for the GPU parity tests: device copies, the stream handle the C ABI
takes, the tolerance rule and seeded synthetic inputs."""
from __future__ import annotations

import numpy as np

# fp32 rule: per row, max|gpu - ref| <= TOL * max|ref| (rows: token rows for
# norms / swiglu / gather, head vectors for RoPE and per-head norm, query rows
# for softmax).  Q8_0 dequantisation is compared bit for bit.
TOL = 1e-5


def torch_mod():
    import torch
    return torch


# Every tensor dev() makes stays referenced until the test ends (conftest
# clears the list), so `dev(x).data_ptr()` written inline in a call cannot be
# freed -- and its memory handed to the next dev() -- before the kernel runs.
LIVE: list = []


def dev(a: np.ndarray):
    torch = torch_mod()
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    LIVE.append(t)
    return t


def host(t) -> np.ndarray:
    torch = torch_mod()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return torch_mod().cuda.current_stream().cuda_stream


def rows_err(got, ref, row_len):
    """Per-row max|got-ref| / max|ref|; returns (worst ratio, worst max-abs)."""
    g = np.asarray(got, np.float64).reshape(-1, row_len)
    r = np.asarray(ref, np.float64).reshape(-1, row_len)
    if not np.array_equal(np.isnan(g), np.isnan(r)):
        return float("inf"), float("inf")
    g = np.nan_to_num(g, nan=0.0)
    r = np.nan_to_num(r, nan=0.0)
    diff = np.max(np.abs(g - r), axis=1)
    scale = np.max(np.abs(r), axis=1)
    ratio = np.where(scale > 0, diff / np.where(scale > 0, scale, 1), np.where(diff > 0, np.inf, 0))
    return float(np.max(ratio)), float(np.max(diff))


def assert_rows_close(got, ref, row_len, what=""):
    ratio, maxabs = rows_err(got, ref, row_len)
    assert ratio <= TOL, f"{what}: per-row rel err {ratio:.3g} > {TOL:g} (max-abs {maxabs:.3g})"
    return ratio, maxabs


def assert_bits_equal(got, ref, what=""):
    a = np.ascontiguousarray(got, np.float32)
    b = np.ascontiguousarray(ref, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), f"{what}: NaN positions differ"
    ua, ub = a.view(np.uint32)[~na], b.view(np.uint32)[~nb]
    if not np.array_equal(ua, ub):
        i = int(np.nonzero(ua != ub)[0][0])
        raise AssertionError(f"{what}: not bit-exact, first diff at {i}: {ua[i]:#x} vs {ub[i]:#x}")


def normal(rng, shape, mean=0.0, std=1.0):
    return (mean + std * rng.standard_normal(shape)).astype(np.float32)


def zipf_ids(rng, n, vocab, s=1.1):
    """Token ids drawn from a Zipf(s) law bounded to [0, vocab) by inverse CDF."""
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, rng.random(n)), vocab - 1).astype(np.int32)
