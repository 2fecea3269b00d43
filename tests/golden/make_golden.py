"""Writes the small fixtures under tests/golden/.

The reference repository holds no test vectors for this path, so the
fixtures come from computations that share no code with the oracle:
  q8_0_kat.npz    special-value Q8_0 blocks, dequantised with numpy's
                  float16 -> float32 conversion times int8 (exact in fp32);
  inv_freq.npz    1.0f / powf(base, (float)(2p)/(float)hd) with glibc powf
                  called through ctypes and numpy fp32 division
                  (the expression of src/kernels/ops.cuh:133);
  rope_small.npz  NeoX and interleaved RoPE of a small q/k in float64 from
                  the fp32 angles (float)pos * inv_freq[p].
Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def libm_inv_freq(hd: int, base: float) -> np.ndarray:
    libm = ctypes.CDLL("libm.so.6")
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    out = np.empty(hd // 2, np.float32)
    for p in range(hd // 2):
        e = np.float32(2 * p) / np.float32(hd)
        out[p] = np.float32(1.0) / np.float32(libm.powf(np.float32(base), e))
    return out


def q8_0_kat():
    scales = [0x0000, 0x8000, 0x0001, 0x0155, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF,
              0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE00, 0x1400, 0x2A3B]
    q = np.array([-128, 127, -127, 0, 1, -1, 64, -64] * 4, dtype=np.int8)
    nb, dim = 3, 96
    rows = []
    for r, s in enumerate(scales):
        blk = np.zeros((nb, 34), np.uint8)
        for b in range(nb):
            sc = scales[(r + 5 * b) % len(scales)]
            blk[b, 0], blk[b, 1] = sc & 0xFF, sc >> 8
            blk[b, 2:] = np.roll(q, r + b).view(np.uint8)
        rows.append(blk.reshape(-1))
    table = np.stack(rows)
    ids = np.array([0, len(scales) - 1] + list(range(1, len(scales) - 1)), np.int32)
    d = table.reshape(-1, nb, 34)[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    qs = table.reshape(-1, nb, 34)[:, :, 2:].copy().view(np.int8).astype(np.float32)
    with np.errstate(invalid="ignore"):  # inf * 0 -> NaN is an intended case
        expected = (d * qs).reshape(-1, dim)[ids]
    return dict(table=table, ids=ids, dim=np.int32(dim), expected=expected)


def rope_ref64(x, pos, inv, style):
    x = x.astype(np.float64).copy()
    hd = x.shape[-1]
    half = hd // 2
    ang = (np.float32(pos) * inv).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    if style == "neox":
        i0, i1 = np.arange(half), np.arange(half) + half
    else:
        i0, i1 = 2 * np.arange(half), 2 * np.arange(half) + 1
    x0, x1 = x[..., i0].copy(), x[..., i1].copy()
    x[..., i0] = x0 * c - x1 * s
    x[..., i1] = x0 * s + x1 * c
    return x


def rope_small():
    rng = np.random.default_rng(2024)
    hd, base = 64, 1e4
    q = rng.standard_normal((3, 2, hd)).astype(np.float32)
    k = rng.standard_normal((3, 1, hd)).astype(np.float32)
    positions = np.array([0, 7, 4000], np.int32)
    inv = libm_inv_freq(hd, base)
    out = dict(q=q, k=k, positions=positions, base=np.float32(base))
    for style in ("neox", "interleaved"):
        out[f"q_{style}"] = np.stack([rope_ref64(q[t], positions[t], inv, style) for t in range(3)])
        out[f"k_{style}"] = np.stack([rope_ref64(k[t], positions[t], inv, style) for t in range(3)])
    return out


def main():
    np.savez(os.path.join(HERE, "q8_0_kat.npz"), **q8_0_kat())
    inv = {f"b{b:g}_hd{hd}": libm_inv_freq(hd, b)
           for b, hd in [(1e6, 128), (5e5, 128), (5e6, 128), (1e4, 64), (1e6, 256)]}
    np.savez(os.path.join(HERE, "inv_freq.npz"), **inv)
    np.savez(os.path.join(HERE, "rope_small.npz"), **rope_small())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
