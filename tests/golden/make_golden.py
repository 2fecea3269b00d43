"""Writes the small fixtures under tests/golden/.

The fixtures come from computations that share no code with the oracle:
  q8_0_kat.npz    special-value Q8_0 blocks, dequantised with numpy's
                  float16 -> float32 conversion times int8 (exact in fp32);
  inv_freq.npz    1.0f / powf(base, (float)(2p)/(float)hd) with glibc powf
                  called through ctypes and numpy fp32 division
                  (the expression of src/kernels/ops.cuh:133);
  rope_small.npz  NeoX and interleaved RoPE of a small q/k in float64 from
                  the fp32 angles (float)pos * inv_freq[p];
  q6k_reference_tests.npz
                  the inputs of the reference's own Q6_K tests
                  (tests/test_q6k_dot.cu TC1-TC6, tests/test_gemv_q6k.cu
                  synthetic 64x256 and 128x512), rebuilt from their constants
                  and their glibc rand() draws, with float64 results from
                  tests/oracle_py.q6k_dequant_numpy (ggml's loop structure, not
                  the oracle's) and the closed forms of TC1-3, 5, 6.
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


class GlibcRand:
    """The C library's srand()/rand(), which the reference's own tests call to
    draw their inputs (tests/test_q6k_dot.cu:284, tests/test_gemv_q6k.cu:175,
    :229); RAND_MAX = 2^31 - 1."""

    def __init__(self, seed):
        self.libc = ctypes.CDLL("libc.so.6")
        self.libc.srand(seed)

    def __call__(self):
        return self.libc.rand()

    def unit(self):
        """(float)rand() / RAND_MAX in fp32 (RAND_MAX converts to 2^31)."""
        return np.float32(self()) / np.float32(2147483647)


def f16(v):
    return np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]


def q6k_dot_cases():
    """The six blocks of tests/test_q6k_dot.cu:242-332 (TC1-TC6) with their
    fp16 activations, rebuilt with the test's own constants and rand() draws."""
    from oracle_py import q6k_pack  # the layout's encoder; decoded independently below
    qs, scs, ds, xs = [], [], [], []

    def case(q, sc, d, x):
        qs.append(q), scs.append(sc), ds.append(f16(d)), xs.append(np.asarray(x, np.float32).astype(np.float16))
    case([32] * 256, [5] * 16, 0.1, [1.0] * 256)                       # TC1 zero-centred
    case([0] * 256, [3] * 16, 0.05, [0.5] * 256)                       # TC2 all minimum
    case([63] * 256, [3] * 16, 0.05, [0.5] * 256)                      # TC3 all maximum
    r = GlibcRand(42)                                                  # TC4 random
    sc4 = [(r() % 21) - 10 for _ in range(16)]
    q4 = [r() % 64 for _ in range(256)]
    x4 = [np.float32(-1.0) + np.float32(2.0) * r.unit() for _ in range(256)]
    case(q4, sc4, 0.02, x4)
    case([40] * 256, [4 if i % 2 == 0 else -4 for i in range(16)], 1.0, [0.25] * 256)  # TC5
    sc6 = [0] * 16
    sc6[7] = 10
    case([45] * 256, sc6, 0.1, [1.0] * 256)                            # TC6 one sub-block
    blocks = q6k_pack(np.array(qs), np.array(scs), np.array(ds, np.uint16))
    x16 = np.stack(xs).view(np.uint16)
    d = np.array([np.uint16(v) for v in ds]).view(np.float16).astype(np.float64)
    closed = np.array([0.0, 256 * d[1] * 3 * -32 * 0.5, 256 * d[2] * 3 * 31 * 0.5, np.nan, 0.0,
                       16 * d[5] * 10 * 13 * 1.0])
    return blocks, x16, closed


def q6k_gemv_case(seed, M, K, d, sc_mod, sc_off, x_expr):
    """tests/test_gemv_q6k.cu:167-269: per block d, 16 scales rand()%sc_mod -
    sc_off, 256 quants rand()%64 (blocks in row order), then K activations."""
    from oracle_py import q6k_pack
    r = GlibcRand(seed)
    nb = K // 256
    qs, scs = [], []
    for _ in range(M * nb):
        scs.append([(r() % sc_mod) - sc_off for _ in range(16)])
        qs.append([r() % 64 for _ in range(256)])
    x = np.array([x_expr(r) for _ in range(K)], np.float32).astype(np.float16)
    W = q6k_pack(np.array(qs), np.array(scs), np.full(M * nb, f16(d), np.uint16)).reshape(M, nb * 210)
    return W, x.view(np.uint16)


def q6k_reference_tests():
    import sys
    sys.path.insert(0, os.path.dirname(HERE))
    from oracle_py import q6k_dequant_numpy
    blocks, x16, closed = q6k_dot_cases()
    deq = q6k_dequant_numpy(blocks, 256)
    dot = np.einsum("ij,ij->i", deq, x16.view(np.float16).astype(np.float64))
    Ws, xs = q6k_gemv_case(123, 64, 256, 0.05, 21, 10,
                           lambda r: np.float32(-1.0) + np.float32(2.0) * np.float32(r()) / np.float32(2147483647))
    Wm, xm = q6k_gemv_case(456, 128, 512, 0.03, 31, 15,
                           lambda r: np.float32(-0.5) + np.float32(r()) / np.float32(2147483647))
    ys = q6k_dequant_numpy(Ws, 256) @ xs.view(np.float16).astype(np.float64)
    ym = q6k_dequant_numpy(Wm, 512) @ xm.view(np.float16).astype(np.float64)
    return dict(dot_blocks=blocks, dot_x=x16, dot_expected=dot, dot_closed=closed,
                small_W=Ws, small_x=xs, small_expected=ys, multi_W=Wm, multi_x=xm, multi_expected=ym)


def main():
    np.savez(os.path.join(HERE, "q8_0_kat.npz"), **q8_0_kat())
    inv = {f"b{b:g}_hd{hd}": libm_inv_freq(hd, b)
           for b, hd in [(1e6, 128), (5e5, 128), (5e6, 128), (1e4, 64), (1e6, 256)]}
    np.savez(os.path.join(HERE, "inv_freq.npz"), **inv)
    np.savez(os.path.join(HERE, "rope_small.npz"), **rope_small())
    np.savez(os.path.join(HERE, "q6k_reference_tests.npz"), **q6k_reference_tests())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
