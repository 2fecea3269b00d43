"""Checks that pin the CPU oracle to the reference's formulas.

Every check compares the oracle with something that does not share its code:
numpy's float16 decode, scipy / torch library routines, closed forms,
invariants, float64 brute force, and fixtures written by
tests/golden/make_golden.py.  Each function returns a list of failure
messages (empty = pass), so the same checks can run against the real oracle
(tests/test_oracle.py) and against mutants with planted mistakes
(tests/test_oracle_mutants.py), where at least one check must fail.
"""
from __future__ import annotations

import os

import numpy as np

from oracle_py import (INTERLEAVED, NEOX, Oracle, make_q6k_matrix, make_q8_0_table, q6k_dequant_numpy,
                       q6k_pack, q8_0_dequant_numpy)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = max(np.max(np.abs(ref)), 1e-30)
    return float(np.max(np.abs(got - ref)) / scale)


def _close(fails, name, got, ref, tol):
    e = _rel_err(got, ref)
    if not np.isfinite(e) or e > tol:
        fails.append(f"{name}: rel err {e:.3g} > {tol:g}")


def _bits_equal_nan_aware(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb]))


# ------------------------------------------------------------------- fp16

def check_fp16(o: Oracle):
    fails = []
    got = o.fp16_to_f32_all()
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = pats.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    gotf = got.view(np.float32)
    if not np.array_equal(np.isnan(gotf), nan):
        fails.append("fp16: NaN set differs from numpy")
    if not np.array_equal(got[~nan], ref.view(np.uint32)[~nan]):
        bad = np.nonzero(got[~nan] != ref.view(np.uint32)[~nan])[0][:4]
        fails.append(f"fp16: finite/inf decode differs from numpy at {bad.tolist()}")
    # NaN: sign and payload kept, quiet bit set
    nb = pats[nan].astype(np.uint32)
    want = ((nb & 0x8000) << 16) | 0x7F800000 | ((nb & 0x3FF) << 13) | 0x00400000
    if not np.array_equal(got[nan], want):
        fails.append("fp16: NaN payload/sign/quiet bit wrong")
    return fails


# ------------------------------------------------------------------- Q8_0

def q8_0_kat_table():
    """Blocks with special scales and extreme int8 values (34-byte blocks)."""
    scales = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xC000, 0x7BFF, 0xFBFF,
              0x7C00, 0xFC00, 0x7E00, 0x7C01, 0x1234, 0x2E66, 0x0200]
    qpat = np.array([-128, -127, -1, 0, 1, 127] + list(range(-13, 13)), dtype=np.int8)
    nb = 4
    dim = nb * 32
    rows = []
    for r in range(len(scales)):
        blk = np.empty((nb, 34), dtype=np.uint8)
        for b in range(nb):
            s = scales[(r + b) % len(scales)]
            blk[b, 0] = s & 0xFF
            blk[b, 1] = s >> 8
            blk[b, 2:] = np.roll(qpat, 3 * b + r).view(np.uint8)
        rows.append(blk.reshape(-1))
    return np.stack(rows), dim


def check_q8_0(o: Oracle):
    fails = []
    table, dim = q8_0_kat_table()
    vocab = table.shape[0]
    for r in range(vocab):
        got = o.embed_q8_0(table, r, dim)
        ref = q8_0_dequant_numpy(table, [r], dim)[0]
        if not _bits_equal_nan_aware(got, ref):
            fails.append(f"q8_0 KAT row {r}: not bit-exact vs numpy dequant")
            break
    # random table, first / last / middle rows, gather with out-of-range ids
    rng = np.random.default_rng(7)
    vocab2, dim2 = 97, 256
    t2 = make_q8_0_table(rng, vocab2, dim2)
    ids = np.array([0, vocab2 - 1, 50, 3, 3, -1, vocab2, 96], dtype=np.int32)
    got, bad = o.embed_q8_0_gather(t2, vocab2, ids, dim2)
    if bad != 2:
        fails.append(f"q8_0 gather: {bad} out-of-range ids reported, want 2")
    ok = (ids >= 0) & (ids < vocab2)
    ref = q8_0_dequant_numpy(t2, ids[ok], dim2)
    if not _bits_equal_nan_aware(got[ok], ref):
        fails.append("q8_0 gather: not bit-exact vs numpy dequant")
    if not np.all(np.isnan(got[~ok])):
        fails.append("q8_0 gather: out-of-range rows are not NaN")
    # committed fixture
    fx = np.load(os.path.join(GOLDEN, "q8_0_kat.npz"))
    got = np.stack([o.embed_q8_0(fx["table"], int(i), int(fx["dim"])) for i in fx["ids"]])
    exp = fx["expected"]
    if not _bits_equal_nan_aware(got, exp):
        fails.append("q8_0: fixture q8_0_kat.npz mismatch")
    return fails


# ---------------------------------------------------------------- RMSNorm

def _rms_ref64(x, w, eps):
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def check_rms_norm(o: Oracle):
    fails = []
    rng = np.random.default_rng(11)
    # closed form: constant vector, unit weight
    for c, eps in [(0.75, 1e-6), (3e-3, 1e-5), (-2.0, 1e-6)]:
        n = 96
        got = o.rms_norm(np.full(n, c, np.float32), np.ones(n, np.float32), eps)
        c32 = float(np.float32(c))
        want = c32 / np.sqrt(c32 * c32 + float(np.float32(eps)))
        _close(fails, f"rms const c={c}", got, np.full(n, want), 2e-7)
    for n, eps in [(96, 1e-6), (1000, 1e-5), (2560, 1e-6), (4096, 1e-5), (7, 1e-6)]:
        x = rng.standard_normal(n).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        got = o.rms_norm(x, w, eps)
        _close(fails, f"rms n={n} vs float64", got, _rms_ref64(x, w, eps), 1e-6)
        if not np.array_equal(o.rms_norm_inplace(x, w, eps), got):
            fails.append(f"rms n={n}: in-place differs from out-of-place")
    # independent library: torch rms_norm in float64
    try:
        import torch
        x = rng.standard_normal((5, 640)).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(640)).astype(np.float32)
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (640,),
                                           weight=torch.from_numpy(w).double(), eps=1e-6).numpy()
        _close(fails, "rms rows vs torch", o.rms_norm_rows(x, w, 1e-6), ref, 1e-6)
    except ImportError:
        pass
    # per-head == rms_norm on each slice (bitwise) and float64 brute force
    xh = rng.standard_normal((6, 128)).astype(np.float32)
    wh = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    got = o.rms_norm_per_head(xh, wh, 1e-6)
    per = np.stack([o.rms_norm(xh[h], wh, 1e-6) for h in range(6)])
    if not np.array_equal(got, per):
        fails.append("per-head norm differs from per-slice rms_norm")
    _close(fails, "per-head vs float64", got, _rms_ref64(xh, wh, 1e-6), 1e-6)
    return fails


# ------------------------------------------------------------------- RoPE

def _inv_freq_ref(hd, base):
    fx = np.load(os.path.join(GOLDEN, "inv_freq.npz"))
    key = f"b{base:g}_hd{hd}"
    return fx[key] if key in fx.files else None


def _rope_ref64(x, pos, inv_freq32, style):
    """float64 rotation with the fp32 angle (float)pos * inv_freq[p]."""
    x = np.asarray(x, np.float64).copy()
    hd = x.shape[-1]
    half = hd // 2
    ang = (np.float32(pos) * inv_freq32.astype(np.float32)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    if style == NEOX:
        i0, i1 = np.arange(half), np.arange(half) + half
    else:
        i0, i1 = 2 * np.arange(half), 2 * np.arange(half) + 1
    x0, x1 = x[..., i0].copy(), x[..., i1].copy()
    x[..., i0] = x0 * c - x1 * s
    x[..., i1] = x0 * s + x1 * c
    return x


def check_inv_freq(o: Oracle):
    fails = []
    for base, hd in [(1e6, 128), (5e5, 128), (5e6, 128), (1e4, 64), (1e6, 256)]:
        got = o.rope_inv_freq(hd, base)
        if got[0] != np.float32(1.0):
            fails.append(f"inv_freq b={base} hd={hd}: pair 0 is not exactly 1")
        fx = _inv_freq_ref(hd, base)
        if fx is not None and not np.array_equal(got.view(np.uint32), fx.view(np.uint32)):
            fails.append(f"inv_freq b={base} hd={hd}: differs from libm-powf fixture")
        exact = base ** (-(2.0 * np.arange(hd // 2)) / hd)
        _close(fails, f"inv_freq b={base} hd={hd} vs float64", got, exact, 2e-6)
        if not np.all(np.diff(got.astype(np.float64)) < 0):
            fails.append(f"inv_freq b={base} hd={hd}: not strictly decreasing")
    return fails


def check_rope(o: Oracle):
    fails = []
    rng = np.random.default_rng(13)
    for hd, base in [(128, 1e6), (64, 1e4), (128, 5e5)]:
        x = rng.standard_normal(hd).astype(np.float32)
        for style in (NEOX, INTERLEAVED):
            if not np.array_equal(o.rope_head(x, 0, base, style), x):
                fails.append(f"rope hd={hd} style={style}: pos 0 is not the identity")
            inv = o.rope_inv_freq(hd, base)
            for pos in (1, 37, 4095, 8191):
                got = o.rope_head(x, pos, base, style)
                _close(fails, f"rope hd={hd} style={style} pos={pos} vs float64", got,
                       _rope_ref64(x, pos, inv, style), 1e-6)
                # pair norms preserved
                half = hd // 2
                idx = (np.arange(half), np.arange(half) + half) if style == NEOX else \
                      (2 * np.arange(half), 2 * np.arange(half) + 1)
                n0 = x[idx[0]].astype(np.float64) ** 2 + x[idx[1]].astype(np.float64) ** 2
                n1 = got[idx[0]].astype(np.float64) ** 2 + got[idx[1]].astype(np.float64) ** 2
                _close(fails, f"rope pair norms hd={hd} style={style} pos={pos}", n1, n0, 1e-6)
                # pair 0 rotates by exactly `pos` radians
                a = float(np.float32(pos))
                want0 = x[idx[0][0]] * np.cos(a) - x[idx[1][0]] * np.sin(a)
                if abs(got[idx[0][0]] - want0) > 1e-5 * max(1.0, abs(want0)):
                    fails.append(f"rope hd={hd} style={style} pos={pos}: pair 0 angle is not pos")
        # NeoX == interleaved under the fixed permutation (even -> first half)
        perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])  # interleaved idx -> neox slot
        for pos in (5, 3000):
            xi = rng.standard_normal(hd).astype(np.float32)
            xn = xi[perm]
            gi = o.rope_head(xi, pos, base, INTERLEAVED)
            gn = o.rope_head(xn, pos, base, NEOX)
            if not np.array_equal(gi[perm], gn):
                fails.append(f"rope hd={hd} pos={pos}: NeoX and interleaved disagree under permutation")
        # composition R(a) R(b) ~ R(a+b)
        y = o.rope_head(o.rope_head(x, 3, base, NEOX), 4, base, NEOX)
        _close(fails, f"rope compose hd={hd}", y, o.rope_head(x, 7, base, NEOX), 1e-5)
    # apply_rope (q and k, NeoX) == per-head rotation
    q = rng.standard_normal((4, 128)).astype(np.float32)
    k = rng.standard_normal((2, 128)).astype(np.float32)
    gq, gk = o.apply_rope(q, k, 99, 1e6)
    for h in range(4):
        if not np.array_equal(gq[h], o.rope_head(q[h], 99, 1e6, NEOX)):
            fails.append("apply_rope q differs from rope_head")
            break
    for h in range(2):
        if not np.array_equal(gk[h], o.rope_head(k[h], 99, 1e6, NEOX)):
            fails.append("apply_rope k differs from rope_head")
            break
    # committed float64 fixture
    fx = np.load(os.path.join(GOLDEN, "rope_small.npz"))
    for style, key in ((NEOX, "neox"), (INTERLEAVED, "interleaved")):
        gq, gk = o.rope_rows(fx["q"], fx["k"], fx["positions"], 0, float(fx["base"]), style)
        _close(fails, f"rope fixture {key} q", gq, fx[f"q_{key}"], 1e-6)
        _close(fails, f"rope fixture {key} k", gk, fx[f"k_{key}"], 1e-6)
    return fails


# ----------------------------------------------------------------- SwiGLU

def check_swiglu(o: Oracle):
    fails = []
    rng = np.random.default_rng(17)
    g = rng.standard_normal(4099).astype(np.float32) * 3
    u = rng.standard_normal(4099).astype(np.float32)
    got = o.silu_mul(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    _close(fails, "swiglu vs float64", got, g64 / (1 + np.exp(-g64)) * u64, 1e-6)
    try:
        import torch
        ref = (torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
        _close(fails, "swiglu vs torch silu", got, ref, 1e-6)
    except ImportError:
        pass
    if np.any(o.silu_mul(np.zeros(8, np.float32), u[:8]) != 0):
        fails.append("swiglu: g = 0 does not give 0")
    if np.any(o.silu_mul(g[:8], np.zeros(8, np.float32)) != 0):
        fails.append("swiglu: up = 0 does not give 0")
    ones = np.ones_like(g)
    diff = o.silu_mul(g, ones).astype(np.float64) - o.silu_mul(-g, ones).astype(np.float64)
    _close(fails, "swiglu silu(g)-silu(-g)=g", diff, g64, 1e-6)
    big = np.array([30.0, 60.0, -30.0, -60.0], np.float32)
    gb = o.silu_mul(big, np.ones(4, np.float32))
    if not (abs(gb[0] - 30) < 1e-5 and abs(gb[1] - 60) < 1e-5 and abs(gb[2]) < 1e-10 and abs(gb[3]) < 1e-20):
        fails.append("swiglu: large-|g| asymptotes wrong")
    return fails


# ---------------------------------------------------------------- softmax

def check_softmax(o: Oracle):
    fails = []
    rng = np.random.default_rng(19)
    from scipy.special import softmax as sp_softmax
    for n in (1, 7, 96, 1000, 2048, 5000):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        got = o.softmax(x)
        _close(fails, f"softmax n={n} vs scipy", got, sp_softmax(x.astype(np.float64)), 1e-6)
        if abs(np.sum(got, dtype=np.float64) - 1) > 1e-5:
            fails.append(f"softmax n={n}: sum != 1")
        _close(fails, f"softmax n={n} shift invariance", o.softmax(x + np.float32(100)), got, 1e-5)
    neg = (rng.standard_normal(64) * 2 - 200).astype(np.float32)
    gn = o.softmax(neg)
    if not (np.all(np.isfinite(gn)) and abs(np.sum(gn, dtype=np.float64) - 1) < 1e-5):
        fails.append("softmax: very negative row is not a distribution")
    u = o.softmax(np.full(10, 1.5, np.float32))
    _close(fails, "softmax uniform", u, np.full(10, 0.1), 1e-7)
    xm = rng.standard_normal(16).astype(np.float32)
    xm[5:] = -np.inf
    gm = o.softmax(xm)
    if np.any(gm[5:] != 0):
        fails.append("softmax: -inf inputs do not give exactly 0")
    # causal: query 0 sees only key 0; matches the generic form on a masked input
    s = (rng.standard_normal((3, 33, 33)) * 3 / np.sqrt(128)).astype(np.float32)
    gc = o.softmax_causal(s)
    if not (np.all(gc[:, 0, 0] == 1) and np.all(gc[:, 0, 1:] == 0)):
        fails.append("causal softmax: row 0 is not [1, 0, ...]")
    masked = s.copy()
    masked[:, np.triu_indices(33, 1)[0], np.triu_indices(33, 1)[1]] = -np.inf
    if not np.array_equal(gc, o.softmax_rows(masked.reshape(-1, 33)).reshape(3, 33, 33)):
        fails.append("causal softmax differs from generic softmax on the masked input")
    ref = np.where(np.isinf(masked), 0.0, sp_softmax(masked.astype(np.float64), axis=-1))
    _close(fails, "causal softmax vs scipy", gc, ref, 1e-6)
    # decode form: sq=1 sees all keys; rows with stride untouched beyond n
    xr = rng.standard_normal((4, 40)).astype(np.float32)
    gr = o.softmax_rows(xr, n=33)
    if not np.array_equal(gr[:, 33:], xr[:, 33:]):
        fails.append("softmax rows: wrote beyond n")
    _close(fails, "softmax rows vs scipy", gr[:, :33], sp_softmax(xr[:, :33].astype(np.float64), axis=1), 1e-6)
    return fails


# ------------------------------------------------------------------ fused

def check_fused(o: Oracle):
    fails = []
    rng = np.random.default_rng(23)
    T, nq, nkv, hd, eps, base = 5, 4, 2, 128, 1e-6, 1e6
    q = rng.standard_normal((T, nq, hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    pos = np.array([0, 1, 17, 2000, 4095], np.int32)
    inv = o.rope_inv_freq(hd, base)
    for style in (NEOX, INTERLEAVED):
        gq, gk = o.qk_norm_rope(q, k, wq, wk, eps, pos, 0, base, style)
        rq = np.stack([_rope_ref64(_rms_ref64(q[t], wq, eps), pos[t], inv, style) for t in range(T)])
        rk = np.stack([_rope_ref64(_rms_ref64(k[t], wk, eps), pos[t], inv, style) for t in range(T)])
        _close(fails, f"qk_norm_rope q style={style}", gq, rq, 2e-6)
        _close(fails, f"qk_norm_rope k style={style}", gk, rk, 2e-6)
    x = rng.standard_normal((T, nq * hd)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(nq * hd)).astype(np.float32)
    for style in (NEOX, INTERLEAVED):
        out, gk = o.rms_norm_rope(x, w, k, nq, hd, 1e-5, None, 10, 5e5, style)
        inv5 = o.rope_inv_freq(hd, 5e5)
        ro = np.stack([_rope_ref64(_rms_ref64(x[t], w, 1e-5).reshape(nq, hd), 10 + t, inv5, style)
                       for t in range(T)]).reshape(T, -1)
        rk = np.stack([_rope_ref64(k[t], 10 + t, inv5, style) for t in range(T)])
        _close(fails, f"rms_norm_rope out style={style}", out, ro, 2e-6)
        _close(fails, f"rms_norm_rope k style={style}", gk, rk, 2e-6)
    vocab, dim = 50, 512
    tab = make_q8_0_table(rng, vocab, dim)
    ids = np.array([3, 49, 0, 3], np.int32)
    wd = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    got, _ = o.embed_q8_0_gather_rms_norm(tab, vocab, ids, dim, wd, 1e-6)
    ref = _rms_ref64(q8_0_dequant_numpy(tab, ids, dim), wd, 1e-6)
    _close(fails, "gather_rms_norm vs float64", got, ref, 1e-6)
    return fails


# ------------------------------------------------------------------- GEMV

def check_gemv(o: Oracle):
    fails = []
    rng = np.random.default_rng(29)
    M, K = 257, 2560
    tab = make_q8_0_table(rng, M, K)
    W = q8_0_dequant_numpy(tab, np.arange(M), K).astype(np.float64)  # independent dequant
    x = rng.standard_normal(K).astype(np.float32)
    got = o.gemv_q8_0(tab, x)
    ref = W @ x.astype(np.float64)
    scale = np.abs(W) @ np.abs(x.astype(np.float64))  # the dot products' natural error scale
    err = np.max(np.abs(got - ref) / scale)
    if not err <= 1e-7:
        fails.append(f"gemv vs float64 matmul: {err:.3g} of sum|w x| > 1e-7")
    # a unit vector picks one dequantised column exactly (one nonzero product)
    for j in (0, 31, 32, 1000, K - 1):
        e = np.zeros(K, np.float32)
        e[j] = 1.0
        col = o.gemv_q8_0(tab, e)
        if not np.array_equal(col.view(np.uint32), W[:, j].astype(np.float32).view(np.uint32)):
            fails.append(f"gemv with unit vector e_{j} is not column {j} of the dequantised table")
            break
    # linearity: W(2x) = 2 W x exactly (scaling by 2 is exact)
    if not np.array_equal(o.gemv_q8_0(tab, 2 * x), 2 * got):
        fails.append("gemv not exactly linear under x -> 2x")
    return fails


# ------------------------------------------------------- f16 and epilogue

def f32_patterns(rng):
    """float32 bit patterns over every exponent: mantissas at and around the
    binary16 rounding point (13 dropped bits), random mantissas, and for the
    binary16-subnormal exponents the exact halfway cases of each shift."""
    mans = [0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x3000, 0x5000, 0x7FE000, 0x7FEFFF,
            0x7FF000, 0x7FF001, 0x7FFFFF, 0x400000]
    pats = []
    for e in range(256):
        ms = np.concatenate([np.array(mans, np.uint32), rng.integers(0, 1 << 23, 48, dtype=np.uint32)])
        pats.append((np.uint32(e) << 23) | ms)
    for e in range(100, 113):  # binary16 subnormal results: shift = 126 - e in [14, 26]
        shift = 126 - e
        k = rng.integers(0, 1 << max(1, 24 - shift), 32, dtype=np.uint32)
        sig = (k << np.uint32(shift)) | np.uint32(1 << (shift - 1))
        sig = sig | np.uint32(0x800000)
        pats.append((np.uint32(e) << 23) | (sig & np.uint32(0x7FFFFF)))
    p = np.concatenate(pats)
    return np.concatenate([p, p | np.uint32(0x80000000)])


def check_f16_epilogue(o: Oracle):
    fails = []
    rng = np.random.default_rng(41)
    bits = f32_patterns(rng)
    x = bits.view(np.float32)
    got = o.f32_to_f16(x)
    nan = np.isnan(x)
    with np.errstate(over="ignore"):
        ref = x[~nan].astype(np.float16).view(np.uint16)
    if not np.array_equal(got[~nan], ref):
        bad = np.nonzero(got[~nan] != ref)[0][:3]
        fails.append(f"f32->f16 differs from numpy's RNE at {[hex(int(b)) for b in bits[~nan][bad]]}")
    gn = got[nan]
    if not np.all(((gn & 0x7C00) == 0x7C00) & ((gn & 0x3FF) != 0)):
        fails.append("f32->f16 of NaN is not a NaN")
    # every binary16 value survives f16 -> f32 -> f16 (NaNs come back quiet)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = o.f32_to_f16(h.view(np.float16).astype(np.float32))
    hn = np.isnan(h.view(np.float16))
    if not np.array_equal(back[~hn], h[~hn]):
        fails.append("f16 -> f32 -> f16 is not the identity")
    # closed forms at the edges of the binary16 range
    cases = {65504.0: 0x7BFF, 65519.99: 0x7BFF, 65520.0: 0x7C00, 2.0 ** -24: 0x0001, 2.0 ** -25: 0x0000,
             1.5 * 2.0 ** -25: 0x0001, 2.0 ** -14: 0x0400, 1.0 + 2.0 ** -11: 0x3C00,
             1.0 + 3 * 2.0 ** -11: 0x3C02, -0.0: 0x8000}
    for v, want in cases.items():
        g = int(o.f32_to_f16(np.array([v], np.float32))[0])
        if g != want:
            fails.append(f"f32->f16({v!r}) = {g:#06x}, want {want:#06x}")
    # residual add is a plain fp32 add
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    if not np.array_equal(o.residual_add(a, b), a + b):
        fails.append("residual_add differs from numpy's fp32 add")
    # the fused epilogue equals its pinned parts, bit for bit
    hid = rng.standard_normal((3, 640)).astype(np.float32)
    res = rng.standard_normal((3, 640)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(640)).astype(np.float32)
    h2, normed, o16 = o.residual_rms_norm_f16(hid, res, w, 1e-6)
    if not np.array_equal(h2, hid + res):
        fails.append("epilogue: hidden is not hidden + residual")
    if not np.array_equal(normed, o.rms_norm_rows(hid + res, w, 1e-6)):
        fails.append("epilogue: normed differs from rms_norm of the sum")
    if not np.array_equal(o16, normed.astype(np.float16).view(np.uint16)):
        fails.append("epilogue: f16 output is not RNE of the normed row")
    h3, normed3, _ = o.residual_rms_norm_f16(hid, None, w, 1e-6)
    if not (np.array_equal(h3, hid) and np.array_equal(normed3, o.rms_norm_rows(hid, w, 1e-6))):
        fails.append("epilogue without residual: hidden changed or norm differs")
    g = rng.standard_normal(999).astype(np.float32)
    u = rng.standard_normal(999).astype(np.float32)
    act, a16 = o.swiglu_f16(g, u)
    if not np.array_equal(act, o.silu_mul(g, u)):
        fails.append("swiglu_f16: fp32 output differs from silu_elementwise_mul")
    if not np.array_equal(a16, act.astype(np.float16).view(np.uint16)):
        fails.append("swiglu_f16: f16 output is not RNE of the fp32 output")
    return fails


# ------------------------------------------------------------------- Q6_K

def check_q6k(o: Oracle):
    fails = []
    fx = np.load(os.path.join(GOLDEN, "q6k_reference_tests.npz"))
    # the reference's dot tests (tests/test_q6k_dot.cu TC1-TC6): closed forms
    # exactly, the random TC4 against the independent float64 dequant
    got = np.array([o.q6k_dot(b, x) for b, x in zip(fx["dot_blocks"], fx["dot_x"])])
    closed = fx["dot_closed"]
    known = ~np.isnan(closed)
    if not np.array_equal(got[known], closed[known]):
        fails.append(f"q6k dot closed forms (TC1-3, 5, 6): {got[known]} != {closed[known]}")
    if not np.allclose(got, fx["dot_expected"], rtol=1e-13, atol=1e-12):
        fails.append("q6k dot differs from the reference tests' vectors")
    # the reference's GEMV tests (tests/test_gemv_q6k.cu synthetic 64x256, 128x512)
    for name, K in (("small", 256), ("multi", 512)):
        W, x, ref = fx[f"{name}_W"], fx[f"{name}_x"], fx[f"{name}_expected"]
        y = o.gemv_q6k(W, x)
        scale = np.abs(q6k_dequant_numpy(W, K)) @ np.abs(x.view(np.float16).astype(np.float64))
        if not np.all(np.abs(y - ref) <= 1e-7 * scale):
            fails.append(f"q6k gemv {name}: differs from the reference test's vector")
    # every quant decodes: pack known values with the ggml-style encoder
    rng = np.random.default_rng(17)
    q6 = rng.integers(0, 64, (4, 256))
    blk = q6k_pack(q6, rng.integers(-128, 128, (4, 16)), np.full(4, 0x3C00, np.uint16))
    for b in range(4):
        if not np.array_equal(o.q6k_quants(blk[b]), q6[b]):
            fails.append("q6k quant layout: decode(pack(q)) != q")
            break
    # a random matrix against float64 matmul; unit vectors select a column; bias adds in fp32
    W = make_q6k_matrix(rng, 37, 1024)
    x = rng.standard_normal(1024).astype(np.float16)
    deq = q6k_dequant_numpy(W, 1024)
    y = o.gemv_q6k(W, x.view(np.uint16))
    ref = deq @ x.astype(np.float64)
    if not np.all(np.abs(y - ref) <= 1e-7 * (np.abs(deq) @ np.abs(x.astype(np.float64)))):
        fails.append("q6k gemv vs float64 matmul")
    for j in (0, 15, 16, 31, 32, 127, 128, 255, 256, 1023):
        e = np.zeros(1024, np.float16)
        e[j] = 1.0
        if not np.array_equal(o.gemv_q6k(W, e.view(np.uint16)), deq[:, j].astype(np.float32)):
            fails.append(f"q6k gemv with e_{j} is not column {j}")
            break
    bias = rng.standard_normal(37).astype(np.float32)
    if not np.array_equal(o.gemv_q6k(W, x.view(np.uint16), bias), y + bias):
        fails.append("q6k gemv bias is not an fp32 add of the sum")
    return fails


# ------------------------------------------------------- decode attention

def attention_ref64(q, kc, vc, n_q, n_kv, hd, seq):
    """float64 softmax(q k^T / sqrt(hd)) v per query head, from binary16 caches."""
    K = kc[:seq].view(np.float16).astype(np.float64).reshape(seq, n_kv, hd)
    V = vc[:seq].view(np.float16).astype(np.float64).reshape(seq, n_kv, hd)
    qh = np.asarray(q, np.float64).reshape(n_q, hd)
    out = np.empty((n_q, hd))
    for h in range(n_q):
        g = h // (n_q // n_kv)
        s = K[:, g, :] @ qh[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[:, g, :]
    return out.reshape(-1)


def check_attention(o: Oracle):
    fails = []
    rng = np.random.default_rng(53)
    n_q, n_kv, hd, ctx = 8, 2, 64, 40
    kc = rng.standard_normal((ctx, n_kv * hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, n_kv * hd)).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(n_q * hd).astype(np.float32)
    for seq in (1, 2, 17, 40):
        got = o.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq)
        ref = attention_ref64(q, kc, vc, n_q, n_kv, hd, seq)
        if not np.allclose(got, ref, rtol=1e-5, atol=1e-6):
            fails.append(f"attention seq={seq}: differs from float64 softmax(qK/sqrt(d))V")
    # one position: the output is that position's V row, exactly
    got = o.gqa_attention(q, kc, vc, n_q, n_kv, hd, 1).reshape(n_q, hd)
    v0 = vc[0].view(np.float16).astype(np.float32).reshape(n_kv, hd)
    if not np.array_equal(got, v0[np.arange(n_q) // (n_q // n_kv)]):
        fails.append("attention over one position is not V[0] of the head's kv group")
    # q = 0: uniform weights, the mean of V
    got = o.gqa_attention(np.zeros_like(q), kc, vc, n_q, n_kv, hd, 40).reshape(n_q, hd)
    mean = vc[:40].view(np.float16).astype(np.float64).reshape(40, n_kv, hd).mean(axis=0)
    if not np.allclose(got, mean[np.arange(n_q) // (n_q // n_kv)], rtol=1e-6, atol=1e-7):
        fails.append("attention with q = 0 is not the mean of V")
    # scores far apart: the softmax must subtract the maximum (no overflow)
    big = (q * 400).astype(np.float32)
    got = o.gqa_attention(big, kc, vc, n_q, n_kv, hd, 40)
    if not np.all(np.isfinite(got)) or not np.allclose(got, attention_ref64(big, kc, vc, n_q, n_kv, hd, 40),
                                                       rtol=1e-5, atol=1e-5):
        fails.append("attention with large scores overflows or differs")
    # store_kv writes binary16 of k and v at row pos, nothing else
    k, v = rng.standard_normal(n_kv * hd).astype(np.float32), rng.standard_normal(n_kv * hd).astype(np.float32)
    kc2, vc2 = o.store_kv(kc, vc, k, v, 7)
    ok = (np.array_equal(kc2[7], k.astype(np.float16).view(np.uint16)) and
          np.array_equal(vc2[7], v.astype(np.float16).view(np.uint16)) and
          np.array_equal(np.delete(kc2, 7, 0), np.delete(kc, 7, 0)) and
          np.array_equal(np.delete(vc2, 7, 0), np.delete(vc, 7, 0)))
    if not ok:
        fails.append("store_kv: row pos is not binary16(k), binary16(v), or other rows changed")
    fails += check_argmax(o, rng)
    return fails


def rev8(v: int) -> int:
    return int(f"{v:08b}"[::-1], 2)


def argmax_closed_form(x: np.ndarray) -> int:
    """The reference argmax's result (src/kernels/ops.cuh:467-505) without
    simulating its block: among the indices holding the largest value above
    -1e30f (NaN never qualifies; -0 == +0), the least (rev8(i mod 256), i);
    0 if none qualifies.  Derivation: thread t = i mod 256 keeps its first
    strict maximum, and tree level s pairs slots that differ in bit log2(s),
    the lower slot keeping an equal value."""
    x = np.asarray(x, np.float32)
    cand = np.nonzero(x > np.float32(-1e30))[0]
    if cand.size == 0:
        return 0
    m = x[cand].max()
    tied = cand[x[cand] == m]
    return int(min(tied, key=lambda i: (rev8(int(i) % 256), int(i))))


def check_argmax(o: Oracle, rng):
    fails = []
    base = np.full(1000, -1.0, np.float32)

    def with_max(idx, n=1000, val=9.0):
        x = base[:n].copy() if n <= 1000 else np.full(n, -1.0, np.float32)
        x[list(idx)] = val
        return x
    # hand-derived tie cases of the 256-thread block
    for idx, want in (((1, 256), 256), ((1, 2), 2), ((0, 255), 0), ((10, 700), 700), ((256, 512), 256),
                      ((3, 259), 3), ((127, 129), 129), ((999,), 999)):
        if o.argmax(with_max(idx)) != want:
            fails.append(f"argmax: maxima at {idx} do not give {want}")
    # NaN never wins; nothing above -1e30 gives 0; n == 0 gives 0
    x = with_max((700,))
    x[[3, 900]] = np.nan
    if o.argmax(x) != 700:
        fails.append("argmax: a NaN won")
    for fill in (-np.inf, np.nan, np.float32(-1e30), -2e30):
        if o.argmax(np.full(600, fill, np.float32)) != 0:
            fails.append(f"argmax of all {fill} is not 0")
    x = np.full(600, -2e30, np.float32)
    x[5] = -1.5e30
    if o.argmax(x) != 0:
        fails.append("argmax: a value below -1e30 qualified")
    if o.argmax(np.zeros(0, np.float32)) != 0:
        fails.append("argmax of an empty vector is not 0")
    # -0 and +0 tie: same thread keeps the first, across threads the tree decides
    x = with_max((), val=0)
    x[3], x[259] = -0.0, 0.0
    if o.argmax(x) != 3:
        fails.append("argmax: -0 then +0 in one thread does not keep the first")
    x = with_max(())
    x[1], x[2] = 0.0, -0.0
    if o.argmax(x) != 2:
        fails.append("argmax: +0 at 1 and -0 at 2 do not tie")
    # many ties at many lengths against the closed form
    for n in (1, 7, 255, 256, 257, 1000, 4099, 151936):
        for trial in range(3):
            x = rng.integers(-20, 3 if trial < 2 else 40, n).astype(np.float32)
            if trial == 1:
                x[rng.integers(0, n, max(1, n // 50))] = np.nan
            if o.argmax(x) != argmax_closed_form(x):
                fails.append(f"argmax n={n} trial {trial}: differs from the closed form")
                break
    return fails


ALL_CHECKS = [check_fp16, check_q8_0, check_rms_norm, check_inv_freq, check_rope, check_swiglu,
              check_softmax, check_fused, check_gemv, check_f16_epilogue, check_q6k, check_attention]


def run_all(o: Oracle):
    return {c.__name__: c(o) for c in ALL_CHECKS}
