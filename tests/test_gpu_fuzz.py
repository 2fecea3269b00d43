"""Seeded random-shape parity through the C ABI: every entry point of the hot
path and its decode-step neighbours, at shapes drawn around the launch
planners' boundaries (row lengths at and next to multiples of 4, 64 and 256
lanes, head counts that are odd or zero, pointers 4 bytes off 16-byte
alignment), each case against the CPU oracle with the bars of the per-op
parity tests: fp32 per row max|gpu - ref| <= 1e-5 max|ref|, GEMVs
|y - ref| <= 1e-5 sum|w x| per row, Q8_0 gathers and argmax exactly.

Every case message names the case (seed, shape, offsets), so a failure can be
rerun alone by its seed.
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, assert_bits_equal, assert_rows_close, dev, host, normal, stream, torch_mod
from oracle_py import INTERLEAVED, NEOX, make_q6k_matrix, make_q8_0_table, q6k_dequant_numpy, q8_0_dequant_numpy

pytestmark = pytest.mark.gpu

SEEDS = range(40)
GEMV_TOL = 1e-5


def boundary_len(rng, cap):
    """A length near a planner boundary (multiples of 4, 64, 256, 1024 lanes
    of float4s), or any length up to cap."""
    kind = rng.integers(0, 4)
    if kind == 0:
        return int(rng.integers(1, cap + 1))
    unit = int(rng.choice([4, 64 * 4, 256 * 4, 1024 * 4]))
    m = int(rng.integers(1, max(2, cap // unit + 1)))
    return int(max(1, min(cap, m * unit + int(rng.integers(-3, 4)))))


def dev_at(a, off):
    """`a` on the device `off` elements past an aligned allocation; returns the
    tensor (kept alive) and the shifted pointer."""
    a = np.ascontiguousarray(a)
    buf = np.zeros(a.size + off, a.dtype)
    buf[off:] = a.ravel()
    t = dev(buf)
    return t, t.data_ptr() + off * a.itemsize


def host_at(t, off, shape):
    return host(t)[off:].reshape(shape)


# ------------------------------------------------------------------ rows

@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_rms_norm_rows(oracle, seed):
    rng = np.random.default_rng(1000 + seed)
    rows, n = int(rng.integers(1, 40)), boundary_len(rng, 24000)
    eps = float(rng.choice([1e-5, 1e-6]))
    xo, oo = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    x, w = normal(rng, (rows, n)), normal(rng, n, 1.0, 0.1)
    tx, px = dev_at(x, xo)
    inplace = bool(rng.integers(0, 2)) and xo == oo
    to, po = (tx, px) if inplace else dev_at(np.zeros((rows, n), np.float32), oo)
    F.rms_norm_rows(po, px, dev(w).data_ptr(), rows, n, eps, stream())
    assert_rows_close(host_at(to, oo, (rows, n)), oracle.rms_norm_rows(x, w, eps), n,
                      f"seed {seed}: rms rows {rows}x{n} offsets x{xo} out{oo} inplace={inplace}")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_softmax_rows(oracle, seed):
    rng = np.random.default_rng(2000 + seed)
    rows, n = int(rng.integers(1, 40)), boundary_len(rng, 24000)
    ld = n + int(rng.choice([0, 0, 1, 3, 4, 64]))
    off = int(rng.integers(0, 2))
    x = normal(rng, (rows, ld), 0.0, float(rng.choice([1.0, 3.0, 30.0])))
    tx, px = dev_at(x, off)
    F.softmax_rows(px, rows, n, ld, stream())
    got = host_at(tx, off, (rows, ld))
    what = f"seed {seed}: softmax rows {rows}x{n} ld {ld} offset {off}"
    assert np.array_equal(got[:, n:], x[:, n:]), f"{what}: wrote beyond n"
    assert_rows_close(got[:, :n], oracle.softmax_rows(x, n)[:, :n], n, what)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_softmax_causal(oracle, seed):
    rng = np.random.default_rng(3000 + seed)
    heads, sq = int(rng.integers(1, 4)), int(rng.integers(1, 200))
    sk = sq + int(rng.choice([0, 0, 1, int(rng.integers(0, 3000))]))
    off = int(rng.integers(0, 2))
    s = (rng.standard_normal((heads, sq, sk)) * 3 / np.sqrt(128)).astype(np.float32)
    mask = np.arange(sk)[None, :] > (np.arange(sq)[:, None] + (sk - sq))
    s[:, mask] = -np.inf
    ts, ps = dev_at(s, off)
    F.softmax_causal(ps, heads, sq, sk, stream())
    got = host_at(ts, off, (heads, sq, sk))
    what = f"seed {seed}: causal {heads}x{sq}x{sk} offset {off}"
    assert_rows_close(got, oracle.softmax_causal(s), sk, what)
    assert np.all(got[:, mask] == 0), f"{what}: masked keys must be exactly 0"


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_swiglu(oracle, seed):
    rng = np.random.default_rng(4000 + seed)
    n = boundary_len(rng, 300000)
    off = int(rng.integers(0, 2))
    g, u = normal(rng, n), normal(rng, n)
    tg, pg = dev_at(g, off)
    _, pu = dev_at(u, off)
    alias = bool(rng.integers(0, 2))
    to, po = (tg, pg) if alias else dev_at(np.zeros(n, np.float32), off)
    F.swiglu(po, pg, pu, n, stream())
    assert_rows_close(host_at(to, off, (n,)), oracle.silu_mul(g, u), n,
                      f"seed {seed}: swiglu n={n} offset {off} out==gate {alias}")


# --------------------------------------------------------------- per head

HDS = [2, 8, 32, 40, 64, 64, 96, 128, 128, 128, 256, 256]


def head_case(rng, seed):
    T = int(rng.integers(1, 40))
    hd = int(rng.choice(HDS))
    nq, nkv = int(rng.integers(0, 20)), int(rng.integers(0, 9))
    if nq + nkv == 0:
        nq = 1
    style = int(rng.choice([NEOX, INTERLEAVED]))
    base = float(rng.choice([1e4, 5e5, 1e6, 5e6]))
    positions = rng.integers(0, 40000, T).astype(np.int32) if rng.integers(0, 2) else None
    pos0 = int(rng.integers(0, 30000))
    off = int(rng.integers(0, 2)) if rng.integers(0, 3) == 0 else 0
    return T, hd, nq, nkv, style, base, positions, pos0, off


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_rope(oracle, seed):
    rng = np.random.default_rng(5000 + seed)
    T, hd, nq, nkv, style, base, positions, pos0, off = head_case(rng, seed)
    q, k = normal(rng, (T, nq, hd)), normal(rng, (T, nkv, hd))
    tq, pq = dev_at(q, off) if nq else (None, None)
    tk, pk = dev_at(k, off) if nkv else (None, None)
    pp = dev(positions).data_ptr() if positions is not None else None
    F.rope(pq, pk, T, nq, nkv, hd, pp, pos0, base, style, stream())
    rq, rk = oracle.rope_rows(q, k if nkv else None, positions, pos0, base, style)
    what = f"seed {seed}: rope T={T} {nq}+{nkv}x{hd} style {style} positions {positions is not None} off {off}"
    if nq:
        assert_rows_close(host_at(tq, off, q.shape), rq, hd, what + " q")
    if nkv:
        assert_rows_close(host_at(tk, off, k.shape), rk, hd, what + " k")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_qk_norm_rope(oracle, seed):
    rng = np.random.default_rng(6000 + seed)
    T, hd, nq, nkv, style, base, positions, pos0, off = head_case(rng, seed)
    q, k = normal(rng, (T, nq, hd)), normal(rng, (T, nkv, hd))
    wq, wk = normal(rng, hd, 1.0, 0.1), normal(rng, hd, 1.0, 0.1)
    tq, pq = dev_at(q, off) if nq else (None, None)
    tk, pk = dev_at(k, off) if nkv else (None, None)
    pp = dev(positions).data_ptr() if positions is not None else None
    F.qk_norm_rope(pq, pk, dev(wq).data_ptr(), dev(wk).data_ptr(), T, nq, nkv, hd, 1e-6, pp, pos0, base, style,
                   stream())
    rq, rk = oracle.qk_norm_rope(q, k if nkv else None, wq, wk, 1e-6, positions, pos0, base, style)
    what = f"seed {seed}: qk_norm_rope T={T} {nq}+{nkv}x{hd} style {style} off {off}"
    if nq:
        assert_rows_close(host_at(tq, off, q.shape), rq, hd, what + " q")
    if nkv:
        assert_rows_close(host_at(tk, off, k.shape), rk, hd, what + " k")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_rms_norm_rope(oracle, seed):
    rng = np.random.default_rng(7000 + seed)
    T, hd, nq, nkv, style, base, positions, pos0, off = head_case(rng, seed)
    nq = max(nq, 1)
    x, w = normal(rng, (T, nq * hd)), normal(rng, nq * hd, 1.0, 0.1)
    k = normal(rng, (T, nkv, hd))
    tx, px = dev_at(x, off)
    tk, pk = dev_at(k, off) if nkv else (None, None)
    inplace = bool(rng.integers(0, 2))
    to, po = (tx, px) if inplace else dev_at(np.zeros_like(x), off)
    pp = dev(positions).data_ptr() if positions is not None else None
    F.rms_norm_rope(po, px, dev(w).data_ptr(), pk, T, nq, nkv, hd, 1e-5, pp, pos0, base, style, stream())
    ro, rk = oracle.rms_norm_rope(x, w, k if nkv else None, nq, hd, 1e-5, positions, pos0, base, style)
    what = f"seed {seed}: rms_norm_rope T={T} {nq}+{nkv}x{hd} style {style} off {off} inplace {inplace}"
    assert_rows_close(host_at(to, off, x.shape), ro, hd, what + " out")
    if nkv:
        assert_rows_close(host_at(tk, off, k.shape), rk, hd, what + " k")


# -------------------------------------------------------------- epilogues

def f16_close(got16, ref32, row_len, what):
    """binary16 bits within half a binary16 ulp of the oracle's fp32 value,
    plus the fp32 row tolerance."""
    g = np.asarray(got16, np.uint16).view(np.float16).astype(np.float64).reshape(-1, row_len)
    r = np.asarray(ref32, np.float64).reshape(-1, row_len)
    bound = 2.0 ** -11 * np.abs(r) + 1e-5 * np.max(np.abs(r), axis=1, keepdims=True) + 2.0 ** -25
    assert not (np.abs(g - r) > bound).any(), f"{what}: binary16 values beyond half an ulp + 1e-5"


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_residual_rms_norm_f16(oracle, seed):
    torch = torch_mod()
    rng = np.random.default_rng(14000 + seed)
    rows, n = int(rng.integers(1, 12)), boundary_len(rng, 20000)
    with_res = bool(rng.integers(0, 2))
    off = int(rng.integers(0, 2))
    h0, res, w = normal(rng, (rows, n)), normal(rng, (rows, n)), normal(rng, n, 1.0, 0.1)
    th, ph = dev_at(h0, off)
    _, pr = dev_at(res, off) if with_res else (None, None)
    normed = torch.zeros(rows * n + off, device="cuda")
    o16 = torch.zeros(rows * n + off, dtype=torch.int16, device="cuda")
    LIVE.extend([normed, o16])
    F.residual_rms_norm_f16(ph, pr, dev(w).data_ptr(), normed.data_ptr() + 4 * off, o16.data_ptr() + 2 * off,
                            rows, n, 1e-6, stream())
    ref_h, ref_n, _ = oracle.residual_rms_norm_f16(h0, res if with_res else None, w, 1e-6)
    what = f"seed {seed}: residual_rms_norm_f16 {rows}x{n} residual {with_res} offset {off}"
    assert_bits_equal(host_at(th, off, (rows, n)), ref_h, what + " hidden")
    got_n = host(normed)[off:].reshape(rows, n)
    assert_rows_close(got_n, ref_n, n, what + " normed")
    got16 = host(o16)[off:].view(np.uint16).reshape(rows, n)
    assert np.array_equal(got16, got_n.astype(np.float16).view(np.uint16)), what + ": f16 != RNE(own fp32)"
    f16_close(got16, ref_n, n, what)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_swiglu_f16(oracle, seed):
    torch = torch_mod()
    rng = np.random.default_rng(15000 + seed)
    n = boundary_len(rng, 300000)
    off = int(rng.integers(0, 2))
    g, u = normal(rng, n), normal(rng, n)
    _, pg = dev_at(g, off)
    _, pu = dev_at(u, off)
    out = torch.zeros(n + off, device="cuda")
    o16 = torch.zeros(n + off, dtype=torch.int16, device="cuda")
    LIVE.extend([out, o16])
    F.swiglu_f16(o16.data_ptr() + 2 * off, out.data_ptr() + 4 * off, pg, pu, n, stream())
    ref, _ = oracle.swiglu_f16(g, u)
    what = f"seed {seed}: swiglu_f16 n={n} offset {off}"
    got = host(out)[off:]
    assert_rows_close(got, ref, n, what + " fp32")
    got16 = host(o16)[off:].view(np.uint16)
    assert np.array_equal(got16, got.astype(np.float16).view(np.uint16)), what + ": f16 != RNE(own fp32)"
    f16_close(got16, ref, n, what)


# ------------------------------------------------------------------ Q8_0

@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gather(oracle, seed):
    rng = np.random.default_rng(8000 + seed)
    vocab, dim, T = int(rng.integers(1, 3000)), 32 * int(rng.integers(1, 200)), int(rng.integers(1, 300))
    table = make_q8_0_table(rng, vocab, dim)
    ids = rng.integers(0, vocab, T).astype(np.int32)
    if rng.integers(0, 3) == 0:
        ids[rng.integers(0, T)] = int(rng.choice([-1, vocab, 2**31 - 1]))
    toff, ooff = int(rng.choice([0, 0, 1, 2])), int(rng.integers(0, 2))
    _, ptab = dev_at(table.reshape(-1), toff)
    to, po = dev_at(np.zeros((T, dim), np.float32), ooff)
    F.embed_q8_0_gather(po, ptab, vocab, dev(ids).data_ptr(), T, dim, stream())
    ref, _ = oracle.embed_q8_0_gather(table, vocab, ids, dim)
    assert_bits_equal(host_at(to, ooff, (T, dim)), ref,
                      f"seed {seed}: gather V={vocab} dim={dim} T={T} table+{toff} out+{ooff}")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gather_rms_norm(oracle, seed):
    rng = np.random.default_rng(9000 + seed)
    vocab, dim, T = int(rng.integers(1, 3000)), 32 * int(rng.integers(1, 200)), int(rng.integers(1, 300))
    table = make_q8_0_table(rng, vocab, dim)
    ids = rng.integers(0, vocab, T).astype(np.int32)
    if rng.integers(0, 3) == 0:
        ids[rng.integers(0, T)] = -5
    toff, ooff = int(rng.choice([0, 0, 1, 2])), int(rng.integers(0, 2))
    w = normal(rng, dim, 1.0, 0.1)
    _, ptab = dev_at(table.reshape(-1), toff)
    to, po = dev_at(np.zeros((T, dim), np.float32), ooff)
    F.embed_q8_0_gather_rms_norm(po, ptab, vocab, dev(ids).data_ptr(), T, dim, dev(w).data_ptr(), 1e-6, stream())
    ref, _ = oracle.embed_q8_0_gather_rms_norm(table, vocab, ids, dim, w, 1e-6)
    assert_rows_close(host_at(to, ooff, (T, dim)), ref, dim,
                      f"seed {seed}: gather+norm V={vocab} dim={dim} T={T} table+{toff} out+{ooff}")


def assert_gemv(got, ref, scale, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{what}: NaN rows differ"
    fin = np.isfinite(ref)
    err = np.abs(got[fin] - ref[fin])
    bad = err > GEMV_TOL * scale[fin]
    assert not bad.any(), (f"{what}: {int(bad.sum())} rows beyond the bar; worst err/scale "
                           f"{np.max(err / np.maximum(scale[fin], 1e-300)):.3g}")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gemv_q8_0(oracle, seed):
    torch = torch_mod()
    rng = np.random.default_rng(10000 + seed)
    K = 32 * int(rng.integers(1, 400))  # up to 12800: every slot count and the wide kernel
    M = int(rng.integers(1, min(4000, 8_000_000 // K) + 1))
    table = make_q8_0_table(rng, M, K)
    x = normal(rng, K)
    toff, xoff = int(rng.choice([0, 0, 2])), int(rng.integers(0, 2))  # blocks hold an fp16: 2-byte aligned
    _, ptab = dev_at(table.reshape(-1), toff)
    _, px = dev_at(x, xoff)
    y = torch.full((M,), float("nan"), device="cuda")
    LIVE.append(y)
    F.gemv_q8_0(ptab, px, y.data_ptr(), M, K, stream())
    scale = np.abs(q8_0_dequant_numpy(table, np.arange(M), K).astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert_gemv(host(y), oracle.gemv_q8_0(table, x), scale, f"seed {seed}: gemv_q8_0 {M}x{K} table+{toff} x+{xoff}")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gemv_q6k(oracle, seed):
    torch = torch_mod()
    rng = np.random.default_rng(11000 + seed)
    K = 256 * int(rng.integers(1, 48))
    M = int(rng.integers(1, min(3000, 8_000_000 // K) + 1))
    W = make_q6k_matrix(rng, M, K)
    x16 = (rng.standard_normal(K)).astype(np.float16).view(np.uint16)
    woff = int(rng.choice([0, 0, 0, 1]))  # in 2-byte units: the blocks' own alignment
    _, pW = dev_at(W.reshape(-1).view(np.int16), woff)
    _, px = dev_at(x16.view(np.int16), int(rng.choice([0, 0, 1])))
    y = torch.full((M,), float("nan"), device="cuda")
    LIVE.append(y)
    F.gemv_q6k(pW, px, y.data_ptr(), M, K, stream())
    scale = np.abs(q6k_dequant_numpy(W, K)) @ np.abs(x16.view(np.float16).astype(np.float64))
    assert_gemv(host(y), oracle.gemv_q6k(W, x16), scale, f"seed {seed}: gemv_q6k {M}x{K} W+{2 * woff}B")


# -------------------------------------------------------- decode attention

@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention(oracle, seed):
    torch = torch_mod()
    rng = np.random.default_rng(12000 + seed)
    n_kv = int(rng.choice([1, 2, 4, 8]))
    n_q = n_kv * int(rng.choice([1, 2, 3, 4, 5, 8]))
    hd = int(rng.choice([128, 128, 128, 64, 96]))
    ctx = int(rng.integers(1, 3500))
    seq = int(rng.integers(1, ctx + 1))
    kc = rng.standard_normal((ctx, n_kv * hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, n_kv * hd)).astype(np.float16).view(np.uint16)
    q = (rng.standard_normal(n_q * hd) * float(rng.choice([0.1, 0.3, 1.0]))).astype(np.float32)
    out = torch.full((n_q * hd,), float("nan"), device="cuda")
    ws = torch.full((n_q * ctx,), float("nan"), device="cuda")
    LIVE.extend([out, ws])
    F.gqa_attention(out.data_ptr(), dev(q).data_ptr(), dev(kc.view(np.int16)).data_ptr(),
                    dev(vc.view(np.int16)).data_ptr(), hd, n_q, n_kv, seq, ctx, ws.data_ptr(), stream())
    got = host(out).reshape(n_q, hd).astype(np.float64)
    ref = oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq).reshape(n_q, hd)
    V = np.abs(vc[:seq].view(np.float16).astype(np.float64).reshape(seq, n_kv, hd))
    for h in range(n_q):
        scale = V[:, h // (n_q // n_kv), :].max()
        err = np.max(np.abs(got[h] - ref[h]))
        assert err <= 1e-5 * scale, (f"seed {seed}: attention {n_q}/{n_kv}x{hd} seq {seq} ctx {ctx}: head {h} "
                                     f"err {err:.3g} > 1e-5 * {scale:.3g}")


# ----------------------------------------------------------------- argmax

@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_argmax(oracle, seed):
    torch = torch_mod()
    rng = np.random.default_rng(13000 + seed)
    n = boundary_len(rng, 400000)
    kind = int(rng.integers(0, 3))
    if kind == 0:
        x = rng.integers(-20, 3, n).astype(np.float32)  # many ties
    elif kind == 1:
        x = rng.standard_normal(n).astype(np.float32)
    else:
        x = np.full(n, -2.0, np.float32)
        x[rng.choice(n, min(n, int(rng.integers(1, 9))), replace=False)] = 5.0
    if rng.integers(0, 3) == 0:
        x[rng.integers(0, n)] = np.nan
    off = int(rng.integers(0, 4))
    _, px = dev_at(x, off)
    want = oracle.argmax(x)
    r = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    ws_bytes = int(rng.choice([8, 64, 8192, 1 << 16]))
    ws = torch.full((ws_bytes // 8,), -1, dtype=torch.int64, device="cuda")
    LIVE.extend([r, ws])
    what = f"seed {seed}: argmax n={n} kind {kind} offset {off}"
    F.argmax(px, r.data_ptr(), n, stream())
    assert int(host(r)[0]) == want, what + " one workgroup"
    F.argmax_ws(px, r.data_ptr(), n, ws.data_ptr(), ws_bytes, stream())
    assert int(host(r)[0]) == want, what + f" workspace {ws_bytes} B"


# ------------------------------------- attention with its q/k prologue fused

@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention_qk_equals_two_calls(seed):
    """fence_gqa_attention_qk_f16 (QK-norm, RoPE and the KV store inside the
    attention launch) against qk_norm_rope_store_kv then gqa_attention_f16:
    outputs and caches bit for bit."""
    from test_gpu_decode_fusions import attention_qk_operands, run_attention_qk
    rng = np.random.default_rng(16000 + seed)
    nkv = int(rng.choice([1, 2, 4, 8]))
    nq = nkv * int(rng.choice([1, 2, 3, 4, 5, 8]))
    hd = int(rng.choice([128, 128, 128, 64]))
    ctx = int(rng.integers(1, 4200))
    pos = int(rng.choice([0, ctx - 1, int(rng.integers(0, ctx)), min(ctx - 1, 64 * int(rng.integers(0, 40)))]))
    norm = bool(rng.integers(0, 4))
    style = int(rng.choice([NEOX, INTERLEAVED]))
    ws_floats = int(rng.choice([1, 2, 4])) * nq * ctx + int(rng.integers(0, 200))
    ops = attention_qk_operands(rng, nq, nkv, hd, ctx, norm)
    got = run_attention_qk(ops, nq, nkv, hd, pos, 1e6, style, ws_floats, fused=True)
    ref = run_attention_qk(ops, nq, nkv, hd, pos, 1e6, style, ws_floats, fused=False)
    what = f"seed {seed}: attention_qk {nq}/{nkv}x{hd} pos {pos} ctx {ctx} norm {norm} style {style} ws {ws_floats}"
    for g, r, part in zip(got, ref, ("fp32 out", "binary16 out", "k cache", "v cache")):
        kind = np.uint32 if g.dtype == np.float32 else np.uint16
        assert np.array_equal(g.view(kind), r.view(kind)), f"{what}: {part}"


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention_qk_arrive_equals_two_launches(seed):
    """fence_gqa_attention_qk_f16_arrive (the last workgroup of each head group
    merges the splits) against fence_gqa_attention_qk_f16 (split + merge
    kernels): outputs and caches bit for bit, arrival counters zero after."""
    from test_gpu_attention_arrive import Setup, bits_equal, operands
    rng = np.random.default_rng(17000 + seed)
    nkv = int(rng.choice([1, 2, 4, 8]))
    nq = nkv * int(rng.choice([1, 2, 3, 4, 5, 8]))
    hd = int(rng.choice([128, 128, 128, 64]))
    ctx = int(rng.integers(1, 4200))
    pos = int(rng.choice([0, ctx - 1, int(rng.integers(0, ctx)), min(ctx - 1, 64 * int(rng.integers(0, 40)))]))
    norm = bool(rng.integers(0, 4))
    style = int(rng.choice([NEOX, INTERLEAVED]))
    ws_floats = int(rng.choice([1, 2, 4])) * nq * ctx + int(rng.integers(0, 200))
    s = Setup(operands(rng, nq, nkv, hd, ctx, norm), ws_floats)
    what = f"seed {seed}: attention_qk_arrive {nq}/{nkv}x{hd} pos {pos} ctx {ctx} norm {norm} style {style} ws {ws_floats}"
    ref32, ref16 = s.call(pos, style, arrive=False)
    kc, vc = s.kcd.clone(), s.vcd.clone()
    got32, got16 = s.call(pos, style, arrive=True)
    assert bits_equal(got32, ref32), f"{what}: fp32 out"
    assert bits_equal(got16, ref16), f"{what}: binary16 out"
    assert bits_equal(s.kcd, kc) and bits_equal(s.vcd, vc), f"{what}: caches"
    assert not host(s.arrive).any(), f"{what}: arrival counters left nonzero"


# ------------------------------------------- Q6_K launches of several matrices

def q6k_shape(rng, max_blocks=40, budget=6_000_000):
    K = 256 * int(rng.integers(1, max_blocks + 1))
    return K, max(1, budget // K)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gemv_q6k_multi_equals_separate_launches(seed):
    import test_gpu_q6k as q6
    rng = np.random.default_rng(17000 + seed)
    K, cap = q6k_shape(rng)
    n = int(rng.integers(1, 5))
    Ms = [int(rng.integers(0, min(3000, cap // n) + 1)) for _ in range(n)]
    if not any(Ms):
        Ms[0] = 1
    Ws = [make_q6k_matrix(rng, M, K) if M else np.zeros((0, K // 256 * 210), np.uint8) for M in Ms]
    x = q6.rand_x(rng, K)
    got = q6.run_q6k_multi([W if W.size else None for W in Ws], x, Ms, K)
    for i, (W, M) in enumerate(zip(Ws, Ms)):
        if M:
            assert np.array_equal(got[i].view(np.uint32), q6.run_q6k(W, x, M, K).view(np.uint32)), \
                f"seed {seed}: multi {Ms} K={K}: matrix {i} differs from its own launch"


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gemv_q6k_swiglu_equals_unfused(seed):
    import test_gpu_q6k as q6
    rng = np.random.default_rng(18000 + seed)
    K, cap = q6k_shape(rng)
    M = int(rng.integers(1, min(6000, cap // 2) + 1))
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    x = q6.rand_x(rng, K, std=0.5)
    got16, got32 = q6.run_swiglu(Wg, Wu, x, M, K)
    ref16, ref32 = q6.unfused_swiglu(Wg, Wu, x, M, K)
    what = f"seed {seed}: gate/up pair {M}x{K}"
    assert np.array_equal(got32.view(np.uint32), ref32.view(np.uint32)), what + ": fp32 act"
    assert np.array_equal(got16, ref16), what + ": binary16 act"


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_gemv_q6k_rms_prologue_equals_norm_then_gemv(seed):
    """The GEMVs that compute their own layer-boundary input row: bit for bit
    the norm launch followed by the plain GEMV (multi and gate/up pair)."""
    import test_gpu_gemv_rms as gr
    rng = np.random.default_rng(19000 + seed)
    K, cap = q6k_shape(rng, max_blocks=36)
    residual = bool(rng.integers(0, 4))
    hid, res, w = gr.row(rng, K, residual)
    if rng.integers(0, 2):
        n = int(rng.integers(1, 4))
        Ms = [int(rng.integers(0, min(2500, cap // n) + 1)) for _ in range(n)]
        if not any(Ms):
            Ms[0] = 1
        Ws = [make_q6k_matrix(rng, M, K) if M else np.zeros((0, K // 256 * 210), np.uint8) for M in Ms]
        gr.check_multi(Ws, Ms, K, hid, res, w, hid_off=int(rng.choice([0, 0, 0, 1])))
        return
    M = int(rng.integers(1, min(5000, cap // 2) + 1))
    Wg, Wu = make_q6k_matrix(rng, M, K), make_q6k_matrix(rng, M, K)
    got16, got32, hout, x16 = gr.run_pair(Wg, Wu, M, K, hid, res, w)
    ref_h, ref_x = gr.unfused_input(hid, res, w, K)
    what = f"seed {seed}: pair with norm {M}x{K} residual {residual}"
    assert np.array_equal(x16, ref_x), what + ": x"
    if residual:
        assert np.array_equal(hout.view(np.uint32), ref_h.view(np.uint32)), what + ": hidden_out"
    ref16, ref32 = __import__("test_gpu_q6k").run_swiglu(Wg, Wu, ref_x, M, K)
    assert np.array_equal(got16, ref16), what + ": binary16 act"
    assert np.array_equal(got32.view(np.uint32), ref32.view(np.uint32)), what + ": fp32 act"


# ------------------------------- QK-norm -> RoPE -> KV store, and attention_f16

@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_qk_norm_rope_store_kv_equals_separate_calls(seed):
    """The fused prologue of a decode step against qk_norm_rope (or rope)
    then one store_kv per token: q, k and both caches bit for bit, with
    device positions (distinct, in range) or consecutive ones from pos0."""
    import test_gpu_decode_fusions as df
    rng = np.random.default_rng(20000 + seed)
    T = int(rng.integers(1, 9))
    hd = int(rng.choice([64, 96, 128, 128, 128, 256]))
    nkv = int(rng.integers(1, 9))
    nq = nkv * int(rng.integers(1, 6))
    ctx = int(rng.integers(T, 5000))
    norm = bool(rng.integers(0, 4))
    style = int(rng.choice([NEOX, INTERLEAVED]))
    positions = rng.choice(ctx, T, replace=False).astype(np.int32) if rng.integers(0, 2) else None
    pos0 = int(rng.integers(0, ctx - T + 1))
    q = rng.standard_normal((T, nq, hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kc, vc = df.caches(rng, ctx, nkv * hd)
    got = df.run_fused_kv(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, positions, pos0, 1e6, style)
    ref = df.run_separate(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, positions, pos0, 1e6, style)
    what = (f"seed {seed}: qk_norm_rope_store_kv T={T} {nq}/{nkv}x{hd} ctx {ctx} norm {norm} style {style} "
            f"positions {positions is not None}")
    for g, r, part in zip(got, ref, ("q", "k", "k cache", "v cache")):
        kind = np.uint32 if g.dtype == np.float32 else np.uint16
        assert np.array_equal(g.view(kind), r.view(kind)), f"{what}: {part}"


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention_f16_equals_attention_then_conversion(seed):
    torch = torch_mod()
    rng = np.random.default_rng(21000 + seed)
    nkv = int(rng.choice([1, 2, 4, 8]))
    n_q = nkv * int(rng.choice([1, 2, 3, 4, 8]))
    hd = int(rng.choice([64, 96, 128, 128, 128]))
    ctx = int(rng.integers(1, 4200))
    seq = int(rng.integers(1, ctx + 1))
    ws_floats = int(rng.choice([1, 2, 4])) * n_q * ctx
    kc = rng.standard_normal((ctx, nkv * hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, nkv * hd)).astype(np.float16).view(np.uint16)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    qd, kd, vd = dev(q), dev(kc.view(np.int16)), dev(vc.view(np.int16))
    ws = torch.empty(ws_floats, dtype=torch.float32, device="cuda")
    ref32 = torch.empty(n_q * hd, dtype=torch.float32, device="cuda")
    ref16 = torch.empty(n_q * hd, dtype=torch.int16, device="cuda")
    got32 = torch.full((n_q * hd,), float("nan"), dtype=torch.float32, device="cuda")
    got16 = torch.full((n_q * hd,), -1, dtype=torch.int16, device="cuda")
    LIVE.extend([ws, ref32, ref16, got32, got16])
    both16 = torch.full((n_q * hd,), -1, dtype=torch.int16, device="cuda")
    LIVE.append(both16)
    # fp32 and binary16 from one call; binary16 alone from another
    F.gqa_attention_f16(got32.data_ptr(), both16.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), hd, n_q,
                        nkv, seq, ctx, ws.data_ptr(), ws_floats, stream())
    F.f32_to_f16(ref16.data_ptr(), got32.data_ptr(), n_q * hd, stream())
    F.gqa_attention_f16(None, got16.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), hd, n_q, nkv, seq, ctx,
                        ws.data_ptr(), ws_floats, stream())
    what = f"seed {seed}: attention_f16 {n_q}/{nkv}x{hd} seq {seq} ctx {ctx} ws {ws_floats}"
    assert np.array_equal(host(both16), host(ref16)), what + ": binary16 != RNE(own fp32)"
    assert np.array_equal(host(got16), host(ref16)), what + ": binary16-only call differs"
    if ws_floats == n_q * ctx:  # the reference's score_buf size: the plain entry point splits the same way
        F.gqa_attention(ref32.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), hd, n_q, nkv, seq, ctx,
                        ws.data_ptr(), stream())
        assert np.array_equal(host(got32).view(np.uint32), host(ref32).view(np.uint32)), what + ": fp32"
