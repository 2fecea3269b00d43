"""GPU checks of the decode-step fusions that replace two reference launches
with one: fence_gqa_attention_f16 (gqa_attention + f32_to_f16,
src/model/qwen3.cu:305-310) and fence_qk_norm_rope_store_kv
(rms_norm_per_head x2 + apply_rope + store_kv, src/model/qwen3.cu:292-303).

The bar is bit equality with the separate entry points on the same operands
(each of which has its own oracle parity tests); one case per function is
also checked against the oracle directly.
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod

pytestmark = pytest.mark.gpu


def caches(rng, ctx, kv_dim):
    return (rng.standard_normal((ctx, kv_dim)).astype(np.float16).view(np.uint16),
            rng.standard_normal((ctx, kv_dim)).astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("hd,n_q,n_kv,seq,ctx", [
    (128, 32, 8, 1, 4096), (128, 32, 8, 100, 4096), (128, 32, 8, 2916, 4096), (128, 32, 8, 4096, 4096),
    (128, 8, 8, 300, 512), (64, 16, 4, 333, 512), (96, 16, 4, 333, 512)])
@pytest.mark.parametrize("with_fp32", [True, False])
def test_attention_f16_equals_attention_then_conversion(oracle, hd, n_q, n_kv, seq, ctx, with_fp32):
    torch = torch_mod()
    rng = np.random.default_rng(seq + hd)
    kc, vc = caches(rng, ctx, n_kv * hd)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    qd, kd, vd = dev(q), dev(kc.view(np.int16)), dev(vc.view(np.int16))
    ws = torch.empty(n_q * ctx, dtype=torch.float32, device="cuda")
    ref32 = torch.empty(n_q * hd, dtype=torch.float32, device="cuda")
    ref16 = torch.empty(n_q * hd, dtype=torch.int16, device="cuda")
    got32 = torch.full((n_q * hd,), float("nan"), dtype=torch.float32, device="cuda")
    got16 = torch.full((n_q * hd,), -1, dtype=torch.int16, device="cuda")
    LIVE.extend([ws, ref32, ref16, got32, got16])
    F.gqa_attention(ref32.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), hd, n_q, n_kv, seq, ctx,
                    ws.data_ptr(), stream())
    F.f32_to_f16(ref16.data_ptr(), ref32.data_ptr(), n_q * hd, stream())
    F.gqa_attention_f16(got32.data_ptr() if with_fp32 else None, got16.data_ptr(), qd.data_ptr(), kd.data_ptr(),
                        vd.data_ptr(), hd, n_q, n_kv, seq, ctx, ws.data_ptr(), stream=stream())
    assert np.array_equal(host(got16), host(ref16))
    if with_fp32:
        assert np.array_equal(host(got32).view(np.uint32), host(ref32).view(np.uint32))
    if seq == 100 and hd == 128:
        r = oracle.f32_to_f16(oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq))
        diff = np.abs(host(got16).view(np.float16).astype(np.float64) - r.view(np.float16).astype(np.float64))
        assert np.max(diff) <= 2.0 ** -10 * np.max(np.abs(r.view(np.float16).astype(np.float64)))


@pytest.mark.parametrize("seq", [1, 65, 700, 2916, 4096])
def test_attention_f16_larger_workspace(oracle, seq):
    """score_buf four times the reference's size: more splits, the same
    result within the attention bar (and exactly V[0] at one position)."""
    torch = torch_mod()
    n_q, n_kv, hd, ctx = 32, 8, 128, 4096
    rng = np.random.default_rng(seq + 5)
    kc, vc = caches(rng, ctx, n_kv * hd)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    ws = torch.empty(4 * n_q * ctx, dtype=torch.float32, device="cuda")
    got32 = torch.full((n_q * hd,), float("nan"), dtype=torch.float32, device="cuda")
    got16 = torch.empty(n_q * hd, dtype=torch.int16, device="cuda")
    LIVE.extend([ws, got32, got16])
    F.gqa_attention_f16(got32.data_ptr(), got16.data_ptr(), dev(q).data_ptr(), dev(kc.view(np.int16)).data_ptr(),
                        dev(vc.view(np.int16)).data_ptr(), hd, n_q, n_kv, seq, ctx, ws.data_ptr(), 4 * n_q * ctx,
                        stream())
    got = host(got32).reshape(n_q, hd).astype(np.float64)
    ref = oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq).reshape(n_q, hd)
    V = np.abs(vc[:seq].view(np.float16).astype(np.float64).reshape(-1, n_kv, hd))
    for h in range(n_q):
        assert np.max(np.abs(got[h] - ref[h])) <= 1e-5 * V[:, h // 4, :].max(), f"head {h}"
    assert np.array_equal(host(got16).view(np.uint16), host(got32).astype(np.float16).view(np.uint16))
    if seq == 1:
        v0 = vc[0].view(np.float16).astype(np.float32).reshape(n_kv, hd)
        assert np.array_equal(host(got32).reshape(n_q, hd), v0[np.arange(n_q) // 4])


def run_fused_kv(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, positions, pos0, base, style, offset=0):
    torch = torch_mod()
    ctx = kc.shape[0]
    qd, kd, vdv = dev(q), dev(k), dev(v)
    kcd, vcd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    pd = None if positions is None else dev(np.asarray(positions, np.int32))
    F.qk_norm_rope_store_kv(qd.data_ptr(), kd.data_ptr(), vdv.data_ptr(),
                            None if wq is None else dev(wq).data_ptr(), None if wk is None else dev(wk).data_ptr(),
                            kcd.data_ptr(), vcd.data_ptr(), ctx, T, nq, nkv, hd, 1e-6,
                            None if pd is None else pd.data_ptr(), pos0, base, style, stream())
    return host(qd), host(kd), host(kcd).view(np.uint16), host(vcd).view(np.uint16)


def run_separate(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, positions, pos0, base, style):
    """qk_norm_rope (or rope) then store_kv per token, the reference's order."""
    ctx = kc.shape[0]
    qd, kd, vdv = dev(q), dev(k), dev(v)
    kcd, vcd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    pd = None if positions is None else dev(np.asarray(positions, np.int32))
    pp = None if pd is None else pd.data_ptr()
    if wq is None:
        F.rope(qd.data_ptr(), kd.data_ptr(), T, nq, nkv, hd, pp, pos0, base, style, stream())
    else:
        F.qk_norm_rope(qd.data_ptr(), kd.data_ptr(), dev(wq).data_ptr(), dev(wk).data_ptr(), T, nq, nkv, hd, 1e-6,
                       pp, pos0, base, style, stream())
    kv = nkv * hd
    for t in range(T):
        pos = positions[t] if positions is not None else pos0 + t
        if 0 <= pos < ctx:
            F.store_kv(kcd.data_ptr(), vcd.data_ptr(), kd.data_ptr() + 4 * t * kv, vdv.data_ptr() + 4 * t * kv, pos,
                       kv, ctx, stream())
    return host(qd), host(kd), host(kcd).view(np.uint16), host(vcd).view(np.uint16)


@pytest.mark.parametrize("T,nq,nkv,hd,norm,style,pos0", [
    (1, 32, 8, 128, True, F.ROPE_NEOX, 2915),     # Qwen3-4B decode step
    (1, 32, 8, 128, False, F.ROPE_NEOX, 17),      # no QK-norm weights: RoPE only
    (1, 64, 8, 128, True, F.ROPE_NEOX, 4095),     # last position; two slots per lane
    (5, 16, 4, 128, True, F.ROPE_INTERLEAVED, 40),
    (3, 8, 2, 64, True, F.ROPE_NEOX, 0),
    (2, 12, 4, 96, True, F.ROPE_NEOX, 9),         # head_dim 96: the scalar kernel
])
def test_qk_norm_rope_store_kv_equals_separate_calls(oracle, T, nq, nkv, hd, norm, style, pos0):
    rng = np.random.default_rng(T * 1000 + nq + hd)
    ctx = 4096
    q = rng.standard_normal((T, nq, hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kc, vc = caches(rng, ctx, nkv * hd)
    got = run_fused_kv(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, None, pos0, 1e6, style)
    ref = run_separate(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, None, pos0, 1e6, style)
    for g, r, what in zip(got, ref, ("q", "k", "k cache", "v cache")):
        assert np.array_equal(g.view(np.uint32 if g.dtype == np.float32 else np.uint16),
                              r.view(np.uint32 if r.dtype == np.float32 else np.uint16)), what
    if T == 1 and norm and style == F.ROPE_NEOX:  # and the oracle's store_kv of the oracle's k
        _, rk = oracle.qk_norm_rope(q, k, wq, wk, 1e-6, None, pos0, 1e6, style)
        rkc, rvc = oracle.store_kv(kc, vc, rk.reshape(-1), v.reshape(-1), pos0)
        assert np.array_equal(got[3], rvc)
        d = np.abs(got[2][pos0].view(np.float16).astype(np.float64) - rkc[pos0].view(np.float16).astype(np.float64))
        assert np.max(d) <= 2.0 ** -10 * np.max(np.abs(rkc[pos0].view(np.float16).astype(np.float64)))
        other = np.arange(ctx) != pos0
        assert np.array_equal(got[2][other], kc[other]) and np.array_equal(got[3][other], vc[other])


def test_qk_norm_rope_store_kv_device_positions_skip_out_of_range():
    """Positions from a device array: one outside [0, max_ctx) stores nothing."""
    T, nq, nkv, hd, ctx = 4, 16, 4, 128, 64
    rng = np.random.default_rng(77)
    q = rng.standard_normal((T, nq, hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kc, vc = caches(rng, ctx, nkv * hd)
    positions = [5, 63, 64, 2]  # 64 is past max_ctx
    got = run_fused_kv(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, positions, 0, 1e6, F.ROPE_NEOX)
    ref = run_separate(q, k, v, wq, wk, kc, vc, T, nq, nkv, hd, positions, 0, 1e6, F.ROPE_NEOX)
    assert np.array_equal(got[2], ref[2]) and np.array_equal(got[3], ref[3])
    assert np.array_equal(got[1].view(np.uint32), ref[1].view(np.uint32))


def attention_qk_operands(rng, nq, nkv, hd, ctx, norm):
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    k = rng.standard_normal((nkv, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kc, vc = caches(rng, ctx, nkv * hd)
    return q, k, v, wq, wk, kc, vc


def run_attention_qk(ops, nq, nkv, hd, pos, base, style, ws_floats, fused):
    """fused: fence_gqa_attention_qk_f16; else qk_norm_rope_store_kv then
    gqa_attention_f16.  Returns (fp32 out, binary16 out, k cache, v cache)."""
    torch = torch_mod()
    q, k, v, wq, wk, kc, vc = ops
    ctx = kc.shape[0]
    qd, kd, vd = dev(q), dev(k), dev(v)
    kcd, vcd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    wqp = None if wq is None else dev(wq).data_ptr()
    wkp = None if wk is None else dev(wk).data_ptr()
    ws = torch.empty(max(ws_floats, nq * ctx), dtype=torch.float32, device="cuda")
    o32 = torch.full((nq * hd,), float("nan"), dtype=torch.float32, device="cuda")
    o16 = torch.full((nq * hd,), -1, dtype=torch.int16, device="cuda")
    LIVE.extend([ws, o32, o16])
    if fused:
        F.gqa_attention_qk_f16(o32.data_ptr(), o16.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), wqp, wkp,
                               kcd.data_ptr(), vcd.data_ptr(), hd, nq, nkv, pos, ctx, 1e-6, base, style,
                               ws.data_ptr(), ws_floats, stream())
    else:
        F.qk_norm_rope_store_kv(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), wqp, wkp, kcd.data_ptr(),
                                vcd.data_ptr(), ctx, 1, nq, nkv, hd, 1e-6, None, pos, base, style, stream())
        F.gqa_attention_f16(o32.data_ptr(), o16.data_ptr(), qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), hd, nq,
                            nkv, pos + 1, ctx, ws.data_ptr(), ws_floats, stream())
    return host(o32), host(o16).view(np.uint16), host(kcd).view(np.uint16), host(vcd).view(np.uint16)


@pytest.mark.parametrize("nq,nkv,hd,pos,ctx,norm,style,wsmul", [
    (32, 8, 128, 2915, 4096, True, F.ROPE_NEOX, 4),    # Qwen3-4B decode step, the model's workspace
    (32, 8, 128, 2915, 4096, True, F.ROPE_NEOX, 1),    # the reference's score_buf size
    (32, 8, 128, 0, 4096, True, F.ROPE_NEOX, 4),       # first position: one key, the new one
    (32, 8, 128, 64, 4096, True, F.ROPE_NEOX, 4),      # 65 keys: pos alone at a split's end
    (32, 8, 128, 4095, 4096, True, F.ROPE_NEOX, 4),    # the last cache row
    (32, 8, 128, 700, 4096, False, F.ROPE_NEOX, 4),    # no QK-norm weights: RoPE only
    (32, 8, 128, 333, 512, True, F.ROPE_INTERLEAVED, 1),
    (8, 8, 128, 300, 512, True, F.ROPE_NEOX, 1),       # MHA: one head per workgroup
    (12, 4, 128, 200, 512, True, F.ROPE_NEOX, 1),      # groups of 3: a workgroup with one head
    (16, 4, 64, 100, 512, True, F.ROPE_NEOX, 1),       # head_dim 64: the two calls
    (32, 8, 128, 63, 4096, True, F.ROPE_NEOX, 4),      # 64 keys: one split, one full sub-chunk
    (32, 8, 128, 127, 4096, True, F.ROPE_NEOX, 4),     # 128 keys: two splits of 64
    (32, 8, 128, 1023, 4096, True, F.ROPE_NEOX, 1),    # splits capped by the workspace
    (32, 8, 128, 2047, 4096, False, F.ROPE_INTERLEAVED, 4),
])
def test_attention_qk_equals_head_ops_then_attention(oracle, nq, nkv, hd, pos, ctx, norm, style, wsmul):
    rng = np.random.default_rng(pos + nq + hd + wsmul)
    ops = attention_qk_operands(rng, nq, nkv, hd, ctx, norm)
    ws_floats = wsmul * nq * ctx
    got = run_attention_qk(ops, nq, nkv, hd, pos, 1e6, style, ws_floats, fused=True)
    ref = run_attention_qk(ops, nq, nkv, hd, pos, 1e6, style, ws_floats, fused=False)
    for g, r, what in zip(got, ref, ("fp32 out", "binary16 out", "k cache", "v cache")):
        assert np.array_equal(g.view(np.uint32 if g.dtype == np.float32 else np.uint16),
                              r.view(np.uint32 if r.dtype == np.float32 else np.uint16)), what
    if pos == 2915 and wsmul == 1:  # and the oracle's chain, at the attention bar
        q, k, v, wq, wk, kc, vc = ops
        rq, rk = oracle.qk_norm_rope(q[None], k[None], wq, wk, 1e-6, None, pos, 1e6, style)
        rkc, rvc = oracle.store_kv(kc, vc, rk.reshape(-1), v.reshape(-1), pos)
        ref_o = oracle.gqa_attention(rq.reshape(-1), rkc, rvc, nq, nkv, hd, pos + 1).reshape(nq, hd)
        V = np.abs(rvc[:pos + 1].view(np.float16).astype(np.float64).reshape(-1, nkv, hd))
        gq = got[0].reshape(nq, hd).astype(np.float64)
        for h in range(nq):
            assert np.max(np.abs(gq[h] - ref_o[h])) <= 1e-5 * V[:, h // (nq // nkv), :].max() + 2e-6, f"head {h}"


def test_attention_qk_first_position_nan_cache():
    """Position 0 with a cache full of NaN bits: the one key is the new row,
    written by this launch; no masked slot may carry a NaN into the output.
    Bit for bit the two calls' result, and finite."""
    rng = np.random.default_rng(31)
    nq, nkv, hd, ctx = 32, 8, 128, 4096
    q, k, v, wq, wk, kc, vc = attention_qk_operands(rng, nq, nkv, hd, ctx, True)
    kc[:] = 0x7E00  # binary16 quiet NaN everywhere
    vc[:] = 0x7E00
    ops = (q, k, v, wq, wk, kc, vc)
    got = run_attention_qk(ops, nq, nkv, hd, 0, 1e6, F.ROPE_NEOX, 4 * nq * ctx, fused=True)
    ref = run_attention_qk(ops, nq, nkv, hd, 0, 1e6, F.ROPE_NEOX, 4 * nq * ctx, fused=False)
    assert np.all(np.isfinite(got[0])) and np.all(np.isfinite(ref[0]))
    for g, r, what in zip(got, ref, ("fp32 out", "binary16 out", "k cache", "v cache")):
        assert np.array_equal(g.view(np.uint32 if g.dtype == np.float32 else np.uint16),
                              r.view(np.uint32 if r.dtype == np.float32 else np.uint16)), what


def test_attention_qk_rejects_bad_arguments():
    torch = torch_mod()
    nq, nkv, hd, ctx = 8, 2, 128, 64
    b = torch.zeros(65536, dtype=torch.float32, device="cuda")
    LIVE.append(b)
    p = b.data_ptr()
    L = F.lib()
    args = [None, p, p + 4096, p + 8192, p + 12288, p + 16384, p + 16896, p + 17408, p + 25600, hd, nq, nkv, 5, ctx,
            1e-6, 1e6, F.ROPE_NEOX, p + 33792, 0, stream()]

    def st(**kw):
        a = list(args)
        for key, val in kw.items():
            a[{"out16": 1, "wk": 6, "pos": 12, "style": 16, "ws_floats": 18}[key]] = val
        return L.fence_gqa_attention_qk_f16(*a)

    assert st(out16=None) == F.EINVAL
    assert st(wk=None) == F.EINVAL        # one norm weight only
    assert st(pos=ctx) == F.EINVAL        # past the cache
    assert st(pos=-1) == F.EINVAL
    assert st(style=7) == F.EINVAL
    assert st(ws_floats=-1) == F.EINVAL
    torch.cuda.synchronize()


def test_attention_qk_error_changes_nothing():
    """head_dim 64 takes the two calls; a score_buf too small for the generic
    attention is EINVAL up front: q, k and the caches are left as they were."""
    torch = torch_mod()
    nq, nkv, hd, ctx, pos = 8, 2, 64, 32, 7
    rng = np.random.default_rng(12)
    q, k, v, wq, wk, kc, vc = attention_qk_operands(rng, nq, nkv, hd, ctx, True)
    qd, kd, kcd, vcd = dev(q), dev(k), dev(kc.view(np.int16)), dev(vc.view(np.int16))
    ws = torch.empty(nq * ctx - 1, dtype=torch.float32, device="cuda")
    o16 = torch.empty(nq * hd, dtype=torch.int16, device="cuda")
    LIVE.extend([ws, o16])
    st = F.lib().fence_gqa_attention_qk_f16(None, o16.data_ptr(), qd.data_ptr(), kd.data_ptr(), dev(v).data_ptr(),
                                            dev(wq).data_ptr(), dev(wk).data_ptr(), kcd.data_ptr(), vcd.data_ptr(),
                                            hd, nq, nkv, pos, ctx, 1e-6, 1e6, F.ROPE_NEOX, ws.data_ptr(),
                                            nq * ctx - 1, stream())
    assert st == F.EINVAL
    assert np.array_equal(host(qd).view(np.uint32), q.view(np.uint32))
    assert np.array_equal(host(kd).view(np.uint32), k.view(np.uint32))
    assert np.array_equal(host(kcd).view(np.uint16), kc) and np.array_equal(host(vcd).view(np.uint16), vc)
