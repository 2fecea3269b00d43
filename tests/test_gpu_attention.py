"""GPU parity of decode attention (fence_gqa_attention) and the KV store
(fence_store_kv) against the oracle, through the C ABI.

Attention bars (fp32), per query head:
  * max|out - out_oracle| <= 1e-5 * the largest |v| among the head's attended
    V rows -- the output is a convex combination of those rows -- on every
    case;
  * and, at the decode lengths of the configs (2915 and 4096 positions) for
    all three entry points (fence_gqa_attention, _f16, _qk_f16),
    max|out - out_oracle| <= 1e-5 * max|out_oracle| of that head: the output's
    own scale, which is ~80x smaller there (random V averages out).
One attended position must give that V row exactly.  The KV store is exact.
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod

pytestmark = pytest.mark.gpu

TOL = 1e-5


def caches(rng, ctx, n_kv, hd, std=1.0):
    kc = (std * rng.standard_normal((ctx, n_kv * hd))).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, n_kv * hd)).astype(np.float16).view(np.uint16)
    return kc, vc


def run_attention(q, kc, vc, hd, n_q, n_kv, seq, with_ws=True):
    torch = torch_mod()
    ctx = kc.shape[0]
    out = torch.full((n_q * hd,), float("nan"), device="cuda")
    ws = torch.full((n_q * ctx,), float("nan"), device="cuda") if with_ws else None
    LIVE.extend([out, ws])
    F.gqa_attention(out.data_ptr(), dev(q).data_ptr(), dev(kc.view(np.int16)).data_ptr(),
                    dev(vc.view(np.int16)).data_ptr(), hd, n_q, n_kv, seq, ctx,
                    ws.data_ptr() if with_ws else None, stream())
    return host(out)


def assert_attention(got, ref, vc, n_q, n_kv, hd, seq, what):
    got, ref = got.reshape(n_q, hd), ref.reshape(n_q, hd)
    V = np.abs(vc[:max(seq, 1)].view(np.float16).astype(np.float64).reshape(-1, n_kv, hd))
    for h in range(n_q):
        scale = V[:, h // (n_q // n_kv), :].max() if seq > 0 else 1.0
        err = np.max(np.abs(got[h].astype(np.float64) - ref[h]))
        assert err <= TOL * scale, f"{what}: head {h} err {err:.3g} > {TOL:g} * {scale:.3g}"


@pytest.mark.parametrize("seq", [1, 2, 63, 64, 65, 100, 1000, 2915, 4096])
def test_attention_qwen3_4b(oracle, seq):
    n_q, n_kv, hd, ctx = 32, 8, 128, 4096
    rng = np.random.default_rng(seq)
    kc, vc = caches(rng, ctx, n_kv, hd)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    got = run_attention(q, kc, vc, hd, n_q, n_kv, seq)
    ref = oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq)
    assert_attention(got, ref, vc, n_q, n_kv, hd, seq, f"seq {seq}")
    if seq == 1:  # one position: exactly its V row
        v0 = vc[0].view(np.float16).astype(np.float32).reshape(n_kv, hd)
        assert np.array_equal(got.reshape(n_q, hd), v0[np.arange(n_q) // 4])


@pytest.mark.parametrize("n_q,n_kv,seq", [(8, 8, 300), (16, 8, 300), (12, 4, 777), (32, 4, 513),
                                          (8, 1, 2000), (40, 8, 129)])
def test_attention_group_shapes(oracle, n_q, n_kv, seq):
    """MHA, groups of 2, 3 (masked heads), 8 (two head blocks), MQA, 5."""
    hd, ctx = 128, 2048
    rng = np.random.default_rng(n_q * 100 + n_kv)
    kc, vc = caches(rng, ctx, n_kv, hd)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    got = run_attention(q, kc, vc, hd, n_q, n_kv, seq)
    assert_attention(got, oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq), vc, n_q, n_kv, hd, seq,
                     f"{n_q}/{n_kv}")


def test_attention_sharp_scores(oracle):
    """Scores hundreds apart: the running max must rescale correctly."""
    n_q, n_kv, hd, ctx, seq = 32, 8, 128, 1024, 1000
    rng = np.random.default_rng(5)
    kc, vc = caches(rng, ctx, n_kv, hd, std=4.0)
    q = (rng.standard_normal(n_q * hd) * 3.0).astype(np.float32)
    got = run_attention(q, kc, vc, hd, n_q, n_kv, seq)
    assert np.all(np.isfinite(got))
    assert_attention(got, oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq), vc, n_q, n_kv, hd, seq, "sharp")


@pytest.mark.parametrize("hd,ws", [(64, True), (96, True), (128, False)])
def test_attention_other_paths(oracle, hd, ws):
    """head_dim other than 128 (scores in score_buf, the reference's passes);
    no score_buf at head_dim 128 (one split per workgroup)."""
    n_q, n_kv, ctx, seq = 16, 4, 512, 333
    rng = np.random.default_rng(hd)
    kc, vc = caches(rng, ctx, n_kv, hd)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    got = run_attention(q, kc, vc, hd, n_q, n_kv, seq, with_ws=ws)
    assert_attention(got, oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq), vc, n_q, n_kv, hd, seq,
                     f"hd {hd}")


def test_attention_empty_sequence():
    n_q, n_kv, hd, ctx = 8, 2, 128, 16
    rng = np.random.default_rng(0)
    kc, vc = caches(rng, ctx, n_kv, hd)
    got = run_attention(np.ones(n_q * hd, np.float32), kc, vc, hd, n_q, n_kv, 0)
    assert np.array_equal(got, np.zeros(n_q * hd, np.float32))


@pytest.mark.parametrize("pos,kv_dim", [(0, 1024), (7, 1024), (4095, 1024), (3, 1022)])
def test_store_kv_bit_exact(oracle, pos, kv_dim):
    torch = torch_mod()
    ctx = 4096
    rng = np.random.default_rng(pos + kv_dim)
    kc = rng.integers(0, 1 << 15, (ctx, kv_dim), dtype=np.uint16)
    vc = rng.integers(0, 1 << 15, (ctx, kv_dim), dtype=np.uint16)
    k = rng.standard_normal(kv_dim).astype(np.float32)
    v = rng.standard_normal(kv_dim).astype(np.float32)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    F.store_kv(kd.data_ptr(), vd.data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), pos, kv_dim, ctx, stream())
    rk, rv = oracle.store_kv(kc, vc, k, v, pos)
    assert np.array_equal(host(kd).view(np.uint16), rk) and np.array_equal(host(vd).view(np.uint16), rv)


def test_store_then_attend(oracle):
    """A decode step's order (qwen3.cu:303-306): store k, v at pos, attend over pos + 1."""
    torch = torch_mod()
    n_q, n_kv, hd, ctx, pos = 32, 8, 128, 4096, 2915
    rng = np.random.default_rng(9)
    kc, vc = caches(rng, ctx, n_kv, hd)
    k = rng.standard_normal(n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    out = torch.empty(n_q * hd, device="cuda")
    ws = torch.empty(n_q * ctx, device="cuda")
    LIVE.extend([out, ws])
    F.store_kv(kd.data_ptr(), vd.data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), pos, n_kv * hd, ctx, stream())
    F.gqa_attention(out.data_ptr(), dev(q).data_ptr(), kd.data_ptr(), vd.data_ptr(), hd, n_q, n_kv, pos + 1, ctx,
                    ws.data_ptr(), stream())
    rk, rv = oracle.store_kv(kc, vc, k, v, pos)
    assert_attention(host(out), oracle.gqa_attention(q, rk, rv, n_q, n_kv, hd, pos + 1), rv, n_q, n_kv, hd,
                     pos + 1, "store then attend")


def out_scale_ratio(got, ref, n_q, hd):
    """Per head max|got - ref| / max|ref|; the worst head's ratio."""
    g = np.asarray(got, np.float64).reshape(n_q, hd)
    r = np.asarray(ref, np.float64).reshape(n_q, hd)
    return float(np.max(np.max(np.abs(g - r), axis=1) / np.max(np.abs(r), axis=1)))


@pytest.mark.parametrize("variant", ["plain", "f16", "qk_f16"])
@pytest.mark.parametrize("seq", [2915, 4096])
def test_attention_bar_relative_to_output(oracle, variant, seq):
    """The tighter bar, relative to each head's own output scale, for the
    three attention entry points at the configs' decode lengths."""
    torch = torch_mod()
    n_q, n_kv, hd, ctx = 32, 8, 128, 4096
    rng = np.random.default_rng(seq + len(variant))
    kc, vc = caches(rng, ctx, n_kv, hd)
    q = (rng.standard_normal(n_q * hd) * 0.3).astype(np.float32)
    ws = torch.empty(4 * n_q * ctx, device="cuda")
    o32 = torch.full((n_q * hd,), float("nan"), device="cuda")
    o16 = torch.full((n_q * hd,), -1, dtype=torch.int16, device="cuda")
    LIVE.extend([ws, o32, o16])
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    if variant == "plain":
        F.gqa_attention(o32.data_ptr(), dev(q).data_ptr(), kd.data_ptr(), vd.data_ptr(), hd, n_q, n_kv, seq, ctx,
                        ws.data_ptr(), stream())
        ref = oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq)
    elif variant == "f16":
        F.gqa_attention_f16(o32.data_ptr(), o16.data_ptr(), dev(q).data_ptr(), kd.data_ptr(), vd.data_ptr(), hd,
                            n_q, n_kv, seq, ctx, ws.data_ptr(), 4 * n_q * ctx, stream())
        ref = oracle.gqa_attention(q, kc, vc, n_q, n_kv, hd, seq)
    else:  # q/k prologue: QK-norm + NeoX RoPE of q and of the new k at pos = seq - 1, stored, then attended
        pos = seq - 1
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
        wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
        F.gqa_attention_qk_f16(o32.data_ptr(), o16.data_ptr(), dev(q).data_ptr(), dev(k).data_ptr(),
                               dev(v).data_ptr(), dev(wq).data_ptr(), dev(wk).data_ptr(), kd.data_ptr(),
                               vd.data_ptr(), hd, n_q, n_kv, pos, ctx, 1e-6, 1e6, F.ROPE_NEOX, ws.data_ptr(),
                               4 * n_q * ctx, stream())
        rq, rk = oracle.qk_norm_rope(q.reshape(1, n_q, hd), k.reshape(1, n_kv, hd), wq, wk, 1e-6, None, pos, 1e6,
                                     F.ROPE_NEOX)
        rkc, rvc = oracle.store_kv(kc, vc, rk.reshape(-1), v, pos)
        ref = oracle.gqa_attention(rq.reshape(-1), rkc, rvc, n_q, n_kv, hd, seq)
    got = host(o32)
    ratio = out_scale_ratio(got, ref, n_q, hd)
    print(f"attention {variant} seq {seq}: worst head max|err| / max|out| = {ratio:.3g}")
    assert ratio <= TOL, f"{variant} seq {seq}: {ratio:.3g} of the output's scale"
