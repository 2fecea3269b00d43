"""The entry points inside a captured HIP graph.  Serving loops capture a decode
step once and replay it; the library neither allocates, synchronises nor
records a memset inside a call, so every entry point can be captured.  Each
case captures a sequence on a side stream, replays the graph several times
with eager work and synchronisations between the replays, and checks every
replay's outputs against the same sequence run eagerly, bit for bit."""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev
from oracle_py import make_q6k_matrix, make_q8_0_table

pytestmark = pytest.mark.gpu


def torch_():
    import torch
    return torch


def bits(t):
    torch = torch_()
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint16 if a.itemsize == 2 else np.uint8)


def check_graph(run, outputs, reset, replays=4):
    """run(stream_handle) issues the sequence; outputs: tensors to compare;
    reset(): restores in-place inputs (eager, outside the graph)."""
    torch = torch_()
    reset()
    run(torch.cuda.current_stream().cuda_stream)
    want = [bits(t).copy() for t in outputs]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    reset()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=side):
        run(side.cuda_stream)
    for r in range(replays):
        for t in outputs:  # clobber the outputs eagerly between replays
            t.view(torch.uint8).fill_(0xA5)
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (t, w) in enumerate(zip(outputs, want)):
            assert np.array_equal(bits(t), w), f"replay {r}: output {i} differs from the eager run"
    del g


def test_prefill_ops_in_a_graph():
    torch = torch_()
    gen = torch.Generator(device="cuda").manual_seed(11)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=gen)  # noqa: E731
    T, nq, nkv, hd, ff, E = 64, 32, 8, 128, 1536, 4096
    x, w = rn(T, E), 1 + 0.1 * rn(E)
    q0, k0 = rn(T, nq * hd), rn(T, nkv * hd)
    wq, wk = 1 + 0.1 * rn(hd), 1 + 0.1 * rn(hd)
    gate, up = rn(T, ff), rn(T, ff)
    s0 = rn(4, 96, 96)
    s0 = s0.masked_fill(torch.ones(96, 96, dtype=torch.bool, device="cuda").triu(1), float("-inf"))
    table = dev(make_q8_0_table(np.random.default_rng(3), 1000, 512))
    ids = torch.randint(0, 1000, (T,), dtype=torch.int32, device="cuda", generator=gen)
    w512 = 1 + 0.1 * rn(512)
    normed, q, k, act, s = (torch.empty_like(x), torch.empty_like(q0), torch.empty_like(k0), torch.empty_like(gate),
                            torch.empty_like(s0))
    gathered = torch.empty(T, 512, device="cuda")
    LIVE.extend([x, w, q0, k0, wq, wk, gate, up, s0, ids, w512, normed, q, k, act, s, gathered])

    def reset():
        q.copy_(q0)
        k.copy_(k0)
        s.copy_(s0)

    def run(sh):
        F.rms_norm_rows(normed.data_ptr(), x.data_ptr(), w.data_ptr(), T, E, 1e-5, sh)
        F.qk_norm_rope(q.data_ptr(), k.data_ptr(), wq.data_ptr(), wk.data_ptr(), T, nq, nkv, hd, 1e-6, None, 0, 1e6,
                       F.ROPE_NEOX, sh)
        F.swiglu(act.data_ptr(), gate.data_ptr(), up.data_ptr(), T * ff, sh)
        F.softmax_causal(s.data_ptr(), 4, 96, 96, sh)
        F.embed_q8_0_gather_rms_norm(gathered.data_ptr(), table.data_ptr(), 1000, ids.data_ptr(), T, 512,
                                     w512.data_ptr(), 1e-6, sh)

    check_graph(run, [normed, q, k, act, s, gathered], reset)


def test_decode_step_in_a_graph():
    """One Qwen3-4B-shaped layer of the fused decode sequence, then the LM
    head and argmax: the form a serving loop captures."""
    torch = torch_()
    rng = np.random.default_rng(12)
    gen = torch.Generator(device="cuda").manual_seed(12)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=gen)  # noqa: E731
    E, nq, nkv, hd, ff, V, ctx, pos = 2560, 32, 8, 128, 9728, 4000, 1024, 700
    QD, KVD = nq * hd, nkv * hd
    Wq, Wk, Wv = (dev(make_q6k_matrix(rng, m, E)) for m in (QD, KVD, KVD))
    Wo = dev(make_q6k_matrix(rng, E, QD))
    Wg, Wu = dev(make_q6k_matrix(rng, ff, E)), dev(make_q6k_matrix(rng, ff, E))
    Wd = dev(make_q6k_matrix(rng, E, ff))
    table = dev(make_q8_0_table(rng, V, E))
    an, fn, qn, kn, on = (1 + 0.1 * rn(n) for n in (E, E, hd, hd, E))
    kc = (rn(ctx, KVD) * 0.5).half()
    vc = rn(ctx, KVD).half()
    kc0, vc0 = kc.clone(), vc.clone()
    hidden, res = rn(E), rn(E)
    h1, h2 = torch.empty(E, device="cuda"), torch.empty(E, device="cuda")
    x16 = torch.empty(E, dtype=torch.int16, device="cuda")
    q, k, v = (torch.empty(n, device="cuda") for n in (QD, KVD, KVD))
    att16 = torch.empty(QD, dtype=torch.int16, device="cuda")
    att16b = torch.empty(QD, dtype=torch.int16, device="cuda")
    arrive = torch.zeros(nq * F.ARRIVE_WORDS_PER_HEAD, dtype=torch.int32, device="cuda")
    o, d = torch.empty(E, device="cuda"), torch.empty(E, device="cuda")
    act16 = torch.empty(ff, dtype=torch.int16, device="cuda")
    normed = torch.empty(E, device="cuda")
    logits = torch.empty(V, device="cuda")
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    tok_na = torch.empty(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(4 * nq * ctx, device="cuda")
    ws2 = torch.empty(4 * nq * ctx, device="cuda")
    LIVE.extend([Wq, Wk, Wv, Wo, Wg, Wu, Wd, table, an, fn, qn, kn, on, kc, vc, kc0, vc0, hidden, res, h1, h2, x16,
                 q, k, v, att16, att16b, arrive, o, d, act16, normed, logits, tok, tok_na, ws, ws2])
    rin_a = F.rms_input(hidden.data_ptr(), res.data_ptr(), h1.data_ptr(), an.data_ptr(), x16.data_ptr(), 1e-6)
    rin_f = F.rms_input(h1.data_ptr(), o.data_ptr(), h2.data_ptr(), fn.data_ptr(), x16.data_ptr(), 1e-6)

    def reset():
        kc.copy_(kc0)
        vc.copy_(vc0)

    def run(sh):
        F.gemv_q6k_multi_rms([Wq.data_ptr(), Wk.data_ptr(), Wv.data_ptr()], [q.data_ptr(), k.data_ptr(), v.data_ptr()],
                             [QD, KVD, KVD], rin_a, E, stream=sh)
        F.gqa_attention_qk_f16(None, att16.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), qn.data_ptr(),
                               kn.data_ptr(), kc.data_ptr(), vc.data_ptr(), hd, nq, nkv, pos, ctx, 1e-6, 1e6,
                               F.ROPE_NEOX, ws.data_ptr(), ws.numel(), sh)
        # the one-launch form (same q, k, v: the launch above leaves them as they were)
        F.gqa_attention_qk_f16_arrive(None, att16b.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                      qn.data_ptr(), kn.data_ptr(), kc.data_ptr(), vc.data_ptr(), hd, nq, nkv, pos,
                                      ctx, 1e-6, 1e6, F.ROPE_NEOX, ws2.data_ptr(), ws2.numel(), arrive.data_ptr(), sh)
        F.gemv_q6k(Wo.data_ptr(), att16.data_ptr(), o.data_ptr(), E, QD, sh)
        F.gemv_q6k_swiglu_rms_f16(Wg.data_ptr(), Wu.data_ptr(), rin_f, act16.data_ptr(), None, ff, E, sh)
        F.gemv_q6k(Wd.data_ptr(), act16.data_ptr(), d.data_ptr(), E, ff, sh)
        F.residual_rms_norm_f16(h2.data_ptr(), d.data_ptr(), on.data_ptr(), normed.data_ptr(), x16.data_ptr(), 1, E,
                                1e-6, sh)
        F.gemv_q8_0(table.data_ptr(), normed.data_ptr(), logits.data_ptr(), V, E, sh)
        F.argmax_ws(logits.data_ptr(), tok.data_ptr(), V, ws.data_ptr(), ws.numel() * 4, sh)
        # the allocation-free form: its first call on the device (possibly this
        # capture) looks up the scratch address; its kernels are captured too
        F.argmax_noalloc(logits.data_ptr(), tok_na.data_ptr(), V, sh)

    # every run recomputes h1, h2 (h2 = h1 + o, then += d) and q/k/v from the unchanged inputs;
    # only the caches' row pos carries over, and reset() restores it
    # (arrive is state, not an output: it must be zero at every call, so it is not clobbered)
    check_graph(run, [q, k, v, att16, att16b, o, act16, d, normed, logits, tok, tok_na, kc, vc, h1, h2], reset)
    assert int(tok_na.item()) == int(tok.item())
    assert np.array_equal(bits(att16b), bits(att16)) and not bits(arrive).any()
