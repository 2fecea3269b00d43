"""HIP graph capture: the C-ABI launches recorded into a graph (as a decode
loop would) and replayed several times, with eager work between the replays,
must give the eager results bit for bit on every replay.  The library records
no memset nodes; every launch is a plain kernel node."""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import dev, host, normal
from oracle_py import make_q8_0_table

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(31)
    T, H, nq, nkv, hd, ff, V = 8, 512, 4, 2, 128, 1024, 300
    table = dev(make_q8_0_table(rng, V, H))
    ids = dev(rng.integers(0, V, T).astype(np.int32))
    w = dev(normal(rng, H, 1.0, 0.1))
    wq, wk = dev(normal(rng, hd, 1.0, 0.1)), dev(normal(rng, hd, 1.0, 0.1))
    x0, q0, k0 = normal(rng, (T, H)), normal(rng, (T, nq, hd)), normal(rng, (T, nkv, hd))
    g0, u0, s0 = normal(rng, (T, ff)), normal(rng, (T, ff)), normal(rng, (nq, T, T))
    x, q, k, g, u, s = dev(x0), dev(q0), dev(k0), dev(g0), dev(u0), dev(s0)
    y, emb, act = (torch.empty((T, H), device="cuda"), torch.empty((T, H), device="cuda"),
                   torch.empty((T, ff), device="cuda"))
    originals = [(q, q0), (k, k0), (s, s0)]  # rewritten in place by the sequence

    def sequence(stream):
        F.rms_norm_rows(y.data_ptr(), x.data_ptr(), w.data_ptr(), T, H, 1e-6, stream)
        F.qk_norm_rope(q.data_ptr(), k.data_ptr(), wq.data_ptr(), wk.data_ptr(), T, nq, nkv, hd, 1e-6,
                       None, 5, 1e6, F.ROPE_NEOX, stream)
        F.swiglu(act.data_ptr(), g.data_ptr(), u.data_ptr(), T * ff, stream)
        F.softmax_causal(s.data_ptr(), nq, T, T, stream)
        F.embed_q8_0_gather_rms_norm(emb.data_ptr(), table.data_ptr(), V, ids.data_ptr(), T, H,
                                     w.data_ptr(), 1e-6, stream)

    def reset():
        for t, a in originals:
            t.copy_(torch.from_numpy(a).to("cuda"))
        for t in (y, emb, act):
            t.zero_()

    outs = (y, q, k, act, s, emb)
    sequence(torch.cuda.current_stream().cuda_stream)
    eager = [host(t).copy() for t in outs]

    reset()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sequence(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, t, ref in zip(("rms_rows", "q", "k", "swiglu", "softmax", "gather_rms"), outs, eager):
            got = host(t)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {rep}: {name} differs"
