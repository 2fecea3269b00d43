"""GPU checks of fence_gqa_attention_qk_f16_arrive: one decode token's
attention block (src/model/qwen3.cu:292-310) in one launch, the last
workgroup of each head group merging that group's split partials in place of
the merge kernel.

The bar is bit equality with fence_gqa_attention_qk_f16 on the same operands
(whose own tests tie it to the head kernels, the attention kernels and the
oracle): fp32 and binary16 outputs and both caches.  After every call the
arrival counters must be zero again.  The partials cross from workgroups on
one XCD to the merging workgroup on another through device-coherent stores
and loads; a visibility fault would show as a mismatch, so one case repeats
the call at many random positions and workspace sizes.
"""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod

pytestmark = pytest.mark.gpu


def operands(rng, nq, nkv, hd, ctx, norm):
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    k = rng.standard_normal((nkv, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kc = rng.standard_normal((ctx, nkv * hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, nkv * hd)).astype(np.float16).view(np.uint16)
    return q, k, v, wq, wk, kc, vc


class Setup:
    """Device copies of one operand set, and both forms' outputs."""

    def __init__(self, ops, ws_floats):
        torch = torch_mod()
        q, k, v, wq, wk, kc, vc = ops
        self.nq, self.hd = q.shape
        self.nkv = k.shape[0]
        self.ctx = kc.shape[0]
        self.qd, self.kd, self.vd = dev(q), dev(k), dev(v)
        self.q0, self.k0 = self.qd.clone(), self.kd.clone()  # the two-call path leaves q, k prepared
        LIVE.extend([self.q0, self.k0])
        self.wq = None if wq is None else dev(wq).data_ptr()
        self.wk = None if wk is None else dev(wk).data_ptr()
        self.kcd, self.vcd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
        self.ws_floats = ws_floats
        self.ws = torch.empty(max(ws_floats, self.nq * self.ctx), dtype=torch.float32, device="cuda")
        self.arrive = torch.zeros(self.nq * F.ARRIVE_WORDS_PER_HEAD, dtype=torch.int32, device="cuda")
        self.o32 = torch.empty(self.nq * self.hd, dtype=torch.float32, device="cuda")
        self.o16 = torch.empty(self.nq * self.hd, dtype=torch.int16, device="cuda")
        LIVE.extend([self.ws, self.arrive, self.o32, self.o16])

    def call(self, pos, style, arrive, ws_floats=None):
        """One call; returns (fp32 out, binary16 out) as device copies."""
        self.qd.copy_(self.q0)
        self.kd.copy_(self.k0)
        self.o32.fill_(float("nan"))
        self.o16.fill_(-1)
        wsf = self.ws_floats if ws_floats is None else ws_floats
        a = (self.o32.data_ptr(), self.o16.data_ptr(), self.qd.data_ptr(), self.kd.data_ptr(), self.vd.data_ptr(),
             self.wq, self.wk, self.kcd.data_ptr(), self.vcd.data_ptr(), self.hd, self.nq, self.nkv, pos, self.ctx,
             1e-6, 1e6, style, self.ws.data_ptr(), wsf)
        if arrive:
            F.gqa_attention_qk_f16_arrive(*a, self.arrive.data_ptr(), stream())
        else:
            F.gqa_attention_qk_f16(*a, stream())
        return self.o32.clone(), self.o16.clone()


def bits_equal(a, b):
    x, y = host(a), host(b)
    return np.array_equal(x.view(np.uint32 if x.dtype == np.float32 else np.uint16),
                          y.view(np.uint32 if y.dtype == np.float32 else np.uint16))


@pytest.mark.parametrize("nq,nkv,hd,pos,ctx,norm,style,wsmul", [
    (32, 8, 128, 2915, 4096, True, F.ROPE_NEOX, 4),    # Qwen3-4B decode step, the model's workspace: 46 splits
    (32, 8, 128, 2915, 4096, True, F.ROPE_NEOX, 1),    # the reference's score_buf size
    (32, 8, 128, 4095, 4096, True, F.ROPE_NEOX, 4),    # the last cache row: 64 splits, the most one launch merges
    (32, 8, 128, 0, 4096, True, F.ROPE_NEOX, 4),       # one key: one split, no partials
    (32, 8, 128, 64, 4096, True, F.ROPE_NEOX, 4),      # 65 keys: two splits
    (32, 8, 128, 127, 4096, True, F.ROPE_NEOX, 4),     # 128 keys: two full splits
    (32, 8, 128, 700, 4096, False, F.ROPE_NEOX, 4),    # RoPE only
    (32, 8, 128, 333, 512, True, F.ROPE_INTERLEAVED, 1),
    (32, 8, 128, 1023, 4096, True, F.ROPE_NEOX, 1),    # splits capped by the workspace
    (8, 8, 128, 300, 512, True, F.ROPE_NEOX, 1),       # MHA: one head per workgroup
    (12, 4, 128, 200, 512, True, F.ROPE_NEOX, 1),      # groups of 3: a workgroup with one head
    (16, 4, 128, 2000, 2048, True, F.ROPE_NEOX, 4),    # groups of 4
    (64, 8, 128, 3000, 4096, True, F.ROPE_NEOX, 4),    # groups of 8: four head groups per kv head
    (8, 8, 128, 8000, 8192, True, F.ROPE_NEOX, 4),     # 126 splits: more than one launch merges, two launches
    (16, 4, 64, 100, 512, True, F.ROPE_NEOX, 1),       # head_dim 64: the two calls
])
def test_arrive_equals_two_launch_form(nq, nkv, hd, pos, ctx, norm, style, wsmul):
    rng = np.random.default_rng(pos + 7 * nq + hd + wsmul)
    s = Setup(operands(rng, nq, nkv, hd, ctx, norm), wsmul * nq * ctx)
    ref32, ref16 = s.call(pos, style, arrive=False)
    kc_ref, vc_ref = s.kcd.clone(), s.vcd.clone()
    got32, got16 = s.call(pos, style, arrive=True)
    assert bits_equal(got32, ref32), "fp32 out"
    assert bits_equal(got16, ref16), "binary16 out"
    assert bits_equal(s.kcd, kc_ref) and bits_equal(s.vcd, vc_ref), "caches"
    assert not host(s.arrive).any(), "arrival counters left nonzero"


def test_arrive_repeated_calls_random_positions():
    """200 calls at random positions and workspace sizes on one cache (Qwen3-4B
    heads): every output bit-equal to the two-launch form's, counters zero
    after every call."""
    torch = torch_mod()
    nq, nkv, hd, ctx = 32, 8, 128, 4096
    rng = np.random.default_rng(2024)
    s = Setup(operands(rng, nq, nkv, hd, ctx, True), 4 * nq * ctx)
    bad = []
    for i in range(200):
        pos = int(rng.integers(0, ctx))
        wsf = int(rng.choice([1, 2, 4])) * nq * ctx
        style = F.ROPE_NEOX if i % 3 else F.ROPE_INTERLEAVED
        ref32, ref16 = s.call(pos, style, arrive=False, ws_floats=wsf)
        got32, got16 = s.call(pos, style, arrive=True, ws_floats=wsf)
        same = bool(torch.equal(got32.view(torch.int32), ref32.view(torch.int32))) and \
            bool(torch.equal(got16, ref16)) and not bool(s.arrive.any())
        if not same:
            bad.append((i, pos, wsf, style))
    assert not bad, f"calls differing from the two-launch form (index, pos, ws_floats, style): {bad[:10]}"


def test_arrive_two_streams_at_once():
    """Two operand sets, each with its own counters and score_buf, called on
    two streams with nothing ordering one stream's calls against the other's:
    every output bit-equal to the two-launch form's.  Positions increase, so
    the cache rows a call attends to were written before it in both passes."""
    torch = torch_mod()
    nq, nkv, hd, ctx, n = 32, 8, 128, 4096, 30
    rng = np.random.default_rng(77)
    sets = [Setup(operands(rng, nq, nkv, hd, ctx, True), 4 * nq * ctx) for _ in range(2)]
    pos = [np.sort(rng.choice(ctx, n, replace=False)) for _ in range(2)]
    ref = {(k, i): sets[k].call(int(pos[k][i]), F.ROPE_NEOX, arrive=False) for i in range(n) for k in range(2)}
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = {}
    for i in range(n):
        for k in range(2):
            with torch.cuda.stream(streams[k]):
                got[(k, i)] = sets[k].call(int(pos[k][i]), F.ROPE_NEOX, arrive=True)
    torch.cuda.synchronize()
    bad = [(k, i, int(pos[k][i])) for (k, i) in got
           if not (torch.equal(got[(k, i)][0].view(torch.int32), ref[(k, i)][0].view(torch.int32))
                   and torch.equal(got[(k, i)][1], ref[(k, i)][1]))]
    assert not bad, f"(stream, call, pos) differing from the two-launch form: {bad[:10]}"
    assert not any(bool(s.arrive.any()) for s in sets), "arrival counters left nonzero"


def test_arrive_rejects_missing_counters():
    torch = torch_mod()
    nq, nkv, hd, ctx = 8, 2, 128, 64
    b = torch.zeros(65536, dtype=torch.float32, device="cuda")
    LIVE.append(b)
    p = b.data_ptr()
    args = [None, p, p + 4096, p + 8192, p + 12288, p + 16384, p + 16896, p + 17408, p + 25600, hd, nq, nkv, 5, ctx,
            1e-6, 1e6, F.ROPE_NEOX, p + 33792, 0]
    L = F.lib()
    assert L.fence_gqa_attention_qk_f16_arrive(*args, None, stream()) == F.EINVAL
    assert L.fence_gqa_attention_qk_f16_arrive(*args, p + 2, stream()) == F.EINVAL  # misaligned counters
    torch.cuda.synchronize()
