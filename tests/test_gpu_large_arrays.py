"""Arrays past one launch's reach: a dispatch's grid size in lanes is 32-bit,
so SwiGLU splits arrays of more than 2^30 float4s into several launches and
RoPE over more heads than one launch's lanes takes its grid-strided kernel.
Each case runs an array a little past that (16 GiB per fp32 operand; the
MI355X holds 288 GB) and checks the elements around the limit and at the end
against a small launch over the same elements, bit for bit (the per-element
arithmetic does not depend on the launch)."""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import stream, torch_mod

pytestmark = pytest.mark.gpu

LANES = 1 << 30          # float4s one launch covers
N = 4 * LANES + 8192 + 13  # two launches and a scalar tail


def windows(n):
    """Element ranges around the launch split and at the end."""
    return [(4 * LANES - 1024, 4 * LANES + 1024), ((n - 2048) // 4 * 4, n)]  # 16-byte aligned starts


def _free_gib(torch):
    torch.cuda.empty_cache()  # blocks the caching allocator still holds from earlier tests
    free, _ = torch.cuda.mem_get_info()
    return free / 2**30


def test_swiglu_past_one_launch():
    torch = torch_mod()
    if _free_gib(torch) < 52:
        pytest.skip("needs 48 GiB of free device memory")
    g = torch.Generator(device="cuda").manual_seed(3)
    gate = torch.randn(N, device="cuda", generator=g)
    up = torch.randn(N, device="cuda", generator=g)
    out = torch.empty(N, device="cuda")
    F.swiglu(out.data_ptr(), gate.data_ptr(), up.data_ptr(), N, stream())
    torch.cuda.synchronize()
    for a, b in windows(N):
        ref = torch.empty(b - a, device="cuda")
        F.swiglu(ref.data_ptr(), gate[a:].data_ptr(), up[a:].data_ptr(), b - a, stream())
        torch.cuda.synchronize()
        got = out[a:b].cpu().numpy().view(np.uint32)
        assert np.array_equal(got, ref.cpu().numpy().view(np.uint32)), f"swiglu elements {a}..{b}"
    del gate, up, out
    torch.cuda.empty_cache()


def test_rope_past_one_launch():
    """RoPE on 10^6 tokens x (32 + 8) heads x 128 (20 GB): the streaming
    kernel's grid would exceed one launch's lanes (its limit is 838,860 such
    tokens), so the launch takes the grid-strided unit kernel.  Tokens in the
    middle and at the end must equal a small launch over them (explicit
    positions; the two kernels' arithmetic is the same)."""
    torch = torch_mod()
    if _free_gib(torch) < 24:
        pytest.skip("needs 21 GiB of free device memory")
    T, nq, nkv, hd = 1_000_000, 32, 8, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn(T, nq * hd, device="cuda", generator=g)
    k = torch.randn(T, nkv * hd, device="cuda", generator=g)
    win = [(T // 2 - 8, T // 2 + 8), (T - 16, T)]
    keep = {ab: (q[ab[0]:ab[1]].clone(), k[ab[0]:ab[1]].clone()) for ab in win}
    F.rope(q.data_ptr(), k.data_ptr(), T, nq, nkv, hd, None, 0, 1e6, F.ROPE_INTERLEAVED, stream())
    torch.cuda.synchronize()
    for (a, b), (q0, k0) in keep.items():
        pos = torch.arange(a, b, dtype=torch.int32, device="cuda")
        F.rope(q0.data_ptr(), k0.data_ptr(), b - a, nq, nkv, hd, pos.data_ptr(), 0, 1e6, F.ROPE_INTERLEAVED,
               stream())
        torch.cuda.synchronize()
        assert np.array_equal(q[a:b].cpu().numpy().view(np.uint32), q0.cpu().numpy().view(np.uint32)), f"q {a}..{b}"
        assert np.array_equal(k[a:b].cpu().numpy().view(np.uint32), k0.cpu().numpy().view(np.uint32)), f"k {a}..{b}"
    del q, k
    torch.cuda.empty_cache()


def test_argmax_near_int_max():
    """argmax over n = 2^31 - 1 floats (8 GiB): a lane's tail index 4 * (n / 4)
    + lane and a grid-strided index + stride pass INT_MAX here, so they must be
    computed in 64 bits.  Maxima at 1 and n - 1 tie; the reference's 256-thread
    rule gives n - 1 (thread 254 = 0b11111110 reverses to 127, below thread
    1's 128).  Every entry point, aligned (float4 path) and one float off
    (scalar path)."""
    torch = torch_mod()
    if _free_gib(torch) < 10:
        pytest.skip("needs 9 GiB of free device memory")
    n = (1 << 31) - 1
    x = torch.full((n + 1,), -1.0, device="cuda")
    r = torch.empty(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(1024, dtype=torch.int64, device="cuda")
    for off in (0, 1):
        x.fill_(-1.0)
        x[off + 1] = 9.0
        x[off + n - 1] = 9.0
        ptr = x.data_ptr() + 4 * off
        for entry in ("one_workgroup", "workspace", "noalloc"):
            r.fill_(-7)
            if entry == "one_workgroup":
                F.argmax(ptr, r.data_ptr(), n, stream())
            elif entry == "workspace":
                F.argmax_ws(ptr, r.data_ptr(), n, ws.data_ptr(), 8 * 1024, stream())
            else:
                F.argmax_noalloc(ptr, r.data_ptr(), n, stream())
            torch.cuda.synchronize()
            assert int(r.item()) == n - 1, f"{entry}, offset {off}"
    del x, r, ws
    torch.cuda.empty_cache()
