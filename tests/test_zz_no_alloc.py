"""The allocation-free argmax, fence_argmax_noalloc: its partials live in the
library's static device scratch instead of a caller workspace.  Through the C
ABI, its index must equal fence_argmax_ws's (the same kernels with a caller
workspace, itself checked against the oracle) and the oracle's, exactly, on
calls in a row -- each later one with a smaller input whose maximum is below
the earlier ones', so a stale partial left in the scratch would win and
show."""
import numpy as np
import pytest

import fence_ops as F
from gpu_util import LIVE, dev, host, stream, torch_mod

pytestmark = pytest.mark.gpu


def noalloc():
    return F.lib().fence_argmax_noalloc


def result_buf():
    torch = torch_mod()
    r = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    LIVE.append(r)
    return r


def call_noalloc(x_dev, n):
    r = result_buf()
    st = noalloc()(x_dev.data_ptr(), r.data_ptr(), n, stream())
    assert st == 0, F.status_string(st)
    return int(host(r)[0])


def call_ws(x_dev, n):
    torch = torch_mod()
    r = result_buf()
    ws = torch.full((1024,), -1, dtype=torch.int64, device="cuda")
    LIVE.append(ws)
    F.argmax_ws(x_dev.data_ptr(), r.data_ptr(), n, ws.data_ptr(), 8192, stream())
    return int(host(r)[0])


def test_noalloc_equals_workspace_form_on_shrinking_calls(oracle):
    rng = np.random.default_rng(2024)
    # sizes shrink call by call: 1024, 149, 10, 2 and 1 partials
    for call, (n, top) in enumerate([(1100000, 100.0), (151936, 50.0), (10000, 20.0), (1027, 10.0), (5, 5.0)]):
        x = rng.integers(-40, 4, n).astype(np.float32)
        x[rng.integers(0, n, 3)] = top        # a three-way tie at this call's maximum
        xd = dev(x)
        want = oracle.argmax(x)
        assert call_ws(xd, n) == want, f"call {call}: workspace form"
        assert call_noalloc(xd, n) == want, f"call {call} (n={n}): allocation-free form"


def test_noalloc_two_calls_second_smaller_unaligned(oracle):
    """Two calls in a row, the second smaller and on the scalar (unaligned) path."""
    rng = np.random.default_rng(7)
    x1 = rng.standard_normal(151936).astype(np.float32)
    x1[140000] = 1e6
    x2 = rng.standard_normal(4097).astype(np.float32)
    x2[[5, 261]] = 3e3                         # one thread's two indices: the first
    d1, d2 = dev(x1), dev(x2)
    assert call_noalloc(d1, x1.size) == call_ws(d1, x1.size) == oracle.argmax(x1) == 140000
    got = call_noalloc(d2, x2.size - 1)         # n = 4096 at an offset of 1 float below
    r = result_buf()
    F.argmax_ws(d2.data_ptr() + 4, r.data_ptr(), x2.size - 1, dev(np.zeros(1024, np.int64)).data_ptr(), 8192,
                stream())
    assert call_noalloc_at(d2, 1, x2.size - 1) == int(host(r)[0]) == oracle.argmax(x2[1:])
    assert got == oracle.argmax(x2[:-1]) == 5


def call_noalloc_at(x_dev, off, n):
    r = result_buf()
    st = noalloc()(x_dev.data_ptr() + 4 * off, r.data_ptr(), n, stream())
    assert st == 0, F.status_string(st)
    return int(host(r)[0])


def test_noalloc_rejects_bad_arguments():
    fn = noalloc()
    assert fn(None, 16, 10, None) == F.EINVAL
    assert fn(16, None, 10, None) == F.EINVAL
    assert fn(16, 32, -1, None) == F.EINVAL
    assert fn(0x1002, 32, 10, None) == F.EINVAL
