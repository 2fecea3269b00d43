"""ctypes binding of libfence_ops.so, the C ABI declared in include/fence/ops.h.

Used by the tests and by bench.py to call the gfx950 kernels with device
pointers (for example ``torch.Tensor.data_ptr()``) and a HIP stream handle.
There is no fallback: if the shared library is missing, loading raises.

Every wrapper raises FenceError on a non-zero status; the raw ctypes
functions stay reachable through ``lib()`` for status-code tests.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# FENCE_OPS_LIB: another build of the same library (a Makefile TAG variant,
# for A/B timing); unset, the package's own.
LIB_PATH = os.environ.get("FENCE_OPS_LIB") or os.path.join(HERE, "libfence_ops.so")

SUCCESS = 0
EINVAL = 22
HIP_BASE = 1000
ROPE_NEOX = 0
ROPE_INTERLEAVED = 1
ARRIVE_WORDS_PER_HEAD = 64  # FENCE_ARRIVE_WORDS_PER_HEAD
QK8_0 = 32
Q8_0_BLOCK_BYTES = 34

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> argument types, in the order of include/fence/ops.h
SIGNATURES = {
    "fence_rms_norm": (_P, _P, _P, _I, _F, _P),
    "fence_rms_norm_inplace": (_P, _P, _I, _F, _P),
    "fence_rms_norm_per_head": (_P, _P, _I, _I, _F, _P),
    "fence_apply_rope": (_P, _P, _I, _I, _I, _I, _F, _P),
    "fence_silu_elementwise_mul": (_P, _P, _P, _I, _P),
    "fence_softmax": (_P, _I, _P),
    "fence_embed_q8_0": (_P, _P, _I, _I, _P),
    "fence_gemv_q8_0": (_P, _P, _P, _I, _I, _P),
    "fence_gemv_q6k": (_P, _P, _P, _I, _I, _P),
    "fence_gemv_q6k_bias": (_P, _P, _P, _P, _I, _I, _P),
    "fence_gqa_attention": (_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P),
    "fence_store_kv": (_P, _P, _P, _P, _I, _I, _I, _P),
    "fence_argmax": (_P, _P, _I, _P),
    "fence_argmax_ws": (_P, _P, _I, _P, _L, _P),
    "fence_argmax_noalloc": (_P, _P, _I, _P),
    "fence_residual_add": (_P, _P, _I, _P),
    "fence_f32_to_f16": (_P, _P, _I, _P),
    "fence_f16_to_f32": (_P, _P, _I, _P),
    "fence_residual_rms_norm_f16": (_P, _P, _P, _P, _P, _L, _I, _F, _P),
    "fence_swiglu_f16": (_P, _P, _P, _P, _L, _P),
    "fence_gemv_q6k_multi": (_I, _P, _P, _P, _P, _P, _I, _P),
    "fence_gemv_q6k_swiglu_f16": (_P, _P, _P, _P, _P, _I, _I, _P),
    "fence_gemv_q6k_multi_rms": (_I, _P, _P, _P, _P, _P, _I, _P),
    "fence_gemv_q6k_swiglu_rms_f16": (_P, _P, _P, _P, _P, _I, _I, _P),
    "fence_rms_norm_rows": (_P, _P, _P, _L, _I, _F, _P),
    "fence_rope": (_P, _P, _L, _I, _I, _I, _P, _I, _F, _I, _P),
    "fence_qk_norm_rope": (_P, _P, _P, _P, _L, _I, _I, _I, _F, _P, _I, _F, _I, _P),
    "fence_gqa_attention_f16": (_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _L, _P),
    "fence_qk_norm_rope_store_kv": (_P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _F, _P, _I, _F, _I, _P),
    "fence_gqa_attention_qk_f16": (_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _I, _P, _L,
                                   _P),
    "fence_gqa_attention_qk_f16_arrive": (_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _I, _P,
                                          _L, _P, _P),
    "fence_rms_norm_rope": (_P, _P, _P, _P, _L, _I, _I, _I, _F, _P, _I, _F, _I, _P),
    "fence_swiglu": (_P, _P, _P, _L, _P),
    "fence_softmax_rows": (_P, _L, _I, _L, _P),
    "fence_softmax_causal": (_P, _L, _I, _I, _P),
    "fence_embed_q8_0_gather": (_P, _P, _L, _P, _L, _I, _P),
    "fence_embed_q8_0_gather_rms_norm": (_P, _P, _L, _P, _L, _I, _P, _F, _P),
    "fence_rope_inv_freq": (_P, _I, _F),
    "fence_time_next_launch": (_P, _P),
    "fence_time_next_launches": (_P, _P, _I),
    "fence_calib_stream": (_P, _P, _P, _L, _I, _I, _P),
    "fence_calib_read": (_P, _P, _L, _I, _I, _P),
    "fence_status_string": (_I,),
    "fence_version": (),
}
_RESTYPES = {"fence_status_string": ctypes.c_char_p, "fence_version": ctypes.c_char_p}

_lib = None


class RmsInput(ctypes.Structure):
    """fence_rms_input: h = hidden + residual, x_f16 = binary16(rms_norm(h))."""
    _fields_ = [("hidden", _P), ("residual", _P), ("hidden_out", _P), ("weight", _P), ("x_f16", _P),
                ("eps", _F)]


class FenceError(RuntimeError):
    def __init__(self, name: str, status: int):
        self.status = status
        super().__init__(f"{name} failed with status {status}: {status_string(status)}")


def lib(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libfence_ops.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        # One HIP runtime per process: PyTorch-ROCm ships its own
        # libamdhip64.so (soname libamdhip64.so.7).  Loading torch first makes
        # this library bind to that copy; loading it first would pull in a
        # second runtime that then finds no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
        handle = ctypes.CDLL(path)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = list(argtypes)
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = handle
    return _lib


def status_string(status: int) -> str:
    return lib().fence_status_string(status).decode()


def version() -> str:
    return lib().fence_version().decode()


def _call(name: str, *args) -> None:
    st = getattr(lib(), name)(*args)
    if st != SUCCESS:
        raise FenceError(name, st)


# ----------------------------------------------------------------- wrappers
# Pointer arguments are integers (device addresses) or None; `stream` is a
# hipStream_t handle as an integer (0 / None = the null stream).

def rms_norm(out, x, w, n, eps, stream=None):
    _call("fence_rms_norm", out, x, w, n, eps, stream)


def rms_norm_inplace(x, w, n, eps, stream=None):
    _call("fence_rms_norm_inplace", x, w, n, eps, stream)


def rms_norm_per_head(x, w, n_heads, head_dim, eps, stream=None):
    _call("fence_rms_norm_per_head", x, w, n_heads, head_dim, eps, stream)


def apply_rope(q, k, head_dim, n_q_heads, n_kv_heads, pos, freq_base, stream=None):
    _call("fence_apply_rope", q, k, head_dim, n_q_heads, n_kv_heads, pos, freq_base, stream)


def silu_elementwise_mul(out, gate, up, n, stream=None):
    _call("fence_silu_elementwise_mul", out, gate, up, n, stream)


def softmax(x, n, stream=None):
    _call("fence_softmax", x, n, stream)


def embed_q8_0(out, weight, token_id, dim, stream=None):
    _call("fence_embed_q8_0", out, weight, token_id, dim, stream)


def gemv_q8_0(W, x, y, M, K, stream=None):
    _call("fence_gemv_q8_0", W, x, y, M, K, stream)


def gemv_q6k(W, x, y, M, K, stream=None):
    _call("fence_gemv_q6k", W, x, y, M, K, stream)


def gemv_q6k_bias(W, x, bias, y, M, K, stream=None):
    _call("fence_gemv_q6k_bias", W, x, bias, y, M, K, stream)


def gqa_attention(attn_out, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads, seq_len, max_ctx,
                  score_buf, stream=None):
    _call("fence_gqa_attention", attn_out, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads,
          seq_len, max_ctx, score_buf, stream)


def store_kv(k_cache, v_cache, k, v, pos, kv_dim, max_ctx, stream=None):
    _call("fence_store_kv", k_cache, v_cache, k, v, pos, kv_dim, max_ctx, stream)


def argmax(x, result, n, stream=None):
    _call("fence_argmax", x, result, n, stream)


def argmax_ws(x, result, n, workspace, workspace_bytes, stream=None):
    _call("fence_argmax_ws", x, result, n, workspace, workspace_bytes, stream)


def argmax_noalloc(x, result, n, stream=None):
    _call("fence_argmax_noalloc", x, result, n, stream)


def residual_add(x, residual, n, stream=None):
    _call("fence_residual_add", x, residual, n, stream)


def f32_to_f16(out, inp, n, stream=None):
    _call("fence_f32_to_f16", out, inp, n, stream)


def f16_to_f32(out, inp, n, stream=None):
    _call("fence_f16_to_f32", out, inp, n, stream)


def residual_rms_norm_f16(hidden, residual, w, normed, out_f16, rows, n, eps, stream=None):
    _call("fence_residual_rms_norm_f16", hidden, residual, w, normed, out_f16, rows, n, eps, stream)


def swiglu_f16(out_f16, out, gate, up, n, stream=None):
    _call("fence_swiglu_f16", out_f16, out, gate, up, n, stream)


def gemv_q6k_multi(Ws, x, ys, Ms, K, biases=None, stream=None):
    """Ws, ys, Ms (and biases, entries may be None): lists of n <= 4 entries."""
    n = len(Ws)
    arr = lambda vals: (ctypes.c_void_p * n)(*vals)  # noqa: E731
    _call("fence_gemv_q6k_multi", n, arr(Ws), arr(ys), None if biases is None else arr(biases),
          (ctypes.c_int * n)(*Ms), x, K, stream)


def gemv_q6k_swiglu_f16(W_gate, W_up, x, out_f16, out, M, K, stream=None):
    _call("fence_gemv_q6k_swiglu_f16", W_gate, W_up, x, out_f16, out, M, K, stream)


def rms_input(hidden, residual, hidden_out, weight, x_f16, eps):
    return RmsInput(hidden, residual, hidden_out, weight, x_f16, eps)


def gemv_q6k_multi_rms(Ws, ys, Ms, rin, K, biases=None, stream=None):
    """As gemv_q6k_multi, with x computed from rin (a RmsInput)."""
    n = len(Ws)
    arr = lambda vals: (ctypes.c_void_p * n)(*vals)  # noqa: E731
    _call("fence_gemv_q6k_multi_rms", n, arr(Ws), arr(ys), None if biases is None else arr(biases),
          (ctypes.c_int * n)(*Ms), ctypes.byref(rin), K, stream)


def gemv_q6k_swiglu_rms_f16(W_gate, W_up, rin, out_f16, out, M, K, stream=None):
    _call("fence_gemv_q6k_swiglu_rms_f16", W_gate, W_up, ctypes.byref(rin), out_f16, out, M, K, stream)


def rms_norm_rows(out, x, w, rows, n, eps, stream=None):
    _call("fence_rms_norm_rows", out, x, w, rows, n, eps, stream)


def rope(q, k, tokens, n_q_heads, n_kv_heads, head_dim, positions, pos0, freq_base, style,
         stream=None):
    _call("fence_rope", q, k, tokens, n_q_heads, n_kv_heads, head_dim, positions, pos0,
          freq_base, style, stream)


def qk_norm_rope(q, k, q_norm_w, k_norm_w, tokens, n_q_heads, n_kv_heads, head_dim, eps,
                 positions, pos0, freq_base, style, stream=None):
    _call("fence_qk_norm_rope", q, k, q_norm_w, k_norm_w, tokens, n_q_heads, n_kv_heads,
          head_dim, eps, positions, pos0, freq_base, style, stream)


def gqa_attention_f16(attn_out, out_f16, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads, seq_len, max_ctx,
                      score_buf, score_buf_floats=0, stream=None):
    _call("fence_gqa_attention_f16", attn_out, out_f16, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads,
          seq_len, max_ctx, score_buf, score_buf_floats, stream)


def qk_norm_rope_store_kv(q, k, v, wq, wk, k_cache, v_cache, max_ctx, tokens, n_q_heads, n_kv_heads, head_dim,
                          eps, positions, pos0, freq_base, style, stream=None):
    _call("fence_qk_norm_rope_store_kv", q, k, v, wq, wk, k_cache, v_cache, max_ctx, tokens, n_q_heads,
          n_kv_heads, head_dim, eps, positions, pos0, freq_base, style, stream)


def gqa_attention_qk_f16(attn_out, out_f16, q, k, v, q_norm_w, k_norm_w, k_cache, v_cache, head_dim, n_q_heads,
                         n_kv_heads, pos, max_ctx, eps, freq_base, style, score_buf, score_buf_floats=0, stream=None):
    _call("fence_gqa_attention_qk_f16", attn_out, out_f16, q, k, v, q_norm_w, k_norm_w, k_cache, v_cache, head_dim,
          n_q_heads, n_kv_heads, pos, max_ctx, eps, freq_base, style, score_buf, score_buf_floats, stream)


def gqa_attention_qk_f16_arrive(attn_out, out_f16, q, k, v, q_norm_w, k_norm_w, k_cache, v_cache, head_dim,
                                n_q_heads, n_kv_heads, pos, max_ctx, eps, freq_base, style, score_buf,
                                score_buf_floats, arrive, stream=None):
    _call("fence_gqa_attention_qk_f16_arrive", attn_out, out_f16, q, k, v, q_norm_w, k_norm_w, k_cache, v_cache,
          head_dim, n_q_heads, n_kv_heads, pos, max_ctx, eps, freq_base, style, score_buf, score_buf_floats, arrive,
          stream)


def rms_norm_rope(out, x, w, k, tokens, n_q_heads, n_kv_heads, head_dim, eps, positions, pos0,
                  freq_base, style, stream=None):
    _call("fence_rms_norm_rope", out, x, w, k, tokens, n_q_heads, n_kv_heads, head_dim, eps,
          positions, pos0, freq_base, style, stream)


def swiglu(out, gate, up, n, stream=None):
    _call("fence_swiglu", out, gate, up, n, stream)


def softmax_rows(x, rows, n, ld, stream=None):
    _call("fence_softmax_rows", x, rows, n, ld, stream)


def softmax_causal(x, heads, sq, sk, stream=None):
    _call("fence_softmax_causal", x, heads, sq, sk, stream)


def embed_q8_0_gather(out, table, vocab, ids, tokens, dim, stream=None):
    _call("fence_embed_q8_0_gather", out, table, vocab, ids, tokens, dim, stream)


def embed_q8_0_gather_rms_norm(out, table, vocab, ids, tokens, dim, w, eps, stream=None):
    _call("fence_embed_q8_0_gather_rms_norm", out, table, vocab, ids, tokens, dim, w, eps, stream)


def time_next_launch(start, stop) -> None:
    """Record hipEvent handles `start`/`stop` around the next kernel this
    thread launches (kernel execution interval only)."""
    _call("fence_time_next_launch", start, stop)


def time_next_launches(start, stop, count) -> None:
    """Hook the next `count` launches: start at the first kernel's start,
    stop at the last one's end."""
    _call("fence_time_next_launches", start, stop, count)


def calib_stream(out, a, b, n, threads=64, vpt=1, stream=None) -> None:
    """Plain stream out = a + b (b given) or out = a (b None) for bandwidth
    calibration; see include/fence/ops.h."""
    _call("fence_calib_stream", out, a, b, n, threads, vpt, stream)


def calib_read(sums, a, n, threads=64, vpt=1, stream=None) -> None:
    """Read-only stream over a[0, n): wave w writes the sum it read to
    sums[w]; see include/fence/ops.h."""
    _call("fence_calib_read", sums, a, n, threads, vpt, stream)


def rope_inv_freq(head_dim: int, freq_base: float):
    """Host-side frequencies the RoPE kernels use, as a list of floats."""
    buf = (ctypes.c_float * (head_dim // 2))()
    _call("fence_rope_inv_freq", ctypes.cast(buf, ctypes.c_void_p), head_dim, freq_base)
    return list(buf)
