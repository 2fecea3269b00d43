"""numpy-facing wrapper of the CPU oracle (oracle/libfence_oracle.so).

Test infrastructure: only the tests, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py use it, as the checker.  Every function copies
its inputs and returns fresh outputs; in-place reference ops are exposed as
functions returning the updated array.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "libfence_oracle.so")

NEOX = 0
INTERLEAVED = 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

_SIGS = {
    "fo_fp16_to_f32": ((ctypes.c_uint16,), ctypes.c_float),
    "fo_rms_norm": ((_P, _P, _P, _I, _F), None),
    "fo_rms_norm_inplace": ((_P, _P, _I, _F), None),
    "fo_rms_norm_rows": ((_P, _P, _P, _L, _I, _F), None),
    "fo_rms_norm_per_head": ((_P, _P, _I, _I, _F), None),
    "fo_rope_inv_freq": ((_P, _I, _F), None),
    "fo_rope_head": ((_P, _I, _I, _F, _I), None),
    "fo_apply_rope": ((_P, _P, _I, _I, _I, _I, _F), None),
    "fo_rope_rows": ((_P, _P, _L, _I, _I, _I, _P, _I, _F, _I), None),
    "fo_silu_elementwise_mul": ((_P, _P, _P, _L), None),
    "fo_softmax": ((_P, _I), None),
    "fo_softmax_rows": ((_P, _L, _I, _L), None),
    "fo_softmax_causal": ((_P, _L, _I, _I), None),
    "fo_embed_q8_0": ((_P, _P, _I, _I), None),
    "fo_embed_q8_0_gather": ((_P, _P, _L, _P, _L, _I), ctypes.c_int64),
    "fo_embed_q8_0_gather_rms_norm": ((_P, _P, _L, _P, _L, _I, _P, _F), ctypes.c_int64),
    "fo_gemv_q8_0": ((_P, _P, _P, _I, _I), None),
    "fo_f32_to_f16": ((_F,), ctypes.c_uint16),
    "fo_f32_to_f16_array": ((_P, _P, _L), None),
    "fo_residual_add": ((_P, _P, _L), None),
    "fo_residual_rms_norm_f16": ((_P, _P, _P, _P, _P, _L, _I, _F), None),
    "fo_swiglu_f16": ((_P, _P, _P, _P, _L), None),
    "fo_q6k_quant": ((_P, _I), ctypes.c_int),
    "fo_q6k_dot": ((_P, _P), ctypes.c_double),
    "fo_gemv_q6k": ((_P, _P, _P, _P, _I, _I), None),
    "fo_store_kv": ((_P, _P, _P, _P, _I, _I), None),
    "fo_gqa_attention": ((_P, _P, _P, _P, _I, _I, _I, _I, _I), None),
    "fo_argmax": ((_P, _I), ctypes.c_int),
    "fo_qk_norm_rope": ((_P, _P, _P, _P, _L, _I, _I, _I, _F, _P, _I, _F, _I), None),
    "fo_rms_norm_rope": ((_P, _P, _P, _P, _L, _I, _I, _I, _F, _P, _I, _F, _I), None),
    "fo_time_elementwise_stage": ((_P, _I, _P, _L, _I, _I, _P, _P, _P, _L, _P, _P, _L, _I, _I, _I, _P, _F, _I),
                                  None),
}


def _ptr(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32).copy()


class Oracle:
    """One loaded oracle library (the real one, or a mutant in the mutation tests)."""

    def __init__(self, path: str = ORACLE_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is missing: run `make -C oracle`")
        self.path = path
        self.lib = ctypes.CDLL(path)
        for name, (argtypes, restype) in _SIGS.items():
            fn = getattr(self.lib, name)
            fn.argtypes = list(argtypes)
            fn.restype = restype

    # fp16 ------------------------------------------------------------------
    def fp16_to_f32(self, bits: int) -> float:
        return self.lib.fo_fp16_to_f32(bits)

    def fp16_to_f32_all(self) -> np.ndarray:
        """Oracle decode of all 65536 binary16 patterns, as fp32 bit patterns."""
        out = np.empty(65536, dtype=np.float32)
        for b in range(65536):
            out[b] = self.lib.fo_fp16_to_f32(b)
        return out.view(np.uint32)

    # RMSNorm ---------------------------------------------------------------
    def rms_norm(self, x, w, eps):
        x = _f32(x); w = _f32(w); out = np.empty_like(x)
        self.lib.fo_rms_norm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
        return out

    def rms_norm_inplace(self, x, w, eps):
        x = _f32(x); w = _f32(w)
        self.lib.fo_rms_norm_inplace(_ptr(x), _ptr(w), x.size, eps)
        return x

    def rms_norm_rows(self, x, w, eps):
        x = _f32(x); w = _f32(w); out = np.empty_like(x)
        rows, n = x.shape
        self.lib.fo_rms_norm_rows(_ptr(out), _ptr(x), _ptr(w), rows, n, eps)
        return out

    def rms_norm_per_head(self, x, w, eps):
        """x [n_heads, head_dim]"""
        x = _f32(x); w = _f32(w)
        n_heads, hd = x.shape
        self.lib.fo_rms_norm_per_head(_ptr(x), _ptr(w), n_heads, hd, eps)
        return x

    # RoPE ------------------------------------------------------------------
    def rope_inv_freq(self, head_dim, base):
        out = np.empty(head_dim // 2, dtype=np.float32)
        self.lib.fo_rope_inv_freq(_ptr(out), head_dim, base)
        return out

    def rope_head(self, x, pos, base, style):
        x = _f32(x)
        self.lib.fo_rope_head(_ptr(x), x.size, pos, base, style)
        return x

    def apply_rope(self, q, k, pos, base):
        """q [nq, hd], k [nkv, hd]; NeoX, one position."""
        q = _f32(q); k = _f32(k)
        self.lib.fo_apply_rope(_ptr(q), _ptr(k), q.shape[1], q.shape[0], k.shape[0], pos, base)
        return q, k

    def rope_rows(self, q, k, positions, pos0, base, style):
        """q [T, nq, hd], k [T, nkv, hd] or None."""
        q = _f32(q); k = None if k is None else _f32(k)
        T, nq, hd = q.shape
        nkv = 0 if k is None else k.shape[1]
        pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
        self.lib.fo_rope_rows(_ptr(q), _ptr(k), T, nq, nkv, hd, _ptr(pos), pos0, base, style)
        return q, k

    # SwiGLU ----------------------------------------------------------------
    def silu_mul(self, gate, up):
        g = _f32(gate); u = _f32(up); out = np.empty_like(g)
        self.lib.fo_silu_elementwise_mul(_ptr(out), _ptr(g), _ptr(u), g.size)
        return out

    # softmax ---------------------------------------------------------------
    def softmax(self, x):
        x = _f32(x)
        self.lib.fo_softmax(_ptr(x), x.size)
        return x

    def softmax_rows(self, x, n=None):
        """x [rows, ld]; softmax over the first n columns of each row."""
        x = _f32(x)
        rows, ld = x.shape
        self.lib.fo_softmax_rows(_ptr(x), rows, ld if n is None else n, ld)
        return x

    def softmax_causal(self, x):
        """x [heads, sq, sk]"""
        x = _f32(x)
        h, sq, sk = x.shape
        self.lib.fo_softmax_causal(_ptr(x), h, sq, sk)
        return x

    # Q8_0 ------------------------------------------------------------------
    def embed_q8_0(self, table_bytes, token_id, dim):
        t = np.ascontiguousarray(table_bytes, dtype=np.uint8)
        out = np.empty(dim, dtype=np.float32)
        self.lib.fo_embed_q8_0(_ptr(out), _ptr(t), token_id, dim)
        return out

    def embed_q8_0_gather(self, table_bytes, vocab, ids, dim):
        t = np.ascontiguousarray(table_bytes, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((ids.size, dim), dtype=np.float32)
        bad = self.lib.fo_embed_q8_0_gather(_ptr(out), _ptr(t), vocab, _ptr(ids), ids.size, dim)
        return out, bad

    def embed_q8_0_gather_rms_norm(self, table_bytes, vocab, ids, dim, w, eps):
        t = np.ascontiguousarray(table_bytes, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        w = _f32(w)
        out = np.empty((ids.size, dim), dtype=np.float32)
        bad = self.lib.fo_embed_q8_0_gather_rms_norm(_ptr(out), _ptr(t), vocab, _ptr(ids), ids.size,
                                                     dim, _ptr(w), eps)
        return out, bad

    def gemv_q8_0(self, table_bytes, x):
        """y[M] = W[M x K] x[K] for a Q8_0 table [M, K/32*34] bytes."""
        t = np.ascontiguousarray(table_bytes, dtype=np.uint8)
        x = _f32(x)
        M, K = t.shape[0], x.size
        y = np.empty(M, dtype=np.float32)
        self.lib.fo_gemv_q8_0(_ptr(t), _ptr(x), _ptr(y), M, K)
        return y

    # Q6_K -------------------------------------------------------------------
    def q6k_quants(self, blk):
        """The 256 6-bit quants (0..63) of one 210-byte block."""
        b = np.ascontiguousarray(blk, dtype=np.uint8)
        return np.array([self.lib.fo_q6k_quant(_ptr(b), i) for i in range(256)], np.int32)

    def q6k_dot(self, blk, x16):
        b = np.ascontiguousarray(blk, dtype=np.uint8)
        x = np.ascontiguousarray(x16, dtype=np.uint16)
        return float(self.lib.fo_q6k_dot(_ptr(b), _ptr(x)))

    def gemv_q6k(self, W, x16, bias=None):
        """y = W x (+ bias) for W [M, K/256*210] bytes and binary16 x [K]."""
        w = np.ascontiguousarray(W, dtype=np.uint8)
        x = np.ascontiguousarray(x16, dtype=np.uint16)
        M, K = w.shape[0], x.size
        bz = None if bias is None else _f32(bias)
        y = np.empty(M, np.float32)
        self.lib.fo_gemv_q6k(_ptr(w), _ptr(x), _ptr(bz), _ptr(y), M, K)
        return y

    # decode attention ------------------------------------------------------
    def store_kv(self, k_cache, v_cache, k, v, pos):
        """Returns updated copies of the binary16 caches [max_ctx, kv_dim]."""
        kc = np.ascontiguousarray(k_cache, np.uint16).copy()
        vc = np.ascontiguousarray(v_cache, np.uint16).copy()
        k, v = _f32(k), _f32(v)
        self.lib.fo_store_kv(_ptr(kc), _ptr(vc), _ptr(k), _ptr(v), pos, k.size)
        return kc, vc

    def gqa_attention(self, q, k_cache, v_cache, n_q_heads, n_kv_heads, head_dim, seq_len):
        """q [n_q*hd] fp32; caches [max_ctx, n_kv*hd] binary16 bits."""
        q = _f32(q)
        kc = np.ascontiguousarray(k_cache, np.uint16)
        vc = np.ascontiguousarray(v_cache, np.uint16)
        out = np.empty(n_q_heads * head_dim, np.float32)
        self.lib.fo_gqa_attention(_ptr(out), _ptr(q), _ptr(kc), _ptr(vc), head_dim, n_q_heads, n_kv_heads,
                                  seq_len, kc.shape[0])
        return out

    def argmax(self, x):
        x = _f32(x)
        return int(self.lib.fo_argmax(_ptr(x), x.size))

    # f16 and residual epilogue -------------------------------------------
    def f32_to_f16(self, x):
        """binary16 bit patterns (uint16) of float32 values, RNE."""
        x = _f32(x)
        out = np.empty(x.shape, dtype=np.uint16)
        self.lib.fo_f32_to_f16_array(_ptr(out), _ptr(x), x.size)
        return out

    def residual_add(self, x, residual):
        x = _f32(x)
        r = _f32(residual)
        self.lib.fo_residual_add(_ptr(x), _ptr(r), x.size)
        return x

    def residual_rms_norm_f16(self, hidden, residual, w, eps):
        """Returns (hidden after the add, normed fp32, normed as binary16 bits)."""
        h = _f32(hidden)
        n = h.shape[-1]
        rows = h.size // n
        r = None if residual is None else _f32(residual)
        w = _f32(w)
        normed = np.empty(h.shape, np.float32)
        out16 = np.empty(h.shape, np.uint16)
        self.lib.fo_residual_rms_norm_f16(_ptr(h), _ptr(r), _ptr(w), _ptr(normed), _ptr(out16),
                                          rows, n, eps)
        return h, normed, out16

    def swiglu_f16(self, gate, up):
        """Returns (fp32 silu(gate) * up, its binary16 bits)."""
        g = _f32(gate)
        u = _f32(up)
        out = np.empty(g.shape, np.float32)
        out16 = np.empty(g.shape, np.uint16)
        self.lib.fo_swiglu_f16(_ptr(out16), _ptr(out), _ptr(g), _ptr(u), g.size)
        return out, out16

    # fused -----------------------------------------------------------------
    def qk_norm_rope(self, q, k, wq, wk, eps, positions, pos0, base, style):
        q = _f32(q); k = None if k is None else _f32(k)
        wq = _f32(wq); wk = None if wk is None else _f32(wk)
        T, nq, hd = q.shape
        nkv = 0 if k is None else k.shape[1]
        pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
        self.lib.fo_qk_norm_rope(_ptr(q), _ptr(k), _ptr(wq), _ptr(wk), T, nq, nkv, hd, eps,
                                 _ptr(pos), pos0, base, style)
        return q, k

    def rms_norm_rope(self, x, w, k, n_q_heads, head_dim, eps, positions, pos0, base, style):
        """x [T, nq*hd] -> out [T, nq*hd]; k [T, nkv, hd] or None (RoPE only)."""
        x = _f32(x); w = _f32(w); k = None if k is None else _f32(k)
        T = x.shape[0]
        nkv = 0 if k is None else k.shape[1]
        out = np.empty_like(x)
        pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
        self.lib.fo_rms_norm_rope(_ptr(out), _ptr(x), _ptr(w), _ptr(k), T, n_q_heads, nkv, head_dim,
                                  eps, _ptr(pos), pos0, base, style)
        return out, k


# ------------------------------------------------------------ data helpers

def make_q8_0_table(rng: np.random.Generator, vocab: int, dim: int) -> np.ndarray:
    """Synthetic Q8_0 table [vocab, dim/32 * 34] bytes: fp16 scale
    RNE(|N(0,0.02)|/127) then 32 int8 uniform in [-127, 127]."""
    nb = dim // 32
    d = (np.abs(rng.standard_normal((vocab, nb))) * 0.02 / 127.0).astype(np.float16)
    qs = rng.integers(-127, 128, size=(vocab, nb, 32), dtype=np.int8)
    blocks = np.empty((vocab, nb, 34), dtype=np.uint8)
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(vocab, nb, 2)
    blocks[:, :, 2:] = qs.view(np.uint8)
    return blocks.reshape(vocab, nb * 34)


def q8_0_dequant_numpy(table_bytes: np.ndarray, ids, dim: int) -> np.ndarray:
    """Independent dequant via numpy's float16 -> float32 conversion (not the
    oracle's bit routine).  Products of an fp16 and an int8 are exact in fp32."""
    nb = dim // 32
    rows = table_bytes[np.asarray(ids)].reshape(-1, nb, 34)
    d = rows[:, :, 0:2].copy().view(np.float16).astype(np.float32)  # [T, nb, 1]
    q = rows[:, :, 2:].copy().view(np.int8).astype(np.float32)      # [T, nb, 32]
    with np.errstate(invalid="ignore"):  # inf scale * 0 -> NaN, as in fp32
        return (d * q).reshape(-1, dim)


# ---------------------------------------------------------------- Q6_K data

def q6k_dequant_numpy(W: np.ndarray, K: int) -> np.ndarray:
    """Independent Q6_K dequantisation in float64, written as ggml's
    dequantize_row_q6_K loop (per half of 128: ql[l], ql[l+32] low/high
    nibbles and the four crumbs of qh[l] give elements l, l+32, l+64, l+96),
    not as the reference's per-element index arithmetic the oracle follows."""
    blk = np.ascontiguousarray(W, np.uint8).reshape(-1, 210)
    ql, qh = blk[:, 0:128].astype(np.int32), blk[:, 128:192].astype(np.int32)
    sc = blk[:, 192:208].view(np.int8).astype(np.float64)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float64)  # [nblk, 1]
    out = np.empty((blk.shape[0], 256), np.float64)
    for h in range(2):
        a, b, c = ql[:, 64 * h:64 * h + 32], ql[:, 64 * h + 32:64 * h + 64], qh[:, 32 * h:32 * h + 32]
        q = [(a & 0xF) | ((c & 3) << 4), (b & 0xF) | (((c >> 2) & 3) << 4),
             (a >> 4) | (((c >> 4) & 3) << 4), (b >> 4) | (((c >> 6) & 3) << 4)]
        for col in range(4):
            for half16 in range(2):
                s_idx = 8 * h + 2 * col + half16
                l = slice(16 * half16, 16 * half16 + 16)
                out[:, 128 * h + 32 * col + 16 * half16:128 * h + 32 * col + 16 * half16 + 16] = (
                    d * sc[:, s_idx:s_idx + 1] * (q[col][:, l] - 32))
    return out.reshape(np.asarray(W).shape[0], -1)[:, :K] if np.asarray(W).ndim == 2 else out.reshape(-1)


def q6k_pack(q6: np.ndarray, scales: np.ndarray, d16: np.ndarray) -> np.ndarray:
    """Blocks [n, 210] from quants [n, 256] (0..63), int8 scales [n, 16] and
    binary16 d bits [n] -- the inverse of the layout above."""
    q6 = np.asarray(q6, np.int32)
    n = q6.shape[0]
    blk = np.zeros((n, 210), np.uint8)
    for h in range(2):
        cols = [q6[:, 128 * h + 32 * c:128 * h + 32 * c + 32] for c in range(4)]
        blk[:, 64 * h:64 * h + 32] = (cols[0] & 0xF) | ((cols[2] & 0xF) << 4)
        blk[:, 64 * h + 32:64 * h + 64] = (cols[1] & 0xF) | ((cols[3] & 0xF) << 4)
        blk[:, 128 + 32 * h:128 + 32 * h + 32] = ((cols[0] >> 4) | ((cols[1] >> 4) << 2) |
                                                  ((cols[2] >> 4) << 4) | ((cols[3] >> 4) << 6))
    blk[:, 192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[:, 208:210] = np.asarray(d16, np.uint16).reshape(n, 1).view(np.uint8)
    return blk


def make_q6k_matrix(rng: np.random.Generator, M: int, K: int) -> np.ndarray:
    """Synthetic Q6_K rows [M, K/256*210]: quants uniform 0..63, scales uniform
    in [-32, 31], d = binary16(|N(0, 1)| / 4096)."""
    nb = K // 256
    q6 = rng.integers(0, 64, (M * nb, 256))
    sc = rng.integers(-32, 32, (M * nb, 16))
    d = (np.abs(rng.standard_normal(M * nb)) / 4096).astype(np.float16).view(np.uint16)
    return q6k_pack(q6, sc, d).reshape(M, nb * 210)
