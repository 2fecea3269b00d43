"""C-ABI checks that need no GPU: the library loads, exports every function
include/fence/ops.h declares with the argument count the Python binding
uses, rejects invalid arguments with EINVAL before touching the device, and
its host-side RoPE frequencies equal the oracle's bit for bit."""
import ctypes
import os
import re

import numpy as np
import pytest

import fence_ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fence", "ops.h")
EINVAL = fence_ops.EINVAL
BAD = 0x1002  # a non-null address that is not 4-byte aligned; never dereferenced


def header_declarations(path=HEADER):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w\s\*]+?\b(fence_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return decls


def test_header_declares_and_library_exports_everything(fence):
    decls = header_declarations()
    assert len(decls) >= 19
    lib = fence.lib()
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} declared in ops.h but not exported"
        assert name in fence_ops.SIGNATURES, f"{name} missing from the Python binding"
        assert len(fence_ops.SIGNATURES[name]) == nargs, f"{name}: argument count differs"
    assert set(fence_ops.SIGNATURES) == set(decls)


def test_model_headers_declare_and_library_exports_everything(fence):
    """include/fence/gguf.h and model.h against the library and fence_model.py."""
    import fence_model
    decls = {}
    for h in ("gguf.h", "model.h"):
        decls.update(header_declarations(os.path.join(ROOT, "include", "fence", h)))
    assert len(decls) >= 25
    lib = fence_model.lib()
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} declared but not exported"
        assert len(fence_model.SIGNATURES[name][0]) == nargs, f"{name}: argument count differs"
    assert set(fence_model.SIGNATURES) == set(decls)


def test_header_constants_match_the_binding():
    """The #define'd sizes the Python binding restates (fence_ops.py)."""
    text = open(HEADER).read()
    defines = dict(re.findall(r"^#define\s+(FENCE_\w+)\s+(\d+)", text, re.M))
    assert int(defines["FENCE_ARRIVE_WORDS_PER_HEAD"]) == fence_ops.ARRIVE_WORDS_PER_HEAD
    assert int(defines["FENCE_QK8_0"]) == 32 and int(defines["FENCE_Q8_0_BLOCK_BYTES"]) == 34


def test_version_and_status_strings(fence):
    assert "gfx950" in fence.version()
    assert fence.status_string(0) == "success"
    assert "invalid" in fence.status_string(EINVAL)
    for st in (2, 12, 74, 75, 95):  # the loader's and model's statuses
        assert fence.status_string(st) != "unknown status"


def _raw(name):
    return getattr(fence_ops.lib(), name)


@pytest.mark.parametrize("name,args", [
    ("fence_rms_norm", (None, 16, 32, 8, 1e-6, None)),
    ("fence_rms_norm", (16, 16, 32, 0, 1e-6, None)),
    ("fence_rms_norm", (BAD, 16, 32, 8, 1e-6, None)),
    ("fence_rms_norm_inplace", (16, None, 8, 1e-6, None)),
    ("fence_rms_norm_rows", (16, 16, 32, -1, 8, 1e-6, None)),
    ("fence_rms_norm_per_head", (16, None, 4, 128, 1e-6, None)),
    ("fence_rms_norm_per_head", (16, 32, 4, 0, 1e-6, None)),
    ("fence_apply_rope", (16, 32, 127, 4, 2, 5, 1e6, None)),      # odd head_dim
    ("fence_apply_rope", (16, 32, 512, 4, 2, 5, 1e6, None)),      # head_dim > 256
    ("fence_apply_rope", (16, 32, 128, 4, 2, 5, -1.0, None)),     # bad base
    ("fence_apply_rope", (16, None, 128, 4, 2, 5, 1e6, None)),    # k null, n_kv > 0
    ("fence_rope", (16, 32, 4, 4, 2, 128, None, 0, 1e6, 7, None)),  # bad style
    ("fence_qk_norm_rope", (16, 32, None, 48, 4, 4, 2, 128, 1e-6, None, 0, 1e6, 0, None)),
    ("fence_rms_norm_rope", (16, 32, None, 48, 4, 4, 2, 128, 1e-6, None, 0, 1e6, 1, None)),
    ("fence_silu_elementwise_mul", (16, None, 32, 8, None)),
    ("fence_silu_elementwise_mul", (16, 32, 48, -3, None)),
    ("fence_swiglu", (16, 32, BAD, 8, None)),
    ("fence_softmax", (None, 8, None)),
    ("fence_softmax", (16, 0, None)),
    ("fence_softmax_rows", (16, 4, 10, 8, None)),                 # ld < n
    ("fence_softmax_causal", (16, 2, 0, 8, None)),
    ("fence_embed_q8_0", (16, 32, -1, 64, None)),                 # negative id
    ("fence_embed_q8_0", (16, 32, 3, 48, None)),                  # dim % 32 != 0
    ("fence_embed_q8_0_gather", (16, 32, 100, None, 4, 64, None)),
    ("fence_embed_q8_0_gather", (16, 32, 0, 48, 4, 64, None)),    # vocab 0
    ("fence_embed_q8_0_gather_rms_norm", (16, 32, 100, 48, 4, 64, None, 1e-6, None)),
    ("fence_gemv_q8_0", (16, 32, 48, 8, 48, None)),               # K % 32 != 0
    ("fence_gemv_q8_0", (0x1001, 32, 48, 8, 64, None)),           # W not 2-byte aligned
    ("fence_gemv_q8_0", (16, 32, None, 8, 64, None)),
    ("fence_gemv_q8_0", (16, 32, 48, -1, 64, None)),
    ("fence_gemv_q6k", (16, 32, 48, 8, 300, None)),               # K % 256 != 0
    ("fence_gemv_q6k", (0x1001, 32, 48, 8, 256, None)),           # W not 2-byte aligned
    ("fence_gemv_q6k", (16, 32, 48, 8, 0, None)),                 # K == 0
    ("fence_gemv_q6k_bias", (16, 32, None, 48, 8, 256, None)),    # bias missing
    ("fence_gqa_attention_f16", (16, None, 32, 48, 64, 128, 8, 2, 10, 100, 80, 0, None)),  # out_f16 missing
    ("fence_gqa_attention_f16", (None, 0x1001, 32, 48, 64, 128, 8, 2, 10, 100, 80, 0, None)),  # misaligned
    ("fence_gqa_attention_f16", (None, 96, 32, 48, 64, 128, 8, 2, 10, 100, 80, -1, None)),  # negative size
    ("fence_gqa_attention_f16", (None, 96, 32, 48, 64, 96, 8, 2, 10, 100, 80, 100, None)),  # generic: too small
    ("fence_qk_norm_rope_store_kv", (16, 32, 48, 64, 80, None, 96, 100, 1, 4, 2, 128, 1e-6, None, 0, 1e6, 0,
                                     None)),                        # k_cache missing
    ("fence_qk_norm_rope_store_kv", (16, 32, 48, 64, None, 96, 112, 100, 1, 4, 2, 128, 1e-6, None, 0, 1e6, 0,
                                     None)),                        # one norm weight only
    ("fence_qk_norm_rope_store_kv", (16, 32, None, 64, 80, 96, 112, 100, 1, 4, 2, 128, 1e-6, None, 0, 1e6, 0,
                                     None)),                        # v missing
    ("fence_qk_norm_rope_store_kv", (16, 32, 48, 64, 80, 96, 112, 100, 1, 4, 2, 128, 1e-6, None, 100, 1e6, 0,
                                     None)),                        # position past max_ctx
    ("fence_qk_norm_rope_store_kv", (16, 32, 48, 64, 80, 96, 112, 100, 1, 4, 2, 128, 1e-6, None, 0, 1e6, 5,
                                     None)),                        # bad style
    ("fence_gemv_q6k_multi", (0, 16, 32, None, 48, 64, 256, None)),   # no matrices
    ("fence_gemv_q6k_multi", (5, 16, 32, None, 48, 64, 256, None)),   # more than four
    ("fence_gemv_q6k_multi", (2, None, 32, None, 48, 64, 256, None)),  # W array missing
    ("fence_gemv_q6k_swiglu_f16", (16, 32, 48, 64, None, 8, 300, None)),  # K % 256 != 0
    ("fence_gemv_q6k_swiglu_f16", (16, 32, 48, 64, None, -1, 256, None)),
    ("fence_gemv_q6k_swiglu_f16", (16, 32, 48, None, None, 8, 256, None)),  # out_f16 missing
    ("fence_gemv_q6k_swiglu_f16", (16, 0x1001, 48, 64, None, 8, 256, None)),  # W_up misaligned
    ("fence_gqa_attention_qk_f16_arrive", (None, 16, 32, 48, 64, 80, 96, 112, 128, 128, 8, 2, 5, 100, 1e-6, 1e6,
                                           0, 144, 0, None, None)),   # no arrival counters
    ("fence_gqa_attention_qk_f16_arrive", (None, 16, 32, 48, 64, 80, 96, 112, 128, 128, 8, 2, 5, 100, 1e-6, 1e6,
                                           0, 144, 0, 0x1002, None)),  # counters misaligned
    ("fence_gqa_attention_qk_f16_arrive", (None, 16, 32, 48, 64, 80, 96, 112, 128, 128, 8, 2, 100, 100, 1e-6, 1e6,
                                           0, 144, 0, 160, None)),     # pos == max_ctx
    ("fence_gqa_attention", (16, 32, 48, 64, 128, 6, 4, 10, 100, 80, None)),   # 6 % 4 != 0
    ("fence_gqa_attention", (16, 32, 48, 64, 128, 8, 2, 101, 100, 80, None)),  # seq_len > max_ctx
    ("fence_store_kv", (16, 32, 48, 64, 100, 512, 100, None)),                # pos == max_ctx
    ("fence_store_kv", (16, 32, 48, 64, -1, 512, 100, None)),
    ("fence_argmax", (16, None, 10, None)),
    ("fence_argmax", (BAD, 32, 10, None)),
    ("fence_argmax", (16, 32, -1, None)),
    ("fence_argmax_ws", (16, 32, 10, None, 64, None)),           # no workspace
    ("fence_argmax_ws", (16, 32, 10, 48, 7, None)),              # under one partial
    ("fence_argmax_ws", (16, 32, 10, 0x1004, 64, None)),         # workspace not 8-byte aligned
    ("fence_argmax_ws", (16, None, 10, 48, 64, None)),
    ("fence_argmax_noalloc", (None, 32, 10, None)),
    ("fence_argmax_noalloc", (16, 32, -1, None)),
    ("fence_residual_add", (16, None, 8, None)),
    ("fence_residual_add", (BAD, 32, 8, None)),
    ("fence_f32_to_f16", (0x1001, 32, 8, None)),                  # binary16 output not 2-byte aligned
    ("fence_f16_to_f32", (16, 32, -1, None)),
    ("fence_residual_rms_norm_f16", (16, 32, 48, None, None, 2, 64, 1e-6, None)),  # no output
    ("fence_residual_rms_norm_f16", (16, 32, 48, 16, None, 2, 64, 1e-6, None)),    # normed == hidden
    ("fence_residual_rms_norm_f16", (16, 32, 48, 64, 80, 2, 0, 1e-6, None)),
    ("fence_swiglu_f16", (None, 16, 32, 48, 8, None)),
    ("fence_swiglu_f16", (0x1001, None, 32, 48, 8, None)),
    ("fence_calib_stream", (16, 32, 48, 6, 64, 1, None)),          # n % 4 != 0
    ("fence_calib_stream", (16, 0x1008, 48, 8, 64, 1, None)),      # a not 16-byte aligned
    ("fence_calib_stream", (16, 32, 48, 8, 128, 1, None)),         # threads not 64 or 256
    ("fence_calib_stream", (16, 32, None, 8, 64, 3, None)),        # vpt not 1, 2 or 4
    ("fence_calib_stream", (16, 32, None, 8 << 30, 64, 1, None)),  # past one launch
    ("fence_calib_stream", (16, None, 48, 8, 64, 1, None)),        # b without a
    ("fence_calib_read", (None, 32, 8, 64, 1, None)),               # no sums
    ("fence_calib_read", (16, None, 8, 64, 1, None)),               # no input
    ("fence_calib_read", (16, 32, 6, 64, 1, None)),                 # n % 4 != 0
    ("fence_calib_read", (16, 0x1008, 8, 64, 1, None)),             # a not 16-byte aligned
    ("fence_calib_read", (16, 32, 8, 128, 1, None)),                # threads not 64 or 256
    ("fence_calib_read", (16, 32, 8, 64, 3, None)),                 # vpt not 1, 2 or 4
    ("fence_calib_read", (16, 32, 8 << 30, 64, 1, None)),           # past one launch
])
def test_invalid_arguments_rejected_on_host(fence, name, args):
    assert _raw(name)(*args) == EINVAL


def test_rms_input_entry_points_reject_on_host(fence):
    """fence_gemv_q6k_multi_rms / fence_gemv_q6k_swiglu_rms_f16: a missing,
    misaligned or overlapping operand of the input row is EINVAL before any
    device work (the addresses are never dereferenced)."""
    L = fence_ops.lib()
    K = 512
    hid, res, hout, w, x16 = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    W = (ctypes.c_void_p * 1)(0x60000)
    y = (ctypes.c_void_p * 1)(0x70000)
    M = (ctypes.c_int * 1)(8)

    def multi(rin, k=K):
        return L.fence_gemv_q6k_multi_rms(1, W, y, None, M, None if rin is None else ctypes.byref(rin), k, None)

    def pair(rin, k=K):
        return L.fence_gemv_q6k_swiglu_rms_f16(0x60000, 0x68000, None if rin is None else ctypes.byref(rin),
                                               0x78000, None, 8, k, None)

    R = fence_ops.rms_input
    for call in (multi, pair):
        assert call(None) == EINVAL
        assert call(R(hid, res, hid, w, x16, 1e-6)) == EINVAL          # the sum in place
        assert call(R(hid, res, res + 8, w, x16, 1e-6)) == EINVAL      # overlaps residual
        assert call(R(hid, res, None, w, x16, 1e-6)) == EINVAL         # residual without hidden_out
        assert call(R(hid, res, hout, w, None, 1e-6)) == EINVAL        # no x
        assert call(R(hid, res, hout, None, x16, 1e-6)) == EINVAL      # no weight
        assert call(R(None, res, hout, w, x16, 1e-6)) == EINVAL        # no hidden
        assert call(R(hid, res, hout, w, hid + 100, 1e-6)) == EINVAL   # x inside hidden
        assert call(R(hid, res, hout, w, x16 + 1, 1e-6)) == EINVAL     # x not 2-byte aligned
        assert call(R(hid + 2, res, hout, w, x16, 1e-6)) == EINVAL     # hidden not 4-byte aligned
        assert call(R(hid, res, hout, w, x16, 1e-6), k=0) == EINVAL
        assert call(R(hid, res, hout, w, x16, 1e-6), k=300) == EINVAL


def test_zero_sized_calls_are_no_ops(fence):
    assert _raw("fence_rms_norm_rows")(16, 16, 32, 0, 8, 1e-6, None) == 0
    assert _raw("fence_swiglu")(16, 32, 48, 0, None) == 0
    assert _raw("fence_rope")(16, 32, 0, 4, 2, 128, None, 0, 1e6, 0, None) == 0
    assert _raw("fence_softmax_causal")(16, 0, 4, 4, None) == 0
    assert _raw("fence_embed_q8_0_gather")(16, 32, 10, 48, 0, 64, None) == 0
    assert _raw("fence_gemv_q8_0")(16, 32, 48, 0, 64, None) == 0
    assert _raw("fence_residual_add")(16, 32, 0, None) == 0
    assert _raw("fence_gemv_q6k")(16, 32, 48, 0, 256, None) == 0
    assert _raw("fence_f32_to_f16")(16, 32, 0, None) == 0
    assert _raw("fence_residual_rms_norm_f16")(16, 32, 48, None, 64, 0, 64, 1e-6, None) == 0
    assert _raw("fence_swiglu_f16")(16, None, 32, 48, 0, None) == 0


@pytest.mark.parametrize("base,hd", [(1e6, 128), (5e5, 128), (5e6, 128), (1e4, 64), (1e6, 256)])
def test_host_inv_freq_bit_exact(oracle, fence, base, hd):
    got = np.array(fence.rope_inv_freq(hd, base), dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), oracle.rope_inv_freq(hd, base).view(np.uint32))
    fx = np.load(os.path.join(ROOT, "tests", "golden", "inv_freq.npz"))[f"b{base:g}_hd{hd}"]
    assert np.array_equal(got.view(np.uint32), fx.view(np.uint32))


def test_inv_freq_rejects_bad_head_dim(fence):
    buf = (ctypes.c_float * 256)()
    assert _raw("fence_rope_inv_freq")(ctypes.cast(buf, ctypes.c_void_p), 127, 1e6) == EINVAL
    assert _raw("fence_rope_inv_freq")(None, 128, 1e6) == EINVAL


def test_wave_clock_only_in_the_instrumented_library(fence):
    """include/fence/wave_clock.h's entry points exist in
    libfence_ops_waveclock.so (gemv_q6k.hip built with FENCE_WAVE_CLOCK=1) and
    not in the product library, whose kernels carry no instrumentation."""
    decls = header_declarations(os.path.join(ROOT, "include", "fence", "wave_clock.h"))
    assert decls == {"fence_wave_clock_clear": 0, "fence_wave_clock_read": 2}
    wc = ctypes.CDLL(os.path.join(os.path.dirname(fence_ops.LIB_PATH), "libfence_ops_waveclock.so"))
    for name in decls:
        assert hasattr(wc, name), f"{name} missing from the instrumented library"
        assert not hasattr(fence.lib(), name), f"{name} exported by the product library"
    for name in header_declarations():  # the same C ABI otherwise
        assert hasattr(wc, name), name
