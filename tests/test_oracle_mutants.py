"""Mutation tests: each plants one plausible mistake in a copy of the oracle
(built on the CPU under pytest's tmp_path) and requires that the pinning
checks of oracle_checks.py catch it.  A mistake no check catches would mean
the oracle is not pinned against it."""
import os
import subprocess

import pytest

import oracle_checks
from oracle_py import Oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "fence_oracle.c")

# (id, exact text in fence_oracle.c, replacement)
MUTANTS = [
    ("rms_divides_by_n_plus_1", "ss / (double)n + (double)eps", "ss / (double)(n + 1) + (double)eps"),
    ("rms_drops_eps", "ss / (double)n + (double)eps", "ss / (double)n"),
    ("rms_adds_weight", "out[i] = (w[i] * x[i]) * r;", "out[i] = (w[i] + x[i]) * r;"),
    ("rope_sign_flip", "x[i1] = x0 * s + x1 * c;", "x[i1] = x0 * s - x1 * c;"),
    ("rope_neox_partner_off_by_one", "? p + half : 2 * p + 1;", "? p + half - 1 : 2 * p + 1;"),
    ("rope_interleaved_as_neox_index", "? p : 2 * p;", "? p : p;"),
    ("rope_freq_exponent_2p_plus_1",
     "const float freq = 1.0f / powf(freq_base, (float)(2 * p) / (float)head_dim);",
     "const float freq = 1.0f / powf(freq_base, (float)(2 * p + 1) / (float)head_dim);"),
    ("inv_freq_table_uses_hd_over_2",
     "inv_freq[p] = 1.0f / powf(freq_base, (float)(2 * p) / (float)head_dim);",
     "inv_freq[p] = 1.0f / powf(freq_base, (float)(2 * p) / (float)(head_dim / 2));"),
    ("swiglu_exp_sign", "g / (1.0f + expf(-g))", "g / (1.0f + expf(g))"),
    ("swiglu_times_gate", "out[i] = silu_g * up[i];", "out[i] = silu_g * gate[i];"),
    ("softmax_no_max_subtraction", "const float e = expf(x[i] - m);", "const float e = expf(x[i]);"),
    ("softmax_drops_last_term", "for (int i = 0; i < n_valid; ++i) {\n        const float e",
     "for (int i = 0; i < n_valid; ++i) {\n        if (i == n_valid - 1 && n_valid > 1) { x[i] = 0.0f; continue; }\n        const float e"),
    ("causal_off_by_one", "int valid = i + 1 + (sk - sq);", "int valid = i + (sk - sq);"),
    ("q8_wrong_quant_offset", "(int8_t)blk[2 + i % FO_QK8_0]", "(int8_t)blk[1 + i % FO_QK8_0]"),
    ("q8_scale_byte_order", "blk[0] | ((uint16_t)blk[1] << 8)", "blk[1] | ((uint16_t)blk[0] << 8)"),
    ("fp16_subnormal_scale", "(float)man * 0x1p-24f", "(float)man * 0x1p-23f"),
    ("fp16_exponent_bias", "((exp + 112u) << 23)", "((exp + 111u) << 23)"),
    ("gemv_drops_scale", "sum += d * block_sum;", "sum += block_sum;"),
    ("gemv_x_offset_off_by_one", "(double)x[b * FO_QK8_0 + i]", "(double)x[b * FO_QK8_0 + i + (i < 31)]"),
    ("f16_ties_away_not_even", "(rem == 0x1000u && (h & 1u))", "(rem == 0x1000u)"),
    ("f16_subnormal_shift", "const uint32_t shift = 126u - exp;", "const uint32_t shift = 127u - exp;"),
    ("residual_overwrites", "x[i] += residual[i];", "x[i] = residual[i];"),
    ("epilogue_f16_of_unnormed", "out16[r * n + i] = fo_f32_to_f16(v);", "out16[r * n + i] = fo_f32_to_f16(h[i]);"),
    ("q6k_ql_offset_wrong_columns", "l + ((col & 1) ? 32 : 0)", "l + ((col >= 2) ? 32 : 0)"),
    ("q6k_qh_shift", "(qh[32 * half + l] >> (2 * col)) & 0x3", "(qh[32 * half + l] >> col) & 0x3"),
    ("q6k_sub_block_32", "(double)scales[i / 16]", "(double)scales[i / 32]"),
    ("q6k_offset_31", "(fo_q6k_quant(blk, i) - 32)", "(fo_q6k_quant(blk, i) - 31)"),
    ("q6k_bias_dropped", "y[r] = bias ? (float)sum + bias[r] : (float)sum;", "y[r] = (float)sum;"),
    ("attn_group_mapping", "const int kvh = h / group;", "const int kvh = h % n_kv_heads;"),
    ("attn_scale_1_over_d", "const float scale = 1.0f / sqrtf((float)head_dim);", "const float scale = 1.0f / (float)head_dim;"),
    ("attn_v_stride", "v_cache[t * kv_dim + (int64_t)kvh * head_dim + d]", "v_cache[t * head_dim + (int64_t)kvh * head_dim + d]"),
    ("store_kv_wrong_row", "k_cache[(int64_t)pos * kv_dim + i] = fo_f32_to_f16(k[i]);", "k_cache[(int64_t)(pos + 1) * kv_dim + i] = fo_f32_to_f16(k[i]);"),
    ("argmax_last_tie", "if (x[i] > local_max) {", "if (x[i] >= local_max) {"),
    ("argmax_tree_upper_slot_wins_ties", "if (sv[u + s] > sv[u]) {", "if (sv[u + s] >= sv[u]) {"),
    ("argmax_1024_threads", "enum { THREADS = 256 };", "enum { THREADS = 1024 };"),
    ("argmax_initial_minus_inf", "float local_max = -1e30f;", "float local_max = -INFINITY;"),
    ("qk_norm_k_uses_q_weight", "fo_rms_norm_per_head(k + t * krow, wk,", "fo_rms_norm_per_head(k + t * krow, wq,"),
]


@pytest.mark.parametrize("mid,old,new", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_mutant_is_caught(tmp_path, mid, old, new):
    src = open(SRC).read()
    assert src.count(old) == 1, f"mutation anchor for {mid} must occur exactly once"
    mpath = tmp_path / "mutant.c"
    mpath.write_text(src.replace(old, new))
    so = tmp_path / f"lib_{mid}.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "oracle"), str(mpath), os.path.join(ROOT, "oracle", "fence_oracle_time.c"),
                    "-o", str(so), "-lm"],
                   check=True)
    results = oracle_checks.run_all(Oracle(str(so)))
    caught = {k: v for k, v in results.items() if v}
    assert caught, f"mutant {mid} passed every oracle check"
