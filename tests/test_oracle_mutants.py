"""The pinning tests fail on plausible slips: each case compiles a copy of
oracle/cx_oracle.c with one deliberate mistake (a flipped rotation, a
dropped attention scale, swapped Box-Muller outputs, a permuted Q6_K group,
a misplaced quantizer bit, a k-quant search with other weights, error or
steps, a forward with a swapped norm, a dropped bias, SiLU on `up`, a
misplaced residual or no final norm), loads it in a child pytest through
CX_ORACLE_LIB, and requires the named tests of test_oracle_pins.py or
test_oracle_forward_pins.py to fail. The mistakes live only in temporary
copies on the CPU."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "cx_oracle.c")
PINS = ["tests/test_oracle_pins.py", "tests/test_oracle_forward_pins.py"]

MUTANTS = {
    "rope_turns_backwards": (
        ["lo[i] = x0 * ct[i] - x1 * st[i];", "lo[i] = x0 * ct[i] + x1 * st[i];",
         "hi[i] = x0 * st[i] + x1 * ct[i];", "hi[i] = x1 * ct[i] - x0 * st[i];"],
        ["test_rope_one_hot_rotation_direction", "test_rope_matches_the_float64_rotation"]),
    "rope_interleaved_pairs": (
        ["float *lo = x + t * width + h * hd, *hi = lo + half;",
         "float *lo = x + t * width + h * hd, *hi = lo + 1;"],
        ["test_rope_one_hot_rotation_direction"]),
    "attention_unscaled": (
        ["tokens;\n  float scale = 1.0f / sqrtf((float)hd);", "tokens;\n  float scale = 1.0f;"],
        ["test_attention_matches_scaled_softmax_closed_form"]),
    "attention_scaled_by_dim": (
        ["tokens;\n  float scale = 1.0f / sqrtf((float)hd);", "tokens;\n  float scale = 1.0f / (float)hd;"],
        ["test_attention_matches_scaled_softmax_closed_form"]),
    "box_muller_swapped": (
        ["*z0 = r * cosf(ang);\n  *z1 = r * sinf(ang);", "*z0 = r * sinf(ang);\n  *z1 = r * cosf(ang);"],
        ["test_normals_are_box_muller_on_the_exact_uniforms"]),
    "box_muller_log_of_u2": (
        ["sqrtf(-2.0f * logf(u1))", "sqrtf(-2.0f * logf(u2))"],
        ["test_normals_are_box_muller_on_the_exact_uniforms"]),
    "seed_row_before_name": (
        ["h ^= row;\n  h *= 0x00000100000001B3ull;", "h *= 0x00000100000001B3ull;\n  h ^= row;"],
        ["test_seed_of_is_fnv1a_then_row_then_model"]),
    "q6k_dequant_groups_1_2_swapped": (
        ["y[base + 32 + l] = d * (float)(int8_t)sc[is + 2] * (float)q2;\n"
         "          y[base + 64 + l] = d * (float)(int8_t)sc[is + 4] * (float)q3;",
         "y[base + 32 + l] = d * (float)(int8_t)sc[is + 2] * (float)q3;\n"
         "          y[base + 64 + l] = d * (float)(int8_t)sc[is + 4] * (float)q2;"],
        ["test_q6k_one_hot_bytes_dequantize_and_unpack_per_the_table"]),
    "q6k_unpack_high_bits_shifted": (
        ["q[base + 96 + l] = (int8_t)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;",
         "q[base + 96 + l] = (int8_t)((ql[l + 32] >> 4) | (((h >> 4) & 3) << 4)) - 32;"],
        ["test_q6k_one_hot_bytes_dequantize_and_unpack_per_the_table"]),
    "q6k_dot_ql_by_group_half": (
        ["const uint8_t *ql = o + 64 * half + 32 * (gi % 2);",
         "const uint8_t *ql = o + 64 * half + 32 * (gi / 2);"],
        ["test_q6k_one_hot_bytes_row_dot_per_the_table"]),
    "q4k_q5k_min_top_bits_in_scale_byte": (
        ["packed[j] |= (uint8_t)((lm >> 4) << 6);", "packed[j - 4] |= (uint8_t)((lm >> 4) << 4);"],
        ["test_q4k_q5k_quantizer_bytes_on_an_exact_grid"]),
    "q5k_high_bits_pair_order": (
        ["qh[i] |= (uint8_t)((l[2 * p][i] >> 4) << (2 * p));",
         "qh[i] |= (uint8_t)((l[2 * p][i] >> 4) << (2 * p + 1));"],
        ["test_q4k_q5k_quantizer_bytes_on_an_exact_grid"]),
    "q4k_search_from_minus_half": (
        ["SEARCH_Q4K = {15, -1.0f, 0.1f, 20, 0};", "SEARCH_Q4K = {15, -0.5f, 0.1f, 20, 0};"],
        ["test_q4k_search_starts_one_level_below_nmax"]),
    "q3k_hmask_bit_order": (
        ["hmask[place] |= (uint8_t)(1 << (half * 4 + round));",
         "hmask[place] |= (uint8_t)(1 << (round * 2 + half));"],
        ["test_q3k_quantizer_bytes_on_an_exact_grid"]),
    "q3k_scale_sign": (
        ["float iscale = -32.0f / big;", "float iscale = 32.0f / big;"],
        ["test_q3k_quantizer_bytes_on_an_exact_grid"]),
    "q2k_min_nibble_low": (
        ["pack[j] = (uint8_t)(le | (lm << 4));", "pack[j] = (uint8_t)(lm | (le << 4));"],
        ["test_q2k_quantizer_bytes_on_an_exact_grid"]),
    # the search on non-grid blocks: its weights, error and steps
    "q4k_q5k_weights_without_the_block_rms": (
        ["for (int i = 0; i < 32; i++) w[i] = mean + fabsf(sub[i]);",
         "for (int i = 0; i < 32; i++) w[i] = fabsf(sub[i]);"],
        ["test_kquant_search_on_random_blocks[Q4_K]", "test_kquant_search_on_random_blocks[Q5_K]"]),
    "q4k_q5k_constant_weights": (
        ["for (int i = 0; i < 32; i++) w[i] = mean + fabsf(sub[i]);",
         "for (int i = 0; i < 32; i++) w[i] = 1.0f + 0.0f * mean;"],
        ["test_kquant_search_on_random_blocks[Q4_K]", "test_kquant_search_on_random_blocks[Q5_K]"]),
    "q2k_weights_with_a_constant": (
        ["for (int i = 0; i < 16; i++) w[i] = fabsf(sub[i]);",
         "for (int i = 0; i < 16; i++) w[i] = 0.01f + fabsf(sub[i]);"],
        ["test_kquant_search_on_random_blocks[Q2_K]"]),
    "q2k_squared_error": (
        ["const search_t s = {3, -0.5f, 0.1f, 15, 1};", "const search_t s = {3, -0.5f, 0.1f, 15, 0};"],
        ["test_kquant_search_on_random_blocks[Q2_K]"]),
    "q4k_one_step_short": (
        ["SEARCH_Q4K = {15, -1.0f, 0.1f, 20, 0};", "SEARCH_Q4K = {15, -1.0f, 0.1f, 19, 0};"],
        ["test_kquant_search_on_random_blocks[Q4_K]"]),
    "q5k_steps_of_q4k": (
        ["SEARCH_Q5K = {31, -0.5f, 0.1f, 15, 0};", "SEARCH_Q5K = {31, -1.0f, 0.1f, 20, 0};"],
        ["test_kquant_search_on_random_blocks[Q5_K]"]),
    "qkx_candidates_from_the_first_min": (
        ["iscale = (b->from + b->step * (float)k + (float)b->nmax) / (mx - mn);\n"
         "    float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;\n"
         "    for (int i = 0; i < n; i++) {\n"
         "      aux[i] = clampi(entero(iscale * (x[i] - mn)), 0, b->nmax);",
         "iscale = (b->from + b->step * (float)k + (float)b->nmax) / (mx - mn0);\n"
         "    float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;\n"
         "    for (int i = 0; i < n; i++) {\n"
         "      aux[i] = clampi(entero(iscale * (x[i] - mn0)), 0, b->nmax);",
         "  float iscale = (float)b->nmax / (mx - mn);",
         "  const float mn0 = mn;\n  float iscale = (float)b->nmax / (mx - mn);"],
        ["test_kquant_search_on_random_blocks[Q4_K]"]),
    # the forward's composition (src/forward.rs:375-505)
    "forward_output_norm_skipped": (
        ["orc_rmsnorm(xn, x + (t - 1) * D, M->out_norm, D, g->eps);",
         "memcpy(xn, x + (t - 1) * D, D * 4);"],
        ["test_identity_layers_leave_the_output_norm_and_head"]),
    "forward_output_norm_of_the_last_layer": (
        ["orc_rmsnorm(xn, x + (t - 1) * D, M->out_norm, D, g->eps);",
         "orc_rmsnorm(xn, x + (t - 1) * D, M->layers[g->layers - 1].ffn_norm, D, g->eps);"],
        ["test_identity_layers_leave_the_output_norm_and_head"]),
    "forward_logits_of_the_first_token": (
        ["orc_rmsnorm(xn, x + (t - 1) * D, M->out_norm, D, g->eps);",
         "orc_rmsnorm(xn, x, M->out_norm, D, g->eps);"],
        ["test_identity_layers_leave_the_output_norm_and_head"]),
    "forward_residual_before_the_o_proj": (
        ["L->o, L->t_o, NULL, pr)) goto done;\n    for (size_t i = 0; i < tr * D; i++) xr[i] += pr[i];",
         "L->o, L->t_o, NULL, pr)) goto done;\n    for (size_t i = 0; i < tr * D; i++) xr[i] += att[i];"],
        ["test_identity_layers_leave_the_output_norm_and_head"]),
    "forward_down_residual_dropped": (
        ["L->down, L->t_down, NULL, pr)) goto done;\n    for (size_t i = 0; i < tr * D; i++) xr[i] += pr[i];",
         "L->down, L->t_down, NULL, pr)) goto done;\n    for (size_t i = 0; i < tr * D; i++) xr[i] += 0.0f * pr[i];"],
        ["test_swiglu_block_closed_form"]),
    "forward_ffn_normed_by_attn_norm": (
        ["orc_rmsnorm(xnr + r * D, xr + r * D, L->ffn_norm, D, g->eps);",
         "orc_rmsnorm(xnr + r * D, xr + r * D, L->attn_norm, D, g->eps);"],
        ["test_swiglu_block_closed_form"]),
    "forward_attention_normed_by_ffn_norm": (
        ["orc_rmsnorm(xn + r * D, x + r * D, L->attn_norm, D, g->eps);",
         "orc_rmsnorm(xn + r * D, x + r * D, L->ffn_norm, D, g->eps);"],
        ["test_scores_from_rotated_biases"]),
    "forward_silu_on_up": (
        ["orc_silu(ga, ga, tr * I);", "orc_silu(up, up, tr * I);"],
        ["test_swiglu_block_closed_form"]),
    "forward_q_bias_dropped": (
        ["L->q, L->t_q, L->q_bias, qr)", "L->q, L->t_q, NULL, qr)"],
        ["test_scores_from_rotated_biases"]),
    "forward_k_bias_dropped": (
        ["L->k, L->t_k, L->k_bias, kk)", "L->k, L->t_k, NULL, kk)"],
        ["test_scores_from_rotated_biases"]),
    "forward_v_bias_dropped": (
        ["L->v, L->t_v, L->v_bias, vv)", "L->v, L->t_v, NULL, vv)"],
        ["test_attention_of_constant_values_is_the_group_bias", "test_scores_from_rotated_biases"]),
    "forward_k_bias_on_v": (
        ["L->v, L->t_v, L->v_bias, vv)", "L->v, L->t_v, L->k_bias, vv)"],
        ["test_attention_of_constant_values_is_the_group_bias"]),
    "forward_query_rotated_at_the_cache_start": (
        ["g->ctx, c->len + r0)) goto done;", "g->ctx, c->len)) goto done;"],
        ["test_scores_from_rotated_biases"]),
    "attention_heads_interleaved_over_groups": (
        ["size_t base = (h / per) * hd;", "size_t base = (h % kvh) * hd;"],
        ["test_attention_of_constant_values_is_the_group_bias", "test_scores_from_rotated_biases"]),
}


@pytest.fixture(scope="module")
def workdir(tmp_path_factory):
    if not shutil.which("gcc"):
        pytest.skip("gcc is needed to build the mutants")
    return tmp_path_factory.mktemp("mutants")


def _run_pins(name, src, tests, workdir):
    c_path = os.path.join(workdir, f"{name}.c")
    so_path = os.path.join(workdir, f"{name}.so")
    with open(c_path, "w") as f:
        f.write(src)
    shutil.copy(os.path.join(ROOT, "oracle", "cx_oracle.h"), os.path.join(workdir, "cx_oracle.h"))
    subprocess.run(["gcc", "-std=c11", "-O3", "-mavx2", "-fPIC", "-ffp-contract=off",
                    "-fno-fast-math", "-fopenmp", "-shared", "-o", so_path, c_path, "-lm"],
                   check=True)  # oracle/Makefile's flags
    args = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider"] + PINS
    if tests:  # parametrized ids select by their function's name
        args += ["-k", " or ".join(sorted({t.split("[")[0] for t in tests}))]
    return subprocess.run(args, cwd=ROOT, env=dict(os.environ, CX_ORACLE_LIB=so_path),
                          capture_output=True, text=True, timeout=300)


def test_the_unchanged_copy_passes(workdir):
    r = _run_pins("unchanged", open(SRC).read(), None, workdir)
    assert r.returncode == 0, r.stdout[-2000:]


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pinning_tests_fail_on_the_mutant(name, workdir):
    edits, tests = MUTANTS[name]
    src = open(SRC).read()
    for old, new in zip(edits[::2], edits[1::2]):
        assert src.count(old) == 1, f"{name}: the text to mutate is not unique in cx_oracle.c: {old!r}"
        src = src.replace(old, new)
    r = _run_pins(name, src, tests, workdir)
    assert r.returncode == 1, f"{name}: the pins did not fail (rc {r.returncode}):\n{r.stdout[-2000:]}"
    for t in tests:
        assert any(f"FAILED {p}::{t}" in r.stdout for p in PINS), \
            f"{name}: {t} did not fail:\n{r.stdout[-2000:]}"
