"""The oracle's pins catch plausible mistakes.  Each case plants one mistake in a copy of the C
oracle (oracle/ud_oracle.c) -- a dropped term, a wrong sign, index or constant, swapped operands or
gates -- builds it into a temporary library, and runs the CPU pinning tests that guard that
function against it (the reference's known-answer tests, the torch / numpy restatements, closed
forms, golden fixtures).  They must fail; the same tests pass against the unmodified source built
the same way.  CPU only; nothing here touches the product library's compute."""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest

from conftest import ROOT

SRC = os.path.join(ROOT, "oracle", "ud_oracle.c")
T = "tests/"

# (case, original text (exactly once in the source), planted mistake, pinning tests that must fail)
MUTANTS = [
    ("lcg_increment", "c = 1442695040888963407ULL", "c = 1442695040888963409ULL",
     [T + "test_oracle.py::test_lcg_golden_fixture"]),
    ("bf16_truncates", "uint32_t rounding = ((u >> 16) & 1u) + 0x7FFFu;", "uint32_t rounding = 0u;",
     [T + "test_oracle.py::test_bf16_rounding_matches_torch"]),
    ("layernorm_unbiased_var", "sqrt(v / D + (double)eps)", "sqrt(v / (D - 1) + (double)eps)",
     [T + "test_oracle.py::test_layer_norm_kat"]),
    ("layernorm_no_beta", "if (beta) y += beta[i];", "(void)beta;",
     [T + "test_oracle.py::test_layer_norm_kat"]),
    ("gemm_scale_inside_act", "v = orc_act(v, act) * out_scale;", "v = orc_act(v * out_scale, act);",
     [T + "test_oracle.py::test_gemm_epilogue_kat"]),
    ("gemm_residual_unscaled", "if (R) v += res_scale * R[(int64_t)m * N + n];", "if (R) v += R[(int64_t)m * N + n];",
     [T + "test_oracle.py::test_gemm_epilogue_kat"]),
    ("glu_halves_swapped", "out[t * D + d] = (float)(a / (1.0 + exp(-b)));", "out[t * D + d] = (float)(b / (1.0 + exp(-a)));",
     [T + "test_oracle.py::test_glu_and_dwconv_kat"]),
    ("dwconv_taps_reversed", "acc += (double)w[d * K + k] * x[(int64_t)(t + k) * D + d];",
     "acc += (double)w[d * K + (K - 1 - k)] * x[(int64_t)(t + k) * D + d];",
     [T + "test_oracle.py::test_glu_and_dwconv_kat"]),
    ("sinusoid_sin_cos_swapped", "pe[i] = (float)sin((double)angle);\n        pe[i + 1] = (float)cos((double)angle);",
     "pe[i] = (float)cos((double)angle);\n        pe[i + 1] = (float)sin((double)angle);",
     [T + "test_oracle.py::test_sinusoid_closed_form"]),
    ("rel_shift_off_by_one", "(shift - j + rel_offset) * (H * dk)", "(shift - j + 1 + rel_offset) * (H * dk)",
     [T + "test_oracle.py::test_relpos_attention_kat_matches_nemo_rel_shift"]),
    ("pos_bias_u_for_v", "((double)q[d] + bias_v[hoff + d]) * pr[d]", "((double)q[d] + bias_u[hoff + d]) * pr[d]",
     [T + "test_oracle.py::test_relpos_attention_kat_matches_nemo_rel_shift"]),
    ("attention_unscaled", "s[j - ks] = a * scale;\n                if (s[j - ks] > m) m = s[j - ks];\n            }\n            double den = 0;\n            for (int j = ks; j < ke; j++) { s[j - ks] = exp(s[j - ks] - m); den += s[j - ks]; }\n            double inv",
     "s[j - ks] = a;\n                if (s[j - ks] > m) m = s[j - ks];\n            }\n            double den = 0;\n            for (int j = ks; j < ke; j++) { s[j - ks] = exp(s[j - ks] - m); den += s[j - ks]; }\n            double inv",
     [T + "test_oracle.py::test_relpos_attention_kat_matches_nemo_rel_shift"]),
    ("macaron_full_step", "orc_gemm_nt(ffh, w[W_FF1_W2], NULL, x, r1, (int)M, D, ff, 1.0f, ORC_ACT_NONE, 0.5f, 1.0f);",
     "orc_gemm_nt(ffh, w[W_FF1_W2], NULL, x, r1, (int)M, D, ff, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);",
     [T + "test_oracle.py::test_encoder_offline_matches_torch_nemo_layer"]),
    ("conv_mask_rows_dropped", "if (v < T) memset(glued + (int64_t)v * D, 0, sizeof(float) * (size_t)(T - v) * D);",
     "(void)v;",
     [T + "test_oracle.py::test_stream_cache_rule"]),
    ("conv_ln_without_silu", "orc_layer_norm(r4, w[W_CONV_LN_W], w[W_CONV_LN_B], tmp, M, D, 1e-5f, ORC_ACT_SILU);",
     "orc_layer_norm(r4, w[W_CONV_LN_W], w[W_CONV_LN_B], tmp, M, D, 1e-5f, ORC_ACT_NONE);",
     [T + "test_oracle.py::test_encoder_offline_matches_torch_nemo_layer"]),
    ("cache_len_advances_by_valid", "cache_len[s] = cache_len[s] + T < L ? cache_len[s] + T : L;",
     "cache_len[s] = cache_len[s] + vclamp[s] < L ? cache_len[s] + vclamp[s] : L;",
     [T + "test_oracle.py::test_stream_cache_rule"]),
    ("chunked_ranges_one_chunk_short", "int lo = (c - lc) * cs, hi = (c + 1) * cs;", "int lo = (c - lc + 1) * cs, hi = (c + 1) * cs;",
     [T + "test_ranges.py::test_chunked_limited_matches_oracle"]),
    ("gqa_head_map_modulo", "const int kvh = h / group;", "const int kvh = h % Hkv;",
     [T + "test_oracle_decode.py"]),
    ("rope_sign", "row[i] = (float)(a * c - b * sn);", "row[i] = (float)(a * c + b * sn);",
     [T + "test_oracle_decode.py::test_rope_kat"]),
    ("conv2d_padding_shift", "const int hi = ho * stride + kh - pad_top;", "const int hi = ho * stride + kh - pad_top + 1;",
     [T + "test_oracle_subsample.py::test_conv2d_reference_kat_against_torch"]),
    ("subsample_out_columns_unpermuted", "wp[((int64_t)o * F3 + f) * C + c] = sw[10][((int64_t)o * C + c) * F3 + f];",
     "wp[((int64_t)o * F3 + f) * C + c] = sw[10][((int64_t)o * F3 + f) * C + c];",
     [T + "test_oracle_subsample.py::test_subsample_matches_nemo_restatement"]),
    ("lstm_input_forget_swapped", "const double ig = orc_sigmoid(gates[j]), fg = orc_sigmoid(gates[H + j])",
     "const double ig = orc_sigmoid(gates[H + j]), fg = orc_sigmoid(gates[j])",
     [T + "test_oracle_rnnt.py::test_predict_matches_lstmcell"]),
    ("greedy_one_symbol_extra", "while (emitted < max_symbols) {", "while (emitted <= max_symbols) {",
     [T + "test_oracle_rnnt.py::test_greedy_matches_nemo_loop_across_chunks"]),
    ("mel_preemphasis", "const float m = 0.97f * audio[idx - 1];", "const float m = 0.95f * audio[idx - 1];",
     [T + "test_oracle_mel.py::test_features_match_torch_stft_and_rfft"]),
]


def _compile(src_text, out_dir):
    os.makedirs(out_dir, exist_ok=True)
    c = os.path.join(out_dir, "ud_oracle.c")
    with open(c, "w") as f:
        f.write(src_text)
    so = os.path.join(out_dir, "libud_oracle.so")
    r = subprocess.run(["gcc", "-O2", "-std=c11", "-mavx2", "-mfma", "-fopenmp", "-fPIC", "-shared", "-fvisibility=hidden",
                        c, "-o", so, "-lm"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    return so if r.returncode == 0 else "compile failed:\n" + r.stdout


@pytest.fixture(scope="module")
def builds(tmp_path_factory):
    """Every mutant (and the unmodified source) built once, in parallel."""
    src = open(SRC).read()
    base = tmp_path_factory.mktemp("mutants")
    jobs = {"control": src}
    for name, old, new, _ in MUTANTS:
        assert src.count(old) == 1, "mutation site of %s not found exactly once" % name
        jobs[name] = src.replace(old, new)
    with ThreadPoolExecutor(max_workers=8) as ex:
        futs = {k: ex.submit(_compile, v, str(base / k)) for k, v in jobs.items()}
        return {k: f.result() for k, f in futs.items()}


def _run_tests(lib_path, tests):
    env = dict(os.environ, UD_ORACLE_LIB=lib_path, OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu"] + tests,
                       cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    return r.returncode, r.stdout


def test_control_passes(builds):
    so = builds["control"]
    assert os.path.exists(so), so
    tests = sorted({t for _, _, _, ts in MUTANTS for t in ts})
    rc, out = _run_tests(so, tests)
    assert rc == 0, out[-3000:]


@pytest.mark.parametrize("name,old,new,tests", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_mutant_is_caught(builds, name, old, new, tests):
    so = builds[name]
    assert os.path.exists(so), so
    rc, out = _run_tests(so, tests)
    assert rc == 1, "planted mistake %r was not caught (pytest exit %d):\n%s" % (name, rc, out[-3000:])
