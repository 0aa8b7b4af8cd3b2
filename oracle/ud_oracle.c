/*
 * ud_oracle.c -- CPU restatement of DictatorEngine's cache-aware streaming
 * FastConformer encoder step.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity reference for the HIP
 * library and the timed CPU baseline of the benchmark.  Only tests/, the
 * smoke entry point and the benchmark's cpu_baseline leg may load it; the
 * product path never calls it.
 *
 * Every function cites the reference file:line whose semantics it restates
 * (paths relative to the reference repository root).  Arithmetic is fp32
 * data with wider accumulation where that tightens the anchor (LayerNorm
 * statistics and attention in double); GEMMs accumulate in fp32 with a SIMD
 * reduction, which is what the reference's fp32 kernels do.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   orc_lcg_floats        reference KAT generator, closed form + fixture
 *   orc_bf16_*            exhaustive/edge cases against the bit rule
 *   orc_layer_norm        numpy float64 LayerNorm + SiLU (library routine)
 *   orc_gemm_nt           numpy float64 matmul, epilogue order KAT
 *   orc_glu               torch.nn.functional.glu
 *   orc_dwconv1d          numpy.convolve per channel
 *   orc_sinusoid          float64 closed form
 *   orc_relpos_attention  NeMo pad/view rel_shift transcription (KAT) and
 *                         softmax invariants
 *   orc_encoder_layer     torch restatement of NeMo's layer on a full
 *                         utterance (conv1d with causal padding, literal
 *                         rel_shift, chunked_limited mask)
 *   orc_stream_step       streaming == offline equivalence through the
 *                         torch restatement, and the cache rule
 *   orc_set_store_limit   the torch restatement with the same clamps at the
 *                         same points (a limit small enough that every clamp
 *                         point engages), and limit 0 == no limit
 *   orc_gqa_attention     reference KAT (VoxtralOpTests.swift:6-38) against a
 *                         numpy float64 softmax attention; GQA head map
 *   orc_rope_rotate_half  reference KAT (VoxtralOpTests.swift:60-75) against
 *                         rotation by a complex exponential (numpy)
 *   orc_conv2d_cl         reference KAT shapes (ConformerOpTests.swift:49-78)
 *                         against torch.nn.functional.conv2d with explicit
 *                         F.pad (library routine)
 *   orc_subsample         torch restatement of NeMo's causal dw_striding
 *                         ConvSubsampling with MaskedConvSequential length
 *                         masks and the (channel, freq) flatten on the
 *                         checkpoint's out.weight (tests/refimpl.py)
 *   orc_rnnt_*            torch.nn.LSTMCell prediction network and NeMo's
 *                         greedy loop without a prediction cache
 *                         (reference/nemo/check_spec.py:176-207 structure,
 *                         tests/refimpl.py), across chunk boundaries
 *   orc_mel_tables/frames torch.stft restatement of NeMo FilterbankFeatures
 *                         (preemphasis, centred constant-padded STFT with the
 *                         400-sample Hann window in 512, |X|^2, filterbank,
 *                         log guard 2^-24) and numpy.fft.rfft; the reference
 *                         KAT NemoMelStream == features (StreamingEquivalence
 *                         Tests.swift:9-20)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

enum { ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_SILU = 2, ORC_ACT_GELU_ERF = 4 };

/* ------------------------------------------------------------------ utils */

/* Tests/DictatorEngineTests/GemmTests.swift:7-14 -- 64-bit LCG, uniform in [-1, 1). */
ORC_API void orc_lcg_floats(float* out, int64_t n, uint64_t seed) {
    const uint64_t a = 6364136223846793005ULL, c = 1442695040888963407ULL;
    uint64_t s = seed * a + c;
    for (int64_t i = 0; i < n; i++) {
        s = s * a + c;
        int64_t v = (int64_t)(s >> 11) % (1LL << 24);
        out[i] = (float)v / (float)(1 << 23) - 1.0f;
    }
}

/* Sources/DictatorEngine/Core/Tensor.swift:116-122 -- RNE, NaN -> 0x7FC0. */
ORC_API uint16_t orc_bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (isnan(f)) return 0x7FC0;
    uint32_t rounding = ((u >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((u + rounding) >> 16);
}

/* Sources/DictatorEngine/Metal/00_common.metal:32 -- widening is a shift. */
ORC_API float orc_bf16_to_float(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

ORC_API void orc_round_bf16(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_bf16_to_float(orc_bf16_bits(x[i]));
}

ORC_API void orc_to_bf16(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_bf16_bits(x[i]);
}

/* Sources/DictatorEngine/Metal/00_common.metal:14-29 -- activations. */
static inline float orc_erf_as(float x) {
    float s = x < 0 ? -1.0f : (x > 0 ? 1.0f : 0.0f);
    float a = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * a);
    float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                      0.254829592f) * t * expf(-a * a);
    return s * y;
}

static inline float orc_act(float x, int act) {
    switch (act) {
        case ORC_ACT_RELU: return x > 0 ? x : 0.0f;
        case ORC_ACT_SILU: return (float)((double)x / (1.0 + exp(-(double)x)));
        case ORC_ACT_GELU_ERF: return 0.5f * x * (1.0f + orc_erf_as(x * 0.7071067811865476f));
        default: return x;
    }
}

/* ------------------------------------------------------------------ ops */

/* Sources/DictatorEngine/Metal/20_conformer.metal:25-49 (layer_norm), dispatched by
 * Core/Ops.swift:27-33: two-pass mean / population variance, y = act((x-mu)*rsqrt(var+eps)*g+b). */
ORC_API void orc_layer_norm(const float* x, const float* gamma, const float* beta, float* out,
                            int64_t rows, int D, float eps, int act) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * D;
        double s = 0;
        for (int i = 0; i < D; i++) s += xr[i];
        double mean = s / D;
        double v = 0;
        for (int i = 0; i < D; i++) { double d = xr[i] - mean; v += d * d; }
        double inv = 1.0 / sqrt(v / D + (double)eps);
        float* o = out + r * D;
        for (int i = 0; i < D; i++) {
            double y = (xr[i] - mean) * inv * gamma[i];
            if (beta) y += beta[i];
            o[i] = orc_act((float)y, act);
        }
    }
}

static inline float orc_dot(const float* a, const float* b, int K) {
    float s = 0.0f;
#pragma omp simd reduction(+ : s)
    for (int k = 0; k < K; k++) s += a[k] * b[k];
    return s;
}

/* Sources/DictatorEngine/Core/Kernels.swift:79-112 and Metal/12_gemm2.metal:111-122 (epilogue):
 * C[M,N] = out_scale * act(alpha * A[M,K] . W[N,K]^T + bias[N]) + res_scale * R[M,N].
 * W stays in the checkpoint's [out, in] layout.  R may alias C (in-place residual). */
ORC_API void orc_gemm_nt(const float* A, const float* W, const float* bias, const float* R, float* C,
                         int M, int N, int K, float alpha, int act, float out_scale, float res_scale) {
    const int NB = 32, MB = 16;
#pragma omp parallel for collapse(2) schedule(static)
    for (int n0 = 0; n0 < N; n0 += NB) {
        for (int m0 = 0; m0 < M; m0 += MB) {
            int n1 = n0 + NB < N ? n0 + NB : N, m1 = m0 + MB < M ? m0 + MB : M;
            for (int m = m0; m < m1; m++) {
                for (int n = n0; n < n1; n++) {
                    float v = alpha * orc_dot(A + (int64_t)m * K, W + (int64_t)n * K, K);
                    if (bias) v += bias[n];
                    v = orc_act(v, act) * out_scale;
                    if (R) v += res_scale * R[(int64_t)m * N + n];
                    C[(int64_t)m * N + n] = v;
                }
            }
        }
    }
}

/* Sources/DictatorEngine/Metal/20_conformer.metal:76-85: out[t,d] = in[t,d] * sigmoid(in[t,D+d]). */
ORC_API void orc_glu(const float* x, float* out, int64_t T, int D) {
    for (int64_t t = 0; t < T; t++)
        for (int d = 0; d < D; d++) {
            double a = x[t * 2 * D + d], b = x[t * 2 * D + D + d];
            out[t * D + d] = (float)(a / (1.0 + exp(-b)));
        }
}

/* Sources/DictatorEngine/Metal/20_conformer.metal:87-102: in [Tout+K-1, D],
 * out[t,d] = act(bias[d] + sum_k w[d,k] * in[t+k,d]); tap K-1 is the current frame. */
ORC_API void orc_dwconv1d(const float* x, const float* w, const float* bias, float* out,
                          int Tout, int D, int K, int act) {
    for (int t = 0; t < Tout; t++)
        for (int d = 0; d < D; d++) {
            double acc = bias ? bias[d] : 0.0;
            for (int k = 0; k < K; k++) acc += (double)w[d * K + k] * x[(int64_t)(t + k) * D + d];
            out[(int64_t)t * D + d] = orc_act((float)acc, act);
        }
}

/* Sources/DictatorEngine/Models/FastConformer.swift:147-158 (sinusoid): the NeMo
 * RelPositionalEncoding row for relative position `pos`, with the reference's mix of float and
 * double evaluation (k and angle in float, exp/sin/cos in double then rounded). */
ORC_API void orc_sinusoid(int pos, int D, float* pe) {
    const float k = -((float)log(10000.0) / (float)D);
    for (int i = 0; i < D; i += 2) {
        float div = (float)exp((double)((float)i * k));
        float angle = (float)pos * div;
        pe[i] = (float)sin((double)angle);
        pe[i + 1] = (float)cos((double)angle);
    }
}

/* FastConformer.swift:161-178 (preparePositionTables), first half: PE rows for rel = lo..hi,
 * row index = rel - lo (so rel_offset = -lo). */
ORC_API void orc_pe_rows(int lo, int hi, int D, float* pe) {
    for (int r = lo; r <= hi; r++) orc_sinusoid(r, D, pe + (int64_t)(r - lo) * D);
}

/* Sources/DictatorEngine/Metal/20_conformer.metal:140-220 (relpos_attention), dispatched by
 * Core/Ops.swift:80-90 with scale 1/sqrt(dk).  For query i, head h and key j in
 * [max(r.x,0), min(r.y,Tk)):
 *   s_j = ((q_i+u_h).K_j + (q_i+v_h).P[(Tk-Tq+i)-j+rel_offset]) * scale
 *   out = sum_j softmax(s)_j V_j ; an empty range gives 0.
 * Row strides ldq/ldk/ldv/ldo are in elements; P rows are H*dk wide. */
ORC_API void orc_relpos_attention(const float* Q, const float* K, const float* V, const float* P,
                                  const float* bias_u, const float* bias_v, const int32_t* ranges,
                                  float* out, int Tq, int Tk, int H, int dk, int ldq, int ldk, int ldv,
                                  int ldo, int rel_offset, int n_rel, float scale) {
    (void)n_rel;
#pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < H; h++) {
        for (int i = 0; i < Tq; i++) {
            const int hoff = h * dk;
            double* s = (double*)malloc(sizeof(double) * (Tk > 0 ? Tk : 1));
            int ks = ranges[2 * i] > 0 ? ranges[2 * i] : 0;
            int ke = ranges[2 * i + 1] < Tk ? ranges[2 * i + 1] : Tk;
            int shift = Tk - Tq + i;
            double m = -INFINITY;
            for (int j = ks; j < ke; j++) {
                const float* kr = K + (int64_t)j * ldk + hoff;
                const float* pr = P + (int64_t)(shift - j + rel_offset) * (H * dk) + hoff;
                const float* q = Q + (int64_t)i * ldq + hoff;
                double a = 0;
                for (int d = 0; d < dk; d++)
                    a += ((double)q[d] + bias_u[hoff + d]) * kr[d] + ((double)q[d] + bias_v[hoff + d]) * pr[d];
                s[j - ks] = a * scale;
                if (s[j - ks] > m) m = s[j - ks];
            }
            double den = 0;
            for (int j = ks; j < ke; j++) { s[j - ks] = exp(s[j - ks] - m); den += s[j - ks]; }
            double inv = den > 0 ? 1.0 / den : 0.0;
            for (int d = 0; d < dk; d++) {
                double acc = 0;
                for (int j = ks; j < ke; j++) acc += s[j - ks] * V[(int64_t)j * ldv + hoff + d];
                out[(int64_t)i * ldo + hoff + d] = (float)(acc * inv);
            }
            free(s);
        }
    }
}

/* ------------------------------------------------------------------ decoder attention */

/* Sources/DictatorEngine/Metal/30_voxtral.metal:45-101 (attention_gqa), dispatched by
 * Sources/DictatorEngine/Core/Ops.swift:136-169: query i, head h uses kv head h / (Hq/Hkv); scores
 * (q . k) * scale over keys [max(r.x, 0), min(r.y, Tk)); softmax; . V; 0 for an empty range.
 * Q [Tq, ldq], K/V [Tk, ldk] (row strides), out [Tq, ldo].  Accumulates in double. */
ORC_API void orc_gqa_attention(const float* Q, const float* K, const float* V, const int32_t* ranges, float* out,
                               int Tq, int Tk, int Hq, int Hkv, int d, int ldq, int ldk, int ldo, float scale) {
    const int group = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < Tq; i++) {
        for (int h = 0; h < Hq; h++) {
            const int kvh = h / group;
            const int ks = ranges[2 * i] > 0 ? ranges[2 * i] : 0;
            const int ke = ranges[2 * i + 1] < Tk ? ranges[2 * i + 1] : Tk;
            const float* q = Q + (int64_t)i * ldq + h * d;
            float* o = out + (int64_t)i * ldo + h * d;
            if (ke <= ks) {
                for (int e = 0; e < d; e++) o[e] = 0.0f;
                continue;
            }
            double* s = (double*)malloc(sizeof(double) * (size_t)(ke - ks));
            double m = -INFINITY;
            for (int j = ks; j < ke; j++) {
                const float* kr = K + (int64_t)j * ldk + kvh * d;
                double a = 0;
                for (int e = 0; e < d; e++) a += (double)q[e] * kr[e];
                s[j - ks] = a * scale;
                if (s[j - ks] > m) m = s[j - ks];
            }
            double den = 0;
            for (int j = ks; j < ke; j++) { s[j - ks] = exp(s[j - ks] - m); den += s[j - ks]; }
            for (int e = 0; e < d; e++) {
                double acc = 0;
                for (int j = ks; j < ke; j++) acc += s[j - ks] * V[(int64_t)j * ldk + kvh * d + e];
                o[e] = (float)(acc / den);
            }
            free(s);
        }
    }
}

/* Sources/DictatorEngine/Metal/30_voxtral.metal:20-36 (rope_rotate_half) in place on x [T, ld]:
 * for head h and pair (i, i + d/2), angle = float(pos(t)) * inv_freq[i] (a float product, as the
 * reference computes it), x_i' = x_i cos - x_{i+d/2} sin, x_{i+d/2}' = x_{i+d/2} cos + x_i sin, with
 * cos/sin of that angle in double.  pos(t) = positions[t] if positions, else pos0 + t. */
ORC_API void orc_rope_rotate_half(float* x, int T, int H, int d, int ld, const int32_t* positions, int pos0,
                                  const float* inv_freq) {
    const int half = d / 2;
    for (int t = 0; t < T; t++) {
        const int p = positions ? positions[t] : pos0 + t;
        for (int h = 0; h < H; h++) {
            float* row = x + (int64_t)t * ld + h * d;
            for (int i = 0; i < half; i++) {
                const float angle = (float)p * inv_freq[i];
                const double c = cos((double)angle), sn = sin((double)angle);
                const double a = row[i], b = row[i + half];
                row[i] = (float)(a * c - b * sn);
                row[i + half] = (float)(b * c + a * sn);
            }
        }
    }
}

/* ------------------------------------------------------------------ encoder */

/* Per-layer weight slots, in the order of ConformerLayerWeights (FastConformer.swift:41-54) with
 * the NeMo names of the checkpoint (loading at FastConformer.swift:96-143). */
enum {
    W_NORM_FF1_W, W_NORM_FF1_B, W_FF1_W1, W_FF1_W2,
    W_NORM_ATT_W, W_NORM_ATT_B, W_Q, W_K, W_V, W_O, W_POS, W_BIAS_U, W_BIAS_V,
    W_NORM_CONV_W, W_NORM_CONV_B, W_PW1, W_DW, W_CONV_LN_W, W_CONV_LN_B, W_PW2,
    W_NORM_FF2_W, W_NORM_FF2_B, W_FF2_W1, W_FF2_W2, W_NORM_OUT_W, W_NORM_OUT_B,
    W_COUNT
};

ORC_API int orc_weight_count(void) { return W_COUNT; }

/* Storage-range model of a 16-bit encoder (not part of the reference, whose activations are fp32):
 * with a limit > 0, every value the 16-bit encoder stores in 16 bits -- the LayerNorm outputs that
 * feed a projection, the FF hidden, q/k/v (and so the cached K/V rows), the attention output and
 * the conv module's LayerNorm + SiLU output -- is clamped to [-limit, limit] (NaN kept), as the
 * HIP library's saturating half stores do at limit 65504.  0 (the default) = no limit. */
static float g_store_limit = 0.0f;
ORC_API void orc_set_store_limit(float limit) { g_store_limit = limit > 0.0f ? limit : 0.0f; }
static void orc_store_clip(float* x, int64_t n) {
    const float lim = g_store_limit;
    if (lim <= 0.0f) return;
    for (int64_t i = 0; i < n; i++)
        if (!isnan(x[i])) x[i] = x[i] < -lim ? -lim : (x[i] > lim ? lim : x[i]);
}

/* FastConformer.swift:161-178: P_l = PE . W_pos,l^T over rel = lo..hi (one table per layer). */
ORC_API void orc_pos_table(const float* wpos, int lo, int hi, int D, float* P) {
    int n = hi - lo + 1;
    float* pe = (float*)malloc(sizeof(float) * (size_t)n * D);
    orc_pe_rows(lo, hi, D, pe);
    orc_gemm_nt(pe, wpos, NULL, NULL, P, n, D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);
    free(pe);
}

/* FastConformer.swift:262-321 (encodeLayer) over a batch of S independent sequences that share
 * weights.  Each sequence s has T query rows x[s] ([T, D]), its own key/value buffers
 * keys[s]/vals[s] ([Tk, D]; the last T rows receive this chunk's projections, earlier rows hold
 * cached projections), its conv input convIn[s] ([K-1+T, D]; rows [K-1, K-1+T) receive this chunk's
 * GLU output), its own per-query key ranges ranges[s] ([T, 2]) and its own valid frame count.
 * Row-wise ops (LayerNorm, GEMMs) run over all S*T rows at once: that is row-for-row the same
 * arithmetic as the reference's per-stream dispatch.  x and out may not alias. */
ORC_API void orc_encoder_layer(const float* const* w, const float* P, int rel_offset, int n_rel,
                               int S, int T, int Tk, int D, int H, int ff, int Kc,
                               const float* x, float* out, float* keys, float* vals, float* convIn,
                               const int32_t* ranges, const int32_t* valid) {
    const int64_t M = (int64_t)S * T;
    const int dk = D / H;
    const int CIN = Kc - 1 + T;
    float* tmp = (float*)malloc(sizeof(float) * M * D);
    float* ffh = (float*)malloc(sizeof(float) * M * ff);
    float* r1 = (float*)malloc(sizeof(float) * M * D);
    float* r2 = (float*)malloc(sizeof(float) * M * D);
    float* r3 = (float*)malloc(sizeof(float) * M * D);
    float* r4 = (float*)malloc(sizeof(float) * M * D);
    float* q = (float*)malloc(sizeof(float) * M * D);
    float* kn = (float*)malloc(sizeof(float) * M * D);
    float* vn = (float*)malloc(sizeof(float) * M * D);
    float* att = (float*)malloc(sizeof(float) * M * D);
    float* pw = (float*)malloc(sizeof(float) * M * 2 * D);

    /* FF1 (macaron, x0.5): FastConformer.swift:276-279 */
    orc_layer_norm(x, w[W_NORM_FF1_W], w[W_NORM_FF1_B], tmp, M, D, 1e-5f, ORC_ACT_NONE);
    orc_store_clip(tmp, M * D);
    orc_gemm_nt(tmp, w[W_FF1_W1], NULL, NULL, ffh, (int)M, ff, D, 1.0f, ORC_ACT_SILU, 1.0f, 1.0f);
    orc_store_clip(ffh, M * ff);
    orc_gemm_nt(ffh, w[W_FF1_W2], NULL, x, r1, (int)M, D, ff, 1.0f, ORC_ACT_NONE, 0.5f, 1.0f);

    /* Self-attention: FastConformer.swift:282-292 */
    orc_layer_norm(r1, w[W_NORM_ATT_W], w[W_NORM_ATT_B], tmp, M, D, 1e-5f, ORC_ACT_NONE);
    orc_store_clip(tmp, M * D);
    orc_gemm_nt(tmp, w[W_Q], NULL, NULL, q, (int)M, D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);
    orc_gemm_nt(tmp, w[W_K], NULL, NULL, kn, (int)M, D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);
    orc_gemm_nt(tmp, w[W_V], NULL, NULL, vn, (int)M, D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);
    orc_store_clip(q, M * D);
    orc_store_clip(kn, M * D);
    orc_store_clip(vn, M * D);
    for (int s = 0; s < S; s++) {
        memcpy(keys + ((int64_t)s * Tk + Tk - T) * D, kn + (int64_t)s * T * D, sizeof(float) * T * D);
        memcpy(vals + ((int64_t)s * Tk + Tk - T) * D, vn + (int64_t)s * T * D, sizeof(float) * T * D);
        orc_relpos_attention(q + (int64_t)s * T * D, keys + (int64_t)s * Tk * D, vals + (int64_t)s * Tk * D, P,
                             w[W_BIAS_U], w[W_BIAS_V], ranges + (int64_t)s * T * 2, att + (int64_t)s * T * D,
                             T, Tk, H, dk, D, D, D, D, rel_offset, n_rel, 1.0f / sqrtf((float)dk));
    }
    orc_store_clip(att, M * D);
    orc_gemm_nt(att, w[W_O], NULL, r1, r2, (int)M, D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);

    /* Convolution module: FastConformer.swift:295-311 (causal conv, conv LayerNorm + SiLU) */
    orc_layer_norm(r2, w[W_NORM_CONV_W], w[W_NORM_CONV_B], tmp, M, D, 1e-5f, ORC_ACT_NONE);
    orc_store_clip(tmp, M * D);
    orc_gemm_nt(tmp, w[W_PW1], NULL, NULL, pw, (int)M, 2 * D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);
    for (int s = 0; s < S; s++) {
        float* ci = convIn + (int64_t)s * CIN * D;
        float* glued = ci + (int64_t)(Kc - 1) * D;
        orc_glu(pw + (int64_t)s * T * 2 * D, glued, T, D);
        /* maskRows (FastConformer.swift:246-250, 302): GLU rows >= valid are zero */
        int v = valid[s] < 0 ? 0 : valid[s];
        if (v < T) memset(glued + (int64_t)v * D, 0, sizeof(float) * (size_t)(T - v) * D);
        orc_dwconv1d(ci, w[W_DW], NULL, r4 + (int64_t)s * T * D, T, D, Kc, ORC_ACT_NONE);
    }
    orc_layer_norm(r4, w[W_CONV_LN_W], w[W_CONV_LN_B], tmp, M, D, 1e-5f, ORC_ACT_SILU);
    orc_store_clip(tmp, M * D);
    orc_gemm_nt(tmp, w[W_PW2], NULL, r2, r3, (int)M, D, D, 1.0f, ORC_ACT_NONE, 1.0f, 1.0f);

    /* FF2 (x0.5) and the output LayerNorm: FastConformer.swift:314-320 */
    orc_layer_norm(r3, w[W_NORM_FF2_W], w[W_NORM_FF2_B], tmp, M, D, 1e-5f, ORC_ACT_NONE);
    orc_store_clip(tmp, M * D);
    orc_gemm_nt(tmp, w[W_FF2_W1], NULL, NULL, ffh, (int)M, ff, D, 1.0f, ORC_ACT_SILU, 1.0f, 1.0f);
    orc_store_clip(ffh, M * ff);
    orc_gemm_nt(ffh, w[W_FF2_W2], NULL, r3, r4, (int)M, D, ff, 1.0f, ORC_ACT_NONE, 0.5f, 1.0f);
    orc_layer_norm(r4, w[W_NORM_OUT_W], w[W_NORM_OUT_B], out, M, D, 1e-5f, ORC_ACT_NONE);

    free(tmp); free(ffh); free(r1); free(r2); free(r3); free(r4);
    free(q); free(kn); free(vn); free(att); free(pw);
}

/* FastConformer.swift:441-480 (encodeStreamStep, from the copy of the kept subsampled rows on):
 * one cache-aware chunk step for S streams of T frames each.
 *   w      : layers * W_COUNT weight pointers (layer-major)
 *   P      : layers position tables [n_rel, D], row = rel + rel_offset
 *   x      : [S, T, D] chunk input (the subsampled frames after the drop)
 *   valid  : [S] valid frames per stream (validT)
 *   kcache/vcache : [S, layers, L, D] logical order (oldest first)
 *   ccache : [S, layers, K-1, D] conv input cache, oldest first
 *   cache_len : [S] valid cached frames, updated to min(cache_len + T, L)
 *   out    : [S, T, D]
 * Keys are [L cached ; T new] for every stream, with ranges [L - cache_len, L + valid) for every
 * query (FastConformer.swift:458-462); the next caches are the last L keys/values and the last K-1
 * conv inputs (FastConformer.swift:469-472), and cache_len advances by T, not by valid (:477). */
ORC_API void orc_stream_step(const float* const* w, const float* const* P, int rel_offset, int n_rel,
                             int layers, int S, int T, int L, int D, int H, int ff, int Kc,
                             const float* x, const int32_t* valid, float* kcache, float* vcache,
                             float* ccache, int32_t* cache_len, float* out) {
    const int Tk = L + T, CIN = Kc - 1 + T;
    const int64_t M = (int64_t)S * T;
    float* keys = (float*)malloc(sizeof(float) * (size_t)S * Tk * D);
    float* vals = (float*)malloc(sizeof(float) * (size_t)S * Tk * D);
    float* conv = (float*)malloc(sizeof(float) * (size_t)S * CIN * D);
    float* xa = (float*)malloc(sizeof(float) * M * D);
    float* xb = (float*)malloc(sizeof(float) * M * D);
    int32_t* ranges = (int32_t*)malloc(sizeof(int32_t) * M * 2);
    int32_t* vclamp = (int32_t*)malloc(sizeof(int32_t) * S);
    for (int s = 0; s < S; s++) {
        int v = valid[s] < 0 ? 0 : (valid[s] > T ? T : valid[s]);
        vclamp[s] = v;
        for (int t = 0; t < T; t++) {
            ranges[((int64_t)s * T + t) * 2] = L - cache_len[s];
            ranges[((int64_t)s * T + t) * 2 + 1] = L + v;
        }
    }
    memcpy(xa, x, sizeof(float) * M * D);
    for (int li = 0; li < layers; li++) {
        for (int s = 0; s < S; s++) {
            const int64_t cb = ((int64_t)s * layers + li) * L * D;
            const int64_t cc = ((int64_t)s * layers + li) * (Kc - 1) * D;
            memcpy(keys + (int64_t)s * Tk * D, kcache + cb, sizeof(float) * (size_t)L * D);
            memcpy(vals + (int64_t)s * Tk * D, vcache + cb, sizeof(float) * (size_t)L * D);
            memcpy(conv + (int64_t)s * CIN * D, ccache + cc, sizeof(float) * (size_t)(Kc - 1) * D);
        }
        orc_encoder_layer(w + (int64_t)li * W_COUNT, P[li], rel_offset, n_rel, S, T, Tk, D, H, ff, Kc, xa, xb,
                          keys, vals, conv, ranges, vclamp);
        for (int s = 0; s < S; s++) {
            const int64_t cb = ((int64_t)s * layers + li) * L * D;
            const int64_t cc = ((int64_t)s * layers + li) * (Kc - 1) * D;
            memcpy(kcache + cb, keys + ((int64_t)s * Tk + T) * D, sizeof(float) * (size_t)L * D);
            memcpy(vcache + cb, vals + ((int64_t)s * Tk + T) * D, sizeof(float) * (size_t)L * D);
            memcpy(ccache + cc, conv + ((int64_t)s * CIN + T) * D, sizeof(float) * (size_t)(Kc - 1) * D);
        }
        float* t = xa; xa = xb; xb = t;
    }
    memcpy(out, xa, sizeof(float) * M * D);
    for (int s = 0; s < S; s++) cache_len[s] = cache_len[s] + T < L ? cache_len[s] + T : L;
    free(keys); free(vals); free(conv); free(xa); free(xb); free(ranges); free(vclamp);
}

/* FastConformer.swift:346-357 (chunkedLimitedRanges): NeMo chunked_limited [left, right] over T
 * frames; chunks of right+1 frames aligned at frame 0, left/(right+1) chunks back. */
ORC_API void orc_chunked_limited_ranges(int T, int left, int right, int32_t* r) {
    int cs = right + 1, lc = left / cs;
    for (int i = 0; i < T; i++) {
        int c = i / cs;
        int lo = (c - lc) * cs, hi = (c + 1) * cs;
        r[2 * i] = lo > 0 ? lo : 0;
        r[2 * i + 1] = hi < T ? hi : T;
    }
}

/* FastConformer.swift:361-398 (forwardOffline) after the subsampling: all layers over one
 * utterance x [T, D] with the given key ranges (already clipped to valid), zero conv padding and
 * keys = the utterance's own projections.  P tables must cover rel = -(T-1)..(T-1). */
ORC_API void orc_encoder_offline(const float* const* w, const float* const* P, int rel_offset, int n_rel,
                                 int layers, int T, int D, int H, int ff, int Kc, const float* x,
                                 const int32_t* ranges, int valid, float* out) {
    float* keys = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* vals = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* conv = (float*)malloc(sizeof(float) * (size_t)(T + Kc - 1) * D);
    float* xa = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* xb = (float*)malloc(sizeof(float) * (size_t)T * D);
    int32_t v = valid;
    memcpy(xa, x, sizeof(float) * (size_t)T * D);
    for (int li = 0; li < layers; li++) {
        memset(conv, 0, sizeof(float) * (size_t)(T + Kc - 1) * D);
        orc_encoder_layer(w + (int64_t)li * W_COUNT, P[li], rel_offset, n_rel, 1, T, T, D, H, ff, Kc, xa, xb,
                          keys, vals, conv, ranges, &v);
        float* t = xa; xa = xb; xb = t;
    }
    memcpy(out, xa, sizeof(float) * (size_t)T * D);
    free(keys); free(vals); free(conv); free(xa); free(xb);
}

/* ------------------------------------------------------------------ subsampling */

/* Sources/DictatorEngine/Metal/20_conformer.metal:104-138 (conv2d_cl), dispatched by
 * Sources/DictatorEngine/Core/Ops.swift:63-75: channel-last x [Hin, Win, Cin], torch-layout
 * w [Cout, Cin/groups, KH, KW], out [Hout, Wout, Cout].  Input coordinates outside the image read
 * as zero (the padding); output rows h >= valid_h are written as zero. */
ORC_API void orc_conv2d_cl(const float* x, int Hin, int Win, int Cin, const float* w, const float* bias, float* out,
                           int Hout, int Wout, int Cout, int KH, int KW, int stride, int pad_top, int pad_left,
                           int groups, int act, int valid_h) {
    const int cpg = Cin / groups, opg = Cout / groups;
#pragma omp parallel for schedule(static)
    for (int ho = 0; ho < Hout; ho++)
        for (int wo = 0; wo < Wout; wo++)
            for (int co = 0; co < Cout; co++) {
                float* o = out + ((int64_t)ho * Wout + wo) * Cout + co;
                if (ho >= valid_h) { *o = 0.0f; continue; }
                const int g0 = (co / opg) * cpg;
                float acc = bias[co];
                for (int kh = 0; kh < KH; kh++) {
                    const int hi = ho * stride + kh - pad_top;
                    if (hi < 0 || hi >= Hin) continue;
                    for (int kw = 0; kw < KW; kw++) {
                        const int wi = wo * stride + kw - pad_left;
                        if (wi < 0 || wi >= Win) continue;
                        const float* xp = x + ((int64_t)hi * Win + wi) * Cin + g0;
                        const float* wp = w + ((int64_t)co * cpg * KH + kh) * KW + kw;
                        for (int ci = 0; ci < cpg; ci++) acc += wp[(int64_t)ci * KH * KW] * xp[ci];
                    }
                }
                *o = orc_act(acc, act);
            }
}

/* FastConformer.swift:219 (nextLen): causal stride-2 stage, L -> L/2 + 1. */
ORC_API int orc_sub_next_len(int t) { return t / 2 + 1; }

static void orc_mask_rows(float* x, int T, int64_t row_elems, int valid) {
    if (valid < 0) valid = 0;
    if (valid < T) memset(x + (int64_t)valid * row_elems, 0, (size_t)(T - valid) * row_elems * sizeof(float));
}

/* FastConformer.swift:219-243 (encodeSubsampling) with the weight set of :72-95.  mel [T0, F0]
 * (F0 = 128 mel bins), the first valid_mel rows real; C = 256 channels.  sw: conv.0 w/b, conv.2
 * w/b, conv.3 w/b, conv.5 w/b, conv.6 w/b, out.weight [D, C*F3] in the checkpoint's (channel, freq)
 * column order, out.bias -- 12 arrays.  The out weight's columns are permuted to (freq, channel)
 * for the channel-last activations, as the reference does at load (:78-89).  out [T3, D].
 * Returns T3. */
ORC_API int orc_subsample(const float* mel, int T0, int F0, int valid_mel, const float* const* sw, int C, int D,
                          float* out) {
    const int T1 = orc_sub_next_len(T0), F1 = orc_sub_next_len(F0), T2 = orc_sub_next_len(T1),
              F2 = orc_sub_next_len(F1), T3 = orc_sub_next_len(T2), F3 = orc_sub_next_len(F2);
    const int v1 = orc_sub_next_len(valid_mel), v2 = orc_sub_next_len(v1), v3 = orc_sub_next_len(v2);
    float* x0 = (float*)malloc((size_t)T0 * F0 * sizeof(float));
    float* a1 = (float*)malloc((size_t)T1 * F1 * C * sizeof(float));
    float* a2 = (float*)malloc((size_t)T2 * F2 * C * sizeof(float));
    float* a3 = (float*)malloc((size_t)T2 * F2 * C * sizeof(float));
    float* a4 = (float*)malloc((size_t)T3 * F3 * C * sizeof(float));
    float* a5 = (float*)malloc((size_t)T3 * F3 * C * sizeof(float));
    float* wp = (float*)malloc((size_t)D * C * F3 * sizeof(float));
    memcpy(x0, mel, (size_t)T0 * F0 * sizeof(float));
    orc_mask_rows(x0, T0, F0, valid_mel);
    orc_conv2d_cl(x0, T0, F0, 1, sw[0], sw[1], a1, T1, F1, C, 3, 3, 2, 2, 2, 1, ORC_ACT_RELU, v1);
    orc_conv2d_cl(a1, T1, F1, C, sw[2], sw[3], a2, T2, F2, C, 3, 3, 2, 2, 2, C, ORC_ACT_NONE, T2);
    orc_gemm_nt(a2, sw[4], sw[5], NULL, a3, T2 * F2, C, C, 1.0f, ORC_ACT_RELU, 1.0f, 0.0f);
    orc_mask_rows(a3, T2, (int64_t)F2 * C, v2);
    orc_conv2d_cl(a3, T2, F2, C, sw[6], sw[7], a4, T3, F3, C, 3, 3, 2, 2, 2, C, ORC_ACT_NONE, T3);
    orc_gemm_nt(a4, sw[8], sw[9], NULL, a5, T3 * F3, C, C, 1.0f, ORC_ACT_RELU, 1.0f, 0.0f);
    orc_mask_rows(a5, T3, (int64_t)F3 * C, v3);
    for (int o = 0; o < D; o++)
        for (int c = 0; c < C; c++)
            for (int f = 0; f < F3; f++)
                wp[((int64_t)o * F3 + f) * C + c] = sw[10][((int64_t)o * C + c) * F3 + f];
    orc_gemm_nt(a5, wp, sw[11], NULL, out, T3, D, F3 * C, 1.0f, ORC_ACT_NONE, 1.0f, 0.0f);
    free(x0); free(a1); free(a2); free(a3); free(a4); free(a5); free(wp);
    return T3;
}

/* ------------------------------------------------------------------ RNN-T decoder (CPU in the reference) */

/* Weights, Sources/DictatorCore/Decoding/RNNT.swift:27-63: w[0] embed [V, H]; per layer l:
 * w[1+4l] weight_ih [4H, H], w[2+4l] weight_hh [4H, H], w[3+4l] bias_ih, w[4+4l] bias_hh; then
 * joint.pred weight [H, H] and bias, joint.joint_net.2 weight [V, H] and bias.  Gate order i, f, g, o. */
typedef struct {
    const float* const* w;
    int H, V, L;
} OrcRnnt;

static double orc_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

/* RNNT.swift:73-107 (predict): x = embed[token] (zeros for blank), per layer gates = b_ih + b_hh +
 * W_ih x + W_hh h, c' = f c + i g, h' = o tanh(c'), next layer input h'; proj = joint.pred(h_top). */
ORC_API void orc_rnnt_predict(const float* const* w, int H, int V, int L, int token, const float* h, const float* c,
                              float* proj, float* h_out, float* c_out) {
    const int blank = V - 1;
    float* x = (float*)calloc((size_t)H, sizeof(float));
    float* gates = (float*)malloc((size_t)4 * H * sizeof(float));
    if (token != blank) memcpy(x, w[0] + (int64_t)token * H, (size_t)H * sizeof(float));
    for (int l = 0; l < L; l++) {
        const float *wih = w[1 + 4 * l], *whh = w[2 + 4 * l], *bih = w[3 + 4 * l], *bhh = w[4 + 4 * l];
        const float* hl = h + (int64_t)l * H;
        for (int r = 0; r < 4 * H; r++) {
            double a = (double)bih[r] + (double)bhh[r];
            for (int k = 0; k < H; k++) a += (double)wih[(int64_t)r * H + k] * x[k] + (double)whh[(int64_t)r * H + k] * hl[k];
            gates[r] = (float)a;
        }
        for (int j = 0; j < H; j++) {
            const double ig = orc_sigmoid(gates[j]), fg = orc_sigmoid(gates[H + j]), gg = tanh((double)gates[2 * H + j]),
                         og = orc_sigmoid(gates[3 * H + j]);
            const double cn = fg * c[(int64_t)l * H + j] + ig * gg;
            c_out[(int64_t)l * H + j] = (float)cn;
            h_out[(int64_t)l * H + j] = (float)(og * tanh(cn));
        }
        memcpy(x, h_out + (int64_t)l * H, (size_t)H * sizeof(float));
    }
    const float *pw = w[1 + 4 * L], *pb = w[2 + 4 * L];
    for (int j = 0; j < H; j++) {
        double a = pb[j];
        for (int k = 0; k < H; k++) a += (double)pw[(int64_t)j * H + k] * x[k];
        proj[j] = (float)a;
    }
    free(x);
    free(gates);
}

/* RNNT.swift:110-116 (jointLogits) + the argmax of :137-139 (first index of the maximum). */
ORC_API int orc_rnnt_joint_argmax(const float* const* w, int H, int V, int L, const float* enc, const float* pred,
                                  float* logits) {
    const float *ow = w[3 + 4 * L], *ob = w[4 + 4 * L];
    int best = 0;
    for (int v = 0; v < V; v++) {
        double a = ob[v];
        for (int k = 0; k < H; k++) {
            const float hs = enc[k] + pred[k];
            a += (double)ow[(int64_t)v * H + k] * (hs > 0 ? hs : 0.0f);
        }
        logits[v] = (float)a;
        if (logits[v] > logits[best]) best = v;
    }
    return best;
}

/* RNNT.swift:120-151 (greedy) over `frames` projected encoder frames [frames, H].  State
 * (carried across calls): h, c [L, H]; *last_token; *pending with pend_proj [H], pend_h/pend_c
 * [L, H] (the prediction for last_token, committed only when a non-blank token is emitted).
 * Appends up to cap tokens; returns the number appended. */
ORC_API int orc_rnnt_greedy(const float* const* w, int H, int V, int L, const float* enc, int frames, int max_symbols,
                            float* h, float* c, int* last_token, int* pending, float* pend_proj, float* pend_h,
                            float* pend_c, int* tokens, int cap) {
    const int blank = V - 1;
    float* logits = (float*)malloc((size_t)V * sizeof(float));
    int n = 0;
    for (int t = 0; t < frames; t++) {
        int emitted = 0;
        while (emitted < max_symbols) {
            if (!*pending) {
                orc_rnnt_predict(w, H, V, L, *last_token, h, c, pend_proj, pend_h, pend_c);
                *pending = 1;
            }
            const int best = orc_rnnt_joint_argmax(w, H, V, L, enc + (int64_t)t * H, pend_proj, logits);
            if (best == blank) break;
            if (n < cap) tokens[n] = best;
            n++;
            emitted++;
            memcpy(h, pend_h, (size_t)L * H * sizeof(float));
            memcpy(c, pend_c, (size_t)L * H * sizeof(float));
            *last_token = best;
            *pending = 0;
        }
    }
    free(logits);
    return n;
}

/* ------------------------------------------------------------ mel frontend */

enum { ORC_MEL_FFT = 512, ORC_MEL_HOP = 160, ORC_MEL_WIN = 400, ORC_MEL_BINS = 257 };

/* NemoMelFrontend.init (Sources/DictatorCore/Audio/NemoMel.swift:23-40): DFT tables with the
 * window folded in, cos_t/sin_t [257][400]: the 400-sample window sits centred in the 512-point
 * frame (offset 56, torch.stft's zero-padded win_length), phase 2 pi k (n + 56) / 512 in double,
 * entry = float(cos phase) * window[n] and float(-sin phase) * window[n] in float arithmetic. */
ORC_API void orc_mel_tables(const float* window, float* cos_t, float* sin_t) {
    const int off = (ORC_MEL_FFT - ORC_MEL_WIN) / 2;
    for (int k = 0; k < ORC_MEL_BINS; k++)
        for (int n = 0; n < ORC_MEL_WIN; n++) {
            const double phase = 2.0 * 3.14159265358979323846 * (double)k * (double)(n + off) / (double)ORC_MEL_FFT;
            cos_t[k * ORC_MEL_WIN + n] = (float)cos(phase) * window[n];
            sin_t[k * ORC_MEL_WIN + n] = (float)(-sin(phase)) * window[n];
        }
}

/* Mel frames [f0, f0 + nf) of one clip audio[0, n) (NemoMelFrontend.features and
 * NemoMelStream.emit, NemoMel.swift:46-67, 85-107, 141-160): frame t takes the preemphasized
 * samples [160 t - 200, 160 t + 200) -- x[0] = a[0], x[i] = a[i] - 0.97 a[i-1] in float, zero
 * outside [0, n) (the centred STFT's constant padding) -- then re/im against the tables, power
 * |X|^2, mel = fb . power, out = log(mel + 2^-24); frames >= valid_end are written as zeros.
 * The DFT, power and mel sums accumulate in double (a tighter anchor than the reference's fp32
 * sgemm); out [nf][n_mels] float.  fb [n_mels][257]. */
ORC_API void orc_mel_frames(const float* audio, int64_t n, int64_t f0, int32_t nf, int64_t valid_end,
                            const float* cos_t, const float* sin_t, const float* fb, int32_t n_mels, float* out) {
    const double guard = ldexp(1.0, -24);
#pragma omp parallel for schedule(static)
    for (int32_t j = 0; j < nf; j++) {
        const int64_t f = f0 + j;
        float* o = out + (int64_t)j * n_mels;
        if (f >= valid_end) {
            memset(o, 0, (size_t)n_mels * sizeof(float));
            continue;
        }
        float x[ORC_MEL_WIN];
        const int64_t start = f * ORC_MEL_HOP - ORC_MEL_FFT / 2 + (ORC_MEL_FFT - ORC_MEL_WIN) / 2;
        for (int i = 0; i < ORC_MEL_WIN; i++) {
            const int64_t idx = start + i;
            if (idx < 0 || idx >= n) x[i] = 0.0f;
            else if (idx == 0) x[i] = audio[0];
            else {
                const float m = 0.97f * audio[idx - 1];
                x[i] = audio[idx] - m;
            }
        }
        double power[ORC_MEL_BINS];
        for (int k = 0; k < ORC_MEL_BINS; k++) {
            double re = 0.0, im = 0.0;
            const float* c = cos_t + (int64_t)k * ORC_MEL_WIN;
            const float* s = sin_t + (int64_t)k * ORC_MEL_WIN;
            for (int i = 0; i < ORC_MEL_WIN; i++) {
                re += (double)c[i] * (double)x[i];
                im += (double)s[i] * (double)x[i];
            }
            power[k] = re * re + im * im;
        }
        for (int m = 0; m < n_mels; m++) {
            double acc = 0.0;
            const float* w = fb + (int64_t)m * ORC_MEL_BINS;
            for (int k = 0; k < ORC_MEL_BINS; k++) acc += (double)w[k] * power[k];
            o[m] = (float)log(acc + guard);
        }
    }
}
