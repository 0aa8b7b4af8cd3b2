// RNN-T joint and greedy decoding, batched over streams (include/ud_rnnt.h).
//
// The reference decodes one stream at a time on the CPU (Sources/DictatorCore/Decoding/RNNT.swift):
// per emitted token one prediction step (embedding, 2 LSTM layers of [4H, 2H] sgemv, joint.pred)
// and per (frame, symbol) one joint evaluation ([V, H] sgemv).  Here one greedy iteration does
// that work for every active stream of the call at once, as fp32 GEMMs over M = active streams
// (the weights are read once per iteration, not once per stream), with split-K partial slabs that
// the following pointwise kernel sums in a fixed order (deterministic, no atomics):
//
//   predict (streams without a cached prediction):
//     rnnt_embed_kernel        h, c <- cached state for a stream that just emitted (the commit of
//                              RNNT.swift:144-147); xh = [embed(last token) ; h_0]
//     per layer: GEMM xh . [W_ih | W_hh]^T -> slabs;  rnnt_cell_kernel: gates = b + sum(slabs),
//                c' = f c + i g, h' = o tanh(c') -> cached state; xh = [h' ; h_{l+1}]
//     GEMM h_top . W_pred^T -> slabs
//   joint (every remaining frame of every active stream, under its current prediction):
//     rnnt_joint_in_kernel     g = b + sum(slabs) for a stream predicted now (cached), else the
//                              cached g; relu(f_t + g)
//     GEMM . W_out^T -> slabs; rnnt_argmax_kernel: logits = b + sum(slabs), first index of the max,
//                              into mapped host memory
//   commit of a stream that emitted and is not predicted next: rnnt_commit_kernel
//
// The host keeps the greedy control (RNNT.swift:125-151): blank ends a frame, at most
// max_symbols tokens per frame, and the prediction for the last token is cached until a token is
// emitted (so frames that end in blank do not rerun the LSTM).  Because a blank leaves the
// prediction unchanged, the joint results of the frames after a blank are known in advance: one
// iteration evaluates them all and the host consumes them up to the first emission.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ud_rnnt.h"
#include "kernels.hpp"
#include "ud_common.hpp"

int ud_set_error(int code, const char* msg);   // encoder.hip

namespace ud {

constexpr int RNNT_KS = 4;          // K splits of the decoder GEMMs

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// xh[b] = [x ; h[slot][0]] with x = embed[tok] (zeros for blank, NeMo's padding row).  A slot
// whose token was just emitted (commit[b]) first takes its cached state: h, c <- ph, pc over all
// layers (RNNT.swift:144-147), and its row reads h from ph (the same values).
__global__ void rnnt_embed_kernel(const float* __restrict__ embed, const int32_t* __restrict__ slot,
                                  const int32_t* __restrict__ tok, const int32_t* __restrict__ commit,
                                  const float* __restrict__ ph, const float* __restrict__ pc, float* __restrict__ h,
                                  float* __restrict__ c, float* __restrict__ xh, int H, int L, int blank) {
    const int b = blockIdx.x, s = slot[b], t = tok[b];
    const bool cm = commit[b] != 0;
    const int64_t o = (int64_t)s * L * H;
    if (cm)
        for (int j = threadIdx.x; j < L * H; j += blockDim.x) {
            h[o + j] = ph[o + j];
            c[o + j] = pc[o + j];
        }
    const float* hr = (cm ? ph : h) + o;
    for (int j = threadIdx.x; j < H; j += blockDim.x) {
        xh[(int64_t)b * 2 * H + j] = t == blank ? 0.0f : embed[(int64_t)t * H + j];
        xh[(int64_t)b * 2 * H + H + j] = hr[j];
    }
}

// One LSTM layer's cell from the gate slabs [ks][n][4H]; writes the cached state of the slot and
// the next layer's input row.
__global__ void rnnt_cell_kernel(const float* __restrict__ slabs, int ks, int n, const float* __restrict__ bias,
                                 const float* __restrict__ h, const float* __restrict__ c, float* __restrict__ ph,
                                 float* __restrict__ pc, float* __restrict__ xh, const int32_t* __restrict__ slot,
                                 int H, int L, int layer) {
    const int b = blockIdx.x, s = slot[b];
    const int64_t G = 4 * (int64_t)H;
    {
        const int j = blockIdx.y * blockDim.x + threadIdx.x;
        if (j >= H) return;
        float g[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float v = bias[q * H + j];
            for (int z = 0; z < ks; z++) v += slabs[((int64_t)z * n + b) * G + q * H + j];
            g[q] = v;
        }
        const float ig = sigmoid_f(g[0]), fg = sigmoid_f(g[1]), gg = tanhf(g[2]), og = sigmoid_f(g[3]);
        const int64_t si = ((int64_t)s * L + layer) * H + j;
        const float cn = fg * c[si] + ig * gg;
        const float hn = og * tanhf(cn);
        pc[si] = cn;
        ph[si] = hn;
        xh[(int64_t)b * 2 * H + j] = hn;
        if (layer + 1 < L) xh[(int64_t)b * 2 * H + H + j] = h[((int64_t)s * L + layer + 1) * H + j];
    }
}

// out[slot(b)] (or out[b] when slot is null) = bias + sum of the slabs [ks][n][N].
__global__ void rnnt_sum_kernel(const float* __restrict__ slabs, int ks, int n, const float* __restrict__ bias,
                                float* __restrict__ out, const int32_t* __restrict__ slot, int N) {
    const int b = blockIdx.x;
    const int64_t o = (int64_t)(slot ? slot[b] : b) * N;
    {
        const int j = blockIdx.y * blockDim.x + threadIdx.x;
        if (j >= N) return;
        float v = bias[j];
        for (int z = 0; z < ks; z++) v += slabs[((int64_t)z * n + b) * N + j];
        out[o + j] = v;
    }
}

// hsum[b] = relu(f[erow(b)] + g) with g the slot's prediction: for a slot predicted in this
// iteration (prow[b] >= 0, its row in the prediction slabs [ks][npred][H]) bias + the sum of its
// slabs, which the slot's first row (first[b]) also caches in gc[slot]; otherwise the cached
// gc[slot(b)].
__global__ void rnnt_joint_in_kernel(const float* __restrict__ f, const int32_t* __restrict__ erow,
                                     float* __restrict__ gc, const int32_t* __restrict__ slot,
                                     const int32_t* __restrict__ prow, const int32_t* __restrict__ first,
                                     const float* __restrict__ slabs, int ks, int npred,
                                     const float* __restrict__ bias, float* __restrict__ hsum, int H) {
    const int b = blockIdx.x, r = prow[b];
    const bool st = r >= 0 && first[b] != 0;
    const float* fr = f + (int64_t)erow[b] * H;
    float* gr = gc + (int64_t)slot[b] * H;
    for (int j = threadIdx.x; j < H; j += blockDim.x) {
        float g;
        if (r >= 0) {
            g = bias[j];
            for (int z = 0; z < ks; z++) g += slabs[((int64_t)z * npred + r) * H + j];
            if (st) gr[j] = g;
        } else {
            g = gr[j];
        }
        const float v = fr[j] + g;
        hsum[(int64_t)b * H + j] = v > 0.0f ? v : 0.0f;
    }
}

// best[b] = the first index of the maximum of bias + sum of the slabs [ks][n][V].
__global__ __launch_bounds__(256) void rnnt_argmax_kernel(const float* __restrict__ slabs, int ks, int n,
                                                          const float* __restrict__ bias, int32_t* __restrict__ best,
                                                          int V) {
    const int b = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v = threadIdx.x; v < V; v += blockDim.x) {
        float x = bias[v];
        for (int z = 0; z < ks; z++) x += slabs[((int64_t)z * n + b) * V + v];
        if (x > bv) { bv = x; bi = v; }        // ascending v per thread: keeps the first maximum
    }
    __shared__ float sv[256];
    __shared__ int si[256];
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) {
            const float ov = sv[threadIdx.x + w];
            const int oi = si[threadIdx.x + w];
            if (ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) best[b] = si[0];
}

// h, c of slot(b) <- the cached state (RNNT.swift:144-147).
__global__ void rnnt_commit_kernel(const float* __restrict__ ph, const float* __restrict__ pc, float* __restrict__ h,
                                   float* __restrict__ c, const int32_t* __restrict__ slot, int LH) {
    const int64_t o = (int64_t)slot[blockIdx.x] * LH;
    for (int j = threadIdx.x; j < LH; j += blockDim.x) {
        h[o + j] = ph[o + j];
        c[o + j] = pc[o + j];
    }
}

}  // namespace ud

using namespace ud;

static int rfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return ud_set_error(code, buf);
}

#define RHIPC(call)                                                                              \
    do {                                                                                         \
        hipError_t e_ = (call);                                                                  \
        if (e_ != hipSuccess) return rfail(UD_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_));  \
    } while (0)
#define RLAUNCH(what)                                                                            \
    do {                                                                                         \
        hipError_t e_ = hipGetLastError();                                                       \
        if (e_ != hipSuccess) return rfail(UD_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e_)); \
    } while (0)

enum RSlot { R_EMBED, R_PRED_W, R_PRED_B, R_OUT_W, R_OUT_B, R_ENC_W, R_ENC_B, R_FIXED };

struct ud_rnnt {
    int H, V, L, E, S, max_sym;
    float* w[R_FIXED] = {};
    std::vector<float*> wcat, bias;             // per layer [4H][2H] = [W_ih | W_hh], b_ih + b_hh
    std::vector<std::vector<float>> ih, hh, bih, bhh;   // host copies until both halves are set
    uint32_t set_fixed = 0;
    std::vector<uint32_t> set_layer;            // bit 0..3: weight_ih, weight_hh, bias_ih, bias_hh
    // per-slot state: committed h, c [S][L][H]; cached prediction ph, pc [S][L][H], pg [S][H]
    float *h = nullptr, *c = nullptr, *ph = nullptr, *pc = nullptr, *pg = nullptr;
    std::vector<int> last, pending;
    // workspace of the prediction network (rows = slots, at most S)
    float *xh = nullptr, *slabs = nullptr;
    // workspace of the joint: one row per (stream, frame) pair, grown to the largest call
    float *hsum = nullptr, *jslabs = nullptr;
    int cap_pairs = 0;
    // split-K slabs of ud_rnnt_project, grown to the largest call
    float* pslabs = nullptr;
    int cap_proj = 0;
    // A greedy iteration's lists, packed and uploaded in one copy from a pinned mirror: [slots to
    // commit alone][slots to predict][their last tokens][their commit flags][joint rows' slots]
    // [joint rows' proj rows][joint rows' prediction rows][joint rows' first-of-slot flags],
    // 4 S + 4 cap_pairs entries.  The host rewrites the mirror only after the iteration's
    // synchronize, when the previous copy from it is done.
    int32_t *dlist = nullptr, *hlist = nullptr;
    // the joint's argmax per row: pinned, mapped host memory the argmax kernel writes (dbest is its
    // device address), read after the iteration's synchronize
    int32_t *hbest = nullptr, *dbest = nullptr;
    // Work order across HIP streams (the calls share the workspaces above): every call that
    // enqueues device work records done_ev on its stream at its end, and a call on a different
    // stream first makes its stream wait for done_ev, so calls run in call order.
    hipEvent_t done_ev = nullptr;
    hipStream_t last_st = nullptr;
    bool has_last = false;
};

static float* ralloc(size_t floats) {
    void* p = nullptr;
    if (hipMalloc(&p, floats ? floats * 4 : 16) != hipSuccess) return nullptr;
    return static_cast<float*>(p);
}

static void free_rnnt(ud_rnnt* r) {
    if (!r) return;
    (void)hipDeviceSynchronize();
    for (float* p : r->w) if (p) (void)hipFree(p);
    for (float* p : r->wcat) if (p) (void)hipFree(p);
    for (float* p : r->bias) if (p) (void)hipFree(p);
    void* ps[] = {r->h, r->c, r->ph, r->pc, r->pg, r->xh, r->slabs, r->hsum, r->jslabs, r->pslabs, r->dlist};
    for (void* p : ps) if (p) (void)hipFree(p);
    for (void* p : {(void*)r->hlist, (void*)r->hbest})
        if (p) (void)hipHostFree(p);
    if (r->done_ev) (void)hipEventDestroy(r->done_ev);
    delete r;
}

extern "C" UD_API int ud_rnnt_create(int32_t hidden, int32_t vocab, int32_t layers, int32_t enc_dim,
                                     int32_t max_streams, int32_t max_symbols_per_frame, ud_rnnt** out) {
    if (!out) return rfail(UD_ERR_INVALID, "ud_rnnt_create: null out pointer");
    *out = nullptr;
    if (hidden < 1 || vocab < 2 || layers < 1 || layers > 8 || enc_dim < 1 || max_streams < 1 || max_symbols_per_frame < 1)
        return rfail(UD_ERR_SHAPE, "ud_rnnt_create: bad dimensions");
    if (hidden % 64 != 0 || enc_dim % 16 != 0)
        return rfail(UD_ERR_SHAPE, "ud_rnnt_create: hidden %d must be a multiple of 64 and enc_dim %d of 16", hidden, enc_dim);
    ud_rnnt* r = new ud_rnnt();
    r->H = hidden; r->V = vocab; r->L = layers; r->E = enc_dim; r->S = max_streams; r->max_sym = max_symbols_per_frame;
    const size_t H = hidden, V = vocab, L = layers, S = max_streams;
    r->wcat.assign(L, nullptr);
    r->bias.assign(L, nullptr);
    r->ih.resize(L); r->hh.resize(L); r->bih.resize(L); r->bhh.resize(L);
    r->set_layer.assign(L, 0);
    const size_t gmax = 4 * H > V ? 4 * H : V;
    bool ok = (r->h = ralloc(S * L * H)) && (r->c = ralloc(S * L * H)) && (r->ph = ralloc(S * L * H)) &&
              (r->pc = ralloc(S * L * H)) && (r->pg = ralloc(S * H)) && (r->xh = ralloc(S * 2 * H)) &&
              (r->slabs = ralloc((size_t)RNNT_KS * S * gmax)) &&
              hipEventCreateWithFlags(&r->done_ev, hipEventDisableTiming) == hipSuccess;
    if (!ok || hipMemset(r->h, 0, S * L * H * 4) != hipSuccess || hipMemset(r->c, 0, S * L * H * 4) != hipSuccess) {
        free_rnnt(r);
        return rfail(UD_ERR_NOMEM, "ud_rnnt_create: device allocation failed");
    }
    r->last.assign(S, vocab - 1);
    r->pending.assign(S, 0);
    *out = r;
    return UD_OK;
}

extern "C" UD_API void ud_rnnt_destroy(ud_rnnt* r) { free_rnnt(r); }

static int rupload(float*& dst, const float* src, size_t n) {
    if (!dst && !(dst = ralloc(n))) return rfail(UD_ERR_NOMEM, "ud_rnnt_set_weight: allocation failed");
    RHIPC(hipMemcpy(dst, src, n * 4, hipMemcpyHostToDevice));
    return UD_OK;
}

extern "C" UD_API int ud_rnnt_get_info(const ud_rnnt* r, int32_t* hidden, int32_t* vocab, int32_t* layers,
                                       int32_t* enc_dim, int32_t* max_streams, int32_t* max_symbols_per_frame) {
    if (!r) return rfail(UD_ERR_INVALID, "ud_rnnt_get_info: null decoder");
    if (hidden) *hidden = r->H;
    if (vocab) *vocab = r->V;
    if (layers) *layers = r->L;
    if (enc_dim) *enc_dim = r->E;
    if (max_streams) *max_streams = r->S;
    if (max_symbols_per_frame) *max_symbols_per_frame = r->max_sym;
    return UD_OK;
}

extern "C" UD_API int ud_rnnt_set_weight(ud_rnnt* r, const char* name, const float* host, int64_t count) {
    if (!r || !name || !host) return rfail(UD_ERR_INVALID, "ud_rnnt_set_weight: null argument");
    const int64_t H = r->H, V = r->V, E = r->E;
    struct Fixed { const char* n; int slot; int64_t count; };
    const Fixed fixed[] = {{"decoder.prediction.embed.weight", R_EMBED, V * H}, {"joint.pred.weight", R_PRED_W, H * H},
                           {"joint.pred.bias", R_PRED_B, H}, {"joint.joint_net.2.weight", R_OUT_W, V * H},
                           {"joint.joint_net.2.bias", R_OUT_B, V}, {"joint.enc.weight", R_ENC_W, H * E},
                           {"joint.enc.bias", R_ENC_B, H}};
    for (const Fixed& f : fixed) {
        if (strcmp(name, f.n) != 0) continue;
        if (count != f.count)
            return rfail(UD_ERR_WEIGHT, "weight '%s': %lld values, expected %lld", name, (long long)count, (long long)f.count);
        int rc = rupload(r->w[f.slot], host, (size_t)count);
        if (rc == UD_OK) r->set_fixed |= 1u << f.slot;
        return rc;
    }
    const char* pre = "decoder.prediction.dec_rnn.lstm.";
    if (strncmp(name, pre, strlen(pre)) == 0) {
        const char* p = name + strlen(pre);
        const char* kinds[4] = {"weight_ih_l", "weight_hh_l", "bias_ih_l", "bias_hh_l"};
        for (int k = 0; k < 4; k++) {
            const size_t kl = strlen(kinds[k]);
            if (strncmp(p, kinds[k], kl) != 0) continue;
            char* end = nullptr;
            const long l = strtol(p + kl, &end, 10);
            if (end == p + kl || *end != '\0' || l < 0 || l >= r->L) break;
            const int64_t want = k < 2 ? 4 * H * H : 4 * H;
            if (count != want)
                return rfail(UD_ERR_WEIGHT, "weight '%s': %lld values, expected %lld", name, (long long)count, (long long)want);
            std::vector<float>& dst = k == 0 ? r->ih[l] : k == 1 ? r->hh[l] : k == 2 ? r->bih[l] : r->bhh[l];
            dst.assign(host, host + count);
            r->set_layer[l] |= 1u << k;
            int rc = UD_OK;
            if ((r->set_layer[l] & 3u) == 3u) {     // both matrices: [4H][2H] = [W_ih | W_hh]
                std::vector<float> cat((size_t)4 * H * 2 * H);
                for (int64_t row = 0; row < 4 * H; row++) {
                    memcpy(&cat[(size_t)row * 2 * H], &r->ih[l][(size_t)row * H], (size_t)H * 4);
                    memcpy(&cat[(size_t)row * 2 * H + H], &r->hh[l][(size_t)row * H], (size_t)H * 4);
                }
                rc = rupload(r->wcat[l], cat.data(), cat.size());
            }
            if (rc == UD_OK && (r->set_layer[l] & 12u) == 12u) {
                std::vector<float> b((size_t)4 * H);
                for (int64_t i = 0; i < 4 * H; i++) b[i] = r->bih[l][i] + r->bhh[l][i];
                rc = rupload(r->bias[l], b.data(), b.size());
            }
            return rc;
        }
    }
    return rfail(UD_ERR_WEIGHT, "unknown RNN-T weight name '%s'", name);
}

static int check_weights(const ud_rnnt* r, const char* who) {
    if (r->set_fixed != (1u << R_FIXED) - 1) return rfail(UD_ERR_STATE, "%s: joint / embedding weights not all set", who);
    for (int l = 0; l < r->L; l++)
        if (r->set_layer[l] != 15u) return rfail(UD_ERR_STATE, "%s: LSTM layer %d weights not all set", who, l);
    return UD_OK;
}

extern "C" UD_API int ud_rnnt_reset(ud_rnnt* r, int32_t slot) {
    if (!r) return rfail(UD_ERR_INVALID, "ud_rnnt_reset: null decoder");
    if (slot < 0 || slot >= r->S) return rfail(UD_ERR_SHAPE, "ud_rnnt_reset: slot %d outside 0..%d", slot, r->S - 1);
    const size_t LH = (size_t)r->L * r->H;
    RHIPC(hipMemset(r->h + slot * LH, 0, LH * 4));
    RHIPC(hipMemset(r->c + slot * LH, 0, LH * 4));
    r->last[slot] = r->V - 1;
    r->pending[slot] = 0;
    return UD_OK;
}

// The start of a call that enqueues device work on `st`: after every earlier call's work.
static int order_after_last(ud_rnnt* r, hipStream_t st) {
    if (r->has_last && st != r->last_st) RHIPC(hipStreamWaitEvent(st, r->done_ev, 0));
    return UD_OK;
}
// The end of such a call: done_ev marks the end of its work.
static int mark_done(ud_rnnt* r, hipStream_t st) {
    RHIPC(hipEventRecord(r->done_ev, st));
    r->last_st = st;
    r->has_last = true;
    return UD_OK;
}

// C[n, N] slabs = A[n, K] (row stride lda) . W[N, K]^T, RNNT_KS K splits, fp32.
static int slab_gemm(float* slabs, const float* A, int lda, const float* W, int n, int N, int K, hipStream_t st,
                     int ks = RNNT_KS) {
    GemmArgs g{};
    g.A = A; g.W = W; g.C = slabs; g.M = n; g.N = N; g.K = K; g.lda = lda; g.ldw = K; g.ldc = N;
    g.epi = EPI_PARTIAL; g.act = ACT_NONE; g.out_scale = 1.0f; g.ksplit = ks;
    const int rc = launch_gemm_f32_small(g, ks, st);
    if (rc != 0) return rfail(rc == -2 ? UD_ERR_SHAPE : UD_ERR_HIP, "rnnt GEMM launch failed (%d x %d x %d)", n, N, K);
    return UD_OK;
}

extern "C" UD_API int ud_rnnt_project(ud_rnnt* r, int32_t rows, const float* enc_dev, float* out_dev, void* hip_stream) {
    if (!r || !enc_dev || !out_dev) return rfail(UD_ERR_INVALID, "ud_rnnt_project: null argument");
    if (!(r->set_fixed & (1u << R_ENC_W)) || !(r->set_fixed & (1u << R_ENC_B)))
        return rfail(UD_ERR_STATE, "ud_rnnt_project: joint.enc weights not set");
    if (rows < 1) return rfail(UD_ERR_SHAPE, "ud_rnnt_project: rows must be >= 1");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    int rc0 = order_after_last(r, st);
    if (rc0 != UD_OK) return rc0;
    if (rows > r->cap_proj) {
        // grown between calls only: st now follows every earlier call's work, so a synchronize
        // covers the previous call's use of the old buffer
        RHIPC(hipStreamSynchronize(st));
        if (r->pslabs) (void)hipFree(r->pslabs);
        r->cap_proj = 0;
        if (!(r->pslabs = ralloc((size_t)RNNT_KS * rows * r->H)))
            return rfail(UD_ERR_NOMEM, "ud_rnnt_project: workspace allocation failed (%d rows)", rows);
        r->cap_proj = rows;
    }
    const int ks = r->E % (16 * RNNT_KS) == 0 ? RNNT_KS : 1;
    int rc = slab_gemm(r->pslabs, enc_dev, r->E, r->w[R_ENC_W], rows, r->H, r->E, st, ks);
    if (rc != UD_OK) return rc;
    hipLaunchKernelGGL(rnnt_sum_kernel, dim3(rows, (r->H + 63) / 64), dim3(64), 0, st, r->pslabs, ks, rows,
                       r->w[R_ENC_B], out_dev, (const int32_t*)nullptr, r->H);
    RLAUNCH("ud_rnnt_project sum");
    return mark_done(r, st);
}

// The prediction network for rows (slots) without a cached prediction.
// dslots: the slots on the device, then their last tokens, then their commit flags (uploaded with
// the iteration's lists).  Leaves the joint.pred projection as split-K slabs in r->slabs; the
// joint input kernel adds them (and caches the sum).
static int predict(ud_rnnt* r, const std::vector<int>& slots, const int32_t* dslots, hipStream_t st) {
    const int n = (int)slots.size(), H = r->H, L = r->L;
    hipLaunchKernelGGL(rnnt_embed_kernel, dim3(n), dim3(256), 0, st, r->w[R_EMBED], dslots, dslots + n, dslots + 2 * n,
                       r->ph, r->pc, r->h, r->c, r->xh, H, L, r->V - 1);
    RLAUNCH("rnnt embed");
    for (int l = 0; l < L; l++) {
        int rc = slab_gemm(r->slabs, r->xh, 2 * H, r->wcat[l], n, 4 * H, 2 * H, st);
        if (rc != UD_OK) return rc;
        hipLaunchKernelGGL(rnnt_cell_kernel, dim3(n, (H + 63) / 64), dim3(64), 0, st, r->slabs, RNNT_KS, n, r->bias[l], r->h, r->c,
                           r->ph, r->pc, r->xh, dslots, H, L, l);
        RLAUNCH("rnnt cell");
    }
    int rc = slab_gemm(r->slabs, r->xh, 2 * H, r->w[R_PRED_W], n, H, H, st);
    if (rc != UD_OK) return rc;
    for (int s : slots) r->pending[s] = 1;
    return UD_OK;
}

// Grows the joint's pair workspace to P rows.  Called between greedy calls only (every call ends
// with a stream synchronize), so nothing in flight uses the old buffers.
static int ensure_pairs(ud_rnnt* r, int P) {
    if (P <= r->cap_pairs) return UD_OK;
    void* ds[] = {r->hsum, r->jslabs, r->dlist};
    for (void* p : ds) if (p) (void)hipFree(p);
    for (void* p : {(void*)r->hlist, (void*)r->hbest}) if (p) (void)hipHostFree(p);
    r->hsum = r->jslabs = nullptr;
    r->dlist = r->hlist = r->hbest = r->dbest = nullptr;
    r->cap_pairs = 0;
    const size_t n = (size_t)P, nl = 4 * (size_t)r->S + 4 * n;
    bool ok = (r->hsum = ralloc(n * r->H)) && (r->jslabs = ralloc((size_t)RNNT_KS * n * r->V)) &&
              (r->dlist = (int32_t*)ralloc(nl)) && hipHostMalloc((void**)&r->hlist, nl * 4) == hipSuccess &&
              hipHostMalloc((void**)&r->hbest, n * 4, hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess &&
              hipHostGetDevicePointer((void**)&r->dbest, r->hbest, 0) == hipSuccess;
    if (!ok) return rfail(UD_ERR_NOMEM, "ud_rnnt_greedy: joint workspace allocation failed (%d pairs)", P);
    r->cap_pairs = P;
    return UD_OK;
}

// Greedy decoding with speculative frames.  The sequential rule (RNNT.swift:125-151) evaluates the
// joint at (frame t, current prediction); a blank moves to t + 1 with the prediction unchanged.  So
// for each active stream one iteration evaluates the joint at EVERY remaining frame of the call
// (up to RNNT_SPEC of them) under the current prediction, and the host walks the results: leading
// blanks advance the frame, the first non-blank is emitted (its frame's symbol count continues
// from the previous emissions there), and later results of that stream are discarded because the
// prediction changes.  Every decision is the one the sequential loop makes; a chunk whose frames
// are all blank costs one iteration instead of one per frame.
constexpr int RNNT_SPEC = 16;

extern "C" UD_API int ud_rnnt_greedy(ud_rnnt* r, int32_t n, const int32_t* slots_host, const float* proj_dev,
                                     int32_t rows_per_stream, const int32_t* frames_host, int32_t* tokens_host,
                                     int32_t cap, int32_t* n_tokens_host, void* hip_stream) {
    if (!r || !slots_host || !proj_dev || !frames_host || !n_tokens_host || (cap > 0 && !tokens_host))
        return rfail(UD_ERR_INVALID, "ud_rnnt_greedy: null argument");
    int rc = check_weights(r, "ud_rnnt_greedy");
    if (rc != UD_OK) return rc;
    if (n < 1 || n > r->S) return rfail(UD_ERR_SHAPE, "ud_rnnt_greedy: n = %d outside 1..%d", n, r->S);
    std::vector<char> seen(r->S, 0);
    int max_frames = 0;
    for (int b = 0; b < n; b++) {
        const int s = slots_host[b];
        if (s < 0 || s >= r->S || seen[s]) return rfail(UD_ERR_INVALID, "ud_rnnt_greedy: bad or repeated slot %d", s);
        seen[s] = 1;
        if (frames_host[b] < 0 || frames_host[b] > rows_per_stream)
            return rfail(UD_ERR_SHAPE, "ud_rnnt_greedy: frames %d outside 0..%d", frames_host[b], rows_per_stream);
        if (frames_host[b] > max_frames) max_frames = frames_host[b];
        n_tokens_host[b] = 0;
    }
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if ((rc = order_after_last(r, st)) != UD_OK) return rc;
    if ((rc = ensure_pairs(r, n * std::min(max_frames, RNNT_SPEC))) != UD_OK) return rc;
    const int H = r->H, V = r->V, blank = V - 1;
    std::vector<int> act, t(n, 0), em(n, 0), pred_slots, commit, rest, p0(n), p1(n), prow_of(r->S, -1);
    std::vector<char> to_commit(r->S, 0);
    int32_t* hl = r->hlist;
    // the commits of the previous iteration's emissions go up with the next lists: a slot predicted
    // in that iteration takes its state in the embedding kernel, the others in the commit kernel
    // (alone at the end)
    auto launch_commit = [&](const std::vector<int>& slots, int oc) -> int {
        if (slots.empty()) return UD_OK;
        hipLaunchKernelGGL(rnnt_commit_kernel, dim3((unsigned)slots.size()), dim3(256), 0, st, r->ph, r->pc, r->h, r->c,
                           r->dlist + oc, r->L * H);
        RLAUNCH("rnnt commit");
        return UD_OK;
    };
    for (;;) {
        act.clear();
        for (int b = 0; b < n; b++)
            if (t[b] < frames_host[b]) act.push_back(b);
        if (act.empty()) break;
        pred_slots.clear();
        for (int b : act)
            if (!r->pending[slots_host[b]]) pred_slots.push_back(slots_host[b]);
        for (int s : commit) to_commit[s] = 1;
        int m = 0;
        for (int b : act) {
            p0[b] = m;
            m += std::min(frames_host[b], t[b] + RNNT_SPEC) - t[b];
            p1[b] = m;
        }
        // one upload: commits, predictions (slots, last tokens, commit flags), joint rows (slots,
        // proj rows, prediction rows, first-of-slot flags)
        int off = 0;
        const int np = (int)pred_slots.size();
        const int op = off;
        for (int s : pred_slots) hl[off++] = s;
        for (int s : pred_slots) hl[off++] = r->last[s];
        for (int i = 0; i < np; i++) {
            const int s = pred_slots[i];
            hl[off++] = to_commit[s];
            to_commit[s] = 0;
            prow_of[s] = i;
        }
        rest.clear();
        for (int s : commit)
            if (to_commit[s]) { rest.push_back(s); to_commit[s] = 0; }
        commit.clear();
        const int oc = off;
        for (int s : rest) hl[off++] = s;
        const int oq = off;
        for (int b : act)
            for (int p = p0[b]; p < p1[b]; p++) {
                const int s = slots_host[b];
                hl[oq + p] = s;
                hl[oq + m + p] = b * rows_per_stream + t[b] + (p - p0[b]);
                hl[oq + 2 * m + p] = prow_of[s];
                hl[oq + 3 * m + p] = p == p0[b] ? 1 : 0;
            }
        off = oq + 4 * m;
        for (int s : pred_slots) prow_of[s] = -1;
        RHIPC(hipMemcpyAsync(r->dlist, hl, (size_t)off * 4, hipMemcpyHostToDevice, st));
        if ((rc = launch_commit(rest, oc)) != UD_OK) return rc;
        if (np && (rc = predict(r, pred_slots, r->dlist + op, st)) != UD_OK) return rc;
        const int32_t* dq = r->dlist + oq;
        hipLaunchKernelGGL(rnnt_joint_in_kernel, dim3(m), dim3(256), 0, st, proj_dev, dq + m, r->pg, dq, dq + 2 * m,
                           dq + 3 * m, r->slabs, RNNT_KS, np, r->w[R_PRED_B], r->hsum, H);
        RLAUNCH("rnnt joint input");
        if ((rc = slab_gemm(r->jslabs, r->hsum, H, r->w[R_OUT_W], m, V, H, st)) != UD_OK) return rc;
        hipLaunchKernelGGL(rnnt_argmax_kernel, dim3(m), dim3(256), 0, st, r->jslabs, RNNT_KS, m, r->w[R_OUT_B], r->dbest, V);
        RLAUNCH("rnnt argmax");
        RHIPC(hipStreamSynchronize(st));
        for (int b : act) {
            const int s = slots_host[b];
            for (int p = p0[b]; p < p1[b]; p++) {
                const int tt = t[b], k = r->hbest[p];
                if (k == blank || k < 0 || k >= V) {   // (out of range only for NaN logits)
                    t[b] = tt + 1;
                    em[b] = 0;
                    continue;
                }
                if (n_tokens_host[b] < cap) tokens_host[(int64_t)b * cap + n_tokens_host[b]] = k;
                n_tokens_host[b]++;
                r->last[s] = k;
                r->pending[s] = 0;
                commit.push_back(s);
                if (++em[b] >= r->max_sym) {
                    t[b] = tt + 1;
                    em[b] = 0;
                }
                break;
            }
        }
    }
    if (!commit.empty()) {
        for (size_t i = 0; i < commit.size(); i++) hl[i] = commit[i];
        RHIPC(hipMemcpyAsync(r->dlist, hl, commit.size() * 4, hipMemcpyHostToDevice, st));
        if ((rc = launch_commit(commit, 0)) != UD_OK) return rc;
    }
    RHIPC(hipStreamSynchronize(st));
    return mark_done(r, st);
}
