// Host layer and C ABI of the gfx950 streaming encoder step (include/ud_encoder.h).
//
// Mirrors FastConformerEncoder + StreamState + encodeStreamStep
// (Sources/DictatorEngine/Models/FastConformer.swift:62-480) for a batch of streams:
//  - one encoder owns device weights, per-layer position tables, a step workspace sized for
//    max_streams x max_chunk rows and a pool of per-stream caches; a 16-bit (UD_BF16) encoder
//    holds bf16-valued weights as IEEE half and computes on the f16 MFMA with half activations,
//    K/V caches and tables (fp32 accumulation, fp32 residual stream, norms and conv cache), an
//    fp32 encoder keeps everything in fp32;
//  - caches are rings updated in place (no ping-pong copies): the K/V rings hold L + max_chunk
//    rows, the QKV projection writes a step's new K/V rows into them and the attention reads its
//    window from them; the conv ring is updated by the conv kernel.  A stream's ring positions
//    derive from its frame counter, so the host carries one integer per stream and uploads a
//    small descriptor {slot, window start, valid, cache_len, conv origin} per step;
//  - the 24-layer kernel sequence of a step is captured once per (batch size, T, input, output)
//    into a hipGraph and replayed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/ud_encoder.h"
#include "kernels.hpp"

using namespace ud;

// ---------------------------------------------------------------- errors

static thread_local std::string g_err;

static int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIPC(call)                                                                               \
    do {                                                                                         \
        hipError_t e_ = (call);                                                                  \
        if (e_ != hipSuccess) return fail(UD_ERR_HIP, "%s: %s (%s:%d)", #call, hipGetErrorString(e_), \
                                          __FILE__, __LINE__);                                   \
    } while (0)

static int launch_status(int rc, const char* what) {
    if (rc == 0) return UD_OK;
    if (rc == -2) return fail(UD_ERR_SHAPE, "%s: shape not supported by the kernel", what);
    return fail(UD_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(hipGetLastError()));
}
#define LAUNCH(expr, what)                                  \
    do {                                                    \
        int r_ = launch_status((expr), what);               \
        if (r_ != UD_OK) return r_;                         \
    } while (0)

extern "C" UD_API const char* ud_last_error(void) { return g_err.c_str(); }

int ud_set_error(int code, const char* msg) {
    g_err = msg;
    return code;
}

// ---------------------------------------------------------------- bf16 host conversion

// Round-to-nearest-even, NaN -> 0x7FC0 (Sources/DictatorEngine/Core/Tensor.swift:116-122).
static inline uint16_t host_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static inline float host_bf16_to_f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static constexpr float kHalfMax = 65504.0f;
// IEEE half (round to nearest even), saturating at +-65504 (NaN stays NaN), as the device stores
// saturate: a 16-bit encoder's storage format for activations, K/V caches and position tables.
static inline uint16_t host_f16(float f) {
    if (!std::isnan(f)) f = f < -kHalfMax ? -kHalfMax : (f > kHalfMax ? kHalfMax : f);
    const _Float16 h = (_Float16)f;
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}
static inline float host_f16_to_f(uint16_t b) {
    _Float16 h;
    memcpy(&h, &b, 2);
    return (float)h;
}
// A linear weight of a 16-bit encoder, held as IEEE half for the f16 MFMA:
//  - UD_BF16: its bf16 value (round to nearest even, Tensor.swift:116-122), exact in half for every
//    bf16 value of magnitude 2^-17 .. 65504 (half's 11-bit significand holds bf16's 8 bits);
//    smaller magnitudes keep half's subnormal resolution, 2^-24;
//  - UD_F16: fp32 rounded straight to half, as WeightConverter.convert(.f16) writes the reference's
//    f16 checkpoint (Sources/DictatorEngine/Core/Convert.swift:99-104, Float16(x)).
// Callers check the range first (a weight beyond 65504 is refused, not saturated).
static inline uint16_t host_weight16(float f, bool f16_weights) {
    return f16_weights ? host_f16(f) : host_f16(host_bf16_to_f(host_bf16(f)));
}
static inline float host_weight16_value(float f, bool f16_weights) {
    return f16_weights ? host_f16_to_f(host_f16(f)) : host_bf16_to_f(host_bf16(f));
}

// ---------------------------------------------------------------- weights

// The 26 tensors of one layer (docs/specs/nemotron.md tensor-name map; loading at
// FastConformer.swift:96-143).
enum WSlot {
    NORM_FF1_W, NORM_FF1_B, FF1_W1, FF1_W2, NORM_ATT_W, NORM_ATT_B, LIN_Q, LIN_K, LIN_V, LIN_OUT, LIN_POS,
    BIAS_U, BIAS_V, NORM_CONV_W, NORM_CONV_B, PW1, DW, CONV_LN_W, CONV_LN_B, PW2, NORM_FF2_W, NORM_FF2_B,
    FF2_W1, FF2_W2, NORM_OUT_W, NORM_OUT_B, NSLOTS
};
static const char* kSuffix[NSLOTS] = {
    "norm_feed_forward1.weight", "norm_feed_forward1.bias", "feed_forward1.linear1.weight",
    "feed_forward1.linear2.weight", "norm_self_att.weight", "norm_self_att.bias", "self_attn.linear_q.weight",
    "self_attn.linear_k.weight", "self_attn.linear_v.weight", "self_attn.linear_out.weight",
    "self_attn.linear_pos.weight", "self_attn.pos_bias_u", "self_attn.pos_bias_v", "norm_conv.weight",
    "norm_conv.bias", "conv.pointwise_conv1.weight", "conv.depthwise_conv.weight", "conv.batch_norm.weight",
    "conv.batch_norm.bias", "conv.pointwise_conv2.weight", "norm_feed_forward2.weight", "norm_feed_forward2.bias",
    "feed_forward2.linear1.weight", "feed_forward2.linear2.weight", "norm_out.weight", "norm_out.bias"};

struct LayerDev {
    void* ff1_w1 = nullptr; void* ff1_w2 = nullptr; void* wqkv = nullptr; void* wo = nullptr;
    void* pw1 = nullptr; void* pw2 = nullptr; void* ff2_w1 = nullptr; void* ff2_w2 = nullptr;
    float* ln[12] = {};          // ff1 g,b; att g,b; conv g,b; conv-ln g,b; ff2 g,b; out g,b
    float* bias_u = nullptr; float* bias_v = nullptr;
    float* dw_t = nullptr;       // [K][D]
    void* P = nullptr;           // [n_rel][D]
    std::vector<float> wpos;     // host copy until finalize (dtype-rounded)
    uint32_t set_mask = 0;
};


struct GraphEntry {
    int n, T;
    const void* x;
    void* out;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

struct ud_stream {
    ud_encoder* enc;
    int slot;
    int64_t frames;   // frames appended so far (ring origin and cache_len derive from it)
    int steps;
};

// Subsampling front-end (encoder.pre_encode.*, FastConformer.swift:56-95): weights and a workspace
// sized on first use for max_streams x the longest mel chunk (8 max_chunk + 9 rows).
enum SubSlot { SUB_C0W, SUB_C0B, SUB_C2W, SUB_C2B, SUB_C3W, SUB_C3B, SUB_C5W, SUB_C5B, SUB_C6W, SUB_C6B, SUB_OUTW,
               SUB_OUTB, SUB_NSLOTS };
static const char* kSubName[SUB_NSLOTS] = {
    "pre_encode.conv.0.weight", "pre_encode.conv.0.bias", "pre_encode.conv.2.weight", "pre_encode.conv.2.bias",
    "pre_encode.conv.3.weight", "pre_encode.conv.3.bias", "pre_encode.conv.5.weight", "pre_encode.conv.5.bias",
    "pre_encode.conv.6.weight", "pre_encode.conv.6.bias", "pre_encode.out.weight", "pre_encode.out.bias"};
constexpr int SUB_CH = 256, SUB_MEL = 128, SUB_F1 = SUB_MEL / 2 + 1, SUB_F2 = SUB_F1 / 2 + 1, SUB_F3 = SUB_F2 / 2 + 1;

struct SubDev {
    void* w[SUB_NSLOTS] = {};      // conv.3 / conv.6 / out weights in the GEMM layout, the rest fp32
    uint32_t set_mask = 0;
    // stage buffers: a2 conv.3's A operand; a3 conv.3's output (fp32, or half for a 16-bit encoder);
    // a4 conv.6's A operand; a5 conv.6's output (fp32 encoders only); af the out Linear's A operand
    void* a2 = nullptr; void* a3 = nullptr; void* a4 = nullptr; float* a5 = nullptr; void* af = nullptr;
    int32_t* vlen = nullptr;
    // the per-stage valid lengths of a call, staged in one of four pinned buffers [max_streams][4]
    // (an event per buffer: a buffer is rewritten only after the copy that read it has run)
    int32_t* vlen_host[4] = {};
    hipEvent_t vlen_ev[4] = {};
    bool vlen_used[4] = {};
    int vlen_next = 0;
    bool ws = false;
};

struct ud_encoder {
    ud_encoder_config cfg;
    bool bf;                        // 16-bit encoder (UD_BF16 or UD_F16): half storage, f16 MFMA
    bool wf16;                      // UD_F16: linear weights rounded fp32 -> half directly
    size_t esz;
    int D, H, dk, ff, Kc, L, layers, n_rel, rel_offset, max_rows;
    int R;                         // K/V ring rows per (slot, head): L + max_chunk
    std::vector<LayerDev> lw;
    // stream pool
    void* kring = nullptr; void* vring = nullptr; float* cring = nullptr;
    size_t ring_layer_elems = 0;   // slots * H * R * dk
    size_t cring_layer_elems = 0;  // slots * (K-1) * D
    std::vector<int> free_slots;
    std::vector<ud_stream*> live;
    // workspace
    float* res = nullptr; void* z = nullptr; void* h = nullptr; void* qkv = nullptr; void* att = nullptr;
    float* pw = nullptr;
    float* part = nullptr;          // split-K residual partial slabs [KSPLIT][max_rows][D]
    void* zero_row = nullptr;       // 256 zero bytes: the attention kernels' loads of masked rows
    void* aux = nullptr;           // ud_encoder_aux_scratch (host-side callers' device scratch)
    size_t aux_bytes = 0;
    int32_t* desc_dev = nullptr;   // [slots][DESC_INTS] descriptors, then the QKV ring-row table
    int32_t* rows_dev = nullptr;   // [slots * max_chunk + 256]: ring element offset of each step row
    int32_t* desc_host[4] = {};
    hipEvent_t desc_ev[4] = {};
    bool desc_used[4] = {};
    int desc_next = 0;
    bool finalized = false;
    // Work order across HIP streams: every call that enqueues device work records done_ev on its
    // stream when it is done enqueueing; a call on a different stream first makes its stream wait
    // for done_ev.  The calls on one encoder therefore run in call order whatever streams they are
    // issued on (they share the workspace), and done_ev always marks the end of all device work
    // enqueued so far.
    hipEvent_t done_ev = nullptr;
    hipStream_t last_st = nullptr;
    bool has_last = false;
    hipEvent_t aux_ev = nullptr;   // recorded by ud_encoder_aux_release after the aux scratch's last use
    bool aux_used = false;
    bool use_graphs = true;
    hipStream_t capture_stream = nullptr;
    std::vector<GraphEntry> graphs;
    SubDev sub;
};

// Whether a rocprofiler-sdk tool is configured for this process (rocprofv3 exports these before it
// starts the program).  Under such a tool the step is launched eagerly, never by hipGraph replay:
// with the kernel tracer active, replaying the captured step ended the host process with a
// SIGSEGV inside the tool's library -- a host memcpy reading a device-mapped address, reached from
// hipGraphLaunch -- while the same kernels launched one by one trace normally.
static bool profiler_tool_loaded() {
    const char* names[] = {"ROCP_TOOL_LIBRARIES", "ROCPROFILER_LIBRARY_CTOR"};
    for (const char* n : names) {
        const char* v = getenv(n);
        if (v && v[0]) return true;
    }
    return false;
}

static void* dev_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
    return p;
}

static void free_encoder(ud_encoder* e) {
    if (!e) return;
    (void)hipDeviceSynchronize();
    for (auto& g : e->graphs) { (void)hipGraphExecDestroy(g.exec); (void)hipGraphDestroy(g.graph); }
    for (auto& l : e->lw) {
        void* ps[] = {l.ff1_w1, l.ff1_w2, l.wqkv, l.wo, l.pw1, l.pw2, l.ff2_w1, l.ff2_w2, l.bias_u, l.bias_v, l.dw_t, l.P};
        for (void* p : ps) if (p) (void)hipFree(p);
        for (float* p : l.ln) if (p) (void)hipFree(p);
    }
    void* ws[] = {e->kring, e->vring, e->cring, e->res, e->z, e->h, e->qkv, e->att, e->pw, e->part, e->desc_dev,
                  e->zero_row, e->aux};
    for (void* p : ws) if (p) (void)hipFree(p);
    for (void* p : e->sub.w) if (p) (void)hipFree(p);
    void* sws[] = {e->sub.a2, e->sub.a3, e->sub.a4, e->sub.a5, e->sub.af, e->sub.vlen};
    for (void* p : sws) if (p) (void)hipFree(p);
    for (int i = 0; i < 4; i++) {
        if (e->desc_host[i]) (void)hipHostFree(e->desc_host[i]);
        if (e->desc_ev[i]) (void)hipEventDestroy(e->desc_ev[i]);
        if (e->sub.vlen_host[i]) (void)hipHostFree(e->sub.vlen_host[i]);
        if (e->sub.vlen_ev[i]) (void)hipEventDestroy(e->sub.vlen_ev[i]);
    }
    if (e->done_ev) (void)hipEventDestroy(e->done_ev);
    if (e->aux_ev) (void)hipEventDestroy(e->aux_ev);
    if (e->capture_stream) (void)hipStreamDestroy(e->capture_stream);
    for (ud_stream* s : e->live) delete s;
    delete e;
}

// Descriptor region: [slots][DESC_INTS], then the ring-row table of up to slots * max_chunk step
// rows, padded by 256 entries (a GEMM tile's row-table load may run past the last row).
static size_t desc_ints(const ud_encoder* e) {
    return (size_t)e->cfg.max_streams * DESC_INTS + (size_t)e->cfg.max_streams * e->cfg.max_chunk + 256;
}

extern "C" UD_API int ud_encoder_create(const ud_encoder_config* cfg, ud_encoder** out) {
    if (!cfg || !out) return fail(UD_ERR_INVALID, "ud_encoder_create: null argument");
    *out = nullptr;
    const ud_encoder_config& c = *cfg;
    if (c.layers < 1 || c.d_model < 1 || c.heads < 1 || c.d_model % c.heads != 0 || c.ff_dim < 1)
        return fail(UD_ERR_SHAPE, "ud_encoder_create: bad model dimensions");
    if (c.d_model / c.heads != 128) return fail(UD_ERR_SHAPE, "ud_encoder_create: head_dim must be 128");
    if (c.d_model != 1024) return fail(UD_ERR_SHAPE, "ud_encoder_create: d_model must be 1024");
    if (c.ff_dim % 64 != 0) return fail(UD_ERR_SHAPE, "ud_encoder_create: ff_dim must be a multiple of 64");
    if (c.conv_kernel != 9) return fail(UD_ERR_SHAPE, "ud_encoder_create: conv_kernel must be 9");
    if (c.left_context < 1 || c.max_chunk < 1 || c.max_chunk > 16 || c.max_chunk > c.left_context)
        return fail(UD_ERR_SHAPE, "ud_encoder_create: need 1 <= max_chunk <= min(16, left_context)");
    if (c.max_streams < 1) return fail(UD_ERR_SHAPE, "ud_encoder_create: max_streams must be >= 1");
    // step rows index the workspaces and kernel grids as 32-bit values
    if ((int64_t)c.max_streams * c.max_chunk > (1 << 20))
        return fail(UD_ERR_SHAPE, "ud_encoder_create: max_streams * max_chunk above 1,048,576 rows");
    if (c.dtype != UD_F32 && c.dtype != UD_BF16 && c.dtype != UD_F16)
        return fail(UD_ERR_INVALID, "ud_encoder_create: bad dtype %d", c.dtype);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1)
        return fail(UD_ERR_HIP, "ud_encoder_create: no HIP device");

    ud_encoder* e = new ud_encoder();
    e->cfg = c;
    e->bf = c.dtype == UD_BF16 || c.dtype == UD_F16;
    e->wf16 = c.dtype == UD_F16;
    e->esz = e->bf ? 2 : 4;
    e->D = c.d_model; e->H = c.heads; e->dk = c.d_model / c.heads; e->ff = c.ff_dim; e->Kc = c.conv_kernel;
    e->L = c.left_context; e->layers = c.layers;
    e->R = c.left_context + c.max_chunk;
    // makeStreamState: tables over rel = -(maxChunk-1) ... L+maxChunk-1 (FastConformer.swift:433)
    e->rel_offset = c.max_chunk - 1;
    e->n_rel = c.left_context + 2 * c.max_chunk - 1;
    e->max_rows = c.max_streams * c.max_chunk;
    const char* ev = getenv("UD_GRAPHS");
    e->use_graphs = !(ev && ev[0] == '0') && !profiler_tool_loaded();
    e->lw.resize(c.layers);

    const size_t D = e->D, ff = e->ff, esz = e->esz;
    bool ok = true;
    for (auto& l : e->lw) {
        ok &= (l.ff1_w1 = dev_alloc(ff * D * esz)) != nullptr;
        ok &= (l.ff1_w2 = dev_alloc(D * ff * esz)) != nullptr;
        ok &= (l.wqkv = dev_alloc(3 * D * D * esz)) != nullptr;
        ok &= (l.wo = dev_alloc(D * D * esz)) != nullptr;
        ok &= (l.pw1 = dev_alloc(2 * D * D * esz)) != nullptr;
        ok &= (l.pw2 = dev_alloc(D * D * esz)) != nullptr;
        ok &= (l.ff2_w1 = dev_alloc(ff * D * esz)) != nullptr;
        ok &= (l.ff2_w2 = dev_alloc(D * ff * esz)) != nullptr;
        for (auto& p : l.ln) ok &= (p = (float*)dev_alloc(D * 4)) != nullptr;
        ok &= (l.bias_u = (float*)dev_alloc(D * 4)) != nullptr;
        ok &= (l.bias_v = (float*)dev_alloc(D * 4)) != nullptr;
        ok &= (l.dw_t = (float*)dev_alloc((size_t)e->Kc * D * 4)) != nullptr;
        ok &= (l.P = dev_alloc((size_t)e->n_rel * D * esz)) != nullptr;
        if (!ok) break;
    }
    const size_t slots = c.max_streams;
    e->ring_layer_elems = slots * e->H * e->R * e->dk;
    e->cring_layer_elems = slots * (e->Kc - 1) * D;
    if (ok) {
        ok &= (e->kring = dev_alloc(e->ring_layer_elems * e->layers * esz)) != nullptr;
        ok &= (e->vring = dev_alloc(e->ring_layer_elems * e->layers * esz)) != nullptr;
        ok &= (e->cring = (float*)dev_alloc(e->cring_layer_elems * e->layers * 4)) != nullptr;
    }
    // GEMM operands (z, h, att) hold whole 16-row tiles in the fragment-major bf16 layout.
    const size_t R = e->max_rows, Rp = (R + 15) / 16 * 16;
    if (ok) {
        ok &= (e->res = (float*)dev_alloc(R * D * 4)) != nullptr;
        ok &= (e->z = dev_alloc(Rp * D * esz)) != nullptr;
        ok &= (e->h = dev_alloc(Rp * ff * esz)) != nullptr;
        ok &= (e->qkv = dev_alloc(R * 3 * D * esz)) != nullptr;
        ok &= (e->att = dev_alloc(Rp * D * esz)) != nullptr;
        ok &= (e->pw = (float*)dev_alloc(R * 2 * D * 4)) != nullptr;
        if (e->bf) ok &= (e->part = (float*)dev_alloc(KSPLIT * R * D * 4)) != nullptr;
        ok &= (e->desc_dev = (int32_t*)dev_alloc(desc_ints(e) * 4)) != nullptr;
        if (ok) e->rows_dev = e->desc_dev + slots * DESC_INTS;
        ok &= (e->zero_row = dev_alloc(256)) != nullptr;
    }
    for (int i = 0; ok && i < 4; i++) {
        ok &= hipHostMalloc((void**)&e->desc_host[i], desc_ints(e) * 4, hipHostMallocDefault) == hipSuccess;
        ok &= hipEventCreateWithFlags(&e->desc_ev[i], hipEventDisableTiming) == hipSuccess;
        ok &= hipHostMalloc((void**)&e->sub.vlen_host[i], slots * 4 * sizeof(int32_t), hipHostMallocDefault) == hipSuccess;
        ok &= hipEventCreateWithFlags(&e->sub.vlen_ev[i], hipEventDisableTiming) == hipSuccess;
    }
    ok = ok && hipEventCreateWithFlags(&e->done_ev, hipEventDisableTiming) == hipSuccess;
    ok = ok && hipEventCreateWithFlags(&e->aux_ev, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        free_encoder(e);
        return fail(UD_ERR_NOMEM, "ud_encoder_create: device allocation failed");
    }
    if (hipMemset(e->zero_row, 0, 256) != hipSuccess ||
        hipMemset(e->kring, 0, e->ring_layer_elems * e->layers * esz) != hipSuccess ||
        hipMemset(e->vring, 0, e->ring_layer_elems * e->layers * esz) != hipSuccess ||
        hipMemset(e->cring, 0, e->cring_layer_elems * e->layers * 4) != hipSuccess ||
        hipStreamCreateWithFlags(&e->capture_stream, hipStreamNonBlocking) != hipSuccess) {
        free_encoder(e);
        return fail(UD_ERR_HIP, "ud_encoder_create: initialisation failed");
    }
    for (int s = (int)slots - 1; s >= 0; s--) e->free_slots.push_back(s);
    *out = e;
    return UD_OK;
}

extern "C" UD_API void ud_encoder_destroy(ud_encoder* enc) { free_encoder(enc); }

extern "C" UD_API int ud_encoder_get_config(const ud_encoder* enc, ud_encoder_config* out) {
    if (!enc || !out) return fail(UD_ERR_INVALID, "ud_encoder_get_config: null argument");
    *out = enc->cfg;
    return UD_OK;
}

static int upload(void* dst, const void* src, size_t bytes) {
    HIPC(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return UD_OK;
}

// Converts a `rows` x `cols` fp32 weight matrix to the encoder dtype and writes it at row offset
// dst_row0 (a multiple of 16) of the destination: bf16 in the fragment-major GEMM layout, fp32
// row-major.
static int upload_matrix(ud_encoder* e, void* dst, size_t dst_row0, const float* src, size_t rows, size_t cols) {
    const size_t n = rows * cols;
    if (e->bf) {
        std::vector<uint16_t> tmp(n);
        const int nk = (int)(cols / 64);
        for (size_t i = 0; i < n; i++)
            if (!(std::fabs(host_weight16_value(src[i], e->wf16)) <= kHalfMax))
                return fail(UD_ERR_WEIGHT, "weight value %g at element %zu is outside the IEEE-half range of a 16-bit encoder",
                            (double)src[i], i);
        for (size_t r = 0; r < rows; r++)
            for (size_t c = 0; c < cols; c++)
                tmp[frag_index((int64_t)r, (int)c, nk)] = host_weight16(src[r * cols + c], e->wf16);
        return upload(static_cast<uint16_t*>(dst) + dst_row0 * cols, tmp.data(), n * 2);
    }
    return upload(static_cast<float*>(dst) + dst_row0 * cols, src, n * 4);
}

static bool parse_name(const char* name, int layers, int* layer, int* slot) {
    const char* p = name;
    if (strncmp(p, "encoder.", 8) == 0) p += 8;
    if (strncmp(p, "layers.", 7) != 0) return false;
    p += 7;
    char* end = nullptr;
    long li = strtol(p, &end, 10);
    if (end == p || *end != '.' || li < 0 || li >= layers) return false;
    p = end + 1;
    for (int s = 0; s < NSLOTS; s++)
        if (strcmp(p, kSuffix[s]) == 0) { *layer = (int)li; *slot = s; return true; }
    return false;
}

// As upload_matrix, for the front-end GEMMs (conv.3, conv.6, out): a 16-bit encoder stores these
// as IEEE half, fp32 rounded straight to half in both 16-bit modes.  (The reference's f16 checkpoint
// keeps conv.3 and conv.6 in fp32 -- WeightConverter.keepF32, Convert.swift:80 -- and rounds out
// to f16; here the front-end's 1x1 convs run on the f16 MFMA as well.)
static int upload_matrix_sub(ud_encoder* e, void* dst, const float* src, size_t rows, size_t cols) {
    if (!e->bf) return upload(dst, src, rows * cols * 4);
    const size_t n = rows * cols;
    for (size_t i = 0; i < n; i++)
        if (!(std::fabs(src[i]) <= kHalfMax))
            return fail(UD_ERR_WEIGHT, "subsampling weight value %g at element %zu is outside the IEEE-half range of a "
                        "16-bit encoder", (double)src[i], i);
    std::vector<uint16_t> tmp(n);
    const int nk = (int)(cols / 64);
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) tmp[frag_index((int64_t)r, (int)c, nk)] = host_f16(src[r * cols + c]);
    return upload(dst, tmp.data(), tmp.size() * 2);
}

static int set_sub_weight(ud_encoder* e, int slot, const char* name, const float* host, int64_t count) {
    const int64_t C = SUB_CH, D = e->D;
    int64_t want = C;
    switch (slot) {
        case SUB_C0W: case SUB_C2W: case SUB_C5W: want = C * 9; break;
        case SUB_C3W: case SUB_C6W: want = C * C; break;
        case SUB_OUTW: want = D * C * SUB_F3; break;
        case SUB_OUTB: want = D; break;
        default: break;
    }
    if (count != want)
        return fail(UD_ERR_WEIGHT, "weight '%s': %lld values, expected %lld", name, (long long)count, (long long)want);
    const bool gemm_w = slot == SUB_C3W || slot == SUB_C6W || slot == SUB_OUTW;
    void*& dst = e->sub.w[slot];
    if (!dst && !(dst = dev_alloc((size_t)want * (gemm_w ? e->esz : 4))))
        return fail(UD_ERR_NOMEM, "ud_encoder_set_weight: allocation failed");
    int rc;
    if (slot == SUB_OUTW) {
        // (channel, freq) columns of the checkpoint -> (freq, channel) for channel-last activations
        // (FastConformer.swift:78-89).
        std::vector<float> perm((size_t)want);
        for (int64_t o = 0; o < D; o++)
            for (int64_t c = 0; c < C; c++)
                for (int64_t f = 0; f < SUB_F3; f++)
                    perm[(size_t)((o * SUB_F3 + f) * C + c)] = host[(o * C + c) * SUB_F3 + f];
        rc = upload_matrix_sub(e, dst, perm.data(), (size_t)D, (size_t)(C * SUB_F3));
    } else if (gemm_w) {
        rc = upload_matrix_sub(e, dst, host, (size_t)C, (size_t)C);
    } else {
        rc = upload(dst, host, (size_t)want * 4);
    }
    if (rc != UD_OK) return rc;
    e->sub.set_mask |= 1u << slot;
    return UD_OK;
}

extern "C" UD_API int ud_encoder_set_weight(ud_encoder* e, const char* name, const float* host, int64_t count) {
    if (!e || !name || !host) return fail(UD_ERR_INVALID, "ud_encoder_set_weight: null argument");
    {
        const char* p = strncmp(name, "encoder.", 8) == 0 ? name + 8 : name;
        for (int s = 0; s < SUB_NSLOTS; s++)
            if (strcmp(p, kSubName[s]) == 0) return set_sub_weight(e, s, name, host, count);
    }
    int li = -1, slot = -1;
    if (!parse_name(name, e->layers, &li, &slot)) return fail(UD_ERR_WEIGHT, "unknown weight name '%s'", name);
    const int64_t D = e->D, ff = e->ff;
    int64_t want = 0;
    switch (slot) {
        case FF1_W1: case FF2_W1: case FF1_W2: case FF2_W2: want = ff * D; break;
        case LIN_Q: case LIN_K: case LIN_V: case LIN_OUT: case LIN_POS: case PW2: want = D * D; break;
        case PW1: want = 2 * D * D; break;
        case DW: want = D * e->Kc; break;
        default: want = D; break;   // norms, pos_bias_u/v ([H, dk] = D values)
    }
    if (count != want)
        return fail(UD_ERR_WEIGHT, "weight '%s': %lld values, expected %lld", name, (long long)count, (long long)want);
    LayerDev& l = e->lw[li];
    int rc = UD_OK;
    switch (slot) {
        case FF1_W1: rc = upload_matrix(e, l.ff1_w1, 0, host, ff, D); break;
        case FF1_W2: rc = upload_matrix(e, l.ff1_w2, 0, host, D, ff); break;
        case FF2_W1: rc = upload_matrix(e, l.ff2_w1, 0, host, ff, D); break;
        case FF2_W2: rc = upload_matrix(e, l.ff2_w2, 0, host, D, ff); break;
        case LIN_Q: rc = upload_matrix(e, l.wqkv, 0, host, D, D); break;
        case LIN_K: rc = upload_matrix(e, l.wqkv, D, host, D, D); break;
        case LIN_V: rc = upload_matrix(e, l.wqkv, 2 * D, host, D, D); break;
        case LIN_OUT: rc = upload_matrix(e, l.wo, 0, host, D, D); break;
        case PW2: rc = upload_matrix(e, l.pw2, 0, host, D, D); break;
        case PW1: {
            if (e->bf) {
                // GLU-pair row order for the fused GLU epilogue: rows 32k .. 32k+15 the value rows of
                // channels 16k .. 16k+15, rows 32k+16 .. 32k+31 their gate rows
                std::vector<float> perm((size_t)2 * D * D);
                for (int64_t r = 0; r < 2 * D; r++)
                    memcpy(&perm[(size_t)glu_row((int)r, (int)D) * D], host + r * D, (size_t)D * 4);
                rc = upload_matrix(e, l.pw1, 0, perm.data(), 2 * D, D);
            } else {
                rc = upload_matrix(e, l.pw1, 0, host, 2 * D, D);
            }
            break;
        }
        case LIN_POS: {
            l.wpos.assign(host, host + D * D);
            if (e->bf) for (auto& v : l.wpos) v = host_weight16_value(v, e->wf16);
            e->finalized = false;
            break;
        }
        case DW: {
            std::vector<float> t((size_t)e->Kc * D);
            for (int64_t d = 0; d < D; d++)
                for (int k = 0; k < e->Kc; k++) t[(size_t)k * D + d] = host[d * e->Kc + k];
            rc = upload(l.dw_t, t.data(), t.size() * 4);
            break;
        }
        case BIAS_U: rc = upload(l.bias_u, host, D * 4); break;
        case BIAS_V: rc = upload(l.bias_v, host, D * 4); break;
        default: {
            static const int ln_index[NSLOTS] = {0, 1, -1, -1, 2, 3, -1, -1, -1, -1, -1, -1, -1, 4, 5,
                                                 -1, -1, 6, 7, -1, 8, 9, -1, -1, 10, 11};
            rc = upload(l.ln[ln_index[slot]], host, D * 4);
        }
    }
    if (rc != UD_OK) return rc;
    l.set_mask |= 1u << slot;
    return UD_OK;
}

// NeMo RelPositionalEncoding row for relative position `pos` (FastConformer.swift:147-158):
// k and the angle in fp32, exp/sin/cos in double then rounded to fp32.
static void sinusoid_row(int pos, int D, float* pe) {
    const float k = -((float)std::log(10000.0) / (float)D);
    for (int i = 0; i < D; i += 2) {
        float div = (float)std::exp((double)((float)i * k));
        float angle = (float)pos * div;
        pe[i] = (float)std::sin((double)angle);
        pe[i + 1] = (float)std::cos((double)angle);
    }
}

extern "C" UD_API int ud_encoder_finalize(ud_encoder* e) {
    if (!e) return fail(UD_ERR_INVALID, "ud_encoder_finalize: null encoder");
    const uint32_t all = (1u << NSLOTS) - 1;
    for (int li = 0; li < e->layers; li++)
        if (e->lw[li].set_mask != all) {
            for (int s = 0; s < NSLOTS; s++)
                if (!(e->lw[li].set_mask & (1u << s)))
                    return fail(UD_ERR_STATE, "ud_encoder_finalize: weight encoder.layers.%d.%s not set", li, kSuffix[s]);
        }
    const int D = e->D, n = e->n_rel;
    std::vector<float> pe((size_t)n * D);
    for (int r = 0; r < n; r++) sinusoid_row(r - e->rel_offset, D, &pe[(size_t)r * D]);
    float *pe_d = nullptr, *w_d = nullptr, *p_d = nullptr;
    pe_d = (float*)dev_alloc(pe.size() * 4);
    w_d = (float*)dev_alloc((size_t)D * D * 4);
    p_d = (float*)dev_alloc(pe.size() * 4);
    int rc = UD_OK;
    if (!pe_d || !w_d || !p_d) rc = fail(UD_ERR_NOMEM, "ud_encoder_finalize: allocation failed");
    if (rc == UD_OK) rc = upload(pe_d, pe.data(), pe.size() * 4);
    std::vector<float> P(pe.size());
    std::vector<uint16_t> Pb(e->bf ? pe.size() : 0);
    for (int li = 0; rc == UD_OK && li < e->layers; li++) {
        LayerDev& l = e->lw[li];
        rc = upload(w_d, l.wpos.data(), (size_t)D * D * 4);
        if (rc != UD_OK) break;
        // P_l = PE . W_pos^T in fp32 (FastConformer.swift:168-174)
        GemmArgs g{};
        g.A = pe_d; g.W = w_d; g.C = p_d; g.M = n; g.N = D; g.K = D; g.lda = D; g.ldw = D; g.ldc = D;
        g.epi = EPI_STORE_F32; g.act = 0; g.out_scale = 1.0f;
        rc = launch_status(launch_gemm(g, false, nullptr), "position table");
        if (rc != UD_OK) break;
        if (e->bf) {
            if (hipMemcpy(P.data(), p_d, P.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) {
                rc = fail(UD_ERR_HIP, "ud_encoder_finalize: copy back failed");
                break;
            }
            for (size_t i = 0; i < P.size(); i++) Pb[i] = host_f16(P[i]);
            rc = upload(l.P, Pb.data(), Pb.size() * 2);
        } else if (hipMemcpy(l.P, p_d, P.size() * 4, hipMemcpyDeviceToDevice) != hipSuccess) {
            rc = fail(UD_ERR_HIP, "ud_encoder_finalize: copy failed");
        }
    }
    if (pe_d) (void)hipFree(pe_d);
    if (w_d) (void)hipFree(w_d);
    if (p_d) (void)hipFree(p_d);
    if (rc != UD_OK) return rc;
    HIPC(hipDeviceSynchronize());
    e->finalized = true;
    return UD_OK;
}

// Device scratch of at least `bytes` owned by the encoder (grown on demand, freed with it), for
// host-side entry points that chain the encoder's calls (ud_nemotron_step).  Growing first waits
// for the event the last user recorded with ud_encoder_aux_release, so no earlier call still uses
// the old buffer (other HIP streams and the rest of the device are not waited for).
void* ud_encoder_aux_scratch(ud_encoder* e, size_t bytes) {
    if (e->aux_bytes >= bytes) return e->aux;
    if (e->aux_used && hipEventSynchronize(e->aux_ev) != hipSuccess) return nullptr;
    if (e->aux) (void)hipFree(e->aux);
    e->aux_bytes = 0;
    e->aux = dev_alloc(bytes);
    if (e->aux) e->aux_bytes = bytes;
    return e->aux;
}

// Marks the end of a use of the aux scratch on `st` (after the last work that reads or writes it).
int ud_encoder_aux_release(ud_encoder* e, hipStream_t st) {
    HIPC(hipEventRecord(e->aux_ev, st));
    e->aux_used = true;
    return UD_OK;
}

// ---------------------------------------------------------------- streams

// Zeroes one slot's rows in every layer: blockIdx.y = layer, blockIdx.z = K ring, V ring, conv
// ring.  16-byte stores where the range is 16-byte aligned, else bytes.
__global__ void slot_zero_kernel(char* kring, char* vring, char* cring, size_t ring_layer_bytes, size_t slot_bytes,
                                 size_t cring_layer_bytes, size_t cslot_bytes, size_t slot_off, size_t cslot_off) {
    const size_t li = blockIdx.y;
    const int which = blockIdx.z;
    char* base = which == 0 ? kring + li * ring_layer_bytes + slot_off
               : which == 1 ? vring + li * ring_layer_bytes + slot_off : cring + li * cring_layer_bytes + cslot_off;
    const size_t n = which < 2 ? slot_bytes : cslot_bytes;
    const size_t stride = (size_t)gridDim.x * blockDim.x, first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t n16 = (reinterpret_cast<uintptr_t>(base) & 15) == 0 ? n / 16 : 0;
    for (size_t i = first; i < n16; i += stride) reinterpret_cast<uint4*>(base)[i] = make_uint4(0u, 0u, 0u, 0u);
    for (size_t i = n16 * 16 + first; i < n; i += stride) base[i] = 0;
}

// One launch on the null stream, waited for (the caller has synchronized the device first).
static int zero_slot(ud_encoder* e, int slot) {
    const size_t per = (size_t)e->H * e->R * e->dk, cper = (size_t)(e->Kc - 1) * e->D;
    const size_t slot_bytes = per * e->esz, cslot_bytes = cper * 4;
    const size_t blocks = std::min<size_t>(64, (std::max(slot_bytes, cslot_bytes) / 16 + 255) / 256);
    hipLaunchKernelGGL(slot_zero_kernel, dim3((unsigned)std::max<size_t>(blocks, 1), e->layers, 3), dim3(256), 0, 0,
                       static_cast<char*>(e->kring), static_cast<char*>(e->vring), reinterpret_cast<char*>(e->cring),
                       e->ring_layer_elems * e->esz, slot_bytes, e->cring_layer_elems * 4, cslot_bytes,
                       (size_t)slot * slot_bytes, (size_t)slot * cslot_bytes);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(0));
    return UD_OK;
}

extern "C" UD_API int ud_stream_create(ud_encoder* e, ud_stream** out) {
    if (!e || !out) return fail(UD_ERR_INVALID, "ud_stream_create: null argument");
    *out = nullptr;
    if (e->free_slots.empty()) return fail(UD_ERR_CAPACITY, "ud_stream_create: all %d stream slots in use", e->cfg.max_streams);
    int slot = e->free_slots.back();
    // The slot may belong to a stream destroyed while a step on another (non-blocking) HIP stream
    // was still writing its ring rows; wait for all device work before clearing it, or the new
    // stream could start with the old one's rows.
    HIPC(hipDeviceSynchronize());
    int rc = zero_slot(e, slot);
    if (rc != UD_OK) return rc;
    e->free_slots.pop_back();
    ud_stream* s = new ud_stream{e, slot, 0, 0};
    e->live.push_back(s);
    *out = s;
    return UD_OK;
}

extern "C" UD_API int ud_stream_reset(ud_stream* s) {
    if (!s) return fail(UD_ERR_INVALID, "ud_stream_reset: null stream");
    HIPC(hipDeviceSynchronize());
    int rc = zero_slot(s->enc, s->slot);
    if (rc != UD_OK) return rc;
    s->frames = 0;
    s->steps = 0;
    return UD_OK;
}

extern "C" UD_API void ud_stream_destroy(ud_stream* s) {
    if (!s) return;
    ud_encoder* e = s->enc;
    for (size_t i = 0; i < e->live.size(); i++)
        if (e->live[i] == s) { e->live.erase(e->live.begin() + i); break; }
    e->free_slots.push_back(s->slot);
    delete s;
}

extern "C" UD_API int ud_stream_info(const ud_stream* s, int32_t* cache_len, int32_t* steps) {
    if (!s) return fail(UD_ERR_INVALID, "ud_stream_info: null stream");
    if (cache_len) *cache_len = (int32_t)(s->frames < s->enc->L ? s->frames : s->enc->L);
    if (steps) *steps = s->steps;
    return UD_OK;
}

static int check_batch(ud_encoder* e, ud_stream* const* streams, int n, int T, const char* who) {
    if (!e || !streams) return fail(UD_ERR_INVALID, "%s: null argument", who);
    if (n < 1 || n > e->cfg.max_streams) return fail(UD_ERR_SHAPE, "%s: n=%d outside [1, %d]", who, n, e->cfg.max_streams);
    if (T < 1 || T > e->cfg.max_chunk) return fail(UD_ERR_SHAPE, "%s: T=%d outside [1, %d]", who, T, e->cfg.max_chunk);
    std::vector<char> seen(e->cfg.max_streams, 0);
    for (int i = 0; i < n; i++) {
        ud_stream* s = streams[i];
        if (!s || s->enc != e) return fail(UD_ERR_INVALID, "%s: stream %d is null or of another encoder", who, i);
        if (seen[s->slot]) return fail(UD_ERR_INVALID, "%s: stream %d appears twice in the batch", who, i);
        seen[s->slot] = 1;
    }
    return UD_OK;
}

// The start of a call that enqueues device work on `st`: after every earlier call's work (see
// ud_encoder::done_ev).
static int order_after_last(ud_encoder* e, hipStream_t st) {
    if (e->has_last && st != e->last_st) HIPC(hipStreamWaitEvent(st, e->done_ev, 0));
    return UD_OK;
}
// The end of such a call: done_ev marks the end of its work.
static int mark_done(ud_encoder* e, hipStream_t st) {
    HIPC(hipEventRecord(e->done_ev, st));
    e->last_st = st;
    e->has_last = true;
    return UD_OK;
}

// Writes the batch descriptor and the QKV projection's ring-row table into the next pinned staging
// buffer and copies both to the device.
static int upload_desc(ud_encoder* e, ud_stream* const* streams, int n, int T, const int32_t* valid, hipStream_t st) {
    const int k = e->desc_next;
    e->desc_next = (k + 1) % 4;
    if (e->desc_used[k]) HIPC(hipEventSynchronize(e->desc_ev[k]));
    int32_t* d = e->desc_host[k];
    int32_t* rows = d + (size_t)e->cfg.max_streams * DESC_INTS;
    for (int i = 0; i < n; i++) {
        int v = valid ? valid[i] : T;
        int32_t* di = d + i * DESC_INTS;
        di[0] = streams[i]->slot;
        // window start (frames - L) mod R: the oldest cached frame's row (frame f lives in row f mod R)
        di[1] = (int32_t)(((streams[i]->frames - e->L) % e->R + e->R) % e->R);
        di[2] = v < 0 ? 0 : (v > T ? T : v);
        di[3] = (int32_t)(streams[i]->frames < e->L ? streams[i]->frames : e->L);
        di[4] = (int32_t)(streams[i]->frames % (e->Kc - 1));
        di[5] = di[6] = di[7] = 0;
        // step row i T + t (frame frames + t) -> element offset of its ring row in the slot's head-0
        // block: (slot H R + (start + L + t) mod R) * 128
        for (int t = 0; t < T; t++)
            rows[(size_t)i * T + t] = (int32_t)(((int64_t)di[0] * e->H * e->R + (di[1] + e->L + t) % e->R) * e->dk);
    }
    HIPC(hipMemcpyAsync(e->desc_dev, d, ((size_t)e->cfg.max_streams * DESC_INTS + (size_t)n * T) * 4,
                        hipMemcpyHostToDevice, st));
    HIPC(hipEventRecord(e->desc_ev[k], st));
    e->desc_used[k] = true;
    return UD_OK;
}

// ---------------------------------------------------------------- the step

// The workspace rows of streams s0 .. s0+n-1 of a step (rows r0 = s0 * T on, r0 a multiple of 16,
// so the fragment-major operands start on a whole 16-row tile: their element offset is r0 * width
// like the row-major buffers').  The split-K slabs are [ks][n*T][D] at KSPLIT * r0 * D.
struct Ws {
    float* res; void* z; void* h; void* qkv; void* att; float* pw; float* part; int32_t* desc; int32_t* rows;
};
static Ws ws_view(ud_encoder* e, int s0, int T) {
    const size_t r0 = (size_t)s0 * T, D = e->D, esz = e->esz;
    Ws w;
    w.res = e->res + r0 * D;
    w.z = static_cast<char*>(e->z) + r0 * D * esz;
    w.h = static_cast<char*>(e->h) + r0 * e->ff * esz;
    w.qkv = static_cast<char*>(e->qkv) + r0 * 3 * D * esz;
    w.att = static_cast<char*>(e->att) + r0 * D * esz;
    w.pw = e->pw + r0 * 2 * D;
    w.part = e->part ? e->part + (size_t)KSPLIT * r0 * D : nullptr;
    w.desc = e->desc_dev + (size_t)s0 * DESC_INTS;
    w.rows = e->rows_dev + r0;
    return w;
}

// encodeLayer (FastConformer.swift:262-321) for every layer, over streams s0 .. s0+n-1 of the step
// (x and out point at their first row), on `st`.  The fp32 residual stream advances in place.  In
// bf16 mode the residual projections write K-split partial slabs that the next LayerNorm folds into
// the residual (in slab order); in fp32 mode they accumulate into it directly.
static int enqueue_rows(ud_encoder* e, int s0, int n, int T, const float* x, float* out, hipStream_t st) {
    const int D = e->D, ff = e->ff, M = n * T;
    const bool bf = e->bf;
    const Ws w = ws_view(e, s0, T);
    Partials pend{w.part, 0};
    auto gemm = [&](const void* A, const void* W, void* C, int N, int K, int ldc, int epi, int act, float scale,
                    const char* what) -> int {
        GemmArgs g{};
        g.A = A; g.W = W; g.C = C; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldw = K; g.ldc = ldc;
        g.epi = epi; g.act = act; g.out_scale = scale; g.ksplit = 1; g.f16 = bf ? 1 : 0;
        return launch_status(launch_gemm(g, bf, st), what);
    };
    // res += scale * A . W^T (N = D)
    auto resid = [&](const void* A, const void* W, int K, float scale, const char* what) -> int {
        if (!bf) return gemm(A, W, w.res, D, K, D, EPI_RESID, ACT_NONE, scale, what);
        GemmArgs g{};
        g.A = A; g.W = W; g.C = w.part; g.M = M; g.N = D; g.K = K; g.lda = K; g.ldw = K; g.ldc = D;
        g.epi = EPI_PARTIAL; g.act = ACT_NONE; g.out_scale = scale; g.f16 = 1;
        g.ksplit = gemm_partial_splits(M, D, K, bf);
        pend.n = g.ksplit;
        return launch_status(launch_gemm(g, bf, st), what);
    };
    auto take = [&]() { Partials p = pend; pend.n = 0; return p; };
    const int EPI_H = bf ? EPI_STORE_FRAG : EPI_STORE;   // FF hidden: operand of the next GEMM
    for (int li = 0; li < e->layers; li++) {
        LayerDev& l = e->lw[li];
        const size_t roff = (size_t)li * e->ring_layer_elems * e->esz;
        // res <- x (layer 0) or norm_out of the previous layer; z <- norm_feed_forward1(res)
        if (li == 0)
            LAUNCH(launch_layernorm2(x, take(), w.res, nullptr, nullptr, l.ln[0], l.ln[1], w.z, bf, M, D, st),
                   "layernorm");
        else
            LAUNCH(launch_layernorm2(w.res, take(), w.res, e->lw[li - 1].ln[10], e->lw[li - 1].ln[11], l.ln[0],
                                     l.ln[1], w.z, bf, M, D, st), "layernorm");
        int rc;
        // FF1: res += 0.5 * linear2(silu(linear1(z)))
        if ((rc = gemm(w.z, l.ff1_w1, w.h, ff, D, ff, EPI_H, ACT_SILU, 1.0f, "ff1.linear1"))) return rc;
        if ((rc = resid(w.h, l.ff1_w2, ff, 0.5f, "ff1.linear2"))) return rc;
        // MHSA: res += linear_out(relpos_attention(q, [cache; k], [cache; v]))
        LAUNCH(launch_layernorm(w.res, take(), l.ln[2], l.ln[3], w.z, bf, M, D, ACT_NONE, st), "layernorm");
        RingArgs ra{};
        ra.kring = static_cast<char*>(e->kring) + roff;
        ra.vring = static_cast<char*>(e->vring) + roff;
        ra.qkv = w.qkv; ra.P = l.P; ra.u = l.bias_u; ra.vb = l.bias_v; ra.att = w.att; ra.desc = w.desc;
        ra.zero_row = e->zero_row;
        ra.n = n; ra.T = T; ra.L = e->L; ra.R = e->R; ra.H = e->H; ra.rel_offset = e->rel_offset;
        ra.n_rel = e->n_rel;
        ra.scale = 1.0f / std::sqrt((float)e->dk);
        ra.att_frag = bf ? 1 : 0;
        if (bf) {
            // q into the qkv buffer, the new K/V rows straight into the rings
            GemmArgs g{};
            g.A = w.z; g.W = l.wqkv; g.C = w.qkv; g.M = M; g.N = 3 * D; g.K = D; g.lda = D; g.ldw = D; g.ldc = 3 * D;
            g.epi = EPI_QKV_RING; g.act = ACT_NONE; g.out_scale = 1.0f; g.ksplit = 1; g.f16 = 1;
            g.ring = QkvRing{ra.kring, ra.vring, w.rows, T, e->L, e->R, e->H};
            if ((rc = launch_status(launch_gemm(g, true, st), "qkv"))) return rc;
        } else {
            if ((rc = gemm(w.z, l.wqkv, w.qkv, 3 * D, D, 3 * D, EPI_STORE, ACT_NONE, 1.0f, "qkv"))) return rc;
            LAUNCH(launch_ring_append(ra, false, st), "ring append");
        }
        LAUNCH(launch_relpos_ring(ra, bf, st), "relpos attention");
        if ((rc = resid(w.att, l.wo, D, 1.0f, "linear_out"))) return rc;
        // Conv module: res += pw2(silu(LN(dwconv([ring; mask(glu(pw1(z)))]))))
        LAUNCH(launch_layernorm(w.res, take(), l.ln[4], l.ln[5], w.z, bf, M, D, ACT_NONE, st), "layernorm");
        // 16-bit: the GLU in pointwise_conv1's epilogue (weight rows in GLU-pair order), half rows
        // [M, D] in the pw buffer; fp32: value | gate rows [M, 2D]
        if (bf) {
            if ((rc = gemm(w.z, l.pw1, w.pw, 2 * D, D, D, EPI_GLU, ACT_NONE, 1.0f, "pointwise_conv1 + GLU"))) return rc;
        } else if ((rc = gemm(w.z, l.pw1, w.pw, 2 * D, D, 2 * D, EPI_STORE_F32, ACT_NONE, 1.0f, "pointwise_conv1"))) {
            return rc;
        }
        ConvArgs ca{};
        ca.pw = bf ? nullptr : w.pw;
        ca.glu = bf ? reinterpret_cast<const uint16_t*>(w.pw) : nullptr;
        ca.ring = e->cring + (size_t)li * e->cring_layer_elems; ca.w_t = l.dw_t;
        ca.ln_g = l.ln[6]; ca.ln_b = l.ln[7]; ca.z = w.z; ca.desc = w.desc;
        ca.n = n; ca.T = T; ca.D = D; ca.K = e->Kc; ca.z16 = bf;
        LAUNCH(launch_dwconv_ln(ca, st), "depthwise conv");
        if ((rc = resid(w.z, l.pw2, D, 1.0f, "pointwise_conv2"))) return rc;
        // FF2: res += 0.5 * linear2(silu(linear1(LN(res))))
        LAUNCH(launch_layernorm(w.res, take(), l.ln[8], l.ln[9], w.z, bf, M, D, ACT_NONE, st), "layernorm");
        if ((rc = gemm(w.z, l.ff2_w1, w.h, ff, D, ff, EPI_H, ACT_SILU, 1.0f, "ff2.linear1"))) return rc;
        if ((rc = resid(w.h, l.ff2_w2, ff, 0.5f, "ff2.linear2"))) return rc;
    }
    LayerDev& last = e->lw[e->layers - 1];
    LAUNCH(launch_layernorm(w.res, take(), last.ln[10], last.ln[11], out, false, M, D, ACT_NONE, st), "layernorm");
    return UD_OK;
}

// The step over all n streams: one chain of dependent launches on `st`.  (Independent chains over
// groups of streams on separate HIP streams, forked and joined inside the graph, were measured on
// MI355X to be slower: 64 x 2 frames 2.19 -> 2.30 ms with 2 groups, 256 x 14 frames 9.8 -> 30 ms;
// the latency-bound kernels of one chain did not overlap another chain's.)
static int enqueue_step(ud_encoder* e, int n, int T, const float* x, float* out, hipStream_t st) {
    return enqueue_rows(e, 0, n, T, x, out, st);
}

static int run_step(ud_encoder* e, int n, int T, const float* x, float* out, hipStream_t st) {
    if (!e->use_graphs) return enqueue_step(e, n, T, x, out, st);
    GraphEntry* ge = nullptr;
    for (auto& g : e->graphs)
        if (g.n == n && g.T == T && g.x == x && g.out == out) { ge = &g; break; }
    if (!ge) {
        if (e->graphs.size() >= 8) {
            // The oldest graph may have been launched last on another HIP stream: wait for all of
            // this encoder's work (done_ev follows every earlier call's) before destroying it.
            if (e->has_last) HIPC(hipEventSynchronize(e->done_ev));
            (void)hipGraphExecDestroy(e->graphs.front().exec);
            (void)hipGraphDestroy(e->graphs.front().graph);
            e->graphs.erase(e->graphs.begin());
        }
        GraphEntry g{n, T, x, out, nullptr, nullptr};
        HIPC(hipStreamBeginCapture(e->capture_stream, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_step(e, n, T, x, out, e->capture_stream);
        hipGraph_t graph = nullptr;
        hipError_t ce = hipStreamEndCapture(e->capture_stream, &graph);
        if (rc != UD_OK) { if (graph) (void)hipGraphDestroy(graph); return rc; }
        if (ce != hipSuccess) return fail(UD_ERR_HIP, "graph capture failed: %s", hipGetErrorString(ce));
        g.graph = graph;
        HIPC(hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0));
        e->graphs.push_back(g);
        ge = &e->graphs.back();
    }
    HIPC(hipGraphLaunch(ge->exec, st));
    return UD_OK;
}

extern "C" UD_API int ud_encoder_step(ud_encoder* e, ud_stream* const* streams, int32_t n, int32_t T,
                                      const float* x_dev, const int32_t* valid_T_host, float* out_dev,
                                      void* hip_stream) {
    int rc = check_batch(e, streams, n, T, "ud_encoder_step");
    if (rc != UD_OK) return rc;
    if (!e->finalized) return fail(UD_ERR_STATE, "ud_encoder_step: encoder not finalized");
    if (!x_dev || !out_dev) return fail(UD_ERR_INVALID, "ud_encoder_step: null input/output");
    if (x_dev == out_dev) return fail(UD_ERR_INVALID, "ud_encoder_step: out_dev aliases x_dev");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if ((rc = order_after_last(e, st)) != UD_OK) return rc;
    if ((rc = upload_desc(e, streams, n, T, valid_T_host, st)) != UD_OK) return rc;
    if ((rc = run_step(e, n, T, x_dev, out_dev, st)) != UD_OK) return rc;
    if ((rc = mark_done(e, st)) != UD_OK) return rc;
    for (int i = 0; i < n; i++) { streams[i]->frames += T; streams[i]->steps++; }
    return UD_OK;
}

// ---------------------------------------------------------------- subsampling front-end

static int sub_len(int t) { return t / 2 + 1; }   // FastConformer.swift:219 (causal stride-2 stage)

static int sub_workspace(ud_encoder* e) {
    if (e->sub.ws) return UD_OK;
    const size_t n = (size_t)e->cfg.max_streams;
    const int T0 = 8 * e->cfg.max_chunk + 9, T2 = sub_len(sub_len(T0)), T3 = sub_len(T2);
    const size_t r2 = n * T2 * SUB_F2, r3 = n * T3 * SUB_F3, rf = n * e->cfg.max_chunk;
    auto pad = [](size_t r) { return (r + 15) / 16 * 16; };
    SubDev& u = e->sub;
    bool ok = (u.a2 = dev_alloc(pad(r2) * SUB_CH * e->esz)) != nullptr;
    ok = ok && (u.a3 = dev_alloc(r2 * SUB_CH * (e->bf ? 2 : 4))) != nullptr;
    ok = ok && (u.a4 = dev_alloc(pad(r3) * SUB_CH * e->esz)) != nullptr;
    if (!e->bf) ok = ok && (u.a5 = (float*)dev_alloc(r3 * SUB_CH * 4)) != nullptr;   // 16-bit: conv.6 writes af
    ok = ok && (u.af = dev_alloc(pad(rf) * SUB_CH * SUB_F3 * e->esz)) != nullptr;
    ok = ok && (u.vlen = (int32_t*)dev_alloc(n * 4 * sizeof(int32_t))) != nullptr;
    if (!ok) return fail(UD_ERR_NOMEM, "ud_encoder_subsample: workspace allocation failed");
    u.ws = true;
    return UD_OK;
}

extern "C" UD_API int ud_encoder_subsample(ud_encoder* e, int32_t n, int32_t mel_rows, const float* mel_dev,
                                           const int32_t* valid_mel_host, int32_t drop, float* out_dev,
                                           int32_t* T_out, int32_t* valid_T_host, void* hip_stream) {
    if (!e || !mel_dev || !out_dev) return fail(UD_ERR_INVALID, "ud_encoder_subsample: null argument");
    if (e->sub.set_mask != (1u << SUB_NSLOTS) - 1) {
        for (int s = 0; s < SUB_NSLOTS; s++)
            if (!(e->sub.set_mask & (1u << s)))
                return fail(UD_ERR_STATE, "ud_encoder_subsample: weight encoder.%s not set", kSubName[s]);
    }
    if (n < 1 || n > e->cfg.max_streams) return fail(UD_ERR_SHAPE, "ud_encoder_subsample: n = %d outside 1..%d", n, e->cfg.max_streams);
    // The front-end workspace holds max_streams chunks of at most 8 max_chunk + 9 mel rows (every
    // stage's length grows with the mel rows, so this bounds all of them); longer chunks are
    // refused before anything is launched, whatever drop would leave.
    const int max_mel = 8 * e->cfg.max_chunk + 9;
    if (mel_rows > max_mel)
        return fail(UD_ERR_SHAPE, "ud_encoder_subsample: %d mel rows exceed the %d this encoder's workspace holds "
                    "(8 * max_chunk + 9)", mel_rows, max_mel);
    const int T0 = mel_rows, T1 = sub_len(T0), T2 = sub_len(T1), T3 = sub_len(T2);
    const int T = T3 - drop;
    if (mel_rows < 1 || drop < 0 || T < 1 || T > e->cfg.max_chunk)
        return fail(UD_ERR_SHAPE, "ud_encoder_subsample: %d mel rows with drop %d give %d frames (need 1..%d)", mel_rows,
                    drop, T, e->cfg.max_chunk);
    int rc = sub_workspace(e);
    if (rc != UD_OK) return rc;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if ((rc = order_after_last(e, st)) != UD_OK) return rc;
    SubDev& u = e->sub;
    // Valid rows per stage (FastConformer.swift:446-450): mel rows, then L -> L/2 + 1 per stage,
    // staged in the next pinned buffer once the copy that last read it has run.
    const int vk = u.vlen_next;
    u.vlen_next = (vk + 1) % 4;
    if (u.vlen_used[vk]) HIPC(hipEventSynchronize(u.vlen_ev[vk]));
    int32_t* vl = u.vlen_host[vk];
    for (int i = 0; i < n; i++) {
        int v = valid_mel_host ? valid_mel_host[i] : T0;
        v = v < 0 ? 0 : (v > T0 ? T0 : v);
        vl[i * 4 + 0] = v;
        for (int k = 1; k < 4; k++) vl[i * 4 + k] = sub_len(vl[i * 4 + k - 1]);
        if (valid_T_host) {
            const int vt = vl[i * 4 + 3] - drop;
            valid_T_host[i] = vt < 0 ? 0 : (vt > T ? T : vt);
        }
    }
    if (T_out) *T_out = T;
    HIPC(hipMemcpyAsync(u.vlen, vl, (size_t)n * 4 * sizeof(int32_t), hipMemcpyHostToDevice, st));
    HIPC(hipEventRecord(u.vlen_ev[vk], st));
    u.vlen_used[vk] = true;
    const bool bf = e->bf;
    SubArgs c01{};
    c01.mel = mel_dev; c01.vlen = u.vlen;
    c01.c0w = (const float*)u.w[SUB_C0W]; c01.c0b = (const float*)u.w[SUB_C0B];
    c01.c2w = (const float*)u.w[SUB_C2W]; c01.c2b = (const float*)u.w[SUB_C2B];
    c01.out = u.a2; c01.n = n; c01.T0 = T0; c01.F0 = SUB_MEL; c01.T1 = T1; c01.F1 = SUB_F1; c01.T2 = T2; c01.F2 = SUB_F2;
    LAUNCH(launch_sub_conv01(c01, bf, st), "subsampling conv.0 + conv.2");
    auto gemm = [&](const void* A, int slot_w, int slot_b, void* C, int M, int N, int K, int act, const char* what) {
        GemmArgs g{};
        g.A = A; g.W = u.w[slot_w]; g.C = C; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldw = K; g.ldc = N;
        g.epi = EPI_STORE_F32; g.act = act; g.out_scale = 1.0f; g.ksplit = 1; g.bias = (const float*)u.w[slot_b];
        g.f16 = bf ? 1 : 0;
        return launch_status(launch_gemm(g, bf, st), what);
    };
    // conv.3: half channel-last rows for a 16-bit encoder (the depthwise conv.5 reads them), fp32 otherwise
    {
        GemmArgs g{};
        g.A = u.a2; g.W = u.w[SUB_C3W]; g.C = u.a3; g.M = n * T2 * SUB_F2; g.N = SUB_CH; g.K = SUB_CH;
        g.lda = SUB_CH; g.ldw = SUB_CH; g.ldc = SUB_CH; g.epi = bf ? EPI_STORE : EPI_STORE_F32; g.act = ACT_RELU;
        g.out_scale = 1.0f; g.ksplit = 1; g.bias = (const float*)u.w[SUB_C3B]; g.f16 = bf ? 1 : 0;
        if ((rc = launch_status(launch_gemm(g, bf, st), "subsampling conv.3"))) return rc;
    }
    SubDwArgs dw{};
    dw.x = u.a3; dw.vlen = u.vlen; dw.w = (const float*)u.w[SUB_C5W]; dw.b = (const float*)u.w[SUB_C5B]; dw.out = u.a4;
    dw.n = n; dw.Hin = T2; dw.Win = SUB_F2; dw.Hout = T3; dw.Wout = SUB_F3; dw.stage = 2;
    LAUNCH(launch_sub_dw(dw, bf, st), "subsampling conv.5");
    if (bf) {
        // conv.6 + ReLU writes the out Linear's rows itself: flatten (freq, channel), mask, drop
        GemmArgs g{};
        g.A = u.a4; g.W = u.w[SUB_C6W]; g.C = u.af; g.M = n * T3 * SUB_F3; g.N = SUB_CH; g.K = SUB_CH;
        g.lda = SUB_CH; g.ldw = SUB_CH; g.ldc = SUB_CH; g.epi = EPI_SUBFLAT; g.act = ACT_RELU; g.out_scale = 1.0f;
        g.ksplit = 1; g.bias = (const float*)u.w[SUB_C6B]; g.f16 = 1;
        g.flat = SubFlat{u.vlen, T3, SUB_F3, T, drop};
        if ((rc = launch_status(launch_gemm(g, true, st), "subsampling conv.6 + flatten"))) return rc;
    } else {
        if ((rc = gemm(u.a4, SUB_C6W, SUB_C6B, u.a5, n * T3 * SUB_F3, SUB_CH, SUB_CH, ACT_RELU, "subsampling conv.6")))
            return rc;
        SubFlatArgs fl{};
        fl.x = u.a5; fl.vlen = u.vlen; fl.out = u.af; fl.n = n; fl.T3 = T3; fl.F3 = SUB_F3; fl.T = T; fl.drop = drop;
        LAUNCH(launch_sub_flatten(fl, bf, st), "subsampling flatten");
    }
    if ((rc = gemm(u.af, SUB_OUTW, SUB_OUTB, out_dev, n * T, e->D, SUB_CH * SUB_F3, ACT_NONE, "subsampling out")))
        return rc;
    return mark_done(e, st);
}

static RingArgs ring_args(ud_encoder* e, int n, int T, int layer, const void* qkv, void* att) {
    const size_t roff = (size_t)layer * e->ring_layer_elems * e->esz;
    const LayerDev& l = e->lw[layer];
    RingArgs ra{};
    ra.kring = static_cast<char*>(e->kring) + roff;
    ra.vring = static_cast<char*>(e->vring) + roff;
    ra.qkv = qkv; ra.P = l.P; ra.u = l.bias_u; ra.vb = l.bias_v; ra.att = att; ra.desc = e->desc_dev;
    ra.zero_row = e->zero_row;
    ra.n = n; ra.T = T; ra.L = e->L; ra.R = e->R; ra.H = e->H; ra.rel_offset = e->rel_offset; ra.n_rel = e->n_rel;
    ra.scale = 1.0f / std::sqrt((float)e->dk);
    return ra;
}

static int check_layer_call(ud_encoder* e, ud_stream* const* streams, int n, int T, int layer, const void* qkv,
                            const void* att, const char* who) {
    int rc = check_batch(e, streams, n, T, who);
    if (rc != UD_OK) return rc;
    if (!e->finalized) return fail(UD_ERR_STATE, "%s: encoder not finalized", who);
    if (layer < 0 || layer >= e->layers) return fail(UD_ERR_SHAPE, "%s: bad layer %d", who, layer);
    if (!qkv || !att) return fail(UD_ERR_INVALID, "%s: null buffer", who);
    return UD_OK;
}

extern "C" UD_API int ud_layer_attention(ud_encoder* e, ud_stream* const* streams, int32_t n, int32_t T, int32_t layer,
                                         const void* qkv_dev, const int32_t* valid_T_host, void* att_dev,
                                         void* hip_stream) {
    int rc = check_layer_call(e, streams, n, T, layer, qkv_dev, att_dev, "ud_layer_attention");
    if (rc != UD_OK) return rc;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if ((rc = order_after_last(e, st)) != UD_OK) return rc;
    if ((rc = upload_desc(e, streams, n, T, valid_T_host, st)) != UD_OK) return rc;
    // the chunk's K/V rows from qkv into the rings, then the attention over the ring windows
    const RingArgs ra = ring_args(e, n, T, layer, qkv_dev, att_dev);
    if ((rc = launch_status(launch_ring_append(ra, e->bf, st), "ring append")) != UD_OK) return rc;
    if ((rc = launch_status(launch_relpos_ring(ra, e->bf, st), "relpos attention")) != UD_OK) return rc;
    return mark_done(e, st);
}

// Launches `iters` kernels back to back between two HIP events, launch i on layer
// (layer + 1 + i) % layers, and returns the average time per launch.
template <typename Launch>
static int time_layers(ud_encoder* e, ud_stream* const* streams, int32_t n, int32_t T, int32_t layer,
                       const void* qkv_dev, void* att_dev, int32_t iters, void* hip_stream, float* avg_ms,
                       const char* what, Launch launch) {
    int rc = check_layer_call(e, streams, n, T, layer, qkv_dev, att_dev, what);
    if (rc != UD_OK) return rc;
    if (iters < 1 || !avg_ms) return fail(UD_ERR_INVALID, "%s: bad iters / output", what);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if ((rc = order_after_last(e, st)) != UD_OK) return rc;
    if ((rc = upload_desc(e, streams, n, T, nullptr, st)) != UD_OK) return rc;
    hipEvent_t ev[2];
    HIPC(hipEventCreate(&ev[0]));
    HIPC(hipEventCreate(&ev[1]));
    // Launch i uses layer (layer + 1 + i) % layers, so the caches come from HBM as in a real step
    // (one layer's rings would otherwise stay in the 256 MB last-level cache across launches).
    rc = launch_status(launch(ring_args(e, n, T, layer, qkv_dev, att_dev), st), what);
    if (rc == UD_OK && hipEventRecord(ev[0], st) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventRecord failed");
    for (int i = 0; rc == UD_OK && i < iters; i++)
        rc = launch_status(launch(ring_args(e, n, T, (layer + 1 + i) % e->layers, qkv_dev, att_dev), st), what);
    if (rc == UD_OK && hipEventRecord(ev[1], st) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventRecord failed");
    float ms = 0.0f;
    if (rc == UD_OK && hipEventSynchronize(ev[1]) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventSynchronize failed");
    if (rc == UD_OK && hipEventElapsedTime(&ms, ev[0], ev[1]) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventElapsedTime failed");
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
    if (rc == UD_OK) *avg_ms = ms / (float)iters;
    if (rc == UD_OK) rc = mark_done(e, st);
    return rc;
}

extern "C" UD_API int ud_time_layer_attention(ud_encoder* e, ud_stream* const* streams, int32_t n, int32_t T,
                                              int32_t layer, const void* qkv_dev, void* att_dev, int32_t iters,
                                              void* hip_stream, float* avg_ms) {
    return time_layers(e, streams, n, T, layer, qkv_dev, att_dev, iters, hip_stream, avg_ms, "ud_time_layer_attention",
                       [e](const RingArgs& a, hipStream_t st) { return launch_relpos_ring(a, e->bf, st); });
}

extern "C" UD_API int ud_time_ring_read_floor(ud_encoder* e, ud_stream* const* streams, int32_t n, int32_t T,
                                              int32_t layer, const void* qkv_dev, void* att_dev, int32_t iters,
                                              void* hip_stream, float* avg_ms) {
    if (e && !e->bf) return fail(UD_ERR_INVALID, "ud_time_ring_read_floor: 16-bit encoders only");
    return time_layers(e, streams, n, T, layer, qkv_dev, att_dev, iters, hip_stream, avg_ms, "ud_time_ring_read_floor",
                       [](const RingArgs& a, hipStream_t st) { return launch_ring_read_floor(a, st); });
}

// One projection of the step as the step launches it (shape, epilogue, split-K, operand layout),
// over the encoder's workspace buffers and layer `layer`'s weights.
static int launch_projection(ud_encoder* e, int which, int layer, int M, hipStream_t st, double* flops) {
    const int D = e->D, ff = e->ff;
    const LayerDev& l = e->lw[layer];
    GemmArgs g{};
    g.M = M; g.ksplit = 1; g.out_scale = 1.0f; g.act = ACT_NONE; g.f16 = e->bf ? 1 : 0;
    switch (which) {
        case UD_PROJ_FF_LINEAR1:
            g.A = e->z; g.W = l.ff1_w1; g.C = e->h; g.N = ff; g.K = D; g.ldc = ff; g.act = ACT_SILU;
            g.epi = e->bf ? EPI_STORE_FRAG : EPI_STORE;
            break;
        case UD_PROJ_FF_LINEAR2:
            g.A = e->h; g.W = l.ff1_w2; g.N = D; g.K = ff; g.out_scale = 0.5f;
            break;
        case UD_PROJ_QKV:
            // timed with the row-major store of all three parts (the step's split store puts K and V
            // into the rings instead: the same bytes, and no stream's cache is touched here)
            g.A = e->z; g.W = l.wqkv; g.C = e->qkv; g.N = 3 * D; g.K = D; g.ldc = 3 * D; g.epi = EPI_STORE;
            break;
        case UD_PROJ_LINEAR_OUT:
            g.A = e->att; g.W = l.wo; g.N = D; g.K = D;
            break;
        case UD_PROJ_PW1:
            g.A = e->z; g.W = l.pw1; g.C = e->pw; g.N = 2 * D; g.K = D;
            if (e->bf) { g.ldc = D; g.epi = EPI_GLU; }
            else { g.ldc = 2 * D; g.epi = EPI_STORE_F32; }
            break;
        case UD_PROJ_PW2:
            g.A = e->z; g.W = l.pw2; g.N = D; g.K = D;
            break;
        default:
            return fail(UD_ERR_INVALID, "ud_time_projection: projection %d", which);
    }
    if (g.N == D) {                       // the residual projections: split-K slabs (16-bit) or +=
        g.ldc = D;
        if (e->bf) { g.C = e->part; g.epi = EPI_PARTIAL; g.ksplit = gemm_partial_splits(M, D, g.K, true); }
        else { g.C = e->res; g.epi = EPI_RESID; }
    }
    g.lda = g.K; g.ldw = g.K;
    if (flops) *flops = 2.0 * M * g.N * g.K;
    return launch_status(launch_gemm(g, e->bf, st), "projection");
}

extern "C" UD_API int ud_time_projection(ud_encoder* e, int32_t which, int32_t rows, int32_t iters, void* hip_stream,
                                         float* avg_ms, double* flops) {
    if (!e || !avg_ms || iters < 1) return fail(UD_ERR_INVALID, "ud_time_projection: bad argument");
    if (!e->finalized) return fail(UD_ERR_STATE, "ud_time_projection: encoder not finalized");
    if (rows < 1 || rows > e->max_rows) return fail(UD_ERR_SHAPE, "ud_time_projection: rows %d outside 1..%d", rows, e->max_rows);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    int rc0 = order_after_last(e, st);
    if (rc0 != UD_OK) return rc0;
    hipEvent_t ev[2];
    HIPC(hipEventCreate(&ev[0]));
    HIPC(hipEventCreate(&ev[1]));
    // launch i uses layer (i + 1) % layers, so the weights stream from HBM as in a real step
    int rc = launch_projection(e, which, 0, rows, st, flops);
    if (rc == UD_OK && hipEventRecord(ev[0], st) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventRecord failed");
    for (int i = 0; rc == UD_OK && i < iters; i++) rc = launch_projection(e, which, (i + 1) % e->layers, rows, st, nullptr);
    if (rc == UD_OK && hipEventRecord(ev[1], st) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventRecord failed");
    float ms = 0.0f;
    if (rc == UD_OK && hipEventSynchronize(ev[1]) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventSynchronize failed");
    if (rc == UD_OK && hipEventElapsedTime(&ms, ev[0], ev[1]) != hipSuccess) rc = fail(UD_ERR_HIP, "hipEventElapsedTime failed");
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
    if (rc == UD_OK) *avg_ms = ms / (float)iters;
    if (rc == UD_OK) rc = mark_done(e, st);
    return rc;
}

extern "C" UD_API int ud_stream_advance(ud_stream* const* streams, int32_t n, int32_t T) {
    if (!streams || n < 0 || T < 0) return fail(UD_ERR_INVALID, "ud_stream_advance: bad argument");
    for (int i = 0; i < n; i++) {
        if (!streams[i]) return fail(UD_ERR_INVALID, "ud_stream_advance: null stream");
        streams[i]->frames += T;
        streams[i]->steps++;
    }
    return UD_OK;
}

// ---------------------------------------------------------------- cache export / import

static int cache_io(ud_stream* s, int layer, float* k, float* v, float* conv, const float* ik, const float* iv,
                    const float* iconv, bool do_import) {
    ud_encoder* e = s->enc;
    if (layer < 0 || layer >= e->layers) return fail(UD_ERR_SHAPE, "cache: bad layer %d", layer);
    HIPC(hipDeviceSynchronize());
    const int L = e->L, R = e->R, H = e->H, dk = e->dk, D = e->D, KC = e->Kc - 1;
    const size_t per = (size_t)H * R * dk, cper = (size_t)KC * D;
    char* kb = static_cast<char*>(e->kring) + ((size_t)layer * e->ring_layer_elems + s->slot * per) * e->esz;
    char* vb = static_cast<char*>(e->vring) + ((size_t)layer * e->ring_layer_elems + s->slot * per) * e->esz;
    float* cb = e->cring + (size_t)layer * e->cring_layer_elems + s->slot * cper;
    // cache row r (oldest first) = frame frames - L + r = ring row (frames - L + r) mod R
    const int start = (int)(((s->frames - L) % R + R) % R), cpos = (int)(s->frames % KC);
    std::vector<uint8_t> kr(per * e->esz), vr(per * e->esz);
    std::vector<float> cr(cper);
    auto get = [&](const std::vector<uint8_t>& buf, size_t i) -> float {
        return e->bf ? host_f16_to_f(reinterpret_cast<const uint16_t*>(buf.data())[i])
                     : reinterpret_cast<const float*>(buf.data())[i];
    };
    auto put = [&](std::vector<uint8_t>& buf, size_t i, float x) {
        if (e->bf) reinterpret_cast<uint16_t*>(buf.data())[i] = host_f16(x);
        else reinterpret_cast<float*>(buf.data())[i] = x;
    };
    if (!do_import) {
        HIPC(hipMemcpy(kr.data(), kb, kr.size(), hipMemcpyDeviceToHost));
        HIPC(hipMemcpy(vr.data(), vb, vr.size(), hipMemcpyDeviceToHost));
        HIPC(hipMemcpy(cr.data(), cb, cr.size() * 4, hipMemcpyDeviceToHost));
    }
    for (int r = 0; r < L; r++) {
        const int sl = (start + r) % R;
        for (int h = 0; h < H; h++)
            for (int d = 0; d < dk; d++) {
                const size_t ri = ((size_t)h * R + sl) * dk + d, li = (size_t)r * D + h * dk + d;
                if (do_import) { put(kr, ri, ik[li]); put(vr, ri, iv[li]); }
                else { if (k) k[li] = get(kr, ri); if (v) v[li] = get(vr, ri); }
            }
    }
    for (int r = 0; r < KC; r++) {
        const int sl = (cpos + r) % KC;
        for (int d = 0; d < D; d++) {
            if (do_import) cr[(size_t)sl * D + d] = iconv[(size_t)r * D + d];
            else if (conv) conv[(size_t)r * D + d] = cr[(size_t)sl * D + d];
        }
    }
    if (do_import) {
        HIPC(hipMemcpy(kb, kr.data(), kr.size(), hipMemcpyHostToDevice));
        HIPC(hipMemcpy(vb, vr.data(), vr.size(), hipMemcpyHostToDevice));
        HIPC(hipMemcpy(cb, cr.data(), cr.size() * 4, hipMemcpyHostToDevice));
    }
    return UD_OK;
}

extern "C" UD_API int ud_stream_export_cache(const ud_stream* s, int32_t layer, float* k_host, float* v_host,
                                             float* conv_host, int32_t* cache_len) {
    if (!s) return fail(UD_ERR_INVALID, "ud_stream_export_cache: null stream");
    int rc = cache_io(const_cast<ud_stream*>(s), layer, k_host, v_host, conv_host, nullptr, nullptr, nullptr, false);
    if (rc == UD_OK && cache_len) *cache_len = (int32_t)(s->frames < s->enc->L ? s->frames : s->enc->L);
    return rc;
}

extern "C" UD_API int ud_stream_import_cache(ud_stream* s, int32_t layer, const float* k_host, const float* v_host,
                                             const float* conv_host, int32_t cache_len) {
    if (!s || !k_host || !v_host || !conv_host) return fail(UD_ERR_INVALID, "ud_stream_import_cache: null argument");
    ud_encoder* e = s->enc;
    if (cache_len < 0 || cache_len > e->L) return fail(UD_ERR_SHAPE, "ud_stream_import_cache: cache_len %d", cache_len);
    // Keep the ring origin when the window length is unchanged, so layers imported one by one stay
    // consistent; otherwise re-base (then every layer should be imported).
    const int64_t cur = s->frames < e->L ? s->frames : e->L;
    if (cur != cache_len) s->frames = cache_len;
    return cache_io(s, layer, nullptr, nullptr, nullptr, k_host, v_host, conv_host, true);
}

// ---------------------------------------------------------------- offline key ranges

// MaskSpec.ranges(T:) (FastConformer.swift:324-343) and chunkedLimitedRanges (:346-357), then the
// clip of every range's end to the utterance's valid length (forwardOffline, :380-381), for B
// utterances of T frames.  Only the end is clipped, as in the reference: a query whose chunk starts
// past the valid length gets lo > hi, an empty range (output 0).
extern "C" UD_API int ud_chunked_limited_ranges(int32_t kind, int32_t B, int32_t T, const int32_t* valid_host,
                                                int32_t left, int32_t chunk, int32_t right, int32_t* ranges_host) {
    if (!ranges_host) return fail(UD_ERR_INVALID, "ud_chunked_limited_ranges: null output");
    if (B < 1 || T < 1) return fail(UD_ERR_SHAPE, "ud_chunked_limited_ranges: B = %d, T = %d", B, T);
    if (left < 0 || right < 0) return fail(UD_ERR_SHAPE, "ud_chunked_limited_ranges: left %d, right %d", left, right);
    int cs = 0, back = 0;
    if (kind == UD_MASK_CHUNKED_LIMITED) {
        cs = right + 1;                    // chunks of right + 1 frames, left / (right + 1) chunks back
        back = left / cs * cs;
    } else if (kind == UD_MASK_CHUNKED_LIMITED_RC) {
        if (chunk < 1) return fail(UD_ERR_SHAPE, "ud_chunked_limited_ranges: chunk %d", chunk);
        cs = chunk;                        // [c chunk - left, c chunk + chunk - 1 + right], inclusive
        back = left;
    } else {
        return fail(UD_ERR_INVALID, "ud_chunked_limited_ranges: mask kind %d", kind);
    }
    const int extra = kind == UD_MASK_CHUNKED_LIMITED ? 0 : right;
    for (int b = 0; b < B; b++) {
        const int v = valid_host ? valid_host[b] : T;
        int32_t* r = ranges_host + (size_t)b * T * 2;
        for (int i = 0; i < T; i++) {
            const int64_t c0 = (int64_t)(i / cs) * cs;
            const int64_t lo = c0 - back, hi = c0 + cs + extra;
            const int64_t end = hi < T ? hi : T;
            r[2 * i] = (int32_t)(lo > 0 ? lo : 0);
            r[2 * i + 1] = (int32_t)(end < v ? end : v);
        }
    }
    return UD_OK;
}

// ---------------------------------------------------------------- single-op entry

extern "C" UD_API int ud_relpos_attention_batched(int32_t dtype, const void* q, const void* k, const void* v,
                                                  const void* p, const float* u, const float* vb,
                                                  const int32_t* ranges, void* out, int32_t B, int32_t T, int32_t H,
                                                  int32_t dk, int32_t rel_offset, int32_t n_rel, void* hip_stream) {
    if (!q || !k || !v || !p || !u || !vb || !ranges || !out) return fail(UD_ERR_INVALID, "ud_relpos_attention_batched: null pointer");
    if (dtype != UD_BF16) return fail(UD_ERR_INVALID, "ud_relpos_attention_batched: bf16 only");
    if (dk != 128) return fail(UD_ERR_SHAPE, "ud_relpos_attention_batched: head_dim %d (128 supported)", dk);
    if (B < 1 || T < 1 || H < 1 || n_rel < 1) return fail(UD_ERR_SHAPE, "ud_relpos_attention_batched: bad sizes");
    const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)p | (uintptr_t)u | (uintptr_t)vb;
    if (al % 16 != 0) return fail(UD_ERR_INVALID, "ud_relpos_attention_batched: pointers must be 16-byte aligned");
    DenseArgs a{};
    a.q = q; a.k = k; a.v = v; a.P = p; a.u = u; a.vb = vb; a.ranges = ranges; a.out = out;
    a.B = B; a.T = T; a.H = H; a.rel_offset = rel_offset; a.n_rel = n_rel;
    a.scale = 1.0f / sqrtf((float)dk);
    return launch_status(launch_relpos_dense(a, static_cast<hipStream_t>(hip_stream)), "offline relpos attention");
}

extern "C" UD_API int ud_relpos_attention(int32_t dtype, const void* q, const void* k, const void* v, const void* p,
                                          const float* u, const float* vb, const int32_t* ranges, void* out,
                                          int32_t Tq, int32_t Tk, int32_t H, int32_t dk, int32_t rel_offset,
                                          int32_t n_rel, void* hip_stream) {
    if (!q || !k || !v || !p || !u || !vb || !ranges || !out) return fail(UD_ERR_INVALID, "ud_relpos_attention: null pointer");
    if (dtype != UD_F32 && dtype != UD_BF16) return fail(UD_ERR_INVALID, "ud_relpos_attention: bad dtype");
    if (dk != 16 && dk != 32 && dk != 64 && dk != 128) return fail(UD_ERR_SHAPE, "ud_relpos_attention: dk=%d", dk);
    if (Tq < 1 || Tq > 16 || Tk < 1 || H < 1 || n_rel < 1) return fail(UD_ERR_SHAPE, "ud_relpos_attention: bad sizes");
    const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)p | (uintptr_t)out;
    if (al % 16 != 0) return fail(UD_ERR_INVALID, "ud_relpos_attention: pointers must be 16-byte aligned");
    OpArgs a{};
    a.q = q; a.k = k; a.v = v; a.p = p; a.u = u; a.vb = vb; a.ranges = ranges; a.out = out;
    a.Tq = Tq; a.Tk = Tk; a.H = H; a.dk = dk; a.rel_offset = rel_offset; a.n_rel = n_rel;
    a.scale = 1.0f / std::sqrt((float)dk);
    return launch_status(launch_relpos_op(a, dtype == UD_BF16, static_cast<hipStream_t>(hip_stream)), "relpos attention");
}
