// Batched cache-aware streaming driver (include/ud_streamer.h): NemotronStreamer's schedule
// (Sources/DictatorCore/Nemotron/NemotronStreamer.swift:70-153, NemotronSchedule.swift:7-17) for
// every open stream at once, each batched step running the device pipeline
//   mel (ud_mel kernel or staged rows) -> subsampling (<= 2 launches) -> encoder step ->
//   joint.enc -> greedy RNN-T.
// Host-only C++ over the library's C ABI and launchers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/ud_streamer.h"
#include "kernels.hpp"

int ud_set_error(int code, const char* msg);   // encoder.hip

using ud::MelJob;

namespace {

int tfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return ud_set_error(code, buf);
}

constexpr int HOP = 160;
constexpr int PRE_CACHE = 9;    // NemotronSchedule.preEncodeCache
constexpr int DROP = 2;         // NemotronSchedule.dropExtra

enum Mode { FRESH = 0, LIVE = 1, BUFFERED = 2 };

struct SStream {
    bool open = false;
    ud_stream* es = nullptr;
    int mode = FRESH;
    int64_t next = 0;           // first mel frame of the next chunk (liveNextFrame / idx)
    bool done = false;          // final chunk run, or the tail dropped
    // live input: samples [audio_start, n_audio)
    std::vector<float> audio;
    int64_t audio_start = 0, n_audio = 0;
    bool finished = false;
    // buffered input (valid during ud_streamer_run_buffered only)
    const float* mel = nullptr;
    int64_t frames = 0, valid_frames = 0;
    std::vector<int32_t> tokens;
    std::vector<float> rec_enc, rec_proj;
    // emissions of live input (token i of tokens is emission i while the stream is live): samples
    // pushed when the token's chunk ran, and that batched step's wall seconds
    std::vector<int64_t> emit_samples;
    std::vector<double> emit_secs;
    std::vector<double> step_secs;   // wall seconds of each chunk's batched step
};

struct Plan {
    int id;
    int64_t cache_start, chunk_end;   // real mel rows: frames [cache_start, chunk_end)
    int valid;                        // valid rows for the subsampling
    bool first, last;
};

}  // namespace

struct ud_streamer {
    ud_encoder* enc = nullptr;
    ud_rnnt* rnnt = nullptr;
    ud_mel* mel = nullptr;
    int la = 0, first_chunk = 0, chunk = 0, T = 0, rows_first = 0, rows_rest = 0;
    int D = 0, Hd = 0, n_mels = 128, S = 0, max_sym = 0;
    bool end_padding = true, record = false;
    std::vector<SStream> st;
    hipStream_t hs = nullptr;
    hipEvent_t uploaded = nullptr;   // the last staging upload (staging is rewritten after it)
    float *dmel = nullptr, *dx = nullptr, *dy = nullptr, *dproj = nullptr;
    char* dstage = nullptr;          // [MelJob x S][samples: S x win]
    char* hstage = nullptr;          // pinned mirror of dstage
    float* hmel = nullptr;           // pinned mirror of dmel
    size_t job_bytes = 0, win = 0;
    int64_t batches = 0, chunks = 0;
    // per-batch host scratch
    std::vector<int32_t> toks, counts, slots, vmel, vt;
    std::vector<ud_stream*> handles;
    std::vector<float> rec_y, rec_p;
};

namespace {

void free_streamer(ud_streamer* s) {
    if (!s) return;
    if (s->hs) (void)hipStreamSynchronize(s->hs);
    for (SStream& x : s->st)
        if (x.es) ud_stream_destroy(x.es);
    for (void* p : {(void*)s->dmel, (void*)s->dx, (void*)s->dy, (void*)s->dproj, (void*)s->dstage})
        if (p) (void)hipFree(p);
    if (s->hstage) (void)hipHostFree(s->hstage);
    if (s->hmel) (void)hipHostFree(s->hmel);
    if (s->uploaded) (void)hipEventDestroy(s->uploaded);
    if (s->hs) (void)hipStreamDestroy(s->hs);
    delete s;
}

int64_t live_have(const SStream& x) {
    if (x.finished) return x.n_audio / HOP + 1;
    return x.n_audio >= 200 ? (x.n_audio - 200) / HOP + 1 : 0;
}

// drainChunks (NemotronStreamer.swift:113-126): the next chunk of a live stream, if it can run.
bool plan_live(const ud_streamer* s, SStream& x, int id, Plan& p) {
    const int64_t have = live_have(x);
    const int64_t idx = x.next;
    const bool first = idx == 0;
    const int64_t size = first ? s->first_chunk : s->chunk;
    const int64_t end = idx + size;
    if (end > have && !x.finished) return false;
    const int64_t chunk_end = std::min(end, have);
    const int64_t chunk_len = chunk_end - idx;
    const int64_t min_len = first ? 1 : 8;
    if (chunk_len <= 0 || (chunk_len < min_len && !(x.finished && s->end_padding))) {
        if (x.finished) x.done = true;
        return false;
    }
    p.id = id;
    p.first = first;
    p.cache_start = first ? idx : std::max<int64_t>(0, idx - PRE_CACHE);
    p.chunk_end = chunk_end;
    p.valid = (int)(chunk_end - p.cache_start);
    p.last = x.finished && end >= have;
    return true;
}

// runBuffered (NemotronStreamer.swift:74-88).
bool plan_buffered(const ud_streamer* s, SStream& x, int id, Plan& p) {
    const int64_t idx = x.next;
    if (idx >= x.frames) {
        x.done = true;
        return false;
    }
    const bool first = idx == 0;
    const int64_t size = first ? s->first_chunk : s->chunk;
    const int64_t end = std::min(idx + size, x.frames);
    const int64_t chunk_len = end - idx;
    if (chunk_len < (first ? 1 : 8)) {
        x.done = true;
        return false;
    }
    p.id = id;
    p.first = first;
    p.cache_start = first ? idx : std::max<int64_t>(0, idx - PRE_CACHE);
    const int64_t added = idx - p.cache_start;
    const int64_t rows = added + chunk_len;
    p.chunk_end = p.cache_start + rows;
    p.valid = (int)std::max<int64_t>(0, std::min<int64_t>(x.valid_frames - idx + added, rows));
    p.last = idx + size >= x.frames;
    return true;
}

#define TCHECK(call, what)                                                                        \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess) return tfail(UD_ERR_HIP, "%s: %s", what, hipGetErrorString(e_));    \
    } while (0)

// One batched step over plans (first chunks ordered first).
int run_batch(ud_streamer* s, std::vector<Plan>& plans) {
    const auto t_start = std::chrono::steady_clock::now();
    std::stable_partition(plans.begin(), plans.end(), [](const Plan& p) { return p.first; });
    const int n = (int)plans.size();
    int nF = 0;
    while (nF < n && plans[nF].first) nF++;
    const int nm = s->n_mels;
    TCHECK(hipEventSynchronize(s->uploaded), "streamer staging wait");

    MelJob* jobs = reinterpret_cast<MelJob*>(s->hstage);
    float* hsamp = reinterpret_cast<float*>(s->hstage + s->job_bytes);
    const float* dsamp = reinterpret_cast<const float*>(s->dstage + s->job_bytes);
    int n_live = 0, max_nf = 0;
    bool any_buf = false;
    size_t mel_off = 0;   // floats into dmel
    for (int b = 0; b < n; b++) {
        const Plan& p = plans[b];
        SStream& x = s->st[p.id];
        const int R = p.first ? s->rows_first : s->rows_rest;
        const int64_t real = p.chunk_end - p.cache_start;
        if (x.mode == BUFFERED) {
            any_buf = true;
            float* dst = s->hmel + mel_off;
            memcpy(dst, x.mel + p.cache_start * nm, (size_t)real * nm * 4);
            memset(dst + real * nm, 0, (size_t)(R - real) * nm * 4);
        } else {
            const int64_t w0 = std::max<int64_t>(0, p.cache_start * HOP - 201);
            const int64_t w1 = std::min<int64_t>(x.n_audio, (p.chunk_end - 1) * HOP + 200);
            if (w1 - w0 > (int64_t)s->win || w0 < x.audio_start)
                return tfail(UD_ERR_STATE, "streamer: sample window [%lld, %lld) not staged", (long long)w0, (long long)w1);
            float* hs = hsamp + (size_t)n_live * s->win;
            if (w1 > w0) memcpy(hs, x.audio.data() + (w0 - x.audio_start), (size_t)(w1 - w0) * 4);
            MelJob& j = jobs[n_live];
            j.src = dsamp + (size_t)n_live * s->win;
            j.dst = s->dmel + mel_off;
            j.first = w0;
            j.n_audio = x.n_audio;
            j.f0 = p.cache_start;
            j.nf = R;
            j.zero_from = std::min<int64_t>(p.chunk_end, x.finished ? x.n_audio / HOP : LLONG_MAX);
            j.pad_ = 0;
            n_live++;
            max_nf = std::max(max_nf, R);
        }
        mel_off += (size_t)R * nm;
        s->slots[b] = p.id;
        s->handles[b] = x.es;
        s->vmel[b] = p.valid;
    }
    if (n_live) {
        const size_t bytes = s->job_bytes + (size_t)n_live * s->win * 4;
        TCHECK(hipMemcpyAsync(s->dstage, s->hstage, bytes, hipMemcpyHostToDevice, s->hs), "streamer sample upload");
    }
    if (any_buf) TCHECK(hipMemcpyAsync(s->dmel, s->hmel, mel_off * 4, hipMemcpyHostToDevice, s->hs), "streamer mel upload");
    TCHECK(hipEventRecord(s->uploaded, s->hs), "streamer event");
    if (n_live) {
        const int rc = ud::launch_mel(ud::mel_tables_of(s->mel), reinterpret_cast<const MelJob*>(s->dstage), n_live,
                                      max_nf, s->hs);
        if (rc != 0) return tfail(UD_ERR_HIP, "streamer: mel launch failed");
    }
    int rc;
    const size_t xrow = (size_t)s->T * s->D;
    if (nF) {
        int T = 0;
        rc = ud_encoder_subsample(s->enc, nF, s->rows_first, s->dmel, s->vmel.data(), 0, s->dx, &T, s->vt.data(), s->hs);
        if (rc != UD_OK) return rc;
        if (T != s->T) return tfail(UD_ERR_STATE, "streamer: first chunk gave %d frames, expected %d", T, s->T);
    }
    if (n > nF) {
        int T = 0;
        rc = ud_encoder_subsample(s->enc, n - nF, s->rows_rest, s->dmel + (size_t)nF * s->rows_first * nm,
                                  s->vmel.data() + nF, DROP, s->dx + nF * xrow, &T, s->vt.data() + nF, s->hs);
        if (rc != UD_OK) return rc;
        if (T != s->T) return tfail(UD_ERR_STATE, "streamer: chunk gave %d frames, expected %d", T, s->T);
    }
    rc = ud_encoder_step(s->enc, s->handles.data(), n, s->T, s->dx, s->vt.data(), s->dy, s->hs);
    if (rc != UD_OK) return rc;
    rc = ud_rnnt_project(s->rnnt, n * s->T, s->dy, s->dproj, s->hs);
    if (rc != UD_OK) return rc;
    const int cap = s->max_sym * s->T;
    rc = ud_rnnt_greedy(s->rnnt, n, s->slots.data(), s->dproj, s->T, s->vt.data(), s->toks.data(), cap,
                        s->counts.data(), s->hs);
    if (rc != UD_OK) return rc;
    if (s->record) {
        TCHECK(hipMemcpy(s->rec_y.data(), s->dy, (size_t)n * xrow * 4, hipMemcpyDeviceToHost), "streamer record");
        TCHECK(hipMemcpy(s->rec_p.data(), s->dproj, (size_t)n * s->T * s->Hd * 4, hipMemcpyDeviceToHost), "streamer record");
    }
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_start).count();
    for (int b = 0; b < n; b++) {
        const Plan& p = plans[b];
        SStream& x = s->st[p.id];
        const int c = std::min(s->counts[b], cap);
        x.tokens.insert(x.tokens.end(), s->toks.begin() + (size_t)b * cap, s->toks.begin() + (size_t)b * cap + c);
        x.step_secs.push_back(secs);
        if (x.mode == LIVE) {
            x.emit_samples.insert(x.emit_samples.end(), (size_t)c, x.n_audio);
            x.emit_secs.insert(x.emit_secs.end(), (size_t)c, secs);
        }
        if (s->record) {
            const int keep = s->vt[b];
            x.rec_enc.insert(x.rec_enc.end(), s->rec_y.begin() + b * xrow, s->rec_y.begin() + b * xrow + (size_t)keep * s->D);
            const size_t po = (size_t)b * s->T * s->Hd;
            x.rec_proj.insert(x.rec_proj.end(), s->rec_p.begin() + po, s->rec_p.begin() + po + (size_t)keep * s->Hd);
        }
        x.next += p.first ? s->first_chunk : s->chunk;
        if (p.last) x.done = true;
        if (x.mode == LIVE) {
            // keep only the samples the next chunk's pre-encode cache frames need
            const int64_t keep_from = std::max<int64_t>(0, (x.next - PRE_CACHE) * HOP - 201);
            if (keep_from > x.audio_start) {
                const int64_t drop = std::min<int64_t>(keep_from - x.audio_start, (int64_t)x.audio.size());
                x.audio.erase(x.audio.begin(), x.audio.begin() + drop);
                x.audio_start += drop;
            }
        }
    }
    s->batches++;
    s->chunks += n;
    return UD_OK;
}

int drain(ud_streamer* s) {
    std::vector<Plan> plans;
    for (;;) {
        plans.clear();
        for (int i = 0; i < s->S; i++) {
            SStream& x = s->st[i];
            if (!x.open || x.done || x.mode == FRESH) continue;
            Plan p;
            if (x.mode == LIVE ? plan_live(s, x, i, p) : plan_buffered(s, x, i, p)) plans.push_back(p);
        }
        if (plans.empty()) return UD_OK;
        const int rc = run_batch(s, plans);
        if (rc != UD_OK) {
            // the batch may have advanced some device state (encoder caches, decoder slots) and
            // not the schedule: its streams end here rather than continue out of step
            for (const Plan& p : plans) s->st[p.id].done = true;
            return rc;
        }
    }
}

int check_id(const ud_streamer* s, int32_t id, const char* who) {
    if (id < 0 || id >= s->S || !s->st[id].open) return tfail(UD_ERR_INVALID, "%s: stream %d is not open", who, id);
    return UD_OK;
}

}  // namespace

extern "C" UD_API int ud_streamer_create(ud_encoder* enc, ud_rnnt* rnnt, ud_mel* mel, int32_t lookahead,
                                         int32_t max_streams, ud_streamer** out) {
    if (!out || !enc || !rnnt) return tfail(UD_ERR_INVALID, "ud_streamer_create: null argument");
    *out = nullptr;
    ud_encoder_config cfg;
    int rc = ud_encoder_get_config(enc, &cfg);
    if (rc != UD_OK) return rc;
    int32_t Hd, V, L, E, RS, MS;
    rc = ud_rnnt_get_info(rnnt, &Hd, &V, &L, &E, &RS, &MS);
    if (rc != UD_OK) return rc;
    if (lookahead < 0 || lookahead + 1 > cfg.max_chunk)
        return tfail(UD_ERR_SHAPE, "ud_streamer_create: lookahead %d needs max_chunk >= %d (encoder has %d)", lookahead,
                     lookahead + 1, cfg.max_chunk);
    if (max_streams < 1 || max_streams > cfg.max_streams || max_streams > RS)
        return tfail(UD_ERR_SHAPE, "ud_streamer_create: max_streams %d outside 1..min(%d, %d)", max_streams, cfg.max_streams, RS);
    if (E != cfg.d_model) return tfail(UD_ERR_SHAPE, "ud_streamer_create: decoder enc_dim %d != d_model %d", E, cfg.d_model);
    ud_streamer* s = new ud_streamer();
    s->enc = enc;
    s->rnnt = rnnt;
    s->mel = mel;
    s->la = lookahead;
    s->first_chunk = 1 + 8 * lookahead;
    s->chunk = 8 + 8 * lookahead;
    s->T = lookahead + 1;
    s->rows_first = s->first_chunk;
    s->rows_rest = PRE_CACHE + s->chunk;
    s->D = cfg.d_model;
    s->Hd = Hd;
    s->n_mels = mel ? ud_mel_bins(mel) : 128;
    s->S = max_streams;
    s->max_sym = MS;
    s->st.resize(max_streams);
    if (s->n_mels != 128) {
        free_streamer(s);
        return tfail(UD_ERR_SHAPE, "ud_streamer_create: the subsampling takes 128 mel bins, frontend has %d", ud_mel_bins(mel));
    }
    const size_t S = max_streams;
    s->job_bytes = (S * sizeof(MelJob) + 255) / 256 * 256;
    s->win = ((size_t)(s->rows_rest - 1) * HOP + 401 + 63) / 64 * 64;
    const size_t stage = s->job_bytes + S * s->win * 4;
    const size_t melf = S * s->rows_rest * s->n_mels;
    bool ok = hipStreamCreateWithFlags(&s->hs, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&s->uploaded, hipEventDisableTiming) == hipSuccess &&
              hipMalloc(&s->dmel, melf * 4) == hipSuccess && hipMalloc(&s->dx, S * s->T * s->D * 4) == hipSuccess &&
              hipMalloc(&s->dy, S * s->T * s->D * 4) == hipSuccess && hipMalloc(&s->dproj, S * s->T * Hd * 4) == hipSuccess &&
              hipMalloc(&s->dstage, stage) == hipSuccess && hipHostMalloc((void**)&s->hstage, stage) == hipSuccess &&
              hipHostMalloc((void**)&s->hmel, melf * 4) == hipSuccess;
    ok = ok && hipEventRecord(s->uploaded, s->hs) == hipSuccess;
    if (!ok) {
        free_streamer(s);
        return tfail(UD_ERR_NOMEM, "ud_streamer_create: allocation failed");
    }
    s->toks.assign(S * s->max_sym * s->T, 0);
    s->counts.assign(S, 0);
    s->slots.assign(S, 0);
    s->vmel.assign(S, 0);
    s->vt.assign(S, 0);
    s->handles.assign(S, nullptr);
    s->rec_y.resize(S * s->T * s->D);
    s->rec_p.resize(S * s->T * Hd);
    *out = s;
    return UD_OK;
}

extern "C" UD_API void ud_streamer_destroy(ud_streamer* s) { free_streamer(s); }

extern "C" UD_API int ud_streamer_open(ud_streamer* s, int32_t* id) {
    if (!s || !id) return tfail(UD_ERR_INVALID, "ud_streamer_open: null argument");
    for (int i = 0; i < s->S; i++) {
        SStream& x = s->st[i];
        if (x.open) continue;
        int rc = x.es ? ud_stream_reset(x.es) : ud_stream_create(s->enc, &x.es);
        if (rc != UD_OK) return rc;
        if ((rc = ud_rnnt_reset(s->rnnt, i)) != UD_OK) return rc;
        ud_stream* es = x.es;
        x = SStream();
        x.es = es;
        x.open = true;
        *id = i;
        return UD_OK;
    }
    return tfail(UD_ERR_CAPACITY, "ud_streamer_open: all %d streams are open", s->S);
}

extern "C" UD_API int ud_streamer_close(ud_streamer* s, int32_t id) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_close: null streamer");
    int rc = check_id(s, id, "ud_streamer_close");
    if (rc != UD_OK) return rc;
    SStream& x = s->st[id];
    ud_stream* es = x.es;
    x = SStream();
    x.es = es;   // kept for the next open (reset there)
    return UD_OK;
}

extern "C" UD_API int ud_streamer_set_options(ud_streamer* s, int32_t end_padding, int32_t record) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_set_options: null streamer");
    s->end_padding = end_padding != 0;
    s->record = record != 0;
    return UD_OK;
}

extern "C" UD_API int ud_streamer_push(ud_streamer* s, int32_t n, const int32_t* ids, const float* const* samples_host,
                                       const int64_t* counts) {
    if (!s || (n > 0 && (!ids || !samples_host || !counts))) return tfail(UD_ERR_INVALID, "ud_streamer_push: null argument");
    if (!s->mel) return tfail(UD_ERR_STATE, "ud_streamer_push: the streamer has no mel frontend");
    for (int b = 0; b < n; b++) {
        int rc = check_id(s, ids[b], "ud_streamer_push");
        if (rc != UD_OK) return rc;
        const SStream& x = s->st[ids[b]];
        if (x.mode == BUFFERED || x.finished)
            return tfail(UD_ERR_STATE, "ud_streamer_push: stream %d is %s", ids[b], x.finished ? "flushed" : "buffered");
        if (counts[b] < 0 || (counts[b] > 0 && !samples_host[b])) return tfail(UD_ERR_INVALID, "ud_streamer_push: bad samples");
    }
    for (int b = 0; b < n; b++) {
        SStream& x = s->st[ids[b]];
        x.mode = LIVE;
        x.audio.insert(x.audio.end(), samples_host[b], samples_host[b] + counts[b]);
        x.n_audio += counts[b];
    }
    return drain(s);
}

extern "C" UD_API int ud_streamer_flush(ud_streamer* s, int32_t n, const int32_t* ids) {
    if (!s || (n > 0 && !ids)) return tfail(UD_ERR_INVALID, "ud_streamer_flush: null argument");
    for (int b = 0; b < n; b++) {
        int rc = check_id(s, ids[b], "ud_streamer_flush");
        if (rc != UD_OK) return rc;
        if (s->st[ids[b]].mode == BUFFERED) return tfail(UD_ERR_STATE, "ud_streamer_flush: stream %d is buffered", ids[b]);
    }
    if (!s->mel && n > 0) return tfail(UD_ERR_STATE, "ud_streamer_flush: the streamer has no mel frontend");
    for (int b = 0; b < n; b++) {
        SStream& x = s->st[ids[b]];
        x.mode = LIVE;
        x.finished = true;
    }
    return drain(s);
}

extern "C" UD_API int ud_streamer_run_buffered(ud_streamer* s, int32_t n, const int32_t* ids, const float* const* mel_host,
                                               const int32_t* frames, const int32_t* valid_frames) {
    if (!s || (n > 0 && (!ids || !mel_host || !frames || !valid_frames)))
        return tfail(UD_ERR_INVALID, "ud_streamer_run_buffered: null argument");
    for (int b = 0; b < n; b++) {
        int rc = check_id(s, ids[b], "ud_streamer_run_buffered");
        if (rc != UD_OK) return rc;
        const SStream& x = s->st[ids[b]];
        if (x.mode != FRESH) return tfail(UD_ERR_STATE, "ud_streamer_run_buffered: stream %d is not fresh", ids[b]);
        if (frames[b] < 0 || (frames[b] > 0 && !mel_host[b])) return tfail(UD_ERR_INVALID, "ud_streamer_run_buffered: bad mel");
        for (int c = 0; c < b; c++)
            if (ids[c] == ids[b]) return tfail(UD_ERR_INVALID, "ud_streamer_run_buffered: repeated stream %d", ids[b]);
    }
    for (int b = 0; b < n; b++) {
        SStream& x = s->st[ids[b]];
        x.mode = BUFFERED;
        x.mel = mel_host[b];
        x.frames = frames[b];
        x.valid_frames = valid_frames[b];
    }
    const int rc = drain(s);
    for (int b = 0; b < n; b++) {
        SStream& x = s->st[ids[b]];
        x.mel = nullptr;
        x.done = true;
    }
    return rc;
}

extern "C" UD_API int ud_streamer_tokens(const ud_streamer* s, int32_t id, int32_t* out, int32_t cap, int32_t* count) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_tokens: null streamer");
    int rc = check_id(s, id, "ud_streamer_tokens");
    if (rc != UD_OK) return rc;
    const std::vector<int32_t>& t = s->st[id].tokens;
    if (out && cap > 0) memcpy(out, t.data(), std::min<size_t>(t.size(), (size_t)cap) * 4);
    if (count) *count = (int32_t)t.size();
    return UD_OK;
}

extern "C" UD_API int ud_streamer_recorded(const ud_streamer* s, int32_t id, int32_t which, float* out, int64_t cap_rows,
                                           int64_t* rows) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_recorded: null streamer");
    int rc = check_id(s, id, "ud_streamer_recorded");
    if (rc != UD_OK) return rc;
    if (which != 0 && which != 1) return tfail(UD_ERR_INVALID, "ud_streamer_recorded: which must be 0 or 1");
    const std::vector<float>& v = which == 0 ? s->st[id].rec_enc : s->st[id].rec_proj;
    const int64_t w = which == 0 ? s->D : s->Hd;
    const int64_t r = (int64_t)v.size() / w;
    if (out && cap_rows > 0) memcpy(out, v.data(), (size_t)std::min(r, cap_rows) * w * 4);
    if (rows) *rows = r;
    return UD_OK;
}

extern "C" UD_API int ud_streamer_emissions(const ud_streamer* s, int32_t id, int32_t* tokens, int64_t* samples_seen,
                                            double* compute_seconds, int32_t cap, int32_t* count) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_emissions: null streamer");
    int rc = check_id(s, id, "ud_streamer_emissions");
    if (rc != UD_OK) return rc;
    const SStream& x = s->st[id];
    const size_t n = x.emit_samples.size(), m = std::min<size_t>(n, cap > 0 ? (size_t)cap : 0);
    if (tokens && m) memcpy(tokens, x.tokens.data(), m * 4);
    if (samples_seen && m) memcpy(samples_seen, x.emit_samples.data(), m * 8);
    if (compute_seconds && m) memcpy(compute_seconds, x.emit_secs.data(), m * 8);
    if (count) *count = (int32_t)n;
    return UD_OK;
}

extern "C" UD_API int ud_streamer_step_times(const ud_streamer* s, int32_t id, double* out, int32_t cap, int32_t* count) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_step_times: null streamer");
    int rc = check_id(s, id, "ud_streamer_step_times");
    if (rc != UD_OK) return rc;
    const std::vector<double>& v = s->st[id].step_secs;
    if (out && cap > 0) memcpy(out, v.data(), std::min<size_t>(v.size(), (size_t)cap) * 8);
    if (count) *count = (int32_t)v.size();
    return UD_OK;
}

extern "C" UD_API int ud_streamer_stats(const ud_streamer* s, int64_t* batches, int64_t* chunks) {
    if (!s) return tfail(UD_ERR_INVALID, "ud_streamer_stats: null streamer");
    if (batches) *batches = s->batches;
    if (chunks) *chunks = s->chunks;
    return UD_OK;
}

// ---------------------------------------------------------------- one chunk step, mel -> joint.enc

static int sub3(int t) {
    for (int k = 0; k < 3; k++) t = t / 2 + 1;   // FastConformer.swift:219, three stride-2 stages
    return t;
}

// NemotronEncoder.step (NemotronStreamer.swift:6-12; MetalNemotronEncoder.step, Nemotron.swift:74-91)
// for n streams at once: streams at their first step subsample with drop 0, the others with
// drop_extra, each group as one ud_encoder_subsample + ud_encoder_step + ud_rnnt_project; the
// kept frames (valid_T, capped at out_frames unless keep_all) are copied to the caller's rows.
extern "C" UD_API int ud_nemotron_step(ud_encoder* enc, ud_rnnt* rnnt, ud_stream* const* streams, int32_t n,
                                       int32_t mel_rows, const float* mel_dev, const int32_t* valid_rows_host,
                                       const int32_t* keep_all_host, int32_t drop_extra, int32_t out_frames,
                                       float* proj_dev, int32_t proj_rows, int32_t* frames_host, void* hip_stream) {
    if (!enc || !rnnt || !streams || !mel_dev || !valid_rows_host || !proj_dev || !frames_host)
        return tfail(UD_ERR_INVALID, "ud_nemotron_step: null argument");
    ud_encoder_config cfg;
    int rc = ud_encoder_get_config(enc, &cfg);
    if (rc != UD_OK) return rc;
    int32_t Hd = 0, V = 0, Lr = 0, E = 0, RS = 0, MS = 0;
    if ((rc = ud_rnnt_get_info(rnnt, &Hd, &V, &Lr, &E, &RS, &MS)) != UD_OK) return rc;
    if (n < 1 || n > cfg.max_streams) return tfail(UD_ERR_SHAPE, "ud_nemotron_step: n = %d outside 1..%d", n, cfg.max_streams);
    if (E != cfg.d_model) return tfail(UD_ERR_SHAPE, "ud_nemotron_step: decoder enc_dim %d != d_model %d", E, cfg.d_model);
    if (mel_rows < 1 || drop_extra < 0 || out_frames < 1 || proj_rows < 1)
        return tfail(UD_ERR_SHAPE, "ud_nemotron_step: bad mel_rows / drop_extra / out_frames / proj_rows");
    // groups: first steps (drop 0) and the rest (drop_extra); each group's frame count must fit
    std::vector<int> grp[2];
    for (int i = 0; i < n; i++) {
        if (!streams[i]) return tfail(UD_ERR_INVALID, "ud_nemotron_step: null stream %d", i);
        int32_t cl = 0, steps = 0;
        if ((rc = ud_stream_info(streams[i], &cl, &steps)) != UD_OK) return rc;
        grp[steps == 0 ? 0 : 1].push_back(i);
    }
    // Every shape check of both groups' calls comes before anything is launched, so a shape error
    // leaves every stream where it was (see ud_streamer.h for the failures that can still come
    // after the first group has advanced).
    if (mel_rows > 8 * cfg.max_chunk + 9)
        return tfail(UD_ERR_SHAPE, "ud_nemotron_step: %d mel rows exceed the encoder's %d", mel_rows,
                     8 * cfg.max_chunk + 9);
    for (int g = 0; g < 2; g++) {
        const int T = sub3(mel_rows) - (g == 0 ? 0 : drop_extra);
        if (!grp[g].empty() && (T < 1 || T > proj_rows || T > cfg.max_chunk))
            return tfail(UD_ERR_SHAPE, "ud_nemotron_step: %d mel rows give %d frames (%s steps); proj_rows is %d, "
                         "max_chunk %d", mel_rows, T, g == 0 ? "first" : "later", proj_rows, cfg.max_chunk);
    }
    // scratch: the group's mel rows, subsampled frames, encoder output, projection
    constexpr int NM = 128;
    auto al = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t rows_max = (size_t)n * cfg.max_chunk;
    const size_t o_x = al((size_t)n * mel_rows * NM * 4), o_y = o_x + al(rows_max * cfg.d_model * 4);
    const size_t o_p = o_y + al(rows_max * cfg.d_model * 4), total = o_p + al(rows_max * Hd * 4);
    char* base = static_cast<char*>(ud_encoder_aux_scratch(enc, total));
    if (!base) return tfail(UD_ERR_NOMEM, "ud_nemotron_step: scratch allocation failed");
    float* gmel = reinterpret_cast<float*>(base);
    float* x = reinterpret_cast<float*>(base + o_x);
    float* y = reinterpret_cast<float*>(base + o_y);
    float* p = reinterpret_cast<float*>(base + o_p);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const size_t chunk = (size_t)mel_rows * NM;
    for (int g = 0; g < 2; g++) {
        const std::vector<int>& idx = grp[g];
        const int ng = (int)idx.size();
        if (ng == 0) continue;
        std::vector<int32_t> vmel(ng), vt(ng);
        std::vector<ud_stream*> hs(ng);
        for (int j = 0; j < ng; j++) {
            TCHECK(hipMemcpyAsync(gmel + j * chunk, mel_dev + idx[j] * chunk, chunk * 4, hipMemcpyDeviceToDevice, st),
                   "ud_nemotron_step: mel gather");
            vmel[j] = valid_rows_host[idx[j]];
            hs[j] = streams[idx[j]];
        }
        int T = 0;
        if ((rc = ud_encoder_subsample(enc, ng, mel_rows, gmel, vmel.data(), g == 0 ? 0 : drop_extra, x, &T, vt.data(),
                                       hip_stream)) != UD_OK)
            return rc;
        if ((rc = ud_encoder_step(enc, hs.data(), ng, T, x, vt.data(), y, hip_stream)) != UD_OK) return rc;
        if ((rc = ud_rnnt_project(rnnt, ng * T, y, p, hip_stream)) != UD_OK) return rc;
        for (int j = 0; j < ng; j++) {
            const bool keep_all = keep_all_host && keep_all_host[idx[j]];
            const int keep = keep_all ? vt[j] : std::min(vt[j], out_frames);
            frames_host[idx[j]] = keep;
            if (keep > 0)
                TCHECK(hipMemcpyAsync(proj_dev + (size_t)idx[j] * proj_rows * Hd, p + (size_t)j * T * Hd,
                                      (size_t)keep * Hd * 4, hipMemcpyDeviceToDevice, st),
                       "ud_nemotron_step: projection copy");
        }
    }
    return ud_encoder_aux_release(enc, st);
}
