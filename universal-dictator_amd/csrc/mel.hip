// NeMo log-mel frontend on the GPU (include/ud_mel.h).
//
// The reference computes the features on the CPU (Sources/DictatorCore/Audio/NemoMel.swift:85-107):
// two sgemms of the [T, 400] frame matrix against window-folded cos/sin tables [257, 400], the
// power |X|^2 (as sqrt then square), a third sgemm against the filterbank and log(x + 2^-24).
// Here one workgroup takes FR frames of one job (8, or 4 when the grid is small) and does all of
// it in LDS:
//
//   stage    the frames' preemphasized samples times the window, sample-major (xs[n][t]), so one
//            16-byte LDS read broadcasts 4 frames' sample n to the whole wave; the 512-entry
//            cos table; all global loads of a thread are issued before its first LDS store
//   DFT      thread k = bin k (0..255) runs over the 400 samples.  The angle of (k, n) is
//            2 pi j / 512 with j = k (n + 56) mod 512 (the window sits at offset 56 of the
//            512-point frame), so cos and -sin are two reads of the LDS cos table, at j and at
//            j + 128; j advances by k per sample.  No global load in the loop: 2 table reads,
//            FR / 4 broadcast frame reads and 2 * FR FMAs per sample.  Bin 256 (Nyquist) is a
//            32-lane split reduction per frame
//   power    into LDS pw[k][t]
//   mel      thread (m, frame quad) sums fbT[k][m] * pw[k][t] over the bins from band m's first
//            to its last nonzero weight (the products outside are +0, so the sum is the same as
//            over all 257 bins for any finite power), then log
//
// Rounding: the reference multiplies x by float(cos) * window (its table entries); here
// (x * window) * float(cos): the same terms to within an ulp each.  Every frame is computed the
// same way wherever it sits in the grid and whatever FR (fixed summation order), so a frame
// recomputed by a later streaming chunk is bit-identical to its first computation.  The preemphasis is evaluated as the
// reference writes it, a[i] - 0.97 * a[i-1] with both roundings (contraction off).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/ud_mel.h"
#include "kernels.hpp"

int ud_set_error(int code, const char* msg);   // encoder.hip

namespace ud {

constexpr int MEL_WIN = 400;
constexpr int MEL_HOP = 160;
constexpr int MEL_NB = 257;        // rfft bins of n_fft 512
constexpr int MEL_OFF = 56;        // (512 - 400) / 2
constexpr int MEL_THREADS = 256;

__device__ __forceinline__ float preemph(float a, float prev) {
#pragma clang fp contract(off)
    return a - 0.97f * prev;
}

__device__ __forceinline__ float mel_power(float re, float im) {
#pragma clang fp contract(off)
    const float mag = sqrtf(re * re + im * im);
    return mag * mag;
}

template <int FR>
__global__ __launch_bounds__(MEL_THREADS) void mel_kernel(const MelJob* __restrict__ jobs, MelTables tb) {
    static_assert(FR == 4 || FR == 8, "frames per workgroup");
    __shared__ float4 xs[MEL_WIN][FR / 4];
    __shared__ float4 pw[MEL_NB][FR / 4];
    __shared__ float cs[512];
    const MelJob J = jobs[blockIdx.y];
    const int j0 = blockIdx.x * FR;
    if (j0 >= J.nf) return;
    const int tid = threadIdx.x;
    const int nfr = min(FR, J.nf - j0);
    const long long fbase = J.f0 + j0;

    constexpr int SU = (FR * MEL_WIN + MEL_THREADS - 1) / MEL_THREADS;
    float* xsf = reinterpret_cast<float*>(xs);
    float va[SU], vb[SU], wv[SU];
    long long ix[SU];
#pragma unroll
    for (int u = 0; u < SU; u++) {
        const int e = tid + MEL_THREADS * u;
        const int t = e / MEL_WIN, i = e - t * MEL_WIN;
        const long long f = fbase + t;
        ix[u] = -1;
        va[u] = vb[u] = wv[u] = 0.0f;
        if (e < FR * MEL_WIN && t < nfr && f < J.zero_from) {
            const long long idx = f * MEL_HOP - 200 + i;
            if (idx >= 0 && idx < J.n_audio) {
                ix[u] = idx;
                va[u] = J.src[idx - J.first];
                if (idx > 0) vb[u] = J.src[idx - 1 - J.first];
                wv[u] = tb.win[i];
            }
        }
    }
    const float c0 = tb.cos512[tid], c1 = tb.cos512[tid + MEL_THREADS];
#pragma unroll
    for (int u = 0; u < SU; u++) {
        const int e = tid + MEL_THREADS * u;
        if (e < FR * MEL_WIN) {
            const int t = e / MEL_WIN, i = e - t * MEL_WIN;
            const float x = ix[u] < 0 ? 0.0f : ix[u] == 0 ? va[u] : preemph(va[u], vb[u]);
            xsf[i * FR + t] = x * wv[u];
        }
    }
    cs[tid] = c0;
    cs[tid + MEL_THREADS] = c1;
    __syncthreads();

    {
        // bin 256: j = 256 (n + 56) mod 512; frame t = tid / 32 (< FR), lane l of 32 takes
        // samples l, l + 32, ...; butterfly over the 32 lanes (xor offsets below 32 stay inside
        // each half of the wave)
        const int t = tid >> 5, l = tid & 31;
        float r = 0.0f, q = 0.0f;
        for (int n = l; t < FR && n < MEL_WIN; n += 32) {
            const int j = (256 * (n + MEL_OFF)) & 511;
            const float x = xsf[n * FR + t];
            r = fmaf(cs[j], x, r);
            q = fmaf(cs[(j + 128) & 511], x, q);
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            r += __shfl_xor(r, o);
            q += __shfl_xor(q, o);
        }
        if (l == 0 && t < FR) reinterpret_cast<float*>(pw[256])[t] = mel_power(r, q);
    }
    {
        float re[FR], im[FR];
#pragma unroll
        for (int t = 0; t < FR; t++) re[t] = im[t] = 0.0f;
        const int k = tid;
        int j = (k * MEL_OFF) & 511;
#pragma unroll 4
        for (int n = 0; n < MEL_WIN; n++) {
            const float c = cs[j], s = cs[(j + 128) & 511];
            j = (j + k) & 511;
#pragma unroll
            for (int q = 0; q < FR / 4; q++) {
                const float4 x = xs[n][q];
                re[4 * q + 0] = fmaf(c, x.x, re[4 * q + 0]); im[4 * q + 0] = fmaf(s, x.x, im[4 * q + 0]);
                re[4 * q + 1] = fmaf(c, x.y, re[4 * q + 1]); im[4 * q + 1] = fmaf(s, x.y, im[4 * q + 1]);
                re[4 * q + 2] = fmaf(c, x.z, re[4 * q + 2]); im[4 * q + 2] = fmaf(s, x.z, im[4 * q + 2]);
                re[4 * q + 3] = fmaf(c, x.w, re[4 * q + 3]); im[4 * q + 3] = fmaf(s, x.w, im[4 * q + 3]);
            }
        }
#pragma unroll
        for (int q = 0; q < FR / 4; q++)
            pw[tid][q] = make_float4(mel_power(re[4 * q], im[4 * q]), mel_power(re[4 * q + 1], im[4 * q + 1]),
                                     mel_power(re[4 * q + 2], im[4 * q + 2]), mel_power(re[4 * q + 3], im[4 * q + 3]));
    }
    __syncthreads();

    constexpr int MT = MEL_THREADS / (FR / 4);   // threads per frame quad
    const int quad = tid / MT;                    // frames 4 quad .. 4 quad + 3
    for (int m = tid % MT; m < tb.n_mels; m += MT) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* w = tb.fbT + m;
        const int2 kr = tb.krange[m];
#pragma unroll 8
        for (int k = kr.x; k < kr.y; k++) {
            const float fw = w[(long long)k * tb.n_mels];
            const float4 p = pw[k][quad];
            acc[0] = fmaf(fw, p.x, acc[0]);
            acc[1] = fmaf(fw, p.y, acc[1]);
            acc[2] = fmaf(fw, p.z, acc[2]);
            acc[3] = fmaf(fw, p.w, acc[3]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 4 * quad + i;
            if (t < nfr) {
                const long long f = fbase + t;
                J.dst[(long long)(j0 + t) * tb.n_mels + m] = f < J.zero_from ? logf(acc[i] + 5.9604644775390625e-8f) : 0.0f;
            }
        }
    }
}

int launch_mel(const MelTables& t, const MelJob* jobs_dev, int n_jobs, int max_nf, hipStream_t st) {
    if (n_jobs < 1 || max_nf < 1) return 0;
    if (t.n_mels < 1 || t.n_mels > 256 || n_jobs > 65535) return -2;
    // 8 frames per workgroup share each cos-table read; below 4 such workgroups per CU the
    // grid is too small to hide the DFT loop's latency, and 4 frames per workgroup halve it
    const int wg8 = (max_nf + 7) / 8 * n_jobs;
    if (wg8 < 1024) mel_kernel<4><<<dim3((max_nf + 3) / 4, n_jobs), MEL_THREADS, 0, st>>>(jobs_dev, t);
    else mel_kernel<8><<<dim3((max_nf + 7) / 8, n_jobs), MEL_THREADS, 0, st>>>(jobs_dev, t);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ud

using namespace ud;

static int mfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return ud_set_error(code, buf);
}

constexpr int MEL_RING = 4;   // job lists of ud_mel_features in flight before a call waits

struct ud_mel {
    int n_mels = 0;
    float *cos512 = nullptr, *win = nullptr, *fbT = nullptr;
    int2* krange = nullptr;
    // ring of job lists for ud_mel_features: slot i's pinned staging is rewritten only after the
    // kernel that read slot i's device copy has finished (its event)
    MelJob* djobs[MEL_RING] = {};
    MelJob* hjobs[MEL_RING] = {};
    hipEvent_t done[MEL_RING] = {};
    int cap_jobs = 0, next = 0;
};

namespace ud {
MelTables mel_tables_of(const ::ud_mel* m) { return MelTables{m->cos512, m->win, m->fbT, m->krange, m->n_mels}; }
}  // namespace ud

static void free_mel(ud_mel* m) {
    if (!m) return;
    (void)hipDeviceSynchronize();
    for (void* p : {(void*)m->cos512, (void*)m->win, (void*)m->fbT, (void*)m->krange}) if (p) (void)hipFree(p);
    for (int i = 0; i < MEL_RING; i++) {
        if (m->djobs[i]) (void)hipFree(m->djobs[i]);
        if (m->hjobs[i]) (void)hipHostFree(m->hjobs[i]);
        if (m->done[i]) (void)hipEventDestroy(m->done[i]);
    }
    delete m;
}

extern "C" UD_API int ud_mel_create(const float* fb_host, int32_t n_mels, const float* window_host, ud_mel** out) {
    if (!out || !fb_host || !window_host) return mfail(UD_ERR_INVALID, "ud_mel_create: null argument");
    *out = nullptr;
    if (n_mels < 1 || n_mels > 256) return mfail(UD_ERR_SHAPE, "ud_mel_create: n_mels %d outside 1..256", n_mels);
    // cos(2 pi j / 512) in double, rounded to float (the reference's float(cos(phase)),
    // NemoMel.swift:33-35), the window as given, the filterbank transposed to [257][n_mels]
    std::vector<float> cs(512), fbT((size_t)MEL_NB * n_mels);
    for (int j = 0; j < 512; j++) cs[j] = (float)cos(2.0 * 3.14159265358979323846 * (double)j / 512.0);
    std::vector<int2> kr(n_mels);
    for (int m = 0; m < n_mels; m++) {
        int lo = MEL_NB, hi = 0;
        for (int k = 0; k < MEL_NB; k++) {
            const float w = fb_host[(size_t)m * MEL_NB + k];
            fbT[(size_t)k * n_mels + m] = w;
            if (w != 0.0f) { lo = std::min(lo, k); hi = k + 1; }
        }
        kr[m] = make_int2(lo < hi ? lo : 0, hi);
    }
    ud_mel* m = new ud_mel();
    m->n_mels = n_mels;
    bool ok = hipMalloc(&m->cos512, 512 * 4) == hipSuccess && hipMalloc(&m->win, MEL_WIN * 4) == hipSuccess &&
              hipMalloc(&m->fbT, fbT.size() * 4) == hipSuccess && hipMalloc(&m->krange, n_mels * sizeof(int2)) == hipSuccess;
    for (int i = 0; ok && i < MEL_RING; i++) ok = hipEventCreateWithFlags(&m->done[i], hipEventDisableTiming) == hipSuccess;
    ok = ok && hipMemcpy(m->cos512, cs.data(), 512 * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(m->win, window_host, MEL_WIN * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(m->fbT, fbT.data(), fbT.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(m->krange, kr.data(), n_mels * sizeof(int2), hipMemcpyHostToDevice) == hipSuccess;
    if (!ok) {
        free_mel(m);
        return mfail(UD_ERR_NOMEM, "ud_mel_create: device allocation or upload failed");
    }
    *out = m;
    return UD_OK;
}

extern "C" UD_API void ud_mel_destroy(ud_mel* m) { free_mel(m); }

extern "C" UD_API int32_t ud_mel_bins(const ud_mel* m) { return m ? m->n_mels : 0; }

extern "C" UD_API int ud_mel_features(ud_mel* m, int32_t n, const float* audio_dev, int64_t audio_stride,
                                      const int64_t* n_samples_host, float* out_dev, int32_t out_rows,
                                      int32_t* frames_host, void* hip_stream) {
    if (!m || !audio_dev || !n_samples_host || !out_dev) return mfail(UD_ERR_INVALID, "ud_mel_features: null argument");
    if (n < 1 || n > 65535) return mfail(UD_ERR_SHAPE, "ud_mel_features: n = %d outside 1..65535", n);
    int max_nf = 0;
    for (int b = 0; b < n; b++) {
        const int64_t ns = n_samples_host[b];
        if (ns < 0 || ns > audio_stride)
            return mfail(UD_ERR_SHAPE, "ud_mel_features: clip %d has %lld samples (stride %lld)", b, (long long)ns,
                         (long long)audio_stride);
        const int64_t T = ns / MEL_HOP + 1;
        if (T > out_rows) return mfail(UD_ERR_SHAPE, "ud_mel_features: clip %d needs %lld rows > out_rows %d", b, (long long)T, out_rows);
        if (T > max_nf) max_nf = (int)T;
    }
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if (n > m->cap_jobs) {
        for (int i = 0; i < MEL_RING; i++) {
            (void)hipEventSynchronize(m->done[i]);
            if (m->djobs[i]) (void)hipFree(m->djobs[i]);
            if (m->hjobs[i]) (void)hipHostFree(m->hjobs[i]);
            m->djobs[i] = nullptr;
            m->hjobs[i] = nullptr;
        }
        m->cap_jobs = 0;
        for (int i = 0; i < MEL_RING; i++)
            if (hipMalloc(&m->djobs[i], (size_t)n * sizeof(MelJob)) != hipSuccess ||
                hipHostMalloc((void**)&m->hjobs[i], (size_t)n * sizeof(MelJob)) != hipSuccess)
                return mfail(UD_ERR_NOMEM, "ud_mel_features: job list allocation failed");
        m->cap_jobs = n;
    }
    const int slot = m->next;
    m->next = (m->next + 1) % MEL_RING;
    if (hipEventSynchronize(m->done[slot]) != hipSuccess) return mfail(UD_ERR_HIP, "ud_mel_features: event wait failed");
    MelJob* hj = m->hjobs[slot];
    for (int b = 0; b < n; b++) {
        const int64_t ns = n_samples_host[b];
        MelJob& j = hj[b];
        j.src = audio_dev + (int64_t)b * audio_stride;
        j.dst = out_dev + (int64_t)b * out_rows * m->n_mels;
        j.first = 0;
        j.n_audio = ns;
        j.f0 = 0;
        j.nf = (int)(ns / MEL_HOP + 1);
        j.zero_from = ns / MEL_HOP;
        j.pad_ = 0;
        if (frames_host) frames_host[b] = j.nf;
    }
    if (hipMemcpyAsync(m->djobs[slot], hj, (size_t)n * sizeof(MelJob), hipMemcpyHostToDevice, st) != hipSuccess)
        return mfail(UD_ERR_HIP, "ud_mel_features: job upload failed");
    const int rc = launch_mel(mel_tables_of(m), m->djobs[slot], n, max_nf, st);
    if (rc != 0) return mfail(rc == -2 ? UD_ERR_SHAPE : UD_ERR_HIP, "ud_mel_features: launch failed");
    if (hipEventRecord(m->done[slot], st) != hipSuccess) return mfail(UD_ERR_HIP, "ud_mel_features: event record failed");
    return UD_OK;
}
