// NeMo log-mel frontend on the GPU (include/ud_mel.h).
//
// The reference computes the features on the CPU (Sources/DictatorCore/Audio/NemoMel.swift:85-107):
// two sgemms of the [T, 400] frame matrix against window-folded cos/sin tables [257, 400], the
// power |X|^2 (as sqrt then square), a third sgemm against the filterbank and log(x + 2^-24).
// Here one workgroup takes MEL_FR frames of one job and does all of it:
//
//   stage    the frames' preemphasized samples into LDS, sample-major (xs[n][t]), so one
//            16-byte LDS read broadcasts 4 frames' sample n to the whole wave
//   DFT      thread k = bin k (0..255) runs over the 400 samples: 2 table loads (tab[n][k],
//            coalesced over the wave, L2-resident: the tables are 820 KB), 2 LDS reads and
//            2 * MEL_FR FMAs per sample; bin 256 (Nyquist) is a 32-lane split reduction per frame
//   power    into LDS pw[k][t]
//   mel      thread (m, frame quad) sums fbT[k][m] * pw[k][t] over the 257 bins, then log
//
// Every frame is computed the same way wherever it sits in the grid (fixed summation order), so a
// frame recomputed by a later streaming chunk is bit-identical to its first computation.  The
// preemphasis is evaluated as the reference writes it, a[i] - 0.97 * a[i-1] with both roundings
// (no contraction), so the staged samples are exactly the reference's.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/ud_mel.h"
#include "kernels.hpp"

int ud_set_error(int code, const char* msg);   // encoder.hip

namespace ud {

constexpr int MEL_FR = 8;          // frames per workgroup
constexpr int MEL_WIN = 400;
constexpr int MEL_HOP = 160;
constexpr int MEL_NB = 257;        // rfft bins of n_fft 512
constexpr int MEL_THREADS = 256;

__device__ __forceinline__ float mel_power(float re, float im) {
    const float mag = __fsqrt_rn(__fadd_rn(__fmul_rn(re, re), __fmul_rn(im, im)));
    return __fmul_rn(mag, mag);
}

__global__ __launch_bounds__(MEL_THREADS) void mel_kernel(const MelJob* __restrict__ jobs, MelTables tb) {
    __shared__ float4 xs[MEL_WIN][MEL_FR / 4];
    __shared__ float4 pw[MEL_NB][MEL_FR / 4];
    const MelJob J = jobs[blockIdx.y];
    const int j0 = blockIdx.x * MEL_FR;
    if (j0 >= J.nf) return;
    const int tid = threadIdx.x;
    const int nfr = min(MEL_FR, J.nf - j0);
    const long long fbase = J.f0 + j0;

    float* xsf = reinterpret_cast<float*>(xs);
    for (int e = tid; e < MEL_FR * MEL_WIN; e += MEL_THREADS) {
        const int t = e / MEL_WIN, i = e - t * MEL_WIN;
        const long long f = fbase + t;
        float v = 0.0f;
        if (t < nfr && f < J.zero_from) {
            const long long idx = f * MEL_HOP - 200 + i;
            if (idx >= 0 && idx < J.n_audio) {
                const float a = J.src[idx - J.first];
                v = idx == 0 ? a : __fsub_rn(a, __fmul_rn(0.97f, J.src[idx - 1 - J.first]));
            }
        }
        xsf[i * MEL_FR + t] = v;
    }
    __syncthreads();

    {
        float re[MEL_FR], im[MEL_FR];
#pragma unroll
        for (int t = 0; t < MEL_FR; t++) re[t] = im[t] = 0.0f;
        const float* tc = tb.tab + tid;
#pragma unroll 8
        for (int n = 0; n < MEL_WIN; n++) {
            const float c = tc[n * 512], s = tc[n * 512 + 256];
#pragma unroll
            for (int q = 0; q < MEL_FR / 4; q++) {
                const float4 x = xs[n][q];
                re[4 * q + 0] = fmaf(c, x.x, re[4 * q + 0]); im[4 * q + 0] = fmaf(s, x.x, im[4 * q + 0]);
                re[4 * q + 1] = fmaf(c, x.y, re[4 * q + 1]); im[4 * q + 1] = fmaf(s, x.y, im[4 * q + 1]);
                re[4 * q + 2] = fmaf(c, x.z, re[4 * q + 2]); im[4 * q + 2] = fmaf(s, x.z, im[4 * q + 2]);
                re[4 * q + 3] = fmaf(c, x.w, re[4 * q + 3]); im[4 * q + 3] = fmaf(s, x.w, im[4 * q + 3]);
            }
        }
#pragma unroll
        for (int q = 0; q < MEL_FR / 4; q++)
            pw[tid][q] = make_float4(mel_power(re[4 * q], im[4 * q]), mel_power(re[4 * q + 1], im[4 * q + 1]),
                                     mel_power(re[4 * q + 2], im[4 * q + 2]), mel_power(re[4 * q + 3], im[4 * q + 3]));
    }
    {
        // bin 256: frame t = tid / 32, lane l of 32 takes samples l, l + 32, ...; butterfly over
        // the 32 lanes (xor offsets below 32 stay inside each half of the wave)
        const int t = tid >> 5, l = tid & 31;
        float r = 0.0f, q = 0.0f;
        for (int n = l; n < MEL_WIN; n += 32) {
            const float x = xsf[n * MEL_FR + t];
            r = fmaf(tb.nyq[n], x, r);
            q = fmaf(tb.nyq[MEL_WIN + n], x, q);
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            r += __shfl_xor(r, o);
            q += __shfl_xor(q, o);
        }
        if (l == 0) reinterpret_cast<float*>(pw[256])[t] = mel_power(r, q);
    }
    __syncthreads();

    const int quad = tid >> 7;   // frames 4 quad .. 4 quad + 3
    for (int m = tid & 127; m < tb.n_mels; m += 128) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* w = tb.fbT + m;
#pragma unroll 8
        for (int k = 0; k < MEL_NB; k++) {
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
    dim3 grid((max_nf + MEL_FR - 1) / MEL_FR, n_jobs);
    mel_kernel<<<grid, MEL_THREADS, 0, st>>>(jobs_dev, t);
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

struct ud_mel {
    int n_mels = 0;
    float *tab = nullptr, *nyq = nullptr, *fbT = nullptr;
    MelJob* djobs = nullptr;     // device job list of ud_mel_features
    MelJob* hjobs = nullptr;     // pinned staging of it
    int cap_jobs = 0;
    hipEvent_t copied = nullptr;  // the last job upload; the staging is rewritten only after it
};

namespace ud {
MelTables mel_tables_of(const ::ud_mel* m) { return MelTables{m->tab, m->nyq, m->fbT, m->n_mels}; }
}  // namespace ud

static void free_mel(ud_mel* m) {
    if (!m) return;
    (void)hipDeviceSynchronize();
    for (void* p : {(void*)m->tab, (void*)m->nyq, (void*)m->fbT, (void*)m->djobs}) if (p) (void)hipFree(p);
    if (m->hjobs) (void)hipHostFree(m->hjobs);
    if (m->copied) (void)hipEventDestroy(m->copied);
    delete m;
}

extern "C" UD_API int ud_mel_create(const float* fb_host, int32_t n_mels, const float* window_host, ud_mel** out) {
    if (!out || !fb_host || !window_host) return mfail(UD_ERR_INVALID, "ud_mel_create: null argument");
    *out = nullptr;
    if (n_mels < 1 || n_mels > 256) return mfail(UD_ERR_SHAPE, "ud_mel_create: n_mels %d outside 1..256", n_mels);
    // Tables as NemoMel.swift:28-39 builds them: phase in double, float(cos) * window in float.
    const int off = (512 - MEL_WIN) / 2;
    std::vector<float> tab((size_t)MEL_WIN * 512), nyq(2 * MEL_WIN), fbT((size_t)MEL_NB * n_mels);
    for (int k = 0; k < MEL_NB; k++)
        for (int n = 0; n < MEL_WIN; n++) {
            const double phase = 2.0 * 3.14159265358979323846 * (double)k * (double)(n + off) / 512.0;
            const float c = (float)cos(phase) * window_host[n];
            const float s = (float)(-sin(phase)) * window_host[n];
            if (k < 256) {
                tab[(size_t)n * 512 + k] = c;
                tab[(size_t)n * 512 + 256 + k] = s;
            } else {
                nyq[n] = c;
                nyq[MEL_WIN + n] = s;
            }
        }
    for (int m = 0; m < n_mels; m++)
        for (int k = 0; k < MEL_NB; k++) fbT[(size_t)k * n_mels + m] = fb_host[(size_t)m * MEL_NB + k];
    ud_mel* m = new ud_mel();
    m->n_mels = n_mels;
    bool ok = hipMalloc(&m->tab, tab.size() * 4) == hipSuccess && hipMalloc(&m->nyq, nyq.size() * 4) == hipSuccess &&
              hipMalloc(&m->fbT, fbT.size() * 4) == hipSuccess && hipEventCreateWithFlags(&m->copied, hipEventDisableTiming) == hipSuccess;
    ok = ok && hipMemcpy(m->tab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(m->nyq, nyq.data(), nyq.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(m->fbT, fbT.data(), fbT.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
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
        (void)hipEventSynchronize(m->copied);
        if (m->djobs) (void)hipFree(m->djobs);
        if (m->hjobs) (void)hipHostFree(m->hjobs);
        m->djobs = nullptr;
        m->hjobs = nullptr;
        m->cap_jobs = 0;
        if (hipMalloc(&m->djobs, (size_t)n * sizeof(MelJob)) != hipSuccess ||
            hipHostMalloc((void**)&m->hjobs, (size_t)n * sizeof(MelJob)) != hipSuccess)
            return mfail(UD_ERR_NOMEM, "ud_mel_features: job list allocation failed");
        m->cap_jobs = n;
    }
    if (hipEventSynchronize(m->copied) != hipSuccess) return mfail(UD_ERR_HIP, "ud_mel_features: event wait failed");
    for (int b = 0; b < n; b++) {
        const int64_t ns = n_samples_host[b];
        MelJob& j = m->hjobs[b];
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
    if (hipMemcpyAsync(m->djobs, m->hjobs, (size_t)n * sizeof(MelJob), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipEventRecord(m->copied, st) != hipSuccess)
        return mfail(UD_ERR_HIP, "ud_mel_features: job upload failed");
    const int rc = launch_mel(mel_tables_of(m), m->djobs, n, max_nf, st);
    if (rc != 0) return mfail(rc == -2 ? UD_ERR_SHAPE : UD_ERR_HIP, "ud_mel_features: launch failed");
    return UD_OK;
}
