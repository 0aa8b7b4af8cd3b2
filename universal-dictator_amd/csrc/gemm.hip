// GEMMs of the encoder step, C = epilogue(A[M,K] . W[N,K]^T), W in the checkpoint's [out, in]
// orientation (Sources/DictatorEngine/Core/Kernels.swift:79-112; epilogue order of
// Sources/DictatorEngine/Metal/12_gemm2.metal:111-122: act, then out_scale, then + residual).
//
// bf16 path: v_mfma_f32_16x16x32_bf16 (gfx950).  The streaming step multiplies M = streams x T
// rows (128 at 64 streams x 2 frames) against 2-8 MB weight matrices.  Measured on MI355X, the
// limit at this shape is not HBM but the L2 -> CU traffic of the activation fragments, which every
// column tile re-reads; so both operands are stored fragment-major (see frag_index): each operand
// fragment is one contiguous 1 KB load, with no partially used cache lines.
//  - each wave owns a [16*MT x 16] output tile (MT = 8: all 128 rows of a 64-stream chunk-2 step)
//    and every WK-th 64-wide K chunk of its workgroup's K range; the WK waves are summed in LDS;
//  - two register buffers, separated by scheduling barriers, keep the next chunk's loads in flight
//    behind the current chunk's MFMAs;
//  - ksplit > 1 splits K over workgroups (parallelism for the N = 1024 projections); each split
//    writes its own fp32 partial slab and the following LayerNorm adds the slabs, in order, to the
//    residual row it reads anyway -- deterministic, no atomics, no extra kernel.
// Epilogues: act + bf16 store (row-major for the QKV buffer the attention reads, fragment-major for
// a following GEMM), fp32 store, in-place fp32 residual accumulate, split-K partial slabs.
#include "ud_common.hpp"
#include "kernels.hpp"

namespace ud {

// Maps the linear workgroup id so that tiles t, t+1, ... of one XCD's share are contiguous
// (workgroups are dealt round-robin to the 8 XCDs): the M tiles and K splits of one N tile then
// run on the same XCD and share its L2.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
    if (total % 8 != 0) return bid;
    return (bid % 8) * (total / 8) + bid / 8;
}

template <int MT>
struct Frag {
    uint4 a[MT][2];
    uint4 b[2];
};

template <int MT>
__device__ __forceinline__ void load_frag(Frag<MT>& f, const bf16* const* ap, const bf16* wp, int64_t off) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        f.a[mt][0] = ld16(ap[mt] + off);
        f.a[mt][1] = ld16(ap[mt] + off + 512);
    }
    f.b[0] = ld16(wp + off);
    f.b[1] = ld16(wp + off + 512);
}

template <int MT>
__device__ __forceinline__ void mma_frag(const Frag<MT>& f, f32x4_t (&acc)[MT]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(f.a[mt][h]), as_bf16x8(f.b[h]), acc[mt], 0, 0, 0);
}

// Grid: (N/16) x ceil(M/(16*MT)) x ksplit workgroups of WK waves.  The host guarantees
// K % (64 * WK * ksplit) == 0.  The epilogue kind and activation are template parameters: a
// runtime-switched, fully unrolled epilogue measured ~3.5 us slower per launch on MI355X (its
// code does not stay in the instruction cache).
template <int MT, int WK, int EPI, int ACT>
__global__ __launch_bounds__(64 * WK, 1) void gemm_bf16_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int nN = a.N / 16, nM = (a.M + 16 * MT - 1) / (16 * MT);
    const int ks = a.ksplit;
    const int t = xcd_tile(blockIdx.x, nN * nM * ks);
    const int kz = t % ks, tile = t / ks;
    const int nt = tile / nM, mb = tile % nM;
    const int nk = a.K / 64;
    const int kper = nk / ks;
    const int kc0 = kz * kper + wave;
    const int rtiles = (a.M + 15) / 16;

    const bf16* A = static_cast<const bf16*>(a.A);
    const bf16* W = static_cast<const bf16*>(a.W);
    const bf16* ap[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int rt = min(mb * MT + mt, rtiles - 1);      // clamped tiles are computed, not stored
        ap[mt] = A + (((int64_t)rt * nk + kc0) << 10) + lane * 8;
    }
    const bf16* wp = W + (((int64_t)nt * nk + kc0) << 10) + lane * 8;

    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int cnt = kper / WK;            // chunks per wave (>= 1)
    constexpr int STEP = WK * 1024;       // element stride between a wave's consecutive chunks
    Frag<MT> f0, f1;
    load_frag(f0, ap, wp, 0);
    int i = 0;
    for (; i + 2 < cnt; i += 2) {
        load_frag(f1, ap, wp, (int64_t)(i + 1) * STEP);
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f0, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_frag(f0, ap, wp, (int64_t)(i + 2) * STEP);
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f1, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (i + 1 < cnt) {
        load_frag(f1, ap, wp, (int64_t)(i + 1) * STEP);
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f0, acc);
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f1, acc);
    } else {
        mma_frag(f0, acc);
    }

    if constexpr (WK > 1) {
        __shared__ f32x4_t red[WK - 1][MT][64];
        if (wave > 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) red[wave - 1][mt][lane] = acc[mt];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < WK - 1; w++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] += red[w][mt][lane];
    }

    // Lane holds rows 16*(mb*MT + mt) + 4*g + i (i < 4) of column 16*nt + r16.
    const int n = nt * 16 + r16;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int i2 = 0; i2 < 4; i2++) {
            const int64_t m = (int64_t)(mb * MT + mt) * 16 + g * 4 + i2;
            if (m >= a.M) continue;
            const float v = acc[mt][i2];
            if constexpr (EPI == EPI_PARTIAL) {
                static_cast<float*>(a.C)[((int64_t)kz * a.M + m) * a.ldc + n] = a.out_scale * v;
            } else if constexpr (EPI == EPI_STORE_F32) {
                static_cast<float*>(a.C)[m * a.ldc + n] = apply_act(v, ACT) * a.out_scale;
            } else if constexpr (EPI == EPI_STORE_FRAG) {
                static_cast<bf16*>(a.C)[frag_index(m, n, a.N / 64)] = f2bf(apply_act(v, ACT) * a.out_scale);
            } else {
                static_cast<bf16*>(a.C)[m * a.ldc + n] = f2bf(apply_act(v, ACT) * a.out_scale);
            }
        }
    }
}

// ---------------------------------------------------------------- fp32 (VALU) GEMM
// 64x64 tiles, 256 threads with 4x4 outputs each, K staged through LDS in slices of 16.
constexpr int F_BM = 64, F_BN = 64, F_BK = 16;

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs a) {
    __shared__ float As[F_BK][F_BM + 4];
    __shared__ float Ws[F_BK][F_BN + 4];
    const float* A = static_cast<const float*>(a.A);
    const float* W = static_cast<const float*>(a.W);
    const int tid = threadIdx.x;
    const int m0 = blockIdx.y * F_BM, n0 = blockIdx.x * F_BN;
    const int tm = (tid / 16) * 4, tn = (tid % 16) * 4;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < a.K; k0 += F_BK) {
        for (int idx = tid; idx < F_BM * F_BK; idx += 256) {
            int r = idx / F_BK, kk = idx % F_BK;
            int m = m0 + r, n = n0 + r, k = k0 + kk;
            As[kk][r] = (m < a.M && k < a.K) ? A[(int64_t)m * a.lda + k] : 0.0f;
            Ws[kk][r] = (n < a.N && k < a.K) ? W[(int64_t)n * a.ldw + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < F_BK; kk++) {
            float av[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) { av[i] = As[kk][tm + i]; wv[i] = Ws[kk][tn + i]; }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] += av[i] * wv[j];
        }
        __syncthreads();
    }
    for (int i = 0; i < 4; i++) {
        int m = m0 + tm + i;
        if (m >= a.M) continue;
        for (int j = 0; j < 4; j++) {
            int n = n0 + tn + j;
            if (n >= a.N) continue;
            float* C = static_cast<float*>(a.C) + (int64_t)m * a.ldc + n;
            if (a.epi == EPI_RESID) *C = *C + a.out_scale * acc[i][j];
            else *C = apply_act(acc[i][j], a.act) * a.out_scale;
        }
    }
}

// ---------------------------------------------------------------- launch

template <int MT, int WK, int EPI, int ACT>
static int launch_bf16_cfg(GemmArgs a, int ksplit, hipStream_t st) {
    if (a.N % 16 != 0 || ksplit < 1 || a.K % (64 * WK * ksplit) != 0) return -2;
    if (ksplit > 1 && EPI != EPI_PARTIAL) return -2;
    if (EPI == EPI_STORE_FRAG && a.N % 64 != 0) return -2;
    a.ksplit = ksplit;
    const int tiles = (a.N / 16) * ((a.M + 16 * MT - 1) / (16 * MT)) * ksplit;
    hipLaunchKernelGGL((gemm_bf16_kernel<MT, WK, EPI, ACT>), dim3(tiles), dim3(64 * WK), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int MT>
static int launch_bf16_mt(const GemmArgs& a, int ks, hipStream_t st) {
    const bool silu = a.act == ACT_SILU;
    if (a.act != ACT_NONE && !silu) return -2;
    switch (a.epi) {
        case EPI_PARTIAL: return silu ? -2 : launch_bf16_cfg<MT, 2, EPI_PARTIAL, ACT_NONE>(a, ks, st);
        case EPI_STORE_F32: return silu ? launch_bf16_cfg<MT, 2, EPI_STORE_F32, ACT_SILU>(a, ks, st)
                                        : launch_bf16_cfg<MT, 2, EPI_STORE_F32, ACT_NONE>(a, ks, st);
        case EPI_STORE_FRAG: return silu ? launch_bf16_cfg<MT, 2, EPI_STORE_FRAG, ACT_SILU>(a, ks, st)
                                         : launch_bf16_cfg<MT, 2, EPI_STORE_FRAG, ACT_NONE>(a, ks, st);
        case EPI_STORE: return silu ? launch_bf16_cfg<MT, 2, EPI_STORE, ACT_SILU>(a, ks, st)
                                    : launch_bf16_cfg<MT, 2, EPI_STORE, ACT_NONE>(a, ks, st);
        default: return -2;   // the residual accumulate is an fp32-path epilogue
    }
}

int launch_gemm(const GemmArgs& a, bool bf16_data, hipStream_t st) {
    if (a.M <= 0 || a.N <= 0 || a.K <= 0) return -2;
    if (!bf16_data) {
        if (a.epi == EPI_STORE_FRAG) return -2;
        dim3 grid((a.N + F_BN - 1) / F_BN, (a.M + F_BM - 1) / F_BM);
        hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, st, a);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (a.K % 128 != 0) return -2;
    // One workgroup per 16-column tile (and K split for EPI_PARTIAL), two waves splitting K.
    const int ks = a.epi == EPI_PARTIAL ? a.ksplit : 1;
    if (a.M <= 64) return launch_bf16_mt<4>(a, ks, st);
    return launch_bf16_mt<8>(a, ks, st);
}

}  // namespace ud
