// GEMMs of the encoder step, C = epilogue(A[M,K] . W[N,K]^T), W in the checkpoint's [out, in]
// orientation (Sources/DictatorEngine/Core/Kernels.swift:79-112; epilogue order of
// Sources/DictatorEngine/Metal/12_gemm2.metal:111-122: act, then out_scale, then + residual).
//
// bf16 path: v_mfma_f32_16x16x32_bf16 (gfx950).  The streaming step multiplies M = streams x T
// rows (128 at 64 streams x 2 frames) against 2-8 MB weight matrices.  Measured on MI355X, the
// limit at this shape is not HBM but the L2 -> CU traffic of the activation fragments, which every
// column tile re-reads; so both operands are stored fragment-major (see frag_index): each operand
// fragment is one contiguous 1 KB load, with no partially used cache lines.
//  - each wave owns a [16*MT x 16*NT] output tile (shapes per GEMM in launch_bf16)
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

template <int MT, int NT>
struct Frag {
    uint4 a[MT][2];
    uint4 b[NT][2];
};

template <int MT, int NT>
__device__ __forceinline__ void load_frag(Frag<MT, NT>& f, const bf16* const* ap, const bf16* const* wp, int64_t off) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        f.a[mt][0] = ld16(ap[mt] + off);
        f.a[mt][1] = ld16(ap[mt] + off + 512);
    }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        f.b[nt][0] = ld16(wp[nt] + off);
        f.b[nt][1] = ld16(wp[nt] + off + 512);
    }
}

template <int MT, int NT>
__device__ __forceinline__ void mma_frag(const Frag<MT, NT>& f, f32x4_t (&acc)[NT][MT]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(f.a[mt][h]), as_bf16x8(f.b[nt][h]),
                                                                      acc[nt][mt], 0, 0, 0);
}

// Grid: (N/16) x ceil(M/(16*MT)) x ksplit workgroups of WK waves.  The host guarantees
// K % (64 * WK * ksplit) == 0.  The epilogue kind and activation are template parameters: a
// runtime-switched, fully unrolled epilogue measured ~3.5 us slower per launch on MI355X (its
// code does not stay in the instruction cache).
template <int MT, int WK, int EPI, int ACT, int NT>
__global__ __launch_bounds__(64 * WK, 1) void gemm_bf16_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int nN = a.N / (16 * NT), nM = (a.M + 16 * MT - 1) / (16 * MT);
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
    const bf16* wp[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) wp[j] = W + (((int64_t)(nt * NT + j) * nk + kc0) << 10) + lane * 8;

    f32x4_t acc[NT][MT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[j][mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int cnt = kper / WK;            // chunks per wave (>= 1)
    constexpr int STEP = WK * 1024;       // element stride between a wave's consecutive chunks
    auto off = [&](int i) { return (int64_t)i * STEP; };
    Frag<MT, NT> f0, f1;
    load_frag(f0, ap, wp, off(0));
    int i = 0;
    for (; i + 2 < cnt; i += 2) {
        load_frag(f1, ap, wp, off(i + 1));
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f0, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_frag(f0, ap, wp, off(i + 2));
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f1, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (i + 1 < cnt) {
        load_frag(f1, ap, wp, off(i + 1));
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f0, acc);
        __builtin_amdgcn_sched_barrier(0);
        mma_frag(f1, acc);
    } else {
        mma_frag(f0, acc);
    }

    if constexpr (WK > 1) {
        __shared__ f32x4_t red[WK - 1][NT][MT][64];
        if (wave > 0) {
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) red[wave - 1][j][mt][lane] = acc[j][mt];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < WK - 1; w++)
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) acc[j][mt] += red[w][j][mt][lane];
    }

    // Lane holds rows 16*(mb*MT + mt) + 4*g + i (i < 4) of column 16*(nt*NT + j) + r16.
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int n = (nt * NT + j) * 16 + r16;
#pragma unroll
        for (int i2 = 0; i2 < 4; i2++) {
            const int64_t m = (int64_t)(mb * MT + mt) * 16 + g * 4 + i2;
            if (m >= a.M) continue;
            const float v = acc[j][mt][i2];
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

template <int MT, int WK, int NT, int EPI, int ACT>
static int launch_bf16_cfg(GemmArgs a, int ksplit, hipStream_t st) {
    if (a.N % (16 * NT) != 0 || ksplit < 1 || a.K % (64 * WK * ksplit) != 0) return -2;
    if (ksplit > 1 && EPI != EPI_PARTIAL) return -2;
    if (EPI == EPI_STORE_FRAG && a.N % 64 != 0) return -2;
    a.ksplit = ksplit;
    const int tiles = (a.N / (16 * NT)) * ((a.M + 16 * MT - 1) / (16 * MT)) * ksplit;
    hipLaunchKernelGGL((gemm_bf16_kernel<MT, WK, EPI, ACT, NT>), dim3(tiles), dim3(64 * WK), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int MT, int WK, int NT, int EPI>
static int launch_act(const GemmArgs& a, int ks, hipStream_t st) {
    if (a.act == ACT_SILU) return launch_bf16_cfg<MT, WK, NT, EPI, ACT_SILU>(a, ks, st);
    if (a.act == ACT_NONE) return launch_bf16_cfg<MT, WK, NT, EPI, ACT_NONE>(a, ks, st);
    return -2;
}

// Tile shapes measured on MI355X for the streaming step's M <= 128 projections (weights from HBM):
// every column tile re-reads its rows of the activation panel, so the output tile of a wave trades
// rows for columns (MT x NT tiles of 16 x 16) to cut that traffic.
//   ff linear1 (N 4096, K 1024, fragment out):   MT 2 x NT 4, 2 waves    9.0 -> 7.7 us
//   q/k/v (N 3072) and pointwise_conv1 (N 2048): MT 4 x NT 2, 4 waves    7.8 -> 6.8 us
//   split-K 4, K >= 4096 (ff linear2):           MT 4 x NT 2, 4 waves    7.8 -> 6.5 us
//   split-K 4, K 1024 (linear_out, pw2):         MT 4 x NT 1, 2 waves    5.0 -> 3.7 us
// Larger M keeps 128-row tiles (MT 8, 2 waves).
static int launch_bf16(const GemmArgs& a, int ks, hipStream_t st) {
    if (a.M <= 128) {
        switch (a.epi) {
            case EPI_STORE_FRAG:
                if (a.N % 64 == 0) return launch_act<2, 2, 4, EPI_STORE_FRAG>(a, ks, st);
                break;
            case EPI_STORE:
                if (a.N % 32 == 0 && a.K % 256 == 0) return launch_act<4, 4, 2, EPI_STORE>(a, ks, st);
                break;
            case EPI_STORE_F32:
                if (a.N % 32 == 0 && a.K % 256 == 0) return launch_act<4, 4, 2, EPI_STORE_F32>(a, ks, st);
                break;
            case EPI_PARTIAL:
                if (a.act != ACT_NONE) return -2;
                if (a.K >= 4096 && a.N % 32 == 0 && a.K % (256 * ks) == 0)
                    return launch_bf16_cfg<4, 4, 2, EPI_PARTIAL, ACT_NONE>(a, ks, st);
                if (a.K % (128 * ks) == 0) return launch_bf16_cfg<4, 2, 1, EPI_PARTIAL, ACT_NONE>(a, ks, st);
                break;
            default: return -2;   // the residual accumulate is an fp32-path epilogue
        }
    }
    switch (a.epi) {
        case EPI_PARTIAL: return a.act == ACT_NONE ? launch_bf16_cfg<8, 2, 1, EPI_PARTIAL, ACT_NONE>(a, ks, st) : -2;
        case EPI_STORE_F32: return launch_act<8, 2, 1, EPI_STORE_F32>(a, ks, st);
        case EPI_STORE_FRAG: return launch_act<8, 2, 1, EPI_STORE_FRAG>(a, ks, st);
        case EPI_STORE: return launch_act<8, 2, 1, EPI_STORE>(a, ks, st);
        default: return -2;
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
    return launch_bf16(a, a.epi == EPI_PARTIAL ? a.ksplit : 1, st);
}

}  // namespace ud
