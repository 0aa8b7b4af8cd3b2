// GEMMs of the encoder step, C = epilogue(A[M,K] . W[N,K]^T), W in the checkpoint's [out, in]
// layout (Sources/DictatorEngine/Core/Kernels.swift:79-112; epilogue order of
// Sources/DictatorEngine/Metal/12_gemm2.metal:111-122: act, then out_scale, then + residual).
//
// bf16 path: v_mfma_f32_16x16x32_bf16 (gfx950).  The streaming step multiplies M = streams x T
// rows (128 at 64 streams x 2 frames) against 2-8 MB weight matrices, so it is bound by streaming
// W from HBM.  Each wave owns a [16*MT x 16*NTL] output tile and a strided subset of the 64-wide
// K chunks; A and W fragments are loaded straight from global memory into MFMA operand registers
// (16 bytes per lane per operand half), double-buffered so the next chunk's loads are in flight
// while the current chunk's MFMAs run.  The WK waves of a workgroup split K and are summed through
// LDS.  Both operands use the same k permutation inside a 64-chunk (lane group g holds k in
// [16g, 16g+16) as two 8-element halves), which leaves the dot products unchanged.
//
// Epilogues are fused: SiLU + bf16 store (FF linear1), plain store (QKV), in-place fp32 residual
// accumulate (FF linear2 x0.5, linear_out, pointwise_conv2), and GLU with the frame mask
// (pointwise_conv1, whose weight rows are interleaved in 16-row value/gate blocks on upload so
// that a value column and its gate column sit in the same lane of two adjacent MFMA tiles).
#include "ud_common.hpp"
#include "kernels.hpp"

namespace ud {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
    bf16x8_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// Maps the linear workgroup id so that tiles t, t+1, ... of one XCD's share are contiguous
// (workgroups are dealt round-robin to the 8 XCDs): the M tiles of one N tile then run on the
// same XCD and reuse the W tile from its L2.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
    if (total % 8 != 0) return bid;
    return (bid % 8) * (total / 8) + bid / 8;
}

template <int MT, int NTL>
struct Frag {
    uint4 a[MT][2];
    uint4 b[NTL][2];
};

template <int MT, int NTL>
__device__ __forceinline__ void load_frag(Frag<MT, NTL>& f, const bf16* const* ap, const bool* aok,
                                          const bf16* const* wp, int k) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        if (aok[mt]) {
            f.a[mt][0] = ld16(ap[mt] + k);
            f.a[mt][1] = ld16(ap[mt] + k + 8);
        } else {
            f.a[mt][0] = make_uint4(0, 0, 0, 0);
            f.a[mt][1] = make_uint4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int nt = 0; nt < NTL; nt++) {
        f.b[nt][0] = ld16(wp[nt] + k);
        f.b[nt][1] = ld16(wp[nt] + k + 8);
    }
}

template <int MT, int NTL>
__device__ __forceinline__ void mma_frag(const Frag<MT, NTL>& f, f32x4_t (&acc)[MT][NTL]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NTL; nt++)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(f.a[mt][h]), as_bf16x8(f.b[nt][h]),
                                                                     acc[mt][nt], 0, 0, 0);
}

template <int MT, int NTL, int WK>
__global__ __launch_bounds__(64 * WK) void gemm_bf16_kernel(GemmArgs a) {
    constexpr int BM = 16 * MT, BN = 16 * NTL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int nN = a.N / BN, nM = (a.M + BM - 1) / BM;
    const int t = xcd_tile(blockIdx.x, nN * nM);
    const int n0 = (t / nM) * BN, m0 = (t % nM) * BM;

    const bf16* A = static_cast<const bf16*>(a.A);
    const bf16* W = static_cast<const bf16*>(a.W);
    const bf16* ap[MT];
    bool aok[MT];
    const bf16* wp[NTL];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        int m = m0 + mt * 16 + r16;
        aok[mt] = m < a.M;
        ap[mt] = A + (int64_t)(aok[mt] ? m : 0) * a.lda + g * 16;
    }
#pragma unroll
    for (int nt = 0; nt < NTL; nt++) wp[nt] = W + (int64_t)(n0 + nt * 16 + r16) * a.ldw + g * 16;

    f32x4_t acc[MT][NTL];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NTL; nt++) acc[mt][nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int nchunks = a.K / 64;
    Frag<MT, NTL> f0, f1;
    int c = wave;
    if (c < nchunks) load_frag(f0, ap, aok, wp, c * 64);
    while (c < nchunks) {
        int cn = c + WK;
        if (cn < nchunks) load_frag(f1, ap, aok, wp, cn * 64);
        mma_frag(f0, acc);
        c = cn;
        if (c >= nchunks) break;
        cn = c + WK;
        if (cn < nchunks) load_frag(f0, ap, aok, wp, cn * 64);
        mma_frag(f1, acc);
        c = cn;
    }

    if constexpr (WK > 1) {
        __shared__ f32x4_t red[WK - 1][MT][NTL][64];
        if (wave > 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NTL; nt++) red[wave - 1][mt][nt][lane] = acc[mt][nt];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < WK - 1; w++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NTL; nt++) acc[mt][nt] += red[w][mt][nt][lane];
    }

    // Lane holds rows m0 + 16*mt + 4*g + i (i < 4) of column n0 + 16*nt + r16.
    if (a.epi == EPI_GLU) {
        float* C = static_cast<float*>(a.C);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int p = 0; p < NTL / 2; p++) {
                const int ch = n0 / 2 + 16 * p + r16;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = m0 + mt * 16 + g * 4 + i;
                    if (m >= a.M) continue;
                    const int s = m / a.T, tt = m - s * a.T;
                    const int valid = a.desc[s * DESC_INTS + 2];
                    float y = acc[mt][2 * p][i] * sigmoidf(acc[mt][2 * p + 1][i]);
                    C[(int64_t)m * a.ldc + ch] = tt < valid ? y : 0.0f;
                }
            }
        return;
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NTL; nt++) {
            const int n = n0 + nt * 16 + r16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + mt * 16 + g * 4 + i;
                if (m >= a.M) continue;
                const float v = acc[mt][nt][i];
                if (a.epi == EPI_RESID) {
                    float* C = static_cast<float*>(a.C) + (int64_t)m * a.ldc + n;
                    *C = *C + a.out_scale * v;
                } else if (a.epi == EPI_STORE_F32) {
                    static_cast<float*>(a.C)[(int64_t)m * a.ldc + n] = apply_act(v, a.act) * a.out_scale;
                } else {
                    static_cast<bf16*>(a.C)[(int64_t)m * a.ldc + n] = f2bf(apply_act(v, a.act) * a.out_scale);
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

template <int MT, int NTL, int WK>
static int launch_bf16_cfg(const GemmArgs& a, hipStream_t st) {
    constexpr int BM = 16 * MT, BN = 16 * NTL;
    if (a.N % BN != 0) return -2;
    const int tiles = (a.N / BN) * ((a.M + BM - 1) / BM);
    hipLaunchKernelGGL((gemm_bf16_kernel<MT, NTL, WK>), dim3(tiles), dim3(64 * WK), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_gemm(const GemmArgs& a, bool bf16_data, hipStream_t st) {
    if (a.M <= 0 || a.N <= 0 || a.K <= 0) return -2;
    if (!bf16_data) {
        if (a.epi == EPI_GLU) return -2;
        dim3 grid((a.N + F_BN - 1) / F_BN, (a.M + F_BM - 1) / F_BM);
        hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, st, a);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    // bf16 MFMA: K in 64-chunks, 16-byte aligned rows.
    if (a.K % 64 != 0 || a.lda % 8 != 0 || a.ldw % 8 != 0) return -2;
    if (a.epi == EPI_GLU && a.N % 32 != 0) return -2;
    // Skinny (streaming) shapes: full M in one tile when M <= 128; 32 output columns per
    // workgroup, K split over 4 waves.
    if (a.M <= 64) return launch_bf16_cfg<4, 2, 4>(a, st);
    return launch_bf16_cfg<8, 2, 4>(a, st);
}

}  // namespace ud
