// Causal dw_striding 8x subsampling of the streaming step (FastConformer.swift:219-243 encodeSubsampling;
// Metal/20_conformer.metal:104-138 conv2d_cl; NeMo ConvSubsampling as in docs/specs/nemotron.md:52-81),
// batched over streams.  Activations are channel-last [stream, time, freq, C = 256]; every stride-2
// stage is a 3 x 3 causal conv with 2 zero rows/columns of top/left padding, L -> L/2 + 1.
//
//   conv.0 (1 -> C) + ReLU, rows >= v1 zero     } sub_conv01_kernel: conv.0's outputs live in a
//   conv.2 (depthwise)                          } register window per channel, so its
//                                                 T1 x 65 x 256 activation never reaches HBM
//   conv.3 (pointwise) + ReLU                   GEMM (bias epilogue); fp32 out, or half for a
//                                               16-bit encoder
//   rows >= v2 zero; conv.5 (depthwise)         sub_dw_kernel (mask applied on read; 4 channels
//                                               of one position per thread, one round trip)
//   conv.6 (pointwise) + ReLU                   GEMM; fp32 out, then
//   rows >= v3 zero; drop; flatten (f, c)       sub_flatten_kernel -> rows of the out Linear's A;
//                                               a 16-bit encoder's conv.6 GEMM writes those rows
//                                               itself (EPI_SUBFLAT epilogue: flatten, mask, drop)
//   out Linear (C*F3 -> D) + bias               GEMM, fp32 out = the encoder's input rows
//
// The GEMM operands (conv.3 / conv.6 inputs, the flattened rows) are written in the GEMM's A
// layout: for a bf16 encoder fragment-major IEEE half (the front-end GEMMs run on the f16 MFMA:
// 11-bit mantissas, where the reference keeps these convolutions in fp32 and its out Linear in f16,
// Sources/DictatorEngine/Core/Convert.swift:74-83), row-major fp32 for an fp32 encoder.
#include "ud_common.hpp"
#include "kernels.hpp"

namespace ud {

constexpr int SUB_C = 256;

template <bool H>
__device__ __forceinline__ void store_a(void* A, int64_t m, int col, int cols, float v) {
    if constexpr (H) static_cast<uint16_t*>(A)[frag_index(m, col, cols / 64)] = f2h(v);
    else static_cast<float*>(A)[m * cols + col] = v;
}

// One workgroup per conv.2 output row (stream s, time t2); thread c = channel.  conv.2 output
// (t2, f2) reads conv.0's output at rows 2 t2 - 2 .. 2 t2 and columns 2 f2 - 2 .. 2 f2; conv.0 at
// (h, w) reads mel rows 2 h - 2 .. 2 h and columns 2 w - 2 .. 2 w.  The 7 mel rows 4 t2 - 6 ..
// 4 t2 sit in LDS with 3 zero columns of left padding (rows outside the chunk or >= v0 are zero).
// Along the row each thread keeps a 3 x 3 window of its channel's conv.0 outputs and the 7 x 5 mel
// values they need in registers: output position f2 adds conv.0 columns 2 f2 - 1 and 2 f2, which
// read mel columns 4 f2 - 4 .. 4 f2, of which 4 f2 - 3 .. 4 f2 are new -- one aligned 16-byte
// LDS read per mel row (patch column = mel column + 3).
// With NS > 1 the row's F2 positions are split into NS runs, one per group of SUB_C threads (for
// launches too small to fill the chip: the chain of positions is each thread's latency).  A run
// starting at p0 > 0 first computes position p0 - 1 without storing it: that iteration leaves the
// window's last conv.0 column (2 p0 - 2) and mel column 4 p0 - 4 where the next one expects them.
constexpr int SUB_PW = 132;       // 3 + 128 mel columns + 1, a multiple of 4

template <bool H, int NS>
__global__ __launch_bounds__(SUB_C * NS) void sub_conv01_kernel(SubArgs a) {
    const int c = NS == 1 ? threadIdx.x : threadIdx.x % SUB_C, run = NS == 1 ? 0 : threadIdx.x / SUB_C;
    const int t2 = blockIdx.x % a.T2, s = blockIdx.x / a.T2;
    const int v0 = a.vlen[s * 4 + 0], v1 = a.vlen[s * 4 + 1];
    __shared__ __align__(16) float patch[7][SUB_PW];
    for (int i = threadIdx.x; i < 7 * SUB_PW; i += SUB_C * NS) {
        const int pr = i / SUB_PW, q = i % SUB_PW - 3;
        const int r = 4 * t2 - 6 + pr;
        float v = 0.0f;
        if (r >= 0 && r < a.T0 && r < v0 && q >= 0 && q < a.F0) v = a.mel[((int64_t)s * a.T0 + r) * a.F0 + q];
        patch[pr][i % SUB_PW] = v;
    }
    float w0[9], w2[9];
#pragma unroll
    for (int k = 0; k < 9; k++) { w0[k] = a.c0w[c * 9 + k]; w2[k] = a.c2w[c * 9 + k]; }
    const float b0 = a.c0b[c], b2 = a.c2b[c];
    bool hv[3];
#pragma unroll
    for (int kh = 0; kh < 3; kh++) {
        const int h = 2 * t2 + kh - 2;
        hv[kh] = h >= 0 && h < a.T1 && h < v1;        // else padding or a masked row: zero
    }
    __syncthreads();
    // mel[r][j]: mel row 4 t2 - 6 + r, columns 4 f2 - 4 + j (j < 5) of the current position
    float mel[7][5];
#pragma unroll
    for (int r = 0; r < 7; r++) mel[r][4] = 0.0f;      // column -4 (read only by conv.0 column -1)
    // conv.0 + ReLU at (row 2 t2 + kh - 2, column w) from mel columns j0 .. j0 + 2 of the window
    auto conv0 = [&](int kh, int w, int j0) -> float {
        if (!hv[kh] || w < 0 || w >= a.F1) return 0.0f;
        float y = b0;
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
            for (int j = 0; j < 3; j++) y += w0[i * 3 + j] * mel[2 * kh + i][j0 + j];
        return y > 0.0f ? y : 0.0f;
    };
    float win[3][3];
#pragma unroll
    for (int kh = 0; kh < 3; kh++) win[kh][2] = 0.0f;     // column -2
    const int64_t row0 = ((int64_t)s * a.T2 + t2) * a.F2;
    const int per = (a.F2 + NS - 1) / NS, p0 = NS == 1 ? 0 : run * per, p1 = NS == 1 ? a.F2 : min(a.F2, p0 + per);
    for (int f2 = p0 > 0 ? p0 - 1 : 0; f2 < p1; f2++) {
#pragma unroll
        for (int r = 0; r < 7; r++) {
            const float4 v = *reinterpret_cast<const float4*>(&patch[r][4 * f2]);
            mel[r][0] = mel[r][4];
            mel[r][1] = v.x; mel[r][2] = v.y; mel[r][3] = v.z; mel[r][4] = v.w;
        }
        float acc = b2;
#pragma unroll
        for (int kh = 0; kh < 3; kh++) {
            win[kh][0] = win[kh][2];
            win[kh][1] = conv0(kh, 2 * f2 - 1, 0);
            win[kh][2] = conv0(kh, 2 * f2, 2);
#pragma unroll
            for (int kw = 0; kw < 3; kw++) acc += w2[kh * 3 + kw] * win[kh][kw];
        }
        if (NS == 1 || f2 >= p0) store_a<H>(a.out, row0 + f2, c, SUB_C, acc);
    }
}

// Depthwise 3 x 3 stride-2 causal conv over x [n, Hin, Win, C] (fp32, or IEEE half when H) whose
// rows >= vlen[s][stage] read as zero (the mask NeMo applies before this layer).  A thread computes 4 channels of one
// output position: its 9 taps are 16-byte loads issued together (one memory round trip per
// thread), its 36 weights 9 more; a workgroup covers 4 consecutive output columns of one output row
// (64 threads per column).  Each output column's 4 channels are one 16-byte (fp32) or 8-byte
// (half, fragment-major: 4 consecutive channels are contiguous) store.
constexpr int SUB_DW_COLS = 4;

template <bool H>
__global__ __launch_bounds__(SUB_C) void sub_dw_kernel(SubDwArgs a) {
    const int tid = threadIdx.x, c4 = (tid & 63) * 4, wsub = tid >> 6;
    const int ncg = (a.Wout + SUB_DW_COLS - 1) / SUB_DW_COLS;
    const int cg = blockIdx.x % ncg, ho = (blockIdx.x / ncg) % a.Hout, s = blockIdx.x / (ncg * a.Hout);
    const int wo = cg * SUB_DW_COLS + wsub;
    if (wo >= a.Wout) return;                     // no barrier below
    const int vin = a.vlen[s * 4 + a.stage];
    // weights [C][9]: channels c4 .. c4+3 are 36 consecutive floats (16-byte aligned)
    float w[4][9];
    {
        const float4* wp = reinterpret_cast<const float4*>(a.w + c4 * 9);
        float f[36];
#pragma unroll
        for (int k = 0; k < 9; k++) {
            const float4 x = wp[k];
            f[4 * k] = x.x; f[4 * k + 1] = x.y; f[4 * k + 2] = x.z; f[4 * k + 3] = x.w;
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int k = 0; k < 9; k++) w[e][k] = f[e * 9 + k];
    }
    const float4 bias = *reinterpret_cast<const float4*>(a.b + c4);
    // The loads are unconditional (row and column clamped into the input, Win >= 1) so all 9 issue
    // together; a padding tap or a masked row's tap is then replaced by zero with a select
    // (v_cndmask), so whatever the clamped load read -- NaN or Inf included -- never reaches the sum.
    float4 tap[3][3];
    uint2 tap16[3][3];
    bool ok[3][3];
#pragma unroll
    for (int kh = 0; kh < 3; kh++) {
        const int h = 2 * ho + kh - 2;
        const bool hv = h >= 0 && h < a.Hin && h < vin;
        const int64_t row = (((int64_t)s * a.Hin + min(max(h, 0), a.Hin - 1)) * a.Win) * SUB_C + c4;
#pragma unroll
        for (int kw = 0; kw < 3; kw++) {
            const int col = 2 * wo + kw - 2;
            ok[kh][kw] = hv && col >= 0 && col < a.Win;
            const int64_t at = row + (int64_t)min(max(col, 0), a.Win - 1) * SUB_C;
            if constexpr (H) tap16[kh][kw] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.x) + at);
            else tap[kh][kw] = *reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + at);
        }
    }
    if constexpr (H) {
#pragma unroll
        for (int kh = 0; kh < 3; kh++)
#pragma unroll
            for (int kw = 0; kw < 3; kw++) {
                const uint2 u = tap16[kh][kw];
                tap[kh][kw] = make_float4(half_lo(u.x), half_hi(u.x), half_lo(u.y), half_hi(u.y));
            }
    }
    float acc[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
    for (int kh = 0; kh < 3; kh++)
#pragma unroll
        for (int kw = 0; kw < 3; kw++) {
            const float4 t = tap[kh][kw];
            const float v[4] = {ok[kh][kw] ? t.x : 0.0f, ok[kh][kw] ? t.y : 0.0f, ok[kh][kw] ? t.z : 0.0f,
                                ok[kh][kw] ? t.w : 0.0f};
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] += w[e][kh * 3 + kw] * v[e];
        }
    const int64_t m = ((int64_t)s * a.Hout + ho) * a.Wout + wo;
    if constexpr (H) {
        const uint2 o = make_uint2((uint32_t)f2h(acc[0]) | ((uint32_t)f2h(acc[1]) << 16),
                                   (uint32_t)f2h(acc[2]) | ((uint32_t)f2h(acc[3]) << 16));
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + frag_index(m, c4, SUB_C / 64)) = o;
    } else {
        *reinterpret_cast<float4*>(static_cast<float*>(a.out) + m * SUB_C + c4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
}

// Rows of the out Linear: row (s, t) for t < T takes conv.6's output frame t3 = t + drop, zero when
// t3 >= v3 (NeMo's final mask), flattened as (freq, channel) -- the column order the out weight
// is permuted to at load.  One workgroup per row.
template <bool H>
__global__ __launch_bounds__(SUB_C) void sub_flatten_kernel(SubFlatArgs a) {
    const int c = threadIdx.x;
    const int row = blockIdx.x, s = row / a.T, t3 = row % a.T + a.drop;
    const bool valid = t3 < a.vlen[s * 4 + 3];
    const float* src = a.x + (((int64_t)s * a.T3 + t3) * a.F3) * SUB_C;
    for (int f = 0; f < a.F3; f++) {
        const float v = valid ? src[f * SUB_C + c] : 0.0f;
        store_a<H>(a.out, row, f * SUB_C + c, a.F3 * SUB_C, v);
    }
}

int launch_sub_conv01(const SubArgs& a, bool half, hipStream_t st) {
    // patch columns: mel + 3 up to F0 + 2; reads up to 4 F2 - 1
    if (a.F0 + 3 > SUB_PW || 4 * a.F2 > SUB_PW || a.F1 > 2 * a.F2) return -2;
    const int blocks = a.n * a.T2;
    if (blocks <= 0) return 0;
    // below ~4 workgroups per CU, two runs per row (the first position of the second run computed
    // twice)
    if (blocks < 1024) {
        if (half) hipLaunchKernelGGL((sub_conv01_kernel<true, 2>), dim3(blocks), dim3(2 * SUB_C), 0, st, a);
        else hipLaunchKernelGGL((sub_conv01_kernel<false, 2>), dim3(blocks), dim3(2 * SUB_C), 0, st, a);
    } else {
        if (half) hipLaunchKernelGGL((sub_conv01_kernel<true, 1>), dim3(blocks), dim3(SUB_C), 0, st, a);
        else hipLaunchKernelGGL((sub_conv01_kernel<false, 1>), dim3(blocks), dim3(SUB_C), 0, st, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_sub_dw(const SubDwArgs& a, bool half, hipStream_t st) {
    if (a.Win < 1 || a.Hin < 1 || a.Wout < 1) return -2;
    const int blocks = a.n * a.Hout * ((a.Wout + SUB_DW_COLS - 1) / SUB_DW_COLS);
    if (blocks <= 0) return 0;
    if (half) hipLaunchKernelGGL(sub_dw_kernel<true>, dim3(blocks), dim3(SUB_C), 0, st, a);
    else hipLaunchKernelGGL(sub_dw_kernel<false>, dim3(blocks), dim3(SUB_C), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_sub_flatten(const SubFlatArgs& a, bool half, hipStream_t st) {
    const int blocks = a.n * a.T;
    if (blocks <= 0) return 0;
    if (half) hipLaunchKernelGGL(sub_flatten_kernel<true>, dim3(blocks), dim3(SUB_C), 0, st, a);
    else hipLaunchKernelGGL(sub_flatten_kernel<false>, dim3(blocks), dim3(SUB_C), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ud
