// Row-wise kernels of the encoder step: LayerNorm (single and fused pair) and the conv module's
// GLU + frame mask + causal depthwise conv + LayerNorm + SiLU, fused with the conv-cache ring.
// 16-bit outputs (IEEE half, a 16-bit encoder's activation format) feed a GEMM and are written
// fragment-major (frag_index); fp32 outputs row-major.
//
// LayerNorm semantics: Sources/DictatorEngine/Metal/20_conformer.metal:25-49 (two passes,
// population variance, y = act((x-mean)*rsqrt(var+eps)*g + b)), eps 1e-5 (Core/Ops.swift:27).
// One wave64 per row: the row lives in registers (D/64 values per lane, 16-byte loads), so the
// two passes cost one HBM read and one write.
#include "ud_common.hpp"
#include "kernels.hpp"

namespace ud {

constexpr float LN_EPS = 1e-5f;

template <int NPER>
__device__ __forceinline__ void ln_row_stats(const float4 (&x)[NPER], int D, float& mean, float& rstd) {
    float s = 0.0f;
#pragma unroll
    for (int p = 0; p < NPER; p++) s += (x[p].x + x[p].y) + (x[p].z + x[p].w);
    mean = wave_sum(s) / (float)D;
    float v = 0.0f;
#pragma unroll
    for (int p = 0; p < NPER; p++) {
        float a = x[p].x - mean, b = x[p].y - mean, c = x[p].z - mean, d = x[p].w - mean;
        v += (a * a + b * b) + (c * c + d * d);
    }
    rstd = 1.0f / sqrtf(wave_sum(v) / (float)D + LN_EPS);
}

// gamma / beta of this lane's columns, loaded up front (independent of the row data)
template <int NPER>
__device__ __forceinline__ void ln_params(float4 (&gg)[NPER], float4 (&bb)[NPER], const float* __restrict__ g,
                                          const float* __restrict__ b, int lane) {
#pragma unroll
    for (int p = 0; p < NPER; p++) {
        const int c = (p * 64 + lane) * 4;
        gg[p] = *reinterpret_cast<const float4*>(g + c);
        bb[p] = *reinterpret_cast<const float4*>(b + c);
    }
}

template <int NPER>
__device__ __forceinline__ void ln_apply(float4 (&x)[NPER], const float4 (&gg)[NPER], const float4 (&bb)[NPER],
                                         float mean, float rstd, int act) {
#pragma unroll
    for (int p = 0; p < NPER; p++) {
        x[p].x = apply_act((x[p].x - mean) * rstd * gg[p].x + bb[p].x, act);
        x[p].y = apply_act((x[p].y - mean) * rstd * gg[p].y + bb[p].y, act);
        x[p].z = apply_act((x[p].z - mean) * rstd * gg[p].z + bb[p].z, act);
        x[p].w = apply_act((x[p].w - mean) * rstd * gg[p].w + bb[p].w, act);
    }
}

// Four consecutive columns c..c+3 (c % 4 == 0) of row `row`: IEEE half fragment-major, 8 bytes.
__device__ __forceinline__ void store4_frag(void* out, int64_t row, int c, int D, float4 v) {
    uint2 u;
    u.x = (uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16);
    u.y = (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + frag_index(row, c, D / 64)) = u;
}

template <int NPER>
__device__ __forceinline__ void store_row(void* out, bool bf, int64_t row, int D, const float4 (&x)[NPER], int lane) {
#pragma unroll
    for (int p = 0; p < NPER; p++) {
        const int c = (p * 64 + lane) * 4;
        if (bf) {
            store4_frag(out, row, c, D, x[p]);
        } else {
            *reinterpret_cast<float4*>(static_cast<float*>(out) + row * D + c) = x[p];
        }
    }
}

// v = row of x plus the pending split-K residual slabs, added in slab order.  NP = number of slabs
// known at compile time (all loads issued before the first add), or -1 for a count known only at
// run time.
template <int NPER, int NP>
__device__ __forceinline__ void load_row(float4 (&v)[NPER], const float* __restrict__ x, Partials parts, int64_t row,
                                         int rows, int D, int lane) {
#pragma unroll
    for (int p = 0; p < NPER; p++) v[p] = *reinterpret_cast<const float4*>(x + row * D + (p * 64 + lane) * 4);
    if constexpr (NP > 0) {
        float4 q[NP][NPER];
#pragma unroll
        for (int j = 0; j < NP; j++)
#pragma unroll
            for (int p = 0; p < NPER; p++)
                q[j][p] = *reinterpret_cast<const float4*>(parts.p + ((int64_t)j * rows + row) * D + (p * 64 + lane) * 4);
#pragma unroll
        for (int j = 0; j < NP; j++)
#pragma unroll
            for (int p = 0; p < NPER; p++) { v[p].x += q[j][p].x; v[p].y += q[j][p].y; v[p].z += q[j][p].z; v[p].w += q[j][p].w; }
    } else if constexpr (NP < 0) {
        for (int j = 0; j < parts.n; j++) {
            const float* pj = parts.p + ((int64_t)j * rows + row) * D;
#pragma unroll
            for (int p = 0; p < NPER; p++) {
                const float4 q = *reinterpret_cast<const float4*>(pj + (p * 64 + lane) * 4);
                v[p].x += q.x; v[p].y += q.y; v[p].z += q.z; v[p].w += q.w;
            }
        }
    }
}

template <int NPER, int NP>
__global__ __launch_bounds__(256) void layernorm_kernel(float* x, Partials parts, const float* __restrict__ g,
                                                        const float* __restrict__ b, void* out, int out16, int rows,
                                                        int D, int act) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    float4 v[NPER], gg[NPER], bb[NPER];
    ln_params(gg, bb, g, b, lane);
    load_row<NPER, NP>(v, x, parts, row, rows, D, lane);
    if (NP != 0 && parts.n > 0) store_row(x, false, row, D, v, lane);
    float mean, rstd;
    ln_row_stats(v, D, mean, rstd);
    ln_apply(v, gg, bb, mean, rstd, act);
    store_row(out, out16 != 0, row, D, v, lane);
}

// res <- LN_a(src) (copy when ga is null), z <- LN_b(res).  Joins one layer's norm_out with the
// next layer's norm_feed_forward1 (FastConformer.swift:320 then :277).
template <int NPER, int NP>
__global__ __launch_bounds__(256) void layernorm2_kernel(const float* src, Partials parts, float* res,
                                                         const float* __restrict__ ga, const float* __restrict__ ba,
                                                         const float* __restrict__ gb, const float* __restrict__ bb,
                                                         void* z, int z16, int rows, int D) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    float4 v[NPER], g1[NPER], b1[NPER], g2[NPER], b2[NPER];
    if (ga != nullptr) ln_params(g1, b1, ga, ba, lane);
    ln_params(g2, b2, gb, bb, lane);
    load_row<NPER, NP>(v, src, parts, row, rows, D, lane);
    float mean, rstd;
    if (ga != nullptr) {
        ln_row_stats(v, D, mean, rstd);
        ln_apply(v, g1, b1, mean, rstd, ACT_NONE);
    }
    store_row(res, false, row, D, v, lane);
    ln_row_stats(v, D, mean, rstd);
    ln_apply(v, g2, b2, mean, rstd, ACT_NONE);
    store_row(z, z16 != 0, row, D, v, lane);
}

// The conv module after pointwise_conv1 (FastConformer.swift:298-306): GLU over channels,
// out[t,d] = pw[t,d] * sigmoid(pw[t,D+d]) (Metal/20_conformer.metal:76-85), rows t >= valid zeroed
// (maskRows, FastConformer.swift:302); causal depthwise conv k=KC+1 over [conv cache (KC rows,
// oldest first) ; T GLU rows] (Metal/20_conformer.metal:87-102, tap KC = the current frame); then
// the conv LayerNorm + SiLU.  With G16 the GLU was applied by pointwise_conv1's epilogue and the
// rows come as IEEE half [n*T, D] (a quarter of the fp32 value | gate bytes).  One workgroup per
// stream, 4 channels per thread, the whole
// [KC + T] x 4 window in registers.  The cache is a ring of KC rows per stream: logical row r is
// slot (frames + r) % KC; new row t (only the last KC matter) goes to slot (frames + t) % KC,
// written by the thread that read the slot, so the update is in place with no hazard.
// The stream's descriptor is the first load; the pointwise_conv1 rows, the weights and the LN
// parameters (none of which depend on it) are in flight before the ring rows, and the frame mask
// is applied to the loaded rows.
template <int KC, int TMAX, bool G16>
__global__ __launch_bounds__(256) void dwconv_ln_kernel(ConvArgs a) {
    const int s = blockIdx.x;
    constexpr int NW = 4;                 // 256 threads, 4 channels each (launch_dwconv_ln)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int D = a.D, T = a.T;
    const int c0 = tid * 4;
    const int4 dsc = *reinterpret_cast<const int4*>(a.desc + s * DESC_INTS);
    const int cpos = a.desc[s * DESC_INTS + 4];
    __builtin_amdgcn_sched_barrier(0);

    float4 pv[TMAX], pg[TMAX];
    uint2 gh[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        if constexpr (G16) {
            gh[t] = *reinterpret_cast<const uint2*>(a.glu + ((int64_t)s * T + min(t, T - 1)) * D + c0);
        } else {
            const float* row = a.pw + ((int64_t)s * T + min(t, T - 1)) * 2 * D;
            pv[t] = *reinterpret_cast<const float4*>(row + c0);
            pg[t] = *reinterpret_cast<const float4*>(row + D + c0);
        }
    }
    float4 w[KC + 1];
#pragma unroll
    for (int k = 0; k <= KC; k++) w[k] = *reinterpret_cast<const float4*>(a.w_t + (int64_t)k * D + c0);
    const float4 gg = *reinterpret_cast<const float4*>(a.ln_g + c0);
    const float4 bb = *reinterpret_cast<const float4*>(a.ln_b + c0);
    __builtin_amdgcn_sched_barrier(0);

    const int slot = dsc.x, valid = dsc.z;
    float* ring = a.ring + (int64_t)slot * KC * D;
    float4 in[KC + TMAX];
#pragma unroll
    for (int r = 0; r < KC; r++) {
        int sr = cpos + r;
        sr -= (sr >= KC) ? KC : 0;
        in[r] = *reinterpret_cast<const float4*>(ring + (int64_t)sr * D + c0);
    }
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        float4 y;
        if constexpr (G16) {
            y = make_float4(half_lo(gh[t].x), half_hi(gh[t].x), half_lo(gh[t].y), half_hi(gh[t].y));
        } else {
            const float4 v = pv[t], gt = pg[t];
            y = make_float4(v.x * sigmoidf(gt.x), v.y * sigmoidf(gt.y), v.z * sigmoidf(gt.z), v.w * sigmoidf(gt.w));
        }
        in[KC + t] = (t < T && t < valid) ? y : make_float4(0.f, 0.f, 0.f, 0.f);
    }

    float4 o[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k <= KC; k++) {
            acc.x += w[k].x * in[t + k].x; acc.y += w[k].y * in[t + k].y;
            acc.z += w[k].z * in[t + k].z; acc.w += w[k].w * in[t + k].w;
        }
        o[t] = acc;
    }
    // Ring update (all reads of this thread's slots are done).
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        if (t < T && t >= T - KC) {
            int sr = (cpos + t) % KC;
            *reinterpret_cast<float4*>(ring + (int64_t)sr * D + c0) = in[KC + t];
        }
    }

    // LayerNorm over the D channels of each frame, two passes: per-wave partial sums through LDS,
    // and every thread adds the waves' partials itself (one barrier per pass; the second pass
    // writes a second buffer, so no barrier separates the passes' reads and writes).
    __shared__ float red[2][NW][TMAX];
    float part[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++) part[t] = wave_sum((o[t].x + o[t].y) + (o[t].z + o[t].w));
    if (lane == 0)
#pragma unroll
        for (int t = 0; t < TMAX; t++) red[0][wave][t] = part[t];
    __syncthreads();
    float mean[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        float sum = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < NW; w2++) sum += red[0][w2][t];
        mean[t] = sum / (float)D;
        float a0 = o[t].x - mean[t], a1 = o[t].y - mean[t], a2 = o[t].z - mean[t], a3 = o[t].w - mean[t];
        part[t] = wave_sum((a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3));
    }
    if (lane == 0)
#pragma unroll
        for (int t = 0; t < TMAX; t++) red[1][wave][t] = part[t];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        if (t < T) {
            float sum = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < NW; w2++) sum += red[1][w2][t];
            const float rstd = 1.0f / sqrtf(sum / (float)D + LN_EPS);
            float4 y;
            y.x = silu((o[t].x - mean[t]) * rstd * gg.x + bb.x);
            y.y = silu((o[t].y - mean[t]) * rstd * gg.y + bb.y);
            y.z = silu((o[t].z - mean[t]) * rstd * gg.z + bb.z);
            y.w = silu((o[t].w - mean[t]) * rstd * gg.w + bb.w);
            const int64_t row = (int64_t)s * T + t;
            if (a.z16) {
                store4_frag(a.z, row, c0, D, y);
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(a.z) + row * D + c0) = y;
            }
        }
    }
}

// ---------------------------------------------------------------- launchers

// Rows (one wave each) per workgroup.  A streaming step has a few hundred rows: one row per
// workgroup spreads them over that many CUs (128 rows: 1.901 -> 1.870 ms per 24-layer step
// against 4 rows per workgroup).
static int ln_rows_per_block(int rows) { return rows <= 1024 ? 1 : 4; }

template <int NPER>
static void ln_dispatch(dim3 grid, dim3 block, hipStream_t st, float* x, Partials parts, const float* g, const float* b,
                        void* out, int ob, int rows, int D, int act) {
    if (parts.n == 0) hipLaunchKernelGGL((layernorm_kernel<NPER, 0>), grid, block, 0, st, x, parts, g, b, out, ob, rows, D, act);
    else if (parts.n == 1) hipLaunchKernelGGL((layernorm_kernel<NPER, 1>), grid, block, 0, st, x, parts, g, b, out, ob, rows, D, act);
    else if (parts.n == 2) hipLaunchKernelGGL((layernorm_kernel<NPER, 2>), grid, block, 0, st, x, parts, g, b, out, ob, rows, D, act);
    else if (parts.n == 4) hipLaunchKernelGGL((layernorm_kernel<NPER, 4>), grid, block, 0, st, x, parts, g, b, out, ob, rows, D, act);
    else hipLaunchKernelGGL((layernorm_kernel<NPER, -1>), grid, block, 0, st, x, parts, g, b, out, ob, rows, D, act);
}

int launch_layernorm(float* x, Partials parts, const float* g, const float* b, void* out, bool out16, int rows,
                     int D, int act, hipStream_t st) {
    if (rows <= 0) return 0;
    const int rpb = ln_rows_per_block(rows);
    dim3 grid((rows + rpb - 1) / rpb), block(64 * rpb);
    const int ob = out16 ? 1 : 0;
    switch (D) {
        case 256: ln_dispatch<1>(grid, block, st, x, parts, g, b, out, ob, rows, D, act); break;
        case 512: ln_dispatch<2>(grid, block, st, x, parts, g, b, out, ob, rows, D, act); break;
        case 1024: ln_dispatch<4>(grid, block, st, x, parts, g, b, out, ob, rows, D, act); break;
        case 2048: ln_dispatch<8>(grid, block, st, x, parts, g, b, out, ob, rows, D, act); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int NPER>
static void ln2_dispatch(dim3 grid, dim3 block, hipStream_t st, const float* src, Partials parts, float* res,
                         const float* ga, const float* ba, const float* gb, const float* bb, void* z, int zb, int rows,
                         int D) {
    if (parts.n == 0) hipLaunchKernelGGL((layernorm2_kernel<NPER, 0>), grid, block, 0, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D);
    else if (parts.n == 1) hipLaunchKernelGGL((layernorm2_kernel<NPER, 1>), grid, block, 0, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D);
    else if (parts.n == 2) hipLaunchKernelGGL((layernorm2_kernel<NPER, 2>), grid, block, 0, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D);
    else if (parts.n == 4) hipLaunchKernelGGL((layernorm2_kernel<NPER, 4>), grid, block, 0, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D);
    else hipLaunchKernelGGL((layernorm2_kernel<NPER, -1>), grid, block, 0, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D);
}

int launch_layernorm2(const float* src, Partials parts, float* res, const float* ga, const float* ba, const float* gb,
                      const float* bb, void* z, bool z16, int rows, int D, hipStream_t st) {
    if (rows <= 0) return 0;
    const int rpb = ln_rows_per_block(rows);
    dim3 grid((rows + rpb - 1) / rpb), block(64 * rpb);
    const int zb = z16 ? 1 : 0;
    switch (D) {
        case 256: ln2_dispatch<1>(grid, block, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D); break;
        case 512: ln2_dispatch<2>(grid, block, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D); break;
        case 1024: ln2_dispatch<4>(grid, block, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D); break;
        case 2048: ln2_dispatch<8>(grid, block, st, src, parts, res, ga, ba, gb, bb, z, zb, rows, D); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <bool G16>
static void dwconv_dispatch(const ConvArgs& a, dim3 grid, dim3 block, hipStream_t st) {
    if (a.T <= 2) hipLaunchKernelGGL((dwconv_ln_kernel<8, 2, G16>), grid, block, 0, st, a);
    else if (a.T <= 4) hipLaunchKernelGGL((dwconv_ln_kernel<8, 4, G16>), grid, block, 0, st, a);
    else if (a.T <= 8) hipLaunchKernelGGL((dwconv_ln_kernel<8, 8, G16>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((dwconv_ln_kernel<8, 16, G16>), grid, block, 0, st, a);
}

int launch_dwconv_ln(const ConvArgs& a, hipStream_t st) {
    if (a.K != 9 || a.D % 256 != 0 || a.D / 4 > 1024 || a.T < 1 || a.T > 16 || a.n < 1) return -2;
    if ((a.pw == nullptr) == (a.glu == nullptr)) return -2;
    dim3 grid(a.n), block(a.D / 4);
    if (a.D / 4 != 256) return -2;   // the block reduction is sized for 4 waves
    if (a.glu) dwconv_dispatch<true>(a, grid, block, st);
    else dwconv_dispatch<false>(a, grid, block, st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ud
