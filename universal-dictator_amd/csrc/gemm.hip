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
// Epilogues: act + bf16 store (row-major, or fragment-major for a following GEMM), fp32 store,
// in-place fp32 residual accumulate, split-K partial slabs, and the QKV projection's split store:
// q row-major into the buffer the attention reads, K and V straight into their K/V ring rows (so
// the new rows are written once, and the attention kernel only reads the rings).
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

// The 16-bit K/V ring element of a QKV projection output in column n of [D, 3D), for an output row
// whose ring row starts at element rowoff of the slot's head-0 block (QkvRing::rows): K for
// n < 2D, V above, head (n - D) mod D / 128.
__device__ __forceinline__ uint16_t* qkv_ring_dst(const QkvRing& r, int rowoff, int n) {
    const int D = r.H * 128;
    const int c = n - D, part = c >= D ? 1 : 0, cc = c - part * D;
    uint16_t* base = static_cast<uint16_t*>(part ? r.vring : r.kring);
    return base + rowoff + (int64_t)(cc >> 7) * r.R * 128 + (cc & 127);
}

// 16 bytes of the QKV ring-row table per lane, global -> LDS at dst + 16 * lane (a plain function:
// the builtin written in a kernel template's body drops the host stub of some instantiations).
__device__ __forceinline__ void lds_direct16_rows(const int32_t* src, int32_t* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// EPI_SUBFLAT: the out Linear's A-operand element of GEMM row m, column n (-1: row not stored), and
// whether the row is masked (written as zero).
__device__ __forceinline__ int64_t subflat_dst(const GemmArgs& a, int64_t m, int n, bool& masked) {
    const SubFlat& f = a.flat;
    const int per = f.T3 * f.F3, mi = (int)m;                 // M < 2^31 (launch_gemm)
    const int s = mi / per, rem = mi - s * per, t3 = rem / f.F3, f3 = rem - t3 * f.F3;
    masked = t3 >= f.vlen[4 * s + 3];
    if (t3 < f.drop) return -1;
    return frag_index((int64_t)s * f.T + t3 - f.drop, f3 * a.N + n, f.F3 * a.N / 64);
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

template <int MT, int NT, bool H>
__device__ __forceinline__ void mma_frag(const Frag<MT, NT>& f, f32x4_t (&acc)[NT][MT]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                if constexpr (H)
                    acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(f.a[mt][h]), as_f16x8(f.b[nt][h]),
                                                                         acc[nt][mt], 0, 0, 0);
                else
                    acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(f.a[mt][h]), as_bf16x8(f.b[nt][h]),
                                                                          acc[nt][mt], 0, 0, 0);
            }
}

// Grid: (N/16) x ceil(M/(16*MT)) x ksplit workgroups of WK waves.  The host guarantees
// K % (64 * ksplit) == 0 and at least WK 64-deep chunks per split: wave w takes chunks w, w + WK,
// .. of its split, so when WK does not divide the chunk count the first waves take one more.  The epilogue kind and activation are template parameters: a
// runtime-switched, fully unrolled epilogue measured ~3.5 us slower per launch on MI355X (its
// code does not stay in the instruction cache).
template <int MT, int WK, int EPI, int ACT, int NT, bool H = false, bool BIAS = false>
__global__ __launch_bounds__(64 * WK, 1) void gemm_bf16_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    // QKV split store: the ring offsets of the workgroup's 16 MT rows, into LDS (read in the
    // epilogue, after the workgroup barrier); the table is padded past the last row
    __shared__ __attribute__((aligned(16))) int32_t rtab[EPI == EPI_QKV_RING ? 16 * MT : 4];
    if constexpr (EPI == EPI_QKV_RING) {
        if (wave == 0 && lane < 4 * MT)
            lds_direct16_rows(a.ring.rows + mb * 16 * MT + 4 * lane, rtab);
    }
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

    const int cnt = (kper - wave + WK - 1) / WK;   // chunks of this wave (>= 1)
    constexpr int STEP = WK * 1024;       // element stride between a wave's consecutive chunks
    auto off = [&](int i) { return (int64_t)i * STEP; };
    Frag<MT, NT> f0, f1;
    load_frag(f0, ap, wp, off(0));
    int i = 0;
    for (; i + 2 < cnt; i += 2) {
        load_frag(f1, ap, wp, off(i + 1));
        __builtin_amdgcn_sched_barrier(0);
        mma_frag<MT, NT, H>(f0, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_frag(f0, ap, wp, off(i + 2));
        __builtin_amdgcn_sched_barrier(0);
        mma_frag<MT, NT, H>(f1, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (i + 1 < cnt) {
        load_frag(f1, ap, wp, off(i + 1));
        __builtin_amdgcn_sched_barrier(0);
        mma_frag<MT, NT, H>(f0, acc);
        __builtin_amdgcn_sched_barrier(0);
        mma_frag<MT, NT, H>(f1, acc);
    } else {
        mma_frag<MT, NT, H>(f0, acc);
    }

    // Epilogue of one finished 16 x 16 accumulator (j, mt): the lane holds rows
    // 16*(mb*MT + mt) + 4*g + i (i < 4) of column 16*(nt*NT + j) + r16.
    auto finish = [&](int j, int mt, const f32x4_t& v4) {
        const int n = (nt * NT + j) * 16 + r16;
#pragma unroll
        for (int i2 = 0; i2 < 4; i2++) {
            const int64_t m = (int64_t)(mb * MT + mt) * 16 + g * 4 + i2;
            if (m >= a.M) continue;
            float v = v4[i2];
            if constexpr (BIAS) v += kz == 0 ? a.bias[n] : 0.0f;
            if constexpr (EPI == EPI_PARTIAL) {
                static_cast<float*>(a.C)[((int64_t)kz * a.M + m) * a.ldc + n] = a.out_scale * v;
            } else if constexpr (EPI == EPI_STORE_F32) {
                static_cast<float*>(a.C)[m * a.ldc + n] = apply_act(v, ACT) * a.out_scale;
            } else if constexpr (EPI == EPI_STORE_FRAG) {
                static_cast<uint16_t*>(a.C)[frag_index(m, n, a.N / 64)] = to16<H>(apply_act(v, ACT) * a.out_scale);
            } else if constexpr (EPI == EPI_QKV_RING) {
                const uint16_t x = to16<H>(apply_act(v, ACT) * a.out_scale);
                if (n < a.ring.H * 128) static_cast<uint16_t*>(a.C)[m * a.ldc + n] = x;
                else *qkv_ring_dst(a.ring, rtab[mt * 16 + g * 4 + i2], n) = x;
            } else if constexpr (EPI == EPI_SUBFLAT) {
                bool masked;
                const int64_t d = subflat_dst(a, m, n, masked);
                if (d >= 0) static_cast<uint16_t*>(a.C)[d] = masked ? (uint16_t)0 : to16<H>(apply_act(v, ACT) * a.out_scale);
            } else {
                static_cast<uint16_t*>(a.C)[m * a.ldc + n] = to16<H>(apply_act(v, ACT) * a.out_scale);
            }
        }
    };
    // EPI_GLU: accumulators j (values) and j + 1 (gates) of the same 16 channels; the lane's
    // channel is (nt NT / 2 + j / 2) * 16 + r16
    auto finish_glu = [&](int j, int mt, const f32x4_t& vv, const f32x4_t& vg) {
        const int c = (nt * NT / 2 + j / 2) * 16 + r16;
#pragma unroll
        for (int i2 = 0; i2 < 4; i2++) {
            const int64_t m = (int64_t)(mb * MT + mt) * 16 + g * 4 + i2;
            if (m >= a.M) continue;
            static_cast<uint16_t*>(a.C)[m * a.ldc + c] = to16<H>(vv[i2] * sigmoidf(vg[i2]));
        }
    };
    if constexpr (EPI == EPI_GLU) {
        static_assert(NT % 2 == 0, "value and gate tiles in pairs");
        if constexpr (WK > 1) {
            __shared__ f32x4_t red[WK][NT][MT][64];
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) red[wave][j][mt][lane] = acc[j][mt];
            __syncthreads();
            for (int idx = wave; idx < NT / 2 * MT; idx += WK) {
                const int j = 2 * (idx / MT), mt = idx % MT;
                f32x4_t vv = red[0][j][mt][lane], vg = red[0][j + 1][mt][lane];
#pragma unroll
                for (int w = 1; w < WK; w++) { vv += red[w][j][mt][lane]; vg += red[w][j + 1][mt][lane]; }
                finish_glu(j, mt, vv, vg);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NT; j += 2)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) finish_glu(j, mt, acc[j][mt], acc[j + 1][mt]);
        }
        return;
    }
    if constexpr (WK > 1) {
        // Every wave parks its partial accumulators in LDS; wave w then finishes the accumulators
        // idx = j*MT + mt with idx % WK == w: the sum of the WK partials in wave order, and the
        // epilogue.  Spreading the sums and the stores over the waves keeps the workgroup's tail
        // short (one wave finishing every accumulator measured ~3 us per launch at 128 rows).
        __shared__ f32x4_t red[WK][NT][MT][64];
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) red[wave][j][mt][lane] = acc[j][mt];
        if constexpr (EPI == EPI_QKV_RING) __builtin_amdgcn_s_waitcnt(0x0F70);   // the row table landed
        __syncthreads();
        for (int idx = wave; idx < NT * MT; idx += WK) {
            const int j = idx / MT, mt = idx % MT;
            f32x4_t v = red[0][j][mt][lane];
#pragma unroll
            for (int w = 1; w < WK; w++) v += red[w][j][mt][lane];
            finish(j, mt, v);
        }
    } else {
        if constexpr (EPI == EPI_QKV_RING) {
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the row table's direct load landed
            __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) finish(j, mt, acc[j][mt]);
    }
}

// ---------------------------------------------------------------- bf16, many rows (LDS-staged)
// For M in the thousands (256 streams x 14 frames = 3584 rows) the projections are MFMA-bound, and
// the register-direct kernel above would re-read each activation fragment once per 16-column tile.
// Here a workgroup of 8 waves (2 per SIMD, so one wave's MFMAs run while the other waits on LDS)
// owns a 256 x 64*NT output tile (or 224 or 128 rows).  Per 32-deep K step it copies the row
// fragments and 4*NT column fragments (each a contiguous 1 KB half of a 2 KB fragment-major block,
// so the copy is linear) into LDS with direct global -> LDS loads (global_load_lds_dwordx4, no
// staging registers).  LDS holds a ring of four steps and the fragments are read one step ahead:
// at step s the wave waits until its own loads of step s+1 have landed (those of s+2 and s+3 may
// still be in flight) and its LDS reads of step s are done, a barrier makes every wave's loads
// visible and frees step s's buffer, the wave reads its step-(s+1) fragments into its second
// register set, issues the loads of step s+4 into step s's buffer, and multiplies step s.  Three
// steps of loads stay in flight behind the MFMAs (with two 64-deep buffers, less than one chunk
// did, and the kernel waited on its loads).  The four buffers are separate arrays and the loop is
// unrolled by four, so the compiler can tell the buffers apart and does not wait for outstanding
// direct loads before the LDS reads of another buffer.
//
// The MFMAs are inline asm with the accumulators pinned in place in the accumulator registers:
// compiled from the builtin, the register allocator copied part of the accumulator between
// register files every chunk, each copy waiting for an MFMA result (measured: a single wave then
// issues an MFMA every ~32 cycles instead of ~20).  The compiler's hazard checks do not see inside
// the asm, so the required wait states are explicit at the two points where compiled code touches
// the accumulators; empty asm statements pin the zeroing before, and the epilogue's reads after,
// those waits.

// 16 bytes per lane from global memory straight into LDS at dst + 16 * lane (dst wave-uniform).
// (A plain function: inside a lambda of a kernel template the host pass drops the kernel's stub.)
__device__ __forceinline__ void lds_direct16(const bf16* src, bf16* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

template <int NT, int MT>
__device__ __forceinline__ void pin_acc(f32x4_t (&acc)[NT][MT]) {
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int i = 0; i < MT; i++) asm volatile("" : "+a"(acc[j][i]));
}

// The activation as a compile-time choice (silu is v_exp_f32 + v_rcp_f32, about 1 ulp each).
template <int ACT>
__device__ __forceinline__ float act_fast(float x) {
    if constexpr (ACT == ACT_SILU) return silu(x);
    else return apply_act(x, ACT);
}

// Waves form a 2 x 4 grid; each owns 16*MT x 16*NT (AB = 16: 256-row tiles, 128 x 16*NT per wave,
// NT = 4: 128 pinned accumulator registers; with about 120 vector registers two waves fit per
// SIMD).  Narrower tiles (NT 3, 2), 224-row tiles (AB = 14, 112 rows per wave) and 128-row tiles
// (AB = 8, 64 rows per wave) give more workgroups where 256 x 256 tiles would leave CUs idle
// (3,584 rows = 14 x 256 = 16 x 224: 224-row tiles turn 224 workgroups into 256).  The MFMA operands are swapped (weights as
// the row operand), so each 16 x 16 accumulator holds C^T: a lane has 4 consecutive output columns
// of one row, and the epilogue writes 16 bytes (fp32) or 8 bytes (bf16, row-major or
// fragment-major) per lane.
template <int NT, int EPI, int ACT, bool H = false, bool BIAS = false, int AB = 16>
__global__ __launch_bounds__(512, 1) void gemm_bf16_lds_kernel(GemmArgs a) {
    static_assert(AB == 16 || AB == 14 || AB == 8, "256-, 224- or 128-row tiles");
    constexpr int MT = AB / 2, BB = 4 * NT;                  // wave row tiles; W blocks (16 columns each) per tile
    constexpr int TR = 16 * AB;                              // tile rows
    constexpr int NBLK = AB + BB;                            // 1 KB half-blocks per 32-deep K step
    constexpr int STAGE = NBLK * 512;                        // halves per LDS stage
    constexpr int CPS = (NBLK + 7) / 8, CMIN = NBLK / 8;     // direct loads per wave per step (max, min)
    __shared__ __attribute__((aligned(16))) bf16 st0[STAGE];
    __shared__ __attribute__((aligned(16))) bf16 st1[STAGE];
    __shared__ __attribute__((aligned(16))) bf16 st2[STAGE];
    __shared__ __attribute__((aligned(16))) bf16 st3[STAGE];
    __shared__ __attribute__((aligned(16))) int32_t rtab[EPI == EPI_QKV_RING ? TR : 4];    // QKV: ring row offsets
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool extra = CPS > CMIN && wave + 8 * CMIN < NBLK;   // this wave copies CPS blocks per step, else CMIN
    const int wm = wave >> 2, wn = wave & 3;
    const int r16 = lane & 15, g = lane >> 4;
    const int nN = a.N / (64 * NT), nM = (a.M + TR - 1) / TR;
    const int ks = a.ksplit;
    const int t = xcd_tile(blockIdx.x, nN * nM * ks);
    const int kz = t % ks, tile = t / ks;
    const int mb = tile / nN, nb = tile % nN;
    const int nk = a.K / 64, kper = nk / ks, kc0 = kz * kper;
    const int nsteps = 2 * kper;                             // 32-deep K steps of this split
    const int rtiles = (a.M + 15) / 16;
    const bf16* A = static_cast<const bf16*>(a.A);
    const bf16* W = static_cast<const bf16*>(a.W);

    // Wave w copies the 1 KB half-blocks u = w + 8j of each step: A's row tiles for u < AB, then W's.
    int soff[CPS];
#pragma unroll
    for (int j = 0; j < CPS; j++) {
        const int u = wave + 8 * j;
        int o = 0;
        if (u < AB) o = (min(mb * AB + u, rtiles - 1) * nk + kc0) << 10;     // clamped rows: not stored
        else if (u < NBLK) o = ((nb * BB + u - AB) * nk + kc0) << 10;
        soff[j] = o;
    }
    const int lo = lane * 8;
    auto copy_step = [&](int s, bf16* dst) __attribute__((always_inline)) {
        const int kofs = ((s >> 1) << 10) + (s & 1) * 512;
#pragma unroll
        for (int j = 0; j < CPS; j++) {
            const int u = wave + 8 * j;
            if (j < CMIN || u < NBLK) lds_direct16((u < AB ? A : W) + soff[j] + kofs + lo, dst + u * 512);
        }
    };

    f32x4_t acc[NT][MT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int i = 0; i < MT; i++) acc[j][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int aoff = (wm * MT) * 512 + lo, boff = (AB + wn * NT) * 512 + lo;
    // Two fragment register sets: the MFMAs of step s run on one while the LDS reads of step s + 1
    // fill the other.
    uint4 fa0[MT], fb0[NT], fa1[MT], fb1[NT];
    auto read_to = [&](const bf16* buf, uint4 (&xa)[MT], uint4 (&xb)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; i++) xa[i] = *reinterpret_cast<const uint4*>(buf + aoff + i * 512);
#pragma unroll
        for (int j = 0; j < NT; j++) xb[j] = *reinterpret_cast<const uint4*>(buf + boff + j * 512);
    };
    auto mma = [&](const uint4 (&xa)[MT], const uint4 (&xb)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int i = 0; i < MT; i++)
                if constexpr (H)
                    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                                 : "+a"(acc[j][i]) : "v"(as_f16x8(xb[j])), "v"(as_f16x8(xa[i])));
                else
                    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                                 : "+a"(acc[j][i]) : "v"(as_bf16x8(xb[j])), "v"(as_bf16x8(xa[i])));
    };
    // This wave's loads of a step have landed once at most `later` steps' loads (issued after it)
    // are outstanding: CPS or CMIN direct loads per step for this wave.
    auto wait_landed = [&](int later) __attribute__((always_inline)) {
        if (extra) {
            if (later >= 3) __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * CPS));
            else if (later == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * CPS));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(CPS));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        } else {
            if (later >= 3) __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * CMIN));
            else if (later == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * CMIN));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(CMIN));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
    };
    // QKV split store: the ring offsets of the tile's TR rows (the table is padded past the last row)
    if constexpr (EPI == EPI_QKV_RING) {
        if (wave == 0 && lane < TR / 4) lds_direct16_rows(a.ring.rows + mb * TR + 4 * lane, rtab);
    }
    // Four-stage ring of 32-deep K steps, fragments one step ahead.  At step s: wait until this
    // wave's loads of step s + 1 have landed and its LDS reads of step s are done; a barrier makes
    // every wave's loads of s + 1 visible and frees step s's buffer (every wave holds its step-s
    // fragments in registers); read the step s + 1 fragments, issue the loads of step s + 4 into
    // step s's buffer, and multiply step s.  So the LDS reads of one step overlap the MFMAs of the
    // previous one, and three steps of loads stay in flight behind them.
    copy_step(0, st0);
    if (1 < nsteps) copy_step(1, st1);
    if (2 < nsteps) copy_step(2, st2);
    if (3 < nsteps) copy_step(3, st3);
    wait_landed(min(3, nsteps - 1));
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    read_to(st0, fa0, fb0);
    pin_acc(acc);
    asm volatile("s_nop 7");                                 // accumulator zeroing -> first MFMA
    auto step = [&](int s, const uint4 (&ca)[MT], const uint4 (&cb)[NT], uint4 (&na)[MT], uint4 (&nb)[NT],
                    const bf16* nbuf, bf16* cbuf) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(0xC07F);                  // lgkmcnt(0): this wave's step-s reads are done
        if (s + 1 < nsteps) {
            wait_landed(min(s + 3, nsteps - 1) - (s + 1));
            __builtin_amdgcn_s_barrier();                    // every wave's loads of step s + 1; step s's buffer free
            __asm__ volatile("" ::: "memory");
            read_to(nbuf, na, nb);
            __builtin_amdgcn_sched_barrier(0);
            if (s + 4 < nsteps) copy_step(s + 4, cbuf);
            __builtin_amdgcn_sched_barrier(0);
        }
        mma(ca, cb);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int s = 0; s < nsteps; s += 4) {
        step(s, fa0, fb0, fa1, fb1, st1, st0);
        if (s + 1 < nsteps) step(s + 1, fa1, fb1, fa0, fb0, st2, st1);
        if (s + 2 < nsteps) step(s + 2, fa0, fb0, fa1, fb1, st3, st2);
        if (s + 3 < nsteps) step(s + 3, fa1, fb1, fa0, fb0, st0, st3);
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");   // last MFMA results -> epilogue reads
    pin_acc(acc);

    // acc[j][i] is tile (column tile j, row tile i) transposed: lane holds row 16*rt + r16 and the
    // 4 columns 16*ct + 4*g + e (e < 4).
    if constexpr (EPI == EPI_GLU) {
        // column tiles j (values) and j + 1 (gates) of channels 16 ((nb BB + wn NT + j) / 2) ..
        static_assert(NT % 2 == 0, "value and gate tiles in pairs");
#pragma unroll
        for (int i = 0; i < MT; i++) {
            const int64_t m = (int64_t)(mb * AB + wm * MT + i) * 16 + r16;
            if (m >= a.M) continue;
#pragma unroll
            for (int j = 0; j < NT; j += 2) {
                const int c = ((nb * BB + wn * NT + j) / 2) * 16 + g * 4;
                const f32x4_t vv = acc[j][i], vg = acc[j + 1][i];
                uint2 o;
                o.x = (uint32_t)to16<H>(vv[0] * sigmoidf(vg[0])) | ((uint32_t)to16<H>(vv[1] * sigmoidf(vg[1])) << 16);
                o.y = (uint32_t)to16<H>(vv[2] * sigmoidf(vg[2])) | ((uint32_t)to16<H>(vv[3] * sigmoidf(vg[3])) << 16);
                *reinterpret_cast<uint2*>(static_cast<bf16*>(a.C) + m * a.ldc + c) = o;
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int64_t m = (int64_t)(mb * AB + wm * MT + i) * 16 + r16;
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int n = (nb * BB + wn * NT + j) * 16 + g * 4;
            f32x4_t v = acc[j][i];
            if constexpr (BIAS) {
                if (kz == 0) v += *reinterpret_cast<const f32x4_t*>(a.bias + n);
            }
            if constexpr (EPI == EPI_PARTIAL) {
                *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.C) + ((int64_t)kz * a.M + m) * a.ldc + n) =
                    v * a.out_scale;
            } else if constexpr (EPI == EPI_STORE_F32) {
                f32x4_t o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = apply_act(v[e], ACT) * a.out_scale;
                *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.C) + m * a.ldc + n) = o;
            } else {
                uint2 o;
                o.x = (uint32_t)to16<H>(act_fast<ACT>(v[0]) * a.out_scale) | ((uint32_t)to16<H>(act_fast<ACT>(v[1]) * a.out_scale) << 16);
                o.y = (uint32_t)to16<H>(act_fast<ACT>(v[2]) * a.out_scale) | ((uint32_t)to16<H>(act_fast<ACT>(v[3]) * a.out_scale) << 16);
                bf16* dst;
                if constexpr (EPI == EPI_QKV_RING) {   // 4 columns of one head: contiguous in the ring row
                    dst = n < a.ring.H * 128 ? static_cast<bf16*>(a.C) + m * a.ldc + n
                                             : qkv_ring_dst(a.ring, rtab[(wm * MT + i) * 16 + r16], n);
                } else if constexpr (EPI == EPI_SUBFLAT) {   // 4 columns: contiguous in the fragment block
                    bool masked;
                    const int64_t d = subflat_dst(a, m, n, masked);
                    if (d < 0) continue;
                    if (masked) o = make_uint2(0, 0);
                    dst = static_cast<bf16*>(a.C) + d;
                } else {
                    dst = static_cast<bf16*>(a.C) + (EPI == EPI_STORE_FRAG ? frag_index(m, n, a.N / 64) : m * a.ldc + n);
                }
                *reinterpret_cast<uint2*>(dst) = o;
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
    // EPI_PARTIAL: blockIdx.z = K split kz over K range [kb, ke), its own fp32 slab.
    const int kz = blockIdx.z;
    const int kper = (a.K + (int)gridDim.z - 1) / (int)gridDim.z;
    const int kb = kz * kper, ke = min(a.K, kb + kper);
    float acc[4][4] = {};
    for (int k0 = kb; k0 < ke; k0 += F_BK) {
        for (int idx = tid; idx < F_BM * F_BK; idx += 256) {
            int r = idx / F_BK, kk = idx % F_BK;
            int m = m0 + r, n = n0 + r, k = k0 + kk;
            As[kk][r] = (m < a.M && k < ke) ? A[(int64_t)m * a.lda + k] : 0.0f;
            Ws[kk][r] = (n < a.N && k < ke) ? W[(int64_t)n * a.ldw + k] : 0.0f;
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
            float* C = static_cast<float*>(a.C) + ((int64_t)kz * a.M + m) * a.ldc + n;
            if (a.bias != nullptr && kz == 0) acc[i][j] += a.bias[n];
            if (a.epi == EPI_RESID) *C = *C + a.out_scale * acc[i][j];
            else if (a.epi == EPI_PARTIAL) *C = a.out_scale * acc[i][j];
            else *C = apply_act(acc[i][j], a.act) * a.out_scale;
        }
    }
}

// ---------------------------------------------------------------- small-M fp32 (MFMA)

// C = A[M, K] . W[N, K]^T in fp32 on the fp32 MFMA (v_mfma_f32_16x16x4_f32), for the decoder's
// weight-streaming shapes (tens of rows against thousands of weight rows).
//   workgroup = 4 waves; wave w owns the 16 output columns n0 = (4 blockIdx.x + w) * 16 ..
//   blockIdx.y = K split kz (EPI_PARTIAL slabs); blockIdx.z = block of MT * 16 rows of M (MT = 4,
//   or the tiles M needs when it is below 64: a greedy iteration after the first often has a few
//   active streams)
//   The workgroup's A rows are shared by its 4 waves: per 64-wide K chunk they are staged in LDS
//   (each thread one float4 per 16 rows), so A crosses L2 once per workgroup, not once per wave.
//   Per 16-wide k group, lane (c = lane % 16, q = lane / 16) takes W[n0 + c][k + 4q .. 4q + 3] as a
//   float4 from global memory and, for each row tile t, A[m0 + 16 t + c][k + 4q .. 4q + 3] from
//   LDS; MFMA k-step s takes element s of both, so A and W see the same permutation of the
//   group's 16 k values.
// Every output sums its K range in the same order whatever M is, so a row's result does not
// depend on the batch it is computed in.
constexpr int FS_MT = 4;
constexpr int FS_KC = 64;                      // K chunk staged in LDS

template <int MT>
__global__ __launch_bounds__(256) void gemm_f32_small_kernel(GemmArgs a, int kper) {
    __shared__ float4 As[16 * MT][FS_KC / 4 + 1];      // +1: conflict-free column reads
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = lane & 15, q = lane >> 4;
    const int n0 = (blockIdx.x * 4 + w) * 16;
    const bool wave_live = n0 < a.N;            // waves past N still help stage A
    const int kz = blockIdx.y;
    const int kb = kz * kper, ke = min(a.K, kb + kper);
    const int m0 = blockIdx.z * 16 * MT;
    const float* W = static_cast<const float*>(a.W) + (int64_t)min(n0 + c, a.N - 1) * a.ldw + 4 * q;
    const float* A = static_cast<const float*>(a.A);
    // staging: thread tid loads row (tid / 16) + 16 i, float4 column tid % 16 of each chunk
    const int sr = tid >> 4, sc4 = tid & 15;
    f32x4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // registers of the next chunk: loaded one chunk ahead, while the current one is multiplied
    float4 st[MT], wv[FS_KC / 16], wn[FS_KC / 16];
    auto load_chunk = [&](int k0, float4 (&wd)[FS_KC / 16]) {
        const int kn = min(FS_KC, ke - k0);     // a multiple of 16
#pragma unroll
        for (int i = 0; i < MT; i++) {
            const int m = m0 + sr + 16 * i;
            st[i] = (m < a.M && 4 * sc4 < kn) ? *reinterpret_cast<const float4*>(A + (int64_t)m * a.lda + k0 + 4 * sc4)
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int g = 0; g < FS_KC / 16; g++)
            wd[g] = (wave_live && 16 * g < kn) ? *reinterpret_cast<const float4*>(W + k0 + 16 * g)
                                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    load_chunk(kb, wv);
    for (int k0 = kb; k0 < ke; k0 += FS_KC) {
        const int kn = min(FS_KC, ke - k0);
        if (k0 != kb) __syncthreads();          // every wave is done with the previous chunk
#pragma unroll
        for (int i = 0; i < MT; i++) As[sr + 16 * i][sc4] = st[i];
        __syncthreads();
        if (k0 + FS_KC < ke) load_chunk(k0 + FS_KC, wn);
        if (wave_live) {
#pragma unroll
            for (int g = 0; g < FS_KC / 16; g++) {
                if (16 * g >= kn) break;
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const float4 xv = As[16 * t + c][4 * g + q];
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, wv[g].x, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, wv[g].y, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, wv[g].z, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, wv[g].w, acc[t], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < FS_KC / 16; g++) wv[g] = wn[g];
    }
    const int n = n0 + c;
    if (!wave_live || n >= a.N) return;
    float* C = static_cast<float*>(a.C);
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = m0 + 16 * t + 4 * q + r;
            if (m >= a.M) continue;
            float v = acc[t][r];
            if (a.epi == EPI_PARTIAL) {
                C[((int64_t)kz * a.M + m) * a.ldc + n] = a.out_scale * v;
            } else {
                if (a.bias != nullptr) v += a.bias[n];
                C[(int64_t)m * a.ldc + n] = apply_act(v, a.act) * a.out_scale;
            }
        }
}

int launch_gemm_f32_small(const GemmArgs& a, int ks, hipStream_t st) {
    if (a.epi != EPI_PARTIAL && a.epi != EPI_STORE) return -2;
    if (ks < 1 || (a.epi != EPI_PARTIAL && ks != 1) || a.M < 1 || a.N < 1) return -2;
    if (a.K % (16 * ks) != 0 || a.lda % 4 != 0 || a.ldw % 4 != 0) return -2;
    if ((reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W)) & 15) return -2;
    const int kper = a.K / ks;
    const int mt = a.M >= 16 * FS_MT ? FS_MT : (a.M + 15) / 16;
    dim3 grid((a.N + 63) / 64, ks, (a.M + 16 * mt - 1) / (16 * mt));
    if (grid.z > 65535) return -2;
    switch (mt) {
        case 1: hipLaunchKernelGGL(gemm_f32_small_kernel<1>, grid, dim3(256), 0, st, a, kper); break;
        case 2: hipLaunchKernelGGL(gemm_f32_small_kernel<2>, grid, dim3(256), 0, st, a, kper); break;
        case 3: hipLaunchKernelGGL(gemm_f32_small_kernel<3>, grid, dim3(256), 0, st, a, kper); break;
        default: hipLaunchKernelGGL(gemm_f32_small_kernel<FS_MT>, grid, dim3(256), 0, st, a, kper); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------- launch

template <int MT, int WK, int NT, int EPI, int ACT, bool H = false, bool BIAS = false>
static int launch_bf16_cfg(GemmArgs a, int ksplit, hipStream_t st) {
    if (a.N % (16 * NT) != 0 || ksplit < 1 || a.K % (64 * ksplit) != 0 || a.K / (64 * ksplit) < WK) return -2;
    if (ksplit > 1 && EPI != EPI_PARTIAL) return -2;
    if (EPI == EPI_STORE_FRAG && a.N % 64 != 0) return -2;
    a.ksplit = ksplit;
    const int tiles = (a.N / (16 * NT)) * ((a.M + 16 * MT - 1) / (16 * MT)) * ksplit;
    hipLaunchKernelGGL((gemm_bf16_kernel<MT, WK, EPI, ACT, NT, H, BIAS>), dim3(tiles), dim3(64 * WK), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int NT, int EPI, int ACT, bool H = false, bool BIAS = false, int AB = 16>
static int launch_lds_cfg(GemmArgs a, int ksplit, hipStream_t st) {
    if (a.N % (64 * NT) != 0 || ksplit < 1 || a.K % (64 * ksplit) != 0 || a.ldc % 4 != 0) return -2;
    if (ksplit > 1 && EPI != EPI_PARTIAL) return -2;
    if ((int64_t)((a.M + 15) / 16) * a.K * 16 >= (1ll << 31) || (int64_t)a.N * a.K >= (1ll << 31)) return -2;
    a.ksplit = ksplit;
    const int tiles = (a.N / (64 * NT)) * ((a.M + 16 * AB - 1) / (16 * AB)) * ksplit;
    hipLaunchKernelGGL((gemm_bf16_lds_kernel<NT, EPI, ACT, H, BIAS, AB>), dim3(tiles), dim3(512), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int NT, int EPI, bool H, int AB>
static int launch_lds_epi(const GemmArgs& a, int ks, hipStream_t st) {
    switch (a.act) {
        case ACT_NONE: return launch_lds_cfg<NT, EPI, ACT_NONE, H, false, AB>(a, ks, st);
        case ACT_SILU: return launch_lds_cfg<NT, EPI, ACT_SILU, H, false, AB>(a, ks, st);
        case ACT_RELU: return launch_lds_cfg<NT, EPI, ACT_RELU, H, false, AB>(a, ks, st);
        default: return -2;
    }
}

template <int NT, bool H, int AB>
static int launch_lds_act(const GemmArgs& a, int ks, hipStream_t st) {
    switch (a.epi) {
        case EPI_PARTIAL: return a.act == ACT_NONE ? launch_lds_cfg<NT, EPI_PARTIAL, ACT_NONE, H, false, AB>(a, ks, st) : -2;
        case EPI_STORE_F32: return launch_lds_epi<NT, EPI_STORE_F32, H, AB>(a, ks, st);
        case EPI_STORE_FRAG: return launch_lds_epi<NT, EPI_STORE_FRAG, H, AB>(a, ks, st);
        case EPI_STORE: return launch_lds_epi<NT, EPI_STORE, H, AB>(a, ks, st);
        case EPI_QKV_RING: return launch_lds_cfg<NT, EPI_QKV_RING, ACT_NONE, H, false, AB>(a, ks, st);
        case EPI_GLU:
            if constexpr (NT % 2 == 0) return a.act == ACT_NONE ? launch_lds_cfg<NT, EPI_GLU, ACT_NONE, H, false, AB>(a, ks, st) : -2;
            return -2;
        default: return -2;
    }
}

static int device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

// Tile shape (256 or 128 rows, NT: 64*NT columns) and K splits of the LDS-staged kernel for one
// projection.  Cost model: rounds of workgroups over the CUs (the wave quantisation: a second,
// partly filled round costs a whole round) x the per-workgroup MFMA work, scaled by the per-flop
// cost of each tile shape (256 rows: NT 4 1.00, 3 1.28, 2 1.36, measured at 3584 rows; 128 rows:
// 2.0), plus for K splits the fp32 partial slabs they write and the LayerNorm after them reads
// back (900 units per slab per 3584 x 1024 outputs: a slab's stores come at the end of the one
// round of workgroups, where nothing hides them, about 2-3 us, and its read in the LayerNorm
// about 2.5 us).
// A 128-row tile re-reads each weight panel twice as often as a 256-row one.  Measured on the
// 24-layer 256-stream x 14-frame step (eager launches, all choices in one process):
// 8.409 ms with 256-row tiles everywhere; 8.218 ms with linear_out and pointwise_conv2 on 128 x 128
// tiles (224 workgroups instead of 112 on 256 CUs: 19.7 -> 14.5 us each); 8.209 ms with the
// subsampling's out projection too; worse with 128-row tiles for q/k/v (+0.134 ms),
// pointwise_conv1 (+0.126 ms) or ff linear2 (+0.05 ms with 2 splits, more without), which already
// launch 224 256-row workgroups.  The 128-row cost of 2.0 makes 128-row tiles win only where
// 256-row tiles leave about half the CUs idle, which is what those runs show.
// 224-row tiles: each weight panel is re-read 8/7 as often per flop as with 256-row tiles.  At
// 3,584 rows they give 256 workgroups instead of 224 (ff linear1, q/k/v, pointwise_conv1, ff
// linear2 with 2 splits); with the fragments read one step ahead that step went 8.02 -> 7.95 ms
// (the same fragment schedule with 256-row tiles only: 8.05 ms).
constexpr double C224 = 1.05;
BigTile big_tile(int M, int N, int K, bool partial, int heights_mask) {
    static const double cost_256[5] = {0.0, 0.0, 1.36, 1.28, 1.0};
    static const double cost_128[5] = {0.0, 0.0, 2.0, 2.0, 2.0};
    const int cus = device_cus();
    BigTile best{0, 1, 16};
    double best_cost = 1e300;
    static const int heights[3] = {16, 14, 8};
    for (int hi = 0; hi < 3; hi++)
        for (int nt = 4; nt >= 2; nt--) {
            if (!(heights_mask & (1 << hi))) continue;
            const int ab = heights[hi];
            // per-flop cost: 256-row measured; 224 rows re-read each weight panel 8/7 as often
            const double pc = ab == 16 ? cost_256[nt] : ab == 14 ? cost_256[nt] * C224 : cost_128[nt];
            if (N % (64 * nt) != 0) continue;
            for (int ks = 1; ks <= (partial ? 4 : 1); ks *= 2) {
                if (K % (64 * ks) != 0 || (ks > 1 && K / ks < 256)) continue;
                const long tiles = (long)(N / (64 * nt)) * ((M + 16 * ab - 1) / (16 * ab)) * ks;
                const long rounds = (tiles + cus - 1) / cus;
                double cost = (double)rounds * (ab / 16.0) * nt * (K / ks) * pc;
                if (ks > 1) cost += 900.0 * ks * ((double)M * N / (3584.0 * 1024.0));
                if (cost < best_cost) { best_cost = cost; best = BigTile{nt, ks, ab}; }
            }
        }
    return best;
}

int gemm_partial_splits(int M, int N, int K, bool bf16_data) {
    if (!bf16_data) return 1;
    if (M >= LDS_MIN_ROWS) {
        const BigTile bt = big_tile(M, N, K, true, TILE_ALL);
        if (bt.nt != 0) return bt.ks;
    }
    if (M <= 128 && K == 1024 && N % 32 == 0) return 2;   // linear_out, pointwise_conv2 (launch_bf16)
    return K % (128 * KSPLIT) == 0 ? KSPLIT : 1;
}

template <int MT, int WK, int NT, int EPI, bool H>
static int launch_act(const GemmArgs& a, int ks, hipStream_t st) {
    if (a.act == ACT_SILU) return launch_bf16_cfg<MT, WK, NT, EPI, ACT_SILU, H>(a, ks, st);
    if (a.act == ACT_NONE) return launch_bf16_cfg<MT, WK, NT, EPI, ACT_NONE, H>(a, ks, st);
    if (a.act == ACT_RELU) return launch_bf16_cfg<MT, WK, NT, EPI, ACT_RELU, H>(a, ks, st);
    return -2;
}

// Tile shapes measured on MI355X for the streaming step's M <= 128 projections (weights from HBM,
// 48 rotating copies; the waves of a workgroup split K and share the reduction and the epilogue):
//   ff linear1 (N 4096, K 1024, fragment out):  MT 2 x NT 4, 8 waves            6.97 -> 5.94 us
//   q/k/v (N 3072, K 1024, bf16 out):           MT 4 x NT 2, 8 waves            5.77 -> 5.53 us
//   pointwise_conv1 (N 2048, K 1024, fp32 out): MT 2 x NT 2, 8 waves            4.31 -> 3.76 us
//   ff linear2 (N 1024, K 4096, split-K 4):     MT 4 x NT 2, 8 waves            5.91 -> 5.76 us
//   linear_out, pw2 (N 1024, K 1024):           MT 2 x NT 2, 8 waves, split-K 2 3.40 -> 3.12 us
//                                               (half the slabs for the LayerNorm that adds them)
// Wider tiles cut the re-reads of the activation panel; more waves per workgroup put more of a
// tile's K range in flight at once.
// Larger M keeps 128-row tiles (MT 8, 2 waves).
// IEEE-half operands with a bias (the subsampling front-end's GEMMs): fp32 outputs (EPI_STORE_F32),
// half outputs (EPI_STORE, row-major) or conv.6's flattened rows (EPI_SUBFLAT); no activation or
// ReLU.  The bias is a template parameter: a runtime-optional bias in the encoder's own GEMMs made
// their epilogues larger and cost ~2 us per launch at 128 rows.
template <int EPI, int ACT>
static int launch_f16(const GemmArgs& a, hipStream_t st) {
    // (the subsampling's out Linear at 128 rows: K = 4,352 is 68 chunks, 8 or 9 per wave over 256
    // workgroups of 8 waves; with 4 waves of 17 chunks over 64 workgroups it took ~4 us longer)
    if (a.M <= 128 && a.N % 16 == 0 && a.K % 64 == 0 && a.K >= 512)
        return launch_bf16_cfg<2, 8, 1, EPI, ACT, true, true>(a, 1, st);
    if (a.M <= 128 && a.N % 32 == 0 && a.K % 256 == 0) return launch_bf16_cfg<4, 4, 2, EPI, ACT, true, true>(a, 1, st);
    // The LDS kernel's 256-row tiles leave most CUs idle below ~64 tiles (the second pointwise conv
    // of 64 streams x 160 ms: 4,352 x 256 x 256, 34 tiles, 10.5 us; the register kernel's 64 x 32
    // tiles 6.6 us, 11.7 us once its epilogue wrote the out Linear's flattened rows, 8.2 us with 4
    // waves of one 64-deep chunk each instead of 2 of two).
    const BigTile b256 = a.M >= LDS_MIN_ROWS ? big_tile(a.M, a.N, a.K, false, TILE_256) : BigTile{0, 1, 16};
    if (b256.nt != 0 && (int64_t)((a.M + 255) / 256) * (a.N / (64 * b256.nt)) < 64 && a.N % 32 == 0 && a.K % 128 == 0)
        return a.K >= 256 ? launch_bf16_cfg<4, 4, 2, EPI, ACT, true, true>(a, 1, st)
                          : launch_bf16_cfg<4, 2, 2, EPI, ACT, true, true>(a, 1, st);
    const BigTile bt = a.M >= LDS_MIN_ROWS ? big_tile(a.M, a.N, a.K, false, TILE_256 | TILE_128) : BigTile{0, 1, 16};
    const int nt = bt.nt;
    if (a.M >= LDS_MIN_ROWS) {
        if (bt.ab == 8) {
            switch (nt) {
                case 4: return launch_lds_cfg<4, EPI, ACT, true, true, 8>(a, 1, st);
                case 3: return launch_lds_cfg<3, EPI, ACT, true, true, 8>(a, 1, st);
                case 2: return launch_lds_cfg<2, EPI, ACT, true, true, 8>(a, 1, st);
                default: break;
            }
        }
        switch (nt) {
            case 4: return launch_lds_cfg<4, EPI, ACT, true, true>(a, 1, st);
            case 3: return launch_lds_cfg<3, EPI, ACT, true, true>(a, 1, st);
            case 2: return launch_lds_cfg<2, EPI, ACT, true, true>(a, 1, st);
            default: break;
        }
    }
    return launch_bf16_cfg<8, 2, 1, EPI, ACT, true, true>(a, 1, st);
}

template <int EPI>
static int launch_f16_act(const GemmArgs& a, hipStream_t st) {
    if (a.act == ACT_NONE) return launch_f16<EPI, ACT_NONE>(a, st);
    if (a.act == ACT_RELU) return launch_f16<EPI, ACT_RELU>(a, st);
    return -2;
}

// The encoder's 16-bit projections: operands (and 16-bit outputs) IEEE half when H, bf16 otherwise;
// no bias.
template <bool H>
static int launch_16(const GemmArgs& a, int ks, hipStream_t st) {
    if (a.bias != nullptr) return -2;   // the encoder's projections have no bias
    if (a.M <= 128) {
        switch (a.epi) {
            case EPI_STORE_FRAG:
                if (a.N % 64 == 0 && a.K % 512 == 0) return launch_act<2, 8, 4, EPI_STORE_FRAG, H>(a, ks, st);
                if (a.N % 64 == 0) return launch_act<2, 2, 4, EPI_STORE_FRAG, H>(a, ks, st);
                break;
            case EPI_STORE:
                if (a.N % 32 == 0 && a.K % 512 == 0) return launch_act<4, 8, 2, EPI_STORE, H>(a, ks, st);
                break;
            case EPI_QKV_RING:
                if (a.N % 32 == 0 && a.K % 512 == 0) return launch_bf16_cfg<4, 8, 2, EPI_QKV_RING, ACT_NONE, H>(a, ks, st);
                break;
            case EPI_STORE_F32:
                if (a.N % 32 == 0 && a.K % 512 == 0) return launch_act<2, 8, 2, EPI_STORE_F32, H>(a, ks, st);
                break;
            case EPI_GLU:
                if (a.K % 512 == 0) return launch_bf16_cfg<2, 8, 2, EPI_GLU, ACT_NONE, H>(a, ks, st);
                break;
            case EPI_PARTIAL:
                if (a.act != ACT_NONE) return -2;
                if (a.N % 32 == 0 && a.K % (512 * ks) == 0)
                    return a.K >= 4096 ? launch_bf16_cfg<4, 8, 2, EPI_PARTIAL, ACT_NONE, H>(a, ks, st)
                                       : launch_bf16_cfg<2, 8, 2, EPI_PARTIAL, ACT_NONE, H>(a, ks, st);
                if (a.K % (128 * ks) == 0) return launch_bf16_cfg<4, 2, 1, EPI_PARTIAL, ACT_NONE, H>(a, ks, st);
                break;
            default: return -2;   // the residual accumulate is an fp32-path epilogue
        }
    }
    if (a.M >= LDS_MIN_ROWS) {
        const BigTile bt = big_tile(a.M, a.N, a.K, a.epi == EPI_PARTIAL, TILE_ALL);
        if (bt.nt != 0 && (a.epi != EPI_PARTIAL || bt.ks == ks) && (a.epi != EPI_GLU || bt.nt % 2 == 0)) {
            if (H && bt.ab == 8) {          // 128- and 224-row tiles: instantiated for the encoder's half operands
                switch (bt.nt) {
                    case 4: return launch_lds_act<4, true, 8>(a, ks, st);
                    case 3: return launch_lds_act<3, true, 8>(a, ks, st);
                    default: return launch_lds_act<2, true, 8>(a, ks, st);
                }
            }
            if (H && bt.ab == 14) {
                switch (bt.nt) {
                    case 4: return launch_lds_act<4, true, 14>(a, ks, st);
                    case 3: return launch_lds_act<3, true, 14>(a, ks, st);
                    default: return launch_lds_act<2, true, 14>(a, ks, st);
                }
            }
            switch (bt.nt) {
                case 4: return launch_lds_act<4, H, 16>(a, ks, st);
                case 3: return launch_lds_act<3, H, 16>(a, ks, st);
                default: return launch_lds_act<2, H, 16>(a, ks, st);
            }
        }
    }
    switch (a.epi) {
        case EPI_PARTIAL: return a.act == ACT_NONE ? launch_bf16_cfg<8, 2, 1, EPI_PARTIAL, ACT_NONE, H>(a, ks, st) : -2;
        case EPI_STORE_F32: return launch_act<8, 2, 1, EPI_STORE_F32, H>(a, ks, st);
        case EPI_STORE_FRAG: return launch_act<8, 2, 1, EPI_STORE_FRAG, H>(a, ks, st);
        case EPI_STORE: return launch_act<8, 2, 1, EPI_STORE, H>(a, ks, st);
        case EPI_QKV_RING: return launch_bf16_cfg<8, 2, 1, EPI_QKV_RING, ACT_NONE, H>(a, ks, st);
        case EPI_GLU: return a.act == ACT_NONE ? launch_bf16_cfg<8, 2, 2, EPI_GLU, ACT_NONE, H>(a, ks, st) : -2;
        default: return -2;
    }
}

static int launch_bf16(const GemmArgs& a, int ks, hipStream_t st) {
    if (a.f16 && a.bias != nullptr) {
        // the subsampling front-end's GEMMs: IEEE half with a bias
        if (ks != 1) return -2;
        switch (a.epi) {
            case EPI_STORE_F32: return launch_f16_act<EPI_STORE_F32>(a, st);
            case EPI_STORE: return launch_f16_act<EPI_STORE>(a, st);
            case EPI_SUBFLAT:
                if (!a.flat.vlen || a.flat.T3 < 1 || a.flat.F3 < 1 || a.flat.drop < 0 || a.flat.T != a.flat.T3 - a.flat.drop ||
                    (int64_t)a.M >= (1ll << 31) ||
                    (int64_t)a.M != (int64_t)a.M / (a.flat.T3 * a.flat.F3) * a.flat.T3 * a.flat.F3 || (a.flat.F3 * a.N) % 64)
                    return -2;
                return launch_f16_act<EPI_SUBFLAT>(a, st);
            default: return -2;
        }
    }
    return a.f16 ? launch_16<true>(a, ks, st) : launch_16<false>(a, ks, st);
}

int launch_gemm(const GemmArgs& a, bool bf16_data, hipStream_t st) {
    if (a.M <= 0 || a.N <= 0 || a.K <= 0) return -2;
    // GLU pairs: 16-bit only, no activation, whole 32-column value/gate blocks, half the columns out
    if (a.epi == EPI_GLU && (!bf16_data || a.act != ACT_NONE || a.bias || a.N % 32 != 0 || a.ldc < a.N / 2 || a.ldc % 4))
        return -2;
    if (a.epi == EPI_QKV_RING) {
        // 16-bit only, no activation; the rows are whole streams of T frames; every ring row written
        // is outside the step's window (L + T <= R)
        const QkvRing& r = a.ring;
        if (!bf16_data || a.act != ACT_NONE || a.bias || !r.kring || !r.vring || !r.rows || r.T < 1 || r.H < 1 ||
            a.N != 3 * r.H * 128 || a.M % r.T != 0 || r.L + r.T > r.R || a.ldc < r.H * 128)
            return -2;
    }
    if (!bf16_data) {
        if (a.epi == EPI_STORE_FRAG) return -2;
        const int ks = a.epi == EPI_PARTIAL ? a.ksplit : 1;
        if (ks < 1 || ks > 64) return -2;
        dim3 grid((a.N + F_BN - 1) / F_BN, (a.M + F_BM - 1) / F_BM, ks);
        hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, st, a);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (a.K % 128 != 0) return -2;
    return launch_bf16(a, a.epi == EPI_PARTIAL ? a.ksplit : 1, st);
}

}  // namespace ud
