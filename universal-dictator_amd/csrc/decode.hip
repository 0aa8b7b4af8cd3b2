// Decoder attention for gfx950: grouped-query attention of one new token per sequence over a paged
// K/V cache, the rotate-half RoPE and the paged cache append (include/ud_decode.h).
//
// Semantics: Sources/DictatorEngine/Metal/30_voxtral.metal:45-101 (attention_gqa: query head h
// reads kv head h / (Hq/Hkv); scores q.k * 1/sqrt(d); softmax over the query's key range; 0 for an
// empty range) and :20-36 (rope_rotate_half), dispatched by Sources/DictatorEngine/Core/Ops.swift
// (Step.attention :136-169, Step.rope).  The reference keeps one sliding K/V window per session
// (Sources/DictatorEngine/Models/Voxtral.swift:206-250); here the caches of many sequences share
// one pool of fixed-size pages addressed through a block table.
//
// Design (HBM-bound: every K/V byte of every sequence is read once per step):
//  - split-K ("flash decoding"): workgroup = (kv head, 128-key split, sequence), 4 wave64s, kv head
//    fastest in the grid so that the workgroups in flight read whole pages.  The Hq/Hkv query heads
//    of a kv head share each K/V row read, so GQA costs no extra traffic;
//  - 16 B per lane loads: a head_dim row is D/8 lanes wide; K and V of the split are all issued
//    before the first score, V zeroed in registers outside the key range;
//  - scores: per-row dot products of the G query heads reduced together with a transposed DPP
//    butterfly inside the row's lanes; softmax of a split in LDS; P.V reduced across row groups with
//    v_permlane32_swap / v_permlane16_swap / DPP and across waves once through LDS;
//  - bf16 pages at head_dim 128 take gqa_split_mfma_kernel instead: the same split with K staged
//    in LDS by direct loads and both products on v_mfma_f32_16x16x32_bf16;
//  - a second kernel merges the splits of each (sequence, head) with the usual max/sum rescaling.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <type_traits>

#include "../../include/ud_decode.h"
#include "ud_common.hpp"

int ud_set_error(int code, const char* msg);   // encoder.hip

namespace ud {

constexpr int SPLIT = 128;      // keys per split workgroup (gqa_split_kernel)
constexpr int MSPLIT = 256;     // keys per split workgroup of gqa_split_mfma_kernel (32 per wave)
constexpr int PAGE = 16;        // block_size

// Element formats of 16-bit K/V and RoPE rows (both stored as uint16_t).
struct BF16 {};
struct F16 {};

template <typename T> struct KvTraits;
template <> struct KvTraits<BF16> {
    static __device__ __forceinline__ void unpack(uint4 v, float* f) { unpack16<bf16>(v, f); }
    static __device__ __forceinline__ float to_f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
    static __device__ __forceinline__ uint16_t from_f(float x) { return f2bf(x); }
};
template <> struct KvTraits<F16> {
    static __device__ __forceinline__ float h2f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }
    static __device__ __forceinline__ void unpack(uint4 v, float* f) {
        f[0] = h2f(v.x & 0xffffu); f[1] = h2f(v.x >> 16);
        f[2] = h2f(v.y & 0xffffu); f[3] = h2f(v.y >> 16);
        f[4] = h2f(v.z & 0xffffu); f[5] = h2f(v.z >> 16);
        f[6] = h2f(v.w & 0xffffu); f[7] = h2f(v.w >> 16);
    }
    static __device__ __forceinline__ float to_f(uint16_t u) { return h2f(u); }
    static __device__ __forceinline__ uint16_t from_f(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
};

// Transposed sum over the W lanes of a row (W in {8, 16}, aligned groups) of Q values per lane
// (Q <= W).  Steps pair lanes with row_mirror (W = 16), row_half_mirror, quad_perm [1,0,3,2] and
// [2,3,0,1]; the first log2(Q) of them keep half of the values (selected by lane bit 3, 2, 0, 1),
// the rest are plain sums.  Returns, in every lane, the row total of value index qidx(lane).
template <int CTRL, int N>
__device__ __forceinline__ void tkeep(float* v, bool bit) {
#pragma unroll
    for (int m = 0; m < N / 2; m++) {
        const float keep = bit ? v[m + N / 2] : v[m], send = bit ? v[m] : v[m + N / 2];
        v[m] = keep + dpp_mov<CTRL>(send);
    }
}
template <int CTRL, int K, int Q>
__device__ __forceinline__ void tstage(float* v, bool bit) {
    if constexpr ((1 << K) < Q) tkeep<CTRL, (Q >> K)>(v, bit);
    else v[0] += dpp_mov<CTRL>(v[0]);
}
template <int W, int Q>
__device__ __forceinline__ float tsum_row(float (&v)[Q], int lane) {
    static_assert((W == 8 || W == 16) && Q >= 1 && Q <= W, "row sum");
    if constexpr (W == 16) {
        tstage<DPP_ROW_MIRROR, 0, Q>(v, lane & 8);
        tstage<DPP_ROW_HALF_MIRROR, 1, Q>(v, lane & 4);
        tstage<DPP_QUAD_1032, 2, Q>(v, lane & 1);
        tstage<DPP_QUAD_2301, 3, Q>(v, lane & 2);
    } else {
        tstage<DPP_ROW_HALF_MIRROR, 0, Q>(v, lane & 4);
        tstage<DPP_QUAD_1032, 1, Q>(v, lane & 1);
        tstage<DPP_QUAD_2301, 2, Q>(v, lane & 2);
    }
    return v[0];
}
// Value index a lane holds after tsum_row, and whether it is the lane that reports it.
template <int W, int Q>
__device__ __forceinline__ int tsum_row_index(int lane, bool& writer) {
    constexpr int b[4] = {W == 16 ? 3 : 2, W == 16 ? 2 : 0, W == 16 ? 0 : 1, 1};
    int m = 0, rest = 0;
#pragma unroll
    for (int k = 0; k < (W == 16 ? 4 : 3); k++) {
        const int bit = (lane >> b[k]) & 1;
        if ((1 << k) < Q) m += bit * (Q >> (k + 1));
        else rest |= bit;
    }
    writer = rest == 0;
    return m;
}

// The packed bf16 dot product a.lo * b.lo + a.hi * b.hi + c (v_dot2_f32_bf16: exact bf16
// products, fp32 sum).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// a + (a from lane l^8) into lanes with bit 3 clear, b + ... into lanes with bit 3 set.
__device__ __forceinline__ float xsum8(float a, float b, bool bit3) {
    const float keep = bit3 ? b : a, send = bit3 ? a : b;
    return keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x128, 0xF, 0xF, false));
}

struct GqaArgs {
    const float* q;                // [n][M][Hq][D]
    const void* kp; const void* vp;
    const int32_t* bt;
    const int32_t* ranges;         // [n][M][2]
    float* part;                   // [n][M][Hq][NS][D + 2]: unnormalised sum, max, sum of exp
    int M;                         // queries per sequence (1 .. 8), all over the sequence's pages
    int max_blocks, Hq, Hkv, NS;
    int kmax;                      // keys the pages and the split grid can hold
    float scale;
};

template <typename KT, int D, int G>
__global__ __launch_bounds__(256) void gqa_split_kernel(GqaArgs a) {
    constexpr int LPR = D / 8, RG = 256 / LPR, NP = SPLIT / RG, NV = G * 8;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid / LPR, sub = tid % LPR;
    const int kvh = blockIdx.x, split = blockIdx.y, seq = blockIdx.z;
    const int M = a.M;
    const int32_t* rg = a.ranges + (int64_t)2 * seq * M;
    // the span of the queries' non-empty key ranges within this split
    int lo = a.kmax, hi = 0;
    for (int m = 0; m < M; m++) {
        const int l = max(rg[2 * m], 0), h = min(rg[2 * m + 1], a.kmax);
        if (l < h) { lo = min(lo, l); hi = max(hi, h); }
    }
    const int s0 = split * SPLIT;
    const int ulo = max(lo, s0), uhi = min(hi, s0 + SPLIT);
    if (ulo >= uhi) return;                       // this split holds no key of any query's range
    __shared__ float sc[G][SPLIT];
    __shared__ float stat[G][2];
    __shared__ __align__(16) float red[4][G][D];
    constexpr bool PK = std::is_same<KT, BF16>::value;

    // ---- K and V rows: key s0 + grp + RG p; pages outside [ulo, uhi) are never looked up.  A pass
    //      covers RG / PAGE whole pages (s0 is a multiple of 128), so a lane's page is
    //      (s0 + RG p) / PAGE + grp / PAGE: the page table entries are scalar loads, and a row's
    //      address is a scalar page base plus the lane's fixed offset (row grp % PAGE, 8 channels).
    const int blo = ulo / PAGE, bhi = (uhi - 1) / PAGE;
    const int32_t* bt = a.bt + (int64_t)seq * a.max_blocks;
    constexpr int PPP = RG / PAGE;                // pages per pass (1 for D = 128, 2 for D = 64)
    const uint32_t lane_off = (uint32_t)(((grp % PAGE) * D + sub * 8) * 2);   // bytes
    const int gp = grp / PAGE;                    // the lane's page within the pass
    const char* kp = static_cast<const char*>(a.kp);
    const char* vp = static_cast<const char*>(a.vp);
    // page bases in 64 bits: a pool may hold 2^32 elements or more (8 GiB of 16-bit K or V)
    const char* kb[NP][PPP];
    const char* vb[NP][PPP];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int e = 0; e < PPP; e++) {
            const int b = min(max((s0 + RG * p) / PAGE + e, blo), bhi);
            const int64_t base = ((int64_t)bt[b] * a.Hkv + kvh) * (PAGE * D * 2);
            kb[p][e] = kp + base;
            vb[p][e] = vp + base;
        }
    uint4 kr[NP], vr[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) kr[p] = ld16((PPP == 1 || gp == 0 ? kb[p][0] : kb[p][PPP - 1]) + lane_off);
#pragma unroll
    for (int p = 0; p < NP; p++) vr[p] = ld16((PPP == 1 || gp == 0 ? vb[p][0] : vb[p][PPP - 1]) + lane_off);

    // The split's K and V rows stay in registers while each query of the sequence is processed in
    // turn (one read of the pages for all M queries).
    for (int qm = 0; qm < M; qm++) {
    const int klo = max(max(rg[2 * qm], 0), s0), khi = min(min(rg[2 * qm + 1], a.kmax), s0 + SPLIT);
    if (klo >= khi) continue;                     // no key of this query's range here (uniform)
    // ---- the G query heads of this kv head (8 channels per lane); for bf16 pages also as bf16
    //      pairs (channels 2e, 2e + 1) for the packed dot products
    float q[G][8];
    uint32_t qb[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float* qr = a.q + ((int64_t)(seq * M + qm) * a.Hq + kvh * G + g) * D + sub * 8;
        const float4 x0 = *reinterpret_cast<const float4*>(qr), x1 = *reinterpret_cast<const float4*>(qr + 4);
        q[g][0] = x0.x; q[g][1] = x0.y; q[g][2] = x0.z; q[g][3] = x0.w;
        q[g][4] = x1.x; q[g][5] = x1.y; q[g][6] = x1.z; q[g][7] = x1.w;
        if constexpr (PK) {
#pragma unroll
            for (int e = 0; e < 4; e++) qb[g][e] = pack_bf16x2(q[g][2 * e], q[g][2 * e + 1]);
        }
    }

    // ---- scores of the G heads -> sc (masked keys -inf)
    bool writer;
    const int qi = tsum_row_index<LPR, G>(sub, writer);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        float part[G];
        if constexpr (PK) {
            const uint32_t kw[4] = {kr[p].x, kr[p].y, kr[p].z, kr[p].w};
#pragma unroll
            for (int g = 0; g < G; g++) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) acc = dot2_bf16(qb[g][e], kw[e], acc);
                part[g] = acc;
            }
        } else {
            float f[8];
            KvTraits<KT>::unpack(kr[p], f);
#pragma unroll
            for (int g = 0; g < G; g++) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) acc += q[g][e] * f[e];
                part[g] = acc;
            }
        }
        const float tot = tsum_row<LPR, G>(part, sub);
        const int jj = grp + RG * p, j = s0 + jj;
        if (writer) sc[qi][jj] = (j >= klo && j < khi) ? tot * a.scale : -INFINITY;
    }
    __syncthreads();

    // ---- softmax of the split, one wave per head: probabilities in sc, (max, sum) in stat
    for (int g = wave; g < G; g += 4) {
        float v[SPLIT / 64];
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < SPLIT / 64; k++) { v[k] = sc[g][lane + 64 * k]; m = fmaxf(m, v[k]); }
        m = wave_max(m);
        float l = 0.0f;
#pragma unroll
        for (int k = 0; k < SPLIT / 64; k++) {
            v[k] = v[k] == -INFINITY ? 0.0f : __expf(v[k] - m);
            l += v[k];
            sc[g][lane + 64 * k] = v[k];
        }
        l = wave_sum(l);
        if (lane == 0) { stat[g][0] = m; stat[g][1] = l; }
    }
    __syncthreads();

    // ---- P.V over this lane's rows (rows outside the range zeroed)
    float acc[NV];
#pragma unroll
    for (int f = 0; f < NV; f++) acc[f] = 0.0f;
    if constexpr (PK) {
        // bf16 pages: keys of passes p and p + 1 (rows jj and jj + RG of this lane) in pairs.
        // Channel c of the two V rows packed into one word, the two probabilities of head g
        // rounded to a bf16 pair, one v_dot2_f32_bf16 per (head, channel).
        static_assert(NP % 2 == 0, "key pairs");
#pragma unroll
        for (int p = 0; p < NP; p += 2) {
            const int jj = grp + RG * p, j = s0 + jj;
            const uint4 z = make_uint4(0, 0, 0, 0);
            const uint4 va = (j >= klo && j < khi) ? vr[p] : z;
            const uint4 vb2 = (j + RG >= klo && j + RG < khi) ? vr[p + 1] : z;
            const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb2.x, vb2.y, vb2.z, vb2.w};
            uint32_t x[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[2 * e] = __builtin_amdgcn_perm(wb[e], wa[e], 0x05040100u);       // (a lo, b lo)
                x[2 * e + 1] = __builtin_amdgcn_perm(wb[e], wa[e], 0x07060302u);   // (a hi, b hi)
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const uint32_t pp = pack_bf16x2(sc[g][jj], sc[g][jj + RG]);
#pragma unroll
                for (int c = 0; c < 8; c++) acc[g * 8 + c] = dot2_bf16(pp, x[c], acc[g * 8 + c]);
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int jj = grp + RG * p, j = s0 + jj;
            const bool in = j >= klo && j < khi;
            float f[8];
            KvTraits<KT>::unpack(in ? vr[p] : make_uint4(0, 0, 0, 0), f);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pg = sc[g][jj];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g * 8 + e] += pg * f[e];
            }
        }
    }
    // over the row groups of the wave (lanes with equal sub): xor 32, 16 (and 8 when LPR = 8)
    constexpr int S1 = NV / 2, S2 = NV / 4;
    float h1[S1], h2[S2];
#pragma unroll
    for (int m = 0; m < S1; m++) h1[m] = xsum32(acc[m], acc[m + S1]);
#pragma unroll
    for (int m = 0; m < S2; m++) h2[m] = xsum16(h1[m], h1[m + S2]);
    int fbase = ((lane >> 5) & 1) * S1 + ((lane >> 4) & 1) * S2;
    if constexpr (LPR == 16) {
#pragma unroll
        for (int m = 0; m < S2; m++) { const int f = fbase + m; red[wave][f / 8][sub * 8 + f % 8] = h2[m]; }
    } else {
        constexpr int S3 = NV / 8;
        float h3[S3];
#pragma unroll
        for (int m = 0; m < S3; m++) h3[m] = xsum8(h2[m], h2[m + S3], lane & 8);
        fbase += ((lane >> 3) & 1) * S3;
#pragma unroll
        for (int m = 0; m < S3; m++) { const int f = fbase + m; red[wave][f / 8][sub * 8 + f % 8] = h3[m]; }
    }
    __syncthreads();

    // ---- partial of each head: sum over the 4 waves, then (max, sum of exp)
    for (int idx = tid; idx < G * D; idx += 256) {
        const int g = idx / D, dd = idx % D;
        const float s = red[0][g][dd] + red[1][g][dd] + red[2][g][dd] + red[3][g][dd];
        float* pr = a.part + ((((int64_t)seq * M + qm) * a.Hq + kvh * G + g) * a.NS + split) * (D + 2);
        pr[dd] = s;
        if (dd == 0) { pr[D] = stat[g][0]; pr[D + 1] = stat[g][1]; }
    }
    if (qm + 1 < M) __syncthreads();              // sc, stat and red are reused by the next query
    }
}

// ---------------------------------------------------------------- bf16 pages, head_dim 128: MFMA
// gqa_split_kernel's design with the products on the matrix cores and no K in registers:
//  - 256-key splits, 8 waves of 32 keys (half the partials of 128-key splits);
//  - one 64 KB LDS tile holds K, then V: K rows go global -> LDS with direct loads
//    (global_load_lds_dwordx4) while V rows are loaded into registers; once every wave has read K,
//    V (rows outside the range zeroed) is written over it.  Rows are 256 bytes, their 16-byte
//    pieces permuted per row (kv_swz) by choosing each lane's source piece, so that the operand
//    reads below fall on distinct banks.  About 68 KB of LDS: two workgroups per CU;
//  - scores S^T = q . K^T on v_mfma_f32_16x16x32_bf16: A = q (rows = the G heads of the kv head,
//    rounded once to bf16, zero rows above G), B = K^T (lane (c, g): key c, channels 8g .. 8g + 7),
//    so lane (c, g) gets heads 4g .. 4g + 3 of key c;
//  - the softmax of the split as in gqa_split_kernel (probabilities in LDS);
//  - out^T = V^T . P^T: A = V^T by ds_read_b64_tr_b16, B = P^T (lane (c, g): head c's
//    probabilities rounded to bf16), wave w owning the 16-channel tiles w, w + (waves per
//    workgroup), .. over the split's keys, so no reduction across waves.
// V rows outside the key range are zeroed (pages may hold NaN there, and 0 x NaN is NaN); K rows
// outside it only feed scores that are replaced by -inf.
typedef short v4i16_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int kv_swz(int r, int p) {
    return r * 256 + ((p ^ (((r & 3) << 1) | ((r >> 2) & 1) | (r & 8))) << 4);
}

// 16 bytes per lane, global -> LDS at dst + 16 * lane (dst wave-uniform)
__device__ __forceinline__ void kv_direct16(const bf16* src, bf16* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

__device__ __forceinline__ v4i16_t kv_tr16(const char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)p);
}

// Query rows: the M queries of a sequence times the G query heads of the kv head, row r = m G + gh
// (QR = M G rows, at most QM; RT = ceil(QM / 16) MFMA tiles of 16 rows).  Every K/V row of the
// split is loaded once and multiplied against all of them.  QM == G is the one-query form.
template <int G, int QM>
__global__ __launch_bounds__(2 * MSPLIT) void gqa_split_mfma_kernel(GqaArgs a) {
    constexpr int D = 128, ROWB = 2 * D, KS = MSPLIT, NWV = KS / 32;
    constexpr int DPW = (8 + NWV - 1) / NWV;      // channel tiles per wave (the last ones may have fewer)
    constexpr int RT = (QM + 15) / 16;
    constexpr bool ONE = QM == G;                 // one query per sequence
    static_assert(KS % 64 == 0 && KS <= 256, "split of 64 .. 256 keys");
    static_assert(QM <= 64 && (ONE || QM % 16 == 0), "query rows");
    // the wave index as a wave-uniform value, so that the page lookups are scalar loads (a vector
    // load there would make the wait for it cover every load in flight)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, g = lane >> 4;
    const int kvh = blockIdx.x, split = blockIdx.y, seq = blockIdx.z;
    const int M = ONE ? 1 : a.M, QR = ONE ? G : M * G;
    const int32_t* rg = a.ranges + (int64_t)2 * seq * M;
    // the span of the queries' non-empty key ranges (scalar loads)
    int lo = a.kmax, hi = 0;
    for (int m = 0; m < M; m++) {
        const int l = max(rg[2 * m], 0), h = min(rg[2 * m + 1], a.kmax);
        if (l < h) { lo = min(lo, l); hi = max(hi, h); }
    }
    const int s0 = split * KS;
    const int klo = max(lo, s0), khi = min(hi, s0 + KS);
    if (klo >= khi) return;                       // this split holds no key of any query's range
    constexpr int PROW = KS * 2 + 16;             // bytes per probability row (bf16, padded by 16 bytes)
    __shared__ __align__(16) char kv[KS * ROWB];         // K, then V
    __shared__ __align__(16) char pl[QM * PROW];         // probabilities, bf16 [row][key]
    __shared__ float pmax[NWV][QM], psum[NWV][QM];       // per wave: row maxima, row sums of its 32 keys
    __shared__ int2 qrng[ONE ? 1 : 8];            // each query's range clipped to the split
    if (!ONE && tid < M) qrng[tid] = make_int2(max(max(rg[2 * tid], 0), s0), min(min(rg[2 * tid + 1], a.kmax), s0 + KS));

    // ---- K of the split into LDS, V into registers: wave w takes pages 2w, 2w + 1 of the split
    //      (rows 32w .. 32w + 31); each instruction covers 4 rows, lane L holding piece L % 16 of
    //      row L / 16 of them, which is source piece (L % 16) xor f(row).  Pages outside [klo, khi)
    //      are clamped to pages inside it (their rows are masked below).
    // q rows first (their loads issued before the K and V rows, so the wait below covers them)
    float4 qx[RT][4][2];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = min(16 * rt + col, QR - 1);
        const int m = ONE ? 0 : r / G, gh = ONE ? r : r % G;
        const float* qr = a.q + ((int64_t)(seq * M + m) * a.Hq + kvh * G + gh) * D + 8 * g;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            qx[rt][kc][0] = *reinterpret_cast<const float4*>(qr + 32 * kc);
            qx[rt][kc][1] = *reinterpret_cast<const float4*>(qr + 32 * kc + 4);
        }
    }
    // The wait below counts vector-memory operations: the 8 RT q loads, then the 8 direct K loads,
    // then the 8 V loads must be issued in that order, which the scheduling barriers pin.
    __builtin_amdgcn_sched_barrier(0);
    const int blo = klo / PAGE, bhi = (khi - 1) / PAGE;
    const int32_t* bt = a.bt + (int64_t)seq * a.max_blocks;
    const char* kp = static_cast<const char*>(a.kp);
    const char* vp = static_cast<const char*>(a.vp);
    // both page lookups before the first direct load (after it, the table is read by vector loads)
    int64_t pbase[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int b = min(max((s0 + 32 * wave + 16 * e) / PAGE, blo), bhi);
        pbase[e] = ((int64_t)bt[b] * a.Hkv + kvh) * (PAGE * ROWB);
    }
    int64_t off[2][4];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int r0 = 32 * wave + 16 * e;                           // first row of the page in the split
        const int64_t base = pbase[e];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int pr = 4 * i + (lane >> 4);                      // row within the page
            const int sp = (lane & 15) ^ (((pr & 3) << 1) | ((pr >> 2) & 1) | (pr & 8));
            off[e][i] = base + pr * ROWB + sp * 16;
            kv_direct16(reinterpret_cast<const bf16*>(kp + off[e][i]), reinterpret_cast<bf16*>(kv + (r0 + 4 * i) * ROWB));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 vr[2][4];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int i = 0; i < 4; i++) vr[e][i] = ld16(vp + off[e][i]);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));     // q and the K rows landed (the 8 V loads may not)
    // q as the A operand: lane (r, g) of tile rt holds row 16 rt + r's q[32kc + 8g .. + 7] in bf16
    // (zero for rows >= QR)
    uint4 qa[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            const float4 x0 = qx[rt][kc][0], x1 = qx[rt][kc][1];
            qa[rt][kc] = 16 * rt + col < QR ? make_uint4(pack_bf16x2(x0.x, x0.y), pack_bf16x2(x0.z, x0.w),
                                                         pack_bf16x2(x1.x, x1.y), pack_bf16x2(x1.z, x1.w))
                                            : make_uint4(0, 0, 0, 0);
        }
    __syncthreads();

    // ---- scores of the wave's keys 32w + 16t + c, in registers: sv[rt][t][i] is row 16 rt + 4g + i
    //      (-inf outside the row's range, and for padding rows)
    float sv[RT][2][4];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int r = 32 * wave + 16 * t + col;
        f32x4_t acc[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) acc[rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            const uint4 kb = *reinterpret_cast<const uint4*>(kv + kv_swz(r, 4 * kc + g));
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa[rt][kc]), as_bf16x8(kb), acc[rt], 0, 0, 0);
        }
        const int j = s0 + r;
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 16 * rt + 4 * g + i;
                bool in;
                if constexpr (ONE) {
                    in = row < QR && j >= klo && j < khi;
                } else {
                    const int2 qq = qrng[min(row, QR - 1) / G];
                    in = row < QR && j >= qq.x && j < qq.y;
                }
                sv[rt][t][i] = in ? acc[rt][i] * a.scale : -INFINITY;
            }
    }
    // the wave's row maxima over its 32 keys (the 16 lanes of a row group hold one key each)
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 16 * rt + 4 * g + i;
            const float m = group_max<16>(fmaxf(sv[rt][0][i], sv[rt][1][i]));
            if (col == 0 && row < QM) pmax[wave][row] = m;
        }
    __syncthreads();                              // every wave has read K and posted its maxima

    // ---- V over K in LDS, where the direct loads put K (rows outside the span zeroed)
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 32 * wave + 16 * e + 4 * i + (lane >> 4), j = s0 + r;
            const uint4 v = (j >= klo && j < khi) ? vr[e][i] : make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4*>(kv + (32 * wave + 16 * e + 4 * i) * ROWB + 16 * lane) = v;
        }

    // ---- softmax of the split from registers: probabilities exp(s - row max) rounded to bf16 into
    //      pl, the wave's row sums into psum (a row with no key in the split: max -inf, all 0)
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 16 * rt + 4 * g + i, rr = min(row, QM - 1);
            float m = pmax[0][rr];
#pragma unroll
            for (int w = 1; w < NWV; w++) m = fmaxf(m, pmax[w][rr]);
            float l = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const float pv = sv[rt][t][i] == -INFINITY ? 0.0f : __expf(sv[rt][t][i] - m);
                l += pv;
                if (row < QM) *reinterpret_cast<uint16_t*>(pl + row * PROW + (32 * wave + 16 * t + col) * 2) = f2bf(pv);
            }
            l = group_sum<16>(l);
            if (col == 0 && row < QM) psum[wave][row] = l;
        }
    __syncthreads();

    // ---- out^T += V^T . P^T per 32-key piece kk.  B (tile rt): lane (c, g) holds row 16 rt + c's
    //      probabilities of keys 32kk + 4g + e (e < 4), then 32kk + 16 + 4g + e; A: V^T over the
    //      same keys (lane c of a 16-lane group reads column c & 3 of rows 32kk + 4g + c / 4 and,
    //      16 keys on, of rows 32kk + 16 + 4g + c / 4: channels 16dt + 4(c & 3) .., half c & 1 of
    //      piece pc), shared by the RT tiles
    f32x4_t oacc[DPW][RT];
#pragma unroll
    for (int u = 0; u < DPW; u++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) oacc[u][rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < KS / 32; kk++) {
        uint4 pb[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const char* pr = pl + min(16 * rt + col, QM - 1) * PROW + (32 * kk + 4 * g) * 2;
            const uint2 p0 = *reinterpret_cast<const uint2*>(pr);           // keys 32kk + 4g .. + 3
            const uint2 p1 = *reinterpret_cast<const uint2*>(pr + 32);      // 16 keys on
            pb[rt] = 16 * rt + col < QR ? make_uint4(p0.x, p0.y, p1.x, p1.y) : make_uint4(0, 0, 0, 0);
        }
        const int k0 = 32 * kk + 4 * g + (col >> 2);
#pragma unroll
        for (int u = 0; u < DPW; u++) {
            const int dt = wave + NWV * u;                // wave-uniform
            if (dt >= 8) break;
            const int pc = 2 * dt + ((col & 3) >> 1), hb = (col & 1) * 8;
            const v4i16_t b0 = kv_tr16(kv + kv_swz(k0, pc) + hb);
            const v4i16_t b1 = kv_tr16(kv + kv_swz(k0 + 16, pc) + hb);
            uint4 av;
            __builtin_memcpy(&av.x, &b0, 8);
            __builtin_memcpy(&av.z, &b1, 8);
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                oacc[u][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(pb[rt]), oacc[u][rt], 0, 0, 0);
        }
    }

    // ---- partial of row 16 rt + c (query m, head gh): out^T lane (c, g) holds channels
    //      16dt + 4g .. + 3; (max, sum) from the waves' row maxima and sums
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int row = 16 * rt + col;
        if (row < QR) {
            const int m = ONE ? 0 : row / G, gh = ONE ? row : row % G;
            float* pr = a.part + ((((int64_t)seq * M + m) * a.Hq + kvh * G + gh) * a.NS + split) * (D + 2);
#pragma unroll
            for (int u = 0; u < DPW; u++) {
                if (wave + NWV * u >= 8) break;
                float* o = pr + 16 * (wave + NWV * u) + 4 * g;
                *reinterpret_cast<float2*>(o) = make_float2(oacc[u][rt][0], oacc[u][rt][1]);
                *reinterpret_cast<float2*>(o + 2) = make_float2(oacc[u][rt][2], oacc[u][rt][3]);
            }
            if (wave == 0 && g == 0) {
                float m = pmax[0][row], l = psum[0][row];
#pragma unroll
                for (int w = 1; w < NWV; w++) { m = fmaxf(m, pmax[w][row]); l += psum[w][row]; }
                pr[D] = m;
                pr[D + 1] = l;
            }
        }
    }
}

// Merge the splits of one (sequence, head), one wave: out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.
// Lane s holds split s's (max, sum) of a chunk of up to 64 splits; the weights reach every lane
// with readlane, and the dims (D/64 per lane) accumulate.  The partials of a chunk's first CB
// splits are loaded together with its statistics, before the reductions that give the weights, so
// a chunk of up to CB splits (4,096 keys) costs one round trip to memory instead of one per 8
// splits after the statistics.
template <int D>
__global__ __launch_bounds__(64) void gqa_combine_kernel(const float* part, const int32_t* ranges, float* out,
                                                         int Hq, int NS, int kmax, int split) {
    constexpr int DL = D / 64, CB = 32;
    const int h = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
    const int lo = max(ranges[2 * seq], 0), hi = min(ranges[2 * seq + 1], kmax);
    float* o = out + ((int64_t)seq * Hq + h) * D;
    if (lo >= hi) {
#pragma unroll
        for (int k = 0; k < DL; k++) o[lane + 64 * k] = 0.0f;
        return;
    }
    const int sa = lo / split, sb = (hi - 1) / split;
    const float* pr = part + ((int64_t)seq * Hq + h) * NS * (D + 2);
    float M = -INFINITY, L = 0.0f, acc[DL];
#pragma unroll
    for (int k = 0; k < DL; k++) acc[k] = 0.0f;
    for (int c0 = sa; c0 <= sb; c0 += 64) {
        const int cnt = min(64, sb - c0 + 1);
        const float m = lane < cnt ? pr[(c0 + lane) * (D + 2) + D] : -INFINITY;
        const float l = lane < cnt ? pr[(c0 + lane) * (D + 2) + D + 1] : 0.0f;
        float x[CB][DL];
#pragma unroll
        for (int u = 0; u < CB; u++) {
            if (u < cnt) {                            // wave-uniform
#pragma unroll
                for (int k = 0; k < DL; k++) x[u][k] = pr[(c0 + u) * (D + 2) + lane + 64 * k];
            }
        }
        const float nm = fmaxf(M, wave_max(m));
        const float keep = M == -INFINITY ? 0.0f : __expf(M - nm);
        const float w = lane < cnt ? __expf(m - nm) : 0.0f;
        L = L * keep + wave_sum(w * l);
#pragma unroll
        for (int k = 0; k < DL; k++) acc[k] *= keep;
#pragma unroll
        for (int u = 0; u < CB; u++) {
            if (u < cnt) {
                const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
#pragma unroll
                for (int k = 0; k < DL; k++) acc[k] += wu * x[u][k];
            }
        }
        for (int s0 = CB; s0 < cnt; s0 += 8) {        // the rest of the chunk, 8 splits' loads in flight at a time
            float ws[8], y[8][DL];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int si = min(s0 + u, cnt - 1);
                ws[u] = s0 + u < cnt ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), si)) : 0.0f;
                const float* ps = pr + (c0 + si) * (D + 2);
#pragma unroll
                for (int k = 0; k < DL; k++) y[u][k] = ps[lane + 64 * k];
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int k = 0; k < DL; k++) acc[k] += ws[u] * y[u][k];
        }
        M = nm;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int k = 0; k < DL; k++) o[lane + 64 * k] = acc[k] * inv;
}

// ---------------------------------------------------------------- RoPE
template <typename T> struct RopeIO;    // fp32 rows, or 16-bit rows of format T
template <> struct RopeIO<float> {
    typedef float S;
    static __device__ float ld(const float* p) { return *p; }
    static __device__ void st(float* p, float v) { *p = v; }
};
template <typename F> struct RopeIO {
    typedef uint16_t S;
    static __device__ float ld(const uint16_t* p) { return KvTraits<F>::to_f(*p); }
    static __device__ void st(uint16_t* p, float v) { *p = KvTraits<F>::from_f(v); }
};

template <typename T>
__global__ void rope_kernel(typename RopeIO<T>::S* x, int rows, int H, int d, int ld, const int32_t* pos, int pos0,
                            const float* inv_freq) {
    const int half = d / 2;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * H * half) return;
    const int i = (int)(idx % half), h = (int)((idx / half) % H), t = (int)(idx / ((int64_t)half * H));
    const int p = pos ? pos[t] : pos0 + t;
    const float angle = (float)p * inv_freq[i];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    typename RopeIO<T>::S* row = x + (int64_t)t * ld + h * d;
    const float u = RopeIO<T>::ld(row + i), v = RopeIO<T>::ld(row + i + half);
    RopeIO<T>::st(row + i, u * cs - v * sn);
    RopeIO<T>::st(row + i + half, v * cs + u * sn);
}

// ---------------------------------------------------------------- paged append
template <int D>
__global__ void kv_append_kernel(const uint16_t* kn, const uint16_t* vn, uint16_t* kp, uint16_t* vp, const int32_t* bt,
                                 int max_blocks, const int32_t* pos, int Hkv) {
    const int seq = blockIdx.x, kvh = blockIdx.y, c = threadIdx.x;   // c: 16-byte chunk of the row
    const int p = min(max(pos[seq], 0), max_blocks * PAGE - 1);
    const int phys = bt[(int64_t)seq * max_blocks + p / PAGE];
    const int64_t dst = (((int64_t)phys * Hkv + kvh) * PAGE + p % PAGE) * D + c * 8;
    const int64_t src = ((int64_t)seq * Hkv + kvh) * D + c * 8;
    st16(kp + dst, ld16(kn + src));
    st16(vp + dst, ld16(vn + src));
}

}  // namespace ud

using namespace ud;

static int dfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return ud_set_error(code, buf);
}

static int nsplits(int32_t max_keys, int split = SPLIT) { return max_keys <= 0 ? 1 : (max_keys + split - 1) / split; }

extern "C" UD_API size_t ud_gqa_workspace_bytes(int32_t n, int32_t q_heads, int32_t head_dim, int32_t max_keys) {
    if (n <= 0 || q_heads <= 0 || head_dim <= 0) return 0;
    return (size_t)n * q_heads * nsplits(max_keys) * (head_dim + 2) * sizeof(float);
}

// The MFMA split kernel for G query heads per kv head and M queries per sequence: QM query rows
// (G for one query, else M G rounded up to whole 16-row tiles).
template <int G>
static int launch_mfma_g(const GqaArgs& a, dim3 grid, dim3 block, hipStream_t st) {
    const int rows = a.M * G;
    if (a.M == 1) { hipLaunchKernelGGL((gqa_split_mfma_kernel<G, G>), grid, block, 0, st, a); return UD_OK; }
    if (rows <= 16) { hipLaunchKernelGGL((gqa_split_mfma_kernel<G, 16>), grid, block, 0, st, a); return UD_OK; }
    if constexpr (G >= 4) {
        if (rows <= 32) { hipLaunchKernelGGL((gqa_split_mfma_kernel<G, 32>), grid, block, 0, st, a); return UD_OK; }
    }
    if constexpr (G == 8) {
        if (rows <= 48) { hipLaunchKernelGGL((gqa_split_mfma_kernel<G, 48>), grid, block, 0, st, a); return UD_OK; }
        if (rows <= 64) { hipLaunchKernelGGL((gqa_split_mfma_kernel<G, 64>), grid, block, 0, st, a); return UD_OK; }
    }
    return UD_ERR_SHAPE;
}

// Grid of the split kernels: (kv head, split, sequence); the combine runs over the n M (sequence,
// query) rows, whose ranges, partials and outputs are contiguous in that order.
template <typename KT, int D>
static int launch_gqa(const GqaArgs& a, int n, int G, int nsplit, float* out, hipStream_t st) {
    if constexpr (std::is_same<KT, BF16>::value && D == 128) {
        // bf16 pages at head_dim 128: the MFMA split kernel (grid as below)
        dim3 grid(a.Hkv, nsplit, n), block(2 * MSPLIT);
        int rc;
        switch (G) {
            case 1: rc = launch_mfma_g<1>(a, grid, block, st); break;
            case 2: rc = launch_mfma_g<2>(a, grid, block, st); break;
            case 4: rc = launch_mfma_g<4>(a, grid, block, st); break;
            case 8: rc = launch_mfma_g<8>(a, grid, block, st); break;
            default: return UD_ERR_SHAPE;
        }
        if (rc != UD_OK) return rc;
        hipLaunchKernelGGL((gqa_combine_kernel<D>), dim3(a.Hq, n * a.M), dim3(64), 0, st, a.part, a.ranges, out, a.Hq,
                           a.NS, a.kmax, MSPLIT);
        return UD_OK;
    }
    // kv head fastest: the Hkv workgroups of one split run side by side and read each physical page's
    // Hkv x 4 KB as one contiguous block ([page][kv head][row][dim]); with the split fastest, the
    // workgroups in flight read scattered 4 KB pieces (measured on MI355X at 64 sequences, 8 kv
    // heads: 123.7 us per call against 143.8, and 106.0 against 113.1 for loads alone)
    dim3 grid(a.Hkv, nsplit, n), block(256);
    switch (G) {
        case 1: hipLaunchKernelGGL((gqa_split_kernel<KT, D, 1>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((gqa_split_kernel<KT, D, 2>), grid, block, 0, st, a); break;
        case 4: hipLaunchKernelGGL((gqa_split_kernel<KT, D, 4>), grid, block, 0, st, a); break;
        case 8: hipLaunchKernelGGL((gqa_split_kernel<KT, D, 8>), grid, block, 0, st, a); break;
        default: return UD_ERR_SHAPE;
    }
    hipLaunchKernelGGL((gqa_combine_kernel<D>), dim3(a.Hq, n * a.M), dim3(64), 0, st, a.part, a.ranges, out, a.Hq, a.NS,
                       a.kmax, SPLIT);
    return UD_OK;
}

// Argument checks shared by both decode entry points (everything but the workspace).
static int gqa_check(const char* who, int32_t kv_dtype, const float* q_dev, const void* k_pages, const void* v_pages,
                     const int32_t* block_table, int32_t max_blocks, const int32_t* ranges_dev, const float* out_dev,
                     int32_t n, int32_t n_queries, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                     int32_t block_size, int32_t max_keys) {
    if (!q_dev || !k_pages || !v_pages || !block_table || !ranges_dev || !out_dev)
        return dfail(UD_ERR_INVALID, "%s: null pointer", who);
    if (n_queries < 1 || n_queries > 8) return dfail(UD_ERR_SHAPE, "%s: %d queries per sequence (1 .. 8)", who, n_queries);
    if (kv_dtype != UD_BF16 && kv_dtype != UD_F16) return dfail(UD_ERR_INVALID, "%s: kv dtype %d", who, kv_dtype);
    if (n < 1 || q_heads < 1 || kv_heads < 1 || q_heads % kv_heads)
        return dfail(UD_ERR_SHAPE, "%s: heads %d/%d, n %d", who, q_heads, kv_heads, n);
    const int G = q_heads / kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) return dfail(UD_ERR_SHAPE, "%s: group %d not in {1,2,4,8}", who, G);
    if (head_dim != 64 && head_dim != 128) return dfail(UD_ERR_SHAPE, "%s: head_dim %d", who, head_dim);
    if (block_size != PAGE) return dfail(UD_ERR_SHAPE, "%s: block_size %d (16 supported)", who, block_size);
    if (max_blocks < 1 || max_keys < 0 || max_keys > max_blocks * PAGE)
        return dfail(UD_ERR_SHAPE, "%s: max_keys %d beyond %d blocks", who, max_keys, max_blocks);
    // grid y (splits) and z (sequences) of the split kernels, and y (sequence x query rows) of the
    // combine, hold at most 65535 workgroups
    if ((int64_t)n * n_queries > 65535 || nsplits(max_keys) > 65535)
        return dfail(UD_ERR_SHAPE, "%s: n %d x %d queries or max_keys %d beyond the grid (65535 rows, 65535 x %d keys)",
                     who, n, n_queries, max_keys, SPLIT);
    if (((uintptr_t)q_dev | (uintptr_t)k_pages | (uintptr_t)v_pages) & 15)
        return dfail(UD_ERR_INVALID, "%s: buffers must be 16-byte aligned", who);
    return UD_OK;
}

// Launches split + combine with `workspace` as the split partials (checked by the caller).
static int gqa_launch(const char* who, int32_t kv_dtype, const float* q_dev, const void* k_pages, const void* v_pages,
                      const int32_t* block_table, int32_t max_blocks, const int32_t* ranges_dev, float* out_dev,
                      int32_t n, int32_t n_queries, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                      int32_t max_keys, float* workspace, hipStream_t st) {
    const int G = q_heads / kv_heads;
    GqaArgs a{};
    a.q = q_dev; a.kp = k_pages; a.vp = v_pages; a.bt = block_table; a.ranges = ranges_dev;
    a.part = workspace;
    a.M = n_queries;
    // keys per split: MSPLIT on the MFMA path (bf16 pages, head_dim 128), SPLIT otherwise; the
    // workspace is sized for SPLIT, the smaller, so it holds either
    const int sp = kv_dtype == UD_BF16 && head_dim == 128 ? MSPLIT : SPLIT;
    a.max_blocks = max_blocks; a.Hq = q_heads; a.Hkv = kv_heads; a.NS = nsplits(max_keys, sp);
    a.kmax = min(max_blocks * PAGE, a.NS * sp);
    a.scale = 1.0f / sqrtf((float)head_dim);
    int rc;
    if (kv_dtype == UD_BF16)
        rc = head_dim == 128 ? launch_gqa<BF16, 128>(a, n, G, a.NS, out_dev, st) : launch_gqa<BF16, 64>(a, n, G, a.NS, out_dev, st);
    else
        rc = head_dim == 128 ? launch_gqa<F16, 128>(a, n, G, a.NS, out_dev, st) : launch_gqa<F16, 64>(a, n, G, a.NS, out_dev, st);
    if (rc != UD_OK) return dfail(rc, "%s: unsupported shape", who);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dfail(UD_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    return UD_OK;
}

extern "C" UD_API int ud_gqa_attention_paged(int32_t kv_dtype, const float* q_dev, const void* k_pages,
                                             const void* v_pages, const int32_t* block_table, int32_t max_blocks,
                                             const int32_t* ranges_dev, float* out_dev, int32_t n, int32_t q_heads,
                                             int32_t kv_heads, int32_t head_dim, int32_t block_size, int32_t max_keys,
                                             void* workspace, size_t workspace_bytes, void* hip_stream) {
    return ud_gqa_attention_paged_mq(kv_dtype, q_dev, k_pages, v_pages, block_table, max_blocks, ranges_dev, out_dev, n,
                                     1, q_heads, kv_heads, head_dim, block_size, max_keys, workspace, workspace_bytes,
                                     hip_stream);
}

extern "C" UD_API int ud_gqa_attention_paged_mq(int32_t kv_dtype, const float* q_dev, const void* k_pages,
                                                const void* v_pages, const int32_t* block_table, int32_t max_blocks,
                                                const int32_t* ranges_dev, float* out_dev, int32_t n, int32_t n_queries,
                                                int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t block_size,
                                                int32_t max_keys, void* workspace, size_t workspace_bytes,
                                                void* hip_stream) {
    const char* who = n_queries == 1 ? "ud_gqa_attention_paged" : "ud_gqa_attention_paged_mq";
    int rc = gqa_check(who, kv_dtype, q_dev, k_pages, v_pages, block_table, max_blocks, ranges_dev, out_dev, n,
                       n_queries, q_heads, kv_heads, head_dim, block_size, max_keys);
    if (rc != UD_OK) return rc;
    const size_t need = ud_gqa_workspace_bytes(n * n_queries, q_heads, head_dim, max_keys);
    if (!workspace) return dfail(UD_ERR_INVALID, "%s: null workspace", who);
    if (workspace_bytes < need) return dfail(UD_ERR_SHAPE, "%s: workspace %zu < %zu bytes", who, workspace_bytes, need);
    if ((uintptr_t)workspace & 15) return dfail(UD_ERR_INVALID, "%s: workspace must be 16-byte aligned", who);
    return gqa_launch(who, kv_dtype, q_dev, k_pages, v_pages, block_table, max_blocks, ranges_dev, out_dev, n, n_queries,
                      q_heads, kv_heads, head_dim, max_keys, static_cast<float*>(workspace),
                      static_cast<hipStream_t>(hip_stream));
}

// ---------------------------------------------------------------- allocation-free variant
// The split partials of ud_gqa_attention_paged_noalloc live in this file-scope device array, one
// copy per device, held until the process ends.  In host code `scratch` names a host-side stand-in,
// not device memory: kernels get the address that hipGetSymbolAddress returned for the current
// device (kept per device below), never the array's name.  No clearing is needed: the combine
// kernel reads only the splits holding a key of the sequence's range, and the split kernel of each
// of them writes its whole partial first (same stream).  Calls that overlap on one device race on
// these bytes.
static __device__ __align__(256) float scratch[UD_GQA_NOALLOC_SCRATCH_BYTES / sizeof(float)];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_dev[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up once per device, with that device current).
static int scratch_of_current_device(const char* who, float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return dfail(UD_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return dfail(UD_ERR_HIP, "%s: device %d beyond %d", who, dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return dfail(UD_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", who, hipGetErrorString(e));
        g_scratch_dev[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_dev[dev];
    return UD_OK;
}

extern "C" UD_API int ud_gqa_attention_paged_noalloc(int32_t kv_dtype, const float* q_dev, const void* k_pages,
                                                     const void* v_pages, const int32_t* block_table,
                                                     int32_t max_blocks, const int32_t* ranges_dev, float* out_dev,
                                                     int32_t n, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                                     int32_t block_size, int32_t max_keys, void* hip_stream) {
    static const char* who = "ud_gqa_attention_paged_noalloc";
    int rc = gqa_check(who, kv_dtype, q_dev, k_pages, v_pages, block_table, max_blocks, ranges_dev, out_dev, n, 1,
                       q_heads, kv_heads, head_dim, block_size, max_keys);
    if (rc != UD_OK) return rc;
    const size_t need = ud_gqa_workspace_bytes(n, q_heads, head_dim, max_keys);
    if (need > (size_t)UD_GQA_NOALLOC_SCRATCH_BYTES)
        return dfail(UD_ERR_SHAPE, "%s: %d sequences x %d heads x %d keys need %zu bytes of split partials, beyond the "
                     "%zu-byte static scratch (UD_GQA_NOALLOC_SCRATCH_BYTES); use ud_gqa_attention_paged with a "
                     "workspace", who, n, q_heads, max_keys, need, (size_t)UD_GQA_NOALLOC_SCRATCH_BYTES);
    float* ws = nullptr;
    if ((rc = scratch_of_current_device(who, &ws)) != UD_OK) return rc;
    return gqa_launch(who, kv_dtype, q_dev, k_pages, v_pages, block_table, max_blocks, ranges_dev, out_dev, n, 1, q_heads,
                      kv_heads, head_dim, max_keys, ws, static_cast<hipStream_t>(hip_stream));
}

extern "C" UD_API int ud_rope_rotate_half(int32_t dtype, void* x_dev, int32_t rows, int32_t heads, int32_t head_dim,
                                          int32_t ld, const int32_t* positions_dev, int32_t pos0,
                                          const float* inv_freq_dev, void* hip_stream) {
    if (!x_dev || !inv_freq_dev) return dfail(UD_ERR_INVALID, "ud_rope_rotate_half: null pointer");
    if (rows < 0 || heads < 1 || head_dim < 2 || head_dim % 2 || ld < heads * head_dim)
        return dfail(UD_ERR_SHAPE, "ud_rope_rotate_half: rows %d heads %d head_dim %d ld %d", rows, heads, head_dim, ld);
    if (rows == 0) return UD_OK;
    const int64_t total = (int64_t)rows * heads * (head_dim / 2);
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    switch (dtype) {
        case UD_F32: hipLaunchKernelGGL(rope_kernel<float>, grid, block, 0, st, static_cast<float*>(x_dev), rows, heads, head_dim, ld, positions_dev, pos0, inv_freq_dev); break;
        case UD_BF16: hipLaunchKernelGGL(rope_kernel<BF16>, grid, block, 0, st, static_cast<uint16_t*>(x_dev), rows, heads, head_dim, ld, positions_dev, pos0, inv_freq_dev); break;
        case UD_F16: hipLaunchKernelGGL(rope_kernel<F16>, grid, block, 0, st, static_cast<uint16_t*>(x_dev), rows, heads, head_dim, ld, positions_dev, pos0, inv_freq_dev); break;
        default: return dfail(UD_ERR_INVALID, "ud_rope_rotate_half: dtype %d", dtype);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dfail(UD_ERR_HIP, "ud_rope_rotate_half: %s", hipGetErrorString(e));
    return UD_OK;
}

extern "C" UD_API int ud_paged_kv_append(int32_t kv_dtype, const void* k_new, const void* v_new, void* k_pages,
                                         void* v_pages, const int32_t* block_table, int32_t max_blocks,
                                         const int32_t* positions_dev, int32_t n, int32_t kv_heads, int32_t head_dim,
                                         int32_t block_size, void* hip_stream) {
    if (!k_new || !v_new || !k_pages || !v_pages || !block_table || !positions_dev)
        return dfail(UD_ERR_INVALID, "ud_paged_kv_append: null pointer");
    if (kv_dtype != UD_BF16 && kv_dtype != UD_F16) return dfail(UD_ERR_INVALID, "ud_paged_kv_append: kv dtype %d", kv_dtype);
    if (n < 0 || kv_heads < 1 || (head_dim != 64 && head_dim != 128) || block_size != PAGE || max_blocks < 1)
        return dfail(UD_ERR_SHAPE, "ud_paged_kv_append: n %d kv_heads %d head_dim %d block %d", n, kv_heads, head_dim, block_size);
    if (((uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)k_pages | (uintptr_t)v_pages) & 15)
        return dfail(UD_ERR_INVALID, "ud_paged_kv_append: buffers must be 16-byte aligned");
    if (n == 0) return UD_OK;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const uint16_t* kn = static_cast<const uint16_t*>(k_new);
    const uint16_t* vn = static_cast<const uint16_t*>(v_new);
    uint16_t* kp = static_cast<uint16_t*>(k_pages);
    uint16_t* vp = static_cast<uint16_t*>(v_pages);
    if (head_dim == 128) hipLaunchKernelGGL(kv_append_kernel<128>, dim3(n, kv_heads), dim3(16), 0, st, kn, vn, kp, vp, block_table, max_blocks, positions_dev, kv_heads);
    else hipLaunchKernelGGL(kv_append_kernel<64>, dim3(n, kv_heads), dim3(8), 0, st, kn, vn, kp, vp, block_table, max_blocks, positions_dev, kv_heads);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dfail(UD_ERR_HIP, "ud_paged_kv_append: %s", hipGetErrorString(e));
    return UD_OK;
}
