// Fused relative-position multi-head attention for gfx950.
//
// Semantics: Sources/DictatorEngine/Metal/20_conformer.metal:140-220 (relpos_attention) as
// dispatched by Sources/DictatorEngine/Core/Ops.swift:80-90.  For query i, head h, key j in the
// query's range:
//     s_ij = ((q_i + u_h) . k_j + (q_i + v_h) . P[(Tk - Tq + i) - j + rel_offset]) * scale
//     out_i = sum_j softmax_j(s_ij) v_j          (0 when the range is empty)
// which is NeMo's  ac + rel_shift(bd)  with the pad/view shift folded into the P row index.
//
// Design (one workgroup of 4 wave64s per (sequence, head)):
//  - keys are processed in blocks of KB rows with an online softmax, so any Tk works;
//  - every K row, V row and P-band row of a block is fetched with one 16-byte load per lane
//    (LPR = head_dim*sizeof/16 lanes per row), all issued before any arithmetic, so a workgroup
//    has the whole block in flight;
//  - bd is computed once per P row of the block's band (band = keys + queries - 1 rows, shared by
//    all queries) rather than once per (query, key): rel_shift becomes the index i - jj + nk - 1;
//  - dot products are reduced inside the LPR-lane row group with DPP; softmax max/sum are wave64
//    DPP/shuffle reductions; V is staged in LDS and the P.V product is done by threads that own
//    (query, channel) outputs.
//  - ring mode: keys are the window [L cached ; T new] of the stream's [H][R][dk] rings, key j in
//    row (start + j) mod R; the QKV projection (or launch_ring_append) has written the T new rows
//    before the launch, so the attention kernels only read the rings.
#include "ud_common.hpp"
#include "kernels.hpp"

namespace ud {

template <typename T, int DK, int TQ, int KB>
struct AttnCfg {
    static constexpr int NT = 256;
    static constexpr int VEC = Vec16<T>::N;
    static constexpr int LPR = DK / VEC;               // lanes per row
    static constexpr int G = NT / LPR;                 // rows per pass
    static constexpr int NB = KB + TQ - 1;             // band rows per block
    static constexpr int KR = (KB + G - 1) / G;        // K (and V) rows per thread
    static constexpr int PR = (NB + G - 1) / G;        // P rows per thread
    static constexpr int OUTS = (TQ * DK + NT - 1) / NT;
    static_assert(LPR >= 1 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "lanes per row");
};

// Source adaptor: reference layout (Q [Tq, H*dk], K/V [Tk, H*dk], P [n_rel, H*dk]).
template <typename T>
struct OpSrc {
    const T* Q; const T* K; const T* V; const T* P; T* O;
    const float* u; const float* vb; const int32_t* ranges;
    int Tq, Tk, ld, hoff, rel_offset, n_rel;
    __device__ const T* qrow(int i) const { return Q + (int64_t)i * ld + hoff; }
    __device__ const T* krow(int j) const { return K + (int64_t)j * ld + hoff; }
    __device__ const T* vrow(int j) const { return V + (int64_t)j * ld + hoff; }
    __device__ const T* prow(int r) const { return P + (int64_t)r * ld + hoff; }
    __device__ void store(int i, int d, float v) const { O[(int64_t)i * ld + hoff + d] = from_f<T>(v); }
    __device__ void range(int i, int& ks, int& ke) const {
        ks = max(ranges[2 * i], 0);
        ke = min(ranges[2 * i + 1], Tk);
    }
};

// Source adaptor: streaming step over one stream's ring caches.
template <typename T>
struct RingSrc {
    const T* kr; const T* vr;      // this (stream, head) ring slice: [R][dk]
    const T* qkv;                  // first row of this stream in [n*T, 3*D] (q columns)
    const T* P; T* O;              // P [n_rel, D]; O = att [n*T, D] (16-bit: fragment-major)
    const float* u; const float* vb;
    int Tq, Tk, R, D, hoff, start, rel_offset, n_rel, ks, ke;
    int64_t row0;                  // global row of this stream's first query
    bool frag;                     // 16-bit output in the fragment-major layout
    __device__ const T* qrow(int i) const { return qkv + (int64_t)i * 3 * D + hoff; }
    // key j < L + T <= R of the window: ring row start + j (< 2R) mod R
    __device__ const T* krow(int j) const { int s = start + j; s -= (s >= R) ? R : 0; return kr + (int64_t)s * 128; }
    __device__ const T* vrow(int j) const { int s = start + j; s -= (s >= R) ? R : 0; return vr + (int64_t)s * 128; }
    __device__ const T* prow(int r) const { return P + (int64_t)r * D + hoff; }
    // The output feeds linear_out: 16-bit goes fragment-major (the GEMM's operand order).
    __device__ void store(int i, int d, float v) const {
        if (sizeof(T) == 2 && frag) O[frag_index(row0 + i, hoff + d, D / 64)] = from_f<T>(v);
        else O[(row0 + i) * D + hoff + d] = from_f<T>(v);
    }
    __device__ void range(int, int& s, int& e) const { s = ks; e = ke; }
};

template <typename T, int DK, int TQ, int KB, typename Src>
__device__ __forceinline__ void relpos_core(const Src& src, float scale) {
    using C = AttnCfg<T, DK, TQ, KB>;
    constexpr int NT = C::NT, VEC = C::VEC, LPR = C::LPR, G = C::G;
    __shared__ float qu[TQ][DK];
    __shared__ float qv[TQ][DK];
    __shared__ float sc[TQ][KB];
    __shared__ float bd[TQ][C::NB];
    __shared__ __attribute__((aligned(16))) T vs[KB][DK];
    __shared__ float mrow[TQ], lrow[TQ], crow[TQ];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid / LPR, sub = tid % LPR;
    const int Tq = src.Tq, Tk = src.Tk;

    for (int idx = tid; idx < Tq * DK; idx += NT) {
        int i = idx / DK, d = idx % DK;
        float q = to_f<T>(src.qrow(i)[d]);
        qu[i][d] = q + src.u[d];
        qv[i][d] = q + src.vb[d];
    }
    if (tid < TQ) { mrow[tid] = -INFINITY; lrow[tid] = 0.0f; crow[tid] = 0.0f; }
    int kl = Tk, kh = 0;
    for (int i = 0; i < Tq; i++) {
        int s, e;
        src.range(i, s, e);
        if (s < e) { kl = min(kl, s); kh = max(kh, e); }
    }
    float acc[C::OUTS];
#pragma unroll
    for (int o = 0; o < C::OUTS; o++) acc[o] = 0.0f;
    __syncthreads();

    const int shift0 = Tk - Tq;
    for (int kb = kl; kb < kh; kb += KB) {
        const int nk = min(KB, kh - kb);
        const int nb = nk + Tq - 1;
        const int rbase = shift0 - (kb + nk - 1) + src.rel_offset;   // table row of band index 0

        uint4 kreg[C::KR], vreg[C::KR], preg[C::PR];
#pragma unroll
        for (int k = 0; k < C::KR; k++) {
            int row = grp + k * G;
            kreg[k] = make_uint4(0, 0, 0, 0);
            vreg[k] = make_uint4(0, 0, 0, 0);
            if (row < nk) {
                kreg[k] = ld16(src.krow(kb + row) + sub * VEC);
                vreg[k] = ld16(src.vrow(kb + row) + sub * VEC);
            }
        }
#pragma unroll
        for (int k = 0; k < C::PR; k++) {
            int b = grp + k * G;
            int r = rbase + b;
            preg[k] = make_uint4(0, 0, 0, 0);
            if (b < nb && r >= 0 && r < src.n_rel) preg[k] = ld16(src.prow(r) + sub * VEC);
        }
        __syncthreads();   // the previous block's P.V no longer reads vs / sc
#pragma unroll
        for (int k = 0; k < C::KR; k++) {
            int row = grp + k * G;
            if (row < nk) st16(&vs[row][sub * VEC], vreg[k]);
        }
        for (int i = 0; i < Tq; i++) {
            float a[VEC], bq[VEC];
#pragma unroll
            for (int e = 0; e < VEC; e++) { a[e] = qu[i][sub * VEC + e]; bq[e] = qv[i][sub * VEC + e]; }
#pragma unroll
            for (int k = 0; k < C::KR; k++) {
                float f[VEC];
                unpack16<T>(kreg[k], f);
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < VEC; e++) s += a[e] * f[e];
                s = group_sum<LPR>(s);
                int row = grp + k * G;
                if (sub == 0 && row < nk) sc[i][row] = s;
            }
#pragma unroll
            for (int k = 0; k < C::PR; k++) {
                float f[VEC];
                unpack16<T>(preg[k], f);
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < VEC; e++) s += bq[e] * f[e];
                s = group_sum<LPR>(s);
                int b = grp + k * G;
                if (sub == 0 && b < nb) bd[i][b] = s;
            }
        }
        __syncthreads();

        // Online softmax, one wave per query.
        for (int i = wave; i < Tq; i += NT / 64) {
            int qs, qe;
            src.range(i, qs, qe);
            const int lo = max(qs, kb) - kb, hi = min(qe, kb + nk) - kb;
            constexpr int PER = (KB + 63) / 64;
            float sv[PER];
            float bm = -INFINITY;
#pragma unroll
            for (int p = 0; p < PER; p++) {
                int jj = lane + p * 64;
                bool ok = jj < nk && jj >= lo && jj < hi;
                sv[p] = ok ? (sc[i][jj] + bd[i][i - jj + nk - 1]) * scale : -INFINITY;
                bm = fmaxf(bm, sv[p]);
            }
            bm = wave_max(bm);
            const float mold = mrow[i];
            const float mnew = fmaxf(mold, bm);
            float ls = 0.0f;
#pragma unroll
            for (int p = 0; p < PER; p++) {
                int jj = lane + p * 64;
                float e = (sv[p] == -INFINITY) ? 0.0f : __expf(sv[p] - mnew);
                if (jj < nk) sc[i][jj] = e;
                ls += e;
            }
            ls = wave_sum(ls);
            if (lane == 0) {
                float c = (mold == -INFINITY) ? 0.0f : __expf(mold - mnew);
                crow[i] = c;
                lrow[i] = lrow[i] * c + ls;
                mrow[i] = mnew;
            }
        }
        __syncthreads();

#pragma unroll
        for (int o = 0; o < C::OUTS; o++) {
            int idx = tid + o * NT;
            if (idx < Tq * DK) {
                int i = idx / DK, d = idx % DK;
                float a = acc[o] * crow[i];
                for (int jj = 0; jj < nk; jj++) a += sc[i][jj] * to_f<T>(vs[jj][d]);
                acc[o] = a;
            }
        }
    }
#pragma unroll
    for (int o = 0; o < C::OUTS; o++) {
        int idx = tid + o * NT;
        if (idx < Tq * DK) {
            int i = idx / DK, d = idx % DK;
            float l = (kl < kh) ? lrow[i] : 0.0f;
            src.store(i, d, l > 0.0f ? acc[o] / l : 0.0f);
        }
    }
}

template <typename T, int DK, int TQ, int KB>
__global__ __launch_bounds__(256) void relpos_op_kernel(const T* Q, const T* K, const T* V, const T* P,
                                                        const float* u, const float* vb, const int32_t* ranges,
                                                        T* O, int Tq, int Tk, int H, int rel_offset, int n_rel,
                                                        float scale) {
    const int h = blockIdx.x;
    OpSrc<T> src;
    src.Q = Q; src.K = K; src.V = V; src.P = P; src.O = O;
    src.u = u + h * DK; src.vb = vb + h * DK; src.ranges = ranges;
    src.Tq = Tq; src.Tk = Tk; src.ld = H * DK; src.hoff = h * DK;
    src.rel_offset = rel_offset; src.n_rel = n_rel;
    relpos_core<T, DK, TQ, KB>(src, scale);
}

// One workgroup per (stream, head): blockIdx.x = stream * H + head, so consecutive heads of a
// layer land on consecutive XCDs and each XCD's L2 serves one head's P rows to every stream.
template <typename T, int TQ, int KB>
__global__ __launch_bounds__(256) void relpos_ring_kernel(RingArgs a) {
    constexpr int DK = 128;
    const int s = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int32_t* d = a.desc + s * DESC_INTS;
    const int slot = d[0], start = d[1], valid = d[2], cache_len = d[3];
    const int D = a.H * DK;
    const T* kr = static_cast<const T*>(a.kring) + ((int64_t)slot * a.H + h) * a.R * DK;
    const T* vr = static_cast<const T*>(a.vring) + ((int64_t)slot * a.H + h) * a.R * DK;
    const T* qkv = static_cast<const T*>(a.qkv) + (int64_t)s * a.T * 3 * D;

    RingSrc<T> src;
    src.kr = kr; src.vr = vr; src.qkv = qkv;
    src.P = static_cast<const T*>(a.P);
    src.O = static_cast<T*>(a.att);
    src.row0 = (int64_t)s * a.T;
    src.frag = a.att_frag != 0;
    src.u = a.u + h * DK; src.vb = a.vb + h * DK;
    src.Tq = a.T; src.Tk = a.L + a.T; src.R = a.R; src.D = D; src.hoff = h * DK;
    src.start = start; src.rel_offset = a.rel_offset; src.n_rel = a.n_rel;
    src.ks = a.L - cache_len;
    src.ke = a.L + min(max(valid, 0), a.T);
    relpos_core<T, DK, TQ, KB>(src, a.scale);
}

// The T new K/V rows of every stream, qkv -> ring rows (start + L + i) mod R; one workgroup per
// (stream, head), 16 bytes per lane.
template <typename T>
__global__ __launch_bounds__(256) void ring_append_kernel(RingArgs a) {
    constexpr int DK = 128, VEC = Vec16<T>::N, LPR = DK / VEC;
    const int s = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int32_t* d = a.desc + s * DESC_INTS;
    const int slot = d[0], start = d[1];
    const int D = a.H * DK;
    const T* qkv = static_cast<const T*>(a.qkv) + (int64_t)s * a.T * 3 * D + h * DK;
    T* kw = static_cast<T*>(a.kring) + ((int64_t)slot * a.H + h) * a.R * DK;
    T* vw = static_cast<T*>(a.vring) + ((int64_t)slot * a.H + h) * a.R * DK;
    for (int idx = threadIdx.x; idx < a.T * LPR; idx += 256) {
        const int i = idx / LPR, c = (idx % LPR) * VEC;
        int row = start + a.L + i;               // < 2R
        row -= (row >= a.R) ? a.R : 0;
        const T* q = qkv + (int64_t)i * 3 * D + c;
        st16(kw + (int64_t)row * DK + c, ld16(q + D));
        st16(vw + (int64_t)row * DK + c, ld16(q + 2 * D));
    }
}

// ------------------------------------------------------------------ streaming ring kernels (T <= 4)
// The chunk shapes of streaming (2..4 queries over L + T <= 96 keys, IEEE half, head_dim 128) get
// kernels built for one memory round trip: relpos_ring_small_kernel (T 3..4) below and
// relpos_ring_wave_kernel (T <= 2) after it.  It works on the whole window [L cached ; T new] and on
// the whole positional band of the chunk (rel = 1-T .. L+T-1, the same rows for every stream), so
// the addresses of q, u/v and the band depend only on the launch, and those of K/V only on the
// stream's ring slot and window start (read first, from a 32-byte descriptor).  Every load is
// unconditional -- lanes past the window read a clamped row and are masked later -- so all of a
// workgroup's loads issue back to back with no wait in between, and bd is computed from the
// L2-resident band while K and V still arrive.  The key range [L - cache_len, L + valid) is a mask
// in the softmax; V rows outside it are zeroed in registers, so probability-0 keys contribute exact
// zeros whatever the pool holds there.
// Reductions: the TQ partial dot products of a 16-lane row group are reduced together with a
// transposed DPP butterfly; P.V is reduced over the 4 row groups of a wave with
// v_permlane32_swap / v_permlane16_swap (each lane keeps a quarter of the sums) and over the 4
// waves once through LDS.

// DPP row rotation (within 16 lanes) by R.
template <int R> __device__ __forceinline__ float dpp_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + R, 0xF, 0xF, false));
}

// Transposed reduction over a 16-lane row for Q in {1, 2, 4} values per lane.  Returns, in every
// lane, the row total of value index qidx(lane) where qidx = bit-reverse of the low log2(Q) lane
// bits.
template <int Q>
__device__ __forceinline__ float tsum16(float (&v)[Q], int lane) {
    if constexpr (Q == 4) {
        const bool b0 = lane & 1;
        float k0 = b0 ? v[2] : v[0], s0 = b0 ? v[0] : v[2];
        float k1 = b0 ? v[3] : v[1], s1 = b0 ? v[1] : v[3];
        k0 += dpp_mov<DPP_QUAD_1032>(s0);
        k1 += dpp_mov<DPP_QUAD_1032>(s1);
        const bool b1 = lane & 2;
        float k = b1 ? k1 : k0, sd = b1 ? k0 : k1;
        k += dpp_mov<DPP_QUAD_2301>(sd);
        k += dpp_ror<4>(k);
        k += dpp_ror<8>(k);
        return k;
    } else if constexpr (Q == 2) {
        const bool b0 = lane & 1;
        float k = b0 ? v[1] : v[0], sd = b0 ? v[0] : v[1];
        k += dpp_mov<DPP_QUAD_1032>(sd);
        k += dpp_ror<2>(k);
        k += dpp_ror<4>(k);
        k += dpp_ror<8>(k);
        return k;
    } else {
        return group_sum<16>(v[0]);
    }
}
template <int Q> __device__ __forceinline__ int tsum16_index(int lane) {
    if constexpr (Q == 4) return ((lane & 1) << 1) | ((lane >> 1) & 1);
    else if constexpr (Q == 2) return lane & 1;
    else return 0;
}

// Window rows of the streaming kernel for one 16-lane group: key j = grp + G k (clamped to W - 1;
// G = the workgroup's number of groups) is ring row (start + j) mod R of the stream's slot.
// prepare() needs only the launch and runs while the stream's descriptor is in flight; load() then
// costs two VALU operations per pass.  Offsets are 32-bit byte offsets from the (slot, head) block,
// the same for the whole workgroup, so the loads take a scalar base plus a vector offset.
template <int KR, int G = 16>
struct WindowRows {
    int j[KR];

    __device__ __forceinline__ void prepare(int grp, int W) {
#pragma unroll
        for (int k = 0; k < KR; k++) j[k] = min(grp + k * G, W - 1);
    }
    __device__ __forceinline__ void load(uint4 (&kreg)[KR], uint4 (&vreg)[KR], const f16* kbase, const f16* vbase,
                                         int start, int R, int sub) const {
        const char* kb = reinterpret_cast<const char*>(kbase);
        const char* vb = reinterpret_cast<const char*>(vbase);
        // ring byte offsets (rows start + j < 2R: one conditional subtraction)
        uint32_t roff[KR];
#pragma unroll
        for (int k = 0; k < KR; k++) {
            const uint32_t r = (uint32_t)(start + j[k]);
            roff[k] = (min(r, r - (uint32_t)R) << 8) | ((uint32_t)sub << 4);
        }
        // ring rows are read once per step: non-temporal loads
#pragma unroll
        for (int k = 0; k < KR; k++) kreg[k] = ld16_nt(kb + roff[k]);
        // every K load before the first V load: loads complete in issue order, so the scores can
        // start while V is still arriving
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < KR; k++) vreg[k] = ld16_nt(vb + roff[k]);
    }
};


// One workgroup (4 waves) per (stream, head).  16 lanes own one 128-wide half row (8 values per
// lane), 16 row groups per pass: KR passes cover the window's L + T keys, PR passes the band's
// L + 2T - 1 rows.  TQ in {2, 4} queries (T < TQ runs with clamped duplicate queries).
template <int TQ, int KR, int PR>
__global__ __launch_bounds__(256) void relpos_ring_small_kernel(RingArgs a) {
    using T = f16;
    constexpr int DK = 128, VEC = 8, LPR = 16, G = 16;
    constexpr int KMAX = KR * G, BMAX = PR * G, NV = TQ * VEC, NQ = NV / 4;
    static_assert(NQ % 4 == 0, "float4 partial sums");
    __shared__ float sc[TQ][KMAX];
    __shared__ float bd[TQ][BMAX];
    __shared__ __align__(16) float red[4][TQ * DK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid / LPR, sub = tid % LPR, row4 = lane >> 4;
    const int s = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int L = a.L, Tq = a.T, D = a.H * DK, W = L + Tq, NB = L + 2 * Tq - 1;
    // the stream's descriptor first: one scalar load, in flight while the launch-only loads issue
    const int4 dsc = *reinterpret_cast<const int4*>(a.desc + s * DESC_INTS);
    __builtin_amdgcn_sched_barrier(0);
    const T* qkvh = static_cast<const T*>(a.qkv) + (int64_t)s * Tq * 3 * D + h * DK;   // the workgroup's
    const T* qkv = qkvh + sub * VEC;
    const T* P = static_cast<const T*>(a.P) + (int64_t)(a.rel_offset + 1 - Tq) * D + h * DK + sub * VEC;

    // ---- launch-only addresses: q, u/v, the band
    uint4 qreg[TQ];
#pragma unroll
    for (int i = 0; i < TQ; i++) qreg[i] = ld16(qkv + (int64_t)min(i, Tq - 1) * 3 * D);
    const float4 u0 = *reinterpret_cast<const float4*>(a.u + h * DK + sub * VEC);
    const float4 u1 = *reinterpret_cast<const float4*>(a.u + h * DK + sub * VEC + 4);
    const float4 v0 = *reinterpret_cast<const float4*>(a.vb + h * DK + sub * VEC);
    const float4 v1 = *reinterpret_cast<const float4*>(a.vb + h * DK + sub * VEC + 4);
    uint4 preg[PR];
#pragma unroll
    for (int k = 0; k < PR; k++) preg[k] = ld16(P + (int64_t)min(grp + k * G, NB - 1) * D);

    // ---- K and V of the window (WindowRows): the launch-only part now, the rest once the
    //      descriptor is here
    WindowRows<KR> win;
    win.prepare(grp, W);
    __builtin_amdgcn_sched_barrier(0);
    const int slot = dsc.x, start = dsc.y, valid = min(max(dsc.z, 0), Tq), cache_len = dsc.w;
    const int ks = L - cache_len, ke = L + valid;
    const T* kbase = static_cast<const T*>(a.kring) + ((int64_t)slot * a.H + h) * a.R * DK;
    const T* vbase = static_cast<const T*>(a.vring) + ((int64_t)slot * a.H + h) * a.R * DK;
    uint4 kreg[KR], vreg[KR];
    win.load(kreg, vreg, kbase, vbase, start, a.R, sub);

    // ---- q + u, q + v, rounded once to IEEE-half pairs: the score products are v_dot2_f32_f16
    //      (two products per instruction, fp32 sum) on the half words of K and the band as loaded
    const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    half2_t qu2[TQ][VEC / 2], qv2[TQ][VEC / 2];
#pragma unroll
    for (int i = 0; i < TQ; i++) {
        float f[VEC];
        unpack16<T>(qreg[i], f);
#pragma unroll
        for (int e = 0; e < VEC / 2; e++) {
            qu2[i][e] = half2_t{f2h_sat(f[2 * e] + uu[2 * e]), f2h_sat(f[2 * e + 1] + uu[2 * e + 1])};
            qv2[i][e] = half2_t{f2h_sat(f[2 * e] + vv[2 * e]), f2h_sat(f[2 * e + 1] + vv[2 * e + 1])};
        }
    }
    const int qi = tsum16_index<TQ>(sub);

    // ---- bd[i][b] = (q_i + v) . band row b
#pragma unroll
    for (int k = 0; k < PR; k++) {
        const uint32_t w[4] = {preg[k].x, preg[k].y, preg[k].z, preg[k].w};
        float part[TQ];
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC / 2; e++) acc = __builtin_amdgcn_fdot2(qv2[i][e], as_half2(w[e]), acc, false);
            part[i] = acc;
        }
        const float tot = tsum16<TQ>(part, sub);
        if (sub < TQ) bd[qi][grp + k * G] = tot;
    }
    // ---- ac[i][j] = (q_i + u) . K_j
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const uint32_t w[4] = {kreg[k].x, kreg[k].y, kreg[k].z, kreg[k].w};
        float part[TQ];
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC / 2; e++) acc = __builtin_amdgcn_fdot2(qu2[i][e], as_half2(w[e]), acc, false);
            part[i] = acc;
        }
        const float tot = tsum16<TQ>(part, sub);
        if (sub < TQ) sc[qi][grp + k * G] = tot;
    }
    __syncthreads();

    // ---- softmax over keys [ks, ke), one wave per query; rel_shift is the band index
    //      W - 1 + i - j (table row (L + i - j) + rel_offset).  Probabilities overwrite sc.
    for (int i = wave; i < Tq; i += 4) {
        constexpr int PER = (KMAX + 63) / 64;
        float sv[PER];
        float m = -INFINITY;
#pragma unroll
        for (int p = 0; p < PER; p++) {
            const int j = lane + p * 64, jc = min(j, W - 1);
            const float x = (sc[i][jc] + bd[i][W - 1 + i - jc]) * a.scale;
            sv[p] = (j >= ks && j < ke) ? x : -INFINITY;
            m = fmaxf(m, sv[p]);
        }
        m = wave_max(m);
        float l = 0.0f;
#pragma unroll
        for (int p = 0; p < PER; p++) {
            sv[p] = sv[p] == -INFINITY ? 0.0f : __expf(sv[p] - m);
            l += sv[p];
        }
        l = wave_sum(l);
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int p = 0; p < PER; p++) {
            const int j = lane + p * 64;
            if (j < KMAX) sc[i][j] = sv[p] * inv;
        }
    }
    __syncthreads();

    // ---- out = P . V from the V registers (rows outside the range zeroed): v_fma_mix_f32 takes the
    //      half V words as they are (fp32 probability, fp32 sum)
    float acc[NV];
#pragma unroll
    for (int f = 0; f < NV; f++) acc[f] = 0.0f;
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int j = grp + k * G;
        const bool in = j >= ks && j < ke;
        const uint4 z = make_uint4(0, 0, 0, 0);
        const uint4 vk = in ? vreg[k] : z;
        const uint32_t w[4] = {vk.x, vk.y, vk.z, vk.w};
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            const float p = sc[i][j];
#pragma unroll
            for (int e = 0; e < VEC / 2; e++) {
                acc[i * VEC + 2 * e] = fmaf(p, half_lo(w[e]), acc[i * VEC + 2 * e]);
                acc[i * VEC + 2 * e + 1] = fmaf(p, half_hi(w[e]), acc[i * VEC + 2 * e + 1]);
            }
        }
    }
    // over the 4 row groups of the wave: lane (row4, sub) ends with flat sums row4*NQ .. +NQ-1
    float h1[NV / 2], h2[NQ];
#pragma unroll
    for (int m = 0; m < NV / 2; m++) h1[m] = xsum32(acc[m], acc[m + NV / 2]);
#pragma unroll
    for (int m = 0; m < NQ; m++) h2[m] = xsum16(h1[m], h1[m + NQ]);
#pragma unroll
    for (int m = 0; m < NQ; m += 4) {
        const int f = row4 * NQ + m, i = f >> 3, e = f & 7;
        *reinterpret_cast<float4*>(&red[wave][i * DK + sub * VEC + e]) = make_float4(h2[m], h2[m + 1], h2[m + 2], h2[m + 3]);
    }
    __syncthreads();

    // ---- output rows (0 for an empty key range), 8 channels per thread
    if (tid < Tq * LPR) {
        const int i = tid / LPR;
        float o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float4 x = *reinterpret_cast<const float4*>(&red[w][i * DK + sub * VEC + e]);
                t.x += x.x; t.y += x.y; t.z += x.z; t.w += x.w;
            }
            o[e] = t.x; o[e + 1] = t.y; o[e + 2] = t.z; o[e + 3] = t.w;
        }
        const bool empty = ke <= ks;
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            pk[e] = empty ? 0u : ((uint32_t)f2h(o[2 * e]) | ((uint32_t)f2h(o[2 * e + 1]) << 16));
        const int64_t row = (int64_t)s * Tq + i;
        T* att = static_cast<T*>(a.att);
        T* dst = a.att_frag ? att + frag_index(row, h * DK + sub * VEC, D / 64) : att + row * D + h * DK + sub * VEC;
        st16(dst, make_uint4(pk[0], pk[1], pk[2], pk[3]));
    }
}

// Streaming kernel, one-barrier form (T <= 4).  One workgroup (4 waves) per (stream, head); a
// 16-lane row group owns key j = grp + 16 p (p < KR), 8 channels per lane.  Each group loads, for
// its keys, the K and V rows and the TQ band rows the keys need (band row W - 1 + i - j for query
// i: rel_shift as the row index), so each score s_ij = ((q_i + u) . k_j + (q_i + v) . P_row) *
// scale is complete inside the group (v_dot2_f32_f16 partials, 16-lane DPP sums) with no table
// shared across waves.  Softmax is online per wave: the wave's running max and sum over its 4
// groups (lane-swap reductions), P.V on its own V rows (v_fma_mix_f32), and the 4 waves' partial
// outputs merge once through LDS with the usual max/sum rescaling.  Keys outside [ks, ke) score
// -inf and their V rows are zeroed by a mask, so they contribute exact zeros.
template <int TQ, int KR>
__global__ __launch_bounds__(256) void relpos_ring_wave_kernel(RingArgs a) {
    using T = f16;
    constexpr int DK = 128, VEC = 8, G = 16, NV = TQ * VEC, NQ = NV / 4;
    static_assert(NQ % 4 == 0, "float4 partial sums");
    __shared__ __align__(16) float red[4][TQ * DK];
    __shared__ float stat[4][TQ][2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid >> 4, sub = tid & 15, row4 = lane >> 4;
    const int s = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int L = a.L, Tq = a.T, D = a.H * DK, W = L + Tq, NB = L + 2 * Tq - 1;
    const int4 dsc = *reinterpret_cast<const int4*>(a.desc + s * DESC_INTS);
    __builtin_amdgcn_sched_barrier(0);
    const T* qkv = static_cast<const T*>(a.qkv) + (int64_t)s * Tq * 3 * D + h * DK + sub * VEC;
    // band row b (0 .. NB-1) is table row rel_offset + 1 - T + b
    const char* Pb = reinterpret_cast<const char*>(static_cast<const T*>(a.P) + (int64_t)(a.rel_offset + 1 - Tq) * D +
                                                   h * DK + sub * VEC);

    // ---- launch-only loads: q, u/v, the band rows of this group's keys
    uint4 qreg[TQ];
#pragma unroll
    for (int i = 0; i < TQ; i++) qreg[i] = ld16(qkv + (int64_t)min(i, Tq - 1) * 3 * D);
    const float4 u0 = *reinterpret_cast<const float4*>(a.u + h * DK + sub * VEC);
    const float4 u1 = *reinterpret_cast<const float4*>(a.u + h * DK + sub * VEC + 4);
    const float4 v0 = *reinterpret_cast<const float4*>(a.vb + h * DK + sub * VEC);
    const float4 v1 = *reinterpret_cast<const float4*>(a.vb + h * DK + sub * VEC + 4);
    uint4 preg[KR][TQ];
#pragma unroll
    for (int p = 0; p < KR; p++) {
        const int j = min(grp + G * p, W - 1);
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            const int b = min(W - 1 + i - j, NB - 1);       // >= 0: j <= W - 1; clamped for i >= T
            preg[p][i] = ld16(Pb + (int64_t)b * D * 2);
        }
    }
    // ---- K and V rows of the window (ring rows start + j mod R), K first
    WindowRows<KR> win;
    win.prepare(grp, W);
    __builtin_amdgcn_sched_barrier(0);
    const int slot = dsc.x, start = dsc.y, valid = min(max(dsc.z, 0), Tq), cache_len = dsc.w;
    const int ks = L - cache_len, ke = L + valid;
    const T* kbase = static_cast<const T*>(a.kring) + ((int64_t)slot * a.H + h) * a.R * DK;
    const T* vbase = static_cast<const T*>(a.vring) + ((int64_t)slot * a.H + h) * a.R * DK;
    uint4 kreg[KR], vreg[KR];
    win.load(kreg, vreg, kbase, vbase, start, a.R, sub);

    // ---- q + u, q + v rounded once to IEEE-half pairs
    const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    half2_t qu2[TQ][VEC / 2], qv2[TQ][VEC / 2];
#pragma unroll
    for (int i = 0; i < TQ; i++) {
        float f[VEC];
        unpack16<T>(qreg[i], f);
#pragma unroll
        for (int e = 0; e < VEC / 2; e++) {
            qu2[i][e] = half2_t{f2h_sat(f[2 * e] + uu[2 * e]), f2h_sat(f[2 * e + 1] + uu[2 * e + 1])};
            qv2[i][e] = half2_t{f2h_sat(f[2 * e] + vv[2 * e]), f2h_sat(f[2 * e + 1] + vv[2 * e + 1])};
        }
    }
    // ---- bd parts (band rows: L2-resident, in before K), then scores; every lane of a group gets
    //      the group's totals
    float sc[KR][TQ];
#pragma unroll
    for (int p = 0; p < KR; p++)
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            const uint32_t w[4] = {preg[p][i].x, preg[p][i].y, preg[p][i].z, preg[p][i].w};
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC / 2; e++) acc = __builtin_amdgcn_fdot2(qv2[i][e], as_half2(w[e]), acc, false);
            sc[p][i] = acc;
        }
    float m[TQ];
#pragma unroll
    for (int i = 0; i < TQ; i++) m[i] = -INFINITY;
#pragma unroll
    for (int p = 0; p < KR; p++) {
        const uint32_t w[4] = {kreg[p].x, kreg[p].y, kreg[p].z, kreg[p].w};
        const int j = grp + G * p;
        const bool in = j >= ks && j < ke;
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            float acc = sc[p][i];
#pragma unroll
            for (int e = 0; e < VEC / 2; e++) acc = __builtin_amdgcn_fdot2(qu2[i][e], as_half2(w[e]), acc, false);
            const float x = group_sum<16>(acc) * a.scale;
            sc[p][i] = (in && i < Tq) ? x : -INFINITY;
            m[i] = fmaxf(m[i], sc[p][i]);
        }
    }
    // ---- wave softmax statistics over the wave's 4 groups (lanes l ^ 16, l ^ 32)
    float l[TQ];
#pragma unroll
    for (int i = 0; i < TQ; i++) {
        m[i] = xmax32(xmax16(m[i]));
        l[i] = 0.0f;
#pragma unroll
        for (int p = 0; p < KR; p++) {
            sc[p][i] = sc[p][i] == -INFINITY ? 0.0f : __expf(sc[p][i] - m[i]);
            l[i] += sc[p][i];
        }
    }
    // ---- P.V on this group's V rows (masked rows zeroed): v_fma_mix_f32 on the half words
    float acc[NV];
#pragma unroll
    for (int f = 0; f < NV; f++) acc[f] = 0.0f;
#pragma unroll
    for (int p = 0; p < KR; p++) {
        const int j = grp + G * p;
        const uint32_t keep = (j >= ks && j < ke) ? 0xFFFFFFFFu : 0u;
        const uint32_t w[4] = {vreg[p].x & keep, vreg[p].y & keep, vreg[p].z & keep, vreg[p].w & keep};
#pragma unroll
        for (int i = 0; i < TQ; i++) {
            const float pr = sc[p][i];
#pragma unroll
            for (int e = 0; e < VEC / 2; e++) {
                acc[i * VEC + 2 * e] = fmaf(pr, half_lo(w[e]), acc[i * VEC + 2 * e]);
                acc[i * VEC + 2 * e + 1] = fmaf(pr, half_hi(w[e]), acc[i * VEC + 2 * e + 1]);
            }
        }
    }
    // over the 4 row groups of the wave: lane (row4, sub) ends with flat sums row4*NQ .. +NQ-1
    float h1[NV / 2], h2[NQ];
#pragma unroll
    for (int k = 0; k < NV / 2; k++) h1[k] = xsum32(acc[k], acc[k + NV / 2]);
#pragma unroll
    for (int k = 0; k < NQ; k++) h2[k] = xsum16(h1[k], h1[k + NQ]);
#pragma unroll
    for (int k = 0; k < NQ; k += 4) {
        const int f = row4 * NQ + k, i = f >> 3, e = f & 7;
        *reinterpret_cast<float4*>(&red[wave][i * DK + sub * VEC + e]) = make_float4(h2[k], h2[k + 1], h2[k + 2], h2[k + 3]);
    }
#pragma unroll
    for (int i = 0; i < TQ; i++) l[i] = xadd32(xadd16(l[i]));     // every lane: the wave's sums
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < TQ; i++) { stat[wave][i][0] = m[i]; stat[wave][i][1] = l[i]; }
    }
    __syncthreads();

    // ---- merge the waves: out_i = sum_w e^(m_w - M) acc_w / sum_w e^(m_w - M) l_w (0 for an empty
    //      range: every weight is 0); 8 channels per thread, 16-byte stores
    if (tid < Tq * 16) {
        const int i = tid >> 4;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, stat[w][i][0]);
        float wt[4], Ls = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            wt[w] = stat[w][i][0] == -INFINITY ? 0.0f : __expf(stat[w][i][0] - M);
            Ls += wt[w] * stat[w][i][1];
        }
        const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
        float o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float4 x = *reinterpret_cast<const float4*>(&red[w][i * DK + sub * VEC + e]);
                t.x += wt[w] * x.x; t.y += wt[w] * x.y; t.z += wt[w] * x.z; t.w += wt[w] * x.w;
            }
            o[e] = t.x * inv; o[e + 1] = t.y * inv; o[e + 2] = t.z * inv; o[e + 3] = t.w * inv;
        }
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; e++) pk[e] = (uint32_t)f2h(o[2 * e]) | ((uint32_t)f2h(o[2 * e + 1]) << 16);
        const int64_t row = (int64_t)s * Tq + i;
        T* att = static_cast<T*>(a.att);
        T* dst = a.att_frag ? att + frag_index(row, h * DK + sub * VEC, D / 64) : att + row * D + h * DK + sub * VEC;
        st16(dst, make_uint4(pk[0], pk[1], pk[2], pk[3]));
    }
}

// Read floor of the streaming kernel's access pattern (relpos_ring_wave_kernel, T <= 2): the same
// grid, the same loads (q, u/v, each key's band rows, K and V of the window, through the same
// addressing), no arithmetic beyond folding the words together, no stores (one store to att[0] on
// a value that never occurs keeps the loads live).  Its time per launch is what memory alone costs
// for this shape; the attention kernel is measured against it.
template <int KR>
__global__ __launch_bounds__(256) void ring_read_floor_kernel(RingArgs a) {
    using T = f16;
    constexpr int TQ = 2, DK = 128, VEC = 8, LPR = 16, G = 16;
    const int tid = threadIdx.x, grp = tid / LPR, sub = tid % LPR;
    const int s = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int L = a.L, Tq = a.T, D = a.H * DK, W = L + Tq, NB = L + 2 * Tq - 1;
    const int4 dsc = *reinterpret_cast<const int4*>(a.desc + s * DESC_INTS);
    __builtin_amdgcn_sched_barrier(0);
    const T* qkvh = static_cast<const T*>(a.qkv) + (int64_t)s * Tq * 3 * D + h * DK;
    const T* qkv = qkvh + sub * VEC;
    const T* P = static_cast<const T*>(a.P) + (int64_t)(a.rel_offset + 1 - Tq) * D + h * DK + sub * VEC;
    uint4 acc = make_uint4(0, 0, 0, 0);
    auto fold = [&](uint4 x) { acc.x ^= x.x; acc.y ^= x.y; acc.z ^= x.z; acc.w ^= x.w; };
    uint4 r[TQ + 4 + KR * TQ + 2 * KR];
    int n = 0;
#pragma unroll
    for (int i = 0; i < TQ; i++) r[n++] = ld16(qkv + (int64_t)min(i, Tq - 1) * 3 * D);
    r[n++] = *reinterpret_cast<const uint4*>(a.u + h * DK + sub * VEC);
    r[n++] = *reinterpret_cast<const uint4*>(a.u + h * DK + sub * VEC + 4);
    r[n++] = *reinterpret_cast<const uint4*>(a.vb + h * DK + sub * VEC);
    r[n++] = *reinterpret_cast<const uint4*>(a.vb + h * DK + sub * VEC + 4);
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int j = min(grp + k * G, W - 1);
#pragma unroll
        for (int i = 0; i < TQ; i++) r[n++] = ld16(P + (int64_t)min(W - 1 + i - j, NB - 1) * D);
    }
    WindowRows<KR> win;
    win.prepare(grp, W);
    __builtin_amdgcn_sched_barrier(0);
    const int slot = dsc.x, start = dsc.y;
    const T* kbase = static_cast<const T*>(a.kring) + ((int64_t)slot * a.H + h) * a.R * DK;
    const T* vbase = static_cast<const T*>(a.vring) + ((int64_t)slot * a.H + h) * a.R * DK;
    uint4 kreg[KR], vreg[KR];
    win.load(kreg, vreg, kbase, vbase, start, a.R, sub);
#pragma unroll
    for (int k = 0; k < KR; k++) r[n++] = kreg[k];
#pragma unroll
    for (int k = 0; k < KR; k++) r[n++] = vreg[k];
#pragma unroll
    for (int i = 0; i < TQ + 4 + KR * TQ + 2 * KR; i++) fold(r[i]);
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u && tid == 0) static_cast<T*>(a.att)[0] = (T)1;
}

int launch_ring_read_floor(const RingArgs& a, hipStream_t st) {
    const bool band_ok = a.rel_offset + 1 - a.T >= 0 && a.rel_offset + a.L + a.T - 1 < a.n_rel;
    const int kr = (a.L + a.T + 15) / 16;
    if (a.T > 2 || a.L < 16 || kr > 5 || !band_ok || a.n < 1 || a.L + a.T > a.R) return -2;
    hipLaunchKernelGGL((ring_read_floor_kernel<5>), dim3(a.n * a.H), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------------ streaming ring kernel on MFMA (T 5..16)
// Longer chunks (config of 14 frames: 256 streams x 8 heads, 103 MB per launch) make the
// per-(stream, head) work a real matrix product: 16 query rows (T of them real) against the
// stream's R <= 96 ring rows and L + 2T - 1 <= 112 band rows, all on v_mfma_f32_16x16x32_f16,
// every product transposed so that a lane ends up holding one query's values:
//   C[band row][query] = P_band . (q+v)^T    (A = band rows from LDS, B = q+v)
//   C[ring row][query] = K . (q+u)^T         (A = K rows loaded straight into registers, B = q+u)
//   C[chan][query]     = V^T . P^T           (A = V^T via transposed LDS reads, B = probabilities)
// Keys are taken in ring order: K tile t holds ring rows 16t .. 16t+15 and V load it ring rows
// 4it .. 4it+3 of the (slot, head) block, so every address is the block's (scalar) base plus a
// lane constant plus an immediate -- no modulo, no wrap.  Ring row r holds window key
// j = (r - start) mod R; the score of (i, r) uses band row W - 1 + i - j (rel_shift as an index,
// gathered from the band tile in LDS), and keys outside [ks, ke) (rows outside the window
// included) score -inf.  Softmax sums and P.V do not depend on the order of the keys.
// Lane (c, g) (c = lane % 16, g = lane / 16) holds the scores of query c at ring rows
// 16t + 4g + r: the softmax statistics reduce over the 4 lanes c, c+16, c+32, c+48 (lane swaps),
// and the probabilities stay in registers as the B operand of P.V, whose k order is the same
// permutation of the 32 rows of a piece: position 8g + e holds row 4g + e (e < 4), then
// 16 + 4g + e - 4.  V is staged into LDS in that order.
// One wave64 per (stream, head); a workgroup is 8 waves = 8 streams of one head, so the head's
// band is loaded once per workgroup into LDS (it is the same for every stream), and every wave
// is resident at once at two waves per SIMD (2,048 waves on 1,024 SIMDs).  Loads are spread over
// the unit so that the wave computes between them instead of stalling on issue: q and K first,
// the first half of V after the band product, the second half after the key product.  When every
// ring row is a valid key (ks = 0, ke = R: the steady state of full chunks) V needs no mask;
// otherwise V rows outside the key range are zeroed before P.V, so probability-0 keys contribute
// exact zeros whatever the ring holds there.
// q+u, q+v and the probabilities enter the MFMA rounded once to IEEE half (relative 2^-12).
typedef short v4i16_t __attribute__((ext_vector_type(4)));

namespace rm {
constexpr int BT = 7;                            // band tiles of 16 rows
constexpr int BMAX = 16 * BT;
constexpr int KMAX = 96;                         // ring rows (6 key tiles)
constexpr int NW = 8;                            // waves (streams of one head) per workgroup
constexpr int RS = 17;                           // 16-byte slots per band row in LDS (16 + 1 pad)
constexpr int BSLOTS = BMAX * RS;                // 16-byte slots of the band rows
constexpr int BINS = (BSLOTS + 64 + 63) / 64;     // direct-load instructions: band rows, u and v
constexpr int SLD = BMAX + 4;                    // floats per row of a wave's bd tile
constexpr int VST = 136;                         // halves per staged V row (128 + 8 pad)
}  // namespace rm

// ds_write / ds_read of one wave that exchange data across its lanes: wait for the wave's own LDS
// operations (no other wave touches the region).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
    __asm__ volatile("" ::: "memory");
}

// fp32 x 8 -> 8 IEEE halves packed for an MFMA operand.
__device__ __forceinline__ uint4 pack_f16x8(const float (&x)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) w[e] = (uint32_t)f2h(x[2 * e]) | ((uint32_t)f2h(x[2 * e + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}
// The same for softmax probabilities (in [0, 1], so no saturation is needed).
__device__ __forceinline__ uint4 pack_f16x8_unit(const float (&x)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        w[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[2 * e]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[2 * e + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// KT key tiles cover ring rows 0 .. 16 KT - 1 (R <= 16 KT); NVL V loads cover rows 0 .. 4 NVL - 1.
// NVL < 4 KT only when NVL == ceil(R / 4) (the launcher checks it), so that only the last V load
// can reach past row R - 1.
template <int KT, int NVL>
__global__ __launch_bounds__(64 * rm::NW, 1) void relpos_ring_mfma_kernel(RingArgs a) {
    using namespace rm;
    using T = f16;
    constexpr int KP = (16 * KT + 31) / 32;       // 32-row V pieces
    constexpr int NV1 = NVL / 2;                  // V loads issued after the band product
    static_assert(KT >= 1 && KT <= 6 && NVL <= 4 * KT && 4 * NVL > 16 * (KT - 1), "ring rows");
    __shared__ __align__(16) uint4 band[BINS * 64];            // band rows (17 slots each), then u, v
    __shared__ __align__(16) float slw[NW][16][SLD];           // per wave: bd tile [query][band row]
    __shared__ __align__(16) uint16_t vpw[NW][32][VST];        // per wave: a 32-row piece of V

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, g = lane >> 4;
    const int H = a.H, L = a.L, Tq = a.T, D = H * 128, W = L + Tq, NB = L + 2 * Tq - 1, R = a.R;
    const int h = blockIdx.x % H;
    const int s = (blockIdx.x / H) * NW + wave;
    const bool live = s < a.n;                                  // wave-uniform
    float (*sl)[SLD] = slw[wave];
    uint16_t (*vp)[VST] = vpw[wave];
    // the descriptor first: read before any store of the kernel, it stays a scalar load.  A wave
    // past the last stream works on stream 0 and stores nothing (no branch around the body).
    const int sx = live ? s : 0;
    const int32_t* d = a.desc + sx * DESC_INTS;
    const int slot = d[0], start = d[1], valid = min(max(d[2], 0), Tq), cache_len = d[3];

    // ---- the head's band -> LDS (rows rel_offset + 1 - T + b, b < NB, of P; rel = 1-T .. L+T-1),
    //      then its u and v biases (32 slots each)
    {
        const char* P = static_cast<const char*>(a.P) + ((int64_t)(a.rel_offset + 1 - Tq) * D + h * 128) * 2;
        const char* zero = static_cast<const char*>(a.zero_row);
#pragma unroll
        for (int m = 0; m < (BINS + NW - 1) / NW; m++) {
            const int ins = wave + NW * m;
            if (ins < BINS) {
                const int slot = 64 * ins + lane, r = slot / RS, c = slot % RS, k = slot - BSLOTS;
                const char* src = (c < 16 && r < NB) ? P + (int64_t)r * D * 2 + c * 16 : zero;
                if (k >= 0) src = k < 64 ? reinterpret_cast<const char*>((k < 32 ? a.u : a.vb) + h * 128 + 4 * (k & 31)) : zero;
                __builtin_amdgcn_global_load_lds(src, &band[64 * ins], 16, 0, 0);
            }
        }
    }
    __asm__ volatile("" ::: "memory");          // the band loads stay ahead of the unit's loads
    // ---- this wave's unit: q and the K tiles (B layout)
    const int ks = L - cache_len, ke = L + valid;
    const T* qkv = static_cast<const T*>(a.qkv) + (int64_t)sx * Tq * 3 * D + h * 128;
    const char* kblk = static_cast<const char*>(a.kring) + ((int64_t)slot * H + h) * R * 256;
    const char* vblk = static_cast<const char*>(a.vring) + ((int64_t)slot * H + h) * R * 256;
    uint4 qraw[4];
#pragma unroll
    for (int st = 0; st < 4; st++) qraw[st] = ld16(qkv + (int64_t)min(col, Tq - 1) * 3 * D + (4 * st + g) * 8);
    uint4 kb[KT][4];
#pragma unroll
    for (int t = 0; t < KT; t++) {
        const uint32_t off = (uint32_t)min(16 * t + col, R - 1) * 256u + (uint32_t)g * 16u;
#pragma unroll
        for (int st = 0; st < 4; st++) kb[t][st] = ld16(kblk + off + 64 * st);
    }
    // V row 4 it + g, 16-byte column col (only the last load can pass row R - 1 when NVL < 4 KT)
    uint4 vr[NVL];
    const uint32_t voff = (uint32_t)g * 256u + (uint32_t)col * 16u;
    auto vload = [&](int it) {
        const bool clamp = NVL == 4 * KT || it == NVL - 1;
        const uint32_t off = clamp ? (uint32_t)min(4 * it + g, R - 1) * 256u + (uint32_t)col * 16u : voff + 1024u * it;
        vr[it] = ld16(vblk + off);
    };
    // Wait for the band (and q): the 4 + 4 KT loads of the unit were issued after the band loads
    // and complete in order, so at most 4 KT outstanding means the band and q are in.  A bare
    // s_barrier, not __syncthreads(): the latter's workgroup fence waits for every outstanding load
    // (vmcnt(0)); the band's direct loads are covered by the wait above.
    static_assert(4 * KT < 64, "vmcnt range");
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * KT));
    __builtin_amdgcn_s_barrier();                // every wave's band loads
    __asm__ volatile("" ::: "memory");
    const float (*uvl)[128] = reinterpret_cast<const float (*)[128]>(&band[BSLOTS]);

    // ---- B operands: q + u, q + v (query col, k-chunk 4 st + g), rounded once to half
    uint4 bqu[4], bqv[4];
#pragma unroll
    for (int st = 0; st < 4; st++) {
        const int c = (4 * st + g) * 8;
        const float4 u0 = *reinterpret_cast<const float4*>(&uvl[0][c]), u1 = *reinterpret_cast<const float4*>(&uvl[0][c + 4]);
        const float4 v0 = *reinterpret_cast<const float4*>(&uvl[1][c]), v1 = *reinterpret_cast<const float4*>(&uvl[1][c + 4]);
        const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
        const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float q[8], x[8], y[8];
        unpack16<T>(qraw[st], q);
#pragma unroll
        for (int e = 0; e < 8; e++) { x[e] = q[e] + uu[e]; y[e] = q[e] + vv[e]; }
        bqu[st] = pack_f16x8(x);
        bqv[st] = pack_f16x8(y);
    }

    // ---- bd tiles -> sl[query][band row] (16-byte writes: lane holds band rows 16t + 4g .. +3 of
    //      query col); the next tile's band fragments are read ahead of the current tile's MFMAs
    {
        uint4 fa[4], fb[4];
#pragma unroll
        for (int st = 0; st < 4; st++) fa[st] = band[col * RS + 4 * st + g];
#pragma unroll
        for (int t = 0; t < BT; t++) {
            if (t + 1 < BT) {
#pragma unroll
                for (int st = 0; st < 4; st++) fb[st] = band[(16 * (t + 1) + col) * RS + 4 * st + g];
            }
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 4; st++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(fa[st]), as_f16x8(bqv[st]), acc, 0, 0, 0);
            *reinterpret_cast<float4*>(&sl[col][16 * t + 4 * g]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
#pragma unroll
            for (int st = 0; st < 4; st++) fa[st] = fb[st];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < NV1; it++) vload(it);
    __builtin_amdgcn_sched_barrier(0);
    // ---- ac tiles: lane holds query col at ring rows 16t + 4g + r
    f32x4_t sacc[KT];
#pragma unroll
    for (int t = 0; t < KT; t++) {
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 4; st++)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(kb[t][st]), as_f16x8(bqu[st]), acc, 0, 0, 0);
        sacc[t] = acc;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = NV1; it < NVL; it++) vload(it);
    __builtin_amdgcn_sched_barrier(0);
    wave_lds_fence();                            // the bd tile is written

    // ---- scores, rel_shift gather, softmax over keys [ks, ke) of query col.  Scores stay unscaled
    //      until the exponential: p = 2^(s c2 - max c2) with c2 = scale log2 e.  When every ring row
    //      is a key (wave-uniform; steady-state full chunks) only the padding rows past R are masked:
    //      lanes of queries i >= T compute finite values that no output uses.
    const int i = col;
    const bool full = ks == 0 && ke == R && W == R;
    const float c2 = a.scale * 1.4426950408889634f;
    float pr[KT][4];
    float mx = -INFINITY;
    if (full) {
#pragma unroll
        for (int t = 0; t < KT; t++) {
            int j0 = 16 * t + 4 * g - start;     // window key of ring row 16t + 4g, before the wrap
            j0 += j0 < 0 ? R : 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int j = j0 + r;
                j -= j >= R ? R : 0;
                const int bi = min(W - 1 + i - j, BMAX - 1);
                const float x = sacc[t][r] + sl[i][bi];
                pr[t][r] = 16 * t + 4 * g + r < R ? x : -INFINITY;     // padding rows past R
                mx = fmaxf(mx, pr[t][r]);
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < KT; t++) {
            int j0 = 16 * t + 4 * g - start;     // window key of ring row 16t + 4g, before the wrap
            j0 += j0 < 0 ? R : 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int rr = 16 * t + 4 * g + r;   // ring row
                int j = j0 + r;
                j -= j >= R ? R : 0;
                const bool kin = i < Tq && rr < R && j >= ks && j < ke;
                const int bi = min(max(W - 1 + i - j, 0), BMAX - 1);
                const float x = sacc[t][r] + sl[i][bi];
                pr[t][r] = kin ? x : -INFINITY;
                mx = fmaxf(mx, pr[t][r]);
            }
        }
    }
    mx = xmax32(xmax16(mx));
    // a masked score is -inf and 2^-inf = 0; a query with no key at all has mx = -inf and any
    // finite offset serves
    const float mc = mx == -INFINITY ? 0.0f : mx * c2;
    float sm = 0.0f;
#pragma unroll
    for (int t = 0; t < KT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            pr[t][r] = __builtin_amdgcn_exp2f(fmaf(pr[t][r], c2, -mc));
            sm += pr[t][r];
        }
    sm = xadd32(xadd16(sm));
    const float inv = sm > 0.0f ? 1.0f / sm : 0.0f;

    // ---- out^T = V^T . P^T, one 32-row piece of V at a time through LDS.  A = V^T by
    //      ds_read_b64_tr_b16: lane c of a 16-lane group gets column c & 3 of the rows named by
    //      lanes c / 4 + 4 e, so lane (c, g) holds positions 8g .. 8g+7 of channel 16 dt + c.
    //      B = this lane's probabilities of the piece's two tiles, positions 8g + e.  Row 4a + g'
    //      of the piece (V load 8 kk + a of lane group g') goes to position 8a + g' (a < 4) or
    //      8(a - 4) + 4 + g'.  Rows outside the key range are zeroed unless every ring row is a
    //      key (wave-uniform).  The transposed product leaves each lane 4 consecutive channels
    //      of query col.
    const bool vfull = ks == 0 && ke == R;
    const int jb = g - start;                    // window key of ring row g, before the wrap
    f32x4_t oacc[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) oacc[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < KP; kk++) {
#pragma unroll
        for (int a8 = 0; a8 < 8; a8++) {
            const int it = 8 * kk + a8;
            const int pos = a8 < 4 ? 8 * a8 + g : 8 * (a8 - 4) + 4 + g;
            uint4 w = make_uint4(0, 0, 0, 0);
            if (it < NVL) {
                if (vfull) {
                    w = vr[it];
                } else {
                    int j = jb + 4 * it;
                    j += j < 0 ? R : 0;
                    const uint32_t keep = (4 * it + g < R && j >= ks && j < ke) ? 0xFFFFFFFFu : 0u;   // a mask, no branch
                    w = make_uint4(vr[it].x & keep, vr[it].y & keep, vr[it].z & keep, vr[it].w & keep);
                }
            }
            *reinterpret_cast<uint4*>(&vp[pos][col * 8]) = w;
        }
        float pf[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            pf[e] = 2 * kk < KT ? pr[2 * kk][e] * inv : 0.0f;
            pf[4 + e] = 2 * kk + 1 < KT ? pr[2 * kk + 1][e] * inv : 0.0f;
        }
        const uint4 pa = pack_f16x8_unit(pf);
        wave_lds_fence();
        const int k0 = 8 * g + (col >> 2);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const int c0 = 16 * dt + 4 * (col & 3);
            const v4i16_t b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)&vp[k0][c0]);
            const v4i16_t b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)&vp[k0 + 4][c0]);
            uint4 bv;
            __builtin_memcpy(&bv.x, &b0, 8);
            __builtin_memcpy(&bv.z, &b1, 8);
            oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(bv), as_f16x8(pa), oacc[dt], 0, 0, 0);
        }
        wave_lds_fence();                        // this piece's reads are done before the next writes
    }

    // ---- output: lane holds out[col][16 dt + 4 g + r], r < 4 (exactly 0 for an empty key range:
    //      every probability is 0 and so is every staged V row); 8-byte stores, contiguous in
    //      either layout
    T* att = static_cast<T*>(a.att);
    if (live && col < Tq) {
        const int64_t orow = (int64_t)s * Tq + col;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const int c = h * 128 + 16 * dt + 4 * g;
            const int64_t idx = a.att_frag ? frag_index(orow, c, D / 64) : orow * D + c;
            const uint2 w = make_uint2((uint32_t)f2h(oacc[dt][0]) | ((uint32_t)f2h(oacc[dt][1]) << 16),
                                       (uint32_t)f2h(oacc[dt][2]) | ((uint32_t)f2h(oacc[dt][3]) << 16));
            *reinterpret_cast<uint2*>(att + idx) = w;
        }
    }
}

int launch_relpos_ring_mfma(const RingArgs& a, hipStream_t st) {
    using namespace rm;
    if (a.T < 1 || a.T > 16 || a.R > KMAX || a.L + 2 * a.T - 1 > BMAX || a.n < 1 || a.H < 1 || !a.zero_row ||
        a.L + a.T > a.R)
        return -2;
    if (a.rel_offset + 1 - a.T < 0 || a.rel_offset + a.L + a.T - 1 >= a.n_rel) return -2;
    const dim3 grid(a.H * ((a.n + NW - 1) / NW)), block(64 * NW);
    const int kt = (a.R + 15) / 16, nvl = (a.R + 3) / 4;
    if (kt == 6 && nvl == 21) hipLaunchKernelGGL((relpos_ring_mfma_kernel<6, 21>), grid, block, 0, st, a);
    else switch (kt) {
        case 1: hipLaunchKernelGGL((relpos_ring_mfma_kernel<1, 4>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((relpos_ring_mfma_kernel<2, 8>), grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL((relpos_ring_mfma_kernel<3, 12>), grid, block, 0, st, a); break;
        case 4: hipLaunchKernelGGL((relpos_ring_mfma_kernel<4, 16>), grid, block, 0, st, a); break;
        case 5: hipLaunchKernelGGL((relpos_ring_mfma_kernel<5, 20>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((relpos_ring_mfma_kernel<6, 24>), grid, block, 0, st, a); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------------ launchers

// Keys per block: as many as keep the workgroup's LDS under 64 KB.
template <typename T, int TQ> struct KeyBlock { static constexpr int KB = sizeof(T) == 2 ? (TQ <= 8 ? 128 : 96) : 64; };

template <typename T, int DK>
static int launch_op_dk(const OpArgs& a, hipStream_t st) {
    dim3 grid(a.H), block(256);
    const T* Q = static_cast<const T*>(a.q); const T* K = static_cast<const T*>(a.k);
    const T* V = static_cast<const T*>(a.v); const T* P = static_cast<const T*>(a.p);
    T* O = static_cast<T*>(a.out);
    if (a.Tq <= 2)
        hipLaunchKernelGGL((relpos_op_kernel<T, DK, 2, KeyBlock<T, 2>::KB>), grid, block, 0, st, Q, K, V, P, a.u,
                           a.vb, a.ranges, O, a.Tq, a.Tk, a.H, a.rel_offset, a.n_rel, a.scale);
    else
        hipLaunchKernelGGL((relpos_op_kernel<T, DK, 16, KeyBlock<T, 16>::KB>), grid, block, 0, st, Q, K, V, P, a.u,
                           a.vb, a.ranges, O, a.Tq, a.Tk, a.H, a.rel_offset, a.n_rel, a.scale);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <typename T>
static int launch_op_t(const OpArgs& a, hipStream_t st) {
    switch (a.dk) {
        case 16: return launch_op_dk<T, 16>(a, st);
        case 32: return launch_op_dk<T, 32>(a, st);
        case 64: return launch_op_dk<T, 64>(a, st);
        case 128: return launch_op_dk<T, 128>(a, st);
        default: return -2;
    }
}

int launch_relpos_op(const OpArgs& a, bool bf16_data, hipStream_t st) {
    if (a.Tq < 1 || a.Tq > 16 || a.H < 1) return -2;
    return bf16_data ? launch_op_t<bf16>(a, st) : launch_op_t<float>(a, st);
}

template <typename T>
static int launch_ring_t(const RingArgs& a, hipStream_t st) {
    dim3 grid(a.n * a.H), block(256);
    // 16-bit streaming chunks (T <= 4, 16 <= L, L + T <= 96 keys, head_dim 128): the one-round-trip kernel.
    // It reads the band rel = 1-T .. L+T-1 (table rows rel_offset+1-T .. rel_offset+L+T-1).
    const bool band_ok = a.rel_offset + 1 - a.T >= 0 && a.rel_offset + a.L + a.T - 1 < a.n_rel;
    if (sizeof(T) == 2 && a.T <= 4 && a.L >= 16 && a.L + a.T <= 96 && a.L + 2 * a.T - 1 <= 112 && band_ok) {
        const int kr = (a.L + a.T + 15) / 16, pr = (a.L + 2 * a.T - 1 + 15) / 16;
        if (a.T <= 2 && kr <= 5) hipLaunchKernelGGL((relpos_ring_wave_kernel<2, 5>), grid, block, 0, st, a);
        else if (a.T <= 2) hipLaunchKernelGGL((relpos_ring_wave_kernel<2, 6>), grid, block, 0, st, a);
        else if (kr <= 5 && pr <= 5) hipLaunchKernelGGL((relpos_ring_small_kernel<4, 5, 5>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((relpos_ring_small_kernel<4, 6, 7>), grid, block, 0, st, a);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    // 16-bit chunks of 5..16 frames (rings of R <= 96 rows): the MFMA kernel, one wave per (stream, head).
    if (sizeof(T) == 2 && a.T <= 16 && a.R <= 96 && a.L + 2 * a.T - 1 <= 112 && band_ok && a.zero_row)
        return launch_relpos_ring_mfma(a, st);
    if (a.T <= 2) hipLaunchKernelGGL((relpos_ring_kernel<T, 2, KeyBlock<T, 2>::KB>), grid, block, 0, st, a);
    else if (a.T <= 4) hipLaunchKernelGGL((relpos_ring_kernel<T, 4, KeyBlock<T, 4>::KB>), grid, block, 0, st, a);
    else if (a.T <= 8) hipLaunchKernelGGL((relpos_ring_kernel<T, 8, KeyBlock<T, 8>::KB>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((relpos_ring_kernel<T, 16, KeyBlock<T, 16>::KB>), grid, block, 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_relpos_ring(const RingArgs& a, bool half_data, hipStream_t st) {
    if (a.T < 1 || a.T > 16 || a.T > a.L || a.n < 1 || a.L + a.T > a.R) return -2;
    return half_data ? launch_ring_t<f16>(a, st) : launch_ring_t<float>(a, st);
}

int launch_ring_append(const RingArgs& a, bool half_data, hipStream_t st) {
    if (a.T < 1 || a.n < 1 || a.H < 1 || a.L + a.T > a.R) return -2;
    if (half_data) hipLaunchKernelGGL(ring_append_kernel<f16>, dim3(a.n * a.H), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(ring_append_kernel<float>, dim3(a.n * a.H), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ud
