// Offline (whole-utterance) fused relative-position attention for gfx950: relpos_dense_kernel.
//
// Semantics as attention.hip (Sources/DictatorEngine/Metal/20_conformer.metal:140-220, dispatched
// by Sources/DictatorEngine/Core/Ops.swift:80-90) over T x T with per-query key ranges.  A file of
// its own so that it compiles with the machine scheduler's max-ilp strategy (build.py): this
// kernel runs at two waves per SIMD and is bound by instruction latency, and that schedule took a
// launch at 8 x 1500 frames from 148.1-148.4 to 144.9-145.2 us with bit-identical output, while
// the streaming ring kernels ran slower under it (6.70 -> 6.86 us at 64 streams x 2 frames).
#include "ud_common.hpp"
#include "kernels.hpp"

namespace ud {

typedef short v4i16_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ offline (dense) MFMA kernel
// Whole-utterance attention (the offline path's relpos_attention over T x T with per-query key
// ranges; key padding and chunked masks are both ranges).  Flash-style: a workgroup of 8 wave64s
// owns 128 queries of one (sequence, head) and sweeps 64-key tiles with an online softmax; each
// wave owns 16 queries, all products on v_mfma_f32_16x16x32_bf16 with plain bf16 operands
// (q+u, q+v and probabilities rounded to bf16: the errors average over the long key range).
//   K and V tiles are staged in LDS (V^T for P.V through ds_read_b64_tr_b16);
//   the positional band: tile t needs table rows rel = i - j over [i0 - 63 - 64t, i0 + 128 - 64t),
//   three 64-row chunks; consecutive tiles share two of them, so LDS keeps a 3-chunk ring and each
//   tile fetches one new chunk;
//   bd tiles are computed per wave over its 80-row sub-band and gathered through LDS for the
//   rel_shift (score (i, j) reads band row i - j + 63 of the wave's window);
//   every product is transposed (C[key][query] = K.(q+u)^T, C[band row][query] = P.(q+v)^T,
//   C[chan][query] = V^T.P^T), so a lane holds one query: its softmax reduces over 4 lanes with
//   lane swaps, its probabilities stay in registers as the B operand of P.V (k order permuted the
//   same way in the transposed V reads), and its output is 4 consecutive channels per store;
//   the next tile's K, V and band chunk are prefetched into registers during the current tile.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): this wave's LDS ops are done
    __asm__ volatile("" ::: "memory");
}

__global__ __launch_bounds__(512) void relpos_dense_kernel(DenseArgs a) {
    using T = bf16;
    // Row strides.  gfx950's LDS serves a ds_read_b128 16 lanes (256 bytes, 64 banks) at a time,
    // but not as lanes 0-15: lanes 0-7 share a cycle with lanes 24-31 (and so on), so 16-byte
    // reads of one piece along 16 consecutive rows (lane c: row c, piece p + lane / 16) are
    // conflict-free only for a row stride of 2 mod 4 16-byte units (measured: 18 and 22 units run
    // at full rate, 17 -- the obvious padding -- at half).  K and band rows therefore take 144 bf16
    // (288 bytes, 18 units), like the V rows, which ds_read_b64_tr_b16 reads 4 consecutive rows per
    // 16 lanes; the bd rows take 84 floats (measured faster than 88).
    constexpr int DK = 128, KT = 64, VST = DK + 16, VVST = DK + 16, NW = 8, SWS = 84;
    __shared__ __align__(16) bf16 kl[KT][VST];
    __shared__ __align__(16) bf16 vl[KT][VVST];
    __shared__ __align__(16) bf16 pl[3 * KT][VST];
    __shared__ __align__(16) float sw[NW][16][SWS];
    __shared__ int kbound[2];

    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: its index math is scalar
    const int Tn = a.T, D = a.H * DK;
    // ---- which (utterance, head, 128-query block) this workgroup owns.  1-D grid; the pairs
    //      (utterance, head) are taken longest utterance first (key span of its first and last
    //      query; up to 64 utterances, else in order), and when they divide among the 8 XCDs
    //      (workgroups are dealt round-robin) all query blocks of a pair run on one XCD, whose L2
    //      then serves their shared K, V and band tiles.  Longest-first dispatch ends the sweep
    //      with the short utterances' workgroups instead of leaving long ones to run alone.
    __shared__ int bord[64];
    const int nq = (Tn + 127) / 128, id = blockIdx.x;
    if (a.B <= 64) {
        __shared__ int bwork[64];
        if (tid < a.B) {
            const int32_t* Rb = a.ranges + (int64_t)tid * Tn * 2;
            bwork[tid] = max(min(Rb[2 * (Tn - 1) + 1], Tn) - max(Rb[0], 0), 0);
        }
        __syncthreads();
        if (tid < a.B) {
            const int w = bwork[tid];
            int rank = 0;
            for (int o = 0; o < a.B; o++) rank += (bwork[o] > w || (bwork[o] == w && o < tid)) ? 1 : 0;
            bord[rank] = tid;
        }
    } else if (tid == 0) {
        bord[0] = -1;
    }
    __syncthreads();
    int pr, qb;
    if ((a.B * a.H) % 8 == 0) {
        const int j = id >> 3;
        pr = (id & 7) + 8 * (j / nq); qb = j % nq;
    } else {
        pr = id / nq; qb = id % nq;
    }
    const int h = pr % a.H, b = a.B <= 64 ? bord[pr / a.H] : pr / a.H;
    const int i0 = qb * 128, iw = i0 + 16 * wave;
    const float c2 = a.scale * 1.4426950408889634f;      // scores in log2 units: exp(s * scale) = 2^(s * c2)
    const T* Q = static_cast<const T*>(a.q) + (int64_t)b * Tn * D + h * DK;
    const T* K = static_cast<const T*>(a.k) + (int64_t)b * Tn * D + h * DK;
    const T* V = static_cast<const T*>(a.v) + (int64_t)b * Tn * D + h * DK;
    const T* P = static_cast<const T*>(a.P) + h * DK;
    const int32_t* R = a.ranges + (int64_t)b * Tn * 2;

    // ---- key range of the block: union of its queries' ranges
    if (tid == 0) { kbound[0] = Tn; kbound[1] = 0; }
    __syncthreads();
    if (tid < 128 && i0 + tid < Tn) {
        const int ks = max(R[2 * (i0 + tid)], 0), ke = min(R[2 * (i0 + tid) + 1], Tn);
        if (ks < ke) { atomicMin(&kbound[0], ks); atomicMax(&kbound[1], ke); }
    }
    __syncthreads();
    const int t_lo = kbound[0] / KT, t_hi = kbound[0] < kbound[1] ? (kbound[1] + KT - 1) / KT : t_lo;

    // ---- the lane's query (row col of the wave's 16) and its key range
    const int qi = iw + col;
    const int qks = qi < Tn ? max(R[2 * qi], 0) : 0, qke = qi < Tn ? min(R[2 * qi + 1], Tn) : 0;
    // ---- B operands: q + u, q + v in bf16 (query iw + col, k-chunk 4st + g)
    uint4 aqu[4], aqv[4];
    {
        const T* qr = Q + (int64_t)min(iw + col, Tn - 1) * D;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int c = (4 * st + g) * 8;
            float qf[8];
            unpack16<T>(ld16(qr + c), qf);
            const float4 u0 = *reinterpret_cast<const float4*>(a.u + h * DK + c);
            const float4 u1 = *reinterpret_cast<const float4*>(a.u + h * DK + c + 4);
            const float4 v0 = *reinterpret_cast<const float4*>(a.vb + h * DK + c);
            const float4 v1 = *reinterpret_cast<const float4*>(a.vb + h * DK + c + 4);
            const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            uint32_t pu[4], pv[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                pu[e / 2] = pack_bf16x2(qf[e] + uu[e], qf[e + 1] + uu[e + 1]);
                pv[e / 2] = pack_bf16x2(qf[e] + vv[e], qf[e + 1] + vv[e + 1]);
            }
            aqu[st] = make_uint4(pu[0], pu[1], pu[2], pu[3]);
            aqv[st] = make_uint4(pv[0], pv[1], pv[2], pv[3]);
        }
    }

    // ---- tile loaders: 1024 16-byte pieces per 64-row tile, 2 per thread
    auto load_rows = [&](const T* base, int r0, uint4 (&x)[2]) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int idx = tid + 512 * e, row = idx >> 4, cc = idx & 15;
            x[e] = ld16(base + (int64_t)min(r0 + row, Tn - 1) * D + cc * 8);
        }
    };
    auto load_chunk = [&](int k, uint4 (&x)[2]) {       // band chunk k: rel in [i0 - 63 - 64k, i0 + 1 - 64k)
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int idx = tid + 512 * e, row = idx >> 4, cc = idx & 15;
            const int tr = min(max(i0 - 63 - 64 * k + row + a.rel_offset, 0), a.n_rel - 1);
            x[e] = ld16(P + (int64_t)tr * D + cc * 8);
        }
    };
    auto store_rows = [&](auto dst, const uint4 (&x)[2]) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int idx = tid + 512 * e, row = idx >> 4, cc = idx & 15;
            *reinterpret_cast<uint4*>(&dst[row][cc * 8]) = x[e];
        }
    };
    auto ring = [](int k) { return ((k % 3) + 3) % 3; };
    // Band row rel = iw - j0 - 63 + 16tb + col of tile t lies in chunk k = t + dch[tb], row boff[tb]
    // of it: k = floor((i0 - rel) / 64) and i0 - rel = 64t + 63 - 16 wave - 16tb - col, whose
    // remainder part lies in [-128, 63].
    int dch[5], boff[5];
#pragma unroll
    for (int tb = 0; tb < 5; tb++) {
        const int x = 63 - 16 * wave - 16 * tb - col;
        dch[tb] = x >= 0 ? 0 : (x >= -64 ? -1 : -2);
        boff[tb] = 16 * wave + 16 * tb + col + 64 * dch[tb];
    }

    // m: the query's exponent offset (a running maximum of its unscaled scores, raised lazily)
    float m = -INFINITY;
    // the query's running sum of its bf16 probabilities, on the matrix cores: every element of
    // ones(16 x 32) . P^T is the sum over the piece's 32 keys, so each lane holds its query's total
    f32x4_t lacc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t oacc[8];                          // out^T: lane holds channels 16dt + 4g + r of query col
#pragma unroll
    for (int dt = 0; dt < 8; dt++) oacc[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    f32x4_t bkeep = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};   // band rows 0..15 of the previous tile
    if (t_lo < t_hi) {                        // prologue: tile t_lo and its three band chunks
        uint4 x[2];
        load_rows(K, t_lo * KT, x); store_rows(kl, x);
        load_rows(V, t_lo * KT, x); store_rows(vl, x);
#pragma unroll
        for (int c = 0; c < 3; c++) { load_chunk(t_lo - c, x); store_rows(&pl[ring(t_lo - c) * KT], x); }
    }
    for (int t = t_lo; t < t_hi; t++) {
        const int j0 = t * KT;
        uint4 nk[2], nv[2], np[2];
        const bool more = t + 1 < t_hi;
        if (more) { load_rows(K, j0 + KT, nk); load_rows(V, j0 + KT, nv); load_chunk(t + 1, np); }
        __syncthreads();

        // ---- ac = K . (q+u)^T: lane holds query col at keys 16ts + 4g + r.  The k chunk is the
        //      outer loop, so the 4 accumulators are independent and a chunk's fragments are read
        //      together.
        f32x4_t sacc[4];
#pragma unroll
        for (int ts = 0; ts < 4; ts++) sacc[ts] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 4; st++) {
            uint4 ak[4];
#pragma unroll
            for (int ts = 0; ts < 4; ts++) ak[ts] = *reinterpret_cast<const uint4*>(&kl[16 * ts + col][(4 * st + g) * 8]);
#pragma unroll
            for (int ts = 0; ts < 4; ts++)
                sacc[ts] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ak[ts]), as_bf16x8(aqu[st]), sacc[ts], 0, 0, 0);
        }
        // ---- bd = P_band . (q+v)^T over the wave's 80 band rows rel = iw - j0 - 63 + n (n < 80);
        //      lane holds band rows 16tb + 4g .. +3 of query col: one 16-byte write per tile.
        //      Rows 64..79 of tile t are rows 0..15 of tile t - 1 (rel depends on j0 - n only), so
        //      after the first tile the wave keeps that accumulator instead of recomputing it: four
        //      independent accumulators (five in the first tile), k chunk outermost.
        {
            const int r0 = t % 3;
            int prow[5];
#pragma unroll
            for (int tb = 0; tb < 5; tb++) {
                int c = r0 + dch[tb] + 3;                      // ring slot of chunk t + dch[tb]
                c = c >= 3 ? c - 3 : c;
                prow[tb] = c * KT + boff[tb];
            }
            f32x4_t bacc[5];
#pragma unroll
            for (int tb = 0; tb < 5; tb++) bacc[tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 4; st++) {
                uint4 ap[4];
#pragma unroll
                for (int tb = 0; tb < 4; tb++) ap[tb] = *reinterpret_cast<const uint4*>(&pl[prow[tb]][(4 * st + g) * 8]);
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
                    bacc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ap[tb]), as_bf16x8(aqv[st]), bacc[tb], 0, 0, 0);
            }
            if (t == t_lo) {
#pragma unroll
                for (int st = 0; st < 4; st++) {
                    const uint4 ap = *reinterpret_cast<const uint4*>(&pl[prow[4]][(4 * st + g) * 8]);
                    bacc[4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ap), as_bf16x8(aqv[st]), bacc[4], 0, 0, 0);
                }
            } else {
                bacc[4] = bkeep;
            }
            bkeep = bacc[0];
#pragma unroll
            for (int tb = 0; tb < 5; tb++)
                *reinterpret_cast<float4*>(&sw[wave][col][16 * tb + 4 * g]) = make_float4(bacc[tb][0], bacc[tb][1], bacc[tb][2], bacc[tb][3]);
        }
        wave_lds_sync();

        // ---- scores and the online softmax of query col.  Key 16ts + 4g + r uses band row
        //      col - 16ts - 4g - r + 63 of the wave's window (0..78): four consecutive floats.
        //      A tile inside every key range of the wave's queries (the common case) skips the
        //      masks; the accumulator is rescaled only when some query's maximum grew by more than 2^8.
        const bool inside = __all(j0 >= qks && j0 + KT <= qke);
        float sc[4][4];
#pragma unroll
        for (int ts = 0; ts < 4; ts++) {              // the 16 band reads are issued together
            const float* bp = &sw[wave][col][col - 16 * ts - 4 * g + 60];
#pragma unroll
            for (int r = 0; r < 4; r++) sc[ts][r] = bp[3 - r];
        }
#pragma unroll
        for (int ts = 0; ts < 4; ts++)
#pragma unroll
            for (int r = 0; r < 4; r++) sc[ts][r] += sacc[ts][r];
        if (!inside) {                                // keys outside a query's range: -inf
#pragma unroll
            for (int ts = 0; ts < 4; ts++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int j = j0 + 16 * ts + 4 * g + r;
                    sc[ts][r] += (j >= qks && j < qke) ? 0.0f : -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int ts = 0; ts < 4; ts++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, sc[ts][r]);
        mx = xmax32(xmax16(mx));
        // The offset m is raised only when a score exceeds it by more than 8 in log2 units (a
        // probability above 2^8): softmax does not depend on the offset, and between raises the
        // probabilities stay in (0, 256], exact enough in fp32 and as bf16 P.V operands, so most
        // tiles skip the accumulator's rescale.  (mx - m) is NaN, not > 8, while a query has no
        // key yet, and +inf on its first key.
        const bool grow = (mx - m) * c2 > 8.0f;
        if (__any(grow)) {
            const float nm = grow ? mx : m;
            const float corr = (m == -INFINITY || !grow) ? 1.0f : __builtin_amdgcn_exp2f((m - nm) * c2);
            lacc *= corr;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) oacc[dt] *= corr;
            m = nm;
        }
        // a masked score is -inf and 2^-inf = 0; while a query has no key yet (m = -inf) every
        // score of it is -inf and any finite offset serves
        const float mc = m == -INFINITY ? 0.0f : m * c2;
#pragma unroll
        for (int ts = 0; ts < 4; ts++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sc[ts][r] = __builtin_amdgcn_exp2f(fmaf(sc[ts][r], c2, -mc));
            }

        // ---- out^T += V^T . P^T per 32-key piece (tiles 2kk, 2kk + 1).  B = this lane's
        //      probabilities: position 8g + e holds key 32kk + 4g + e (e < 4), then 32kk + 16 + 4g + e - 4;
        //      A = V^T by ds_read_b64_tr_b16 over the same keys (lane c of a 16-lane group gets column
        //      c & 3 of the rows named by lanes c / 4 + 4e: rows 32kk + 4g .. +3, then 32kk + 16 + 4g ..).
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const float* p0 = sc[2 * kk];
            const float* p1 = sc[2 * kk + 1];
            const uint4 pb = make_uint4(pack_bf16x2(p0[0], p0[1]), pack_bf16x2(p0[2], p0[3]),
                                        pack_bf16x2(p1[0], p1[1]), pack_bf16x2(p1[2], p1[3]));
            const int k0 = 32 * kk + 4 * g + (col >> 2);
            lacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u)),
                                                          as_bf16x8(pb), lacc, 0, 0, 0);
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const int c0 = 16 * dt + 4 * (col & 3);
                const v4i16_t b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)&vl[k0][c0]);
                const v4i16_t b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)&vl[k0 + 16][c0]);
                uint4 av;
                __builtin_memcpy(&av.x, &b0, 8);
                __builtin_memcpy(&av.z, &b1, 8);
                oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(pb), oacc[dt], 0, 0, 0);
            }
        }
        wave_lds_sync();                          // every lane's reads of sw are done before the next tile writes it
        __syncthreads();
        if (more) {
            store_rows(kl, nk);
            store_rows(vl, nv);
            store_rows(&pl[ring(t + 1) * KT], np);
        }
    }

    // ---- output: out[iw + col][16dt + 4g .. +3] (0 for an empty key range): 8-byte stores
    T* O = static_cast<T*>(a.out) + (int64_t)b * Tn * D + h * DK;
    const float l = lacc[0];
    if (qi < Tn) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const uint2 w = make_uint2(pack_bf16x2(oacc[dt][0] * inv, oacc[dt][1] * inv),
                                       pack_bf16x2(oacc[dt][2] * inv, oacc[dt][3] * inv));
            *reinterpret_cast<uint2*>(O + (int64_t)qi * D + 16 * dt + 4 * g) = w;
        }
    }
}

int launch_relpos_dense(const DenseArgs& a, hipStream_t st) {
    if (a.B < 1 || a.T < 1 || a.H < 1) return -2;
    const int64_t blocks = (int64_t)((a.T + 127) / 128) * a.H * a.B;
    if (blocks >= (1ll << 31)) return -2;
    hipLaunchKernelGGL(relpos_dense_kernel, dim3((unsigned)blocks), dim3(512), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ud
