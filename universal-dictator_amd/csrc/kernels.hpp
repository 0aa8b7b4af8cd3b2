// Host-side launch interface of the encoder-step kernels (one translation unit per kernel family;
// the encoder host layer calls these launchers).  Launchers return 0, -1 (HIP launch error) or
// -2 (shape outside what the kernel supports).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct ud_mel;
struct ud_encoder;
// Device scratch of at least `bytes` owned by the encoder (grown on demand, freed with it; growing
// waits for the event of the last ud_encoder_aux_release); nullptr when the allocation fails.
void* ud_encoder_aux_scratch(ud_encoder* e, size_t bytes);
// Records, on `st`, the end of a use of that scratch (after the last work that touches it).
int ud_encoder_aux_release(ud_encoder* e, hipStream_t st);

namespace ud {

// Activation codes (Sources/DictatorEngine/Core/Kernels.swift:4-6).
enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };

// Per-stream step descriptor, int32 x8: {pool slot, K/V window start ((frames - L) mod R), valid
// frames this step, cached frames (min(frames, L)), conv ring origin (frames mod (K-1)), 0, 0, 0}.
// 32 bytes: one scalar load per workgroup.
//
// K/V rings: each (slot, head) holds R = L + max_chunk rows of 128 values; frame f of the stream
// lives in row f mod R.  A step over frames F .. F+T-1 (T <= max_chunk) attends to the window of
// keys j = 0 .. L+T-1 = frames F-L+j, rows (start + j) mod R with start = (F - L) mod R: the L
// cached frames and the T new ones, which the QKV projection has already written to rows
// (F + i) mod R -- with R >= L + T they overwrite no row of the window.  The attention kernels only
// read the rings.
constexpr int DESC_INTS = 8;

// ---------------------------------------------------------------- attention
struct OpArgs {
    const void* q; const void* k; const void* v; const void* p;
    const float* u; const float* vb; const int32_t* ranges; void* out;
    int Tq, Tk, H, dk, rel_offset, n_rel;
    float scale;
};
int launch_relpos_op(const OpArgs& a, bool bf16_data, hipStream_t st);

// Offline (whole-utterance) rel-pos attention over a batch of B sequences of T frames, bf16,
// head_dim 128: q/k/v/out [B][T][H*128], P [n_rel][H*128], ranges int32 [B][T][2].
struct DenseArgs {
    const void* q; const void* k; const void* v; const void* P;
    const float* u; const float* vb; const int32_t* ranges;
    void* out;
    int B, T, H, rel_offset, n_rel;
    float scale;
};
int launch_relpos_dense(const DenseArgs& a, hipStream_t st);

struct RingArgs {
    void* kring; void* vring;       // layer base of the pool: [slots][H][R][128]
    const void* qkv;                // [n*T, 3*D]: the attention kernels read q (columns 0..D-1);
                                    // launch_ring_append reads K and V
    const void* P;                  // [n_rel, D]
    const float* u; const float* vb;   // [H*128]
    void* att;                      // [n*T, D]: row-major, or fragment-major when att_frag (bf16)
    const int32_t* desc;            // [n][DESC_INTS]
    const void* zero_row;           // >= 256 zero bytes, 16-byte aligned (masked rows' loads)
    int n, T, L, R, H, rel_offset, n_rel;
    float scale;
    int att_frag;
};
int launch_relpos_ring(const RingArgs& a, bool bf16_data, hipStream_t st);
// Copies the T new K/V rows of every stream from qkv into rows (start + L + i) mod R of its rings
// (for callers whose K/V come in a qkv buffer rather than from the fused QKV projection).
int launch_ring_append(const RingArgs& a, bool half_data, hipStream_t st);
// Read floor of the bf16 streaming kernel (chunks of <= 2 frames, L + T <= 80): its loads only.
int launch_ring_read_floor(const RingArgs& a, hipStream_t st);

// ---------------------------------------------------------------- fragment-major layout
// bf16 GEMM operands live in HBM in the order the v_mfma_f32_16x16x32_bf16 lanes consume them:
// a [R, K] matrix (R padded to 16, K % 64 == 0) is a sequence of 2 KB blocks, block (rt, kc) =
// rows [16rt, 16rt+16) x cols [64kc, 64kc+64) at element offset (rt * K/64 + kc) * 1024; inside a
// block, element h*512 + lane*8 + e (lane = 16*g + r) holds X[16rt + r][64kc + 32h + 8g + e].
// Every fragment load of a wave is then one contiguous, fully used 1 KB access.
__host__ __device__ inline int64_t frag_index(int64_t m, int c, int nk) {
    const int rt = (int)(m >> 4), r = (int)(m & 15), kc = c >> 6, w = c & 63;
    const int h = w >> 5, g = (w >> 3) & 3, e = w & 7;
    return (((int64_t)rt * nk + kc) << 10) + (h << 9) + ((g * 16 + r) << 3) + e;
}

// ---------------------------------------------------------------- GEMM  C = epi(A . W^T)
enum Epi : int {
    EPI_STORE = 0,      // C[m,n] = act(acc) * out_scale, activation dtype, row-major
    EPI_RESID = 1,      // C[m,n] += out_scale * acc   (C fp32 residual, in place)
    EPI_STORE_F32 = 3,  // C[m,n] = act(acc) * out_scale as fp32, row-major
    EPI_STORE_FRAG = 4, // as EPI_STORE but bf16 in fragment-major layout (the next GEMM's A)
    EPI_PARTIAL = 5,    // C[kz][m][n] = out_scale * (K-split kz partial), fp32; slabs M*ldc apart
    EPI_QKV_RING = 6,   // 16-bit QKV projection (N = 3 D): columns < D (q) as EPI_STORE, K and V
                        // into their K/V ring rows (GemmArgs::ring)
    EPI_GLU = 7,        // 16-bit pointwise_conv1 with its weight rows in GLU-pair order (glu_row):
                        // output columns 32k .. 32k+15 are the values and 32k+16 .. 32k+31 the
                        // gates of channels 16k .. 16k+15; C[m][c] = value * sigmoid(gate), IEEE
                        // half row-major [M, N/2] (ldc = N/2)
    EPI_SUBFLAT = 8     // IEEE-half subsampling conv.6 (GemmArgs::flat): row m = (s T3 + t3) F3 + f3
                        // of act(acc + bias) goes to row s T + t3 - drop, column f3 N + n of the out
                        // Linear's fragment-major A operand [n T, F3 N] (rows t3 < drop skipped,
                        // rows t3 >= vlen[4 s + 3] written as 0) -- the flatten, mask and drop
};
// EPI_SUBFLAT geometry.
struct SubFlat {
    const int32_t* vlen;            // [n][4]: valid rows per stage (index 3: after conv.5)
    int T3, F3, T, drop;
};
// Row of a GLU-pair-ordered pointwise_conv1 weight that holds checkpoint row r of [2 D, K]
// (r < D: value channel r; r >= D: gate channel r - D).
__host__ __device__ inline int glu_row(int r, int D) {
    const int gate = r >= D ? 1 : 0, c = r - gate * D;
    return (c >> 4) * 32 + gate * 16 + (c & 15);
}
// Where EPI_QKV_RING puts K and V: row m = stream s * T + i goes to ring row (start_s + L + i) mod R
// of the stream's slot, head (n - D) mod D / 128; rows[m] holds that row's element offset in the
// slot's head-0 block, (slot H R + ring row) * 128 (the host computes it with the descriptor).
struct QkvRing {
    void* kring; void* vring;       // layer base of the pool: [slots][H][R][128]
    const int32_t* rows;            // [M + 256]: ring element offset per output row (padded)
    int T, L, R, H;
};
// bf16: A [M, K] and W [N, K] in fragment-major layout (lda/ldw unused); M may be any size, the
// A buffer holding ceil(M/16)*16 rows.  fp32: row-major with leading dimensions lda/ldw/ldc.
struct GemmArgs {
    const void* A; const void* W; void* C;
    int M, N, K, lda, ldw, ldc;
    int epi, act;
    float out_scale;
    int ksplit;                     // EPI_PARTIAL: K splits chosen by the caller (gemm_partial_splits)
    const float* bias;              // [N] added before the activation: fp32 path (optional) and the
                                    // IEEE-half path (required); not the bf16 path
    int f16;                        // 16-bit path: operands (and 16-bit outputs) are IEEE half
                                    // instead of bf16
    QkvRing ring;                   // EPI_QKV_RING only
    SubFlat flat;                   // EPI_SUBFLAT only
};
int launch_gemm(const GemmArgs& a, bool bf16_data, hipStream_t st);
// fp32 GEMM for few rows (tens) on the fp32 MFMA: EPI_PARTIAL with ks K splits (slabs
// [ks][M][ldc]) or EPI_STORE (ks = 1, optional bias, act).  K % (16 ks) == 0, lda and ldw multiples
// of 4, A and W 16-byte aligned; any M and N.
int launch_gemm_f32_small(const GemmArgs& a, int ks, hipStream_t st);
// Most K splits of a bf16 residual projection (partial slabs the workspace holds).
constexpr int KSPLIT = 4;
// Rows from which the bf16 projections use the LDS-staged kernel (256- or 128-row tiles).
constexpr int LDS_MIN_ROWS = 2048;
struct BigTile { int nt, ks, ab; };   // 16*ab-row x 64*nt-column tiles (ab 16, 14 or 8), ks K splits
                                      // (nt 0: shape not supported)
// heights_mask: the tile heights that are candidates (TILE_256 | TILE_224 | TILE_128)
constexpr int TILE_256 = 1, TILE_224 = 2, TILE_128 = 4, TILE_ALL = 7;
BigTile big_tile(int M, int N, int K, bool partial, int heights_mask);
// K splits (partial slabs) a residual projection of this shape writes; launch_gemm expects it in
// GemmArgs::ksplit for EPI_PARTIAL.
int gemm_partial_splits(int M, int N, int K, bool bf16_data);

// ---------------------------------------------------------------- LayerNorm / conv / misc
// Pending residual update: nparts fp32 slabs [rows, D] (stride rows*D) that a split-K residual
// GEMM left; the LayerNorm kernels add them to the residual row in slab order before normalising.
struct Partials {
    const float* p;
    int n;
};
// x <- x + sum(parts) (written back when parts.n > 0); out = act(LN(x; g, b)), fp32 row-major
// or (out16) IEEE half fragment-major.
int launch_layernorm(float* x, Partials parts, const float* g, const float* b, void* out, bool out16, int rows,
                     int D, int act, hipStream_t st);
// v = src + sum(parts); res <- LN_a(v) (v itself when ga == nullptr); z <- LN_b(res) (fp32
// row-major or (z16) IEEE half fragment-major).
int launch_layernorm2(const float* src, Partials parts, float* res, const float* ga, const float* ba, const float* gb,
                      const float* bb, void* z, bool z16, int rows, int D, hipStream_t st);
// GLU of pointwise_conv1's fp32 [n*T, 2D] output (value | gate), or its half GLU rows, with the
// frame mask, causal depthwise conv over [conv ring (K-1 rows) ; T new GLU rows], conv LayerNorm +
// SiLU; writes z and the updated conv ring (which holds GLU rows).
struct ConvArgs {
    const float* pw;                // [n*T, 2D] pointwise_conv1 output (value | gate), fp32; or
    const uint16_t* glu;            // [n*T, D] the GLU already applied (EPI_GLU), IEEE half
                                    // (exactly one of pw / glu is set)
    float* ring;                    // layer base of the conv pool: [slots][K-1][D]
    const float* w_t;               // [K][D] depthwise weights, tap-major
    const float* ln_g; const float* ln_b;
    void* z;                        // [n*T, D]: fp32 row-major, or IEEE half fragment-major (z16)
    const int32_t* desc;
    int n, T, D, K;
    bool z16;
};
int launch_dwconv_ln(const ConvArgs& a, hipStream_t st);

// ---------------------------------------------------------------- subsampling front-end
// vlen: per stream 4 ints, the valid rows before conv.0 (mel) and after each stride-2 stage.
struct SubArgs {
    const float* mel;               // [n, T0, F0]
    const int32_t* vlen;            // [n][4]
    const float* c0w; const float* c0b; const float* c2w; const float* c2b;   // [C][9], [C]
    void* out;                      // conv.2 output as the conv.3 GEMM's A: [n*T2*F2, C]
    int n, T0, F0, T1, F1, T2, F2;
};
int launch_sub_conv01(const SubArgs& a, bool half_out, hipStream_t st);
struct SubDwArgs {
    const void* x;                  // [n, Hin, Win, C] fp32, or IEEE half for a half launch
    const int32_t* vlen;
    const float* w; const float* b; // [C][9], [C]
    void* out;                      // [n*Hout*Wout, C] GEMM A operand
    int n, Hin, Win, Hout, Wout, stage;   // stage: vlen index of x's valid rows
};
int launch_sub_dw(const SubDwArgs& a, bool half_out, hipStream_t st);
struct SubFlatArgs {
    const float* x;                 // [n, T3, F3, C] fp32
    const int32_t* vlen;
    void* out;                      // [n*T, F3*C] GEMM A operand
    int n, T3, F3, T, drop;
};
int launch_sub_flatten(const SubFlatArgs& a, bool half_out, hipStream_t st);

// Mel frontend (mel.hip).  One job = frames [f0, f0 + nf) of one clip, written as rows
// dst[(f - f0) * n_mels + m]; frame f takes the preemphasized samples [160 f - 200, 160 f + 200),
// read from src[idx - first] (the caller stages every sample the frames need plus the one before);
// indices >= n_audio are zero padding; frames >= zero_from are written as zeros.
struct MelJob {
    const float* src;
    float* dst;
    long long first, n_audio, f0, zero_from;
    int nf, pad_;
};
struct MelTables {
    const float* cos512; // cos(2 pi j / 512), j < 512
    const float* win;    // [400] analysis window
    const float* fbT;    // [257][n_mels]
    const int2* krange;  // [n_mels] bins lo .. hi-1 hold band m's nonzero filterbank weights
    int n_mels;
};
int launch_mel(const MelTables& t, const MelJob* jobs_dev, int n_jobs, int max_nf, hipStream_t st);
// The device tables of a ud_mel (include/ud_mel.h).
MelTables mel_tables_of(const struct ::ud_mel* m);

}  // namespace ud
