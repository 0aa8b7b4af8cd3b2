// Host-side launch interface of the encoder-step kernels (one translation unit per kernel family;
// the encoder host layer calls these launchers).  Launchers return 0, -1 (HIP launch error) or
// -2 (shape outside what the kernel supports).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ud {

// Activation codes (Sources/DictatorEngine/Core/Kernels.swift:4-6).
enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };

// Per-stream step descriptor, int32 x4: {pool slot, frames appended so far modulo L*(K-1) (the
// ring origins are frames % L and frames % (K-1)), valid frames this step, cached frames}.
constexpr int DESC_INTS = 4;

// ---------------------------------------------------------------- attention
struct OpArgs {
    const void* q; const void* k; const void* v; const void* p;
    const float* u; const float* vb; const int32_t* ranges; void* out;
    int Tq, Tk, H, dk, rel_offset, n_rel;
    float scale;
};
int launch_relpos_op(const OpArgs& a, bool bf16_data, hipStream_t st);

struct RingArgs {
    void* kring; void* vring;       // layer base of the pool: [slots][H][L][128]
    const void* qkv;                // [n*T, 3*D]
    const void* P;                  // [n_rel, D]
    const float* u; const float* vb;   // [H*128]
    void* att;                      // [n*T, D]
    const int32_t* desc;            // [n][DESC_INTS]
    int n, T, L, H, rel_offset, n_rel;
    float scale;
};
int launch_relpos_ring(const RingArgs& a, bool bf16_data, hipStream_t st);

// ---------------------------------------------------------------- GEMM  C = epi(A . W^T)
enum Epi : int {
    EPI_STORE = 0,     // C[m,n] = act(acc)                        (C in the activation dtype)
    EPI_RESID = 1,     // C[m,n] += out_scale * acc                (C fp32 residual, in place)
    EPI_GLU = 2,       // C[m,c] = value * sigmoid(gate), rows >= valid zeroed   (C fp32 [M, N/2])
    EPI_STORE_F32 = 3  // C[m,n] = act(acc) as fp32
};
struct GemmArgs {
    const void* A; const void* W; void* C;
    int M, N, K, lda, ldw, ldc;
    int epi, act;
    float out_scale;
    const int32_t* desc;            // EPI_GLU: per-stream valid frames (desc[s*4+2]), rows = s*T+t
    int T;
};
int launch_gemm(const GemmArgs& a, bool bf16_data, hipStream_t st);

// ---------------------------------------------------------------- LayerNorm / conv / misc
// z = act(LN(x; g, b)) for rows of D (fp32 in), out in fp32 or bf16.
int launch_layernorm(const float* x, const float* g, const float* b, void* out, bool out_bf16, int rows, int D,
                     int act, hipStream_t st);
// res <- LN_a(src) (or a plain copy of src when ga == nullptr); z <- LN_b(res) in fp32/bf16.
int launch_layernorm2(const float* src, float* res, const float* ga, const float* ba, const float* gb,
                      const float* bb, void* z, bool z_bf16, int rows, int D, hipStream_t st);
// GLU of an unpermuted [M, 2D] fp32 buffer with rows >= valid zeroed (fp32 encoder mode).
int launch_glu_mask(const float* pw, float* g, int M, int D, const int32_t* desc, int T, hipStream_t st);
// Causal depthwise conv over [conv ring (K-1 rows) ; T new rows of g] + conv LayerNorm + SiLU;
// writes z and the updated conv ring.
struct ConvArgs {
    const float* g;                 // [n*T, D] GLU output
    float* ring;                    // layer base of the conv pool: [slots][K-1][D]
    const float* w_t;               // [K][D] depthwise weights, tap-major
    const float* ln_g; const float* ln_b;
    void* z;                        // [n*T, D]
    const int32_t* desc;
    int n, T, D, K;
    bool z_bf16;
};
int launch_dwconv_ln(const ConvArgs& a, hipStream_t st);

}  // namespace ud
