/*
 * ud_encoder.h -- C ABI of the MI355X (gfx950) cache-aware streaming FastConformer encoder step.
 *
 * This is the drop-in boundary for DictatorEngine's encoder step.  Each entry point names the
 * reference interface it replaces (paths relative to the reference repository root).
 *
 * Conventions (all entry points):
 *  - Return UD_OK (0) or a negative ud_status.  Nothing throws or aborts across the ABI; the
 *    message of the last failure on the calling thread is available from ud_last_error().
 *    (Reference: Swift `throws EngineError.io`, Sources/DictatorCore/Errors.swift:3-11; GPU faults
 *    `fatalError`, Sources/DictatorEngine/Core/Kernels.swift:40; shape misuse `precondition`,
 *    Sources/DictatorEngine/Models/FastConformer.swift:450.)
 *  - Pointers named *_dev are device (HBM) pointers; *_host are host pointers.  Caller buffers are
 *    borrowed for the duration of the call only.
 *  - `hip_stream` is a hipStream_t (NULL = the null stream).  Device work is enqueued on it and
 *    the call returns without waiting, except where a function says it synchronizes.
 *  - One encoder may be stepped by one thread at a time; distinct encoders are independent.
 *  - The device work of one encoder's calls runs in call order whatever HIP streams the calls are
 *    given: a call on a different stream than the encoder's previous call first makes its stream
 *    wait for that call's work (the calls share the encoder's workspace).
 */
#ifndef UD_ENCODER_H
#define UD_ENCODER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UD_API __attribute__((visibility("default")))

typedef enum {
    UD_OK = 0,
    UD_ERR_INVALID = -1,      /* null handle / bad argument */
    UD_ERR_SHAPE = -2,        /* size outside what the encoder or kernel supports */
    UD_ERR_NOMEM = -3,        /* device or host allocation failed */
    UD_ERR_HIP = -4,          /* a HIP runtime call failed */
    UD_ERR_STATE = -5,        /* call order violated (e.g. step before finalize) */
    UD_ERR_WEIGHT = -6,       /* unknown weight name or wrong element count */
    UD_ERR_CAPACITY = -7      /* stream pool exhausted */
} ud_status;

typedef enum {
    UD_F32 = 0,               /* fp32 weights, activations, caches */
    UD_BF16 = 1,              /* encoder, 16-bit: bf16-valued linear weights (each rounded to bf16,
                                 RNE, Tensor.swift:116-122 -- the bf16-weight setting) held as IEEE
                                 half (exactly, for |w| >= 2^-17) and multiplied on the f16 MFMA.
                                 What runs in 16 bits is IEEE half, not bfloat16: activations
                                 (GEMM inputs, FF hidden, q/k/v, attention output), K/V caches and
                                 position tables; fp32 accumulation, residual stream, norms,
                                 pos_bias, depthwise conv and conv cache.  Half's 11-bit significand
                                 (bf16: 8) keeps a 24-layer step within 2e-2 of the fp32-activation
                                 reference at 14-frame chunks, where bf16 activations exceed it.
                                 Range: every 16-bit store saturates at +-65504 (NaN stays NaN), so
                                 an activation past half's range is clipped, not turned into inf; a
                                 weight past it is refused (UD_ERR_WEIGHT).
                                 Front-end: conv.3 / conv.6 / out weights are rounded fp32 -> half
                                 and run on the f16 MFMA with half activations; conv.0 / 2 / 5 stay
                                 fp32.  (The reference's f16 checkpoint keeps every
                                 encoder.pre_encode.conv.* fp32, Convert.swift:80; the half
                                 conv.3 / conv.6 are a measured deviation.)
                                 Single-op attention entries: bfloat16 operands. */
    UD_F16 = 2                /* encoder: as UD_BF16 but the linear weights are rounded fp32 -> half
                                 directly, the reference's f16 checkpoint
                                 (WeightConverter.convert(.f16), Convert.swift:76-112: the
                                 precision of its published step times); the same kernels.
                                 Decode entry points: IEEE half K/V pages, the decoder K/V cache
                                 format of the reference (Sources/DictatorEngine/Core/Ops.swift:147). */
} ud_dtype;

/* FastConformerConfig (Sources/DictatorEngine/Models/FastConformer.swift:5-38) plus the streaming
 * geometry of StreamState (FastConformer.swift:406-435) and a stream pool capacity. */
typedef struct {
    int32_t layers;           /* 24 */
    int32_t d_model;          /* 1024 */
    int32_t heads;            /* 8 (head_dim = d_model / heads must be 128) */
    int32_t ff_dim;           /* 4096 */
    int32_t conv_kernel;      /* 9 (causal depthwise conv) */
    int32_t left_context;     /* L = 70 cached frames */
    int32_t max_chunk;        /* largest T per step (position tables cover -(T-1)..L+T-1) */
    int32_t max_streams;      /* stream pool capacity of this encoder; max_streams * max_chunk
                                 <= 1,048,576 step rows */
    int32_t dtype;            /* ud_dtype */
} ud_encoder_config;

typedef struct ud_encoder ud_encoder;
typedef struct ud_stream ud_stream;

/* Human-readable message of the last failure on this thread ("" if none). */
UD_API const char* ud_last_error(void);

/* ---------------------------------------------------------------- encoder lifetime */

/* Replaces FastConformerEncoder.init (FastConformer.swift:72-144) and makeWorkspace (:211-213):
 * allocates device weights, the per-step workspace and the stream pool on the current device. */
UD_API int ud_encoder_create(const ud_encoder_config* cfg, ud_encoder** out);
UD_API void ud_encoder_destroy(ud_encoder* enc);
/* The configuration an encoder was created with (FastConformerEncoder.config, FastConformer.swift:62). */
UD_API int ud_encoder_get_config(const ud_encoder* enc, ud_encoder_config* out);

/* Replaces the per-tensor loads of FastConformer.swift:72-143.  `name` is a NeMo state_dict
 * name ("encoder.layers.{i}.feed_forward1.linear1.weight", ..., the 26 per-layer tensors of the
 * checkpoint's name map, and the 12 optional encoder.pre_encode.* subsampling tensors); `host`
 * holds `count` fp32 values in the checkpoint layout ([out, in] for linears, k=1 axes squeezed,
 * depthwise [D, 1, K], conv2d [256, 1, 3, 3]).  The values are converted to the
 * encoder's dtype on upload (UD_BF16: linear weights rounded to bf16, round-to-nearest-even,
 * Tensor.swift:116-122; UD_F16: rounded to half; both held as half, see ud_dtype).  Synchronous. */
UD_API int ud_encoder_set_weight(ud_encoder* enc, const char* name, const float* host, int64_t count);

/* Replaces preparePositionTables (FastConformer.swift:161-178) as called by makeStreamState
 * (:431-435): builds P_l = PE . W_pos,l^T over rel = -(max_chunk-1) .. L+max_chunk-1 for every
 * layer.  Every weight must have been set.  Synchronous. */
UD_API int ud_encoder_finalize(ud_encoder* enc);

/* ---------------------------------------------------------------- streams */

/* Replaces makeStreamState / StreamState (FastConformer.swift:406-435): takes one slot of the
 * encoder's stream pool (K/V ring caches [layers][heads][L + max_chunk][head_dim], frame f in row
 * f mod (L + max_chunk), and the conv ring [layers][K-1][d_model]), zero-initialised, cache_len 0.  Create and reset wait for all work
 * on the device (hipDeviceSynchronize) before clearing the slot, so a slot freed while a step
 * that used it was still running starts clean.  Destroy only returns the slot to the pool; it
 * does not wait. */
UD_API int ud_stream_create(ud_encoder* enc, ud_stream** out);
UD_API int ud_stream_reset(ud_stream* s);              /* zero caches, cache_len 0, steps 0 */
UD_API void ud_stream_destroy(ud_stream* s);
/* StreamState.cacheLen / .step (FastConformer.swift:413-414). */
UD_API int ud_stream_info(const ud_stream* s, int32_t* cache_len, int32_t* steps);

/* ---------------------------------------------------------------- the step */

/* Replaces encodeStreamStep (FastConformer.swift:441-480) from the kept subsampled rows on, for a
 * batch of independent streams (the reference runs one stream per NemotronEncoder.step,
 * Sources/DictatorCore/Nemotron/NemotronStreamer.swift:6-12).
 *   streams[n]     distinct streams of this encoder
 *   T              frames per stream this step (1 <= T <= max_chunk, T <= L)
 *   x_dev          fp32 [n, T, d_model] chunk input, stream-major
 *   valid_T_host   [n] valid frames per stream (clamped to [0, T]); frames >= valid are masked
 *                  as keys and their GLU rows are zeroed, but all T frames enter the caches and
 *                  cache_len advances by T (FastConformer.swift:449, 459-462, 302, 477)
 *   out_dev        fp32 [n, T, d_model] encoder output; may not alias x_dev
 * Each stream's caches advance in place (ring buffers).  Asynchronous on hip_stream. */
UD_API int ud_encoder_step(ud_encoder* enc, ud_stream* const* streams, int32_t n, int32_t T,
                           const float* x_dev, const int32_t* valid_T_host, float* out_dev,
                           void* hip_stream);

/* Replaces encodeSubsampling (FastConformer.swift:219-243) and the drop/validT rule of
 * encodeStreamStep (:444-453): NeMo's causal dw_striding 8x subsampling of a batch of mel chunks.
 *   n              streams (1 <= n <= max_streams); all chunks have mel_rows rows
 *   mel_rows       1 <= mel_rows <= 8 * max_chunk + 9 (the workspace's chunk length); longer
 *                  chunks return UD_ERR_SHAPE before anything is launched
 *   mel_dev        fp32 [n, mel_rows, 128] mel rows, pre-encode cache rows included
 *   valid_mel_host [n] real rows per chunk (NULL = all); rows beyond are masked as NeMo's
 *                  MaskedConvSequential does, and the valid length follows L -> L/2 + 1 per stage
 *   drop           leading subsampled frames to discard, >= 0 (2 after a stream's first step,
 *                  NemotronSchedule.swift dropExtra; 0 on the first)
 *   out_dev        fp32 [n, T, d_model] encoder input rows, T = mel_rows -> 3 x (L/2 + 1) - drop,
 *                  1 <= T <= max_chunk; feed it to ud_encoder_step
 *   T_out          (may be NULL) receives T;  valid_T_host (may be NULL) receives [n] valid frames,
 *                  clamp(valid_sub - drop, 0, T), the valid_T_host of ud_encoder_step
 * Weights: the 12 encoder.pre_encode.* tensors via ud_encoder_set_weight (checkpoint layout;
 * out.weight [d_model, 256*17] with NeMo's (channel, freq) column order).  The first call
 * allocates the front-end workspace.  Asynchronous on hip_stream. */
UD_API int ud_encoder_subsample(ud_encoder* enc, int32_t n, int32_t mel_rows, const float* mel_dev,
                                const int32_t* valid_mel_host, int32_t drop, float* out_dev, int32_t* T_out,
                                int32_t* valid_T_host, void* hip_stream);

/* Cache window of one stream and layer in logical (time) order, oldest row first, as fp32:
 * k/v [L, d_model], conv [K-1, d_model]; rows older than cache_len are whatever the pool holds
 * (zeros for a fresh stream).  This is the StreamState content after a step
 * (FastConformer.swift:469-472, the rows the next step reads).  Synchronous. */
UD_API int ud_stream_export_cache(const ud_stream* s, int32_t layer, float* k_host, float* v_host,
                                  float* conv_host, int32_t* cache_len);
/* Inverse of export: loads a logical window (converted to the cache dtype) and sets cache_len
 * (shared by all layers; the last import wins).  Synchronous. */
UD_API int ud_stream_import_cache(ud_stream* s, int32_t layer, const float* k_host, const float* v_host,
                                  const float* conv_host, int32_t cache_len);

/* ---------------------------------------------------------------- single ops (KATs, one 72-key window) */

/* Replaces Step.relPosAttention (Sources/DictatorEngine/Core/Ops.swift:80-90) and its kernel
 * (Sources/DictatorEngine/Metal/20_conformer.metal:140-220):
 *   score[i,j] = ((q_i+u_h).k_j + (q_i+v_h).P[(Tk-Tq+i)-j+rel_offset]) / sqrt(dk)
 * for j in [max(r_i.x,0), min(r_i.y,Tk)), softmax, . V; an empty range gives 0.
 *   q [Tq, H*dk], k/v [Tk, H*dk], P [n_rel, H*dk], u/v [H, dk] (fp32), ranges int32 [Tq, 2],
 *   out [Tq, H*dk]; all device pointers, dtype UD_F32 or UD_BF16 for q/k/v/P/out.
 * Supported: dk in {16, 32, 64, 128}, Tq <= 16; rows 16-byte aligned.  UD_BF16 here means
 * bfloat16 operands.
 * Rows referenced by a valid (i, j) pair must lie inside P (caller contract, as in the
 * reference).  Asynchronous on hip_stream. */
UD_API int ud_relpos_attention(int32_t dtype, const void* q_dev, const void* k_dev, const void* v_dev,
                               const void* p_dev, const float* u_dev, const float* vb_dev,
                               const int32_t* ranges_dev, void* out_dev, int32_t Tq, int32_t Tk,
                               int32_t H, int32_t dk, int32_t rel_offset, int32_t n_rel,
                               void* hip_stream);

/* Replaces Step.relPosAttention (Ops.swift:80-90) on the offline path, forwardOffline
 * (Sources/DictatorEngine/Models/FastConformer.swift:361-398): whole utterances, every frame a
 * query over the same frames as keys (Tq = Tk = T), key ranges per query (chunked masks clipped to
 * the valid length, or plain key padding), for a batch of B utterances:
 *   q/k/v/out  bf16 [B, T, H*128]   P bf16 [n_rel, H*128] (rel -(T-1)..T-1 at rel_offset = T-1)
 *   u/v        fp32 [H, 128]        ranges int32 [B, T, 2]
 * Same formula and empty-range rule as ud_relpos_attention.  bf16 and head_dim 128 only.
 * Asynchronous on hip_stream. */
UD_API int ud_relpos_attention_batched(int32_t dtype, const void* q, const void* k, const void* v, const void* p,
                                       const float* u, const float* vb, const int32_t* ranges, void* out,
                                       int32_t B, int32_t T, int32_t H, int32_t dk, int32_t rel_offset,
                                       int32_t n_rel, void* hip_stream);

/* Key ranges of the offline path's streaming masks: replaces MaskSpec.ranges(T:) and
 * chunkedLimitedRanges (Sources/DictatorEngine/Models/FastConformer.swift:324-357) together with
 * forwardOffline's clip of each range's end to the valid length (:380-381), for B utterances of T
 * frames, giving the ranges argument of ud_relpos_attention_batched:
 *   UD_MASK_CHUNKED_LIMITED     NeMo chunked_limited [left, right] (chunk ignored): chunks of
 *                               right+1 frames aligned at frame 0, left/(right+1) chunks back;
 *                               query i sees [(c - left/(right+1)) (right+1), (c+1)(right+1)) with
 *                               c = i / (right+1), clipped to [0, T)
 *   UD_MASK_CHUNKED_LIMITED_RC  NeMo chunked_limited_with_rc [left, chunk, right]: query i sees
 *                               [c chunk - left, c chunk + chunk + right) with c = i / chunk
 *   valid_host    [B] valid frames per utterance (NULL = T); every range's end is clipped to it
 *                 (its start is not, so a chunk past the valid length is an empty range)
 *   ranges_host   int32 [B, T, 2], written
 * Host computation only (no device work). */
typedef enum { UD_MASK_CHUNKED_LIMITED = 0, UD_MASK_CHUNKED_LIMITED_RC = 1 } ud_mask_kind;
UD_API int ud_chunked_limited_ranges(int32_t kind, int32_t B, int32_t T, const int32_t* valid_host, int32_t left,
                                     int32_t chunk, int32_t right, int32_t* ranges_host);

/* The streaming attention of one layer on its own, over the stream's ring caches: the fused
 * kernel the step runs between the QKV projection and linear_out (FastConformer.swift:285-291 with
 * the cache rule of :458-472).
 *   qkv_dev  [n, T, 3*d_model]: q | k_new | v_new per row; fp32, or IEEE half for a 16-bit
 *            (UD_BF16) encoder
 *   att_dev  [n, T, d_model], row-major, in the same format as qkv_dev
 * Keys are [L cached ; T new], range [L - cache_len, L + valid).  The T new K/V rows are first
 * copied from qkv_dev into the rings, next to the cached ones (the step's QKV projection writes
 * them there directly), then the attention reads the window from the rings.  Does not advance
 * cache_len or the ring position (a repeated call rewrites the same rows): call
 * ud_stream_advance to commit the step (ud_encoder_step does both).  Asynchronous on hip_stream. */
UD_API int ud_layer_attention(ud_encoder* enc, ud_stream* const* streams, int32_t n, int32_t T,
                              int32_t layer, const void* qkv_dev, const int32_t* valid_T_host,
                              void* att_dev, void* hip_stream);

/* Advances cache_len = min(cache_len + T, L), the ring positions and the step counter of each
 * stream (FastConformer.swift:476-478).  Host-side bookkeeping only. */
UD_API int ud_stream_advance(ud_stream* const* streams, int32_t n, int32_t T);

/* Profiling hook (no reference counterpart; the reference times whole command buffers,
 * Sources/DictatorEngine/Core/Kernels.swift:33-42): uploads the batch descriptor once, then
 * launches the fused attention kernel `iters` times back to back between two HIP events on
 * hip_stream -- launch i on layer (layer + 1 + i) % layers, so that, as in a real step, the ring
 * caches stream from HBM -- and returns the average kernel duration in milliseconds.  Only the
 * attention kernel is timed: it reads q from qkv_dev and the window from the rings (whatever the
 * new rows' ring rows hold) and writes att_dev, nothing else.  Synchronizes hip_stream. */
UD_API int ud_time_layer_attention(ud_encoder* enc, ud_stream* const* streams, int32_t n, int32_t T,
                                   int32_t layer, const void* qkv_dev, void* att_dev, int32_t iters,
                                   void* hip_stream, float* avg_ms);

/* Profiling hook (no reference counterpart): like ud_time_layer_attention, but each launch is a
 * kernel that performs only the loads of the bf16 streaming attention kernel (same grid, same
 * addresses, no arithmetic and no stores to the rings) -- the memory floor that kernel is measured
 * against.  16-bit encoders, T <= 2, L + T <= 80.  att_dev may be written with garbage.  Synchronizes
 * hip_stream. */
UD_API int ud_time_ring_read_floor(ud_encoder* enc, ud_stream* const* streams, int32_t n, int32_t T,
                                   int32_t layer, const void* qkv_dev, void* att_dev, int32_t iters,
                                   void* hip_stream, float* avg_ms);

/* Profiling hook (no reference counterpart): times one of the step's projection GEMMs exactly as
 * the step launches it for `rows` rows (tile shape, epilogue, split-K, operand format), `iters`
 * launches back to back between two HIP events on hip_stream, launch i on layer (i + 1) % layers
 * so the weights stream from HBM.  Inputs are whatever the workspace holds; the workspace's
 * outputs are overwritten.  avg_ms receives the average launch duration, flops (may be NULL) the
 * 2 rows N K flops of one launch.  Synchronizes hip_stream. */
typedef enum {
    UD_PROJ_FF_LINEAR1 = 0,   /* feed_forward{1,2}.linear1: N ff_dim, K d_model, SiLU */
    UD_PROJ_FF_LINEAR2 = 1,   /* feed_forward{1,2}.linear2: N d_model, K ff_dim, x0.5, residual */
    UD_PROJ_QKV = 2,          /* linear_q | linear_k | linear_v: N 3 d_model, K d_model */
    UD_PROJ_LINEAR_OUT = 3,   /* linear_out: N d_model, K d_model, residual */
    UD_PROJ_PW1 = 4,          /* conv.pointwise_conv1: N 2 d_model, K d_model; fp32 value | gate out, or for
                                 a 16-bit encoder the GLU applied in the epilogue, half out */
    UD_PROJ_PW2 = 5           /* conv.pointwise_conv2: N d_model, K d_model, residual */
} ud_projection;
UD_API int ud_time_projection(ud_encoder* enc, int32_t which, int32_t rows, int32_t iters, void* hip_stream,
                              float* avg_ms, double* flops);

#ifdef __cplusplus
}
#endif

#endif /* UD_ENCODER_H */
