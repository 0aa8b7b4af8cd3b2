/*
 * ud_rnnt.h -- C ABI of the RNN-T joint and greedy decoder on MI355X (gfx950), batched over streams.
 *
 * Replaces the joint-encoder projection of MetalNemotronEncoder.step
 * (Sources/DictatorEngine/Models/Nemotron.swift:82-90) and RNNTDecoder
 * (Sources/DictatorCore/Decoding/RNNT.swift:1-151), which the reference runs on the CPU one
 * stream at a time.  Here each greedy iteration evaluates the prediction network (embedding,
 * stacked LSTM, joint.pred) and the joint (joint_net.2 over relu(f + g)) for every active stream
 * as one batch of fp32 GEMMs (the reference keeps decoder.* and joint.* other than joint.enc in
 * fp32, Sources/DictatorEngine/Core/Convert.swift:74-83); the greedy control (blank, max symbols
 * per frame, the cached prediction of RNNT.swift:18-26) runs on the host.
 *
 * Conventions as in ud_encoder.h: 0 or a negative ud_status, ud_last_error() for the message,
 * *_dev device pointers, *_host host pointers.  The calls on one decoder share its workspaces and
 * run in call order whatever HIP streams they are issued on: a call on a stream other than the
 * previous call's first makes its stream wait for the previous call's work.
 */
#ifndef UD_RNNT_H
#define UD_RNNT_H

#include <stdint.h>

#include "ud_encoder.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ud_rnnt ud_rnnt;

/* RNNTDecoder.init (RNNT.swift:27-63): hidden 640, vocab 1025 (blank = vocab - 1), 2 LSTM layers,
 * enc_dim 1024 (joint.enc input), max_symbols_per_frame 10; decoder states for `max_streams`
 * stream slots, all in RNNTDecoder.initialState() (RNNT.swift:66-70).  hidden must be a multiple of
 * 64 and enc_dim of 16 (the GEMM tiles), else UD_ERR_SHAPE. */
UD_API int ud_rnnt_create(int32_t hidden, int32_t vocab, int32_t layers, int32_t enc_dim, int32_t max_streams,
                          int32_t max_symbols_per_frame, ud_rnnt** out);
UD_API void ud_rnnt_destroy(ud_rnnt* r);

/* Dimensions the decoder was created with (any pointer may be NULL). */
UD_API int ud_rnnt_get_info(const ud_rnnt* r, int32_t* hidden, int32_t* vocab, int32_t* layers, int32_t* enc_dim,
                            int32_t* max_streams, int32_t* max_symbols_per_frame);

/* Checkpoint tensors by NeMo name, fp32 host values in the checkpoint layout:
 * decoder.prediction.embed.weight [V, H]; decoder.prediction.dec_rnn.lstm.{weight_ih,weight_hh}_l{l}
 * [4H, H] and {bias_ih,bias_hh}_l{l} [4H] (gate order i, f, g, o); joint.pred.{weight,bias};
 * joint.enc.{weight,bias} ([H, enc_dim], [H]); joint.joint_net.2.{weight,bias} ([V, H], [V]).
 * Synchronous. */
UD_API int ud_rnnt_set_weight(ud_rnnt* r, const char* name, const float* host, int64_t count);

/* RNNTDecoder.initialState for one stream slot: h = c = 0, last token = blank, no cached
 * prediction.  Synchronous. */
UD_API int ud_rnnt_reset(ud_rnnt* r, int32_t slot);

/* The joint's encoder projection (Nemotron.swift:82-90; NeMo joint.enc): out [rows, hidden] =
 * enc [rows, enc_dim] . W_enc^T + b_enc, fp32.  Asynchronous on hip_stream. */
UD_API int ud_rnnt_project(ud_rnnt* r, int32_t rows, const float* enc_dev, float* out_dev, void* hip_stream);

/* RNNTDecoder.greedy (RNNT.swift:125-151) for n streams at once.
 *   slots_host[n]     distinct stream slots; their states advance
 *   proj_dev          fp32 projected frames: stream b's frame t is row b * rows_per_stream + t
 *   frames_host[n]    frames to decode per stream (<= rows_per_stream)
 *   tokens_host       [n][cap] emitted token ids (the first cap per stream)
 *   n_tokens_host[n]  tokens emitted per stream this call (may exceed cap)
 * Synchronizes hip_stream (the greedy control reads each iteration's argmax). */
UD_API int ud_rnnt_greedy(ud_rnnt* r, int32_t n, const int32_t* slots_host, const float* proj_dev,
                          int32_t rows_per_stream, const int32_t* frames_host, int32_t* tokens_host, int32_t cap,
                          int32_t* n_tokens_host, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif
