/*
 * ud_streamer.h -- cache-aware streaming transcription of many streams at once.
 *
 * Replaces NemotronStreamer (Sources/DictatorCore/Nemotron/NemotronStreamer.swift:16-153) with
 * the schedule of NemotronSchedule (Sources/DictatorCore/Nemotron/NemotronSchedule.swift:7-17)
 * and the encoder step of MetalNemotronEncoder.step (Sources/DictatorEngine/Models/Nemotron.swift:
 * 74-92).  The reference runs one streamer per stream, one chunk at a time.  Here every open
 * stream of the streamer that has a chunk ready joins ONE batched step:
 *
 *   mel frames (live input: ud_mel from the stream's samples; buffered input: the caller's rows)
 *   -> ud_encoder_subsample twice at most (streams at their first chunk: 1 + 8 lookahead rows,
 *      drop 0; the others: 9 pre-encode cache rows + 8 + 8 lookahead rows, drop 2; both give
 *      T = lookahead + 1 frames) -> one ud_encoder_step -> ud_rnnt_project -> ud_rnnt_greedy.
 *
 * A final chunk shorter than the schedule's is zero-extended to the full chunk and its real rows
 * passed as the valid count: the subsampling convolutions are causal and mask rows past the
 * valid count, and the step masks frames past valid_T as keys, so the kept frames equal the
 * reference's unpadded final step (the extra frames are computed and discarded; only the caches,
 * which a final chunk leaves unused, differ).  Kept frames per chunk: valid_T (the reference's
 * keepAll ? validT : min(validT, lookahead + 1), which equals valid_T here).
 *
 * Live input (push / flush) follows drainChunks (NemotronStreamer.swift:109-153): a chunk runs once
 * its mel frames are complete (frame f needs samples up to 160 f + 199); flush runs the remainder,
 * padding a final chunk shorter than 8 frames when end padding is on (the default) and dropping
 * it when off (NeMo's batch-1 schedule).  Buffered input (run_buffered) follows runBuffered
 * (:70-91) over full-utterance mel rows.  Each mel frame of a live stream is computed from the
 * stream's samples by ud_mel (the 9 pre-encode cache rows of a chunk are recomputed from samples,
 * bit-identical to their first computation), so no mel state is kept on the device.
 *
 * The streamer owns one encoder stream (ud_stream) and one RNN-T slot per open stream; stream ids
 * are the slot numbers 0 .. max_streams-1.  Calls are synchronous (each batched step ends with
 * the greedy decoder's readback) and not thread-safe; one streamer at a time may drive a given
 * encoder and decoder.  If a batched step fails, the call returns its error and the streams of
 * that batch take no further chunks (their tokens so far stay readable); close and reopen them.
 *
 * Conventions as in ud_encoder.h (0 or a negative ud_status, ud_last_error()).
 */
#ifndef UD_STREAMER_H
#define UD_STREAMER_H

#include <stdint.h>

#include "ud_encoder.h"
#include "ud_mel.h"
#include "ud_rnnt.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ud_streamer ud_streamer;

/* enc: finalized, with subsampling weights; its max_chunk >= lookahead + 1 and max_streams >=
 * max_streams.  rnnt: weights set, enc_dim = d_model, max_streams >= max_streams.  mel: the
 * frontend for live input (may be NULL: buffered input only).  lookahead >= 0 (NeMo's right
 * context: 1 = 160 ms chunks, 6 = 560 ms, 13 = 1120 ms). */
UD_API int ud_streamer_create(ud_encoder* enc, ud_rnnt* rnnt, ud_mel* mel, int32_t lookahead, int32_t max_streams,
                              ud_streamer** out);
UD_API void ud_streamer_destroy(ud_streamer* s);

/* Opens a stream (fresh encoder caches, decoder initial state); *id receives its id. */
UD_API int ud_streamer_open(ud_streamer* s, int32_t* id);
UD_API int ud_streamer_close(ud_streamer* s, int32_t id);

/* end_padding (NemotronStreamer.endPadding, default 1); record = 1 keeps every stream's kept
 * encoder output rows and joint.enc rows for ud_streamer_recorded (parity checks; default 0). */
UD_API int ud_streamer_set_options(ud_streamer* s, int32_t end_padding, int32_t record);

/* Appends samples_host[b][0 .. counts[b]) (16 kHz mono fp32) to stream ids[b], then runs batched
 * steps until no open stream has a complete chunk. */
UD_API int ud_streamer_push(ud_streamer* s, int32_t n, const int32_t* ids, const float* const* samples_host,
                            const int64_t* counts);
/* Ends streams ids[0 .. n) (NemotronStreamer.flush): their remaining frames run as final chunks. */
UD_API int ud_streamer_flush(ud_streamer* s, int32_t n, const int32_t* ids);

/* runBuffered for streams ids[0 .. n) at once: mel_host[b] fp32 [frames[b], n_mels] full-utterance
 * features, valid_frames[b] NeMo's processed length.  The streams must be fresh (just opened). */
UD_API int ud_streamer_run_buffered(ud_streamer* s, int32_t n, const int32_t* ids, const float* const* mel_host,
                                    const int32_t* frames, const int32_t* valid_frames);

/* All tokens of a stream so far (the first cap of them); *count receives the total. */
UD_API int ud_streamer_tokens(const ud_streamer* s, int32_t id, int32_t* out, int32_t cap, int32_t* count);
/* Recorded rows (record = 1): which = 0 encoder output [rows, d_model], 1 joint.enc [rows, hidden];
 * the first cap_rows rows are written; *rows receives the total. */
UD_API int ud_streamer_recorded(const ud_streamer* s, int32_t id, int32_t which, float* out, int64_t cap_rows,
                                int64_t* rows);
/* Emission records of a live stream (NemotronStreamer's emissions, NemotronStreamer.swift:145,
 * 158; Emission, Sources/DictatorCore/Nemotron/Streaming.swift:6-13): for each token emitted by
 * ud_streamer_push or ud_streamer_flush, in order, the token, the samples pushed to the stream when
 * its chunk ran (samplesSeen: / 16000 is the token's algorithmic emission time) and the wall
 * seconds of the batched step that ran the chunk (computeSeconds).  Buffered input records none,
 * as the reference's runBuffered.  Any of tokens / samples_seen / compute_seconds may be NULL; the
 * first cap records are written; *count receives the total. */
UD_API int ud_streamer_emissions(const ud_streamer* s, int32_t id, int32_t* tokens, int64_t* samples_seen,
                                 double* compute_seconds, int32_t cap, int32_t* count);
/* Wall seconds of each chunk of the stream (NemotronStreamer.wallTimes / stepWallTimes,
 * NemotronStreamer.swift:24, 63, 159): the batched step that ran it, from its mel frames to its
 * tokens (shared by the streams of that step).  The first cap go to out; *count receives the total. */
UD_API int ud_streamer_step_times(const ud_streamer* s, int32_t id, double* out, int32_t cap, int32_t* count);
/* Batched steps run and stream chunks processed since creation. */
UD_API int ud_streamer_stats(const ud_streamer* s, int64_t* batches, int64_t* chunks);

/* Replaces NemotronEncoder.step(mel:nRows:validRows:keepAll:) -> (proj, frames)
 * (Sources/DictatorCore/Nemotron/NemotronStreamer.swift:6-12; the GPU body
 * MetalNemotronEncoder.step, Sources/DictatorEngine/Models/Nemotron.swift:74-91) for n streams in
 * one call, without the streamer's scheduling:
 *   mel_dev          fp32 [n, mel_rows, 128]: each stream's chunk rows, pre-encode cache rows included
 *   valid_rows_host  [n] real rows of each chunk (validRows)
 *   keep_all_host    [n] nonzero for a final chunk (keepAll); NULL = none
 *   drop_extra       frames dropped after subsampling on every step but a stream's first
 *                    (NemotronSchedule.dropExtra; a first step drops 0)
 *   out_frames       kept frames per chunk unless keep_all (NemotronSchedule.outFramesPerChunk)
 *   proj_dev         fp32 [n, proj_rows, hidden]: stream i's kept joint.enc rows at row 0 on
 *   frames_host      [n] kept frames: keep_all ? valid_T : min(valid_T, out_frames)
 * Streams at their first step and the others run as two groups (a subsample, an encoder step and
 * a projection each), so the call may mix them.  The encoder and decoder are used as by
 * ud_encoder_subsample / ud_encoder_step / ud_rnnt_project, with scratch owned by the encoder
 * (calls on one encoder must not overlap).  Asynchronous on hip_stream (frames_host is written
 * before the call returns).
 * Errors: every argument and shape check of both groups comes before anything is launched, so such
 * an error leaves every stream unchanged.  A HIP or allocation failure inside the second group's
 * calls (later steps) comes after the first group's streams (first steps) have advanced and their
 * frames_host entries have been written; after any error other than a shape or argument error the
 * caller should reset the call's streams. */
UD_API int ud_nemotron_step(ud_encoder* enc, ud_rnnt* rnnt, ud_stream* const* streams, int32_t n, int32_t mel_rows,
                            const float* mel_dev, const int32_t* valid_rows_host, const int32_t* keep_all_host,
                            int32_t drop_extra, int32_t out_frames, float* proj_dev, int32_t proj_rows,
                            int32_t* frames_host, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif
