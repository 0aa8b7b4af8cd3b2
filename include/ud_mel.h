/*
 * ud_mel.h -- NeMo log-mel frontend on the GPU.
 *
 * Replaces NemoMelFrontend (Sources/DictatorCore/Audio/NemoMel.swift:11-108): preemphasis 0.97
 * (first sample kept), centred STFT (n_fft 512, hop 160, the 400-sample window zero-padded to 512,
 * constant zero padding of 256 on both sides), power |X|^2, the checkpoint's mel filterbank,
 * log(x + 2^-24), the frame at samples/160 (the extra final frame) zeroed.  The DFT is a product
 * with window-folded cos/sin tables built as the reference builds them (NemoMel.swift:27-39).
 * The streaming form (NemoMelStream, NemoMel.swift:113-161) is part of ud_streamer (ud_streamer.h),
 * which computes each chunk's frames from the stream's samples.
 *
 * Conventions as in ud_encoder.h (0 or a negative ud_status, ud_last_error()).
 */
#ifndef UD_MEL_H
#define UD_MEL_H

#include <stdint.h>

#include "ud_encoder.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ud_mel ud_mel;

/* fb_host [n_mels, 257] (preprocessor.featurizer.fb), window_host [400]
 * (preprocessor.featurizer.window); 1 <= n_mels <= 256.  Builds the device tables.  Synchronous. */
UD_API int ud_mel_create(const float* fb_host, int32_t n_mels, const float* window_host, ud_mel** out);
UD_API void ud_mel_destroy(ud_mel* m);
/* Number of mel bins (NemoMelFrontend.nMels). */
UD_API int32_t ud_mel_bins(const ud_mel* m);

/* NemoMelFrontend.features for n clips at once.
 *   audio_dev       fp32 samples; clip b is audio_dev[b * audio_stride + i], i < n_samples_host[b]
 *   n_samples_host  [n] clip lengths (0 <= n_b <= audio_stride)
 *   out_dev         fp32 [n, out_rows, n_mels]: clip b's frames 0 .. n_b / 160 (n_b / 160 + 1
 *                   frames, time-major, the last one zero); rows past them are left untouched
 *   frames_host     (may be NULL) receives [n] frame counts; each must be <= out_rows
 * Asynchronous on hip_stream. */
UD_API int ud_mel_features(ud_mel* m, int32_t n, const float* audio_dev, int64_t audio_stride,
                           const int64_t* n_samples_host, float* out_dev, int32_t out_rows, int32_t* frames_host,
                           void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif
