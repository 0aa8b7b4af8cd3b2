/*
 * ud_safetensors.h -- weight ingestion: safetensors files and the NeMo tensor-name map.
 *
 * Replaces SafeTensorsHeader / SafeTensorsReader / widenToFloats
 * (Sources/DictatorCore/Weights/WeightSource.swift:13-90), the memory-mapped SafeTensorsFile
 * (Sources/DictatorEngine/Core/SafeTensors.swift:6-112) and the name handling of the model loaders
 * (docs/specs/nemotron.md:246-287: NeMo state_dict names, and the HF model.safetensors aliases).  The
 * file is memory-mapped read-only; tensors are widened to fp32 on request (F32, F16, BF16) and the
 * encoder / decoder convert them to their storage dtype on upload (the keep-fp32 policy of
 * Sources/DictatorEngine/Core/Convert.swift:74-83).  Host-only; no device work.
 *
 * Conventions as in ud_encoder.h (0 or a negative ud_status, ud_last_error()).
 */
#ifndef UD_SAFETENSORS_H
#define UD_SAFETENSORS_H

#include <stdint.h>

#include "ud_encoder.h"
#include "ud_mel.h"
#include "ud_rnnt.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ud_safetensors ud_safetensors;

typedef enum { UD_ST_F32 = 0, UD_ST_BF16 = 1, UD_ST_F16 = 2, UD_ST_OTHER = 3 } ud_st_dtype;

/* Maps `path` and parses its header (8-byte little-endian length, JSON).  Malformed headers,
 * offsets outside the file and byte ranges that do not match dtype x shape are UD_ERR_WEIGHT. */
UD_API int ud_safetensors_open(const char* path, ud_safetensors** out);
UD_API void ud_safetensors_close(ud_safetensors* st);
/* Tensors in the file (the __metadata__ entry excluded), in name order. */
UD_API int32_t ud_safetensors_count(const ud_safetensors* st);
UD_API const char* ud_safetensors_name(const ud_safetensors* st, int32_t i);
/* dtype (ud_st_dtype), shape (up to 8 dims) and rank of a tensor; UD_ERR_WEIGHT if absent. */
UD_API int ud_safetensors_info(const ud_safetensors* st, const char* name, int32_t* dtype, int64_t* shape,
                               int32_t* ndim);
/* The tensor widened to fp32 (WeightSource.floats); count must equal its element count. */
UD_API int ud_safetensors_read_f32(const ud_safetensors* st, const char* name, float* out, int64_t count);
/* The NeMo state_dict name of a tensor name: HF model.safetensors aliases are mapped
 * (docs/specs/nemotron.md:246-287), NeMo names are returned unchanged.  Writes at most cap bytes. */
UD_API int ud_nemo_name(const char* name, char* out, int32_t cap);

/* Sets every encoder tensor of the file (encoder.layers.{l}.* for l < the encoder's layer count,
 * encoder.pre_encode.*; NeMo or HF names) through ud_encoder_set_weight.  *n_loaded (may be NULL)
 * receives the number set.  Call ud_encoder_finalize afterwards. */
UD_API int ud_encoder_load_safetensors(ud_encoder* enc, const ud_safetensors* st, int32_t* n_loaded);
/* Sets every RNN-T tensor of the file (decoder.prediction.*, joint.*) through ud_rnnt_set_weight. */
UD_API int ud_rnnt_load_safetensors(ud_rnnt* r, const ud_safetensors* st, int32_t* n_loaded);
/* ud_mel_create from the file's preprocessor.featurizer.fb [1, n_mels, 257] and
 * preprocessor.featurizer.window [400] (NemotronModel.init, Sources/DictatorEngine/Models/
 * Nemotron.swift:45-46); UD_ERR_WEIGHT if either is missing (the HF model.safetensors has neither). */
UD_API int ud_mel_load_safetensors(const ud_safetensors* st, ud_mel** out);

#ifdef __cplusplus
}
#endif

#endif
