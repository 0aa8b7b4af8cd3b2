/*
 * ud_runtime.h -- device-memory, stream and timing helpers of the encoder library.
 *
 * The reference has no counterpart: Metal buffers are unified memory (storageModeShared,
 * Sources/DictatorEngine/Core/MetalContext.swift:73-78), filled with memcpy and read back with
 * Tensor.toFloats() (Sources/DictatorEngine/Core/Tensor.swift:75-90), and a step is timed by
 * MTLCommandBuffer gpuStartTime/gpuEndTime (Sources/DictatorEngine/Core/Kernels.swift:33-42).
 * On MI355X the host owns explicit HBM buffers; these helpers let a host binding (Swift, Python)
 * stage step inputs in HBM and time steps on a HIP stream without linking HIP itself.
 * Return codes and ud_last_error() as in ud_encoder.h.
 */
#ifndef UD_RUNTIME_H
#define UD_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef UD_API
#define UD_API __attribute__((visibility("default")))
#endif

UD_API int ud_device_count(int32_t* count);
/* Name of the current device's architecture (e.g. "gfx950") into buf. */
UD_API int ud_device_arch(char* buf, int32_t len);
UD_API int ud_malloc(void** dev, size_t bytes);
UD_API int ud_free(void* dev);
/* Synchronous copies (the device is synchronised first). */
UD_API int ud_memcpy_htod(void* dst_dev, const void* src_host, size_t bytes);
UD_API int ud_memcpy_dtoh(void* dst_host, const void* src_dev, size_t bytes);
UD_API int ud_memcpy_dtod(void* dst_dev, const void* src_dev, size_t bytes);
UD_API int ud_memset(void* dev, int32_t byte, size_t bytes);
UD_API int ud_device_synchronize(void);

/* HIP streams (default priority) and events for timing. */
UD_API int ud_hip_stream_create(void** stream);
UD_API int ud_hip_stream_destroy(void* stream);
UD_API int ud_hip_stream_synchronize(void* stream);
UD_API int ud_event_create(void** event);
UD_API int ud_event_destroy(void* event);
UD_API int ud_event_record(void* event, void* stream);
UD_API int ud_event_synchronize(void* event);
UD_API int ud_event_elapsed_ms(float* ms, void* start, void* stop);

#ifdef __cplusplus
}
#endif

#endif /* UD_RUNTIME_H */
