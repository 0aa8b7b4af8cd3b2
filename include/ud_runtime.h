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

/* Free and total device memory of the current device (hipMemGetInfo). */
UD_API int ud_mem_get_info(size_t* free_bytes, size_t* total_bytes);

/* Stream capture into a HIP graph, for callers that replay library calls (e.g. the allocation-free
 * decode entry point): begin capturing `stream` (not the null stream; thread-local capture mode),
 * end it and instantiate the graph (*graph receives an owned handle), launch it on a stream,
 * destroy it.  Work enqueued on the stream between begin and end is recorded, not run. */
UD_API int ud_graph_capture_begin(void* stream);
UD_API int ud_graph_capture_end(void* stream, void** graph);
UD_API int ud_graph_launch(void* graph, void* stream);
UD_API int ud_graph_destroy(void* graph);

/* Measured peaks of the current device, the denominators of measured roofline fractions.  No
 * reference counterpart beyond the same idea: the reference quotes its M3 roofline from its own
 * micro-benchmarks (docs/PERF_LOG.md:7-16: read GB/s, GEMM TFLOPS).
 *   ud_measure_hbm   streams a `bytes` buffer (>= 64 MiB; use >> the 256 MB last-level cache)
 *                    `iters` times: read_gbs = bytes read per second by a read-only kernel;
 *                    copy_gbs = bytes read + written per second by a device-to-device copy kernel.
 *                    Allocates (and frees) two buffers of `bytes`.
 *   ud_measure_mfma  dense v_mfma_f32_32x32x16 throughput in TFLOP/s, f16 and bf16 operands,
 *                    register-only chains on every SIMD, `iters` loop trips per wave.
 * Both synchronize hip_stream. */
UD_API int ud_measure_hbm(size_t bytes, int32_t iters, void* hip_stream, float* read_gbs, float* copy_gbs);
UD_API int ud_measure_mfma(int32_t iters, void* hip_stream, float* f16_tflops, float* bf16_tflops);

#ifdef __cplusplus
}
#endif

#endif /* UD_RUNTIME_H */
