/*
 * tfq_runtime.h — device-memory, stream, event and graph plumbing exported
 * by libtfq so that hosts without a HIP toolchain of their own (the Swift
 * package, the Python tests and bench) can drive the kernels in tfq.h.
 *
 * These have no counterpart among the reference's quantized-matmul entry
 * points; they stand in for the Metal device/queue/buffer objects the
 * reference's wrappers receive. Thin wrappers over the HIP runtime: every
 * call returns TFQ_OK or TFQ_E_HIP (code kept for tfq_last_hip_error()).
 */
#ifndef TFQ_RUNTIME_H
#define TFQ_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int tfq_rt_device_count(int *count);
int tfq_rt_set_device(int device);
/* Writes the device name and gcnArchName ("gfx950:...") of the current device. */
int tfq_rt_device_info(char *name, size_t name_len, char *arch, size_t arch_len);

int tfq_rt_malloc(void **ptr, size_t bytes);
int tfq_rt_free(void *ptr);
int tfq_rt_memcpy_htod(void *dst, const void *src, size_t bytes);   /* synchronous */
int tfq_rt_memcpy_dtoh(void *dst, const void *src, size_t bytes);   /* synchronous */
int tfq_rt_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream);
int tfq_rt_memset(void *dst, int value, size_t bytes);             /* synchronous */

int tfq_rt_stream_create(void **stream);    /* default priority */
int tfq_rt_stream_destroy(void *stream);
int tfq_rt_stream_sync(void *stream);
int tfq_rt_device_sync(void);

int tfq_rt_event_create(void **event);
int tfq_rt_event_destroy(void *event);
int tfq_rt_event_record(void *event, void *stream);
int tfq_rt_event_sync(void *event);
int tfq_rt_event_elapsed_ms(float *ms, void *start, void *end);

/* Stream capture into a HIP graph: begin, enqueue work, end -> executable. */
int tfq_rt_capture_begin(void *stream);
int tfq_rt_capture_end(void *stream, void **graph_exec);
int tfq_rt_graph_launch(void *graph_exec, void *stream);
int tfq_rt_graph_destroy(void *graph_exec);

#ifdef __cplusplus
}
#endif
#endif /* TFQ_RUNTIME_H */
