/*
 * arclight_util.h - device plumbing for harnesses that drive the C ABI
 * without a framework: device memory, streams, events, graph capture and
 * seeded synthetic inputs. No counterpart in the reference (its tensors live
 * in host bump buffers, nnml/src/memory.cpp:402-446); these exist so tests and
 * benchmarks can place operands in HBM and time kernels on their own stream.
 * All functions return AL_OK or a negative al status (al_last_error()).
 */
#ifndef ARCLIGHT_UTIL_H
#define ARCLIGHT_UTIL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int al_util_device_count(int * n);
int al_util_set_device(int dev);
/* name, compute units, HBM bytes, gcnArchName into caller buffers */
int al_util_device_info(char * name, size_t name_len, int * n_cu, uint64_t * hbm_bytes,
                        char * arch, size_t arch_len);

int al_util_malloc(void ** ptr, uint64_t bytes);
int al_util_free(void * ptr);
int al_util_memcpy_h2d(void * dst, const void * src, uint64_t bytes);
int al_util_memcpy_d2h(void * dst, const void * src, uint64_t bytes);
int al_util_memcpy_d2d(void * dst, const void * src, uint64_t bytes, void * stream);
int al_util_memset(void * ptr, int value, uint64_t bytes);
int al_util_device_synchronize(void);

int al_util_stream_create(void ** stream);
int al_util_stream_destroy(void * stream);
int al_util_stream_synchronize(void * stream);

int al_util_event_create(void ** event);
int al_util_event_destroy(void * event);
int al_util_event_record(void * event, void * stream);
int al_util_event_synchronize(void * event);
int al_util_event_elapsed_ms(void * start, void * stop, float * ms);

/* Stream capture into a HIP graph, instantiation and replay. */
int al_util_graph_begin(void * stream);
int al_util_graph_end(void * stream, void ** graph_exec);
int al_util_graph_launch(void * graph_exec, void * stream);
int al_util_graph_destroy(void * graph_exec);

/*
 * Seeded ~N(0,1) fill: element i gets a Box-Muller normal from a
 * counter-based hash of (seed, offset + i), then rounding to f16 (RNE) for
 * the f16 variant. Deterministic for a given (seed, offset) on any device.
 */
int al_util_fill_randn_f32(float * dst, uint64_t n, uint64_t seed, uint64_t offset, void * stream);
int al_util_fill_randn_f16(uint16_t * dst, uint64_t n, uint64_t seed, uint64_t offset, void * stream);

/* dst[i] = f16(src[i]) with IEEE round-to-nearest-even (the Q -> f16 and
 * KV-write rounding of the reference, nnml/include/ops.h:299-323). */
int al_util_f32_to_f16(uint16_t * dst, const float * src, uint64_t n, void * stream);

/* Plain device copy by a 16-byte vector kernel (bytes and both pointers
 * 16-byte aligned): a kernel of known traffic, 2 * bytes, that calibrates
 * hardware byte counters. */
int al_util_copy_kernel(void * dst, const void * src, uint64_t bytes, void * stream);

/* One launch of a kernel that does nothing, with `grid` workgroups of `block`
 * threads and `lds_bytes` of dynamic LDS (at most 160 KiB): graphs of such
 * launches measure the dispatch floor of a grid shape and a tracer's
 * per-dispatch overhead. */
int al_util_empty_launch(int grid, int block, int lds_bytes, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* ARCLIGHT_UTIL_H */
