// Device plumbing for harnesses (include/arclight_util.h).
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/arclight_fattn.h"
#include "../../include/arclight_util.h"
#include "runtime.hpp"

#define AL_HIP(call, what)                                  \
    do {                                                    \
        const hipError_t e_ = (call);                       \
        if (e_ != hipSuccess) return al_hip_fail(e_, what); \
    } while (0)

extern "C" int al_util_device_count(int * n) { AL_HIP(hipGetDeviceCount(n), "hipGetDeviceCount"); return AL_OK; }
extern "C" int al_util_set_device(int dev) { AL_HIP(hipSetDevice(dev), "hipSetDevice"); return AL_OK; }

extern "C" int al_util_device_info(char * name, size_t name_len, int * n_cu, uint64_t * hbm_bytes, char * arch, size_t arch_len) {
    int dev = 0;
    AL_HIP(hipGetDevice(&dev), "hipGetDevice");
    hipDeviceProp_t prop;
    AL_HIP(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    if (name && name_len) { strncpy(name, prop.name, name_len - 1); name[name_len - 1] = 0; }
    if (arch && arch_len) { strncpy(arch, prop.gcnArchName, arch_len - 1); arch[arch_len - 1] = 0; }
    if (n_cu) *n_cu = prop.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
    return AL_OK;
}

extern "C" int al_util_malloc(void ** ptr, uint64_t bytes) { AL_HIP(hipMalloc(ptr, bytes), "hipMalloc"); return AL_OK; }
extern "C" int al_util_free(void * ptr) { AL_HIP(hipFree(ptr), "hipFree"); return AL_OK; }
extern "C" int al_util_memcpy_h2d(void * dst, const void * src, uint64_t bytes) {
    AL_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return AL_OK;
}
extern "C" int al_util_memcpy_d2h(void * dst, const void * src, uint64_t bytes) {
    AL_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return AL_OK;
}
extern "C" int al_util_memcpy_d2d(void * dst, const void * src, uint64_t bytes, void * stream) {
    AL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t) stream), "hipMemcpyAsync D2D");
    return AL_OK;
}
extern "C" int al_util_memset(void * ptr, int value, uint64_t bytes) { AL_HIP(hipMemset(ptr, value, bytes), "hipMemset"); return AL_OK; }
extern "C" int al_util_device_synchronize(void) { AL_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize"); return AL_OK; }

extern "C" int al_util_stream_create(void ** stream) {
    hipStream_t s;
    AL_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return AL_OK;
}
extern "C" int al_util_stream_destroy(void * stream) { AL_HIP(hipStreamDestroy((hipStream_t) stream), "hipStreamDestroy"); return AL_OK; }
extern "C" int al_util_stream_synchronize(void * stream) { AL_HIP(hipStreamSynchronize((hipStream_t) stream), "hipStreamSynchronize"); return AL_OK; }

extern "C" int al_util_event_create(void ** event) {
    hipEvent_t e;
    AL_HIP(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return AL_OK;
}
extern "C" int al_util_event_destroy(void * event) { AL_HIP(hipEventDestroy((hipEvent_t) event), "hipEventDestroy"); return AL_OK; }
extern "C" int al_util_event_record(void * event, void * stream) {
    AL_HIP(hipEventRecord((hipEvent_t) event, (hipStream_t) stream), "hipEventRecord");
    return AL_OK;
}
extern "C" int al_util_event_synchronize(void * event) { AL_HIP(hipEventSynchronize((hipEvent_t) event), "hipEventSynchronize"); return AL_OK; }
extern "C" int al_util_event_elapsed_ms(void * start, void * stop, float * ms) {
    AL_HIP(hipEventElapsedTime(ms, (hipEvent_t) start, (hipEvent_t) stop), "hipEventElapsedTime");
    return AL_OK;
}

extern "C" int al_util_graph_begin(void * stream) {
    AL_HIP(hipStreamBeginCapture((hipStream_t) stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return AL_OK;
}
extern "C" int al_util_graph_end(void * stream, void ** graph_exec) {
    hipGraph_t g;
    AL_HIP(hipStreamEndCapture((hipStream_t) stream, &g), "hipStreamEndCapture");
    hipGraphExec_t ge;
    const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void) hipGraphDestroy(g);
    if (e != hipSuccess) return al_hip_fail(e, "hipGraphInstantiate");
    *graph_exec = ge;
    return AL_OK;
}
extern "C" int al_util_graph_launch(void * graph_exec, void * stream) {
    AL_HIP(hipGraphLaunch((hipGraphExec_t) graph_exec, (hipStream_t) stream), "hipGraphLaunch");
    return AL_OK;
}
extern "C" int al_util_graph_destroy(void * graph_exec) { AL_HIP(hipGraphExecDestroy((hipGraphExec_t) graph_exec), "hipGraphExecDestroy"); return AL_OK; }

// ---------------------------------------------------------------------------
// seeded synthetic inputs
// ---------------------------------------------------------------------------

namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ float randn_at(uint64_t seed, uint64_t i) {
    const uint64_t h = splitmix64(splitmix64(seed) ^ i);
    const float u1 = ((float) (uint32_t) (h >> 40) + 1.0f) * (1.0f / 16777216.0f);        // (0, 1]
    const float u2 = (float) (uint32_t) ((h >> 16) & 0xffffffu) * (1.0f / 16777216.0f);   // [0, 1)
    return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__global__ void fill_randn_f32_kernel(float * dst, uint64_t n, uint64_t seed, uint64_t offset) {
    for (uint64_t i = blockIdx.x * (uint64_t) blockDim.x + threadIdx.x; i < n; i += (uint64_t) gridDim.x * blockDim.x)
        dst[i] = randn_at(seed, offset + i);
}

__global__ void fill_randn_f16_kernel(_Float16 * dst, uint64_t n, uint64_t seed, uint64_t offset) {
    for (uint64_t i = blockIdx.x * (uint64_t) blockDim.x + threadIdx.x; i < n; i += (uint64_t) gridDim.x * blockDim.x)
        dst[i] = (_Float16) randn_at(seed, offset + i);
}

__global__ void f32_to_f16_kernel(_Float16 * dst, const float * src, uint64_t n) {
    for (uint64_t i = blockIdx.x * (uint64_t) blockDim.x + threadIdx.x; i < n; i += (uint64_t) gridDim.x * blockDim.x)
        dst[i] = (_Float16) src[i];
}

// 16-byte vector copy, grid-stride; n16 = number of 16-byte words
__global__ void copy16_kernel(uint4 * __restrict__ dst, const uint4 * __restrict__ src, uint64_t n16) {
    for (uint64_t i = blockIdx.x * (uint64_t) blockDim.x + threadIdx.x; i < n16; i += (uint64_t) gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Does nothing: launches of it measure the dispatch cost of a grid shape.
__global__ void empty_kernel() {}

unsigned grid_for(uint64_t n) {
    const uint64_t b = (n + 255) / 256;
    return (unsigned) (b < 8192 ? (b ? b : 1) : 8192);
}

}  // namespace

extern "C" int al_util_fill_randn_f32(float * dst, uint64_t n, uint64_t seed, uint64_t offset, void * stream) {
    if (!n) return AL_OK;
    hipLaunchKernelGGL(fill_randn_f32_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t) stream, dst, n, seed, offset);
    AL_HIP(hipGetLastError(), "fill_randn_f32 launch");
    return AL_OK;
}

extern "C" int al_util_fill_randn_f16(uint16_t * dst, uint64_t n, uint64_t seed, uint64_t offset, void * stream) {
    if (!n) return AL_OK;
    hipLaunchKernelGGL(fill_randn_f16_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t) stream, (_Float16 *) dst, n, seed, offset);
    AL_HIP(hipGetLastError(), "fill_randn_f16 launch");
    return AL_OK;
}

extern "C" int al_util_f32_to_f16(uint16_t * dst, const float * src, uint64_t n, void * stream) {
    if (!n) return AL_OK;
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t) stream, (_Float16 *) dst, src, n);
    AL_HIP(hipGetLastError(), "f32_to_f16 launch");
    return AL_OK;
}

extern "C" int al_util_copy_kernel(void * dst, const void * src, uint64_t bytes, void * stream) {
    if (bytes % 16 || ((uintptr_t) dst | (uintptr_t) src) % 16)
        return al_fail(AL_ERR_INVALID, "al_util_copy_kernel: bytes and pointers must be 16-byte aligned");
    if (!bytes) return AL_OK;
    const uint64_t n16 = bytes / 16;
    const uint64_t blocks = (n16 + 255) / 256;
    hipLaunchKernelGGL(copy16_kernel, dim3((unsigned) (blocks < 16384 ? blocks : 16384)), dim3(256), 0,
                       (hipStream_t) stream, (uint4 *) dst, (const uint4 *) src, n16);
    AL_HIP(hipGetLastError(), "copy16 launch");
    return AL_OK;
}

extern "C" int al_util_empty_launch(int grid, int block, int lds_bytes, void * stream) {
    if (grid < 1 || block < 1 || block > 1024 || lds_bytes < 0 || lds_bytes > 160 * 1024)
        return al_fail(AL_ERR_INVALID, "al_util_empty_launch: grid >= 1, block 1..1024, lds_bytes 0..163840");
    static const hipError_t attr =
        hipFuncSetAttribute((const void *) empty_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    AL_HIP(attr, "hipFuncSetAttribute");
    hipLaunchKernelGGL(empty_kernel, dim3((unsigned) grid), dim3((unsigned) block), (unsigned) lds_bytes,
                       (hipStream_t) stream);
    AL_HIP(hipGetLastError(), "empty_kernel launch");
    return AL_OK;
}
