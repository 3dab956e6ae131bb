/*
 * eas_hip.h — C ABI of the MI355X (gfx950) backend of the eas kernel DSL.
 *
 * This library replaces the reference's native layer, the ObjC++ CPython
 * extension `eas._metal` (eas/runtime/_metal.mm).  Everything here is plain C:
 * opaque handles, raw pointers, sizes and int status codes; no Python, torch
 * or HIP types cross the boundary.  The CPython module `easy_as_amd._hip`
 * (easy_as_amd/csrc/hip_module.cpp) is one binding of it; INTEGRATION.md shows
 * how a ctypes binding would call it.
 *
 * Conventions
 *   - Every function returns EAS_HIP_OK (0) or a negative eas_hip_status.
 *   - On error, eas_hip_last_error() returns a thread-local message that stays
 *     valid until the next call into this library on the same thread.
 *   - `stream` arguments are hipStream_t values passed as void*; NULL is the
 *     default (null) stream of the current device.
 *   - Device memory comes from hipMalloc; "shared" memory is pinned host
 *     memory from hipHostMalloc (never hipHostRegister).
 */
#ifndef EAS_HIP_H
#define EAS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EAS_HIP_ABI_VERSION 2

typedef enum eas_hip_status {
  EAS_HIP_OK = 0,
  EAS_HIP_ERR_INVALID = -1,   /* bad argument (maps to ValueError/TypeError)  */
  EAS_HIP_ERR_NODEV = -2,     /* no usable GPU                                 */
  EAS_HIP_ERR_COMPILE = -3,   /* hiprtc compilation failed (log available)     */
  EAS_HIP_ERR_RUNTIME = -4,   /* a HIP runtime call failed                     */
  EAS_HIP_ERR_NOMEM = -5      /* allocation failed                             */
} eas_hip_status;

typedef enum eas_hip_storage {
  EAS_HIP_STORAGE_DEVICE = 0, /* reference "private": GPU-only memory          */
  EAS_HIP_STORAGE_SHARED = 1  /* reference "shared": pinned, host-visible      */
} eas_hip_storage;

/* Opaque compiled kernel: a loaded code object plus one function in it. */
typedef struct eas_hip_kernel eas_hip_kernel;

typedef struct eas_hip_device_props {
  char arch[64];              /* gcnArchName without feature suffix, e.g. "gfx950" */
  int compute_units;
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width;
  size_t total_global_mem;
  size_t lds_per_block;       /* bytes of LDS a workgroup can allocate          */
  int warp_size;              /* 64 on CDNA                                     */
  int max_threads_per_block;
} eas_hip_device_props;

/* ABI version of the loaded library (EAS_HIP_ABI_VERSION it was built with). */
int eas_hip_abi_version(void);

/* Thread-local message describing the last error on this thread. */
const char* eas_hip_last_error(void);

/* 1 if at least one HIP device is usable, else 0.
 * Replaces `is_available()` (_metal.mm:178-183). */
int eas_hip_is_available(void);

/* Properties of `device` (the current device if device < 0). */
int eas_hip_device_props_get(int device, eas_hip_device_props* out);

/* Compile HIP C++ source to a code object with hiprtc; no GPU needed.
 * `options` are hiprtc/clang options (e.g. "--offload-arch=gfx950", "-O3").
 * On success *code is malloc'ed (free with eas_hip_free_host) and *code_size set.
 * On EAS_HIP_ERR_COMPILE the compiler log is written to `log` (truncated).
 * Replaces the source->library half of `compile(src, name)` (_metal.mm:185-235). */
int eas_hip_compile_source(const char* src, const char* name, const char* const* options, int noptions,
                           void** code, size_t* code_size, char* log, size_t loglen);

/* Release memory returned by eas_hip_compile_source. */
void eas_hip_free_host(void* p);

/* Version of the hiprtc that eas_hip_compile_source uses, and the path it was
 * loaded from (copied into `path`, truncated to pathlen).  No reference
 * counterpart: Metal's compiler is part of the OS; here the code-object cache
 * key includes it.  Returns EAS_HIP_ERR_COMPILE if no hiprtc can be loaded. */
int eas_hip_compiler_version(int* major, int* minor, char* path, size_t pathlen);

/* Load a code object on the current device and look up `name`.
 * Replaces the library->pipeline half of `compile(src, name)` (_metal.mm:236-260). */
int eas_hip_kernel_load(const void* code, size_t code_size, const char* name, eas_hip_kernel** out);

/* Unload the module behind a kernel handle (pipeline capsule destructor, _metal.mm:104-112). */
void eas_hip_kernel_release(eas_hip_kernel* k);

/* Static resources of a loaded kernel (values < 0 when unknown). */
int eas_hip_kernel_attrs(const eas_hip_kernel* k, int* max_threads_per_block, int* static_lds_bytes,
                         int* num_vgprs, int* num_sgprs, int* private_bytes);

/* Allocate `nbytes` > 0 bytes of `storage` memory; *out receives the pointer.
 * Replaces `alloc_buffer(nbytes, storage)` (_metal.mm:262-307). */
int eas_hip_alloc(size_t nbytes, int storage, void** out);

/* Free memory from eas_hip_alloc (buffer capsule destructor, _metal.mm:80-102). */
int eas_hip_free(void* ptr, int storage);

/* Synchronous copies. Replace `copy_from_host` / `copy_to_host` (_metal.mm:309-493). */
int eas_hip_copy_h2d(void* dst, const void* src, size_t nbytes);
int eas_hip_copy_d2h(void* dst, const void* src, size_t nbytes);
int eas_hip_copy_d2d(void* dst, const void* src, size_t nbytes);

/* Fill `nbytes` of device memory with a byte value on `stream` (async). */
int eas_hip_memset(void* dst, int value, size_t nbytes, void* stream);

/* Enqueue `repeat` >= 1 launches of `k` on `stream` with a packed kernel-argument
 * blob (arguments at natural alignment, in the kernel's parameter order).
 * grid = workgroup counts, block = threads per workgroup.  Asynchronous.
 * Replaces `launch` / `launch_tg` (_metal.mm:1013-1222, 1232-1379); the
 * threads->workgroups conversion and the hidden extent arguments that emulate
 * Metal's non-uniform dispatchThreads are done by the caller. */
int eas_hip_launch(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                   const uint32_t block[3], uint32_t dynamic_lds, void* stream, int repeat);

/* `warmup` untimed launches, then `repeat` launches bracketed by events recorded
 * on `stream`; blocks until done and writes the mean milliseconds per launch.
 * The timing half of `runtime.benchmark` (eas/runtime/metal.py:466-506). */
int eas_hip_launch_timed(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                         const uint32_t block[3], uint32_t dynamic_lds, void* stream, int warmup, int repeat,
                         float* mean_ms);

/* Events: completion tracking for async launches (Pending capsules, _metal.mm:73-78, 1397-1434). */
int eas_hip_event_create(void** ev);
int eas_hip_event_record(void* ev, void* stream);
int eas_hip_event_synchronize(void* ev);
int eas_hip_event_query(void* ev);               /* 1 done, 0 pending, <0 error */
int eas_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int eas_hip_event_destroy(void* ev);

/* Wait for all work on `stream` / on the device. Replaces `queue_synchronize` (_metal.mm:676-708). */
int eas_hip_stream_synchronize(void* stream);
int eas_hip_device_synchronize(void);

/* DLPack (v0.8 ABI, kDLROCM = 10, kDLCPU = 1).
 * View a DLManagedTensor: accepts float16/float32, C-contiguous, element-aligned
 * byte_offset; writes the data pointer (byte_offset applied), total bytes, element
 * bits, ndim (<= max_ndim), shape and device type/id.
 * Validation half of `dlpack_import` (_metal.mm:530-638). */
int eas_hip_dlpack_view(const void* managed_tensor, void** data, uint64_t* nbytes, int* bits, int* ndim,
                        int64_t* shape, int max_ndim, int* device_type, int* device_id);

/* Build a DLManagedTensor over `data` (kDLROCM, device `device_id`, C-contiguous).
 * When the consumer calls its deleter, release(ctx) runs and the struct is freed.
 * Construction half of `dlpack_export` (_metal.mm:710-822). */
int eas_hip_dlpack_make(void* data, int device_id, const int64_t* shape, int ndim, int bits,
                        void (*release)(void* ctx), void* ctx, void** managed_out);

/* Call the deleter of a DLManagedTensor (no-op for NULL). */
void eas_hip_dlpack_delete(void* managed_tensor);

#ifdef __cplusplus
}
#endif

#endif /* EAS_HIP_H */
