/*
 * eas_hip.h — C ABI of the MI355X (gfx950) backend of the eas kernel DSL.
 *
 * This library replaces the reference's native layer, the ObjC++ CPython
 * extension `eas._metal` (eas/runtime/_metal.mm).  Everything here is plain C:
 * opaque handles, raw pointers, sizes and int status codes; no Python, torch
 * or HIP types cross the boundary.  The CPython module `easy_as_amd._hip`
 * (easy_as_amd/csrc/hip_module.cpp) is one binding of it; a ctypes binding
 * needs only the functions below and their status codes.
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

#define EAS_HIP_ABI_VERSION 4

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

/* ---- launch shapes --------------------------------------------------------
 * How the reference's dispatch sizes map onto HIP workgroups for one compiled
 * eas kernel.  The reference dispatches Metal threads (`launch`: threads per
 * grid, non-uniform last threadgroup) or threadgroups (`launch_tg`).  Here an
 * SPMD program (one Metal thread) is spread over HIP threads, and a thread-mode
 * kernel's threadgroup is one workgroup; the kernels take their true extent as
 * hidden u32 arguments after their own, because HIP has no non-uniform
 * dispatch.  Every generated source carries its shape on a marker line
 * (`// eas-launch: kind=... block=... wg=... ppw=... split=... args=... hidden=...`). */
typedef enum eas_hip_launch_kind {
  EAS_HIP_KIND_RAW = 0,    /* shape unknown: only eas_hip_launch (workgroups) runs it      */
  EAS_HIP_KIND_SPMD = 1,   /* a Metal thread is a program of block_size lanes (mk.arange)   */
  EAS_HIP_KIND_THREAD = 2, /* a Metal thread is a HIP thread, a threadgroup a workgroup     */
  EAS_HIP_KIND_GEMM = 3    /* lifted MFMA GEMM: planned from M, N, K and its buffers        */
} eas_hip_launch_kind;

typedef struct eas_hip_launch_shape {
  int kind;                 /* eas_hip_launch_kind                                        */
  uint32_t block_size;      /* the kernel's BLOCK (lanes per program, threads per group)   */
  uint32_t wg_size;         /* HIP threads per workgroup                                   */
  uint32_t programs_per_wg; /* programs (SPMD) or threadgroups (thread mode emitted as lanes)
                               each group of `split` workgroups runs; 1 for one workgroup per
                               threadgroup                                                  */
  uint32_t split;           /* workgroups a program's (threadgroup's) lanes are spread over */
  uint32_t arg_bytes;       /* packed bytes of the kernel's own arguments (0: not checked) */
  uint32_t hidden;          /* u32 extents that follow them (<= EAS_HIP_MAX_HIDDEN)        */
} eas_hip_launch_shape;

#define EAS_HIP_MAX_HIDDEN 8

/* Parse the `// eas-launch:` marker line of a generated source into *out.
 * EAS_HIP_ERR_INVALID if the source has none or it is malformed.  No GPU needed. */
int eas_hip_launch_shape_parse(const char* src, eas_hip_launch_shape* out);

/* Attach a launch shape to a loaded kernel (validated), or read it back. */
int eas_hip_kernel_set_shape(eas_hip_kernel* k, const eas_hip_launch_shape* shape);
int eas_hip_kernel_get_shape(const eas_hip_kernel* k, eas_hip_launch_shape* out);

/* The HIP dispatch of a reference-convention launch, without launching (no GPU
 * needed).  by_groups = 0: `size` is threads per grid, as `launch(pipeline, argv,
 * writable, threads_per_grid, threads_per_threadgroup)` passes it
 * (_metal.mm:1013-1222, 1381-1383); by_groups = 1: `size` is threadgroups, as
 * `launch_tg` passes it (_metal.mm:1232-1379).  `tptg` is the threads per
 * threadgroup the reference runtime passes ((BLOCK,1,1) for thread-mode kernels,
 * (1,1,1) for SPMD ones, eas/runtime/metal.py:259-326); all zeros means the kernel's
 * own.  Writes the workgroup grid, the workgroup shape and the shape->hidden
 * extents.  A zero size dimension is EAS_HIP_ERR_INVALID, as in the reference. */
int eas_hip_plan_dispatch(const eas_hip_launch_shape* shape, int by_groups, const uint64_t size[3],
                          const uint32_t tptg[3], uint32_t grid[3], uint32_t block[3], uint32_t* hidden,
                          int max_hidden);

/* ---- lifted GEMMs ---------------------------------------------------------
 * A kernel that the GEMM lift proved to be C = A @ B is compiled to several entry
 * points, and each launch picks one from the matrix sizes, the buffers and the number
 * of compute units.  Its source carries a second marker line with what that plan
 * needs (`// eas-gemm: entry=... K=... tm=... ...`): the position of M, N (the row
 * stride of B and C) and the tile-base scalars in the packed arguments, where A, B and
 * C are, the reference's tile per threadgroup and the entry points present.  No
 * counterpart in the reference, whose one pipeline per kernel runs any grid. */
typedef enum eas_hip_gemm_entry {
  EAS_HIP_GEMM_MAIN = 0,      /* the kernel's own name: 4 waves (skinny path, register-staged body, fp32 64 x 64) */
  EAS_HIP_GEMM_PP = 1,        /* <name>__pp: 8 waves on 256 x 256 tiles                                          */
  EAS_HIP_GEMM_T128 = 2,      /* <name>__t128: 128 x 128 tiles                                                   */
  EAS_HIP_GEMM_T128X256 = 3,  /* <name>__t128x256                                                                 */
  EAS_HIP_GEMM_T128X64 = 4,   /* <name>__t128x64                                                                  */
  EAS_HIP_GEMM_T64X64 = 5,    /* <name>__t64x64                                                                   */
  EAS_HIP_GEMM_NENTRIES = 6
} eas_hip_gemm_entry;

typedef struct eas_hip_gemm_shape {
  char entry[128];            /* the kernel's own entry point; the others append their suffix      */
  uint32_t entries;           /* bit e set: entry point e (eas_hip_gemm_entry) is in the code object */
  uint32_t K;                 /* reduction length (a constexpr of the kernel)                        */
  uint32_t tm, tn;            /* rows and columns of C per reference threadgroup                     */
  uint32_t row_axis;          /* threadgroup axis (0 or 1) that indexes tile rows                    */
  uint32_t bm, bn;            /* tile of the kernel's own entry                                      */
  uint32_t threads, pp_threads, t128_threads; /* workgroup sizes: own, 8-wave, smaller-tile entries  */
  uint32_t skinny_m, skinny_n;  /* launches of <= skinny_m rows: one workgroup per skinny_n columns  */
  uint32_t skinny_cut, wide_m;  /* rows that always stay skinny; rows that may take 2 x skinny_n     */
  uint32_t f32;               /* fp32 operands (the tiled `dot` GEMM), else 16-bit                   */
  uint32_t col_masked;        /* columns bounded by N (else by the launched grid only)               */
  int32_t m_off;              /* byte offset of the u32 M in the packed arguments; -1: no row bound  */
  int32_t ldb_off;            /* byte offset of the u32 N (row stride of B and C)                    */
  int32_t row_base_off, col_base_off; /* byte offsets of the u32 tile bases; -1: none                */
  uint32_t a_arg, b_arg, c_arg;       /* argument positions of A, B and C                            */
  uint32_t a_off, b_off;              /* byte offsets of A's and B's pointers                        */
  uint32_t a_elem, b_elem, c_elem;    /* bytes per element of A, B and C                             */
} eas_hip_gemm_shape;

typedef struct eas_hip_gemm_plan {
  int launch;                 /* 0: the launch covers no element of C; nothing runs     */
  int entry;                  /* eas_hip_gemm_entry to launch                            */
  uint32_t grid[3], block[3]; /* workgroups and threads per workgroup                    */
  uint32_t hidden[4];         /* the covered rectangle: m_lo, m_hi, n_lo, n_hi           */
} eas_hip_gemm_plan;

/* Parse the `// eas-gemm:` marker line of a lifted GEMM's source.  No GPU needed. */
int eas_hip_gemm_shape_parse(const char* src, eas_hip_gemm_shape* out);

/* Attach a GEMM shape to a kernel with a GEMM launch shape, resolving every entry
 * point it names in the kernel's code object. */
int eas_hip_kernel_set_gemm(eas_hip_kernel* k, const eas_hip_gemm_shape* gemm);

/* The launch plan of a lifted GEMM for a reference-convention launch, without
 * launching (no GPU needed).  `size`, `tptg` and `by_groups` as for
 * eas_hip_plan_dispatch; the grid must consist of whole threadgroups.  `kernarg`
 * holds the kernel's own arguments (M, N, the tile bases and the A and B pointers
 * are read from it), `arg_bytes[i]` the byte length of the buffer behind argument i
 * (nargs entries).  The launch covers rows [m_lo, m_hi) and columns [n_lo, n_hi):
 * the origin is tm * row_base (tn * col_base) when the kernel offsets its threadgroup
 * ids by a scalar, the extent the launched grid, clamped to M (N) when the kernel
 * bounds rows (columns).  A launch that would read or write past a buffer, or whose
 * matrices exceed u32 indexing, is EAS_HIP_ERR_INVALID.  `choice` names the entry
 * ("auto", "8wave", "tile128", "tile128x256", "tile128x64", "tile64", "4wave");
 * NULL reads EAS_HIP_GEMM_ENTRY (default "auto"). */
int eas_hip_plan_gemm(const eas_hip_launch_shape* shape, const eas_hip_gemm_shape* gemm, const void* kernarg,
                      size_t kernarg_size, const uint64_t* arg_bytes, int nargs, int by_groups,
                      const uint64_t size[3], const uint32_t tptg[3], int compute_units, const char* choice,
                      eas_hip_gemm_plan* out);

/* Enqueue `repeat` >= 1 launches by the reference's conventions: `kernarg` holds the
 * kernel's own arguments only (shape->arg_bytes when known); the hidden extents are
 * appended here.  `arg_bytes` (nargs entries, one per kernel argument: the byte length
 * of a buffer, 0 for a scalar) stands for the lengths the reference's buffer objects
 * carry; a lifted GEMM needs it to check its extents and rejects NULL, the other kinds
 * ignore it.  Asynchronous.  Replaces `launch` / `launch_async` (_metal.mm:1013-1222,
 * 1381-1383) and `launch_tg` / `launch_tg_async` (_metal.mm:1232-1379). */
int eas_hip_launch_threads(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size,
                           const uint64_t* arg_bytes, int nargs, const uint64_t threads_per_grid[3],
                           const uint32_t threads_per_threadgroup[3], void* stream, int repeat);
int eas_hip_launch_threadgroups(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size,
                                const uint64_t* arg_bytes, int nargs, const uint64_t threadgroups[3],
                                const uint32_t threads_per_threadgroup[3], void* stream, int repeat);

/* Enqueue `repeat` >= 1 launches of `k` on `stream` with a packed kernel-argument
 * blob (arguments at natural alignment, in the kernel's parameter order, then the
 * hidden u32 extents).  grid = workgroup counts, block = threads per workgroup.
 * Asynchronous.  The HIP-level dispatch under both reference launch forms; the
 * Python runtime plans its launches itself and uses this one (with a lifted GEMM
 * entry point `k` loaded by that entry's name).  When the kernel's shape knows its
 * argument bytes, a blob of any other size is EAS_HIP_ERR_INVALID. */
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
