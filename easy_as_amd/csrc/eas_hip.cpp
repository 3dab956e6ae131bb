// eas_hip.cpp — implementation of the C ABI declared in include/eas_hip.h.
//
// One process drives the GPU(s) through the HIP runtime directly: kernels are
// compiled in-process with hiprtc (gfx950 code objects), loaded with
// hipModuleLoadData and launched with hipModuleLaunchKernel from a packed
// kernel-argument blob.  No Python in here; see hip_module.cpp for the
// CPython binding.
//
// hiprtc is loaded with dlmopen into a link namespace of its own.  A process
// that already holds another hiprtc/comgr pair (PyTorch wheels bundle an older
// one with the same SONAMEs) would otherwise hand us that copy, and with it an
// older LLVM; hiprtc itself has no HIP-runtime dependency, so a private copy
// touches no GPU state.  The namespace has its own libc, whose `environ` is the
// main program's environment array as it was at dlmopen time; setenv in the
// main program can reallocate (free) that array, so every call into hiprtc
// first points the namespace's `environ` at the current array (under a lock).

#include "eas_hip.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <dlfcn.h>
#include <link.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

struct eas_hip_kernel {
  hipModule_t module;
  hipFunction_t function;
  int device;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(EAS_HIP_ERR_RUNTIME, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(call)                            \
  do {                                           \
    hipError_t e_ = (call);                      \
    if (e_ != hipSuccess) return hip_fail(e_, #call); \
  } while (0)

// ---- DLPack v0.8 structs (the stable ABI shared with torch/numpy) ----------
constexpr int kDLCPU = 1;
constexpr int kDLROCM = 10;
constexpr uint8_t kDLFloat = 2;

struct DLDevice {
  int32_t device_type;
  int32_t device_id;
};
struct DLDataType {
  uint8_t code;
  uint8_t bits;
  uint16_t lanes;
};
struct DLTensor {
  void* data;
  DLDevice device;
  int32_t ndim;
  DLDataType dtype;
  int64_t* shape;
  int64_t* strides;
  uint64_t byte_offset;
};
struct DLManagedTensor {
  DLTensor dl_tensor;
  void* manager_ctx;
  void (*deleter)(DLManagedTensor* self);
};

struct ExportCtx {
  void (*release)(void*);
  void* ctx;
  int64_t shape[8];
};

void export_deleter(DLManagedTensor* self) {
  if (!self) return;
  auto* c = static_cast<ExportCtx*>(self->manager_ctx);
  if (c) {
    if (c->release) c->release(c->ctx);
    delete c;
  }
  delete self;
}

// ---- hiprtc, resolved at first use -----------------------------------------
struct Rtc {
  hiprtcResult (*create)(hiprtcProgram*, const char*, const char*, int, const char**, const char**) = nullptr;
  hiprtcResult (*compile)(hiprtcProgram, int, const char**) = nullptr;
  hiprtcResult (*log_size)(hiprtcProgram, size_t*) = nullptr;
  hiprtcResult (*log)(hiprtcProgram, char*) = nullptr;
  hiprtcResult (*code_size)(hiprtcProgram, size_t*) = nullptr;
  hiprtcResult (*code)(hiprtcProgram, char*) = nullptr;
  hiprtcResult (*destroy)(hiprtcProgram*) = nullptr;
  const char* (*error_string)(hiprtcResult) = nullptr;
  hiprtcResult (*version)(int*, int*) = nullptr;
  char*** ns_environ = nullptr;  // `environ` of the namespace's libc (null when not in a namespace)
  std::string path;
  std::string error;
  bool ok = false;
};

std::mutex g_rtc_mutex;

// Held around every call into hiprtc: serialises them and refreshes the namespace's environment.
struct RtcCall {
  std::lock_guard<std::mutex> lock;
  explicit RtcCall(const Rtc& r) : lock(g_rtc_mutex) {
    if (r.ns_environ) *r.ns_environ = environ;
  }
};

bool bind_rtc(Rtc& r, void* h) {
  r.create = reinterpret_cast<decltype(r.create)>(dlsym(h, "hiprtcCreateProgram"));
  r.compile = reinterpret_cast<decltype(r.compile)>(dlsym(h, "hiprtcCompileProgram"));
  r.log_size = reinterpret_cast<decltype(r.log_size)>(dlsym(h, "hiprtcGetProgramLogSize"));
  r.log = reinterpret_cast<decltype(r.log)>(dlsym(h, "hiprtcGetProgramLog"));
  r.code_size = reinterpret_cast<decltype(r.code_size)>(dlsym(h, "hiprtcGetCodeSize"));
  r.code = reinterpret_cast<decltype(r.code)>(dlsym(h, "hiprtcGetCode"));
  r.destroy = reinterpret_cast<decltype(r.destroy)>(dlsym(h, "hiprtcDestroyProgram"));
  r.error_string = reinterpret_cast<decltype(r.error_string)>(dlsym(h, "hiprtcGetErrorString"));
  r.version = reinterpret_cast<decltype(r.version)>(dlsym(h, "hiprtcVersion"));
  return r.create && r.compile && r.log_size && r.log && r.code_size && r.code && r.destroy && r.error_string &&
         r.version;
}

const Rtc& rtc() {
  static Rtc r;
  static std::once_flag once;
  std::call_once(once, [] {
    std::vector<std::string> candidates;
    if (const char* e = getenv("EAS_HIPRTC_LIB")) candidates.emplace_back(e);
    if (const char* e = getenv("ROCM_PATH")) candidates.emplace_back(std::string(e) + "/lib/libhiprtc.so.7");
    candidates.emplace_back("/opt/rocm/lib/libhiprtc.so.7");
    for (const std::string& c : candidates) {
      void* h = dlmopen(LM_ID_NEWLM, c.c_str(), RTLD_NOW | RTLD_LOCAL);
      if (!h) {
        const char* d = dlerror();
        r.error += c + ": " + (d ? d : "dlmopen failed") + "; ";
        continue;
      }
      if (bind_rtc(r, h)) {
        Lmid_t lmid;
        if (dlinfo(h, RTLD_DI_LMID, &lmid) == 0) {
          if (void* ns_libc = dlmopen(lmid, "libc.so.6", RTLD_NOW | RTLD_NOLOAD))
            r.ns_environ = reinterpret_cast<char***>(dlsym(ns_libc, "environ"));
        }
        if (!r.ns_environ) {  // cannot keep its environment current: do not use this copy
          r.error += c + ": namespace libc `environ` not found; ";
          continue;
        }
        r.path = c;
        r.ok = true;
        return;
      }
      r.error += c + ": missing hiprtc symbols; ";
      dlclose(h);
    }
    // last resort: whatever hiprtc the process can load in its own namespace
    if (void* h = dlopen("libhiprtc.so.7", RTLD_NOW | RTLD_LOCAL)) {
      if (bind_rtc(r, h)) {
        r.path = "libhiprtc.so.7";
        r.ok = true;
        return;
      }
    }
    r.error += "libhiprtc.so.7: not loadable";
  });
  return r;
}

}  // namespace

extern "C" {

int eas_hip_abi_version(void) { return EAS_HIP_ABI_VERSION; }

const char* eas_hip_last_error(void) { return g_err.c_str(); }

int eas_hip_is_available(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n > 0 ? 1 : 0;
}

int eas_hip_device_props_get(int device, eas_hip_device_props* out) {
  if (!out) return fail(EAS_HIP_ERR_INVALID, "out must not be NULL");
  if (!eas_hip_is_available()) return fail(EAS_HIP_ERR_NODEV, "no HIP device available");
  if (device < 0) HIP_TRY(hipGetDevice(&device));
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, device));
  memset(out, 0, sizeof(*out));
  size_t i = 0;
  for (; i + 1 < sizeof(out->arch) && p.gcnArchName[i] && p.gcnArchName[i] != ':'; ++i) out->arch[i] = p.gcnArchName[i];
  out->arch[i] = 0;
  out->compute_units = p.multiProcessorCount;
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_width = p.memoryBusWidth;
  out->total_global_mem = p.totalGlobalMem;
  out->lds_per_block = p.sharedMemPerBlock;
  out->warp_size = p.warpSize;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  return EAS_HIP_OK;
}

int eas_hip_compile_source(const char* src, const char* name, const char* const* options, int noptions, void** code,
                           size_t* code_size, char* log, size_t loglen) {
  if (!src || !code || !code_size) return fail(EAS_HIP_ERR_INVALID, "src/code/code_size must not be NULL");
  if (noptions < 0 || (noptions > 0 && !options)) return fail(EAS_HIP_ERR_INVALID, "bad options array");
  if (log && loglen) log[0] = 0;
  const Rtc& rt = rtc();
  if (!rt.ok) return fail(EAS_HIP_ERR_COMPILE, "hiprtc not available: %s", rt.error.c_str());
  RtcCall guard(rt);
  hiprtcProgram prog;
  hiprtcResult r = rt.create(&prog, src, name ? name : "eas_kernel.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(EAS_HIP_ERR_COMPILE, "hiprtcCreateProgram: %s", rt.error_string(r));
  r = rt.compile(prog, noptions, const_cast<const char**>(options));
  size_t lsz = 0;
  rt.log_size(prog, &lsz);
  std::string text(lsz, '\0');
  if (lsz) rt.log(prog, &text[0]);
  if (log && loglen) {
    size_t n = text.size() < loglen - 1 ? text.size() : loglen - 1;
    memcpy(log, text.data(), n);
    log[n] = 0;
  }
  if (r != HIPRTC_SUCCESS) {
    rt.destroy(&prog);
    return fail(EAS_HIP_ERR_COMPILE, "hiprtc compile of %s failed: %s", name ? name : "kernel", rt.error_string(r));
  }
  size_t sz = 0;
  r = rt.code_size(prog, &sz);
  if (r != HIPRTC_SUCCESS || sz == 0) {
    rt.destroy(&prog);
    return fail(EAS_HIP_ERR_COMPILE, "hiprtc produced no code");
  }
  void* buf = malloc(sz);
  if (!buf) {
    rt.destroy(&prog);
    return fail(EAS_HIP_ERR_NOMEM, "out of host memory");
  }
  rt.code(prog, static_cast<char*>(buf));
  rt.destroy(&prog);
  *code = buf;
  *code_size = sz;
  return EAS_HIP_OK;
}

int eas_hip_compiler_version(int* major, int* minor, char* path, size_t pathlen) {
  if (!major || !minor) return fail(EAS_HIP_ERR_INVALID, "major/minor must not be NULL");
  const Rtc& rt = rtc();
  if (!rt.ok) return fail(EAS_HIP_ERR_COMPILE, "hiprtc not available: %s", rt.error.c_str());
  RtcCall guard(rt);
  hiprtcResult r = rt.version(major, minor);
  if (r != HIPRTC_SUCCESS) return fail(EAS_HIP_ERR_COMPILE, "hiprtcVersion: %s", rt.error_string(r));
  if (path && pathlen) {
    size_t n = rt.path.size() < pathlen - 1 ? rt.path.size() : pathlen - 1;
    memcpy(path, rt.path.data(), n);
    path[n] = 0;
  }
  return EAS_HIP_OK;
}

void eas_hip_free_host(void* p) { free(p); }

int eas_hip_kernel_load(const void* code, size_t code_size, const char* name, eas_hip_kernel** out) {
  if (!code || !code_size || !name || !out) return fail(EAS_HIP_ERR_INVALID, "code/name/out must not be NULL");
  if (!eas_hip_is_available()) return fail(EAS_HIP_ERR_NODEV, "no HIP device available");
  auto* k = new (std::nothrow) eas_hip_kernel{};
  if (!k) return fail(EAS_HIP_ERR_NOMEM, "out of host memory");
  hipError_t e = hipGetDevice(&k->device);
  if (e == hipSuccess) e = hipModuleLoadData(&k->module, code);
  if (e != hipSuccess) {
    delete k;
    return hip_fail(e, "hipModuleLoadData");
  }
  e = hipModuleGetFunction(&k->function, k->module, name);
  if (e != hipSuccess) {
    (void)hipModuleUnload(k->module);
    delete k;
    return fail(EAS_HIP_ERR_RUNTIME, "kernel function %s not found in code object: %s", name, hipGetErrorString(e));
  }
  *out = k;
  return EAS_HIP_OK;
}

void eas_hip_kernel_release(eas_hip_kernel* k) {
  if (!k) return;
  if (k->module) (void)hipModuleUnload(k->module);
  delete k;
}

int eas_hip_kernel_attrs(const eas_hip_kernel* k, int* max_threads_per_block, int* static_lds_bytes, int* num_vgprs,
                         int* num_sgprs, int* private_bytes) {
  if (!k) return fail(EAS_HIP_ERR_INVALID, "kernel must not be NULL");
  struct Item {
    int* dst;
    hipFunction_attribute a;
  } items[] = {{max_threads_per_block, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK},
               {static_lds_bytes, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES},
               {num_vgprs, HIP_FUNC_ATTRIBUTE_NUM_REGS},
               {private_bytes, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES}};
  if (num_sgprs) *num_sgprs = -1;  // not exposed by hipFuncGetAttribute
  for (auto& it : items) {
    if (!it.dst) continue;
    int v = -1;
    if (hipFuncGetAttribute(&v, it.a, k->function) != hipSuccess) {
      (void)hipGetLastError();
      v = -1;
    }
    *it.dst = v;
  }
  return EAS_HIP_OK;
}

int eas_hip_alloc(size_t nbytes, int storage, void** out) {
  if (!out) return fail(EAS_HIP_ERR_INVALID, "out must not be NULL");
  if (nbytes == 0) return fail(EAS_HIP_ERR_INVALID, "nbytes must be > 0");
  if (storage != EAS_HIP_STORAGE_DEVICE && storage != EAS_HIP_STORAGE_SHARED)
    return fail(EAS_HIP_ERR_INVALID, "storage must be device(0) or shared(1)");
  if (!eas_hip_is_available()) return fail(EAS_HIP_ERR_NODEV, "no HIP device available");
  void* p = nullptr;
  hipError_t e = storage == EAS_HIP_STORAGE_DEVICE ? hipMalloc(&p, nbytes) : hipHostMalloc(&p, nbytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(EAS_HIP_ERR_NOMEM, "allocation of %zu bytes failed: %s", nbytes, hipGetErrorString(e));
  }
  *out = p;
  return EAS_HIP_OK;
}

int eas_hip_free(void* ptr, int storage) {
  if (!ptr) return EAS_HIP_OK;
  HIP_TRY(storage == EAS_HIP_STORAGE_SHARED ? hipHostFree(ptr) : hipFree(ptr));
  return EAS_HIP_OK;
}

int eas_hip_copy_h2d(void* dst, const void* src, size_t nbytes) {
  if (!nbytes) return EAS_HIP_OK;
  if (!dst || !src) return fail(EAS_HIP_ERR_INVALID, "NULL pointer in copy");
  HIP_TRY(hipMemcpy(dst, src, nbytes, hipMemcpyHostToDevice));
  return EAS_HIP_OK;
}

int eas_hip_copy_d2h(void* dst, const void* src, size_t nbytes) {
  if (!nbytes) return EAS_HIP_OK;
  if (!dst || !src) return fail(EAS_HIP_ERR_INVALID, "NULL pointer in copy");
  HIP_TRY(hipMemcpy(dst, src, nbytes, hipMemcpyDeviceToHost));
  return EAS_HIP_OK;
}

int eas_hip_copy_d2d(void* dst, const void* src, size_t nbytes) {
  if (!nbytes) return EAS_HIP_OK;
  if (!dst || !src) return fail(EAS_HIP_ERR_INVALID, "NULL pointer in copy");
  HIP_TRY(hipMemcpy(dst, src, nbytes, hipMemcpyDeviceToDevice));
  return EAS_HIP_OK;
}

int eas_hip_memset(void* dst, int value, size_t nbytes, void* stream) {
  if (!nbytes) return EAS_HIP_OK;
  if (!dst) return fail(EAS_HIP_ERR_INVALID, "NULL pointer in memset");
  HIP_TRY(hipMemsetAsync(dst, value, nbytes, static_cast<hipStream_t>(stream)));
  return EAS_HIP_OK;
}

static int launch_n(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                    const uint32_t block[3], uint32_t dynamic_lds, void* stream, int n) {
  if (!k || !grid || !block) return fail(EAS_HIP_ERR_INVALID, "kernel/grid/block must not be NULL");
  if (kernarg_size && !kernarg) return fail(EAS_HIP_ERR_INVALID, "kernarg is NULL with nonzero size");
  for (int i = 0; i < 3; ++i) {
    if (grid[i] == 0 || block[i] == 0) return fail(EAS_HIP_ERR_INVALID, "grid/block dims must be > 0");
  }
  const uint64_t threads = (uint64_t)block[0] * block[1] * block[2];
  if (threads > 1024) return fail(EAS_HIP_ERR_INVALID, "threads per workgroup too large: %llu", (unsigned long long)threads);
  for (int i = 0; i < 3; ++i) {
    if ((uint64_t)grid[i] * block[i] > 0xFFFFFFFFull)
      return fail(EAS_HIP_ERR_INVALID, "grid dim %d exceeds 2^32 work-items", i);
  }
  // hipModuleLaunchKernel copies the blob; an empty blob still needs a valid pointer.
  static const uint64_t kEmpty = 0;
  size_t size = kernarg_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(kernarg_size ? kernarg : &kEmpty),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  for (int r = 0; r < n; ++r) {
    HIP_TRY(hipModuleLaunchKernel(k->function, grid[0], grid[1], grid[2], block[0], block[1], block[2], dynamic_lds,
                                  static_cast<hipStream_t>(stream), nullptr, config));
  }
  return EAS_HIP_OK;
}

int eas_hip_launch(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                   const uint32_t block[3], uint32_t dynamic_lds, void* stream, int repeat) {
  if (repeat <= 0) return fail(EAS_HIP_ERR_INVALID, "repeat must be > 0");
  return launch_n(k, kernarg, kernarg_size, grid, block, dynamic_lds, stream, repeat);
}

int eas_hip_launch_timed(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                         const uint32_t block[3], uint32_t dynamic_lds, void* stream, int warmup, int repeat,
                         float* mean_ms) {
  if (repeat <= 0 || warmup < 0 || !mean_ms) return fail(EAS_HIP_ERR_INVALID, "repeat > 0, warmup >= 0, mean_ms required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (warmup) {
    int rc = launch_n(k, kernarg, kernarg_size, grid, block, dynamic_lds, stream, warmup);
    if (rc) return rc;
  }
  hipEvent_t t0, t1;
  HIP_TRY(hipEventCreate(&t0));
  hipError_t e = hipEventCreate(&t1);
  if (e != hipSuccess) {
    (void)hipEventDestroy(t0);
    return hip_fail(e, "hipEventCreate");
  }
  int rc = EAS_HIP_OK;
  e = hipEventRecord(t0, s);
  if (e != hipSuccess) rc = hip_fail(e, "hipEventRecord");
  if (!rc) rc = launch_n(k, kernarg, kernarg_size, grid, block, dynamic_lds, stream, repeat);
  if (!rc && (e = hipEventRecord(t1, s)) != hipSuccess) rc = hip_fail(e, "hipEventRecord");
  if (!rc && (e = hipEventSynchronize(t1)) != hipSuccess) rc = hip_fail(e, "hipEventSynchronize");
  float ms = 0.f;
  if (!rc && (e = hipEventElapsedTime(&ms, t0, t1)) != hipSuccess) rc = hip_fail(e, "hipEventElapsedTime");
  (void)hipEventDestroy(t0);
  (void)hipEventDestroy(t1);
  if (!rc) *mean_ms = ms / (float)repeat;
  return rc;
}

int eas_hip_event_create(void** ev) {
  if (!ev) return fail(EAS_HIP_ERR_INVALID, "ev must not be NULL");
  hipEvent_t e;
  HIP_TRY(hipEventCreate(&e));
  *ev = e;
  return EAS_HIP_OK;
}

int eas_hip_event_record(void* ev, void* stream) {
  HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream)));
  return EAS_HIP_OK;
}

int eas_hip_event_synchronize(void* ev) {
  HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(ev)));
  return EAS_HIP_OK;
}

int eas_hip_event_query(void* ev) {
  hipError_t e = hipEventQuery(static_cast<hipEvent_t>(ev));
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  return hip_fail(e, "hipEventQuery");
}

int eas_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!ms) return fail(EAS_HIP_ERR_INVALID, "ms must not be NULL");
  HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return EAS_HIP_OK;
}

int eas_hip_event_destroy(void* ev) {
  if (!ev) return EAS_HIP_OK;
  HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return EAS_HIP_OK;
}

int eas_hip_stream_synchronize(void* stream) {
  HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return EAS_HIP_OK;
}

int eas_hip_device_synchronize(void) {
  HIP_TRY(hipDeviceSynchronize());
  return EAS_HIP_OK;
}

int eas_hip_dlpack_view(const void* managed_tensor, void** data, uint64_t* nbytes, int* bits, int* ndim,
                        int64_t* shape, int max_ndim, int* device_type, int* device_id) {
  if (!managed_tensor || !data || !nbytes || !bits || !ndim) return fail(EAS_HIP_ERR_INVALID, "NULL argument");
  const DLTensor& t = static_cast<const DLManagedTensor*>(managed_tensor)->dl_tensor;
  if (t.device.device_type != kDLROCM && t.device.device_type != kDLCPU)
    return fail(EAS_HIP_ERR_INVALID, "dlpack_import expects a kDLROCM(10) or kDLCPU(1) tensor, got device_type=%d",
                t.device.device_type);
  if (t.dtype.code != kDLFloat || t.dtype.lanes != 1 || (t.dtype.bits != 16 && t.dtype.bits != 32))
    return fail(EAS_HIP_ERR_INVALID, "dlpack_import only supports float32/float16 tensors");
  if (t.ndim < 0 || t.ndim > max_ndim) return fail(EAS_HIP_ERR_INVALID, "dlpack ndim %d unsupported", t.ndim);
  const uint64_t elem = t.dtype.bits / 8;
  uint64_t numel = 1;
  int64_t expect = 1;
  bool contiguous = true;
  for (int i = t.ndim - 1; i >= 0; --i) {
    const int64_t d = t.shape[i];
    if (d < 0) return fail(EAS_HIP_ERR_INVALID, "invalid dlpack shape");
    if (t.strides && d > 1 && t.strides[i] != expect) contiguous = false;
    expect *= d;
    if (d && numel > UINT64_MAX / (uint64_t)d) return fail(EAS_HIP_ERR_INVALID, "dlpack tensor too large");
    numel *= (uint64_t)d;
  }
  if (!contiguous) return fail(EAS_HIP_ERR_INVALID, "dlpack_import requires a contiguous tensor");
  if (t.byte_offset % elem) return fail(EAS_HIP_ERR_INVALID, "dlpack byte_offset must be aligned to element size");
  if (numel && !t.data) return fail(EAS_HIP_ERR_INVALID, "dlpack tensor has null data pointer");
  *data = static_cast<char*>(t.data) + t.byte_offset;
  *nbytes = numel * elem;
  *bits = t.dtype.bits;
  *ndim = t.ndim;
  for (int i = 0; shape && i < t.ndim; ++i) shape[i] = t.shape[i];
  if (device_type) *device_type = t.device.device_type;
  if (device_id) *device_id = t.device.device_id;
  return EAS_HIP_OK;
}

int eas_hip_dlpack_make(void* data, int device_id, const int64_t* shape, int ndim, int bits, void (*release)(void*),
                        void* ctx, void** managed_out) {
  if (!managed_out || (ndim > 0 && !shape)) return fail(EAS_HIP_ERR_INVALID, "NULL argument");
  if (ndim < 0 || ndim > 8) return fail(EAS_HIP_ERR_INVALID, "ndim must be in [0, 8]");
  if (bits != 16 && bits != 32) return fail(EAS_HIP_ERR_INVALID, "dtype_bits must be 16 or 32");
  for (int i = 0; i < ndim; ++i)
    if (shape[i] < 0) return fail(EAS_HIP_ERR_INVALID, "invalid shape");
  auto* c = new (std::nothrow) ExportCtx{};
  auto* m = new (std::nothrow) DLManagedTensor{};
  if (!c || !m) {
    delete c;
    delete m;
    return fail(EAS_HIP_ERR_NOMEM, "out of host memory");
  }
  c->release = release;
  c->ctx = ctx;
  for (int i = 0; i < ndim; ++i) c->shape[i] = shape[i];
  m->dl_tensor.data = data;
  m->dl_tensor.device.device_type = kDLROCM;
  m->dl_tensor.device.device_id = device_id;
  m->dl_tensor.ndim = ndim;
  m->dl_tensor.dtype.code = kDLFloat;
  m->dl_tensor.dtype.bits = (uint8_t)bits;
  m->dl_tensor.dtype.lanes = 1;
  m->dl_tensor.shape = c->shape;
  m->dl_tensor.strides = nullptr;
  m->dl_tensor.byte_offset = 0;
  m->manager_ctx = c;
  m->deleter = export_deleter;
  *managed_out = m;
  return EAS_HIP_OK;
}

void eas_hip_dlpack_delete(void* managed_tensor) {
  auto* m = static_cast<DLManagedTensor*>(managed_tensor);
  if (m && m->deleter) m->deleter(m);
}

}  // extern "C"
