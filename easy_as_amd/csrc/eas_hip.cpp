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
  eas_hip_launch_shape shape;  // kind EAS_HIP_KIND_RAW until set
  // lifted GEMMs: every entry point of the code object, set by eas_hip_kernel_set_gemm
  bool has_gemm;
  eas_hip_gemm_shape gemm;
  hipFunction_t gemm_fn[EAS_HIP_GEMM_NENTRIES];
  int compute_units;
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

static int launch_fn(hipFunction_t fn, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                     const uint32_t block[3], uint32_t dynamic_lds, void* stream, int n) {
  if (!fn || !grid || !block) return fail(EAS_HIP_ERR_INVALID, "kernel/grid/block must not be NULL");
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
    HIP_TRY(hipModuleLaunchKernel(fn, grid[0], grid[1], grid[2], block[0], block[1], block[2], dynamic_lds,
                                  static_cast<hipStream_t>(stream), nullptr, config));
  }
  return EAS_HIP_OK;
}

static int launch_n(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                    const uint32_t block[3], uint32_t dynamic_lds, void* stream, int n) {
  if (!k) return fail(EAS_HIP_ERR_INVALID, "kernel must not be NULL");
  return launch_fn(k->function, kernarg, kernarg_size, grid, block, dynamic_lds, stream, n);
}

// ---- launch shapes -----------------------------------------------------------

static int check_shape(const eas_hip_launch_shape* s) {
  if (!s) return fail(EAS_HIP_ERR_INVALID, "launch shape must not be NULL");
  if (s->kind < EAS_HIP_KIND_RAW || s->kind > EAS_HIP_KIND_GEMM) return fail(EAS_HIP_ERR_INVALID, "unknown launch kind %d", s->kind);
  if (s->hidden > EAS_HIP_MAX_HIDDEN) return fail(EAS_HIP_ERR_INVALID, "too many hidden arguments: %u", s->hidden);
  if (s->kind == EAS_HIP_KIND_RAW) return EAS_HIP_OK;
  if (s->block_size == 0 || s->wg_size == 0 || s->wg_size > 1024 || s->programs_per_wg == 0 || s->split == 0)
    return fail(EAS_HIP_ERR_INVALID, "launch shape has a zero or oversized dimension");
  if ((s->kind == EAS_HIP_KIND_SPMD || s->kind == EAS_HIP_KIND_THREAD) && s->hidden != 1)
    return fail(EAS_HIP_ERR_INVALID, "spmd and thread kernels take exactly one hidden extent");
  if (s->kind == EAS_HIP_KIND_GEMM && s->hidden != 4)
    return fail(EAS_HIP_ERR_INVALID, "a lifted GEMM takes four hidden extents (m_lo, m_hi, n_lo, n_hi)");
  return EAS_HIP_OK;
}

using Items = std::vector<std::pair<std::string, std::string>>;

// The `key=value` items on the marker line `tag` of a generated source.
static int marker_items(const char* src, const char* tag, const char* label, Items& items) {
  const char* p = strstr(src, tag);
  if (!p) return fail(EAS_HIP_ERR_INVALID, "source has no '%s' line", tag);
  p += strlen(tag);
  const char* end = strchr(p, '\n');
  std::string line(p, end ? (size_t)(end - p) : strlen(p));
  size_t pos = 0;
  while (pos < line.size()) {
    while (pos < line.size() && line[pos] == ' ') ++pos;
    size_t stop = line.find(' ', pos);
    std::string item = line.substr(pos, stop == std::string::npos ? std::string::npos : stop - pos);
    pos = stop == std::string::npos ? line.size() : stop;
    if (item.empty()) continue;
    size_t eq = item.find('=');
    if (eq == std::string::npos) return fail(EAS_HIP_ERR_INVALID, "malformed %s item '%s'", label, item.c_str());
    items.emplace_back(item.substr(0, eq), item.substr(eq + 1));
  }
  return EAS_HIP_OK;
}

// A decimal u32 (digits only).
static bool parse_u32(const std::string& val, uint32_t* out) {
  if (val.empty() || val.size() > 10) return false;
  uint64_t v = 0;
  for (char c : val) {
    if (c < '0' || c > '9') return false;
    v = v * 10 + (uint64_t)(c - '0');
  }
  if (v > 0xFFFFFFFFull) return false;
  *out = (uint32_t)v;
  return true;
}

int eas_hip_launch_shape_parse(const char* src, eas_hip_launch_shape* out) {
  if (!src || !out) return fail(EAS_HIP_ERR_INVALID, "src/out must not be NULL");
  Items items;
  int rc = marker_items(src, "// eas-launch:", "eas-launch", items);
  if (rc) return rc;
  eas_hip_launch_shape s{};
  s.programs_per_wg = 1;
  s.split = 1;
  bool have_kind = false;
  for (const auto& [key, val] : items) {
    if (key == "kind") {
      have_kind = true;
      if (val == "spmd") s.kind = EAS_HIP_KIND_SPMD;
      else if (val == "thread") s.kind = EAS_HIP_KIND_THREAD;
      else if (val == "gemm") s.kind = EAS_HIP_KIND_GEMM;
      else if (val == "raw") s.kind = EAS_HIP_KIND_RAW;
      else return fail(EAS_HIP_ERR_INVALID, "unknown eas-launch kind '%s'", val.c_str());
      continue;
    }
    uint32_t v;
    if (!parse_u32(val, &v)) return fail(EAS_HIP_ERR_INVALID, "bad eas-launch value '%s=%s'", key.c_str(), val.c_str());
    if (key == "block") s.block_size = v;
    else if (key == "wg") s.wg_size = v;
    else if (key == "ppw") s.programs_per_wg = v;
    else if (key == "split") s.split = v;
    else if (key == "args") s.arg_bytes = v;
    else if (key == "hidden") s.hidden = v;
    else return fail(EAS_HIP_ERR_INVALID, "unknown eas-launch key '%s'", key.c_str());
  }
  if (!have_kind) return fail(EAS_HIP_ERR_INVALID, "eas-launch line has no kind");
  rc = check_shape(&s);
  if (rc) return rc;
  *out = s;
  return EAS_HIP_OK;
}

int eas_hip_kernel_set_shape(eas_hip_kernel* k, const eas_hip_launch_shape* shape) {
  if (!k) return fail(EAS_HIP_ERR_INVALID, "kernel must not be NULL");
  int rc = check_shape(shape);
  if (rc) return rc;
  k->shape = *shape;
  if (shape->kind != EAS_HIP_KIND_GEMM) k->has_gemm = false;
  return EAS_HIP_OK;
}

int eas_hip_kernel_get_shape(const eas_hip_kernel* k, eas_hip_launch_shape* out) {
  if (!k || !out) return fail(EAS_HIP_ERR_INVALID, "kernel/out must not be NULL");
  *out = k->shape;
  return EAS_HIP_OK;
}

// ---- lifted GEMMs ------------------------------------------------------------

static const char* const kGemmSuffix[EAS_HIP_GEMM_NENTRIES] = {"", "__pp", "__t128", "__t128x256", "__t128x64",
                                                               "__t64x64"};

static int check_gemm(const eas_hip_gemm_shape* g) {
  if (!g) return fail(EAS_HIP_ERR_INVALID, "GEMM shape must not be NULL");
  const size_t len = strnlen(g->entry, sizeof(g->entry));
  if (len == 0 || len == sizeof(g->entry)) return fail(EAS_HIP_ERR_INVALID, "GEMM shape has no entry name");
  for (size_t i = 0; i < len; ++i) {
    const char c = g->entry[i];
    if (!(c == '_' || (c >= '0' && c <= '9') || (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z')))
      return fail(EAS_HIP_ERR_INVALID, "GEMM entry name '%s' is not an identifier", g->entry);
  }
  if (!(g->entries & 1u) || g->entries >> EAS_HIP_GEMM_NENTRIES)
    return fail(EAS_HIP_ERR_INVALID, "GEMM entry mask %#x must hold the kernel's own entry and no unknown one", g->entries);
  if (!g->K || !g->tm || !g->tn || !g->bm || !g->bn || !g->skinny_n || g->row_axis > 1)
    return fail(EAS_HIP_ERR_INVALID, "GEMM shape has a zero tile, K or skinny width, or a row axis other than 0 or 1");
  for (uint32_t t : {g->threads, g->pp_threads, g->t128_threads})
    if (!t || t > 1024 || t % 64) return fail(EAS_HIP_ERR_INVALID, "GEMM workgroup size %u is not 64..1024 in waves", t);
  for (uint32_t e : {g->a_elem, g->b_elem, g->c_elem})
    if (e != 2 && e != 4) return fail(EAS_HIP_ERR_INVALID, "GEMM element size %u is not 2 or 4", e);
  if (g->ldb_off < 0) return fail(EAS_HIP_ERR_INVALID, "GEMM shape has no N (row stride) argument");
  for (int32_t off : {g->m_off, g->ldb_off, g->row_base_off, g->col_base_off})
    if (off >= 0 && off % 4) return fail(EAS_HIP_ERR_INVALID, "GEMM scalar offset %d is not u32-aligned", off);
  if (g->a_off % 8 || g->b_off % 8) return fail(EAS_HIP_ERR_INVALID, "GEMM buffer offsets must be pointer-aligned");
  return EAS_HIP_OK;
}

int eas_hip_gemm_shape_parse(const char* src, eas_hip_gemm_shape* out) {
  if (!src || !out) return fail(EAS_HIP_ERR_INVALID, "src/out must not be NULL");
  Items items;
  int rc = marker_items(src, "// eas-gemm:", "eas-gemm", items);
  if (rc) return rc;
  eas_hip_gemm_shape g{};
  g.m_off = g.ldb_off = g.row_base_off = g.col_base_off = -1;
  struct U32 {
    const char* key;
    uint32_t* dst;
    bool seen;
  } u32s[] = {{"entries", &g.entries, false}, {"K", &g.K, false}, {"tm", &g.tm, false},
              {"tn", &g.tn, false}, {"row_axis", &g.row_axis, false}, {"bm", &g.bm, false},
              {"bn", &g.bn, false}, {"threads", &g.threads, false}, {"pp_threads", &g.pp_threads, false},
              {"t128_threads", &g.t128_threads, false}, {"skinny_m", &g.skinny_m, false},
              {"skinny_n", &g.skinny_n, false}, {"skinny_cut", &g.skinny_cut, false},
              {"wide_m", &g.wide_m, false}, {"f32", &g.f32, false}, {"col_masked", &g.col_masked, false},
              {"a", &g.a_arg, false}, {"b", &g.b_arg, false}, {"c", &g.c_arg, false},
              {"a_off", &g.a_off, false}, {"b_off", &g.b_off, false}, {"a_elem", &g.a_elem, false},
              {"b_elem", &g.b_elem, false}, {"c_elem", &g.c_elem, false}};
  struct Off {
    const char* key;
    int32_t* dst;
  } offs[] = {{"m", &g.m_off}, {"ldb", &g.ldb_off}, {"row_base", &g.row_base_off}, {"col_base", &g.col_base_off}};
  bool have_entry = false;
  for (const auto& [key, val] : items) {
    if (key == "entry") {
      if (val.size() >= sizeof(g.entry)) return fail(EAS_HIP_ERR_INVALID, "eas-gemm entry name too long");
      memcpy(g.entry, val.c_str(), val.size() + 1);
      have_entry = true;
      continue;
    }
    uint32_t v;
    if (!parse_u32(val, &v)) return fail(EAS_HIP_ERR_INVALID, "bad eas-gemm value '%s=%s'", key.c_str(), val.c_str());
    bool known = false;
    for (auto& u : u32s)
      if (key == u.key) {
        *u.dst = v;
        u.seen = known = true;
      }
    for (auto& o : offs)
      if (key == o.key) {
        if (v > 0x7FFFFFFFu) return fail(EAS_HIP_ERR_INVALID, "eas-gemm offset '%s' too large", key.c_str());
        *o.dst = (int32_t)v;
        known = true;
      }
    if (!known) return fail(EAS_HIP_ERR_INVALID, "unknown eas-gemm key '%s'", key.c_str());
  }
  if (!have_entry) return fail(EAS_HIP_ERR_INVALID, "eas-gemm line has no entry");
  for (const auto& u : u32s)
    if (!u.seen) return fail(EAS_HIP_ERR_INVALID, "eas-gemm line lacks '%s'", u.key);
  rc = check_gemm(&g);
  if (rc) return rc;
  *out = g;
  return EAS_HIP_OK;
}

int eas_hip_kernel_set_gemm(eas_hip_kernel* k, const eas_hip_gemm_shape* g) {
  if (!k) return fail(EAS_HIP_ERR_INVALID, "kernel must not be NULL");
  if (k->shape.kind != EAS_HIP_KIND_GEMM)
    return fail(EAS_HIP_ERR_INVALID, "the kernel's launch shape is not a lifted GEMM's (set its eas-launch shape first)");
  int rc = check_gemm(g);
  if (rc) return rc;
  hipFunction_t fn[EAS_HIP_GEMM_NENTRIES] = {};
  for (int e = 0; e < EAS_HIP_GEMM_NENTRIES; ++e) {
    if (!(g->entries >> e & 1u)) continue;
    const std::string name = std::string(g->entry) + kGemmSuffix[e];
    hipError_t err = hipModuleGetFunction(&fn[e], k->module, name.c_str());
    if (err != hipSuccess)
      return fail(EAS_HIP_ERR_RUNTIME, "GEMM entry point %s is not in the code object: %s", name.c_str(),
                  hipGetErrorString(err));
  }
  int cus = 0;
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, k->device));
  k->gemm = *g;
  memcpy(k->gemm_fn, fn, sizeof(fn));
  k->compute_units = cus;
  k->has_gemm = true;
  return EAS_HIP_OK;
}

namespace {

using u128 = unsigned __int128;

enum Choice { kAuto, k8Wave, kTile128, kTile128x256, kTile128x64, kTile64, k4Wave, kChoices };
const char* const kChoiceNames[kChoices] = {"auto", "8wave", "tile128", "tile128x256", "tile128x64", "tile64", "4wave"};

// The entry override: `choice`, or EAS_HIP_GEMM_ENTRY when NULL; blank means auto.
int entry_choice(const char* choice, int* out) {
  const char* raw = choice ? choice : getenv("EAS_HIP_GEMM_ENTRY");
  std::string v = raw ? raw : "";
  const size_t b = v.find_first_not_of(" \t\n\r\f\v"), e = v.find_last_not_of(" \t\n\r\f\v");
  v = b == std::string::npos ? std::string() : v.substr(b, e - b + 1);
  for (char& c : v) c = (char)((c >= 'A' && c <= 'Z') ? c - 'A' + 'a' : c);
  if (v.empty()) v = "auto";
  for (int i = 0; i < kChoices; ++i)
    if (v == kChoiceNames[i]) {
      *out = i;
      return EAS_HIP_OK;
    }
  return fail(EAS_HIP_ERR_INVALID, "EAS_HIP_GEMM_ENTRY must be one of auto, 8wave, tile128, tile128x256, tile128x64, "
                                   "tile64, 4wave; got '%s'", v.c_str());
}

int read_arg(const void* kernarg, size_t size, int32_t off, size_t bytes, const char* what, uint64_t* v) {
  if (off < 0 || (size_t)off + bytes > size)
    return fail(EAS_HIP_ERR_INVALID, "the packed arguments (%zu bytes) do not hold %s at byte %d", size, what, off);
  uint64_t x = 0;
  memcpy(&x, static_cast<const char*>(kernarg) + off, bytes);
  *v = x;
  return EAS_HIP_OK;
}

// Whether the DMA entries take the launch: every row of A and B (after the move to the
// rectangle's origin) 4-byte aligned for 16-bit operands, 16-byte aligned for fp32; each
// operand's extent under 2 GiB; A and B at such an alignment.
bool dma_fits(uint64_t a_ptr, uint64_t b_ptr, uint64_t K, uint64_t ldb, uint64_t m, uint64_t n_lo, uint64_t n,
              uint64_t elem) {
  const uint64_t step = elem == 2 ? 2 : 4;
  if (K % step || ldb % step || n_lo % step) return false;
  if ((u128)m * K * elem >= ((u128)1 << 31) || ((u128)(K - 1) * ldb + n) * elem >= ((u128)1 << 31)) return false;
  const uint64_t align = elem == 2 ? 4 : 16;
  return a_ptr % align == 0 && b_ptr % align == 0;
}

uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

}  // namespace

int eas_hip_plan_gemm(const eas_hip_launch_shape* s, const eas_hip_gemm_shape* g, const void* kernarg,
                      size_t kernarg_size, const uint64_t* arg_bytes, int nargs, int by_groups, const uint64_t size[3],
                      const uint32_t tptg[3], int compute_units, const char* choice, eas_hip_gemm_plan* out) {
  int rc = check_shape(s);
  if (rc) return rc;
  if (s->kind != EAS_HIP_KIND_GEMM) return fail(EAS_HIP_ERR_INVALID, "the kernel is not a lifted GEMM");
  rc = check_gemm(g);
  if (rc) return rc;
  if (!size || !tptg || !out) return fail(EAS_HIP_ERR_INVALID, "size/tptg/out must not be NULL");
  if (kernarg_size && !kernarg) return fail(EAS_HIP_ERR_INVALID, "kernarg is NULL with nonzero size");
  if (compute_units <= 0) return fail(EAS_HIP_ERR_INVALID, "compute_units must be > 0");
  const char* what = by_groups ? "threadgroups" : "threads_per_grid";
  for (int i = 0; i < 3; ++i)
    if (size[i] == 0) return fail(EAS_HIP_ERR_INVALID, "%s dims must be > 0", what);
  const bool auto_tg = tptg[0] == 0 && tptg[1] == 0 && tptg[2] == 0;
  if (!auto_tg && (tptg[0] != s->block_size || tptg[1] != 1 || tptg[2] != 1))
    return fail(EAS_HIP_ERR_INVALID, "threads_per_threadgroup must be (%u, 1, 1) for this kernel, which was compiled "
                                     "for BLOCK=%u threadgroups; got (%u, %u, %u)",
                s->block_size, s->block_size, tptg[0], tptg[1], tptg[2]);
  uint64_t groups[3] = {size[0], size[1], size[2]};
  if (!by_groups) {
    // the lift proved what whole threadgroups compute; a partial last one is another kernel
    if (size[0] % s->block_size)
      return fail(EAS_HIP_ERR_INVALID, "a lifted GEMM kernel runs whole threadgroups of %u threads: threads_per_grid "
                                       "x = %llu is not a multiple of it", s->block_size, (unsigned long long)size[0]);
    groups[0] = size[0] / s->block_size;
  }
  int ch = kAuto;
  rc = entry_choice(choice, &ch);
  if (rc) return rc;
  uint64_t ldb = 0, M = 0, rb = 0, cb = 0, a_ptr = 0, b_ptr = 0;
  if ((rc = read_arg(kernarg, kernarg_size, g->ldb_off, 4, "N", &ldb)) ||
      (g->m_off >= 0 && (rc = read_arg(kernarg, kernarg_size, g->m_off, 4, "M", &M))) ||
      (g->row_base_off >= 0 && (rc = read_arg(kernarg, kernarg_size, g->row_base_off, 4, "the row base", &rb))) ||
      (g->col_base_off >= 0 && (rc = read_arg(kernarg, kernarg_size, g->col_base_off, 4, "the column base", &cb))) ||
      (rc = read_arg(kernarg, kernarg_size, (int32_t)g->a_off, 8, "A", &a_ptr)) ||
      (rc = read_arg(kernarg, kernarg_size, (int32_t)g->b_off, 8, "B", &b_ptr)))
    return rc;
  const u128 g_rows = groups[g->row_axis], g_cols = groups[1 - g->row_axis];
  u128 m_lo = (u128)g->tm * rb, n_lo = (u128)g->tn * cb;
  u128 m_hi = m_lo + g_rows * g->tm, n_hi = n_lo + g_cols * g->tn;
  if (g->m_off >= 0 && m_hi > M) m_hi = M;
  if (g->col_masked && n_hi > ldb) n_hi = ldb;
  *out = eas_hip_gemm_plan{};
  if (m_hi <= m_lo || n_hi <= n_lo) return EAS_HIP_OK;  // no element of C: nothing to run
  const u128 K = g->K, wide = n_hi > ldb ? n_hi : (u128)ldb, lim = (u128)1 << 32;
  if (m_hi * K >= lim || K * wide >= lim || m_hi * wide >= lim)
    return fail(EAS_HIP_ERR_INVALID, "lifted GEMM: matrix too large for u32 indexing");
  if (!arg_bytes)
    return fail(EAS_HIP_ERR_INVALID, "a lifted GEMM's launch needs the byte length of each buffer argument (arg_bytes)");
  const struct {
    const char* name;
    uint32_t arg, elem;
    u128 need;
  } bufs[] = {{"A", g->a_arg, g->a_elem, m_hi * K},
              {"B", g->b_arg, g->b_elem, (K - 1) * ldb + n_hi},
              {"C", g->c_arg, g->c_elem, (m_hi - 1) * ldb + n_hi}};
  for (const auto& b : bufs) {
    if (nargs < 0 || b.arg >= (uint32_t)nargs)
      return fail(EAS_HIP_ERR_INVALID, "arg_bytes holds %d entries; %s is argument %u", nargs, b.name, b.arg);
    const uint64_t have = arg_bytes[b.arg] / b.elem;
    if (have < b.need)
      return fail(EAS_HIP_ERR_INVALID, "buffer %s (argument %u) holds %llu elements; this launch touches %llu", b.name,
                  b.arg, (unsigned long long)have, (unsigned long long)b.need);
  }
  const uint64_t m = (uint64_t)(m_hi - m_lo), n = (uint64_t)(n_hi - n_lo), cus = (uint64_t)compute_units;
  const uint64_t tiles = cdiv(m, g->bm) * cdiv(n, g->bn), tiles128 = cdiv(m, 128) * cdiv(n, 128);
  const uint64_t tiles128x256 = cdiv(m, 128) * cdiv(n, 256), tiles128x64 = cdiv(m, 128) * cdiv(n, 64);
  const uint64_t tiles64 = cdiv(m, 64) * cdiv(n, 64);
  const uint64_t elem = g->f32 ? 4 : 2;
  auto has = [&](int e) { return (g->entries >> e & 1u) != 0; };
  auto fits = [&] { return dma_fits(a_ptr, b_ptr, g->K, ldb, m, (uint64_t)n_lo, n, elem); };
  int entry = EAS_HIP_GEMM_MAIN;
  uint64_t wgs = tiles;
  uint32_t threads = g->threads;
  auto pick = [&](int e, uint64_t w, uint32_t t) {
    entry = e;
    wgs = w;
    threads = t;
  };
  if (m <= g->skinny_m) {
    // The 4-wave entry runs its skinny path for every launch of at most skinny_m rows (one
    // workgroup per skinny_n columns, all rows), so it is only ever launched on that grid.  Up to
    // wide_m rows, a launch whose groups would take more than one round of CUs gets twice the
    // columns per workgroup (the kernel reads which from the grid).  Above skinny_cut rows, a
    // launch whose groups still take more than one round goes to the 128 x 128 entry instead.
    uint64_t grp = cdiv(n, g->skinny_n);
    if (m <= g->wide_m && grp > cus) grp = cdiv(n, 2ull * g->skinny_n);
    pick(EAS_HIP_GEMM_MAIN, grp, g->threads);
    if (m > g->skinny_cut && has(EAS_HIP_GEMM_PP) && fits()) {
      if (ch == kTile128 || (ch == kAuto && grp > cus)) pick(EAS_HIP_GEMM_T128, tiles128, g->t128_threads);
      else if (ch == kTile128x256) pick(EAS_HIP_GEMM_T128X256, tiles128x256, g->t128_threads);
      else if (ch == kTile128x64) pick(EAS_HIP_GEMM_T128X64, tiles128x64, g->t128_threads);
      else if (ch == kTile64) pick(EAS_HIP_GEMM_T64X64, tiles64, g->t128_threads);
      else if (ch == k8Wave) pick(EAS_HIP_GEMM_PP, tiles, g->pp_threads);
    }
  } else if (g->f32) {
    // fp32: 128 x 128 tiles (a quarter of the DMA bytes per flop) while they still give every CU one
    if (has(EAS_HIP_GEMM_T128) && fits() && (ch == kTile128 || (ch == kAuto && tiles128 >= cus)))
      pick(EAS_HIP_GEMM_T128, tiles128, g->t128_threads);
  } else if (has(EAS_HIP_GEMM_PP) && ch != k4Wave && fits()) {
    // When 256 x 256 tiles would fill at most half of the CUs: 128 x 128 tiles if they take one
    // round of CUs, else 128 x 256 ones.  If even 128 x 128 would fill at most half of the CUs:
    // 64 x 64 tiles while they need at most 1.75 rounds of CUs, else 128 x 64.
    const bool small = ch == kAuto && 2 * tiles <= cus;
    const bool tiny = small && 2 * tiles128 <= cus;
    if (ch == kTile128x256 || (small && tiles128 > cus)) pick(EAS_HIP_GEMM_T128X256, tiles128x256, g->t128_threads);
    else if (ch == kTile64 || (tiny && 4 * tiles64 <= 7 * cus)) pick(EAS_HIP_GEMM_T64X64, tiles64, g->t128_threads);
    else if (ch == kTile128x64 || tiny) pick(EAS_HIP_GEMM_T128X64, tiles128x64, g->t128_threads);
    else if (ch == kTile128 || small) pick(EAS_HIP_GEMM_T128, tiles128, g->t128_threads);
    else pick(EAS_HIP_GEMM_PP, tiles, g->pp_threads);
  }
  if (!has(entry))
    return fail(EAS_HIP_ERR_INVALID, "GEMM entry %s%s is not in the code object", g->entry, kGemmSuffix[entry]);
  if (wgs * threads > 0xFFFFFFFFull) return fail(EAS_HIP_ERR_INVALID, "lifted GEMM launch exceeds 2^32 work-items");
  out->launch = 1;
  out->entry = entry;
  out->grid[0] = (uint32_t)wgs;
  out->grid[1] = out->grid[2] = 1;
  out->block[0] = threads;
  out->block[1] = out->block[2] = 1;
  out->hidden[0] = (uint32_t)m_lo;
  out->hidden[1] = (uint32_t)m_hi;
  out->hidden[2] = (uint32_t)n_lo;
  out->hidden[3] = (uint32_t)n_hi;
  return EAS_HIP_OK;
}

int eas_hip_plan_dispatch(const eas_hip_launch_shape* s, int by_groups, const uint64_t size[3], const uint32_t tptg[3],
                          uint32_t grid[3], uint32_t block[3], uint32_t* hidden, int max_hidden) {
  int rc = check_shape(s);
  if (rc) return rc;
  if (!size || !tptg || !grid || !block || (!hidden && s->hidden))
    return fail(EAS_HIP_ERR_INVALID, "size/tptg/grid/block/hidden must not be NULL");
  if (max_hidden < (int)s->hidden) return fail(EAS_HIP_ERR_INVALID, "hidden holds %d, the kernel needs %u", max_hidden, s->hidden);
  if (s->kind == EAS_HIP_KIND_RAW)
    return fail(EAS_HIP_ERR_INVALID, "the kernel's launch shape is unknown (a source without an eas-launch line): "
                                     "launch it with workgroup counts (launch_groups / eas_hip_launch)");
  if (s->kind == EAS_HIP_KIND_GEMM)
    return fail(EAS_HIP_ERR_INVALID, "a lifted GEMM's dispatch depends on M, N, K and its buffers: plan it with "
                                     "eas_hip_plan_gemm");
  const char* what = by_groups ? "threadgroups" : "threads_per_grid";
  for (int i = 0; i < 3; ++i)
    if (size[i] == 0) return fail(EAS_HIP_ERR_INVALID, "%s dims must be > 0", what);
  const bool auto_tg = tptg[0] == 0 && tptg[1] == 0 && tptg[2] == 0;
  if (s->kind == EAS_HIP_KIND_THREAD) {
    if (!auto_tg && (tptg[0] != s->block_size || tptg[1] != 1 || tptg[2] != 1))
      return fail(EAS_HIP_ERR_INVALID, "threads_per_threadgroup must be (%u, 1, 1) for this kernel, which was compiled "
                                       "for BLOCK=%u threadgroups; got (%u, %u, %u)",
                  s->block_size, s->block_size, tptg[0], tptg[1], tptg[2]);
    // bounded before multiplying, so a huge threadgroup count cannot wrap past the checks
    if (by_groups && size[0] > 0xFFFFFFFFull / s->block_size)
      return fail(EAS_HIP_ERR_INVALID, "%s x exceeds 2^32 threads", what);
    uint64_t groups_x = by_groups ? size[0] : (size[0] + s->block_size - 1) / s->block_size;
    uint64_t live = by_groups ? size[0] * s->block_size : size[0];
    if (live > 0xFFFFFFFFull || groups_x * s->block_size > 0xFFFFFFFFull)
      return fail(EAS_HIP_ERR_INVALID, "%s x exceeds 2^32 threads", what);
    // one workgroup per threadgroup (programs_per_wg = split = 1, wg_size = BLOCK), or a kernel
    // emitted as lanes: threadgroups mapped like SPMD programs
    grid[0] = (uint32_t)((groups_x + s->programs_per_wg - 1) / s->programs_per_wg * s->split);
    hidden[0] = (uint32_t)live;
  } else {
    // SPMD: a Metal thread is a program; the reference dispatches them as threads with
    // threadgroups of one (eas/runtime/metal.py:284-295), so both forms count programs
    if (!auto_tg && (tptg[0] != 1 || tptg[1] != 1 || tptg[2] != 1))
      return fail(EAS_HIP_ERR_INVALID, "threads_per_threadgroup must be (1, 1, 1) for an SPMD kernel (one program per "
                                       "Metal thread); got (%u, %u, %u)", tptg[0], tptg[1], tptg[2]);
    if (size[0] > 0xFFFFFFFFull) return fail(EAS_HIP_ERR_INVALID, "%s x exceeds 2^32 programs", what);
    uint64_t groups_x = (size[0] + s->programs_per_wg - 1) / s->programs_per_wg * s->split;
    if (groups_x * s->wg_size > 0xFFFFFFFFull) return fail(EAS_HIP_ERR_INVALID, "%s x exceeds 2^32 threads", what);
    grid[0] = (uint32_t)groups_x;
    hidden[0] = (uint32_t)size[0];
  }
  for (int i = 1; i < 3; ++i) {
    if (size[i] > 0xFFFFFFFFull) return fail(EAS_HIP_ERR_INVALID, "%s dim %d too large", what, i);
    grid[i] = (uint32_t)size[i];
  }
  block[0] = s->wg_size;
  block[1] = block[2] = 1;
  return EAS_HIP_OK;
}

// Size of the blob a launch of `k` must carry: its own arguments, padded to 4 bytes when
// hidden u32 extents follow (0 when the shape does not record it).
static size_t expected_kernarg(const eas_hip_launch_shape& s, bool with_hidden) {
  if (!s.arg_bytes) return 0;
  if (!with_hidden || !s.hidden) return s.arg_bytes;
  return ((size_t)s.arg_bytes + 3) / 4 * 4 + 4 * (size_t)s.hidden;
}

// A workgroup-level launch carries the kernel's arguments and its hidden extents.
static int check_group_blob(const eas_hip_kernel* k, size_t kernarg_size) {
  if (!k) return EAS_HIP_OK;  // launch_n reports it
  size_t want = expected_kernarg(k->shape, true);
  if (want && kernarg_size != want)
    return fail(EAS_HIP_ERR_INVALID, "kernel argument blob of %zu bytes does not match the kernel's parameters "
                                     "(%u bytes of arguments, then %u hidden u32: %zu bytes)",
                kernarg_size, k->shape.arg_bytes, k->shape.hidden, want);
  return EAS_HIP_OK;
}

int eas_hip_launch(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                   const uint32_t block[3], uint32_t dynamic_lds, void* stream, int repeat) {
  if (repeat <= 0) return fail(EAS_HIP_ERR_INVALID, "repeat must be > 0");
  int rc = check_group_blob(k, kernarg_size);
  if (rc) return rc;
  return launch_n(k, kernarg, kernarg_size, grid, block, dynamic_lds, stream, repeat);
}

static int launch_reference(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size,
                            const uint64_t* arg_bytes, int nargs, int by_groups, const uint64_t size[3],
                            const uint32_t tptg[3], void* stream, int repeat) {
  if (!k) return fail(EAS_HIP_ERR_INVALID, "kernel must not be NULL");
  if (repeat <= 0) return fail(EAS_HIP_ERR_INVALID, "repeat must be > 0");
  static const uint32_t kAuto[3] = {0, 0, 0};
  const size_t want = expected_kernarg(k->shape, false);
  if (want && kernarg_size != want)
    return fail(EAS_HIP_ERR_INVALID, "kernel argument blob of %zu bytes does not match the kernel's %u bytes of "
                                     "arguments (the hidden extents are appended by the launch)",
                kernarg_size, k->shape.arg_bytes);
  if (kernarg_size && !kernarg) return fail(EAS_HIP_ERR_INVALID, "kernarg is NULL with nonzero size");
  uint32_t grid[3], block[3], hidden[EAS_HIP_MAX_HIDDEN];
  hipFunction_t fn = k->function;
  if (k->shape.kind == EAS_HIP_KIND_GEMM) {
    if (!k->has_gemm)
      return fail(EAS_HIP_ERR_INVALID, "this lifted GEMM kernel has no GEMM shape attached (eas_hip_kernel_set_gemm "
                                       "with its source's eas-gemm line)");
    eas_hip_gemm_plan plan;
    int rc = eas_hip_plan_gemm(&k->shape, &k->gemm, kernarg, kernarg_size, arg_bytes, nargs, by_groups, size,
                               tptg ? tptg : kAuto, k->compute_units, nullptr, &plan);
    if (rc) return rc;
    if (!plan.launch) return EAS_HIP_OK;
    memcpy(grid, plan.grid, sizeof(grid));
    memcpy(block, plan.block, sizeof(block));
    memcpy(hidden, plan.hidden, sizeof(plan.hidden));
    fn = k->gemm_fn[plan.entry];
  } else {
    int rc = eas_hip_plan_dispatch(&k->shape, by_groups, size, tptg ? tptg : kAuto, grid, block, hidden,
                                   EAS_HIP_MAX_HIDDEN);
    if (rc) return rc;
  }
  std::vector<uint8_t> blob((kernarg_size + 3) / 4 * 4 + 4 * k->shape.hidden, 0);
  if (kernarg_size) memcpy(blob.data(), kernarg, kernarg_size);
  memcpy(blob.data() + (kernarg_size + 3) / 4 * 4, hidden, 4 * k->shape.hidden);
  return launch_fn(fn, blob.data(), blob.size(), grid, block, 0, stream, repeat);
}

int eas_hip_launch_threads(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint64_t* arg_bytes,
                           int nargs, const uint64_t threads_per_grid[3], const uint32_t threads_per_threadgroup[3],
                           void* stream, int repeat) {
  return launch_reference(k, kernarg, kernarg_size, arg_bytes, nargs, 0, threads_per_grid, threads_per_threadgroup,
                          stream, repeat);
}

int eas_hip_launch_threadgroups(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size,
                                const uint64_t* arg_bytes, int nargs, const uint64_t threadgroups[3],
                                const uint32_t threads_per_threadgroup[3], void* stream, int repeat) {
  return launch_reference(k, kernarg, kernarg_size, arg_bytes, nargs, 1, threadgroups, threads_per_threadgroup, stream,
                          repeat);
}

int eas_hip_launch_timed(const eas_hip_kernel* k, const void* kernarg, size_t kernarg_size, const uint32_t grid[3],
                         const uint32_t block[3], uint32_t dynamic_lds, void* stream, int warmup, int repeat,
                         float* mean_ms) {
  if (repeat <= 0 || warmup < 0 || !mean_ms) return fail(EAS_HIP_ERR_INVALID, "repeat > 0, warmup >= 0, mean_ms required");
  int crc = check_group_blob(k, kernarg_size);
  if (crc) return crc;
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
