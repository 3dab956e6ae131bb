// hip_module.cpp — CPython binding `easy_as_amd._hip` over the C ABI in
// include/eas_hip.h.
//
// It exposes the method names the reference runtime requires of its native
// module (eas/runtime/metal_ext.py:22-33: is_available, compile, launch,
// synchronize, alloc_buffer, copy_from_host, copy_to_host, dlpack_import,
// dlpack_export, queue_synchronize) plus launch_async / launch_tg /
// launch_tg_async, and the HIP-specific compile_to_code / load / launch_groups
// / launch_groups_async / launch_timed / wrap_pointer / device_props /
// kernel_attrs / kernel_shape / launch_shape / plan_dispatch.
//
// Objects crossing into Python are PyCapsules:
//   "eas._hip.kernel"  -> eas_hip_kernel*       (module unloaded on destruction)
//   "eas._hip.buffer"  -> Buffer                (memory freed / DLPack deleter run)
//   "eas._hip.pending" -> Pending               (completion batch + keepalives of a launch)
// launch/launch_tg take the reference's thread and threadgroup counts and plan the
// workgroups from the kernel's launch shape (the C ABI appends the hidden extents
// that stand in for Metal's non-uniform dispatchThreads); launch_groups takes HIP
// workgroups directly, as the Python runtime plans every launch itself.

#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "eas_hip.h"

namespace {

const char* kKernelCap = "eas._hip.kernel";
const char* kBufferCap = "eas._hip.buffer";
const char* kPendingCap = "eas._hip.pending";

struct Buffer {
  void* ptr;
  size_t nbytes;
  int storage;         // EAS_HIP_STORAGE_*
  bool owns;           // free with eas_hip_free on destruction
  void* dl_managed;    // imported DLManagedTensor to delete on destruction
  PyObject* owner;     // object kept alive by a wrapped pointer
};

// Async launches on one stream share completion events.  Consecutive launches on a stream
// join its open batch, whose event is recorded after the batch's last permitted launch (at
// most kBatchLaunches, fewer when the caller asks: `batch=`), when a launch arrives on another
// stream, or as soon as someone waits on a launch in it; the stream runs in order, so that
// event marks the completion of every launch in the batch.  Waiting on a pending launch
// therefore also waits for the later launches of its batch, and for any other work queued on
// that stream before the event was recorded.  At most one batch is open, and its stream is
// the one the latest async launch used, so the event is recorded on a stream that was in use
// moments before (a caller that destroys a stream must first wait on its pending launches).
// On MI355X recording an event costs ~4.5 us of host time against ~2.7 us for the launch
// itself, so one event per launch would almost triple the cost of an async call.  All batch
// state is touched with the GIL held.
struct Batch {
  void* stream;
  void* event;     // recorded completion event (nullptr while open, or if recording failed)
  int launches;
  int limit;       // launches after which the batch closes
  int refs;        // unreleased pending capsules in this batch
  bool closed;     // no further launches join it
};
constexpr int kBatchLaunches = 16;
std::vector<Batch*> g_open_batches;  // the open batch (at most one)

struct Pending {
  Batch* batch;    // nullptr once released
  std::vector<PyObject*> keepalive;
};

PyObject* raise_status(int rc) {
  PyObject* exc = PyExc_RuntimeError;
  if (rc == EAS_HIP_ERR_INVALID) exc = PyExc_ValueError;
  if (rc == EAS_HIP_ERR_NOMEM) exc = PyExc_MemoryError;
  PyErr_SetString(exc, eas_hip_last_error());
  return nullptr;
}

void kernel_destructor(PyObject* cap) {
  auto* k = static_cast<eas_hip_kernel*>(PyCapsule_GetPointer(cap, kKernelCap));
  if (k) eas_hip_kernel_release(k);
  else PyErr_Clear();
}

void buffer_destructor(PyObject* cap) {
  auto* b = static_cast<Buffer*>(PyCapsule_GetPointer(cap, kBufferCap));
  if (!b) {
    PyErr_Clear();
    return;
  }
  if (b->dl_managed) eas_hip_dlpack_delete(b->dl_managed);
  else if (b->owns) eas_hip_free(b->ptr, b->storage);
  Py_XDECREF(b->owner);
  delete b;
}

// Completion events of async launches are reused: an event whose wait succeeded goes back to
// this pool (touched only with the GIL held), so a launch does not create and destroy one.
std::vector<void*> g_event_pool;
constexpr size_t kEventPoolMax = 64;

int acquire_event(void** ev) {
  if (!g_event_pool.empty()) {
    *ev = g_event_pool.back();
    g_event_pool.pop_back();
    return EAS_HIP_OK;
  }
  return eas_hip_event_create(ev);
}

void recycle_event(void* ev, bool ok) {
  if (ok && g_event_pool.size() < kEventPoolMax) g_event_pool.push_back(ev);
  else eas_hip_event_destroy(ev);
}

int close_batch(Batch* b);

// The batch a launch just enqueued on `stream` belongs to: the open one if it is that
// stream's (an open batch of another stream is closed first), else a new one that closes
// after `limit` launches.  *rc receives the status of closing the other stream's batch.
Batch* join_batch(void* stream, int limit, int* rc) {
  *rc = EAS_HIP_OK;
  while (!g_open_batches.empty()) {
    Batch* b = g_open_batches.back();
    if (b->stream == stream) {
      ++b->launches;
      ++b->refs;
      return b;
    }
    int crc = close_batch(b);  // removes it from g_open_batches
    if (!*rc) *rc = crc;
  }
  auto* b = new Batch{stream, nullptr, 1, limit, 1, false};
  g_open_batches.push_back(b);
  return b;
}

// Record the batch's completion event on its stream; later launches start a new batch.
int close_batch(Batch* b) {
  for (size_t i = 0; i < g_open_batches.size(); ++i) {
    if (g_open_batches[i] == b) {
      g_open_batches.erase(g_open_batches.begin() + (std::ptrdiff_t)i);
      break;
    }
  }
  b->closed = true;
  void* ev = nullptr;
  int rc = acquire_event(&ev);
  if (!rc) {
    rc = eas_hip_event_record(ev, b->stream);
    if (rc) {
      recycle_event(ev, false);
      ev = nullptr;
    }
  }
  b->event = ev;
  return rc;
}

// Wait (GIL released) until the pending launch has completed, then drop its keepalives.
int release_pending(Pending* p) {
  int rc = EAS_HIP_OK;
  if (Batch* b = p->batch) {
    p->batch = nullptr;
    if (!b->closed) rc = close_batch(b);
    void* ev = b->event;
    void* stream = b->stream;
    int wrc;
    Py_BEGIN_ALLOW_THREADS
    // without an event (recording failed) the whole stream is waited on instead
    wrc = ev ? eas_hip_event_synchronize(ev) : eas_hip_stream_synchronize(stream);
    Py_END_ALLOW_THREADS
    if (!rc) rc = wrc;
    if (--b->refs == 0) {
      if (b->event) recycle_event(b->event, wrc == EAS_HIP_OK);
      delete b;
    }
  }
  for (PyObject* o : p->keepalive) Py_XDECREF(o);
  p->keepalive.clear();
  return rc;
}

void pending_destructor(PyObject* cap) {
  auto* p = static_cast<Pending*>(PyCapsule_GetPointer(cap, kPendingCap));
  if (!p) {
    PyErr_Clear();
    return;
  }
  release_pending(p);
  delete p;
}

Buffer* as_buffer(PyObject* obj) {
  if (!PyCapsule_IsValid(obj, kBufferCap)) return nullptr;
  return static_cast<Buffer*>(PyCapsule_GetPointer(obj, kBufferCap));
}

PyObject* new_buffer(void* ptr, size_t nbytes, int storage, bool owns, void* dl, PyObject* owner) {
  auto* b = new Buffer{ptr, nbytes, storage, owns, dl, owner};
  Py_XINCREF(owner);
  PyObject* cap = PyCapsule_New(b, kBufferCap, buffer_destructor);
  if (!cap) {
    Py_XDECREF(owner);
    delete b;
  }
  return cap;
}

bool parse_dim3(PyObject* obj, uint32_t out[3], const char* what) {
  out[0] = out[1] = out[2] = 1;
  if (PyLong_Check(obj)) {
    unsigned long long v = PyLong_AsUnsignedLongLong(obj);
    if (PyErr_Occurred()) return false;
    if (v > 0xFFFFFFFFull) {
      PyErr_Format(PyExc_OverflowError, "%s too large", what);
      return false;
    }
    out[0] = (uint32_t)v;
    return true;
  }
  PyObject* seq = PySequence_Fast(obj, "expected an int or a tuple/list of ints");
  if (!seq) return false;
  Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  if (n < 1 || n > 3) {
    Py_DECREF(seq);
    PyErr_Format(PyExc_ValueError, "%s must have 1..3 dims", what);
    return false;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* it = PySequence_Fast_GET_ITEM(seq, i);
    if (!PyLong_Check(it)) {
      Py_DECREF(seq);
      PyErr_Format(PyExc_TypeError, "%s dim %zd must be int", what, i);
      return false;
    }
    unsigned long long v = PyLong_AsUnsignedLongLong(it);
    if (PyErr_Occurred() || v > 0xFFFFFFFFull) {
      Py_DECREF(seq);
      if (!PyErr_Occurred()) PyErr_Format(PyExc_OverflowError, "%s too large", what);
      return false;
    }
    out[i] = (uint32_t)v;
  }
  Py_DECREF(seq);
  return true;
}

void append_aligned(std::vector<uint8_t>& blob, const void* data, size_t size, size_t align) {
  size_t off = (blob.size() + align - 1) / align * align;
  blob.resize(off + size);
  memcpy(blob.data() + off, data, size);
}

// Pack argv into a kernel-argument blob at natural alignment; buffer capsules
// become device pointers (and are appended to `keep`), bytes are copied raw,
// int -> u32, float -> f32.  `sizes` (when given) receives each item's buffer length,
// 0 for a scalar, as the reference's buffer objects carry theirs.  A NULL `writable_obj`
// marks every item read-only.  Mirrors bind_args_fast (_metal.mm:855-951).
bool pack_args(PyObject* argv_obj, PyObject* writable_obj, std::vector<uint8_t>& blob, std::vector<PyObject*>* keep,
               std::vector<uint64_t>* sizes = nullptr) {
  PyObject* argv = PySequence_Fast(argv_obj, "argv must be a sequence");
  if (!argv) return false;
  PyObject* writable = writable_obj ? PySequence_Fast(writable_obj, "writable must be a sequence") : nullptr;
  if (writable_obj && !writable) {
    Py_DECREF(argv);
    return false;
  }
  bool ok = true;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(argv);
  if (writable && PySequence_Fast_GET_SIZE(writable) != n) {
    PyErr_SetString(PyExc_ValueError, "writable must have same length as argv");
    ok = false;
  }
  for (Py_ssize_t i = 0; ok && i < n; ++i) {
    PyObject* obj = PySequence_Fast_GET_ITEM(argv, i);
    int want_write = writable ? PyObject_IsTrue(PySequence_Fast_GET_ITEM(writable, i)) : 0;
    if (want_write < 0) {
      ok = false;
      break;
    }
    if (sizes) sizes->push_back(0);
    if (Buffer* b = as_buffer(obj)) {
      uint64_t p = (uint64_t)(uintptr_t)b->ptr;
      append_aligned(blob, &p, 8, 8);
      if (sizes) sizes->back() = (uint64_t)b->nbytes;
      if (keep) {
        Py_INCREF(obj);
        keep->push_back(obj);
      }
      continue;
    }
    if (want_write) {
      PyErr_Format(PyExc_TypeError, "writable arg %zd must be a buffer capsule (use alloc_buffer/dlpack_import)", i);
      ok = false;
      break;
    }
    if (PyBytes_Check(obj) || PyByteArray_Check(obj)) {
      const char* data = PyBytes_Check(obj) ? PyBytes_AS_STRING(obj) : PyByteArray_AS_STRING(obj);
      Py_ssize_t len = PyBytes_Check(obj) ? PyBytes_GET_SIZE(obj) : PyByteArray_GET_SIZE(obj);
      if (len <= 0) {
        PyErr_SetString(PyExc_ValueError, "scalar bytes cannot be empty");
        ok = false;
        break;
      }
      size_t align = 1;
      while (align < 8 && (size_t)len % (align * 2) == 0) align *= 2;
      append_aligned(blob, data, (size_t)len, align);
      continue;
    }
    if (PyLong_Check(obj)) {
      unsigned long long v = PyLong_AsUnsignedLongLong(obj);
      if (PyErr_Occurred()) {
        ok = false;
        break;
      }
      if (v > 0xFFFFFFFFull) {
        PyErr_SetString(PyExc_OverflowError, "int scalar too large (expected uint32); pass bytes for larger types");
        ok = false;
        break;
      }
      uint32_t u = (uint32_t)v;
      append_aligned(blob, &u, 4, 4);
      continue;
    }
    if (PyFloat_Check(obj)) {
      float f = (float)PyFloat_AsDouble(obj);
      append_aligned(blob, &f, 4, 4);
      continue;
    }
    PyErr_Format(PyExc_TypeError, "unsupported arg %zd type (expected buffer capsule or scalar bytes/int/float)", i);
    ok = false;
  }
  Py_XDECREF(writable);
  Py_DECREF(argv);
  if (!ok && keep) {
    for (PyObject* o : *keep) Py_DECREF(o);
    keep->clear();
  }
  return ok;
}

eas_hip_kernel* as_kernel(PyObject* cap) {
  return static_cast<eas_hip_kernel*>(PyCapsule_GetPointer(cap, kKernelCap));
}

void* as_stream(PyObject* obj) {
  if (!obj || obj == Py_None) return nullptr;
  return PyLong_AsVoidPtr(obj);
}

// ---------------------------------------------------------------------------

PyObject* py_is_available(PyObject*, PyObject*) { return PyBool_FromLong(eas_hip_is_available()); }

PyObject* py_device_props(PyObject*, PyObject* args) {
  int dev = -1;
  if (!PyArg_ParseTuple(args, "|i", &dev)) return nullptr;
  eas_hip_device_props p;
  int rc = eas_hip_device_props_get(dev, &p);
  if (rc) return raise_status(rc);
  return Py_BuildValue("{s:s,s:i,s:i,s:i,s:i,s:K,s:K,s:i,s:i}", "arch", p.arch, "compute_units", p.compute_units,
                       "clock_khz", p.clock_khz, "memory_clock_khz", p.memory_clock_khz, "memory_bus_width",
                       p.memory_bus_width, "total_global_mem", (unsigned long long)p.total_global_mem, "lds_per_block",
                       (unsigned long long)p.lds_per_block, "warp_size", p.warp_size, "max_threads_per_block",
                       p.max_threads_per_block);
}

bool collect_options(PyObject* opts, std::vector<std::string>& store, std::vector<const char*>& ptrs) {
  if (!opts || opts == Py_None) return true;
  PyObject* seq = PySequence_Fast(opts, "options must be a sequence of str");
  if (!seq) return false;
  for (Py_ssize_t i = 0; i < PySequence_Fast_GET_SIZE(seq); ++i) {
    const char* s = PyUnicode_AsUTF8(PySequence_Fast_GET_ITEM(seq, i));
    if (!s) {
      Py_DECREF(seq);
      return false;
    }
    store.emplace_back(s);
  }
  Py_DECREF(seq);
  for (auto& s : store) ptrs.push_back(s.c_str());
  return true;
}

// compile_to_code(src, name, options) -> bytes (code object); no GPU required.
PyObject* py_compile_to_code(PyObject*, PyObject* args) {
  const char* src;
  const char* name;
  PyObject* opts = nullptr;
  if (!PyArg_ParseTuple(args, "ss|O", &src, &name, &opts)) return nullptr;
  std::vector<std::string> store;
  std::vector<const char*> ptrs;
  if (!collect_options(opts, store, ptrs)) return nullptr;
  void* code = nullptr;
  size_t size = 0;
  std::string log(1 << 16, '\0');
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = eas_hip_compile_source(src, name, ptrs.data(), (int)ptrs.size(), &code, &size, &log[0], log.size());
  Py_END_ALLOW_THREADS
  if (rc) {
    if (rc == EAS_HIP_ERR_COMPILE) {
      PyErr_Format(PyExc_RuntimeError, "HIP compile failed: %s\n%s", eas_hip_last_error(), log.c_str());
      return nullptr;
    }
    return raise_status(rc);
  }
  PyObject* out = PyBytes_FromStringAndSize(static_cast<const char*>(code), (Py_ssize_t)size);
  eas_hip_free_host(code);
  return out;
}

// compiler_version() -> (major, minor, path) of the hiprtc in use; no GPU required.
PyObject* py_compiler_version(PyObject*, PyObject*) {
  int major = 0, minor = 0;
  char path[1024];
  int rc = eas_hip_compiler_version(&major, &minor, path, sizeof(path));
  if (rc) {
    PyErr_Format(PyExc_RuntimeError, "%s", eas_hip_last_error());
    return nullptr;
  }
  return Py_BuildValue("(iis)", major, minor, path);
}

// Attach the launch shape on `src`'s eas-launch line to `k` (a source without one leaves the
// kernel's shape unknown: it then runs only through launch_groups), and a lifted GEMM's
// plan inputs on its eas-gemm line.
int attach_shape(eas_hip_kernel* k, const char* src) {
  if (!src || !strstr(src, "// eas-launch:")) return EAS_HIP_OK;
  eas_hip_launch_shape s;
  int rc = eas_hip_launch_shape_parse(src, &s);
  if (!rc) rc = eas_hip_kernel_set_shape(k, &s);
  if (rc || s.kind != EAS_HIP_KIND_GEMM) return rc;
  eas_hip_gemm_shape g;
  rc = eas_hip_gemm_shape_parse(src, &g);
  return rc ? rc : eas_hip_kernel_set_gemm(k, &g);
}

PyObject* new_kernel_capsule(eas_hip_kernel* k, const char* src) {
  int rc = attach_shape(k, src);
  if (rc) {
    eas_hip_kernel_release(k);
    return raise_status(rc);
  }
  PyObject* cap = PyCapsule_New(k, kKernelCap, kernel_destructor);
  if (!cap) eas_hip_kernel_release(k);
  return cap;
}

// load(code: bytes, name, src=None) -> kernel capsule; `src` (the source the code object was
// compiled from) gives the kernel its launch shape.
PyObject* py_load(PyObject*, PyObject* args, PyObject* kwargs) {
  static const char* kw[] = {"code", "name", "src", nullptr};
  Py_buffer code;
  const char* name;
  const char* src = nullptr;
  if (!PyArg_ParseTupleAndKeywords(args, kwargs, "y*s|z", const_cast<char**>(kw), &code, &name, &src)) return nullptr;
  eas_hip_kernel* k = nullptr;
  int rc = eas_hip_kernel_load(code.buf, (size_t)code.len, name, &k);
  PyBuffer_Release(&code);
  if (rc) return raise_status(rc);
  return new_kernel_capsule(k, src);
}

// compile(src, name, options=None) -> kernel capsule (reference: compile(msl, name))
// The options `compile` uses when given none: gfx950, -O3, FMAs only where the IR has
// them (no contraction), packed FP32 off.  Exposed as DEFAULT_OPTIONS; the Python
// runtime's COMPILE_OPTIONS are the same list (checked by the tests).
const char* const kDefaultOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                                       "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};

PyObject* default_options() {
  const Py_ssize_t n = (Py_ssize_t)(sizeof(kDefaultOptions) / sizeof(kDefaultOptions[0]));
  PyObject* t = PyTuple_New(n);
  for (Py_ssize_t i = 0; t && i < n; ++i) PyTuple_SET_ITEM(t, i, PyUnicode_FromString(kDefaultOptions[i]));
  return t;
}

PyObject* py_compile(PyObject* self, PyObject* args) {
  const char* src;
  const char* name;
  PyObject* opts = nullptr;
  if (!PyArg_ParseTuple(args, "ss|O", &src, &name, &opts)) return nullptr;
  PyObject* call = nullptr;
  if (!opts || opts == Py_None) {
    PyObject* defaults = default_options();
    if (!defaults) return nullptr;
    call = Py_BuildValue("(ssN)", src, name, defaults);
    if (!call) return nullptr;
  }
  PyObject* code = py_compile_to_code(self, call ? call : args);
  Py_XDECREF(call);
  if (!code) return nullptr;
  eas_hip_kernel* k = nullptr;
  int rc = eas_hip_kernel_load(PyBytes_AS_STRING(code), (size_t)PyBytes_GET_SIZE(code), name, &k);
  Py_DECREF(code);
  if (rc) return raise_status(rc);
  return new_kernel_capsule(k, src);
}

PyObject* py_kernel_attrs(PyObject*, PyObject* args) {
  PyObject* cap;
  if (!PyArg_ParseTuple(args, "O", &cap)) return nullptr;
  eas_hip_kernel* k = as_kernel(cap);
  if (!k) return nullptr;
  int mt, lds, vg, sg, priv;
  int rc = eas_hip_kernel_attrs(k, &mt, &lds, &vg, &sg, &priv);
  if (rc) return raise_status(rc);
  return Py_BuildValue("{s:i,s:i,s:i,s:i}", "max_threads_per_block", mt, "static_lds_bytes", lds, "num_vgprs", vg,
                       "private_bytes", priv);
}

// alloc_buffer(nbytes, storage="private") -> buffer capsule
PyObject* py_alloc_buffer(PyObject*, PyObject* args) {
  long long nbytes;
  const char* storage = "private";
  if (!PyArg_ParseTuple(args, "L|s", &nbytes, &storage)) return nullptr;
  if (nbytes <= 0) {
    PyErr_SetString(PyExc_ValueError, "nbytes must be > 0");
    return nullptr;
  }
  int kind;
  if (!strcmp(storage, "private")) kind = EAS_HIP_STORAGE_DEVICE;
  else if (!strcmp(storage, "shared")) kind = EAS_HIP_STORAGE_SHARED;
  else {
    PyErr_SetString(PyExc_ValueError, "storage must be 'private' or 'shared'");
    return nullptr;
  }
  void* p = nullptr;
  int rc = eas_hip_alloc((size_t)nbytes, kind, &p);
  if (rc) return raise_status(rc);
  PyObject* cap = new_buffer(p, (size_t)nbytes, kind, true, nullptr, nullptr);
  if (!cap) eas_hip_free(p, kind);
  return cap;
}

// wrap_pointer(ptr, nbytes, owner=None) -> non-owning buffer capsule over device memory
PyObject* py_wrap_pointer(PyObject*, PyObject* args) {
  unsigned long long ptr;
  long long nbytes;
  PyObject* owner = Py_None;
  if (!PyArg_ParseTuple(args, "KL|O", &ptr, &nbytes, &owner)) return nullptr;
  if (nbytes < 0) {
    PyErr_SetString(PyExc_ValueError, "nbytes must be >= 0");
    return nullptr;
  }
  return new_buffer((void*)(uintptr_t)ptr, (size_t)nbytes, EAS_HIP_STORAGE_DEVICE, false, nullptr,
                    owner == Py_None ? nullptr : owner);
}

PyObject* py_buffer_info(PyObject*, PyObject* args) {
  PyObject* cap;
  if (!PyArg_ParseTuple(args, "O", &cap)) return nullptr;
  Buffer* b = as_buffer(cap);
  if (!b) {
    PyErr_SetString(PyExc_TypeError, "expected a buffer capsule");
    return nullptr;
  }
  return Py_BuildValue("(KKs)", (unsigned long long)(uintptr_t)b->ptr, (unsigned long long)b->nbytes,
                       b->storage == EAS_HIP_STORAGE_SHARED ? "shared" : "private");
}

// copy_from_host(buf, src) / copy_to_host(buf, dst): synchronous, size-checked.
PyObject* copy_impl(PyObject* args, bool to_device) {
  PyObject* cap;
  PyObject* host;
  if (!PyArg_ParseTuple(args, "OO", &cap, &host)) return nullptr;
  Buffer* b = as_buffer(cap);
  if (!b) {
    PyErr_SetString(PyExc_TypeError, "expected a buffer capsule");
    return nullptr;
  }
  Py_buffer view;
  if (PyObject_GetBuffer(host, &view, to_device ? PyBUF_C_CONTIGUOUS : (PyBUF_C_CONTIGUOUS | PyBUF_WRITABLE)) != 0)
    return nullptr;
  size_t n = (size_t)view.len;
  int rc = EAS_HIP_OK;
  if (n == 0) {
    PyBuffer_Release(&view);
    PyErr_SetString(PyExc_ValueError, "host buffer is empty");
    return nullptr;
  }
  if (to_device && n > b->nbytes) {
    PyBuffer_Release(&view);
    PyErr_SetString(PyExc_ValueError, "source is larger than destination buffer");
    return nullptr;
  }
  if (!to_device && n < b->nbytes) {
    PyBuffer_Release(&view);
    PyErr_SetString(PyExc_ValueError, "destination is smaller than source buffer");
    return nullptr;
  }
  size_t count = to_device ? n : b->nbytes;
  if (b->storage == EAS_HIP_STORAGE_SHARED) {
    // Pinned host memory: make prior GPU writes visible, then a plain memcpy.
    Py_BEGIN_ALLOW_THREADS
    rc = eas_hip_device_synchronize();
    if (!rc) {
      if (to_device) memcpy(b->ptr, view.buf, count);
      else memcpy(view.buf, b->ptr, count);
    }
    Py_END_ALLOW_THREADS
  } else {
    Py_BEGIN_ALLOW_THREADS
    rc = to_device ? eas_hip_copy_h2d(b->ptr, view.buf, count) : eas_hip_copy_d2h(view.buf, b->ptr, count);
    Py_END_ALLOW_THREADS
  }
  PyBuffer_Release(&view);
  if (rc) return raise_status(rc);
  Py_RETURN_NONE;
}

PyObject* py_copy_from_host(PyObject*, PyObject* args) { return copy_impl(args, true); }
PyObject* py_copy_to_host(PyObject*, PyObject* args) { return copy_impl(args, false); }

// copy_buffer(dst, src, nbytes): device-to-device copy.
PyObject* py_copy_buffer(PyObject*, PyObject* args) {
  PyObject *dcap, *scap;
  long long n;
  if (!PyArg_ParseTuple(args, "OOL", &dcap, &scap, &n)) return nullptr;
  Buffer* d = as_buffer(dcap);
  Buffer* s = as_buffer(scap);
  if (!d || !s) {
    PyErr_SetString(PyExc_TypeError, "expected buffer capsules");
    return nullptr;
  }
  if (n < 0 || (size_t)n > d->nbytes || (size_t)n > s->nbytes) {
    PyErr_SetString(PyExc_ValueError, "copy size exceeds a buffer");
    return nullptr;
  }
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = eas_hip_copy_d2d(d->ptr, s->ptr, (size_t)n);
  Py_END_ALLOW_THREADS
  if (rc) return raise_status(rc);
  Py_RETURN_NONE;
}

// ---- launches ------------------------------------------------------------------
//
// Three argument forms over one implementation:
//   launch / launch_async (reference: _metal.mm:1013-1222, 1381-1383):
//       (kernel, argv, writable, threads_per_grid, threads_per_threadgroup=None, repeat=1, *, stream=None)
//   launch_tg / launch_tg_async (reference: _metal.mm:1232-1379):
//       (kernel, argv, writable, threadgroups, threads_per_threadgroup, repeat=1, *, stream=None)
//   launch_groups / launch_groups_async (HIP workgroups; argv ends with the hidden extents):
//       (kernel, argv, writable, grid, block, repeat=1, lds=0, stream=None)
// In the first two forms argv holds the kernel's own arguments, as the reference runtime
// builds it; the C ABI plans the workgroups from the kernel's launch shape and appends
// the hidden extents.

enum class Form { kThreads, kThreadgroups, kGroups };

struct LaunchArgs {
  PyObject* kernel = nullptr;
  PyObject* argv = nullptr;
  PyObject* writable = nullptr;
  PyObject* size = nullptr;
  PyObject* tptg = nullptr;
  int repeat = 1;
  unsigned int lds = 0;
  PyObject* stream = nullptr;
  int batch = kBatchLaunches;  // async: launches per completion event
  uint32_t g[3], b[3];
  uint64_t sz[3];
  uint32_t tg[3] = {0, 0, 0};
  eas_hip_kernel* k = nullptr;
};

// An int (x, 1, 1) or a 1..3 tuple/list of non-negative ints, as the reference's parse_size3
// (_metal.mm:955-1011).
bool parse_size3(PyObject* obj, uint64_t out[3], const char* what) {
  out[0] = out[1] = out[2] = 1;
  if (PyLong_Check(obj)) {
    unsigned long long v = PyLong_AsUnsignedLongLong(obj);
    if (PyErr_Occurred()) return false;
    out[0] = v;
    return true;
  }
  if (!PyTuple_Check(obj) && !PyList_Check(obj)) {
    PyErr_Format(PyExc_TypeError, "%s must be int or tuple/list of ints", what);
    return false;
  }
  PyObject* seq = PySequence_Fast(obj, "expected a tuple/list");
  if (!seq) return false;
  Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  if (n < 1 || n > 3) {
    Py_DECREF(seq);
    PyErr_Format(PyExc_ValueError, "%s must have 1..3 dims", what);
    return false;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* it = PySequence_Fast_GET_ITEM(seq, i);
    if (!PyLong_Check(it)) {
      Py_DECREF(seq);
      PyErr_Format(PyExc_TypeError, "%s dim %zd must be int", what, i);
      return false;
    }
    unsigned long long v = PyLong_AsUnsignedLongLong(it);
    if (PyErr_Occurred()) {
      Py_DECREF(seq);
      return false;
    }
    out[i] = v;
  }
  Py_DECREF(seq);
  return true;
}

// threads_per_threadgroup: None or 0 means the kernel's own (all zeros for the C ABI).
bool parse_tptg(PyObject* obj, uint32_t out[3]) {
  out[0] = out[1] = out[2] = 0;
  if (!obj || obj == Py_None) return true;
  uint64_t v[3];
  if (!parse_size3(obj, v, "threads_per_threadgroup")) return false;
  if (PyLong_Check(obj) && v[0] == 0) return true;
  for (int i = 0; i < 3; ++i) {
    if (v[i] == 0) {
      PyErr_SetString(PyExc_ValueError, "threads_per_threadgroup dims must be > 0");
      return false;
    }
    if (v[i] > 1024) {
      PyErr_Format(PyExc_ValueError, "threads_per_threadgroup too large: %llu", (unsigned long long)v[i]);
      return false;
    }
    out[i] = (uint32_t)v[i];
  }
  return true;
}

bool parse_launch(PyObject* args, PyObject* kwargs, Form form, LaunchArgs& a) {
  if (form == Form::kGroups) {
    static const char* kw[] = {"kernel", "argv", "writable", "grid", "block", "repeat", "lds", "stream", "batch",
                               nullptr};
    if (!PyArg_ParseTupleAndKeywords(args, kwargs, "OOOOO|iIO$i", const_cast<char**>(kw), &a.kernel, &a.argv,
                                     &a.writable, &a.size, &a.tptg, &a.repeat, &a.lds, &a.stream, &a.batch))
      return false;
  } else if (form == Form::kThreads) {
    static const char* kw[] = {"kernel", "argv", "writable", "threads_per_grid", "threads_per_threadgroup", "repeat",
                               "stream", "batch", nullptr};
    if (!PyArg_ParseTupleAndKeywords(args, kwargs, "OOOO|Oi$Oi", const_cast<char**>(kw), &a.kernel, &a.argv,
                                     &a.writable, &a.size, &a.tptg, &a.repeat, &a.stream, &a.batch))
      return false;
  } else {
    static const char* kw[] = {"kernel", "argv", "writable", "threadgroups", "threads_per_threadgroup", "repeat",
                               "stream", "batch", nullptr};
    if (!PyArg_ParseTupleAndKeywords(args, kwargs, "OOOOO|i$Oi", const_cast<char**>(kw), &a.kernel, &a.argv,
                                     &a.writable, &a.size, &a.tptg, &a.repeat, &a.stream, &a.batch))
      return false;
  }
  if (a.repeat <= 0) {
    PyErr_SetString(PyExc_ValueError, "repeat must be > 0");
    return false;
  }
  if (a.batch < 1 || a.batch > kBatchLaunches) {
    PyErr_Format(PyExc_ValueError, "batch must be in [1, %d]", kBatchLaunches);
    return false;
  }
  a.k = as_kernel(a.kernel);
  if (!a.k) return false;
  if (form == Form::kGroups) {
    if (!parse_dim3(a.size, a.g, "grid") || !parse_dim3(a.tptg, a.b, "block")) return false;
    if (a.g[0] == 0 || a.g[1] == 0 || a.g[2] == 0) {
      PyErr_SetString(PyExc_ValueError, "grid dims must be > 0");
      return false;
    }
    if (a.b[0] == 0 || a.b[1] == 0 || a.b[2] == 0) {
      PyErr_SetString(PyExc_ValueError, "block dims must be > 0");
      return false;
    }
    if ((uint64_t)a.b[0] * a.b[1] * a.b[2] > 1024) {
      PyErr_Format(PyExc_ValueError, "threads_per_threadgroup too large: %llu",
                   (unsigned long long)a.b[0] * a.b[1] * a.b[2]);
      return false;
    }
    return true;
  }
  const char* what = form == Form::kThreads ? "threads_per_grid" : "threadgroups";
  if (!parse_size3(a.size, a.sz, what)) return false;
  if (a.sz[0] == 0 || a.sz[1] == 0 || a.sz[2] == 0) {
    PyErr_Format(PyExc_ValueError, "%s dims must be > 0", what);
    return false;
  }
  return parse_tptg(a.tptg, a.tg);
}

int dispatch(const LaunchArgs& a, Form form, const std::vector<uint8_t>& blob, const std::vector<uint64_t>& sizes,
             void* stream) {
  const int nargs = (int)sizes.size();
  switch (form) {
    case Form::kGroups:
      return eas_hip_launch(a.k, blob.data(), blob.size(), a.g, a.b, a.lds, stream, a.repeat);
    case Form::kThreads:
      return eas_hip_launch_threads(a.k, blob.data(), blob.size(), sizes.data(), nargs, a.sz, a.tg, stream, a.repeat);
    default:
      return eas_hip_launch_threadgroups(a.k, blob.data(), blob.size(), sizes.data(), nargs, a.sz, a.tg, stream,
                                         a.repeat);
  }
}

// Enqueue; the synchronous forms then wait with the GIL released, like the reference's.
PyObject* launch_impl(PyObject* args, PyObject* kwargs, Form form, bool async) {
  LaunchArgs a;
  if (!parse_launch(args, kwargs, form, a)) return nullptr;
  std::vector<uint8_t> blob;
  std::vector<uint64_t> sizes;
  auto* pending = async ? new Pending{nullptr, {}} : nullptr;
  if (!pack_args(a.argv, a.writable, blob, pending ? &pending->keepalive : nullptr, &sizes)) {
    delete pending;
    return nullptr;
  }
  void* stream = as_stream(a.stream);
  if (PyErr_Occurred()) {
    if (pending) release_pending(pending);
    delete pending;
    return nullptr;
  }
  int rc = dispatch(a, form, blob, sizes, stream);
  if (rc) {
    if (pending) release_pending(pending);
    delete pending;
    return raise_status(rc);
  }
  if (!async) {
    Py_BEGIN_ALLOW_THREADS
    rc = eas_hip_stream_synchronize(stream);
    Py_END_ALLOW_THREADS
    if (rc) return raise_status(rc);
    Py_RETURN_NONE;
  }
  Py_INCREF(a.kernel);
  pending->keepalive.push_back(a.kernel);
  Batch* b = join_batch(stream, a.batch, &rc);
  pending->batch = b;
  if (b->launches >= b->limit) {
    int crc = close_batch(b);
    if (!rc) rc = crc;
  }
  if (rc) {
    release_pending(pending);
    delete pending;
    return raise_status(rc);
  }
  PyObject* cap = PyCapsule_New(pending, kPendingCap, pending_destructor);
  if (!cap) {
    release_pending(pending);
    delete pending;
  }
  return cap;
}

PyObject* py_launch(PyObject*, PyObject* args, PyObject* kw) { return launch_impl(args, kw, Form::kThreads, false); }
PyObject* py_launch_async(PyObject*, PyObject* args, PyObject* kw) { return launch_impl(args, kw, Form::kThreads, true); }
PyObject* py_launch_tg(PyObject*, PyObject* args, PyObject* kw) {
  return launch_impl(args, kw, Form::kThreadgroups, false);
}
PyObject* py_launch_tg_async(PyObject*, PyObject* args, PyObject* kw) {
  return launch_impl(args, kw, Form::kThreadgroups, true);
}
PyObject* py_launch_groups(PyObject*, PyObject* args, PyObject* kw) { return launch_impl(args, kw, Form::kGroups, false); }
PyObject* py_launch_groups_async(PyObject*, PyObject* args, PyObject* kw) {
  return launch_impl(args, kw, Form::kGroups, true);
}

// launch_timed(kernel, argv, writable, grid, block, repeat=1, lds=0, stream=None, warmup=0) -> mean ms per launch
// (workgroup form, argv ending with the hidden extents)
PyObject* py_launch_timed(PyObject*, PyObject* args, PyObject* kwargs) {
  PyObject* warm_obj = kwargs ? PyDict_GetItemString(kwargs, "warmup") : nullptr;
  long warmup = 0;
  PyObject* kw2 = nullptr;
  if (warm_obj) {
    warmup = PyLong_AsLong(warm_obj);
    if (PyErr_Occurred()) return nullptr;
    kw2 = PyDict_Copy(kwargs);
    if (!kw2) return nullptr;
    PyDict_DelItemString(kw2, "warmup");
  }
  LaunchArgs a;
  bool ok = parse_launch(args, kw2 ? kw2 : kwargs, Form::kGroups, a);
  Py_XDECREF(kw2);
  if (!ok) return nullptr;
  if (warmup < 0) {
    PyErr_SetString(PyExc_ValueError, "warmup must be >= 0");
    return nullptr;
  }
  std::vector<uint8_t> blob;
  if (!pack_args(a.argv, a.writable, blob, nullptr)) return nullptr;
  void* stream = as_stream(a.stream);
  if (PyErr_Occurred()) return nullptr;
  float ms = 0.f;
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = eas_hip_launch_timed(a.k, blob.data(), blob.size(), a.g, a.b, a.lds, stream, (int)warmup, a.repeat, &ms);
  Py_END_ALLOW_THREADS
  if (rc) return raise_status(rc);
  return PyFloat_FromDouble((double)ms);
}

// ---- the call memo's launch, in one native call ---------------------------------------
//
// A repeated eas call with the same argument types (torch GPU tensors and Python scalars, no
// launch options) launches what its first call planned, but on the arguments it is given now.
// fast_make records, per argument, what the first call's specialisation expects; fast_call
// checks the new arguments against it (exact types, the tensor's dtype object, is_cuda,
// contiguity), packs the device pointers and scalars, plans the dispatch from N as launch_tg
// would (cached for the last N), launches on torch's current stream of the last torch tensor's
// device (the default stream when every buffer is an eas.Tensor) and, when asynchronous, returns a
// pending capsule of the stream's batch.  Any argument it does
// not take returns NotImplemented before anything is launched, and the caller takes its full
// path, which launches or raises as it always does.

enum FastKind { kFastTensor = 0, kFastU32 = 1, kFastF32 = 2, kFastBool = 3, kFastEasTensor = 4 };

struct FastArg {
  int kind;
  PyObject* expect;  // tensor: its dtype object; scalar: its Python type (owned)
  uint32_t offset;   // byte offset in the packed arguments
};

struct Fast {
  PyObject* kernel = nullptr;       // kernel capsule (owned)
  eas_hip_kernel* k = nullptr;
  eas_hip_launch_shape shape{};
  std::vector<FastArg> args;
  int n_index = -1;                 // position of the u32 argument N
  bool by_groups = true;            // SPMD: N lanes are ceil(N / BLOCK) programs; thread mode: N threads
  bool sync = true;
  int batch = kBatchLaunches;
  PyObject* tensor_type = nullptr;  // torch.Tensor (owned)
  PyObject* eas_type = nullptr;     // eas.Tensor (owned)
  PyObject* raw_stream = nullptr;   // callable: device index -> current raw stream (owned)
  bool have_plan = false;
  uint64_t plan_n = 0;
  uint32_t grid[3] = {1, 1, 1}, block[3] = {1, 1, 1}, hidden[EAS_HIP_MAX_HIDDEN] = {};
};

const char* kFastCap = "eas._hip.fast";

void free_fast(Fast* f) {
  Py_XDECREF(f->kernel);
  Py_XDECREF(f->tensor_type);
  Py_XDECREF(f->eas_type);
  Py_XDECREF(f->raw_stream);
  for (auto& a : f->args) Py_XDECREF(a.expect);
  delete f;
}

void fast_destructor(PyObject* cap) {
  auto* f = static_cast<Fast*>(PyCapsule_GetPointer(cap, kFastCap));
  if (!f) {
    PyErr_Clear();
    return;
  }
  free_fast(f);
}

// fast_make(kernel, specs, n_index, sync, batch, tensor_type, raw_stream, eas_type) -> fast capsule.
// specs: one (kind, expect) per kernel argument, kind 0 torch tensor (expect: its torch dtype),
// 1 u32 (int), 2 f32 (float), 3 bool, 4 eas.Tensor on the GPU (expect: its NumPy dtype); the kernel
// must have an SPMD or thread-mode launch shape.
PyObject* py_fast_make(PyObject*, PyObject* args) {
  PyObject *kcap, *specs, *tensor_type, *raw_stream, *eas_type;
  int n_index, sync, batch;
  if (!PyArg_ParseTuple(args, "OOipiOOO", &kcap, &specs, &n_index, &sync, &batch, &tensor_type, &raw_stream,
                        &eas_type))
    return nullptr;
  eas_hip_kernel* k = as_kernel(kcap);
  if (!k) return nullptr;
  eas_hip_launch_shape s;
  int rc = eas_hip_kernel_get_shape(k, &s);
  if (rc) return raise_status(rc);
  if (s.kind != EAS_HIP_KIND_SPMD && s.kind != EAS_HIP_KIND_THREAD) {
    PyErr_SetString(PyExc_ValueError, "fast_make: the kernel needs an SPMD or thread-mode launch shape");
    return nullptr;
  }
  if (batch < 1 || batch > kBatchLaunches || !PyCallable_Check(raw_stream)) {
    PyErr_SetString(PyExc_ValueError, "fast_make: bad batch or stream getter");
    return nullptr;
  }
  PyObject* seq = PySequence_Fast(specs, "specs must be a sequence");
  if (!seq) return nullptr;
  auto* f = new Fast;
  f->shape = s;
  uint32_t off = 0;
  bool ok = true;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  for (Py_ssize_t i = 0; ok && i < n; ++i) {
    int kind;
    PyObject* expect;
    if (!PyArg_ParseTuple(PySequence_Fast_GET_ITEM(seq, i), "iO", &kind, &expect)) {
      ok = false;
      break;
    }
    const uint32_t size = (kind == kFastTensor || kind == kFastEasTensor) ? 8 : kind == kFastBool ? 1 : 4;
    if (kind < kFastTensor || kind > kFastEasTensor) {
      PyErr_SetString(PyExc_ValueError, "fast_make: unknown argument kind");
      ok = false;
      break;
    }
    off = (off + size - 1) / size * size;
    Py_INCREF(expect);
    f->args.push_back({kind, expect, off});
    off += size;
  }
  Py_DECREF(seq);
  if (ok && (n_index < 0 || n_index >= (int)f->args.size() || f->args[n_index].kind != kFastU32)) {
    PyErr_SetString(PyExc_ValueError, "fast_make: N must be a u32 argument");
    ok = false;
  }
  if (ok && s.arg_bytes && off != s.arg_bytes) {
    PyErr_Format(PyExc_ValueError, "fast_make: %u bytes of arguments, the kernel takes %u", off, s.arg_bytes);
    ok = false;
  }
  if (!ok) {
    free_fast(f);
    return nullptr;
  }
  f->n_index = n_index;
  f->by_groups = s.kind == EAS_HIP_KIND_SPMD;
  f->sync = sync != 0;
  f->batch = batch;
  Py_INCREF(kcap);
  f->kernel = kcap;
  f->k = k;
  Py_INCREF(tensor_type);
  f->tensor_type = tensor_type;
  Py_INCREF(eas_type);
  f->eas_type = eas_type;
  Py_INCREF(raw_stream);
  f->raw_stream = raw_stream;
  PyObject* cap = PyCapsule_New(f, kFastCap, fast_destructor);
  if (!cap) free_fast(f);
  return cap;
}

PyObject* g_s_dtype = nullptr;
PyObject* g_s_is_cuda = nullptr;
PyObject* g_s_is_contiguous = nullptr;
PyObject* g_s_data_ptr = nullptr;
PyObject* g_s_get_device = nullptr;
PyObject* g_s_device_attr = nullptr;  // eas.Tensor._device
PyObject* g_s_dtype_attr = nullptr;   // eas.Tensor._dtype
PyObject* g_s_hip_attr = nullptr;     // eas.Tensor._hip (its storage; .buf the buffer capsule)
PyObject* g_s_buf = nullptr;

// The boolean result of calling obj.name(): 1, 0, or -1 on error.
int call_true(PyObject* obj, PyObject* name) {
  PyObject* r = PyObject_CallMethodNoArgs(obj, name);
  if (!r) return -1;
  int t = r == Py_True;
  Py_DECREF(r);
  return t;
}

// fast_call(fast, args: tuple) -> None (launched and, if synchronous, done), a pending capsule
// (asynchronous), or NotImplemented (an argument this specialisation's fast path does not take;
// nothing was launched).
PyObject* py_fast_call(PyObject*, PyObject* const* argv, Py_ssize_t nargv) {
  if (nargv != 2 || !PyTuple_Check(argv[1])) {
    PyErr_SetString(PyExc_TypeError, "fast_call(fast, args: tuple)");
    return nullptr;
  }
  auto* f = static_cast<Fast*>(PyCapsule_GetPointer(argv[0], kFastCap));
  if (!f) return nullptr;
  PyObject* args = argv[1];
  const size_t n = f->args.size();
  if ((size_t)PyTuple_GET_SIZE(args) != n) Py_RETURN_NOTIMPLEMENTED;
  uint8_t blob[512];
  const size_t arg_bytes = f->shape.arg_bytes, total = (arg_bytes + 3) / 4 * 4 + 4 * (size_t)f->shape.hidden;
  if (total > sizeof(blob)) Py_RETURN_NOTIMPLEMENTED;
  memset(blob, 0, total);
  PyObject* last_tensor = nullptr;
  uint64_t nval = 0;
  for (size_t i = 0; i < n; ++i) {
    const FastArg& a = f->args[i];
    PyObject* obj = PyTuple_GET_ITEM(args, (Py_ssize_t)i);
    if (a.kind == kFastTensor) {
      if (Py_TYPE(obj) != (PyTypeObject*)f->tensor_type) Py_RETURN_NOTIMPLEMENTED;
      PyObject* dt = PyObject_GetAttr(obj, g_s_dtype);
      if (!dt) return nullptr;
      Py_DECREF(dt);  // dtypes are singletons held by torch; only their identity is compared
      if (dt != a.expect) Py_RETURN_NOTIMPLEMENTED;
      PyObject* cuda = PyObject_GetAttr(obj, g_s_is_cuda);
      if (!cuda) return nullptr;
      Py_DECREF(cuda);
      if (cuda != Py_True) Py_RETURN_NOTIMPLEMENTED;
      int contiguous = call_true(obj, g_s_is_contiguous);
      if (contiguous < 0) return nullptr;
      if (!contiguous) Py_RETURN_NOTIMPLEMENTED;
      PyObject* p = PyObject_CallMethodNoArgs(obj, g_s_data_ptr);
      if (!p) return nullptr;
      uint64_t ptr = PyLong_AsUnsignedLongLong(p);
      Py_DECREF(p);
      if (PyErr_Occurred()) return nullptr;
      memcpy(blob + a.offset, &ptr, 8);
      last_tensor = obj;
      continue;
    }
    if (a.kind == kFastEasTensor) {
      // an eas.Tensor's device, dtype and storage are fixed when it is made
      if (Py_TYPE(obj) != (PyTypeObject*)f->eas_type) Py_RETURN_NOTIMPLEMENTED;
      PyObject* dev = PyObject_GetAttr(obj, g_s_device_attr);
      if (!dev) return nullptr;
      const int on_gpu = PyUnicode_Check(dev) && PyUnicode_CompareWithASCIIString(dev, "hip") == 0;
      Py_DECREF(dev);
      if (!on_gpu) Py_RETURN_NOTIMPLEMENTED;
      PyObject* dt = PyObject_GetAttr(obj, g_s_dtype_attr);
      if (!dt) return nullptr;
      const int same = PyObject_RichCompareBool(dt, a.expect, Py_EQ);
      Py_DECREF(dt);
      if (same < 0) return nullptr;
      if (!same) Py_RETURN_NOTIMPLEMENTED;
      PyObject* st = PyObject_GetAttr(obj, g_s_hip_attr);
      if (!st) return nullptr;
      PyObject* cap = PyObject_GetAttr(st, g_s_buf);
      Py_DECREF(st);
      if (!cap) return nullptr;
      Buffer* b = as_buffer(cap);
      Py_DECREF(cap);  // the tensor holds its storage, and the storage its buffer
      if (!b) Py_RETURN_NOTIMPLEMENTED;
      const uint64_t ptr = (uint64_t)(uintptr_t)b->ptr;
      memcpy(blob + a.offset, &ptr, 8);
      continue;
    }
    if ((PyObject*)Py_TYPE(obj) != a.expect) Py_RETURN_NOTIMPLEMENTED;
    if (a.kind == kFastU32) {
      unsigned long long v = PyLong_AsUnsignedLongLong(obj);
      if (PyErr_Occurred() || v > 0xFFFFFFFFull) {
        PyErr_Clear();  // the full path raises the packing error
        Py_RETURN_NOTIMPLEMENTED;
      }
      const uint32_t u = (uint32_t)v;
      memcpy(blob + a.offset, &u, 4);
      if ((int)i == f->n_index) nval = v;
    } else if (a.kind == kFastF32) {
      const double d = PyFloat_AS_DOUBLE(obj);
      const float x = (float)d;
      if (std::isinf(x) && !std::isinf(d)) Py_RETURN_NOTIMPLEMENTED;  // the full path raises OverflowError
      memcpy(blob + a.offset, &x, 4);
    } else {
      blob[a.offset] = obj == Py_True ? 1 : 0;
    }
  }
  if (nval == 0) Py_RETURN_NONE;  // a zero extent launches nothing
  if (!f->have_plan || f->plan_n != nval) {
    const uint32_t block = f->shape.block_size;
    const uint64_t size[3] = {f->by_groups ? (nval + block - 1) / block : nval, 1, 1};
    static const uint32_t kAuto[3] = {0, 0, 0};
    int rc = eas_hip_plan_dispatch(&f->shape, f->by_groups, size, kAuto, f->grid, f->block, f->hidden,
                                   EAS_HIP_MAX_HIDDEN);
    if (rc) {
      PyErr_Clear();
      Py_RETURN_NOTIMPLEMENTED;  // the full path reports the size error
    }
    f->plan_n = nval;
    f->have_plan = true;
  }
  memcpy(blob + (arg_bytes + 3) / 4 * 4, f->hidden, 4 * f->shape.hidden);
  void* stream = nullptr;  // torch's current stream of the last torch tensor's device, else the default
  if (last_tensor) {
    PyObject* dev = PyObject_CallMethodNoArgs(last_tensor, g_s_get_device);
    if (!dev) return nullptr;
    PyObject* sobj = PyObject_CallOneArg(f->raw_stream, dev);
    Py_DECREF(dev);
    if (!sobj) return nullptr;
    stream = PyLong_AsVoidPtr(sobj);
    Py_DECREF(sobj);
    if (PyErr_Occurred()) return nullptr;
  }
  int rc = eas_hip_launch(f->k, blob, total, f->grid, f->block, 0, stream, 1);
  if (rc) return raise_status(rc);
  if (f->sync) {
    Py_BEGIN_ALLOW_THREADS
    rc = eas_hip_stream_synchronize(stream);
    Py_END_ALLOW_THREADS
    if (rc) return raise_status(rc);
    Py_RETURN_NONE;
  }
  auto* pending = new Pending{nullptr, {}};
  for (size_t i = 0; i < n; ++i) {
    if (f->args[i].kind != kFastTensor && f->args[i].kind != kFastEasTensor) continue;
    PyObject* obj = PyTuple_GET_ITEM(args, (Py_ssize_t)i);
    Py_INCREF(obj);
    pending->keepalive.push_back(obj);
  }
  Py_INCREF(f->kernel);
  pending->keepalive.push_back(f->kernel);
  Batch* b = join_batch(stream, f->batch, &rc);
  pending->batch = b;
  if (b->launches >= b->limit) {
    int crc = close_batch(b);
    if (!rc) rc = crc;
  }
  if (rc) {
    release_pending(pending);
    delete pending;
    return raise_status(rc);
  }
  PyObject* cap = PyCapsule_New(pending, kPendingCap, pending_destructor);
  if (!cap) {
    release_pending(pending);
    delete pending;
  }
  return cap;
}

const char* kind_name(int kind) {
  switch (kind) {
    case EAS_HIP_KIND_SPMD: return "spmd";
    case EAS_HIP_KIND_THREAD: return "thread";
    case EAS_HIP_KIND_GEMM: return "gemm";
    default: return "raw";
  }
}

PyObject* shape_dict(const eas_hip_launch_shape& s) {
  return Py_BuildValue("{s:s,s:I,s:I,s:I,s:I,s:I,s:I}", "kind", kind_name(s.kind), "block_size", s.block_size,
                       "wg_size", s.wg_size, "programs_per_wg", s.programs_per_wg, "split", s.split, "arg_bytes",
                       s.arg_bytes, "hidden", s.hidden);
}

// kernel_shape(kernel) -> dict: the launch shape attached to a loaded kernel.
PyObject* py_kernel_shape(PyObject*, PyObject* args) {
  PyObject* cap;
  if (!PyArg_ParseTuple(args, "O", &cap)) return nullptr;
  eas_hip_kernel* k = as_kernel(cap);
  if (!k) return nullptr;
  eas_hip_launch_shape s;
  int rc = eas_hip_kernel_get_shape(k, &s);
  if (rc) return raise_status(rc);
  return shape_dict(s);
}

PyObject* gemm_dict(const eas_hip_gemm_shape& g) {
  return Py_BuildValue("{s:s,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:I,s:i,s:i,s:i,s:i,s:I,"
                       "s:I,s:I,s:I,s:I,s:I,s:I,s:I}",
                       "entry", g.entry, "entries", g.entries, "K", g.K, "tm", g.tm, "tn", g.tn, "row_axis",
                       g.row_axis, "bm", g.bm, "bn", g.bn, "threads", g.threads, "pp_threads", g.pp_threads,
                       "t128_threads", g.t128_threads, "skinny_m", g.skinny_m, "skinny_n", g.skinny_n, "skinny_cut",
                       g.skinny_cut, "wide_m", g.wide_m, "f32", g.f32, "col_masked", g.col_masked, "m_off", g.m_off,
                       "ldb_off", g.ldb_off, "row_base_off", g.row_base_off, "col_base_off", g.col_base_off, "a_arg",
                       g.a_arg, "b_arg", g.b_arg, "c_arg", g.c_arg, "a_off", g.a_off, "b_off", g.b_off, "a_elem",
                       g.a_elem, "b_elem", g.b_elem, "c_elem", g.c_elem);
}

// launch_shape(src) -> dict: the shape on a generated source's eas-launch line (no GPU needed);
// a lifted GEMM's also holds its eas-gemm line under "gemm".
PyObject* py_launch_shape(PyObject*, PyObject* args) {
  const char* src;
  if (!PyArg_ParseTuple(args, "s", &src)) return nullptr;
  eas_hip_launch_shape s;
  int rc = eas_hip_launch_shape_parse(src, &s);
  if (rc) return raise_status(rc);
  PyObject* d = shape_dict(s);
  if (!d || s.kind != EAS_HIP_KIND_GEMM) return d;
  eas_hip_gemm_shape g;
  rc = eas_hip_gemm_shape_parse(src, &g);
  if (rc) {
    Py_DECREF(d);
    return raise_status(rc);
  }
  PyObject* gd = gemm_dict(g);
  if (!gd || PyDict_SetItemString(d, "gemm", gd) != 0) {
    Py_XDECREF(gd);
    Py_DECREF(d);
    return nullptr;
  }
  Py_DECREF(gd);
  return d;
}

const char* const kGemmSuffixes[EAS_HIP_GEMM_NENTRIES] = {"", "__pp", "__t128", "__t128x256", "__t128x64",
                                                          "__t64x64"};

// plan_dispatch(src, size, threads_per_threadgroup=None, by_groups=False, argv=None, compute_units=256,
//               entry_choice=None):
// the HIP dispatch that launch (by_groups False) or launch_tg (True) makes for a kernel compiled
// from `src`, without a GPU: (grid, block, hidden).  A lifted GEMM's plan reads M, N, the tile
// bases and the A and B addresses from `argv` (the kernel's own arguments, as launch takes them;
// wrap_pointer capsules stand for buffers) and returns (grid, block, hidden, entry), entry None
// for the kernel's own, or None when the launch covers no element of C.
PyObject* py_plan_dispatch(PyObject*, PyObject* args, PyObject* kwargs) {
  static const char* kw[] = {"src", "size", "threads_per_threadgroup", "by_groups", "argv", "compute_units",
                             "entry_choice", nullptr};
  const char* src;
  PyObject* size_obj;
  PyObject* tptg_obj = nullptr;
  int by_groups = 0;
  PyObject* argv = nullptr;
  int cus = 256;
  const char* choice = nullptr;
  if (!PyArg_ParseTupleAndKeywords(args, kwargs, "sO|OpOiz", const_cast<char**>(kw), &src, &size_obj, &tptg_obj,
                                   &by_groups, &argv, &cus, &choice))
    return nullptr;
  eas_hip_launch_shape s;
  int rc = eas_hip_launch_shape_parse(src, &s);
  if (rc) return raise_status(rc);
  uint64_t sz[3];
  uint32_t tg[3];
  if (!parse_size3(size_obj, sz, by_groups ? "threadgroups" : "threads_per_grid") || !parse_tptg(tptg_obj, tg))
    return nullptr;
  if (s.kind == EAS_HIP_KIND_GEMM) {
    if (!argv || argv == Py_None) {
      PyErr_SetString(PyExc_TypeError, "a lifted GEMM's plan needs argv (its M, N and buffers)");
      return nullptr;
    }
    eas_hip_gemm_shape g;
    rc = eas_hip_gemm_shape_parse(src, &g);
    if (rc) return raise_status(rc);
    std::vector<uint8_t> blob;
    std::vector<uint64_t> sizes;
    if (!pack_args(argv, nullptr, blob, nullptr, &sizes)) return nullptr;
    eas_hip_gemm_plan p;
    rc = eas_hip_plan_gemm(&s, &g, blob.data(), blob.size(), sizes.data(), (int)sizes.size(), by_groups, sz, tg, cus,
                           choice, &p);
    if (rc) return raise_status(rc);
    if (!p.launch) Py_RETURN_NONE;
    PyObject* entry = p.entry == EAS_HIP_GEMM_MAIN ? (Py_INCREF(Py_None), Py_None)
                                                   : PyUnicode_FromFormat("%s%s", g.entry, kGemmSuffixes[p.entry]);
    if (!entry) return nullptr;
    return Py_BuildValue("((III)(III)(IIII)N)", p.grid[0], p.grid[1], p.grid[2], p.block[0], p.block[1], p.block[2],
                         p.hidden[0], p.hidden[1], p.hidden[2], p.hidden[3], entry);
  }
  uint32_t grid[3], block[3], hidden[EAS_HIP_MAX_HIDDEN];
  rc = eas_hip_plan_dispatch(&s, by_groups, sz, tg, grid, block, hidden, EAS_HIP_MAX_HIDDEN);
  if (rc) return raise_status(rc);
  PyObject* h = PyTuple_New(s.hidden);
  for (uint32_t i = 0; h && i < s.hidden; ++i) PyTuple_SET_ITEM(h, i, PyLong_FromUnsignedLong(hidden[i]));
  if (!h) return nullptr;
  return Py_BuildValue("((III)(III)N)", grid[0], grid[1], grid[2], block[0], block[1], block[2], h);
}

// pending_info(pending) -> dict: the launch's completion batch (stream, launches, closed), or
// released True once it was waited on.
PyObject* py_pending_info(PyObject*, PyObject* args) {
  PyObject* cap;
  if (!PyArg_ParseTuple(args, "O", &cap)) return nullptr;
  auto* p = static_cast<Pending*>(PyCapsule_GetPointer(cap, kPendingCap));
  if (!p) return nullptr;
  if (!p->batch) return Py_BuildValue("{s:O}", "released", Py_True);
  const Batch* b = p->batch;
  return Py_BuildValue("{s:O,s:K,s:i,s:i,s:O}", "released", Py_False, "stream",
                       (unsigned long long)(uintptr_t)b->stream, "launches", b->launches, "limit", b->limit, "closed",
                       b->closed ? Py_True : Py_False);
}

PyObject* py_synchronize(PyObject*, PyObject* args) {
  PyObject* cap;
  if (!PyArg_ParseTuple(args, "O", &cap)) return nullptr;
  auto* p = static_cast<Pending*>(PyCapsule_GetPointer(cap, kPendingCap));
  if (!p) return nullptr;
  int rc = release_pending(p);
  if (rc) return raise_status(rc);
  Py_RETURN_NONE;
}

PyObject* py_queue_synchronize(PyObject*, PyObject* args) {
  PyObject* stream = nullptr;
  if (!PyArg_ParseTuple(args, "|O", &stream)) return nullptr;
  void* s = as_stream(stream);
  if (PyErr_Occurred()) return nullptr;
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = s ? eas_hip_stream_synchronize(s) : eas_hip_device_synchronize();
  Py_END_ALLOW_THREADS
  if (rc) return raise_status(rc);
  Py_RETURN_NONE;
}

// dlpack_import(capsule 'dltensor') -> (buffer capsule, shape tuple, dtype bits).
// Takes ownership (capsule renamed 'used_dltensor'); the deleter runs when the
// buffer capsule dies.  Reference: _metal.mm:530-638.
PyObject* py_dlpack_import(PyObject*, PyObject* args) {
  PyObject* cap;
  if (!PyArg_ParseTuple(args, "O", &cap)) return nullptr;
  if (!PyCapsule_CheckExact(cap)) {
    PyErr_SetString(PyExc_TypeError, "expected a DLPack capsule (PyCapsule)");
    return nullptr;
  }
  const char* name = PyCapsule_GetName(cap);
  if (!name || strcmp(name, "dltensor") != 0) {
    PyErr_SetString(PyExc_ValueError, "expected a DLPack capsule with name 'dltensor'");
    return nullptr;
  }
  void* managed = PyCapsule_GetPointer(cap, "dltensor");
  if (!managed) return nullptr;
  void* data = nullptr;
  uint64_t nbytes = 0;
  int bits = 0, ndim = 0, dev_type = 0, dev_id = 0;
  int64_t shape[16];
  int rc = eas_hip_dlpack_view(managed, &data, &nbytes, &bits, &ndim, shape, 16, &dev_type, &dev_id);
  if (rc) {
    PyErr_SetString(strstr(eas_hip_last_error(), "only supports") ? PyExc_TypeError : PyExc_ValueError,
                    eas_hip_last_error());
    return nullptr;
  }
  if (dev_type != 10) {
    PyErr_Format(PyExc_ValueError, "dlpack_import expects kDLROCM device_type=10, got %d", dev_type);
    return nullptr;
  }
  if (PyCapsule_SetName(cap, "used_dltensor") != 0) return nullptr;
  if (PyCapsule_SetDestructor(cap, nullptr) != 0) return nullptr;
  PyObject* buf = new_buffer(data, (size_t)nbytes, EAS_HIP_STORAGE_DEVICE, false, managed, nullptr);
  if (!buf) return nullptr;
  PyObject* shp = PyTuple_New(ndim);
  for (int i = 0; shp && i < ndim; ++i) PyTuple_SET_ITEM(shp, i, PyLong_FromLongLong(shape[i]));
  if (!shp) {
    Py_DECREF(buf);
    return nullptr;
  }
  return Py_BuildValue("(NNi)", buf, shp, bits);
}

void export_release(void* ctx) {
  PyGILState_STATE st = PyGILState_Ensure();
  Py_XDECREF(static_cast<PyObject*>(ctx));
  PyGILState_Release(st);
}

void dltensor_capsule_destructor(PyObject* cap) {
  // Only an unconsumed capsule still owns its tensor.
  if (!PyCapsule_IsValid(cap, "dltensor")) return;
  void* m = PyCapsule_GetPointer(cap, "dltensor");
  if (m) eas_hip_dlpack_delete(m);
}

// dlpack_export(buf, shape, dtype_bits) -> 'dltensor' capsule (kDLROCM).
// Waits for the device first, like the reference's full-queue sync (_metal.mm:786-793).
PyObject* py_dlpack_export(PyObject*, PyObject* args) {
  PyObject* cap;
  PyObject* shape_obj;
  int bits = 32;
  int device_id = 0;
  if (!PyArg_ParseTuple(args, "OO|ii", &cap, &shape_obj, &bits, &device_id)) return nullptr;
  Buffer* b = as_buffer(cap);
  if (!b) {
    PyErr_SetString(PyExc_TypeError, "expected a buffer capsule");
    return nullptr;
  }
  PyObject* seq = PySequence_Fast(shape_obj, "shape must be a sequence of ints");
  if (!seq) return nullptr;
  Py_ssize_t ndim = PySequence_Fast_GET_SIZE(seq);
  if (ndim <= 0 || ndim > 8) {
    Py_DECREF(seq);
    PyErr_SetString(PyExc_ValueError, "shape must have 1..8 dims");
    return nullptr;
  }
  int64_t shape[8];
  unsigned long long numel = 1;
  for (Py_ssize_t i = 0; i < ndim; ++i) {
    long long d = PyLong_AsLongLong(PySequence_Fast_GET_ITEM(seq, i));
    if (PyErr_Occurred() || d < 0) {
      Py_DECREF(seq);
      if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "invalid shape");
      return nullptr;
    }
    shape[i] = d;
    numel *= (unsigned long long)d;
  }
  Py_DECREF(seq);
  if (bits != 16 && bits != 32) {
    PyErr_SetString(PyExc_ValueError, "dtype_bits must be 16 or 32");
    return nullptr;
  }
  if (numel * (unsigned long long)(bits / 8) > b->nbytes) {
    PyErr_SetString(PyExc_ValueError, "shape exceeds buffer view size");
    return nullptr;
  }
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = eas_hip_device_synchronize();
  Py_END_ALLOW_THREADS
  if (rc) return raise_status(rc);
  void* managed = nullptr;
  Py_INCREF(cap);
  rc = eas_hip_dlpack_make(b->ptr, device_id, shape, (int)ndim, bits, export_release, cap, &managed);
  if (rc) {
    Py_DECREF(cap);
    return raise_status(rc);
  }
  PyObject* out = PyCapsule_New(managed, "dltensor", dltensor_capsule_destructor);
  if (!out) eas_hip_dlpack_delete(managed);
  return out;
}

PyMethodDef kMethods[] = {
    {"is_available", py_is_available, METH_NOARGS, "1 if a HIP GPU is usable."},
    {"device_props", py_device_props, METH_VARARGS, "Properties of a device (default: current)."},
    {"compile_to_code", py_compile_to_code, METH_VARARGS, "hiprtc: source -> code object bytes (no GPU needed)."},
    {"compiler_version", py_compiler_version, METH_NOARGS, "(major, minor, path) of the hiprtc in use."},
    {"load", (PyCFunction)(void (*)(void))py_load, METH_VARARGS | METH_KEYWORDS,
     "Load a code object and look up a kernel (src= gives it its launch shape)."},
    {"kernel_shape", py_kernel_shape, METH_VARARGS, "Launch shape attached to a loaded kernel."},
    {"launch_shape", py_launch_shape, METH_VARARGS, "Launch shape on a generated source's eas-launch line."},
    {"plan_dispatch", (PyCFunction)(void (*)(void))py_plan_dispatch, METH_VARARGS | METH_KEYWORDS,
     "HIP dispatch (grid, block, hidden[, entry]) of a reference-convention launch, without a GPU."},
    {"compile", py_compile, METH_VARARGS,
     "compile(src, name, options=None): compile_to_code (DEFAULT_OPTIONS when none are given) + load."},
    {"kernel_attrs", py_kernel_attrs, METH_VARARGS, "Static resources of a loaded kernel."},
    {"alloc_buffer", py_alloc_buffer, METH_VARARGS, "Allocate device ('private') or pinned ('shared') memory."},
    {"wrap_pointer", py_wrap_pointer, METH_VARARGS, "Non-owning buffer capsule over existing device memory."},
    {"buffer_info", py_buffer_info, METH_VARARGS, "(ptr, nbytes, storage) of a buffer capsule."},
    {"copy_from_host", py_copy_from_host, METH_VARARGS, "Synchronous host -> buffer copy."},
    {"copy_to_host", py_copy_to_host, METH_VARARGS, "Synchronous buffer -> host copy."},
    {"copy_buffer", py_copy_buffer, METH_VARARGS, "Synchronous buffer -> buffer copy."},
    {"launch", (PyCFunction)(void (*)(void))py_launch, METH_VARARGS | METH_KEYWORDS,
     "launch(kernel, argv, writable, threads_per_grid, threads_per_threadgroup=None, repeat=1): dispatch by "
     "threads and wait."},
    {"launch_async", (PyCFunction)(void (*)(void))py_launch_async, METH_VARARGS | METH_KEYWORDS,
     "As launch; returns a pending capsule (batch=: launches per completion event, 1-16)."},
    {"launch_tg", (PyCFunction)(void (*)(void))py_launch_tg, METH_VARARGS | METH_KEYWORDS,
     "launch_tg(kernel, argv, writable, threadgroups, threads_per_threadgroup, repeat=1): dispatch by "
     "threadgroups and wait."},
    {"launch_tg_async", (PyCFunction)(void (*)(void))py_launch_tg_async, METH_VARARGS | METH_KEYWORDS,
     "As launch_tg; returns a pending capsule (batch= as for launch_async)."},
    {"launch_groups", (PyCFunction)(void (*)(void))py_launch_groups, METH_VARARGS | METH_KEYWORDS,
     "launch_groups(kernel, argv, writable, grid, block, repeat=1, lds=0, stream=None): HIP workgroups, argv "
     "ending with the hidden extents; waits."},
    {"launch_groups_async", (PyCFunction)(void (*)(void))py_launch_groups_async, METH_VARARGS | METH_KEYWORDS,
     "As launch_groups; returns a pending capsule (batch= as for launch_async)."},
    {"launch_timed", (PyCFunction)(void (*)(void))py_launch_timed, METH_VARARGS | METH_KEYWORDS,
     "Event-timed repeat launches; mean ms per launch."},
    {"synchronize", py_synchronize, METH_VARARGS, "Wait for a pending launch and drop its keepalives."},
    {"fast_make", py_fast_make, METH_VARARGS, "The call memo's native launch for one specialisation."},
    {"fast_call", (PyCFunction)(void (*)(void))py_fast_call, METH_FASTCALL,
     "fast_call(fast, args): launch the memoized specialisation, or NotImplemented."},
    {"pending_info", py_pending_info, METH_VARARGS, "Completion batch of a pending launch (stream, launches, closed)."},
    {"queue_synchronize", py_queue_synchronize, METH_VARARGS, "Wait for a stream (default: whole device)."},
    {"dlpack_import", py_dlpack_import, METH_VARARGS, "Zero-copy import of a kDLROCM DLPack capsule."},
    {"dlpack_export", py_dlpack_export, METH_VARARGS, "Export a buffer as a kDLROCM DLPack capsule."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_hip", "MI355X (gfx950) HIP backend of eas.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__hip(void) {
  g_s_dtype = PyUnicode_InternFromString("dtype");
  g_s_is_cuda = PyUnicode_InternFromString("is_cuda");
  g_s_is_contiguous = PyUnicode_InternFromString("is_contiguous");
  g_s_data_ptr = PyUnicode_InternFromString("data_ptr");
  g_s_get_device = PyUnicode_InternFromString("get_device");
  g_s_device_attr = PyUnicode_InternFromString("_device");
  g_s_dtype_attr = PyUnicode_InternFromString("_dtype");
  g_s_hip_attr = PyUnicode_InternFromString("_hip");
  g_s_buf = PyUnicode_InternFromString("buf");
  if (!g_s_dtype || !g_s_is_cuda || !g_s_is_contiguous || !g_s_data_ptr || !g_s_get_device || !g_s_device_attr ||
      !g_s_dtype_attr || !g_s_hip_attr || !g_s_buf)
    return nullptr;
  PyObject* m = PyModule_Create(&kModule);
  if (m) PyModule_AddIntConstant(m, "ABI_VERSION", eas_hip_abi_version());
  if (m && PyModule_AddObject(m, "DEFAULT_OPTIONS", default_options()) != 0) {
    Py_DECREF(m);
    return nullptr;
  }
  return m;
}
