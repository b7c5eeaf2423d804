// Host side of a decode tick, native: the row tables of a pass and one call
// that uploads a tick's tables and replays its captured graph.
//
// A scheduler tick hands the engine up to T_total + 2 passes (P, R..., C) of
// a few to a few hundred rows each. Built with numpy, the tables of one pass
// cost ~15 us of small-array calls, and the GPU idles through them: the tick
// cannot launch before its tables exist. Here each pass is one call that
// validates the rows, forms the attention groups and writes the tables in
// place, and the upload + graph launch is a second call that makes three HIP
// runtime calls (copy, event record, graph launch) with no Python in between.
// A greedy tick's accept flags come back through mapped, coherent pinned host
// memory that the argmax kernel stores into and the host polls (host_alloc,
// clear_flags, wait_flags), with no device->host copy behind the graph.
//
// Table layout of one pass over nb rows (rows n..nb-1 are padding aimed at the
// trash rows / trash ring slot; L = the pass's layer count):
//   int32  [pos | kv_len = pos + 1 | pool_row | ring_slot (C only)
//           | group_first (grouped passes, nb + 1 entries)]
//   int64  [ids (P only) | row_base x L | flat_row x L | expected token (C only)]
// row_base of (slot, seq b) = (slot * B + b) * S and flat_row = row_base + pos
// (src/decoding/batch_kv_cache.py:64-65); pool_row = b * R + pos % R.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

// engine constants of one (model, cache) pair, passed as a tuple of ints
enum Param {
  kB, kS, kTrashRow, kPoolR, kTrashPoolRow, kNPrelude, kNCore, kNCoda, kTTotal, kCodaBase, kRingLen,
  kMaxBatch, kMaxSeqLen, kMaxRows, kUseGraphs, kGroupAttention, kGroupMaxRows, kGroupMinWorkgroups,
  kNKvHeads, kNumParams
};

constexpr int64_t kNoExpect = -(int64_t(1) << 62);  // an expected-token entry that asks for no comparison

bool read_params(PyObject* t, int64_t* p) {
  if (!PyTuple_Check(t) || PyTuple_GET_SIZE(t) != kNumParams) {
    PyErr_Format(PyExc_TypeError, "params: a tuple of %d ints", int(kNumParams));
    return false;
  }
  for (int i = 0; i < kNumParams; ++i) {
    p[i] = PyLong_AsLongLong(PyTuple_GET_ITEM(t, i));
    if (p[i] == -1 && PyErr_Occurred()) return false;
  }
  return true;
}

// ints of a list / tuple / 1-D int32 or int64 buffer (numpy array) into out
bool read_ints(PyObject* obj, std::vector<int64_t>& out, const char* what) {
  if (PyObject_CheckBuffer(obj)) {
    Py_buffer v;
    if (PyObject_GetBuffer(obj, &v, PyBUF_FORMAT | PyBUF_ND | PyBUF_STRIDES) == 0) {
      bool ok = v.ndim == 1 && v.format != nullptr && v.format[1] == '\0' &&
                (v.itemsize == 8 || v.itemsize == 4) &&
                (v.format[0] == 'l' || v.format[0] == 'q' || v.format[0] == 'i');
      if (ok) {
        const Py_ssize_t n = v.shape[0], st = v.strides[0];
        out.resize(n);
        const char* base = static_cast<const char*>(v.buf);
        for (Py_ssize_t i = 0; i < n; ++i) {
          const char* e = base + i * st;
          if (v.itemsize == 8) {
            int64_t x;
            std::memcpy(&x, e, 8);
            out[i] = x;
          } else {
            int32_t x;
            std::memcpy(&x, e, 4);
            out[i] = x;
          }
        }
        PyBuffer_Release(&v);
        return true;
      }
      PyBuffer_Release(&v);
    } else {
      PyErr_Clear();
    }
  }
  PyObject* fast = PySequence_Fast(obj, what);
  if (fast == nullptr) return false;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(fast);
  PyObject** items = PySequence_Fast_ITEMS(fast);
  out.resize(n);
  for (Py_ssize_t i = 0; i < n; ++i) {
    const long long x = PyLong_AsLongLong(items[i]);
    if (x == -1 && PyErr_Occurred()) {
      Py_DECREF(fast);
      return false;
    }
    out[i] = x;
  }
  Py_DECREF(fast);
  return true;
}

// a writable C-contiguous buffer of `itemsize`-byte items
struct OutBuf {
  Py_buffer v{};
  bool held = false;
  bool get(PyObject* obj, Py_ssize_t itemsize, const char* what) {
    if (PyObject_GetBuffer(obj, &v, PyBUF_WRITABLE | PyBUF_C_CONTIGUOUS) != 0) return false;
    held = true;
    if (v.itemsize != itemsize) {
      PyErr_Format(PyExc_TypeError, "%s: items of %zd bytes expected", what, itemsize);
      return false;
    }
    return true;
  }
  Py_ssize_t size() const { return v.len / v.itemsize; }
  ~OutBuf() {
    if (held) PyBuffer_Release(&v);
  }
};

int64_t bucket(int64_t n) {
  // powers of two up to 64, then multiples of 64 (one captured graph per count)
  if (n > 64) return (n + 63) / 64 * 64;
  int64_t b = 1;
  while (b < n) b *= 2;
  return b;
}

std::vector<int64_t> g_seqs, g_pos, g_extra, g_first;

// plan_pass(out32, o32, out64, o64, params, kind, seqs, positions, extra,
//           nb_force, grouped_force, ring_base)
//   -> (nb, n32, n64, grouped, kv_max, position_sum)
// kind "P" (extra = token ids or ring handles), "R" (extra = core steps) or
// "C" (extra = expected tokens or None). nb_force < 0: nb = the row bucket
// under graphs, else n; grouped_force < 0: group when it pays, else 0 / 1.
// ring_base < 0: the C rows' ids go to the trash ring slot.
PyObject* plan_pass(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 12) {
    PyErr_SetString(PyExc_TypeError, "plan_pass takes 12 arguments");
    return nullptr;
  }
  int64_t p[kNumParams];
  if (!read_params(args[4], p)) return nullptr;
  if (!PyUnicode_Check(args[5]) || PyUnicode_GET_LENGTH(args[5]) != 1) {
    PyErr_SetString(PyExc_ValueError, "kind: 'P', 'R' or 'C'");
    return nullptr;
  }
  const Py_UCS4 kind = PyUnicode_READ_CHAR(args[5], 0);
  if (kind != 'P' && kind != 'R' && kind != 'C') {
    PyErr_SetString(PyExc_ValueError, "kind: 'P', 'R' or 'C'");
    return nullptr;
  }
  const long long o32 = PyLong_AsLongLong(args[1]), o64 = PyLong_AsLongLong(args[3]);
  const long long nb_force = PyLong_AsLongLong(args[9]), grouped_force = PyLong_AsLongLong(args[10]);
  const long long ring_base = PyLong_AsLongLong(args[11]);
  if (PyErr_Occurred()) return nullptr;
  if (!read_ints(args[6], g_seqs, "seqs") || !read_ints(args[7], g_pos, "positions")) return nullptr;
  const bool has_extra = args[8] != Py_None;
  if (has_extra && !read_ints(args[8], g_extra, "extra")) return nullptr;
  const int64_t n = int64_t(g_pos.size());
  if (int64_t(g_seqs.size()) != n) {
    PyErr_SetString(PyExc_ValueError, "seqs and positions differ in length");
    return nullptr;
  }

  // -- validation (the row tables index the caches and the pool with these)
  const int64_t B = p[kB], S = p[kS];
  int64_t kv_max = 0, pos_sum = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t q = g_pos[i];
    if (q < 0 || q >= S) {
      PyErr_Format(PyExc_IndexError, "position out of range [0, %lld)", (long long)S);
      return nullptr;
    }
    if (q + 1 > kv_max) kv_max = q + 1;
    pos_sum += q;
  }
  for (int64_t i = 0; i < n; ++i) {
    const int64_t b = g_seqs[i];
    if (b < 0 || b >= B || b >= p[kMaxBatch]) {
      PyErr_SetString(PyExc_IndexError, "sequence index out of range");
      return nullptr;
    }
  }
  if (S > p[kMaxSeqLen]) {
    PyErr_SetString(PyExc_ValueError, "cache longer than the engine's tables (max_seq_len)");
    return nullptr;
  }
  const bool is_p = kind == 'P', is_r = kind == 'R', is_c = kind == 'C';
  if ((is_p || is_r) && !has_extra) {
    PyErr_SetString(PyExc_ValueError, is_p ? "a P pass needs token ids" : "an R pass needs core steps");
    return nullptr;
  }
  const bool expect = is_c && has_extra && !g_extra.empty();
  if ((is_p || is_r || expect) && int64_t(g_extra.size()) != n) {
    PyErr_SetString(PyExc_ValueError, "extra (ids / steps / expected tokens) differs in length from positions");
    return nullptr;
  }
  if (is_r) {
    for (int64_t i = 0; i < n; ++i) {
      if (g_extra[i] < 0 || g_extra[i] >= p[kTTotal]) {
        PyErr_Format(PyExc_ValueError, "core step out of range [0, %lld)", (long long)p[kTTotal]);
        return nullptr;
      }
    }
  }
  int64_t nb;
  if (nb_force >= 0) {
    nb = nb_force;
    if (nb < n) {
      PyErr_SetString(PyExc_ValueError, "nb below the row count");
      return nullptr;
    }
  } else {
    nb = p[kUseGraphs] ? bucket(n) : n;
    if (nb > p[kMaxRows]) {
      PyErr_Format(PyExc_ValueError, "union of %lld rows exceeds max_rows=%lld", (long long)n,
                   (long long)p[kMaxRows]);
      return nullptr;
    }
  }

  // -- attention groups: adjacent rows reading the same slots (same sequence,
  // for R the same depth), at most kGroupMaxRows rows each
  const int64_t L = is_p ? p[kNPrelude] : is_r ? p[kNCore] : p[kNCoda];
  auto key = [&](int64_t i) { return is_r ? g_seqs[i] * (p[kTTotal] + 1) + g_extra[i] : g_seqs[i]; };
  bool grouped = false;
  g_first.clear();
  if (grouped_force > 0 || (grouped_force < 0 && p[kGroupAttention] && n >= 2)) {
    bool shared = grouped_force > 0;
    for (int64_t i = 1; i < n && !shared; ++i) shared = key(i) == key(i - 1);
    if (shared) {
      if (n > 0) g_first.push_back(0);
      for (int64_t i = 1; i < n; ++i)
        if (key(i) != key(i - 1) || i - g_first.back() >= p[kGroupMaxRows]) g_first.push_back(i);
      grouped = grouped_force > 0 || int64_t(g_first.size()) * p[kNKvHeads] >= p[kGroupMinWorkgroups];
    }
  }

  // -- tables
  const int64_t nblk = is_c ? 4 : 3;
  const int64_t n32 = nblk * nb + (grouped ? nb + 1 : 0);
  const int64_t n64 = (is_p ? nb : 0) + 2 * L * nb + (is_c ? nb : 0);
  OutBuf b32, b64;
  if (!b32.get(args[0], 4, "out32") || !b64.get(args[2], 8, "out64")) return nullptr;
  if (o32 < 0 || o64 < 0 || o32 + n32 > b32.size() || o64 + n64 > b64.size()) {
    PyErr_SetString(PyExc_ValueError, "table scratch too small for the pass");
    return nullptr;
  }
  int32_t* t32 = static_cast<int32_t*>(b32.v.buf) + o32;
  int64_t* t64 = static_cast<int64_t*>(b64.v.buf) + o64;
  const int64_t R = p[kPoolR];
  for (int64_t i = 0; i < nb; ++i) {
    const bool live = i < n;
    t32[i] = live ? int32_t(g_pos[i]) : 0;
    t32[nb + i] = live ? int32_t(g_pos[i] + 1) : 1;
    t32[2 * nb + i] = live ? int32_t(g_seqs[i] * R + g_pos[i] % R) : int32_t(p[kTrashPoolRow]);
    if (is_c) t32[3 * nb + i] = (live && ring_base >= 0) ? int32_t(ring_base + i) : int32_t(p[kRingLen]);
  }
  if (grouped) {
    int32_t* gf = t32 + nblk * nb;
    int64_t k = 0;
    for (int64_t f : g_first) gf[k++] = int32_t(f);
    for (int64_t i = n; i <= nb; ++i) gf[k++] = int32_t(i);  // padding rows one by one, then the end
    for (; k <= nb; ++k) gf[k] = int32_t(nb);
  }
  int64_t* rb = t64 + (is_p ? nb : 0);
  int64_t* fr = rb + L * nb;
  if (is_p)
    for (int64_t i = 0; i < nb; ++i) t64[i] = i < n ? g_extra[i] : 0;
  for (int64_t l = 0; l < L; ++l) {
    for (int64_t i = 0; i < nb; ++i) {
      if (i >= n) {
        rb[l * nb + i] = fr[l * nb + i] = p[kTrashRow];
        continue;
      }
      const int64_t slot = is_p ? l : is_r ? p[kNPrelude] + g_extra[i] * p[kNCore] + l : p[kCodaBase] + l;
      rb[l * nb + i] = (slot * B + g_seqs[i]) * S;
      fr[l * nb + i] = rb[l * nb + i] + g_pos[i];
    }
  }
  if (is_c) {
    int64_t* ex = fr + L * nb;
    for (int64_t i = 0; i < nb; ++i) ex[i] = (expect && i < n) ? g_extra[i] : kNoExpect;
  }
  return Py_BuildValue("(LLLOLL)", (long long)nb, (long long)n32, (long long)n64, grouped ? Py_True : Py_False,
                       (long long)kv_max, (long long)pos_sum);
}

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  PyErr_Format(PyExc_RuntimeError, "%s failed: %s", what, hipGetErrorString(e));
  return false;
}

void* as_ptr(PyObject* o) { return PyLong_AsVoidPtr(o); }

// Accept flags in mapped, coherent pinned host memory: the argmax kernel
// stores each C row's flag (0 / 1) straight into it, and the host polls for
// the tick's flags instead of copying them back behind the graph. A flag
// reads -1 until the tick's kernel has written it.
void clear_flags(void* flags, long long n) {
  volatile int32_t* f = static_cast<volatile int32_t*>(flags);
  for (long long i = 0; i < n; ++i) f[i] = -1;
  std::atomic_thread_fence(std::memory_order_seq_cst);  // cleared before the launch that rewrites them
}

// launch(graph_exec, stream, event, pinned, dev, out64, n64, out32, n32, flags, nflags)
// Waits for `event` (the last upload out of `pinned`), packs the first n64
// words of out64 and n32 of out32 into `pinned` ([int64 | int32]), copies them
// to `dev` on `stream`, records `event` behind the copy, clears the first
// nflags accept flags at `flags` (host address; 0: none) and launches the
// graph (graph_exec 0: the copy only).
PyObject* launch(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 11) {
    PyErr_SetString(PyExc_TypeError, "launch takes 11 arguments");
    return nullptr;
  }
  auto exec = static_cast<hipGraphExec_t>(as_ptr(args[0]));
  auto stream = static_cast<hipStream_t>(as_ptr(args[1]));
  auto event = static_cast<hipEvent_t>(as_ptr(args[2]));
  auto* pinned = static_cast<char*>(as_ptr(args[3]));
  void* dev = as_ptr(args[4]);
  const long long n64 = PyLong_AsLongLong(args[6]), n32 = PyLong_AsLongLong(args[8]);
  void* flags = as_ptr(args[9]);
  const long long nflags = PyLong_AsLongLong(args[10]);
  if (PyErr_Occurred()) return nullptr;
  if (nflags < 0 || (nflags > 0 && flags == nullptr)) {
    PyErr_SetString(PyExc_ValueError, "launch: bad accept flag buffer");
    return nullptr;
  }
  if (event == nullptr || pinned == nullptr || dev == nullptr) {
    PyErr_SetString(PyExc_ValueError, "launch: null event / pinned / device buffer");
    return nullptr;
  }
  OutBuf b64, b32;
  if (!b64.get(args[5], 8, "out64") || !b32.get(args[7], 4, "out32")) return nullptr;
  if (n64 < 0 || n32 < 0 || n64 > b64.size() || n32 > b32.size()) {
    PyErr_SetString(PyExc_ValueError, "launch: table sizes beyond the scratch");
    return nullptr;
  }
  if (!hip_ok(hipEventSynchronize(event), "hipEventSynchronize")) return nullptr;
  std::memcpy(pinned, b64.v.buf, size_t(n64) * 8);
  std::memcpy(pinned + n64 * 8, b32.v.buf, size_t(n32) * 4);
  const size_t bytes = size_t(n64) * 8 + size_t(n32) * 4;
  if (!hip_ok(hipMemcpyAsync(dev, pinned, bytes, hipMemcpyHostToDevice, stream), "hipMemcpyAsync")) return nullptr;
  if (!hip_ok(hipEventRecord(event, stream), "hipEventRecord")) return nullptr;
  if (nflags > 0) clear_flags(flags, nflags);
  if (exec != nullptr && !hip_ok(hipGraphLaunch(exec, stream), "hipGraphLaunch")) return nullptr;
  Py_RETURN_NONE;
}

// host_alloc(nbytes) -> (host address, device address) of mapped, coherent
// pinned memory, every byte 0xff (flags read -1)
PyObject* host_alloc(PyObject*, PyObject* arg) {
  const size_t n = PyLong_AsSize_t(arg);
  if (PyErr_Occurred()) return nullptr;
  void* h = nullptr;
  if (!hip_ok(hipHostMalloc(&h, n ? n : 1, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc"))
    return nullptr;
  void* d = nullptr;
  if (!hip_ok(hipHostGetDevicePointer(&d, h, 0), "hipHostGetDevicePointer")) {
    (void)hipHostFree(h);
    return nullptr;
  }
  std::memset(h, 0xff, n);
  return Py_BuildValue("(NN)", PyLong_FromVoidPtr(h), PyLong_FromVoidPtr(d));
}

PyObject* host_free(PyObject*, PyObject* arg) {
  void* h = as_ptr(arg);
  if (PyErr_Occurred()) return nullptr;
  if (h != nullptr && !hip_ok(hipHostFree(h), "hipHostFree")) return nullptr;
  Py_RETURN_NONE;
}

// clear_flags(host address, n): every flag -1 (for launches made without `launch`)
PyObject* clear_flags_py(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 2) {
    PyErr_SetString(PyExc_TypeError, "clear_flags takes 2 arguments");
    return nullptr;
  }
  void* f = as_ptr(args[0]);
  const long long n = PyLong_AsLongLong(args[1]);
  if (PyErr_Occurred()) return nullptr;
  if (f == nullptr || n < 0) {
    PyErr_SetString(PyExc_ValueError, "clear_flags: bad flag buffer");
    return nullptr;
  }
  clear_flags(f, n);
  Py_RETURN_NONE;
}

// wait_flags(host address, n, timeout_s) -> [bool] * n once every flag is
// written (>= 0), or None after timeout_s seconds (the GIL is released while
// polling)
PyObject* wait_flags(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 3) {
    PyErr_SetString(PyExc_TypeError, "wait_flags takes 3 arguments");
    return nullptr;
  }
  const volatile int32_t* f = static_cast<const volatile int32_t*>(as_ptr(args[0]));
  const long long n = PyLong_AsLongLong(args[1]);
  const double timeout = PyFloat_AsDouble(args[2]);
  if (PyErr_Occurred()) return nullptr;
  if (f == nullptr || n < 0) {
    PyErr_SetString(PyExc_ValueError, "wait_flags: bad flag buffer");
    return nullptr;
  }
  bool done = false;
  Py_BEGIN_ALLOW_THREADS
  const auto t0 = std::chrono::steady_clock::now();
  for (long long spin = 0;; ++spin) {
    long long i = 0;
    while (i < n && f[i] >= 0) ++i;
    if (i == n) {
      done = true;
      break;
    }
    if ((spin & 255) == 0 &&
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() >= timeout)
      break;
    __builtin_ia32_pause();
  }
  Py_END_ALLOW_THREADS
  std::atomic_thread_fence(std::memory_order_acquire);
  if (!done) Py_RETURN_NONE;
  PyObject* out = PyList_New(n);
  if (out == nullptr) return nullptr;
  for (long long i = 0; i < n; ++i) {
    PyObject* b = f[i] ? Py_True : Py_False;
    Py_INCREF(b);
    PyList_SET_ITEM(out, i, b);
  }
  return out;
}

// event_create(device) -> handle of a timing-free event on that device
PyObject* event_create(PyObject*, PyObject* arg) {
  const long dev = PyLong_AsLong(arg);
  if (dev == -1 && PyErr_Occurred()) return nullptr;
  int old = 0;
  if (!hip_ok(hipGetDevice(&old), "hipGetDevice")) return nullptr;
  if (!hip_ok(hipSetDevice(int(dev)), "hipSetDevice")) return nullptr;
  hipEvent_t e = nullptr;
  const hipError_t rc = hipEventCreateWithFlags(&e, hipEventDisableTiming);
  hipSetDevice(old);
  if (!hip_ok(rc, "hipEventCreateWithFlags")) return nullptr;
  return PyLong_FromVoidPtr(e);
}

// event_destroy(handle): waits for the event first, so the copy it follows
// no longer reads the pinned buffer its owner is about to free
PyObject* event_destroy(PyObject*, PyObject* arg) {
  auto e = static_cast<hipEvent_t>(as_ptr(arg));
  if (PyErr_Occurred()) return nullptr;
  if (e == nullptr) Py_RETURN_NONE;
  if (!hip_ok(hipEventSynchronize(e), "hipEventSynchronize")) return nullptr;
  if (!hip_ok(hipEventDestroy(e), "hipEventDestroy")) return nullptr;
  Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"plan_pass", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(plan_pass)), METH_FASTCALL,
     "Validate one pass's rows and write its row tables; returns (nb, n32, n64, grouped, kv_max, position_sum)."},
    {"launch", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(launch)), METH_FASTCALL,
     "Upload a tick's tables through a pinned buffer and launch its graph."},
    {"host_alloc", host_alloc, METH_O, "Mapped, coherent pinned host memory: (host address, device address)."},
    {"host_free", host_free, METH_O, "Free memory from host_alloc."},
    {"clear_flags", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(clear_flags_py)), METH_FASTCALL,
     "Set n int32 accept flags to -1."},
    {"wait_flags", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(wait_flags)), METH_FASTCALL,
     "Poll n int32 accept flags until all are written; [bool] or None on timeout."},
    {"event_create", event_create, METH_O, "A timing-free HIP event on the given device."},
    {"event_destroy", event_destroy, METH_O, "Wait for and destroy an event made by event_create."},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_tick", "Host side of a decode tick (row tables, upload, launch).",
                       -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__tick(void) {
  PyObject* m = PyModule_Create(&kModule);
  if (m == nullptr) return nullptr;
  if (PyModule_AddIntConstant(m, "NUM_PARAMS", kNumParams) != 0) return nullptr;
  return m;
}
