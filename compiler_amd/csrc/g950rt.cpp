// g950rt -- the single gfx950 module loader and launcher (C ABI in
// include/g950rt.h).
//
// It takes the place of the reference's native runtime for the hot-path
// operators: the bundle/pool/operator_entry machinery of
// a100c/runtime/{main.c,pool.c,bundle.c} and the per-operator assembly that
// a100c/backend emits.  One code object holds every kernel; an operator call
// is (op contract, views, scalars) in the reference's sorted-argument-name
// order (a100_support/native_io.py:74,81).  The launcher
//   1. validates every view against its allocation (reach inside storage,
//      dtype, rank, contiguity the kernel assumes) and every scalar against
//      the views (the reference passes redundant shape/stride scalars; a
//      mismatch is a refusal, never a silent reinterpretation),
//   2. picks the kernel variant from dtypes, extents, strides and alignment,
//   3. fills the kernel's argument block and launches it on the caller's
//      stream.
// Nothing is launched unless every check passed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/g950rt.h"
#include "g950_args.h"

using namespace g950;

struct g950_module {
  hipModule_t mod = nullptr;
  int device = -1;
  int cus = 256;  // compute units of the device (persistent grid sizing)
  std::mutex mu;
  std::unordered_map<std::string, hipFunction_t> fns;
  // per-stream device workspace (split-row partials, the widened and
  // transposed copies of B, unsigned int8 sums); launches on one stream are
  // ordered, so each stream owns one buffer, grown on demand
  std::mutex ws_mu;
  std::unordered_map<void*, std::pair<void*, size_t>> ws;
  // device address of the library's static scratch array on this device
  // (g950_launch_noalloc), looked up at open; null with scratch_err set if the
  // lookup failed
  char* scratch = nullptr;
  hipError_t scratch_err = hipSuccess;
};

// g950_scratch.hip (same library)
hipError_t g950_scratch_address(int device, void** out);

namespace {

thread_local std::string t_error;
thread_local std::string t_kernel;
// Set while a g950_launch_noalloc call is dispatched on this thread: the
// device address of the module's scratch array, which then serves every
// workspace request instead of hipMalloc.
thread_local char* t_scratch = nullptr;
constexpr size_t kScratchWorkspace = G950_NOALLOC_SCRATCH_BYTES;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_error = buf;
  return code;
}

int itemsize(uint32_t dt) {
  static const int sizes[] = {0, 1, 1, 1, 2, 2, 4, 4, 8, 8, 2, 2, 4, 8};
  return dt < 14 ? sizes[dt] : 0;
}

const char* dtname(uint32_t dt) {
  static const char* names[] = {"?", "bool", "int8", "uint8", "int16", "uint16", "int32",
                                "uint32", "int64", "uint64", "float16", "bfloat16",
                                "float32", "float64"};
  return dt < 14 ? names[dt] : "?";
}

bool is_float16ish(uint32_t dt) { return dt == G950_DTYPE_BFLOAT16 || dt == G950_DTYPE_FLOAT16; }
bool is_float(uint32_t dt) { return is_float16ish(dt) || dt == G950_DTYPE_FLOAT32; }

// A checked view: extents and ELEMENT strides.
struct View {
  const char* name = "";
  const g950_view* v = nullptr;
  int nd = 0;
  int64_t shape[8] = {};
  int64_t stride[8] = {};  // elements
  int isz = 0;
  uintptr_t addr() const { return (uintptr_t)v->data; }
};

// ndim < 0: any rank from 1 to 8 (views the kernel addresses as flat arrays)
int check_view(const g950_view* views, uint32_t idx, const char* name, int ndim, View& out,
               bool output) {
  const g950_view& v = views[idx];
  out.name = name;
  out.v = &v;
  if (ndim < 0) {
    if (v.ndim < 1 || v.ndim > 8) return fail(G950_REJECTED, "view %s: rank %u (1..8 accepted)", name, v.ndim);
    ndim = (int)v.ndim;
  }
  if ((int)v.ndim != ndim)
    return fail(G950_REJECTED, "view %s: rank %u, contract needs %d", name, v.ndim, ndim);
  if (!v.shape || !v.strides) return fail(G950_REJECTED, "view %s: null shape/strides", name);
  out.isz = itemsize(v.dtype);
  if (!out.isz) return fail(G950_REJECTED, "view %s: unknown dtype code %u", name, v.dtype);
  if (v.flags & ~1u) return fail(G950_REJECTED, "view %s: reserved flag bits set", name);
  if (output && !(v.flags & G950_VIEW_OUTPUT))
    return fail(G950_REJECTED, "view %s: output argument lacks the output flag", name);
  out.nd = ndim;
  __int128 lo = 0, hi = 0;  // 128-bit: caller strides times extents cannot wrap
  bool empty = false;
  for (int i = 0; i < ndim; ++i) {
    out.shape[i] = v.shape[i];
    if (v.shape[i] < 0) return fail(G950_REJECTED, "view %s: negative extent", name);
    if (v.shape[i] == 0) empty = true;
    if (v.strides[i] % out.isz)
      return fail(G950_REJECTED, "view %s: byte stride %lld not a multiple of the item size",
                  name, (long long)v.strides[i]);
    out.stride[i] = v.strides[i] / out.isz;
    if (v.strides[i] < 0) lo += (__int128)v.strides[i] * (v.shape[i] - 1);
    else hi += (__int128)v.strides[i] * (v.shape[i] - 1);
  }
  // an empty view is never dereferenced and may carry null pointers
  if (!empty && (!v.data || !v.storage)) return fail(G950_REJECTED, "view %s: null device pointer", name);
  if (!empty) {
    const __int128 base = (intptr_t)v.data - (intptr_t)v.storage;
    if (base + lo < 0 || base + hi + out.isz > (__int128)v.storage_size)
      return fail(G950_REJECTED, "view %s: reach [%lld, %lld) outside its %llu-byte storage", name,
                  (long long)(base + lo), (long long)(base + hi + out.isz),
                  (unsigned long long)v.storage_size);
  }
  return G950_OK;
}

// A view the reference kernel addresses as one flat element array (base
// pointer plus scalar offsets): any rank, C-contiguous; `elems` = its length.
int flat_view(const g950_view* views, uint32_t idx, const char* name, View& out, bool output,
              long long& elems) {
  if (int rc = check_view(views, idx, name, -1, out, output)) return rc;
  elems = 1;
  long long expect = 1;
  for (int i = out.nd - 1; i >= 0; --i) {
    if (out.shape[i] > 1 && out.stride[i] != expect)
      return fail(G950_USAGE, "view %s: must be contiguous (the kernel indexes it as a flat array)", name);
    expect *= out.shape[i];
    elems *= out.shape[i];
  }
  return G950_OK;
}

int scalar_int(const g950_scalar* s, const char* name, long long& out) {
  switch (s->dtype) {
    case G950_DTYPE_BOOL: case G950_DTYPE_UINT8: out = (long long)(s->bits & 0xFF); break;
    case G950_DTYPE_INT8: out = (int8_t)(s->bits & 0xFF); break;
    case G950_DTYPE_INT16: out = (int16_t)(s->bits & 0xFFFF); break;
    case G950_DTYPE_UINT16: out = (long long)(s->bits & 0xFFFF); break;
    case G950_DTYPE_INT32: out = (int32_t)(s->bits & 0xFFFFFFFFu); break;
    case G950_DTYPE_UINT32: out = (long long)(s->bits & 0xFFFFFFFFu); break;
    case G950_DTYPE_INT64: case G950_DTYPE_UINT64: out = (long long)s->bits; break;
    default: return fail(G950_USAGE, "scalar %s: dtype %s is not an integer", name, dtname(s->dtype));
  }
  return G950_OK;
}

int scalar_float(const g950_scalar* s, const char* name, double& out) {
  if (s->dtype == G950_DTYPE_FLOAT32) {
    float f;
    uint32_t b = (uint32_t)s->bits;
    memcpy(&f, &b, 4);
    out = f;
  } else if (s->dtype == G950_DTYPE_FLOAT64) {
    memcpy(&out, &s->bits, 8);
  } else {
    long long i;
    if (scalar_int(s, name, i)) return fail(G950_USAGE, "scalar %s: not a number", name);
    out = (double)i;
  }
  return G950_OK;
}

int expect_int(const g950_scalar* scalars, uint32_t idx, const char* name, long long want) {
  long long got;
  if (int rc = scalar_int(&scalars[idx], name, got)) return rc;
  if (got != want)
    return fail(G950_USAGE, "scalar %s = %lld disagrees with the views (%lld)", name, got, want);
  return G950_OK;
}

hipFunction_t function(g950_module* m, const std::string& name) {
  std::lock_guard<std::mutex> lock(m->mu);
  auto it = m->fns.find(name);
  if (it != m->fns.end()) return it->second;
  hipFunction_t f = nullptr;
  if (hipModuleGetFunction(&f, m->mod, name.c_str()) != hipSuccess) {
    // a kernel the code object does not hold is an answer, not an error:
    // clear the thread's last-error state so the caller's next check (a
    // framework's launch check, say) does not report it
    (void)hipGetLastError();
    return nullptr;
  }
  m->fns.emplace(name, f);
  return f;
}

template <class Args>
int launch(g950_module* m, const std::string& name, unsigned grid, unsigned block, Args& args,
           void* stream) {
  if (!m) {  // validation only (g950_validate): report the choice, launch nothing
    t_kernel = name;
    return G950_OK;
  }
  hipFunction_t f = function(m, name);
  if (!f) return fail(G950_RESOURCE, "kernel %s not found in the code object", name.c_str());
  if (grid == 0) {  // nothing to do (empty extent)
    t_kernel = name;
    return G950_OK;
  }
  void* params[] = {&args};
  hipError_t e = hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, (hipStream_t)stream, params,
                                       nullptr);
  if (e != hipSuccess)
    return fail(G950_RESOURCE, "launch of %s failed: %s", name.c_str(), hipGetErrorString(e));
  t_kernel = name;
  return G950_OK;
}

bool aligned16(uintptr_t p) { return (p & 15) == 0; }

// Workgroup size a kernel was built for (its launch bounds); `dflt` when
// validating without a module.
int kernel_threads(g950_module* m, const char* name, int dflt) {
  if (!m) return dflt;
  hipFunction_t f = function(m, name);
  int v = 0;
  if (!f || hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f) != hipSuccess || v <= 0)
    return dflt;
  return v;
}

// ------------------------------------------------------------ row reductions
// Register configurations in order of preference: the first whose
// items*block vectors cover the row is used.  One wavefront per row while the
// row fits (no LDS round trip in the reductions), then 4-wave workgroups.
// `waves` is the resident-wave target per CU that sizes the persistent grid
// (measured on MI355X: one-row-per-wave shapes do best with many small
// workgroups, the 16-vector shapes with fewer, longer-lived ones).
struct RowCfg { int items, block, waves; };
const RowCfg kRowCfgs[] = {{1, 64, 32}, {2, 64, 32}, {4, 64, 32}, {6, 64, 32}, {8, 64, 32},
                           {16, 64, 8}, {8, 256, 16}, {16, 256, 8}};

// Persistent grid for `rows` rows of BLOCK-thread workgroups: at most
// `waves` resident waves per CU, balanced so every workgroup gets
// ceil(rows / grid) or one fewer rows.
unsigned row_grid(const g950_module* m, long long rows, int block, int waves) {
  const long long cus = m ? m->cus : 256;
  const long long per_cu = waves / (block / 64) > 0 ? waves / (block / 64) : 1;
  const long long cap = cus * per_cu;
  if (rows <= cap) return (unsigned)rows;
  const long long k = (rows + cap - 1) / cap;
  return (unsigned)((rows + k - 1) / k);
}

const char* rr_dtype(uint32_t dt) {
  return dt == G950_DTYPE_FLOAT32 ? "f32" : dt == G950_DTYPE_BFLOAT16 ? "bf16" : "f16";
}

// Device workspace of at least `bytes` for launches on `stream`.  Growing it
// waits for the stream (the old buffer may still be read by queued work).
int workspace(g950_module* m, void* stream, size_t bytes, void** out) {
  if (t_scratch) {
    if (bytes > kScratchWorkspace)
      return fail(G950_USAGE, "no-alloc launch: the call needs %zu bytes of workspace, the scratch array holds %zu",
                  bytes, kScratchWorkspace);
    *out = t_scratch;
    return G950_OK;
  }
  std::lock_guard<std::mutex> lock(m->ws_mu);
  auto& w = m->ws[stream];
  if (w.second < bytes) {
    if (w.first) {
      if (hipError_t e = hipStreamSynchronize((hipStream_t)stream))
        return fail(G950_SYNC, "workspace: %s", hipGetErrorString(e));
      (void)hipFree(w.first);
      w = {nullptr, 0};
    }
    // headroom for a larger next call, at most 64 MiB beyond the request
    const size_t grow = std::min(bytes, (size_t)64 << 20);
    const size_t n = (bytes < (size_t)65536 ? (size_t)65536 : bytes + grow + 255) & ~(size_t)255;
    if (hipError_t e = hipMalloc(&w.first, n)) {
      w = {nullptr, 0};
      return fail(G950_RESOURCE, "workspace: hipMalloc(%zu): %s", n, hipGetErrorString(e));
    }
    w.second = n;
  }
  *out = w.first;
  return G950_OK;
}

template <class Args>
int launch(g950_module* m, const std::string& name, unsigned grid, unsigned block, Args& args, void* stream);

// Split rows (rowreduce.hip, rs_*): chunks of 1024 vectors (RS_BLOCK 256 x
// RS_ITEMS 4), one workgroup per (row, chunk), two launches.
constexpr long long kRsChunkVecs = 1024;

int launch_split_rows(g950_module* m, const char* op, RowArgs& a, uint32_t dt, int v, void* stream) {
  const long long nvec = a.cols / v;
  const long long splits = (nvec + kRsChunkVecs - 1) / kRsChunkVecs;
  const long long blocks = (long long)a.rows * splits;
  if (blocks > 0x7FFFFFFF) return fail(G950_USAGE, "%s: too many row chunks", op);
  a.splits = (int)splits;
  a.part = nullptr;
  if (m && blocks) {
    if (int rc = workspace(m, stream, (size_t)blocks * 16, &a.part)) return rc;
  }
  char name[128];
  snprintf(name, sizeof name, "g950_rs_part_%s_%s_v%d", op, rr_dtype(dt), v);
  if (int rc = launch(m, name, (unsigned)blocks, 256u, a, stream)) return rc;
  snprintf(name, sizeof name, "g950_rs_final_%s_%s_v%d", op, rr_dtype(dt), v);
  const bool lse = strcmp(op, "logsumexp") == 0;
  return launch(m, name, (unsigned)(lse ? a.rows : blocks), 256u, a, stream);
}

// Pick and launch the row kernel.  `params` are the per-column parameter
// views (W, B) whose alignment the vector form also needs.
int launch_rows(g950_module* m, const char* op, RowArgs& a, uint32_t dt, const View& x,
                const View& y, const View* p0, const View* p1, void* stream) {
  const int isz = itemsize(dt);
  const int vmax = 16 / isz;
  bool vec = (a.cols % vmax == 0) && aligned16(x.addr()) && aligned16(y.addr()) &&
             ((a.x_row * isz) % 16 == 0) && ((a.y_row * isz) % 16 == 0);
  if (p0) vec = vec && aligned16(p0->addr());
  if (p1) vec = vec && aligned16(p1->addr());
  char name[128];
  // rows that are not whole aligned 16-byte vectors: masked aligned vectors
  // when one wave holds a row at any phase and y's rows share x's phase
  // (empty rows never: their start address need not lie in any allocation)
  if (!vec && a.cols > 0 && (isz == 2 || isz == 4) && ((x.addr() - y.addr()) % 16) == 0 &&
      (((a.x_row - a.y_row) * isz) % 16) == 0 && (x.addr() % isz) == 0) {
    static const int kItems[] = {1, 2, 4, 6, 8};
    for (int items : kItems) {
      if ((long long)items * 64 * vmax >= (long long)a.cols + vmax - 1) {
        snprintf(name, sizeof name, "g950_rm_%s_%s_v%d_i%d", op, rr_dtype(dt), vmax, items);
        return launch(m, name, (unsigned)((a.rows + 7) / 8), 256u, a, stream);
      }
    }
  }
  const int v = vec ? vmax : 1;
  const int nvec = a.cols / v;
  const RowCfg* pick = nullptr;
  for (const RowCfg& c : kRowCfgs)
    if (c.items * c.block >= nvec) { pick = &c; break; }
  // one workgroup per row leaves most of the chip idle when rows are few and
  // long: split them (two or more chunks each) instead
  const long long cus = m ? m->cus : 256;
  const bool few = (long long)a.rows * 2 < cus && nvec > kRsChunkVecs;
  // LayerNorm over many rows of at most 512 vectors: parameters staged in LDS
  // once per 4-wave workgroup of 8 rows (g950_rw_*) instead of once per
  // one-row wave
  const bool ln = !strcmp(op, "layernorm") || !strcmp(op, "lnrow");
  if (ln && vec && pick && pick->block == 64 && pick->items <= 8 && (long long)a.rows >= 16 * cus) {
    snprintf(name, sizeof name, "g950_rw_%s_%s_v%d_i%d", op, rr_dtype(dt), v, pick->items);
    return launch(m, name, (unsigned)((a.rows + 7) / 8), 256u, a, stream);
  }
  if (pick && !few) {
    snprintf(name, sizeof name, "g950_rr_%s_%s_v%d_i%d_b%d", op, rr_dtype(dt), v, pick->items,
             pick->block);
    return launch(m, name, row_grid(m, a.rows, pick->block, pick->waves), (unsigned)pick->block, a,
                  stream);
  }
  return launch_split_rows(m, op, a, dt, v, stream);
}

int row_common(const View& x, const View& y) {
  if (!is_float(x.v->dtype) || x.v->dtype != y.v->dtype)
    return fail(G950_USAGE, "row op: x/y dtypes %s/%s unsupported (float32, bfloat16, float16, same)",
                dtname(x.v->dtype), dtname(y.v->dtype));
  if (x.shape[0] != y.shape[0] || x.shape[1] != y.shape[1])
    return fail(G950_USAGE, "row op: x and y shapes differ");
  if (x.shape[1] > 1 && (x.stride[1] != 1 || y.stride[1] != 1))
    return fail(G950_USAGE, "row op: the reduced (last) axis must be contiguous");
  if (x.shape[0] > 0x7FFFFFFF || x.shape[1] > 0x7FFFFFFF)
    return fail(G950_USAGE, "row op: extent too large");
  return G950_OK;
}

int op_softmax(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
               uint32_t nsc, void* stream) {
  if (nviews != 2 || nsc != 1) return fail(G950_USAGE, "softmax: needs views (x_ptr, y_ptr), scalars (n_cols)");
  View x, y;
  if (int rc = check_view(views, 0, "x_ptr", 2, x, false)) return rc;
  if (int rc = check_view(views, 1, "y_ptr", 2, y, true)) return rc;
  if (int rc = row_common(x, y)) return rc;
  if (int rc = expect_int(sc, 0, "n_cols", x.shape[1])) return rc;
  RowArgs a{};
  a.x = x.v->data; a.y = y.v->data;
  a.x_row = x.stride[0]; a.y_row = y.stride[0];
  a.rows = (int)x.shape[0]; a.cols = (int)x.shape[1];
  if (a.cols == 0) return fail(G950_USAGE, "softmax: empty row");
  return launch_rows(m, "softmax", a, x.v->dtype, x, y, nullptr, nullptr, stream);
}

int op_logsumexp(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                 uint32_t nsc, void* stream) {
  if (nviews != 2 || nsc != 1) return fail(G950_USAGE, "logsumexp: needs views (x_ptr, y_ptr), scalars (n_cols)");
  View x, y;
  if (int rc = check_view(views, 0, "x_ptr", 2, x, false)) return rc;
  if (int rc = check_view(views, 1, "y_ptr", 1, y, true)) return rc;
  if (!is_float(x.v->dtype) || !is_float(y.v->dtype))
    return fail(G950_USAGE, "logsumexp: x/y dtypes %s/%s unsupported (float32, bfloat16, float16)",
                dtname(x.v->dtype), dtname(y.v->dtype));
  if (y.shape[0] != x.shape[0]) return fail(G950_USAGE, "logsumexp: y needs one entry per row");
  if (int rc = expect_int(sc, 0, "n_cols", x.shape[1])) return rc;
  RowArgs a{};
  a.x = x.v->data;
  a.x_row = x.stride[0]; a.y_row = x.stride[0];
  a.stat0 = y.v->data; a.stat0_stride = y.stride[0]; a.stat_dtype = (int)y.v->dtype;
  a.rows = (int)x.shape[0]; a.cols = (int)x.shape[1];
  // an empty row reduces to max = -inf, which is its result (logsumexp.py:23-38)
  // no row output: x stands in for y in the vector-path alignment checks
  return launch_rows(m, "logsumexp", a, x.v->dtype, x, x, nullptr, nullptr, stream);
}

int stat_view(const View& s, const View& x, const char* what) {
  if (!is_float(s.v->dtype)) return fail(G950_USAGE, "%s: dtype %s unsupported", what, dtname(s.v->dtype));
  if (s.shape[0] != x.shape[0]) return fail(G950_USAGE, "%s: needs one entry per row", what);
  return G950_OK;
}

int param_view(const View& p, const View& x, const char* what) {
  if (p.v->dtype != x.v->dtype) return fail(G950_USAGE, "%s: dtype must match X", what);
  if (p.shape[0] != x.shape[1]) return fail(G950_USAGE, "%s: needs one entry per column", what);
  if (p.shape[0] > 1 && p.stride[0] != 1) return fail(G950_USAGE, "%s: must be contiguous", what);
  return G950_OK;
}

int op_rms(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
           uint32_t nsc, void* stream) {
  if (nviews != 4 || nsc != 6)
    return fail(G950_USAGE, "rms_layernorm: needs views (W, X, Y, r) and 6 scalars");
  View w, x, y, r;
  if (int rc = check_view(views, 0, "W", 1, w, false)) return rc;
  if (int rc = check_view(views, 1, "X", 2, x, false)) return rc;
  if (int rc = check_view(views, 2, "Y", 2, y, true)) return rc;
  if (int rc = check_view(views, 3, "r", 1, r, true)) return rc;
  if (int rc = row_common(x, y)) return rc;
  if (int rc = param_view(w, x, "W")) return rc;
  if (int rc = stat_view(r, x, "r")) return rc;
  long long wrs;
  if (int rc = scalar_int(&sc[0], "W_row_stride", wrs)) return rc;
  if (int rc = expect_int(sc, 1, "X_row_stride", x.stride[0])) return rc;
  if (int rc = expect_int(sc, 2, "Y_row_stride", y.stride[0])) return rc;
  double eps;
  if (int rc = scalar_float(&sc[3], "eps", eps)) return rc;
  if (int rc = expect_int(sc, 4, "n_cols", x.shape[1])) return rc;
  if (int rc = expect_int(sc, 5, "r_row_stride", r.stride[0])) return rc;
  RowArgs a{};
  a.x = x.v->data; a.y = y.v->data; a.w = w.v->data; a.stat0 = r.v->data;
  a.x_row = x.stride[0]; a.y_row = y.stride[0]; a.stat0_stride = r.stride[0];
  a.rows = (int)x.shape[0]; a.cols = (int)x.shape[1];
  a.eps = (float)eps; a.stat_dtype = (int)r.v->dtype;
  if (a.cols == 0) return fail(G950_USAGE, "rms_layernorm: empty row");
  return launch_rows(m, "rmsnorm", a, x.v->dtype, x, y, &w, nullptr, stream);
}

int op_layernorm(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                 uint32_t nsc, void* stream) {
  if (nviews != 6 || nsc != 3)
    return fail(G950_USAGE, "layernorm: needs views (B, Mean, Rstd, W, X, Y), scalars (N, eps, stride)");
  View b, mean, rstd, w, x, y;
  if (int rc = check_view(views, 0, "B", 1, b, false)) return rc;
  if (int rc = check_view(views, 1, "Mean", 1, mean, true)) return rc;
  if (int rc = check_view(views, 2, "Rstd", 1, rstd, true)) return rc;
  if (int rc = check_view(views, 3, "W", 1, w, false)) return rc;
  if (int rc = check_view(views, 4, "X", 2, x, false)) return rc;
  if (int rc = check_view(views, 5, "Y", 2, y, true)) return rc;
  if (int rc = row_common(x, y)) return rc;
  if (int rc = param_view(w, x, "W")) return rc;
  if (int rc = param_view(b, x, "B")) return rc;
  if (int rc = stat_view(mean, x, "Mean")) return rc;
  if (int rc = stat_view(rstd, x, "Rstd")) return rc;
  if (mean.v->dtype != rstd.v->dtype) return fail(G950_USAGE, "layernorm: Mean/Rstd dtypes differ");
  if (int rc = expect_int(sc, 0, "N", x.shape[1])) return rc;
  double eps;
  if (int rc = scalar_float(&sc[1], "eps", eps)) return rc;
  if (x.stride[0] != y.stride[0]) return fail(G950_USAGE, "layernorm: X and Y share one row stride");
  if (int rc = expect_int(sc, 2, "stride", x.stride[0])) return rc;
  RowArgs a{};
  a.x = x.v->data; a.y = y.v->data; a.w = w.v->data; a.b = b.v->data;
  a.stat0 = mean.v->data; a.stat1 = rstd.v->data;
  a.x_row = x.stride[0]; a.y_row = y.stride[0];
  a.stat0_stride = mean.stride[0]; a.stat1_stride = rstd.stride[0];
  a.rows = (int)x.shape[0]; a.cols = (int)x.shape[1];
  a.eps = (float)eps; a.stat_dtype = (int)mean.v->dtype;
  if (a.cols == 0) return fail(G950_USAGE, "layernorm: empty row");
  return launch_rows(m, "layernorm", a, x.v->dtype, x, y, &w, &b, stream);
}

// softmax_kernel_inner (ops/suite/dev/softmax_kernel_inner.py:12-72): row
// softmax of M rows of N contiguous elements at input_ptr + m * N, written to
// output_ptr + m * N (flat buffers; the masked tail reads -inf).  With the
// constexprs given (scalars M, N, ONE_TILE_PER_CTA, TILE_N), the one-tile
// form with TILE_N < N normalises only the first TILE_N elements of each
// row and leaves the rest of the output row untouched (:13-24: one
// tl.arange(0, TILE_N) tile, masked by n < N); every other combination
// covers the whole row (:25-72).
int op_softmax_inner(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                     uint32_t nsc, void* stream) {
  if (nviews != 2 || (nsc != 2 && nsc != 4))
    return fail(G950_USAGE, "softmax_inner: needs views (input_ptr, output_ptr), scalars (M, N) or "
                "(M, N, ONE_TILE_PER_CTA, TILE_N)");
  View x, y;
  long long nx, ny, M, N;
  if (int rc = flat_view(views, 0, "input_ptr", x, false, nx)) return rc;
  if (int rc = flat_view(views, 1, "output_ptr", y, true, ny)) return rc;
  if (!is_float(x.v->dtype) || x.v->dtype != y.v->dtype)
    return fail(G950_USAGE, "softmax_inner: input/output dtypes %s/%s unsupported (float32, bfloat16, float16, same)",
                dtname(x.v->dtype), dtname(y.v->dtype));
  if (int rc = scalar_int(&sc[0], "M", M)) return rc;
  if (int rc = scalar_int(&sc[1], "N", N)) return rc;
  if (M < 0 || N < 0 || M > 0x7FFFFFFF || N > 0x7FFFFFFF) return fail(G950_USAGE, "softmax_inner: M, N out of range");
  if (M * N > nx || M * N > ny)
    return fail(G950_USAGE, "softmax_inner: M x N = %lld elements exceed input_ptr (%lld) or output_ptr (%lld)",
                M * N, nx, ny);
  long long cols = N;
  if (nsc == 4) {
    long long one_tile, tile_n;
    if (int rc = scalar_int(&sc[2], "ONE_TILE_PER_CTA", one_tile)) return rc;
    if (int rc = scalar_int(&sc[3], "TILE_N", tile_n)) return rc;
    if (tile_n <= 0) return fail(G950_USAGE, "softmax_inner: TILE_N = %lld must be positive", tile_n);
    if (one_tile && tile_n < N) cols = tile_n;
  }
  RowArgs a{};
  a.x = x.v->data; a.y = y.v->data;
  a.x_row = N; a.y_row = N;
  a.rows = (int)M; a.cols = (int)cols;
  if (M == 0 || N == 0) return launch(m, "g950_rr_softmax_f32_v1_i1_b64", 0, 64u, a, stream);  // nothing stored
  return launch_rows(m, "softmax", a, x.v->dtype, x, y, nullptr, nullptr, stream);
}

// _layer_norm_forward_row (ops/suite/dev/layer_norm_forward_row.py:11-36):
// flat buffers addressed by the row-stride scalars; n_rows, n_cols and eps
// are the kernel's constexprs.
int op_layernorm_row(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                     uint32_t nsc, void* stream) {
  if (nviews != 6 || nsc != 7)
    return fail(G950_USAGE, "layer_norm_forward_row: needs views (B_ptr, Mean_ptr, RSTD_ptr, W_ptr, X_ptr, Y_ptr), "
                "scalars (Mean_row_stride, RSTD_row_stride, X_row_stride, Y_row_stride, eps, n_cols, n_rows)");
  View b, mean, rstd, w, x, y;
  long long nb, nm, nr, nw, nx, ny;
  if (int rc = flat_view(views, 0, "B_ptr", b, false, nb)) return rc;
  if (int rc = flat_view(views, 1, "Mean_ptr", mean, true, nm)) return rc;
  if (int rc = flat_view(views, 2, "RSTD_ptr", rstd, true, nr)) return rc;
  if (int rc = flat_view(views, 3, "W_ptr", w, false, nw)) return rc;
  if (int rc = flat_view(views, 4, "X_ptr", x, false, nx)) return rc;
  if (int rc = flat_view(views, 5, "Y_ptr", y, true, ny)) return rc;
  const uint32_t dt = x.v->dtype;
  if (!is_float(dt) || y.v->dtype != dt || w.v->dtype != dt || b.v->dtype != dt)
    return fail(G950_USAGE, "layer_norm_forward_row: X_ptr, Y_ptr, W_ptr, B_ptr must share one float dtype");
  if (!is_float(mean.v->dtype) || mean.v->dtype != rstd.v->dtype)
    return fail(G950_USAGE, "layer_norm_forward_row: Mean_ptr/RSTD_ptr must share one float dtype");
  long long ms, rs, xs, ys, nc, nrow;
  double eps;
  if (int rc = scalar_int(&sc[0], "Mean_row_stride", ms)) return rc;
  if (int rc = scalar_int(&sc[1], "RSTD_row_stride", rs)) return rc;
  if (int rc = scalar_int(&sc[2], "X_row_stride", xs)) return rc;
  if (int rc = scalar_int(&sc[3], "Y_row_stride", ys)) return rc;
  if (int rc = scalar_float(&sc[4], "eps", eps)) return rc;
  if (int rc = scalar_int(&sc[5], "n_cols", nc)) return rc;
  if (int rc = scalar_int(&sc[6], "n_rows", nrow)) return rc;
  if (nc <= 0 || nrow < 0 || nc > 0x7FFFFFFF || nrow > 0x7FFFFFFF)
    return fail(G950_USAGE, "layer_norm_forward_row: n_cols must be positive, n_rows non-negative");
  if (ms < 0 || rs < 0 || xs < 0 || ys < 0) return fail(G950_USAGE, "layer_norm_forward_row: negative row stride");
  if (nrow > 1 && (ys < nc || ms < 1 || rs < 1))
    return fail(G950_USAGE, "layer_norm_forward_row: output rows overlap (Y_row_stride < n_cols or a zero statistic stride)");
  if (nw < nc || nb < nc) return fail(G950_USAGE, "layer_norm_forward_row: W_ptr/B_ptr need n_cols entries");
  // (n_rows - 1) * stride + width <= elements, in 128-bit arithmetic (the
  // strides are caller scalars)
  auto fits = [&](long long stride, long long width, long long n) {
    return (__int128)(nrow - 1) * stride + width <= (__int128)n;
  };
  if (nrow > 0 && !(fits(xs, nc, nx) && fits(ys, nc, ny) && fits(ms, 1, nm) && fits(rs, 1, nr)))
    return fail(G950_USAGE, "layer_norm_forward_row: n_rows rows exceed X_ptr, Y_ptr, Mean_ptr or RSTD_ptr");
  RowArgs a{};
  a.x = x.v->data; a.y = y.v->data; a.w = w.v->data; a.b = b.v->data;
  a.stat0 = mean.v->data; a.stat1 = rstd.v->data;
  a.x_row = xs; a.y_row = ys; a.stat0_stride = ms; a.stat1_stride = rs;
  a.rows = (int)nrow; a.cols = (int)nc;
  a.eps = (float)eps; a.stat_dtype = (int)mean.v->dtype;
  if (nrow == 0) return launch(m, "g950_rr_lnrow_f32_v1_i1_b64", 0, 64u, a, stream);
  return launch_rows(m, "lnrow", a, dt, x, y, &w, &b, stream);
}

// --------------------------------------------------------------------- GEMM
int gemm_tiles(GemmArgs& g) {
  const long long tm = (g.M + 255) / 256, tn = (g.N + 255) / 256;
  if (tm * tn > 0x7FFFFFFF) return -1;
  g.tiles_m = (int)tm;
  g.tiles_n = (int)tn;
  return (int)(tm * tn);
}

// A[M,K] and B[K,N] both K-contiguous with 16-byte rows (K a whole number of
// 16-byte chunks): the MFMA kernels apply -- the plain ones when K is a whole
// number of 128-byte slabs, else the _kt ones (gemm_ktail).
bool gemm_fast_ok(const View& a, const View& b, int K, int esz) {
  return a.stride[1] == 1 && b.stride[0] == 1 && (K * esz) % 16 == 0 && K > 0 &&
         aligned16(a.addr()) && aligned16(b.addr()) && (a.stride[0] * esz) % 16 == 0 &&
         (b.stride[1] * esz) % 16 == 0 && a.shape[0] > 0 && b.shape[1] > 0;
}

bool gemm_ktail(int K, int esz) { return (K * esz) % 128 != 0; }

// The whole-slab MFMA kernels address a lane's DMA rows by 32-bit byte
// offsets from the operand base (gemm.hip, gemm_mfma_body): the farthest row
// either operand can reach plus a slab's last 16-byte chunk must lie below
// 4 GiB, or the _kt kernels (64-bit addresses) serve the call.
bool gemm_off32(const GemmArgs& g, int esz) {
  auto fits = [esz](long long rows, long long s0) {
    return (__int128)(rows - 1) * s0 * esz + 128 <= (__int128)0xFFFFFFFFll;
  };
  return fits(g.M, g.a_s0) && fits(g.N, g.b_s0);
}

// Row-major B[K,N] (N-contiguous, the reference matmul's layout,
// ops/suite/perf/matmul.py:33) with A K-contiguous, 16-byte aligned rows: the
// 16-bit shapes the `_rb` MFMA kernels take are read as they lie; the others
// (fp32, a dimension under one tile, a K tail) copy B once into a
// K-contiguous Bt in the workspace (g950_transpose_b16/_b32) first.
bool gemm_rowb_ok(const View& a, const View& b, int K, int N, int esz) {
  const int per16 = 16 / esz;  // elements per 16-byte vector
  return (esz == 2 || esz == 4) && a.stride[1] == 1 && b.stride[1] == 1 && K % per16 == 0 && N % per16 == 0 &&
         K > 0 && aligned16(a.addr()) && aligned16(b.addr()) &&
         (a.stride[0] * esz) % 16 == 0 && (b.stride[0] * esz) % 16 == 0 && a.shape[0] > 0 && N > 0;
}

int gemm_views(const View& a, const View& b, const View& y, const g950_scalar* sc, long long& M,
               long long& N, long long& K) {
  M = a.shape[0]; K = a.shape[1]; N = b.shape[1];
  if (b.shape[0] != K) return fail(G950_USAGE, "matmul: a is [%lld,%lld] but b has %lld rows", M, K, (long long)b.shape[0]);
  if (y.shape[0] != M || y.shape[1] != N) return fail(G950_USAGE, "matmul: output must be [M,N]");
  if (M > 0x7FFFFFFF || N > 0x7FFFFFFF || K > 0x7FFFFFFF) return fail(G950_USAGE, "matmul: extent too large");
  if (int rc = expect_int(sc, 0, "K", K)) return rc;
  if (int rc = expect_int(sc, 1, "M", M)) return rc;
  if (int rc = expect_int(sc, 2, "N", N)) return rc;
  return G950_OK;
}

int op_matmul(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
              uint32_t nsc, void* stream) {
  if (nviews != 3 || nsc != 3) return fail(G950_USAGE, "matmul: needs views (a_ptr, b_ptr, y_ptr), scalars (K, M, N)");
  View a, b, y;
  if (int rc = check_view(views, 0, "a_ptr", 2, a, false)) return rc;
  if (int rc = check_view(views, 1, "b_ptr", 2, b, false)) return rc;
  if (int rc = check_view(views, 2, "y_ptr", 2, y, true)) return rc;
  long long M, N, K;
  if (int rc = gemm_views(a, b, y, sc, M, N, K)) return rc;
  if (!is_float(a.v->dtype) || !is_float(b.v->dtype) || !is_float(y.v->dtype))
    return fail(G950_USAGE, "matmul: float32/bfloat16/float16 operands only");
  GemmArgs g{};
  g.a = a.v->data; g.b = b.v->data; g.c = y.v->data;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.a_dtype = (int)a.v->dtype; g.b_dtype = (int)b.v->dtype; g.c_dtype = (int)y.v->dtype;
  g.c_s0 = y.stride[0]; g.c_s1 = y.stride[1];
  if (M == 0 || N == 0) return launch(m, "g950_gemm_general", 0, 256, g, stream);
  // both operands of one dtype: bf16 / f16 (v_mfma_f32_32x32x16) or fp32
  // (v_mfma_f32_32x32x2_f32) on the 256x256 MFMA kernel
  const bool same16 = a.v->dtype == b.v->dtype && is_float(a.v->dtype);
  const int esz = a.isz;
  const bool out16 = y.stride[1] == 1 && aligned16(y.addr());
  char mfma_name[48];
  // (call once g.a_s0 / g.b_s0 hold the operand row strides)
  auto mfma_kernel = [&]() -> const char* {
    snprintf(mfma_name, sizeof mfma_name, "g950_gemm_%s_256x256%s", rr_dtype(a.v->dtype),
             gemm_ktail((int)K, esz) || !gemm_off32(g, esz) ? "_kt" : "");
    return mfma_name;
  };
  if (same16 && gemm_fast_ok(a, b, (int)K, esz) && out16) {
    g.a_s0 = a.stride[0];
    g.b_s0 = b.stride[1];  // Bt row (n) stride
    const int tiles = gemm_tiles(g);
    if (tiles < 0) return fail(G950_USAGE, "matmul: too many tiles");
    const char* name = mfma_kernel();
    return launch(m, name, (unsigned)tiles, (unsigned)kernel_threads(m, name, 512), g, stream);
  }
  const bool rowb_ok = same16 && out16 && gemm_rowb_ok(a, b, (int)K, (int)N, esz);
  // Row-major B read directly by the 16x16 MFMA kernel (transposing LDS
  // reads): 16-bit operands, at least one 256 tile each way, whole 64-k
  // slabs, A's farthest DMA row within a 32-bit offset (B's lane offsets
  // span 16 k-rows of one slab)
  if (rowb_ok && esz == 2 && M >= 256 && N >= 256 && K % 64 == 0 &&
      (__int128)(M - 1) * a.stride[0] * 2 + 128 <= (__int128)0xFFFFFFFFll) {
    g.a_s0 = a.stride[0];
    g.b_s0 = b.stride[0];  // k-row stride of B
    const int tiles = gemm_tiles(g);
    if (tiles < 0) return fail(G950_USAGE, "matmul: too many tiles");
    const char* name = a.v->dtype == G950_DTYPE_BFLOAT16 ? "g950_gemm_bf16_256x256_rb" : "g950_gemm_f16_256x256_rb";
    return launch(m, name, (unsigned)tiles, 512u, g, stream);
  }
  // Other row-major shapes (fp32, a dimension under one tile, a K tail): B
  // is copied once into a K-contiguous Bt in the workspace, then the MFMA
  // kernel runs on the copy.  A failed allocation is an error; under
  // g950_launch_noalloc a copy larger than the scratch array runs the
  // general kernel instead (the documented no-alloc fallback).
  void* bt = nullptr;
  const size_t bt_bytes = (size_t)N * (size_t)K * esz;
  bool rowb = rowb_ok && bt_bytes <= ((size_t)1 << 31);
  if (rowb && m) {
    if (t_scratch && bt_bytes > kScratchWorkspace) {
      rowb = false;
    } else if (int rc = workspace(m, stream, bt_bytes, &bt)) {
      return rc;
    }
  }
  if (rowb) {
    GemmArgs t{};
    t.b = g.b; t.b_s0 = b.stride[0]; t.c = bt; t.N = (int)N; t.K = (int)K;
    const long long tblocks = ((K + 63) / 64) * ((N + 63) / 64);
    if (tblocks > 0x7FFFFFFF) return fail(G950_USAGE, "matmul: too many tiles");
    if (int rc = launch(m, esz == 2 ? "g950_transpose_b16" : "g950_transpose_b32", (unsigned)tblocks, 256u, t,
                        stream))
      return rc;
    g.b = bt;
    g.a_s0 = a.stride[0];
    g.b_s0 = K;
    const int tiles = gemm_tiles(g);
    if (tiles < 0) return fail(G950_USAGE, "matmul: too many tiles");
    const char* name = mfma_kernel();
    return launch(m, name, (unsigned)tiles, (unsigned)kernel_threads(m, name, 512), g, stream);
  }
  g.a_s0 = a.stride[0]; g.a_s1 = a.stride[1];
  g.b_s0 = b.stride[0]; g.b_s1 = b.stride[1];
  g.tiles_n = (int)((N + 63) / 64);
  const long long blocks = ((M + 63) / 64) * g.tiles_n;
  if (blocks > 0x7FFFFFFF) return fail(G950_USAGE, "matmul: too many tiles");
  return launch(m, "g950_gemm_general", (unsigned)blocks, 256u, g, stream);
}

int op_matmul_i8(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                 uint32_t nsc, bool dequant, void* stream) {
  const uint32_t want = dequant ? 5 : 3;
  if (nviews != want || nsc != 3)
    return fail(G950_USAGE, dequant ? "matmul_i8_dequant: needs views (a_ptr, b_ptr, sa_ptr, sb_ptr, y_ptr), scalars (K, M, N)"
                                    : "matmul_i8: needs views (a_ptr, b_ptr, c_ptr), scalars (K, M, N)");
  View a, b, y, sa, sb;
  if (int rc = check_view(views, 0, "a_ptr", 2, a, false)) return rc;
  if (int rc = check_view(views, 1, "b_ptr", 2, b, false)) return rc;
  if (dequant) {
    if (int rc = check_view(views, 2, "sa_ptr", 1, sa, false)) return rc;
    if (int rc = check_view(views, 3, "sb_ptr", 1, sb, false)) return rc;
    if (int rc = check_view(views, 4, "y_ptr", 2, y, true)) return rc;
  } else {
    if (int rc = check_view(views, 2, "c_ptr", 2, y, true)) return rc;
  }
  auto byte_int = [](uint32_t dt) { return dt == G950_DTYPE_INT8 || dt == G950_DTYPE_UINT8; };
  if (!byte_int(a.v->dtype) || !byte_int(b.v->dtype))
    return fail(G950_USAGE, "matmul_i8: operands must be int8 or uint8");
  long long M, N, K;
  if (int rc = gemm_views(a, b, y, sc, M, N, K)) return rc;
  GemmArgs g{};
  g.a = a.v->data; g.b = b.v->data;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.a_dtype = (int)a.v->dtype;
  g.b_dtype = (int)b.v->dtype;
  // signedness pair (a100c/plan/tiles.py:121-126): bit 0 A unsigned, bit 1 B unsigned
  const int umask = (a.v->dtype == G950_DTYPE_UINT8 ? 1 : 0) | (b.v->dtype == G950_DTYPE_UINT8 ? 2 : 0);
  if (dequant) {
    if (sa.v->dtype != G950_DTYPE_FLOAT32 || sb.v->dtype != G950_DTYPE_FLOAT32)
      return fail(G950_USAGE, "matmul_i8_dequant: scales must be float32");
    if (sa.shape[0] != M || sb.shape[0] != N) return fail(G950_USAGE, "matmul_i8_dequant: scale extents");
    if ((M > 1 && sa.stride[0] != 1) || (N > 1 && sb.stride[0] != 1))
      return fail(G950_USAGE, "matmul_i8_dequant: scales must be contiguous");
    if (!is_float(y.v->dtype)) return fail(G950_USAGE, "matmul_i8_dequant: float output only");
    g.sa = (const float*)sa.v->data; g.sb = (const float*)sb.v->data;
    g.c = y.v->data; g.c_dtype = (int)y.v->dtype;
    g.c_s0 = y.stride[0]; g.c_s1 = y.stride[1];
  } else {
    if (y.v->dtype != G950_DTYPE_INT32) return fail(G950_USAGE, "matmul_i8: c_ptr must be int32");
    if (N > 1 && y.stride[1] != 1) return fail(G950_USAGE, "matmul_i8: c_ptr rows must be contiguous");
    g.acc_out = (int*)y.v->data; g.acc_s0 = y.stride[0];
  }
  if (M == 0 || N == 0) return launch(m, "g950_gemm_general_i8", 0, 256, g, stream);
  const bool out_ok = dequant ? (y.stride[1] == 1 && aligned16(y.addr())) : aligned16(y.addr());
  // an unsigned operand's flipped bytes would read the zero tail as -128:
  // the signedness variants need whole 128-byte K slabs and 32-bit row
  // offsets (they have no _kt form)
  g.a_s0 = a.stride[0];
  g.b_s0 = b.stride[1];
  const bool ktail = gemm_ktail((int)K, 1) || !gemm_off32(g, 1);
  if (gemm_fast_ok(a, b, (int)K, 1) && out_ok && (umask == 0 || !ktail)) {
    const int tiles = gemm_tiles(g);
    if (tiles < 0) return fail(G950_USAGE, "matmul_i8: too many tiles");
    static const char* const names[4] = {"g950_gemm_i8_256x256", "g950_gemm_u8s8_256x256",
                                         "g950_gemm_s8u8_256x256", "g950_gemm_u8u8_256x256"};
    if (umask) {
      // the MFMA multiplies u - 128 for an unsigned operand: first the sums
      // over k its correction needs (A's rows if B is unsigned, B's columns
      // if A is), into the workspace
      I8SumArgs sa{};
      sa.a = g.a; sa.b = g.b; sa.a_s0 = g.a_s0; sa.b_s0 = g.b_s0;
      sa.a_rows = (umask & 2) ? (int)M : 0;
      sa.b_rows = (umask & 1) ? (int)N : 0;
      sa.a_signed = a.v->dtype == G950_DTYPE_INT8;
      sa.b_signed = b.v->dtype == G950_DTYPE_INT8;
      sa.K = (int)K;
      const long long rows = (long long)sa.a_rows + sa.b_rows;
      void* ws = nullptr;
      if (m)
        if (int rc = workspace(m, stream, (size_t)rows * 4, &ws)) return rc;
      sa.out = (int*)ws;
      g.rsum = (umask & 2) ? sa.out : nullptr;
      g.csum = (umask & 1) ? sa.out + sa.a_rows : nullptr;
      if (int rc = launch(m, "g950_i8_sums", (unsigned)((rows + 3) / 4), 256u, sa, stream)) return rc;
    }
    {
      const char* name = ktail ? "g950_gemm_i8_256x256_kt" : names[umask];
      return launch(m, name, (unsigned)tiles, (unsigned)kernel_threads(m, name, 512), g, stream);
    }
  }
  if (!dequant && N > 1 && y.stride[1] != 1) return fail(G950_USAGE, "matmul_i8: c_ptr layout");
  g.a_s0 = a.stride[0]; g.a_s1 = a.stride[1];
  g.b_s0 = b.stride[0]; g.b_s1 = b.stride[1];
  g.tiles_n = (int)((N + 63) / 64);
  const long long blocks = ((M + 63) / 64) * g.tiles_n;
  if (blocks > 0x7FFFFFFF) return fail(G950_USAGE, "matmul_i8: too many tiles");
  return launch(m, "g950_gemm_general_i8", (unsigned)blocks, 256u, g, stream);
}

// ---------------------------------------------------------- dequantisation
// The reference passes the strides as scalars; they must name the same
// elements as the views (checked wherever the extent makes them matter).
int stride_agrees(const g950_scalar* sc, uint32_t idx, const char* name, const View& v, int dim) {
  long long got;
  if (int rc = scalar_int(&sc[idx], name, got)) return rc;
  if (v.shape[dim] > 1 && got != v.stride[dim])
    return fail(G950_USAGE, "scalar %s = %lld disagrees with view %s (stride %lld)", name, got, v.name,
                (long long)v.stride[dim]);
  return G950_OK;
}

int op_dequantize(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                  uint32_t nsc, void* stream) {
  if (nviews != 3 || nsc != 6)
    return fail(G950_USAGE, "dequantize: needs views (b_ptr, b_scale_ptr, fpb_ptr), scalars "
                "(K, N, stride_bk, stride_bn, stride_fpbk, stride_fpbn)");
  View b, s, y;
  if (int rc = check_view(views, 0, "b_ptr", 2, b, false)) return rc;
  if (int rc = check_view(views, 1, "b_scale_ptr", 1, s, false)) return rc;
  if (int rc = check_view(views, 2, "fpb_ptr", 2, y, true)) return rc;
  if (b.v->dtype != G950_DTYPE_INT8) return fail(G950_USAGE, "dequantize: b_ptr must be int8");
  if (!is_float(y.v->dtype) || s.v->dtype != y.v->dtype)
    return fail(G950_USAGE, "dequantize: b_scale_ptr/fpb_ptr dtypes %s/%s (one of float32, bfloat16, float16)",
                dtname(s.v->dtype), dtname(y.v->dtype));
  const long long K = b.shape[0], N = b.shape[1];
  if (y.shape[0] != K || y.shape[1] != N) return fail(G950_USAGE, "dequantize: fpb_ptr must be [K, N]");
  if (s.shape[0] != N) return fail(G950_USAGE, "dequantize: b_scale_ptr needs one entry per column");
  if (int rc = expect_int(sc, 0, "K", K)) return rc;
  if (int rc = expect_int(sc, 1, "N", N)) return rc;
  if (int rc = stride_agrees(sc, 2, "stride_bk", b, 0)) return rc;
  if (int rc = stride_agrees(sc, 3, "stride_bn", b, 1)) return rc;
  if (int rc = stride_agrees(sc, 4, "stride_fpbk", y, 0)) return rc;
  if (int rc = stride_agrees(sc, 5, "stride_fpbn", y, 1)) return rc;
  DequantArgs a{};
  a.b = b.v->data; a.scale = s.v->data; a.y = y.v->data;
  a.b_sk = b.stride[0]; a.b_sn = b.stride[1];
  a.y_sk = y.stride[0]; a.y_sn = y.stride[1];
  a.s_sn = s.stride[0];
  a.k = K; a.n = N;
  a.y_dtype = (int)y.v->dtype;
  if (K == 0 || N == 0) return launch(m, "g950_dequant_i8_general", 0, 256u, a, stream);
  const int ysz = y.isz;
  const bool unit = (N == 1) || (b.stride[1] == 1 && y.stride[1] == 1 && s.stride[0] == 1);
  const int cols = 16 / ysz;  // one 16-byte y vector (4 fp32 / 8 16-bit) per lane and row
  const bool vec = unit && N % cols == 0 && (b.addr() % cols) == 0 && aligned16(y.addr()) &&
                   aligned16(s.addr()) && (K == 1 || ((b.stride[0] % cols) == 0 && (y.stride[0] * ysz) % 16 == 0));
  const unsigned cap = m ? (unsigned)m->cus * 8u : 2048u;
  if (vec) {
    const long long groups = (K + 3) / 4;  // DQ_ROWS rows per lane
    a.work = groups * (N / cols);
    if (a.work < 0x7FFFFFFF) {
      const long long blocks = (a.work + 255) / 256;
      const char* name = y.v->dtype == G950_DTYPE_FLOAT32 ? "g950_dequant_i8_f32"
                         : y.v->dtype == G950_DTYPE_BFLOAT16 ? "g950_dequant_i8_bf16" : "g950_dequant_i8_f16";
      return launch(m, name, (unsigned)(blocks < cap ? blocks : cap), 256u, a, stream);
    }
  }
  const long long blocks = (K * N + 255) / 256;
  return launch(m, "g950_dequant_i8_general", (unsigned)(blocks < cap ? blocks : cap), 256u, a, stream);
}

// Fused weight dequantisation + GEMM (W8A16): y = a . (b * b_scale[n]).
int op_dequant_matmul(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                      uint32_t nsc, void* stream) {
  if (nviews != 4 || nsc != 3)
    return fail(G950_USAGE, "dequant_matmul: needs views (a_ptr, b_ptr, b_scale_ptr, y_ptr), scalars (K, M, N)");
  View a, b, s, y;
  if (int rc = check_view(views, 0, "a_ptr", 2, a, false)) return rc;
  if (int rc = check_view(views, 1, "b_ptr", 2, b, false)) return rc;
  if (int rc = check_view(views, 2, "b_scale_ptr", 1, s, false)) return rc;
  if (int rc = check_view(views, 3, "y_ptr", 2, y, true)) return rc;
  long long M, N, K;
  if (int rc = gemm_views(a, b, y, sc, M, N, K)) return rc;
  if (b.v->dtype != G950_DTYPE_INT8) return fail(G950_USAGE, "dequant_matmul: b_ptr must be int8");
  if (!is_float(a.v->dtype) || !is_float(y.v->dtype) || s.v->dtype != a.v->dtype)
    return fail(G950_USAGE, "dequant_matmul: a_ptr, b_scale_ptr (same dtype) and y_ptr must be float");
  if (s.shape[0] != N) return fail(G950_USAGE, "dequant_matmul: b_scale_ptr needs one entry per column");
  GemmArgs g{};
  g.a = a.v->data; g.b = b.v->data; g.c = y.v->data;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.a_dtype = (int)a.v->dtype; g.b_dtype = G950_DTYPE_INT8; g.c_dtype = (int)y.v->dtype;
  g.c_s0 = y.stride[0]; g.c_s1 = y.stride[1];
  g.bscale = s.v->data; g.bscale_dtype = (int)s.v->dtype;
  if (M == 0 || N == 0) return launch(m, "g950_gemm_general", 0, 256, g, stream);
  if (N > 1 && s.stride[0] != 1) {
    // the kernels index the scale densely: only a contiguous scale row is taken
    return fail(G950_USAGE, "dequant_matmul: b_scale_ptr must be contiguous");
  }
  // 16-bit A with K-contiguous rows, output rows contiguous
  const bool a16 = is_float16ish(a.v->dtype) && K % 16 == 0 && (K < 2 || a.stride[1] == 1) && a.stride[0] % 8 == 0 &&
                   aligned16(a.addr()) && y.stride[1] == 1 && aligned16(y.addr());
  // int8 B stored K-contiguous (Bt [N, K]) with 16-byte rows
  bool fast = a16 && (K < 2 || b.stride[0] == 1) && b.stride[1] % 16 == 0 && aligned16(b.addr());
  long long bts = b.stride[1];  // Bt row (n) stride of the operand the fast routes read
  const long long cus = m ? m->cus : 256;
  const bool bf16 = a.v->dtype == G950_DTYPE_BFLOAT16;
  // The reference's own weight layout, int8 b row-major [K, N] (stride_bk = N,
  // stride_bn = 1, ops/suite/perf/dequantize_matmul.py:62-65):
  //   * at least one 256 tile each way and whole 64-k slabs: the weights are
  //     widened as they lie into an exact bf16 / f16 [K, N] copy in the
  //     workspace, and the row-major-B MFMA kernel runs on it with the scale
  //     in its epilogue;
  //   * otherwise the int8 weights are transposed once into a K-contiguous
  //     copy in the workspace and the routes below (B-streaming decode
  //     kernels, fused 128x128 kernel) run on it.
  // Under g950_launch_noalloc a copy larger than the scratch array leaves
  // the call to the general kernel (the documented no-alloc fallback).
  const bool nrow = a16 && !fast && K > 1 && N > 1 && b.stride[1] == 1 && N % 16 == 0 && b.stride[0] % 16 == 0 &&
                    aligned16(b.addr());
  auto fits = [&](unsigned long long bytes) {
    return bytes <= (1ull << 31) && !(t_scratch && bytes > kScratchWorkspace);
  };
  if (nrow && M >= 256 && N >= 256 && K % 64 == 0 && fits((unsigned long long)K * N * 2) &&
      (__int128)(M - 1) * a.stride[0] * 2 + 128 <= (__int128)0xFFFFFFFFll) {
    void* wide = nullptr;
    if (m)
      if (int rc = workspace(m, stream, (size_t)(K * N * 2), &wide)) return rc;
    GemmArgs w{};
    w.b = g.b; w.b_s0 = b.stride[0]; w.N = (int)K; w.K = (int)N;  // K rows of N weights
    w.c = wide;
    const long long chunks = K * (N / 16);
    if (int rc = launch(m, bf16 ? "g950_widen_i8_bf16" : "g950_widen_i8_f16", (unsigned)((chunks + 255) / 256), 256u,
                        w, stream))
      return rc;
    g.b = wide; g.b_dtype = (int)a.v->dtype;
    g.a_s0 = a.stride[0];
    g.b_s0 = N;  // k-row stride of the copy
    g.bscale = nullptr;
    g.cscale = s.v->data; g.cscale_dtype = (int)s.v->dtype;
    const int tiles = gemm_tiles(g);
    if (tiles < 0) return fail(G950_USAGE, "dequant_matmul: too many tiles");
    const char* name = bf16 ? "g950_gemm_bf16_256x256_rb" : "g950_gemm_f16_256x256_rb";
    return launch(m, name, (unsigned)tiles, 512u, g, stream);
  }
  bool transposed = false;
  if (nrow && fits((unsigned long long)K * N)) {
    void* bt = nullptr;
    if (m)
      if (int rc = workspace(m, stream, (size_t)(K * N), &bt)) return rc;
    GemmArgs t{};
    t.b = g.b; t.b_s0 = b.stride[0]; t.c = bt; t.N = (int)N; t.K = (int)K;
    const long long tblocks = ((K + 63) / 64) * ((N + 63) / 64);
    if (tblocks > 0x7FFFFFFF) return fail(G950_USAGE, "dequant_matmul: too many tiles");
    if (int rc = launch(m, "g950_transpose_b8", (unsigned)tblocks, 256u, t, stream)) return rc;
    g.b = bt;
    bts = K;
    fast = true;
    transposed = true;  // the workspace now holds the copy: no second copy below
  }
  if (fast && M <= 64) {
    // decode shapes: the few-row kernels stream B, 32 columns and all of K
    // per workgroup (8 waves, one K range each, summed in LDS), for up to 16,
    // 32 or 64 rows of A.  With at most 16 rows, 16 columns per workgroup
    // (twice the workgroups, each reading all of A) where the 32-column grid
    // leaves CUs idle or exceeds them by more than a quarter, and for one row
    // of A.  Measured on MI355X (rotating inputs): 16x4096x4096 12.3 -> 9.1 us,
    // 16x4096x11008 27.1 -> 19.8, 16x11008x4096 22.2 -> 21.1, 1x8192x8192
    // 20.9 -> 15.1; 16x8192x8192 ties and 16x8192x8000 loses (21.7 -> 24.8).
    g.a_s0 = a.stride[0];
    g.b_s0 = bts;
    const long long blocks32 = (N + 31) / 32;
    const bool c16 = M <= 16 && (M == 1 || blocks32 < cus || 4 * blocks32 > 5 * cus);
    const long long blocks = c16 ? (N + 15) / 16 : blocks32;
    if (blocks > 0x7FFFFFFF) return fail(G950_USAGE, "dequant_matmul: too many tiles");
    char name[48];
    snprintf(name, sizeof name, "g950_gemm_w8a16_skinny%s_%s", c16 ? "_c16" : M <= 16 ? "" : M <= 32 ? "32" : "64",
             bf16 ? "bf16" : "f16");
    return launch(m, name, (unsigned)blocks, 512u, g, stream);
  }
  // Many output tiles: widen B once into an exact bf16 / f16 copy in the
  // workspace and run the 256x256 GEMM with the column scale in its epilogue.
  // The fused kernel converts every B element once per 128-row output tile,
  // which costs more than one copy (3 bytes per weight through HBM) once the
  // 256x256 tiles outnumber half the CUs.  Measured on MI355X at N = K = 8192:
  // M = 1024 (128 tiles) 186 us fused vs 148 + 36 us; M = 1536 334 vs 172 + 36.
  void* wide = nullptr;
  bool widened = fast && !transposed && K > 0 && K % 64 == 0 && 2 * ((M + 255) / 256) * ((N + 255) / 256) > cus &&
                 (unsigned long long)N * K * 2 <= (1ull << 31);
  // without room for the copy in the no-alloc scratch, the fused kernel below
  // (which needs none) serves the call; a failed allocation is an error
  if (widened && t_scratch && (size_t)(N * K * 2) > kScratchWorkspace) widened = false;
  if (widened && m)
    if (int rc = workspace(m, stream, (size_t)(N * K * 2), &wide)) return rc;
  if (widened) {
    GemmArgs w{};
    w.b = g.b; w.b_s0 = bts; w.N = (int)N; w.K = (int)K;
    void* ws = wide;
    w.c = ws;
    const long long chunks = N * (K / 16);
    if (int rc = launch(m, bf16 ? "g950_widen_i8_bf16" : "g950_widen_i8_f16", (unsigned)((chunks + 255) / 256), 256u,
                        w, stream))
      return rc;
    g.b = ws; g.b_dtype = (int)a.v->dtype;
    g.a_s0 = a.stride[0];
    g.b_s0 = K;
    g.bscale = nullptr;
    g.cscale = s.v->data; g.cscale_dtype = (int)s.v->dtype;
    const int tiles = gemm_tiles(g);
    if (tiles < 0) return fail(G950_USAGE, "dequant_matmul: too many tiles");
    {
      const bool off32 = gemm_off32(g, 2);
      const char* name = bf16 ? (off32 ? "g950_gemm_bf16_256x256" : "g950_gemm_bf16_256x256_kt")
                              : (off32 ? "g950_gemm_f16_256x256" : "g950_gemm_f16_256x256_kt");
      return launch(m, name, (unsigned)tiles, (unsigned)kernel_threads(m, name, 512), g, stream);
    }
  }
  if (fast) {
    g.a_s0 = a.stride[0];
    g.b_s0 = bts;  // Bt row (n) stride
    g.tiles_m = (int)((M + 127) / 128);
    g.tiles_n = (int)((N + 127) / 128);
    const long long tiles = (long long)g.tiles_m * g.tiles_n;
    if (tiles > 0x7FFFFFFF) return fail(G950_USAGE, "dequant_matmul: too many tiles");
    return launch(m, bf16 ? "g950_gemm_w8a16_bf16_128x128" : "g950_gemm_w8a16_f16_128x128", (unsigned)tiles, 256u, g,
                  stream);
  }
  g.a_s0 = a.stride[0]; g.a_s1 = a.stride[1];
  g.b_s0 = b.stride[0]; g.b_s1 = b.stride[1];
  g.tiles_n = (int)((N + 63) / 64);
  const long long blocks = ((M + 63) / 64) * g.tiles_n;
  if (blocks > 0x7FFFFFFF) return fail(G950_USAGE, "dequant_matmul: too many tiles");
  return launch(m, "g950_gemm_general", (unsigned)blocks, 256u, g, stream);
}

// ---------------------------------------------------------------- attention
int launch_attention(g950_module* m, AttnArgs& a, uint32_t dt, long long D, const View& q, const View& k,
                     const View& v, const View& o, void* stream);

int op_attention(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                 uint32_t nsc, bool with_lse, void* stream) {
  const uint32_t want = with_lse ? 5 : 4;
  if (nviews != want || nsc != 21)
    return fail(G950_USAGE, "attention: needs views (k_ptr,%s out_ptr, q_ptr, v_ptr) and 21 scalars "
                "(CAUSAL, H, N_CTX, Z, scale, 16 strides)", with_lse ? " lse_ptr," : "");
  View k, lse, o, q, v;
  uint32_t i = 0;
  if (int rc = check_view(views, i++, "k_ptr", 4, k, false)) return rc;
  if (with_lse)
    if (int rc = check_view(views, i++, "lse_ptr", 3, lse, true)) return rc;
  if (int rc = check_view(views, i++, "out_ptr", 4, o, true)) return rc;
  if (int rc = check_view(views, i++, "q_ptr", 4, q, false)) return rc;
  if (int rc = check_view(views, i++, "v_ptr", 4, v, false)) return rc;
  const uint32_t dt = q.v->dtype;
  if (!is_float(dt) || k.v->dtype != dt || v.v->dtype != dt || o.v->dtype != dt)
    return fail(G950_USAGE, "attention: q/k/v/out must share one float dtype");
  const long long Z = q.shape[0], H = q.shape[1], S = q.shape[2], D = q.shape[3];
  const long long Hkv = k.shape[1], Sk = k.shape[2];
  if (k.shape[0] != Z || k.shape[3] != D || v.shape[0] != Z || v.shape[1] != Hkv ||
      v.shape[2] != Sk || v.shape[3] != D)
    return fail(G950_USAGE, "attention: k/v shapes must be [Z, Hkv, Sk, D] matching q");
  if (o.shape[0] != Z || o.shape[1] != H || o.shape[2] != S || o.shape[3] != D)
    return fail(G950_USAGE, "attention: out must have q's shape");
  if (Hkv <= 0 || H % Hkv) return fail(G950_USAGE, "attention: H must be a multiple of the KV heads");
  if (with_lse) {
    if (lse.v->dtype != G950_DTYPE_FLOAT32) return fail(G950_USAGE, "attention: lse must be float32");
    if (lse.shape[0] != Z || lse.shape[1] != H || lse.shape[2] != S)
      return fail(G950_USAGE, "attention: lse must be [Z, H, N_CTX]");
  }
  if (D > 1 && (q.stride[3] != 1 || k.stride[3] != 1 || v.stride[3] != 1 || o.stride[3] != 1))
    return fail(G950_USAGE, "attention: head_dim must be contiguous");
  long long causal;
  if (int rc = scalar_int(&sc[0], "CAUSAL", causal)) return rc;
  if (int rc = expect_int(sc, 1, "H", H)) return rc;
  if (int rc = expect_int(sc, 2, "N_CTX", S)) return rc;
  if (int rc = expect_int(sc, 3, "Z", Z)) return rc;
  double scale;
  if (int rc = scalar_float(&sc[4], "scale", scale)) return rc;
  // stride scalars, sorted: k(h,k,n,z) o(h,m,n,z) q(h,k,m,z) v(h,k,n,z)
  const struct { const View* vw; const char* names[4]; int dims[4]; } st[4] = {
      {&k, {"stride_kh", "stride_kk", "stride_kn", "stride_kz"}, {1, 3, 2, 0}},
      {&o, {"stride_oh", "stride_om", "stride_on", "stride_oz"}, {1, 2, 3, 0}},
      {&q, {"stride_qh", "stride_qk", "stride_qm", "stride_qz"}, {1, 3, 2, 0}},
      {&v, {"stride_vh", "stride_vk", "stride_vn", "stride_vz"}, {1, 2, 3, 0}},
  };
  uint32_t si = 5;
  for (const auto& e : st)
    for (int j = 0; j < 4; ++j)
      if (int rc = expect_int(sc, si++, e.names[j], e.vw->stride[e.dims[j]])) return rc;
  if (Z * H > 0x7FFFFFF || S > 0x7FFFFFF || Sk > 0x7FFFFFF)
    return fail(G950_USAGE, "attention: extent too large");
  AttnArgs a{};
  a.q = q.v->data; a.k = k.v->data; a.v = v.v->data; a.o = o.v->data;
  a.lse = with_lse ? (float*)lse.v->data : nullptr;
  a.q_sz = q.stride[0]; a.q_sh = q.stride[1]; a.q_ss = q.stride[2];
  a.k_sz = k.stride[0]; a.k_sh = k.stride[1]; a.k_ss = k.stride[2];
  a.v_sz = v.stride[0]; a.v_sh = v.stride[1]; a.v_ss = v.stride[2];
  a.o_sz = o.stride[0]; a.o_sh = o.stride[1]; a.o_ss = o.stride[2];
  if (with_lse) { a.lse_sz = lse.stride[0]; a.lse_sh = lse.stride[1]; a.lse_ss = lse.stride[2]; }
  a.Z = (int)Z; a.Hq = (int)H; a.Hkv = (int)Hkv; a.Sq = (int)S; a.Sk = (int)Sk;
  a.scale_log2 = (float)(scale * 1.4426950408889634);
  a.causal = causal ? 1 : 0;
  a.group = (int)(H / Hkv);
  return launch_attention(m, a, dt, D, q, k, v, o, stream);
}

// Pick and launch the attention kernel for checked views (q/k/v/o head_dim
// contiguous) and a filled argument block.
int launch_attention(g950_module* m, AttnArgs& a, uint32_t dt, long long D, const View& q, const View& k,
                     const View& v, const View& o, void* stream) {
  if (a.Z == 0 || a.Hq == 0 || a.Sq == 0) return launch(m, "g950_attn_fwd_general", 0, 64, a, stream);
  if (a.Sk == 0) return fail(G950_USAGE, "attention: no keys");
  const long long Z = a.Z, H = a.Hq, S = a.Sq;
  // the MFMA kernel's running maximum assumes scale > 0 (scaling then commutes
  // with the maximum); other scales take the general kernel
  const bool mfma = is_float16ish(dt) && (D == 64 || D == 128) && a.scale_log2 > 0.0f &&
                    std::isfinite(a.scale_log2) &&
                    aligned16(q.addr()) && aligned16(k.addr()) && aligned16(v.addr()) &&
                    (o.addr() & 7) == 0 && q.stride[0] % 8 == 0 && q.stride[1] % 8 == 0 &&
                    q.stride[2] % 8 == 0 && k.stride[0] % 8 == 0 && k.stride[1] % 8 == 0 &&
                    k.stride[2] % 8 == 0 && v.stride[0] % 8 == 0 && v.stride[1] % 8 == 0 &&
                    v.stride[2] % 8 == 0 && o.stride[0] % 4 == 0 && o.stride[1] % 4 == 0 &&
                    o.stride[2] % 4 == 0;
  if (mfma) {
    // waves x 32 queries per workgroup (attention.hip instantiations)
    char name[64];
    snprintf(name, sizeof name, "g950_attn_fwd_%s_d%lld", dt == G950_DTYPE_BFLOAT16 ? "bf16" : "f16", D);
    const int threads = kernel_threads(m, name, 512);
    const int bq = threads / 2;
    a.nqb = (int)((S + bq - 1) / bq);
    const long long grid = (long long)a.nqb * Z * H;
    if (grid > 0x7FFFFFFF) return fail(G950_USAGE, "attention: grid too large");
    return launch(m, name, (unsigned)grid, (unsigned)threads, a, stream);
  }
  AttnGenArgs ga{};
  ga.a = a;
  ga.D = (int)D;
  ga.dtype = (int)dt;
  // the fp32 MFMA kernel's vector staging reads K/V rows as 16-byte vectors
  // at every (z, head, row): only for aligned bases and strides of whole vectors
  ga.kv_vec = dt == G950_DTYPE_FLOAT32 && aligned16(k.addr()) && aligned16(v.addr()) && a.k_sz % 4 == 0 &&
              a.k_sh % 4 == 0 && a.k_ss % 4 == 0 && a.v_sz % 4 == 0 && a.v_sh % 4 == 0 && a.v_ss % 4 == 0;
  if (D == 32 || D == 64 || D == 128) {
    // fp32 (and 16-bit inputs the kernel above does not take) on the fp32
    // MFMA: 4 waves x 32 queries per workgroup, any scale
    char name[48];
    snprintf(name, sizeof name, "g950_attn_fwd_f32mfma_d%lld", D);
    ga.a.nqb = (int)((S + 127) / 128);
    const long long grid = (long long)ga.a.nqb * Z * H;
    if (grid > 0x7FFFFFFF) return fail(G950_USAGE, "attention: grid too large");
    return launch(m, name, (unsigned)grid, 256u, ga, stream);
  }
  const long long rows = Z * H * S;
  return launch(m, "g950_attn_fwd_general", (unsigned)((rows + 63) / 64), 64u, ga, stream);
}

// gqa_kernel (ops/suite/dev/gqa.py:20-59): non-causal GQA attention over
// [Z, H_Q, N_CTX, HEAD_DIM] queries and [Z, H_KV, N_CTX, HEAD_DIM] keys and
// values.  The kernel addresses batch z at z * H * stride_h (gqa.py:30-33),
// so each view's batch stride must be its head count times its head stride;
// query head h reads KV head h // GROUP.
int op_gqa(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc, uint32_t nsc,
           void* stream) {
  if (nviews != 4 || nsc != 18)
    return fail(G950_USAGE, "gqa: needs views (K, Out, Q, V) and 18 scalars (GROUP, HEAD_DIM, H_KV, H_Q, "
                "N_CTX, scale, 12 strides)");
  View k, o, q, v;
  if (int rc = check_view(views, 0, "K", 4, k, false)) return rc;
  if (int rc = check_view(views, 1, "Out", 4, o, true)) return rc;
  if (int rc = check_view(views, 2, "Q", 4, q, false)) return rc;
  if (int rc = check_view(views, 3, "V", 4, v, false)) return rc;
  const uint32_t dt = q.v->dtype;
  if (!is_float(dt) || k.v->dtype != dt || v.v->dtype != dt || o.v->dtype != dt)
    return fail(G950_USAGE, "gqa: Q/K/V/Out must share one float dtype");
  long long group, hd, hkv, hq, n;
  double scale;
  if (int rc = scalar_int(&sc[0], "GROUP", group)) return rc;
  if (int rc = scalar_int(&sc[1], "HEAD_DIM", hd)) return rc;
  if (int rc = scalar_int(&sc[2], "H_KV", hkv)) return rc;
  if (int rc = scalar_int(&sc[3], "H_Q", hq)) return rc;
  if (int rc = scalar_int(&sc[4], "N_CTX", n)) return rc;
  if (int rc = scalar_float(&sc[5], "scale", scale)) return rc;
  const long long Z = q.shape[0];
  if (q.shape[1] != hq || o.shape[1] != hq || k.shape[1] != hkv || v.shape[1] != hkv)
    return fail(G950_USAGE, "gqa: Q/Out need H_Q heads and K/V H_KV heads");
  for (const View* w : {&k, &o, &q, &v})
    if (w->shape[0] != Z || w->shape[2] != n || w->shape[3] != hd)
      return fail(G950_USAGE, "gqa: view %s must be [Z, heads, N_CTX, HEAD_DIM]", w->name);
  if (hq <= 0 || hkv <= 0 || group < 1 || (hq - 1) / group >= hkv)
    return fail(G950_USAGE, "gqa: GROUP must map every query head to a KV head ((H_Q - 1) // GROUP < H_KV)");
  if (hd > 1 && (q.stride[3] != 1 || k.stride[3] != 1 || v.stride[3] != 1 || o.stride[3] != 1))
    return fail(G950_USAGE, "gqa: head_dim must be contiguous");
  // stride scalars, sorted: k(h,k,n) o(h,m,n) q(h,k,m) v(h,k,n) -> view dims
  const struct { const View* vw; const char* names[3]; int dims[3]; long long heads; } st[4] = {
      {&k, {"stride_kh", "stride_kk", "stride_kn"}, {1, 3, 2}, hkv},
      {&o, {"stride_oh", "stride_om", "stride_on"}, {1, 2, 3}, hq},
      {&q, {"stride_qh", "stride_qk", "stride_qm"}, {1, 3, 2}, hq},
      {&v, {"stride_vh", "stride_vk", "stride_vn"}, {1, 2, 3}, hkv},
  };
  uint32_t si = 6;
  for (const auto& e : st) {
    for (int j = 0; j < 3; ++j)
      if (int rc = stride_agrees(sc, si++, e.names[j], *e.vw, e.dims[j])) return rc;
    if (Z > 1 && e.vw->stride[0] != e.heads * e.vw->stride[1])
      return fail(G950_USAGE, "gqa: view %s batch stride must be heads x head stride (the kernel's batch offset)",
                  e.vw->name);
  }
  if (Z * hq > 0x7FFFFFF || n > 0x7FFFFFF) return fail(G950_USAGE, "gqa: extent too large");
  AttnArgs a{};
  a.q = q.v->data; a.k = k.v->data; a.v = v.v->data; a.o = o.v->data;
  a.lse = nullptr;
  a.q_sz = q.stride[0]; a.q_sh = q.stride[1]; a.q_ss = q.stride[2];
  a.k_sz = k.stride[0]; a.k_sh = k.stride[1]; a.k_ss = k.stride[2];
  a.v_sz = v.stride[0]; a.v_sh = v.stride[1]; a.v_ss = v.stride[2];
  a.o_sz = o.stride[0]; a.o_sh = o.stride[1]; a.o_ss = o.stride[2];
  a.Z = (int)Z; a.Hq = (int)hq; a.Hkv = (int)hkv; a.Sq = (int)n; a.Sk = (int)n;
  a.scale_log2 = (float)(scale * 1.4426950408889634);
  a.causal = 0;
  a.group = (int)group;
  return launch_attention(m, a, dt, hd, q, k, v, o, stream);
}

// ------------------------------------------------------ varlen attention
// flash_varlen_fwd_kernel (ops/suite/dev/flash_varlen_fwd_kernel.py:22-320):
// 12 pointer views (all 1-D flat buffers) and the kernel's 46 non-pointer
// arguments with semantics (runtime scalars and constexprs; the tile-shape
// constexprs BLOCK_M/N/K, KERNEL_NUM_WARPS, PIPELINE_STAGES, d_rounded are
// not part of the contract), both in sorted-name order.
const char* const kVarlenScalars[] = {
    "alibi_slopes_batch_stride", "b", "bk", "block_size", "d", "h", "h_hk_ratio", "hk", "is_alibi",
    "is_causal", "is_cu_seqlens_k", "is_cu_seqlens_q", "is_dropout", "is_local", "is_paged",
    "is_seqused_k", "is_softcap", "k_batch_stride", "k_head_stride", "k_page_stride", "k_row_stride",
    "o_batch_stride", "o_head_stride", "o_row_stride", "p_dropout", "p_dropout_in_uint8_t",
    "page_table_batch_stride", "q_batch_stride", "q_head_stride", "q_row_stride", "return_softmax",
    "rp_dropout", "scale_softmax", "scale_softmax_log2", "seqlen_k", "seqlen_k_rounded", "seqlen_q",
    "seqlen_q_rounded", "seqlenq_ngroups_swapped", "softcap", "total_q", "v_batch_stride", "v_head_stride",
    "v_row_stride", "window_size_left", "window_size_right"};
constexpr uint32_t kVarlenNsc = sizeof(kVarlenScalars) / sizeof(kVarlenScalars[0]);

int varlen_index(const char* name) {
  for (uint32_t i = 0; i < kVarlenNsc; ++i)
    if (!strcmp(kVarlenScalars[i], name)) return (int)i;
  return -1;
}

// Rows a flat buffer holds for (row stride rs, heads nh at head stride hs,
// d contiguous elements): the largest R with (R-1)*rs + (nh-1)*hs + d <= n.
long long rows_held(long long n, long long rs, long long nh, long long hs, long long d) {
  const __int128 fixed = (__int128)(nh - 1) * hs + d;
  if ((__int128)n < fixed) return 0;
  return rs > 0 ? (long long)((n - fixed) / rs) + 1 : 0x7FFFFFFF;
}

int op_flash_varlen(g950_module* m, const g950_view* views, uint32_t nviews, const g950_scalar* sc,
                    uint32_t nsc, void* stream) {
  if (nviews != 12 || nsc != kVarlenNsc)
    return fail(G950_USAGE, "flash_varlen: needs 12 views (alibi_slopes_ptr .. v_ptr) and %u scalars",
                kVarlenNsc);
  View alibi, cuk, cuq, k, o, pp, pt, philox, q, used, lse, v;
  const struct { View* vw; const char* name; bool out; } vs[12] = {
      {&alibi, "alibi_slopes_ptr", false}, {&cuk, "cu_seqlens_k_ptr", false}, {&cuq, "cu_seqlens_q_ptr", false},
      {&k, "k_ptr", false}, {&o, "o_ptr", true}, {&pp, "p_ptr", false}, {&pt, "page_table_ptr", false},
      {&philox, "philox_args", false}, {&q, "q_ptr", false}, {&used, "seqused_k_ptr", false},
      {&lse, "softmax_lse_ptr", true}, {&v, "v_ptr", false}};
  for (uint32_t i = 0; i < 12; ++i)
    if (int rc = check_view(views, i, vs[i].name, 1, *vs[i].vw, vs[i].out)) return rc;
  long long val[kVarlenNsc];
  double fval[kVarlenNsc];
  for (uint32_t i = 0; i < kVarlenNsc; ++i) {
    if (int rc = scalar_float(&sc[i], kVarlenScalars[i], fval[i])) return rc;
    val[i] = (long long)fval[i];
    if (sc[i].dtype != G950_DTYPE_FLOAT32 && sc[i].dtype != G950_DTYPE_FLOAT64)
      if (int rc = scalar_int(&sc[i], kVarlenScalars[i], val[i])) return rc;
  }
  auto I = [&](const char* n) { return val[varlen_index(n)]; };
  auto F = [&](const char* n) { return fval[varlen_index(n)]; };
  for (const char* flag : {"is_softcap", "is_dropout", "return_softmax", "seqlenq_ngroups_swapped", "is_alibi"})
    if (I(flag)) return fail(G950_USAGE, "flash_varlen: %s is not supported by this build", flag);
  const uint32_t dt = q.v->dtype;
  if (!is_float(dt) || k.v->dtype != dt || v.v->dtype != dt || o.v->dtype != dt)
    return fail(G950_USAGE, "flash_varlen: q/k/v/o must share one float dtype");
  if (lse.v->dtype != G950_DTYPE_FLOAT32) return fail(G950_USAGE, "flash_varlen: softmax_lse_ptr must be float32");
  const long long B = I("b"), H = I("h"), HK = I("hk"), D = I("d"), SQ = I("seqlen_q"), SK = I("seqlen_k");
  const long long TQ = I("total_q");
  if (B < 0 || H <= 0 || HK <= 0 || D <= 0 || SQ < 0 || SK < 0 || TQ < 0 || H % HK || I("h_hk_ratio") != H / HK)
    return fail(G950_USAGE, "flash_varlen: b/h/hk/h_hk_ratio/d/seqlen/total_q inconsistent");
  if (B > 0x7FFFFFF || H * B > 0x7FFFFFF || SQ > 0x7FFFFFF || SK > 0x7FFFFFF || TQ > 0x7FFFFFFF || D > 4096)
    return fail(G950_USAGE, "flash_varlen: extent too large");
  const double scale = F("scale_softmax"), scale_log2 = F("scale_softmax_log2");
  if (!(std::fabs(scale * 1.4426950408889634 - scale_log2) <= 1e-6 * std::fabs(scale_log2) + 1e-30))
    return fail(G950_USAGE, "flash_varlen: scale_softmax_log2 must equal scale_softmax * log2(e)");
  const char* strides[] = {"q_row_stride", "k_row_stride", "v_row_stride", "o_row_stride", "q_head_stride",
                           "k_head_stride", "v_head_stride", "o_head_stride", "q_batch_stride", "k_batch_stride",
                           "v_batch_stride", "o_batch_stride", "k_page_stride", "page_table_batch_stride"};
  for (const char* n : strides)
    if (I(n) < 0) return fail(G950_USAGE, "flash_varlen: %s must be >= 0", n);
  // highest element offset + 1 of (nb batches, nr rows, nh heads, d) at the
  // named strides, in 128-bit arithmetic (the strides are caller scalars)
  auto reach = [&](long long nb, const char* bst, long long nr, const char* rst, long long nh, const char* hst,
                   long long d) {
    return (__int128)(nb - 1) * I(bst) + (__int128)(nr - 1) * I(rst) + (__int128)(nh - 1) * I(hst) + d;
  };
  const bool cu_q = I("is_cu_seqlens_q") != 0, cu_k = I("is_cu_seqlens_k") != 0;
  const bool seqused = I("is_seqused_k") != 0, paged = I("is_paged") != 0, local = I("is_local") != 0;
  const long long bs = I("block_size");
  auto int_view = [&](const View& w, const char* name, long long need) {
    if (w.v->dtype != G950_DTYPE_INT32) return fail(G950_USAGE, "flash_varlen: %s must be int32", name);
    if (w.shape[0] < need) return fail(G950_USAGE, "flash_varlen: %s needs %lld entries", name, need);
    if (w.shape[0] > 1 && w.stride[0] != 1) return fail(G950_USAGE, "flash_varlen: %s must be contiguous", name);
    return G950_OK;
  };
  if (cu_q) if (int rc = int_view(cuq, "cu_seqlens_q_ptr", B + 1)) return rc;
  if (cu_k) if (int rc = int_view(cuk, "cu_seqlens_k_ptr", B + 1)) return rc;
  if (seqused) if (int rc = int_view(used, "seqused_k_ptr", B)) return rc;
  for (const View* w : {&q, &k, &v, &o, &lse})
    if (w->shape[0] > 1 && w->stride[0] != 1) return fail(G950_USAGE, "flash_varlen: %s must be contiguous", w->name);
  // every address the kernel can form stays inside the views: rows held by
  // q/o and k/v bound the device-held lengths, the fixed-length modes are
  // checked here in full
  VarlenArgs vl{};
  const long long qe = q.shape[0], oe = o.shape[0], ke = k.shape[0], ve = v.shape[0];
  vl.q_rows = std::min(rows_held(qe, I("q_row_stride"), H, I("q_head_stride"), D),
                       rows_held(oe, I("o_row_stride"), H, I("o_head_stride"), D));
  if (!cu_q && B > 0 && SQ > 0) {
    if (reach(B, "q_batch_stride", SQ, "q_row_stride", H, "q_head_stride", D) > qe ||
        reach(B, "o_batch_stride", SQ, "o_row_stride", H, "o_head_stride", D) > oe)
      return fail(G950_USAGE, "flash_varlen: b x seqlen_q rows exceed q_ptr/o_ptr");
    if (B * SQ > TQ) return fail(G950_USAGE, "flash_varlen: b x seqlen_q exceeds total_q");
  }
  if (H * TQ > lse.shape[0]) return fail(G950_USAGE, "flash_varlen: softmax_lse_ptr needs h x total_q entries");
  if (paged) {
    if (bs <= 0) return fail(G950_USAGE, "flash_varlen: block_size must be positive");
    if (int rc = int_view(pt, "page_table_ptr", 1)) return rc;
    const long long ps = I("k_page_stride"), krs = I("k_row_stride");
    const __int128 kfix = (__int128)(bs - 1) * krs + (__int128)(HK - 1) * I("k_head_stride") + D;
    const __int128 vfix = (__int128)(bs - 1) * krs + (__int128)(HK - 1) * I("v_head_stride") + D;
    long long pages = 0;
    if (ke >= kfix && ve >= vfix)
      pages = ps > 0 ? (long long)std::min((ke - kfix) / ps, (ve - vfix) / ps) + 1 : 1;
    vl.pages = pages;
    vl.pt_elems = pt.shape[0];
    vl.pt_stride = I("page_table_batch_stride");
    vl.page_stride = ps;
    vl.block_size = (int)bs;
    vl.tile_pages = bs % 64 == 0 ? 1 : 0;
    vl.page_table = (const int*)pt.v->data;
  } else {
    vl.k_rows = std::min(rows_held(ke, I("k_row_stride"), HK, I("k_head_stride"), D),
                         rows_held(ve, I("v_row_stride"), HK, I("v_head_stride"), D));
    if (!cu_k && B > 0 && SK > 0 &&
        (reach(B, "k_batch_stride", SK, "k_row_stride", HK, "k_head_stride", D) > ke ||
         reach(B, "v_batch_stride", SK, "v_row_stride", HK, "v_head_stride", D) > ve))
      return fail(G950_USAGE, "flash_varlen: b x seqlen_k rows exceed k_ptr/v_ptr");
  }
  vl.cu_q = cu_q ? (const int*)cuq.v->data : nullptr;
  vl.cu_k = cu_k ? (const int*)cuk.v->data : nullptr;
  vl.used_k = seqused ? (const int*)used.v->data : nullptr;
  vl.q_bs = I("q_batch_stride"); vl.k_bs = I("k_batch_stride");
  vl.v_bs = I("v_batch_stride"); vl.o_bs = I("o_batch_stride");
  vl.total_q = (int)TQ;
  vl.local = local ? 1 : 0;
  vl.wl = (int)I("window_size_left");
  vl.wr = (int)I("window_size_right");
  AttnArgs a{};
  a.q = q.v->data; a.k = k.v->data; a.v = v.v->data; a.o = o.v->data;
  a.lse = (float*)lse.v->data;
  a.q_ss = I("q_row_stride"); a.q_sh = I("q_head_stride");
  a.k_ss = I("k_row_stride"); a.k_sh = I("k_head_stride");
  a.v_ss = I("v_row_stride"); a.v_sh = I("v_head_stride");
  a.o_ss = I("o_row_stride"); a.o_sh = I("o_head_stride");
  a.lse_sh = TQ; a.lse_ss = 1;
  a.Z = (int)B; a.Hq = (int)H; a.Hkv = (int)HK; a.Sq = (int)SQ; a.Sk = (int)SK;
  a.scale_log2 = (float)scale_log2;
  a.causal = I("is_causal") ? 1 : 0;
  a.group = (int)(H / HK);
  AttnVarArgs va{};
  va.a = a; va.v = vl; va.D = (int)D; va.dtype = (int)dt;
  if (B == 0 || SQ == 0) return launch(m, "g950_attn_varlen_general", 0, 64u, va, stream);
  auto m8 = [](long long x) { return x % 8 == 0; };
  const bool mfma = is_float16ish(dt) && (D == 64 || D == 128) && a.scale_log2 > 0.0f &&
                    std::isfinite(a.scale_log2) && aligned16(q.addr()) && aligned16(k.addr()) &&
                    aligned16(v.addr()) && (o.addr() & 7) == 0 && m8(a.q_ss) && m8(a.q_sh) && m8(a.k_ss) &&
                    m8(a.k_sh) && m8(a.v_ss) && m8(a.v_sh) && a.o_ss % 4 == 0 && a.o_sh % 4 == 0 &&
                    m8(vl.q_bs) && m8(vl.k_bs) && m8(vl.v_bs) && vl.o_bs % 4 == 0 && (!paged || m8(vl.page_stride));
  if (mfma) {
    // paging is compiled into the kernel: contiguous rows, pages of whole
    // 64-key tiles, or a page-table read per DMA lane
    char name[64];
    snprintf(name, sizeof name, "g950_attn_fwd_%s_d%lld_varlen%s", dt == G950_DTYPE_BFLOAT16 ? "bf16" : "f16", D,
             !paged ? "" : vl.tile_pages ? "_pt" : "_pl");
    const int threads = kernel_threads(m, name, 512);
    const int bq = threads / 2;
    va.a.nqb = (int)((SQ + bq - 1) / bq);
    const long long grid = (long long)va.a.nqb * B * H;
    if (grid > 0x7FFFFFFF) return fail(G950_USAGE, "flash_varlen: grid too large");
    return launch(m, name, (unsigned)grid, (unsigned)threads, va, stream);
  }
  const long long rows = B * H * SQ;
  if ((rows + 63) / 64 > 0x7FFFFFFF) return fail(G950_USAGE, "flash_varlen: grid too large");
  return launch(m, "g950_attn_varlen_general", (unsigned)((rows + 63) / 64), 64u, va, stream);
}

// ------------------------------------------------------------------- copy
int op_copy(g950_module* m, const g950_view* views, uint32_t nviews, uint32_t nsc, void* stream) {
  if (nviews != 2 || nsc != 0) return fail(G950_USAGE, "copy: needs views (x, y) and no scalars");
  const g950_view& x = views[0];
  const g950_view& y = views[1];
  View vx, vy;
  if (int rc = check_view(views, 0, "x", (int)x.ndim, vx, false)) return rc;
  if (int rc = check_view(views, 1, "y", (int)y.ndim, vy, true)) return rc;
  if (x.ndim != y.ndim || x.dtype != y.dtype) return fail(G950_USAGE, "copy: x and y differ in rank or dtype");
  long long n = 1, expect = vx.isz;
  for (int i = (int)x.ndim - 1; i >= 0; --i) {
    if (vx.shape[i] != vy.shape[i]) return fail(G950_USAGE, "copy: shapes differ");
    if (vx.shape[i] > 1 && (x.strides[i] != expect || y.strides[i] != expect))
      return fail(G950_USAGE, "copy: views must be contiguous");
    expect *= vx.shape[i];
    n *= vx.shape[i];
  }
  const long long bytes = n * vx.isz;
  if (bytes % 16 || !aligned16(vx.addr()) || !aligned16(vy.addr()))
    return fail(G950_USAGE, "copy: size and addresses must be multiples of 16 bytes");
  CopyArgs a{};
  a.x = x.data; a.y = y.data; a.n16 = bytes / 16;
  const long long blocks = (a.n16 + 1023) / 1024;
  const unsigned grid = (unsigned)(blocks < 4096 ? blocks : 4096);
  return launch(m, "g950_stream_copy", grid, 256u, a, stream);
}

}  // namespace

// Shared with g950_bundle.cpp (same library; not part of the C ABI).
__attribute__((visibility("hidden"))) int g950rt_fail(int code, const std::string& msg) {
  return fail(code, "%s", msg.c_str());
}

extern "C" {

int g950_open(const char* path, g950_module** out) {
  if (!path || !out) return fail(G950_USAGE, "g950_open: null argument");
  *out = nullptr;
  auto* m = new (std::nothrow) g950_module();
  if (!m) return fail(G950_RESOURCE, "g950_open: out of host memory");
  hipError_t e = hipGetDevice(&m->device);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&m->cus, hipDeviceAttributeMultiprocessorCount, m->device);
  if (e == hipSuccess) e = hipModuleLoad(&m->mod, path);
  if (e != hipSuccess) {
    delete m;
    return fail(G950_RESOURCE, "g950_open: loading %s failed: %s", path, hipGetErrorString(e));
  }
  // the no-alloc entry's scratch array on this (current) device; a failed
  // lookup only disables g950_launch_noalloc
  void* sp = nullptr;
  m->scratch_err = g950_scratch_address(m->device, &sp);
  m->scratch = (char*)sp;
  *out = m;
  return G950_OK;
}

namespace {
int dispatch(g950_module* m, uint32_t op, const g950_view* views, uint32_t nviews,
             const g950_scalar* scalars, uint32_t nscalars, void* stream) {
  t_kernel.clear();
  if ((!views && nviews) || (!scalars && nscalars)) return fail(G950_USAGE, "null argument");
  try {
    switch (op) {
      case G950_OP_SOFTMAX: return op_softmax(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_RMS_LAYERNORM: return op_rms(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_LAYERNORM: return op_layernorm(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_LOGSUMEXP: return op_logsumexp(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_MATMUL: return op_matmul(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_MATMUL_I8: return op_matmul_i8(m, views, nviews, scalars, nscalars, false, stream);
      case G950_OP_MATMUL_I8_DEQUANT:
        return op_matmul_i8(m, views, nviews, scalars, nscalars, true, stream);
      case G950_OP_ATTENTION: return op_attention(m, views, nviews, scalars, nscalars, false, stream);
      case G950_OP_ATTENTION_LSE: return op_attention(m, views, nviews, scalars, nscalars, true, stream);
      case G950_OP_COPY: return op_copy(m, views, nviews, nscalars, stream);
      case G950_OP_DEQUANTIZE: return op_dequantize(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_FLASH_VARLEN: return op_flash_varlen(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_DEQUANT_MATMUL: return op_dequant_matmul(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_SOFTMAX_INNER: return op_softmax_inner(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_LAYERNORM_ROW: return op_layernorm_row(m, views, nviews, scalars, nscalars, stream);
      case G950_OP_GQA: return op_gqa(m, views, nviews, scalars, nscalars, stream);
      default: return fail(G950_USAGE, "g950_launch: unknown operator contract %u", op);
    }
  } catch (...) {
    return fail(G950_RESOURCE, "g950_launch: internal error");
  }
}
}  // namespace

int g950_launch(g950_module* m, uint32_t op, const g950_view* views, uint32_t nviews,
                const g950_scalar* scalars, uint32_t nscalars, void* stream) {
  if (!m) return fail(G950_USAGE, "g950_launch: null module");
  return dispatch(m, op, views, nviews, scalars, nscalars, stream);
}

int g950_launch_noalloc(g950_module* m, uint32_t op, const g950_view* views, uint32_t nviews,
                        const g950_scalar* scalars, uint32_t nscalars, void* stream) {
  if (!m) return fail(G950_USAGE, "g950_launch_noalloc: null module");
  if (!m->scratch)
    return fail(G950_RESOURCE, "g950_launch_noalloc: the scratch array's address is unknown: %s",
                hipGetErrorString(m->scratch_err));
  t_scratch = m->scratch;
  const int rc = dispatch(m, op, views, nviews, scalars, nscalars, stream);
  t_scratch = nullptr;
  return rc;
}

int g950_validate(uint32_t op, const g950_view* views, uint32_t nviews, const g950_scalar* scalars,
                  uint32_t nscalars) {
  return dispatch(nullptr, op, views, nviews, scalars, nscalars, nullptr);
}

const char* g950_last_kernel(void) { return t_kernel.c_str(); }

size_t g950_workspace_bytes(g950_module* m, void* stream) {
  if (!m) return 0;
  std::lock_guard<std::mutex> lock(m->ws_mu);
  const auto it = m->ws.find(stream);
  return it == m->ws.end() ? 0 : it->second.second;
}

int g950_sync(void* stream) {
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail(G950_SYNC, "g950_sync: %s", hipGetErrorString(e));
  return G950_OK;
}

const char* g950_strerror(int code) {
  switch (code) {
    case G950_OK: return "ok";
    case G950_USAGE: return "operator contract refused";
    case G950_REJECTED: return "view rejected";
    case G950_RESOURCE: return "HIP resource or launch failure";
    case G950_REPEAT_MISMATCH: return "repeats produced different outputs";
    case G950_SYNC: return "stream synchronisation failed";
    default: return "unknown";
  }
}

const char* g950_last_error(void) { return t_error.c_str(); }

void g950_close(g950_module* m) {
  if (!m) return;
  for (auto& kv : m->ws)
    if (kv.second.first) {
      (void)hipStreamSynchronize((hipStream_t)kv.first);
      (void)hipFree(kv.second.first);
    }
  if (m->mod) (void)hipModuleUnload(m->mod);
  delete m;
}

}  // extern "C"
