// g950_exec -- run one hot-path operator on an a100-native-io/v1 bundle on
// the current GPU: the command-line counterpart of the reference's
// single-operator executable `operator_exec --bundle <path> --threads <n>
// [--repeats <k>]` (a100c/runtime/main.c:50-177).
//
//   g950_exec --bundle <bundle.bin | dir> --op <operator> [--repeats <k>]
//             [--module <g950.hsaco>] [--write] [--compare <rtol> <atol>]
//
// The operator is named by its reference kernel (softmax_kernel, matmul_kernel,
// attention_forward_kernel, ...) or contract (softmax, matmul, ...); the
// reference executable has it compiled in.  Flow as in the reference: validate
// the bundle before anything runs (rejection -> one status line, exit 3), run
// the operator --repeats times, each an independent execution of the same
// case, and require identical outputs from every repeat (exit 5 otherwise).
// --write maps the file shared so the outputs land in it (the reference's
// behaviour); by default the file is left unchanged.  --compare checks the
// outputs against the output values the bundle already holds (a post-run
// bundle of the reference) with the corpus rule |a - b| <= atol + rtol*|b|
// (ops/harness/opslib/compare.py:107-140; NaN equals NaN), exit 7 on failure.
//
// One JSON status line on stdout.  Exit codes: 0 ok, 2 usage / operator
// contract refused, 3 bundle rejected, 4 HIP resource, 5 repeat mismatch,
// 6 sync failure (a100c/runtime/a100rt.h:50-55), 7 comparison failed.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "../../include/g950rt.h"

namespace {

struct OpName {
  const char* name;
  uint32_t op;
  int causal;  // -1: no leading CAUSAL scalar; else its value
};

const OpName kOps[] = {
    {"softmax_kernel", G950_OP_SOFTMAX, -1},
    {"softmax", G950_OP_SOFTMAX, -1},
    {"logsumexp_kernel", G950_OP_LOGSUMEXP, -1},
    {"logsumexp", G950_OP_LOGSUMEXP, -1},
    {"rms_layernorm_forward_kernel", G950_OP_RMS_LAYERNORM, -1},
    {"rms_layernorm", G950_OP_RMS_LAYERNORM, -1},
    {"layernorm_kernel", G950_OP_LAYERNORM, -1},
    {"layernorm", G950_OP_LAYERNORM, -1},
    {"matmul_kernel", G950_OP_MATMUL, -1},
    {"matmul", G950_OP_MATMUL, -1},
    {"matmul_i8", G950_OP_MATMUL_I8, -1},
    {"matmul_i8_dequant", G950_OP_MATMUL_I8_DEQUANT, -1},
    {"dequantize_kernel", G950_OP_DEQUANTIZE, -1},
    {"dequantize", G950_OP_DEQUANTIZE, -1},
    // attention's CAUSAL is a constexpr of the reference kernels, not in the image
    {"attention_forward_kernel", G950_OP_ATTENTION, 0},
    {"attn_fwd_causal_kernel", G950_OP_ATTENTION, 1},
    {"attention", G950_OP_ATTENTION, -1},
    {"attention_lse", G950_OP_ATTENTION_LSE, -1},
};

int usage() {
  fprintf(stderr,
          "usage: g950_exec --bundle <bundle.bin|dir> --op <operator> [--repeats <k>]\n"
          "                 [--module <g950.hsaco>] [--write] [--compare <rtol> <atol>]\n"
          "  operators:");
  for (const auto& o : kOps) fprintf(stderr, " %s", o.name);
  fprintf(stderr, "\n");
  return G950_USAGE;
}

void json_str(const char* s) {
  putchar('"');
  for (; *s; ++s) {
    if (*s == '"' || *s == '\\') putchar('\\');
    if ((unsigned char)*s < 0x20) printf("\\u%04x", (unsigned char)*s);
    else putchar(*s);
  }
  putchar('"');
}

void status_line(const char* status, const char* detail) {
  printf("{\"runtime\":\"g950rt/v1\",\"status\":\"%s\"", status);
  if (detail) {
    printf(",\"reason\":");
    json_str(detail);
  }
  printf("}\n");
}

double f16_value(uint16_t h) {
  const int e = (h >> 10) & 0x1F, m = h & 0x3FF;
  const double sgn = (h & 0x8000) ? -1.0 : 1.0;
  if (e == 0) return sgn * std::ldexp((double)m, -24);
  if (e == 31) return m ? NAN : sgn * INFINITY;
  return sgn * std::ldexp((double)(m | 0x400), e - 25);
}

// One element of a host view as a double (exact for every supported dtype
// except 64-bit integers beyond 2^53, which no hot-path output uses).
double element(const g950_view& v, int64_t byte_off) {
  const unsigned char* p = (const unsigned char*)v.data + byte_off;
  switch (v.dtype) {
    case G950_DTYPE_BOOL: case G950_DTYPE_UINT8: return *p;
    case G950_DTYPE_INT8: return (int8_t)*p;
    case G950_DTYPE_INT16: { int16_t x; memcpy(&x, p, 2); return x; }
    case G950_DTYPE_UINT16: { uint16_t x; memcpy(&x, p, 2); return x; }
    case G950_DTYPE_INT32: { int32_t x; memcpy(&x, p, 4); return x; }
    case G950_DTYPE_UINT32: { uint32_t x; memcpy(&x, p, 4); return x; }
    case G950_DTYPE_INT64: { int64_t x; memcpy(&x, p, 8); return (double)x; }
    case G950_DTYPE_UINT64: { uint64_t x; memcpy(&x, p, 8); return (double)x; }
    case G950_DTYPE_FLOAT16: { uint16_t x; memcpy(&x, p, 2); return f16_value(x); }
    case G950_DTYPE_BFLOAT16: {
      uint16_t x; memcpy(&x, p, 2);
      const uint32_t w = (uint32_t)x << 16;
      float f; memcpy(&f, &w, 4);
      return f;
    }
    case G950_DTYPE_FLOAT32: { float x; memcpy(&x, p, 4); return x; }
    case G950_DTYPE_FLOAT64: { double x; memcpy(&x, p, 8); return x; }
    default: return NAN;
  }
}

// Every element's byte offset of a view, in row-major index order.
std::vector<int64_t> offsets(const g950_view& v) {
  std::vector<int64_t> out;
  int64_t n = 1;
  for (uint32_t a = 0; a < v.ndim; ++a) n *= v.shape[a];
  if (n <= 0) return out;
  out.reserve((size_t)n);
  std::vector<int64_t> idx(v.ndim, 0);
  for (int64_t k = 0; k < n; ++k) {
    int64_t off = 0;
    for (uint32_t a = 0; a < v.ndim; ++a) off += idx[a] * v.strides[a];
    out.push_back(off);
    for (int a = (int)v.ndim - 1; a >= 0; --a) {
      if (++idx[a] < v.shape[a]) break;
      idx[a] = 0;
    }
  }
  return out;
}

}  // namespace

int main(int argc, char** argv) {
  std::string bundle_path, op_name, module_path;
  uint32_t repeats = 1;
  bool write = false, compare = false;
  double rtol = 0, atol = 0;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--bundle" && i + 1 < argc && bundle_path.empty()) bundle_path = argv[++i];
    else if (a == "--op" && i + 1 < argc && op_name.empty()) op_name = argv[++i];
    else if (a == "--module" && i + 1 < argc) module_path = argv[++i];
    else if (a == "--write") write = true;
    else if (a == "--repeats" && i + 1 < argc) {
      char* end = nullptr;
      const unsigned long r = strtoul(argv[++i], &end, 10);
      if (!end || *end || r < 1 || r > 0xFFFFFFFFul) return usage();
      repeats = (uint32_t)r;
    } else if (a == "--compare" && i + 2 < argc) {
      char *e1 = nullptr, *e2 = nullptr;
      rtol = strtod(argv[++i], &e1);
      atol = strtod(argv[++i], &e2);
      if (!e1 || *e1 || !e2 || *e2 || rtol < 0 || atol < 0) return usage();
      compare = true;
    } else {
      return usage();
    }
  }
  if (bundle_path.empty() || op_name.empty()) return usage();
  const OpName* op = nullptr;
  for (const auto& o : kOps)
    if (op_name == o.name) op = &o;
  if (!op) return usage();
  struct stat sb;
  if (stat(bundle_path.c_str(), &sb) == 0 && S_ISDIR(sb.st_mode)) bundle_path += "/bundle.bin";
  if (stat(bundle_path.c_str(), &sb) != 0) sb.st_size = 0;
  if (module_path.empty()) {
    // default: the code object next to this program (compiler_amd/lib/)
    std::string self = argv[0];
    const size_t slash = self.rfind('/');
    module_path = (slash == std::string::npos ? std::string(".") : self.substr(0, slash)) + "/g950.hsaco";
  }

  g950_bundle* b = nullptr;
  int reason = 0;
  if (g950_bundle_open(bundle_path.c_str(), write ? G950_BUNDLE_WRITE_BACK : 0, &b, &reason)) {
    status_line("rejected", reason ? g950_bundle_reason(reason) : g950_last_error());
    return G950_REJECTED;
  }
  const uint32_t nviews = g950_bundle_count(b, 1);
  std::vector<g950_view> views(nviews);
  for (uint32_t i = 0; i < nviews; ++i) g950_bundle_view(b, i, &views[i]);

  // the outputs the image already holds (expected values of a post-run bundle)
  std::vector<std::vector<double>> expected(nviews);
  if (compare)
    for (uint32_t i = 0; i < nviews; ++i)
      if (views[i].flags & G950_VIEW_OUTPUT)
        for (int64_t off : offsets(views[i])) expected[i].push_back(element(views[i], off));

  g950_module* m = nullptr;
  if (int rc = g950_open(module_path.c_str(), &m)) {
    status_line("resource", g950_last_error());
    g950_bundle_close(b);
    return rc;
  }
  g950_scalar lead{G950_DTYPE_INT32, 4, (uint64_t)(op->causal > 0 ? 1 : 0)};
  int equal = 1;
  int rc = g950_bundle_exec(m, b, op->op, op->causal >= 0 ? &lead : nullptr, op->causal >= 0 ? 1u : 0u,
                            repeats, nullptr, &equal);
  const std::string kernel = g950_last_kernel();
  g950_close(m);
  if (rc) {
    const char* st = rc == G950_USAGE ? "refused" : rc == G950_REJECTED ? "rejected"
                     : rc == G950_SYNC ? "sync-failed" : "resource";
    status_line(st, g950_last_error());
    g950_bundle_close(b);
    return rc;
  }

  // comparison against the held outputs
  bool pass = true;
  std::string cmp;
  if (compare) {
    cmp = ",\"comparison\":{\"max_abs_error\":{";
    bool first = true;
    for (uint32_t i = 0; i < nviews; ++i) {
      if (!(views[i].flags & G950_VIEW_OUTPUT)) continue;
      double worst = 0.0;
      size_t k = 0;
      for (int64_t off : offsets(views[i])) {
        const double a = element(views[i], off), e = expected[i][k++];
        if (std::isnan(a) || std::isnan(e)) {
          if (!(std::isnan(a) && std::isnan(e))) pass = false, worst = INFINITY;
          continue;
        }
        if (a == e) continue;  // equal entries (also equal infinities) carry no error
        const double d = std::fabs(a - e);
        if (!(d <= atol + rtol * std::fabs(e))) pass = false;
        if (d > worst || std::isnan(d)) worst = d;
      }
      char buf[64];
      snprintf(buf, sizeof buf, "%s\"view%u\":%.9g", first ? "" : ",", i, worst);
      cmp += buf;
      first = false;
    }
    cmp += std::string("},\"status\":\"") + (pass ? "PASS" : "FAIL") + "\"}";
  }
  const int close_rc = g950_bundle_close(b);
  const char* status = close_rc ? "sync-failed" : (equal ? (pass ? "ok" : "mismatch") : "repeat-mismatch");
  printf("{\"runtime\":\"g950rt/v1\",\"status\":\"%s\",\"op\":", status);
  json_str(op->name);
  printf(",\"kernel\":");
  json_str(kernel.c_str());
  printf(",\"repeats\":%u,\"repeats_all_equal\":%s,\"written\":%s,\"bundle_bytes\":%lld%s}\n", repeats,
         equal ? "true" : "false", write ? "true" : "false", (long long)sb.st_size, cmp.c_str());
  if (close_rc) return G950_SYNC;
  if (!equal) return G950_REPEAT_MISMATCH;
  if (!pass) return 7;
  return G950_OK;
}
