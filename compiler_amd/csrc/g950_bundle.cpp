// a100-native-io/v1 bundles on the GPU: validation, device staging and the
// repeat loop of the reference's single-operator executable.
//
// Format semantics follow the reference reader (a100c/runtime/bundle.c:10-19,
// 111-339): the whole image is validated before anything is used, in the same
// order and with the same rejection reasons, so a corrupted bundle is refused
// with the reason the reference would give.  Execution follows
// a100c/runtime/main.c:96-150 -- every repeat is an independent run of the
// same case (all storages restored from the image first) and the outputs of
// every repeat must equal the first's byte for byte -- with the storages
// staged into device memory: each storage becomes one device allocation, a
// view keeps its byte offset inside it (storages are 64-byte aligned in the
// file, so a view's alignment is preserved), and pointer tables
// (relocations) are patched with DEVICE addresses in the staged copy only.
// The mapped image changes only where outputs are written back after the
// last repeat; with G950_BUNDLE_WRITE_BACK the mapping is shared and closing
// syncs it to the file, otherwise it is a private copy and the file is never
// modified.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "../../include/g950rt.h"

// g950rt.cpp: records the message g950_last_error() returns
__attribute__((visibility("hidden"))) int g950rt_fail(int code, const std::string& msg);

struct g950_bundle {
  int fd = -1;
  uint32_t flags = 0;
  unsigned char* map = nullptr;
  uint64_t size = 0;
  uint32_t nstorage = 0, nviews = 0, nscalars = 0, nrelocations = 0;
  std::vector<uint64_t> st_off, st_size;
  struct ViewRec {
    uint32_t storage, dtype, ndim, flags;
    int64_t offset;
    std::vector<int64_t> shape, strides;
  };
  std::vector<ViewRec> views;
  std::vector<g950_scalar> scalars;
  struct Reloc {
    uint32_t table, target;
    uint64_t entry;
    int64_t offset;
  };
  std::vector<Reloc> relocs;
};

namespace {

const char* const kReasons[] = {
    "",           "open",          "size",           "magic",          "version",
    "reserved",   "map",           "storage-bounds", "count-bounds",   "alloc",
    "view-truncated", "view-storage", "view-dtype",  "view-offset",    "view-dim",
    "view-reach", "view-flags",    "scalar-truncated", "scalar-width", "reloc-truncated",
    "reloc-view", "reloc-table-width", "reloc-table-output", "reloc-entry", "reloc-offset",
    "storage-overlaps-metadata"};

int itemsize(uint32_t dt) {
  static const int sizes[] = {0, 1, 1, 1, 2, 2, 4, 4, 8, 8, 2, 2, 4, 8};
  return dt < sizeof(sizes) / sizeof(sizes[0]) ? sizes[dt] : 0;
}

bool within(uint64_t n, uint64_t off, uint64_t len) { return off <= n && len <= n - off; }

uint32_t u32(const unsigned char* p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}
uint64_t u64(const unsigned char* p) {
  uint64_t v;
  memcpy(&v, p, 8);
  return v;
}

// Validate an image and decode its records into `b` (which may be a scratch
// object).  Returns 0 or the G950_R_* reason.  Check order is the reference
// reader's, so the first violated rule is the one reported.
int decode(const unsigned char* p, uint64_t size, g950_bundle& b) {
  if (size < 32) return G950_R_SIZE;
  if (memcmp(p, "A100IO01", 8) != 0) return G950_R_MAGIC;
  if (u32(p + 8) != 1) return G950_R_VERSION;
  if (u32(p + 28) != 0) return G950_R_RESERVED;
  b.nstorage = u32(p + 12);
  b.nviews = u32(p + 16);
  b.nscalars = u32(p + 20);
  b.nrelocations = u32(p + 24);
  if (!within(size, 32, (uint64_t)b.nstorage * 16)) return G950_R_STORAGE_BOUNDS;
  const unsigned char* st = p + 32;
  for (uint32_t i = 0; i < b.nstorage; ++i)
    if (!within(size, u64(st + 16 * i), u64(st + 16 * i + 8))) return G950_R_STORAGE_BOUNDS;
  if ((uint64_t)b.nviews > size / 24 || (uint64_t)b.nscalars > size / 16 ||
      (uint64_t)b.nrelocations > size / 24)
    return G950_R_COUNT_BOUNDS;
  b.st_off.resize(b.nstorage);
  b.st_size.resize(b.nstorage);
  for (uint32_t i = 0; i < b.nstorage; ++i) {
    b.st_off[i] = u64(st + 16 * i);
    b.st_size[i] = u64(st + 16 * i + 8);
  }

  uint64_t cur = 32 + (uint64_t)b.nstorage * 16;
  b.views.assign(b.nviews, {});
  for (uint32_t i = 0; i < b.nviews; ++i) {
    if (!within(size, cur, 24)) return G950_R_VIEW_TRUNCATED;
    const unsigned char* v = p + cur;
    auto& r = b.views[i];
    r.storage = u32(v);
    r.dtype = u32(v + 4);
    r.ndim = u32(v + 8);
    r.flags = u32(v + 12);
    r.offset = (int64_t)u64(v + 16);
    if (r.storage >= b.nstorage) return G950_R_VIEW_STORAGE;
    if (!itemsize(r.dtype)) return G950_R_VIEW_DTYPE;
    if (r.flags & ~G950_VIEW_OUTPUT) return G950_R_VIEW_FLAGS;
    if (!within(size, cur + 24, (uint64_t)r.ndim * 16)) return G950_R_VIEW_TRUNCATED;
    const uint64_t ssize = b.st_size[r.storage];
    if (r.offset < 0 || (uint64_t)r.offset > ssize) return G950_R_VIEW_OFFSET;
    r.shape.resize(r.ndim);
    r.strides.resize(r.ndim);
    __int128 lo = r.offset, hi = r.offset;
    bool empty = false;
    for (uint32_t a = 0; a < r.ndim; ++a) {
      r.shape[a] = (int64_t)u64(v + 24 + 8 * (uint64_t)a);
      r.strides[a] = (int64_t)u64(v + 24 + 8 * (uint64_t)r.ndim + 8 * (uint64_t)a);
      if (r.shape[a] < 0) return G950_R_VIEW_DIM;
      if (r.shape[a] == 0) empty = true;
      const __int128 ext = (__int128)(r.shape[a] ? r.shape[a] - 1 : 0) * r.strides[a];
      if (ext < 0) lo += ext;
      else hi += ext;
    }
    if (!empty && (lo < 0 || hi + itemsize(r.dtype) > (__int128)ssize)) return G950_R_VIEW_REACH;
    cur += 24 + (uint64_t)r.ndim * 16;
  }

  if (!within(size, cur, (uint64_t)b.nscalars * 16)) return G950_R_SCALAR_TRUNCATED;
  b.scalars.resize(b.nscalars);
  for (uint32_t i = 0; i < b.nscalars; ++i) {
    memcpy(&b.scalars[i], p + cur + 16 * (uint64_t)i, 16);
    const int w = itemsize(b.scalars[i].dtype);
    if (!w || (uint32_t)w != b.scalars[i].size) return G950_R_SCALAR_WIDTH;
  }
  cur += (uint64_t)b.nscalars * 16;

  if (!within(size, cur, (uint64_t)b.nrelocations * 24)) return G950_R_RELOC_TRUNCATED;
  const uint64_t meta_end = cur + (uint64_t)b.nrelocations * 24;
  for (uint32_t i = 0; i < b.nstorage; ++i)
    if (b.st_off[i] < meta_end) return G950_R_STORAGE_OVERLAPS_METADATA;
  b.relocs.resize(b.nrelocations);
  for (uint32_t i = 0; i < b.nrelocations; ++i) {
    const unsigned char* r = p + cur + 24 * (uint64_t)i;
    auto& rec = b.relocs[i];
    rec.table = u32(r);
    rec.target = u32(r + 4);
    rec.entry = u64(r + 8);
    rec.offset = (int64_t)u64(r + 16);
    if (rec.table >= b.nviews || rec.target >= b.nviews) return G950_R_RELOC_VIEW;
    const auto& t = b.views[rec.table];
    const auto& d = b.views[rec.target];
    if (t.dtype != G950_DTYPE_INT64 && t.dtype != G950_DTYPE_UINT64) return G950_R_RELOC_TABLE_WIDTH;
    if (t.flags & G950_VIEW_OUTPUT) return G950_R_RELOC_TABLE_OUTPUT;
    // the slot must lie inside the table's storage (computed without wrap-around)
    if (rec.entry > UINT64_MAX / 8 ||
        (unsigned __int128)t.offset + (unsigned __int128)rec.entry * 8 + 8 > b.st_size[t.storage])
      return G950_R_RELOC_ENTRY;
    if (rec.offset < 0 || (uint64_t)rec.offset > b.st_size[d.storage] - (uint64_t)d.offset)
      return G950_R_RELOC_OFFSET;
  }
  return 0;
}

int reject(int reason, int* out) {
  if (out) *out = reason;
  return g950rt_fail(G950_REJECTED, std::string("bundle rejected: ") + kReasons[reason]);
}

struct DeviceStage {
  std::vector<void*> mem;
  ~DeviceStage() {
    for (void* p : mem)
      if (p) (void)hipFree(p);
  }
};

int hip_fail(const char* what, hipError_t e) {
  return g950rt_fail(G950_RESOURCE, std::string("bundle exec: ") + what + ": " + hipGetErrorString(e));
}

}  // namespace

extern "C" {

const char* g950_bundle_reason(int reason) {
  if (reason <= 0 || reason > G950_R_STORAGE_OVERLAPS_METADATA) return "unknown";
  return kReasons[reason];
}

int g950_bundle_check(const void* image, uint64_t size, int* reason) {
  if (reason) *reason = 0;
  if (!image && size) return g950rt_fail(G950_USAGE, "g950_bundle_check: null image");
  g950_bundle scratch;
  const int r = decode((const unsigned char*)image, size, scratch);
  return r ? reject(r, reason) : G950_OK;
}

int g950_bundle_open(const char* path, uint32_t flags, g950_bundle** out, int* reason) {
  if (reason) *reason = 0;
  if (!path || !out) return g950rt_fail(G950_USAGE, "g950_bundle_open: null argument");
  *out = nullptr;
  if (flags & ~G950_BUNDLE_WRITE_BACK) return g950rt_fail(G950_USAGE, "g950_bundle_open: unknown flags");
  auto* b = new (std::nothrow) g950_bundle();
  if (!b) return reject(G950_R_ALLOC, reason);
  b->flags = flags;
  const bool shared = flags & G950_BUNDLE_WRITE_BACK;
  struct stat sb;
  b->fd = open(path, shared ? O_RDWR : O_RDONLY);
  if (b->fd < 0 || fstat(b->fd, &sb) != 0) {
    if (b->fd >= 0) close(b->fd);
    delete b;
    return reject(G950_R_OPEN, reason);
  }
  int r = 0;
  if (sb.st_size < 32) {
    r = G950_R_SIZE;
  } else {
    b->size = (uint64_t)sb.st_size;
    void* m = mmap(nullptr, (size_t)b->size, PROT_READ | PROT_WRITE, shared ? MAP_SHARED : MAP_PRIVATE, b->fd, 0);
    if (m == MAP_FAILED) r = G950_R_MAP;
    else b->map = (unsigned char*)m;
  }
  if (!r) r = decode(b->map, b->size, *b);
  if (r) {
    g950_bundle_close(b);
    return reject(r, reason);
  }
  *out = b;
  return G950_OK;
}

uint32_t g950_bundle_count(const g950_bundle* b, int what) {
  if (!b) return 0;
  switch (what) {
    case 0: return b->nstorage;
    case 1: return b->nviews;
    case 2: return b->nscalars;
    case 3: return b->nrelocations;
    default: return 0;
  }
}

int g950_bundle_view(const g950_bundle* b, uint32_t i, g950_view* out) {
  if (!b || !out || i >= b->nviews) return g950rt_fail(G950_USAGE, "g950_bundle_view: bad index");
  const auto& r = b->views[i];
  unsigned char* base = b->map + b->st_off[r.storage];
  out->data = base + r.offset;
  out->shape = r.shape.data();
  out->strides = r.strides.data();
  out->storage_size = b->st_size[r.storage];
  out->dtype = r.dtype;
  out->ndim = r.ndim;
  out->flags = r.flags;
  out->reserved_ = 0;
  out->storage = base;
  return G950_OK;
}

int g950_bundle_scalar(const g950_bundle* b, uint32_t i, g950_scalar* out) {
  if (!b || !out || i >= b->nscalars) return g950rt_fail(G950_USAGE, "g950_bundle_scalar: bad index");
  *out = b->scalars[i];
  return G950_OK;
}

int g950_bundle_exec(g950_module* m, g950_bundle* b, uint32_t op, const g950_scalar* lead, uint32_t nlead,
                     uint32_t repeats, void* stream, int* repeats_equal) {
  if (!m || !b || repeats < 1 || (nlead && !lead))
    return g950rt_fail(G950_USAGE, "g950_bundle_exec: null module/bundle, or repeats < 1");
  if (repeats_equal) *repeats_equal = 1;
  const hipStream_t s = (hipStream_t)stream;

  // host images of every storage, pointer tables patched with device addresses
  DeviceStage dev;
  dev.mem.assign(b->nstorage, nullptr);
  for (uint32_t i = 0; i < b->nstorage; ++i) {
    const size_t bytes = (size_t)((b->st_size[i] + 255) & ~(uint64_t)255);
    if (hipError_t e = hipMalloc(&dev.mem[i], bytes ? bytes : 256)) return hip_fail("hipMalloc", e);
  }
  std::vector<std::vector<unsigned char>> patched(b->nstorage);
  for (const auto& r : b->relocs) {
    const auto& t = b->views[r.table];
    const auto& d = b->views[r.target];
    auto& img = patched[t.storage];
    if (img.empty()) img.assign(b->map + b->st_off[t.storage], b->map + b->st_off[t.storage] + b->st_size[t.storage]);
    const uint64_t ptr = (uint64_t)(uintptr_t)((unsigned char*)dev.mem[d.storage] + d.offset + r.offset);
    memcpy(img.data() + t.offset + r.entry * 8, &ptr, 8);
  }
  auto upload = [&]() -> int {
    for (uint32_t i = 0; i < b->nstorage; ++i) {
      if (!b->st_size[i]) continue;
      const void* src = patched[i].empty() ? (const void*)(b->map + b->st_off[i]) : (const void*)patched[i].data();
      if (hipError_t e = hipMemcpyAsync(dev.mem[i], src, b->st_size[i], hipMemcpyHostToDevice, s))
        return hip_fail("upload", e);
    }
    return G950_OK;
  };

  std::vector<g950_view> views(b->nviews);
  std::vector<bool> out_storage(b->nstorage, false);
  for (uint32_t i = 0; i < b->nviews; ++i) {
    const auto& r = b->views[i];
    g950_view& v = views[i];
    v.storage = dev.mem[r.storage];
    v.data = (unsigned char*)dev.mem[r.storage] + r.offset;
    v.shape = r.shape.data();
    v.strides = r.strides.data();
    v.storage_size = b->st_size[r.storage];
    v.dtype = r.dtype;
    v.ndim = r.ndim;
    v.flags = r.flags;
    v.reserved_ = 0;
    if (r.flags & G950_VIEW_OUTPUT) out_storage[r.storage] = true;
  }
  std::vector<g950_scalar> scalars(lead, lead + nlead);
  scalars.insert(scalars.end(), b->scalars.begin(), b->scalars.end());

  std::vector<std::vector<unsigned char>> first(b->nstorage), now(b->nstorage);
  for (uint32_t rep = 0; rep < repeats; ++rep) {
    if (int rc = upload()) return rc;
    int rc = g950_launch(m, op, views.data(), (uint32_t)views.size(), scalars.data(), (uint32_t)scalars.size(), stream);
    if (rc) return rc;  // g950_last_error() already holds the launcher's message
    auto& dst = rep ? now : first;
    for (uint32_t i = 0; i < b->nstorage; ++i) {
      if (!out_storage[i] || !b->st_size[i]) continue;
      dst[i].resize(b->st_size[i]);
      if (hipError_t e = hipMemcpyAsync(dst[i].data(), dev.mem[i], b->st_size[i], hipMemcpyDeviceToHost, s))
        return hip_fail("download", e);
    }
    if (hipError_t e = hipStreamSynchronize(s))
      return g950rt_fail(G950_SYNC, std::string("bundle exec: ") + hipGetErrorString(e));
    if (rep && repeats_equal)
      for (uint32_t i = 0; i < b->nstorage; ++i)
        if (out_storage[i] && now[i] != first[i]) *repeats_equal = 0;
  }
  for (uint32_t i = 0; i < b->nstorage; ++i)
    if (out_storage[i] && b->st_size[i]) memcpy(b->map + b->st_off[i], first[i].data(), b->st_size[i]);
  return G950_OK;
}

int g950_bundle_close(g950_bundle* b) {
  if (!b) return G950_OK;
  int rc = G950_OK;
  if (b->map) {
    if ((b->flags & G950_BUNDLE_WRITE_BACK) && msync(b->map, (size_t)b->size, MS_SYNC) != 0)
      rc = g950rt_fail(G950_SYNC, "g950_bundle_close: msync failed");
    munmap(b->map, (size_t)b->size);
  }
  if (b->fd >= 0) close(b->fd);
  delete b;
  return rc;
}

}  // extern "C"
