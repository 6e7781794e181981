// int8 weight dequantisation: y[k, n] = float(b[k, n]) * scale[n]
// (ops/suite/perf/dequantize_matmul.py:28-43, dequantize_kernel), the
// producer of the reference's dequantize_matmul.
//
// The product b * scale is formed in fp32 and rounded once to y's dtype.  It is
// exact in fp32 for every supported scale dtype (8 significant bits of int8
// times at most 24 of the scale, rounded once; for bf16/fp16 scales the product
// has at most 19 significant bits), so the result equals the float64 product
// rounded to y's dtype, bit for bit.
//
// HBM-bound: per element one int8 read and one y write; the scale row is tiny
// and stays in L2.  The vector kernel gives each lane one 16-byte vector of y
// (4 fp32 or 8 16-bit columns; the matching 4 or 8 int8 bytes of b) in
// DQ_ROWS consecutive rows, so a lane loads its scales once and reuses them
// DQ_ROWS times, and consecutive lanes take consecutive vectors: every load
// and store instruction of a wavefront covers one contiguous span of a row.
#include "g950_common.h"

namespace g950 {

constexpr int DQ_ROWS = 4;
constexpr int DQ_BLOCK = 256;

template <typename T> struct DqType;
template <> struct DqType<float> {
  static constexpr int COLS = 4;
  using Raw = uint32_t;  // 4 int8
  static __device__ __forceinline__ void load_scale(const void* s, long long n0, float* out) {
    const f32x4 v = *(const f32x4*)((const float*)s + n0);
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
  }
  static __device__ __forceinline__ void widen(Raw w, float* out) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = (float)(int)(int8_t)((w >> (8 * j)) & 0xFFu);
  }
  static __device__ __forceinline__ void store(void* y, long long idx, const float* v) {
    const f32x4 o = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(o, (f32x4*)((float*)y + idx));
  }
};

template <bool BF16>
struct DqType16 {
  static constexpr int COLS = 8;
  using Raw = u32x2;  // 8 int8
  static __device__ __forceinline__ float from(uint16_t v) { return BF16 ? bf16_to_f32(v) : f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t to(float v) { return BF16 ? f32_to_bf16(v) : f32_to_f16(v); }
  static __device__ __forceinline__ void load_scale(const void* s, long long n0, float* out) {
    const u32x4 v = *(const u32x4*)((const uint16_t*)s + n0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = from((uint16_t)(v[j] & 0xFFFFu));
      out[2 * j + 1] = from((uint16_t)(v[j] >> 16));
    }
  }
  static __device__ __forceinline__ void widen(Raw w, float* out) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * i + j] = (float)(int)(int8_t)((w[i] >> (8 * j)) & 0xFFu);
  }
  static __device__ __forceinline__ void store(void* y, long long idx, const float* v) {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = (uint32_t)to(v[2 * j]) | ((uint32_t)to(v[2 * j + 1]) << 16);
    __builtin_nontemporal_store(o, (u32x4*)((uint16_t*)y + idx));
  }
};
template <> struct DqType<bf16_t> : DqType16<true> {};
template <> struct DqType<f16_t> : DqType16<false> {};

// Host guarantees: unit column strides, n % COLS == 0, b rows aligned to COLS
// bytes, scale and y rows 16-byte aligned, and work < 2^31.
template <typename T>
__device__ __forceinline__ void dequant_vec_body(const DequantArgs& a) {
  using D = DqType<T>;
  constexpr int C = D::COLS;
  const uint32_t nvec = (uint32_t)(a.n / C);
  const uint32_t total = (uint32_t)a.work;
  const uint32_t step = gridDim.x * DQ_BLOCK;
  for (uint32_t t = blockIdx.x * DQ_BLOCK + threadIdx.x; t < total; t += step) {
    const uint32_t g = t / nvec;
    const uint32_t c = t - g * nvec;
    const long long row0 = (long long)g * DQ_ROWS;
    const long long n0 = (long long)c * C;
    float s[C];
    D::load_scale(a.scale, n0, s);
    typename D::Raw w[DQ_ROWS];
#pragma unroll
    for (int r = 0; r < DQ_ROWS; ++r)
      if (row0 + r < a.k)
        w[r] = __builtin_nontemporal_load(
            (const typename D::Raw*)((const int8_t*)a.b + (row0 + r) * a.b_sk + n0));
#pragma unroll
    for (int r = 0; r < DQ_ROWS; ++r) {
      if (row0 + r < a.k) {
        float v[C];
        D::widen(w[r], v);
#pragma unroll
        for (int e = 0; e < C; ++e) v[e] *= s[e];
        D::store(a.y, (row0 + r) * a.y_sk + n0, v);
      }
    }
  }
}

// Any strides and extents: one element per lane.
__device__ __forceinline__ void dequant_general_body(const DequantArgs& a) {
  const long long total = a.k * a.n;
  const long long step = (long long)gridDim.x * DQ_BLOCK;
  for (long long t = (long long)blockIdx.x * DQ_BLOCK + threadIdx.x; t < total; t += step) {
    const long long k = t / a.n;
    const long long n = t - k * a.n;
    const float b = (float)((const int8_t*)a.b)[k * a.b_sk + n * a.b_sn];
    const float s = load_as_f32(a.scale, n * a.s_sn, a.y_dtype);
    store_from_f32(a.y, k * a.y_sk + n * a.y_sn, a.y_dtype, b * s);
  }
}

}  // namespace g950

extern "C" __global__ __launch_bounds__(g950::DQ_BLOCK) void g950_dequant_i8_f32(const g950::DequantArgs a) {
  g950::dequant_vec_body<float>(a);
}
extern "C" __global__ __launch_bounds__(g950::DQ_BLOCK) void g950_dequant_i8_bf16(const g950::DequantArgs a) {
  g950::dequant_vec_body<g950::bf16_t>(a);
}
extern "C" __global__ __launch_bounds__(g950::DQ_BLOCK) void g950_dequant_i8_f16(const g950::DequantArgs a) {
  g950::dequant_vec_body<g950::f16_t>(a);
}
extern "C" __global__ __launch_bounds__(g950::DQ_BLOCK) void g950_dequant_i8_general(const g950::DequantArgs a) {
  g950::dequant_general_body(a);
}
