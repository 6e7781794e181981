// Shared device helpers for the gfx950 hot-path kernels.
//
// Storage types: fp32 is `float`, bf16 and fp16 are carried as 16-bit bit
// patterns (`uint16_t`) and converted explicitly, so every kernel sees the
// same rounding rule the reference host uses for bf16
// (ops/harness/opslib/case.py:214-220: round-to-nearest-even, NaN quieted).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "g950_args.h"

namespace g950 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// dtype codes of the a100-native-io/v1 format (a100c/runtime/a100rt.h:58-72)
enum : int { DT_INT8 = 2, DT_UINT8 = 3, DT_INT32 = 6, DT_F16 = 10, DT_BF16 = 11, DT_F32 = 12 };

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// float -> bf16 bits, round-to-nearest-even (gfx950 v_cvt_pk_bf16_f32).  For
// every non-NaN input this is the reference host rule bit for bit; a NaN stays
// a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element load/store through a runtime dtype code (used by the general,
// non-hot kernels and per-row statistics).
__device__ __forceinline__ float load_as_f32(const void* p, long long i, int dt) {
  if (dt == DT_F32) return ((const float*)p)[i];
  if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return f16_to_f32(((const uint16_t*)p)[i]);
}

__device__ __forceinline__ void store_from_f32(void* p, long long i, int dt, float v) {
  if (dt == DT_F32) ((float*)p)[i] = v;
  else if (dt == DT_BF16) ((uint16_t*)p)[i] = f32_to_bf16(v);
  else ((uint16_t*)p)[i] = f32_to_f16(v);
}

// max(a, b, c) in one v_max3_f32.  For values that may not be canonical
// (loaded bits, MFMA results) fmaxf first canonicalises each operand (one
// v_max_f32 x, x per value, its rule for possibly signalling NaNs); v_max3
// directly treats a quiet NaN as missing, as fmaxf does.  Used where NaN
// handling beyond that is not needed (attention's score maxima).
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// ---------------------------------------------------------------- DPP
// Wavefront (64-lane) reductions with DPP row operations: quad swaps, half-row
// and row mirrors, then row_bcast15 / row_bcast31 to fold the four 16-lane
// rows; lane 63 ends with the total, which is then broadcast.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float identity, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      __builtin_bit_cast(int, identity), __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

struct OpSum {
  static __device__ __forceinline__ float apply(float a, float b) { return a + b; }
  static constexpr float identity = 0.0f;
};
struct OpMax {
  static __device__ __forceinline__ float apply(float a, float b) { return fmaxf(a, b); }
  static constexpr float identity = -__builtin_huge_valf();
};

// 32-bit modular integer sum (carried through the float-typed DPP helper as bits)
struct OpSumU32 {
  static __device__ __forceinline__ float apply(float a, float b) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, a) + __builtin_bit_cast(uint32_t, b));
  }
  static constexpr float identity = 0.0f;
};

template <class Op>
__device__ __forceinline__ float wave_reduce(float v) {
  const float id = Op::identity;
  v = Op::apply(v, dpp_f32<0xB1, 0xF>(id, v));   // quad_perm [1,0,3,2]
  v = Op::apply(v, dpp_f32<0x4E, 0xF>(id, v));   // quad_perm [2,3,0,1]
  v = Op::apply(v, dpp_f32<0x141, 0xF>(id, v));  // row_half_mirror
  v = Op::apply(v, dpp_f32<0x140, 0xF>(id, v));  // row_mirror
  v = Op::apply(v, dpp_f32<0x142, 0xA>(id, v));  // row_bcast15 -> rows 1,3
  v = Op::apply(v, dpp_f32<0x143, 0xC>(id, v));  // row_bcast31 -> rows 2,3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Block reduction over BLOCK threads (BLOCK a multiple of 64); `scratch`
// holds BLOCK/64 floats.  Ends with a barrier so scratch can be reused.
template <class Op, int BLOCK>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
  v = wave_reduce<Op>(v);
  if constexpr (BLOCK == 64) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
#pragma unroll
    for (int i = 1; i < BLOCK / 64; ++i) r = Op::apply(r, scratch[i]);
    __syncthreads();
    return r;
  }
}

}  // namespace g950
