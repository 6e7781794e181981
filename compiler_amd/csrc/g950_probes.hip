// Micro-probes of gfx950 issue and throughput rates behind the kernel design
// choices (LDS read bandwidth, VALU and transcendental rates, how much VALU
// work issues beside a 32x32x16 MFMA, the issue cost of 16-byte loads).
// Measurement only: no hot-path kernel is in this code object.  Every wave
// times a fixed instruction sequence with s_memtime (the shader clock) and
// stores the best of four repetitions; compiler_amd/probes.py launches the
// kernels and converts the counts.  All accesses stay inside the workgroup's
// LDS array or the caller's buffers, and every loop has a fixed trip count.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 p_bf16x8 __attribute__((ext_vector_type(8)));
typedef float p_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned p_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned p_u32x2 __attribute__((ext_vector_type(2)));

namespace g950p {

__device__ __forceinline__ uint64_t clk() {
  uint64_t t;
  asm volatile("s_memtime %0\n s_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}

enum Probe : int {
  LDS_B128 = 0,     // 64 ds_read_b128 (1 KiB each), 8 in flight
  LDS_TR_B16 = 1,   // 64 ds_read_b64_tr_b16 (512 B each), 8 in flight
  EXP = 2,          // 256 v_exp_f32 in 8 independent chains
  FMA = 3,          // 256 v_fma_f32 in 8 independent chains
  MFMA = 4,         // 64 v_mfma_f32_32x32x16_bf16, 4 accumulators
  MFMA_EXP2 = 5,    // the same, each followed by 2 independent v_exp_f32
  MFMA_FMA4 = 6,    // ... by 4 independent v_fma_f32
  MFMA_FMA8 = 7,    // ... by 8 independent v_fma_f32
  MFMA_LDS = 8,     // ... by 1 ds_read_b128, 4 reads in flight
  MFMA_MIX = 9,     // ... by one step of a software-pipelined softmax: v_fma_f32,
                    //     v_exp_f32, v_add_f32, every 2nd a v_cvt_pk_bf16_f32,
                    //     9 of 16 a v_max3_f32 (all independent of the MFMAs)
  MFMA_MIX_LDS = 10,  // both of the above
};

#define P8(I) I " %0, %0\n\t" I " %1, %1\n\t" I " %2, %2\n\t" I " %3, %3\n\t" \
              I " %4, %4\n\t" I " %5, %5\n\t" I " %6, %6\n\t" I " %7, %7"
#define F8 "v_fma_f32 %0, %0, %0, %0\n\tv_fma_f32 %1, %1, %1, %1\n\tv_fma_f32 %2, %2, %2, %2\n\t" \
           "v_fma_f32 %3, %3, %3, %3\n\tv_fma_f32 %4, %4, %4, %4\n\tv_fma_f32 %5, %5, %5, %5\n\t" \
           "v_fma_f32 %6, %6, %6, %6\n\tv_fma_f32 %7, %7, %7, %7"

template <int MODE>
__device__ __forceinline__ void rate_body(unsigned long long* out, float* sink) {
  __shared__ __attribute__((aligned(1024))) char lds[32768];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < 32768 / 4; i += blockDim.x) ((float*)lds)[i] = (float)(i & 7);
  __syncthreads();
  const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
  // conflict-free: consecutive lanes read consecutive 16 / 8 bytes
  const uint32_t a128 = base + lane * 16 + (wave & 3) * 1024;
  const uint32_t a64 = base + lane * 8 + (wave & 7) * 512;
  float x0 = lane * 1e-3f, x1 = x0 + 1e-4f, x2 = x0 + 2e-4f, x3 = x0 + 3e-4f;
  float x4 = x0 + 4e-4f, x5 = x0 + 5e-4f, x6 = x0 + 6e-4f, x7 = x0 + 7e-4f;
  p_u32x4 r[8];
  p_u32x2 q[8];
  for (int i = 0; i < 8; ++i) {
    r[i] = (p_u32x4){};
    q[i] = (p_u32x2){};
  }
  p_f32x16 acc[4];
  for (int i = 0; i < 4; ++i) acc[i] = (p_f32x16){};
  p_bf16x8 av, bv;
  for (int i = 0; i < 8; ++i) {
    av[i] = (__bf16)(lane * 0.01f);
    bv[i] = (__bf16)(i * 0.02f);
  }
  uint64_t best = ~0ull;
  for (int rep = 0; rep < 4; ++rep) {
    __syncthreads();
    const uint64_t c0 = clk();
    if constexpr (MODE == LDS_B128) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        asm volatile(
            "ds_read_b128 %0, %8 offset:0\n ds_read_b128 %1, %8 offset:4096\n"
            "ds_read_b128 %2, %8 offset:8192\n ds_read_b128 %3, %8 offset:12288\n"
            "ds_read_b128 %4, %8 offset:16384\n ds_read_b128 %5, %8 offset:20480\n"
            "ds_read_b128 %6, %8 offset:24576\n ds_read_b128 %7, %8 offset:28672\n"
            "s_waitcnt lgkmcnt(0)"
            : "=v"(r[0]), "=v"(r[1]), "=v"(r[2]), "=v"(r[3]), "=v"(r[4]), "=v"(r[5]), "=v"(r[6]), "=v"(r[7])
            : "v"(a128)
            : "memory");
        x0 += __builtin_bit_cast(float, r[i][0]);
      }
    } else if constexpr (MODE == LDS_TR_B16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %8 offset:0\n ds_read_b64_tr_b16 %1, %8 offset:4096\n"
            "ds_read_b64_tr_b16 %2, %8 offset:8192\n ds_read_b64_tr_b16 %3, %8 offset:12288\n"
            "ds_read_b64_tr_b16 %4, %8 offset:16384\n ds_read_b64_tr_b16 %5, %8 offset:20480\n"
            "ds_read_b64_tr_b16 %6, %8 offset:24576\n ds_read_b64_tr_b16 %7, %8 offset:28672\n"
            "s_waitcnt lgkmcnt(0)"
            : "=v"(q[0]), "=v"(q[1]), "=v"(q[2]), "=v"(q[3]), "=v"(q[4]), "=v"(q[5]), "=v"(q[6]), "=v"(q[7])
            : "v"(a64)
            : "memory");
        x0 += __builtin_bit_cast(float, q[i][0]);
      }
    } else if constexpr (MODE == EXP) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        asm volatile(P8("v_exp_f32")
                     : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7));
    } else if constexpr (MODE == FMA) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        asm volatile(F8 : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7));
    } else {
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc[i & 3]) : "v"(av), "v"(bv));
        if constexpr (MODE == MFMA_EXP2)
          asm volatile("v_exp_f32 %0, %0\n\tv_exp_f32 %1, %1" : "+v"(x0), "+v"(x1));
        else if constexpr (MODE == MFMA_FMA4)
          asm volatile("v_fma_f32 %0, %0, %0, %0\n\tv_fma_f32 %1, %1, %1, %1\n\tv_fma_f32 %2, %2, %2, %2\n\t"
                       "v_fma_f32 %3, %3, %3, %3"
                       : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
        else if constexpr (MODE == MFMA_FMA8)
          asm volatile(F8 : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7));
        if constexpr (MODE == MFMA_MIX || MODE == MFMA_MIX_LDS) {
          // step i: exponent argument of score i, exp of i-1, sum of i-2
          float xn, en;
          unsigned pk;
          asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(xn) : "v"(x4), "v"(x5), "v"(x6));
          asm volatile("v_exp_f32 %0, %1" : "=v"(en) : "v"(x0));
          asm volatile("v_add_f32 %0, %0, %1" : "+v"(x2) : "v"(x7));
          if (i & 1) {
            asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(pk) : "v"(x1), "v"(x7));
            x3 += __builtin_bit_cast(float, pk);
          }
          if ((i & 15) < 9) asm volatile("v_max3_f32 %0, %0, %1, %2" : "+v"(x3) : "v"(x5), "v"(x6));
          x0 = xn;
          x1 = x7;
          x7 = en;
        }
        if constexpr (MODE == MFMA_LDS || MODE == MFMA_MIX_LDS) {
          asm volatile("ds_read_b128 %0, %1 offset:0\n\ts_waitcnt lgkmcnt(4)"
                       : "+v"(r[1 + (i & 3)]) : "v"(a128) : "memory");
        }
      }
      // let the last MFMAs retire before the accumulators are read
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
      x0 += acc[0][0] + acc[1][1] + acc[2][2] + acc[3][3];
    }
    const uint64_t c1 = clk();
    if (c1 - c0 < best) best = c1 - c0;
  }
  if (lane == 0) out[blockIdx.x * 16 + wave] = best;
  const float tot = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7 +
                    __builtin_bit_cast(float, r[1][0] ^ r[2][1] ^ r[3][2] ^ r[4][3] ^ r[5][2] ^ q[6][1]);
  if (tot == 12345.0f) sink[tid] = tot;  // keeps the chains live; never true for these inputs
}

// Issue cost of 8 back-to-back 16-byte-per-lane loads (1 KiB each) from every
// wave of the workgroup at once: cycles until the 8th instruction issued, and
// until its data arrived.  Wave w of block b reads 8 KiB at (b*16 + w)*8 KiB.
enum Issue : int { ISSUE_LDS_DMA = 0, ISSUE_GLOBAL = 1 };

template <int MODE>
__device__ __forceinline__ void issue_body(const char* src, unsigned long long* out, p_u32x4* sink) {
  __shared__ __attribute__((aligned(1024))) char lds[65536];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const char* p = src + ((long long)blockIdx.x * 16 + wave) * 8 * 1024 + lane * 16;
  p_u32x4 r[8];
  __syncthreads();
  const uint64_t c0 = clk();
  if constexpr (MODE == ISSUE_LDS_DMA) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p + i * 1024),
                                       (__attribute__((address_space(3))) void*)(lds + wave * 8192 + i * 1024),
                                       16, 0, 0);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = *(const p_u32x4*)(p + i * 1024);
  }
  const uint64_t c1 = clk();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const uint64_t c2 = clk();
  if (lane == 0) {
    out[(blockIdx.x * 16 + wave) * 2] = c1 - c0;
    out[(blockIdx.x * 16 + wave) * 2 + 1] = c2 - c0;
  }
  if constexpr (MODE == ISSUE_LDS_DMA) {
    __syncthreads();
    if (((const unsigned*)lds)[tid] == 0x12345678u) sink[tid] = (p_u32x4){};
  } else {
    p_u32x4 s = r[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) s ^= r[i];
    if (s[0] == 0x12345678u) sink[tid] = s;
  }
}

// Shader clock against the 100 MHz real-time counter over a fixed loop.
__device__ __forceinline__ void clock_body(unsigned long long* out) {
  float x0 = threadIdx.x * 1e-3f, x1 = x0 + 1e-4f, x2 = x0 + 2e-4f, x3 = x0 + 3e-4f;
  float x4 = x0 + 4e-4f, x5 = x0 + 5e-4f, x6 = x0 + 6e-4f, x7 = x0 + 7e-4f;
  uint64_t r0, r1;
  asm volatile("s_memrealtime %0\n s_waitcnt lgkmcnt(0)" : "=s"(r0)::"memory");
  const uint64_t c0 = clk();
  for (int i = 0; i < 4096; ++i)
    asm volatile(P8("v_exp_f32") : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7));
  const uint64_t c1 = clk();
  asm volatile("s_memrealtime %0\n s_waitcnt lgkmcnt(0)" : "=s"(r1)::"memory");
  if (threadIdx.x == 0) {
    out[blockIdx.x * 2] = c1 - c0;
    out[blockIdx.x * 2 + 1] = r1 - r0;
  }
  if (x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7 == 12345.0f) out[0] = 0;
}

}  // namespace g950p

#define G950_RATE_PROBE(NAME, MODE)                                             \
  extern "C" __global__ __launch_bounds__(512) void NAME(unsigned long long* out, float* sink) { \
    g950p::rate_body<g950p::MODE>(out, sink);                                  \
  }
G950_RATE_PROBE(g950p_lds_b128, LDS_B128)
G950_RATE_PROBE(g950p_lds_tr_b16, LDS_TR_B16)
G950_RATE_PROBE(g950p_exp, EXP)
G950_RATE_PROBE(g950p_fma, FMA)
G950_RATE_PROBE(g950p_mfma, MFMA)
G950_RATE_PROBE(g950p_mfma_exp2, MFMA_EXP2)
G950_RATE_PROBE(g950p_mfma_fma4, MFMA_FMA4)
G950_RATE_PROBE(g950p_mfma_fma8, MFMA_FMA8)
G950_RATE_PROBE(g950p_mfma_lds, MFMA_LDS)
G950_RATE_PROBE(g950p_mfma_mix, MFMA_MIX)
G950_RATE_PROBE(g950p_mfma_mix_lds, MFMA_MIX_LDS)

extern "C" __global__ __launch_bounds__(512) void g950p_issue_lds_dma(const char* src, unsigned long long* out,
                                                                        p_u32x4* sink) {
  g950p::issue_body<g950p::ISSUE_LDS_DMA>(src, out, sink);
}
extern "C" __global__ __launch_bounds__(512) void g950p_issue_global(const char* src, unsigned long long* out,
                                                                       p_u32x4* sink) {
  g950p::issue_body<g950p::ISSUE_GLOBAL>(src, out, sink);
}
extern "C" __global__ __launch_bounds__(64) void g950p_clock(unsigned long long* out) { g950p::clock_body(out); }

// Sustained MFMA throughput by output shape, under the chip's power limit
// (timed by the host over back-to-back launches): 8 waves per workgroup,
// every MFMA taking a different pair of the wave's eight operand registers
// (random bf16 from the caller, so the datapath toggles as in a GEMM), the
// same FLOPs per iteration for both shapes -- 32 v_mfma_f32_32x32x16_bf16
// into 4 accumulators, or 64 v_mfma_f32_16x16x32_bf16 into 8.  Each thread
// stores the sum of its accumulators so none of the work is dead.
typedef float p_f32x4 __attribute__((ext_vector_type(4)));
template <bool S16>
__device__ __forceinline__ void mfma_rate_body(const p_u32x4* in, float* out, int iters) {
  const int t = threadIdx.x + blockIdx.x * 512;
  p_u32x4 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = in[(t * 16 + i) & 65535];
    b[i] = in[(t * 16 + 8 + i) & 65535];
  }
  float s = 0.0f;
  if constexpr (S16) {
    p_f32x4 acc[8] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(p_bf16x8, a[(i + j) & 7]),
                                                           __builtin_bit_cast(p_bf16x8, b[(i + 3 * j) & 7]), acc[j],
                                                           0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      for (int e = 0; e < 4; ++e) s += acc[j][e];
  } else {
    p_f32x16 acc[4] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(p_bf16x8, a[(i + j) & 7]),
                                                           __builtin_bit_cast(p_bf16x8, b[(i + 3 * j) & 7]), acc[j],
                                                           0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 16; ++e) s += acc[j][e];
  }
  out[t] = s;
}
extern "C" __global__ __launch_bounds__(512) void g950p_mfma_rate32(const p_u32x4* in, float* out, int iters) {
  mfma_rate_body<false>(in, out, iters);
}
extern "C" __global__ __launch_bounds__(512) void g950p_mfma_rate16(const p_u32x4* in, float* out, int iters) {
  mfma_rate_body<true>(in, out, iters);
}
