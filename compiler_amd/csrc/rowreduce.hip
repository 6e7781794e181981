// Row-reduction family on gfx950: softmax, logsumexp, RMSNorm, LayerNorm.
//
// Operator semantics (reference, per row of the last axis):
//   softmax   ops/suite/perf/softmax.py:21-32 (masked tail reads -inf,
//             contributes exp(-inf)=0)
//   logsumexp ops/suite/perf/logsumexp.py:16-38 (NaN-ignoring max plus a NaN
//             flag; an infinite max is the result)
//   RMSNorm   ops/suite/perf/fast_rms_layernorm.py:20-42:
//             inv = 1/sqrt(sum(x^2)/n + eps); r[row] = inv; Y = (x*inv)*w
//   LayerNorm ops/suite/dev/fused_layernorm_triton.py:27-42: mean; centered
//             variance; rstd = 1/sqrt(var+eps); Y = (x-mean)*rstd*w + b
//   LayerNorm row form ops/suite/dev/layer_norm_forward_row.py:11-36:
//             mean = sum(x)/n, rstd = 1/sqrt(sum(x^2)/n - mean^2 + eps)
//             (one pass, both sums together); x_hat = (x-mean)*rstd rounded
//             to X's dtype, then Y = x_hat*W + B in X's dtype (16-bit types
//             round the product and the sum, as the reference's typed ops do)
// All arithmetic is fp32; 16-bit inputs widen exactly and outputs round once.
//
// Two kernel shapes:
//   rr_regs  -- the row lives in registers.  Each thread owns ITEMS vectors of
//               VEC elements (VEC*sizeof(T) = 16 B => one 128-bit nontemporal
//               load each) of a row handled by one BLOCK-thread workgroup.
//               Workgroups are persistent: the launcher sizes the grid to the
//               resident capacity (balanced so every workgroup gets the same
//               number of rows), each workgroup walks rows g, g+G, ..., and the
//               next row's loads are in flight while the current row is
//               reduced.  The tail of a non-power-of-two row is a per-vector
//               predicate; x is read from HBM once and y written once.
//   rs       -- rows longer than the register budget, or too few rows to
//               fill the chip: each row is cut into register-resident chunks,
//               one workgroup per chunk, partial statistics go through a small
//               workspace and a second launch merges them and writes y.
#include "g950_common.h"

#include <type_traits>

namespace g950 {

enum RowOp : int { ROW_SOFTMAX = 0, ROW_RMSNORM = 1, ROW_LAYERNORM = 2, ROW_LOGSUMEXP = 3, ROW_LNROW = 4 };

// ops with per-column weight (and bias) rows
constexpr bool row_has_w(int op) { return op == ROW_RMSNORM || op == ROW_LAYERNORM || op == ROW_LNROW; }
constexpr bool row_has_b(int op) { return op == ROW_LAYERNORM || op == ROW_LNROW; }



template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int VEC = 4;
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
};
template <> struct Elem<bf16_t> {
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f32(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f32(float v) { return f32_to_bf16(v); }
};
template <> struct Elem<f16_t> {
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f32(uint16_t v) { return f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f32(float v) { return f32_to_f16(v); }
};

// Load VEC elements (VEC>1: one aligned 16-byte load) widened to fp32.
template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const void* base, long long idx, float* out) {
  if constexpr (sizeof(T) == 4) {
    if constexpr (VEC == 4) {
      f32x4 v = __builtin_nontemporal_load((const f32x4*)((const float*)base + idx));
      out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
    } else {
      out[0] = ((const float*)base)[idx];
    }
  } else {
    if constexpr (VEC == 8) {
      u32x4 v = __builtin_nontemporal_load((const u32x4*)((const uint16_t*)base + idx));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[2 * i] = Elem<T>::to_f32((uint16_t)(v[i] & 0xFFFFu));
        out[2 * i + 1] = Elem<T>::to_f32((uint16_t)(v[i] >> 16));
      }
    } else {
      out[0] = Elem<T>::to_f32(((const uint16_t*)base)[idx]);
    }
  }
}

// Store VEC fp32 values as T; NT: 16-byte vectors non-temporally (y is not
// re-read), else write-back.
template <typename T, int VEC, bool NT = true>
__device__ __forceinline__ void store_vec(void* base, long long idx, const float* in) {
  if constexpr (sizeof(T) == 4) {
    if constexpr (VEC == 4) {
      f32x4 v = {in[0], in[1], in[2], in[3]};
      if constexpr (NT) __builtin_nontemporal_store(v, (f32x4*)((float*)base + idx));
      else *(f32x4*)((float*)base + idx) = v;
    } else {
      ((float*)base)[idx] = in[0];
    }
  } else {
    if constexpr (VEC == 8) {
      u32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = (uint32_t)Elem<T>::from_f32(in[2 * i]) | ((uint32_t)Elem<T>::from_f32(in[2 * i + 1]) << 16);
      if constexpr (NT) __builtin_nontemporal_store(v, (u32x4*)((uint16_t*)base + idx));
      else *(u32x4*)((uint16_t*)base + idx) = v;
    } else {
      ((uint16_t*)base)[idx] = Elem<T>::from_f32(in[0]);
    }
  }
}

// A row vector store in a kernel whose workgroup writes neighbouring rows:
// a vector in the row's first or last 128-byte line, when that line is
// shared with the neighbouring row, is stored write-back so the two rows'
// halves meet in L2 and leave as one line; the rest stream non-temporally.
// Measured on MI355X for LayerNorm bf16 [8191, 3000] (6000-byte rows; a
// workgroup writes 8 consecutive rows, so 7 of every 8 row boundaries lie
// inside one workgroup): 19.4 -> 18.0 us, the same bits.  The persistent
// one-wave softmax, whose neighbouring rows run on other XCDs, measured
// 2-4% slower with it and keeps non-temporal stores throughout.
template <typename T, int VEC>
__device__ __forceinline__ void store_vec_row_edge(void* row, long long idx, const float* in, long long row_bytes) {
  const uintptr_t first = (uintptr_t)row, last = first + (uintptr_t)row_bytes - 1;
  const uintptr_t at = first + (uintptr_t)(idx * (long long)sizeof(T));
  const bool shared = ((at >> 7) == (first >> 7) && (first & 127) != 0) ||
                      ((at >> 7) == (last >> 7) && ((last + 1) & 127) != 0);
  if (shared) store_vec<T, VEC, false>(row, idx, in);
  else store_vec<T, VEC, true>(row, idx, in);
}

// Weights are re-read by every row: keep them cacheable (plain loads).
template <typename T, int VEC>
__device__ __forceinline__ void load_param(const void* base, long long idx, float* out) {
  if constexpr (sizeof(T) == 4) {
    if constexpr (VEC == 4) {
      f32x4 v = *(const f32x4*)((const float*)base + idx);
      out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
    } else {
      out[0] = ((const float*)base)[idx];
    }
  } else {
    if constexpr (VEC == 8) {
      u32x4 v = *(const u32x4*)((const uint16_t*)base + idx);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[2 * i] = Elem<T>::to_f32((uint16_t)(v[i] & 0xFFFFu));
        out[2 * i + 1] = Elem<T>::to_f32((uint16_t)(v[i] >> 16));
      }
    } else {
      out[0] = Elem<T>::to_f32(((const uint16_t*)base)[idx]);
    }
  }
}

// Raw (undecoded) row vectors: what one 16-byte (or scalar) load returns.
template <typename T, int VEC> struct RawIO;
template <> struct RawIO<float, 4> {
  using type = f32x4;
  static __device__ __forceinline__ type load(const void* base, long long idx) {
    return __builtin_nontemporal_load((const f32x4*)((const float*)base + idx));
  }
  static __device__ __forceinline__ type load_cached(const void* base, long long idx) {
    return *(const f32x4*)((const float*)base + idx);
  }
  static __device__ __forceinline__ void unpack(const type& r, float* out) {
    out[0] = r[0]; out[1] = r[1]; out[2] = r[2]; out[3] = r[3];
  }
};
template <> struct RawIO<float, 1> {
  using type = float;
  static __device__ __forceinline__ type load(const void* base, long long idx) {
    return ((const float*)base)[idx];
  }
  static __device__ __forceinline__ type load_cached(const void* base, long long idx) {
    return ((const float*)base)[idx];
  }
  static __device__ __forceinline__ void unpack(const type& r, float* out) { out[0] = r; }
};
template <typename T> struct RawIO16 {
  using type = u32x4;
  static __device__ __forceinline__ type load(const void* base, long long idx) {
    return __builtin_nontemporal_load((const u32x4*)((const uint16_t*)base + idx));
  }
  static __device__ __forceinline__ type load_cached(const void* base, long long idx) {
    return *(const u32x4*)((const uint16_t*)base + idx);
  }
  static __device__ __forceinline__ void unpack(const type& r, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = Elem<T>::to_f32((uint16_t)(r[i] & 0xFFFFu));
      out[2 * i + 1] = Elem<T>::to_f32((uint16_t)(r[i] >> 16));
    }
  }
};
template <typename T> struct RawIO16s {
  using type = uint16_t;
  static __device__ __forceinline__ type load(const void* base, long long idx) {
    return ((const uint16_t*)base)[idx];
  }
  static __device__ __forceinline__ type load_cached(const void* base, long long idx) {
    return ((const uint16_t*)base)[idx];
  }
  static __device__ __forceinline__ void unpack(const type& r, float* out) { out[0] = Elem<T>::to_f32(r); }
};
template <> struct RawIO<bf16_t, 8> : RawIO16<bf16_t> {};
template <> struct RawIO<f16_t, 8> : RawIO16<f16_t> {};
template <> struct RawIO<bf16_t, 1> : RawIO16s<bf16_t> {};
template <> struct RawIO<f16_t, 1> : RawIO16s<f16_t> {};

// e^(x - m) with v_exp_f32.  FMA form (|m| < 2^24): exp2(fma(x, log2(e),
// -mL)) with mL = m * log2(e) rounded, one rounding before the exponential.
// The rounding of mL (at most half an ulp of mL, <= 1 below 2^24 * log2(e))
// shifts every exponent of a row by the same amount, which the softmax
// normalisation cancels (and which moves a logsumexp by |m| * 2^-24); the
// fma's own rounding gives a relative error of |x - m| * 2^-24 (6e-7 at
// x - m = -10) on top of v_exp_f32's ~1 ulp -- inside the fp32 bar of 1e-5
// relative.  Larger or infinite m: exp2((x - m) * log2(e)), the same error
// bound with two roundings (the FMA form's shift would leave the exponent
// range).  Masked lanes (x = -inf, m finite) give 0; an infinite m gives
// NaN where x is infinite too, as x - m does.
constexpr float kLog2e = 1.4426950408889634f;
template <bool FMA>
__device__ __forceinline__ float row_exp(float x, float m, float mL) {
  if constexpr (FMA) return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -mL));
  else return __builtin_amdgcn_exp2f((x - m) * kLog2e);
}
// calls f(std::true_type) when |m| < 2^24 (the FMA form of row_exp
// applies), f(std::false_type) otherwise: one wave-uniform branch
template <class F>
__device__ __forceinline__ void with_exp_form(float m, F&& f) {
  if (__builtin_fabsf(m) < 16777216.0f) f(std::true_type{});
  else f(std::false_type{});
}

// v rounded to T's precision (the value a store of T would keep)
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (sizeof(T) == 4) return v;
  else return Elem<T>::to_f32(Elem<T>::from_f32(v));
}

// layer_norm_forward_row's affine on one element: x_hat = (x - mean) * rstd
// in X's dtype, then x_hat * w + b with the reference's typed rounding
template <typename T>
__device__ __forceinline__ float lnrow_affine(float x, float mean, float rstd, float w, float b) {
  const float xh = round_to<T>((x - mean) * rstd);
  if constexpr (sizeof(T) == 4) return fmaf(xh, w, b);
  else return round_to<T>(xh * w) + b;
}

// logsumexp of one row from its NaN-ignoring max m, sum s = sum(exp(x - m))
// and NaN flag (ops/suite/perf/logsumexp.py kernel: a row with any NaN gives
// NaN; an infinite max is returned as is; else m + log(s)).
__device__ __forceinline__ float lse_finish(float m, float s, bool nan) {
  if (nan) return __builtin_nanf("");
  if (__builtin_fabsf(m) == __builtin_huge_valf()) return m;
  return m + logf(s);
}

// How a row kernel's lane vectors meet the row: live(i) -- vector i of the
// lane holds row elements; ok(i, e) -- element e of it is one; params(i, w,
// b) -- the weight / bias of its elements; store(i, o) -- write its row
// elements of y.  The aligned kernels' vectors are whole row vectors (ok is
// always true); the masked kernel's start at the 16-byte boundary below the
// row, so its edge vectors hold elements of the neighbouring rows.
template <class L, class O, class P, class S>
struct RowEdge {
  L live;
  O ok;
  P params;
  S store;
};
template <class L, class O, class P, class S>
__device__ __forceinline__ RowEdge<L, O, P, S> row_edge(L l, O o, P p, S s) {
  return {l, o, p, s};
}

// The per-row work once the row is in registers as fp32 (v, elements outside
// the row holding the op's identity): the reductions, statistics and y.
template <int OP, typename T, int VEC, int ITEMS, int BLOCK, class EG>
__device__ __forceinline__ void row_finish(const RowArgs& a, int row, float (&v)[ITEMS][VEC], int tid, float* scratch,
                                           const EG& eg) {
  if constexpr (OP == ROW_LOGSUMEXP) {
    // max ignores NaN (fmaxf), a separate flag carries it
    float m = -__builtin_huge_valf(), nan = 0.0f;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        m = fmaxf(m, v[i][e]);
        nan = (v[i][e] != v[i][e]) ? 1.0f : nan;
      }
    m = block_reduce<OpMax, BLOCK>(m, scratch);
    nan = block_reduce<OpMax, BLOCK>(nan, scratch);
    float s = 0.0f;
    if (__builtin_fabsf(m) != __builtin_huge_valf()) {
      const float mL = m * kLog2e;
      with_exp_form(m, [&](auto fc) {
        constexpr bool F = decltype(fc)::value;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
#pragma unroll
          for (int e = 0; e < VEC; ++e) s += row_exp<F>(v[i][e], m, mL);  // tail: exp(-inf) = 0
      });
    }
    s = block_reduce<OpSum, BLOCK>(s, scratch);
    if (tid == 0)
      store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, lse_finish(m, s, nan != 0.0f));
  } else if constexpr (OP == ROW_SOFTMAX) {
    // four independent max and sum chains per lane (a dependent VALU
    // operation waits ~11 cycles on gfx950)
    float m4[4] = {-__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf(),
                   -__builtin_huge_valf()};
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) m4[(i * VEC + e) & 3] = fmaxf(m4[(i * VEC + e) & 3], v[i][e]);
    float m = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
    m = block_reduce<OpMax, BLOCK>(m, scratch);
    const float mL = m * kLog2e;
    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    with_exp_form(m, [&](auto fc) {
      constexpr bool F = decltype(fc)::value;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          v[i][e] = row_exp<F>(v[i][e], m, mL);  // masked lanes: exp(-inf) = 0
          s4[(i * VEC + e) & 3] += v[i][e];
        }
    });
    float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    s = block_reduce<OpSum, BLOCK>(s, scratch);
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (eg.live(i)) {
        float o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = v[i][e] * inv;
        eg.store(i, o);
      }
    }
  } else if constexpr (OP == ROW_RMSNORM) {
    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four independent chains
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s4[(i * VEC + e) & 3] = fmaf(v[i][e], v[i][e], s4[(i * VEC + e) & 3]);
    float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    ss = block_reduce<OpSum, BLOCK>(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
    if (tid == 0) store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, inv);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (eg.live(i)) {
        float o[VEC], w[VEC], bb[VEC];
        eg.params(i, w, bb);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = (v[i][e] * inv) * w[e];
        eg.store(i, o);
      }
    }
  } else if constexpr (OP == ROW_LNROW) {
    // both sums in one pass (the reference's E[x^2] - mean^2 form)
    float s2[2] = {0.0f, 0.0f}, q2[2] = {0.0f, 0.0f};  // two chains each
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        s2[e & 1] += v[i][e];
        q2[e & 1] = fmaf(v[i][e], v[i][e], q2[e & 1]);
      }
    float s = s2[0] + s2[1], q = q2[0] + q2[1];
    s = block_reduce<OpSum, BLOCK>(s, scratch);
    q = block_reduce<OpSum, BLOCK>(q, scratch);
    const float inv_n = 1.0f / (float)a.cols;
    const float mean = s * inv_n;
    const float rstd = 1.0f / sqrtf(q * inv_n - mean * mean + a.eps);
    if (tid == 0) {
      store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, mean);
      store_from_f32(a.stat1, (long long)row * a.stat1_stride, a.stat_dtype, rstd);
    }
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (eg.live(i)) {
        float o[VEC], w[VEC], bb[VEC];
        eg.params(i, w, bb);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = lnrow_affine<T>(v[i][e], mean, rstd, w[e], bb[e]);
        eg.store(i, o);
      }
    }
  } else {  // LayerNorm, centered two-pass from registers
    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four independent chains
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s4[(i * VEC + e) & 3] += v[i][e];
    float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    s = block_reduce<OpSum, BLOCK>(s, scratch);
    const float mean = s / (float)a.cols;
    float q4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (eg.live(i)) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          if (eg.ok(i, e)) {
            v[i][e] -= mean;
            q4[(i * VEC + e) & 3] = fmaf(v[i][e], v[i][e], q4[(i * VEC + e) & 3]);
          }
        }
      }
    }
    float q = (q4[0] + q4[1]) + (q4[2] + q4[3]);
    q = block_reduce<OpSum, BLOCK>(q, scratch);
    const float rstd = 1.0f / sqrtf(q / (float)a.cols + a.eps);
    if (tid == 0) {
      store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, mean);
      store_from_f32(a.stat1, (long long)row * a.stat1_stride, a.stat_dtype, rstd);
    }
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (eg.live(i)) {
        float o[VEC], w[VEC], bb[VEC];
        eg.params(i, w, bb);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = v[i][e] * rstd * w[e] + bb[e];
        eg.store(i, o);
      }
    }
  }
}

// Persistent register-resident row kernel.  Workgroup g handles rows
// g, g + G, g + 2G, ... (the reference's persistent form
// tl.range(pid, n_rows, num_progs), ops/suite/dev/layer_norm_forward_row.py);
// the next row's loads are issued before the current row is reduced, and the
// per-column parameters (weight, bias) are loaded once per workgroup.
template <int OP, typename T, int VEC, int ITEMS, int BLOCK>
__device__ __forceinline__ void rr_regs_body(const RowArgs& a) {
  using IO = RawIO<T, VEC>;
  using R = typename IO::type;
  __shared__ float scratch[BLOCK / 64 > 0 ? BLOCK / 64 : 1];
  const int tid = threadIdx.x;
  const int nvec = a.cols / VEC;  // host guarantees cols % VEC == 0
  const long long xstride = a.x_row * (long long)sizeof(T);
  const long long ystride = a.y_row * (long long)sizeof(T);

  // parameters stay packed in registers (16-bit types: half the VGPRs)
  R wr[ITEMS], br[ITEMS];
  if constexpr (row_has_w(OP)) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int j = tid + i * BLOCK;
      if (j < nvec) {
        wr[i] = IO::load_cached(a.w, (long long)j * VEC);
        if constexpr (row_has_b(OP)) br[i] = IO::load_cached(a.b, (long long)j * VEC);
      }
    }
  }

  R cur[ITEMS], nxt[ITEMS];
  int row = blockIdx.x;
  {
    const char* xrow = (const char*)a.x + (long long)row * xstride;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int j = tid + i * BLOCK;
      if (j < nvec) cur[i] = IO::load(xrow, (long long)j * VEC);
    }
  }
  for (; row < a.rows; row += gridDim.x) {
    const int nrow = row + gridDim.x;
    if (nrow < a.rows) {
      const char* xrow = (const char*)a.x + (long long)nrow * xstride;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        const int j = tid + i * BLOCK;
        if (j < nvec) nxt[i] = IO::load(xrow, (long long)j * VEC);
      }
    }
    if constexpr (row_has_w(OP)) {
      // keep the decode of the packed parameters inside the loop: hoisting it
      // would hold them as fp32 for the whole kernel (twice the VGPRs)
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        asm volatile("" : "+v"(wr[i]));
        if constexpr (row_has_b(OP)) asm volatile("" : "+v"(br[i]));
      }
    }
    void* yrow = (char*)a.y + (long long)row * ystride;
    float v[ITEMS][VEC];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int j = tid + i * BLOCK;
      if (j < nvec) {
        IO::unpack(cur[i], v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          v[i][e] = (OP == ROW_SOFTMAX || OP == ROW_LOGSUMEXP) ? -__builtin_huge_valf() : 0.0f;
      }
    }

    row_finish<OP, T, VEC, ITEMS, BLOCK>(
        a, row, v, tid, scratch,
        row_edge([&](int i) { return tid + i * BLOCK < nvec; }, [](int, int) { return true; },
                 [&](int i, float* w, float* bb) {
                   if constexpr (row_has_w(OP)) IO::unpack(wr[i], w);
                   if constexpr (row_has_b(OP)) IO::unpack(br[i], bb);
                 },
                 [&](int i, const float* o) { store_vec<T, VEC>(yrow, (long long)(tid + i * BLOCK) * VEC, o); }));
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) cur[i] = nxt[i];
  }
}

// Row kernel for many rows of an op with per-column parameters, each row
// short enough for one wavefront: the parameters are staged in LDS once per
// workgroup of WAVES waves instead of once per wave, and each wave reduces
// RPW rows (its first row's loads are in flight while the parameters are
// staged, its next row's while the current one is reduced).  Workgroup g
// takes rows g*WAVES*RPW + wave + k*WAVES.  Measured on MI355X for C2
// LayerNorm (bf16 [8191, 3000]): 19.2 us against 20.2 for the one-row
// workgroups with parameters in registers (146 -> 107 VGPRs, and one
// parameter fetch per 8 rows instead of per row).
template <int OP, typename T, int VEC, int ITEMS, int WAVES, int RPW>
__device__ __forceinline__ void rw_body(const RowArgs& a) {
  using IO = RawIO<T, VEC>;
  using R = typename IO::type;
  __shared__ R wl[row_has_w(OP) ? ITEMS * 64 : 1];
  __shared__ R bl[row_has_b(OP) ? ITEMS * 64 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nvec = a.cols / VEC;  // host guarantees cols % VEC == 0 and nvec <= ITEMS * 64
  const long long xstride = a.x_row * (long long)sizeof(T);
  const long long ystride = a.y_row * (long long)sizeof(T);
  const int row0 = blockIdx.x * WAVES * RPW + wave;
  R cur[ITEMS], nxt[ITEMS];
  auto load = [&](int row, R (&dst)[ITEMS]) {
    const char* xrow = (const char*)a.x + (long long)row * xstride;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int j = lane + i * 64;
      if (j < nvec) dst[i] = IO::load(xrow, (long long)j * VEC);
    }
  };
  if (row0 < a.rows) load(row0, cur);
  if constexpr (row_has_w(OP)) {
    for (int j = threadIdx.x; j < nvec; j += WAVES * 64) {
      wl[j] = IO::load_cached(a.w, (long long)j * VEC);
      if constexpr (row_has_b(OP)) bl[j] = IO::load_cached(a.b, (long long)j * VEC);
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int row = row0 + k * WAVES;
    if (row >= a.rows) break;
    if (k + 1 < RPW && row + WAVES < a.rows) load(row + WAVES, nxt);
    float v[ITEMS][VEC];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int j = lane + i * 64;
      if (j < nvec) {
        IO::unpack(cur[i], v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          v[i][e] = (OP == ROW_SOFTMAX || OP == ROW_LOGSUMEXP) ? -__builtin_huge_valf() : 0.0f;
      }
    }
    char* yrow = (char*)a.y + (long long)row * ystride;
    row_finish<OP, T, VEC, ITEMS, 64>(
        a, row, v, lane, nullptr,
        row_edge([&](int i) { return lane + i * 64 < nvec; }, [](int, int) { return true; },
                 [&](int i, float* w, float* bb) {
                   if constexpr (row_has_w(OP)) IO::unpack(wl[lane + i * 64], w);
                   if constexpr (row_has_b(OP)) IO::unpack(bl[lane + i * 64], bb);
                 },
                 [&](int i, const float* o) {
                   store_vec_row_edge<T, VEC>(yrow, (long long)(lane + i * 64) * VEC, o, (long long)nvec * VEC * (long long)sizeof(T));
                 }));
    if (k + 1 < RPW) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) cur[i] = nxt[i];
    }
  }
}

// Parameters (gamma / beta, staged in LDS at their column index) of the
// columns v*VEC - ph .. v*VEC - ph + VEC-1 of a row whose start lies ph
// elements past a 16-byte boundary: the 32 bytes of LDS vectors v-1 and v,
// funnel-shifted by (VEC - ph) elements (v_alignbyte_b32 per dword), one
// branch per row phase (ph is wave-uniform).  Vector v-1 of v = 0 is
// replaced by vector 0: its columns lie before the row and are masked.
template <typename T, int VEC, int PH>
__device__ __forceinline__ u32x4 shift_pair(const u32x4& lo, const u32x4& hi) {
  constexpr int O = (VEC - PH) * (int)sizeof(T);  // byte offset of the first column in lo|hi
  constexpr int Q = O / 4, SH = O % 4;
  auto d = [&](int j) { return j < 4 ? lo[j] : hi[j - 4]; };
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if constexpr (SH == 0) r[k] = d(Q + k);
    else r[k] = __builtin_amdgcn_alignbyte(d(Q + k + 1), d(Q + k), SH);
  }
  return r;
}

template <typename T, int VEC, typename S>
__device__ __forceinline__ void shifted_params(const S* arr, int v, int ph, float* out) {
  using IO = RawIO<T, VEC>;
  using R = typename IO::type;
  const u32x4 hi = __builtin_bit_cast(u32x4, ((const R*)arr)[v]);
  const u32x4 lo = v > 0 ? __builtin_bit_cast(u32x4, ((const R*)arr)[v - 1]) : hi;
  u32x4 r;
  switch (ph) {
    case 0: r = hi; break;
    case 1: r = shift_pair<T, VEC, 1>(lo, hi); break;
    case 2: r = shift_pair<T, VEC, 2>(lo, hi); break;
    case 3: r = shift_pair<T, VEC, 3>(lo, hi); break;
    case 4: r = shift_pair<T, VEC, (VEC > 4 ? 4 : 0)>(lo, hi); break;
    case 5: r = shift_pair<T, VEC, (VEC > 5 ? 5 : 0)>(lo, hi); break;
    case 6: r = shift_pair<T, VEC, (VEC > 6 ? 6 : 0)>(lo, hi); break;
    default: r = shift_pair<T, VEC, (VEC > 7 ? 7 : 0)>(lo, hi); break;
  }
  IO::unpack(__builtin_bit_cast(R, r), out);
}

// Rows whose length is not a whole number of 16-byte vectors, or whose
// starts are not 16-byte aligned (e.g. bf16 [8191, 3001]): 16-byte aligned
// vector loads still, from the boundary at or below the row start, with a
// per-element mask at the two edge vectors -- elements of the neighbouring
// rows read as the op's identity, and the edge vectors' row elements are
// stored one by one (y's rows must share x's 16-byte phase).  An aligned
// 16-byte block holding a row element lies within the same page as that
// element, so the edge reads stay inside mapped memory.  The per-column
// parameters are staged in LDS element by element and read as two aligned
// vectors shifted to the row's phase (shifted_params).  Same workgroup shape
// as rw_body: WAVES waves, RPW rows each, one row per wave at a time.
template <int OP, typename T, int VEC, int ITEMS, int WAVES, int RPW>
__device__ __forceinline__ void rm_body(const RowArgs& a) {
  using IO = RawIO<T, VEC>;
  using R = typename IO::type;
  using S = typename std::conditional<sizeof(T) == 4, float, uint16_t>::type;  // storage element
  constexpr int MAXC = ITEMS * 64 * VEC;
  __shared__ __attribute__((aligned(16))) S wl[row_has_w(OP) ? MAXC : 1];
  __shared__ __attribute__((aligned(16))) S bl[row_has_b(OP) ? MAXC : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int cols = a.cols;  // host guarantees 0 < cols and ph + cols <= ITEMS * 64 * VEC
  if (cols <= 0) return;    // no row element: no vector may be read
  const int row0 = blockIdx.x * WAVES * RPW + wave;
  // 16-byte boundary at or below a row start and the start's phase (elements)
  auto base = [&](const void* p, long long row, long long stride, int& ph) -> char* {
    const uintptr_t at = (uintptr_t)p + (uintptr_t)(row * stride * (long long)sizeof(T));
    ph = (int)((at & 15) / sizeof(T));
    return (char*)(at & ~(uintptr_t)15);
  };
  R cur[ITEMS], nxt[ITEMS];
  int cph = 0, nph = 0;
  auto load = [&](int row, R (&dst)[ITEMS], int& ph) {
    const char* xlo = base(a.x, row, a.x_row, ph);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int j = lane + i * 64;
      if (j * VEC - ph < cols) dst[i] = IO::load(xlo, (long long)j * VEC);
    }
  };
  if (row0 < a.rows) load(row0, cur, cph);
  if constexpr (row_has_w(OP)) {
    for (int c = threadIdx.x; c < cols; c += WAVES * 64) {
      wl[c] = ((const S*)a.w)[c];
      if constexpr (row_has_b(OP)) bl[c] = ((const S*)a.b)[c];
    }
    __syncthreads();
  }
  constexpr float ident = (OP == ROW_SOFTMAX || OP == ROW_LOGSUMEXP) ? -__builtin_huge_valf() : 0.0f;
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int row = row0 + k * WAVES;
    if (row >= a.rows) break;
    if (k + 1 < RPW && row + WAVES < a.rows) load(row + WAVES, nxt, nph);
    const int ph = __builtin_amdgcn_readfirstlane(cph);  // one phase per row: wave-uniform
    auto col = [&](int i, int e) { return (lane + i * 64) * VEC + e - ph; };
    // LayerNorm: item i whole for every lane of the wave (wave-uniform, no
    // element before or after the row) skips the element masks, here and in
    // the centered pass ([8191, 3001] bf16: 25.5 -> 23.9 us, same bits; the
    // softmax measured 1.5% slower with it, so it keeps the masks)
    auto whole = [&](int i) {
      return OP == ROW_LAYERNORM && (i > 0 || ph == 0) && (i * 64 + 64) * VEC - ph <= cols;
    };
    auto ok = [&](int i, int e) {
      if (whole(i)) return true;
      const int c = col(i, e);
      return c >= 0 && c < cols;
    };
    float v[ITEMS][VEC];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      float t[VEC];
      if (whole(i)) {
        IO::unpack(cur[i], t);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[i][e] = t[e];
      } else {
        if ((lane + i * 64) * VEC - ph < cols) IO::unpack(cur[i], t);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[i][e] = ok(i, e) ? t[e] : ident;
      }
    }
    int yph;
    char* ylo = base(a.y, row, a.y_row, yph);  // yph == ph (host-checked)
    row_finish<OP, T, VEC, ITEMS, 64>(
        a, row, v, lane, nullptr,
        row_edge([&](int i) { return (lane + i * 64) * VEC - ph < cols; }, ok,
                 [&](int i, float* w, float* bb) {
                   if constexpr (row_has_w(OP)) shifted_params<T, VEC>(wl, lane + i * 64, ph, w);
                   if constexpr (row_has_b(OP)) shifted_params<T, VEC>(bl, lane + i * 64, ph, bb);
                 },
                 [&](int i, const float* o) {
                   const long long j = lane + i * 64;
                   if (j * VEC - ph >= 0 && j * VEC - ph + VEC <= cols) {
                     store_vec<T, VEC>(ylo, j * VEC, o);
                   } else {
#pragma unroll
                     for (int e = 0; e < VEC; ++e)
                       if (ok(i, e)) store_vec<T, 1>(ylo, j * VEC + e, &o[e]);
                   }
                 }));
    if (k + 1 < RPW) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) cur[i] = nxt[i];
      cph = nph;
    }
  }
}

// ------------------------------------------------------------- split rows
// Rows longer than one workgroup's registers hold, or too few rows to fill
// the chip, are cut into chunks of RS_CHUNK_VECS vectors; one RS_BLOCK-thread
// workgroup per (row, chunk).  Two launches, the reference's two-phase
// split with the merge in the second (a100c/plan/stages.py:668-752):
//   part   each workgroup reduces its register-resident chunk to a partial
//          record in the workspace: softmax/logsumexp (max, sum of
//          exp(x - max), NaN flag), RMSNorm (sum of squares), LayerNorm
//          (count, chunk mean, centered M2);
//   final  each workgroup merges its row's partials (max then rescaled sums;
//          Chan's pairwise moments for LayerNorm, exact in the count and
//          robust to offsets), re-reads its chunk and writes y; chunk 0 writes
//          the row statistics.  Logsumexp's final step is one workgroup per
//          row that only merges.
// x is read twice (the second read mostly from the MALL for the few-row
// shapes this path serves) and y written once.
constexpr int RS_BLOCK = 256;
constexpr int RS_ITEMS = 4;

// cached: the partial pass's loads are cacheable, so the final pass's
// re-read of the same chunk (one launch later) finds it in the MALL; the
// final pass reads it for the last time, nontemporally.  Measured on MI355X
// (six rotating input sets): bf16 [4, 2^22] softmax 18.7 -> 15.8 us,
// [64, 2^20] 66.6 -> 63.5 us against nontemporal loads in both passes.
template <int OP, typename T, int VEC>
__device__ __forceinline__ void rs_load(const RowArgs& a, int row, int split, float (&v)[RS_ITEMS][VEC],
                                        bool (&ok)[RS_ITEMS], bool cached) {
  using IO = RawIO<T, VEC>;
  const char* xrow = (const char*)a.x + (long long)row * a.x_row * (long long)sizeof(T);
  const int nvec = a.cols / VEC;
  const int base = split * (RS_BLOCK * RS_ITEMS);
  typename IO::type raw[RS_ITEMS];
#pragma unroll
  for (int i = 0; i < RS_ITEMS; ++i) {
    const int j = base + threadIdx.x + i * RS_BLOCK;
    ok[i] = j < nvec;
    if (ok[i]) raw[i] = cached ? IO::load_cached(xrow, (long long)j * VEC) : IO::load(xrow, (long long)j * VEC);
  }
#pragma unroll
  for (int i = 0; i < RS_ITEMS; ++i) {
    if (ok[i]) {
      IO::unpack(raw[i], v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        v[i][e] = (OP == ROW_SOFTMAX || OP == ROW_LOGSUMEXP) ? -__builtin_huge_valf() : 0.0f;
    }
  }
}

template <int OP, typename T, int VEC>
__device__ __forceinline__ void rs_part_body(const RowArgs& a) {
  __shared__ float scratch[RS_BLOCK / 64];
  const int row = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
  float v[RS_ITEMS][VEC];
  bool ok[RS_ITEMS];
  rs_load<OP, T, VEC>(a, row, split, v, ok, true);
  f32x4 p = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (OP == ROW_SOFTMAX || OP == ROW_LOGSUMEXP) {
    float m = -__builtin_huge_valf(), nan = 0.0f;
#pragma unroll
    for (int i = 0; i < RS_ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        m = fmaxf(m, v[i][e]);
        if constexpr (OP == ROW_LOGSUMEXP) nan = (v[i][e] != v[i][e]) ? 1.0f : nan;
      }
    m = block_reduce<OpMax, RS_BLOCK>(m, scratch);
    if constexpr (OP == ROW_LOGSUMEXP) nan = block_reduce<OpMax, RS_BLOCK>(nan, scratch);
    // a chunk without a finite max contributes nothing to a finite row max
    // (and must not form inf - inf); an infinite row max is handled at merge
    float z = 0.0f;
    if (__builtin_fabsf(m) != __builtin_huge_valf()) {
#pragma unroll
      for (int i = 0; i < RS_ITEMS; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) z += row_exp<false>(v[i][e], m, 0.0f);
    }
    z = block_reduce<OpSum, RS_BLOCK>(z, scratch);
    p[0] = m; p[1] = z; p[2] = nan;
  } else if constexpr (OP == ROW_RMSNORM) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < RS_ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss = fmaf(v[i][e], v[i][e], ss);
    p[0] = block_reduce<OpSum, RS_BLOCK>(ss, scratch);
  } else if constexpr (OP == ROW_LNROW) {
    float s = 0.0f, q = 0.0f;
#pragma unroll
    for (int i = 0; i < RS_ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        s += v[i][e];
        q = fmaf(v[i][e], v[i][e], q);
      }
    p[0] = block_reduce<OpSum, RS_BLOCK>(s, scratch);
    p[1] = block_reduce<OpSum, RS_BLOCK>(q, scratch);
  } else {
    const int first = split * (RS_BLOCK * RS_ITEMS * VEC);
    const float n = (float)min(RS_BLOCK * RS_ITEMS * VEC, a.cols - first);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < RS_ITEMS; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += v[i][e];
    const float mean = block_reduce<OpSum, RS_BLOCK>(s, scratch) / n;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < RS_ITEMS; ++i)
      if (ok[i]) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float c = v[i][e] - mean;
          q = fmaf(c, c, q);
        }
      }
    p[0] = n; p[1] = mean; p[2] = block_reduce<OpSum, RS_BLOCK>(q, scratch);
  }
  if (threadIdx.x == 0) ((f32x4*)a.part)[blockIdx.x] = p;
}

// Merge the partial records of one row (all RS_BLOCK threads take part).
// softmax / logsumexp: (max, sum at that max, NaN); norms: (statistic 0, 1).
template <int OP>
__device__ __forceinline__ f32x4 rs_merge(const RowArgs& a, int row, float* scratch) {
  const f32x4* part = (const f32x4*)a.part + (long long)row * a.splits;
  f32x4 r = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (OP == ROW_SOFTMAX || OP == ROW_LOGSUMEXP) {
    float m = -__builtin_huge_valf(), nan = 0.0f;
    for (int k = threadIdx.x; k < a.splits; k += RS_BLOCK) {
      m = fmaxf(m, part[k][0]);
      nan = fmaxf(nan, part[k][2]);
    }
    m = block_reduce<OpMax, RS_BLOCK>(m, scratch);
    nan = block_reduce<OpMax, RS_BLOCK>(nan, scratch);
    float z = 0.0f;
    for (int k = threadIdx.x; k < a.splits; k += RS_BLOCK) {
      const f32x4 q = part[k];
      if constexpr (OP == ROW_LOGSUMEXP) {
        if (__builtin_fabsf(m) != __builtin_huge_valf() && q[0] != -__builtin_huge_valf())
          z += q[1] * expf(q[0] - m);
      } else {
        // the reference's single-pass arithmetic: an all -inf or +inf row
        // ends in NaN, a finite row ignores its all -inf chunks
        z += (q[0] == -__builtin_huge_valf() && m != -__builtin_huge_valf()) ? 0.0f : q[1] * expf(q[0] - m);
      }
    }
    r[0] = m; r[1] = block_reduce<OpSum, RS_BLOCK>(z, scratch); r[2] = nan;
  } else if constexpr (OP == ROW_RMSNORM) {
    float ss = 0.0f;
    for (int k = threadIdx.x; k < a.splits; k += RS_BLOCK) ss += part[k][0];
    r[0] = block_reduce<OpSum, RS_BLOCK>(ss, scratch);
  } else if constexpr (OP == ROW_LNROW) {
    float s = 0.0f, q = 0.0f;
    for (int k = threadIdx.x; k < a.splits; k += RS_BLOCK) {
      s += part[k][0];
      q += part[k][1];
    }
    r[0] = block_reduce<OpSum, RS_BLOCK>(s, scratch);
    r[1] = block_reduce<OpSum, RS_BLOCK>(q, scratch);
  } else {
    // Chan et al.: mean = sum(n_k mean_k) / n; M2 = sum(M2_k + n_k (mean_k - mean)^2)
    float s = 0.0f;
    for (int k = threadIdx.x; k < a.splits; k += RS_BLOCK) s += part[k][0] * part[k][1];
    const float mean = block_reduce<OpSum, RS_BLOCK>(s, scratch) / (float)a.cols;
    float q = 0.0f;
    for (int k = threadIdx.x; k < a.splits; k += RS_BLOCK) {
      const float d = part[k][1] - mean;
      q += part[k][2] + part[k][0] * d * d;
    }
    r[0] = mean; r[1] = block_reduce<OpSum, RS_BLOCK>(q, scratch);
  }
  return r;
}

template <int OP, typename T, int VEC>
__device__ __forceinline__ void rs_final_body(const RowArgs& a) {
  __shared__ float scratch[RS_BLOCK / 64];
  if constexpr (OP == ROW_LOGSUMEXP) {
    const int row = blockIdx.x;
    const f32x4 r = rs_merge<OP>(a, row, scratch);
    if (threadIdx.x == 0)
      store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, lse_finish(r[0], r[1], r[2] != 0.0f));
  } else {
    const int row = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
    float v[RS_ITEMS][VEC];
    bool ok[RS_ITEMS];
    rs_load<OP, T, VEC>(a, row, split, v, ok, false);  // in flight during the merge
    const f32x4 r = rs_merge<OP>(a, row, scratch);
    void* yrow = (char*)a.y + (long long)row * a.y_row * (long long)sizeof(T);
    const int base = split * (RS_BLOCK * RS_ITEMS);
    float mul = 1.0f, sub = 0.0f;
    if constexpr (OP == ROW_SOFTMAX) {
      sub = r[0];
      mul = 1.0f / r[1];
    } else if constexpr (OP == ROW_RMSNORM) {
      mul = 1.0f / sqrtf(r[0] / (float)a.cols + a.eps);
      if (split == 0 && threadIdx.x == 0) store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, mul);
    } else if constexpr (OP == ROW_LNROW) {
      const float inv_n = 1.0f / (float)a.cols;
      sub = r[0] * inv_n;
      mul = 1.0f / sqrtf(r[1] * inv_n - sub * sub + a.eps);
      if (split == 0 && threadIdx.x == 0) {
        store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, sub);
        store_from_f32(a.stat1, (long long)row * a.stat1_stride, a.stat_dtype, mul);
      }
    } else {
      sub = r[0];
      mul = 1.0f / sqrtf(r[1] / (float)a.cols + a.eps);
      if (split == 0 && threadIdx.x == 0) {
        store_from_f32(a.stat0, (long long)row * a.stat0_stride, a.stat_dtype, sub);
        store_from_f32(a.stat1, (long long)row * a.stat1_stride, a.stat_dtype, mul);
      }
    }
#pragma unroll
    for (int i = 0; i < RS_ITEMS; ++i) {
      if (!ok[i]) continue;
      const int j = base + threadIdx.x + i * RS_BLOCK;
      float o[VEC];
      if constexpr (OP == ROW_SOFTMAX) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = row_exp<false>(v[i][e], sub, 0.0f) * mul;
      } else if constexpr (OP == ROW_RMSNORM) {
        float w[VEC];
        load_param<T, VEC>(a.w, (long long)j * VEC, w);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = (v[i][e] * mul) * w[e];
      } else if constexpr (OP == ROW_LNROW) {
        float w[VEC], bb[VEC];
        load_param<T, VEC>(a.w, (long long)j * VEC, w);
        load_param<T, VEC>(a.b, (long long)j * VEC, bb);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = lnrow_affine<T>(v[i][e], sub, mul, w[e], bb[e]);
      } else {
        float w[VEC], bb[VEC];
        load_param<T, VEC>(a.w, (long long)j * VEC, w);
        load_param<T, VEC>(a.b, (long long)j * VEC, bb);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = (v[i][e] - sub) * mul * w[e] + bb[e];
      }
      store_vec<T, VEC>(yrow, (long long)j * VEC, o);
    }
  }
}

}  // namespace g950

// ------------------------------------------------------------------ symbols
// Kernel names: g950_rr_<op>_<dtype>_v<VEC>_i<ITEMS>_b<BLOCK> and the split
// pair g950_rs_{part,final}_<op>_<dtype>_v<VEC>.  The launcher (g950rt.cpp)
// picks the smallest register configuration whose BLOCK*ITEMS*VEC covers the
// row, or the split pair for long rows and for too few rows.
#define G950_RR_REGS(OPNAME, OP, TNAME, T, VEC, ITEMS, BLOCK)                              \
  extern "C" __global__ __launch_bounds__(BLOCK) void                                    \
      g950_rr_##OPNAME##_##TNAME##_v##VEC##_i##ITEMS##_b##BLOCK(const g950::RowArgs a) { \
    g950::rr_regs_body<OP, T, VEC, ITEMS, BLOCK>(a);                                     \
  }

#define G950_RS(OPNAME, OP, TNAME, T, VEC)                                                       \
  extern "C" __global__ __launch_bounds__(g950::RS_BLOCK) void                                      \
      g950_rs_part_##OPNAME##_##TNAME##_v##VEC(const g950::RowArgs a) {                             \
    g950::rs_part_body<OP, T, VEC>(a);                                                              \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(g950::RS_BLOCK) void                                      \
      g950_rs_final_##OPNAME##_##TNAME##_v##VEC(const g950::RowArgs a) {                            \
    g950::rs_final_body<OP, T, VEC>(a);                                                             \
  }

// register configurations: (VEC, ITEMS, BLOCK).  Vector forms need
// cols % VEC == 0 and 16-byte aligned rows; VEC=1 forms take any row.
#define G950_RR_SET(OPNAME, OP, TNAME, T, V)            \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 1, 64)          \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 2, 64)          \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 4, 64)          \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 6, 64)          \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 8, 64)          \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 16, 64)         \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 8, 256)         \
  G950_RR_REGS(OPNAME, OP, TNAME, T, V, 16, 256)

#define G950_RR_ALL(OPNAME, OP)                                          \
  G950_RR_SET(OPNAME, OP, f32, float, 4)                                 \
  G950_RR_SET(OPNAME, OP, f32, float, 1)                                 \
  G950_RR_SET(OPNAME, OP, bf16, g950::bf16_t, 8)                         \
  G950_RR_SET(OPNAME, OP, bf16, g950::bf16_t, 1)                         \
  G950_RR_SET(OPNAME, OP, f16, g950::f16_t, 8)                           \
  G950_RR_SET(OPNAME, OP, f16, g950::f16_t, 1)                           \
  G950_RS(OPNAME, OP, f32, float, 4)                                     \
  G950_RS(OPNAME, OP, f32, float, 1)                                     \
  G950_RS(OPNAME, OP, bf16, g950::bf16_t, 8)                             \
  G950_RS(OPNAME, OP, bf16, g950::bf16_t, 1)                             \
  G950_RS(OPNAME, OP, f16, g950::f16_t, 8)                               \
  G950_RS(OPNAME, OP, f16, g950::f16_t, 1)

G950_RR_ALL(softmax, g950::ROW_SOFTMAX)
G950_RR_ALL(rmsnorm, g950::ROW_RMSNORM)
G950_RR_ALL(layernorm, g950::ROW_LAYERNORM)
G950_RR_ALL(logsumexp, g950::ROW_LOGSUMEXP)
G950_RR_ALL(lnrow, g950::ROW_LNROW)

// Parameter rows in LDS (rw_body): g950_rw_<op>_<dtype>_v<VEC>_i<ITEMS>,
// 4 waves x 2 rows per workgroup, vector forms only.
#define G950_RW(OPNAME, OP, TNAME, T, VEC, ITEMS)                                        \
  extern "C" __global__ __launch_bounds__(256) void                                      \
      g950_rw_##OPNAME##_##TNAME##_v##VEC##_i##ITEMS(const g950::RowArgs a) {            \
    g950::rw_body<OP, T, VEC, ITEMS, 4, 2>(a);                                           \
  }
#define G950_RW_SET(OPNAME, OP, TNAME, T, VEC) \
  G950_RW(OPNAME, OP, TNAME, T, VEC, 1)        \
  G950_RW(OPNAME, OP, TNAME, T, VEC, 2)        \
  G950_RW(OPNAME, OP, TNAME, T, VEC, 4)        \
  G950_RW(OPNAME, OP, TNAME, T, VEC, 6)        \
  G950_RW(OPNAME, OP, TNAME, T, VEC, 8)
#define G950_RW_ALL(OPNAME, OP)                  \
  G950_RW_SET(OPNAME, OP, f32, float, 4)         \
  G950_RW_SET(OPNAME, OP, bf16, g950::bf16_t, 8) \
  G950_RW_SET(OPNAME, OP, f16, g950::f16_t, 8)
G950_RW_ALL(layernorm, g950::ROW_LAYERNORM)
G950_RW_ALL(lnrow, g950::ROW_LNROW)

// Masked aligned vectors (rm_body) for rows that are not whole, aligned
// 16-byte vectors: g950_rm_<op>_<dtype>_v<VEC>_i<ITEMS>, 4 waves x 2 rows.
#define G950_RM(OPNAME, OP, TNAME, T, VEC, ITEMS)                                        \
  extern "C" __global__ __launch_bounds__(256) void                                      \
      g950_rm_##OPNAME##_##TNAME##_v##VEC##_i##ITEMS(const g950::RowArgs a) {            \
    g950::rm_body<OP, T, VEC, ITEMS, 4, 2>(a);                                           \
  }
#define G950_RM_SET(OPNAME, OP, TNAME, T, VEC) \
  G950_RM(OPNAME, OP, TNAME, T, VEC, 1)        \
  G950_RM(OPNAME, OP, TNAME, T, VEC, 2)        \
  G950_RM(OPNAME, OP, TNAME, T, VEC, 4)        \
  G950_RM(OPNAME, OP, TNAME, T, VEC, 6)        \
  G950_RM(OPNAME, OP, TNAME, T, VEC, 8)
#define G950_RM_ALL(OPNAME, OP)                  \
  G950_RM_SET(OPNAME, OP, f32, float, 4)         \
  G950_RM_SET(OPNAME, OP, bf16, g950::bf16_t, 8) \
  G950_RM_SET(OPNAME, OP, f16, g950::f16_t, 8)
G950_RM_ALL(softmax, g950::ROW_SOFTMAX)
G950_RM_ALL(logsumexp, g950::ROW_LOGSUMEXP)
G950_RM_ALL(rmsnorm, g950::ROW_RMSNORM)
G950_RM_ALL(layernorm, g950::ROW_LAYERNORM)
G950_RM_ALL(lnrow, g950::ROW_LNROW)

// ------------------------------------------------------------- stream copy
// y = x for n 16-byte vectors, grid-stride, nontemporal loads and stores --
// the same memory path as the row kernels.  It is the calibration kernel for
// the HBM traffic counters (its bytes are known exactly) and a plain copy op.
extern "C" __global__ __launch_bounds__(256) void g950_stream_copy(const g950::CopyArgs a) {
  using g950::u32x4;
  const u32x4* x = (const u32x4*)a.x;
  u32x4* y = (u32x4*)a.y;
  const long long stride = (long long)gridDim.x * 256 * 4;
  for (long long i = (long long)blockIdx.x * 256 * 4 + threadIdx.x; i < a.n16; i += stride) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + u * 256 < a.n16) v[u] = __builtin_nontemporal_load(x + i + u * 256);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + u * 256 < a.n16) __builtin_nontemporal_store(v[u], y + i + u * 256);
  }
}

