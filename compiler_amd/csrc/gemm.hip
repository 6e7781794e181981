// GEMM family on gfx950: bf16/fp16 (fp32 accumulate) and int8 (int32
// accumulate, bit-exact) with a fused epilogue.
//
// Operator semantics: ops/suite/perf/matmul.py:21-37 (Y = A.B, fp32
// accumulator, masked M/N/K edges, store in the output pointer dtype);
// int8 dot family a100c/plan/tiles.py:118-131 (signed operands, modular int32
// accumulator); dequant rule ops/suite/perf/dequantize_matmul.py:29-38
// (per-column scale), here with the per-row A scale as well:
// Y[m,n] = bf16(float(acc[m,n]) * sa[m] * sb[n]).
//
// MFMA kernel (g950_gemm_*_256x256): both operands K-contiguous (A row-major
// [M,K]; B stored as Bt[N,K], i.e. column-major [K,N]).  The `_rb` variants
// (16-bit) read the reference's row-major B[K,N] as it lies, with
// transposing LDS reads (the BROW notes above gemm_mfma16_body).
//   * workgroup tile 256x256, 8 waves (4 x 2, two per SIMD), wave tile
//     64 x 128: 4 x 8 fragments of v_mfma_f32_16x16x32_{bf16,f16} /
//     v_mfma_i32_16x16x64_i8 for whole-slab 16-bit / int8 shapes with
//     M, N >= 256 (gemm_mfma16_body), else 2 x 4 fragments of the 32x32
//     forms; the B tile feeds the MFMA A port so each lane ends with four
//     consecutive output columns of one output row
//   * K in slabs of 128 bytes per row (64 bf16 / 128 int8); two LDS stages
//     of 64 KiB (A rows then B rows, 128-byte rows), filled by direct
//     global->LDS 16-byte DMA (global_load_lds_dwordx4) of whole 128-byte
//     lines (measured on MI355X: 64-byte row pieces cost the load path 1.5x
//     per byte); the DMA takes a scalar base plus a fixed 32-bit lane offset
//     and the fragment reads fixed per-lane LDS offsets plus immediates, so
//     the main loop holds MFMAs, LDS reads, DMAs and scalar work only
//   * the eight 16-byte chunks of a 128-byte LDS row are XOR-swizzled with
//     (row >> 1) & 7, so the 32 rows an MFMA operand read touches spread over
//     all 64 banks
//   * per slab: four k-steps; each k-step's MFMAs run with the next k-step's
//     fragment reads (second register set) spread between them, and the
//     slab's DMA is spread over k-step 3 of the previous slab and k-step 0
//     (sched_group_barrier), issued by one wave of each SIMD only, so the
//     other wave's MFMAs fill the matrix core while the DMA wave waits on the
//     load path; one workgroup barrier per slab, before k-step 3
//   * XCD-aware block order: consecutive tiles go to the same XCD (the
//     hardware deals workgroups round-robin over 8 XCDs), grouped 4 tile-rows
//     deep for L2 reuse (4 beat 2, 8, 16 and 32 at 8192^3)
//   * M/N edges: loads clamp the row index (the duplicated rows only feed
//     output rows/cols that are never stored); stores are masked.  K must be a
//     whole number of slabs (host checks), otherwise the general kernel runs.
//
// General kernel (g950_gemm_general): any strides, any K, fp32/fp16/bf16
// inputs (fp32 FMA) or int8 (int32 exact); 64x64 tiles.  It serves the
// layouts no MFMA route takes (unaligned rows, non-unit inner strides) and
// the no-alloc entry when a copy of B would not fit its scratch array.
#include "g950_common.h"

#include <utility>

namespace g950 {

enum GemmMode : int { GEMM_BF16 = 0, GEMM_F16 = 1, GEMM_I8 = 2, GEMM_F32 = 3 };

// MFMAs per 16-byte operand chunk: the 16-bit and int8 forms consume a whole
// chunk per lane in one v_mfma (K 16 / 32); fp32 (v_mfma_f32_32x32x2_f32,
// one value per lane) takes the chunk's four values in four MFMAs
constexpr int mfma_per_chunk(int mode) { return mode == GEMM_F32 ? 4 : 1; }

// 1: whole-slab 16-bit / int8 GEMMs with M, N >= 256 run on 16x16 output
// fragments (gemm_mfma16_body); 0: every shape on the 32x32 form
#ifndef G950_GEMM16
#define G950_GEMM16 1
#endif
constexpr int BM = 256, BN = 256;  // workgroup tile
constexpr int SLAB = 128;          // bytes of K per row per LDS stage (two stages)

// 128 zero bytes: the DMA source of every 16-byte chunk past K in the last
// (partial) K slab, so the tail multiplies zeros instead of reading past a
// row (K % 64 != 0 kernels only)
__device__ __attribute__((aligned(128))) const uint32_t g950_zero_line[32] = {};

// One 16-byte-per-lane global->LDS DMA instruction (global_load_lds_dwordx4,
// scalar base + 32-bit lane offset, LDS destination in M0) written as inline
// asm: the compiler then sees no LDS write in flight and adds no vmcnt wait
// before the transposing LDS reads (ds_read_tr16_b64), whose address it
// cannot compare with a DMA destination.  Completion is the slab protocol's
// explicit vmcnt(0) + barrier.  (s_nop 0: one wait state between the M0
// write and the DMA.)
__device__ __forceinline__ void dma16_asm(const char* sbase, uint32_t voff, uint32_t lds_dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_dst);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// Map the linear workgroup id to a (tile_m, tile_n): XCD-contiguous, then
// grouped by 4 tile-rows.  The hardware deals workgroups round-robin over
// the 8 XCDs, so XCD x runs ids x, x + 8, ...: it takes the contiguous run of
// floor(total / 8) tiles (one more for x < total % 8) starting at
// x * floor(total / 8) + min(x, total % 8).  Tile counts that are not a
// multiple of 8 took ids in plain order before: 4097x11008x4096 (731 tiles)
// 283 -> 268 us, the same bits.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int x = pid & 7;
  pid = x * (total >> 3) + min(x, total & 7) + (pid >> 3);
  const int group = 4;
  const int per_group = group * tiles_n;
  const int gid = pid / per_group;
  const int first = gid * group;
  const int gsize = min(tiles_m - first, group);
  const int in = pid - gid * per_group;
  tm = first + in % gsize;
  tn = in / gsize;
}

// Epilogue: lane holds C[m][n..n+3] for m = row r of each 32-row fragment,
// n = 8q + 4g + {0..3} of each 32-column fragment; (wm0, wn0) is the first
// output row / column of the wave's tile.  UMASK (int8 only): bit 0 A
// unsigned, bit 1 B unsigned -- the accumulator of the offset operands gets
// its exact correction (modulo 2^32, GemmArgs::rsum / csum).
template <int MODE, int FM, int FN, int UMASK = 0, int RF = 32, class FA = f32x16, class IA = i32x16>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& p, const FA (&accf)[FM][FN],
                                              const IA (&acci)[FM][FN], int wm0, int wn0,
                                              int lane, int m_lo = 0, int n_lo = 0) {
  // only rows >= m_lo and columns >= n_lo are stored (a tile computed over a
  // window shifted back from the matrix edge owns only its own part)
  // RF x RF output fragments: lane holds C[m][n..n+3] for m = row lane % RF of
  // each fragment and n = 4 * (lane / RF) + (64 / RF) * 4 * q, q < QN
  constexpr int QN = RF * RF / 256;
  const int r = lane % RF, g = lane / RF;
  const bool vec_ok = ((p.c_s0 & 3) == 0);
  // per-row factors
  bool live[FM];
  float rs[FM];
  uint32_t rcorr[FM];
#pragma unroll
  for (int mi = 0; mi < FM; ++mi) {
    const int m = wm0 + mi * RF + r;
    live[mi] = m < p.M && m >= m_lo;
    rs[mi] = 1.0f;
    rcorr[mi] = 0;
    if constexpr (MODE == GEMM_I8) {
      if (live[mi] && p.sa) rs[mi] = p.sa[m];
      if constexpr (UMASK & 2) rcorr[mi] = live[mi] ? 128u * (uint32_t)p.rsum[m] : 0u;
      if constexpr (UMASK == 3) rcorr[mi] -= 16384u * (uint32_t)p.K;
    }
  }
  // one group: C[m][n..n+3] of fragment (mi, ni), column factors colf
  // (sb for int8, cscale for the 16-bit / fp32 GEMMs) and colc (128 * csum)
  auto group = [&](int mi, int ni, int q, int n, bool full, const float (&colf)[4], const uint32_t (&colc)[4]) {
    const int m = wm0 + mi * RF + r;
    float v[4];
    if constexpr (MODE == GEMM_I8) {
      int iv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) iv[e] = (int)((uint32_t)acci[mi][ni][q * 4 + e] + rcorr[mi] + colc[e]);
      if (p.acc_out) {
        int* dst = p.acc_out + (long long)m * p.acc_s0 + n;
        if (((p.acc_s0 & 3) == 0) && full) {
          *(i32x4*)dst = (i32x4){iv[0], iv[1], iv[2], iv[3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.N && n + e >= n_lo) dst[e] = iv[e];
        }
      }
      if (!p.sa) return;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = ((float)iv[e] * rs[mi]) * colf[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = accf[mi][ni][q * 4 + e];
      if (p.cscale) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= colf[e];
      }
    }
    char* crow = (char*)p.c + (long long)m * p.c_s0 * (p.c_dtype == DT_F32 ? 4 : 2);
    if (p.c_dtype == DT_F32) {
      float* dst = (float*)crow + n;
      if (vec_ok && full) {
        *(f32x4*)dst = (f32x4){v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < p.N && n + e >= n_lo) dst[e] = v[e];
      }
    } else {
      uint16_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = (p.c_dtype == DT_BF16) ? f32_to_bf16(v[e]) : f32_to_f16(v[e]);
      uint16_t* dst = (uint16_t*)crow + n;
      if (vec_ok && full) {
        *(u32x2*)dst = (u32x2){(uint32_t)h[0] | ((uint32_t)h[1] << 16),
                               (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < p.N && n + e >= n_lo) dst[e] = h[e];
      }
    }
  };
  const bool colwise = MODE == GEMM_I8 || p.cscale;
  if (!colwise) {
    // no column factors: row by row, the stores of a row back to back
    const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    const uint32_t zero[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int mi = 0; mi < FM; ++mi) {
      if (!live[mi]) continue;
#pragma unroll
      for (int ni = 0; ni < FN; ++ni)
#pragma unroll
        for (int q = 0; q < QN; ++q) {
          const int n = wn0 + ni * RF + q * (256 / RF) + g * 4;
          if (n + 3 < n_lo) continue;
          group(mi, ni, q, n, n + 3 < p.N && n >= n_lo && (n & 3) == 0, one, zero);
        }
    }
    return;
  }
  // column factors: loaded once per group of four columns and shared by the
  // fragment rows, as one vector load where the group lies inside N and the
  // vector is aligned -- a scalar load per element cost a load-path slot
  // each (128 per lane per tile for the int8 dequant scale)
  const bool sb_vec = MODE == GEMM_I8 && p.sb && ((uintptr_t)p.sb & 15) == 0;
  const bool cs_vec = MODE != GEMM_I8 && p.cscale &&
                      ((uintptr_t)p.cscale & (p.cscale_dtype == DT_F32 ? 15 : 7)) == 0;
  const bool csum_vec = (UMASK & 1) && ((uintptr_t)p.csum & 15) == 0;
#pragma unroll
  for (int ni = 0; ni < FN; ++ni) {
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      const int n = wn0 + ni * RF + q * (256 / RF) + g * 4;
      if (n >= p.N || n + 3 < n_lo) continue;
      const bool full = n + 3 < p.N && n >= n_lo && (n & 3) == 0;
      float colf[4] = {1.0f, 1.0f, 1.0f, 1.0f};
      uint32_t colc[4] = {0u, 0u, 0u, 0u};
      if constexpr (MODE == GEMM_I8) {
        if (p.sa) {
          if (sb_vec && full) {
            const f32x4 t = *(const f32x4*)(p.sb + n);
#pragma unroll
            for (int e = 0; e < 4; ++e) colf[e] = t[e];
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) colf[e] = (n + e < p.N) ? p.sb[n + e] : 0.0f;
          }
        }
        if constexpr (UMASK & 1) {
          if (csum_vec && full) {
            const i32x4 t = *(const i32x4*)(p.csum + n);
#pragma unroll
            for (int e = 0; e < 4; ++e) colc[e] = 128u * (uint32_t)t[e];
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) colc[e] = (n + e < p.N) ? 128u * (uint32_t)p.csum[n + e] : 0u;
          }
        }
      } else {
        if (cs_vec && full) {
          if (p.cscale_dtype == DT_F32) {
            const f32x4 t = *(const f32x4*)((const float*)p.cscale + n);
#pragma unroll
            for (int e = 0; e < 4; ++e) colf[e] = t[e];
          } else {
            const u32x2 t = *(const u32x2*)((const uint16_t*)p.cscale + n);
            const bool bf = p.cscale_dtype == DT_BF16;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint16_t hb = (uint16_t)(t[e >> 1] >> (16 * (e & 1)));
              colf[e] = bf ? bf16_to_f32(hb) : f16_to_f32(hb);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            colf[e] = (n + e < p.N) ? load_as_f32(p.cscale, n + e, p.cscale_dtype) : 0.0f;
        }
      }
#pragma unroll
      for (int mi = 0; mi < FM; ++mi)
        if (live[mi]) group(mi, ni, q, n, full, colf, colc);
    }
  }
}

// One operand chunk into the accumulator.  fp32: lane half h of both
// operands holds k = 4c + e (c the chunk index of the half), so MFMA e sums
// A[m][k] B[k][n] over the two halves' k -- every k of the slab exactly once,
// in an order both operands share.
template <int MODE>
__device__ __forceinline__ void mfma_step(const u32x4& bfrag, const u32x4& afrag, f32x16& accf,
                                          i32x16& acci) {
  if constexpr (MODE == GEMM_F32) {
    // bit-cast the whole vectors, then index: this compiler reads element 0
    // for every __builtin_bit_cast of a single ext_vector element
    const f32x4 bv = __builtin_bit_cast(f32x4, bfrag), av = __builtin_bit_cast(f32x4, afrag);
#pragma unroll
    for (int e = 0; e < 4; ++e) accf = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[e], av[e], accf, 0, 0, 0);
  } else if constexpr (MODE == GEMM_BF16) {
    accf = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, bfrag),
                                                   __builtin_bit_cast(bf16x8, afrag), accf, 0, 0, 0);
  } else if constexpr (MODE == GEMM_F16) {
    accf = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, bfrag),
                                                  __builtin_bit_cast(f16x8, afrag), accf, 0, 0, 0);
  } else {
    acci = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, bfrag),
                                                 __builtin_bit_cast(i32x4, afrag), acci, 0, 0, 0);
  }
}

// Epilogue of the 16x16 form for a 16-bit output whose tile owns all of its
// window's columns: the wave's 64 x 128 output tile passes through its own
// 16 KiB of LDS and leaves as whole 256-byte row pieces, 16 bytes per lane,
// in non-temporal stores.  Lane (g4, l16) of fragment (mi, ni) holds C[row
// mi*16 + l16][cols ni*16 + 4 g4 .. + 3]: 8 bytes into 16-byte chunk
// ni*2 + g4/2 of its LDS row, the chunk index XOR-swizzled by row & 15 (the
// 16 rows of one write spread over the 64 banks; a read of 16 chunks of one
// row covers them once).  Rows below m_lo belong to the tile above (a
// window shifted back from the bottom edge) and are not stored.  Measured
// on MI355X against row-by-row 8-byte stores: 8192^3 bf16 757 -> 694 us,
// row-major B 785 -> 708, W8A16 8192^3 816 -> 750, int8 4096x8192x8192
// 199 -> 194, 4097x11008x4096 287 -> 281, the same bits; non-temporal 8-byte
// stores without the staging cost 4097x11008x4096 9% and the int8 GEMM 19%
// (partial lines), and the staging with write-back stores gained 1%.
template <int MODE, int FM, int FN, int UMASK>
__device__ __forceinline__ void gemm_epilogue_lds(const GemmArgs& p, const f32x4 (&accf)[FM][FN],
                                                  const i32x4 (&acci)[FM][FN], int wm0, int wn0, int lane,
                                                  int m_lo, char* reg) {
  constexpr int RB = FN * 32;         // bytes of one wave-tile row
  constexpr int CPR = RB / 16;        // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;       // rows per store instruction
  static_assert(CPR == 16, "the row swizzle spans 16 chunks");
  const int l16 = lane & 15, g4 = lane >> 4;
  const bool bf = p.c_dtype == DT_BF16;
  float rs[FM];
  uint32_t rcorr[FM];
#pragma unroll
  for (int mi = 0; mi < FM; ++mi) {
    const int m = wm0 + mi * 16 + l16;
    rs[mi] = 1.0f;
    rcorr[mi] = 0;
    if constexpr (MODE == GEMM_I8) {
      rs[mi] = p.sa[m];
      if constexpr (UMASK & 2) rcorr[mi] = 128u * (uint32_t)p.rsum[m];
      if constexpr (UMASK == 3) rcorr[mi] -= 16384u * (uint32_t)p.K;
    }
  }
#pragma unroll
  for (int ni = 0; ni < FN; ++ni) {
    const int n = wn0 + ni * 16 + g4 * 4;
    float colf[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    uint32_t colc[4] = {0u, 0u, 0u, 0u};
    if constexpr (MODE == GEMM_I8) {
      if (((uintptr_t)p.sb & 15) == 0) {
        const f32x4 t = *(const f32x4*)(p.sb + n);
#pragma unroll
        for (int e = 0; e < 4; ++e) colf[e] = t[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) colf[e] = p.sb[n + e];
      }
      if constexpr (UMASK & 1) {
        if (((uintptr_t)p.csum & 15) == 0) {
          const i32x4 t = *(const i32x4*)(p.csum + n);
#pragma unroll
          for (int e = 0; e < 4; ++e) colc[e] = 128u * (uint32_t)t[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) colc[e] = 128u * (uint32_t)p.csum[n + e];
        }
      }
    } else if (p.cscale) {
      if (p.cscale_dtype == DT_F32 && ((uintptr_t)p.cscale & 15) == 0) {
        const f32x4 t = *(const f32x4*)((const float*)p.cscale + n);
#pragma unroll
        for (int e = 0; e < 4; ++e) colf[e] = t[e];
      } else if (p.cscale_dtype != DT_F32 && ((uintptr_t)p.cscale & 7) == 0) {
        const u32x2 t = *(const u32x2*)((const uint16_t*)p.cscale + n);
        const bool cbf = p.cscale_dtype == DT_BF16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t hb = (uint16_t)(t[e >> 1] >> (16 * (e & 1)));
          colf[e] = cbf ? bf16_to_f32(hb) : f16_to_f32(hb);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) colf[e] = load_as_f32(p.cscale, n + e, p.cscale_dtype);
      }
    }
#pragma unroll
    for (int mi = 0; mi < FM; ++mi) {
      // the same arithmetic, in the same order, as gemm_epilogue
      float v[4];
      if constexpr (MODE == GEMM_I8) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = ((float)(int)((uint32_t)acci[mi][ni][e] + rcorr[mi] + colc[e]) * rs[mi]) * colf[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = accf[mi][ni][e] * colf[e];
      }
      uint16_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = bf ? f32_to_bf16(v[e]) : f32_to_f16(v[e]);
      const int row = mi * 16 + l16, chunk = ni * 2 + (g4 >> 1);
      *(u32x2*)(reg + row * RB + ((chunk ^ l16) << 4) + (g4 & 1) * 8) =
          (u32x2){(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
    }
  }
  const long long cs = (long long)p.c_s0 * 2;
  char* cbase = (char*)p.c + (long long)wm0 * cs + (long long)wn0 * 2;
#pragma unroll
  for (int it = 0; it < FM * 16 / RPI; ++it) {
    const int r = it * RPI + lane / CPR, c = lane % CPR;
    const u32x4 v = *(const u32x4*)(reg + r * RB + ((c ^ (r & 15)) << 4));
    if (wm0 + r >= m_lo) __builtin_nontemporal_store(v, (u32x4*)(cbase + r * cs + c * 16));
  }
}

// 16x16-fragment form of the 256x256 kernel, for M and N of at least one
// tile: a tile at the bottom / right edge computes the 256 x 256 window
// ending at the matrix edge (every DMA row lies inside the operands, so a
// lane's DMA source is a fixed 32-bit offset plus a wave-uniform base, no
// per-row clamp) and stores only its own rows and columns.
//
// BROW (16-bit only): B is the reference matmul's own row-major [K, N]
// (N-contiguous, ops/suite/perf/matmul.py:33) and is read as it lies, with
// no transposed copy.  A slab's 64 k-rows of the tile's 256 columns land in
// LDS as four 64-column blocks of 64 rows x 128 bytes -- the same 8-row x
// 128-byte DMA instruction as the K-contiguous operands, whole 128-byte
// lines of B -- and each B fragment (16 columns x 8 k per lane) comes out of
// two ds_read_b64_tr_b16 (gfx950's transposing read: in each 16-lane group,
// lane 4r + j reads 4 columns of k-row r and lane i receives column i of the
// four rows).  The 16-byte chunks of k-row k are XOR-swizzled by
// 2 * (((k >> 1) & 1) | (((k >> 3) & 1) << 1)), so the eight k-rows a half
// wave reads (k, k+1, k+2, k+3 and the same eight rows on) cover the 64 banks
// once.  Stages sit as [A0][B0][B1][A1] so a B read of either stage is one
// per-lane base plus an immediate below 64 KiB.
template <int MODE, int WM, int WN, int UMASK, bool BROW = false>
__device__ __forceinline__ void gemm_mfma16_body(const GemmArgs& p, char* lds) {
  constexpr int NW = WM * WN;
  constexpr int STAGE = (BM + BN) * SLAB;     // 64 KiB
  constexpr int DW = NW / 2;                  // DMA waves: the first half, one per SIMD
  constexpr int GROUPS = (BM + BN) / 8 / DW;  // 8-row DMA groups per DMA wave per slab
  constexpr int H = GROUPS / 2;
  static_assert(GROUPS * 8 * DW == BM + BN && GROUPS % 2 == 0 && (BM / 8) % GROUPS == 0,
                "each DMA wave's groups lie in one operand");
  static_assert(!BROW || (MODE == GEMM_BF16 || MODE == GEMM_F16), "row-major B: 16-bit operands");
  // LDS byte offsets of stage s's A and B slabs
  constexpr int A_OFF[2] = {0, BROW ? STAGE + BN * SLAB : STAGE};
  constexpr int B_OFF[2] = {BM * SLAB, BROW ? BM * SLAB + BN * SLAB : STAGE + BM * SLAB};
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m_own = tm * BM, n_own = tn * BN;
  const int m0 = min(m_own, p.M - BM);  // the window the tile computes
  const int n0 = min(n_own, p.N - BN);
  constexpr int ES = (MODE == GEMM_I8) ? 1 : 2;  // element bytes
  const long long lda_b = p.a_s0 * ES;
  const long long ldb_b = p.b_s0 * ES;
  const char* abase = (const char*)p.a + (long long)m0 * lda_b;
  const char* bbase = (const char*)p.b + (long long)n0 * ldb_b;
  const int kslabs = p.K * ES / SLAB;
  const int last = kslabs - 1;
  // DMA: wave w < DW owns row groups w*GROUPS .. +GROUPS-1 (A rows for the
  // first BM/8 groups, B rows after), 8 rows x 128 bytes per instruction
  // (lane: row lane / 8, 16-byte slot lane % 8 holding chunk slot ^ ((row >>
  // 1) & 7)).  Group t's rows are the first group's plus 8t, and the
  // swizzle repeats every second group, so a lane needs two offsets.
  // Row-major B: group g (of the slab's 32) is column block g / 8, k-rows
  // 8 (g % 8) .. +7; its swizzle repeats every second group too.
  const bool dma_a = wave * GROUPS < BM / 8;
  const bool dma_brow = BROW && !dma_a;
  const long long ld = dma_a ? lda_b : ldb_b;
  // per-slab step of the DMA source: 128 bytes of K, or 64 k-rows of row-major B
  const long long slab_step = dma_brow ? 64 * ldb_b : SLAB;
  const int g0 = dma_a ? wave * GROUPS : wave * GROUPS - BM / 8;  // first group of this wave in its operand
  const char* obase = dma_a ? abase : dma_brow ? (const char*)p.b + (long long)n0 * 2 + (g0 >> 3) * 128 : bbase;
  uint32_t doff[2];
  {
    const int r8 = lane >> 3;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (dma_brow) {
        const int k = 8 * j + r8;
        const int sw = 2 * (((k >> 1) & 1) | (((k >> 3) & 1) << 1));
        doff[j] = (uint32_t)((long long)k * ld + (((lane & 7) ^ sw) * 16));
      } else {
        const int row = g0 * 8 + r8 + 8 * j;
        doff[j] = (uint32_t)((long long)row * ld + (((lane & 7) ^ ((row >> 1) & 7)) * 16));
      }
    }
  }
  // LDS byte address of the stages (the asm DMA's M0)
  const uint32_t lds32 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
  auto issue = [&](int stage, int slab, int t0, int t1) {
    char* st = lds + (dma_a ? A_OFF[stage] : B_OFF[stage]);
#pragma unroll
    for (int t = t0; t < t1; ++t) {
      // wave-uniform part of group t's source: column block and row pair
      const long long grp = dma_brow ? (long long)(t >> 3) * 128 + (long long)((t & 7) & ~1) * 8 * ld
                                     : (long long)(t & ~1) * 8 * ld;
      const char* ub = obase + (long long)slab * slab_step + grp;
      if constexpr (BROW) {
        dma16_asm(ub, doff[t & 1], lds32 + (uint32_t)((dma_a ? A_OFF[stage] : B_OFF[stage]) + (g0 + t) * 1024));
      } else {
        asm volatile("" : "+v"(doff[t & 1]));
        const char* src = ub + (uint64_t)doff[t & 1];
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(st + (g0 + t) * 1024),
                                         16, 0, 0);
      }
    }
  };
  // ---- 16x16 output fragments (v_mfma_f32_16x16x32_{bf16,f16} /
  // v_mfma_i32_16x16x64_i8: 16 bytes of K per lane, the 64-byte k-step
  // split over the four 16-lane groups).  Under the power limit these
  // sustain more FLOP/s than the 32x32x16 form with the same operand
  // traffic (half the accumulator register traffic per FLOP).  Wave tile
  // 64 x 128 = 4 x 8 fragments; per slab two k-steps of 64 bytes.  Lane
  // (g4, l16) reads row l16 of each 16-row fragment, chunk 4 ks + g4; the
  // swizzle (row >> 1) & 7 depends on l16 alone, so fragment i is the
  // lane's offset plus an immediate i * 16 rows (conflict-free: each
  // 16-lane group covers the 64 banks once).
  constexpr int FM16 = BM / WM / 16, FN16 = BN / WN / 16;
  f32x4 acf[FM16][FN16];
  i32x4 aci[FM16][FN16];
#pragma unroll
  for (int i = 0; i < FM16; ++i)
#pragma unroll
    for (int j = 0; j < FN16; ++j) {
      if constexpr (MODE == GEMM_I8) aci[i][j] = (i32x4){};
      else acf[i][j] = (f32x4){};
    }
  const int l16 = lane & 15, g4 = lane >> 4;
  int aoff[2][2], boff[2][2];
#pragma unroll
  for (int s_ = 0; s_ < 2; ++s_)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int sw = (((ks * 4 + g4) ^ ((l16 >> 1) & 7)) << 4) + l16 * SLAB;
      aoff[s_][ks] = A_OFF[s_] + wm * (BM / WM) * SLAB + sw;
      boff[s_][ks] = B_OFF[s_] + wn * (BN / WN) * SLAB + sw;
    }
  // Row-major B fragment ni of k-step ks: lane (g4, 4 r + j) reads k-rows
  // 32 ks + 8 g4 + r (and + 4) at columns 4 j .. 4 j + 3 of the fragment's 16,
  // in column block 2 wn + ni / 4, chunk pair (ni % 4) ^ swizzle: the lane's
  // base for each ni % 4 (stage 0), everything else an immediate (stage 1 is
  // the next 32 KiB).
  int btr[4];
  if constexpr (BROW) {
    const int r = l16 >> 2, j = l16 & 3;
    const int sw = ((r >> 1) & 1) | ((g4 & 1) << 1);
#pragma unroll
    for (int cp = 0; cp < 4; ++cp)
      btr[cp] = B_OFF[0] + (2 * wn) * 64 * SLAB + (8 * g4 + r) * SLAB + 32 * (cp ^ sw) + 8 * j;
  }
  u32x4 a16[2][FM16], b16[FN16];
  auto afrag = [&](auto sc, int ks, int buf) {
    constexpr int S = decltype(sc)::value;
#pragma unroll
    for (int mi = 0; mi < FM16; ++mi) a16[buf][mi] = *(const u32x4*)(lds + aoff[S][ks] + mi * 16 * SLAB);
  };
  auto bfrag = [&](auto sc, int ks, int ni) {
    constexpr int S = decltype(sc)::value;
    if constexpr (BROW) {
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      const int off = btr[ni & 3] + S * BN * SLAB + (ni >> 2) * 64 * SLAB + ks * 32 * SLAB;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(lds + off));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(lds + off + 4 * SLAB));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      b16[ni] = (u32x4){l2[0], l2[1], h2[0], h2[1]};
    } else {
      b16[ni] = *(const u32x4*)(lds + boff[S][ks] + ni * 16 * SLAB);
    }
  };
  auto mma = [&](const u32x4& bv, const u32x4& av, f32x4& cf, i32x4& ci) {
    if constexpr (MODE == GEMM_BF16)
      cf = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, bv), __builtin_bit_cast(bf16x8, av),
                                                   cf, 0, 0, 0);
    else if constexpr (MODE == GEMM_F16)
      cf = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bv), __builtin_bit_cast(f16x8, av), cf,
                                                  0, 0, 0);
    else
      ci = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, bv), __builtin_bit_cast(i32x4, av), ci,
                                                 0, 0, 0);
  };
  // One k-step: the MFMAs of (a16[buf], b16) with the next k-step's
  // fragments read behind them -- stage NS, k-step nks: A into the other
  // buffer (first four slots), each B fragment into its own registers once
  // its last MFMA has issued -- and ndma DMA instructions spread over the
  // slots; an explicit lgkmcnt(0) closes the k-step (the compiler cannot
  // count LDS reads issued behind a DMA).
  // (BROW: the DMA is inline asm, which the scheduling groups cannot place,
  // so the k-step issues its ndma DMA groups itself, dt0.. of slab dslab into
  // stage dst: two among the next k-step's A reads, then one behind each B
  // fragment's reads; the asm keeps its place among the LDS reads.  Issued
  // one behind each B fragment from the first, the last DMA of a k-step
  // lands just before the slab barrier's vmcnt(0): measured 812 -> 798 us at
  // 8192^3.)
  constexpr int NMF16 = FM16 * FN16;
  constexpr int EARLY = 2;  // BROW: DMA groups issued among the A reads
  auto kstep = [&](auto bc, auto nsc, int nks, int ndma, int dst = 0, int dslab = 0, int dt0 = 0) {
    constexpr int buf = decltype(bc)::value;
    if constexpr (BROW) {
      constexpr int S = decltype(nsc)::value;
#pragma unroll
      for (int mi = 0; mi < FM16; ++mi) {
        a16[buf ^ 1][mi] = *(const u32x4*)(lds + aoff[S][nks] + mi * 16 * SLAB);
        if (mi >= 1 && mi <= EARLY && mi - 1 < ndma) issue(dst, dslab, dt0 + mi - 1, dt0 + mi);
      }
    } else {
      afrag(nsc, nks, buf ^ 1);
    }
    if constexpr (UMASK & 1) {
#pragma unroll
      for (int mi = 0; mi < FM16; ++mi) a16[buf][mi] ^= 0x80808080u;
    }
#pragma unroll
    for (int ni = 0; ni < FN16; ++ni) {
      if constexpr (UMASK & 2) b16[ni] ^= 0x80808080u;
#pragma unroll
      for (int mi = 0; mi < FM16; ++mi) mma(b16[ni], a16[buf][mi], acf[mi][ni], aci[mi][ni]);
      bfrag(nsc, nks, ni);
      if constexpr (BROW) {
        const int dj = ni + EARLY;
        if (dj < ndma) issue(dst, dslab, dt0 + dj, dt0 + dj + 1);
      }
    }
#pragma unroll
    for (int i = 0; i < NMF16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < FM16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (i % FM16 == FM16 - 1) __builtin_amdgcn_sched_group_barrier(0x100, BROW ? 2 : 1, 0);
      if (!BROW && ndma && i % (NMF16 / ndma) == 1 && i / (NMF16 / ndma) < ndma)
        __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  };
  // Two-stage protocol as below, with two k-steps per slab: the barrier
  // sits between them, after every read of slab kt (k-step 1's fragments
  // are read during k-step 0) and after the slab kt + 1 DMA landed.
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  const bool dwave = wave < DW;
  if (dwave) issue(0, 0, 0, GROUPS);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  afrag(S0{}, 0, 0);
#pragma unroll
  for (int ni = 0; ni < FN16; ++ni) bfrag(S0{}, 0, ni);
  if (dwave) issue(1, min(1, last), 0, H);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  auto run = [&](auto dc) {
    constexpr bool DMA = decltype(dc)::value;
    auto slab_iter = [&](auto cc, int kt) {
      constexpr int CUR = decltype(cc)::value, NXT = CUR ^ 1;
      if constexpr (DMA && !BROW) issue(NXT, min(kt + 1, last), H, GROUPS);
      kstep(S0{}, cc, 1, DMA ? H : 0, NXT, min(kt + 1, last), H);
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DMA && !BROW) issue(CUR, min(kt + 2, last), 0, H);
      // (after the last slab: a stale stage, never used)
      kstep(S1{}, std::integral_constant<int, NXT>{}, 0, DMA ? H : 0, CUR, min(kt + 2, last), 0);
    };
    int kt = 0;
    for (; kt + 1 < kslabs; kt += 2) {
      slab_iter(S0{}, kt);
      slab_iter(S1{}, kt + 1);
    }
    if (kt < kslabs) slab_iter(S0{}, kt);
  };
  if (dwave) run(std::true_type{});
  else run(std::false_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // 16-bit output, the tile owning its window's columns, 16-byte aligned
  // rows: staged through LDS (uniform over the workgroup, so every wave
  // reaches the barrier that frees the stages: each wave's reads ended with
  // its last k-step's lgkmcnt(0), each DMA wave's loads with the vmcnt(0))
  if (n0 == n_own && p.c_dtype != DT_F32 && (p.c_s0 & 7) == 0 && ((uintptr_t)p.c & 15) == 0 &&
      (MODE != GEMM_I8 || (p.sa && !p.acc_out))) {
    __syncthreads();
    gemm_epilogue_lds<MODE, FM16, FN16, UMASK>(p, acf, aci, m0 + wm * (BM / WM), n0 + wn * (BN / WN), lane, m_own,
                                               lds + wave * (BM / WM) * (BN / WN) * 2);
    return;
  }
  gemm_epilogue<MODE, FM16, FN16, UMASK, 16>(p, acf, aci, m0 + wm * (BM / WM), n0 + wn * (BN / WN), lane, m_own,
                                              n_own);
}

// WM x WN waves; wave tile (BM/WM) x (BN/WN) = FM x FN fragments of 32x32.
// UMASK (int8): bit 0 A unsigned, bit 1 B unsigned.  An unsigned operand's
// bytes are flipped (XOR 0x80: u - 128, a signed int8) as its fragments enter
// the MFMA; the epilogue adds the exact correction.
template <int MODE, int WM, int WN, int UMASK = 0, bool KTAIL = false>
__device__ __forceinline__ void gemm_mfma_body(const GemmArgs& p) {
  constexpr int NW = WM * WN;
  constexpr int FM = BM / WM / 32;
  constexpr int FN = BN / WN / 32;
  constexpr int STAGE = (BM + BN) * SLAB;     // 64 KiB
  constexpr int DW = NW / 2;                  // DMA waves: the first half, one per SIMD
  constexpr int GROUPS = (BM + BN) / 8 / DW;  // 8-row DMA groups per DMA wave per slab
  constexpr int H = GROUPS / 2;
  static_assert(GROUPS * 8 * DW == BM + BN && GROUPS % 2 == 0, "DMA split over waves and halves");
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];
  if constexpr (G950_GEMM16 && MODE != GEMM_F32 && !KTAIL) {
    // whole-slab 16-bit / int8 GEMMs of at least one tile each way take the
    // 16x16-fragment form (uniform per launch)
    if (p.M >= BM && p.N >= BN) {
      gemm_mfma16_body<MODE, WM, WN, UMASK>(p, lds);
      return;
    }
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  constexpr int ES = (MODE == GEMM_I8) ? 1 : (MODE == GEMM_F32) ? 4 : 2;  // element bytes
  const long long lda_b = p.a_s0 * ES;
  const long long ldb_b = p.b_s0 * ES;  // Bt row stride (n) in bytes
  const char* abase = (const char*)p.a + (long long)m0 * lda_b;
  const char* bbase = (const char*)p.b + (long long)n0 * ldb_b;
  const int a_lim = p.M - 1 - m0;
  const int b_lim = p.N - 1 - n0;
  // KTAIL: K need only be a whole number of 16-byte chunks; the last slab's
  // chunks past K come from g950_zero_line
  const int kbytes = p.K * ES;
  const int kslabs = KTAIL ? (kbytes + SLAB - 1) / SLAB : kbytes / SLAB;
  const int last = kslabs - 1;

  f32x16 accf[FM][FN];
  i32x16 acci[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (MODE == GEMM_I8) acci[i][j] = (i32x16){};
      else accf[i][j] = (f32x16){};
    }

  // DMA: one wave instruction moves 8 rows x 128 bytes (lane: row lane / 8,
  // 16-byte slot lane % 8, which holds the swizzled chunk).  Row groups
  // 0..BM/8-1 are A rows, the rest B rows; DMA wave w (w < DW) owns groups
  // w*GROUPS .. w*GROUPS+GROUPS-1, issued in two halves.  Waves are dealt to
  // the four SIMDs round-robin, so each SIMD pairs one DMA wave with one
  // wave that only multiplies: while the DMA wave waits on the load path
  // (every wave issuing at once left both waves of a SIMD stalled together),
  // the other keeps the matrix core busy (measured on MI355X at 8192^3:
  // 1361 -> 1415 TFLOP/s).
  const int dr = lane >> 3;
  const int dslot = lane & 7;
  // Whole-slab kernels: a lane's DMA rows are fixed for the whole kernel, so
  // its byte offsets from the operand base are computed once (32-bit: the
  // host routes operands whose rows reach past 4 GiB to the _kt kernels) and
  // each slab's source is a wave-uniform base plus that offset -- the
  // scalar-base form of the load, no vector address arithmetic per DMA.  The
  // empty asm re-defines the offset inside the loop so instruction selection
  // sees the (scalar + 32-bit lane offset) shape there instead of a 64-bit
  // address hoisted out of it.  _kt kernels keep 64-bit addresses.
  uint32_t doff[GROUPS];
#pragma unroll
  for (int t = 0; t < GROUPS; ++t) {
    const int rg = wave * GROUPS + t;
    const bool is_a = rg < BM / 8;
    const int row = (is_a ? rg : rg - BM / 8) * 8 + dr;
    const int grow = min(row, is_a ? a_lim : b_lim);
    const int chunk = dslot ^ ((row >> 1) & 7);
    doff[t] = (uint32_t)((long long)grow * (is_a ? lda_b : ldb_b) + chunk * 16);
  }
  auto issue = [&](int stage, int slab, int t0, int t1) {
    char* st = lds + stage * STAGE;
    const long long kb = (long long)slab * SLAB;
#pragma unroll
    for (int t = t0; t < t1; ++t) {
      const int rg = wave * GROUPS + t;
      const bool is_a = rg < BM / 8;
      const char* src;
      if constexpr (KTAIL) {
        const int row = (is_a ? rg : rg - BM / 8) * 8 + dr;
        const int grow = min(row, is_a ? a_lim : b_lim);
        const int chunk = dslot ^ ((row >> 1) & 7);
        src = (is_a ? abase : bbase) + (long long)grow * (is_a ? lda_b : ldb_b) + kb + chunk * 16;
        if (kb + chunk * 16 >= kbytes) src = (const char*)g950_zero_line;
      } else {
        const char* ub = (is_a ? abase : bbase) + kb;
        asm volatile("" : "+v"(doff[t]));
        src = ub + (uint64_t)doff[t];
      }
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(st + rg * 1024),
                                       16, 0, 0);
    }
  };

  // Fragments of k-step ks (16 bf16 / 32 int8 of K) of one stage: lane
  // (g, r) reads 16 bytes of row r of each 32-row fragment, chunk 2 ks + g.
  const int g = lane >> 5;
  const int r = lane & 31;
  u32x4 af[2][FM], bfr[2][FN];
  // Per-lane LDS offsets of k-step ks's fragments in stage s, computed once:
  // the swizzle (row >> 1) & 7 depends on r alone (fragment rows start at
  // multiples of 32), so fragment mi (ni) is that offset plus an immediate
  // mi (ni) * 32 rows, and the loop does no address arithmetic.
  int aoff[2][4], boff[2][4];
#pragma unroll
  for (int s_ = 0; s_ < 2; ++s_)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int sw = ((((ks * 2 + g) ^ ((r >> 1) & 7))) << 4) + r * SLAB;
      aoff[s_][ks] = s_ * STAGE + wm * (BM / WM) * SLAB + sw;
      boff[s_][ks] = s_ * STAGE + BM * SLAB + wn * (BN / WN) * SLAB + sw;
    }
  auto frags = [&](auto sc, int ks, int buf) {
    constexpr int S = decltype(sc)::value;
#pragma unroll
    for (int mi = 0; mi < FM; ++mi) af[buf][mi] = *(const u32x4*)(lds + aoff[S][ks] + mi * 32 * SLAB);
#pragma unroll
    for (int ni = 0; ni < FN; ++ni) bfr[buf][ni] = *(const u32x4*)(lds + boff[S][ks] + ni * 32 * SLAB);
  };
  auto mfmas = [&](int buf) {
    if constexpr (UMASK & 1) {
#pragma unroll
      for (int mi = 0; mi < FM; ++mi) af[buf][mi] ^= 0x80808080u;
    }
    if constexpr (UMASK & 2) {
#pragma unroll
      for (int ni = 0; ni < FN; ++ni) bfr[buf][ni] ^= 0x80808080u;
    }
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
      for (int ni = 0; ni < FN; ++ni)
        mfma_step<MODE>(bfr[buf][ni], af[buf][mi], accf[mi][ni], acci[mi][ni]);
  };
  // One MFMA per slot; the next k-step's LDS reads in the first FM + FN
  // slots; ndma DMA instructions spread evenly over the slots.  The compiler
  // cannot count LDS reads issued behind a DMA, so each k-step ends with an
  // explicit lgkmcnt(0), by when its reads are long done.
  constexpr int NMF = FM * FN * mfma_per_chunk(MODE);  // MFMAs per k-step
  auto kstep = [&](int buf, int ndma) {
    mfmas(buf);
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < FM + FN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (ndma && i % (NMF / ndma) == 0 && i / (NMF / ndma) < ndma)
        __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  };

  // Two-stage protocol.  Iteration kt consumes slab kt from stage kt % 2.
  // Slab kt + 1 goes to the other stage: its first DMA half in k-step 3 of
  // iteration kt - 1, its second half in k-step 0 of iteration kt, both past
  // the barrier after which nobody reads slab kt - 1 again.  The barrier
  // before k-step 3 comes after every read of slab kt (the k-step 3
  // fragments are read during k-step 2) and after each DMA wave's loads of
  // slab kt + 1 have landed (its vmcnt(0) just before the barrier); k-step 3
  // then reads slab kt + 1's first fragments.
  // Past the end of K the DMA re-reads the last slab into a stage nobody
  // reads again, so the loop body has no branch.
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  const bool dwave = wave < DW;
  if (dwave) issue(0, 0, 0, GROUPS);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  frags(S0{}, 0, 0);
  if (dwave) issue(1, min(1, last), 0, H);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  // the main loop in two compiled forms, with and without the DMA: same
  // barriers, so the two wave roles stay in step slab by slab; two slabs per
  // trip, so each stage's fragment offsets are compile-time picks (an odd
  // last slab runs from stage 0)
  auto run = [&](auto dc) {
    constexpr bool DMA = decltype(dc)::value;
    auto slab_iter = [&](auto cc, int kt) {
      constexpr int CUR = decltype(cc)::value, NXT = CUR ^ 1;
      if constexpr (DMA) issue(NXT, min(kt + 1, last), H, GROUPS);
      frags(cc, 1, 1);
      kstep(0, DMA ? H : 0);
      frags(cc, 2, 0);
      kstep(1, 0);
      frags(cc, 3, 1);
      kstep(0, 0);
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DMA) issue(CUR, min(kt + 2, last), 0, H);
      frags(std::integral_constant<int, NXT>{}, 0, 0);  // (after the last slab: a stale stage, never used)
      kstep(1, DMA ? H : 0);
    };
    int kt = 0;
    for (; kt + 1 < kslabs; kt += 2) {
      slab_iter(S0{}, kt);
      slab_iter(S1{}, kt + 1);
    }
    if (kt < kslabs) slab_iter(S0{}, kt);
  };
  if (dwave) run(std::true_type{});
  else run(std::false_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  gemm_epilogue<MODE, FM, FN, UMASK>(p, accf, acci, m0 + wm * (BM / WM), n0 + wn * (BN / WN), lane);
}

// Bt[n][k] = B[k][n] for 16-bit elements: B [K, N] row-major with row stride
// b_s0 elements (16-byte aligned rows, N % 8 == 0), Bt contiguous [N, K] at
// p.c (K % 8 == 0).  64 x 64 tiles through LDS, one 32-bit slot per element
// with a 65-slot row pitch, so the column reads of the transposition and the
// row writes are both conflict-free; 16-byte loads and stores.
__device__ __forceinline__ void transpose16_body(const GemmArgs& p) {
  __shared__ uint32_t t[64][65];
  const int tiles_n = (p.N + 63) / 64;
  const int k0 = (blockIdx.x / tiles_n) * 64, n0 = (blockIdx.x % tiles_n) * 64;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i, k = c >> 3, n8 = (c & 7) * 8;
    if (k0 + k < p.K && n0 + n8 < p.N) {
      const u32x4 w = *(const u32x4*)((const uint16_t*)p.b + (long long)(k0 + k) * p.b_s0 + n0 + n8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t[k][n8 + 2 * e] = w[e] & 0xFFFFu;
        t[k][n8 + 2 * e + 1] = w[e] >> 16;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i, n = c >> 3, k8 = (c & 7) * 8;
    if (n0 + n < p.N && k0 + k8 < p.K) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = t[k8 + 2 * e][n] | (t[k8 + 2 * e + 1][n] << 16);
      *(u32x4*)((uint16_t*)p.c + (long long)(n0 + n) * p.K + k0 + k8) = w;
    }
  }
}

// The same for 32-bit elements (N % 4 == 0, K % 4 == 0): 16-byte vectors of 4.
__device__ __forceinline__ void transpose32_body(const GemmArgs& p) {
  __shared__ uint32_t t[64][65];
  const int tiles_n = (p.N + 63) / 64;
  const int k0 = (blockIdx.x / tiles_n) * 64, n0 = (blockIdx.x % tiles_n) * 64;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + 256 * i, k = c >> 4, n4 = (c & 15) * 4;
    if (k0 + k < p.K && n0 + n4 < p.N) {
      const u32x4 w = *(const u32x4*)((const uint32_t*)p.b + (long long)(k0 + k) * p.b_s0 + n0 + n4);
#pragma unroll
      for (int e = 0; e < 4; ++e) t[k][n4 + e] = w[e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + 256 * i, n = c >> 4, k4 = (c & 15) * 4;
    if (n0 + n < p.N && k0 + k4 < p.K) {
      const u32x4 w = {t[k4][n], t[k4 + 1][n], t[k4 + 2][n], t[k4 + 3][n]};
      *(u32x4*)((uint32_t*)p.c + (long long)(n0 + n) * p.K + k0 + k4) = w;
    }
  }
}

// The same for bytes (int8 weights, N % 16 == 0, K % 16 == 0, 16-byte aligned
// rows): 64 x 64 byte tiles, one 16-byte load (a k-row's 16 columns) and one
// 16-byte store (an n-row's 16 k) per thread, bytes staged as 32-bit slots
// with a 65-slot pitch.
__device__ __forceinline__ void transpose8_body(const GemmArgs& p) {
  __shared__ uint32_t t[64][65];
  const int tiles_n = (p.N + 63) / 64;
  const int k0 = (blockIdx.x / tiles_n) * 64, n0 = (blockIdx.x % tiles_n) * 64;
  {
    const int k = threadIdx.x >> 2, n16 = (threadIdx.x & 3) * 16;
    if (k0 + k < p.K && n0 + n16 < p.N) {
      const u32x4 w = *(const u32x4*)((const uint8_t*)p.b + (long long)(k0 + k) * p.b_s0 + n0 + n16);
#pragma unroll
      for (int e = 0; e < 16; ++e) t[k][n16 + e] = (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
    }
  }
  __syncthreads();
  {
    const int n = threadIdx.x >> 2, k16 = (threadIdx.x & 3) * 16;
    if (n0 + n < p.N && k0 + k16 < p.K) {
      u32x4 w = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 16; ++e) w[e >> 2] |= t[k16 + e][n] << (8 * (e & 3));
      *(u32x4*)((uint8_t*)p.c + (long long)(n0 + n) * p.K + k0 + k16) = w;
    }
  }
}

// Row sums over k of int8 / uint8 operands (I8SumArgs), modulo 2^32: one wave
// per row, 16-byte loads.  A byte's value is (byte ^ 0x80) - 128 when signed,
// the byte itself when unsigned, so every row sums unsigned bytes of
// byte ^ flip and subtracts 128 K for a signed row.
__device__ __forceinline__ uint32_t byte_sum(uint32_t w) {
  const uint32_t t = (w & 0x00FF00FFu) + ((w >> 8) & 0x00FF00FFu);
  return (t & 0xFFFFu) + (t >> 16);
}

__device__ __forceinline__ void i8_sums_body(const I8SumArgs& p) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= (long long)p.a_rows + p.b_rows) return;
  const bool is_a = row < p.a_rows;
  const char* src = is_a ? (const char*)p.a + row * p.a_s0 : (const char*)p.b + (row - p.a_rows) * p.b_s0;
  const bool sgn = is_a ? p.a_signed : p.b_signed;
  const uint32_t flip = sgn ? 0x80808080u : 0u;
  uint32_t s = 0;
  const int full = p.K / 16;
  for (int c = lane; c < full; c += 64) {
    const u32x4 w = __builtin_nontemporal_load((const u32x4*)(src + (long long)c * 16));
    s += byte_sum(w[0] ^ flip) + byte_sum(w[1] ^ flip) + byte_sum(w[2] ^ flip) + byte_sum(w[3] ^ flip);
  }
  for (int k = full * 16 + lane; k < p.K; k += 64) s += (uint32_t)(((const uint8_t*)src)[k] ^ (flip & 0xFFu));
  s = __builtin_bit_cast(uint32_t, wave_reduce<OpSumU32>(__builtin_bit_cast(float, s)));
  if (lane == 0) p.out[row] = (int)(s - (sgn ? 128u * (uint32_t)p.K : 0u));
}

// --------------------------------------------- fused weight dequantisation
// W8A16 (dequantize_matmul fused into the GEMM): Y = A . (B * scale[n]) for A
// bf16/fp16 [M,K] (K-contiguous) and B int8 stored as Bt[N,K] (K-contiguous),
// scale per column (ops/suite/perf/dequantize_matmul.py:28-43 followed by
// matmul.py:21-37).  int8 values are exact in bf16/fp16, so A.B accumulates
// exactly as the unfused pair would from exact weights; the scale multiplies
// the fp32 accumulator and the result rounds once at the store.
//   * workgroup tile 128 x 128, 4 waves (2 x 2), wave tile 64 x 64 = 2 x 2
//     fragments of v_mfma_f32_32x32x16; K in tiles of 64
//   * register-staged: each thread loads its 4 A and 2 B 16-byte vectors of
//     the next K tile while the current one is multiplied, widens the 32 int8
//     weights to 16-bit once (per workgroup, not per wave), and writes both
//     to the other LDS stage (128-byte rows, the main kernel's XOR swizzle, so
//     fragment reads are the main kernel's); one barrier per K tile
//   * B moves as int8: half the weight bytes of the unfused path, which
//     matters where the product is bandwidth-bound (few rows of A)
//   * K must be a multiple of 16 (whole 16-byte B vectors); a K tile past K
//     is zero-filled; M/N edges clamp loads and mask stores
template <bool F16>
__device__ __forceinline__ void gemm_w8a16_body(const GemmArgs& p) {
  constexpr int TM = 128, TN = 128, TK = 64;
  constexpr int ROW = TK * 2;              // LDS row bytes (16-bit elements)
  constexpr int STAGE = (TM + TN) * ROW;   // 32 KiB
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * TM, n0 = tn * TN;
  const long long lda = p.a_s0 * 2, ldb = p.b_s0;  // bytes
  const int kend = p.K;
  const int nk = (p.K + TK - 1) / TK;

  // register staging: A vector i (of 4): row (tid + 256 i) >> 3, chunk & 7;
  // B vector i (of 2): row (tid + 256 i) >> 2, 16-int8 part & 3
  u32x4 ra[4], rb[2];
  auto load = [&](int kt) {
    const int k0 = kt * TK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i, row = v >> 3, ch = v & 7;
      const int k = k0 + ch * 8;
      const char* src = (const char*)p.a + (long long)min(m0 + row, p.M - 1) * lda + (long long)k * 2;
      ra[i] = k < kend ? *(const u32x4*)src : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int v = tid + 256 * i, row = v >> 2, part = v & 3;
      const int k = k0 + part * 16;
      const char* src = (const char*)p.b + (long long)min(n0 + row, p.N - 1) * ldb + k;
      rb[i] = k < kend ? *(const u32x4*)src : (u32x4){0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int stage) {
    char* st = lds + stage * STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i, row = v >> 3, ch = v & 7;
      *(u32x4*)(st + row * ROW + ((ch ^ ((row >> 1) & 7)) << 4)) = ra[i];
    }
    char* sb = st + TM * ROW;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int v = tid + 256 * i, row = v >> 2, part = v & 3;
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // 8 int8 -> 8 16-bit values = one 16-byte chunk
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = rb[i][2 * h + j / 2];
          const int sh = (j & 1) * 16;
          const float lo = (float)(int8_t)((w >> sh) & 0xFFu);
          const float hi = (float)(int8_t)((w >> (sh + 8)) & 0xFFu);
          o[j] = F16 ? (uint32_t)f32_to_f16(lo) | ((uint32_t)f32_to_f16(hi) << 16)
                     : (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
        }
        const int ch = part * 2 + h;
        *(u32x4*)(sb + row * ROW + ((ch ^ ((row >> 1) & 7)) << 4)) = o;
      }
    }
  };

  const int g = lane >> 5, r = lane & 31;
  f32x16 acc[2][2];
  i32x16 unused[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){};
  if (nk > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  int cur = 0;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load(kt + 1);
    const char* st = lds + cur * STAGE;
    const char* sb = st + TM * ROW;
#pragma unroll
    for (int ks = 0; ks < TK / 16; ++ks) {
      const int chunk = ks * 2 + g;
      u32x4 af[2], bf[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int row = wm * 64 + mi * 32 + r;
        af[mi] = *(const u32x4*)(st + row * ROW + ((chunk ^ ((row >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int row = wn * 64 + ni * 32 + r;
        bf[ni] = *(const u32x4*)(sb + row * ROW + ((chunk ^ ((row >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          mfma_step<F16 ? GEMM_F16 : GEMM_BF16>(bf[ni], af[mi], acc[mi][ni], unused[mi][ni]);
    }
    if (kt + 1 < nk) store(cur ^ 1);
    __syncthreads();
    cur ^= 1;
  }
  const int wm0 = m0 + wm * 64, wn0 = n0 + wn * 64;
  // scale the accumulator by its column's scale (lane layout of gemm_epilogue)
#pragma unroll
  for (int ni = 0; ni < 2; ++ni)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = wn0 + ni * 32 + q * 8 + g * 4 + e;
        const float sc = n < p.N ? load_as_f32(p.bscale, n, p.bscale_dtype) : 0.0f;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) acc[mi][ni][q * 4 + e] *= sc;
      }
  gemm_epilogue<F16 ? GEMM_F16 : GEMM_BF16, 2, 2>(p, acc, unused, wm0, wn0, lane);
}

// -------------------------------------- W8A16 for few rows of A (decode)
// M <= 64: the 128-row tile would multiply mostly padding and stage 128 A
// rows per K tile, so a decode-shaped product streams B instead.  A
// workgroup of 8 waves owns 32 columns (two 16-column tiles) and the whole
// K: wave w sums K range w of 8, and the waves' partial tiles are added in
// wave order through LDS (no workspace, no second launch, no workgroup
// waits on another, the same result every run).  A holds R groups of 16 rows
// (R = 1, 2, 4: M <= 16, 32, 64); each widened B operand feeds all R groups.
// Each wave multiplies with v_mfma_f32_16x16x32 (the A rows on the A port,
// B columns widened from int8 on the B port).  Per 64-element K step, lane
// (g = lane/16, i = lane%16) loads 16 contiguous int8 of column n0 + 16t + i
// at k + 16g (64-byte runs per column) and the 32 bytes of A row 16r + i at
// the same k: its first 8 k feed one MFMA, the next 8 a second one (the two
// MFMAs' k sets interleave, which leaves each dot product unchanged).
// SKINNY_STEPS / R steps are in flight per wave, each reloaded with the next
// batch's step once its MFMAs have issued.
constexpr int SKINNY_STEPS = 8;   // 64-element K steps loaded together (R = 1)
constexpr int SKINNY_WAVES = 8;   // K ranges (waves) per workgroup
constexpr int SKINNY_TILES = 2;   // 16-column tiles per workgroup

template <bool F16>
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
}

// 16 int8 -> 16 exact 16-bit floats, as two 8-element operands (k 0..7, 8..15)
template <bool F16>
__device__ __forceinline__ void widen_i8x16(const u32x4& w, u32x4& lo, u32x4& hi) {
  uint32_t o[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int x = (int)w[d];
    const float f0 = (float)((x << 24) >> 24), f1 = (float)((x << 16) >> 24);
    const float f2 = (float)((x << 8) >> 24), f3 = (float)(x >> 24);
    if constexpr (F16) {
      o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f0, f1}, f16x2));
      o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f2, f3}, f16x2));
    } else {
      o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f0, f1}, bf16x2));
      o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f2, f3}, bf16x2));
    }
  }
  lo = (u32x4){o[0], o[1], o[2], o[3]};
  hi = (u32x4){o[4], o[5], o[6], o[7]};
}

// Exact copy of an int8 weight matrix Bt[N, K] (row stride b_s0 bytes, K a
// multiple of 16) into a contiguous bf16 / f16 Bt[N, K] at p.c: one thread per
// 16 int8 values, one 16-byte load and two 16-byte stores.  Every int8 value
// is representable in both formats, so the copy loses nothing.
template <bool F16>
__device__ __forceinline__ void widen_i8_body(const GemmArgs& p) {
  const long long chunks = p.K / 16;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)p.N * chunks) return;
  const long long n = i / chunks, c = i - n * chunks;
  const u32x4 w = *(const u32x4*)((const char*)p.b + n * p.b_s0 + c * 16);
  u32x4 lo, hi;
  widen_i8x16<F16>(w, lo, hi);
  u32x4* dst = (u32x4*)((char*)p.c + (n * p.K + c * 16) * 2);
  dst[0] = lo;
  dst[1] = hi;
}

// T: 16-column tiles per workgroup (SKINNY_TILES, or 1 for the 16-column form)
template <bool F16, int R, int T = SKINNY_TILES>
__device__ __forceinline__ void gemm_w8a16_skinny_body(const GemmArgs& p) {
  constexpr int STEPS = SKINNY_STEPS / R;
  __shared__ f32x4 part[SKINNY_WAVES][R][T][64];
  if (blockDim.x != SKINNY_WAVES * 64) return;  // launch shape must match the kernel
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int i = lane & 15;
  const int n0 = blockIdx.x * 16 * T;
  const int kw = (p.K + SKINNY_WAVES * 64 - 1) / (SKINNY_WAVES * 64) * 64;  // K range of one wave
  const int kb = wave * kw;
  const int ke = min(p.K, kb + kw);
  // rows past M repeat row M-1 and columns past N repeat column N-1: their
  // outputs are never stored
  const char* arow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) arow[r] = (const char*)p.a + (long long)min(16 * r + i, p.M - 1) * p.a_s0 * 2;
  const char* bcol[T];
#pragma unroll
  for (int t = 0; t < T; ++t) bcol[t] = (const char*)p.b + (long long)min(n0 + 16 * t + i, p.N - 1) * p.b_s0;
  f32x4 acc[R][T];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[r][t] = (f32x4){};
  // Weights use plain (cacheable) loads: an instruction reads 64 bytes of
  // each of its 16 columns, so every 128-byte line is requested in two halves
  // by consecutive steps, and with nontemporal loads the line was fetched
  // again for its second half (rocprofv3 FETCH_SIZE 1.20x the algorithmic
  // bytes at 16 x 8192 x 8192; 16 x 8192 x 8192 25.4 -> 23.0 us and
  // 32 x 8192 x 8192 32.8 -> 30.0 us with six rotating input sets).
  // STEPS 64-element K steps in flight per wave.  Over whole batches, step st
  // of the next batch is loaded into step st's registers as soon as their
  // MFMAs have issued, so the loads stream without a gap between batches (no
  // per-lane branch around them, so each MFMA waits only for its own
  // step's loads).  A last partial batch loads per lane: a lane whose 16 k
  // lie past the range contributes zeros (K % 16 == 0).
  u32x4 a0[STEPS][R], a1[STEPS][R], bw[STEPS][T];
  auto load = [&](int st, int k0) {
    const int kk = k0 + st * 64 + 16 * g;
#pragma unroll
    for (int t = 0; t < T; ++t) bw[st][t] = *(const u32x4*)(bcol[t] + kk);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      a0[st][r] = *(const u32x4*)(arow[r] + 2 * (long long)kk);
      a1[st][r] = *(const u32x4*)(arow[r] + 2 * (long long)kk + 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the steps' loads in step order
  };
  auto mma = [&](int st) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      u32x4 lo, hi;
      widen_i8x16<F16>(bw[st][t], lo, hi);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        acc[r][t] = mfma16x16x32<F16>(a0[st][r], lo, acc[r][t]);
        acc[r][t] = mfma16x16x32<F16>(a1[st][r], hi, acc[r][t]);
      }
    }
  };
  constexpr int BK = STEPS * 64;
  int k0 = kb;
  const int kwhole = kb + (ke > kb ? (ke - kb) / BK * BK : 0);  // end of the whole batches
  if (k0 < kwhole) {
#pragma unroll
    for (int st = 0; st < STEPS; ++st) load(st, k0);
    for (; k0 + BK < kwhole; k0 += BK) {
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        mma(st);
        load(st, k0 + BK);
      }
    }
#pragma unroll
    for (int st = 0; st < STEPS; ++st) mma(st);
    k0 += BK;
  }
  if (k0 < ke) {
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      if (k0 + st * 64 + 16 * g < ke) {
        load(st, k0);
      } else {
#pragma unroll
        for (int t = 0; t < T; ++t) bw[st][t] = (u32x4){};
#pragma unroll
        for (int r = 0; r < R; ++r) a0[st][r] = a1[st][r] = (u32x4){};
      }
    }
#pragma unroll
    for (int st = 0; st < STEPS; ++st) mma(st);
  }
  // lane (g, i) holds rows 16r + 4g .. +3 of column n0 + 16t + i; wave 0
  // adds the waves' tiles in wave order, scales and stores
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) part[wave][r][t][lane] = acc[r][t];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int n = n0 + 16 * t + i;
    if (n >= p.N) continue;
    const float sc = load_as_f32(p.bscale, n, p.bscale_dtype);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f32x4 sum = part[0][r][t][lane];
#pragma unroll
      for (int w = 1; w < SKINNY_WAVES; ++w) sum += part[w][r][t][lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = 16 * r + 4 * g + j;
        if (m < p.M) store_from_f32(p.c, (long long)m * p.c_s0 + n, p.c_dtype, sum[j] * sc);
      }
    }
  }
}

// ------------------------------------------------------------ general GEMM
// 64x64 output tile, 256 threads, each 4x4 outputs; K in steps of 16 staged
// through LDS with bounds-checked element loads (zero fill past the edges).
template <bool INT8>
__device__ __forceinline__ void gemm_general_body(const GemmArgs& p) {
  __shared__ float As[16][64 + 1];
  __shared__ float Bs[16][64 + 1];
  __shared__ int Ai[16][64 + 1];
  __shared__ int Bi[16][64 + 1];
  const int tid = threadIdx.x;
  const int tm = blockIdx.x / p.tiles_n;
  const int tn = blockIdx.x % p.tiles_n;
  const int m0 = tm * 64, n0 = tn * 64;
  const int tx = tid & 15, ty = tid >> 4;  // 16 x 16 threads, 4x4 each
  float accf[4][4] = {};
  int acci[4][4] = {};
  for (int k0 = 0; k0 < p.K; k0 += 16) {
    for (int e = tid; e < 16 * 64; e += 256) {
      const int kk = e / 64, mm = e % 64;
      const int m = m0 + mm, k = k0 + kk;
      const bool inb = (m < p.M) && (k < p.K);
      const long long ia = (long long)m * p.a_s0 + (long long)k * p.a_s1;
      if (INT8) Ai[kk][mm] = !inb ? 0 : p.a_dtype == DT_UINT8 ? (int)((const uint8_t*)p.a)[ia]
                                                             : (int)((const int8_t*)p.a)[ia];
      else As[kk][mm] = inb ? load_as_f32(p.a, ia, p.a_dtype) : 0.0f;
      const int n = n0 + mm;
      const bool inbb = (n < p.N) && (k < p.K);
      const long long ib = (long long)k * p.b_s0 + (long long)n * p.b_s1;
      if (INT8) Bi[kk][mm] = !inbb ? 0 : p.b_dtype == DT_UINT8 ? (int)((const uint8_t*)p.b)[ib]
                                                               : (int)((const int8_t*)p.b)[ib];
      else if (p.b_dtype == DT_INT8) Bs[kk][mm] = inbb ? (float)((const int8_t*)p.b)[ib] : 0.0f;
      else Bs[kk][mm] = inbb ? load_as_f32(p.b, ib, p.b_dtype) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (INT8) acci[i][j] = (int)((uint32_t)acci[i][j] + (uint32_t)(Ai[kk][ty * 4 + i] * Bi[kk][tx * 4 + j]));
          else accf[i][j] = fmaf(As[kk][ty * 4 + i], Bs[kk][tx * 4 + j], accf[i][j]);
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= p.N) continue;
      float v;
      if (INT8) {
        if (p.acc_out) p.acc_out[(long long)m * p.acc_s0 + n] = acci[i][j];
        if (!p.sa) continue;
        v = ((float)acci[i][j] * p.sa[m]) * p.sb[n];
      } else {
        v = accf[i][j];
        if (p.bscale) v *= load_as_f32(p.bscale, n, p.bscale_dtype);
      }
      store_from_f32(p.c, (long long)m * p.c_s0 + (long long)n * p.c_s1, p.c_dtype, v);
    }
  }
}

}  // namespace g950

#define G950_GEMM_MFMA(NAME, MODE, WM, WN, UMASK, KT)                                        \
  extern "C" __global__ __launch_bounds__(WM * WN * 64) void NAME(const g950::GemmArgs p) {  \
    g950::gemm_mfma_body<MODE, WM, WN, UMASK, KT>(p);                                      \
  }
// row-major B [K, N] read directly (M, N >= 256, whole 64-k slabs; host checks)
#define G950_GEMM_MFMA_RB(NAME, MODE)                                                       \
  extern "C" __global__ __launch_bounds__(512) void NAME(const g950::GemmArgs p) {         \
    __shared__ __attribute__((aligned(1024))) char lds[4 * g950::BM * g950::SLAB];        \
    g950::gemm_mfma16_body<MODE, 4, 2, 0, true>(p, lds);                                   \
  }
G950_GEMM_MFMA_RB(g950_gemm_bf16_256x256_rb, g950::GEMM_BF16)
G950_GEMM_MFMA_RB(g950_gemm_f16_256x256_rb, g950::GEMM_F16)
G950_GEMM_MFMA(g950_gemm_bf16_256x256, g950::GEMM_BF16, 4, 2, 0, false)
G950_GEMM_MFMA(g950_gemm_f16_256x256, g950::GEMM_F16, 4, 2, 0, false)
G950_GEMM_MFMA(g950_gemm_i8_256x256, g950::GEMM_I8, 4, 2, 0, false)
// K not a whole 128-byte slab (16-byte rows): the last slab's tail reads zeros
G950_GEMM_MFMA(g950_gemm_bf16_256x256_kt, g950::GEMM_BF16, 4, 2, 0, true)
G950_GEMM_MFMA(g950_gemm_f16_256x256_kt, g950::GEMM_F16, 4, 2, 0, true)
G950_GEMM_MFMA(g950_gemm_i8_256x256_kt, g950::GEMM_I8, 4, 2, 0, true)
extern "C" __global__ __launch_bounds__(256) void g950_transpose_b16(const g950::GemmArgs p) {
  g950::transpose16_body(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_transpose_b32(const g950::GemmArgs p) {
  g950::transpose32_body(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_transpose_b8(const g950::GemmArgs p) {
  g950::transpose8_body(p);
}
// fp32 on v_mfma_f32_32x32x2_f32 (the matmul corpus's base dtype)
G950_GEMM_MFMA(g950_gemm_f32_256x256, g950::GEMM_F32, 4, 2, 0, false)
G950_GEMM_MFMA(g950_gemm_f32_256x256_kt, g950::GEMM_F32, 4, 2, 0, true)
// int8 signedness variants of the reference family (a100c/plan/tiles.py:121-126):
// uint8 A x int8 B, int8 A x uint8 B, uint8 x uint8
G950_GEMM_MFMA(g950_gemm_u8s8_256x256, g950::GEMM_I8, 4, 2, 1, false)
G950_GEMM_MFMA(g950_gemm_s8u8_256x256, g950::GEMM_I8, 4, 2, 2, false)
G950_GEMM_MFMA(g950_gemm_u8u8_256x256, g950::GEMM_I8, 4, 2, 3, false)
extern "C" __global__ __launch_bounds__(256) void g950_i8_sums(const g950::I8SumArgs p) {
  g950::i8_sums_body(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_gemm_w8a16_bf16_128x128(const g950::GemmArgs p) {
  g950::gemm_w8a16_body<false>(p);
}
// W8A16 decode: up to 16, 32 and 64 rows of A
#define G950_W8A16_SKINNY(NAME, F16, R, T)                                                 \
  extern "C" __global__ __launch_bounds__(512) void NAME(const g950::GemmArgs p) {        \
    g950::gemm_w8a16_skinny_body<F16, R, T>(p);                                            \
  }
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny_bf16, false, 1, 2)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny_f16, true, 1, 2)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny32_bf16, false, 2, 2)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny32_f16, true, 2, 2)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny64_bf16, false, 4, 2)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny64_f16, true, 4, 2)
// 16 columns per workgroup: twice the workgroups, for grids the 32-column
// form leaves short of the CUs and for a one-row A (whose loads cost little)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny_c16_bf16, false, 1, 1)
G950_W8A16_SKINNY(g950_gemm_w8a16_skinny_c16_f16, true, 1, 1)
extern "C" __global__ __launch_bounds__(256) void g950_gemm_w8a16_f16_128x128(const g950::GemmArgs p) {
  g950::gemm_w8a16_body<true>(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_gemm_general(const g950::GemmArgs p) {
  g950::gemm_general_body<false>(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_gemm_general_i8(const g950::GemmArgs p) {
  g950::gemm_general_body<true>(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_widen_i8_bf16(const g950::GemmArgs p) {
  g950::widen_i8_body<false>(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_widen_i8_f16(const g950::GemmArgs p) {
  g950::widen_i8_body<true>(p);
}
