// Flash-style attention forward on gfx950 (bf16 / fp16 in, fp32 softmax).
//
// Operator semantics: ops/suite/perf/attn_fwd_causal.py:20-55 (scores
// q.k*scale, causal mask key <= query, softmax, P.V); GQA head map
// h_kv = h // (Hq/Hkv) (ops/suite/dev/gqa.py:29); online softmax over key
// tiles (gqa.py:43-58); per-row logsumexp of the scaled scores,
// lse = rowmax + log(rowsum), +inf for an empty row
// (ops/suite/dev/flash_varlen_fwd_kernel.py:309, :318-320).
//
// Mapping (one workgroup = one (z, q-head) and 256 queries, 8 waves x 32):
//   * S^T = K . Q^T with v_mfma_f32_32x32x16: the K tile (LDS) feeds the A
//     port, the wave's Q fragment (registers, loaded once) the B port.  Each
//     lane then holds 16 scores of ONE query (lane%32) per 32-key block, so
//     the running max / sum of the online softmax are per-lane scalars; the
//     two half-waves holding the same query combine with one cross-lane swap.
//   * O^T = V^T . P^T: V^T (LDS, written transposed from the row-major V tile)
//     feeds the A port and the lane's own probabilities, packed to 16 bits in
//     register order, feed the B port -- P never leaves registers.  The O^T
//     accumulator again holds one query per lane, so the rescale by
//     exp2(m_old - m_new) is a per-lane scalar multiply.
//   * exp2 domain: scores are pre-multiplied by scale*log2(e) and exponentiated
//     with v_exp_f32; lse is converted back to natural log at the end.
//   * K/V tiles of 64 keys are register-staged: the next tile's global loads
//     are issued before the current tile's MFMAs and written to LDS after.
//   * causal: a q-block stops at its diagonal tile, waves skip key tiles that
//     lie wholly above their queries, and the mask is applied only on tiles
//     crossing the diagonal.  Q-blocks are issued longest-first, and the Hq/Hkv
//     query heads sharing a KV head are placed on the same XCD so the shared
//     K/V tiles hit in that XCD's L2.
#include "g950_common.h"

namespace g950 {



constexpr int ATT_BK = 64;    // keys per tile
constexpr int ATT_STAGES = 3; // LDS ring depth (one barrier per key tile)

template <int D, int NW>
struct AttnCfg {
  static constexpr int NT = NW * 64;              // threads per workgroup
  static constexpr int BQ = NW * 32;              // queries per workgroup
  static constexpr int KROW = D * 2;              // K tile row bytes
  static constexpr int KCHUNKS = D / 8;           // 16-byte chunks per K row
  static constexpr int VT_PITCH = ATT_BK + 4;     // V^T row pitch in elements (pad: conflict-free reads)
  static constexpr int K_BYTES = ATT_BK * KROW;
  static constexpr int VT_BYTES = D * VT_PITCH * 2;
  static constexpr int STAGE = K_BYTES + VT_BYTES;
  static constexpr int K_TOTAL = ATT_BK * KCHUNKS;           // 16-B chunks per K tile
  static constexpr int V_TOTAL = (ATT_BK / 2) * (D / 8);     // key-pair x 8-d units per V tile
  static constexpr int K_LOADS = (K_TOTAL + NT - 1) / NT;    // per thread
  static constexpr int V_UNITS = (V_TOTAL + NT - 1) / NT;
  static constexpr int DBLK = D / 32;
  static constexpr int DSTEPS = D / 16;
};

template <int D>
__device__ __forceinline__ int kslot(int key, int chunk) {
  if constexpr (D == 128) return chunk ^ (key & 15);
  else return chunk ^ ((key >> 1) & 7);
}

__device__ __forceinline__ uint32_t pack2(float a, float b, bool f16) {
  if (f16)
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}

template <bool F16>
__device__ __forceinline__ f32x16 mfma16(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// NW waves x 32 queries of one (z, q-head); key tiles of 64 in a 3-stage LDS
// ring.  Iteration j: barrier; stage tile j+2 (already in registers) into LDS;
// issue the global loads of tile j+3; issue the S^T MFMAs of tile j+1; run the
// online softmax of tile j on the VALU while those MFMAs execute; O^T += V^T.P^T
// for tile j.
template <int D, bool F16, int NW>
__device__ __forceinline__ void attn_body(const AttnArgs& p) {
  using C = AttnCfg<D, NW>;
  __shared__ __attribute__((aligned(16))) char lds[ATT_STAGES * C::STAGE];
  if (blockDim.x != C::NT) return;  // launch shape must match the instantiation

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int r = lane & 31;

  // ---- block -> (q-block, z, head): longest q-blocks first; heads sharing a
  // KV head 8 ids apart (same XCD under round-robin dispatch).
  const int per_qb = p.Z * p.Hq;
  const int pid = blockIdx.x;
  const int qb = p.nqb - 1 - pid / per_qb;
  const int i = pid % per_qb;
  int z, h;
  const int G = p.Hq / p.Hkv;
  if ((per_qb % (8 * G)) == 0) {
    const int xcd = i & 7;
    const int j = i >> 3;
    const int zk = xcd + 8 * (j / G);  // (z, kv-head) pair index
    const int hs = j % G;
    z = zk / p.Hkv;
    h = (zk % p.Hkv) * G + hs;
  } else {
    z = i / p.Hq;
    h = i % p.Hq;
  }
  const int hk = h / G;

  const char* qbase = (const char*)p.q + 2 * ((long long)z * p.q_sz + (long long)h * p.q_sh);
  const char* kbase = (const char*)p.k + 2 * ((long long)z * p.k_sz + (long long)hk * p.k_sh);
  const char* vbase = (const char*)p.v + 2 * ((long long)z * p.v_sz + (long long)hk * p.v_sh);

  const int q0 = qb * C::BQ;
  const int qw = q0 + wave * 32;  // first query of this wave
  const int my_q = qw + r;        // this lane's query
  const int q_last_block = min(q0 + C::BQ, p.Sq) - 1;

  // ---- Q fragment (B port of S^T = K.Q^T): lane holds Q[my_q][16*ks + 8*g .. +8]
  u32x4 qf[C::DSTEPS];
  {
    const int qrow = min(my_q, p.Sq - 1);
    const char* src = qbase + 2 * (long long)qrow * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < C::DSTEPS; ++ks) qf[ks] = *(const u32x4*)(src + (ks * 16 + g * 8) * 2);
  }

  int kend = p.Sk;
  if (p.causal) kend = min(kend, q_last_block + 1);
  const int ntiles = (kend + ATT_BK - 1) / ATT_BK;

  // ---- register staging of one tile
  u32x4 kst[C::K_LOADS];
  u32x4 vst[C::V_UNITS][2];
  auto gload = [&](int t) {
    const int kv0 = t * ATT_BK;
#pragma unroll
    for (int u = 0; u < C::K_LOADS; ++u) {
      const int c = tid + u * C::NT;
      if (C::K_TOTAL % C::NT && c >= C::K_TOTAL) break;
      const int key = c / C::KCHUNKS, ch = c % C::KCHUNKS;
      const int gk = min(kv0 + key, p.Sk - 1);
      kst[u] = *(const u32x4*)(kbase + 2 * (long long)gk * p.k_ss + ch * 16);
    }
#pragma unroll
    for (int u = 0; u < C::V_UNITS; ++u) {
      const int c = tid + u * C::NT;
      if (C::V_TOTAL % C::NT && c >= C::V_TOTAL) break;
      const int kp = c % (ATT_BK / 2), dc = c / (ATT_BK / 2);
      const int k0 = min(kv0 + 2 * kp, p.Sk - 1), k1 = min(kv0 + 2 * kp + 1, p.Sk - 1);
      vst[u][0] = *(const u32x4*)(vbase + 2 * (long long)k0 * p.v_ss + dc * 16);
      vst[u][1] = *(const u32x4*)(vbase + 2 * (long long)k1 * p.v_ss + dc * 16);
    }
  };
  auto lstore = [&](int stage) {
    char* k_lds = lds + stage * C::STAGE;
    char* vt_lds = k_lds + C::K_BYTES;
#pragma unroll
    for (int u = 0; u < C::K_LOADS; ++u) {
      const int c = tid + u * C::NT;
      if (C::K_TOTAL % C::NT && c >= C::K_TOTAL) break;
      const int key = c / C::KCHUNKS, ch = c % C::KCHUNKS;
      *(u32x4*)(k_lds + key * C::KROW + (kslot<D>(key, ch) << 4)) = kst[u];
    }
#pragma unroll
    for (int u = 0; u < C::V_UNITS; ++u) {
      const int c = tid + u * C::NT;
      if (C::V_TOTAL % C::NT && c >= C::V_TOTAL) break;
      const int kp = c % (ATT_BK / 2), dc = c / (ATT_BK / 2);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // element pair (2e, 2e+1) of the 8 d-values, for keys 2kp and 2kp+1
        const uint32_t a = vst[u][0][e], b = vst[u][1][e];
        const uint32_t lo = (a & 0xFFFFu) | (b << 16);      // d = 8dc+2e
        const uint32_t hi = (a >> 16) | (b & 0xFFFF0000u);  // d = 8dc+2e+1
        const int d = dc * 8 + 2 * e;
        *(uint32_t*)(vt_lds + (d * C::VT_PITCH + 2 * kp) * 2) = lo;
        *(uint32_t*)(vt_lds + ((d + 1) * C::VT_PITCH + 2 * kp) * 2) = hi;
      }
    }
  };
  auto active = [&](int t) { return !(p.causal && t * ATT_BK > qw + 31) && (qw < p.Sq); };
  // S^T tile (2 blocks of 32 keys) from the K tile in `stage`
  auto qk = [&](int stage, f32x16* s) {
    const char* k_lds = lds + stage * C::STAGE;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = (f32x16){};
      const int key = kb * 32 + r;
#pragma unroll
      for (int ks = 0; ks < C::DSTEPS; ++ks) {
        const u32x4 kf = *(const u32x4*)(k_lds + key * C::KROW + (kslot<D>(key, ks * 2 + g) << 4));
        s[kb] = mfma16<F16>(kf, qf[ks], s[kb]);
      }
    }
  };

  f32x16 oacc[C::DBLK];
#pragma unroll
  for (int b = 0; b < C::DBLK; ++b) oacc[b] = (f32x16){};
  const float c2 = p.scale_log2;
  float m_run = -__builtin_huge_valf();  // running max of the RAW scores
  float l_run = 0.0f;                    // this lane's partial row sum

  // softmax of one S^T tile + O^T += V^T P^T
  auto consume = [&](int t, f32x16* s) {
    const int kv0 = t * ATT_BK;
    const bool need_mask = (p.causal && kv0 + ATT_BK - 1 > qw) || (kv0 + ATT_BK > p.Sk);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) {
          const int key = kv0 + kb * 32 + 8 * (vv >> 2) + 4 * g + (vv & 3);
          if (key >= p.Sk || (p.causal && key > my_q)) s[kb][vv] = -__builtin_huge_valf();
        }
    }
    float mt = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int vv = 2; vv < 16; vv += 2) mt = fmaxf(mt, fmaxf(s[0][vv], s[0][vv + 1]));
#pragma unroll
    for (int vv = 0; vv < 16; vv += 2) mt = fmaxf(mt, fmaxf(s[1][vv], s[1][vv + 1]));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    // rows whose keys so far are all masked keep m = -inf; exponent base 0
    // then gives exp2(-inf) = 0 instead of NaN
    const float mb = (m_new == -__builtin_huge_valf()) ? 0.0f : m_new * c2;
    if (__any(m_new > m_run)) {  // wave-uniform: skip the O rescale when no max moved
      const float alpha = __builtin_amdgcn_exp2f(m_run * c2 - mb);
      l_run *= alpha;
#pragma unroll
      for (int b = 0; b < C::DBLK; ++b) oacc[b] *= alpha;
    }
    m_run = m_new;
    const char* vt_lds = lds + (t % ATT_STAGES) * C::STAGE + C::K_BYTES;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int vv = 0; vv < 16; ++vv) {
        s[kb][vv] = __builtin_amdgcn_exp2f(fmaf(s[kb][vv], c2, -mb));
        l_run += s[kb][vv];
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        u32x4 pf;
#pragma unroll
        for (int e = 0; e < 4; ++e) pf[e] = pack2(s[kb][8 * tt + 2 * e], s[kb][8 * tt + 2 * e + 1], F16);
        const int kcol = kb * 32 + 16 * tt + 4 * g;
#pragma unroll
        for (int b = 0; b < C::DBLK; ++b) {
          const char* row = vt_lds + (b * 32 + r) * C::VT_PITCH * 2;
          const u32x2 lo = *(const u32x2*)(row + kcol * 2);
          const u32x2 hi = *(const u32x2*)(row + (kcol + 8) * 2);
          const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
          oacc[b] = mfma16<F16>(vf, pf, oacc[b]);
        }
      }
    }
  };

  // ---- prologue: tiles 0 and 1 in LDS, tile 2 in registers, S of tile 0
  f32x16 sa[2], sb[2];
  if (ntiles > 0) { gload(0); lstore(0); }
  if (ntiles > 1) { gload(1); lstore(1); }
  __syncthreads();
  if (ntiles > 2) gload(2);
  if (ntiles > 0 && active(0)) qk(0, sa);

  // ---- main loop, unrolled by two so the S buffers alternate without copies
  auto iteration = [&](int t, f32x16* s_cur, f32x16* s_next) {
    __syncthreads();  // every wave is done with tile t-1 (its stage is free)
    if (t + 2 < ntiles) lstore((t + 2) % ATT_STAGES);
    if (t + 3 < ntiles) gload(t + 3);
    if (t + 1 < ntiles && active(t + 1)) qk((t + 1) % ATT_STAGES, s_next);
    if (active(t)) consume(t, s_cur);
  };
  int t = 0;
  for (; t + 1 < ntiles; t += 2) {
    iteration(t, sa, sb);
    iteration(t + 1, sb, sa);
  }
  if (t < ntiles) iteration(t, sa, sb);

  // ---- epilogue: O = O / l ; lse = (m*c2 + log2 l) * ln2
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (my_q < p.Sq) {
    const bool empty = !(l_tot > 0.0f);  // zero or NaN
    const float inv = empty ? 1.0f : 1.0f / l_tot;
    char* orow = (char*)p.o + 2 * ((long long)z * p.o_sz + (long long)h * p.o_sh + (long long)my_q * p.o_ss);
#pragma unroll
    for (int b = 0; b < C::DBLK; ++b)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = b * 32 + 8 * q4 + 4 * g;
        uint16_t hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float val = oacc[b][4 * q4 + e] * inv;
          hv[e] = F16 ? f32_to_f16(val) : f32_to_bf16(val);
        }
        *(u32x2*)(orow + d * 2) = (u32x2){(uint32_t)hv[0] | ((uint32_t)hv[1] << 16),
                                          (uint32_t)hv[2] | ((uint32_t)hv[3] << 16)};
      }
    if (p.lse && g == 0) {
      const float lse = empty ? __builtin_huge_valf()
                              : (m_run * c2 + __log2f(l_tot)) * 0.69314718055994530942f;
      p.lse[(long long)z * p.lse_sz + (long long)h * p.lse_sh + (long long)my_q * p.lse_ss] = lse;
    }
  }
}

// ------------------------------------------------------------- general path
// fp32 (or any float dtype) attention for small problems: one thread per
// query row, two passes over the keys (max, then exp-sum and P.V).


__device__ __forceinline__ void attn_general_body(const AttnGenArgs& g) {
  const AttnArgs& p = g.a;
  const long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)p.Z * p.Hq * p.Sq;
  if (row >= total) return;
  const int qi = row % p.Sq;
  const int h = (row / p.Sq) % p.Hq;
  const int z = row / ((long long)p.Sq * p.Hq);
  const int hk = h / (p.Hq / p.Hkv);
  const long long qo = (long long)z * p.q_sz + (long long)h * p.q_sh + (long long)qi * p.q_ss;
  const long long kb = (long long)z * p.k_sz + (long long)hk * p.k_sh;
  const long long vb = (long long)z * p.v_sz + (long long)hk * p.v_sh;
  const int kend = p.causal ? min(p.Sk, qi + 1) : p.Sk;
  float m = -__builtin_huge_valf();
  for (int j = 0; j < kend; ++j) {
    float s = 0.0f;
    for (int d = 0; d < g.D; ++d)
      s = fmaf(load_as_f32(p.q, qo + d, g.dtype), load_as_f32(p.k, kb + (long long)j * p.k_ss + d, g.dtype), s);
    m = fmaxf(m, s * p.scale_log2);
  }
  const long long oo = (long long)z * p.o_sz + (long long)h * p.o_sh + (long long)qi * p.o_ss;
  float l = 0.0f;
  // one sweep over the keys per output column (small problems only)
  for (int d = 0; d < g.D; ++d) {
    float acc = 0.0f;
    float ld = 0.0f;
    for (int j = 0; j < kend; ++j) {
      float s = 0.0f;
      for (int e = 0; e < g.D; ++e)
        s = fmaf(load_as_f32(p.q, qo + e, g.dtype), load_as_f32(p.k, kb + (long long)j * p.k_ss + e, g.dtype), s);
      const float w = exp2f(s * p.scale_log2 - m);
      ld += w;
      acc = fmaf(w, load_as_f32(p.v, vb + (long long)j * p.v_ss + d, g.dtype), acc);
    }
    l = ld;
    store_from_f32(p.o, oo + d, g.dtype, (l > 0.0f) ? acc / l : 0.0f);
  }
  if (p.lse) {
    const float lse = (l > 0.0f) ? (m + log2f(l)) * 0.69314718055994530942f : __builtin_huge_valf();
    p.lse[(long long)z * p.lse_sz + (long long)h * p.lse_sh + (long long)qi * p.lse_ss] = lse;
  }
}

}  // namespace g950

#define G950_ATTN(NAME, D, F16, NW)                                                     \
  extern "C" __global__ __launch_bounds__(NW * 64) void NAME(const g950::AttnArgs p) {   \
    g950::attn_body<D, F16, NW>(p);                                                    \
  }
// 8 waves = 256 queries per workgroup (the launcher's grid assumes this)
G950_ATTN(g950_attn_fwd_bf16_d128, 128, false, 8)
G950_ATTN(g950_attn_fwd_bf16_d64, 64, false, 8)
G950_ATTN(g950_attn_fwd_f16_d128, 128, true, 8)
G950_ATTN(g950_attn_fwd_f16_d64, 64, true, 8)
extern "C" __global__ __launch_bounds__(64) void g950_attn_fwd_general(const g950::AttnGenArgs p) {
  g950::attn_general_body(p);
}
