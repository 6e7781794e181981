// Flash-style attention forward on gfx950 (bf16 / fp16 in, fp32 softmax).
//
// Operator semantics: ops/suite/perf/attn_fwd_causal.py:20-55 (scores
// q.k*scale, causal mask key <= query, softmax, P.V); GQA head map
// h_kv = h // GROUP (ops/suite/dev/gqa.py:29; GROUP = Hq/Hkv for the
// attention contracts, the kernel's own constexpr for gqa_kernel); online softmax over key
// tiles (gqa.py:43-58); per-row logsumexp of the scaled scores,
// lse = rowmax + log(rowsum), +inf for an empty row
// (ops/suite/dev/flash_varlen_fwd_kernel.py:309, :318-320).
//
// Mapping (one workgroup = one (z, q-head) and 256 queries, 8 waves x 32):
//   * S^T = K . Q^T with v_mfma_f32_32x32x16: the K tile (LDS) feeds the A
//     port, the wave's Q fragment (registers, loaded once) the B port.  Each
//     lane then holds 16 scores of ONE query (lane%32) per 32-key block, so
//     the running max / sum of the online softmax are per-lane scalars; the
//     two half-waves holding the same query exchange their maxima only on a
//     tile where some lane's exceeds the running reference.
//   * O^T = V^T . P^T: the A port takes V^T straight from the row-major V
//     tile through ds_read_b64_tr_b16 (gfx950's transposing LDS read: in each
//     16-lane group, output lane i, slot k = element i%4 of the 8 bytes read
//     by lane 4k + i/4; lane j therefore reads V[key0 + j/4][d0 + 4(j%4)..+3]
//     and receives V[key0..key0+3][d0 + i]).  The lane's own probabilities,
//     packed to 16 bits in register order, feed the B port -- P never leaves
//     registers.  The O^T accumulator holds one query per lane, so the online
//     rescale is a per-lane scalar multiply.
//   * exp2 domain: scores are scaled by scale*log2(e) inside the exponent's
//     fma and exponentiated with v_exp_f32; lse returns to natural log at the
//     end.  The reference max of a row is only moved when the tile max exceeds
//     it by more than 8 (p <= 2^8, exact because l and O share the reference);
//     the O rescale is skipped when no row of the wave moved.
//   * K and V tiles (64 keys) are filled by direct global->LDS DMA
//     (global_load_lds_dwordx4) into two-slot K and V rings (64 KiB at
//     d = 128): K two tiles ahead (K of tile t is dead once S^T of tile t is
//     formed, an iteration before P.V of tile t), V one tile ahead.  Tile
//     layouts make every MFMA operand read a per-lane base plus a compile-time
//     offset, bank-conflict free:  K as [16-d slab][key][32 B] with the two
//     16-byte halves swapped on odd (key>>3); V as [32-d block][key][64 B], so
//     the four rows a transposing read touches form one contiguous 256 B run.
//   * ping-pong: waves w and w+4 share a SIMD.  Per key tile, the MFMA phase
//     (P.V of tile t and S^T of tile t+1, 32 MFMAs at d = 128, operand reads
//     software-pipelined two V groups / eight K fragments ahead) of one wave
//     runs while the other wave of the pair runs its softmax; waves 0-3 take
//     the MFMA phase first, waves 4-7 the softmax, then the roles swap.  The
//     MFMA phase runs at raised wave priority so its issue slots come first.
//   * causal: a q-block stops at its diagonal tile, waves skip key tiles that
//     lie wholly above their queries, and the mask is applied only on tiles
//     crossing the diagonal.  Q-blocks are issued longest-first, and the Hq/Hkv
//     query heads sharing a KV head are placed on the same XCD so the shared
//     K/V tiles hit in that XCD's L2.
#include "g950_common.h"

#include <utility>

namespace g950 {

constexpr int ATT_BK = 64;     // keys per tile
constexpr int ATT_KSLOTS = 2;  // K tiles in LDS: the one in use and the one in flight
constexpr int ATT_VSLOTS = 2;  // V tiles in LDS: the one in use, the one in flight

template <int D, int NW>
struct AttnCfg {
  static constexpr int NT = NW * 64;              // threads per workgroup
  static constexpr int BQ = NW * 32;              // queries per workgroup
  static constexpr int ROW = D * 2;               // tile row bytes (K and V)
  static constexpr int CHUNKS = D / 8;            // 16-byte chunks per row
  static constexpr int TILE = ATT_BK * ROW;       // one K or V tile
  static constexpr int LDS = (ATT_KSLOTS + ATT_VSLOTS) * TILE;  // K ring, then V ring
  static constexpr int DMAS = TILE / 1024;        // wave-instructions per tile
  static constexpr int DBLK = D / 32;
  static constexpr int DSTEPS = D / 16;
};


// two fp32 -> one packed 16-bit pair (a in the low half): one
// v_cvt_pk_bf16_f32 / v_cvt_pkrtz-free f16 conversion
__device__ __forceinline__ uint32_t pack2(float a, float b, bool f16) {
  if (f16) return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
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

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Eight ds_read_b64_tr_b16 of the V tile (transposed across each 16-lane
// group) at `base` + compile-time offsets, followed by their completion wait.
// Written as one asm block because the compiler, unable to see the address of
// a transposing read, would otherwise wait for every outstanding
// global->LDS DMA before it -- the in-flight prefetch of the next tile; the
// ring's own vmcnt wait + barrier already order these reads after the DMA
// that filled this tile.
template <int O0, int O1, int O2, int O3>
__device__ __forceinline__ void read_tr4(uint32_t base, u32x2 (&v)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4 offset:%5\n\t"
      "ds_read_b64_tr_b16 %1, %4 offset:%6\n\t"
      "ds_read_b64_tr_b16 %2, %4 offset:%7\n\t"
      "ds_read_b64_tr_b16 %3, %4 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(base), "i"(O0), "i"(O1), "i"(O2), "i"(O3)
      : "memory");
}
template <int O0, int O1, int O2, int O3, int O4, int O5, int O6, int O7>
__device__ __forceinline__ void read_tr8(uint32_t base, u32x2 (&v)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%9\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%10\n\t"
      "ds_read_b64_tr_b16 %2, %8 offset:%11\n\t"
      "ds_read_b64_tr_b16 %3, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %4, %8 offset:%13\n\t"
      "ds_read_b64_tr_b16 %5, %8 offset:%14\n\t"
      "ds_read_b64_tr_b16 %6, %8 offset:%15\n\t"
      "ds_read_b64_tr_b16 %7, %8 offset:%16\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7])
      : "v"(base), "i"(O0), "i"(O1), "i"(O2), "i"(O3), "i"(O4), "i"(O5), "i"(O6), "i"(O7)
      : "memory");
}

// compile-time loop: f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS reads issued without a completion wait, for software pipelining.
// lds_wait<N> completes every LDS read of the wave but the newest N (LDS
// reads return in order; any other outstanding LDS or scalar operation only
// makes the wait longer) and names the destination registers as in/out
// operands, so no use of them can be scheduled before the wait and the
// registers stay reserved while their data is in flight.
template <int OFF>
__device__ __forceinline__ void lds_rd128(u32x4& d, uint32_t a) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(a), "n"(OFF) : "memory");
}
template <int OFF>
__device__ __forceinline__ void lds_rdtr(u32x2& d, uint32_t a) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(d) : "v"(a), "n"(OFF) : "memory");
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& d) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(d) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x2 (&v)[8]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
               : "n"(N)
               : "memory");
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x2 (&v)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "n"(N) : "memory");
}

// Maximum of one tile's 32 scores (per lane) with v_max3_f32 (vmax3): four
// independent chains of eight, then their maximum -- 18 instructions where
// fmaxf's per-operand canonicalisation of the MFMA results made ~55.  The
// scores are MFMA results of finite inputs or the -inf of a mask.
__device__ __forceinline__ float tile_max(const f32x16* s) {
  float c[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const f32x16& t = s[h >> 1];
    const int o = (h & 1) * 8;
    float m = vmax3(t[o], t[o + 1], t[o + 2]);
    m = vmax3(m, t[o + 3], t[o + 4]);
    m = vmax3(m, t[o + 5], t[o + 6]);
    c[h] = vmax3(m, t[o + 7], t[o + 7]);
  }
  return vmax3(vmax3(c[0], c[1], c[2]), c[3], c[3]);
}

// Rows of sequence z of a variable-length batch (flash_varlen_fwd_kernel.py:
// 24-52): cu_seqlens row starts or fixed lengths with batch strides, and
// seqused_k overriding the key count; paged K/V carries no key offset (the
// page table addresses the keys, :99-117).  Device-held values that would
// address outside the views make the sequence empty (no rows, no keys).
struct SeqGeom {
  long long q_off, k_off, v_off, o_off, lse_off;  // elements
  int q_len, k_len;
};

__device__ __forceinline__ SeqGeom varlen_geom(const AttnArgs& p, const VarlenArgs& vl, int z) {
  SeqGeom g;
  if (vl.cu_q) {
    const int b0 = vl.cu_q[z], b1 = vl.cu_q[z + 1];
    g.q_len = b1 - b0;
    if (b0 < 0 || g.q_len < 0 || (long long)b1 > vl.q_rows || b1 > vl.total_q) g.q_len = 0;
    g.q_off = (long long)b0 * p.q_ss;
    g.o_off = (long long)b0 * p.o_ss;
    g.lse_off = b0;
  } else {
    g.q_len = p.Sq;
    g.q_off = z * vl.q_bs;
    g.o_off = z * vl.o_bs;
    g.lse_off = (long long)z * p.Sq;
  }
  int kcache, kbos = 0;
  if (vl.cu_k) {
    kbos = vl.cu_k[z];
    kcache = vl.cu_k[z + 1] - kbos;
    g.k_off = (long long)kbos * p.k_ss;
    g.v_off = (long long)kbos * p.v_ss;
  } else {
    kcache = p.Sk;
    g.k_off = z * vl.k_bs;
    g.v_off = z * vl.v_bs;
  }
  g.k_len = vl.used_k ? vl.used_k[z] : kcache;
  if (vl.page_table) {
    g.k_off = g.v_off = 0;
    if (g.k_len < 0) g.k_len = 0;
  } else if (vl.cu_k ? (kbos < 0 || g.k_len < 0 || (long long)kbos + g.k_len > vl.k_rows)
                     : (g.k_len < 0 || g.k_len > p.Sk)) {
    g.k_len = 0;
  }
  return g;
}

// Offset (elements, past the head offset) of key j's row in K (and, with
// pages, in V): the page table entry of its page with K's page and row
// strides for both (flash_varlen_fwd_kernel.py:101-104); entries outside the
// table or the pool read page 0.
__device__ __forceinline__ long long paged_row(const VarlenArgs& vl, int z, int j, long long row_stride) {
  const long long e = (long long)z * vl.pt_stride + j / vl.block_size;
  int ph = e < vl.pt_elems ? vl.page_table[e] : 0;
  if (ph < 0 || ph >= vl.pages) ph = 0;
  return (long long)ph * vl.page_stride + (long long)(j % vl.block_size) * row_stride;
}

// NW waves x 32 queries of one (z, q-head); key tiles of 64 in two-slot K and
// V rings.  Iteration t: wait for this wave's DMA of K(t+1) and V(t);
// barrier; DMA of K(t+2) and V(t+1); then, in the order of the wave's half
// of the ping-pong, the softmax of tile t and the MFMA phase (O^T += V^T.P^T
// of tile t, S^T of tile t+1), or the MFMA phase and the softmax of tile t+1.
// PG (varlen only): how K/V rows are found -- 0 contiguous rows (no page
// table), 1 pages holding whole 64-key tiles (one page-table read per tile),
// 2 any page size (a page-table read per DMA lane).  A compile-time choice:
// the unused paths cost the contiguous kernel 10% when they were run-time
// branches inside the DMA loop (4 x 4096 tokens, 32/8 heads, d 128: 595 ->
// 538 us; the fixed-shape kernel takes 516 us on the same tensors).
template <int D, bool F16, int NW, bool VL, int PG = 0>
__device__ __forceinline__ void attn_body(const AttnArgs& p, const VarlenArgs* vl) {
  using C = AttnCfg<D, NW>;
  __shared__ __attribute__((aligned(1024))) char lds[C::LDS];
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
  const int G = p.group;
  if (p.Hq == p.Hkv * G && (per_qb % (8 * G)) == 0) {
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

  // ---- sequence geometry: element offsets of this (z, head)'s rows, lengths,
  // and the key window of query row i: keys <= i + hi_off (has_hi) and
  // >= i + lo_off (has_lo).  Fixed-length attention: causal is key <= query.
  const int q0 = qb * C::BQ;
  long long q_off, k_off, v_off, o_off, lse_off;
  int Sq = p.Sq, Sk = p.Sk;
  bool has_hi = p.causal, has_lo = false;
  int hi_off = 0, lo_off = 0;
  if constexpr (VL) {
    const SeqGeom sg = varlen_geom(p, *vl, z);
    q_off = sg.q_off; k_off = sg.k_off; v_off = sg.v_off; o_off = sg.o_off; lse_off = sg.lse_off;
    Sq = sg.q_len;
    Sk = sg.k_len;
    if (q0 >= Sq) return;  // whole workgroup past this sequence's queries
    has_hi = p.causal || vl->local;
    has_lo = vl->local;
    hi_off = Sk - Sq + vl->wr;
    lo_off = Sk - Sq - vl->wl;
  } else {
    q_off = (long long)z * p.q_sz;
    k_off = (long long)z * p.k_sz;
    v_off = (long long)z * p.v_sz;
    o_off = (long long)z * p.o_sz;
    lse_off = (long long)z * p.lse_sz;
  }
  const char* qbase = (const char*)p.q + 2 * (q_off + (long long)h * p.q_sh);
  const char* kbase = (const char*)p.k + 2 * (k_off + (long long)hk * p.k_sh);
  const char* vbase = (const char*)p.v + 2 * (v_off + (long long)hk * p.v_sh);

  const int qw = q0 + wave * 32;  // first query of this wave
  const int my_q = qw + r;        // this lane's query
  const int q_last_block = min(q0 + C::BQ, Sq) - 1;

  // ---- Q fragment (B port of S^T = K.Q^T): lane holds Q[my_q][16*ks + 8*g .. +8]
  u32x4 qf[C::DSTEPS];
  {
    const int qrow = min(my_q, Sq - 1);
    const char* src = qbase + 2 * (long long)qrow * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < C::DSTEPS; ++ks) qf[ks] = *(const u32x4*)(src + (ks * 16 + g * 8) * 2);
  }

  int kend = Sk;
  if (has_hi) kend = min(kend, q_last_block + hi_off + 1);
  // first key tile: 0, or the left window edge of the block's first query
  const int kbeg = has_lo ? (max(0, q0 + lo_off) / ATT_BK) * ATT_BK : 0;
  const int ntiles = kend > kbeg ? (kend - kbeg + ATT_BK - 1) / ATT_BK : 0;

  // ---- DMA of one K+V tile: wave-instruction d (0..2*DMAS-1) fills 1 KiB,
  // dealt round-robin over the first NL = NW/2 waves only: those are the
  // waves that start an iteration in the MFMA phase, so the DMA issue stalls
  // land in front of MFMA work while the other half of each SIMD pair starts
  // its softmax straight after the barrier (1.2% over dealing the DMA to all
  // NW waves; dealing it to the softmax half instead loses 7%).  K
  // instruction d = (slab ks, key half kh): 32 keys x 32 B; V instruction
  // (block b, key quarter kq): 16 keys x 64 B.  Per-lane tile-relative source
  // offsets are computed once: instruction u of a DMA wave is a K instruction
  // for u < DPW / 2, a V one after.  Interior tiles then cost one 64-bit add
  // per instruction; only a tile that runs past Sk clamps key indices.
  constexpr int NL = NW / 2;
  constexpr int DPW = 2 * C::DMAS / NL;
  static_assert(C::DMAS % NL == 0, "DMA deal");
  const int dwave = wave % NL;
  const long long kstride = 2 * (long long)p.k_ss, vstride = 2 * (long long)p.v_ss;
  int dkey[DPW], dcol[DPW];
#pragma unroll
  for (int u = 0; u < DPW; ++u) {
    const int d = dwave + u * NL;
    if (u < DPW / 2) {
      const int ks = d >> 1, key = (d & 1) * 32 + (lane >> 1);
      dkey[u] = key;
      dcol[u] = ks * 32 + (((lane & 1) ^ ((key >> 3) & 1)) * 16);
    } else {
      const int dv = d - C::DMAS;
      dkey[u] = (dv & 3) * 16 + (lane >> 2);
      dcol[u] = (dv >> 2) * 64 + (lane & 3) * 16;
    }
  }
  // Pages of a multiple of 64 keys hold whole tiles: one uniform page-table
  // read per tile, issued one DMA round ahead so its latency is hidden.
  constexpr bool tile_pages = VL && PG == 1;
  auto tile_page = [&](int t) -> long long {
    if (!tile_pages || t >= ntiles) return 0;
    const long long e = (long long)z * vl->pt_stride + (kbeg + t * ATT_BK) / vl->block_size;
    int ph = e < vl->pt_elems ? vl->page_table[e] : 0;
    if (ph < 0 || ph >= vl->pages) ph = 0;
    return (long long)ph * vl->page_stride * 2 - (long long)((kbeg + t * ATT_BK) / vl->block_size) *
                                                     vl->block_size * kstride;
  };
  // K tiles and V tiles are each issued in increasing order, so each keeps
  // its next page shift prefetched
  long long kpage_next = tile_page(0), vpage_next = kpage_next;
  // DMA of the K half (instructions u < DPW / 2) or the V half of tile t into
  // its ring slot; waves NL.. issue none
  auto dma_part = [&](bool kpart, int t) {
    if (wave >= NL) return;
    char* slot = kpart ? lds + (t % ATT_KSLOTS) * C::TILE : lds + (ATT_KSLOTS - 1 + t % ATT_VSLOTS) * C::TILE;
    const int kv0 = kbeg + t * ATT_BK;
    const bool tail = kv0 + ATT_BK > Sk;
    long long page_shift = 0;
    if constexpr (VL) {
      if (tile_pages) {
        long long& next = kpart ? kpage_next : vpage_next;
        page_shift = next;
        next = tile_page(t + 1);
      }
    }
#pragma unroll
    for (int u = 0; u < DPW; ++u) {
      const bool is_k = u < DPW / 2;
      if (is_k != kpart) continue;
      const char* base = is_k ? kbase : vbase;
      const long long stride = is_k ? kstride : vstride;
      const int key = tail ? min(kv0 + dkey[u], Sk - 1) : kv0 + dkey[u];
      const char* src = base + key * stride + dcol[u];
      if constexpr (VL) {
        // page rows use K's row stride for K and V (flash_varlen_fwd_kernel.py:101-104)
        if constexpr (PG == 1) src = base + page_shift + key * kstride + dcol[u];
        else if constexpr (PG == 2) src = base + 2 * paged_row(*vl, z, key, p.k_ss) + dcol[u];
      }
      // instruction d = wave + u * NW fills 1 KiB at d * 1024 of the K tile,
      // or (d - DMAS) * 1024 of the V tile (the V slot pointer is pre-shifted)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(slot + (dwave + u * NL) * 1024),
                                       16, 0, 0);
    }
  };
  auto active = [&](int t) {
    const int kv0 = kbeg + t * ATT_BK;
    const int qlast = VL ? min(qw + 31, Sq - 1) : qw + 31;
    if (qw >= Sq || (has_hi && kv0 > qlast + hi_off)) return false;
    return !(has_lo && kv0 + ATT_BK - 1 < qw + lo_off);
  };
  // S^T tile (2 blocks of 32 keys) from the K tile of tile t; lane (g, r)
  // reads 16 B of key kb*32 + r in slab ks at ks*2048 + kb*1024 + k_lane
  const int k_lane = r * 32 + ((g ^ ((r >> 3) & 1)) << 4);
  auto qk = [&](int t, f32x16* s) {
    const char* k_lds = lds + (t % ATT_KSLOTS) * C::TILE + k_lane;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = (f32x16){};
#pragma unroll
      for (int ks = 0; ks < C::DSTEPS; ++ks) {
        const u32x4 kf = *(const u32x4*)(k_lds + ks * 2048 + kb * 1024);
        s[kb] = mfma16<F16>(kf, qf[ks], s[kb]);
      }
    }
  };

  f32x16 oacc[C::DBLK];
#pragma unroll
  for (int b = 0; b < C::DBLK; ++b) oacc[b] = (f32x16){};
  const float c2 = p.scale_log2;
  float ms = -__builtin_huge_valf();  // reference max of the row, scaled (log2 units)
  float l_run[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // this lane's partial row sums (four chains)
  // transposing-read geometry: lane j of 16-lane group (g, half) reads key
  // 4g + j/4 (+ kb*32 + 16tt (+8)), d = 32b + 16*half + 4*(j%4) .. +3
  const int trj = lane & 15;
  const int v_lane = ((lane >> 5) * 4 + (trj >> 2)) * 64 + ((lane >> 4) & 1) * 32 + (trj & 3) * 8;

  // O^T += V^T . P^T for tile t (P packed in registers), reads completed per
  // group; the edge tiles' counterpart of mma_phase
  auto pv = [&](int t, const u32x4 (&pf)[2][2]) {
    const char* v_lds = lds + (ATT_KSLOTS + t % ATT_VSLOTS) * C::TILE;
    const uint32_t vb = lds_addr(v_lds) + v_lane;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        u32x2 vt[8];
        // offsets: 32-d block b at b*4096, key row (kb*32 + 16tt [+8]) * 64
        if constexpr (C::DBLK == 4) {
          if (kb == 0 && tt == 0) read_tr8<0, 512, 4096, 4608, 8192, 8704, 12288, 12800>(vb, vt);
          if (kb == 0 && tt == 1) read_tr8<1024, 1536, 5120, 5632, 9216, 9728, 13312, 13824>(vb, vt);
          if (kb == 1 && tt == 0) read_tr8<2048, 2560, 6144, 6656, 10240, 10752, 14336, 14848>(vb, vt);
          if (kb == 1 && tt == 1) read_tr8<3072, 3584, 7168, 7680, 11264, 11776, 15360, 15872>(vb, vt);
        } else {
          if (kb == 0 && tt == 0) read_tr4<0, 512, 4096, 4608>(vb, vt);
          if (kb == 0 && tt == 1) read_tr4<1024, 1536, 5120, 5632>(vb, vt);
          if (kb == 1 && tt == 0) read_tr4<2048, 2560, 6144, 6656>(vb, vt);
          if (kb == 1 && tt == 1) read_tr4<3072, 3584, 7168, 7680>(vb, vt);
        }
#pragma unroll
        for (int b = 0; b < C::DBLK; ++b) {
          const u32x4 vf = {vt[2 * b][0], vt[2 * b][1], vt[2 * b + 1][0], vt[2 * b + 1][1]};
          oacc[b] = mfma16<F16>(vf, pf[kb][tt], oacc[b]);
        }
      }
  };

  // MFMA phase of iteration t with its operand reads software-pipelined: P.V
  // of tile t (four groups of transposing V reads, DBLK MFMAs each) and S^T
  // of tile t+1 (NK K fragments, one MFMA each).  Two V groups and up to
  // eight K fragments are in flight ahead of the MFMAs that consume them.
  auto mma_phase = [&](int t, f32x16* s, const u32x4 (&pf)[2][2]) {
    constexpr int R = 2 * C::DBLK;     // transposing reads per V group
    constexpr int NK = 2 * C::DSTEPS;  // K fragments of one S^T tile
    const uint32_t vaddr = lds_addr(lds + (ATT_KSLOTS + t % ATT_VSLOTS) * C::TILE) + v_lane;
    const uint32_t kaddr = lds_addr(lds + ((t + 1) % ATT_KSLOTS) * C::TILE + k_lane);
    u32x2 vt[2][R];
    u32x4 kf[8];
    // V group I = (kb, tt) = (I >> 1, I & 1): read Q of group I at 32-d block
    // Q >> 1 (4096 B apart), key rows kb*32 + 16tt + 8(Q & 1) (64 B each)
    auto vread = [&](auto ic) {
      constexpr int I = decltype(ic)::value;
      static_for<R>([&](auto qc) {
        constexpr int Q = decltype(qc)::value;
        lds_rdtr<(Q >> 1) * 4096 + (Q & 1) * 512 + (I >> 1) * 2048 + (I & 1) * 1024>(vt[I & 1][Q], vaddr);
      });
    };
    auto vmma = [&](auto ic) {
      constexpr int I = decltype(ic)::value;
      static_for<C::DBLK>([&](auto bc) {
        constexpr int B = decltype(bc)::value;
        const u32x4 vf = {vt[I & 1][2 * B][0], vt[I & 1][2 * B][1], vt[I & 1][2 * B + 1][0],
                          vt[I & 1][2 * B + 1][1]};
        oacc[B] = mfma16<F16>(vf, pf[I >> 1][I & 1], oacc[B]);
      });
    };
    // K fragment J = (kb, ks) = (J / DSTEPS, J % DSTEPS), as in qk()
    auto kread = [&](auto jc) {
      constexpr int J = decltype(jc)::value;
      if constexpr (J < NK) lds_rd128<(J % C::DSTEPS) * 2048 + (J / C::DSTEPS) * 1024>(kf[J & 7], kaddr);
    };
    auto kmma = [&](auto jc) {
      constexpr int J = decltype(jc)::value;
      constexpr int KB = J / C::DSTEPS, KS = J % C::DSTEPS;
      s[KB] = mfma16<F16>(kf[J & 7], qf[KS], KS == 0 ? (f32x16){} : s[KB]);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    // each wait names how many reads were issued after the group it completes
    vread(I0{});
    vread(I1{});
    lds_wait<R>(vt[0]);
    vmma(I0{});
    vread(I2{});
    lds_wait<R>(vt[1]);
    vmma(I1{});
    vread(I3{});
    lds_wait<R>(vt[0]);
    vmma(I2{});
    static_for<4>([&](auto jc) { kread(jc); });
    lds_wait<4>(vt[1]);
    vmma(I3{});
    static_for<4>([&](auto jc) { kread(std::integral_constant<int, decltype(jc)::value + 4>{}); });
    static_for<NK>([&](auto jc) {
      constexpr int J = decltype(jc)::value;
      constexpr int after = (NK - J - 1) < 7 ? (NK - J - 1) : 7;  // K reads issued after fragment J
      lds_wait<after>(kf[J & 7]);
      kmma(jc);
      kread(std::integral_constant<int, J + 8>{});
    });
  };

  // online softmax of the S^T tile t held in s: mask, running max, O and l
  // rescale, P packed to 16 bits for the B port of P.V
  auto softmax = [&](int t, f32x16* s, u32x4 (&pf)[2][2]) {
    const int kv0 = kbeg + t * ATT_BK;
    const bool need_mask = (has_hi && kv0 + ATT_BK - 1 > qw + hi_off) || (has_lo && kv0 < qw + 31 + lo_off) ||
                           (kv0 + ATT_BK > Sk);
    if (need_mask) {
      // key kv0 + 32kb + 8(vv>>2) + 4g + (vv&3) of this lane's query my_q
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) {
          const int key = kv0 + kb * 32 + 8 * (vv >> 2) + 4 * g + (vv & 3);
          if (key >= Sk || (has_hi && key > my_q + hi_off) || (has_lo && key < my_q + lo_off))
            s[kb][vv] = -__builtin_huge_valf();
        }
    }
    // this half-wave's tile maximum (scale > 0, so scaling commutes with the
    // maximum); the two halves holding a query combine theirs only when some
    // lane's exceeds the reference by more than 8 -- otherwise no row moves
    const float mh = tile_max(s) * c2;
    if (__any(mh > ms + 8.0f)) {
      const float mt = fmaxf(mh, __shfl_xor(mh, 32));
      const bool move = mt > ms + 8.0f;
      const float ms_new = move ? mt : ms;
      // 0 on a row's first keys; 1 on rows that keep their reference (also a
      // row with no visible key yet, ms = -inf, beside rows that moved)
      const float alpha = move ? __builtin_amdgcn_exp2f(ms - ms_new) : 1.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) l_run[j] *= alpha;
#pragma unroll
      for (int b = 0; b < C::DBLK; ++b) oacc[b] *= alpha;
      ms = ms_new;
    }
    // a row whose keys so far are all masked keeps ms = -inf: exponent base 0
    // gives exp2(-inf) = 0 instead of NaN
    const float mb = (ms == -__builtin_huge_valf()) ? 0.0f : ms;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int vv = 0; vv < 16; ++vv) {
        s[kb][vv] = __builtin_amdgcn_exp2f(fmaf(s[kb][vv], c2, -mb));
        l_run[vv & 3] += s[kb][vv];
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pf[kb][tt][e] = pack2(s[kb][8 * tt + 2 * e], s[kb][8 * tt + 2 * e + 1], F16);
    }
  };

  // ---- prologue: DMA of K(0), V(0), K(1); S^T of tile 0
  f32x16 s[2];
  u32x4 pf[2][2];
  if (ntiles > 0) {
    dma_part(true, 0);
    dma_part(false, 0);
  }
  if (ntiles > 1) dma_part(true, 1);
  // K of tile 0 has landed (V of tile 0 and K of tile 1 may be in flight)
  if (ntiles > 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DPW) : "memory");
  else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DPW / 2) : "memory");
  __syncthreads();
  if (ntiles > 0 && active(0)) qk(0, s);
  // waves w and w + NW/2 share a SIMD (waves are dealt round-robin over the
  // four SIMDs) and run opposite halves of the ping-pong
  const bool lead = wave < NW / 2;
  if (lead && ntiles > 0 && active(0)) softmax(0, s, pf);

  // ---- main loop.  Iteration t: K of tile t+1 and V of tile t have landed
  // (this wave's DMAs: vmcnt(0); everyone's: the barrier), and every wave is
  // done with K of tile t (its S^T was formed in iteration t-1) and V of
  // tile t-1, whose slots now take K of tile t+2 and V of tile t+1.
  for (int t = 0; t < ntiles; ++t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 2 < ntiles) dma_part(true, t + 2);
    if (t + 1 < ntiles) dma_part(false, t + 1);
    const bool cur = active(t);
    const bool nxt = t + 1 < ntiles && active(t + 1);
    if (!lead && cur) softmax(t, s, pf);
    if (cur && nxt) {
      __builtin_amdgcn_s_setprio(2);
      mma_phase(t, s, pf);
      __builtin_amdgcn_s_setprio(0);
    } else {
      if (cur) pv(t, pf);
      if (nxt) qk(t + 1, s);
    }
    if (lead && nxt) softmax(t + 1, s, pf);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: O = O / l ; lse = (ms + log2 l) * ln2
  const float l_sum = (l_run[0] + l_run[1]) + (l_run[2] + l_run[3]);
  const float l_tot = l_sum + __shfl_xor(l_sum, 32);
  const bool empty = !(l_tot > 0.0f);  // zero or NaN
  const float inv = empty ? 1.0f : 1.0f / l_tot;
  // 16-byte aligned output rows: the wave's 32 x D output tile passes through
  // its own 32 rows of LDS (the K/V rings are free once every wave has passed
  // the barrier) and leaves as whole rows in 16-byte non-temporal stores.
  // Lane (g, r) holds d = 32 b + 8 q4 + 4 g .. + 3 of query r: 8 bytes of
  // 16-byte chunk 4 b + q4, the chunk index XOR-swizzled by the row.
  // Measured on MI355X against per-lane 8-byte stores, same bits: [4, 32,
  // 4096, 128] causal 534 -> 518 us, [16, 32, 1024, 128] causal 210 -> 186,
  // non-causal 295 -> 268; the staging with write-back stores gained a third
  // of that.  The condition is uniform over the workgroup.
  char* ohead = (char*)p.o + 2 * (o_off + (long long)h * p.o_sh);
  if (((uintptr_t)ohead & 15) == 0 && (p.o_ss & 7) == 0) {
    constexpr int CH = C::CHUNKS, RPI = 64 / CH;  // chunks per row, rows per store
    static_assert(NW * 32 * C::ROW <= C::LDS, "output staging fits the K/V rings");
    __syncthreads();
    char* reg = lds + wave * 32 * C::ROW;
#pragma unroll
    for (int b = 0; b < C::DBLK; ++b)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint16_t hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float val = oacc[b][4 * q4 + e] * inv;
          hv[e] = F16 ? f32_to_f16(val) : f32_to_bf16(val);
        }
        const int chunk = 4 * b + q4;
        *(u32x2*)(reg + r * C::ROW + ((chunk ^ (r & (CH - 1))) << 4) + g * 8) =
            (u32x2){(uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16)};
      }
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
      const int row = it * RPI + lane / CH, c = lane % CH;
      const u32x4 v = *(const u32x4*)(reg + row * C::ROW + ((c ^ (row & (CH - 1))) << 4));
      if (qw + row < Sq)
        __builtin_nontemporal_store(v, (u32x4*)(ohead + 2 * (long long)(qw + row) * p.o_ss + c * 16));
    }
    if (p.lse && g == 0 && my_q < Sq) {
      const float lse = empty ? __builtin_huge_valf() : (ms + __log2f(l_tot)) * 0.69314718055994530942f;
      p.lse[lse_off + (long long)h * p.lse_sh + (long long)my_q * p.lse_ss] = lse;
    }
    return;
  }
  if (my_q < Sq) {
    char* orow = (char*)p.o + 2 * (o_off + (long long)h * p.o_sh + (long long)my_q * p.o_ss);
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
      const float lse = empty ? __builtin_huge_valf() : (ms + __log2f(l_tot)) * 0.69314718055994530942f;
      p.lse[lse_off + (long long)h * p.lse_sh + (long long)my_q * p.lse_ss] = lse;
    }
  }
}

// ------------------------------------------------------------ fp32 MFMA path
// Flash-style attention on v_mfma_f32_32x32x2_f32 for fp32 inputs (and for
// 16-bit inputs the 16-bit kernel does not take: head dim 32, a scale <= 0):
// every score is computed once.  Workgroup = 4 waves x 32 queries of one
// (z, head); key tiles of 64 staged in LDS as fp32 (converted on load, keys
// past Sk as zeros), 129-float rows so the per-key column reads hit distinct
// banks; fp32 tiles are prefetched into registers one tile ahead.  Per wave
// and tile:
//   * S^T = K.Q^T: the K tile (LDS) on the A port, Q (registers, lane half
//     h holding d = 2s + h of its query) on the B port; each lane then holds
//     16 scores of ONE query per 32-key block (keys 8(v/4) + 4h + v%4), so
//     the online softmax state is per lane, the two halves of a query
//     combining their tile maxima with one lane swap;
//   * scores are scaled (log2 units) before the maximum, which holds for any
//     sign of the scale;
//   * O^T += V^T.P^T: step (q, e) of a 32-key block takes key 8q + 4h + e
//     for lane half h -- exactly the keys that half's score registers hold,
//     so P feeds the B port from the score registers in fp32, unrounded.
constexpr int AF_BQ = 128;  // queries per workgroup (4 waves x 32)
constexpr int AF_BK = 64;   // keys per tile

template <int D>
__device__ __forceinline__ void attn_f32_body(const AttnGenArgs& g) {
  const AttnArgs& p = g.a;
  __shared__ float Ks[AF_BK][D + 1];
  __shared__ float Vs[AF_BK][D + 1];
  if (blockDim.x != 256) return;  // launch shape must match the kernel
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, r = lane & 31;
  const int per_qb = p.Z * p.Hq;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / per_qb);  // longest (causal) first
  const int zh = blockIdx.x % per_qb;
  const int z = zh / p.Hq, h = zh % p.Hq, hk = h / p.group;
  const int q0 = qb * AF_BQ;
  const int qw = q0 + wave * 32;
  const int my_q = qw + r;
  const long long qoff = (long long)z * p.q_sz + (long long)h * p.q_sh;
  const long long koff = (long long)z * p.k_sz + (long long)hk * p.k_sh;
  const long long voff = (long long)z * p.v_sz + (long long)hk * p.v_sh;
  float qr[D / 2];
  {
    const long long row = qoff + (long long)min(my_q, p.Sq - 1) * p.q_ss;
#pragma unroll
    for (int s = 0; s < D / 2; ++s) qr[s] = load_as_f32(p.q, row + 2 * s + hh, g.dtype);
  }
  int kend = p.Sk;
  if (p.causal) kend = min(kend, min(q0 + AF_BQ, p.Sq));
  const int ntiles = (kend + AF_BK - 1) / AF_BK;
  f32x16 o[D / 32];
#pragma unroll
  for (int b = 0; b < D / 32; ++b) o[b] = (f32x16){};
  float m = -__builtin_huge_valf(), l = 0.0f;
  // fp32 inputs whose K/V rows are whole aligned 16-byte vectors (the host's
  // kv_vec): the next tile's K and V rows are loaded into registers as
  // 16-byte vectors while the current tile is multiplied, then written to
  // LDS behind the next barrier; vector i of a thread is key (tid + 256 i) /
  // (D / 4), columns 4 * ((tid + 256 i) % (D / 4)) .. +3.  Other inputs are
  // staged element by element between the barriers.
  constexpr int NV = AF_BK * D / 4 / 256;
  const bool f32 = g.dtype == DT_F32 && g.kv_vec;
  const float* kf = (const float*)p.k + koff;
  const float* vf = (const float*)p.v + voff;
  f32x4 kst[NV], vst[NV];
  auto stage_load = [&](int t) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + 256 * i, key = idx / (D / 4), c = 4 * (idx % (D / 4));
      const int j = t * AF_BK + key;
      kst[i] = vst[i] = (f32x4){};
      if (j < p.Sk) {
        kst[i] = *(const f32x4*)(kf + (long long)j * p.k_ss + c);
        vst[i] = *(const f32x4*)(vf + (long long)j * p.v_ss + c);
      }
    }
  };
  if (f32 && ntiles > 0) stage_load(0);
  for (int t = 0; t < ntiles; ++t) {
    const int kv0 = t * AF_BK;
    __syncthreads();  // every wave is done with the previous tile
    if (f32) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int idx = tid + 256 * i, key = idx / (D / 4), c = 4 * (idx % (D / 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          Ks[key][c + e] = kst[i][e];
          Vs[key][c + e] = vst[i][e];
        }
      }
    } else {
      for (int idx = tid; idx < AF_BK * D; idx += 256) {
        const int key = idx / D, d = idx - key * D;
        const int j = kv0 + key;
        const bool in = j < p.Sk;
        Ks[key][d] = in ? load_as_f32(p.k, koff + (long long)j * p.k_ss + d, g.dtype) : 0.0f;
        Vs[key][d] = in ? load_as_f32(p.v, voff + (long long)j * p.v_ss + d, g.dtype) : 0.0f;
      }
    }
    __syncthreads();
    if (f32 && t + 1 < ntiles) stage_load(t + 1);
    // the whole wave past Sq, or (causal) every query of the wave before the tile
    if (qw >= p.Sq || (p.causal && kv0 > qw + 31)) continue;
    f32x16 sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = (f32x16){};
#pragma unroll
      for (int s = 0; s < D / 2; ++s)
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[kb * 32 + r][2 * s + hh], qr[s], sc[kb], 0, 0, 0);
    }
    float tmax = -__builtin_huge_valf();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = kv0 + kb * 32 + 8 * (v >> 2) + 4 * hh + (v & 3);
        float x = sc[kb][v] * p.scale_log2;
        if (key >= p.Sk || (p.causal && key > my_q)) x = -__builtin_huge_valf();
        sc[kb][v] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m, tmax);
    // a query without a visible key so far keeps m = -inf: base 0 gives
    // exp2(-inf) = 0 instead of inf - inf
    const float mb = (m_new == -__builtin_huge_valf()) ? 0.0f : m_new;
    const float alpha = exp2f(m - mb);
    l *= alpha;
#pragma unroll
    for (int b = 0; b < D / 32; ++b) o[b] *= alpha;
    m = m_new;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        sc[kb][v] = exp2f(sc[kb][v] - mb);
        l += sc[kb][v];
      }
#pragma unroll
    for (int b = 0; b < D / 32; ++b)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[kb * 32 + 8 * (v >> 2) + 4 * hh + (v & 3)][32 * b + r],
                                                      sc[kb][v], o[b], 0, 0, 0);
  }
  const float l_tot = l + __shfl_xor(l, 32);
  if (my_q >= p.Sq) return;
  const bool empty = !(l_tot > 0.0f);
  const float inv = empty ? 0.0f : 1.0f / l_tot;
  const long long orow = (long long)z * p.o_sz + (long long)h * p.o_sh + (long long)my_q * p.o_ss;
#pragma unroll
  for (int b = 0; b < D / 32; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v)
      store_from_f32(p.o, orow + 32 * b + 8 * (v >> 2) + 4 * hh + (v & 3), g.dtype, o[b][v] * inv);
  if (p.lse && hh == 0) {
    const float lse = empty ? __builtin_huge_valf() : (m + __log2f(l_tot)) * 0.69314718055994530942f;
    p.lse[(long long)z * p.lse_sz + (long long)h * p.lse_sh + (long long)my_q * p.lse_ss] = lse;
  }
}

// ------------------------------------------------------------- general path
// Any float dtype and head dim the MFMA kernels do not take: one thread per
// query row, two passes over the keys (max, then exp-sum and P.V).


__device__ __forceinline__ void attn_general_body(const AttnGenArgs& g) {
  const AttnArgs& p = g.a;
  const long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)p.Z * p.Hq * p.Sq;
  if (row >= total) return;
  const int qi = row % p.Sq;
  const int h = (row / p.Sq) % p.Hq;
  const int z = row / ((long long)p.Sq * p.Hq);
  const int hk = h / p.group;
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

// Variable-length attention, any float dtype and head dim: one thread per
// query row (grid over batch x heads x seqlen_q rows), two passes over the
// row's key window.
__device__ __forceinline__ void attn_varlen_general_body(const AttnVarArgs& g) {
  const AttnArgs& p = g.a;
  const VarlenArgs& vl = g.v;
  const long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= (long long)p.Z * p.Hq * p.Sq) return;
  const int qi = row % p.Sq;
  const int h = (row / p.Sq) % p.Hq;
  const int z = row / ((long long)p.Sq * p.Hq);
  const SeqGeom sg = varlen_geom(p, vl, z);
  if (qi >= sg.q_len) return;
  const int hk = h / p.group;
  const int dg = sg.k_len - sg.q_len;
  const int jlo = vl.local ? max(0, qi + dg - vl.wl) : 0;
  const int jhi = (p.causal || vl.local) ? min(sg.k_len - 1, qi + dg + vl.wr) : sg.k_len - 1;
  const long long qo = sg.q_off + (long long)h * p.q_sh + (long long)qi * p.q_ss;
  auto krow = [&](int j) {
    return vl.page_table ? paged_row(vl, z, j, p.k_ss) + (long long)hk * p.k_sh
                         : sg.k_off + (long long)hk * p.k_sh + (long long)j * p.k_ss;
  };
  auto vrow = [&](int j) {
    return vl.page_table ? paged_row(vl, z, j, p.k_ss) + (long long)hk * p.v_sh
                         : sg.v_off + (long long)hk * p.v_sh + (long long)j * p.v_ss;
  };
  auto score = [&](int j) {
    const long long kb = krow(j);
    float s = 0.0f;
    for (int d = 0; d < g.D; ++d)
      s = fmaf(load_as_f32(p.q, qo + d, g.dtype), load_as_f32(p.k, kb + d, g.dtype), s);
    return s * p.scale_log2;
  };
  float m = -__builtin_huge_valf();
  for (int j = jlo; j <= jhi; ++j) m = fmaxf(m, score(j));
  const long long oo = sg.o_off + (long long)h * p.o_sh + (long long)qi * p.o_ss;
  float l = 0.0f;
  for (int d = 0; d < g.D; ++d) {
    float acc = 0.0f, ld = 0.0f;
    for (int j = jlo; j <= jhi; ++j) {
      const float w = exp2f(score(j) - m);
      ld += w;
      acc = fmaf(w, load_as_f32(p.v, vrow(j) + d, g.dtype), acc);
    }
    l = ld;
    store_from_f32(p.o, oo + d, g.dtype, (l > 0.0f) ? acc / l : 0.0f);
  }
  if (g.D == 0) {
    for (int j = jlo; j <= jhi; ++j) l += exp2f(score(j) - m);
  }
  const float lse = (l > 0.0f) ? (m + log2f(l)) * 0.69314718055994530942f : __builtin_huge_valf();
  p.lse[sg.lse_off + (long long)h * p.lse_sh + qi] = lse;
}

}  // namespace g950

#define G950_ATTN(NAME, D, F16, NW)                                                     \
  extern "C" __global__ __launch_bounds__(NW * 64) void NAME(const g950::AttnArgs p) {   \
    g950::attn_body<D, F16, NW, false>(p, nullptr);                                    \
  }                                                                                     \
  extern "C" __global__ __launch_bounds__(NW * 64) void NAME##_varlen(const g950::AttnVarArgs p) { \
    g950::attn_body<D, F16, NW, true, 0>(p.a, &p.v);                                   \
  }                                                                                     \
  extern "C" __global__ __launch_bounds__(NW * 64) void NAME##_varlen_pt(const g950::AttnVarArgs p) { \
    g950::attn_body<D, F16, NW, true, 1>(p.a, &p.v);                                   \
  }                                                                                     \
  extern "C" __global__ __launch_bounds__(NW * 64) void NAME##_varlen_pl(const g950::AttnVarArgs p) { \
    g950::attn_body<D, F16, NW, true, 2>(p.a, &p.v);                                   \
  }
// waves per workgroup (32 queries each); the launcher reads the workgroup
// size back from the kernel's launch bounds
#ifndef G950_ATT_WAVES
#define G950_ATT_WAVES 8
#endif
G950_ATTN(g950_attn_fwd_bf16_d128, 128, false, G950_ATT_WAVES)
G950_ATTN(g950_attn_fwd_bf16_d64, 64, false, G950_ATT_WAVES)
G950_ATTN(g950_attn_fwd_f16_d128, 128, true, G950_ATT_WAVES)
G950_ATTN(g950_attn_fwd_f16_d64, 64, true, G950_ATT_WAVES)
extern "C" __global__ __launch_bounds__(64) void g950_attn_fwd_general(const g950::AttnGenArgs p) {
  g950::attn_general_body(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_attn_fwd_f32mfma_d32(const g950::AttnGenArgs p) {
  g950::attn_f32_body<32>(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_attn_fwd_f32mfma_d64(const g950::AttnGenArgs p) {
  g950::attn_f32_body<64>(p);
}
extern "C" __global__ __launch_bounds__(256) void g950_attn_fwd_f32mfma_d128(const g950::AttnGenArgs p) {
  g950::attn_f32_body<128>(p);
}
extern "C" __global__ __launch_bounds__(64) void g950_attn_varlen_general(const g950::AttnVarArgs p) {
  g950::attn_varlen_general_body(p);
}
