// Kernel argument blocks shared by the gfx950 kernels and the host launcher.
// Each kernel takes exactly one of these structs by value; the launcher fills
// it after validating the operator contract.  Plain C layout only.
#pragma once

namespace g950 {

struct RowArgs {
  const void* x;
  void* y;
  const void* w;      // RMSNorm / LayerNorm weight (same dtype as x)
  const void* b;      // LayerNorm bias
  void* stat0;        // RMSNorm r / LayerNorm Mean
  void* stat1;        // LayerNorm Rstd
  long long x_row;    // row strides in elements
  long long y_row;
  long long stat0_stride;
  long long stat1_stride;
  int rows;
  int cols;
  float eps;
  int stat_dtype;     // dtype code of stat0/stat1
  void* part;         // split rows: [rows * splits] partial records of 4 floats
  int splits;         // split rows: chunks per row
};

struct GemmArgs {
  const void* a;      // fast: [M,K] K-contiguous; general: element strides below
  const void* b;      // fast: Bt[N,K] K-contiguous
  void* c;            // output [M,N]
  const float* sa;    // int8 dequant: per-row A scale (may be null -> no dequant output)
  const float* sb;    // per-column B scale
  int* acc_out;       // int8: optional int32 accumulator output [M,N]
  long long a_s0, a_s1;   // element strides of A along (m, k)
  long long b_s0, b_s1;   // element strides of B along (k, n)
  long long c_s0, c_s1;   // element strides of C along (m, n)
  long long acc_s0;       // row stride of acc_out
  int M, N, K;
  int tiles_m, tiles_n;
  int a_dtype, b_dtype, c_dtype;
  const void* bscale; // fused weight dequantisation: per-column scale of an int8 B
  int bscale_dtype;   //   (float dtype code), applied to the fp32 accumulator
  const void* cscale; // bf16/f16 MFMA GEMM: optional per-column output scale
  int cscale_dtype;   //   (float dtype code), applied in the epilogue
  // int8 MFMA GEMM with an unsigned operand: the kernel multiplies u - 128
  // (the byte XOR 0x80, a signed int8) and adds back, modulo 2^32,
  //   128 * rsum[m] (B unsigned) + 128 * csum[n] (A unsigned) - 16384 * K (both)
  // where rsum / csum are the int32 sums over k of A's rows / B's columns
  const int* rsum;
  const int* csum;
};

// Sums over k of int8 / uint8 rows (A[m, :] and Bt[n, :], K-contiguous):
// out[0 .. a_rows) for A, out[a_rows .. a_rows + b_rows) for B, modulo 2^32.
struct I8SumArgs {
  const void* a;
  const void* b;
  int* out;
  long long a_s0, b_s0;  // row strides in bytes
  int a_rows, b_rows;    // 0: that operand's sums are not needed
  int a_signed, b_signed;
  int K;
};

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;  // may be null
  long long q_sz, q_sh, q_ss;  // element strides (z, h, s); d stride is 1
  long long k_sz, k_sh, k_ss;
  long long v_sz, v_sh, v_ss;
  long long o_sz, o_sh, o_ss;
  long long lse_sz, lse_sh, lse_ss;
  int Z, Hq, Hkv, Sq, Sk;
  float scale_log2;  // scale * log2(e)
  int causal;
  int nqb;           // query blocks
  int group;         // query heads per KV head: KV head of query head h is h / group
};

struct CopyArgs {
  const void* x;
  void* y;
  long long n16;  // 16-byte vectors
};

struct DequantArgs {
  const void* b;      // int8 [k, n]
  const void* scale;  // [n], same dtype as y
  void* y;            // [k, n]
  long long b_sk, b_sn;  // element strides
  long long y_sk, y_sn;
  long long s_sn;
  long long k, n;
  long long work;     // vector kernel: row groups x column vectors
  int y_dtype;
};

struct AttnGenArgs {
  AttnArgs a;
  int D;
  int dtype;
  int kv_vec;  // fp32 K/V reachable as 16-byte vectors: base 16-byte aligned,
               // every z / head / row stride a multiple of 4 elements
};

// Variable-length attention (flash_varlen_fwd_kernel): per-batch sequences.
// With it, AttnArgs' *_ss are the row strides, *_sh the head strides, *_sz
// unused; Z is the batch count, Sq / Sk the fixed lengths of the non-cu modes.
// Values read from device memory (cu_seqlens, seqused_k, page table) are
// checked against the extents below before they address anything.
struct VarlenArgs {
  const int* cu_q;          // [b + 1] query row starts, or null (fixed seqlen_q)
  const int* cu_k;          // [b + 1] key row starts, or null (fixed seqlen_k)
  const int* used_k;        // [b] keys used per batch, or null
  const int* page_table;    // [b * pt_stride] physical page per key page, or null
  long long pt_stride;      // page_table_batch_stride
  long long pt_elems;       // entries of the page-table view
  long long page_stride;    // k_page_stride (elements)
  long long q_bs, k_bs, v_bs, o_bs;  // batch strides of the fixed-length modes
  long long q_rows, k_rows; // rows the q/o and k/v views hold (cu modes)
  long long pages;          // physical pages the k/v views hold (paged mode)
  int total_q;              // lse head stride
  int block_size;           // keys per page
  int tile_pages;           // block_size is a multiple of the 64-key tile
  int local;                // is_local
  int wl, wr;               // window_size_left / window_size_right
};

struct AttnVarArgs {
  AttnArgs a;
  VarlenArgs v;
  int D;       // general kernel: head dim
  int dtype;   // general kernel: q/k/v/o dtype
};

}  // namespace g950
