// Measurement-only code object: the attention kernels with s_memtime stamps
// at the phase boundaries of the main loop (loop top, after the barrier,
// after the K/V DMA issue, after the first-half softmax, after the MFMA
// phase, after the lead waves' softmax), for the first 64 key tiles of ONE
// workgroup (blockIdx.x == G950_ATT_STAMP_WG).  That workgroup writes its
// stamps over its own output rows (wave w: 64 x 6 little-endian uint64 at
// the start of its 32 rows of O) instead of storing O; every other
// workgroup runs the product kernel unchanged.  compiler_amd/probes.py
// loads this code object in place of the product one for one launch and
// turns the stamps into a per-phase cycle table.  Not used by any operator.
#define G950_ATT_STAMP 1
#define G950_ATT_STAMP_WG 1000
#define G950_ATT_STAMP_DECL __shared__ unsigned long long att_stamps[NW][64][6];
#define G950_ATT_STAMP(t, e)                                                 \
  do {                                                                       \
    if ((t) < 64) {                                                          \
      const unsigned long long st_v = __builtin_amdgcn_s_memtime();          \
      if (lane == 0) att_stamps[wave][(t)][(e)] = st_v;                      \
    }                                                                        \
  } while (0)
#define G950_ATT_STAMP_OUT                                                   \
  if (blockIdx.x == G950_ATT_STAMP_WG) {                                     \
    __syncthreads();                                                         \
    unsigned long long* st_dst = (unsigned long long*)((char*)p.o +          \
        2 * (o_off + (long long)h * p.o_sh + (long long)qw * p.o_ss));       \
    const unsigned long long* st_src = &att_stamps[wave][0][0];              \
    for (int st_i = lane; st_i < 64 * 6; st_i += 64) st_dst[st_i] = st_src[st_i]; \
    return;                                                                  \
  }
#include "attention.hip"
