// Internal launch interfaces shared by the kernel files and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "elsa_hip.h"

namespace elsa {


struct BiasView {
  const void* ptr;
  int dtype;
  int64_t sb, sh, sq, sk;
};

// One Phase-1 launch covers query rows [q_start, q_start + q_len) of every head
// and all K partitions.  Summaries are written to
//   m[(kb * BH + bh) * rows_pad + r], z[...], s[((kb * BH + bh) * rows_pad + r) * D + d]
// with r = row - q_start.
struct Phase1Params {
  const void* q;
  const void* k;
  const void* v;
  BiasView bias;
  float* m_buf;
  float* z_buf;
  void* s_buf;
  int s_dtype;
  int H, N, D, BH;
  int q_start, q_len;
  int part_len, P;
  int causal;
  float scale_log2;  // log2(e) / sqrt(D_model)
  float bias_log2;   // log2(e)
  // q rounded to the input dtype after scaling by scale_log2, so the scores come out of the
  // QK^T product in the base-2 domain (the reference's fp16 d64 fold without bias or
  // causal mask, attention_parallel_scan.py:257-259); otherwise fp32 scores are scaled
  int prescale_q;
  // exact_max == 0: the row state may keep the lazy reference (at most kLazyTau below the row
  // maximum, z relative to it) instead of the maximum; the fold then forms each stage's row
  // maximum only where its partial sums show a score past the reference + kLazyTau
  int exact_max;
  int64_t rows_pad;
  // direct != 0 (only with P == 1): apply Phase 2's finalize in the epilogue and write
  // out (the input dtype, layout os) and the row state instead of the summary
  int direct;
  void* out;
  float* row_m;
  float* row_z;
  // element strides (batch, head, row) of q, k, v and out; the head dim is contiguous
  int64_t qs[3], ks[3], vs[3], os[3];
  // causal split (launch1h): the 4-wave fold skips the pairs of 512-row block R and partition
  // kb that lie wholly below the diagonal (causal_full_row0), which a ping-pong launch folds
  int skip_full;
};

// Causal split of a whole-sequence causal Phase 1: partition kb's keys all precede the rows of
// 512-row block R (a pair the fold needs no mask for) from R = causal_full_row0(kb, part_len) on.
__host__ __device__ inline int causal_full_row0(int kb, int part_len) {
  return (int)(((int64_t)(kb + 1) * part_len + 511) / 512);
}
// Such pairs per (batch, head): sum over the partitions of the 512-row blocks from that row on.
__host__ __device__ inline int causal_full_pairs(int n, int P, int part_len) {
  const int nrb = (n + 511) / 512;
  int cnt = 0;
  for (int kb = 0; kb < P; ++kb) cnt += max(0, nrb - causal_full_row0(kb, part_len));
  return cnt;
}

struct Phase2Params {
  const float* m_buf;
  const float* z_buf;
  const void* s_buf;
  int s_dtype;
  void* out;
  int out_dtype;
  float* row_m;
  float* row_z;
  int N, D, BH;
  int q_start, q_len;
  int part_len, P;
  int causal;
  int64_t rows_pad;
  int H;
  int64_t os[3];  // element strides (batch, head, row) of out
};

// Launch helpers (return hipError_t of the launch).
hipError_t launch_phase1(const Phase1Params& p, int dtype, int block_m, hipStream_t stream);
hipError_t launch_phase2(const Phase2Params& p, hipStream_t stream);
int phase1_key_tile(int dtype, int head_dim_padded);
// rows per Phase-1 workgroup for a sequence of n query rows over bh (batch, head) pairs
int phase1_block_m(int dtype, int head_dim_padded, int64_t n, int64_t bh, bool causal, bool bias);
int pad_head_dim(int d);

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  const float* row_m;
  const float* row_z;
  void* dq;
  void* dk;
  void* dv;
  BiasView bias;
  float* d_row;    // [BH, N]
  float* lse_row;  // [BH, N]: LSE2 rounded to fp32
  float* lse_lo;   // [BH, N]: LSE2 - lse_row (fp32 kernels subtract both: p is exact to fp32 rounding)
  // biased dk/dv kernels: when set, also store dS = p * (dP - D) in fp32, [BH, N, N]
  float* ds_out;
  int H, N, D, BH;
  int causal;
  float scale;       // 1/sqrt(D_model)
  float scale_log2;  // scale * log2(e)
  // element strides (batch, head, row) of q, k, v, out, dout and of dq, dk, dv
  int64_t qs[3], ks[3], vs[3], os[3], gs[3], dqs[3], dks[3], dvs[3];
  // split > 1 (bwd_splits): the 4-wave dq and dK/dV kernels cut their key (dq) or row (dK/dV)
  // loop into `split` ranges of split_len (a multiple of 64; of 32 for fp32) over grid z, and write unscaled fp32
  // partials, [split][BH][N][dp] each for dq, dK and dV from part on; a combine kernel sums them
  int split, split_len, dp;
  float* part;
  int64_t part_stride;  // floats from the dq partials to the dK ones and from those to the dV ones
};

// Ranges the backward (fp16, bf16 and fp32) cuts its loops into when its unsplit grid (128 rows or
// keys per work-group) leaves the chip under-filled: doubled from 1 while the doubled grid stays
// within 512 work-groups (causal fp32: 512 that hold work) and n / (2 * split) is at least 256 (64
// for fp32).  Each range is
// split_len = ceil(n / split) rounded up to whole stages (64 rows; 32 for fp32), so the last one can be shorter
// (B1 H4 N2049: 576, 576, 576 and 321 rows) or start past n (B1 H2 N2049: 8 ranges of 320, the last
// from 2240); the launch lasts as long as the longest range,
// which no choice of whole-stage ranges makes shorter.  Biased calls and head dims above 64 keep 1.
int bwd_splits(int dtype, int dp, int64_t bh, int64_t n, bool bias, bool causal);

// stage < 0: preprocess, dq and dk/dv; 0: preprocess only; 1: dq only; 2: dk/dv only.
hipError_t launch_bwd(const BwdParams& p, int dtype, int stage, hipStream_t stream);
hipError_t launch_row_stats(const BwdParams& p, float* row_m, float* row_z, int dtype, hipStream_t stream);
// Number of ranges the dbias reduction over broadcast (b, h) pairs is cut into (1 = direct).
int dbias_splits(int N, int batch, int heads, int bias_batch, int bias_heads);
// part: nsplit * bias_batch * bias_heads * N * N floats of scratch when nsplit > 1.
hipError_t launch_dbias(const BwdParams& p, float* dbias, int bias_batch, int bias_heads, int dtype, int nsplit,
                        float* part, hipStream_t stream);
hipError_t launch_debug_mfma(int variant, const void* a, const void* b, float* d, hipStream_t stream);
hipError_t launch_debug_mfma_rate(int variant, const void* src, float* out, int iters, int workgroups,
                                  hipStream_t stream);
// dbias[bb', hb'] = sum over the (b, h) pairs broadcast onto it of ds[b, h], in a fixed order;
// with part (dbias_sum_splits * bias_batch * bias_heads * N * N floats) the pairs are summed in
// ranges across workgroups and the ranges added in order.
int dbias_sum_splits(int B, int H, int bias_batch, int bias_heads);
hipError_t launch_dbias_sum(const float* ds, float* dbias, int B, int H, int N, int bias_batch, int bias_heads,
                            float* part, hipStream_t stream);
// n floats of zeros (a kernel, so that graph capture records no memset node)
hipError_t launch_zero_fill(float* dst, int64_t n, hipStream_t stream);

}  // namespace elsa
