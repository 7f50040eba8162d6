/*
 * elsa_hip.h -- C ABI of libelsa_hip.so, the MI355X (gfx950) implementation of
 * ELSA two-pass exact monoid-scan attention.
 *
 * Conventions
 *   - Every tensor is caller-allocated device memory, row-major and contiguous:
 *     q, k, v, out, dout, dq, dk, dv are [B, H, N, D]; row state and the
 *     backward's D/LSE2 rows are [B*H, N] fp32.  The library never allocates
 *     device memory (callers size `workspace` with the *_plan / *_workspace_bytes
 *     queries), so every entry point may be recorded into a hipGraph.
 *   - Kernels are enqueued on `stream` (a hipStream_t passed as void*; NULL is
 *     the default stream).  Calls return after enqueueing.
 *   - Return 0 (ELSA_OK) or a negative elsa_status.  Nothing is thrown across
 *     the ABI.  elsa_last_error() gives a thread-local message for the last
 *     failing call on the calling thread.
 *   - Row state is in the base-2 domain: row_m = max_k(s*log2(e)),
 *     row_z = sum_k exp2(s*log2(e) - row_m) with s = q.k/sqrt(D) (+ bias);
 *     rows without any valid key have row_m = -inf, row_z = 0 and out = 0.
 *   - The library is stateless and re-entrant.
 *
 * Reference interfaces replaced (paths under the reference's
 * src/elsa_twopass_clean/):
 *   elsa_fwd         the forward orchestrators _twopass_attention_d64_parallel_final
 *                    (attention_parallel_scan.py:443-584),
 *                    twopass_attention_blelloch_final_scan (:762-961) and
 *                    twopass_attention_hillis_steele_scan (:587-759).
 *   elsa_phase1      the Phase-1 launches of the 5 Triton summary kernels
 *                    (attention_parallel_scan.py:486-563, :680-708, :881-909;
 *                    attention.py:22-106).
 *   elsa_phase2      the pybind Phase-2 FFI final_reduce(m,z,s,out,row_m,row_z,
 *                    q_start,n_ctx,k_blocks,q_blocks,bh,block_m,store_state)
 *                    (cuda/paper_scan_d64.cpp:18-20, paper_scan_d64_cuda.py:37-67)
 *                    and the Triton up-sweep / Hillis-Steele / finalize launches
 *                    (attention_parallel_scan.py:710-753, :911-955).
 *   elsa_bwd         twopass_attention_backward's launches of the preprocess,
 *                    dq and dk/dv kernels (attention_bwd.py:765-838);
 *                    elsa_bwd_stage issues one of them (:767, :786, :812).
 *   elsa_row_stats   the _row_stats_kernel launch (attention_bwd.py:741-764).
 *   elsa_dbias       the _dbias_dense_kernel launch (attention_bwd.py:926-971).
 */
#ifndef ELSA_HIP_H
#define ELSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ELSA_ABI_VERSION 4

typedef enum elsa_dtype { ELSA_F16 = 0, ELSA_BF16 = 1, ELSA_F32 = 2 } elsa_dtype;

typedef enum elsa_status {
  ELSA_OK = 0,
  ELSA_ERR_INVALID = -1,     /* bad shape, dtype, pointer or option           */
  ELSA_ERR_WORKSPACE = -2,   /* workspace missing or smaller than required     */
  ELSA_ERR_LAUNCH = -3,      /* HIP runtime / kernel launch error              */
  ELSA_ERR_UNSUPPORTED = -4  /* valid request this build does not implement    */
} elsa_status;

/* Optional additive bias on the natural-log scores, broadcast by zero strides
 * (attention.py:120-159).  Strides are in elements. */
typedef struct elsa_bias_desc {
  const void* ptr;      /* NULL: no bias                                       */
  int32_t dtype;        /* elsa_dtype of the bias values                       */
  int32_t _pad;
  int64_t stride_b, stride_h, stride_q, stride_k;
} elsa_bias_desc;

/* Element strides of a [B, H, N, D] operand whose last dimension is contiguous.
 * All zero means the dense layout (H*N*D, N*D, D).  Non-dense layouts let callers hand
 * over views without a copy, e.g. q/k/v sliced out of a fused [B, N, 3, H, D] projection
 * or an output written straight into [B, N, H, D].  Strides must be multiples of 8
 * elements, the row stride at least head_dim and below 2^25, and base pointers 16-byte
 * aligned.
 * Outputs (out; dq, dk, dv) must not alias themselves or each other: their strides are
 * positive. */
typedef struct elsa_layout {
  int64_t batch, head, row;
} elsa_layout;

typedef struct elsa_fwd_args {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* row_m;          /* [B*H, N] or NULL                                   */
  float* row_z;          /* [B*H, N] or NULL (both or neither)                 */
  elsa_bias_desc bias;
  int32_t batch, heads, seq_len, head_dim;
  int32_t dtype;         /* elsa_dtype of q, k, v, out                         */
  int32_t summary_dtype; /* elsa_dtype of the Phase-1 s summaries in HBM       */
  int32_t is_causal;
  int32_t partition_len; /* keys per K partition (block_n); 0 = auto routing   */
  int32_t q_chunk;       /* query rows per Phase1+Phase2 pass; 0 = auto        */
  float scale;           /* softmax scale on q.k; 0 = 1/sqrt(head_dim)          */
  void* workspace;
  size_t workspace_bytes;
  elsa_layout q_layout, k_layout, v_layout, out_layout; /* zero = dense [B,H,N,D]  */
  /* Row state.  1: row_m is each row's maximum base-2 score and row_z the sum of
   * exp2(score - row_m), as twopass_attention_with_state returns them (attention_bwd.py:77-185).
   * 0: row_m may be any reference from that maximum - 8 up to the maximum, with row_z relative
   * to it: the same log-sum-exp row_m + log2(row_z), which is all elsa_bwd reads (the training
   * path).  The fp16/bf16 d64 fold then forms a 64-key stage's row maximum only where the
   * stage's partial sums show a score past the reference + 8. */
  int32_t exact_row_max;
} elsa_fwd_args;

typedef struct elsa_fwd_plan {
  int32_t partitions;    /* P: number of K partitions (Phase-1 summaries/row)  */
  int32_t partition_len; /* keys per partition                                 */
  int32_t q_chunk;       /* query rows per pass                                */
  int32_t block_m;       /* query rows per Phase-1 workgroup                   */
  int32_t key_tile;      /* keys per LDS stage inside a partition              */
  int32_t _pad;
  size_t workspace_bytes;
} elsa_fwd_plan;

typedef struct elsa_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  const float* row_m;    /* [B*H, N] forward row state (required)              */
  const float* row_z;
  void* dq;
  void* dk;
  void* dv;
  elsa_bias_desc bias;
  int32_t batch, heads, seq_len, head_dim;
  int32_t dtype;
  int32_t is_causal;
  float scale;           /* softmax scale on q.k; 0 = 1/sqrt(head_dim)          */
  int32_t _pad;
  void* workspace;       /* elsa_bwd_workspace_bytes: 3*B*H*N floats (D, LSE2 and its low part),
                          * and for short sequences with few heads the fp32 partials of the split
                          * backward (3*split*B*H*N*dp floats, split <= 8).  The size depends on
                          * the shape, dtype, head_dim, is_causal and bias fields: set them first */
  size_t workspace_bytes;
  /* zero = dense [B,H,N,D].  The reference backward reads contiguous copies
   * (attention_bwd.py:722-726); strided views avoid them. */
  elsa_layout q_layout, k_layout, v_layout, out_layout, dout_layout;
  elsa_layout dq_layout, dk_layout, dv_layout;
} elsa_bwd_args;

int elsa_abi_version(void);
const char* elsa_last_error(void);
/* sizeof of the argument structs as compiled into the library (ABI check). */
size_t elsa_struct_size(int which); /* 0 fwd_args, 1 fwd_plan, 2 bwd_args, 3 bias_desc, 4 layout */

/* Tiling, partition routing and workspace size for a forward call. */
int elsa_fwd_plan_get(const elsa_fwd_args* args, elsa_fwd_plan* plan);
/* Full forward: for each q-chunk, Phase 1 (summaries -> workspace) then Phase 2. */
int elsa_fwd(const elsa_fwd_args* args, void* stream);
/* elsa_fwd without a caller workspace: the Phase-1 summaries go to a 64 MiB device array built
 * into the library (one per GPU, held until the process ends), so the call allocates nothing.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops).  args->workspace and workspace_bytes
 * are ignored; out and the row state are written exactly as elsa_fwd writes them (the same
 * partitions, q-chunked to fit the array).  A call whose single query row needs more than
 * 64 MiB of summaries (partitions x B*H x (8 + head_dim * summary bytes)) returns
 * ELSA_ERR_WORKSPACE.  `stream` must belong to the current device.  All calls on one GPU share
 * its array: calls that overlap on one GPU race (keep them on one stream).  A device's first call
 * resolves the array's address (hipGetSymbolAddress): make one eager call on the device before
 * capturing this entry point into a graph. */
int elsa_fwd_noalloc(const elsa_fwd_args* args, void* stream);
/* The two passes separately, for rows [q_start, q_start+q_len) (q_len <= plan.q_chunk). */
int elsa_phase1(const elsa_fwd_args* args, int32_t q_start, int32_t q_len, void* stream);
int elsa_phase2(const elsa_fwd_args* args, int32_t q_start, int32_t q_len, void* stream);

size_t elsa_bwd_workspace_bytes(const elsa_bwd_args* args);
/* dq, dk, dv from the saved row state (exact recompute of p). */
int elsa_bwd(const elsa_bwd_args* args, void* stream);
/* One stage of elsa_bwd: 0 = D/LSE2 preprocess (into the workspace), 1 = dq kernel,
 * 2 = dk/dv kernel (stages 1 and 2 read what stage 0 wrote); -1 = all three. */
int elsa_bwd_stage(const elsa_bwd_args* args, int32_t stage, void* stream);
/* Recompute the base-2 row state (row_m, row_z) from q, k (and bias). Uses
 * args->q, k, bias, shape fields; writes row_m/row_z [B*H, N]. */
int elsa_row_stats(const elsa_bwd_args* args, float* row_m, float* row_z, void* stream);
/* Workspace for elsa_dbias: elsa_bwd_workspace_bytes plus room for the partial sums of a
 * reduction split over the broadcast (b, h) pairs.  No counterpart in the reference (its
 * dbias kernel loops over the broadcast dims in one program per tile,
 * attention_bwd.py:529-624); like elsa_bwd_workspace_bytes it lets the caller allocate. */
size_t elsa_dbias_workspace_bytes(const elsa_bwd_args* args, int32_t bias_batch, int32_t bias_heads);
/* dbias[b', h', i, j] = sum over broadcast (b, h) of p*(dp - D), fp32 output of
 * shape [bias_batch, bias_heads, N, N] (bias_batch in {1,B}, bias_heads in {1,H}).
 * Needs args->row_m/row_z and the bias descriptor.  With a workspace of
 * elsa_dbias_workspace_bytes the reduction is split across work-groups and summed in a
 * fixed order (deterministic); with only elsa_bwd_workspace_bytes it runs unsplit. */
int elsa_dbias(const elsa_bwd_args* args, float* dbias, int32_t bias_batch, int32_t bias_heads,
               void* stream);

/* dq, dk, dv and dbias in one call: the dk/dv kernel stores dS = p*(dP - D) (fp32), which is
 * dbias itself when the bias broadcasts over nothing and is otherwise summed over the
 * broadcast (b, h) pairs in a fixed order.  Replaces elsa_bwd followed by elsa_dbias (the
 * reference's backward launches and its _dbias_dense_kernel, attention_bwd.py:765-838 and
 * :926-971), whose dbias kernel recomputes S and dP.  The dS buffer is limited to 1 GiB
 * (B*H*N*N floats); past that the call runs elsa_bwd and elsa_dbias.  No counterpart in the
 * reference as a single call. */
size_t elsa_bwd_dbias_workspace_bytes(const elsa_bwd_args* args, int32_t bias_batch, int32_t bias_heads);
int elsa_bwd_dbias(const elsa_bwd_args* args, float* dbias, int32_t bias_batch, int32_t bias_heads,
                   void* stream);

/* Device check of the MFMA operand/result layout: variant 0 fp16, 1 bf16, 2 fp32.
 * a, b: [64 lanes][KP] operand elements; d: [64 lanes][16] floats. */
int elsa_debug_mfma(int32_t variant, const void* a, const void* b, float* d, void* stream);

/* Measurement probe (no counterpart in the reference): the sustained matrix-core rate on the
 * operand values in src, which decide the power drawn and so the clock the part holds.
 * variant 0 fp16 / 1 bf16 (v_mfma_f32_32x32x16, 32768 flop each), 2 fp32 (v_mfma_f32_32x32x2_f32,
 * 4096 flop).  src: [16][256][KP] elements (KP = 8 for 16-bit types, 1 for fp32); out:
 * workgroups * 256 floats.  One launch runs workgroups * 4 waves * iters * 8 MFMAs.
 * iters in [1, 1e6], workgroups in [1, 65536], iters x workgroups at most 2^26 (one launch stays within
 * tens of milliseconds). */
int elsa_debug_mfma_rate(int32_t variant, const void* src, float* out, int32_t iters, int32_t workgroups,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ELSA_HIP_H */
