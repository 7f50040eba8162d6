// C ABI of libelsa_hip.so: argument validation, partition routing, workspace
// layout and the q-chunk loop.  No device memory is allocated here.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "elsa_hip.h"

#include "elsa_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  return fail(ELSA_ERR_LAUNCH, "%s: %s", where, hipGetErrorString(e));
}

size_t dtype_size(int dt) { return dt == ELSA_F32 ? 4 : 2; }
bool dtype_ok(int dt) { return dt == ELSA_F16 || dt == ELSA_BF16 || dt == ELSA_F32; }
int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
double softmax_scale(float s, int d) { return s > 0.f ? (double)s : 1.0 / std::sqrt((double)d); }

int check_common(int batch, int heads, int n, int d, int dtype, const void* q, const void* k, const void* v) {
  if (batch <= 0 || heads <= 0 || n <= 0 || d <= 0)
    return fail(ELSA_ERR_INVALID, "batch, heads, seq_len and head_dim must be positive (got %d,%d,%d,%d)", batch,
                heads, n, d);
  if (d > 128) return fail(ELSA_ERR_INVALID, "head_dim > 128 is not supported (got %d)", d);
  if (d % 8 != 0) return fail(ELSA_ERR_INVALID, "head_dim must be a multiple of 8 (got %d)", d);
  if (!dtype_ok(dtype)) return fail(ELSA_ERR_INVALID, "unknown dtype %d", dtype);
  if (!q || !k || !v) return fail(ELSA_ERR_INVALID, "q, k and v must be non-null device pointers");
  if ((int64_t)batch * heads > 65535)
    return fail(ELSA_ERR_UNSUPPORTED, "batch*heads > 65535 is not supported (got %lld)", (long long)batch * heads);
  return ELSA_OK;
}

int check_bias(const elsa_bias_desc& b) {
  if (b.ptr == nullptr) return ELSA_OK;
  if (!dtype_ok(b.dtype)) return fail(ELSA_ERR_INVALID, "unknown bias dtype %d", b.dtype);
  return ELSA_OK;
}

elsa::BiasView bias_view(const elsa_bias_desc& b) {
  return elsa::BiasView{b.ptr, b.dtype, b.stride_b, b.stride_h, b.stride_q, b.stride_k};
}

// Phase-1 summaries of P partitions x bh heads x q_chunk rows: m and z (fp32), s (summary dtype)
size_t fwd_workspace_bytes(int64_t parts, int64_t bh, int64_t q_chunk, int64_t d, int sdt) {
  const size_t rows = (size_t)parts * bh * q_chunk;
  return 2 * align256(rows * 4) + align256(rows * d * dtype_size(sdt));
}

// Partition routing for 256 CUs: about 1024 Phase-1 workgroups when the query side alone
// does not provide them, partitions of >= 512 keys (>= 1024 and one round of the chip where
// the ping-pong fold runs), and at least two partitions from 8K keys on so long sequences
// keep the two-pass merge.
int plan_fwd(const elsa_fwd_args* a, elsa_fwd_plan* pl) {
  if (!a || !pl) return fail(ELSA_ERR_INVALID, "null argument");
  int rc = check_common(a->batch, a->heads, a->seq_len, a->head_dim, a->dtype, a->q, a->k, a->v);
  if (rc) return rc;
  if (!dtype_ok(a->summary_dtype)) return fail(ELSA_ERR_INVALID, "unknown summary_dtype %d", a->summary_dtype);
  if ((rc = check_bias(a->bias))) return rc;
  if ((a->row_m == nullptr) != (a->row_z == nullptr))
    return fail(ELSA_ERR_INVALID, "row_m and row_z must be given together");
  if (a->partition_len < 0 || a->q_chunk < 0) return fail(ELSA_ERR_INVALID, "partition_len and q_chunk must be >= 0");

  const int64_t n = a->seq_len, bh = (int64_t)a->batch * a->heads, d = a->head_dim;
  const int dp = elsa::pad_head_dim(a->head_dim);
  const int bm = elsa::phase1_block_m(a->dtype, dp, n, bh, a->is_causal != 0, a->bias.ptr != nullptr);
  const int kt = elsa::phase1_key_tile(a->dtype, dp);
  const size_t row_bytes = 8 + (size_t)d * dtype_size(a->summary_dtype);

  int64_t part;
  if (a->partition_len > 0) {
    part = std::min<int64_t>(a->partition_len, n);
  } else {
    const int64_t q_rows = a->q_chunk > 0 ? std::min<int64_t>(a->q_chunk, n) : n;
    const int64_t q_tiles = bh * cdiv(q_rows, bm);
    // about 1024 Phase-1 workgroups (4 per CU): at B1 H8 d64 fp16 16K, Phase 1 + Phase 2 took
    // 0.594 ms with 2 partitions against 0.605 ms with 4 (2048 workgroups); 64K 9.06 / 9.17 /
    // 9.35 ms with 4 / 8 / 16; the forward at 1K and at ViT's 1025 tokens (B8 H3) stays within
    // 3% from 1 to 8 partitions
    int64_t p = cdiv(1024, q_tiles);
    p = std::min<int64_t>(p, std::max<int64_t>(1, n / 512));
    // fp32: its fold spends 16 times longer per key than fp16's, so short partitions cost little
    // and the grid's fill decides: where the rule above leaves fewer than 256 work-groups,
    // partitions down to 64 keys until about 512.  Forward ms (Phase 1 + Phase 2, d64): B1 H8 1K
    // 0.050 -> 0.029 (2 -> 8 partitions), causal 1K 0.051 -> 0.029, B8 H3 N197 0.024 -> 0.015 (1 ->
    // 3), B1 H8 N512 0.047 -> 0.014 (1 -> 8); B8 H3 N1025 (432 work-groups) keeps 2 partitions
    // (0.086 against 0.089 ms with 3).  The count is capped at ceil(n / 64), not floor(n / 64): a
    // short tail partition costs less than a third 32-key stage in every work-group: B8 H3 N197
    // 0.0154 -> 0.0127 ms (3 -> 4 partitions), B2 H3 N300 0.0149 -> 0.0131, B1 H2 N90 0.0124 ->
    // 0.0112 (1 -> 2)
    // Causal grids, whose work-groups above the diagonal return at once, fill below 512 work-groups
    // too: B2 H8 N1024 causal 0.0515 -> 0.0380 ms (2 -> 4 partitions), B8 H3 N1025 causal 0.0656 ->
    // 0.0644 (2 -> 3); non-causal ones there went both ways (B2 H8 N1024 0.051 -> 0.047, B8 H3 N1025
    // 0.0856 -> 0.0890, B3 H8 N1024 0.083 -> 0.086) and keep the 256 bound.
    if (a->dtype == ELSA_F32 && q_tiles * p < (a->is_causal ? 512 : 256))
      p = std::max<int64_t>(p, std::min<int64_t>(cdiv(512, q_tiles), cdiv(n, 64)));
    // fp16/bf16 grids at d <= 64 from 512 keys under 192 work-groups (a few heads of at most 2K rows):
    // partitions down to 128 keys until about 256 work-groups.  Forward ms (fp16 d64): B1 H8 1K 0.012
    // -> 0.010 (2 -> 4 partitions), N512 0.0099 -> 0.0084 (1 -> 4), causal N1025 0.0139 -> 0.0121
    // (3 -> 5); B8 H3 N1025 (240 work-groups) keeps its two (5: 0.026 against 0.021 ms), and shorter
    // sequences their one fused partition (B8 H3 N197: more measured slower)
    if (a->dtype != ELSA_F32 && dp <= 64 && n >= 512 && q_tiles * p < 192)
      p = std::max<int64_t>(p, std::min<int64_t>(cdiv(256, q_tiles), std::max<int64_t>(1, n / 128)));
    if (n >= 8192) p = std::max<int64_t>(p, 2);
    // causal from 8K keys: partitions of n/4 keys within [2048, 8192].  About half of the
    // causal workgroups have no keys to fold; Phase 1 dispatches the rest longest first.
    // Phase 1 + Phase 2 at B1 H8 d64 fp16 against 1024 / 2048 / 4096 / 8192-key partitions:
    // 8K 0.114 / 0.114 / 0.119 / 0.187 ms, 16K 0.380 / 0.342 / 0.343 / 0.366 ms, 32K 1.518 /
    // 1.344 / 1.227 / 1.199 ms.
    if (a->is_causal && n >= 8192) p = cdiv(n, std::min<int64_t>(8192, std::max<int64_t>(2048, n / 4)));
    p = std::max<int64_t>(p, 1);
    // the ping-pong fold (fp16/bf16 at d = 64 without bias or causal mask, 16-bit summaries; the
    // launcher's condition) runs 512-row work-groups over partitions of at least 1024 keys: B1 H8 4K
    // forward 0.060 -> 0.052 ms (fp16) and 0.060 -> 0.054 ms (bf16) with four of them against eight
    // of 512 (2K keeps four of 512: 0.025 against 0.040 ms with two).  Its partition count minimises
    // rounds x (partition keys + 768): ceil(work-groups / 256 CUs) rounds, each as long as a
    // partition plus a work-group's fixed cost (Q load, summary stores, the two fill phases),
    // which the measurements put near 768 keys; ties keep fewer partitions.  Forward ms (Phase 1 +
    // Phase 2, fp16 d64) against the 1024-workgroup target of 256-row blocks: B1 H8 8K 0.155 ->
    // 0.134 (4 -> 2 partitions), B2 H8 4K 0.097 -> 0.079 (4 -> 2), B4 H8 4K 0.158 -> 0.133 (2 -> 1),
    // B8 H3 N4097 0.155 -> 0.128 (3 -> 1), B1 H4 16K 0.269 -> 0.256 (4 -> 2), B1 H8 N6000 0.129 ->
    // 0.092 (6 -> 2), B1 H8 N12000 0.352 -> 0.323 (3 -> 2); the north star keeps 2.
    const bool pp = !a->is_causal && !a->bias.ptr && a->dtype != ELSA_F32 && dp == 64 && bm == 256 &&
                    !(a->dtype == ELSA_F16 && a->summary_dtype == ELSA_F32);
    if (pp && n >= 4096) {
      const int64_t tiles = bh * cdiv(q_rows, 512);
      const int64_t p_lo = n >= 8192 ? 2 : 1, p_hi = std::max<int64_t>(p_lo, n / 1024);
      int64_t best_cost = -1;
      for (int64_t c = p_lo; c <= p_hi; ++c) {
        const int64_t len = cdiv(cdiv(n, c), kt) * kt;
        const int64_t cost = cdiv(tiles * cdiv(n, len), 256) * (len + 768);
        if (best_cost < 0 || cost < best_cost) {
          best_cost = cost;
          p = c;
        }
      }
    }
    part = cdiv(cdiv(n, p), kt) * kt;
    if (!a->is_causal && !a->bias.ptr && a->dtype != ELSA_F32 && dp == 64 && n >= 4096 && part < 1024) part = 1024;
    if (a->is_causal && p > 1) {  // one partition stays whole: its launch applies the finalize
      // causal partitions hold whole row blocks, which Phase 1's longest-first order needs;
      // the nearest multiple, not the next: a short causal launch has fewer workgroups than
      // the chip holds and lasts as long as its longest one (B1 H8 d64 fp16, Phase 1 + Phase 2
      // with 512 / 768-key partitions: 1025 tokens 0.024 / 0.029 ms, 2048 0.025 / 0.030 ms;
      // 4097 tokens goes the other way, 0.049 / 0.044 ms)
      const int64_t unit = std::max<int64_t>(kt, bm);
      part = std::max<int64_t>(unit, (cdiv(n, p) + unit / 2) / unit * unit);
    }
    part = std::min<int64_t>(part, n);
  }
  const int64_t parts = cdiv(n, part);
  if (parts > 65535) return fail(ELSA_ERR_UNSUPPORTED, "too many K partitions (%lld)", (long long)parts);

  int64_t q_chunk = a->q_chunk > 0 ? std::min<int64_t>(a->q_chunk, n) : n;
  if (a->q_chunk == 0) {
    // keep the summary workspace under 4 GiB by chunking the query rows
    const size_t cap = size_t(4) << 30;
    const size_t per_row = (size_t)parts * bh * row_bytes;
    if (per_row * q_chunk > cap) q_chunk = std::max<int64_t>(bm, (int64_t)(cap / per_row) / bm * bm);
  }
  pl->partitions = (int32_t)parts;
  pl->partition_len = (int32_t)part;
  pl->q_chunk = (int32_t)q_chunk;
  pl->block_m = bm;
  pl->key_tile = kt;
  pl->_pad = 0;
  pl->workspace_bytes = fwd_workspace_bytes(parts, bh, q_chunk, d, a->summary_dtype);
  return ELSA_OK;
}

struct FwdBuffers {
  float* m;
  float* z;
  void* s;
};

FwdBuffers carve(const elsa_fwd_args* a, const elsa_fwd_plan& pl) {
  const size_t rows = (size_t)pl.partitions * a->batch * a->heads * pl.q_chunk;
  char* base = static_cast<char*>(a->workspace);
  FwdBuffers b;
  b.m = reinterpret_cast<float*>(base);
  b.z = reinterpret_cast<float*>(base + align256(rows * 4));
  b.s = base + 2 * align256(rows * 4);
  return b;
}

// Element strides (batch, head, row) of a [B,H,N,D] operand; an all-zero layout is dense.
void resolve_layout(const elsa_layout& l, int H, int N, int D, int64_t out[3]) {
  if (l.batch == 0 && l.head == 0 && l.row == 0) {
    out[0] = (int64_t)H * N * D;
    out[1] = (int64_t)N * D;
    out[2] = D;
  } else {
    out[0] = l.batch;
    out[1] = l.head;
    out[2] = l.row;
  }
}

// which: 1 = Phase 1 (summaries), 2 = Phase 2, 3 = Phase 1 with Phase 2's finalize fused
// into its epilogue (only for a single partition, where the merge is the identity)
int run_phase(const elsa_fwd_args* a, const elsa_fwd_plan& pl, int q_start, int q_len, hipStream_t st, int which) {
  FwdBuffers wb = carve(a, pl);
  const int bh = a->batch * a->heads;
  if (which == 1 || which == 3) {
    elsa::Phase1Params p{};
    p.direct = which == 3 ? 1 : 0;
    p.out = a->out;
    p.row_m = a->row_m;
    p.row_z = a->row_z;
    resolve_layout(a->q_layout, a->heads, a->seq_len, a->head_dim, p.qs);
    resolve_layout(a->k_layout, a->heads, a->seq_len, a->head_dim, p.ks);
    resolve_layout(a->v_layout, a->heads, a->seq_len, a->head_dim, p.vs);
    resolve_layout(a->out_layout, a->heads, a->seq_len, a->head_dim, p.os);
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.bias = bias_view(a->bias);
    p.m_buf = wb.m;
    p.z_buf = wb.z;
    p.s_buf = wb.s;
    p.s_dtype = a->summary_dtype;
    p.H = a->heads;
    p.N = a->seq_len;
    p.D = a->head_dim;
    p.BH = bh;
    p.q_start = q_start;
    p.q_len = q_len;
    p.part_len = pl.partition_len;
    p.P = pl.partitions;
    p.causal = a->is_causal ? 1 : 0;
    p.scale_log2 = (float)(1.4426950408889634 * softmax_scale(a->scale, a->head_dim));
    p.bias_log2 = 1.4426950408889634f;
    // the reference's d64 fast path (attention_parallel_scan.py:418-440, :983-1018): fp16 without
    // bias or causal mask, a user block_n that is a multiple of 64, summaries in the input dtype
    p.prescale_q = (a->dtype == ELSA_F16 && a->head_dim == 64 && !p.bias.ptr && !a->is_causal &&
                    a->summary_dtype == a->dtype && a->partition_len % 64 == 0)
                       ? 1
                       : 0;
    p.exact_max = a->exact_row_max ? 1 : 0;
    p.rows_pad = pl.q_chunk;
    hipError_t e = elsa::launch_phase1(p, a->dtype, pl.block_m, st);
    if (e != hipSuccess) return hip_fail(e, "phase1 launch");
  } else {
    elsa::Phase2Params p{};
    p.m_buf = wb.m;
    p.z_buf = wb.z;
    p.s_buf = wb.s;
    p.s_dtype = a->summary_dtype;
    p.out = a->out;
    p.out_dtype = a->dtype;
    p.row_m = a->row_m;
    p.row_z = a->row_z;
    p.N = a->seq_len;
    p.D = a->head_dim;
    p.BH = bh;
    p.q_start = q_start;
    p.q_len = q_len;
    p.part_len = pl.partition_len;
    p.P = pl.partitions;
    p.causal = a->is_causal ? 1 : 0;
    p.rows_pad = pl.q_chunk;
    p.H = a->heads;
    resolve_layout(a->out_layout, a->heads, a->seq_len, a->head_dim, p.os);
    hipError_t e = elsa::launch_phase2(p, st);
    if (e != hipSuccess) return hip_fail(e, "phase2 launch");
  }
  return ELSA_OK;
}

// Rules every operand layout follows: non-negative strides, a row stride of at least
// head_dim and below 2^25 elements (the kernels keep a 64-row stage's offsets in 32 bits),
// strides in multiples of 8 elements (16-byte chunks stay aligned) and a 16-byte aligned
// base.  Outputs also need positive batch and head strides where that dimension
// has more than one entry, so that no two output rows share memory.
int check_layout_rules(const char* name, const void* ptr, const elsa_layout& l, int B, int H, int N, int D,
                       bool output, int64_t s[3]) {
  resolve_layout(l, H, N, D, s);
  if (s[0] < 0 || s[1] < 0 || s[2] < D)
    return fail(ELSA_ERR_INVALID, "%s layout (%lld, %lld, %lld) needs non-negative strides and a row stride >= "
                "head_dim", name, (long long)s[0], (long long)s[1], (long long)s[2]);
  if (output && ((B > 1 && s[0] == 0) || (H > 1 && s[1] == 0)))
    return fail(ELSA_ERR_INVALID, "%s is an output: its batch and head strides must be positive", name);
  if ((s[0] | s[1] | s[2]) % 8 != 0 || reinterpret_cast<uintptr_t>(ptr) % 16 != 0)
    return fail(ELSA_ERR_INVALID, "%s: strides must be multiples of 8 elements and the pointer 16-byte aligned",
                name);
  if (s[2] >= (int64_t(1) << 25))
    return fail(ELSA_ERR_UNSUPPORTED, "%s: row stride %lld is not below 2^25 elements", name, (long long)s[2]);
  return ELSA_OK;
}

int check_layout(const char* name, const void* ptr, const elsa_layout& l, const elsa_fwd_args* a,
                 int64_t part_len, bool output) {
  int64_t s[3];
  int rc = check_layout_rules(name, ptr, l, a->batch, a->heads, a->seq_len, a->head_dim, output, s);
  if (rc) return rc;
  if (part_len * s[2] * (int64_t)dtype_size(a->dtype) >= (int64_t(1) << 31))
    return fail(ELSA_ERR_UNSUPPORTED, "%s: a K partition spans >= 2 GiB (partition_len %lld x row stride %lld)",
                name, (long long)part_len, (long long)s[2]);
  return ELSA_OK;
}

// A forward call's plan and operands; the caller's workspace too unless own_workspace is false
// (elsa_fwd_noalloc brings its own).
int check_fwd_operands(const elsa_fwd_args* a, elsa_fwd_plan* pl, bool own_workspace) {
  int rc = plan_fwd(a, pl);
  if (rc) return rc;
  if (!a->out) return fail(ELSA_ERR_INVALID, "out must be a non-null device pointer");
  if (own_workspace && (!a->workspace || a->workspace_bytes < pl->workspace_bytes))
    return fail(ELSA_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", a->workspace_bytes,
                pl->workspace_bytes);
  if ((rc = check_layout("q", a->q, a->q_layout, a, pl->partition_len, false)) ||
      (rc = check_layout("k", a->k, a->k_layout, a, pl->partition_len, false)) ||
      (rc = check_layout("v", a->v, a->v_layout, a, pl->partition_len, false)) ||
      (rc = check_layout("out", a->out, a->out_layout, a, pl->partition_len, true)))
    return rc;
  return ELSA_OK;
}

int check_fwd_call(const elsa_fwd_args* a, elsa_fwd_plan* pl) { return check_fwd_operands(a, pl, true); }

// The forward's q-chunk loop: Phase 1 then Phase 2 per chunk, or the single-partition fold
// with the finalize in its epilogue.
int run_fwd(const elsa_fwd_args* a, const elsa_fwd_plan& pl, hipStream_t st) {
  int rc;
  for (int q0 = 0; q0 < a->seq_len; q0 += pl.q_chunk) {
    const int len = std::min(pl.q_chunk, a->seq_len - q0);
    if (pl.partitions == 1) {
      if ((rc = run_phase(a, pl, q0, len, st, 3))) return rc;
      continue;
    }
    if ((rc = run_phase(a, pl, q0, len, st, 1))) return rc;
    if ((rc = run_phase(a, pl, q0, len, st, 2))) return rc;
  }
  return ELSA_OK;
}

int check_rows(const elsa_fwd_args* a, const elsa_fwd_plan& pl, int q_start, int q_len) {
  if (q_start < 0 || q_len <= 0 || q_start + (int64_t)q_len > a->seq_len || q_len > pl.q_chunk)
    return fail(ELSA_ERR_INVALID, "row range [%d, %d) invalid for seq_len %d and q_chunk %d", q_start, q_start + q_len,
                a->seq_len, pl.q_chunk);
  return ELSA_OK;
}

// What a backward entry point reads and writes: q, k (row stats); + v, out, dout (dbias);
// + dq, dk, dv (dq/dk/dv).
enum BwdUse { kUseQK = 0, kUseDbias = 1, kUseGrads = 2 };

int check_bwd_layout(const elsa_bwd_args* a, const char* name, const void* ptr, const elsa_layout& l, bool output) {
  int64_t s[3];
  return check_layout_rules(name, ptr, l, a->batch, a->heads, a->seq_len, a->head_dim, output, s);
}

int check_bwd(const elsa_bwd_args* a, BwdUse use) {
  if (!a) return fail(ELSA_ERR_INVALID, "null argument");
  int rc = check_common(a->batch, a->heads, a->seq_len, a->head_dim, a->dtype, a->q, a->k, a->v);
  if (rc) return rc;
  if ((rc = check_bias(a->bias))) return rc;
  if (use == kUseGrads) {
    if (!a->out || !a->dout || !a->dq || !a->dk || !a->dv)
      return fail(ELSA_ERR_INVALID, "out, dout, dq, dk and dv must be non-null device pointers");
    if (!a->row_m || !a->row_z) return fail(ELSA_ERR_INVALID, "row_m and row_z are required");
  }
  if (use == kUseDbias && (!a->out || !a->dout || !a->row_m || !a->row_z))
    return fail(ELSA_ERR_INVALID, "out, dout, row_m, row_z and dbias must be non-null");
  if ((rc = check_bwd_layout(a, "q", a->q, a->q_layout, false)) ||
      (rc = check_bwd_layout(a, "k", a->k, a->k_layout, false)))
    return rc;
  if (use == kUseQK) return ELSA_OK;
  if ((rc = check_bwd_layout(a, "v", a->v, a->v_layout, false)) ||
      (rc = check_bwd_layout(a, "out", a->out, a->out_layout, false)) ||
      (rc = check_bwd_layout(a, "dout", a->dout, a->dout_layout, false)))
    return rc;
  if (use == kUseDbias) return ELSA_OK;
  if ((rc = check_bwd_layout(a, "dq", a->dq, a->dq_layout, true)) ||
      (rc = check_bwd_layout(a, "dk", a->dk, a->dk_layout, true)) ||
      (rc = check_bwd_layout(a, "dv", a->dv, a->dv_layout, true)))
    return rc;
  return ELSA_OK;
}

elsa::BwdParams bwd_params(const elsa_bwd_args* a) {
  elsa::BwdParams p{};
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.out = a->out;
  p.dout = a->dout;
  p.row_m = a->row_m;
  p.row_z = a->row_z;
  p.dq = a->dq;
  p.dk = a->dk;
  p.dv = a->dv;
  p.bias = bias_view(a->bias);
  p.H = a->heads;
  p.N = a->seq_len;
  p.D = a->head_dim;
  p.BH = a->batch * a->heads;
  p.causal = a->is_causal ? 1 : 0;
  p.scale = (float)softmax_scale(a->scale, a->head_dim);
  p.scale_log2 = (float)(1.4426950408889634 * softmax_scale(a->scale, a->head_dim));
  const size_t rows = (size_t)p.BH * p.N;
  char* base = static_cast<char*>(a->workspace);
  p.d_row = reinterpret_cast<float*>(base);
  p.lse_row = reinterpret_cast<float*>(base + align256(rows * 4));
  p.lse_lo = reinterpret_cast<float*>(base + 2 * align256(rows * 4));
  p.dp = elsa::pad_head_dim(a->head_dim);
  p.split = elsa::bwd_splits(a->dtype, p.dp, p.BH, p.N, a->bias.ptr != nullptr, a->is_causal != 0);
  // rows (dK/dV) or keys (dq) per range: whole stages, 64 rows in the fp16/bf16 kernels and 32 in the
  // fp32 ones (against 64 for fp32: B1 H8 N1025 causal backward 0.161 -> 0.143 ms with 8 ranges of 160
  // keys instead of 192, B2 H3 N300 0.063 -> 0.054, B8 H3 N1025 0.335 -> 0.320)
  {
    const int64_t st = a->dtype == ELSA_F32 ? 32 : 64;
    p.split_len = p.split > 1 ? (int)((((int64_t)p.N + p.split - 1) / p.split + st - 1) / st * st) : p.N;
  }
  p.part = p.split > 1 ? reinterpret_cast<float*>(base + 3 * align256(rows * 4)) : nullptr;
  p.part_stride = (int64_t)(align256((size_t)p.split * rows * p.dp * 4) / 4);
  const int H = a->heads, N = a->seq_len, D = a->head_dim;
  resolve_layout(a->q_layout, H, N, D, p.qs);
  resolve_layout(a->k_layout, H, N, D, p.ks);
  resolve_layout(a->v_layout, H, N, D, p.vs);
  resolve_layout(a->out_layout, H, N, D, p.os);
  resolve_layout(a->dout_layout, H, N, D, p.gs);
  resolve_layout(a->dq_layout, H, N, D, p.dqs);
  resolve_layout(a->dk_layout, H, N, D, p.dks);
  resolve_layout(a->dv_layout, H, N, D, p.dvs);
  return p;
}

}  // namespace

// ------------------------------------------------------------------ allocation-free forward
// Workspace of elsa_fwd_noalloc: the Phase-1 summaries in a file-scope device array, one copy
// per GPU, held from the library's load until the process ends.  64 MiB takes the north
// star's summaries (B1 H8 N16384 d64 fp16, two partitions: 35.7 MB) in one q-chunk; larger
// calls run in several q-chunks over it.  Every call on one GPU uses the same array, so calls
// that overlap on one GPU (concurrent streams, threads) race on it.
namespace elsa {
constexpr size_t kScratchBytes = size_t(64) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
}  // namespace elsa

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of this GPU's scratch.  Host code never passes the array's own name (a
// host-side stand-in, not a device address): hipGetSymbolAddress resolves it once per device,
// with that device current, and the address is kept.
int scratch_for_stream(void* stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (stream != nullptr) {
    int sdev = -1;
    if ((e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev)) != hipSuccess)
      return hip_fail(e, "hipStreamGetDevice");
    if (sdev != dev)
      return fail(ELSA_ERR_INVALID, "elsa_fwd_noalloc: the stream belongs to device %d, the current device is %d",
                  sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(ELSA_ERR_UNSUPPORTED, "device index %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(elsa::scratch))) != hipSuccess)
      return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ELSA_OK;
}

// elsa_fwd's plan with its q-chunk shortened until the summaries fit the scratch (the same
// partitions, so every row gets the same fold and merge as from elsa_fwd, bit for bit).
int fit_plan_to_scratch(const elsa_fwd_args* a, elsa_fwd_plan* pl) {
  if (pl->workspace_bytes <= elsa::kScratchBytes) return ELSA_OK;
  const int64_t bh = (int64_t)a->batch * a->heads;
  const size_t per_row = (size_t)pl->partitions * bh * (8 + (size_t)a->head_dim * dtype_size(a->summary_dtype));
  int64_t rows = (int64_t)((elsa::kScratchBytes - 3 * 256) / per_row);
  if (rows >= pl->block_m) rows = rows / pl->block_m * pl->block_m;
  if (rows < 1)
    return fail(ELSA_ERR_WORKSPACE,
                "elsa_fwd_noalloc: one query row needs %zu bytes of Phase-1 summaries (%d partitions x %lld heads), "
                "beyond the %zu-byte built-in scratch; use elsa_fwd with a workspace",
                per_row, pl->partitions, (long long)bh, elsa::kScratchBytes);
  pl->q_chunk = (int32_t)std::min<int64_t>(rows, pl->q_chunk);
  pl->workspace_bytes = fwd_workspace_bytes(pl->partitions, bh, pl->q_chunk, a->head_dim, a->summary_dtype);
  if (pl->workspace_bytes > elsa::kScratchBytes)
    return fail(ELSA_ERR_WORKSPACE, "elsa_fwd_noalloc: %zu bytes of summaries do not fit the scratch",
                pl->workspace_bytes);
  return ELSA_OK;
}

}  // namespace

extern "C" {

int elsa_abi_version(void) { return ELSA_ABI_VERSION; }

const char* elsa_last_error(void) { return g_last_error.c_str(); }

size_t elsa_struct_size(int which) {
  switch (which) {
    case 0: return sizeof(elsa_fwd_args);
    case 1: return sizeof(elsa_fwd_plan);
    case 2: return sizeof(elsa_bwd_args);
    case 3: return sizeof(elsa_bias_desc);
    case 4: return sizeof(elsa_layout);
    default: return 0;
  }
}

int elsa_fwd_plan_get(const elsa_fwd_args* args, elsa_fwd_plan* plan) { return plan_fwd(args, plan); }

int elsa_fwd(const elsa_fwd_args* a, void* stream) {
  elsa_fwd_plan pl;
  int rc = check_fwd_call(a, &pl);
  if (rc) return rc;
  return run_fwd(a, pl, static_cast<hipStream_t>(stream));
}

int elsa_fwd_noalloc(const elsa_fwd_args* args, void* stream) {
  elsa_fwd_plan pl;
  int rc = check_fwd_operands(args, &pl, false);
  if (rc) return rc;
  if ((rc = fit_plan_to_scratch(args, &pl))) return rc;
  void* ws = nullptr;
  if ((rc = scratch_for_stream(stream, &ws))) return rc;
  elsa_fwd_args a = *args;  // the same call with the scratch as its workspace
  a.workspace = ws;
  a.workspace_bytes = elsa::kScratchBytes;
  return run_fwd(&a, pl, static_cast<hipStream_t>(stream));
}

int elsa_phase1(const elsa_fwd_args* a, int32_t q_start, int32_t q_len, void* stream) {
  elsa_fwd_plan pl;
  int rc = check_fwd_call(a, &pl);
  if (rc) return rc;
  if ((rc = check_rows(a, pl, q_start, q_len))) return rc;
  return run_phase(a, pl, q_start, q_len, static_cast<hipStream_t>(stream), 1);
}

int elsa_phase2(const elsa_fwd_args* a, int32_t q_start, int32_t q_len, void* stream) {
  elsa_fwd_plan pl;
  int rc = check_fwd_call(a, &pl);
  if (rc) return rc;
  if ((rc = check_rows(a, pl, q_start, q_len))) return rc;
  return run_phase(a, pl, q_start, q_len, static_cast<hipStream_t>(stream), 2);
}

// fp32 partials of a split backward (dq, dK, dV): split * rows * dp floats each
static size_t bwd_part_bytes(const elsa_bwd_args* a) {
  const int dp = elsa::pad_head_dim(a->head_dim);
  const int split = elsa::bwd_splits(a->dtype, dp, (int64_t)a->batch * a->heads, a->seq_len, a->bias.ptr != nullptr,
                                     a->is_causal != 0);
  if (split <= 1) return 0;
  const size_t rows = (size_t)a->batch * a->heads * a->seq_len;
  return 3 * align256((size_t)split * rows * dp * 4);
}

size_t elsa_bwd_workspace_bytes(const elsa_bwd_args* a) {
  if (!a || a->batch <= 0 || a->heads <= 0 || a->seq_len <= 0) return 0;
  const size_t rows = (size_t)a->batch * a->heads * a->seq_len;
  // D, LSE2 and LSE2's low part, one float per row each; then a split backward's partials
  return 3 * align256(rows * 4) + bwd_part_bytes(a);
}

int elsa_bwd(const elsa_bwd_args* a, void* stream) { return elsa_bwd_stage(a, -1, stream); }

int elsa_bwd_stage(const elsa_bwd_args* a, int32_t stage, void* stream) {
  int rc = check_bwd(a, kUseGrads);
  if (rc) return rc;
  if (stage < -1 || stage > 2) return fail(ELSA_ERR_INVALID, "stage must be -1, 0, 1 or 2 (got %d)", stage);
  const size_t need = elsa_bwd_workspace_bytes(a);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(ELSA_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", a->workspace_bytes,
                need);
  hipError_t e = elsa::launch_bwd(bwd_params(a), a->dtype, stage, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "backward launch");
  return ELSA_OK;
}

int elsa_row_stats(const elsa_bwd_args* a, float* row_m, float* row_z, void* stream) {
  int rc = check_bwd(a, kUseQK);
  if (rc) return rc;
  if (!row_m || !row_z) return fail(ELSA_ERR_INVALID, "row_m and row_z must be non-null");
  hipError_t e = elsa::launch_row_stats(bwd_params(a), row_m, row_z, a->dtype, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "row_stats launch");
  return ELSA_OK;
}

static size_t dbias_part_bytes(const elsa_bwd_args* a, int nsplit, int32_t bias_batch, int32_t bias_heads) {
  if (nsplit <= 1) return 0;
  return align256((size_t)nsplit * bias_batch * bias_heads * a->seq_len * a->seq_len * sizeof(float));
}

size_t elsa_dbias_workspace_bytes(const elsa_bwd_args* a, int32_t bias_batch, int32_t bias_heads) {
  if (!a || a->batch <= 0 || a->heads <= 0 || a->seq_len <= 0 || bias_batch <= 0 || bias_heads <= 0) return 0;
  const int ns = elsa::dbias_splits(a->seq_len, a->batch, a->heads, bias_batch, bias_heads);
  return elsa_bwd_workspace_bytes(a) + dbias_part_bytes(a, ns, bias_batch, bias_heads);
}

int elsa_dbias(const elsa_bwd_args* a, float* dbias, int32_t bias_batch, int32_t bias_heads, void* stream) {
  int rc = check_bwd(a, kUseDbias);
  if (rc) return rc;
  if (!dbias) return fail(ELSA_ERR_INVALID, "out, dout, row_m, row_z and dbias must be non-null");
  if (!(bias_batch == 1 || bias_batch == a->batch) || !(bias_heads == 1 || bias_heads == a->heads))
    return fail(ELSA_ERR_INVALID, "dbias shape [%d,%d] does not broadcast against [%d,%d]", bias_batch, bias_heads,
                a->batch, a->heads);
  const size_t need = elsa_bwd_workspace_bytes(a);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(ELSA_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", a->workspace_bytes,
                need);
  // split the reduction over broadcast (b, h) pairs when the workspace has room for the partials
  int nsplit = elsa::dbias_splits(a->seq_len, a->batch, a->heads, bias_batch, bias_heads);
  if (a->workspace_bytes < need + dbias_part_bytes(a, nsplit, bias_batch, bias_heads)) nsplit = 1;
  float* part = nsplit > 1 ? reinterpret_cast<float*>(static_cast<char*>(a->workspace) + need) : nullptr;
  hipError_t e = elsa::launch_dbias(bwd_params(a), dbias, bias_batch, bias_heads, a->dtype, nsplit, part,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "dbias launch");
  return ELSA_OK;
}

// The fused dbias needs dS = p * (dP - D) for every (b, h, row, key) in fp32: straight into
// dbias when the bias broadcasts over nothing, else into the workspace and then summed.  Up
// to this many bytes of dS; beyond, dbias is recomputed by elsa_dbias's own kernel.
static constexpr size_t kFusedDbiasBytes = size_t(1) << 30;

static size_t ds_bytes(const elsa_bwd_args* a) {
  return (size_t)a->batch * a->heads * a->seq_len * a->seq_len * sizeof(float);
}

size_t elsa_bwd_dbias_workspace_bytes(const elsa_bwd_args* a, int32_t bias_batch, int32_t bias_heads) {
  if (!a || a->batch <= 0 || a->heads <= 0 || a->seq_len <= 0 || bias_batch <= 0 || bias_heads <= 0) return 0;
  if (ds_bytes(a) > kFusedDbiasBytes) {
    return std::max(elsa_bwd_workspace_bytes(a), elsa_dbias_workspace_bytes(a, bias_batch, bias_heads));
  }
  const bool direct = bias_batch == a->batch && bias_heads == a->heads;
  if (direct) return elsa_bwd_workspace_bytes(a);
  const int ns = elsa::dbias_sum_splits(a->batch, a->heads, bias_batch, bias_heads);
  const size_t part = ns > 1 ? align256((size_t)ns * bias_batch * bias_heads * a->seq_len * a->seq_len * 4) : 0;
  return elsa_bwd_workspace_bytes(a) + align256(ds_bytes(a)) + part;
}

int elsa_bwd_dbias(const elsa_bwd_args* a, float* dbias, int32_t bias_batch, int32_t bias_heads, void* stream) {
  int rc = check_bwd(a, kUseGrads);
  if (rc) return rc;
  if (!dbias || !a->bias.ptr) return fail(ELSA_ERR_INVALID, "dbias and a bias are required");
  if (!(bias_batch == 1 || bias_batch == a->batch) || !(bias_heads == 1 || bias_heads == a->heads))
    return fail(ELSA_ERR_INVALID, "dbias shape [%d,%d] does not broadcast against [%d,%d]", bias_batch, bias_heads,
                a->batch, a->heads);
  const size_t need = elsa_bwd_dbias_workspace_bytes(a, bias_batch, bias_heads);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(ELSA_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", a->workspace_bytes,
                need);
  if (ds_bytes(a) > kFusedDbiasBytes) {  // the backward, then dbias with its own recompute
    if ((rc = elsa_bwd_stage(a, -1, stream))) return rc;
    return elsa_dbias(a, dbias, bias_batch, bias_heads, stream);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool direct = bias_batch == a->batch && bias_heads == a->heads;
  float* ds = direct ? dbias
                     : reinterpret_cast<float*>(static_cast<char*>(a->workspace) + elsa_bwd_workspace_bytes(a));
  hipError_t e = hipSuccess;
  // causal dk/dv workgroups skip the stages above their keys: those dS entries stay zero
  if (a->is_causal && (e = elsa::launch_zero_fill(ds, (int64_t)(ds_bytes(a) / sizeof(float)), st)) != hipSuccess)
    return hip_fail(e, "zero fill");
  elsa::BwdParams p = bwd_params(a);
  p.ds_out = ds;
  if ((e = elsa::launch_bwd(p, a->dtype, -1, st)) != hipSuccess) return hip_fail(e, "backward launch");
  if (!direct) {
    float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(ds) + align256(ds_bytes(a)));
    if ((e = elsa::launch_dbias_sum(ds, dbias, a->batch, a->heads, a->seq_len, bias_batch, bias_heads, part, st)) !=
        hipSuccess)
      return hip_fail(e, "dbias sum launch");
  }
  return ELSA_OK;
}

int elsa_debug_mfma(int32_t variant, const void* a, const void* b, float* d, void* stream) {
  if (variant < 0 || variant > 2) return fail(ELSA_ERR_INVALID, "variant must be 0, 1 or 2");
  if (!a || !b || !d) return fail(ELSA_ERR_INVALID, "null pointer");
  hipError_t e = elsa::launch_debug_mfma(variant, a, b, d, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "debug_mfma launch");
  return ELSA_OK;
}

int elsa_debug_mfma_rate(int32_t variant, const void* src, float* out, int32_t iters, int32_t workgroups,
                         void* stream) {
  if (variant < 0 || variant > 2) return fail(ELSA_ERR_INVALID, "variant must be 0, 1 or 2");
  if (!src || !out) return fail(ELSA_ERR_INVALID, "null pointer");
  if (iters < 1 || iters > 1000000) return fail(ELSA_ERR_INVALID, "iters must be in [1, 1000000]");
  if (workgroups < 1 || workgroups > 65536) return fail(ELSA_ERR_INVALID, "workgroups must be in [1, 65536]");
  // bounds one launch to about 2^31 MFMAs (tens of milliseconds)
  if ((int64_t)iters * workgroups > (int64_t)1 << 26)
    return fail(ELSA_ERR_INVALID, "iters x workgroups must be at most 2^26");
  hipError_t e = elsa::launch_debug_mfma_rate(variant, src, out, iters, workgroups, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "debug_mfma_rate launch");
  return ELSA_OK;
}

}  // extern "C"
