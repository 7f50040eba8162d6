// ELSA forward on gfx950: Phase 1 (per-K-partition monoid fold on MFMA) and
// Phase 2 (per-row up-sweep merge of the partition summaries read back from HBM).
//
// Phase 1 (replaces the Triton summary kernels of the reference,
// attention_parallel_scan.py:123-372 and attention.py:22-106):
//   one workgroup = 32*WAVES query rows of one head x one K partition.
//   Each wave owns a 32-row tile and computes S^T = K Q^T on 32x32 MFMA tiles
//   (Q^T fragments live in registers for the whole partition, K tiles come from
//   LDS), folds the running (m, z) in registers, and accumulates
//   O^T = V^T P^T with V^T staged transposed in LDS.  Because the A operand rows
//   of K are permuted by swap23, the D-layout registers of S^T are already the
//   B operand of the P^T product: no LDS round trip for P.
//   Masked keys (>= partition end, or > row when causal) score -inf; a row with
//   no valid key keeps the identity summary (-inf, 0, 0) (attention.py:91-100).
//   The running max is exact per 64-key stage; the O rescale is skipped when
//   no row of the wave raised its max.
//
// Phase 2 (replaces paper_scan_d64_kernel.cu:10-96 and the Triton up-sweep /
// Hillis-Steele / finalize kernels, attention_parallel_scan.py:13-120, :375-415):
//   one thread = one row x 8 head-dim elements; partition summaries are merged
//   pairwise level by level in registers (Blelloch up-sweep order with identity
//   padding, groups of 8 partitions; up to 8 partitions with the leaf count fixed
//   at compile time), then out = s * (1/z) with the z>0 guard and the base-2 row
//   state is stored.  For causal attention only partitions that start
//   at or before the row are read: later ones are the identity, so this is the
//   inclusive prefix at the row's own partition (the value the reference's
//   Hillis-Steele scan hands to its finalize, attention_parallel_scan.py:745).
#include "elsa_internal.h"
#include "elsa_mfma.h"

namespace elsa {

int pad_head_dim(int d) { return d <= 32 ? 32 : (d <= 64 ? 64 : 128); }

template <typename T, int DP>
struct FwdCfg {
  static constexpr int KP = Mfma<T>::KP;
  static constexpr int KSTEP = 2 * KP;  // contraction length of one MFMA
  static constexpr int NKK = DP / KSTEP;
  static constexpr bool HALF = sizeof(T) == 2;
  static constexpr int KT = ((HALF && DP == 128) || (!HALF && DP >= 64)) ? 32 : 64;  // keys per LDS stage
  static constexpr int NSUB = KT / 32;
  static constexpr int KPAD = HALF ? 8 : 4;  // fp32: K rows stay 16-byte aligned for 4-float loads
  // fp32 V^T keeps stride KT + 1: its transposing scalar writes are conflict-free there, and
  // 16-byte reads at stride KT + 4 cost more in those writes than they saved (16K Phase 1
  // 4.68 against 4.52 ms)
  static constexpr int VPAD = HALF ? 8 : 1;
  static constexpr int KS = DP + KPAD;  // LDS row stride of K   [KT][KS]
  static constexpr int VS = KT + VPAD;  // LDS row stride of V^T [DP][VS]
  static constexpr int LDS_ONE = (KT * KS + DP * VS) * (int)sizeof(T);
  static constexpr int NBUF = (2 * LDS_ONE <= 98304) ? 2 : 1;
  static constexpr int NDT = DP / 32;  // 32-wide head-dim tiles of O^T
  static constexpr int NJ = 16 / KP;   // P^T.V^T MFMAs per 32-key sub-tile
  static constexpr int CE = 16 / (int)sizeof(T);
};

int phase1_key_tile(int dtype, int dp) {
  if (dtype == ELSA_F32) return dp >= 64 ? 32 : 64;
  return 64;
}

__device__ inline float load_bias(const BiasView& b, int bi, int hi, int row, int key) {
  const int64_t off = (int64_t)bi * b.sb + (int64_t)hi * b.sh + (int64_t)row * b.sq + (int64_t)key * b.sk;
  if (b.dtype == ELSA_F32) return static_cast<const float*>(b.ptr)[off];
  if (b.dtype == ELSA_F16) return static_cast<float>(static_cast<const f16*>(b.ptr)[off]);
  return static_cast<float>(static_cast<const bf16*>(b.ptr)[off]);
}

// Bias rows that 16-byte loads can read: 16-bit values, key stride 1, batch / head / row
// strides in multiples of 8 elements and a 16-byte aligned base.
__device__ inline bool bias_rows_vectorizable(const BiasView& b) {
  return b.dtype != ELSA_F32 && b.sk == 1 && b.sq % 8 == 0 && b.sb % 8 == 0 && b.sh % 8 == 0 &&
         reinterpret_cast<uintptr_t>(b.ptr) % 16 == 0;
}

// Bias of one query row (element offset row_off) at keys key0 + 16 j + t (j < 2, t < 8) into
// v[8 j + t]: the keys the D-layout registers of one 32-key sub-tile hold (key_of_reg).
// Keys at or past k_end read as 0 (the caller masks them).  vec: one 16-byte load per 8 keys.
template <typename B16>
__device__ inline void bias_keys16_vec(const BiasView& b, int64_t row_off, int key0, int k_end, float (&v)[16]) {
  typedef B16 b8 __attribute__((ext_vector_type(8)));
  const B16* base = static_cast<const B16*>(b.ptr) + row_off;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int k = key0 + 16 * j;
    if (k + 8 <= k_end) {
      const b8 c = *reinterpret_cast<const b8*>(base + k);
#pragma unroll
      for (int t = 0; t < 8; ++t) v[8 * j + t] = static_cast<float>(c[t]);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) v[8 * j + t] = k + t < k_end ? static_cast<float>(base[k + t]) : 0.f;
    }
  }
}

__device__ inline void bias_keys16(const BiasView& b, int64_t row_off, int key0, int k_end, bool vec, float (&v)[16]) {
  if (vec) {
    if (b.dtype == ELSA_F16)
      bias_keys16_vec<f16>(b, row_off, key0, k_end, v);
    else
      bias_keys16_vec<bf16>(b, row_off, key0, k_end, v);
    return;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = key0 + 16 * (r >> 3) + (r & 7);
    float x = 0.f;
    if (key < k_end) {
      const int64_t off = row_off + (int64_t)key * b.sk;
      if (b.dtype == ELSA_F32)
        x = static_cast<const float*>(b.ptr)[off];
      else if (b.dtype == ELSA_F16)
        x = static_cast<float>(static_cast<const f16*>(b.ptr)[off]);
      else
        x = static_cast<float>(static_cast<const bf16*>(b.ptr)[off]);
    }
    v[r] = x;
  }
}

__device__ inline void store4(void* base, int64_t off, int dtype, float a, float b, float c, float d) {
  if (dtype == ELSA_F32) {
    f32x4 v = {a, b, c, d};
    *reinterpret_cast<f32x4*>(static_cast<float*>(base) + off) = v;
  } else if (dtype == ELSA_F16) {
    typedef f16 h4 __attribute__((ext_vector_type(4)));
    h4 v = {(f16)a, (f16)b, (f16)c, (f16)d};
    *reinterpret_cast<h4*>(static_cast<f16*>(base) + off) = v;
  } else {
    typedef bf16 b4 __attribute__((ext_vector_type(4)));
    b4 v = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
    *reinterpret_cast<b4*>(static_cast<bf16*>(base) + off) = v;
  }
}

// The finalize's normaliser: out = s * (1 / z), with one correctly rounded reciprocal per row
// (0 when z == 0: a row without a valid key has s = 0 and gets out = 0).  Phase 2 and the
// fused single-partition epilogue both use it, so the two give the same bits.
__device__ inline float inv_z(float z) { return z > 0.f ? 1.f / z : 0.f; }

// Epilogue of one row of one partition: the summary (m, z, s) for Phase 2, or, when the
// partition is the whole row (p.direct), Phase 2's finalize in place: s rounded to the
// summary dtype as the summary store would round it, out = s * inv_z(z), and the
// row state (m, z) -- the values Phase 2 computes for a single partition.
__device__ inline float round_to(int dtype, float x) {
  if (dtype == ELSA_F16) return static_cast<float>(static_cast<f16>(x));
  if (dtype == ELSA_BF16) return static_cast<float>(static_cast<bf16>(x));
  return x;
}
__device__ inline void emit_state(const Phase1Params& p, int64_t ridx, int64_t orow, float m, float z) {
  if (!p.direct) {
    p.m_buf[ridx] = m;
    p.z_buf[ridx] = z;
  } else if (p.row_m != nullptr) {
    p.row_m[orow] = z > 0.f ? m : kNegInf;
    p.row_z[orow] = z;
  }
}
template <typename T>
__device__ inline void emit4(const Phase1Params& p, int64_t ridx, int64_t ooff, int d, float z, float a, float b,
                             float c, float e) {
  if (!p.direct) {
    store4(p.s_buf, ridx * p.D + d, p.s_dtype, a, b, c, e);
    return;
  }
  typedef T t4 __attribute__((ext_vector_type(4)));
  const float v[4] = {a, b, c, e};
  const float iz = inv_z(z);
  t4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = static_cast<T>(round_to(p.s_dtype, v[i]) * iz);
  *reinterpret_cast<t4*>(static_cast<T*>(p.out) + ooff + d) = o;
}

template <typename T, int DP, int WAVES, bool HAS_BIAS>
__global__ __launch_bounds__(64 * WAVES) void phase1_kernel(const Phase1Params p) {
  static_assert(sizeof(T) == 4, "fp32 fold (fp16 / bf16: phase1_half_kernel)");
  using C = FwdCfg<T, DP>;
  using M = Mfma<T>;
  // The fp32 MFMA takes one operand element per lane and k-step, and the contraction order
  // over d is free: k-step kk = 4m + u of lane group g takes d = 8m + 4g + u, so one 16-byte
  // LDS load of a K row gives a lane four k-steps (4K Phase 1 0.328 -> 0.317 ms, 16K 4.573
  // -> 4.515 ms against one 4-byte load per k-step).
  constexpr int NM = DP / 8;
  constexpr int NT = 64 * WAVES;
  constexpr int BM = 32 * WAVES;
  constexpr int CPR = DP / C::CE;  // 16-byte chunks per key row
  static_assert((C::KT * CPR) % NT == 0, "staging must divide evenly");
  constexpr int NCH = C::KT * CPR / NT;

  __shared__ __attribute__((aligned(16))) T Ks[C::NBUF][C::KT * C::KS];
  __shared__ __attribute__((aligned(16))) T Vt[C::NBUF][DP * C::VS];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31, g = lane >> 5;
  // causal over the whole sequence with partitions of whole row blocks: longest first
  const bool lpt = p.causal && p.q_start == 0 && p.q_len == p.N && p.part_len % BM == 0;
  const WgCoord wg = lpt ? causal_longest_first((int)gridDim.x, p.BH, p.P, p.part_len / BM) : phase1_order(p.causal);
  const int bh = wg.y, kb = wg.z;
  const int q_end = p.q_start + p.q_len;
  const int wg_row0 = p.q_start + wg.x * BM;
  const int wg_last = min(q_end, wg_row0 + BM) - 1;
  const int k_begin = kb * p.part_len;
  int k_end = min(p.N, k_begin + p.part_len);
  if (p.causal) k_end = min(k_end, wg_last + 1);
  if (k_begin >= k_end) return;  // every row of this workgroup sees the identity here

  const int row0 = wg_row0 + wave * 32;
  const int my_row = row0 + c;
  const bool row_ok = my_row < q_end;
  const int bi = bh / p.H, hi = bh - (bh / p.H) * p.H;
  const T* __restrict__ Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* __restrict__ K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* __restrict__ V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];

  // Q^T operand of S^T = K Q^T: lane (c, g) holds Q[row c][d = 8m + 4g .. + 3]
  f32x4 qf[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int d0 = 8 * m + 4 * g;
    qf[m] = (row_ok && d0 < p.D) ? *reinterpret_cast<const f32x4*>(Q + (int64_t)my_row * p.qs[2] + d0) : f32x4{};
  }

  Chunk16 kreg[NCH], vreg[NCH];
  auto gload = [&](int t0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ci = tid + i * NT;
      const int key = ci / CPR, d0 = (ci % CPR) * C::CE;
      const int ka = t0 + key;
      if (ka < k_end && d0 < p.D) {
        kreg[i] = *reinterpret_cast<const Chunk16*>(K + (int64_t)ka * p.ks[2] + d0);
        vreg[i] = *reinterpret_cast<const Chunk16*>(V + (int64_t)ka * p.vs[2] + d0);
      } else {
        kreg[i] = Chunk16{};
        vreg[i] = Chunk16{};
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ci = tid + i * NT;
      const int key = ci / CPR, d0 = (ci % CPR) * C::CE;
      *reinterpret_cast<Chunk16*>(&Ks[buf][key * C::KS + d0]) = kreg[i];
      const T* vs = reinterpret_cast<const T*>(&vreg[i]);
#pragma unroll
      for (int e = 0; e < C::CE; ++e) Vt[buf][(d0 + e) * C::VS + key] = vs[e];
    }
  };

  f32x16 oacc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) oacc[dt] = f32x16{};
  float m_run = kNegInf, z_lane = 0.f;
  const float cs = p.scale_log2;
  const int ntiles = (k_end - k_begin + C::KT - 1) / C::KT;

  gload(k_begin);
  sstore(0);
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int buf = (C::NBUF == 2) ? (it & 1) : 0;
    const int t0 = k_begin + it * C::KT;
    const bool has_next = it + 1 < ntiles;
    if (C::NBUF == 2 && has_next) gload(t0 + C::KT);
    const T* ks = Ks[buf];
    const T* vt = Vt[buf];

    // S^T = K Q^T : lane (c, g) register r <-> key t0 + 32*sub + key_of_reg(r, g), row c.
    f32x16 s[C::NSUB];
#pragma unroll
    for (int sub = 0; sub < C::NSUB; ++sub) {
      s[sub] = f32x16{};
      const T* krow = ks + (sub * 32 + swap23(c)) * C::KS + 4 * g;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const f32x4 ka = *reinterpret_cast<const f32x4*>(krow + 8 * m);
#pragma unroll
        for (int u = 0; u < 4; ++u) s[sub] = M::mma(ka[u], qf[m][u], s[sub]);
      }
    }

    float mx = kNegInf;
    if constexpr (HAS_BIAS) {
#pragma unroll
      for (int sub = 0; sub < C::NSUB; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = t0 + sub * 32 + key_of_reg(r, g);
          const bool ok = row_ok && key < k_end && (!p.causal || key <= my_row);
          const float x = ok ? fmaf(s[sub][r], cs, load_bias(p.bias, bi, hi, my_row, key) * p.bias_log2) : kNegInf;
          s[sub][r] = x;
          mx = fmaxf(mx, x);
        }
    } else {
      const bool need_mask = (t0 + C::KT > k_end) || (p.causal && (t0 + C::KT - 1 > row0));
      if (need_mask) {
#pragma unroll
        for (int sub = 0; sub < C::NSUB; ++sub)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = t0 + sub * 32 + key_of_reg(r, g);
            const bool ok = key < k_end && (!p.causal || key <= my_row);
            if (!ok) s[sub][r] = kNegInf;
          }
      }
#pragma unroll
      for (int sub = 0; sub < C::NSUB; ++sub)
#pragma unroll
        for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[sub][r], s[sub][r + 1]));
    }
    mx = wave_max_pair(mx);
    const float m_tile = HAS_BIAS ? mx : mx * cs;
    const float m_new = fmaxf(m_run, m_tile);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float zs = 0.f;
#pragma unroll
    for (int sub = 0; sub < C::NSUB; ++sub)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = HAS_BIAS ? fast_exp2(s[sub][r] - m_use) : fast_exp2(fmaf(s[sub][r], cs, -m_use));
        s[sub][r] = pr;
        zs += pr;
      }
    z_lane = fmaf(z_lane, alpha, zs);
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
    }
    m_run = m_new;

    // O^T += V^T P^T : A = V^T rows d, B = P^T straight from the S^T registers; k-step
    // 4 jb + u takes key key_of_reg(4 jb + u, g) = k0 + u.
#pragma unroll
    for (int sub = 0; sub < C::NSUB; ++sub)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int k0 = sub * 32 + 16 * (jb >> 1) + 8 * g + 4 * (jb & 1);  // key_of_reg(4 jb, g)
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
          const T* vrow = vt + (dt * 32 + c) * C::VS + k0;
#pragma unroll
          for (int u = 0; u < 4; ++u) oacc[dt] = M::mma(vrow[u], s[sub][4 * jb + u], oacc[dt]);
        }
      }

    if constexpr (C::NBUF == 2) {
      if (has_next) sstore(buf ^ 1);
      __syncthreads();
    } else {
      __syncthreads();
      if (has_next) {
        gload(t0 + C::KT);
        sstore(0);
        __syncthreads();
      }
    }
  }

  const float z = wave_sum_pair(z_lane);
  if (!row_ok) return;
  const int64_t ridx = ((int64_t)kb * p.BH + bh) * p.rows_pad + (my_row - p.q_start);
  const int64_t orow = (int64_t)bh * p.N + my_row;
  const int64_t ooff = bi * p.os[0] + hi * p.os[1] + (int64_t)my_row * p.os[2];
  if (g == 0) emit_state(p, ridx, orow, m_run, z);
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = dt * 32 + q4 * 8 + 4 * g;
      if (d < p.D)
        emit4<T>(p, ridx, ooff, d, z, oacc[dt][4 * q4], oacc[dt][4 * q4 + 1], oacc[dt][4 * q4 + 2],
                 oacc[dt][4 * q4 + 3]);
    }
}

// ------------------------------------------------------------------ Phase 1, fp16 / bf16
// Each wave owns RT 32-row tiles (RT = 2 for head dims <= 64) so one K/V
// fragment read from LDS feeds RT MFMAs.  K and V are staged row-major with
// 16-byte copies; the V^T operand of O^T += V^T P^T is read with the transposing
// LDS load.  The running max is lazy: it is raised only when a 64-key stage
// exceeds it by more than kLazyTau (p stays <= 2^kLazyTau, exact in fp16/bf16 and
// fp32), and the summary is renormalised to the exact row maximum at the end.
// The row sum accumulates the fp32 p values; the MFMA takes them rounded to T.
//
// PRE (prescale_q): q is rounded to T after scaling by scale*log2(e), as the reference's fp16
// d64 fold does, so the QK^T product yields base-2 scores.  The product then starts from
// -m_run (the MFMA's accumulator input, a register set refreshed only when the lazy max
// moves), so its output is already score - m_run and p = exp2 of it, with no per-score
// scale-and-subtract.
constexpr float kLazyTau = 8.0f;
constexpr float kLazySum = 256.0f;  // 2^kLazyTau

// PV32 (fp16 inputs with fp32 summaries): the P.V product takes p unrounded, as the reference's
// summary kernel does under SUMMARY_DOT_FP32 (attention_parallel_scan.py:701, :902;
// attention.py:96-99).  p is split into p_hi = fp16(p) and p_lo = fp16(p - p_hi), and both halves
// go through the fp16 MFMA (exact products, fp32 sums): p is carried to about 22 bits.
//
// 2 waves per SIMD, except the 1- and 2-wave variants at D >= 64 (sequences of at most 64
// keys): their register staging of a whole 64-key stage does not fit that budget.
template <typename T, int DP, int RT, int WAVES, bool HAS_BIAS, bool PRE, bool PV32 = false, bool LD = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu((WAVES <= 2 && DP >= 64) ? 1 : 2, 2)))
void phase1_half_kernel(const Phase1Params p) {
  static_assert(!(PRE && HAS_BIAS), "the prescaled fold has no bias");
  static_assert(!PV32 || (std::is_same<T, f16>::value && !PRE), "PV32 is the fp16 fold with fp32 summaries");
  using M = Mfma<T>;
  typedef typename M::frag F;
  constexpr int KT = 64;          // keys per LDS stage
  constexpr int NSUB = KT / 32;   // 32-key sub-tiles per stage
  constexpr int NKK = DP / 16;    // MFMAs over the head dim
  constexpr int NDT = DP / 32;    // 32-wide head-dim tiles of O^T
  constexpr int KS = DP + 8;      // LDS row stride (elements) of the K and V tiles
  constexpr int NT = 64 * WAVES;
  constexpr int ROWS_W = 32 * RT;
  constexpr int BM = ROWS_W * WAVES;
  constexpr int CPR = DP / 8;     // 16-byte chunks per key row
  static_assert((KT * CPR) % NT == 0, "staging must divide evenly");
  constexpr int NCH = KT * CPR / NT;

  static_assert(!LD || (WAVES == 4 && DP == 64 && !HAS_BIAS && !PV32 && KS == 72),
                "LDS-direct staging: the 4-wave D = 64 fold, padded 144-byte rows");
  // LD: one array per buffer, so that the compiler sees the loads into one buffer leave the other
  // one's reads alone
  __shared__ __attribute__((aligned(16))) T Ks[LD ? 1 : 2][KT * KS];
  __shared__ __attribute__((aligned(16))) T Vs[LD ? 1 : 2][KT * KS];
  __shared__ __attribute__((aligned(16))) T Ks1[LD ? KT * KS : 1];
  __shared__ __attribute__((aligned(16))) T Vs1[LD ? KT * KS : 1];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31, g = lane >> 5;
  // causal over the whole sequence with partitions of whole row blocks: longest first (the
  // prescaled fold is never causal: no registers spent on it there)
  const bool lpt = !PRE && p.causal && p.q_start == 0 && p.q_len == p.N && p.part_len % BM == 0;
  const WgCoord wg = lpt ? causal_longest_first((int)gridDim.x, p.BH, p.P, p.part_len / BM)
                         : (PRE ? panel_order() : phase1_order(p.causal));
  const int bh = wg.y, kb = wg.z;
  const int q_end = p.q_start + p.q_len;
  const int wg_row0 = p.q_start + wg.x * BM;
  const int wg_last = min(q_end, wg_row0 + BM) - 1;
  const int k_begin = kb * p.part_len;
  int k_end = min(p.N, k_begin + p.part_len);
  if (p.causal) k_end = min(k_end, wg_last + 1);
  if (k_begin >= k_end) return;  // every row of this workgroup sees the identity here
  // causal split: a partition wholly before this work-group's 512-row block is the ping-pong
  // launch's (causal_full_row0)
  if (p.skip_full && (wg_row0 - p.q_start) / 512 >= causal_full_row0(kb, p.part_len)) return;

  const int row0 = wg_row0 + wave * ROWS_W;
  const int bi = bh / p.H, hi = bh - (bh / p.H) * p.H;
  const T* __restrict__ Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* __restrict__ K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* __restrict__ V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];

  F qf[RT][NKK];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = row0 + rt * 32 + c;
    const bool ok = row < q_end;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const int d0 = kk * 16 + g * 8;
      qf[rt][kk] = load_frag<T>(Q + (int64_t)(ok ? row : 0) * p.qs[2] + d0, ok && d0 < p.D);
      if constexpr (PRE) {
#pragma unroll
        for (int t = 0; t < 8; ++t) qf[rt][kk][t] = static_cast<T>(static_cast<float>(qf[rt][kk][t]) * p.scale_log2);
      }
    }
  }

  // transposing-read coordinates of this lane (see lds_read_tr16)
  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // K/V of this partition through buffer resources: keys past k_end and head-dim
  // padding (d0 >= D) read as zeros
  // (row strides below 2^31 / part_len bytes: checked by the planner)
  const uint32_t krs = (uint32_t)p.ks[2] * (uint32_t)sizeof(T), vrs = (uint32_t)p.vs[2] * (uint32_t)sizeof(T);
  const auto rk = make_rsrc(K + (int64_t)k_begin * p.ks[2], (uint32_t)(k_end - k_begin) * krs);
  const auto rv = make_rsrc(V + (int64_t)k_begin * p.vs[2], (uint32_t)(k_end - k_begin) * vrs);
  uint32_t kvoff[NCH], vvoff[NCH];
  static_for<0, NCH>([&](auto I) {
    constexpr int i = decltype(I)::value;
    const int ci = tid + i * NT;
    const int key = ci / CPR, d0 = (ci % CPR) * 8;
    const uint32_t dofs = (uint32_t)d0 * (uint32_t)sizeof(T);
    kvoff[i] = d0 < p.D ? (uint32_t)key * krs + dofs : kBufferOff;
    vvoff[i] = d0 < p.D ? (uint32_t)key * vrs + dofs : kBufferOff;
  });
  Chunk16 kreg[LD ? 1 : NCH], vreg[LD ? 1 : NCH];
  // LD: K and V stage tiles straight into LDS (buffer_load_dwordx4 ... lds, one stage ahead).  A
  // tile is 64 padded rows of 9 16-byte slots (8 of data, 1 of padding, never read), 576 slots; the
  // lanes of wave w fill slots 64 (w + 4 j) .. + 63 (j = 0, 1, and j = 2 for wave 0 only): slot f
  // holds chunk f % 9 of key row f / 9, the padding slot that row's chunk 0.  Keys past k_end read
  // as zeros from the buffer range (LD runs only at D = 64, where every chunk is data).
  uint32_t ldk[LD ? 3 : 1], ldv[LD ? 3 : 1];
  if constexpr (LD) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int f = 64 * (wave + 4 * j) + lane;
      const int r = f / 9, ch = f % 9 == 8 ? 0 : f % 9;
      ldk[j] = (uint32_t)r * krs + (uint32_t)ch * 16u;
      ldv[j] = (uint32_t)r * vrs + (uint32_t)ch * 16u;
    }
  }
  auto ldload = [&](int t0, T* kdst, T* vdst) {
    if constexpr (LD) {
      const uint32_t kt = (uint32_t)(t0 - k_begin);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        buffer_load16_lds(rk, kdst + 64 * (wave + 4 * j) * 8, ldk[j] + kt * krs);
        buffer_load16_lds(rv, vdst + 64 * (wave + 4 * j) * 8, ldv[j] + kt * vrs);
      }
      if (wave == 0) {
        buffer_load16_lds(rk, kdst + 512 * 8, ldk[2] + kt * krs);
        buffer_load16_lds(rv, vdst + 512 * 8, ldv[2] + kt * vrs);
      }
    }
  };
  auto gload = [&](int t0) {
    if constexpr (LD) return;
    // the stage offset goes into the VGPR offset, so that the range check sees it
    const uint32_t kt = (uint32_t)(t0 - k_begin);
    static_for<0, NCH>([&](auto I) {
      constexpr int i = decltype(I)::value;
      kreg[i] = buffer_load16(rk, kvoff[i] + kt * krs, 0);
      vreg[i] = buffer_load16(rv, vvoff[i] + kt * vrs, 0);
    });
  };
  auto sstore = [&](int buf) {
    if constexpr (LD) return;
    static_for<0, NCH>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const int ci = tid + i * NT;
      const int key = ci / CPR, d0 = (ci % CPR) * 8;
      *reinterpret_cast<Chunk16*>(&Ks[buf][key * KS + d0]) = kreg[i];
      *reinterpret_cast<Chunk16*>(&Vs[buf][key * KS + d0]) = vreg[i];
    });
  };

  f32x16 oacc[RT][NDT];
  float m_run[RT], m_true[RT], z_lane[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = kNegInf;
    m_true[rt] = kNegInf;
    z_lane[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] = f32x16{};
  }
  const float cs = p.scale_log2;
  const bool bias_vec = HAS_BIAS && bias_rows_vectorizable(p.bias);
  const int ntiles = (k_end - k_begin + KT - 1) / KT;
  // PRE: accumulator input of the QK^T product, -ref with ref = m_run (0 while m_run = -inf)
  f32x16 negref[PRE ? RT : 1];
#pragma unroll
  for (int rt = 0; rt < (PRE ? RT : 1); ++rt) negref[rt] = f32x16{};

  // stage keys [t0, t0 + KT) from the LDS tiles ks, vs
  auto stage = [&](int t0, const T* ks, const T* vs) __attribute__((always_inline)) {
    // a causal wave whose rows all precede this stage has nothing to add
    const bool active = !p.causal || t0 <= row0 + ROWS_W - 1;
    if (active) {
      f32x16 s[RT][NSUB];
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const T* krow = ks + (sub * 32 + swap23(c)) * KS + g * 8;
        F kf[NKK];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) kf[kk] = *reinterpret_cast<const F*>(krow + kk * 16);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          s[rt][sub] = M::mma(kf[0], qf[rt][0], PRE ? negref[PRE ? rt : 0] : f32x16{});
#pragma unroll
          for (int kk = 1; kk < NKK; ++kk) s[rt][sub] = M::mma(kf[kk], qf[rt][kk], s[rt][sub]);
        }
      }

      float m_tile[RT];
      bool raise = false;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int my_row = row0 + rt * 32 + c;
        float mx = kNegInf;
        if constexpr (HAS_BIAS) {
          const bool row_ok = my_row < q_end;
          const int64_t roff = bi * p.bias.sb + hi * p.bias.sh + (int64_t)(row_ok ? my_row : p.q_start) * p.bias.sq;
#pragma unroll
          for (int sub = 0; sub < NSUB; ++sub) {
            float bv[16];
            bias_keys16(p.bias, roff, t0 + sub * 32 + 8 * g, k_end, bias_vec, bv);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = t0 + sub * 32 + key_of_reg(r, g);
              const bool ok = row_ok && key < k_end && (!p.causal || key <= my_row);
              const float x = ok ? fmaf(s[rt][sub][r], cs, bv[r] * p.bias_log2) : kNegInf;
              s[rt][sub][r] = x;
              mx = fmaxf(mx, x);
            }
          }
        } else {
          const bool need_mask = (t0 + KT > k_end) || (p.causal && (t0 + KT - 1 > row0 + rt * 32));
          if (need_mask) {
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int key = t0 + sub * 32 + key_of_reg(r, g);
                if (!(key < k_end && (!p.causal || key <= my_row))) s[rt][sub][r] = kNegInf;
              }
          }
          float mx1 = kNegInf;  // two v_max3 chains
#pragma unroll
          for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
              mx = fmaxf(fmaxf(mx, s[rt][sub][r]), s[rt][sub][r + 1]);
              mx1 = fmaxf(fmaxf(mx1, s[rt][sub][r + 2]), s[rt][sub][r + 3]);
            }
          mx = fmaxf(mx, mx1);
        }
        mx = wave_max_pair(mx);
        if constexpr (PRE) {
          m_tile[rt] = mx - negref[rt][0];  // the product started from -ref
        } else {
          m_tile[rt] = HAS_BIAS ? mx : mx * cs;
        }
        m_true[rt] = fmaxf(m_true[rt], m_tile[rt]);
        raise |= m_tile[rt] > m_run[rt] + kLazyTau;
      }
      if (__any(raise)) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const float m_new = fmaxf(m_run[rt], m_tile[rt]);
          const float alpha = (m_run[rt] == kNegInf) ? 0.f : fast_exp2(m_run[rt] - m_new);
          z_lane[rt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[rt][dt][r] *= alpha;
          m_run[rt] = m_new;
          if constexpr (PRE) {
            // the scores are relative to the old reference: move them to the new one (a row
            // still at -inf has only -inf scores and keeps reference 0)
            const float ref = (m_new == kNegInf) ? 0.f : m_new;
            const float shift = ref + negref[rt][0];
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
              for (int r = 0; r < 16; ++r) s[rt][sub][r] -= shift;
#pragma unroll
            for (int r = 0; r < 16; ++r) negref[rt][r] = -ref;
          }
        }
      }

      // p = exp2(score - m_run); O^T += V^T P^T with V^T fragments shared by the RT row tiles
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float nm = (m_run[rt] == kNegInf) ? 0.f : -m_run[rt];
        float zs = 0.f;
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float pr;
            if constexpr (PRE) {
              pr = fast_exp2(s[rt][sub][r]);
            } else {
              pr = HAS_BIAS ? fast_exp2(s[rt][sub][r] + nm) : fast_exp2(fmaf(s[rt][sub][r], cs, nm));
            }
            s[rt][sub][r] = pr;
            zs += pr;
          }
        z_lane[rt] += zs;
      }
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          F va[NDT];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const T* base = vs + (sub * 32 + 16 * j + tr_row) * KS + dt * 32 + tr_col;
            const i16x4 lo = lds_read_tr16(base);
            const i16x4 hi4 = lds_read_tr16(base + 4 * KS);
            const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            va[dt] = __builtin_bit_cast(F, both);
          }
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            F b;
#pragma unroll
            for (int t = 0; t < 8; ++t) b[t] = static_cast<T>(s[rt][sub][j * 8 + t]);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] = M::mma(va[dt], b, oacc[rt][dt]);
            if constexpr (PV32) {
              F lo;
#pragma unroll
              for (int t = 0; t < 8; ++t) lo[t] = static_cast<T>(s[rt][sub][j * 8 + t] - static_cast<float>(b[t]));
#pragma unroll
              for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] = M::mma(va[dt], lo, oacc[rt][dt]);
            }
          }
        }
    }
  };
  if constexpr (LD) {
    // stage it + 1 goes into the other LDS buffer while stage it computes; all loads land before
    // the barrier that ends the stage
    ldload(k_begin, Ks[0], Vs[0]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int it = 0; it < ntiles; it += 2) {
      const int t0 = k_begin + it * KT;
      if (it + 1 < ntiles) ldload(t0 + KT, Ks1, Vs1);
      stage(t0, Ks[0], Vs[0]);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (it + 1 < ntiles) {
        if (it + 2 < ntiles) ldload(t0 + 2 * KT, Ks[0], Vs[0]);
        stage(t0 + KT, Ks1, Vs1);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
  } else {
    gload(k_begin);
    sstore(0);
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
      const int buf = it & 1;
      const int t0 = k_begin + it * KT;
      const bool has_next = it + 1 < ntiles;
      if (has_next) gload(t0 + KT);
      stage(t0, Ks[buf], Vs[buf]);
      if (has_next) sstore(buf ^ 1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float z_raw = wave_sum_pair(z_lane[rt]);
    const int my_row = row0 + rt * 32 + c;
    if (my_row >= q_end) continue;
    // renormalise to the exact row maximum (m_run <= m_true <= m_run + kLazyTau)
    const float f = (m_true[rt] == kNegInf) ? 1.f : fast_exp2(m_run[rt] - m_true[rt]);
    const int64_t ridx = ((int64_t)kb * p.BH + bh) * p.rows_pad + (my_row - p.q_start);
    const int64_t orow = (int64_t)bh * p.N + my_row;
    const int64_t ooff = bi * p.os[0] + hi * p.os[1] + (int64_t)my_row * p.os[2];
    const float z = z_raw * f;
    if (g == 0) emit_state(p, ridx, orow, m_true[rt], z);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = dt * 32 + q4 * 8 + 4 * g;
        if (d < p.D)
          emit4<T>(p, ridx, ooff, d, z, oacc[rt][dt][4 * q4] * f, oacc[rt][dt][4 * q4 + 1] * f,
                   oacc[rt][dt][4 * q4 + 2] * f, oacc[rt][dt][4 * q4 + 3] * f);
      }
  }
}

// ------------------------------------------------------------------ Phase 1, ping-pong
// The ping-pong launch of a causal split: a 1-D grid of BH * causal_full_pairs work-groups, one per
// pair of 512-row block and partition wholly below the diagonal.  The pairs are numbered head-major,
// then by partition, then by row block (fastest), and xcd_linear gives each XCD a contiguous range of
// that numbering, so its resident work-groups share one (head, partition) K/V panel in its L2.
__device__ inline WgCoord causal_full_pair(int n, int BH, int P, int part_len) {
  const int nrb = (n + 511) / 512;
  const int cnt = causal_full_pairs(n, P, part_len);
  const int idx = xcd_linear();
  const int bh = idx / cnt;
  int rem = idx - bh * cnt;
  for (int kb = 0; kb < P; ++kb) {
    const int r0 = causal_full_row0(kb, part_len);
    const int m = max(0, nrb - r0);
    if (rem < m) return {r0 + rem, min(bh, BH - 1), kb};
    rem -= m;
  }
  return {0, min(bh, BH - 1), 0};  // not reached: idx < BH * cnt
}

// The fp16/bf16 fold without bias or causal mask, with 8 waves of 64 rows per workgroup,
// two per SIMD, in two groups (waves 0-3 and 4-7) that take turns: while one group's waves
// run the matrix products of a stage, the other group's waves on the same SIMDs run the
// softmax of theirs.  Workgroup barriers delimit the phases, so the matrix core and the
// vector ALU of a SIMD each serve one wave at a time instead of both waves queueing for the
// same unit.  A wave's stage i is
//   M_i (matrix): P^T V of stage i-1 (packed p kept from V_{i-1}), then S = K Q^T of stage i
//                 (PRE, q prescaled: from the reference -m_run, as in phase1_half_kernel);
//   V_i (vector): mask, max, lazy raise, p = exp2(S), row sums, packing of p.
// Phase ph: group 0 runs M_i at ph = 2i and V_i at ph = 2i+1, group 1 one phase later; both
// run 2n + 2 phases (n key stages), so every wave meets every barrier.
// LDS: K of stage i in Ks[i % 2], V of stage i in Vs[i % 2].  Group 0 stages: the global loads
// of K_{i+1} and V_i are issued at ph = 2i and written at the end of ph = 2i+1, into the slots
// of K_{i-1} (last read at ph = 2i-1) and V_{i-2} (last read at ph = 2i-1); M_{i+1} reads them
// from ph = 2i+2 on.
// Measured (per-wave timestamps): the matrix phase takes about three times as long as the
// vector phase, and the kernel is 5% faster than the two-waves-per-SIMD fold at 16K-64K keys.
// CF: the ping-pong launch of a causal split (causal_full_pair): every work-group's partition lies
// wholly before its rows, so the fold needs no mask.
// LD (D = 64): group 0 loads each stage's K and V tiles straight into LDS (buffer_load_dwordx4 ...
// lds) at the start of its softmax phase, instead of into registers in its matrix phase and from
// there into LDS at the end of the softmax phase.  The targets hold K_{i-1} and V_{i-2}, which the
// other group last read in its M_{i-1} and (K, the relaxed state's rare re-formed scores) V_{i-1}
// phases, both before this one; the barrier at the end of the phase waits for the loads.
template <typename T, int DP, bool PRE, bool EXACT, bool CF = false, bool LD = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void phase1_pp_kernel(const Phase1Params p) {
  using M = Mfma<T>;
  typedef typename M::frag F;
  constexpr int RT = 2, WAVES = 8, KT = 64, NSUB = KT / 32, NKK = DP / 16, NDT = DP / 32;
  constexpr int KS = DP + 8, NT = 64 * WAVES, ROWS_W = 32 * RT, BM = ROWS_W * WAVES;
  constexpr int CPR = DP / 8;
  static_assert(KT * CPR == NT, "one 16-byte chunk of K and one of V per thread and stage");

  __shared__ __attribute__((aligned(16))) T Ks[2][KT * KS];
  __shared__ __attribute__((aligned(16))) T Vs[2][KT * KS];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int grp = wave >> 2;
  WgCoord wg;
  if constexpr (CF) {
    wg = causal_full_pair(p.N, p.BH, p.P, p.part_len);
  } else {
    wg = panel_order();
  }
  const int bh = wg.y, kb = wg.z;
  const int q_end = p.q_start + p.q_len;
  const int wg_row0 = p.q_start + wg.x * BM;
  const int k_begin = kb * p.part_len;
  const int k_end = min(p.N, k_begin + p.part_len);
  if (k_begin >= k_end) return;  // uniform over the workgroup

  const int row0 = wg_row0 + wave * ROWS_W;
  const int bi = bh / p.H, hi = bh - (bh / p.H) * p.H;
  const T* __restrict__ Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* __restrict__ K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* __restrict__ V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];

  F qf[RT][NKK];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = row0 + rt * 32 + c;
    const bool ok = row < q_end;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const int d0 = kk * 16 + g * 8;
      qf[rt][kk] = load_frag<T>(Q + (int64_t)(ok ? row : 0) * p.qs[2] + d0, ok && d0 < p.D);
      if constexpr (PRE) {
#pragma unroll
        for (int t = 0; t < 8; ++t) qf[rt][kk][t] = static_cast<T>(static_cast<float>(qf[rt][kk][t]) * p.scale_log2);
      }
    }
  }
  const float cs = p.scale_log2;

  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  const int ntiles = (k_end - k_begin + KT - 1) / KT;
  // staging (group 0 only, at its own phases): thread tid < 256 moves chunks tid and tid + 256
  // of the 64 x DP tiles of K and V (key ci / CPR, head-dim chunk ci % CPR).  Chunk tid + 256 ii
  // sits 256 / CPR keys below chunk tid, so its offsets differ by constants, and an out-of-range
  // offset stays out of range (the buffer ranges are below 2^31 bytes).
  constexpr int NCH = KT * CPR / 256, KSTEP = 256 / CPR;
  const uint32_t krs = (uint32_t)p.ks[2] * (uint32_t)sizeof(T), vrs = (uint32_t)p.vs[2] * (uint32_t)sizeof(T);
  const auto rk = make_rsrc(K + (int64_t)k_begin * p.ks[2], (uint32_t)(k_end - k_begin) * krs);
  const auto rv = make_rsrc(V + (int64_t)k_begin * p.vs[2], (uint32_t)(k_end - k_begin) * vrs);
  const int skey = (tid & 255) / CPR, sd0 = ((tid & 255) % CPR) * 8;
  const uint32_t kvoff = sd0 < p.D ? (uint32_t)skey * krs + (uint32_t)sd0 * (uint32_t)sizeof(T) : kBufferOff;
  const uint32_t vvoff = sd0 < p.D ? (uint32_t)skey * vrs + (uint32_t)sd0 * (uint32_t)sizeof(T) : kBufferOff;
  const int soff = skey * KS + sd0;
  Chunk16 kreg[LD ? 1 : NCH], vreg[LD ? 1 : NCH];
  // LD: a stage tile is 64 padded rows of 9 16-byte slots (8 of data, 1 of padding, never read);
  // the lanes of group 0's wave w fill slots 64 (w + 4 j) .. + 63 (j = 0, 1, and j = 2 for wave 0
  // only): slot f holds chunk f % 9 of key row f / 9, the padding slot that row's chunk 0
  uint32_t ldk[LD ? 3 : 1], ldv[LD ? 3 : 1];
  if constexpr (LD) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int f = 64 * ((wave & 3) + 4 * j) + lane;
      const int r = f / 9, ch = f % 9 == 8 ? 0 : f % 9;
      ldk[j] = (uint32_t)r * krs + (uint32_t)ch * 16u;
      ldv[j] = (uint32_t)r * vrs + (uint32_t)ch * 16u;
    }
  }
  // group 0: K of stage i (when i < ntiles) into kdst and V of stage iv into vdst
  auto ldload = [&](int i, T* kdst, int iv, T* vdst) {
    if constexpr (LD) {
      const uint32_t kt = (uint32_t)(i * KT), vt = (uint32_t)(iv * KT);
      const bool k_on = i < ntiles, v_on = iv >= 0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (k_on) buffer_load16_lds(rk, kdst + 64 * (wave + 4 * j) * 8, ldk[j] + kt * krs);
        if (v_on) buffer_load16_lds(rv, vdst + 64 * (wave + 4 * j) * 8, ldv[j] + vt * vrs);
      }
      if (wave == 0) {
        if (k_on) buffer_load16_lds(rk, kdst + 512 * 8, ldk[2] + kt * krs);
        if (v_on) buffer_load16_lds(rv, vdst + 512 * 8, ldv[2] + vt * vrs);
      }
    }
  };

  f32x16 oacc[RT][NDT];
  // PRE: -ref in every register, the accumulator input of the stage's QK^T product
  f32x16 negref[PRE ? RT : 1];
  float m_run[RT], m_true[RT], z_lane[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = kNegInf;
    m_true[rt] = kNegInf;
    z_lane[rt] = 0.f;
    if constexpr (PRE) negref[rt] = f32x16{};
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] = f32x16{};
  }
  F pk[RT][NSUB][2];  // p of the last folded stage, for its P^T V in the next M phase

  if (grp == 0) {
    if constexpr (LD) {
      ldload(0, Ks[0], -1, Vs[0]);
      __builtin_amdgcn_s_waitcnt(0);  // the loads land before the barrier below
    } else {
      static_for<0, NCH>([&](auto I) {
        constexpr int ii = decltype(I)::value;
        kreg[ii] = buffer_load16(rk, kvoff + (uint32_t)(ii * KSTEP) * krs, 0);
        *reinterpret_cast<Chunk16*>(&Ks[0][soff + ii * KSTEP * KS]) = kreg[ii];
      });
    }
  }
  __syncthreads();
  if (grp == 1) __syncthreads();  // group 1 sits out phase 0

  // O^T += V^T P^T of stage j (V^T fragments from Vs[j % 2], p from pk)
  auto pv = [&](int j0) {
    const T* vs = Vs[j0 & 1];
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        F va[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const T* base = vs + (sub * 32 + 16 * j + tr_row) * KS + dt * 32 + tr_col;
          const i16x4 lo = lds_read_tr16(base);
          const i16x4 hi4 = lds_read_tr16(base + 4 * KS);
          const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          va[dt] = __builtin_bit_cast(F, both);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] = M::mma(va[dt], pk[rt][sub][j], oacc[rt][dt]);
      }
  };

  for (int i = 0; i < ntiles; ++i) {
    f32x16 s[RT][NSUB];
    // ---- M_i: P^T V of stage i-1, S = K Q^T - ref of stage i
    if (!LD && grp == 0) {  // K_{i+1}, V_i: written at the end of this group's V_i
      const uint32_t kt = (uint32_t)(i * KT);
      static_for<0, NCH>([&](auto I) {
        constexpr int ii = decltype(I)::value;
        if (i + 1 < ntiles) kreg[ii] = buffer_load16(rk, kvoff + (kt + KT + ii * KSTEP) * krs, 0);
        vreg[ii] = buffer_load16(rv, vvoff + (kt + ii * KSTEP) * vrs, 0);
      });
    }
    __builtin_amdgcn_s_setprio(1);
    if (i >= 1) pv(i - 1);
    {
      const T* ks = Ks[i & 1];
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const T* krow = ks + (sub * 32 + swap23(c)) * KS + g * 8;
        F kf[NKK];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) kf[kk] = *reinterpret_cast<const F*>(krow + kk * 16);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          if constexpr (PRE) {
            s[rt][sub] = M::mma(kf[0], qf[rt][0], negref[rt]);
          } else {
            s[rt][sub] = M::mma(kf[0], qf[rt][0], f32x16{});
          }
#pragma unroll
          for (int kk = 1; kk < NKK; ++kk) s[rt][sub] = M::mma(kf[kk], qf[rt][kk], s[rt][sub]);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    // ---- V_i: softmax of stage i
    if (LD && grp == 0) ldload(i + 1, Ks[(i + 1) & 1], i, Vs[i & 1]);
    const int t0 = k_begin + i * KT;
    if (t0 + KT > k_end) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (t0 + sub * 32 + key_of_reg(r, g) >= k_end) s[rt][sub][r] = kNegInf;
    }
    if constexpr (EXACT) {
      float m_tile[RT];
      bool raise = false;
  #pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float mx = kNegInf, mx1 = kNegInf;
  #pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
  #pragma unroll
          for (int r = 0; r < 16; r += 4) {
            mx = fmaxf(fmaxf(mx, s[rt][sub][r]), s[rt][sub][r + 1]);
            mx1 = fmaxf(fmaxf(mx1, s[rt][sub][r + 2]), s[rt][sub][r + 3]);
          }
        mx = wave_max_pair(fmaxf(mx, mx1));
        if constexpr (PRE) {
          m_tile[rt] = mx - negref[rt][0];  // the product started from -ref
        } else {
          m_tile[rt] = mx * cs;
        }
        m_true[rt] = fmaxf(m_true[rt], m_tile[rt]);
        raise |= m_tile[rt] > m_run[rt] + kLazyTau;
      }
      if (__any(raise)) {
  #pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const float m_new = fmaxf(m_run[rt], m_tile[rt]);
          const float alpha = (m_run[rt] == kNegInf) ? 0.f : fast_exp2(m_run[rt] - m_new);
          z_lane[rt] *= alpha;
  #pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
  #pragma unroll
            for (int r = 0; r < 16; ++r) oacc[rt][dt][r] *= alpha;
          m_run[rt] = m_new;
          if constexpr (PRE) {
            // the scores are relative to the old reference: move them to the new one (a row still
            // at -inf has only -inf scores and keeps reference 0)
            const float ref = (m_new == kNegInf) ? 0.f : m_new;
            const float shift = ref + negref[rt][0];
  #pragma unroll
            for (int sub = 0; sub < NSUB; ++sub)
  #pragma unroll
              for (int r = 0; r < 16; ++r) s[rt][sub][r] -= shift;
  #pragma unroll
            for (int r = 0; r < 16; ++r) negref[rt][r] = -ref;
          }
        }
      }
      // the row sums in phase1_half_kernel's order, so that both kernels give the same bits
  #pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float nm = (m_run[rt] == kNegInf) ? 0.f : -m_run[rt];
        float zs = 0.f;
  #pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
  #pragma unroll
          for (int j = 0; j < 2; ++j)
  #pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float pr = PRE ? fast_exp2(s[rt][sub][j * 8 + t]) : fast_exp2(fmaf(s[rt][sub][j * 8 + t], cs, nm));
              pk[rt][sub][j][t] = static_cast<T>(pr);
              zs += pr;
            }
        z_lane[rt] += zs;
      }
    } else {
      // p in place of the scores and the lane's row sums, against the current reference.  A
      // lane whose sum stays at or below 2^kLazyTau has no p above it, so the reference stands
      // and the stage needs no row maximum.  Otherwise (and on the first stage) the scores are
      // formed again from Ks[i % 2], which is rewritten only at the end of group 0's V_{i+1},
      // and the stage raises the reference to its maximum as the exact path does.
      float zsv[RT];
      auto expo = [&]() {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const float nm = (m_run[rt] == kNegInf) ? 0.f : -m_run[rt];
          float zs = 0.f;
#pragma unroll
          for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float pr = PRE ? fast_exp2(s[rt][sub][r]) : fast_exp2(fmaf(s[rt][sub][r], cs, nm));
              s[rt][sub][r] = pr;
              zs += pr;
            }
          zsv[rt] = zs;
        }
      };
      expo();
      bool redo = false;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) redo |= !(zsv[rt] <= kLazySum) || m_run[rt] == kNegInf;
      if (__any(redo)) {
        const T* ks = Ks[i & 1];
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) {
          const T* krow = ks + (sub * 32 + swap23(c)) * KS + g * 8;
          F kf[NKK];
#pragma unroll
          for (int kk = 0; kk < NKK; ++kk) kf[kk] = *reinterpret_cast<const F*>(krow + kk * 16);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            if constexpr (PRE) {
              s[rt][sub] = M::mma(kf[0], qf[rt][0], negref[rt]);
            } else {
              s[rt][sub] = M::mma(kf[0], qf[rt][0], f32x16{});
            }
#pragma unroll
            for (int kk = 1; kk < NKK; ++kk) s[rt][sub] = M::mma(kf[kk], qf[rt][kk], s[rt][sub]);
          }
        }
        if (t0 + KT > k_end) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
              for (int r = 0; r < 16; ++r)
                if (t0 + sub * 32 + key_of_reg(r, g) >= k_end) s[rt][sub][r] = kNegInf;
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float mx = kNegInf, mx1 = kNegInf;
#pragma unroll
          for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
              mx = fmaxf(fmaxf(mx, s[rt][sub][r]), s[rt][sub][r + 1]);
              mx1 = fmaxf(fmaxf(mx1, s[rt][sub][r + 2]), s[rt][sub][r + 3]);
            }
          mx = wave_max_pair(fmaxf(mx, mx1));
          const float m_tile = PRE ? mx - negref[rt][0] : mx * cs;
          const float m_new = fmaxf(m_run[rt], m_tile);
          const float alpha = (m_run[rt] == kNegInf) ? 0.f : fast_exp2(m_run[rt] - m_new);
          z_lane[rt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[rt][dt][r] *= alpha;
          m_run[rt] = m_new;
          if constexpr (PRE) {
            const float ref = (m_new == kNegInf) ? 0.f : m_new;
            const float shift = ref + negref[rt][0];
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
              for (int r = 0; r < 16; ++r) s[rt][sub][r] -= shift;
#pragma unroll
            for (int r = 0; r < 16; ++r) negref[rt][r] = -ref;
          }
        }
        expo();
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        z_lane[rt] += zsv[rt];
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int t = 0; t < 8; ++t) pk[rt][sub][j][t] = static_cast<T>(s[rt][sub][j * 8 + t]);
      }
    }
    if (!LD && grp == 0) {
      static_for<0, NCH>([&](auto I) {
        constexpr int ii = decltype(I)::value;
        if (i + 1 < ntiles) *reinterpret_cast<Chunk16*>(&Ks[(i + 1) & 1][soff + ii * KSTEP * KS]) = kreg[ii];
        *reinterpret_cast<Chunk16*>(&Vs[i & 1][soff + ii * KSTEP * KS]) = vreg[ii];
      });
    }
    if constexpr (LD) __builtin_amdgcn_s_waitcnt(0);  // this phase's loads land before the barrier
    __syncthreads();
  }
  // M_n: the last stage's P^T V (group 0 at phase 2n, group 1 at 2n + 1)
  __builtin_amdgcn_s_setprio(1);
  pv(ntiles - 1);
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();
  if (grp == 0) __syncthreads();  // group 0 sits out phase 2n + 1

#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float z_raw = wave_sum_pair(z_lane[rt]);
    // the relaxed summary, relative to m_run, can be up to 2^kLazyTau times the one relative to the
    // row maximum: where the row's |s| passes half the fp16 range, an fp16 summary is stored
    // relative to m_run + kLazyTau instead, no larger than the exact-maximum summary (which the
    // reference also stores in fp16, attention_parallel_scan.py:476-478)
    bool shift = false;
    if constexpr (!EXACT) {
      if (!p.direct && p.s_dtype == ELSA_F16) {
        float amax = 0.f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) amax = fmaxf(amax, fabsf(oacc[rt][dt][r]));
        shift = wave_max_pair(amax) > 32768.f;
      }
    }
    const int my_row = row0 + rt * 32 + c;
    if (my_row >= q_end) continue;
    // renormalise to the exact row maximum (m_run <= m_true <= m_run + kLazyTau); the
    // relaxed state keeps the reference m_run, at most kLazyTau below the maximum (or
    // m_run + kLazyTau, at most kLazyTau above it, for a shifted fp16 summary)
    if constexpr (!EXACT) m_true[rt] = shift ? m_run[rt] + kLazyTau : m_run[rt];
    const float f = (m_true[rt] == kNegInf) ? 1.f : fast_exp2(m_run[rt] - m_true[rt]);
    const int64_t ridx = ((int64_t)kb * p.BH + bh) * p.rows_pad + (my_row - p.q_start);
    const int64_t orow = (int64_t)bh * p.N + my_row;
    const int64_t ooff = bi * p.os[0] + hi * p.os[1] + (int64_t)my_row * p.os[2];
    const float z = z_raw * f;
    if (g == 0) emit_state(p, ridx, orow, m_true[rt], z);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = dt * 32 + q4 * 8 + 4 * g;
        if (d < p.D)
          emit4<T>(p, ridx, ooff, d, z, oacc[rt][dt][4 * q4] * f, oacc[rt][dt][4 * q4 + 1] * f,
                   oacc[rt][dt][4 * q4 + 2] * f, oacc[rt][dt][4 * q4 + 3] * f);
      }
  }
}

// ------------------------------------------------------------------ Phase 2
template <typename ST>
__device__ inline void load8(const void* base, int64_t off, float (&dst)[8]) {
  const ST* ptr = static_cast<const ST*>(base) + off;
  if constexpr (sizeof(ST) == 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(ptr);
    const f32x4 b = *reinterpret_cast<const f32x4*>(ptr + 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      dst[t] = a[t];
      dst[t + 4] = b[t];
    }
  } else {
    typedef ST v8 __attribute__((ext_vector_type(8)));
    const v8 a = *reinterpret_cast<const v8*>(ptr);
#pragma unroll
    for (int t = 0; t < 8; ++t) dst[t] = static_cast<float>(a[t]);
  }
}

// (m, z, s) <- merge(a, b), attention_parallel_scan.py:55-60 / :111-116.
__device__ inline void mono_merge(float ma, float za, const float (&sa)[8], float mb, float zb, const float (&sb)[8],
                                  float& mo, float& zo, float (&so)[8]) {
  const float m = fmaxf(ma, mb);
  const float al = za > 0.f ? fast_exp2(ma - m) : 0.f;
  const float be = zb > 0.f ? fast_exp2(mb - m) : 0.f;
  float tmp[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) tmp[t] = fmaf(sa[t], al, sb[t] * be);
  const float z = fmaf(za, al, zb * be);
#pragma unroll
  for (int t = 0; t < 8; ++t) so[t] = tmp[t];
  zo = z;
  mo = z > 0.f ? m : kNegInf;
}

// Phase 2 for calls with at most NP partitions (NP = 2, 4 or 8).  A row merges its live
// leaves n = P (non-causal) or min(P, row / part_len + 1) (causal: the partitions at or below
// the row's own) with the generic kernel's up-sweep: the same merges in the same order, and a
// pair whose right leaf is past n copies its left one.  FULL (non-causal, P == NP): every
// leaf is live, so the loads are unconditional.
template <typename ST, typename TO, int NP, bool FULL>
__global__ __launch_bounds__(256) void phase2_np_kernel(const Phase2Params p) {
  static_assert(NP == 2 || NP == 4 || NP == 8, "power-of-two leaf count");
  const int cpr = p.D >> 3;
  const int lid = blockIdx.x * 256 + threadIdx.x, bh = blockIdx.y;
  if (lid >= p.q_len * cpr) return;
  const int r = lid / cpr, ch = lid - r * cpr;
  const int row = p.q_start + r;
  int n = NP;
  if constexpr (!FULL) n = p.causal ? min(p.P, row / p.part_len + 1) : p.P;
  const int64_t idx0 = (int64_t)bh * p.rows_pad + r, pstride = (int64_t)p.BH * p.rows_pad;
  float m[NP], z[NP], sv[NP][8];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    if (FULL || i < n) {
      const int64_t idx = idx0 + i * pstride;
      m[i] = p.m_buf[idx];
      z[i] = p.z_buf[idx];
      load8<ST>(p.s_buf, idx * p.D + ch * 8, sv[i]);
    }
  }
#pragma unroll
  for (int w = NP / 2; w >= 1; w >>= 1) {
#pragma unroll
    for (int i = 0; i < w; ++i) {
      if (FULL || 2 * i + 1 < n) {
        mono_merge(m[2 * i], z[2 * i], sv[2 * i], m[2 * i + 1], z[2 * i + 1], sv[2 * i + 1], m[i], z[i], sv[i]);
      } else if (2 * i < n) {
        m[i] = m[2 * i];
        z[i] = z[2 * i];
#pragma unroll
        for (int t = 0; t < 8; ++t) sv[i][t] = sv[2 * i][t];
      }
    }
    if constexpr (!FULL) n = (n + 1) >> 1;
  }
  const int bi = bh / p.H, hi = bh - bi * p.H;
  TO* out = static_cast<TO*>(p.out) + bi * p.os[0] + hi * p.os[1] + (int64_t)row * p.os[2] + ch * 8;
  typedef TO o8 __attribute__((ext_vector_type(8)));
  o8 ov;
  const float iz = inv_z(z[0]);
#pragma unroll
  for (int t = 0; t < 8; ++t) ov[t] = static_cast<TO>(sv[0][t] * iz);
  *reinterpret_cast<o8*>(out) = ov;
  if (p.row_m != nullptr && ch == 0) {
    p.row_m[(int64_t)bh * p.N + row] = z[0] > 0.f ? m[0] : kNegInf;
    p.row_z[(int64_t)bh * p.N + row] = z[0];
  }
}

template <typename ST, typename TO>
// Grid: x = block of 256 (row, 8-column chunk) pairs of one (batch, head), y = batch * head.
__global__ __launch_bounds__(256) void phase2_kernel(const Phase2Params p) {
  const int cpr = p.D >> 3;
  const int lid = blockIdx.x * 256 + threadIdx.x, bh = blockIdx.y;
  if (lid >= p.q_len * cpr) return;
  const int r = lid / cpr, ch = lid - r * cpr;
  const int row = p.q_start + r;
  int kb_hi = p.P - 1;
  if (p.causal) kb_hi = min(kb_hi, row / p.part_len);

  float am = kNegInf, az = 0.f, as[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) as[t] = 0.f;

  for (int base = 0; base <= kb_hi; base += 8) {
    float m[8], z[8], s[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kb = base + i;
      if (kb <= kb_hi) {
        const int64_t idx = ((int64_t)kb * p.BH + bh) * p.rows_pad + r;
        m[i] = p.m_buf[idx];
        z[i] = p.z_buf[idx];
        load8<ST>(p.s_buf, idx * p.D + ch * 8, s[i]);
      } else {
        m[i] = kNegInf;
        z[i] = 0.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) s[i][t] = 0.f;
      }
    }
    // up-sweep: level widths 4, 2, 1; out[i] = merge(in[2i], in[2i+1]).  Leaves past kb_hi
    // are the identity (-inf, 0, 0), and merging with the identity returns the other operand
    // bit for bit, so those merges are skipped (n = live entries of the current level).
    int n = min(8, kb_hi - base + 1);
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1) {
#pragma unroll
      for (int i = 0; i < w; ++i) {
        if (2 * i + 1 < n) {
          mono_merge(m[2 * i], z[2 * i], s[2 * i], m[2 * i + 1], z[2 * i + 1], s[2 * i + 1], m[i], z[i], s[i]);
        } else if (2 * i < n) {
          m[i] = m[2 * i];
          z[i] = z[2 * i];
#pragma unroll
          for (int t = 0; t < 8; ++t) s[i][t] = s[2 * i][t];
        }
      }
      n = (n + 1) >> 1;
    }
    if (base == 0) {
      am = m[0];
      az = z[0];
#pragma unroll
      for (int t = 0; t < 8; ++t) as[t] = s[0][t];
    } else {
      mono_merge(am, az, as, m[0], z[0], s[0], am, az, as);
    }
  }

  const int bi = bh / p.H, hi = bh - bi * p.H;
  TO* out = static_cast<TO*>(p.out) + bi * p.os[0] + hi * p.os[1] + (int64_t)row * p.os[2] + ch * 8;
  typedef TO o8 __attribute__((ext_vector_type(8)));
  o8 ov;
  const float iz = inv_z(az);
#pragma unroll
  for (int t = 0; t < 8; ++t) ov[t] = static_cast<TO>(as[t] * iz);
  *reinterpret_cast<o8*>(out) = ov;
  if (p.row_m != nullptr && ch == 0) {
    p.row_m[(int64_t)bh * p.N + row] = az > 0.f ? am : kNegInf;
    p.row_z[(int64_t)bh * p.N + row] = az;
  }
}

// ------------------------------------------------------------------ launchers
template <typename T, int DP, int W, bool B>
static hipError_t launch1(const Phase1Params& p, hipStream_t st) {
  const dim3 grid((p.q_len + 32 * W - 1) / (32 * W), p.BH, p.P);
  hipLaunchKernelGGL((phase1_kernel<T, DP, W, B>), grid, dim3(64 * W), 0, st, p);
  return hipGetLastError();
}

// The causal split pays where its ping-pong launch fills whole rounds of the chip: B1 H8 d64 fp16
// forward 32K 1.250 -> 1.205 ms, 64K 4.97 -> 4.72 ms; but 16K 0.358 -> 0.429 ms (384 ping-pong
// work-groups, a half-empty second round), B8 H3 N16385 1.02 -> 1.08 ms, 8K 0.116 -> 0.155 ms.
constexpr int kCausalSplitMin = 32768;

template <typename T, int DP, int RT, int W, bool B>
static hipError_t launch1h(const Phase1Params& p, hipStream_t st) {
  constexpr int BM = 32 * RT * W;
  const dim3 grid((p.q_len + BM - 1) / BM, p.BH, p.P);
  if constexpr (!B && DP == 64 && RT == 2 && W == 4) {
    // 512-row ping-pong workgroups for partitions of at least 16 key stages (the 2n + 2 phases
    // of n stages pay two phases of fill): B1 H8 fp16 Phase 1 at 16K keys 0.599 -> 0.564 ms,
    // 64K 8.59 -> 8.13 ms, 8K 0.181 -> 0.175 ms; at 4K (256-key partitions) 0.054 against
    // 0.061 ms.  Both kernels give the same bits, so the choice never changes a result.
    const dim3 g2((p.q_len + 511) / 512, p.BH, p.P);
    const bool pv32 = std::is_same<T, f16>::value && p.s_dtype == ELSA_F32;
    // causal split (whole-sequence causal calls from kCausalSplitMin keys): the pairs of 512-row
    // block and partition wholly below the diagonal, three quarters of the work at P = 4, go to
    // the ping-pong fold (no mask there), the rest to the 4-wave fold, which skips the former;
    // both write their own summaries and Phase 2 merges them as before.  With the exact row
    // state both folds give the same bits as the 4-wave fold alone.
    if (p.causal && p.q_start == 0 && p.q_len == p.N && p.part_len % BM == 0 && p.part_len >= 1024 && p.P > 1 &&
        !p.direct && !pv32 && !p.prescale_q && p.N >= kCausalSplitMin) {
      const int pairs = p.BH * causal_full_pairs(p.N, p.P, p.part_len);
      if (pairs > 0) {
        const bool ld = p.D == 64;
        if (p.exact_max) {
          if (ld) {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, true, true, true>), dim3(pairs), dim3(512), 0, st, p);
          } else {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, true, true>), dim3(pairs), dim3(512), 0, st, p);
          }
        } else {
          if (ld) {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, false, true, true>), dim3(pairs), dim3(512), 0, st, p);
          } else {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, false, true>), dim3(pairs), dim3(512), 0, st, p);
          }
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
      Phase1Params pd = p;
      pd.skip_full = 1;
      hipLaunchKernelGGL((phase1_half_kernel<T, DP, RT, W, false, false>), grid, dim3(64 * W), 0, st, pd);
      return hipGetLastError();
    }
    if (!p.causal && p.part_len >= 1024 && !pv32) {
      bool done = false;
      // D = 64: K/V staged straight into LDS (phase1_pp_kernel's LD)
      const bool ld = p.D == 64;
      if constexpr (std::is_same<T, f16>::value) {
        if (p.prescale_q) {
          if (p.exact_max) {
            if (ld) {
              hipLaunchKernelGGL((phase1_pp_kernel<T, DP, true, true, false, true>), g2, dim3(512), 0, st, p);
            } else {
              hipLaunchKernelGGL((phase1_pp_kernel<T, DP, true, true>), g2, dim3(512), 0, st, p);
            }
          } else {
            if (ld) {
              hipLaunchKernelGGL((phase1_pp_kernel<T, DP, true, false, false, true>), g2, dim3(512), 0, st, p);
            } else {
              hipLaunchKernelGGL((phase1_pp_kernel<T, DP, true, false>), g2, dim3(512), 0, st, p);
            }
          }
          done = true;
        }
      }
      if (!done) {
        if (p.exact_max) {
          if (ld) {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, true, false, true>), g2, dim3(512), 0, st, p);
          } else {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, true>), g2, dim3(512), 0, st, p);
          }
        } else {
          if (ld) {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, false, false, true>), g2, dim3(512), 0, st, p);
          } else {
            hipLaunchKernelGGL((phase1_pp_kernel<T, DP, false, false>), g2, dim3(512), 0, st, p);
          }
        }
      }
      return hipGetLastError();
    }
  }
  // the 4-wave one-tile D = 64 fold (128-row blocks) stages K and V straight into LDS (LD): causal
  // B1 H8 Phase 1 at 4097 tokens 0.0377 -> 0.0356 ms, B8 H3 N1025 0.0143 -> 0.0140 ms, 2K 0.0145 ->
  // 0.0143 ms.  The two-tile fold keeps registers: with LD its unrolled loop took 256 VGPRs against
  // 238, and causal 8K-32K and bf16 2K ran 0.5-5% slower.
  constexpr bool LDOK = !B && DP == 64 && W == 4 && RT == 1;
  if constexpr (!B && DP == 64 && std::is_same<T, f16>::value) {
    if (p.prescale_q) {
      if (LDOK && p.D == 64) {
        hipLaunchKernelGGL((phase1_half_kernel<T, DP, RT, W, false, true, false, LDOK>), grid, dim3(64 * W), 0, st, p);
      } else {
        hipLaunchKernelGGL((phase1_half_kernel<T, DP, RT, W, false, true>), grid, dim3(64 * W), 0, st, p);
      }
      return hipGetLastError();
    }
  }
  if constexpr (std::is_same<T, f16>::value) {
    if (p.s_dtype == ELSA_F32) {  // p unrounded for P.V (the ping-pong fold has no such variant)
      hipLaunchKernelGGL((phase1_half_kernel<T, DP, RT, W, B, false, true>), grid, dim3(64 * W), 0, st, p);
      return hipGetLastError();
    }
  }
  if (LDOK && p.D == 64) {
    hipLaunchKernelGGL((phase1_half_kernel<T, DP, RT, W, B, false, false, LDOK>), grid, dim3(64 * W), 0, st, p);
  } else {
    hipLaunchKernelGGL((phase1_half_kernel<T, DP, RT, W, B, false>), grid, dim3(64 * W), 0, st, p);
  }
  return hipGetLastError();
}

// Rows per Phase-1 workgroup (block_m).  fp16/bf16 at head dims <= 64: 64 rows per wave
// in 4 waves (256 rows); sequences of at most kSmallSeq rows use 32 rows per wave (128-row
// workgroups: twice the workgroups, half the MFMA chain per key stage, which is what
// bounds a launch that fits on the chip in one go); at most 64 rows, one 64-row wave.
// Head dim 128 and fp32: 32 rows per wave, 4 waves (2 for at most 64 rows).
// Measured on MI355X (Phase 1 + Phase 2, 256- against 128-row workgroups): B8 H3 N197
// 11 against 8 us, B1 H8 N1024 22 against 15 us, B8 H3 N1025 25 against 24 us, B1 H8 N4096
// 64 against 70 us, B1 H8 N16384 617 against 703 us.
// With a bias the 64-row waves hold the bias values of two row tiles and spill (252 bytes
// per lane at D = 64), so biased sequences stay at 128 rows: B1 H8 d64 fp16 with an
// [H, N, N] bias, forward 2K 0.068 -> 0.040 ms, 4K 0.211 -> 0.162 ms, 8K 0.688 -> 0.555 ms.
// Causal calls whose 256-row blocks number fewer than 256 over all heads (one per CU) take
// 128-row blocks as well: about half of their workgroups have no keys to fold and the rest
// differ in length, so the launch lasts as long as its longest workgroups, which 128 rows
// halve (B1 H8 d64 fp16 forward, 256 against 128 rows: 1025 tokens 0.024 -> 0.017 ms, 2K
// 0.026 -> 0.020 ms, 4097 0.052 -> 0.044 ms, d32 2K 0.022 -> 0.016 ms; B8 H3 1025 0.026 ->
// 0.019 ms).  Larger causal grids keep 256 (8K level; 16K 0.332 -> 0.367 ms, 32K 1.15 ->
// 1.35 ms with 128), and so do non-causal ones (B2 H8 2K 0.035 -> 0.038 ms with 128).
constexpr int64_t kSmallSeq = 1024;
int phase1_block_m(int dtype, int dp, int64_t n, int64_t bh, bool causal, bool bias) {
  if (n <= 64) return 64;
  if (dtype == ELSA_F32 || dp > 64 || bias) return 128;
  if (causal && bh * ((n + 255) / 256) < 256) return 128;
  return n <= kSmallSeq ? 128 : 256;
}

template <typename T, int DP>
static hipError_t launch1h_wb(const Phase1Params& p, int block_m, hipStream_t st) {
  const bool b = p.bias.ptr != nullptr;
  if constexpr (DP <= 64) {
    // 64 rows with a bias: two waves of 32 rows.  One wave of 64 rows holds the bias values of
    // both row tiles and spilled 148 bytes per lane at D = 32 (Swin-T's 49-token windows: its
    // 224 px forward 1.531 -> 1.469 ms, 512 px 4.371 -> 4.253 ms).
    if (block_m == 64) return b ? launch1h<T, DP, 1, 2, true>(p, st) : launch1h<T, DP, 2, 1, false>(p, st);
    if (block_m == 128) return b ? launch1h<T, DP, 1, 4, true>(p, st) : launch1h<T, DP, 1, 4, false>(p, st);
    // the planner gives biased calls 128-row blocks (phase1_block_m); the grid follows the kernel
    return b ? launch1h<T, DP, 1, 4, true>(p, st) : launch1h<T, DP, 2, 4, false>(p, st);
  } else {
    if (block_m == 64) return b ? launch1h<T, DP, 1, 2, true>(p, st) : launch1h<T, DP, 1, 2, false>(p, st);
    return b ? launch1h<T, DP, 1, 4, true>(p, st) : launch1h<T, DP, 1, 4, false>(p, st);
  }
}

template <typename T>
static hipError_t launch1h_d(const Phase1Params& p, int block_m, hipStream_t st) {
  switch (pad_head_dim(p.D)) {
    case 32: return launch1h_wb<T, 32>(p, block_m, st);
    case 64: return launch1h_wb<T, 64>(p, block_m, st);
    default: return launch1h_wb<T, 128>(p, block_m, st);
  }
}

template <int DP>
static hipError_t launch1_f32_wb(const Phase1Params& p, int block_m, hipStream_t st) {
  const bool b = p.bias.ptr != nullptr;
  if (block_m == 64) return b ? launch1<float, DP, 2, true>(p, st) : launch1<float, DP, 2, false>(p, st);
  return b ? launch1<float, DP, 4, true>(p, st) : launch1<float, DP, 4, false>(p, st);
}

hipError_t launch_phase1(const Phase1Params& p, int dtype, int block_m, hipStream_t st) {
  if (dtype == ELSA_F16) return launch1h_d<f16>(p, block_m, st);
  if (dtype == ELSA_BF16) return launch1h_d<bf16>(p, block_m, st);
  switch (pad_head_dim(p.D)) {
    case 32: return launch1_f32_wb<32>(p, block_m, st);
    case 64: return launch1_f32_wb<64>(p, block_m, st);
    default: return launch1_f32_wb<128>(p, block_m, st);
  }
}

template <typename ST, typename TO>
static hipError_t launch2(const Phase2Params& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.q_len * (p.D >> 3) + 255) / 256), (unsigned)p.BH);
  const bool full = !p.causal;
  if (full && p.P == 2)
    hipLaunchKernelGGL((phase2_np_kernel<ST, TO, 2, true>), grid, dim3(256), 0, st, p);
  else if (full && p.P == 4)
    hipLaunchKernelGGL((phase2_np_kernel<ST, TO, 4, true>), grid, dim3(256), 0, st, p);
  else if (full && p.P == 8)
    hipLaunchKernelGGL((phase2_np_kernel<ST, TO, 8, true>), grid, dim3(256), 0, st, p);
  else if (p.P == 2)
    hipLaunchKernelGGL((phase2_np_kernel<ST, TO, 2, false>), grid, dim3(256), 0, st, p);
  else if (p.P >= 3 && p.P <= 4)
    hipLaunchKernelGGL((phase2_np_kernel<ST, TO, 4, false>), grid, dim3(256), 0, st, p);
  else if (p.P >= 5 && p.P <= 8)
    hipLaunchKernelGGL((phase2_np_kernel<ST, TO, 8, false>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((phase2_kernel<ST, TO>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename ST>
static hipError_t launch2_o(const Phase2Params& p, hipStream_t st) {
  if (p.out_dtype == ELSA_F16) return launch2<ST, f16>(p, st);
  if (p.out_dtype == ELSA_BF16) return launch2<ST, bf16>(p, st);
  return launch2<ST, float>(p, st);
}

hipError_t launch_phase2(const Phase2Params& p, hipStream_t st) {
  if (p.s_dtype == ELSA_F16) return launch2_o<f16>(p, st);
  if (p.s_dtype == ELSA_BF16) return launch2_o<bf16>(p, st);
  return launch2_o<float>(p, st);
}

// ------------------------------------------------------------------ layout probe
template <typename T>
__global__ void debug_mfma_kernel(const T* a, const T* b, float* d) {
  const int l = threadIdx.x;
  typename Mfma<T>::frag fa, fb;
  if constexpr (Mfma<T>::KP == 1) {
    fa = a[l];
    fb = b[l];
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      fa[t] = a[l * 8 + t];
      fb[t] = b[l * 8 + t];
    }
  }
  f32x16 acc = Mfma<T>::mma(fa, fb, f32x16{});
#pragma unroll
  for (int r = 0; r < 16; ++r) d[l * 16 + r] = acc[r];
}

hipError_t launch_debug_mfma(int variant, const void* a, const void* b, float* d, hipStream_t st) {
  if (variant == 0)
    hipLaunchKernelGGL(debug_mfma_kernel<f16>, dim3(1), dim3(64), 0, st, (const f16*)a, (const f16*)b, d);
  else if (variant == 1)
    hipLaunchKernelGGL(debug_mfma_kernel<bf16>, dim3(1), dim3(64), 0, st, (const bf16*)a, (const bf16*)b, d);
  else
    hipLaunchKernelGGL(debug_mfma_kernel<float>, dim3(1), dim3(64), 0, st, (const float*)a, (const float*)b, d);
  return hipGetLastError();
}

// ------------------------------------------------------------------ MFMA rate probe
// Sustained matrix-core rate on given operand values: every lane of a 256-thread work-group
// holds 8 A and 8 B fragments (src: [16][256][KP] elements, fragment 2j is A and 2j+1 is B
// of chain j) and advances 8 independent 32x32 accumulator chains `iters` times.  The
// accumulator sums are written out so that nothing is dead code.
template <typename T>
__global__ __launch_bounds__(256) void debug_mfma_rate_kernel(const T* __restrict__ src, float* out, int iters) {
  using M = Mfma<T>;
  typedef typename M::frag F;
  constexpr int NJ = 8, KP = M::KP;
  const int lane = threadIdx.x;
  F a[NJ], b[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if constexpr (KP == 1) {
      a[j] = src[(2 * j) * 256 + lane];
      b[j] = src[(2 * j + 1) * 256 + lane];
    } else {
#pragma unroll
      for (int t = 0; t < KP; ++t) {
        a[j][t] = src[((2 * j) * 256 + lane) * KP + t];
        b[j][t] = src[((2 * j + 1) * 256 + lane) * KP + t];
      }
    }
  }
  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] = M::mma(a[j], b[j], acc[j]);
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[j][r];
  out[(int64_t)blockIdx.x * 256 + lane] = sum;
}

hipError_t launch_debug_mfma_rate(int variant, const void* src, float* out, int iters, int workgroups,
                                  hipStream_t st) {
  const dim3 grid(workgroups), block(256);
  if (variant == 0)
    hipLaunchKernelGGL(debug_mfma_rate_kernel<f16>, grid, block, 0, st, (const f16*)src, out, iters);
  else if (variant == 1)
    hipLaunchKernelGGL(debug_mfma_rate_kernel<bf16>, grid, block, 0, st, (const bf16*)src, out, iters);
  else
    hipLaunchKernelGGL(debug_mfma_rate_kernel<float>, grid, block, 0, st, (const float*)src, out, iters);
  return hipGetLastError();
}

}  // namespace elsa
