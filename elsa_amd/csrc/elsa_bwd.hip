// ELSA backward on gfx950: exact recompute of p from the saved base-2 row state.
//
//   preprocess  D = rowsum(O * dO), LSE2 = m + log2(max(z, 1e-30))   (attention_bwd.py:188-224)
//   dq kernel   per 32-row wave tile, loop over 32-key tiles:         (attention_bwd.py:309-412)
//               S^T = K Q^T, dP^T = V dO^T, p = exp2(S^T*c - LSE2), dS^T = p (dP^T - D)
//               (cast to the input dtype, :404), dQ^T += K^T dS^T, dq = scale * dQ.
//   dk/dv kernel per 32-key wave tile, loop over 32-row tiles:        (attention_bwd.py:415-527)
//               S = Q K^T, dP = dO V^T, p = exp2(S*c - LSE2); dV^T += dO^T p (p cast, :512),
//               dK^T += Q^T dS (dS cast, :514), dk = scale * dK.
//   row stats   online (m, z) over all keys when no state was saved   (attention_bwd.py:227-306)
//   dbias       per 32x32 score tile: sum over broadcast (b, h) of p (dp - D)  (attention_bwd.py:529-624)
//
// The same swap23 row permutation as the forward makes the D-layout registers of
// S^T / S directly usable as the B operand of the following MFMA.
#include <algorithm>

#include "elsa_internal.h"
#include "elsa_mfma.h"

namespace elsa {

template <typename T, int DP>
struct BwdCfg {
  static constexpr int KP = Mfma<T>::KP;
  static constexpr int KSTEP = 2 * KP;
  static constexpr int NKK = DP / KSTEP;
  static constexpr bool HALF = sizeof(T) == 2;
  static constexpr int TT = 32;  // keys (dq) or rows (dk/dv) per LDS stage
  static constexpr int KPAD = HALF ? 8 : 1;
  static constexpr int VPAD = HALF ? 8 : 1;
  static constexpr int RS = DP + KPAD;  // row-major tile stride [TT][RS]
  static constexpr int TS = TT + VPAD;  // transposed tile stride [DP][TS]
  static constexpr int NDT = DP / 32;
  static constexpr int NJ = 16 / KP;
  static constexpr int CE = 16 / (int)sizeof(T);
};

__device__ inline float load_bias_b(const BiasView& b, int bi, int hi, int row, int key) {
  const int64_t off = (int64_t)bi * b.sb + (int64_t)hi * b.sh + (int64_t)row * b.sq + (int64_t)key * b.sk;
  if (b.dtype == ELSA_F32) return static_cast<const float*>(b.ptr)[off];
  if (b.dtype == ELSA_F16) return static_cast<float>(static_cast<const f16*>(b.ptr)[off]);
  return static_cast<float>(static_cast<const bf16*>(b.ptr)[off]);
}

// Copy rows [row0, row0+TT) x [0, DP) of an [N, D] matrix with row stride rs (elements)
// into LDS, row-major (stride RS) and/or transposed (stride TS); rows >= row_end and
// d >= D are zero.
template <typename T, int DP, int NT, bool RM, bool TR>
__device__ inline void stage_tile(const T* __restrict__ src, int64_t rs, int row0, int row_end, int D, T* rm, T* tr,
                                  int tid) {
  using C = BwdCfg<T, DP>;
  constexpr int CPR = DP / C::CE;
  constexpr int TOTAL = C::TT * CPR;
#pragma unroll
  for (int ci = tid; ci < TOTAL; ci += NT) {
    const int r = ci / CPR, d0 = (ci % CPR) * C::CE;
    const int ra = row0 + r;
    Chunk16 v{};
    if (ra < row_end && d0 < D) v = *reinterpret_cast<const Chunk16*>(src + (int64_t)ra * rs + d0);
    const T* e = reinterpret_cast<const T*>(&v);
    if constexpr (RM) {
      if constexpr (C::HALF) {
        *reinterpret_cast<Chunk16*>(rm + r * C::RS + d0) = v;
      } else {
#pragma unroll
        for (int t = 0; t < C::CE; ++t) rm[r * C::RS + d0 + t] = e[t];
      }
    }
    if constexpr (TR) {
#pragma unroll
      for (int t = 0; t < C::CE; ++t) tr[(d0 + t) * C::TS + r] = e[t];
    }
  }
}

// A-operand fragment for rows swap23(c) of a 32-row tile: from the row-major
// copy for 16-bit types, from the transposed copy for fp32 (one element per lane).
template <typename T, int DP>
__device__ inline typename Mfma<T>::frag a_frag(const T* rm, const T* tr, int c, int g, int kk) {
  using C = BwdCfg<T, DP>;
  if constexpr (C::HALF) {
    return *reinterpret_cast<const typename Mfma<T>::frag*>(rm + swap23(c) * C::RS + kk * C::KSTEP + g * C::KP);
  } else {
    return tr[(kk * C::KSTEP + g * C::KP) * C::TS + swap23(c)];
  }
}

// fp32 stage staging, double-buffered: each thread first loads its 16-byte chunks of the
// next TT rows into registers (f32_stage_load, issued before the current stage's MFMAs),
// then writes them into the other LDS buffer (f32_stage_store2).  Rows >= row_end and
// d >= D read as zeros.
template <int DP, int NT>
struct F32Stage {
  static constexpr int CPR = DP / 4;              // 16-byte chunks per row
  static constexpr int TOTAL = BwdCfg<float, DP>::TT * CPR;
  static constexpr int NCH = (TOTAL + NT - 1) / NT;  // chunks per thread
};

template <int DP, int NT, int NR>
__device__ inline void f32_stage_load(Chunk16 (&reg)[NR], const float* __restrict__ src, int64_t rs, int row0,
                                      int row_end, int D, int tid) {
  using S = F32Stage<DP, NT>;
  static_assert(NR == S::NCH, "one register chunk per staged chunk of this thread");
  static_for<0, S::NCH>([&](auto I) {
    constexpr int i = decltype(I)::value;
    const int ci = tid + i * NT;
    const int r = ci / S::CPR, d0 = (ci % S::CPR) * 4;
    Chunk16 v{};
    if (ci < S::TOTAL && row0 + r < row_end && d0 < D)
      v = *reinterpret_cast<const Chunk16*>(src + (int64_t)(row0 + r) * rs + d0);
    reg[i] = v;
  });
}

// fp32 dk/dv staging: the register chunks written transposed (row stride TS) and row-major
// with stride RS4 (four consecutive d of one row in one 16-byte load).
template <int DP, int NT, int NR, int TS, int RS4>
__device__ inline void f32_stage_store2(const Chunk16 (&reg)[NR], float* tr, float* rm, int tid) {
  using S = F32Stage<DP, NT>;
  static_assert(NR == S::NCH, "one register chunk per staged chunk of this thread");
  static_for<0, S::NCH>([&](auto I) {
    constexpr int i = decltype(I)::value;
    const int ci = tid + i * NT;
    if (S::TOTAL % NT == 0 || ci < S::TOTAL) {
      const int r = ci / S::CPR, d0 = (ci % S::CPR) * 4;
#pragma unroll
      for (int t = 0; t < 4; ++t) tr[(d0 + t) * TS + r] = __uint_as_float(reg[i][t]);
      *reinterpret_cast<Chunk16*>(rm + r * RS4 + d0) = reg[i];
    }
  });
}

// ------------------------------------------------------------------ preprocess
// LSE2 = m + log2(max(z, 1e-30)) (attention_bwd.py:224), formed in double and split into its fp32
// rounding hi and the remainder lo, so that the fp32 kernels' p = exp2(s*c - LSE2) does not carry
// the half-ulp of a ~15-magnitude LSE2 (3e-7 relative, the same for a whole row) into every
// gradient of that row.  A row with no valid key (z == 0) gets +inf instead of -inf, so that p is 0
// without a test.
__device__ inline void lse2_split(float m, float z, float& hi, float& lo) {
  if (z > 0.f) {
    const double l = (double)m + log2((double)fmaxf(z, 1.0e-30f));
    hi = (float)l;
    lo = (float)(l - (double)hi);
  } else {
    hi = __builtin_huge_valf();
    lo = 0.f;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void bwd_pre_kernel(const BwdParams p) {
  // grid: x = block of 32 rows, y = batch * head.  The 8 lanes of a row read its 16-byte
  // chunks side by side (lane j takes chunks j, j + 8, ...), so every load instruction
  // covers whole 128-byte row segments, and add their partial sums with three xor shuffles.
  constexpr int CE = 16 / (int)sizeof(T);
  const int sub = threadIdx.x & 7, row = blockIdx.x * 32 + (threadIdx.x >> 3), bh = blockIdx.y;
  const bool ok = row < p.N;  // uniform over the 8 lanes of a row: no lane leaves before the shuffles
  const int bi = bh / p.H, hi = bh - bi * p.H;
  float acc = 0.f;
  if (ok) {
    const T* o = static_cast<const T*>(p.out) + bi * p.os[0] + hi * p.os[1] + (int64_t)row * p.os[2];
    const T* g = static_cast<const T*>(p.dout) + bi * p.gs[0] + hi * p.gs[1] + (int64_t)row * p.gs[2];
    for (int d = sub * CE; d < p.D; d += 8 * CE) {
      const Chunk16 a = *reinterpret_cast<const Chunk16*>(o + d);
      const Chunk16 b = *reinterpret_cast<const Chunk16*>(g + d);
      const T* ea = reinterpret_cast<const T*>(&a);
      const T* eb = reinterpret_cast<const T*>(&b);
#pragma unroll
      for (int t = 0; t < CE; ++t) acc = fmaf(static_cast<float>(ea[t]), static_cast<float>(eb[t]), acc);
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  if (!ok || sub != 0) return;
  const int64_t i = (int64_t)bh * p.N + row;
  p.d_row[i] = acc;
  float lhi, llo;
  lse2_split(p.row_m[i], p.row_z[i], lhi, llo);
  p.lse_row[i] = lhi;
  p.lse_lo[i] = llo;
}

// ------------------------------------------------------------------ dq
// fp32 only (the fp16 / bf16 kernel follows below).  The fp32 MFMA takes one operand
// element per lane and k-step; over d the contraction order is k-step kk = 4m + u of lane
// group g at d = 8m + 4g + u, so one 16-byte load of a row-major K or V row gives a lane
// four k-steps.  The transposed K tile (dQ operand) keeps stride TT + 1 and 4-byte loads.
template <typename T, int DP, int WAVES, bool HAS_BIAS>
__global__ __launch_bounds__(64 * WAVES) void bwd_dq_kernel(const BwdParams p) {
  static_assert(sizeof(T) == 4, "fp32 kernel");
  using C = BwdCfg<T, DP>;
  using M = Mfma<T>;
  constexpr int NT = 64 * WAVES, BM = 32 * WAVES;
  constexpr int TT = C::TT;       // keys per stage
  constexpr int TS1 = TT + 1;     // transposed K tile [DP][TS1]: conflict-free transposing writes
  constexpr int RS4 = DP + 4;     // row-major K and V tiles [TT][RS4]
  constexpr int NM = DP / 8;
  // two buffers: stage i + 1 goes from global memory into registers while stage i computes, and
  // from there into the other buffer
  __shared__ __attribute__((aligned(16))) float Kr[2][TT * RS4];
  __shared__ __attribute__((aligned(16))) float Vr[2][TT * RS4];
  __shared__ __attribute__((aligned(16))) float Kt[2][DP * TS1];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
            g = lane >> 5;
  WgCoord wg = xcd_order();
  if (p.causal) wg.x = (int)gridDim.x - 1 - wg.x;  // causal: heaviest row blocks first
  const int bh = wg.y;
  const int wg_row0 = wg.x * BM;
  const int wg_last = min(p.N, wg_row0 + BM) - 1;
  const int my_row = wg_row0 + wave * 32 + c;
  const bool row_ok = my_row < p.N;
  const int bi = bh / p.H, hi = bh % p.H;
  const T* Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];
  const T* dO = static_cast<const T*>(p.dout) + bi * p.gs[0] + hi * p.gs[1];

  // this lane's row of Q and dO at d = 8m + 4g .. + 3 (the B operands of S and dP)
  f32x4 qf[NM], gf[NM];
  const int rsafe = row_ok ? my_row : 0;
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int d0 = 8 * m + 4 * g;
    const bool ok = row_ok && d0 < p.D;
    qf[m] = ok ? *reinterpret_cast<const f32x4*>(Q + (int64_t)rsafe * p.qs[2] + d0) : f32x4{};
    gf[m] = ok ? *reinterpret_cast<const f32x4*>(dO + (int64_t)rsafe * p.gs[2] + d0) : f32x4{};
  }
  float lse, lse_lo, dd;
  const int64_t ri = (int64_t)bh * p.N + rsafe;
  if constexpr (DP <= 64) {
    // the preprocess of these rows, in bwd_pre_kernel's order: that kernel's lane j of a row chains
    // fmas over the 4-float chunks j, j + 8, ... below D, and the 8 lanes' sums add pairwise,
    // ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)).  Here chunk 2m + g is this lane's m-th
    // load, so lane group g forms a_{2i+g} over m = i, i + 4, and lanes c and c + 32 add the pairs.
    // The work-groups of the first key range store D and LSE2 for the dK/dV kernel, so a whole
    // backward launches no preprocess.
    const T* O = static_cast<const T*>(p.out) + bi * p.os[0] + hi * p.os[1] + (int64_t)rsafe * p.os[2];
    float pair[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = 0.f;
#pragma unroll
      for (int m = i; m < NM; m += 4) {
        const int d0 = 8 * m + 4 * g;
        if (d0 < p.D) {
          const f32x4 o4 = row_ok ? *reinterpret_cast<const f32x4*>(O + d0) : f32x4{};
#pragma unroll
          for (int t = 0; t < 4; ++t) a = fmaf(o4[t], gf[m][t], a);
        }
      }
      pair[i] = a + __shfl_xor(a, 32);
    }
    const float dsum = (pair[0] + pair[1]) + (pair[2] + pair[3]);
    float lhi, llo;
    lse2_split(p.row_m[ri], p.row_z[ri], lhi, llo);
    if (row_ok && g == 0 && wg.z == 0) {
      p.d_row[ri] = dsum;
      p.lse_row[ri] = lhi;
      p.lse_lo[ri] = llo;
    }
    lse = row_ok ? lhi : 0.f;
    lse_lo = row_ok ? llo : 0.f;
    dd = row_ok ? dsum : 0.f;
  } else {
    lse = row_ok ? p.lse_row[ri] : 0.f;
    lse_lo = row_ok ? p.lse_lo[ri] : 0.f;
    dd = row_ok ? p.d_row[ri] : 0.f;
  }
  const bool live = row_ok && lse > kNegInf;

  f32x16 acc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) acc[dt] = f32x16{};
  const int k_end = p.causal ? wg_last + 1 : p.N;
  // split (bwd_splits; 1 range of N keys otherwise): this work-group's keys [k_lo, k_hi) over grid z,
  // whole 32-key stages, so a stage never straddles a range end short of k_end.  An empty range
  // writes no partial, and the combine (kind 0 past N, kind 1 past a causal row block) skips it.
  const int k_lo = min(k_end, (int)wg.z * p.split_len), k_hi = min(k_end, k_lo + p.split_len);
  if (p.split > 1 && k_lo >= k_hi) return;
  constexpr int CPR = DP / 4;  // 16-byte chunks per key row
  constexpr int NCH = TT * CPR / NT;
  static_assert((TT * CPR) % NT == 0, "staging must divide evenly");
  // chunk tid + i NT of a stage: key row ci / CPR, head dims (ci % CPR) * 4 .. + 3; keys >= k_hi
  // and d >= D are zeros
  f32x4 kreg[NCH], vreg[NCH];
  auto gload = [&](int t0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ci = tid + i * NT;
      const int r = ci / CPR, d0 = (ci % CPR) * 4, key = t0 + r;
      const bool ok = key < k_hi && d0 < p.D;
      kreg[i] = ok ? *reinterpret_cast<const f32x4*>(K + (int64_t)key * p.ks[2] + d0) : f32x4{};
      vreg[i] = ok ? *reinterpret_cast<const f32x4*>(V + (int64_t)key * p.vs[2] + d0) : f32x4{};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ci = tid + i * NT;
      const int r = ci / CPR, d0 = (ci % CPR) * 4;
      *reinterpret_cast<f32x4*>(&Kr[buf][r * RS4 + d0]) = kreg[i];
      *reinterpret_cast<f32x4*>(&Vr[buf][r * RS4 + d0]) = vreg[i];
#pragma unroll
      for (int u = 0; u < 4; ++u) Kt[buf][(d0 + u) * TS1 + r] = kreg[i][u];
    }
  };
  if (k_lo < k_hi) {
    gload(k_lo);
    sstore(0);
  }
  __syncthreads();

  for (int t0 = k_lo, buf = 0; t0 < k_hi; t0 += TT, buf ^= 1) {
    // buffer buf ^ 1 was last read by the previous stage, before the barrier that ended it
    const bool has_next = t0 + TT < k_hi;
    if (has_next) gload(t0 + TT);
    f32x16 s = f32x16{}, dp = f32x16{};
    {
      // A operands: stage key swap23(c), d = 8m + 4g .. + 3
      const float* kr = Kr[buf] + swap23(c) * RS4 + 4 * g;
      const float* vr = Vr[buf] + swap23(c) * RS4 + 4 * g;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const f32x4 ka = *reinterpret_cast<const f32x4*>(kr + 8 * m);
        const f32x4 va = *reinterpret_cast<const f32x4*>(vr + 8 * m);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          s = M::mma(ka[u], qf[m][u], s);
          dp = M::mma(va[u], gf[m][u], dp);
        }
      }
    }
    const bool full = !HAS_BIAS && (t0 + TT <= k_hi) && (!p.causal || t0 + TT - 1 <= wg_row0 + wave * 32);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t0 + key_of_reg(r, g);
      bool ok = live;
      if (!full) ok = ok && key < k_hi && (!p.causal || key <= my_row);
      // s*c - LSE2 with one rounding of the (small) difference, then LSE2's low part
      float x = fmaf(s[r], p.scale_log2, -lse) - lse_lo;
      if constexpr (HAS_BIAS) x = ok ? fmaf(load_bias_b(p.bias, bi, hi, my_row, key), kLog2e, x) : x;
      const float pr = ok ? fast_exp2(x) : 0.f;
      s[r] = pr * (dp[r] - dd);
    }
    // this stage's 32 keys into a fresh accumulator, then one add into the running sum: each
    // dq element is a chain of N/32 adds plus 16 MFMA steps, not N/2 MFMA steps (B8 H3 N1025:
    // 1.06e-6 from the exact dq against the 1e-6 bar, sequential over 513 steps)
    f32x16 st[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) st[dt] = f32x16{};
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int k0 = 16 * (jb >> 1) + 8 * g + 4 * (jb & 1);  // key_of_reg(4 jb, g)
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        const float* ka = Kt[buf] + (dt * 32 + c) * TS1 + k0;
#pragma unroll
        for (int u = 0; u < 4; ++u) st[dt] = M::mma(ka[u], s[4 * jb + u], st[dt]);
      }
    }
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) acc[dt] += st[dt];
    if (has_next) sstore(buf ^ 1);
    __syncthreads();
  }
  if (!row_ok) return;
  if (p.split > 1) {  // this key range's unscaled dQ: the combine sums the ranges and scales
    float* dst = p.part + (((int64_t)wg.z * p.BH + bh) * p.N + my_row) * p.dp;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[dt * 32 + drow(r, g)] = acc[dt][r];
    return;
  }
  T* out = static_cast<T*>(p.dq) + bi * p.dqs[0] + hi * p.dqs[1] + (int64_t)my_row * p.dqs[2];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {  // 16-byte stores, as in bwd_dkdv_kernel
      const int d = dt * 32 + drow(4 * q4, g);
      if (d < p.D)
        *reinterpret_cast<f32x4*>(out + d) = f32x4{acc[dt][4 * q4] * p.scale, acc[dt][4 * q4 + 1] * p.scale,
                                                   acc[dt][4 * q4 + 2] * p.scale, acc[dt][4 * q4 + 3] * p.scale};
    }
}

// ------------------------------------------------------------------ dk / dv
// fp32 only (the fp16 / bf16 kernels follow below).
// 2 waves per SIMD up to D = 64 (243 VGPRs, no AGPRs, no spills).  With one 16-byte LDS load
// per four k-steps the waves keep their operand reads ahead of the MFMAs (B1 H8 d64: 16K
// 10.92 -> 9.23 ms, 4K 0.764 -> 0.703 ms against one 4-byte load per k-step).
template <typename T, int DP, int WAVES, bool HAS_BIAS>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(DP >= 128 ? 1 : 2, 2)))
void bwd_dkdv_kernel(const BwdParams p) {
  static_assert(sizeof(T) == 4, "fp32 kernel");
  using C = BwdCfg<T, DP>;
  using M = Mfma<T>;
  constexpr int NT = 64 * WAVES, BN = 32 * WAVES;
  constexpr int TT = C::TT;       // stage rows
  constexpr int TS1 = TT + 1;     // transposed tiles [DP][TS1]: conflict-free transposing writes
  constexpr int RS4 = DP + 4;     // row-major tiles [TT][RS4]
  constexpr int NM = DP / 8;      // 16-byte operand loads per lane over the head dim
  // The fp32 MFMA takes one operand element per lane and k-step, and the contraction order
  // is free: over d, k-step kk = 4m + u of lane group g takes d = 8m + 4g + u, so one
  // 16-byte load of a row-major Q or dO row gives a lane four k-steps.  The transposed tiles
  // (dK / dV operands) keep stride TT + 1 and 4-byte loads: at a 16-byte aligned stride
  // their transposing writes conflicted 4-way (16K 9.20 against 9.01 ms).
  __shared__ __attribute__((aligned(16))) float Qt[2][DP * TS1];
  __shared__ __attribute__((aligned(16))) float Gt[2][DP * TS1];
  __shared__ __attribute__((aligned(16))) float Qr[2][TT * RS4];
  __shared__ __attribute__((aligned(16))) float Gr[2][TT * RS4];
  __shared__ float lse_s[2][TT], lo_s[2][TT], dd_s[2][TT];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
            g = lane >> 5;
  // causal: the work of a key block shrinks with its index (heaviest first; paired heavy with
  // light where the grid fits in one round)
  const WgCoord wg = (p.causal && WAVES == 4) ? xcd_order_paired() : xcd_order();
  const int bh = wg.y;
  const int wg_key0 = wg.x * BN;
  const int key0 = wg_key0 + wave * 32;
  const int my_key = key0 + c;
  const bool key_ok = my_key < p.N;
  const int bi = bh / p.H, hi = bh % p.H;
  const T* Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];
  const T* dO = static_cast<const T*>(p.dout) + bi * p.gs[0] + hi * p.gs[1];

  // this lane's key row of K and V at d = 8m + 4g .. + 3 (the B operands of S and dP)
  f32x4 kf[NM], vf[NM];
  const int ksafe = key_ok ? my_key : 0;
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int d0 = 8 * m + 4 * g;
    const bool ok = key_ok && d0 < p.D;
    kf[m] = ok ? *reinterpret_cast<const f32x4*>(K + (int64_t)ksafe * p.ks[2] + d0) : f32x4{};
    vf[m] = ok ? *reinterpret_cast<const f32x4*>(V + (int64_t)ksafe * p.vs[2] + d0) : f32x4{};
  }
  f32x16 dk[C::NDT], dv[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }
  const int r_begin = p.causal ? (wg_key0 / TT) * TT : 0;
  // split (bwd_splits; 1 range of N rows otherwise): this work-group's rows [r_lo, r_hi) over grid z,
  // whole 32-row stages.  An empty range writes no partial, and the combine (kind 0 past N, kind 2
  // before a causal key block) skips it.
  const int r_lo = max(r_begin, (int)wg.z * p.split_len), r_hi = min(p.N, (int)wg.z * p.split_len + p.split_len);
  if (p.split > 1 && r_lo >= r_hi) return;
  const int ntiles = r_hi > r_lo ? (r_hi - r_lo + TT - 1) / TT : 0;
  Chunk16 qreg[F32Stage<DP, NT>::NCH], greg[F32Stage<DP, NT>::NCH];
  float lreg = 0.f, loreg = 0.f, dreg = 0.f;
  auto gload = [&](int t0) {
    f32_stage_load<DP, NT>(qreg, Q, p.qs[2], t0, p.N, p.D, tid);
    f32_stage_load<DP, NT>(greg, dO, p.gs[2], t0, p.N, p.D, tid);
    if (tid < TT) {
      const int ra = t0 + tid;
      lreg = ra < p.N ? p.lse_row[(int64_t)bh * p.N + ra] : kNegInf;
      loreg = ra < p.N ? p.lse_lo[(int64_t)bh * p.N + ra] : 0.f;
      dreg = ra < p.N ? p.d_row[(int64_t)bh * p.N + ra] : 0.f;
    }
  };
  auto sstore = [&](int buf) {
    f32_stage_store2<DP, NT, F32Stage<DP, NT>::NCH, TS1, RS4>(qreg, Qt[buf], Qr[buf], tid);
    f32_stage_store2<DP, NT, F32Stage<DP, NT>::NCH, TS1, RS4>(greg, Gt[buf], Gr[buf], tid);
    if (tid < TT) {
      lse_s[buf][tid] = lreg;
      lo_s[buf][tid] = loreg;
      dd_s[buf][tid] = dreg;
    }
  };
  if (ntiles > 0) {
    gload(r_lo);
    sstore(0);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int t0 = r_lo + it * TT, buf = it & 1;
    const bool has_next = it + 1 < ntiles;
    if (has_next) gload(t0 + TT);
    f32x16 s = f32x16{}, dp = f32x16{};
    {
      // A operands: stage row swap23(c), d = 8m + 4g .. + 3
      const float* qr = Qr[buf] + swap23(c) * RS4 + 4 * g;
      const float* gr = Gr[buf] + swap23(c) * RS4 + 4 * g;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const f32x4 qa = *reinterpret_cast<const f32x4*>(qr + 8 * m);
        const f32x4 ga = *reinterpret_cast<const f32x4*>(gr + 8 * m);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          s = M::mma(qa[u], kf[m][u], s);
          dp = M::mma(ga[u], vf[m][u], dp);
        }
      }
    }
    f32x16 pv;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rl = key_of_reg(r, g);
      const int row = t0 + rl;
      const float lse = lse_s[buf][rl];
      bool ok = key_ok && row < p.N && lse > kNegInf;
      if (p.causal) ok = ok && row >= my_key;
      // s*c - LSE2 with one rounding of the (small) difference, then LSE2's low part
      float x = fmaf(s[r], p.scale_log2, -lse) - lo_s[buf][rl];
      if constexpr (HAS_BIAS) x = ok ? fmaf(load_bias_b(p.bias, bi, hi, row, my_key), kLog2e, x) : x;
      const float pr = ok ? fast_exp2(x) : 0.f;
      pv[r] = pr;
      s[r] = pr * (dp[r] - dd_s[buf][rl]);
      if constexpr (HAS_BIAS) {
        if (p.ds_out != nullptr && key_ok && row < p.N) p.ds_out[((int64_t)bh * p.N + row) * p.N + my_key] = s[r];
      }
    }
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int row0 = 16 * (jb >> 1) + 8 * g + 4 * (jb & 1);  // key_of_reg(4 jb, g)
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        const int off = (dt * 32 + c) * TS1 + row0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          dv[dt] = M::mma(Gt[buf][off + u], pv[4 * jb + u], dv[dt]);
          dk[dt] = M::mma(Qt[buf][off + u], s[4 * jb + u], dk[dt]);
        }
      }
    }
    if (has_next) sstore(buf ^ 1);
    __syncthreads();
  }
  if (!key_ok) return;
  // registers 4q .. 4q + 3 hold head dims dt * 32 + drow(4q, g) .. + 3: one 16-byte store each
  // (pointers are 16-byte aligned and strides multiples of 8 elements; D is a multiple of 8, so a
  // group starting below D ends below it)
  if (p.split > 1) {  // this row range's unscaled dK and dV: the combine sums the ranges and scales dK
    const int64_t o = (((int64_t)wg.z * p.BH + bh) * p.N + my_key) * p.dp;
    float* dkp = p.part + p.part_stride + o;
    float* dvp = p.part + 2 * p.part_stride + o;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = dt * 32 + drow(4 * q4, g);
        *reinterpret_cast<f32x4*>(dkp + d) =
            f32x4{dk[dt][4 * q4], dk[dt][4 * q4 + 1], dk[dt][4 * q4 + 2], dk[dt][4 * q4 + 3]};
        *reinterpret_cast<f32x4*>(dvp + d) =
            f32x4{dv[dt][4 * q4], dv[dt][4 * q4 + 1], dv[dt][4 * q4 + 2], dv[dt][4 * q4 + 3]};
      }
    return;
  }
  T* okp = static_cast<T*>(p.dk) + bi * p.dks[0] + hi * p.dks[1] + (int64_t)my_key * p.dks[2];
  T* ovp = static_cast<T*>(p.dv) + bi * p.dvs[0] + hi * p.dvs[1] + (int64_t)my_key * p.dvs[2];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = dt * 32 + drow(4 * q4, g);
      if (d < p.D) {
        *reinterpret_cast<f32x4*>(okp + d) = f32x4{dk[dt][4 * q4] * p.scale, dk[dt][4 * q4 + 1] * p.scale,
                                                   dk[dt][4 * q4 + 2] * p.scale, dk[dt][4 * q4 + 3] * p.scale};
        *reinterpret_cast<f32x4*>(ovp + d) =
            f32x4{dv[dt][4 * q4], dv[dt][4 * q4 + 1], dv[dt][4 * q4 + 2], dv[dt][4 * q4 + 3]};
      }
    }
}

// ------------------------------------------------------------------ fp16 / bf16 dq and dk/dv
// Same tiling ideas as the fp16/bf16 Phase 1: tiles are staged row-major with
// 16-byte copies (double-buffered through registers) and transposed MFMA operands
// (K^T for dq; Q^T, dO^T for dk/dv) come from the transposing LDS load.  RT (dq)
// and KRT (dk/dv) are the 32-wide tiles per wave.
template <typename T, int DP, bool SWIZZLE>
struct HalfStage {
  static constexpr int ST = 64;       // rows (or keys) per LDS stage (the 8-wave dK/dV kernel: 128)
  // At DP = 64 and SWIZZLE: unpadded rows with XOR-swizzled chunks (lds_swz_off).  Over the
  // whole chip in a read-only loop, the transposing reads of padded 72-element rows ran at 74
  // against 133 TB/s of LDS reads swizzled (they conflicted 2-way on a quarter of the banks), the
  // row fragments at 119-120 TB/s either way.
  static constexpr bool SWZ = SWIZZLE && DP == 64;
  static constexpr int KS = SWZ ? DP : DP + 8;  // LDS row stride in elements
  static constexpr int CPR = DP / 8;            // 16-byte chunks per row
  // element offset of (row r, column col) of a stage tile; col / 8 is its chunk
  __device__ static inline int off(int r, int col) {
    if constexpr (SWZ) {
      return lds_swz_off(r, col);
    } else {
      return r * KS + col;
    }
  }
};

// 8 consecutive rows of a column: two transposing reads at this lane's element offsets o0 (rows
// r0..r0+3) and o1 (rows r0+4..r0+7)
template <typename T>
__device__ inline typename Mfma<T>::frag tr_frag_off(const T* base, int o0, int o1) {
  const i16x4 lo = lds_read_tr16(base + o0);
  const i16x4 hi = lds_read_tr16(base + o1);
  const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Mfma<T>::frag, both);
}

// 8 consecutive rows (k) r0..r0+7 of a HalfStage tile at column `col` of this lane: two
// transposing reads of 4 rows
template <typename T, typename Tile>
__device__ inline typename Mfma<T>::frag tr_frag_at(const T* tile, int r0, int col) {
  static_assert(!Tile::SWZ, "padded rows (swizzled tiles read through tr_frag_off)");
  const T* row0 = tile + r0 * Tile::KS;
  const i16x4 lo = lds_read_tr16(row0 + col);
  const i16x4 hi = lds_read_tr16(row0 + 4 * Tile::KS + col);
  const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Mfma<T>::frag, both);
}


// LD (the two-tile 8-wave kernel at D = 64): the K and V stage tiles go straight from global memory
// into LDS (buffer_load_dwordx4 ... lds, one stage ahead) instead of through staging registers.
template <typename T, int DP, int RT, int WAVES, bool HAS_BIAS, bool LD = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bwd_dq_half_kernel(const BwdParams p) {
  using M = Mfma<T>;
  typedef typename M::frag F;
  // padded rows: with the swizzled tiles of bwd_dkdv_half_kernel the one-tile dq measured 1-2% slower,
  // and the two-tile one has no registers for the lane offsets
  using Tile = HalfStage<T, DP, false>;
  constexpr int KT = Tile::ST, KS = Tile::KS, CPR = Tile::CPR;
  constexpr int NKK = DP / 16, NDT = DP / 32;
  constexpr int NT = 64 * WAVES, ROWS_W = 32 * RT, BM = ROWS_W * WAVES;
  static_assert((KT * CPR) % NT == 0, "staging must divide evenly");
  constexpr int NCH = KT * CPR / NT;
  static_assert(!LD || ((WAVES == 4 || WAVES == 8) && DP == 64 && !HAS_BIAS && KT == 64 && KS == 72),
                "LDS-direct staging: the 4- and 8-wave D = 64 kernels, padded 144-byte rows");
  // LD: one array per buffer (see bwd_dkdv_half_kernel)
  __shared__ __attribute__((aligned(16))) T Ks[LD ? 1 : 2][KT * KS];
  __shared__ __attribute__((aligned(16))) T Vs[LD ? 1 : 2][KT * KS];
  __shared__ __attribute__((aligned(16))) T Ks1[LD ? KT * KS : 1];
  __shared__ __attribute__((aligned(16))) T Vs1[LD ? KT * KS : 1];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
            g = lane >> 5;
  // causal: the work of a row block grows with its index; each XCD takes its range of
  // row blocks heaviest first (paired heavy with light where the grid fits in one round)
  WgCoord wg = (p.causal && WAVES == 4) ? xcd_order_paired() : xcd_order();
  if (p.causal) wg.x = (int)gridDim.x - 1 - wg.x;
  const int bh = wg.y;
  const int wg_row0 = wg.x * BM;
  const int wg_last = min(p.N, wg_row0 + BM) - 1;
  const int row0 = wg_row0 + wave * ROWS_W;
  const int bi = bh / p.H, hi = bh % p.H;
  const T* Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];
  const T* dO = static_cast<const T*>(p.dout) + bi * p.gs[0] + hi * p.gs[1];
  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // split (the 4-wave one-tile kernel only, below): grid z cuts the key loop into ranges
  constexpr bool CAN_SPLIT = RT == 1 && WAVES == 4 && (DP == 128 || (!HAS_BIAS && DP <= 64));
  F qf[RT][NKK], gf[RT][NKK];
  float lse[RT], dd[RT];
  bool live[RT];
  // LD (unbiased, D = 64): the preprocess of these rows runs here, in bwd_pre_kernel's order (per
  // 16-byte chunk of a row an fma chain over its 8 elements from zero, then the chunk sums pairwise,
  // ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)); lanes c and c + 32 hold the even and odd
  // chunks of row c), so a whole backward needs no preprocess launch; the work-groups of the first
  // key range store D and LSE2 for the dK/dV kernel
  const T* O = static_cast<const T*>(p.out) + bi * p.os[0] + hi * p.os[1];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = row0 + rt * 32 + c;
    const bool ok = row < p.N;
    const int rs = ok ? row : 0;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const int d0 = kk * 16 + g * 8;
      qf[rt][kk] = load_frag<T>(Q + (int64_t)rs * p.qs[2] + d0, ok && d0 < p.D);
      gf[rt][kk] = load_frag<T>(dO + (int64_t)rs * p.gs[2] + d0, ok && d0 < p.D);
    }
    const int64_t ri = (int64_t)bh * p.N + rs;
    if constexpr (LD) {
      float pair[NKK];
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const F of = load_frag<T>(O + (int64_t)rs * p.os[2] + kk * 16 + g * 8, ok);
        float a = 0.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) a = fmaf(static_cast<float>(of[t]), static_cast<float>(gf[rt][kk][t]), a);
        pair[kk] = a + __shfl_xor(a, 32);
      }
      const float dsum = (pair[0] + pair[1]) + (pair[2] + pair[3]);
      float lhi, llo;
      lse2_split(p.row_m[ri], p.row_z[ri], lhi, llo);
      if (ok && g == 0 && (!CAN_SPLIT || wg.z == 0)) {
        p.d_row[ri] = dsum;
        p.lse_row[ri] = lhi;
        p.lse_lo[ri] = llo;
      }
      lse[rt] = ok ? lhi : __builtin_huge_valf();
      dd[rt] = ok ? dsum : 0.f;
    } else {
      lse[rt] = ok ? p.lse_row[ri] : __builtin_huge_valf();
      dd[rt] = ok ? p.d_row[ri] : 0.f;
    }
    live[rt] = ok && lse[rt] < __builtin_huge_valf();
  }
  const int k_end = p.causal ? wg_last + 1 : p.N;
  // split (the 4-wave one-tile kernel only): this work-group's keys [k_lo, k_hi), whole 64-key
  // stages (one range when unsplit).  D = 128 never splits (bwd_splits) but keeps these run-time
  // bounds: with constant ones its register allocation spilled (20 bytes per lane, 468 biased;
  // 16K dq 1.698 -> 1.653 ms without)
  const int k_lo = CAN_SPLIT ? min(k_end, wg.z * p.split_len) : 0;
  const int k_hi = CAN_SPLIT ? min(k_end, k_lo + p.split_len) : k_end;
  // a causal key range past this row block's last row adds nothing: no partial is written, and
  // the combine (bwd_combine_kernel, kind 1) skips the same ranges
  if (CAN_SPLIT && p.split > 1 && p.causal && k_lo >= k_hi) return;
  // -D of this lane's row: the dP^T product starts from it and yields dP - D directly.  The
  // 16 registers per row tile of that constant would spill in the bias, D = 128 and two-tile
  // variants, which subtract D from each score instead.
  constexpr bool SEED_D = !HAS_BIAS && DP <= 64 && RT == 1;
  f32x16 ndd[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int r = 0; r < 16; ++r) ndd[rt][r] = SEED_D ? -dd[rt] : 0.f;
  // The two-tile kernel (no registers for the seeds) adds -D with one more MFMA per row tile and
  // sub-tile instead: A = (2^15, 1, 1) at k = 0, 1, 2 for every key and B = (b0, b1, b2) of the
  // lane's row there, with b0 = T(-D / 2^15), r = -D - 2^15 b0, b1 = T(r), b2 = T(r - b1): the
  // products are exact and their fp32 sum is -D within 2^-22 relative plus 3e-8 absolute (fp16
  // subnormals), for |D| up to 1.4e8 with fp16 (bf16 has fp32's range); an fp16 -D alone would
  // overflow past 65504, e.g. under loss-scaled gradients.  The vector work per
  // score loses its subtract; the matrix work gains 1 MFMA in 12 (the 8-wave kernel then spills 12
  // bytes per lane).  B1 H8 16K d64: dq 0.740 -> 0.720 ms (fp16), 0.702 -> 0.684 ms (bf16); B2 H8
  // 8K 0.384 -> 0.372 ms.
  constexpr bool MFMA_D = !HAS_BIAS && DP <= 64 && RT == 2;
  F ones_a{}, nd_b[MFMA_D ? RT : 1];
  if constexpr (MFMA_D) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) nd_b[rt] = F{};
    if (g == 0) {
      ones_a[0] = static_cast<T>(32768.f);
      ones_a[1] = static_cast<T>(1.f);
      ones_a[2] = static_cast<T>(1.f);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const T b0 = static_cast<T>(-dd[rt] * (1.f / 32768.f));
        const float r = -dd[rt] - static_cast<float>(b0) * 32768.f;
        const T b1 = static_cast<T>(r);
        nd_b[rt][0] = b0;
        nd_b[rt][1] = b1;
        nd_b[rt][2] = static_cast<T>(r - static_cast<float>(b1));
      }
    }
  }

  // element offsets of this thread's staging chunks inside a stage (row strides are
  // below 2^25 elements, checked by the API, so 64 rows fit in 32 bits)
  // (chunk tid + NT i sits NT / CPR rows below chunk tid)
  const int32_t koff0 = (tid / CPR) * (int32_t)p.ks[2] + (tid % CPR) * 8;
  const int32_t voff0 = (tid / CPR) * (int32_t)p.vs[2] + (tid % CPR) * 8;
  // staging registers: set S holds one 64-key stage on its way from global memory to LDS
  Chunk16 kreg[LD ? 1 : 2][LD ? 1 : NCH], vreg[LD ? 1 : 2][LD ? 1 : NCH];
  // LD: a stage tile is 64 padded rows of 9 16-byte slots (8 of data, 1 of padding), 576 slots; the
  // lanes of wave w fill slots 64 (w + WAVES j) .. + 63 for j < LDJ, the last j (slots 512-575) by
  // wave 0 only: slot f holds chunk f % 9 of row f / 9, and a padding slot (f % 9 == 8, never read)
  // takes that row's chunk 0.  Keys past N read as zeros: the buffer range ends at row N (the
  // launcher checks that N rows of K and of V span less than 2^31 bytes).
  constexpr int LDJ = 512 / (64 * WAVES) + 1;
  uint32_t ldk[LD ? LDJ : 1], ldv[LD ? LDJ : 1];
  const uint32_t krb = (uint32_t)p.ks[2] * (uint32_t)sizeof(T), vrb = (uint32_t)p.vs[2] * (uint32_t)sizeof(T);
  const auto rk = make_rsrc(K, LD ? (uint32_t)p.N * krb : 0u);
  const auto rv = make_rsrc(V, LD ? (uint32_t)p.N * vrb : 0u);
  if constexpr (LD) {
#pragma unroll
    for (int j = 0; j < LDJ; ++j) {
      const int f = 64 * (wave + WAVES * j) + lane;
      const int r = f / 9, ch = f % 9 == 8 ? 0 : f % 9;
      ldk[j] = (uint32_t)r * krb + (uint32_t)ch * 16u;
      ldv[j] = (uint32_t)r * vrb + (uint32_t)ch * 16u;
    }
  }
  auto ldload = [&](int t0, T* kdst, T* vdst) {
    if constexpr (LD) {
#pragma unroll
      for (int j = 0; j + 1 < LDJ; ++j) {
        buffer_load16_lds(rk, kdst + 64 * (wave + WAVES * j) * 8, ldk[j] + (uint32_t)t0 * krb);
        buffer_load16_lds(rv, vdst + 64 * (wave + WAVES * j) * 8, ldv[j] + (uint32_t)t0 * vrb);
      }
      if (wave == 0) {
        buffer_load16_lds(rk, kdst + 512 * 8, ldk[LDJ - 1] + (uint32_t)t0 * krb);
        buffer_load16_lds(rv, vdst + 512 * 8, ldv[LDJ - 1] + (uint32_t)t0 * vrb);
      }
    }
  };
  auto gload = [&](int t0, auto SET) {
    if constexpr (LD) return;
    constexpr int S = decltype(SET)::value;
    const T* kt = K + (int64_t)t0 * p.ks[2];
    const T* vt = V + (int64_t)t0 * p.vs[2];
static_for<0, NCH>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const int ci = tid + i * NT;
      const int r = ci / CPR, d0 = (ci % CPR) * 8;
      if (t0 + r < k_end && d0 < p.D) {
        kreg[S][i] = *reinterpret_cast<const Chunk16*>(kt + koff0 + (int64_t)(i * (NT / CPR)) * p.ks[2]);
        vreg[S][i] = *reinterpret_cast<const Chunk16*>(vt + voff0 + (int64_t)(i * (NT / CPR)) * p.vs[2]);
      } else {
        kreg[S][i] = Chunk16{};
        vreg[S][i] = Chunk16{};
      }
    });
  };
  auto sstore = [&](int buf, auto SET) {
    if constexpr (LD) return;
    constexpr int S = decltype(SET)::value;
static_for<0, NCH>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const int ci = tid + i * NT;
      const int r = ci / CPR, d0 = (ci % CPR) * 8;
      *reinterpret_cast<Chunk16*>(&Ks[buf][r * KS + d0]) = kreg[S][i];
      *reinterpret_cast<Chunk16*>(&Vs[buf][r * KS + d0]) = vreg[S][i];
    });
  };

  f32x16 acc[RT][NDT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[rt][dt] = f32x16{};

  const int ntiles = (k_hi - k_lo + KT - 1) / KT;
  // stage keys [t0, t0 + KT) from LDS buffer buf into the dQ accumulators
  auto compute = [&](int t0, const T* ks, const T* vs) __attribute__((always_inline)) {
    if (!p.causal || t0 <= row0 + ROWS_W - 1) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        F kf[NKK], vf[NKK];
        const T* krow = ks + (sub * 32 + swap23(c)) * KS + g * 8;
        const T* vrow = vs + (sub * 32 + swap23(c)) * KS + g * 8;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          kf[kk] = *reinterpret_cast<const F*>(krow + kk * 16);
          vf[kk] = *reinterpret_cast<const F*>(vrow + kk * 16);
        }
        F dsp[RT][2];  // dS of the sub-tile, rounded to T: the B operand of the dQ^T product
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          f32x16 ds;
          f32x16 s = M::mma(kf[0], qf[rt][0], f32x16{}), dp = M::mma(vf[0], gf[rt][0], ndd[rt]);
#pragma unroll
          for (int kk = 1; kk < NKK; ++kk) {
            s = M::mma(kf[kk], qf[rt][kk], s);
            dp = M::mma(vf[kk], gf[rt][kk], dp);
          }
          if constexpr (MFMA_D) dp = M::mma(ones_a, nd_b[rt], dp);
          const int my_row = row0 + rt * 32 + c;
          const bool full = (t0 + KT <= k_end) && (!p.causal || t0 + KT - 1 <= row0 + rt * 32);
          const float nl = -lse[rt];
          if constexpr (HAS_BIAS) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = t0 + sub * 32 + key_of_reg(r, g);
              const bool ok = live[rt] && key < k_end && (!p.causal || key <= my_row);
              const float x = fmaf(s[r], p.scale_log2, nl);
              const float pr = ok ? fast_exp2(fmaf(load_bias_b(p.bias, bi, hi, my_row, key), kLog2e, x)) : 0.f;
              ds[r] = pr * (dp[r] - dd[rt]);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(fmaf(s[r], p.scale_log2, nl));
            if (!full) {
              asm volatile("");  // keep this a branch: boundary tiles only
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int key = t0 + sub * 32 + key_of_reg(r, g);
                if (!(key < k_end && (!p.causal || key <= my_row))) ds[r] = 0.f;
              }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) ds[r] *= (SEED_D || MFMA_D) ? dp[r] : dp[r] - dd[rt];
          }
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int t = 0; t < 8; ++t) dsp[rt][j][t] = static_cast<T>(ds[j * 8 + t]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          F ka[NDT];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) ka[dt] = tr_frag_at<T, Tile>(ks, sub * 32 + 16 * j + tr_row, dt * 32 + tr_col);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[rt][dt] = M::mma(ka[dt], dsp[rt][j], acc[rt][dt]);
        }
      }
    }
  };
  const auto S0 = std::integral_constant<int, 0>{};
  const auto S1 = std::integral_constant<int, 1>{};
  if constexpr (LD) {
    // stage it + 1 goes into the other LDS buffer while stage it computes; all loads land before
    // the barrier that ends the stage
    if (ntiles > 0) ldload(k_lo, Ks[0], Vs[0]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int it = 0; it < ntiles; it += 2) {
      const int t0 = k_lo + it * KT;
      if (it + 1 < ntiles) ldload(t0 + KT, Ks1, Vs1);
      compute(t0, Ks[0], Vs[0]);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (it + 1 < ntiles) {
        if (it + 2 < ntiles) ldload(t0 + 2 * KT, Ks[0], Vs[0]);
        compute(t0 + KT, Ks1, Vs1);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
  } else if constexpr (DP <= 64 && RT == 1) {
    // global loads two stages ahead (as in dK/dV; 16K d64: 0.857 -> 0.842 ms).  At D = 128 the
    // second register set spills at two waves per SIMD, and one wave per SIMD is slower still
    // (1.64 against 1.87-2.07 ms), so that width keeps one stage of prefetch, and so does the
    // two-tile variant (255 VGPRs with one set)
    gload(k_lo, S0);
    sstore(0, S0);
    if (ntiles > 1) gload(k_lo + KT, S1);
    __syncthreads();
    auto step = [&](int it, auto NEXT, auto FREE) __attribute__((always_inline)) {
      const int buf = it & 1;
      const int t0 = k_lo + it * KT;
      if (it + 2 < ntiles) gload(t0 + 2 * KT, FREE);
      compute(t0, Ks[buf], Vs[buf]);
      if (it + 1 < ntiles) sstore(buf ^ 1, NEXT);
      __syncthreads();
    };
    for (int it = 0; it < ntiles; it += 2) {
      step(it, S1, S0);
      if (it + 1 < ntiles) step(it + 1, S0, S1);
    }
  } else {
    gload(k_lo, S0);
    sstore(0, S0);
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
      const int buf = it & 1;
      const int t0 = k_lo + it * KT;
      const bool has_next = it + 1 < ntiles;
      if (has_next) gload(t0 + KT, S0);
      compute(t0, Ks[buf], Vs[buf]);
      if (has_next) sstore(buf ^ 1, S0);
      __syncthreads();
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int my_row = row0 + rt * 32 + c;
    if (my_row >= p.N) continue;
    if (CAN_SPLIT && p.split > 1) {  // this key range's unscaled dQ, fp32
      float* dst = p.part + (((int64_t)wg.z * p.BH + bh) * p.N + my_row) * p.dp;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = dt * 32 + q4 * 8 + 4 * g;
          *reinterpret_cast<f32x4*>(dst + d) =
              f32x4{acc[rt][dt][4 * q4], acc[rt][dt][4 * q4 + 1], acc[rt][dt][4 * q4 + 2], acc[rt][dt][4 * q4 + 3]};
        }
      continue;
    }
    T* out = static_cast<T*>(p.dq) + bi * p.dqs[0] + hi * p.dqs[1] + (int64_t)my_row * p.dqs[2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = dt * 32 + q4 * 8 + 4 * g;
        if (d < p.D) {
          typedef T t4 __attribute__((ext_vector_type(4)));
          t4 v4 = {static_cast<T>(acc[rt][dt][4 * q4] * p.scale), static_cast<T>(acc[rt][dt][4 * q4 + 1] * p.scale),
                   static_cast<T>(acc[rt][dt][4 * q4 + 2] * p.scale), static_cast<T>(acc[rt][dt][4 * q4 + 3] * p.scale)};
          *reinterpret_cast<t4*>(out + d) = v4;
        }
      }
  }
}

// 2 waves per SIMD up to D = 64; at D = 128 the dK/dV accumulators and the wave's K/V
// fragments alone need more than the 256 registers of that budget, so 1 wave per SIMD
// LD (8 waves, D = 64, no bias): the Q and dO stage tiles go straight from global memory into LDS
// (buffer_load_dwordx4 ... lds, one stage ahead) instead of through staging registers.
template <typename T, int DP, int KRT, int WAVES, bool HAS_BIAS, bool LD = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(DP >= 128 ? 1 : 2, 2)))
void bwd_dkdv_half_kernel(const BwdParams p) {
  using M = Mfma<T>;
  typedef typename M::frag F;
  // swizzled tiles in the 8-wave kernel: 16K d64 1.093 -> 1.081 ms (fp16), 1.045 -> 1.028 ms (bf16),
  // causal 0.574 -> 0.564 ms; the 4-wave one has no registers for it
  using Tile = HalfStage<T, DP, true>;
  // rows per stage: 128 in the 8-wave kernel, so that one barrier serves twice the rows (16K d64 dK/dV
  // 1.056 -> 1.042 ms fp16, 1.005 -> 0.992 ms bf16, causal 0.556 -> 0.551 ms; 256 VGPRs, no spill)
  constexpr int RTS = WAVES == 8 ? 128 : Tile::ST, KS = Tile::KS, CPR = Tile::CPR;
  constexpr int NKK = DP / 16, NDT = DP / 32;
  constexpr int NT = 64 * WAVES, KEYS_W = 32 * KRT, BN = KEYS_W * WAVES;
  static_assert((RTS * CPR) % NT == 0, "staging must divide evenly");
  constexpr int NCH = RTS * CPR / NT;
  static_assert(!LD || ((WAVES == 4 || WAVES == 8) && KRT == 1 && DP == 64 && !HAS_BIAS && Tile::SWZ && NCH == 2),
                "LDS-direct staging: the one-tile D = 64 kernels");
  // LD: one array per buffer, so that the compiler sees the loads into one buffer leave the other
  // one's reads alone (with one two-buffer array it waited for them before every stage's reads)
  __shared__ __attribute__((aligned(16))) T Qs[LD ? 1 : 2][RTS * KS];
  __shared__ __attribute__((aligned(16))) T Gs[LD ? 1 : 2][RTS * KS];
  __shared__ __attribute__((aligned(16))) T Qs1[LD ? RTS * KS : 1];
  __shared__ __attribute__((aligned(16))) T Gs1[LD ? RTS * KS : 1];
  __shared__ __attribute__((aligned(16))) float lse_s[2][RTS];
  __shared__ __attribute__((aligned(16))) float ndd_s[2][RTS];  // -D of the stage's rows

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
            g = lane >> 5;
  // causal: the work of a key block shrinks with its index (heaviest first; paired heavy with
  // light where the grid fits in one round)
  const WgCoord wg = (p.causal && WAVES == 4) ? xcd_order_paired() : xcd_order();
  const int bh = wg.y;
  const int wg_key0 = wg.x * BN;
  const int key0 = wg_key0 + wave * KEYS_W;
  const int bi = bh / p.H, hi = bh % p.H;
  const T* Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  const T* V = static_cast<const T*>(p.v) + bi * p.vs[0] + hi * p.vs[1];
  const T* dO = static_cast<const T*>(p.dout) + bi * p.gs[0] + hi * p.gs[1];
  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  // swizzled tiles: this lane's element offsets within a 32-row sub-tile, for its row fragments
  // (row swap23(c), chunk g + 2 kk) and its transposing reads (rows tr_row + 4h, column
  // 32 dt + tr_col); the swizzle reads bits 1-3 of a row only, so they hold in every sub-tile
  int o_row[Tile::SWZ ? NKK : 1], o_tr[Tile::SWZ ? NDT : 1][2];
  if constexpr (Tile::SWZ) {
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) o_row[kk] = Tile::off(swap23(c), g * 8 + kk * 16);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int h = 0; h < 2; ++h) o_tr[dt][h] = Tile::off(tr_row + 4 * h, dt * 32 + tr_col);
  }

  F kf[KRT][NKK], vf[KRT][NKK];
  bool key_ok[KRT];
#pragma unroll
  for (int kt = 0; kt < KRT; ++kt) {
    const int key = key0 + kt * 32 + c;
    key_ok[kt] = key < p.N;
    const int ksafe = key_ok[kt] ? key : 0;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const int d0 = kk * 16 + g * 8;
      kf[kt][kk] = load_frag<T>(K + (int64_t)ksafe * p.ks[2] + d0, key_ok[kt] && d0 < p.D);
      vf[kt][kk] = load_frag<T>(V + (int64_t)ksafe * p.vs[2] + d0, key_ok[kt] && d0 < p.D);
    }
  }
  f32x16 dk[KRT][NDT], dv[KRT][NDT];
#pragma unroll
  for (int kt = 0; kt < KRT; ++kt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      dk[kt][dt] = f32x16{};
      dv[kt][dt] = f32x16{};
    }

  // element offsets of this thread's staging chunks inside a stage (row strides are
  // below 2^25 elements, checked by the API, so the 128 rows of a stage fit in 32 unsigned bits)
  uint32_t qoff[NCH], goff[NCH];
  static_for<0, NCH>([&](auto I) {
    constexpr int i = decltype(I)::value;
    const int ci = tid + i * NT;
    const int r = ci / CPR, d0 = (ci % CPR) * 8;
    qoff[i] = (uint32_t)r * (uint32_t)p.qs[2] + (uint32_t)d0;
    goff[i] = (uint32_t)r * (uint32_t)p.gs[2] + (uint32_t)d0;
  });
  // staging registers: set S holds one stage (RTS rows) on its way from global memory to LDS
  Chunk16 qreg[LD ? 1 : 2][LD ? 1 : NCH], greg[LD ? 1 : 2][LD ? 1 : NCH];
  float lreg[2] = {0.f, 0.f}, dreg[2] = {0.f, 0.f};
  // LD: lane l of wave w fills the 16 bytes at LDS byte 16 (64 w + 64 WAVES i + l) of a stage tile
  // for i = 0, 1: row 8 w + 8 WAVES i + l / 8 of the stage, swizzle slot l % 8, which holds chunk
  // (l % 8) ^ lds_swz(row) of that row.  Rows past N read as zeros: the buffer range ends at row N
  // (the launcher checks that N rows of Q and of dO span less than 2^31 bytes).
  uint32_t ldq[LD ? NCH : 1], ldg[LD ? NCH : 1];
  const uint32_t qrb = (uint32_t)p.qs[2] * (uint32_t)sizeof(T), grb = (uint32_t)p.gs[2] * (uint32_t)sizeof(T);
  const auto rq = make_rsrc(Q, LD ? (uint32_t)p.N * qrb : 0u);
  const auto rg = make_rsrc(dO, LD ? (uint32_t)p.N * grb : 0u);
  if constexpr (LD) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int r = 8 * wave + 8 * WAVES * i + (lane >> 3);
      const uint32_t ch = (uint32_t)((lane & 7) ^ lds_swz(r));
      ldq[i] = (uint32_t)r * qrb + ch * 16u;
      ldg[i] = (uint32_t)r * grb + ch * 16u;
    }
  }
  auto ldload = [&](int t0, T* qdst, T* gdst) {
    if constexpr (LD) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        buffer_load16_lds(rq, qdst + (64 * wave + 64 * WAVES * i) * 8, ldq[i] + (uint32_t)t0 * qrb);
        buffer_load16_lds(rg, gdst + (64 * wave + 64 * WAVES * i) * 8, ldg[i] + (uint32_t)t0 * grb);
      }
      // rows past N: LSE2 = +inf makes their p exactly 0.  D is negated at the store, so that no
      // instruction here waits for these loads (and with them for the LDS loads issued before)
      if (tid < RTS) {
        const int ra = t0 + tid;
        lreg[0] = ra < p.N ? p.lse_row[(int64_t)bh * p.N + ra] : __builtin_huge_valf();
        dreg[0] = ra < p.N ? p.d_row[(int64_t)bh * p.N + ra] : 0.f;
      }
    }
  };
  auto ldstore = [&](int buf) {
    if (tid < RTS) {
      lse_s[buf][tid] = lreg[0];
      ndd_s[buf][tid] = -dreg[0];
    }
  };
  auto gload = [&](int t0, auto SET) {
    if constexpr (LD) return;
    constexpr int S = decltype(SET)::value;
    const T* qt = Q + (int64_t)t0 * p.qs[2];
    const T* gt = dO + (int64_t)t0 * p.gs[2];
static_for<0, NCH>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const int ci = tid + i * NT;
      const int r = ci / CPR, d0 = (ci % CPR) * 8;
      if (t0 + r < p.N && d0 < p.D) {
        qreg[S][i] = *reinterpret_cast<const Chunk16*>(qt + qoff[i]);
        greg[S][i] = *reinterpret_cast<const Chunk16*>(gt + goff[i]);
      } else {
        qreg[S][i] = Chunk16{};
        greg[S][i] = Chunk16{};
      }
    });
    if (tid < RTS) {  // rows past N: LSE2 = +inf makes their p exactly 0
      const int ra = t0 + tid;
      lreg[S] = ra < p.N ? p.lse_row[(int64_t)bh * p.N + ra] : __builtin_huge_valf();
      dreg[S] = ra < p.N ? -p.d_row[(int64_t)bh * p.N + ra] : 0.f;
    }
  };
  auto sstore = [&](int buf, auto SET) {
    if constexpr (LD) return;
    constexpr int S = decltype(SET)::value;
static_for<0, NCH>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const int ci = tid + i * NT;
      const int r = ci / CPR, d0 = (ci % CPR) * 8;
      const int lo = Tile::SWZ ? Tile::off(r, d0) : r * KS + d0;
      *reinterpret_cast<Chunk16*>(&Qs[buf][lo]) = qreg[S][i];
      *reinterpret_cast<Chunk16*>(&Gs[buf][lo]) = greg[S][i];
    });
    if (tid < RTS) {
      lse_s[buf][tid] = lreg[S];
      ndd_s[buf][tid] = dreg[S];
    }
  };

  // split (the 4-wave one-tile kernel only): this work-group's rows [r_lo, r_hi), whole 64-row
  // stages (one range when unsplit)
  constexpr bool CAN_SPLIT = KRT == 1 && WAVES == 4 && !HAS_BIAS && DP <= 64;
  const int r_lo = max(p.causal ? (wg_key0 / RTS) * RTS : 0, CAN_SPLIT ? wg.z * p.split_len : 0);
  const int r_hi = CAN_SPLIT ? min(p.N, wg.z * p.split_len + p.split_len) : p.N;
  const int ntiles = r_hi > r_lo ? (r_hi - r_lo + RTS - 1) / RTS : 0;
  // a causal row range before this key block's first row adds nothing: no partials are written,
  // and the combine (bwd_combine_kernel, kind 2) skips the same ranges
  if (CAN_SPLIT && p.split > 1 && p.causal && ntiles == 0) return;
  // stage rows [t0, t0 + RTS) from LDS buffer buf into the dK / dV accumulators
  auto compute = [&](int buf, int t0, const T* qs, const T* gs) __attribute__((always_inline)) {
    if (!p.causal || t0 + RTS - 1 >= key0) {
#pragma unroll
      for (int sub = 0; sub < RTS / 32; ++sub) {
        F qa[NKK], ga[NKK];
        if constexpr (Tile::SWZ) {
#pragma unroll
          for (int kk = 0; kk < NKK; ++kk) {
            qa[kk] = *reinterpret_cast<const F*>(qs + sub * 32 * KS + o_row[kk]);
            ga[kk] = *reinterpret_cast<const F*>(gs + sub * 32 * KS + o_row[kk]);
          }
        } else {
          const T* qrow = qs + (sub * 32 + swap23(c)) * KS + g * 8;
          const T* grow = gs + (sub * 32 + swap23(c)) * KS + g * 8;
#pragma unroll
          for (int kk = 0; kk < NKK; ++kk) {
            qa[kk] = *reinterpret_cast<const F*>(qrow + kk * 16);
            ga[kk] = *reinterpret_cast<const F*>(grow + kk * 16);
          }
        }
        // transposed Q^T / dO^T fragments for the dK / dV products, shared by the KRT key tiles
        F gta[2][NDT], qta[2][NDT];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            if constexpr (Tile::SWZ) {
              gta[j][dt] = tr_frag_off<T>(gs + (sub * 32 + 16 * j) * KS, o_tr[dt][0], o_tr[dt][1]);
              qta[j][dt] = tr_frag_off<T>(qs + (sub * 32 + 16 * j) * KS, o_tr[dt][0], o_tr[dt][1]);
            } else {
              gta[j][dt] = tr_frag_at<T, Tile>(gs, sub * 32 + 16 * j + tr_row, dt * 32 + tr_col);
              qta[j][dt] = tr_frag_at<T, Tile>(qs, sub * 32 + 16 * j + tr_row, dt * 32 + tr_col);
            }
          }
        // -D of the rows of registers 8j..8j+7 (sub*32 + 16j + 8g + t): the dP^T product starts
        // from it and yields dP - D directly
        f32x16 ndd;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float* e8 = &ndd_s[buf][sub * 32 + 16 * j + 8 * g];
          const f32x4 e0 = *reinterpret_cast<const f32x4*>(e8), e1 = *reinterpret_cast<const f32x4*>(e8 + 4);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            ndd[8 * j + t] = e0[t];
            ndd[8 * j + 4 + t] = e1[t];
          }
        }
#pragma unroll
        for (int kt = 0; kt < KRT; ++kt) {
          f32x16 s = M::mma(qa[0], kf[kt][0], f32x16{}), dp = M::mma(ga[0], vf[kt][0], ndd);
#pragma unroll
          for (int kk = 1; kk < NKK; ++kk) {
            s = M::mma(qa[kk], kf[kt][kk], s);
            dp = M::mma(ga[kk], vf[kt][kk], dp);
          }
          const int my_key = key0 + kt * 32 + c;
          const bool full = (key0 + kt * 32 + 31 < p.N) && (t0 + RTS <= p.N) && (!p.causal || t0 + sub * 32 >= key0 + kt * 32 + 31);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            // rows of registers 8j..8j+7: sub*32 + 16j + 8g + t (consecutive)
            const float* lp = &lse_s[buf][sub * 32 + 16 * j + 8 * g];
            const f32x4 l0 = *reinterpret_cast<const f32x4*>(lp), l1 = *reinterpret_cast<const f32x4*>(lp + 4);
            float pr[8];
            if constexpr (HAS_BIAS) {
#pragma unroll
              for (int t = 0; t < 8; ++t) {
                const int row = t0 + sub * 32 + key_of_reg(8 * j + t, g);
                const float lr = t < 4 ? l0[t] : l1[t - 4];
                const bool ok = key_ok[kt] && row < p.N && (!p.causal || row >= my_key);
                const float x = fmaf(s[8 * j + t], p.scale_log2, -lr);
                pr[t] = ok ? fast_exp2(fmaf(load_bias_b(p.bias, bi, hi, row, my_key), kLog2e, x)) : 0.f;
              }
              if (p.ds_out != nullptr && key_ok[kt]) {  // lanes of one t: 32 consecutive keys of a row
                float* dso = p.ds_out + (int64_t)bh * p.N * p.N + my_key;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                  const int row = t0 + sub * 32 + key_of_reg(8 * j + t, g);
                  if (row < p.N) dso[(int64_t)row * p.N] = pr[t] * dp[8 * j + t];
                }
              }
            } else {
#pragma unroll
              for (int t = 0; t < 8; ++t) pr[t] = fast_exp2(fmaf(s[8 * j + t], p.scale_log2, t < 4 ? -l0[t] : -l1[t - 4]));
              if (!full) {
                asm volatile("");  // keep this a branch: boundary tiles only
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                  const int row = t0 + sub * 32 + key_of_reg(8 * j + t, g);
                  if (!(key_ok[kt] && row < p.N && (!p.causal || row >= my_key))) pr[t] = 0.f;
                }
              }
            }
            F bp, bs;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              bp[t] = static_cast<T>(pr[t]);
              bs[t] = static_cast<T>(pr[t] * dp[8 * j + t]);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
              dv[kt][dt] = M::mma(gta[j][dt], bp, dv[kt][dt]);
              dk[kt][dt] = M::mma(qta[j][dt], bs, dk[kt][dt]);
            }
          }
        }
      }
    }
  };
  const auto S0 = std::integral_constant<int, 0>{};
  const auto S1 = std::integral_constant<int, 1>{};
  if constexpr (LD) {
    // stage it + 1 goes into the other LDS buffer while stage it computes (that buffer was last
    // read by stage it - 1, before the barrier that ended it); all loads land before the barrier
    if (ntiles > 0) {
      ldload(r_lo, Qs[0], Gs[0]);
      ldstore(0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int it = 0; it < ntiles; it += 2) {
      const int t0 = r_lo + it * RTS;
      if (it + 1 < ntiles) ldload(t0 + RTS, Qs1, Gs1);
      compute(0, t0, Qs[0], Gs[0]);
      if (it + 1 < ntiles) ldstore(1);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (it + 1 < ntiles) {
        if (it + 2 < ntiles) ldload(t0 + 2 * RTS, Qs[0], Gs[0]);
        compute(1, t0 + RTS, Qs1, Gs1);
        if (it + 2 < ntiles) ldstore(0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
  } else {
  // global loads two stages ahead: stage it + 2 goes into the register set that stage it
  // left, while stage it + 1 waits in the other one for the end of this stage
  gload(r_lo, S0);
  sstore(0, S0);
  if (ntiles > 1) gload(r_lo + RTS, S1);
  __syncthreads();
  auto step = [&](int it, auto NEXT, auto FREE) __attribute__((always_inline)) {
    const int buf = it & 1;
    const int t0 = r_lo + it * RTS;
    if (it + 2 < ntiles) gload(t0 + 2 * RTS, FREE);
    compute(buf, t0, Qs[buf], Gs[buf]);
    if (it + 1 < ntiles) sstore(buf ^ 1, NEXT);
    __syncthreads();
  };
  for (int it = 0; it < ntiles; it += 2) {
    step(it, S1, S0);
    if (it + 1 < ntiles) step(it + 1, S0, S1);
  }
  }
#pragma unroll
  for (int kt = 0; kt < KRT; ++kt) {
    const int my_key = key0 + kt * 32 + c;
    if (my_key >= p.N) continue;
    if (CAN_SPLIT && p.split > 1) {  // this row range's unscaled dK and dV, fp32
      float* dkp = p.part + p.part_stride + (((int64_t)wg.z * p.BH + bh) * p.N + my_key) * p.dp;
      float* dvp = dkp + p.part_stride;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = dt * 32 + q4 * 8 + 4 * g;
          *reinterpret_cast<f32x4*>(dkp + d) = f32x4{dk[kt][dt][4 * q4], dk[kt][dt][4 * q4 + 1], dk[kt][dt][4 * q4 + 2],
                                                     dk[kt][dt][4 * q4 + 3]};
          *reinterpret_cast<f32x4*>(dvp + d) = f32x4{dv[kt][dt][4 * q4], dv[kt][dt][4 * q4 + 1], dv[kt][dt][4 * q4 + 2],
                                                     dv[kt][dt][4 * q4 + 3]};
        }
      continue;
    }
    T* okp = static_cast<T*>(p.dk) + bi * p.dks[0] + hi * p.dks[1] + (int64_t)my_key * p.dks[2];
    T* ovp = static_cast<T*>(p.dv) + bi * p.dvs[0] + hi * p.dvs[1] + (int64_t)my_key * p.dvs[2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = dt * 32 + q4 * 8 + 4 * g;
        if (d < p.D) {
          typedef T t4 __attribute__((ext_vector_type(4)));
          t4 k4 = {static_cast<T>(dk[kt][dt][4 * q4] * p.scale), static_cast<T>(dk[kt][dt][4 * q4 + 1] * p.scale),
                   static_cast<T>(dk[kt][dt][4 * q4 + 2] * p.scale), static_cast<T>(dk[kt][dt][4 * q4 + 3] * p.scale)};
          t4 v4 = {static_cast<T>(dv[kt][dt][4 * q4]), static_cast<T>(dv[kt][dt][4 * q4 + 1]),
                   static_cast<T>(dv[kt][dt][4 * q4 + 2]), static_cast<T>(dv[kt][dt][4 * q4 + 3])};
          *reinterpret_cast<t4*>(okp + d) = k4;
          *reinterpret_cast<t4*>(ovp + d) = v4;
        }
      }
  }
}

// ------------------------------------------------------------------ row stats
template <typename T, int DP, int WAVES, bool HAS_BIAS>
__global__ __launch_bounds__(64 * WAVES) void row_stats_kernel(const BwdParams p, float* row_m, float* row_z) {
  using C = BwdCfg<T, DP>;
  using M = Mfma<T>;
  typedef typename M::frag F;
  constexpr int NT = 64 * WAVES, BM = 32 * WAVES;
  __shared__ __attribute__((aligned(16))) T Ks[C::HALF ? C::TT * C::RS : 1];
  __shared__ __attribute__((aligned(16))) T Kt[C::HALF ? 1 : DP * C::TS];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, c = lane & 31,
            g = lane >> 5;
  WgCoord wg = xcd_order();
  if (p.causal) wg.x = (int)gridDim.x - 1 - wg.x;  // causal: heaviest row blocks first
  const int bh = wg.y;
  const int wg_row0 = wg.x * BM;
  const int wg_last = min(p.N, wg_row0 + BM) - 1;
  const int my_row = wg_row0 + wave * 32 + c;
  const bool row_ok = my_row < p.N;
  const int bi = bh / p.H, hi = bh % p.H;
  const T* Q = static_cast<const T*>(p.q) + bi * p.qs[0] + hi * p.qs[1];
  const T* K = static_cast<const T*>(p.k) + bi * p.ks[0] + hi * p.ks[1];
  F qf[C::NKK];
#pragma unroll
  for (int kk = 0; kk < C::NKK; ++kk) {
    const int d0 = kk * C::KSTEP + g * C::KP;
    qf[kk] = load_frag<T>(Q + (int64_t)(row_ok ? my_row : 0) * p.qs[2] + d0, row_ok && d0 < p.D);
  }
  float m_run = kNegInf, z_lane = 0.f;
  const int k_end = p.causal ? wg_last + 1 : p.N;
  for (int t0 = 0; t0 < k_end; t0 += C::TT) {
    __syncthreads();
    stage_tile<T, DP, NT, C::HALF, !C::HALF>(K, p.ks[2], t0, k_end, p.D, Ks, Kt, tid);
    __syncthreads();
    f32x16 s = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::NKK; ++kk) s = M::mma(a_frag<T, DP>(Ks, Kt, c, g, kk), qf[kk], s);
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t0 + key_of_reg(r, g);
      const bool ok = row_ok && key < k_end && (!p.causal || key <= my_row);
      float x = s[r] * p.scale_log2;
      if constexpr (HAS_BIAS) x = ok ? fmaf(load_bias_b(p.bias, bi, hi, my_row, key), kLog2e, x) : x;
      s[r] = ok ? x : kNegInf;
      mx = fmaxf(mx, s[r]);
    }
    mx = wave_max_pair(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    float zs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) zs += fast_exp2(s[r] - m_use);
    z_lane = fmaf(z_lane, fast_exp2(m_run - m_use), zs);
    m_run = m_new;
  }
  const float z = wave_sum_pair(z_lane);
  if (row_ok && g == 0) {
    row_m[(int64_t)bh * p.N + my_row] = z > 0.f ? m_run : kNegInf;
    row_z[(int64_t)bh * p.N + my_row] = z;
  }
}

// ------------------------------------------------------------------ dbias
// One wave per 32x32 (row, key) tile of one (b', h'); operands straight from HBM.
template <typename T, int DP>
// Grid: x = 32x32 output tile, y = bias head, z = bias batch x nsplit.  The sum over the
// broadcast (b, h) pairs is cut into nsplit contiguous ranges; with nsplit > 1 each range
// writes its partial tile to part[split] and dbias_reduce_kernel adds them in order.
__global__ __launch_bounds__(64) void dbias_kernel(const BwdParams p, float* dbias, int bias_batch, int bias_heads,
                                                   int nsplit, float* part) {
  using C = BwdCfg<T, DP>;
  using M = Mfma<T>;
  const int lane = threadIdx.x, c = lane & 31, g = lane >> 5;
  const int tiles = (p.N + 31) / 32;
  const int ti = blockIdx.x / tiles, tj = blockIdx.x % tiles;
  const int hb = blockIdx.y, bb = blockIdx.z / nsplit, split = blockIdx.z - bb * nsplit;
  const int my_row = ti * 32 + c;
  const int krow = tj * 32 + swap23(c);  // key loaded by this lane for the A operand
  const bool row_ok = my_row < p.N, krow_ok = krow < p.N;
  const int B = p.BH / p.H;
  const int b_lo = bias_batch == 1 ? 0 : bb, nb = bias_batch == 1 ? B : 1;
  const int h_lo = bias_heads == 1 ? 0 : hb, nh = bias_heads == 1 ? p.H : 1;
  const int64_t pairs = (int64_t)nb * nh;
  const int64_t r_lo = pairs * split / nsplit, r_hi = pairs * (split + 1) / nsplit;
  f32x16 acc = f32x16{};
  for (int64_t pair = r_lo; pair < r_hi; ++pair) {
    {
      const int b = b_lo + (int)(pair / nh), h = h_lo + (int)(pair % nh);
      const int bh = b * p.H + h;
      const T* Q = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1];
      const T* K = static_cast<const T*>(p.k) + b * p.ks[0] + h * p.ks[1];
      const T* V = static_cast<const T*>(p.v) + b * p.vs[0] + h * p.vs[1];
      const T* dO = static_cast<const T*>(p.dout) + b * p.gs[0] + h * p.gs[1];
      // S and dP over the head dim in NC interleaved accumulator chains, added at the end:
      // the fp32 MFMA adds two products per step, and one chain over d = 32 rounded 16 times
      // at the magnitude of dP (~8: 1e-6 per rounding), about as much as everything else in
      // a dS entry's fp32 error together
      constexpr int NC = C::NKK >= 8 ? 4 : (C::NKK >= 2 ? 2 : 1);
      f32x16 sc[NC], dc[NC];
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        sc[i] = f32x16{};
        dc[i] = f32x16{};
      }
#pragma unroll
      for (int kk = 0; kk < C::NKK; ++kk) {
        const int d0 = kk * C::KSTEP + g * C::KP;
        const bool dok = d0 < p.D;
        const auto qb = load_frag<T>(Q + (int64_t)(row_ok ? my_row : 0) * p.qs[2] + d0, row_ok && dok);
        const auto gb = load_frag<T>(dO + (int64_t)(row_ok ? my_row : 0) * p.gs[2] + d0, row_ok && dok);
        const auto ka = load_frag<T>(K + (int64_t)(krow_ok ? krow : 0) * p.ks[2] + d0, krow_ok && dok);
        const auto va = load_frag<T>(V + (int64_t)(krow_ok ? krow : 0) * p.vs[2] + d0, krow_ok && dok);
        sc[kk % NC] = M::mma(ka, qb, sc[kk % NC]);
        dc[kk % NC] = M::mma(va, gb, dc[kk % NC]);
      }
#pragma unroll
      for (int w = NC / 2; w >= 1; w /= 2)
#pragma unroll
        for (int i = 0; i < w; ++i) {
          sc[i] += sc[i + w];
          dc[i] += dc[i + w];
        }
      const f32x16& s = sc[0];
      const f32x16& dp = dc[0];
      const float lse = row_ok ? p.lse_row[(int64_t)bh * p.N + my_row] : kNegInf;
      const float lse_lo = row_ok ? p.lse_lo[(int64_t)bh * p.N + my_row] : 0.f;
      const float dd = row_ok ? p.d_row[(int64_t)bh * p.N + my_row] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = tj * 32 + key_of_reg(r, g);
        bool ok = row_ok && key < p.N && lse > kNegInf && (!p.causal || key <= my_row);
        // s*c - LSE2 rounded once (then LSE2's low part), before the bias: as the dq and dk/dv kernels
        const float x = fmaf(s[r], p.scale_log2, -lse) - lse_lo;
        const float pr = ok ? fast_exp2(fmaf(load_bias_b(p.bias, b, h, my_row, key), kLog2e, x)) : 0.f;
        acc[r] += pr * (dp[r] - dd);
      }
    }
  }
  if (!row_ok) return;
  const int64_t plane = (int64_t)bias_batch * bias_heads * p.N * p.N;
  float* outp = (nsplit == 1 ? dbias : part + split * plane) + (((int64_t)bb * bias_heads + hb) * p.N + my_row) * p.N;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = tj * 32 + key_of_reg(r, g);
    if (key < p.N) outp[key] = acc[r];
  }
}

// dbias = sum over split of part[split], in split order (deterministic).
__global__ __launch_bounds__(256) void dbias_reduce_kernel(const float* part, float* dbias, int nsplit, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float acc = 0.f;
  for (int sp = 0; sp < nsplit; ++sp) acc += part[sp * n + i];
  dbias[i] = acc;
}

// dbias[bb', hb', i, j] = sum over the (b, h) pairs broadcast onto (bb', hb') of ds[b, h, i, j].
// The pairs (b-major, increasing) are cut into nsplit contiguous ranges; each range's sum goes
// to part[split] (to dbias when nsplit == 1) and dbias_reduce_kernel adds the ranges in order,
// so the result does not depend on scheduling.  grid: x = blocks of 256 elements of one
// (bb', hb') plane, y = bias head, z = bias batch x nsplit.
__global__ __launch_bounds__(256) void dbias_sum_kernel(const float* __restrict__ ds, float* __restrict__ dbias,
                                                        int B, int H, int N, int bias_batch, int bias_heads, int nsplit,
                                                        float* __restrict__ part) {
  const int64_t nn = (int64_t)N * N;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= nn) return;
  const int hb = blockIdx.y, bb = blockIdx.z / nsplit, split = blockIdx.z - bb * nsplit;
  const int b_lo = bias_batch == 1 ? 0 : bb, nb = bias_batch == 1 ? B : 1;
  const int h_lo = bias_heads == 1 ? 0 : hb, nh = bias_heads == 1 ? H : 1;
  const int64_t pairs = (int64_t)nb * nh;
  const int64_t r_lo = pairs * split / nsplit, r_hi = pairs * (split + 1) / nsplit;
  float acc = 0.f;
  for (int64_t r = r_lo; r < r_hi; ++r) {
    const int b = b_lo + (int)(r / nh), h = h_lo + (int)(r % nh);
    acc += ds[((int64_t)b * H + h) * nn + e];
  }
  const int64_t plane = (int64_t)bias_batch * bias_heads * nn;
  (nsplit == 1 ? dbias : part + split * plane)[((int64_t)bb * bias_heads + hb) * nn + e] = acc;
}

__global__ __launch_bounds__(256) void zero_fill_kernel(float* dst, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 3 < n) {
    *reinterpret_cast<f32x4*>(dst + i) = f32x4{};
  } else {
    for (int64_t k = i; k < n; ++k) dst[k] = 0.f;
  }
}

int dbias_sum_splits(int B, int H, int bias_batch, int bias_heads) {
  const int64_t pairs = (int64_t)(bias_batch == 1 ? B : 1) * (bias_heads == 1 ? H : 1);
  return (int)std::max<int64_t>(1, std::min<int64_t>(256, (pairs + 63) / 64));  // ranges of about 64 pairs
}

hipError_t launch_dbias_sum(const float* ds, float* dbias, int B, int H, int N, int bias_batch, int bias_heads,
                            float* part, hipStream_t st) {
  const int64_t nn = (int64_t)N * N;
  const int nsplit = part ? dbias_sum_splits(B, H, bias_batch, bias_heads) : 1;
  hipLaunchKernelGGL(dbias_sum_kernel,
                     dim3((unsigned)((nn + 255) / 256), (unsigned)bias_heads, (unsigned)(bias_batch * nsplit)),
                     dim3(256), 0, st, ds, dbias, B, H, N, bias_batch, bias_heads, nsplit, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  const int64_t n = (int64_t)bias_batch * bias_heads * nn;
  hipLaunchKernelGGL(dbias_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, dbias, nsplit, n);
  return hipGetLastError();
}

hipError_t launch_zero_fill(float* dst, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, dst, n);
  return hipGetLastError();
}

// ------------------------------------------------------------------ split backward
// Work-groups of a causal backward split into s ranges that hold work: a 128-row block's dq covers
// the keys below k_end = min(n, 128 * (block + 1)), so its ranges from ceil(k_end / split_len) on
// return at once (the dK/dV grid mirrors this count).
static int64_t causal_live_wgs(int64_t bh, int64_t n, int s) {
  const int64_t len = ((n + s - 1) / s + 31) / 32 * 32;  // the fp32 split_len: whole 32-key stages
  int64_t live = 0;
  for (int64_t b0 = 0; b0 < n; b0 += 128) live += (std::min(n, b0 + 128) + len - 1) / len;
  return bh * live;
}

int bwd_splits(int dtype, int dp, int64_t bh, int64_t n, bool bias, bool causal) {
  if (bias || dp > 64) return 1;
  const int64_t wgs = bh * ((n + 127) / 128);  // the unsplit 4-wave grid
  // double while the doubled grid stays within one round of 512 work-groups (two per CU): whole
  // backward, fp16 d64, against doubling while the grid was short of 512: B8 H3 N1025 0.083 ->
  // 0.065 ms (4 -> 2 ranges), causal 0.073 -> 0.057, B8 H3 N2305 0.188 -> 0.170 (2 -> 1), causal
  // 0.150 -> 0.119, B16 H3 N1025 0.115 -> 0.087 (2 -> 1); fp32 B8 H3 N1025 0.394 -> 0.339 ms.
  // Ranges stay at least 256 keys or rows for fp16 and bf16 (128: B1 H8 N1024 0.038 -> 0.044 ms)
  // and 64 for fp32, whose stages take several times longer (against 256: B8 H3 N197 0.089 ->
  // 0.064 ms, B1 H8 N512 0.103 -> 0.061, B2 H3 N300 0.118 -> 0.064; 128 gave 0.089, 0.069, 0.082)
  // Causal fp32 calls count only the work-groups that hold work (the others return at once): the
  // doubling splits the longest rows' key ranges, and an fp32 stage is long enough that those set
  // the time.  Against the count of every work-group: B1 H8 N1025 0.202 -> 0.162 ms (4 -> 8 ranges),
  // B2 H8 N2049 0.895 -> 0.571 (1 -> 2), B1 H8 N4097 1.305 -> 1.098, N5000 1.773 -> 1.333, N3000
  // 0.800 -> 0.723 (2 -> 4).  fp16 went both ways (B2 H8 N2049 0.103 -> 0.085 ms, but B1 H12 N2048
  // 0.076 -> 0.083 and B1 H8 N5000 0.169 -> 0.177), so 16-bit calls count every work-group.
  const int64_t min_range = dtype == ELSA_F32 ? 64 : 256;
  const bool live_only = causal && dtype == ELSA_F32 && wgs <= 512;
  int s = 1;
  while (s < 8 && n / (2 * s) >= min_range &&
         (wgs * s * 2 <= 512 || (live_only && causal_live_wgs(bh, n, 2 * s) <= 512)))
    s *= 2;
  return s;
}

// out[b, h, n, d] = scale * sum over the split ranges of part[z][b*H + h][n][d], 4 head-dim
// elements per thread (head dims are multiples of 8); grid y picks one of up to three such sums.
// kind 0 sums every range.  Causal calls skip the ranges whose work-groups wrote nothing (the
// split kernels are the 4-wave ones: 128 rows or keys per work-group):
//   kind 1 (dQ of row n): key ranges z with z * split_len >= k_end = min(N, 128 * (n / 128 + 1));
//   kind 2 (dK, dV of key n): row ranges z with (z + 1) * split_len <= 128 * (n / 128).
// Every kind skips ranges that start at or past N.  Those ranges would add zeros, so the sums are
// the same up to the sign of a zero.
struct CombineOut {
  const float* part;
  void* out;
  int64_t os[3];
  float scale;
  int kind;
};
template <typename T>
__global__ __launch_bounds__(256) void bwd_combine_kernel(CombineOut c0, CombineOut c1, CombineOut c2, int split,
                                                          int split_len, int64_t sstride, int H, int N, int D,
                                                          int dp) {
  const CombineOut& cj = blockIdx.y == 0 ? c0 : (blockIdx.y == 1 ? c1 : c2);
  const float* __restrict__ part = cj.part;
  T* __restrict__ out = static_cast<T*>(cj.out);
  const int64_t o0 = cj.os[0], o1 = cj.os[1], o2 = cj.os[2];
  const float scale = cj.scale;
  const int c4 = D / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = i / c4;  // over B*H*N
  if (row >= sstride / dp) return;
  const int d = (int)(i - row * c4) * 4;
  const int64_t bh = row / N, n = row - bh * N;
  // ranges that start at or past N (split_len is rounded up to whole stages) hold nothing either
  int z_lo = 0, z_hi = min(split, (N + split_len - 1) / split_len);
  if (cj.kind == 1) {
    const int k_end = min(N, 128 * ((int)n / 128 + 1));
    z_hi = min(z_hi, (k_end + split_len - 1) / split_len);
  } else if (cj.kind == 2) {
    z_lo = 128 * ((int)n / 128) / split_len;  // < z_hi: 128 * (n / 128) <= n < N
  }
  const float* src = part + row * dp + d;
  f32x4 acc = *reinterpret_cast<const f32x4*>(src + z_lo * sstride);
  for (int z = z_lo + 1; z < z_hi; ++z) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + z * sstride);
    acc[0] += v[0];
    acc[1] += v[1];
    acc[2] += v[2];
    acc[3] += v[3];
  }
  typedef T t4 __attribute__((ext_vector_type(4)));
  const t4 o = {static_cast<T>(acc[0] * scale), static_cast<T>(acc[1] * scale), static_cast<T>(acc[2] * scale),
                static_cast<T>(acc[3] * scale)};
  *reinterpret_cast<t4*>(out + (bh / H) * o0 + (bh % H) * o1 + n * o2 + d) = o;
}

// one launch for up to three sums (n = 1, 2 or 3 of c[0..2])
template <typename T>
static hipError_t combine_launch(const BwdParams& p, const CombineOut* c, int n, hipStream_t st) {
  const int64_t rows = (int64_t)p.BH * p.N;
  const int64_t threads = rows * (p.D / 4);
  hipLaunchKernelGGL(bwd_combine_kernel<T>, dim3((unsigned)((threads + 255) / 256), (unsigned)n), dim3(256), 0, st,
                     c[0], c[n > 1 ? 1 : 0], c[n > 2 ? 2 : 0], p.split, p.split_len, rows * p.dp, p.H, p.N, p.D,
                     p.dp);
  return hipGetLastError();
}

// ------------------------------------------------------------------ launchers
template <typename T>
static hipError_t pre_launch(const BwdParams& p, hipStream_t st) {
  hipLaunchKernelGGL(bwd_pre_kernel<T>, dim3((unsigned)((p.N + 31) / 32), (unsigned)p.BH), dim3(256), 0, st, p);
  return hipGetLastError();
}

// fp16/bf16 kernels: 32 rows (dq) or 32 keys (dk/dv) per wave, 4 waves per
// workgroup, register budget capped for 2 waves per SIMD (measured on MI355X at
// B1 H8 N16K d64: dq 1.36 ms / dk-dv 1.68 ms versus 2.27 / 2.76 ms with 64-wide
// wave tiles at 1 wave per SIMD).  fp32 keeps the 32-wide kernels above.
// Sequences of at most 64 rows at head dims up to 32 (Swin's 49-token windows): 2-wave
// work-groups of 64 rows or keys, so that no wave of a work-group lies wholly past N (with 4
// waves of 32, waves 2 and 3 only staged and waited).  The split backward never applies there
// (bwd_splits).  Wider heads keep 4 waves: at D = 64 the 2-wave fp16/bf16 dK/dV kernel spills
// (its staging share per thread doubles) and the fp32 one drops to 1 wave per SIMD.
template <typename T, int DP, bool B>
static hipError_t bwd_launch_short(const BwdParams& p, int stage, hipStream_t st) {
  constexpr int W = 2;
  const dim3 grid((p.N + 32 * W - 1) / (32 * W), p.BH);
  hipError_t e = hipSuccess;
  if (stage < 0 || stage == 1) {
    if constexpr (sizeof(T) == 2) {
      hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, 1, W, B>), grid, dim3(64 * W), 0, st, p);
    } else {
      hipLaunchKernelGGL((bwd_dq_kernel<T, DP, W, B>), grid, dim3(64 * W), 0, st, p);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (stage < 0 || stage == 2) {
    if constexpr (sizeof(T) == 2) {
      hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, 1, W, B>), grid, dim3(64 * W), 0, st, p);
    } else {
      hipLaunchKernelGGL((bwd_dkdv_kernel<T, DP, W, B>), grid, dim3(64 * W), 0, st, p);
    }
    e = hipGetLastError();
  }
  return e;
}

template <typename T, int DP, bool B>
static hipError_t bwd_launch3(const BwdParams& p, int stage, hipStream_t st) {
  constexpr int W = 4;
  hipError_t e = hipSuccess;
  // LDS-direct staging (unbiased fp16/bf16 D = 64 kernels) where the buffer ranges of N rows stay
  // below 2^31 bytes: K/V for dq, Q/dO for dK/dV.  The LDS-direct dq kernels also run the
  // preprocess of their rows, so a whole backward then launches no bwd_pre_kernel.
  const int64_t lim = int64_t(1) << 31, es = (int64_t)sizeof(T);
  const bool ld_kv = sizeof(T) == 2 && !B && DP == 64 && p.D == 64 && (int64_t)p.N * p.ks[2] * es < lim &&
                     (int64_t)p.N * p.vs[2] * es < lim;
  const bool ld_qg = sizeof(T) == 2 && !B && DP == 64 && p.D == 64 && (int64_t)p.N * p.qs[2] * es < lim &&
                     (int64_t)p.N * p.gs[2] * es < lim;
  // the fp32 dq kernels at D <= 64 run the preprocess of their rows too
  const bool pre_in_dq = ld_kv || (sizeof(T) == 4 && DP <= 64);
  if (stage == 0 || (stage < 0 && !pre_in_dq)) {
    if ((e = pre_launch<T>(p, st)) != hipSuccess) return e;
  }
  if constexpr (DP == 32) {
    if (p.N <= 64) return stage == 0 ? e : bwd_launch_short<T, DP, B>(p, stage, st);
  }
  if constexpr (sizeof(T) == 2) {
    constexpr int R = 1;  // one 32-wide tile per wave: 2 waves per SIMD beat wider tiles at 1
    const dim3 grid((p.N + 32 * R * W - 1) / (32 * R * W), p.BH);
    if constexpr (!B && DP <= 64) {
      if (p.split > 1) {
        // an under-filled grid (short sequences, few heads): the key (dq) or row (dK/dV) loop cut
        // into p.split ranges over grid z, fp32 partials summed by a combine launch
        const dim3 gs(grid.x, grid.y, (unsigned)p.split);
        const int kq = p.causal ? 1 : 0, kkv = p.causal ? 2 : 0;
        const CombineOut cq{p.part, p.dq, {p.dqs[0], p.dqs[1], p.dqs[2]}, p.scale, kq};
        const CombineOut ck{p.part + p.part_stride, p.dk, {p.dks[0], p.dks[1], p.dks[2]}, p.scale, kkv};
        const CombineOut cv{p.part + 2 * p.part_stride, p.dv, {p.dvs[0], p.dvs[1], p.dvs[2]}, 1.f, kkv};
        if (stage < 0 || stage == 1) {
          if (ld_kv) {
            hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, R, W, false, DP == 64>), gs, dim3(64 * W), 0, st, p);
          } else {
            hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, R, W, false>), gs, dim3(64 * W), 0, st, p);
          }
          if ((e = hipGetLastError()) != hipSuccess) return e;
          if (stage == 1 && (e = combine_launch<T>(p, &cq, 1, st)) != hipSuccess) return e;
        }
        if (stage < 0 || stage == 2) {
          if (ld_qg) {
            hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, W, false, DP == 64>), gs, dim3(64 * W), 0, st, p);
          } else {
            hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, W, false>), gs, dim3(64 * W), 0, st, p);
          }
          if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        // the whole backward sums the three gradients' partials in one launch
        if (stage < 0) {
          const CombineOut all[3] = {cq, ck, cv};
          e = combine_launch<T>(p, all, 3, st);
        } else if (stage == 2) {
          const CombineOut kv[2] = {ck, cv};
          e = combine_launch<T>(p, kv, 2, st);
        }
        return e;
      }
    }
    if (stage < 0 || stage == 1) {
      // dq with two 32-row tiles per wave: each K/V fragment read from LDS feeds both tiles,
      // halving the LDS reads per MFMA.  Unbiased, D <= 64 (causal: below), and only where the grid
      // still puts two 256-row work-groups on every CU.  B1 H8 d64 16K: fp16 0.875 -> 0.814 ms, bf16
      // 0.841 -> 0.768 ms; causal 16K 0.479 against 0.510 ms and 4K (128 work-groups) 0.074 against
      // 0.111 ms stay on the 32-row kernel.  At D = 64, 8-wave work-groups of 512 rows (one per CU,
      // 246 VGPRs), so each K/V stage staged once serves twice the rows: 16K 0.794 -> 0.766 ms (fp16),
      // 0.750 -> 0.720 ms (bf16), B2 H8 8K 0.404 -> 0.388 ms, 64K 12.13 -> 11.86 ms.
      const dim3 grid2((p.N + 255) / 256, p.BH);
      bool wide = false;
      if constexpr (DP <= 64 && !B) {
        // causal calls take the two-tile kernel where its 512-row work-groups come in whole pairs of
        // rounds (a multiple of 512) over heads of at least 32 row blocks, so that the heaviest-first
        // order balances: dq causal 32K 1.616 -> 1.514 ms, 64K 6.35 -> 5.89 ms, B1 H16 16K 0.829 ->
        // 0.787 ms, B2 H8 16K bf16 0.778 -> 0.738 ms; one round (B1 H8 16K, 256 work-groups) took
        // 0.427 -> 0.605 ms, B4 H8 8K 0.457 -> 0.555 ms and B8 H3 N16385 (792) 1.25 -> 1.37 ms
        const dim3 grid8((p.N + 511) / 512, p.BH);
        const int64_t n8 = (int64_t)grid8.x * grid8.y;
        // non-causal D = 64 also where the 512-row work-groups take fewer rounds of the chip (256 at
        // one per CU) than the 128-row ones (512 at two per CU): B8 H3 N4097 dq 0.190 -> 0.170 ms
        // (792 work-groups, 2 rounds, against 216, 1); with the rounds level, B1 H8 8K 0.206 -> 0.282 ms
        const int64_t g1 = (int64_t)((p.N + 127) / 128) * p.BH;
        const bool fewer_rounds = DP == 64 && !p.causal && (g1 + 511) / 512 > (n8 + 255) / 256;
        wide = ((int64_t)grid2.x * grid2.y >= 512 && (!p.causal || (DP == 64 && p.N >= 16384 && n8 % 512 == 0))) ||
               fewer_rounds;
        bool w8 = false;
        if constexpr (DP == 64) {
          if (wide && (n8 >= 256 || fewer_rounds)) {
            // LDS-direct staging where every head dim chunk is data (D = 64) and the buffer ranges of
            // N rows of K and V stay below 2^31 bytes
            if (ld_kv) {
              hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, 2, 8, false, true>), grid8, dim3(512), 0, st, p);
            } else {
              hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, 2, 8, false>), grid8, dim3(512), 0, st, p);
            }
            w8 = true;
          }
        }
        if (wide && !w8) hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, 2, W, false>), grid2, dim3(64 * W), 0, st, p);
      }
      // otherwise, at D = 64 with the same grid condition, 8-wave work-groups of 32-row tiles
      // (256 rows): the K/V stage staged once for twice the rows.  Causal 16K dq 0.466 -> 0.412 ms,
      // 32K 1.675 -> 1.589 ms.
      if (!wide) {
        if constexpr (DP == 64) {
          if ((int64_t)grid2.x * grid2.y >= 512) {
            if (ld_kv) {
              hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, R, 8, false, !B>), grid2, dim3(512), 0, st, p);
            } else {
              hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, R, 8, B>), grid2, dim3(512), 0, st, p);
            }
            wide = true;
          }
        }
      }
      if (!wide) {
        if (ld_kv) {
          hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, R, W, false, !B && DP == 64>), grid, dim3(64 * W), 0, st, p);
        } else {
          hipLaunchKernelGGL((bwd_dq_half_kernel<T, DP, R, W, B>), grid, dim3(64 * W), 0, st, p);
        }
      }
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (stage < 0 || stage == 2) {
      // dK/dV in 8-wave work-groups (256 keys) at D = 64 where that grid still puts two
      // work-groups on every CU: 16K 1.109 -> 1.078 ms, causal 16K 0.602 -> 0.569 ms, bf16 16K
      // 1.053 -> 1.028 ms; at 4K (128 work-groups) 0.101 against 0.130 ms, so smaller grids keep 4.
      // Non-causal grids of 256-511 work-groups (one round at one per CU) take 8 too: dK/dV B8 H3
      // N4097 0.290 -> 0.278 ms, B1 H8 8K 0.267 -> 0.261 ms, B2 H8 4K 0.138 -> 0.136 ms
      bool w8 = false;
      if constexpr (DP == 64) {
        const dim3 g8((p.N + 255) / 256, p.BH);
        if ((int64_t)g8.x * g8.y >= (p.causal ? 512 : 256)) {
          // LDS-direct staging where every head dim chunk is data (D = 64) and the buffer ranges of
          // N rows of Q and dO stay below 2^31 bytes
          if constexpr (!B) {
            if (ld_qg) {
              hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, 8, false, true>), g8, dim3(512), 0, st, p);
            } else {
              hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, 8, B>), g8, dim3(512), 0, st, p);
            }
          } else {
            hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, 8, B>), g8, dim3(512), 0, st, p);
          }
          w8 = true;
        }
      }
      if (!w8) {
        if (ld_qg) {
          hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, W, false, !B && DP == 64>), grid, dim3(64 * W), 0, st, p);
        } else {
          hipLaunchKernelGGL((bwd_dkdv_half_kernel<T, DP, R, W, B>), grid, dim3(64 * W), 0, st, p);
        }
      }
      e = hipGetLastError();
    }
  } else {
    // fp32: the key (dq) and row (dK/dV) loops split over grid z for under-filled grids, as above
    const dim3 grid((p.N + 32 * W - 1) / (32 * W), p.BH, (unsigned)(p.split > 1 ? p.split : 1));
    const int kq = p.causal ? 1 : 0, kkv = p.causal ? 2 : 0;
    const CombineOut cq{p.part, p.dq, {p.dqs[0], p.dqs[1], p.dqs[2]}, p.scale, kq};
    const CombineOut ck{p.part + p.part_stride, p.dk, {p.dks[0], p.dks[1], p.dks[2]}, p.scale, kkv};
    const CombineOut cv{p.part + 2 * p.part_stride, p.dv, {p.dvs[0], p.dvs[1], p.dvs[2]}, 1.f, kkv};
    if (stage < 0 || stage == 1) {
      hipLaunchKernelGGL((bwd_dq_kernel<T, DP, W, B>), grid, dim3(64 * W), 0, st, p);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      if (p.split > 1 && stage == 1 && (e = combine_launch<T>(p, &cq, 1, st)) != hipSuccess) return e;
    }
    if (stage < 0 || stage == 2) {
      hipLaunchKernelGGL((bwd_dkdv_kernel<T, DP, W, B>), grid, dim3(64 * W), 0, st, p);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      if (p.split > 1 && stage == 2) {
        const CombineOut kv[2] = {ck, cv};
        e = combine_launch<T>(p, kv, 2, st);
      }
    }
    if (p.split > 1 && stage < 0) {
      const CombineOut all[3] = {cq, ck, cv};
      e = combine_launch<T>(p, all, 3, st);
    }
  }
  return e;
}

template <typename T, int DP>
static hipError_t bwd_launch2(const BwdParams& p, int stage, hipStream_t st) {
  return p.bias.ptr ? bwd_launch3<T, DP, true>(p, stage, st) : bwd_launch3<T, DP, false>(p, stage, st);
}

template <typename T>
static hipError_t bwd_launch1(const BwdParams& p, int stage, hipStream_t st) {
  switch (pad_head_dim(p.D)) {
    case 32: return bwd_launch2<T, 32>(p, stage, st);
    case 64: return bwd_launch2<T, 64>(p, stage, st);
    default: return bwd_launch2<T, 128>(p, stage, st);
  }
}

hipError_t launch_bwd(const BwdParams& p, int dtype, int stage, hipStream_t st) {
  if (dtype == ELSA_F16) return bwd_launch1<f16>(p, stage, st);
  if (dtype == ELSA_BF16) return bwd_launch1<bf16>(p, stage, st);
  return bwd_launch1<float>(p, stage, st);
}

template <typename T, int DP>
static hipError_t rs_launch2(const BwdParams& p, float* m, float* z, hipStream_t st) {
  constexpr int W = 4;
  const dim3 grid((p.N + 32 * W - 1) / (32 * W), p.BH);
  if (p.bias.ptr)
    hipLaunchKernelGGL((row_stats_kernel<T, DP, W, true>), grid, dim3(64 * W), 0, st, p, m, z);
  else
    hipLaunchKernelGGL((row_stats_kernel<T, DP, W, false>), grid, dim3(64 * W), 0, st, p, m, z);
  return hipGetLastError();
}

template <typename T>
static hipError_t rs_launch1(const BwdParams& p, float* m, float* z, hipStream_t st) {
  switch (pad_head_dim(p.D)) {
    case 32: return rs_launch2<T, 32>(p, m, z, st);
    case 64: return rs_launch2<T, 64>(p, m, z, st);
    default: return rs_launch2<T, 128>(p, m, z, st);
  }
}

hipError_t launch_row_stats(const BwdParams& p, float* row_m, float* row_z, int dtype, hipStream_t st) {
  if (dtype == ELSA_F16) return rs_launch1<f16>(p, row_m, row_z, st);
  if (dtype == ELSA_BF16) return rs_launch1<bf16>(p, row_m, row_z, st);
  return rs_launch1<float>(p, row_m, row_z, st);
}

template <typename T, int DP>
static hipError_t db_launch2(const BwdParams& p, float* dbias, int bb, int hb, int nsplit, float* part,
                             hipStream_t st) {
  hipError_t e = pre_launch<T>(p, st);
  if (e != hipSuccess) return e;
  const int tiles = (p.N + 31) / 32;
  const dim3 grid(tiles * tiles, hb, bb * nsplit);
  hipLaunchKernelGGL((dbias_kernel<T, DP>), grid, dim3(64), 0, st, p, dbias, bb, hb, nsplit, part);
  if ((e = hipGetLastError()) != hipSuccess || nsplit == 1) return e;
  const int64_t n = (int64_t)bb * hb * p.N * p.N;
  hipLaunchKernelGGL(dbias_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, dbias, nsplit, n);
  return hipGetLastError();
}

template <typename T>
static hipError_t db_launch1(const BwdParams& p, float* dbias, int bb, int hb, int nsplit, float* part,
                             hipStream_t st) {
  switch (pad_head_dim(p.D)) {
    case 32: return db_launch2<T, 32>(p, dbias, bb, hb, nsplit, part, st);
    case 64: return db_launch2<T, 64>(p, dbias, bb, hb, nsplit, part, st);
    default: return db_launch2<T, 128>(p, dbias, bb, hb, nsplit, part, st);
  }
}

int dbias_splits(int N, int batch, int heads, int bias_batch, int bias_heads) {
  const int64_t tiles = (N + 31) / 32;
  const int64_t blocks = tiles * tiles * bias_batch * bias_heads;
  const int64_t pairs = (int64_t)(bias_batch == 1 ? batch : 1) * (bias_heads == 1 ? heads : 1);
  int64_t ns = (2048 + blocks - 1) / blocks;  // enough work-groups to fill 256 CUs several times
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, pairs / 4));  // at least 4 (b, h) pairs per split
  return (int)std::max<int64_t>(1, std::min<int64_t>(ns, 256));
}

hipError_t launch_dbias(const BwdParams& p, float* dbias, int bias_batch, int bias_heads, int dtype, int nsplit,
                        float* part, hipStream_t st) {
  if (dtype == ELSA_F16) return db_launch1<f16>(p, dbias, bias_batch, bias_heads, nsplit, part, st);
  if (dtype == ELSA_BF16) return db_launch1<bf16>(p, dbias, bias_batch, bias_heads, nsplit, part, st);
  return db_launch1<float>(p, dbias, bias_batch, bias_heads, nsplit, part, st);
}

}  // namespace elsa
