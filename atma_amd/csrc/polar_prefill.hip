// Polar attention forward (prefill): flash-style, MFMA, one pass over the keys.
//
// Reference: _polar_fwd_kernel / _polar_forward / polar_attention_fwd,
// kernel/polar_triton.py:49-191,505-609 (math: model/blocks.py:171-250).  Per query
// the kernel streams key blocks keeping (m, l = sum p, q2 = sum p^2, acc = sum p v),
// folds the null sink once at the end and emits the unit direction c and the
// bounded magnitude mag = tanh(beta*log1p(L^3/(Q2*Z))).
//
// MI355X design (gfx950, wave64, MFMA 32x32):
//  * A workgroup owns 128 query rows of one query head (4 waves x 32 rows).  The
//    query tile stays in registers as the MFMA B operand for the whole key loop.
//  * Each wave computes S^T = K Q^T (rows = keys, columns = its 32 queries) and
//    O^T = V^T P^T (rows = head dims, columns = queries).  With queries on the
//    MFMA column axis every per-query quantity (temperature, running max, L, Q2,
//    the output row) lives in one lane pair (l, l^32): the softmax needs a single
//    cross-lane exchange per 64-key block and no shuffles of the accumulator.
//  * K rows are loaded into the S^T A operand in a permuted order so that the
//    S^T accumulator registers ARE the P^T B operand of the next MFMA: no LDS
//    round trip for P.
//  * K and V tiles (64 keys) are staged in LDS once per workgroup; V is stored
//    transposed ([d][key]) because the PV MFMA contracts over keys.  The next
//    tile is prefetched into registers while the current one is consumed.
//  * GQA is resolved in-kernel (kv head = q head / group), and the grid is
//    ordered so the workgroups of one KV group land on the same XCD (shared L2).
//    A workgroup runs two query tiles, the i-th longest and the i-th shortest of
//    its head, so causal work is the same for every workgroup.
//  * 16-bit inputs skip the per-block max: p is formed against the running max as
//    it stands, and v_dot2 sums p and p^2 from the same 16-bit pairs the PV MFMA
//    consumes; the max is taken (and the state rescaled) only when a lane's sum
//    leaves the safe range -- the first block, or a new maximum far above the old.
//  * bf16/fp16 use v_mfma_f32_32x32x16_{bf16,f16}; fp32 inputs use
//    v_mfma_f32_32x32x2f32 (full fp32 products: the 1e-4 mode).
#include <type_traits>

#include "common.h"

namespace atma {

struct PolarFwdArgs {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  const void* k;
  int64_t k_sb, k_sh, k_st;
  const void* v;
  int64_t v_sb, v_sh, v_st;
  const float* n_keys;
  const float* v_null;
  const float* null_base;
  const float* null_slope_raw;
  const float* len_gain_raw;
  const float* mag_beta_raw;
  void* c;
  void* mag;
  float* stat_m;
  float* stat_l;
  float* stat_q2;
  float* stat_s;
  int B, Hq, Hkv, Tq, Tk;
  int is_causal;
  int window;
  float eps;
  int n_qtiles;
  int xcd_remap;
  int preserve_length;  // temp / null from the raw count even under a window
  // output strides (elements) of c (b, head, query) and of mag; the saved statistics
  // keep the (B, Hq, Tq) layout
  int64_t c_sb, c_sh, c_st, m_sb, m_sh, m_st;
  // packed ragged fresh prefill (16-bit kernel only; null otherwise): tile i covers query
  // rows tile_q_start[i] .. + 127 of the sequence stored at packed tokens
  // tile_seq_start[i] .. + tile_seq_len[i] - 1; n = local position + 1, causal
  const int* tile_seq_start;
  const int* tile_q_start;
  const int* tile_seq_len;
  int total_tokens;
};

template <typename T, int D>
struct FwdCfg {
  static constexpr bool kHalf = sizeof(T) == 2;
  static constexpr int BM = 128;                 // query rows per workgroup
  static constexpr int BN = 64;                  // keys per block
  static constexpr int VE = 16 / (int)sizeof(T); // elements per 16-byte chunk
  static constexpr int CPR = D / VE;             // chunks per row
  static constexpr int KP = D + VE;              // K tile pitch (elements)
  static constexpr int VP = BN + VE;             // V^T tile pitch (elements)
  static constexpr int KCH = BN * CPR / 256;     // K chunks per thread
  static constexpr int VGROUPS = (BN / 4) * CPR; // (4 keys x 1 chunk) groups
  static constexpr int VG_PT = (VGROUPS + 255) / 256;
  static constexpr int NT = D / 32;              // O^T tiles (32 dims each)
  static constexpr int QSTEPS = kHalf ? D / 16 : D / 2;
};

// Key held by S^T register i (0..15) of 32-key tile j for lane half h.
__device__ __forceinline__ int st_key(int j, int i, int h) {
  return 32 * j + 16 * (i >> 3) + 8 * h + (i & 7);
}
// Key loaded into S^T A-operand row r (0..31) -- the inverse view of st_key.
__device__ __forceinline__ int a_row_key(int r) {
  const int a = r >> 3, hh = (r >> 2) & 1, b = r & 3;
  return 16 * (a >> 1) + 8 * hh + 4 * (a & 1) + b;
}

template <typename T>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  Pack8 pa, pb;
  pa.u = a;
  pb.u = b;
  if constexpr (__is_same(T, bf16)) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa.b, pb.b, c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(pa.h, pb.h, c, 0, 0, 0);
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(256, 2) polar_fwd_kernel(PolarFwdArgs args) {
  using Cfg = FwdCfg<T, D>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, VE = Cfg::VE, CPR = Cfg::CPR;
  constexpr int KP = Cfg::KP, VP = Cfg::VP, NT = Cfg::NT;
  __shared__ __attribute__((aligned(16))) T Ks[2 * BN * KP];  // double-buffered key tile
  __shared__ __attribute__((aligned(16))) T Vt[2 * D * VP];   // double-buffered V^T tile
  __shared__ float s_bounds[4][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ql = lane & 31, h = lane >> 5;

  // ---- workgroup -> (b, q head, query tile), XCD-aware, longest tile first
  const int G = args.Hq / args.Hkv;
  int bid = blockIdx.x;
  if (args.xcd_remap) {
    const int x = bid & 7, p = bid >> 3;
    bid = (x + 8 * (p / G)) * G + p % G;
  }
  const int g = bid % G;
  const int unit = bid / G;
  // A workgroup takes a pair of query tiles, the i-th longest and the i-th shortest
  // of its head, so under a causal mask every pair costs the same number of key
  // blocks: the grid has no long tail.
  const int npairs = (args.n_qtiles + 1) / 2;
  const int pair = unit % npairs;
  const int grp = unit / npairs;  // b * Hkv + kv head
  const int b = grp / args.Hkv, hk = grp % args.Hkv;
  const int hq = hk * G + g;
  const int npass = pair < args.n_qtiles - 1 - pair ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
  const int qt = pass == 0 ? args.n_qtiles - 1 - pair : pair;
  const int q0 = qt * BM;

  const T* qp = (const T*)args.q + b * args.q_sb + hq * args.q_sh;
  const T* kp = (const T*)args.k + b * args.k_sb + hk * args.k_sh;
  const T* vp = (const T*)args.v + b * args.v_sb + hk * args.v_sh;

  // ---- per-query calibration (lane pair owns query row qi)
  const int qi = q0 + wave * 32 + ql;
  const bool q_ok = qi < args.Tq;
  const float n_raw = q_ok ? args.n_keys[qi] : 0.f;
  float n_cal = n_raw;
  if (args.window > 0 && !args.preserve_length) n_cal = fminf(n_cal, (float)args.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float spg = softplus(args.len_gain_raw[hq]);
  const float sps = softplus(args.null_slope_raw[hq]);
  const float nb = args.null_base[hq];
  const float mbeta = softplus(args.mag_beta_raw[hq]);
  const float temp = 1.f + spg * logf(n_cal);
  const float nullv = nb + sps * sqrtf(logf(n_cal + 1.f));
  const float c1 = temp * kLog2e * (1.f / sqrtf((float)D));

  // ---- key-loop bounds from the valid counts of this tile (raw n, window band)
  {
    float lo = q_ok ? n_raw : 3.0e38f, hi = q_ok ? n_raw : -1.f;
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) {
      s_bounds[wave][0] = lo;
      s_bounds[wave][1] = hi;
    }
  }
  __syncthreads();
  const float w_nlo = s_bounds[wave][0], w_nhi = s_bounds[wave][1];
  float g_nlo = s_bounds[0][0], g_nhi = s_bounds[0][1];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    g_nlo = fminf(g_nlo, s_bounds[w][0]);
    g_nhi = fmaxf(g_nhi, s_bounds[w][1]);
  }
  int kend = 0, kbeg = 0;
  if (g_nhi > 0.f) {
    float hiF = fminf(g_nhi, (float)args.Tk);
    kend = (int)ceilf(hiF);
    if (args.is_causal) kend = min(kend, min(q0 + BM, args.Tk));
    if (args.window > 0) kbeg = max((int)floorf(g_nlo) - args.window, 0);
    kbeg = (kbeg / BN) * BN;
  }
  const int nblk_beg = kbeg / BN, nblk_end = (kend + BN - 1) / BN;

  // ---- query operand (B of S^T) in registers
  u32x4 qreg16[Cfg::kHalf ? Cfg::QSTEPS : 1];
  float qregf[Cfg::kHalf ? 1 : Cfg::QSTEPS];
  if constexpr (Cfg::kHalf) {
#pragma unroll
    for (int s = 0; s < Cfg::QSTEPS; ++s) {
      qreg16[s] = q_ok ? *(const u32x4*)(qp + (int64_t)qi * args.q_st + 16 * s + 8 * h)
                       : u32x4{0, 0, 0, 0};
    }
    // Consume the query registers here: a first use inside the key loop would make the
    // compiler drain every load in flight there (the next tile's prefetch included) at
    // each block.
#pragma unroll
    for (int s = 0; s < Cfg::QSTEPS; ++s) asm volatile("" ::"v"(qreg16[s]));
  } else {
#pragma unroll
    for (int s4 = 0; s4 < Cfg::QSTEPS / 4; ++s4) {
      f32x4 x = q_ok ? *(const f32x4*)(qp + (int64_t)qi * args.q_st + (D / 2) * h + 4 * s4)
                     : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) qregf[4 * s4 + e] = x[e];
    }
  }

  // ---- running statistics (log2 domain) and O^T accumulators
  float m_run = kSentinel, l_part = 0.f, q2_part = 0.f;
  f32x16 oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};

  // ---- per-thread offsets inside a key block.
  //  K: 16-byte chunk cidx = tid + 256 r -> key cidx / CPR, chunk cidx % CPR (a row per
  //     CPR consecutive lanes: coalesced loads, contiguous LDS rows).
  //  V: (4-key, 16-byte) group = tid + 256 gi -> key group kg = group % 16, chunk
  //     ch = group / 16, so 16 consecutive lanes write one V^T row contiguously.
  const int kst = (int)args.k_st, vst = (int)args.v_st;
  int koff[Cfg::KCH], klds[Cfg::KCH];
#pragma unroll
  for (int r = 0; r < Cfg::KCH; ++r) {
    const int cidx = tid + 256 * r;
    koff[r] = (cidx / CPR) * kst + (cidx % CPR) * VE;
    klds[r] = (cidx / CPR) * KP + (cidx % CPR) * VE;
  }
  int voff[Cfg::VG_PT], vkg[Cfg::VG_PT], vch[Cfg::VG_PT];
#pragma unroll
  for (int gi = 0; gi < Cfg::VG_PT; ++gi) {
    const int grpi = tid + 256 * gi;
    vkg[gi] = grpi & 15;
    vch[gi] = grpi >> 4;
    voff[gi] = 4 * vkg[gi] * vst + vch[gi] * VE;
  }
  auto v_active = [&](int gi) { return Cfg::VG_PT * 256 == Cfg::VGROUPS || tid + 256 * gi < Cfg::VGROUPS; };

  u32x4 kpre[Cfg::KCH];
  u32x4 vpre[Cfg::VG_PT][4];
  // Rows past Tk are read from row Tk - 1 instead (finite values: their scores are
  // masked and their p is exactly 0), so every block issues the same unconditional
  // loads and the compiler never has to drain them early.
  auto prefetch = [&](int blk) {
    const T* kb = kp + (int64_t)blk * BN * args.k_st;
    const T* vb = vp + (int64_t)blk * BN * args.v_st;
    const int lim = args.Tk - blk * BN;  // keys of this block below Tk
    if (lim >= BN) {
#pragma unroll
      for (int r = 0; r < Cfg::KCH; ++r) kpre[r] = *(const u32x4*)(kb + koff[r]);
#pragma unroll
      for (int gi = 0; gi < Cfg::VG_PT; ++gi)
        if (v_active(gi)) {
#pragma unroll
          for (int r = 0; r < 4; ++r) vpre[gi][r] = *(const u32x4*)(vb + voff[gi] + r * vst);
        }
    } else {
#pragma unroll
      for (int r = 0; r < Cfg::KCH; ++r) {
        const int cidx = tid + 256 * r;
        const int row = min(cidx / CPR, lim - 1);
        kpre[r] = *(const u32x4*)(kb + (int64_t)row * kst + (cidx % CPR) * VE);
      }
#pragma unroll
      for (int gi = 0; gi < Cfg::VG_PT; ++gi)
        if (v_active(gi)) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = min(4 * vkg[gi] + r, lim - 1);
            vpre[gi][r] = *(const u32x4*)(vb + (int64_t)row * vst + vch[gi] * VE);
          }
        }
    }
  };
  auto commit = [&](int buf) {
    T* kd = Ks + buf * (BN * KP);
    T* vd = Vt + buf * (D * VP);
#pragma unroll
    for (int r = 0; r < Cfg::KCH; ++r) *(u32x4*)(kd + klds[r]) = kpre[r];
#pragma unroll
    for (int gi = 0; gi < Cfg::VG_PT; ++gi)
      if (v_active(gi)) {
        T* vrow = vd + vch[gi] * VE * VP + 4 * vkg[gi];
        if constexpr (Cfg::kHalf) {
          // 4 keys x 8 dims -> 8 rows of V^T holding 4 keys (8 bytes) each
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t lo01 = __builtin_amdgcn_perm(vpre[gi][1][w], vpre[gi][0][w], 0x05040100u);
            const uint32_t hi01 = __builtin_amdgcn_perm(vpre[gi][1][w], vpre[gi][0][w], 0x07060302u);
            const uint32_t lo23 = __builtin_amdgcn_perm(vpre[gi][3][w], vpre[gi][2][w], 0x05040100u);
            const uint32_t hi23 = __builtin_amdgcn_perm(vpre[gi][3][w], vpre[gi][2][w], 0x07060302u);
            *(u32x2*)(vrow + (2 * w) * VP) = u32x2{lo01, lo23};
            *(u32x2*)(vrow + (2 * w + 1) * VP) = u32x2{hi01, hi23};
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *(u32x4*)(vrow + e * VP) = u32x4{vpre[gi][0][e], vpre[gi][1][e], vpre[gi][2][e], vpre[gi][3][e]};
        }
      }
  };

  const int nblk = nblk_end - nblk_beg;
  if (nblk > 0) {
    prefetch(nblk_beg);
    commit(0);
  }
  __syncthreads();
  const int arow = a_row_key(ql);
  constexpr float kRescale = 8.f;  // fp32 inputs, lazy rescale: p <= 2^8 between max updates

  for (int it = 0; it < nblk; ++it) {
    const int blk = nblk_beg + it, buf = it & 1;
    const int k0 = blk * BN;
    const bool more = it + 1 < nblk;
    if (more) prefetch(blk + 1);
    const T* Kb = Ks + buf * (BN * KP);
    const T* Vb = Vt + buf * (D * VP);

    // ---- S^T = K Q^T  (two 32-key tiles)
    f32x16 sacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      sacc[j] = f32x16{};
      const T* krow = Kb + (32 * j + arow) * KP;
      if constexpr (Cfg::kHalf) {
#pragma unroll
        for (int s = 0; s < Cfg::QSTEPS; ++s) {
          u32x4 a = *(const u32x4*)(krow + 16 * s + 8 * h);
          sacc[j] = mfma32<T>(a, qreg16[s], sacc[j]);
        }
      } else {
#pragma unroll
        for (int s4 = 0; s4 < Cfg::QSTEPS / 4; ++s4) {
          f32x4 a = *(const f32x4*)(krow + (D / 2) * h + 4 * s4);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sacc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qregf[4 * s4 + e], sacc[j], 0, 0, 0);
        }
      }
    }

    // ---- online softmax (+ sum of p^2); scores scaled inside one FMA per element
    const bool full = (k0 + BN <= (int)fminf(w_nlo, (float)args.Tk)) &&
                      (args.window <= 0 || (float)k0 >= w_nhi - (float)args.window);
    if (!full) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + st_key(j, i, h);
          bool ok = (float)key < n_raw && key < args.Tk;
          if (args.window > 0) ok = ok && (float)key >= n_raw - (float)args.window;
          sacc[j][i] = ok ? sacc[j][i] : -INFINITY;
        }
    }
    if constexpr (Cfg::kHalf) {
      // Optimistic pass: p = 2^(s c1 - m_run) against the running max as it stands, the
      // 16-bit pairs feed the PV MFMA and v_dot2 gives sum p and sum p^2 from the very
      // same rounded values.  Only when some lane's sum leaves the safe range (a new
      // maximum far above the old one, or the first block) is the block max taken and
      // the state rescaled, then p recomputed.
      constexpr float kSafe = __is_same(T, bf16) ? 1048576.f : 16384.f;
      u32x4 pb[4];
      float ls = 0.f, qs = 0.f;
      auto exp_pack = [&]() {
        const float neg_m = -m_run;
        ls = qs = 0.f;
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
          const int j = ps >> 1, base = 8 * (ps & 1);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[j][base + 2 * w], c1, neg_m));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[j][base + 2 * w + 1], c1, neg_m));
            pb[ps][w] = pack2<T>(p0, p1);
          }
        }
        const uint32_t one2 = pack2<T>(1.f, 1.f);
#pragma unroll
        for (int ps = 0; ps < 4; ++ps)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            ls = dot2<T>(pb[ps][w], one2, ls);
            qs = dot2<T>(pb[ps][w], pb[ps][w], qs);
          }
      };
      exp_pack();
      if (__ballot(!(ls <= kSafe)) != 0) {
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[j][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx * c1);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
        q2_part *= alpha * alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t) oacc[t] *= alpha;
        exp_pack();
      }
      l_part += ls;
      q2_part += qs;

      // ---- O^T += V^T P^T
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const T* vrow = Vb + (32 * t + ql) * VP + 8 * h;
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
          u32x4 a = *(const u32x4*)(vrow + 16 * ps);
          oacc[t] = mfma32<T>(a, pb[ps], oacc[t]);
        }
      }
    } else {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[j][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mxs = mx * c1;
      if (__ballot(mxs > m_run + kRescale) != 0) {
        const float m_new = fmaxf(m_run, mxs);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
        q2_part *= alpha * alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t) oacc[t] *= alpha;
      }
      const float neg_m = -m_run;
      float ls = 0.f, qs = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sacc[j][i], c1, neg_m));
          sacc[j][i] = p;
          ls += p;
          qs = fmaf(p, p, qs);
        }
      l_part += ls;
      q2_part += qs;

      // ---- O^T += V^T P^T (fp32 operands)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const T* vrow = Vb + (32 * t + ql) * VP + 8 * h;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int w = 0; w < 2; ++w) {
              f32x4 a = *(const f32x4*)(vrow + 32 * j + 16 * u + 4 * w);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], sacc[j][8 * u + 4 * w + e],
                                                              oacc[t], 0, 0, 0);
            }
          }
        }
      }
    }
    if (more) commit(buf ^ 1);
    __syncthreads();
  }

  // ---- fold the null sink, normalise, magnitude
  float L = l_part + __shfl_xor(l_part, 32, 64);
  float Q2 = q2_part + __shfl_xor(q2_part, 32, 64);
  const float an2 = temp * nullv * kLog2e;
  const float mn = fmaxf(m_run, an2);
  const float al = exp2f(m_run - mn);
  L *= al;
  Q2 *= al * al;
  const float pn = exp2f(an2 - mn);
  const float Z = L + pn;
  const float* vn = args.v_null + (int64_t)hq * D;
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
      const float s = oacc[t][i] * al + pn * vn[d];
      oacc[t][i] = s;
      ss += s * s;
    }
  }
  ss += __shfl_xor(ss, 32, 64);
  const float inv = 1.f / fmaxf(sqrtf(ss), args.eps);
  const float n_eff = L * L / fmaxf(Q2, 1e-30f);
  const float m_eff = n_eff * (L / fmaxf(Z, args.eps));
  const float magv = tanhf(mbeta * log1pf(m_eff));

  if (q_ok) {
    const int64_t row = ((int64_t)b * args.Hq + hq) * args.Tq + qi;
    T* cp = (T*)args.c + row * D;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d = 32 * t + 8 * gq + 4 * h;
        if constexpr (Cfg::kHalf) {
          u32x2 pk = {pack2<T>(oacc[t][4 * gq] * inv, oacc[t][4 * gq + 1] * inv),
                      pack2<T>(oacc[t][4 * gq + 2] * inv, oacc[t][4 * gq + 3] * inv)};
          *(u32x2*)(cp + d) = pk;
        } else {
          f32x4 x = {oacc[t][4 * gq] * inv, oacc[t][4 * gq + 1] * inv, oacc[t][4 * gq + 2] * inv,
                     oacc[t][4 * gq + 3] * inv};
          *(f32x4*)(cp + d) = x;
        }
      }
    }
    if (h == 0) {
      ((T*)args.mag)[row] = (T)magv;
      if (args.stat_m) args.stat_m[row] = mn * kLn2;
      if (args.stat_l) args.stat_l[row] = L;
      if (args.stat_q2) args.stat_q2[row] = Q2;
    }
    if (args.stat_s) {
      float* sp = args.stat_s + row * D;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int d = 32 * t + 8 * gq + 4 * h;
          f32x4 x = {oacc[t][4 * gq], oacc[t][4 * gq + 1], oacc[t][4 * gq + 2], oacc[t][4 * gq + 3]};
          *(f32x4*)(sp + d) = x;
        }
    }
  }
  __syncthreads();  // the next pass reuses the LDS tiles and bounds
  }  // pass
}

// 16-bit inputs.  Same math and wave layout as polar_fwd_kernel, with the key / value
// tiles staged by direct global->LDS copies (global_load_lds_dwordx4, no VGPR
// staging, no commit pass): K and V both row-major in LDS, unpadded, their 16-byte
// chunks XOR-swizzled by row (chunk c of row r at c ^ (r % CPR)) so the operand reads
// below are bank-conflict free.  V^T, the A operand of O^T = V^T P^T, comes out of
// the row-major V tile through ds_read_b64_tr_b16 (two per operand: keys +0..3 and
// +4..7).  A wave copies its 16 rows of the next block while the current one is
// consumed; one barrier per block.
template <typename T, int D>
__global__ void __launch_bounds__(256, 2) polar_fwd16_kernel(PolarFwdArgs args) {
  constexpr int BM = 128, BN = 64, CPR = D / 8, NT = D / 32, QSTEPS = D / 16;
  constexpr int RPI = 64 / CPR;            // rows per wave copy instruction (1 KB)
  constexpr int TILE = BN * D;             // elements of one K or V tile
  static_assert(BN / 4 % RPI == 0, "a wave copies whole rows");
  __shared__ __attribute__((aligned(16))) T Ks[2 * TILE];
  __shared__ __attribute__((aligned(16))) T Vs[2 * TILE];
  __shared__ float s_bounds[4][2];
  __shared__ float s_vnull[D];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ql = lane & 31, h = lane >> 5;

  // ---- workgroup -> (query tile, b, q head): one tile per workgroup.  Dense: tiles in
  // order of decreasing length (causal: the last tile first) so the dispatcher balances
  // the triangle; within a rank the G query heads of a KV group share an XCD (its L2).
  // Packed: workgroup = (tile of the map, q head), the G heads of a group adjacent.
  const int G = args.Hq / args.Hkv;
  const bool packed = args.tile_seq_start != nullptr;
  int b, hq, q0, Tq = args.Tq, Tk = args.Tk;
  int64_t tok0 = 0;  // packed: first token of the sequence
  if (!packed) {
    const int per_rank = args.B * args.Hq;
    const int rank = blockIdx.x / per_rank;
    int u = blockIdx.x % per_rank;
    if (args.xcd_remap) {
      const int x = u & 7, p = u >> 3;
      u = (x + 8 * (p / G)) * G + p % G;
    }
    const int grp = u / G;  // b * Hkv + kv head
    b = grp / args.Hkv;
    hq = (grp % args.Hkv) * G + u % G;
    q0 = (args.n_qtiles - 1 - rank) * BM;
  } else {
    int u = blockIdx.x;
    if (args.xcd_remap) {
      const int x = u & 7, p = u >> 3;
      u = (x + 8 * (p / G)) * G + p % G;
    }
    const int tile = u / args.Hq;
    const int seq_start = args.tile_seq_start[tile], q_start = args.tile_q_start[tile];
    const int seq_len = args.tile_seq_len[tile];
    // a tile outside the packed tokens (or not on a 128-row boundary) is skipped whole
    if (seq_start < 0 || seq_len < 1 || seq_len > args.total_tokens - seq_start || q_start < 0 ||
        q_start >= seq_len || q_start % BM)
      return;
    b = 0;
    hq = u % args.Hq;
    q0 = q_start;
    Tq = Tk = seq_len;
    tok0 = seq_start;
  }
  const int hk = hq / G;

  // ---- the head's parameters and this lane's key count are read first: later reads
  // sit behind the direct copies, whose memory clobber would turn the uniform parameter
  // reads into vector loads, each waited on in turn
  const int hq_u = __builtin_amdgcn_readfirstlane(hq);
  const float lg_raw = args.len_gain_raw[hq_u], ns_raw = args.null_slope_raw[hq_u];
  const float nb = args.null_base[hq_u], mb_raw = args.mag_beta_raw[hq_u];
  const int qi = q0 + wave * 32 + ql;
  const bool q_ok = qi < Tq;
  const float n_ld = packed ? 0.f : args.n_keys[min(qi, Tq - 1)];

  const T* qp = (const T*)args.q + b * args.q_sb + hq * args.q_sh + tok0 * args.q_st;
  const T* kp = (const T*)args.k + b * args.k_sb + hk * args.k_sh + tok0 * args.k_st;
  const T* vp = (const T*)args.v + b * args.v_sb + hk * args.v_sh + tok0 * args.v_st;

  // ---- direct copies of one key block: this wave's rows 16 wave .. 16 wave + 15 of K
  // and V, RPI rows per instruction; lane l lands at chunk position l % CPR of row
  // l / CPR and fetches the logical chunk stored there.  The buffer ends after the
  // last key row, so in a partial last block rows past Tk read as zeros (finite; their
  // scores are masked and their p is exactly 0).  The descriptor's range check covers
  // the per-lane and instruction offsets, not the scalar one: a full block keeps one
  // byte offset per lane and copy instruction and puts the wave's row in the scalar
  // offset, a partial block puts the whole row offset into the per-lane offset
  // (recomputed from a laundered lane index, so it holds no extra registers).
  const uint32_t kst2 = (uint32_t)args.k_st * 2u, vst2 = (uint32_t)args.v_st * 2u;
  constexpr int NCP = BN / 4 / RPI;  // copy instructions per wave and tensor
  static_assert(RPI * NCP == 16, "a wave copies 16 rows");
  const uint32_t lrow = (uint32_t)(lane / CPR);
  uint32_t coff[NCP];
#pragma unroll
  for (int r = 0; r < NCP; ++r) coff[r] = 16u * ((lane % CPR) ^ lds_swizzle<CPR>(RPI * r + lane / CPR));
  const uint32_t krow_off = lrow * kst2, vrow_off = lrow * vst2;
  auto copy_block = [&](int blk, int buf) {
    const int rows = min(Tk - blk * BN, BN);
    const auto krs = buffer_rsrc(kp + (int64_t)blk * BN * args.k_st,
                                 (uint32_t)((rows - 1) * args.k_st + D) * 2u);
    const auto vrs = buffer_rsrc(vp + (int64_t)blk * BN * args.v_st,
                                 (uint32_t)((rows - 1) * args.v_st + D) * 2u);
    if (rows == BN) {
#pragma unroll
      for (int r = 0; r < NCP; ++r) {
        const uint32_t row0 = 16u * wave + RPI * r;
        dma_buf16(krs, krow_off + coff[r], row0 * kst2, Ks + buf * TILE + row0 * D);
        dma_buf16(vrs, vrow_off + coff[r], row0 * vst2, Vs + buf * TILE + row0 * D);
      }
    } else {
      uint32_t ln = (uint32_t)lane;
      asm volatile("" : "+v"(ln));
      const uint32_t lr = ln / CPR;
#pragma unroll
      for (int r = 0; r < NCP; ++r) {
        const uint32_t row0 = 16u * wave + RPI * r;
        const uint32_t co = 16u * ((ln % CPR) ^ lds_swizzle<CPR>(RPI * r + lr));
        dma_buf16(krs, (row0 + lr) * kst2 + co, 0, Ks + buf * TILE + row0 * D);
        dma_buf16(vrs, (row0 + lr) * vst2 + co, 0, Vs + buf * TILE + row0 * D);
      }
    }
  };
  // element offset of logical chunk c of row r
  auto swz = [](int r, int c) { return r * D + 8 * (c ^ lds_swizzle<CPR>(r)); };

  // ---- every load of the prologue is issued before any is consumed, so the tile pays
  // one memory latency: after the parameters and key count, the query operand (B of
  // S^T, consumed by the key loop), then the direct copies -- key block 0 when the loop
  // starts there (no window) and the null value vector for the epilogue.
  u32x4 qreg16[QSTEPS];
#pragma unroll
  for (int s = 0; s < QSTEPS; ++s)
    qreg16[s] = q_ok ? *(const u32x4*)(qp + (int64_t)qi * args.q_st + 16 * s + 8 * h)
                     : u32x4{0, 0, 0, 0};
  const bool early_copy = args.window <= 0 && Tk > 0;
  if (early_copy) copy_block(0, 0);
  if (64 * wave < D)  // 64 floats per wave, straight into LDS
    dma_buf4(buffer_rsrc(args.v_null + (int64_t)hq * D, (uint32_t)D * 4u), 4u * (uint32_t)lane,
             256u * (uint32_t)wave, s_vnull + 64 * wave);

  // ---- per-query calibration (lane pair owns query row qi)
  const float n_raw = q_ok ? (packed ? (float)(qi + 1) : n_ld) : 0.f;
  float n_cal = n_raw;
  if (args.window > 0 && !args.preserve_length) n_cal = fminf(n_cal, (float)args.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float spg = softplus(lg_raw);
  const float sps = softplus(ns_raw);
  const float mbeta = softplus(mb_raw);
  const float temp = 1.f + spg * logf(n_cal);
  const float nullv = nb + sps * sqrtf(logf(n_cal + 1.f));
  const float c1 = temp * kLog2e * (1.f / sqrtf((float)D));

  // ---- key-loop bounds from the valid counts of this tile (raw n, window band)
  {
    float lo = q_ok ? n_raw : 3.0e38f, hi = q_ok ? n_raw : -1.f;
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) {
      s_bounds[wave][0] = lo;
      s_bounds[wave][1] = hi;
    }
  }
  __syncthreads();
  const float w_nlo = s_bounds[wave][0], w_nhi = s_bounds[wave][1];
  float g_nlo = s_bounds[0][0], g_nhi = s_bounds[0][1];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    g_nlo = fminf(g_nlo, s_bounds[w][0]);
    g_nhi = fmaxf(g_nhi, s_bounds[w][1]);
  }
  int kend = 0, kbeg = 0;
  if (g_nhi > 0.f) {
    float hiF = fminf(g_nhi, (float)Tk);
    kend = (int)ceilf(hiF);
    if (args.is_causal) kend = min(kend, min(q0 + BM, Tk));
    if (args.window > 0) kbeg = max((int)floorf(g_nlo) - args.window, 0);
    kbeg = (kbeg / BN) * BN;
  }
  const int nblk_beg = kbeg / BN, nblk_end = (kend + BN - 1) / BN;


#pragma unroll
  for (int s = 0; s < QSTEPS; ++s) asm volatile("" ::"v"(qreg16[s]));

  float m_run = kSentinel, l_part = 0.f, q2_part = 0.f;
  f32x16 oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};


  const int nblk = nblk_end - nblk_beg;
  if (nblk > 0 && !early_copy) copy_block(nblk_beg, 0);
  const int arow = a_row_key(ql);
  // V^T operand reads: lane group gq = lane / 16 holds d rows 16 (gq % 2) + (lane % 16)
  // and keys 8 (gq / 2) + 0..7 of a 16-key step; lane s of the group reads key
  // row + s / 4, columns 4 (s % 4) .. + 3 of its 16-column slice.
  const int gq = lane >> 4, sl = lane & 15;
  const int vkey = 8 * (gq >> 1) + (sl >> 2);
  const int vcol = 16 * (gq & 1) + 4 * (sl & 3);

  // One 64-key block.  BUF, the LDS half that holds it, is a compile-time constant (the
  // loop below runs blocks in pairs), so every LDS operand address is a loop-invariant
  // lane offset plus an immediate.
  auto key_block = [&](int it, auto BUF) {
    constexpr int buf = decltype(BUF)::value;
    const int blk = nblk_beg + it;
    const int k0 = blk * BN;
    wait_vmcnt<0>();  // this wave's copies of block blk have landed
    lds_barrier();    // everyone's have; everyone is done with buf ^ 1
    if (it + 1 < nblk) copy_block(blk + 1, buf ^ 1);
    const T* Kb = Ks + buf * TILE;
    const T* Vb = Vs + buf * TILE;

    // ---- S^T = K Q^T  (two 32-key tiles, their MFMA chains interleaved; the K
    // fragments of step s + 1 are requested before the MFMAs of step s)
    f32x16 sacc[2] = {f32x16{}, f32x16{}};
    {
      u32x4 kc0 = *(const u32x4*)(Kb + swz(arow, h));
      u32x4 kc1 = *(const u32x4*)(Kb + swz(32 + arow, h));
#pragma unroll
      for (int s = 0; s < QSTEPS; ++s) {
        u32x4 kn0, kn1;
        if (s + 1 < QSTEPS) {
          kn0 = *(const u32x4*)(Kb + swz(arow, 2 * (s + 1) + h));
          kn1 = *(const u32x4*)(Kb + swz(32 + arow, 2 * (s + 1) + h));
        }
        sacc[0] = mfma32<T>(kc0, qreg16[s], sacc[0]);
        sacc[1] = mfma32<T>(kc1, qreg16[s], sacc[1]);
        kc0 = kn0;
        kc1 = kn1;
      }
      // keep two fragment pairs in flight: 4 reads, then (2 MFMAs, 2 reads) per step
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int s = 0; s < QSTEPS - 1; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }

    // ---- online softmax: optimistic pass against the running max (see polar_fwd_kernel)
    const bool full = (k0 + BN <= (int)fminf(w_nlo, (float)Tk)) &&
                      (args.window <= 0 || (float)k0 >= w_nhi - (float)args.window);
    if (!full) {
      // key valid <=> key_lo <= key < key_hi (integer keys: key < n <=> key < ceil n,
      // key >= x <=> key >= ceil x)
      const float tkf = (float)Tk;
      const int key_hi = (int)ceilf(fminf(n_raw, tkf)) - k0;
      const int key_lo =
          args.window > 0 ? (int)ceilf(fminf(n_raw - (float)args.window, tkf)) - k0 : -(1 << 30);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = st_key(j, i, h);
          sacc[j][i] = ((key < key_hi) & (key >= key_lo)) ? sacc[j][i] : -INFINITY;
        }
    }
    constexpr float kSafe = __is_same(T, bf16) ? 1048576.f : 16384.f;
    u32x4 pb[4];
    float ls = 0.f, qs = 0.f;
    auto exp_pack = [&]() {
      const float neg_m = -m_run;
      ls = qs = 0.f;
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const int j = ps >> 1, base = 8 * (ps & 1);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[j][base + 2 * w], c1, neg_m));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[j][base + 2 * w + 1], c1, neg_m));
          pb[ps][w] = pack2<T>(p0, p1);
        }
      }
      const uint32_t one2 = pack2<T>(1.f, 1.f);
#pragma unroll
      for (int ps = 0; ps < 4; ++ps)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          ls = dot2<T>(pb[ps][w], one2, ls);
          qs = dot2<T>(pb[ps][w], pb[ps][w], qs);
        }
    };
    // the first block takes its maximum at once (against the initial sentinel every p
    // would overflow); later blocks try the running maximum first
    bool redo = it == 0;
    if (!redo) {
      exp_pack();
      redo = __ballot(!(ls <= kSafe)) != 0;
    }
    if (redo) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[j][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx * c1);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
      q2_part *= alpha * alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) oacc[t] *= alpha;
      exp_pack();
    }
    l_part += ls;
    q2_part += qs;

    // ---- O^T += V^T P^T, V^T fragments by transposing reads of the row-major V tile,
    // the next fragment requested before each MFMA
    {
      auto vfrag = [&](int t, int ps) {
        const int kr = 16 * ps + vkey, col = 32 * t + vcol;
        const u32x2 lo = lds_read_tr16(Vb + swz(kr, col >> 3) + (col & 7));
        const u32x2 hi = lds_read_tr16(Vb + swz(kr + 4, col >> 3) + (col & 7));
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vc = vfrag(0, 0);
#pragma unroll
      for (int i = 0; i < 4 * NT; ++i) {
        const int t = i % NT, ps = i / NT;  // alternate the NT accumulator chains
        u32x4 vn;
        if (i + 1 < 4 * NT) vn = vfrag((i + 1) % NT, (i + 1) / NT);
        oacc[t] = mfma32<T>(vc, pb[ps], oacc[t]);
        vc = vn;
      }
    }
  };
  for (int it = 0; it < nblk; it += 2) {
    key_block(it, std::integral_constant<int, 0>{});
    if (it + 1 == nblk) break;
    key_block(it + 1, std::integral_constant<int, 1>{});
  }
  wait_vmcnt<0>();  // the copies have landed (also with no key block to consume them) ...
  __syncthreads();  // ... for every wave: the epilogue reads the null vector

  // ---- fold the null sink, normalise, magnitude
  float L = l_part + __shfl_xor(l_part, 32, 64);
  float Q2 = q2_part + __shfl_xor(q2_part, 32, 64);
  const float an2 = temp * nullv * kLog2e;
  const float mn = fmaxf(m_run, an2);
  const float al = exp2f(m_run - mn);
  L *= al;
  Q2 *= al * al;
  const float pn = exp2f(an2 - mn);
  const float Z = L + pn;
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
      const float s = oacc[t][i] * al + pn * s_vnull[d];
      oacc[t][i] = s;
      ss += s * s;
    }
  }
  ss += __shfl_xor(ss, 32, 64);
  const float inv = 1.f / fmaxf(sqrtf(ss), args.eps);
  const float n_eff = L * L / fmaxf(Q2, 1e-30f);
  const float m_eff = n_eff * (L / fmaxf(Z, args.eps));
  const float magv = tanhf(mbeta * log1pf(m_eff));

  if (q_ok) {
    const int64_t row = ((int64_t)b * args.Hq + hq) * args.Tq + qi;  // saved statistics
    T* cp = (T*)args.c + b * args.c_sb + hq * args.c_sh + (tok0 + qi) * args.c_st;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d = 32 * t + 8 * gq + 4 * h;
        if constexpr (true) {
          u32x2 pk = {pack2<T>(oacc[t][4 * gq] * inv, oacc[t][4 * gq + 1] * inv),
                      pack2<T>(oacc[t][4 * gq + 2] * inv, oacc[t][4 * gq + 3] * inv)};
          *(u32x2*)(cp + d) = pk;
        } else {
          f32x4 x = {oacc[t][4 * gq] * inv, oacc[t][4 * gq + 1] * inv, oacc[t][4 * gq + 2] * inv,
                     oacc[t][4 * gq + 3] * inv};
          *(f32x4*)(cp + d) = x;
        }
      }
    }
    if (h == 0) {
      ((T*)args.mag)[b * args.m_sb + hq * args.m_sh + (tok0 + qi) * args.m_st] = (T)magv;
      if (args.stat_m) args.stat_m[row] = mn * kLn2;
      if (args.stat_l) args.stat_l[row] = L;
      if (args.stat_q2) args.stat_q2[row] = Q2;
    }
    if (args.stat_s) {
      float* sp = args.stat_s + row * D;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int d = 32 * t + 8 * gq + 4 * h;
          f32x4 x = {oacc[t][4 * gq], oacc[t][4 * gq + 1], oacc[t][4 * gq + 2], oacc[t][4 * gq + 3]};
          *(f32x4*)(sp + d) = x;
        }
    }
  }
}

// 16-bit inputs, two query heads of one KV group per workgroup (G even): the ping-pong
// schedule.  A workgroup of 8 waves owns one 128-row query tile of query heads 2p and
// 2p + 1 of a KV group; waves 0-3 (group A) serve the first head and waves 4-7 (group B)
// the second, 32 rows per wave, with the per-wave math of polar_fwd16_kernel.  The two
// waves that share a SIMD (wave w and wave w + 4) are kept in opposite phases: a wave
// alternates an MFMA phase -- O^T += V^T P^T for block j - 1, then S^T = K Q^T for block
// j -- and a VALU phase -- the softmax of block j (exponentials, packing, sums, the rare
// rescale) -- and group B runs one phase behind group A, with one workgroup barrier per
// phase.  So while one wave of a SIMD issues its 32 MFMAs the other runs its softmax,
// instead of the two drifting into step and leaving the matrix unit idle; the MFMA wave
// holds a raised issue priority.  A wave issues VALU at about half its SIMD's rate on its
// own (about 7.5 cycles per wave64 FMA, 16 per exp2), so the softmax phase (~1,200
// cycles) and the MFMA phase (32 MFMAs, ~1,100 cycles) are about even.  Every wave runs
// the same 2 * nblk + 2 phases (the first and last are idle for one group), so the
// barrier counts match by construction.
//
// K and V tiles are double-buffered with different lifetimes: K(j) is read in phases
// 2j (A) and 2j + 1 (B), V(j) in phases 2j + 2 and 2j + 3.  At phase 2m group B (then in
// its softmax phase) copies K(m + 1) (into the K buffer K(m - 1) held) and V(m) (into the
// buffer of V(m - 2)); both have two phases to land and are waited on at the end of phase
// 2m + 1.  The two heads share every K / V tile, so a tile is copied once for 256 query
// rows.  Each wave's arithmetic is polar_fwd16_kernel's, in the same order: the two
// kernels give the same bits.
template <typename T, int D>
__global__ void __launch_bounds__(512, 1) polar_fwd16_pp_kernel(PolarFwdArgs args) {
  constexpr int BM = 128, BN = 64, CPR = D / 8, NT = D / 32, QSTEPS = D / 16;
  constexpr int RPI = 64 / CPR;  // rows per wave copy instruction (1 KB)
  constexpr int TILE = BN * D;   // elements of one K or V tile
  constexpr int NCP = 16 / RPI;  // copy instructions per wave and tile (16 rows per wave)
  static_assert(RPI * NCP == 16, "a wave copies 16 rows");
  __shared__ __attribute__((aligned(16))) T Ks[2 * TILE];
  __shared__ __attribute__((aligned(16))) T Vs[2 * TILE];
  __shared__ float s_bounds[4][2];
  __shared__ float s_vnull[2][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wq = wave & 3;
  const int ql = lane & 31, h = lane >> 5;

  // ---- workgroup -> (query tile, b, head pair): tiles in order of decreasing length; the
  // pairs of one KV group adjacent (and on one XCD when the remap applies)
  const int G = args.Hq / args.Hkv, G2 = G / 2;
  const int per_rank = args.B * args.Hkv * G2;
  const int rank = blockIdx.x / per_rank;
  int u = blockIdx.x % per_rank;
  if (args.xcd_remap) {
    const int x = u & 7, p = u >> 3;
    u = (x + 8 * (p / G2)) * G2 + p % G2;
  }
  const int kvg = u / G2;  // b * Hkv + kv head
  const int b = kvg / args.Hkv, hk = kvg % args.Hkv;
  const int hq = hk * G + 2 * (u % G2) + grp;
  const int q0 = (args.n_qtiles - 1 - rank) * BM;
  const int Tq = args.Tq, Tk = args.Tk;

  const int hq_u = __builtin_amdgcn_readfirstlane(hq);
  const float lg_raw = args.len_gain_raw[hq_u], ns_raw = args.null_slope_raw[hq_u];
  const float nb = args.null_base[hq_u], mb_raw = args.mag_beta_raw[hq_u];
  const int qi = q0 + wq * 32 + ql;
  const bool q_ok = qi < Tq;
  const float n_ld = args.n_keys[min(qi, Tq - 1)];

  const T* qp = (const T*)args.q + b * args.q_sb + hq * args.q_sh;
  const T* kp = (const T*)args.k + b * args.k_sb + hk * args.k_sh;
  const T* vp = (const T*)args.v + b * args.v_sb + hk * args.v_sh;

  // ---- direct copies, issued by group B only (at even phases it is in its softmax
  // phase, so the MFMA group's instruction stream carries no copies): wave w of the group
  // copies rows 16 w .. 16 w + 15 of a tile, RPI rows per
  // instruction, lane l at chunk position l % CPR of row row0 + l / CPR (the logical
  // chunk the swizzle of that tile row stores there: the swizzle depends on the row
  // modulo 16, so it is taken from the tile row, not from the row within the wave's 8).  Full blocks put the wave's row in the scalar offset; a partial last
  // block puts the whole row offset into the range-checked per-lane offset.
  // (the per-lane offsets are recomputed from a laundered lane index at each tile, where
  // keeping them would hold registers through the whole loop.  Instruction r covers tile
  // rows row0 .. row0 + RPI - 1 with row0 a multiple of RPI, and for these widths the
  // swizzle splits as f(row0 + lr) = f(lr) ^ f(row0): the lane's chunk position lc ^ f(lr)
  // is computed once per tile and each instruction XORs in the wave-uniform f(row0).)
  // One buffer descriptor per tensor slice, built once: the range ends at the last key row,
  // so rows past Tk (only ever addressed through the range-checked per-lane offset of a
  // partial last block) read as zeros; a full block puts its offset in the scalar offset.
  const uint32_t kst2 = (uint32_t)args.k_st * 2u, vst2 = (uint32_t)args.v_st * 2u;
  const auto krs = buffer_rsrc(kp, Tk > 0 ? (uint32_t)(Tk - 1) * kst2 + 2u * D : 0u);
  const auto vrs = buffer_rsrc(vp, Tk > 0 ? (uint32_t)(Tk - 1) * vst2 + 2u * D : 0u);
  auto copy_tile = [&](__amdgpu_buffer_rsrc_t rs, uint32_t st2, int blk, T* dst) __attribute__((always_inline)) {
    const uint32_t boff = (uint32_t)blk * (uint32_t)BN * st2;
    uint32_t ln = (uint32_t)lane;
    asm volatile("" : "+v"(ln));
    const uint32_t lr = (ln / CPR) % RPI, lc = ln % CPR;
    const uint32_t cl = lc ^ (uint32_t)lds_swizzle<CPR>((int)lr);  // chunk position, lane part
    const uint32_t ro = lr * st2;                                   // row offset, lane part
    if (blk * BN + BN <= Tk) {
#pragma unroll
      for (int r = 0; r < NCP; ++r) {
        const uint32_t row0 = 16u * wq + RPI * r;
        dma_buf16(rs, ro + 16u * (cl ^ (uint32_t)lds_swizzle<CPR>((int)row0)), boff + row0 * st2, dst + row0 * D);
      }
    } else {
#pragma unroll
      for (int r = 0; r < NCP; ++r) {
        const uint32_t row0 = 16u * wq + RPI * r;
        dma_buf16(rs, boff + ro + row0 * st2 + 16u * (cl ^ (uint32_t)lds_swizzle<CPR>((int)row0)), 0,
                  dst + row0 * D);
      }
    }
  };
  auto swz = [](int r, int c) { return r * D + 8 * (c ^ lds_swizzle<CPR>(r)); };

  // ---- prologue: the query operand, the null vector of the wave's head
  u32x4 qreg16[QSTEPS];
#pragma unroll
  for (int s = 0; s < QSTEPS; ++s)
    qreg16[s] = q_ok ? *(const u32x4*)(qp + (int64_t)qi * args.q_st + 16 * s + 8 * h)
                     : u32x4{0, 0, 0, 0};
  if (64 * wq < D)
    dma_buf4(buffer_rsrc(args.v_null + (int64_t)hq * D, (uint32_t)D * 4u), 4u * (uint32_t)lane,
             256u * (uint32_t)wq, s_vnull[grp] + 64 * wq);

  const float n_raw = q_ok ? n_ld : 0.f;
  float n_cal = n_raw;
  if (args.window > 0 && !args.preserve_length) n_cal = fminf(n_cal, (float)args.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float spg = softplus(lg_raw);
  const float sps = softplus(ns_raw);
  const float mbeta = softplus(mb_raw);
  const float temp = 1.f + spg * logf(n_cal);
  const float nullv = nb + sps * sqrtf(logf(n_cal + 1.f));
  const float c1 = temp * kLog2e * (1.f / sqrtf((float)D));

  // ---- key-loop bounds: both groups hold the same query rows, so group A's waves publish
  {
    float lo = q_ok ? n_raw : 3.0e38f, hi = q_ok ? n_raw : -1.f;
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0 && grp == 0) {
      s_bounds[wq][0] = lo;
      s_bounds[wq][1] = hi;
    }
  }
  __syncthreads();
  const float w_nlo = s_bounds[wq][0], w_nhi = s_bounds[wq][1];
  float g_nlo = s_bounds[0][0], g_nhi = s_bounds[0][1];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    g_nlo = fminf(g_nlo, s_bounds[w][0]);
    g_nhi = fmaxf(g_nhi, s_bounds[w][1]);
  }
  int kend = 0, kbeg = 0;
  if (g_nhi > 0.f) {
    const float hiF = fminf(g_nhi, (float)Tk);
    kend = (int)ceilf(hiF);
    if (args.is_causal) kend = min(kend, min(q0 + BM, Tk));
    if (args.window > 0) kbeg = max((int)floorf(g_nlo) - args.window, 0);
    kbeg = (kbeg / BN) * BN;
  }
  // the bounds are uniform (read from LDS by every lane): made scalar here, so every copy's
  // block offset is scalar arithmetic -- a vector-computed scalar offset would reach the
  // inline-asm copies through v_readfirstlane, whose SGPR write the copy may read stale
  const int nblk_beg = __builtin_amdgcn_readfirstlane(kbeg / BN);
  const int nblk_end = __builtin_amdgcn_readfirstlane((kend + BN - 1) / BN);
  const int nblk = nblk_end > nblk_beg ? nblk_end - nblk_beg : 0;
  if (nblk > 0 && grp == 1) copy_tile(krs, kst2, nblk_beg, Ks);  // K(0) into K buffer 0

#pragma unroll
  for (int s = 0; s < QSTEPS; ++s) asm volatile("" ::"v"(qreg16[s]));

  float m_run = kSentinel, l_part = 0.f, q2_part = 0.f;
  f32x16 oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};
  f32x16 sacc[2] = {f32x16{}, f32x16{}};
  u32x4 pb[4] = {};

  const int arow = a_row_key(ql);
  const int gq = lane >> 4, sl = lane & 15;
  const int vkey = 8 * (gq >> 1) + (sl >> 2);
  const int vcol = 16 * (gq & 1) + 4 * (sl & 3);

  // MFMA phase of local block j: PV(j - 1) from V buffer (j - 1) % 2, then S(j) from K
  // buffer j % 2.  JP = j % 2 is a compile-time constant, so every LDS operand address is
  // a loop-invariant lane offset plus an immediate.
  // MFMA phase of local block j: PV(j - 1) from V buffer (j - 1) % 2, then S(j) from K
  // buffer j % 2.  JP = j % 2 is a compile-time constant, so every LDS operand address is
  // a loop-invariant lane offset plus an immediate.  One wave per SIMD issues MFMAs in
  // this phase, so its operand reads run ahead explicitly: V^T fragments three MFMAs
  // ahead, K fragments two steps (four MFMAs) ahead.
  auto mfma_phase = [&](int j, auto JP) __attribute__((always_inline)) {
    constexpr int jp = decltype(JP)::value;
    __builtin_amdgcn_s_setprio(1);  // the MFMA wave first when both waves of a SIMD can issue
    if (j >= 1) {
      const T* Vb = Vs + (jp ^ 1) * TILE;
      auto vfrag = [&](int i) __attribute__((always_inline)) {
        const int t = i % NT, ps = i / NT;
        const int kr = 16 * ps + vkey, col = 32 * t + vcol;
        const u32x2 lo = lds_read_tr16(Vb + swz(kr, col >> 3) + (col & 7));
        const u32x2 hi = lds_read_tr16(Vb + swz(kr + 4, col >> 3) + (col & 7));
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      constexpr int NV = 4 * NT, VD = 3;
      u32x4 vq[VD];
#pragma unroll
      for (int i = 0; i < VD; ++i) vq[i] = vfrag(i);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        oacc[i % NT] = mfma32<T>(vq[i % VD], pb[i / NT], oacc[i % NT]);
        if (i + VD < NV) vq[i % VD] = vfrag(i + VD);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * VD, 0);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i + VD < NV) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
    }
    if (j < nblk) {
      const T* Kb = Ks + jp * TILE;
      u32x4 kf[2][2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        kf[st][0] = *(const u32x4*)(Kb + swz(arow, 2 * st + h));
        kf[st][1] = *(const u32x4*)(Kb + swz(32 + arow, 2 * st + h));
      }
#pragma unroll
      for (int st = 0; st < QSTEPS; ++st) {
        sacc[0] = mfma32<T>(kf[st & 1][0], qreg16[st], st ? sacc[0] : f32x16{});
        sacc[1] = mfma32<T>(kf[st & 1][1], qreg16[st], st ? sacc[1] : f32x16{});
        if (st + 2 < QSTEPS) {
          kf[st & 1][0] = *(const u32x4*)(Kb + swz(arow, 2 * (st + 2) + h));
          kf[st & 1][1] = *(const u32x4*)(Kb + swz(32 + arow, 2 * (st + 2) + h));
        }
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int st = 0; st < QSTEPS; ++st) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        if (st + 2 < QSTEPS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // VALU phase of local block j: mask (blocks crossing a row's valid range), the
  // optimistic exponentials against the running max, the sums, and the rare rescale
  constexpr float kSafe = __is_same(T, bf16) ? 1048576.f : 16384.f;
  auto valu_phase = [&](int j) __attribute__((always_inline)) {
    const int k0 = (nblk_beg + j) * BN;
    const bool full = (k0 + BN <= (int)fminf(w_nlo, (float)Tk)) &&
                      (args.window <= 0 || (float)k0 >= w_nhi - (float)args.window);
    if (!full) {
      const float tkf = (float)Tk;
      const int key_hi = (int)ceilf(fminf(n_raw, tkf)) - k0;
      const int key_lo =
          args.window > 0 ? (int)ceilf(fminf(n_raw - (float)args.window, tkf)) - k0 : -(1 << 30);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = st_key(jj, i, h);
          sacc[jj][i] = ((key < key_hi) & (key >= key_lo)) ? sacc[jj][i] : -INFINITY;
        }
    }
    float ls = 0.f, qs = 0.f;
    auto exp_pack = [&]() __attribute__((always_inline)) {
      const float neg_m = -m_run;
      ls = qs = 0.f;
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const int jj = ps >> 1, base = 8 * (ps & 1);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[jj][base + 2 * w], c1, neg_m));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[jj][base + 2 * w + 1], c1, neg_m));
          pb[ps][w] = pack2<T>(p0, p1);
        }
      }
      const uint32_t one2 = pack2<T>(1.f, 1.f);
#pragma unroll
      for (int ps = 0; ps < 4; ++ps)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          ls = dot2<T>(pb[ps][w], one2, ls);
          qs = dot2<T>(pb[ps][w], pb[ps][w], qs);
        }
    };
    bool redo = j == 0;
    if (!redo) {
      exp_pack();
      redo = __ballot(!(ls <= kSafe)) != 0;
    }
    if (redo) {
      float mx = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[jj][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx * c1);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
      q2_part *= alpha * alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) oacc[t] *= alpha;
      exp_pack();
    }
    l_part += ls;
    q2_part += qs;
  };

  // ---- the phases.  Global phase p ends with a workgroup barrier for every wave, NP =
  // 2 nblk + 2 of them.  Group A: MFMA(j) at p = 2j (j = 0 .. nblk), softmax(j) at 2j + 1;
  // group B one phase later (idle at p = 0).  Copies K(m + 1), V(m) at every even p = 2m,
  // waited on at the end of the odd phase that follows.  Each group runs its own straight
  // loop over pairs of blocks, so buffer parities are compile-time constants.
  auto copies = [&](int m, auto MP) __attribute__((always_inline)) {
    constexpr int mp = decltype(MP)::value;  // m % 2
    if (grp == 0) return;
    if (m + 1 < nblk) copy_tile(krs, kst2, nblk_beg + m + 1, Ks + (mp ^ 1) * TILE);
    if (m < nblk) copy_tile(vrs, vst2, nblk_beg + m, Vs + mp * TILE);
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  if (nblk > 0) {
    wait_vmcnt<0>();
    lds_barrier();  // K(0) has landed for every wave
    if (grp == 0) {
      for (int j = 0;; j += 2) {
        copies(j, C0{});            // p = 2j
        mfma_phase(j, C0{});
        lds_barrier();
        if (j == nblk) break;
        valu_phase(j);              // p = 2j + 1
        wait_vmcnt<0>();
        lds_barrier();
        copies(j + 1, C1{});        // p = 2j + 2
        mfma_phase(j + 1, C1{});
        lds_barrier();
        if (j + 1 == nblk) break;
        valu_phase(j + 1);          // p = 2j + 3
        wait_vmcnt<0>();
        lds_barrier();
      }
      wait_vmcnt<0>();              // p = 2 nblk + 1: idle
      lds_barrier();
    } else {
      copies(0, C0{});              // p = 0: idle
      lds_barrier();
      for (int j = 0;; j += 2) {
        mfma_phase(j, C0{});        // p = 2j + 1
        wait_vmcnt<0>();
        lds_barrier();
        if (j == nblk) break;
        copies(j + 1, C1{});        // p = 2j + 2
        valu_phase(j);
        lds_barrier();
        mfma_phase(j + 1, C1{});    // p = 2j + 3
        wait_vmcnt<0>();
        lds_barrier();
        if (j + 1 == nblk) break;
        copies(j + 2, C0{});        // p = 2j + 4
        valu_phase(j + 1);
        lds_barrier();
      }
    }
  }
  wait_vmcnt<0>();  // the null vector has landed (also with no key block) ...
  __syncthreads();  // ... for every wave

  // ---- fold the null sink, normalise, magnitude (as polar_fwd16_kernel)
  float L = l_part + __shfl_xor(l_part, 32, 64);
  float Q2 = q2_part + __shfl_xor(q2_part, 32, 64);
  const float an2 = temp * nullv * kLog2e;
  const float mn = fmaxf(m_run, an2);
  const float al = exp2f(m_run - mn);
  L *= al;
  Q2 *= al * al;
  const float pn = exp2f(an2 - mn);
  const float Z = L + pn;
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
      const float s = oacc[t][i] * al + pn * s_vnull[grp][d];
      oacc[t][i] = s;
      ss += s * s;
    }
  }
  ss += __shfl_xor(ss, 32, 64);
  const float inv = 1.f / fmaxf(sqrtf(ss), args.eps);
  const float n_eff = L * L / fmaxf(Q2, 1e-30f);
  const float m_eff = n_eff * (L / fmaxf(Z, args.eps));
  const float magv = tanhf(mbeta * log1pf(m_eff));

  if (q_ok) {
    const int64_t row = ((int64_t)b * args.Hq + hq) * args.Tq + qi;
    T* cp = (T*)args.c + b * args.c_sb + hq * args.c_sh + qi * args.c_st;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * t + 8 * g4 + 4 * h;
        u32x2 pk = {pack2<T>(oacc[t][4 * g4] * inv, oacc[t][4 * g4 + 1] * inv),
                    pack2<T>(oacc[t][4 * g4 + 2] * inv, oacc[t][4 * g4 + 3] * inv)};
        *(u32x2*)(cp + d) = pk;
      }
    }
    if (h == 0) {
      ((T*)args.mag)[b * args.m_sb + hq * args.m_sh + qi * args.m_st] = (T)magv;
      if (args.stat_m) args.stat_m[row] = mn * kLn2;
      if (args.stat_l) args.stat_l[row] = L;
      if (args.stat_q2) args.stat_q2[row] = Q2;
    }
    if (args.stat_s) {
      float* sp = args.stat_s + row * D;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d = 32 * t + 8 * g4 + 4 * h;
          f32x4 x = {oacc[t][4 * g4], oacc[t][4 * g4 + 1], oacc[t][4 * g4 + 2], oacc[t][4 * g4 + 3]};
          *(f32x4*)(sp + d) = x;
        }
    }
  }
}

template <typename T, int D>
static int launch_fwd(PolarFwdArgs a, hipStream_t stream) {
  const int G = a.Hq / a.Hkv;
  if constexpr (sizeof(T) == 2) {
    // the ping-pong kernel addresses a (b, KV head) slice of k / v through one 32-bit buffer range
    const bool slices32 = (int64_t)a.Tk * a.k_st * 2 < (1ll << 32) && (int64_t)a.Tk * a.v_st * 2 < (1ll << 32);
    if (G % 2 == 0 && !a.tile_seq_start && slices32) {
      // two query heads of a KV group per workgroup, the ping-pong schedule
      const int64_t per_rank = (int64_t)a.B * a.Hkv * (G / 2);
      a.xcd_remap = (per_rank % (8 * (G / 2)) == 0) ? 1 : 0;
      polar_fwd16_pp_kernel<T, D><<<dim3((unsigned)(a.n_qtiles * per_rank)), dim3(512), 0, stream>>>(a);
      return check_launch("polar_attention_fwd");
    }
    // one query tile per workgroup
    const int64_t per_rank = (int64_t)a.B * a.Hq;
    a.xcd_remap = (per_rank % (8 * G) == 0) ? 1 : 0;
    polar_fwd16_kernel<T, D><<<dim3((unsigned)(a.n_qtiles * per_rank)), dim3(256), 0, stream>>>(a);
  } else {
    // a pair of query tiles (the i-th longest and the i-th shortest) per workgroup
    const int64_t units = (int64_t)((a.n_qtiles + 1) / 2) * a.B * a.Hq;
    a.xcd_remap = (units % (8 * G) == 0) ? 1 : 0;
    polar_fwd_kernel<T, D><<<dim3((unsigned)units), dim3(256), 0, stream>>>(a);
  }
  return check_launch("polar_attention_fwd");
}

}  // namespace atma

extern "C" int atma_polar_attention_fwd(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb,
    int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const float* n_keys, const float* v_null, const float* null_base, const float* null_slope_raw,
    const float* len_gain_raw, const float* mag_beta_raw, void* c, void* mag, float* stat_m,
    float* stat_l, float* stat_q2, float* stat_s, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq,
    int64_t Tk, int64_t d, int dtype, int is_causal, int64_t window, int preserve_length, float eps,
    void* stream) {
  using namespace atma;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Tq < 0 || Tk < 0)
    return set_error(ATMA_ERR_INVALID, "polar_attention_fwd: bad sizes");
  if (Hq % Hkv) return set_error(ATMA_ERR_INVALID, "polar_attention_fwd: Hq %% Hkv != 0");
  if (is_causal && Tq != Tk)
    return set_error(ATMA_ERR_INVALID,
                     "polar_attention_fwd: is_causal=True requires Tq == Tk (got Tq=%lld, Tk=%lld)",
                     (long long)Tq, (long long)Tk);
  if (d != 64 && d != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_fwd: head_dim %lld (supported: 64, 128)",
                     (long long)d);
  if (Tq > (1 << 30) || Tk > (1 << 30) || B * Hq > (1 << 24) || (Tq + 127) / 128 * B * Hq > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "polar_attention_fwd: sizes too large");
  if (B == 0 || Tq == 0) return ATMA_OK;
  if (!q || !k || !v || !n_keys || !v_null || !null_base || !null_slope_raw || !len_gain_raw ||
      !mag_beta_raw || !c || !mag)
    return set_error(ATMA_ERR_INVALID, "polar_attention_fwd: null pointer");
  const int es = dtype_size(dtype);
  if (!es) return set_error(ATMA_ERR_INVALID, "polar_attention_fwd: unknown dtype %d", dtype);
  auto al16 = [&](const void* p, int64_t s1, int64_t s2, int64_t s3) {
    return ((uintptr_t)p % 16 == 0) && ((s1 * es) % 16 == 0) && ((s2 * es) % 16 == 0) &&
           ((s3 * es) % 16 == 0);
  };
  if (!al16(q, q_sb, q_sh, q_st) || !al16(k, k_sb, k_sh, k_st) || !al16(v, v_sb, v_sh, v_st) ||
      (uintptr_t)c % 16)
    return set_error(ATMA_ERR_INVALID, "polar_attention_fwd: tensors must be 16-byte aligned rows");
  if (k_st >= (1 << 24) || v_st >= (1 << 24))
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_fwd: key/value row stride too large");
  PolarFwdArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.n_keys = n_keys; a.v_null = v_null; a.null_base = null_base;
  a.null_slope_raw = null_slope_raw; a.len_gain_raw = len_gain_raw; a.mag_beta_raw = mag_beta_raw;
  a.c = c; a.mag = mag; a.stat_m = stat_m; a.stat_l = stat_l; a.stat_q2 = stat_q2; a.stat_s = stat_s;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.Tq = (int)Tq; a.Tk = (int)Tk;
  a.is_causal = is_causal ? 1 : 0;
  a.window = window > 0 ? (int)window : 0;
  a.preserve_length = preserve_length ? 1 : 0;
  a.eps = eps;
  a.n_qtiles = (int)((Tq + 127) / 128);
  a.c_st = d; a.c_sh = Tq * d; a.c_sb = Hq * Tq * d;  // c, mag contiguous (B, Hq, Tq[, d])
  a.m_st = 1; a.m_sh = Tq; a.m_sb = Hq * Tq;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_BF16: return d == 128 ? launch_fwd<bf16, 128>(a, s) : launch_fwd<bf16, 64>(a, s);
    case ATMA_F16: return d == 128 ? launch_fwd<f16, 128>(a, s) : launch_fwd<f16, 64>(a, s);
    default: return d == 128 ? launch_fwd<float, 128>(a, s) : launch_fwd<float, 64>(a, s);
  }
}

extern "C" int atma_polar_attention_packed_fwd(
    const void* q, int64_t q_st, int64_t q_sh, const void* k, int64_t k_st, int64_t k_sh,
    const void* v, int64_t v_st, int64_t v_sh, const int32_t* tile_seq_start,
    const int32_t* tile_q_start, const int32_t* tile_seq_len, int64_t n_tiles,
    const float* v_null, const float* null_base, const float* null_slope_raw,
    const float* len_gain_raw, const float* mag_beta_raw, void* c, int64_t c_st, int64_t c_sh,
    void* mag, int64_t m_st, int64_t m_sh, int64_t total_tokens, int64_t Hq, int64_t Hkv,
    int64_t d, int dtype, int64_t window, float eps, void* stream) {
  using namespace atma;
  if (n_tiles < 0 || total_tokens < 0 || Hq <= 0 || Hkv <= 0)
    return set_error(ATMA_ERR_INVALID, "polar_attention_packed_fwd: bad sizes");
  if (Hq % Hkv) return set_error(ATMA_ERR_INVALID, "polar_attention_packed_fwd: Hq %% Hkv != 0");
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_packed_fwd: 16-bit inputs only");
  if (d != 64 && d != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_packed_fwd: head_dim %lld (supported: 64, 128)",
                     (long long)d);
  if (total_tokens > (1 << 30) || n_tiles * Hq > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "polar_attention_packed_fwd: sizes too large");
  if (n_tiles == 0 || total_tokens == 0) return ATMA_OK;
  if (!q || !k || !v || !tile_seq_start || !tile_q_start || !tile_seq_len || !v_null || !null_base ||
      !null_slope_raw || !len_gain_raw || !mag_beta_raw || !c || !mag)
    return set_error(ATMA_ERR_INVALID, "polar_attention_packed_fwd: null pointer");
  auto al16 = [](const void* p, int64_t s1, int64_t s2) {
    return ((uintptr_t)p % 16 == 0) && ((s1 * 2) % 16 == 0) && ((s2 * 2) % 16 == 0);
  };
  if (!al16(q, q_st, q_sh) || !al16(k, k_st, k_sh) || !al16(v, v_st, v_sh) || !al16(c, c_st, c_sh))
    return set_error(ATMA_ERR_INVALID, "polar_attention_packed_fwd: tensors must be 16-byte aligned rows");
  if (q_st >= (1 << 24) || k_st >= (1 << 24) || v_st >= (1 << 24))
    // a 64-row key block is copied through one buffer descriptor with 32-bit offsets
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_packed_fwd: token stride too large");
  PolarFwdArgs a{};
  a.q = q; a.q_st = q_st; a.q_sh = q_sh;
  a.k = k; a.k_st = k_st; a.k_sh = k_sh;
  a.v = v; a.v_st = v_st; a.v_sh = v_sh;
  a.v_null = v_null; a.null_base = null_base; a.null_slope_raw = null_slope_raw;
  a.len_gain_raw = len_gain_raw; a.mag_beta_raw = mag_beta_raw;
  a.c = c; a.mag = mag;
  a.c_st = c_st; a.c_sh = c_sh; a.m_st = m_st; a.m_sh = m_sh;
  a.B = 1; a.Hq = (int)Hq; a.Hkv = (int)Hkv;
  a.is_causal = 1;
  a.window = window > 0 ? (int)window : 0;
  a.eps = eps;
  a.tile_seq_start = tile_seq_start; a.tile_q_start = tile_q_start; a.tile_seq_len = tile_seq_len;
  a.total_tokens = (int)total_tokens;
  const int64_t G = Hq / Hkv;
  const int64_t grid = n_tiles * Hq;
  a.xcd_remap = (grid % (8 * G) == 0) ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16) {
    if (d == 128) polar_fwd16_kernel<bf16, 128><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
    else polar_fwd16_kernel<bf16, 64><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
  } else {
    if (d == 128) polar_fwd16_kernel<f16, 128><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
    else polar_fwd16_kernel<f16, 64><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
  }
  return check_launch("polar_attention_packed_fwd");
}
