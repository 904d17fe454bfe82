// Polar attention backward: the two O(T^2) loops of _polar_backward
// (kernel/polar_triton.py:861-1155).  The per-query preamble (gs, gL, gQ2 from the saved
// statistics M, L, Q2, s and the output cotangents) and the parameter-gradient assembly
// are O(B*H*T*d) and stay on the host side; these kernels take their results.
//
// For a valid (query i, key j) pair, with sig = q_i.k_j / sqrt(d), a = sig * temp_i and
// p = exp(a - M_i) (the saved reference max; 0 for masked pairs):
//   dLdp = gs_i.v_j + gL_i + 2 gQ2_i p,   da = dLdp * p,   gsig = da * temp_i
//   dq_i += gsig * k_j / sqrt(d)     dt_i += da * sig
//   dk_j += gsig * q_i / sqrt(d)     dv_j += p * gs_i
// Validity is the forward's: key j < min(n_i, Tk) and, with a window, j >= n_i - window.
//
// MI355X mapping.  16-wide MFMA tiles (v_mfma_f32_16x16x32_{bf16,f16} for 16-bit inputs,
// v_mfma_f32_16x16x4f32 for fp32), operands staged in padded row-major LDS tiles:
//  * dq kernel: a workgroup owns 64 query rows of one head (16 per wave, q and gs as A
//    fragments in registers) and walks 64-key blocks: S and dP (queries x keys) on MFMA,
//    the elementwise gradient in registers, dS through a per-wave LDS tile (row-major, so
//    it is read back as the A operand), then dQ += dS K with K^T fragments taken by
//    transposing reads of the row-major K tile.
//  * dk/dv kernel: a workgroup owns 64 keys of one KV head for ONE query head (k and v
//    rows as A fragments) and walks its 64-query blocks: S^T and dP^T on MFMA, P^T and
//    dS^T through per-wave LDS tiles, dV += P^T gs and dK += dS^T Q with gs / Q fragments
//    by transposing reads.  Its dk / dv rows go to that query head's slice of a
//    (B, Hq, Tk, D) output (written once, no atomics); with grouped heads the caller sums
//    the G slices of a group.  One workgroup per query head (not per KV head) gives G
//    times the workgroups, which a causal T = 2,048 grid needs to fill 256 CUs.
//  * Both kernels keep the next block's tiles in flight in registers while the current
//    block is computed (one LDS buffer, two barriers per block), and order the grid
//    longest-first (the causal work of a query block grows with its index, of a key
//    block shrinks), so the short tail fills in behind the long blocks.
// Products accumulate in fp32; 16-bit inputs round P and dS to the input dtype for the
// second products, as the reference does (kernel/polar_triton.py:942,1023-1024).
#include <type_traits>

#include "common.h"

namespace atma {

struct PolarBwdArgs {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  const void* k;
  int64_t k_sb, k_sh, k_st;
  const void* v;
  int64_t v_sb, v_sh, v_st;
  const void* gs;
  int64_t g_sb, g_sh, g_st;
  const float* gL;      // (B, Hq, Tq)
  const float* gQ2;     // (B, Hq, Tq)
  const float* M;       // (B, Hq, Tq) natural-log reference max of the forward
  const float* temp;    // (Hq, Tq)
  const float* n_keys;  // (Tq,)
  void* dq;             // (B, Hq, Tq, D) in the input dtype
  float* dt;            // (B, Hq, Tq)
  // (B, Hq, Tk, D): each query head's share, grouped heads summed by the caller; fp32 for
  // fp32 and fp16 inputs, bf16 for bf16 inputs (BwShare<T>)
  void* dk;
  void* dv;
  int B, Hq, Hkv, Tq, Tk;
  int is_causal, window;
  float scale;
};

template <typename T>
using BwFrag = std::conditional_t<sizeof(T) == 2, u32x4, float>;
template <typename T>
using BwShare = std::conditional_t<std::is_same_v<T, bf16>, bf16, float>;
template <typename T>
constexpr int kBwK = sizeof(T) == 2 ? 32 : 4;  // MFMA k depth
template <typename T>
constexpr int kBwPad = sizeof(T) == 2 ? 8 : 4;  // LDS row padding (elements): 16 B

template <typename T>
__device__ __forceinline__ f32x4 bw_mma(const BwFrag<T>& a, const BwFrag<T>& b, const f32x4& c) {
  if constexpr (sizeof(T) == 2) return mfma16x16x32<T>(a, b, c);
  else return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Fragment (A rows or B columns) whose 16 lines are rows r0.. of a row-major tile with
// the k dimension contiguous: lane l takes line r0 + l % 16 at k = k0 + (8 | 1) (l / 16) ...
template <typename T>
__device__ __forceinline__ BwFrag<T> bw_rows(const T* base, int ld, int r0, int k0, int lane) {
  if constexpr (sizeof(T) == 2)
    return *(const u32x4*)(base + (r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
  else
    return base[(r0 + (lane & 15)) * ld + k0 + (lane >> 4)];
}
// B fragment with k along the rows of a row-major tile: lane l takes column n0 + l % 16 at
// rows k0 + 8 (l / 16) .. + 7 (two transposing reads of 4 rows) or, for fp32, row
// k0 + l / 16.
template <typename T>
__device__ __forceinline__ BwFrag<T> bw_cols(const T* base, int ld, int k0, int n0, int lane) {
  if constexpr (sizeof(T) == 2) {
    const int g = lane >> 4, i = lane & 15;
    const T* p = base + (k0 + 8 * g + (i >> 2)) * ld + n0 + 4 * (i & 3);
    const u32x2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * ld);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  } else {
    return base[(k0 + (lane >> 4)) * ld + n0 + (lane & 15)];
  }
}
// A fragment of 16 rows straight from global memory (rows past `rows` read as zeros).
template <typename T>
__device__ __forceinline__ BwFrag<T> bw_global_rows(const T* base, int64_t st, int r0, int rows, int k0,
                                                     int lane) {
  const int r = r0 + (lane & 15);
  if constexpr (sizeof(T) == 2) {
    return r < rows ? *(const u32x4*)(base + (int64_t)r * st + k0 + 8 * (lane >> 4)) : u32x4{0, 0, 0, 0};
  } else {
    return r < rows ? base[(int64_t)r * st + k0 + (lane >> 4)] : 0.f;
  }
}
// Cooperative copy of rows r0 .. r0 + 63 of a row-major (rows, D) source with row stride st
// into a padded LDS tile (rows past `rows` become zeros), 16 bytes per thread and step, in
// two halves: bw_fetch issues the global loads into registers, bw_put writes them to LDS,
// so the loads of the next block can be in flight during the current block's products.
template <typename T, int D>
struct BwTile {
  static constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  static constexpr int CPR = D / EPC;              // chunks per row
  static constexpr int N = 64 * CPR / 256;         // chunks per thread
  u32x4 x[N];
};
template <typename T, int D>
__device__ __forceinline__ void bw_fetch(BwTile<T, D>& t, const T* src, int64_t st, int r0, int rows, int tid) {
  using TT = BwTile<T, D>;
#pragma unroll
  for (int i = 0; i < TT::N; ++i) {
    const int c = tid + 256 * i, r = c / TT::CPR, e = (c % TT::CPR) * TT::EPC;
    const int gr = r0 + r;
    t.x[i] = gr < rows ? *(const u32x4*)(src + (int64_t)gr * st + e) : u32x4{0, 0, 0, 0};
  }
}
template <typename T, int D>
__device__ __forceinline__ void bw_put(T* dst, const BwTile<T, D>& t, int tid) {
  using TT = BwTile<T, D>;
  constexpr int LD = D + kBwPad<T>;
#pragma unroll
  for (int i = 0; i < TT::N; ++i) {
    const int c = tid + 256 * i, r = c / TT::CPR, e = (c % TT::CPR) * TT::EPC;
    *(u32x4*)(dst + r * LD + e) = t.x[i];
  }
}

template <typename T>
__device__ __forceinline__ T bw_round(float x) {
  return (T)x;
}

// ---------------------------------------------------------------------------------------
// dq, dt: workgroup = (64-row query tile, b * Hq + hq)
template <typename T, int D>
__global__ void __launch_bounds__(256) polar_bwd_dq_kernel(PolarBwdArgs a) {
  constexpr int BM = 64, BN = 64, KD = kBwK<T>, LD = D + kBwPad<T>, SLD = BN + kBwPad<T>;
  __shared__ __attribute__((aligned(16))) T Ks[BN * LD];
  __shared__ __attribute__((aligned(16))) T Vs[BN * LD];
  __shared__ __attribute__((aligned(16))) T Sd[4][16 * SLD];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.Hq / a.Hkv;
  // grid (B * Hq, query blocks) with the last query block (the most keys) first
  const int bh = blockIdx.x, b = bh / a.Hq, hq = bh % a.Hq, hk = hq / G;
  const int q0 = ((int)gridDim.y - 1 - (int)blockIdx.y) * BM, r0 = q0 + 16 * wave;
  const T* qp = (const T*)a.q + b * a.q_sb + hq * a.q_sh;
  const T* gp = (const T*)a.gs + b * a.g_sb + hq * a.g_sh;
  const T* kp = (const T*)a.k + b * a.k_sb + hk * a.k_sh;
  const T* vp = (const T*)a.v + b * a.v_sb + hk * a.v_sh;

  BwFrag<T> qf[D / KD], gf[D / KD];
#pragma unroll
  for (int s = 0; s < D / KD; ++s) {
    qf[s] = bw_global_rows<T>(qp, a.q_st, r0, a.Tq, KD * s, lane);
    gf[s] = bw_global_rows<T>(gp, a.g_st, r0, a.Tq, KD * s, lane);
  }
  // per-row values for the C rows of this lane: r0 + 4 (lane / 16) + j
  float m2[4], c1[4], gl[4], gq2[4], nr[4], tp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = r0 + 4 * (lane >> 4) + j;
    const bool ok = row < a.Tq;
    const int64_t i = (int64_t)bh * a.Tq + row;
    tp[j] = ok ? a.temp[(int64_t)hq * a.Tq + row] : 1.f;
    m2[j] = ok ? a.M[i] * kLog2e : 0.f;
    c1[j] = a.scale * tp[j] * kLog2e;
    gl[j] = ok ? a.gL[i] : 0.f;
    gq2[j] = ok ? a.gQ2[i] : 0.f;
    nr[j] = ok ? a.n_keys[row] : 0.f;  // no valid key for rows past Tq
  }

  f32x4 dq[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) dq[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float dt[4] = {0.f, 0.f, 0.f, 0.f};

  const int hi = a.is_causal ? min(q0 + BM, a.Tk) : a.Tk;
  const int lo = a.window > 0 ? (max(q0 - a.window, 0) / BN) * BN : 0;
  T* sd = Sd[wave];
  BwTile<T, D> kn, vn;  // the next key block, in flight
  if (lo < hi) {
    bw_fetch<T, D>(kn, kp, a.k_st, lo, a.Tk, tid);
    bw_fetch<T, D>(vn, vp, a.v_st, lo, a.Tk, tid);
  }
  for (int k0 = lo; k0 < hi; k0 += BN) {
    __syncthreads();  // every wave is done with the previous block
    bw_put<T, D>(Ks, kn, tid);
    bw_put<T, D>(Vs, vn, tid);
    if (k0 + BN < hi) {
      bw_fetch<T, D>(kn, kp, a.k_st, k0 + BN, a.Tk, tid);
      bw_fetch<T, D>(vn, vp, a.v_st, k0 + BN, a.Tk, tid);
    }
    __syncthreads();
    // S = Q K^T and dP = gs V^T for 4 key tiles of 16
    f32x4 s[4], p[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[t] = p[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / KD; ++ks) {
        s[t] = bw_mma<T>(qf[ks], bw_rows<T>(Ks, LD, 16 * t, KD * ks, lane), s[t]);
        p[t] = bw_mma<T>(gf[ks], bw_rows<T>(Vs, LD, 16 * t, KD * ks, lane), p[t]);
      }
    }
    // elementwise gradient; C element (row 4 (lane / 16) + j, key k0 + 16 t + lane % 16)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int key = k0 + 16 * t + (lane & 15);
      const float kf = (float)key;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool valid = key < a.Tk && kf < nr[j] && (a.window <= 0 || kf >= nr[j] - (float)a.window);
        const float pr = valid ? __builtin_amdgcn_exp2f(s[t][j] * c1[j] - m2[j]) : 0.f;
        const float da = valid ? (p[t][j] + gl[j] + 2.f * gq2[j] * pr) * pr : 0.f;
        dt[j] += da * (s[t][j] * a.scale);
        sd[(4 * (lane >> 4) + j) * SLD + 16 * t + (lane & 15)] = bw_round<T>(da * tp[j]);
      }
    }
    wave_sync();
    // dQ += dS K: A = dS rows (k = keys), B = K with k along its rows
#pragma unroll
    for (int nt = 0; nt < D / 16; ++nt)
#pragma unroll
      for (int ks = 0; ks < BN / KD; ++ks)
        dq[nt] = bw_mma<T>(bw_rows<T>(sd, SLD, 0, KD * ks, lane), bw_cols<T>(Ks, LD, KD * ks, 16 * nt, lane),
                           dq[nt]);
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = r0 + 4 * (lane >> 4) + j;
    float x = dt[j];
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) x += __shfl_xor(x, m, 64);  // the 16 key columns of the row
    if (row < a.Tq) {
      T* out = (T*)a.dq + ((int64_t)bh * a.Tq + row) * D + (lane & 15);
#pragma unroll
      for (int nt = 0; nt < D / 16; ++nt) out[16 * nt] = from_f32<T>(dq[nt][j] * a.scale);
      if ((lane & 15) == 0) a.dt[(int64_t)bh * a.Tq + row] = x;
    }
  }
}

// ---------------------------------------------------------------------------------------
// dk, dv: workgroup = (b * Hq + hq, 64-key tile); writes hq's slice of (B, Hq, Tk, D)
template <typename T, int D>
__global__ void __launch_bounds__(256) polar_bwd_dkdv_kernel(PolarBwdArgs a) {
  constexpr int BK = 64, BQ = 64, KD = kBwK<T>, LD = D + kBwPad<T>, SLD = BQ + kBwPad<T>;
  __shared__ __attribute__((aligned(16))) T Qs[BQ * LD];
  __shared__ __attribute__((aligned(16))) T Gs[BQ * LD];
  __shared__ __attribute__((aligned(16))) T Pt[4][16 * SLD];
  __shared__ __attribute__((aligned(16))) T Dt[4][16 * SLD];
  __shared__ float s_m2[BQ], s_c1[BQ], s_gl[BQ], s_gq2[BQ], s_nr[BQ], s_tp[BQ];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.Hq / a.Hkv;
  // grid (B * Hq, key blocks), key block 0 (the most queries) first
  const int bh = blockIdx.x, b = bh / a.Hq, hq = bh % a.Hq, hk = hq / G;
  const int k0 = blockIdx.y * BK, kr0 = k0 + 16 * wave;
  const T* kp = (const T*)a.k + b * a.k_sb + hk * a.k_sh;
  const T* vp = (const T*)a.v + b * a.v_sb + hk * a.v_sh;
  const T* qp = (const T*)a.q + b * a.q_sb + hq * a.q_sh;
  const T* gp = (const T*)a.gs + b * a.g_sb + hq * a.g_sh;

  BwFrag<T> kf[D / KD], vf[D / KD];
#pragma unroll
  for (int s = 0; s < D / KD; ++s) {
    kf[s] = bw_global_rows<T>(kp, a.k_st, kr0, a.Tk, KD * s, lane);
    vf[s] = bw_global_rows<T>(vp, a.v_st, kr0, a.Tk, KD * s, lane);
  }
  f32x4 dk[D / 16], dv[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) dk[t] = dv[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lo = a.is_causal ? (k0 / BQ) * BQ : 0;
  const int hi = a.window > 0 ? min(k0 + BK + a.window, a.Tq) : a.Tq;
  T* pt = Pt[wave];
  T* dst = Dt[wave];
  // per-query scalars of the next block (thread tid < 64 holds row q0 + tid)
  auto row_vals = [&](int q0, float& tp, float& m, float& gl, float& gq2, float& nr) {
    const int row = q0 + tid;
    const bool ok = tid < BQ && row < a.Tq;
    const int64_t i = (int64_t)bh * a.Tq + row;
    tp = ok ? a.temp[(int64_t)hq * a.Tq + row] : 1.f;
    m = ok ? a.M[i] : 0.f;
    gl = ok ? a.gL[i] : 0.f;
    gq2 = ok ? a.gQ2[i] : 0.f;
    nr = ok ? a.n_keys[row] : 0.f;  // no valid key for rows past Tq
  };
  BwTile<T, D> qn, gn;
  float n_tp = 1.f, n_m = 0.f, n_gl = 0.f, n_gq2 = 0.f, n_nr = 0.f;
  if (lo < hi) {
    bw_fetch<T, D>(qn, qp, a.q_st, lo, a.Tq, tid);
    bw_fetch<T, D>(gn, gp, a.g_st, lo, a.Tq, tid);
    row_vals(lo, n_tp, n_m, n_gl, n_gq2, n_nr);
  }
  for (int q0 = lo; q0 < hi; q0 += BQ) {
    __syncthreads();  // every wave is done with the previous block
    bw_put<T, D>(Qs, qn, tid);
    bw_put<T, D>(Gs, gn, tid);
    if (tid < BQ) {
      s_tp[tid] = n_tp;
      s_c1[tid] = a.scale * n_tp * kLog2e;
      s_m2[tid] = n_m * kLog2e;
      s_gl[tid] = n_gl;
      s_gq2[tid] = n_gq2;
      s_nr[tid] = n_nr;
    }
    if (q0 + BQ < hi) {
      bw_fetch<T, D>(qn, qp, a.q_st, q0 + BQ, a.Tq, tid);
      bw_fetch<T, D>(gn, gp, a.g_st, q0 + BQ, a.Tq, tid);
      row_vals(q0 + BQ, n_tp, n_m, n_gl, n_gq2, n_nr);
    }
    __syncthreads();
    // S^T = K Q^T and dP^T = V gs^T for 4 query tiles of 16
    f32x4 s[4], p[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[t] = p[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / KD; ++ks) {
        s[t] = bw_mma<T>(kf[ks], bw_rows<T>(Qs, LD, 16 * t, KD * ks, lane), s[t]);
        p[t] = bw_mma<T>(vf[ks], bw_rows<T>(Gs, LD, 16 * t, KD * ks, lane), p[t]);
      }
    }
    // C element (key kr0 + 4 (lane / 16) + j, query q0 + 16 t + lane % 16)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int qi = 16 * t + (lane & 15);
      const float nrq = s_nr[qi], c1 = s_c1[qi], m2 = s_m2[qi], glq = s_gl[qi], gq2 = s_gq2[qi];
      const float tpq = s_tp[qi];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = kr0 + 4 * (lane >> 4) + j;
        const float kf_ = (float)key;
        const bool valid = key < a.Tk && kf_ < nrq && (a.window <= 0 || kf_ >= nrq - (float)a.window);
        const float pr = valid ? __builtin_amdgcn_exp2f(s[t][j] * c1 - m2) : 0.f;
        const float da = valid ? (p[t][j] + glq + 2.f * gq2 * pr) * pr : 0.f;
        const int e = (4 * (lane >> 4) + j) * SLD + qi;
        pt[e] = bw_round<T>(pr);
        dst[e] = bw_round<T>(da * tpq);
      }
    }
    wave_sync();
    // dV += P^T gs, dK += dS^T Q: A = the per-wave tiles (k = queries), B = gs / Q
#pragma unroll
    for (int nt = 0; nt < D / 16; ++nt)
#pragma unroll
      for (int ks = 0; ks < BQ / KD; ++ks) {
        dv[nt] = bw_mma<T>(bw_rows<T>(pt, SLD, 0, KD * ks, lane), bw_cols<T>(Gs, LD, KD * ks, 16 * nt, lane),
                           dv[nt]);
        dk[nt] = bw_mma<T>(bw_rows<T>(dst, SLD, 0, KD * ks, lane), bw_cols<T>(Qs, LD, KD * ks, 16 * nt, lane),
                           dk[nt]);
      }
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = kr0 + 4 * (lane >> 4) + j;
    if (row < a.Tk) {
      const int64_t base = ((int64_t)bh * a.Tk + row) * D + (lane & 15);
#pragma unroll
      for (int nt = 0; nt < D / 16; ++nt) {
        ((BwShare<T>*)a.dk)[base + 16 * nt] = from_f32<BwShare<T>>(dk[nt][j] * a.scale);
        ((BwShare<T>*)a.dv)[base + 16 * nt] = from_f32<BwShare<T>>(dv[nt][j]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// 16-bit loops.  Both compute the score tile transposed relative to the output they
// accumulate, so the elementwise results (dS, P) are already the B operand of the second
// products and never go through LDS:
//  * dq: S^T = K Q^T, dP^T = V gs^T (rows = keys, columns = the wave's 16 queries), then
//    dQ^T += K^T dS^T with K^T fragments from transposing LDS reads;
//  * dk/dv: S = Q K^T, dP = gs V^T (rows = queries, columns = the wave's 16 keys), then
//    dV^T += gs^T P and dK^T += Q^T dS with gs^T / Q^T from transposing reads.
// A 32-wide contraction over keys (or queries) takes them in the order the accumulator
// tiles hold them: lane group g's 8 values are rows 32 j + 4 g + [0, 4) of tile 2 j and
// 32 j + 16 + 4 g + [0, 4) of tile 2 j + 1; the transposing reads fetch the A operand in the
// same order.  Shared tiles use unpadded rows with 16-byte chunk c of row r stored at
// c ^ f(r), f(r) = 2 (r mod 8) + (r / 8 mod 2) for 128-element rows: f is a bijection on
// 16 rows (row-fragment reads: 16 rows x one chunk hit 16 distinct positions) and 2 (r mod 8)
// is distinct on the 8 rows a half wave's transposing reads touch (two adjacent chunks per
// row), so both read patterns are free of bank conflicts.  Blocks whose every (key, query)
// pair is valid skip the mask.
template <int CPR>
__device__ __forceinline__ int bw_swz(int r) {
  if constexpr (CPR == 16) return 2 * (r & 7) + ((r >> 3) & 1);
  else return lds_swizzle<CPR>(r);
}
template <int D>
__device__ __forceinline__ int bw_off(int r, int e) {  // element e of row r (e % 8 < 8)
  return r * D + 8 * ((e >> 3) ^ bw_swz<D / 8>(r)) + (e & 7);
}
template <typename T, int D>
__device__ __forceinline__ void bw_put_swz(T* dst, const BwTile<T, D>& t, int tid) {
  using TT = BwTile<T, D>;
#pragma unroll
  for (int i = 0; i < TT::N; ++i) {
    const int c = tid + 256 * i, r = c / TT::CPR, e = (c % TT::CPR) * TT::EPC;
    *(u32x4*)(dst + bw_off<D>(r, e)) = t.x[i];
  }
}
// A fragment: rows r0 + lane % 16 of a swizzled tile, k = k0 + 8 (lane / 16) .. + 7
template <int D, typename T>
__device__ __forceinline__ u32x4 bw_rows_swz(const T* tile, int r0, int k0, int lane) {
  return *(const u32x4*)(tile + bw_off<D>(r0 + (lane & 15), k0 + 8 * (lane >> 4)));
}
// A fragment of the transposed tile: lane (g, i) holds column n0 + i at rows
// 32 j + 4 g + [0, 4) and 32 j + 16 + 4 g + [0, 4) (the accumulator-tile order)
template <int D, typename T>
__device__ __forceinline__ u32x4 bw_tcols_swz(const T* tile, int j, int n0, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int r = 32 * j + 4 * g + (i >> 2), e = n0 + 4 * (i & 3);
  const u32x2 lo = lds_read_tr16(tile + bw_off<D>(r, e)), hi = lds_read_tr16(tile + bw_off<D>(r + 16, e));
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}
// B fragment of the accumulator tiles 2 j, 2 j + 1, rounded to 16 bits
template <typename T>
__device__ __forceinline__ u32x4 bw_pack_b(const f32x4& lo, const f32x4& hi) {
  return u32x4{pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3]), pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3])};
}
__device__ __forceinline__ float bw_uniform(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ float bw_lane(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

// dq, dt for 16-bit inputs: workgroup = (b * Hq + hq, 64-row query tile, last tile first)
template <typename T, int D>
__global__ void __launch_bounds__(256, 3) polar_bwd16_dq_kernel(PolarBwdArgs a) {
  constexpr int BM = 64, BN = 64, KS = D / 32, CPR = D / 8, NDMA = CPR / 4;
  // one key block in LDS, filled by direct-to-LDS copies once every wave is done with the
  // previous one: 32 KiB and at most 168 VGPRs give three workgroups per CU, whose copies
  // and products overlap (a second LDS buffer would allow only two)
  __shared__ __attribute__((aligned(16))) T Ks[BN * D];
  __shared__ __attribute__((aligned(16))) T Vs[BN * D];

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.Hq / a.Hkv;
  const int bh = blockIdx.x, b = bh / a.Hq, hq = bh % a.Hq, hk = hq / G;
  const int q0 = ((int)gridDim.y - 1 - (int)blockIdx.y) * BM, r0 = q0 + 16 * wave;
  const T* qp = (const T*)a.q + b * a.q_sb + hq * a.q_sh;
  const T* gp = (const T*)a.gs + b * a.g_sb + hq * a.g_sh;
  const T* kp = (const T*)a.k + b * a.k_sb + hk * a.k_sh;
  const T* vp = (const T*)a.v + b * a.v_sb + hk * a.v_sh;

  // the wave's 16 query rows as B operands; the lane's query is row r0 + c16
  u32x4 qf[KS], gf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qf[s] = bw_global_rows<T>(qp, a.q_st, r0, a.Tq, 32 * s, lane);
    gf[s] = bw_global_rows<T>(gp, a.g_st, r0, a.Tq, 32 * s, lane);
  }
  const int row = r0 + c16;
  const bool rok = row < a.Tq;
  const int64_t ri = (int64_t)bh * a.Tq + row;
  const float tp = rok ? a.temp[(int64_t)hq * a.Tq + row] : 1.f;
  const float c1 = a.scale * tp * kLog2e;
  const float nm2 = rok ? -a.M[ri] * kLog2e : 0.f;
  const float gl = rok ? a.gL[ri] : 0.f;
  const float g2 = rok ? 2.f * a.gQ2[ri] : 0.f;
  const float nr = rok ? a.n_keys[row] : 0.f;  // no valid key for rows past Tq
  const float nmin = bw_uniform(-row16_max(-nr)), nmax = bw_uniform(row16_max(nr));

  f32x4 dqT[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) dqT[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float dt = 0.f;

  const int hi = a.is_causal ? min(q0 + BM, a.Tk) : a.Tk;
  const int lo = a.window > 0 ? (max(q0 - a.window, 0) / BN) * BN : 0;
  // the (b, hk) slices of k and v as buffers: rows past Tk read as zeros; copy k of wave w
  // fills LDS chunks (NDMA w + k) 64 + lane (row chunk / CPR, stored position chunk % CPR,
  // loaded from global chunk position ^ f(row))
  const auto krs = buffer_rsrc(kp, (uint32_t)((int64_t)a.Tk * a.k_st * 2));
  const auto vrs = buffer_rsrc(vp, (uint32_t)((int64_t)a.Tk * a.v_st * 2));
  uint32_t koff[NDMA], voff[NDMA];
#pragma unroll
  for (int k = 0; k < NDMA; ++k) {
    const int q = (NDMA * wave + k) * 64 + lane, r = q / CPR, c = (q % CPR) ^ bw_swz<CPR>(r);
    koff[k] = (uint32_t)((r * a.k_st + 8 * c) * 2);
    voff[k] = (uint32_t)((r * a.v_st + 8 * c) * 2);
  }
  auto dma_block = [&](int k0) {
    const uint32_t kb = (uint32_t)((int64_t)k0 * a.k_st * 2), vb = (uint32_t)((int64_t)k0 * a.v_st * 2);
#pragma unroll
    for (int k = 0; k < NDMA; ++k) {
      dma_buf16(krs, koff[k] + kb, 0, &Ks[(NDMA * wave + k) * 64 * 8]);
      dma_buf16(vrs, voff[k] + vb, 0, &Vs[(NDMA * wave + k) * 64 * 8]);
    }
  };
  if (lo < hi) dma_block(lo);
  for (int k0 = lo; k0 < hi; k0 += BN) {
    wait_vmcnt<0>();  // this wave's copies of block k0 (and every earlier load) are done
    __syncthreads();  // ... and every wave's
    const T* Kc = Ks;
    const T* Vc = Vs;
    // S^T = K Q^T, dP^T = V gs^T: tile t holds keys k0 + 16 t + 4 g + i, query row
    f32x4 st[4], pt[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u32x4 ka[KS], va[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        ka[s] = bw_rows_swz<D>(Kc, 16 * t, 32 * s, lane);
        va[s] = bw_rows_swz<D>(Vc, 16 * t, 32 * s, lane);
      }
      st[t] = pt[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        st[t] = mfma16x16x32<T>(ka[s], qf[s], st[t]);
        pt[t] = mfma16x16x32<T>(va[s], gf[s], pt[t]);
      }
    }
    const bool full = k0 + BN <= a.Tk && (float)(k0 + BN - 1) < nmin &&
                      (a.window <= 0 || (float)k0 >= nmax - (float)a.window);
    f32x4 ds[4];
    if (full) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(fmaf(st[t][i], c1, nm2));
          const float da = fmaf(g2, pr, pt[t][i] + gl) * pr;
          dt = fmaf(da, st[t][i], dt);
          ds[t][i] = da * tp;
        }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * t + 4 * g + i;
          const float kf = (float)key;
          const bool valid = key < a.Tk && kf < nr && (a.window <= 0 || kf >= nr - (float)a.window);
          const float pr = valid ? __builtin_amdgcn_exp2f(fmaf(st[t][i], c1, nm2)) : 0.f;
          const float da = valid ? fmaf(g2, pr, pt[t][i] + gl) * pr : 0.f;
          dt = fmaf(da, st[t][i], dt);
          ds[t][i] = da * tp;
        }
    }
    // dQ^T += K^T dS^T
    const u32x4 b0 = bw_pack_b<T>(ds[0], ds[1]), b1 = bw_pack_b<T>(ds[2], ds[3]);
#pragma unroll
    for (int nt = 0; nt < D / 16; nt += 4) {
      u32x4 ka[4][2];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j) ka[u][j] = bw_tcols_swz<D>(Kc, j, 16 * (nt + u), lane);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        dqT[nt + u] = mfma16x16x32<T>(ka[u][0], b0, dqT[nt + u]);
        dqT[nt + u] = mfma16x16x32<T>(ka[u][1], b1, dqT[nt + u]);
      }
    }
    __syncthreads();  // every wave is done with the block's tiles
    if (k0 + BN < hi) dma_block(k0 + BN);
  }

  dt += __shfl_xor(dt, 16, 64);
  dt += __shfl_xor(dt, 32, 64);
  if (rok) {
    T* out = (T*)a.dq + ri * D + 4 * g;
#pragma unroll
    for (int nt = 0; nt < D / 16; ++nt) {
      const f32x4 x = dqT[nt] * a.scale;
      *(u32x2*)(out + 16 * nt) = u32x2{pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3])};
    }
    if (g == 0) a.dt[ri] = dt * a.scale;
  }
}

// dk, dv for 16-bit inputs: workgroup = (b * Hq + hq, 64-key tile); writes hq's slice of
// (B, Hq, Tk, D)
template <typename T, int D>
__global__ void __launch_bounds__(256, 2) polar_bwd16_dkdv_kernel(PolarBwdArgs a) {
  constexpr int BK = 64, BQ = 64, KS = D / 32, CPR = D / 8, NDMA = CPR / 4;
  // double-buffered query blocks, filled by direct-to-LDS copies one block ahead
  __shared__ __attribute__((aligned(16))) T Qs[2][BQ * D];
  __shared__ __attribute__((aligned(16))) T Gs[2][BQ * D];
  __shared__ __attribute__((aligned(16))) float s_c1[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_nm2[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_gl[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_g2[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_nr[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_tp[2][BQ];
  __shared__ float s_lim[2][2];

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.Hq / a.Hkv;
  const int bh = blockIdx.x, b = bh / a.Hq, hq = bh % a.Hq, hk = hq / G;
  const int k0 = blockIdx.y * BK, kr0 = k0 + 16 * wave;
  const T* kp = (const T*)a.k + b * a.k_sb + hk * a.k_sh;
  const T* vp = (const T*)a.v + b * a.v_sb + hk * a.v_sh;
  const T* qp = (const T*)a.q + b * a.q_sb + hq * a.q_sh;
  const T* gp = (const T*)a.gs + b * a.g_sb + hq * a.g_sh;
  // the (b, hq) slices of q and gs as buffers: rows past Tq read as zeros
  const auto qrs = buffer_rsrc(qp, (uint32_t)((int64_t)a.Tq * a.q_st * 2));
  const auto grs = buffer_rsrc(gp, (uint32_t)((int64_t)a.Tq * a.g_st * 2));
  // copy k of wave w fills LDS chunks (NDMA w + k) 64 + lane: row r = chunk / CPR, stored
  // position chunk % CPR, so it loads global chunk position ^ f(r)
  uint32_t qoff[NDMA], goff[NDMA];
#pragma unroll
  for (int k = 0; k < NDMA; ++k) {
    const int q = (NDMA * wave + k) * 64 + lane, r = q / CPR, c = (q % CPR) ^ bw_swz<CPR>(r);
    qoff[k] = (uint32_t)((r * a.q_st + 8 * c) * 2);
    goff[k] = (uint32_t)((r * a.g_st + 8 * c) * 2);
  }
  auto dma_block = [&](int q0, int buf) {
    const uint32_t qb = (uint32_t)((int64_t)q0 * a.q_st * 2), gb = (uint32_t)((int64_t)q0 * a.g_st * 2);
#pragma unroll
    for (int k = 0; k < NDMA; ++k) {
      dma_buf16(qrs, qoff[k] + qb, 0, &Qs[buf][(NDMA * wave + k) * 64 * 8]);
      dma_buf16(grs, goff[k] + gb, 0, &Gs[buf][(NDMA * wave + k) * 64 * 8]);
    }
  };

  // the wave's 16 keys as B operands; the lane's key is kr0 + c16
  u32x4 kf[KS], vf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    kf[s] = bw_global_rows<T>(kp, a.k_st, kr0, a.Tk, 32 * s, lane);
    vf[s] = bw_global_rows<T>(vp, a.v_st, kr0, a.Tk, 32 * s, lane);
  }
  const int key = kr0 + c16;
  const float keyf = (float)key;
  f32x4 dkT[D / 16], dvT[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) dkT[t] = dvT[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lo = a.is_causal ? (k0 / BQ) * BQ : 0;
  const int hi = a.window > 0 ? min(k0 + BK + a.window, a.Tq) : a.Tq;
  // per-query scalars of a block, wave 0 (one query per lane), into buffer buf
  float n_tp = 1.f, n_m = 0.f, n_gl = 0.f, n_gq2 = 0.f, n_nr = 0.f;
  auto row_vals = [&](int q0) {
    const int row = q0 + lane;
    const bool ok = row < a.Tq;
    const int64_t i = (int64_t)bh * a.Tq + row;
    n_tp = ok ? a.temp[(int64_t)hq * a.Tq + row] : 1.f;
    n_m = ok ? a.M[i] : 0.f;
    n_gl = ok ? a.gL[i] : 0.f;
    n_gq2 = ok ? a.gQ2[i] : 0.f;
    n_nr = ok ? a.n_keys[row] : 0.f;  // no valid key for rows past Tq
  };
  auto put_vals = [&](int buf) {
    s_tp[buf][lane] = n_tp;
    s_c1[buf][lane] = a.scale * n_tp * kLog2e;
    s_nm2[buf][lane] = -n_m * kLog2e;
    s_gl[buf][lane] = n_gl;
    s_g2[buf][lane] = 2.f * n_gq2;
    s_nr[buf][lane] = n_nr;
    // min / max of the block's key counts: DPP within rows of 16, then the four rows
    float mn = -row16_max(-n_nr), mx = row16_max(n_nr);
    mn = fminf(fminf(bw_lane(mn, 0), bw_lane(mn, 16)), fminf(bw_lane(mn, 32), bw_lane(mn, 48)));
    mx = fmaxf(fmaxf(bw_lane(mx, 0), bw_lane(mx, 16)), fmaxf(bw_lane(mx, 32), bw_lane(mx, 48)));
    if (lane == 0) {
      s_lim[buf][0] = mn;
      s_lim[buf][1] = mx;
    }
  };
  if (lo < hi) {
    dma_block(lo, 0);
    if (wave == 0) {
      row_vals(lo);
      put_vals(0);
    }
  }
  int cur = 0;
  for (int q0 = lo; q0 < hi; q0 += BQ) {
    wait_vmcnt<0>();  // this wave's copies of block q0 (and every earlier load) are done
    __syncthreads();  // ... and every wave's; buffer cur ^ 1 is no longer read
    const bool more = q0 + BQ < hi;
    if (more) {
      dma_block(q0 + BQ, cur ^ 1);
      if (wave == 0) row_vals(q0 + BQ);
    }
    const T* Qc = Qs[cur];
    const T* Gc = Gs[cur];
    const float nmin = s_lim[cur][0], nmax = s_lim[cur][1];
    const bool full = kr0 + 16 <= a.Tk && (float)(kr0 + 15) < nmin &&
                      (a.window <= 0 || (float)kr0 >= nmax - (float)a.window);
    // two query halves of 32: S and dP of tiles 2 j, 2 j + 1 (each tile's operands read
    // before its products are issued), the elementwise gradient, then P and dS packed as
    // the B operands of half j
    u32x4 pb[2], db[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 sq[2], pq[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = 2 * j + u;
        u32x4 qa[KS], ga[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          qa[s] = bw_rows_swz<D>(Qc, 16 * t, 32 * s, lane);
          ga[s] = bw_rows_swz<D>(Gc, 16 * t, 32 * s, lane);
        }
        sq[u] = pq[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          sq[u] = mfma16x16x32<T>(qa[s], kf[s], sq[u]);
          pq[u] = mfma16x16x32<T>(ga[s], vf[s], pq[u]);
        }
      }
      // S element (query q0 + 16 t + 4 g + i, the lane's key)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int qb = 16 * (2 * j + u) + 4 * g;
        const f32x4 c1 = *(const f32x4*)(s_c1[cur] + qb), nm2 = *(const f32x4*)(s_nm2[cur] + qb);
        const f32x4 gl = *(const f32x4*)(s_gl[cur] + qb), g2 = *(const f32x4*)(s_g2[cur] + qb);
        const f32x4 tp = *(const f32x4*)(s_tp[cur] + qb);
        if (full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sq[u][i], c1[i], nm2[i]));
            pq[u][i] = fmaf(g2[i], p, pq[u][i] + gl[i]) * p * tp[i];
            sq[u][i] = p;
          }
        } else {
          const f32x4 nr = *(const f32x4*)(s_nr[cur] + qb);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool valid = (key < a.Tk) & (keyf < nr[i]) & ((a.window <= 0) | (keyf >= nr[i] - (float)a.window));
            const float p = valid ? __builtin_amdgcn_exp2f(fmaf(sq[u][i], c1[i], nm2[i])) : 0.f;
            pq[u][i] = valid ? fmaf(g2[i], p, pq[u][i] + gl[i]) * p * tp[i] : 0.f;
            sq[u][i] = p;
          }
        }
      }
      pb[j] = bw_pack_b<T>(sq[0], sq[1]);
      db[j] = bw_pack_b<T>(pq[0], pq[1]);
    }
    // dV^T += gs^T P, dK^T += Q^T dS
#pragma unroll
    for (int nt = 0; nt < D / 16; ++nt) {
      u32x4 ga[2], qa[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        ga[j] = bw_tcols_swz<D>(Gc, j, 16 * nt, lane);
        qa[j] = bw_tcols_swz<D>(Qc, j, 16 * nt, lane);
      }
      dvT[nt] = mfma16x16x32<T>(ga[0], pb[0], dvT[nt]);
      dkT[nt] = mfma16x16x32<T>(qa[0], db[0], dkT[nt]);
      dvT[nt] = mfma16x16x32<T>(ga[1], pb[1], dvT[nt]);
      dkT[nt] = mfma16x16x32<T>(qa[1], db[1], dkT[nt]);
    }
    if (more && wave == 0) put_vals(cur ^ 1);
    cur ^= 1;
  }

  if (key < a.Tk) {
    const int64_t base = ((int64_t)bh * a.Tk + key) * D + 4 * g;
#pragma unroll
    for (int nt = 0; nt < D / 16; ++nt) {
      const f32x4 x = dkT[nt] * a.scale, y = dvT[nt];
      if constexpr (std::is_same_v<BwShare<T>, float>) {
        *(f32x4*)((float*)a.dk + base + 16 * nt) = x;
        *(f32x4*)((float*)a.dv + base + 16 * nt) = y;
      } else {
        *(u32x2*)((bf16*)a.dk + base + 16 * nt) = u32x2{pack2<bf16>(x[0], x[1]), pack2<bf16>(x[2], x[3])};
        *(u32x2*)((bf16*)a.dv + base + 16 * nt) = u32x2{pack2<bf16>(y[0], y[1]), pack2<bf16>(y[2], y[3])};
      }
    }
  }
}

template <typename T, int D>
static int launch_bwd(const PolarBwdArgs& a, hipStream_t s) {
  const dim3 gq((unsigned)(a.B * a.Hq), (unsigned)((a.Tq + 63) / 64));
  const dim3 gk((unsigned)(a.B * a.Hq), (unsigned)((a.Tk + 63) / 64));
  // the 16-bit loops address a (b, head) slice of k / v (dq) or q / gs (dk/dv) through a
  // 32-bit buffer range; larger slices take the register-staged loops
  constexpr int64_t kMax = 1ll << 32;
  const bool kv_fits = (int64_t)a.Tk * a.k_st * 2 < kMax && (int64_t)a.Tk * a.v_st * 2 < kMax;
  const bool qg_fits = (int64_t)a.Tq * a.q_st * 2 < kMax && (int64_t)a.Tq * a.g_st * 2 < kMax;
  if constexpr (sizeof(T) == 2) {
    if (kv_fits) polar_bwd16_dq_kernel<T, D><<<gq, dim3(256), 0, s>>>(a);
    else polar_bwd_dq_kernel<T, D><<<gq, dim3(256), 0, s>>>(a);
  } else {
    polar_bwd_dq_kernel<T, D><<<gq, dim3(256), 0, s>>>(a);
  }
  int rc = check_launch("polar_attention_bwd(dq)");
  if (rc) return rc;
  if constexpr (sizeof(T) == 2) {
    if (qg_fits) polar_bwd16_dkdv_kernel<T, D><<<gk, dim3(256), 0, s>>>(a);
    else polar_bwd_dkdv_kernel<T, D><<<gk, dim3(256), 0, s>>>(a);
  } else {
    polar_bwd_dkdv_kernel<T, D><<<gk, dim3(256), 0, s>>>(a);
  }
  return check_launch("polar_attention_bwd(dkdv)");
}

// ---------------------------------------------------------------------------------------
// Per-query preamble and parameter-gradient partial sums (kernel/polar_triton.py:1049-1155).
// Four query rows per wave (one per 16 lanes), 16 per workgroup: the row's direction
// cotangent gs = (gc - (gc.c) c) / max(|s|, eps) with c = s / max(|s|, eps), the
// magnitude path's cotangents of L and Q2 through m_eff = L^3 / (Q2 Z), Z = L + p_null,
// and the null sink's share.  Everything the parameter gradients need except the real
// keys' dL/dtemp (the dq loop's dt) is summed per workgroup into one record
// [v_null (D) | sum g_anull nu log n | sum g_anull temp | sum g_anull temp sqrt(log(n+1)) |
// sum gm (1 - mag^2) log1p(m_eff)], summed over workgroups by the caller (fixed order).
struct PolarPrepArgs {
  const void* gc;  // (B, H, T, D) dtype, or null (zero cotangent)
  const void* gm;  // (B, H, T) dtype, or null
  const float* S;  // (B, H, T, D) the forward's unnormalised direction s
  const float* M;  // (B, H, T) natural-log reference max
  const float* L;
  const float* Q2;
  const float* n_keys;  // (T,)
  const float* v_null;  // (H, D)
  const float *null_base, *null_slope_raw, *len_gain_raw, *mag_beta_raw;  // (H,)
  void* gs;       // (B, H, T, D) dtype
  float* gL;      // (B, H, T)
  float* gQ2;     // (B, H, T)
  float* temp;    // (H, T), written by the b == 0 workgroups
  float* part;    // (B * ceil(T / 16), H, D + 4)
  int B, H, T, window, preserve_length;
  float eps;
};

// The preamble's per-row scalar chain runs on every lane of the row's 16-lane group, so it
// takes the hardware forms: exp2 / log2 (about 1 ulp) and reciprocals, instead of the
// library's correctly rounded sequences, which were most of the kernel's instructions.
__device__ __forceinline__ float pp_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float pp_log(float x) { return __builtin_amdgcn_logf(x) * kLn2; }
__device__ __forceinline__ float pp_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
// log1p(y) for y >= 0: log(u) y / (u - 1) with u = 1 + y rounded, exact to rounding for small y
__device__ __forceinline__ float pp_log1p(float y) {
  const float u = 1.f + y;
  return u == 1.f ? y : pp_log(u) * (y * pp_rcp(u - 1.f));
}
// softplus with torch's threshold (x > 20 -> x), as softplus()
__device__ __forceinline__ float pp_softplus(float x) { return x > 20.f ? x : pp_log1p(pp_exp(x)); }
// tanh(x) for x >= 0
__device__ __forceinline__ float pp_tanh_pos(float x) {
  const float e = pp_exp(-2.f * x);
  return (1.f - e) * pp_rcp(1.f + e);
}

template <typename T, int D>
__global__ void __launch_bounds__(256) polar_bwd_prep_kernel(PolarPrepArgs a) {
  // one query row per group of 16 lanes (E elements per lane): the row sums are DPP
  // reductions within the group, and every lane of the group runs the row's scalar chain
  constexpr int E = D / 16;
  constexpr float kTiny = 1.0e-30f;
  __shared__ float s_vn[4][D];
  __shared__ float s_sc[4][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4, l16 = lane & 15;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int t = blockIdx.x * 16 + wave * 4 + grp;
  const bool ok = t < a.T;
  const int64_t row = (int64_t)bh * a.T + (ok ? t : 0);
  float n = a.n_keys[ok ? t : 0];
  if (a.window > 0 && !a.preserve_length) n = fminf(n, (float)a.window);
  n = fmaxf(n, 1.f);
  const float logn = pp_log(n), root = sqrtf(pp_log(n + 1.f));
  const float temp = 1.f + pp_softplus(a.len_gain_raw[h]) * logn;
  const float nu = a.null_base[h] + pp_softplus(a.null_slope_raw[h]) * root;
  const float p_null = ok ? pp_exp(temp * nu - a.M[row]) : 0.f;
  const float Lr = ok ? a.L[row] : 0.f, Q2r = ok ? a.Q2[row] : 0.f;
  const float gmr = (ok && a.gm) ? to_f32(((const T*)a.gm)[row]) : 0.f;

  float sv[E], gv[E], vnull[E];
  {
    // 16-byte loads (rows of S, gc and v_null are 16-byte aligned)
    const float* sp = a.S + row * D + l16 * E;
    const float* vp = a.v_null + (int64_t)h * D + l16 * E;
#pragma unroll
    for (int e4 = 0; e4 < E; e4 += 4) {
      const f32x4 x = ok ? *(const f32x4*)(sp + e4) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 y = *(const f32x4*)(vp + e4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sv[e4 + e] = x[e];
        vnull[e4 + e] = y[e];
      }
    }
    if constexpr (sizeof(T) == 2) {
      const T* gp = (const T*)a.gc + row * D + l16 * E;
#pragma unroll
      for (int e8 = 0; e8 < E; e8 += 8) {
        u32x4 x = u32x4{0u, 0u, 0u, 0u};
        if (ok && a.gc) {
          if constexpr (E >= 8) x = *(const u32x4*)(gp + e8);
          else { const u32x2 y = *(const u32x2*)gp; x = u32x4{y[0], y[1], 0u, 0u}; }
        }
#pragma unroll
        for (int e = 0; e < (E < 8 ? E : 8); ++e) gv[e8 + e] = elem16<T>(x, e);
      }
    } else {
#pragma unroll
      for (int e4 = 0; e4 < E; e4 += 4) {
        const f32x4 x = (ok && a.gc) ? *(const f32x4*)((const float*)a.gc + row * D + l16 * E + e4)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e4 + e] = x[e];
      }
    }
  }
  float ss = 0.f, gcs = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    ss = fmaf(sv[e], sv[e], ss);
    gcs = fmaf(gv[e], sv[e], gcs);
  }
  ss = row16_sum(ss);
  gcs = row16_sum(gcs);
  // gs = (gc - (gc.c) c) / |s|  with c = s / |s|:  (gc - (gc.s / |s|) s / |s|) / |s|
  const float inv = pp_rcp(fmaxf(sqrtf(ss), a.eps));
  const float gcc = gcs * inv;
  float g[E], gsv = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    g[e] = (gv[e] - gcc * (sv[e] * inv)) * inv;
    gsv = fmaf(g[e], vnull[e], gsv);
  }
  if (ok) {
    T* out = (T*)a.gs + row * D + l16 * E;
    if constexpr (sizeof(T) == 2 && E == 8) {
      *(u32x4*)out = u32x4{pack2<T>(g[0], g[1]), pack2<T>(g[2], g[3]), pack2<T>(g[4], g[5]), pack2<T>(g[6], g[7])};
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) out[e] = from_f32<T>(g[e]);
    }
  }
  gsv = row16_sum(gsv);
  // the magnitude path through m_eff = L^3 / (Q2 Z), Z = L + p_null
  const float beta = pp_softplus(a.mag_beta_raw[h]);
  const float Z = Lr + p_null;
  const float Zc = fmaxf(Z, kTiny), Q2c = fmaxf(Q2r, kTiny);
  const float rQ2 = pp_rcp(Q2c), rZ = pp_rcp(Zc);
  const float me = (Lr * Lr * rQ2) * (Lr * rZ);
  const float lm = pp_log1p(me);
  const float mag = pp_tanh_pos(beta * lm);
  const float gme = gmr * beta * (1.f - mag * mag) * pp_rcp(1.f + me);
  const float dme_dL = Lr > 0.f ? 3.f * me * pp_rcp(Lr) : 0.f;
  const float dme_dQ2 = Q2r > kTiny ? -me * rQ2 : 0.f;
  const float dme_dZ = Z > kTiny ? -me * rZ : 0.f;
  const float g_anull = (gsv + gme * dme_dZ) * p_null;
  if (ok && l16 == 0) {
    a.gL[row] = gme * (dme_dL + dme_dZ);
    a.gQ2[row] = gme * dme_dQ2;
    if (b == 0) a.temp[(int64_t)h * a.T + t] = temp;
  }
  // the workgroup's record: sums over its 16 rows (the wave's 4 groups, then the waves)
  float sc[4] = {ok ? g_anull * nu * logn : 0.f, ok ? g_anull * temp : 0.f, ok ? g_anull * temp * root : 0.f,
                 ok ? gmr * (1.f - mag * mag) * lm : 0.f};
  float vn[E];
#pragma unroll
  for (int e = 0; e < E; ++e) vn[e] = p_null * g[e];
#pragma unroll
  for (int m = 16; m < 64; m <<= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) vn[e] += __shfl_xor(vn[e], m, 64);
#pragma unroll
    for (int k = 0; k < 4; ++k) sc[k] += __shfl_xor(sc[k], m, 64);
  }
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) s_vn[wave][l16 * E + e] = vn[e];
    if (l16 == 0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) s_sc[wave][k] = sc[k];
    }
  }
  __syncthreads();
  float* rec = a.part + ((int64_t)(b * gridDim.x + blockIdx.x) * a.H + h) * (D + 4);
  if (tid < D) rec[tid] = s_vn[0][tid] + s_vn[1][tid] + s_vn[2][tid] + s_vn[3][tid];
  else if (tid < D + 4) {
    const int k = tid - D;
    rec[D + k] = s_sc[0][k] + s_sc[1][k] + s_sc[2][k] + s_sc[3][k];
  }
}

// Sum of the G consecutive query heads' shares of dk / dv (or, with G = 1, a copy) into
// the output dtype: out[b, hk, r] = sum_g part[b, hk G + g, r], r over Tk * D elements,
// four per thread, accumulated in fp32 (shares fp32 or bf16).
template <typename TI, typename T>
__global__ void __launch_bounds__(256) polar_bwd_group_sum_kernel(const TI* __restrict__ part, T* __restrict__ out,
                                                                   int64_t rows4, int G) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 4-element index within (b, hk)
  if (i >= rows4) return;
  const int64_t bhk = blockIdx.y;
  auto load4 = [&](int64_t j) -> f32x4 {
    if constexpr (sizeof(TI) == 4) {
      return ((const f32x4*)part)[j];
    } else {
      const u32x2 x = ((const u32x2*)part)[j];
      const u32x4 y = {x[0], x[1], 0u, 0u};
      return f32x4{elem16<TI>(y, 0), elem16<TI>(y, 1), elem16<TI>(y, 2), elem16<TI>(y, 3)};
    }
  };
  const int64_t j0 = bhk * G * rows4 + i;
  f32x4 acc = load4(j0);
  for (int g = 1; g < G; ++g) {
    const f32x4 x = load4(j0 + (int64_t)g * rows4);
    acc = f32x4{acc[0] + x[0], acc[1] + x[1], acc[2] + x[2], acc[3] + x[3]};
  }
  T* o = out + (bhk * rows4 + i) * 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(acc[e]);
}

// Parameter gradients from the preamble's per-block partial sums and the dq loop's dt
// (kernel/polar_triton.py:1139-1150): with temp = 1 + softplus(lg) log n,
// nu = nb + softplus(ns) sqrt(log(n + 1)), mag = tanh(softplus(mb) log1p(m_eff)) and
// d softplus = sigmoid:  g_v_null = sum_blocks part[:, :D];
// g_len_gain = (sum_{b,t} dt log n + sum part[:, D]) sigmoid(lg); g_null_base = sum part[:, D+1];
// g_null_slope = sum part[:, D+2] sigmoid(ns); g_mag_beta = sum part[:, D+3] sigmoid(mb).
// Two launches, every sum in a fixed order (deterministic): kParamSplit workgroups per
// head each sum a slice of the blocks and of the (b, t) pairs into a workspace row, then
// one workgroup per head adds the rows and applies the chain rule.
constexpr int kParamSplit = 32;

__global__ void __launch_bounds__(256) polar_bwd_params_partial_kernel(const float* __restrict__ part,
                                                                        const float* __restrict__ dt,
                                                                        const float* __restrict__ n_keys,
                                                                        float* __restrict__ ws, int nblk, int B,
                                                                        int H, int T, int D, int window,
                                                                        int preserve_length) {
  __shared__ float red[256];
  const int h = blockIdx.x, sp = blockIdx.y, tid = threadIdx.x, W = D + 4;
  const int r0 = (int)((int64_t)nblk * sp / kParamSplit), r1 = (int)((int64_t)nblk * (sp + 1) / kParamSplit);
  float* out = ws + ((int64_t)sp * H + h) * (W + 1);
  if (tid < W) {
    float col = 0.f;
#pragma unroll 8
    for (int r = r0; r < r1; ++r) col += part[((int64_t)r * H + h) * W + tid];
    out[tid] = col;
  }
  const int64_t n = (int64_t)B * T, i0 = n * sp / kParamSplit, i1 = n * (sp + 1) / kParamSplit;
  float acc = 0.f;
  for (int64_t i = i0 + tid; i < i1; i += 256) {
    const int b = (int)(i / T), t = (int)(i % T);
    float nk = n_keys[t];
    if (window > 0 && !preserve_length) nk = fminf(nk, (float)window);
    acc += dt[((int64_t)b * H + h) * T + t] * logf(fmaxf(nk, 1.f));
  }
  red[tid] = acc;
  __syncthreads();
  for (int m = 128; m > 0; m >>= 1) {
    if (tid < m) red[tid] += red[tid + m];
    __syncthreads();
  }
  if (tid == 0) out[W] = red[0];
}

__global__ void __launch_bounds__(256) polar_bwd_params_final_kernel(const float* __restrict__ ws,
                                                                      const float* __restrict__ len_gain_raw,
                                                                      const float* __restrict__ null_slope_raw,
                                                                      const float* __restrict__ mag_beta_raw,
                                                                      float* __restrict__ g_v_null,
                                                                      float* __restrict__ g4, int H, int D) {
  __shared__ float dt_logn;
  const int h = blockIdx.x, tid = threadIdx.x, W = D + 4;
  float col = 0.f;
  if (tid <= W)
    for (int sp = 0; sp < kParamSplit; ++sp) col += ws[((int64_t)sp * H + h) * (W + 1) + tid];
  if (tid == W) dt_logn = col;
  __syncthreads();
  auto sig = [](float x) { return 1.f / (1.f + expf(-x)); };
  // g4 rows: null_base, null_slope_raw, len_gain_raw, mag_beta_raw
  if (tid < D) g_v_null[(int64_t)h * D + tid] = col;
  else if (tid == D) g4[2 * H + h] = (dt_logn + col) * sig(len_gain_raw[h]);
  else if (tid == D + 1) g4[0 * H + h] = col;
  else if (tid == D + 2) g4[1 * H + h] = col * sig(null_slope_raw[h]);
  else if (tid == D + 3) g4[3 * H + h] = col * sig(mag_beta_raw[h]);
}

template <typename T, int D>
static int launch_prep(const PolarPrepArgs& a, hipStream_t s) {
  polar_bwd_prep_kernel<T, D><<<dim3((unsigned)((a.T + 15) / 16), (unsigned)(a.B * a.H)), dim3(256), 0, s>>>(a);
  return check_launch("polar_attention_bwd_prep");
}

}  // namespace atma

extern "C" int atma_polar_attention_bwd(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb, int64_t k_sh,
    int64_t k_st, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, const void* gs,
    int64_t g_sb, int64_t g_sh, int64_t g_st, const float* gL, const float* gQ2, const float* M,
    const float* temp, const float* n_keys, void* dq, float* dt, void* dk, void* dv, int64_t B,
    int64_t Hq, int64_t Hkv, int64_t Tq, int64_t Tk, int64_t d, int dtype, int is_causal,
    int64_t window, void* stream) {
  using namespace atma;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Tq < 0 || Tk < 0)
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: bad sizes");
  if (Hq % Hkv) return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: Hq %% Hkv != 0");
  if (is_causal && Tq != Tk)
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: is_causal=True requires Tq == Tk");
  if (d != 64 && d != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_bwd: head_dim %lld (supported: 64, 128)",
                     (long long)d);
  if (Tq > 64 * 65535 || Tk > 64 * 65535 || B * Hq > 0x7fffffffll)
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: sizes too large");
  if (B == 0 || Tq == 0) return ATMA_OK;
  const int es = dtype_size(dtype);
  if (!es) return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: unknown dtype %d", dtype);
  if (!q || !k || !v || !gs || !gL || !gQ2 || !M || !temp || !n_keys || !dq || !dt || !dk || !dv)
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: null pointer");
  auto al16 = [&](const void* p, int64_t s1, int64_t s2, int64_t s3) {
    return ((uintptr_t)p % 16 == 0) && ((s1 * es) % 16 == 0) && ((s2 * es) % 16 == 0) &&
           ((s3 * es) % 16 == 0);
  };
  if (!al16(q, q_sb, q_sh, q_st) || !al16(k, k_sb, k_sh, k_st) || !al16(v, v_sb, v_sh, v_st) ||
      !al16(gs, g_sb, g_sh, g_st))
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd: tensors must be 16-byte aligned rows");
  if (Tk == 0) {
    // no keys: every gradient of the O(T^2) part is zero (the callers' buffers are zeroed)
    return ATMA_OK;
  }
  PolarBwdArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.gs = gs; a.g_sb = g_sb; a.g_sh = g_sh; a.g_st = g_st;
  a.gL = gL; a.gQ2 = gQ2; a.M = M; a.temp = temp; a.n_keys = n_keys;
  a.dq = dq; a.dt = dt; a.dk = dk; a.dv = dv;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.Tq = (int)Tq; a.Tk = (int)Tk;
  a.is_causal = is_causal ? 1 : 0;
  a.window = window > 0 ? (int)window : 0;
  a.scale = 1.f / sqrtf((float)d);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_BF16: return d == 128 ? launch_bwd<bf16, 128>(a, s) : launch_bwd<bf16, 64>(a, s);
    case ATMA_F16: return d == 128 ? launch_bwd<f16, 128>(a, s) : launch_bwd<f16, 64>(a, s);
    default: return d == 128 ? launch_bwd<float, 128>(a, s) : launch_bwd<float, 64>(a, s);
  }
}

extern "C" int atma_polar_attention_bwd_prep(
    const void* gc, const void* gm, const float* S, const float* M, const float* L, const float* Q2,
    const float* n_keys, const float* v_null, const float* null_base, const float* null_slope_raw,
    const float* len_gain_raw, const float* mag_beta_raw, void* gs, float* gL, float* gQ2, float* temp,
    float* part, int64_t B, int64_t H, int64_t T, int64_t d, int dtype, int64_t window,
    int preserve_length, float eps, void* stream) {
  using namespace atma;
  if (B < 0 || H <= 0 || T < 0) return set_error(ATMA_ERR_INVALID, "polar_attention_bwd_prep: bad sizes");
  if (d != 64 && d != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_bwd_prep: head_dim %lld (supported: 64, 128)",
                     (long long)d);
  if (B * H > 65535 || T > (1ll << 30))
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd_prep: sizes too large");
  if (B == 0 || T == 0) return ATMA_OK;
  if (!dtype_size(dtype)) return set_error(ATMA_ERR_INVALID, "polar_attention_bwd_prep: unknown dtype %d", dtype);
  if (!S || !M || !L || !Q2 || !n_keys || !v_null || !null_base || !null_slope_raw || !len_gain_raw ||
      !mag_beta_raw || !gs || !gL || !gQ2 || !temp || !part)
    return set_error(ATMA_ERR_INVALID, "polar_attention_bwd_prep: null pointer");
  PolarPrepArgs a{};
  a.gc = gc; a.gm = gm; a.S = S; a.M = M; a.L = L; a.Q2 = Q2; a.n_keys = n_keys; a.v_null = v_null;
  a.null_base = null_base; a.null_slope_raw = null_slope_raw; a.len_gain_raw = len_gain_raw;
  a.mag_beta_raw = mag_beta_raw; a.gs = gs; a.gL = gL; a.gQ2 = gQ2; a.temp = temp; a.part = part;
  a.B = (int)B; a.H = (int)H; a.T = (int)T;
  a.window = window > 0 ? (int)window : 0; a.preserve_length = preserve_length ? 1 : 0; a.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_BF16: return d == 128 ? launch_prep<bf16, 128>(a, s) : launch_prep<bf16, 64>(a, s);
    case ATMA_F16: return d == 128 ? launch_prep<f16, 128>(a, s) : launch_prep<f16, 64>(a, s);
    default: return d == 128 ? launch_prep<float, 128>(a, s) : launch_prep<float, 64>(a, s);
  }
}

extern "C" int atma_polar_bwd_group_sum(const void* part, int part_dtype, void* out, int64_t n_groups, int64_t G,
                                        int64_t elems, int dtype, void* stream) {
  using namespace atma;
  if (n_groups < 0 || G <= 0 || elems < 0 || elems % 4)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: bad sizes (elems %% 4 == 0)");
  if (n_groups == 0 || elems == 0) return ATMA_OK;
  if (n_groups > 65535 || elems / 4 > 0x7fffffffll * 256)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: sizes too large");
  if (part_dtype != ATMA_F32 && part_dtype != ATMA_BF16)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: shares are fp32 or bf16");
  if (!part || !out || (uintptr_t)part % 16)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: null or misaligned pointer");
  const int64_t rows4 = elems / 4;
  const dim3 grid((unsigned)((rows4 + 255) / 256), (unsigned)n_groups);
  hipStream_t s = (hipStream_t)stream;
  auto run = [&](auto ti) -> int {
    using TI = decltype(ti);
    const TI* p = (const TI*)part;
    switch (dtype) {
      case ATMA_BF16: polar_bwd_group_sum_kernel<TI, bf16><<<grid, dim3(256), 0, s>>>(p, (bf16*)out, rows4, (int)G); break;
      case ATMA_F16: polar_bwd_group_sum_kernel<TI, f16><<<grid, dim3(256), 0, s>>>(p, (f16*)out, rows4, (int)G); break;
      case ATMA_F32: polar_bwd_group_sum_kernel<TI, float><<<grid, dim3(256), 0, s>>>(p, (float*)out, rows4, (int)G); break;
      default: return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: unknown dtype %d", dtype);
    }
    return check_launch("polar_bwd_group_sum");
  };
  return part_dtype == ATMA_F32 ? run(float{}) : run(bf16{});
}

extern "C" size_t atma_polar_bwd_param_grads_workspace_bytes(int64_t H, int64_t d) {
  return (size_t)atma::kParamSplit * (size_t)(H > 0 ? H : 0) * (size_t)(d + 5) * sizeof(float);
}

extern "C" int atma_polar_bwd_param_grads(const float* part, const float* dt, const float* n_keys,
                                          const float* len_gain_raw, const float* null_slope_raw,
                                          const float* mag_beta_raw, float* g_v_null, float* g_params,
                                          int64_t B, int64_t H, int64_t T, int64_t d, int64_t window,
                                          int preserve_length, void* workspace, size_t workspace_bytes,
                                          void* stream) {
  using namespace atma;
  if (B < 0 || H <= 0 || T < 0 || (d != 64 && d != 128))
    return set_error(ATMA_ERR_INVALID, "polar_bwd_param_grads: bad sizes (d = 64 or 128)");
  if (H > 65535 || B * T > (1ll << 40)) return set_error(ATMA_ERR_INVALID, "polar_bwd_param_grads: sizes too large");
  if (!part || !dt || !n_keys || !len_gain_raw || !null_slope_raw || !mag_beta_raw || !g_v_null || !g_params)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_param_grads: null pointer");
  if (!workspace || workspace_bytes < atma_polar_bwd_param_grads_workspace_bytes(H, d))
    return set_error(ATMA_ERR_WORKSPACE, "polar_bwd_param_grads: workspace too small");
  const int64_t nblk = B * ((T + 15) / 16);
  hipStream_t s = (hipStream_t)stream;
  float* ws = (float*)workspace;
  polar_bwd_params_partial_kernel<<<dim3((unsigned)H, kParamSplit), dim3(256), 0, s>>>(
      part, dt, n_keys, ws, (int)nblk, (int)B, (int)H, (int)T, (int)d, window > 0 ? (int)window : 0,
      preserve_length ? 1 : 0);
  int rc = check_launch("polar_bwd_param_grads(partial)");
  if (rc) return rc;
  polar_bwd_params_final_kernel<<<dim3((unsigned)H), dim3(256), 0, s>>>(ws, len_gain_raw, null_slope_raw,
                                                                          mag_beta_raw, g_v_null, g_params,
                                                                          (int)H, (int)d);
  return check_launch("polar_bwd_param_grads(final)");
}
