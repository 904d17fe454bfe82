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
  float* dq;            // (B, Hq, Tq, D)
  float* dt;            // (B, Hq, Tq)
  float* dk;            // (B, Hq, Tk, D): each query head's share; grouped heads summed by the caller
  float* dv;            // (B, Hq, Tk, D)
  int B, Hq, Hkv, Tq, Tk;
  int is_causal, window;
  float scale;
};

template <typename T>
using BwFrag = std::conditional_t<sizeof(T) == 2, u32x4, float>;
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
      float* out = a.dq + ((int64_t)bh * a.Tq + row) * D + (lane & 15);
#pragma unroll
      for (int nt = 0; nt < D / 16; ++nt) out[16 * nt] = dq[nt][j] * a.scale;
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
        a.dk[base + 16 * nt] = dk[nt][j] * a.scale;
        a.dv[base + 16 * nt] = dv[nt][j];
      }
    }
  }
}

template <typename T, int D>
static int launch_bwd(const PolarBwdArgs& a, hipStream_t s) {
  polar_bwd_dq_kernel<T, D><<<dim3((unsigned)(a.B * a.Hq), (unsigned)((a.Tq + 63) / 64)), dim3(256), 0, s>>>(a);
  int rc = check_launch("polar_attention_bwd(dq)");
  if (rc) return rc;
  polar_bwd_dkdv_kernel<T, D><<<dim3((unsigned)(a.B * a.Hq), (unsigned)((a.Tk + 63) / 64)), dim3(256), 0, s>>>(a);
  return check_launch("polar_attention_bwd(dkdv)");
}

// ---------------------------------------------------------------------------------------
// Per-query preamble and parameter-gradient partial sums (kernel/polar_triton.py:1049-1155).
// One wave per query row (4 rows per wave, 16 per workgroup): the row's direction
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

template <typename T, int D>
__global__ void __launch_bounds__(256) polar_bwd_prep_kernel(PolarPrepArgs a) {
  constexpr int E = D / 64;  // elements per lane
  constexpr int R = 4;       // rows per wave, processed together (independent chains)
  constexpr float kTiny = 1.0e-30f;
  __shared__ float s_vn[4][D];
  __shared__ float s_sc[4][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int t0 = blockIdx.x * 16 + wave * R;
  // The per-row scalar chain (log, exp, log1p, tanh, divisions) runs once per row: lane
  // i < R computes row t0 + i, and the results are read back with shuffles.
  const int my = lane & (R - 1);
  const bool my_ok = t0 + my < a.T;
  const int64_t my_row = (int64_t)bh * a.T + (my_ok ? t0 + my : 0);
  float n = a.n_keys[my_ok ? t0 + my : 0];
  if (a.window > 0 && !a.preserve_length) n = fminf(n, (float)a.window);
  n = fmaxf(n, 1.f);
  const float logn = logf(n), root = sqrtf(logf(n + 1.f));
  const float temp = 1.f + softplus(a.len_gain_raw[h]) * logn;
  const float nu = a.null_base[h] + softplus(a.null_slope_raw[h]) * root;
  const float p_null = my_ok ? expf(temp * nu - a.M[my_row]) : 0.f;
  const float Lr = my_ok ? a.L[my_row] : 0.f, Q2r = my_ok ? a.Q2[my_row] : 0.f;
  const float gmr = (my_ok && a.gm) ? to_f32(((const T*)a.gm)[my_row]) : 0.f;

  bool ok[R];
  int64_t row[R];
  float sv[R][E], gv[R][E], vnull[E];
#pragma unroll
  for (int e = 0; e < E; ++e) vnull[e] = a.v_null[(int64_t)h * D + 64 * e + lane];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    ok[i] = t0 + i < a.T;
    row[i] = (int64_t)bh * a.T + (ok[i] ? t0 + i : 0);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      sv[i][e] = ok[i] ? a.S[row[i] * D + 64 * e + lane] : 0.f;
      gv[i][e] = (ok[i] && a.gc) ? to_f32(((const T*)a.gc)[row[i] * D + 64 * e + lane]) : 0.f;
    }
  }
  float ss[R], gcs[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    ss[i] = 0.f;
    gcs[i] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ss[i] = fmaf(sv[i][e], sv[i][e], ss[i]);
      gcs[i] = fmaf(gv[i][e], sv[i][e], gcs[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    ss[i] = wave_sum(ss[i]);
    gcs[i] = wave_sum(gcs[i]);
  }
  float vn[E];
#pragma unroll
  for (int e = 0; e < E; ++e) vn[e] = 0.f;
  float gsv[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const float pn = __shfl(p_null, i, 64);
    // gs = (gc - (gc.c) c) / |s|  with c = s / |s|:  (gc - (gc.s / |s|) s / |s|) / |s|
    const float inv = 1.f / fmaxf(sqrtf(ss[i]), a.eps);
    const float gcc = gcs[i] * inv;
    gsv[i] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float g = (gv[i][e] - gcc * (sv[i][e] * inv)) * inv;
      if (ok[i]) ((T*)a.gs)[row[i] * D + 64 * e + lane] = from_f32<T>(g);
      gsv[i] = fmaf(g, vnull[e], gsv[i]);
      vn[e] = fmaf(pn, g, vn[e]);
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) gsv[i] = wave_sum(gsv[i]);
  // lane my: the rest of row t0 + my's chain
  float my_gsv = gsv[0];
#pragma unroll
  for (int i = 1; i < R; ++i) my_gsv = my == i ? gsv[i] : my_gsv;
  const float beta = softplus(a.mag_beta_raw[h]);
  const float Z = Lr + p_null;
  const float Zc = fmaxf(Z, kTiny), Q2c = fmaxf(Q2r, kTiny);
  const float me = (Lr * Lr / Q2c) * (Lr / Zc);
  const float lm = log1pf(me);
  const float mag = tanhf(beta * lm);
  const float gme = gmr * beta * (1.f - mag * mag) / (1.f + me);
  const float dme_dL = Lr > 0.f ? 3.f * me / Lr : 0.f;
  const float dme_dQ2 = Q2r > kTiny ? -me / Q2c : 0.f;
  const float dme_dZ = Z > kTiny ? -me / Zc : 0.f;
  const float g_anull = (my_gsv + gme * dme_dZ) * p_null;
  const bool lead = lane < R && my_ok;
  if (lead) {
    a.gL[my_row] = gme * (dme_dL + dme_dZ);
    a.gQ2[my_row] = gme * dme_dQ2;
    if (b == 0) a.temp[(int64_t)h * a.T + t0 + my] = temp;
  }
  float t1 = lead ? g_anull * nu * logn : 0.f;
  float t2 = lead ? g_anull * temp : 0.f;
  float t3 = lead ? g_anull * temp * root : 0.f;
  float t4 = lead ? gmr * (1.f - mag * mag) * lm : 0.f;
#pragma unroll
  for (int m = 1; m < R; m <<= 1) {  // sum over the R leading lanes
    t1 += __shfl_xor(t1, m, 64);
    t2 += __shfl_xor(t2, m, 64);
    t3 += __shfl_xor(t3, m, 64);
    t4 += __shfl_xor(t4, m, 64);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) s_vn[wave][64 * e + lane] = vn[e];
  if (lane == 0) {
    s_sc[wave][0] = t1;
    s_sc[wave][1] = t2;
    s_sc[wave][2] = t3;
    s_sc[wave][3] = t4;
  }
  __syncthreads();
  float* rec = a.part + ((int64_t)(b * gridDim.x + blockIdx.x) * a.H + h) * (D + 4);
  if (tid < D) rec[tid] = s_vn[0][tid] + s_vn[1][tid] + s_vn[2][tid] + s_vn[3][tid];
  else if (tid < D + 4) {
    const int j = tid - D;
    rec[D + j] = s_sc[0][j] + s_sc[1][j] + s_sc[2][j] + s_sc[3][j];
  }
}

// Sum of the G consecutive query heads' shares of dk / dv (or, with G = 1, a copy) into
// the output dtype: out[b, hk, r] = sum_g part[b, hk G + g, r], r over Tk * D elements,
// four per thread.
template <typename T>
__global__ void __launch_bounds__(256) polar_bwd_group_sum_kernel(const float* __restrict__ part, T* __restrict__ out,
                                                                   int64_t rows4, int G) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index within (b, hk)
  if (i >= rows4) return;
  const int64_t bhk = blockIdx.y;
  const f32x4* src = (const f32x4*)part + bhk * G * rows4 + i;
  f32x4 acc = src[0];
  for (int g = 1; g < G; ++g) {
    const f32x4 x = src[(int64_t)g * rows4];
    acc = f32x4{acc[0] + x[0], acc[1] + x[1], acc[2] + x[2], acc[3] + x[3]};
  }
  T* o = out + (bhk * rows4 + i) * 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(acc[e]);
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
    const float* temp, const float* n_keys, float* dq, float* dt, float* dk, float* dv, int64_t B,
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

extern "C" int atma_polar_bwd_group_sum(const float* part, void* out, int64_t n_groups, int64_t G,
                                        int64_t elems, int dtype, void* stream) {
  using namespace atma;
  if (n_groups < 0 || G <= 0 || elems < 0 || elems % 4)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: bad sizes (elems %% 4 == 0)");
  if (n_groups == 0 || elems == 0) return ATMA_OK;
  if (n_groups > 65535 || elems / 4 > 0x7fffffffll * 256)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: sizes too large");
  if (!part || !out || (uintptr_t)part % 16)
    return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: null or misaligned pointer");
  const int64_t rows4 = elems / 4;
  const dim3 grid((unsigned)((rows4 + 255) / 256), (unsigned)n_groups);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_BF16: polar_bwd_group_sum_kernel<bf16><<<grid, dim3(256), 0, s>>>(part, (bf16*)out, rows4, (int)G); break;
    case ATMA_F16: polar_bwd_group_sum_kernel<f16><<<grid, dim3(256), 0, s>>>(part, (f16*)out, rows4, (int)G); break;
    case ATMA_F32: polar_bwd_group_sum_kernel<float><<<grid, dim3(256), 0, s>>>(part, (float*)out, rows4, (int)G); break;
    default: return set_error(ATMA_ERR_INVALID, "polar_bwd_group_sum: unknown dtype %d", dtype);
  }
  return check_launch("polar_bwd_group_sum");
}
