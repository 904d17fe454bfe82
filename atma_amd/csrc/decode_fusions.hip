// Fusions of the served model's decode step (one token per sequence), each one launch
// where the eager model makes several, with the eager model's roundings:
//
//  * residual_rms_norm: branch + residual stream -> new stream, RMSNorm(stream) * w.  The
//    pre-norm block (inference/models/atma.py:680-713: x + attn(norm1 x), x + mlp(norm2 x))
//    adds every branch to the stream and normalises the sum for the next branch, so the add
//    and the norm read and write the row once together.  The branch is a 16-bit tensor or
//    fp32 partial sums (linear_tokens' chunks form) plus biases and a low-rank term (the
//    global layer's mu_proj(mag), 4, 8 or 16 inputs), added in fp32 and rounded once.
//  * lfm2_conv_step: the LFM2 block's gated conv for one token, c * conv(b * x)
//    (model/reference.py:31-48, inference/models/atma.py:625-673) from the rows of its
//    in_proj output, state table advanced in place.
//  * global_decode_prep: the global layer's per-head RMSNorm of q and k, Canon residual
//    convs of q / k / v (inference/models/atma.py:546-575) and the memory gates
//    (model/blocks.py:426-490) from one row of its fused input projection.
//  (the gated inputs of the global layer's output projections, global_decode_gate, are
//  layer_fusions.hip's global_gate at one token per sequence)
//
// All are latency-bound at decode sizes (a few KB per row); a row is one wave (64 lanes,
// 8 contiguous 16-bit values per lane per pass), reductions stay inside the wave.
#include "common.h"
#include "gated_delta.h"

namespace atma {

template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v) {
  u32x4 u;
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = pack2<T>(v[2 * e], v[2 * e + 1]);
  *(u32x4*)p = u;
}
template <typename T>
__device__ __forceinline__ float rnd(float x) { return to_f32(from_f32<T>(x)); }

// ------------------------------------------------------------------ residual_rms_norm
constexpr int kResMaxBias = 3;

struct ResNormArgs {
  const void* y;  // branch (M, D) in T, row stride ldy; or null: the branch is `parts`
  int64_t ldy;
  const float* parts;  // (n_parts, M, D) fp32
  int n_parts;
  const void* bias[kResMaxBias];  // (D,) T, added to the parts' sum
  int n_bias;
  const void* mu_x;  // (M, mu_k) T: the low-rank term sum_h mu_x[m, h] mu_w[n, h]
  int64_t ldmu;
  const void* mu_w;  // (D, mu_k) T, contiguous
  int mu_k;
  const void* res;  // residual stream in (M, D) T, or null (the branch starts the stream)
  int64_t ldr;
  void* res_out;  // new stream (may be null when res is null)
  int64_t ldro;
  const void* w;  // (D,) T RMSNorm gain
  void* out;      // (M, D) T
  int64_t ldo;
  float eps;
  int M, D;
};

constexpr int kResMaxParts = 8;

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& u, float* v) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = elem16<T>(u, e);
}
__device__ __forceinline__ f32x4 ld4(const float* p) { return *(const f32x4*)p; }

// One wave per RPW consecutive rows, P passes of 512 columns (8 per lane).  The gain and the
// low-rank weights of a lane's columns are loaded once for the wave's rows (at RPW = 1 and
// MU = 8 every row re-read its lanes' share of mu_w: the whole 16 KB weight per row, twice
// the row's own HBM bytes).  A pass issues every load it needs (branch or partial sums,
// biases, residual) before its first arithmetic, so a row costs one memory round trip per
// pass.  MU: the low-rank term's width (0: none), a template so that its weights index
// registers statically.
template <typename T, int P, int MU, int RPW, bool PARTS>
__global__ void __launch_bounds__(256) residual_rms_norm_kernel(ResNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int m0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (m0 >= a.M) return;
  u32x4 wv[P];
  u32x4 mwv[P][MU > 0 ? MU : 1];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = (p * 64 + lane) * 8;
    const int cc = c < a.D ? c : 0;  // lanes past the row read column 0 and drop it
    wv[p] = *(const u32x4*)((const T*)a.w + cc);
    if constexpr (MU > 0) {
      // rows cc .. cc + 7 of mu_w (D, MU): 8 MU contiguous values, MU 16-byte vectors
#pragma unroll
      for (int i = 0; i < MU; ++i) mwv[p][i] = *(const u32x4*)((const T*)a.mu_w + (int64_t)cc * MU + 8 * i);
    }
  }
  for (int k = 0; k < RPW; ++k) {
    const int m = m0 + k;
    if (m >= a.M) break;
    // the low-rank term's inputs of this row as packed 16-bit pairs (v_dot2 operands)
    uint32_t mu2[MU > 0 ? MU / 2 : 1];
    if constexpr (MU > 0) {
      const uint32_t* mx = (const uint32_t*)((const T*)a.mu_x + (int64_t)m * a.ldmu);
#pragma unroll
      for (int i = 0; i < MU / 2; ++i) mu2[i] = mx[i];
    }
    float s[P][8];
    float sq = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = (p * 64 + lane) * 8;
      const bool in = c < a.D;
      const int cc = in ? c : 0;  // lanes past the row read column 0 and drop it
      u32x4 rv = {0u, 0u, 0u, 0u};
      if (a.res) rv = *(const u32x4*)((const T*)a.res + (int64_t)m * a.ldr + cc);
      float br[8];
      // the branch: a 16-bit tensor or the fp32 partial sums, plus the biases and the
      // low-rank term (fp32), rounded once whenever anything was added in fp32
      // (PARTS: the branch is the partial sums; a template, so that the 16-bit form holds no
      // registers for them)
      u32x4 yv = {0u, 0u, 0u, 0u};
      if constexpr (!PARTS) yv = *(const u32x4*)((const T*)a.y + (int64_t)m * a.ldy + cc);
      f32x4 pv[PARTS ? kResMaxParts : 1][2];
      if constexpr (PARTS) {
#pragma unroll
        for (int q = 0; q < kResMaxParts; ++q)
          if (q < a.n_parts) {
            const float* pp = a.parts + ((int64_t)q * a.M + m) * a.D + cc;
            pv[q][0] = ld4(pp);
            pv[q][1] = ld4(pp + 4);
          }
      }
      u32x4 bv[kResMaxBias];
#pragma unroll
      for (int b = 0; b < kResMaxBias; ++b)
        if (b < a.n_bias) bv[b] = *(const u32x4*)((const T*)a.bias[b] + cc);
      if constexpr (!PARTS) {
        unpack8<T>(yv, br);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) br[e] = pv[0][e >> 2][e & 3];
#pragma unroll
        for (int q = 1; q < kResMaxParts; ++q)
          if (q < a.n_parts) {
#pragma unroll
            for (int e = 0; e < 8; ++e) br[e] += pv[q][e >> 2][e & 3];
          }
      }
#pragma unroll
      for (int b = 0; b < kResMaxBias; ++b)
        if (b < a.n_bias) {
#pragma unroll
          for (int e = 0; e < 8; ++e) br[e] += elem16<T>(bv[b], e);
        }
      if constexpr (MU > 0) {
        // element e's MU weights are words e MU / 2 .. e MU / 2 + MU / 2 - 1 of the block
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < MU / 2; ++i) {
            const int wd = e * (MU / 2) + i;
            acc = dot2<T>(mwv[p][wd >> 2][wd & 3], mu2[i], acc);
          }
          br[e] += acc;
        }
      }
      if (PARTS || a.n_bias > 0 || MU > 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) br[e] = rnd<T>(br[e]);
      }
      if (a.res) {
        float x[8];
        unpack8<T>(rv, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[p][e] = rnd<T>(x[e] + br[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) s[p][e] = br[e];
      }
      if (!in) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s[p][e] = 0.f;
      } else if (a.res_out) {
        store8((T*)a.res_out + (int64_t)m * a.ldro + c, s[p]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sq += s[p][e] * s[p][e];
    }
    const float rstd = rsqrtf(wave_sum(sq) / (float)a.D + a.eps);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = (p * 64 + lane) * 8;
      if (c >= a.D) continue;
      float w8[8], o[8];
      unpack8<T>(wv[p], w8);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (s[p][e] * rstd) * w8[e];
      store8((T*)a.out + (int64_t)m * a.ldo + c, o);
    }
  }
}

template <typename T, int MU, int RPW, bool PARTS>
static void launch_res_norm_form(const ResNormArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.M + 4 * RPW - 1) / (4 * RPW))), block(256);
  if (a.D <= 512) residual_rms_norm_kernel<T, 1, MU, RPW, PARTS><<<grid, block, 0, s>>>(a);
  else if (a.D <= 1024) residual_rms_norm_kernel<T, 2, MU, RPW, PARTS><<<grid, block, 0, s>>>(a);
  else if (a.D <= 2048) residual_rms_norm_kernel<T, 4, MU, RPW, PARTS><<<grid, block, 0, s>>>(a);
  else residual_rms_norm_kernel<T, 8, MU, RPW, PARTS><<<grid, block, 0, s>>>(a);
}

template <typename T, int MU, int RPW>
static void launch_res_norm_rows(const ResNormArgs& a, hipStream_t s) {
  if (a.y) launch_res_norm_form<T, MU, RPW, false>(a, s);
  else launch_res_norm_form<T, MU, RPW, true>(a, s);
}

// the low-rank form over many rows shares its weights across 8 rows per wave; few rows (the
// decode step) keep one row per wave, so no wave walks rows in sequence
constexpr int kResShareRows = 8192;

template <typename T, int MU>
static void launch_res_norm_mu(const ResNormArgs& a, hipStream_t s) {
  if constexpr (MU > 0) {
    if (a.M >= kResShareRows) return launch_res_norm_rows<T, MU, 8>(a, s);
  }
  launch_res_norm_rows<T, MU, 1>(a, s);
}

template <typename T>
static void launch_res_norm(const ResNormArgs& a, hipStream_t s) {
  switch (a.mu_x ? a.mu_k : 0) {
    case 4: launch_res_norm_mu<T, 4>(a, s); break;
    case 8: launch_res_norm_mu<T, 8>(a, s); break;
    case 16: launch_res_norm_mu<T, 16>(a, s); break;
    default: launch_res_norm_mu<T, 0>(a, s); break;
  }
}

// ------------------------------------------------------------------ lfm2_conv_step
// out[b, d] = c * conv(b * x) with bx = round(b x) pushed into the channel's state, the
// depthwise conv in fp32 in causal_conv1d_step's order (newest tap first), and each
// product rounded as the eager block rounds it.
template <typename T>
__global__ void __launch_bounds__(256)
lfm2_conv_step_kernel(const T* __restrict__ bcx, int64_t ld, const T* __restrict__ w, int K,
                      const int64_t* __restrict__ slots, T* __restrict__ state, int64_t s_ss, int64_t max_seqs,
                      T* __restrict__ out, int64_t ldo, int D) {
  const int b = blockIdx.x;
  const int d = blockIdx.y * 256 + threadIdx.x;
  if (d >= D) return;
  const T* row = bcx + (int64_t)b * ld;
  const float bx = rnd<T>(to_f32(row[d]) * to_f32(row[2 * D + d]));
  const T* wd = w + (int64_t)d * K;
  float acc = bx * to_f32(wd[K - 1]);
  if (K > 1) {
    const int64_t slot = slots[b];
    if (slot < 0 || slot >= max_seqs) {
      out[(int64_t)b * ldo + d] = from_f32<T>(__builtin_nanf(""));
      return;
    }
    T* st = state + slot * s_ss + (int64_t)d * (K - 1);
    for (int j = 0; j < K - 1; ++j) {
      const T old = st[j];
      acc += to_f32(old) * to_f32(wd[j]);
      if (j > 0) st[j - 1] = old;
    }
    st[K - 2] = from_f32<T>(bx);
  }
  out[(int64_t)b * ldo + d] = from_f32<T>(to_f32(row[D + d]) * rnd<T>(acc));
}

// ------------------------------------------------------------------ global_decode_prep
struct GlobalPrepArgs {
  const void* y;  // (B, ldy) fused projection rows: q|gate per head at 0, k at ck, v at cv,
  int64_t ldy;    // gamma / beta logits at cg / cb
  int64_t ck, cv, cg, cb;
  const void* wq;  // Canon taps (H d, Kc), (Hkv d, Kc), (Hkv d, Kc)
  const void* wk;
  const void* wv;
  int Kc;
  void* tq;  // Canon state tables (S, H d, Kc - 1), (S, Hkv d, Kc - 1) x 2
  void* tk;
  void* tv;
  int64_t tq_ss, tk_ss, tv_ss, max_seqs;
  const int64_t* slots;
  void* q;  // (B, H, d), (B, Hkv, d) x 2
  void* k;
  void* v;
  float* gamma;  // (B, H)
  float* beta;
  float eps;  // the head RMSNorm's (torch's default: the dtype's epsilon)
  float g_bias, b_bias;
  int B, H, Hkv, d;
};

// one wave per (sequence, head): heads [0, H) q, [H, H + Hkv) k, then v
template <typename T, int CPL>
__global__ void __launch_bounds__(64) global_decode_prep_kernel(GlobalPrepArgs a) {
  const int lane = threadIdx.x;
  const int b = blockIdx.x, j = blockIdx.y;
  const T* row = (const T*)a.y + (int64_t)b * a.ldy;
  const int kind = j < a.H ? 0 : (j < a.H + a.Hkv ? 1 : 2);
  const int h = kind == 0 ? j : (kind == 1 ? j - a.H : j - a.H - a.Hkv);
  const T* src = kind == 0 ? row + (int64_t)h * 2 * a.d : row + (kind == 1 ? a.ck : a.cv) + (int64_t)h * a.d;
  const T* wt = (const T*)(kind == 0 ? a.wq : (kind == 1 ? a.wk : a.wv));
  T* tab = (T*)(kind == 0 ? a.tq : (kind == 1 ? a.tk : a.tv));
  const int64_t tss = kind == 0 ? a.tq_ss : (kind == 1 ? a.tk_ss : a.tv_ss);
  T* dst = kind == 0 ? (T*)a.q + ((int64_t)b * a.H + h) * a.d
                     : (T*)(kind == 1 ? a.k : a.v) + ((int64_t)b * a.Hkv + h) * a.d;
  float x[CPL];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    x[i] = to_f32(src[i * 64 + lane]);
    ss += x[i] * x[i];
  }
  if (kind < 2) {
    const float rstd = rsqrtf(wave_sum(ss) / (float)a.d + a.eps);
#pragma unroll
    for (int i = 0; i < CPL; ++i) x[i] = rnd<T>(x[i] * rstd);
  }
  const int64_t slot = a.slots[b];
  const bool ok = slot >= 0 && slot < a.max_seqs;
  const int ch0 = h * a.d;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = ch0 + i * 64 + lane;
    const T* wd = wt + (int64_t)ch * a.Kc;
    float acc = x[i] * to_f32(wd[a.Kc - 1]);
    if (a.Kc > 1) {
      if (!ok) {
        dst[i * 64 + lane] = from_f32<T>(__builtin_nanf(""));
        continue;
      }
      T* st = tab + slot * tss + (int64_t)ch * (a.Kc - 1);
      for (int t = 0; t < a.Kc - 1; ++t) {
        const T old = st[t];
        acc += to_f32(old) * to_f32(wd[t]);
        if (t > 0) st[t - 1] = old;
      }
      st[a.Kc - 2] = from_f32<T>(x[i]);
    }
    dst[i * 64 + lane] = from_f32<T>(x[i] + acc);
  }
  if (kind == 0 && lane == 0 && a.gamma) {
    const int64_t o = (int64_t)b * a.H + h;
    a.gamma[o] = expf(gdn_log_decay(to_f32(row[a.cg + h]), a.g_bias));
    a.beta[o] = gdn_write_strength(to_f32(row[a.cb + h]), a.b_bias);
  }
}

}  // namespace atma

// ---------------------------------------------------------------------------- C ABI
using namespace atma;

extern "C" int atma_residual_rms_norm(const void* y, int64_t ldy, const float* parts, int64_t n_parts,
                                      const void* const* bias, int64_t n_bias, const void* mu_x, int64_t ldmu,
                                      const void* mu_w, int64_t mu_k, const void* res, int64_t ldr,
                                      void* res_out, int64_t ldro, const void* weight, void* out, int64_t ldo,
                                      int64_t M, int64_t D, float eps, int dtype, void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "residual_rms_norm: 16-bit only (dtype %d)", dtype);
  if (M < 0 || D < 8 || D % 8 || D > 4096 || M > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "residual_rms_norm: D must be a multiple of 8 in [8, 4096] (got %lld)",
                     (long long)D);
  if (M == 0) return ATMA_OK;
  if (!weight || !out || (!y && !parts) || (y && parts))
    return set_error(ATMA_ERR_INVALID, "residual_rms_norm: need weight, out and exactly one of y / parts");
  if ((parts && (n_parts < 1 || n_parts > kResMaxParts)) || n_bias < 0 || n_bias > kResMaxBias || (n_bias && !bias))
    return set_error(ATMA_ERR_INVALID, "residual_rms_norm: 1 to %d parts and at most %d biases", kResMaxParts,
                     kResMaxBias);
  if (mu_x && (!mu_w || (mu_k != 4 && mu_k != 8 && mu_k != 16) || ldmu < mu_k || ldmu % 2 || ((uintptr_t)mu_x & 3) ||
               ((uintptr_t)mu_w & 15)))
    return set_error(ATMA_ERR_INVALID, "residual_rms_norm: the low-rank term needs a 16-byte aligned mu_w of width 4, 8 "
                     "or 16");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if ((y && (!al16(y) || ldy % 8 || ldy < D)) || (parts && !al16(parts)) || (res && (!al16(res) || ldr % 8 || ldr < D)) ||
      (res_out && (!al16(res_out) || ldro % 8 || ldro < D)) || !al16(weight) || !al16(out) || ldo % 8 || ldo < D)
    return set_error(ATMA_ERR_INVALID, "residual_rms_norm: rows must be 16-byte aligned and at least D long");
  ResNormArgs a{};
  a.y = y;
  a.ldy = ldy;
  a.parts = parts;
  a.n_parts = parts ? (int)n_parts : 0;
  a.n_bias = (int)n_bias;
  for (int i = 0; i < a.n_bias; ++i) {
    if (!bias[i] || !al16(bias[i])) return set_error(ATMA_ERR_INVALID, "residual_rms_norm: bias %d null or unaligned", i);
    a.bias[i] = bias[i];
  }
  a.mu_x = mu_x;
  a.ldmu = ldmu;
  a.mu_w = mu_w;
  a.mu_k = (int)mu_k;
  a.res = res;
  a.ldr = ldr;
  a.res_out = res_out;
  a.ldro = ldro;
  a.w = weight;
  a.out = out;
  a.ldo = ldo;
  a.eps = eps;
  a.M = (int)M;
  a.D = (int)D;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16) launch_res_norm<bf16>(a, s);
  else launch_res_norm<f16>(a, s);
  return check_launch("residual_rms_norm");
}

extern "C" int atma_lfm2_conv_step(const void* bcx, int64_t ld, const void* weight, int64_t K, const int64_t* slots,
                                   void* state, int64_t s_ss, int64_t max_seqs, void* out, int64_t ldo, int64_t B,
                                   int64_t D, int dtype, void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16 && dtype != ATMA_F32)
    return set_error(ATMA_ERR_INVALID, "lfm2_conv_step: unknown dtype %d", dtype);
  if (B < 0 || D < 1 || K < 1 || K > 16 || ld < 3 * D || ldo < D || B > 0x7fffffff || D > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "lfm2_conv_step: bad sizes (rows of 3 D, 1 <= K <= 16)");
  if (B == 0) return ATMA_OK;
  if (!bcx || !weight || !out || (K > 1 && (!slots || !state)))
    return set_error(ATMA_ERR_INVALID, "lfm2_conv_step: null pointer");
  const dim3 grid((unsigned)B, (unsigned)((D + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
#define ATMA_LFM2_LAUNCH(T)                                                                                  \
  lfm2_conv_step_kernel<T><<<grid, dim3(256), 0, s>>>((const T*)bcx, ld, (const T*)weight, (int)K, slots, \
                                                      (T*)state, s_ss, max_seqs, (T*)out, ldo, (int)D)
  if (dtype == ATMA_BF16) ATMA_LFM2_LAUNCH(bf16);
  else if (dtype == ATMA_F16) ATMA_LFM2_LAUNCH(f16);
  else ATMA_LFM2_LAUNCH(float);
#undef ATMA_LFM2_LAUNCH
  return check_launch("lfm2_conv_step");
}

extern "C" int atma_global_decode_prep(const void* y, int64_t ldy, int64_t ck, int64_t cv, int64_t cg, int64_t cb,
                                       const void* wq, const void* wk, const void* wv, int64_t Kc, void* tq,
                                       int64_t tq_ss, void* tk, int64_t tk_ss, void* tv, int64_t tv_ss,
                                       int64_t max_seqs, const int64_t* slots, void* q, void* k, void* v,
                                       float* gamma, float* beta, float eps, float g_bias, float b_bias, int64_t B,
                                       int64_t H, int64_t Hkv, int64_t d, int dtype, void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "global_decode_prep: 16-bit only (dtype %d)", dtype);
  if (B < 0 || H < 1 || Hkv < 1 || H % Hkv || (d != 64 && d != 128) || Kc < 1 || Kc > 16 || B > 0x7fffffff ||
      H > 64)
    return set_error(ATMA_ERR_INVALID, "global_decode_prep: bad sizes (d 64 or 128, 1 <= Kc <= 16)");
  if (B == 0) return ATMA_OK;
  if (!y || !wq || !wk || !wv || !slots || !q || !k || !v || (Kc > 1 && (!tq || !tk || !tv)) ||
      ((gamma == nullptr) != (beta == nullptr)))
    return set_error(ATMA_ERR_INVALID, "global_decode_prep: null pointer");
  if (ck < 2 * H * d || cv < ck + Hkv * d || (gamma && (cg < 0 || cb < 0 || cg + H > ldy || cb + H > ldy)) ||
      cv + Hkv * d > ldy)
    return set_error(ATMA_ERR_INVALID, "global_decode_prep: column offsets outside the projection row");
  GlobalPrepArgs a{y, ldy, ck, cv, cg, cb, wq, wk, wv, (int)Kc, tq, tk, tv, tq_ss, tk_ss, tv_ss, max_seqs, slots,
                   q, k, v, gamma, beta, eps, g_bias, b_bias, (int)B, (int)H, (int)Hkv, (int)d};
  const dim3 grid((unsigned)B, (unsigned)(H + 2 * Hkv));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16) {
    if (d == 128) global_decode_prep_kernel<bf16, 2><<<grid, dim3(64), 0, s>>>(a);
    else global_decode_prep_kernel<bf16, 1><<<grid, dim3(64), 0, s>>>(a);
  } else {
    if (d == 128) global_decode_prep_kernel<f16, 2><<<grid, dim3(64), 0, s>>>(a);
    else global_decode_prep_kernel<f16, 1><<<grid, dim3(64), 0, s>>>(a);
  }
  return check_launch("global_decode_prep");
}
