// Per-head glue of the global layer, for prefill rows and decode rows alike (no reference
// counterpart as one call; the layer's eager chain is inference/models/atma.py:227-252,
// 397-437 with model/reference.py:131-139 and model/blocks.py:470-490):
//
//  * head_rms_norm: out[m, h] = rms_norm(x[m, h, :]) over each d-wide head (no gain), for a
//    strided view -- q is the first half of every head of the q|gate projection's row, so
//    the norm reads it in place and writes q contiguous, where the eager chain copies the
//    view and then runs a generic norm over rows of d = 128 (about 0.5 TB/s).
//  * lfm2_conv_packed: the LFM2 block's fresh-prefill mixer input, c * conv(b * x) from the
//    rows of its in_proj output over packed ragged sequences (model/reference.py:31-48,
//    inference/models/atma.py:625-673): packed_causal_conv1d's strip walk with the gate b
//    applied as each row enters the window and c as each output leaves, and the sequence's
//    K - 1 newest b * x values written to its state row -- one pass where the eager chain
//    makes three (each rounding as that chain rounds, so the result is the chain's bit for bit).
//  * global_gate: the two gated inputs of the layer's output projections,
//      a[m, h d + e] = c[m, h, e] sigmoid(gate[m, h, e])
//      g[m, h d + e] = round(rms_norm(r[m, h, :])[e]) sigmoid(mem_gate[m, h d + e])
//    with c read in Polar's head-major layout (the eager chain transposes it with a copy) and
//    r the memory readout (fp32 at decode, 16-bit at prefill), each sigmoid and product rounded to 16 bits as eager
//    torch rounds them.
//
// Layout: a head-row of d 16-bit values is d / 8 lanes with 16 bytes each (16 lanes at d =
// 128, 8 at d = 64), so a wave holds 4 or 8 head-rows; the RMS sums reduce over those lanes
// with DPP row operations.  HBM streams: every byte is read once and written once.
#include "common.h"

namespace atma {

template <int LPH>
__device__ __forceinline__ float head_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f32<0x141>(x);  // row_half_mirror: the two quads of 8 lanes
  if constexpr (LPH == 16) x += dpp_f32<0x140>(x);  // row_mirror: the two halves of 16 lanes
  return x;
}

__device__ __forceinline__ float sigmoid_fl(float x) { return 1.f / (1.f + expf(-x)); }

template <typename T>
__device__ __forceinline__ float rnd16(float x) {
  return to_f32(from_f32<T>(x));
}

template <typename T>
__device__ __forceinline__ void unpack8v(const u32x4& u, float* v) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = elem16<T>(u, e);
}
template <typename T>
__device__ __forceinline__ u32x4 pack8v(const float* v) {
  u32x4 u;
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = pack2<T>(v[2 * e], v[2 * e + 1]);
  return u;
}

// ------------------------------------------------------------------ head_rms_norm
struct HeadNormArgs {
  const void* x;  // element (m, h, e) at m ldr + h ldh + e
  int64_t ldr, ldh;
  void* out;  // (rows, H, d) contiguous
  int64_t rows;
  int H;
  float eps;
};

template <typename T, int LPH>
__global__ void __launch_bounds__(256) head_rms_norm_kernel(HeadNormArgs a) {
  constexpr int D = LPH * 8, HPW = 64 / LPH;
  const int lane = threadIdx.x & 63;
  const int64_t hr = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * HPW + lane / LPH;  // head-row
  const bool ok = hr < a.rows * a.H;
  const int64_t hrc = ok ? hr : 0;
  const int64_t m = hrc / a.H;
  const int h = (int)(hrc - m * a.H);
  const int e0 = 8 * (lane % LPH);
  float v[8];
  unpack8v<T>(*(const u32x4*)((const T*)a.x + m * a.ldr + h * a.ldh + e0), v);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  const float rstd = rsqrtf(head_sum<LPH>(ss) / (float)D + a.eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] *= rstd;
  if (ok) *(u32x4*)((T*)a.out + hrc * D + e0) = pack8v<T>(v);
}

// ------------------------------------------------------------------ global_gate
struct GateArgs {
  const void* c;  // element (b, t, h, e) at b c_sb + t c_st + h c_sh + e; row m = b T + t
  int64_t c_sb, c_st, c_sh;
  int T;
  const void* gate;  // (m, h, e) at m g_sr + h g_sh + e
  int64_t g_sr, g_sh;
  const void* r;  // (m, h, e) at m r_sr + h d + e, fp32 (r_f32) or T; null: no memory branch
  int64_t r_sr;
  int r_f32;
  const void* mgate;  // (m, h, e) at m mg_sr + h d + e
  int64_t mg_sr;
  void* xa;  // (m, h d + e) at m a_sr
  int64_t a_sr;
  void* xm;  // (m, h d + e) at m m_sr
  int64_t m_sr;
  int64_t rows;
  int H;
  float mem_eps;
};

template <typename T, int LPH>
__global__ void __launch_bounds__(256) global_gate_kernel(GateArgs a) {
  constexpr int D = LPH * 8, HPW = 64 / LPH;
  const int lane = threadIdx.x & 63;
  const int64_t hr = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * HPW + lane / LPH;
  const bool ok = hr < a.rows * a.H;
  const int64_t hrc = ok ? hr : 0;
  const int64_t m = hrc / a.H;
  const int h = (int)(hrc - m * a.H);
  const int64_t b = m / a.T, t = m - b * a.T;
  const int e0 = 8 * (lane % LPH);
  float cv[8], gv[8], o[8];
  unpack8v<T>(*(const u32x4*)((const T*)a.c + b * a.c_sb + t * a.c_st + h * a.c_sh + e0), cv);
  unpack8v<T>(*(const u32x4*)((const T*)a.gate + m * a.g_sr + h * a.g_sh + e0), gv);
  float rv[8], mv[8];
  if (a.r) {
    if (a.r_f32) {
      const float* rp = (const float*)a.r + m * a.r_sr + h * D + e0;
      const f32x4 r0 = *(const f32x4*)rp, r1 = *(const f32x4*)(rp + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) rv[e] = r0[e], rv[4 + e] = r1[e];
    } else {
      unpack8v<T>(*(const u32x4*)((const T*)a.r + m * a.r_sr + h * D + e0), rv);
    }
    unpack8v<T>(*(const u32x4*)((const T*)a.mgate + m * a.mg_sr + h * D + e0), mv);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = cv[e] * rnd16<T>(sigmoid_fl(gv[e]));
  if (ok) *(u32x4*)((T*)a.xa + m * a.a_sr + h * D + e0) = pack8v<T>(o);
  if (!a.r) return;
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += rv[e] * rv[e];
  const float rstd = rsqrtf(head_sum<LPH>(ss) / (float)D + a.mem_eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = rnd16<T>(rv[e] * rstd) * rnd16<T>(sigmoid_fl(mv[e]));
  if (ok) *(u32x4*)((T*)a.xm + m * a.m_sr + h * D + e0) = pack8v<T>(o);
}

// ------------------------------------------------------------------ lfm2_conv_packed
constexpr int kLfmStrip = 32;  // tokens per lane strip

// One lane = 8 consecutive channels x a strip of kLfmStrip tokens (packed_causal_conv1d's
// walk: the K - 1 previous rows stay in registers as the strip advances).
template <typename T, int K>
__global__ void __launch_bounds__(64)
lfm2_conv_packed_kernel(const T* __restrict__ bcx, int64_t ld, const T* __restrict__ w, T* __restrict__ out,
                        int64_t ldo, T* __restrict__ state, int64_t s_ss, int64_t num_slots,
                        const int32_t* __restrict__ seq_start, const int32_t* __restrict__ seq_end,
                        const int32_t* __restrict__ seq_slot, int64_t total, int D) {
  const int c0 = (blockIdx.y * 64 + threadIdx.x) * 8;
  if (c0 >= D) return;
  const int64_t t_beg = (int64_t)blockIdx.x * kLfmStrip;
  const int64_t t_end = min(t_beg + kLfmStrip, total);
  float wt[K][8];
#pragma unroll
  for (int j = 0; j < K; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) wt[j][e] = to_f32(w[(int64_t)(c0 + e) * K + j]);
  auto load_bx = [&](int64_t t, float* v) {  // round(b * x) of row t
    float b[8], x[8];
    unpack8v<T>(*(const u32x4*)(bcx + t * ld + c0), b);
    unpack8v<T>(*(const u32x4*)(bcx + t * ld + 2 * D + c0), x);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = rnd16<T>(b[e] * x[e]);
  };
  float win[K][8];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int64_t t = t_beg - (K - 1) + j;
    if (t >= 0) {
      load_bx(t, win[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[j][e] = 0.f;
    }
  }
#pragma unroll 4
  for (int64_t t = t_beg; t < t_end; ++t) {
    load_bx(t, win[K - 1]);
    const int64_t start = seq_start[t];
    float acc[8], cg[8], o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const bool live = t - (K - 1 - j) >= start;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(live ? win[j][e] : 0.f, wt[j][e], acc[e]);
    }
    unpack8v<T>(*(const u32x4*)(bcx + t * ld + D + c0), cg);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = cg[e] * rnd16<T>(acc[e]);
    *(u32x4*)(out + t * ldo + c0) = pack8v<T>(o);
    if (t == (int64_t)seq_end[t] - 1) {  // the sequence's K - 1 newest b * x into its state row
      const int64_t slot = seq_slot[t];
      if (slot >= 0 && slot < num_slots) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
          const bool live = t - (K - 2 - j) >= start;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            state[slot * s_ss + (int64_t)(c0 + e) * (K - 1) + j] = from_f32<T>(live ? win[j + 1][e] : 0.f);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[j][e] = win[j + 1][e];
  }
}

template <typename T>
static int launch_gate(const GateArgs& a, int d, hipStream_t s) {
  const int hpw = 64 / (d / 8);
  const int64_t waves = (a.rows * a.H + hpw - 1) / hpw;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (d == 128) global_gate_kernel<T, 16><<<grid, dim3(256), 0, s>>>(a);
  else global_gate_kernel<T, 8><<<grid, dim3(256), 0, s>>>(a);
  return check_launch("global_gate");
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace atma

using namespace atma;

extern "C" int atma_head_rms_norm(const void* x, int64_t ldr, int64_t ldh, void* out, int64_t rows, int64_t H,
                                  int64_t d, float eps, int dtype, void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "head_rms_norm: 16-bit only (dtype %d)", dtype);
  if (rows < 0 || H < 1 || (d != 64 && d != 128) || rows * H > (int64_t)1 << 40)
    return set_error(ATMA_ERR_INVALID, "head_rms_norm: bad sizes (d 64 or 128)");
  if (rows == 0) return ATMA_OK;
  if (!x || !out) return set_error(ATMA_ERR_INVALID, "head_rms_norm: null pointer");
  if (!al16(x) || !al16(out) || ldr % 8 || ldh % 8 || ldh < d || ldr < ldh * (H - 1) + d)
    return set_error(ATMA_ERR_INVALID, "head_rms_norm: heads must be 16-byte aligned and not overlap");
  HeadNormArgs a{x, ldr, ldh, out, rows, (int)H, eps};
  const int64_t waves = (rows * H + 64 / (d / 8) - 1) / (64 / (d / 8));
  const dim3 grid((unsigned)((waves + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16) {
    if (d == 128) head_rms_norm_kernel<bf16, 16><<<grid, dim3(256), 0, s>>>(a);
    else head_rms_norm_kernel<bf16, 8><<<grid, dim3(256), 0, s>>>(a);
  } else {
    if (d == 128) head_rms_norm_kernel<f16, 16><<<grid, dim3(256), 0, s>>>(a);
    else head_rms_norm_kernel<f16, 8><<<grid, dim3(256), 0, s>>>(a);
  }
  return check_launch("head_rms_norm");
}

extern "C" int atma_global_gate(const void* c, int64_t c_sb, int64_t c_st, int64_t c_sh, int64_t T, const void* gate,
                                int64_t g_sr, int64_t g_sh, const void* r, int64_t r_sr, int r_dtype, const void* mgate,
                                int64_t mg_sr, void* xa, int64_t a_sr, void* xm, int64_t m_sr, int64_t rows,
                                int64_t H, int64_t d, float mem_eps, int dtype, void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "global_gate: 16-bit only (dtype %d)", dtype);
  if (rows < 0 || H < 1 || H > 64 || (d != 64 && d != 128) || T < 1 || rows % T || rows * H > (int64_t)1 << 40)
    return set_error(ATMA_ERR_INVALID, "global_gate: bad sizes (d 64 or 128, rows a multiple of T)");
  if (rows == 0) return ATMA_OK;
  if (!c || !gate || !xa || (r && (!mgate || !xm)))
    return set_error(ATMA_ERR_INVALID, "global_gate: null pointer");
  if (r && r_dtype != ATMA_F32 && r_dtype != dtype)
    return set_error(ATMA_ERR_INVALID, "global_gate: r must be fp32 or the inputs' dtype");
  const int r_f32 = r_dtype == ATMA_F32;
  const bool aligned = al16(c) && al16(gate) && al16(xa) && c_sb % 8 == 0 && c_st % 8 == 0 && c_sh % 8 == 0 &&
                       g_sr % 8 == 0 && g_sh % 8 == 0 && a_sr % 8 == 0 &&
                       (!r || (al16(r) && al16(mgate) && al16(xm) && r_sr % (r_f32 ? 4 : 8) == 0 && mg_sr % 8 == 0 &&
                        m_sr % 8 == 0));
  if (!aligned) return set_error(ATMA_ERR_INVALID, "global_gate: every head-row must be 16-byte aligned");
  GateArgs a{c, c_sb, c_st, c_sh, (int)T, gate, g_sr, g_sh, r, r_sr, r_f32, mgate, mg_sr, xa, a_sr, xm, m_sr,
             rows, (int)H, mem_eps};
  hipStream_t s = (hipStream_t)stream;
  return dtype == ATMA_BF16 ? launch_gate<bf16>(a, (int)d, s) : launch_gate<f16>(a, (int)d, s);
}

extern "C" int atma_global_decode_gate(const void* c, const float* r, const void* y, int64_t ldy, int64_t cm, void* x2,
                                       int64_t ldx2, float mem_eps, int64_t B, int64_t H, int64_t d, int dtype,
                                       void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "global_decode_gate: 16-bit only (dtype %d)", dtype);
  if (B < 0 || H < 1 || (d != 64 && d != 128) || B > 0x7fffffff || H > 64)
    return set_error(ATMA_ERR_INVALID, "global_decode_gate: bad sizes (d 64 or 128)");
  if (B == 0) return ATMA_OK;
  if (!c || !y || !x2) return set_error(ATMA_ERR_INVALID, "global_decode_gate: null pointer");
  if (ldy < 2 * H * d || (r && (cm < 0 || cm + H * d > ldy)) || ldx2 < (r ? 2 : 1) * H * d)
    return set_error(ATMA_ERR_INVALID, "global_decode_gate: column offsets outside the rows");
  const char* yb = (const char*)y;
  const int64_t esz = 2;
  return atma_global_gate(c, H * d, H * d, d, 1, yb + d * esz, ldy, 2 * d, r, H * d, ATMA_F32, r ? yb + cm * esz : nullptr,
                          ldy, x2, ldx2, r ? (char*)x2 + H * d * esz : nullptr, ldx2, B, H, d, mem_eps, dtype,
                          stream);
}

extern "C" int atma_lfm2_conv_packed(const void* bcx, int64_t ld, const void* weight, int64_t K, void* out,
                                    int64_t ldo, void* state, int64_t s_ss, int64_t num_slots,
                                    const int32_t* token_seq_starts, const int32_t* token_seq_ends,
                                    const int32_t* token_seq_slots, int64_t total, int64_t D, int dtype,
                                    void* stream) {
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "lfm2_conv_packed: 16-bit only (dtype %d)", dtype);
  if (K != 3 && K != 4)
    return set_error(ATMA_ERR_UNSUPPORTED, "lfm2_conv_packed: kernel size %lld (ATMA's sizes 3 and 4)", (long long)K);
  if (total < 0 || D < 8 || D % 8 || D > 0x7fffffff || total > 0x7fffffffll * kLfmStrip || num_slots < 0)
    return set_error(ATMA_ERR_INVALID, "lfm2_conv_packed: bad sizes (D a multiple of 8)");
  if (total == 0) return ATMA_OK;
  if (!bcx || !weight || !out || !state || !token_seq_starts || !token_seq_ends || !token_seq_slots)
    return set_error(ATMA_ERR_INVALID, "lfm2_conv_packed: null pointer");
  if (!al16(bcx) || !al16(out) || ld % 8 || ld < 3 * D || ldo % 8 || ldo < D)
    return set_error(ATMA_ERR_INVALID, "lfm2_conv_packed: rows must be 16-byte aligned (bcx rows of 3 D)");
  const dim3 grid((unsigned)((total + kLfmStrip - 1) / kLfmStrip), (unsigned)((D / 8 + 63) / 64));
  hipStream_t s = (hipStream_t)stream;
#define ATMA_LFM2P(TT, KK)                                                                                    \
  lfm2_conv_packed_kernel<TT, KK><<<grid, dim3(64), 0, s>>>((const TT*)bcx, ld, (const TT*)weight, (TT*)out, ldo, \
                                                            (TT*)state, s_ss, num_slots, token_seq_starts,        \
                                                            token_seq_ends, token_seq_slots, total, (int)D)
  if (dtype == ATMA_BF16) {
    if (K == 3) ATMA_LFM2P(bf16, 3);
    else ATMA_LFM2P(bf16, 4);
  } else {
    if (K == 3) ATMA_LFM2P(f16, 3);
    else ATMA_LFM2P(f16, 4);
  }
#undef ATMA_LFM2P
  return check_launch("lfm2_conv_packed");
}
