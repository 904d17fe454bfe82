// Paged Polar GQA decode: split-K over the page table, then a merge.
//
// Reference: _polar_decode_kernel / polar_attention_decode,
// kernel/polar_triton.py:682-858 -- one program per (sequence, KV head), the G
// query heads of the group as tile rows, keys read straight from the paged cache
// (phys = block_tables[b, pos // page], row pos % page), the same online
// (m, L, Q2, S) statistics and null-sink fold as the prefill.
//
// MI355X design: decode is HBM-bound (4 FLOP per cached byte), and 64 sequences
// x 2 KV heads is far too few programs for 256 CUs, so:
//  * pass 1 (split): one workgroup per (sequence, KV head, 256-token span).  Its
//    4 waves take 64-key sub-blocks; QK^T runs on v_mfma_f32_16x16x32 (query
//    heads = rows, zero-padded to 16; keys = columns) with K read directly from
//    the page into the operand registers (each lane one 64-byte run of a row);
//    p goes through a small LDS tile and PV runs on VALU with each lane owning 8
//    contiguous head dims, so a wave reads 4 whole 256-byte V rows per load.
//    Keys past the context, past the window or on an out-of-range page are never
//    loaded.  The span's (m, L, Q2, acc) goes to the workspace.
//  * pass 2 (merge): one workgroup per (sequence, query head) combines the live
//    spans (m = max, rescale by 2^(m_i - m)), folds the null sink and writes c, mag.
// The grid depends only on (B, Hq, max_pages): graph capturable.
#include "common.h"

namespace atma {

constexpr int kSplitTokens = 256;

struct DecodeArgs {
  const void* q;
  int64_t q_sb, q_sh;
  const void* kc;
  const void* vc;
  int64_t num_pages;
  int page_size;
  int Hkv;
  const int32_t* bt;
  int64_t bt_sb;
  int max_pages;
  const int32_t* ctx;
  const float* v_null;
  const float* null_base;
  const float* null_slope_raw;
  const float* len_gain_raw;
  const float* mag_beta_raw;
  void* c;
  void* mag;
  int B, Hq, G;
  int window;
  float eps;
  int max_splits;
  float* ws;  // [B][Hq][max_splits][D + 4]
};

__device__ __forceinline__ void span_of(int ctx, int window, int sp, int& t0, int& t1) {
  const int lo = window > 0 ? max(ctx - window, 0) : 0;
  t0 = max(sp * kSplitTokens, lo);
  t1 = min((sp + 1) * kSplitTokens, ctx);
}

__device__ __forceinline__ void unpack8(const u32x4& x, float* out, bf16) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    out[2 * w] = __uint_as_float(x[w] << 16);
    out[2 * w + 1] = __uint_as_float(x[w] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack8(const u32x4& x, float* out, f16) {
  Pack8 p;
  p.u = x;
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)p.h[e];
}

// GP = query-head rows per KV group, padded (4 / 8 / 16).
template <typename T, int D, int GP>
__global__ void __launch_bounds__(256) polar_decode_split_kernel(DecodeArgs a) {
  constexpr bool kHalf = sizeof(T) == 2;
  constexpr int DCH = D / 8;        // lanes per key row in the PV pass (8 dims each)
  constexpr int KPI = 64 / DCH;     // keys per PV step
  constexpr int QK_E = D / 4;       // elements of a K row per lane (one quarter)
  __shared__ __attribute__((aligned(16))) float Ps[4][64][GP];
  __shared__ float Alpha[4][GP];
  __shared__ float Wst[4][GP][3];
  __shared__ __attribute__((aligned(16))) float Wacc[4][GP][D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bhk = blockIdx.x, sp = blockIdx.y;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int ctx = a.ctx[b];
  int t0, t1;
  span_of(ctx, a.window, sp, t0, t1);
  if (t0 >= t1) return;  // uniform across the workgroup

  const int col = lane & 15, grp4 = lane >> 4;  // MFMA: key column, K-quarter / row group
  // per-row (query head) calibration: rows 4*grp4 + i held by this lane
  float n_cal = (float)ctx;
  if (a.window > 0) n_cal = fminf(n_cal, (float)a.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float logn = logf(n_cal);
  float c1r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * grp4 + i;
    const int hq = hk * a.G + (row < a.G ? row : 0);
    const float temp = 1.f + softplus(a.len_gain_raw[hq]) * logn;
    c1r[i] = temp * kLog2e * (1.f / sqrtf((float)D));
  }

  // q operand (A of QK^T): row = head (lane & 15), quarter = lane >> 4
  u32x4 qa[kHalf ? D / 32 : 1];
  float qf[kHalf ? 1 : D / 4];
  {
    const int row = col;
    const bool ok = row < a.G;
    const T* qp = (const T*)a.q + b * a.q_sb + (int64_t)(hk * a.G + (ok ? row : 0)) * a.q_sh +
                  QK_E * grp4;
    if constexpr (kHalf) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) qa[s] = ok ? *(const u32x4*)(qp + 8 * s) : u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int s4 = 0; s4 < D / 16; ++s4) {
        f32x4 x = ok ? *(const f32x4*)(qp + 4 * s4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[4 * s4 + e] = x[e];
      }
    }
  }

  const T* kc = (const T*)a.kc;
  const T* vc = (const T*)a.vc;
  const int32_t* btb = a.bt + (int64_t)b * a.bt_sb;
  const int64_t row_elems = (int64_t)a.Hkv * D;
  // Offset of key `pos` in the cache (elements); ok=false for pages outside the table.
  auto key_off = [&](int pos, bool& ok) -> int64_t {
    const int lp = pos / a.page_size;
    int phys = (lp < a.max_pages) ? btb[lp] : -1;
    ok = phys >= 0 && phys < a.num_pages;
    if (!ok) phys = 0;
    return ((int64_t)phys * a.page_size + (pos - lp * a.page_size)) * row_elems + (int64_t)hk * D;
  };
  // With 64-aligned sub-blocks and page_size % 64 == 0 a sub-block lies in one page.
  const bool page_aligned = (a.page_size % 64) == 0;

  float m_run[4], l_part[4], q2_part[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = kSentinel;
    l_part[i] = 0.f;
    q2_part[i] = 0.f;
  }
  float acc[GP][8];
#pragma unroll
  for (int r = 0; r < GP; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;

  const int dch = lane % DCH, kg = lane / DCH;
  for (int sb = (t0 & ~63) + 64 * wave; sb < t1; sb += 256) {
    int64_t sb_off = 0;
    bool sb_page_ok = true;
    if (page_aligned) sb_off = key_off(sb, sb_page_ok);
    // ---- S = Q K^T over four 16-key tiles
    f32x4 sc[4];
    bool kok[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = sb + 16 * j + col;
      bool ok = pos >= t0 && pos < t1;
      int64_t off = 0;
      if (page_aligned) {
        ok = ok && sb_page_ok;
        off = sb_off + (int64_t)(16 * j + col) * row_elems;
      } else if (ok) {
        off = key_off(pos, ok);
      }
      kok[j] = ok;
      const T* kr = kc + off + QK_E * grp4;
      sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (kHalf) {
        u32x4 kb[D / 32];
#pragma unroll
        for (int s = 0; s < D / 32; ++s) kb[s] = ok ? *(const u32x4*)(kr + 8 * s) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < D / 32; ++s) sc[j] = mfma16x16x32<T>(qa[s], kb[s], sc[j]);
      } else {
        f32x4 kb[D / 16];
#pragma unroll
        for (int s4 = 0; s4 < D / 16; ++s4)
          kb[s4] = ok ? *(const f32x4*)(kr + 4 * s4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < D / 16; ++s4)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[4 * s4 + e], kb[s4][e], sc[j], 0, 0, 0);
      }
    }
    // ---- online softmax; rows = heads 4*grp4+i, column key = sb + 16 j + col
    float alpha_r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = kSentinel;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = kok[j] ? sc[j][i] * c1r[i] : kSentinel;
        sc[j][i] = x;
        mx = fmaxf(mx, x);
      }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
      const float m_new = fmaxf(m_run[i], mx);
      const float alpha = exp2f(m_run[i] - m_new);
      m_run[i] = m_new;
      float ls = 0.f, qs = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = kok[j] ? exp2f(sc[j][i] - m_new) : 0.f;
        sc[j][i] = p;
        ls += p;
        qs += p * p;
      }
      l_part[i] = l_part[i] * alpha + ls;
      q2_part[i] = q2_part[i] * alpha * alpha + qs;
      alpha_r[i] = alpha;
    }
    if (4 * grp4 < GP) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        *(f32x4*)&Ps[wave][16 * j + col][4 * grp4] = sc[j];
      }
      if (col == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) Alpha[wave][4 * grp4 + i] = alpha_r[i];
      }
    }
    wave_sync();
    // ---- acc = acc * alpha + P V   (lane: dims 8*dch.., keys kg, kg+KPI, ...)
    {
      float al[GP];
#pragma unroll
      for (int r = 0; r < GP; ++r) al[r] = Alpha[wave][r];
#pragma unroll
      for (int r = 0; r < GP; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] *= al[r];
    }
#pragma unroll 4
    for (int it = 0; it < 64 / KPI; ++it) {
      const int kk = it * KPI + kg;
      const int pos = sb + kk;
      bool ok = pos >= t0 && pos < t1;
      int64_t off = 0;
      if (page_aligned) {
        ok = ok && sb_page_ok;
        off = sb_off + (int64_t)kk * row_elems;
      } else if (ok) {
        off = key_off(pos, ok);
      }
      float vv[8];
      if (ok) {
        const T* vr = vc + off + 8 * dch;
        if constexpr (kHalf) {
          unpack8(*(const u32x4*)vr, vv, T{});
        } else {
          f32x4 x0 = *(const f32x4*)vr, x1 = *(const f32x4*)(vr + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vv[e] = x0[e];
            vv[4 + e] = x1[e];
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[e] = 0.f;
      }
#pragma unroll
      for (int r4 = 0; r4 < GP / 4; ++r4) {
        const f32x4 p4 = *(const f32x4*)&Ps[wave][kk][4 * r4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[4 * r4 + rr][e] += p4[rr] * vv[e];
      }
    }
    wave_sync();
  }

  // ---- reduce this wave: L, Q2 over the 16 key columns; acc over the key groups
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {
      l_part[i] += __shfl_xor(l_part[i], m, 64);
      q2_part[i] += __shfl_xor(q2_part[i], m, 64);
    }
  }
#pragma unroll
  for (int r = 0; r < GP; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int m = DCH; m < 64; m <<= 1) acc[r][e] += __shfl_xor(acc[r][e], m, 64);
    }
  if (col == 0 && 4 * grp4 < GP) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      Wst[wave][4 * grp4 + i][0] = m_run[i];
      Wst[wave][4 * grp4 + i][1] = l_part[i];
      Wst[wave][4 * grp4 + i][2] = q2_part[i];
    }
  }
  if (kg == 0) {
#pragma unroll
    for (int r = 0; r < GP; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) Wacc[wave][r][8 * dch + e] = acc[r][e];
  }
  __syncthreads();
  // ---- combine the 4 waves (a wave with no keys keeps m = sentinel, L = 0)
  const int nrow = a.G < GP ? a.G : GP;
  for (int idx = tid; idx < nrow * D; idx += 256) {
    const int r = idx / D, d = idx % D;
    float M = kSentinel;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, Wst[w][r][0]);
    float S = 0.f, L = 0.f, Q2 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = exp2f(Wst[w][r][0] - M);
      S += Wacc[w][r][d] * f;
      L += Wst[w][r][1] * f;
      Q2 += Wst[w][r][2] * f * f;
    }
    const int hq = hk * a.G + r;
    float* rec = a.ws + (((int64_t)b * a.Hq + hq) * a.max_splits + sp) * (D + 4);
    rec[4 + d] = S;
    if (d == 0) {
      rec[0] = M;
      rec[1] = L;
      rec[2] = Q2;
    }
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(D) polar_decode_merge_kernel(DecodeArgs a) {
  __shared__ float red[D / 64];
  const int bh = blockIdx.x;
  const int b = bh / a.Hq, hq = bh % a.Hq;
  const int d = threadIdx.x;
  const int ctx = a.ctx[b];
  const int lo = a.window > 0 ? max(ctx - a.window, 0) : 0;
  const int sp0 = lo / kSplitTokens;
  const int sp1 = min(ctx > lo ? (ctx + kSplitTokens - 1) / kSplitTokens : sp0, a.max_splits);
  const float* recs = a.ws + ((int64_t)b * a.Hq + hq) * a.max_splits * (D + 4);
  float M = kSentinel, L = 0.f, Q2 = 0.f, S = 0.f;
  for (int sp = sp0; sp < sp1; ++sp) {
    const float* rec = recs + (int64_t)sp * (D + 4);
    const float mi = rec[0];
    const float mn = fmaxf(M, mi);
    const float fo = exp2f(M - mn), fi = exp2f(mi - mn);
    L = L * fo + rec[1] * fi;
    Q2 = Q2 * fo * fo + rec[2] * fi * fi;
    S = S * fo + rec[4 + d] * fi;
    M = mn;
  }
  float n_cal = (float)ctx;
  if (a.window > 0) n_cal = fminf(n_cal, (float)a.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float temp = 1.f + softplus(a.len_gain_raw[hq]) * logf(n_cal);
  const float nullv = a.null_base[hq] + softplus(a.null_slope_raw[hq]) * sqrtf(logf(n_cal + 1.f));
  const float an2 = temp * nullv * kLog2e;
  const float mn = fmaxf(M, an2);
  const float al = exp2f(M - mn);
  L *= al;
  Q2 *= al * al;
  const float pn = exp2f(an2 - mn);
  const float Z = L + pn;
  const float s = S * al + pn * a.v_null[(int64_t)hq * D + d];
  float ss = wave_sum(s * s);
  if ((d & 63) == 0) red[d >> 6] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int w = 0; w < D / 64; ++w) ss += red[w];
  const float inv = 1.f / fmaxf(sqrtf(ss), a.eps);
  ((T*)a.c)[((int64_t)b * a.Hq + hq) * D + d] = (T)(s * inv);
  if (d == 0) {
    const float n_eff = L * L / fmaxf(Q2, 1e-30f);
    const float m_eff = n_eff * (L / fmaxf(Z, a.eps));
    const float beta = softplus(a.mag_beta_raw[hq]);
    ((T*)a.mag)[(int64_t)b * a.Hq + hq] = (T)tanhf(beta * log1pf(m_eff));
  }
}

static int max_splits_for(int64_t max_pages, int64_t page_size) {
  return (int)((max_pages * page_size + kSplitTokens - 1) / kSplitTokens);
}

template <typename T, int D, int GP>
static int launch_decode(DecodeArgs a, hipStream_t s) {
  if (a.max_splits > 0) {
    polar_decode_split_kernel<T, D, GP>
        <<<dim3((unsigned)(a.B * a.Hkv), (unsigned)a.max_splits), dim3(256), 0, s>>>(a);
    int rc = check_launch("polar_attention_decode(split)");
    if (rc) return rc;
  }
  polar_decode_merge_kernel<T, D><<<dim3((unsigned)(a.B * a.Hq)), dim3(D), 0, s>>>(a);
  return check_launch("polar_attention_decode(merge)");
}

template <typename T, int D>
static int dispatch_gp(DecodeArgs a, hipStream_t s) {
  if (a.G <= 4) return launch_decode<T, D, 4>(a, s);
  if (a.G <= 8) return launch_decode<T, D, 8>(a, s);
  return launch_decode<T, D, 16>(a, s);
}

}  // namespace atma

extern "C" size_t atma_polar_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t max_pages,
                                                    int64_t page_size, int64_t d) {
  if (B <= 0 || Hq <= 0 || max_pages <= 0 || page_size <= 0 || d <= 0) return 0;
  return (size_t)B * Hq * atma::max_splits_for(max_pages, page_size) * (d + 4) * sizeof(float);
}

extern "C" int atma_polar_attention_decode(
    const void* q, int64_t q_sb, int64_t q_sh, const void* k_cache, const void* v_cache,
    int64_t num_pages, int64_t page_size, int64_t Hkv, const int32_t* block_tables, int64_t bt_sb,
    int64_t max_pages, const int32_t* context_lens, const float* v_null, const float* null_base,
    const float* null_slope_raw, const float* len_gain_raw, const float* mag_beta_raw, void* c,
    void* mag, int64_t B, int64_t Hq, int64_t d, int dtype, int64_t window, float eps,
    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace atma;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || page_size <= 0 || max_pages < 0 || num_pages < 0)
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: bad sizes");
  if (Hq % Hkv) return set_error(ATMA_ERR_INVALID, "polar_attention_decode: Hq %% Hkv != 0");
  if (Hq / Hkv > 16)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_decode: GQA group %lld > 16",
                     (long long)(Hq / Hkv));
  if (d != 64 && d != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "polar_attention_decode: head_dim %lld (supported: 64, 128)",
                     (long long)d);
  if (B == 0) return ATMA_OK;
  if (!q || !c || !mag || !context_lens || !v_null || !null_base || !null_slope_raw ||
      !len_gain_raw || !mag_beta_raw)
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: null pointer");
  if (max_pages > 0 && (!k_cache || !v_cache || !block_tables))
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: null cache pointer");
  const int es = dtype_size(dtype);
  if (!es) return set_error(ATMA_ERR_INVALID, "polar_attention_decode: unknown dtype %d", dtype);
  if ((uintptr_t)q % 16 || (q_sb * es) % 16 || (q_sh * es) % 16 || (uintptr_t)k_cache % 16 ||
      (uintptr_t)v_cache % 16)
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: tensors must be 16-byte aligned");
  const size_t need = atma_polar_decode_workspace_bytes(B, Hq, max_pages, page_size, d);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(ATMA_ERR_WORKSPACE, "polar_attention_decode: workspace %zu < %zu bytes",
                     workspace_bytes, need);
  if (max_pages * page_size > (1ll << 30) || B * Hkv > 0x7fffffffll)
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: sizes too large");
  DecodeArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.kc = k_cache; a.vc = v_cache;
  a.num_pages = num_pages; a.page_size = (int)page_size; a.Hkv = (int)Hkv;
  a.bt = block_tables; a.bt_sb = bt_sb; a.max_pages = (int)max_pages; a.ctx = context_lens;
  a.v_null = v_null; a.null_base = null_base; a.null_slope_raw = null_slope_raw;
  a.len_gain_raw = len_gain_raw; a.mag_beta_raw = mag_beta_raw;
  a.c = c; a.mag = mag; a.B = (int)B; a.Hq = (int)Hq; a.G = (int)(Hq / Hkv);
  a.window = window > 0 ? (int)window : 0; a.eps = eps;
  a.max_splits = max_splits_for(max_pages, page_size);
  a.ws = (float*)workspace;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_BF16: return d == 128 ? dispatch_gp<bf16, 128>(a, s) : dispatch_gp<bf16, 64>(a, s);
    case ATMA_F16: return d == 128 ? dispatch_gp<f16, 128>(a, s) : dispatch_gp<f16, 64>(a, s);
    default: return d == 128 ? dispatch_gp<float, 128>(a, s) : dispatch_gp<float, 64>(a, s);
  }
}
