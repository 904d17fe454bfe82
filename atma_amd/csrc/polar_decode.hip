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
//  * pass 1 (split): one workgroup per (sequence, KV head, 2048-token span); each
//    of its 4 waves walks a quarter of the span in 32-key sub-blocks.  QK^T runs
//    on v_mfma_f32_16x16x32 (query heads = rows, zero-padded to 16; keys =
//    columns) with K read from the page straight into the operand registers; p
//    goes through a small LDS tile and PV runs on VALU with each lane owning 8
//    contiguous head dims, so one V load covers 4 whole 256-byte rows.  Pages
//    whose size is a multiple of 32 are read with buffer loads (page base in
//    scalar registers, page ids fetched once per wave and picked with
//    v_readlane), and K of the next sub-block is issued after QK^T, V of the next
//    after PV, so ~16 KB per wave stay in flight without any full drain.  Keys
//    past the context, past the window or on an out-of-range page never reach
//    the sums.  The span's (m, L, Q2, acc) goes to the workspace.
//  * pass 2 (merge): one workgroup per (sequence, query head) combines the live
//    spans (m = max, rescale by 2^(m_i - m)), folds the null sink and writes c, mag.
// The grid depends only on (B, Hq, max_pages): graph capturable.
#include <algorithm>
#include <mutex>
#include "common.h"
#include "gated_delta_step.h"

namespace atma {

#ifndef ATMA_SPLIT_TOKENS
#define ATMA_SPLIT_TOKENS 2048
#endif
constexpr int kSplitTokens = ATMA_SPLIT_TOKENS;  // tokens per span
constexpr int kWaveTokens = kSplitTokens / 4;    // a wave's share of a span
// a wave's sub-blocks have one page id per lane, with lane 63 always left at -1
static_assert(kWaveTokens % 32 == 0 && kWaveTokens / 32 < 64, "span split");

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
  float* ws;  // [B][Hq][max_splits][D + 4] (span split) or [NW + B*Hkv][G][D + 4] (balanced)
  int nw;     // waves launched by the balanced split
  // Fused decode step (balanced split only): the split streams keys [.., ctx - 1) of the
  // cache and the tail adds the newest key ctx - 1 from k_new / v_new (B, Hkv, D rows), then
  // writes that row into the cache at slot_mapping[b] (skipped when outside the cache).
  int excl_last;
  const void* k_new;
  int64_t kn_sb, kn_sh;
  const void* v_new;
  int64_t vn_sb, vn_sh;
  const int32_t* slot_mapping;
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

// GP = query-head rows per KV group, padded (4 / 8 / 16).  kAligned: page_size is a
// multiple of the 32-key sub-block, so a sub-block lies in one page and each wave
// reads its (at most 8) page ids once, up front; otherwise every key looks its page
// up on its own.
template <typename T, int D, int GP, bool kAligned>
__global__ void __launch_bounds__(256, GP == 4 ? 2 : 1) polar_decode_split_kernel(DecodeArgs a) {
  constexpr bool kHalf = sizeof(T) == 2;
  constexpr int DCH = D / 8;        // lanes per key row in the PV pass (8 dims each)
  constexpr int KPI = 64 / DCH;     // keys per PV step
  constexpr int SUBK = 32;          // keys per sub-block (two 16-key MFMA tiles)
  constexpr int NT16 = SUBK / 16;   // 16-key tiles per sub-block
  constexpr int NIT = SUBK / KPI;   // PV steps per sub-block
  // A lane's 16-byte pieces of a q / K row: piece s of row quarter g holds elements
  // (4 s + g) * EP ...; the four quarters of one load instruction then cover 64
  // contiguous bytes of each key row (the dot product is order-free over dims).
  constexpr int EP = 16 / (int)sizeof(T);
  constexpr int KV = kHalf ? D / 32 : D / 16;  // 16-byte K loads per lane per 16-key tile
  constexpr int VV = kHalf ? 1 : 2;            // 16-byte V loads per lane per key
  __shared__ __attribute__((aligned(16))) float Ps[4][32][GP];
  __shared__ float Alpha[4][GP];
  __shared__ float Wst[4][GP][3];
  __shared__ __attribute__((aligned(16))) float Wacc[4][GP][D];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bhk = blockIdx.x, sp = blockIdx.y;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int ctx = a.ctx[b];
  int t0, t1;
  span_of(ctx, a.window, sp, t0, t1);
  if (t0 >= t1) return;  // uniform across the workgroup

  const int col = lane & 15, grp4 = lane >> 4;  // MFMA: key column, K-quarter / row group
  float n_cal = (float)ctx;
  if (a.window > 0) n_cal = fminf(n_cal, (float)a.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float logn = logf(n_cal);
  // temperature of query head `col` (one softplus per lane), shuffled to the rows
  // 4*grp4 + i this lane holds in the MFMA output layout
  const float c1_col =
      (1.f + softplus(a.len_gain_raw[hk * a.G + (col < a.G ? col : 0)]) * logn) * kLog2e *
      (1.f / sqrtf((float)D));
  float c1r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c1r[i] = __shfl(c1_col, (4 * grp4 + i) & 15, 64);

  // q operand (A of QK^T): row = head (lane & 15), quarter = lane >> 4
  u32x4 qa[kHalf ? D / 32 : 1];
  float qf[kHalf ? 1 : D / 4];
  {
    const int row = col;
    const bool ok = row < a.G;
    const T* qp = (const T*)a.q + b * a.q_sb + (int64_t)(hk * a.G + (ok ? row : 0)) * a.q_sh +
                  EP * grp4;
    if constexpr (kHalf) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) qa[s] = ok ? *(const u32x4*)(qp + 4 * EP * s) : u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int s4 = 0; s4 < D / 16; ++s4) {
        f32x4 x = ok ? *(const f32x4*)(qp + 4 * EP * s4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[4 * s4 + e] = x[e];
      }
    }
  }

  const T* kc = (const T*)a.kc;
  const T* vc = (const T*)a.vc;
  const int32_t* btb = a.bt + (int64_t)b * a.bt_sb;
  const int64_t row_elems = (int64_t)a.Hkv * D;
  // Element offset of key `pos` in the cache.  Pages outside the table are clamped to
  // page 0 (always a valid address) and reported through `ok`; callers zero them.
  auto key_off = [&](int pos, bool& ok) -> int64_t {
    const int lp = pos / a.page_size;
    int phys = (lp < a.max_pages) ? btb[lp] : -1;
    ok = phys >= 0 && phys < a.num_pages;
    if (!ok) phys = 0;
    return ((int64_t)phys * a.page_size + (pos - lp * a.page_size)) * row_elems + (int64_t)hk * D;
  };

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
  // this wave's share of the span, walked in 32-key sub-blocks
  const int w_lo = sp * kSplitTokens + kWaveTokens * wave;
  const int sb_beg = max(w_lo, t0 & ~(SUBK - 1));
  const int sb_end = min(w_lo + kWaveTokens, t1);
  // Aligned pages: lane j holds the physical page of sub-block w_lo + 32 j (-1 past
  // the context or the table), read out with v_readlane inside the loop, so no page
  // lookup there waits on memory (a vector load feeding an address would make the
  // wave drain every K/V load in flight at each sub-block).
  int wave_pages = -1;
  if constexpr (kAligned) {
    const int pos = w_lo + SUBK * lane;
    const int lp = pos / a.page_size;
    if (lane < kWaveTokens / SUBK && pos < t1 && lp < a.max_pages) wave_pages = btb[lp];
  }
  // Aligned pages are read with buffer loads: the page is the buffer (base and size
  // in scalar registers, size 0 for a page outside the pool so nothing is fetched),
  // a lane keeps one 32-bit offset for its row / columns, and the sub-block's row
  // within the page is a scalar offset.
  const uint32_t row_bytes = (uint32_t)row_elems * sizeof(T);
  const uint32_t page_bytes = (uint32_t)a.page_size * row_bytes;
  const uint32_t head_b = (uint32_t)(hk * D * sizeof(T));
  const uint32_t k_voff = col * row_bytes + head_b + (uint32_t)(EP * grp4 * sizeof(T));
  const uint32_t v_voff = kg * row_bytes + head_b + (uint32_t)(8 * dch * sizeof(T));
  const int np32 = (int)min(a.num_pages, (int64_t)0x7fffffff);
  auto sub_page = [&](int sb, bool& ok) -> int64_t {
    const int phys = __builtin_amdgcn_readlane(wave_pages, min((sb - w_lo) / SUBK, 63));
    ok = (phys >= 0) & (phys < np32);
    return ok ? (int64_t)phys * a.page_size * row_elems : 0;
  };

  // ---- K of one sub-block (16-key tiles: lane = key column x row quarter)
  bool kok[NT16];
  u32x4 kb[NT16][KV];
  auto load_k = [&](int sb) {
    if constexpr (kAligned) {
      bool pg;
      const int64_t pbase = sub_page(sb, pg);
      const auto rs = buffer_rsrc(kc + pbase, pg ? page_bytes : 0u);
      const uint32_t soff = (uint32_t)(sb % a.page_size) * row_bytes;
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        const int pos = sb + 16 * j + col;
        kok[j] = pg & (pos >= t0) & (pos < t1);
#pragma unroll
        for (int s = 0; s < KV; ++s)
          kb[j][s] = buffer_load16_nt(rs, k_voff + 64u * s, soff + 16u * j * row_bytes);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        const int pos = sb + 16 * j + col;
        bool pok;
        const int64_t off = key_off(pos, pok);
        kok[j] = pok && pos >= t0 && pos < t1;
        const T* kr = kc + off + EP * grp4;
#pragma unroll
        for (int s = 0; s < KV; ++s) kb[j][s] = *(const u32x4*)(kr + 4 * EP * s);
      }
    }
  };
  // ---- V of one sub-block (lane = 8 dims x keys kg, kg + KPI, ...)
  bool vok[NIT];
  u32x4 vb[NIT][VV];
  auto load_v = [&](int sb) {
    if constexpr (kAligned) {
      bool pg;
      const int64_t pbase = sub_page(sb, pg);
      const auto rs = buffer_rsrc(vc + pbase, pg ? page_bytes : 0u);
      const uint32_t soff = (uint32_t)(sb % a.page_size) * row_bytes;
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int pos = sb + it * KPI + kg;
        vok[it] = pg & (pos >= t0) & (pos < t1);
#pragma unroll
        for (int w = 0; w < VV; ++w)
          vb[it][w] = buffer_load16_nt(rs, v_voff + 16u * w, soff + (uint32_t)(it * KPI) * row_bytes);
      }
    } else {
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int pos = sb + it * KPI + kg;
        bool pok;
        const int64_t off = key_off(pos, pok);
        vok[it] = pok && pos >= t0 && pos < t1;
        const T* vr = vc + off + 8 * dch;
#pragma unroll
        for (int w = 0; w < VV; ++w) vb[it][w] = *(const u32x4*)(vr + 4 * w);
      }
    }
  };

  // K(sb + 32) is issued right after QK^T(sb) and V(sb + 32) right after PV(sb), so
  // each has a whole sub-block of work to arrive behind
  // (On aligned pages the loads are issued unconditionally: past the wave's range the
  // page id is -1, the buffer is empty and nothing is fetched, and the compiler sees
  // one fixed order of loads, so its waits stay partial.)
  if (kAligned || sb_beg < sb_end) {
    load_k(sb_beg);
    load_v(sb_beg);
  }
  for (int sb = sb_beg; sb < sb_end; sb += SUBK) {
    // ---- S = Q K^T over four 16-key tiles (rows = heads, columns = keys)
    f32x4 sc[NT16];
#pragma unroll
    for (int j = 0; j < NT16; ++j) {
      sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (kHalf) {
#pragma unroll
        for (int s = 0; s < KV; ++s) sc[j] = mfma16x16x32<T>(qa[s], kb[j][s], sc[j]);
      } else {
#pragma unroll
        for (int s4 = 0; s4 < KV; ++s4) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[4 * s4 + e], __uint_as_float(kb[j][s4][e]),
                                                         sc[j], 0, 0, 0);
        }
      }
    }
    bool kok_cur[NT16];
#pragma unroll
    for (int j = 0; j < NT16; ++j) kok_cur[j] = kok[j];
    const bool full = sb >= t0 && sb + SUBK <= t1 && vok[0] && vok[NIT - 1];
    if (kAligned || sb + SUBK < sb_end) load_k(sb + SUBK);  // in flight during the softmax and PV
    // ---- online softmax; rows = heads 4*grp4+i, column key = sb + 16 j + col
    float alpha_r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        sc[j][i] = kok_cur[j] ? sc[j][i] : -INFINITY;
        mx = fmaxf(mx, sc[j][i]);
      }
      mx = row16_max(mx);  // over the 16 key columns of the row
      const float m_new = fmaxf(m_run[i], mx * c1r[i]);
      const float alpha = __builtin_amdgcn_exp2f(m_run[i] - m_new);
      m_run[i] = m_new;
      float ls = 0.f, qs = 0.f;
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sc[j][i], c1r[i], -m_new));
        sc[j][i] = p;
        ls += p;
        qs = fmaf(p, p, qs);
      }
      l_part[i] = l_part[i] * alpha + ls;
      q2_part[i] = q2_part[i] * alpha * alpha + qs;
      alpha_r[i] = alpha;
    }
    if (4 * grp4 < GP) {
#pragma unroll
      for (int j = 0; j < NT16; ++j) *(f32x4*)&Ps[wave][16 * j + col][4 * grp4] = sc[j];
      if (col == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) Alpha[wave][4 * grp4 + i] = alpha_r[i];
      }
    }
    wave_sync();
    // ---- acc = acc * alpha + P V
    {
      float al[GP];
#pragma unroll
      for (int r = 0; r < GP; ++r) al[r] = Alpha[wave][r];
#pragma unroll
      for (int r = 0; r < GP; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] *= al[r];
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int kk = it * KPI + kg;
      float vv[8];
      if constexpr (kHalf) {
        unpack8(vb[it][0], vv, T{});
      } else {
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
          for (int e = 0; e < 4; ++e) vv[4 * w + e] = __uint_as_float(vb[it][w][e]);
      }
      if (!full) {  // masked rows (even NaN) never enter the sums
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[e] = vok[it] ? vv[e] : 0.f;
      }
#pragma unroll
      for (int r4 = 0; r4 < GP / 4; ++r4) {
        const f32x4 p4 = *(const f32x4*)&Ps[wave][kk][4 * r4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[4 * r4 + rr][e] = fmaf(p4[rr], vv[e], acc[4 * r4 + rr][e]);
      }
    }
    if (kAligned || sb + SUBK < sb_end) load_v(sb + SUBK);
    wave_sync();
  }

  // ---- reduce this wave: L, Q2 over the 16 key columns; acc over the key groups
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    l_part[i] = row16_sum(l_part[i]);
    q2_part[i] = row16_sum(q2_part[i]);
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

// One workgroup (256 threads) per (sequence, query head): combine the live spans.
// Pass 1 finds the common max M over the spans' running maxima (one span per
// thread, in parallel); pass 2 sums L, Q2 and the direction with factors
// 2^(m_i - M), D threads per span group so the span records are read in parallel.
template <typename T, int D>
__global__ void __launch_bounds__(256) polar_decode_merge_kernel(DecodeArgs a) {
  constexpr int NG = 256 / D;  // span groups
  __shared__ float red[4];
  __shared__ float s_part[NG][D];
  __shared__ float s_lq[NG][2];
  const int bh = blockIdx.x;
  const int b = bh / a.Hq, hq = bh % a.Hq;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ctx = a.ctx[b];
  const int lo = a.window > 0 ? max(ctx - a.window, 0) : 0;
  const int sp0 = lo / kSplitTokens;
  const int sp1 = min(ctx > lo ? (ctx + kSplitTokens - 1) / kSplitTokens : sp0, a.max_splits);
  const float* recs = a.ws + ((int64_t)b * a.Hq + hq) * a.max_splits * (D + 4);

  float M = kSentinel;
  for (int sp = sp0 + tid; sp < sp1; sp += 256) M = fmaxf(M, recs[(int64_t)sp * (D + 4)]);
  M = wave_max(M);
  if (lane == 0) red[wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));

  const int grp = tid / D, d = tid % D;
  float S = 0.f, L = 0.f, Q2 = 0.f;
#pragma unroll 16
  for (int sp = sp0 + grp; sp < sp1; sp += NG) {
    const float* rec = recs + (int64_t)sp * (D + 4);
    const float f = exp2f(rec[0] - M);
    S = fmaf(rec[4 + d], f, S);
    if (d == 0) {
      L = fmaf(rec[1], f, L);
      Q2 = fmaf(rec[2], f * f, Q2);
    }
  }
  s_part[grp][d] = S;
  if (d == 0) {
    s_lq[grp][0] = L;
    s_lq[grp][1] = Q2;
  }
  __syncthreads();
  // every thread stays to the last barrier; only the first D (one per head dim) finish
  const bool act = tid < D;
  S = 0.f;
  L = 0.f;
  Q2 = 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    S += s_part[g][d];
    L += s_lq[g][0];
    Q2 += s_lq[g][1];
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
  const float s = act ? S * al + pn * a.v_null[(int64_t)hq * D + d] : 0.f;
  const float ss_w = wave_sum(s * s);
  __syncthreads();  // red[] reused
  if (lane == 0) red[wave] = ss_w;
  __syncthreads();
  float ss = 0.f;
#pragma unroll
  for (int w = 0; w < D / 64; ++w) ss += red[w];
  const float inv = 1.f / fmaxf(sqrtf(ss), a.eps);
  if (act) ((T*)a.c)[((int64_t)b * a.Hq + hq) * D + d] = (T)(s * inv);
  if (tid == 0) {
    const float n_eff = L * L / fmaxf(Q2, 1e-30f);
    const float m_eff = n_eff * (L / fmaxf(Z, a.eps));
    const float beta = softplus(a.mag_beta_raw[hq]);
    ((T*)a.mag)[(int64_t)b * a.Hq + hq] = (T)tanhf(beta * log1pf(m_eff));
  }
}

// ---------------------------------------------------------------------------------------
// Length-balanced split (16-bit K/V, pages a multiple of 32 keys).
//
// The unit of work is one 32-key sub-block of one (sequence, KV head) pair, counted from
// the window start rounded down to 32.  All KV heads of a sequence have the same number
// of units, so the per-sequence prefix pre[b] orders the units as (b, head, sub-block).
// Every workgroup recomputes pre[] in LDS from context_lens (so the launch depends only
// on the shapes: graph capturable), and wave w of NW = min(waves launched, U) takes the
// contiguous range [w U / NW, (w + 1) U / NW): every wave streams the same number of keys
// (+-32) whatever the context lengths.  A wave keeps the online statistics of the pair it
// is in; when its range moves to the next pair it writes the partial (m, L, Q2, acc) as
// record w + sh (sh = b Hkv + h; injective over the pairs a wave touches, since the
// ranges are ordered) and starts afresh.  The merge combines the records of waves
// w_first(sh) .. w_last(sh).
constexpr int kBalWaves = 2048;     // at most this many waves (512 workgroups of 4)
constexpr int kBalMaxSeqs = 8192;   // sequences the in-LDS prefix holds

// Balanced-split workspace: the unit prefix pre[0 .. B] (written by workgroup 0 of the
// split, read by the merge) in a header of whole 256-byte blocks, then the records.
__host__ __device__ __forceinline__ int64_t bal_header_floats(int64_t B) {
  return ((B + 1) * 4 + 255) / 256 * 64;
}

// Units of one (sequence, KV head): keys [lo, ctx - excl) from the window start lo (of the
// full context) rounded down to 32.
__device__ __forceinline__ int bal_units(int ctx, int window, int excl) {
  const int lo = window > 0 ? max(ctx - window, 0) : 0;
  const int hi = ctx - excl;
  return hi > lo ? (hi - (lo & ~31) + 31) >> 5 : 0;
}

// Exclusive prefix over the sequences' unit counts into pre[0 .. B] (pre[B] = total);
// the whole workgroup takes part, and a barrier ends it.
__device__ void bal_prefix(const DecodeArgs& a, int* pre) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = (a.B + 255) / 256;
  const int i0 = min(tid * E, a.B), i1 = min(i0 + E, a.B);
  int sum = 0;
  for (int i = i0; i < i1; ++i) sum += bal_units(a.ctx[i], a.window, a.excl_last);
  int incl = sum;  // inclusive scan within the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  __shared__ int wave_tot[4];
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int v = 0; v < wave; ++v) base += wave_tot[v];
  int run = base + incl - sum;
  for (int i = i0; i < i1; ++i) {
    pre[i] = run;
    run += bal_units(a.ctx[i], a.window, a.excl_last);
  }
  if (tid == 255) pre[a.B] = base + incl;
  __syncthreads();
}

template <typename T, int D, int GP>
__global__ void __launch_bounds__(256, 2) polar_decode_balanced_kernel(DecodeArgs a) {
  static_assert(sizeof(T) == 2, "balanced split: 16-bit K/V");
  constexpr int DCH = D / 8;        // lanes per key row in the PV pass (8 dims each)
  constexpr int KPI = 64 / DCH;     // keys per PV step
  constexpr int SUBK = 32;          // keys per unit
  constexpr int NT16 = SUBK / 16;   // 16-key MFMA tiles per unit
  constexpr int NIT = SUBK / KPI;   // PV steps per unit
  constexpr int EP = 8;             // 16-bit elements per 16-byte piece
  constexpr int KV = D / 32;        // 16-byte K loads per lane per 16-key tile
  __shared__ int pre[kBalMaxSeqs + 1];
  __shared__ __attribute__((aligned(16))) float Ps[4][32][GP];
  __shared__ float Alpha[4][GP];
  // per wave, per unit of the current 63-unit chunk: pair, first key, physical page,
  // context length of the pair's sequence.  Read back as one uniform 16-byte LDS load,
  // whose wait (lgkmcnt) leaves the K / V loads in flight alone.
  __shared__ __attribute__((aligned(16))) int uinfo[4][64][4];

  bal_prefix(a, pre);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (blockIdx.x == 0) {  // publish the prefix for the merge
    int* hdr = (int*)a.ws;
    for (int i = tid; i <= a.B; i += 256) hdr[i] = pre[i];
  }
  const int U = a.Hkv * pre[a.B];
  const int NW = min(a.nw, U);
  const int w = blockIdx.x * 4 + wave;
  if (w >= NW) return;  // no barrier follows
  const int u_beg = (int)((int64_t)w * U / NW), u_end = (int)((int64_t)(w + 1) * U / NW);

  const int col = lane & 15, grp4 = lane >> 4;
  const int dch = lane % DCH, kg = lane / DCH;
  const T* kc = (const T*)a.kc;
  const T* vc = (const T*)a.vc;
  const uint32_t row_bytes = (uint32_t)a.Hkv * D * sizeof(T);
  const uint32_t page_bytes = (uint32_t)a.page_size * row_bytes;
  const uint32_t k_voff = col * row_bytes + (uint32_t)(EP * grp4 * sizeof(T));
  const uint32_t v_voff = kg * row_bytes + (uint32_t)(8 * dch * sizeof(T));
  const int np32 = (int)min(a.num_pages, (int64_t)0x7fffffff);
  const int64_t page_elems = (int64_t)a.page_size * a.Hkv * D;

  // per-pair state
  int cur = -1, cur_b = 0, t0 = 0, t1 = 0;
  float m_run[4], l_part[4], q2_part[4], c1r[4];
  float acc[GP][8];
  u32x4 qa[KV];

  auto setup = [&](int sh) {
    cur = sh;
    cur_b = sh / a.Hkv;
    const int hk = sh - cur_b * a.Hkv;
    const int ctx = __builtin_amdgcn_readfirstlane(a.ctx[cur_b]);
    t0 = a.window > 0 ? max(ctx - a.window, 0) : 0;
    t1 = ctx - a.excl_last;  // the fused step's tail adds key ctx - 1
    float n_cal = (float)ctx;
    if (a.window > 0) n_cal = fminf(n_cal, (float)a.window);
    const float logn = logf(fmaxf(n_cal, 1.f));
    const float c1_col = (1.f + softplus(a.len_gain_raw[hk * a.G + (col < a.G ? col : 0)]) * logn) *
                         kLog2e * (1.f / sqrtf((float)D));
#pragma unroll
    for (int i = 0; i < 4; ++i) c1r[i] = __shfl(c1_col, (4 * grp4 + i) & 15, 64);
    const bool ok = col < a.G;
    const T* qp = (const T*)a.q + cur_b * a.q_sb + (int64_t)(hk * a.G + (ok ? col : 0)) * a.q_sh + EP * grp4;
#pragma unroll
    for (int s = 0; s < KV; ++s) qa[s] = ok ? *(const u32x4*)(qp + 4 * EP * s) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_run[i] = kSentinel;
      l_part[i] = 0.f;
      q2_part[i] = 0.f;
    }
#pragma unroll
    for (int r = 0; r < GP; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
    // q and the parameters arrive before the run starts (once per pair): otherwise the
    // wait for them, the newest loads, would be merged into every iteration's wait for
    // its K and drain the V loads in flight.  A compiler-visible s_waitcnt vmcnt(0)
    // (expcnt / lgkmcnt fields at their maxima), so its wait bookkeeping sees q complete.
    __builtin_amdgcn_s_waitcnt(0x0F70);
  };
  // this pair's partial statistics -> record (w + sh), one row per query head of the group
  auto flush = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      l_part[i] = row16_sum(l_part[i]);
      q2_part[i] = row16_sum(q2_part[i]);
    }
#pragma unroll
    for (int r = 0; r < GP; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int m = DCH; m < 64; m <<= 1) acc[r][e] += __shfl_xor(acc[r][e], m, 64);
      }
    float* rec = a.ws + bal_header_floats(a.B) + (int64_t)(w + cur) * a.G * (D + 4);
    if (col == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * grp4 + i;
        if (r < a.G) {
          rec[(int64_t)r * (D + 4) + 0] = m_run[i];
          rec[(int64_t)r * (D + 4) + 1] = l_part[i];
          rec[(int64_t)r * (D + 4) + 2] = q2_part[i];
        }
      }
    }
    if (kg == 0) {
#pragma unroll
      for (int r = 0; r < GP; ++r) {
        if (r < a.G) {
          float* dst = rec + (int64_t)r * (D + 4) + 4 + 8 * dch;
          *(f32x4*)dst = f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
          *(f32x4*)(dst + 4) = f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
        }
      }
    }
  };

  // unit info of the chunk starting at unit c0, lane s -> unit c0 + s
  auto fill = [&](int c0) {
    const int u = c0 + lane;
    int info_sh = 0, info_pos = 0, info_pg = -1, info_ctx = 0;
    if (lane < 63 && u < u_end) {
      int lo = 0, hi = a.B - 1;  // last b with Hkv pre[b] <= u (it has units; see above)
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.Hkv * pre[mid] <= u) lo = mid; else hi = mid - 1;
      }
      const int b = lo;
      const int nb = pre[b + 1] - pre[b];
      const int rr = u - a.Hkv * pre[b];
      const int hk = rr / nb, j = rr - hk * nb;
      const int ctx = a.ctx[b];
      const int lw = a.window > 0 ? max(ctx - a.window, 0) : 0;
      info_ctx = ctx;
      info_sh = b * a.Hkv + hk;
      info_pos = (lw & ~31) + SUBK * j;
      const int lp = info_pos / a.page_size;
      info_pg = lp < a.max_pages ? a.bt[(int64_t)b * a.bt_sb + lp] : -1;
    }
    *(int4*)&uinfo[wave][lane][0] = make_int4(info_sh, info_pos, info_pg, info_ctx);
    wave_sync();
  };
  auto unit_info = [&](int s) {   // (pair, first key, page, ctx) of unit s, in scalar registers
    const int4 v = *(const int4*)&uinfo[wave][s][0];
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                     __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
  };

  bool kok[NT16];
  u32x4 kb[NT16][KV];
  bool vok[NIT];
  u32x4 vb[NIT];
  // unit s: buffer over its page (empty for a page outside the pool), the scalar offset
  // of its first row plus the pair's head, and the key bounds [lw, ctx) of its sequence
  // (ctx excluding the newest key when the fused step's tail adds it)
  auto unit_rsrc = [&](int s, const T* base, int& pos, int& lw, int& ctx, uint32_t& soff, bool& pg) {
    const int4 ui = unit_info(s);
    const int sh = ui.x;
    pos = ui.y;
    ctx = ui.w;
    lw = a.window > 0 ? max(ctx - a.window, 0) : 0;
    ctx -= a.excl_last;
    const int phys = ui.z;
    pg = (phys >= 0) & (phys < np32);
    const int hk = sh % a.Hkv;
    soff = (uint32_t)(pos % a.page_size) * row_bytes + (uint32_t)(hk * D * sizeof(T));
    return buffer_rsrc(base + (pg ? (int64_t)phys * page_elems : 0), pg ? page_bytes : 0u);
  };
  // K / V of unit s; keys outside [lw, ctx) of the unit's own sequence are flagged (one
  // lane value against scalar bounds; constant offsets ride in the scalar offset)
  auto load_k = [&](int s) {
    int pos, lw, ctx;
    uint32_t soff;
    bool pg;
    const auto rs = unit_rsrc(s, kc, pos, lw, ctx, soff, pg);
#pragma unroll
    for (int j = 0; j < NT16; ++j) {
      const int rel = pos + 16 * j;
      kok[j] = pg & (col >= lw - rel) & (col < ctx - rel);
#pragma unroll
      for (int q = 0; q < KV; ++q) kb[j][q] = buffer_load16_nt(rs, k_voff, soff + 16u * j * row_bytes + 64u * q);
    }
  };
  auto load_v = [&](int s) {
    int pos, lw, ctx;
    uint32_t soff;
    bool pg;
    const auto rs = unit_rsrc(s, vc, pos, lw, ctx, soff, pg);
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int rel = pos + it * KPI;
      vok[it] = pg & (kg >= lw - rel) & (kg < ctx - rel);
      vb[it] = buffer_load16_nt(rs, v_voff, soff + (uint32_t)(it * KPI) * row_bytes);
    }
  };

  for (int c0 = u_beg; c0 < u_end; c0 += 63) {
    fill(c0);
    const int n = min(63, u_end - c0);
    load_k(0);
    load_v(0);
    int s = 0;
    while (s < n) {
      // a run of units of one pair: its statistics start afresh unless the run
      // continues the pair the previous chunk ended in
      const int run_sh = unit_info(s).x;
      if (run_sh != cur) {
        if (cur >= 0) flush();
        setup(run_sh);
      }
      for (; s < n && unit_info(s).x == run_sh; ++s) {
      const int sb = unit_info(s).y;
      // ---- S = Q K^T (rows = query heads of the group, columns = keys)
      f32x4 sc[NT16];
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < KV; ++q) sc[j] = mfma16x16x32<T>(qa[q], kb[j][q], sc[j]);
      }
      bool kok_cur[NT16];
#pragma unroll
      for (int j = 0; j < NT16; ++j) kok_cur[j] = kok[j];
      const bool full = sb >= t0 && sb + SUBK <= t1 && vok[0] && vok[NIT - 1];
      // K of unit s + 1 in flight during the softmax and PV.  Issued unconditionally: past
      // the chunk's last unit the unit info holds page -1, an empty buffer that fetches
      // nothing, and the compiler sees one fixed order of loads, so its waits stay partial.
      load_k(s + 1);
      float alpha_r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < NT16; ++j) {
          sc[j][i] = kok_cur[j] ? sc[j][i] : -INFINITY;
          mx = fmaxf(mx, sc[j][i]);
        }
        mx = row16_max(mx);  // over the 16 key columns of the row
        const float m_new = fmaxf(m_run[i], mx * c1r[i]);
        const float alpha = __builtin_amdgcn_exp2f(m_run[i] - m_new);
        m_run[i] = m_new;
        float ls = 0.f, qs = 0.f;
#pragma unroll
        for (int j = 0; j < NT16; ++j) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(sc[j][i], c1r[i], -m_new));
          sc[j][i] = pv;
          ls += pv;
          qs = fmaf(pv, pv, qs);
        }
        l_part[i] = l_part[i] * alpha + ls;
        q2_part[i] = q2_part[i] * alpha * alpha + qs;
        alpha_r[i] = alpha;
      }
      if (4 * grp4 < GP) {
#pragma unroll
        for (int j = 0; j < NT16; ++j) *(f32x4*)&Ps[wave][16 * j + col][4 * grp4] = sc[j];
        if (col == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) Alpha[wave][4 * grp4 + i] = alpha_r[i];
        }
      }
      wave_sync();
      {
        float al[GP];
#pragma unroll
        for (int r = 0; r < GP; ++r) al[r] = Alpha[wave][r];
#pragma unroll
        for (int r = 0; r < GP; ++r)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r][e] *= al[r];
      }
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int kk = it * KPI + kg;
        float vv[8];
        unpack8(vb[it], vv, T{});
        if (!full) {  // masked rows (even NaN) never enter the sums
#pragma unroll
          for (int e = 0; e < 8; ++e) vv[e] = vok[it] ? vv[e] : 0.f;
        }
#pragma unroll
        for (int r4 = 0; r4 < GP / 4; ++r4) {
          const f32x4 p4 = *(const f32x4*)&Ps[wave][kk][4 * r4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[4 * r4 + rr][e] = fmaf(p4[rr], vv[e], acc[4 * r4 + rr][e]);
        }
      }
      load_v(s + 1);
      wave_sync();
      }
    }
  }
  if (cur >= 0) flush();
}

// One workgroup (256 threads) per (sequence, query head): combine the records of the
// waves that streamed its pair (sh = b Hkv + h) in one pass -- each thread group keeps a
// running max and rescales as it goes -- then fold the null sink.  The unit prefix comes
// from the workspace header the split wrote.  In the fused decode step (excl_last) the
// newest key, ctx - 1, joins as one more partial (score from q . k_new, weight 1, value
// v_new), and the first query head of each KV group writes the k_new / v_new row into the
// cache at slot_mapping[b].
template <typename T, int D>
__device__ __forceinline__ void bal_merge_block(const DecodeArgs& a, int bh) {
  constexpr int NG = 256 / D;
  __shared__ float red[4];
  __shared__ float s_part[NG][D];
  __shared__ float s_mlq[NG][3];
  const int b = bh / a.Hq, hq = bh % a.Hq;
  const int hk = hq / a.G, r = hq - hk * a.G;
  const int sh = b * a.Hkv + hk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int* hdr = (const int*)a.ws;
  // every input of the epilogue is read up front, beside the header and the records, so
  // the workgroup waits on memory once
  const float lg_raw = a.len_gain_raw[hq], nbase = a.null_base[hq];
  const float ns_raw = a.null_slope_raw[hq], mb_raw = a.mag_beta_raw[hq];
  const float vnull = a.v_null[(int64_t)hq * D + (tid % D)];
  const int ctx = a.ctx[b];
  const bool add_new = a.excl_last && ctx >= 1;
  float qk = 0.f, vnew = 0.f;
  if (a.excl_last) {
    const int d = tid % D;
    const T* kn = (const T*)a.k_new + b * a.kn_sb + hk * a.kn_sh;
    const T* vn = (const T*)a.v_new + b * a.vn_sb + hk * a.vn_sh;
    if (tid < D) qk = to_f32(((const T*)a.q)[b * a.q_sb + hq * a.q_sh + d]) * to_f32(kn[d]);
    vnew = to_f32(vn[d]);
    if (r == 0 && tid < 2 * D / 8) {  // the cache row: 16 bytes per thread, K then V
      const int64_t slot = a.slot_mapping[b];
      if (slot >= 0 && slot < a.num_pages * (int64_t)a.page_size) {
        const bool is_v = tid >= D / 8;
        const int e = 8 * (tid % (D / 8));
        const T* src = (is_v ? vn : kn) + e;
        T* dst = (T*)(is_v ? a.vc : a.kc) + (slot * a.Hkv + hk) * D + e;
        *(u32x4*)dst = *(const u32x4*)src;
      }
    }
  }
  const int pb = hdr[b], nb = hdr[b + 1] - pb;
  const int U = a.Hkv * hdr[a.B];
  const int NW = min(a.nw, U);
  int w0 = 0, w1 = -1;  // the waves that own this pair's units (none without keys)
  if (nb > 0) {
    const int64_t x0 = (int64_t)a.Hkv * pb + (int64_t)hk * nb;
    w0 = (int)(((x0 + 1) * NW - 1) / U);
    w1 = (int)(((x0 + nb) * NW - 1) / U);
  }
  const float* recs = a.ws + bal_header_floats(a.B);
  const int grp = tid / D, d = tid % D;
  float M = kSentinel, S = 0.f, L = 0.f, Q2 = 0.f;
#pragma unroll 4
  for (int wv = w0 + grp; wv <= w1; wv += NG) {
    const float* rc = recs + ((int64_t)(wv + sh) * a.G + r) * (D + 4);
    const float mi = rc[0];
    const float mn = fmaxf(M, mi);
    const float fo = exp2f(M - mn), fi = exp2f(mi - mn);
    S = S * fo + rc[4 + d] * fi;
    L = L * fo + rc[1] * fi;
    Q2 = Q2 * fo * fo + rc[2] * fi * fi;
    M = mn;
  }
  s_part[grp][d] = S;
  if (d == 0) {
    s_mlq[grp][0] = M;
    s_mlq[grp][1] = L;
    s_mlq[grp][2] = Q2;
  }
  if (a.excl_last) {  // q . k_new over the head dims
    const float w = wave_sum(qk);
    if (lane == 0) red[wave] = w;
  }
  __syncthreads();
  float n_cal = (float)ctx;
  if (a.window > 0) n_cal = fminf(n_cal, (float)a.window);
  n_cal = fmaxf(n_cal, 1.f);
  const float temp = 1.f + softplus(lg_raw) * logf(n_cal);
  const bool act = tid < D;
  M = kSentinel;
#pragma unroll
  for (int g = 0; g < NG; ++g) M = fmaxf(M, s_mlq[g][0]);
  float m_new = kSentinel;
  if (add_new) {
    float sdot = 0.f;
#pragma unroll
    for (int v = 0; v < D / 64; ++v) sdot += red[v];
    m_new = sdot * (temp * kLog2e * (1.f / sqrtf((float)D)));
    M = fmaxf(M, m_new);
  }
  S = 0.f;
  L = 0.f;
  Q2 = 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const float f = exp2f(s_mlq[g][0] - M);
    S += s_part[g][d] * f;
    L += s_mlq[g][1] * f;
    Q2 += s_mlq[g][2] * f * f;
  }
  if (add_new) {  // the newest key: p = 2^(m_new - M), value v_new
    const float f = exp2f(m_new - M);
    S += vnew * f;
    L += f;
    Q2 += f * f;
  }
  const float nullv = nbase + softplus(ns_raw) * sqrtf(logf(n_cal + 1.f));
  const float an2 = temp * nullv * kLog2e;
  const float mn = fmaxf(M, an2);
  const float al = exp2f(M - mn);
  L *= al;
  Q2 *= al * al;
  const float pn = exp2f(an2 - mn);
  const float Z = L + pn;
  const float sv = act ? S * al + pn * vnull : 0.f;
  const float ss_w = wave_sum(sv * sv);
  __syncthreads();  // red is reused
  if (lane == 0) red[wave] = ss_w;
  __syncthreads();
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < D / 64; ++v) ss += red[v];
  const float inv = 1.f / fmaxf(sqrtf(ss), a.eps);
  if (act) ((T*)a.c)[((int64_t)b * a.Hq + hq) * D + d] = (T)(sv * inv);
  if (tid == 0) {
    const float n_eff = L * L / fmaxf(Q2, 1e-30f);
    const float m_eff = n_eff * (L / fmaxf(Z, a.eps));
    const float beta = softplus(mb_raw);
    ((T*)a.mag)[(int64_t)b * a.Hq + hq] = (T)tanhf(beta * log1pf(m_eff));
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(256) polar_decode_balanced_merge_kernel(DecodeArgs a) {
  bal_merge_block<T, D>(a, blockIdx.x);
}

// The fused decode step's tail: the merge workgroups (with the newest key and the cache
// row write) first, then the gated-delta memory step's workgroups, in one launch -- the
// merge is latency bound, the memory step bandwidth bound, so they overlap.
template <typename T, int D>
__global__ void __launch_bounds__(256) global_decode_tail_kernel(DecodeArgs a, GdnStepArgs m) {
  const int nm = a.B * a.Hq;
  if ((int)blockIdx.x < nm) {
    bal_merge_block<T, D>(a, blockIdx.x);
  } else {
    const int i = (int)blockIdx.x - nm;
    gdn_step_block<T, D>(m, i / gdn_step_slabs<D>(), i % gdn_step_slabs<D>());
  }
}

static int max_splits_for(int64_t max_pages, int64_t page_size) {
  return (int)((max_pages * page_size + kSplitTokens - 1) / kSplitTokens);
}

// The balanced split serves 16-bit caches whose pages hold whole 32-key units; the span
// split serves the rest (fp32, other page sizes, more sequences than the LDS prefix holds).
static bool use_balanced(int dtype, int64_t page_size, int64_t B) {
  return (dtype == ATMA_BF16 || dtype == ATMA_F16) && page_size % 32 == 0 && B <= kBalMaxSeqs;
}

// Waves the balanced split launches: enough for every unit a shape can hold, at most
// kBalWaves (a function of the shapes only, so a captured graph stays valid).
static int balanced_waves(int64_t B, int64_t Hkv, int64_t max_pages, int64_t page_size) {
  const int64_t units = B * Hkv * ((max_pages * page_size + 31) / 32);
  return (int)(4 * std::min<int64_t>(kBalWaves / 4, (units + 3) / 4));
}

template <typename T, int D, int GP>
static int launch_decode(DecodeArgs a, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {
    if (a.nw > 0) {  // balanced split (chosen by the host; nw = waves launched)
      polar_decode_balanced_kernel<T, D, GP><<<dim3((unsigned)(a.nw / 4)), dim3(256), 0, s>>>(a);
      int rc = check_launch("polar_attention_decode(balanced split)");
      if (rc) return rc;
      polar_decode_balanced_merge_kernel<T, D><<<dim3((unsigned)(a.B * a.Hq)), dim3(256), 0, s>>>(a);
      return check_launch("polar_attention_decode(balanced merge)");
    }
  }
  if (a.max_splits > 0) {
    const dim3 grid((unsigned)(a.B * a.Hkv), (unsigned)a.max_splits);
    if (a.page_size % 32 == 0)
      polar_decode_split_kernel<T, D, GP, true><<<grid, dim3(256), 0, s>>>(a);
    else
      polar_decode_split_kernel<T, D, GP, false><<<grid, dim3(256), 0, s>>>(a);
    int rc = check_launch("polar_attention_decode(split)");
    if (rc) return rc;
  }
  polar_decode_merge_kernel<T, D><<<dim3((unsigned)(a.B * a.Hq)), dim3(256), 0, s>>>(a);
  return check_launch("polar_attention_decode(merge)");
}

template <typename T, int D>
static int dispatch_gp(DecodeArgs a, hipStream_t s) {
  if (a.G <= 4) return launch_decode<T, D, 4>(a, s);
  if (a.G <= 8) return launch_decode<T, D, 8>(a, s);
  return launch_decode<T, D, 16>(a, s);
}

}  // namespace atma

extern "C" size_t atma_polar_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_pages,
                                                    int64_t page_size, int64_t d, int dtype) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || max_pages <= 0 || page_size <= 0 || d <= 0) return 0;
  if (atma::use_balanced(dtype, page_size, B)) {
    // one (m, L, Q2, pad, acc[d]) row per query head of each (wave, pair) record
    const int64_t nw = atma::balanced_waves(B, Hkv, max_pages, page_size);
    return (size_t)(atma::bal_header_floats(B) + (nw + B * Hkv) * (Hq / Hkv) * (d + 4)) * sizeof(float);
  }
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
  if (max_pages > 0 && (!k_cache || !v_cache || !block_tables || num_pages <= 0))
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: empty or null cache");
  const int es = dtype_size(dtype);
  if (!es) return set_error(ATMA_ERR_INVALID, "polar_attention_decode: unknown dtype %d", dtype);
  if ((uintptr_t)q % 16 || (q_sb * es) % 16 || (q_sh * es) % 16 || (uintptr_t)k_cache % 16 ||
      (uintptr_t)v_cache % 16)
    return set_error(ATMA_ERR_INVALID, "polar_attention_decode: tensors must be 16-byte aligned");
  const size_t need = atma_polar_decode_workspace_bytes(B, Hq, Hkv, max_pages, page_size, d, dtype);
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
  a.nw = (max_pages > 0 && use_balanced(dtype, page_size, B)) ? balanced_waves(B, Hkv, max_pages, page_size) : 0;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_BF16: return d == 128 ? dispatch_gp<bf16, 128>(a, s) : dispatch_gp<bf16, 64>(a, s);
    case ATMA_F16: return d == 128 ? dispatch_gp<f16, 128>(a, s) : dispatch_gp<f16, 64>(a, s);
    default: return d == 128 ? dispatch_gp<float, 128>(a, s) : dispatch_gp<float, 64>(a, s);
  }
}

// ---------------------------------------------------------------------------------------
// Fused decode step of the global layer: store_kvcache + polar_attention_decode +
// gated_delta_decode_step in two launches (the balanced split over the cached keys, then
// one tail launch: merge with the newest key taken from k_new / v_new, the cache row
// write, and the memory step).  Same results as the three calls in that order when
// slot_mapping[b] is the cache slot of position context_lens[b] - 1 (the engine's
// invariant); a row whose slot is -1 is not written and still attends k_new / v_new as
// its newest key.
namespace atma {

template <typename T, int D>
static int launch_global_step(DecodeArgs a, GdnStepArgs m, hipStream_t s) {
  const int GP = a.G <= 4 ? 4 : a.G <= 8 ? 8 : 16;
  if (GP == 4) polar_decode_balanced_kernel<T, D, 4><<<dim3((unsigned)(a.nw / 4)), dim3(256), 0, s>>>(a);
  else if (GP == 8) polar_decode_balanced_kernel<T, D, 8><<<dim3((unsigned)(a.nw / 4)), dim3(256), 0, s>>>(a);
  else polar_decode_balanced_kernel<T, D, 16><<<dim3((unsigned)(a.nw / 4)), dim3(256), 0, s>>>(a);
  int rc = check_launch("global_decode_step(split)");
  if (rc) return rc;
  const unsigned grid = (unsigned)(a.B * a.Hq + a.B * m.H * gdn_step_slabs<D>());
  global_decode_tail_kernel<T, D><<<dim3(grid), dim3(256), 0, s>>>(a, m);
  return check_launch("global_decode_step(tail)");
}

}  // namespace atma

extern "C" int atma_global_decode_step_supported(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_pages,
                                                 int64_t page_size, int64_t d, int dtype) {
  return B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16 && (d == 64 || d == 128) &&
         max_pages > 0 && atma::use_balanced(dtype, page_size, B);
}

extern "C" int atma_global_decode_step(
    const void* q, int64_t q_sb, int64_t q_sh, const void* k_new, int64_t kn_sb, int64_t kn_sh,
    const void* v_new, int64_t vn_sb, int64_t vn_sh, void* k_cache, void* v_cache, int64_t num_pages,
    int64_t page_size, int64_t Hkv, const int32_t* slot_mapping, const int32_t* block_tables,
    int64_t bt_sb, int64_t max_pages, const int32_t* context_lens, const float* v_null,
    const float* null_base, const float* null_slope_raw, const float* len_gain_raw,
    const float* mag_beta_raw, void* c, void* mag, const float* gamma, const float* beta,
    float* state_table, int64_t max_seqs, const int64_t* slots, float* r, int64_t B, int64_t Hq,
    int64_t d, int dtype, int64_t window, float eps, float mem_eps, void* workspace,
    size_t workspace_bytes, void* stream) {
  using namespace atma;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || page_size <= 0 || max_pages < 0 || num_pages < 0 || max_seqs < 0)
    return set_error(ATMA_ERR_INVALID, "global_decode_step: bad sizes");
  if (B == 0) return ATMA_OK;
  if (!atma_global_decode_step_supported(B, Hq, Hkv, max_pages, page_size, d, dtype))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "global_decode_step: 16-bit caches with pages of whole 32-key units, a page "
                     "table, head_dim 64 / 128, groups <= 16 and at most %d sequences", kBalMaxSeqs);
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !slot_mapping || !block_tables ||
      !context_lens || !v_null || !null_base || !null_slope_raw || !len_gain_raw || !mag_beta_raw ||
      !c || !mag || !gamma || !beta || !state_table || !slots || !r || num_pages <= 0)
    return set_error(ATMA_ERR_INVALID, "global_decode_step: null pointer or empty cache");
  const int es = 2;
  auto al16 = [&](const void* p, int64_t s1, int64_t s2) {
    return (uintptr_t)p % 16 == 0 && (s1 * es) % 16 == 0 && (s2 * es) % 16 == 0;
  };
  if (!al16(q, q_sb, q_sh) || !al16(k_new, kn_sb, kn_sh) || !al16(v_new, vn_sb, vn_sh) ||
      (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16)
    return set_error(ATMA_ERR_INVALID, "global_decode_step: tensors must be 16-byte aligned rows");
  const size_t need = atma_polar_decode_workspace_bytes(B, Hq, Hkv, max_pages, page_size, d, dtype);
  if (!workspace || workspace_bytes < need)
    return set_error(ATMA_ERR_WORKSPACE, "global_decode_step: workspace %zu < %zu bytes",
                     workspace_bytes, need);
  if (max_pages * page_size > (1ll << 30) || B * Hkv > 0x7fffffffll || B * Hq > 0x7fffffffll)
    return set_error(ATMA_ERR_INVALID, "global_decode_step: sizes too large");
  DecodeArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.kc = k_cache; a.vc = v_cache;
  a.num_pages = num_pages; a.page_size = (int)page_size; a.Hkv = (int)Hkv;
  a.bt = block_tables; a.bt_sb = bt_sb; a.max_pages = (int)max_pages; a.ctx = context_lens;
  a.v_null = v_null; a.null_base = null_base; a.null_slope_raw = null_slope_raw;
  a.len_gain_raw = len_gain_raw; a.mag_beta_raw = mag_beta_raw;
  a.c = c; a.mag = mag; a.B = (int)B; a.Hq = (int)Hq; a.G = (int)(Hq / Hkv);
  a.window = window > 0 ? (int)window : 0; a.eps = eps;
  a.ws = (float*)workspace;
  a.nw = balanced_waves(B, Hkv, max_pages, page_size);
  a.excl_last = 1;
  a.k_new = k_new; a.kn_sb = kn_sb; a.kn_sh = kn_sh;
  a.v_new = v_new; a.vn_sb = vn_sb; a.vn_sh = vn_sh;
  a.slot_mapping = slot_mapping;
  GdnStepArgs m{q, q_sb, q_sh, k_new, kn_sb, kn_sh, v_new, vn_sb, vn_sh, gamma, beta, state_table,
                max_seqs, slots, r, (int)Hq, (int)(Hq / Hkv), mem_eps};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16)
    return d == 128 ? launch_global_step<bf16, 128>(a, m, s) : launch_global_step<bf16, 64>(a, m, s);
  return d == 128 ? launch_global_step<f16, 128>(a, m, s) : launch_global_step<f16, 64>(a, m, s);
}

// ---------------------------------------------------------------------------------------
// No-allocation variant.  The split records live in a file-scope device array instead of
// a caller workspace.  Each GPU holds its own copy of the array (at its own address) from
// the library's load until the process ends; the host keeps that address per device,
// looked up once with hipGetSymbolAddress on the entry point's first call on the device
// (which may be inside a stream capture: the lookup runs in relaxed capture mode).
// Calls that overlap on one GPU share the array and race; nothing in it needs to start at
// zero (every record the merge reads is written by the split pass of the same call).
namespace atma {
namespace {
constexpr size_t kDecodeScratchBytes = size_t(32) << 20;
__device__ __align__(256) unsigned char decode_scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int decode_scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(ATMA_ERR_HIP, "polar_attention_decode_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    // The first call may come while the caller's stream is being captured into a graph.
    // The lookup is no stream work; relaxed capture mode lets it run there, and the
    // thread's own mode is put back whatever the lookup returns.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t em = hipThreadExchangeStreamCaptureMode(&mode);
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(decode_scratch));
    if (em == hipSuccess) hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || !ptr)
      return set_error(ATMA_ERR_HIP, "polar_attention_decode_noalloc: hipGetSymbolAddress: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ATMA_OK;
}
}  // namespace
}  // namespace atma

extern "C" size_t atma_polar_decode_noalloc_max_bytes(void) { return atma::kDecodeScratchBytes; }

extern "C" int atma_polar_attention_decode_noalloc(
    const void* q, int64_t q_sb, int64_t q_sh, const void* k_cache, const void* v_cache,
    int64_t num_pages, int64_t page_size, int64_t Hkv, const int32_t* block_tables, int64_t bt_sb,
    int64_t max_pages, const int32_t* context_lens, const float* v_null, const float* null_base,
    const float* null_slope_raw, const float* len_gain_raw, const float* mag_beta_raw, void* c,
    void* mag, int64_t B, int64_t Hq, int64_t d, int dtype, int64_t window, float eps, void* stream) {
  using namespace atma;
  const size_t need = atma_polar_decode_workspace_bytes(B, Hq, Hkv, max_pages, page_size, d, dtype);
  if (need > kDecodeScratchBytes)
    return set_error(ATMA_ERR_WORKSPACE,
                     "polar_attention_decode_noalloc: this launch needs %zu bytes of split records, "
                     "above the fixed scratch maximum of %zu bytes (use atma_polar_attention_decode "
                     "with a workspace)", need, kDecodeScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = decode_scratch_ptr(&ws);
    if (rc) return rc;
  }
  return atma_polar_attention_decode(q, q_sb, q_sh, k_cache, v_cache, num_pages, page_size, Hkv,
                                     block_tables, bt_sb, max_pages, context_lens, v_null, null_base,
                                     null_slope_raw, len_gain_raw, mag_beta_raw, c, mag, B, Hq, d, dtype,
                                     window, eps, ws, need > 0 ? kDecodeScratchBytes : 0, stream);
}
