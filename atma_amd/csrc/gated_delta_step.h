// Gated-delta decode step on one workgroup's slab, shared by the standalone step kernel
// and the fused decode-step tail.
#pragma once

#include "common.h"

namespace atma {

struct GdnStepArgs {
  const void* q;
  int64_t q_sb, q_sh;
  const void* k;
  int64_t k_sb, k_sh;
  const void* v;
  int64_t v_sb, v_sh;
  const float* gamma;
  const float* beta;
  float* state;
  int64_t max_seqs;
  const int64_t* slots;
  float* r;
  int H, G;
  float eps;
};

// Workgroups of one step launch: (sequence * head) x 64-column slabs of V.
template <int D>
constexpr int gdn_step_slabs() { return D / 64; }

// One workgroup (256 threads) of the step: sequence-head bh, V columns
// 64 col_block .. + 63.
template <typename T, int D>
__device__ __forceinline__ void gdn_step_block(const GdnStepArgs& a, int bh, int col_block) {
  constexpr int VC = 64;            // state columns per workgroup
  constexpr int RPT = D / 16;       // state rows per thread
  __shared__ float s_q[D], s_k[D], s_v[VC], s_u[VC];
  __shared__ float s_red[16][VC + 4];
  __shared__ float s_norm[2];

  const int H = a.H, G = a.G;
  const int b = bh / H, h = bh % H;
  const int col0 = col_block * VC;
  const T* q = (const T*)a.q;
  const T* k = (const T*)a.k;
  const T* v = (const T*)a.v;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;

  // the slot, the gates and this thread's state rows are read first, so their latency
  // overlaps the operand loads and the norms (one wait on memory)
  const int64_t slot = a.slots[b];
  const bool ok = slot >= 0 && slot < a.max_seqs;
  const int cg = tid & 15;   // float4 column group
  const int rg = tid >> 4;   // row group
  float* base = a.state + ((ok ? slot : 0) * H + h) * (int64_t)D * D + col0 + cg * 4;
  const float g = a.gamma[b * H + h];
  const float bt = a.beta[b * H + h];
  f32x4 sd[RPT];
  if (ok) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) sd[j] = *(const f32x4*)(base + (int64_t)(rg + 16 * j) * D);
  }

  if (tid < D) {
    s_q[tid] = to_f32(q[b * a.q_sb + h * a.q_sh + tid]);
    s_k[tid] = to_f32(k[b * a.k_sb + (h / G) * a.k_sh + tid]);
  }
  if (tid < VC) s_v[tid] = to_f32(v[b * a.v_sb + (h / G) * a.v_sh + col0 + tid]);
  __syncthreads();
  if (wave < 2) {  // wave 0: |q|^2, wave 1: |k|^2
    const float* src = wave == 0 ? s_q : s_k;
    float acc = 0.f;
    for (int i = lane; i < D; i += 64) acc += src[i] * src[i];
    acc = wave_sum(acc);
    if (lane == 0) s_norm[wave] = 1.f / fmaxf(sqrtf(acc), a.eps);
  }
  __syncthreads();
  const float inv_q = s_norm[0], inv_k = s_norm[1];

  f32x4 pred = {0.f, 0.f, 0.f, 0.f};
  if (ok) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + 16 * j;
      sd[j] = g * sd[j];
      pred += (s_k[row] * inv_k) * sd[j];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) s_red[rg][cg * 4 + e] = pred[e];
  __syncthreads();
  if (tid < VC) {
    float p = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) p += s_red[i][tid];
    s_u[tid] = bt * (s_v[tid] - p);
  }
  __syncthreads();
  f32x4 u = *(const f32x4*)(s_u + cg * 4);
  f32x4 racc = {0.f, 0.f, 0.f, 0.f};
  if (ok) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + 16 * j;
      f32x4 sn = sd[j] + (s_k[row] * inv_k) * u;
      *(f32x4*)(base + (int64_t)row * D) = sn;
      racc += (s_q[row] * inv_q) * sn;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) s_red[rg][cg * 4 + e] = racc[e];
  __syncthreads();
  if (tid < VC) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += s_red[i][tid];
    a.r[((int64_t)b * H + h) * D + col0 + tid] = ok ? acc : __builtin_nanf("");
  }
}

}  // namespace atma
