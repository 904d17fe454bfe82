// Shared declarations of the chunked gated-delta prefill (fp32 VALU path and the
// 16-bit MFMA path).
#pragma once

#include "common.h"

namespace atma {

constexpr int kChunk = 64;

struct GdnArgs {
  const void* q;
  int64_t q_sb, q_st, q_sh;
  const void* k;
  int64_t k_sb, k_st, k_sh;
  const void* v;
  int64_t v_sb, v_st, v_sh;
  const float* g;
  const float* beta;
  const float* s0;
  float* s_out;
  void* o;
  int B, T, H, NC;
  int G;  // query heads per k / v head (k, v carry H / G heads)
  float scale;
  int l2norm;
  int gate_logits;  // g, beta hold raw logits: the activations below are applied on load
  float g_bias, b_bias;
  void* ws;
  int* start_flag;  // optional: the scan's first workgroup stores start_epoch here on entry
  int start_epoch;
};

// Start signal of the recurrence kernel.  The scan is latency-bound and needs a whole CU
// per workgroup (its LDS), so a long prefill overlaps it with Polar attention on another
// stream only if the scan's workgroups are resident before Polar's fill the GPU: the
// caller orders the two launches with atma_wait_start_flag on Polar's stream.
__device__ __forceinline__ void gdn_signal_start(const GdnArgs& a) {
  if (a.start_flag && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.start_flag, a.start_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The memory branch's gate activations (TitansMemory, model/blocks.py:426-490), shared by
// the stand-alone gate kernel and the prefill's fused load so both give the same bits:
// log-decay logsigmoid(z + bias) = min(x, 0) - log1p(exp(-|x|)) (stable for either sign)
// and write strength sigmoid(z + bias).
__device__ __forceinline__ float gdn_log_decay(float z, float bias) {
  const float x = z + bias;
  return fminf(x, 0.f) - log1pf(expf(-fabsf(x)));
}
__device__ __forceinline__ float gdn_write_strength(float z, float bias) {
  const float y = z + bias;
  return 1.f / (1.f + expf(-y));
}
// g and beta of one token as the recurrence takes them (log-decay, write strength)
__device__ __forceinline__ float gdn_load_g(const GdnArgs& a, int64_t i) {
  return a.gate_logits ? gdn_log_decay(a.g[i], a.g_bias) : a.g[i];
}
__device__ __forceinline__ float gdn_load_beta(const GdnArgs& a, int64_t i) {
  return a.gate_logits ? gdn_write_strength(a.beta[i], a.b_bias) : a.beta[i];
}

// Workspace of the 16-bit path: for each of the n = B*H*NC (sequence, head, chunk)
// records, these fields, each stored as its own array [n][...] so that consecutive
// chunks of one head are adjacent in memory (element offsets in 16-bit units; C = 64
// tokens, D = head dim):
//   w   [C][D]  T diag(beta * ge) Kn      (the state's pull on each row's update)
//   us  [D/32][4][64][8]  u = T diag(beta) V in the scan's register order: for column
//               slab s, wave w, lane l = 16 g + c, entries vt*4 + i hold u at token
//               16 w + 4 g + i, column 32 s + 16 vt + c (one 16-byte load per lane)
//   rq  [C][C]  exp(lg_p - lg_s) qn_p . kn_s for s <= p, else 0
//   f32 [3][C]  per token (fp32; f32_byte is a byte offset): lg, the inclusive
//               log-decays; kf = exp(lg_C - lg) / |k| (the write-back weight of the raw
//               key row, 1 / |k| only with l2norm); qs = scale / |q| (the raw query row's
//               factor, 1 / |q| only with l2norm)
// T = (I + A)^-1 with A[p,s] = beta_p exp(lg_p - lg_s) kn_p . kn_s (s < p), ge_p = exp(lg_p).
// The scan reads q and k rows straight from the inputs and applies qs and kf itself.
struct Gdn16Ws {
  int D;
  int64_t n;
  __host__ __device__ constexpr int64_t cd() const { return (int64_t)kChunk * D; }
  __host__ __device__ constexpr int64_t w(int64_t i) const { return i * cd(); }
  __host__ __device__ constexpr int64_t us(int64_t i) const { return (n + i) * cd(); }
  __host__ __device__ constexpr int64_t rq(int64_t i) const { return 2 * n * cd() + i * kChunk * kChunk; }
  __host__ __device__ constexpr int64_t f32_byte(int64_t i) const { return rq(n) * 2 + i * 3 * kChunk * 4; }
  __host__ __device__ constexpr int64_t bytes() const { return f32_byte(n); }
};

int launch_gdn16(const GdnArgs& a, int dtype, int D, hipStream_t stream);

}  // namespace atma
