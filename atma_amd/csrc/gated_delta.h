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
  // Segmented recurrence (16-bit path, long sequences with few heads): blockIdx.z = segment
  // seg runs chunks [seg * seg_len, min(NC, (seg + 1) * seg_len)).  seg_mode 0: one segment,
  // the plain scan.  1: segment summaries -- no output; state columns >= D start from the
  // identity with v = 0, so a segment's exit state holds its affine map [B | M] (exit = M
  // entry + B), written to seg_sum.  2: replay -- each segment starts from seg_in and
  // writes its output; the last one writes s_out.
  int seg_len, nseg, seg_mode;
  float* seg_sum;  // [B*H][nseg][D][2D] fp32
  float* seg_in;   // [B*H][nseg][D][D] fp32
};

// Segments of the 16-bit recurrence for B*H sequence-heads of NC chunks at head dim D on a
// device with `cus` compute units: enough that the summary pass (B*H*(2D/32) workgroups
// per segment, one per CU) fills the device, each segment at least 8 chunks; 1 (the plain
// scan) when the heads alone fill half of it.
inline int gdn16_segments(int64_t BH, int64_t NC, int D, int cus) {
  const int64_t per = BH * (2 * D / 32);  // summary workgroups of one segment
  if (NC < 16 || 2 * per > cus) return 1;
  int64_t n = 1 + cus / per;
  n = n < NC / 8 ? n : NC / 8;
  return n < 2 ? 1 : (int)n;
}

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

// Workspace of the 16-bit path: one record of kGdn16RecBytes per (sequence, head, chunk)
// item, item = (b * H + h) * NC + chunk, written by the prep kernel and copied whole into
// LDS by the scan.  With C = 64 tokens, T = (I + A)^-1, A[p,s] = beta_p exp(lg_p - lg_s)
// kn_p . kn_s (s < p) and Rq[p,s] = exp(lg_p - lg_s) qn_p . kn_s (s <= p):
//   Tb  [6][64 lanes][8]  T diag(beta), lower 16 x 32 blocks as MFMA A fragments: fragment
//       f = (P, j) in the order (0,0) (1,0) (2,0) (2,1) (3,0) (3,1); lane (g, r) holds row
//       16 P + r, columns 32 j + 4 g + [0, 4) and 32 j + 16 + 4 g + [0, 4)
//   Rb  [6][64 lanes][8]  Rq in the same fragment order: lane (g, c) holds row 16 P + c,
//       columns 32 j + 4 g + [0, 4) and 32 j + 16 + 4 g + [0, 4) (the MFMA B operand of
//       U^T Rq^T)
//   F   [4][64] fp32  per token: kf = exp(lg_C - lg) ik (the key row's write-back weight),
//       geik = exp(lg) ik (its weight in the state readout), geqs = exp(lg) iq (the query
//       row's weight, scale included); F[3][0] = exp(lg_C)
// with ik = 1 / |k|, iq = scale / |q| (1 and scale without l2norm; 0 past T) and lg the
// inclusive log-decays (13 KiB in all).
constexpr int kGdn16Tb = 0, kGdn16Rb = 6144, kGdn16F = 12288, kGdn16RecBytes = 13312;

int launch_gdn16(const GdnArgs& a, int dtype, int D, hipStream_t stream);
// Workspace of the 16-bit path: the records, plus the segment summaries and entry states
// when the launch splits the recurrence into segments.
size_t gdn16_workspace_bytes(int64_t BH, int64_t NC, int D);

}  // namespace atma
