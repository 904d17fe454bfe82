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
  float scale;
  int l2norm;
  void* ws;
};

// Per-chunk record of the 16-bit path: T*diag(beta) and Rq as 64x64 16-bit matrices
// (zero above the diagonal), then the 64 inclusive log-decays (fp32).
constexpr int64_t kGdn16RecBytes = 2 * kChunk * kChunk * 2 + kChunk * 4;

int launch_gdn16(const GdnArgs& a, int dtype, int D, hipStream_t stream);

}  // namespace atma
