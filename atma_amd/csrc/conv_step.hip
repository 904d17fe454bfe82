// Depthwise causal convolution for one new token per sequence, with the slot-indexed
// state of the last K - 1 inputs advanced in place.
//
// Reference: _causal_conv1d_step_kernel / causal_conv1d_decode_step
// (kernel/causal_conv1d_triton.py:18-63), used for the global layer's Canon q / k / v
// convolutions at decode (inference/models/atma.py:160-192):
//   out[b, d] = x[b, d] w[d, K-1] + sum_{j < K-1} state[slot, d, j] w[d, j]
//   state[slot, d, :] <- (state[slot, d, 1:], x[b, d])
// One thread per (sequence, channel): the state row of a channel is K - 1 <= 15 values,
// read once and written once; products accumulate in fp32 in the reference's order and
// round once to the input dtype.  A slot outside [0, max_seqs) leaves the table untouched
// and yields NaN outputs (as the gated-delta decode step does).
#include "common.h"

namespace atma {

template <typename T>
__global__ void __launch_bounds__(256)
causal_conv1d_step_kernel(const T* __restrict__ x, int64_t x_sb, const T* __restrict__ w, int64_t w_sd,
                          int64_t w_sk, const int64_t* __restrict__ slots, T* __restrict__ state,
                          int64_t s_ss, int64_t s_sd, int64_t s_sk, int64_t max_seqs, T* __restrict__ out,
                          int64_t o_sb, int D, int K, int residual) {
  const int b = blockIdx.x;
  const int d = blockIdx.y * 256 + threadIdx.x;
  if (d >= D) return;
  const T xt = x[(int64_t)b * x_sb + d];
  const float xv = to_f32(xt);
  const T* wd = w + (int64_t)d * w_sd;
  float acc = xv * to_f32(wd[(int64_t)(K - 1) * w_sk]);
  if (K > 1) {
    const int64_t slot = slots[b];
    if (slot < 0 || slot >= max_seqs) {
      out[(int64_t)b * o_sb + d] = from_f32<T>(__builtin_nanf(""));
      return;
    }
    T* st = state + slot * s_ss + (int64_t)d * s_sd;
    for (int j = 0; j < K - 1; ++j) {
      const T old = st[(int64_t)j * s_sk];
      acc += to_f32(old) * to_f32(wd[(int64_t)j * w_sk]);
      if (j > 0) st[(int64_t)(j - 1) * s_sk] = old;  // shift left, each value read before overwritten
    }
    st[(int64_t)(K - 2) * s_sk] = xt;
  }
  out[(int64_t)b * o_sb + d] = from_f32<T>(residual ? xv + acc : acc);
}

template <typename T>
static int launch_conv_step(const void* x, int64_t x_sb, const void* w, int64_t w_sd, int64_t w_sk,
                            const int64_t* slots, void* state, int64_t s_ss, int64_t s_sd, int64_t s_sk,
                            int64_t max_seqs, void* out, int64_t o_sb, int64_t B, int64_t D, int64_t K,
                            int residual, hipStream_t s) {
  const dim3 grid((unsigned)B, (unsigned)((D + 255) / 256));
  causal_conv1d_step_kernel<T><<<grid, dim3(256), 0, s>>>(
      (const T*)x, x_sb, (const T*)w, w_sd, w_sk, slots, (T*)state, s_ss, s_sd, s_sk, max_seqs,
      (T*)out, o_sb, (int)D, (int)K, residual);
  return check_launch("causal_conv1d_decode_step");
}

}  // namespace atma

extern "C" int atma_causal_conv1d_decode_step(const void* x, int64_t x_sb, const void* weight,
                                              int64_t w_sd, int64_t w_sk, const int64_t* slots,
                                              void* state_table, int64_t s_ss, int64_t s_sd,
                                              int64_t s_sk, int64_t max_seqs, void* out,
                                              int64_t o_sb, int64_t B, int64_t D, int64_t K,
                                              int residual, int dtype, void* stream) {
  using namespace atma;
  if (B < 0 || D < 0 || K < 1 || K > 16 || max_seqs < 0)
    return set_error(ATMA_ERR_INVALID, "causal_conv1d_decode_step: bad sizes (1 <= K <= 16)");
  if (B == 0 || D == 0) return ATMA_OK;
  if (B > 0x7fffffff || D > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "causal_conv1d_decode_step: sizes too large");
  if (!x || !weight || !out || (K > 1 && (!slots || !state_table)))
    return set_error(ATMA_ERR_INVALID, "causal_conv1d_decode_step: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_F32:
      return launch_conv_step<float>(x, x_sb, weight, w_sd, w_sk, slots, state_table, s_ss, s_sd, s_sk,
                                     max_seqs, out, o_sb, B, D, K, residual, s);
    case ATMA_BF16:
      return launch_conv_step<bf16>(x, x_sb, weight, w_sd, w_sk, slots, state_table, s_ss, s_sd, s_sk,
                                    max_seqs, out, o_sb, B, D, K, residual, s);
    case ATMA_F16:
      return launch_conv_step<f16>(x, x_sb, weight, w_sd, w_sk, slots, state_table, s_ss, s_sd, s_sk,
                                   max_seqs, out, o_sb, B, D, K, residual, s);
    default:
      return set_error(ATMA_ERR_INVALID, "causal_conv1d_decode_step: unknown dtype %d", dtype);
  }
}
