// Gated-delta decode step, in place on the slot-indexed [K, V] fp32 state table.
//
// Reference: _gated_delta_step_kernel / gated_delta_decode_step,
// kernel/gated_delta_triton.py:36-117:
//   qn, kn = q/max(|q|,eps), k/max(|k|,eps);  Sd = gamma*S;  pred_v = sum_k kn_k Sd[k,v]
//   u = beta*(v - pred);  S' = Sd + kn u^T (stored in place);  r_v = sum_k qn_k S'[k,v]
//
// MI355X mapping: the state is pure HBM traffic (64 KiB per (sequence, head) read
// once and written once), so one workgroup owns a 64-column slab of one head's
// state: 16 column groups x float4 = 64 contiguous floats (256 B) per row, 16 row
// groups covering the dk rows.  The slab sits in registers between the two
// column reductions (pred, then r), so each state byte crosses HBM exactly once
// in each direction.
#include "gated_delta.h"
#include "gated_delta_step.h"

namespace atma {

template <typename T, int D>
__global__ void __launch_bounds__(256) gated_delta_step_kernel(GdnStepArgs a) {
  gdn_step_block<T, D>(a, blockIdx.x, blockIdx.y);
}

template <typename T, int D>
static int launch_step(const void* q, int64_t q_sb, int64_t q_sh, const void* k, int64_t k_sb,
                       int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sh, const float* gamma,
                       const float* beta, float* state, int64_t max_seqs, const int64_t* slots,
                       float* r, int64_t B, int64_t H, int64_t G, float eps, hipStream_t stream) {
  GdnStepArgs a{q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, gamma, beta, state, max_seqs, slots, r,
                (int)H, (int)G, eps};
  gated_delta_step_kernel<T, D><<<dim3((unsigned)(B * H), gdn_step_slabs<D>()), dim3(256), 0, stream>>>(a);
  return check_launch("gated_delta_decode_step");
}

template <typename T>
static int dispatch_step(int64_t D, const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                         int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sh,
                         const float* gamma, const float* beta, float* state, int64_t max_seqs,
                         const int64_t* slots, float* r, int64_t B, int64_t H, int64_t G,
                         float eps, hipStream_t s) {
  if (D == 128)
    return launch_step<T, 128>(q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, gamma, beta, state,
                               max_seqs, slots, r, B, H, G, eps, s);
  return launch_step<T, 64>(q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, gamma, beta, state,
                            max_seqs, slots, r, B, H, G, eps, s);
}

}  // namespace atma

extern "C" int atma_gated_delta_decode_step(const void* q, int64_t q_sb, int64_t q_sh,
                                            const void* k, int64_t k_sb, int64_t k_sh,
                                            const void* v, int64_t v_sb, int64_t v_sh,
                                            const float* gamma, const float* beta,
                                            float* state_table, int64_t max_seqs,
                                            const int64_t* slots, float* r, int64_t B, int64_t H,
                                            int64_t Hkv, int64_t dk, int64_t dv, int dtype,
                                            float eps, void* stream) {
  using namespace atma;
  if (dk != dv || (dk != 128 && dk != 64))
    return set_error(ATMA_ERR_UNSUPPORTED, "gated_delta_decode_step: dk=dv in {64,128} (got %lld,%lld)",
                     (long long)dk, (long long)dv);
  if (B < 0 || H <= 0 || max_seqs < 0 || Hkv <= 0 || H % Hkv)
    return set_error(ATMA_ERR_INVALID, "gated_delta_decode_step: bad sizes (H must be a multiple of Hkv)");
  const int64_t G = H / Hkv;
  if (B == 0) return ATMA_OK;
  if (!q || !k || !v || !gamma || !beta || !state_table || !slots || !r)
    return set_error(ATMA_ERR_INVALID, "gated_delta_decode_step: null pointer");
  if (B * H > 0x7fffffff) return set_error(ATMA_ERR_INVALID, "gated_delta_decode_step: B*H too large");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_F32:
      return dispatch_step<float>(dk, q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, gamma, beta,
                                  state_table, max_seqs, slots, r, B, H, G, eps, s);
    case ATMA_BF16:
      return dispatch_step<bf16>(dk, q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, gamma, beta,
                                 state_table, max_seqs, slots, r, B, H, G, eps, s);
    case ATMA_F16:
      return dispatch_step<f16>(dk, q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, gamma, beta,
                                state_table, max_seqs, slots, r, B, H, G, eps, s);
    default:
      return set_error(ATMA_ERR_INVALID, "gated_delta_decode_step: unknown dtype %d", dtype);
  }
}

// ---------------------------------------------------------------------------------------
// Gate activations of the memory branch in one pass: g = logsigmoid(zg + g_bias) (the
// log-decay the chunked rule takes) and beta = sigmoid(zb + b_bias), or with
// decay_as_prob the decode step's gamma = sigmoid(zg + g_bias).  Replaces the
// torch add / logsigmoid / sigmoid launches of TitansMemory (model/blocks.py:426-490).
namespace atma {
__global__ void gdn_gates_kernel(const float* __restrict__ zg, const float* __restrict__ zb,
                                 float g_bias, float b_bias, float* __restrict__ g,
                                 float* __restrict__ beta, int64_t n, int decay_as_prob) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float ls = gdn_log_decay(zg[i], g_bias);
  g[i] = decay_as_prob ? expf(ls) : ls;
  beta[i] = gdn_write_strength(zb[i], b_bias);
}
}  // namespace atma

extern "C" int atma_gated_delta_gates(const float* zg, const float* zb, float g_bias, float b_bias,
                                      float* g, float* beta, int64_t n, int decay_as_prob,
                                      void* stream) {
  if (n < 0) return atma::set_error(ATMA_ERR_INVALID, "gated_delta_gates: n < 0");
  if (n == 0) return ATMA_OK;
  if (!zg || !zb || !g || !beta) return atma::set_error(ATMA_ERR_INVALID, "gated_delta_gates: null pointer");
  const int64_t blocks = (n + 255) / 256;
  atma::gdn_gates_kernel<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
      zg, zb, g_bias, b_bias, g, beta, n, decay_as_prob ? 1 : 0);
  return atma::check_launch("gated_delta_gates");
}
