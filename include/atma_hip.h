/*
 * atma_hip.h -- C ABI of libatma_hip.so, the MI355X (gfx950) implementation of
 * ATMA's global-layer mixer: Polar attention prefill and paged decode, the paged
 * KV write, and the gated-delta memory (chunked prefill + single-token step).
 *
 * Conventions (every entry point):
 *   - plain device pointers, element strides (int64, in elements, not bytes),
 *     dimensions and float scalars; no framework types;
 *   - `dtype` selects the element type of the activation tensors (q/k/v, caches,
 *     outputs c/mag/o): ATMA_F32, ATMA_BF16 or ATMA_F16.  Parameters, n_keys,
 *     gates and memory states are always fp32;
 *   - the innermost (head_dim) stride of every activation tensor is 1;
 *   - `stream` is a hipStream_t (NULL = the legacy default stream);
 *   - kernels are only enqueued: no host synchronisation, no device allocation
 *     (scratch comes in through `workspace`), no memset -- every entry point is
 *     safe under stream / graph capture;
 *   - return ATMA_OK (0) or an ATMA_ERR_* code; atma_last_error() then returns a
 *     message (thread-local, valid until the next call on that thread).
 *
 * Each declaration cites the reference operation it replaces (paths relative to
 * the akbar2habibullah/atma repository).
 */
#ifndef ATMA_HIP_H
#define ATMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ATMA_F32 = 0, ATMA_BF16 = 1, ATMA_F16 = 2 };

enum {
  ATMA_OK = 0,
  ATMA_ERR_INVALID = 1,     /* bad shape / stride / argument            */
  ATMA_ERR_UNSUPPORTED = 2, /* valid request this build does not cover  */
  ATMA_ERR_WORKSPACE = 3,   /* workspace missing or too small           */
  ATMA_ERR_HIP = 4          /* a HIP runtime call or launch failed      */
};

/* Version of this ABI (bumped on any signature change). */
int atma_abi_version(void);

/* Message describing the last non-zero return on the calling thread. */
const char* atma_last_error(void);

/*
 * Paged KV write.  Replaces store_kvcache (inference/layers/attention.py:30-56).
 * key/value: (n_tokens, Hkv, d) rows, row stride key_stride / value_stride
 * elements, each row `row_elems` = Hkv*d contiguous elements.  k_cache/v_cache:
 * contiguous (num_pages, page_size, Hkv, d) = `total_slots` rows of row_elems.
 * Token i is copied bit-for-bit into row slot_mapping[i]; slots < 0 are skipped
 * (reference: -1 = skip) and slots >= total_slots are skipped too.
 */
int atma_store_kvcache(const void* key, int64_t key_stride, const void* value,
                       int64_t value_stride, void* k_cache, void* v_cache,
                       const int32_t* slot_mapping, int64_t n_tokens, int64_t row_elems,
                       int64_t total_slots, int dtype, void* stream);

/*
 * Flash-style Polar attention forward (prefill).  Replaces polar_attention_fwd /
 * _polar_forward (kernel/polar_triton.py:505-609).
 * q: (B, Hq, Tq, d) strides (q_sb, q_sh, q_st, 1);  k, v: (B, Hkv, Tk, d) with
 * Hq % Hkv == 0 (GQA handled in-kernel; Hkv == Hq is the reference's expanded
 * form).  n_keys: (Tq,) fp32 valid-key count per query (the mask uses it raw,
 * temp/null use max(min(n, window), 1)).  Raw Polar parameters, fp32, contiguous:
 * v_null (Hq, d), null_base / null_slope_raw / len_gain_raw / mag_beta_raw (Hq,).
 * Outputs (dtype, contiguous): c (B, Hq, Tq, d), mag (B, Hq, Tq).  Optional fp32
 * saved statistics for a backward pass (any may be NULL): stat_m / stat_l /
 * stat_q2 (B, Hq, Tq) as a natural-log reference m with sum p and sum p^2 taken
 * relative to it (p = exp(score - m)), after the null fold -- m is the running max
 * for fp32 inputs and at most it (the kernel's rescaling point) for 16-bit inputs,
 * so (m, sum p) fix the normaliser either way -- and stat_s (B, Hq, Tq, d) the
 * unnormalised direction.
 * is_causal requires Tq == Tk and bounds each query tile's key loop at the tile's
 * last row (kernel/polar_triton.py:110-113,522-526).  window <= 0 disables the
 * sliding window; with preserve_length != 0, temp / null use the raw count even under
 * a window (kernel/polar_triton.py:93-96).  d must be 64 or 128.
 */
int atma_polar_attention_fwd(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                             const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                             const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                             const float* n_keys, const float* v_null, const float* null_base,
                             const float* null_slope_raw, const float* len_gain_raw,
                             const float* mag_beta_raw, void* c, void* mag, float* stat_m,
                             float* stat_l, float* stat_q2, float* stat_s, int64_t B,
                             int64_t Hq, int64_t Hkv, int64_t Tq, int64_t Tk, int64_t d,
                             int dtype, int is_causal, int64_t window, int preserve_length,
                             float eps, void* stream);

/*
 * Grouped fresh-prefill Polar attention over packed ragged requests.  Replaces
 * polar_attention_packed_fwd / _polar_packed_fwd_kernel (kernel/polar_triton.py:194-309,
 * 613-669).  q: (total_tokens, Hq, d) strides (q_st, q_sh, 1); k, v: (total_tokens, Hkv, d)
 * with Hq % Hkv == 0 (Hkv == Hq is the reference's expanded form).  Tile map (device,
 * int32, n_tiles entries each, as the serving context builds it,
 * inference/engine/model_runner.py:390-404): tile i covers query rows
 * tile_q_start[i] .. + 127 (a multiple of 128) of the sequence stored at packed tokens
 * tile_seq_start[i] .. + tile_seq_len[i] - 1.  Every sequence is a fresh causal prompt:
 * query j sees keys 0..j of its own sequence (n = j + 1; with window > 0 only the last
 * `window` of them, temp/null from max(min(n, window), 1)).  A tile outside
 * [0, total_tokens) or off a 128-row boundary is skipped (its rows are not written).
 * Outputs (dtype): c with strides (c_st, c_sh, 1), mag with strides (m_st, m_sh).
 * Raw Polar parameters as atma_polar_attention_fwd.  bf16 / fp16 only; d = 64 or 128.
 */
int atma_polar_attention_packed_fwd(const void* q, int64_t q_st, int64_t q_sh, const void* k,
                                    int64_t k_st, int64_t k_sh, const void* v, int64_t v_st,
                                    int64_t v_sh, const int32_t* tile_seq_start,
                                    const int32_t* tile_q_start, const int32_t* tile_seq_len,
                                    int64_t n_tiles, const float* v_null, const float* null_base,
                                    const float* null_slope_raw, const float* len_gain_raw,
                                    const float* mag_beta_raw, void* c, int64_t c_st,
                                    int64_t c_sh, void* mag, int64_t m_st, int64_t m_sh,
                                    int64_t total_tokens, int64_t Hq, int64_t Hkv, int64_t d,
                                    int dtype, int64_t window, float eps, void* stream);

/*
 * Polar attention backward: the two O(T^2) loops of _polar_backward
 * (kernel/polar_triton.py:861-1155; _polar_bwd_dq_kernel :870-947,
 * _polar_bwd_dkdv_kernel :951-1030).  q, gs: (B, Hq, Tq, d) and k, v: (B, Hkv, Tk, d)
 * in dtype with strides (x_sb, x_sh, x_st, 1) (GQA resolved in-kernel: query head h
 * reads KV head h / (Hq / Hkv)); gL, gQ2, M: (B, Hq, Tq) fp32 contiguous (the
 * preamble's per-query cotangents and the forward's natural-log reference max);
 * temp: (Hq, Tq) fp32; n_keys: (Tq,) raw counts (the mask).  Outputs, contiguous, every
 * element written when Tk > 0: dq (B, Hq, Tq, d) in dtype, and fp32 dt (B, Hq, Tq) (= sum_j da * sig,
 * the real keys' share of dL/dtemp), dk, dv (B, Hq, Tk, d) (fp32 for fp32 and fp16 inputs, bf16 for
 * bf16 inputs): each query head's share, so
 * with Hkv < Hq the caller sums the Hq / Hkv consecutive heads of a group (one workgroup
 * per query head fills the GPU at causal T = 2,048; a deterministic sum, no atomics).
 * d = 64 or 128.
 */
/*
 * Polar attention backward, per-query preamble (kernel/polar_triton.py:1049-1088) and
 * parameter-gradient partial sums (:1139-1150).  gc: (B, H, T, d), gm: (B, H, T) in dtype
 * (nullable: a zero cotangent); S: (B, H, T, d), M, L, Q2: (B, H, T) fp32, the forward's
 * statistics (M in natural-log units); n_keys: (T,); the five Polar parameters (fp32);
 * window / preserve_length as in the forward.  Writes gs (B, H, T, d) in dtype, gL, gQ2
 * (B, H, T) fp32 (the inputs of atma_polar_attention_bwd), temp (H, T) fp32, and per
 * 16-row block part (B * ceil(T / 16), H, d + 4) fp32: [sum p_null gs | sum dL/da_null nu
 * log n | sum dL/da_null temp | sum dL/da_null temp sqrt(log(n + 1)) | sum gm (1 - mag^2)
 * log1p(m_eff)], which the caller sums over blocks.  d = 64 or 128.
 */
int atma_polar_attention_bwd_prep(const void* gc, const void* gm, const float* S, const float* M,
                                  const float* L, const float* Q2, const float* n_keys,
                                  const float* v_null, const float* null_base,
                                  const float* null_slope_raw, const float* len_gain_raw,
                                  const float* mag_beta_raw, void* gs, float* gL, float* gQ2,
                                  float* temp, float* part, int64_t B, int64_t H, int64_t T,
                                  int64_t d, int dtype, int64_t window, int preserve_length,
                                  float eps, void* stream);

/*
 * Final step of the backward's dk / dv, no reference
 * counterpart (the reference's loops write per-KV-head fp32 gradients that autograd casts):
 * out[g0, r] = sum_{g < G} part[g0 * G + g, r] in dtype, for n_groups groups of G
 * consecutive slices of `elems` elements of part_dtype (ATMA_F32 or ATMA_BF16; elems % 4 == 0;
 * part 16-byte aligned), summed in fp32.
 * With the (B, Hq, Tk, d) shares of atma_polar_attention_bwd: n_groups = B * Hkv,
 * G = Hq / Hkv, elems = Tk * d.  A fixed-order sum: deterministic.
 */
int atma_polar_bwd_group_sum(const void* part, int part_dtype, void* out, int64_t n_groups, int64_t G,
                             int64_t elems, int dtype, void* stream);

/*
 * The parameter gradients of the Polar backward (kernel/polar_triton.py:1139-1150) from the
 * preamble's per-block sums `part` (B * ceil(T / 16), H, d + 4) and the loops' dt (B, H, T),
 * with n_keys (T,) and window / preserve_length as in the forward: g_v_null (H, d) and
 * g_params (4, H) fp32 = the gradients of null_base, null_slope_raw, len_gain_raw and
 * mag_beta_raw (two launches, fixed-order sums; workspace of
 * atma_polar_bwd_param_grads_workspace_bytes).  d = 64 or 128.
 */
size_t atma_polar_bwd_param_grads_workspace_bytes(int64_t H, int64_t d);
int atma_polar_bwd_param_grads(const float* part, const float* dt, const float* n_keys,
                               const float* len_gain_raw, const float* null_slope_raw,
                               const float* mag_beta_raw, float* g_v_null, float* g_params, int64_t B,
                               int64_t H, int64_t T, int64_t d, int64_t window, int preserve_length,
                               void* workspace, size_t workspace_bytes, void* stream);

int atma_polar_attention_bwd(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                             const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                             const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                             const void* gs, int64_t g_sb, int64_t g_sh, int64_t g_st,
                             const float* gL, const float* gQ2, const float* M,
                             const float* temp, const float* n_keys, void* dq, float* dt,
                             void* dk, void* dv, int64_t B, int64_t Hq, int64_t Hkv,
                             int64_t Tq, int64_t Tk, int64_t d, int dtype, int is_causal,
                             int64_t window, void* stream);

/*
 * Workspace bytes atma_polar_attention_decode needs for this launch shape (a function of
 * the shapes and dtype only, never of the context lengths).
 */
size_t atma_polar_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_pages,
                                         int64_t page_size, int64_t d, int dtype);

/*
 * Paged Polar GQA decode (split-K over pages + merge).  Replaces
 * polar_attention_decode / _polar_decode_kernel (kernel/polar_triton.py:682-858).
 * q: (B, Hq, d) strides (q_sb, q_sh, 1).  k_cache / v_cache: contiguous
 * (num_pages, page_size, Hkv, d).  block_tables: (B, max_pages) int32 with row
 * stride bt_sb; context_lens: (B,) int32, keys 0..ctx-1 of sequence b live at
 * page block_tables[b, pos / page_size], row pos % page_size.  Entries past a
 * sequence's last page are never read; page ids outside [0, num_pages) are
 * treated as empty keys.  Outputs (dtype, contiguous): c (B, Hq, d), mag (B, Hq).
 * The launch shape depends only on (B, Hq, max_pages): graph capturable.
 */
int atma_polar_attention_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* k_cache,
                                const void* v_cache, int64_t num_pages, int64_t page_size,
                                int64_t Hkv, const int32_t* block_tables, int64_t bt_sb,
                                int64_t max_pages, const int32_t* context_lens,
                                const float* v_null, const float* null_base,
                                const float* null_slope_raw, const float* len_gain_raw,
                                const float* mag_beta_raw, void* c, void* mag, int64_t B,
                                int64_t Hq, int64_t d, int dtype, int64_t window, float eps,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * atma_polar_attention_decode with the split records in a fixed file-scope device
 * array of atma_polar_decode_noalloc_max_bytes() bytes (32 MiB) instead of a caller
 * workspace; same arguments minus the workspace, same kernels, same results.  A launch
 * whose records need more (atma_polar_decode_workspace_bytes) is rejected with
 * ATMA_ERR_WORKSPACE.  Allocates nothing; every call on one GPU shares that GPU's array,
 * so calls that overlap on one GPU race.
 */
size_t atma_polar_decode_noalloc_max_bytes(void);
int atma_polar_attention_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                        const void* k_cache, const void* v_cache, int64_t num_pages,
                                        int64_t page_size, int64_t Hkv, const int32_t* block_tables,
                                        int64_t bt_sb, int64_t max_pages,
                                        const int32_t* context_lens, const float* v_null,
                                        const float* null_base, const float* null_slope_raw,
                                        const float* len_gain_raw, const float* mag_beta_raw,
                                        void* c, void* mag, int64_t B, int64_t Hq, int64_t d,
                                        int dtype, int64_t window, float eps, void* stream);

/*
 * One gated-delta decode step, IN PLACE on the slot-indexed fp32 state table.
 * Replaces gated_delta_decode_step (kernel/gated_delta_triton.py:78-117).
 * q: (B, H, d), k, v: (B, Hkv, d) with H % Hkv == 0, strides (x_sb, x_sh, 1) -- query
 * head h reads k / v head h / (H / Hkv); Hkv == H is the reference's expanded form;
 * gamma, beta: (B, H) fp32 contiguous; state_table: contiguous fp32
 * (max_seqs, H, dk, dv) in [K, V] layout; slots: (B,) int64 rows of the table
 * (a slot outside [0, max_seqs) leaves the table untouched and yields NaN r).
 * Output r: (B, H, dv) fp32 contiguous.  dk = dv = 128 or 64.
 */
int atma_gated_delta_decode_step(const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                                 int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb,
                                 int64_t v_sh, const float* gamma, const float* beta,
                                 float* state_table, int64_t max_seqs, const int64_t* slots,
                                 float* r, int64_t B, int64_t H, int64_t Hkv, int64_t dk,
                                 int64_t dv, int dtype, float eps, void* stream);

/*
 * The global layer's decode mixer in two launches: the calls
 *   store_kvcache(k_new, v_new, caches, slot_mapping)      (inference/layers/attention.py:30-56)
 *   polar_attention_decode(q, caches, block_tables, ...)    (kernel/polar_triton.py:682-858)
 *   gated_delta_decode_step(q, k_new, v_new, gamma, beta, state_table, slots)
 *                                                           (kernel/gated_delta_triton.py:78-117)
 * as made in that order by the reference's decode route (inference/models/atma.py:546-618,
 * _mem_decode :341-375).  The length-balanced split streams the cached keys before the
 * newest; one tail launch merges the splits with the newest key taken from k_new / v_new,
 * writes the k_new / v_new rows into the caches at slot_mapping, and runs the memory step.
 * Equal to the three calls when slot_mapping[b] is the cache slot of position
 * context_lens[b] - 1 (a slot outside the cache is not written; that row still attends
 * k_new / v_new as its newest key).  Arguments are those of the three entries:
 * k_new, v_new: (B, Hkv, d) strides (x_sb, x_sh, 1); caches written in place;
 * workspace: atma_polar_decode_workspace_bytes() bytes.  Serves 16-bit caches whose pages
 * hold whole 32-key units (atma_global_decode_step_supported); ATMA_ERR_UNSUPPORTED
 * otherwise, and the caller makes the three calls.
 */
int atma_global_decode_step_supported(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_pages,
                                      int64_t page_size, int64_t d, int dtype);
int atma_global_decode_step(const void* q, int64_t q_sb, int64_t q_sh, const void* k_new,
                            int64_t kn_sb, int64_t kn_sh, const void* v_new, int64_t vn_sb,
                            int64_t vn_sh, void* k_cache, void* v_cache, int64_t num_pages,
                            int64_t page_size, int64_t Hkv, const int32_t* slot_mapping,
                            const int32_t* block_tables, int64_t bt_sb, int64_t max_pages,
                            const int32_t* context_lens, const float* v_null,
                            const float* null_base, const float* null_slope_raw,
                            const float* len_gain_raw, const float* mag_beta_raw, void* c,
                            void* mag, const float* gamma, const float* beta, float* state_table,
                            int64_t max_seqs, const int64_t* slots, float* r, int64_t B,
                            int64_t Hq, int64_t d, int dtype, int64_t window, float eps,
                            float mem_eps, void* workspace, size_t workspace_bytes, void* stream);

/*
 * One depthwise causal-convolution step, slot-indexed state advanced IN PLACE.
 * Replaces causal_conv1d_decode_step (kernel/causal_conv1d_triton.py:18-63), the
 * global layer's Canon q / k / v convolution at decode (inference/models/atma.py:160-192).
 * x: (B, D) strides (x_sb, 1); weight: (D, K) strides (w_sd, w_sk), x's dtype;
 * state_table: (max_seqs, D, K - 1) strides (s_ss, s_sd, s_sk), x's dtype; slots: (B,)
 * int64 rows of the table.  out (B, D) strides (o_sb, 1):
 * x w[:, K-1] + sum_j state[slot, :, j] w[:, j] (plus x when residual != 0), accumulated
 * in fp32; the state row becomes (state[slot, :, 1:], x).  K = 1 touches no state.  A
 * slot outside [0, max_seqs) leaves the table untouched and yields NaN.  1 <= K <= 16.
 */
int atma_causal_conv1d_decode_step(const void* x, int64_t x_sb, const void* weight, int64_t w_sd,
                                   int64_t w_sk, const int64_t* slots, void* state_table,
                                   int64_t s_ss, int64_t s_sd, int64_t s_sk, int64_t max_seqs,
                                   void* out, int64_t o_sb, int64_t B, int64_t D, int64_t K,
                                   int residual, int dtype, void* stream);

/*
 * Backward of the gated-delta recurrence, the training path of chunk_gated_delta_rule
 * (FLA autograd in the reference: model/blocks.py:44-84, caller TitansMemory.forward
 * model/blocks.py:470-479; recurrence scripts/titans_proto.py:53-76).  All fp32 and
 * contiguous: q (scaled and normalised), k (normalised): (B, T, H, dk); v, d_out: (B, T, H, dv);
 * g (log decay), beta: (B, T, H); initial_state, d_final_state: (B, H, dk, dv) [K, V] or NULL
 * (zero).  Writes dv (B, T, H, dv) and d_initial_state (B, H, dk, dv) in full, and per
 * 16-column block of V (JB = dv / 16) the partial sums dq_part, dk_part (JB, B, T, H, dk) and
 * dg_part (d/dg, already times exp(g)), dbeta_part (JB, B, T, H): the caller sums axis 0.
 * dk in {64, 128}; dv a multiple of 16.  workspace: atma_gated_delta_bwd_workspace_bytes
 * (state checkpoints every 64 tokens).
 */
size_t atma_gated_delta_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv);
int atma_gated_delta_bwd(const float* q, const float* k, const float* v, const float* g, const float* beta,
                         const float* initial_state, const float* d_out, const float* d_final_state,
                         float* dq_part, float* dk_part, float* dv, float* dg_part, float* dbeta_part,
                         float* d_initial_state, int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv_dim,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Chunked (WY) backward of the same recurrence for 16-bit training, in three launches: the
 * algorithm of the FLA chunk_gated_delta_rule autograd the reference trains through
 * (model/blocks.py:44-84), which carries the state gradient across 64-token chunks and
 * forms every other gradient within a chunk.  N = B * H * NC chunk-head items,
 * n = (b * H + h) * NC + c, NC = ceil(T / 64); d in {64, 128}; dtype ATMA_BF16 / ATMA_F16
 * names the 16-bit type of v, d_out and every tile; all operands contiguous and 16-byte
 * aligned.  Tokens past T act as zero-padding (k = q = v = dO = 0, beta = 0, log decay 0),
 * which leaves every gradient exact.
 *
 * prep: q, k, v, d_out: (B, T, H, d) 16-bit (q and k raw: with l2norm != 0 each row is
 * divided by max(|x|, 1e-12), q then times scale, as the forward with
 * use_qk_l2norm_in_kernel); g (log decay), beta: (B, T, H) fp32.  Writes the 16-bit tiles
 * kr, qr (N, 64, d) rows of the normalised k and scaled q;
 * kt, qt, vt, ot, got (N, d, 64) = k^T, q^T, v^T, dO^T, (diag(Ga) dO)^T; tm, tt (N, 64, 64)
 * T = (I + diag(beta) A)^-1 and T^T, A[p,s] = exp(lg_p - lg_s) k_p.k_s (s < p); rt
 * (N, 64, 64) Rq^T, Rq[p,s] = exp(lg_p - lg_s) q_p.k_s (s <= p); and f (N, 5, 64) fp32 per
 * token: Ga = exp(lg), w = exp(lg_C - lg), beta, Ga_C, lg (lg the in-chunk inclusive
 * cumulative log decay), and the row-norm factors iq = scale / max(|q|, eps),
 * ik = 1 / max(|k|, eps), uq2 = 1 / |q|^2, uk2 = 1 / |k|^2 (0 where |x| <= eps; without
 * l2norm: scale, 1, 0, 0) -- f is (N, 9, 64).
 *
 * chain: the prep's tiles (BH = B * H); s0, dst (BH, d, d) [K, V] fp32 initial state and
 * final-state cotangent, or NULL (zero).  Runs the state forward over the chunks, then the
 * state gradient backwards (dU = Rq^T dO + diag(w) K dS, dY = T^T dU,
 * dS <- Ga_C dS + Q^T diag(Ga) dO - K^T diag(Ga beta) dY), writing s_entry and ds_end
 * (N, d, d) 16-bit (each chunk's entry state, the gradient of its exit state), u (N, 64, d)
 * 16-bit (U = T diag(beta)(V - diag(Ga) K S)), dy (N, 64, d) fp32 and ds0 (BH, d, d) fp32.
 *
 * local: the prep's kr, kt, qr, qt, f, the chain's s_entry, ds_end, u, dy, and q, k, v,
 * d_out as given to the prep.  Writes dq, dk, dv (B, T, H, d) 16-bit (dq, dk through the
 * l2 norm and scale to the raw rows), dg, dbeta (B, T, H) fp32 (dg the gradient of the
 * per-token log decay).
 */
int atma_gated_delta_bwd16_prep(const void* q, const void* k, const void* v, const void* d_out,
                                const float* g, const float* beta, void* kr, void* kt, void* qr, void* qt,
                                void* tm, void* tt, void* rt, void* vt, void* ot, void* got, float* f,
                                int64_t B, int64_t T, int64_t H, int64_t d, float scale, int l2norm, int dtype,
                                void* stream);
int atma_gated_delta_bwd16_chain(const void* kr, const void* kt, const void* qt, const void* tm,
                                 const void* tt, const void* rt, const void* vt, const void* ot,
                                 const void* got, const float* f, const float* s0, const float* dst,
                                 void* s_entry, void* ds_end, void* u, float* dy, float* ds0, int64_t BH,
                                 int64_t NC, int64_t d, int dtype, void* stream);
int atma_gated_delta_bwd16_local(const void* kr, const void* kt, const void* qr, const void* qt,
                                 const void* q, const void* k, const void* v, const void* d_out,
                                 const float* f, const void* s_entry, const void* ds_end, const void* u,
                                 const float* dy, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                                 int64_t B, int64_t T, int64_t H, int64_t d, int dtype, void* stream);

/*
 * Fused MLP activation out = gate * relu(x)^2.  Replaces squared_relu_gate
 * (kernel/inference_ops_triton.py:102-135), called by InferenceMLP.forward
 * (inference/models/atma.py:87-96).  x, gate: (rows, width) with strides (x_s0, x_s1),
 * (g_s0, g_s1) -- typically the two halves of one fc output; out: (rows, width)
 * contiguous, same dtype.  bf16 inputs round relu(x)^2 to bf16 before the gate multiply
 * (eager bf16's intermediate rounding); the product is computed in fp32 and rounded once.
 */
int atma_squared_relu_gate(const void* x, int64_t x_s0, int64_t x_s1, const void* gate, int64_t g_s0,
                           int64_t g_s1, void* out, int64_t rows, int64_t width, int dtype, void* stream);

/*
 * Output soft cap out = 15 x / sqrt(x^2 + 225) over n contiguous elements.  Replaces
 * softcap_logits (kernel/inference_ops_triton.py:194-223), called by compute_logits
 * (inference/models/atma.py:750-754).  For bf16, 15 x, x^2, x^2 + 225 and the reciprocal
 * square root (the correctly rounded 1 / sqrt) are each rounded to bf16 before the final
 * product; fp32 / fp16 round only the output.
 */
int atma_softcap_logits(const void* logits, void* out, int64_t n, int dtype, void* stream);

/*
 * Depthwise causal convolution over packed variable-length sequences.  Replaces
 * packed_causal_conv1d (kernel/inference_ops_triton.py:17-63, 138-160), called by the
 * grouped fresh prefill (inference/models/atma.py:431-442, 648-652).
 * x: (total, channels) strides (x_st, x_sc); weight: (channels, K) strides (w_sc, w_sk),
 * x's dtype; out: (total, channels) contiguous, x's dtype:
 *   out[t, c] = sum_{j < K} [t - (K-1-j) >= token_seq_starts[t]] x[t - (K-1-j), c] w[c, j]
 * accumulated in fp32 (fused multiply-add in tap order).  token_seq_starts / ends / slots:
 * (total,) int32, the packed start, end and state-table row of each token's sequence.
 * The last token of each sequence (t == ends[t] - 1) writes state_table[slot, c, j] =
 * x[ends - (K-1) + j, c] for j < K - 1 (0 before the sequence's start), in state_dtype;
 * state_table: (num_slots, channels, K - 1) strides (s_ss, s_sc, s_sk).  A slot outside
 * [0, num_slots) writes nothing.  2 <= K <= 8.
 */
int atma_packed_causal_conv1d(const void* x, int64_t x_st, int64_t x_sc, const void* weight, int64_t w_sc,
                              int64_t w_sk, void* out, void* state_table, int64_t s_ss, int64_t s_sc,
                              int64_t s_sk, int64_t num_slots, const int32_t* token_seq_starts,
                              const int32_t* token_seq_ends, const int32_t* token_seq_slots, int64_t total,
                              int64_t channels, int64_t K, int dtype, int state_dtype, void* stream);

/*
 * Gate activations of the memory branch in one launch.  Replaces the torch
 * add / logsigmoid / sigmoid of TitansMemory (model/blocks.py:426-490,
 * inference/models/atma.py:305-375): g = logsigmoid(zg + g_bias) -- the log-decay
 * atma_chunk_gated_delta_rule takes -- or, with decay_as_prob != 0, the decode step's
 * gamma = sigmoid(zg + g_bias); beta = sigmoid(zb + b_bias).  All fp32 contiguous,
 * n elements each.
 */
int atma_gated_delta_gates(const float* zg, const float* zb, float g_bias, float b_bias,
                           float* g, float* beta, int64_t n, int decay_as_prob, void* stream);

/*
 * Workspace bytes atma_chunk_gated_delta_rule needs for this shape and dtype.
 */
size_t atma_chunk_gated_delta_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t dk,
                                              int64_t dv, int64_t chunk, int dtype);

/*
 * Chunked gated-delta prefill with state carry.  Replaces the third-party
 * fla.ops.gated_delta_rule.chunk_gated_delta_rule as the reference calls it
 * (model/blocks.py:44-49, inference/models/atma.py:285-287,318-322), with the
 * arithmetic of gated_delta_chunked (model/blocks.py:375-423).
 * q: (B, T, H, dk), k: (B, T, Hkv, dk), v: (B, T, Hkv, dv) with H % Hkv == 0, strides
 * (x_sb, x_st, x_sh, 1) -- query head h reads k / v head h / (H / Hkv); Hkv == H is
 * the expanded form FLA and the reference use;
 * g (log-decay) and beta: (B, T, H) fp32 contiguous; initial_state (nullable =
 * zeros) and final_state (nullable = not written): (B, H, dk, dv) fp32 [K, V].
 * Output o: (B, T, H, dv) dtype contiguous.  q, k are L2-normalised when
 * use_qk_l2norm != 0, then q is multiplied by `scale`.  With gate_logits != 0, g and
 * beta hold the memory branch's raw gate logits and the kernel applies the activations
 * of atma_gated_delta_gates on load (log-decay logsigmoid(g + g_bias), write strength
 * sigmoid(beta + b_bias)), bit-identical to calling it first (an extension with no
 * FLA counterpart: one launch fewer for TitansMemory).  chunk must be 64;
 * dk = dv = 128 or 64.  start_flag (nullable; no FLA counterpart): the recurrence
 * kernel's first workgroup stores start_epoch there as it starts, for
 * atma_wait_start_flag; with a flag, 16-bit inputs take the unsegmented recurrence
 * (one workgroup per sequence-head and 32 columns, to run beside the caller's other
 * kernel), whose results can differ from the segmented one's in rounding.
 */
int atma_chunk_gated_delta_rule(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                                const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                                const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                                const float* g, const float* beta, const float* initial_state,
                                float* final_state, void* o, int64_t B, int64_t T, int64_t H,
                                int64_t Hkv, int64_t dk, int64_t dv, int dtype, float scale,
                                int use_qk_l2norm, int gate_logits, float g_bias, float b_bias,
                                int64_t chunk, void* workspace, size_t workspace_bytes,
                                int32_t* start_flag, int32_t start_epoch, void* stream);

/*
 * Launch-order helper with no counterpart in the reference: a one-wave kernel on
 * `stream` that returns once *flag == epoch (the store atma_chunk_gated_delta_rule's
 * recurrence kernel makes as it starts) or after timeout_us, whichever is first.
 * Work queued behind it on `stream` is therefore dispatched after the recurrence's
 * workgroups hold their CUs.  The overlapped prefill of the global layer uses it so that
 * Polar attention (which fills every CU) runs beside the latency-bound recurrence
 * instead of before it.  A timeout changes timing only, never results.
 * timeout_us in (0, 1e7].
 */
int atma_wait_start_flag(const int32_t* flag, int32_t epoch, int64_t timeout_us, void* stream);

/*
 * The decode step's soft cap and greedy pick in one pass (softcap_logits, then the
 * sampler's argmax for temperature-0 rows, inference/layers/sampler.py:5-10; no
 * reference counterpart as one call): per row, out = 15 x / sqrt(x^2 + 225) with
 * atma_softcap_logits' roundings (out may equal logits), and idx[row] = the index of the
 * largest out value, the first among equals, NaN above every number (torch.argmax).
 * 16-bit rows (16-byte vectors when every row is 16-byte aligned); one workgroup per row.
 */
int atma_softcap_argmax(const void* logits, int64_t ldx, void* out, int64_t ldo, int64_t* idx, int64_t rows,
                        int64_t V, int dtype, void* stream);

/*
 * Projection of a few token rows, with no counterpart in the reference (whose nn.Linear
 * calls the vendor GEMM, model/reference.py:22-28): y[m, n] = sum_k x[m, k] w[n, k]
 * (+ bias[n]) for M <= 32 rows, in 16 bits with fp32 accumulation and one rounding.  It
 * is the served model's decode projection (one token per sequence): the weights are
 * streamed once at memory speed, where a library GEMM tile walks K serially.  x (M, K),
 * w (N, K), y (M, N) row-major with row strides ldx, ldw, ldy (elements); bias (N,) or
 * NULL; dtype ATMA_BF16 / ATMA_F16.  x / w rows 16-byte aligned, y rows 8-byte aligned.
 * atma_linear_tokens_supported returns 1 for shapes the kernel serves (M <= 32,
 * N % 16 == 0, K 256, 512, 1024 or 2048), 0 otherwise.  Deterministic (fixed summation
 * order).
 */
int atma_linear_tokens_supported(int64_t M, int64_t N, int64_t K, int dtype);
int atma_linear_tokens(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, void* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype, void* stream);

/*
 * The same projection for up to 8 weight matrices that read one x (no reference
 * counterpart; the decode step's q / k / v / gate projections of a layer in one launch):
 * for s < n_segs, y[s][m, n] = sum_k x[m, k] w[s][n, k] (+ bias[s][n]), n < n[s].
 * Host arrays w, ldw, bias (entries may be NULL), y, ldy, n of n_segs entries; n[s] % 4
 * == 0; K 256, 512, 1024 or 2048; alignment as atma_linear_tokens.
 */
int atma_linear_tokens_multi(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t n_segs,
                             const void* const* w, const int64_t* ldw, const void* const* bias, void* const* y,
                             const int64_t* ldy, const int64_t* n, int dtype, void* stream);

/*
 * The MLP's first projection with its activation (model/layers.py:19-31; no reference
 * counterpart as one call): with w (2H, K) -- the a rows, then the gate rows -- and bias
 * (2H,) or NULL, y[m, n] = gate * relu(a)^2 for a = round(x[m] . w[n] + bias[n]),
 * gate = round(x[m] . w[H + n] + bias[H + n]), n < H, in squared_relu_gate's arithmetic.
 * H % 16 == 0; K, M and alignment as atma_linear_tokens.
 */
int atma_linear_tokens_gated(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, void* y,
                             int64_t ldy, int64_t M, int64_t H, int64_t K, int dtype, void* stream);

/*
 * The MLP's first projection with its activation over many token rows (model/layers.py:19-31,
 * inference/models/atma.py:87-96; no reference counterpart as one call): with w (2H, K) -- the
 * a rows, then the gate rows -- and bias (2H,) or NULL, y[m, n] = gate * relu(a)^2 for
 * a = round(x[m] . w[n] + bias[n]), gate = round(x[m] . w[H + n] + bias[H + n]), n < H, in
 * squared_relu_gate's arithmetic; each projection value is one fp32 sum rounded once (the
 * products' order is the kernel's).  The served prefill's MFMA GEMM: the 2H-wide projection
 * is never written.  x (M, K), w, y (M, H) row-major with row strides ldx, ldw, ldy; rows
 * 16-byte aligned, bias 4-byte aligned; H a multiple of 128, K of 128; x and w each under
 * 4 GiB.
 */
int atma_linear_gated(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, void* y,
                      int64_t ldy, int64_t M, int64_t H, int64_t K, int dtype, void* stream);

/*
 * The LFM2 block's in_proj and decode mixer in one call (model/reference.py:31-48,
 * inference/models/atma.py:625-673; no reference counterpart as one call): with w (3H, K)
 * -- the b rows, the c rows, the x rows -- and bias (3H,) or NULL, b, c, x of row m are
 * round(x[m] . w[n] + bias[n]) for the three blocks, and y[m, n] = c * conv(b * x) in
 * atma_lfm2_conv_step's arithmetic: taps (H, ktaps), state (max_seqs, H, ktaps - 1) with
 * row stride s_ss, row slots[m], advanced in place (a slot outside [0, max_seqs) yields NaN
 * outputs and leaves the table untouched).  Equal to atma_linear_tokens then
 * atma_lfm2_conv_step, bit for bit.  H % 16 == 0, 2 <= ktaps <= 4, max_seqs >= 1; K, M and
 * alignment as atma_linear_tokens.
 */
int atma_linear_tokens_conv(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                            const void* taps, int64_t ktaps, const int64_t* slots, void* state, int64_t s_ss,
                            int64_t max_seqs, void* y, int64_t ldy, int64_t M, int64_t H, int64_t K, int dtype,
                            void* stream);

/*
 * K split across workgroups, fp32 partial sums out (no reference counterpart; the decode
 * step's 4096-wide MLP projection and the global layer's two output projections):
 * parts[c][m][n] = sum_{k < chunk_k} x[m, c chunk_k + k] w[c][n, k] for c < n_chunks
 * (<= 8).  chunk_k 256, 512 or 1024; parts (n_chunks, M, N) fp32 contiguous, 16-byte
 * aligned; N % 4 == 0; no bias.
 */
int atma_linear_tokens_chunks(const void* x, int64_t ldx, int64_t M, int64_t chunk_k, int64_t n_chunks,
                              const void* const* w, const int64_t* ldw, int64_t N, float* parts, int dtype,
                              void* stream);

/*
 * Residual add + RMSNorm of the pre-norm block (inference/models/atma.py:680-713, norm
 * model/layers.py:6-16), no reference counterpart as one call: per row m,
 *   br  = round(y[m] or sum_p parts[p][m], + sum_i bias[i] + mu_x[m] . mu_w^T)  (y[m] itself when
 *         y comes with no bias and no low-rank term)
 *   s   = res ? round(res[m] + br) : br        (written to res_out when non-NULL)
 *   out = round(s * rsqrt(mean(s^2) + eps) * weight)
 * Exactly one of y / parts; parts (n_parts, M, D) fp32; up to 3 biases (D,); mu_x (M,
 * mu_k) and mu_w (D, mu_k), mu_k 4, 8 or 16 (the global layer's mu_proj(mag)); 16-bit rows,
 * D % 8 == 0, D <= 4096, every row 16-byte aligned.
 */
int atma_residual_rms_norm(const void* y, int64_t ldy, const float* parts, int64_t n_parts, const void* const* bias,
                           int64_t n_bias, const void* mu_x, int64_t ldmu, const void* mu_w, int64_t mu_k,
                           const void* res, int64_t ldr, void* res_out, int64_t ldro, const void* weight, void* out,
                           int64_t ldo, int64_t M, int64_t D, float eps, int dtype, void* stream);

/*
 * The LFM2 block's decode mixer (model/reference.py:31-48, inference/models/atma.py:
 * 625-673) as one call: with b, c, x the three D-wide thirds of each bcx row (in_proj's
 * output), out = c * conv(b * x), the depthwise conv of K taps (weight (D, K)) over the
 * sequence's last K - 1 values of b * x held in state (S, D, K - 1) row slots[b], which
 * is advanced in place.  Eager roundings: b * x, the conv, c * conv.  A slot outside
 * [0, max_seqs) yields NaN outputs and leaves the table untouched.
 */
int atma_lfm2_conv_step(const void* bcx, int64_t ld, const void* weight, int64_t K, const int64_t* slots,
                        void* state, int64_t s_ss, int64_t max_seqs, void* out, int64_t ldo, int64_t B, int64_t D,
                        int dtype, void* stream);

/*
 * The global layer's decode inputs from one fused projection row y[b] (q and its output
 * gate interleaved per head from column 0, k at ck, v at cv, gate logits at cg / cb;
 * inference/models/atma.py:546-575 and model/blocks.py:426-490), no reference
 * counterpart as one call: q, k = per-head rms_norm (eps), then q, k, v = x + conv(x),
 * the Canon depthwise convs (taps wq / wk / wv (C, Kc)) over state tables tq / tk / tv
 * (S, C, Kc - 1) row slots[b], advanced in place; gamma = exp(logsigmoid(z_g + g_bias)),
 * beta = sigmoid(z_b + b_bias) fp32 (B, H) unless gamma and beta are NULL.  q (B, H, d),
 * k, v (B, Hkv, d) contiguous; d 64 or 128; 16-bit.
 */
int atma_global_decode_prep(const void* y, int64_t ldy, int64_t ck, int64_t cv, int64_t cg, int64_t cb,
                            const void* wq, const void* wk, const void* wv, int64_t Kc, void* tq, int64_t tq_ss,
                            void* tk, int64_t tk_ss, void* tv, int64_t tv_ss, int64_t max_seqs, const int64_t* slots,
                            void* q, void* k, void* v, float* gamma, float* beta, float eps, float g_bias,
                            float b_bias, int64_t B, int64_t H, int64_t Hkv, int64_t d, int dtype, void* stream);

/*
 * Per-head RMSNorm of a strided view (no reference counterpart as one call; the global
 * layer's q / k norms, model/reference.py:136-137): out[m, h, :] = x[m, h, :] *
 * rsqrt(mean(x[m, h, :]^2) + eps), element (m, h, e) of x at m ldr + h ldh + e, out
 * (rows, H, d) contiguous.  d 64 or 128; 16-bit; 16-byte aligned heads.
 */
int atma_head_rms_norm(const void* x, int64_t ldr, int64_t ldh, void* out, int64_t rows, int64_t H, int64_t d,
                       float eps, int dtype, void* stream);

/*
 * The gated inputs of the global layer's output projections (inference/models/atma.py:
 * 246-252, model/blocks.py:470-490), no reference counterpart as one call.  Row m = b T + t:
 *   xa[m, h d + e] = c[b, t, h, e] * sigmoid(gate[m, h, e])
 *   xm[m, h d + e] = round(rms_norm(r[m, h, :])[e] (eps mem_eps)) * sigmoid(mgate[m, h d + e])
 * with c at b c_sb + t c_st + h c_sh + e (Polar's head-major output, or one row per sequence),
 * gate at m g_sr + h g_sh + e, r at m r_sr + h d + e (r_dtype ATMA_F32 or dtype), mgate at m mg_sr + h d + e; each
 * sigmoid and product rounded to 16 bits.  r NULL: no memory branch (xm, mgate unused).
 * d 64 or 128; every head-row 16-byte aligned.  atma_global_decode_gate is the decode
 * form: c (B, H, d) contiguous, the output gate of head h at y[b, 2 h d + d ..], the memory
 * gate at y[b, cm + h d ..], x2 = [xa | xm] per row.
 */
int atma_global_gate(const void* c, int64_t c_sb, int64_t c_st, int64_t c_sh, int64_t T, const void* gate,
                     int64_t g_sr, int64_t g_sh, const void* r, int64_t r_sr, int r_dtype, const void* mgate, int64_t mg_sr,
                     void* xa, int64_t a_sr, void* xm, int64_t m_sr, int64_t rows, int64_t H, int64_t d,
                     float mem_eps, int dtype, void* stream);
int atma_global_decode_gate(const void* c, const float* r, const void* y, int64_t ldy, int64_t cm, void* x2,
                            int64_t ldx2, float mem_eps, int64_t B, int64_t H, int64_t d, int dtype, void* stream);

/*
 * The LFM2 block's fresh-prefill mixer input over packed ragged sequences
 * (model/reference.py:31-48, inference/models/atma.py:625-673 with packed_causal_conv1d
 * :138-160), no reference counterpart as one call: with b, c, x the three D-wide thirds of
 * each bcx row, out[t] = c * conv(b * x)[t], the depthwise causal conv of K taps (weight
 * (D, K)) over each token's own sequence (token maps as atma_packed_causal_conv1d), and each
 * sequence's last K - 1 values of b * x (zero before its start) written to its row of state
 * (S, D, K - 1).  Eager roundings: b * x, the conv, c * conv.  K 3 or 4; 16-bit; D % 8 == 0.
 */
int atma_lfm2_conv_packed(const void* bcx, int64_t ld, const void* weight, int64_t K, void* out, int64_t ldo,
                          void* state, int64_t s_ss, int64_t num_slots, const int32_t* token_seq_starts,
                          const int32_t* token_seq_ends, const int32_t* token_seq_slots, int64_t total, int64_t D,
                          int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATMA_HIP_H */
