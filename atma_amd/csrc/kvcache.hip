// Paged KV write: bit-exact scatter of token rows into cache slots.
//
// Reference: store_kvcache, inference/layers/attention.py:7-56 (one program per
// token, slot -1 skipped).  Here one thread moves one 16/8/4/2-byte vector of a
// row; the widest vector the pointers and strides allow is chosen on the host, so
// a 512-byte (Hkv=2, d=128, bf16) row is 32 lanes of 16-byte loads/stores.
#include "common.h"

namespace atma {

template <typename V>
__global__ void __launch_bounds__(256)
store_kvcache_kernel(const V* __restrict__ key, int64_t key_stride, const V* __restrict__ value,
                     int64_t value_stride, V* __restrict__ k_cache, V* __restrict__ v_cache,
                     const int32_t* __restrict__ slot_mapping, int64_t n_tokens, int64_t row_vecs,
                     int64_t total_slots) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t tok = idx / row_vecs;
  if (tok >= n_tokens) return;
  const int64_t i = idx - tok * row_vecs;
  const int64_t slot = slot_mapping[tok];
  if (slot < 0 || slot >= total_slots) return;
  k_cache[slot * row_vecs + i] = key[tok * key_stride + i];
  v_cache[slot * row_vecs + i] = value[tok * value_stride + i];
}

template <typename V>
static int launch_store(const void* key, int64_t ks, const void* value, int64_t vs, void* kc,
                        void* vc, const int32_t* slots, int64_t n, int64_t row_bytes,
                        int64_t total_slots, hipStream_t stream) {
  const int64_t row_vecs = row_bytes / (int64_t)sizeof(V);
  const int64_t total = n * row_vecs;
  const int64_t blocks = (total + 255) / 256;
  store_kvcache_kernel<V><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
      (const V*)key, ks / (int64_t)sizeof(V), (const V*)value, vs / (int64_t)sizeof(V), (V*)kc,
      (V*)vc, slots, n, row_vecs, total_slots);
  return check_launch("store_kvcache");
}

}  // namespace atma

extern "C" int atma_store_kvcache(const void* key, int64_t key_stride, const void* value,
                                  int64_t value_stride, void* k_cache, void* v_cache,
                                  const int32_t* slot_mapping, int64_t n_tokens, int64_t row_elems,
                                  int64_t total_slots, int dtype, void* stream) {
  using namespace atma;
  const int es = dtype_size(dtype);
  if (!es) return set_error(ATMA_ERR_INVALID, "store_kvcache: unknown dtype %d", dtype);
  if (n_tokens < 0 || row_elems <= 0 || total_slots < 0)
    return set_error(ATMA_ERR_INVALID, "store_kvcache: bad sizes n=%lld row=%lld slots=%lld",
                     (long long)n_tokens, (long long)row_elems, (long long)total_slots);
  if (n_tokens == 0) return ATMA_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return set_error(ATMA_ERR_INVALID, "store_kvcache: null pointer");
  if (key_stride < row_elems || value_stride < row_elems)
    return set_error(ATMA_ERR_INVALID, "store_kvcache: token stride smaller than the row");
  if ((uint64_t)n_tokens * (uint64_t)row_elems > (1ull << 40))
    return set_error(ATMA_ERR_INVALID, "store_kvcache: too many elements");
  const int64_t row_bytes = row_elems * es, ksb = key_stride * es, vsb = value_stride * es;
  auto aligned = [&](int64_t a) {
    return ((uintptr_t)key % a == 0) && ((uintptr_t)value % a == 0) &&
           ((uintptr_t)k_cache % a == 0) && ((uintptr_t)v_cache % a == 0) && (row_bytes % a == 0) &&
           (ksb % a == 0) && (vsb % a == 0);
  };
  hipStream_t s = (hipStream_t)stream;
  if (aligned(16))
    return launch_store<u32x4>(key, ksb, value, vsb, k_cache, v_cache, slot_mapping, n_tokens,
                               row_bytes, total_slots, s);
  if (aligned(4))
    return launch_store<uint32_t>(key, ksb, value, vsb, k_cache, v_cache, slot_mapping, n_tokens,
                                  row_bytes, total_slots, s);
  return launch_store<uint16_t>(key, ksb, value, vsb, k_cache, v_cache, slot_mapping, n_tokens,
                                row_bytes, total_slots, s);
}
