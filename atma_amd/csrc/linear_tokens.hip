// Projections of a few token rows: Y[m, n] = sum_k X[m, k] W[n, k] (+ bias[n]), m < 32.
//
// The served model's decode step multiplies one token per sequence (32 rows at configs[4])
// by every weight matrix of the model: 650 MB of bf16 weights per step against 64 KB of
// activations per matrix.  That is a weight stream, not a GEMM tile problem: a library
// tile of 32 x 32 outputs walks K serially and reads each weight slice through one
// workgroup, so a 2-16 MB matrix takes 8-12 us.  Here a workgroup owns 16 output features
// (32 for wide outputs) and its waves split K, 256 per wave; every MFMA operand comes straight
// from memory in the lane layout of v_mfma_f32_16x16x32 (A lane l: weight row l % 16,
// k = 8 (l / 16) .. + 7, one 16-byte load; B lane l: token row l % 16, the same k), a wave
// issues the loads
// of all eight of its 32-wide K steps before its first product (one memory latency per
// launch), weights with the non-temporal hint (read once per step) and the activation rows
// through L2 (read by every workgroup).  The waves' partial sums are added in a fixed
// order through LDS (deterministic), then the bias in fp32 and one rounding to the output
// type.
//
// No reference counterpart: the reference's nn.Linear calls the vendor GEMM
// (model/reference.py:22-28); this is the engine's kernel for that call at decode shapes.

#include "common.h"

namespace atma {

struct LinTokArgs {
  const void* x;  // (M, K), row stride ldx
  int64_t ldx;
  const void* w;  // (N, K), row stride ldw
  int64_t ldw;
  const void* bias;  // (N,) or null
  void* y;           // (M, N), row stride ldy
  int64_t ldy;
  int M, N, K;
};

constexpr int kLinKPerWave = 256;  // K per wave: eight 32-wide steps, all loaded at once
constexpr int kLinSteps = kLinKPerWave / 32;
constexpr int kLinMaxWaves = 8;

// NW waves per workgroup (K = NW * 256); FT 16-feature tiles per workgroup, which share
// each activation load (for wide outputs, where the activation rows would otherwise be
// read from L2 once per 16 features)
template <typename T, int NW, int FT>
__global__ void __launch_bounds__(64 * NW) linear_tokens_kernel(LinTokArgs a) {
  __shared__ f32x4 red[NW - 1][FT][2][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int f0 = blockIdx.x * 16 * FT;
  const int k0 = wave * kLinKPerWave + 8 * g;
  const T* X = (const T*)a.x;
  const T* W = (const T*)a.w;
  // token rows r and 16 + r (rows past M read row M - 1 and are zeroed: no divergent loads)
  const bool ok0 = r < a.M, ok1 = 16 + r < a.M;
  const T* x0 = X + (int64_t)min(r, a.M - 1) * a.ldx + k0;
  const T* x1 = X + (int64_t)min(16 + r, a.M - 1) * a.ldx + k0;

  u32x4 wv[kLinSteps][FT], xv0[kLinSteps], xv1[kLinSteps];
#pragma unroll
  for (int u = 0; u < kLinSteps; ++u) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
      wv[u][f] = __builtin_nontemporal_load((const u32x4*)(W + (int64_t)(f0 + 16 * f + r) * a.ldw + k0 + 32 * u));
    xv0[u] = *(const u32x4*)(x0 + 32 * u);
    xv1[u] = *(const u32x4*)(x1 + 32 * u);
  }
  const u32x4 zero = {0u, 0u, 0u, 0u};
  f32x4 acc[FT][2];
#pragma unroll
  for (int f = 0; f < FT; ++f) acc[f][0] = acc[f][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kLinSteps; ++u) {
    const u32x4 b0 = ok0 ? xv0[u] : zero, b1 = ok1 ? xv1[u] : zero;
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      acc[f][0] = mfma16x16x32<T>(wv[u][f], b0, acc[f][0]);
      acc[f][1] = mfma16x16x32<T>(wv[u][f], b1, acc[f][1]);
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      red[wave - 1][f][0][lane] = acc[f][0];
      red[wave - 1][f][1][lane] = acc[f][1];
    }
  }
  __syncthreads();
  if (wave > 0) return;
  // lane l holds features 4 (l / 16) + [0, 4) of tile f, token 16 t + l % 16
  T* Y = (T*)a.y;
#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int n = f0 + 16 * f + 4 * g;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (a.bias) {
      const T* bp = (const T*)a.bias + n;
      bv = f32x4{to_f32(bp[0]), to_f32(bp[1]), to_f32(bp[2]), to_f32(bp[3])};
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 v = acc[f][t];
#pragma unroll
      for (int w = 0; w < NW - 1; ++w) v += red[w][f][t][lane];
      v += bv;
      const int m = 16 * t + r;
      if (m < a.M) {
        const u32x2 pk = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
        *(u32x2*)(Y + (int64_t)m * a.ldy + n) = pk;
      }
    }
  }
}

template <typename T>
static void launch_linear_tokens(const LinTokArgs& a, hipStream_t s) {
  const bool wide = a.N >= 4096 && a.N % 32 == 0;
  const dim3 grid((unsigned)(a.N / (wide ? 32 : 16)));
  if (a.K == 1024) {
    if (wide) linear_tokens_kernel<T, 4, 2><<<grid, dim3(256), 0, s>>>(a);
    else linear_tokens_kernel<T, 4, 1><<<grid, dim3(256), 0, s>>>(a);
  } else {
    if (wide) linear_tokens_kernel<T, 8, 2><<<grid, dim3(512), 0, s>>>(a);
    else linear_tokens_kernel<T, 8, 1><<<grid, dim3(512), 0, s>>>(a);
  }
}

}  // namespace atma

extern "C" int atma_linear_tokens_supported(int64_t M, int64_t N, int64_t K, int dtype) {
  return (dtype == ATMA_BF16 || dtype == ATMA_F16) && M >= 1 && M <= 32 && N >= 16 && N % 16 == 0 &&
                 (K == 1024 || K == 2048) && N <= (1 << 24)
             ? 1
             : 0;
}

extern "C" int atma_linear_tokens(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                                  void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                                  void* stream) {
  using namespace atma;
  if (!atma_linear_tokens_supported(M, N, K, dtype))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_tokens: unsupported shape M=%lld N=%lld K=%lld dtype=%d (16-bit, M <= 32, "
                     "N %% 16 == 0, K 1024 or 2048)",
                     (long long)M, (long long)N, (long long)K, dtype);
  if (!x || !w || !y) return set_error(ATMA_ERR_INVALID, "linear_tokens: null pointer");
  if (ldx < K || ldw < K || ldy < N) return set_error(ATMA_ERR_INVALID, "linear_tokens: row stride below row length");
  if ((uintptr_t)x % 16 || (uintptr_t)w % 16 || (uintptr_t)y % 8 || ldx % 8 || ldw % 8 || ldy % 4 ||
      (bias && (uintptr_t)bias % 2))
    return set_error(ATMA_ERR_INVALID, "linear_tokens: x / w rows must be 16-byte aligned, y rows 8-byte aligned");
  LinTokArgs a{x, ldx, w, ldw, bias, y, ldy, (int)M, (int)N, (int)K};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16) launch_linear_tokens<bf16>(a, s);
  else launch_linear_tokens<f16>(a, s);
  return check_launch("linear_tokens");
}
