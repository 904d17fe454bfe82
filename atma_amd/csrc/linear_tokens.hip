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
// issues the loads of all eight of its 32-wide K steps before its first product (one memory
// latency per launch), weights with the non-temporal hint (read once per step) and the
// activation rows through L2 (read by every workgroup).  The waves' partial sums are added
// in a fixed order through LDS (deterministic).
//
// Two launch forms share the kernel:
//  * segments: up to 8 weight matrices that read the same activations (the q / k / v /
//    gate projections of one layer), each with its own bias and output rows; the launch's
//    workgroups are laid over the segments' 16-feature tiles one after another, so the
//    projections cost one launch.  Bias added in fp32, one rounding to the output type.
//  * gated: the MLP's first projection with its activation, h[m, n] = gate * relu(a)^2
//    of a = (x W^T + b)[m, n], gate = (x W^T + b)[m, H + n] (each rounded to the output
//    type first, then squared_relu_gate's arithmetic): a workgroup computes the a and
//    gate tiles of the same 16 features, so the 2H-wide projection is never written.
//  * conv: the LFM2 block's in_proj with its gated conv step, h = c * conv(b * x) for
//    b, c, x = (x W^T + bias).chunk(3) (each rounded to the output type, then
//    lfm2_conv_step's arithmetic, the channel's conv state advanced in place; 2 to 4 taps): a
//    workgroup computes the b, c and x tiles of the same 16 channels, so the 3H-wide
//    projection is never written and the conv step costs no launch of its own.
//  * chunks: K split into chunks of 256-1024 across workgroups (blockIdx.y), chunk c with its
//    own weight pointer, writing fp32 partial sums parts[c] (no bias, no rounding) for the
//    consumer to add in chunk order (the residual RMSNorm).  That spreads a 4096-wide
//    projection over 4x the workgroups, and lets two projections of different inputs whose
//    outputs are summed (the global layer's output and memory projections) run as one.
//
// No reference counterpart: the reference's nn.Linear calls the vendor GEMM
// (model/reference.py:22-28); this is the engine's kernel for that call at decode shapes.

#include "common.h"

namespace atma {

constexpr int kLinKPerWave = 256;  // K per wave: eight 32-wide steps, all loaded at once
constexpr int kLinSteps = kLinKPerWave / 32;
constexpr int kLinMaxSegs = 8;
constexpr int kLinMaxChunks = 8;
constexpr int kLinMaxWaves = 8;  // K per launch (segments) up to 2048, per chunk up to 1024

struct LinSeg {
  const void* w;  // (n, K), row stride ldw
  int64_t ldw;
  const void* bias;  // (n,) or null
  void* y;           // (M, n), row stride ldy
  int64_t ldy;
  int n;
  int tile0;  // the segment's first tile in the launch
};

struct LinTokArgs {
  const void* x;  // (M, *), row stride ldx
  int64_t ldx;
  int M;
  // segments form
  int n_segs;
  LinSeg seg[kLinMaxSegs];
  // chunks form: chunk c reads x columns [c K, c K + K) and weights cw[c] (N, K) with row
  // stride cldw[c]
  const void* cw[kLinMaxChunks];
  int64_t cldw[kLinMaxChunks];
  float* parts;  // (chunks, M, N) fp32
  int N;
  // conv form: depthwise taps (n, ktaps) and the state table (max_seqs, n, ktaps - 1) rows slots[m]
  const void* taps;
  int ktaps;
  const int64_t* slots;
  void* state;
  int64_t s_ss, max_seqs;
};

// kLinGated and kLinConv use segment 0: its n is H, its weight has 2H rows (a, then gate) or
// 3H rows (b, c, x), its output H
enum LinMode { kLinSegments = 0, kLinChunks = 1, kLinGated = 2, kLinConv = 3 };

// NW waves per workgroup (K per launch or chunk = NW * 256, NW <= kLinMaxWaves); FT 16-feature tiles per
// workgroup, which share each activation load; KT the conv form's taps (2 to 4)
template <typename T, int NW, int FT, int MODE, int KT = 0>
__global__ void __launch_bounds__(64 * NW) linear_tokens_kernel(LinTokArgs a) {
  __shared__ f32x4 red[NW > 1 ? NW - 1 : 1][FT][2][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int tile = blockIdx.x;

  // this workgroup's weights, feature range and activation columns (constant-index
  // selects over the argument arrays, so they stay in scalar registers)
  const void* wp = nullptr;
  int64_t ldw = 0, xoff = 0;
  int f0 = 0, n_lim = 0, seg = 0;
  if constexpr (MODE == kLinSegments) {
#pragma unroll
    for (int s = 1; s < kLinMaxSegs; ++s)
      if (s < a.n_segs && tile >= a.seg[s].tile0) seg = s;
#pragma unroll
    for (int s = 0; s < kLinMaxSegs; ++s)
      if (s == seg) {
        wp = a.seg[s].w;
        ldw = a.seg[s].ldw;
        n_lim = a.seg[s].n;
        f0 = (tile - a.seg[s].tile0) * 16 * FT;
      }
  } else if constexpr (MODE == kLinGated || MODE == kLinConv) {
    static_assert(MODE == kLinGated ? FT == 2 : FT == 3,
                  "the gated form pairs an a tile with its gate tile, the conv form takes b, c and x tiles");
    wp = a.seg[0].w;
    ldw = a.seg[0].ldw;
    n_lim = a.seg[0].n;
    f0 = tile * 16;
  } else {
    const int c = blockIdx.y;
#pragma unroll
    for (int s = 0; s < kLinMaxChunks; ++s)
      if (s == c) {
        wp = a.cw[s];
        ldw = a.cldw[s];
      }
    n_lim = a.N;
    f0 = tile * 16 * FT;
    xoff = (int64_t)c * (NW * kLinKPerWave);
  }
  const int k0 = wave * kLinKPerWave + 8 * g;
  const T* X = (const T*)a.x;
  const T* W = (const T*)wp;
  // token rows r and 16 + r (rows past M read row M - 1 and are zeroed: no divergent loads)
  const bool ok0 = r < a.M, ok1 = 16 + r < a.M;
  const T* x0 = X + (int64_t)min(r, a.M - 1) * a.ldx + xoff + k0;
  const T* x1 = X + (int64_t)min(16 + r, a.M - 1) * a.ldx + xoff + k0;

  u32x4 wv[kLinSteps][FT], xv0[kLinSteps], xv1[kLinSteps];
#pragma unroll
  for (int u = 0; u < kLinSteps; ++u) {
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      // rows past the segment are clamped and discarded; the gated and conv forms' tile f
      // is block f (a / gate, or b / c / x) of the same features
      const int row = MODE == kLinGated || MODE == kLinConv ? f * n_lim + f0 + r : min(f0 + 16 * f + r, n_lim - 1);
      wv[u][f] = __builtin_nontemporal_load((const u32x4*)(W + (int64_t)row * ldw + k0 + 32 * u));
    }
    xv0[u] = *(const u32x4*)(x0 + 32 * u);
    xv1[u] = *(const u32x4*)(x1 + 32 * u);
  }
  // conv form: the epilogue's small operands (biases, taps, the tokens' state slots) go out
  // behind the projection's loads, unconditionally (a missing bias reads x and is not used;
  // rows past M read row M - 1), so no wait of the epilogue stands alone
  constexpr int KS = KT > 1 ? KT - 1 : 1;
  T cbias[3][4], ctap[4][KT > 0 ? KT : 1];
  int64_t cslot[2];
  if constexpr (MODE == kLinConv) {
    static_assert(KT >= 2 && KT <= 4, "the conv form takes 2 to 4 taps");
    const int n = f0 + 4 * g;
    const T* bsrc = a.seg[0].bias ? (const T*)a.seg[0].bias : X;
    const int bstep = a.seg[0].bias ? 1 : 0;
#pragma unroll
    for (int f = 0; f < 3; ++f)
#pragma unroll
      for (int e = 0; e < 4; ++e) cbias[f][e] = bsrc[bstep * (f * n_lim + n + e)];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int j = 0; j < KT; ++j) ctap[e][j] = ((const T*)a.taps)[(int64_t)(n + e) * KT + j];
    cslot[0] = a.slots[min(r, a.M - 1)];
    cslot[1] = a.slots[min(16 + r, a.M - 1)];
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
  // conv form: the state rows of the tokens' channels, read before the partial sums meet
  // (a token without a state row reads row 0 and discards it)
  T cold[2][4][KS];
  if constexpr (MODE == kLinConv) {
    const int n = f0 + 4 * g;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t slot = cslot[t] >= 0 && cslot[t] < a.max_seqs ? cslot[t] : 0;
      const T* st = (const T*)a.state + slot * a.s_ss + (int64_t)n * KS;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < KS; ++j) cold[t][e][j] = st[e * KS + j];
    }
  }

  if constexpr (NW > 1) {
    if (wave > 0) {
#pragma unroll
      for (int f = 0; f < FT; ++f) {
        red[wave - 1][f][0][lane] = acc[f][0];
        red[wave - 1][f][1][lane] = acc[f][1];
      }
    }
    __syncthreads();
    if (wave > 0) return;
  }
  // lane l holds features 4 (l / 16) + [0, 4) of tile f, token 16 t + l % 16
  auto reduced = [&](int f, int t) {
    f32x4 v = acc[f][t];
#pragma unroll
    for (int w = 0; w < NW - 1; ++w) v += red[w][f][t][lane];
    return v;
  };
  auto bias4 = [&](const void* b, int n) {
    if (!b) return f32x4{0.f, 0.f, 0.f, 0.f};
    const T* bp = (const T*)b + n;
    return f32x4{to_f32(bp[0]), to_f32(bp[1]), to_f32(bp[2]), to_f32(bp[3])};
  };
  if constexpr (MODE == kLinGated) {
    const int n = f0 + 4 * g;
    const f32x4 ba = bias4(a.seg[0].bias, n), bg = bias4(a.seg[0].bias, n_lim + n);
    T* Y = (T*)a.seg[0].y;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const f32x4 va = reduced(0, t) + ba, vg = reduced(1, t) + bg;
      const int m = 16 * t + r;
      if (m >= a.M) continue;
      float h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = sq_relu_gate1<T>(to_f32(from_f32<T>(va[e])), to_f32(from_f32<T>(vg[e])));
      const u32x2 pk = {pack2<T>(h[0], h[1]), pack2<T>(h[2], h[3])};
      *(u32x2*)(Y + (int64_t)m * a.seg[0].ldy + n) = pk;
    }
    return;
  }
  if constexpr (MODE == kLinConv) {
    const int n = f0 + 4 * g;
    T* Y = (T*)a.seg[0].y;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 v[3];
#pragma unroll
      for (int f = 0; f < 3; ++f) {
        v[f] = reduced(f, t);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[f][e] += a.seg[0].bias ? to_f32(cbias[f][e]) : 0.f;
      }
      const int m = 16 * t + r;
      if (m >= a.M) continue;
      T* Ym = Y + (int64_t)m * a.seg[0].ldy + n;
      if (cslot[t] < 0 || cslot[t] >= a.max_seqs) {  // no state row: the output says so
        // (the scalar conversion's NaN, as lfm2_conv_step writes it)
        const uint32_t nb = __builtin_bit_cast(uint16_t, from_f32<T>(__builtin_nanf("")));
        *(u32x2*)Ym = u32x2{nb | nb << 16, nb | nb << 16};
        continue;
      }
      T* st = (T*)a.state + cslot[t] * a.s_ss + (int64_t)n * KS;
      float h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // lfm2_conv_step on the rounded projections b, c, x: newest tap first, then the
        // state's inputs oldest first; the state shifts and takes the new input
        const float bx = to_f32(from_f32<T>(to_f32(from_f32<T>(v[0][e])) * to_f32(from_f32<T>(v[2][e]))));
        // fused multiply-adds in lfm2_conv_step's order (written out: unrolled, the first
        // product could otherwise be the one fused)
        float acc = bx * to_f32(ctap[e][KT - 1]);
#pragma unroll
        for (int j = 0; j < KS; ++j) {
          acc = __builtin_fmaf(to_f32(cold[t][e][j]), to_f32(ctap[e][j]), acc);
          if (j > 0) st[e * KS + j - 1] = cold[t][e][j];
        }
        st[e * KS + KS - 1] = from_f32<T>(bx);
        // the sum is rounded to fp32 and then to T, as in lfm2_conv_step: kept as an fp32
        // register, the last multiply-add cannot fold into a mixed-precision one that rounds
        // to T directly (v_fma_mixlo: one rounding instead of two, which moves ties)
        asm volatile("" : "+v"(acc));
        h[e] = to_f32(from_f32<T>(v[1][e])) * to_f32(from_f32<T>(acc));
      }
      // scalar conversions, as lfm2_conv_step rounds (the packed conversion can differ from
      // them on fp16 subnormals)
      uint32_t hb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) hb[e] = __builtin_bit_cast(uint16_t, from_f32<T>(h[e]));
      *(u32x2*)Ym = u32x2{hb[0] | hb[1] << 16, hb[2] | hb[3] << 16};
    }
    return;
  }
#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int n = f0 + 16 * f + 4 * g;  // n_lim % 4 == 0: a lane's four features are all in or all out
    if (n >= n_lim) continue;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    T* Y = nullptr;
    int64_t ldy = 0;
    if constexpr (MODE == kLinSegments) {
#pragma unroll
      for (int s = 0; s < kLinMaxSegs; ++s)
        if (s == seg) {
          Y = (T*)a.seg[s].y;
          ldy = a.seg[s].ldy;
          bv = bias4(a.seg[s].bias, n);
        }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 v = reduced(f, t);
      const int m = 16 * t + r;
      if (m >= a.M) continue;
      if constexpr (MODE == kLinSegments) {
        v += bv;
        const u32x2 pk = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
        *(u32x2*)(Y + (int64_t)m * ldy + n) = pk;
      } else {
        *(f32x4*)(a.parts + ((int64_t)blockIdx.y * a.M + m) * a.N + n) = v;
      }
    }
  }
}

template <typename T, int NW>
static void launch_segments(const LinTokArgs& a, int tiles, bool wide, hipStream_t s) {
  const dim3 grid((unsigned)tiles);
  if (wide) linear_tokens_kernel<T, NW, 2, kLinSegments><<<grid, dim3(64 * NW), 0, s>>>(a);
  else linear_tokens_kernel<T, NW, 1, kLinSegments><<<grid, dim3(64 * NW), 0, s>>>(a);
}

template <typename T, int NW>
static void launch_chunks(const LinTokArgs& a, int chunks, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 15) / 16), (unsigned)chunks);
  linear_tokens_kernel<T, NW, 1, kLinChunks><<<grid, dim3(64 * NW), 0, s>>>(a);
}

template <typename T, int NW>
static void launch_gated(const LinTokArgs& a, hipStream_t s) {
  linear_tokens_kernel<T, NW, 2, kLinGated><<<dim3((unsigned)(a.seg[0].n / 16)), dim3(64 * NW), 0, s>>>(a);
}

template <typename T, int NW>
static void launch_conv(const LinTokArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.seg[0].n / 16)), block(64 * NW);
  switch (a.ktaps) {
    case 2: linear_tokens_kernel<T, NW, 3, kLinConv, 2><<<grid, block, 0, s>>>(a); break;
    case 3: linear_tokens_kernel<T, NW, 3, kLinConv, 3><<<grid, block, 0, s>>>(a); break;
    default: linear_tokens_kernel<T, NW, 3, kLinConv, 4><<<grid, block, 0, s>>>(a); break;
  }
}

template <typename T>
static void launch_conv_k(const LinTokArgs& a, int64_t K, hipStream_t s) {
  switch (K) {
    case 256: launch_conv<T, 1>(a, s); break;
    case 512: launch_conv<T, 2>(a, s); break;
    case 1024: launch_conv<T, 4>(a, s); break;
    default: launch_conv<T, 8>(a, s); break;
  }
}

template <typename T>
static void launch_segments_k(const LinTokArgs& a, int64_t K, int tiles, bool wide, hipStream_t s) {
  switch (K) {
    case 256: launch_segments<T, 1>(a, tiles, wide, s); break;
    case 512: launch_segments<T, 2>(a, tiles, wide, s); break;
    case 1024: launch_segments<T, 4>(a, tiles, wide, s); break;
    default: launch_segments<T, 8>(a, tiles, wide, s); break;
  }
}

template <typename T>
static void launch_chunks_k(const LinTokArgs& a, int64_t chunk_k, int chunks, hipStream_t s) {
  switch (chunk_k) {
    case 256: launch_chunks<T, 1>(a, chunks, s); break;
    case 512: launch_chunks<T, 2>(a, chunks, s); break;
    default: launch_chunks<T, 4>(a, chunks, s); break;
  }
}

template <typename T>
static void launch_gated_k(const LinTokArgs& a, int64_t K, hipStream_t s) {
  switch (K) {
    case 256: launch_gated<T, 1>(a, s); break;
    case 512: launch_gated<T, 2>(a, s); break;
    case 1024: launch_gated<T, 4>(a, s); break;
    default: launch_gated<T, 8>(a, s); break;
  }
}

static bool lin_common_ok(int64_t M, int dtype) {
  return (dtype == ATMA_BF16 || dtype == ATMA_F16) && M >= 1 && M <= 32;
}
static bool lin_k_ok(int64_t K, int max_waves) {
  return K == 256 || K == 512 || K == 1024 || (max_waves >= 8 && K == 2048);
}

}  // namespace atma

extern "C" int atma_linear_tokens_supported(int64_t M, int64_t N, int64_t K, int dtype) {
  return atma::lin_common_ok(M, dtype) && N >= 16 && N % 16 == 0 && atma::lin_k_ok(K, 8) && N <= (1 << 24)
             ? 1
             : 0;
}

extern "C" int atma_linear_tokens_multi(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t n_segs,
                                        const void* const* w, const int64_t* ldw, const void* const* bias,
                                        void* const* y, const int64_t* ldy, const int64_t* n, int dtype,
                                        void* stream) {
  using namespace atma;
  if (!lin_common_ok(M, dtype) || !lin_k_ok(K, kLinMaxWaves))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_tokens: unsupported shape M=%lld K=%lld dtype=%d (16-bit, 1 <= M <= 32, K 256, 512, "
                     "1024 or 2048)",
                     (long long)M, (long long)K, dtype);
  if (n_segs < 1 || n_segs > kLinMaxSegs)
    return set_error(ATMA_ERR_INVALID, "linear_tokens: 1 to %d weight segments, got %lld", kLinMaxSegs,
                     (long long)n_segs);
  if (!x || !w || !ldw || !bias || !y || !ldy || !n) return set_error(ATMA_ERR_INVALID, "linear_tokens: null pointer");
  if ((uintptr_t)x % 16 || ldx % 8 || ldx < K)
    return set_error(ATMA_ERR_INVALID, "linear_tokens: x rows must be 16-byte aligned and at least K long");
  LinTokArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.M = (int)M;
  a.n_segs = (int)n_segs;
  bool wide = true;
  int64_t total = 0;
  for (int s = 0; s < n_segs; ++s) {
    if (!w[s] || !y[s]) return set_error(ATMA_ERR_INVALID, "linear_tokens: null pointer in segment %d", s);
    if (n[s] < 4 || n[s] % 4 || n[s] > (1 << 24))
      return set_error(ATMA_ERR_INVALID, "linear_tokens: segment %d has %lld features (a multiple of 4 needed)", s,
                       (long long)n[s]);
    if ((uintptr_t)w[s] % 16 || ldw[s] % 8 || ldw[s] < K || (uintptr_t)y[s] % 8 || ldy[s] % 4 || ldy[s] < n[s] ||
        (bias[s] && (uintptr_t)bias[s] % 2))
      return set_error(ATMA_ERR_INVALID,
                       "linear_tokens: segment %d: weight rows must be 16-byte aligned, output rows 8-byte aligned", s);
    wide = wide && n[s] % 32 == 0;
    total += n[s];
  }
  wide = wide && total >= 4096;
  int tiles = 0;
  for (int s = 0; s < n_segs; ++s) {
    const int per = wide ? 32 : 16;
    a.seg[s] = LinSeg{w[s], ldw[s], bias[s], y[s], ldy[s], (int)n[s], tiles};
    tiles += (int)((n[s] + per - 1) / per);
  }
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ATMA_BF16) launch_segments_k<bf16>(a, K, tiles, wide, st);
  else launch_segments_k<f16>(a, K, tiles, wide, st);
  return check_launch("linear_tokens");
}

extern "C" int atma_linear_tokens(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                                  void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                                  void* stream) {
  using namespace atma;
  if (!atma_linear_tokens_supported(M, N, K, dtype))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_tokens: unsupported shape M=%lld N=%lld K=%lld dtype=%d (16-bit, M <= 32, "
                     "N %% 16 == 0, K 256, 512, 1024 or 2048)",
                     (long long)M, (long long)N, (long long)K, dtype);
  if (!x || !w || !y) return set_error(ATMA_ERR_INVALID, "linear_tokens: null pointer");
  if (ldy < N) return set_error(ATMA_ERR_INVALID, "linear_tokens: row stride below row length");
  return atma_linear_tokens_multi(x, ldx, M, K, 1, &w, &ldw, &bias, &y, &ldy, &N, dtype, stream);
}

extern "C" int atma_linear_tokens_gated(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                                        void* y, int64_t ldy, int64_t M, int64_t H, int64_t K, int dtype,
                                        void* stream) {
  using namespace atma;
  if (!lin_common_ok(M, dtype) || !lin_k_ok(K, kLinMaxWaves) || H < 16 || H % 16 || H > (1 << 23))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_tokens_gated: unsupported shape M=%lld H=%lld K=%lld dtype=%d (16-bit, 1 <= M <= 32, "
                     "H %% 16 == 0, K 256, 512, 1024 or 2048)",
                     (long long)M, (long long)H, (long long)K, dtype);
  if (!x || !w || !y) return set_error(ATMA_ERR_INVALID, "linear_tokens_gated: null pointer");
  if ((uintptr_t)x % 16 || ldx % 8 || ldx < K || (uintptr_t)w % 16 || ldw % 8 || ldw < K || (uintptr_t)y % 8 ||
      ldy % 4 || ldy < H || (bias && (uintptr_t)bias % 2))
    return set_error(ATMA_ERR_INVALID,
                     "linear_tokens_gated: x / w rows must be 16-byte aligned and y rows 8-byte aligned");
  LinTokArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.M = (int)M;
  a.n_segs = 1;
  a.seg[0] = LinSeg{w, ldw, bias, y, ldy, (int)H, 0};
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ATMA_BF16) launch_gated_k<bf16>(a, K, st);
  else launch_gated_k<f16>(a, K, st);
  return check_launch("linear_tokens_gated");
}

extern "C" int atma_linear_tokens_conv(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                                       const void* taps, int64_t ktaps, const int64_t* slots, void* state,
                                       int64_t s_ss, int64_t max_seqs, void* y, int64_t ldy, int64_t M, int64_t H,
                                       int64_t K, int dtype, void* stream) {
  using namespace atma;
  if (!lin_common_ok(M, dtype) || !lin_k_ok(K, kLinMaxWaves) || H < 16 || H % 16 || H > (1 << 22) || ktaps < 2 ||
      ktaps > 4)
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_tokens_conv: unsupported shape M=%lld H=%lld K=%lld taps=%lld dtype=%d (16-bit, "
                     "1 <= M <= 32, H %% 16 == 0, K 256, 512, 1024 or 2048, 2 to 4 taps)",
                     (long long)M, (long long)H, (long long)K, (long long)ktaps, dtype);
  if (!x || !w || !taps || !y || !slots || !state)
    return set_error(ATMA_ERR_INVALID, "linear_tokens_conv: null pointer");
  if ((uintptr_t)x % 16 || ldx % 8 || ldx < K || (uintptr_t)w % 16 || ldw % 8 || ldw < K || (uintptr_t)y % 8 ||
      ldy % 4 || ldy < H || (bias && (uintptr_t)bias % 2) || (uintptr_t)taps % 2 || (uintptr_t)state % 2 ||
      max_seqs < 1 || s_ss < H * (ktaps - 1))
    return set_error(ATMA_ERR_INVALID,
                     "linear_tokens_conv: x / w rows must be 16-byte aligned, y rows 8-byte aligned, state rows "
                     "(H, taps - 1)");
  LinTokArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.M = (int)M;
  a.n_segs = 1;
  a.seg[0] = LinSeg{w, ldw, bias, y, ldy, (int)H, 0};
  a.taps = taps;
  a.ktaps = (int)ktaps;
  a.slots = slots;
  a.state = state;
  a.s_ss = s_ss;
  a.max_seqs = max_seqs;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ATMA_BF16) launch_conv_k<bf16>(a, K, st);
  else launch_conv_k<f16>(a, K, st);
  return check_launch("linear_tokens_conv");
}

extern "C" int atma_linear_tokens_chunks(const void* x, int64_t ldx, int64_t M, int64_t chunk_k, int64_t n_chunks,
                                         const void* const* w, const int64_t* ldw, int64_t N, float* parts,
                                         int dtype, void* stream) {
  using namespace atma;
  if (!lin_common_ok(M, dtype) || !lin_k_ok(chunk_k, 4) || n_chunks < 1 || n_chunks > kLinMaxChunks || N < 4 ||
      N % 4 || N > (1 << 24))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_tokens_chunks: unsupported shape M=%lld chunk_k=%lld chunks=%lld N=%lld dtype=%d "
                     "(16-bit, 1 <= M <= 32, 1 to %d chunks of K 256, 512 or 1024, N %% 4 == 0)",
                     (long long)M, (long long)chunk_k, (long long)n_chunks, (long long)N, dtype, kLinMaxChunks);
  if (!x || !w || !ldw || !parts) return set_error(ATMA_ERR_INVALID, "linear_tokens_chunks: null pointer");
  if ((uintptr_t)x % 16 || ldx % 8 || ldx < n_chunks * chunk_k || (uintptr_t)parts % 16)
    return set_error(ATMA_ERR_INVALID,
                     "linear_tokens_chunks: x rows must be 16-byte aligned and hold every chunk; parts 16-byte aligned");
  LinTokArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.M = (int)M;
  a.N = (int)N;
  a.parts = parts;
  for (int c = 0; c < n_chunks; ++c) {
    if (!w[c] || (uintptr_t)w[c] % 16 || ldw[c] % 8 || ldw[c] < chunk_k)
      return set_error(ATMA_ERR_INVALID, "linear_tokens_chunks: chunk %d weight rows must be 16-byte aligned", c);
    a.cw[c] = w[c];
    a.cldw[c] = ldw[c];
  }
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ATMA_BF16) launch_chunks_k<bf16>(a, chunk_k, (int)n_chunks, st);
  else launch_chunks_k<f16>(a, chunk_k, (int)n_chunks, st);
  return check_launch("linear_tokens_chunks");
}
