// Elementwise and depthwise-convolution fusions of the paged inference model.
//
// Reference: kernel/inference_ops_triton.py --
//  * _squared_relu_gate_kernel / squared_relu_gate (:102-135): out = gate * relu(x)^2,
//    with relu(x)^2 rounded to bf16 before the gate multiply when the inputs are bf16
//    (eager bf16's intermediate rounding); the MLP activation of
//    inference/models/atma.py:87-96.
//  * _softcap_kernel / softcap_logits (:194-223): out = 15 x / sqrt(x^2 + 225), with
//    15 x, x^2, x^2 + 225 and the reciprocal square root each rounded to bf16 for bf16
//    logits; the output soft cap of inference/models/atma.py:750-754.
//  * _packed_causal_conv1d_kernel / packed_causal_conv1d (:17-63, :138-160): depthwise
//    causal convolution over variable-length sequences packed along the token axis,
//    out[t, c] = sum_j x[t - (K-1-j), c] w[c, j] over sources inside t's sequence
//    (fp32 accumulation in tap order), and the sequence's last K - 1 inputs (zero before
//    its start) written into its slot of the convolution state table.
//
// MI355X design: all three are HBM-bound streams.  The elementwise ops move 16 bytes
// per lane per access (8 bf16 values) when rows are 16-byte aligned, fall back to one
// element per lane otherwise, and evaluate each operation in the reference's order
// with contraction off, so results equal the reference's arithmetic bit for bit
// (the reciprocal square root is the correctly rounded 1 / sqrt).  The convolution
// gives each lane 8 channels (16 bytes) of a 32-token strip: the K - 1 previous rows
// stay in registers as the strip advances, so x is fetched from HBM about once (the
// K - 1 rows before a strip come from L2) instead of K times, and each token's
// sequence start masks the taps that fall before it.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace atma {

// ------------------------------------------------------------------ squared_relu_gate

template <typename T, int VEC>
__global__ void __launch_bounds__(256)
squared_relu_gate_kernel(const T* __restrict__ x, int64_t x_s0, int64_t x_s1, const T* __restrict__ gate,
                         int64_t g_s0, int64_t g_s1, T* __restrict__ out, int64_t rows, int64_t width) {
  const int64_t vw = width / VEC;  // vectors per row
  const int64_t n = rows * vw;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / vw, c = (i - r * vw) * VEC;
    if constexpr (VEC == 1) {
      const float xv = to_f32(x[r * x_s0 + c * x_s1]);
      const float gv = to_f32(gate[r * g_s0 + c * g_s1]);
      out[r * width + c] = from_f32<T>(sq_relu_gate1<T>(xv, gv));
    } else {
      typedef T tv __attribute__((ext_vector_type(VEC)));
      const tv xv = *(const tv*)(x + r * x_s0 + c);
      const tv gv = *(const tv*)(gate + r * g_s0 + c);
      tv o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = from_f32<T>(sq_relu_gate1<T>(to_f32(xv[e]), to_f32(gv[e])));
      *(tv*)(out + r * width + c) = o;
    }
  }
}

// Rows of at least 256 vectors: blockIdx.y walks the rows, each lane owns two 16-byte vectors
// of a row and issues all four loads before any arithmetic (no per-element index division).
// NT: non-temporal loads and stores, for streams larger than the GPU's last-level cache
// (1.61 GB at 65,536 x 4,096 bf16: 265 against 308 us for the flat loop).
constexpr int kSqRowVecs = 2;

template <typename T, bool NT>
__global__ void __launch_bounds__(256)
squared_relu_gate_rows_kernel(const T* __restrict__ x, int64_t x_s0, const T* __restrict__ gate, int64_t g_s0,
                              T* __restrict__ out, int64_t rows, int64_t width) {
  constexpr int V = 16 / (int)sizeof(T);
  typedef T tv __attribute__((ext_vector_type(V)));
  const int64_t c0 = ((int64_t)blockIdx.x * 256 * kSqRowVecs + threadIdx.x) * V;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    u32x4 xv[kSqRowVecs], gv[kSqRowVecs];
#pragma unroll
    for (int u = 0; u < kSqRowVecs; ++u) {
      const int64_t c = c0 + (int64_t)u * 256 * V;
      if (c < width) {
        const u32x4* px = (const u32x4*)(x + r * x_s0 + c);
        const u32x4* pg = (const u32x4*)(gate + r * g_s0 + c);
        if constexpr (NT) {
          xv[u] = __builtin_nontemporal_load(px);
          gv[u] = __builtin_nontemporal_load(pg);
        } else {
          xv[u] = *px;
          gv[u] = *pg;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kSqRowVecs; ++u) {
      const int64_t c = c0 + (int64_t)u * 256 * V;
      if (c < width) {
        const tv a = __builtin_bit_cast(tv, xv[u]), b = __builtin_bit_cast(tv, gv[u]);
        tv o;
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = from_f32<T>(sq_relu_gate1<T>(to_f32(a[e]), to_f32(b[e])));
        u32x4* po = (u32x4*)(out + r * width + c);
        if constexpr (NT)
          __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), po);
        else
          *po = __builtin_bit_cast(u32x4, o);
      }
    }
  }
}

// ------------------------------------------------------------------ softcap_logits
template <typename T>
__device__ __forceinline__ float softcap1(float x) {
#pragma clang fp contract(off)
  constexpr bool kB = std::is_same<T, bf16>::value;
  float left = 15.f * x;
  float square = x * x;
  if constexpr (kB) {
    left = round_bf16(left);
    square = round_bf16(square);
  }
  float denom = square + 225.f;
  if constexpr (kB) denom = round_bf16(denom);
  float inv = 1.f / __builtin_sqrtf(denom);
  if constexpr (kB) inv = round_bf16(inv);
  return left * inv;
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256) softcap_kernel(const T* __restrict__ x, T* __restrict__ out, int64_t n) {
  const int64_t nv = n / VEC;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv; i += (int64_t)gridDim.x * 256) {
    if constexpr (VEC == 1) {
      out[i] = from_f32<T>(softcap1<T>(to_f32(x[i])));
    } else {
      typedef T tv __attribute__((ext_vector_type(VEC)));
      const tv xv = *(const tv*)(x + i * VEC);
      tv o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = from_f32<T>(softcap1<T>(to_f32(xv[e])));
      *(tv*)(out + i * VEC) = o;
    }
  }
  // the tail (n % VEC elements) goes to the first lanes of block 0
  if (VEC > 1 && blockIdx.x == 0 && threadIdx.x < n - nv * VEC) {
    const int64_t i = nv * VEC + threadIdx.x;
    out[i] = from_f32<T>(softcap1<T>(to_f32(x[i])));
  }
}

// ------------------------------------------------------------------ softcap_argmax
// The decode step's soft cap and greedy pick in one pass over a row of logits: out =
// softcap(x) (softcap_logits' arithmetic) and the index of its largest value as
// torch.argmax over those 16-bit values returns it -- the first index among equal values,
// NaN above every number.  One workgroup of 512 threads per row; a thread issues the loads
// of up to kPickVecs 16-byte vectors before it converts any (one memory latency for a row
// of up to 512 * kPickVecs * 8 values, 65,536: the served vocabulary is 50,304).  The cap
// (a correctly rounded square root and division per value) is the costly part, and one
// workgroup per row puts a 32-row decode step on 32 CUs: contiguous rows are therefore
// capped by the elementwise softcap kernel over the whole grid first, and this kernel then
// only picks (CAPPED: x holds the capped values, nothing is written but idx).
__device__ __forceinline__ bool argmax_before(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

constexpr int kPickVecs = 16;

template <typename T, bool CAPPED>
__global__ void __launch_bounds__(512)
softcap_argmax_kernel(const T* __restrict__ x, int64_t ldx, T* __restrict__ out, int64_t ldo,
                      int64_t* __restrict__ idx, int V, int vec) {
  const T* xr = x + (int64_t)blockIdx.x * ldx;
  T* orow = out + (int64_t)blockIdx.x * ldo;
  float best = -__builtin_inff();
  int bi = 0x7fffffff;
  const int nv = vec ? V / 8 : 0;  // 16-byte vectors when every row is 16-byte aligned
  // argmax_before is a strict total order on (value, index), so the pick does not depend on
  // the order in which a thread visits its vectors
  for (int i0 = threadIdx.x; i0 < nv; i0 += 512 * kPickVecs) {
    u32x4 u[kPickVecs];
#pragma unroll
    for (int j = 0; j < kPickVecs; ++j)  // past the row: a repeat of its last vector, unused
      u[j] = *(const u32x4*)(xr + 8 * min(i0 + 512 * j, nv - 1));
#pragma unroll
    for (int j = 0; j < kPickVecs; ++j) {
      // every vector is converted (so no load is moved next to a conditional use); only
      // those inside the row are stored and compared
      const int i = i0 + 512 * j;
      const bool in = i < nv;
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y0 = elem16<T>(u[j], 2 * e), y1 = elem16<T>(u[j], 2 * e + 1);
        if constexpr (!CAPPED) {
          y0 = to_f32(from_f32<T>(softcap1<T>(y0)));
          y1 = to_f32(from_f32<T>(softcap1<T>(y1)));
          o[e] = pack2<T>(y0, y1);
        }
        if (in && argmax_before(y0, 8 * i + 2 * e, best, bi)) best = y0, bi = 8 * i + 2 * e;
        if (in && argmax_before(y1, 8 * i + 2 * e + 1, best, bi)) best = y1, bi = 8 * i + 2 * e + 1;
      }
      if (!CAPPED && in) *(u32x4*)(orow + 8 * i) = o;
    }
  }
  for (int i = 8 * nv + threadIdx.x; i < V; i += 512) {
    float y = to_f32(xr[i]);
    if constexpr (!CAPPED) {
      y = to_f32(from_f32<T>(softcap1<T>(y)));
      orow[i] = from_f32<T>(y);
    }
    if (argmax_before(y, i, best, bi)) best = y, bi = i;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(best, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (argmax_before(ov, oi, best, bi)) best = ov, bi = oi;
  }
  __shared__ float sv[8];
  __shared__ int si[8];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 8; ++w)
      if (argmax_before(sv[w], si[w], best, bi)) best = sv[w], bi = si[w];
    idx[blockIdx.x] = bi;
  }
}

// ------------------------------------------------------------------ packed_causal_conv1d
constexpr int kConvStrip = 32;  // tokens per lane strip
constexpr int kConvMaxK = 8;

// One lane = VEC consecutive channels x a strip of kConvStrip tokens.
template <typename T, typename TS, int VEC, int K>
__global__ void __launch_bounds__(64)
packed_causal_conv1d_kernel(const T* __restrict__ x, int64_t x_st, int64_t x_sc, const T* __restrict__ w,
                            int64_t w_sc, int64_t w_sk, T* __restrict__ out, TS* __restrict__ state,
                            int64_t s_ss, int64_t s_sc, int64_t s_sk, int64_t num_slots,
                            const int32_t* __restrict__ seq_start, const int32_t* __restrict__ seq_end,
                            const int32_t* __restrict__ seq_slot, int64_t total, int64_t channels) {
  const int64_t c0 = ((int64_t)blockIdx.y * 64 + threadIdx.x) * VEC;
  // the host takes VEC > 1 only when channels % VEC == 0, so every lane past this check owns
  // VEC whole channels
  if (c0 >= channels) return;
  const int64_t t_beg = (int64_t)blockIdx.x * kConvStrip;
  const int64_t t_end = min(t_beg + kConvStrip, total);

  // a contiguous, 16-byte aligned (channels, K) weight: the lane's VEC x K taps are K whole
  // 16-byte words, read as such (gathered one element at a time through the runtime
  // strides, the taps took a fifth of the kernel's time at 65,536 x 1,024)
  float wt[K][VEC];
  bool wide = false;
  if constexpr (VEC > 1) {
    struct Words { u32x4 q[K]; };
    struct Taps { T v[VEC * K]; };
    static_assert(sizeof(Words) == sizeof(Taps), "VEC x K taps fill K 16-byte words");
    wide = w_sk == 1 && w_sc == K && ((uintptr_t)w & 15) == 0;
    if (wide) {
      Words raw;
      const u32x4* src = (const u32x4*)(w + c0 * K);
#pragma unroll
      for (int q = 0; q < K; ++q) raw.q[q] = src[q];
      const Taps tp = __builtin_bit_cast(Taps, raw);
#pragma unroll
      for (int j = 0; j < K; ++j)
#pragma unroll
        for (int e = 0; e < VEC; ++e) wt[j][e] = to_f32(tp.v[e * K + j]);
    }
  }
  if (!wide) {
#pragma unroll
    for (int j = 0; j < K; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) wt[j][e] = to_f32(w[(c0 + e) * w_sc + j * w_sk]);
  }

  auto load_row = [&](int64_t t, float* v) {
    if constexpr (VEC == 1) {
      v[0] = to_f32(x[t * x_st + c0 * x_sc]);
    } else {
      typedef T tv __attribute__((ext_vector_type(VEC)));
      const tv xv = *(const tv*)(x + t * x_st + c0);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = to_f32(xv[e]);
    }
  };
  // win[K-1] is row t; win[j] is row t - (K-1-j).  Rows before the tensor's start are 0
  // (they are always masked: a sequence starts at token 0 or later).
  float win[K][VEC];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int64_t t = t_beg - (K - 1) + j;
    if (t >= 0) {
      load_row(t, win[j]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) win[j][e] = 0.f;
    }
  }
#pragma unroll 8
  for (int64_t t = t_beg; t < t_end; ++t) {
    load_row(t, win[K - 1]);
    const int64_t start = seq_start[t];
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const bool live = t - (K - 1 - j) >= start;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = fmaf(live ? win[j][e] : 0.f, wt[j][e], acc[e]);
    }
    if constexpr (VEC == 1) {
      out[t * channels + c0] = from_f32<T>(acc[0]);
    } else {
      typedef T tv __attribute__((ext_vector_type(VEC)));
      tv o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = from_f32<T>(acc[e]);
      *(tv*)(out + t * channels + c0) = o;
    }
    // the sequence's last token writes its K - 1 newest inputs into the state row
    if (t == (int64_t)seq_end[t] - 1) {
      const int64_t slot = seq_slot[t];
      if (slot >= 0 && slot < num_slots) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
          const bool live = t - (K - 2 - j) >= start;
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            state[slot * s_ss + (c0 + e) * s_sc + j * s_sk] = from_f32<TS>(live ? win[j + 1][e] : 0.f);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) win[j][e] = win[j + 1][e];
  }
}

// streams beyond the MI355X's 256 MiB last-level cache take non-temporal accesses
constexpr int64_t kSqStreamBytes = 256ll << 20;

static unsigned elementwise_grid(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks, 256 * 64));
}

template <typename T>
static int launch_sq(const void* x, int64_t x_s0, int64_t x_s1, const void* g, int64_t g_s0, int64_t g_s1,
                     void* out, int64_t rows, int64_t width, hipStream_t s) {
  constexpr int V = 16 / (int)sizeof(T);
  const bool vec = x_s1 == 1 && g_s1 == 1 && width % V == 0 && (uintptr_t)x % 16 == 0 &&
                   (uintptr_t)g % 16 == 0 && (uintptr_t)out % 16 == 0 && (x_s0 * sizeof(T)) % 16 == 0 &&
                   (g_s0 * sizeof(T)) % 16 == 0;
  if (vec && width / V >= 256) {
    const dim3 grid((unsigned)((width / V + 256 * kSqRowVecs - 1) / (256 * kSqRowVecs)),
                    (unsigned)std::min<int64_t>(rows, 8192));
    if (3 * rows * width * (int64_t)sizeof(T) > kSqStreamBytes)
      squared_relu_gate_rows_kernel<T, true><<<grid, 256, 0, s>>>((const T*)x, x_s0, (const T*)g, g_s0, (T*)out,
                                                                 rows, width);
    else
      squared_relu_gate_rows_kernel<T, false><<<grid, 256, 0, s>>>((const T*)x, x_s0, (const T*)g, g_s0, (T*)out,
                                                                  rows, width);
  } else if (vec)
    squared_relu_gate_kernel<T, V><<<elementwise_grid(rows * width / V), 256, 0, s>>>(
        (const T*)x, x_s0, x_s1, (const T*)g, g_s0, g_s1, (T*)out, rows, width);
  else
    squared_relu_gate_kernel<T, 1><<<elementwise_grid(rows * width), 256, 0, s>>>(
        (const T*)x, x_s0, x_s1, (const T*)g, g_s0, g_s1, (T*)out, rows, width);
  return check_launch("squared_relu_gate");
}

template <typename T>
static int launch_softcap(const void* x, void* out, int64_t n, hipStream_t s) {
  constexpr int V = 16 / (int)sizeof(T);
  if ((uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0)
    softcap_kernel<T, V><<<elementwise_grid(std::max<int64_t>(n / V, 1)), 256, 0, s>>>((const T*)x, (T*)out, n);
  else
    softcap_kernel<T, 1><<<elementwise_grid(n), 256, 0, s>>>((const T*)x, (T*)out, n);
  return check_launch("softcap_logits");
}

template <typename T, typename TS, int VEC, int K>
static void launch_conv_k(const void* x, int64_t x_st, int64_t x_sc, const void* w, int64_t w_sc,
                          int64_t w_sk, void* out, void* state, int64_t s_ss, int64_t s_sc, int64_t s_sk,
                          int64_t num_slots, const int32_t* st, const int32_t* en, const int32_t* sl,
                          int64_t total, int64_t channels, hipStream_t s) {
  const dim3 grid((unsigned)((total + kConvStrip - 1) / kConvStrip),
                  (unsigned)((channels + 64 * VEC - 1) / (64 * VEC)));
  packed_causal_conv1d_kernel<T, TS, VEC, K><<<grid, 64, 0, s>>>(
      (const T*)x, x_st, x_sc, (const T*)w, w_sc, w_sk, (T*)out, (TS*)state, s_ss, s_sc, s_sk, num_slots, st,
      en, sl, total, channels);
}

template <typename T, typename TS, int VEC>
static void launch_conv_v(int64_t K, const void* x, int64_t x_st, int64_t x_sc, const void* w, int64_t w_sc,
                          int64_t w_sk, void* out, void* state, int64_t s_ss, int64_t s_sc, int64_t s_sk,
                          int64_t num_slots, const int32_t* st, const int32_t* en, const int32_t* sl,
                          int64_t total, int64_t channels, hipStream_t s) {
#define ATMA_CONV_K(KK)                                                                                   \
  case KK:                                                                                                \
    launch_conv_k<T, TS, VEC, KK>(x, x_st, x_sc, w, w_sc, w_sk, out, state, s_ss, s_sc, s_sk, num_slots, \
                                  st, en, sl, total, channels, s);                                        \
    break;
  switch (K) {
    ATMA_CONV_K(2)
    ATMA_CONV_K(3)
    ATMA_CONV_K(4)
    ATMA_CONV_K(5)
    ATMA_CONV_K(6)
    ATMA_CONV_K(7)
    ATMA_CONV_K(8)
    default: break;
  }
#undef ATMA_CONV_K
}

template <typename T, typename TS>
static int launch_conv(int64_t K, const void* x, int64_t x_st, int64_t x_sc, const void* w, int64_t w_sc,
                       int64_t w_sk, void* out, void* state, int64_t s_ss, int64_t s_sc, int64_t s_sk,
                       int64_t num_slots, const int32_t* st, const int32_t* en, const int32_t* sl,
                       int64_t total, int64_t channels, hipStream_t s) {
  constexpr int V = 16 / (int)sizeof(T);
  const bool vec = x_sc == 1 && channels % V == 0 && (uintptr_t)x % 16 == 0 && (x_st * sizeof(T)) % 16 == 0 &&
                   (uintptr_t)out % 16 == 0;
  if (vec)
    launch_conv_v<T, TS, V>(K, x, x_st, x_sc, w, w_sc, w_sk, out, state, s_ss, s_sc, s_sk, num_slots, st, en, sl,
                            total, channels, s);
  else
    launch_conv_v<T, TS, 1>(K, x, x_st, x_sc, w, w_sc, w_sk, out, state, s_ss, s_sc, s_sk, num_slots, st, en, sl,
                            total, channels, s);
  return check_launch("packed_causal_conv1d");
}

template <typename T>
static int conv_state_dtype(int state_dtype, int64_t K, const void* x, int64_t x_st, int64_t x_sc, const void* w,
                            int64_t w_sc, int64_t w_sk, void* out, void* state, int64_t s_ss, int64_t s_sc,
                            int64_t s_sk, int64_t num_slots, const int32_t* st, const int32_t* en,
                            const int32_t* sl, int64_t total, int64_t channels, hipStream_t s) {
  switch (state_dtype) {
    case ATMA_F32:
      return launch_conv<T, float>(K, x, x_st, x_sc, w, w_sc, w_sk, out, state, s_ss, s_sc, s_sk, num_slots, st,
                                   en, sl, total, channels, s);
    case ATMA_BF16:
      return launch_conv<T, bf16>(K, x, x_st, x_sc, w, w_sc, w_sk, out, state, s_ss, s_sc, s_sk, num_slots, st,
                                  en, sl, total, channels, s);
    case ATMA_F16:
      return launch_conv<T, f16>(K, x, x_st, x_sc, w, w_sc, w_sk, out, state, s_ss, s_sc, s_sk, num_slots, st,
                                 en, sl, total, channels, s);
    default:
      return set_error(ATMA_ERR_INVALID, "packed_causal_conv1d: unknown state dtype %d", state_dtype);
  }
}

}  // namespace atma

extern "C" int atma_squared_relu_gate(const void* x, int64_t x_s0, int64_t x_s1, const void* gate, int64_t g_s0,
                                      int64_t g_s1, void* out, int64_t rows, int64_t width, int dtype,
                                      void* stream) {
  using namespace atma;
  if (rows < 0 || width < 0) return set_error(ATMA_ERR_INVALID, "squared_relu_gate: bad sizes");
  if (rows == 0 || width == 0) return ATMA_OK;
  if (!x || !gate || !out) return set_error(ATMA_ERR_INVALID, "squared_relu_gate: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_F32: return launch_sq<float>(x, x_s0, x_s1, gate, g_s0, g_s1, out, rows, width, s);
    case ATMA_BF16: return launch_sq<bf16>(x, x_s0, x_s1, gate, g_s0, g_s1, out, rows, width, s);
    case ATMA_F16: return launch_sq<f16>(x, x_s0, x_s1, gate, g_s0, g_s1, out, rows, width, s);
    default: return set_error(ATMA_ERR_INVALID, "squared_relu_gate: unknown dtype %d", dtype);
  }
}

extern "C" int atma_softcap_logits(const void* logits, void* out, int64_t n, int dtype, void* stream) {
  using namespace atma;
  if (n < 0) return set_error(ATMA_ERR_INVALID, "softcap_logits: bad size");
  if (n == 0) return ATMA_OK;
  if (!logits || !out) return set_error(ATMA_ERR_INVALID, "softcap_logits: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_F32: return launch_softcap<float>(logits, out, n, s);
    case ATMA_BF16: return launch_softcap<bf16>(logits, out, n, s);
    case ATMA_F16: return launch_softcap<f16>(logits, out, n, s);
    default: return set_error(ATMA_ERR_INVALID, "softcap_logits: unknown dtype %d", dtype);
  }
}

extern "C" int atma_softcap_argmax(const void* logits, int64_t ldx, void* out, int64_t ldo, int64_t* idx,
                                   int64_t rows, int64_t V, int dtype, void* stream) {
  using namespace atma;
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "softcap_argmax: 16-bit logits only (dtype %d)", dtype);
  if (rows < 0 || V < 1 || V > 0x7fffffff || rows > 0x7fffffff || ldx < V || ldo < V)
    return set_error(ATMA_ERR_INVALID, "softcap_argmax: bad sizes");
  if (rows == 0) return ATMA_OK;
  if (!logits || !out || !idx) return set_error(ATMA_ERR_INVALID, "softcap_argmax: null pointer");
  const int vec = !((uintptr_t)logits % 16 || (uintptr_t)out % 16 || ldx % 8 || ldo % 8);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows), block(512);
  if (ldx == V && ldo == V && rows * V >= (1 << 16)) {
    // contiguous rows: cap them over the whole grid, then pick from the capped values
    const int rc = dtype == ATMA_BF16 ? launch_softcap<bf16>(logits, out, rows * V, s)
                                      : launch_softcap<f16>(logits, out, rows * V, s);
    if (rc != ATMA_OK) return rc;
    if (dtype == ATMA_BF16)
      softcap_argmax_kernel<bf16, true><<<grid, block, 0, s>>>((const bf16*)out, ldo, nullptr, 0, idx, (int)V, vec);
    else
      softcap_argmax_kernel<f16, true><<<grid, block, 0, s>>>((const f16*)out, ldo, nullptr, 0, idx, (int)V, vec);
  } else if (dtype == ATMA_BF16) {
    softcap_argmax_kernel<bf16, false><<<grid, block, 0, s>>>((const bf16*)logits, ldx, (bf16*)out, ldo, idx, (int)V,
                                                              vec);
  } else {
    softcap_argmax_kernel<f16, false><<<grid, block, 0, s>>>((const f16*)logits, ldx, (f16*)out, ldo, idx, (int)V,
                                                             vec);
  }
  return check_launch("softcap_argmax");
}

extern "C" int atma_packed_causal_conv1d(const void* x, int64_t x_st, int64_t x_sc, const void* weight,
                                         int64_t w_sc, int64_t w_sk, void* out, void* state_table, int64_t s_ss,
                                         int64_t s_sc, int64_t s_sk, int64_t num_slots,
                                         const int32_t* token_seq_starts, const int32_t* token_seq_ends,
                                         const int32_t* token_seq_slots, int64_t total, int64_t channels,
                                         int64_t K, int dtype, int state_dtype, void* stream) {
  using namespace atma;
  if (total < 0 || channels < 0 || num_slots < 0)
    return set_error(ATMA_ERR_INVALID, "packed_causal_conv1d: bad sizes");
  if (K < 2 || K > kConvMaxK)
    return set_error(ATMA_ERR_UNSUPPORTED, "packed_causal_conv1d: kernel size %lld (supported: 2..%d)",
                     (long long)K, kConvMaxK);
  if (total == 0 || channels == 0) return ATMA_OK;
  if (total > 0x7fffffffll * kConvStrip || channels > 0x7fffffffll)
    return set_error(ATMA_ERR_INVALID, "packed_causal_conv1d: sizes too large");
  if (!x || !weight || !out || !state_table || !token_seq_starts || !token_seq_ends || !token_seq_slots)
    return set_error(ATMA_ERR_INVALID, "packed_causal_conv1d: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ATMA_F32:
      return conv_state_dtype<float>(state_dtype, K, x, x_st, x_sc, weight, w_sc, w_sk, out, state_table, s_ss,
                                     s_sc, s_sk, num_slots, token_seq_starts, token_seq_ends, token_seq_slots,
                                     total, channels, s);
    case ATMA_BF16:
      return conv_state_dtype<bf16>(state_dtype, K, x, x_st, x_sc, weight, w_sc, w_sk, out, state_table, s_ss,
                                    s_sc, s_sk, num_slots, token_seq_starts, token_seq_ends, token_seq_slots,
                                    total, channels, s);
    case ATMA_F16:
      return conv_state_dtype<f16>(state_dtype, K, x, x_st, x_sc, weight, w_sc, w_sk, out, state_table, s_ss,
                                   s_sc, s_sk, num_slots, token_seq_starts, token_seq_ends, token_seq_slots,
                                   total, channels, s);
    default:
      return set_error(ATMA_ERR_INVALID, "packed_causal_conv1d: unknown dtype %d", dtype);
  }
}
