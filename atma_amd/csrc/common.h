// Shared device/host helpers for libatma_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "atma_hip.h"

namespace atma {

using bf16 = __bf16;
using f16 = _Float16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Masked logits use this finite sentinel (never -inf * temp) and contribute p = 0.
constexpr float kSentinel = -1e38f;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x) { return (T)x; }

__device__ __forceinline__ float round_bf16(float x) { return (float)(bf16)x; }

// gate * relu(x)^2 in eager 16-bit order: the square rounded to bf16 for bf16 inputs
// before the gate multiply (the output's rounding is the caller's).
template <typename T>
__device__ __forceinline__ float sq_relu_gate1(float x, float g) {
#pragma clang fp contract(off)
  const float pos = x < 0.f ? 0.f : x;  // NaN passes through, as torch's relu
  float sq = pos * pos;
  if constexpr (__is_same(T, bf16)) sq = round_bf16(sq);
  return g * sq;
}

// softplus with torch's default threshold (x > 20 -> x).
__device__ __forceinline__ float softplus(float x) {
  return x > 20.f ? x : log1pf(expf(x));
}

// 16-byte vector of 8 two-byte elements, reinterpretable for MFMA operands.
union Pack8 {
  u32x4 u;
  bf16x8 b;
  f16x8 h;
};

// v_mfma_f32_16x16x32_{bf16,f16}: A lane l holds row l%16, k = 8*(l/16)+[0,8);
// B lane l holds column l%16, same k; C lane l holds rows 4*(l/16)+[0,4), column l%16.
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  Pack8 pa, pb;
  pa.u = a;
  pb.u = b;
  if constexpr (__is_same(T, bf16)) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa.b, pb.b, c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(pa.h, pb.h, c, 0, 0, 0);
  }
}

// Two floats -> one dword of two 16-bit values (x in the low half).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  // one v_cvt_pk_{bf16,f16}_f32 (round to nearest even, as the scalar conversions)
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){x, y}, t2));
}

// Dot product of two packed 16-bit pairs accumulated in fp32 (v_dot2_f32_{bf16,f16}).
template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (__is_same(T, bf16)) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  } else {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
}

// 16-bit element e (0..7) of a 16-byte vector, as float.
template <typename T>
__device__ __forceinline__ float elem16(const u32x4& x, int e) {
  const uint16_t u = (uint16_t)(x[e >> 1] >> ((e & 1) * 16));
  return (float)__builtin_bit_cast(T, u);
}

// Raw buffer access (gfx9 descriptor: no stride, no swizzle, dword format).  The base
// and size live in scalar registers, a lane contributes a 32-bit byte offset, and
// reads past `bytes` return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                               uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// The same load marked non-temporal (nt): data read once (a KV cache streamed by decode)
// does not displace reusable lines in L2 / MALL, and streams measurably faster.
__device__ __forceinline__ u32x4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                  uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2));
}

template <typename T>
__device__ __forceinline__ void buffer_store16b(__amdgpu_buffer_rsrc_t r, uint32_t voff, T x) {
  static_assert(sizeof(T) == 2, "16-bit element");
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, x), r, voff, 0, 0);
}

// LDS byte offset of a pointer into __shared__ memory: a flat address in the LDS
// aperture carries the offset in its low 32 bits (the aperture base is 4 GiB aligned), so
// a truncation suffices -- no null-pointer select as with an address-space cast.
__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)p; }

// Direct global->LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane i's
// bytes land at lds_wave_base + 16*i.  Issued through inline asm so the compiler does
// not serialise later LDS reads behind it; completion is tracked by vmcnt, so the
// caller waits with s_waitcnt vmcnt(N) and a barrier before reading the data.
// The compiler inserts no wait states around inline asm, so each copy below starts with
// the one a GFX9 LDS DMA needs after the scalar write of m0 that precedes it (s_nop 0).
// Its other scalar operands (descriptor, scalar offset) must not come from a VALU write
// (v_readfirstlane, v_readlane) in the five wait states before it; the callers keep them
// in SALU arithmetic, and a CPU test checks the generated code for both rules.
__device__ __forceinline__ void dma_load16(const void* gptr, const void* lds_wave_base) {
  const uint32_t off = lds_offset(lds_wave_base);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr),
               "{m0}"(__builtin_amdgcn_readfirstlane(off))
               : "memory");
}

// The same copy through a buffer descriptor (buffer_load_dwordx4 ... lds): lane i
// reads 16 bytes at voff + soff of the buffer (zeros past its size) into
// lds_wave_base + 16*i.  The address arithmetic stays in one 32-bit offset per lane
// and one scalar offset, so per-copy cost is a scalar move into m0.
__device__ __forceinline__ void dma_buf16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          const void* lds_wave_base) {
  const uint32_t off = lds_offset(lds_wave_base);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff),
               "{m0}"(__builtin_amdgcn_readfirstlane(off))
               : "memory");
}

// The same copy with the LDS destination given as a wave-uniform byte offset (for
// callers that keep their LDS bases in scalar registers).
__device__ __forceinline__ void dma_buf16_at(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                             uint32_t lds_byte_offset) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_byte_offset))
               : "memory");
}

// 4 bytes per lane (buffer_load_dword ... lds): lane i's dword lands at lds_wave_base + 4*i.
__device__ __forceinline__ void dma_buf4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                         const void* lds_wave_base) {
  const uint32_t off = lds_offset(lds_wave_base);
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff),
               "{m0}"(__builtin_amdgcn_readfirstlane(off))
               : "memory");
}
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t r, uint32_t voff, u32x4 x) {
  __builtin_amdgcn_raw_buffer_store_b128(x, r, voff, 0, 0);
}

// Wait until at most N vector-memory operations of this wave are outstanding (the
// compiler does not count the inline-asm direct-to-LDS loads above).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// LDS writes of this wave done, then a workgroup barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element i % 4
// of the 64-bit words read by lanes i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12 (in that
// order).  With lane s reading row r0 + s / 4, columns c0 + 4 (s % 4) .. + 3 of a
// row-major 16-bit matrix, lane i gets rows r0 .. r0 + 3 of column c0 + i.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
  return __builtin_bit_cast(u32x2, r);
}

// Chunk swizzle of row-major 16-bit tiles in LDS (rows of CPR 16-byte chunks): logical
// 16-byte chunk c of row r is stored at chunk position c ^ f(r).  With 256-byte rows
// (CPR 16) f is a bijection on r mod 16, so row reads (one chunk of 16 different rows per
// 16 lanes) hit 16 distinct bank groups, and f(r) >> 2 differs across any 4 consecutive
// rows 4k .. 4k + 3, so transposing reads (4 rows x 4 adjacent chunks per 32 lanes) hit 16
// distinct positions too.  With 128-byte rows (CPR 8) rows r and r + 2 share banks and f
// takes 8 values, so 16-row reads pair up two ways (the d = 64 tiles; gemm_gated.hip uses
// its own f for such rows).
template <int CPR>
__device__ __forceinline__ int lds_swizzle(int r) {
  if constexpr (CPR == 16) return 4 * (r & 3) + ((r >> 2) & 3);
  else return 2 * (r & 3) + ((r >> 2) & 1);
}

// X Y of fp32 16 x 16 blocks on v_mfma_f32_16x16x4f32, with X entering transposed: xt and y
// are in the accumulator layout (lane (g, c) register i = row 4g + i, column c), and step i
// contracts k = 4g + i, so xt[i] is the A operand (X[c][4g + i]) and y[i] the B operand.
__device__ __forceinline__ f32x4 blk_mul(const f32x4& xt, const f32x4& y, f32x4 acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xt[i], y[i], acc, 0, 0, 0);
  return acc;
}

// Lower-triangle 16-token block pairs (k, P), k <= P, in the order (0,0) (0,1) (1,1) (0,2) ...
__host__ __device__ constexpr int tri(int k, int P) { return P * (P + 1) / 2 + k; }

// Wave-local barrier: orders LDS traffic between lanes of one wavefront.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T>
__device__ __forceinline__ T wave_xor(T x, int mask) {
  return __shfl_xor(x, mask, 64);
}

// Lane exchange inside each row of 16 lanes through DPP (no LDS crossbar round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, false));
}
// Max / sum over the 16 lanes of each row, the result in every lane of the row: pairs
// within quads (quad_perm [1,0,3,2], then [2,3,0,1]), then the two quads of each half
// row (row_half_mirror: lane i with 7 - i), then the two half rows (row_mirror: lane i
// with 15 - i).  Every step combines one lane of each group, so all lanes agree.
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));
  x = fmaxf(x, dpp_f32<0x4E>(x));
  x = fmaxf(x, dpp_f32<0x141>(x));
  return fmaxf(x, dpp_f32<0x140>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);
  x += dpp_f32<0x4E>(x);
  x += dpp_f32<0x141>(x);
  return x + dpp_f32<0x140>(x);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}
__device__ __forceinline__ float wave_min(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fminf(x, __shfl_xor(x, m, 64));
  return x;
}

// ---------------------------------------------------------------- host side
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Compute units of the current device (cached per device; 256 if the query fails).
int device_cu_count();
int dtype_size(int dtype);

}  // namespace atma
