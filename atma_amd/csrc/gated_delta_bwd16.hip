// Chunked backward of the gated-delta recurrence for 16-bit training: the sequential part.
//
// Reference: the memory branch trains through FLA's chunk_gated_delta_rule autograd
// (model/blocks.py:44-84); the recurrence is scripts/titans_proto.py:53-76 in the [K, V]
// layout.  Inside a 64-token chunk with inclusive log decays lg, Ga = exp(lg),
// w = exp(lg_C - lg), T = (I + diag(beta) A)^-1 (A[p,s] = exp(lg_p - lg_s) k_p.k_s, s < p)
// and Rq[p,s] = exp(lg_p - lg_s) q_p.k_s (s <= p), the forward is
//   U = T diag(beta) (V - diag(Ga) K S),   S' = Ga_C S + K^T diag(w) U,
// and the backward carries dS = dL/dS' from the last chunk to the first:
//   dU = Rq^T dO + diag(w) K dS,   dY = T^T dU,
//   dS <- Ga_C dS + Q^T diag(Ga) dO - K^T diag(Ga beta) dY.
// This kernel runs both chains (the forward one to recover each chunk's entry state,
// then the backward one) and writes, per chunk, the entry state S, the exit-state
// gradient dS and dY; every other gradient is a product within one chunk, formed by the
// caller from these (dV = diag(beta) dY, the rest batched over chunks).
//
// MI355X mapping: one workgroup of 4 waves per (sequence-head, 64 state columns), each
// wave owning 16 columns (the recurrence never mixes V columns).  The chunk's shared
// operands -- k rows, k^T, q^T, T (forward) or T^T (backward), Rq^T, 64 x 64 or 64 x d
// bf16 tiles the caller lays out -- are staged in LDS with rows padded by 16 bytes (the
// 16-lane fragment reads then touch 16 distinct bank groups).  Products run on
// v_mfma_f32_16x16x32 (fp32 accumulation); the state and every per-column intermediate
// (Y, U, dU, dY) go through a per-wave transposed bf16 buffer ([column][k], 16 bytes per
// lane per fragment) to become the B operand of the next product.
#include "common.h"

namespace atma {

struct Bwd16ChainArgs {
  const void* kr;    // [N][64][D]  k rows of each chunk (N = BH * NC, chunk-head major)
  const void* kt;    // [N][D][64]  k^T
  const void* qt;    // [N][D][64]  q^T (scaled, normalised)
  const void* tm;    // [N][64][64] T
  const void* tt;    // [N][64][64] T^T
  const void* rt;    // [N][64][64] Rq^T
  const void* vt;    // [N][D][64]  v^T
  const void* ot;    // [N][D][64]  dO^T
  const void* got;   // [N][D][64]  (diag(Ga) dO)^T
  const float* f;    // [N][4][64]  Ga, w, beta, then Ga_C at [3][0]
  const float* s0;   // [BH][D][D] initial state, or null (zero)
  const float* dst;  // [BH][D][D] final-state cotangent, or null (zero)
  float* s_entry;    // [N][D][D]  out: each chunk's entry state
  float* ds_end;     // [N][D][D]  out: the gradient of each chunk's exit state
  float* dy;         // [N][64][D] out: dY
  float* ds0;        // [BH][D][D] out: the gradient of the initial state
  int BH, NC;
};

template <typename T, int D>
__global__ void __launch_bounds__(256, 1) gdn_bwd16_chain_kernel(Bwd16ChainArgs a) {
  constexpr int C = 64, PD = D + 8, PC = C + 8;  // padded LDS pitches (elements)
  constexpr int KS = D / 32;                      // 32-wide k steps over D
  constexpr int DT = D / 16;                      // 16-row tiles over D
  __shared__ __attribute__((aligned(16))) T Kr[C * PD];
  __shared__ __attribute__((aligned(16))) T Kt[D * PC];
  __shared__ __attribute__((aligned(16))) T Qt[D * PC];
  __shared__ __attribute__((aligned(16))) T Tm[C * PC];  // T in the forward chain, T^T in the backward
  __shared__ __attribute__((aligned(16))) T Rt[C * PC];
  __shared__ float Fs[4 * C];
  __shared__ __attribute__((aligned(16))) T Sb[4][16 * PD];  // S^T / dS^T of the wave's columns
  __shared__ __attribute__((aligned(16))) T X1[4][16 * PC];
  __shared__ __attribute__((aligned(16))) T X2[4][16 * PC];
  __shared__ __attribute__((aligned(16))) T XO[4][16 * PC];  // dO^T rows of the wave's columns
  __shared__ __attribute__((aligned(16))) T XG[4][16 * PC];  // (Ga dO)^T rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int bh = blockIdx.x / (D / 64);
  const int v0 = 64 * (blockIdx.x % (D / 64)) + 16 * wave;  // the wave's first column
  const int col = v0 + c16;                                  // the lane's column (C layout)

  // 64-row x `cols` tile from global (row-major, unpadded) into padded LDS, all threads
  auto copy_tile = [&](T* dst, const void* src, int rows, int cols, int pitch) {
    const int cpr = cols / 8;
    const T* s = (const T*)src;
    for (int i = tid; i < rows * cpr; i += 256) {
      const int r = i / cpr, ch = i - r * cpr;
      *(u32x4*)(dst + r * pitch + 8 * ch) = *(const u32x4*)(s + (int64_t)r * cols + 8 * ch);
    }
  };
  // the wave's 16 rows of a [D][64] tile
  auto copy_rows16 = [&](T* dst, const void* src) {
    const T* s = (const T*)src;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = lane + 64 * k, r = i >> 3, ch = i & 7;
      *(u32x4*)(dst + r * PC + 8 * ch) = *(const u32x4*)(s + r * C + 8 * ch);
    }
  };
  // fragment: row (row0 + c16) of a padded tile, 8 elements from column k0 + 8 g (the A
  // operand of rows row0 .. + 15, or the B operand of 16 columns from a [column][k] buffer)
  auto frag = [&](const T* tile, int pitch, int row0, int k0) {
    return *(const u32x4*)(tile + (row0 + c16) * pitch + k0 + 8 * g);
  };
  // C tile t (rows 16 t + 4 g + i, column c16) into a [column][row] buffer
  auto put_t = [&](T* buf, int pitch, int t, const f32x4& x) {
    const u32x2 pk = {pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3])};
    *(u32x2*)(buf + c16 * pitch + 16 * t + 4 * g) = pk;
  };
  auto rows_of = [&](int t, int i) { return 16 * t + 4 * g + i; };

  // ---------------------------------------------------------------- forward chain
  f32x4 S[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[t][i] = a.s0 ? a.s0[((int64_t)bh * D + rows_of(t, i)) * D + col] : 0.f;

  for (int c = 0; c < a.NC; ++c) {
    const int64_t n = (int64_t)bh * a.NC + c;
    __syncthreads();  // every wave is done with the previous chunk's tiles
    copy_tile(Kr, (const T*)a.kr + n * C * D, C, D, PD);
    copy_tile(Kt, (const T*)a.kt + n * D * C, D, C, PC);
    copy_tile(Tm, (const T*)a.tm + n * C * C, C, C, PC);
    if (tid < 4 * C) Fs[tid] = a.f[n * 4 * C + tid];
    f32x4 Vc[4];  // v of the lane's column, C layout (rows = tokens)
    {
      const T* vrow = (const T*)a.vt + (n * D + col) * C;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const u32x2 x = *(const u32x2*)(vrow + 16 * rt + 4 * g);
        Vc[rt] = f32x4{elem16<T>(u32x4{x[0], x[1], 0, 0}, 0), elem16<T>(u32x4{x[0], x[1], 0, 0}, 1),
                       elem16<T>(u32x4{x[0], x[1], 0, 0}, 2), elem16<T>(u32x4{x[0], x[1], 0, 0}, 3)};
      }
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) put_t(Sb[wave], PD, t, S[t]);
    __syncthreads();

    // Z = K S
    f32x4 Z[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) Z[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 bf = frag(Sb[wave], PD, 0, 32 * s);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) Z[rt] = mfma16x16x32<T>(frag(Kr, PD, 16 * rt, 32 * s), bf, Z[rt]);
    }
    // Y = diag(beta) (V - diag(Ga) Z)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4 y;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = rows_of(rt, i);
        y[i] = Fs[2 * C + p] * (Vc[rt][i] - Fs[p] * Z[rt][i]);
      }
      put_t(X1[wave], PC, rt, y);
    }
    wave_sync();
    // U = T Y, then w U
    f32x4 U[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) U[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 bf = frag(X1[wave], PC, 0, 32 * s);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) U[rt] = mfma16x16x32<T>(frag(Tm, PC, 16 * rt, 32 * s), bf, U[rt]);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = Fs[C + rows_of(rt, i)] * U[rt][i];
      put_t(X2[wave], PC, rt, x);
    }
    wave_sync();
    // the entry state, then S <- Ga_C S + K^T diag(w) U
    float* se = a.s_entry + n * D * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) se[rows_of(t, i) * D + col] = S[t][i];
    const float gC = Fs[3 * C];
#pragma unroll
    for (int t = 0; t < DT; ++t) S[t] *= gC;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 bf = frag(X2[wave], PC, 0, 32 * s);
#pragma unroll
      for (int t = 0; t < DT; ++t) S[t] = mfma16x16x32<T>(frag(Kt, PC, 16 * t, 32 * s), bf, S[t]);
    }
  }

  // ---------------------------------------------------------------- backward chain
  f32x4 dS[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dS[t][i] = a.dst ? a.dst[((int64_t)bh * D + rows_of(t, i)) * D + col] : 0.f;

  for (int c = a.NC - 1; c >= 0; --c) {
    const int64_t n = (int64_t)bh * a.NC + c;
    __syncthreads();
    copy_tile(Kr, (const T*)a.kr + n * C * D, C, D, PD);
    copy_tile(Kt, (const T*)a.kt + n * D * C, D, C, PC);
    copy_tile(Qt, (const T*)a.qt + n * D * C, D, C, PC);
    copy_tile(Tm, (const T*)a.tt + n * C * C, C, C, PC);
    copy_tile(Rt, (const T*)a.rt + n * C * C, C, C, PC);
    if (tid < 4 * C) Fs[tid] = a.f[n * 4 * C + tid];
    copy_rows16(XO[wave], (const T*)a.ot + (n * D + v0) * C);
    copy_rows16(XG[wave], (const T*)a.got + (n * D + v0) * C);
    // the exit-state gradient of this chunk
    float* de = a.ds_end + n * D * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) de[rows_of(t, i) * D + col] = dS[t][i];
#pragma unroll
    for (int t = 0; t < DT; ++t) put_t(Sb[wave], PD, t, dS[t]);
    __syncthreads();

    // dU = diag(w) K dS + Rq^T dO
    f32x4 dU[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) dU[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 bf = frag(Sb[wave], PD, 0, 32 * s);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) dU[rt] = mfma16x16x32<T>(frag(Kr, PD, 16 * rt, 32 * s), bf, dU[rt]);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) dU[rt][i] *= Fs[C + rows_of(rt, i)];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 bf = frag(XO[wave], PC, 0, 32 * s);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) dU[rt] = mfma16x16x32<T>(frag(Rt, PC, 16 * rt, 32 * s), bf, dU[rt]);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) put_t(X1[wave], PC, rt, dU[rt]);
    wave_sync();
    // dY = T^T dU
    f32x4 dY[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) dY[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 bf = frag(X1[wave], PC, 0, 32 * s);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) dY[rt] = mfma16x16x32<T>(frag(Tm, PC, 16 * rt, 32 * s), bf, dY[rt]);
    }
    float* dyo = a.dy + n * C * D;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = rows_of(rt, i);
        dyo[p * D + col] = dY[rt][i];
        x[i] = -Fs[p] * Fs[2 * C + p] * dY[rt][i];
      }
      put_t(X2[wave], PC, rt, x);
    }
    wave_sync();
    // dS <- Ga_C dS + Q^T diag(Ga) dO - K^T diag(Ga beta) dY
    const float gC = Fs[3 * C];
#pragma unroll
    for (int t = 0; t < DT; ++t) dS[t] *= gC;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 b1 = frag(XG[wave], PC, 0, 32 * s);
      const u32x4 b2 = frag(X2[wave], PC, 0, 32 * s);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        dS[t] = mfma16x16x32<T>(frag(Qt, PC, 16 * t, 32 * s), b1, dS[t]);
        dS[t] = mfma16x16x32<T>(frag(Kt, PC, 16 * t, 32 * s), b2, dS[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) a.ds0[((int64_t)bh * D + rows_of(t, i)) * D + col] = dS[t][i];
}

}  // namespace atma

extern "C" int atma_gated_delta_bwd16_chain(const void* kr, const void* kt, const void* qt, const void* tm,
                                            const void* tt, const void* rt, const void* vt, const void* ot,
                                            const void* got, const float* f, const float* s0,
                                            const float* dst, float* s_entry, float* ds_end, float* dy,
                                            float* ds0, int64_t BH, int64_t NC, int64_t d, int dtype,
                                            void* stream) {
  using namespace atma;
  if (BH < 0 || NC < 0) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: bad sizes");
  if (d != 64 && d != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "gated_delta_bwd16_chain: d = %lld (supported: 64, 128)",
                     (long long)d);
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "gated_delta_bwd16_chain: 16-bit operands only");
  if (BH == 0 || NC == 0) return ATMA_OK;
  if (!kr || !kt || !qt || !tm || !tt || !rt || !vt || !ot || !got || !f || !s_entry || !ds_end || !dy ||
      !ds0)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: null pointer");
  const void* ptrs[] = {kr, kt, qt, tm, tt, rt, vt, ot, got};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: tiles must be 16-byte aligned");
  if (BH * (d / 64) > 0x7fffffff || BH * NC > (1ll << 31))
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: sizes too large");
  Bwd16ChainArgs a{kr, kt, qt, tm, tt, rt, vt, ot, got, f, s0, dst, s_entry, ds_end, dy, ds0, (int)BH, (int)NC};
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(BH * (d / 64)));
  if (dtype == ATMA_BF16) {
    if (d == 128) gdn_bwd16_chain_kernel<bf16, 128><<<grid, dim3(256), 0, s>>>(a);
    else gdn_bwd16_chain_kernel<bf16, 64><<<grid, dim3(256), 0, s>>>(a);
  } else {
    if (d == 128) gdn_bwd16_chain_kernel<f16, 128><<<grid, dim3(256), 0, s>>>(a);
    else gdn_bwd16_chain_kernel<f16, 64><<<grid, dim3(256), 0, s>>>(a);
  }
  return check_launch("gated_delta_bwd16_chain");
}
