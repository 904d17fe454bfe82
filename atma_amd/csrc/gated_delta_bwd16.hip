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
// MI355X mapping: one workgroup of kChainWaves waves per (sequence-head, 16 kChainWaves
// state columns), each wave owning 16 columns (the recurrence never mixes V columns).
// The chunk's shared operands -- k rows, k^T, q^T, T (forward) or T^T (backward), Rq^T,
// 64 x 64 or 64 x d bf16 tiles the caller lays out -- are staged in LDS with rows padded
// by 16 bytes (the
// 16-lane fragment reads then touch 16 distinct bank groups).  Products run on
// v_mfma_f32_16x16x32 (fp32 accumulation); the state and every per-column intermediate
// (Y, U, dU, dY) go through a per-wave transposed bf16 buffer ([column][k], 16 bytes per
// lane per fragment) to become the B operand of the next product.
#include <initializer_list>
#include <type_traits>

#include "common.h"

namespace atma {

// Per-token factor rows of a chunk: Ga, w, beta, Ga_C, lg, then the l2-norm factors of
// the q and k rows: iq = scale / max(|q|, eps), ik = 1 / max(|k|, eps) (scale and 1 without
// l2norm) and uq2 = 1 / |q|^2, uk2 = 1 / |k|^2 where the norm exceeds eps (else 0; 0
// without l2norm), all 0 past the sequence's end.
constexpr int kFRows = 9;

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
  const float* f;    // [N][5][64]  Ga, w, beta, Ga_C (all 64 entries), lg
  const float* s0;   // [BH][D][D] initial state, or null (zero)
  const float* dst;  // [BH][D][D] final-state cotangent, or null (zero)
  void* s_entry;     // [N][D][D]  out (16-bit): each chunk's entry state
  void* ds_end;      // [N][D][D]  out (16-bit): the gradient of each chunk's exit state
  void* u;           // [N][64][D] out (16-bit): U = T diag(beta) (V - diag(Ga) K S)
  float* dy;         // [N][64][D] out: dY
  float* ds0;        // [BH][D][D] out: the gradient of the initial state
  int BH, NC;
};

// A contiguous 16-bit tile of N * NTH 16-byte chunks: thread tid (of NTH) holds chunks
// tid + NTH j.
template <int N, int NTH = 256>
__device__ __forceinline__ void tile_load(u32x4 (&r)[N], const void* src, int tid) {
  const u32x4* s = (const u32x4*)src;
#pragma unroll
  for (int j = 0; j < N; ++j) r[j] = s[tid + NTH * j];
}
// ... into LDS rows of CPR chunks, padded to PITCH elements
template <int N, int CPR, int PITCH, int NTH = 256, typename T>
__device__ __forceinline__ void tile_store(T* dst, const u32x4 (&r)[N], int tid) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int i = tid + NTH * j;
    *(u32x4*)(dst + (i / CPR) * PITCH + 8 * (i % CPR)) = r[j];
  }
}

// Waves (16 state columns each) per workgroup of the chain kernel: two, so a configs[1]
// shape (64 sequence-heads, d = 128) runs 256 workgroups, one per CU (the LDS of one
// workgroup's tiles allows no second).
constexpr int kChainWaves = 2;

template <typename T, int D>
__global__ void __launch_bounds__(64 * kChainWaves, 1) gdn_bwd16_chain_kernel(Bwd16ChainArgs a) {
  constexpr int NW = kChainWaves, NTH = 64 * NW, WC = 16 * NW;  // waves, threads, columns
  constexpr int C = 64, PD = D + 8, PC = C + 8;  // padded LDS pitches (elements)
  constexpr int KS = D / 32;                      // 32-wide k steps over D
  constexpr int DT = D / 16;                      // 16-row tiles over D
  static_assert(D % WC == 0 && 4 * C % NTH == 0, "whole column slabs and factor rows");
  __shared__ __attribute__((aligned(16))) T Kr[C * PD];
  __shared__ __attribute__((aligned(16))) T Kt[D * PC];
  __shared__ __attribute__((aligned(16))) T Qt[D * PC];
  __shared__ __attribute__((aligned(16))) T Tm[C * PC];  // T in the forward chain, T^T in the backward
  __shared__ __attribute__((aligned(16))) T Rt[C * PC];
  __shared__ float Fs[4 * C];
  __shared__ __attribute__((aligned(16))) T Sb[NW][16 * PD];  // S^T / dS^T of the wave's columns
  __shared__ __attribute__((aligned(16))) T X1[NW][16 * PC];
  __shared__ __attribute__((aligned(16))) T X2[NW][16 * PC];
  __shared__ __attribute__((aligned(16))) T XO[NW][16 * PC];  // dO^T rows of the wave's columns
  __shared__ __attribute__((aligned(16))) T XG[NW][16 * PC];  // (Ga dO)^T rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int bh = blockIdx.x / (D / WC);
  const int v0 = WC * (blockIdx.x % (D / WC)) + 16 * wave;  // the wave's first column
  const int col = v0 + c16;                                  // the lane's column (C layout)

  constexpr int NT = C * D / 8 / NTH;   // chunks per thread of a 64 x D or D x 64 tile
  constexpr int NTM = C * C / 8 / NTH;  // ... of a 64 x 64 tile
  constexpr int NF = 4 * C / NTH;       // factor entries per thread
  // the wave's 16 rows of a [D][64] tile: 2 chunks per lane
  auto rows16_load = [&](u32x4 (&r)[2], const void* src) {
    const u32x4* s = (const u32x4*)src;
    r[0] = s[lane];
    r[1] = s[lane + 64];
  };
  auto rows16_store = [&](T* dst, const u32x4 (&r)[2]) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = lane + 64 * k;
      *(u32x4*)(dst + (i >> 3) * PC + 8 * (i & 7)) = r[k];
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
  // the wave's [16 columns][K] 16-bit tile (pitch P) out as K rows of a [K][D] output at
  // columns v0 .. v0 + 15, by transposing reads: 16-byte stores of 8 columns of one row
  // instead of one 2-byte store per element
  auto store_cols = [&](const T* buf, int pitch, auto K_c, T* out) {
    constexpr int K = decltype(K_c)::value;
    const int q = lane >> 4, sl = lane & 15, rr = sl >> 2, cc = 4 * (sl & 3);
#pragma unroll
    for (int u = q; u < 2 * (K / 16); u += 4) {
      const int r0 = 8 * (u & 1), c0 = 16 * (u >> 1);
      const u32x2 lo = lds_read_tr16(buf + (r0 + rr) * pitch + c0 + cc);
      const u32x2 hi = lds_read_tr16(buf + (r0 + 4 + rr) * pitch + c0 + cc);
      *(u32x4*)(out + (int64_t)(c0 + sl) * D + v0 + r0) = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };

  // ---------------------------------------------------------------- forward chain
  f32x4 S[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[t][i] = a.s0 ? a.s0[((int64_t)bh * D + rows_of(t, i)) * D + col] : 0.f;

  // the next chunk's operands are loaded into registers while this one computes
  u32x4 rk[NT], rkt[NT], rtm[NTM];
  u32x2 rv[4];
  float rf[NF];
  auto fwd_load = [&](int64_t n) {
    tile_load<NT, NTH>(rk, (const T*)a.kr + n * C * D, tid);
    tile_load<NT, NTH>(rkt, (const T*)a.kt + n * D * C, tid);
    tile_load<NTM, NTH>(rtm, (const T*)a.tm + n * C * C, tid);
#pragma unroll
    for (int j = 0; j < NF; ++j) rf[j] = a.f[n * kFRows * C + tid + NTH * j];
    const T* vrow = (const T*)a.vt + (n * D + col) * C;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) rv[rt] = *(const u32x2*)(vrow + 16 * rt + 4 * g);
  };
  fwd_load((int64_t)bh * a.NC);
  for (int c = 0; c < a.NC; ++c) {
    const int64_t n = (int64_t)bh * a.NC + c;
    __syncthreads();  // every wave is done with the previous chunk's tiles
    tile_store<NT, D / 8, PD, NTH>(Kr, rk, tid);
    tile_store<NT, 8, PC, NTH>(Kt, rkt, tid);
    tile_store<NTM, 8, PC, NTH>(Tm, rtm, tid);
#pragma unroll
    for (int j = 0; j < NF; ++j) Fs[tid + NTH * j] = rf[j];
    f32x4 Vc[4];  // v of the lane's column, C layout (rows = tokens)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const u32x4 x = {rv[rt][0], rv[rt][1], 0, 0};
      Vc[rt] = f32x4{elem16<T>(x, 0), elem16<T>(x, 1), elem16<T>(x, 2), elem16<T>(x, 3)};
    }
    if (c + 1 < a.NC) fwd_load(n + 1);
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
    // U out through the wave's X1 buffer (its Y^T operand reads are done: in order, one wave)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) put_t(X1[wave], PC, rt, U[rt]);
    wave_sync();
    store_cols(X1[wave], PC, std::integral_constant<int, C>{}, (T*)a.u + n * C * D);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = Fs[C + rows_of(rt, i)] * U[rt][i];
      put_t(X2[wave], PC, rt, x);
    }
    wave_sync();
    // the entry state, then S <- Ga_C S + K^T diag(w) U
    store_cols(Sb[wave], PD, std::integral_constant<int, D>{}, (T*)a.s_entry + n * D * D);  // S^T of this step
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

  u32x4 rq[NT], rrt[NTM], ro[2], rgo[2];
  auto bwd_load = [&](int64_t n) {
    tile_load<NT, NTH>(rk, (const T*)a.kr + n * C * D, tid);
    tile_load<NT, NTH>(rkt, (const T*)a.kt + n * D * C, tid);
    tile_load<NT, NTH>(rq, (const T*)a.qt + n * D * C, tid);
    tile_load<NTM, NTH>(rtm, (const T*)a.tt + n * C * C, tid);
    tile_load<NTM, NTH>(rrt, (const T*)a.rt + n * C * C, tid);
#pragma unroll
    for (int j = 0; j < NF; ++j) rf[j] = a.f[n * kFRows * C + tid + NTH * j];
    rows16_load(ro, (const T*)a.ot + (n * D + v0) * C);
    rows16_load(rgo, (const T*)a.got + (n * D + v0) * C);
  };
  bwd_load((int64_t)bh * a.NC + a.NC - 1);
  for (int c = a.NC - 1; c >= 0; --c) {
    const int64_t n = (int64_t)bh * a.NC + c;
    __syncthreads();
    tile_store<NT, D / 8, PD, NTH>(Kr, rk, tid);
    tile_store<NT, 8, PC, NTH>(Kt, rkt, tid);
    tile_store<NT, 8, PC, NTH>(Qt, rq, tid);
    tile_store<NTM, 8, PC, NTH>(Tm, rtm, tid);
    tile_store<NTM, 8, PC, NTH>(Rt, rrt, tid);
#pragma unroll
    for (int j = 0; j < NF; ++j) Fs[tid + NTH * j] = rf[j];
    rows16_store(XO[wave], ro);
    rows16_store(XG[wave], rgo);
    if (c > 0) bwd_load(n - 1);
#pragma unroll
    for (int t = 0; t < DT; ++t) put_t(Sb[wave], PD, t, dS[t]);
    __syncthreads();
    // the exit-state gradient of this chunk, from its 16-bit transpose
    store_cols(Sb[wave], PD, std::integral_constant<int, D>{}, (T*)a.ds_end + n * D * D);

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

// ------------------------------------------------------------------------------ prep
// One workgroup per chunk-head item n (4 waves): the operand tiles of the chain and of the
// chunk-local gradients.  The raw k, q rows are l2-normalised (q also scaled, as the
// forward does: x / max(|x|, 1e-12)) and rounded to 16 bits once; wave P
// forms row block P of K K^T and Q K^T on MFMA and from them Rq^T and the 16 x 16 blocks of
// N = diag(beta) A (fp32, LDS); then wave 0 inverts I + N -- the four diagonal blocks by
// forward substitution (lane (g, c) solves column c of block g), the blocks below them by
// fp32 block products on v_mfma_f32_16x16x4f32 -- while waves 1-3 write the transposed
// tiles k^T, q^T, v^T, dO^T and (diag(Ga) dO)^T from the LDS rows by transposing reads;
// last, every wave writes T and T^T.
struct Bwd16PrepArgs {
  const void* q;      // (B, T, H, D) 16-bit, raw
  const void* k;      // (B, T, H, D) 16-bit, raw
  const void* v;      // (B, T, H, D) 16-bit
  const void* dO;     // (B, T, H, D) 16-bit
  const float* g;     // (B, T, H) log decay
  const float* beta;  // (B, T, H)
  void *kr, *kt, *qr, *qt, *tm, *tt, *rt, *vt, *ot, *got;
  float* f;
  float scale;
  int l2norm;
  int B, T, H, NC;
};

// Sum over each group of 8 lanes (the two quads of each half row), in every lane.
__device__ __forceinline__ float row8_sum(float x) {
  x += dpp_f32<0xB1>(x);
  x += dpp_f32<0x4E>(x);
  return x + dpp_f32<0x141>(x);
}

// e^x on the hardware exp2 (about 1 ulp), for the prep's per-element decay factors
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

template <typename T, int D>
__global__ void __launch_bounds__(256) gdn_bwd16_prep_kernel(Bwd16PrepArgs a) {
  constexpr int C = 64, PD = D + 8, PT = C + 8, KS = D / 32;
  constexpr int NV = D / 32;  // 16-byte row chunks per thread
  __shared__ __attribute__((aligned(16))) T Ks[C * PD];
  __shared__ __attribute__((aligned(16))) T Qs[C * PD];
  __shared__ __attribute__((aligned(16))) T Vs[C * PD];
  __shared__ __attribute__((aligned(16))) T Os[C * PD];
  // N = diag(beta) A in 16 x 16 blocks: the diagonal blocks as N^T (rows of 16 floats, the
  // substitution's columns) and the six blocks below them in the transposed accumulator
  // layout the block products take (register i of lane (g, c) of block (S, P), S < P:
  // N[16P + c][16S + 4g + i]).  Only wave 0 reads them, in order, so the substitution's
  // T^T diagonal blocks (Mb) overwrite the N^T ones it has consumed, and T, row-major 16-bit,
  // overwrites all of it at the end (84 KiB in all would allow one workgroup per CU; 79 KiB
  // allows two, so one's loads overlap the other's products)
  __shared__ __attribute__((aligned(16))) float Nd[4 * 256 + 6 * 256];
  __shared__ float Lg[C], Bt[C], Gs[C];
  float* Mb = Nd;  // T^T of the diagonal blocks
  T* Tl = (T*)Nd;  // T, row-major, pitch PT
  static_assert(C * PT * (int)sizeof(T) <= (int)sizeof(Nd), "T fits the N blocks' bytes");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t n = blockIdx.x;
  const int bh = (int)(n / a.NC), c = (int)(n % a.NC);
  const int b = bh / a.H, h = bh % a.H;
  const int rows = min(a.T - c * C, C);
  const int64_t tok0 = (int64_t)b * a.T + (int64_t)c * C;
  const int64_t rs = (int64_t)a.H * D;  // token stride (elements)
  const int64_t base = tok0 * rs + (int64_t)h * D;

  // rows (zero past the sequence's end), all loads issued before the stores
  {
    u32x4 kx[NV], qx[NV], vx[NV], ox[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = tid + 256 * j, r = i / (D / 8), ch = i % (D / 8);
      kx[j] = qx[j] = vx[j] = ox[j] = u32x4{0u, 0u, 0u, 0u};
      if (r < rows) {
        const int64_t o = base + r * rs + 8 * ch;
        kx[j] = *(const u32x4*)((const T*)a.k + o);
        qx[j] = *(const u32x4*)((const T*)a.q + o);
        vx[j] = *(const u32x4*)((const T*)a.v + o);
        ox[j] = *(const u32x4*)((const T*)a.dO + o);
      }
    }
    float gl = 0.f, bt = 0.f;
    if (wave == 0 && lane < rows) {
      gl = a.g[(tok0 + lane) * a.H + h];
      bt = a.beta[(tok0 + lane) * a.H + h];
    }
    float* fo = a.f + n * kFRows * C;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = tid + 256 * j, r = i / (D / 8), ch = i % (D / 8);
      // row norms: a row's D / 8 chunks sit in D / 8 consecutive lanes
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {  // packed pairs (v_dot2)
        sk = dot2<T>(kx[j][e], kx[j][e], sk);
        sq = dot2<T>(qx[j][e], qx[j][e], sq);
      }
      if constexpr (D == 128) {
        sk = row16_sum(sk);
        sq = row16_sum(sq);
      } else {
        sk = row8_sum(sk);
        sq = row8_sum(sq);
      }
      const float nk = sqrtf(sk), nq = sqrtf(sq);
      const bool ok = r < rows;
      const float ik = !ok ? 0.f : a.l2norm ? __builtin_amdgcn_rcpf(fmaxf(nk, 1e-12f)) : 1.f;
      const float iq = !ok ? 0.f : (a.l2norm ? __builtin_amdgcn_rcpf(fmaxf(nq, 1e-12f)) : 1.f) * a.scale;
      if (ch == 0) {
        fo[5 * C + r] = iq;
        fo[6 * C + r] = ik;
        fo[7 * C + r] = ok && a.l2norm && nq > 1e-12f ? __builtin_amdgcn_rcpf(sq) : 0.f;
        fo[8 * C + r] = ok && a.l2norm && nk > 1e-12f ? __builtin_amdgcn_rcpf(sk) : 0.f;
      }
      u32x4 kp, qp;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kp[e] = pack2<T>(ik * elem16<T>(kx[j], 2 * e), ik * elem16<T>(kx[j], 2 * e + 1));
        qp[e] = pack2<T>(iq * elem16<T>(qx[j], 2 * e), iq * elem16<T>(qx[j], 2 * e + 1));
      }
      *(u32x4*)(Ks + r * PD + 8 * ch) = kp;
      *(u32x4*)(Qs + r * PD + 8 * ch) = qp;
      *(u32x4*)((T*)a.kr + (n * C + r) * D + 8 * ch) = kp;
      *(u32x4*)((T*)a.qr + (n * C + r) * D + 8 * ch) = qp;
      *(u32x4*)(Vs + r * PD + 8 * ch) = vx[j];
      *(u32x4*)(Os + r * PD + 8 * ch) = ox[j];
    }
    if (wave == 0) {  // inclusive prefix sum of the log decays, per-token factors
      float lg = gl;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(lg, off, 64);
        if (lane >= off) lg += y;
      }
      const float lgC = __shfl(lg, 63, 64);
      const float ga = exp_hw(lg);
      Lg[lane] = lg;
      Bt[lane] = bt;
      Gs[lane] = ga;
      fo[lane] = ga;
      fo[C + lane] = exp_hw(lgC - lg);
      fo[2 * C + lane] = bt;
      fo[3 * C + lane] = exp_hw(lgC);
      fo[4 * C + lane] = lg;
    }
  }
  __syncthreads();

  // row block P = wave of K K^T and Q K^T: Rq^T, the diagonal N block and, from the blocks
  // right of the diagonal (Gram symmetry), the N blocks below it in the block products' layout
  {
    const int P = wave;
    u32x4 ka[KS], qa[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      ka[s] = *(const u32x4*)(Ks + (16 * P + c16) * PD + 32 * s + 8 * g);
      qa[s] = *(const u32x4*)(Qs + (16 * P + c16) * PD + 32 * s + 8 * g);
    }
#pragma unroll
    for (int S = 0; S < 4; ++S) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 kb = *(const u32x4*)(Ks + (16 * S + c16) * PD + 32 * s + 8 * g);
        kk = mfma16x16x32<T>(ka[s], kb, kk);
        qk = mfma16x16x32<T>(qa[s], kb, qk);
      }
      // lane (g, c16) register i: token pair (16 P + 4g + i, 16 S + c16)
      const int sc = 16 * S + c16;
      const float lgs = Lg[sc];
      f32x4 rq;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 16 * P + 4 * g + i;
        rq[i] = sc <= p ? exp_hw(Lg[p] - lgs) * qk[i] : 0.f;
      }
      *(u32x2*)((T*)a.rt + (n * C + sc) * C + 16 * P + 4 * g) = u32x2{pack2<T>(rq[0], rq[1]), pack2<T>(rq[2], rq[3])};
      if (S == P) {  // N^T[c][4g + i] = N[16P + 4g + i][16P + c], strictly lower
        f32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = 16 * P + 4 * g + i;
          v[i] = c16 < 4 * g + i ? Bt[p] * exp_hw(Lg[p] - lgs) * kk[i] : 0.f;
        }
        *(f32x4*)(Nd + P * 256 + c16 * 16 + 4 * g) = v;
      } else if (S > P) {  // N[16S + c][16P + 4g + i] = beta_r e^(lg_r - lg_s) k_s . k_r
        const int r = sc;
        f32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = Bt[r] * exp_hw(Lg[r] - Lg[16 * P + 4 * g + i]) * kk[i];
        *(f32x4*)(Nd + 4 * 256 + tri(P, S - 1) * 256 + lane * 4) = v;
      }
    }
  }
  __syncthreads();

  if (wave == 0) {
    // T = (I + N)^-1.  The diagonal blocks by forward substitution in fp32: lane (g, c) solves
    // column c of block g, N^T rows read from LDS
    {
      const float* nt = Nd + g * 256;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = (r == c16) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < 15; ++j) {
        float nv[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 v = *(const f32x4*)(nt + j * 16 + 4 * q4);  // column j of N
#pragma unroll
          for (int e = 0; e < 4; ++e) nv[4 * q4 + e] = v[e];
        }
#pragma unroll
        for (int r = j + 1; r < 16; ++r) x[r] = fmaf(-nv[r], x[j], x[r]);
      }
      float* mt = Mb + g * 256 + c16 * 16;  // T^T row c = column c of T
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) *(f32x4*)(mt + 4 * q4) = f32x4{x[4 * q4], x[4 * q4 + 1], x[4 * q4 + 2], x[4 * q4 + 3]};
    }
    wave_sync();
    f32x4 tpp[4], tppT[4], at[6];  // T_PP and T_PP^T in the accumulator layout
#pragma unroll
    for (int P = 0; P < 4; ++P) {
      tpp[P] = *(const f32x4*)(Mb + P * 256 + c16 * 16 + 4 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) tppT[P][i] = Mb[P * 256 + (4 * g + i) * 16 + c16];
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) at[k] = *(const f32x4*)(Nd + 4 * 256 + k * 256 + lane * 4);
    // off-diagonal blocks, level L = P - S: T_PS = -T_PP Y_PS with Y_PS = sum_{k=S}^{P-1}
    // N_Pk T_kS, and (T^T)_SP = -Y_PS^T T_PP^T (at(k, P) = block (k, P) of the layout above)
    auto atb = [&](int k, int P) { return at[tri(k, P - 1)]; };
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    const f32x4 y10 = blk_mul(atb(0, 1), tpp[0], z);
    const f32x4 y21 = blk_mul(atb(1, 2), tpp[1], z);
    const f32x4 y32 = blk_mul(atb(2, 3), tpp[2], z);
    const f32x4 t10 = -blk_mul(tppT[1], y10, z);
    const f32x4 t21 = -blk_mul(tppT[2], y21, z);
    const f32x4 tt01 = -blk_mul(y10, tppT[1], z);
    const f32x4 tt12 = -blk_mul(y21, tppT[2], z);
    const f32x4 tt23 = -blk_mul(y32, tppT[3], z);
    const f32x4 y20 = blk_mul(atb(1, 2), t10, blk_mul(atb(0, 2), tpp[0], z));
    const f32x4 y31 = blk_mul(atb(2, 3), t21, blk_mul(atb(1, 3), tpp[1], z));
    const f32x4 t20 = -blk_mul(tppT[2], y20, z);
    const f32x4 tt02 = -blk_mul(y20, tppT[2], z);
    const f32x4 tt13 = -blk_mul(y31, tppT[3], z);
    const f32x4 y30 = blk_mul(atb(2, 3), t20, blk_mul(atb(1, 3), t10, blk_mul(atb(0, 3), tpp[0], z)));
    const f32x4 tt03 = -blk_mul(y30, tppT[3], z);
    // T row-major in 16 bits over the N blocks (every read of them is above): the T^T-form
    // block (S, P) gives row 16P + c, columns 16S + 4g .. + 3 of T (zeros above the diagonal)
    const f32x4 tb[4][4] = {{tppT[0], z, z, z}, {tt01, tppT[1], z, z}, {tt02, tt12, tppT[2], z},
                            {tt03, tt13, tt23, tppT[3]}};
#pragma unroll
    for (int P = 0; P < 4; ++P)
#pragma unroll
      for (int S = 0; S < 4; ++S) {
        const f32x4 v = tb[P][S];
        *(u32x2*)(Tl + (16 * P + c16) * PT + 16 * S + 4 * g) = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
      }
  } else {
    // [D][64] tiles from the LDS rows by transposing reads: a 16-lane group reads 8 rows x 16
    // columns (lane s: row r0 + s / 4 (+ 4), columns c0 + 4 (s % 4) ..), lane i then holds
    // tokens r0 .. r0 + 7 of column c0 + i, one 16-byte chunk of row d = c0 + i of the tile
    const int gi = (tid - 64) >> 4, sl = lane & 15;  // 12 groups of 16 lanes
    const int rr = sl >> 2, cc = 4 * (sl & 3);
    constexpr int UNITS = 5 * (D / 16) * 8;          // (tile, 16-column block, 8-row block)
    for (int u = gi; u < UNITS; u += 12) {
      const int tile = u / ((D / 16) * 8), rem = u % ((D / 16) * 8);
      const int c0 = 16 * (rem / 8), r0 = 8 * (rem % 8);
      const T* src = tile == 0 ? Ks : tile == 1 ? Qs : tile == 2 ? Vs : Os;
      const u32x2 lo = lds_read_tr16(src + (r0 + rr) * PD + c0 + cc);
      const u32x2 hi = lds_read_tr16(src + (r0 + 4 + rr) * PD + c0 + cc);
      u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
      if (tile == 4) {  // (diag(Ga) dO)^T
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack2<T>(Gs[r0 + 2 * e] * elem16<T>(w, 2 * e), Gs[r0 + 2 * e + 1] * elem16<T>(w, 2 * e + 1));
      }
      void* dst = tile == 0 ? a.kt : tile == 1 ? a.qt : tile == 2 ? a.vt : tile == 3 ? a.ot : a.got;
      *(u32x4*)((T*)dst + (n * D + c0 + sl) * C + r0) = w;
    }
  }
  __syncthreads();
  // T and T^T out: 64 rows of 128 bytes each, two 16-byte chunks per thread
  {
    const int row = tid >> 2, ch = 2 * (tid & 3);  // ... chunks ch, ch + 1 of T's row
    T* tmo = (T*)a.tm + (n * C + row) * C;
#pragma unroll
    for (int k = 0; k < 2; ++k) *(u32x4*)(tmo + 8 * (ch + k)) = *(const u32x4*)(Tl + row * PT + 8 * (ch + k));
    // T^T by transposing reads: group gi (16 lanes) takes 16-column block c0 and two 8-row
    // blocks of T
    const int gi = tid >> 4, sl = lane & 15, rr = sl >> 2, cc = 4 * (sl & 3);
    const int c0 = 16 * (gi & 3);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int r0 = 8 * (2 * (gi >> 2) + k);
      const u32x2 lo = lds_read_tr16(Tl + (r0 + rr) * PT + c0 + cc);
      const u32x2 hi = lds_read_tr16(Tl + (r0 + 4 + rr) * PT + c0 + cc);
      *(u32x4*)((T*)a.tt + (n * C + c0 + sl) * C + r0) = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
}

// ------------------------------------------------------------------------------ local
// One workgroup per chunk-head item n (4 waves); wave w owns token rows 16 w .. 16 w + 15 of
// every row-indexed product.  Staged in LDS: the entry state S0 (then the exit-state
// gradient dS, same buffer), U, k rows, k^T, q^T, and the 64 x 64 weight matrices
// GA + GA^T, GR, GR^T built by the waves.  Products on v_mfma_f32_16x16x32 (16-bit
// operands, fp32 accumulation): K K^T, Q K^T, dY U^T, dO U^T (64 x 64), dY S0^T, dO S0^T,
// U dS^T (64 x d), then dK = (GA + GA^T) K + GR^T Q - diag(Ga beta) dY S0^T + diag(w) U dS^T
// and dQ = GR K + diag(Ga) dO S0^T.  The sums over d that the gradients of beta and the
// log decays take reduce to row sums of these products with k and q:
// rowsum(dY o K S0) = rowsum(K o dY S0^T), rowsum(dO o Q S0) = rowsum(Q o dO S0^T),
// rowsum(K dS o U) = rowsum(K o U dS^T).
struct Bwd16LocalArgs {
  const void *kr, *kt, *qr, *qt;
  const void* v;   // (B, T, H, D) 16-bit
  const void* dO;  // (B, T, H, D) 16-bit
  const void *q, *k;  // (B, T, H, D) 16-bit, raw (the l2 norm's backward)
  const float* f;  // [N][kFRows][64]
  const void *s_entry, *ds_end, *u;
  const float* dy;
  void *dq, *dk, *dv;  // (B, T, H, D) 16-bit
  float *dg, *db;  // (B, T, H)
  int B, T, H, NC;
};

template <typename T, int D>
__global__ void __launch_bounds__(256, 1) gdn_bwd16_local_kernel(Bwd16LocalArgs a) {
  constexpr int C = 64, PD = D + 8, PC = C + 8, KS = D / 32, DT = D / 16, NT = D / 32, NSS = D * D / 2048;
  __shared__ __attribute__((aligned(16))) T SS[D * PD];
  __shared__ __attribute__((aligned(16))) T Us[C * PD];
  __shared__ __attribute__((aligned(16))) T Kr[C * PD];
  __shared__ __attribute__((aligned(16))) T Kt[D * PC];
  __shared__ __attribute__((aligned(16))) T Qt[D * PC];
  __shared__ __attribute__((aligned(16))) T M1[C * PC];   // GA
  __shared__ __attribute__((aligned(16))) T M1t[C * PC];  // GA^T
  __shared__ __attribute__((aligned(16))) T GRs[C * PC];  // GR
  __shared__ __attribute__((aligned(16))) T GRt[C * PC];  // GR^T
  __shared__ float Fs[kFRows * C];
  __shared__ float colp[4][C];
  __shared__ float dyv[C], dlgs[C], red[2][4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t n = blockIdx.x;
  const int bh = (int)(n / a.NC), c = (int)(n % a.NC);
  const int b = bh / a.H, h = bh % a.H;
  const int rows = min(a.T - c * C, C);
  const int64_t tok0 = (int64_t)b * a.T + (int64_t)c * C;
  const int64_t rs = (int64_t)a.H * D;
  const int64_t base = tok0 * rs + (int64_t)h * D;
  const int ra = 16 * wave + c16;  // the lane's row as an A operand

  // staged tiles and the wave's A-operand rows, all loads first
  u32x4 rss[NSS], rds[NSS], ru[NT], rk[NT], rkt[NT], rqt[NT];
  tile_load(rss, (const T*)a.s_entry + n * D * D, tid);
  tile_load(rds, (const T*)a.ds_end + n * D * D, tid);
  tile_load(ru, (const T*)a.u + n * C * D, tid);
  tile_load(rk, (const T*)a.kr + n * C * D, tid);
  tile_load(rkt, (const T*)a.kt + n * D * C, tid);
  tile_load(rqt, (const T*)a.qt + n * D * C, tid);
  f32x4 dyl[KS][2];
  u32x4 doA[KS], vA[KS], uA[KS], kA[KS], qA[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const float* yr = a.dy + (n * C + ra) * D + 32 * s + 8 * g;
    dyl[s][0] = *(const f32x4*)yr;
    dyl[s][1] = *(const f32x4*)(yr + 4);
    doA[s] = vA[s] = u32x4{0u, 0u, 0u, 0u};
    if (ra < rows) {
      doA[s] = *(const u32x4*)((const T*)a.dO + base + ra * rs + 32 * s + 8 * g);
      vA[s] = *(const u32x4*)((const T*)a.v + base + ra * rs + 32 * s + 8 * g);
    }
    uA[s] = *(const u32x4*)((const T*)a.u + (n * C + ra) * D + 32 * s + 8 * g);
    kA[s] = *(const u32x4*)((const T*)a.kr + (n * C + ra) * D + 32 * s + 8 * g);
    qA[s] = *(const u32x4*)((const T*)a.qr + (n * C + ra) * D + 32 * s + 8 * g);
  }
  for (int i = tid; i < kFRows * C; i += 256) Fs[i] = a.f[n * kFRows * C + i];
  // the raw k and q elements of the lane's dK / dQ tile entries (row 16 wave + 4g + i, column
  // 16 t + c16), for the l2 norm's backward at the end: loaded now, so their latency passes
  // under the products
  T kraw16[DT][4], qraw16[DT][4];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 16 * wave + 4 * g + i;
      kraw16[t][i] = qraw16[t][i] = from_f32<T>(0.f);
      if (p < rows) {
        kraw16[t][i] = ((const T*)a.k)[base + p * rs + 16 * t + c16];
        qraw16[t][i] = ((const T*)a.q)[base + p * rs + 16 * t + c16];
      }
    }
  tile_store<NSS, D / 8, PD>(SS, rss, tid);
  tile_store<NT, D / 8, PD>(Us, ru, tid);
  tile_store<NT, D / 8, PD>(Kr, rk, tid);
  tile_store<NT, 8, PC>(Kt, rkt, tid);
  tile_store<NT, 8, PC>(Qt, rqt, tid);
  const float* Ga = Fs;
  const float* Wf = Fs + C;
  const float* Bf = Fs + 2 * C;
  const float* Lgf = Fs + 4 * C;
  __syncthreads();

  // dV = diag(beta) dY and rowsum(dY o V) from the wave's rows; dY as A operand
  u32x4 dyA[KS];
  {
    const float bt = Bf[ra];
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const f32x4 y0 = dyl[s][0], y1 = dyl[s][1];
      dyA[s] = u32x4{pack2<T>(y0[0], y0[1]), pack2<T>(y0[2], y0[3]), pack2<T>(y1[0], y1[1]), pack2<T>(y1[2], y1[3])};
#pragma unroll
      for (int e = 0; e < 4; ++e) part = fmaf(y0[e], elem16<T>(vA[s], e), fmaf(y1[e], elem16<T>(vA[s], 4 + e), part));
      if (ra < rows)
        *(u32x4*)((T*)a.dv + base + ra * rs + 32 * s + 8 * g) =
            u32x4{pack2<T>(bt * y0[0], bt * y0[1]), pack2<T>(bt * y0[2], bt * y0[3]),
                  pack2<T>(bt * y1[0], bt * y1[1]), pack2<T>(bt * y1[2], bt * y1[3])};
    }
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    if (g == 0) dyv[ra] = part;
  }

  // 64 x 64 products of the wave's rows: A, Rq, dL, dRq, and the weights GA, GR
  float dbl[4] = {0.f, 0.f, 0.f, 0.f}, lgl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int S = 0; S < 4; ++S) {
    f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk, yl = kk, ou = kk;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 kb = *(const u32x4*)(Kr + (16 * S + c16) * PD + 32 * s + 8 * g);
      const u32x4 ub = *(const u32x4*)(Us + (16 * S + c16) * PD + 32 * s + 8 * g);
      kk = mfma16x16x32<T>(kA[s], kb, kk);
      qk = mfma16x16x32<T>(qA[s], kb, qk);
      yl = mfma16x16x32<T>(dyA[s], ub, yl);
      ou = mfma16x16x32<T>(doA[s], ub, ou);
    }
    const int sc = 16 * S + c16;
    const float lgs = Lgf[sc];
    f32x4 ga, gr;
    float colv = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 16 * wave + 4 * g + i;
      const float e = sc <= p ? exp_hw(Lgf[p] - lgs) : 0.f;
      const float A = sc < p ? e * kk[i] : 0.f;
      const float Rq = e * qk[i];
      const float dL = sc < p ? -yl[i] : 0.f;
      const float dA = Bf[p] * dL;
      const float dRq = sc <= p ? ou[i] : 0.f;
      ga[i] = dA * e;
      gr[i] = dRq * e;
      dbl[i] = fmaf(dL, A, dbl[i]);
      const float x = fmaf(dA, A, dRq * Rq);
      lgl[i] += x;
      colv += x;
      M1[p * PC + sc] = from_f32<T>(ga[i]);
      GRs[p * PC + sc] = from_f32<T>(gr[i]);
    }
    const int p0 = 16 * wave + 4 * g;
    *(u32x2*)(M1t + sc * PC + p0) = u32x2{pack2<T>(ga[0], ga[1]), pack2<T>(ga[2], ga[3])};
    *(u32x2*)(GRt + sc * PC + p0) = u32x2{pack2<T>(gr[0], gr[1]), pack2<T>(gr[2], gr[3])};
    colv += __shfl_xor(colv, 16, 64);
    colv += __shfl_xor(colv, 32, 64);
    if (g == 0) colp[wave][sc] = colv;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dbl[i] = row16_sum(dbl[i]);
    lgl[i] = row16_sum(lgl[i]);
  }

  // dY S0^T and dO S0^T (B operand: S0 rows = output columns)
  f32x4 P1[DT], P2[DT], P3[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    P1[t] = P2[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 sb = *(const u32x4*)(SS + (16 * t + c16) * PD + 32 * s + 8 * g);
      P1[t] = mfma16x16x32<T>(dyA[s], sb, P1[t]);
      P2[t] = mfma16x16x32<T>(doA[s], sb, P2[t]);
    }
  }
  // <dS, S0> over the thread's chunks, then dS replaces S0
  {
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < NSS; ++j) {
      const int i = tid + 256 * j;
      const u32x4 sx = *(const u32x4*)(SS + (i / (D / 8)) * PD + 8 * (i % (D / 8)));
#pragma unroll
      for (int e = 0; e < 8; ++e) part = fmaf(elem16<T>(sx, e), elem16<T>(rds[j], e), part);
    }
    part = wave_sum(part);
    if (lane == 0) red[0][wave] = part;
  }
  __syncthreads();
  tile_store<NSS, D / 8, PD>(SS, rds, tid);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    P3[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
      P3[t] = mfma16x16x32<T>(uA[s], *(const u32x4*)(SS + (16 * t + c16) * PD + 32 * s + 8 * g), P3[t]);
  }

  // dK, dQ: A operands (GA + GA^T), GR^T, GR rows; B operands k^T, q^T rows (= columns d)
  u32x4 g1A[2], grtA[2], grA[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const u32x4 m = *(const u32x4*)(M1 + ra * PC + 32 * j + 8 * g);
    const u32x4 mt = *(const u32x4*)(M1t + ra * PC + 32 * j + 8 * g);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = pack2<T>(elem16<T>(m, 2 * e) + elem16<T>(mt, 2 * e), elem16<T>(m, 2 * e + 1) + elem16<T>(mt, 2 * e + 1));
    g1A[j] = u32x4{w[0], w[1], w[2], w[3]};
    grtA[j] = *(const u32x4*)(GRt + ra * PC + 32 * j + 8 * g);
    grA[j] = *(const u32x4*)(GRs + ra * PC + 32 * j + 8 * g);
  }
  float rk1[4] = {0.f, 0.f, 0.f, 0.f}, rq2[4] = {0.f, 0.f, 0.f, 0.f}, rk3[4] = {0.f, 0.f, 0.f, 0.f};
  // gradients of the normalised rows (dKn, dQs), then the l2 norm's backward:
  // dx = i_x dX - i_x u_x2 x (x . dX) with x the raw row
  f32x4 dKn[DT], dQs[DT], kraw[DT], qraw[DT];
  float xk[4] = {0.f, 0.f, 0.f, 0.f}, xq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    f32x4 dk = {0.f, 0.f, 0.f, 0.f}, dq = dk;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 kb = *(const u32x4*)(Kt + (16 * t + c16) * PC + 32 * j + 8 * g);
      const u32x4 qb = *(const u32x4*)(Qt + (16 * t + c16) * PC + 32 * j + 8 * g);
      dk = mfma16x16x32<T>(g1A[j], kb, dk);
      dk = mfma16x16x32<T>(grtA[j], qb, dk);
      dq = mfma16x16x32<T>(grA[j], kb, dq);
    }
    const int d = 16 * t + c16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 16 * wave + 4 * g + i;
      const float kv = to_f32(Kt[d * PC + p]), qv = to_f32(Qt[d * PC + p]);
      rk1[i] = fmaf(kv, P1[t][i], rk1[i]);
      rq2[i] = fmaf(qv, P2[t][i], rq2[i]);
      rk3[i] = fmaf(kv, P3[t][i], rk3[i]);
      dKn[t][i] = dk[i] - Ga[p] * Bf[p] * P1[t][i] + Wf[p] * P3[t][i];
      dQs[t][i] = dq[i] + Ga[p] * P2[t][i];
      kraw[t][i] = to_f32(kraw16[t][i]);
      qraw[t][i] = to_f32(qraw16[t][i]);
      xk[i] = fmaf(kraw[t][i], dKn[t][i], xk[i]);
      xq[i] = fmaf(qraw[t][i], dQs[t][i], xq[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 16 * wave + 4 * g + i;
    const float iq = Fs[5 * C + p], ik = Fs[6 * C + p];
    const float pq = iq * Fs[7 * C + p] * row16_sum(xq[i]), pk = ik * Fs[8 * C + p] * row16_sum(xk[i]);
    if (p < rows) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int64_t o = base + p * rs + 16 * t + c16;
        ((T*)a.dk)[o] = from_f32<T>(ik * dKn[t][i] - pk * kraw[t][i]);
        ((T*)a.dq)[o] = from_f32<T>(iq * dQs[t][i] - pq * qraw[t][i]);
      }
    }
  }
  // gradients of beta and of the log decays, per row
  float wsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 16 * wave + 4 * g + i;
    const float k1 = row16_sum(rk1[i]), q2 = row16_sum(rq2[i]), k3 = row16_sum(rk3[i]);
    if (c16 == 0) {
      if (p < rows) a.db[(tok0 + p) * a.H + h] = dyv[p] - Ga[p] * k1 + dbl[i];
      dlgs[p] = lgl[i] + Ga[p] * (q2 - Bf[p] * k1) - Wf[p] * k3;
      wsum = fmaf(Wf[p], k3, wsum);
    }
  }
  wsum = wave_sum(wsum);
  if (lane == 0) red[1][wave] = wsum;
  __syncthreads();
  if (wave == 0) {
    float x = dlgs[lane] - (colp[0][lane] + colp[1][lane] + colp[2][lane] + colp[3][lane]);
    if (lane == C - 1)
      x += red[1][0] + red[1][1] + red[1][2] + red[1][3] +
           Fs[3 * C] * (red[0][0] + red[0][1] + red[0][2] + red[0][3]);
    // reverse cumulative sum: dg[p] = sum over s >= p
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_down(x, off, 64);
      if (lane + off < 64) x += y;
    }
    if (lane < rows) a.dg[(tok0 + lane) * a.H + h] = x;
  }
}

}  // namespace atma

// ------------------------------------------------------------------------------ C ABI
namespace {

bool bwd16_dims_ok(int64_t d, int dtype, const char* who) {
  using namespace atma;
  if (d != 64 && d != 128) {
    set_error(ATMA_ERR_UNSUPPORTED, "%s: d = %lld (supported: 64, 128)", who, (long long)d);
    return false;
  }
  if (dtype != ATMA_BF16 && dtype != ATMA_F16) {
    set_error(ATMA_ERR_UNSUPPORTED, "%s: 16-bit operands only", who);
    return false;
  }
  return true;
}

bool aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if ((uintptr_t)p % 16) return false;
  return true;
}

}  // namespace

#define ATMA_BWD16_DISPATCH_NT(KERNEL, grid, nthreads, stream, args)                          \
  do {                                                                                        \
    if (dtype == ATMA_BF16) {                                                                 \
      if (d == 128) atma::KERNEL<atma::bf16, 128><<<grid, dim3(nthreads), 0, stream>>>(args); \
      else atma::KERNEL<atma::bf16, 64><<<grid, dim3(nthreads), 0, stream>>>(args);           \
    } else {                                                                                  \
      if (d == 128) atma::KERNEL<atma::f16, 128><<<grid, dim3(nthreads), 0, stream>>>(args);  \
      else atma::KERNEL<atma::f16, 64><<<grid, dim3(nthreads), 0, stream>>>(args);            \
    }                                                                                         \
  } while (0)
#define ATMA_BWD16_DISPATCH(KERNEL, grid, stream, args) ATMA_BWD16_DISPATCH_NT(KERNEL, grid, 256, stream, args)

extern "C" int atma_gated_delta_bwd16_prep(const void* q, const void* k, const void* v, const void* d_out,
                                           const float* g, const float* beta, void* kr, void* kt, void* qr,
                                           void* qt, void* tm, void* tt, void* rt, void* vt, void* ot, void* got,
                                           float* f, int64_t B, int64_t T, int64_t H, int64_t d, float scale,
                                           int l2norm, int dtype, void* stream) {
  using namespace atma;
  if (!bwd16_dims_ok(d, dtype, "gated_delta_bwd16_prep")) return ATMA_ERR_UNSUPPORTED;
  if (B < 0 || T < 0 || H <= 0) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_prep: bad sizes");
  const int64_t NC = (T + 63) / 64;
  if (B == 0 || NC == 0) return ATMA_OK;
  if (!q || !k || !v || !d_out || !g || !beta || !kr || !kt || !qr || !qt || !tm || !tt || !rt || !vt || !ot ||
      !got || !f)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_prep: null pointer");
  if (!aligned16({q, k, v, d_out, kr, kt, qr, qt, tm, tt, rt, vt, ot, got}))
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_prep: operands must be 16-byte aligned");
  if (B * H * NC > 0x7fffffff || B * T > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_prep: sizes too large");
  Bwd16PrepArgs a{q, k, v, d_out, g, beta, kr, kt, qr, qt, tm, tt, rt, vt, ot, got, f, scale, l2norm ? 1 : 0,
                  (int)B, (int)T, (int)H, (int)NC};
  const dim3 grid((unsigned)(B * H * NC));
  ATMA_BWD16_DISPATCH(gdn_bwd16_prep_kernel, grid, (hipStream_t)stream, a);
  return check_launch("gated_delta_bwd16_prep");
}

extern "C" int atma_gated_delta_bwd16_chain(const void* kr, const void* kt, const void* qt, const void* tm,
                                            const void* tt, const void* rt, const void* vt, const void* ot,
                                            const void* got, const float* f, const float* s0, const float* dst,
                                            void* s_entry, void* ds_end, void* u, float* dy, float* ds0,
                                            int64_t BH, int64_t NC, int64_t d, int dtype, void* stream) {
  using namespace atma;
  if (!bwd16_dims_ok(d, dtype, "gated_delta_bwd16_chain")) return ATMA_ERR_UNSUPPORTED;
  if (BH < 0 || NC < 0) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: bad sizes");
  if (BH == 0 || NC == 0) return ATMA_OK;
  if (!kr || !kt || !qt || !tm || !tt || !rt || !vt || !ot || !got || !f || !s_entry || !ds_end || !u || !dy ||
      !ds0)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: null pointer");
  if (!aligned16({kr, kt, qt, tm, tt, rt, vt, ot, got, s_entry, ds_end, u, dy}))
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: tiles and outputs must be 16-byte aligned");
  const int64_t slabs = d / (16 * kChainWaves);  // column slabs (workgroups) per sequence-head
  if (BH * slabs > 0x7fffffff || BH * NC > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_chain: sizes too large");
  Bwd16ChainArgs a{kr, kt, qt, tm, tt, rt, vt, ot, got, f, s0, dst, s_entry, ds_end, u, dy, ds0,
                   (int)BH, (int)NC};
  const dim3 grid((unsigned)(BH * slabs));
  ATMA_BWD16_DISPATCH_NT(gdn_bwd16_chain_kernel, grid, 64 * kChainWaves, (hipStream_t)stream, a);
  return check_launch("gated_delta_bwd16_chain");
}

extern "C" int atma_gated_delta_bwd16_local(const void* kr, const void* kt, const void* qr, const void* qt,
                                            const void* q, const void* k, const void* v, const void* d_out,
                                            const float* f, const void* s_entry, const void* ds_end, const void* u,
                                            const float* dy, void* dq, void* dk, void* dv, float* dg, float* dbeta,
                                            int64_t B, int64_t T, int64_t H, int64_t d, int dtype, void* stream) {
  using namespace atma;
  if (!bwd16_dims_ok(d, dtype, "gated_delta_bwd16_local")) return ATMA_ERR_UNSUPPORTED;
  if (B < 0 || T < 0 || H <= 0) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_local: bad sizes");
  const int64_t NC = (T + 63) / 64;
  if (B == 0 || NC == 0) return ATMA_OK;
  if (!kr || !kt || !qr || !qt || !q || !k || !v || !d_out || !f || !s_entry || !ds_end || !u || !dy || !dq ||
      !dk || !dv || !dg || !dbeta)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_local: null pointer");
  if (!aligned16({kr, kt, qr, qt, v, d_out, s_entry, ds_end, u, dy, dv}))
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_local: operands must be 16-byte aligned");
  if (B * H * NC > 0x7fffffff || B * T > 0x7fffffff)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd16_local: sizes too large");
  Bwd16LocalArgs a{kr, kt, qr, qt, v, d_out, q, k, f, s_entry, ds_end, u, dy, dq, dk, dv, dg, dbeta,
                   (int)B, (int)T, (int)H, (int)NC};
  const dim3 grid((unsigned)(B * H * NC));
  ATMA_BWD16_DISPATCH(gdn_bwd16_local_kernel, grid, (hipStream_t)stream, a);
  return check_launch("gated_delta_bwd16_local");
}
