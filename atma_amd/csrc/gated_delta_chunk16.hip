// Chunked gated-delta prefill for bf16 / fp16 inputs on MFMA (v_mfma_f32_16x16x32).
//
// Same algebra as the fp32 path (gated_delta_chunk.hip, after gated_delta_chunked,
// model/blocks.py:375-423), split so the sequential part is short:
//
//  pass 1, gdn_prep16 -- one workgroup per (sequence, head, chunk), fully parallel:
//    L2-normalise the chunk's q/k rows, form the Gram blocks K K^T and Q K^T on
//    MFMA, build A[p,s] = beta_p exp(lg_p - lg_s) k_p.k_s (s < p) and
//    Rq[p,s] = exp(lg_p - lg_s) q_p.k_s (s <= p), invert the unit lower-triangular
//    I + A in fp32 by 16x16 blocks (forward substitution on the diagonal blocks,
//    then three levels of block products), and store T diag(beta) and Rq as 16-bit
//    64x64 matrices plus the chunk's inclusive log-decays (16.6 KB per chunk).
//
//  pass 2, gdn_scan16 -- one workgroup per (sequence, head, 32-column slab of the
//    [K, V] state), chunks in order.  The 128 x 32 fp32 slab lives in MFMA
//    accumulator registers for the whole sequence (a 16-bit copy in LDS feeds the
//    B operands).  Per chunk, with ge_p = exp(lg_p), tail_p = exp(lg_C - lg_p):
//        X = V - diag(ge) K S          (K: normalised keys)
//        U = (T diag(beta)) X
//        O = diag(ge) Q S + Rq U       -> output rows
//        S = exp(lg_C) S + (diag(tail) K)^T U
//    The products run on 16-bit MFMA with fp32 accumulation (the state itself stays
//    fp32); the next chunk's rows are prefetched into registers during the math.
#include "gated_delta.h"

namespace atma {

__device__ __forceinline__ u32x4 lds16(const void* p) { return *(const u32x4*)p; }

template <typename T, int D>
__global__ void __launch_bounds__(256) gdn_prep16_kernel(GdnArgs a) {
  constexpr int C = kChunk, KP = D + 8, FP = C + 1;
  constexpr int EPT = D / 4, VPT = EPT / 8;  // 4 threads per row
  __shared__ __attribute__((aligned(16))) T Kn[C * KP];
  __shared__ __attribute__((aligned(16))) T Qn[C * KP];
  __shared__ float Af[C * FP], Tf[C * FP], Rf[C * FP];
  __shared__ float Yf[3 * 256];
  __shared__ float lg[C], bet[C];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;
  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int t0 = c * C;

  {  // rows: load, L2-normalise, scale q
    const int p = tid >> 2, qq = tid & 3;
    const int t = t0 + p;
    const bool ok = t < a.T;
    const T* kr = (const T*)a.k + b * a.k_sb + (int64_t)t * a.k_st + h * a.k_sh + qq * EPT;
    const T* qr = (const T*)a.q + b * a.q_sb + (int64_t)t * a.q_st + h * a.q_sh + qq * EPT;
    u32x4 kv[VPT], qv[VPT];
    float ks = 0.f, qs = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      kv[i] = ok ? *(const u32x4*)(kr + 8 * i) : u32x4{0, 0, 0, 0};
      qv[i] = ok ? *(const u32x4*)(qr + 8 * i) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = elem16<T>(kv[i], e), y = elem16<T>(qv[i], e);
        ks += x * x;
        qs += y * y;
      }
    }
    ks += __shfl_xor(ks, 1, 64);
    ks += __shfl_xor(ks, 2, 64);
    qs += __shfl_xor(qs, 1, 64);
    qs += __shfl_xor(qs, 2, 64);
    const float ik = a.l2norm ? 1.f / fmaxf(sqrtf(ks), 1e-12f) : 1.f;
    const float iq = (a.l2norm ? 1.f / fmaxf(sqrtf(qs), 1e-12f) : 1.f) * a.scale;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      u32x4 ko, qo;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        ko[w] = pack2<T>(elem16<T>(kv[i], 2 * w) * ik, elem16<T>(kv[i], 2 * w + 1) * ik);
        qo[w] = pack2<T>(elem16<T>(qv[i], 2 * w) * iq, elem16<T>(qv[i], 2 * w + 1) * iq);
      }
      *(u32x4*)(Kn + p * KP + qq * EPT + 8 * i) = ko;
      *(u32x4*)(Qn + p * KP + qq * EPT + 8 * i) = qo;
    }
    if (tid < C) {
      const int tt = t0 + tid;
      const int64_t gi = ((int64_t)b * a.T + tt) * a.H + h;
      lg[tid] = tt < a.T ? a.g[gi] : 0.f;
      bet[tid] = tt < a.T ? a.beta[gi] : 0.f;
    }
  }
  __syncthreads();
  if (wave == 0) {  // inclusive prefix sum of the log-decays
    float x = lg[lane];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    lg[lane] = x;
  }
  __syncthreads();

  // ---- Gram tiles on the lower block triangle: 10 (tp >= ts) for K K^T and Q K^T each
  {
    for (int task = wave; task < 20; task += 4) {
      const int which = task / 10, idx = task % 10;
      const int tp = (idx >= 1) + (idx >= 3) + (idx >= 6);
      const int ts = idx - tp * (tp + 1) / 2;
      const T* arow = (which ? Qn : Kn) + (16 * tp + c16) * KP + 8 * g;
      const T* brow = Kn + (16 * ts + c16) * KP + 8 * g;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < D / 32; ++s) acc = mfma16x16x32<T>(lds16(arow + 32 * s), lds16(brow + 32 * s), acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 16 * tp + 4 * g + i, s = 16 * ts + c16;
        const float dec = s <= p ? expf(lg[p] - lg[s]) : 0.f;
        if (which == 0)
          Af[p * FP + s] = s < p ? bet[p] * dec * acc[i] : 0.f;
        else
          Rf[p * FP + s] = s <= p ? dec * acc[i] : 0.f;
      }
    }
  }
  __syncthreads();

  // ---- T = (I + A)^-1: diagonal 16x16 blocks by forward substitution (lane = column)
  if (wave == 0) {
    const int bb = lane >> 4, cc = lane & 15;
    float col[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float acc = (r == cc) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < r; ++j) acc -= Af[(16 * bb + r) * FP + 16 * bb + j] * col[j];
      col[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Tf[(16 * bb + r) * FP + 16 * bb + cc] = col[r];
  }
  __syncthreads();
  // ---- off-diagonal blocks: T_ij = -T_ii * sum_{k=j}^{i-1} A_ik T_kj, level L = i - j
  for (int L = 1; L < 4; ++L) {
    const int nblk = 4 - L;
    for (int e = tid; e < nblk * 256; e += 256) {
      const int blk = e >> 8, r = (e >> 4) & 15, cc = e & 15;
      const int i = L + blk, j = blk;
      float y = 0.f;
      for (int kk = j; kk < i; ++kk)
#pragma unroll
        for (int m = 0; m < 16; ++m) y += Af[(16 * i + r) * FP + 16 * kk + m] * Tf[(16 * kk + m) * FP + 16 * j + cc];
      Yf[e] = y;
    }
    __syncthreads();
    for (int e = tid; e < nblk * 256; e += 256) {
      const int blk = e >> 8, r = (e >> 4) & 15, cc = e & 15;
      const int i = L + blk, j = blk;
      float x = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m) x -= Tf[(16 * i + r) * FP + 16 * i + m] * Yf[blk * 256 + m * 16 + cc];
      Tf[(16 * i + r) * FP + 16 * j + cc] = x;
    }
    __syncthreads();
  }

  // ---- record: T diag(beta), Rq (16-bit, zero above the diagonal), log-decays
  char* rec = (char*)a.ws + ((int64_t)bh * a.NC + c) * kGdn16RecBytes;
  T* tb = (T*)rec;
  T* rq = tb + C * C;
  float* lgo = (float*)(rq + C * C);
  for (int e = tid; e < C * C / 8; e += 256) {
    const int p = e >> 3, s0 = (e & 7) * 8;
    u32x4 xt, xr;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int s = s0 + 2 * w;
      const float t0v = s <= p ? Tf[p * FP + s] * bet[s] : 0.f;
      const float t1v = s + 1 <= p ? Tf[p * FP + s + 1] * bet[s + 1] : 0.f;
      const float r0v = s <= p ? Rf[p * FP + s] : 0.f;
      const float r1v = s + 1 <= p ? Rf[p * FP + s + 1] : 0.f;
      xt[w] = pack2<T>(t0v, t1v);
      xr[w] = pack2<T>(r0v, r1v);
    }
    *(u32x4*)(tb + p * C + s0) = xt;
    *(u32x4*)(rq + p * C + s0) = xr;
  }
  if (tid < C) lgo[tid] = lg[tid];
}

template <typename T, int D>
__global__ void __launch_bounds__(256) gdn_scan16_kernel(GdnArgs a) {
  constexpr int C = kChunk, VS = 32, KP = D + 8, CP = C + 8;
  constexpr int EPT = D / 4, VPT = EPT / 8;
  constexpr int KTW = D / 64;  // 16-row state tiles per wave
  __shared__ __attribute__((aligned(16))) T Kn[C * KP];
  __shared__ __attribute__((aligned(16))) T Qn[C * KP];
  __shared__ __attribute__((aligned(16))) T KdT[D * CP];
  __shared__ __attribute__((aligned(16))) T Tb[C * CP];
  __shared__ __attribute__((aligned(16))) T Rq[C * CP];
  __shared__ __attribute__((aligned(16))) T Sb[VS * KP];
  __shared__ __attribute__((aligned(16))) T XT[VS * CP];
  __shared__ __attribute__((aligned(16))) T UT[VS * CP];
  __shared__ float s_ge[C], s_tail[C];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;
  const int bh = blockIdx.x, v0 = blockIdx.y * VS;
  const int b = bh / a.H, h = bh % a.H;

  // ---- state slab in accumulators: tiles (k-tile wave*KTW + j, v-tile vt)
  f32x4 S[KTW][2];
#pragma unroll
  for (int j = 0; j < KTW; ++j)
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      const int kt = wave * KTW + j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kx = 16 * kt + 4 * g + i, vx = v0 + 16 * vt + c16;
        S[j][vt][i] = a.s0 ? a.s0[((int64_t)bh * D + kx) * D + vx] : 0.f;
      }
      u32x2 pk = {pack2<T>(S[j][vt][0], S[j][vt][1]), pack2<T>(S[j][vt][2], S[j][vt][3])};
      *(u32x2*)(Sb + (16 * vt + c16) * KP + 16 * kt + 4 * g) = pk;
    }

  // ---- register prefetch of one chunk's rows and record
  const int rp = tid >> 2, rq4 = tid & 3;
  u32x4 kpre[VPT], qpre[VPT], tpre[2], rpre[2];
  float vpre[2][4];  // V at rows 16*wave + 4g + i, columns v0 + 16vt + c16
  float lgpre = 0.f, lgcpre = 0.f;
  auto prefetch = [&](int c) {
#pragma unroll
    for (int vt = 0; vt < 2; ++vt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = c * C + 16 * wave + 4 * g + i;
        vpre[vt][i] =
            t < a.T ? to_f32(((const T*)a.v)[b * a.v_sb + (int64_t)t * a.v_st + h * a.v_sh + v0 + 16 * vt + c16])
                    : 0.f;
      }
    const int t = c * C + rp;
    const bool ok = t < a.T;
    const T* kr = (const T*)a.k + b * a.k_sb + (int64_t)t * a.k_st + h * a.k_sh + rq4 * EPT;
    const T* qr = (const T*)a.q + b * a.q_sb + (int64_t)t * a.q_st + h * a.q_sh + rq4 * EPT;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      kpre[i] = ok ? *(const u32x4*)(kr + 8 * i) : u32x4{0, 0, 0, 0};
      qpre[i] = ok ? *(const u32x4*)(qr + 8 * i) : u32x4{0, 0, 0, 0};
    }
    const T* rec = (const T*)((const char*)a.ws + ((int64_t)bh * a.NC + c) * kGdn16RecBytes);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int e = tid + 256 * r;
      tpre[r] = *(const u32x4*)(rec + 8 * e);
      rpre[r] = *(const u32x4*)(rec + C * C + 8 * e);
    }
    const float* lgr = (const float*)(rec + 2 * C * C);
    if (tid < C) lgpre = lgr[tid];
    lgcpre = lgr[C - 1];
  };
  prefetch(0);

  for (int c = 0; c < a.NC; ++c) {
    // ---- phase L: normalised rows, record matrices, decays
    {
      float ks = 0.f, qs = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = elem16<T>(kpre[i], e), y = elem16<T>(qpre[i], e);
          ks += x * x;
          qs += y * y;
        }
      ks += __shfl_xor(ks, 1, 64);
      ks += __shfl_xor(ks, 2, 64);
      qs += __shfl_xor(qs, 1, 64);
      qs += __shfl_xor(qs, 2, 64);
      const float ik = a.l2norm ? 1.f / fmaxf(sqrtf(ks), 1e-12f) : 1.f;
      const float iq = (a.l2norm ? 1.f / fmaxf(sqrtf(qs), 1e-12f) : 1.f) * a.scale;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        u32x4 ko, qo;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          ko[w] = pack2<T>(elem16<T>(kpre[i], 2 * w) * ik, elem16<T>(kpre[i], 2 * w + 1) * ik);
          qo[w] = pack2<T>(elem16<T>(qpre[i], 2 * w) * iq, elem16<T>(qpre[i], 2 * w + 1) * iq);
        }
        *(u32x4*)(Kn + rp * KP + rq4 * EPT + 8 * i) = ko;
        *(u32x4*)(Qn + rp * KP + rq4 * EPT + 8 * i) = qo;
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = tid + 256 * r;
        const int p = e >> 3, s0 = (e & 7) * 8;
        *(u32x4*)(Tb + p * CP + s0) = tpre[r];
        *(u32x4*)(Rq + p * CP + s0) = rpre[r];
      }
      if (tid < C) {
        s_ge[tid] = expf(lgpre);
        s_tail[tid] = expf(lgcpre - lgpre);
      }
    }
    const float gC = expf(lgcpre);
    float vcur[2][4];
#pragma unroll
    for (int vt = 0; vt < 2; ++vt)
#pragma unroll
      for (int i = 0; i < 4; ++i) vcur[vt][i] = vpre[vt][i];
    __syncthreads();
    if (c + 1 < a.NC) prefetch(c + 1);

    // ---- phase K: KdT[k][p] = tail_p * Kn[p][k]  (4 rows x 8 dims per thread)
    for (int e = tid; e < (C / 4) * (D / 8); e += 256) {
      const int p4 = e & 15, kc = e >> 4;
      u32x4 r[4];
      float tl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r[i] = lds16(Kn + (4 * p4 + i) * KP + 8 * kc);
        tl[i] = s_tail[4 * p4 + i];
      }
#pragma unroll
      for (int ee = 0; ee < 8; ++ee) {
        u32x2 pk = {pack2<T>(elem16<T>(r[0], ee) * tl[0], elem16<T>(r[1], ee) * tl[1]),
                    pack2<T>(elem16<T>(r[2], ee) * tl[2], elem16<T>(r[3], ee) * tl[3])};
        *(u32x2*)(KdT + (8 * kc + ee) * CP + 4 * p4) = pk;
      }
    }
    // ---- phase X: X = V - diag(ge) K S   (wave: 16 rows, 32 columns)
    u32x4 sfrag[2][D / 32];  // S (16-bit) B fragments, reused by phase O
#pragma unroll
    for (int vt = 0; vt < 2; ++vt)
#pragma unroll
      for (int s = 0; s < D / 32; ++s) sfrag[vt][s] = lds16(Sb + (16 * vt + c16) * KP + 8 * g + 32 * s);
    u32x4 kfrag[D / 32];
#pragma unroll
    for (int s = 0; s < D / 32; ++s) kfrag[s] = lds16(Kn + (16 * wave + c16) * KP + 8 * g + 32 * s);
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < D / 32; ++s) acc = mfma16x16x32<T>(kfrag[s], sfrag[vt][s], acc);
      float xv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[i] = vcur[vt][i] - s_ge[16 * wave + 4 * g + i] * acc[i];
      u32x2 pk = {pack2<T>(xv[0], xv[1]), pack2<T>(xv[2], xv[3])};
      *(u32x2*)(XT + (16 * vt + c16) * CP + 16 * wave + 4 * g) = pk;
    }
    __syncthreads();

    // ---- phase U: U = (T diag(beta)) X
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const T* arow = Tb + (16 * wave + c16) * CP + 8 * g;
      const T* brow = XT + (16 * vt + c16) * CP + 8 * g;
#pragma unroll
      for (int s = 0; s < 2; ++s) acc = mfma16x16x32<T>(lds16(arow + 32 * s), lds16(brow + 32 * s), acc);
      u32x2 pk = {pack2<T>(acc[0], acc[1]), pack2<T>(acc[2], acc[3])};
      *(u32x2*)(UT + (16 * vt + c16) * CP + 16 * wave + 4 * g) = pk;
    }
    __syncthreads();

    // ---- phase O: O = diag(ge) Q S + Rq U
    u32x4 ufrag[2][2];  // U^T B fragments, reused by phase S
#pragma unroll
    for (int vt = 0; vt < 2; ++vt)
#pragma unroll
      for (int s = 0; s < 2; ++s) ufrag[vt][s] = lds16(UT + (16 * vt + c16) * CP + 8 * g + 32 * s);
    u32x4 qfrag[D / 32], rfrag[2];
#pragma unroll
    for (int s = 0; s < D / 32; ++s) qfrag[s] = lds16(Qn + (16 * wave + c16) * KP + 8 * g + 32 * s);
#pragma unroll
    for (int s = 0; s < 2; ++s) rfrag[s] = lds16(Rq + (16 * wave + c16) * CP + 8 * g + 32 * s);
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < D / 32; ++s) acc = mfma16x16x32<T>(qfrag[s], sfrag[vt][s], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] *= s_ge[16 * wave + 4 * g + i];
#pragma unroll
      for (int s = 0; s < 2; ++s) acc = mfma16x16x32<T>(rfrag[s], ufrag[vt][s], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = c * C + 16 * wave + 4 * g + i;
        if (t < a.T)
          ((T*)a.o)[(((int64_t)b * a.T + t) * a.H + h) * D + v0 + 16 * vt + c16] = (T)acc[i];
      }
    }
    // ---- phase S: S = gC S + Kd^T U
#pragma unroll
    for (int j = 0; j < KTW; ++j) {
      const int kt = wave * KTW + j;
      u32x4 kdfrag[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) kdfrag[s] = lds16(KdT + (16 * kt + c16) * CP + 8 * g + 32 * s);
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        f32x4 acc = S[j][vt] * gC;
#pragma unroll
        for (int s = 0; s < 2; ++s) acc = mfma16x16x32<T>(kdfrag[s], ufrag[vt][s], acc);
        S[j][vt] = acc;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KTW; ++j)
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        const int kt = wave * KTW + j;
        u32x2 pk = {pack2<T>(S[j][vt][0], S[j][vt][1]), pack2<T>(S[j][vt][2], S[j][vt][3])};
        *(u32x2*)(Sb + (16 * vt + c16) * KP + 16 * kt + 4 * g) = pk;
      }
  }

  if (a.s_out) {
#pragma unroll
    for (int j = 0; j < KTW; ++j)
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        const int kt = wave * KTW + j;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kx = 16 * kt + 4 * g + i, vx = v0 + 16 * vt + c16;
          a.s_out[((int64_t)bh * D + kx) * D + vx] = S[j][vt][i];
        }
      }
  }
}

template <typename T, int D>
static int launch16(const GdnArgs& a, hipStream_t s) {
  gdn_prep16_kernel<T, D><<<dim3((unsigned)a.NC, (unsigned)(a.B * a.H)), dim3(256), 0, s>>>(a);
  int rc = check_launch("chunk_gated_delta_rule(prep16)");
  if (rc) return rc;
  gdn_scan16_kernel<T, D><<<dim3((unsigned)(a.B * a.H), D / 32), dim3(256), 0, s>>>(a);
  return check_launch("chunk_gated_delta_rule(scan16)");
}

int launch_gdn16(const GdnArgs& a, int dtype, int D, hipStream_t s) {
  if (dtype == ATMA_BF16) return D == 128 ? launch16<bf16, 128>(a, s) : launch16<bf16, 64>(a, s);
  return D == 128 ? launch16<f16, 128>(a, s) : launch16<f16, 64>(a, s);
}

}  // namespace atma
