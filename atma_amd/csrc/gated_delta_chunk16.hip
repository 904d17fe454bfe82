// Chunked gated-delta prefill for bf16 / fp16 inputs on MFMA (v_mfma_f32_16x16x32).
//
// Algebra of gated_delta_chunked (model/blocks.py:375-423; FLA convention: decay
// first, undecayed write, self-inclusive readout).  Inside a 64-token chunk with
// inclusive log-decays lg_p, ge_p = exp(lg_p), A[p,s] = beta_p exp(lg_p - lg_s)
// kn_p.kn_s (s < p) and T = (I + A)^-1, the carried state S ([K, V]) gives
//     U = T diag(beta) V - T diag(beta ge) Kn S  =  u - w S
//     O = diag(ge) Qn S + Rq U,          Rq[p,s] = exp(lg_p - lg_s) qn_p.kn_s (s <= p)
//     S <- exp(lg_C) S + (diag(exp(lg_C - lg)) Kn)^T U
// Everything that does not depend on S is computed chunk-parallel, so the
// sequential pass only runs two dependent products per chunk (plus two independent
// ones for the output):
//
//  pass 1, gdn_prep16 -- one workgroup per (sequence, head, chunk): L2-normalise the
//    rows, Gram blocks Kn Kn^T and Qn Kn^T on MFMA, T by a blocked fp32 inverse
//    (forward substitution on the 16x16 diagonal blocks, then three levels of block
//    products), then w = T (beta ge Kn) and u = T (beta V) on MFMA.  Writes the
//    per-chunk record (w, qn, kdT, u, rq in 16 bits; lg in fp32).
//
//  pass 2, gdn_scan16 -- one workgroup per (sequence, head, 32-column slab of the
//    [K, V] state), chunks in order.  The 128 x 32 fp32 slab stays in VGPRs; a 16-bit
//    copy in LDS feeds the B operands.  Per chunk: U = u - w S and O = diag(ge) Qn S,
//    U^T to LDS, then S <- gC S + kdT U and O += Rq U: two dependent products and two
//    workgroup barriers on the recurrence, the output products beside them.  The
//    recurrence operands of the next three chunks are in flight into registers (A
//    fragments straight from memory); qn, rq and lg of the next two chunks are copied
//    straight into LDS.  The output slab leaves through LDS as 16-byte stores.
#include <algorithm>
#include <type_traits>

#include "gated_delta.h"

namespace atma {

__device__ __forceinline__ u32x4 lds16(const void* p) { return *(const u32x4*)p; }

template <typename T>
__device__ __forceinline__ u32x4 scale8(const u32x4& x, float f) {
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w) o[w] = pack2<T>(elem16<T>(x, 2 * w) * f, elem16<T>(x, 2 * w + 1) * f);
  return o;
}

// (tp, ts) of the 6 strictly-upper 16x16 blocks of a 64x64 matrix, blk = 0..5
__device__ __forceinline__ void upper_block(int blk, int& tp, int& ts) {
  tp = blk < 3 ? 0 : (blk < 5 ? 1 : 2);
  ts = blk < 3 ? blk + 1 : (blk < 5 ? blk - 1 : 3);
}

template <typename T, int D>
__global__ void __launch_bounds__(256, 2) gdn_prep16_kernel(GdnArgs a) {
  constexpr int C = kChunk, KP = D + 8, FP = C + 4;
  constexpr int DC = D / 8;           // 16-byte chunks per row
  constexpr int NE = (C / 4) * DC;    // (4 tokens x 8 dims) groups
  __shared__ __attribute__((aligned(16))) T R1[C * KP];  // Kn rows, then beta ge Kn rows
  __shared__ __attribute__((aligned(16))) T R2[C * KP];  // Qn rows, then beta V rows
  __shared__ __attribute__((aligned(16))) float Af[C * FP];
  __shared__ float Tf[C * FP];
  __shared__ float Yf[3 * 256];
  __shared__ __attribute__((aligned(16))) float lg[C], bet[C], sge[C], ikn[C], iqs[C];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int c16 = lane & 15, g = lane >> 4;
  const Gdn16Ws W{D, (int64_t)a.B * a.H * a.NC};
  T* ws16 = (T*)a.ws;
  const bool act = tid < NE;
  const int p4 = tid / DC, dc = tid % DC;

  // ---- the rows of one (sequence, head, chunk) item: thread (p4, dc) holds tokens
  // 4p4..4p4+3, dims 8dc..8dc+7 of k, q, v; threads < C one token's g and beta
  struct Rows {
    u32x4 k[4], q[4], v[4];
    float gl, bt;
  };
  auto load_rows = [&](Rows& r, int item) {
    const int bh = item / a.NC, c = item % a.NC;
    const int b = bh / a.H, h = bh % a.H;
    if (act) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t t = (int64_t)c * C + 4 * p4 + i;
        const bool ok = t < a.T;
        r.k[i] = ok ? *(const u32x4*)((const T*)a.k + b * a.k_sb + t * a.k_st + (h / a.G) * a.k_sh + 8 * dc)
                    : u32x4{0, 0, 0, 0};
        r.q[i] = ok ? *(const u32x4*)((const T*)a.q + b * a.q_sb + t * a.q_st + h * a.q_sh + 8 * dc)
                    : u32x4{0, 0, 0, 0};
        r.v[i] = ok ? *(const u32x4*)((const T*)a.v + b * a.v_sb + t * a.v_st + (h / a.G) * a.v_sh + 8 * dc)
                    : u32x4{0, 0, 0, 0};
      }
    }
    if (tid < C) {
      const int tt = c * C + tid;
      const int64_t gi = ((int64_t)b * a.T + tt) * a.H + h;
      r.gl = tt < a.T ? gdn_load_g(a, gi) : 0.f;
      r.bt = tt < a.T ? gdn_load_beta(a, gi) : 0.f;
    }
  };

  auto process = [&](Rows& r, int item, int next) {
  const int bh = item / a.NC, c = item % a.NC;
  const int64_t ri = (int64_t)bh * a.NC + c;
  lds_barrier();  // the previous item is done with every LDS buffer
  u32x4* kn = r.k;
  u32x4* vr = r.v;
  if (act) {
    float ks[4], qs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ks[i] = qs[i] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = elem16<T>(kn[i], e), y = elem16<T>(r.q[i], e);
        ks[i] = fmaf(x, x, ks[i]);
        qs[i] = fmaf(y, y, qs[i]);
      }
    }
#pragma unroll
    for (int m = 1; m < DC; m <<= 1)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ks[i] += __shfl_xor(ks[i], m, 64);
        qs[i] += __shfl_xor(qs[i], m, 64);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ik = a.l2norm ? 1.f / fmaxf(sqrtf(ks[i]), 1e-12f) : 1.f;
      const float iq = (a.l2norm ? 1.f / fmaxf(sqrtf(qs[i]), 1e-12f) : 1.f) * a.scale;
      const int p = 4 * p4 + i;
      kn[i] = scale8<T>(kn[i], ik);
      *(u32x4*)(R1 + p * KP + 8 * dc) = kn[i];
      *(u32x4*)(R2 + p * KP + 8 * dc) = scale8<T>(r.q[i], iq);
      if (dc == 0) {
        ikn[p] = ik;
        iqs[p] = iq;
      }
    }
  }
  if (tid < C) {
    lg[tid] = r.gl;
    bet[tid] = r.bt;
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
    sge[lane] = expf(x);
    const float last = __shfl(x, 63, 64);
    const float tail = expf(last - x);
    float* rec = (float*)((char*)a.ws + W.f32_byte(ri));
    rec[lane] = x;
    rec[C + lane] = tail * ikn[lane];
    rec[2 * C + lane] = iqs[lane];
  }
  __syncthreads();

  // ---- Gram tiles, transposed: for the 10 lower-triangle block pairs (tp >= ts) the
  // tile rows are keys s (16 ts + 4g + i) and the columns tokens p (16 tp + c16), so a
  // lane holds 4 consecutive s of one row p: one 16-byte LDS write of A[p][s..s+3] and
  // one 8-byte store of rq[p][s..s+3].
  {
    // this wave's 5 tasks (wave, wave + 4, ..., wave + 16) as independent MFMA chains
    constexpr int NT = 5;
    int tp_[NT], ts_[NT];
    const T* ar[NT];
    const T* br[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int task = wave + 4 * k, which = task / 10, idx = task % 10;
      tp_[k] = (idx >= 1) + (idx >= 3) + (idx >= 6);
      ts_[k] = idx - tp_[k] * (tp_[k] + 1) / 2;
      ar[k] = R1 + (16 * ts_[k] + c16) * KP + 8 * g;
      br[k] = (which ? R2 : R1) + (16 * tp_[k] + c16) * KP + 8 * g;
    }
    f32x4 acc[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
#pragma unroll
      for (int k = 0; k < NT; ++k) acc[k] = mfma16x16x32<T>(lds16(ar[k] + 32 * s), lds16(br[k] + 32 * s), acc[k]);
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int which = (wave + 4 * k) / 10;
      const int p = 16 * tp_[k] + c16, s0 = 16 * ts_[k] + 4 * g;
      // decays and masks without branches (an overflowing exp above the diagonal is
      // discarded by the select)
      const float lgp = lg[p], bp = which == 0 ? bet[p] : 1.f;
      const f32x4 lgs = *(const f32x4*)(lg + s0);
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sx = s0 + i;
        const float dec = __builtin_amdgcn_exp2f((lgp - lgs[i]) * kLog2e);
        const bool keep = which == 0 ? sx < p : sx <= p;
        v[i] = keep ? bp * dec * acc[k][i] : 0.f;
      }
      if (which == 0) {
        *(f32x4*)(Af + p * FP + s0) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
        *(u32x2*)(ws16 + W.rq(ri) + p * C + s0) = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
      }
    }
  }
  for (int e = tid; e < 6 * 64; e += 256) {  // rq is zero above the block diagonal
    int tp, ts;
    upper_block(e >> 6, tp, ts);
    const int r = (e >> 2) & 15, c4 = e & 3;
    *(u32x2*)(ws16 + W.rq(ri) + (16 * tp + r) * C + 16 * ts + 4 * c4) = u32x2{0u, 0u};
  }
  __syncthreads();  // Gram done: R1 / R2 are free, A is complete

  // ---- scaled operands of the w / u products, row-major like Kn (conflict-free writes;
  // the products read them transposed)
  if (act) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 4 * p4 + i;
      const float fv = bet[p], fk = fv * sge[p];
      *(u32x4*)(R1 + p * KP + 8 * dc) = scale8<T>(kn[i], fk);
      *(u32x4*)(R2 + p * KP + 8 * dc) = scale8<T>(vr[i], fv);
    }
  }
  // the row registers are free from here: the next item's rows load during the inverse
  if (next < a.B * a.H * a.NC) load_rows(r, next);
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
  for (int e = tid; e < 6 * 256; e += 256) {  // T is zero above the block diagonal
    int tp, ts;
    upper_block(e >> 8, tp, ts);
    Tf[(16 * tp + ((e >> 4) & 15)) * FP + 16 * ts + (e & 15)] = 0.f;
  }
  __syncthreads();
  // ---- off-diagonal blocks: T_ij = -T_ii * sum_{k=j}^{i-1} A_ik T_kj, level L = i - j,
  // one wave per block, 16x16 products on v_mfma_f32_16x16x4f32 (full fp32)
  for (int L = 1; L < 4; ++L) {
    if (wave < 4 - L) {
      const int i = L + wave, j = wave;
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
      for (int kk = j; kk < i; ++kk)
#pragma unroll
        for (int st = 0; st < 4; ++st)
          y = __builtin_amdgcn_mfma_f32_16x16x4f32(Af[(16 * i + c16) * FP + 16 * kk + 4 * st + g],
                                                   Tf[(16 * kk + 4 * st + g) * FP + 16 * j + c16], y, 0, 0, 0);
      float* yw = Yf + wave * 256;  // this wave's 16x16 scratch, [row][col]
#pragma unroll
      for (int r = 0; r < 4; ++r) yw[(4 * g + r) * 16 + c16] = y[r];
      wave_sync();
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st)
        t = __builtin_amdgcn_mfma_f32_16x16x4f32(Tf[(16 * i + c16) * FP + 16 * i + 4 * st + g],
                                                 yw[(4 * st + g) * 16 + c16], t, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) Tf[(16 * i + 4 * g + r) * FP + 16 * j + c16] = -t[r];
    }
    __syncthreads();
  }

  // ---- w = T (beta ge Kn), u = T (beta V): wave = 16-row block of T, all column tiles.
  // Both products take 8 consecutive tokens of one head-dim column per lane from the
  // row-major tiles: two transposing reads (ds_read_b64_tr_b16) of 4 tokens each.
  {
    const int rb = wave;
    const int nsteps = rb < 2 ? 1 : 2;  // T is lower triangular: later tokens are 0
    u32x4 tfrag[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float* tr = Tf + (16 * rb + c16) * FP + 32 * s + 8 * g;
#pragma unroll
      for (int w = 0; w < 4; ++w) tfrag[s][w] = pack2<T>(tr[2 * w], tr[2 * w + 1]);
    }
    // lane (g, c16) reads token row 32 s + 8 g + c16 / 4 (+4), columns 16 ct + 4 (c16 % 4)
    auto colfrag = [&](const T* R, int ct, int s) {
      const T* p = R + (32 * s + 8 * g + (c16 >> 2)) * KP + 16 * ct + 4 * (c16 & 3);
      const u32x2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * KP);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) {
      f32x4 aw = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < nsteps; ++s) {
        // w^T = (beta ge Kn)^T T^T: the T fragment is the B operand here (same registers)
        aw = mfma16x16x32<T>(colfrag(R1, ct, s), tfrag[s], aw);
        au = mfma16x16x32<T>(tfrag[s], colfrag(R2, ct, s), au);
      }
      // w row 16rb + c16, columns 16ct + 4g ..;  u in the scan's register order
      *(u32x2*)(ws16 + W.w(ri) + (16 * rb + c16) * D + 16 * ct + 4 * g) =
          u32x2{pack2<T>(aw[0], aw[1]), pack2<T>(aw[2], aw[3])};
      u32x2 pk = {pack2<T>(au[0], au[1]), pack2<T>(au[2], au[3])};
      *(u32x2*)(ws16 + W.us(ri) + (((ct >> 1) * 4 + rb) * 64 + lane) * 8 + (ct & 1) * 4) = pk;
    }
  }
  };

  // ---- persistent: workgroup w takes items w, w + G, w + 2G, ...; the rows of the next
  // item load while the current one finishes its inverse and w / u products
  const int total = a.B * a.H * a.NC, step = gridDim.x;
  Rows r;
  if ((int)blockIdx.x < total) load_rows(r, blockIdx.x);
  for (int item = blockIdx.x; item < total; item += step) process(r, item, item + step);
}

// Swizzle of 16-byte chunks in the LDS copies of the qn / rq records: logical chunk c of
// row r sits at chunk position c ^ f(r), so the 16 rows an A-fragment read touches (one
// chunk each) fall in distinct banks: f(r) = r mod 16 for 256-byte rows, (r / 2) mod 8
// for 128-byte rows (two rows share one 256-byte bank line).
template <int CPR>
__device__ __forceinline__ int rec_swizzle(int r) {
  static_assert(CPR == 8 || CPR == 16, "64- or 128-element rows");
  return CPR == 16 ? (r & 15) : ((r >> 1) & 7);
}

template <typename T, int D>
__global__ void __launch_bounds__(256, 1) gdn_scan16_kernel(GdnArgs a) {
  constexpr int C = kChunk, VS = 32, KP = D + 8, CP = C + 8, OP = VS + 8;
  constexpr int KS = D / 32;   // MFMA k-steps over the head dim
  constexpr int KTW = D / 64;  // 16-row state tiles per wave
  constexpr int QCPR = D / 8, RCPR = C / 8;  // 16-byte chunks per q / k and rq row
  constexpr int QB = C * D, RB = C * C;      // elements of one q / k block and rq record
  __shared__ __attribute__((aligned(16))) T Sb[VS * KP];   // S^T slab, 16-bit: [v][k]
  __shared__ __attribute__((aligned(16))) T Ub[VS * CP];   // U^T, 16-bit: [v][token]
  __shared__ __attribute__((aligned(16))) T Ubk[VS * CP];  // (diag(kf) U)^T
  __shared__ __attribute__((aligned(16))) T Qs[3 * QB];    // raw q rows of chunk j in slot j % 3
  __shared__ __attribute__((aligned(16))) T Kr[3 * QB];    // raw k rows of chunk j in slot j % 3
  __shared__ __attribute__((aligned(16))) T Rs[3 * RB];    // rq of chunk j in slot j % 3
  __shared__ __attribute__((aligned(16))) float Fs[3 * 3 * C];  // lg, kf, qs of chunk j
  gdn_signal_start(a);
  __shared__ __attribute__((aligned(16))) T Os[4 * 16 * OP];   // per-wave O tile, [row][v]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int bh = blockIdx.x, v0 = blockIdx.y * VS;
  const int b = bh / a.H, h = bh % a.H;
  const Gdn16Ws W{D, (int64_t)a.B * a.H * a.NC};
  const int64_t ri0 = (int64_t)bh * a.NC;
  const T* ws16 = (const T*)a.ws;

  // ---- state slab: tile (k-tile wave*KTW + j, v-tile vt); rows k = 16kt + 4g + i, cols v
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
    }
  // 16-bit copy of the state entering the next chunk, in LDS (B operands)
  auto publish_state = [&]() {
#pragma unroll
    for (int j = 0; j < KTW; ++j)
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        const int kt = wave * KTW + j;
        const u32x2 pk = {pack2<T>(S[j][vt][0], S[j][vt][1]), pack2<T>(S[j][vt][2], S[j][vt][3])};
        *(u32x2*)(Sb + (16 * vt + c16) * KP + 16 * kt + 4 * g) = pk;
      }
  };

  // ---- raw q and k rows, rq and the per-token factors of chunk j, copied straight into
  // LDS slot j % 3 (buffer DMA, no registers): wave w copies token rows 16w .. 16w + 15
  // of q, k and rq, wave 0 the 3 x 64 factors.  Rows past T read as zeros.  q rows use
  // the A-fragment swizzle, k rows the transposing-read swizzle (lds_swizzle).
  constexpr int QRPI = 64 / QCPR, RRPI = 64 / RCPR;  // rows per copy instruction
  constexpr int NQ = 16 / QRPI, NR = 16 / RRPI;
  constexpr int NDMA = 2 * NQ + NR;  // copy instructions of waves 1..3 per chunk
  constexpr int NLOAD = KS + 1;      // register loads per chunk (w, u)
  const uint32_t qst2 = (uint32_t)a.q_st * 2u, kst2 = (uint32_t)a.k_st * 2u;
  auto copy_rec = [&](int j, int slot) {
    const int64_t ri = ri0 + j;
    const int rows = min(a.T - j * C, C);
    const auto qrs = buffer_rsrc((const T*)a.q + b * a.q_sb + (int64_t)j * C * a.q_st + h * a.q_sh,
                                 (uint32_t)((rows - 1) * a.q_st + D) * 2u);
    const auto krs = buffer_rsrc((const T*)a.k + b * a.k_sb + (int64_t)j * C * a.k_st + (h / a.G) * a.k_sh,
                                 (uint32_t)((rows - 1) * a.k_st + D) * 2u);
    const auto rrs = buffer_rsrc(ws16 + W.rq(ri), RB * 2);
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int row = 16 * wave + QRPI * r + lane / QCPR, pc = lane % QCPR;
      const uint32_t lq = pc ^ rec_swizzle<QCPR>(row), lk = pc ^ lds_swizzle<QCPR>(row);
      dma_buf16(qrs, row * qst2 + 16u * lq, 0, Qs + slot * QB + (16 * wave + QRPI * r) * D);
      dma_buf16(krs, row * kst2 + 16u * lk, 0, Kr + slot * QB + (16 * wave + QRPI * r) * D);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int row = 16 * wave + RRPI * r + lane / RCPR, pc = lane % RCPR;
      const int lc = pc ^ rec_swizzle<RCPR>(row);
      dma_buf16(rrs, (uint32_t)(row * C + 8 * lc) * 2u, 0, Rs + slot * RB + (16 * wave + RRPI * r) * C);
    }
    if (wave == 0) {
      const auto frs = buffer_rsrc((const char*)a.ws + W.f32_byte(ri), 3 * C * 4);
#pragma unroll
      for (int r = 0; r < 3; ++r)
        dma_buf4(frs, (uint32_t)(r * C + lane) * 4u, 0, Fs + slot * 3 * C + r * C);
    }
  };

  // ---- one chunk's recurrence operands in registers (A fragments straight from
  // memory).  Three sets rotate with the three LDS slots: a set is refilled with chunk
  // c + 3 right after chunk c used it, so each load has two chunk steps to arrive, no
  // set is ever copied, and every slot index is a constant.
  struct Frag {
    u32x4 w[KS], u;
  };
  auto load = [&](Frag& f, int c) {
    const int64_t ri = ri0 + c;
    const int row = 16 * wave + c16;
#pragma unroll
    for (int s = 0; s < KS; ++s) f.w[s] = *(const u32x4*)(ws16 + W.w(ri) + row * D + 32 * s + 8 * g);
    f.u = *(const u32x4*)(ws16 + W.us(ri) + ((blockIdx.y * 4 + wave) * 64 + lane) * 8);
  };

  // this sequence's output rows as one buffer: rows past T are dropped
  const auto orsrc = buffer_rsrc((const T*)a.o + (int64_t)b * a.T * a.H * D,
                                 (uint32_t)((int64_t)a.T * a.H * D * 2));
  const int last = a.NC - 1;
  const int qrow = 16 * wave + c16;
  auto body = [&](const Frag& f, int c, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;  // c % 3, a constant per call site
    const T* qs = Qs + slot * QB + qrow * D;
    const T* rs = Rs + slot * RB + qrow * C;
    const T* kr = Kr + slot * QB;
    const float* fs = Fs + slot * 3 * C;
    // ---- U = u - w S and O = diag(ge qs) Q S (rows 16*wave + 4g + i, columns v0 + 16vt + c16);
    // all B fragments of S and A fragments of Q are requested before the first product
    u32x4 sbf[2][KS], qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qf[s] = lds16(qs + 8 * ((4 * s + g) ^ rec_swizzle<QCPR>(qrow)));
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) sbf[vt][s] = lds16(Sb + (16 * vt + c16) * KP + 32 * s + 8 * g);
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[2], o[2];
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) acc[vt] = o[vt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        acc[vt] = mfma16x16x32<T>(f.w[s], sbf[vt][s], acc[vt]);
        o[vt] = mfma16x16x32<T>(qf[s], sbf[vt][s], o[vt]);
      }
    const f32x4 lg4 = *(const f32x4*)(fs + 16 * wave + 4 * g);
    const f32x4 kf4 = *(const f32x4*)(fs + C + 16 * wave + 4 * g);
    const f32x4 qs4 = *(const f32x4*)(fs + 2 * C + 16 * wave + 4 * g);
#pragma unroll
    for (int vt = 0; vt < 2; ++vt) {
      float uv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) uv[i] = elem16<T>(f.u, 4 * vt + i) - acc[vt][i];
      const u32x2 pk = {pack2<T>(uv[0], uv[1]), pack2<T>(uv[2], uv[3])};
      const u32x2 pkk = {pack2<T>(uv[0] * kf4[0], uv[1] * kf4[1]), pack2<T>(uv[2] * kf4[2], uv[3] * kf4[3])};
      *(u32x2*)(Ub + (16 * vt + c16) * CP + 16 * wave + 4 * g) = pk;
      *(u32x2*)(Ubk + (16 * vt + c16) * CP + 16 * wave + 4 * g) = pkk;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sc = __builtin_amdgcn_exp2f(lg4[i] * kLog2e) * qs4[i];
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) o[vt][i] *= sc;
    }
    const float gC = __builtin_amdgcn_exp2f(fs[C - 1] * kLog2e);
    __syncthreads();
    // ---- S = gC S + K^T diag(kf) U  (A fragments: raw k columns by transposing reads);
    // O += Rq U
    u32x4 uf[2][2], ukf[2][2], rf[2], kt_[KTW][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      rf[s] = lds16(rs + 8 * ((4 * s + g) ^ rec_swizzle<RCPR>(qrow)));
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
        uf[vt][s] = lds16(Ub + (16 * vt + c16) * CP + 32 * s + 8 * g);
        ukf[vt][s] = lds16(Ubk + (16 * vt + c16) * CP + 32 * s + 8 * g);
      }
      // lane (g, c16) reads token rows 32 s + 8 g + c16 / 4 (+4), columns 16 kt + 4 (c16 % 4)
#pragma unroll
      for (int jj = 0; jj < KTW; ++jj) {
        const int kt = wave * KTW + jj, r0 = 32 * s + 8 * g + (c16 >> 2), col = 16 * kt + 4 * (c16 & 3);
        const int c8 = col >> 3, e = col & 7;
        const u32x2 lo = lds_read_tr16(kr + r0 * D + 8 * (c8 ^ lds_swizzle<QCPR>(r0)) + e);
        const u32x2 hi = lds_read_tr16(kr + (r0 + 4) * D + 8 * (c8 ^ lds_swizzle<QCPR>(r0 + 4)) + e);
        kt_[jj][s] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int vt = 0; vt < 2; ++vt)
#pragma unroll
      for (int jj = 0; jj < KTW; ++jj) S[jj][vt] *= gC;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int vt = 0; vt < 2; ++vt) {
#pragma unroll
        for (int jj = 0; jj < KTW; ++jj) S[jj][vt] = mfma16x16x32<T>(kt_[jj][s], ukf[vt][s], S[jj][vt]);
        o[vt] = mfma16x16x32<T>(rf[s], uf[vt][s], o[vt]);
      }
    publish_state();
    // ---- O tile (16 tokens x 32 columns) through LDS to one 16-byte store per lane
    {
      T* ow = Os + wave * 16 * OP;
#pragma unroll
      for (int vt = 0; vt < 2; ++vt)
#pragma unroll
        for (int i = 0; i < 4; ++i) ow[(4 * g + i) * OP + 16 * vt + c16] = (T)o[vt][i];
      wave_sync();
      const int r = lane >> 2, q = lane & 3;
      const uint32_t t = c * C + 16 * wave + r;
      buffer_store16(orsrc, ((t * a.H + h) * D + v0 + 8 * q) * 2u, lds16(ow + r * OP + 8 * q));
    }
    // copies of chunk c + 2 into the slot chunk c - 1 used (its readers are past the
    // barrier that began this step)
    copy_rec(min(c + 2, last), (slot + 2) % 3);
    // this wave's copies of chunk c + 1 (issued one step earlier) have landed: after them
    // came the register loads of step c - 1 and this step's copies (wave 0 issues more
    // copies, so the count is the smaller one).  The O store issued between them is not
    // counted: a store may complete before older loads, so only loads are counted.
    wait_vmcnt<NDMA + NLOAD>();
    __syncthreads();
  };

  // (Past the last chunk the loads and copies re-read it: every step issues the same
  // memory operations in the same order, so all waits on them stay partial.)
  publish_state();
  copy_rec(0, 0);
  copy_rec(min(1, last), 1);
  Frag f0, f1, f2;
  load(f0, 0);
  load(f1, min(1, last));
  load(f2, min(2, last));
  wait_vmcnt<0>();
  __syncthreads();
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  for (int c = 0; c < a.NC; c += 3) {
    body(f0, c, S0{});
    load(f0, min(c + 3, last));
    if (c + 1 < a.NC) body(f1, c + 1, S1{});
    load(f1, min(c + 4, last));
    if (c + 2 < a.NC) body(f2, c + 2, S2{});
    load(f2, min(c + 5, last));
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
  // persistent prep: two workgroups per CU (its LDS footprint), each walking items
  const int64_t items = (int64_t)a.NC * a.B * a.H;
  const int64_t grid = std::min<int64_t>(items, 2 * (int64_t)device_cu_count());
  gdn_prep16_kernel<T, D><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
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
