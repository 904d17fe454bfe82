// Backward of the gated-delta recurrence (training).
//
// Reference: the memory branch trains through FLA's chunk_gated_delta_rule autograd
// (model/blocks.py:44-84, called from TitansMemory.forward, model/blocks.py:470-479);
// the recurrence it differentiates is the sequential definition of
// scripts/titans_proto.py:53-76 (decay first, predict on the decayed state, undecayed
// write, self-inclusive readout), with the state in the [K, V] layout:
//   St = g_t S_{t-1};  pred = St^T k_t;  u = b_t (v_t - pred);  S_t = St + k_t u^T;
//   o_t = S_t^T q_t                                  (q already scaled, q / k normalised)
// Reverse-mode, with G = dL/dS_t (carried from the future, plus q_t dO_t^T):
//   dq_t = S_t dO_t;  du = G^T k_t;  dv_t = b_t du;  db_t = du . (v_t - pred);
//   dpred = -b_t du;  dSt = G + k_t dpred^T;  dk_t = G u + St dpred;
//   dg_t = <dSt, S_{t-1}>;  G <- g_t dSt;  and finally dS_0 = G.
//
// MI355X design: the recurrence never mixes V columns, so one workgroup owns 16 columns
// of one (sequence, head) state (dk x 16 fp32, RPT = dk / 16 rows per lane; lane =
// column * 16 + row group, so a column's row reduction is a 16-lane shuffle).  Pass 1
// walks forward and checkpoints the state every 64 tokens in the workspace.  Pass 2
// walks the chunks backwards.  Each chunk's operands (k rows, the block's 16 columns
// of v and dO, gamma, beta) are staged in LDS once, since the recomputation
// reads them several times; each 8-token sub-block is recomputed from its chunk's
// checkpoint into registers (the states before and after each token, u and v - pred),
// then the 8 reverse steps run on registers.  Row sums are DPP row reductions; sums
// over columns (dq, dk, db, dg) go through LDS once per sub-block, and each workgroup
// writes its column block's partial sums; the caller adds the dv / 16 partials.
#include "common.h"

namespace atma {

constexpr int kBwdChunk = 64;  // checkpoint interval
constexpr int kBwdSub = 8;     // tokens per register-resident sub-block

struct GdnBwdArgs {
  const float* q;     // (B, T, H, DK) scaled, normalised
  const float* k;     // (B, T, H, DK) normalised
  const float* v;     // (B, T, H, DV)
  const float* g;     // (B, T, H) log decay
  const float* beta;  // (B, T, H)
  const float* s0;    // (B, H, DK, DV) or null
  const float* dO;    // (B, T, H, DV)
  const float* dST;   // (B, H, DK, DV) or null
  float* dq_part;     // (JB, B, T, H, DK)
  float* dk_part;     // (JB, B, T, H, DK)
  float* dv;          // (B, T, H, DV)
  float* dg_part;     // (JB, B, T, H)
  float* db_part;     // (JB, B, T, H)
  float* ds0;         // (B, H, DK, DV)
  float* ckpt;        // (B * H * JB, NC, 256, RPT)
  int B, T, H, DV;
};

template <int RPT>
__global__ void __launch_bounds__(256) gdn_bwd_kernel(GdnBwdArgs a) {
  constexpr int DK = 16 * RPT;
  constexpr int NRED = 2 * DK + 2;  // dq[DK], dk[DK], db, dg per wave
  __shared__ float red[kBwdSub][4][NRED];
  // the current chunk's operands: k rows, this block's 16 columns of v and dO, gamma, beta
  // (q is read once per token, from memory), 73.5 KiB in all with red: two workgroups per CU
  __shared__ __attribute__((aligned(16))) float sk[kBwdChunk][DK];
  __shared__ float sv[kBwdChunk][16];
  __shared__ float sdo[kBwdChunk][16];
  __shared__ float sgam[kBwdChunk];
  __shared__ float sbet[kBwdChunk];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = tid >> 4, rg = tid & 15;
  const int JB = a.DV / 16;
  const int wg = blockIdx.x;
  const int jb = wg % JB, bh = wg / JB;
  const int b = bh / a.H, h = bh % a.H;
  const int j = jb * 16 + col;
  const int T = a.T, H = a.H, DV = a.DV;
  const int NC = (T + kBwdChunk - 1) / kBwdChunk;
  const int64_t tok0 = (int64_t)b * T;  // token row base of this sequence

  // rows rg * RPT .. of a DK-float row
  auto rows = [&](const float* p0, float* out) {
    const float* p = p0 + rg * RPT;
#pragma unroll
    for (int i = 0; i < RPT; i += 4) {
      const f32x4 x = *(const f32x4*)(p + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[i + e] = x[e];
    }
  };
  // stage chunk c (tokens cb .. ce) into LDS; with_grad adds dO
  auto stage = [&](int cb, int ce, bool with_grad) {
    __syncthreads();  // the previous chunk's readers are done
    const int n = ce - cb;
    for (int idx = tid; idx < n * (DK / 4); idx += 256) {
      const int tl = idx / (DK / 4), e4 = idx % (DK / 4);
      const int64_t off = ((tok0 + cb + tl) * H + h) * DK + 4 * e4;
      *(f32x4*)&sk[tl][4 * e4] = *(const f32x4*)(a.k + off);
    }
    for (int idx = tid; idx < n * 16; idx += 256) {
      const int tl = idx / 16, cc = idx % 16;
      const int64_t th = (tok0 + cb + tl) * H + h;
      sv[tl][cc] = a.v[th * DV + jb * 16 + cc];
      if (with_grad) sdo[tl][cc] = a.dO[th * DV + jb * 16 + cc];
    }
    for (int tl = tid; tl < n; tl += 256) {
      const int64_t th = (tok0 + cb + tl) * H + h;
      sgam[tl] = __expf(a.g[th]);
      sbet[tl] = a.beta[th];
    }
    __syncthreads();
  };
  // sum over the 16 row groups of a column = one 16-lane DPP row: swap neighbours and
  // pairs within quads, then rotate the row by 4 and by 8 (every lane ends with the sum)
  auto dpp = [](float x, int ctrl) -> float {
    switch (ctrl) {  // the control must be a constant
      case 0xB1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
      case 0x4E: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
      case 0x124: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xF, 0xF, false));
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, false));
    }
  };
  auto row_sum = [&](float x) {
    x += dpp(x, 0xB1);   // quad_perm [1,0,3,2]
    x += dpp(x, 0x4E);   // quad_perm [2,3,0,1]
    x += dpp(x, 0x124);  // row_ror:4
    x += dpp(x, 0x128);  // row_ror:8
    return x;
  };
  // one forward step: S (state before t) -> S (state after t); returns v - pred and u
  auto step = [&](int tl, float* S, float& vm, float& u) {  // tl: index in the staged chunk
    float kr[RPT];
    rows(sk[tl], kr);
    const float gam = sgam[tl];
    const float bet = sbet[tl];
    const float vj = sv[tl][col];
    float pred = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] *= gam;
      pred = fmaf(S[i], kr[i], pred);
    }
    pred = row_sum(pred);
    vm = vj - pred;
    u = bet * vm;
#pragma unroll
    for (int i = 0; i < RPT; ++i) S[i] = fmaf(kr[i], u, S[i]);
  };

  float* ck = a.ckpt + ((int64_t)wg * NC) * 256 * RPT + tid * RPT;
  const int64_t sidx = (((int64_t)b * H + h) * DK + rg * RPT) * DV + j;  // S[row0][j]

  // ---- pass 1: forward, checkpoint at every chunk start
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = a.s0 ? a.s0[sidx + (int64_t)i * DV] : 0.f;
  for (int c = 0; c < NC; ++c) {
    float* cp = ck + (int64_t)c * 256 * RPT;
#pragma unroll
    for (int i = 0; i < RPT; i += 4) *(f32x4*)(cp + i) = f32x4{S[i], S[i + 1], S[i + 2], S[i + 3]};
    const int te = min((c + 1) * kBwdChunk, T);
    stage(c * kBwdChunk, te, false);
    for (int tl = 0; tl < te - c * kBwdChunk; ++tl) {
      float vm, u;
      step(tl, S, vm, u);
    }
  }

  // ---- pass 2: reverse
  float G[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) G[i] = a.dST ? a.dST[sidx + (int64_t)i * DV] : 0.f;
  for (int c = NC - 1; c >= 0; --c) {
    const int cb = c * kBwdChunk, ce = min(cb + kBwdChunk, T);
    const int nsub = (ce - cb + kBwdSub - 1) / kBwdSub;
    stage(cb, ce, true);
    for (int sb = nsub - 1; sb >= 0; --sb) {
      const int t0 = cb + sb * kBwdSub;
      const int n = min(kBwdSub, ce - t0);  // tokens in this sub-block (uniform)
      // recompute: checkpoint -> state before t0 -> the sub-block's states
      float Sb[kBwdSub + 1][RPT];  // Sb[i] = state before token t0 + i; Sb[n] = after the last
      {
        const float* cp = ck + (int64_t)c * 256 * RPT;
#pragma unroll
        for (int i = 0; i < RPT; i += 4) {
          const f32x4 x = *(const f32x4*)(cp + i);
#pragma unroll
          for (int e = 0; e < 4; ++e) Sb[0][i + e] = x[e];
        }
        for (int tl = 0; tl < t0 - cb; ++tl) {
          float vm, u;
          step(tl, Sb[0], vm, u);
        }
      }
      float VM[kBwdSub], U[kBwdSub];
#pragma unroll
      for (int s = 0; s < kBwdSub; ++s) {
        if (s < n) {
#pragma unroll
          for (int i = 0; i < RPT; ++i) Sb[s + 1][i] = Sb[s][i];
          step(t0 - cb + s, Sb[s + 1], VM[s], U[s]);
        }
      }
      // reverse steps on registers; column sums of each token to LDS slot s
#pragma unroll
      for (int s = kBwdSub - 1; s >= 0; --s) {
        if (s < n) {
          const int tl = t0 - cb + s;
          const int64_t th = (tok0 + t0 + s) * H + h;
          float qr[RPT], kr[RPT];
          rows(a.q + th * DK, qr);
          rows(sk[tl], kr);
          const float gam = sgam[tl];
          const float bet = sbet[tl];
          const float dOj = sdo[tl][col];
          float dq[RPT], dk[RPT];
          float du = 0.f;
#pragma unroll
          for (int i = 0; i < RPT; ++i) {
            G[i] = fmaf(qr[i], dOj, G[i]);
            dq[i] = Sb[s + 1][i] * dOj;
            du = fmaf(G[i], kr[i], du);
          }
          du = row_sum(du);
          const float dpred = -bet * du;
          float dgl = 0.f;
#pragma unroll
          for (int i = 0; i < RPT; ++i) {
            const float st = gam * Sb[s][i];
            dk[i] = fmaf(G[i], U[s], st * dpred);
            const float dst = fmaf(kr[i], dpred, G[i]);
            dgl = fmaf(dst, Sb[s][i], dgl);
            G[i] = gam * dst;
          }
          if (rg == 0) a.dv[th * DV + j] = bet * du;
          float dbl = rg == 0 ? du * VM[s] : 0.f;  // one copy per column
          // sums over the wave's 4 columns (lanes 16 apart); dg also over the row groups
#pragma unroll
          for (int i = 0; i < RPT; ++i) {
            dq[i] += __shfl_xor(dq[i], 16, 64);
            dq[i] += __shfl_xor(dq[i], 32, 64);
            dk[i] += __shfl_xor(dk[i], 16, 64);
            dk[i] += __shfl_xor(dk[i], 32, 64);
          }
          dgl = wave_sum(dgl);
          dbl = wave_sum(dbl);
          float* r = red[s][wave];
          if (lane < 16) {
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
              r[rg * RPT + i] = dq[i];
              r[DK + rg * RPT + i] = dk[i];
            }
          }
          if (lane == 0) {
            r[2 * DK] = dbl;
            r[2 * DK + 1] = dgl;
          }
        }
      }
      __syncthreads();
      // add the 4 waves and write this column block's partial sums
      for (int idx = tid; idx < n * NRED; idx += 256) {
        const int s = idx / NRED, e = idx % NRED;
        const float* r0 = red[s][0];
        const float sum = r0[e] + r0[NRED + e] + r0[2 * NRED + e] + r0[3 * NRED + e];
        const int64_t th = (tok0 + t0 + s) * H + h;
        const int64_t plane = (int64_t)a.B * T * H;
        if (e < DK)
          a.dq_part[(jb * plane + th) * DK + e] = sum;
        else if (e < 2 * DK)
          a.dk_part[(jb * plane + th) * DK + e - DK] = sum;
        else if (e == 2 * DK)
          a.db_part[jb * plane + th] = sum;
        else
          a.dg_part[jb * plane + th] = sum * sgam[t0 - cb + s];  // d/d(log decay) = dgamma * gamma
      }
      __syncthreads();  // red is reused by the next sub-block
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) a.ds0[sidx + (int64_t)i * DV] = G[i];
}

}  // namespace atma

extern "C" size_t atma_gated_delta_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t dk, int64_t dv) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0) return 0;
  const int64_t nc = (T + atma::kBwdChunk - 1) / atma::kBwdChunk;
  return (size_t)(B * H * (dv / 16)) * nc * 16 * dk * sizeof(float);
}

extern "C" int atma_gated_delta_bwd(const float* q, const float* k, const float* v, const float* g,
                                    const float* beta, const float* initial_state, const float* d_out,
                                    const float* d_final_state, float* dq_part, float* dk_part, float* dv,
                                    float* dg_part, float* dbeta_part, float* d_initial_state, int64_t B,
                                    int64_t T, int64_t H, int64_t dk, int64_t dv_dim, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  using namespace atma;
  if (B < 0 || T < 0 || H <= 0) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd: bad sizes");
  if (dk != 64 && dk != 128)
    return set_error(ATMA_ERR_UNSUPPORTED, "gated_delta_bwd: dk %lld (supported: 64, 128)", (long long)dk);
  if (dv_dim <= 0 || dv_dim % 16)
    return set_error(ATMA_ERR_UNSUPPORTED, "gated_delta_bwd: dv %lld must be a multiple of 16",
                     (long long)dv_dim);
  if (B == 0) return ATMA_OK;
  if (B * H * (dv_dim / 16) > 0x7fffffffll || B * T * H * dv_dim > (1ll << 40) || T > 0x3fffffffll)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd: sizes too large");
  if (!d_initial_state) return set_error(ATMA_ERR_INVALID, "gated_delta_bwd: null pointer");
  if (T > 0 && (!q || !k || !v || !g || !beta || !d_out || !dq_part || !dk_part || !dv || !dg_part ||
                !dbeta_part))
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd: null pointer");
  const size_t need = atma_gated_delta_bwd_workspace_bytes(B, T, H, dk, dv_dim);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(ATMA_ERR_WORKSPACE, "gated_delta_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  if (((uintptr_t)q | (uintptr_t)k) % 16)
    return set_error(ATMA_ERR_INVALID, "gated_delta_bwd: q / k must be 16-byte aligned");
  GdnBwdArgs a{};
  a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta; a.s0 = initial_state; a.dO = d_out;
  a.dST = d_final_state; a.dq_part = dq_part; a.dk_part = dk_part; a.dv = dv; a.dg_part = dg_part;
  a.db_part = dbeta_part; a.ds0 = d_initial_state; a.ckpt = (float*)workspace;
  a.B = (int)B; a.T = (int)T; a.H = (int)H; a.DV = (int)dv_dim;
  const dim3 grid((unsigned)(B * H * (dv_dim / 16)));
  hipStream_t s = (hipStream_t)stream;
  if (dk == 128)
    gdn_bwd_kernel<8><<<grid, 256, 0, s>>>(a);
  else
    gdn_bwd_kernel<4><<<grid, 256, 0, s>>>(a);
  return check_launch("gated_delta_bwd");
}
