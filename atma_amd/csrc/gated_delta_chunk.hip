// Chunked gated-delta prefill with state carry (FLA chunk_gated_delta_rule contract).
//
// Reference arithmetic: gated_delta_chunked, model/blocks.py:375-423 (UT form,
// chunk C; decay first, undecayed write, self-inclusive readout), called through
// the FLA signature at model/blocks.py:44-49 and inference/models/atma.py:285-287.
//
// With lg_p = sum_{l<=p} g_l (g = log gamma) inside a chunk, ge_p = exp(lg_p),
// A[p,s] = beta_p exp(lg_p - lg_s) k_p.k_s (s < p) and T = (I + A)^-1 (unit lower
// triangular), the UT solve of the reference is folded into state-independent
// per-chunk operands (the WY form):
//     W  = T diag(beta ge) K          U0 = T diag(beta) V
//     Rq[p,s] = exp(lg_p - lg_s) q_p.k_s (s <= p)
//     Qt = diag(ge) Q - Rq W          R0 = Rq U0
//     Kd = diag(exp(lg_C - lg_s)) K   gC = exp(lg_C)
// after which one chunk of the recurrence on the [K, V] state S is
//     U = U0 - W S,   O = Qt S + R0,   S <- gC S + Kd^T U.
//
// Pass 1 (prep) is parallel over every (sequence, head, chunk); pass 2 runs the
// chunks in order, parallel over (sequence, head) x 16-column slabs of S (the
// state columns are independent), with the slab resident in LDS for the whole
// sequence.  All arithmetic is fp32.
#include "gated_delta.h"

namespace atma {

template <int D>
__host__ __device__ constexpr int64_t gdn_rec_floats() {
  return 5 * (int64_t)kChunk * D + 4;
}

template <typename T, int D>
__global__ void __launch_bounds__(256) gdn_prep_kernel(GdnArgs a) {
  constexpr int C = kChunk, P = D + 1;
  constexpr int CPT = D / 16;  // output columns per thread
  __shared__ float Ks[C * P], Qs[C * P], Vs[C * P];
  __shared__ float As[C * (C + 1)], Rs[C * (C + 1)];
  __shared__ float lg[C], bet[C], ge[C];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int t0 = c * C;

  // ---- rows: load, L2-normalise q/k, scale q; padded rows are zero with g = beta = 0
  for (int r = wave; r < C; r += 4) {
    const int t = t0 + r;
    const bool ok = t < a.T;
    const T* qr = (const T*)a.q + b * a.q_sb + (int64_t)t * a.q_st + h * a.q_sh;
    const T* kr = (const T*)a.k + b * a.k_sb + (int64_t)t * a.k_st + (h / a.G) * a.k_sh;
    const T* vr = (const T*)a.v + b * a.v_sb + (int64_t)t * a.v_st + (h / a.G) * a.v_sh;
    float qv[D / 64 > 0 ? D / 64 : 1], kv[D / 64 > 0 ? D / 64 : 1];
    float qq = 0.f, kk = 0.f;
#pragma unroll
    for (int e = 0; e < D / 64; ++e) {
      const int d = lane + 64 * e;
      qv[e] = ok ? to_f32(qr[d]) : 0.f;
      kv[e] = ok ? to_f32(kr[d]) : 0.f;
      Vs[r * P + d] = ok ? to_f32(vr[d]) : 0.f;
      qq += qv[e] * qv[e];
      kk += kv[e] * kv[e];
    }
    float iq = 1.f, ik = 1.f;
    if (a.l2norm) {
      iq = 1.f / fmaxf(sqrtf(wave_sum(qq)), 1e-12f);
      ik = 1.f / fmaxf(sqrtf(wave_sum(kk)), 1e-12f);
    }
#pragma unroll
    for (int e = 0; e < D / 64; ++e) {
      const int d = lane + 64 * e;
      Qs[r * P + d] = qv[e] * iq * a.scale;
      Ks[r * P + d] = kv[e] * ik;
    }
    if (lane == 0) {
      const int64_t gi = ((int64_t)b * a.T + t) * a.H + h;
      lg[r] = ok ? gdn_load_g(a, gi) : 0.f;
      bet[r] = ok ? gdn_load_beta(a, gi) : 0.f;
    }
  }
  __syncthreads();
  if (tid == 0) {
    float run = 0.f;
    for (int r = 0; r < C; ++r) {
      run += lg[r];
      lg[r] = run;
    }
  }
  __syncthreads();
  if (tid < C) ge[tid] = expf(lg[tid]);

  // ---- Gram blocks: A (strict lower, scaled by beta_p) and Rq (lower incl.)
  {
    const int tp = tid >> 4, ts = tid & 15;
    float kk[4][4] = {}, qk[4][4] = {};
    for (int d = 0; d < D; ++d) {
      float kp[4], qp[4], ks[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kp[i] = Ks[(4 * tp + i) * P + d];
        qp[i] = Qs[(4 * tp + i) * P + d];
        ks[i] = Ks[(4 * ts + i) * P + d];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kk[i][j] += kp[i] * ks[j];
          qk[i][j] += qp[i] * ks[j];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int p = 4 * tp + i, s = 4 * ts + j;
        const float dec = s <= p ? expf(lg[p] - lg[s]) : 0.f;
        As[p * (C + 1) + s] = s < p ? bet[p] * dec * kk[i][j] : 0.f;
        Rs[p * (C + 1) + s] = s <= p ? dec * qk[i][j] : 0.f;
      }
  }
  __syncthreads();

  // ---- T = (I + A)^-1 by forward substitution; lane s owns column s
  if (wave == 0) {
    const int s = lane;
    float col[C];
#pragma unroll
    for (int p = 0; p < C; ++p) {
      float accv = (p == s) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < p; ++j) accv -= As[p * (C + 1) + j] * col[j];
      col[p] = accv;
    }
#pragma unroll
    for (int p = 0; p < C; ++p) As[p * (C + 1) + s] = col[p];
  }
  __syncthreads();

  float* rec = (float*)a.ws + ((int64_t)bh * a.NC + c) * gdn_rec_floats<D>();
  float* Wg = rec;
  float* U0g = rec + C * D;
  float* Qtg = rec + 2 * C * D;
  float* R0g = rec + 3 * C * D;
  float* Kdg = rec + 4 * C * D;

  const int rg = tid >> 4, cg = tid & 15;
  float w[4][CPT], u[4][CPT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < CPT; ++e) w[i][e] = u[i][e] = 0.f;
  for (int s = 0; s < C; ++s) {
    float tv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) tv[i] = As[(4 * rg + i) * (C + 1) + s];
    const float bk = bet[s] * ge[s], bv = bet[s];
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const float kx = Ks[s * P + cg + 16 * e] * bk;
      const float vx = Vs[s * P + cg + 16 * e] * bv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i][e] += tv[i] * kx;
        u[i][e] += tv[i] * vx;
      }
    }
  }
  const float lgC = lg[C - 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 4 * rg + i;
    const float tail = expf(lgC - lg[p]);
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int d = cg + 16 * e;
      Wg[p * D + d] = w[i][e];
      U0g[p * D + d] = u[i][e];
      Kdg[p * D + d] = tail * Ks[p * P + d];
    }
  }
  if (tid == 0) rec[5 * C * D] = expf(lgC);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      Ks[(4 * rg + i) * P + cg + 16 * e] = w[i][e];
      Vs[(4 * rg + i) * P + cg + 16 * e] = u[i][e];
    }
  __syncthreads();
  float qt[4][CPT], r0[4][CPT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < CPT; ++e) qt[i][e] = r0[i][e] = 0.f;
  for (int s = 0; s < C; ++s) {
    float rv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rv[i] = Rs[(4 * rg + i) * (C + 1) + s];
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const float wx = Ks[s * P + cg + 16 * e];
      const float ux = Vs[s * P + cg + 16 * e];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qt[i][e] += rv[i] * wx;
        r0[i][e] += rv[i] * ux;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 4 * rg + i;
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int d = cg + 16 * e;
      Qtg[p * D + d] = ge[p] * Qs[p * P + d] - qt[i][e];
      R0g[p * D + d] = r0[i][e];
    }
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(256) gdn_scan_kernel(GdnArgs a) {
  constexpr int C = kChunk, VS = 16, P = D + 1;
  __shared__ float Wl[C * P], Ql[C * P], Kl[C * P];
  __shared__ float Ss[D * (VS + 1)], Ul[C * (VS + 1)];
  __shared__ float U0l[C * VS], R0l[C * VS];
  gdn_signal_start(a);

  const int tid = threadIdx.x;
  const int bh = blockIdx.x, v0 = blockIdx.y * VS;
  const int b = bh / a.H, h = bh % a.H;

  // initial state slab S[k][v0 .. v0+VS)
  for (int i = tid; i < D * VS; i += 256) {
    const int kx = i / VS, vx = i % VS;
    Ss[kx * (VS + 1) + vx] = a.s0 ? a.s0[((int64_t)bh * D + kx) * D + v0 + vx] : 0.f;
  }

  for (int c = 0; c < a.NC; ++c) {
    const float* rec = (const float*)a.ws + ((int64_t)bh * a.NC + c) * gdn_rec_floats<D>();
    __syncthreads();  // previous chunk finished with the LDS operands
    for (int i = tid; i < C * D / 4; i += 256) {
      const int p = (4 * i) / D, d = (4 * i) % D;
      const f32x4 wv = *(const f32x4*)(rec + 4 * i);
      const f32x4 qv = *(const f32x4*)(rec + 2 * C * D + 4 * i);
      const f32x4 kv = *(const f32x4*)(rec + 4 * C * D + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Wl[p * P + d + e] = wv[e];
        Ql[p * P + d + e] = qv[e];
        Kl[p * P + d + e] = kv[e];
      }
    }
    for (int i = tid; i < C * VS; i += 256) {
      const int p = i / VS, vx = i % VS;
      U0l[i] = rec[C * D + p * D + v0 + vx];
      R0l[i] = rec[3 * C * D + p * D + v0 + vx];
    }
    const float gC = rec[5 * C * D];
    __syncthreads();

    // U = U0 - W S ; O = Qt S + R0   (thread: row p, 4 columns)
    {
      const int p = tid >> 2, vq = (tid & 3) * 4;
      float uu[4], oo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uu[e] = U0l[p * VS + vq + e];
        oo[e] = R0l[p * VS + vq + e];
      }
      for (int kx = 0; kx < D; ++kx) {
        const float wv = Wl[p * P + kx], qv = Ql[p * P + kx];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sv = Ss[kx * (VS + 1) + vq + e];
          uu[e] -= wv * sv;
          oo[e] += qv * sv;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) Ul[p * (VS + 1) + vq + e] = uu[e];
      const int t = c * C + p;
      if (t < a.T) {
        T* op = (T*)a.o + (((int64_t)b * a.T + t) * a.H + h) * D + v0 + vq;
#pragma unroll
        for (int e = 0; e < 4; ++e) op[e] = from_f32<T>(oo[e]);
      }
    }
    __syncthreads();
    // S <- gC S + Kd^T U   (thread: D*VS/256 entries of one row)
    {
      constexpr int EPT = D * VS / 256;
      const int kx = (tid * EPT) / VS, vq = (tid * EPT) % VS;
      float sn[EPT];
#pragma unroll
      for (int e = 0; e < EPT; ++e) sn[e] = gC * Ss[kx * (VS + 1) + vq + e];
      for (int p = 0; p < C; ++p) {
        const float kd = Kl[p * P + kx];
#pragma unroll
        for (int e = 0; e < EPT; ++e) sn[e] += kd * Ul[p * (VS + 1) + vq + e];
      }
#pragma unroll
      for (int e = 0; e < EPT; ++e) Ss[kx * (VS + 1) + vq + e] = sn[e];
    }
  }
  __syncthreads();
  if (a.s_out) {
    for (int i = tid; i < D * VS; i += 256) {
      const int kx = i / VS, vx = i % VS;
      a.s_out[((int64_t)bh * D + kx) * D + v0 + vx] = Ss[kx * (VS + 1) + vx];
    }
  }
}

template <typename T, int D>
static int launch_gdn(GdnArgs a, hipStream_t s) {
  gdn_prep_kernel<T, D><<<dim3((unsigned)a.NC, (unsigned)(a.B * a.H)), dim3(256), 0, s>>>(a);
  int rc = check_launch("chunk_gated_delta_rule(prep)");
  if (rc) return rc;
  gdn_scan_kernel<T, D><<<dim3((unsigned)(a.B * a.H), D / 16), dim3(256), 0, s>>>(a);
  return check_launch("chunk_gated_delta_rule(scan)");
}

}  // namespace atma

extern "C" size_t atma_chunk_gated_delta_workspace_bytes(int64_t B, int64_t T, int64_t H,
                                                         int64_t dk, int64_t dv, int64_t chunk,
                                                         int dtype) {
  (void)dv;
  if (B <= 0 || T <= 0 || H <= 0 || chunk != atma::kChunk || (dk != 64 && dk != 128)) return 0;
  const int64_t nc = (T + chunk - 1) / chunk;
  if (dtype == ATMA_BF16 || dtype == ATMA_F16)
    return atma::gdn16_workspace_bytes(B * H, nc, (int)dk);
  const int64_t rec = 5 * chunk * dk + 4;
  return (size_t)(B * H * nc * rec) * sizeof(float);
}

extern "C" int atma_chunk_gated_delta_rule(
    const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_st, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
    const float* g, const float* beta, const float* initial_state, float* final_state, void* o,
    int64_t B, int64_t T, int64_t H, int64_t Hkv, int64_t dk, int64_t dv, int dtype, float scale,
    int use_qk_l2norm, int gate_logits, float g_bias, float b_bias, int64_t chunk, void* workspace,
    size_t workspace_bytes, int32_t* start_flag, int32_t start_epoch, void* stream) {
  using namespace atma;
  if (chunk != kChunk)
    return set_error(ATMA_ERR_UNSUPPORTED, "chunk_gated_delta_rule: chunk must be %d", kChunk);
  if (dk != dv || (dk != 64 && dk != 128))
    return set_error(ATMA_ERR_UNSUPPORTED, "chunk_gated_delta_rule: dk=dv in {64,128} (got %lld,%lld)",
                     (long long)dk, (long long)dv);
  if (B < 0 || T < 0 || H <= 0) return set_error(ATMA_ERR_INVALID, "chunk_gated_delta_rule: bad sizes");
  if (Hkv <= 0 || H % Hkv)
    return set_error(ATMA_ERR_INVALID, "chunk_gated_delta_rule: H=%lld not a multiple of Hkv=%lld",
                     (long long)H, (long long)Hkv);
  if (B * H > 0x7fffffffll || T > (1ll << 30))
    return set_error(ATMA_ERR_INVALID, "chunk_gated_delta_rule: sizes too large");
  const int es = dtype_size(dtype);
  if (!es) return set_error(ATMA_ERR_INVALID, "chunk_gated_delta_rule: unknown dtype %d", dtype);
  if (B == 0) return ATMA_OK;
  if (T == 0) {
    // no tokens: the final state is the initial state -- not representable without a copy
    // kernel; callers short-circuit T == 0 on the host.
    return set_error(ATMA_ERR_INVALID, "chunk_gated_delta_rule: T must be > 0");
  }
  if (!q || !k || !v || !g || !beta || !o)
    return set_error(ATMA_ERR_INVALID, "chunk_gated_delta_rule: null pointer");
  if (es == 2 && T * H * dk * 2 >= (1ll << 32))  // one sequence's output rows form one buffer
    return set_error(ATMA_ERR_UNSUPPORTED, "chunk_gated_delta_rule: T*H*d too large for one sequence");
  if (es == 2 && (q_st >= (1 << 24) || k_st >= (1 << 24) || v_st >= (1 << 24) || q_st < dk || k_st < dk ||
                  v_st < dv))
    // the kernels copy a chunk's q / k / v rows through one buffer descriptor each
    return set_error(ATMA_ERR_UNSUPPORTED, "chunk_gated_delta_rule: q/k/v token stride out of range");
  if (es == 2 && B * H * ((T + 63) / 64) >= (1ll << 31))  // the prep kernel indexes items in 32 bits
    return set_error(ATMA_ERR_UNSUPPORTED, "chunk_gated_delta_rule: B*H*chunks too large");
  const size_t need = atma_chunk_gated_delta_workspace_bytes(B, T, H, dk, dv, chunk, dtype);
  if (!workspace || workspace_bytes < need)
    return set_error(ATMA_ERR_WORKSPACE, "chunk_gated_delta_rule: workspace %zu < %zu bytes",
                     workspace_bytes, need);
  GdnArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_st = q_st; a.q_sh = q_sh;
  a.k = k; a.k_sb = k_sb; a.k_st = k_st; a.k_sh = k_sh;
  a.v = v; a.v_sb = v_sb; a.v_st = v_st; a.v_sh = v_sh;
  a.g = g; a.beta = beta; a.s0 = initial_state; a.s_out = final_state; a.o = o;
  a.B = (int)B; a.T = (int)T; a.H = (int)H; a.NC = (int)((T + chunk - 1) / chunk);
  a.G = (int)(H / Hkv);
  a.scale = scale; a.l2norm = use_qk_l2norm ? 1 : 0; a.ws = workspace;
  a.gate_logits = gate_logits ? 1 : 0; a.g_bias = g_bias; a.b_bias = b_bias;
  a.start_flag = start_flag; a.start_epoch = start_epoch;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16 || dtype == ATMA_F16) return launch_gdn16(a, dtype, (int)dk, s);
  return dk == 128 ? launch_gdn<float, 128>(a, s) : launch_gdn<float, 64>(a, s);
}

namespace atma {

// One lane polls the flag (agent-scope loads, which see another kernel's store across the
// XCDs' L2s) with a sleep between polls, and gives up after limit_ticks of the constant
// wall clock, so the kernel always ends; a timeout only costs the overlap, never results.
__global__ void __launch_bounds__(64) start_wait_kernel(const int* flag, int epoch, uint64_t limit_ticks) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = wall_clock64();
  while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch) {
    if (wall_clock64() - t0 > limit_ticks) break;
    __builtin_amdgcn_s_sleep(2);
  }
}

}  // namespace atma

extern "C" int atma_wait_start_flag(const int32_t* flag, int32_t epoch, int64_t timeout_us, void* stream) {
  using namespace atma;
  if (!flag) return set_error(ATMA_ERR_INVALID, "wait_start_flag: null flag");
  if (timeout_us <= 0 || timeout_us > 10000000)
    return set_error(ATMA_ERR_INVALID, "wait_start_flag: timeout_us must be in (0, 1e7]");
  static int rate_khz = 0;  // wall clock rate; the same for every MI355X device
  if (!rate_khz) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || rate_khz <= 0)
      return set_error(ATMA_ERR_HIP, "wait_start_flag: wall clock rate unavailable");
  }
  const uint64_t ticks = (uint64_t)timeout_us * (uint64_t)rate_khz / 1000u;
  start_wait_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>(flag, epoch, ticks);
  return check_launch("wait_start_flag");
}
