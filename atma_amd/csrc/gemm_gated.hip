// The MLP's first projection with its activation over many token rows (the served prefill):
//   y[m, n] = gate * relu(a)^2,  a = round(x[m] . w[n] + b[n]),  gate = round(x[m] . w[H + n] + b[H + n])
// for n < H, with w (2H, K) -- the a rows, then the gate rows -- in squared_relu_gate's
// arithmetic on the rounded projections.  The vendor GEMM writes the 2H-wide projection
// (65,536 x 8,192 x 2 B = 1.07 GB at configs[4]) and the activation kernel reads it back and
// writes the H-wide result: 1.6 GB of traffic this kernel never makes.
//
// No reference counterpart as one call: model/layers.py:19-31 (the MLP) runs nn.Linear
// (model/reference.py:22-28) and then the activation; inference/models/atma.py:87-96 is the
// inference form.
//
// Layout.  A workgroup of 8 waves owns 256 token rows x 128 output features, i.e. 256 weight
// rows: the 128 a rows and the 128 gate rows of the same features.  K runs in steps of 64:
// the x tile (256 x 64) and the weight tile (256 x 64) of a step go straight from memory
// into LDS with buffer_load ... lds (rows past M read as zeros), double-buffered, the copies
// of step k + 1 issued right after the one barrier of step k.  Rows are 128 bytes (8
// chunks of 16); chunk c of row r sits at chunk position c ^ f(r), f(r) = (r / 2) mod 8
// (gg_swizzle), so the MFMA operand reads (16 bytes of 32 consecutive rows at one chunk)
// are conflict-free: each 16-lane group of a ds_read_b128 covers all 64 banks.  The grid is
// persistent (one workgroup per CU): the next tile's first copies fly during the current
// tile's epilogue.
//
// Products.  v_mfma_f32_32x32x16 with the weights as the A operand (MFMA rows = features)
// and the tokens as the B operand (columns = tokens).  Wave (wm, wn) computes tokens
// 128 wm .. + 127 and features 32 wn .. + 31: 4 token tiles x (a tile, gate tile), so the a
// and gate values of one output sit in the same register of the same lane and the
// activation is formed in registers and stored from them.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace atma {

template <typename T>
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  Pack8 pa, pb;
  pa.u = a;
  pb.u = b;
  if constexpr (__is_same(T, bf16)) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa.b, pb.b, c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(pa.h, pb.h, c, 0, 0, 0);
  }
}

constexpr int kGgBM = 256;       // token rows per workgroup
constexpr int kGgBF = 128;       // output features per workgroup (256 weight rows)
constexpr int kGgBK = 64;        // K per step

// Chunk position offset of row r in the 128-byte-row tiles: rows r and r + 2 are 256 bytes
// apart (the same banks), so 16 consecutive rows need 8 distinct offsets per row parity.
__device__ __forceinline__ int gg_swizzle(int r) { return (r >> 1) & 7; }

struct GatedArgs {
  const void* x;  // (M, K) row stride ldx
  int64_t ldx;
  const void* w;  // (2H, K) row stride ldw
  int64_t ldw;
  const void* bias;  // (2H,) or null
  void* y;           // (M, H) row stride ldy
  int64_t ldy;
  int M, H, K;
  int m_tiles, f_tiles, per_xcd;
};

// (m0, f0) of XCD-local tile u of XCD x: each XCD owns a contiguous range of tiles, walked as
// groups of 4 token tiles x all feature tiles with the token tile fastest, so the ~32 tiles
// an XCD has in flight share 4 x tiles and 8 weight tiles in its L2
__device__ __forceinline__ bool gated_tile(const GatedArgs& a, int x, int u, int& m0, int& f0) {
  const int t = x * a.per_xcd + u;
  if (u >= a.per_xcd || t >= a.m_tiles * a.f_tiles) return false;
  const int grp = t / (4 * a.f_tiles), r = t - grp * 4 * a.f_tiles;
  const int gm = min(4, a.m_tiles - 4 * grp);
  m0 = (4 * grp + r % gm) * kGgBM;
  f0 = (r / gm) * kGgBF;
  return true;
}

// Persistent: one workgroup per CU walks its XCD's tiles (workgroup b runs on XCD b % 8).  The
// first copies of the next tile are issued during the last K step of the current one, and the
// epilogue (bias, rounding, activation, stores straight from the accumulators) runs while
// they are in flight.
template <typename T>
__global__ void __launch_bounds__(512, 1) linear_gated_kernel(GatedArgs a) {
  // [stage][x tile, weight tile][256 rows x 64]: 128 KB
  __shared__ __attribute__((aligned(16))) T lds[2][2][kGgBM * kGgBK];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: copy destinations stay in SALU
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, h = lane >> 5;
  const int xcd = blockIdx.x & 7, nper = gridDim.x >> 3;
  int u = blockIdx.x >> 3, m0, f0;
  if (!gated_tile(a, xcd, u, m0, f0)) return;

  // ---- copies: wave w moves rows 32 w .. + 31 of both tiles, 8 rows per instruction; lane l
  // writes row (l / 8), chunk position l % 8, i.e. logical chunk (l % 8) ^ f(row); rows
  // past M land past the buffer's end (zeros)
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * sizeof(T)));
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w, (uint32_t)((int64_t)2 * a.H * a.ldw * sizeof(T)));
  // copy i writes tile rows 8 i + crow (mod 16: the wave's rows start at a multiple of 32)
  const int crow = lane >> 3;
  const uint32_t cchunk[2] = {16u * (uint32_t)((lane & 7) ^ gg_swizzle(crow)),
                              16u * (uint32_t)((lane & 7) ^ gg_swizzle(8 + crow))};
  uint32_t xv0, wv0;
  auto aim = [&](int tm0, int tf0) {  // the copy offsets of tile (tm0, tf0)
    xv0 = (uint32_t)((int64_t)(tm0 + 32 * wave + crow) * a.ldx * sizeof(T));
    const int wrow0 = (wave < 4 ? tf0 : a.H + tf0 - 128) + 32 * wave + crow;
    wv0 = (uint32_t)((int64_t)wrow0 * a.ldw * sizeof(T));
  };
  const uint32_t xstep8 = (uint32_t)(8 * a.ldx * sizeof(T)), wstep8 = (uint32_t)(8 * a.ldw * sizeof(T));
  const uint32_t dst0 = lds_offset(&lds[0][0][0]) + (uint32_t)(32 * wave * kGgBK * sizeof(T));
  constexpr uint32_t kTileBytes = kGgBM * kGgBK * sizeof(T);
  auto issue = [&](auto stage_c, int kb) {
    constexpr int S = decltype(stage_c)::value;
    const uint32_t kofs = (uint32_t)kb * (kGgBK * sizeof(T));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = dst0 + S * 2 * kTileBytes + i * (8 * kGgBK * sizeof(T));
      dma_buf16_at(xr, xv0 + i * xstep8 + kofs + cchunk[i & 1], 0u, d);
      dma_buf16_at(wr, wv0 + i * wstep8 + kofs + cchunk[i & 1], 0u, d + kTileBytes);
    }
  };

  // ---- operand reads: 16 bytes of row (tile row + l32), logical chunk 2 s + h
  const int sw = gg_swizzle(l32 & 15);
  uint32_t chk[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) chk[s] = 16u * (uint32_t)((2 * s + h) ^ sw);
  const uint32_t arow_a = (uint32_t)((32 * wn + l32) * kGgBK * sizeof(T));
  const uint32_t arow_g = (uint32_t)((128 + 32 * wn + l32) * kGgBK * sizeof(T));
  const uint32_t brow = (uint32_t)((128 * wm + l32) * kGgBK * sizeof(T));

  f32x16 acc_a[4], acc_g[4];
  auto compute = [&](auto stage_c) {
    constexpr int S = decltype(stage_c)::value;
    const char* xs = (const char*)&lds[S][0][0];
    const char* ws = (const char*)&lds[S][1][0];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4 fa = *(const u32x4*)(ws + arow_a + chk[s]);
      const u32x4 fg = *(const u32x4*)(ws + arow_g + chk[s]);
      u32x4 fb[4];
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
        fb[tm] = *(const u32x4*)(xs + brow + tm * (32 * kGgBK * sizeof(T)) + chk[s]);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        acc_a[tm] = mfma32x32x16<T>(fa, fb[tm], acc_a[tm]);
        acc_g[tm] = mfma32x32x16<T>(fg, fb[tm], acc_g[tm]);
      }
    }
  };

  // this lane's features in accumulator register group j: 32 wn + 8 j + 4 h + e; their
  // biases (a, then gate) as packed 16-bit pairs, loaded a tile ahead of the epilogue
  uint32_t bias2[4][2][2];
  auto load_bias = [&](uint32_t (&dst)[4][2][2], int tf0) {
    const uint32_t* bp = (const uint32_t*)((const T*)(a.bias ? a.bias : a.x) + (a.bias ? tf0 : 0));
    const int hstep = a.bias ? a.H / 2 : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int fw = (32 * wn + 8 * j + 4 * h) / 2;
      dst[j][0][0] = bp[fw];
      dst[j][0][1] = bp[fw + 1];
      dst[j][1][0] = bp[hstep + fw];
      dst[j][1][1] = bp[hstep + fw + 1];
    }
  };
  load_bias(bias2, f0);

  const int nk = a.K / kGgBK;
  std::integral_constant<int, 0> s0;
  std::integral_constant<int, 1> s1;
  aim(m0, f0);
  issue(s0, 0);
  while (true) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc_a[i] = acc_g[i] = f32x16{};
    // ---- the K loop: step k waits for its own copies, one barrier (every wave's copies of
    // step k landed, every wave done reading the other stage), then issues the next copies
    // into the other stage and computes step k; the last step issues the next tile's first
    int nm0 = 0, nf0 = 0;
    bool more = false;
    for (int kb = 0; kb < nk; kb += 2) {  // nk is even
      wait_vmcnt<0>();
      lds_barrier();
      issue(s1, kb + 1);
      compute(s0);
      wait_vmcnt<0>();
      lds_barrier();
      if (kb + 2 < nk) {
        issue(s0, kb + 2);
      } else {
        u += nper;
        more = gated_tile(a, xcd, u, nm0, nf0);
        if (more) {
          aim(nm0, nf0);
          issue(s0, 0);
        }
      }
      compute(s1);
    }

    // ---- epilogue of tile (m0, f0) from the accumulators: token 128 wm + 32 tm + l32 gets
    // 4 consecutive features per register group (8-byte stores; the workgroup writes whole
    // 256-byte row pieces, which L2 merges)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int fl = 32 * wn + 8 * j + 4 * h;
      float ba[4], bg[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ba[e] = a.bias ? elem16<T>(u32x4{bias2[j][0][0], bias2[j][0][1], 0u, 0u}, e) : 0.f;
        bg[e] = a.bias ? elem16<T>(u32x4{bias2[j][1][0], bias2[j][1][1], 0u, 0u}, e) : 0.f;
      }
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        const int row = m0 + 128 * wm + 32 * tm + l32;
        float hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float av = to_f32(from_f32<T>(acc_a[tm][4 * j + e] + ba[e]));
          const float gv = to_f32(from_f32<T>(acc_g[tm][4 * j + e] + bg[e]));
          hv[e] = sq_relu_gate1<T>(av, gv);
        }
        if (row < a.M)
          *(u32x2*)((T*)a.y + (int64_t)row * a.ldy + f0 + fl) = u32x2{pack2<T>(hv[0], hv[1]), pack2<T>(hv[2], hv[3])};
      }
    }
    if (!more) break;
    m0 = nm0;
    f0 = nf0;
    load_bias(bias2, f0);
  }
}

}  // namespace atma

extern "C" int atma_linear_gated(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, void* y,
                                 int64_t ldy, int64_t M, int64_t H, int64_t K, int dtype, void* stream) {
  using namespace atma;
  if (dtype != ATMA_BF16 && dtype != ATMA_F16)
    return set_error(ATMA_ERR_UNSUPPORTED, "linear_gated: 16-bit inputs only (dtype %d)", dtype);
  if (M < 0 || H < kGgBF || H % kGgBF || K < 2 * kGgBK || K % (2 * kGgBK) || M > 0x7fffffff || H > (1 << 24))
    return set_error(ATMA_ERR_UNSUPPORTED,
                     "linear_gated: unsupported shape M=%lld H=%lld K=%lld (H a multiple of %d, K of %d)",
                     (long long)M, (long long)H, (long long)K, kGgBF, 2 * kGgBK);
  if (M == 0) return ATMA_OK;
  if (!x || !w || !y) return set_error(ATMA_ERR_INVALID, "linear_gated: null pointer");
  if ((uintptr_t)x % 16 || ldx % 8 || ldx < K || (uintptr_t)w % 16 || ldw % 8 || ldw < K || (uintptr_t)y % 16 ||
      ldy % 8 || ldy < H || (bias && (uintptr_t)bias % 4))
    return set_error(ATMA_ERR_INVALID, "linear_gated: x, w and y rows must be 16-byte aligned, bias 4-byte");
  // byte offsets of the copies (rows up to M + 255 of x, 2H of w) stay 32-bit
  if ((M + kGgBM) * ldx * 2 >= (1ll << 32) || 2 * H * ldw * 2 >= (1ll << 32))
    return set_error(ATMA_ERR_UNSUPPORTED, "linear_gated: x or w spans 4 GiB or more");
  GatedArgs a{x, ldx, w, ldw, bias, y, ldy, (int)M, (int)H, (int)K, 0, 0, 0};
  a.m_tiles = (int)((M + kGgBM - 1) / kGgBM);
  a.f_tiles = (int)(H / kGgBF);
  const int64_t tiles = (int64_t)a.m_tiles * a.f_tiles;
  a.per_xcd = (int)((tiles + 7) / 8);
  // one workgroup per CU (its 128 KB of LDS), at most one per tile; a multiple of 8
  const int64_t wgs = std::min<int64_t>(256, 8 * (int64_t)a.per_xcd);
  const dim3 grid((unsigned)wgs), block(512);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ATMA_BF16) linear_gated_kernel<bf16><<<grid, block, 0, s>>>(a);
  else linear_gated_kernel<f16><<<grid, block, 0, s>>>(a);
  return check_launch("linear_gated");
}
