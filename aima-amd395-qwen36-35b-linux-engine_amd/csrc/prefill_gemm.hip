// Prefill projections of the attention layers: y[M, N] = x[M, K] W[N, K]^T,
// bf16 in and out, fp32 accumulation -- the reference's `inp @ W.t()`
// (four_layer_mini_engine.py:6566-6573 full attention q|gate, k, v and
// o_proj; :6386-6395 Gated-DeltaNet in_proj qkv, z, b, a and out_proj),
// which its native prefill runs as hipBLASLt plans
// (native_full_prefill.hip.cpp:552-560, native_prefill_gemm_plans.hip.cpp).
// Both operands are K-contiguous (x row-major, W row-major [out, in]).
//
// Tiling: the shared tile machinery of gemm_tile.h (8 waves of 32 x 32
// MFMA blocks, direct-to-LDS fetches into a swizzled ring, a half-step
// register pipeline).
//
// Three tile shapes (256x256, 128x256, 128x128); the host picks the one
// with the lowest tiles-per-CU x measured tile time, so short prompts still
// spread over the chip.  Work items are dealt to the 8 XCDs in
// contiguous ranges that sweep 8 row tiles per column tile, so the
// workgroups of one XCD share A rows and W rows through its L2.
#include "gemm_tile.h"

#include <mutex>

namespace q36 {
namespace {

// K = 64 per stage, two stages: each fetch instruction reads 8 whole 128-byte
// rows (with 32 per stage it read 16 half lines); measured on MI355X
// 8-13% faster than 32 per stage x 4 stages at every model shape.
using CfgL = GemmCfg<4, 2, 2, 4, 1, 64, 2>;   // 256 x 256, 128 KiB LDS
using CfgM = GemmCfg<2, 2, 2, 4, 1, 64, 2>;   // 128 x 256,  96 KiB LDS
using CfgS = GemmCfg<2, 1, 2, 4, 2, 64, 2>;   // 128 x 128,  64 KiB LDS, 2 per CU

struct GemmArgs {
  const bf16* x;
  const bf16* w;
  bf16* y;
  unsigned ldx, ldy, M, N, K;
  unsigned m_tiles, n_tiles, share;
};

// kVec: y 16-byte aligned and ldy % 8 == 0, so the tile leaves through LDS
// as 16-byte row chunks (gemm_store_tile_lds); otherwise one bf16 store per
// element.
template <class C, bool kVec>
__global__ __launch_bounds__(64 * C::Waves, C::MINWG) void prefill_gemm_kernel(GemmArgs p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  // item -> (row tile, column tile): XCD x = blockIdx % 8 takes items
  // [x * share, (x + 1) * share); items sweep groups of 8 row tiles per
  // column tile.
  const unsigned items = p.m_tiles * p.n_tiles;
  const unsigned xi = blockIdx.x >> 3;
  if (xi >= p.share) return;
  const unsigned item = (blockIdx.x & 7) * p.share + xi;
  if (item >= items) return;
  const unsigned grp = item / (8 * p.n_tiles), rem = item % (8 * p.n_tiles);
  const unsigned mg = min(8u, p.m_tiles - grp * 8);
  const unsigned nt = rem / mg, mt = grp * 8 + rem % mg;
  const unsigned row0 = mt * C::BM, n0 = nt * C::BN;
  const int rows = (int)min((unsigned)C::BM, p.M - row0);
  const int cols = (int)min((unsigned)C::BN, p.N - n0);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const u32x4 ars = g_rsrc(p.x + (size_t)row0 * p.ldx, (unsigned)rows * p.ldx * 2u);
  const u32x4 brs = g_rsrc(p.w + (size_t)n0 * p.K, (unsigned)cols * p.K * 2u);

  FetchPlan<C> fp;
#pragma unroll
  for (int j = 0; j < C::Instr; ++j) {
    const int srow = fetch_stage_row<C>(wave, j, lane);
    const bool is_a = srow < C::BM;
    const int r = is_a ? srow : srow - C::BM;
    const bool live = is_a ? r < rows : r < cols;
    const unsigned off = is_a ? (unsigned)r * p.ldx * 2u : (unsigned)r * p.K * 2u;
    fp.off[j] = live ? off + fetch_chunk_off<C>(srow, lane) : kGOob;
    const u32x4 rs = is_a ? ars : brs;
#pragma unroll
    for (int c = 0; c < 4; ++c) fp.rs[j][c] = __builtin_amdgcn_readfirstlane(rs[c]);
  }

  const int wm = wave % C::WM, wn = wave / C::WM;
  const int li = lane & 31, kh = lane >> 5;
  const int arow = C::RB * 32 * wm + li;
  int brow[C::CB];
#pragma unroll
  for (int cb = 0; cb < C::CB; ++cb) brow[cb] = C::BM + C::CB * 32 * wn + 32 * cb + li;
  f32x16 acc[C::RB][C::CB];
#pragma unroll
  for (int i = 0; i < C::RB; ++i)
#pragma unroll
    for (int j = 0; j < C::CB; ++j) acc[i][j] = f32x16{};
  gemm_mainloop<C>(lds, fp, (int)p.K, arow, brow, acc);

  if constexpr (kVec) {
    bf16* y0 = p.y + (size_t)row0 * p.ldy + n0;
    gemm_store_tile_lds<C>(
        lds, acc, cols, [&](int r) { return r < rows ? y0 + (size_t)r * p.ldy : nullptr; },
        [](float x, int) { return f2bf(x); });
    return;
  }
  // acc[rb][cb][i]: tile row RB*32 wm + 32 rb + 8 (i / 4) + 4 kh + i % 4,
  // column CB*32 wn + 32 cb + li.
#pragma unroll
  for (int rb = 0; rb < C::RB; ++rb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = C::RB * 32 * wm + 32 * rb + 8 * (i >> 2) + 4 * kh + (i & 3);
      if (r >= rows) continue;
      bf16* yr = p.y + (size_t)(row0 + r) * p.ldy + n0;
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb) {
        const int c = C::CB * 32 * wn + 32 * cb + li;
        if (c < cols) yr[c] = f2bf(acc[rb][cb][i]);
      }
    }
}

// Cost of a launch = tiles per CU (workgroups / 256, rounded up) x the
// measured time of one tile of the shape on MI355X (K = 2048): 256x256
// 58 us, 128x256 35 us, 128x128 18 us (two per CU).  Fitted on
// M = 1024..8192 x N = 2048, 9216; it picks the fastest of the three at each
// of those shapes.
template <class C>
long long tile_cost(unsigned M, unsigned N, int tile_time) {
  const long long wgs = (long long)((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN);
  return (wgs + 255) / 256 * tile_time;
}

std::once_flag g_gemm_attr_once;
hipError_t g_gemm_attr_status = hipSuccess;

template <class C>
int launch_cfg(const GemmArgs& base, bool vec, hipStream_t stream) {
  GemmArgs a = base;
  a.m_tiles = (a.M + C::BM - 1) / C::BM;
  a.n_tiles = (a.N + C::BN - 1) / C::BN;
  a.share = (a.m_tiles * a.n_tiles + 7) / 8;
  auto kernel = vec ? prefill_gemm_kernel<C, true> : prefill_gemm_kernel<C, false>;
  hipLaunchKernelGGL(kernel, dim3(8 * a.share), dim3(64 * C::Waves), C::Lds, stream, a);
  return static_cast<int>(hipGetLastError());
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; }

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT int qwen36_prefill_gemm_bf16(const void* x, unsigned ldx, const void* w, void* y,
                                        unsigned ldy, unsigned m, unsigned n, unsigned k,
                                        void* stream) {
  if (x == nullptr || w == nullptr || y == nullptr || m == 0 || n == 0 || k == 0 ||
      m > kMaxTokens || n > 65536u || k > 16384u || (k % 64) != 0 || ldx < k ||
      (ldx % 8) != 0 || ldy < n || !al16(x) || !al16(w) || (size_t)256 * ldx * 2 >= kGOob ||
      (size_t)256 * k * 2 >= kGOob)
    return Q36_EINVAL;
  std::call_once(g_gemm_attr_once, [] {
    const std::pair<const void*, int> fs[] = {
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgL, true>), CfgL::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgM, true>), CfgM::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgS, true>), CfgS::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgL, false>), CfgL::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgM, false>), CfgM::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgS, false>), CfgS::Lds}};
    for (const auto& f : fs) {
      const hipError_t e =
          hipFuncSetAttribute(f.first, hipFuncAttributeMaxDynamicSharedMemorySize, f.second);
      if (e != hipSuccess) g_gemm_attr_status = e;
    }
  });
  if (g_gemm_attr_status != hipSuccess) return (int)g_gemm_attr_status;
  GemmArgs a{};
  a.x = static_cast<const bf16*>(x);
  a.w = static_cast<const bf16*>(w);
  a.y = static_cast<bf16*>(y);
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = m;
  a.N = n;
  a.K = k;
  const bool vec = (ldy % 8) == 0 && al16(y);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long long cl = tile_cost<CfgL>(m, n, 58), cm = tile_cost<CfgM>(m, n, 35),
                  cs = tile_cost<CfgS>(m, n, 18);
  if (cl <= cm && cl <= cs) return launch_cfg<CfgL>(a, vec, st);
  if (cm <= cs) return launch_cfg<CfgM>(a, vec, st);
  return launch_cfg<CfgS>(a, vec, st);
}
