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
  float* part;          // split-K: fp32 partial products [ksplit][M][N]
  unsigned ldx, ldy, M, N, K;
  unsigned m_tiles, n_tiles, share;
  unsigned ksplit, kslice;   // K is cut into ksplit slices of kslice
};

enum GemmOut { kOutBf16 = 0, kOutBf16Staged = 1, kOutPartial = 2 };

// kOut: kOutBf16Staged when y is 16-byte aligned and ldy % 8 == 0 (the tile
// leaves through LDS as 16-byte row chunks, gemm_store_tile_lds), kOutBf16
// otherwise (one store per element), kOutPartial for a split-K slice (fp32
// products into the slice's plane of p.part; gemm_splitk_reduce_kernel sums
// the planes in slice order and rounds once).
template <class C, int kOut>
__global__ __launch_bounds__(64 * C::Waves, C::MINWG) void prefill_gemm_kernel(GemmArgs p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  // item -> (K slice, row tile, column tile): XCD x = blockIdx % 8 takes
  // items [x * share, (x + 1) * share); within a K slice, items sweep groups
  // of 8 row tiles per column tile.
  const unsigned tiles = p.m_tiles * p.n_tiles;
  const unsigned items = tiles * p.ksplit;
  const unsigned xi = blockIdx.x >> 3;
  if (xi >= p.share) return;
  const unsigned item_all = (blockIdx.x & 7) * p.share + xi;
  if (item_all >= items) return;
  const unsigned ks = item_all / tiles, item = item_all % tiles;
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
    const unsigned off = (is_a ? (unsigned)r * p.ldx * 2u : (unsigned)r * p.K * 2u) +
                         ks * p.kslice * 2u;
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
  gemm_mainloop<C>(lds, fp, (int)p.kslice, arow, brow, acc);

  if constexpr (kOut == kOutPartial) {
    float* pp = p.part + (size_t)ks * p.M * p.N + (size_t)row0 * p.N + n0;
#pragma unroll
    for (int rb = 0; rb < C::RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = C::RB * 32 * wm + 32 * rb + 8 * (i >> 2) + 4 * kh + (i & 3);
        if (r >= rows) continue;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) {
          const int c = C::CB * 32 * wn + 32 * cb + li;
          if (c < cols) pp[(size_t)r * p.N + c] = acc[rb][cb][i];
        }
      }
    return;
  }
  if constexpr (kOut == kOutBf16Staged) {
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

// y[r][c] = bf16(sum over slices s = 0, 1, ... of part[s][r][c]): one
// rounding, slices added in order (deterministic); 4 columns per thread.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part,
                                                                 unsigned ksplit, unsigned M,
                                                                 unsigned N, bf16* __restrict__ y,
                                                                 unsigned ldy) {
  const unsigned n4 = (N + 3) / 4;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)M * n4) return;
  const unsigned r = (unsigned)(idx / n4), c = (unsigned)(idx % n4) * 4;
  const size_t plane = (size_t)M * N;
  const float* src = part + (size_t)r * N + c;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (unsigned k = 0; k < ksplit; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < N) s[e] += src[k * plane + e];
  bf16* yr = y + (size_t)r * ldy + c;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c + e < N) yr[e] = f2bf(s[e]);
}

// Launch plan: tile shape and K split.  Cost = rounds of 256 workgroups x
// the measured tile time (K = 2048: 256x256 58 us, 128x256 35 us, 128x128
// 18 us, two per CU) scaled by the slice length, plus, for a split, the
// fp32 partial planes written and read back (at ~5 TB/s) -- so short prompts
// with a long K (the K = 4096 output projections at T = 1024 fill half the
// GPU with whole-K tiles) spread K over more workgroups.
struct GemmPlan {
  int cfg;            // 0: 256x256, 1: 128x256, 2: 128x128
  unsigned ksplit;
};

GemmPlan gemm_plan(unsigned M, unsigned N, unsigned K, bool allow_split) {
  const int bm[3] = {CfgL::BM, CfgM::BM, CfgS::BM}, bn[3] = {CfgL::BN, CfgM::BN, CfgS::BN};
  const double tt[3] = {58.0, 35.0, 18.0};
  GemmPlan best{0, 1};
  double best_cost = 1e30;
  for (int c = 0; c < 3; ++c) {
    const long long wgs = (long long)((M + bm[c] - 1) / bm[c]) * ((N + bn[c] - 1) / bn[c]);
    for (unsigned s = 1; s <= 8; s *= 2) {
      if (s > 1 && (!allow_split || (K / s) % 64 != 0 || K / s < 512)) continue;
      const double rounds = (double)((wgs * s + 255) / 256);
      double cost = rounds * tt[c] * ((double)K / s) / 2048.0;
      if (s > 1) cost += (double)M * N * 4.0 * (2.0 * s) / 5.0e6;
      if (cost < best_cost) {
        best_cost = cost;
        best = GemmPlan{c, s};
      }
    }
  }
  return best;
}

std::once_flag g_gemm_attr_once;
hipError_t g_gemm_attr_status = hipSuccess;

template <class C>
int launch_cfg(const GemmArgs& base, bool vec, hipStream_t stream) {
  GemmArgs a = base;
  a.m_tiles = (a.M + C::BM - 1) / C::BM;
  a.n_tiles = (a.N + C::BN - 1) / C::BN;
  a.share = (a.m_tiles * a.n_tiles * a.ksplit + 7) / 8;
  auto kernel = a.ksplit > 1 ? prefill_gemm_kernel<C, kOutPartial>
                : vec        ? prefill_gemm_kernel<C, kOutBf16Staged>
                             : prefill_gemm_kernel<C, kOutBf16>;
  hipLaunchKernelGGL(kernel, dim3(8 * a.share), dim3(64 * C::Waves), C::Lds, stream, a);
  if (a.ksplit > 1) {
    const size_t n = (size_t)a.M * ((a.N + 3) / 4);
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       stream, a.part, a.ksplit, a.M, a.N, a.y, a.ldy);
  }
  return static_cast<int>(hipGetLastError());
}

size_t splitk_bytes(unsigned m, unsigned n, unsigned ksplit) {
  return ksplit > 1 ? (size_t)ksplit * m * n * sizeof(float) : 0;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; }

}  // namespace
}  // namespace q36

using namespace q36;

namespace {

bool gemm_args_ok(const void* x, unsigned ldx, const void* w, const void* y, unsigned ldy,
                  unsigned m, unsigned n, unsigned k) {
  return !(x == nullptr || w == nullptr || y == nullptr || m == 0 || n == 0 || k == 0 ||
           m > kMaxTokens || n > 65536u || k > 16384u || (k % 64) != 0 || ldx < k ||
           (ldx % 8) != 0 || ldy < n || !al16(x) || !al16(w) ||
           (size_t)256 * ldx * 2 >= kGOob || (size_t)256 * k * 2 >= kGOob);
}

int gemm_run(const void* x, unsigned ldx, const void* w, void* y, unsigned ldy, unsigned m,
             unsigned n, unsigned k, const GemmPlan& plan, float* part, void* stream) {
  std::call_once(g_gemm_attr_once, [] {
    const std::pair<const void*, int> fs[] = {
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgL, kOutBf16>), CfgL::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgM, kOutBf16>), CfgM::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgS, kOutBf16>), CfgS::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgL, kOutBf16Staged>), CfgL::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgM, kOutBf16Staged>), CfgM::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgS, kOutBf16Staged>), CfgS::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgL, kOutPartial>), CfgL::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgM, kOutPartial>), CfgM::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgS, kOutPartial>), CfgS::Lds}};
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
  a.part = part;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = m;
  a.N = n;
  a.K = k;
  a.ksplit = plan.ksplit;
  a.kslice = k / plan.ksplit;
  const bool vec = (ldy % 8) == 0 && al16(y);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (plan.cfg == 0) return launch_cfg<CfgL>(a, vec, st);
  if (plan.cfg == 1) return launch_cfg<CfgM>(a, vec, st);
  return launch_cfg<CfgS>(a, vec, st);
}

}  // namespace

Q36_EXPORT int qwen36_prefill_gemm_bf16(const void* x, unsigned ldx, const void* w, void* y,
                                        unsigned ldy, unsigned m, unsigned n, unsigned k,
                                        void* stream) {
  if (!gemm_args_ok(x, ldx, w, y, ldy, m, n, k)) return Q36_EINVAL;
  return gemm_run(x, ldx, w, y, ldy, m, n, k, gemm_plan(m, n, k, false), nullptr, stream);
}

Q36_EXPORT size_t qwen36_prefill_gemm_workspace_bytes(unsigned m, unsigned n, unsigned k) {
  if (m == 0 || n == 0 || k == 0 || m > kMaxTokens || n > 65536u || k > 16384u ||
      (k % 64) != 0)
    return 0;   // geometry the launch rejects
  return splitk_bytes(m, n, gemm_plan(m, n, k, true).ksplit);
}

Q36_EXPORT int qwen36_prefill_gemm_bf16_ws(const void* x, unsigned ldx, const void* w, void* y,
                                           unsigned ldy, unsigned m, unsigned n, unsigned k,
                                           void* ws, size_t ws_bytes, void* stream) {
  if (!gemm_args_ok(x, ldx, w, y, ldy, m, n, k)) return Q36_EINVAL;
  GemmPlan plan = gemm_plan(m, n, k, true);
  const size_t need = splitk_bytes(m, n, plan.ksplit);
  if (need > 0 && (ws == nullptr || ws_bytes < need || !al16(ws))) return Q36_EINVAL;
  return gemm_run(x, ldx, w, y, ldy, m, n, k, plan, static_cast<float*>(ws), stream);
}
