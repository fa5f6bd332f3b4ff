// Prefill projections of the attention layers: y[M, N] = x[M, K] W[N, K]^T,
// bf16 in and out, fp32 accumulation -- the reference's `inp @ W.t()`
// (four_layer_mini_engine.py:6566-6573 full attention q|gate, k, v and
// o_proj; :6386-6395 Gated-DeltaNet in_proj qkv, z, b, a and out_proj),
// which its native prefill runs as hipBLASLt plans
// (native_full_prefill.hip.cpp:552-560, native_prefill_gemm_plans.hip.cpp).
// Both operands are K-contiguous (x row-major, W row-major [out, in]).
//
// Tiling (gfx950): a workgroup of 8 waves computes a BM x BN tile; wave
// (wm, wn) owns RB x CB blocks of 32 x 32 on v_mfma_f32_32x32x16_bf16 (one
// 16-byte LDS read per operand fragment).  K advances 64 per stage through
// an LDS ring filled straight from global memory by buffer_load ...
// lds (16 bytes per lane, 1 KiB per instruction; rows past M or N read as
// zeros through the buffer range check).  The 16-byte chunks of a stage row
// are XOR-swizzled by (row / rows per 256-byte window) mod chunks per row,
// which keeps the ds_read_b128 operand reads free of bank conflicts.  One
// barrier per stage; the refill of a stage is issued once every wave has
// finished reading it, explicit vmcnt waits keep later fetches in flight,
// and the operand fragments of the next 32 K are read into a second register
// set while the current ones feed the MFMAs.
//
// Three tile shapes (256x256, 128x256, 128x128); the host picks the one
// with the lowest tiles-per-CU x measured tile time, so short prompts still
// spread over the chip.  Work items are dealt to the 8 XCDs in
// contiguous ranges that sweep 8 row tiles per column tile, so the
// workgroups of one XCD share A rows and W rows through its L2.
#include "common.h"

#include <mutex>

namespace q36 {
namespace {

constexpr unsigned kGOob = 0x80000000u;  // an offset past every buffer range

template <int RB_, int CB_, int WM_, int WN_, int MINWG_, int BK_, int STAGES_>
struct GemmCfg {
  static constexpr int RB = RB_, CB = CB_, WM = WM_, WN = WN_, MINWG = MINWG_;
  static constexpr int BM = WM * RB * 32, BN = WN * CB * 32, Waves = WM * WN;
  static constexpr int BK = BK_;                  // K per stage
  static constexpr int Stages = STAGES_;
  static constexpr int RowB = BK * 2;             // bytes per row per stage
  static constexpr int Cpr = RowB / 16;           // 16-byte chunks per row
  static constexpr int Rpi = 1024 / RowB;         // rows per fetch instruction
  static constexpr int Rpw = 256 / RowB;          // rows per 256-byte bank window
  static constexpr int StageB = (BM + BN) * RowB;
  static constexpr int Lds = Stages * StageB;
  static constexpr int Instr = (BM + BN) / Rpi / Waves;   // fetches per wave per stage
  static_assert((BM + BN) / Rpi % Waves == 0, "fetch split");
  static_assert(BM % Rpi == 0, "A rows fill whole instructions");
  static_assert(Stages >= 2 && Stages <= 4, "ring depth");
};
// K = 64 per stage, two stages: each fetch instruction reads 8 whole 128-byte
// rows (with 32 per stage it read 16 half lines); measured on MI355X
// 8-13% faster than 32 per stage x 4 stages at every model shape.
using CfgL = GemmCfg<4, 2, 2, 4, 1, 64, 2>;   // 256 x 256, 128 KiB LDS
using CfgM = GemmCfg<2, 2, 2, 4, 1, 64, 2>;   // 128 x 256,  96 KiB LDS
using CfgS = GemmCfg<2, 1, 2, 4, 2, 64, 2>;   // 128 x 128,  64 KiB LDS, 2 per CU

__device__ __forceinline__ void g_fetch(unsigned lds_addr, int voff, const u32x4& rsrc) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ u32x4 g_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  return u32x4{(unsigned)a, (unsigned)(a >> 32), bytes, 0x00020000u};
}

// s_waitcnt immediate: at most n vector-memory operations outstanding.
constexpr int g_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

struct GemmArgs {
  const bf16* x;
  const bf16* w;
  bf16* y;
  unsigned ldx, ldy, M, N, K;
  unsigned m_tiles, n_tiles, share;
};

template <class C>
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

  // Fetch plan: instruction ins moves stage rows 16 ins .. +15 (A rows
  // first, then W rows); lane = (row in instruction, chunk position), the
  // source chunk being position ^ key(stage row).
  const int rin = lane / C::Cpr, cpos = lane % C::Cpr;
  unsigned f_off[C::Instr];
  u32x4 f_rs[C::Instr];
#pragma unroll
  for (int j = 0; j < C::Instr; ++j) {
    const int ins = wave * C::Instr + j;
    const int srow = ins * C::Rpi + rin;
    const bool is_a = srow < C::BM;
    const int r = is_a ? srow : srow - C::BM;
    const bool live = is_a ? r < rows : r < cols;
    const unsigned off = is_a ? (unsigned)r * p.ldx * 2u : (unsigned)r * p.K * 2u;
    f_off[j] = live ? off + ((cpos ^ ((srow / C::Rpw) % C::Cpr)) * 16) : kGOob;
    const u32x4 rs = is_a ? ars : brs;
#pragma unroll
    for (int c = 0; c < 4; ++c) f_rs[j][c] = __builtin_amdgcn_readfirstlane(rs[c]);
  }
  const unsigned lds0 = static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds));
  auto fetch = [&](int step) {
    const unsigned sbase = lds0 + (step % C::Stages) * C::StageB;
    const unsigned kb = (unsigned)step * C::RowB;
#pragma unroll
    for (int j = 0; j < C::Instr; ++j) {
      const int ins = wave * C::Instr + j;
      // a dead row keeps its out-of-range offset (nothing is read), so every
      // wave issues the same number of loads per stage for the vmcnt waits
      const int off = f_off[j] == kGOob ? (int)kGOob : (int)(f_off[j] + kb);
      g_fetch(sbase + ins * C::Rpi * C::RowB, off, f_rs[j]);
    }
  };

  const int wm = wave % C::WM, wn = wave / C::WM;
  const int li = lane & 31, kh = lane >> 5;
  const int arow = C::RB * 32 * wm + li;
  const int brow = C::BM + C::CB * 32 * wn + li;
  int koff[C::BK / 16];
#pragma unroll
  for (int s = 0; s < C::BK / 16; ++s) koff[s] = ((2 * s + kh) ^ ((li / C::Rpw) % C::Cpr)) * 16;

  f32x16 acc[C::RB][C::CB];
#pragma unroll
  for (int i = 0; i < C::RB; ++i)
#pragma unroll
    for (int j = 0; j < C::CB; ++j) acc[i][j] = f32x16{};

  // Software pipeline over half-steps of 32 K (a stage holds BK / 32 of
  // them; the fetch of step t is issued Stages steps ahead, into the stage
  // whose fragments were just taken):
  //   half-step h: if h + 1 starts a new step t, wait for this wave's fetch
  //   of t, barrier (every wave's fetches of t landed, every read of step
  //   t - 1 done), fetch step t - 1 + Stages into the stage of t - 1; read
  //   half h + 1's fragments into the other register set; then the MFMAs of
  //   half h on fragments already in registers -- so the LDS reads of the
  //   next half overlap this half's MFMAs.
  constexpr int kHS = C::BK / 32;        // half-steps per stage
  const int nsteps = (int)(p.K / C::BK);
  const int nh = nsteps * kHS;
  bf16x8 fa[2][2][C::RB], fb[2][2][C::CB];
  auto read_half = [&](int h, bf16x8 (&a)[2][C::RB], bf16x8 (&b)[2][C::CB]) {
    const char* st = lds + ((h / kHS) % C::Stages) * C::StageB;
    const int sub0 = (h % kHS) * 2;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb)
        b[s][cb] = *reinterpret_cast<const bf16x8*>(st + (brow + 32 * cb) * C::RowB + koff[sub0 + s]);
#pragma unroll
      for (int rb = 0; rb < C::RB; ++rb)
        a[s][rb] = *reinterpret_cast<const bf16x8*>(st + (arow + 32 * rb) * C::RowB + koff[sub0 + s]);
    }
  };
  auto mfmas = [&](const bf16x8 (&a)[2][C::RB], const bf16x8 (&b)[2][C::CB]) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int rb = 0; rb < C::RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) acc[rb][cb] = mfma32x32x16(a[s][rb], b[s][cb], acc[rb][cb]);
  };
  // wait until this wave's fetch of `step` landed, given the fetches issued
  // so far (steps up to issued - 1)
  auto wait_fetch = [&](int step, int issued) {
    const int later = issued - 1 - step;   // fetch groups issued after `step`
    if (later >= 3) __builtin_amdgcn_s_waitcnt(g_vmcnt(3 * C::Instr));
    else if (later == 2) __builtin_amdgcn_s_waitcnt(g_vmcnt(2 * C::Instr));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(g_vmcnt(C::Instr));
    else __builtin_amdgcn_s_waitcnt(g_vmcnt(0));
  };
  int issued = min(C::Stages, nsteps);
  for (int st = 0; st < issued; ++st) fetch(st);
  wait_fetch(0, issued);
  __syncthreads();
  read_half(0, fa[0], fb[0]);
  auto iteration = [&](int h, bf16x8 (&ca)[2][C::RB], bf16x8 (&cb)[2][C::CB],
                       bf16x8 (&na)[2][C::RB], bf16x8 (&nb)[2][C::CB]) {
    if (h + 1 < nh) {
      if ((h + 1) % kHS == 0) {
        const int t = (h + 1) / kHS;
        wait_fetch(t, issued);
        // this wave's reads of step t - 1 are complete (their registers are
        // about to be consumed), so after the barrier its stage may be refilled
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        __syncthreads();
        if (t - 1 + C::Stages < nsteps) {
          fetch(t - 1 + C::Stages);
          ++issued;
        }
      }
      read_half(h + 1, na, nb);
    }
    mfmas(ca, cb);
  };
  int h = 0;
  for (; h + 1 < nh; h += 2) {
    iteration(h, fa[0], fb[0], fa[1], fb[1]);
    iteration(h + 1, fa[1], fb[1], fa[0], fb[0]);
  }
  if (h < nh) iteration(h, fa[0], fb[0], fa[1], fb[1]);

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
int launch_cfg(const GemmArgs& base, hipStream_t stream) {
  GemmArgs a = base;
  a.m_tiles = (a.M + C::BM - 1) / C::BM;
  a.n_tiles = (a.N + C::BN - 1) / C::BN;
  a.share = (a.m_tiles * a.n_tiles + 7) / 8;
  hipLaunchKernelGGL(prefill_gemm_kernel<C>, dim3(8 * a.share), dim3(64 * C::Waves), C::Lds,
                     stream, a);
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
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgL>), CfgL::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgM>), CfgM::Lds},
        {reinterpret_cast<const void*>(prefill_gemm_kernel<CfgS>), CfgS::Lds}};
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long long cl = tile_cost<CfgL>(m, n, 58), cm = tile_cost<CfgM>(m, n, 35),
                  cs = tile_cost<CfgS>(m, n, 18);
  if (cl <= cm && cl <= cs) return launch_cfg<CfgL>(a, st);
  if (cm <= cs) return launch_cfg<CfgM>(a, st);
  return launch_cfg<CfgS>(a, st);
}
