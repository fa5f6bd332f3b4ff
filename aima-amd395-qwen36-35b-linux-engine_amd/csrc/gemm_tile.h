// bf16 GEMM tile machinery for gfx950 shared by the prefill projections
// (prefill_gemm.hip) and the MoE block's grouped expert GEMMs
// (moe_prefill.hip): y[rows, cols] = a[rows, K] b[cols, K]^T with both
// operands K-contiguous.
//
// A workgroup of WM x WN waves computes a BM x BN tile; wave (wm, wn) owns
// RB x CB blocks of 32 x 32 on v_mfma_f32_32x32x16_bf16 (one 16-byte LDS
// read per operand fragment).  K advances BK per stage through an LDS ring
// of Stages stages filled straight from global memory by buffer_load ... lds
// (16 bytes per lane, 1 KiB per instruction; a dead row carries an offset
// past the buffer range and reads nothing).  The 16-byte chunks of a stage
// row are XOR-swizzled by (row / rows per 256-byte window) mod chunks per
// row, which keeps the ds_read_b128 operand reads free of bank conflicts.
// One barrier per stage; the refill of a stage is issued once every wave has
// finished reading it, explicit vmcnt waits keep later fetches in flight,
// and the operand fragments of the next 32 K are read into a second
// register set while the current ones feed the MFMAs.
#pragma once

#include "common.h"

namespace q36 {

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
  static_assert(BK % 32 == 0, "whole half-steps per stage");
};

// The leading s_nop covers the hazard the compiler cannot see through the
// inline assembly: the resource SGPRs (and m0) are written by VALU
// readfirstlane / SALU instructions right before, and a VMEM instruction
// reading an SGPR that a VALU wrote needs 5 wait states on gfx950 (an
// instruction issued too early reads the old descriptor).
__device__ __forceinline__ void g_fetch(unsigned lds_addr, int voff, const u32x4& rsrc) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ u32x4 g_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  return u32x4{(unsigned)a, (unsigned)(a >> 32), bytes, 0x00020000u};
}

// s_waitcnt immediate: at most n vector-memory operations outstanding.
constexpr int g_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Per-lane fetch plan: fetch instruction ins = wave * Instr + j moves stage
// rows Rpi ins .. +Rpi-1 (A rows 0..BM-1 first, then B rows); the lane
// (row in instruction, chunk position cpos) reads source chunk cpos ^
// key(stage row).  off[j] is the lane's byte offset in rs[j] at K = 0, or
// kGOob for a dead row.
template <class C>
struct FetchPlan {
  unsigned off[C::Instr];
  u32x4 rs[C::Instr];
};

template <class C>
__device__ __forceinline__ int fetch_stage_row(int wave, int j, int lane) {
  return (wave * C::Instr + j) * C::Rpi + lane / C::Cpr;
}

// Byte offset of the lane's chunk within its (unswizzled) source row.
template <class C>
__device__ __forceinline__ unsigned fetch_chunk_off(int srow, int lane) {
  return (unsigned)(((lane % C::Cpr) ^ ((srow / C::Rpw) % C::Cpr)) * 16);
}

// The K loop for one tile: acc[rb][cb] += A rows (arow + 32 rb) x B rows
// brow[cb] over K (a multiple of BK); arow and brow[] are stage rows of
// this lane's fragments (B rows are offset by BM).
//
// Software pipeline over half-steps of 32 K (a stage holds BK / 32 of
// them; the fetch of step t is issued Stages steps ahead, into the stage
// whose fragments were just taken): half-step h: if h + 1 starts a new step
// t, wait for this wave's fetch of t, barrier (every wave's fetches of t
// landed, every read of step t - 1 done), fetch step t - 1 + Stages into the
// stage of t - 1; read half h + 1's fragments into the other register set;
// then the MFMAs of half h on fragments already in registers -- so the LDS
// reads of the next half overlap this half's MFMAs.
template <class C>
__device__ __forceinline__ void gemm_mainloop(char* lds, const FetchPlan<C>& fp, int K, int arow,
                                              const int (&brow)[C::CB],
                                              f32x16 (&acc)[C::RB][C::CB]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
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
      const int off = fp.off[j] == kGOob ? (int)kGOob : (int)(fp.off[j] + kb);
      g_fetch(sbase + ins * C::Rpi * C::RowB, off, fp.rs[j]);
    }
  };
  const int li = lane & 31, kh = lane >> 5;
  int koff[C::BK / 16];
#pragma unroll
  for (int s = 0; s < C::BK / 16; ++s) koff[s] = ((2 * s + kh) ^ ((li / C::Rpw) % C::Cpr)) * 16;

  constexpr int kHS = C::BK / 32;        // half-steps per stage
  const int nsteps = K / C::BK;
  const int nh = nsteps * kHS;
  bf16x8 fa[2][2][C::RB], fb[2][2][C::CB];
  auto read_half = [&](int h, bf16x8 (&a)[2][C::RB], bf16x8 (&b)[2][C::CB]) {
    const char* st = lds + ((h / kHS) % C::Stages) * C::StageB;
    const int sub0 = (h % kHS) * 2;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb)
        b[s][cb] = *reinterpret_cast<const bf16x8*>(st + brow[cb] * C::RowB + koff[sub0 + s]);
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
}

// Epilogue through LDS (after the K loop; the ring is free once every wave
// has passed the barrier at its start): each wave stages its RB*32 x CB*32
// sub-tile as bf16 rows in a private LDS region -- lanes 2j and 2j+1 swap
// one value each (DPP) so that every LDS write is a dword of two adjacent
// columns -- and then writes whole 16-byte row chunks (full 128-byte lines
// for CB = 2), 8x fewer store instructions than one per element.
// val(x, r) rounds accumulator x of tile row r to the stored bf16;
// row_ptr(r) is the destination of tile row r at the tile's first column
// (16-byte aligned), or nullptr for a row that is not stored; cols is the
// number of valid tile columns.
template <class C, class RowPtr, class Val>
__device__ __forceinline__ void gemm_store_tile_lds(char* lds, const f32x16 (&acc)[C::RB][C::CB],
                                                    int cols, RowPtr row_ptr, Val val) {
  constexpr int kRows = C::RB * 32, kCols = C::CB * 32, kPitch = kCols * 2;
  static_assert(C::Waves * kRows * kPitch <= C::Lds, "staging fits the ring");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave % C::WM, wn = wave / C::WM;
  const int li = lane & 31, kh = lane >> 5, odd = li & 1;
  const int r_base = kRows * wm, c_base = kCols * wn;
  char* base = lds + wave * kRows * kPitch;
  __syncthreads();
#pragma unroll
  for (int rb = 0; rb < C::RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < C::CB; ++cb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        // rows lr (value i) and lr + 1 (value i + 1) of column 32 cb + li
        const int lr = 32 * rb + 8 * (i >> 2) + 4 * kh + (i & 3);
        const unsigned a = __builtin_bit_cast(unsigned short, val(acc[rb][cb][i], r_base + lr));
        const unsigned b =
            __builtin_bit_cast(unsigned short, val(acc[rb][cb][i + 1], r_base + lr + 1));
        // even lane keeps row lr and takes its odd neighbour's value of that
        // row; odd lane keeps row lr + 1 and takes the even neighbour's
        const unsigned give = odd ? a : b;
        const unsigned got = (unsigned)__builtin_amdgcn_mov_dpp((int)give, 0xB1, 0xF, 0xF, false);
        const unsigned word = odd ? (got | (b << 16)) : (a | (got << 16));
        const int row = lr + odd, col = 32 * cb + li - odd;
        *reinterpret_cast<unsigned*>(base + row * kPitch + col * 2) = word;
      }
  // the wave reads back only its own region, so no barrier is needed
  constexpr int kChunks = kPitch / 16;            // 16-byte chunks per row
  constexpr int kRowsPer = 64 / kChunks;          // rows per read instruction
#pragma unroll
  for (int it = 0; it < kRows / kRowsPer; ++it) {
    const int lr = it * kRowsPer + lane / kChunks, ch = lane % kChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(base + lr * kPitch + ch * 16);
    bf16* yr = row_ptr(r_base + lr);
    const int c = c_base + 8 * ch;
    if (yr == nullptr) continue;
    if (c + 8 <= cols) {
      *reinterpret_cast<u32x4*>(yr + c) = v;
    } else {
      const bf16x8 e = __builtin_bit_cast(bf16x8, v);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (c + k < cols) yr[c + k] = e[k];
    }
  }
}

}  // namespace q36
