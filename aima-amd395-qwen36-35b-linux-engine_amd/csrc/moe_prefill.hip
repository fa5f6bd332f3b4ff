// MoE block of the Qwen3.6-35B-A3B layer for a batch of T tokens (prefill).
//
// Replaces the reference's native MoE prefill (native/src/
// native_moe_prefill.hip.cpp: router GEMM + router_topk8_softmax_256_kernel
// :234-323, moe_align_block32_256_kernel :325-382, the two AOT vLLM
// fused_moe_kernel expert GEMMs with expert_silu_multiply_kernel :384-402
// between them, the shared-expert GEMMs and pointwise kernels :210-232,
// moe_sum8_kernel :404-430 and the residual add), with the arithmetic of
// the eager text four_layer_mini_engine.py:8479-8650 (router :7775-7789,
// routed experts :7791-7803, shared expert :8240-8300) -- the same formulas
// as the one-token qwen36_moe_decode:
//   after = bf16(inp + attn);  h2 = bf16(rmsnorm(after) * (w + 1))
//   logits = bf16(h2 @ router^T);  ids = top-8;  rw = bf16(softmax(top-8))
//   [gate | up] = bf16(h2 @ gate_up_e^T);  act = bf16(silu(gate) * up)
//   y_k = bf16(bf16(act @ down_e^T) * rw_k)
//   shared: same expert form with the shared weights, scaled by
//           bf16(sigmoid(bf16(h2 . shared_gate)))
//   out = bf16(after + bf16(bf16(sum_k y_k) + shared))
//
// Launches (T tokens, E experts; the shared expert's rows are every token
// in order, so its two GEMMs need no routing and run on a side stream,
// forked after 1 and joined before 7, beside 2-4):
//  1. moe_pre_kernel       residual + RMSNorm, one wave per token.
//  2. moe_gemm<kRouter>    logits [T, E + 1] = h2 [router | shared_gate]^T;
//                          up to 8192 tokens in K slices whose fp32
//                          partials 3 sums.
//  3. moe_topk_kernel      top-8 + routing softmax + shared gate, a wave per token.
//  4. alignment            (token, rank) slots sorted by expert, each group
//                          padded to 32 rows and cut into tiles of up to 128
//                          rows: one workgroup up to 2048 tokens
//                          (moe_align_one), else per-chunk histograms, one
//                          scan workgroup and a per-chunk scatter.
//  5. moe_gemm<kGateUp>    act [tile rows, 512] = silu(gate) * up per tile,
//                          gate and up columns of one group in one workgroup
//                          (side stream: the shared expert's T rows).
//  6. moe_gemm<kDown>      y rows scaled by their routing weight, scattered to
//                          their (token, rank) slot (side stream: the shared
//                          rows, unscaled).
//  7. moe_combine_kernel   per token: sum of the 8 routed rows, + the shared
//                          row scaled by its gate, + after.
//
// Grouped GEMM: a workgroup computes one tile of up to 128 rows of one
// group against 256 weight rows, K in steps of 32, with 8 waves of 64 x 64 on
// v_mfma_f32_32x32x16_bf16 (one 16-byte LDS read per MFMA); 32-row blocks past
// the tile's rows are neither computed nor fetched.  Both operands are
// K-contiguous in memory, so they are fetched straight into LDS
// (buffer_load ... lds, 16 bytes per lane, 1 KiB per instruction) with an XOR
// swizzle of the 16-byte chunks chosen by each lane's source address, which
// makes the ds_read_b128 operand reads bank-conflict-free.  A 3-stage ring,
// two workgroups per CU; the fetch is issued through inline asm (the
// compiler would otherwise wait for it before reading the current stage) and
// ordered by explicit vmcnt waits + barriers.  Work items (tile, column block)
// are dealt to the 8 XCDs in contiguous ranges, so a tile's column blocks
// and an expert's tiles share an L2.  Measured on MI355X: the loop is bound
// by the L2/MALL -> LDS fill rate (~20-30 B/clk per CU), at ~87 flop per
// fetched byte for this tile; the tile shape was chosen from a sweep of
// 64..256-row x 128..256-column tiles, K steps of 32/64 and 2..4 stages.
#include "moe_common.h"

#include <algorithm>
#include <mutex>

namespace q36 {
namespace {

constexpr int kPfBM = 128;                // rows per tile (at most)
constexpr int kPfPad = 32;                // group padding (rows)
constexpr int kPfBN = 256;                // weight rows per workgroup
constexpr int kPfWR = 64;                 // rows per wave (32-row blocks: kPfWR / 32)
constexpr int kPfStages = 3;              // fetch ring depth
constexpr int kPfMinWG = 2;               // workgroups per CU the kernel is built for
constexpr int kPfBK = 32;                 // K per stage (32 or 64)
constexpr int kPfRowB = kPfBK * 2;        // bytes per row per stage
constexpr int kPfCpr = kPfRowB / 16;      // 16-byte chunks per row
constexpr int kPfRpi = 1024 / kPfRowB;    // rows per fetch instruction
constexpr int kPfRpw = 256 / kPfRowB;     // rows per 256-byte bank window
constexpr int kPfAStage = kPfBM * kPfRowB;
constexpr int kPfStage = kPfAStage + kPfBN * kPfRowB;
constexpr int kPfLds = kPfStages * kPfStage;
constexpr int kPfRB = kPfWR / 32;                        // row blocks per wave
constexpr int kPfWaves = (kPfBM / kPfWR) * (kPfBN / 64); // each wave: kPfWR x 64
constexpr int kPfInstr = (kPfBM + kPfBN) / kPfRpi / kPfWaves;  // fetch instructions per wave
static_assert((kPfBM + kPfBN) / kPfRpi % kPfWaves == 0, "fetch split");
static_assert(kPfBK == 32 || kPfBK == 64, "K step");
// Swizzle: chunk c of stage row r sits at position c ^ key(r), key(r) =
// (r / kPfRpw) % kPfCpr, so the 16 rows one ds_read_b128 pass serves fall in
// 16 distinct 16-byte bank groups of the 256-byte bank window.
constexpr unsigned kPfMaxTokens = 262144;
constexpr unsigned kAlignChunk = 4096;    // expert ids per histogram / scatter workgroup (least)
constexpr unsigned kMaxAlignChunks = 256;

enum GemmMode { kRouter = 0, kGateUp = 1, kDown = 2 };

// Workspace layout for (T, E); every region 256-byte aligned.  The first
// three regions (expert ids, routing weights, router logits) are read back by
// the host's debug path at these fixed offsets.
struct PfLayout {
  size_t ids, rw, logits, sgw, meta, sorted, hist, after, h2, act, y, act_shared, part, total;
  unsigned ld_logits, max_tiles, max_rows, n_chunks, chunk_ids, router_splits;
};

// K slices of the router GEMM: its T / 128 x 2 tiles leave most CUs idle
// at short prompts, each tile a chain of 64 K steps, so up to 8192 tokens
// the K range is cut into slices whose fp32 partials the top-8 kernel sums
// (MI355X, whole block: T = 1024 0.420 vs 0.431 ms with 4 slices, 8 and 16
// no better; T = 2048 0.473 vs 0.481 with 2; T = 8192 0.920 vs 0.925 with 2,
// 4 slices slower there).
unsigned router_splits(unsigned T) { return T <= 1024 ? 4u : T <= 8192 ? 2u : 1u; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

PfLayout pf_layout(unsigned T, unsigned E) {
  PfLayout L;
  L.ld_logits = (E + 1 + 7) & ~7u;
  L.max_tiles = (9u * T + kPfBM - 1) / kPfBM + E + 1;   // sum over groups of ceil(n / 128)
  L.max_rows = 9u * T + (kPfPad - 1) * (E + 1);         // sum of n rounded up to 32
  size_t o = 0;
  L.ids = o;     o = align256(o + (size_t)T * kMoeTopK * 4);
  L.rw = o;      o = align256(o + (size_t)T * kMoeTopK * 4);
  L.logits = o;  o = align256(o + (size_t)T * L.ld_logits * 2);
  L.sgw = o;     o = align256(o + (size_t)T * 4);
  L.meta = o;    o = align256(o + (size_t)(L.max_tiles + 1) * 16);
  L.sorted = o;  o = align256(o + (size_t)L.max_rows * 4);
  // at most kMaxAlignChunks chunks, each a multiple of 1024 ids
  L.n_chunks = std::min(kMaxAlignChunks, (kMoeTopK * T + kAlignChunk - 1) / kAlignChunk);
  L.chunk_ids = ((kMoeTopK * T + L.n_chunks - 1) / L.n_chunks + 1023) / 1024 * 1024;
  L.hist = o;    o = align256(o + (size_t)E * L.n_chunks * 4);
  L.after = o;   o = align256(o + (size_t)T * kMoeHidden * 2);
  L.h2 = o;      o = align256(o + (size_t)T * kMoeHidden * 2);
  L.act = o;     o = align256(o + (size_t)L.max_rows * kMoeInter * 2);
  L.y = o;       o = align256(o + (size_t)9 * T * kMoeHidden * 2);
  L.act_shared = o;  o = align256(o + (size_t)T * kMoeInter * 2);
  L.router_splits = router_splits(T);
  L.part = o;
  if (L.router_splits > 1) o = align256(o + (size_t)L.router_splits * T * L.ld_logits * 4);
  L.total = o;
  return L;
}

// ---- 1. residual + RMSNorm (arithmetic of moe_router_kernel) ---------------
__global__ __launch_bounds__(256) void moe_pre_kernel(
    const bf16* __restrict__ inp, const bf16* __restrict__ attn,
    const bf16* __restrict__ norm_w, bf16* __restrict__ after,
    bf16* __restrict__ h2, unsigned T) {
  const int lane = threadIdx.x & 63;
  const unsigned t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const size_t base = (size_t)t * kMoeHidden;
  float xa[4][8], ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(inp + base + 512 * j + 8 * lane);
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(attn + base + 512 * j + 8 * lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xa[j][e] = bf2f(f2bf(bf2f(a[e]) + bf2f(b[e])));
      ss = __builtin_fmaf(xa[j][e], xa[j][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float inv = (float)(1.0 / sqrt((double)(ss / (float)kMoeHidden + kMoeEps)));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 w = *reinterpret_cast<const bf16x8*>(norm_w + 512 * j + 8 * lane);
    bf16x8 oa, oh;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      oa[e] = f2bf(xa[j][e]);
      oh[e] = f2bf((xa[j][e] * inv) * (bf2f(w[e]) + 1.0f));
    }
    *reinterpret_cast<bf16x8*>(after + base + 512 * j + 8 * lane) = oa;
    *reinterpret_cast<bf16x8*>(h2 + base + 512 * j + 8 * lane) = oh;
  }
}

// ---- 3. top-8 + routing weights + shared gate, one wave per token ---------
// With `splits` > 1 the router GEMM left fp32 partials of its K slices
// (part [splits][T][ld]): the wave sums them in slice order, rounds to bf16
// and writes the logits row itself.
__global__ __launch_bounds__(256) void moe_topk_kernel(
    bf16* __restrict__ logits, const float* __restrict__ part, unsigned splits, unsigned ld,
    unsigned E, unsigned T, int* __restrict__ ids_out, float* __restrict__ rw_out,
    float* __restrict__ sgw) {
  const int lane = threadIdx.x & 63;
  const unsigned t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  bf16* row = logits + (size_t)t * ld;
  int ids[kMoeTopK];
  float vals[kMoeTopK], rw[kMoeTopK];
  float sg_logit;
  if (splits > 1) {
    // lane l: columns l + 64i, i < 5 (E + 1 <= 257 columns: experts + shared gate)
    float acc[5];
    for (unsigned k = 0; k < splits; ++k) {
      const float* pr = part + ((size_t)k * T + t) * ld;
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        const unsigned e = lane + 64 * i;
        const float x = pr[e <= E ? e : 0u];
        acc[i] = k == 0 ? x : acc[i] + x;   // slice 0 as is (keeps a -0 sum)
      }
    }
    unsigned short raw[4];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      const unsigned e = lane + 64 * i;
      const bf16 b = f2bf(acc[i]);
      if (e <= E) row[e] = b;
      if (i < 4) raw[i] = __builtin_bit_cast(unsigned short, b);
    }
    select_top8_bits(raw, E, ids, vals);
    // column E sits in lane E % 64, slot E / 64
    float v = acc[0];
#pragma unroll
    for (int i = 1; i < 5; ++i) v = (int)(E >> 6) == i ? acc[i] : v;
    sg_logit = bf2f(f2bf(__shfl(v, (int)(E & 63), 64)));
  } else {
    select_top8(row, E, ids, vals);
    sg_logit = bf2f(row[E]);
  }
  routing_weights(vals, rw);
  if (lane < kMoeTopK) {
    int id = ids[0];
    float w = rw[0];
#pragma unroll
    for (int k = 1; k < kMoeTopK; ++k) {
      id = lane == k ? ids[k] : id;
      w = lane == k ? rw[k] : w;
    }
    ids_out[(size_t)t * kMoeTopK + lane] = id;
    rw_out[(size_t)t * kMoeTopK + lane] = w;
  }
  if (lane == 0) sgw[t] = bf2f(f2bf(1.0f / (1.0f + expf(-sg_logit))));
}

// ---- 4. slots sorted by group, groups padded to 32 rows, 128-row tiles ----
// sorted[p] = slot (t * 8 + k for routed rank k of token t) or -1 for
// padding (the shared expert, every token, runs as launches of its own);
// group g occupies rows [row_off[g], row_off[g] + roundup32(n_g)).  meta
// (int4) [0] = {tiles}, [1 + i] = {group, first row, rows, 0} for tile i.
// The 8T ids are cut into chunks of kAlignChunk: hist[g][chunk] counts, the
// scan turns them into each chunk's first row per group, the scatter places
// the chunk's slots.  Order inside a
// group is arbitrary: every GEMM row is computed independently, so it does
// not affect any value.

// 4a. per-chunk expert histogram.
__global__ __launch_bounds__(256) void moe_hist_kernel(const int* __restrict__ ids, unsigned T,
                                                       unsigned E, unsigned n_chunks,
                                                       unsigned chunk_ids,
                                                       int* __restrict__ hist) {
  __shared__ int cnt[kMoeMaxExperts];
  const unsigned tid = threadIdx.x, routed4 = kMoeTopK * T / 4;
  for (unsigned g = tid; g < E; g += blockDim.x) cnt[g] = 0;
  __syncthreads();
  const int4* ids4 = reinterpret_cast<const int4*>(ids);   // 8T ids: whole int4s
  const unsigned i0 = blockIdx.x * (chunk_ids / 4), i1 = min(i0 + chunk_ids / 4, routed4);
  for (unsigned b = i0; b < i1; b += 4 * 256) {
    int4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const unsigned i = b + tid + 256 * u;
      v[u] = i < i1 ? ids4[i] : int4{-1, -1, -1, -1};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (v[u].x >= 0) {
        atomicAdd(&cnt[v[u].x], 1);
        atomicAdd(&cnt[v[u].y], 1);
        atomicAdd(&cnt[v[u].z], 1);
        atomicAdd(&cnt[v[u].w], 1);
      }
    }
  }
  __syncthreads();
  for (unsigned g = tid; g < E; g += blockDim.x) hist[(size_t)g * n_chunks + blockIdx.x] = cnt[g];
}

// From the group counts cnt[0, G): exclusive offsets of the padded rows and
// of the tiles (one wave's scans; [G] = totals), the tile table meta and
// the padding rows of `sorted` (-1).  Called by every thread of the
// workgroup; ends with the offsets visible to all of them.
__device__ __forceinline__ void group_offsets(const int* cnt, unsigned G, unsigned tid,
                                              int* row_off, int* tile_off,
                                              int4* __restrict__ meta,
                                              int* __restrict__ sorted) {
  if (tid < 64) {   // one wave: exclusive scans of padded rows and tiles per group
    constexpr int kPer = (kMoeMaxExperts + 1 + 63) / 64;   // 5 groups per lane
    int rows[kPer], tiles[kPer], rsum = 0, tsum = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const unsigned g = tid * kPer + j;
      const int c = g < G ? cnt[g] : 0;
      rows[j] = (c + kPfPad - 1) / kPfPad * kPfPad;
      tiles[j] = (c + kPfBM - 1) / kPfBM;
      rsum += rows[j];
      tsum += tiles[j];
    }
    int rincl = rsum, tincl = tsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int ru = __shfl_up(rincl, o, 64), tu = __shfl_up(tincl, o, 64);
      if ((int)tid >= o) {
        rincl += ru;
        tincl += tu;
      }
    }
    int roff = rincl - rsum, toff = tincl - tsum;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const unsigned g = tid * kPer + j;
      if (g <= G) {   // [G] = totals
        row_off[g] = roff;
        tile_off[g] = toff;
      }
      roff += rows[j];
      toff += tiles[j];
    }
    if (tid == 63) meta[0] = int4{tincl, 0, 0, 0};
  }
  __syncthreads();
  for (unsigned g = tid; g < G; g += blockDim.x) {
    const int c = cnt[g], r0 = row_off[g];
    for (int j = 0; j < tile_off[g + 1] - tile_off[g]; ++j)
      meta[1 + tile_off[g] + j] = int4{(int)g, r0 + kPfBM * j, min(kPfBM, c - kPfBM * j), 0};
    for (int p = r0 + c; p < row_off[g + 1]; ++p) sorted[p] = -1;
  }
}

// 4b. one workgroup: group totals, row / tile offsets (one-wave scans), tile
// table, padding, shared-expert rows, and hist turned into each chunk's
// first row per group.
__global__ __launch_bounds__(1024) void moe_scan_kernel(unsigned E, unsigned n_chunks,
                                                        int* __restrict__ hist,
                                                        int4* __restrict__ meta,
                                                        int* __restrict__ sorted) {
  __shared__ int cnt[kMoeMaxExperts + 1];
  __shared__ int row_off[kMoeMaxExperts + 2];
  __shared__ int tile_off[kMoeMaxExperts + 2];
  const unsigned G = E + 1, tid = threadIdx.x;
  // totals: 4 threads per group, each summing a quarter of the chunks
  {
    const unsigned g = tid >> 2, part = tid & 3;
    int sum = 0;
    if (g < E)
      for (unsigned c = part; c < n_chunks; c += 4) sum += hist[(size_t)g * n_chunks + c];
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if (g < E && part == 0) cnt[g] = sum;
    if (tid == 0) cnt[E] = 0;   // the shared expert runs as launches of its own
  }
  __syncthreads();
  group_offsets(cnt, G, tid, row_off, tile_off, meta, sorted);
  {   // chunk bases: one wave per group, exclusive prefix over the chunks
    const unsigned wave = tid >> 6, lane = tid & 63, waves = blockDim.x / 64;
    if (n_chunks <= 64) {   // every group's counts loaded up front (one round trip)
      constexpr int kGpw = (kMoeMaxExperts + 15) / 16;   // groups per wave (16 waves)
      int n[kGpw];
#pragma unroll
      for (int j = 0; j < kGpw; ++j) {
        const unsigned g = wave + waves * j;
        n[j] = (g < E && lane < n_chunks) ? hist[(size_t)g * n_chunks + lane] : 0;
      }
#pragma unroll
      for (int j = 0; j < kGpw; ++j) {
        const unsigned g = wave + waves * j;
        int incl = n[j];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int up = __shfl_up(incl, o, 64);
          if ((int)lane >= o) incl += up;
        }
        if (g < E && lane < n_chunks) hist[(size_t)g * n_chunks + lane] = row_off[g] + incl - n[j];
      }
    } else
    for (unsigned g = wave; g < E; g += waves) {
      int run = row_off[g];
      for (unsigned c0 = 0; c0 < n_chunks; c0 += 64) {
        const unsigned ch = c0 + lane;
        const int n = ch < n_chunks ? hist[(size_t)g * n_chunks + ch] : 0;
        int incl = n;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int up = __shfl_up(incl, o, 64);
          if ((int)lane >= o) incl += up;
        }
        if (ch < n_chunks) hist[(size_t)g * n_chunks + ch] = run + incl - n;
        run += __shfl(incl, 63, 64);
      }
    }
  }
}

// 4c. per-chunk scatter: slot i goes to its group's next row of this chunk.
__global__ __launch_bounds__(256) void moe_scatter_kernel(const int* __restrict__ ids, unsigned T,
                                                          unsigned E, unsigned n_chunks,
                                                          unsigned chunk_ids,
                                                          const int* __restrict__ base,
                                                          int* __restrict__ sorted) {
  __shared__ int pos[kMoeMaxExperts];
  const unsigned tid = threadIdx.x, routed4 = kMoeTopK * T / 4;
  for (unsigned g = tid; g < E; g += blockDim.x) pos[g] = base[(size_t)g * n_chunks + blockIdx.x];
  __syncthreads();
  const int4* ids4 = reinterpret_cast<const int4*>(ids);
  const unsigned i0 = blockIdx.x * (chunk_ids / 4), i1 = min(i0 + chunk_ids / 4, routed4);
  for (unsigned b = i0; b < i1; b += 4 * 256) {
    int4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const unsigned i = b + tid + 256 * u;
      v[u] = i < i1 ? ids4[i] : int4{-1, -1, -1, -1};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (v[u].x >= 0) {
        const int i = (int)(4 * (b + tid + 256 * u));
        sorted[atomicAdd(&pos[v[u].x], 1)] = i;
        sorted[atomicAdd(&pos[v[u].y], 1)] = i + 1;
        sorted[atomicAdd(&pos[v[u].z], 1)] = i + 2;
        sorted[atomicAdd(&pos[v[u].w], 1)] = i + 3;
      }
    }
  }
}

// 4'. short prompts (8T <= kAlignOneIds): histogram, offsets and scatter in
// one workgroup, the ids held in registers (16 per thread) -- one launch
// instead of 4a-4c.
constexpr unsigned kAlignOneIds = 16384;
__global__ __launch_bounds__(1024) void moe_align_one_kernel(const int* __restrict__ ids,
                                                             unsigned T, unsigned E,
                                                             int4* __restrict__ meta,
                                                             int* __restrict__ sorted) {
  __shared__ int cnt[kMoeMaxExperts + 1];
  __shared__ int row_off[kMoeMaxExperts + 2];
  __shared__ int tile_off[kMoeMaxExperts + 2];
  constexpr int kU = kAlignOneIds / 4 / 1024;
  const unsigned G = E + 1, tid = threadIdx.x, routed4 = kMoeTopK * T / 4;
  const int4* ids4 = reinterpret_cast<const int4*>(ids);
  int4 v[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const unsigned i = tid + 1024 * u;
    v[u] = i < routed4 ? ids4[i] : int4{-1, -1, -1, -1};
  }
  for (unsigned g = tid; g < G; g += blockDim.x) cnt[g] = 0;   // [E]: shared expert, no rows
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    if (v[u].x >= 0) {
      atomicAdd(&cnt[v[u].x], 1);
      atomicAdd(&cnt[v[u].y], 1);
      atomicAdd(&cnt[v[u].z], 1);
      atomicAdd(&cnt[v[u].w], 1);
    }
  }
  __syncthreads();
  group_offsets(cnt, G, tid, row_off, tile_off, meta, sorted);
  __syncthreads();
  for (unsigned g = tid; g < G; g += blockDim.x) cnt[g] = row_off[g];   // next row per group
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    if (v[u].x >= 0) {
      const int i = (int)(4 * (tid + 1024 * u));
      sorted[atomicAdd(&cnt[v[u].x], 1)] = i;
      sorted[atomicAdd(&cnt[v[u].y], 1)] = i + 1;
      sorted[atomicAdd(&cnt[v[u].z], 1)] = i + 2;
      sorted[atomicAdd(&cnt[v[u].w], 1)] = i + 3;
    }
  }
}

// ---- 2/5/6. grouped GEMM ----------------------------------------------------
struct GemmArgs {
  const bf16* a;            // h2 [T, 2048] (router, gate/up) or act [rows, 512] (down)
  const bf16* w;            // router: w_in; gate/up: expert_gate_up; down: expert_down
  const bf16* w_shared;     // gate/up: shared [gate_proj | up_proj]; down: shared_down
  const int4* meta;
  const int* sorted;
  const float* rw;
  const float* sgw;
  bf16* out;                // logits / act / y
  float* part;              // router with K slices: fp32 partials [slices][T][ld_out]
  unsigned T, E, ld_out, max_items;
  unsigned shared;          // gate/up, down: the shared expert's T rows in token order
};

// The leading s_nop covers a hazard the compiler cannot see through the
// inline assembly: the resource SGPRs (and m0) are written by VALU
// readfirstlane / SALU instructions right before, and a VMEM instruction
// reading an SGPR that a VALU wrote needs 5 wait states on gfx950 (issued
// earlier, it reads the old descriptor).
__device__ __forceinline__ void fetch_rows(unsigned lds_addr, int voff, const u32x4& rsrc) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  return u32x4{(unsigned)a, (unsigned)(a >> 32), bytes, 0x00020000u};
}

constexpr unsigned kOob = 0x80000000u;   // a row offset past every buffer's range

template <int MODE>
__host__ __device__ constexpr unsigned n_blocks(unsigned E) {
  return MODE == kRouter ? (E + 1 + kPfBN - 1) / kPfBN
                         : (MODE == kGateUp ? kMoeInter / (kPfBN / 2) : kMoeHidden / kPfBN);
}

// s_waitcnt immediate that waits until at most n vector-memory operations of
// this wave are outstanding (expcnt and lgkmcnt not waited on).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// The K loop for a wave computing NRB (0..kPfRB) row blocks of 32.  Every
// wave fetches and meets the barriers whatever its NRB.  Stage s of the ring
// holds K step s mod kPfStages; the fetch of step + kPfStages - 1 is issued
// once every wave has finished reading step - 1.
template <int NRB, int NSTEPS, typename Fetch>
__device__ __forceinline__ void gemm_k_loop(Fetch& fetch, const char* lds, int arow, int brow0,
                                            int brow1, const int (&koff)[kPfBK / 16],
                                            f32x16 (&acc)[kPfRB][2]) {
#pragma unroll
  for (int st = 0; st < kPfStages - 1; ++st) fetch(st);
  for (int step = 0; step < NSTEPS; ++step) {
    // this wave's fetches of `step` landed (later ones may stay in flight)
    if (step + kPfStages - 2 < NSTEPS)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((kPfStages - 2) * kPfInstr));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();   // every wave's fetches landed; stage (step - 1) is free
    if (step + kPfStages - 1 < NSTEPS) fetch(step + kPfStages - 1);
    if constexpr (NRB > 0) {
      const char* st = lds + (step % kPfStages) * kPfStage;
#pragma unroll
      for (int s = 0; s < kPfBK / 16; ++s) {
        const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(st + brow0 * kPfRowB + koff[s]);
        const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(st + brow1 * kPfRowB + koff[s]);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(
              st + (arow + 32 * rb) * kPfRowB + koff[s]);
          acc[rb][0] = mfma32x32x16(a, b0, acc[rb][0]);
          acc[rb][1] = mfma32x32x16(a, b1, acc[rb][1]);
        }
      }
    }
  }
}

// Wave (wm = w % (BM / WR), wn = w / (BM / WR)) computes tile rows
// WR wm + 32 rb against weight rows (gate/up: gate 32wn.. and up BN/2 +
// 32wn.., i.e. act columns 32wn..; else 64wn.. and 64wn + 32..).  Fetch
// instruction i (of (BM + BN) / 8) moves rows 8i..8i+7 of the stage: A rows
// first, then B rows; wave w issues instructions w * kPfInstr + j.
// KS > 1 (router only): item i covers K slice i % KS of tile i / KS.
template <int MODE, int KS = 1>
__global__ __launch_bounds__(64 * kPfWaves, kPfMinWG) void moe_gemm_kernel(GemmArgs p) {
  static_assert(KS == 1 || MODE == kRouter, "K slices are for the router");
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int K = MODE == kDown ? kMoeInter : kMoeHidden;
  constexpr int nsteps = K / kPfBK / KS;
  static_assert(nsteps * kPfBK * KS == K, "K slices");
  const unsigned nb = n_blocks<MODE>(p.E);
  const unsigned m_tiles = (MODE == kRouter || p.shared) ? (p.T + kPfBM - 1) / kPfBM
                                                          : (unsigned)p.meta[0].x;
  const unsigned items = m_tiles * nb * KS;
  const unsigned share = (items + 7) / 8;
  const unsigned xi = blockIdx.x >> 3;
  if (xi >= share) return;
  const unsigned item = (blockIdx.x & 7) * share + xi;
  if (item >= items) return;
  const unsigned ks = item % KS;
  const unsigned mt = item / KS / nb, nt = item / KS % nb;
  int group = 0, row0, rows;
  if (MODE == kRouter || p.shared) {
    group = MODE == kRouter ? 0 : (int)p.E;
    row0 = (int)(mt * kPfBM);
    rows = min(kPfBM, (int)p.T - row0);
  } else {
    const int4 m = p.meta[1 + mt];
    group = m.x;
    row0 = m.y;
    rows = m.z;
  }

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  // Operand sources (buffer resources: out-of-range rows read as zero).
  u32x4 ars, brs;
  if constexpr (MODE == kDown)
    ars = buffer_rsrc(p.a + (size_t)row0 * kMoeInter, (unsigned)rows * kMoeInter * 2u);
  else
    ars = buffer_rsrc(p.a, p.T * (unsigned)kMoeHidden * 2u);
  if constexpr (MODE == kRouter) {
    brs = buffer_rsrc(p.w, (p.E + 1) * (unsigned)kMoeHidden * 2u);
  } else if constexpr (MODE == kGateUp) {
    const bf16* wg = group < (int)p.E ? p.w + (size_t)group * (2 * kMoeInter) * kMoeHidden
                                      : p.w_shared;
    brs = buffer_rsrc(wg, 2u * kMoeInter * kMoeHidden * 2u);
  } else {
    const bf16* wg = group < (int)p.E ? p.w + (size_t)group * kMoeHidden * kMoeInter
                                      : p.w_shared;
    brs = buffer_rsrc(wg, (unsigned)kMoeHidden * kMoeInter * 2u);
  }

  // Fetch plan: one instruction moves 1 KiB, kPfRpi rows of kPfRowB bytes
  // (lane = row in the instruction x chunk position; the source chunk is
  // position ^ key(row), so LDS holds the swizzled layout).  A instructions
  // whose rows are all past the tile's rows load nothing (an out-of-range
  // offset), which keeps every wave's count of loads per stage equal.
  const int rin = lane / kPfCpr, cpos = lane % kPfCpr;   // row in the instruction, chunk
  unsigned f_off[kPfInstr];
  u32x4 f_rs[kPfInstr];
  bool f_live[kPfInstr];
#pragma unroll
  for (int j = 0; j < kPfInstr; ++j) {
    const int ins = wave * kPfInstr + j;
    const bool is_a = ins < kPfBM / kPfRpi;
    unsigned off;
    if (is_a) {
      const int r = ins * kPfRpi + rin;
      if constexpr (MODE == kRouter) {
        off = r < rows ? (unsigned)(row0 + r) * kMoeHidden * 2u : kOob;
      } else if constexpr (MODE == kGateUp) {
        const int slot = r >= rows ? -1
                         : p.shared ? (int)(kMoeTopK * p.T) + row0 + r : p.sorted[row0 + r];
        const unsigned routed = kMoeTopK * p.T;
        const unsigned t = slot < 0 ? 0u : ((unsigned)slot < routed ? (unsigned)slot / kMoeTopK
                                                                    : (unsigned)slot - routed);
        off = slot < 0 ? kOob : t * (unsigned)kMoeHidden * 2u;
      } else {
        off = (unsigned)r * kMoeInter * 2u;
      }
    } else {
      const int r = (ins - kPfBM / kPfRpi) * kPfRpi + rin;
      unsigned row;
      if constexpr (MODE == kGateUp)
        row = r < kPfBN / 2 ? nt * (kPfBN / 2) + r : kMoeInter + nt * (kPfBN / 2) + (r - kPfBN / 2);
      else
        row = nt * kPfBN + r;
      off = row * (unsigned)K * 2u;
    }
    const int srow = ins * kPfRpi + rin;   // stage row this lane fills
    f_off[j] = off + ((cpos ^ ((srow / kPfRpw) % kPfCpr)) * 16);
    f_live[j] = !is_a || ins * kPfRpi < rows;
    const u32x4 r = is_a ? ars : brs;
#pragma unroll
    for (int c = 0; c < 4; ++c) f_rs[j][c] = __builtin_amdgcn_readfirstlane(r[c]);
  }
  const unsigned lds0 = static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds));
  auto fetch = [&](int step) {
    const unsigned sbase = lds0 + (step % kPfStages) * kPfStage;
    const unsigned kb = (ks * nsteps + (unsigned)step) * kPfRowB;
#pragma unroll
    for (int j = 0; j < kPfInstr; ++j) {
      // a dead instruction is still issued, with an out-of-range offset (no
      // memory is read), so every wave keeps the same count of outstanding
      // loads per stage for the vmcnt waits
      const int ins = wave * kPfInstr + j;
      fetch_rows(sbase + ins * kPfRpi * kPfRowB, f_live[j] ? (int)(f_off[j] + kb) : (int)kOob,
                 f_rs[j]);
    }
  };

  constexpr int kWm = kPfBM / kPfWR;
  const int wm = wave % kWm, wn = wave / kWm;
  const int li = lane & 31, kh = lane >> 5;
  const int arow = kPfWR * wm + li;
  const int brow0 = kPfBM + (MODE == kGateUp ? 32 * wn + li : 64 * wn + li);
  const int brow1 = kPfBM + (MODE == kGateUp ? kPfBN / 2 + 32 * wn + li : 64 * wn + 32 + li);
  int koff[kPfBK / 16];
#pragma unroll
  for (int s = 0; s < kPfBK / 16; ++s) koff[s] = (((2 * s + kh) ^ ((li / kPfRpw) % kPfCpr)) * 16);
  const int nrb = min(kPfRB, max(0, (rows - kPfWR * wm + 31) / 32));

  f32x16 acc[kPfRB][2];
#pragma unroll
  for (int i = 0; i < kPfRB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  if (nrb == 0) {
    gemm_k_loop<0, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc);
  } else if constexpr (kPfRB == 1) {
    gemm_k_loop<1, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc);
  } else if constexpr (kPfRB == 2) {
    if (nrb == 1) gemm_k_loop<1, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc);
    else gemm_k_loop<2, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc);
  } else {
    switch (nrb) {
      case 1: gemm_k_loop<1, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc); break;
      case 2: gemm_k_loop<2, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc); break;
      case 3: gemm_k_loop<3, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc); break;
      default: gemm_k_loop<kPfRB, nsteps>(fetch, lds, arow, brow0, brow1, koff, acc); break;
    }
  }

  // acc[rb][cb][i] = tile row WR wm + 32rb + 8(i/4) + 4kh + i%4, weight row
  // brow_cb.
  const unsigned routed = kMoeTopK * p.T;
#pragma unroll
  for (int rb = 0; rb < kPfRB; ++rb) {
    if (rb >= nrb) break;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = kPfWR * wm + 32 * rb + 8 * (i >> 2) + 4 * kh + (i & 3);
      if (r >= rows) continue;
      if constexpr (MODE == kRouter && KS > 1) {
        const unsigned n = nt * kPfBN + 64 * wn + li;
        float* o = p.part + ((size_t)ks * p.T + row0 + r) * p.ld_out;
        if (n <= p.E) o[n] = acc[rb][0][i];
        if (n + 32 <= p.E) o[n + 32] = acc[rb][1][i];
      } else if constexpr (MODE == kRouter) {
        const unsigned n = nt * kPfBN + 64 * wn + li;
        bf16* o = p.out + (size_t)(row0 + r) * p.ld_out;
        if (n <= p.E) o[n] = f2bf(acc[rb][0][i]);
        if (n + 32 <= p.E) o[n + 32] = f2bf(acc[rb][1][i]);
      } else if constexpr (MODE == kGateUp) {
        const unsigned c = nt * (kPfBN / 2) + 32 * wn + li;
        const float g = bf2f(f2bf(acc[rb][0][i])), u = bf2f(f2bf(acc[rb][1][i]));
        p.out[(size_t)(row0 + r) * kMoeInter + c] = f2bf(silu_f(g) * u);
      } else if (p.shared) {
        // the shared expert's row, unscaled: the combine applies the shared
        // gate (known only after the router) with this epilogue's roundings
        bf16* y = p.out + (size_t)(routed + row0 + r) * kMoeHidden + nt * kPfBN + 64 * wn + li;
        y[0] = f2bf(acc[rb][0][i]);
        y[32] = f2bf(acc[rb][1][i]);
      } else {
        const int slot = p.sorted[row0 + r];
        const float w = p.rw[slot];
        bf16* y = p.out + (size_t)slot * kMoeHidden + nt * kPfBN + 64 * wn + li;
        y[0] = f2bf(bf2f(f2bf(acc[rb][0][i])) * w);
        y[32] = f2bf(bf2f(f2bf(acc[rb][1][i])) * w);
      }
    }
  }
}

// ---- 7. per-token combine --------------------------------------------------
// moe = bf16(sum over ranks 0..7 of y, fp32 in rank order); out = bf16(after +
// bf16(moe + shared)) -- the order of qwen36_moe_decode's combine.
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const bf16* __restrict__ y, const bf16* __restrict__ after, const float* __restrict__ sgw,
    bf16* __restrict__ out, unsigned T) {
  const unsigned t = blockIdx.x;
  const int c = 8 * threadIdx.x;
  float moe[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  bf16x8 yk[kMoeTopK];
#pragma unroll
  for (int k = 0; k < kMoeTopK; ++k)
    yk[k] = *reinterpret_cast<const bf16x8*>(y + ((size_t)t * kMoeTopK + k) * kMoeHidden + c);
  const bf16x8 ys = *reinterpret_cast<const bf16x8*>(
      y + ((size_t)kMoeTopK * T + t) * kMoeHidden + c);
  const bf16x8 af = *reinterpret_cast<const bf16x8*>(after + (size_t)t * kMoeHidden + c);
  const float sg = sgw[t];
#pragma unroll
  for (int k = 0; k < kMoeTopK; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) moe[e] += bf2f(yk[k][e]);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float shared = bf2f(f2bf(bf2f(ys[e]) * sg));   // the shared row scaled by its gate
    const float total = bf2f(f2bf(bf2f(f2bf(moe[e])) + shared));
    o[e] = f2bf(bf2f(af[e]) + total);
  }
  *reinterpret_cast<bf16x8*>(out + (size_t)t * kMoeHidden + c) = o;
}

// The shared expert depends only on the normalised rows (its gate is applied
// in the combine), so its two GEMMs run on a side stream while the router,
// top-8 and alignment chain -- a few latency-bound launches that leave most
// CUs idle -- runs on the caller's stream, and the routed GEMMs then hold
// only the routed tiles.  One side stream and a fork / join event pair per
// device, created on first use; the mutex keeps each call's record / wait
// pairs together when several host threads enqueue at once.  If they cannot
// be created, everything runs on the caller's stream.
constexpr int kPfMaxDevices = 64;
struct SideStream {
  bool tried = false;
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mutex;
SideStream g_side[kPfMaxDevices];

}  // namespace
}  // namespace q36

using namespace q36;

// Workspace bytes of qwen36_moe_prefill for `tokens` tokens and `n_experts`
// experts (0 for invalid arguments).
Q36_EXPORT size_t qwen36_moe_prefill_workspace_bytes(unsigned tokens, unsigned n_experts) {
  if (tokens == 0 || tokens > kPfMaxTokens || n_experts < (unsigned)kMoeTopK ||
      n_experts > (unsigned)kMoeMaxExperts || (n_experts % 4) != 0)
    return 0;
  return pf_layout(tokens, n_experts).total;
}

// MoE block for T = `tokens` rows: out [T, 2048] = after + moe + shared with
// after = inp + attn_out (all bf16, row-major, 16-byte aligned).  Weights as
// in qwen36_moe_decode: w_in [E + 1 + 1024, 2048] = [router | shared_gate |
// shared gate_proj | shared up_proj], expert_gate_up [E, 1024, 2048],
// expert_down [E, 2048, 512], shared_down [2048, 512].  The workspace starts
// with the expert ids (int32 [T, 8]), the routing weights (fp32 [T, 8], bf16
// values) and the router logits (bf16 [T, ld], ld = (E + 8) & ~7, column E =
// the shared gate) at 256-byte-aligned offsets.
Q36_EXPORT int qwen36_moe_prefill(const void* inp, const void* attn_out, const void* post_norm_w,
                                  const void* w_in, const void* expert_gate_up,
                                  const void* expert_down, const void* shared_down,
                                  unsigned n_experts, unsigned tokens, void* out,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  const size_t need = qwen36_moe_prefill_workspace_bytes(tokens, n_experts);
  if (need == 0 || inp == nullptr || attn_out == nullptr || post_norm_w == nullptr ||
      w_in == nullptr || expert_gate_up == nullptr || expert_down == nullptr ||
      shared_down == nullptr || out == nullptr || workspace == nullptr ||
      workspace_bytes < need || !aligned16(inp) || !aligned16(attn_out) ||
      !aligned16(post_norm_w) || !aligned16(w_in) || !aligned16(expert_gate_up) ||
      !aligned16(expert_down) || !aligned16(shared_down) || !aligned16(out) ||
      !aligned16(workspace))
    return Q36_EINVAL;
  const unsigned T = tokens, E = n_experts;
  static std::once_flag attr_once;   // 80 KiB of dynamic LDS per GEMM workgroup
  static hipError_t attr_status = hipSuccess;
  std::call_once(attr_once, [] {
    for (const void* f : {reinterpret_cast<const void*>(moe_gemm_kernel<kRouter>),
                          reinterpret_cast<const void*>(moe_gemm_kernel<kRouter, 2>),
                          reinterpret_cast<const void*>(moe_gemm_kernel<kRouter, 4>),
                          reinterpret_cast<const void*>(moe_gemm_kernel<kGateUp>),
                          reinterpret_cast<const void*>(moe_gemm_kernel<kDown>)}) {
      const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kPfLds);
      if (e != hipSuccess) attr_status = e;
    }
  });
  if (attr_status != hipSuccess) return (int)attr_status;
  const PfLayout L = pf_layout(T, E);
  char* ws = static_cast<char*>(workspace);
  int* ids = reinterpret_cast<int*>(ws + L.ids);
  float* rw = reinterpret_cast<float*>(ws + L.rw);
  bf16* logits = reinterpret_cast<bf16*>(ws + L.logits);
  float* sgw = reinterpret_cast<float*>(ws + L.sgw);
  int4* meta = reinterpret_cast<int4*>(ws + L.meta);
  int* sorted = reinterpret_cast<int*>(ws + L.sorted);
  bf16* after = reinterpret_cast<bf16*>(ws + L.after);
  bf16* h2 = reinterpret_cast<bf16*>(ws + L.h2);
  bf16* act = reinterpret_cast<bf16*>(ws + L.act);
  bf16* y = reinterpret_cast<bf16*>(ws + L.y);
  const bf16* win = static_cast<const bf16*>(w_in);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned tok_blocks = (T + 3) / 4;

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kPfMaxDevices) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(g_side_mutex);
  SideStream& side = g_side[dev];
  if (!side.tried) {
    side.tried = true;
    if (hipStreamCreateWithFlags(&side.s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&side.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&side.join, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      side.s = nullptr;
    }
  }
  hipStream_t ss = side.s != nullptr ? side.s : st;

  hipLaunchKernelGGL(moe_pre_kernel, dim3(tok_blocks), dim3(256), 0, st,
                     static_cast<const bf16*>(inp), static_cast<const bf16*>(attn_out),
                     static_cast<const bf16*>(post_norm_w), after, h2, T);

  GemmArgs g{};
  g.T = T;
  g.E = E;
  g.meta = meta;
  g.sorted = sorted;
  g.rw = rw;
  g.sgw = sgw;
  auto grid_for = [](unsigned max_items) { return dim3(8 * ((max_items + 7) / 8)); };

  // shared expert: gate/up then down (unscaled rows into its y slots) on
  // the side stream
  if (ss != st) {
    if (hipEventRecord(side.fork, st) != hipSuccess || hipStreamWaitEvent(ss, side.fork, 0) != hipSuccess)
      return static_cast<int>(hipGetLastError());
  }
  bf16* act_shared = reinterpret_cast<bf16*>(ws + L.act_shared);
  const unsigned shared_items = (T + kPfBM - 1) / kPfBM;
  GemmArgs gs = g;
  gs.shared = 1;
  gs.a = h2;
  gs.w = static_cast<const bf16*>(expert_gate_up);
  gs.w_shared = win + (size_t)(E + 1) * kMoeHidden;
  gs.out = act_shared;
  gs.max_items = shared_items * n_blocks<kGateUp>(E);
  hipLaunchKernelGGL(moe_gemm_kernel<kGateUp>, grid_for(gs.max_items), dim3(64 * kPfWaves), kPfLds, ss, gs);
  gs.a = act_shared;
  gs.w = static_cast<const bf16*>(expert_down);
  gs.w_shared = static_cast<const bf16*>(shared_down);
  gs.out = y;
  gs.max_items = shared_items * n_blocks<kDown>(E);
  hipLaunchKernelGGL(moe_gemm_kernel<kDown>, grid_for(gs.max_items), dim3(64 * kPfWaves), kPfLds, ss, gs);
  if (ss != st && hipEventRecord(side.join, ss) != hipSuccess) return static_cast<int>(hipGetLastError());

  g.a = h2;
  g.w = win;
  g.out = logits;
  g.ld_out = L.ld_logits;
  g.part = reinterpret_cast<float*>(ws + L.part);
  const unsigned router_items = ((T + kPfBM - 1) / kPfBM) * n_blocks<kRouter>(E) * L.router_splits;
  g.max_items = router_items;
  auto router = L.router_splits == 4   ? moe_gemm_kernel<kRouter, 4>
                : L.router_splits == 2 ? moe_gemm_kernel<kRouter, 2>
                                       : moe_gemm_kernel<kRouter>;
  hipLaunchKernelGGL(router, grid_for(router_items), dim3(64 * kPfWaves), kPfLds, st, g);

  hipLaunchKernelGGL(moe_topk_kernel, dim3(tok_blocks), dim3(256), 0, st, logits, g.part,
                     L.router_splits, L.ld_logits, E, T, ids, rw, sgw);
  if (kMoeTopK * T <= kAlignOneIds) {
    hipLaunchKernelGGL(moe_align_one_kernel, dim3(1), dim3(1024), 0, st, ids, T, E, meta, sorted);
  } else {
    int* hist = reinterpret_cast<int*>(ws + L.hist);
    hipLaunchKernelGGL(moe_hist_kernel, dim3(L.n_chunks), dim3(256), 0, st, ids, T, E,
                       L.n_chunks, L.chunk_ids, hist);
    hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(1024), 0, st, E, L.n_chunks, hist, meta,
                       sorted);
    hipLaunchKernelGGL(moe_scatter_kernel, dim3(L.n_chunks), dim3(256), 0, st, ids, T, E,
                       L.n_chunks, L.chunk_ids, hist, sorted);
  }

  g.a = h2;
  g.w = static_cast<const bf16*>(expert_gate_up);
  g.w_shared = win + (size_t)(E + 1) * kMoeHidden;
  g.out = act;
  g.max_items = L.max_tiles * n_blocks<kGateUp>(E);
  hipLaunchKernelGGL(moe_gemm_kernel<kGateUp>, grid_for(g.max_items), dim3(64 * kPfWaves), kPfLds, st, g);

  g.a = act;
  g.w = static_cast<const bf16*>(expert_down);
  g.w_shared = static_cast<const bf16*>(shared_down);
  g.out = y;
  g.max_items = L.max_tiles * n_blocks<kDown>(E);
  hipLaunchKernelGGL(moe_gemm_kernel<kDown>, grid_for(g.max_items), dim3(64 * kPfWaves), kPfLds, st, g);

  if (ss != st && hipStreamWaitEvent(st, side.join, 0) != hipSuccess)
    return static_cast<int>(hipGetLastError());
  hipLaunchKernelGGL(moe_combine_kernel, dim3(T), dim3(256), 0, st, y, after, sgw,
                     static_cast<bf16*>(out), T);
  return static_cast<int>(hipGetLastError());
}
