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
// Launches (T tokens, E experts, G = E + 1 groups: the shared expert is group
// E, holding every token, so it rides the same grouped GEMMs):
//  1. moe_pre_kernel       residual + RMSNorm, one wave per token.
//  2. moe_gemm<kRouter>    logits [T, E + 1] = h2 [router | shared_gate]^T.
//  3. moe_topk_kernel      top-8 + routing softmax + shared gate, a wave per token.
//  4. moe_align_kernel     (token, rank) slots sorted by expert, each group
//                          padded to 64-row tiles; one workgroup.
//  5. moe_gemm<kGateUp>    act [tile rows, 512] = silu(gate) * up per tile,
//                          gate and up columns of one group in one workgroup.
//  6. moe_gemm<kDown>      y rows scaled by their routing weight, scattered to
//                          their (token, rank) slot.
//  7. moe_combine_kernel   per token: sum of the 8 routed rows, + shared, +
//                          after.
//
// Grouped GEMM (MFMA-bound at large T; HBM-bound on the expert weights at
// small T): workgroup tile 64 rows x 128 weight rows x 64 of K, 4 waves of
// 32 x 64 on v_mfma_f32_32x32x16_bf16.  Both operands are K-contiguous in
// memory, so tiles are fetched straight into LDS (buffer_load ... lds, 16
// bytes per lane, 8 rows of 128 bytes per instruction) with an XOR swizzle
// of the 16-byte chunks (chunk c of row r sits at c ^ (r & 7)) chosen by each
// lane's source address, which makes the ds_read_b128 operand reads
// conflict-free.  Double-buffered: the next K step's fetch is in flight
// during the current step's MFMAs.  Work items (tile, column block) are dealt
// to the 8 XCDs in contiguous ranges, so the tiles of one expert share an L2.
#include "moe_common.h"

namespace q36 {
namespace {

constexpr int kPfBM = 64;                 // rows per tile
constexpr int kPfBN = 128;                // weight rows per workgroup
constexpr int kPfBK = 64;                 // K per step (128 bytes per row)
constexpr int kPfRowB = kPfBK * 2;        // 128
constexpr int kPfAStage = kPfBM * kPfRowB;        // 8192
constexpr int kPfStage = kPfAStage + kPfBN * kPfRowB;   // 24576
constexpr unsigned kPfMaxTokens = 262144;

enum GemmMode { kRouter = 0, kGateUp = 1, kDown = 2 };

// Workspace layout for (T, E); every region 256-byte aligned.  The first
// three regions (expert ids, routing weights, router logits) are read back by
// the host's debug path at these fixed offsets.
struct PfLayout {
  size_t ids, rw, logits, sgw, meta, sorted, after, h2, act, y, total;
  unsigned ld_logits, max_tiles;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

PfLayout pf_layout(unsigned T, unsigned E) {
  PfLayout L;
  L.ld_logits = (E + 1 + 7) & ~7u;
  L.max_tiles = (9u * T + kPfBM - 1) / kPfBM + E + 1;
  size_t o = 0;
  L.ids = o;     o = align256(o + (size_t)T * kMoeTopK * 4);
  L.rw = o;      o = align256(o + (size_t)T * kMoeTopK * 4);
  L.logits = o;  o = align256(o + (size_t)T * L.ld_logits * 2);
  L.sgw = o;     o = align256(o + (size_t)T * 4);
  L.meta = o;    o = align256(o + (size_t)(L.max_tiles + 1) * 4);
  L.sorted = o;  o = align256(o + (size_t)L.max_tiles * kPfBM * 4);
  L.after = o;   o = align256(o + (size_t)T * kMoeHidden * 2);
  L.h2 = o;      o = align256(o + (size_t)T * kMoeHidden * 2);
  L.act = o;     o = align256(o + (size_t)L.max_tiles * kPfBM * kMoeInter * 2);
  L.y = o;       o = align256(o + (size_t)9 * T * kMoeHidden * 2);
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
__global__ __launch_bounds__(256) void moe_topk_kernel(
    const bf16* __restrict__ logits, unsigned ld, unsigned E, unsigned T,
    int* __restrict__ ids_out, float* __restrict__ rw_out, float* __restrict__ sgw) {
  const int lane = threadIdx.x & 63;
  const unsigned t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const bf16* row = logits + (size_t)t * ld;
  int ids[kMoeTopK];
  float vals[kMoeTopK], rw[kMoeTopK];
  select_top8(row, E, ids, vals);
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
  if (lane == 0) sgw[t] = bf2f(f2bf(1.0f / (1.0f + expf(-bf2f(row[E])))));
}

// ---- 4. slots sorted by group, each group padded to 64-row tiles ----------
// meta[0] = number of tiles, meta[1 + i] = group of tile i; sorted[p] = slot
// (t * 8 + k for routed rank k of token t, 8T + t for the shared expert) or
// -1 for padding.  Order inside a group is arbitrary: every row of the GEMMs
// is computed independently, so it does not affect any value.
__global__ __launch_bounds__(1024) void moe_align_kernel(
    const int* __restrict__ ids, unsigned T, unsigned E, int* __restrict__ meta,
    int* __restrict__ sorted) {
  __shared__ int cnt[kMoeMaxExperts + 1];
  __shared__ int tile_off[kMoeMaxExperts + 2];
  __shared__ int wpos[kMoeMaxExperts + 1];
  const unsigned G = E + 1, tid = threadIdx.x, routed = kMoeTopK * T;
  for (unsigned g = tid; g < G; g += blockDim.x) cnt[g] = 0;
  __syncthreads();
  for (unsigned i = tid; i < routed; i += blockDim.x) atomicAdd(&cnt[ids[i]], 1);
  __syncthreads();
  if (tid == 0) {
    cnt[E] = (int)T;
    tile_off[0] = 0;
    for (unsigned g = 0; g < G; ++g) tile_off[g + 1] = tile_off[g] + (cnt[g] + kPfBM - 1) / kPfBM;
    meta[0] = tile_off[G];
  }
  __syncthreads();
  for (unsigned g = tid; g < G; g += blockDim.x) {
    wpos[g] = tile_off[g] * kPfBM;
    for (int i = tile_off[g]; i < tile_off[g + 1]; ++i) meta[1 + i] = (int)g;
    for (int p = tile_off[g] * kPfBM + cnt[g]; p < tile_off[g + 1] * kPfBM; ++p) sorted[p] = -1;
  }
  __syncthreads();
  for (unsigned i = tid; i < routed; i += blockDim.x) {
    const int p = atomicAdd(&wpos[ids[i]], 1);
    sorted[p] = (int)i;
  }
  const int shared0 = tile_off[E] * kPfBM;
  for (unsigned t = tid; t < T; t += blockDim.x) sorted[shared0 + t] = (int)(routed + t);
}

// ---- 2/5/6. grouped GEMM ----------------------------------------------------
struct GemmArgs {
  const bf16* a;            // h2 [T, 2048] (router, gate/up) or act [tiles*64, 512] (down)
  const bf16* w;            // router: w_in; gate/up: expert_gate_up; down: expert_down
  const bf16* w_shared;     // gate/up: shared [gate_proj | up_proj]; down: shared_down
  const int* meta;
  const int* sorted;
  const float* rw;
  const float* sgw;
  bf16* out;                // logits / act / y
  unsigned T, E, ld_out, max_items;
};

__device__ __forceinline__ void fetch_rows(unsigned lds_addr, int voff, const u32x4& rsrc) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  return u32x4{(unsigned)a, (unsigned)(a >> 32), bytes, 0x00020000u};
}

constexpr unsigned kOob = 0x80000000u;   // a row offset past every buffer's range

template <int MODE>
__global__ __launch_bounds__(256, 2) void moe_gemm_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) char lds[2 * kPfStage];
  __shared__ int row_slot[kPfBM];
  __shared__ float row_w[kPfBM];
  constexpr int K = MODE == kDown ? kMoeInter : kMoeHidden;
  constexpr int nsteps = K / kPfBK;
  const unsigned n_tiles_n = MODE == kRouter ? (p.E + 1 + kPfBN - 1) / kPfBN
                                             : (MODE == kGateUp ? kMoeInter / 64 : kMoeHidden / kPfBN);
  const unsigned m_tiles = MODE == kRouter ? (p.T + kPfBM - 1) / kPfBM : (unsigned)p.meta[0];
  const unsigned items = m_tiles * n_tiles_n;
  const unsigned share = (items + 7) / 8;
  const unsigned xi = blockIdx.x >> 3;
  if (xi >= share) return;
  const unsigned item = (blockIdx.x & 7) * share + xi;
  if (item >= items) return;
  const unsigned mt = item / n_tiles_n, nt = item % n_tiles_n;
  const int group = MODE == kRouter ? 0 : p.meta[1 + mt];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  // Operand sources (buffer resources: out-of-range rows read as zero).
  u32x4 ars, brs;
  if constexpr (MODE == kDown) {
    ars = buffer_rsrc(p.a + (size_t)mt * kPfBM * kMoeInter, kPfBM * kMoeInter * 2);
  } else {
    ars = buffer_rsrc(p.a, p.T * (unsigned)kMoeHidden * 2u);
  }
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

  // Per-lane fetch offsets: wave w fills A instructions 2w, 2w+1 (8 rows each)
  // and B instructions 4w..4w+3; lane = (row in the 8, chunk position), and
  // the source chunk is position ^ row so LDS holds the swizzled layout.
  const int r8 = lane >> 3, cpos = lane & 7;
  const int csrc = (cpos ^ r8) * 16;
  unsigned a_off[2], b_off[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = (2 * wave + j) * 8 + r8;   // tile row 0..63
    unsigned off;
    if constexpr (MODE == kRouter) {
      const unsigned t = mt * kPfBM + r;
      off = t < p.T ? t * (unsigned)kMoeHidden * 2u : kOob;
    } else if constexpr (MODE == kGateUp) {
      const int slot = p.sorted[mt * kPfBM + r];
      const unsigned routed = kMoeTopK * p.T;
      const unsigned t = slot < 0 ? 0u : ((unsigned)slot < routed ? (unsigned)slot / kMoeTopK
                                                                  : (unsigned)slot - routed);
      off = slot < 0 ? kOob : t * (unsigned)kMoeHidden * 2u;
    } else {
      off = (unsigned)r * kMoeInter * 2u;
    }
    a_off[j] = off + csrc;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = (4 * wave + j) * 8 + r8;   // tile weight row 0..127
    unsigned row;
    if constexpr (MODE == kGateUp)
      row = r < 64 ? nt * 64 + r : kMoeInter + nt * 64 + (r - 64);
    else
      row = nt * kPfBN + r;
    b_off[j] = row * (unsigned)K * 2u + csrc;
  }
  if constexpr (MODE == kDown) {
    if (tid < kPfBM) {
      const int slot = p.sorted[mt * kPfBM + tid];
      const unsigned routed = kMoeTopK * p.T;
      row_slot[tid] = slot;
      row_w[tid] = slot < 0 ? 0.f : ((unsigned)slot < routed ? p.rw[slot] : p.sgw[slot - routed]);
    }
  }

  const unsigned lds0 = static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds));
  auto fetch = [&](int step, int stage) {
    const unsigned sbase = lds0 + stage * kPfStage;
    const unsigned kb = (unsigned)step * kPfRowB;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      fetch_rows(sbase + ((2 * wave + j) * 8) * kPfRowB, (int)(a_off[j] + kb), ars);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      fetch_rows(sbase + kPfAStage + ((4 * wave + j) * 8) * kPfRowB, (int)(b_off[j] + kb), brs);
  };

  // MFMA operand addresses: wave (wm, wn) owns rows 32wm.. and weight rows
  // (gate/up: 32wn.. and 64 + 32wn..; else 64wn.. and 64wn + 32..).
  const int wm = wave & 1, wn = wave >> 1;
  const int li = lane & 31, kh = lane >> 5;
  const int arow = 32 * wm + li;
  const int brow0 = MODE == kGateUp ? 32 * wn + li : 64 * wn + li;
  const int brow1 = MODE == kGateUp ? 64 + 32 * wn + li : 64 * wn + 32 + li;
  int koff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) koff[s] = (((2 * s + kh) ^ (lane & 7)) * 16);

  f32x16 acc0 = f32x16{}, acc1 = f32x16{};
  fetch(0, 0);
  for (int step = 0; step < nsteps; ++step) {
    const int stage = step & 1;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's fetches of this step landed
    __syncthreads();                 // ... and every wave's; the other stage is free
    if (step + 1 < nsteps) fetch(step + 1, stage ^ 1);
    const char* sa = lds + stage * kPfStage;
    const char* sb = sa + kPfAStage;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 af = *reinterpret_cast<const bf16x8*>(sa + arow * kPfRowB + koff[s]);
      const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(sb + brow0 * kPfRowB + koff[s]);
      const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(sb + brow1 * kPfRowB + koff[s]);
      acc0 = mfma32x32x16(af, b0, acc0);
      acc1 = mfma32x32x16(af, b1, acc1);
    }
  }

  // Lane holds rows 32wm + 8(i/4) + 4kh + i%4 of weight rows brow0 / brow1.
  if constexpr (MODE == kRouter) {
    const unsigned n0 = nt * kPfBN + 64 * wn + li, n1 = n0 + 32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const unsigned t = mt * kPfBM + 32 * wm + 8 * (i >> 2) + 4 * kh + (i & 3);
      if (t < p.T) {
        if (n0 <= p.E) p.out[(size_t)t * p.ld_out + n0] = f2bf(acc0[i]);
        if (n1 <= p.E) p.out[(size_t)t * p.ld_out + n1] = f2bf(acc1[i]);
      }
    }
  } else if constexpr (MODE == kGateUp) {
    const unsigned c = nt * 64 + 32 * wn + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const unsigned r = mt * kPfBM + 32 * wm + 8 * (i >> 2) + 4 * kh + (i & 3);
      const float g = bf2f(f2bf(acc0[i])), u = bf2f(f2bf(acc1[i]));
      p.out[(size_t)r * kMoeInter + c] = f2bf(silu_f(g) * u);
    }
  } else {
    const unsigned n0 = nt * kPfBN + 64 * wn + li, n1 = n0 + 32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 32 * wm + 8 * (i >> 2) + 4 * kh + (i & 3);
      const int slot = row_slot[r];
      if (slot >= 0) {
        const float w = row_w[r];
        bf16* y = p.out + (size_t)slot * kMoeHidden;
        y[n0] = f2bf(bf2f(f2bf(acc0[i])) * w);
        y[n1] = f2bf(bf2f(f2bf(acc1[i])) * w);
      }
    }
  }
}

// ---- 7. per-token combine --------------------------------------------------
// moe = bf16(sum over ranks 0..7 of y, fp32 in rank order); out = bf16(after +
// bf16(moe + shared)) -- the order of qwen36_moe_decode's combine.
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const bf16* __restrict__ y, const bf16* __restrict__ after, bf16* __restrict__ out,
    unsigned T) {
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
#pragma unroll
  for (int k = 0; k < kMoeTopK; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) moe[e] += bf2f(yk[k][e]);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float total = bf2f(f2bf(bf2f(f2bf(moe[e])) + bf2f(ys[e])));
    o[e] = f2bf(bf2f(af[e]) + total);
  }
  *reinterpret_cast<bf16x8*>(out + (size_t)t * kMoeHidden + c) = o;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; }

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
  const PfLayout L = pf_layout(T, E);
  char* ws = static_cast<char*>(workspace);
  int* ids = reinterpret_cast<int*>(ws + L.ids);
  float* rw = reinterpret_cast<float*>(ws + L.rw);
  bf16* logits = reinterpret_cast<bf16*>(ws + L.logits);
  float* sgw = reinterpret_cast<float*>(ws + L.sgw);
  int* meta = reinterpret_cast<int*>(ws + L.meta);
  int* sorted = reinterpret_cast<int*>(ws + L.sorted);
  bf16* after = reinterpret_cast<bf16*>(ws + L.after);
  bf16* h2 = reinterpret_cast<bf16*>(ws + L.h2);
  bf16* act = reinterpret_cast<bf16*>(ws + L.act);
  bf16* y = reinterpret_cast<bf16*>(ws + L.y);
  const bf16* win = static_cast<const bf16*>(w_in);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned tok_blocks = (T + 3) / 4;

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

  g.a = h2;
  g.w = win;
  g.out = logits;
  g.ld_out = L.ld_logits;
  const unsigned router_items = ((T + kPfBM - 1) / kPfBM) * ((E + 1 + kPfBN - 1) / kPfBN);
  g.max_items = router_items;
  hipLaunchKernelGGL(moe_gemm_kernel<kRouter>, grid_for(router_items), dim3(256), 0, st, g);

  hipLaunchKernelGGL(moe_topk_kernel, dim3(tok_blocks), dim3(256), 0, st, logits,
                     L.ld_logits, E, T, ids, rw, sgw);
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(1024), 0, st, ids, T, E, meta, sorted);

  g.a = h2;
  g.w = static_cast<const bf16*>(expert_gate_up);
  g.w_shared = win + (size_t)(E + 1) * kMoeHidden;
  g.out = act;
  g.max_items = L.max_tiles * (kMoeInter / 64);
  hipLaunchKernelGGL(moe_gemm_kernel<kGateUp>, grid_for(g.max_items), dim3(256), 0, st, g);

  g.a = act;
  g.w = static_cast<const bf16*>(expert_down);
  g.w_shared = static_cast<const bf16*>(shared_down);
  g.out = y;
  g.max_items = L.max_tiles * (kMoeHidden / kPfBN);
  hipLaunchKernelGGL(moe_gemm_kernel<kDown>, grid_for(g.max_items), dim3(256), 0, st, g);

  hipLaunchKernelGGL(moe_combine_kernel, dim3(T), dim3(256), 0, st, y, after,
                     static_cast<bf16*>(out), T);
  return static_cast<int>(hipGetLastError());
}
