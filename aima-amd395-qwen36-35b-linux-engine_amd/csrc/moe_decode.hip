// One-token MoE block of the Qwen3.6-35B-A3B layer (the step after
// attention), in three launches.
//
// Restates, for one decode token, layer_body's tail in
// four_layer_mini_engine.py:8479-8650 with the router of :7775-7789, the
// routed experts of :7791-7803 ("expanded" reference form) and the shared
// expert of :8240-8300 -- the reference's native decode runs these as the
// router top-k Triton kernels (:391-460), the native MoE consumer
// (:1066-1200) and the shared-expert projections:
//   after = inp + attn;  h2 = rmsnorm(after) * (w + 1)       (eps 1e-6)
//   logits = h2 @ router^T (bf16);  top-8 of logits (fp32)
//   rw = bf16(softmax(top-8 logits))
//   expert e: [gate | up] = bf16(h2 @ gate_up_e^T) ([1024] = 512 | 512)
//             act = bf16(silu(gate) * up);  y_e = bf16(act @ down_e^T)
//   moe = bf16(sum_k bf16(y_k * rw_k));  shared analogous with its own
//   weights, scaled by bf16(sigmoid(shared_gate . h2))
//   out = bf16(after + bf16(moe + shared))
// with every bf16 rounding of the eager PyTorch text.
//
// Launches (all HBM-bound GEMV shapes, 16-byte nontemporal weight loads):
//  1. moe_router_kernel: each wave first requests its weight row, then
//     residual add + RMSNorm (every wave recomputes h2 from the 2048
//     inputs; block 0 stores `after` and h2), then a GEMV over the rows
//     [router (E) | shared_gate (1)] -> bf16.
//  2. moe_expert_up_kernel: grid (9 slots, 64 tiles of 8 rows): slot k < 8
//     selects the top-8 experts from the E logits itself (one wave, packed
//     32-bit keys reduced with DPP and permlane swaps; ties to the lower
//     index) and computes 8 act rows of expert k (gate and up rows
//     together); slot 8 computes the shared expert's act rows from the
//     shared gate_proj | up_proj rows of w_in, without waiting for a top-8;
//     workgroup (0, 0) stores the ids and routing weights.
//  3. moe_down_kernel: each wave owns 1 output row and reads that row of
//     the 8 selected down matrices and the shared one, then combines.
#include "moe_common.h"

namespace q36 {
namespace {

// Workspace layout (bytes).
constexpr size_t kWsAfter = 0;                                   // bf16 [2048]
constexpr size_t kWsH2 = kWsAfter + kMoeHidden * 2;               // bf16 [2048]
constexpr size_t kWsIds = kWsH2 + kMoeHidden * 2;                 // int [8]
constexpr size_t kWsRw = kWsIds + kMoeTopK * 4;                   // float [8] (bf16 values)
constexpr size_t kWsAct = kWsRw + kMoeTopK * 4;                   // bf16 [9][512]
constexpr size_t kWsProj = kWsAct + (kMoeTopK + 1) * kMoeInter * 2;   // bf16 [E + 1]: logits, shared gate
constexpr size_t kWsBytes = kWsProj + (kMoeMaxExperts + 1) * 2;

// Router GEMV rows per wave (launch 1 runs one row group per wave; 1 row:
// 65 workgroups for 257 rows, measured 2% faster per token than 2 rows).
constexpr int kRouterRows = 1;
// Expert act rows per wave (launch 2; each needs a gate and an up row).
constexpr int kUpRows = 2;
// Down-projection output rows per wave (launch 3).
constexpr int kDownRows = 1;

// GEMV of one row r (K = 2048) with x held as lane l's columns 8l + 512j.
__device__ __forceinline__ float dot2048(const u32x4 (&wr)[4], const float (&xv)[4][8]) {
  float a = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 v = __builtin_bit_cast(bf16x8, wr[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) a = __builtin_fmaf(bf2f(v[e]), xv[j][e], a);
  }
  return a;
}

// ---- 1. residual + RMSNorm + fused router / shared-input GEMV -------------
__global__ __launch_bounds__(256, 2) void moe_router_kernel(
    const bf16* __restrict__ inp, const bf16* __restrict__ attn,
    const bf16* __restrict__ norm_w, const bf16* __restrict__ w_in,
    unsigned n_rows, char* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const unsigned wave_g = blockIdx.x * 4 + (threadIdx.x >> 6);
  const unsigned waves = gridDim.x * 4;
  // This wave's first weight rows are requested before the RMSNorm prologue,
  // so their HBM latency overlaps it.
  u32x4 wr[kRouterRows][4];
  auto load_rows = [&](unsigned r0) {
#pragma unroll
    for (int r = 0; r < kRouterRows; ++r) {
      const unsigned row = min(r0 + r, n_rows - 1);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wr[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            w_in + (size_t)row * kMoeHidden + 512 * j + 8 * lane));
    }
  };
  unsigned r0 = wave_g * kRouterRows;
  load_rows(r0);   // rows clamp to n_rows - 1, so a spare wave's loads stay in bounds
  __builtin_amdgcn_sched_barrier(0);
  // after = bf16(inp + attn); h2 = bf16(after * rsqrt(mean(after^2) + eps) * (w + 1))
  float xa[4][8], ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(inp + 512 * j + 8 * lane);
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(attn + 512 * j + 8 * lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xa[j][e] = bf2f(f2bf(bf2f(a[e]) + bf2f(b[e])));
      ss = __builtin_fmaf(xa[j][e], xa[j][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float inv = (float)(1.0 / sqrt((double)(ss / (float)kMoeHidden + kMoeEps)));
  float xv[4][8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 w = *reinterpret_cast<const bf16x8*>(norm_w + 512 * j + 8 * lane);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      xv[j][e] = bf2f(f2bf((xa[j][e] * inv) * (bf2f(w[e]) + 1.0f)));
  }
  if (blockIdx.x == 0 && threadIdx.x < 64) {
    bf16x8 oa, oh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        oa[e] = f2bf(xa[j][e]);
        oh[e] = f2bf(xv[j][e]);
      }
      *reinterpret_cast<bf16x8*>(ws + kWsAfter + 2 * (512 * j + 8 * lane)) = oa;
      *reinterpret_cast<bf16x8*>(ws + kWsH2 + 2 * (512 * j + 8 * lane)) = oh;
    }
  }
  bf16* proj = reinterpret_cast<bf16*>(ws + kWsProj);
  for (; r0 < n_rows; r0 += waves * kRouterRows) {
    float acc[kRouterRows];
#pragma unroll
    for (int r = 0; r < kRouterRows; ++r) acc[r] = wave_sum(dot2048(wr[r], xv));
    if (lane < kRouterRows && r0 + lane < n_rows) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < kRouterRows; ++r) v = lane == r ? acc[r] : v;
      proj[r0 + lane] = f2bf(v);
    }
    if (r0 + waves * kRouterRows < n_rows) {
      load_rows(r0 + waves * kRouterRows);
      __builtin_amdgcn_sched_barrier(0);   // keep every weight load in flight before the FMAs
    }
  }
}

// ---- 2. expert gate/up + SiLU ---------------------------------------------
// grid = (9, 64); block = 256: wave w computes act rows tile*8 + 2w .. +2 of
// slot blockIdx.x (its 2 gate rows and 2 up rows, 4 rows x 4 KiB in flight;
// 4 + 4 rows per wave over half the workgroups measured 10% slower per token).
__global__ __launch_bounds__(256, 2) void moe_expert_up_kernel(
    const bf16* __restrict__ gate_up, const bf16* __restrict__ w_in, unsigned n_experts,
    char* __restrict__ ws) {
  const int slot = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j0 = blockIdx.y * (4 * kUpRows) + kUpRows * wave;
  const bf16* proj = reinterpret_cast<const bf16*>(ws + kWsProj);
  bf16* act = reinterpret_cast<bf16*>(ws + kWsAct);
  const bf16* wexp;
  if (slot == kMoeTopK) {
    // shared expert: its gate_proj | up_proj rows follow the router and
    // shared_gate rows of w_in, in an expert's gate_up layout
    wexp = w_in + (size_t)(n_experts + 1) * kMoeHidden;
  } else {
    int ids[kMoeTopK];
    float vals[kMoeTopK];
    select_top8(proj, n_experts, ids, vals);
    if (blockIdx.y == 0 && slot == 0 && wave == 0 && lane == 0) {
      float rw[kMoeTopK];
      routing_weights(vals, rw);
#pragma unroll
      for (int k = 0; k < kMoeTopK; ++k) {
        reinterpret_cast<int*>(ws + kWsIds)[k] = ids[k];
        reinterpret_cast<float*>(ws + kWsRw)[k] = rw[k];
      }
    }
    int e = ids[0];
#pragma unroll
    for (int k = 1; k < kMoeTopK; ++k) e = slot == k ? ids[k] : e;
    wexp = gate_up + (size_t)e * (2 * kMoeInter) * kMoeHidden;
  }
  float xv[4][8];
  const bf16* h2 = reinterpret_cast<const bf16*>(ws + kWsH2);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(h2 + 512 * j + 8 * lane);
#pragma unroll
    for (int q = 0; q < 8; ++q) xv[j][q] = bf2f(v[q]);
  }
  u32x4 wr[2 * kUpRows][4];
#pragma unroll
  for (int r = 0; r < 2 * kUpRows; ++r) {
    const int row = (r < kUpRows) ? (j0 + r) : (kMoeInter + j0 + r - kUpRows);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wr[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          wexp + (size_t)row * kMoeHidden + 512 * j + 8 * lane));
  }
  __builtin_amdgcn_sched_barrier(0);   // keep every weight load in flight before the FMAs
  float acc[2 * kUpRows];
#pragma unroll
  for (int r = 0; r < 2 * kUpRows; ++r) acc[r] = wave_sum(dot2048(wr[r], xv));
  if (lane < kUpRows) {
    float g = acc[0], u = acc[kUpRows];
#pragma unroll
    for (int r = 1; r < kUpRows; ++r) {
      g = lane == r ? acc[r] : g;
      u = lane == r ? acc[kUpRows + r] : u;
    }
    const float gb = bf2f(f2bf(g)), ub = bf2f(f2bf(u));
    act[slot * kMoeInter + j0 + lane] = f2bf(silu_f(gb) * ub);
  }
}

// ---- 3. down projections + combine + residual ----------------------------
// grid = 2048 / 4 workgroups of 4 waves; a wave owns one output row.
// Lane l covers the 8 intermediate columns 8l..8l+7 of every down row.
__global__ __launch_bounds__(256, 2) void moe_down_kernel(
    const bf16* __restrict__ down, const bf16* __restrict__ shared_down,
    unsigned n_experts, const char* __restrict__ ws, bf16* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * (4 * kDownRows) + kDownRows * wave;
  const int* ids = reinterpret_cast<const int*>(ws + kWsIds);
  const float* rw = reinterpret_cast<const float*>(ws + kWsRw);
  const bf16* act = reinterpret_cast<const bf16*>(ws + kWsAct);
  const bf16* proj = reinterpret_cast<const bf16*>(ws + kWsProj);
  const bf16* after = reinterpret_cast<const bf16*>(ws + kWsAfter);
  u32x4 wr[kDownRows][kMoeTopK + 1];
  // the shared rows do not depend on the routing: request them first
#pragma unroll
  for (int r = 0; r < kDownRows; ++r)
    wr[r][kMoeTopK] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
        shared_down + (size_t)(r0 + r) * kMoeInter + 8 * lane));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < kDownRows; ++r)
#pragma unroll
    for (int k = 0; k < kMoeTopK; ++k)
      wr[r][k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          down + (size_t)ids[k] * kMoeHidden * kMoeInter + (size_t)(r0 + r) * kMoeInter +
          8 * lane));
  __builtin_amdgcn_sched_barrier(0);   // keep every weight load in flight before the FMAs
  float xa[kMoeTopK + 1][8];
#pragma unroll
  for (int k = 0; k <= kMoeTopK; ++k) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(act + k * kMoeInter + 8 * lane);
#pragma unroll
    for (int q = 0; q < 8; ++q) xa[k][q] = bf2f(v[q]);
  }
  float y[kDownRows][kMoeTopK + 1];
#pragma unroll
  for (int r = 0; r < kDownRows; ++r)
#pragma unroll
    for (int k = 0; k <= kMoeTopK; ++k) {
      const bf16x8 v = __builtin_bit_cast(bf16x8, wr[r][k]);
      float a = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) a = __builtin_fmaf(bf2f(v[q]), xa[k][q], a);
      y[r][k] = wave_sum(a);
    }
  if (lane < kDownRows) {
    const int r = lane;
    float yr[kMoeTopK + 1];
#pragma unroll
    for (int k = 0; k <= kMoeTopK; ++k) {
      yr[k] = y[0][k];
#pragma unroll
      for (int q = 1; q < kDownRows; ++q) yr[k] = r == q ? y[q][k] : yr[k];
    }
    // routed: sum_k bf16(bf16(y_k) * rw_k), accumulated in fp32, rounded once
    float moe = 0.f;
#pragma unroll
    for (int k = 0; k < kMoeTopK; ++k) moe += bf2f(f2bf(bf2f(f2bf(yr[k])) * rw[k]));
    const float moe_b = bf2f(f2bf(moe));
    // shared: bf16(sigmoid(shared_gate)) * bf16(y_shared)
    const float sgate = bf2f(f2bf(1.0f / (1.0f + expf(-bf2f(proj[n_experts])))));
    const float shared = bf2f(f2bf(sgate * bf2f(f2bf(yr[kMoeTopK]))));
    const float total = bf2f(f2bf(moe_b + shared));
    out[r0 + r] = f2bf(bf2f(after[r0 + r]) + total);
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT size_t qwen36_moe_decode_workspace_bytes(void) { return kWsBytes; }

// One token through the MoE block.  inp, attn_out [2048] bf16 (the layer's
// residual input and attention output); post_norm_w [2048] bf16 (weight + 1
// convention); w_in [E + 1 + 1024, 2048] bf16 = rows [router | shared_gate |
// shared gate_proj | shared up_proj]; expert_gate_up [E, 1024, 2048] (gate
// rows 0..511, up rows 512..1023); expert_down [E, 2048, 512];
// shared_down [2048, 512]; out [2048] bf16 = after + MoE(h2).  8 <= E <= 256,
// E a multiple of 4.
Q36_EXPORT int qwen36_moe_decode(const void* inp, const void* attn_out,
                                 const void* post_norm_w, const void* w_in,
                                 const void* expert_gate_up, const void* expert_down,
                                 const void* shared_down, unsigned n_experts, void* out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  if (inp == nullptr || attn_out == nullptr || post_norm_w == nullptr || w_in == nullptr ||
      expert_gate_up == nullptr || expert_down == nullptr || shared_down == nullptr ||
      out == nullptr || workspace == nullptr || workspace_bytes < kWsBytes ||
      n_experts < (unsigned)kMoeTopK || n_experts > (unsigned)kMoeMaxExperts ||
      (n_experts % 4) != 0)
    return Q36_EINVAL;
  for (const void* p : {inp, attn_out, post_norm_w, w_in, expert_gate_up, expert_down,
                        shared_down, static_cast<const void*>(workspace)})
    if ((reinterpret_cast<uintptr_t>(p) % 16) != 0) return Q36_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const unsigned n_in = n_experts + 1;   // router + shared_gate rows
  const unsigned groups = (n_in + kRouterRows - 1) / kRouterRows;
  hipLaunchKernelGGL(moe_router_kernel, dim3((groups + 3) / 4), dim3(256), 0, st,
                     static_cast<const bf16*>(inp), static_cast<const bf16*>(attn_out),
                     static_cast<const bf16*>(post_norm_w), static_cast<const bf16*>(w_in),
                     n_in, ws);
  hipLaunchKernelGGL(moe_expert_up_kernel, dim3(kMoeTopK + 1, kMoeInter / (4 * kUpRows)), dim3(256), 0,
                     st, static_cast<const bf16*>(expert_gate_up),
                     static_cast<const bf16*>(w_in), n_experts, ws);
  hipLaunchKernelGGL(moe_down_kernel, dim3(kMoeHidden / (4 * kDownRows)), dim3(256), 0, st,
                     static_cast<const bf16*>(expert_down), static_cast<const bf16*>(shared_down),
                     n_experts, ws, static_cast<bf16*>(out));
  return static_cast<int>(hipGetLastError());
}
