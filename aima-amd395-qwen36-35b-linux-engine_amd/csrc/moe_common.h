// Device helpers shared by the MoE decode and prefill kernels: geometry,
// SiLU, wave reductions and the router's top-8 selection with its softmax.
#pragma once
#include "common.h"

namespace q36 {
namespace {

constexpr int kMoeHidden = 2048;
constexpr int kMoeInter = 512;          // expert and shared intermediate size
constexpr int kMoeTopK = 8;
constexpr int kMoeMaxExperts = 256;
constexpr float kMoeEps = 1e-6f;

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Max of a 32-bit unsigned key over the wave, result in every lane: DPP
// within rows of 16 (quad perms, half mirror, mirror), then the row-pair and
// half swaps of v_permlane16/32_swap -- no LDS round trips.
__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));  // quad xor 1
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));  // quad xor 2
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false)); // half mirror
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false)); // mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((unsigned)r16[0], (unsigned)r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((unsigned)r32[0], (unsigned)r32[1]);
}

// Top-8 of the E router logits, ties to the lower expert index, by one wave:
// a bf16 logit maps to an order-preserving 16-bit key (sign set: all bits
// flipped; else sign bit set), packed above 0xFFFF - expert so one unsigned
// max picks the largest logit and, among equal ones, the lowest expert.
// Lane l holds experts l + 64i.  (-0 ranks below +0; NaN logits unsupported.)
__device__ void select_top8_bits(const unsigned short (&raw)[4], unsigned n_experts,
                                 int (&ids)[kMoeTopK], float (&vals)[kMoeTopK]) {
  const int lane = threadIdx.x & 63;
  unsigned key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned e = lane + 64 * i;
    const unsigned b = raw[i];
    const unsigned ord = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
    key[i] = e < n_experts ? (ord << 16) | (0xFFFFu - e) : 0u;
  }
#pragma unroll
  for (int r = 0; r < kMoeTopK; ++r) {
    unsigned best = max(max(key[0], key[1]), max(key[2], key[3]));
    best = wave_max_u32(best);
    const unsigned e = 0xFFFFu - (best & 0xFFFFu);
    const unsigned ord = best >> 16;
    const unsigned b = (ord & 0x8000u) ? (ord & 0x7FFFu) : (~ord & 0xFFFFu);
    ids[r] = (int)e;
    vals[r] = bf2f(__builtin_bit_cast(bf16, (unsigned short)b));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (key[i] == best) key[i] = 0u;
  }
}

// select_top8_bits over logits[0, n_experts) read from memory.
__device__ void select_top8(const bf16* __restrict__ logits, unsigned n_experts,
                            int (&ids)[kMoeTopK], float (&vals)[kMoeTopK]) {
  const int lane = threadIdx.x & 63;
  // all four logits are requested before any is used (clamped index: one
  // memory round trip, not one per branch)
  unsigned short raw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned e = lane + 64 * i;
    raw[i] = __builtin_bit_cast(unsigned short, logits[e < n_experts ? e : 0u]);
  }
  select_top8_bits(raw, n_experts, ids, vals);
}

// Routing weights of the reference router (four_layer_mini_engine.py:7775-7789:
// softmax over the 8 selected fp32 logits, rounded to bf16), returned as the
// fp32 value of each bf16 weight.
__device__ __forceinline__ void routing_weights(const float (&vals)[kMoeTopK],
                                                float (&rw)[kMoeTopK]) {
  float sum = 0.f, ex[kMoeTopK];
#pragma unroll
  for (int k = 0; k < kMoeTopK; ++k) {
    ex[k] = expf(vals[k] - vals[0]);
    sum += ex[k];
  }
#pragma unroll
  for (int k = 0; k < kMoeTopK; ++k) rw[k] = bf2f(f2bf(ex[k] / sum));
}

}  // namespace
}  // namespace q36
