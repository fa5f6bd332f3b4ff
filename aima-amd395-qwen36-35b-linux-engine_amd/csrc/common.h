// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// MFMA operand layouts used throughout (measured on gfx950, wave64):
//   v_mfma_f32_16x16x32_bf16: A lane l holds A[l%16][8*(l/16) .. +8],
//     B lane l holds B[8*(l/16) .. +8][l%16], D lane l holds
//     D[4*(l/16) + r][l%16], r = 0..3.
//   v_mfma_f32_32x32x16_bf16: A lane l holds A[l%32][8*(l/32) .. +8],
//     B lane l holds B[8*(l/32) .. +8][l%32], D lane l holds
//     D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
//   v_mfma_f32_16x16x4_f32: A lane l holds A[l%16][l/16], B lane l holds
//     B[l/16][l%16], D as for 16x16x32.
//   ds_read_b64_tr_b16 (per 16-lane group, lane m supplies address a_m of
//     four consecutive b16 values): result lane i, element e =
//     mem[a_{4e + i/4} + (i%4)].
// Because the reduction index of an MFMA may be permuted freely (as long as
// A and B agree), kernels choose k-orderings that make every global or LDS
// access a contiguous 8- or 16-byte vector.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

namespace q36 {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kHq = 16;        // query heads (full attention)
constexpr int kHkv = 2;        // KV heads
constexpr int kGroup = kHq / kHkv;
constexpr int kD = 256;        // head dim
constexpr int kQDim = kHq * kD;     // 4096
constexpr int kKvRow = kHkv * kD;   // 512 elements per cache row
constexpr int kRotary = 64;
constexpr int kRotaryPairs = kRotary / 2;
constexpr float kRopeTheta = 1.0e7f;
constexpr unsigned kMaxTokens = 262144u;

// Gated DeltaNet geometry.
constexpr int kGdnHk = 16, kGdnHv = 32, kGdnDk = 128, kGdnDv = 128;
constexpr int kGdnConvDim = 2 * kGdnHk * kGdnDk + kGdnHv * kGdnDv;  // 8192
constexpr int kGdnConvK = 4;

constexpr float kLog2e = 1.4426950408889634f;

__host__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }  // RNE

// Sigmoid output gate of one attention value (native_pointwise.hip.cpp:
// 207-222, :339-359): the attention rounded to bf16, sigmoid(gate) rounded
// to bf16, their product rounded to bf16.  Shared by every kernel that
// applies the gate so they round identically.
__device__ __forceinline__ bf16 gate_bf16(float attn, bf16 gate) {
  const bf16 a = f2bf(attn);
  const bf16 sg = f2bf(1.0f / (1.0f + expf(-bf2f(gate))));
  return f2bf(__fmul_rn(bf2f(a), bf2f(sg)));
}

// log2(e) split for exp2 arguments: g * kLog2eHi is exact for bf16 g.
constexpr float kLog2eHi = 1.44268798828125f;       // 47274 / 2^15
constexpr float kLn2Lo = 4.888495152129525e-06f;    // (log2(e) - kLog2eHi) ln 2

// x / (1 + e^-x) (SiLU as the reference's conv writes it) for a bf16 x,
// from the hardware exp2 and reciprocal with the split log2(e) of
// gate4_bf16_fast: within ~5 ulps of the exact form's value.  Sets `slow`
// when that value could round to another bf16 than the exact one (within
// 32 ulps of a rounding midpoint), or |x| > 60, or x is not finite.
__device__ __forceinline__ float silu_fast(float x, bool& slow) {
  const float th = __builtin_amdgcn_exp2f(x * -kLog2eHi);
  const float t = __builtin_fmaf(th, x * -kLn2Lo, th);
  const float s = x * __builtin_amdgcn_rcpf(1.0f + t);
  const int mid = (int)(__float_as_uint(s) & 0xffffu) - 0x8000;
  slow = !(fabsf(x) <= 60.0f) || (mid >= -32 && mid <= 32);
  return s;
}

// gate_bf16 for four values, with the sigmoid from the hardware exp2 and
// reciprocal.  g is bf16 (8 significant bits) and log2(e)'s high part has
// 16, so g * kLog2eHi is exact and the low part enters as a first-order
// factor: e^-g = 2^(-g kLog2eHi) (1 - g kLn2Lo) within ~2 ulps, 1/(1 + e^-g)
// within ~4, the exact form's expf and division within 2 -- so unless the
// fast value lies within 32 ulps of a bf16 rounding midpoint (low 16 bits
// 0x8000) both round to the same bf16.  Such values (about 1 in 1000), |g|
// > 60 and non-finite g take the exact form; the group of four branches
// once.  Same bits as gate_bf16 for every non-NaN gate (checked over all
// 65536 bf16 gates; a NaN gate gives a NaN) at a fraction of the
// instructions -- for epilogues, where the gate's math is not spread over a
// whole elementwise launch.
__device__ __forceinline__ bf16x4 gate4_bf16_fast(const f32x4& attn, const bf16x4& gate) {
  float sg[4];
  bool slow = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float g = bf2f(gate[e]);
    const float th = __builtin_amdgcn_exp2f(g * -kLog2eHi);
    const float t = __builtin_fmaf(th, g * -kLn2Lo, th);
    sg[e] = __builtin_amdgcn_rcpf(1.0f + t);
    const int mid = (int)(__float_as_uint(sg[e]) & 0xffffu) - 0x8000;
    slow |= !(fabsf(g) <= 60.0f) || (mid >= -32 && mid <= 32);
  }
  if (slow) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g = bf2f(gate[e]);
      const int mid = (int)(__float_as_uint(sg[e]) & 0xffffu) - 0x8000;
      if (!(fabsf(g) <= 60.0f) || (mid >= -32 && mid <= 32)) sg[e] = 1.0f / (1.0f + expf(-g));
    }
  }
  bf16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = f2bf(__fmul_rn(bf2f(f2bf(attn[e])), bf2f(f2bf(sg[e]))));
  return o;
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Transposed LDS read of four b16 values (see layout note above).
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

__device__ __forceinline__ bf16x8 cat_bf16x8(i16x4 lo, i16x4 hi) {
  i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations
// (lgkmcnt) but, unlike __syncthreads(), not for its outstanding global loads,
// so prefetches stay in flight across the barrier.  The signal fences keep
// the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt(63) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}

// ---- head RMSNorm + partial RoPE (shared by the prefill pointwise kernel
// and the fused decode step, so both round identically) -------------------
// RoPE inverse frequencies 1 / 1e7^(2i/64), i < 32, each correctly rounded
// to fp32 (computed on the host in double; each translation unit keeps its
// own __constant__ copy).
inline void rope_inv_freq_host(float* h) {
  for (int i = 0; i < kRotaryPairs; ++i)
    h[i] = (float)(1.0 / pow(1.0e7, (2.0 * i) / (double)kRotary));
}

// RoPE cos/sin for one position as one wave needs them: lane p < 32 computes
// pair p (fp32 angle = pos * inv_freq[p], cosf/sinf), and lane l < 16 then
// gathers pairs (4l + e) mod 32, e < 4 -- the pairs of its dims 4l..4l+3.
__device__ __forceinline__ void rope_cos_sin_wave(unsigned pos, const float* inv_freq,
                                                  float (&c)[4], float (&s)[4]) {
  const int lane = threadIdx.x & 63;
  const float angle = __fmul_rn((float)pos, inv_freq[lane & (kRotaryPairs - 1)]);
  const float cv = cosf(angle), sv = sinf(angle);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    c[e] = __shfl(cv, (4 * lane + e) & (kRotaryPairs - 1), 64);
    s[e] = __shfl(sv, (4 * lane + e) & (kRotaryPairs - 1), 64);
  }
}

// One 256-wide head held by one wave, lane l holding dims 4l..4l+3: RMSNorm
// with the (w + 1) weight (fp32, every product and sum rounded separately,
// eps 1e-6, correctly rounded rsqrt), rounded to bf16, then rotate-half RoPE
// on dims [0, 64) with the cos/sin of rope_cos_sin_wave (lanes 0-7 pair with
// lanes 8-15).
// Returns the fp32 values before the final bf16 rounding.
// (four_layer_mini_engine.py:5151-5162; native_pointwise.hip.cpp:242-337.)
__device__ __forceinline__ void head_norm_rope_wave_wp1(const float (&x)[4],
                                                        const float (&wp1)[4],
                                                        const float (&cs)[4],
                                                        const float (&sn)[4],
                                                        float (&y)[4]) {
  const int lane = threadIdx.x & 63;
  float sq[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) sq[e] = __fmul_rn(x[e], x[e]);
  float sum = __fadd_rn(__fadd_rn(sq[0], sq[1]), __fadd_rn(sq[2], sq[3]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, o, 64));
  const float var = __fmul_rn(sum, 1.0f / 256.0f);
  const float inv = (float)(1.0 / sqrt((double)__fadd_rn(var, 1e-6f)));
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = bf2f(f2bf(__fmul_rn(__fmul_rn(x[e], inv), wp1[e])));
  float mate[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) mate[e] = __shfl_xor(y[e], 8, 64);
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      y[e] = lane < 8 ? __fsub_rn(__fmul_rn(y[e], cs[e]), __fmul_rn(mate[e], sn[e]))
                      : __fadd_rn(__fmul_rn(y[e], cs[e]), __fmul_rn(mate[e], sn[e]));
  }
}

// The (w + 1) factors of this lane's four dims.
__device__ __forceinline__ void head_norm_wp1(const bf16* __restrict__ w, float (&wp1)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < 4; ++e) wp1[e] = __fadd_rn(bf2f(w[4 * lane + e]), 1.0f);
}

__device__ __forceinline__ void head_norm_rope_wave(const float (&x)[4],
                                                    const bf16* __restrict__ w,
                                                    const float (&cs)[4],
                                                    const float (&sn)[4],
                                                    float (&y)[4]) {
  float wp1[4];
  head_norm_wp1(w, wp1);
  head_norm_rope_wave_wp1(x, wp1, cs, sn, y);
}

}  // namespace q36

#define Q36_EXPORT extern "C" __attribute__((visibility("default")))

// hipError_t values returned through the C ABI (the reference's providers
// return a hipError_t as int, qrt_ck_fmha_q8192_provider.cpp:141-146).
#define Q36_OK 0
#define Q36_EINVAL 1  // hipErrorInvalidValue
