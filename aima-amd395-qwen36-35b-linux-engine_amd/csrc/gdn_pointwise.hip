// Gated-DeltaNet memory-bound pieces around the delta rule.
//
//  * qwen36_gdn_conv1d    -- depthwise causal conv (kernel 4) over
//    [state(3) | x] then SiLU; new state = last three inputs
//    (four_layer_mini_engine.py:5293-5403, direct form :5368-5386).
//  * qwen36_gdn_gating    -- beta = sigmoid(b), g = -exp(A_log) *
//    softplus(a + dt_bias) (fle:6507-6511; softplus threshold 20 as torch).
//  * qwen36_gdn_gated_norm -- per 128-wide v-head RMSNorm * w (no +1),
//    rounded to bf16, times SiLU(z), rounded to bf16 (fle:6531-6541;
//    native_pointwise.hip.cpp:376-430).
#include "common.h"

namespace q36 {
namespace {

__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float rsqrt_rn(float x) { return (float)(1.0 / sqrt((double)x)); }

constexpr int kConvTokensPerThread = 16;

// grid = (C/256, ceil(T/16)); thread = one channel, 16 consecutive tokens.
__global__ __launch_bounds__(256) void gdn_conv1d_kernel(
    const bf16* __restrict__ x, unsigned x_row_stride,
    const bf16* __restrict__ weight, const bf16* __restrict__ state_in,
    bf16* __restrict__ state_out, bf16* __restrict__ out, unsigned tokens) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const unsigned t0 = blockIdx.y * kConvTokensPerThread;
  float w[kGdnConvK];
#pragma unroll
  for (int i = 0; i < kGdnConvK; ++i) w[i] = bf2f(weight[c * kGdnConvK + i]);
  // window[j] = input at token t0 - 3 + j (j < 3 from history).
  float hist[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int tok = (int)t0 - 3 + j;
    hist[j] = tok >= 0 ? bf2f(x[(size_t)tok * x_row_stride + c])
                       : bf2f(state_in[c * 3 + (tok + 3)]);
  }
  const unsigned t_end = min(t0 + kConvTokensPerThread, tokens);
  for (unsigned t = t0; t < t_end; ++t) {
    const float cur = bf2f(x[(size_t)t * x_row_stride + c]);
    float acc = mul_rn(hist[0], w[0]);
    acc = add_rn(acc, mul_rn(hist[1], w[1]));
    acc = add_rn(acc, mul_rn(hist[2], w[2]));
    acc = add_rn(acc, mul_rn(cur, w[3]));
    const float cv = bf2f(f2bf(acc));
    const float s = cv / (1.0f + expf(-cv));
    out[(size_t)t * kGdnConvDim + c] = f2bf(s);
    hist[0] = hist[1];
    hist[1] = hist[2];
    hist[2] = cur;
  }
  // The first token block owns the state update, so a state_in that aliases
  // state_out is read before it is written by the same thread.
  if (blockIdx.y == 0) {
    float ns[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int tok = (int)tokens - 3 + j;
      ns[j] = tok >= 0 ? bf2f(x[(size_t)tok * x_row_stride + c])
                       : bf2f(state_in[c * 3 + (tok + 3)]);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) state_out[c * 3 + j] = f2bf(ns[j]);
  }
}

__global__ void gdn_gating_kernel(const bf16* __restrict__ a,
                                  const bf16* __restrict__ b,
                                  unsigned ab_row_stride,
                                  const float* __restrict__ a_log,
                                  const float* __restrict__ dt_bias,
                                  float* __restrict__ g, float* __restrict__ beta,
                                  unsigned tokens, bool beta_fp32) {
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * kGdnHv) return;
  const unsigned t = i / kGdnHv, h = i % kGdnHv;
  const float av = bf2f(a[(size_t)t * ab_row_stride + h]);
  const float bv = bf2f(b[(size_t)t * ab_row_stride + h]);
  const float xs = add_rn(av, dt_bias[h]);
  const float sp = xs > 20.0f ? xs : log1pf(expf(xs));
  g[i] = mul_rn(-expf(a_log[h]), sp);
  const float sb = 1.0f / (1.0f + expf(-bv));
  beta[i] = beta_fp32 ? sb : bf2f(f2bf(sb));
}

// grid = T*32/4 blocks of 4 waves; one wave per (token, v-head); lane holds
// dims 2*lane, 2*lane+1.
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(
    const bf16* __restrict__ core, const bf16* __restrict__ z,
    unsigned z_row_stride, const bf16* __restrict__ weight,
    bf16* __restrict__ out, unsigned rows) {
  const unsigned row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const unsigned t = row / kGdnHv, h = row % kGdnHv;
  const bf16* cp = core + (size_t)row * kGdnDv + 2 * lane;
  const float x0 = bf2f(cp[0]), x1 = bf2f(cp[1]);
  float sum = add_rn(mul_rn(x0, x0), mul_rn(x1, x1));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum = add_rn(sum, __shfl_xor(sum, o, 64));
  const float inv = rsqrt_rn(add_rn(mul_rn(sum, 1.0f / 128.0f), 1e-6f));
  const bf16* zp = z + (size_t)t * z_row_stride + h * kGdnDv + 2 * lane;
  bf16* op = out + (size_t)t * (kGdnHv * kGdnDv) + h * kGdnDv + 2 * lane;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float xv = e ? x1 : x0;
    const float nv = bf2f(f2bf(mul_rn(mul_rn(xv, inv), bf2f(weight[2 * lane + e]))));
    const float zv = bf2f(zp[e]);
    const float silu = zv / (1.0f + expf(-zv));
    op[e] = f2bf(mul_rn(nv, silu));
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT int qwen36_gdn_conv1d(const void* x, unsigned x_row_stride,
                                 const void* weight, const void* state_in,
                                 void* state_out, void* out, unsigned tokens,
                                 void* stream) {
  if (x == nullptr || weight == nullptr || state_in == nullptr ||
      state_out == nullptr || out == nullptr || tokens == 0 ||
      tokens > kMaxTokens || x_row_stride < (unsigned)kGdnConvDim)
    return Q36_EINVAL;
  const dim3 grid(kGdnConvDim / 256,
                  (tokens + kConvTokensPerThread - 1) / kConvTokensPerThread);
  hipLaunchKernelGGL(gdn_conv1d_kernel, grid, dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(x), x_row_stride,
                     static_cast<const bf16*>(weight),
                     static_cast<const bf16*>(state_in),
                     static_cast<bf16*>(state_out), static_cast<bf16*>(out),
                     tokens);
  return static_cast<int>(hipGetLastError());
}

Q36_EXPORT int qwen36_gdn_gating(const void* a, const void* b,
                                 unsigned ab_row_stride, const void* a_log,
                                 const void* dt_bias, void* g, void* beta,
                                 unsigned tokens, unsigned flags, void* stream) {
  if (a == nullptr || b == nullptr || a_log == nullptr || dt_bias == nullptr ||
      g == nullptr || beta == nullptr || tokens == 0 || tokens > kMaxTokens ||
      ab_row_stride < (unsigned)kGdnHv || (flags & ~1u) != 0)
    return Q36_EINVAL;
  const unsigned n = tokens * kGdnHv;
  hipLaunchKernelGGL(gdn_gating_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(a), static_cast<const bf16*>(b),
                     ab_row_stride, static_cast<const float*>(a_log),
                     static_cast<const float*>(dt_bias),
                     static_cast<float*>(g), static_cast<float*>(beta), tokens,
                     (flags & 1u) != 0);
  return static_cast<int>(hipGetLastError());
}

Q36_EXPORT int qwen36_gdn_gated_norm(const void* core, const void* z,
                                     unsigned z_row_stride, const void* weight,
                                     void* out, unsigned tokens, void* stream) {
  if (core == nullptr || z == nullptr || weight == nullptr || out == nullptr ||
      tokens == 0 || tokens > kMaxTokens ||
      z_row_stride < (unsigned)(kGdnHv * kGdnDv))
    return Q36_EINVAL;
  const unsigned rows = tokens * kGdnHv;
  hipLaunchKernelGGL(gdn_gated_norm_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(core), static_cast<const bf16*>(z),
                     z_row_stride, static_cast<const bf16*>(weight),
                     static_cast<bf16*>(out), rows);
  return static_cast<int>(hipGetLastError());
}
