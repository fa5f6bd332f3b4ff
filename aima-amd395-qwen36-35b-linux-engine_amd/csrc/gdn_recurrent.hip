// Gated-DeltaNet recurrent (decode) step with an fp32 state.
//
// Restates torch_recurrent_gated_delta_rule
// (benchmarks/shape-lab/four_layer_mini_engine.py:5242-5276), the role the
// reference fills with vLLM's fused_sigmoid_gating_delta_rule_update
// (fle:6417-6447, launched natively by native_linear_layer.hip.cpp:84-95).
// Per token t and v-head h (key head h * qk_heads / 32):
//   q, k <- l2norm (x * rsqrt(sum x^2 + 1e-6)); q *= 1/sqrt(128)
//   S <- S * exp(g);  kv = S^T k;  delta = (v - kv) * beta
//   S <- S + k (x) delta;  o = S^T q
// State layout [32][128 (k)][128 (v)] fp32, as the torch oracle keeps it.
//
// HBM-bound (2 MiB read + 2 MiB write per layer step).  grid = 32 heads x 8
// column blocks of 16 v; a thread owns 8 rows x 1 column of S in registers,
// so S is read once and written once however many tokens are processed, and
// state_in may alias state_out.
#include "common.h"

namespace q36 {
namespace {

constexpr int kRecVBlock = 16;
constexpr int kRecRows = 8;   // k rows per thread: 16 groups x 8 = 128

__global__ __launch_bounds__(256) void gdn_recurrent_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, unsigned qk_heads, unsigned qk_token_stride,
    unsigned v_token_stride, const float* __restrict__ g,
    const float* __restrict__ beta, const float* state_in, float* state_out,
    bf16* __restrict__ out, unsigned tokens) {
  __shared__ float red[2][4][kRecVBlock];
  const int h = blockIdx.x;
  const int v0 = blockIdx.y * kRecVBlock;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int vi = lane & 15;
  const int kq = wave * 4 + (lane >> 4);
  const int kh = h * (int)qk_heads / kGdnHv;
  const size_t sbase = (size_t)h * kGdnDk * kGdnDv + v0 + vi;

  float s[kRecRows];
#pragma unroll
  for (int j = 0; j < kRecRows; ++j)
    s[j] = state_in[sbase + (size_t)(kq * kRecRows + j) * kGdnDv];

  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  for (unsigned t = 0; t < tokens; ++t) {
    const bf16* qp = q + (size_t)t * qk_token_stride + kh * kGdnDk;
    const bf16* kp = k + (size_t)t * qk_token_stride + kh * kGdnDk;
    // every per-token input is requested up front (one memory round trip)
    const float vv = bf2f(v[(size_t)t * v_token_stride + h * kGdnDv + v0 + vi]);
    const float gt = g[(size_t)t * kGdnHv + h];
    const float bt = beta[(size_t)t * kGdnHv + h];
    // Full-row sums of squares (every wave computes them redundantly).
    float qa = bf2f(qp[2 * lane]), qb = bf2f(qp[2 * lane + 1]);
    float ka = bf2f(kp[2 * lane]), kb = bf2f(kp[2 * lane + 1]);
    float qss = qa * qa + qb * qb, kss = ka * ka + kb * kb;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      qss += __shfl_xor(qss, o, 64);
      kss += __shfl_xor(kss, o, 64);
    }
    const float qinv = 1.0f / sqrtf(qss + 1e-6f);
    const float kinv = 1.0f / sqrtf(kss + 1e-6f);
    float kr[kRecRows], qr[kRecRows];
    {
      const bf16x8 kv8 = *reinterpret_cast<const bf16x8*>(kp + kq * kRecRows);
      const bf16x8 qv8 = *reinterpret_cast<const bf16x8*>(qp + kq * kRecRows);
#pragma unroll
      for (int j = 0; j < kRecRows; ++j) {
        kr[j] = bf2f(kv8[j]) * kinv;
        qr[j] = (bf2f(qv8[j]) * qinv) * qscale;
      }
    }
    const float eg = expf(gt);
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < kRecRows; ++j) {
      s[j] *= eg;
      part += s[j] * kr[j];
    }
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    const int buf = t & 1;
    if (lane < 16) red[buf][wave][vi] = part;
    lds_barrier();
    const float kv = red[buf][0][vi] + red[buf][1][vi] + red[buf][2][vi] +
                     red[buf][3][vi];
    const float delta = (vv - kv) * bt;
    float op = 0.f;
#pragma unroll
    for (int j = 0; j < kRecRows; ++j) {
      s[j] += kr[j] * delta;
      op += s[j] * qr[j];
    }
    op += __shfl_xor(op, 16, 64);
    op += __shfl_xor(op, 32, 64);
    lds_barrier();  // everyone has read red[buf] for kv
    if (lane < 16) red[buf][wave][vi] = op;
    lds_barrier();
    if (wave == 0 && lane < 16) {
      const float o = red[buf][0][vi] + red[buf][1][vi] + red[buf][2][vi] +
                      red[buf][3][vi];
      out[((size_t)t * kGdnHv + h) * kGdnDv + v0 + vi] = f2bf(o);
    }
  }
#pragma unroll
  for (int j = 0; j < kRecRows; ++j)
    state_out[sbase + (size_t)(kq * kRecRows + j) * kGdnDv] = s[j];
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT int qwen36_gdn_recurrent(const void* q, const void* k, const void* v,
                                    unsigned qk_heads, unsigned qk_token_stride,
                                    unsigned v_token_stride, const void* g,
                                    const void* beta, const void* state_in,
                                    void* state_out, void* out, unsigned tokens,
                                    void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
      beta == nullptr || state_in == nullptr || state_out == nullptr ||
      out == nullptr || tokens == 0 || tokens > kMaxTokens ||
      (qk_heads != 16u && qk_heads != 32u) ||
      qk_token_stride < qk_heads * kGdnDk ||
      v_token_stride < (unsigned)(kGdnHv * kGdnDv))
    return Q36_EINVAL;
  hipLaunchKernelGGL(gdn_recurrent_kernel, dim3(kGdnHv, kGdnDv / kRecVBlock),
                     dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                     static_cast<const bf16*>(v), qk_heads, qk_token_stride,
                     v_token_stride, static_cast<const float*>(g),
                     static_cast<const float*>(beta),
                     static_cast<const float*>(state_in),
                     static_cast<float*>(state_out), static_cast<bf16*>(out),
                     tokens);
  return static_cast<int>(hipGetLastError());
}
