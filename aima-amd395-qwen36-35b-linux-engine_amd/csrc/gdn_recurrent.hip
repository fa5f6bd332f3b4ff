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
// HBM-bound (2 MiB read + 2 MiB write per layer step).  Both reductions of
// a token are done in one round: with kv_old = S^T k and sq_old = S^T q,
//   kv = e^g kv_old,  delta = (v - kv) beta,  o = e^g sq_old + delta (k.q)
// (o = S'^T q expanded), so a token costs one cross-wave exchange.
// grid = 32 heads x 8 blocks of 16 v-columns; thread (rg, cq) owns rows
// 2rg, 2rg+1 and columns 4cq .. 4cq+3 of its block as two float4, so S is
// read once and written once however many tokens are processed, and
// state_in may alias state_out.
#include "common.h"

namespace q36 {
namespace {

constexpr int kRecVBlock = 16;

__global__ __launch_bounds__(256) void gdn_recurrent_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, unsigned qk_heads, unsigned qk_token_stride,
    unsigned v_token_stride, const float* __restrict__ g,
    const float* __restrict__ beta, const float* state_in, float* state_out,
    bf16* __restrict__ out, unsigned tokens) {
  __shared__ f32x4 red[2][4][2][4];   // [parity][wave][kv | sq][col quad]
  const int h = blockIdx.x;
  const int v0 = blockIdx.y * kRecVBlock;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cq = tid & 3, rg = tid >> 2;
  const int r0 = 2 * rg;
  const int kh = h * (int)qk_heads / kGdnHv;
  const size_t sbase = (size_t)h * kGdnDk * kGdnDv + v0 + 4 * cq;

  f32x4 s0 = *reinterpret_cast<const f32x4*>(state_in + sbase + (size_t)r0 * kGdnDv);
  f32x4 s1 = *reinterpret_cast<const f32x4*>(state_in + sbase + (size_t)(r0 + 1) * kGdnDv);

  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  for (unsigned t = 0; t < tokens; ++t) {
    const bf16* qp = q + (size_t)t * qk_token_stride + kh * kGdnDk;
    const bf16* kp = k + (size_t)t * qk_token_stride + kh * kGdnDk;
    // every per-token input is requested up front (one memory round trip)
    const bf16x4 v4 = *reinterpret_cast<const bf16x4*>(
        v + (size_t)t * v_token_stride + h * kGdnDv + v0 + 4 * cq);
    const float gt = g[(size_t)t * kGdnHv + h];
    const float bt = beta[(size_t)t * kGdnHv + h];
    const float qa = bf2f(qp[2 * lane]), qb = bf2f(qp[2 * lane + 1]);
    const float ka = bf2f(kp[2 * lane]), kb = bf2f(kp[2 * lane + 1]);
    const float k0 = bf2f(kp[r0]), k1 = bf2f(kp[r0 + 1]);
    const float q0 = bf2f(qp[r0]), q1 = bf2f(qp[r0 + 1]);
    // partial S^T k and S^T q over this thread's two rows (raw q, k)
    f32x4 pk = s0 * k0 + s1 * k1;
    f32x4 pq = s0 * q0 + s1 * q1;
    // full-row sums (every wave computes them redundantly)
    float qss = qa * qa + qb * qb, kss = ka * ka + kb * kb, kq = qa * ka + qb * kb;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      qss += __shfl_xor(qss, o, 64);
      kss += __shfl_xor(kss, o, 64);
      kq += __shfl_xor(kq, o, 64);
    }
    // reduce the partials over the wave's 16 row groups (lanes with equal cq)
#pragma unroll
    for (int o = 4; o < 64; o <<= 1)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pk[e] += __shfl_xor(pk[e], o, 64);
        pq[e] += __shfl_xor(pq[e], o, 64);
      }
    const int par = t & 1;
    if (lane < 4) {
      red[par][wave][0][cq] = pk;
      red[par][wave][1][cq] = pq;
    }
    lds_barrier();
    const f32x4 kv_raw = red[par][0][0][cq] + red[par][1][0][cq] + red[par][2][0][cq] +
                         red[par][3][0][cq];
    const f32x4 sq_raw = red[par][0][1][cq] + red[par][1][1][cq] + red[par][2][1][cq] +
                         red[par][3][1][cq];
    const float qinv = 1.0f / sqrtf(qss + 1e-6f);
    const float kinv = 1.0f / sqrtf(kss + 1e-6f);
    const float qn = qinv * qscale;
    const float eg = expf(gt);
    const float kqn = (kq * kinv) * qn;
    f32x4 delta, o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float kv = eg * (kv_raw[e] * kinv);
      delta[e] = (bf2f(v4[e]) - kv) * bt;
      o[e] = eg * (sq_raw[e] * qn) + delta[e] * kqn;
    }
    s0 = s0 * eg + delta * (k0 * kinv);
    s1 = s1 * eg + delta * (k1 * kinv);
    if (rg == 0) {
      bf16x4 ob;
#pragma unroll
      for (int e = 0; e < 4; ++e) ob[e] = f2bf(o[e]);
      *reinterpret_cast<bf16x4*>(out + ((size_t)t * kGdnHv + h) * kGdnDv + v0 + 4 * cq) = ob;
    }
  }
  *reinterpret_cast<f32x4*>(state_out + sbase + (size_t)r0 * kGdnDv) = s0;
  *reinterpret_cast<f32x4*>(state_out + sbase + (size_t)(r0 + 1) * kGdnDv) = s1;
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
      v_token_stride < (unsigned)(kGdnHv * kGdnDv) || (v_token_stride % 4) != 0 ||
      (reinterpret_cast<uintptr_t>(v) % 8) != 0 || (reinterpret_cast<uintptr_t>(out) % 8) != 0 ||
      (reinterpret_cast<uintptr_t>(state_in) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(state_out) % 16) != 0)
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
