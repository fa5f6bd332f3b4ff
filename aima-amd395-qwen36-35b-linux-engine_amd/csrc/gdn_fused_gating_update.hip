// Gated-DeltaNet decode update in vLLM's orientation, with the gating fused:
// the role of fused_sigmoid_gating_delta_rule_update, which the reference's
// decode calls at four_layer_mini_engine.py:6429-6440 (vLLM
// 0.19.1rc1.dev300+g29e5d1020; the native engine launches the same kernel,
// native_linear_layer.hip.cpp:84-95).  Per token t and value head j (key
// head j * qk_heads / 32):
//   g = -exp(A_log) * softplus(a + dt_bias)  (linear above 20)
//   beta = sigmoid(b)                         (fp32)
//   q, k <- x * rsqrt(sum x^2 + 1e-6) when l2-normalising; q *= scale
//   H <- H e^g;  v' = (v - H k) beta;  H <- H + v' (x) k;  o = H q
// with H = the head's fp32 state stored [Hv][dv][dk] (row v holds the
// 128 key columns contiguously; the transpose of the torch rule's state).
//
// In this orientation every state row evolves on its own: the two
// reductions of a token (H k, H q) run along a row, so a row is owned by 8
// lanes (16 key columns each) and reduced by three shuffles, with no LDS and
// no barrier.  The squared norms of q and k and q.k come out of the same
// shuffles (the 8 lanes of a row cover all 128 key columns), and
// o = e^g (H_old q) + v' (k.q) (H' q expanded) keeps one reduction round per
// token.  grid = 32 heads x 8 blocks of 16 rows; 128 threads; the state is
// read once and written once per call (state_out may alias state_in).
#include "common.h"

namespace q36 {
namespace {

constexpr int kFguRows = 16;                    // state rows per workgroup
constexpr int kFguLanesPerRow = 8;
constexpr int kFguCols = kGdnDk / kFguLanesPerRow;   // 16 key columns per lane

__global__ __launch_bounds__(kFguRows * kFguLanesPerRow) void gdn_fused_gating_update_kernel(
    const float* __restrict__ a_log, const bf16* __restrict__ a,
    const bf16* __restrict__ b, unsigned ab_row_stride,
    const float* __restrict__ dt_bias, const bf16* __restrict__ q,
    const bf16* __restrict__ k, unsigned qk_heads, unsigned qk_token_stride,
    const bf16* __restrict__ v, unsigned v_token_stride, const float* state_in,
    float* state_out, bf16* __restrict__ out, unsigned tokens, float scale,
    bool l2norm, const int* __restrict__ cu_seqlens, const int* __restrict__ state_indices,
    unsigned n_slots) {
  const int h = blockIdx.x;
  const unsigned seq = blockIdx.z;
  unsigned t_begin = 0, t_end = tokens;
  size_t slot = 0;
  if (gridDim.z > 1 || cu_seqlens != nullptr || state_indices != nullptr) {
    if (cu_seqlens != nullptr) {
      t_begin = (unsigned)max(cu_seqlens[seq], 0);
      t_end = min((unsigned)max(cu_seqlens[seq + 1], 0), tokens);
    } else {
      t_begin = seq;
      t_end = seq + 1;
    }
    const int sl = state_indices != nullptr ? state_indices[seq] : (int)seq;
    if (sl < 0 || (unsigned)sl >= n_slots || t_begin >= t_end) return;   // padding
    slot = (size_t)sl * kGdnHv * kGdnDv * kGdnDk;
  }
  state_in += slot;
  state_out += slot;
  const int row = blockIdx.y * kFguRows + (threadIdx.x / kFguLanesPerRow);
  const int part = threadIdx.x % kFguLanesPerRow;
  const int c0 = part * kFguCols;
  const int kh = h * (int)qk_heads / kGdnHv;
  float* so = state_out + ((size_t)h * kGdnDv + row) * kGdnDk + c0;
  const float* si = state_in + ((size_t)h * kGdnDv + row) * kGdnDk + c0;
  float s[kFguCols];
#pragma unroll
  for (int i = 0; i < kFguCols; i += 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(si + i);
    s[i] = x[0]; s[i + 1] = x[1]; s[i + 2] = x[2]; s[i + 3] = x[3];
  }
  const float A = expf(a_log[h]);
  const float dtb = dt_bias[h];
  for (unsigned t = t_begin; t < t_end; ++t) {
    // every per-token input is requested up front (one memory round trip)
    const bf16x8* qp = reinterpret_cast<const bf16x8*>(q + (size_t)t * qk_token_stride + kh * kGdnDk + c0);
    const bf16x8* kp = reinterpret_cast<const bf16x8*>(k + (size_t)t * qk_token_stride + kh * kGdnDk + c0);
    const bf16x8 q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
    const float vv = bf2f(v[(size_t)t * v_token_stride + h * kGdnDv + row]);
    const float av = bf2f(a[(size_t)t * ab_row_stride + h]);
    const float bv = bf2f(b[(size_t)t * ab_row_stride + h]);
    float qf[kFguCols], kf[kFguCols];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qf[i] = bf2f(q0[i]); qf[8 + i] = bf2f(q1[i]);
      kf[i] = bf2f(k0[i]); kf[8 + i] = bf2f(k1[i]);
    }
    float hk = 0.f, hq = 0.f, kk = 0.f, qq = 0.f, kq = 0.f;
#pragma unroll
    for (int i = 0; i < kFguCols; ++i) {
      hk += s[i] * kf[i];
      hq += s[i] * qf[i];
      kk += kf[i] * kf[i];
      qq += qf[i] * qf[i];
      kq += kf[i] * qf[i];
    }
#pragma unroll
    for (int o = 1; o < kFguLanesPerRow; o <<= 1) {
      hk += __shfl_xor(hk, o, 64);
      hq += __shfl_xor(hq, o, 64);
      kk += __shfl_xor(kk, o, 64);
      qq += __shfl_xor(qq, o, 64);
      kq += __shfl_xor(kq, o, 64);
    }
    const float xs = av + dtb;
    const float sp = xs > 20.0f ? xs : log1pf(expf(xs));
    const float eg = expf(-A * sp);
    const float beta = 1.0f / (1.0f + expf(-bv));
    const float kinv = l2norm ? 1.0f / sqrtf(kk + 1e-6f) : 1.0f;
    const float qn = (l2norm ? 1.0f / sqrtf(qq + 1e-6f) : 1.0f) * scale;
    const float vn = (vv - eg * (hk * kinv)) * beta;
    const float o = eg * (hq * qn) + vn * ((kq * kinv) * qn);
    const float vk = vn * kinv;
#pragma unroll
    for (int i = 0; i < kFguCols; ++i) s[i] = s[i] * eg + vk * kf[i];
    if (part == 0) out[((size_t)t * kGdnHv + h) * kGdnDv + row] = f2bf(o);
  }
#pragma unroll
  for (int i = 0; i < kFguCols; i += 4)
    *reinterpret_cast<f32x4*>(so + i) = f32x4{s[i], s[i + 1], s[i + 2], s[i + 3]};
}

}  // namespace
}  // namespace q36

using namespace q36;

namespace {
int fgu_launch(const void* a_log, const void* a, const void* b, unsigned ab_row_stride,
               const void* dt_bias, const void* q, const void* k, unsigned qk_heads,
               unsigned qk_token_stride, const void* v, unsigned v_token_stride,
               const void* state_in, void* state_out, void* out, unsigned tokens,
               const int* cu_seqlens, const int* state_indices, unsigned n_seqs,
               unsigned n_slots, float scale, unsigned flags, void* stream) {
  if (a_log == nullptr || a == nullptr || b == nullptr || dt_bias == nullptr ||
      q == nullptr || k == nullptr || v == nullptr || state_in == nullptr ||
      state_out == nullptr || out == nullptr || tokens == 0 || tokens > kMaxTokens ||
      n_seqs == 0 || n_seqs > 65535u || n_slots == 0 ||
      (qk_heads != 16u && qk_heads != 32u) || ab_row_stride < (unsigned)kGdnHv ||
      qk_token_stride < qk_heads * kGdnDk || (qk_token_stride % 8) != 0 ||
      v_token_stride < (unsigned)(kGdnHv * kGdnDv) || (flags & ~1u) != 0 ||
      !(scale > 0.f) ||
      (reinterpret_cast<uintptr_t>(q) % 16) != 0 || (reinterpret_cast<uintptr_t>(k) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(state_in) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(state_out) % 16) != 0)
    return Q36_EINVAL;
  hipLaunchKernelGGL(gdn_fused_gating_update_kernel,
                     dim3(kGdnHv, kGdnDv / kFguRows, n_seqs), dim3(kFguRows * kFguLanesPerRow), 0,
                     static_cast<hipStream_t>(stream), static_cast<const float*>(a_log),
                     static_cast<const bf16*>(a), static_cast<const bf16*>(b), ab_row_stride,
                     static_cast<const float*>(dt_bias), static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), qk_heads, qk_token_stride,
                     static_cast<const bf16*>(v), v_token_stride,
                     static_cast<const float*>(state_in), static_cast<float*>(state_out),
                     static_cast<bf16*>(out), tokens, scale, (flags & 1u) != 0, cu_seqlens,
                     state_indices, n_slots);
  return static_cast<int>(hipGetLastError());
}
}  // namespace

Q36_EXPORT int qwen36_gdn_fused_gating_update(
    const void* a_log, const void* a, const void* b, unsigned ab_row_stride,
    const void* dt_bias, const void* q, const void* k, unsigned qk_heads,
    unsigned qk_token_stride, const void* v, unsigned v_token_stride,
    const void* state_in, void* state_out, void* out, unsigned tokens,
    float scale, unsigned flags, void* stream) {
  return fgu_launch(a_log, a, b, ab_row_stride, dt_bias, q, k, qk_heads, qk_token_stride, v,
                    v_token_stride, state_in, state_out, out, tokens, nullptr, nullptr, 1u, 1u,
                    scale, flags, stream);
}

Q36_EXPORT int qwen36_gdn_fused_gating_update_varlen(
    const void* a_log, const void* a, const void* b, unsigned ab_row_stride,
    const void* dt_bias, const void* q, const void* k, unsigned qk_heads,
    unsigned qk_token_stride, const void* v, unsigned v_token_stride,
    const void* state_in, void* state_out, void* out, unsigned tokens,
    const void* cu_seqlens, const void* state_indices, unsigned n_seqs, unsigned n_slots,
    float scale, unsigned flags, void* stream) {
  if (cu_seqlens == nullptr && n_seqs != tokens) return Q36_EINVAL;
  return fgu_launch(a_log, a, b, ab_row_stride, dt_bias, q, k, qk_heads, qk_token_stride, v,
                    v_token_stride, state_in, state_out, out, tokens,
                    static_cast<const int*>(cu_seqlens), static_cast<const int*>(state_indices),
                    n_seqs, n_slots, scale, flags, stream);
}
