// Pointwise pieces of the gated full-attention layer.
//
//  * qwen36_rotary_table      -- fp32 cos/sin of (position * inv_freq[i]),
//    i < 32 (native_pointwise.hip.cpp:224-238; four_layer_mini_engine.py
//    :4470-4471, :4489-4498).
//  * qwen36_head_norm_rope    -- per-head RMSNorm with the (w + 1) weight,
//    then rotate-half RoPE on dims [0, 64), for the 16 query heads and the 2
//    key heads; K and the raw V are written straight into the cache rows
//    [position_start, position_start + T) (native_pointwise.hip.cpp:242-337,
//    four_layer_mini_engine.py:5151-5162, :5980-5986).
//  * qwen36_output_gate       -- attn * sigmoid(gate) with the gate read from
//    the fused [Q | Gate] q-projection rows (native_pointwise.hip.cpp:207-222
//    for bf16 attention, :339-359 for fp32 attention; fle:6650).
//
// Rounding points follow the eager PyTorch text: every fp32 product and sum
// that the reference materialises is rounded separately (no contraction).
#include "common.h"

#include <mutex>

namespace q36 {
namespace {

// 1 / 1e7^(2i/64), i = 0..31, each correctly rounded to fp32.
__constant__ float c_inv_freq[kRotaryPairs];

__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }

__global__ void rotary_table_kernel(float* __restrict__ cosv,
                                    float* __restrict__ sinv, unsigned tokens,
                                    unsigned position_start) {
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * kRotaryPairs) return;
  const unsigned t = i / kRotaryPairs, pair = i % kRotaryPairs;
  const float angle = mul_rn((float)(position_start + t), c_inv_freq[pair]);
  cosv[i] = cosf(angle);
  sinv[i] = sinf(angle);
}

// grid = (T, 18): y < 16 -> query head y, else key head y - 16.  block = 64;
// lane holds dims 4*lane .. 4*lane+3 (lanes 0-7: [0,32), lanes 8-15: [32,64)).
__global__ __launch_bounds__(64) void head_norm_rope_kernel(
    const bf16* __restrict__ q_gate, unsigned q_row_stride,
    const bf16* __restrict__ k_raw, unsigned k_row_stride,
    const bf16* __restrict__ v_raw, unsigned v_row_stride,
    const bf16* __restrict__ q_weight, const bf16* __restrict__ k_weight,
    unsigned position_start, bf16* __restrict__ q_out,
    bf16* __restrict__ k_cache, bf16* __restrict__ v_cache) {
  const unsigned t = blockIdx.x;
  const int hsel = blockIdx.y;
  const bool is_q = hsel < kHq;
  const int head = is_q ? hsel : hsel - kHq;
  const int lane = threadIdx.x;
  const bf16* src = is_q ? q_gate + (size_t)t * q_row_stride + head * 2 * kD
                         : k_raw + (size_t)t * k_row_stride + head * kD;
  const bf16* w = is_q ? q_weight : k_weight;

  float x[4], y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = bf2f(src[4 * lane + e]);
  float cs[4], sn[4];
  rope_cos_sin_wave(position_start + t, c_inv_freq, cs, sn);
  head_norm_rope_wave(x, w, cs, sn, y);
  const size_t pos = position_start + t;
  bf16* dst = is_q ? q_out + ((size_t)t * kHq + head) * kD
                   : k_cache + (pos * kHkv + head) * kD;
#pragma unroll
  for (int e = 0; e < 4; ++e) dst[4 * lane + e] = f2bf(y[e]);
  if (!is_q) {
    const bf16* vs = v_raw + (size_t)t * v_row_stride + head * kD;
    bf16* vd = v_cache + (pos * kHkv + head) * kD;
#pragma unroll
    for (int e = 0; e < 4; ++e) vd[4 * lane + e] = vs[4 * lane + e];
  }
}

// One wave per token (block = 4 tokens): the token's 16 query heads and 2
// key heads through the same per-head arithmetic as head_norm_rope_kernel,
// with the RoPE cos/sin and the (w + 1) factors formed once per wave and
// every input row requested up front (8-byte pieces per lane).
__global__ __launch_bounds__(256) void head_norm_rope_rows_kernel(
    const bf16* __restrict__ q_gate, unsigned q_row_stride,
    const bf16* __restrict__ k_raw, unsigned k_row_stride,
    const bf16* __restrict__ v_raw, unsigned v_row_stride,
    const bf16* __restrict__ q_weight, const bf16* __restrict__ k_weight,
    unsigned position_start, bf16* __restrict__ q_out,
    bf16* __restrict__ k_cache, bf16* __restrict__ v_cache, unsigned tokens) {
  const unsigned t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;   // wave-uniform
  const int lane = threadIdx.x & 63;
  bf16x4 xin[kHq + kHkv], vin[kHkv];
#pragma unroll
  for (int h = 0; h < kHq; ++h)
    xin[h] = *reinterpret_cast<const bf16x4*>(q_gate + (size_t)t * q_row_stride + h * 2 * kD + 4 * lane);
#pragma unroll
  for (int h = 0; h < kHkv; ++h) {
    xin[kHq + h] = *reinterpret_cast<const bf16x4*>(k_raw + (size_t)t * k_row_stride + h * kD + 4 * lane);
    vin[h] = *reinterpret_cast<const bf16x4*>(v_raw + (size_t)t * v_row_stride + h * kD + 4 * lane);
  }
  float wq[4], wk[4], cs[4], sn[4];
  head_norm_wp1(q_weight, wq);
  head_norm_wp1(k_weight, wk);
  rope_cos_sin_wave(position_start + t, c_inv_freq, cs, sn);
  const size_t pos = position_start + t;
#pragma unroll
  for (int h = 0; h < kHq + kHkv; ++h) {
    float x[4], y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = bf2f(xin[h][e]);
    head_norm_rope_wave_wp1(x, h < kHq ? wq : wk, cs, sn, y);
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f2bf(y[e]);
    bf16* dst = h < kHq ? q_out + ((size_t)t * kHq + h) * kD
                        : k_cache + (pos * kHkv + (h - kHq)) * kD;
    *reinterpret_cast<bf16x4*>(dst + 4 * lane) = o;
  }
#pragma unroll
  for (int h = 0; h < kHkv; ++h)
    *reinterpret_cast<bf16x4*>(v_cache + (pos * kHkv + h) * kD + 4 * lane) = vin[h];
}

template <bool kF32>
__global__ void output_gate_kernel(const void* __restrict__ attn,
                                   const bf16* __restrict__ q_gate,
                                   unsigned q_row_stride, bf16* __restrict__ out,
                                   unsigned tokens) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)tokens * kQDim) return;
  const size_t t = i / kQDim;
  const int f = (int)(i - t * kQDim);
  const int head = f / kD, d = f % kD;
  const float a = kF32 ? static_cast<const float*>(attn)[i]
                       : bf2f(static_cast<const bf16*>(attn)[i]);
  out[i] = gate_bf16(a, q_gate[t * q_row_stride + head * 2 * kD + kD + d]);
}

std::mutex g_freq_mutex;   // first calls may come from several host threads
bool g_freq_ready[64] = {};

int ensure_inv_freq() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(g_freq_mutex);
  if (g_freq_ready[dev]) return Q36_OK;
  float h[kRotaryPairs];
  rope_inv_freq_host(h);
  const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(c_inv_freq), h, sizeof(h));
  if (e != hipSuccess) return (int)e;
  g_freq_ready[dev] = true;
  return Q36_OK;
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT int qwen36_rotary_table(float* cosv, float* sinv, unsigned tokens,
                                   unsigned position_start, void* stream) {
  if (cosv == nullptr || sinv == nullptr || tokens == 0 ||
      (size_t)position_start + tokens > kMaxTokens)
    return Q36_EINVAL;
  const int st = ensure_inv_freq();
  if (st != Q36_OK) return st;
  const unsigned n = tokens * kRotaryPairs;
  hipLaunchKernelGGL(rotary_table_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), cosv, sinv, tokens,
                     position_start);
  return static_cast<int>(hipGetLastError());
}

Q36_EXPORT int qwen36_head_norm_rope(
    const void* q_gate, unsigned q_row_stride, const void* k_raw,
    unsigned k_row_stride, const void* v_raw, unsigned v_row_stride,
    const void* q_weight, const void* k_weight, unsigned tokens,
    unsigned position_start, void* q_out, void* k_cache, void* v_cache,
    void* stream) {
  if (q_gate == nullptr || k_raw == nullptr || v_raw == nullptr ||
      q_weight == nullptr || k_weight == nullptr || q_out == nullptr ||
      k_cache == nullptr || v_cache == nullptr || tokens == 0 ||
      (size_t)position_start + tokens > kMaxTokens ||
      q_row_stride < 2 * kQDim || k_row_stride < kKvRow ||
      v_row_stride < kKvRow)
    return Q36_EINVAL;
  const int st = ensure_inv_freq();
  if (st != Q36_OK) return st;
  const auto a8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; };
  // One wave per token needs long prompts to fill the GPU; shorter ones run
  // one wave per (token, head).  Graph-replayed on MI355X, rows form vs
  // per-head form: T = 512 10.4 vs 5.2 us, 1024 11.3 vs 7.9, 2048 14.1 vs
  // 12.5, 4096 21.1 vs 22.0, 8192 33.1 vs 41.4 (bit-identical forms).
  constexpr unsigned kRowsFormMinTokens = 3072;
  if (tokens >= kRowsFormMinTokens && a8(q_gate) && a8(k_raw) && a8(v_raw) && a8(q_out) && a8(k_cache) && a8(v_cache) &&
      (q_row_stride % 4) == 0 && (k_row_stride % 4) == 0 && (v_row_stride % 4) == 0) {
    hipLaunchKernelGGL(head_norm_rope_rows_kernel, dim3((tokens + 3) / 4), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const bf16*>(q_gate),
                       q_row_stride, static_cast<const bf16*>(k_raw), k_row_stride,
                       static_cast<const bf16*>(v_raw), v_row_stride,
                       static_cast<const bf16*>(q_weight), static_cast<const bf16*>(k_weight),
                       position_start, static_cast<bf16*>(q_out), static_cast<bf16*>(k_cache),
                       static_cast<bf16*>(v_cache), tokens);
    return static_cast<int>(hipGetLastError());
  }
  hipLaunchKernelGGL(head_norm_rope_kernel, dim3(tokens, kHq + kHkv), dim3(64),
                     0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(q_gate), q_row_stride,
                     static_cast<const bf16*>(k_raw), k_row_stride,
                     static_cast<const bf16*>(v_raw), v_row_stride,
                     static_cast<const bf16*>(q_weight),
                     static_cast<const bf16*>(k_weight), position_start,
                     static_cast<bf16*>(q_out), static_cast<bf16*>(k_cache),
                     static_cast<bf16*>(v_cache));
  return static_cast<int>(hipGetLastError());
}

Q36_EXPORT int qwen36_output_gate(const void* attn, int attn_is_f32,
                                  const void* q_gate, unsigned q_row_stride,
                                  void* out, unsigned tokens, void* stream) {
  if (attn == nullptr || q_gate == nullptr || out == nullptr || tokens == 0 ||
      q_row_stride < 2 * kQDim)
    return Q36_EINVAL;
  const size_t n = (size_t)tokens * kQDim;
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (attn_is_f32)
    hipLaunchKernelGGL(output_gate_kernel<true>, grid, dim3(256), 0, st, attn,
                       static_cast<const bf16*>(q_gate), q_row_stride,
                       static_cast<bf16*>(out), tokens);
  else
    hipLaunchKernelGGL(output_gate_kernel<false>, grid, dim3(256), 0, st, attn,
                       static_cast<const bf16*>(q_gate), q_row_stride,
                       static_cast<bf16*>(out), tokens);
  return static_cast<int>(hipGetLastError());
}
