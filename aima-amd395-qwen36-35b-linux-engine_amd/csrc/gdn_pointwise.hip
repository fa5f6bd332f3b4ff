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

constexpr int kConvTokensPerThread = 8;

// grid = (C/256, ceil(T/8)); thread = one channel, 8 consecutive tokens.
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

// Vector form of gdn_conv1d_kernel (16-byte loads and stores, the same
// conv arithmetic; SiLU through silu_fast with the exact form where it could
// differ, so the same bits for every finite input): grid = (C/2048,
// ceil(T/TPT)); thread = 8 consecutive channels, TPT consecutive tokens.
// Two load orders (MI355X, graph-replayed):
//  * kUpfront: every row and the state requested unconditionally before
//    the first use (the first block's three history rows read row 0 and
//    are replaced by the state at use) -- one memory round trip, for short
//    prompts, where few waves are resident (TPT = 4: T = 512 7.3 us,
//    1024 11.6, 2048 18.4, 4096 30.8);
//  * otherwise each row behind its own (tok >= 0) test, which costs a round
//    trip per row but keeps fewer registers live -- at T = 8192 the
//    occupancy hides the latency (TPT = 8: 54 us; 16: 63, 4: 66, 32: 76;
//    the up-front form there: 57.6-59.6 us).
template <int TPT, bool kUpfront>
__global__ __launch_bounds__(256) void gdn_conv1d_vec_kernel(
    const bf16* __restrict__ x, unsigned x_row_stride,
    const bf16* __restrict__ weight, const bf16* __restrict__ state_in,
    bf16* __restrict__ state_out, bf16* __restrict__ out, unsigned tokens) {
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  const unsigned t0 = blockIdx.y * TPT;
  float w[8][kGdnConvK];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16x8 wv = *reinterpret_cast<const bf16x8*>(weight + c0 * kGdnConvK + 8 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) w[2 * i + e / 4][e % 4] = bf2f(wv[e]);
  }
  // window rows t0-3 .. t0-1 (from the state before the first token), then
  // the thread's TPT rows (rows past the end re-read the last row, not stored)
  bf16x8 rows[3 + TPT];
  bf16 st[24] = {};
  if constexpr (kUpfront) {
    const bf16x8* sp = reinterpret_cast<const bf16x8*>(state_in + c0 * 3);
    const bf16x8 a = sp[0], b = sp[1], c = sp[2];
#pragma unroll
    for (int j = 0; j < 3 + TPT; ++j) {
      const int tok = (int)t0 - 3 + j;
      const unsigned tc = min((unsigned)max(tok, 0), tokens - 1);
      rows[j] = *reinterpret_cast<const bf16x8*>(x + (size_t)tc * x_row_stride + c0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      st[e] = a[e];
      st[8 + e] = b[e];
      st[16 + e] = c[e];
    }
  } else {
    if (blockIdx.y == 0) {   // only the first token block reads the state
      const bf16x8* sp = reinterpret_cast<const bf16x8*>(state_in + c0 * 3);
      const bf16x8 a = sp[0], b = sp[1], c = sp[2];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        st[e] = a[e];
        st[8 + e] = b[e];
        st[16 + e] = c[e];
      }
    }
#pragma unroll
    for (int j = 0; j < 3 + TPT; ++j) {
      const int tok = (int)t0 - 3 + j;
      if (tok >= 0) {
        const unsigned tc = min((unsigned)tok, tokens - 1);
        rows[j] = *reinterpret_cast<const bf16x8*>(x + (size_t)tc * x_row_stride + c0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) rows[j][e] = st[e * 3 + (tok + 3)];
      }
    }
  }
  // row j's value of channel e (up-front: the first block's history rows
  // come from the state)
  const bool from_state = kUpfront && blockIdx.y == 0;
  auto val = [&](int j, int e) {
    return (j < 3 && from_state) ? bf2f(st[e * 3 + j]) : bf2f(rows[j][e]);
  };
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const unsigned t = t0 + j;
    // SiLU from the hardware exp2 / rcp; the exact form only where the fast
    // value could round to another bf16 (one branch per row of 8)
    float cv[8], sv[8];
    bool slow = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = mul_rn(val(j, e), w[e][0]);
      acc = add_rn(acc, mul_rn(val(j + 1, e), w[e][1]));
      acc = add_rn(acc, mul_rn(val(j + 2, e), w[e][2]));
      acc = add_rn(acc, mul_rn(val(j + 3, e), w[e][3]));
      cv[e] = bf2f(f2bf(acc));
      bool sl;
      sv[e] = silu_fast(cv[e], sl);
      slow |= sl;
    }
    if (slow) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bool sl;
        silu_fast(cv[e], sl);
        if (sl) sv[e] = cv[e] / (1.0f + expf(-cv[e]));
      }
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f2bf(sv[e]);
    if (t < tokens) *reinterpret_cast<bf16x8*>(out + (size_t)t * kGdnConvDim + c0) = o;
  }
  // The first token block owns the state update (state_in may alias
  // state_out: this thread read its state above).
  if (blockIdx.y == 0) {
    bf16 ns[24];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int tok = (int)tokens - 3 + j;
      bf16x8 r;
      if (tok >= 0) {
        r = *reinterpret_cast<const bf16x8*>(x + (size_t)tok * x_row_stride + c0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = st[e * 3 + (tok + 3)];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ns[e * 3 + j] = r[e];
    }
    bf16x8* dp = reinterpret_cast<bf16x8*>(state_out + c0 * 3);
#pragma unroll
    for (int v8 = 0; v8 < 3; ++v8) {
      bf16x8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = ns[8 * v8 + e];
      dp[v8] = r;
    }
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

// Vector form of gdn_gated_norm_kernel: thread = 8 dims of one (token,
// v-head) row, 16 threads per row, 16 rows per block; 16-byte loads and
// stores.  The sum of squares is reduced in the scalar kernel's exact order
// (its lane 4s + i holds this thread's pair i; its xor-32 .. xor-4 steps
// are xor 8 .. 1 here, its xor-2 and xor-1 steps pair the thread's own
// partials), so the bits are the same.
__global__ __launch_bounds__(256) void gdn_gated_norm_vec_kernel(
    const bf16* __restrict__ core, const bf16* __restrict__ z,
    unsigned z_row_stride, const bf16* __restrict__ weight,
    bf16* __restrict__ out, unsigned rows) {
  const unsigned row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const bool live = row < rows;
  const unsigned rr = live ? row : rows - 1;
  const unsigned t = rr / kGdnHv, h = rr % kGdnHv;
  const bf16x8 xv = *reinterpret_cast<const bf16x8*>(core + (size_t)rr * kGdnDv + 8 * sub);
  const bf16x8 zv = *reinterpret_cast<const bf16x8*>(z + (size_t)t * z_row_stride + h * kGdnDv + 8 * sub);
  const bf16x8 wv = *reinterpret_cast<const bf16x8*>(weight + 8 * sub);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = bf2f(xv[2 * i]), x1 = bf2f(xv[2 * i + 1]);
    p[i] = add_rn(mul_rn(x0, x0), mul_rn(x1, x1));
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1)
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = add_rn(p[i], __shfl_xor(p[i], o, 16));
  const float sum = add_rn(add_rn(p[0], p[2]), add_rn(p[1], p[3]));
  const float inv = rsqrt_rn(add_rn(mul_rn(sum, 1.0f / 128.0f), 1e-6f));
  bf16x8 o8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float nv = bf2f(f2bf(mul_rn(mul_rn(bf2f(xv[e]), inv), bf2f(wv[e]))));
    const float zf = bf2f(zv[e]);
    const float silu = zf / (1.0f + expf(-zf));
    o8[e] = f2bf(mul_rn(nv, silu));
  }
  if (live)
    *reinterpret_cast<bf16x8*>(out + (size_t)t * (kGdnHv * kGdnDv) + h * kGdnDv + 8 * sub) = o8;
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
  const unsigned tblocks = (tokens + kConvTokensPerThread - 1) / kConvTokensPerThread;
  const bool vec = aligned16(x) && aligned16(weight) && aligned16(state_in) &&
                   aligned16(state_out) && aligned16(out) && (x_row_stride % 8) == 0;
  if (vec) {
    // short prompts: 4 tokens per thread, every load up front (see the kernel)
    const bool short_form = tokens <= 4096u;
    const unsigned tpt = short_form ? 4u : 8u;
    auto kernel = short_form ? gdn_conv1d_vec_kernel<4, true> : gdn_conv1d_vec_kernel<8, false>;
    hipLaunchKernelGGL(kernel, dim3(kGdnConvDim / 2048, (tokens + tpt - 1) / tpt), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const bf16*>(x),
                       x_row_stride, static_cast<const bf16*>(weight),
                       static_cast<const bf16*>(state_in), static_cast<bf16*>(state_out),
                       static_cast<bf16*>(out), tokens);
    return static_cast<int>(hipGetLastError());
  }
  const dim3 grid(kGdnConvDim / 256, tblocks);
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
  if (aligned16(core) && aligned16(z) && aligned16(weight) && aligned16(out) &&
      (z_row_stride % 8) == 0) {
    hipLaunchKernelGGL(gdn_gated_norm_vec_kernel, dim3((rows + 15) / 16), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const bf16*>(core),
                       static_cast<const bf16*>(z), z_row_stride,
                       static_cast<const bf16*>(weight), static_cast<bf16*>(out), rows);
    return static_cast<int>(hipGetLastError());
  }
  hipLaunchKernelGGL(gdn_gated_norm_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(core), static_cast<const bf16*>(z),
                     z_row_stride, static_cast<const bf16*>(weight),
                     static_cast<bf16*>(out), rows);
  return static_cast<int>(hipGetLastError());
}
