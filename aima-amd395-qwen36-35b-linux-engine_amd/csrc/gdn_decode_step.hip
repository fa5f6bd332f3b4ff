// Fused Gated-DeltaNet decode step: one launch per layer step.
//
// The reference's native decode runs the linear-attention layer as separate
// launches -- the fused input-projection/conv kernel, the post-conv prep and
// fused_sigmoid_gating_delta_rule_update, then the gated RMSNorm
// (native_linear_layer.hip.cpp:84-157; torch form four_layer_mini_engine.py
// :6378-6544).  This kernel does everything between the input projections and
// out_proj for T (>= 1) tokens in one launch:
//   conv:   y = SiLU(conv4([state | x])) per channel, rounded to bf16
//           (fle:5368-5386), new conv state = last three inputs;
//   gating: g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
//           rounded to bf16 (b is bf16 and torch evaluates the sigmoid in
//           its dtype, fle:6507-6511);
//   delta:  q, k <- l2norm; q *= 1/sqrt(128); S <- S e^g; kv = S^T k;
//           delta = (v - kv) beta; S <- S + k (x) delta; o = S^T q
//           (fle:5242-5276), o rounded to bf16;
//   norm:   out = bf16(bf16(rmsnorm_128(o) * w) * SiLU(z)) (fle:6531-6541).
// Numerics follow the unfused kernels (gdn_pointwise.hip, gdn_recurrent.hip)
// term by term; only the order of the S^T k / S^T q partial sums differs.
//
// grid = 32 workgroups, one per v-head, so the head's RMSNorm over its 128
// outputs needs no cross-workgroup step; 512 threads, thread (rg, cq) keeps
// rows 8rg..8rg+7 and columns 4cq..4cq+3 of the head's fp32 state in
// registers across all tokens (state read once, written once; ssm state_in
// may alias state_out).  Both v-heads of a key head read that key head's
// q/k conv channels and the even one writes their new conv state, so the
// conv state must be double-buffered (conv_state_in != conv_state_out).
#include "common.h"

namespace q36 {
namespace {

#ifndef DS_THREADS
#define DS_THREADS 512   // 1024 measured 14% slower (more waves, same per-CU bytes)
#endif
constexpr int kDsThreads = DS_THREADS;
constexpr int kDsWaves = kDsThreads / 64;
constexpr int kDsRowsPerThread = kGdnDk / (kDsThreads / 32);   // row groups of 32 threads

__device__ __forceinline__ float ds_mul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float ds_add(float a, float b) { return __fadd_rn(a, b); }

__global__ __launch_bounds__(kDsThreads) void gdn_decode_step_kernel(
    const bf16* __restrict__ x, unsigned x_row_stride,
    const bf16* __restrict__ conv_w, const bf16* __restrict__ conv_in,
    bf16* __restrict__ conv_out, const bf16* __restrict__ a,
    const bf16* __restrict__ b, unsigned ab_row_stride,
    const float* __restrict__ a_log, const float* __restrict__ dt_bias,
    const bf16* __restrict__ z, unsigned z_row_stride,
    const bf16* __restrict__ norm_w, const float* state_in, float* state_out,
    bf16* __restrict__ out, unsigned tokens) {
  __shared__ float ych[2][3 * kGdnDk];              // [parity][q | k | v] conv outputs
  __shared__ float gb[2][2];                        // [parity][g, beta]
  __shared__ f32x4 red[2][kDsWaves][2][32];         // [parity][wave][kv | sq][col quad]
  const int h = blockIdx.x;
  const int kh = h >> 1;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cq = tid & 31, rg = tid >> 5;
  const int r0 = rg * kDsRowsPerThread;

  // ---- conv channel owned by this thread (threads 0..383) ----------------
  // local 0..127: q of key head kh; 128..255: k of key head kh; 256..383: v.
  // Threads 384.. own no channel and read channel 0's inputs (unused), so
  // every load below is unconditional: all of a token's inputs and the state
  // are requested before any is used (one memory round trip; loads inside
  // divergent branches made the compiler wait at each branch's end).
  const bool conv_thread = tid < 3 * kGdnDk;
  int ch = 0;
  if (tid < kGdnDk) ch = kh * kGdnDk + tid;
  else if (tid < 2 * kGdnDk) ch = kGdnHk * kGdnDk + kh * kGdnDk + (tid - kGdnDk);
  else if (conv_thread) ch = 2 * kGdnHk * kGdnDk + h * kGdnDv + (tid - 2 * kGdnDk);
  const bf16x4 w_raw = *reinterpret_cast<const bf16x4*>(conv_w + ch * kGdnConvK);
  const bf16 h0_raw = conv_in[ch * 3], h1_raw = conv_in[ch * 3 + 1], h2_raw = conv_in[ch * 3 + 2];
  // the first token's inputs: x channel, a and b of this head, z columns
  bf16 x_raw = x[ch];
  bf16 a_raw = a[h], b_raw = b[h];
  bf16x4 z_raw = *reinterpret_cast<const bf16x4*>(z + h * kGdnDv + 4 * cq);

  // ---- state tile --------------------------------------------------------
  const size_t sbase = (size_t)h * kGdnDk * kGdnDv + 4 * cq;
  f32x4 s[kDsRowsPerThread];
#pragma unroll
  for (int i = 0; i < kDsRowsPerThread; ++i)
    s[i] = *reinterpret_cast<const f32x4*>(state_in + sbase + (size_t)(r0 + i) * kGdnDv);
  const float A = expf(a_log[h]);
  const float dtb = dt_bias[h];
  const bf16x4 nw_raw = *reinterpret_cast<const bf16x4*>(norm_w + 4 * cq);
  float w[kGdnConvK], hist[3], nw[4];
#pragma unroll
  for (int i = 0; i < kGdnConvK; ++i) w[i] = bf2f(w_raw[i]);
  hist[0] = bf2f(h0_raw);
  hist[1] = bf2f(h1_raw);
  hist[2] = bf2f(h2_raw);
#pragma unroll
  for (int e = 0; e < 4; ++e) nw[e] = bf2f(nw_raw[e]);

  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  // tokens >= 1 (the entry point rejects 0): a do-while has no guard
  // branch, so the compiler keeps every input load above in the first
  // block instead of sinking them below the guard after the state loads'
  // wait (a second memory round trip)
  unsigned t = 0;
  do {
    const int par = t & 1;
    const float cur = bf2f(x_raw);
    const float av = bf2f(a_raw), bv = bf2f(b_raw);
    const bf16x4 zrow = z_raw;
    // -- phase A: conv + SiLU (bf16-rounded, as the conv kernel), gating --
    if (conv_thread) {
      float acc = ds_mul(hist[0], w[0]);
      acc = ds_add(acc, ds_mul(hist[1], w[1]));
      acc = ds_add(acc, ds_mul(hist[2], w[2]));
      acc = ds_add(acc, ds_mul(cur, w[3]));
      const float cv = bf2f(f2bf(acc));
      ych[par][tid] = bf2f(f2bf(cv / (1.0f + expf(-cv))));
      hist[0] = hist[1];
      hist[1] = hist[2];
      hist[2] = cur;
    } else if (tid == 3 * kGdnDk) {
      const float xs = ds_add(av, dtb);
      const float sp = xs > 20.0f ? xs : log1pf(expf(xs));
      gb[par][0] = ds_mul(-A, sp);
      gb[par][1] = bf2f(f2bf(1.0f / (1.0f + expf(-bv))));   // sigmoid of bf16 b, in bf16
    }
    __syncthreads();
    // request the next token's inputs (this token's are consumed; the last
    // token re-reads its own row, so every load stays in bounds)
    {
      const size_t tn = t + 1 < tokens ? t + 1 : t;
      x_raw = x[tn * x_row_stride + ch];
      a_raw = a[tn * ab_row_stride + h];
      b_raw = b[tn * ab_row_stride + h];
      z_raw = *reinterpret_cast<const bf16x4*>(z + tn * z_row_stride + h * kGdnDv + 4 * cq);
    }
    const float* qv = ych[par];
    const float* kvec = ych[par] + kGdnDk;
    const float* vvec = ych[par] + 2 * kGdnDk;
    // full q/k sums, in the recurrent kernel's lane-pair order
    const float qa = qv[2 * lane], qb = qv[2 * lane + 1];
    const float ka = kvec[2 * lane], kb = kvec[2 * lane + 1];
    float qss = qa * qa + qb * qb, kss = ka * ka + kb * kb, kq = qa * ka + qb * kb;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      qss += __shfl_xor(qss, o, 64);
      kss += __shfl_xor(kss, o, 64);
      kq += __shfl_xor(kq, o, 64);
    }
    // partial S^T k, S^T q over this thread's 8 rows (raw q, k)
    f32x4 pk = {0.f, 0.f, 0.f, 0.f}, pq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kDsRowsPerThread; ++i) {
      pk += s[i] * kvec[r0 + i];
      pq += s[i] * qv[r0 + i];
    }
    // the wave holds row groups 2*wave and 2*wave+1 (lanes l and l^32)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pk[e] += __shfl_xor(pk[e], 32, 64);
      pq[e] += __shfl_xor(pq[e], 32, 64);
    }
    if (lane < 32) {
      red[par][wave][0][cq] = pk;
      red[par][wave][1][cq] = pq;
    }
    __syncthreads();
    f32x4 kv_raw = red[par][0][0][cq], sq_raw = red[par][0][1][cq];
#pragma unroll
    for (int wv = 1; wv < kDsWaves; ++wv) {
      kv_raw += red[par][wv][0][cq];
      sq_raw += red[par][wv][1][cq];
    }
    const float gt = gb[par][0], bt = gb[par][1];
    const float qinv = 1.0f / sqrtf(qss + 1e-6f);
    const float kinv = 1.0f / sqrtf(kss + 1e-6f);
    const float qn = qinv * qscale;
    const float eg = expf(gt);
    const float kqn = (kq * kinv) * qn;
    f32x4 delta, o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float kvv = eg * (kv_raw[e] * kinv);
      delta[e] = (vvec[4 * cq + e] - kvv) * bt;
      o[e] = eg * (sq_raw[e] * qn) + delta[e] * kqn;
    }
#pragma unroll
    for (int i = 0; i < kDsRowsPerThread; ++i) s[i] = s[i] * eg + delta * (kvec[r0 + i] * kinv);
    // -- phase C: gated RMSNorm over the head's 128 outputs (wave 0, lanes
    // 0..31 hold 4 columns each; every row group holds the same o) --
    if (wave == 0) {
      float ob[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ob[e] = bf2f(f2bf(o[e]));
      float ss = ds_add(ds_add(ds_mul(ob[0], ob[0]), ds_mul(ob[1], ob[1])),
                        ds_add(ds_mul(ob[2], ob[2]), ds_mul(ob[3], ob[3])));
      if (lane >= 32) ss = 0.f;
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) ss = ds_add(ss, __shfl_xor(ss, off, 64));
      const float inv = (float)(1.0 / sqrt((double)ds_add(ds_mul(ss, 1.0f / 128.0f), 1e-6f)));
      if (lane < 32) {
        bf16x4 res;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float nv = bf2f(f2bf(ds_mul(ds_mul(ob[e], inv), nw[e])));
          const float zv = bf2f(zrow[e]);
          const float silu = zv / (1.0f + expf(-zv));
          res[e] = f2bf(ds_mul(nv, silu));
        }
        *reinterpret_cast<bf16x4*>(out + (size_t)t * (kGdnHv * kGdnDv) + h * kGdnDv + 4 * cq) = res;
      }
    }
  } while (++t < tokens);
#pragma unroll
  for (int i = 0; i < kDsRowsPerThread; ++i)
    *reinterpret_cast<f32x4*>(state_out + sbase + (size_t)(r0 + i) * kGdnDv) = s[i];
  if (conv_thread && (tid >= 2 * kGdnDk || (h & 1) == 0)) {
#pragma unroll
    for (int j = 0; j < 3; ++j) conv_out[ch * 3 + j] = f2bf(hist[j]);
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

static bool ranges_overlap(const void* p, const void* q, size_t n) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
  return a < b + n && b < a + n;
}

Q36_EXPORT int qwen36_gdn_decode_step(
    const void* mixed_qkv, unsigned x_row_stride, const void* conv_weight,
    const void* conv_state_in, void* conv_state_out, const void* a,
    const void* b, unsigned ab_row_stride, const void* a_log,
    const void* dt_bias, const void* z, unsigned z_row_stride,
    const void* norm_weight, const void* state_in, void* state_out, void* out,
    unsigned tokens, void* stream) {
  const size_t conv_bytes = (size_t)kGdnConvDim * 3 * sizeof(bf16);
  if (mixed_qkv == nullptr || conv_weight == nullptr || conv_state_in == nullptr ||
      conv_state_out == nullptr || a == nullptr || b == nullptr || a_log == nullptr ||
      dt_bias == nullptr || z == nullptr || norm_weight == nullptr ||
      state_in == nullptr || state_out == nullptr || out == nullptr || tokens == 0 ||
      tokens > kMaxTokens || x_row_stride < (unsigned)kGdnConvDim ||
      ab_row_stride < (unsigned)kGdnHv || z_row_stride < (unsigned)(kGdnHv * kGdnDv) ||
      (z_row_stride % 4) != 0 || ranges_overlap(conv_state_in, conv_state_out, conv_bytes) ||
      (reinterpret_cast<uintptr_t>(z) % 8) != 0 || (reinterpret_cast<uintptr_t>(out) % 8) != 0 ||
      (reinterpret_cast<uintptr_t>(state_in) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(state_out) % 16) != 0)
    return Q36_EINVAL;
  hipLaunchKernelGGL(gdn_decode_step_kernel, dim3(kGdnHv), dim3(kDsThreads), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(mixed_qkv), x_row_stride,
                     static_cast<const bf16*>(conv_weight),
                     static_cast<const bf16*>(conv_state_in),
                     static_cast<bf16*>(conv_state_out), static_cast<const bf16*>(a),
                     static_cast<const bf16*>(b), ab_row_stride,
                     static_cast<const float*>(a_log), static_cast<const float*>(dt_bias),
                     static_cast<const bf16*>(z), z_row_stride,
                     static_cast<const bf16*>(norm_weight),
                     static_cast<const float*>(state_in), static_cast<float*>(state_out),
                     static_cast<bf16*>(out), tokens);
  return static_cast<int>(hipGetLastError());
}
