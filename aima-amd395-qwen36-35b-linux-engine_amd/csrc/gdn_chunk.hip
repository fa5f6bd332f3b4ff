// Gated-DeltaNet chunked (WY/UT) prefill with an fp32 state.
//
// Restates torch_chunk_gated_delta_rule
// (benchmarks/shape-lab/four_layer_mini_engine.py:5167-5240); the reference
// product runs vLLM FLA Triton code objects for this role
// (native/src/native_linear_prefill.hip.cpp:474-836).  Per v-head h and
// chunk c of C = 64 tokens (G = in-chunk cumsum of g, q pre-scaled by
// 1/sqrt(128), q and k l2-normalised):
//   L   = (k*beta) k^T (.) exp(G_i - G_j), strictly lower
//   T   = (I + L)^-1                       (fle:5207-5211 forward substitution)
//   U   = T (v*beta),  W = T (k*beta*exp(G))
//   Aqk = (q k^T) (.) exp(G_i - G_j), lower incl. diagonal
//   then sequentially over chunks, with the state S [128 k][128 v]:
//   v' = U - W S;  o = (q*exp(G)) S + Aqk v'
//   S  = exp(G_last) S + (k*exp(G_last - G))^T v'
//
// Two kernels:
//  * gdn_chunk_prep  (parallel over chunk x head): everything that does not
//    depend on S -- U, W, Qg = q*exp(G), Kd = k*exp(G_last-G), Aqk and
//    exp(G_last) -- written to a workspace.
//  * gdn_chunk_scan  (grid = 32 heads x 8 blocks of 16 v-columns, sequential
//    over chunks): the state slice stays in registers for the whole sequence;
//    each wave owns 32 k-rows of it.
// All matrix products run on v_mfma_f32_16x16x4_f32 so the arithmetic is
// fp32 like the reference (no bf16 rounding of derived operands).
#include "common.h"

namespace q36 {
namespace {

constexpr int kC = 64;            // chunk length
constexpr int kPK = 132;          // LDS pitch (floats) of 64x128 tiles
constexpr int kPT = 68;           // LDS pitch (floats) of 64x64 tiles
constexpr int kScanVB = 16;       // v-columns per scan workgroup

struct PrepLds {
  float kn[kC * kPK];   // normalised k
  float qn[kC * kPK];   // normalised, scaled q
  float vv[kC * kPK];   // raw v
  float lt[kC * kPT];   // L, then T in place
  float aq[kC * kPT];   // Aqk
  float gs[kC];         // in-chunk cumsum of g
  float bs[kC];         // beta
};

__device__ __forceinline__ float rsqrt_rn(float x) {
  return (float)(1.0 / sqrt((double)x));
}

__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, unsigned qk_heads, unsigned qk_token_stride,
    unsigned v_token_stride, const float* __restrict__ g,
    const float* __restrict__ beta, unsigned tokens, float* __restrict__ ws_u,
    float* __restrict__ ws_w, float* __restrict__ ws_qg,
    float* __restrict__ ws_kd, float* __restrict__ ws_aq,
    float* __restrict__ ws_egl) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PrepLds& s = *reinterpret_cast<PrepLds*>(smem);
  const unsigned c = blockIdx.x;
  const int h = blockIdx.y;
  const int kh = h * (int)qk_heads / kGdnHv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const size_t unit = (size_t)c * kGdnHv + h;

  // 1. load + l2-normalise rows: thread -> (row tid/4, dims 32*(tid%4)..+32)
  {
    const int r = tid >> 2, p = tid & 3;
    const unsigned tok = c * kC + r;
    const bool valid = tok < tokens;
    float kx[32], qx[32], vx[32];
    if (valid) {
      const bf16* kp = k + (size_t)tok * qk_token_stride + kh * kGdnDk + 32 * p;
      const bf16* qp = q + (size_t)tok * qk_token_stride + kh * kGdnDk + 32 * p;
      const bf16* vp = v + (size_t)tok * v_token_stride + h * kGdnDv + 32 * p;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8 k8 = reinterpret_cast<const bf16x8*>(kp)[i];
        const bf16x8 q8 = reinterpret_cast<const bf16x8*>(qp)[i];
        const bf16x8 v8 = reinterpret_cast<const bf16x8*>(vp)[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kx[8 * i + e] = bf2f(k8[e]);
          qx[8 * i + e] = bf2f(q8[e]);
          vx[8 * i + e] = bf2f(v8[e]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) kx[i] = qx[i] = vx[i] = 0.f;
    }
    float kss = 0.f, qss = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      kss += kx[i] * kx[i];
      qss += qx[i] * qx[i];
    }
    kss += __shfl_xor(kss, 1, 64);
    kss += __shfl_xor(kss, 2, 64);
    qss += __shfl_xor(qss, 1, 64);
    qss += __shfl_xor(qss, 2, 64);
    const float kinv = rsqrt_rn(kss + 1e-6f);
    const float qinv = rsqrt_rn(qss + 1e-6f);
    const float qscale = 0.08838834764831845f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      s.kn[r * kPK + 32 * p + i] = kx[i] * kinv;
      s.qn[r * kPK + 32 * p + i] = (qx[i] * qinv) * qscale;
      s.vv[r * kPK + 32 * p + i] = vx[i];
    }
    if (p == 0) {
      s.gs[r] = valid ? g[(size_t)tok * kGdnHv + h] : 0.f;
      s.bs[r] = valid ? beta[(size_t)tok * kGdnHv + h] : 0.f;
    }
  }
  __syncthreads();
  if (tid == 0) {  // sequential fp32 cumsum, as torch.cumsum
    float acc = 0.f;
    for (int i = 0; i < kC; ++i) {
      acc += s.gs[i];
      s.gs[i] = acc;
    }
    ws_egl[unit] = expf(acc);
  }
  __syncthreads();

  // 2. Qg and Kd to the workspace (fp32, [unit][64][128]).
  {
    const int r = tid >> 2, p = tid & 3;
    const float eg = expf(s.gs[r]);
    const float ed = expf(s.gs[kC - 1] - s.gs[r]);
    float* qg = ws_qg + (unit * kC + r) * kGdnDk + 32 * p;
    float* kd = ws_kd + (unit * kC + r) * kGdnDk + 32 * p;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
      const float* qs = &s.qn[r * kPK + 32 * p + i];
      const float* ks = &s.kn[r * kPK + 32 * p + i];
      *reinterpret_cast<f32x4*>(qg + i) =
          f32x4{qs[0] * eg, qs[1] * eg, qs[2] * eg, qs[3] * eg};
      *reinterpret_cast<f32x4*>(kd + i) =
          f32x4{ks[0] * ed, ks[1] * ed, ks[2] * ed, ks[3] * ed};
    }
  }

  // 3. K K^T and Q K^T on the 10 lower 16x16 tiles (20 tile jobs, 5/wave).
  const int li = lane & 15, kk = lane >> 4;
  for (int job = wave; job < 20; job += 4) {
    const bool is_q = job >= 10;
    int t = is_q ? job - 10 : job;
    int rt = 0;
    while (t > rt) { t -= rt + 1; ++rt; }
    const int ct = t;
    const float* arow = (is_q ? s.qn : s.kn) + (16 * rt + li) * kPK + kk;
    const float* brow = s.kn + (16 * ct + li) * kPK + kk;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int st = 0; st < kGdnDk / 4; ++st)
      acc = mfma16x16x4f32(arow[4 * st], brow[4 * st], acc);
    // acc[r] = dot(row 16rt + 4kk + r, col 16ct + li)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * rt + 4 * kk + r, j = 16 * ct + li;
      const float decay = j <= i ? expf(s.gs[i] - s.gs[j]) : 0.f;
      if (is_q) {
        s.aq[i * kPT + j] = j <= i ? acc[r] * decay : 0.f;
      } else {
        s.lt[i * kPT + j] = j < i ? (acc[r] * s.bs[i]) * decay : 0.f;
      }
    }
  }
  // zero the strictly-upper 16x16 tiles of both matrices
  for (int idx = tid; idx < kC * kC; idx += 256) {
    const int i = idx >> 6, j = idx & 63;
    if ((j >> 4) > (i >> 4)) {
      s.lt[i * kPT + j] = 0.f;
      s.aq[i * kPT + j] = 0.f;
    }
  }
  __syncthreads();

  // 4. T = (I + L)^-1 by forward substitution, row by row (wave 0, lane = col).
  if (wave == 0) {
    const int j = lane;
    s.lt[0 * kPT + j] = j == 0 ? 1.f : 0.f;
    for (int i = 1; i < kC; ++i) {
      float acc = 0.f;
      // The wave reads all of row i of L before any lane overwrites it: the
      // lanes run the loop in lockstep and LDS operations of one wave retire
      // in order.
      for (int m = 0; m < i; ++m) acc += s.lt[i * kPT + m] * s.lt[m * kPT + j];
      s.lt[i * kPT + j] = j < i ? -acc : (j == i ? 1.f : 0.f);
    }
  }
  __syncthreads();

  // 5. U = T (v*beta), W = T (k*beta*exp(G)); wave w -> column tiles 2w, 2w+1.
  for (int ctl = 0; ctl < 2; ++ctl) {
    const int ct = 2 * wave + ctl;
    const int col = 16 * ct + li;
    for (int rt = 0; rt < 4; ++rt) {
      f32x4 au = {0.f, 0.f, 0.f, 0.f}, aw = {0.f, 0.f, 0.f, 0.f};
      const int nst = 4 * (rt + 1);   // T is lower triangular
      for (int st = 0; st < nst; ++st) {
        const int m = 4 * st + kk;
        const float a = s.lt[(16 * rt + li) * kPT + m];
        const float bm = s.bs[m];
        const float bu = s.vv[m * kPK + col] * bm;
        const float bw = s.kn[m * kPK + col] * (bm * expf(s.gs[m]));
        au = mfma16x16x4f32(a, bu, au);
        aw = mfma16x16x4f32(a, bw, aw);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t o = (unit * kC + 16 * rt + 4 * kk + r) * kGdnDv + col;
        ws_u[o] = au[r];
        ws_w[o] = aw[r];
      }
    }
  }
  // 6. Aqk to the workspace.
  for (int idx = tid; idx < kC * kC; idx += 256)
    ws_aq[unit * kC * kC + idx] = s.aq[(idx >> 6) * kPT + (idx & 63)];
}

// grid = (32 heads, 8 v-blocks); block = 4 waves; wave w owns k-rows
// 32w .. 32w+31 of the state slice S[:, v0 .. v0+16).
__global__ __launch_bounds__(256) void gdn_chunk_scan_kernel(
    const float* __restrict__ ws_u, const float* __restrict__ ws_w,
    const float* __restrict__ ws_qg, const float* __restrict__ ws_kd,
    const float* __restrict__ ws_aq, const float* __restrict__ ws_egl,
    const float* state_in, float* state_out, bf16* __restrict__ out,
    unsigned tokens, unsigned n_chunks) {
  __shared__ float red_v[4][kC][kScanVB];
  __shared__ float red_o[4][kC][kScanVB];
  __shared__ float vp[kC][kScanVB];
  __shared__ float oq[kC][kScanVB];
  const int h = blockIdx.x;
  const int v0 = blockIdx.y * kScanVB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, kk = lane >> 4;

  // S in MFMA C-layout: sreg[kt][r] = S[32w + 16kt + 4kk + r][v0 + li].
  f32x4 sreg[2];
  const size_t sb = (size_t)h * kGdnDk * kGdnDv + v0 + li;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 32 * wave + 16 * kt + 4 * kk + r;
      sreg[kt][r] = state_in ? state_in[sb + (size_t)row * kGdnDv] : 0.f;
    }

  for (unsigned c = 0; c < n_chunks; ++c) {
    const size_t unit = (size_t)c * kGdnHv + h;
    const float* W = ws_w + unit * kC * kGdnDk;
    const float* Qg = ws_qg + unit * kC * kGdnDk;
    const float* Kd = ws_kd + unit * kC * kGdnDk;
    const float* U = ws_u + unit * kC * kGdnDv;
    const float* Aq = ws_aq + unit * kC * kC;
    // a. partial (W S) and (Qg S) over this wave's 32 k-rows.  Reduction
    //    step (kt, r) <-> k = 32w + 16kt + 4kk + r, matching sreg's layout.
    f32x4 pv[4], po[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      pv[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
      po[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int tok = 16 * tt + li;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int kc = 32 * wave + 16 * kt + 4 * kk;
        const f32x4 w4 = *reinterpret_cast<const f32x4*>(W + tok * kGdnDk + kc);
        const f32x4 q4 = *reinterpret_cast<const f32x4*>(Qg + tok * kGdnDk + kc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // B operand: lane (li, kk) supplies S[k(step)][v0 + li]; the step's
          // k for lane group kk is 32w + 16kt + 4kk + r -- exactly sreg[kt][r].
          pv[tt] = mfma16x16x4f32(w4[r], sreg[kt][r], pv[tt]);
          po[tt] = mfma16x16x4f32(q4[r], sreg[kt][r], po[tt]);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red_v[wave][16 * tt + 4 * kk + r][li] = pv[tt][r];
        red_o[wave][16 * tt + 4 * kk + r][li] = po[tt][r];
      }
    }
    __syncthreads();
    // b. reduce over waves: v' = U - W S; o partial = Qg S.
    for (int e = tid; e < kC * kScanVB; e += 256) {
      const int tok = e >> 4, col = e & 15;
      const float ws = red_v[0][tok][col] + red_v[1][tok][col] +
                       red_v[2][tok][col] + red_v[3][tok][col];
      vp[tok][col] = U[tok * kGdnDv + v0 + col] - ws;
      oq[tok][col] = red_o[0][tok][col] + red_o[1][tok][col] +
                     red_o[2][tok][col] + red_o[3][tok][col];
    }
    __syncthreads();
    // c. o rows 16w .. 16w+15 = oq + Aqk v'  (Aqk lower triangular).
    {
      f32x4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = oq[16 * wave + 4 * kk + r][li];
      const int nst = 4 * (wave + 1);
      for (int st = 0; st < nst; ++st) {
        const int m = 4 * st + kk;
        acc = mfma16x16x4f32(Aq[(16 * wave + li) * kC + m], vp[m][li], acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned tok = c * kC + 16 * wave + 4 * kk + r;
        if (tok < tokens)
          out[((size_t)tok * kGdnHv + h) * kGdnDv + v0 + li] = f2bf(acc[r]);
      }
    }
    // d. S = exp(G_last) S + Kd^T v'.
    const float egl = ws_egl[unit];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f32x4 acc = sreg[kt] * egl;
      const int krow = 32 * wave + 16 * kt + li;
#pragma unroll 4
      for (int st = 0; st < kC / 4; ++st) {
        const int m = 4 * st + kk;
        acc = mfma16x16x4f32(Kd[m * kGdnDk + krow], vp[m][li], acc);
      }
      sreg[kt] = acc;
    }
  }
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 32 * wave + 16 * kt + 4 * kk + r;
      state_out[sb + (size_t)row * kGdnDv] = sreg[kt][r];
    }
}

size_t ws_floats(unsigned n_chunks) {
  const size_t units = (size_t)n_chunks * kGdnHv;
  return units * (4 * kC * kGdnDk + kC * kC + 1);
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT size_t qwen36_gdn_chunk_prefill_workspace_bytes(unsigned tokens) {
  const unsigned n_chunks = (tokens + kC - 1) / kC;
  return ws_floats(n_chunks) * sizeof(float);
}

Q36_EXPORT int qwen36_gdn_chunk_prefill(
    const void* q, const void* k, const void* v, unsigned qk_heads,
    unsigned qk_token_stride, unsigned v_token_stride, const void* g,
    const void* beta, const void* state_in, void* state_out, void* out,
    unsigned tokens, void* workspace, size_t workspace_bytes, void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
      beta == nullptr || state_out == nullptr || out == nullptr ||
      workspace == nullptr || tokens == 0 || tokens > kMaxTokens ||
      (qk_heads != 16u && qk_heads != 32u) ||
      qk_token_stride < qk_heads * kGdnDk ||
      v_token_stride < (unsigned)(kGdnHv * kGdnDv))
    return Q36_EINVAL;
  const unsigned n_chunks = (tokens + kC - 1) / kC;
  if (workspace_bytes < ws_floats(n_chunks) * sizeof(float)) return Q36_EINVAL;
  float* base = static_cast<float*>(workspace);
  const size_t big = (size_t)n_chunks * kGdnHv * kC * kGdnDk;
  float* ws_u = base;
  float* ws_w = ws_u + big;
  float* ws_qg = ws_w + big;
  float* ws_kd = ws_qg + big;
  float* ws_aq = ws_kd + big;
  float* ws_egl = ws_aq + (size_t)n_chunks * kGdnHv * kC * kC;
  hipStream_t st = static_cast<hipStream_t>(stream);
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gdn_chunk_prep_kernel),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(PrepLds));
    if (e != hipSuccess) return (int)e;
    attr_set = true;
  }
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(n_chunks, kGdnHv), dim3(256),
                     sizeof(PrepLds), st, static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                     qk_heads, qk_token_stride, v_token_stride,
                     static_cast<const float*>(g),
                     static_cast<const float*>(beta), tokens, ws_u, ws_w, ws_qg,
                     ws_kd, ws_aq, ws_egl);
  hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3(kGdnHv, kGdnDv / kScanVB),
                     dim3(256), 0, st, ws_u, ws_w, ws_qg, ws_kd, ws_aq, ws_egl,
                     static_cast<const float*>(state_in),
                     static_cast<float*>(state_out), static_cast<bf16*>(out),
                     tokens, n_chunks);
  return static_cast<int>(hipGetLastError());
}
