// Gated-DeltaNet chunked (WY/UT) prefill with an fp32 state.
//
// Restates torch_chunk_gated_delta_rule
// (benchmarks/shape-lab/four_layer_mini_engine.py:5167-5240); the reference
// product runs vLLM FLA Triton code objects for this role
// (native/src/native_linear_prefill.hip.cpp:474-836).  Per v-head h and chunk
// of C = 64 tokens (G = in-chunk cumsum of g; q, k l2-normalised; q scaled by
// 1/sqrt(128)):
//   L   = (k*beta) k^T (.) exp(G_i - G_j), strictly lower
//   T   = (I + L)^-1                     (fle:5207-5211 forward substitution)
//   U   = T (v*beta),  W = T (k*beta*exp(G))
//   Aqk = (q k^T) (.) exp(G_i - G_j), lower incl. diagonal
//   then sequentially over chunks, with the state S [128 k][128 v]:
//   v' = U - W S;  o = (q*exp(G)) S + Aqk v'
//   S  = exp(G_last) S + (k*exp(G_last - G))^T v'
//
// Arithmetic is fp32-accurate on bf16 matrix cores: every fp32 operand x of a
// product is split as x = hi + lo (hi = bf16(x), lo = bf16(x - hi)) and
// x*y ~ hi*hi' + hi*lo' + lo*hi' (relative error ~2^-16), while the raw
// q/k/v inputs are exact in bf16 and enter single-sided (2 products).  The
// l2-norm, beta and decay factors are row/column scalings applied in fp32
// around those products:  k k^T = kinv_i kinv_j (k_raw k_raw^T),
// W = (T diag(beta e^G kinv)) k_raw,  U = (T diag(beta)) v,
// Qg S = diag(qinv e^G / sqrt(128)) (q_raw S),
// Kd^T v' = k_raw^T (diag(kinv e^(G_last - G)) v').
//
// Two kernels:
//  * gdn_chunk_prep (grid = chunks x 32 heads): everything independent of S
//    -- U (fp32), W and Aqk (hi/lo bf16), the two row scales and
//    exp(G_last) -- into the workspace.  T = (I+L)^-1 is formed blockwise:
//    16x16 diagonal blocks by forward substitution, off-diagonal blocks by
//    fp32 MFMA products.  LDS is kept near 72 KB so two workgroups share a CU.
//  * gdn_chunk_scan (grid = 32 heads x 8 groups of 16 v-columns, sequential
//    over chunks): wave w owns token tile w of each chunk and state rows
//    32w .. 32w+31 of its 16 columns, in registers in the MFMA accumulator
//    layout.  That layout is also the B-operand layout of the next products
//    (the reduction index -- state row or token -- is permuted to match, and
//    prep stores the A operands in the same order, fragment-major), so per
//    chunk only the state tiles and v' (hi/lo bf16) pass through LDS.
#include "common.h"

#include <algorithm>
#include <mutex>

namespace q36 {
namespace {

constexpr int kC = 64;
constexpr int kPitchR = 136;   // bf16 row pitch (272 B) of [64][128] tiles
constexpr int kPitchT = 72;    // bf16 row pitch (144 B) of transposed tiles
constexpr int kPitchF = 68;    // fp32 row pitch of [64][64] matrices
constexpr float kQScale = 0.08838834764831845f;   // 1/sqrt(128)

// Workspace: one record per (chunk, head).  The matrices the scan consumes
// as MFMA A operands are stored fragment-major (frag_off), so each operand
// is one contiguous 1 KB wave load.
constexpr size_t kOffU = 0;                           // fp32 [4 tt][8 cg][64 lane][4]
constexpr size_t kOffWh = kOffU + 64 * 128 * 4;       // bf16 frag [64][128]
constexpr size_t kOffWl = kOffWh + 64 * 128 * 2;
constexpr size_t kOffAh = kOffWl + 64 * 128 * 2;      // bf16 frag [64][64]
constexpr size_t kOffAl = kOffAh + 64 * 64 * 2;
constexpr size_t kOffRsq = kOffAl + 64 * 64 * 2;      // fp32 [64]
constexpr size_t kOffRsk = kOffRsq + 256;             // fp32 [64]
constexpr size_t kOffEgl = kOffRsk + 256;             // fp32 [1]
constexpr size_t kOffKt = kOffEgl + 256;              // bf16 frag [128][64] k_raw^T
constexpr size_t kOffQ = kOffKt + 128 * 64 * 2;       // bf16 frag [64][128] q_raw
constexpr size_t kUnitBytes = kOffQ + 64 * 128 * 2;
struct Unit {
  float* U;
  bf16* Wh;
  bf16* Wl;
  bf16* Ah;
  bf16* Al;
  float* rsq;
  float* rsk;
  float* egl;
  bf16* kt;
  bf16* q;
};

__device__ __forceinline__ Unit unit_at(char* ws, size_t unit) {
  char* b = ws + unit * kUnitBytes;
  return Unit{reinterpret_cast<float*>(b + kOffU), reinterpret_cast<bf16*>(b + kOffWh),
              reinterpret_cast<bf16*>(b + kOffWl), reinterpret_cast<bf16*>(b + kOffAh),
              reinterpret_cast<bf16*>(b + kOffAl), reinterpret_cast<float*>(b + kOffRsq),
              reinterpret_cast<float*>(b + kOffRsk), reinterpret_cast<float*>(b + kOffEgl),
              reinterpret_cast<bf16*>(b + kOffKt),
              reinterpret_cast<bf16*>(b + kOffQ)};
}

__device__ __forceinline__ void split2(float x, bf16& h, bf16& l) {
  h = f2bf(x);
  l = f2bf(x - bf2f(h));
}

__device__ __forceinline__ float rsqrt_rn(float x) {
  return (float)(1.0 / sqrt((double)x));
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

// Element offset of M[row][col] in the fragment-major layout of a matrix
// with nkb blocks of 32 reduction columns: [row/16][col/32][lane][8].  Lane
// 16g + row%16 holds columns 4g..4g+3 and 16+4g..16+4g+3 of its block (the
// accumulator row order of two stacked 16x16 tiles, which is how the scan's
// B operands arrive), so an A operand is 16 contiguous bytes per lane.
__device__ __forceinline__ int frag_off(int row, int col, int nkb) {
  const int c = col & 31, a = c >> 4, g = (c >> 2) & 3, r = c & 3;
  return ((((row >> 4) * nkb + (col >> 5)) * 64 + 16 * g + (row & 15)) << 3) + 4 * a + r;
}

// ---------------------------------------------------------------------------
// Phase A
// ---------------------------------------------------------------------------

struct PrepLds {
  // k_raw (row-major) is dead once k k^T is in registers; L reuses its space.
  union {
    bf16 kr[kC * kPitchR];          // k_raw row-major [tok][d]
    float lm[kC * kPitchF];         // L (strictly lower)
  } u;
  bf16 kt[128 * kPitchT];           // k_raw transposed [d][tok]
  bf16 vt[128 * kPitchT];           // v transposed [d][tok]
  float tm[kC * kPitchF];           // T; its upper blocks hold scratch products
  float gs[kC], bs[kC], kinv[kC], qinv[kC], sw[kC];
};

// C = A B for 16x16 fp32 blocks of [64][kPitchF] matrices (v_mfma 16x16x4).
__device__ __forceinline__ f32x4 mm16(const float* a, int ar, int ac,
                                      const float* b, int br, int bc, f32x4 acc,
                                      int li, int kk) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
    acc = mfma16x16x4f32(a[(ar + li) * kPitchF + ac + 4 * s + kk],
                         b[(br + 4 * s + kk) * kPitchF + bc + li], acc);
  return acc;
}

// hi/lo bf16 A operand of row i, columns m0 .. m0+8 of T diag(scale).
__device__ __forceinline__ void t_operand(const float* tm, const float* scale,
                                          int i, int m0, bf16x8& hi, bf16x8& lo) {
  const f32x4 t0 = *reinterpret_cast<const f32x4*>(tm + i * kPitchF + m0);
  const f32x4 t1 = *reinterpret_cast<const f32x4*>(tm + i * kPitchF + m0 + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(scale + m0);
  const f32x4 s1 = *reinterpret_cast<const f32x4*>(scale + m0 + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    bf16 h, l;
    split2(t0[e] * s0[e], h, l);
    hi[e] = h;
    lo[e] = l;
    split2(t1[e] * s1[e], h, l);
    hi[4 + e] = h;
    lo[4 + e] = l;
  }
}

__global__ __launch_bounds__(256, 2) void gdn_chunk_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, unsigned qk_heads, unsigned qk_token_stride,
    unsigned v_token_stride, const float* __restrict__ g,
    const float* __restrict__ beta, unsigned tokens, char* __restrict__ ws, unsigned c0) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PrepLds& s = *reinterpret_cast<PrepLds*>(smem);
  const unsigned c = c0 + blockIdx.x;
  const int h = blockIdx.y;
  const int kh = h * (int)qk_heads / kGdnHv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const unsigned tok0 = c * kC;
  const Unit un = unit_at(ws, (size_t)c * kGdnHv + h);

  // S1. rows -> LDS (row-major k; transposed k, v); l2 norms of k and q.
  {
    const int r = tid >> 2, p = tid & 3;
    const unsigned tok = tok0 + r;
    const bool valid = tok < tokens;
    bf16x8 k8[4], q8[4], v8[4];
    if (valid) {
      const bf16* kp = k + (size_t)tok * qk_token_stride + kh * kGdnDk + 32 * p;
      const bf16* qp = q + (size_t)tok * qk_token_stride + kh * kGdnDk + 32 * p;
      const bf16* vp = v + (size_t)tok * v_token_stride + h * kGdnDv + 32 * p;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        k8[i] = ld8(kp + 8 * i);
        q8[i] = ld8(qp + 8 * i);
        v8[i] = ld8(vp + 8 * i);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) k8[i] = q8[i] = v8[i] = bf16x8{};
    }
    float kss = 0.f, qss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<bf16x8*>(&s.u.kr[r * kPitchR + 32 * p + 8 * i]) = k8[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float kx = bf2f(k8[i][e]), qx = bf2f(q8[i][e]);
        kss += kx * kx;
        qss += qx * qx;
        s.kt[(32 * p + 8 * i + e) * kPitchT + r] = k8[i][e];
        s.vt[(32 * p + 8 * i + e) * kPitchT + r] = v8[i][e];
      }
    }
    // q_raw fragments (tile r/16, column block p) for the scan
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const bf16x8 x = q8[g4 >> 1], y = q8[2 + (g4 >> 1)];
      const int o = 4 * (g4 & 1);
      *reinterpret_cast<bf16x8*>(un.q + ((((r >> 4) * 4 + p) * 64 + 16 * g4 + (r & 15)) << 3)) =
          bf16x8{x[o], x[o + 1], x[o + 2], x[o + 3], y[o], y[o + 1], y[o + 2], y[o + 3]};
    }
    kss += __shfl_xor(kss, 1, 64);
    kss += __shfl_xor(kss, 2, 64);
    qss += __shfl_xor(qss, 1, 64);
    qss += __shfl_xor(qss, 2, 64);
    if (p == 0) {
      s.kinv[r] = rsqrt_rn(kss + 1e-6f);
      s.qinv[r] = rsqrt_rn(qss + 1e-6f);
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
    un.egl[0] = expf(acc);
  }

  // S2. raw k k^T and q k^T on the 10 lower 16x16 tiles (bf16 MFMA: exact
  // products of the raw inputs); q fragments come straight from global.
  f32x4 acc_job[5];
#pragma unroll
  for (int jj = 0; jj < 5; ++jj) {
    const int job = wave + 4 * jj;
    const bool is_q = job >= 10;
    int t = is_q ? job - 10 : job;
    int rt = 0;
    while (t > rt) { t -= rt + 1; ++rt; }
    const int ct = t;
    const bf16* brow = s.u.kr + (16 * ct + li) * kPitchR + 8 * lg;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (is_q) {
      const unsigned tok = tok0 + 16 * rt + li;
      const bf16* qrow = q + (size_t)tok * qk_token_stride + kh * kGdnDk + 8 * lg;
#pragma unroll
      for (int st = 0; st < 4; ++st)   // transposed: D[j][i] = k_j . q_i
        acc = mfma16x16x32(ld8(brow + 32 * st), tok < tokens ? ld8(qrow + 32 * st) : bf16x8{}, acc);
    } else {
      const bf16* arow = s.u.kr + (16 * rt + li) * kPitchR + 8 * lg;
#pragma unroll
      for (int st = 0; st < 4; ++st) acc = mfma16x16x32(ld8(arow + 32 * st), ld8(brow + 32 * st), acc);
    }
    acc_job[jj] = acc;
  }
  __syncthreads();  // k_raw row-major no longer needed; cumsum visible
  if (tid < kC) {
    const int r = tid;
    const float eg = expf(s.gs[r]);
    un.rsq[r] = (s.qinv[r] * kQScale) * eg;
    un.rsk[r] = s.kinv[r] * expf(s.gs[kC - 1] - s.gs[r]);
    s.sw[r] = (s.bs[r] * eg) * s.kinv[r];
  }
#pragma unroll
  for (int jj = 0; jj < 5; ++jj) {
    const int job = wave + 4 * jj;
    const bool is_q = job >= 10;
    int t = is_q ? job - 10 : job;
    int rt = 0;
    while (t > rt) { t -= rt + 1; ++rt; }
    const int ct = t;
    if (is_q) {
      // lane holds Aqk[i][j] for i = 16rt + li, j = 16ct + 4lg + r: exactly
      // half of its A-operand fragment (column block ct/2, half ct%2)
      const int i = 16 * rt + li;
      bf16x4 vh, vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * ct + 4 * lg + r;
        const float decay = j <= i ? expf(s.gs[i] - s.gs[j]) : 0.f;
        const float a = j <= i ? (((s.qinv[i] * kQScale) * s.kinv[j]) * acc_job[jj][r]) * decay : 0.f;
        bf16 ah, al;
        split2(a, ah, al);
        vh[r] = ah;
        vl[r] = al;
      }
      const int o = frag_off(i, 16 * ct + 4 * lg, 2);
      *reinterpret_cast<bf16x4*>(un.Ah + o) = vh;
      *reinterpret_cast<bf16x4*>(un.Al + o) = vl;
    } else {
      const int j = 16 * ct + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * rt + 4 * lg + r;
        const float decay = j <= i ? expf(s.gs[i] - s.gs[j]) : 0.f;
        s.u.lm[i * kPitchF + j] =
            j < i ? (((s.kinv[i] * s.kinv[j]) * acc_job[jj][r]) * s.bs[i]) * decay : 0.f;
      }
    }
  }
  // zero the strictly-upper 16x16 tiles of L and T, and of the stored Aqk
  for (int idx = tid; idx < kC * kC; idx += 256) {
    const int i = idx >> 6, j = idx & 63;
    if ((j >> 4) > (i >> 4)) {
      s.u.lm[i * kPitchF + j] = 0.f;
      s.tm[i * kPitchF + j] = 0.f;
    }
  }
  for (int idx = tid; idx < 6 * 64; idx += 256) {   // 6 upper tiles x 64 lanes
    const int t = idx >> 6, ln = idx & 63;
    const int rt = t < 3 ? 0 : (t < 5 ? 1 : 2);
    const int ct = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3);
    const int o = frag_off(16 * rt + (ln & 15), 16 * ct + 4 * (ln >> 4), 2);
    *reinterpret_cast<bf16x4*>(un.Ah + o) = bf16x4{};
    *reinterpret_cast<bf16x4*>(un.Al + o) = bf16x4{};
  }
  __syncthreads();

  // S3. diagonal 16x16 blocks of T = (I + L)^-1: wave b inverts block b,
  // lane j < 16 owns column j (forward substitution, as fle:5207-5211).
  if (li == lane) {
    const int b = wave, j = lane;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc += s.u.lm[(16 * b + i) * kPitchF + 16 * b + m] * t[m];
      t[i] = i == j ? 1.f : (i > j ? -acc : 0.f);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) s.tm[(16 * b + i) * kPitchF + 16 * b + j] = t[i];
  }
  __syncthreads();
  // S4. off-diagonal blocks by distance d: T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj.
  // The intermediate sum is parked in the (still zero) upper block (j, i).
  for (int d = 1; d < 4; ++d) {
    const int bj = wave, bi = wave + d;
    if (bi < 4) {
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      for (int kb = bj; kb < bi; ++kb)
        x = mm16(s.u.lm, 16 * bi, 16 * kb, s.tm, 16 * kb, 16 * bj, x, li, lg);
#pragma unroll
      for (int r = 0; r < 4; ++r) s.tm[(16 * bj + 4 * lg + r) * kPitchF + 16 * bi + li] = x[r];
      // the same wave reads its own LDS writes back in order
      f32x4 y = mm16(s.tm, 16 * bi, 16 * bi, s.tm, 16 * bj, 16 * bi,
                     f32x4{0.f, 0.f, 0.f, 0.f}, li, lg);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s.tm[(16 * bi + 4 * lg + r) * kPitchF + 16 * bj + li] = -y[r];
        s.tm[(16 * bj + 4 * lg + r) * kPitchF + 16 * bi + li] = 0.f;
      }
    }
    __syncthreads();
  }

  // S5. U = (T diag beta) v, W = (T diag(beta e^G kinv)) k_raw; wave w takes
  // the 16-column tiles 2w, 2w+1 of both.  The hi/lo A operands are formed
  // on the fly; T is lower triangular, so the second 32-token step is skipped
  // for the first two row tiles.
  const int col0 = 32 * wave + li;   // ct = 2w: col0, ct = 2w+1: col0 + 16
  for (int rt = 0; rt < 4; ++rt) {
    f32x4 au[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    f32x4 aw[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const int nst = rt < 2 ? 1 : 2;
    for (int st = 0; st < nst; ++st) {
      bf16x8 tuh, tul, twh, twl;
      t_operand(s.tm, s.bs, 16 * rt + li, 32 * st + 8 * lg, tuh, tul);
      t_operand(s.tm, s.sw, 16 * rt + li, 32 * st + 8 * lg, twh, twl);
#pragma unroll
      for (int ctl = 0; ctl < 2; ++ctl) {
        const int col = col0 + 16 * ctl;
        const bf16x8 bv = ld8(s.vt + col * kPitchT + 32 * st + 8 * lg);
        const bf16x8 bk = ld8(s.kt + col * kPitchT + 32 * st + 8 * lg);
        au[ctl] = mfma16x16x32(tuh, bv, au[ctl]);
        au[ctl] = mfma16x16x32(tul, bv, au[ctl]);
        aw[ctl] = mfma16x16x32(bk, twh, aw[ctl]);   // transposed: W^T
        aw[ctl] = mfma16x16x32(bk, twl, aw[ctl]);
      }
    }
#pragma unroll
    for (int ctl = 0; ctl < 2; ++ctl) {
      const int col = col0 + 16 * ctl;
      reinterpret_cast<f32x4*>(un.U)[(rt * 8 + (col >> 4)) * 64 + 16 * lg + li] = au[ctl];
    }
    // aw[ctl][r] = W[16rt + li][32w + 16ctl + 4lg + r]: together the whole
    // A-operand fragment (row tile rt, column block w) of lane 16lg + li
    bf16x8 wh, wl;
#pragma unroll
    for (int ctl = 0; ctl < 2; ++ctl)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bf16 h, l;
        split2(aw[ctl][r], h, l);
        wh[4 * ctl + r] = h;
        wl[4 * ctl + r] = l;
      }
    const int fo = ((rt * 4 + wave) * 64 + 16 * lg + li) * 8;
    *reinterpret_cast<bf16x8*>(un.Wh + fo) = wh;
    *reinterpret_cast<bf16x8*>(un.Wl + fo) = wl;
  }
  // k_raw^T (fragment-major) for the scan's state update.
  for (int idx = tid; idx < 128 * 8; idx += 256) {
    const int row = idx >> 3, ch = idx & 7, t2 = ch >> 2, g4 = ch & 3;
    const bf16* src = s.kt + row * kPitchT + 32 * t2 + 4 * g4;
    const bf16x4 a = *reinterpret_cast<const bf16x4*>(src);
    const bf16x4 b = *reinterpret_cast<const bf16x4*>(src + 16);
    *reinterpret_cast<bf16x8*>(un.kt + ((((row >> 4) * 2 + t2) * 64 + 16 * g4 + (row & 15)) << 3)) =
        bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
}

// ---------------------------------------------------------------------------
// Phase B
// ---------------------------------------------------------------------------

constexpr int kScanGroups = kGdnDv / 16;   // 16 v-columns per workgroup

struct ScanLds {
  bf16x8 st[8][64];      // [state tile][lane]: S hi (0..3) | lo (4..7)
  bf16x8 vp[4][64][2];   // [token tile][lane]: {v' hi|lo, rsk v' hi|lo}
};

__device__ __forceinline__ bf16x8 split4(const f32x4& x) {
  bf16x8 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    bf16 h, l;
    split2(x[e], h, l);
    out[e] = h;
    out[4 + e] = l;
  }
  return out;
}

// B operands (hi, lo) from two published accumulator tiles.
__device__ __forceinline__ void join_pair(const bf16x8& a, const bf16x8& b,
                                          bf16x8& hi, bf16x8& lo) {
  hi = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  lo = bf16x8{a[4], a[5], a[6], a[7], b[4], b[5], b[6], b[7]};
}

// grid = 256 workgroups (32 heads x 8 groups of 16 v-columns; the 8 groups
// of a head share an XCD, so W/q/Aqk/k^T of a chunk are fetched from HBM once
// per head).  Wave w owns token tile w of every chunk and state tiles 2w,
// 2w+1 (rows 32w .. 32w+31), in the MFMA accumulator layout:
//   sreg[i][r] = S[16(2w+i) + 4lg + r][col].
// Per chunk: every wave publishes its state tiles (hi/lo) to LDS; computes
// v' and q S for its 16 tokens and publishes v'; then forms its tokens'
// outputs and updates its state rows.  Operands come straight from global
// memory in their stored (pre-permuted) order, one chunk ahead.
__global__ __launch_bounds__(256, 1) void gdn_chunk_scan_kernel(
    const char* __restrict__ ws, const float* state_in, float* state_out,
    bf16* __restrict__ out, unsigned tokens, unsigned c_begin, unsigned c_end) {
  __shared__ ScanLds s;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int h = 4 * xcd + (slot >> 3);
  const int cg = slot & 7;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int col = 16 * cg + li;

  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      out, 0, (int)(tokens * kGdnHv * kGdnDv * 2), 0x00020000);
  f32x4 sreg[2];
  const size_t sb = (size_t)h * kGdnDk * kGdnDv + col;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sreg[i][r] = state_in ? state_in[sb + (size_t)(16 * (2 * w + i) + 4 * lg + r) * kGdnDv] : 0.f;

  struct Stage {
    bf16x8 wh[4], wl[4], qa[4], ah[2], al[2], kt[2][2];
    f32x4 u, rsq, rsk;
    float egl;
  };
  auto fetch = [&](unsigned c, Stage& st) {
    const char* b = ws + ((size_t)c * kGdnHv + h) * kUnitBytes;
    const bf16x8* Wh = reinterpret_cast<const bf16x8*>(b + kOffWh) + 256 * w + lane;
    const bf16x8* Wl = reinterpret_cast<const bf16x8*>(b + kOffWl) + 256 * w + lane;
    const bf16x8* Q = reinterpret_cast<const bf16x8*>(b + kOffQ) + 256 * w + lane;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      st.wh[k4] = Wh[64 * k4];
      st.wl[k4] = Wl[64 * k4];
      st.qa[k4] = Q[64 * k4];
    }
    const bf16x8* Ah = reinterpret_cast<const bf16x8*>(b + kOffAh) + 128 * w + lane;
    const bf16x8* Al = reinterpret_cast<const bf16x8*>(b + kOffAl) + 128 * w + lane;
    const bf16x8* Kt = reinterpret_cast<const bf16x8*>(b + kOffKt) + 256 * w + lane;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      st.ah[t2] = Ah[64 * t2];
      st.al[t2] = Al[64 * t2];
      st.kt[0][t2] = Kt[64 * t2];
      st.kt[1][t2] = Kt[128 + 64 * t2];
    }
    st.u = reinterpret_cast<const f32x4*>(b + kOffU)[(8 * w + cg) * 64 + lane];
    st.rsq = *reinterpret_cast<const f32x4*>(b + kOffRsq + 4 * (16 * w + 4 * lg));
    st.rsk = *reinterpret_cast<const f32x4*>(b + kOffRsk + 4 * (16 * w + 4 * lg));
    st.egl = *reinterpret_cast<const float*>(b + kOffEgl);
  };

  auto step = [&](const Stage& st, unsigned c) {
    // publish this wave's state tiles
#pragma unroll
    for (int i = 0; i < 2; ++i) s.st[2 * w + i][lane] = split4(sreg[i]);
    lds_barrier();
    // v' = U - W S and q_raw S for token tile w (reduction over 128 rows)
    f32x4 aw = {0.f, 0.f, 0.f, 0.f}, aq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      bf16x8 shi, slo;
      join_pair(s.st[2 * k4][lane], s.st[2 * k4 + 1][lane], shi, slo);
      aw = mfma16x16x32(st.wh[k4], shi, aw);
      aq = mfma16x16x32(st.qa[k4], shi, aq);
      aw = mfma16x16x32(st.wh[k4], slo, aw);
      aq = mfma16x16x32(st.qa[k4], slo, aq);
      aw = mfma16x16x32(st.wl[k4], shi, aw);
    }
    const f32x4 vp = st.u - aw;
    const f32x4 vz = st.rsk * vp;
    s.vp[w][lane][0] = split4(vp);
    s.vp[w][lane][1] = split4(vz);
    f32x4 acc = st.rsq * aq;
    lds_barrier();
    // o = rsq (q_raw S) + Aqk v'  (Aqk is lower triangular: tiles 0, 1 only
    // need the first 32 tokens)
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      if (t2 == 1 && w < 2) break;
      bf16x8 vh, vl;
      join_pair(s.vp[2 * t2][lane][0], s.vp[2 * t2 + 1][lane][0], vh, vl);
      acc = mfma16x16x32(st.ah[t2], vh, acc);
      acc = mfma16x16x32(st.ah[t2], vl, acc);
      acc = mfma16x16x32(st.al[t2], vh, acc);
    }
    // S = exp(G_last) S + k_raw^T (rsk v')
    f32x4 sn[2] = {sreg[0] * st.egl, sreg[1] * st.egl};
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      bf16x8 zh, zl;
      join_pair(s.vp[2 * t2][lane][1], s.vp[2 * t2 + 1][lane][1], zh, zl);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        sn[i] = mfma16x16x32(st.kt[i][t2], zh, sn[i]);
        sn[i] = mfma16x16x32(st.kt[i][t2], zl, sn[i]);
      }
    }
    sreg[0] = sn[0];
    sreg[1] = sn[1];
    // Output rows past the end fall outside the buffer range and are dropped
    // by the hardware (no branch, so no uncertain store count).
    const unsigned tb = c * kC + 16 * w + 4 * lg;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      __builtin_amdgcn_raw_buffer_store_b16(
          __builtin_bit_cast(unsigned short, f2bf(acc[r])), out_rsrc,
          (int)((((tb + r) * kGdnHv + h) * kGdnDv + col) * 2), 0, 0);
  };

  // Two operand stages alternate (loop unrolled by two): chunk c+1's loads
  // are in flight while chunk c is computed.
  // Two operand stages alternate (loop unrolled by two): chunk c+1's loads
  // are in flight while chunk c is computed.  Fetches past the last chunk
  // re-read it, keeping every fetch unconditional.
  Stage s0, s1;
  const unsigned last = c_end - 1;
  fetch(c_begin, s0);
  for (unsigned c = c_begin; c < c_end; c += 2) {
    fetch(c + 1 < last ? c + 1 : last, s1);
    step(s0, c);
    if (c + 1 >= c_end) break;
    fetch(c + 2 < last ? c + 2 : last, s0);
    step(s1, c + 1);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      state_out[sb + (size_t)(16 * (2 * w + i) + 4 * lg + r) * kGdnDv] = sreg[i][r];
}

// Prep / scan overlap: a second stream and events per device, created on
// first use and kept for the life of the process.
constexpr unsigned kMaxRanges = 8;        // chunk ranges per call
constexpr unsigned kMinRangeChunks = 16;  // below 2 x 16 chunks: one prep + one scan
struct Overlap {
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t done[kMaxRanges] = {};
};
std::mutex g_overlap_mutex;     // one enqueue sequence at a time (shared events)
Overlap g_overlap[64];
bool g_overlap_ready[64] = {};

Overlap* overlap_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  Overlap& o = g_overlap[dev];
  if (!g_overlap_ready[dev]) {
    if (hipStreamCreateWithFlags(&o.side, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&o.fork, hipEventDisableTiming) != hipSuccess) return nullptr;
    for (auto& ev : o.done)
      if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return nullptr;
    g_overlap_ready[dev] = true;
  }
  return &o;
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT size_t qwen36_gdn_chunk_prefill_workspace_bytes(unsigned tokens) {
  const size_t n_chunks = (tokens + kC - 1) / kC;
  return n_chunks * kGdnHv * kUnitBytes;
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
      v_token_stride < (unsigned)(kGdnHv * kGdnDv) ||
      (qk_token_stride % 8) != 0 || (v_token_stride % 8) != 0)
    return Q36_EINVAL;
  const unsigned n_chunks = (tokens + kC - 1) / kC;
  if (workspace_bytes < (size_t)n_chunks * kGdnHv * kUnitBytes) return Q36_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  static std::once_flag attr_once;
  static hipError_t attr_status = hipSuccess;
  std::call_once(attr_once, [] {
    attr_status = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_chunk_prep_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)sizeof(PrepLds));
  });
  if (attr_status != hipSuccess) return (int)attr_status;
  char* wsb = static_cast<char*>(workspace);
  const bf16* qb = static_cast<const bf16*>(q);
  const bf16* kb = static_cast<const bf16*>(k);
  const bf16* vb = static_cast<const bf16*>(v);
  const float* gb = static_cast<const float*>(g);
  const float* bb = static_cast<const float*>(beta);
  float* so = static_cast<float*>(state_out);
  auto prep = [&](unsigned c0, unsigned c1, hipStream_t s) {
    hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(c1 - c0, kGdnHv), dim3(256),
                       sizeof(PrepLds), s, qb, kb, vb, qk_heads, qk_token_stride,
                       v_token_stride, gb, bb, tokens, wsb, c0);
  };
  auto scan = [&](unsigned c0, unsigned c1, const float* sin) {
    hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3(kGdnHv * kScanGroups), dim3(256), 0, st,
                       wsb, sin, so, static_cast<bf16*>(out), tokens, c0, c1);
  };
  const unsigned ranges = std::min(kMaxRanges, n_chunks / kMinRangeChunks);
  if (ranges < 2) {
    prep(0, n_chunks, st);
    scan(0, n_chunks, static_cast<const float*>(state_in));
    return static_cast<int>(hipGetLastError());
  }
  // Prep of chunk range r + 1 overlaps the scan of range r: prep ranges run
  // in order on a second stream, each scan range waits for its prep range's
  // event; the state is carried through state_out.
  std::lock_guard<std::mutex> lock(g_overlap_mutex);
  Overlap* ov = overlap_for_current_device();
  if (ov == nullptr) return Q36_EINVAL;
  hipError_t e = hipEventRecord(ov->fork, st);
  if (e == hipSuccess) e = hipStreamWaitEvent(ov->side, ov->fork, 0);
  if (e != hipSuccess) return (int)e;
  for (unsigned r = 0; r < ranges; ++r) {
    const unsigned c0 = (unsigned)((uint64_t)n_chunks * r / ranges);
    const unsigned c1 = (unsigned)((uint64_t)n_chunks * (r + 1) / ranges);
    prep(c0, c1, ov->side);
    e = hipEventRecord(ov->done[r], ov->side);
    if (e != hipSuccess) return (int)e;
  }
  for (unsigned r = 0; r < ranges; ++r) {
    const unsigned c0 = (unsigned)((uint64_t)n_chunks * r / ranges);
    const unsigned c1 = (unsigned)((uint64_t)n_chunks * (r + 1) / ranges);
    e = hipStreamWaitEvent(st, ov->done[r], 0);
    if (e != hipSuccess) return (int)e;
    scan(c0, c1, r == 0 ? static_cast<const float*>(state_in) : so);
  }
  return static_cast<int>(hipGetLastError());
}
