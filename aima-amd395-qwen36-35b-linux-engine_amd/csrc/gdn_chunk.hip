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
// The decomposition used by the two kernels below:
//   W S = T diag(beta e^G kinv) (k_raw S)   and   U = T diag(beta) v, so
//   v' = U - W S = (T diag(beta)) (v - diag(e^G kinv) (k_raw S)),
//   Aqk = diag(qinv / sqrt(128)) (q_raw k_raw^T) diag(kinv) (.) exp(G_i - G_j).
//
// Two kernels:
//  * gdn_chunk_prep (grid = chunks x 32 heads): the state-independent part
//    that is sequential inside a chunk -- T = (I+L)^-1, formed blockwise
//    (16x16 diagonal blocks by forward substitution, off-diagonal blocks by
//    fp32 MFMA products) -- stored as T diag(beta) in hi/lo bf16 A-operand
//    fragments, Aqk in the same form, and the chunk's per-token scalars (G,
//    kinv, q scale, row scales, exp(G_last)): a 34,560-byte record per
//    (chunk, head).
//  * gdn_chunk_scan (grid = 32 heads x 8 groups of 16 v-columns, sequential
//    over chunks, 12 waves in three roles): producer waves stage each
//    chunk's q and k rows (read straight from the inputs) and scalars into
//    LDS a chunk ahead; chain wave w owns token tile w of each chunk and
//    state rows 32w .. 32w+31 of its 16 columns, in registers in the MFMA
//    accumulator layout, and carries the recurrence; output wave w forms
//    token tile w's output from the published state and v'.  The
//    accumulator layout is also the B-operand layout of the next products
//    (the reduction index -- state row or token -- is permuted to match, and
//    the A operands are read in the same order), so per chunk only the state
//    tiles, (v - ..) and v' (hi/lo bf16) pass between waves through LDS.
#include "common.h"

#include <mutex>

namespace q36 {
namespace {

constexpr int kC = 64;
// qwen36_gdn_chunk_prefill_ex flags (same values as the public header's)
constexpr unsigned kFlagQkNormalized = 1u;   // q, k already l2-normalised
constexpr unsigned kFlagStateVk = 2u;        // states in [Hv, dv, dk] order

constexpr int kPitchR = 136;   // bf16 row pitch (272 B) of [64][128] tiles
constexpr int kPitchF = 68;    // fp32 row pitch of [64][64] matrices
constexpr float kQScale = 0.08838834764831845f;   // 1/sqrt(128)

// Workspace: one record per (chunk, head): T diag(beta) as hi/lo bf16 A
// operands, fragment-major (frag_off, two 32-token blocks), the per-token
// scalars as [kNsc][64] fp32, and Aqk as hi/lo A operands (same layout).
constexpr size_t kOffTh = 0;
constexpr size_t kOffTl = kOffTh + 64 * 64 * 2;
constexpr size_t kOffSc = kOffTl + 64 * 64 * 2;
enum {
  kScG = 0,   // G = in-chunk cumsum of g
  kScKin,     // kinv = 1 / |k|
  kScQs,      // qinv / sqrt(128)
  kScCy,      // e^G kinv: row scale of k_raw S
  kScRsq,     // qinv e^G / sqrt(128): row scale of q_raw S
  kScRsk,     // kinv e^(G_last - G): row scale of v' in the state update
  kScEgl,     // [0] = e^(G_last)
  kNsc
};
constexpr size_t kOffAh = kOffSc + kNsc * 64 * 4;  // bf16 frag [64][64] Aqk hi
constexpr size_t kOffAl = kOffAh + 64 * 64 * 2;     //                  Aqk lo
constexpr size_t kUnitBytes = kOffAl + 64 * 64 * 2;
static_assert(kUnitBytes % 256 == 0, "records stay 256-byte aligned");

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
  float tm[kC * kPitchF];           // T; its upper blocks hold scratch products
  float gs[kC], bs[kC], kinv[kC], qinv[kC];
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

// Lower-triangular 16x16 tile t (0..9) of a 64x64 matrix, row-major over
// the tiles: row tile rt, column tile ct <= rt.
__device__ __forceinline__ int tri_row(int t) { return (t >= 1) + (t >= 3) + (t >= 6); }
__device__ __forceinline__ int tri_col(int t) {
  const int rt = tri_row(t);
  return t - rt * (rt + 1) / 2;
}

__global__ __launch_bounds__(256, 2) void gdn_chunk_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, unsigned qk_heads,
    unsigned qk_token_stride, const float* __restrict__ g,
    const float* __restrict__ beta, unsigned tokens, char* __restrict__ ws, unsigned c0,
    bool l2norm) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  PrepLds& s = *reinterpret_cast<PrepLds*>(smem);
  const unsigned c = c0 + blockIdx.x;
  const int h = blockIdx.y;
  const int kh = h * (int)qk_heads / kGdnHv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const unsigned tok0 = c * kC;
  char* rec = ws + ((size_t)c * kGdnHv + h) * kUnitBytes;
  bf16* th = reinterpret_cast<bf16*>(rec + kOffTh);
  bf16* tl = reinterpret_cast<bf16*>(rec + kOffTl);
  float* sc = reinterpret_cast<float*>(rec + kOffSc);

  // Every input load is unconditional and issued up front (one memory
  // round trip): rows past the last token read as zeros through the buffer
  // ranges, g and beta are read at a clamped row and zeroed.
  const unsigned rows = min((unsigned)kC, tokens - tok0);
  const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(q) + (size_t)tok0 * qk_token_stride + kh * kGdnDk, 0,
      (int)(rows * qk_token_stride * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(k) + (size_t)tok0 * qk_token_stride + kh * kGdnDk, 0,
      (int)(rows * qk_token_stride * 2), 0x00020000);
  auto ldq = [&](const __amdgpu_buffer_rsrc_t& rs, int row, int col) {
    return __builtin_bit_cast(
        bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((row * qk_token_stride + col) * 2), 0, 0));
  };
  // q fragments of this wave's q k^T jobs (jobs 10..19: jj = 2 for waves 2
  // and 3, jj = 3, 4 for every wave)
  bf16x8 qpre[3][4];
#pragma unroll
  for (int jq = 0; jq < 3; ++jq) {
    const int job = wave + 4 * (jq + 2);
    const int rt = tri_row(job >= 10 ? job - 10 : 0);
#pragma unroll
    for (int st = 0; st < 4; ++st) qpre[jq][st] = ldq(qrs, 16 * rt + li, 8 * lg + 32 * st);
  }

  // S1 inputs: this thread's k and q row pieces, g and beta.  All loads
  // are in flight before any is used (the sched_barrier keeps the compiler
  // from deferring the q fragments behind the first waits: a second round
  // trip).
  const int r1 = tid >> 2, p1 = tid & 3;
  const unsigned tok1 = tok0 + r1;
  const bool valid1 = tok1 < tokens;
  const unsigned tcl1 = valid1 ? tok1 : tokens - 1;
  const float gval = g[(size_t)tcl1 * kGdnHv + h], bval = beta[(size_t)tcl1 * kGdnHv + h];
  bf16x8 k8[4], q8[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k8[i] = ldq(krs, r1, 32 * p1 + 8 * i);
    q8[i] = ldq(qrs, r1, 32 * p1 + 8 * i);
  }
  __builtin_amdgcn_sched_barrier(0);

  // S1. k rows -> LDS; l2 norms of k and q; g, beta.
  {
    const int r = r1, p = p1;
    const bool valid = valid1;
    float kss = 0.f, qss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<bf16x8*>(&s.u.kr[r * kPitchR + 32 * p + 8 * i]) = k8[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float kx = bf2f(k8[i][e]), qx = bf2f(q8[i][e]);
        kss += kx * kx;
        qss += qx * qx;
      }
    }
    kss += __shfl_xor(kss, 1, 64);
    kss += __shfl_xor(kss, 2, 64);
    qss += __shfl_xor(qss, 1, 64);
    qss += __shfl_xor(qss, 2, 64);
    if (p == 0) {   // q, k already unit-norm (vLLM's use_qk_l2norm_in_kernel=False): 1
      s.kinv[r] = l2norm ? rsqrt_rn(kss + 1e-6f) : 1.f;
      s.qinv[r] = l2norm ? rsqrt_rn(qss + 1e-6f) : 1.f;
    }
    // written by all four lanes of the row (the same value), so the g and
    // beta loads are not sunk into a branch behind the first waits
    s.gs[r] = valid ? gval : 0.f;
    s.bs[r] = valid ? bval : 0.f;
  }
  lds_barrier();
  if (tid == 0) {  // sequential fp32 cumsum, as torch.cumsum (in registers)
    f32x4 gv[kC / 4];
#pragma unroll
    for (int i = 0; i < kC / 4; ++i) gv[i] = reinterpret_cast<const f32x4*>(s.gs)[i];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kC / 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc += gv[i][e];
        gv[i][e] = acc;
      }
#pragma unroll
    for (int i = 0; i < kC / 4; ++i) reinterpret_cast<f32x4*>(s.gs)[i] = gv[i];
    sc[kScEgl * 64] = expf(acc);
  }

  // S2. raw k k^T and q k^T on the 10 lower 16x16 tiles each (bf16 MFMA:
  // exact products of the raw inputs); q fragments come straight from global.
  f32x4 acc_job[5];
#pragma unroll
  for (int jj = 0; jj < 5; ++jj) {
    const int job = wave + 4 * jj;
    const bool is_q = job >= 10;
    const int t = is_q ? job - 10 : job;
    const int rt = tri_row(t), ct = tri_col(t);
    const bf16* brow = s.u.kr + (16 * ct + li) * kPitchR + 8 * lg;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (is_q) {
#pragma unroll
      for (int st = 0; st < 4; ++st)   // transposed: D[j][i] = k_j . q_i
        acc = mfma16x16x32(ld8(brow + 32 * st), qpre[jj >= 2 ? jj - 2 : 0][st], acc);
    } else {
      const bf16* arow = s.u.kr + (16 * rt + li) * kPitchR + 8 * lg;
#pragma unroll
      for (int st = 0; st < 4; ++st) acc = mfma16x16x32(ld8(arow + 32 * st), ld8(brow + 32 * st), acc);
    }
    acc_job[jj] = acc;
  }
  lds_barrier();  // k_raw row-major no longer needed; cumsum visible
  if (tid < kC) {
    const int r = tid;
    const float eg = expf(s.gs[r]);
    const float qs = s.qinv[r] * kQScale;
    sc[kScG * 64 + r] = s.gs[r];
    sc[kScKin * 64 + r] = s.kinv[r];
    sc[kScQs * 64 + r] = qs;
    sc[kScCy * 64 + r] = eg * s.kinv[r];
    sc[kScRsq * 64 + r] = qs * eg;
    sc[kScRsk * 64 + r] = s.kinv[r] * expf(s.gs[kC - 1] - s.gs[r]);
  }
  bf16* ah = reinterpret_cast<bf16*>(rec + kOffAh);
  bf16* al = reinterpret_cast<bf16*>(rec + kOffAl);
#pragma unroll
  for (int jj = 0; jj < 5; ++jj) {
    const int job = wave + 4 * jj;
    const bool is_q = job >= 10;
    const int t = is_q ? job - 10 : job;
    const int rt = tri_row(t), ct = tri_col(t);
    // Branch-free: every LDS scalar the four elements use is read first (one
    // vector read per row of scalars), the decays of entries past the
    // diagonal are computed and discarded by the selects (a select, not a
    // product, so an infinite exp2 there cannot leak).
    if (is_q) {
      // lane holds Aqk[i][j] for i = 16rt + li, j = 16ct + 4lg + r: exactly
      // half of its A-operand fragment (column block ct/2, half ct%2)
      const int i = 16 * rt + li, j0 = 16 * ct + 4 * lg;
      const float gi = s.gs[i], qsi = s.qinv[i] * kQScale;
      const f32x4 gj = *reinterpret_cast<const f32x4*>(s.gs + j0);
      const f32x4 kj = *reinterpret_cast<const f32x4*>(s.kinv + j0);
      bf16x4 vh, vl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool on = j0 + r <= i;
        const float decay = __builtin_amdgcn_exp2f((gi - gj[r]) * kLog2e);
        const float a = on ? ((qsi * kj[r]) * acc_job[jj][r]) * decay : 0.f;
        bf16 hh, ll;
        split2(a, hh, ll);
        vh[r] = hh;
        vl[r] = ll;
      }
      const int o = frag_off(i, j0, 2);
      *reinterpret_cast<bf16x4*>(ah + o) = vh;
      *reinterpret_cast<bf16x4*>(al + o) = vl;
    } else {
      const int j = 16 * ct + li, i0 = 16 * rt + 4 * lg;
      const float gj = s.gs[j], kj = s.kinv[j];
      const f32x4 gi = *reinterpret_cast<const f32x4*>(s.gs + i0);
      const f32x4 ki = *reinterpret_cast<const f32x4*>(s.kinv + i0);
      const f32x4 bi = *reinterpret_cast<const f32x4*>(s.bs + i0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float decay = __builtin_amdgcn_exp2f((gi[r] - gj) * kLog2e);
        s.u.lm[(i0 + r) * kPitchF + j] =
            j < i0 + r ? (((ki[r] * kj) * acc_job[jj][r]) * bi[r]) * decay : 0.f;
      }
    }
  }
  // Aqk's upper tiles (0, 1) and (2, 3) complete the A operands the scan
  // uses (token tiles 0 and 2 with 32-token blocks 0 and 1); the other upper
  // tiles are never used.
  if (tid < 128) {
    const int t = tid >> 6, ln = tid & 63;
    const int o = frag_off(32 * t + (ln & 15), 32 * t + 16 + 4 * (ln >> 4), 2);
    *reinterpret_cast<bf16x4*>(ah + o) = bf16x4{};
    *reinterpret_cast<bf16x4*>(al + o) = bf16x4{};
  }
  // (The strictly-upper tiles of L are never read, and every entry of T is
  // written below: S3 fills the diagonal blocks, S4 the lower blocks and
  // clears the upper blocks it parks its sums in.)
  lds_barrier();

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
  lds_barrier();
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
    lds_barrier();
  }

  // S5. T diag(beta) as hi/lo A-operand fragments: item (row i, 32-token
  // block kb, group g) forms columns 32kb + 4g .. +3 and 32kb + 16 + 4g .. +3,
  // the 8 elements of one fragment slot, stored as one 16-byte write per
  // plane.  Rows 0-31 against columns 32-63 (the second 32-token block of
  // token tiles 0 and 1) are zero and never read by the scan: not stored.
  for (int idx = tid; idx < kC * 8; idx += 256) {
    const int i = idx >> 3, kb = (idx >> 2) & 1, g = idx & 3;
    if (i < 32 && kb == 1) continue;
    const int j0 = 32 * kb + 4 * g;
    const f32x4 ta = *reinterpret_cast<const f32x4*>(s.tm + i * kPitchF + j0);
    const f32x4 tb = *reinterpret_cast<const f32x4*>(s.tm + i * kPitchF + j0 + 16);
    const f32x4 ba = *reinterpret_cast<const f32x4*>(s.bs + j0);
    const f32x4 bb = *reinterpret_cast<const f32x4*>(s.bs + j0 + 16);
    bf16x8 hv, lv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bf16 hh, ll;
      split2(ta[e] * ba[e], hh, ll);
      hv[e] = hh;
      lv[e] = ll;
      split2(tb[e] * bb[e], hh, ll);
      hv[4 + e] = hh;
      lv[4 + e] = ll;
    }
    const int o = frag_off(i, j0, 2);
    *reinterpret_cast<bf16x8*>(th + o) = hv;
    *reinterpret_cast<bf16x8*>(tl + o) = lv;
  }
}

// ---------------------------------------------------------------------------
// Phase B
// ---------------------------------------------------------------------------

constexpr int kScanGroups = kGdnDv / 16;   // 16 v-columns per workgroup

// Scan LDS.  The chain waves' exchange buffers, then the chunk operands the
// producer waves stage one chunk ahead (by chunk parity): q and k rows
// (row-major, pitch kPitchR: conflict-free 16-byte row writes and
// fragment reads; k^T operands come from the same rows through transposed
// reads) and the record's scalars.
typedef bf16x4 XBlk[2][2][2][64];

struct ScanLds {
  bf16x8 st[4][2][64];        // [state tile pair][hi, lo][lane]: B operands
  // Exchanged token tiles: [32-token block][hi, lo][tile parity][lane];
  // token tile t holds elements 4 (t % 2) .. +3 of its block's B operand,
  // so a reader joins the two parities (one ds_read2_b64) and every writer
  // lane stores 8 contiguous bytes.
  XBlk z;                     // v - cy (k S)
  XBlk vp[2];                 // v', rsk v'
  bf16 qr[2][kC * kPitchR];
  bf16 kr[2][kC * kPitchR];
  float sc[2][kNsc * 64];
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// split2 on a pair, converting two values per instruction: hi = bf16(x),
// lo = bf16(x - hi), with hi widened back by shifting / masking the pair.
__device__ __forceinline__ void split_pair(float x0, float x1, bf16x2& hi, bf16x2& lo) {
  hi = __builtin_convertvector(f32x2{x0, x1}, bf16x2);
  const unsigned u = __builtin_bit_cast(unsigned, hi);
  const float h0 = __builtin_bit_cast(float, u << 16);
  const float h1 = __builtin_bit_cast(float, u & 0xffff0000u);
  lo = __builtin_convertvector(f32x2{x0 - h0, x1 - h1}, bf16x2);
}

__device__ __forceinline__ void split4x(const f32x4& x, bf16x4& hi, bf16x4& lo) {
  bf16x2 h01, l01, h23, l23;
  split_pair(x[0], x[1], h01, l01);
  split_pair(x[2], x[3], h23, l23);
  hi = bf16x4{h01[0], h01[1], h23[0], h23[1]};
  lo = bf16x4{l01[0], l01[1], l23[0], l23[1]};
}

__device__ __forceinline__ bf16x8 split4(const f32x4& x) {
  bf16x4 hi, lo;
  split4x(x, hi, lo);
  return bf16x8{hi[0], hi[1], hi[2], hi[3], lo[0], lo[1], lo[2], lo[3]};
}

// Publish token tile t of an exchanged pair of B operands (see ScanLds).
__device__ __forceinline__ void put_tile(XBlk& blk, int t, int lane, const f32x4& x) {
  bf16x4 hi, lo;
  split4x(x, hi, lo);
  blk[t >> 1][0][t & 1][lane] = hi;
  blk[t >> 1][1][t & 1][lane] = lo;
}

// The B operand of 32-token block b, plane pl (0 = hi, 1 = lo).
__device__ __forceinline__ bf16x8 get_blk(const XBlk& blk, int b, int pl, int lane) {
  const bf16x4 a = blk[b][pl][0][lane], c = blk[b][pl][1][lane];
  return bf16x8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
}

// B operands (hi, lo) from two published accumulator tiles.
__device__ __forceinline__ void join_pair(const bf16x8& a, const bf16x8& b,
                                          bf16x8& hi, bf16x8& lo) {
  hi = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  lo = bf16x8{a[4], a[5], a[6], a[7], b[4], b[5], b[6], b[7]};
}

// A operand of a row-major LDS matrix: row `row`, reduction elements
// c0 .. c0+3 and c0+16 .. c0+19 (the permuted order of frag_off).
__device__ __forceinline__ bf16x8 frag_row(const bf16* m, int pitch, int row, int c0) {
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(m + row * pitch + c0);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(m + row * pitch + c0 + 16);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// grid = 256 workgroups of 12 waves (32 heads x 8 groups of 16 v-columns;
// the 8 groups of a head -- and the two heads of a key head -- share an
// XCD, so a chunk's q, k and prep record come from HBM once per XCD).
//  * Chain waves 0-3 (one per SIMD) carry the state recurrence only: wave w
//    owns token tile w of every chunk and state tiles 2w, 2w+1 (rows
//    32w .. 32w+31), in the MFMA accumulator layout:
//    sreg[i][r] = S[16(2w+i) + 4lg + r][col].  Per chunk:
//      (a) publish the state tiles (hi/lo);
//      (b) Y = k_raw S for the wave's 16 tokens, publish Z = v - cy Y;
//      (c) v' = (T diag beta) Z for the wave's tokens; publish v', rsk v';
//      (d) S = e^(G_last) S + k^T (rsk v'), published for the next chunk.
//  * Producer waves 4-7: in (a) of chunk c they stage chunk c+1's q rows
//    and scalars into LDS (read from (b) of chunk c+1 on), in (b) its k
//    rows (read by the chain from (d) of chunk c on), and then request
//    chunk c+2's rows.
//  * Output waves 8-11: token tile w's o = rsq (q_raw S) + Aqk v', with
//    q_raw S in (b) (beside the chain's k_raw S, from the same published
//    state) and Aqk v' and the store in (d).
// The roles share the SIMDs, so each one's work fills the others' stalls;
// the split was measured against others on MI355X (T = 8192, scan alone):
// the chain also forming the output 187 us, the output on the producer
// waves 238 us, these three roles 170 us; moving part of q_raw S into (c)
// or part of the output into the next chunk's (b) put work on the chain's
// busiest windows (264-279 us).
// Each phase ends at a workgroup barrier, and every staged buffer is
// double-buffered by chunk parity, so a buffer is rewritten only after the
// barrier that follows its last read.
__global__ __launch_bounds__(768, 1) void gdn_chunk_scan_kernel(
    const char* __restrict__ ws, const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, unsigned qk_heads, unsigned qk_token_stride,
    unsigned v_token_stride, const float* state_in, float* state_out,
    bf16* __restrict__ out, unsigned tokens, unsigned c_begin, unsigned c_end,
    bool state_vk) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  ScanLds& s = *reinterpret_cast<ScanLds*>(smem);
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int h = 4 * xcd + (slot >> 3);
  const int kh = h * (int)qk_heads / kGdnHv;
  const int cg = slot & 7;
  const int tid = threadIdx.x, w = (tid >> 6) & 3, lane = tid & 63;
  const bool producer = tid >= 256 && tid < 512, outputs = tid >= 512;
  const int li = lane & 15, lg = lane >> 4;
  const int col = 16 * cg + li;
  const unsigned last = c_end - 1;

  // ---- producer side ------------------------------------------------------
  // Rows past the last token read as zeros through the buffer ranges (each
  // range starts at the chunk's first row); loads are unconditional.
  u32x4 pq[4], pk[4], psc;
  auto p_fetch = [&](unsigned c) {
    const unsigned rows = min((unsigned)kC, tokens - c * kC);
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(q) + (size_t)c * kC * qk_token_stride + kh * kGdnDk, 0,
        (int)(rows * qk_token_stride * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(k) + (size_t)c * kC * qk_token_stride + kh * kGdnDk, 0,
        (int)(rows * qk_token_stride * 2), 0x00020000);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 16 * w + 4 * u + (lane >> 4);
      const int off = (int)((row * qk_token_stride + 8 * (lane & 15)) * 2);
      pq[u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, off, 0, 0);
      pk[u] = __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0);
    }
    const char* b = ws + ((size_t)c * kGdnHv + h) * kUnitBytes + kOffSc;
    const int pt = tid - 256;
    psc = reinterpret_cast<const u32x4*>(b)[pt < kNsc * 16 ? pt : 0];
  };
  // Stage the fetched rows of chunk c (lane: dims 8p .. 8p+7 of row
  // 16w + 4u + lane/16, p = lane % 16).
  auto p_stage_k = [&](unsigned c) {
    const int par = c & 1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 16 * w + 4 * u + (lane >> 4), d0 = 8 * (lane & 15);
      *reinterpret_cast<u32x4*>(s.kr[par] + row * kPitchR + d0) = pk[u];
    }
  };
  auto p_stage = [&](unsigned c) {
    const int par = c & 1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 16 * w + 4 * u + (lane >> 4), d0 = 8 * (lane & 15);
      *reinterpret_cast<u32x4*>(s.qr[par] + row * kPitchR + d0) = pq[u];
    }
    const int pt = tid - 256;
    if (pt < kNsc * 16) reinterpret_cast<u32x4*>(s.sc[par])[pt] = psc;
  };
  // ---- chain side -----------------------------------------------------------
  // state element (k row, v column): [Hv, dk, dv], or vLLM's [Hv, dv, dk]
  const size_t srow = state_vk ? 1 : kGdnDv;
  const size_t sb = (size_t)h * kGdnDk * kGdnDv + (size_t)col * (state_vk ? kGdnDk : 1);
  f32x4 sreg[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  bf16x8 th[2], tl[2];
  unsigned vv[4];
  auto c_fetch_v = [&](unsigned c) {
    const unsigned rows = min((unsigned)kC, tokens - c * kC);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(v) + (size_t)c * kC * v_token_stride + h * kGdnDv + 16 * cg, 0,
        (int)(rows * v_token_stride * 2), 0x00020000);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      vv[r] = __builtin_amdgcn_raw_buffer_load_b16(
          vrs, (int)(((16 * w + 4 * lg + r) * v_token_stride + li) * 2), 0, 0);
  };
  // (Token tiles 0 and 1 never use the second 32-token block, which the prep
  // does not store: their second load re-reads the first block, so the loads
  // stay unconditional and no unwritten workspace byte is read.)
  const int t2_hi = w < 2 ? 0 : 64;
  auto c_fetch_t = [&](unsigned c) {
    const char* b = ws + ((size_t)c * kGdnHv + h) * kUnitBytes;
    const bf16x8* Th = reinterpret_cast<const bf16x8*>(b + kOffTh) + 128 * w + lane;
    const bf16x8* Tl = reinterpret_cast<const bf16x8*>(b + kOffTl) + 128 * w + lane;
    th[0] = Th[0];
    tl[0] = Tl[0];
    th[1] = Th[t2_hi];
    tl[1] = Tl[t2_hi];
  };

  // The three roles run separate loops (straight-line code per role, so the
  // compiler's in-order wait counts follow each role's own loads) with the
  // same barrier sequence: one after the prologue, three per chunk.
  if (outputs) {
    // Output waves 8-11: token tile w's o = rsq (q_raw S) + Aqk v'; q_raw S
    // in (b) beside the chain's k_raw S (same published state), Aqk v' in
    // (d) once v' is published.
    const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        out, 0, (int)(tokens * kGdnHv * kGdnDv * 2), 0x00020000);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    bf16x8 ah[2], al[2];   // token tile w's rows of Aqk (hi / lo), 32-token blocks
    auto c_fetch_a = [&](unsigned c) {
      const char* b = ws + ((size_t)c * kGdnHv + h) * kUnitBytes;
      const bf16x8* Ah = reinterpret_cast<const bf16x8*>(b + kOffAh) + 128 * w + lane;
      const bf16x8* Al = reinterpret_cast<const bf16x8*>(b + kOffAl) + 128 * w + lane;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        ah[t2] = Ah[64 * t2];
        al[t2] = Al[64 * t2];
      }
    };
    c_fetch_a(c_begin);
    lds_barrier();
    for (unsigned c = c_begin; c < c_end; ++c) {
      const int par = c & 1;
      const unsigned nxt = c + 1 < last ? c + 1 : last;
      lds_barrier();
      {
        f32x4 a1 = zero, a2 = zero;
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
          const bf16x8 qfa = frag_row(s.qr[par], kPitchR, 16 * w + li, 32 * k4 + 4 * lg);
          a1 = mfma16x16x32(qfa, s.st[k4][0][lane], a1);
          a2 = mfma16x16x32(qfa, s.st[k4][1][lane], a2);
        }
        const f32x4 rsq = *reinterpret_cast<const f32x4*>(s.sc[par] + kScRsq * 64 + 16 * w + 4 * lg);
        acc = rsq * (a1 + a2);
      }
      lds_barrier();
      lds_barrier();
      f32x4 acc2 = zero, acc3 = zero;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        if (t2 == 1 && w < 2) break;
        const bf16x8 vh = get_blk(s.vp[0], t2, 0, lane), vl = get_blk(s.vp[0], t2, 1, lane);
        acc = mfma16x16x32(ah[t2], vh, acc);
        acc2 = mfma16x16x32(ah[t2], vl, acc2);
        acc3 = mfma16x16x32(al[t2], vh, acc3);
      }
      acc += acc2 + acc3;
      c_fetch_a(nxt);
      // Output rows past the end fall outside the buffer range and are
      // dropped by the hardware (no branch, so no uncertain store count).
      const unsigned tb = c * kC + 16 * w + 4 * lg;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __builtin_amdgcn_raw_buffer_store_b16(
            __builtin_bit_cast(unsigned short, f2bf(acc[r])), out_rsrc,
            (int)((((tb + r) * kGdnHv + h) * kGdnDv + col) * 2), 0, 0);
    }
    return;
  }
  if (producer) {
    p_fetch(c_begin);
    p_stage(c_begin);
    p_stage_k(c_begin);
    p_fetch(c_begin + 1 < last ? c_begin + 1 : last);
    lds_barrier();
    for (unsigned c = c_begin; c < c_end; ++c) {
      // (a) chunk c+1's q rows and scalars (the buffers of chunk c-1, whose
      // q rows the output waves last read in (b) of chunk c-1 and whose
      // scalars the chain read in (d) of chunk c-2)
      if (c + 1 < c_end) p_stage(c + 1);
      lds_barrier();
      // (b) chunk c+1's k rows (last read by the chain in (d) of chunk
      // c-1), then request chunk c+2's rows
      if (c + 1 < c_end) p_stage_k(c + 1);
      p_fetch(c + 2 < last ? c + 2 : last);
      lds_barrier();
      lds_barrier();
    }
    return;
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sreg[i][r] = state_in ? state_in[sb + (size_t)(16 * (2 * w + i) + 4 * lg + r) * srow] : 0.f;
  c_fetch_v(c_begin);
  c_fetch_t(c_begin);
  lds_barrier();
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  // (a) publish the state tiles as the hi / lo B operands of tile pair w
  // (for chunk c+1 this happens in (d) of chunk c, right after the update)
  auto publish_state = [&]() {
    bf16x8 hi, lo;
    join_pair(split4(sreg[0]), split4(sreg[1]), hi, lo);
    s.st[w][0][lane] = hi;
    s.st[w][1][lane] = lo;
  };
  publish_state();
  // A chunk's k fragments and row scalars, read from LDS at the end of the
  // previous chunk (staged before its second barrier), so (b) starts with
  // the state operands only.
  bf16x8 kfa[4];
  f32x4 cy, rsk;
  float egl;
  auto read_chunk = [&](unsigned c) {
    const int par = c & 1;
    const int r0 = 16 * w + 4 * lg;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4)
      kfa[k4] = frag_row(s.kr[par], kPitchR, 16 * w + li, 32 * k4 + 4 * lg);
    cy = *reinterpret_cast<const f32x4*>(s.sc[par] + kScCy * 64 + r0);
    rsk = *reinterpret_cast<const f32x4*>(s.sc[par] + kScRsk * 64 + r0);
    egl = s.sc[par][kScEgl * 64];
  };
  read_chunk(c_begin);
  for (unsigned c = c_begin; c < c_end; ++c) {
    const int par = c & 1;
    const unsigned nxt = c + 1 < last ? c + 1 : last;
    lds_barrier();
    // (b) Y = k_raw S (two accumulator chains: the hi and lo halves of S),
    // Z = v - cy Y published
    bf16x8 shi[4], slo[4];
    f32x4 ay = zero, ay2 = zero;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      shi[k4] = s.st[k4][0][lane];
      slo[k4] = s.st[k4][1][lane];
      ay = mfma16x16x32(kfa[k4], shi[k4], ay);
      ay2 = mfma16x16x32(kfa[k4], slo[k4], ay2);
    }
    ay += ay2;
    f32x4 zv;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      zv[r] = bf2f(__builtin_bit_cast(bf16, (unsigned short)vv[r])) - cy[r] * ay[r];
    put_tile(s.z, w, lane, zv);
    c_fetch_v(nxt);
    lds_barrier();
    // (c) v' = (T diag beta) Z: T is lower triangular, so token tiles 0, 1
    // only reduce over the first 32 tokens
    {
      f32x4 vp = zero, vp2 = zero, vp3 = zero;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        if (t2 == 1 && w < 2) break;
        const bf16x8 zh = get_blk(s.z, t2, 0, lane), zl = get_blk(s.z, t2, 1, lane);
        vp = mfma16x16x32(th[t2], zh, vp);
        vp2 = mfma16x16x32(th[t2], zl, vp2);
        vp3 = mfma16x16x32(tl[t2], zh, vp3);
      }
      vp += vp2 + vp3;
      put_tile(s.vp[1], w, lane, rsk * vp);
      put_tile(s.vp[0], w, lane, vp);
    }
    c_fetch_t(nxt);
    lds_barrier();
    // (d) S = exp(G_last) S + k_raw^T (rsk v'), published for chunk c+1,
    // and chunk c+1's k fragments and scalars
    f32x4 sn[2] = {sreg[0] * egl, sreg[1] * egl};
    f32x4 sl[2] = {zero, zero};
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      const bf16x8 zh = get_blk(s.vp[1], t2, 0, lane), zl = get_blk(s.vp[1], t2, 1, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        // k^T A operand (row = dim 16(2w+i) + li, reduction = tokens
        // 32t2 + 4lg + e and +16) by transposed reads of the k rows
        const bf16* ra = s.kr[par] + (32 * t2 + 4 * lg + (li >> 2)) * kPitchR +
                         16 * (2 * w + i) + 4 * (li & 3);
        const bf16x8 ktf = cat_bf16x8(lds_read_tr16(ra), lds_read_tr16(ra + 16 * kPitchR));
        sn[i] = mfma16x16x32(ktf, zh, sn[i]);
        sl[i] = mfma16x16x32(ktf, zl, sl[i]);
      }
    }
    sreg[0] = sn[0] + sl[0];
    sreg[1] = sn[1] + sl[1];
    if (c + 1 < c_end) {
      publish_state();
      read_chunk(c + 1);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      state_out[sb + (size_t)(16 * (2 * w + i) + 4 * lg + r) * srow] = sreg[i][r];
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT size_t qwen36_gdn_chunk_prefill_workspace_bytes(unsigned tokens) {
  const size_t n_chunks = (tokens + kC - 1) / kC;
  return n_chunks * kGdnHv * kUnitBytes;
}

Q36_EXPORT int qwen36_gdn_chunk_prefill_ex(
    const void* q, const void* k, const void* v, unsigned qk_heads,
    unsigned qk_token_stride, unsigned v_token_stride, const void* g,
    const void* beta, const void* state_in, void* state_out, void* out,
    unsigned tokens, unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
      beta == nullptr || state_out == nullptr || out == nullptr ||
      workspace == nullptr || tokens == 0 || tokens > kMaxTokens ||
      (flags & ~(kFlagQkNormalized | kFlagStateVk)) != 0 ||
      (qk_heads != 16u && qk_heads != 32u) ||
      qk_token_stride < qk_heads * kGdnDk ||
      v_token_stride < (unsigned)(kGdnHv * kGdnDv) ||
      (qk_token_stride % 8) != 0 || (v_token_stride % 8) != 0 ||
      !aligned16(q) || !aligned16(k) || !aligned16(v))
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
    if (attr_status == hipSuccess)
      attr_status = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_chunk_scan_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)sizeof(ScanLds));
  });
  if (attr_status != hipSuccess) return (int)attr_status;
  char* wsb = static_cast<char*>(workspace);
  const bf16* qb = static_cast<const bf16*>(q);
  const bf16* kb = static_cast<const bf16*>(k);
  const bf16* vb = static_cast<const bf16*>(v);
  const float* gb = static_cast<const float*>(g);
  const float* bb = static_cast<const float*>(beta);
  float* so = static_cast<float*>(state_out);
  const bool l2norm = (flags & kFlagQkNormalized) == 0;
  const bool state_vk = (flags & kFlagStateVk) != 0;
  // Prep over every chunk, then the scan.  Run side by side (two streams, no
  // dependency; timing only) they barely overlap: a scan workgroup (93.7 KB
  // of LDS) cannot join a CU that holds two prep workgroups (2 x 35.8 KB), so
  // the scan starts as the prep drains (MI355X: T = 8192 0.229 vs 0.230 ms,
  // 32768 0.892 vs 0.972 ms, 2048 0.075 vs 0.064 ms with the stream fork).
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(n_chunks, kGdnHv), dim3(256), sizeof(PrepLds), st,
                     qb, kb, qk_heads, qk_token_stride, gb, bb, tokens, wsb, 0u, l2norm);
  hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3(kGdnHv * kScanGroups), dim3(768),
                     sizeof(ScanLds), st, wsb, qb, kb, vb, qk_heads, qk_token_stride,
                     v_token_stride, static_cast<const float*>(state_in), so,
                     static_cast<bf16*>(out), tokens, 0u, n_chunks, state_vk);
  return static_cast<int>(hipGetLastError());
}

Q36_EXPORT int qwen36_gdn_chunk_prefill(
    const void* q, const void* k, const void* v, unsigned qk_heads,
    unsigned qk_token_stride, unsigned v_token_stride, const void* g,
    const void* beta, const void* state_in, void* state_out, void* out,
    unsigned tokens, void* workspace, size_t workspace_bytes, void* stream) {
  return qwen36_gdn_chunk_prefill_ex(q, k, v, qk_heads, qk_token_stride, v_token_stride, g, beta,
                                     state_in, state_out, out, tokens, 0u, workspace,
                                     workspace_bytes, stream);
}
