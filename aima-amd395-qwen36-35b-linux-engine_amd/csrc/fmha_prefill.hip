// Causal GQA flash-attention prefill (BF16 in, FP32 out) for gfx950.
//
// Drop-in for the reference's dlopen'd FMHA provider C ABI
// (benchmarks/shape-lab/native/src/qrt_ck_fmha_q8192_provider.cpp:134-325,
// consumed by native/src/native_full_prefill.hip.cpp:140-266):
//   Q [q_tokens, 16, 256] bf16 (token stride 4096), K/V [kv_tokens, 2, 256]
//   bf16 (token stride 512), out fp32 [q_tokens, 4096]; scale 1/sqrt(256);
//   query head h reads KV head h/8; top-left causal mask when
//   q_tokens == kv_tokens, bottom-right (query i sees keys
//   j <= i + kv_tokens - q_tokens) when kv_tokens > q_tokens.
//
// Kernel plan (MFMA-bound, 16384 flop per unmasked (q,k) pair):
//  * workgroup = 4 waves = 128 query rows of one head; wave = 32 rows.
//  * per 64-key tile: K and V are staged in LDS (XOR-swizzled 16-byte chunks,
//    no padding); S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = K from LDS,
//    B = Q^T held in registers for the whole kernel), online softmax per row
//    in fp32 (exp2 domain), O^T += V^T P^T (A = V^T read with
//    ds_read_b64_tr_b16, B = P^T taken straight from the S^T accumulator).
//  * K/V tiles are fetched straight into LDS (global_load_lds_dwordx4, no
//    register staging) into a double buffer, so the next tile's HBM/L2
//    latency overlaps the current tile's MFMA work.
//  * the O accumulator is rescaled only when a row's running max changes.
//  * blockIdx -> (KV head, query head, query tile) is XCD-aware: the 8 XCDs
//    receive workgroups round-robin, so XCDs 0-3 serve KV head 0 and 4-7 KV
//    head 1 (their L2s then hold one head's K/V), and every XCD issues its
//    heaviest (latest) causal tiles first.
#include "common.h"

namespace q36 {
namespace {

constexpr int kFmWaves = 4;
constexpr int kFmRowsPerWave = 32;
constexpr int kFmRows = kFmWaves * kFmRowsPerWave;   // 128
constexpr int kFmKv = 64;                             // keys per tile
constexpr int kFmTileBytes = kFmKv * kD * 2;          // 32 KiB
constexpr int kFmStage = 2 * kFmTileBytes;            // K + V
constexpr int kFmLds = 2 * kFmStage;                  // double buffered, 128 KiB
constexpr int kFmLoadsPerWave = kFmTileBytes / 1024 / kFmWaves;  // 8

typedef __attribute__((address_space(3))) void lds_void;

// Physical 16-byte chunk of logical chunk c in row r (XOR swizzles are
// involutions, so the same map converts physical to logical).
__device__ __forceinline__ int k_swz(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_swz(int r, int c) { return c ^ ((r & 3) << 2); }

__global__ __launch_bounds__(256, 1) void fmha_prefill_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, float* __restrict__ out, unsigned q_tokens,
    unsigned kv_tokens, unsigned n_qtiles) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];

  // XCD-aware tile mapping (see header).
  const unsigned b = blockIdx.x;
  const unsigned xcd = b & 7u, n = b >> 3;
  const int kvh = xcd >> 2;
  const int head = kvh * kGroup + (xcd & 3) * 2 + (n & 1);
  const unsigned qtile = n_qtiles - 1 - (n >> 1);
  const unsigned q0 = qtile * kFmRows;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lj = lane & 31;     // MFMA column (query row within the wave)
  const int lg = lane >> 5;     // k-half
  const unsigned off = kv_tokens - q_tokens;   // bottom-right shift
  const unsigned row = q0 + wave * kFmRowsPerWave + lj;   // this lane's query
  const bool row_valid = row < q_tokens;
  const unsigned row_lim = (row_valid ? row : q_tokens - 1) + off;  // last key
  const unsigned wave_first = q0 + wave * kFmRowsPerWave;
  const unsigned wave_lim =
      min(wave_first + kFmRowsPerWave - 1, q_tokens - 1) + off;
  const unsigned kv_end = min(kv_tokens, min(q0 + kFmRows, q_tokens) + off);

  // Q^T operand: step s covers dims s*16 + 8*lg .. +8 of this lane's row.
  bf16x8 qf[16];
  {
    const bf16* qp = q + (size_t)row * kQDim + head * kD + 8 * lg;
#pragma unroll
    for (int s = 0; s < 16; ++s)
      qf[s] = row_valid ? *reinterpret_cast<const bf16x8*>(qp + s * 16)
                        : bf16x8{};
  }

  f32x16 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = f32x16{};
  float m = -INFINITY, l = 0.f;
  const float scale = 0.0625f * kLog2e;

  // Direct global->LDS tile fetch through buffer resources (base in SGPRs,
  // bounds = kv_end rows, so rows past kv_end read as zeros).  Wave
  // instruction j writes 1 KiB = two 512-byte rows at LDS offset
  // 1024*(8*wave + j); lane -> (row, physical chunk lane%32) loads the
  // logical chunk that the swizzle maps there.
  const int nrec = (int)(kv_end * (unsigned)(kHkv * kD * 2));
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)k, 0, nrec, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)v, 0, nrec, 0x00020000);
  int koff[kFmLoadsPerWave], voff[kFmLoadsPerWave];
#pragma unroll
  for (int j = 0; j < kFmLoadsPerWave; ++j) {
    const int r = 2 * (kFmLoadsPerWave * wave + j) + (lane >> 5);
    const int p = lane & 31;
    const int base = r * (kHkv * kD * 2) + kvh * kD * 2;
    koff[j] = base + k_swz(r, p) * 16;
    voff[j] = base + v_swz(r, p) * 16;
  }
  auto fetch = [&](unsigned kv0, int stage) {
    char* ks = lds + stage * kFmStage;
    char* vs = ks + kFmTileBytes;
    const int soff = (int)(kv0 * (unsigned)(kHkv * kD * 2));
#pragma unroll
    for (int j = 0; j < kFmLoadsPerWave; ++j) {
      const int blk = kFmLoadsPerWave * wave + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(ks + blk * 1024), 16,
                                               koff[j], soff, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(vs + blk * 1024), 16,
                                               voff[j], soff, 0, 0);
    }
  };

  // Per-lane LDS byte offsets of the K (A-operand) and V^T (transposed) reads.
  const int krow0 = lj * 512;                       // tile half tt adds 32 rows
  const int kx = lj & 15;
  const int grp = lane >> 4, m16 = lane & 15;
  const int vrow = 4 * lg + (m16 >> 2);             // + 32tt + 16st (+8)
  const int vsw = (vrow & 3) << 2;                  // v_swz term (row & 3)
  const int vcol = 2 * (grp & 1) + ((m16 & 3) >> 1);
  const int vwb = (m16 & 1) * 8;

  const unsigned n_tiles = (kv_end + kFmKv - 1) / kFmKv;
  fetch(0, 0);
  for (unsigned t = 0; t < n_tiles; ++t) {
    const unsigned kv0 = t * kFmKv;
    const int stage = t & 1;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's fetches of tile t landed
    __syncthreads();                 // ... and every wave's; tile t-1 consumed
    if (t + 1 < n_tiles) fetch(kv0 + kFmKv, stage ^ 1);
    if (kv0 > wave_lim) continue;    // every key of the tile is masked for us
    const char* ks = lds + stage * kFmStage;
    const char* vs = ks + kFmTileBytes;

    // S^T[key][row] for two 32-key halves; K fragments are read one step
    // ahead of the MFMAs that consume them.
    f32x16 s0 = f32x16{}, s1 = f32x16{};
    bf16x8 ka = *reinterpret_cast<const bf16x8*>(ks + krow0 + ((lg ^ kx) << 4));
    bf16x8 kb = *reinterpret_cast<const bf16x8*>(ks + 32 * 512 + krow0 + ((lg ^ kx) << 4));
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      bf16x8 na, nb;
      if (st + 1 < 16) {
        const int c = ((2 * (st + 1) + lg) ^ kx) << 4;
        na = *reinterpret_cast<const bf16x8*>(ks + krow0 + c);
        nb = *reinterpret_cast<const bf16x8*>(ks + 32 * 512 + krow0 + c);
      }
      s0 = mfma32x32x16(ka, qf[st], s0);
      s1 = mfma32x32x16(kb, qf[st], s1);
      if (st + 1 < 16) {
        ka = na;
        kb = nb;
      }
    }
    // Lane holds keys kv0 + 32*tt + 8*(r/4) + 4*lg + r%4 of its row.
    float mx = -INFINITY;
    const bool diag = kv0 + kFmKv - 1 > wave_first + off || kv0 + kFmKv > kv_tokens;
    if (diag) {  // wave-uniform: only diagonal / ragged tiles pay for masking
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const unsigned key = kv0 + 8 * (r >> 2) + 4 * lg + (r & 3);
        const bool ok0 = key <= row_lim && key < kv_tokens;
        const bool ok1 = key + 32 <= row_lim && key + 32 < kv_tokens;
        s0[r] = ok0 ? s0[r] * scale : -INFINITY;
        s1[r] = ok1 ? s1[r] * scale : -INFINITY;
        mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] *= scale;
        s1[r] *= scale;
        mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
      }
    }
    mx = wave_max_xor(mx, 32);
    const float mnew = fmaxf(m, mx);
    // Rescale the accumulator only when some row's running max moved.
    if (__any(mnew > m)) {
      const float alpha = exp2f(m - mnew);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] *= alpha;
    }
    m = mnew;
    float psum = 0.f;
    bf16x8 pb[2][2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p0 = exp2f(s0[r] - mnew);
      const float p1 = exp2f(s1[r] - mnew);
      psum += p0 + p1;
      pb[0][r >> 3][r & 7] = f2bf(p0);
      pb[1][r >> 3][r & 7] = f2bf(p1);
    }
    l += psum;

    // O^T[d][row] += V^T[d][key] P^T[key][row]; step (tt, st) reduction
    // slots (lg, e) <-> keys 32tt + 16st + 4lg + e and +8 for e >= 4.
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const char* r0p = vs + (32 * tt + 16 * st + vrow) * 512 + vwb;
        const char* r1p = r0p + 8 * 512;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int c = ((4 * dt + vcol) ^ vsw) << 4;
          const i16x4 a0 = lds_read_tr16(r0p + c);
          const i16x4 a1 = lds_read_tr16(r1p + c);
          o[dt] = mfma32x32x16(cat_bf16x8(a0, a1), pb[tt][st], o[dt]);
        }
      }
    }
  }
  l += __shfl_xor(l, 32, 64);
  if (!row_valid) return;
  const float inv = 1.0f / l;
  float* op = out + (size_t)row * kQDim + head * kD + 4 * lg;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      f32x4 val = {o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv,
                   o[dt][4 * r4 + 2] * inv, o[dt][4 * r4 + 3] * inv};
      *reinterpret_cast<f32x4*>(op + dt * 32 + 8 * r4) = val;
    }
  }
}

int launch_fmha(const void* q, const void* k, const void* v, float* out,
                unsigned q_tokens, unsigned kv_tokens, hipStream_t stream) {
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr ||
      q_tokens == 0u || q_tokens > kMaxTokens || kv_tokens < q_tokens ||
      kv_tokens > kMaxTokens)
    return Q36_EINVAL;
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(fmha_prefill_kernel),
        hipFuncAttributeMaxDynamicSharedMemorySize, kFmLds);
    if (e != hipSuccess) return (int)e;
    attr_set = true;
  }
  const unsigned n_qtiles = (q_tokens + kFmRows - 1) / kFmRows;
  hipLaunchKernelGGL(fmha_prefill_kernel, dim3(n_qtiles * kHq), dim3(256), kFmLds,
                     stream, static_cast<const bf16*>(q),
                     static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                     out, q_tokens, kv_tokens, n_qtiles);
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace q36

// ---- provider ABI ---------------------------------------------------------
// The launch path owns no device memory, so prepare/release only validate.

Q36_EXPORT int qrt_ck_fmha_prepare(unsigned tokens) {
  return (tokens > 0u && tokens <= q36::kMaxTokens) ? Q36_OK : Q36_EINVAL;
}

Q36_EXPORT int qrt_ck_fmha_bf16_launch(const void* q, const void* k,
                                       const void* v, float* out,
                                       unsigned tokens, void* stream) {
  return q36::launch_fmha(q, k, v, out, tokens, tokens,
                          static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qrt_ck_fmha_bf16_launch_ex(const void* q, const void* k,
                                          const void* v, float* out,
                                          unsigned query_tokens,
                                          unsigned kv_tokens, void* stream) {
  return q36::launch_fmha(q, k, v, out, query_tokens, kv_tokens,
                          static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qrt_ck_fmha_release(void) { return Q36_OK; }

// Legacy fixed-shape q8192 exports (qrt_ck_fmha_q8192_provider.cpp:214-300).
Q36_EXPORT int qrt_ck_fmha_q8192_prepare(void) { return Q36_OK; }

Q36_EXPORT int qrt_ck_fmha_q8192_bf16_launch(const void* q, const void* k,
                                             const void* v, float* out,
                                             void* stream) {
  return q36::launch_fmha(q, k, v, out, 8192u, 8192u,
                          static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qrt_ck_fmha_q8192_release(void) { return Q36_OK; }
