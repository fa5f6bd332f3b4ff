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
//  * the next tile's K/V is fetched into registers while the current one is
//    consumed, so HBM/L2 latency overlaps the MFMA work.
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
constexpr int kFmLds = 2 * kFmTileBytes;              // K + V
constexpr int kFmChunksPerThread = kFmTileBytes / 16 / (kFmWaves * 64);  // 8

// Physical 16-byte chunk of logical chunk c in row r.
__device__ __forceinline__ int k_swz(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_swz(int r, int c) { return c ^ ((r & 3) << 2); }

__global__ __launch_bounds__(256, 1) void fmha_prefill_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, float* __restrict__ out, unsigned q_tokens,
    unsigned kv_tokens, unsigned n_qtiles) {
  __shared__ __attribute__((aligned(16))) char lds[kFmLds];
  char* ks = lds;
  char* vs = lds + kFmTileBytes;

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

  // Cooperative tile fetch: chunk id = tid + 256*i -> (row id/32, chunk id%32).
  uint4 kr[kFmChunksPerThread], vr[kFmChunksPerThread];
  auto fetch = [&](unsigned kv0) {
#pragma unroll
    for (int i = 0; i < kFmChunksPerThread; ++i) {
      const int id = tid + 256 * i;
      const unsigned key = kv0 + (id >> 5);
      const size_t g = ((size_t)key * kHkv + kvh) * kD + (id & 31) * 8;
      if (key < kv_end) {
        kr[i] = *reinterpret_cast<const uint4*>(k + g);
        vr[i] = *reinterpret_cast<const uint4*>(v + g);
      } else {
        kr[i] = uint4{0u, 0u, 0u, 0u};
        vr[i] = uint4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < kFmChunksPerThread; ++i) {
      const int id = tid + 256 * i;
      const int r = id >> 5, c = id & 31;
      *reinterpret_cast<uint4*>(ks + r * 512 + k_swz(r, c) * 16) = kr[i];
      *reinterpret_cast<uint4*>(vs + r * 512 + v_swz(r, c) * 16) = vr[i];
    }
  };

  const unsigned n_tiles = (kv_end + kFmKv - 1) / kFmKv;
  fetch(0);
  for (unsigned t = 0; t < n_tiles; ++t) {
    const unsigned kv0 = t * kFmKv;
    __syncthreads();               // previous tile fully consumed
    stash();
    __syncthreads();               // tile visible to every wave
    if (t + 1 < n_tiles) fetch(kv0 + kFmKv);
    if (kv0 > wave_lim) continue;  // every key of the tile is masked for us

    // S^T[key][row] for two 32-key halves.
    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int r = tt * 32 + lj;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(
            ks + r * 512 + k_swz(r, 2 * st + lg) * 16);
        s[tt] = mfma32x32x16(a, qf[st], s[tt]);
      }
    }
    // Lane holds keys kv0 + 32*tt + 8*(r/4) + 4*lg + r%4 of its row.
    const bool need_mask = kv0 + kFmKv - 1 > row_lim - 0u ||
                           kv0 + kFmKv > kv_tokens;
    float mx = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[tt][r] * scale;
        if (need_mask) {
          const unsigned key = kv0 + 32 * tt + 8 * (r >> 2) + 4 * lg + (r & 3);
          if (key > row_lim || key >= kv_tokens) x = -INFINITY;
        }
        s[tt][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = wave_max_xor(mx, 32);
    const float mnew = fmaxf(m, mx);
    const float alpha = exp2f(m - mnew);
    float psum = 0.f;
    bf16x8 pb[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(s[tt][r] - mnew);
        psum += p;
        pb[tt][r >> 3][r & 7] = f2bf(p);
      }
    }
    l = l * alpha + psum;
    m = mnew;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= alpha;

    // O^T[d][row] += V^T[d][key] P^T[key][row]; step (tt, st) reduction
    // slots (lg, e) <-> keys 32tt + 16st + 4lg + e and +8 for e >= 4.
    const int grp = lane >> 4, m16 = lane & 15;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int r0 = 32 * tt + 16 * st + 4 * lg + (m16 >> 2);
        const int r1 = r0 + 8;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int c = 4 * dt + 2 * (grp & 1) + ((m16 & 3) >> 1);
          const int wb = (m16 & 1) * 8;
          const i16x4 a0 = lds_read_tr16(vs + r0 * 512 + v_swz(r0, c) * 16 + wb);
          const i16x4 a1 = lds_read_tr16(vs + r1 * 512 + v_swz(r1, c) * 16 + wb);
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
  const unsigned n_qtiles = (q_tokens + kFmRows - 1) / kFmRows;
  hipLaunchKernelGGL(fmha_prefill_kernel, dim3(n_qtiles * kHq), dim3(256), 0,
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
