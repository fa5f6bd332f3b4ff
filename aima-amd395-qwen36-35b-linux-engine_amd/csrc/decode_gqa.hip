// Split-K GQA flash-decode over a resident sequence-major BF16 KV cache.
//
// Replaces the reference's decode core launch_native_grouped_full_attention
// (native/src/native_full_attention.hip.cpp:681-765): write the new K/V row,
// then softmax(q K^T / 16) V for 16 query heads over 2 KV heads (head h reads
// KV head h/8), D = 256, cache rows [0, cache_end).  The reference streams
// the whole cache through hipBLASLt QK, 1-5 softmax kernels over bf16 scores
// and a hipBLASLt PV; here one pass streams K and V exactly once.
//
// Layout: k_cache, v_cache are [capacity, 2, 256] bf16 (token stride 512).
//
// Kernel plan (HBM-bound, 2048 bytes of K+V per token):
//  * grid = nsplit x 2 KV heads (head = workgroup index % 2, so each XCD
//    serves one head); the cache's 32-token blocks are dealt to
//    the splits round-robin (and to the 4 waves of a split in turn), so the
//    grid sweeps the cache as one contiguous window.
//  * K and V are read as whole 512-byte half-rows (two rows per load
//    instruction) by unconditional buffer loads -- rows past cache_end read
//    as zeros, so no load sits in a branch and the compiler's in-order wait
//    counts keep the next block's loads in flight; K then passes through
//    the wave's LDS slot into the MFMA operand layout.
//  * per block: S^T = K Q^T on MFMA 16x16x32 (A = K from LDS, B = the 8
//    query heads of the group, padded to 16 columns),
//    online softmax per head in fp32 (exp2 domain), then O^T += V^T P^T on
//    MFMA with V staged row-major in LDS and read transposed with
//    ds_read_b64_tr_b16.  The P^T operand is the S^T accumulator itself
//    (same lane mapping), so no shuffles are needed between the two MFMAs.
//  * the 4 waves merge in LDS; the workgroup writes one (m, l, O) partial.
//  * decode_gqa_combine_wave merges the partials of all splits (one wave per
//    query head and 16 dims, one load round, shuffle reductions), normalises,
//    optionally applies the sigmoid output gate and writes bf16.  Tried and measured slower on MI355X: merging in the
//    split kernel (a "last workgroup merges" tree or a grid barrier: device-
//    scope fences write back/invalidate the whole L2, and workgroups polling
//    a counter slow the stream), and dynamic tail balancing through global
//    ticket counters (atomic latency and contention exceed the tail saved).
#include "common.h"

#include <mutex>

namespace q36 {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecBlock = 32;          // tokens per wave iteration
constexpr int kVPitch = 544;           // LDS row pitch in bytes (512 + 32)
constexpr int kVLds = kDecWaves * kDecBlock * kVPitch;   // 69632 bytes
constexpr int kQPitch = 528;           // LDS row pitch of the Q^T operand
constexpr int kKPitch = 528;           // LDS row pitch of the staged K rows
constexpr int kKLds = kDecWaves * kDecBlock * kKPitch;   // 67584 bytes
constexpr int kDecLds = kVLds + kKLds + 16 * kQPitch;    // 145664 bytes

constexpr unsigned kMaxSplits = 256;
// Default split count: 128 splits x 2 KV heads = one workgroup per CU.
// (Measured on MI355X at 128K: 128 splits beat 256 -- two workgroups per CU
// -- and 64..192; one workgroup holding both KV heads was no faster.)
constexpr unsigned kTargetSplits = 128;

// RoPE inverse frequencies for the fused decode step (this translation
// unit's copy; see rope_inv_freq_host).
__constant__ float c_dec_inv_freq[kRotaryPairs];

// Raw inputs of the fused decode step (qwen36_decode_step): the q-projection
// row [16 heads x (256 query | 256 gate)], the raw k and v rows [2 x 256]
// and the head-norm weights.  Unused (null) for qwen36_decode_gqa.
struct FuseArgs {
  const bf16* q_gate;
  const bf16* k_raw;
  const bf16* v_raw;
  const bf16* q_w;
  const bf16* k_w;
};

// Workspace carve-up (fp32).
struct DecodeWs {
  float* o;            // [2][nsplit][8][256] split partials (unnormalised)
  float* ml;           // [2][nsplit][8][2]   running max (log2 domain), sum
};

__device__ __forceinline__ void store_partial(float* o, float* ml,
                                              const float* acc, float M,
                                              float L) {
  *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
  *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
  if ((threadIdx.x & 31) == 0) {
    ml[0] = M;
    ml[1] = L;
  }
}

template <bool kFuse>
__global__ __launch_bounds__(256, 1) void decode_gqa_split_kernel(
    const bf16* __restrict__ q, bf16* __restrict__ k_cache,
    bf16* __restrict__ v_cache, const bf16* __restrict__ k_new,
    const bf16* __restrict__ v_new, unsigned position, unsigned cache_end,
    unsigned nsplit, DecodeWs ws, FuseArgs fz) {
  __shared__ __attribute__((aligned(16))) char lds[kDecLds];
  // Workgroup i streams KV head i % 2: consecutive workgroups are dealt to
  // the 8 XCDs in turn, so each XCD serves one head (the half of every
  // 1 KiB cache row that head owns).  Measured on MI355X against a
  // (split, head) grid that gives every XCD both heads: 128K 496 vs 507 us,
  // 32K 194 vs 210 us per 10 layers, same box.
  const int kvh = blockIdx.x & 1;
  const unsigned split = blockIdx.x >> 1;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;   // MFMA row/column index
  const int lg = lane >> 4;   // 16-lane group
  // 32-token blocks are dealt round-robin: split s owns blocks s, s+nsplit,
  // ... and its wave w takes every 4th of those.  At any moment the whole
  // grid therefore reads one contiguous window of the cache (both KV heads of
  // each row at about the same time), which keeps HBM pages and channels
  // evenly and sequentially used.
  const unsigned end = cache_end;
  // The workgroup that owns the new row's block writes the row into the
  // cache (this KV head's half: the copy of k_new / v_new, or in the fused
  // step K after head norm and RoPE and V raw) and is its only reader, so it
  // then streams that row from the cache like every other.  If the row lies
  // in one of the first blocks (round < 4: short caches) the write completes
  // before any load is issued; otherwise it overlaps the first loads and the
  // workgroup barrier after Q staging orders it before the row's block is
  // read.  Raw inputs of the fused step are requested before the first K/V
  // block so that their (short) round trip does not queue behind it.
  const bool owner = (position / kDecBlock) % nsplit == split;
  const bool new_row = owner && (kFuse || k_new != nullptr);
  float xq[2][4], xk[4];
  bf16x4 vrow;
  if constexpr (kFuse) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bf16x4 r = *reinterpret_cast<const bf16x4*>(
          fz.q_gate + (size_t)(kvh * kGroup + 2 * wave + u) * 2 * kD + 4 * lane);
#pragma unroll
      for (int e = 0; e < 4; ++e) xq[u][e] = bf2f(r[e]);
    }
    if (owner && wave == 0) {
      const bf16x4 r = *reinterpret_cast<const bf16x4*>(fz.k_raw + kvh * kD + 4 * lane);
#pragma unroll
      for (int e = 0; e < 4; ++e) xk[e] = bf2f(r[e]);
    }
    if (owner && wave == 1) vrow = *reinterpret_cast<const bf16x4*>(fz.v_raw + kvh * kD + 4 * lane);
  }
  auto write_new_row = [&]() {
    const size_t o = ((size_t)position * kHkv + kvh) * kD;
    if constexpr (kFuse) {
      if (wave == 0) {
        float y[4];
        float cs[4], sn[4];
        rope_cos_sin_wave(position, c_dec_inv_freq, cs, sn);
        head_norm_rope_wave(xk, fz.k_w, cs, sn, y);
        bf16x4 yb;
#pragma unroll
        for (int e = 0; e < 4; ++e) yb[e] = f2bf(y[e]);
        *reinterpret_cast<bf16x4*>(k_cache + o + 4 * lane) = yb;
      } else if (wave == 1) {
        *reinterpret_cast<bf16x4*>(v_cache + o + 4 * lane) = vrow;
      }
    } else if (wave == 0) {
      if (lane < 32) {
        reinterpret_cast<uint4*>(k_cache + o)[lane] =
            reinterpret_cast<const uint4*>(k_new + kvh * kD)[lane];
      } else {
        reinterpret_cast<uint4*>(v_cache + o)[lane - 32] =
            reinterpret_cast<const uint4*>(v_new + kvh * kD)[lane - 32];
      }
    }
  };
  const bool early_row = new_row && (position / kDecBlock) / nsplit < (unsigned)kDecWaves;
  if (early_row) {
    write_new_row();
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }


  f32x4 o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale = 0.0625f * kLog2e;
  char* vbuf = lds + wave * kDecBlock * kVPitch;

  // Software pipeline: the K fragments and V rows of the next block are
  // requested as soon as the registers holding the current block are free,
  // so HBM latency overlaps the softmax and PV work.
  // K and V rows are both read as whole 512-byte half-rows (two rows per
  // load instruction, every 128-byte line fully used); K then passes
  // through this wave's LDS slot into the MFMA operand layout (16 rows x 64
  // bytes per operand read).  Measured on MI355X with a read-only kernel
  // over a 128K cache: reading K directly in the operand layout (16 rows x
  // 64 bytes per load instruction, half lines) streams a layer in 41.8 us,
  // whole half-rows in 38.8 us.
  u32x4 kr[16];
  u32x4 vr[16];
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)k_cache, 0, (int)(end * (unsigned)kKvRow * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)v_cache, 0, (int)(end * (unsigned)kKvRow * 2u), 0x00020000);
  auto load_k = [&](unsigned t0) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const unsigned tok = t0 + 2 * c + (lane >> 5);
      const int off = (int)(tok * (unsigned)kKvRow * 2u + kvh * kD * 2 + (lane & 31) * 16);
      kr[c] = __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 2);
    }
  };
  char* kbuf = lds + kVLds + wave * kDecBlock * kKPitch;
  auto stage_k = [&]() {
#pragma unroll
    for (int c = 0; c < 16; ++c)
      *reinterpret_cast<u32x4*>(kbuf + (2 * c + (lane >> 5)) * kKPitch + (lane & 31) * 16) = kr[c];
  };
  // V rows: row = 2c + lane/32, 16-byte chunk = lane%32 (fully coalesced).
  auto load_v = [&](unsigned t0) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const unsigned tok = t0 + 2 * c + (lane >> 5);
      const int off = (int)(tok * (unsigned)kKvRow * 2u + kvh * kD * 2 + (lane & 31) * 16);
      vr[c] = __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 2);
    }
  };

  const unsigned stride = nsplit * kDecWaves * kDecBlock;
  unsigned t0 = (split + nsplit * wave) * kDecBlock;
  if (t0 < end) {
    load_k(t0);
    load_v(t0);
  }

  // Q staging overlaps the first block's HBM latency.
  // B operand Q^T: column li = query head (kvh*8 + li) for li < 8, zero
  // padding otherwise; kept in LDS (rows of kQPitch bytes) and re-read per
  // block to free registers for the load pipeline.  Reduction step s covers
  // dims s*32 + 8*lg .. +8, so one K load instruction reads 16 rows x 64
  // contiguous bytes.
  char* qs = lds + kVLds + kKLds;
  const bool late_row = new_row && !early_row;
  if (late_row) write_new_row();
  if constexpr (kFuse) {
    // Head norm + RoPE of this group's 8 query heads (wave w: heads 2w,
    // 2w+1) straight into the Q^T operand rows; rows 8..15 are zero padding.
    float cs[4], sn[4];
    rope_cos_sin_wave(position, c_dec_inv_freq, cs, sn);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int hh = 2 * wave + u;
      float y[4];
      head_norm_rope_wave(xq[u], fz.q_w, cs, sn, y);
      bf16x4 yb;
#pragma unroll
      for (int e = 0; e < 4; ++e) yb[e] = f2bf(y[e]);
      *reinterpret_cast<bf16x4*>(qs + hh * kQPitch + 8 * lane) = yb;
    }
    {
      const int r = kGroup + (threadIdx.x >> 5), c = threadIdx.x & 31;
      *reinterpret_cast<uint4*>(qs + r * kQPitch + c * 16) = uint4{0u, 0u, 0u, 0u};
    }
  } else {
    const int r = threadIdx.x >> 4, c = threadIdx.x & 15;   // 16 rows x 16 chunks
    uint4 a = uint4{0u, 0u, 0u, 0u}, b = uint4{0u, 0u, 0u, 0u};
    if (r < kGroup) {
      const uint4* src = reinterpret_cast<const uint4*>(q + (size_t)(kvh * kGroup + r) * kD);
      a = src[c];
      b = src[c + 16];
    }
    *reinterpret_cast<uint4*>(qs + r * kQPitch + c * 16) = a;
    *reinterpret_cast<uint4*>(qs + r * kQPitch + (c + 16) * 16) = b;
  }
  // the new row's stores complete before the barrier (the waves that wrote)
  if (late_row && wave < 2) __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const char* qrow = qs + li * kQPitch + lg * 16;
  const char* krow0 = kbuf + li * kKPitch + lg * 16;
  for (; t0 < end; t0 += stride) {
    const unsigned tn = t0 + stride;
    // K of this block into the operand layout; the next block's K is then
    // requested at once (its registers are free)
    stage_k();
    if (tn < end) load_k(tn);
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8 qf = *reinterpret_cast<const bf16x8*>(qrow + 64 * s);
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(krow0 + 64 * s);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(krow0 + 16 * kKPitch + 64 * s);
      s0 = mfma16x16x32(k0, qf, s0);
      s1 = mfma16x16x32(k1, qf, s1);
    }
    // Lane holds S^T[token t0 + 16*tt + 4*lg + r][head li].
    float sc[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const unsigned ta = t0 + 4 * lg + r;
      sc[r] = ta < end ? s0[r] * scale : -INFINITY;
      sc[4 + r] = ta + 16 < end ? s1[r] * scale : -INFINITY;
    }
    float mx = sc[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) mx = fmaxf(mx, sc[r]);
    mx = wave_max_xor(mx, 16);
    mx = wave_max_xor(mx, 32);
    const float mnew = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      p[r] = __builtin_amdgcn_exp2f(sc[r] - mnew);
      psum += p[r];
    }
    l = l * alpha + psum;
    m = mnew;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] *= alpha;

    // Stage V (row-major, padded pitch) in this wave's private LDS slot.
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      *reinterpret_cast<u32x4*>(vbuf + (2 * c + (lane >> 5)) * kVPitch +
                                (lane & 31) * 16) = vr[c];
    }
    if (tn < end) load_v(tn);
    bf16x8 pb;
#pragma unroll
    for (int r = 0; r < 8; ++r) pb[r] = f2bf(p[r]);
    // O^T[d][head] += V^T[d][tok] P^T[tok][head]; reduction slots (lg, e)
    // map to tokens 4*lg + e (e < 4) and 16 + 4*lg + (e-4) (e >= 4).
    const char* row_a = vbuf + (4 * lg + (li >> 2)) * kVPitch + (li & 3) * 8;
    const char* row_b = row_a + 16 * kVPitch;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const i16x4 a0 = lds_read_tr16(row_a + dt * 32);
      const i16x4 a1 = lds_read_tr16(row_b + dt * 32);
      o[dt] = mfma16x16x32(cat_bf16x8(a0, a1), pb, o[dt]);
    }
  }
  // Row sums are split over the 4 lane groups; max is already uniform.
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);

  // Merge the 4 waves: O^T lane (head li, dims dt*16 + 4*lg + r).
  __syncthreads();
  float* mo = reinterpret_cast<float*>(lds);          // [4][8][256]
  float* mml = mo + kDecWaves * kGroup * kD;           // [4][8][2]
  if (li < kGroup) {
    float* dst = mo + (wave * kGroup + li) * kD + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
      *reinterpret_cast<f32x4*>(dst + dt * 16) = o[dt];
    if (lg == 0) {
      mml[(wave * kGroup + li) * 2 + 0] = m;
      mml[(wave * kGroup + li) * 2 + 1] = l;
    }
  }
  __syncthreads();
  const int h = threadIdx.x >> 5;          // 0..7: head within the group
  const int d0 = (threadIdx.x & 31) * 8;   // 8 dims per thread
  {
    float mw[kDecWaves], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      mw[w] = mml[(w * kGroup + h) * 2];
      M = fmaxf(M, mw[w]);
    }
    float L = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float f = (mw[w] == -INFINITY) ? 0.f : exp2f(mw[w] - M);
      L += f * mml[(w * kGroup + h) * 2 + 1];
      const float* src = mo + (w * kGroup + h) * kD + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += f * src[e];
    }
    const size_t slot = ((size_t)kvh * nsplit + split) * kGroup + h;
    store_partial(ws.o + slot * kD + d0, ws.ml + slot * 2, acc, M, L);
  }

}

// Combine: one wave per (query head, 16 dims), grid = 256 single-wave
// workgroups.  Every load (the split partials, their (m, l), the gate) is
// issued up front: one memory round trip.
constexpr int kCombineDims = 16;
static_assert(kMaxSplits % 16 == 0, "16 split groups per combine wave");

// Lane = (split group sg = lane / 4, dim quad dq = lane % 4); split group sg
// takes splits sg, sg + 16, ...  The max, the weights 2^(m - M) and the sums
// reduce over the 16 split groups with xor shuffles (lane bits 2..5): no LDS,
// no barrier.  Measured on MI355X against a 4-wave combine with LDS
// reductions: -0.2 to -0.7 us per layer.
__global__ __launch_bounds__(64) void decode_gqa_combine_wave_kernel(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    unsigned nsplit, const bf16* __restrict__ gate, unsigned gate_head_stride,
    bf16* __restrict__ out) {
  const int head = blockIdx.x & 15;
  const int kvh = head / kGroup, hh = head % kGroup;
  const int lane = threadIdx.x;
  const int dq = lane & 3, sg = lane >> 2;
  const int d0 = (blockIdx.x >> 4) * kCombineDims + 4 * dq;
  const size_t base = (size_t)kvh * nsplit * kGroup + hh;
  constexpr int kPer = kMaxSplits / 16;   // at most 16 splits per group
  float2 ml[kPer];
  f32x4 os[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const unsigned sp = sg + 16 * u;
    if (sp < nsplit) {
      ml[u] = *reinterpret_cast<const float2*>(ws_ml + (base + (size_t)sp * kGroup) * 2);
      os[u] = *reinterpret_cast<const f32x4*>(ws_o + (base + (size_t)sp * kGroup) * kD + d0);
    } else {
      ml[u] = float2{-INFINITY, 0.f};
      os[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // the gate is requested after the partials (and every lane reads it, kept
  // as raw bits), so its load joins their round trip instead of preceding it
  bf16 graw[4] = {};
  if (gate != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) graw[e] = gate[(size_t)head * gate_head_stride + d0 + e];
  }
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < kPer; ++u) mx = fmaxf(mx, ml[u].x);
  mx = wave_max_xor(mx, 4);
  mx = wave_max_xor(mx, 8);
  mx = wave_max_xor(mx, 16);
  mx = wave_max_xor(mx, 32);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const float f = ml[u].x == -INFINITY ? 0.f : exp2f(ml[u].x - mx);
    L += f * ml[u].y;
    acc += f * os[u];
  }
#pragma unroll
  for (int o = 4; o < 64; o <<= 1) {
    L += __shfl_xor(L, o, 64);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
  }
  if (sg == 0) {
    bf16x4 ob;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bf16 x = f2bf(acc[e] / L);
      if (gate != nullptr) {
        const bf16 sg_b = f2bf(1.0f / (1.0f + expf(-bf2f(graw[e]))));
        x = f2bf(bf2f(x) * bf2f(sg_b));
      }
      ob[e] = x;
    }
    *reinterpret_cast<bf16x4*>(out + head * kD + d0) = ob;
  }
}

unsigned choose_split_tokens(unsigned cache_end) {
  // Aim for one workgroup per CU (256 CUs) over both KV heads while keeping
  // at least one 32-token block per wave.
  const unsigned target_splits = kTargetSplits;
  unsigned per = (cache_end + target_splits - 1) / target_splits;
  const unsigned quantum = kDecWaves * kDecBlock;  // 128
  per = (per + quantum - 1) / quantum * quantum;
  if (per < quantum) per = quantum;
  return per;
}

size_t workspace_bytes(unsigned nsplit) {
  return (size_t)nsplit * kHkv * kGroup * (kD + 2) * sizeof(float);
}

// Library-owned split-partial buffer of qwen36_decode_gqa_noalloc: the
// workspace of the largest split count (256), one copy per GPU, held until
// the process ends.  Host code never passes `scratch` itself to a kernel
// (its host-side name is not a device address): the device address is
// taken once per device with hipGetSymbolAddress and kept in g_scratch_ptr.
constexpr size_t kScratchBytes = (size_t)kMaxSplits * kHkv * kGroup * (kD + 2) * sizeof(float);
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_init_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
bool g_dec_freq_ready[kMaxDevices] = {};

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT size_t qwen36_decode_gqa_workspace_bytes(unsigned cache_end,
                                                    unsigned split_tokens) {
  if (cache_end == 0) return 0;
  const unsigned per = split_tokens ? split_tokens : choose_split_tokens(cache_end);
  return workspace_bytes((cache_end + per - 1) / per);
}

static int launch_decode(bool fuse, const void* q, const void* k_new,
                         const void* v_new, const FuseArgs& fz, void* k_cache,
                         void* v_cache, unsigned position, unsigned cache_end,
                         unsigned capacity, const void* gate,
                         unsigned gate_head_stride, void* out, void* workspace,
                         size_t workspace_bytes_given, unsigned split_tokens,
                         void* stream) {
  const unsigned per = split_tokens ? split_tokens : choose_split_tokens(cache_end);
  const unsigned nsplit = (cache_end + per - 1) / per;
  if (nsplit > kMaxSplits) return Q36_EINVAL;
  if (workspace_bytes_given < workspace_bytes(nsplit)) return Q36_EINVAL;
  DecodeWs ws;
  ws.o = static_cast<float*>(workspace);
  ws.ml = ws.o + (size_t)nsplit * kHkv * kGroup * kD;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto kernel = fuse ? decode_gqa_split_kernel<true> : decode_gqa_split_kernel<false>;
  hipLaunchKernelGGL(kernel, dim3(nsplit * kHkv), dim3(256), 0, st,
                     static_cast<const bf16*>(q), static_cast<bf16*>(k_cache),
                     static_cast<bf16*>(v_cache), static_cast<const bf16*>(k_new),
                     static_cast<const bf16*>(v_new), position, cache_end, nsplit, ws,
                     fz);
  hipLaunchKernelGGL(decode_gqa_combine_wave_kernel, dim3(kHq * (kD / kCombineDims)), dim3(64),
                     0, st, ws.o, ws.ml, nsplit, static_cast<const bf16*>(gate),
                     gate_head_stride, static_cast<bf16*>(out));
  return static_cast<int>(hipGetLastError());
}

// One-time per-device set-up under g_init_mutex (callers may make their first
// calls from several host threads at once).
static int ensure_dec_inv_freq() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(g_init_mutex);
  if (g_dec_freq_ready[dev]) return Q36_OK;
  float h[kRotaryPairs];
  rope_inv_freq_host(h);
  const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(c_dec_inv_freq), h, sizeof(h));
  if (e != hipSuccess) return (int)e;
  g_dec_freq_ready[dev] = true;
  return Q36_OK;
}

// Device address of this device's `scratch` (taken on the first call on
// each device, with that device current).
static int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(g_init_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return Q36_EINVAL;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return Q36_OK;
}

Q36_EXPORT int qwen36_decode_gqa(const void* q, const void* k_new,
                                 const void* v_new, void* k_cache,
                                 void* v_cache, unsigned position,
                                 unsigned cache_end, unsigned capacity,
                                 const void* gate, unsigned gate_head_stride,
                                 void* out, void* workspace,
                                 size_t workspace_bytes_given,
                                 unsigned split_tokens, void* stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      out == nullptr || workspace == nullptr || cache_end == 0 ||
      cache_end > capacity || capacity > kMaxTokens ||
      ((k_new == nullptr) != (v_new == nullptr)) ||
      (k_new != nullptr && position >= cache_end) ||
      (split_tokens % (kDecWaves * kDecBlock)) != 0)
    return Q36_EINVAL;
  return launch_decode(false, q, k_new, v_new, FuseArgs{}, k_cache, v_cache, position,
                       cache_end, capacity, gate, gate_head_stride, out, workspace,
                       workspace_bytes_given, split_tokens, stream);
}

Q36_EXPORT int qwen36_decode_step(const void* q_gate, const void* k_raw,
                                  const void* v_raw, const void* q_norm_weight,
                                  const void* k_norm_weight, void* k_cache,
                                  void* v_cache, unsigned position,
                                  unsigned cache_end, unsigned capacity,
                                  void* out, void* workspace,
                                  size_t workspace_bytes_given,
                                  unsigned split_tokens, void* stream) {
  if (q_gate == nullptr || k_raw == nullptr || v_raw == nullptr ||
      q_norm_weight == nullptr || k_norm_weight == nullptr || k_cache == nullptr ||
      v_cache == nullptr || out == nullptr || workspace == nullptr || cache_end == 0 ||
      cache_end > capacity || capacity > kMaxTokens || position >= cache_end ||
      (split_tokens % (kDecWaves * kDecBlock)) != 0 ||
      (reinterpret_cast<uintptr_t>(q_gate) % 8) != 0 ||
      (reinterpret_cast<uintptr_t>(k_raw) % 8) != 0 ||
      (reinterpret_cast<uintptr_t>(v_raw) % 8) != 0 ||
      (reinterpret_cast<uintptr_t>(k_cache) % 8) != 0 ||
      (reinterpret_cast<uintptr_t>(v_cache) % 8) != 0)
    return Q36_EINVAL;
  const int st = ensure_dec_inv_freq();
  if (st != Q36_OK) return st;
  FuseArgs fz;
  fz.q_gate = static_cast<const bf16*>(q_gate);
  fz.k_raw = static_cast<const bf16*>(k_raw);
  fz.v_raw = static_cast<const bf16*>(v_raw);
  fz.q_w = static_cast<const bf16*>(q_norm_weight);
  fz.k_w = static_cast<const bf16*>(k_norm_weight);
  // The gate is the second half of each head's 512-wide q-projection slice.
  return launch_decode(true, nullptr, nullptr, nullptr, fz, k_cache, v_cache, position,
                       cache_end, capacity, static_cast<const bf16*>(q_gate) + kD, 2 * kD,
                       out, workspace, workspace_bytes_given, split_tokens, stream);
}

Q36_EXPORT int qwen36_decode_gqa_noalloc(const void* q, const void* k_new,
                                         const void* v_new, void* k_cache,
                                         void* v_cache, unsigned position,
                                         unsigned cache_end, unsigned capacity,
                                         const void* gate, unsigned gate_head_stride,
                                         void* out, unsigned split_tokens,
                                         void* stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      out == nullptr || cache_end == 0 || cache_end > capacity || capacity > kMaxTokens ||
      ((k_new == nullptr) != (v_new == nullptr)) ||
      (k_new != nullptr && position >= cache_end) ||
      (split_tokens % (kDecWaves * kDecBlock)) != 0)
    return Q36_EINVAL;
  const unsigned per = split_tokens ? split_tokens : choose_split_tokens(cache_end);
  const unsigned nsplit = (cache_end + per - 1) / per;
  if (nsplit > kMaxSplits || workspace_bytes(nsplit) > kScratchBytes) return Q36_EINVAL;
  void* ws = nullptr;
  const int st = scratch_ptr(&ws);
  if (st != Q36_OK) return st;
  return launch_decode(false, q, k_new, v_new, FuseArgs{}, k_cache, v_cache, position,
                       cache_end, capacity, gate, gate_head_stride, out, ws, kScratchBytes,
                       split_tokens, stream);
}
