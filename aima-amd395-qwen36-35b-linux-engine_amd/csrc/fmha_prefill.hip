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
//  * workgroup = 8 waves = 256 query rows of one head; wave = 32 rows; one
//    workgroup per CU (two waves per SIMD) shares each staged K/V tile
//    among 256 rows (measured 5-7% faster than two 4-wave workgroups per
//    CU, which stage every tile twice).  Short square prompts (fewer than
//    256 such workgroups) use 4- or 2-wave workgroups (128 or 64 rows).
//  * per 32-key tile: K and V are staged in LDS (padded row-pair blocks, so
//    every LDS address is a per-lane base plus an immediate); S^T = K Q^T on
//    v_mfma_f32_32x32x16_bf16 (A = K from LDS, B = Q^T held in registers for
//    the whole kernel), online softmax per row
//    in fp32 (exp2 domain), O^T += V^T P^T (A = V^T read with
//    ds_read_b64_tr_b16, B = P^T taken straight from the S^T accumulator).
//  * LDS operand reads run 4 MFMAs ahead of their use (register rings whose
//    issue order is pinned by sched_group_barrier), so the dependent QK^T
//    chain and the PV MFMAs do not wait on LDS latency.
//  * K/V tiles are fetched straight into LDS (global_load_lds_dwordx4, no
//    register staging) into a double buffer (64 KiB), so the next tile's
//    HBM/L2 latency overlaps the current tile's MFMA work; the two waves
//    on each SIMD let one wave's softmax overlap the other's MFMAs.
//  * no per-tile row max: the reference max is the first tile's, raised
//    (with a rescale of O) only when a tile's probabilities would exceed
//    2^20, which the per-lane probability sum detects.
//  * blockIdx -> (KV head, query head, query tile) is XCD-aware: the 8 XCDs
//    receive workgroups round-robin, so XCDs 0-3 serve KV head 0 and 4-7 KV
//    head 1 (their L2s then hold one head's K/V), and every XCD issues its
//    heaviest (latest) causal tiles first.
#include "common.h"

#include <mutex>

namespace q36 {
namespace {

constexpr int kFmRowsPerWave = 32;
constexpr int kFmKv = 32;                             // keys per tile
constexpr int kRowBytes = kD * 2;                     // 512
constexpr int kTokBytes = kHkv * kD * 2;              // 1024: one cache row
// LDS tile layout: block b (0..15) holds key rows b and b+16 back to back
// (1 KiB, one direct-to-LDS instruction) followed by padding, so that every
// LDS address below is a per-lane base plus a compile-time offset and both
// access patterns are bank-conflict-free:
//  * K blocks are 1040 B apart: 16 rows at one 16-byte column fall in 16
//    distinct 16-byte bank groups (ds_read_b128 A operand);
//  * V blocks are 1088 B apart: 8 rows x 64 bytes (ds_read_b64_tr_b16) take
//    the minimum two passes.
constexpr int kKBlk = 1040, kVBlk = 1088;
constexpr int kKTile = 16 * kKBlk;                    // 16640
constexpr int kVTile = 16 * kVBlk;                    // 17408
constexpr int kFmStage = kKTile + kVTile;             // 34048
constexpr int kFmLds = 2 * kFmStage;                  // 68096: double buffer
// Gated kernels also prefetch the gate values of output rounds 0-1 (dims
// 0-127 of the head) of their 256 rows into LDS after the ring.
constexpr int kFmGateLds = 256 * 256;
constexpr int kFmLdsGated = kFmLds + kFmGateLds;      // 133632

typedef __attribute__((address_space(3))) void lds_void;

// Split-K partials (kSplit): workgroup (q tile, chunk, head) writes its
// unnormalised O rows and (m, l) for keys [chunk * chunk_keys, +chunk_keys).
struct SplitArgs {
  float* o;             // [tile][chunk][head][256 rows][256]
  float* ml;            // [tile][chunk][head][256 rows][2]
  unsigned chunk_keys;  // multiple of 32
  unsigned n_chunks;
};

// Gated output (kGate): out_bf16[row][h*256 + d] = gate_bf16(O, gate[row *
// gate_stride + h*512 + 256 + d]) -- the gate half of each head's 512-wide
// slice of the fused q projection -- in place of the fp32 attention rows.
struct GateArgs {
  const bf16* gate;
  unsigned gate_stride;   // elements between token rows of the q projection
  bf16* out;
};

template <int kFmWaves, bool kSplit, bool kGate = false>
__global__ __launch_bounds__(64 * kFmWaves, 1) void fmha_prefill_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, float* __restrict__ out, unsigned q_tokens,
    unsigned kv_tokens, unsigned n_qtiles, SplitArgs sp, GateArgs ga) {
  static_assert(!(kSplit && kGate), "split partials are gated by the combine");
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int kFmRows = kFmWaves * kFmRowsPerWave;
  constexpr int kFmLoadsPerWave = 16 / kFmWaves;       // 16 row-pair blocks per tile

  // XCD-aware tile mapping (see header); split: (tile, chunk, head).
  const unsigned b = blockIdx.x;
  int kvh, head;
  unsigned qtile, chunk = 0;
  if constexpr (kSplit) {
    head = (int)(b % kHq);
    kvh = head / kGroup;
    qtile = (b / kHq) / sp.n_chunks;
    chunk = (b / kHq) % sp.n_chunks;
  } else {
    const unsigned xcd = b & 7u, n = b >> 3;
    kvh = xcd >> 2;
    head = kvh * kGroup + (xcd & 3) * 2 + (n & 1);
    qtile = n_qtiles - 1 - (n >> 1);
  }
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
  // key range of this workgroup: whole rows, or one chunk of them
  const unsigned kv_first = kSplit ? chunk * sp.chunk_keys : 0u;
  const unsigned kv_stop = kSplit ? min(kv_end, kv_first + sp.chunk_keys) : kv_end;
  if (kSplit && kv_first >= kv_end) return;   // past the tile's last key

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

  // Direct global->LDS fetch through buffer resources (base in SGPRs; rows at
  // or past kv_end are out of bounds and read as zeros).  Wave instruction j
  // fills block 2*wave + j: lanes 0-31 key row b, lanes 32-63 key row b+16.
  const int nrec = (int)(kv_end * (unsigned)kTokBytes);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)k, 0, nrec, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)v, 0, nrec, 0x00020000);
  const int fvoff = (kFmLoadsPerWave * wave + 16 * (lane >> 5)) * kTokBytes +
                    kvh * kRowBytes + (lane & 31) * 16;
  // gated: the gate values of output rounds 0-1 of this workgroup's rows
  // (row-major [256 rows][256 B]), fetched now so they are resident when the
  // epilogue starts; rows past the end read as zeros.
  if constexpr (kGate) {
    const unsigned rows_here = min(q_tokens - q0, (unsigned)kFmRows);
    const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(ga.gate) + (size_t)q0 * ga.gate_stride + head * 2 * kD + kD, 0,
        (int)(rows_here * ga.gate_stride * 2), 0x00020000);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r0 = wave * kFmRowsPerWave + 4 * j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          grs, (lds_void*)(lds + kFmLds + r0 * 256), 16,
          (int)(((r0 + (lane >> 4)) * ga.gate_stride) * 2 + (lane & 15) * 16), 0, 0, 0);
    }
  }
  auto fetch = [&](unsigned kv0, int stage) {
    char* ks = lds + stage * kFmStage;
    char* vs = ks + kKTile;
    const int soff = (int)(kv0 * (unsigned)kTokBytes);
#pragma unroll
    for (int j = 0; j < kFmLoadsPerWave; ++j) {
      const int blk = kFmLoadsPerWave * wave + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(ks + blk * kKBlk), 16,
                                               fvoff + j * kTokBytes, soff, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(vs + blk * kVBlk), 16,
                                               fvoff + j * kTokBytes, soff, 0, 0);
    }
  };

  // Per-lane LDS bases.  K A operand: key row lj, 16-byte chunk 2*st + lg.
  const int kbase = (lj & 15) * kKBlk + (lj >> 4) * kRowBytes + lg * 16;
  // V^T (transposed read): for step st and half h (keys +8), lane reads row
  // 16*st + 8*h + x, x = 4*lg + (lane%16)/4, 8 bytes at column
  // 32*((lane/16)&1) + 8*(lane%4) within the 64-byte block of dims dt.
  const int grp = lane >> 4, m16 = lane & 15;
  const int vx = 4 * lg + (m16 >> 2);
  const int vbase = vx * kVBlk + 32 * (grp & 1) + 8 * (m16 & 3);

  const unsigned t_first = kv_first / kFmKv;
  const unsigned n_tiles = (kv_stop + kFmKv - 1) / kFmKv;
  fetch(kv_first, t_first & 1);
  for (unsigned t = t_first; t < n_tiles; ++t) {
    const unsigned kv0 = t * kFmKv;
    const int stage = t & 1;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's fetches of tile t landed
    __syncthreads();                 // ... and every wave's; tile t-1 consumed
    if (t + 1 < n_tiles) fetch(kv0 + kFmKv, stage ^ 1);
    if (kv0 > wave_lim) continue;    // every key of the tile is masked for us
    const char* kp = lds + stage * kFmStage + kbase;
    const char* vp = lds + stage * kFmStage + kKTile + vbase;

    // S^T[key][row] for the 32-key tile.
    // K operands go through a 4-deep register ring: the read for step st + 4
    // is issued right after step st's MFMA (the sched_group_barrier sequence
    // pins that order; left alone, the scheduler keeps only 2 reads in flight
    // and each MFMA of the dependent chain waits a full LDS latency).
    bf16x8 kr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kr[i] = *reinterpret_cast<const bf16x8*>(kp + i * 32);
    f32x16 s0 = f32x16{};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      s0 = mfma32x32x16(kr[st & 3], qf[st], s0);
      if (st + 4 < 16) kr[st & 3] = *reinterpret_cast<const bf16x8*>(kp + (st + 4) * 32);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    // Lane holds keys kv0 + 8*(r/4) + 4*lg + r%4 of its row.
    const bool diag = kv0 + kFmKv - 1 > wave_first + off || kv0 + kFmKv > kv_tokens;
    if (diag) {  // wave-uniform: only diagonal / ragged tiles pay for masking
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const unsigned key = kv0 + 8 * (r >> 2) + 4 * lg + (r & 3);
        s0[r] = (key <= row_lim && key < kv_tokens) ? s0[r] : -INFINITY;
      }
    }
    // Reference max, kept in the scaled log2 domain: m is the row max of the
    // first tile (key 0 is visible to every row) and is raised only when a
    // later tile's p = 2^(s*scale - m) would exceed 2^20.  Each lane's p sum
    // bounds its p values, so no per-tile max is taken on the common path;
    // p up to 2^20 is exact to bf16 rounding and O, l cannot overflow.  An
    // overflowed or non-finite sum also takes the rescale branch, which
    // recomputes P against the new max.
    auto row_max = [&]() {
      float mx = s0[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s0[r]);
      mx = wave_max_xor(mx, 32);
      return mx * scale;
    };
    if (t == t_first) {
      // a row whose keys all precede this chunk sees only masked scores in
      // its first tile (and in every later one): any finite m keeps p = 0
      m = row_max();
      if (kSplit && m == -INFINITY) m = 0.f;
    }
    float psum = 0.f;
    bf16x8 pb[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], scale, -m));
      psum += p0;
      pb[r >> 3][r & 7] = f2bf(p0);
    }
    if (__any(!(psum <= 1048576.0f))) {
      const float mnew = fmaxf(m, row_max());
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] *= alpha;
      m = mnew;
      psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], scale, -m));
        psum += p0;
        pb[r >> 3][r & 7] = f2bf(p0);
      }
    }
    l += psum;

    // O^T[d][row] += V^T[d][key] P^T[key][row]; step st reduction slots
    // (lg, e) <-> keys 16st + 4lg + e and +8 for e >= 4.
    // V^T operands: the same ring, 4 MFMAs (8 transposed reads) deep.
    i16x4 va[4][2];
    auto vread = [&](int i, int slot) {
      const char* p = vp + (i >> 3) * kRowBytes + (i & 7) * 64;
      va[slot][0] = lds_read_tr16(p);
      va[slot][1] = lds_read_tr16(p + 8 * kVBlk);
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) vread(i, i);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o[i & 7] = mfma32x32x16(cat_bf16x8(va[i & 3][0], va[i & 3][1]), pb[i >> 3], o[i & 7]);
      if (i + 4 < 16) vread(i + 4, i & 3);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
  }
  l += __shfl_xor(l, 32, 64);
  if constexpr (kSplit) {
    if (!row_valid) return;
    const size_t item = ((size_t)qtile * sp.n_chunks + chunk) * kHq + head;
    const unsigned r = row - q0;
    float* op = sp.o + (item * kFmRows + r) * kD + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<f32x4*>(op + dt * 32 + 8 * r4) =
            f32x4{o[dt][4 * r4], o[dt][4 * r4 + 1], o[dt][4 * r4 + 2], o[dt][4 * r4 + 3]};
    if (lg == 0) *reinterpret_cast<float2*>(sp.ml + (item * kFmRows + r) * 2) = float2{m, l};
    return;
  } else {
    // The output leaves through LDS in four rounds of 64 dims: each wave
    // stages its 32 rows x 64 dims (8 KiB, 16-byte chunks XOR-swizzled by
    // row so both the staging writes and the row reads are conflict-free)
    // and stores whole 256-byte row segments, instead of 32-byte pieces of
    // 32 rows per store instruction.
    const float inv = row_valid ? 1.0f / l : 0.f;
    const unsigned wrow0 = q0 + wave * kFmRowsPerWave;
    // gated: rounds 0-1 take their gate values from the LDS prefetch; the
    // register loads of rounds 2-3 are issued now and land behind rounds 0-1
    // (rows past the end read the last row's and are not stored)
    bf16x4 gv[2][8];
    if constexpr (kGate) {
      __builtin_amdgcn_s_waitcnt(0);   // this wave's gate prefetch landed
#pragma unroll
      for (int rd = 0; rd < 2; ++rd)
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const unsigned r = min(wrow0 + it * 4 + (lane >> 4), q_tokens - 1);
          gv[rd][it] = *reinterpret_cast<const bf16x4*>(
              ga.gate + (size_t)r * ga.gate_stride + head * 2 * kD + kD + (rd + 2) * 64 +
              (lane & 15) * 4);
        }
    }
    __syncthreads();   // every wave is done with the K/V ring
    char* stg = lds + wave * 8192;
#pragma unroll
    for (int rd = 0; rd < 4; ++rd) {
#pragma unroll
      for (int d2 = 0; d2 < 2; ++d2) {
        const int dt = 2 * rd + d2;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int ch = d2 * 8 + 2 * r4 + lg;   // dims 4 ch .. 4 ch + 3 of the round
          *reinterpret_cast<f32x4*>(stg + lj * 256 + ((ch ^ (lj & 15)) * 16)) =
              f32x4{o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv, o[dt][4 * r4 + 2] * inv,
                    o[dt][4 * r4 + 3] * inv};
        }
      }
      // this wave's staging writes land before its reads (and its reads
      // before the next round's writes): LDS serves one wave in order
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int r = it * 4 + (lane >> 4), ch = lane & 15;
        const f32x4 v = *reinterpret_cast<const f32x4*>(stg + r * 256 + ((ch ^ (r & 15)) * 16));
        if constexpr (kGate) {
          if (wrow0 + r < q_tokens) {
            const bf16x4 g4 =
                rd < 2 ? *reinterpret_cast<const bf16x4*>(lds + kFmLds + (wave * kFmRowsPerWave + r) * 256 +
                                                          rd * 128 + ch * 8)
                       : gv[rd - 2][it];
            *reinterpret_cast<bf16x4*>(ga.out + (size_t)(wrow0 + r) * kQDim + head * kD +
                                       rd * 64 + ch * 4) = gate4_bf16_fast(v, g4);
          }
        } else if (wrow0 + r < q_tokens) {
          // nontemporal: the output is not re-read here (459.0 vs 460.0 us at 8K)
          __builtin_nontemporal_store(
              v, reinterpret_cast<f32x4*>(out + (size_t)(wrow0 + r) * kQDim + head * kD +
                                          rd * 64 + ch * 4));
        }
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
  }
}

// Split-K combine: thread (row, 8 dims) of (q tile, head) merges the live
// chunks' partials: M = max m_c, L = sum l_c 2^(m_c - M), O = sum O_c 2^(m_c -
// M) / L (chunks where the row saw no key have l = 0 and weigh nothing).
// grid = tiles x 16 heads x 16 row groups; block = 512 (16 rows x 32 dims/8).
// Every (m, l) pair, the first four chunks' O partials and the gate are
// requested together (indices clamped to the live range, so every load is
// unconditional and in bounds): one memory round trip for up to four live
// chunks, where per-chunk loads behind the l > 0 test cost two each.
constexpr int kCombineMaxChunks = 16;   // split_plan: n_chunks <= 256 / 16
template <int kMaxC>   // n_chunks <= kMaxC (4 or kCombineMaxChunks)
__global__ __launch_bounds__(512) void fmha_split_combine_kernel(
    const float* __restrict__ po, const float* __restrict__ pml, float* __restrict__ out,
    unsigned q_tokens, unsigned kv_tokens, unsigned chunk_keys, unsigned n_chunks,
    GateArgs ga) {
  constexpr int kRows = 256;
  const unsigned rg = blockIdx.x % 16, head = (blockIdx.x / 16) % kHq, qtile = blockIdx.x / (16 * kHq);
  const unsigned r = rg * 16 + (threadIdx.x >> 5);
  const unsigned row = qtile * kRows + r;
  if (row >= q_tokens) return;
  const int d0 = 8 * (threadIdx.x & 31);
  const unsigned off = kv_tokens - q_tokens;
  const unsigned kv_end = min(kv_tokens, min(qtile * kRows + kRows, q_tokens) + off);
  const unsigned live = (kv_end + chunk_keys - 1) / chunk_keys;   // 1 .. n_chunks
  auto item_of = [&](unsigned c) {
    return ((size_t)qtile * n_chunks + min(c, live - 1)) * kHq + head;
  };
  float2 ml[kMaxC];
#pragma unroll
  for (int c = 0; c < kMaxC; ++c)
    ml[c] = *reinterpret_cast<const float2*>(pml + (item_of(c) * kRows + r) * 2);
  f32x4 oa[4], ob[4];
  auto load_o = [&](int c0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4* src = reinterpret_cast<const f32x4*>(po + (item_of(c0 + j) * kRows + r) * kD + d0);
      oa[j] = src[0];
      ob[j] = src[1];
    }
  };
  load_o(0);
  // gated: the gate row (any valid address otherwise; the value is unused)
  const bf16* gp = ga.out != nullptr
                       ? ga.gate + (size_t)row * ga.gate_stride + head * 2 * kD + kD + d0
                       : reinterpret_cast<const bf16*>(po + (item_of(0) * kRows + r) * kD + d0);
  const bf16x8 g = *reinterpret_cast<const bf16x8*>(gp);
  __builtin_amdgcn_sched_barrier(0);
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < kMaxC; ++c)
    if ((unsigned)c < live && ml[c].y > 0.f) M = fmaxf(M, ml[c].x);
  float L = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int c0 = 0; c0 < kMaxC; c0 += 4) {
    if ((unsigned)c0 >= live) break;
    if (c0 > 0) load_o(c0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float2 m_l = ml[c0 + j];
      if ((unsigned)(c0 + j) < live && m_l.y > 0.f) {
        const float w = __builtin_amdgcn_exp2f(m_l.x - M);
        L += w * m_l.y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] += w * oa[j][e];
          acc[4 + e] += w * ob[j][e];
        }
      }
    }
  }
  const float inv = 1.0f / L;
  if (ga.out != nullptr) {   // gated bf16 rows (see GateArgs)
    const bf16x4 lo = gate4_bf16_fast(f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv},
                                      bf16x4{g[0], g[1], g[2], g[3]});
    const bf16x4 hi = gate4_bf16_fast(f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv},
                                      bf16x4{g[4], g[5], g[6], g[7]});
    *reinterpret_cast<bf16x8*>(ga.out + (size_t)row * kQDim + head * kD + d0) =
        bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return;
  }
  f32x4* dst = reinterpret_cast<f32x4*>(out + (size_t)row * kQDim + head * kD + d0);
  dst[0] = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
  dst[1] = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
}

// Split-K scratch: room for kSplitItems (tile, chunk, head) partials of 256
// rows.  The reference's provider ABI has no workspace argument, so the
// provider owns one scratch per device (allocated by qrt_ck_fmha_prepare,
// kept until the process ends: graphs captured with a split launch hold its
// address).  The first split launch on a device claims that scratch for its
// stream; split launches on that stream are ordered by it, and launches on
// any other stream run unsplit (same results, slower for short prompts), so
// concurrent streams never share partials.  qwen36_fmha_prefill takes a
// caller workspace instead and splits on any stream.
constexpr unsigned kSplitItems = 512;
constexpr size_t kSplitItemBytes = (size_t)256 * (kD + 2) * sizeof(float);
constexpr size_t kSplitScratchBytes = kSplitItems * kSplitItemBytes;
constexpr int kFmMaxDevices = 64;
std::mutex g_fm_mutex;
struct ProviderScratch {
  void* ptr = nullptr;
  bool claimed = false;
  hipStream_t owner = nullptr;
};
ProviderScratch g_fm_scratch[kFmMaxDevices];

// The provider scratch if `stream` may use it (claiming it on first use).
void* provider_scratch_for(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kFmMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_fm_mutex);
  ProviderScratch& ps = g_fm_scratch[dev];
  if (ps.ptr == nullptr) return nullptr;
  if (!ps.claimed) {
    ps.claimed = true;
    ps.owner = stream;
  }
  return ps.owner == stream ? ps.ptr : nullptr;
}

std::once_flag g_fm_attr_once;
hipError_t g_fm_attr_status = hipSuccess;

// Split plan for short prompts: too few 256-row tiles to fill the GPU, so
// each tile's key range is cut into n chunks (a multiple of 32 keys; a
// tile's chunks past its last key exit at once).  The chunk count was
// swept on MI355X (n = 2 .. 16 and unsplit, graph-replayed):
//  * square prompts (no cached prefix): the best n by 256-row tile count,
//    kSquareChunks below (T = 256: 23.9 us at n = 2 against 27.7 at 16;
//    T = 2304 / 2560: 85 / 97 us at n = 3 against 92 / 107 at 2);
//  * rows over a prefix: about 256 workgroups (n = 256 / (16 tiles));
//  * from 11 tiles on (T > 2560) the unsplit kernel is faster than any
//    split that fits the scratch (T = 3072 128 vs 137 us, T = 3840 165 vs
//    182; 3072 rows over a 4096 prefix 290 vs 327).
struct SplitPlan {
  unsigned n_chunks, chunk_keys, items;
};

constexpr unsigned kSplitMaxTiles = 10;
constexpr unsigned char kSquareChunks[kSplitMaxTiles + 1] = {0, 2, 8, 6, 4, 4, 3, 3, 2, 3, 3};

SplitPlan split_plan(unsigned q_tokens, unsigned kv_tokens) {
  const unsigned tiles = (q_tokens + 255) / 256;
  SplitPlan p{1u, kv_tokens, 0u};
  if (tiles > kSplitMaxTiles) return p;
  p.n_chunks = kv_tokens - q_tokens < 256u ? kSquareChunks[tiles]
                                           : (256u + tiles * kHq - 1) / (tiles * kHq);
  p.chunk_keys = (((kv_tokens + p.n_chunks - 1) / p.n_chunks) + kFmKv - 1) / kFmKv * kFmKv;
  p.n_chunks = (kv_tokens + p.chunk_keys - 1) / p.chunk_keys;   // after rounding up
  p.items = tiles * p.n_chunks * kHq;
  if (p.n_chunks < 2 || p.items > kSplitItems) p = SplitPlan{1u, kv_tokens, 0u};
  static_assert(256 / kHq <= kCombineMaxChunks, "the combine holds every chunk's (m, l)");
  return p;
}

size_t split_workspace_bytes(const SplitPlan& p) {
  return p.n_chunks > 1 ? (size_t)p.items * kSplitItemBytes : 0;
}

bool valid_geometry(const void* q, const void* k, const void* v, const float* out,
                    unsigned q_tokens, unsigned kv_tokens) {
  return q != nullptr && k != nullptr && v != nullptr && out != nullptr && q_tokens != 0u &&
         q_tokens <= kMaxTokens && kv_tokens >= q_tokens && kv_tokens <= kMaxTokens;
}

// `scratch` null: run unsplit.  `ga.out` non-null: gated bf16 output (and
// `out` unused).
int launch_fmha(const void* q, const void* k, const void* v, float* out,
                unsigned q_tokens, unsigned kv_tokens, void* scratch, hipStream_t stream,
                const GateArgs& ga = GateArgs{nullptr, 0u, nullptr}) {
  std::call_once(g_fm_attr_once, [] {
    for (const void* f : {reinterpret_cast<const void*>(fmha_prefill_kernel<8, false>),
                          reinterpret_cast<const void*>(fmha_prefill_kernel<4, false>),
                          reinterpret_cast<const void*>(fmha_prefill_kernel<2, false>),
                          reinterpret_cast<const void*>(fmha_prefill_kernel<8, true>)}) {
      const hipError_t e =
          hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kFmLds);
      if (e != hipSuccess) g_fm_attr_status = e;
    }
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(fmha_prefill_kernel<8, false, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, kFmLdsGated);
    if (e != hipSuccess) g_fm_attr_status = e;
  });
  if (g_fm_attr_status != hipSuccess) return (int)g_fm_attr_status;
  auto tiles = [&](unsigned rows) { return (q_tokens + rows - 1) / rows; };
  const bf16* qb = static_cast<const bf16*>(q);
  const bf16* kb = static_cast<const bf16*>(k);
  const bf16* vb = static_cast<const bf16*>(v);
  const SplitArgs none{nullptr, nullptr, 0u, 1u};
  const SplitPlan plan = split_plan(q_tokens, kv_tokens);
  if (plan.n_chunks > 1 && scratch != nullptr) {
    SplitArgs sp;
    sp.o = static_cast<float*>(scratch);
    sp.ml = sp.o + (size_t)plan.items * 256 * kD;   // (O partials, then (m, l) pairs)
    sp.chunk_keys = plan.chunk_keys;
    sp.n_chunks = plan.n_chunks;
    hipLaunchKernelGGL((fmha_prefill_kernel<8, true>), dim3(plan.items), dim3(512), kFmLds,
                       stream, qb, kb, vb, out, q_tokens, kv_tokens, tiles(256), sp, ga);
    auto combine = plan.n_chunks <= 4 ? fmha_split_combine_kernel<4>
                                      : fmha_split_combine_kernel<kCombineMaxChunks>;
    hipLaunchKernelGGL(combine, dim3(tiles(256) * kHq * 16), dim3(512), 0, stream, sp.o, sp.ml,
                       out, q_tokens, kv_tokens, plan.chunk_keys, plan.n_chunks, ga);
    return static_cast<int>(hipGetLastError());
  }
  if (ga.out != nullptr) {   // gated: 256-row workgroups at every length
    hipLaunchKernelGGL((fmha_prefill_kernel<8, false, true>), dim3(tiles(256) * kHq), dim3(512),
                       kFmLdsGated, stream, qb, kb, vb, out, q_tokens, kv_tokens, tiles(256), none, ga);
    return static_cast<int>(hipGetLastError());
  }
  // Query rows per workgroup: 256 (8 waves) when that gives at least 256
  // workgroups or the rows extend a cached prefix (long rows); short square
  // prompts use 128 or 64 rows so they still spread over the CUs (measured on
  // MI355X: T = 1024 51 vs 54 us, T = 2048 96 vs 97-102 us; 8 waves stay best
  // from T = 4096 and for 1024 rows over a 4096-token prefix).
  if (tiles(256) * kHq >= 256u || kv_tokens > q_tokens) {
    hipLaunchKernelGGL((fmha_prefill_kernel<8, false>), dim3(tiles(256) * kHq), dim3(512),
                       kFmLds, stream, qb, kb, vb, out, q_tokens, kv_tokens, tiles(256), none, ga);
  } else if (tiles(128) * kHq >= 256u) {
    hipLaunchKernelGGL((fmha_prefill_kernel<4, false>), dim3(tiles(128) * kHq), dim3(256),
                       kFmLds, stream, qb, kb, vb, out, q_tokens, kv_tokens, tiles(128), none, ga);
  } else {
    hipLaunchKernelGGL((fmha_prefill_kernel<2, false>), dim3(tiles(64) * kHq), dim3(128),
                       kFmLds, stream, qb, kb, vb, out, q_tokens, kv_tokens, tiles(64), none, ga);
  }
  return static_cast<int>(hipGetLastError());
}

int provider_launch(const void* q, const void* k, const void* v, float* out,
                    unsigned q_tokens, unsigned kv_tokens, hipStream_t stream) {
  if (!valid_geometry(q, k, v, out, q_tokens, kv_tokens)) return Q36_EINVAL;
  void* scratch = split_plan(q_tokens, kv_tokens).n_chunks > 1 ? provider_scratch_for(stream)
                                                                : nullptr;
  return launch_fmha(q, k, v, out, q_tokens, kv_tokens, scratch, stream);
}

}  // namespace
}  // namespace q36

// ---- provider ABI ---------------------------------------------------------
// prepare allocates the split-K scratch on the current device (once, 132 MiB);
// it stays allocated until the process ends -- a graph captured with a split
// launch holds its address -- so release has nothing to free.

// Returns 0 for a valid token count, hipErrorInvalidValue otherwise (the
// reference's contract); if the scratch cannot be allocated (no device, out
// of memory) the provider simply stays without it and launches run unsplit.
Q36_EXPORT int qrt_ck_fmha_prepare(unsigned tokens) {
  if (tokens == 0u || tokens > q36::kMaxTokens) return Q36_EINVAL;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= q36::kFmMaxDevices) {
    (void)hipGetLastError();
    return Q36_OK;
  }
  std::lock_guard<std::mutex> lock(q36::g_fm_mutex);
  q36::ProviderScratch& ps = q36::g_fm_scratch[dev];
  if (ps.ptr == nullptr && hipMalloc(&ps.ptr, q36::kSplitScratchBytes) != hipSuccess) {
    ps.ptr = nullptr;
    (void)hipGetLastError();
  }
  return Q36_OK;
}

Q36_EXPORT int qrt_ck_fmha_bf16_launch(const void* q, const void* k,
                                       const void* v, float* out,
                                       unsigned tokens, void* stream) {
  return q36::provider_launch(q, k, v, out, tokens, tokens,
                              static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qrt_ck_fmha_bf16_launch_ex(const void* q, const void* k,
                                          const void* v, float* out,
                                          unsigned query_tokens,
                                          unsigned kv_tokens, void* stream) {
  return q36::provider_launch(q, k, v, out, query_tokens, kv_tokens,
                              static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qrt_ck_fmha_release(void) { return Q36_OK; }

// Legacy fixed-shape q8192 exports (qrt_ck_fmha_q8192_provider.cpp:214-300).
// The fp32-packed launch takes rows of [q (4096) | 4096 more q_proj features
// | k (512) | v (512)] fp32 (9216 per token, the q_proj + k_proj + v_proj
// outputs side by side), rounds q, k and v to bf16 into provider staging
// (q8192_prepare allocates it, 80 MiB per device; q8192_release frees it),
// and runs the square causal attention over the staged tensors.
namespace q36 {
namespace {
constexpr unsigned kQ8192 = 8192u;
constexpr unsigned kPackedRow = 2u * kQDim + 2u * kKvRow;   // 9216

// thread = 8 consecutive features of one token's q, k or v
__global__ __launch_bounds__(256) void fmha_pack_q8192_kernel(const float* __restrict__ packed,
                                                             bf16* __restrict__ qs,
                                                             bf16* __restrict__ ks,
                                                             bf16* __restrict__ vs) {
  constexpr unsigned kPerTok = (kQDim + 2u * kKvRow) / 8u;   // 640 octets per token
  const unsigned idx = blockIdx.x * 256u + threadIdx.x;
  if (idx >= kQ8192 * kPerTok) return;
  const unsigned tok = idx / kPerTok, o = idx % kPerTok;
  const float* src;
  bf16* dst;
  if (o < kQDim / 8u) {
    src = packed + (size_t)tok * kPackedRow + 8u * o;
    dst = qs + (size_t)tok * kQDim + 8u * o;
  } else if (o < (kQDim + kKvRow) / 8u) {
    const unsigned f = 8u * o - kQDim;
    src = packed + (size_t)tok * kPackedRow + 2u * kQDim + f;
    dst = ks + (size_t)tok * kKvRow + f;
  } else {
    const unsigned f = 8u * o - kQDim - kKvRow;
    src = packed + (size_t)tok * kPackedRow + 2u * kQDim + kKvRow + f;
    dst = vs + (size_t)tok * kKvRow + f;
  }
  const f32x4 a = reinterpret_cast<const f32x4*>(src)[0];
  const f32x4 b = reinterpret_cast<const f32x4*>(src)[1];
  // round to nearest even (NaN stays NaN), as the provider's packing does
  *reinterpret_cast<bf16x8*>(dst) = bf16x8{f2bf(a[0]), f2bf(a[1]), f2bf(a[2]), f2bf(a[3]),
                                           f2bf(b[0]), f2bf(b[1]), f2bf(b[2]), f2bf(b[3])};
}

struct Q8192Staging {
  bf16* q = nullptr;
  bf16* k = nullptr;
  bf16* v = nullptr;
};
Q8192Staging g_q8192[kFmMaxDevices];

// Allocates the current device's staging if absent (caller holds g_fm_mutex).
int q8192_prepare_locked(int dev) {
  Q8192Staging& st = g_q8192[dev];
  if (st.q != nullptr) return Q36_OK;
  const size_t qb = (size_t)kQ8192 * kQDim * 2, kvb = (size_t)kQ8192 * kKvRow * 2;
  void *q = nullptr, *k = nullptr, *v = nullptr;
  hipError_t e = hipMalloc(&q, qb);
  if (e == hipSuccess) e = hipMalloc(&k, kvb);
  if (e == hipSuccess) e = hipMalloc(&v, kvb);
  if (e != hipSuccess) {
    (void)hipFree(q);
    (void)hipFree(k);
    (void)hipFree(v);
    return static_cast<int>(e);
  }
  st.q = static_cast<bf16*>(q);
  st.k = static_cast<bf16*>(k);
  st.v = static_cast<bf16*>(v);
  return Q36_OK;
}

int current_device(int* dev) {
  if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= kFmMaxDevices) {
    (void)hipGetLastError();
    return static_cast<int>(hipErrorInvalidDevice);
  }
  return Q36_OK;
}
}  // namespace
}  // namespace q36

Q36_EXPORT int qrt_ck_fmha_q8192_prepare(void) {
  int dev = 0;
  const int e = q36::current_device(&dev);
  if (e != Q36_OK) return e;
  std::lock_guard<std::mutex> lock(q36::g_fm_mutex);
  return q36::q8192_prepare_locked(dev);
}

Q36_EXPORT int qrt_ck_fmha_q8192_f32_launch(const float* packed_qkv, float* out, void* stream) {
  if (packed_qkv == nullptr || out == nullptr) return Q36_EINVAL;
  int dev = 0;
  int e = q36::current_device(&dev);
  if (e != Q36_OK) return e;
  q36::Q8192Staging st;
  {
    std::lock_guard<std::mutex> lock(q36::g_fm_mutex);
    e = q36::q8192_prepare_locked(dev);
    if (e != Q36_OK) return e;
    st = q36::g_q8192[dev];
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr unsigned kThreads = q36::kQ8192 * ((q36::kQDim + 2u * q36::kKvRow) / 8u);
  hipLaunchKernelGGL(q36::fmha_pack_q8192_kernel, dim3((kThreads + 255u) / 256u), dim3(256), 0,
                     s, packed_qkv, st.q, st.k, st.v);
  const hipError_t le = hipGetLastError();
  if (le != hipSuccess) return static_cast<int>(le);
  return q36::provider_launch(st.q, st.k, st.v, out, q36::kQ8192, q36::kQ8192, s);
}

Q36_EXPORT int qrt_ck_fmha_q8192_bf16_launch(const void* q, const void* k,
                                             const void* v, float* out,
                                             void* stream) {
  return q36::provider_launch(q, k, v, out, 8192u, 8192u,
                              static_cast<hipStream_t>(stream));
}

// Frees the fp32 path's staging (the caller has finished every launch that
// uses it, as with the reference's release).
Q36_EXPORT int qrt_ck_fmha_q8192_release(void) {
  int dev = 0;
  if (q36::current_device(&dev) != Q36_OK) return Q36_OK;
  std::lock_guard<std::mutex> lock(q36::g_fm_mutex);
  q36::Q8192Staging& st = q36::g_q8192[dev];
  (void)hipFree(st.q);
  (void)hipFree(st.k);
  (void)hipFree(st.v);
  st = q36::Q8192Staging{};
  return Q36_OK;
}

// ---- workspace form (no counterpart in the reference's provider ABI) -------
Q36_EXPORT size_t qwen36_fmha_prefill_workspace_bytes(unsigned query_tokens,
                                                      unsigned kv_tokens) {
  if (query_tokens == 0u || query_tokens > q36::kMaxTokens || kv_tokens < query_tokens ||
      kv_tokens > q36::kMaxTokens)
    return 0;
  return q36::split_workspace_bytes(q36::split_plan(query_tokens, kv_tokens));
}

Q36_EXPORT int qwen36_fmha_prefill(const void* q, const void* k, const void* v, float* out,
                                   unsigned query_tokens, unsigned kv_tokens, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (!q36::valid_geometry(q, k, v, out, query_tokens, kv_tokens)) return Q36_EINVAL;
  const size_t need = q36::split_workspace_bytes(q36::split_plan(query_tokens, kv_tokens));
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return Q36_EINVAL;
  return q36::launch_fmha(q, k, v, out, query_tokens, kv_tokens, need > 0 ? workspace : nullptr,
                          static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qwen36_fmha_prefill_gated(const void* q, const void* k, const void* v,
                                         const void* q_gate, unsigned q_gate_row_stride,
                                         void* out, unsigned query_tokens, unsigned kv_tokens,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  // (out stands in for the fp32 pointer in the geometry check)
  if (!q36::valid_geometry(q, k, v, static_cast<const float*>(out), query_tokens, kv_tokens) ||
      q_gate == nullptr || q_gate_row_stride < 2u * q36::kQDim ||
      (reinterpret_cast<uintptr_t>(q_gate) & 7u) != 0 || (q_gate_row_stride & 7u) != 0 ||
      (reinterpret_cast<uintptr_t>(out) & 15u) != 0)
    return Q36_EINVAL;
  const size_t need = q36::split_workspace_bytes(q36::split_plan(query_tokens, kv_tokens));
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return Q36_EINVAL;
  const q36::GateArgs ga{static_cast<const q36::bf16*>(q_gate), q_gate_row_stride,
                         static_cast<q36::bf16*>(out)};
  return q36::launch_fmha(q, k, v, nullptr, query_tokens, kv_tokens,
                          need > 0 ? workspace : nullptr, static_cast<hipStream_t>(stream), ga);
}
