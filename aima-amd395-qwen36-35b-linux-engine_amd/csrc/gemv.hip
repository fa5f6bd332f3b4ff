// BF16 GEMV for the one-token decode projections: y = W x.
//
// Replaces the reference decode's projection GEMVs -- the AOT
// triton_matvec_kernel / triton_fused_input_proj_conv_kernel and vLLM's
// bf16_wvsplitk skinny GEMM (native_full_layer.hip.cpp:154-174,
// native_linear_layer.hip.cpp:151-157; torch form `inp @ W.t()` in
// four_layer_mini_engine.py:6566-6573, :6386-6395 with one token).
// W is row-major [N, K] bf16 (the reference's [out_features, in_features]
// weights, e.g. the fused [q_proj | k_proj | v_proj] rows), x [K] bf16, y [N]
// bf16 = RNE(fp32 sum); accumulation in fp32.
//
// HBM-bound: 2 N K bytes of W per call.  A wave owns 2 rows at a time (4
// rows per wave measured 3-5% slower over the 80 decode GEMVs: the
// 2048-row output projections then fill only 128 workgroups) and
// streams them with 16-byte nontemporal loads (lane l reads columns
// 8l + 512j .. +8, so one load instruction covers 1 KiB of a row); x is
// loaded once per wave into registers in the matching column order.  Each row
// is reduced over the wave's 64 lanes by shuffles.  K is a template parameter
// (2048: every input projection; 4096: o_proj / out_proj).
#include "common.h"

namespace q36 {
namespace {

constexpr int kGvRows = 2;        // rows per wave in flight
constexpr int kGvWaves = 4;       // waves per workgroup

template <int K>
__global__ __launch_bounds__(64 * kGvWaves) void gemv_bf16_kernel(
    const bf16* __restrict__ w, const bf16* __restrict__ x, bf16* __restrict__ y,
    unsigned n_rows) {
  constexpr int kSteps = K / 512;   // 1 KiB load instructions per row
  const int lane = threadIdx.x & 63;
  const unsigned wave_g = blockIdx.x * kGvWaves + (threadIdx.x >> 6);
  const unsigned waves = gridDim.x * kGvWaves;
  float xv[kSteps][8];
#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(x + 512 * j + 8 * lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[j][e] = bf2f(v[e]);
  }
  for (unsigned r0 = wave_g * kGvRows; r0 < n_rows; r0 += waves * kGvRows) {
    u32x4 wr[kGvRows][kSteps];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r) {
      const unsigned row = min(r0 + r, n_rows - 1);   // clamped: loads stay in bounds
      const bf16* wp = w + (size_t)row * K + 8 * lane;
#pragma unroll
      for (int j = 0; j < kSteps; ++j)
        wr[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp + 512 * j));
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every weight load in flight before the FMAs
    float acc[kGvRows];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        const bf16x8 v = __builtin_bit_cast(bf16x8, wr[r][j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) a = __builtin_fmaf(bf2f(v[e]), xv[j][e], a);
      }
      acc[r] = a;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int r = 0; r < kGvRows; ++r) acc[r] += __shfl_xor(acc[r], o, 64);
    if (lane < kGvRows && r0 + lane < n_rows) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < kGvRows; ++r) v = lane == r ? acc[r] : v;
      y[r0 + lane] = f2bf(v);
    }
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

// y[N] = W[N,K] x[K] (bf16 in and out, fp32 accumulation).  K must be 2048 or
// 4096; W, x 16-byte aligned; y 2-byte aligned.
Q36_EXPORT int qwen36_gemv_bf16(const void* w, unsigned n_rows, unsigned k,
                                const void* x, void* y, void* stream) {
  if (w == nullptr || x == nullptr || y == nullptr || n_rows == 0 || n_rows > (1u << 24) ||
      (k != 2048u && k != 4096u) || (reinterpret_cast<uintptr_t>(w) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(x) % 16) != 0)
    return Q36_EINVAL;
  const unsigned groups = (n_rows + kGvRows - 1) / kGvRows;          // row groups
  unsigned blocks = (groups + kGvWaves - 1) / kGvWaves;
  if (blocks > 2048u) blocks = 2048u;                                  // grid-stride beyond
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (k == 2048u)
    hipLaunchKernelGGL(gemv_bf16_kernel<2048>, dim3(blocks), dim3(64 * kGvWaves), 0, st,
                       static_cast<const bf16*>(w), static_cast<const bf16*>(x),
                       static_cast<bf16*>(y), n_rows);
  else
    hipLaunchKernelGGL(gemv_bf16_kernel<4096>, dim3(blocks), dim3(64 * kGvWaves), 0, st,
                       static_cast<const bf16*>(w), static_cast<const bf16*>(x),
                       static_cast<bf16*>(y), n_rows);
  return static_cast<int>(hipGetLastError());
}
