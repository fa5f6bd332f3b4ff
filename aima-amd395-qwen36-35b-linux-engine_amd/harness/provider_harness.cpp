// Caller-side harness for the FMHA provider C ABI, written the way the
// reference engine consumes its provider: NativeQ8192CkProvider::load /
// launch (benchmarks/shape-lab/native/src/native_full_prefill.hip.cpp:140-266)
// dlopen()s the provider library, resolves qrt_ck_fmha_prepare /
// _bf16_launch / _bf16_launch_ex / _release with dlsym(), treats a non-zero
// return as a hip error code, and launches on its own stream with
// caller-owned device buffers (Q [T,16,256] bf16, K/V [S,2,256] bf16,
// out fp32 [T,4096]).
//
// usage: provider_harness <path to libqwen36_attn.so>
// Exit status: 0 = all checks passed, 1 = a check failed, 2 = the library or
// a symbol could not be loaded, 3 = a HIP runtime call failed.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

using PrepareFn = int (*)(unsigned);
using LaunchFn = int (*)(const void*, const void*, const void*, float*, unsigned, void*);
using LaunchExFn = int (*)(const void*, const void*, const void*, float*, unsigned, unsigned, void*);
using ReleaseFn = int (*)();

constexpr int kHeads = 16, kKvHeads = 2, kDim = 256;

// bf16 storage (round to nearest even) and back.
uint16_t to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
float from_bf16(uint16_t h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

// Deterministic inputs in [-2, 2).
std::vector<uint16_t> make_input(size_t n, uint64_t seed) {
  std::vector<uint16_t> v(n);
  uint64_t s = seed * 6364136223846793005ull + 1442695040888963407ull;
  for (size_t i = 0; i < n; ++i) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    const double u = static_cast<double>(s >> 11) / 9007199254740992.0;
    v[i] = to_bf16(static_cast<float>(4.0 * u - 2.0));
  }
  return v;
}

// softmax(Q K^T / 16 + mask) V in double: query i of T sees keys
// j <= i + (S - T) (top-left causal when S == T, bottom-right when S > T);
// query head h reads KV head h / 8.
std::vector<double> reference(const std::vector<uint16_t>& q, const std::vector<uint16_t>& k,
                              const std::vector<uint16_t>& v, unsigned T, unsigned S) {
  std::vector<double> out(static_cast<size_t>(T) * kHeads * kDim, 0.0);
  std::vector<double> p(S);
  for (unsigned i = 0; i < T; ++i) {
    const unsigned last = i + (S - T);
    for (int h = 0; h < kHeads; ++h) {
      const int kvh = h / 8;
      double mx = -INFINITY;
      for (unsigned j = 0; j <= last; ++j) {
        double dot = 0.0;
        for (int d = 0; d < kDim; ++d)
          dot += static_cast<double>(from_bf16(q[(static_cast<size_t>(i) * kHeads + h) * kDim + d])) *
                 from_bf16(k[(static_cast<size_t>(j) * kKvHeads + kvh) * kDim + d]);
        p[j] = dot / 16.0;
        mx = std::max(mx, p[j]);
      }
      double sum = 0.0;
      for (unsigned j = 0; j <= last; ++j) {
        p[j] = std::exp(p[j] - mx);
        sum += p[j];
      }
      double* o = &out[(static_cast<size_t>(i) * kHeads + h) * kDim];
      for (unsigned j = 0; j <= last; ++j)
        for (int d = 0; d < kDim; ++d)
          o[d] += p[j] / sum * from_bf16(v[(static_cast<size_t>(j) * kKvHeads + kvh) * kDim + d]);
    }
  }
  return out;
}

bool hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) std::fprintf(stderr, "HIP error %d in %s\n", static_cast<int>(e), what);
  return e == hipSuccess;
}

// One launch through the provider and a comparison with the reference.
// Returns 0 pass, 1 fail, 3 HIP error.
int run_case(LaunchFn launch, LaunchExFn launch_ex, unsigned T, unsigned S, hipStream_t st) {
  const auto q = make_input(static_cast<size_t>(T) * kHeads * kDim, 11 + T);
  const auto k = make_input(static_cast<size_t>(S) * kKvHeads * kDim, 23 + S);
  const auto v = make_input(static_cast<size_t>(S) * kKvHeads * kDim, 37 + S);
  void *dq = nullptr, *dk = nullptr, *dv = nullptr;
  float* dout = nullptr;
  const size_t out_n = static_cast<size_t>(T) * kHeads * kDim;
  if (!hip_ok(hipMalloc(&dq, q.size() * 2), "hipMalloc q") ||
      !hip_ok(hipMalloc(&dk, k.size() * 2), "hipMalloc k") ||
      !hip_ok(hipMalloc(&dv, v.size() * 2), "hipMalloc v") ||
      !hip_ok(hipMalloc(reinterpret_cast<void**>(&dout), out_n * 4), "hipMalloc out"))
    return 3;
  if (!hip_ok(hipMemcpy(dq, q.data(), q.size() * 2, hipMemcpyHostToDevice), "copy q") ||
      !hip_ok(hipMemcpy(dk, k.data(), k.size() * 2, hipMemcpyHostToDevice), "copy k") ||
      !hip_ok(hipMemcpy(dv, v.data(), v.size() * 2, hipMemcpyHostToDevice), "copy v"))
    return 3;
  const int status = (S == T) ? launch(dq, dk, dv, dout, T, st)
                              : launch_ex(dq, dk, dv, dout, T, S, st);
  if (status != 0) {
    std::printf("FAIL launch T=%u S=%u returned %d\n", T, S, status);
    return 1;
  }
  std::vector<float> got(out_n);
  if (!hip_ok(hipStreamSynchronize(st), "sync") ||
      !hip_ok(hipMemcpy(got.data(), dout, out_n * 4, hipMemcpyDeviceToHost), "copy out"))
    return 3;
  (void)hipFree(dq);
  (void)hipFree(dk);
  (void)hipFree(dv);
  (void)hipFree(dout);
  const auto ref = reference(q, k, v, T, S);
  double err = 0.0;
  for (size_t i = 0; i < out_n; ++i) {
    if (!std::isfinite(got[i])) {
      err = INFINITY;
      break;
    }
    err = std::max(err, std::fabs(got[i] - ref[i]));
  }
  const bool ok = err <= 2e-2;
  std::printf("%s T=%u S=%u max-abs-err %.3e (bar 2e-2)\n", ok ? "ok" : "FAIL", T, S, err);
  return ok ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s <provider library>\n", argv[0]);
    return 2;
  }
  void* handle = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (handle == nullptr) {
    std::printf("FAIL dlopen: %s\n", dlerror());
    return 2;
  }
  auto prepare = reinterpret_cast<PrepareFn>(dlsym(handle, "qrt_ck_fmha_prepare"));
  auto launch = reinterpret_cast<LaunchFn>(dlsym(handle, "qrt_ck_fmha_bf16_launch"));
  auto launch_ex = reinterpret_cast<LaunchExFn>(dlsym(handle, "qrt_ck_fmha_bf16_launch_ex"));
  auto release = reinterpret_cast<ReleaseFn>(dlsym(handle, "qrt_ck_fmha_release"));
  if (!prepare || !launch || !launch_ex || !release) {
    std::printf("FAIL missing provider symbol\n");
    return 2;
  }
  int fails = 0;
  // Argument validation, as the engine relies on it (hipErrorInvalidValue = 1).
  if (prepare(0) != 1 || prepare(262145) != 1 || prepare(8192) != 0) {
    std::printf("FAIL prepare limits\n");
    ++fails;
  }
  if (launch_ex(nullptr, nullptr, nullptr, nullptr, 16, 8, nullptr) != 1 ||
      launch(nullptr, nullptr, nullptr, nullptr, 0, nullptr) != 1) {
    std::printf("FAIL launch argument checks\n");
    ++fails;
  }
  hipStream_t st;
  if (!hip_ok(hipStreamCreate(&st), "hipStreamCreate")) return 3;
  // square causal (top-left mask) and prefix extension (bottom-right mask),
  // both with ragged tile tails
  const unsigned cases[3][2] = {{77, 77}, {64, 150}, {130, 130}};
  for (const auto& c : cases) {
    const int r = run_case(launch, launch_ex, c[0], c[1], st);
    if (r == 3) return 3;
    fails += r;
  }
  (void)hipStreamDestroy(st);
  if (release() != 0) {
    std::printf("FAIL release\n");
    ++fails;
  }
  dlclose(handle);
  std::printf(fails == 0 ? "PASS\n" : "FAIL (%d)\n", fails);
  return fails == 0 ? 0 : 1;
}
