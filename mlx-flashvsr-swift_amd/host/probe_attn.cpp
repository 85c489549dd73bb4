// fvsr_probe_attn — the reference's attention probe (`probeAttention`, Sources/Smoke/Diag.swift:86-145) on MI355X,
// through the C++ host layer:
//   1. kernel vs dense on random q/k/v and a random block mask with a forced empty query block, fp32 and bf16
//      (Diag.swift:87-98);
//   2. bf16 dense and bf16 kernel against the fp32 dense result on the same bf16-representable inputs (:100-110);
//   3. timing of dense and kernel on the real chunk shapes, 12 heads, bf16, random masks at the stated densities
//      (:122-144): 1280x768 chunk 0 (180 x 180 blocks, 67 %), later chunks (60 x 240, 50 %), 1920x1152 later chunks
//      (135 x 540, 22 %). The reference reports min of 3; this prints min and median of `--reps` (default 10).
// rel = max|got - ref| / max|ref| (Sources/Smoke/Gates.swift:19-29).
//
//   fvsr_probe_attn [--quick] [--reps N]
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "FlashVSRLCSA.hpp"

#define HIPCHECK(x)                                                                            \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) {                                                                    \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(1);                                                                            \
    }                                                                                          \
  } while (0)

// counter-based normal / uniform generator (splitmix64 + Box-Muller), deterministic per (seed, index)
__device__ inline uint64_t mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
__device__ inline float u01(uint64_t x) { return ((mix64(x) >> 40) + 0.5f) * (1.0f / 16777216.0f); }

__global__ void fill_normal(float* f32, __hip_bfloat16* bf, int64_t n, uint64_t seed) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float u1 = u01(seed * 0x100000001B3ull + 2 * i), u2 = u01(seed * 0x100000001B3ull + 2 * i + 1);
    float z = sqrtf(-2.f * logf(u1)) * cosf(6.2831853f * u2);
    if (bf) {
      bf[i] = __float2bfloat16(z);
      z = __bfloat162float(bf[i]);   // the fp32 copy holds the same (bf16-representable) values
    }
    if (f32) f32[i] = z;
  }
}

__global__ void fill_mask(float* m, int64_t n, float density, uint64_t seed) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    m[i] = u01(seed * 0x9E3779B97F4A7C15ull + i) < density ? 1.f : 0.f;
}

struct Buf {
  void* p = nullptr;
  size_t bytes = 0;
  explicit Buf(size_t b) : bytes(b) { HIPCHECK(hipMalloc(&p, b)); }
  ~Buf() { (void)hipFree(p); }
};

static std::vector<float> to_host(const Buf& b, bool is_bf16, size_t n) {
  std::vector<float> out(n);
  if (is_bf16) {
    std::vector<uint16_t> raw(n);
    HIPCHECK(hipMemcpy(raw.data(), b.p, n * 2, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < n; ++i) {
      uint32_t w = (uint32_t)raw[i] << 16;
      std::memcpy(&out[i], &w, 4);
    }
  } else {
    HIPCHECK(hipMemcpy(out.data(), b.p, n * 4, hipMemcpyDeviceToHost));
  }
  return out;
}

static double rel(const std::vector<float>& got, const std::vector<float>& ref) {
  double d = 0, r = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    d = std::max(d, (double)std::fabs(got[i] - ref[i]));
    r = std::max(r, (double)std::fabs(ref[i]));
  }
  return d / std::max(r, 1e-12);
}

struct Case {
  int heads, lqb, lkb;
  bool bf16;
  // device data
  Buf q32, k32, v32, q16, k16, v16, mask;
  Case(int h, int lqb_, int lkb_, bool bf)
      : heads(h), lqb(lqb_), lkb(lkb_), bf16(bf),
        q32((size_t)lqb_ * 128 * h * 128 * 4), k32((size_t)lkb_ * 128 * h * 128 * 4),
        v32((size_t)lkb_ * 128 * h * 128 * 4), q16((size_t)lqb_ * 128 * h * 128 * 2),
        k16((size_t)lkb_ * 128 * h * 128 * 2), v16((size_t)lkb_ * 128 * h * 128 * 2),
        mask((size_t)h * lqb_ * lkb_ * 4) {}
  int64_t lq() const { return (int64_t)lqb * 128; }
  int64_t lk() const { return (int64_t)lkb * 128; }
  size_t qn() const { return (size_t)lq() * heads * 128; }
  void fill(uint64_t seed, float density) {
    hipLaunchKernelGGL(fill_normal, dim3(1024), dim3(256), 0, 0, (float*)q32.p, (__hip_bfloat16*)q16.p,
                       (int64_t)qn(), seed * 3 + 0);
    hipLaunchKernelGGL(fill_normal, dim3(1024), dim3(256), 0, 0, (float*)k32.p, (__hip_bfloat16*)k16.p,
                       lk() * heads * 128, seed * 3 + 1);
    hipLaunchKernelGGL(fill_normal, dim3(1024), dim3(256), 0, 0, (float*)v32.p, (__hip_bfloat16*)v16.p,
                       lk() * heads * 128, seed * 3 + 2);
    hipLaunchKernelGGL(fill_mask, dim3(256), dim3(256), 0, 0, (float*)mask.p, (int64_t)heads * lqb * lkb,
                       density, seed);
    HIPCHECK(hipGetLastError());
  }
  flashvsr::Tokens tq(bool b) const { return {b ? q16.p : q32.p, lq(), b ? FVSR_DTYPE_BF16 : FVSR_DTYPE_F32}; }
  flashvsr::Tokens tk(bool b) const { return {b ? k16.p : k32.p, lk(), b ? FVSR_DTYPE_BF16 : FVSR_DTYPE_F32}; }
  flashvsr::Tokens tv(bool b) const { return {b ? v16.p : v32.p, lk(), b ? FVSR_DTYPE_BF16 : FVSR_DTYPE_F32}; }
};

int main(int argc, char** argv) {
  bool quick = false;
  int reps = 10;
  for (int i = 1; i < argc; ++i) {
    if (!std::strcmp(argv[i], "--quick")) quick = true;
    else if (!std::strcmp(argv[i], "--reps") && i + 1 < argc) reps = std::max(1, std::atoi(argv[++i]));
  }
  flashvsr::LCSA lcsa(0);
  int worst_fail = 0;

  // 1. kernel vs dense (Diag.swift:87-98)
  struct Acc { bool bf; int lqb, lkb; float density; };
  for (const Acc& c : {Acc{false, 4, 6, 0.5f}, Acc{false, 12, 36, 0.3f}, Acc{true, 12, 36, 0.6f}}) {
    Case cs(2, c.lqb, c.lkb, c.bf);
    cs.fill(c.lqb * 1000 + c.lkb, c.density);
    HIPCHECK(hipMemset((char*)cs.mask.p + (size_t)1 * c.lkb * 4, 0, (size_t)c.lkb * 4));   // m[0, 1] = 0
    Buf o1(cs.qn() * (c.bf ? 2 : 4)), o2(cs.qn() * (c.bf ? 2 : 4));
    lcsa.dense(cs.tq(c.bf), cs.tk(c.bf), cs.tv(c.bf), (const float*)cs.mask.p, 2, o1.p);
    lcsa.kernel(cs.tq(c.bf), cs.tk(c.bf), cs.tv(c.bf), (const float*)cs.mask.p, 2, o2.p);
    HIPCHECK(hipDeviceSynchronize());
    const double r = rel(to_host(o2, c.bf, cs.qn()), to_host(o1, c.bf, cs.qn()));
    std::printf("  kernel %s %dx%d d%.1f  rel %.3e%s\n", c.bf ? "bf16" : "fp32", c.lqb, c.lkb, c.density, r,
                r > 1e-6 ? "   FAIL (> 1e-6)" : "");
    if (r > 1e-6) worst_fail = 1;
  }

  // 2. bf16 paths vs the fp32 dense result (Diag.swift:100-110)
  {
    Case cs(2, 12, 36, true);
    cs.fill(77, 0.5f);
    Buf ref(cs.qn() * 4), od(cs.qn() * 2), ok(cs.qn() * 2);
    lcsa.dense(cs.tq(false), cs.tk(false), cs.tv(false), (const float*)cs.mask.p, 2, ref.p);
    lcsa.dense(cs.tq(true), cs.tk(true), cs.tv(true), (const float*)cs.mask.p, 2, od.p);
    lcsa.kernel(cs.tq(true), cs.tk(true), cs.tv(true), (const float*)cs.mask.p, 2, ok.p);
    HIPCHECK(hipDeviceSynchronize());
    const auto r32 = to_host(ref, false, cs.qn());
    const double rd = rel(to_host(od, true, cs.qn()), r32), rk = rel(to_host(ok, true, cs.qn()), r32);
    std::printf("  bf16 dense  vs fp32  rel %.3e\n  bf16 kernel vs fp32  rel %.3e%s\n", rd, rk,
                rk > 1e-2 ? "   FAIL (> 1e-2)" : "");
    if (rk > 1e-2) worst_fail = 1;
  }
  if (quick) return worst_fail;

  // 3. timing on the real chunk shapes (Diag.swift:122-144)
  struct Shape { const char* label; int lqb, lkb; float density; };
  for (const Shape& sh : {Shape{"720p c0", 180, 180, 0.67f}, Shape{"720p c1+", 60, 240, 0.5f},
                          Shape{"1152p c1+", 135, 540, 0.22f}}) {
    Case cs(12, sh.lqb, sh.lkb, true);
    cs.fill(sh.lqb + sh.lkb, sh.density);
    lcsa.reserve(12, cs.lq(), cs.lk());
    Buf o(cs.qn() * 2);
    hipEvent_t e0, e1;
    HIPCHECK(hipEventCreate(&e0));
    HIPCHECK(hipEventCreate(&e1));
    for (int arm = 0; arm < 2; ++arm) {
      auto run = [&] {
        if (arm == 0) lcsa.dense(cs.tq(true), cs.tk(true), cs.tv(true), (const float*)cs.mask.p, 12, o.p);
        else lcsa.kernel(cs.tq(true), cs.tk(true), cs.tv(true), (const float*)cs.mask.p, 12, o.p);
      };
      run();
      HIPCHECK(hipDeviceSynchronize());
      std::vector<float> ts;
      for (int r = 0; r < reps; ++r) {
        HIPCHECK(hipEventRecord(e0));
        run();
        HIPCHECK(hipEventRecord(e1));
        HIPCHECK(hipEventSynchronize(e1));
        float ms = 0;
        HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
        ts.push_back(ms);
      }
      std::sort(ts.begin(), ts.end());
      const double kept = [&] {
        std::vector<float> m((size_t)12 * sh.lqb * sh.lkb);
        HIPCHECK(hipMemcpy(m.data(), cs.mask.p, m.size() * 4, hipMemcpyDeviceToHost));
        double s = 0;
        for (float x : m) s += x > 0.5f;
        return s;
      }();
      const double tflop = kept * 4.0 * 128 * 128 * 128 / 1e12;
      std::printf("  %-10s %-8s density %.2f: %8.3f ms (min of %d), median %.3f ms, %.1f TFLOP/s on kept blocks\n",
                  sh.label, arm == 0 ? "dense" : "kernel", sh.density, ts.front(), reps, ts[ts.size() / 2],
                  tflop / (ts.front() * 1e-3));
      std::fflush(stdout);
    }
    HIPCHECK(hipEventDestroy(e0));
    HIPCHECK(hipEventDestroy(e1));
  }
  return worst_fail;
}
