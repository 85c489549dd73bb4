// The dense parts of one FlashVSR DiT block around the LCSA layer call, for gfx950 (MI355X): the projections and the
// FFN on hipBLASLt (bf16 in, fp32 accumulate, bias / GELU fused into the GEMM epilogue), the norms, modulation and
// residual updates as one-pass wave-per-token kernels, and the cross-attention over the cached context K/V on the
// block-sparse attention kernel with every context block listed.
//
// Reference semantics (blockForward, DiT.swift:491-551; modules DiT.swift:317-381):
//   mod = modulation + t_mod (6 x C); shift/scale/gate for the self-attention (0..2) and the FFN (3..5)  :495-497
//   inX = norm1(x) * (1 + scaleMSA) + shiftMSA          norm1 = LayerNorm(affine: false)               :498
//   q/k/v = Linear(inX) -> LCSA layer call -> o = Linear(attn in natural order)                          :500-539
//   x = x + gateMSA * o                                                                                  :541
//   caIn = norm3(x) (LayerNorm, affine); x = x + Linear_o(SDPA(normQ(Linear_q(caIn)), cacheK, cacheV))  :542-545
//   inF = norm2(x) * (1 + scaleMLP) + shiftMLP; x = x + gateMLP * Linear2(GELU_tanh(Linear1(inF)))      :546-548
// Every elementwise step rounds to the storage type (bf16) as MLX does between ops; norms reduce in fp32.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "common.hpp"

namespace fvsr {

// ------------------------------------------------------------------------------------------------------------
// hipBLASLt: Y (L, N) = X (L, K) W^T + b, W (N, K) row-major (PyTorch Linear layout), all bf16, fp32 accumulate.
// Column-major view: Y^T (N x L) = W (N x K, i.e. col-major K x N transposed) * X^T (col-major K x L).
// ------------------------------------------------------------------------------------------------------------
struct BlasState {
  int device = 0;
  hipblasLtHandle_t handle = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  std::map<std::tuple<int, int64_t, int, int>, hipblasLtMatmulAlgo_t> algos;   // (N, L, K, epilogue) -> algo
};

constexpr size_t kBlasWorkspace = 64u << 20;

#define FVSR_BLAS_CHECK(expr)                                                                          \
  do {                                                                                                 \
    hipblasStatus_t s_ = (expr);                                                                       \
    if (s_ != HIPBLAS_STATUS_SUCCESS)                                                                  \
      return ::fvsr::set_error(FVSR_ERR_HIP, std::string(#expr) + ": hipBLASLt status " + std::to_string((int)s_)); \
  } while (0)

int blas_create(int device, void** out) {
  auto* b = new BlasState;
  b->device = device;
  FVSR_HIP_CHECK(hipSetDevice(device));
  if (hipblasLtCreate(&b->handle) != HIPBLAS_STATUS_SUCCESS) {
    delete b;
    return set_error(FVSR_ERR_HIP, "hipblasLtCreate failed");
  }
  if (hipMalloc(&b->ws, kBlasWorkspace) != hipSuccess) {
    hipblasLtDestroy(b->handle);
    delete b;
    return set_error(FVSR_ERR_OUT_OF_MEMORY, "GEMM workspace allocation failed");
  }
  b->ws_bytes = kBlasWorkspace;
  *out = b;
  return FVSR_OK;
}

void blas_destroy(void* p) {
  auto* b = (BlasState*)p;
  if (!b) return;
  (void)hipSetDevice(b->device);
  if (b->ws) (void)hipFree(b->ws);
  if (b->handle) hipblasLtDestroy(b->handle);
  delete b;
}

// epilogue: 0 = bias (if given), 1 = bias + GELU (tanh form)
int linear_bf16(void* state, const void* x, int64_t L, int K, const void* w, int N, const void* bias, int epilogue,
                void* y, hipStream_t stream) {
  auto* b = (BlasState*)state;
  if (L <= 0) return FVSR_OK;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  int rc = FVSR_OK;
  auto fail = [&](const std::string& m) {
    rc = set_error(FVSR_ERR_HIP, m);
  };
  do {
    if (hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) {
      fail("hipblasLtMatmulDescCreate failed");
      break;
    }
    // every attribute must take: a dropped epilogue or bias would compute a different function without an error
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_DEFAULT;
    if (epilogue == 1) ep = bias ? HIPBLASLT_EPILOGUE_GELU_BIAS : HIPBLASLT_EPILOGUE_GELU;
    else if (bias) ep = HIPBLASLT_EPILOGUE_BIAS;
    const hipDataType bt = HIP_R_16BF;
    bool ok = hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)) ==
                  HIPBLAS_STATUS_SUCCESS;
    if (ok && bias)
      ok = hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) ==
               HIPBLAS_STATUS_SUCCESS;
    if (!ok) {
      fail("hipblasLtMatmulDescSetAttribute failed (transpose, epilogue or bias)");
      break;
    }
    if (hipblasLtMatrixLayoutCreate(&la, HIP_R_16BF, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&lb, HIP_R_16BF, K, L, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&lc, HIP_R_16BF, N, L, N) != HIPBLAS_STATUS_SUCCESS) {
      fail("hipblasLtMatrixLayoutCreate failed");
      break;
    }
    const auto key = std::make_tuple(N, L, K, (bias ? 2 : 0) + epilogue);
    auto it = b->algos.find(key);
    if (it == b->algos.end()) {
      hipblasLtMatmulPreference_t pref = nullptr;
      if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) {
        fail("hipblasLtMatmulPreferenceCreate failed");
        break;
      }
      uint64_t wsb = b->ws_bytes;
      hipblasLtMatmulHeuristicResult_t heur[1];
      int n = 0;
      hipblasStatus_t hs =
          hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
      if (hs == HIPBLAS_STATUS_SUCCESS)
        hs = hipblasLtMatmulAlgoGetHeuristic(b->handle, desc, la, lb, lc, lc, pref, 1, heur, &n);
      hipblasLtMatmulPreferenceDestroy(pref);
      if (hs != HIPBLAS_STATUS_SUCCESS || n < 1) {
        rc = set_error(FVSR_ERR_UNSUPPORTED, "hipBLASLt has no algorithm for a " + std::to_string(L) + " x " +
                                                 std::to_string(N) + " x " + std::to_string(K) + " bf16 GEMM");
        break;
      }
      it = b->algos.emplace(key, heur[0].algo).first;
    }
    const float alpha = 1.f, beta = 0.f;
    if (hipblasLtMatmul(b->handle, desc, &alpha, w, la, x, lb, &beta, y, lc, y, lc, &it->second, b->ws, b->ws_bytes,
                        stream) != HIPBLAS_STATUS_SUCCESS)
      fail("hipblasLtMatmul failed");
  } while (false);
  if (la) hipblasLtMatrixLayoutDestroy(la);
  if (lb) hipblasLtMatrixLayoutDestroy(lb);
  if (lc) hipblasLtMatrixLayoutDestroy(lc);
  if (desc) hipblasLtMatmulDescDestroy(desc);
  return rc;
}

// ------------------------------------------------------------------------------------------------------------
// elementwise / norm kernels (one wave per token, C = 64 lanes x nv 16-byte vectors of 8 bf16)
// ------------------------------------------------------------------------------------------------------------
typedef unsigned u4 __attribute__((ext_vector_type(4)));
constexpr int kMaxVecs = 6;   // C <= 64 * 6 * 8 = 3072 channels

__device__ __forceinline__ float rb(float x) { return (float)(bf16)x; }

// mod[r * C + c] = bf16(modulation[r * C + c] + t_mod[r * C + c]), 6 rows (DiT.swift:495)
__global__ void modulation_kernel(const bf16* __restrict__ m, const bf16* __restrict__ t, bf16* __restrict__ out,
                                  int n) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n) out[e] = (bf16)((float)m[e] + (float)t[e]);
}

// Per token (row of x, C channels), in this order:
//   1. residual (y != null): x = bf16(x + bf16(gate * y)) (gate null: x = bf16(x + y)), written back to x
//   2. norm (out != null): LayerNorm over C in fp32 (two-pass mean / variance, eps), then
//        affine (w, b): out = bf16(n * w + b)       (MLX's fused layer norm applies the affine in fp32)
//        modulation (scale, shift): out = bf16(bf16(bf16(n) * bf16(1 + scale)) + shift)
//        neither: out = bf16(n)
// The same pass serves x + gate * attn -> norm3, x + ca -> norm2 + modulation, and the final x + gate * ffn.
__global__ __launch_bounds__(256) void residual_norm_kernel(bf16* __restrict__ x, const bf16* __restrict__ y,
                                                            const bf16* __restrict__ gate, int64_t L, int C,
                                                            float eps, const bf16* __restrict__ w,
                                                            const bf16* __restrict__ bias,
                                                            const bf16* __restrict__ scale,
                                                            const bf16* __restrict__ shift, bf16* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= L) return;
  const int nvec = C / 8;
  u4 xv[kMaxVecs];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVecs; ++j) {
    const int cv = lane + 64 * j;
    if (cv >= nvec) continue;
    u4 v = *(const u4*)(x + n * C + cv * 8);
    if (y) {
      const u4 yv = *(const u4*)(y + n * C + cv * 8);
      u4 gv = u4{0, 0, 0, 0};
      if (gate) gv = *(const u4*)(gate + cv * 8);
      bf16* a = (bf16*)&v;
      const bf16* yy = (const bf16*)&yv;
      const bf16* gg = (const bf16*)&gv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float add = gate ? rb((float)gg[e] * (float)yy[e]) : (float)yy[e];
        a[e] = (bf16)((float)a[e] + add);
      }
      *(u4*)(x + n * C + cv * 8) = v;
    }
    xv[j] = v;
    const bf16* a = (const bf16*)&v;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += (float)a[e];
  }
  if (!out) return;
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  const float mean = sum / (float)C;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVecs; ++j) {
    const int cv = lane + 64 * j;
    if (cv >= nvec) continue;
    const bf16* a = (const bf16*)&xv[j];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = (float)a[e] - mean;
      sq = fmaf(d, d, sq);
    }
  }
  for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o);
  const float inv = 1.f / sqrtf(sq / (float)C + eps);
#pragma unroll
  for (int j = 0; j < kMaxVecs; ++j) {
    const int cv = lane + 64 * j;
    if (cv >= nvec) continue;
    const bf16* a = (const bf16*)&xv[j];
    u4 ov;
    bf16* o = (bf16*)&ov;
    if (w) {
      const u4 wv = *(const u4*)(w + cv * 8);
      u4 bv = u4{0, 0, 0, 0};
      if (bias) bv = *(const u4*)(bias + cv * 8);
      const bf16* ww = (const bf16*)&wv;
      const bf16* bb = (const bf16*)&bv;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)(((float)a[e] - mean) * inv * (float)ww[e] + (float)bb[e]);
    } else if (scale) {
      const u4 sv = *(const u4*)(scale + cv * 8), hv = *(const u4*)(shift + cv * 8);
      const bf16* ss = (const bf16*)&sv;
      const bf16* hh = (const bf16*)&hv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float nn = rb(((float)a[e] - mean) * inv);
        o[e] = (bf16)(rb(nn * rb(1.f + (float)ss[e])) + (float)hh[e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)(((float)a[e] - mean) * inv);
    }
    *(u4*)(out + n * C + cv * 8) = ov;
  }
}

// WanRMSNorm over the full width (DiT.swift:34-47), natural order: out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)
__global__ __launch_bounds__(256) void rms_norm_kernel(const bf16* __restrict__ x, int64_t L, int C, float eps,
                                                       const bf16* __restrict__ w, bf16* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= L) return;
  const int nvec = C / 8;
  u4 xv[kMaxVecs];
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVecs; ++j) {
    const int cv = lane + 64 * j;
    if (cv >= nvec) continue;
    xv[j] = *(const u4*)(x + n * C + cv * 8);
    const bf16* a = (const bf16*)&xv[j];
#pragma unroll
    for (int e = 0; e < 8; ++e) sq = fmaf((float)a[e], (float)a[e], sq);
  }
  for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o);
  const float inv = 1.f / sqrtf(sq / (float)C + eps);
#pragma unroll
  for (int j = 0; j < kMaxVecs; ++j) {
    const int cv = lane + 64 * j;
    if (cv >= nvec) continue;
    const bf16* a = (const bf16*)&xv[j];
    const u4 wv = *(const u4*)(w + cv * 8);
    const bf16* ww = (const bf16*)&wv;
    u4 ov;
    bf16* o = (bf16*)&ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (bf16)(rb(__fmul_rn((float)a[e], inv)) * (float)ww[e]);
    *(u4*)(out + n * C + cv * 8) = ov;
  }
}

// every query block lists every context block: kcnt[r] = nkc, kidx[r * nkc + j] = j
__global__ void full_lists_kernel(int rows, int nkc, int32_t* __restrict__ kidx, int32_t* __restrict__ kcnt) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * nkc) return;
  kidx[e] = e % nkc;
  if (e % nkc == 0) kcnt[e / nkc] = nkc;
}

int launch_modulation(const void* m, const void* t, void* out, int C, hipStream_t stream) {
  const int n = 6 * C;
  hipLaunchKernelGGL(modulation_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, (const bf16*)m, (const bf16*)t,
                     (bf16*)out, n);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

int launch_residual_norm(void* x, const void* y, const void* gate, int64_t L, int C, float eps, const void* w,
                         const void* bias, const void* scale, const void* shift, void* out, hipStream_t stream) {
  if (L <= 0) return FVSR_OK;
  if (C % 8 || C / 8 > 64 * kMaxVecs) return set_error(FVSR_ERR_UNSUPPORTED, "norm: channels must be a multiple of 8, <= 3072");
  hipLaunchKernelGGL(residual_norm_kernel, dim3((unsigned)ceil_div(L, 4)), dim3(256), 0, stream, (bf16*)x,
                     (const bf16*)y, (const bf16*)gate, L, C, eps, (const bf16*)w, (const bf16*)bias,
                     (const bf16*)scale, (const bf16*)shift, (bf16*)out);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

int launch_rms_norm(const void* x, int64_t L, int C, float eps, const void* w, void* out, hipStream_t stream) {
  if (L <= 0) return FVSR_OK;
  if (C % 8 || C / 8 > 64 * kMaxVecs) return set_error(FVSR_ERR_UNSUPPORTED, "norm: channels must be a multiple of 8, <= 3072");
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)ceil_div(L, 4)), dim3(256), 0, stream, (const bf16*)x, L, C, eps,
                     (const bf16*)w, (bf16*)out);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

int launch_full_lists(int rows, int nkc, int32_t* kidx, int32_t* kcnt, hipStream_t stream) {
  const int n = rows * nkc;
  if (n <= 0) return FVSR_OK;
  hipLaunchKernelGGL(full_lists_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, rows, nkc, kidx, kcnt);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

}  // namespace fvsr
