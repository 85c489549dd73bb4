// Fused epilogue of the self-attention projections for gfx950 (MI355X): full-width RMSNorm of q and k, 3-D RoPE,
// window partition, and the write of K and V into the streaming KV ring (with the pooled keys the selection reads).
//
// Reference semantics (blockForward, DiT.swift:496-511):
//   q = ropeApply(normQ(q_proj)), k = ropeApply(normK(k_proj)), v = v_proj           DiT.swift:498-502
//   WanRMSNorm: xf = fp32(x); n = xf * rsqrt(mean(xf^2) + eps); out = T(T(n) * weight)   DiT.swift:34-47
//   ropeApply: (re, im) pairs of each head, out = (re cos - im sin, re sin + im cos) in fp32, cast to T
//                                                                                      DiT.swift:100-107
//   RopeTables: per axis (t: 22 pairs, h: 21, w: 21 of the 64 per head) cos/sin of p * theta^(-2j/dim), built in
//   double, stored fp32; token (t, y, x) of a chunk starting at temporal position t0 uses rows t0 + t, y, x
//                                                                                      DiT.swift:52-97
//   windowPartition: (f, h, w) tokens -> 128-token windows (nf, nh, nw) x (wf, wh, ww)  DiT.swift:111-118
//   the window K/V cache concat                                                         DiT.swift:507-511
// The reference runs these as separate MLX ops (each a full pass over the tensors, plus the concat copy of the
// cache); here one pass reads q, k, v once and writes Q (window order) and the new K/V slices once.
//
// Kernel: one wave per token (4 per workgroup), tokens in natural order so every wave reads three contiguous rows.
// Each lane holds C / 64 / 8 vectors of 8 channels (bf16) of q, k and v; the sum of squares of a row is a wave
// butterfly; every lane then normalises, weights and rotates its own channels and writes them to the token's window
// position. The pooled keys of a ring append are made afterwards by the same pooling kernel as for plain buffers
// (pool_mean_kernel over the new ring slots), so they are bit-identical to pooling the written K.
#include <type_traits>

#include "common.hpp"

namespace fvsr {

// layout of the RoPE tables buffer (fp32): cos_t, sin_t (end x 22), cos_h, sin_h (end x 21), cos_w, sin_w (end x 21)
constexpr int kRopeEnd = 1024;
constexpr int kRopeT = 22, kRopeH = 21, kRopeW = 21;   // complex pairs per axis for a 128-wide head
constexpr int kRopeCosT = 0, kRopeSinT = kRopeEnd * kRopeT;
constexpr int kRopeCosH = 2 * kRopeEnd * kRopeT, kRopeSinH = kRopeCosH + kRopeEnd * kRopeH;
constexpr int kRopeCosW = kRopeCosH + 2 * kRopeEnd * kRopeH, kRopeSinW = kRopeCosW + kRopeEnd * kRopeW;
constexpr int kRopeFloats = kRopeCosW + 2 * kRopeEnd * kRopeW;

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return (float)(T)x;
}

// NV = 16-byte vectors per lane (C * sizeof(T) / 16 / 64, rounded up; at most 6): the token's q, k and v stay in
// registers, so sizing them to the width keeps the register count, and with it the waves in flight, where this
// memory-bound pass needs them (3 vectors for 1536 bf16 channels).
template <typename T, int NV>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, int64_t L, int C, int nbh, int nbw,
    int t0, const T* __restrict__ wq, const T* __restrict__ wk, float eps, const float* __restrict__ rope,
    T* __restrict__ q_out, T* __restrict__ k_out, T* __restrict__ v_out, int dst_slot0, int capacity,
    int slice_blocks, int64_t kv_head_stride) {
  constexpr int VN = 16 / sizeof(T);
  constexpr int kMaxVec = NV;
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // natural token index
  if (n >= L) return;
  const int nvec = C / VN;
  const int W = 8 * nbw, H = 8 * nbh;
  const int x = (int)(n % W), y = (int)((n / W) % H), fi = (int)(n / ((int64_t)W * H));
  // window position of the token: window (fi/2, y/8, x/8), token (fi%2, y%8, x%8) (DiT.swift:113-118)
  const int b = ((fi >> 1) * nbh + (y >> 3)) * nbw + (x >> 3);
  const int t = ((fi & 1) << 6) | ((y & 7) << 3) | (x & 7);
  const int64_t db = (int64_t)((dst_slot0 + b / slice_blocks) % capacity) * slice_blocks + (b % slice_blocks);

  u4 xq[kMaxVec], xk[kMaxVec], xv[kMaxVec];
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int cv = lane + 64 * j;
    if (cv < nvec) {
      xq[j] = *(const u4*)(q + n * C + cv * VN);
      xk[j] = *(const u4*)(k + n * C + cv * VN);
      xv[j] = *(const u4*)(v + n * C + cv * VN);
      const T* aq = (const T*)&xq[j];
      const T* ak = (const T*)&xk[j];
#pragma unroll
      for (int e = 0; e < VN; ++e) {
        sq = fmaf((float)aq[e], (float)aq[e], sq);
        sk = fmaf((float)ak[e], (float)ak[e], sk);
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    sq += __shfl_xor(sq, o);
    sk += __shfl_xor(sk, o);
  }
  // rsqrt(mean + eps) as a correctly rounded square root and division
  const float inv_q = 1.f / sqrtf(sq / (float)C + eps);
  const float inv_k = 1.f / sqrtf(sk / (float)C + eps);
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int cv = lane + 64 * j;
    if (cv >= nvec) continue;
    const int c0 = cv * VN;
    const int j0 = (c0 % kHeadDim) / 2;   // first complex pair (within the head) of this vector
    const T* aq = (const T*)&xq[j];
    const T* ak = (const T*)&xk[j];
    // the norm weights of these channels, one 16-byte load each
    const u4 wqv = *(const u4*)(wq + c0), wkv = *(const u4*)(wk + c0);
    const T* wqe = (const T*)&wqv;
    const T* wke = (const T*)&wkv;
    u4 oq, ok;
    T* rq = (T*)&oq;
    T* rk = (T*)&ok;
#pragma unroll
    for (int p = 0; p < VN / 2; ++p) {
      const int jj = j0 + p;
      int ci, si;
      if (jj < kRopeT) {
        ci = kRopeCosT + (t0 + fi) * kRopeT + jj;
        si = kRopeSinT + (t0 + fi) * kRopeT + jj;
      } else if (jj < kRopeT + kRopeH) {
        ci = kRopeCosH + y * kRopeH + (jj - kRopeT);
        si = kRopeSinH + y * kRopeH + (jj - kRopeT);
      } else {
        ci = kRopeCosW + x * kRopeW + (jj - kRopeT - kRopeH);
        si = kRopeSinW + x * kRopeW + (jj - kRopeT - kRopeH);
      }
      const float cs = rope[ci], sn = rope[si];
      // normalise, round to T, weight, round to T (WanRMSNorm), then rotate in fp32 with one rounding per product
      // and sum, and round to T (ropeApply)
      const float wq0 = (float)wqe[2 * p], wq1 = (float)wqe[2 * p + 1];
      const float wk0 = (float)wke[2 * p], wk1 = (float)wke[2 * p + 1];
      const float qre = round_to<T>(round_to<T>(__fmul_rn((float)aq[2 * p], inv_q)) * wq0);
      const float qim = round_to<T>(round_to<T>(__fmul_rn((float)aq[2 * p + 1], inv_q)) * wq1);
      const float kre = round_to<T>(round_to<T>(__fmul_rn((float)ak[2 * p], inv_k)) * wk0);
      const float kim = round_to<T>(round_to<T>(__fmul_rn((float)ak[2 * p + 1], inv_k)) * wk1);
      rq[2 * p] = (T)__fsub_rn(__fmul_rn(qre, cs), __fmul_rn(qim, sn));
      rq[2 * p + 1] = (T)__fadd_rn(__fmul_rn(qre, sn), __fmul_rn(qim, cs));
      rk[2 * p] = (T)__fsub_rn(__fmul_rn(kre, cs), __fmul_rn(kim, sn));
      rk[2 * p + 1] = (T)__fadd_rn(__fmul_rn(kre, sn), __fmul_rn(kim, cs));
    }
    *(u4*)(q_out + ((int64_t)b * kBlock + t) * C + c0) = oq;
    const int64_t kvo = kv_offset(db * kBlock + t, c0, C, kv_head_stride);   // token-major, or head-major (a ring)
    *(u4*)(k_out + kvo) = ok;
    *(u4*)(v_out + kvo) = xv[j];
  }
}

int launch_qkv_epilogue(int dtype, const void* q, const void* k, const void* v, int f, int h, int w, int C, int t0,
                        const void* wq, const void* wk, float eps, const float* rope, void* q_out, void* k_out,
                        void* v_out, int dst_slot0, int capacity, int slice_blocks, int64_t kv_head_stride,
                        hipStream_t stream) {
  const int nbh = h / 8, nbw = w / 8;
  const int64_t L = (int64_t)f * h * w;
  if (L <= 0) return FVSR_OK;
  const int es = dtype == FVSR_DTYPE_BF16 ? 2 : 4;
  if (C * es / 16 > 64 * 6) return set_error(FVSR_ERR_UNSUPPORTED, "qkv epilogue: at most 384 16-byte vectors per token");
  const dim3 grid((unsigned)ceil_div(L, 4));
  const int nv = (int)ceil_div((int64_t)C * es / 16, 64);   // 1 .. 6, checked above
  auto go = [&](auto nv_c) {
    constexpr int NV = decltype(nv_c)::value;
    if (dtype == FVSR_DTYPE_BF16)
      hipLaunchKernelGGL((qkv_epilogue_kernel<bf16, NV>), grid, dim3(256), 0, stream, (const bf16*)q,
                         (const bf16*)k, (const bf16*)v, L, C, nbh, nbw, t0, (const bf16*)wq, (const bf16*)wk, eps,
                         rope, (bf16*)q_out, (bf16*)k_out, (bf16*)v_out, dst_slot0, capacity, slice_blocks,
                         kv_head_stride);
    else
      hipLaunchKernelGGL((qkv_epilogue_kernel<float, NV>), grid, dim3(256), 0, stream, (const float*)q,
                         (const float*)k, (const float*)v, L, C, nbh, nbw, t0, (const float*)wq, (const float*)wk,
                         eps, rope, (float*)q_out, (float*)k_out, (float*)v_out, dst_slot0, capacity, slice_blocks,
                         kv_head_stride);
  };
  switch (nv) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    case 5: go(std::integral_constant<int, 5>{}); break;
    default: go(std::integral_constant<int, 6>{}); break;
  }
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

int rope_table_floats() { return kRopeFloats; }

// RopeTables.init (DiT.swift:58-78) for a 128-wide head: per axis dim (44, 42, 42), pair j has frequency
// theta^(-2j/dim); row p holds cos/sin(p * freq) computed in double and stored fp32, in the layout above.
void rope_tables_host(double theta, float* out) {
  const int dims[3] = {kHeadDim - 2 * (kHeadDim / 3), kHeadDim / 3, kHeadDim / 3};
  const int cos_off[3] = {kRopeCosT, kRopeCosH, kRopeCosW}, sin_off[3] = {kRopeSinT, kRopeSinH, kRopeSinW};
  for (int a = 0; a < 3; ++a) {
    const int n = dims[a] / 2;
    for (int p = 0; p < kRopeEnd; ++p)
      for (int j = 0; j < n; ++j) {
        const double freq = 1.0 / pow(theta, (double)(2 * j) / (double)dims[a]);
        const double ang = (double)p * freq;
        out[cos_off[a] + p * n + j] = (float)cos(ang);
        out[sin_off[a] + p * n + j] = (float)sin(ang);
      }
  }
}

}  // namespace fvsr
