// Streaming KV window cache (ring) and window-layout kernels for gfx950 (MI355X).
//
// Reference semantics: the window K/V cache of `blockForward` (DiT.swift:507-511 concat, :532-538 trim) and
// `windowPartition` / `windowReverse` (DiT.swift:113-126).
//
// Design: the reference rebuilds the whole window each chunk (concat = read cache + new, write all). Here each
// layer owns `capacity` slots of one temporal slice (s blocks x 128 tokens x C) in window order; an append writes
// only the new slices into the next free slots (and mean-pools each new key block on the way, so selection never
// re-reads cached keys); evict moves the ring head. Attention and selection address key block j through
// slot = (head + j / s) % capacity. All kernels are pure HBM streams: one workgroup per 128-token block, 16-byte
// loads/stores, 8 tokens in flight per thread.
#include "common.hpp"

namespace fvsr {

// Copies 128-token blocks between layouts (16 bytes per vector). Block b of the source maps to block dst_block(b)
// of the destination; tokens inside a block may be gathered from grid order (src_grid) or scattered to grid order
// (dst_grid). Grid (blocks, kPoolParts): each workgroup moves one run of 32 tokens, so a one-slice append still
// spreads over every CU. When `partial` is set it also writes the fp32 sum of its run of src (the keys) to
// partial[(b * kPoolParts + part) * C + c]; pool_finish_kernel turns the runs into the block mean.
template <typename T>
__global__ void block_copy_kernel(const T* __restrict__ src, T* __restrict__ dst, int C, bool src_grid,
                                  bool dst_grid, int nbh, int nbw, int dst_slot0, int capacity, int slice_blocks,
                                  float* __restrict__ partial, const T* __restrict__ src2, T* __restrict__ dst2,
                                  int64_t dst_head_stride) {
  constexpr int VN = 16 / sizeof(T);
  constexpr int kRun = kBlock / kPoolParts;
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int b = blockIdx.x, part = blockIdx.y;
  // destination block: ring slot (dst_slot0 + b / s) % capacity, block b % s; identity when capacity == 1 and
  // slice_blocks >= the block count
  const int64_t db = (int64_t)((dst_slot0 + b / slice_blocks) % capacity) * slice_blocks + (b % slice_blocks);
  const int nvec = C / VN;
  for (int cv = threadIdx.x; cv < nvec; cv += blockDim.x) {
    float acc[VN];
#pragma unroll
    for (int e = 0; e < VN; ++e) acc[e] = 0.f;
#pragma unroll 8
    for (int t = part * kRun; t < (part + 1) * kRun; ++t) {
      const int64_t si = src_grid ? window_token_to_grid(b, t, nbh, nbw) : (int64_t)b * kBlock + t;
      const int64_t di = dst_grid ? window_token_to_grid((int)db, t, nbh, nbw) : db * kBlock + t;
      const int64_t dof = kv_offset(di, cv * VN, C, dst_head_stride);   // token-major, or head-major (a ring)
      const u4 x = *(const u4*)(src + si * C + cv * VN);
      *(u4*)(dst + dof) = x;
      if (src2) *(u4*)(dst2 + dof) = *(const u4*)(src2 + si * C + cv * VN);
      if (partial) {
        const T* xv = (const T*)&x;
#pragma unroll
        for (int e = 0; e < VN; ++e) acc[e] += (float)xv[e];
      }
    }
    if (partial) {
      float* o = partial + ((int64_t)b * kPoolParts + part) * C + cv * VN;
#pragma unroll
      for (int e = 0; e < VN; ++e) o[e] = acc[e];
    }
  }
}

// Block means from the per-run sums: out[dst(b) * C + c] = ((p0 + p1) + (p2 + p3)) / n_b, n_b = the valid tokens
// of block b (L tokens in all), dst(b) the ring mapping of block_copy_kernel (identity for plain buffers). The fixed
// order makes the pooled keys of a ring append and of a plain-buffer pool bit-identical. One launch finishes up to
// two targets (d0's elements first) and also clears `zero` (nzero words), the selection's histogram, which saves a
// launch of its own.
__global__ void pool_finish_kernel(PoolDst d0, PoolDst d1, int C, unsigned* __restrict__ zero, int64_t nzero) {
  int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < nzero) zero[e] = 0u;
  PoolDst d = d0;
  const int64_t n0 = (int64_t)d0.nb * C;
  if (e >= n0) {
    e -= n0;
    d = d1;
  }
  if (e >= (int64_t)d.nb * C) return;
  const int b = (int)(e / C), c = (int)(e - (int64_t)b * C);
  const float* p = d.partial + (int64_t)b * kPoolParts * C + c;
  const float sum = (p[0] + p[C]) + (p[2 * C] + p[3 * C]);
  const int n = (int)min<int64_t>(kBlock, d.L - (int64_t)b * kBlock);
  const int64_t db = (int64_t)((d.slot0 + b / d.slice_blocks) % d.capacity) * d.slice_blocks + (b % d.slice_blocks);
  d.out[db * C + c] = sum / (float)n;
}

// n targets (0..2); zero / nzero may be null / 0
int launch_pool_finish(const PoolDst* dst, int n, int C, unsigned* zero, int64_t nzero, hipStream_t stream) {
  PoolDst d[2] = {};
  for (int i = 0; i < n && i < 2; ++i) d[i] = dst[i];
  const int64_t total = std::max((int64_t)d[0].nb * C + (int64_t)d[1].nb * C, zero ? nzero : 0);
  if (total <= 0) return FVSR_OK;
  hipLaunchKernelGGL(pool_finish_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, stream, d[0], d[1], C,
                     zero, zero ? nzero : 0);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

// Ring -> window order: logical block j of the held window (slot (head + j/s) % capacity) -> block j of dst.
template <typename T>
__global__ void ring_read_kernel(const T* __restrict__ rk, const T* __restrict__ rv, T* __restrict__ ok,
                                 T* __restrict__ ov, int C, int64_t head_stride, KeyMap map) {
  constexpr int VN = 16 / sizeof(T);
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int j = blockIdx.x;
  const int64_t sr = map.row(j), dr = (int64_t)j * kBlock;
  const int nvec = C / VN;
  for (int e = threadIdx.x; e < kBlock * nvec; e += blockDim.x) {
    const int t = e / nvec, cv = e % nvec;
    const int64_t so = kv_offset(sr + t, cv * VN, C, head_stride);
    *(u4*)(ok + (dr + t) * C + cv * VN) = *(const u4*)(rk + so);
    *(u4*)(ov + (dr + t) * C + cv * VN) = *(const u4*)(rv + so);
  }
}

static int copy_threads(int C, int esize) {
  const int nvec = C * esize / 16;
  return std::min(1024, ((nvec + 63) / 64) * 64);
}

// partial: (n_blocks * kPoolParts, C) fp32 scratch for the pooled-key runs
int launch_ring_append(int dtype, const void* k_new, const void* v_new, int n_blocks, int C, bool grid_layout,
                       int nbh, int nbw, int slot0, int capacity, void* ring_k, void* ring_v, int64_t head_stride,
                       float* pooled, float* partial, hipStream_t stream) {
  if (n_blocks <= 0) return FVSR_OK;
  const int s = nbh * nbw;
  const dim3 grid(n_blocks, kPoolParts);
  if (dtype == FVSR_DTYPE_BF16) {
    hipLaunchKernelGGL(block_copy_kernel<bf16>, grid, dim3(copy_threads(C, 2)), 0, stream, (const bf16*)k_new,
                       (bf16*)ring_k, C, grid_layout, false, nbh, nbw, slot0, capacity, s, partial,
                       (const bf16*)v_new, (bf16*)ring_v, head_stride);
  } else {
    hipLaunchKernelGGL(block_copy_kernel<float>, grid, dim3(copy_threads(C, 4)), 0, stream, (const float*)k_new,
                       (float*)ring_k, C, grid_layout, false, nbh, nbw, slot0, capacity, s, partial,
                       (const float*)v_new, (float*)ring_v, head_stride);
  }
  FVSR_HIP_CHECK(hipGetLastError());
  const PoolDst d{partial, pooled, (int64_t)n_blocks * kBlock, n_blocks, slot0, capacity, s};
  return launch_pool_finish(&d, 1, C, nullptr, 0, stream);
}

int launch_ring_read(int dtype, const void* rk, const void* rv, void* ok, void* ov, int n_blocks, int C,
                     int64_t head_stride, KeyMap map, hipStream_t stream) {
  if (n_blocks <= 0) return FVSR_OK;
  if (dtype == FVSR_DTYPE_BF16)
    hipLaunchKernelGGL(ring_read_kernel<bf16>, dim3(n_blocks), dim3(256), 0, stream, (const bf16*)rk,
                       (const bf16*)rv, (bf16*)ok, (bf16*)ov, C, head_stride, map);
  else
    hipLaunchKernelGGL(ring_read_kernel<float>, dim3(n_blocks), dim3(256), 0, stream, (const float*)rk,
                       (const float*)rv, (float*)ok, (float*)ov, C, head_stride, map);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

// natural (f, h, w) order <-> window order, one workgroup per window
int launch_window_layout(int dtype, const void* x, void* out, int f, int h, int w, int C, bool to_windows,
                         hipStream_t stream) {
  const int nbh = h / 8, nbw = w / 8;
  const int n_blocks = (f / 2) * nbh * nbw;
  if (n_blocks <= 0) return FVSR_OK;
  const int big = 1 << 30;   // identity destination mapping
  if (dtype == FVSR_DTYPE_BF16)
    hipLaunchKernelGGL(block_copy_kernel<bf16>, dim3(n_blocks, kPoolParts), dim3(copy_threads(C, 2)), 0, stream,
                       (const bf16*)x, (bf16*)out, C, to_windows, !to_windows, nbh, nbw, 0, 1, big,
                       (float*)nullptr, (const bf16*)nullptr, (bf16*)nullptr, (int64_t)0);
  else
    hipLaunchKernelGGL(block_copy_kernel<float>, dim3(n_blocks, kPoolParts), dim3(copy_threads(C, 4)), 0, stream,
                       (const float*)x, (float*)out, C, to_windows, !to_windows, nbh, nbw, 0, 1, big,
                       (float*)nullptr, (const float*)nullptr, (float*)nullptr, (int64_t)0);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

}  // namespace fvsr
