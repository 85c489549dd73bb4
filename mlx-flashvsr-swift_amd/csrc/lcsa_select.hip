// LCSA block selection for gfx950 (MI355X).
//
// Reference semantics: `draftBlockMaskAndProbs` (DiT.swift:158-174) and the kcnt/kidx build of
// `kernelBlockAttention` (SparseAttention.swift:175-177):
//   pq, pk = fp32 mean of each 128-token window, per head;
//   scores = pq . pk^T / sqrt(128) (a true divide), -inf where the local window (tiled over every (query slice,
//   key slice) pair) hides the key block; probs = softmax over the key blocks;
//   per (head, query temporal slice) keep the entries STRICTLY above the (k+1)-th largest of the s*Nk probs,
//   k = min(n - 1, topk).
//
// Kernels (all HBM/L2-bound, no MFMA — the score product is 0.1 GFLOP):
//   pool_part_kernel     one workgroup per run of 32 tokens of a block: coalesced 16-byte loads, fp32 sums; the
//                        means come from pool_finish_kernel (kv_ring.hip) in a fixed order
//   scores_softmax_kernel one workgroup per (8 query blocks, head): pooled-key rows read once per 8 query rows,
//                         scores + local mask staged in LDS, one wave per row for max / exp / sum / normalise
//   scores_softmax_kernel also counts the nonzero probs of each (head, query slice) per top-12-bit bin
//   topk_threshold_kernel one 1024-thread workgroup per (head, query slice): exact (k+1)-th largest over the fp32
//                         bit patterns (probs are >= 0, so bit order = value order): the histogram picks the bin,
//                         its elements are gathered to LDS and three radix passes finish the low 19 bits (full-row
//                         4-pass radix select when the bin is too large)
//   topk_emit_kernel     one wave per query row: mask, selection bytes and compacted key lists (ballot + popcount)
#include "common.hpp"

namespace fvsr {

// ------------------------------------------------------------------------------------------------------------
// pooling
// ------------------------------------------------------------------------------------------------------------
template <typename T>
struct Vec16;   // 16-byte vector of T
template <>
struct Vec16<float> {
  static constexpr int N = 4;
  typedef f32x4 type;
};
template <>
struct Vec16<bf16> {
  static constexpr int N = 8;
  typedef bf16x8 type;
};

// x: (L, C) tokens; grid (nb, kPoolParts): run `part` of block b sums rows [b*128 + 32*part, +32) that exist into
// partial[(b * kPoolParts + part) * C + c] (fp32); pool_finish_kernel forms the block means.
template <typename T>
__global__ void pool_part_kernel(const T* __restrict__ x, int64_t L, int C, float* __restrict__ partial) {
  constexpr int VN = Vec16<T>::N;
  constexpr int kRun = kBlock / kPoolParts;
  typedef typename Vec16<T>::type VT;
  const int b = blockIdx.x, part = blockIdx.y;
  const int64_t r0 = (int64_t)b * kBlock + part * kRun;
  const int n = (int)max<int64_t>(0, min<int64_t>(kRun, L - r0));
  const int nvec = C / VN;
  for (int cv = threadIdx.x; cv < nvec; cv += blockDim.x) {
    float acc[VN];
#pragma unroll
    for (int e = 0; e < VN; ++e) acc[e] = 0.f;
    const T* p = x + r0 * C + cv * VN;
#pragma unroll 8
    for (int r = 0; r < n; ++r) {
      const VT v = *(const VT*)(p + (int64_t)r * C);
#pragma unroll
      for (int e = 0; e < VN; ++e) acc[e] += (float)v[e];
    }
    float* o = partial + ((int64_t)b * kPoolParts + part) * C + cv * VN;
#pragma unroll
    for (int e = 0; e < VN; ++e) o[e] = acc[e];
  }
}

// ------------------------------------------------------------------------------------------------------------
// scores + softmax
// ------------------------------------------------------------------------------------------------------------
constexpr int kScoreRows = 8;   // query blocks per workgroup
constexpr int kHistBins = 4096; // top-12-bit bins (bits 30..19) of the prob bit patterns

// pq: (nq, C) pooled queries; pk: pooled keys, logical key block j at row map.row(j)/128 of pk (C floats each);
// local: (s, s) bytes; probs: (H, nq, nk).
// hist: (H * q_slices, kHistBins) u32, the count of the nonzero probs of each (head, query slice) row per top-12-bit
// bin (bits 30..19; zeros are left out); zeroed before the launch.
__global__ __launch_bounds__(256) void scores_softmax_kernel(const float* __restrict__ pq,
                                                             const float* __restrict__ pk, KeyMap kmap, int C,
                                                             int nq, int nk, int s,
                                                             const uint8_t* __restrict__ local,
                                                             float* __restrict__ probs,
                                                             unsigned* __restrict__ hist, int q_slices) {
  extern __shared__ float sm[];
  __shared__ unsigned lhist[2][kHistBins];   // the (up to) two query slices of this workgroup's rows
  float* qs = sm;                          // [kScoreRows][128]
  float* ss = sm + kScoreRows * kHeadDim;  // [kScoreRows][nk]
  const int h = blockIdx.y;
  const int i0 = blockIdx.x * kScoreRows;
  const int tid = threadIdx.x;
  const int sq = nq / q_slices;                 // query blocks per slice
  const int t_first = i0 / sq;
  for (int e = tid; e < 2 * kHistBins; e += blockDim.x) (&lhist[0][0])[e] = 0;
  for (int e = tid; e < kScoreRows * kHeadDim; e += blockDim.x) {
    const int r = e / kHeadDim, d = e % kHeadDim;
    qs[e] = (i0 + r < nq) ? pq[(int64_t)(i0 + r) * C + h * kHeadDim + d] : 0.f;
  }
  __syncthreads();
  const float sqrt_d = sqrtf((float)kHeadDim);
#pragma unroll 1
  for (int j = tid; j < nk; j += blockDim.x) {
    // keep the (loop-invariant) pooled-query reads inside the loop: hoisting 8 x 128 floats spills
    asm volatile("" ::: "memory");
    const float* krow = pk + (kmap.row(j) / kBlock) * C + h * kHeadDim;
    float acc[kScoreRows];
#pragma unroll
    for (int r = 0; r < kScoreRows; ++r) acc[r] = 0.f;
#pragma unroll 4
    for (int d0 = 0; d0 < kHeadDim; d0 += 4) {
      const f32x4 kv = *(const f32x4*)(krow + d0);
#pragma unroll
      for (int r = 0; r < kScoreRows; ++r) {
        const f32x4 qv = *(const f32x4*)(qs + r * kHeadDim + d0);
        acc[r] = fmaf(qv[0], kv[0], acc[r]);
        acc[r] = fmaf(qv[1], kv[1], acc[r]);
        acc[r] = fmaf(qv[2], kv[2], acc[r]);
        acc[r] = fmaf(qv[3], kv[3], acc[r]);
      }
    }
    const int ksp = j % s;
#pragma unroll
    for (int r = 0; r < kScoreRows; ++r) {
      const int qsp = (i0 + r) % s;
      ss[r * nk + j] = local[qsp * s + ksp] ? acc[r] / sqrt_d : -INFINITY;
    }
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, nwaves = blockDim.x >> 6;
  for (int r = wave; r < kScoreRows; r += nwaves) {
    if (i0 + r >= nq) break;
    const float* srow = ss + r * nk;
    float mx = -INFINITY;
    for (int j = lane; j < nk; j += 64) mx = fmaxf(mx, srow[j]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.f;
    for (int j = lane; j < nk; j += 64) sum += expf(srow[j] - mx);
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    float* prow = probs + ((int64_t)h * nq + i0 + r) * nk;
    const int dt = (i0 + r) / sq - t_first;   // 0 or 1 unless a slice holds fewer than kScoreRows blocks
    unsigned* grow = hist + ((int64_t)h * q_slices + (i0 + r) / sq) * kHistBins;
    for (int j = lane; j < nk; j += 64) {
      const float p = expf(srow[j] - mx) / sum;
      prow[j] = p;
      const unsigned u = __float_as_uint(p);
      if (u != 0u) {
        if (dt < 2) atomicAdd(&lhist[dt][u >> 19], 1u);
        else atomicAdd(&grow[u >> 19], 1u);
      }
    }
  }
  __syncthreads();
  // flush the nonzero bins of the workgroup histograms
  const int t_last = min(q_slices - 1, (min(i0 + kScoreRows, nq) - 1) / sq);
  for (int dt = 0; dt < 2 && t_first + dt <= t_last; ++dt) {
    unsigned* g = hist + ((int64_t)h * q_slices + t_first + dt) * kHistBins;
    for (int bn = tid; bn < kHistBins; bn += blockDim.x) {
      const unsigned c = lhist[dt][bn];
      if (c) atomicAdd(&g[bn], c);
    }
  }
}

__global__ void fill_zero_u32_kernel(unsigned* __restrict__ p, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n) p[e] = 0u;
}

// ------------------------------------------------------------------------------------------------------------
// exact top-k threshold + mask / list emit
// ------------------------------------------------------------------------------------------------------------
constexpr int kTopkThreads = 1024;
constexpr int kTopkRegs = 80;   // elements per thread kept in registers (rows up to 81920 entries)

// One 1024-thread workgroup per (head, query slice) row of s*Nk probs: the (k+1)-th largest, k = min(n-1, topk), by
// an exact radix select over the fp32 bit patterns (probs are >= 0, so bit order = value order and bit 31 is 0).
// Digits follow the float layout — exponent [30:23], then mantissa [22:15], [14:7], [6:0] — so the first pass
// spreads the row over its octaves. The row stays in registers across the passes (re-read from memory only for
// rows longer than 1024 * kTopkRegs). Exact zeros (key blocks outside the local window) are counted with a wave
// ballot instead of 64 colliding LDS atomics.
// One workgroup per (head, query slice) row. First the top-12-bit histogram that scores_softmax_kernel built picks
// the bin holding the (k+1)-th largest; its elements are gathered into LDS and the remaining 19 bits are resolved
// there by three small radix passes. A bin holding more than kCand elements (e.g. the threshold falls on the zeros)
// takes the full-row radix select below instead.
constexpr int kCand = 16384;

__global__ __launch_bounds__(kTopkThreads) void topk_threshold_kernel(const float* __restrict__ probs, int nq,
                                                                      int nk, int q_slices, int topk,
                                                                      const unsigned* __restrict__ hist12,
                                                                      float* __restrict__ thr_out) {
  __shared__ unsigned hist[kTopkThreads / 64][256];
  __shared__ unsigned tot[256];
  __shared__ unsigned s_prefix, s_rank;
  __shared__ unsigned cand[kCand];
  __shared__ unsigned bins[kHistBins];
  __shared__ unsigned s_ncand;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row = blockIdx.x;                       // (head, query slice)
  const int h = row / q_slices, t = row % q_slices;
  const int sq = nq / q_slices;
  const int64_t base = ((int64_t)h * nq + (int64_t)t * sq) * nk;
  const unsigned* bits = (const unsigned*)(probs + base);
  const int64_t n = (int64_t)sq * nk;
  const int64_t k = min<int64_t>(n - 1, topk);

  // ---- histogram-guided path ----
  {
    const unsigned* hrow = hist12 + (int64_t)row * kHistBins;
    unsigned part = 0;
#pragma unroll
    for (int i = 0; i < kHistBins / kTopkThreads; ++i) {
      const unsigned c = hrow[tid * (kHistBins / kTopkThreads) + i];
      bins[tid * (kHistBins / kTopkThreads) + i] = c;
      part += c;
    }
    // inclusive scan of the per-thread sums (1024 threads)
    unsigned incl = part;
    for (int o = 1; o < 64; o <<= 1) {
      const unsigned y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) tot[wave] = incl;
    __syncthreads();
    unsigned wbase = 0;
    for (int w = 0; w < wave; ++w) wbase += tot[w];
    unsigned all = 0;
    for (int w = 0; w < kTopkThreads / 64; ++w) all += tot[w];
    const unsigned zeros = (unsigned)n - all;          // the zeros sort first and sit in bin 0
    const unsigned rank = (unsigned)(n - 1 - k);      // ascending rank of the (k+1)-th largest
    // thread-local exclusive start of its 4 bins, counting the zeros in bin 0
    unsigned cum = wbase + incl - part + (tid > 0 ? zeros : 0u);
    if (tid == 0) s_ncand = 0xffffffffu;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kHistBins / kTopkThreads; ++i) {
      const int bn = tid * (kHistBins / kTopkThreads) + i;
      const unsigned c = bins[bn] + (bn == 0 ? zeros : 0u);
      if (rank >= cum && rank < cum + c) {
        s_prefix = (unsigned)bn << 19;
        s_rank = rank - cum;
        s_ncand = c;
      }
      cum += c;
    }
    __syncthreads();
    const unsigned ncand = s_ncand;
    if (ncand <= (unsigned)kCand) {   // workgroup-uniform
      const unsigned bin = s_prefix >> 19;
      if (tid == 0) s_ncand = 0;
      __syncthreads();
      // gather the elements of the bin (wave-aggregated slot reservation)
      for (int64_t e0 = 0; e0 < n; e0 += kTopkThreads) {
        const int64_t e = e0 + tid;
        const unsigned u = e < n ? bits[e] : 0xffffffffu;
        const bool in = (u >> 19) == bin;
        const uint64_t m = __ballot(in);
        unsigned slot = 0;
        if (lane == 0 && m) slot = atomicAdd(&s_ncand, (unsigned)__popcll(m));
        slot = __shfl(slot, 0);
        if (in) cand[slot + __popcll(m & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))))] = u;
      }
      __syncthreads();
      unsigned prefix = s_prefix, rk = s_rank;
      unsigned pmask = 0xfff80000u;
      const int shifts[3] = {11, 3, 0};
      const unsigned dmasks[3] = {255u, 255u, 7u};
      for (int pass = 0; pass < 3; ++pass) {
        const int shift = shifts[pass];
        const unsigned dmask = dmasks[pass];
        for (int e = tid; e < (kTopkThreads / 64) * 256; e += kTopkThreads) (&hist[0][0])[e] = 0;
        __syncthreads();
        for (int e = tid; e < (int)ncand; e += kTopkThreads) {
          const unsigned u = cand[e];
          if ((u & pmask) == prefix) atomicAdd(&hist[wave][(u >> shift) & dmask], 1u);
        }
        __syncthreads();
        if (tid < 256) {
          unsigned c = 0;
#pragma unroll
          for (int w = 0; w < kTopkThreads / 64; ++w) c += hist[w][tid];
          tot[tid] = c;
        }
        __syncthreads();
        if (wave == 0) {
          const unsigned c0 = tot[4 * lane], c1 = tot[4 * lane + 1], c2 = tot[4 * lane + 2], c3 = tot[4 * lane + 3];
          const unsigned lsum = c0 + c1 + c2 + c3;
          unsigned inc = lsum;
          for (int o = 1; o < 64; o <<= 1) {
            const unsigned y = __shfl_up(inc, o);
            if (lane >= o) inc += y;
          }
          const unsigned excl = inc - lsum;
          if (rk >= excl && rk < inc) {
            unsigned cm = excl, d = 4 * lane;
            const unsigned cs[4] = {c0, c1, c2, c3};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (rk < cm + cs[q]) { d = 4 * lane + q; break; }
              cm += cs[q];
            }
            s_prefix = prefix | (d << shift);
            s_rank = rk - cm;
          }
        }
        __syncthreads();
        prefix = s_prefix;
        rk = s_rank;
        pmask |= dmask << shift;
      }
      if (tid == 0) thr_out[row] = __uint_as_float(prefix);
      return;
    }
    __syncthreads();
  }

  // ---- full-row radix select (the bin is too large for LDS) ----
  const bool in_regs = n <= (int64_t)kTopkThreads * kTopkRegs;
  unsigned v[kTopkRegs];
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kTopkRegs; ++i) {
      const int64_t e = (int64_t)i * kTopkThreads + tid;
      v[i] = e < n ? bits[e] : 0xffffffffu;   // padding never matches a prefix (bit 31 set)
    }
  }
  unsigned rank = (unsigned)(n - 1 - k);            // ascending rank of the (k+1)-th largest
  unsigned prefix = 0, pmask = 0x80000000u;
  if (tid == 0) {
    s_prefix = 0;
    s_rank = rank;
  }
  const int shifts[4] = {23, 15, 7, 0};
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = shifts[pass];
    const unsigned dmask = pass == 3 ? 127u : 255u;
    for (int e = tid; e < (kTopkThreads / 64) * 256; e += kTopkThreads) (&hist[0][0])[e] = 0;
    __syncthreads();
    unsigned zeros = 0;   // elements equal to 0 that match the prefix (all fall in digit 0), counted per wave
    auto count = [&](unsigned u) {
      const bool match = (u & pmask) == prefix;
      const bool z = match && u == 0u;
      zeros += __popcll(__ballot(z));
      if (match && !z) atomicAdd(&hist[wave][(u >> shift) & dmask], 1u);
    };
    if (in_regs) {
#pragma unroll
      for (int i = 0; i < kTopkRegs; ++i) count(v[i]);
    } else {
      for (int64_t e0 = 0; e0 < n; e0 += kTopkThreads) {
        const int64_t e = e0 + tid;
        count(e < n ? bits[e] : 0xffffffffu);
      }
    }
    if (lane == 0 && zeros) atomicAdd(&hist[wave][0], zeros);
    __syncthreads();
    if (tid < 256) {
      unsigned c = 0;
#pragma unroll
      for (int w = 0; w < kTopkThreads / 64; ++w) c += hist[w][tid];
      tot[tid] = c;
    }
    __syncthreads();
    if (wave == 0) {
      // lane owns bins 4*lane .. 4*lane+3
      const unsigned c0 = tot[4 * lane], c1 = tot[4 * lane + 1], c2 = tot[4 * lane + 2], c3 = tot[4 * lane + 3];
      const unsigned lsum = c0 + c1 + c2 + c3;
      unsigned incl = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const unsigned excl = incl - lsum;
      if (rank >= excl && rank < incl) {
        unsigned cum = excl, d = 4 * lane;
        const unsigned cs[4] = {c0, c1, c2, c3};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (rank < cum + cs[q]) { d = 4 * lane + q; break; }
          cum += cs[q];
        }
        s_prefix = prefix | (d << shift);
        s_rank = rank - cum;
      }
    }
    __syncthreads();
    prefix = s_prefix;
    rank = s_rank;
    pmask |= dmask << shift;
  }
  if (tid == 0) thr_out[row] = __uint_as_float(prefix);
}

// Mask, selection bytes and key lists from the row thresholds: one wave per query row (head, query block). Lists
// hold the selected key blocks ascending, then the unselected ascending (argSort(!sel) of SparseAttention.swift:177
// with a stable order).
__global__ __launch_bounds__(256) void topk_emit_kernel(const float* __restrict__ probs,
                                                        const float* __restrict__ thr, int heads, int nq, int nk,
                                                        int q_slices, float* __restrict__ mask_out,
                                                        uint8_t* __restrict__ sel, int32_t* __restrict__ kidx,
                                                        int32_t* __restrict__ kcnt) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);   // h * nq + qi
  if (row >= heads * nq) return;
  const int h = row / nq, qi = row - h * nq;
  const int sq = nq / q_slices;
  const float th = thr[h * q_slices + qi / sq];
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t roff = (int64_t)row * nk;
  const float* prow = probs + roff;
  int32_t* krow = kidx + roff;
  int n_sel = 0;
  for (int j0 = 0; j0 < nk; j0 += 64) {
    const int j = j0 + lane;
    const bool s = j < nk && prow[j] > th;
    const uint64_t b = __ballot(s);
    if (s) krow[n_sel + __popcll(b & lt)] = j;
    if (j < nk) {
      sel[roff + j] = s ? 1 : 0;
      if (mask_out) mask_out[roff + j] = s ? 1.f : 0.f;
    }
    n_sel += __popcll(b);
  }
  int n_un = n_sel;
  for (int j0 = 0; j0 < nk; j0 += 64) {
    const int j = j0 + lane;
    const bool u = j < nk && !(prow[j] > th);
    const uint64_t b = __ballot(u);
    if (u) krow[n_un + __popcll(b & lt)] = j;
    n_un += __popcll(b);
  }
  if (lane == 0) kcnt[row] = n_sel;
}

// ------------------------------------------------------------------------------------------------------------
// launch
// ------------------------------------------------------------------------------------------------------------
int launch_pool_finish(const float* partial, int nb, int C, int64_t L, int dst_slot0, int capacity,
                       int slice_blocks, float* out, hipStream_t stream);   // kv_ring.hip

// the per-run block sums of x (L tokens): partial[(b * kPoolParts + part) * C + c], (ceil(L/128) * kPoolParts, C)
int launch_pool_parts(int dtype, const void* x, int64_t L, int C, float* partial, hipStream_t stream) {
  const int nb = (int)ceil_div(L, kBlock);
  if (nb <= 0) return FVSR_OK;
  const int vn = dtype == FVSR_DTYPE_BF16 ? 8 : 4;
  const int nvec = C / vn;
  const int threads = std::min(1024, ((nvec + 63) / 64) * 64);
  const dim3 grid(nb, kPoolParts);
  if (dtype == FVSR_DTYPE_BF16)
    hipLaunchKernelGGL(pool_part_kernel<bf16>, grid, dim3(threads), 0, stream, (const bf16*)x, L, C, partial);
  else
    hipLaunchKernelGGL(pool_part_kernel<float>, grid, dim3(threads), 0, stream, (const float*)x, L, C, partial);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

// block means of x: partial (ceil(L/128) * kPoolParts, C) fp32 scratch
int launch_pool(int dtype, const void* x, int64_t L, int C, float* out, float* partial, hipStream_t stream) {
  const int nb = (int)ceil_div(L, kBlock);
  if (nb <= 0) return FVSR_OK;
  const int rc = launch_pool_parts(dtype, x, L, C, partial, stream);
  if (rc) return rc;
  return launch_pool_finish(partial, nb, C, L, 0, 1, 1 << 30, out, stream);
}

size_t scores_smem_bytes(int nk) { return sizeof(float) * (size_t)kScoreRows * (kHeadDim + nk); }

// hist: (heads * q_slices * kHistBins) u32 workspace, zeroed here before the scores
int launch_scores_softmax(const float* pq, const float* pk, KeyMap kmap, int heads, int C, int nq, int nk, int s,
                          const uint8_t* local, float* probs, unsigned* hist, int q_slices, hipStream_t stream) {
  if (nq <= 0 || nk <= 0) return FVSR_OK;
  const int64_t nh = (int64_t)heads * q_slices * kHistBins;
  hipLaunchKernelGGL(fill_zero_u32_kernel, dim3((unsigned)ceil_div(nh, 256)), dim3(256), 0, stream, hist, nh);
  FVSR_HIP_CHECK(hipGetLastError());
  dim3 grid((nq + kScoreRows - 1) / kScoreRows, heads);
  hipLaunchKernelGGL(scores_softmax_kernel, grid, dim3(256), scores_smem_bytes(nk), stream, pq, pk, kmap, C, nq,
                     nk, s, local, probs, hist, q_slices);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

size_t hist12_bytes(int heads, int q_slices) { return (size_t)heads * q_slices * kHistBins * sizeof(unsigned); }

int launch_topk_emit(const float* probs, int heads, int nq, int nk, int q_slices, int topk, const unsigned* hist,
                     float* thr, float* mask_out, uint8_t* sel, int32_t* kidx, int32_t* kcnt, hipStream_t stream) {
  if (nq <= 0 || nk <= 0) return FVSR_OK;
  hipLaunchKernelGGL(topk_threshold_kernel, dim3(heads * q_slices), dim3(kTopkThreads), 0, stream, probs, nq, nk,
                     q_slices, topk, hist, thr);
  FVSR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(topk_emit_kernel, dim3((heads * nq + 3) / 4), dim3(256), 0, stream, probs, thr, heads, nq, nk,
                     q_slices, mask_out, sel, kidx, kcnt);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

}  // namespace fvsr
