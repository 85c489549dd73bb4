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
//   pool_part_kernel     one workgroup per run of 32 tokens of a block: coalesced 16-byte loads, fp32 sums (Q
//                        and K, or Q and the new ring keys, in one launch); the means come from pool_finish_kernel
//                        (kv_ring.hip) in a fixed order, which also clears the histogram below
//   scores_softmax_kernel one workgroup per (8 query blocks, head): pooled-key rows staged through LDS in coalesced
//                         chunks of 64 keys and read once per 8 query rows, scores + local mask in LDS, one wave per
//                         row for max / exp / sum / normalise; it also counts the nonzero probs of each (head,
//                         query slice) per top-12-bit bin
//   topk_threshold_kernel one 1024-thread workgroup per (head, query slice): exact (k+1)-th largest over the fp32
//                         bit patterns (probs are >= 0, so bit order = value order): the row is loaded into
//                         registers at once, the histogram picks the bin, its elements are gathered to LDS and
//                         three radix passes finish the low 19 bits (full-row 4-pass radix select when the bin is
//                         too large)
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

// Sources s0, s1, s2 ((L, C) tokens each) share one launch: grid (s0.nb + s1.nb + s2.nb, kPoolParts), block
// index b of the grid runs over s0's blocks, then s1's, then s2's. Run `part` of block b sums rows
// [b*128 + 32*part, +32) that exist into partial[(b * kPoolParts + part) * C + c] (fp32); pool_finish_kernel forms
// the block means.
template <typename T>
__global__ void pool_part_kernel(PoolSrc s0, PoolSrc s1, PoolSrc s2, int C) {
  constexpr int VN = Vec16<T>::N;
  constexpr int kRun = kBlock / kPoolParts;
  typedef typename Vec16<T>::type VT;
  int b = blockIdx.x;
  const int part = blockIdx.y;
  PoolSrc src = s0;
  if (b >= s0.nb) {
    b -= s0.nb;
    src = s1;
    if (b >= s1.nb) {
      b -= s1.nb;
      src = s2;
    }
  }
  const T* __restrict__ x = (const T*)src.x;
  const int64_t r0 = (int64_t)b * kBlock + part * kRun;
  const int n = (int)max<int64_t>(0, min<int64_t>(kRun, src.L - r0));
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
    float* o = src.partial + ((int64_t)b * kPoolParts + part) * C + cv * VN;
#pragma unroll
    for (int e = 0; e < VN; ++e) o[e] = acc[e];
  }
}

// Adds 1 to h[key] for every lane with `valid`; must be called by all 64 lanes of the wave together. Lanes with
// equal keys are merged first (up to kPeel distinct keys, each by one atomic of the group's size from its lowest
// lane): probs that cluster in a few bins would otherwise put up to 64 atomics on one LDS address, which execute
// one after another. Keys left after the merge rounds (a spread-out wave) take one atomic per lane.
constexpr int kPeel = 4;
__device__ __forceinline__ void wave_hist_add(unsigned* h, unsigned key, bool valid) {
  const int lane = threadIdx.x & 63;
  uint64_t todo = __ballot(valid);
#pragma unroll
  for (int it = 0; it < kPeel; ++it) {
    if (todo == 0ull) break;   // wave-uniform
    const int leader = __builtin_ctzll(todo);
    const unsigned lkey = (unsigned)__builtin_amdgcn_readlane((int)key, leader);
    const uint64_t grp = todo & __ballot(key == lkey);
    if (lane == leader) atomicAdd(&h[lkey], (unsigned)__popcll(grp));
    todo &= ~grp;
  }
  if ((todo >> lane) & 1ull) atomicAdd(&h[key], 1u);
}

// ------------------------------------------------------------------------------------------------------------
// scores + softmax
// ------------------------------------------------------------------------------------------------------------
constexpr int kScoreRows = 8;   // query blocks per workgroup (2 per wave of 256 threads)
constexpr int kKeyChunk = 64;   // key blocks staged in LDS at a time
constexpr int kKStride = kHeadDim + 4;   // padded LDS row of a pooled key (floats)
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
  float* qs = sm;                                      // [kScoreRows][128]
  float* ks = qs + kScoreRows * kHeadDim;              // [kKeyChunk][kKStride]
  // the workgroup histograms of the (up to) two query slices of its rows, [2][kHistBins]: they reuse the key chunk
  // staging once the scores are done (keeping the LDS of a workgroup small enough for 3 per CU)
  unsigned* lhist = (unsigned*)ks;
  float* ss = ks + kKeyChunk * kKStride;               // [kScoreRows][nk]
  const int sw = min(s, nk);                           // local-window columns that key blocks 0..nk-1 use
  uint8_t* lm = (uint8_t*)(ss + kScoreRows * nk);      // [kScoreRows][sw] local-window bytes of this group's rows
  const int h = blockIdx.y;
  const int i0 = blockIdx.x * kScoreRows;
  const int tid = threadIdx.x;
  const int sq = nq / q_slices;                 // query blocks per slice
  const int t_first = i0 / sq;
  for (int e = tid; e < kScoreRows * kHeadDim; e += blockDim.x) {
    const int r = e / kHeadDim, d = e % kHeadDim;
    qs[e] = (i0 + r < nq) ? pq[(int64_t)(i0 + r) * C + h * kHeadDim + d] : 0.f;
  }
  for (int e = tid; e < kScoreRows * sw; e += blockDim.x) {
    const int r = e / sw, c = e - r * sw;
    lm[e] = local[((i0 + r) % s) * s + c];
  }
  __syncthreads();
  const float sqrt_d = sqrtf((float)kHeadDim);
  // Key blocks in chunks of 64: the chunk's pooled-key rows (64 x 512 B) are read with coalesced 16-byte loads
  // (each wave load covers two whole rows) into padded LDS rows, the loads of the next two chunks in flight while
  // the current one is multiplied. The products run on the matrix cores in fp32 (v_mfma_f32_16x16x4_f32): wave w takes keys
  // 16w .. 16w + 15 of the chunk against the 8 query rows (padded to 16). Lane l holds A = Q[l % 16][32 (l / 16) + t]
  // and B = K[16w + l % 16][32 (l / 16) + t] at step t (the reduction index of step t, lane group g is dim 32 g + t,
  // so each lane reads 32 contiguous floats), and the 16 x 16 product lands as D[4 (l / 16) + v][l % 16], v < 4.
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const float* kbase = pk + h * kHeadDim;
  constexpr int kLoads = kKeyChunk * (kHeadDim / 4) / 256;   // 16-byte loads per thread per chunk
  auto load_chunk = [&](f32x4 (&pre)[kLoads], int j0) {
    const int nj = min(kKeyChunk, nk - j0);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int e = i * 256 + tid, jj = e >> 5, c4 = e & 31;
      if (jj < nj) pre[i] = *(const f32x4*)(kbase + (kmap.row(j0 + jj) / kBlock) * C + 4 * c4);
    }
  };
  float qa[32];   // this lane's A operands (query row li, dims 32 lg .. 32 lg + 31; rows >= 8 are zero)
#pragma unroll
  for (int t = 0; t < 32; t += 4) {
    const f32x4 x = li < kScoreRows ? *(const f32x4*)(qs + li * kHeadDim + 32 * lg + t) : f32x4{0.f, 0.f, 0.f, 0.f};
    qa[t] = x[0];
    qa[t + 1] = x[1];
    qa[t + 2] = x[2];
    qa[t + 3] = x[3];
  }
  // one chunk: its rows to LDS, the loads of the chunk after next into the same registers, the products
  auto chunk = [&](f32x4 (&pre)[kLoads], int j0) {
    const int nj = min(kKeyChunk, nk - j0);
    __syncthreads();   // the previous chunk's rows have been read
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int e = i * 256 + tid, jj = e >> 5, c4 = e & 31;
      if (jj < nj) *(f32x4*)(ks + jj * kKStride + 4 * c4) = pre[i];
    }
    __syncthreads();
    if (j0 + 2 * kKeyChunk < nk) load_chunk(pre, j0 + 2 * kKeyChunk);
    if (16 * wave < nj) {   // wave-uniform; rows of keys past nj hold stale data and are not stored
      const float* krow = ks + (16 * wave + li) * kKStride + 32 * lg;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 32; t += 4) {
        const f32x4 kb = *(const f32x4*)(krow + t);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t], kb[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t + 1], kb[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t + 2], kb[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t + 3], kb[3], acc, 0, 0, 0);
      }
      const int jj = 16 * wave + li, j = j0 + jj;
      if (4 * lg < kScoreRows && jj < nj) {   // rows 4 lg .. 4 lg + 3 that are query rows of the group
        const int ksp = j % s;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 4 * lg + v;
          if (r < kScoreRows) ss[r * nk + j] = lm[r * sw + ksp] ? acc[v] / sqrt_d : -INFINITY;
        }
      }
    }
  };
  f32x4 pa[kLoads], pb[kLoads];
  load_chunk(pa, 0);
  if (kKeyChunk < nk) load_chunk(pb, kKeyChunk);
  for (int j0 = 0; j0 < nk; j0 += 2 * kKeyChunk) {
    chunk(pa, j0);
    if (j0 + kKeyChunk < nk) chunk(pb, j0 + kKeyChunk);
  }
  __syncthreads();
  for (int e = tid; e < 2 * kHistBins; e += blockDim.x) lhist[e] = 0u;
  __syncthreads();
  const int nwaves = blockDim.x >> 6;
  for (int r = wave; r < kScoreRows; r += nwaves) {
    if (i0 + r >= nq) break;
    float* srow = ss + r * nk;
    float mx = -INFINITY;
    for (int j = lane; j < nk; j += 64) mx = fmaxf(mx, srow[j]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.f;
    for (int j = lane; j < nk; j += 64) {
      const float ex = expf(srow[j] - mx);
      srow[j] = ex;   // each lane re-reads only its own entries below
      sum += ex;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    float* prow = probs + ((int64_t)h * nq + i0 + r) * nk;
    const int dt = (i0 + r) / sq - t_first;   // 0 or 1 unless a slice holds fewer than kScoreRows blocks
    unsigned* grow = hist + ((int64_t)h * q_slices + (i0 + r) / sq) * kHistBins;
    for (int j0 = 0; j0 < nk; j0 += 64) {   // wave-uniform trip count (the histogram add needs every lane)
      const int j = j0 + lane;
      unsigned u = 0u;
      if (j < nk) {
        const float p = srow[j] / sum;
        prow[j] = p;
        u = __float_as_uint(p);
      }
      // probs are in [0, 1], so u >> 19 < kHistBins; the mask only keeps a NaN (from NaN inputs) in bounds
      const unsigned bin = (u >> 19) & (kHistBins - 1);
      if (dt == 0) wave_hist_add(lhist, bin, u != 0u);   // dt is wave-uniform
      else if (dt == 1) wave_hist_add(lhist + kHistBins, bin, u != 0u);
      else wave_hist_add(grow, bin, u != 0u);
    }
  }
  __syncthreads();
  // flush the nonzero bins of the workgroup histograms
  const int t_last = min(q_slices - 1, (min(i0 + kScoreRows, nq) - 1) / sq);
  for (int dt = 0; dt < 2 && t_first + dt <= t_last; ++dt) {
    unsigned* g = hist + ((int64_t)h * q_slices + t_first + dt) * kHistBins;
    for (int bn = tid; bn < kHistBins; bn += blockDim.x) {
      const unsigned c = lhist[dt * kHistBins + bn];
      if (c) atomicAdd(&g[bn], c);
    }
  }
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
  __shared__ unsigned s_ncand, s_fill;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row = blockIdx.x;                       // (head, query slice)
  const int h = row / q_slices, t = row % q_slices;
  const int sq = nq / q_slices;
  const int64_t base = ((int64_t)h * nq + (int64_t)t * sq) * nk;
  const unsigned* bits = (const unsigned*)(probs + base);
  const int64_t n = (int64_t)sq * nk;
  const int64_t k = min<int64_t>(n - 1, topk);

  // the whole row, when it fits, with every load in flight at once (thread tid holds elements i*1024 + tid); it
  // serves both paths below. Padding never matches a bin or a prefix (bit 31 set).
  const unsigned* hrow = hist12 + (int64_t)row * kHistBins;
  unsigned hv[kHistBins / kTopkThreads];
#pragma unroll
  for (int i = 0; i < kHistBins / kTopkThreads; ++i) hv[i] = hrow[tid * (kHistBins / kTopkThreads) + i];
  const bool in_regs = n <= (int64_t)kTopkThreads * kTopkRegs;
  unsigned v[kTopkRegs];
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kTopkRegs; ++i) {
      const int64_t e = (int64_t)i * kTopkThreads + tid;
      v[i] = e < n ? bits[e] : 0xffffffffu;
    }
  }

  // ---- histogram-guided path ----
  {
    unsigned part = 0;
#pragma unroll
    for (int i = 0; i < kHistBins / kTopkThreads; ++i) {
      bins[tid * (kHistBins / kTopkThreads) + i] = hv[i];
      part += hv[i];
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
      if (in_regs) {
        // gather the elements of the bin from registers: per-thread counts, a workgroup exclusive scan for the
        // slots, then the writes (no atomics)
        unsigned cnt = 0;
#pragma unroll
        for (int i = 0; i < kTopkRegs; ++i) cnt += (v[i] >> 19) == bin ? 1u : 0u;
        unsigned inc = cnt;
        for (int o = 1; o < 64; o <<= 1) {
          const unsigned y = __shfl_up(inc, o);
          if (lane >= o) inc += y;
        }
        __syncthreads();   // every thread has read tot[] of the bin search above
        if (lane == 63) tot[wave] = inc;
        __syncthreads();
        unsigned slot = inc - cnt;
        for (int w = 0; w < wave; ++w) slot += tot[w];
#pragma unroll
        for (int i = 0; i < kTopkRegs; ++i)
          if ((v[i] >> 19) == bin && slot < (unsigned)kCand) cand[slot++] = v[i];
      } else {
        // (a counter of its own: s_ncand may still be read by waves that have not reached this point)
        if (tid == 0) s_fill = 0;
        __syncthreads();
        // gather the elements of the bin from memory (wave-aggregated slot reservation)
        for (int64_t e0 = 0; e0 < n; e0 += kTopkThreads) {
          const int64_t e = e0 + tid;
          const unsigned u = e < n ? bits[e] : 0xffffffffu;
          const bool in = (u >> 19) == bin;
          const uint64_t m = __ballot(in);
          unsigned slot = 0;
          if (lane == 0 && m) slot = atomicAdd(&s_fill, (unsigned)__popcll(m));
          slot = __shfl(slot, 0);
          const unsigned at = slot + __popcll(m & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
          if (in && at < (unsigned)kCand) cand[at] = u;
        }
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
        for (int e0 = 0; e0 < (int)ncand; e0 += kTopkThreads) {   // uniform trip count for wave_hist_add
          const int e = e0 + tid;
          const unsigned u = e < (int)ncand ? cand[e] : 0xffffffffu;
          wave_hist_add(hist[wave], (u >> shift) & dmask, (u & pmask) == prefix);
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
      wave_hist_add(hist[wave], (u >> shift) & dmask, match && !z);
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
// the per-run block sums of n (1..3) sources in one launch; each source's nb is set here from its L
int launch_pool_parts(int dtype, PoolSrc* src, int n, int C, hipStream_t stream) {
  PoolSrc s[3] = {};
  int nb = 0;
  for (int i = 0; i < n && i < 3; ++i) {
    s[i] = src[i];
    s[i].nb = (int)ceil_div(std::max<int64_t>(0, s[i].L), kBlock);
    src[i].nb = s[i].nb;
    nb += s[i].nb;
  }
  if (nb <= 0) return FVSR_OK;
  const int vn = dtype == FVSR_DTYPE_BF16 ? 8 : 4;
  const int nvec = C / vn;
  const int threads = std::min(1024, ((nvec + 63) / 64) * 64);
  const dim3 grid(nb, kPoolParts);
  if (dtype == FVSR_DTYPE_BF16)
    hipLaunchKernelGGL(pool_part_kernel<bf16>, grid, dim3(threads), 0, stream, s[0], s[1], s[2], C);
  else
    hipLaunchKernelGGL(pool_part_kernel<float>, grid, dim3(threads), 0, stream, s[0], s[1], s[2], C);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

size_t scores_smem_bytes(int nk, int s) {
  static_assert(kKeyChunk * kKStride * sizeof(float) >= 2 * kHistBins * sizeof(unsigned), "histograms alias ks");
  return sizeof(float) * ((size_t)kScoreRows * (kHeadDim + nk) + (size_t)kKeyChunk * kKStride) +
         (size_t)kScoreRows * std::min(s, nk);
}

// hist: (heads * q_slices * kHistBins) u32 workspace, zeroed by the caller before the launch (pool_finish_kernel
// clears it together with the pooled queries)
int launch_scores_softmax(const float* pq, const float* pk, KeyMap kmap, int heads, int C, int nq, int nk, int s,
                          const uint8_t* local, float* probs, unsigned* hist, int q_slices, hipStream_t stream) {
  if (nq <= 0 || nk <= 0) return FVSR_OK;
  dim3 grid((nq + kScoreRows - 1) / kScoreRows, heads);
  const size_t smem = scores_smem_bytes(nk, s);
  if (smem > 160 * 1024)
    return set_error(FVSR_ERR_UNSUPPORTED, "scores stage: too many key blocks for LDS");
  hipLaunchKernelGGL(scores_softmax_kernel, grid, dim3(256), smem, stream, pq, pk, kmap, C, nq,
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
