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
// Kernels (HBM- or latency-bound; the score product, 0.1 GFLOP, runs on the fp32 matrix cores):
//   pool_mean_kernel     one workgroup per 128-token block and run of 64 channel vectors: its four
//                        quarters sum one run of 32 tokens each (coalesced 16-byte loads, fp32), the runs meet in
//                        LDS and the block mean ((r0 + r1) + (r2 + r3)) / n is stored (Q and K, or Q and the new
//                        ring keys, in one launch); the launch also clears the histogram below
//   scores_softmax_kernel one 8-wave workgroup per (8 query blocks, head), a head's workgroups on one XCD (its L2
//                         serves their pooled keys): pooled-key rows staged through LDS in
//                         coalesced chunks of 64 keys, two chunks side by side, read once per 8 query rows; scores
//                         + local mask in LDS, one wave per row for max / exp / sum / normalise; it also counts the
//                         nonzero probs of each (head, query slice) per top-12-bit bin
//   topk_threshold_kernel 16 workgroups of 256 threads per (head, query slice): exact (k+1)-th largest over the
//                         fp32 bit patterns (probs are >= 0, so bit order = value order): the histogram picks the
//                         bin, each workgroup gathers the bin's elements of its share of the row (held in
//                         registers), and the last to arrive finishes the low 19 bits by three radix passes in LDS
//                         (full-row 4-pass radix select when the bin is too large)
//   topk_emit_kernel     one wave per query row: mask, selection bytes and compacted key lists (ballot + popcount),
//                        the row's probs loaded into registers at once
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

// Jobs j0, j1, j2 share one launch: grid (j0.nb + j1.nb + j2.nb, ceil(nvec / per)) with `per` threads per quarter,
// block index b of the grid runs over j0's blocks, then j1's, then j2's. Quarter `part` of the workgroup sums the
// rows [b*128 + 32*part, +32) that exist, in row order, for channel vectors y*per .. y*per + per - 1; the mean is
// ((r0 + r1) + (r2 + r3)) / n, the order the ring append's runs are finished in (pool_finish_kernel), so pooled keys
// are bit-identical whichever path wrote them. Every workgroup also clears its share of `zero` (nzero words).
constexpr int kPoolVecs = 64;   // channel vectors per workgroup quarter: a 1536-channel block takes 3 workgroups, so
                                // even a one-slice append (135 blocks) spreads over every CU
template <typename T>
__global__ __launch_bounds__(kPoolParts * kPoolVecs) void pool_mean_kernel(PoolMean j0, PoolMean j1, PoolMean j2,
                                                                          int C, unsigned* __restrict__ zero,
                                                                          int64_t nzero) {
  constexpr int VN = Vec16<T>::N;
  constexpr int kRun = kBlock / kPoolParts;
  typedef typename Vec16<T>::type VT;
  __shared__ float red[kPoolParts - 1][kPoolVecs][VN];   // runs 1..3; run 0 stays in registers
  const int64_t nthreads = (int64_t)gridDim.x * gridDim.y * blockDim.x;
  for (int64_t e = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; e < nzero;
       e += nthreads)
    zero[e] = 0u;
  int b = blockIdx.x;
  PoolMean job = j0;
  if (b >= j0.nb) {
    b -= j0.nb;
    job = j1;
    if (b >= j1.nb) {
      b -= j1.nb;
      job = j2;
    }
  }
  if (b >= job.nb) return;   // a launch that only clears `zero`
  const int per = blockDim.x / kPoolParts;   // threads per quarter
  const int part = threadIdx.x / per, t = threadIdx.x - part * per;
  const int cv = blockIdx.y * per + t;
  const int nvec = C / VN;
  const T* __restrict__ x = (const T*)job.x;
  const int64_t r0 = (int64_t)b * kBlock + part * kRun;
  const int n = (int)max<int64_t>(0, min<int64_t>(kRun, job.L - r0));
  const int64_t rstride = job.head_stride == 0 ? C : kHeadDim;   // elements between token rows
  float acc[VN];
#pragma unroll
  for (int e = 0; e < VN; ++e) acc[e] = 0.f;
  if (cv < nvec) {
    const T* p = x + kv_offset(r0, cv * VN, C, job.head_stride);
#pragma unroll 8
    for (int r = 0; r < n; ++r) {
      const VT v = *(const VT*)(p + (int64_t)r * rstride);
#pragma unroll
      for (int e = 0; e < VN; ++e) acc[e] += (float)v[e];
    }
  }
  if (part > 0) {
#pragma unroll
    for (int e = 0; e < VN; ++e) red[part - 1][t][e] = acc[e];
  }
  __syncthreads();
  if (part != 0 || cv >= nvec) return;
  const float cnt = (float)min<int64_t>(kBlock, job.L - (int64_t)b * kBlock);
  const int64_t db =
      (int64_t)((job.slot0 + b / job.slice_blocks) % job.capacity) * job.slice_blocks + (b % job.slice_blocks);
  float* o = job.out + db * C + cv * VN;
#pragma unroll
  for (int e = 0; e < VN; ++e) o[e] = ((acc[e] + red[0][t][e]) + (red[1][t][e] + red[2][t][e])) / cnt;
}

// Adds 1 to h[key] for every lane with `valid`: one LDS atomic per lane. Merging the lanes of equal keys first (a
// ballot round per distinct key, one atomic of the group's size) was slower on every workload measured, clustered
// i.i.d. probabilities included: a round's readlane / ballot chain costs more than the LDS serialising the atomics
// of one address (headline scores 17.9 -> 15.5 us, streaming rows 29.8 -> 25.7 us without it).
__device__ __forceinline__ void wave_hist_add(unsigned* h, unsigned key, bool valid) {
  if (valid) atomicAdd(&h[key], 1u);
}

// ------------------------------------------------------------------------------------------------------------
// scores + softmax
// ------------------------------------------------------------------------------------------------------------
constexpr int kScoreRows = 8;   // query blocks per workgroup (one per wave in the softmax)
constexpr int kScoreThreads = 512;   // 8 waves: two halves of 4 stage alternate key chunks side by side
constexpr int kKeyChunk = 64;   // key blocks staged in LDS at a time by one half
constexpr int kChunksInFlight = 1;   // chunk loads each half keeps in flight (registers): with the two halves
                                     // alternating, one is enough; 92 VGPRs (2 took 118 and ran 3 % slower, 3 took
                                     // 159 and 8 % slower, 4 slower still)
constexpr int kKStride = kHeadDim + 4;   // padded LDS row of a pooled key (floats)
constexpr int kHistBins = 4096; // top-12-bit bins (bits 30..19) of the prob bit patterns

// pq: (nq, C) pooled queries; pk: pooled keys, logical key block j at row map.row(j)/128 of pk (C floats each);
// local: (s, s) bytes; probs: (H, nq, nk).
// hist: (H * q_slices, kHistBins) u32, the count of the nonzero probs of each (head, query slice) row per top-12-bit
// bin (bits 30..19; zeros are left out); zeroed before the launch.
__global__ __launch_bounds__(kScoreThreads) void scores_softmax_kernel(const float* __restrict__ pq,
                                                                       const float* __restrict__ pk, KeyMap kmap,
                                                                       int C, int nq, int nk, int s,
                                                                       const uint8_t* __restrict__ local,
                                                                       float* __restrict__ probs,
                                                                       unsigned* __restrict__ hist, int q_slices) {
  extern __shared__ float sm[];
  float* qs = sm;                                      // [kScoreRows][128]
  float* ks = qs + kScoreRows * kHeadDim;              // [2 halves][kKeyChunk][kKStride]
  // the workgroup histograms of the (up to) two query slices of its rows, [2][kHistBins]: they reuse the key chunk
  // staging once the scores are done
  unsigned* lhist = (unsigned*)ks;
  float* ss = ks + 2 * kKeyChunk * kKStride;           // [kScoreRows][nk]
  const int sw = min(s, nk);                           // local-window columns that key blocks 0..nk-1 use
  uint8_t* lm = (uint8_t*)(ss + kScoreRows * nk);      // [kScoreRows][sw] local-window bytes of this group's rows
  // (head, query group) from the XCD-remapped workgroup index, head-major: each XCD's L2 then serves the pooled keys
  // of one or two heads to all of its workgroups, instead of every head's to a few of each
  const int ngroups = (nq + kScoreRows - 1) / kScoreRows;
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int h = lid / ngroups;
  const int i0 = (lid - h * ngroups) * kScoreRows;
  const int tid = threadIdx.x;
  const int sq = nq / q_slices;                 // query blocks per slice
  const int t_first = i0 / sq;
  const float sqrt_d = sqrtf((float)kHeadDim);
  // Key blocks in chunks of 64, the two halves of the workgroup on alternate chunks (half 0: chunks 0, 2, ..; half
  // 1: chunks 1, 3, ..) with a staging buffer each: the chunk's pooled-key rows (64 x 512 B) are read with coalesced
  // 16-byte loads (each wave load covers two whole rows) into padded LDS rows, the loads of the half's next chunk in
  // flight while the current one is multiplied. The products run on the matrix cores in fp32
  // (v_mfma_f32_16x16x4_f32): wave w of a half takes keys 16w .. 16w + 15 of the chunk against the 8 query rows
  // (padded to 16). Lane l holds A = Q[l % 16][32 (l / 16) + t] and B = K[16w + l % 16][32 (l / 16) + t] at step t
  // (the reduction index of step t, lane group g is dim 32 g + t, so each lane reads 32 contiguous floats), and the
  // 16 x 16 product lands as D[4 (l / 16) + v][l % 16], v < 4.
  const int wave = tid >> 6, lane = tid & 63;
  const int half = wave >> 2, hw = wave & 3, htid = tid & 255;
  const int li = lane & 15, lg = lane >> 4;
  const float* kbase = pk + h * kHeadDim;
  float* kst = ks + half * kKeyChunk * kKStride;
  constexpr int kLoads = kKeyChunk * (kHeadDim / 4) / 256;   // 16-byte loads per thread of a half per chunk
  // every call issues the same kLoads loads (key blocks past nk read block nk - 1, which is never stored), so the
  // compiler can count the first chunks' loads and store the queries before they land
  auto load_chunk = [&](f32x4 (&pre)[kLoads], int j0) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int e = i * 256 + htid, jj = e >> 5, c4 = e & 31;
      pre[i] = *(const f32x4*)(kbase + (kmap.row(min(j0 + jj, nk - 1)) / kBlock) * C + 4 * c4);
    }
  };
  // this lane's A operands, read from LDS at each step: query row li, dims 32 lg .. 32 lg + 31 (lanes li >= 8 read
  // row 7 again: rows >= 8 of the product are not stored)
  const float* qrow = qs + min(li, kScoreRows - 1) * kHeadDim + 32 * lg;
  // one round: each half stages its chunk (j0 < nk) and multiplies it; both halves take part in the barriers
  auto chunk = [&](f32x4 (&pre)[kLoads], int j0, int j_next) {
    const int nj = j0 < nk ? min(kKeyChunk, nk - j0) : 0;
    __syncthreads();   // the previous round's rows have been read
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int e = i * 256 + htid, jj = e >> 5, c4 = e & 31;
      if (jj < nj) *(f32x4*)(kst + jj * kKStride + 4 * c4) = pre[i];
    }
    __syncthreads();
    if (j_next < nk) load_chunk(pre, j_next);   // no loads past the last chunk
    if (16 * hw < nj) {   // wave-uniform; rows of keys past nj hold stale data and are not stored
      const float* krow = kst + (16 * hw + li) * kKStride + 32 * lg;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 32; t += 4) {
        const f32x4 kb = *(const f32x4*)(krow + t);
        const f32x4 qv = *(const f32x4*)(qrow + t);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[0], kb[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[1], kb[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[2], kb[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[3], kb[3], acc, 0, 0, 0);
      }
      const int jj = 16 * hw + li, j = j0 + jj;
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
  // round r: half h multiplies chunk 2 r + h; each half keeps the chunks of its next kChunksInFlight rounds in flight
  // (a register ring), so a round waits on loads issued that many rounds before
  f32x4 pre[kChunksInFlight][kLoads];
  const int rounds = (nk + 2 * kKeyChunk - 1) / (2 * kKeyChunk);
  auto chunk_of = [&](int r) { return (2 * r + half) * kKeyChunk; };
  // the group's pooled queries (two floats per thread) and local-window bytes are loaded first, then the first chunks:
  // loads complete in order, so the queries and bytes can be stored to LDS while the chunks are still in flight (rows
  // past nq read row nq - 1 and store zeros; indices are clamped rather than branched around, so the compiler can
  // count the loads)
  static_assert(kScoreRows * kHeadDim == 2 * kScoreThreads, "two query floats per thread");
  const int qr = 2 * tid / kHeadDim, qd = 2 * tid % kHeadDim;
  const float2 qv = *(const float2*)(pq + (int64_t)min(i0 + qr, nq - 1) * C + h * kHeadDim + qd);
  // local-window bytes: wave r stages row r (its local row (i0 + r) mod s), lane c0 its columns c0 + 64 u; no
  // division per byte
  constexpr int kLmRegs = 4;   // columns per lane held at once: one pass up to 256 columns
  static_assert(kScoreThreads == 64 * kScoreRows, "one wave per local-window row");
  const bool lm_regs = sw <= 64 * kLmRegs;
  const uint8_t* const lrow = local + (int64_t)((i0 + wave) % s) * s;
  uint8_t* const lmrow = lm + wave * sw;
  unsigned lv[kLmRegs];   // a register each: packing the bytes would wait for their loads before the chunks' issue
  if (lm_regs) {
#pragma unroll
    for (int u = 0; u < kLmRegs; ++u) lv[u] = lrow[min(lane + 64 * u, sw - 1)];
  } else {
    for (int c = lane; c < sw; c += 64) lmrow[c] = lrow[c];
  }
  static_for<0, kChunksInFlight>([&](auto d_c) { load_chunk(pre[decltype(d_c)::value], chunk_of(decltype(d_c)::value)); });
  if (lm_regs) {
#pragma unroll
    for (int u = 0; u < kLmRegs; ++u)
      if (lane + 64 * u < sw) lmrow[lane + 64 * u] = (uint8_t)lv[u];
  }
  qs[2 * tid] = i0 + qr < nq ? qv.x : 0.f;
  qs[2 * tid + 1] = i0 + qr < nq ? qv.y : 0.f;
  __syncthreads();
  for (int r0 = 0; r0 < rounds; r0 += kChunksInFlight) {
    static_for<0, kChunksInFlight>([&](auto d_c) {
      constexpr int D = decltype(d_c)::value;
      if (r0 + D < rounds) chunk(pre[D], chunk_of(r0 + D), chunk_of(r0 + D + kChunksInFlight));   // uniform
    });
  }
  __syncthreads();
  // the group's rows fall in one or two query slices: clear the histograms they use
  const int t_last = min(q_slices - 1, (min(i0 + kScoreRows, nq) - 1) / sq);
  const int nlh = min(2, t_last - t_first + 1);
  for (int e = tid; e < nlh * kHistBins; e += kScoreThreads) lhist[e] = 0u;
  __syncthreads();
  for (int r = wave; r < kScoreRows; r += kScoreThreads / 64) {
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
    for (int j0 = 0; j0 < nk; j0 += 64) {
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
  for (int dt = 0; dt < 2 && t_first + dt <= t_last; ++dt) {
    unsigned* g = hist + ((int64_t)h * q_slices + t_first + dt) * kHistBins;
    for (int bn = tid; bn < kHistBins; bn += kScoreThreads) {
      const unsigned c = lhist[dt * kHistBins + bn];
      if (c) atomicAdd(&g[bn], c);
    }
  }
}

// ------------------------------------------------------------------------------------------------------------
// exact top-k threshold + mask / list emit
// ------------------------------------------------------------------------------------------------------------
// The (k+1)-th largest of each (head, query slice) row of s*Nk probs, k = min(n-1, topk), by an exact select over
// the fp32 bit patterns (probs are >= 0, so bit order = value order and bit 31 is 0). kThrParts or more workgroups
// share a row. Each reads the row's top-12-bit histogram (built by scores_softmax_kernel), finds the bin that holds the
// threshold and its rank in the bin (all of them find the same), then scans its share of the row and gathers the
// elements of that bin into the row's candidate area of the workspace. The candidates and the arrival count move
// as relaxed agent-scope atomics (coherent stores and loads past this XCD's L2), ordered by the wait for the stores
// and the barrier before the arrival add; the workgroup that arrives last loads the candidates into LDS and
// resolves the remaining 19 bits by three radix passes (digits [18:11], [10:3], [2:0]). A bin too large for the
// candidate area (e.g. the threshold falls on the exact zeros outside the local window) makes that last workgroup
// run a full-row radix select from memory instead: exponent [30:23], then mantissa [22:15], [14:7], [6:0], with the
// zeros counted by a wave ballot instead of 64 colliding LDS atomics.
constexpr int kThrParts = 16;           // workgroups per (head, query slice) row, at least (more for long rows)
constexpr int kThrMaxParts = 64;
constexpr int kThrThreads = 256;
constexpr int kThrLdsCand = 16384;      // candidates the last workgroup holds in LDS
constexpr int kCandPerBlock = 128;      // candidate words of the workspace per (head, query block)
constexpr int kThrRegs = 16;            // elements per thread held in registers (a share of up to 4096)

// per-row control words after the histograms: [0] candidates gathered, [1] workgroups arrived
__device__ __forceinline__ unsigned* thr_ctl(unsigned* hist12, int rows, int row) {
  return hist12 + (int64_t)rows * kHistBins + 2 * row;
}

// One radix digit over `count(visit)` of a workgroup of kThrThreads: every (masked) element visited is histogrammed
// by its digit (u >> shift) & dmask; the digit holding ascending rank `rank` extends `prefix`, `rank` becomes the
// rank inside it. Zeros matching the prefix are counted by ballot (they all fall in digit 0).
template <class Visit>
__device__ __forceinline__ void radix_digit(unsigned (&hist)[kThrThreads / 64][256], unsigned* tot,
                                            unsigned& prefix, unsigned& rank, unsigned pmask, int shift,
                                            unsigned dmask, Visit&& visit, unsigned* s_prefix, unsigned* s_rank) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int e = tid; e < (kThrThreads / 64) * 256; e += kThrThreads) (&hist[0][0])[e] = 0;
  __syncthreads();
  unsigned zeros = 0;
  visit([&](unsigned u) {   // called by every lane of the wave together
    const bool match = (u & pmask) == prefix;
    const bool z = match && u == 0u;
    zeros += __popcll(__ballot(z));
    wave_hist_add(hist[wave], (u >> shift) & dmask, match && !z);
  });
  if (lane == 0 && zeros) atomicAdd(&hist[wave][0], zeros);
  __syncthreads();
  {
    unsigned c = 0;
#pragma unroll
    for (int w = 0; w < kThrThreads / 64; ++w) c += hist[w][tid];
    tot[tid] = c;
  }
  __syncthreads();
  if (wave == 0) {
    const unsigned c0 = tot[4 * lane], c1 = tot[4 * lane + 1], c2 = tot[4 * lane + 2], c3 = tot[4 * lane + 3];
    const unsigned lsum = c0 + c1 + c2 + c3;
    const unsigned incl = wave_incl_scan(lsum);
    const unsigned excl = incl - lsum;
    if (rank >= excl && rank < incl) {
      unsigned cum = excl, d = 4 * lane;
      const unsigned cs[4] = {c0, c1, c2, c3};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (rank < cum + cs[q]) {
          d = 4 * lane + q;
          break;
        }
        cum += cs[q];
      }
      *s_prefix = prefix | (d << shift);
      *s_rank = rank - cum;
    }
  }
  __syncthreads();
  prefix = *s_prefix;
  rank = *s_rank;
}

// per: the elements of a row each workgroup scans, ceil(sq * nk / gridDim.x) (a host-side division: a 64-bit divide
// here would put branches between the histogram's loads and the share's)
__global__ __launch_bounds__(kThrThreads) void topk_threshold_kernel(const float* __restrict__ probs, int nq,
                                                                     int nk, int q_slices, int topk, int64_t per,
                                                                     unsigned* __restrict__ hist12,
                                                                     unsigned* __restrict__ cand_ws,
                                                                     float* __restrict__ thr_out) {
  static_assert(kThrThreads == 256, "the digit scan gives each thread of a 256-thread workgroup one digit");
  __shared__ unsigned hist[kThrThreads / 64][256];
  __shared__ unsigned tot[256];
  __shared__ unsigned wsum[kThrThreads / 64];
  __shared__ unsigned s_prefix, s_rank, s_ncand, s_arrived;
  __shared__ unsigned cand[kThrLdsCand];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int part = blockIdx.x, row = blockIdx.y;   // row = (head, query slice)
  const int rows = gridDim.y;
  const int h = row / q_slices, t = row % q_slices;
  const int sq = nq / q_slices;
  const unsigned* __restrict__ bits = (const unsigned*)(probs + ((int64_t)h * nq + (int64_t)t * sq) * nk);
  const int64_t n = (int64_t)sq * nk;
  const int64_t k = min<int64_t>(n - 1, topk);
  const unsigned rank0 = (unsigned)(n - 1 - k);   // ascending rank of the (k+1)-th largest
  const unsigned cap = (unsigned)min<int64_t>((int64_t)sq * kCandPerBlock, kThrLdsCand);
  unsigned* const cw = cand_ws + ((int64_t)h * nq + (int64_t)t * sq) * kCandPerBlock;
  unsigned* const ctl = thr_ctl(hist12, rows, row);
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  // 1. the threshold's bin from the histogram: thread tid owns bins 16 tid .. 16 tid + 15
  const unsigned* hrow = hist12 + (int64_t)row * kHistBins;
  unsigned hv[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 x = *(const u32x4*)(hrow + 16 * tid + 4 * i);
    hv[4 * i] = x[0];
    hv[4 * i + 1] = x[1];
    hv[4 * i + 2] = x[2];
    hv[4 * i + 3] = x[3];
  }
  // this workgroup's share of the row: up to kThrRegs * kThrThreads elements are loaded into registers here, every
  // load in flight with the histogram's (they do not depend on the bin; indices are clamped rather than branched
  // around, so the histogram can be waited for alone), and both counted and gathered from there in step 2; a larger
  // share is read twice there
  const int64_t e0 = part * per, e1 = min<int64_t>(n, e0 + per);
  const bool in_regs = per <= (int64_t)kThrRegs * kThrThreads;
  unsigned rv[kThrRegs];   // loaded even when unused (a larger share): a branch here would drain the histogram's
                           // loads and these together
#pragma unroll
  for (int i = 0; i < kThrRegs; ++i) {
    const int64_t e = e0 + tid + (int64_t)i * kThrThreads;
    rv[i] = bits[min(e, n - 1)];   // entries past the share are masked where they are used (in_share)
  }
  unsigned psum = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) psum += hv[i];
  const unsigned incl = wave_incl_scan(psum);
  if (lane == 63) wsum[wave] = incl;
  if (tid == 0) s_ncand = 0xffffffffu;
  __syncthreads();
  unsigned wbase = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kThrThreads / 64; ++w) {
    wbase += w < wave ? wsum[w] : 0u;
    all += wsum[w];
  }
  const unsigned zeros = (unsigned)n - all;        // the zeros sort first and sit in bin 0
  unsigned cum = wbase + incl - psum + (tid > 0 ? zeros : 0u);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int bn = 16 * tid + i;
    const unsigned c = hv[i] + (bn == 0 ? zeros : 0u);
    if (rank0 >= cum && rank0 < cum + c) {
      s_prefix = (unsigned)bn << 19;
      s_rank = rank0 - cum;
      s_ncand = c;
    }
    cum += c;
  }
  __syncthreads();
  const unsigned bin = s_prefix >> 19, ncand = s_ncand;
  const bool gather = ncand <= cap;   // workgroup-uniform (every workgroup of the row decides the same)

  // 2. this workgroup's share of the row: the elements of the bin go to the candidate area. The share is counted
  // first, so one atomic per workgroup reserves its slots (a returning device-scope atomic per wave and step would
  // put a memory round trip on every step).
  if (gather) {
    auto in_share = [&](int i) { return e0 + tid + (int64_t)i * kThrThreads < e1; };
    unsigned mine = 0;
    if (in_regs) {
#pragma unroll
      for (int i = 0; i < kThrRegs; ++i) mine += (rv[i] >> 19) == bin && in_share(i) ? 1u : 0u;
    } else {
      for (int64_t e = e0 + tid; e < e1; e += kThrThreads) mine += (bits[e] >> 19) == bin ? 1u : 0u;
    }
    const unsigned minc = wave_incl_scan(mine);
    if (lane == 63) wsum[wave] = minc;
    __syncthreads();
    unsigned off = minc - mine, wg_total = 0;
#pragma unroll
    for (int w = 0; w < kThrThreads / 64; ++w) {
      off += w < wave ? wsum[w] : 0u;
      wg_total += wsum[w];
    }
    if (tid == 0) s_arrived = wg_total ? __hip_atomic_fetch_add(ctl, wg_total, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT) : 0u;
    __syncthreads();
    unsigned at = s_arrived + off;
    if (mine) {
      if (in_regs) {
#pragma unroll
        for (int i = 0; i < kThrRegs; ++i) {
          if ((rv[i] >> 19) == bin && in_share(i)) {
            if (at < cap) __hip_atomic_store(cw + at, rv[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ++at;
          }
        }
      } else {
        for (int64_t e = e0 + tid; e < e1; e += kThrThreads) {
          const unsigned u = bits[e];
          if ((u >> 19) == bin) {
            if (at < cap) __hip_atomic_store(cw + at, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ++at;
          }
        }
      }
    }
    __syncthreads();   // every thread has read s_arrived
  }
  // Arrival. The candidates are relaxed agent-scope atomic stores (coherent past this XCD's L2); each wave waits for
  // its stores to complete, and only then does thread 0 add the arrival, also relaxed. What keeps the order: the
  // compiler does not move the stores or the add across the barrier's workgroup fences, and the wait means the
  // stores have reached the coherence point before any wave arrives; the last workgroup reads the candidates with
  // relaxed agent-scope loads from that same point. The C++/HIP model asks for a release on the add and an acquire
  // in the last workgroup instead; that form (an acquire-release add plus an agent acquire fence) writes back and
  // invalidates this XCD's L2 and measured 12.1 us per call against 10.2 us here, so the relaxed form is kept.
  FVSR_WAIT_VM0();   // this wave's candidates are stored at device scope
  __syncthreads();
  if (tid == 0) s_arrived = __hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_arrived != gridDim.x - 1) return;   // workgroup-uniform

  // 3. the last workgroup of the row
  unsigned prefix, rk;
  if (gather) {
    for (unsigned e = tid; e < ncand; e += kThrThreads)
      cand[e] = __hip_atomic_load(cw + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    prefix = s_prefix;
    rk = s_rank;
    unsigned pmask = 0xfff80000u;
    const int shifts[3] = {11, 3, 0};
    const unsigned dmasks[3] = {255u, 255u, 7u};
    for (int pass = 0; pass < 3; ++pass) {
      radix_digit(hist, tot, prefix, rk, pmask, shifts[pass], dmasks[pass], [&](auto&& f) {
        for (unsigned b0 = 0; b0 < ncand; b0 += kThrThreads) {
          const unsigned e = b0 + tid;
          f(e < ncand ? cand[e] : 0xffffffffu);
        }
      }, &s_prefix, &s_rank);
      pmask |= dmasks[pass] << shifts[pass];
    }
  } else {
    if (tid == 0) {
      s_prefix = 0;
      s_rank = rank0;
    }
    __syncthreads();
    prefix = 0;
    rk = rank0;
    unsigned pmask = 0x80000000u;
    const int shifts[4] = {23, 15, 7, 0};
    for (int pass = 0; pass < 4; ++pass) {
      const unsigned dmask = pass == 3 ? 127u : 255u;
      radix_digit(hist, tot, prefix, rk, pmask, shifts[pass], dmask, [&](auto&& f) {
        for (int64_t b0 = 0; b0 < n; b0 += kThrThreads) {
          const int64_t e = b0 + tid;
          f(e < n ? bits[e] : 0xffffffffu);
        }
      }, &s_prefix, &s_rank);
      pmask |= dmask << shifts[pass];
    }
  }
  if (tid == 0) thr_out[row] = __uint_as_float(prefix);
}

// Mask, selection bytes and key lists from the row thresholds: one wave per query row (head, query block). Lists
// hold the selected key blocks ascending, then the unselected ascending (argSort(!sel) of SparseAttention.swift:177
// with a stable order). A row of up to 64 * kEmitChunks key blocks is loaded into registers first, every load in
// flight at once (the probs were just written on other XCDs, so each load waits on the memory-side cache); longer
// rows are read chunk by chunk, twice.
constexpr int kEmitChunks = 12;
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
  // selected keys of chunk j0 (lanes j0 + lane < nk whose prob p is above the threshold) go to krow[n_sel ..]
  auto emit_selected = [&](int j0, float p, int& n_sel) {
    const int j = j0 + lane;
    const bool s = j < nk && p > th;
    const uint64_t b = __ballot(s);
    if (s) krow[n_sel + __popcll(b & lt)] = j;
    if (j < nk) {
      sel[roff + j] = s ? 1 : 0;
      if (mask_out) mask_out[roff + j] = s ? 1.f : 0.f;
    }
    n_sel += __popcll(b);
  };
  auto emit_unselected = [&](int j0, float p, int& n_un) {
    const int j = j0 + lane;
    const bool u = j < nk && !(p > th);
    const uint64_t b = __ballot(u);
    if (u) krow[n_un + __popcll(b & lt)] = j;
    n_un += __popcll(b);
  };
  int n_sel = 0, n_un;
  if (nk <= 64 * kEmitChunks) {
    float pv[kEmitChunks];
#pragma unroll
    for (int c = 0; c < kEmitChunks; ++c) pv[c] = prow[min(64 * c + lane, nk - 1)];   // no branch between loads
#pragma unroll
    for (int c = 0; c < kEmitChunks; ++c)
      if (64 * c < nk) emit_selected(64 * c, pv[c], n_sel);
    n_un = n_sel;
#pragma unroll
    for (int c = 0; c < kEmitChunks; ++c)
      if (64 * c < nk) emit_unselected(64 * c, pv[c], n_un);
  } else {
    for (int j0 = 0; j0 < nk; j0 += 64) emit_selected(j0, j0 + lane < nk ? prow[j0 + lane] : 0.f, n_sel);
    n_un = n_sel;
    for (int j0 = 0; j0 < nk; j0 += 64) emit_unselected(j0, j0 + lane < nk ? prow[j0 + lane] : 0.f, n_un);
  }
  if (lane == 0) kcnt[row] = n_sel;
}

// ------------------------------------------------------------------------------------------------------------
// launch
// ------------------------------------------------------------------------------------------------------------
// the block means of n (1..3) jobs in one launch (each job's nb is set here from its L); it also clears
// zero[0 .. nzero) (zero may be null)
int launch_pool_mean(int dtype, PoolMean* jobs, int n, int C, unsigned* zero, int64_t nzero, hipStream_t stream) {
  PoolMean j[3] = {};
  int nb = 0;
  for (int i = 0; i < n && i < 3; ++i) {
    j[i] = jobs[i];
    j[i].nb = (int)ceil_div(std::max<int64_t>(0, j[i].L), kBlock);
    jobs[i].nb = j[i].nb;
    nb += j[i].nb;
  }
  if (!zero) nzero = 0;
  if (nb <= 0 && nzero <= 0) return FVSR_OK;
  const int vn = dtype == FVSR_DTYPE_BF16 ? 8 : 4;
  const int nvec = C / vn;
  const int per = kPoolVecs;   // threads per quarter
  const dim3 grid(std::max(nb, 1), (unsigned)ceil_div(nvec, per));
  if (dtype == FVSR_DTYPE_BF16)
    hipLaunchKernelGGL(pool_mean_kernel<bf16>, grid, dim3(kPoolParts * per), 0, stream, j[0], j[1], j[2], C, zero,
                       nzero);
  else
    hipLaunchKernelGGL(pool_mean_kernel<float>, grid, dim3(kPoolParts * per), 0, stream, j[0], j[1], j[2], C, zero,
                       nzero);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

size_t scores_smem_bytes(int nk, int s) {
  static_assert(2 * kKeyChunk * kKStride * sizeof(float) >= 2 * kHistBins * sizeof(unsigned), "histograms alias ks");
  return sizeof(float) * ((size_t)kScoreRows * (kHeadDim + nk) + (size_t)2 * kKeyChunk * kKStride) +
         (size_t)kScoreRows * std::min(s, nk);
}

// hist: (heads * q_slices * kHistBins) u32 workspace, zeroed by the caller before the launch (pool_mean_kernel
// clears it while it pools the queries)
int launch_scores_softmax(const float* pq, const float* pk, KeyMap kmap, int heads, int C, int nq, int nk, int s,
                          const uint8_t* local, float* probs, unsigned* hist, int q_slices, hipStream_t stream) {
  if (nq <= 0 || nk <= 0) return FVSR_OK;
  dim3 grid((unsigned)(ceil_div(nq, kScoreRows) * heads));   // (head, query group), remapped by XCD in the kernel
  const size_t smem = scores_smem_bytes(nk, s);
  if (smem > 160 * 1024)
    return set_error(FVSR_ERR_UNSUPPORTED, "scores stage: too many key blocks for LDS");
  hipLaunchKernelGGL(scores_softmax_kernel, grid, dim3(kScoreThreads), smem, stream, pq, pk, kmap, C, nq,
                     nk, s, local, probs, hist, q_slices);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

// the (head, query slice) histograms and, after them, two control words per row (all cleared before a selection)
size_t hist12_bytes(int heads, int q_slices) {
  return (size_t)heads * q_slices * (kHistBins + 2) * sizeof(unsigned);
}

// candidate area of the threshold select for `heads` x `nq` query blocks
size_t topk_cand_bytes(int heads, int64_t nq) { return (size_t)heads * nq * kCandPerBlock * sizeof(unsigned); }

int launch_topk_emit(const float* probs, int heads, int nq, int nk, int q_slices, int topk, unsigned* hist,
                     unsigned* cand, float* thr, float* mask_out, uint8_t* sel, int32_t* kidx, int32_t* kcnt,
                     hipStream_t stream) {
  if (nq <= 0 || nk <= 0) return FVSR_OK;
  // enough workgroups per row that each one's share fits its registers (kThrRegs elements per thread)
  const int64_t row_n = (int64_t)(nq / q_slices) * nk;
  const int parts = (int)std::min<int64_t>(kThrMaxParts, std::max<int64_t>(kThrParts,
                                                             ceil_div(row_n, (int64_t)kThrRegs * kThrThreads)));
  hipLaunchKernelGGL(topk_threshold_kernel, dim3(parts, heads * q_slices), dim3(kThrThreads), 0, stream, probs,
                     nq, nk, q_slices, topk, ceil_div(row_n, (int64_t)parts), hist, cand, thr);
  FVSR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(topk_emit_kernel, dim3((heads * nq + 3) / 4), dim3(256), 0, stream, probs, thr, heads, nq, nk,
                     q_slices, mask_out, sel, kidx, kcnt);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

}  // namespace fvsr
