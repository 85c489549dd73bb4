// Block-sparse flash attention over 128x128 blocks for gfx950 (MI355X).
//
// Reference semantics: the Metal kernel of SparseAttention.swift:17-154 (launched at :180-185) and the dense path
// blockMaskedAttention (DiT.swift:279-313): per head, o = softmax(q k^T / sqrt(128)) v over the listed key blocks,
// fp32 online softmax, a query block with no listed key block writes zeros.
//
// bf16 (the production lane): a persistent walk over rows (head, 128-query block); a workgroup = 4 wave64s x 32
// queries, two waves per SIMD; K/V tiles of 32 keys reach LDS by direct buffer->LDS copies into 4-slot rings;
// S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16_bf16 so each lane owns one query row; the softmax keeps a fixed
// reference per row (see the kernel's comment). fp32 (the parity lane): 4 wave64s x 32 queries on
// v_mfma_f32_32x32x2_f32 with a lazy online-softmax rescale; workgroup ids are remapped so each XCD (own L2) walks a
// contiguous run of (head, query block) items.
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace fvsr {

__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) char lds_char;


// O^T += A B on the matrix core. The library is compiled with the MFMA VGPR form (-amdgpu-mfma-vgpr-form): the score
// MFMAs, whose results the VALU reads, and this accumulation write VGPRs (the working set, about 230 registers, fits
// the 256 of two waves per SIMD). The accumulation is the compiler's builtin, so it sees every hazard and keeps one
// register assignment for O across the walk's control paths (the reference raise); successive accumulations into
// one block are >= 7 MFMAs apart.
__device__ __forceinline__ void mfma_acc(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
}
// >= 19 wait states after the last MFMA of a walk (the compiler also inserts what it needs)
__device__ __forceinline__ void acc_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// Lazy online-softmax rescale. The running reference max m_run (log2 domain, per query row) is raised only when a
// tile's row max exceeds it by more than 8, i.e. a factor 2^8: exponentials then stay <= 256 (no overflow in fp32 or
// bf16) and the softmax is mathematically unchanged, while the O/l rescale — a multiply over the whole accumulator —
// runs only on the few tiles where some row of the wave grows (wave-uniform branch). Returns the max to subtract.
template <int NACC>
__device__ __forceinline__ float rescale_if_grown(float mxc, float& m_run, float& l_run, f32x16 (&acc)[NACC]) {
  const bool grow = mxc > m_run + 8.f;
  if (__ballot(grow) != 0) {
    const float m_new = grow ? mxc : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // m_run = -inf -> 0; unchanged row -> 1
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < NACC; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[d][r] *= alpha;
    m_run = m_new;
  }
  return m_run == -INFINITY ? 0.f : m_run;
}

// ------------------------------------------------------------------------------------------------------------
// bf16
// ------------------------------------------------------------------------------------------------------------
// One workgroup = one (head, 128-query block) at a time, two workgroups per CU. QG = 1 (the default): 4 wave64s x 32
// queries, two waves per SIMD (at most 256 registers each), so one wave's LDS, memory and VALU stalls are covered by
// the other's MFMAs. QG = 2: 2 wave64s x 64 queries held as two 32-query groups, one wave per SIMD; every K or V
// operand read from LDS then feeds two MFMAs.
//
// Keys stream in tiles of 32 (a quarter of a 128-key block). K and V tiles land in two LDS rings of kSlots slots by
// buffer_load ... lds (16 B per lane, no VGPR staging); a tile's rows are 256 B (one head) with the 16-byte chunks
// XOR-swizzled by row so the ds_read_b128 (K) and ds_read_b64_tr_b16 (V^T) operand reads are bank-conflict free.
// While tile T is processed (step T), K of tile T+4 and V of tile T+2 are requested; each step ends by waiting for
// the copies of the step before it, so a tile is in LDS a step before the step that first reads it.
//
// Softmax with a lazily raised reference per query row: S = K Q^T in fp32 from the bf16 inputs (keys that do not
// take part score -2^100: in the dense walk by one extra rank-1 MFMA per tile, in the sparse walk by a select on the
// rare tile with fewer than 32 keys: a ragged end, an index outside [0, nk), the tile past the walk's end), then
// P = exp2(c S - m) with one v_fma per score (c = log2(e)/sqrt(128), applied to the fp32 scores as the reference
// does, SparseAttention.swift:96; m, the row's reference, first the exact max of its first tile). A tile whose
// partial row sum exceeds 2^32 (its scores outgrew the reference by about 27 or more, in log2 units) raises the
// reference to the tile's max: its exponentials are recomputed and O and l rescaled (a wave-uniform branch, rare:
// rows with sharp attention raise it a few times). Rows whose exponentials all underflowed (a reference from a tile
// with no valid key, and every real score 2^-32 below it) make the workgroup redo its rows exactly (row-max pass,
// then attention with that max). The result is the softmax whatever the reference is.
//
// Software pipeline per wave, step T: the exponentials of S(T) are issued between the MFMAs of PV(T-1) and QK(T+1),
// so the VALU work hides under matrix-core time. The walk is unrolled by one 128-key block (4 steps); block indices
// are read three blocks ahead so no scalar load latency sits on the step.
namespace {

constexpr int kTileKeys = 32;
constexpr int kRowBytes = kHeadDim * 2;                // one head of one token, bf16
constexpr int kTileBytes = kTileKeys * kRowBytes;      // 8 KB
constexpr int kSlots = 4;                              // per ring: slot of tile T = T mod 4 = its quarter of the block
constexpr int kVRing = kSlots * kTileBytes;            // byte offset of the V ring
constexpr float kMaskedScore = -1.2676506e30f;         // -2^100: exp2 of a masked key is exactly 0
constexpr float kGrowSum = 4294967296.f;               // 2^32: a larger partial row sum raises the reference
constexpr int kMaxPersistentWgs = 1024;                // persistent grid cap (the order kernel's first-row deal)

// 16-byte chunk swizzles. K: the 8 (or 16) lanes one ds_read_b128 cycle serves read 8 (16) consecutive rows of one
// chunk -> distinct positions. V: a ds_read_b64_tr_b16 half-wave (32 lanes, 256 B, one pass over the 64 banks of a
// 256-byte row) reads 4 consecutive rows (a multiple of 4 apart) x 4 adjacent chunks (two 16-lane groups of 2):
// XOR-ing the chunk index with 4 * (row mod 4) puts the 4 rows' aligned 4-chunk groups on 4 different groups, so the
// 32 lanes cover all 64 banks once (the SQ_LDS_BANK_CONFLICT counter reads 0; the former (2 * row) mod 16 swizzle
// left every second cycle a conflict).
__device__ __forceinline__ int swz_k(int r) { return r & 15; }
__device__ __forceinline__ int swz_v(int r) { return (r & 3) << 2; }

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
#define FVSR_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | ((((n) >> 4) & 3) << 14) | (7 << 4))

// 16 bytes per lane from a buffer straight into LDS at lds_base + OFF + 16 * lane. Issued as inline assembly so the
// compiler does not order every later LDS read behind it: the kernel orders the copies itself (vmcnt + barrier).
// M0 is written without a clobber declaration (the compiler reserves it); nothing else in these kernels uses M0. It
// is loaded with s_mov_b32 from an address computed outside the asm. GFX9 requires one wait state between an SALU
// write of M0 and an LDS DMA that reads it; the compiler inserts it for its own code but not inside an asm
// statement, so the s_nop is written out.
// The row's offset `voff` and the block's offset `boff` are added into the one VGPR offset (the SGPR offset is 0):
// the raw buffer's range check covers the VGPR offset and the instruction offset, not the SGPR offset, so only an
// offset held there makes a row past the buffer (a ragged last block, a listed index outside [0, nk), the tiles past
// the end of the walk, whose block offset is the buffer's size) load zeros without touching memory.
template <int OFF>
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t lds_base, int voff, int boff) {
  const uint32_t off = (uint32_t)voff + (uint32_t)boff;   // < 2^31 + 2^17: no wrap
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds_base + OFF),
               "v"(off), "s"(rsrc));
}

__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}


}  // namespace

// The next position of the per-XCD queues of attn_order_kernel's dealt order, starting with this workgroup's XCD
// (dispatch is round-robin over the XCDs: XCD of workgroup b = b % 8), then stealing from the others; `rows` when
// every queue is empty. Queue y holds, wave by wave, the positions w * grid + y + 8 i, i < per_y = ceil((grid - y)
// / 8); its counter (counters[8 y]) starts past the first wave, which the workgroups take without it. Positions
// grow with the counter, so the first one past `rows` means the queue is empty. Called by one thread.
__device__ __forceinline__ int next_dealt_item(int32_t* counters, int rows) {
  const int grid = (int)gridDim.x;
  for (int t = 0; t < kXcds; ++t) {
    const int y = ((int)blockIdx.x + t) & (kXcds - 1);
    const int per = (grid - y + kXcds - 1) / kXcds;
    if (per <= 0) continue;
    const int k = atomicAdd(counters + 8 * y, 1);
    const int p = (k / per) * grid + y + kXcds * (k % per);
    if (p < rows) return p;
  }
  return rows;
}

// LDS operand requests of chunk / pair j >= 2 (j = 0, 1: micro-round 0), in micro-rounds of a step with QG query
// groups per wave and EXT mask MFMAs ahead of the first QK chunk: 7 (QG 2) or 4 (QG 1) micro-rounds before the QK
// MFMA that uses them, micro-round 0 at the earliest
template <int QG, int EXT>
constexpr int attn_read_at(int j) {
  const int r = EXT + 2 * QG * j - (QG == 2 ? 7 : 4);
  return r > 0 ? r : 0;
}

template <bool DENSE, int QG>
__global__ __attribute__((amdgpu_flat_work_group_size(256 / QG, 256 / QG), amdgpu_waves_per_eu(3 - QG, 3 - QG)))
void attn_bf16_kernel(AttnArgs a, const int32_t* __restrict__ kidx, const int32_t* __restrict__ kcnt,
                      const uint8_t* __restrict__ sel, const bf16* __restrict__ Q, bf16* __restrict__ O,
                      const int32_t* __restrict__ order, int32_t* __restrict__ counter) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kVRing];
  __shared__ int item_s;

  // QG 32-query groups per wave: 4 / QG waves of 32 * QG queries; every wave copies 8 * QG rows of each tile
  constexpr int kWaves = 4 / QG, kThreads = 64 * kWaves, kQW = 32 * QG, kWaveRows = 8 * QG;
  constexpr int kDmaK = 2 * QG, kDmaStep = 4 * QG;   // per wave: copies of one K (V) tile, of one step
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int rows = a.heads * a.nq;
  // Persistent: the grid is sized to the resident workgroups. attn_order_kernel sorts the rows longest key list
  // first and deals every wave of gridDim.x of them by XCD (re-sorted by row id, XCD x holds positions x, x + 8, ..
  // of the wave: one contiguous row range, whose key lists overlap). Workgroup b starts on position b of the first
  // wave; after that it takes the next position of its XCD's queue (positions x, x + 8, .. of the first wave, then
  // of the second, ...) and, once that queue is empty, of the other XCDs' queues in turn. So the long rows start
  // early, the rows running together on one XCD share key blocks in its L2, and the short ones balance the tail.
  bool first_item = true;
  for (;;) {
  int item;
  if (first_item) {
    item = blockIdx.x;
    first_item = false;
  } else {
    if (tid == 0) item_s = next_dealt_item(counter, rows);
    __syncthreads();
    item = item_s;
    __syncthreads();
  }
  if (item >= rows) break;
  const int row_id = order[item];
  const int h = row_id / a.nq, qb = row_id - h * a.nq;
  const int hc = h * kHeadDim;
  const int cnt = kcnt[row_id];

  if (cnt <= 0) {   // empty query block -> zeros (SparseAttention.swift:47-53; DiT.swift:300-304)
    for (int e = tid; e < kBlock * 16; e += kThreads) {
      const int64_t row = (int64_t)qb * kBlock + (e >> 4);
      if (row < a.lq) *(u32x4*)(O + a.out_row(row) * a.ld + hc + (e & 15) * 8) = u32x4{0, 0, 0, 0};
    }
    continue;
  }
  const int32_t* __restrict__ klist = kidx + (int64_t)row_id * a.nk_stride;
  const uint8_t* __restrict__ srow = DENSE ? sel + (int64_t)row_id * a.nk : nullptr;
  const int nblocks = DENSE ? a.nk : min(cnt, a.nk_stride);

  // Q as the B operand of S^T = K Q^T (the bf16 inputs as they are; the scale c is applied to the fp32 scores):
  // group q holds queries qb*128 + kQW*wave + 32*q + l32, lane (query, k-half g) dims 16t + 8g .. +7
  bf16x8 qop[QG][8];
#pragma unroll
  for (int q = 0; q < QG; ++q) {
    const int64_t qrow = (int64_t)qb * kBlock + wave * kQW + q * 32 + l32;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      bf16x8 x = bf16x8{};
      if (qrow < a.lq) x = *(const bf16x8*)(Q + qrow * a.ld + hc + 16 * t + 8 * g);
      qop[q][t] = x;
    }
  }

  // tile loads: the buffer spans the physical K/V rows; a row past it reads as 0, so a ragged last block, a listed
  // index outside [0, nk) and the tiles past the end of the walk load zeros without per-lane guards. K/V rows are
  // token-major (head h's 128 channels at 256 h bytes of each row) or head-major (a KV ring: head h's rows from
  // h * kv_head_stride on, 256 bytes each; every block whole, so no row past a head's region is read)
  const uint32_t row_bytes = (uint32_t)a.kv_ld * 2;
  const uint32_t range = (uint32_t)a.kv_bytes;
  const int head_off = (int)(h * a.kv_head_stride * 2);
  const u32x4 krs = buffer_rsrc(a.k, range), vrs = buffer_rsrc(a.v, range);
  // a DMA load writes 1 KB of LDS (lane i -> bytes 16i..16i+15) = 4 rows; wave w fills rows kWaveRows * w ..
  int voff_k[kDmaK], voff_v[kDmaK];
#pragma unroll
  for (int p = 0; p < kDmaK; ++p) {
    const int r = wave * kWaveRows + 4 * p + (lane >> 4), pos = lane & 15;
    voff_k[p] = r * (int)row_bytes + head_off + ((pos ^ swz_k(r)) << 4);
    voff_v[p] = r * (int)row_bytes + head_off + ((pos ^ swz_v(r)) << 4);
  }
  const uint32_t smem_lds = lds_addr(smem);
  const uint32_t dma_base = smem_lds + wave * kWaveRows * kRowBytes;
  // buffer byte offset of block j's first row (j outside [0, nk): past the buffer -> zeros)
  auto block_soff = [&](int j) -> int {
    return (unsigned)j < (unsigned)a.nk ? (int)(a.map.row(j) * row_bytes) : (int)range;
  };
  const int sub_bytes = kTileKeys * (int)row_bytes;   // 32 rows
  // K / V of quarter SUB of the block at soff into ring slot SLOT
  auto issue_k = [&](auto slot_c, int soff) {
    constexpr int SLOT = decltype(slot_c)::value;
    static_for<0, kDmaK>([&](auto p_c) {
      constexpr int P = decltype(p_c)::value;
      dma16<SLOT * kTileBytes + P * 4 * kRowBytes>(krs, dma_base, voff_k[P], soff);
    });
  };
  auto issue_v = [&](auto slot_c, int soff) {
    constexpr int SLOT = decltype(slot_c)::value;
    static_for<0, kDmaK>([&](auto p_c) {
      constexpr int P = decltype(p_c)::value;
      dma16<kVRing + SLOT * kTileBytes + P * 4 * kRowBytes>(vrs, dma_base, voff_v[P], soff);
    });
  };
  // one of the kDmaK copies (rows 4P .. 4P+3 of this wave's share) of K / V into ring slot SLOT
  auto dma_k = [&](auto slot_c, auto p_c, int soff) {
    constexpr int SLOT = decltype(slot_c)::value, P = decltype(p_c)::value;
    dma16<SLOT * kTileBytes + P * 4 * kRowBytes>(krs, dma_base, voff_k[P], soff);
  };
  auto dma_v = [&](auto slot_c, auto p_c, int soff) {
    constexpr int SLOT = decltype(slot_c)::value, P = decltype(p_c)::value;
    dma16<kVRing + SLOT * kTileBytes + P * 4 * kRowBytes>(vrs, dma_base, voff_v[P], soff);
  };
  // walked block b: buffer offset of its first row (past the buffer past the end of the walk) and its keys taking
  // part (0 if unselected in the dense walk or outside [0, nk); else up to 128, fewer for a ragged last block)
  // A walked block's entry e: its key block index (sparse walk) or its selection byte (dense walk), -1 past the
  // end. The loop loads each entry one block before it derives the offset and key count from it, so the load's
  // wait is covered by the waits of the steps in between.
  auto walk_entry = [&](int b) -> int { return b < nblocks ? (DENSE ? (int)srow[b] : klist[b]) : -1; };
  auto entry_soff = [&](int b, int e) -> int { return b < nblocks ? block_soff(DENSE ? b : e) : (int)range; };
  auto entry_keys = [&](int b, int e) -> int {
    if (b >= nblocks) return 0;
    const int j = DENSE ? b : e;
    if ((unsigned)j >= (unsigned)a.nk || (DENSE && e == 0)) return 0;
    return (int)min<int64_t>(kBlock, a.lk - (int64_t)j * kBlock);
  };
  auto walk_soff = [&](int b) -> int { return entry_soff(b, walk_entry(b)); };
  auto walk_keys = [&](int b) -> int { return entry_keys(b, walk_entry(b)); };
  auto sub_valid = [&](int keys, int sub) -> int { return min(max(keys - sub * kTileKeys, 0), kTileKeys); };

  // LDS operand addresses within a slot. K: row l32, chunk 2t+g. V^T (ds_read_b64_tr_b16): 16-lane group G, member
  // mm reads row 16u + 8ab + 4(G/2) + mm/4, bf16 columns 32dt + 16(G%2) + 4(mm%4) .. +3.
  int k_off[8], v_off[4];
#pragma unroll
  for (int t = 0; t < 8; ++t) k_off[t] = l32 * kRowBytes + (((2 * t + g) ^ swz_k(l32)) << 4);
  const int G = lane >> 4, mm = lane & 15;
  const int vr = 4 * (G >> 1) + (mm >> 2);   // + 16u + 8ab: the swizzle depends on the row mod 4 only
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    v_off[dt] = vr * kRowBytes + (((4 * dt + 2 * (G & 1) + ((mm & 3) >> 1)) ^ swz_v(vr)) << 4) + (mm & 1) * 8;

  f32x16 acc[QG][4];
  float l_run[QG], m_row[QG], part_max[QG], m_ref[QG], negm[QG];
  constexpr float kNoKey = -1e29f;   // a raw row max below this saw masked keys only
  const float c_scale = a.c;         // softmax scale * log2(e)
  // the reference (log2 units, fp32) of each query row: P = exp2(c S - m), one v_fma per score
  auto set_ref = [&](int q, float m) {
    m_ref[q] = m;
    negm[q] = -m;
  };
  // the reference of a raw row max (masked keys only: 0)
  auto ref_of = [&](float mx) -> float { return mx > kNoKey ? mx * c_scale : 0.f; };
  // the extra MFMA step, a v_mfma_f32_32x32x8_bf16 (k = 8, half the cost of a k = 16 step): A lane (key l32, g = 0)
  // holds k-slot {masked}, B lane (query, g = 0) {-2^100}, all other k-slots 0: keys that do not take part score
  // -2^100 and their exponentials are exactly 0
  i16x4 bext;
  {
    bf16x4 b = bf16x4{};
    if (g == 0) b[0] = (bf16)kMaskedScore;
    bext = __builtin_bit_cast(i16x4, b);
  }
  auto aext = [&](int valid) -> i16x4 {
    bf16x4 x = bf16x4{};
    if (g == 0) x[0] = l32 >= valid ? (bf16)1.0f : (bf16)0.0f;
    return __builtin_bit_cast(i16x4, x);
  };
  auto mfma_ext = [&](const i16x4& ax, const i16x4& bx) -> f32x16 {
    return __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(ax, bx, f32x16{}, 0, 0, 0);
  };
  // The sparse walk lists selected blocks only, so its tiles are whole (32 keys) but for a ragged last block, a listed
  // index outside [0, nk) and the tile past the end of the walk, whose rows all load as zeros. It starts S at zero
  // (no mask MFMA) and, on a tile with fewer than 32 keys taking part (a wave-uniform branch), sets the scores of the
  // keys at or past `valid` to -2^100 afterwards: the values the mask MFMA gives there (their K rows are zeros).
  // Lane element i of a 32 x 32 MFMA result is key row 8 (i / 4) + 4 g + i % 4.
  auto mask_tile = [&](f32x16& s, int valid) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 8 * (i >> 2) + 4 * g + (i & 3) >= valid ? kMaskedScore : s[i];
  };
  // mask MFMAs per step: the dense walk's tiles mix selected and unselected blocks
  constexpr int kExt = DENSE ? QG : 0;
  lds_char* const lds = (lds_char*)(uintptr_t)smem_lds;
  // S^T = K Q^T (keys that do not take part: - 2^100) for both groups, K from ring slot SLOT
  auto qk = [&](auto slot_c, int valid, f32x16 (&s)[QG]) {
    constexpr int SLOT = decltype(slot_c)::value;
    bf16x8 kk[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) kk[t] = *(const lds_bf16x8*)(lds + SLOT * kTileBytes + k_off[t]);
    if constexpr (DENSE) {
      const i16x4 ax = aext(valid);
#pragma unroll
      for (int q = 0; q < QG; ++q) s[q] = mfma_ext(ax, bext);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int q = 0; q < QG; ++q)
        s[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kk[t], qop[q][t], (DENSE || t > 0) ? s[q] : f32x16{}, 0, 0, 0);
    if (!DENSE && valid < kTileKeys) {
#pragma unroll
      for (int q = 0; q < QG; ++q) mask_tile(s[q], valid);
    }
  };
  // O^T += V^T P^T, V from ring slot SLOT
  auto pv = [&](auto slot_c, const bf16x8 (&p)[QG][2]) {
    constexpr int SLOT = decltype(slot_c)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        lds_char* const pa = lds + kVRing + SLOT * kTileBytes + v_off[dt] + 16 * u * kRowBytes;
        const i16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)pa);
        const i16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pa + 8 * kRowBytes));
        // whole-vector concatenation: element-wise assembly of the operand is mis-lowered (one dword duplicated)
        const bf16x8 vv = __builtin_bit_cast(bf16x8, __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int q = 0; q < QG; ++q)
          mfma_acc(acc[q][dt], vv, p[q][u]);
      }
  };
  auto row_max = [&](const f32x16& s) -> float {
    // plain fmaxf, not v_max3 in inline asm: s comes straight from an MFMA (VGPR form), and the compiler inserts the
    // MFMA -> VALU wait states only for instructions it can see
    float mx = fmaxf(s[0], s[1]);
#pragma unroll
    for (int r = 2; r < 15; r += 2) mx = fmaxf(mx, fmaxf(s[r], s[r + 1]));
    return pair_max(fmaxf(mx, s[15]));
  };
  // all of this wave's copies but the last `keep` steps' have landed, and every wave is past its LDS reads
  auto sync_steps = [&](int keep) {
    if (keep >= 2) FVSR_WAIT_VM_LGKM0(2 * kDmaStep);
    else if (keep == 1) FVSR_WAIT_VM_LGKM0(kDmaStep);
    else FVSR_WAIT_VM_LGKM0(0);
    __builtin_amdgcn_s_barrier();
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  using C3 = std::integral_constant<int, 3>;

  // One pass over the key tiles. MODE 0 (main): the reference m := the exact row max of the first tile (0 if it
  // has no valid key), then P = exp2(S - m); the largest partial row sum is tracked. MODE 1: row max only. MODE 2:
  // attention with m fixed to the exact row max.
  // Step T (tile T = 4b + sub, ring slot = sub): request K(T+4) and V(T+2); S(T+1) = QK(T+1); O += PV(T-1);
  // exponentials of S(T); then K(T+2) and V(T) must have landed (requested at step T-2).
  auto run = [&](auto mode_c) {
    constexpr int MODE = decltype(mode_c)::value;
#pragma unroll
    for (int q = 0; q < QG; ++q) {
      l_run[q] = 0.f;
      part_max[q] = 0.f;
#pragma unroll
      for (int d = 0; d < 4; ++d) acc[q][d] = f32x16{};
      set_ref(q, MODE == 2 ? m_row[q] : 0.f);
      if (MODE == 1) m_row[q] = kMaskedScore;
    }
    f32x16 sA[QG], sB[QG];
    bf16x8 pA[QG][2], pB[QG][2];
    // per walked block: first-row buffer offset and keys taking part, read two blocks ahead of use
    int o0 = walk_soff(0), o1 = walk_soff(1), o2 = walk_soff(2);
    int n0 = walk_keys(0), n1 = walk_keys(1), n2 = walk_keys(2);
    int e3 = walk_entry(3);
    if (MODE == 0 && DENSE) {
      // the reference comes from the tile the sparse walk starts with (the first tile of the first listed block),
      // so both walks do the same arithmetic on every selected tile and agree bit for bit
      const int jr = klist[0];
      issue_k(C0{}, block_soff(jr));
      FVSR_WAIT_VM_LGKM0(0);
      __builtin_amdgcn_s_barrier();
      qk(C0{}, (unsigned)jr < (unsigned)a.nk ? sub_valid((int)min<int64_t>(kBlock, a.lk - (int64_t)jr * kBlock), 0)
                                             : 0,
         sA);
#pragma unroll
      for (int q = 0; q < QG; ++q) set_ref(q, ref_of(row_max(sA[q])));
      __builtin_amdgcn_s_barrier();   // every wave is done with K slot 0 before the walk refills it
    }
    // prologue = virtual steps -4 .. -1: K(0..3) and V(-2..1); V(-2), V(-1) are zeros, so step 0's PV of the
    // (zero) previous P adds exact zeros
    issue_k(C0{}, o0);                issue_v(C2{}, (int)range);
    issue_k(C1{}, o0 + sub_bytes);    issue_v(C3{}, (int)range);
    issue_k(C2{}, o0 + 2 * sub_bytes); issue_v(C0{}, o0);
    issue_k(C3{}, o0 + 3 * sub_bytes); issue_v(C1{}, o0 + sub_bytes);
    sync_steps(3);   // K(0) landed
    qk(C0{}, sub_valid(n0, 0), sA);
    if (MODE == 0 && !DENSE) {
      // reference = the exact row max of tile 0 (scaled), as the dense walk's pre-step computes it
#pragma unroll
      for (int q = 0; q < QG; ++q) set_ref(q, ref_of(row_max(sA[q])));
    }
#pragma unroll
    for (int q = 0; q < QG; ++q)
#pragma unroll
      for (int u = 0; u < 2; ++u) pB[q][u] = bf16x8{};
    sync_steps(1);   // K(1), K(2), V(-1), V(0) landed
    // the first LDS operands of a step (K chunk 0 of its QK tile, V^T pair 0 of its PV tile) are read at the end of
    // the step before it, so no operand read sits between the step's barrier and its first MFMA; for step 0:
    // K(1) in slot 1, V(-1) in slot 3
    bf16x8 hk;
    i16x4 hva, hvb;
    auto read_first = [&](auto kslot_c, auto vslot_c) {
      constexpr int KSL = decltype(kslot_c)::value, VSL = decltype(vslot_c)::value;
      lds_char* const pa = lds + kVRing + VSL * kTileBytes + v_off[0];
      hva = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)pa);
      hvb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pa + 8 * kRowBytes));
      hk = *(const lds_bf16x8*)(lds + KSL * kTileBytes + k_off[0]);
    };
    if (MODE != 1) read_first(C1{}, C3{});

    // step with tile T in ring slot SUB: K(T+4) -> slot SUB, V(T+2) -> slot SUB+2, QK(T+1) <- K slot SUB+1,
    // PV(T-1) <- V slot SUB+3 (all mod 4)
    auto step = [&](auto sub_c, int valid_next, int soff_k, int soff_v, f32x16 (&s_cur)[QG], f32x16 (&s_nxt)[QG],
                    bf16x8 (&p_prev)[QG][2], bf16x8 (&p_cur)[QG][2], auto&& pre_sync) {
      constexpr int SUB = decltype(sub_c)::value;
      using KS = std::integral_constant<int, SUB>;
      using VS = std::integral_constant<int, (SUB + 2) & 3>;
      if (MODE == 1) {
        issue_k(KS{}, soff_k);
        issue_v(VS{}, soff_v);
        qk(std::integral_constant<int, (SUB + 1) & 3>{}, valid_next, s_nxt);
#pragma unroll
        for (int q = 0; q < QG; ++q) m_row[q] = fmaxf(m_row[q], row_max(s_cur[q]));
      } else {
        // 16 * QG micro-rounds with one MFMA each (17 * QG in the dense walk), fenced so the order below is the
        // issue order, then one more for the last exponential. A wave issues in order and an MFMA occupies the
        // matrix core for 32 cycles: every MFMA is followed by a slice of the other work, which issues while it runs
        // (MFMAs grouped back to back would leave that work unoverlapped). MFMA order: (dense walk) the mask MFMA of
        // QK(T+1) for each query group, then for c = 0..7 QK chunk c (each group) and PV pair c (each group).
        // Slices: exponential I of S(T) in micro-round I (pairs packed to bf16 and summed a micro-round later); the
        // LDS operands of chunk / pair j requested up to 4 micro-rounds before use (attn_read_at); one of the step's
        // buffer->LDS copies every 4 micro-rounds.
        lds_char* const vbase = lds + kVRing + ((SUB + 3) & 3) * kTileBytes;
        lds_char* const kbase = lds + ((SUB + 1) & 3) * kTileBytes;
        i16x4 va[8], vb[8];
        bf16x8 kk[8];
        // operands of QK chunk j and PV pair j: K chunk j and V^T pair j
        auto read_ops = [&](int j) {
          if (j == 0) {   // read at the end of the step before
            va[0] = hva;
            vb[0] = hvb;
            kk[0] = hk;
            return;
          }
          lds_char* const pa = vbase + v_off[j & 3] + 16 * (j >> 2) * kRowBytes;
          va[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)pa);
          vb[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pa + 8 * kRowBytes));
          kk[j] = *(const lds_bf16x8*)(kbase + k_off[j]);
        };
        auto dma = [&](auto r_c) {
          constexpr int R = decltype(r_c)::value;
          if constexpr (R < kDmaK) dma_k(KS{}, std::integral_constant<int, R>{}, soff_k);
          else dma_v(VS{}, std::integral_constant<int, R - kDmaK>{}, soff_v);
        };
        i16x4 ax{};
        if constexpr (DENSE) ax = aext(valid_next);
        float sum[QG][2];
        float xv[2];   // the exponentials of the last two micro-rounds
        auto micro = [&](auto i_c) {
          constexpr int I = decltype(i_c)::value;
          if constexpr (I == 0) {
            read_ops(0);
            read_ops(1);
          }
          static_for<2, 8>([&](auto j_c) {
            constexpr int J = decltype(j_c)::value;
            if constexpr (attn_read_at<QG, kExt>(J) == I) read_ops(J);
          });
          if constexpr (I < kExt) {
            s_nxt[I] = mfma_ext(ax, bext);
          } else if constexpr (I < kExt + 16 * QG) {
            constexpr int c = (I - kExt) / (2 * QG), w = (I - kExt) % (2 * QG);
            if constexpr (w < QG) {
              if constexpr (DENSE || c > 0)
                s_nxt[w] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kk[c], qop[w][c], s_nxt[w], 0, 0, 0);
              else
                s_nxt[w] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kk[0], qop[w][0], f32x16{}, 0, 0, 0);
            } else {
              // whole-vector concatenation: element-wise assembly of the operand is mis-lowered (one dword
              // duplicated)
              const bf16x8 vv =
                  __builtin_bit_cast(bf16x8, __builtin_shufflevector(va[c], vb[c], 0, 1, 2, 3, 4, 5, 6, 7));
              mfma_acc(acc[w - QG][c & 3], vv, p_prev[w - QG][c >> 2]);
            }
          }
          // exponential I of S(T) (entry idx of group q); the exponential of the micro-round before is summed (fp32
          // sums: v_dot2 would wait for the matrix core) and, completing a pair, packed to bf16 here, a micro-round
          // after it was issued, so no wait state follows the transcendental
          if constexpr (I >= 1 && I <= 16 * QG) {
            constexpr int J = I - 1, qj = J >> 4, ij = J & 15;
            if constexpr (ij < 2) sum[qj][ij] = xv[J & 1];
            else sum[qj][ij & 1] += xv[J & 1];
            if constexpr ((J & 1) == 1) {
              p_cur[qj][ij >> 3][(ij & 7) - 1] = (bf16)xv[0];
              p_cur[qj][ij >> 3][ij & 7] = (bf16)xv[1];
              // the pair is packed here, in this micro-round: without a use before the reference check the
              // compiler sinks the packs past it (the raise recomputes them) into the step's tail
              const u32x4 pw = __builtin_bit_cast(u32x4, p_cur[qj][ij >> 3]);
              asm volatile("" ::"v"(pw[(ij & 7) >> 1]));
            }
          }
          if constexpr (I < 16 * QG) {
            constexpr int q = I >> 4, idx = I & 15;
            xv[I & 1] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[q][idx], c_scale, negm[q]));
          }
          if constexpr ((I & 3) == 1 && I / 4 < kDmaStep) dma(std::integral_constant<int, I / 4>{});
          if constexpr (I == kExt + 16 * QG - (DENSE ? 1 : 0))
            read_first(std::integral_constant<int, (SUB + 2) & 3>{}, std::integral_constant<int, SUB>{});
          __builtin_amdgcn_sched_barrier(0);
        };
        static_for<0, kExt + 16 * QG + (DENSE ? 0 : 1)>(micro);
        float part[QG];
        bool grow = false;
#pragma unroll
        for (int q = 0; q < QG; ++q) {
          part[q] = sum[q][0] + sum[q][1];
          grow |= !(part[q] <= kGrowSum);   // either half of a row; also inf / NaN
        }
        if (__ballot(grow) != 0) {
          // raise the reference of the rows that grew to their max in S(T); the other rows keep theirs (their
          // scale is 1 and every operation below is exact and changes nothing)
          acc_drain();
#pragma unroll
          for (int q = 0; q < QG; ++q) {
            const bool gq = !(pair_max(part[q]) <= kGrowSum);
            const float m_new = gq ? row_max(s_cur[q]) * c_scale : m_ref[q];
            const float sc = __builtin_amdgcn_exp2f(m_ref[q] - m_new);
            set_ref(q, m_new);
            float t[2] = {0.f, 0.f};
#pragma unroll
            for (int idx = 1; idx < 16; idx += 2) {
              const float x0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[q][idx - 1], c_scale, negm[q]));
              const float x1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[q][idx], c_scale, negm[q]));
              p_cur[q][idx >> 3][(idx & 7) - 1] = (bf16)x0;
              p_cur[q][idx >> 3][idx & 7] = (bf16)x1;
              t[(idx >> 1) & 1] += x0 + x1;
            }
            part[q] = t[0] + t[1];
            l_run[q] *= sc;
            part_max[q] *= sc;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
              for (int i = 0; i < 16; ++i) acc[q][dt][i] *= sc;
          }
        }
#pragma unroll
        for (int q = 0; q < QG; ++q) {
          l_run[q] += part[q];
          part_max[q] = fmaxf(part_max[q], part[q]);
        }
        // last in the step: a branch before the row sums would let the compiler sink the exponentials past it
        if (!DENSE && valid_next < kTileKeys) {
#pragma unroll
          for (int q = 0; q < QG; ++q) mask_tile(s_nxt[q], valid_next);
        }
      }
      // keep every instruction of this step on its side of the barrier; the copies of the step before have landed
      // (the next step's first operands, read above, were waited for one step earlier)
      __builtin_amdgcn_sched_barrier(0);
      pre_sync();
      sync_steps(1);
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int b = 0; b < nblocks; ++b) {
      const int o3 = entry_soff(b + 3, e3), n3 = entry_keys(b + 3, e3);
      // step 4b+s: QK tile 4b+s+1, K tile 4b+s+4 (block b+1), V tile 4b+s+2
      auto nop = [] {};
      step(C0{}, sub_valid(n0, 1), o1, o0 + 2 * sub_bytes, sA, sB, pB, pA, nop);
      step(C1{}, sub_valid(n0, 2), o1 + sub_bytes, o0 + 3 * sub_bytes, sB, sA, pA, pB, nop);
      step(C2{}, sub_valid(n0, 3), o1 + 2 * sub_bytes, o1, sA, sB, pB, pA, nop);
      // the next block's list entry loads right before the step's wait, which absorbs it
      step(C3{}, sub_valid(n1, 0), o1 + 3 * sub_bytes, o1 + sub_bytes, sB, sA, pA, pB,
           [&] { e3 = walk_entry(b + 4); });
      o0 = o1; o1 = o2; o2 = o3;
      n0 = n1; n1 = n2; n2 = n3;
    }
    if (MODE != 1) {
      pv(C3{}, pB);   // PV of the last tile (4 * nblocks - 1, slot 3)
      acc_drain();
    }
    // drain the zero-fill copies requested past the end before LDS is reused
    FVSR_WAIT_VM_LGKM0(0);
    __builtin_amdgcn_s_barrier();
  };

  run(std::integral_constant<int, 0>{});
  // rows whose exponentials all underflowed (the reference came from a tile with no valid key and every score is
  // far below it): redo the workgroup exactly (row max pass, then attention with that max); workgroup-uniform so the
  // barriers match
  {
    bool bad = false;
#pragma unroll
    for (int q = 0; q < QG; ++q) bad |= !(pair_max(part_max[q]) >= 2.3283064e-10f);
    int* flag = (int*)smem;
    if (tid == 0) flag[0] = 0;
    __syncthreads();
    if (__ballot(bad) != 0 && lane == 0) flag[0] = 1;
    __syncthreads();
    const bool redo = flag[0] != 0;
    __syncthreads();
    if (redo) {
      run(std::integral_constant<int, 1>{});
#pragma unroll
      for (int q = 0; q < QG; ++q) m_row[q] = ref_of(m_row[q]);
      run(std::integral_constant<int, 2>{});
    }
  }

#pragma unroll
  for (int q = 0; q < QG; ++q) {
    const float l = pair_sum(l_run[q]);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t qrow = (int64_t)qb * kBlock + wave * kQW + q * 32 + l32;
    if (qrow < a.lq) {
      bf16* orow = O + a.out_row(qrow) * a.ld + hc;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          bf16x4 ov;
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[e] = (bf16)(acc[q][dt][4 * r4 + e] * inv);
          *(bf16x4*)(orow + 32 * dt + 8 * r4 + 4 * g) = ov;
        }
    }
  }
  }   // next row
}

// Rows (head, query block) for the persistent bf16 walk, and the per-XCD queue counters. One workgroup. First a
// counting sort by decreasing key-list length in 255 bins of ceil(longest / 255) blocks (exact lengths up to 255
// blocks; the dense walk: every non-empty row is a full walk). Then every wave of `grid` consecutive items of that order (one
// item per workgroup) is re-sorted by row id (head-major, neighbouring query blocks together) and dealt so that XCD x
// (workgroups b with b % 8 == x, dispatch is round-robin over the XCDs) holds positions x, x + 8, .. of the wave:
// one contiguous range of rows, whose key lists overlap, so the XCD's L2 serves the key blocks they share.
// next_dealt_item hands the positions out per XCD. The order does not affect results. Scans are wave-wide
// (shuffles) with one step across the waves. Up to kOrderLdsRows rows the lengths' bins and the sorted order stay in
// LDS (kcnt is read once, the dealt order written once) and, while the waves' bitmaps fit together, every wave is
// ranked in one pass (one bitmap segment per wave, one scan); beyond, the sorted order is staged in `order` itself
// and the waves are ranked one after another. When every list has the same length the row-id order is such an order
// already and is dealt as it stands.
constexpr int kOrderLdsRows = 8192;
__global__ __launch_bounds__(1024) void attn_order_kernel(const int32_t* __restrict__ kcnt, int rows, int nk_stride,
                                                          int dense, int grid, int32_t* __restrict__ order,
                                                          int32_t* __restrict__ counters) {
  constexpr int kBins = 256;
  constexpr int kWords = 4096;   // row-id bitmap words: the bitmap rank serves up to 32 x 4096 rows
  __shared__ int bin_start[kBins];
  __shared__ int wtot[16];
  __shared__ __attribute__((aligned(16))) int first[kMaxPersistentWgs];   // one wave; padded with INT_MAX
  __shared__ unsigned bm[kWords];
  __shared__ int wpre[kWords];                                            // set bits in the words before word w
  __shared__ int lord[kOrderLdsRows];                                     // the sorted order (rows <= kOrderLdsRows)
  __shared__ uint8_t lbin[kOrderLdsRows];                                 // each row's bin (rows <= kOrderLdsRows)
  __shared__ int s_longest, s_mixed;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool in_lds = rows <= kOrderLdsRows;
  int* const sorted = in_lds ? lord : order;
  if (tid < kBins) bin_start[tid] = 0;
  if (tid == 0) {
    s_longest = 0;
    s_mixed = 0;
  }
  __syncthreads();
  auto list_len = [&](int r) -> int { return max(0, min(kcnt[r], nk_stride)); };
  // the longest list, and whether the lengths differ at all (the lengths wait in lord until the sort overwrites it);
  // a thread's loads are issued together, so their latencies overlap
  {
    const int c0 = list_len(0);
    int m = 0;
    bool mixed = false;
    for (int r0 = tid; r0 < rows; r0 += 4 * 1024) {
      int c[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) c[u] = list_len(min(r0 + u * 1024, rows - 1));   // loads without branches
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (r0 + u * 1024 < rows) {
          if (in_lds) lord[r0 + u * 1024] = c[u];
          m = max(m, c[u]);
          mixed |= c[u] != c0;
        }
      }
    }
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o));
    if (lane == 0) atomicMax(&s_longest, m);
    if (__ballot(mixed) != 0 && lane == 0) s_mixed = 1;
  }
  __syncthreads();
  // every list of one length (the cross-attention's and the dense fallback's lists): the row-id order is already
  // sorted by length and each of its waves by row id, so the sort and the ranking are skipped and the rows are dealt
  // where they stand
  const bool one_len = s_mixed == 0;
  if (!one_len) {
    const int width = max(1, (s_longest + kBins - 2) / (kBins - 1));   // blocks per bin
    auto bin_len = [&](int c) -> int {   // bin 0 = the longest lists
      const int len = c <= 0 ? 0 : (dense ? 1 : min((c + width - 1) / width, kBins - 1));
      return kBins - 1 - len;
    };
    auto bin_of = [&](int r) -> int { return bin_len(list_len(r)); };
    for (int r = tid; r < rows; r += 1024) {
      const int bn = in_lds ? bin_len(lord[r]) : bin_of(r);
      if (in_lds) lbin[r] = (uint8_t)bn;
      atomicAdd(&bin_start[bn], 1);
    }
    __syncthreads();
    // exclusive scan of the 256 bin counts by waves 0..3
    {
      const int v = tid < kBins ? bin_start[tid] : 0;
      const int incl = (int)wave_incl_scan((unsigned)v);
      if (tid < kBins && lane == 63) wtot[wave] = incl;
      __syncthreads();
      if (tid < kBins) {
        int base = 0;
        for (int w = 0; w < wave; ++w) base += wtot[w];
        bin_start[tid] = base + incl - v;
      }
    }
    __syncthreads();
    for (int r = tid; r < rows; r += 1024) sorted[atomicAdd(&bin_start[in_lds ? (int)lbin[r] : bin_of(r)], 1)] = r;
  }
  __threadfence_block();
  __syncthreads();
  grid = min(grid, kMaxPersistentWgs);
  // position p of the sorted order goes to wave p / grid; XCD x holds m_x = (nw - x + 7) / 8 positions x, x + 8, ..
  // of a wave of nw items, and ranks s_x .. s_x + m_x - 1 (by row id) go to it
  auto deal = [&](int w0, int nw, int rank, int r) {
    int x = 0, s0 = 0;
    while (s0 + (nw - x + kXcds - 1) / kXcds <= rank) {
      s0 += (nw - x + kXcds - 1) / kXcds;
      ++x;
    }
    order[w0 + (rank - s0) * kXcds + x] = r;
  };
  // exclusive scan of the popcounts of bm[0 .. n) into wpre (4 words per thread, n <= kWords)
  auto scan_words = [&](int n) {
    int c[4], csum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = 4 * tid + i;
      c[i] = w < n ? __popc(bm[w]) : 0;
      csum += c[i];
    }
    const int incl = (int)wave_incl_scan((unsigned)csum);
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    int run = incl - csum;
    for (int w = 0; w < wave; ++w) run += wtot[w];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (4 * tid + i < n) wpre[4 * tid + i] = run;
      run += c[i];
    }
    __syncthreads();
  };
  const int rwords = (rows + 31) / 32;
  const int nwaves = (rows + grid - 1) / grid;
  if (one_len) {
    for (int p = tid; p < rows; p += 1024) {
      const int w0 = p / grid * grid;
      deal(w0, min(grid, rows - w0), p - w0, p);
    }
  } else if (in_lds && nwaves * rwords <= kWords) {
    // every wave at once: wave w's rows set their bits in bitmap segment w, one scan covers all segments
    for (int i = tid; i < nwaves * rwords; i += 1024) bm[i] = 0u;
    __syncthreads();
    for (int p = tid; p < rows; p += 1024) {
      const int r = sorted[p];
      atomicOr(&bm[(p / grid) * rwords + (r >> 5)], 1u << (r & 31));
    }
    __syncthreads();
    scan_words(nwaves * rwords);
    for (int p = tid; p < rows; p += 1024) {
      const int r = sorted[p], w = p / grid, wi = w * rwords + (r >> 5);
      const int rank = wpre[wi] - wpre[w * rwords] + __popc(bm[wi] & ((1u << (r & 31)) - 1u));
      deal(w * grid, min(grid, rows - w * grid), rank, r);
    }
  } else {
    const bool use_bitmap = rows <= kWords * 32;
    const int words = use_bitmap ? rwords : 0;
    for (int w0 = 0; w0 < rows; w0 += grid) {
      const int nw = min(grid, rows - w0);
      for (int i = tid; i < kMaxPersistentWgs; i += 1024) first[i] = i < nw ? sorted[w0 + i] : 0x7fffffff;
      for (int w = tid; w < words; w += 1024) bm[w] = 0u;
      __syncthreads();
      // rank of each row of the wave among them by row id: a bitmap over the row ids and a scan of its per-word
      // popcounts; beyond 32 x 4096 rows, a scan of the wave's rows themselves
      if (use_bitmap) {
        for (int i = tid; i < nw; i += 1024) atomicOr(&bm[first[i] >> 5], 1u << (first[i] & 31));
        __syncthreads();
        scan_words(words);
      }
      const int n4 = (nw + 31) / 32 * 8;   // int4 groups to scan, a multiple of the unroll
      for (int i = tid; i < nw; i += 1024) {
        const int r = first[i];
        int rank = 0;   // rows are distinct: ranks are a permutation of 0 .. nw - 1
        if (use_bitmap) {
          rank = wpre[r >> 5] + __popc(bm[r >> 5] & ((1u << (r & 31)) - 1u));
        } else {
#pragma unroll 8
          for (int j = 0; j < n4; ++j) {
            const int4 f = reinterpret_cast<const int4*>(first)[j];
            rank += (f.x < r) + (f.y < r) + (f.z < r) + (f.w < r);
          }
        }
        deal(w0, nw, rank, r);
      }
      __syncthreads();
    }
  }
  // queue y's counter starts past the first wave (the workgroups take it without the counters)
  if (tid < kXcds) counters[8 * tid] = (grid - tid + kXcds - 1) / kXcds;
}

// ------------------------------------------------------------------------------------------------------------
// fp32 (parity lane)
// ------------------------------------------------------------------------------------------------------------
template <bool DENSE>
__global__ __launch_bounds__(256) void attn_f32_kernel(AttnArgs a) {
  constexpr int BK = 32;          // keys per tile
  constexpr int LDR = 132;        // padded fp32 row stride (floats): conflict-free operand reads
  constexpr int TILE = BK * LDR;  // floats per tile
  __shared__ __attribute__((aligned(16))) float smem[2 * 2 * TILE];

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int h = lid / a.nq, qb = lid - h * a.nq;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int hc = h * kHeadDim;
  const float* __restrict__ Q = (const float*)a.q;
  const float* __restrict__ K = (const float*)a.k;
  const float* __restrict__ V = (const float*)a.v;
  float* __restrict__ O = (float*)a.o;
  const int row_id = h * a.nq + qb;
  const int cnt = a.kcnt[row_id];

  if (cnt <= 0) {
    for (int e = tid; e < kBlock * 32; e += 256) {
      const int64_t row = (int64_t)qb * kBlock + (e >> 5);
      if (row < a.lq) *(f32x4*)(O + a.out_row(row) * a.ld + hc + (e & 31) * 4) = f32x4{0, 0, 0, 0};
    }
    return;
  }
  const int32_t* __restrict__ klist = a.kidx + (int64_t)row_id * a.nk_stride;
  const uint8_t* __restrict__ srow = DENSE ? a.sel + (int64_t)row_id * a.nk : nullptr;
  const int nblocks = DENSE ? a.nk : min(cnt, a.nk_stride);
  const int ntiles = nblocks * (kBlock / BK);
  auto valid_keys = [&](int j, int part) -> int64_t {
    return (unsigned)j < (unsigned)a.nk ? a.lk - ((int64_t)j * kBlock + part * BK) : 0;
  };

  // Q as the B operand of 32x32x2 steps: step (a, b) pairs dim 8a + 4g + b with k-index g
  const int64_t qrow = (int64_t)qb * kBlock + wave * 32 + l32;
  f32x4 qf[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (qrow < a.lq) qf[i] = *(const f32x4*)(Q + qrow * a.ld + hc + 8 * i + 4 * g);
    else qf[i] = f32x4{0, 0, 0, 0};
  }

  f32x4 kreg[4], vreg[4];
  const int ld_row = tid >> 5, ld_c4 = tid & 31;
  auto load_tile = [&](int T) {
    const int jj = T >> 2, part = T & 3;
    const int j = DENSE ? jj : klist[jj];
    const int64_t valid = valid_keys(j, part);
    const int64_t row0 = valid > 0 ? a.map.row(j) + part * BK : 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int r = p * 8 + ld_row;
      if (r < valid) {
        const int64_t off = (row0 + r) * a.kv_ld + h * a.kv_head_stride + ld_c4 * 4;
        kreg[p] = *(const f32x4*)(K + off);
        vreg[p] = *(const f32x4*)(V + off);
      } else {
        kreg[p] = f32x4{0, 0, 0, 0};
        vreg[p] = f32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int st) {
    float* ks = smem + st * 2 * TILE;
    float* vs = ks + TILE;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int r = p * 8 + ld_row;
      *(f32x4*)(ks + r * LDR + ld_c4 * 4) = kreg[p];
      *(f32x4*)(vs + r * LDR + ld_c4 * 4) = vreg[p];
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  f32x16 acc_o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) acc_o[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = a.c;

  for (int T = 0; T < ntiles; ++T) {
    const int st = T & 1;
    const bool has_next = T + 1 < ntiles;
    if (has_next) load_tile(T + 1);
    const float* ks = smem + st * 2 * TILE;
    const float* vs = ks + TILE;

    f32x16 s = f32x16{};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const f32x4 kf = *(const f32x4*)(ks + l32 * LDR + 8 * i + 4 * g);
#pragma unroll
      for (int b = 0; b < 4; ++b) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[b], qf[i][b], s, 0, 0, 0);
    }

    const int jj = T >> 2;
    bool dead = false;
    if (DENSE) dead = srow[jj] == 0;
    const int j = DENSE ? jj : klist[jj];
    const int64_t valid = valid_keys(j, T & 3);
    if (dead) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = -INFINITY;
    } else if (valid < BK) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + 4 * g + (r & 3) >= valid) s[r] = -INFINITY;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = pair_max(mx);
    const float m_use = rescale_if_grown<4>(mx * c, m_run, l_run, acc_o);
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(fmaf(s[r], c, -m_use));
      lsum += s[r];
    }
    l_run += lsum;

    // O^T += V^T P^T: k-step r pairs key 8(r/4) + 4g + r%4 (this lane's P entry r) with k-index g
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const float vv = vs[key * LDR + 32 * dt + l32];
        acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, s[r], acc_o[dt], 0, 0, 0);
      }
    }

    if (has_next) store_tile(st ^ 1);
    __syncthreads();
  }

  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qrow < a.lq) {
    float* orow = O + a.out_row(qrow) * a.ld + hc;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        f32x4 ov;
        ov[0] = acc_o[dt][4 * r4 + 0] * inv;
        ov[1] = acc_o[dt][4 * r4 + 1] * inv;
        ov[2] = acc_o[dt][4 * r4 + 2] * inv;
        ov[3] = acc_o[dt][4 * r4 + 3] * inv;
        *(f32x4*)(orow + 32 * dt + 8 * r4 + 4 * g) = ov;
      }
  }
}

// ------------------------------------------------------------------------------------------------------------
// key lists
// ------------------------------------------------------------------------------------------------------------
// Mask (rows, nk) f32 -> kcnt, kidx (selected ascending, then unselected ascending: argSort(!sel) of
// SparseAttention.swift:175-177 with a stable order), sel bytes. One wave per row.
__global__ __launch_bounds__(256) void lists_from_mask_kernel(const float* __restrict__ mask, int rows, int nk,
                                                              int32_t* __restrict__ kidx,
                                                              int32_t* __restrict__ kcnt,
                                                              uint8_t* __restrict__ sel) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* mrow = mask + (int64_t)row * nk;
  int32_t* krow = kidx + (int64_t)row * nk;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int n_sel = 0;
  for (int j0 = 0; j0 < nk; j0 += 64) {
    const int j = j0 + lane;
    const bool s = j < nk && mrow[j] > 0.5f;
    const uint64_t b = __ballot(s);
    if (s) krow[n_sel + __popcll(b & lt)] = j;
    if (j < nk) sel[(int64_t)row * nk + j] = s ? 1 : 0;
    n_sel += __popcll(b);
  }
  int n_un = n_sel;
  for (int j0 = 0; j0 < nk; j0 += 64) {
    const int j = j0 + lane;
    const bool u = j < nk && !(mrow[j] > 0.5f);
    const uint64_t b = __ballot(u);
    if (u) krow[n_un + __popcll(b & lt)] = j;
    n_un += __popcll(b);
  }
  if (lane == 0) kcnt[row] = n_sel;
}

// (kidx, kcnt) -> sel bytes (rows, nk), for the dense walk over caller-supplied lists. One wave per row.
__global__ __launch_bounds__(256) void sel_from_lists_kernel(const int32_t* __restrict__ kidx,
                                                             const int32_t* __restrict__ kcnt, int rows,
                                                             int nk_stride, int nk, uint8_t* __restrict__ sel) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  uint8_t* srow = sel + (int64_t)row * nk;
  for (int j = lane; j < nk; j += 64) srow[j] = 0;
  __builtin_amdgcn_wave_barrier();
  __threadfence_block();
  const int c = min(kcnt[row], nk_stride);
  for (int jj = lane; jj < c; jj += 64) {
    const int j = kidx[(int64_t)row * nk_stride + jj];
    if (j >= 0 && j < nk) srow[j] = 1;
  }
}

// ------------------------------------------------------------------------------------------------------------
// launch
// ------------------------------------------------------------------------------------------------------------
// compute units of the current device (cached per device)
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// query groups per wave of the bf16 walk: 1 (4 waves of 32 queries, two waves per SIMD) unless FVSR_ATTN_QG=2
// (2 waves of 64 queries, one wave per SIMD)
static int attn_query_groups() {
  static const int qg = [] {
    const char* e = getenv("FVSR_ATTN_QG");
    return (e && e[0] == '2') ? 2 : 1;
  }();
  return qg;
}

int launch_attention(int dtype, bool dense, const AttnArgs& a, hipStream_t stream) {
  const int nwg = a.heads * a.nq;
  if (nwg <= 0) return FVSR_OK;
  dim3 grid(nwg), block(256);
  if (dtype == FVSR_DTYPE_BF16) {
    if (!a.order || !a.counter) return set_error(FVSR_ERR_INVALID_ARG, "attention: no workspace for the row order");
    // two workgroups (64 KB of LDS each) are resident per CU
    const int pwgs = std::min(nwg, std::min(2 * device_cus(), kMaxPersistentWgs));
    hipLaunchKernelGGL(attn_order_kernel, dim3(1), dim3(1024), 0, stream, a.kcnt, nwg, a.nk_stride, dense ? 1 : 0,
                       pwgs, a.order, a.counter);
    const dim3 pgrid(pwgs);
    if (attn_query_groups() == 2) {
      if (dense)
        hipLaunchKernelGGL((attn_bf16_kernel<true, 2>), pgrid, dim3(128), 0, stream, a, a.kidx, a.kcnt, a.sel,
                           (const bf16*)a.q, (bf16*)a.o, (const int32_t*)a.order, a.counter);
      else
        hipLaunchKernelGGL((attn_bf16_kernel<false, 2>), pgrid, dim3(128), 0, stream, a, a.kidx, a.kcnt, a.sel,
                           (const bf16*)a.q, (bf16*)a.o, (const int32_t*)a.order, a.counter);
    } else {
      if (dense)
        hipLaunchKernelGGL((attn_bf16_kernel<true, 1>), pgrid, dim3(256), 0, stream, a, a.kidx, a.kcnt, a.sel,
                           (const bf16*)a.q, (bf16*)a.o, (const int32_t*)a.order, a.counter);
      else
        hipLaunchKernelGGL((attn_bf16_kernel<false, 1>), pgrid, dim3(256), 0, stream, a, a.kidx, a.kcnt, a.sel,
                           (const bf16*)a.q, (bf16*)a.o, (const int32_t*)a.order, a.counter);
    }
  } else {
    if (dense) hipLaunchKernelGGL(attn_f32_kernel<true>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(attn_f32_kernel<false>, grid, block, 0, stream, a);
  }
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

// ------------------------------------------------------------------------------------------------------------
// allocation-free scratch of fvsr_lcsa_attention_noalloc
// ------------------------------------------------------------------------------------------------------------
// The persistent walk's row order (one int32 per (head, query block) row) and its work counter live in a file-scope
// device array instead of the context workspace: bytes [0, 256) hold the counter, the order starts at byte 256.
// Every GPU holds its own copy for the life of the process. In host code `scratch` names a host-side stand-in, so
// the device address is taken once per device with hipGetSymbolAddress (noalloc_scratch_init, called by
// fvsr_ctx_create with the device current) and only that address reaches kernels. The order kernel rewrites the
// counter and every order entry it uses on each call, so nothing needs clearing; calls that overlap on one GPU
// share the array and race.
constexpr int kNoAllocRows = 1 << 18;
constexpr size_t kNoAllocScratchBytes = 256 + (size_t)kNoAllocRows * sizeof(int32_t);
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxDevices] = {};

int noalloc_max_rows() { return kNoAllocRows; }

int noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(FVSR_ERR_UNSUPPORTED, "device index beyond " + std::to_string(kMaxDevices));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device]) return FVSR_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return set_error(FVSR_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  g_scratch_ptr[device] = p;
  return FVSR_OK;
}

// the row order and counter of `device`'s scratch for `rows` rows (FVSR_ERR_STATE before noalloc_scratch_init)
int noalloc_scratch(int device, int64_t rows, int32_t** order, int32_t** counter) {
  if (rows > kNoAllocRows)
    return set_error(FVSR_ERR_UNSUPPORTED, "fvsr_lcsa_attention_noalloc: " + std::to_string(rows) +
                                               " (head, query block) rows exceed its static scratch of " +
                                               std::to_string(kNoAllocRows));
  void* p = nullptr;
  if (device >= 0 && device < kMaxDevices) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[device];
  }
  if (!p) return set_error(FVSR_ERR_STATE, "no scratch address for this device: create its context first");
  *counter = (int32_t*)p;
  *order = (int32_t*)((char*)p + 256);
  return FVSR_OK;
}

int launch_lists_from_mask(const float* mask, int rows, int nk, int32_t* kidx, int32_t* kcnt, uint8_t* sel,
                           hipStream_t stream) {
  if (rows <= 0) return FVSR_OK;
  hipLaunchKernelGGL(lists_from_mask_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, mask, rows, nk, kidx,
                     kcnt, sel);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

int launch_sel_from_lists(const int32_t* kidx, const int32_t* kcnt, int rows, int nk_stride, int nk, uint8_t* sel,
                          hipStream_t stream) {
  if (rows <= 0) return FVSR_OK;
  hipLaunchKernelGGL(sel_from_lists_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, kidx, kcnt, rows,
                     nk_stride, nk, sel);
  FVSR_HIP_CHECK(hipGetLastError());
  return FVSR_OK;
}

}  // namespace fvsr
