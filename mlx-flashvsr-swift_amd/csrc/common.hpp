// Shared types and helpers for the gfx950 LCSA kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>
#include <type_traits>

#include "../../include/fvsr_lcsa.h"

namespace fvsr {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 128;     // tokens per LCSA window / block
constexpr int kHeadDim = 128;   // head dim of every FlashVSR head
constexpr int kXcds = 8;        // MI355X: 8 XCDs, workgroups dispatched round-robin across them
constexpr int kMaxDevices = 64; // device indices with per-device state (scratch addresses, CU counts)

// s_waitcnt vmcnt(0) lgkmcnt(0): every memory operation of this wave, stores included, has completed (gfx9 counts
// stores in vmcnt; encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
#define FVSR_WAIT_VM0() __builtin_amdgcn_s_waitcnt(7 << 4)
constexpr int kPoolParts = 4;   // a block mean is summed as 4 runs of 32 tokens, then ((p0 + p1) + (p2 + p3)) / n

// Records the failure message for fvsr_last_error() and returns the status (defined in api.hip).
int set_error(int status, const std::string& msg);

#define FVSR_HIP_CHECK(expr)                                                                          \
  do {                                                                                                \
    hipError_t e_ = (expr);                                                                           \
    if (e_ != hipSuccess)                                                                             \
      return ::fvsr::set_error(FVSR_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_));      \
  } while (0)

// Workgroups are dispatched round-robin over the XCDs (each with its own L2). Remap so that every XCD owns one
// contiguous range of logical work items: neighbouring (head, query block) items — which select overlapping key
// blocks — then share one L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  const int xcd = bid % kXcds, idx = bid / kXcds;
  const int q = nwg / kXcds, rem = nwg % kXcds;
  return xcd < rem ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
}

// f(integral_constant<I>) for I = B .. E-1, unrolled at compile time
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// inclusive scan over the 64 lanes of a wave
__device__ __forceinline__ unsigned wave_incl_scan(unsigned x) {
  const int lane = threadIdx.x & 63;
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Logical key block j of the key range -> first token row of that block in the K/V buffer.
// Plain buffers: plain_key_map() (slot_head 0, capacity 1, slice_blocks 65536 >= Nk) gives row j*128.
// Ring: block j lives in slot (head + j / s) % capacity at block j % s of that slot.
// The walks evaluate this once per key block, so the division is a multiply: with inv = floor(2^32 / s) + 1 (33 bits
// for s = 1), floor(j / s) = (j * inv) >> 32 exactly for 0 <= j < 2^16 and 1 <= s <= 2^16 (inv * s = 2^32 + e with 0 < e <= s, so
// the error term j * e / (s * 2^32) stays below 1 / s). Both hold: K/V buffers and ring layers are below 2 GiB, so a
// key range has fewer than 2^16 blocks. The ring holds at most `capacity` slices (j / s < capacity), so the slot
// wraps at most once.
struct KeyMap {
  int slot_head;
  int capacity;
  int slice_blocks;
  uint64_t inv;
  __device__ __forceinline__ int64_t row(int j) const {
    const int q = (int)(((uint64_t)(unsigned)j * inv) >> 32);
    int slot = slot_head + q;
    if (slot >= capacity) slot -= capacity;
    return ((int64_t)slot * slice_blocks + (j - q * slice_blocks)) * kBlock;
  }
};
inline KeyMap make_key_map(int slot_head, int capacity, int slice_blocks) {
  return KeyMap{slot_head, capacity, slice_blocks, (((uint64_t)1) << 32) / (uint64_t)slice_blocks + 1};
}
inline KeyMap plain_key_map() { return make_key_map(0, 1, 1 << 16); }

// One job of pool_mean_kernel (lcsa_select.hip): the block means of the L tokens of x (nb = ceil(L / 128) blocks);
// block b is written to row ((slot0 + b / slice_blocks) % capacity) * slice_blocks + b % slice_blocks of out (a ring
// slot mapping; slot0 0, capacity 1, slice_blocks >= nb for a plain buffer). x is token-major (rows of C channels)
// when head_stride is 0, else head-major: channel c of token t at (c / 128) * head_stride + t * 128 + c % 128.
struct PoolMean {
  const void* x;
  int64_t L;
  float* out;
  int nb, slot0, capacity, slice_blocks;
  int64_t head_stride;
};

// element offset of (token t, channel c) in a buffer of C channels per token: token-major when head_stride is 0,
// else head-major (each head's 128 channels of all tokens contiguous, head h at h * head_stride)
__host__ __device__ __forceinline__ int64_t kv_offset(int64_t t, int c, int C, int64_t head_stride) {
  return head_stride == 0 ? t * C + c : (int64_t)(c / kHeadDim) * head_stride + t * kHeadDim + c % kHeadDim;
}

// One block-mean target of pool_finish_kernel (kv_ring.hip): nb blocks (L tokens) of run sums in partial; block b
// is written to row ((slot0 + b / slice_blocks) % capacity) * slice_blocks + b % slice_blocks of out (a ring
// slot mapping; slot0 0, capacity 1, slice_blocks >= nb for a plain buffer).
struct PoolDst {
  const float* partial;
  float* out;
  int64_t L;
  int nb, slot0, capacity, slice_blocks;
};

// Arguments of the attention kernels (lcsa_attn.hip).
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t lq;            // valid query tokens
  int64_t lk;            // valid key tokens (logical key range)
  int heads;
  int ld;                // channels per token = heads * 128
  const int32_t* kidx;   // (H, nq, nk_stride) listed key blocks
  const int32_t* kcnt;   // (H, nq)
  const uint8_t* sel;    // (H, nq, nk) selection bytes, dense mode only
  int nk_stride;
  int nq;
  int nk;
  KeyMap map;
  int64_t kv_head_stride;   // elements from head h's K/V to head h + 1's: 128 in token-major buffers (rows of
                            // heads * 128), rows * 128 in head-major ones (each head's rows contiguous: the KV ring)
  int kv_ld;                // elements between consecutive K/V token rows: heads * 128 or 128
  int64_t kv_bytes;         // bytes of each of the k and v buffers (the buffer-load range), < 2 GiB
  float c;               // softmax scale * log2(e)
  int32_t* order;        // (H * nq) rows, longest key list first (bf16 persistent walk; workspace)
  int32_t* counter;      // per-XCD queue counters of the walk, counter[8 x] for XCD x (workspace, 256 bytes; set by
                         // the order kernel)
  int o_nbh, o_nbw;      // > 0: write o in natural (f, h, w) token order of an (8 o_nbh, 8 o_nbw) grid (the
                         // reference's windowReverse, DiT.swift:121-126) instead of window order
  // output row of window-order query row r
  __device__ __forceinline__ int64_t out_row(int64_t r) const;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// token t (0..127) of window b -> natural (f, h, w) token index, windows ordered (nf, nh, nw), tokens (wf, wh, ww)
// (windowPartition, DiT.swift:113-118)
__device__ __forceinline__ int64_t window_token_to_grid(int b, int t, int nbh, int nbw) {
  const int per_slice = nbh * nbw;
  const int nf = b / per_slice, rem = b % per_slice;
  const int nh = rem / nbw, nw = rem % nbw;
  const int wf = t >> 6, wh = (t >> 3) & 7, ww = t & 7;
  const int64_t H = 8 * nbh, W = 8 * nbw;
  return ((int64_t)(2 * nf + wf) * H + 8 * nh + wh) * W + 8 * nw + ww;
}

__device__ __forceinline__ int64_t AttnArgs::out_row(int64_t r) const {
  return o_nbw > 0 ? window_token_to_grid((int)(r >> 7), (int)(r & 127), o_nbh, o_nbw) : r;
}

}  // namespace fvsr
