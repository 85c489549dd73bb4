// Block-sparse flash attention over 128x128 blocks for gfx950 (MI355X).
//
// Reference semantics: the Metal kernel of SparseAttention.swift:17-154 (launched at :180-185) and the dense path
// blockMaskedAttention (DiT.swift:279-313): per head, o = softmax(q k^T / sqrt(128)) v over the listed key blocks,
// fp32 online softmax, a query block with no listed key block writes zeros.
//
// Design (not the reference's): one workgroup = one (head, 128-query block); 4 wave64s x 32 queries.
//   S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (keys = M, queries = N), so each lane owns ONE query row: the row max and
//   row sum are per-lane scalars (plus one permlane32 swap), no LDS round trip.
//   O^T += V^T P^T on the same MFMA: P^T comes straight from the S^T accumulator registers (bf16-packed), V^T is read
//   from row-major LDS with ds_read_b64_tr_b16, so V needs no transpose anywhere.
//   K/V tiles of 64 keys are double-buffered in LDS (70 KB per workgroup -> 2 workgroups per CU), prefetched to
//   registers one tile ahead; padded LDS rows keep the MFMA operand reads bank-conflict free.
//   Workgroup ids are remapped so each XCD (own L2) walks a contiguous run of (head, query block) items: adjacent
//   query blocks select overlapping key blocks (spatial locality), so K/V tiles hit in L2.
// fp32 I/O (the parity lane) runs the same scheme on v_mfma_f32_32x32x2_f32 with 32-key fp32 tiles.
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

// 3-input max without the NaN-quieting canonicalisation the compiler wraps around fmaxf (inputs are MFMA results
// or -inf, never NaN)
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

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
template <bool DENSE>
__global__ __launch_bounds__(256, 2) void attn_bf16_kernel(AttnArgs a) {
  constexpr int BK = 64;                        // keys per tile
  // Padded LDS rows (16 B of pad for K, 32 B for V) instead of an XOR swizzle: every MFMA operand address is then
  // a per-lane base plus an immediate offset (few address registers), and the access patterns stay conflict-free:
  //   K (ds_read_b128): 16 lanes read one 16-B column of 16 consecutive rows; 272 B = 68 dwords = 4 banks apart.
  //   V (ds_read_b64_tr_b16): a 16-lane group reads 4 rows x 2 chunks x 2 halves; with 288 B = 72 dwords per row
  //   the 32 dwords land in 8*row + 4*chunk + 2*half + {0, 1}: all distinct.
  constexpr int KST = 272, VST = 288;
  constexpr int TILE_K = BK * KST, TILE_V = BK * VST, STAGE = TILE_K + TILE_V;
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];   // [stage][K, V]

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int h = lid / a.nq, qb = lid - h * a.nq;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int hc = h * kHeadDim;
  const bf16* __restrict__ Q = (const bf16*)a.q;
  bf16* __restrict__ O = (bf16*)a.o;
  const int row_id = h * a.nq + qb;
  const int cnt = a.kcnt[row_id];

  if (cnt <= 0) {   // empty query block -> zeros (SparseAttention.swift:47-53; DiT.swift:300-304)
    for (int e = tid; e < kBlock * 16; e += 256) {
      const int64_t row = (int64_t)qb * kBlock + (e >> 4);
      if (row < a.lq) *(u32x4*)(O + row * a.ld + hc + (e & 15) * 8) = u32x4{0, 0, 0, 0};
    }
    return;
  }
  const int32_t* __restrict__ klist = a.kidx + (int64_t)row_id * a.nk_stride;
  const uint8_t* __restrict__ srow = DENSE ? a.sel + (int64_t)row_id * a.nk : nullptr;
  const int nblocks = DENSE ? a.nk : min(cnt, a.nk_stride);
  const int ntiles = nblocks * 2;
  // keys of logical block j in tile half `half` that exist; a listed index outside [0, nk) contributes nothing
  auto valid_keys = [&](int j, int half) -> int {
    return (unsigned)j < (unsigned)a.nk ? (int)min<int64_t>(BK, a.lk - ((int64_t)j * kBlock + half * BK)) : 0;
  };

  // Q as the B operand: lane (query l32, k-half g) holds dims 16t + 8g .. +7 for t = 0..7.
  const int64_t qrow = (int64_t)qb * kBlock + wave * 32 + l32;
  bf16x8 qreg[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (qrow < a.lq) qreg[t] = *(const bf16x8*)(Q + qrow * a.ld + hc + 16 * t + 8 * g);
    else qreg[t] = bf16x8{};
  }

  // K/V tiles through buffer loads: the resource spans the physical rows, so any row past it reads back as zero
  // (the ragged last block needs no per-lane guard); the tile base goes in the scalar offset.
  const uint32_t row_bytes = (uint32_t)a.ld * 2;
  const int32_t range = (int32_t)(a.kv_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)a.k, 0, range, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)a.v, 0, range, 0x00020000);
  const int ld_row = tid >> 4, ld_chunk = tid & 15;          // thread -> (row p*16 + tid/16, 16-byte chunk)
  const int voff = ld_row * (int)row_bytes + hc * 2 + ld_chunk * 16;
  u32x4 kreg[4], vreg[4];
  auto load_tile = [&](int T) {
    const int jj = T >> 1, half = T & 1;
    const int j = DENSE ? jj : klist[jj];
    if (valid_keys(j, half) > 0) {
      const int soff = (int)((a.map.row(j) + half * BK) * row_bytes);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        kreg[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, voff, soff + p * 16 * (int)row_bytes, 0));
        vreg[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff, soff + p * 16 * (int)row_bytes, 0));
      }
    } else {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        kreg[p] = u32x4{0, 0, 0, 0};
        vreg[p] = u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int st) {
    char* ks = smem + st * STAGE + ld_row * KST + ld_chunk * 16;
    char* vs = smem + st * STAGE + TILE_K + ld_row * VST + ld_chunk * 16;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      *(u32x4*)(ks + p * 16 * KST) = kreg[p];
      *(u32x4*)(vs + p * 16 * VST) = vreg[p];
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
  // ds_read_tr addressing for the V^T operand (see file header): 16-lane group G, member m reads
  // V[16u + 4(G/2) + m/4 (+8)][32dt + 16(G%2) + 4(m%4) .. +3]
  const int G = lane >> 4, m = lane & 15;
  const int tr_base = (4 * (G >> 1) + (m >> 2)) * VST + (2 * (G & 1) + ((m & 3) >> 1)) * 16 + (m & 1) * 8;
  const int k_base = l32 * KST + g * 16;                       // K operand: row l32 (+32), chunk 2t + g
  const bf16x2 ones = {(bf16)1.0f, (bf16)1.0f};

  for (int T = 0; T < ntiles; ++T) {
    const int st = T & 1;
    const bool has_next = T + 1 < ntiles;
    if (has_next) load_tile(T + 1);
    const char* ks = smem + st * STAGE + k_base;
    const char* vs = smem + st * STAGE + TILE_K + tr_base;

    // S^T (64 keys x 32 queries) = K (64 x 128) . Q^T (128 x 32)
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bf16x8 k0 = *(const bf16x8*)(ks + t * 32);
      const bf16x8 k1 = *(const bf16x8*)(ks + 32 * KST + t * 32);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k0, qreg[t], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k1, qreg[t], s1, 0, 0, 0);
    }

    // mask: unselected block (dense walk) or keys past the logical end (ragged last block); uniform branches
    const int jj = T >> 1;
    const int j = DENSE ? jj : klist[jj];
    const int valid = (DENSE && srow[jj] == 0) ? 0 : valid_keys(j, T & 1);
    if (valid < BK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = 8 * (r >> 2) + 4 * g + (r & 3);
        if (kk >= valid) s0[r] = -INFINITY;
        if (kk + 32 >= valid) s1[r] = -INFINITY;
      }
    }

    // online softmax in the log2 domain; this lane's query row is l32
    float mx0 = vmax3(s0[0], s0[1], s0[2]), mx1 = vmax3(s1[0], s1[1], s1[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) {
      mx0 = vmax3(mx0, s0[r], s0[r + 1]);
      mx1 = vmax3(mx1, s1[r], s1[r + 1]);
    }
    const float mx = pair_max(vmax3(mx0, mx1, fmaxf(s0[15], s1[15])));
    const float m_use = rescale_if_grown<4>(mx * c, m_run, l_run, acc_o);

    // P = exp2(S c - m) packed to bf16 (the B operand of the PV product); the row sum is taken over the same
    // bf16-rounded P with v_dot2 (two keys per instruction)
    bf16x8 pop[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f32x16& sp = (u >> 1) ? s1 : s0;
      const int hh = u & 1;
#pragma unroll
      for (int e = 0; e < 8; ++e) pop[u][e] = (bf16)__builtin_amdgcn_exp2f(fmaf(sp[8 * hh + e], c, -m_use));
    }
    float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ls0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pop[u], pop[u], 0, 1), ones, ls0, false);
      ls1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pop[u], pop[u], 2, 3), ones, ls1, false);
      ls0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pop[u], pop[u], 4, 5), ones, ls0, false);
      ls1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pop[u], pop[u], 6, 7), ones, ls1, false);
    }
    l_run += ls0 + ls1;

    // O^T (128 dims x 32 queries) += V^T (128 x 64 keys) . P^T (64 x 32), 4 k-steps of 16 keys
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const char* pa = vs + 16 * u * VST + dt * 64;
        const char* pb = pa + 8 * VST;
        const i16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)pa);
        const i16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)pb);
        // whole-vector concatenation: element-wise assembly of the operand is mis-lowered (one dword duplicated)
        const i16x8 vcat = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
        acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vcat), pop[u], acc_o[dt], 0,
                                                           0, 0);
      }
    }

    if (has_next) store_tile(st ^ 1);
    __syncthreads();
  }

  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qrow < a.lq) {
    bf16* orow = O + qrow * a.ld + hc;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        bf16x4 ov;
        ov[0] = (bf16)(acc_o[dt][4 * r4 + 0] * inv);
        ov[1] = (bf16)(acc_o[dt][4 * r4 + 1] * inv);
        ov[2] = (bf16)(acc_o[dt][4 * r4 + 2] * inv);
        ov[3] = (bf16)(acc_o[dt][4 * r4 + 3] * inv);
        *(bf16x4*)(orow + 32 * dt + 8 * r4 + 4 * g) = ov;
      }
  }
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
      if (row < a.lq) *(f32x4*)(O + row * a.ld + hc + (e & 31) * 4) = f32x4{0, 0, 0, 0};
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
        const int64_t off = (row0 + r) * a.ld + hc + ld_c4 * 4;
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
    float* orow = O + qrow * a.ld + hc;
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
int launch_attention(int dtype, bool dense, const AttnArgs& a, hipStream_t stream) {
  const int nwg = a.heads * a.nq;
  if (nwg <= 0) return FVSR_OK;
  dim3 grid(nwg), block(256);
  if (dtype == FVSR_DTYPE_BF16) {
    if (dense) hipLaunchKernelGGL(attn_bf16_kernel<true>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(attn_bf16_kernel<false>, grid, block, 0, stream, a);
  } else {
    if (dense) hipLaunchKernelGGL(attn_f32_kernel<true>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(attn_f32_kernel<false>, grid, block, 0, stream, a);
  }
  FVSR_HIP_CHECK(hipGetLastError());
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
