// extern "C" entry points of libfvsr_lcsa (declared in include/fvsr_lcsa.h).
//
// Host-side responsibilities: argument validation before any device work (the reference traps on the same shape
// preconditions, SparseAttention.swift:173; DiT.swift:166,297), the context workspace, the KV-ring bookkeeping
// (slot head / count per layer, the trim rule of DiT.swift:532-538) and kernel launches on the caller's stream.
// No entry point synchronises the host with the device.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "common.hpp"

namespace fvsr {

static thread_local std::string g_last_error;

int set_error(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

// kernels (lcsa_attn.hip, lcsa_select.hip, kv_ring.hip)
int launch_attention(int dtype, bool dense, const AttnArgs& a, hipStream_t stream);
int launch_lists_from_mask(const float* mask, int rows, int nk, int32_t* kidx, int32_t* kcnt, uint8_t* sel,
                           hipStream_t stream);
int launch_sel_from_lists(const int32_t* kidx, const int32_t* kcnt, int rows, int nk_stride, int nk, uint8_t* sel,
                          hipStream_t stream);
int launch_scores_softmax(const float* pq, const float* pk, KeyMap kmap, int heads, int C, int nq, int nk, int s,
                          const uint8_t* local, float* probs, unsigned* hist, int q_slices, hipStream_t stream);
size_t hist12_bytes(int heads, int q_slices);
size_t topk_cand_bytes(int heads, int64_t nq);
int launch_topk_emit(const float* probs, int heads, int nq, int nk, int q_slices, int topk, unsigned* hist,
                     unsigned* cand, float* thr, float* mask_out, uint8_t* sel, int32_t* kidx, int32_t* kcnt,
                     hipStream_t stream);
int launch_qkv_epilogue(int dtype, const void* q, const void* k, const void* v, int f, int h, int w, int C, int t0,
                        const void* wq, const void* wk, float eps, const float* rope, void* q_out, void* k_out,
                        void* v_out, int dst_slot0, int capacity, int slice_blocks, int64_t kv_head_stride,
                        hipStream_t stream);
int launch_pool_mean(int dtype, PoolMean* jobs, int n, int C, unsigned* zero, int64_t nzero, hipStream_t stream);
int launch_pool_finish(const PoolDst* dst, int n, int C, unsigned* zero, int64_t nzero, hipStream_t stream);
int rope_table_floats();
int blas_create(int device, void** out);
void blas_destroy(void* p);
int linear_bf16(void* state, const void* x, int64_t L, int K, const void* w, int N, const void* bias, int epilogue,
                void* y, hipStream_t stream);
int launch_modulation(const void* m, const void* t, void* out, int C, hipStream_t stream);
int launch_residual_norm(void* x, const void* y, const void* gate, int64_t L, int C, float eps, const void* w,
                         const void* bias, const void* scale, const void* shift, void* out, hipStream_t stream);
int launch_rms_norm(const void* x, int64_t L, int C, float eps, const void* w, void* out, hipStream_t stream);
int launch_full_lists(int rows, int nkc, int32_t* kidx, int32_t* kcnt, hipStream_t stream);
int noalloc_scratch_init(int device);
int noalloc_scratch(int device, int64_t rows, int32_t** order, int32_t** counter);
void rope_tables_host(double theta, float* out);
int launch_ring_append(int dtype, const void* k_new, const void* v_new, int n_blocks, int C, bool grid_layout,
                       int nbh, int nbw, int slot0, int capacity, void* ring_k, void* ring_v, int64_t head_stride,
                       float* pooled, float* partial, hipStream_t stream);
int launch_ring_read(int dtype, const void* rk, const void* rv, void* ok, void* ov, int n_blocks, int C,
                     int64_t head_stride, KeyMap map, hipStream_t stream);
int launch_window_layout(int dtype, const void* x, void* out, int f, int h, int w, int C, bool to_windows,
                         hipStream_t stream);

constexpr int kMaxSelectKeyBlocks = 1920;    // scores stage LDS: (8 x (128 + Nk) + 2 x 64 x 132) fp32 + 8 x Nk B
constexpr double kAutoThreshold = 0.45;      // DiT.swift:210

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// workspace carve for one select + attention call
struct Carve {
  size_t pq, pk, probs, kidx, kcnt, sel, order, counter, thr, hist, cand, total;
};
static Carve carve(int heads, int64_t nq, int64_t nk, int C) {
  Carve c;
  size_t off = 0;
  c.pq = off; off += align256((size_t)nq * C * 4);
  c.pk = off; off += align256((size_t)nk * C * 4);
  c.probs = off; off += align256((size_t)heads * nq * nk * 4);
  c.kidx = off; off += align256((size_t)heads * nq * nk * 4);
  c.kcnt = off; off += align256((size_t)heads * nq * 4);
  c.sel = off; off += align256((size_t)heads * nq * nk);
  c.order = off; off += align256((size_t)heads * nq * 4);
  c.counter = off; off += 256;
  c.thr = off; off += align256((size_t)heads * nq * 4);   // per (head, query slice) thresholds (nq >= slices)
  c.hist = off; off += align256(hist12_bytes(heads, (int)nq));   // nq >= query slices
  c.cand = off; off += align256(topk_cand_bytes(heads, nq));
  c.total = off;
  return c;
}

static bool valid_dtype(int d) { return d == FVSR_DTYPE_F32 || d == FVSR_DTYPE_BF16; }
static int esize(int d) { return d == FVSR_DTYPE_BF16 ? 2 : 4; }

}  // namespace fvsr

using namespace fvsr;

struct fvsr_ctx {
  int device = 0;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  void* block_ws = nullptr;   // DiT block activations (separate from ws, which the layer call may grow)
  size_t block_ws_bytes = 0;
  void* blas = nullptr;       // hipBLASLt handle, GEMM workspace and algorithm cache (dit_block.hip)
};

struct fvsr_kv_ring {
  fvsr_ctx* ctx = nullptr;
  int dtype = 0, layers = 0, heads = 0, bh = 0, bw = 0, s = 0, capacity = 0, kv_len = 0, C = 0;
  std::vector<int> head, count;
  // (layers, heads, capacity * s * 128, 128): head-major per layer, so a 32-key tile of one head is one contiguous
  // 8 KB run (bf16) rather than 32 rows 3 KB apart
  void* k = nullptr;
  void* v = nullptr;
  float* pooled = nullptr;   // (layers, capacity * s, C)
  float* partial = nullptr;  // (capacity * s * kPoolParts, C): pooled-key runs of one append
  size_t layer_tokens() const { return (size_t)capacity * s * kBlock; }
  char* layer_k(int l) const { return (char*)k + (size_t)l * layer_tokens() * C * esize(dtype); }
  char* layer_v(int l) const { return (char*)v + (size_t)l * layer_tokens() * C * esize(dtype); }
  float* layer_pooled(int l) const { return pooled + (size_t)l * capacity * s * C; }
  KeyMap map(int l) const { return make_key_map(head[l], capacity, s); }
  int64_t head_stride() const { return (int64_t)layer_tokens() * kHeadDim; }   // elements between heads of a layer
};

#define FVSR_REQUIRE(cond, status, msg) \
  do {                                  \
    if (!(cond)) return set_error((status), (msg)); \
  } while (0)

static int ensure_ws(fvsr_ctx* ctx, size_t bytes) {
  if (ctx->ws_bytes >= bytes) return FVSR_OK;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  if (ctx->ws) FVSR_HIP_CHECK(hipFree(ctx->ws));
  ctx->ws = nullptr;
  ctx->ws_bytes = 0;
  if (hipMalloc(&ctx->ws, bytes) != hipSuccess) {
    ctx->ws = nullptr;
    return set_error(FVSR_ERR_OUT_OF_MEMORY, "workspace allocation of " + std::to_string(bytes) + " bytes failed");
  }
  ctx->ws_bytes = bytes;
  return FVSR_OK;
}

static int check_heads(int heads) {
  FVSR_REQUIRE(heads > 0 && heads <= 4096, FVSR_ERR_INVALID_ARG, "heads must be in [1, 4096]");
  return FVSR_OK;
}

extern "C" {

int fvsr_abi_version(void) { return FVSR_ABI_VERSION; }

const char* fvsr_last_error(void) { return g_last_error.c_str(); }

int fvsr_device_props(int device, int* cu_count, int* xcd_count, size_t* lds_bytes, char* arch, size_t arch_len) {
  hipDeviceProp_t p;
  FVSR_HIP_CHECK(hipGetDeviceProperties(&p, device));
  if (cu_count) *cu_count = p.multiProcessorCount;
  // gfx950 (MI355X) packs 32 CUs per XCD
  if (xcd_count) *xcd_count = std::max(1, p.multiProcessorCount / 32);
  if (lds_bytes) *lds_bytes = p.sharedMemPerBlock;
  if (arch && arch_len) {
    std::strncpy(arch, p.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = 0;
  }
  return FVSR_OK;
}

int fvsr_ctx_create(int device, fvsr_ctx** out) {
  FVSR_REQUIRE(out != nullptr, FVSR_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  int n = 0;
  FVSR_HIP_CHECK(hipGetDeviceCount(&n));
  FVSR_REQUIRE(device >= 0 && device < n, FVSR_ERR_INVALID_ARG, "no such device");
  // the device address of the allocation-free entry point's static scratch, taken once per device with the
  // device current
  int prev = 0;
  FVSR_HIP_CHECK(hipGetDevice(&prev));
  FVSR_HIP_CHECK(hipSetDevice(device));
  const int rc = noalloc_scratch_init(device);
  FVSR_HIP_CHECK(hipSetDevice(prev));
  if (rc) return rc;
  fvsr_ctx* c = new (std::nothrow) fvsr_ctx();
  FVSR_REQUIRE(c != nullptr, FVSR_ERR_OUT_OF_MEMORY, "context allocation failed");
  c->device = device;
  *out = c;
  return FVSR_OK;
}

int fvsr_ctx_destroy(fvsr_ctx* ctx) {
  if (!ctx) return FVSR_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->ws) (void)hipFree(ctx->ws);
  if (ctx->block_ws) (void)hipFree(ctx->block_ws);
  blas_destroy(ctx->blas);
  delete ctx;
  return FVSR_OK;
}

int fvsr_ctx_reserve(fvsr_ctx* ctx, size_t bytes) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  return ensure_ws(ctx, bytes);
}

size_t fvsr_ctx_workspace_bytes(const fvsr_ctx* ctx) { return ctx ? ctx->ws_bytes : 0; }

size_t fvsr_workspace_size(int heads, int64_t lq, int64_t lk, int channels) {
  if (heads <= 0 || lq < 0 || lk < 0 || channels <= 0) return 0;
  return carve(heads, ceil_div(lq, kBlock), ceil_div(lk, kBlock), channels).total;
}

int fvsr_local_block_mask(int bh, int bw, int range, uint8_t* out) {
  FVSR_REQUIRE(out != nullptr, FVSR_ERR_INVALID_ARG, "out is NULL");
  FVSR_REQUIRE(bh > 0 && bw > 0 && range >= 0, FVSR_ERR_INVALID_ARG, "bh, bw must be > 0 and range >= 0");
  const int half = range / 2, s = bh * bw;
  for (int qr = 0; qr < bh; ++qr)
    for (int qc = 0; qc < bw; ++qc)
      for (int kr = 0; kr < bh; ++kr)
        for (int kc = 0; kc < bw; ++kc) {
          const bool in_row = kr >= qr - half && kr <= qr - half + range - 1;
          const bool in_col = kc >= qc - half && kc <= qc - half + range - 1;
          out[(size_t)(qr * bw + qc) * s + kr * bw + kc] = (in_row && in_col) ? 1 : 0;
        }
  return FVSR_OK;
}

int fvsr_attention_mode_auto(int topk, int s, int nk, double threshold, double* expected, int* mode) {
  FVSR_REQUIRE(s > 0 && nk > 0, FVSR_ERR_INVALID_ARG, "s and nk must be > 0");
  const double e = std::min(1.0, (double)(topk + 1) / ((double)s * (double)nk));
  if (expected) *expected = e;
  if (mode) *mode = e <= threshold ? FVSR_ATTN_KERNEL : FVSR_ATTN_DENSE;
  return FVSR_OK;
}

// ---------------------------------------------------------------------------------------------------------------
// selection
// ---------------------------------------------------------------------------------------------------------------
// q_pooled: the caller has already written the pooled queries to the workspace's pq and cleared its histogram
// (the qkv layer call does both in the launches of its ring append)
static int select_impl(fvsr_ctx* ctx, int dtype, const void* qW, int64_t lq, const float* pk_src, bool pk_ready,
                       const void* kW, int64_t lk, KeyMap kmap, int nk, int heads, int q_slices, int s,
                       const uint8_t* local, int topk, float* mask_out, float* probs_out, int32_t* kidx,
                       int32_t* kcnt, uint8_t* sel_out, hipStream_t stream, bool q_pooled = false) {
  const int C = heads * kHeadDim;
  const int64_t nq = ceil_div(lq, kBlock);
  FVSR_REQUIRE(nq == (int64_t)q_slices * s, FVSR_ERR_INVALID_ARG,
               "ceil(lq/128) must equal q_slices * s (query blocks split evenly into temporal slices)");
  FVSR_REQUIRE(nk > 0 && nk <= kMaxSelectKeyBlocks, FVSR_ERR_UNSUPPORTED,
               "key blocks must be in [1, " + std::to_string(kMaxSelectKeyBlocks) + "]");
  FVSR_REQUIRE(topk >= 0, FVSR_ERR_INVALID_ARG, "topk must be >= 0");
  const Carve cv = carve(heads, nq, nk, C);
  int rc = ensure_ws(ctx, cv.total);
  if (rc) return rc;
  char* ws = (char*)ctx->ws;
  float* pq = (float*)(ws + cv.pq);
  float* probs = probs_out ? probs_out : (float*)(ws + cv.probs);
  uint8_t* sel = sel_out ? sel_out : (uint8_t*)(ws + cv.sel);
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  unsigned* hist = (unsigned*)(ws + cv.hist);
  const float* pk = pk_ready ? pk_src : (const float*)(ws + cv.pk);
  if (!q_pooled || !pk_ready) {
    // block means of Q (and K) and the histogram reset, one launch
    PoolMean jobs[2];
    int n = 0;
    if (!q_pooled) jobs[n++] = PoolMean{qW, lq, pq, 0, 0, 1, 1 << 30, 0};
    if (!pk_ready) jobs[n++] = PoolMean{kW, lk, (float*)(ws + cv.pk), 0, 0, 1, 1 << 30, 0};
    if ((rc = launch_pool_mean(dtype, jobs, n, C, q_pooled ? nullptr : hist,
                               (int64_t)(hist12_bytes(heads, q_slices) / sizeof(unsigned)), stream)))
      return rc;
  }
  if ((rc = launch_scores_softmax(pq, pk, kmap, heads, C, (int)nq, nk, s, local, probs, hist, q_slices, stream)))
    return rc;
  return launch_topk_emit(probs, heads, (int)nq, nk, q_slices, topk, hist, (unsigned*)(ws + cv.cand),
                          (float*)(ws + cv.thr), mask_out, sel, kidx, kcnt, stream);
}

int fvsr_lcsa_select(fvsr_ctx* ctx, int dtype, const void* qW, int64_t lq, const void* kW, int64_t lk, int heads,
                     int q_slices, int s, const uint8_t* local_dev, int topk, float* mask_out, float* probs_out,
                     int32_t* kidx_out, int32_t* kcnt_out, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  FVSR_REQUIRE(valid_dtype(dtype), FVSR_ERR_INVALID_ARG, "dtype must be FVSR_DTYPE_F32 or FVSR_DTYPE_BF16");
  int rc = check_heads(heads);
  if (rc) return rc;
  FVSR_REQUIRE(qW && kW && local_dev && kidx_out && kcnt_out, FVSR_ERR_INVALID_ARG,
               "qW, kW, local, kidx and kcnt must be non-NULL");
  FVSR_REQUIRE(lq > 0 && lk > 0, FVSR_ERR_INVALID_ARG, "lq and lk must be > 0");
  FVSR_REQUIRE(q_slices > 0 && s > 0, FVSR_ERR_INVALID_ARG, "q_slices and s must be > 0");
  const int64_t nk = ceil_div(lk, kBlock);
  FVSR_REQUIRE(nk <= kMaxSelectKeyBlocks, FVSR_ERR_UNSUPPORTED, "too many key blocks for selection");
  return select_impl(ctx, dtype, qW, lq, nullptr, false, kW, lk, plain_key_map(), (int)nk, heads, q_slices,
                     s, local_dev, topk, mask_out, probs_out, kidx_out, kcnt_out, nullptr, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------------------------------------------
// K/V token-major (rows of heads * 128 elements of es bytes, lk rows); the ring's head-major layout is set by its caller
static AttnArgs make_args(const void* q, int64_t lq, const void* k, const void* v, int64_t lk, int heads,
                          const int32_t* kidx, const int32_t* kcnt, const uint8_t* sel, int nk_stride, int nk,
                          KeyMap map, void* o, int es) {
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.lq = lq; a.lk = lk;
  a.heads = heads; a.ld = heads * kHeadDim;
  a.kidx = kidx; a.kcnt = kcnt; a.sel = sel;
  a.nk_stride = nk_stride;
  a.nq = (int)ceil_div(lq, kBlock);
  a.nk = nk;
  a.map = map;
  a.kv_head_stride = kHeadDim;
  a.kv_ld = a.ld;
  a.kv_bytes = lk * a.ld * es;
  a.c = (float)(1.4426950408889634 / std::sqrt((double)kHeadDim));
  return a;
}

// the persistent walk's row order and work counter, carved from the context workspace (grown if needed)
static int attach_order(fvsr_ctx* ctx, AttnArgs& a, int64_t nk) {
  const Carve cv = carve(a.heads, a.nq, nk, a.ld);
  int rc = ensure_ws(ctx, cv.total);
  if (rc) return rc;
  a.order = (int32_t*)((char*)ctx->ws + cv.order);
  a.counter = (int32_t*)((char*)ctx->ws + cv.counter);
  return FVSR_OK;
}

static int check_attn_common(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                             int64_t lk, int heads, void* o) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  FVSR_REQUIRE(valid_dtype(dtype), FVSR_ERR_INVALID_ARG, "dtype must be FVSR_DTYPE_F32 or FVSR_DTYPE_BF16");
  int rc = check_heads(heads);
  if (rc) return rc;
  FVSR_REQUIRE(q && k && v && o, FVSR_ERR_INVALID_ARG, "q, k, v and o must be non-NULL");
  FVSR_REQUIRE(lq > 0 && lk > 0, FVSR_ERR_INVALID_ARG, "lq and lk must be > 0");
  FVSR_REQUIRE((int64_t)heads * ceil_div(lq, kBlock) < (int64_t)1 << 31, FVSR_ERR_UNSUPPORTED, "grid too large");
  // K/V are addressed with 32-bit buffer offsets
  FVSR_REQUIRE(lk * heads * kHeadDim * esize(dtype) < ((int64_t)1 << 31), FVSR_ERR_UNSUPPORTED,
               "k/v buffers above 2 GiB are not supported");
  return FVSR_OK;
}

int fvsr_lcsa_attention(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                        int64_t lk, int heads, const int32_t* kidx, const int32_t* kcnt, int nk_stride, void* o,
                        void* stream) {
  int rc = check_attn_common(ctx, dtype, q, lq, k, v, lk, heads, o);
  if (rc) return rc;
  FVSR_REQUIRE(kidx && kcnt, FVSR_ERR_INVALID_ARG, "kidx and kcnt must be non-NULL");
  FVSR_REQUIRE(nk_stride > 0, FVSR_ERR_INVALID_ARG, "nk_stride must be > 0");
  const int nk = (int)ceil_div(lk, kBlock);
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  AttnArgs a = make_args(q, lq, k, v, lk, heads, kidx, kcnt, nullptr, nk_stride, nk, plain_key_map(), o, esize(dtype));
  if ((rc = attach_order(ctx, a, nk))) return rc;
  return launch_attention(dtype, false, a, (hipStream_t)stream);
}

int fvsr_lcsa_attention_noalloc(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                                int64_t lk, int heads, const int32_t* kidx, const int32_t* kcnt, int nk_stride,
                                void* o, void* stream) {
  int rc = check_attn_common(ctx, dtype, q, lq, k, v, lk, heads, o);
  if (rc) return rc;
  FVSR_REQUIRE(kidx && kcnt, FVSR_ERR_INVALID_ARG, "kidx and kcnt must be non-NULL");
  FVSR_REQUIRE(nk_stride > 0, FVSR_ERR_INVALID_ARG, "nk_stride must be > 0");
  const int nk = (int)ceil_div(lk, kBlock);
  AttnArgs a = make_args(q, lq, k, v, lk, heads, kidx, kcnt, nullptr, nk_stride, nk, plain_key_map(), o, esize(dtype));
  // only the bf16 walk keeps a row order and a work counter; the fp32 kernel has neither, so no row cap applies
  if (dtype == FVSR_DTYPE_BF16 &&
      (rc = noalloc_scratch(ctx->device, (int64_t)heads * a.nq, &a.order, &a.counter)))
    return rc;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_attention(dtype, false, a, (hipStream_t)stream);
}

int fvsr_lcsa_attention_mask(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                             int64_t lk, int heads, const float* block_mask, int mode, void* o, void* stream) {
  int rc = check_attn_common(ctx, dtype, q, lq, k, v, lk, heads, o);
  if (rc) return rc;
  FVSR_REQUIRE(block_mask != nullptr, FVSR_ERR_INVALID_ARG, "block_mask is NULL");
  FVSR_REQUIRE(mode == FVSR_ATTN_KERNEL || mode == FVSR_ATTN_DENSE, FVSR_ERR_INVALID_ARG,
               "mode must be FVSR_ATTN_KERNEL or FVSR_ATTN_DENSE (auto needs topk: use fvsr_attention_mode_auto)");
  const int64_t nq = ceil_div(lq, kBlock), nk = ceil_div(lk, kBlock);
  const Carve cv = carve(heads, nq, nk, heads * kHeadDim);
  if ((rc = ensure_ws(ctx, cv.total))) return rc;
  char* ws = (char*)ctx->ws;
  int32_t* kidx = (int32_t*)(ws + cv.kidx);
  int32_t* kcnt = (int32_t*)(ws + cv.kcnt);
  uint8_t* sel = (uint8_t*)(ws + cv.sel);
  hipStream_t st = (hipStream_t)stream;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  if ((rc = launch_lists_from_mask(block_mask, (int)(heads * nq), (int)nk, kidx, kcnt, sel, st))) return rc;
  AttnArgs a = make_args(q, lq, k, v, lk, heads, kidx, kcnt, sel, (int)nk, (int)nk, plain_key_map(), o, esize(dtype));
  if ((rc = attach_order(ctx, a, nk))) return rc;
  return launch_attention(dtype, mode == FVSR_ATTN_DENSE, a, st);
}

// ---------------------------------------------------------------------------------------------------------------
// window layout
// ---------------------------------------------------------------------------------------------------------------
static int window_layout(int dtype, const void* x, void* out, int f, int h, int w, int channels, void* stream,
                         bool to_windows) {
  FVSR_REQUIRE(valid_dtype(dtype), FVSR_ERR_INVALID_ARG, "dtype must be FVSR_DTYPE_F32 or FVSR_DTYPE_BF16");
  FVSR_REQUIRE(x && out, FVSR_ERR_INVALID_ARG, "x and out must be non-NULL");
  FVSR_REQUIRE(f > 0 && h > 0 && w > 0 && f % 2 == 0 && h % 8 == 0 && w % 8 == 0, FVSR_ERR_INVALID_ARG,
               "window (2, 8, 8) must tile (f, h, w)");
  FVSR_REQUIRE(channels > 0 && (channels * esize(dtype)) % 16 == 0, FVSR_ERR_INVALID_ARG,
               "channels * element size must be a multiple of 16 bytes");
  return launch_window_layout(dtype, x, out, f, h, w, channels, to_windows, (hipStream_t)stream);
}

int fvsr_window_partition(int dtype, const void* x, void* out, int f, int h, int w, int channels, void* stream) {
  return window_layout(dtype, x, out, f, h, w, channels, stream, true);
}

int fvsr_window_reverse(int dtype, const void* x, void* out, int f, int h, int w, int channels, void* stream) {
  return window_layout(dtype, x, out, f, h, w, channels, stream, false);
}

// ---------------------------------------------------------------------------------------------------------------
// fused QKV epilogue (RMSNorm + RoPE + window partition)
// ---------------------------------------------------------------------------------------------------------------
size_t fvsr_rope_tables_size(void) { return (size_t)rope_table_floats(); }

int fvsr_rope_tables(double theta, float* out, size_t n_floats) {
  FVSR_REQUIRE(out != nullptr, FVSR_ERR_INVALID_ARG, "out is NULL");
  FVSR_REQUIRE(n_floats >= (size_t)rope_table_floats(), FVSR_ERR_INVALID_ARG,
               "out holds fewer than fvsr_rope_tables_size() floats");
  FVSR_REQUIRE(theta > 1.0, FVSR_ERR_INVALID_ARG, "theta must be > 1");
  rope_tables_host(theta, out);
  return FVSR_OK;
}

static int check_epilogue(int dtype, const void* q, const void* k, const void* v, int f, int h, int w, int heads,
                          int t0, const void* wq, const void* wk, float eps, const float* rope) {
  FVSR_REQUIRE(valid_dtype(dtype), FVSR_ERR_INVALID_ARG, "dtype must be FVSR_DTYPE_F32 or FVSR_DTYPE_BF16");
  FVSR_REQUIRE(q && k && v && wq && wk && rope, FVSR_ERR_INVALID_ARG,
               "q, k, v, the norm weights and the RoPE tables must be non-NULL");
  FVSR_REQUIRE(f > 0 && h > 0 && w > 0 && f % 2 == 0 && h % 8 == 0 && w % 8 == 0, FVSR_ERR_INVALID_ARG,
               "window (2, 8, 8) must tile (f, h, w)");
  int rc = check_heads(heads);
  if (rc) return rc;
  FVSR_REQUIRE(heads * 128 * esize(dtype) / 16 <= 384, FVSR_ERR_UNSUPPORTED,
               "the epilogue handles at most 384 16-byte vectors per token (64 lanes x 6)");
  FVSR_REQUIRE(t0 >= 0 && t0 + f <= 1024 && h <= 1024 && w <= 1024, FVSR_ERR_INVALID_ARG,
               "token positions must lie inside the 1024-row RoPE tables");
  FVSR_REQUIRE(eps >= 0.f, FVSR_ERR_INVALID_ARG, "eps must be >= 0");
  return FVSR_OK;
}

int fvsr_qkv_epilogue(fvsr_ctx* ctx, int dtype, const void* q, const void* k, const void* v, int f, int h, int w,
                      int heads, int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                      const float* rope_tables, void* q_out, void* k_out, void* v_out, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_epilogue(dtype, q, k, v, f, h, w, heads, t0, norm_q_weight, norm_k_weight, eps, rope_tables);
  if (rc) return rc;
  FVSR_REQUIRE(q_out && k_out && v_out, FVSR_ERR_INVALID_ARG, "q_out, k_out and v_out must be non-NULL");
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_qkv_epilogue(dtype, q, k, v, f, h, w, heads * 128, t0, norm_q_weight, norm_k_weight, eps,
                             rope_tables, q_out, k_out, v_out, 0, 1, 1 << 30, 0, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// KV ring
// ---------------------------------------------------------------------------------------------------------------
int fvsr_kv_ring_create(fvsr_ctx* ctx, int dtype, int layers, int heads, int bh, int bw, int capacity_slices,
                        int kv_len, fvsr_kv_ring** out) {
  FVSR_REQUIRE(out != nullptr, FVSR_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  FVSR_REQUIRE(valid_dtype(dtype), FVSR_ERR_INVALID_ARG, "dtype must be FVSR_DTYPE_F32 or FVSR_DTYPE_BF16");
  int rc = check_heads(heads);
  if (rc) return rc;
  FVSR_REQUIRE(layers > 0 && bh > 0 && bw > 0, FVSR_ERR_INVALID_ARG, "layers, bh, bw must be > 0");
  FVSR_REQUIRE(kv_len > 0 && capacity_slices > kv_len, FVSR_ERR_INVALID_ARG,
               "need kv_len > 0 and capacity_slices > kv_len (the window is read before the trim)");
  fvsr_kv_ring* r = new (std::nothrow) fvsr_kv_ring();
  FVSR_REQUIRE(r != nullptr, FVSR_ERR_OUT_OF_MEMORY, "ring allocation failed");
  r->ctx = ctx;
  r->dtype = dtype; r->layers = layers; r->heads = heads; r->bh = bh; r->bw = bw; r->s = bh * bw;
  r->capacity = capacity_slices; r->kv_len = kv_len; r->C = heads * kHeadDim;
  r->head.assign(layers, 0);
  r->count.assign(layers, 0);
  const size_t kv_bytes = (size_t)layers * r->layer_tokens() * r->C * esize(dtype);
  if ((int64_t)r->layer_tokens() * r->C * esize(dtype) >= ((int64_t)1 << 31)) {
    delete r;
    return set_error(FVSR_ERR_UNSUPPORTED, "a ring layer above 2 GiB is not supported (32-bit buffer offsets)");
  }
  const size_t pooled_bytes = (size_t)layers * capacity_slices * r->s * r->C * sizeof(float);
  const size_t partial_bytes = (size_t)capacity_slices * r->s * kPoolParts * r->C * sizeof(float);
  if (hipSetDevice(ctx->device) != hipSuccess || hipMalloc(&r->k, kv_bytes) != hipSuccess ||
      hipMalloc(&r->v, kv_bytes) != hipSuccess || hipMalloc((void**)&r->pooled, pooled_bytes) != hipSuccess ||
      hipMalloc((void**)&r->partial, partial_bytes) != hipSuccess) {
    if (r->k) (void)hipFree(r->k);
    if (r->v) (void)hipFree(r->v);
    if (r->pooled) (void)hipFree(r->pooled);
    if (r->partial) (void)hipFree(r->partial);
    delete r;
    return set_error(FVSR_ERR_OUT_OF_MEMORY, "ring allocation of 2 x " + std::to_string(kv_bytes) + " bytes failed");
  }
  *out = r;
  return FVSR_OK;
}

int fvsr_kv_ring_destroy(fvsr_kv_ring* r) {
  if (!r) return FVSR_OK;
  (void)hipSetDevice(r->ctx->device);
  (void)hipFree(r->k);
  (void)hipFree(r->v);
  (void)hipFree(r->pooled);
  (void)hipFree(r->partial);
  delete r;
  return FVSR_OK;
}

int fvsr_kv_ring_reset(fvsr_kv_ring* r) {
  FVSR_REQUIRE(r != nullptr, FVSR_ERR_INVALID_ARG, "ring is NULL");
  std::fill(r->head.begin(), r->head.end(), 0);
  std::fill(r->count.begin(), r->count.end(), 0);
  return FVSR_OK;
}

// a layer's ring position before a layer call, so that a call failing after its append leaves the ring as it
// found it (the slots the append wrote are free again) instead of holding one slice more than the trim rule allows
struct RingMark {
  int head, count;
};
static RingMark ring_mark(const fvsr_kv_ring* r, int layer) { return RingMark{r->head[layer], r->count[layer]}; }
static int ring_rewind(fvsr_kv_ring* r, int layer, RingMark m, int rc) {
  r->head[layer] = m.head;
  r->count[layer] = m.count;
  return rc;
}

static int check_layer(const fvsr_kv_ring* r, int layer) {
  FVSR_REQUIRE(r != nullptr, FVSR_ERR_INVALID_ARG, "ring is NULL");
  FVSR_REQUIRE(layer >= 0 && layer < r->layers, FVSR_ERR_INVALID_ARG, "layer out of range");
  return FVSR_OK;
}

int fvsr_kv_ring_append(fvsr_kv_ring* r, int layer, const void* k_new, const void* v_new, int n_slices, int layout,
                        void* stream) {
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(k_new && v_new, FVSR_ERR_INVALID_ARG, "k_new and v_new must be non-NULL");
  FVSR_REQUIRE(n_slices > 0, FVSR_ERR_INVALID_ARG, "n_slices must be > 0");
  FVSR_REQUIRE(layout == FVSR_LAYOUT_WINDOWS || layout == FVSR_LAYOUT_GRID, FVSR_ERR_INVALID_ARG, "bad layout");
  FVSR_REQUIRE(r->count[layer] + n_slices <= r->capacity, FVSR_ERR_CAPACITY,
               "append of " + std::to_string(n_slices) + " slices exceeds the ring capacity of " +
                   std::to_string(r->capacity) + " (held " + std::to_string(r->count[layer]) + ")");
  FVSR_HIP_CHECK(hipSetDevice(r->ctx->device));
  const int slot0 = (r->head[layer] + r->count[layer]) % r->capacity;
  rc = launch_ring_append(r->dtype, k_new, v_new, n_slices * r->s, r->C, layout == FVSR_LAYOUT_GRID, r->bh, r->bw,
                          slot0, r->capacity, r->layer_k(layer), r->layer_v(layer), r->head_stride(),
                          r->layer_pooled(layer), r->partial, (hipStream_t)stream);
  if (rc) return rc;
  r->count[layer] += n_slices;
  return FVSR_OK;
}

}  // extern "C"

// The ring append of fvsr_kv_ring_append_qkv. With q_pooled set (the layer call), the block means of the written
// queries ride in the same pooling launch as the new keys' (to q_pooled), which also clears the selection
// histogram `hist` (nhist words).
static int append_qkv_impl(fvsr_kv_ring* r, int layer, const void* q, const void* k, const void* v, int n_slices,
                           int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                           const float* rope_tables, void* q_out, hipStream_t stream, float* q_pooled = nullptr,
                           unsigned* hist = nullptr, int64_t nhist = 0) {
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(n_slices > 0, FVSR_ERR_INVALID_ARG, "n_slices must be > 0");
  rc = check_epilogue(r->dtype, q, k, v, 2 * n_slices, 8 * r->bh, 8 * r->bw, r->heads, t0, norm_q_weight,
                      norm_k_weight, eps, rope_tables);
  if (rc) return rc;
  FVSR_REQUIRE(q_out != nullptr, FVSR_ERR_INVALID_ARG, "q_out is NULL");
  FVSR_REQUIRE(r->count[layer] + n_slices <= r->capacity, FVSR_ERR_CAPACITY,
               "append of " + std::to_string(n_slices) + " slices exceeds the ring capacity of " +
                   std::to_string(r->capacity) + " (held " + std::to_string(r->count[layer]) + ")");
  FVSR_HIP_CHECK(hipSetDevice(r->ctx->device));
  const int slot0 = (r->head[layer] + r->count[layer]) % r->capacity;
  const int nb = n_slices * r->s;
  rc = launch_qkv_epilogue(r->dtype, q, k, v, 2 * n_slices, 8 * r->bh, 8 * r->bw, r->C, t0, norm_q_weight,
                           norm_k_weight, eps, rope_tables, q_out, r->layer_k(layer), r->layer_v(layer), slot0,
                           r->capacity, r->s, r->head_stride(), stream);
  if (rc) return rc;
  // pooled keys of the new slots, as for plain buffers: block means over the slots up to the end of the ring, then
  // the wrapped remainder from slot 0 (and the queries' means, and the histogram reset), one launch; a slot's first
  // token in head 0's region of the (head-major) ring is s * 128 rows of 128 elements past the previous slot's
  const int first = std::min(n_slices, r->capacity - slot0);
  const size_t slot_bytes = (size_t)r->s * kBlock * kHeadDim * esize(r->dtype);
  const int64_t lq = (int64_t)nb * kBlock;
  PoolMean jobs[3];
  int nj = 0;
  jobs[nj++] = PoolMean{r->layer_k(layer) + slot0 * slot_bytes, (int64_t)first * r->s * kBlock,
                        r->layer_pooled(layer), 0, slot0, r->capacity, r->s, r->head_stride()};
  if (first < n_slices)
    jobs[nj++] = PoolMean{r->layer_k(layer), (int64_t)(n_slices - first) * r->s * kBlock, r->layer_pooled(layer), 0,
                          0, r->capacity, r->s, r->head_stride()};
  if (q_pooled) jobs[nj++] = PoolMean{q_out, lq, q_pooled, 0, 0, 1, 1 << 30, 0};
  if ((rc = launch_pool_mean(r->dtype, jobs, nj, r->C, hist, nhist, stream))) return rc;
  r->count[layer] += n_slices;
  return FVSR_OK;
}

extern "C" {

int fvsr_kv_ring_append_qkv(fvsr_kv_ring* r, int layer, const void* q, const void* k, const void* v, int n_slices,
                            int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                            const float* rope_tables, void* q_out, void* stream) {
  return append_qkv_impl(r, layer, q, k, v, n_slices, t0, norm_q_weight, norm_k_weight, eps, rope_tables, q_out,
                         (hipStream_t)stream);
}

int fvsr_kv_ring_evict(fvsr_kv_ring* r, int layer) {
  int rc = check_layer(r, layer);
  if (rc) return rc;
  // DiT.swift:532-538: more than kv_len slices held -> drop exactly one (the oldest)
  if (r->count[layer] > r->kv_len) {
    r->head[layer] = (r->head[layer] + 1) % r->capacity;
    r->count[layer] -= 1;
  }
  return FVSR_OK;
}

int fvsr_kv_ring_slices(const fvsr_kv_ring* r, int layer, int* out) {
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(out != nullptr, FVSR_ERR_INVALID_ARG, "out is NULL");
  *out = r->count[layer];
  return FVSR_OK;
}

int fvsr_kv_ring_read(fvsr_kv_ring* r, int layer, void* k_out, void* v_out, void* stream) {
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(k_out && v_out, FVSR_ERR_INVALID_ARG, "k_out and v_out must be non-NULL");
  FVSR_HIP_CHECK(hipSetDevice(r->ctx->device));
  return launch_ring_read(r->dtype, r->layer_k(layer), r->layer_v(layer), k_out, v_out, r->count[layer] * r->s,
                          r->C, r->head_stride(), r->map(layer), (hipStream_t)stream);
}

int fvsr_lcsa_select_ring(fvsr_ctx* ctx, fvsr_kv_ring* r, int layer, const void* qW, int64_t lq, int q_slices,
                          const uint8_t* local_dev, int topk, float* mask_out, float* probs_out, int32_t* kidx_out,
                          int32_t* kcnt_out, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(r->count[layer] > 0, FVSR_ERR_STATE, "ring layer holds no keys");
  FVSR_REQUIRE(qW && local_dev && kidx_out && kcnt_out, FVSR_ERR_INVALID_ARG,
               "qW, local, kidx and kcnt must be non-NULL");
  FVSR_REQUIRE(lq > 0 && q_slices > 0, FVSR_ERR_INVALID_ARG, "lq and q_slices must be > 0");
  const int nk = r->count[layer] * r->s;
  return select_impl(ctx, r->dtype, qW, lq, r->layer_pooled(layer), true, nullptr, (int64_t)nk * kBlock,
                     r->map(layer), nk, r->heads, q_slices, r->s, local_dev, topk, mask_out, probs_out, kidx_out,
                     kcnt_out, nullptr, (hipStream_t)stream);
}

static int attention_ring_impl(fvsr_ctx* ctx, fvsr_kv_ring* r, int layer, const void* q, int64_t lq,
                               const int32_t* kidx, const int32_t* kcnt, int nk_stride, const uint8_t* sel,
                               bool dense, void* o, hipStream_t stream, bool o_grid = false) {
  const int nk = r->count[layer] * r->s;
  AttnArgs a = make_args(q, lq, r->layer_k(layer), r->layer_v(layer), (int64_t)nk * kBlock, r->heads, kidx, kcnt,
                         sel, nk_stride, nk, r->map(layer), o, esize(r->dtype));
  a.kv_head_stride = r->head_stride();   // head-major
  a.kv_ld = kHeadDim;
  a.kv_bytes = (int64_t)r->heads * r->head_stride() * esize(r->dtype);
  if (o_grid) {   // whole windows of the ring's (8 bh, 8 bw) grid: write o in natural token order
    a.o_nbh = r->bh;
    a.o_nbw = r->bw;
  }
  int rc = attach_order(ctx, a, nk);
  if (rc) return rc;
  return launch_attention(r->dtype, dense, a, stream);
}

int fvsr_lcsa_attention_ring(fvsr_ctx* ctx, fvsr_kv_ring* r, int layer, const void* q, int64_t lq,
                             const int32_t* kidx, const int32_t* kcnt, int nk_stride, int mode, void* o,
                             void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(r->count[layer] > 0, FVSR_ERR_STATE, "ring layer holds no keys");
  FVSR_REQUIRE(q && kidx && kcnt && o, FVSR_ERR_INVALID_ARG, "q, kidx, kcnt and o must be non-NULL");
  FVSR_REQUIRE(lq > 0 && nk_stride > 0, FVSR_ERR_INVALID_ARG, "lq and nk_stride must be > 0");
  FVSR_REQUIRE(mode == FVSR_ATTN_KERNEL || mode == FVSR_ATTN_DENSE, FVSR_ERR_INVALID_ARG,
               "mode must be FVSR_ATTN_KERNEL or FVSR_ATTN_DENSE");
  hipStream_t st = (hipStream_t)stream;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  const int64_t nq = ceil_div(lq, kBlock);
  const int nk = r->count[layer] * r->s;
  uint8_t* sel = nullptr;
  if (mode == FVSR_ATTN_DENSE) {
    const Carve cv = carve(r->heads, nq, nk, r->C);
    if ((rc = ensure_ws(ctx, cv.total))) return rc;
    sel = (uint8_t*)((char*)ctx->ws + cv.sel);
    if ((rc = launch_sel_from_lists(kidx, kcnt, (int)(r->heads * nq), nk_stride, nk, sel, st))) return rc;
  }
  return attention_ring_impl(ctx, r, layer, q, lq, kidx, kcnt, nk_stride, sel, mode == FVSR_ATTN_DENSE, o, st);
}

int fvsr_lcsa_layer(fvsr_ctx* ctx, fvsr_kv_ring* r, int layer, const void* qW, int64_t lq, const void* k_new,
                    const void* v_new, int n_new_slices, int layout, int q_slices, const uint8_t* local_dev,
                    int topk, int mode, void* o, float* mask_out, float* probs_out, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(qW && o && local_dev, FVSR_ERR_INVALID_ARG, "qW, o and local must be non-NULL");
  FVSR_REQUIRE(mode == FVSR_ATTN_AUTO || mode == FVSR_ATTN_KERNEL || mode == FVSR_ATTN_DENSE,
               FVSR_ERR_INVALID_ARG, "bad attention mode");
  FVSR_REQUIRE(lq > 0 && q_slices > 0 && topk >= 0, FVSR_ERR_INVALID_ARG, "lq, q_slices must be > 0, topk >= 0");
  FVSR_REQUIRE(ceil_div(lq, kBlock) == (int64_t)q_slices * r->s, FVSR_ERR_INVALID_ARG,
               "ceil(lq/128) must equal q_slices * s");
  FVSR_REQUIRE(r->count[layer] + n_new_slices <= r->capacity, FVSR_ERR_CAPACITY,
               "append would exceed the ring capacity");
  const int nk_after = (r->count[layer] + n_new_slices) * r->s;
  FVSR_REQUIRE(nk_after <= kMaxSelectKeyBlocks, FVSR_ERR_UNSUPPORTED, "too many key blocks for selection");
  hipStream_t st = (hipStream_t)stream;
  // workspace first, so that no allocation happens between the append and the evict
  const int64_t nq = ceil_div(lq, kBlock);
  const Carve cv = carve(r->heads, nq, nk_after, r->C);
  if ((rc = ensure_ws(ctx, cv.total))) return rc;
  const RingMark mark = ring_mark(r, layer);
  if ((rc = fvsr_kv_ring_append(r, layer, k_new, v_new, n_new_slices, layout, stream))) return rc;
  const int nk = r->count[layer] * r->s;
  char* ws = (char*)ctx->ws;
  int32_t* kidx = (int32_t*)(ws + cv.kidx);
  int32_t* kcnt = (int32_t*)(ws + cv.kcnt);
  uint8_t* sel = (uint8_t*)(ws + cv.sel);
  rc = select_impl(ctx, r->dtype, qW, lq, r->layer_pooled(layer), true, nullptr, (int64_t)nk * kBlock,
                   r->map(layer), nk, r->heads, q_slices, r->s, local_dev, topk, mask_out, probs_out, kidx, kcnt,
                   sel, st);
  if (rc) return ring_rewind(r, layer, mark, rc);
  int use = mode;
  if (use == FVSR_ATTN_AUTO) fvsr_attention_mode_auto(topk, r->s, nk, kAutoThreshold, nullptr, &use);
  rc = attention_ring_impl(ctx, r, layer, qW, lq, kidx, kcnt, nk, sel, use == FVSR_ATTN_DENSE, o, st);
  if (rc) return ring_rewind(r, layer, mark, rc);
  return fvsr_kv_ring_evict(r, layer);
}

int fvsr_lcsa_layer_qkv(fvsr_ctx* ctx, fvsr_kv_ring* r, int layer, const void* q, const void* k, const void* v,
                        int n_new_slices, int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                        const float* rope_tables, const uint8_t* local_dev, int topk, int mode, void* q_work, void* o,
                        float* mask_out, float* probs_out, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_layer(r, layer);
  if (rc) return rc;
  FVSR_REQUIRE(q_work && o && local_dev, FVSR_ERR_INVALID_ARG, "q_work, o and local must be non-NULL");
  FVSR_REQUIRE(mode == FVSR_ATTN_AUTO || mode == FVSR_ATTN_KERNEL || mode == FVSR_ATTN_DENSE,
               FVSR_ERR_INVALID_ARG, "bad attention mode");
  FVSR_REQUIRE(n_new_slices > 0 && topk >= 0, FVSR_ERR_INVALID_ARG, "n_new_slices must be > 0, topk >= 0");
  FVSR_REQUIRE(r->count[layer] + n_new_slices <= r->capacity, FVSR_ERR_CAPACITY,
               "append would exceed the ring capacity");
  const int nk_after = (r->count[layer] + n_new_slices) * r->s;
  FVSR_REQUIRE(nk_after <= kMaxSelectKeyBlocks, FVSR_ERR_UNSUPPORTED, "too many key blocks for selection");
  hipStream_t st = (hipStream_t)stream;
  // the chunk's queries: q_slices = n_new_slices slices of s windows (DiT.swift:478-485: seqlen = f / 2)
  const int q_slices = n_new_slices;
  const int64_t lq = (int64_t)q_slices * r->s * kBlock;
  const int64_t nq = (int64_t)q_slices * r->s;
  const Carve cv = carve(r->heads, nq, nk_after, r->C);
  if ((rc = ensure_ws(ctx, cv.total))) return rc;
  char* ws = (char*)ctx->ws;
  const RingMark mark = ring_mark(r, layer);
  // the pooled queries and the histogram reset ride in the append's pooling launches
  if ((rc = append_qkv_impl(r, layer, q, k, v, n_new_slices, t0, norm_q_weight, norm_k_weight, eps, rope_tables,
                            q_work, st, (float*)(ws + cv.pq), (unsigned*)(ws + cv.hist),
                            (int64_t)(hist12_bytes(r->heads, q_slices) / sizeof(unsigned)))))
    return rc;
  const int nk = r->count[layer] * r->s;
  int32_t* kidx = (int32_t*)(ws + cv.kidx);
  int32_t* kcnt = (int32_t*)(ws + cv.kcnt);
  uint8_t* sel = (uint8_t*)(ws + cv.sel);
  rc = select_impl(ctx, r->dtype, q_work, lq, r->layer_pooled(layer), true, nullptr, (int64_t)nk * kBlock,
                   r->map(layer), nk, r->heads, q_slices, r->s, local_dev, topk, mask_out, probs_out, kidx, kcnt,
                   sel, st, true);
  if (rc) return ring_rewind(r, layer, mark, rc);
  int use = mode;
  if (use == FVSR_ATTN_AUTO) fvsr_attention_mode_auto(topk, r->s, nk, kAutoThreshold, nullptr, &use);
  rc = attention_ring_impl(ctx, r, layer, q_work, lq, kidx, kcnt, nk, sel, use == FVSR_ATTN_DENSE, o, st, true);
  if (rc) return ring_rewind(r, layer, mark, rc);
  return fvsr_kv_ring_evict(r, layer);
}


// ---------------------------------------------------------------------------------------------------------------
// (f3) the dense parts of the DiT block
// ---------------------------------------------------------------------------------------------------------------
}  // extern "C"

static int ensure_blas(fvsr_ctx* ctx) {
  if (ctx->blas) return FVSR_OK;
  return blas_create(ctx->device, &ctx->blas);
}

static int ensure_block_ws(fvsr_ctx* ctx, size_t bytes) {
  if (ctx->block_ws_bytes >= bytes) return FVSR_OK;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  if (ctx->block_ws) FVSR_HIP_CHECK(hipFree(ctx->block_ws));
  ctx->block_ws = nullptr;
  ctx->block_ws_bytes = 0;
  if (hipMalloc(&ctx->block_ws, bytes) != hipSuccess) {
    ctx->block_ws = nullptr;
    return set_error(FVSR_ERR_OUT_OF_MEMORY, "block workspace allocation of " + std::to_string(bytes) + " bytes failed");
  }
  ctx->block_ws_bytes = bytes;
  return FVSR_OK;
}

// activations of one block call: L tokens of C channels, FFN width F, cross-attention lists for nq query blocks
struct BlockCarve {
  size_t mod, in, q, k, v, qw, attn, tmp, ffn, kidx, kcnt, total;
};
static BlockCarve block_carve(int64_t L, int C, int F, int64_t nq, int nkc) {
  BlockCarve c;
  size_t off = 0;
  const size_t tok = align256((size_t)L * C * 2);
  c.mod = off; off += align256((size_t)6 * C * 2);
  c.in = off; off += tok;
  c.q = off; off += tok;
  c.k = off; off += tok;
  c.v = off; off += tok;
  c.qw = off; off += tok;
  c.attn = off; off += tok;
  c.tmp = off; off += tok;
  c.ffn = off; off += align256((size_t)L * F * 2);
  c.kidx = off; off += align256((size_t)nq * nkc * 4);
  c.kcnt = off; off += align256((size_t)nq * 4);
  c.total = off;
  return c;
}

static int check_block_weights(const fvsr_dit_block_weights* w, bool need_self, bool need_cross_kv) {
  FVSR_REQUIRE(w != nullptr, FVSR_ERR_INVALID_ARG, "weights is NULL");
  if (need_self)
    FVSR_REQUIRE(w->modulation && w->q_weight && w->k_weight && w->v_weight && w->o_weight && w->norm_q_weight &&
                     w->norm_k_weight && w->cross_q_weight && w->cross_o_weight && w->cross_norm_q_weight &&
                     w->norm3_weight && w->ffn1_weight && w->ffn2_weight && w->cross_k && w->cross_v,
                 FVSR_ERR_INVALID_ARG, "a weight pointer of the block is NULL (biases may be NULL)");
  if (need_cross_kv)
    FVSR_REQUIRE(w->cross_k_weight && w->cross_v_weight && w->cross_norm_k_weight, FVSR_ERR_INVALID_ARG,
                 "cross k / v / norm_k weights must be non-NULL");
  FVSR_REQUIRE(w->ffn_dim > 0 && w->ffn_dim % 8 == 0, FVSR_ERR_INVALID_ARG, "ffn_dim must be a positive multiple of 8");
  return FVSR_OK;
}

extern "C" {

int fvsr_ctx_reserve_block(fvsr_ctx* ctx, int heads, int64_t tokens, int ffn_dim, int ctx_len, int64_t key_tokens) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_heads(heads);
  if (rc) return rc;
  FVSR_REQUIRE(tokens > 0 && ffn_dim > 0 && ctx_len > 0 && key_tokens > 0, FVSR_ERR_INVALID_ARG,
               "tokens, ffn_dim, ctx_len and key_tokens must be > 0");
  const int C = heads * kHeadDim;
  const int64_t nq = ceil_div(tokens, kBlock);
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  if ((rc = ensure_blas(ctx))) return rc;
  const BlockCarve bc = block_carve(tokens, C, ffn_dim, (int64_t)heads * nq, (int)ceil_div(ctx_len, kBlock));
  if ((rc = ensure_block_ws(ctx, bc.total))) return rc;
  // the layer call's selection and attention over the ring window, and the cross-attention over the context
  const int64_t lk = std::max<int64_t>(key_tokens, ctx_len);
  return ensure_ws(ctx, carve(heads, nq, ceil_div(lk, kBlock), C).total);
}

size_t fvsr_ctx_block_workspace_bytes(const fvsr_ctx* ctx) { return ctx ? ctx->block_ws_bytes : 0; }

int fvsr_linear(fvsr_ctx* ctx, const void* x, int64_t rows, int in_features, const void* weight, int out_features,
                const void* bias, int gelu, void* y, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  FVSR_REQUIRE(x && weight && y, FVSR_ERR_INVALID_ARG, "x, weight and y must be non-NULL");
  FVSR_REQUIRE(rows >= 0 && in_features > 0 && out_features > 0, FVSR_ERR_INVALID_ARG, "bad GEMM shape");
  FVSR_REQUIRE(in_features % 8 == 0 && out_features % 8 == 0, FVSR_ERR_UNSUPPORTED,
               "in_features and out_features must be multiples of 8");
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  int rc = ensure_blas(ctx);
  if (rc) return rc;
  return linear_bf16(ctx->blas, x, rows, in_features, weight, out_features, bias, gelu ? 1 : 0, y,
                     (hipStream_t)stream);
}

int fvsr_dit_cross_kv(fvsr_ctx* ctx, const fvsr_dit_block_weights* w, int heads, const void* context, int ctx_len,
                      float eps, void* k_out, void* v_out, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_block_weights(w, false, true);
  if (rc) return rc;
  if ((rc = check_heads(heads))) return rc;
  FVSR_REQUIRE(context && k_out && v_out && ctx_len > 0, FVSR_ERR_INVALID_ARG, "context, k_out, v_out, ctx_len");
  const int C = heads * kHeadDim;
  hipStream_t st = (hipStream_t)stream;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  if ((rc = ensure_blas(ctx))) return rc;
  // k = normK(k(ctx)), v = v(ctx) (CrossAttention.initCache, DiT.swift:346-350); k_out doubles as the scratch
  if ((rc = linear_bf16(ctx->blas, context, ctx_len, C, w->cross_k_weight, C, w->cross_k_bias, 0, k_out, st))) return rc;
  if ((rc = launch_rms_norm(k_out, ctx_len, C, eps, w->cross_norm_k_weight, k_out, st))) return rc;
  return linear_bf16(ctx->blas, context, ctx_len, C, w->cross_v_weight, C, w->cross_v_bias, 0, v_out, st);
}

int fvsr_dit_block(fvsr_ctx* ctx, fvsr_kv_ring* r, int layer, const fvsr_dit_block_weights* w, const void* t_mod,
                   void* x, int n_new_slices, int t0, float eps, const float* rope_tables, const uint8_t* local_dev,
                   int topk, int mode, void* stream) {
  FVSR_REQUIRE(ctx != nullptr, FVSR_ERR_INVALID_ARG, "ctx is NULL");
  int rc = check_layer(r, layer);
  if (rc) return rc;
  if ((rc = check_block_weights(w, true, false))) return rc;
  FVSR_REQUIRE(r->dtype == FVSR_DTYPE_BF16, FVSR_ERR_UNSUPPORTED, "the DiT block runs in bf16");
  FVSR_REQUIRE(t_mod && x && rope_tables && local_dev, FVSR_ERR_INVALID_ARG, "t_mod, x, rope_tables, local");
  FVSR_REQUIRE(n_new_slices > 0 && w->ctx_len > 0, FVSR_ERR_INVALID_ARG, "n_new_slices and ctx_len must be > 0");
  const int C = r->C, F = w->ffn_dim;
  const int64_t L = (int64_t)n_new_slices * r->s * kBlock;   // 2 * n_new_slices frames of 8bh x 8bw tokens
  const int64_t nq = ceil_div(L, kBlock);
  const int nkc = (int)ceil_div(w->ctx_len, kBlock);
  hipStream_t st = (hipStream_t)stream;
  FVSR_HIP_CHECK(hipSetDevice(ctx->device));
  if ((rc = ensure_blas(ctx))) return rc;
  const BlockCarve bc = block_carve(L, C, F, (int64_t)r->heads * nq, nkc);
  if ((rc = ensure_block_ws(ctx, bc.total))) return rc;
  char* ws = (char*)ctx->block_ws;
  bf16* mod = (bf16*)(ws + bc.mod);
  void *in = ws + bc.in, *q = ws + bc.q, *k = ws + bc.k, *v = ws + bc.v, *qw = ws + bc.qw, *attn = ws + bc.attn;
  void *tmp = ws + bc.tmp, *ffn = ws + bc.ffn;
  int32_t* kidx = (int32_t*)(ws + bc.kidx);
  int32_t* kcnt = (int32_t*)(ws + bc.kcnt);
  auto row = [&](int i) -> const void* { return mod + (size_t)i * C; };   // shift/scale/gate MSA, shift/scale/gate MLP
  void* blas = ctx->blas;
  // mod = modulation + t_mod; inX = norm1(x) * (1 + scaleMSA) + shiftMSA (DiT.swift:495-498)
  if ((rc = launch_modulation(w->modulation, t_mod, mod, C, st))) return rc;
  if ((rc = launch_residual_norm(x, nullptr, nullptr, L, C, eps, nullptr, nullptr, row(1), row(0), in, st))) return rc;
  // self-attention: projections, the LCSA layer call (norm + RoPE + partition + ring + select + attend + evict,
  // output in natural order), o projection (DiT.swift:500-539)
  if ((rc = linear_bf16(blas, in, L, C, w->q_weight, C, w->q_bias, 0, q, st))) return rc;
  if ((rc = linear_bf16(blas, in, L, C, w->k_weight, C, w->k_bias, 0, k, st))) return rc;
  if ((rc = linear_bf16(blas, in, L, C, w->v_weight, C, w->v_bias, 0, v, st))) return rc;
  if ((rc = fvsr_lcsa_layer_qkv(ctx, r, layer, q, k, v, n_new_slices, t0, w->norm_q_weight, w->norm_k_weight, eps,
                                rope_tables, local_dev, topk, mode, qw, attn, nullptr, nullptr, stream)))
    return rc;
  if ((rc = linear_bf16(blas, attn, L, C, w->o_weight, C, w->o_bias, 0, tmp, st))) return rc;
  // x = x + gateMSA * o; caIn = norm3(x) (affine) (DiT.swift:541-542)
  if ((rc = launch_residual_norm(x, tmp, row(2), L, C, eps, w->norm3_weight, w->norm3_bias, nullptr, nullptr, in, st)))
    return rc;
  // cross-attention: q = normQ(q(caIn)); SDPA over the cached context K/V (every context block listed, scale
  // 1/sqrt(128)); o projection (DiT.swift:352-361)
  if ((rc = linear_bf16(blas, in, L, C, w->cross_q_weight, C, w->cross_q_bias, 0, q, st))) return rc;
  if ((rc = launch_rms_norm(q, L, C, eps, w->cross_norm_q_weight, q, st))) return rc;
  if ((rc = launch_full_lists((int)(r->heads * nq), nkc, kidx, kcnt, st))) return rc;
  if ((rc = fvsr_lcsa_attention(ctx, FVSR_DTYPE_BF16, q, L, w->cross_k, w->cross_v, w->ctx_len, r->heads, kidx, kcnt,
                                nkc, attn, stream)))
    return rc;
  if ((rc = linear_bf16(blas, attn, L, C, w->cross_o_weight, C, w->cross_o_bias, 0, tmp, st))) return rc;
  // x = x + caOut; inF = norm2(x) * (1 + scaleMLP) + shiftMLP (DiT.swift:545-546)
  if ((rc = launch_residual_norm(x, tmp, nullptr, L, C, eps, nullptr, nullptr, row(4), row(3), in, st))) return rc;
  // FFN: Linear(C, F) + GELU(tanh) fused, Linear(F, C); x = x + gateMLP * ffn (DiT.swift:547)
  if ((rc = linear_bf16(blas, in, L, C, w->ffn1_weight, F, w->ffn1_bias, 1, ffn, st))) return rc;
  if ((rc = linear_bf16(blas, ffn, L, F, w->ffn2_weight, C, w->ffn2_bias, 0, tmp, st))) return rc;
  return launch_residual_norm(x, tmp, row(5), L, C, eps, nullptr, nullptr, nullptr, nullptr, nullptr, st);
}

}  // extern "C"
