/* fvsr_lcsa.h — C ABI of the MI355X (gfx950) LCSA path: FlashVSR's locality-constrained block-sparse
 * self-attention as called from the DiT self-attention block.
 *
 * Every entry point replaces one piece of the reference's call surface (xocialize/mlx-flashvsr-swift); the
 * reference function is cited beside each declaration. Conventions:
 *   - plain pointers and sizes only; device pointers are HIP device memory owned by the caller;
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream); no entry point synchronises the
 *     host, except that a call which needs more context workspace than the context holds grows it (hipFree +
 *     hipMalloc, and hipFree synchronises the device): fvsr_ctx_reserve / fvsr_ctx_reserve_block size it up front,
 *     after which calls of at most that size allocate nothing;
 *   - every function returns an fvsr_status; on failure fvsr_last_error() returns a message for the calling thread;
 *   - token buffers are token-major (L, H*128) in window order (128-token windows ordered (nf, nh, nw), tokens in a
 *     window ordered (wf, wh, ww)), exactly the reference's (1, L, H*128) layout (DiT.swift:111-118,514);
 *   - a context is bound to one device and is not re-entrant: calls on one context must not overlap (the reference's
 *     "one stream per pipeline" rule, Pipeline.swift:179).
 */
#ifndef FVSR_LCSA_H
#define FVSR_LCSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FVSR_ABI_VERSION 1

typedef enum fvsr_status {
  FVSR_OK = 0,
  FVSR_ERR_INVALID_ARG = 1,   /* shape/pointer/argument rejected before any device work */
  FVSR_ERR_UNSUPPORTED = 2,   /* valid but outside what this build implements (head_dim != 128, batch != 1, ...) */
  FVSR_ERR_HIP = 3,           /* a HIP runtime call failed */
  FVSR_ERR_OUT_OF_MEMORY = 4, /* device allocation failed */
  FVSR_ERR_CAPACITY = 5,      /* a ring append would exceed its slot capacity */
  FVSR_ERR_STATE = 6          /* call out of sequence (e.g. select on an empty ring) */
} fvsr_status;

typedef enum fvsr_dtype { FVSR_DTYPE_F32 = 0, FVSR_DTYPE_BF16 = 1 } fvsr_dtype;

/* Attention implementation, mirroring `FlashVSRAttention` (DiT.swift:193-203). `gathered` (2) is not built: the
 * reference documents it as 2-4x slower than dense and keeps it for study only. */
typedef enum fvsr_attn_mode {
  FVSR_ATTN_AUTO = 0,    /* kernel when the expected kept fraction <= threshold, else dense (DiT.swift:517-522) */
  FVSR_ATTN_DENSE = 1,   /* every key block visited, unselected blocks masked (blockMaskedAttention) */
  FVSR_ATTN_KERNEL = 3   /* only the selected key blocks visited (kernelBlockAttention) */
} fvsr_attn_mode;

/* Token order of K/V handed to a ring append. */
typedef enum fvsr_token_layout {
  FVSR_LAYOUT_WINDOWS = 0, /* (n_slices*s*128, C) already window-partitioned (the reference's kW/vW) */
  FVSR_LAYOUT_GRID = 1     /* (f*h*w, C) natural (f, h, w) token order; the append partitions on the fly */
} fvsr_token_layout;

typedef struct fvsr_ctx fvsr_ctx;
typedef struct fvsr_kv_ring fvsr_kv_ring;

/* ---- library / device ------------------------------------------------------------------------------------ */
int fvsr_abi_version(void);
/* Message of the last failing call on this thread ("" if none). Valid until the next call on this thread. */
const char* fvsr_last_error(void);
/* Device facts used for launch shaping: compute units, XCDs, LDS bytes per workgroup, arch name (e.g. "gfx950"). */
int fvsr_device_props(int device, int* cu_count, int* xcd_count, size_t* lds_bytes, char* arch, size_t arch_len);

/* ---- context: device binding + workspace ------------------------------------------------------------------ */
int fvsr_ctx_create(int device, fvsr_ctx** out);
int fvsr_ctx_destroy(fvsr_ctx* ctx);
/* Grow the context workspace to at least `bytes` now, so later calls of that size do not allocate. */
int fvsr_ctx_reserve(fvsr_ctx* ctx, size_t bytes);
size_t fvsr_ctx_workspace_bytes(const fvsr_ctx* ctx);
/* Workspace bytes the select/attention entry points need for a geometry (so a caller can reserve up front). */
size_t fvsr_workspace_size(int heads, int64_t lq, int64_t lk, int channels);

/* ---- (a2) local window ------------------------------------------------------------------------------------ */
/* Replaces `localBlockMask(bh:bw:range:)` (DiT.swift:130-145). HOST function: writes (bh*bw)^2 bytes, 1 = key block
 * (kr, kc) visible to query block (qr, qc), i.e. kr in [qr - r/2, qr - r/2 + r - 1] and likewise for columns. */
int fvsr_local_block_mask(int bh, int bw, int range, uint8_t* out);

/* Expected kept fraction min(1, (topk+1)/(s*nk)) and the `auto` choice against `threshold` (the reference uses
 * 0.45, DiT.swift:210,517-522). HOST function. Returns FVSR_ATTN_KERNEL or FVSR_ATTN_DENSE in *mode. */
int fvsr_attention_mode_auto(int topk, int s, int nk, double threshold, double* expected, int* mode);

/* ---- (a3 + a7 list build) block selection ----------------------------------------------------------------- */
/* Replaces `draftBlockMaskAndProbs(qW:kW:heads:qSlices:spatialBlocks:local:topk:)` (DiT.swift:158-174) and the
 * kcnt/kidx build of `kernelBlockAttention` (SparseAttention.swift:175-177).
 *   qW  (lq, heads*128) queries, window order; lq/128 blocks (a partial last block pools its valid tokens)
 *   kW  (lk, heads*128) keys (cache ++ new), window order
 *   local_dev  device (s*s) bytes from fvsr_local_block_mask, tiled over every (query slice, key slice) pair
 *   Nq = ceil(lq/128) must be q_slices * s; key block j takes local row j mod s.
 * Outputs (device; mask_out and probs_out may be NULL):
 *   mask_out  (H, Nq, Nk) f32 0/1: probs STRICTLY above the (k+1)-th largest of each (head, query slice) row,
 *             k = min(n-1, topk), n = s*Nk
 *   probs_out (H, Nq, Nk) f32 softmax over key blocks of the pooled scores / sqrt(128) (+ -inf outside the window)
 *   kidx_out  (H, Nq, Nk) i32 selected key blocks first (ascending), then the unselected (ascending)
 *   kcnt_out  (H, Nq) i32 selected count */
int fvsr_lcsa_select(fvsr_ctx* ctx, int dtype, const void* qW, int64_t lq, const void* kW, int64_t lk, int heads,
                     int q_slices, int s, const uint8_t* local_dev, int topk, float* mask_out, float* probs_out,
                     int32_t* kidx_out, int32_t* kcnt_out, void* stream);

/* ---- (a7-a9) block-sparse attention ----------------------------------------------------------------------- */
/* Replaces the Metal launch of `kernelBlockAttention` (SparseAttention.swift:180-185): o = softmax(q k^T / sqrt(128))
 * v per head over the first kcnt[h][i] key blocks listed in kidx[h][i][*] (row stride nk_stride); a query block
 * with kcnt 0 writes zeros. q (lq, H*128), k/v (lk, H*128), o (lq, H*128), all `dtype`. lq, lk need not be
 * multiples of 128: keys past lk are excluded, rows past lq are not written. */
int fvsr_lcsa_attention(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                        int64_t lk, int heads, const int32_t* kidx, const int32_t* kcnt, int nk_stride, void* o,
                        void* stream);

/* No counterpart in the reference: fvsr_lcsa_attention for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments and results as
 * fvsr_lcsa_attention; the persistent walk's row order and work counter live in a static device array of the
 * library (1 MiB + 256 B per GPU, held until the process ends) instead of the context workspace, so the call
 * allocates nothing. For bf16, heads * ceil(lq / 128) must be <= 262144 (FVSR_ERR_UNSUPPORTED otherwise, before any
 * device work); the fp32 kernel keeps no row order, so fp32 calls have no such cap. The context must exist
 * (fvsr_ctx_create takes the array's device address). Calls that overlap on one GPU share the array and race:
 * serialise them (one stream, or events). The call may be captured into a HIP graph: the order kernel rewrites the
 * row order and the work counter on every launch, so each replay starts from a clean scratch. */
int fvsr_lcsa_attention_noalloc(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                                int64_t lk, int heads, const int32_t* kidx, const int32_t* kcnt, int nk_stride,
                                void* o, void* stream);

/* Replaces `FlashVSRAttentionOps.kernel` / `.dense` (SparseAttention.swift:190-202): attention under a block mask
 * (H, Nq, Nk) f32 tested > 0.5. mode FVSR_ATTN_KERNEL visits only the selected blocks; FVSR_ATTN_DENSE is the
 * dense fallback of `blockMaskedAttention` (DiT.swift:279-313): the same kernel walks EVERY key block and masks the
 * unselected ones, so its cost is that of full attention. Both return the same values. */
int fvsr_lcsa_attention_mask(fvsr_ctx* ctx, int dtype, const void* q, int64_t lq, const void* k, const void* v,
                             int64_t lk, int heads, const float* block_mask, int mode, void* o, void* stream);

/* ---- (a5) streaming KV window cache as a ring --------------------------------------------------------------- */
/* Replaces the per-block window cache of `blockForward` (DiT.swift:507-511 concat, :532-538 trim) held in
 * `ChunkState` (Pipeline.swift:87-91). One ring holds `layers` independent windows of up to `capacity_slices`
 * temporal slices (s = bh*bw blocks of 128 tokens each). Append writes a chunk's new slices into the next free slots
 * (no copy of the cached ones); evict applies the reference trim rule — if more than kv_len slices are held, drop the
 * oldest one — by moving the ring head (0 bytes). The ring also keeps each block's fp32 mean-pooled key, so
 * selection never re-reads cached keys. */
int fvsr_kv_ring_create(fvsr_ctx* ctx, int dtype, int layers, int heads, int bh, int bw, int capacity_slices,
                        int kv_len, fvsr_kv_ring** out);
int fvsr_kv_ring_destroy(fvsr_kv_ring* ring);
/* Empty every layer (a new clip: `FlashVSRPipeline.begin`, Pipeline.swift:105-109). */
int fvsr_kv_ring_reset(fvsr_kv_ring* ring);
/* k_new/v_new: n_slices*s*128 tokens of (H*128) channels in `layout` order; for FVSR_LAYOUT_GRID the tokens are
 * (f = 2*n_slices, h = 8*bh, w = 8*bw) natural order. */
int fvsr_kv_ring_append(fvsr_kv_ring* ring, int layer, const void* k_new, const void* v_new, int n_slices,
                        int layout, void* stream);
int fvsr_kv_ring_evict(fvsr_kv_ring* ring, int layer);
/* Slices currently held by `layer` (HOST, no device work). */
int fvsr_kv_ring_slices(const fvsr_kv_ring* ring, int layer, int* out);
/* Copy the held window of `layer` out in window order, (slices*s*128, H*128) each: the reference's cacheK/cacheV. */
int fvsr_kv_ring_read(fvsr_kv_ring* ring, int layer, void* k_out, void* v_out, void* stream);

/* Selection over the ring's held keys of `layer` (uses the cached pooled keys); outputs as fvsr_lcsa_select. */
int fvsr_lcsa_select_ring(fvsr_ctx* ctx, fvsr_kv_ring* ring, int layer, const void* qW, int64_t lq, int q_slices,
                          const uint8_t* local_dev, int topk, float* mask_out, float* probs_out, int32_t* kidx_out,
                          int32_t* kcnt_out, void* stream);
/* Attention over the ring's held keys/values of `layer` from lists (mode KERNEL) or, mode DENSE, every held block
 * with the unselected masked (kidx/kcnt still name the selection). */
int fvsr_lcsa_attention_ring(fvsr_ctx* ctx, fvsr_kv_ring* ring, int layer, const void* q, int64_t lq,
                             const int32_t* kidx, const int32_t* kcnt, int nk_stride, int mode, void* o,
                             void* stream);

/* One LCSA layer call — the self-attention core of `blockForward` (DiT.swift:504-538) after the projections:
 * append the chunk's new K/V, select over cache ++ new, attend (mode AUTO uses threshold 0.45 like the reference),
 * then evict. qW (lq, C) window order; k_new/v_new as fvsr_kv_ring_append. mask_out/probs_out may be NULL. */
int fvsr_lcsa_layer(fvsr_ctx* ctx, fvsr_kv_ring* ring, int layer, const void* qW, int64_t lq, const void* k_new,
                    const void* v_new, int n_new_slices, int layout, int q_slices, const uint8_t* local_dev,
                    int topk, int mode, void* o, float* mask_out, float* probs_out, void* stream);

/* ---- (f1) fused QKV epilogue: RMSNorm + 3-D RoPE + window partition ------------------------------------------ */
/* RoPE tables of `RopeTables(headDim: 128, theta:)` (DiT.swift:52-97), HOST function: fills `out` (at least
 * fvsr_rope_tables_size() floats) with cos_t, sin_t (1024 x 22), cos_h, sin_h (1024 x 21), cos_w, sin_w (1024 x 21),
 * row p = position p, computed in double and stored fp32 like the reference. Upload them once per device. */
size_t fvsr_rope_tables_size(void);
int fvsr_rope_tables(double theta, float* out, size_t n_floats);

/* The projections' epilogue of `blockForward` (DiT.swift:496-506): q' = ropeApply(normQ(q)), k' = ropeApply(normK(k))
 * with WanRMSNorm over the full width (DiT.swift:34-47: fp32 normalise with eps, cast, times weight) and ropeApply
 * at temporal positions t0 .. t0+f-1 (DiT.swift:100-107), then windowPartition (DiT.swift:111-118) of q', k' and v.
 * q, k, v: (f*h*w, heads*128) natural (f, h, w) token order, `dtype`; norm weights: (heads*128) `dtype`;
 * rope_tables: device copy of fvsr_rope_tables. Outputs q_out, k_out, v_out: (f*h*w, heads*128) window order. */
int fvsr_qkv_epilogue(fvsr_ctx* ctx, int dtype, const void* q, const void* k, const void* v, int f, int h, int w,
                      int heads, int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                      const float* rope_tables, void* q_out, void* k_out, void* v_out, void* stream);
/* The same epilogue straight into the KV ring: appends the chunk's k' and v (f = 2*n_slices, h = 8*bh, w = 8*bw,
 * natural token order) to `layer` like fvsr_kv_ring_append (pooled keys included) and writes q' in window order to
 * q_out. Replaces the projection epilogue and the cache concat of blockForward (DiT.swift:496-511). */
int fvsr_kv_ring_append_qkv(fvsr_kv_ring* ring, int layer, const void* q, const void* k, const void* v, int n_slices,
                            int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                            const float* rope_tables, void* q_out, void* stream);

/* The LCSA layer call from the projections: the self-attention core of `blockForward` (DiT.swift:496-539) between
 * the q/k/v projections and the o projection. fvsr_kv_ring_append_qkv (normQ/normK + RoPE + window partition +
 * cache append), selection over cache ++ new, attention (mode AUTO: threshold 0.45), evict; the attention output
 * is written in natural (f, h, w) token order, i.e. the reference's windowReverse (DiT.swift:121-126,539) is fused
 * into the attention kernel's store. q, k, v: (2*n_new_slices*8bh*8bw, C) projections in natural order; q_work:
 * (same shape) receives q' in window order; o: (same shape) the attention output in natural order. The queries
 * are the chunk's own n_new_slices slices. mask_out/probs_out may be NULL. */
int fvsr_lcsa_layer_qkv(fvsr_ctx* ctx, fvsr_kv_ring* ring, int layer, const void* q, const void* k, const void* v,
                        int n_new_slices, int t0, const void* norm_q_weight, const void* norm_k_weight, float eps,
                        const float* rope_tables, const uint8_t* local_dev, int topk, int mode, void* q_work, void* o,
                        float* mask_out, float* probs_out, void* stream);

/* ---- (f3) the dense parts of the DiT block ------------------------------------------------------------------ */
/* No reference counterpart (MLX allocates lazily): make the DiT-block entry points allocation-free for blocks of up to
 * `tokens` tokens (heads * 128 channels, FFN width ffn_dim, ctx_len context tokens) whose attention sees up to
 * `key_tokens` keys. A layer call attends over the held slices plus the chunk's new ones before the trim, so
 * key_tokens must cover min(capacity, kv_len + largest n_new_slices) * s * 128 (not kv_len slices alone: a call
 * past the reserved size grows the workspace, and that hipFree synchronises the device). Creates the context's
 * hipBLASLt handle and 64 MB GEMM workspace, grows the block workspace (about (8 C + F) * tokens * 2 bytes) and the
 * select/attention workspace. */
int fvsr_ctx_reserve_block(fvsr_ctx* ctx, int heads, int64_t tokens, int ffn_dim, int ctx_len, int64_t key_tokens);
size_t fvsr_ctx_block_workspace_bytes(const fvsr_ctx* ctx);

/* `Linear` (MLX, DiT.swift:319-321,371): y = x W^T + b on hipBLASLt, bf16 in/out, fp32 accumulate. x: (rows,
 * in_features); weight: (out_features, in_features) row-major; bias: (out_features) or NULL; gelu != 0 applies the
 * tanh-form GELU of `GELU(approximation: .tanh)` (DiT.swift:371) to the fp32 result before the bf16 store. Feature
 * counts must be multiples of 8. The first call on a context creates its hipBLASLt handle and 64 MB GEMM workspace
 * (fvsr_ctx_reserve_block creates it up front). */
int fvsr_linear(fvsr_ctx* ctx, const void* x, int64_t rows, int in_features, const void* weight, int out_features,
                const void* bias, int gelu, void* y, void* stream);

/* Weights of one `DiTBlock` (DiT.swift:363-375), bf16 device pointers, Linear weights (out, in) row-major; any
 * bias may be NULL. C = heads * 128. */
typedef struct fvsr_dit_block_weights {
  const void* modulation;                                      /* (6, C) */
  const void *q_weight, *q_bias, *k_weight, *k_bias;           /* self-attention (C, C), (C) */
  const void *v_weight, *v_bias, *o_weight, *o_bias;
  const void *norm_q_weight, *norm_k_weight;                   /* WanRMSNorm weights (C) */
  const void *cross_q_weight, *cross_q_bias, *cross_k_weight, *cross_k_bias;   /* cross-attention */
  const void *cross_v_weight, *cross_v_bias, *cross_o_weight, *cross_o_bias;
  const void *cross_norm_q_weight, *cross_norm_k_weight;
  const void *cross_k, *cross_v;                               /* (ctx_len, C) cached context K/V */
  int ctx_len;
  const void *norm3_weight, *norm3_bias;                       /* LayerNorm(affine) (C) */
  const void *ffn1_weight, *ffn1_bias, *ffn2_weight, *ffn2_bias; /* (F, C), (F), (C, F), (C) */
  int ffn_dim;                                                 /* F, a multiple of 8 */
} fvsr_dit_block_weights;

/* `CrossAttention.initCache` (DiT.swift:346-350): k_out = normK(k(context)), v_out = v(context), context (ctx_len, C)
 * bf16 (the text-embedded prompt); the results go to cross_k / cross_v of the weights. Once per context. */
int fvsr_dit_cross_kv(fvsr_ctx* ctx, const fvsr_dit_block_weights* w, int heads, const void* context, int ctx_len,
                      float eps, void* k_out, void* v_out, void* stream);

/* One streaming `blockForward` (DiT.swift:491-551) of block `layer`: x (L, C) bf16 in natural (f, h, w) token
 * order, L = 2*n_new_slices * 8bh * 8bw, updated in place. t_mod: (6, C) bf16 time modulation. norm1 / norm2 /
 * norm3 (eps), modulation, the q/k/v projections, fvsr_lcsa_layer_qkv on `ring` (selection + attention + cache
 * append/evict; topk, mode, local window and RoPE as there), the o projection and gated residual, the
 * cross-attention over w->cross_k / cross_v, and the FFN with its gated residual. Activations live in a block
 * workspace of the context (about (8 * C + F) * L * 2 bytes), grown on the first call of a size unless
 * fvsr_ctx_reserve_block sized it. */
int fvsr_dit_block(fvsr_ctx* ctx, fvsr_kv_ring* ring, int layer, const fvsr_dit_block_weights* w, const void* t_mod,
                   void* x, int n_new_slices, int t0, float eps, const float* rope_tables, const uint8_t* local_dev,
                   int topk, int mode, void* stream);

/* ---- (a1) window layout ------------------------------------------------------------------------------------ */
/* Replace `windowPartition` / `windowReverse` (DiT.swift:113-126): (f*h*w, C) natural <-> window order. */
int fvsr_window_partition(int dtype, const void* x, void* out, int f, int h, int w, int channels, void* stream);
int fvsr_window_reverse(int dtype, const void* x, void* out, int f, int h, int w, int channels, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FVSR_LCSA_H */
