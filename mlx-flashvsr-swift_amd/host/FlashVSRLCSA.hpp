// FlashVSRLCSA.hpp — C++ host layer over the libfvsr_lcsa C ABI, mirroring the reference's Swift call surface
// (xocialize/mlx-flashvsr-swift, Sources/FlashVSRMLX):
//
//   flashvsr::localBlockMask                     localBlockMask(bh:bw:range:)              DiT.swift:130-145
//   flashvsr::LCSA::draftBlockMaskAndProbs       draftBlockMaskAndProbs(qW:kW:...)          DiT.swift:158-174
//   flashvsr::LCSA::kernelBlockAttention         kernelBlockAttention(q:k:v:blockMask:...)  SparseAttention.swift:169-187
//   flashvsr::LCSA::blockMaskedAttention         blockMaskedAttention(q:k:v:blockMask:...)  DiT.swift:279-313
//   flashvsr::FlashVSRAttention / current()      FlashVSRAttention (FLASHVSR_ATTN)          DiT.swift:193-203
//   flashvsr::WindowKVCache                      the per-block window cache of blockForward  DiT.swift:507-511,532-538
//   flashvsr::DiTBlock                           DiTBlock + the streaming blockForward       DiT.swift:363-375,491-551
//
// The reference traps on bad shapes (precondition); here a non-zero fvsr_status throws flashvsr::LCSAError carrying
// the status and fvsr_last_error(). Device buffers are caller-owned HIP allocations.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "fvsr_lcsa.h"

namespace flashvsr {

struct LCSAError : std::runtime_error {
  int status;
  LCSAError(int st, const std::string& what) : std::runtime_error(what), status(st) {}
};

inline void check(int rc, const char* fn) {
  if (rc != FVSR_OK) throw LCSAError(rc, std::string(fn) + ": " + fvsr_last_error());
}

// `FlashVSRAttention` (DiT.swift:193-203): auto | dense | kernel. `gathered` is not built.
enum class FlashVSRAttention { automatic = FVSR_ATTN_AUTO, dense = FVSR_ATTN_DENSE, kernel = FVSR_ATTN_KERNEL };

// FLASHVSR_ATTN=auto|dense|kernel, default auto (the reference's GPU default).
inline FlashVSRAttention currentAttention() {
  const char* e = std::getenv("FLASHVSR_ATTN");
  if (!e) return FlashVSRAttention::automatic;
  const std::string s(e);
  if (s == "dense") return FlashVSRAttention::dense;
  if (s == "kernel") return FlashVSRAttention::kernel;
  return FlashVSRAttention::automatic;
}

// `kernelDensityThreshold` (DiT.swift:210).
constexpr double kernelDensityThreshold = 0.45;

// (s*s) visibility of key block (kr, kc) from query block (qr, qc).
inline std::vector<uint8_t> localBlockMask(int bh, int bw, int range) {
  std::vector<uint8_t> m((size_t)bh * bw * bh * bw);
  check(fvsr_local_block_mask(bh, bw, range, m.data()), "fvsr_local_block_mask");
  return m;
}

// A token buffer (L, H*128) on the device, window order.
struct Tokens {
  const void* ptr;
  int64_t tokens;
  fvsr_dtype dtype;
};

class LCSA {
 public:
  explicit LCSA(int device = 0) { check(fvsr_ctx_create(device, &ctx_), "fvsr_ctx_create"); }
  ~LCSA() { fvsr_ctx_destroy(ctx_); }
  LCSA(const LCSA&) = delete;
  LCSA& operator=(const LCSA&) = delete;

  fvsr_ctx* handle() const { return ctx_; }
  void reserve(int heads, int64_t lq, int64_t lk) {
    check(fvsr_ctx_reserve(ctx_, fvsr_workspace_size(heads, lq, lk, heads * 128)), "fvsr_ctx_reserve");
  }

  // mask / probs may be null; kidx (H, Nq, Nk) and kcnt (H, Nq) receive the compacted key lists.
  void draftBlockMaskAndProbs(const Tokens& qW, const Tokens& kW, int heads, int qSlices, int spatialBlocks,
                              const uint8_t* localDev, int topk, float* mask, float* probs, int32_t* kidx,
                              int32_t* kcnt, hipStream_t stream = nullptr) {
    check(fvsr_lcsa_select(ctx_, qW.dtype, qW.ptr, qW.tokens, kW.ptr, kW.tokens, heads, qSlices, spatialBlocks,
                           localDev, topk, mask, probs, kidx, kcnt, stream),
          "fvsr_lcsa_select");
  }

  void kernelBlockAttention(const Tokens& q, const Tokens& k, const Tokens& v, const float* blockMask, int heads,
                            void* out, hipStream_t stream = nullptr) {
    check(fvsr_lcsa_attention_mask(ctx_, q.dtype, q.ptr, q.tokens, k.ptr, v.ptr, k.tokens, heads, blockMask,
                                   FVSR_ATTN_KERNEL, out, stream),
          "fvsr_lcsa_attention_mask");
  }

  void blockMaskedAttention(const Tokens& q, const Tokens& k, const Tokens& v, const float* blockMask, int heads,
                            void* out, hipStream_t stream = nullptr) {
    check(fvsr_lcsa_attention_mask(ctx_, q.dtype, q.ptr, q.tokens, k.ptr, v.ptr, k.tokens, heads, blockMask,
                                   FVSR_ATTN_DENSE, out, stream),
          "fvsr_lcsa_attention_mask");
  }

  // `FlashVSRAttentionOps` (SparseAttention.swift:190-202).
  void dense(const Tokens& q, const Tokens& k, const Tokens& v, const float* m, int heads, void* out,
             hipStream_t s = nullptr) {
    blockMaskedAttention(q, k, v, m, heads, out, s);
  }
  void kernel(const Tokens& q, const Tokens& k, const Tokens& v, const float* m, int heads, void* out,
              hipStream_t s = nullptr) {
    kernelBlockAttention(q, k, v, m, heads, out, s);
  }

 private:
  fvsr_ctx* ctx_ = nullptr;
};

// The window K/V cache of every DiT block as one ring: `ChunkState` (Pipeline.swift:87-91) plus the concat / trim of
// `blockForward`. step() is the LCSA core of one block for one chunk (DiT.swift:504-538).
class WindowKVCache {
 public:
  WindowKVCache(LCSA& lcsa, fvsr_dtype dtype, int layers, int heads, int bh, int bw, int kvLen = 3)
      : lcsa_(lcsa), heads_(heads), s_(bh * bw) {
    // capacity: the window is read before the trim, so it holds kvLen + the largest chunk (3 slices in chunk 0)
    check(fvsr_kv_ring_create(lcsa.handle(), dtype, layers, heads, bh, bw, kvLen + 3, kvLen, &ring_),
          "fvsr_kv_ring_create");
  }
  ~WindowKVCache() { fvsr_kv_ring_destroy(ring_); }
  WindowKVCache(const WindowKVCache&) = delete;
  WindowKVCache& operator=(const WindowKVCache&) = delete;

  void reset() { check(fvsr_kv_ring_reset(ring_), "fvsr_kv_ring_reset"); }
  int slices(int layer) const {
    int n = 0;
    check(fvsr_kv_ring_slices(ring_, layer, &n), "fvsr_kv_ring_slices");
    return n;
  }

  void step(int layer, const Tokens& qW, const void* kNew, const void* vNew, int newSlices, int qSlices,
            const uint8_t* localDev, int topk, void* out, FlashVSRAttention mode = currentAttention(),
            float* mask = nullptr, float* probs = nullptr, hipStream_t stream = nullptr) {
    check(fvsr_lcsa_layer(lcsa_.handle(), ring_, layer, qW.ptr, qW.tokens, kNew, vNew, newSlices,
                          FVSR_LAYOUT_WINDOWS, qSlices, localDev, topk, static_cast<int>(mode), out, mask, probs,
                          stream),
          "fvsr_lcsa_layer");
  }

  fvsr_kv_ring* handle() const { return ring_; }
  LCSA& lcsa() const { return lcsa_; }

 private:
  LCSA& lcsa_;
  fvsr_kv_ring* ring_ = nullptr;
  int heads_, s_;
};

// `DiTBlock` (DiT.swift:363-375) over caller-owned bf16 device tensors: `weights` holds every field of
// fvsr_dit_block_weights but the cross K/V, which initCache() computes from the text-embedded prompt
// (CrossAttention.initCache, DiT.swift:346-350) into caller-provided (ctxLen, C) buffers. forward() is the
// streaming blockForward (DiT.swift:491-551) on tokens x (natural order), updated in place.
class DiTBlock {
 public:
  DiTBlock(const fvsr_dit_block_weights& weights, int heads, float eps = 1e-6f)
      : w_(weights), heads_(heads), eps_(eps) {}

  void initCache(LCSA& lcsa, const void* context, int ctxLen, void* crossK, void* crossV,
                 hipStream_t stream = nullptr) {
    check(fvsr_dit_cross_kv(lcsa.handle(), &w_, heads_, context, ctxLen, eps_, crossK, crossV, stream),
          "fvsr_dit_cross_kv");
    w_.cross_k = crossK;
    w_.cross_v = crossV;
    w_.ctx_len = ctxLen;
  }

  void forward(WindowKVCache& cache, int layer, void* x, const void* tMod, int newSlices, int t0,
               const float* ropeTables, const uint8_t* localDev, int topk,
               FlashVSRAttention mode = currentAttention(), hipStream_t stream = nullptr) {
    check(fvsr_dit_block(cache.lcsa().handle(), cache.handle(), layer, &w_, tMod, x, newSlices, t0, eps_, ropeTables,
                         localDev, topk, static_cast<int>(mode), stream),
          "fvsr_dit_block");
  }

 private:
  fvsr_dit_block_weights w_;
  int heads_;
  float eps_;
};

}  // namespace flashvsr
