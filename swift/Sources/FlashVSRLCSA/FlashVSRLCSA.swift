// FlashVSRLCSA — the Swift call surface of the reference's LCSA path (xocialize/mlx-flashvsr-swift), backed by
// libfvsr_lcsa.so on an MI355X. Each function keeps the name and argument meaning of the reference function it
// replaces (cited beside it); buffers are HIP device memory the caller owns (MLX arrays live in Metal memory and
// cannot be handed to HIP). A non-zero status traps with the library's message, as the reference's preconditions do.
// This image has no Swift toolchain: the file is written against include/fvsr_lcsa.h and not compiled here.
import CFlashVSRLCSA

/// A caller-owned HIP device buffer: token tensors (rows, heads * 128) in window order, masks, key lists.
public struct DeviceTensor {
    public let ptr: UnsafeMutableRawPointer
    public let rows: Int
    /// FVSR_DTYPE_F32 or FVSR_DTYPE_BF16 for token tensors (ignored for masks and lists)
    public let dtype: Int32

    public init(ptr: UnsafeMutableRawPointer, rows: Int, dtype: Int32 = Int32(FVSR_DTYPE_BF16.rawValue)) {
        self.ptr = ptr
        self.rows = rows
        self.dtype = dtype
    }

    public var floatPtr: UnsafeMutablePointer<Float> { ptr.assumingMemoryBound(to: Float.self) }
    public var int32Ptr: UnsafeMutablePointer<Int32> { ptr.assumingMemoryBound(to: Int32.self) }
    public var bytePtr: UnsafePointer<UInt8> { UnsafePointer(ptr.assumingMemoryBound(to: UInt8.self)) }
}

/// hipStream_t as the C ABI takes it (NULL = the default stream).
public typealias HIPStream = UnsafeMutableRawPointer?

@inline(__always) func fvsrCheck(_ rc: Int32, _ fn: String) {
    precondition(rc == 0, "\(fn): \(String(cString: fvsr_last_error()))")
}

/// One device binding with its workspace; not re-entrant, like the reference's stateful modules
/// (Pipeline.swift:179).
public final class LCSAContext {
    public let ctx: OpaquePointer

    public init(device: Int32 = 0) {
        var c: OpaquePointer?
        fvsrCheck(fvsr_ctx_create(device, &c), "fvsr_ctx_create")
        ctx = c!
    }

    deinit { fvsr_ctx_destroy(ctx) }

    /// Size the select/attention workspace for (heads, lq, lk) so hot calls never allocate.
    public func reserve(heads: Int, lq: Int, lk: Int) {
        let bytes = fvsr_workspace_size(Int32(heads), Int64(lq), Int64(lk), Int32(heads * 128))
        fvsrCheck(fvsr_ctx_reserve(ctx, bytes), "fvsr_ctx_reserve")
    }

    /// Size everything a DiT block call of up to `tokens` tokens over a window of `keyTokens` keys needs.
    public func reserveBlock(heads: Int, tokens: Int, ffnDim: Int, contextLength: Int, keyTokens: Int) {
        fvsrCheck(fvsr_ctx_reserve_block(ctx, Int32(heads), Int64(tokens), Int32(ffnDim), Int32(contextLength),
                                         Int64(keyTokens)), "fvsr_ctx_reserve_block")
    }
}

/// `localBlockMask(bh:bw:range:)` (DiT.swift:130-145); upload once per geometry like `FlashVSRDiT.local`.
public func localBlockMask(bh: Int, bw: Int, range r: Int) -> [UInt8] {
    var m = [UInt8](repeating: 0, count: bh * bw * bh * bw)
    fvsrCheck(fvsr_local_block_mask(Int32(bh), Int32(bw), Int32(r), &m), "fvsr_local_block_mask")
    return m
}

/// The `auto` rule of blockForward (DiT.swift:517-522): kernel when the expected kept fraction is <= 0.45.
public func attentionModeAuto(topk: Int, spatialBlocks s: Int, keyBlocks nk: Int,
                              threshold: Double = 0.45) -> (expected: Double, mode: fvsr_attn_mode) {
    var e = 0.0
    var m: Int32 = 0
    fvsrCheck(fvsr_attention_mode_auto(Int32(topk), Int32(s), Int32(nk), threshold, &e, &m),
              "fvsr_attention_mode_auto")
    return (e, fvsr_attn_mode(rawValue: UInt32(m)))
}

/// `draftBlockMaskAndProbs` (DiT.swift:158-174) plus the kernel's key lists (SparseAttention.swift:175-177).
/// mask / probs (heads, Nq, Nk) f32 may be nil; kidx (heads, Nq, Nk) i32, kcnt (heads, Nq) i32.
public func draftBlockMaskAndProbs(_ c: LCSAContext, qW: DeviceTensor, kW: DeviceTensor, heads: Int, qSlices: Int,
                                   spatialBlocks s: Int, local: DeviceTensor, topk: Int, mask: DeviceTensor?,
                                   probs: DeviceTensor?, kidx: DeviceTensor, kcnt: DeviceTensor,
                                   stream: HIPStream = nil) {
    fvsrCheck(fvsr_lcsa_select(c.ctx, qW.dtype, qW.ptr, Int64(qW.rows), kW.ptr, Int64(kW.rows), Int32(heads),
                               Int32(qSlices), Int32(s), local.bytePtr, Int32(topk), mask?.floatPtr, probs?.floatPtr,
                               kidx.int32Ptr, kcnt.int32Ptr, stream), "fvsr_lcsa_select")
}

/// `draftBlockMask` (DiT.swift:150-154): the mask only.
public func draftBlockMask(_ c: LCSAContext, qW: DeviceTensor, kW: DeviceTensor, heads: Int, qSlices: Int,
                           spatialBlocks s: Int, local: DeviceTensor, topk: Int, mask: DeviceTensor,
                           kidx: DeviceTensor, kcnt: DeviceTensor, stream: HIPStream = nil) {
    draftBlockMaskAndProbs(c, qW: qW, kW: kW, heads: heads, qSlices: qSlices, spatialBlocks: s, local: local,
                           topk: topk, mask: mask, probs: nil, kidx: kidx, kcnt: kcnt, stream: stream)
}

/// `kernelBlockAttention(q:k:v:blockMask:heads:)` (SparseAttention.swift:169-187): only the selected blocks.
public func kernelBlockAttention(_ c: LCSAContext, q: DeviceTensor, k: DeviceTensor, v: DeviceTensor,
                                 blockMask: DeviceTensor, heads: Int, out: DeviceTensor, stream: HIPStream = nil) {
    fvsrCheck(fvsr_lcsa_attention_mask(c.ctx, q.dtype, q.ptr, Int64(q.rows), k.ptr, v.ptr, Int64(k.rows),
                                       Int32(heads), blockMask.floatPtr, Int32(FVSR_ATTN_KERNEL.rawValue), out.ptr,
                                       stream), "fvsr_lcsa_attention_mask")
}

/// `blockMaskedAttention` (DiT.swift:279-313): the dense fallback (same values, every key block visited).
public func blockMaskedAttention(_ c: LCSAContext, q: DeviceTensor, k: DeviceTensor, v: DeviceTensor,
                                 blockMask: DeviceTensor, heads: Int, out: DeviceTensor, stream: HIPStream = nil) {
    fvsrCheck(fvsr_lcsa_attention_mask(c.ctx, q.dtype, q.ptr, Int64(q.rows), k.ptr, v.ptr, Int64(k.rows),
                                       Int32(heads), blockMask.floatPtr, Int32(FVSR_ATTN_DENSE.rawValue), out.ptr,
                                       stream), "fvsr_lcsa_attention_mask")
}

/// The Metal launch ABI of kernelBlockAttention (SparseAttention.swift:180-185): attention from key lists.
/// `noAlloc` selects the entry point that allocates nothing (for callers under graph capture or in serving
/// loops); it has no reference counterpart.
public func blockSparseAttention(_ c: LCSAContext, q: DeviceTensor, k: DeviceTensor, v: DeviceTensor,
                                 kidx: DeviceTensor, kcnt: DeviceTensor, listStride: Int, heads: Int,
                                 out: DeviceTensor, noAlloc: Bool = false, stream: HIPStream = nil) {
    if noAlloc {
        fvsrCheck(fvsr_lcsa_attention_noalloc(c.ctx, q.dtype, q.ptr, Int64(q.rows), k.ptr, v.ptr, Int64(k.rows),
                                              Int32(heads), kidx.int32Ptr, kcnt.int32Ptr, Int32(listStride),
                                              out.ptr, stream), "fvsr_lcsa_attention_noalloc")
    } else {
        fvsrCheck(fvsr_lcsa_attention(c.ctx, q.dtype, q.ptr, Int64(q.rows), k.ptr, v.ptr, Int64(k.rows),
                                      Int32(heads), kidx.int32Ptr, kcnt.int32Ptr, Int32(listStride), out.ptr,
                                      stream), "fvsr_lcsa_attention")
    }
}

/// `FlashVSRAttentionOps` (SparseAttention.swift:189-202): the public probe entry points. `gathered` is not
/// built (the reference keeps it for study only).
public enum FlashVSRAttentionOps {
    public static func dense(_ c: LCSAContext, q: DeviceTensor, k: DeviceTensor, v: DeviceTensor,
                             blockMask: DeviceTensor, heads: Int, out: DeviceTensor, stream: HIPStream = nil) {
        blockMaskedAttention(c, q: q, k: k, v: v, blockMask: blockMask, heads: heads, out: out, stream: stream)
    }

    public static func kernel(_ c: LCSAContext, q: DeviceTensor, k: DeviceTensor, v: DeviceTensor,
                              blockMask: DeviceTensor, heads: Int, out: DeviceTensor, stream: HIPStream = nil) {
        kernelBlockAttention(c, q: q, k: k, v: v, blockMask: blockMask, heads: heads, out: out, stream: stream)
    }
}

/// `windowPartition` / `windowReverse` (DiT.swift:113-126): (f*h*w, C) natural order <-> window order.
public func windowPartition(_ x: DeviceTensor, into out: DeviceTensor, f: Int, h: Int, w: Int, channels: Int,
                            stream: HIPStream = nil) {
    fvsrCheck(fvsr_window_partition(x.dtype, x.ptr, out.ptr, Int32(f), Int32(h), Int32(w), Int32(channels), stream),
              "fvsr_window_partition")
}

public func windowReverse(_ x: DeviceTensor, into out: DeviceTensor, f: Int, h: Int, w: Int, channels: Int,
                          stream: HIPStream = nil) {
    fvsrCheck(fvsr_window_reverse(x.dtype, x.ptr, out.ptr, Int32(f), Int32(h), Int32(w), Int32(channels), stream),
              "fvsr_window_reverse")
}

/// `RopeTables(headDim: 128, theta:)` (DiT.swift:52-97) on the host; upload once per device.
public func ropeTables(theta: Double = 10000) -> [Float] {
    var t = [Float](repeating: 0, count: Int(fvsr_rope_tables_size()))
    fvsrCheck(fvsr_rope_tables(theta, &t, t.count), "fvsr_rope_tables")
    return t
}

/// The per-block window caches of `ChunkState` (Pipeline.swift:87-91) as one ring of `layers` windows. `step`
/// replaces DiT.swift:504-538 (concat, draft mask, auto / kernel / dense dispatch, trim) for block `layer`;
/// `stepFromProjections` replaces DiT.swift:496-539 (norms, RoPE, window partitions, concat, selection,
/// attention, trim, window reverse).
public final class WindowKVCache {
    public let ring: OpaquePointer
    public let lcsa: LCSAContext

    public init(_ lcsa: LCSAContext, dtype: fvsr_dtype, layers: Int = 30, heads: Int = 12, bh: Int, bw: Int,
                kvLen: Int = 3, capacitySlices: Int = 6) {
        var r: OpaquePointer?
        fvsrCheck(fvsr_kv_ring_create(lcsa.ctx, Int32(dtype.rawValue), Int32(layers), Int32(heads), Int32(bh),
                                      Int32(bw), Int32(capacitySlices), Int32(kvLen), &r), "fvsr_kv_ring_create")
        ring = r!
        self.lcsa = lcsa
    }

    deinit { fvsr_kv_ring_destroy(ring) }

    /// A new clip: `FlashVSRPipeline.begin` (Pipeline.swift:105-109).
    public func reset() { fvsrCheck(fvsr_kv_ring_reset(ring), "fvsr_kv_ring_reset") }

    public func slices(layer: Int) -> Int {
        var n: Int32 = 0
        fvsrCheck(fvsr_kv_ring_slices(ring, Int32(layer), &n), "fvsr_kv_ring_slices")
        return Int(n)
    }

    /// The held window of `layer` in window order (the reference's cacheK / cacheV).
    public func read(layer: Int, k: DeviceTensor, v: DeviceTensor, stream: HIPStream = nil) {
        fvsrCheck(fvsr_kv_ring_read(ring, Int32(layer), k.ptr, v.ptr, stream), "fvsr_kv_ring_read")
    }

    public func step(layer: Int, qW: DeviceTensor, kNew: DeviceTensor, vNew: DeviceTensor, newSlices: Int,
                     qSlices: Int, local: DeviceTensor, topk: Int, mode: fvsr_attn_mode, out: DeviceTensor,
                     mask: DeviceTensor? = nil, probs: DeviceTensor? = nil, stream: HIPStream = nil) {
        fvsrCheck(fvsr_lcsa_layer(lcsa.ctx, ring, Int32(layer), qW.ptr, Int64(qW.rows), kNew.ptr, vNew.ptr,
                                  Int32(newSlices), Int32(FVSR_LAYOUT_WINDOWS.rawValue), Int32(qSlices),
                                  local.bytePtr, Int32(topk), Int32(mode.rawValue), out.ptr, mask?.floatPtr,
                                  probs?.floatPtr, stream), "fvsr_lcsa_layer")
    }

    public func stepFromProjections(layer: Int, q: DeviceTensor, k: DeviceTensor, v: DeviceTensor, newSlices: Int,
                                    t0: Int, normQ: DeviceTensor, normK: DeviceTensor, eps: Float = 1e-6,
                                    ropeTables: DeviceTensor, local: DeviceTensor, topk: Int, mode: fvsr_attn_mode,
                                    qWork: DeviceTensor, out: DeviceTensor, stream: HIPStream = nil) {
        fvsrCheck(fvsr_lcsa_layer_qkv(lcsa.ctx, ring, Int32(layer), q.ptr, k.ptr, v.ptr, Int32(newSlices),
                                      Int32(t0), normQ.ptr, normK.ptr, eps, ropeTables.floatPtr, local.bytePtr,
                                      Int32(topk), Int32(mode.rawValue), qWork.ptr, out.ptr, nil, nil, stream),
                  "fvsr_lcsa_layer_qkv")
    }
}

/// One streaming `blockForward` (DiT.swift:491-551) of block `layer` with its weights on the device; `tokens`
/// (f*h*w, 1536) bf16 in natural order is updated in place. `crossKV` fills the weights' cross_k / cross_v once
/// per prompt (`CrossAttention.initCache`, DiT.swift:346-350).
public struct DiTBlockCall {
    public var weights: fvsr_dit_block_weights

    public init(weights: fvsr_dit_block_weights) { self.weights = weights }

    public mutating func crossKV(_ c: LCSAContext, heads: Int = 12, context: DeviceTensor, crossK: DeviceTensor,
                                 crossV: DeviceTensor, eps: Float = 1e-6, stream: HIPStream = nil) {
        fvsrCheck(fvsr_dit_cross_kv(c.ctx, &weights, Int32(heads), context.ptr, Int32(context.rows), eps, crossK.ptr,
                                    crossV.ptr, stream), "fvsr_dit_cross_kv")
        weights.cross_k = UnsafeRawPointer(crossK.ptr)
        weights.cross_v = UnsafeRawPointer(crossV.ptr)
        weights.ctx_len = Int32(context.rows)
    }

    public mutating func forward(_ cache: WindowKVCache, layer: Int, tMod: DeviceTensor, tokens: DeviceTensor,
                                 newSlices: Int, t0: Int, eps: Float = 1e-6, ropeTables: DeviceTensor,
                                 local: DeviceTensor, topk: Int, mode: fvsr_attn_mode = FVSR_ATTN_AUTO,
                                 stream: HIPStream = nil) {
        fvsrCheck(fvsr_dit_block(cache.lcsa.ctx, cache.ring, Int32(layer), &weights, tMod.ptr, tokens.ptr,
                                 Int32(newSlices), Int32(t0), eps, ropeTables.floatPtr, local.bytePtr, Int32(topk),
                                 Int32(mode.rawValue), stream), "fvsr_dit_block")
    }
}
