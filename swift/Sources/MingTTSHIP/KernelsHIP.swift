// The operator layer of MingTTS on Linux over the MI355X C ABI (include/mingtts_hip.h).
//
// It keeps the names, argument labels and argument meaning of the reference's Metal operator
// layer (Sources/MingTTS/Engine/Kernels.swift:7-44, 89-289), so the Swift code above it
// (QwenForward, DiTForward, VAEDecoder, MingEngine) calls the same signatures.  What
// changes underneath:
//   - a buffer is a device address (hipMalloc'd by the caller) instead of an MTLBuffer;
//     offsets stay in bytes, as in the reference;
//   - an Encoder holds a HIP stream instead of a compute-command encoder, and every method
//     enqueues on it;
//   - Encoder.rmsnorm launches the norm on its own (mt_rmsnorm), so its output holds the
//     rows as in the reference; Encoder.linearNormed is the pair rmsnorm + linear of a layer
//     (Qwen.swift:84-85, 89-90; DiT.swift:42-43, 46-47, 50-51) as one mt_linear_rmsnorm
//     launch, for the forward passes that never read the normalised rows otherwise;
//   - shape errors come back from the C ABI as MT_EINVAL and stop here with the library's
//     message, where the reference stops on its own preconditions (Kernels.swift:105, 147).
#if os(Linux)
import CMingHIP

/// A device allocation: the address hipMalloc returned (MTLBuffer on the reference's side).
typealias DeviceBuffer = UnsafeMutableRawPointer

/// A tensor at a byte offset of a device buffer (GPUTensor, Kernels.swift:7-11).  `dtype`
/// names its element type: bf16 weights as the reference's checkpoints, or fp16 when the
/// WeightArena converted them.
struct GPUTensor {
    let buffer: DeviceBuffer
    let offset: Int
    let count: Int
    var dtype: mt_dtype = MT_BF16

    var address: UnsafeMutableRawPointer { buffer + offset }
}

/// y = x W^T (+ bias), `w` [n, k] row-major (Linear, Kernels.swift:13-19).
struct Linear {
    let w: GPUTensor
    let bias: GPUTensor?
    let n: Int
    let k: Int
}

/// GemvFlags (Kernels.swift:21-28); the raw values are the C ABI's MT_BIAS .. MT_SILU.
struct GemvFlags: OptionSet {
    let rawValue: UInt32
    static let bias = GemvFlags(rawValue: 1)
    static let accumulate = GemvFlags(rawValue: 2)
    static let gelu = GemvFlags(rawValue: 4)
    static let siluGate = GemvFlags(rawValue: 8)
    static let silu = GemvFlags(rawValue: 16)
}

/// An fp32 activation view: rows of floats at `offset` bytes, row stride `ld` floats
/// (ActView, Kernels.swift:30-44).
struct ActView {
    let buffer: DeviceBuffer
    let offset: Int
    let ld: Int

    init(_ buffer: DeviceBuffer, offset: Int = 0, ld: Int) {
        self.buffer = buffer
        self.offset = offset
        self.ld = ld
    }

    func row(_ r: Int) -> ActView { ActView(buffer, offset: offset + r * ld * 4, ld: ld) }
    func column(_ c: Int) -> ActView { ActView(buffer, offset: offset + c * 4, ld: ld) }

    var floats: UnsafeMutablePointer<Float> { (buffer + offset).assumingMemoryBound(to: Float.self) }
}

/// One layer's K and V cache, [kvHeads, capacity, 64] each (KVCacheLayer, Kernels.swift:
/// 285-289); `dtype` MT_F32 as the reference or MT_F16.
struct KVCacheLayer {
    let k: GPUTensor
    let v: GPUTensor
    let capacity: Int
    var dtype: mt_dtype = MT_F32
}

/// Enqueues the path's kernels on one HIP stream (Encoder, Kernels.swift:89-283).
struct Encoder {
    let stream: mt_stream_t?

    init(stream: mt_stream_t?) {
        self.stream = stream
    }

    private func check(_ rc: Int32, _ what: StaticString) {
        precondition(rc == 0, "\(what): \(String(cString: mt_last_error()))")
    }

    /// Encoder.linear (Kernels.swift:132-161): y[m, n] (op)= sum_k x[m, k] w[n, k] with the
    /// epilogue in `flags`; `gate` is the up projection of `.siluGate`.  The library picks the
    /// kernel for the shape (mt_linear_kernel reports which); bias sets MT_BIAS as the
    /// reference does.
    func linear(_ x: ActView, rows m: Int, _ linear: Linear, _ y: ActView, flags: GemvFlags = [], gate: GPUTensor? = nil) {
        var f = flags
        if linear.bias != nil { f.insert(.bias) }
        let bias = linear.bias.map { UnsafeRawPointer($0.address) }
        let w2 = gate.map { UnsafeRawPointer($0.address) }
        let p = mt_gemv_params(M: UInt32(m), N: UInt32(linear.n), K: UInt32(linear.k), ldx: UInt32(x.ld),
                               ldy: UInt32(y.ld), flags: f.rawValue, eps: 0)
        check(mt_linear(UnsafeRawPointer(x.floats), MT_F32, UnsafeRawPointer(linear.w.address), w2, linear.w.dtype,
                        bias, y.floats, p, stream), "Encoder.linear")
    }

    /// Encoder.rmsnorm (Kernels.swift:163-171): y = x * rsqrt(mean(x^2) + eps) * weight per row.
    func rmsnorm(_ x: ActView, rows: Int, width: Int, weight: GPUTensor, _ y: ActView, eps: Float = 1e-6) {
        check(mt_rmsnorm(x.floats, UInt32(x.ld), UInt32(rows), UInt32(width), UnsafeRawPointer(weight.address),
                         weight.dtype, y.floats, UInt32(y.ld), eps, stream), "Encoder.rmsnorm")
    }

    /// rmsnorm(x, weight: norm) into a scratch view followed by linear(scratch, ...), as one
    /// launch with the norm in the linear's prologue; the scratch rows are never written.
    func linearNormed(_ x: ActView, rows m: Int, norm: GPUTensor, eps: Float = 1e-6, _ linear: Linear, _ y: ActView,
                      flags: GemvFlags = [], gate: GPUTensor? = nil) {
        var f = flags
        if linear.bias != nil { f.insert(.bias) }
        let p = mt_gemv_params(M: UInt32(m), N: UInt32(linear.n), K: UInt32(linear.k), ldx: UInt32(x.ld),
                               ldy: UInt32(y.ld), flags: f.rawValue, eps: eps)
        check(mt_linear_rmsnorm(UnsafeRawPointer(x.floats), MT_F32, UnsafeRawPointer(norm.address),
                                UnsafeRawPointer(linear.w.address), gate.map { UnsafeRawPointer($0.address) },
                                linear.w.dtype, linear.bias.map { UnsafeRawPointer($0.address) }, y.floats, p, stream),
              "Encoder.linearNormed")
    }

    /// Encoder.ropeCache (Kernels.swift:180-191): NeoX RoPE on the q heads of `qkv` in place,
    /// rotated k and v appended to the cache at pos0 ..< pos0 + m.
    func ropeCache(_ qkv: ActView, rows m: Int, heads hq: Int, kvHeads hkv: Int, pos0: Int, cache: KVCacheLayer,
                   invFreq: DeviceBuffer) {
        check(mt_rope_cache(qkv.floats, UInt32(qkv.ld), UInt32(m), UInt32(hq), UInt32(hkv), UInt32(pos0),
                            cache.k.address, cache.v.address, cache.dtype, UInt32(cache.capacity),
                            invFreq.assumingMemoryBound(to: Float.self), stream), "Encoder.ropeCache")
    }

    /// Encoder.attention (Kernels.swift:193-206): causal GQA of the m rows at pos0 ..< pos0 + m
    /// over the cache, scale 1 / sqrt(64).
    func attention(_ q: ActView, rows m: Int, heads hq: Int, kvHeads hkv: Int, pos0: Int, window: Int,
                   cache: KVCacheLayer, _ out: ActView) {
        check(mt_attention(q.floats, UInt32(q.ld), UInt32(m), UInt32(hq), UInt32(hkv), UInt32(pos0), UInt32(window),
                           UnsafeRawPointer(cache.k.address), UnsafeRawPointer(cache.v.address), cache.dtype,
                           UInt32(cache.capacity), out.floats, UInt32(out.ld), 1 / Float(64).squareRoot(), stream),
              "Encoder.attention")
    }

    /// Encoder.ditAttention (Kernels.swift:208-220): full attention with interleaved RoPE
    /// inside each of `batch` sequences of `seq` <= 8 rows.
    func ditAttention(_ qkv: ActView, batch: Int, seq: Int, heads: Int, invFreq: DeviceBuffer, _ out: ActView) {
        check(mt_dit_attention(qkv.floats, UInt32(qkv.ld), UInt32(batch), UInt32(seq), UInt32(heads),
                               invFreq.assumingMemoryBound(to: Float.self), out.floats, UInt32(out.ld),
                               1 / Float(64).squareRoot(), stream), "Encoder.ditAttention")
    }

    /// Encoder.flowAssemble (Kernels.swift:222-235): the six flow-input rows.
    func flowAssemble(y: DeviceBuffer, history: DeviceBuffer, cemb: DeviceBuffer, condBias: GPUTensor, temb: ActView,
                      xEmbedder: Linear, _ x: ActView) {
        check(mt_flow_assemble(y.assumingMemoryBound(to: Float.self), history.assumingMemoryBound(to: Float.self),
                               cemb.assumingMemoryBound(to: Float.self), UnsafeRawPointer(condBias.address), temb.floats,
                               UnsafeRawPointer(xEmbedder.w.address), UnsafeRawPointer(xEmbedder.bias!.address),
                               xEmbedder.w.dtype, x.floats, UInt32(x.ld), UInt32(xEmbedder.n), UInt32(xEmbedder.k),
                               stream), "Encoder.flowAssemble")
    }

    /// Encoder.flowEuler (Kernels.swift:237-246): the CFG Euler step, c and u captured.
    func flowEuler(y: DeviceBuffer, pred: ActView, predRow: Int, nullRow: Int, latentDim: Int, cfg: Float, dt: Float,
                   capture: ActView) {
        check(mt_flow_euler(y.assumingMemoryBound(to: Float.self), pred.floats, UInt32(pred.ld), UInt32(predRow),
                            UInt32(nullRow), capture.floats, UInt32(latentDim), cfg, dt, stream), "Encoder.flowEuler")
    }

    /// Encoder.upsample4 (Kernels.swift:247-257): the four frames of a latent.
    func upsample4(prev: ActView?, cur: ActView, next: ActView?, hidden: Int, _ frames: ActView) {
        check(mt_upsample4(prev.map { UnsafePointer($0.floats) }, cur.floats, next.map { UnsafePointer($0.floats) },
                           frames.floats, UInt32(frames.ld), UInt32(hidden), stream), "Encoder.upsample4")
    }

    /// Encoder.istftFrames (Kernels.swift:259-270): windowed frames into ring slots from frame0.
    func istftFrames(spec: ActView, count: Int, nfft: Int, cosTable: DeviceBuffer, window: DeviceBuffer,
                     frames: DeviceBuffer, frame0: Int, ring: Int) {
        check(mt_istft_frames(spec.floats, UInt32(spec.ld), UInt32(count), UInt32(nfft),
                              cosTable.assumingMemoryBound(to: Float.self), window.assumingMemoryBound(to: Float.self),
                              frames.assumingMemoryBound(to: Float.self), UInt32(frame0), UInt32(ring), stream),
              "Encoder.istftFrames")
    }

    /// Encoder.istftEmit (Kernels.swift:272-283): samples s0 ..< s0 + count by overlap-add.
    func istftEmit(frames: DeviceBuffer, window: DeviceBuffer, nfft: Int, hop: Int, s0: Int, count: Int, lastFrame: Int,
                   ring: Int, _ out: ActView) {
        guard count > 0 else { return }
        check(mt_istft_emit(frames.assumingMemoryBound(to: Float.self), window.assumingMemoryBound(to: Float.self),
                            UInt32(nfft), UInt32(hop), UInt32(s0), UInt32(count), UInt32(lastFrame), UInt32(ring),
                            out.floats, stream), "Encoder.istftEmit")
    }
}

extension Encoder {
    /// Kernels.usesGemm / scalarRowsMax (Kernels.swift:81-86, 126): the kernel family the
    /// library runs for a linear of this shape (MT_KERNEL_GEMV, _GEMM or _GEMV_MFMA).
    static func kernelFamily(rows m: Int, _ linear: Linear) -> Int32 {
        mt_linear_kernel(UInt32(m), UInt32(linear.n), UInt32(linear.k), MT_F32, linear.w.dtype)
    }
}
#endif
