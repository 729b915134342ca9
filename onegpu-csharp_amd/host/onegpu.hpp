// The host side of the MI355X int8 path: the reference's kernel-family API (RecursiveAI.OneGpu.Kernels — Int8Gemm,
// DynamicQuantizeKernels, DequantizeKernels) and the slice of its device layer they need (GpuDevice, GpuBuffer,
// GpuCommandEncoder, the exceptions), in C++ over the C ABI of libonegpu_hip.so (include/onegpu_hip.h).
//
// Names, argument meaning, validation order and the exception raised for each bad argument follow the C# sources cited
// at each member, so code written against the reference API reads the same here. What differs is only what HIP makes
// moot: a kernel's arguments travel by value in the launch packet, so the bind groups become argument blocks that are
// only counted (ArgumentBlocks), and buffers carry their element type at run time where the C# API has a generic
// parameter, so the type checks the C# compiler or RequireInt8 makes happen at the call.
#pragma once

#include <cstdint>
#include <functional>
#include <initializer_list>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "onegpu_hip.h"

namespace onegpu {

// ------------------------------------------------------------------ exceptions (src/RecursiveAI.OneGpu/GpuDevice.cs:266-396;
// src/RecursiveAI.OneGpu.Kernels/GpuKernelShapeException.cs:7-25)

class GpuException : public std::runtime_error {
public:
    explicit GpuException(const std::string &m) : std::runtime_error(m) {}
};

// A shape, stride, offset or size is invalid for the operation; raised before any work is recorded.
class GpuKernelShapeException : public GpuException {
public:
    GpuKernelShapeException(std::string operation, std::string argument, const std::string &message)
        : GpuException(operation + ": " + argument + ": " + message), Operation(std::move(operation)),
          Argument(std::move(argument)), Detail(message) {}
    std::string Operation, Argument, Detail;
};

class GpuUnsupportedException : public GpuException {
public:
    GpuUnsupportedException(const std::string &message, std::string capability = "", std::string expected = "",
                            std::string actual = "")
        : GpuException(message), Capability(std::move(capability)), Expected(std::move(expected)), Actual(std::move(actual)) {}
    std::string Capability, Expected, Actual;
};

class GpuOutOfMemoryException : public GpuException {
public:
    using GpuException::GpuException;
};

class GpuDeviceLostException : public GpuException {
public:
    using GpuException::GpuException;
};

class GpuCommandFailedException : public GpuException {
public:
    using GpuException::GpuException;
};

// An index given to a gather was outside its axis (GpuIndexStatus.cs:66-80).
class GpuKernelIndexException : public GpuException {
public:
    GpuKernelIndexException(std::string operation, int64_t position)
        : GpuException(operation + ": the index at position " + std::to_string(position) +
                       " of the indices is outside its axis"),
          Operation(std::move(operation)), Position(position) {}
    std::string Operation;
    int64_t Position;
};

// ------------------------------------------------------------------ device layer

// The element types the path uses; the C# names are what its messages print (typeof(T).Name).
enum class ElementType { UInt8, Int8, Int32, Float32, Float16, UInt32, UInt16, Int16, Int64 };
size_t ElementSize(ElementType t);
const char *ElementName(ElementType t);

// The limits the families consult (src/RecursiveAI.OneGpu/ComputeCapabilities.cs:86-203).
struct GpuComputeCapabilities {
    uint64_t MaxStorageBufferBindingBytes = 0;  // 0: no limit per binding (HIP binds plain device addresses)
    uint32_t MaxWorkgroupCount = 0;             // 0: no per-axis grid limit the families must fold around
    bool Int8DotProduct = true;                 // int8 MFMA and v_dot4_i32_i8
    uint32_t ComputeUnits = 0;
};

struct GpuDeviceOptions {
    // Lower than the hardware's, to run a product the way a device with small bindings (llvmpipe: 128 MB) refuses it.
    uint64_t MaxStorageBufferBindingBytes = 0;
    // This library's own: Submit runs consecutive DequantizeLinear passes of one shape whose buffers are independent
    // as one launch (og_dequantize_batch). false keeps a launch a pass. The results are the same either way.
    bool BatchDispatches = true;
};

class GpuDevice;

// A typed device buffer (src/RecursiveAI.OneGpu/GpuBufferOfT.cs:11-89). Length counts elements; byte buffers are
// allocated to a whole 32-bit word as CreateBuffer<T> does (src/RecursiveAI.OneGpu/ComputeKernel.cs:93-95).
class GpuBuffer {
public:
    struct Impl;
    GpuBuffer() = default;
    explicit GpuBuffer(std::shared_ptr<Impl> impl) : impl_(std::move(impl)) {}
    int Length() const;
    ElementType Type() const;
    uint64_t Size() const;        // bytes
    void *DevicePointer() const;  // device address (host address on a host-only device)
    void Write(const void *src, uint64_t bytes, uint64_t byte_offset = 0) const;
    void Read(void *dst, uint64_t bytes, uint64_t byte_offset = 0) const;
    void Dispose();
    bool Valid() const { return impl_ != nullptr; }
    og_buffer Binding() const;
    const std::shared_ptr<Impl> &impl() const { return impl_; }

private:
    std::shared_ptr<Impl> impl_;
};

// A recorded DequantizeLinear pass, kept whole so that Submit can run consecutive passes of one shape together.
struct DequantCommand {
    int kind = 0;
    bool half = false;
    og_dequant_params params{};
    GpuBuffer x, scale, zero, out;
};

// Records work; nothing runs until GpuDevice::Submit (src/RecursiveAI.OneGpu/GpuDevice.cs:155-161; Resources.cs:148-316).
class GpuCommandEncoder {
public:
    using Command = std::function<void(og_ctx *)>;
    void Record(Command c, std::vector<std::shared_ptr<GpuBuffer::Impl>> keep);
    void RecordDequant(DequantCommand c, std::vector<std::shared_ptr<GpuBuffer::Impl>> keep);
    // A host step that runs in its place at Submit: no dispatch, nothing launched (an empty ranged product's count).
    void RecordHost(Command c);
    int DispatchCount() const;
    // Per-dispatch timing of the commands recorded between the two calls (Resources.cs:216-222).
    void BeginPassTiming(int max_passes);
    int EndPassTiming();

private:
    friend class GpuDevice;
    struct Entry {
        Command run;
        std::vector<std::shared_ptr<GpuBuffer::Impl>> keep;
        std::shared_ptr<const DequantCommand> dq;   // set for a DequantizeLinear pass
        bool host = false;                          // a host step (RecordHost)
    };
    std::vector<Entry> commands_;
    int timing_start_ = -1;  // first timed command
    int timing_stop_ = -1;   // last timed command
    int timing_slots_ = 0;
    bool submitted_ = false;
};

class GpuDevice : public std::enable_shared_from_this<GpuDevice> {
public:
    // A HIP device (og_init). Throws GpuUnsupportedException when there is none.
    static std::shared_ptr<GpuDevice> Create(int ordinal = 0, GpuDeviceOptions options = {});
    // No GPU: buffers live in host memory and every family validates and records as usual, but Submit of a non-empty
    // encoder throws. Lets argument checks run where no GPU exists.
    static std::shared_ptr<GpuDevice> CreateHostOnly(GpuDeviceOptions options = {});
    ~GpuDevice();

    GpuBuffer CreateBuffer(ElementType type, int length);
    GpuCommandEncoder BeginCommands() { return GpuCommandEncoder(); }
    void Submit(GpuCommandEncoder &encoder);
    void WaitIdle();
    // GPU milliseconds and kernel name of each dispatch timed by the last submitted encoder (TryReadTimestamps).
    std::vector<std::pair<double, std::string>> ReadPassTimes();

    const GpuComputeCapabilities &Capabilities() const { return caps_; }
    const std::string &AdapterName() const { return name_; }
    std::string Backend() const { return ctx_ ? "Hip" : "HostOnly"; }
    og_ctx *Context() const { return ctx_; }
    bool HasGpu() const { return ctx_ != nullptr; }

private:
    GpuDevice() = default;
    static bool dequant_joins(const DequantCommand &first, const std::vector<GpuCommandEncoder::Entry> &cmds, int begin,
                              int j);
    og_ctx *ctx_ = nullptr;
    GpuComputeCapabilities caps_;
    std::string name_;
    int timed_ = 0;
    bool batch_ = true;
};

// Maps a C-ABI status to the reference's exception (operation names the family).
void ThrowIfFailed(og_ctx *ctx, int status, const std::string &operation);

// ------------------------------------------------------------------ Int8Gemm (src/RecursiveAI.OneGpu.Kernels/Int8Gemm.cs)

struct Int8GemmOptions {
    bool AllowPackedDot = true;  // false forces the portable kernel (Int8Gemm.cs:9-13)
    // Test hook (Int8Gemm.cs:15-16): 0 chooses by size; any other value keeps the few-rows kernel off so every shape
    // runs on the tiled MFMA kernel (64), or keeps the few-rows kernel but always splits k (32: the split-k kernel and
    // its reduction pass, not the tiled one). 256 is this library's own: every shape on the 256 x 256 tile kernels,
    // which otherwise only large products reach.
    int Tile = 0;
    // This library's own: EncodeRequantized in one launch, the requantization applied where the product stores its
    // sums (og_int8_gemm_requantized), so no scratch is written. false keeps the reference's two passes (the product
    // into scratch, then Finish). The bytes written are the same either way.
    bool FusedRequantize = true;
    // This library's own: the tiled few-rows kernel (M <= 16) adds its tiles' parts in the same launch (the last tile
    // of a column slab finishes it). false keeps the two-launch form (a second kernel adds the parts). Same output.
    bool FewRowsOneLaunch = true;
};

// A zero point, scale, multiplier or bias operand (Int8Gemm.cs:23-29).
struct Int8Operand {
    GpuBuffer Buffer;
    int Offset = 0;
    bool IsVector = false;
};

// Caller-placed int32 scratch for EncodeRequantized (Int8Gemm.cs:31-37).
struct Int8Scratch {
    GpuBuffer Buffer;
    int Offset = 0;
};

// This library's own: where a ranged float product (Int8Gemm::EncodeFloatRanged) records the range of what it stores,
// for DynamicQuantizeKernels::EncodeRanged to quantize that output with no read pass. Buffer: 2 * OG_RANGES_MAX float32
// (a GpuBuffer of that length, or one the instance creates); Groups: the (min, max) pairs the last ranged product
// recorded into it wrote, known once that product has run (Submit), read by the quantize pass when it runs.
struct Int8Ranges {
    Int8Ranges() = default;
    explicit Int8Ranges(GpuBuffer buffer);
    GpuBuffer Buffer;
    std::shared_ptr<uint32_t> Groups = std::make_shared<uint32_t>(0);
};

// What a kernel family's bind groups (Int8Gemm.cs:365-375; BindingCacheTests.cs:141-197) become on HIP. Nothing is
// bound: a dispatch's arguments travel by value in its launch packet. A family instead remembers the argument blocks it
// has recorded, one per dispatch kind and set of buffers (offsets and sizes are launch arguments, as they are uniforms
// in the reference), at most maxCachedBindGroups of them, the least recently recorded dropped first. Created() counts
// the blocks added since the family was made: recording a call again with buffers it has seen adds none, and after
// Release() (ReleaseBindings: the cache emptied, the count kept) the same call adds its blocks again.
class ArgumentBlocks {
public:
    explicit ArgumentBlocks(int capacity);
    void Note(uint64_t kind, std::initializer_list<const GpuBuffer *> buffers);
    int Created() const { return created_; }
    void Release() { blocks_.clear(); }

private:
    int capacity_;
    int created_ = 0;
    uint64_t clock_ = 0;
    std::vector<std::pair<std::vector<uintptr_t>, uint64_t>> blocks_;   // (kind and buffer identities, last use)
};

// Int8Gemm.cs:39-95.
struct Int8GemmProblem {
    Int8GemmProblem() = default;
    Int8GemmProblem(int m, int n, int k) : M(m), N(n), K(k), Batch(1) {}
    int M = 0, N = 0, K = 0, Batch = 1;
    bool TransposeB = false;
    int Lda = 0, Ldb = 0, OffsetA = 0, OffsetB = 0, OffsetC = 0, StrideA = 0, StrideB = 0;
    double Ops() const { return 2.0 * Batch * M * N * K; }
};

class Int8Gemm {
public:
    explicit Int8Gemm(std::shared_ptr<GpuDevice> device, Int8GemmOptions options = {}, int maxCachedBindGroups = 1024);
    ~Int8Gemm();

    // Int8Gemm.cs:217-253: C = (A - zeroA)(B - zeroB) (+ bias per column), int32.
    void EncodeInt32(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a, const GpuBuffer &b,
                     const GpuBuffer &c, const std::optional<Int8Operand> &zeroPointA = std::nullopt,
                     const std::optional<Int8Operand> &zeroPointB = std::nullopt,
                     const std::optional<Int8Operand> &bias = std::nullopt);
    // Int8Gemm.cs:255-314: float(sum + intBias) * scale + floatBias, one dispatch.
    void EncodeFloat(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a, const GpuBuffer &b,
                     const GpuBuffer &c, const Int8Operand &scale, const std::optional<Int8Operand> &zeroPointA = std::nullopt,
                     const std::optional<Int8Operand> &zeroPointB = std::nullopt,
                     const std::optional<Int8Operand> &floatBias = std::nullopt,
                     const std::optional<Int8Operand> &intBias = std::nullopt);
    // This library's own: EncodeFloat whose column scale is fl(activationScale * weightScale[n or 0]), the product
    // the reference computes with an elementwise Mul before EncodeFloat (Int8Tests.cs:738-745); one launch, the same
    // bits. activationScale is one float32 (e.g. DynamicQuantizeLinear's scale output).
    void EncodeFloatScaled(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                           const GpuBuffer &b, const GpuBuffer &c, const Int8Operand &activationScale,
                           const Int8Operand &weightScale, const std::optional<Int8Operand> &zeroPointA = std::nullopt,
                           const std::optional<Int8Operand> &zeroPointB = std::nullopt,
                           const std::optional<Int8Operand> &floatBias = std::nullopt,
                           const std::optional<Int8Operand> &intBias = std::nullopt);
    // This library's own: EncodeFloat (or EncodeFloatScaled, with activationScale) that also records the range of the
    // values it stores in `ranges`, so DynamicQuantizeKernels::EncodeRanged can quantize c without a read pass. The same
    // bits in c; c is dense (Int8GemmProblem's C always is) and holds at most 2^31 - 1 elements.
    void EncodeFloatRanged(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                           const GpuBuffer &b, const GpuBuffer &c, const Int8Operand &scale, const Int8Ranges &ranges,
                           const std::optional<Int8Operand> &zeroPointA = std::nullopt,
                           const std::optional<Int8Operand> &zeroPointB = std::nullopt,
                           const std::optional<Int8Operand> &floatBias = std::nullopt,
                           const std::optional<Int8Operand> &intBias = std::nullopt,
                           const std::optional<Int8Operand> &activationScale = std::nullopt);
    // Int8Gemm.cs:316-363: QLinearMatMul, the sums in scratch, then the requantizing pass.
    void EncodeRequantized(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                           const GpuBuffer &b, const GpuBuffer &y, const Int8Operand &multiplier, int zeroPointY,
                           const std::optional<Int8Operand> &zeroPointA = std::nullopt,
                           const std::optional<Int8Operand> &zeroPointB = std::nullopt,
                           const std::optional<Int8Operand> &intBias = std::nullopt,
                           const std::optional<Int8Scratch> &scratch = std::nullopt);

    static int64_t ScratchElements(const Int8GemmProblem &problem);   // Int8Gemm.cs:525-531
    void ReserveScratch(int64_t elements);                            // Int8Gemm.cs:533-549
    const std::string &Variant() const { return variant_; }           // Int8Gemm.cs:214-215
    int BindGroupsCreated() const { return blocks_.Created(); }       // Int8Gemm.cs:365-366
    void ReleaseBindings() { blocks_.Release(); }                     // Int8Gemm.cs:368-375
    void Dispose();

private:
    struct Prepared {
        int Lda, Ldb;
        bool Ok;
    };
    struct Epilogue {
        uint32_t Flags = 0;
        bool Requantized = false;   // C is the 8-bit output; Scale holds the multiplier (og_int8_gemm_requantized)
        GpuBuffer ActScale;         // when valid: the column scale is fl(ActScale[OffActScale] * Scale[..])
        uint32_t OffActScale = 0;
        const Int8Ranges *Ranges = nullptr;   // a ranged float product (og_int8_gemm_float_ranged)
        int ZeroPointY = 0;
        bool SignedY = false;
        GpuBuffer IntBias;
        uint32_t OffIntBias = 0;
        GpuBuffer Scale;
        uint32_t OffScale = 0;
        GpuBuffer FloatBias;
        uint32_t OffFloatBias = 0;
    };
    Prepared Prepare(const Int8GemmProblem &p, const GpuBuffer &a, const GpuBuffer &b,
                     const std::optional<Int8Operand> &zpA, const std::optional<Int8Operand> &zpB);
    void CheckBindable(const std::string &operand, const GpuBuffer &buffer) const;
    void FloatProduct(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                      const GpuBuffer &b, const GpuBuffer &c, const Int8Operand *activationScale,
                      const Int8Operand &scale, const std::optional<Int8Operand> &zeroPointA,
                      const std::optional<Int8Operand> &zeroPointB, const std::optional<Int8Operand> &floatBias,
                      const std::optional<Int8Operand> &intBias, const Int8Ranges *ranges = nullptr);
    void Multiply(GpuCommandEncoder &encoder, const Int8GemmProblem &p, const GpuBuffer &a, bool aSigned,
                  const GpuBuffer &b, bool bSigned, const GpuBuffer &c, int offsetC,
                  const std::optional<Int8Operand> &za, const std::optional<Int8Operand> &zb, const Epilogue &epi);
    std::pair<GpuBuffer, int> Scratch(int64_t count, const std::optional<Int8Scratch> &given);

    std::shared_ptr<GpuDevice> device_;
    Int8GemmOptions options_;
    std::string variant_;
    std::vector<GpuBuffer> scratch_;
    ArgumentBlocks blocks_;
};

// ------------------------------------------------------------------ DynamicQuantizeKernels (DynamicQuantizeKernels.cs)

class DynamicQuantizeKernels {
public:
    explicit DynamicQuantizeKernels(std::shared_ptr<GpuDevice> device, int maxCachedBindGroups = 1024);
    // DynamicQuantizeKernels.cs:47-90.
    void Encode(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, int count, const GpuBuffer &y, int offsetY,
                const GpuBuffer &scale, int offsetScale, const GpuBuffer &zeroPoint, int offsetZeroPoint);
    // This library's own: Encode of x, the output a ranged product (Int8Gemm::EncodeFloatRanged) recorded the range of
    // in `ranges`: the quantize pass alone, one dispatch. The same y, scale and zero point.
    void EncodeRanged(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, int count, const GpuBuffer &y,
                      int offsetY, const GpuBuffer &scale, int offsetScale, const GpuBuffer &zeroPoint,
                      int offsetZeroPoint, const Int8Ranges &ranges);
    int BindGroupsCreated() const { return blocks_.Created(); }
    void ReleaseBindings() { blocks_.Release(); }
    void Dispose() {}

private:
    std::shared_ptr<GpuDevice> device_;
    ArgumentBlocks blocks_;
};

// ------------------------------------------------------------------ DequantizeKernels (DequantizeKernels.cs)

class DequantizeKernels {
public:
    explicit DequantizeKernels(std::shared_ptr<GpuDevice> device, int maxCachedBindGroups = 1024);
    // DequantizeKernels.cs:158-260 (DequantizeLinear).
    void Encode(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, const std::vector<int> &shape, int axis,
                bool perAxis, const GpuBuffer &scale, int offsetScale, const std::optional<GpuBuffer> &zeroPoint,
                int offsetZeroPoint, const GpuBuffer &output, int offsetOutput);
    // DequantizeKernels.cs:298-382 (QuantizeLinear).
    void EncodeQuantize(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, const std::vector<int> &shape,
                        int axis, bool perAxis, const GpuBuffer &scale, int offsetScale,
                        const std::optional<GpuBuffer> &zeroPoint, int offsetZeroPoint, const GpuBuffer &output,
                        int offsetOutput);
    int BindGroupsCreated() const { return blocks_.Created(); }
    void ReleaseBindings() { blocks_.Release(); }
    void Dispose() {}

private:
    std::shared_ptr<GpuDevice> device_;
    ArgumentBlocks blocks_;
};

// The geometry of a convolution (src/RecursiveAI.OneGpu.Kernels/ConvProblem.cs:107-235): NCHW input, OIHW weights,
// strides, dilations, asymmetric padding, groups; offsets in elements. Activation must stay 0 for ConvInteger.
struct ConvProblem {
    int Batch = 1, InChannels = 1, Height = 1, Width = 1, OutChannels = 1, KernelHeight = 1, KernelWidth = 1;
    int StrideHeight = 1, StrideWidth = 1, DilationHeight = 1, DilationWidth = 1;
    int PadTop = 0, PadLeft = 0, PadBottom = 0, PadRight = 0, Groups = 1;
    int Activation = 0;
    int OffsetX = 0, OffsetW = 0, OffsetBias = 0, OffsetResidual = 0, OffsetY = 0;
    ConvProblem() = default;
    ConvProblem(int batch, int inChannels, int height, int width, int outChannels, int kernelHeight, int kernelWidth)
        : Batch(batch), InChannels(inChannels), Height(height), Width(width), OutChannels(outChannels),
          KernelHeight(kernelHeight), KernelWidth(kernelWidth) {}
    // ConvProblem.Conv1D (ConvProblem.cs:127-136): height 1.
    static ConvProblem Conv1D(int batch, int inChannels, int length, int outChannels, int kernel, int stride = 1,
                              int dilation = 1, int padBegin = 0, int padEnd = 0, int groups = 1);
    int OutHeight() const;   // GpuWindow.OutputExtent without auto padding or ceil mode (ConvProblem.cs:36-73)
    int OutWidth() const;
};

// ONNX ConvInteger (ConvIntegerKernels.cs:6-351): the column matrix and the int8 products, or a direct kernel when
// every group has one input channel. Same checks, exceptions and scratch rules as the reference; the column rows are
// padded to 16 bytes here, so ScratchBytesPerImage is Groups * K * round16(OutHeight * OutWidth), with K padded to a
// multiple of 64 (and room for the weights in rows of that length) when 64 <= K and K % 64 != 0.
class ConvIntegerKernels {
public:
    explicit ConvIntegerKernels(std::shared_ptr<GpuDevice> device, Int8GemmOptions options = {},
                                int maxCachedBindGroups = 1024);
    std::string Variant() const { return gemm_.Variant(); }
    int BindGroupsCreated() const { return blocks_.Created() + gemm_.BindGroupsCreated(); }
    static int64_t ScratchBytesPerImage(const ConvProblem &problem);
    // ConvIntegerKernels.cs:97-253.
    void Encode(GpuCommandEncoder &encoder, const ConvProblem &problem, const GpuBuffer &x, const GpuBuffer &w,
                const GpuBuffer &y, const std::optional<Int8Operand> &xZeroPoint = std::nullopt,
                const std::optional<Int8Operand> &wZeroPoint = std::nullopt,
                const std::optional<GpuBuffer> &scratch = std::nullopt, int scratchOffset = 0);
    void ReleaseBindings()
    {
        blocks_.Release();
        gemm_.ReleaseBindings();
    }
    void Dispose();
    // This library's own: convolutions with one input channel a group run on the direct kernel (true, the default)
    // or through the column matrix and the products like the others (false; a test hook).
    bool DirectDepthwise = true;

private:
    GpuBuffer Own(ElementType t, int64_t bytes);
    std::shared_ptr<GpuDevice> device_;
    Int8GemmOptions options_;
    Int8Gemm gemm_;
    GpuBuffer own_u8_, own_i8_;
    std::vector<GpuBuffer> retired_;   // smaller columns buffers that recorded commands may still name
    ArgumentBlocks blocks_;
};

// Where a gather records the position of an invalid index (GpuIndexStatus.cs:13-63): one uint32 on the device, reset to
// "none" (0xFFFFFFFF) before the work and read back after it.
class GpuIndexStatus {
public:
    explicit GpuIndexStatus(std::shared_ptr<GpuDevice> device);
    void Reset();            // the write happens before the next submitted commands
    void ThrowIfFailed();    // waits for the device, reads the word, throws GpuKernelIndexException
    void Dispose() { buffer_.Dispose(); }
    const GpuBuffer &Buffer() const { return buffer_; }
    void Note(const std::string &operation) { operation_ = operation; }

private:
    std::shared_ptr<GpuDevice> device_;
    GpuBuffer buffer_;
    std::string operation_;
};

// The ONNX Gather of GatherKernels (GatherKernels.cs:22-118): EncodeGather over every payload type the reference
// takes (uint8/int8, half, int32/uint32/float32, int64), int32 or int64 indices. GatherElements and GatherND are not
// part of this library.
class GatherKernels {
public:
    explicit GatherKernels(std::shared_ptr<GpuDevice> device, int maxCachedBindGroups = 1024);
    // GatherKernels.cs:66-118: output[o, i, n] = data[o, indices[i], n] around `axis`.
    void EncodeGather(GpuCommandEncoder &encoder, const GpuBuffer &data, int offsetData, const std::vector<int> &dataShape,
                      int axis, const GpuBuffer &indices, int offsetIndices, int indexCount, const GpuBuffer &output,
                      int offsetOutput, GpuIndexStatus *status = nullptr);
    int BindGroupsCreated() const { return blocks_.Created(); }
    void ReleaseBindings() { blocks_.Release(); }
    void Dispose() {}

private:
    std::shared_ptr<GpuDevice> device_;
    ArgumentBlocks blocks_;
};

// ------------------------------------------------------------------ shared checks (KernelSupport.cs:68-131)

namespace Check {
constexpr int64_t MaxElements = 2147483647;
void Range(const std::string &operation, const std::string &name, int64_t bufferLength, int64_t offset, int64_t extent,
           bool half = false);
void RangeBytes(const std::string &operation, const std::string &name, int64_t bufferLength, int64_t offset,
                int64_t extent);
int64_t Product(const std::string &operation, const std::string &name, const std::vector<int> &shape);
}  // namespace Check

}  // namespace onegpu
