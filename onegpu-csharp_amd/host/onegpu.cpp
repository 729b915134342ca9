// Host layer over the C ABI: validation and parameter blocks as the reference's C# families build them.
#include "onegpu.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <sstream>

namespace onegpu {

namespace {

std::string fmt_long(int64_t v) { return std::to_string(v); }

}  // namespace

size_t ElementSize(ElementType t)
{
    switch (t) {
    case ElementType::UInt8:
    case ElementType::Int8: return 1;
    case ElementType::Float16:
    case ElementType::UInt16:
    case ElementType::Int16: return 2;
    case ElementType::Int64: return 8;
    default: return 4;
    }
}

const char *ElementName(ElementType t)
{
    switch (t) {
    case ElementType::UInt8: return "Byte";
    case ElementType::Int8: return "SByte";
    case ElementType::Int32: return "Int32";
    case ElementType::Float32: return "Single";
    case ElementType::Float16: return "Half";
    case ElementType::UInt32: return "UInt32";
    case ElementType::UInt16: return "UInt16";
    case ElementType::Int16: return "Int16";
    default: return "Int64";
    }
}

// ------------------------------------------------------------------ status mapping

void ThrowIfFailed(og_ctx *ctx, int status, const std::string &operation)
{
    if (status == OG_OK) return;
    std::string msg = og_last_error(ctx);
    std::string arg = og_last_error_argument(ctx);
    switch (status) {
    case OG_ERR_INVALID_ARG: throw GpuKernelShapeException(operation, arg.empty() ? "arguments" : arg, msg);
    case OG_ERR_UNSUPPORTED: throw GpuUnsupportedException(operation + ": " + msg);
    case OG_ERR_OUT_OF_MEMORY: throw GpuOutOfMemoryException(operation + ": " + msg);
    case OG_ERR_DEVICE_LOST: throw GpuDeviceLostException(operation + ": " + msg);
    case OG_ERR_NO_DEVICE: throw GpuUnsupportedException(operation + ": " + msg, "Device", "a HIP device", "none");
    default: throw GpuCommandFailedException(operation + ": " + msg);
    }
}

// ------------------------------------------------------------------ buffers

struct GpuBuffer::Impl {
    std::shared_ptr<GpuDevice> device;  // a buffer keeps its device (and so the context it frees into) alive
    og_ctx *ctx = nullptr;  // null: host-only buffer
    void *ptr = nullptr;
    int length = 0;
    ElementType type = ElementType::UInt8;
    uint64_t bytes = 0;  // allocated bytes
    ~Impl()
    {
        if (!ptr) return;
        if (ctx) og_free(ctx, ptr);
        else std::free(ptr);
    }
};

int GpuBuffer::Length() const { return impl_ ? impl_->length : 0; }
ElementType GpuBuffer::Type() const { return impl_ ? impl_->type : ElementType::UInt8; }
uint64_t GpuBuffer::Size() const { return impl_ ? impl_->bytes : 0; }
void *GpuBuffer::DevicePointer() const { return impl_ ? impl_->ptr : nullptr; }
og_buffer GpuBuffer::Binding() const { return og_buffer{impl_ ? impl_->ptr : nullptr, impl_ ? impl_->bytes : 0}; }

void GpuBuffer::Write(const void *src, uint64_t bytes, uint64_t byte_offset) const
{
    if (!impl_ || !impl_->ptr) throw GpuException("GpuBuffer: disposed");
    if (byte_offset > impl_->bytes || bytes > impl_->bytes - byte_offset)
        throw std::out_of_range("GpuBuffer.Write: range past the buffer");
    if (!bytes) return;
    if (impl_->ctx) ThrowIfFailed(impl_->ctx, og_memcpy_h2d(impl_->ctx, static_cast<uint8_t *>(impl_->ptr) + byte_offset, src, bytes), "GpuBuffer.Write");
    else std::memcpy(static_cast<uint8_t *>(impl_->ptr) + byte_offset, src, bytes);
}

void GpuBuffer::Read(void *dst, uint64_t bytes, uint64_t byte_offset) const
{
    if (!impl_ || !impl_->ptr) throw GpuException("GpuBuffer: disposed");
    if (byte_offset > impl_->bytes || bytes > impl_->bytes - byte_offset)
        throw std::out_of_range("GpuBuffer.Read: range past the buffer");
    if (!bytes) return;
    if (impl_->ctx) ThrowIfFailed(impl_->ctx, og_memcpy_d2h(impl_->ctx, dst, static_cast<uint8_t *>(impl_->ptr) + byte_offset, bytes), "GpuBuffer.Read");
    else std::memcpy(dst, static_cast<uint8_t *>(impl_->ptr) + byte_offset, bytes);
}

void GpuBuffer::Dispose() { impl_.reset(); }

// ------------------------------------------------------------------ encoder and device

void GpuCommandEncoder::Record(Command c, std::vector<std::shared_ptr<GpuBuffer::Impl>> keep)
{
    if (submitted_) throw GpuException("GpuCommandEncoder: already submitted");
    commands_.push_back(Entry{std::move(c), std::move(keep), nullptr});
}

void GpuCommandEncoder::RecordHost(Command c)
{
    if (submitted_) throw GpuException("GpuCommandEncoder: already submitted");
    commands_.push_back(Entry{std::move(c), {}, nullptr, true});
}

int GpuCommandEncoder::DispatchCount() const
{
    int n = 0;
    for (const Entry &e : commands_) n += e.host ? 0 : 1;
    return n;
}

void GpuCommandEncoder::RecordDequant(DequantCommand c, std::vector<std::shared_ptr<GpuBuffer::Impl>> keep)
{
    if (submitted_) throw GpuException("GpuCommandEncoder: already submitted");
    auto dq = std::make_shared<const DequantCommand>(std::move(c));
    Command run = [dq](og_ctx *ctx) {
        ThrowIfFailed(ctx, og_dequantize(ctx, dq->kind, dq->half ? 1 : 0, &dq->params, dq->x.Binding(), dq->scale.Binding(),
                                         dq->zero.Binding(), dq->out.Binding()),
                      "DequantizeLinear");
    };
    commands_.push_back(Entry{std::move(run), std::move(keep), std::move(dq)});
}

void GpuCommandEncoder::BeginPassTiming(int max_passes)
{
    if (max_passes < 1) throw std::invalid_argument("BeginPassTiming: max_passes must be at least 1");
    timing_start_ = (int)commands_.size();
    timing_stop_ = -1;
    timing_slots_ = max_passes;
}

int GpuCommandEncoder::EndPassTiming()
{
    if (timing_start_ < 0) return 0;
    timing_stop_ = (int)commands_.size() - 1;
    return timing_stop_ - timing_start_ + 1;
}

std::shared_ptr<GpuDevice> GpuDevice::Create(int ordinal, GpuDeviceOptions options)
{
    std::shared_ptr<GpuDevice> d(new GpuDevice());
    og_ctx *ctx = nullptr;
    int st = og_init(ordinal, &ctx);
    if (st != OG_OK) {
        std::string msg = og_last_error(nullptr);
        if (st == OG_ERR_NO_DEVICE) throw GpuUnsupportedException("GpuDevice: " + msg, "Device", "a HIP device", "none");
        ThrowIfFailed(nullptr, st, "GpuDevice");
    }
    d->ctx_ = ctx;
    char name[256];
    og_device_name(ctx, name, sizeof name);
    d->name_ = name;
    uint64_t maxbuf = 0;
    uint32_t cus = 0, lds = 0;
    og_device_limits(ctx, &maxbuf, &cus, &lds);
    d->caps_.ComputeUnits = cus;
    d->caps_.MaxStorageBufferBindingBytes = options.MaxStorageBufferBindingBytes;
    d->batch_ = options.BatchDispatches;
    return d;
}

std::shared_ptr<GpuDevice> GpuDevice::CreateHostOnly(GpuDeviceOptions options)
{
    std::shared_ptr<GpuDevice> d(new GpuDevice());
    d->name_ = "host only (no GPU)";
    d->caps_.MaxStorageBufferBindingBytes = options.MaxStorageBufferBindingBytes;
    return d;
}

GpuDevice::~GpuDevice()
{
    if (ctx_) og_destroy(ctx_);
}

GpuBuffer GpuDevice::CreateBuffer(ElementType type, int length)
{
    if (length < 0) throw std::invalid_argument("CreateBuffer: length must not be negative");
    auto impl = std::make_shared<GpuBuffer::Impl>();
    impl->device = shared_from_this();
    impl->length = length;
    impl->type = type;
    uint64_t bytes = (uint64_t)length * ElementSize(type);
    bytes = (bytes + 3) / 4 * 4;  // a whole 32-bit word, as the reference pads
    if (bytes == 0) bytes = 4;
    impl->bytes = bytes;
    if (ctx_) {
        impl->ctx = ctx_;
        ThrowIfFailed(ctx_, og_alloc(ctx_, bytes, &impl->ptr), "CreateBuffer");
        ThrowIfFailed(ctx_, og_fill_bytes(ctx_, impl->ptr, 0, bytes), "CreateBuffer");
    } else {
        impl->ptr = std::calloc(1, bytes);
        if (!impl->ptr) throw GpuOutOfMemoryException("CreateBuffer: host allocation failed");
    }
    return GpuBuffer(impl);
}

namespace {

// The device bytes of a pass's operand: [begin, end).
struct Span {
    uintptr_t begin = 0, end = 0;
};

bool overlaps(const Span &a, const Span &b) { return a.begin < a.end && b.begin < b.end && a.begin < b.end && b.begin < a.end; }

// Pass c's input spans (x, scale, zero point) and its output span.
void dequant_spans(const DequantCommand &c, Span in[3], Span &out)
{
    const og_dequant_params &p = c.params;
    const uint64_t esz = c.kind == OG_KIND_I32 ? 4 : 1, osz = c.half ? 2 : 4, params = (p.Flags & 1u) ? p.AxisLen : 1;
    auto span = [](const GpuBuffer &b, uint64_t off, uint64_t bytes) {
        const uintptr_t base = (uintptr_t)b.Binding().ptr + (uintptr_t)off;
        return Span{base, base + (uintptr_t)bytes};
    };
    in[0] = span(c.x, (uint64_t)p.OffX * esz, (uint64_t)p.Count * esz);
    in[1] = span(c.scale, (uint64_t)p.OffS * 4, params * 4);
    in[2] = (p.Flags & 2u) ? span(c.zero, (uint64_t)p.OffZ * esz, params * esz) : Span{};
    out = span(c.out, (uint64_t)p.OffO * osz, (uint64_t)p.Count * osz);
}

}  // namespace

// Whether pass j can join the run of passes first .. j - 1: the same kind, output type, count, flags and axis as the
// first, and no output overlapping another pass's operands or output.
bool GpuDevice::dequant_joins(const DequantCommand &first, const std::vector<GpuCommandEncoder::Entry> &cmds, int begin,
                              int j)
{
    const DequantCommand &c = *cmds[j].dq;
    const og_dequant_params &a = first.params, &b = c.params;
    if (c.kind != first.kind || c.half != first.half || b.Count != a.Count || b.Flags != a.Flags || b.Count == 0) return false;
    if ((b.Flags & 1u) && (b.AxisLen != a.AxisLen || b.Inner != a.Inner)) return false;
    Span cin[3], cout;
    dequant_spans(c, cin, cout);
    for (int k = begin; k < j; k++) {
        Span kin[3], kout;
        dequant_spans(*cmds[k].dq, kin, kout);
        if (overlaps(cout, kout)) return false;
        for (int t = 0; t < 3; t++)
            if (overlaps(cout, kin[t]) || overlaps(kout, cin[t])) return false;
    }
    return true;
}

void GpuDevice::Submit(GpuCommandEncoder &encoder)
{
    if (encoder.submitted_) throw GpuException("GpuDevice.Submit: encoder already submitted");
    encoder.submitted_ = true;
    if (encoder.commands_.empty()) return;
    if (!ctx_) {
        if (encoder.DispatchCount() > 0)
            throw GpuUnsupportedException("GpuDevice.Submit: a host-only device cannot run work", "Device", "a HIP device", "none");
        for (const auto &c : encoder.commands_) c.run(nullptr);   // host steps only
        return;
    }
    timed_ = 0;
    const int start = encoder.timing_start_, stop = encoder.timing_stop_, n = (int)encoder.commands_.size();
    const auto &cmds = encoder.commands_;
    for (int i = 0; i < n;) {
        // A command may launch more than one kernel (a split product, the two passes of a quantizer): 4 slots each.
        if (i == start && stop >= start) ThrowIfFailed(ctx_, og_timing_begin(ctx_, std::max(encoder.timing_slots_, stop - start + 1) * 4), "BeginPassTiming");
        // Consecutive DequantizeLinear passes of one shape run as one launch when no pass writes what another reads or
        // writes (in order they would be independent too, so the result is the same); a run does not cross the start
        // or the end of pass timing.
        int j = i + 1;
        if (batch_ && cmds[i].dq) {
            while (j < n && j - i < (int)OG_DEQUANT_BATCH_MAX && j != start && j - 1 != stop && cmds[j].dq &&
                   dequant_joins(*cmds[i].dq, cmds, i, j))
                j++;
        }
        if (j - i >= 2) {
            std::vector<og_dequant_params> p;
            std::vector<og_buffer> x, sc, z, o;
            for (int k = i; k < j; k++) {
                const DequantCommand &c = *cmds[k].dq;
                p.push_back(c.params);
                x.push_back(c.x.Binding());
                sc.push_back(c.scale.Binding());
                z.push_back(c.zero.Binding());
                o.push_back(c.out.Binding());
            }
            const DequantCommand &c0 = *cmds[i].dq;
            ThrowIfFailed(ctx_, og_dequantize_batch(ctx_, c0.kind, c0.half ? 1 : 0, (uint32_t)(j - i), p.data(), x.data(),
                                                     sc.data(), z.data(), o.data()),
                          "DequantizeLinear");
        } else {
            cmds[i].run(ctx_);
        }
        if (stop >= start && i <= stop && stop < j) ThrowIfFailed(ctx_, og_timing_end(ctx_, &timed_), "EndPassTiming");
        i = j;
    }
}

void GpuDevice::WaitIdle()
{
    if (ctx_) ThrowIfFailed(ctx_, og_sync(ctx_), "GpuDevice.WaitIdle");
}

std::vector<std::pair<double, std::string>> GpuDevice::ReadPassTimes()
{
    std::vector<std::pair<double, std::string>> out;
    for (int i = 0; i < timed_; i++) {
        float ms = 0;
        const char *name = "";
        ThrowIfFailed(ctx_, og_timing_read(ctx_, i, &ms, &name), "ReadPassTimes");
        out.emplace_back((double)ms, name);
    }
    return out;
}

// ------------------------------------------------------------------ Check (KernelSupport.cs:68-131)

namespace Check {

void Range(const std::string &operation, const std::string &name, int64_t bufferLength, int64_t offset, int64_t extent,
           bool half)
{
    if (offset < 0) throw GpuKernelShapeException(operation, name + "Offset", "offset " + fmt_long(offset) + " is negative");
    if (extent < 0 || offset + extent > bufferLength)
        throw GpuKernelShapeException(operation, name, "elements " + fmt_long(offset) + ".." + fmt_long(offset + extent) +
                                                           " reach past the buffer of " + fmt_long(bufferLength));
    if (half && extent > 0 && (((offset + extent + 1) >> 1) << 1) > bufferLength)
        throw GpuKernelShapeException(operation, name, "the buffer of " + fmt_long(bufferLength) +
                                                           " halves ends inside a 32-bit word; allocate GpuKernelBuffers.PaddedHalfLength(n) elements");
}

void RangeBytes(const std::string &operation, const std::string &name, int64_t bufferLength, int64_t offset, int64_t extent)
{
    if (offset < 0) throw GpuKernelShapeException(operation, name + "Offset", "offset " + fmt_long(offset) + " is negative");
    if (extent < 0 || offset + extent > bufferLength)
        throw GpuKernelShapeException(operation, name, "elements " + fmt_long(offset) + ".." + fmt_long(offset + extent) +
                                                           " reach past the buffer of " + fmt_long(bufferLength));
    if (extent > 0 && (((offset + extent + 3) >> 2) << 2) > bufferLength)
        throw GpuKernelShapeException(operation, name, "the buffer of " + fmt_long(bufferLength) +
                                                           " bytes ends inside a 32-bit word; allocate GpuKernelBuffers.PaddedBoolLength(n) elements");
}

int64_t Product(const std::string &operation, const std::string &name, const std::vector<int> &shape)
{
    int64_t n = 1;
    for (size_t i = 0; i < shape.size(); i++) {
        std::string dim = name + "[" + std::to_string(i) + "]";
        if (shape[i] < 0) throw GpuKernelShapeException(operation, dim, "dimension " + std::to_string(shape[i]) + " is negative");
        n *= shape[i];
        if (n > MaxElements) throw GpuKernelShapeException(operation, dim, "the tensor holds more than 2147483647 elements");
    }
    return n;
}

}  // namespace Check

namespace {

std::vector<std::shared_ptr<GpuBuffer::Impl>> keep_of(std::initializer_list<const GpuBuffer *> bs)
{
    std::vector<std::shared_ptr<GpuBuffer::Impl>> k;
    for (auto *b : bs)
        if (b && b->Valid()) k.push_back(b->impl());
    return k;
}

og_buffer bind(const GpuBuffer &b) { return b.Binding(); }

int axis_of(const std::string &operation, int axis, int rank)
{
    if (axis < -rank || axis >= rank)
        throw GpuKernelShapeException(operation, "axis", "axis " + std::to_string(axis) + " is outside [" +
                                                             std::to_string(-rank) + ", " + std::to_string(rank) + ")");
    return axis < 0 ? axis + rank : axis;
}

}  // namespace

// ------------------------------------------------------------------ Int8Gemm

static const char *kGemm = "Int8Gemm";

static bool is_int8(ElementType t) { return t == ElementType::UInt8 || t == ElementType::Int8; }

// Int8Gemm.cs:393-400.
static void RequireInt8(const GpuBuffer &b, const std::string &argument)
{
    if (!is_int8(b.Type()))
        throw GpuKernelShapeException(kGemm, argument, std::string("element type ") + ElementName(b.Type()) +
                                                           " is not supported; use byte (uint8) or sbyte (int8)");
}

// The C# signature types an operand by its generic parameter; here the buffer carries it.
static void RequireType(const std::string &op, const GpuBuffer &b, ElementType t, const std::string &argument)
{
    if (b.Type() != t)
        throw GpuKernelShapeException(op, argument, std::string("element type ") + ElementName(b.Type()) + " is not " + ElementName(t));
}

static void NonNegative(const std::string &argument, int value)
{
    if (value < 0) throw GpuKernelShapeException(kGemm, argument, "must not be negative, got " + std::to_string(value));
}

// Int8Gemm.cs:411-416.
static void CheckVector(const std::string &name, const GpuBuffer &buffer, int offset, bool isVector, int n)
{
    if (!buffer.Valid()) throw GpuKernelShapeException(kGemm, name, "buffer is null");
    Check::Range(kGemm, name, buffer.Length(), offset, isVector ? n : 1);
}

// Int8Gemm.cs:494-501.
static void CheckRange(const std::string &operand, int offset, int stride, int rows, int cols, int ld, int batch, int length)
{
    int64_t last = offset + ((int64_t)(batch - 1) * stride) + ((int64_t)(rows - 1) * ld) + (cols - 1);
    if (last >= length)
        throw GpuKernelShapeException(kGemm, "Offset" + operand, "operand " + operand + " reaches byte " + fmt_long(last) +
                                                                     " but its buffer holds " + std::to_string(length));
}

// ------------------------------------------------------------------ ArgumentBlocks

ArgumentBlocks::ArgumentBlocks(int capacity) : capacity_(capacity < 1 ? 1 : capacity) {}

void ArgumentBlocks::Note(uint64_t kind, std::initializer_list<const GpuBuffer *> buffers)
{
    std::vector<uintptr_t> key;
    key.reserve(buffers.size() + 1);
    key.push_back((uintptr_t)kind);
    for (const GpuBuffer *b : buffers) key.push_back((uintptr_t)(b && b->Valid() ? b->impl().get() : nullptr));
    ++clock_;
    for (auto &entry : blocks_)
        if (entry.first == key) {
            entry.second = clock_;
            return;
        }
    ++created_;
    if ((int)blocks_.size() >= capacity_) {
        auto oldest = blocks_.begin();
        for (auto it = blocks_.begin(); it != blocks_.end(); ++it)
            if (it->second < oldest->second) oldest = it;
        blocks_.erase(oldest);
    }
    blocks_.emplace_back(std::move(key), clock_);
}

Int8Gemm::Int8Gemm(std::shared_ptr<GpuDevice> device, Int8GemmOptions options, int maxCachedBindGroups)
    : device_(std::move(device)), options_(options), blocks_(maxCachedBindGroups)
{
    if (!device_) throw std::invalid_argument("device");
    if (maxCachedBindGroups < 1) throw std::out_of_range("maxCachedBindGroups");
    variant_ = options_.AllowPackedDot ? "mfma-i8-gfx950" : "portable-tile64x64x16";
}

Int8Gemm::~Int8Gemm() = default;

void Int8Gemm::Dispose() { scratch_.clear(); }

void Int8Gemm::CheckBindable(const std::string &operand, const GpuBuffer &buffer) const
{
    uint64_t maxBinding = device_->Capabilities().MaxStorageBufferBindingBytes;
    if (maxBinding != 0 && buffer.Size() > maxBinding)
        throw GpuUnsupportedException(std::string(kGemm) + ": operand " + operand + " is " + std::to_string(buffer.Size()) +
                                          " bytes, more than one storage binding can cover on " + device_->AdapterName(),
                                      "MaxStorageBufferBindingBytes", "at most " + std::to_string(maxBinding) + " bytes",
                                      std::to_string(buffer.Size()) + " bytes");
}

// Int8Gemm.cs:418-484.
Int8Gemm::Prepared Int8Gemm::Prepare(const Int8GemmProblem &p, const GpuBuffer &a, const GpuBuffer &b,
                                     const std::optional<Int8Operand> &zpA, const std::optional<Int8Operand> &zpB)
{
    if (!a.Valid()) throw GpuKernelShapeException(kGemm, "a", "buffer is null");
    if (!b.Valid()) throw GpuKernelShapeException(kGemm, "b", "buffer is null");
    RequireInt8(a, "a");
    RequireInt8(b, "b");
    NonNegative("M", p.M);
    NonNegative("N", p.N);
    NonNegative("K", p.K);
    NonNegative("OffsetA", p.OffsetA);
    NonNegative("OffsetB", p.OffsetB);
    NonNegative("OffsetC", p.OffsetC);
    NonNegative("StrideA", p.StrideA);
    NonNegative("StrideB", p.StrideB);
    NonNegative("Lda", p.Lda);
    NonNegative("Ldb", p.Ldb);
    if (p.Batch < 1) throw GpuKernelShapeException(kGemm, "Batch", "must be at least 1, got " + std::to_string(p.Batch));
    int lda = p.Lda == 0 ? std::max(p.K, 1) : p.Lda;
    int colsB = p.TransposeB ? p.K : p.N;
    int rowsB = p.TransposeB ? p.N : p.K;
    int ldb = p.Ldb == 0 ? std::max(colsB, 1) : p.Ldb;
    if (lda < p.K) throw GpuKernelShapeException(kGemm, "Lda", std::to_string(lda) + " is smaller than K = " + std::to_string(p.K));
    if (ldb < colsB) throw GpuKernelShapeException(kGemm, "Ldb", std::to_string(ldb) + " is smaller than the stored row length " + std::to_string(colsB));
    if ((int64_t)p.Batch * p.M * p.N > Check::MaxElements)
        throw GpuKernelShapeException(kGemm, "Batch", "the result holds more elements than the kernels address");
    if (p.M > 0 && p.N > 0 && p.K > 0) {
        CheckRange("A", p.OffsetA, p.StrideA, p.M, p.K, lda, p.Batch, a.Length());
        CheckRange("B", p.OffsetB, p.StrideB, rowsB, colsB, ldb, p.Batch, b.Length());
    }
    if (zpA) {
        if (zpA->Buffer.Valid()) RequireType(kGemm, zpA->Buffer, a.Type(), "zpA");
        CheckVector("zpA", zpA->Buffer, zpA->Offset, zpA->IsVector, p.M);
        CheckBindable("zero point A", zpA->Buffer);
    }
    if (zpB) {
        if (zpB->Buffer.Valid()) RequireType(kGemm, zpB->Buffer, b.Type(), "zpB");
        CheckVector("zpB", zpB->Buffer, zpB->Offset, zpB->IsVector, p.N);
        CheckBindable("zero point B", zpB->Buffer);
    }
    CheckBindable("A", a);
    CheckBindable("B", b);
    return Prepared{lda, ldb, p.M > 0 && p.N > 0};
}

void Int8Gemm::EncodeInt32(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                           const GpuBuffer &b, const GpuBuffer &c, const std::optional<Int8Operand> &zeroPointA,
                           const std::optional<Int8Operand> &zeroPointB, const std::optional<Int8Operand> &bias)
{
    if (!c.Valid()) throw GpuKernelShapeException(kGemm, "c", "buffer is null");
    auto prep = Prepare(problem, a, b, zeroPointA, zeroPointB);
    RequireType(kGemm, c, ElementType::Int32, "c");
    int64_t count = (int64_t)problem.Batch * problem.M * problem.N;
    Check::Range(kGemm, "c", c.Length(), problem.OffsetC, count);
    CheckBindable("C", c);
    Epilogue epi;
    if (bias) {
        if (bias->Buffer.Valid()) RequireType(kGemm, bias->Buffer, ElementType::Int32, "bias");
        CheckVector("bias", bias->Buffer, bias->Offset, true, problem.N);
        CheckBindable("bias", bias->Buffer);
        epi.Flags = OG_EPI_INT_BIAS;
        epi.IntBias = bias->Buffer;
        epi.OffIntBias = (uint32_t)bias->Offset;
    }
    if (!prep.Ok) return;
    Multiply(encoder, problem, a, a.Type() == ElementType::Int8, b, b.Type() == ElementType::Int8, c, problem.OffsetC,
             zeroPointA, zeroPointB, epi);
}

void Int8Gemm::EncodeFloat(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                           const GpuBuffer &b, const GpuBuffer &c, const Int8Operand &scale,
                           const std::optional<Int8Operand> &zeroPointA, const std::optional<Int8Operand> &zeroPointB,
                           const std::optional<Int8Operand> &floatBias, const std::optional<Int8Operand> &intBias)
{
    FloatProduct(encoder, problem, a, b, c, nullptr, scale, zeroPointA, zeroPointB, floatBias, intBias);
}

void Int8Gemm::EncodeFloatScaled(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                                 const GpuBuffer &b, const GpuBuffer &c, const Int8Operand &activationScale,
                                 const Int8Operand &weightScale, const std::optional<Int8Operand> &zeroPointA,
                                 const std::optional<Int8Operand> &zeroPointB,
                                 const std::optional<Int8Operand> &floatBias, const std::optional<Int8Operand> &intBias)
{
    FloatProduct(encoder, problem, a, b, c, &activationScale, weightScale, zeroPointA, zeroPointB, floatBias, intBias);
}

void Int8Gemm::EncodeFloatRanged(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                                 const GpuBuffer &b, const GpuBuffer &c, const Int8Operand &scale,
                                 const Int8Ranges &ranges, const std::optional<Int8Operand> &zeroPointA,
                                 const std::optional<Int8Operand> &zeroPointB,
                                 const std::optional<Int8Operand> &floatBias, const std::optional<Int8Operand> &intBias,
                                 const std::optional<Int8Operand> &activationScale)
{
    if (!ranges.Buffer.Valid()) throw GpuKernelShapeException(kGemm, "ranges", "buffer is null");
    RequireType(kGemm, ranges.Buffer, ElementType::Float32, "ranges");
    Check::Range(kGemm, "ranges", ranges.Buffer.Length(), 0, 2 * (int64_t)OG_RANGES_MAX);
    if ((int64_t)problem.Batch * problem.M * problem.N > 0x7FFFFFFF)
        throw GpuKernelShapeException(kGemm, "c", "a ranged product's output holds more than 2147483647 elements");
    FloatProduct(encoder, problem, a, b, c, activationScale ? &*activationScale : nullptr, scale, zeroPointA, zeroPointB,
                 floatBias, intBias, &ranges);
}

// EncodeFloat's checks and recording (Int8Gemm.cs:270-314), with the activation scale when there is one.
void Int8Gemm::FloatProduct(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                            const GpuBuffer &b, const GpuBuffer &c, const Int8Operand *activationScale,
                            const Int8Operand &scale, const std::optional<Int8Operand> &zeroPointA,
                            const std::optional<Int8Operand> &zeroPointB, const std::optional<Int8Operand> &floatBias,
                            const std::optional<Int8Operand> &intBias, const Int8Ranges *ranges)
{
    if (!c.Valid()) throw GpuKernelShapeException(kGemm, "c", "buffer is null");
    auto prep = Prepare(problem, a, b, zeroPointA, zeroPointB);
    RequireType(kGemm, c, ElementType::Float32, "c");
    int64_t count = (int64_t)problem.Batch * problem.M * problem.N;
    Check::Range(kGemm, "c", c.Length(), problem.OffsetC, count);
    CheckBindable("C", c);
    if (scale.Buffer.Valid()) RequireType(kGemm, scale.Buffer, ElementType::Float32, "scale");
    CheckVector("scale", scale.Buffer, scale.Offset, scale.IsVector, problem.N);
    if (activationScale) {
        if (activationScale->Buffer.Valid()) RequireType(kGemm, activationScale->Buffer, ElementType::Float32, "activationScale");
        CheckVector("activationScale", activationScale->Buffer, activationScale->Offset, false, problem.N);
    }
    if (floatBias) {
        if (floatBias->Buffer.Valid()) RequireType(kGemm, floatBias->Buffer, ElementType::Float32, "floatBias");
        CheckVector("floatBias", floatBias->Buffer, floatBias->Offset, true, problem.N);
    }
    if (!prep.Ok) {
        // An empty ranged product stores nothing and records no pairs: from its place in the submission on, its count
        // reads 0 (a host step, not a dispatch).
        if (ranges) encoder.RecordHost([groups = ranges->Groups](og_ctx *) { *groups = 0; });
        return;
    }
    Epilogue epi;
    epi.Flags = OG_EPI_FLOAT | (scale.IsVector ? OG_EPI_SCALE_PER_COL : 0u);
    if (intBias) {
        if (intBias->Buffer.Valid()) RequireType(kGemm, intBias->Buffer, ElementType::Int32, "intBias");
        CheckVector("intBias", intBias->Buffer, intBias->Offset, true, problem.N);
        CheckBindable("bias", intBias->Buffer);
        epi.Flags |= OG_EPI_INT_BIAS;
        epi.IntBias = intBias->Buffer;
        epi.OffIntBias = (uint32_t)intBias->Offset;
    }
    if (floatBias) {
        CheckBindable("float bias", floatBias->Buffer);
        epi.Flags |= OG_EPI_FLOAT_BIAS;
        epi.FloatBias = floatBias->Buffer;
        epi.OffFloatBias = (uint32_t)floatBias->Offset;
    }
    CheckBindable("scale", scale.Buffer);
    epi.Scale = scale.Buffer;
    epi.OffScale = (uint32_t)scale.Offset;
    if (activationScale) {
        epi.ActScale = activationScale->Buffer;
        epi.OffActScale = (uint32_t)activationScale->Offset;
    }
    epi.Ranges = ranges;
    Multiply(encoder, problem, a, a.Type() == ElementType::Int8, b, b.Type() == ElementType::Int8, c, problem.OffsetC,
             zeroPointA, zeroPointB, epi);
}

void Int8Gemm::EncodeRequantized(GpuCommandEncoder &encoder, const Int8GemmProblem &problem, const GpuBuffer &a,
                                 const GpuBuffer &b, const GpuBuffer &y, const Int8Operand &multiplier, int zeroPointY,
                                 const std::optional<Int8Operand> &zeroPointA, const std::optional<Int8Operand> &zeroPointB,
                                 const std::optional<Int8Operand> &intBias, const std::optional<Int8Scratch> &scratch)
{
    if (!y.Valid()) throw GpuKernelShapeException(kGemm, "y", "buffer is null");
    auto prep = Prepare(problem, a, b, zeroPointA, zeroPointB);
    RequireInt8(y, "y");
    bool outSigned = y.Type() == ElementType::Int8;
    if (zeroPointY < (outSigned ? -128 : 0) || zeroPointY > (outSigned ? 127 : 255))
        throw GpuKernelShapeException(kGemm, "zeroPointY", std::to_string(zeroPointY) + " is outside the output type's range");
    int64_t count = (int64_t)problem.Batch * problem.M * problem.N;
    Check::Range(kGemm, "y", y.Length(), problem.OffsetC, count);
    CheckBindable("Y", y);
    if (multiplier.Buffer.Valid()) RequireType(kGemm, multiplier.Buffer, ElementType::Float32, "multiplier");
    CheckVector("multiplier", multiplier.Buffer, multiplier.Offset, multiplier.IsVector, problem.N);
    if (!prep.Ok) return;
    if (options_.FusedRequantize) {
        // One launch; a given scratch is still checked as the two-pass form checks it (Int8Gemm.cs:503-523), and the
        // int bias as Finish checks it (655-661).
        if (scratch) Scratch(count, scratch);
        Epilogue rq;
        rq.Requantized = true;
        rq.ZeroPointY = zeroPointY;
        rq.SignedY = outSigned;
        rq.Scale = multiplier.Buffer;
        rq.OffScale = (uint32_t)multiplier.Offset;
        rq.Flags = multiplier.IsVector ? OG_EPI_SCALE_PER_COL : 0u;
        if (intBias) {
            if (intBias->Buffer.Valid()) RequireType(kGemm, intBias->Buffer, ElementType::Int32, "intBias");
            CheckVector("intBias", intBias->Buffer, intBias->Offset, true, problem.N);
            rq.Flags |= OG_EPI_INT_BIAS;
            rq.IntBias = intBias->Buffer;
            rq.OffIntBias = (uint32_t)intBias->Offset;
        }
        Multiply(encoder, problem, a, a.Type() == ElementType::Int8, b, b.Type() == ElementType::Int8, y,
                 problem.OffsetC, zeroPointA, zeroPointB, rq);
        return;
    }
    auto [sums, at] = Scratch(count, scratch);
    Epilogue none;
    Multiply(encoder, problem, a, a.Type() == ElementType::Int8, b, b.Type() == ElementType::Int8, sums, at, zeroPointA,
             zeroPointB, none);
    // Int8Gemm.Finish (Int8Gemm.cs:649-682), mode 2.
    uint32_t flags = (multiplier.IsVector ? 2u : 0u) | (outSigned ? 0u : 8u);
    uint32_t offBias = 0;
    GpuBuffer biasBuf;
    if (intBias) {
        if (intBias->Buffer.Valid()) RequireType(kGemm, intBias->Buffer, ElementType::Int32, "intBias");
        CheckVector("intBias", intBias->Buffer, intBias->Offset, true, problem.N);
        flags |= 1u;
        offBias = (uint32_t)intBias->Offset;
        biasBuf = intBias->Buffer;
    }
    og_int8_epilogue_params w{};
    w.Count = (uint32_t)count;
    w.OffAcc = (uint32_t)at;
    w.OffOut = (uint32_t)problem.OffsetC;
    w.N = (uint32_t)problem.N;
    w.Mode = 2;
    w.Flags = flags;
    w.OffBias = offBias;
    w.OffScale = (uint32_t)multiplier.Offset;
    w.ZeroPoint = zeroPointY;
    GpuBuffer mult = multiplier.Buffer;
    blocks_.Note(4, {&sums, &y, &biasBuf, &mult});
    encoder.Record(
        [w, sums, y, biasBuf, mult](og_ctx *ctx) {
            ThrowIfFailed(ctx, og_int8_epilogue(ctx, &w, bind(sums), bind(y), bind(biasBuf), bind(mult), og_buffer{nullptr, 0}), kGemm);
        },
        keep_of({&sums, &y, &biasBuf, &mult}));
}

int64_t Int8Gemm::ScratchElements(const Int8GemmProblem &problem)
{
    return problem.M <= 0 || problem.N <= 0 || problem.Batch <= 0 ? 0 : (int64_t)problem.Batch * problem.M * problem.N;
}

void Int8Gemm::ReserveScratch(int64_t elements)
{
    if (elements < 0 || elements > Check::MaxElements) throw std::out_of_range("elements");
    if (elements == 0 || (!scratch_.empty() && scratch_.back().Length() >= elements)) return;
    scratch_.push_back(device_->CreateBuffer(ElementType::Int32, (int)std::max<int64_t>(elements, 4096)));
}

// Int8Gemm.cs:503-523.
std::pair<GpuBuffer, int> Int8Gemm::Scratch(int64_t count, const std::optional<Int8Scratch> &given)
{
    if (given) {
        if (!given->Buffer.Valid()) throw GpuKernelShapeException(kGemm, "given", "buffer is null");
        RequireType(kGemm, given->Buffer, ElementType::Int32, "scratch");
        Check::Range(kGemm, "scratch", given->Buffer.Length(), given->Offset, count);
        CheckBindable("scratch", given->Buffer);
        return {given->Buffer, given->Offset};
    }
    if (!scratch_.empty() && scratch_.back().Length() >= count) return {scratch_.back(), 0};
    int64_t length = std::min<int64_t>(Check::MaxElements, std::max<int64_t>(count, !scratch_.empty() ? (int64_t)scratch_.back().Length() * 2 : 4096));
    scratch_.push_back(device_->CreateBuffer(ElementType::Int32, (int)length));
    return {scratch_.back(), 0};
}

// The library's product flags for Int8GemmOptions: the portable kernel, and the test hooks that pin a kernel.
static uint32_t OptionFlags(const Int8GemmOptions &o)
{
    uint32_t flags = 0;
    if (!o.AllowPackedDot) flags |= OG_GEMM_PORTABLE;
    if (o.Tile == 64) flags |= OG_GEMM_NO_SKINNY;
    if (o.Tile == 256) flags |= OG_GEMM_NO_SKINNY | OG_GEMM_LARGE_TILE;
    if (o.Tile == 32) flags |= OG_GEMM_NO_DIRECT | OG_GEMM_NO_STREAM;
    if (!o.FewRowsOneLaunch) flags |= OG_GEMM_TWO_PASS;
    return flags;
}

// Int8Gemm.cs:554-639: the 19 parameter words, then one og_int8_gemm call when the encoder is submitted.
void Int8Gemm::Multiply(GpuCommandEncoder &encoder, const Int8GemmProblem &p, const GpuBuffer &a, bool aSigned,
                        const GpuBuffer &b, bool bSigned, const GpuBuffer &c, int offsetC,
                        const std::optional<Int8Operand> &za, const std::optional<Int8Operand> &zb, const Epilogue &epi)
{
    int lda = p.Lda == 0 ? std::max(p.K, 1) : p.Lda;
    int ldb = p.Ldb == 0 ? std::max(p.TransposeB ? p.K : p.N, 1) : p.Ldb;
    uint32_t flags = (aSigned ? OG_GEMM_A_INT8 : 0u) | (bSigned ? OG_GEMM_B_INT8 : 0u) | (p.TransposeB ? OG_GEMM_TRANSPOSE_B : 0u);
    uint32_t offZa = 0, offZb = 0;
    GpuBuffer zaBuf, zbBuf;
    if (za) {
        flags |= OG_GEMM_ZA | (za->IsVector ? OG_GEMM_ZA_PER_ROW : 0u);
        offZa = (uint32_t)za->Offset;
        zaBuf = za->Buffer;
    }
    if (zb) {
        flags |= OG_GEMM_ZB | (zb->IsVector ? OG_GEMM_ZB_PER_COL : 0u);
        offZb = (uint32_t)zb->Offset;
        zbBuf = zb->Buffer;
    }
    // The reference's word-alignment bits (informational here: the library checks the addresses itself).
    if (((p.OffsetA | p.StrideA | lda) & 3) == 0) flags |= 128u;
    if (((p.OffsetB | p.StrideB | ldb) & 3) == 0) flags |= 256u;
    flags |= OptionFlags(options_);

    og_int8_gemm_params w{};
    w.M = (uint32_t)p.M;
    w.N = (uint32_t)p.N;
    w.K = (uint32_t)p.K;
    w.OffA = (uint32_t)p.OffsetA;
    w.OffB = (uint32_t)p.OffsetB;
    w.OffC = (uint32_t)offsetC;
    w.StrideA = (uint32_t)p.StrideA;
    w.StrideB = (uint32_t)p.StrideB;
    w.StrideC = (uint32_t)((int64_t)p.M * p.N);
    w.Lda = (uint32_t)lda;
    w.Ldb = (uint32_t)ldb;
    w.Flags = flags;
    w.OffZA = offZa;
    w.OffZB = offZb;
    w.Epi = epi.Flags;
    w.OffBias = epi.OffIntBias;
    w.OffScale = epi.OffScale;
    w.OffFBias = epi.OffFloatBias;
    w.GridX = 0;
    uint32_t batch = (uint32_t)p.Batch;
    GpuBuffer A = a, B = b, C = c, ib = epi.IntBias, sc = epi.Scale, fb = epi.FloatBias;
    if (epi.Requantized) {
        const int32_t zy = epi.ZeroPointY;
        const uint32_t ys = epi.SignedY ? 1u : 0u;
        blocks_.Note(3, {&A, &B, &C, &zaBuf, &zbBuf, &ib, &sc});
        encoder.Record(
            [w, batch, A, B, C, zaBuf, zbBuf, ib, sc, zy, ys](og_ctx *ctx) {
                ThrowIfFailed(ctx, og_int8_gemm_requantized(ctx, &w, batch, bind(A), bind(B), bind(C), bind(zaBuf), bind(zbBuf), bind(ib), bind(sc), zy, ys), kGemm);
            },
            keep_of({&A, &B, &C, &zaBuf, &zbBuf, &ib, &sc}));
        return;
    }
    if (epi.Ranges) {
        GpuBuffer as = epi.ActScale, rg = epi.Ranges->Buffer;
        const uint32_t aoff = epi.OffActScale;
        std::shared_ptr<uint32_t> groups = epi.Ranges->Groups;
        blocks_.Note(4, {&A, &B, &C, &zaBuf, &zbBuf, &ib, &as, &sc, &fb, &rg});
        encoder.Record(
            [w, batch, A, B, C, zaBuf, zbBuf, ib, as, aoff, sc, fb, rg, groups](og_ctx *ctx) {
                ThrowIfFailed(ctx, og_int8_gemm_float_ranged(ctx, &w, batch, bind(A), bind(B), bind(C), bind(zaBuf), bind(zbBuf), bind(ib), bind(as), aoff, bind(sc), bind(fb), bind(rg), groups.get()), kGemm);
            },
            keep_of({&A, &B, &C, &zaBuf, &zbBuf, &ib, &as, &sc, &fb, &rg}));
        return;
    }
    if (epi.ActScale.Valid()) {
        GpuBuffer as = epi.ActScale;
        const uint32_t aoff = epi.OffActScale;
        blocks_.Note(2, {&A, &B, &C, &zaBuf, &zbBuf, &ib, &as, &sc, &fb});
        encoder.Record(
            [w, batch, A, B, C, zaBuf, zbBuf, ib, as, aoff, sc, fb](og_ctx *ctx) {
                ThrowIfFailed(ctx, og_int8_gemm_float_scaled(ctx, &w, batch, bind(A), bind(B), bind(C), bind(zaBuf), bind(zbBuf), bind(ib), bind(as), aoff, bind(sc), bind(fb)), kGemm);
            },
            keep_of({&A, &B, &C, &zaBuf, &zbBuf, &ib, &as, &sc, &fb}));
        return;
    }
    blocks_.Note(1, {&A, &B, &C, &zaBuf, &zbBuf, &ib, &sc, &fb});
    encoder.Record(
        [w, batch, A, B, C, zaBuf, zbBuf, ib, sc, fb](og_ctx *ctx) {
            ThrowIfFailed(ctx, og_int8_gemm(ctx, &w, batch, bind(A), bind(B), bind(C), bind(zaBuf), bind(zbBuf), bind(ib), bind(sc), bind(fb)), kGemm);
        },
        keep_of({&A, &B, &C, &zaBuf, &zbBuf, &ib, &sc, &fb}));
}

Int8Ranges::Int8Ranges(GpuBuffer buffer) : Buffer(std::move(buffer)) {}

// ------------------------------------------------------------------ DynamicQuantizeKernels

DynamicQuantizeKernels::DynamicQuantizeKernels(std::shared_ptr<GpuDevice> device, int maxCachedBindGroups)
    : device_(std::move(device)), blocks_(maxCachedBindGroups)
{
    if (!device_) throw std::invalid_argument("device");
    if (maxCachedBindGroups < 1) throw std::out_of_range("maxCachedBindGroups");
}

void DynamicQuantizeKernels::Encode(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, int count,
                                    const GpuBuffer &y, int offsetY, const GpuBuffer &scale, int offsetScale,
                                    const GpuBuffer &zeroPoint, int offsetZeroPoint)
{
    const std::string Name = "DynamicQuantizeLinear";
    if (!x.Valid()) throw GpuKernelShapeException(Name, "x", "buffer is null");
    if (!y.Valid()) throw GpuKernelShapeException(Name, "y", "buffer is null");
    if (!scale.Valid()) throw GpuKernelShapeException(Name, "scale", "buffer is null");
    if (!zeroPoint.Valid()) throw GpuKernelShapeException(Name, "zeroPoint", "buffer is null");
    RequireType(Name, x, ElementType::Float32, "x");
    RequireType(Name, y, ElementType::UInt8, "y");
    RequireType(Name, scale, ElementType::Float32, "scale");
    RequireType(Name, zeroPoint, ElementType::UInt8, "zeroPoint");
    if (count < 1) throw GpuKernelShapeException(Name, "count", "count " + std::to_string(count) + " must be at least 1");
    Check::Range(Name, "x", x.Length(), offsetX, count);
    Check::Range(Name, "y", y.Length(), offsetY, count);
    Check::Range(Name, "scale", scale.Length(), offsetScale, 1);
    Check::Range(Name, "zeroPoint", zeroPoint.Length(), offsetZeroPoint, 1);
    og_dq_params w{};
    w.Count = (uint32_t)count;
    w.OffX = (uint32_t)offsetX;
    w.OffY = (uint32_t)offsetY;
    w.OffScale = (uint32_t)offsetScale;
    w.OffZero = (uint32_t)offsetZeroPoint;
    GpuBuffer X = x, Y = y, S = scale, Z = zeroPoint;
    blocks_.Note(1, {&X});                 // the range pass
    blocks_.Note(2, {&X, &Y, &S, &Z});     // the quantize pass
    encoder.Record(
        [w, X, Y, S, Z](og_ctx *ctx) {
            ThrowIfFailed(ctx, og_dynamic_quantize(ctx, &w, bind(X), bind(Y), bind(S), bind(Z)), "DynamicQuantizeLinear");
        },
        keep_of({&X, &Y, &S, &Z}));
}

void DynamicQuantizeKernels::EncodeRanged(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, int count,
                                          const GpuBuffer &y, int offsetY, const GpuBuffer &scale, int offsetScale,
                                          const GpuBuffer &zeroPoint, int offsetZeroPoint, const Int8Ranges &ranges)
{
    const std::string Name = "DynamicQuantizeLinear";
    if (!x.Valid()) throw GpuKernelShapeException(Name, "x", "buffer is null");
    if (!y.Valid()) throw GpuKernelShapeException(Name, "y", "buffer is null");
    if (!scale.Valid()) throw GpuKernelShapeException(Name, "scale", "buffer is null");
    if (!zeroPoint.Valid()) throw GpuKernelShapeException(Name, "zeroPoint", "buffer is null");
    if (!ranges.Buffer.Valid()) throw GpuKernelShapeException(Name, "ranges", "buffer is null");
    RequireType(Name, x, ElementType::Float32, "x");
    RequireType(Name, y, ElementType::UInt8, "y");
    RequireType(Name, scale, ElementType::Float32, "scale");
    RequireType(Name, zeroPoint, ElementType::UInt8, "zeroPoint");
    RequireType(Name, ranges.Buffer, ElementType::Float32, "ranges");
    if (count < 1) throw GpuKernelShapeException(Name, "count", "count " + std::to_string(count) + " must be at least 1");
    Check::Range(Name, "x", x.Length(), offsetX, count);
    Check::Range(Name, "y", y.Length(), offsetY, count);
    Check::Range(Name, "scale", scale.Length(), offsetScale, 1);
    Check::Range(Name, "zeroPoint", zeroPoint.Length(), offsetZeroPoint, 1);
    Check::Range(Name, "ranges", ranges.Buffer.Length(), 0, 2 * (int64_t)OG_RANGES_MAX);
    og_dq_params w{};
    w.Count = (uint32_t)count;
    w.OffX = (uint32_t)offsetX;
    w.OffY = (uint32_t)offsetY;
    w.OffScale = (uint32_t)offsetScale;
    w.OffZero = (uint32_t)offsetZeroPoint;
    GpuBuffer X = x, Y = y, S = scale, Z = zeroPoint, R = ranges.Buffer;
    std::shared_ptr<uint32_t> groups = ranges.Groups;
    blocks_.Note(3, {&X, &Y, &S, &Z, &R});   // the quantize pass over the recorded ranges
    encoder.Record(
        [w, X, Y, S, Z, R, groups](og_ctx *ctx) {
            // The ranged product recorded before this pass has run by now (Submit runs the recorded work in order).
            ThrowIfFailed(ctx, og_dynamic_quantize_ranged(ctx, &w, bind(X), bind(Y), bind(S), bind(Z), bind(R), *groups),
                          "DynamicQuantizeLinear");
        },
        keep_of({&X, &Y, &S, &Z, &R}));
}

// ------------------------------------------------------------------ DequantizeKernels

DequantizeKernels::DequantizeKernels(std::shared_ptr<GpuDevice> device, int maxCachedBindGroups)
    : device_(std::move(device)), blocks_(maxCachedBindGroups)
{
    if (!device_) throw std::invalid_argument("device");
    if (maxCachedBindGroups < 1) throw std::out_of_range("maxCachedBindGroups");
}

// KernelTypes.IsHalf<T> (KernelSupport.cs:49-65): float or Half, anything else named as T.
static bool IsHalf(const std::string &operation, ElementType t)
{
    switch (t) {
    case ElementType::Float32: return false;
    case ElementType::Float16: return true;
    case ElementType::Int32:
    case ElementType::Int64:
    case ElementType::UInt32:
        throw GpuKernelShapeException(operation, "T", std::string("element type ") + ElementName(t) + " is not supported; use float or Half");
    default:
        throw GpuKernelShapeException(operation, "T", std::string("element type ") + ElementName(t) +
                                                          " is not supported; use float, Half, int, long or uint as the operation allows");
    }
}

static void split_axis(const std::string &op, const std::vector<int> &shape, int axis, bool perAxis, int64_t &axisLen,
                       int64_t &inner)
{
    axisLen = 1;
    inner = 1;
    if (!perAxis) return;
    int rank = (int)shape.size();
    int ax = axis_of(op, axis, rank);
    axisLen = shape[ax];
    for (int i = ax + 1; i < rank; i++) inner *= shape[i];
}

void DequantizeKernels::Encode(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX, const std::vector<int> &shape,
                               int axis, bool perAxis, const GpuBuffer &scale, int offsetScale,
                               const std::optional<GpuBuffer> &zeroPoint, int offsetZeroPoint, const GpuBuffer &output,
                               int offsetOutput)
{
    const std::string Name = "DequantizeLinear";
    if (!x.Valid()) throw GpuKernelShapeException(Name, "x", "buffer is null");
    if (!scale.Valid()) throw GpuKernelShapeException(Name, "scale", "buffer is null");
    if (!output.Valid()) throw GpuKernelShapeException(Name, "output", "buffer is null");
    int kind;
    switch (x.Type()) {
    case ElementType::UInt8: kind = OG_KIND_U8; break;
    case ElementType::Int8: kind = OG_KIND_I8; break;
    case ElementType::Int32: kind = OG_KIND_I32; break;
    default:
        throw GpuKernelShapeException(Name, "TIn", std::string("element type ") + ElementName(x.Type()) +
                                                       " is not supported; use byte (uint8), sbyte (int8) or int");
    }
    bool half = IsHalf(Name, output.Type());
    int64_t count = Check::Product(Name, "shape", shape);
    int64_t axisLen, inner;
    split_axis(Name, shape, axis, perAxis, axisLen, inner);
    int64_t parameters = perAxis ? axisLen : 1;
    RequireType(Name, scale, ElementType::Float32, "scale");
    Check::Range(Name, "scale", scale.Length(), offsetScale, parameters);
    if (kind == OG_KIND_I32) Check::Range(Name, "x", x.Length(), offsetX, count);
    else Check::RangeBytes(Name, "x", x.Length(), offsetX, count);
    if (zeroPoint) {
        RequireType(Name, *zeroPoint, x.Type(), "zeroPoint");
        if (kind == OG_KIND_I32) Check::Range(Name, "zeroPoint", zeroPoint->Length(), offsetZeroPoint, parameters);
        else Check::RangeBytes(Name, "zeroPoint", zeroPoint->Length(), offsetZeroPoint, parameters);
    }
    Check::Range(Name, "output", output.Length(), offsetOutput, count, half);
    if (count == 0) return;
    og_dequant_params w{};
    w.Count = (uint32_t)count;
    w.OffX = (uint32_t)offsetX;
    w.OffO = (uint32_t)offsetOutput;
    w.OffS = (uint32_t)offsetScale;
    w.OffZ = (uint32_t)offsetZeroPoint;
    w.Flags = (perAxis ? 1u : 0u) | (zeroPoint ? 2u : 0u);
    w.AxisLen = (uint32_t)axisLen;
    w.Inner = (uint32_t)std::max<int64_t>(inner, 1);
    GpuBuffer X = x, S = scale, Z = zeroPoint ? *zeroPoint : GpuBuffer(), O = output;
    blocks_.Note(1 + 2 * (uint64_t)kind + (half ? 1 : 0), {&X, &S, &Z, &O});
    DequantCommand c;
    c.kind = kind;
    c.half = half;
    c.params = w;
    c.x = X;
    c.scale = S;
    c.zero = Z;
    c.out = O;
    encoder.RecordDequant(std::move(c), keep_of({&X, &S, &Z, &O}));
}

void DequantizeKernels::EncodeQuantize(GpuCommandEncoder &encoder, const GpuBuffer &x, int offsetX,
                                       const std::vector<int> &shape, int axis, bool perAxis, const GpuBuffer &scale,
                                       int offsetScale, const std::optional<GpuBuffer> &zeroPoint, int offsetZeroPoint,
                                       const GpuBuffer &output, int offsetOutput)
{
    const std::string QName = "QuantizeLinear";
    if (!x.Valid()) throw GpuKernelShapeException(QName, "x", "buffer is null");
    if (!scale.Valid()) throw GpuKernelShapeException(QName, "scale", "buffer is null");
    if (!output.Valid()) throw GpuKernelShapeException(QName, "output", "buffer is null");
    bool isSigned;
    switch (output.Type()) {
    case ElementType::UInt8: isSigned = false; break;
    case ElementType::Int8: isSigned = true; break;
    default:
        throw GpuKernelShapeException(QName, "TOut", std::string("element type ") + ElementName(output.Type()) +
                                                         " is not supported; use byte (uint8) or sbyte (int8)");
    }
    bool half = IsHalf(QName, x.Type());
    int64_t count = Check::Product(QName, "shape", shape);
    int64_t axisLen, inner;
    split_axis(QName, shape, axis, perAxis, axisLen, inner);
    int64_t parameters = perAxis ? axisLen : 1;
    Check::Range(QName, "x", x.Length(), offsetX, count, half);
    RequireType(QName, scale, ElementType::Float32, "scale");
    Check::Range(QName, "scale", scale.Length(), offsetScale, parameters);
    if (zeroPoint) {
        RequireType(QName, *zeroPoint, output.Type(), "zeroPoint");
        Check::RangeBytes(QName, "zeroPoint", zeroPoint->Length(), offsetZeroPoint, parameters);
    }
    Check::RangeBytes(QName, "output", output.Length(), offsetOutput, count);
    if (count == 0) return;
    og_dequant_params w{};
    w.Count = (uint32_t)count;
    w.OffX = (uint32_t)offsetX;
    w.OffO = (uint32_t)offsetOutput;
    w.OffS = (uint32_t)offsetScale;
    w.OffZ = (uint32_t)offsetZeroPoint;
    w.Flags = (perAxis ? 1u : 0u) | (zeroPoint ? 2u : 0u);
    w.AxisLen = (uint32_t)axisLen;
    w.Inner = (uint32_t)std::max<int64_t>(inner, 1);
    GpuBuffer X = x, S = scale, Z = zeroPoint ? *zeroPoint : GpuBuffer(), O = output;
    blocks_.Note(16 + 2 * (isSigned ? 1 : 0) + (half ? 1 : 0), {&X, &S, &Z, &O});
    encoder.Record(
        [w, isSigned, half, X, S, Z, O](og_ctx *ctx) {
            ThrowIfFailed(ctx, og_quantize(ctx, isSigned ? 1 : 0, half ? 1 : 0, &w, bind(X), bind(S), bind(Z), bind(O)), "QuantizeLinear");
        },
        keep_of({&X, &S, &Z, &O}));
}

// ------------------------------------------------------------------ Gather

GpuIndexStatus::GpuIndexStatus(std::shared_ptr<GpuDevice> device) : device_(std::move(device))
{
    if (!device_) throw std::invalid_argument("device");
    buffer_ = device_->CreateBuffer(ElementType::UInt32, 1);
    Reset();
}

void GpuIndexStatus::Reset()
{
    const uint32_t none = 0xFFFFFFFFu;
    buffer_.Write(&none, 4);
}

void GpuIndexStatus::ThrowIfFailed()
{
    uint32_t word = 0;
    device_->WaitIdle();
    buffer_.Read(&word, 4);
    if (word != 0xFFFFFFFFu) throw GpuKernelIndexException(operation_.empty() ? "index operation" : operation_, word);
}

GatherKernels::GatherKernels(std::shared_ptr<GpuDevice> device, int maxCachedBindGroups)
    : device_(std::move(device)), blocks_(maxCachedBindGroups)
{
    if (!device_) throw std::invalid_argument("device");
    if (maxCachedBindGroups < 1) throw std::out_of_range("maxCachedBindGroups");
}

// IndexSupport.Width (IndexSupport.cs:7-28): 0 halves, 1 four-byte values, 2 eight-byte values, 3 bytes.
static int PayloadWidth(const std::string &operation, ElementType t)
{
    switch (t) {
    case ElementType::UInt8:
    case ElementType::Int8: return 3;
    case ElementType::Float16: return 0;
    case ElementType::Int64: return 2;
    case ElementType::Float32:
    case ElementType::Int32:
    case ElementType::UInt32: return 1;
    default: throw GpuKernelShapeException(operation, "T", std::string("element type ") + ElementName(t) + " is not supported here");
    }
}

// GatherKernels.cs:66-118.
void GatherKernels::EncodeGather(GpuCommandEncoder &encoder, const GpuBuffer &data, int offsetData,
                                 const std::vector<int> &dataShape, int axis, const GpuBuffer &indices, int offsetIndices,
                                 int indexCount, const GpuBuffer &output, int offsetOutput, GpuIndexStatus *status)
{
    const std::string Name = "Gather";
    if (!data.Valid()) throw GpuKernelShapeException(Name, "data", "buffer is null");
    if (!indices.Valid()) throw GpuKernelShapeException(Name, "indices", "buffer is null");
    if (!output.Valid()) throw GpuKernelShapeException(Name, "output", "buffer is null");
    const int width = PayloadWidth(Name, data.Type());
    if (output.Type() != data.Type()) throw GpuKernelShapeException(Name, "output", "the output's element type differs from the data's");
    if (indices.Type() != ElementType::Int32 && indices.Type() != ElementType::Int64)
        throw GpuKernelShapeException(Name, "TIndex", std::string("index type ") + ElementName(indices.Type()) + " is not supported; use int or long");
    const bool wide = indices.Type() == ElementType::Int64;
    const int rank = (int)dataShape.size();
    if (rank == 0) throw GpuKernelShapeException(Name, "dataShape", "a scalar has no axis to gather along");
    if (axis < -rank || axis >= rank)
        throw GpuKernelShapeException(Name, "axis", "axis " + std::to_string(axis) + " is outside [" + std::to_string(-rank) + ", " + std::to_string(rank) + ")");
    const int ax = axis < 0 ? axis + rank : axis;
    const int64_t dataCount = Check::Product(Name, "dataShape", dataShape);
    if (indexCount < 0) throw GpuKernelShapeException(Name, "indexCount", "count " + std::to_string(indexCount) + " is negative");
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < ax; i++) outer *= dataShape[i];
    for (int i = ax + 1; i < rank; i++) inner *= dataShape[i];
    const int64_t axisLength = dataShape[ax];
    const int64_t total = outer * indexCount * inner;
    if (total > Check::MaxElements)
        throw GpuKernelShapeException(Name, "indexCount", "the output holds " + std::to_string(total) + " elements, more than the " + std::to_string(Check::MaxElements) + " the kernels address");
    const int64_t elemWidth = width == 2 ? 2 : 1;
    auto range = [&](const char *name, const GpuBuffer &b, int offset, int64_t extent) {
        if (width == 3) Check::RangeBytes(Name, name, b.Length(), offset, extent);
        else Check::Range(Name, name, b.Length(), offset, extent, width == 0);
    };
    range("data", data, offsetData, dataCount);
    Check::Range(Name, "indices", indices.Length(), offsetIndices, indexCount);
    range("output", output, offsetOutput, total);
    const int64_t limit = 0xFFFFFFFFll / 2;   // GatherKernels.CheckAddressable (GatherKernels.cs:393-400)
    if (dataCount * elemWidth > limit || total * elemWidth > limit || (int64_t)indexCount * (wide ? 2 : 1) > limit)
        throw GpuKernelShapeException(Name, "shape", "a tensor is too large for 32-bit word addressing");
    if (total == 0) return;
    if (status) status->Note(Name);
    og_gather_params w{};
    w.Count = (uint32_t)total;
    w.OffData = (uint32_t)offsetData;
    w.OffOut = (uint32_t)offsetOutput;
    w.OffIdx = (uint32_t)offsetIndices;
    w.Flags = wide ? 1u : 0u;
    w.Inner = (uint32_t)inner;
    w.IdxCount = (uint32_t)indexCount;
    w.AxisLen = (uint32_t)axisLength;
    const uint32_t eb = (uint32_t)ElementSize(data.Type());
    GpuBuffer D = data, I = indices, O = output, S = status ? status->Buffer() : GpuBuffer();
    blocks_.Note(eb, {&D, &I, &O, &S});
    encoder.Record(
        [w, eb, D, I, O, S](og_ctx *ctx) {
            ThrowIfFailed(ctx, og_gather(ctx, eb, &w, bind(D), bind(I), bind(O), bind(S)), "Gather");
        },
        keep_of({&D, &I, &O, &S}));
}

// ------------------------------------------------------------------ ConvInteger

ConvProblem ConvProblem::Conv1D(int batch, int inChannels, int length, int outChannels, int kernel, int stride,
                                int dilation, int padBegin, int padEnd, int groups)
{
    ConvProblem p(batch, inChannels, 1, length, outChannels, 1, kernel);
    p.StrideWidth = stride;
    p.DilationWidth = dilation;
    p.PadLeft = padBegin;
    p.PadRight = padEnd;
    p.Groups = groups;
    return p;
}

static int OutputExtent(int input, int kernel, int stride, int dilation, int padBegin, int padEnd)
{
    if (input < 1 || kernel < 1 || stride < 1 || dilation < 1) return 0;
    const int64_t effective = (int64_t)dilation * (kernel - 1) + 1;
    const int64_t span = (int64_t)input + padBegin + padEnd - effective;
    if (span < 0) return 0;
    const int64_t extent = span / stride + 1;
    return extent > INT32_MAX ? 0 : (int)extent;
}

int ConvProblem::OutHeight() const { return OutputExtent(Height, KernelHeight, StrideHeight, DilationHeight, PadTop, PadBottom); }
int ConvProblem::OutWidth() const { return OutputExtent(Width, KernelWidth, StrideWidth, DilationWidth, PadLeft, PadRight); }

static const char *kConv = "ConvInteger";

// ConvKernels.CheckWindow / CheckConv (ConvKernels.cs:895-956).
static void CheckWindow(const std::string &axis, int input, int kernel, int stride, int dilation, int padBegin, int padEnd)
{
    if (input < 1) throw GpuKernelShapeException(kConv, axis + " input", "extent " + std::to_string(input) + " must be at least 1");
    if (kernel < 1) throw GpuKernelShapeException(kConv, axis + " kernel", "extent " + std::to_string(kernel) + " must be at least 1");
    if (stride < 1) throw GpuKernelShapeException(kConv, axis + " stride", "stride " + std::to_string(stride) + " must be at least 1");
    if (dilation < 1) throw GpuKernelShapeException(kConv, axis + " dilation", "dilation " + std::to_string(dilation) + " must be at least 1");
    if (padBegin < 0 || padEnd < 0) throw GpuKernelShapeException(kConv, axis + " padding", "padding must not be negative");
    if ((int64_t)kernel * dilation > Check::MaxElements || (int64_t)padBegin + padEnd + input > Check::MaxElements)
        throw GpuKernelShapeException(kConv, axis, "the window or padding is larger than the supported sizes");
}

// ConvIntegerKernels.Geometry (ConvIntegerKernels.cs:296-318), with the column rows padded to 16 bytes.
static void ConvGeometry(const ConvProblem &p, int &oh, int &ow, int64_t &k, int64_t &ldb)
{
    oh = p.OutHeight();
    ow = p.OutWidth();
    if (p.Batch < 1) throw GpuKernelShapeException(kConv, "Batch", "batch " + std::to_string(p.Batch) + " must be at least 1");
    if (p.InChannels < 1 || p.OutChannels < 1)
        throw GpuKernelShapeException(kConv, p.InChannels < 1 ? "InChannels" : "OutChannels", "channel counts must be at least 1");
    if (p.Groups < 1 || p.InChannels % p.Groups != 0 || p.OutChannels % p.Groups != 0)
        throw GpuKernelShapeException(kConv, "Groups", std::to_string(p.Groups) + " groups do not divide " + std::to_string(p.InChannels) +
                                                          " input and " + std::to_string(p.OutChannels) + " output channels");
    CheckWindow("height", p.Height, p.KernelHeight, p.StrideHeight, p.DilationHeight, p.PadTop, p.PadBottom);
    CheckWindow("width", p.Width, p.KernelWidth, p.StrideWidth, p.DilationWidth, p.PadLeft, p.PadRight);
    if (oh < 1) throw GpuKernelShapeException(kConv, "height", "the kernel does not fit the padded input");
    if (ow < 1) throw GpuKernelShapeException(kConv, "width", "the kernel does not fit the padded input");
    k = (int64_t)(p.InChannels / p.Groups) * p.KernelHeight * p.KernelWidth;
    ldb = ((int64_t)oh * ow + 15) / 16 * 16;
    if (k > Check::MaxElements || ldb > Check::MaxElements || (int64_t)p.Batch * p.InChannels * p.Height * p.Width > Check::MaxElements)
        throw GpuKernelShapeException(kConv, "shape", "the convolution is larger than the supported sizes");
}

ConvIntegerKernels::ConvIntegerKernels(std::shared_ptr<GpuDevice> device, Int8GemmOptions options, int maxCachedBindGroups)
    : device_(device), options_(options), gemm_(device, options, maxCachedBindGroups), blocks_(maxCachedBindGroups)
{
    if (!device_) throw std::invalid_argument("device");
}

int64_t ConvIntegerKernels::ScratchBytesPerImage(const ConvProblem &problem)
{
    int oh, ow;
    int64_t k, ldb;
    ConvGeometry(problem, oh, ow, k, ldb);   // throws for a geometry the library would refuse
    // The library's figure: one image's column matrices, with their depth padded to a multiple of 64 (and the padded
    // weight copy ahead of them) where that lets the products take the LDS-DMA kernel.
    og_conv_params c{};
    c.Batch = 1;
    c.InChannels = (uint32_t)problem.InChannels;
    c.Height = (uint32_t)problem.Height;
    c.Width = (uint32_t)problem.Width;
    c.OutChannels = (uint32_t)problem.OutChannels;
    c.KernelHeight = (uint32_t)problem.KernelHeight;
    c.KernelWidth = (uint32_t)problem.KernelWidth;
    c.StrideHeight = (uint32_t)problem.StrideHeight;
    c.StrideWidth = (uint32_t)problem.StrideWidth;
    c.DilationHeight = (uint32_t)problem.DilationHeight;
    c.DilationWidth = (uint32_t)problem.DilationWidth;
    c.PadTop = (uint32_t)problem.PadTop;
    c.PadLeft = (uint32_t)problem.PadLeft;
    c.PadBottom = (uint32_t)problem.PadBottom;
    c.PadRight = (uint32_t)problem.PadRight;
    c.Groups = (uint32_t)problem.Groups;
    const uint64_t bytes = og_conv_integer_scratch_bytes(&c);
    if (bytes == 0 || bytes > (uint64_t)Check::MaxElements)
        throw GpuKernelShapeException(kConv, "InChannels", "the column matrix of one image is larger than the supported sizes");
    return (int64_t)bytes;
}

GpuBuffer ConvIntegerKernels::Own(ElementType t, int64_t bytes)
{
    GpuBuffer &own = t == ElementType::Int8 ? own_i8_ : own_u8_;
    int64_t want = std::min<int64_t>(Check::MaxElements, std::max<int64_t>(bytes, 4096));
    if (!own.Valid() || own.Length() < want) {
        if (own.Valid()) {
            retired_.push_back(own);
            want = std::min<int64_t>(Check::MaxElements, std::max<int64_t>(want, (int64_t)own.Length() * 2));
        }
        own = device_->CreateBuffer(t, (int)want);
    }
    return own;
}

void ConvIntegerKernels::Encode(GpuCommandEncoder &encoder, const ConvProblem &problem, const GpuBuffer &x,
                                const GpuBuffer &w, const GpuBuffer &y, const std::optional<Int8Operand> &xZeroPoint,
                                const std::optional<Int8Operand> &wZeroPoint, const std::optional<GpuBuffer> &scratch,
                                int scratchOffset)
{
    if (!x.Valid()) throw GpuKernelShapeException(kConv, "x", "buffer is null");
    if (!w.Valid()) throw GpuKernelShapeException(kConv, "w", "buffer is null");
    if (!y.Valid()) throw GpuKernelShapeException(kConv, "y", "buffer is null");
    auto requireInt8 = [](const GpuBuffer &b, const char *arg) {
        if (b.Type() != ElementType::UInt8 && b.Type() != ElementType::Int8)
            throw GpuKernelShapeException(kConv, arg, std::string("element type ") + ElementName(b.Type()) +
                                                          " is not supported; use byte (uint8) or sbyte (int8)");
    };
    requireInt8(x, "x");
    requireInt8(w, "w");
    RequireType(kConv, y, ElementType::Int32, "y");
    const ConvProblem &p = problem;
    int oh, ow;
    int64_t k, ldb;
    ConvGeometry(p, oh, ow, k, ldb);
    const int64_t nCols = (int64_t)oh * ow;
    if (p.Activation != 0) throw GpuKernelShapeException(kConv, "Activation", "an integer convolution has no fused activation");
    const int64_t xImage = (int64_t)p.InChannels * p.Height * p.Width;
    const int64_t yImage = (int64_t)p.OutChannels * nCols;
    Check::Range(kConv, "x", x.Length(), p.OffsetX, xImage * p.Batch);
    Check::Range(kConv, "w", w.Length(), p.OffsetW, (int64_t)p.OutChannels * k);
    Check::Range(kConv, "y", y.Length(), p.OffsetY, yImage * p.Batch);
    if (p.OffsetY < 0 || (int64_t)p.OffsetY + yImage * p.Batch > Check::MaxElements)
        throw GpuKernelShapeException(kConv, "y", "the result is larger than the supported sizes");
    if (xZeroPoint) {
        if (!xZeroPoint->Buffer.Valid()) throw GpuKernelShapeException(kConv, "xZeroPoint", "buffer is null");
        if (xZeroPoint->Buffer.Type() != x.Type()) throw GpuKernelShapeException(kConv, "xZeroPoint", "the zero point has a different type than x");
        Check::Range(kConv, "xZeroPoint", xZeroPoint->Buffer.Length(), xZeroPoint->Offset, 1);
        if (xZeroPoint->IsVector) throw GpuKernelShapeException(kConv, "xZeroPoint", "the zero point of x is a single value");
    }
    if (wZeroPoint) {
        if (!wZeroPoint->Buffer.Valid()) throw GpuKernelShapeException(kConv, "wZeroPoint", "buffer is null");
        if (wZeroPoint->Buffer.Type() != w.Type()) throw GpuKernelShapeException(kConv, "wZeroPoint", "the zero point has a different type than w");
        Check::Range(kConv, "wZeroPoint", wZeroPoint->Buffer.Length(), wZeroPoint->Offset, wZeroPoint->IsVector ? p.OutChannels : 1);
    }
    const int64_t perImage = ScratchBytesPerImage(p);
    const bool depthwise = DirectDepthwise && p.InChannels == p.Groups;   // one input channel a group: convolved directly
    // x is the matrix as it lies (the library's rule: a 1 x 1 window, unit strides, no padding, 16-byte rows and start)
    const bool pointwise = p.KernelHeight == 1 && p.KernelWidth == 1 && p.StrideHeight == 1 && p.StrideWidth == 1 &&
                           p.PadTop == 0 && p.PadLeft == 0 && p.PadBottom == 0 && p.PadRight == 0 &&
                           ((int64_t)p.Height * p.Width) % 16 == 0 &&
                           ((uintptr_t)x.DevicePointer() + (uintptr_t)p.OffsetX) % 16 == 0;
    GpuBuffer columns;
    int64_t columnBase = 0;
    if (scratch) {
        if (!scratch->Valid()) throw GpuKernelShapeException(kConv, "scratch", "buffer is null");
        if (scratch->Type() != x.Type()) throw GpuKernelShapeException(kConv, "scratch", "the scratch has a different type than x");
        if (scratchOffset < 0 || (scratchOffset & 3) != 0)
            throw GpuKernelShapeException(kConv, "scratchOffset", "offset " + std::to_string(scratchOffset) + " must be a non-negative multiple of 4");
        if ((int64_t)scratchOffset + perImage > scratch->Length())
            throw GpuKernelShapeException(kConv, "scratch", "bytes " + std::to_string(scratchOffset) + ".." + std::to_string(scratchOffset + perImage) +
                                                                " (one image's columns) reach past the buffer of " + std::to_string(scratch->Length()));
        columns = *scratch;
        columnBase = scratchOffset;
    } else if (!depthwise && !pointwise) {
        const int64_t ownScratchBytes = int64_t(64) << 20;   // ConvIntegerKernels.cs:33
        const int64_t imagesPerChunk = std::clamp<int64_t>(ownScratchBytes / perImage, 1, p.Batch);
        columns = Own(x.Type(), imagesPerChunk * perImage);
    }
    og_conv_params c{};
    c.Batch = (uint32_t)p.Batch;
    c.InChannels = (uint32_t)p.InChannels;
    c.Height = (uint32_t)p.Height;
    c.Width = (uint32_t)p.Width;
    c.OutChannels = (uint32_t)p.OutChannels;
    c.KernelHeight = (uint32_t)p.KernelHeight;
    c.KernelWidth = (uint32_t)p.KernelWidth;
    c.StrideHeight = (uint32_t)p.StrideHeight;
    c.StrideWidth = (uint32_t)p.StrideWidth;
    c.DilationHeight = (uint32_t)p.DilationHeight;
    c.DilationWidth = (uint32_t)p.DilationWidth;
    c.PadTop = (uint32_t)p.PadTop;
    c.PadLeft = (uint32_t)p.PadLeft;
    c.PadBottom = (uint32_t)p.PadBottom;
    c.PadRight = (uint32_t)p.PadRight;
    c.Groups = (uint32_t)p.Groups;
    c.OffsetX = (uint32_t)p.OffsetX;
    c.OffsetW = (uint32_t)p.OffsetW;
    c.OffsetY = (uint32_t)p.OffsetY;
    c.Flags = (x.Type() == ElementType::Int8 ? OG_CONV_X_INT8 : 0u) | (w.Type() == ElementType::Int8 ? OG_CONV_W_INT8 : 0u) |
              (xZeroPoint ? OG_CONV_XZ : 0u) | (wZeroPoint ? OG_CONV_WZ : 0u) |
              (wZeroPoint && wZeroPoint->IsVector ? OG_CONV_WZ_PER_CHANNEL : 0u) | (DirectDepthwise ? 0u : OG_CONV_NO_DEPTHWISE);
    c.OffXZero = xZeroPoint ? (uint32_t)xZeroPoint->Offset : 0u;
    c.OffWZero = wZeroPoint ? (uint32_t)wZeroPoint->Offset : 0u;
    c.GemmFlags = OptionFlags(options_);
    GpuBuffer X = x, W = w, Y = y, XZ = xZeroPoint ? xZeroPoint->Buffer : GpuBuffer(),
              WZ = wZeroPoint ? wZeroPoint->Buffer : GpuBuffer(), S = columns;
    const uint64_t off = (uint64_t)columnBase;
    blocks_.Note(1, {&X, &W, &Y, &XZ, &WZ, &S});
    encoder.Record(
        [c, X, W, Y, XZ, WZ, S, off](og_ctx *ctx) {
            ThrowIfFailed(ctx, og_conv_integer(ctx, &c, bind(X), bind(W), bind(Y), bind(XZ), bind(WZ), bind(S), off), kConv);
        },
        keep_of({&X, &W, &Y, &XZ, &WZ, &S}));
}

void ConvIntegerKernels::Dispose()
{
    gemm_.Dispose();
    own_u8_.Dispose();
    own_i8_.Dispose();
    for (auto &b : retired_) b.Dispose();
    retired_.clear();
}

}  // namespace onegpu
