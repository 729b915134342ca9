// Python binding of the host layer (onegpu.hpp): the same class and member names as the reference's C# API, so a test
// written against Int8Gemm / DynamicQuantizeKernels / DequantizeKernels reads as the reference's tests do. Buffers
// move to and from numpy arrays; exceptions arrive as onegpu_hip.errors classes with the reference's properties.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "onegpu.hpp"

namespace py = pybind11;
using namespace onegpu;

namespace {

ElementType type_of_dtype(const py::dtype &dt)
{
    char k = dt.kind();
    size_t n = dt.itemsize();
    if (k == 'u' && n == 1) return ElementType::UInt8;
    if (k == 'i' && n == 1) return ElementType::Int8;
    if (k == 'i' && n == 4) return ElementType::Int32;
    if (k == 'f' && n == 4) return ElementType::Float32;
    if (k == 'f' && n == 2) return ElementType::Float16;
    if (k == 'u' && n == 4) return ElementType::UInt32;
    if (k == 'u' && n == 2) return ElementType::UInt16;
    if (k == 'i' && n == 2) return ElementType::Int16;
    if (k == 'i' && n == 8) return ElementType::Int64;
    throw std::invalid_argument("unsupported dtype " + std::string(py::str(dt)));
}

py::dtype dtype_of(ElementType t)
{
    switch (t) {
    case ElementType::UInt8: return py::dtype("uint8");
    case ElementType::Int8: return py::dtype("int8");
    case ElementType::Int32: return py::dtype("int32");
    case ElementType::Float32: return py::dtype("float32");
    case ElementType::Float16: return py::dtype("float16");
    case ElementType::UInt32: return py::dtype("uint32");
    case ElementType::UInt16: return py::dtype("uint16");
    case ElementType::Int16: return py::dtype("int16");
    default: return py::dtype("int64");
    }
}

GpuBuffer create_from(GpuDevice &d, py::array arr)
{
    py::array c = py::array::ensure(arr, py::array::c_style);
    ElementType t = type_of_dtype(c.dtype());
    GpuBuffer b = d.CreateBuffer(t, (int)c.size());
    if (c.size()) b.Write(c.data(), (uint64_t)c.nbytes());
    return b;
}

py::array read_all(const GpuBuffer &b)
{
    py::array out = py::module_::import("numpy").attr("empty")(b.Length(), dtype_of(b.Type()));
    if (b.Length()) b.Read(out.mutable_data(), (uint64_t)b.Length() * ElementSize(b.Type()));
    return out;
}

void write_from(const GpuBuffer &b, py::array arr, int offset)
{
    py::array c = py::array::ensure(arr, py::array::c_style);
    b.Write(c.data(), (uint64_t)c.nbytes(), (uint64_t)offset * ElementSize(b.Type()));
}

}  // namespace

PYBIND11_MODULE(_onegpu_host, m)
{
    m.doc() = "MI355X int8 quantized-matmul path: the reference's kernel-family API over libonegpu_hip.so";

    // The exception classes live as long as the interpreter: hold them as released handles, never as static
    // py::objects whose destructors would run after the interpreter is gone.
    py::module_ errors = py::module_::import("onegpu_hip.errors");
    static py::handle ShapeErr = py::object(errors.attr("GpuKernelShapeException")).release();
    static py::handle UnsupErr = py::object(errors.attr("GpuUnsupportedException")).release();
    static py::handle OomErr = py::object(errors.attr("GpuOutOfMemoryException")).release();
    static py::handle LostErr = py::object(errors.attr("GpuDeviceLostException")).release();
    static py::handle CmdErr = py::object(errors.attr("GpuCommandFailedException")).release();
    static py::handle BaseErr = py::object(errors.attr("GpuException")).release();
    static py::handle IndexErr = py::object(errors.attr("GpuKernelIndexException")).release();
    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const GpuKernelShapeException &e) {
            py::object ex = ShapeErr(e.Operation, e.Argument, e.Detail);
            PyErr_SetObject(ShapeErr.ptr(), ex.ptr());
        } catch (const GpuUnsupportedException &e) {
            py::object ex = UnsupErr(std::string(e.what()), e.Capability, e.Expected, e.Actual);
            PyErr_SetObject(UnsupErr.ptr(), ex.ptr());
        } catch (const GpuOutOfMemoryException &e) {
            PyErr_SetString(OomErr.ptr(), e.what());
        } catch (const GpuDeviceLostException &e) {
            PyErr_SetString(LostErr.ptr(), e.what());
        } catch (const GpuKernelIndexException &e) {
            py::object ex = IndexErr(e.Operation, e.Position);
            PyErr_SetObject(IndexErr.ptr(), ex.ptr());
        } catch (const GpuCommandFailedException &e) {
            PyErr_SetString(CmdErr.ptr(), e.what());
        } catch (const GpuException &e) {
            PyErr_SetString(BaseErr.ptr(), e.what());
        }
    });

    py::enum_<ElementType>(m, "ElementType")
        .value("UInt8", ElementType::UInt8)
        .value("Int8", ElementType::Int8)
        .value("Int32", ElementType::Int32)
        .value("Float32", ElementType::Float32)
        .value("Float16", ElementType::Float16)
        .value("UInt32", ElementType::UInt32)
        .value("UInt16", ElementType::UInt16)
        .value("Int16", ElementType::Int16)
        .value("Int64", ElementType::Int64);

    py::class_<GpuComputeCapabilities>(m, "GpuComputeCapabilities")
        .def_readonly("MaxStorageBufferBindingBytes", &GpuComputeCapabilities::MaxStorageBufferBindingBytes)
        .def_readonly("MaxWorkgroupCount", &GpuComputeCapabilities::MaxWorkgroupCount)
        .def_readonly("Int8DotProduct", &GpuComputeCapabilities::Int8DotProduct)
        .def_readonly("ComputeUnits", &GpuComputeCapabilities::ComputeUnits);

    py::class_<GpuBuffer>(m, "GpuBuffer")
        .def_property_readonly("Length", &GpuBuffer::Length)
        .def_property_readonly("Type", &GpuBuffer::Type)
        .def_property_readonly("Size", &GpuBuffer::Size)
        .def_property_readonly("DevicePointer", [](const GpuBuffer &b) { return (uintptr_t)b.DevicePointer(); })
        .def("Read", &read_all, "All elements as a numpy array (waits for the device).")
        .def("Write", &write_from, py::arg("data"), py::arg("offset") = 0)
        .def("Dispose", &GpuBuffer::Dispose)
        .def("__enter__", [](GpuBuffer &b) -> GpuBuffer & { return b; })
        .def("__exit__", [](GpuBuffer &b, py::args) { b.Dispose(); });

    py::class_<GpuCommandEncoder>(m, "GpuCommandEncoder")
        .def_property_readonly("DispatchCount", &GpuCommandEncoder::DispatchCount)
        .def("BeginPassTiming", &GpuCommandEncoder::BeginPassTiming, py::arg("max_passes"))
        .def("EndPassTiming", &GpuCommandEncoder::EndPassTiming)
        // Benchmark utility (no counterpart in the reference's kernel families): records out[i] = fl(a[0] * b[i]) for
        // i < n, the elementwise Mul of the reference's MatMulIntegerToFloat chain, as one dispatch of this encoder.
        .def("RecordScaleProduct", [](GpuCommandEncoder &e, const GpuBuffer &a, const GpuBuffer &b, uint32_t n,
                                      const GpuBuffer &out) {
            og_buffer ba = a.Binding(), bb = b.Binding(), bo = out.Binding();
            e.Record(
                [ba, bb, n, bo](og_ctx *ctx) {
                    if (og_util_scale_product(ctx, ba, bb, n, bo) != OG_OK)
                        throw std::runtime_error(std::string("scale product: ") + og_last_error(ctx));
                },
                {a.impl(), b.impl(), out.impl()});
        }, py::arg("a"), py::arg("b"), py::arg("n"), py::arg("out"));

    py::class_<GpuDevice, std::shared_ptr<GpuDevice>>(m, "GpuDevice")
        .def_static("Create", [](int ordinal, uint64_t max_binding, bool batch) {
                        GpuDeviceOptions o;
                        o.MaxStorageBufferBindingBytes = max_binding;
                        o.BatchDispatches = batch;
                        return GpuDevice::Create(ordinal, o);
                    },
                    py::arg("ordinal") = 0, py::arg("max_binding_bytes") = 0, py::arg("BatchDispatches") = true)
        .def_static("CreateHostOnly", [](uint64_t max_binding) { GpuDeviceOptions o; o.MaxStorageBufferBindingBytes = max_binding; return GpuDevice::CreateHostOnly(o); },
                    py::arg("max_binding_bytes") = 0)
        .def("CreateBuffer", [](GpuDevice &d, py::array data) { return create_from(d, data); }, py::arg("data"),
             "A buffer holding a copy of the numpy array, typed by its dtype.")
        .def("CreateBufferOf", [](GpuDevice &d, ElementType t, int length) { return d.CreateBuffer(t, length); })
        .def("BeginCommands", &GpuDevice::BeginCommands)
        .def("Submit", &GpuDevice::Submit)
        .def("WaitIdle", &GpuDevice::WaitIdle)
        .def("ReadPassTimes", &GpuDevice::ReadPassTimes)
        .def_property_readonly("Capabilities", &GpuDevice::Capabilities)
        .def_property_readonly("AdapterName", &GpuDevice::AdapterName)
        .def_property_readonly("Backend", &GpuDevice::Backend)
        .def_property_readonly("HasGpu", &GpuDevice::HasGpu)
        .def_property_readonly("LastKernel", [](const GpuDevice &d) { return std::string(d.HasGpu() ? og_last_kernel(d.Context()) : ""); })
        .def_property_readonly("Context", [](const GpuDevice &d) { return (uintptr_t)d.Context(); });

    py::class_<Int8GemmOptions>(m, "Int8GemmOptions")
        .def(py::init([](bool allow, int tile, bool fused, bool one_launch) {
                 Int8GemmOptions o;
                 o.AllowPackedDot = allow;
                 o.Tile = tile;
                 o.FusedRequantize = fused;
                 o.FewRowsOneLaunch = one_launch;
                 return o;
             }),
             py::arg("AllowPackedDot") = true, py::arg("Tile") = 0, py::arg("FusedRequantize") = true,
             py::arg("FewRowsOneLaunch") = true)
        .def_readwrite("AllowPackedDot", &Int8GemmOptions::AllowPackedDot)
        .def_readwrite("Tile", &Int8GemmOptions::Tile)
        .def_readwrite("FusedRequantize", &Int8GemmOptions::FusedRequantize)
        .def_readwrite("FewRowsOneLaunch", &Int8GemmOptions::FewRowsOneLaunch);

    py::class_<Int8Operand>(m, "Int8Operand")
        .def(py::init([](GpuBuffer b, int off, bool vec) { return Int8Operand{b, off, vec}; }), py::arg("Buffer"),
             py::arg("Offset") = 0, py::arg("IsVector") = false)
        .def_readwrite("Buffer", &Int8Operand::Buffer)
        .def_readwrite("Offset", &Int8Operand::Offset)
        .def_readwrite("IsVector", &Int8Operand::IsVector);

    py::class_<Int8Ranges>(m, "Int8Ranges")
        .def(py::init([](GpuBuffer b) { return Int8Ranges(std::move(b)); }), py::arg("Buffer"))
        .def_readwrite("Buffer", &Int8Ranges::Buffer)
        .def_property_readonly("Groups", [](const Int8Ranges &r) { return *r.Groups; });
    m.attr("OG_RANGES_MAX") = (int)OG_RANGES_MAX;

    py::class_<Int8Scratch>(m, "Int8Scratch")
        .def(py::init([](GpuBuffer b, int off) { return Int8Scratch{b, off}; }), py::arg("Buffer"), py::arg("Offset") = 0)
        .def_readwrite("Buffer", &Int8Scratch::Buffer)
        .def_readwrite("Offset", &Int8Scratch::Offset);

    py::class_<Int8GemmProblem>(m, "Int8GemmProblem")
        .def(py::init<int, int, int>(), py::arg("m"), py::arg("n"), py::arg("k"))
        .def_readwrite("M", &Int8GemmProblem::M)
        .def_readwrite("N", &Int8GemmProblem::N)
        .def_readwrite("K", &Int8GemmProblem::K)
        .def_readwrite("Batch", &Int8GemmProblem::Batch)
        .def_readwrite("TransposeB", &Int8GemmProblem::TransposeB)
        .def_readwrite("Lda", &Int8GemmProblem::Lda)
        .def_readwrite("Ldb", &Int8GemmProblem::Ldb)
        .def_readwrite("OffsetA", &Int8GemmProblem::OffsetA)
        .def_readwrite("OffsetB", &Int8GemmProblem::OffsetB)
        .def_readwrite("OffsetC", &Int8GemmProblem::OffsetC)
        .def_readwrite("StrideA", &Int8GemmProblem::StrideA)
        .def_readwrite("StrideB", &Int8GemmProblem::StrideB)
        .def_property_readonly("Ops", &Int8GemmProblem::Ops);

    py::class_<Int8Gemm>(m, "Int8Gemm")
        .def(py::init([](std::shared_ptr<GpuDevice> d, std::optional<Int8GemmOptions> o, int maxGroups) {
                 return new Int8Gemm(std::move(d), o.value_or(Int8GemmOptions{}), maxGroups);
             }),
             py::arg("device"), py::arg("options") = py::none(), py::arg("maxCachedBindGroups") = 1024)
        .def("EncodeInt32", &Int8Gemm::EncodeInt32, py::arg("encoder"), py::arg("problem"), py::arg("a"), py::arg("b"),
             py::arg("c"), py::arg("zeroPointA") = py::none(), py::arg("zeroPointB") = py::none(), py::arg("bias") = py::none())
        .def("EncodeFloat", &Int8Gemm::EncodeFloat, py::arg("encoder"), py::arg("problem"), py::arg("a"), py::arg("b"),
             py::arg("c"), py::arg("scale"), py::arg("zeroPointA") = py::none(), py::arg("zeroPointB") = py::none(),
             py::arg("floatBias") = py::none(), py::arg("intBias") = py::none())
        .def("EncodeFloatRanged", &Int8Gemm::EncodeFloatRanged, py::arg("encoder"), py::arg("problem"), py::arg("a"),
             py::arg("b"), py::arg("c"), py::arg("scale"), py::arg("ranges"), py::arg("zeroPointA") = py::none(),
             py::arg("zeroPointB") = py::none(), py::arg("floatBias") = py::none(), py::arg("intBias") = py::none(),
             py::arg("activationScale") = py::none())
        .def("EncodeFloatScaled", &Int8Gemm::EncodeFloatScaled, py::arg("encoder"), py::arg("problem"), py::arg("a"),
             py::arg("b"), py::arg("c"), py::arg("activationScale"), py::arg("weightScale"),
             py::arg("zeroPointA") = py::none(), py::arg("zeroPointB") = py::none(), py::arg("floatBias") = py::none(),
             py::arg("intBias") = py::none())
        .def("EncodeRequantized", &Int8Gemm::EncodeRequantized, py::arg("encoder"), py::arg("problem"), py::arg("a"),
             py::arg("b"), py::arg("y"), py::arg("multiplier"), py::arg("zeroPointY"), py::arg("zeroPointA") = py::none(),
             py::arg("zeroPointB") = py::none(), py::arg("intBias") = py::none(), py::arg("scratch") = py::none())
        .def_static("ScratchElements", &Int8Gemm::ScratchElements)
        .def("ReserveScratch", &Int8Gemm::ReserveScratch)
        .def_property_readonly("Variant", &Int8Gemm::Variant)
        .def_property_readonly("BindGroupsCreated", &Int8Gemm::BindGroupsCreated)
        .def("ReleaseBindings", &Int8Gemm::ReleaseBindings)
        .def("Dispose", &Int8Gemm::Dispose)
        .def("__enter__", [](Int8Gemm &g) -> Int8Gemm & { return g; })
        .def("__exit__", [](Int8Gemm &g, py::args) { g.Dispose(); });

    py::class_<DynamicQuantizeKernels>(m, "DynamicQuantizeKernels")
        .def(py::init<std::shared_ptr<GpuDevice>, int>(), py::arg("device"), py::arg("maxCachedBindGroups") = 1024)
        .def("Encode", &DynamicQuantizeKernels::Encode, py::arg("encoder"), py::arg("x"), py::arg("offsetX"),
             py::arg("count"), py::arg("y"), py::arg("offsetY"), py::arg("scale"), py::arg("offsetScale"),
             py::arg("zeroPoint"), py::arg("offsetZeroPoint"))
        .def("EncodeRanged", &DynamicQuantizeKernels::EncodeRanged, py::arg("encoder"), py::arg("x"),
             py::arg("offsetX"), py::arg("count"), py::arg("y"), py::arg("offsetY"), py::arg("scale"),
             py::arg("offsetScale"), py::arg("zeroPoint"), py::arg("offsetZeroPoint"), py::arg("ranges"))
        .def_property_readonly("BindGroupsCreated", &DynamicQuantizeKernels::BindGroupsCreated)
        .def("ReleaseBindings", &DynamicQuantizeKernels::ReleaseBindings)
        .def("Dispose", &DynamicQuantizeKernels::Dispose)
        .def("__enter__", [](DynamicQuantizeKernels &g) -> DynamicQuantizeKernels & { return g; })
        .def("__exit__", [](DynamicQuantizeKernels &g, py::args) { g.Dispose(); });

    py::class_<ConvProblem>(m, "ConvProblem")
        .def(py::init<>())
        .def(py::init<int, int, int, int, int, int, int>(), py::arg("batch"), py::arg("inChannels"), py::arg("height"),
             py::arg("width"), py::arg("outChannels"), py::arg("kernelHeight"), py::arg("kernelWidth"))
        .def_static("Conv1D", &ConvProblem::Conv1D, py::arg("batch"), py::arg("inChannels"), py::arg("length"),
                    py::arg("outChannels"), py::arg("kernel"), py::arg("stride") = 1, py::arg("dilation") = 1,
                    py::arg("padBegin") = 0, py::arg("padEnd") = 0, py::arg("groups") = 1)
        .def_readwrite("Batch", &ConvProblem::Batch)
        .def_readwrite("InChannels", &ConvProblem::InChannels)
        .def_readwrite("Height", &ConvProblem::Height)
        .def_readwrite("Width", &ConvProblem::Width)
        .def_readwrite("OutChannels", &ConvProblem::OutChannels)
        .def_readwrite("KernelHeight", &ConvProblem::KernelHeight)
        .def_readwrite("KernelWidth", &ConvProblem::KernelWidth)
        .def_readwrite("StrideHeight", &ConvProblem::StrideHeight)
        .def_readwrite("StrideWidth", &ConvProblem::StrideWidth)
        .def_readwrite("DilationHeight", &ConvProblem::DilationHeight)
        .def_readwrite("DilationWidth", &ConvProblem::DilationWidth)
        .def_readwrite("PadTop", &ConvProblem::PadTop)
        .def_readwrite("PadLeft", &ConvProblem::PadLeft)
        .def_readwrite("PadBottom", &ConvProblem::PadBottom)
        .def_readwrite("PadRight", &ConvProblem::PadRight)
        .def_readwrite("Groups", &ConvProblem::Groups)
        .def_readwrite("Activation", &ConvProblem::Activation)
        .def_readwrite("OffsetX", &ConvProblem::OffsetX)
        .def_readwrite("OffsetW", &ConvProblem::OffsetW)
        .def_readwrite("OffsetY", &ConvProblem::OffsetY)
        .def_property_readonly("OutHeight", &ConvProblem::OutHeight)
        .def_property_readonly("OutWidth", &ConvProblem::OutWidth);

    py::class_<ConvIntegerKernels>(m, "ConvIntegerKernels")
        .def(py::init([](std::shared_ptr<GpuDevice> d, std::optional<Int8GemmOptions> o, int maxGroups) {
                 return new ConvIntegerKernels(std::move(d), o.value_or(Int8GemmOptions{}), maxGroups);
             }),
             py::arg("device"), py::arg("options") = py::none(), py::arg("maxCachedBindGroups") = 1024)
        .def_static("ScratchBytesPerImage", &ConvIntegerKernels::ScratchBytesPerImage, py::arg("problem"))
        .def("Encode", &ConvIntegerKernels::Encode, py::arg("encoder"), py::arg("problem"), py::arg("x"), py::arg("w"),
             py::arg("y"), py::arg("xZeroPoint") = py::none(), py::arg("wZeroPoint") = py::none(),
             py::arg("scratch") = py::none(), py::arg("scratchOffset") = 0)
        .def_readwrite("DirectDepthwise", &ConvIntegerKernels::DirectDepthwise)
        .def_property_readonly("Variant", &ConvIntegerKernels::Variant)
        .def_property_readonly("BindGroupsCreated", &ConvIntegerKernels::BindGroupsCreated)
        .def("ReleaseBindings", &ConvIntegerKernels::ReleaseBindings)
        .def("Dispose", &ConvIntegerKernels::Dispose)
        .def("__enter__", [](ConvIntegerKernels &g) -> ConvIntegerKernels & { return g; })
        .def("__exit__", [](ConvIntegerKernels &g, py::args) { g.Dispose(); });

    py::class_<GpuIndexStatus>(m, "GpuIndexStatus")
        .def(py::init<std::shared_ptr<GpuDevice>>(), py::arg("device"))
        .def("Reset", &GpuIndexStatus::Reset)
        .def("ThrowIfFailed", &GpuIndexStatus::ThrowIfFailed)
        .def("Dispose", &GpuIndexStatus::Dispose)
        .def("__enter__", [](GpuIndexStatus &g) -> GpuIndexStatus & { return g; })
        .def("__exit__", [](GpuIndexStatus &g, py::args) { g.Dispose(); });

    py::class_<GatherKernels>(m, "GatherKernels")
        .def(py::init<std::shared_ptr<GpuDevice>, int>(), py::arg("device"), py::arg("maxCachedBindGroups") = 1024)
        .def("EncodeGather", &GatherKernels::EncodeGather, py::arg("encoder"), py::arg("data"), py::arg("offsetData"),
             py::arg("dataShape"), py::arg("axis"), py::arg("indices"), py::arg("offsetIndices"), py::arg("indexCount"),
             py::arg("output"), py::arg("offsetOutput"), py::arg("status") = nullptr)
        .def_property_readonly("BindGroupsCreated", &GatherKernels::BindGroupsCreated)
        .def("ReleaseBindings", &GatherKernels::ReleaseBindings)
        .def("Dispose", &GatherKernels::Dispose)
        .def("__enter__", [](GatherKernels &g) -> GatherKernels & { return g; })
        .def("__exit__", [](GatherKernels &g, py::args) { g.Dispose(); });

    py::class_<DequantizeKernels>(m, "DequantizeKernels")
        .def(py::init<std::shared_ptr<GpuDevice>, int>(), py::arg("device"), py::arg("maxCachedBindGroups") = 1024)
        .def("Encode", &DequantizeKernels::Encode, py::arg("encoder"), py::arg("x"), py::arg("offsetX"), py::arg("shape"),
             py::arg("axis"), py::arg("perAxis"), py::arg("scale"), py::arg("offsetScale"), py::arg("zeroPoint"),
             py::arg("offsetZeroPoint"), py::arg("output"), py::arg("offsetOutput"))
        .def("EncodeQuantize", &DequantizeKernels::EncodeQuantize, py::arg("encoder"), py::arg("x"), py::arg("offsetX"),
             py::arg("shape"), py::arg("axis"), py::arg("perAxis"), py::arg("scale"), py::arg("offsetScale"),
             py::arg("zeroPoint"), py::arg("offsetZeroPoint"), py::arg("output"), py::arg("offsetOutput"))
        .def_property_readonly("BindGroupsCreated", &DequantizeKernels::BindGroupsCreated)
        .def("ReleaseBindings", &DequantizeKernels::ReleaseBindings)
        .def("Dispose", &DequantizeKernels::Dispose)
        .def("__enter__", [](DequantizeKernels &g) -> DequantizeKernels & { return g; })
        .def("__exit__", [](DequantizeKernels &g, py::args) { g.Dispose(); });

    m.def("version", []() { return std::string(og_version()); });
}
