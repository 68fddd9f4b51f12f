// pybind11 module `_tbn`: the Python face of the tbn host runtime, in the
// shape of the reference's binding (tbn-runtime/python/bindings.cpp:53-168:
// Model.run / run_quantized / input_names / output_names / input_shape) plus
// what a graph-building, device-resident runtime needs: Tensor, ModelGraph,
// TBNModel, Session, InferenceSession and the operator entry points.
//
// numpy arrays cross as host tensors (copied); Tensor.wrap() views existing
// device memory (for example a torch tensor's data_ptr()) without a copy.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <string>
#include <vector>

#include "tbn/gemm_engine.hpp"
#include "tbn/tbn.hpp"

namespace py = pybind11;
using namespace tbn;

namespace {

DataType parse_dtype(const std::string& s) {
    static const std::pair<const char*, DataType> table[] = {
        {"float32", DataType::FLOAT32}, {"binary", DataType::BINARY}, {"ternary", DataType::TERNARY},
        {"int8", DataType::INT8},       {"uint8", DataType::UINT8},   {"int32", DataType::INT32},
        {"int64", DataType::INT64},     {"bool", DataType::BOOL}};
    for (auto& e : table)
        if (s == e.first) return e.second;
    throw InvalidArgumentError("unknown dtype '" + s + "'");
}

std::string dtype_name(DataType d) {
    switch (d) {
        case DataType::FLOAT32: return "float32";
        case DataType::BINARY: return "binary";
        case DataType::TERNARY: return "ternary";
        case DataType::INT8: return "int8";
        case DataType::UINT8: return "uint8";
        case DataType::INT32: return "int32";
        case DataType::INT64: return "int64";
        case DataType::BOOL: return "bool";
        case DataType::FLOAT16: return "float16";
        case DataType::BFLOAT16: return "bfloat16";
        case DataType::INT16: return "int16";
        case DataType::UINT16: return "uint16";
        case DataType::UINT32: return "uint32";
        case DataType::UINT64: return "uint64";
        default: return "other";
    }
}

DeviceType parse_device(const std::string& s) {
    if (s == "cpu") return DeviceType::CPU;
    if (s == "hip" || s == "cuda" || s == "gpu") return DeviceType::HIP;
    throw InvalidArgumentError("unknown device '" + s + "'");
}

// numpy element type expected for each tensor dtype.
py::dtype np_dtype(DataType d) {
    switch (d) {
        case DataType::FLOAT32: return py::dtype::of<float>();
        case DataType::BINARY: case DataType::UINT8: case DataType::BOOL: return py::dtype::of<uint8_t>();
        case DataType::TERNARY: case DataType::INT8: return py::dtype::of<int8_t>();
        case DataType::INT32: return py::dtype::of<int32_t>();
        case DataType::INT64: return py::dtype::of<int64_t>();
        case DataType::UINT16: case DataType::BFLOAT16: return py::dtype::of<uint16_t>();  // bf16 as its bits
        case DataType::INT16: return py::dtype::of<int16_t>();
        case DataType::FLOAT16: return py::dtype("float16");
        case DataType::UINT32: return py::dtype::of<uint32_t>();
        case DataType::UINT64: return py::dtype::of<uint64_t>();
        default: throw InvalidArgumentError("dtype has no numpy equivalent");
    }
}

DataType default_dtype(const py::array& a) {
    if (a.dtype().is(py::dtype::of<float>())) return DataType::FLOAT32;
    if (a.dtype().is(py::dtype::of<uint8_t>())) return DataType::UINT8;
    if (a.dtype().is(py::dtype::of<int8_t>())) return DataType::INT8;
    if (a.dtype().is(py::dtype::of<int32_t>())) return DataType::INT32;
    if (a.dtype().is(py::dtype::of<int64_t>())) return DataType::INT64;
    throw InvalidArgumentError("unsupported numpy dtype");
}

Tensor from_numpy(const py::array& arr, const std::string& dtype, const std::string& device) {
    const DataType dt = dtype.empty() ? default_dtype(arr) : parse_dtype(dtype);
    py::array a = py::array::ensure(arr, py::array::c_style | py::array::forcecast);
    if (!a.dtype().is(np_dtype(dt))) a = a.attr("astype")(np_dtype(dt));
    a = py::array::ensure(a, py::array::c_style);
    Shape shape;
    for (py::ssize_t i = 0; i < a.ndim(); ++i) shape.dims.push_back(a.shape(i));
    return Tensor(shape, dt, a.data(), parse_device(device));
}

py::array to_numpy(const Tensor& t) {
    std::vector<py::ssize_t> shape(t.shape().dims.begin(), t.shape().dims.end());
    py::array out(np_dtype(t.dtype()), shape);
    const Tensor host = t.on_device() ? t.to_device(DeviceType::CPU) : t;
    if (host.data_size()) std::memcpy(out.mutable_data(), host.data(), host.data_size());
    return out;
}

// Accepts a Tensor or anything numpy can read.
Tensor as_tensor(const py::object& o) {
    if (py::isinstance<Tensor>(o)) return o.cast<Tensor>();
    return from_numpy(py::array::ensure(o), "", "cpu");
}

const Tensor* opt_tensor(const py::object& o, Tensor& holder) {
    if (o.is_none()) return nullptr;
    holder = as_tensor(o);
    return &holder;
}

AttributeValue to_attr(const py::handle& v) {
    if (py::isinstance<py::bool_>(v)) return AttributeValue(static_cast<int64_t>(v.cast<bool>()));
    if (py::isinstance<py::int_>(v)) return AttributeValue(v.cast<int64_t>());
    if (py::isinstance<py::float_>(v)) return AttributeValue(v.cast<float>());
    if (py::isinstance<py::str>(v)) return AttributeValue(v.cast<std::string>());
    if (py::isinstance<Tensor>(v)) return AttributeValue(v.cast<Tensor>());
    if (py::isinstance<py::list>(v) || py::isinstance<py::tuple>(v)) {
        py::sequence seq = py::reinterpret_borrow<py::sequence>(v);
        if (seq.size() == 0) return AttributeValue(std::vector<int64_t>{});
        if (py::isinstance<py::str>(seq[0])) return AttributeValue(seq.cast<std::vector<std::string>>());
        if (py::isinstance<py::float_>(seq[0])) return AttributeValue(seq.cast<std::vector<float>>());
        return AttributeValue(seq.cast<std::vector<int64_t>>());
    }
    throw InvalidArgumentError("unsupported attribute value");
}

py::object from_attr(const AttributeValue& a) {
    if (a.is_int()) return py::int_(a.as_int());
    if (a.is_float()) return py::float_(a.as_float());
    if (a.is_string()) return py::str(a.as_string());
    if (a.is_tensor()) return to_numpy(a.as_tensor());
    if (a.is_ints()) return py::cast(a.as_ints());
    if (a.is_floats()) return py::cast(a.as_floats());
    return py::cast(a.as_strings());
}

Conv2DParams conv_params(const Tensor& w, std::vector<int64_t> stride, std::vector<int64_t> pad,
                         std::vector<int64_t> dilation, int64_t groups) {
    Conv2DParams p;
    p.kernel_h = w.shape().rank() == 4 ? w.shape().dims[2] : 3;
    p.kernel_w = w.shape().rank() == 4 ? w.shape().dims[3] : 3;
    TBN_CHECK(stride.size() == 2 && pad.size() == 2 && dilation.size() == 2, InvalidArgumentError,
              "stride, pad and dilation take two values");
    p.stride_h = stride[0]; p.stride_w = stride[1];
    p.pad_h = pad[0]; p.pad_w = pad[1];
    p.dilation_h = dilation[0]; p.dilation_w = dilation[1];
    p.groups = groups;
    return p;
}

QuantArithmetic parse_arithmetic(const std::string& a) {
    if (a == "f32") return QuantArithmetic::F32;
    if (a == "tbn") return QuantArithmetic::TBN;
    throw InvalidArgumentError("arithmetic must be 'f32' or 'tbn', got '" + a + "'");
}

const char* arithmetic_name(QuantArithmetic a) { return a == QuantArithmetic::TBN ? "tbn" : "f32"; }

// The reference's PyModel (bindings.cpp:53-110): an ONNX file (or a graph)
// with one Session reused by every run().  `arithmetic` picks the quantized
// layers' arithmetic: "f32" (float x binary) or "tbn" (the reference's own
// ternarized integer product, bit for bit).
class PyModel {
public:
    PyModel(TBNModel model, uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk, uint32_t nmk,
            const std::string& arithmetic = "f32")
        : model_(std::move(model)) {
        TilingParams t{mblk, nblk, kblk, mmk, nmk};
        session_ = std::make_unique<TBNModel::Session>(model_.create_session(t));
        session_->set_quant_arithmetic(parse_arithmetic(arithmetic));
    }
    py::array run(const py::object& input, bool use_quantization) {
        const auto& ins = model_.graph().inputs;
        const auto& outs = model_.graph().outputs;
        if (ins.empty()) throw std::runtime_error("Model has no inputs");
        if (outs.empty()) throw std::runtime_error("Model has no outputs");
        session_->set_quantization(use_quantization);
        session_->set_input(ins[0], as_tensor(input));
        session_->run();
        return to_numpy(session_->get_output(outs[0]));
    }
    std::vector<std::string> input_names() const { return model_.graph().inputs; }
    std::vector<std::string> output_names() const { return model_.graph().outputs; }
    Shape input_shape(const std::string& name) const {
        auto it = model_.graph().value_info.find(name);
        if (it == model_.graph().value_info.end()) throw std::runtime_error("Input not found: " + name);
        return it->second;
    }
    const TBNModel& model() const { return model_; }
    TBNModel::Session& session() { return *session_; }

private:
    TBNModel model_;
    std::unique_ptr<TBNModel::Session> session_;
};

}  // namespace

PYBIND11_MODULE(_tbn, m) {
    m.doc() = "tbn runtime on the MI355X: device-resident Session and operators over libtbn_hip";

    static py::exception<TBNError> tbn_error(m, "TBNError", PyExc_RuntimeError);
    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const TBNError& e) {
            py::object type = py::reinterpret_borrow<py::object>(tbn_error.ptr());
            py::object inst = type(py::str(e.what()));
            inst.attr("code") = static_cast<int>(e.code());
            PyErr_SetObject(type.ptr(), inst.ptr());
        }
    });

    m.def("get_version", &get_version);
    m.def("set_current_stream", [](uintptr_t s) { device::set_current_stream(reinterpret_cast<void*>(s)); },
          py::arg("stream"));
    m.def("current_stream", []() { return reinterpret_cast<uintptr_t>(device::current_stream()); });
    m.def("synchronize", &device::synchronize);
    m.def("empty_cache", &device::empty_cache);
    m.def("allocated_bytes", &device::allocated_bytes);
    m.def("cached_bytes", &device::cached_bytes);

    py::class_<Shape>(m, "Shape")
        .def(py::init<>())
        .def(py::init<std::vector<int64_t>>())
        .def_readwrite("dims", &Shape::dims)
        .def("__repr__", [](const Shape& s) { return "Shape(" + shape_to_string(s) + ")"; });

    py::class_<Tensor>(m, "Tensor")
        .def(py::init([](const py::array& a, const std::string& dtype, const std::string& device) {
                 return from_numpy(a, dtype, device);
             }),
             py::arg("array"), py::arg("dtype") = "", py::arg("device") = "cpu")
        .def_static("wrap",
                    [](uintptr_t ptr, std::vector<int64_t> shape, const std::string& dtype, const std::string& device) {
                        return Tensor::wrap(Shape(shape), parse_dtype(dtype), reinterpret_cast<void*>(ptr),
                                            parse_device(device));
                    },
                    py::arg("ptr"), py::arg("shape"), py::arg("dtype") = "float32", py::arg("device") = "hip")
        .def_static("empty",
                    [](std::vector<int64_t> shape, const std::string& dtype, const std::string& device) {
                        return Tensor::empty(Shape(shape), parse_dtype(dtype), parse_device(device));
                    },
                    py::arg("shape"), py::arg("dtype") = "float32", py::arg("device") = "hip")
        .def_property_readonly("shape", [](const Tensor& t) { return t.shape().dims; })
        .def_property_readonly("dtype", [](const Tensor& t) { return dtype_name(t.dtype()); })
        .def_property_readonly("device", [](const Tensor& t) { return t.on_device() ? "hip" : "cpu"; })
        .def("data_ptr", [](const Tensor& t) { return reinterpret_cast<uintptr_t>(t.data()); })
        .def("numpy", &to_numpy)
        .def("to", [](const Tensor& t, const std::string& d) { return t.to_device(parse_device(d)); })
        .def("copy", &Tensor::copy)
        .def("reshaped", [](const Tensor& t, std::vector<int64_t> s) { return t.reshaped(Shape(s)); })
        .def("num_elements", &Tensor::num_elements);

    py::class_<PackedWeights>(m, "PackedWeights")
        .def_readonly("K", &PackedWeights::K)
        .def_readonly("N", &PackedWeights::N)
        .def_readonly("K_pad", &PackedWeights::K_pad)
        .def_readonly("N_pad", &PackedWeights::N_pad)
        .def_property_readonly("ternary", [](const PackedWeights& p) { return p.kind == PackedWeights::Kind::Ternary; })
        .def_readonly("bits", &PackedWeights::bits);

    // ---- operators ----
    m.def("quantize_to_binary", [](const py::object& w, float thr) { return quantize_to_binary(as_tensor(w), thr); },
          py::arg("weights"), py::arg("threshold") = 0.0f);
    m.def("quantize_to_ternary",
          [](const py::object& w, float lo, float hi) { return quantize_to_ternary(as_tensor(w), lo, hi); },
          py::arg("weights"), py::arg("threshold_low") = -0.1f, py::arg("threshold_high") = 0.1f);
    m.def("pack_binary_weights",
          [](const py::object& w, bool nk, bool ge_zero) { return pack_binary_weights(as_tensor(w), nk, ge_zero); },
          py::arg("weights"), py::arg("nk_layout") = false, py::arg("ge_zero") = false);
    m.def("pack_ternary_weights", [](const py::object& w, bool nk) { return pack_ternary_weights(as_tensor(w), nk); },
          py::arg("weights"), py::arg("nk_layout") = false);
    m.def("qlinear_matmul_binary",
          [](const py::object& a, const py::object& b, float s) {
              return qlinear_matmul_binary(as_tensor(a), as_tensor(b), s);
          },
          py::arg("a"), py::arg("b_binary"), py::arg("b_scale") = 1.0f);
    m.def("qlinear_matmul_binary_float",
          [](const py::object& a, const py::object& b, float s) {
              return qlinear_matmul_binary_float(as_tensor(a), as_tensor(b), s);
          },
          py::arg("a"), py::arg("b_binary_float"), py::arg("b_scale") = 1.0f);
    m.def("qlinear_matmul_binary_tbn",
          [](const py::object& a, const py::object& b, float s, float lo, float hi) {
              return qlinear_matmul_binary_tbn(as_tensor(a), as_tensor(b), s, TilingParams{}, lo, hi);
          },
          py::arg("a"), py::arg("b_binary"), py::arg("b_scale") = 1.0f, py::arg("threshold_low") = -0.1f,
          py::arg("threshold_high") = 0.1f);
    m.def("qlinear_matmul_packed_tbn",
          [](const py::object& a, const PackedWeights& w, float s, float lo, float hi) {
              return qlinear_matmul_packed_tbn(as_tensor(a), w, s, lo, hi);
          },
          py::arg("a"), py::arg("weights"), py::arg("scale") = 1.0f, py::arg("threshold_low") = -0.1f,
          py::arg("threshold_high") = 0.1f);
    m.def("qlinear_matmul_ternary",
          [](const py::object& a, const py::object& b, float s) {
              return qlinear_matmul_ternary(as_tensor(a), as_tensor(b), s);
          },
          py::arg("a"), py::arg("b_ternary"), py::arg("b_scale") = 1.0f);
    m.def("qlinear_matmul_packed",
          [](const py::object& a, const PackedWeights& w, float s, const py::object& cs, const py::object& bias,
             bool relu) {
              Tensor hs, hb;
              return qlinear_matmul_packed(as_tensor(a), w, s, opt_tensor(cs, hs), opt_tensor(bias, hb), relu);
          },
          py::arg("a"), py::arg("weights"), py::arg("scale") = 1.0f, py::arg("channel_scales") = py::none(),
          py::arg("bias") = py::none(), py::arg("relu") = false);
    m.def("gemm",
          [](const py::object& A, const py::object& B, const py::object& C, float alpha, float beta, bool ta,
             bool tb) {
              Tensor hc;
              return gemm(as_tensor(A), as_tensor(B), opt_tensor(C, hc), alpha, beta, ta, tb);
          },
          py::arg("A"), py::arg("B"), py::arg("C") = py::none(), py::arg("alpha") = 1.0f, py::arg("beta") = 0.0f,
          py::arg("transA") = false, py::arg("transB") = false);

    // ---- the GeMM engine API (GeMM/05-final/GeMM.hpp:16-239) ----
    py::class_<TilingParams>(m, "TilingParams")
        .def(py::init([](uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk, uint32_t nmk) {
                 return TilingParams{mblk, nblk, kblk, mmk, nmk};
             }),
             py::arg("mblk") = 64, py::arg("nblk") = 64, py::arg("kblk") = 128, py::arg("mmk") = 32,
             py::arg("nmk") = 32)
        .def_readwrite("mblk", &TilingParams::mblk)
        .def_readwrite("nblk", &TilingParams::nblk)
        .def_readwrite("kblk", &TilingParams::kblk)
        .def_readwrite("mmk", &TilingParams::mmk)
        .def_readwrite("nmk", &TilingParams::nmk)
        .def("validate", &TilingParams::validate, py::arg("m"), py::arg("n"), py::arg("k"))
        .def_static("default_128x128", &TilingParams::default_128x128);
    auto bytes_of = [](std::span<const std::uint8_t> s) {
        py::array_t<uint8_t> out(static_cast<py::ssize_t>(s.size()));
        if (!s.empty()) std::memcpy(out.mutable_data(), s.data(), s.size());
        return out;
    };
    auto int8_span = [](const py::array_t<int8_t, py::array::c_style | py::array::forcecast>& a) {
        return std::span<const std::int8_t>(a.data(), static_cast<size_t>(a.size()));
    };
    py::class_<TernaryMatrix>(m, "TernaryMatrix")
        .def(py::init<>())
        .def_static("pack",
                    [int8_span](const py::array_t<int8_t, py::array::c_style | py::array::forcecast>& a,
                                uint32_t rows, uint32_t cols) { return TernaryMatrix::pack(int8_span(a), rows, cols); },
                    py::arg("data"), py::arg("rows"), py::arg("cols"))
        .def_static("pack_from_float",
                    [](const py::array_t<float, py::array::c_style | py::array::forcecast>& a, uint32_t rows,
                       uint32_t cols, float lo, float hi) {
                        if (static_cast<size_t>(a.size()) != static_cast<size_t>(rows) * cols)
                            throw std::invalid_argument("TernaryMatrix: data size doesn't match dimensions");
                        return TernaryMatrix::pack_from_float(a.data(), rows, cols, lo, hi);
                    },
                    py::arg("data"), py::arg("rows"), py::arg("cols"), py::arg("threshold_low") = -0.1f,
                    py::arg("threshold_high") = 0.1f)
        .def_property_readonly("rows", &TernaryMatrix::rows)
        .def_property_readonly("cols", &TernaryMatrix::cols)
        .def("empty", &TernaryMatrix::empty)
        .def_property_readonly("positive", [bytes_of](const TernaryMatrix& t) { return bytes_of(t.view().positive); })
        .def_property_readonly("negative", [bytes_of](const TernaryMatrix& t) { return bytes_of(t.view().negative); });
    py::class_<BinaryMatrix>(m, "BinaryMatrix")
        .def(py::init<>())
        .def_static("pack",
                    [int8_span](const py::array_t<int8_t, py::array::c_style | py::array::forcecast>& a,
                                uint32_t rows, uint32_t cols) { return BinaryMatrix::pack(int8_span(a), rows, cols); },
                    py::arg("data"), py::arg("rows"), py::arg("cols"))
        .def_property_readonly("rows", &BinaryMatrix::rows)
        .def_property_readonly("cols", &BinaryMatrix::cols)
        .def("empty", &BinaryMatrix::empty)
        .def_property_readonly("bits", [bytes_of](const BinaryMatrix& b) { return bytes_of(b.view().bits); });
    py::class_<GemmEngine>(m, "GemmEngine")
        .def(py::init<>())
        .def("compute",
             [](GemmEngine& e, const TernaryMatrix& A, const BinaryMatrix& B, const py::object& params) {
                 const TilingParams p =
                     params.is_none() ? TilingParams::default_128x128() : params.cast<TilingParams>();
                 const Int32Matrix C = e.compute(A.view(), B.view(), p);
                 py::array_t<int32_t> out({static_cast<py::ssize_t>(C.rows()), static_cast<py::ssize_t>(C.cols())});
                 if (C.size()) std::memcpy(out.mutable_data(), C.data().data(), C.size() * sizeof(int32_t));
                 return out;
             },
             py::arg("A"), py::arg("B"), py::arg("params") = py::none())
        .def("last_flops", &GemmEngine::last_flops);
    py::class_<PackedBinaryWeights>(m, "PackedBinaryWeights")
        .def_static("from_int8",
                    [int8_span](const py::array_t<int8_t, py::array::c_style | py::array::forcecast>& w,
                                uint32_t rows, uint32_t cols, const TilingParams& t) {
                        return PackedBinaryWeights::from_int8(int8_span(w), rows, cols, t);
                    },
                    py::arg("weights"), py::arg("rows"), py::arg("cols"),
                    py::arg("tiling") = TilingParams::default_128x128())
        .def("valid", &PackedBinaryWeights::valid)
        .def_readonly("b_packed", &PackedBinaryWeights::b_packed)
        .def_readonly("tiling", &PackedBinaryWeights::tiling)
        .def_readonly("original_m", &PackedBinaryWeights::original_m)
        .def_readonly("original_n", &PackedBinaryWeights::original_n)
        .def_readonly("original_k", &PackedBinaryWeights::original_k);
    m.def("qlinear_matmul_binary_blocked_packed",
          [](const py::object& a, const BinaryMatrix& b, uint32_t n_orig, float scale, const TilingParams& p,
             float lo, float hi) { return qlinear_matmul_binary_blocked_packed(as_tensor(a), b, n_orig, scale, p, lo, hi); },
          py::arg("a"), py::arg("b_packed"), py::arg("n_orig"), py::arg("scale") = 1.0f,
          py::arg("params") = TilingParams::default_128x128(), py::arg("threshold_low") = -0.1f,
          py::arg("threshold_high") = 0.1f);
    m.def("qlinear_matmul_binary_blocked_prepacked", &qlinear_matmul_binary_blocked_prepacked, py::arg("a_packed"),
          py::arg("b_packed"), py::arg("m_orig"), py::arg("n_orig"), py::arg("scale") = 1.0f,
          py::arg("params") = TilingParams::default_128x128());

    auto conv_def = [&m](const char* name, Tensor (*fn)(const Tensor&, const Tensor&, const Tensor*,
                                                          const Conv2DParams&)) {
        m.def(name,
              [fn](const py::object& x, const py::object& w, const py::object& bias, std::vector<int64_t> stride,
                   std::vector<int64_t> pad, std::vector<int64_t> dilation, int64_t groups) {
                  Tensor hb;
                  Tensor wt = as_tensor(w);
                  return fn(as_tensor(x), wt, opt_tensor(bias, hb), conv_params(wt, stride, pad, dilation, groups));
              },
              py::arg("input"), py::arg("weights"), py::arg("bias") = py::none(),
              py::arg("stride") = std::vector<int64_t>{1, 1}, py::arg("pad") = std::vector<int64_t>{0, 0},
              py::arg("dilation") = std::vector<int64_t>{1, 1}, py::arg("groups") = 1);
    };
    conv_def("conv2d", &conv2d);
    conv_def("conv2d_binary", &conv2d_binary);
    conv_def("conv2d_ternary", &conv2d_ternary);
    conv_def("depthwise_conv2d", &depthwise_conv2d);
    m.def("conv2d_grouped",
          [](const py::object& x, const py::object& w, const py::object& bias, int64_t groups,
             std::vector<int64_t> stride, std::vector<int64_t> pad, std::vector<int64_t> dilation) {
              Tensor hb;
              Tensor wt = as_tensor(w);
              return conv2d_grouped(as_tensor(x), wt, opt_tensor(bias, hb), groups,
                                    conv_params(wt, stride, pad, dilation, groups));
          },
          py::arg("input"), py::arg("weights"), py::arg("bias") = py::none(), py::arg("groups") = 1,
          py::arg("stride") = std::vector<int64_t>{1, 1}, py::arg("pad") = std::vector<int64_t>{0, 0},
          py::arg("dilation") = std::vector<int64_t>{1, 1});
    m.def("batch_norm",
          [](const py::object& x, const py::object& scale, const py::object& B, const py::object& mean,
             const py::object& var, float eps) {
              return batch_norm(as_tensor(x), as_tensor(scale), as_tensor(B), as_tensor(mean), as_tensor(var), eps);
          },
          py::arg("input"), py::arg("scale"), py::arg("B"), py::arg("mean"), py::arg("var"),
          py::arg("epsilon") = 1e-5f);
    m.def("conv2d_binary_with_scales",
          [](const py::object& x, const py::object& w, const py::object& bias, std::vector<float> scales,
             std::vector<int64_t> stride, std::vector<int64_t> pad, std::vector<int64_t> dilation) {
              Tensor hb;
              Tensor wt = as_tensor(w);
              return conv2d_binary_with_scales(as_tensor(x), wt, opt_tensor(bias, hb),
                                               conv_params(wt, stride, pad, dilation, 1), scales);
          },
          py::arg("input"), py::arg("weights"), py::arg("bias"), py::arg("channel_scales"),
          py::arg("stride") = std::vector<int64_t>{1, 1}, py::arg("pad") = std::vector<int64_t>{0, 0},
          py::arg("dilation") = std::vector<int64_t>{1, 1});
    m.def("maxpool2d",
          [](const py::object& x, std::vector<int64_t> kernel, std::vector<int64_t> stride, std::vector<int64_t> pad,
             bool ceil_mode) {
              TBN_CHECK(kernel.size() == 2 && stride.size() == 2 && pad.size() == 2, InvalidArgumentError,
                        "kernel, stride and pad take two values");
              Pool2DParams p(kernel[0], kernel[1], stride[0], stride[1], pad[0], pad[1]);
              p.ceil_mode = ceil_mode;
              return maxpool2d(as_tensor(x), p);
          },
          py::arg("input"), py::arg("kernel") = std::vector<int64_t>{2, 2},
          py::arg("stride") = std::vector<int64_t>{2, 2}, py::arg("pad") = std::vector<int64_t>{0, 0},
          py::arg("ceil_mode") = false);
    m.def("avgpool2d",
          [](const py::object& x, std::vector<int64_t> kernel, std::vector<int64_t> stride, std::vector<int64_t> pad,
             bool ceil_mode, bool count_include_pad) {
              TBN_CHECK(kernel.size() == 2 && stride.size() == 2 && pad.size() == 2, InvalidArgumentError,
                        "kernel, stride and pad take two values");
              Pool2DParams p(kernel[0], kernel[1], stride[0], stride[1], pad[0], pad[1]);
              p.ceil_mode = ceil_mode;
              p.count_include_pad = count_include_pad;
              return avgpool2d(as_tensor(x), p);
          },
          py::arg("input"), py::arg("kernel") = std::vector<int64_t>{2, 2},
          py::arg("stride") = std::vector<int64_t>{2, 2}, py::arg("pad") = std::vector<int64_t>{0, 0},
          py::arg("ceil_mode") = false, py::arg("count_include_pad") = false);
    m.def("global_maxpool2d", [](const py::object& x) { return global_maxpool2d(as_tensor(x)); });
    m.def("global_avgpool2d", [](const py::object& x) { return global_avgpool2d(as_tensor(x)); });
    m.def("relu", [](const py::object& x) { return relu(as_tensor(x)); });
    m.def("add", [](const py::object& a, const py::object& b) { return add(as_tensor(a), as_tensor(b)); });

    // ---- graph ----
    py::class_<ModelGraph, std::shared_ptr<ModelGraph>>(m, "ModelGraph")
        .def(py::init<>())
        .def("add_input",
             [](ModelGraph& g, const std::string& n, std::vector<int64_t> s) {
                 g.inputs.push_back(n);
                 g.value_info[n] = Shape(s);
             })
        .def("add_output",
             [](ModelGraph& g, const std::string& n, std::vector<int64_t> s) {
                 g.outputs.push_back(n);
                 g.value_info[n] = Shape(s);
             })
        .def("set_value_info", [](ModelGraph& g, const std::string& n, std::vector<int64_t> s) { g.value_info[n] = Shape(s); })
        .def("add_initializer",
             [](ModelGraph& g, const std::string& n, const py::object& t, const std::string& dtype) {
                 g.initializers[n] = py::isinstance<Tensor>(t) ? t.cast<Tensor>()
                                                               : from_numpy(py::array::ensure(t), dtype, "cpu");
             },
             py::arg("name"), py::arg("tensor"), py::arg("dtype") = "")
        .def("add_node",
             [](ModelGraph& g, const std::string& name, const std::string& op, std::vector<std::string> ins,
                std::vector<std::string> outs, const py::dict& attrs) {
                 ModelNode node;
                 node.name = name;
                 node.op_type = op;
                 node.inputs = std::move(ins);
                 node.outputs = std::move(outs);
                 for (auto kv : attrs) node.attributes[kv.first.cast<std::string>()] = to_attr(kv.second);
                 g.nodes.push_back(std::move(node));
             },
             py::arg("name"), py::arg("op_type"), py::arg("inputs"), py::arg("outputs"), py::arg("attributes") = py::dict())
        .def_property_readonly("inputs", [](const ModelGraph& g) { return g.inputs; })
        .def_property_readonly("outputs", [](const ModelGraph& g) { return g.outputs; })
        .def("num_nodes", [](const ModelGraph& g) { return g.nodes.size(); })
        .def_property_readonly("value_info",
                               [](const ModelGraph& g) {
                                   py::dict d;
                                   for (const auto& [n, s] : g.value_info) d[py::str(n)] = py::cast(s.dims);
                                   return d;
                               })
        .def("initializer_names",
             [](const ModelGraph& g) {
                 std::vector<std::string> v;
                 for (const auto& kv : g.initializers) v.push_back(kv.first);
                 return v;
             })
        .def("initializer", [](const ModelGraph& g, const std::string& n) { return to_numpy(g.initializers.at(n)); })
        .def("initializer_dtype",
             [](const ModelGraph& g, const std::string& n) { return dtype_name(g.initializers.at(n).dtype()); })
        .def("nodes", [](const ModelGraph& g) {
            py::list out;
            for (const auto& nd : g.nodes) {
                py::dict attrs;
                for (const auto& [k, v] : nd.attributes) attrs[py::str(k)] = from_attr(v);
                py::dict d;
                d["name"] = nd.name;
                d["op_type"] = nd.op_type;
                d["inputs"] = nd.inputs;
                d["outputs"] = nd.outputs;
                d["attributes"] = attrs;
                out.append(d);
            }
            return out;
        });

    py::class_<TBNModel::Session>(m, "Session")
        .def("set_quantization", &TBNModel::Session::set_quantization)
        .def("is_quantization_enabled", &TBNModel::Session::is_quantization_enabled)
        .def("set_quant_arithmetic",
             [](TBNModel::Session& s, const std::string& a) { s.set_quant_arithmetic(parse_arithmetic(a)); },
             py::arg("arithmetic"))
        .def("quant_arithmetic", [](const TBNModel::Session& s) { return arithmetic_name(s.quant_arithmetic()); })
        .def("set_input", [](TBNModel::Session& s, const std::string& n, const py::object& t) { s.set_input(n, as_tensor(t)); })
        .def("run", &TBNModel::Session::run)
        .def("get_output", [](const TBNModel::Session& s, const std::string& n) { return to_numpy(s.get_output(n)); })
        .def("get_output_device", &TBNModel::Session::get_output_device)
        .def("set_graph_replay", &TBNModel::Session::set_graph_replay)
        .def("synchronize", &TBNModel::Session::synchronize)
        .def("planned_launches", &TBNModel::Session::planned_launches)
        .def("device_bytes", &TBNModel::Session::device_bytes);

    py::class_<TBNModel, std::shared_ptr<TBNModel>>(m, "TBNModel")
        .def(py::init<std::shared_ptr<ModelGraph>>())
        .def("validate", &TBNModel::validate)
        .def("inputs", &TBNModel::inputs)
        .def("outputs", &TBNModel::outputs)
        .def("create_session", [](TBNModel& mdl) { return mdl.create_session(); })
        .def("graph", &TBNModel::graph_ptr)
        .def("producer_name", &TBNModel::producer_name)
        .def("producer_version", &TBNModel::producer_version)
        .def("get_input_shape", [](const TBNModel& mdl, const std::string& n) { return mdl.get_input_shape(n).dims; })
        .def("get_output_shape", [](const TBNModel& mdl, const std::string& n) { return mdl.get_output_shape(n).dims; });

    py::class_<InferenceSessionOptions>(m, "InferenceSessionOptions")
        .def(py::init<>())
        .def_readwrite("num_threads", &InferenceSessionOptions::num_threads)
        .def_readwrite("enable_profiling", &InferenceSessionOptions::enable_profiling)
        .def_readwrite("use_quantization", &InferenceSessionOptions::use_quantization);

    py::class_<InferenceSession>(m, "InferenceSession")
        .def(py::init([](std::shared_ptr<TBNModel> mdl, const InferenceSessionOptions& o) {
                 return std::make_unique<InferenceSession>(mdl, o);
             }),
             py::arg("model"), py::arg("options") = InferenceSessionOptions())
        .def("initialize", &InferenceSession::initialize)
        .def("set_input", [](InferenceSession& s, const std::string& n, const py::object& t) { s.set_input(n, as_tensor(t)); })
        .def("run", &InferenceSession::run)
        .def("get_output", [](const InferenceSession& s, const std::string& n) { return to_numpy(s.get_output(n)); })
        .def("get_input_names", &InferenceSession::get_input_names)
        .def("get_output_names", &InferenceSession::get_output_names)
        .def("last_run_us", &InferenceSession::last_run_us);

    py::class_<PyModel>(m, "Model")
        .def(py::init([](const std::string& path, uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk,
                         uint32_t nmk, const std::string& arithmetic) {
                 return new PyModel(load_onnx_model(path), mblk, nblk, kblk, mmk, nmk, arithmetic);
             }),
             py::arg("path"), py::arg("mblk") = 64, py::arg("nblk") = 64, py::arg("kblk") = 128,
             py::arg("mmk") = 32, py::arg("nmk") = 32, py::arg("arithmetic") = "f32",
             "Load an ONNX model; the tiling arguments are accepted for compatibility.")
        .def(py::init([](std::shared_ptr<ModelGraph> g, uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk,
                         uint32_t nmk, const std::string& arithmetic) {
                 return new PyModel(TBNModel(std::move(g)), mblk, nblk, kblk, mmk, nmk, arithmetic);
             }),
             py::arg("graph"), py::arg("mblk") = 64, py::arg("nblk") = 64, py::arg("kblk") = 128,
             py::arg("mmk") = 32, py::arg("nmk") = 32, py::arg("arithmetic") = "f32")
        .def("run", &PyModel::run, py::arg("input"), py::arg("use_quantization") = false)
        .def("run_quantized", [](PyModel& p, const py::object& x) { return p.run(x, true); }, py::arg("input"))
        .def("input_names", &PyModel::input_names)
        .def("output_names", &PyModel::output_names)
        .def("input_shape", &PyModel::input_shape, py::arg("name"))
        .def("producer", [](const PyModel& p) { return py::make_tuple(p.model().producer_name(), p.model().producer_version()); })
        .def("session", &PyModel::session, py::return_value_policy::reference_internal);

    // bindings.cpp:154-167 of the reference: load_model returns a Model.
    m.def("load_model",
          [](const std::string& path, uint32_t mblk, uint32_t nblk, uint32_t kblk, uint32_t mmk, uint32_t nmk,
             const std::string& arithmetic) {
              return new PyModel(load_onnx_model(path), mblk, nblk, kblk, mmk, nmk, arithmetic);
          },
          py::arg("path"), py::arg("mblk") = 64, py::arg("nblk") = 64, py::arg("kblk") = 128, py::arg("mmk") = 32,
          py::arg("nmk") = 32, py::arg("arithmetic") = "f32", py::return_value_policy::take_ownership);

    // The C++ reader itself, for inspecting a model without a Session.
    py::class_<OnnxParser>(m, "OnnxParser")
        .def(py::init<>())
        .def("parse_from_file", &OnnxParser::parse_from_file, py::arg("path"))
        .def("parse_from_buffer",
             [](OnnxParser& p, const py::bytes& b, const std::string& base_dir) {
                 const std::string s = b;
                 p.parse_from_buffer(s.data(), s.size(), base_dir);
             },
             py::arg("data"), py::arg("base_dir") = "")
        .def("get_graph", &OnnxParser::get_graph)
        .def("get_producer_name", &OnnxParser::get_producer_name)
        .def("get_producer_version", &OnnxParser::get_producer_version)
        .def("ir_version", &OnnxParser::ir_version)
        .def("opset_version", &OnnxParser::opset_version, py::arg("domain") = "")
        .def("warnings", &OnnxParser::warnings);
    m.def("load_onnx_model", [](const std::string& path) { return std::make_shared<TBNModel>(load_onnx_model(path)); },
          py::arg("path"));
}
