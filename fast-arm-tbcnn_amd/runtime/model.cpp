// TBNModel and the device-resident TBNModel::Session.
//
// The Session compiles the graph once per (quantization flag, input shapes):
//   1. lowering   every node becomes an Op with resolved value ids, output
//                 shapes and, for quantized layers, packed device weights
//                 (computed once and cached by initializer name for the
//                 Session's lifetime);
//   2. fusion     Relu into the preceding Conv/Gemm/Add, a 2x2/2 MaxPool into
//                 the preceding Conv, and a residual Add (+ Relu) into the
//                 preceding quantized Conv, each only when the intermediate
//                 value has no other reader and is not a graph output;
//   3. memory     every activation gets an offset in one device arena, chosen
//                 greedily so values with overlapping lifetimes never share
//                 bytes; Reshape / Flatten / Cast are views (no copy);
//   4. launch     the ops become a list of C ABI calls on the current stream,
//                 optionally recorded once into a HIP graph and replayed.
// The arithmetic of each op follows the reference's execute_* functions
// (tbn-runtime/include/tbn/runtime/model.hpp:277-1300) in mode F32.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "internal.hpp"
#include "tbn/device.hpp"
#include "tbn/model.hpp"
#include "tbn/onnx_parser.hpp"
#include "tbn/session.hpp"
#include "tbn_hip.h"

namespace tbn {

// ===========================================================================
// TBNModel
// ===========================================================================

TBNModel::TBNModel() : graph_(std::make_shared<ModelGraph>()) {}
TBNModel::TBNModel(std::shared_ptr<ModelGraph> graph) : graph_(std::move(graph)) {
    TBN_CHECK(graph_ != nullptr, InvalidArgumentError, "graph is null");
}

bool TBNModel::has_input(const std::string& name) const {
    return std::find(graph_->inputs.begin(), graph_->inputs.end(), name) != graph_->inputs.end();
}

bool TBNModel::has_output(const std::string& name) const {
    return std::find(graph_->outputs.begin(), graph_->outputs.end(), name) != graph_->outputs.end();
}

const Shape& TBNModel::get_input_shape(const std::string& name) const {
    auto it = graph_->value_info.find(name);
    TBN_CHECK(it != graph_->value_info.end(), InvalidArgumentError, "Input '" + name + "' not found in model");
    return it->second;
}

const Shape& TBNModel::get_output_shape(const std::string& name) const {
    auto it = graph_->value_info.find(name);
    TBN_CHECK(it != graph_->value_info.end(), InvalidArgumentError, "Output '" + name + "' not found in model");
    return it->second;
}

void TBNModel::validate() const {
    TBN_CHECK(!graph_->inputs.empty(), InvalidModelError, "Model has no inputs");
    TBN_CHECK(!graph_->outputs.empty(), InvalidModelError, "Model has no outputs");
    TBN_CHECK(!graph_->nodes.empty(), InvalidModelError, "Model has no computation nodes");
    for (const auto& in : graph_->inputs)
        TBN_CHECK(graph_->value_info.count(in) > 0, InvalidModelError, "Input '" + in + "' shape not defined");
    for (const auto& out : graph_->outputs)
        TBN_CHECK(graph_->value_info.count(out) > 0, InvalidModelError, "Output '" + out + "' shape not defined");
    for (const auto& node : graph_->nodes) {
        for (const auto& in : node.inputs)
            TBN_CHECK(graph_->value_info.count(in) > 0 || graph_->initializers.count(in) > 0, InvalidModelError,
                      "Node input '" + in + "' not defined");
        for (const auto& out : node.outputs)
            TBN_CHECK(graph_->value_info.count(out) > 0, InvalidModelError,
                      "Node output '" + out + "' shape not defined");
    }
}

// model.cpp:10-21 of the reference: both go through the ONNX reader.
TBNModel load_model(const std::string& path) { return load_onnx_model(path); }

TBNModel load_model_from_buffer(const void* data, size_t size) { return load_onnx_model_from_buffer(data, size); }

const char* get_version() { return "0.1.0"; }

// ===========================================================================
// Session internals
// ===========================================================================

namespace {

tbn_stream_t cur_stream() { return device::current_stream(); }

// ---- attribute helpers ------------------------------------------------------

const AttributeValue* find_attr(const ModelNode& n, const char* key) {
    auto it = n.attributes.find(key);
    return it == n.attributes.end() ? nullptr : &it->second;
}

bool quantize_allowed(const ModelNode& n) {
    const AttributeValue* a = find_attr(n, "tbn_quantize");
    return !(a && a->is_int() && a->as_int() == 0);
}

// Conv2DParams from ONNX attributes as execute_conv reads them (model.hpp:296-352).
Conv2DParams conv_params(const ModelNode& node, const Shape& w) {
    Conv2DParams p;
    p.kernel_h = w.dims[2];
    p.kernel_w = w.dims[3];
    if (auto a = find_attr(node, "strides"); a && a->is_ints() && a->as_ints().size() >= 2) {
        p.stride_h = a->as_ints()[0];
        p.stride_w = a->as_ints()[1];
    }
    if (auto a = find_attr(node, "pads"); a && a->is_ints() && a->as_ints().size() >= 4) {
        p.pad_h = a->as_ints()[0];
        p.pad_w = a->as_ints()[1];
    }
    if (auto a = find_attr(node, "auto_pad"); a && a->is_string() &&
        (a->as_string() == "SAME_UPPER" || a->as_string() == "SAME_LOWER")) {
        p.pad_h = (p.kernel_h - 1) * p.dilation_h / 2;
        p.pad_w = (p.kernel_w - 1) * p.dilation_w / 2;
    }
    if (auto a = find_attr(node, "dilations"); a && a->is_ints() && a->as_ints().size() >= 2) {
        p.dilation_h = a->as_ints()[0];
        p.dilation_w = a->as_ints()[1];
    }
    if (auto a = find_attr(node, "group"); a && a->is_int()) p.groups = a->as_int();
    return p;
}

// Pool2DParams as execute_maxpool reads them (model.hpp:577-628): strides
// default to the kernel size.
// MaxPool (model.hpp:578-629) and AveragePool (model.hpp:632-682) attributes:
// strides default to the kernel, pads read as [top, left, ...]; MaxPool reads
// ceil_mode, AveragePool count_include_pad (and never ceil_mode).
Pool2DParams pool_params(const ModelNode& node, bool average = false) {
    Pool2DParams p;
    if (auto a = find_attr(node, "kernel_shape"); a && a->is_ints() && a->as_ints().size() >= 2) {
        p.kernel_h = a->as_ints()[0];
        p.kernel_w = a->as_ints()[1];
    }
    if (auto a = find_attr(node, "strides"); a && a->is_ints()) {
        if (a->as_ints().size() >= 2) {
            p.stride_h = a->as_ints()[0];
            p.stride_w = a->as_ints()[1];
        }
    } else {
        p.stride_h = p.kernel_h;
        p.stride_w = p.kernel_w;
    }
    if (auto a = find_attr(node, "pads"); a && a->is_ints() && a->as_ints().size() >= 4) {
        p.pad_h = a->as_ints()[0];
        p.pad_w = a->as_ints()[1];
    }
    if (average) {
        if (auto a = find_attr(node, "count_include_pad"); a && a->is_int()) p.count_include_pad = a->as_int() != 0;
    } else if (auto a = find_attr(node, "ceil_mode"); a && a->is_int()) {
        p.ceil_mode = a->as_int() != 0;
    }
    return p;
}

// ---- the lowered program ---------------------------------------------------

enum class OpKind {
    ConvF32,
    ConvQuant,
    ConvDepthwise,  // one input channel per group: fp32 weights (exact +-1 / ternary when quantized)
    ChannelAffine,  // BatchNormalization not folded into a conv
    GemmF32,
    GemmQuant,
    Add,
    Relu,
    TernaryAct,
    MaxPool,
    AvgPool,
    GlobalAvgPool,
    GlobalMaxPool,
    Elementwise,
    View,
};

struct Op {
    OpKind kind;
    std::string node;        // node name (for error messages)
    std::vector<int> in;     // value ids read
    int out = -1;            // value id written
    bool dead = false;       // removed by fusion
    // conv
    tbn_conv2d_desc desc{};
    int flags = 0;
    int residual = -1;       // value id of a fused residual addend
    const PackedWeights* pw = nullptr;
    const Tensor* conv_w = nullptr;  // conv-layout weights of the patch conv path
    int64_t groups = 1;              // > 1: one dense conv per group on channel slices
    std::string weight_name, scale_name, bias_name;  // initializers behind w / scale / bias
    std::vector<float> bn_k, bn_t;   // ChannelAffine: y = x * k + t per channel (host copy)
    std::vector<const Tensor*> group_conv_w;  // per-group conv-layout weights (grouped patch conv)
    int workspace = -1;              // value id of the op's transient workspace (grouped conv slices,
                                     // a TBN Gemm's fp4 activation rows)
    bool tbn = false;                // TBN arithmetic (ternarized activations, integer products)
    int pair = -1;                   // a 1x1 projection of the same input run in this conv's launch
    bool paired = false;             // this projection runs in its pair's launch (at the pair's position)
    int64_t tbn_scratch = 0;         // bytes of a TBN conv's record scratch (0: the fused kernel needs none)
    const Tensor* tbn_w = nullptr;   // its fp4 weights: TBN conv layout, or [N_pad, K_pad / 2] rows
    const float* scale = nullptr;  // per-channel scale (device)
    const float* w = nullptr;      // fp32 weights (device)
    const float* bias = nullptr;   // device
    int bias_value = -1;           // or a bias computed / supplied at run time
    // gemm
    int64_t M = 0, K = 0, N = 0;
    float alpha = 1.0f, beta = 0.0f;
    bool transA = false, transB = false;
    const float* cin = nullptr;    // constant addend (device) or null
    int cin_value = -1;            // or an activation addend
    const float* bt = nullptr;     // a constant fp32 B kept as [N, K] (the launch passes transB)
    int cin_1d = 0;
    int dyn_b = -1;                // quantized Gemm whose B is packed on every run
    // pooling / elementwise
    Pool2DParams pool;
    int64_t outer = 0, inner = 0, rest = 0;
    int elem_op = 0;
    float scalar = 0.0f;
    int rhs_value = -1;
    int64_t rhs_n = 0;
    const float* rhs_const = nullptr;
};

struct Value {
    std::string name;
    Shape shape;
    DataType dtype = DataType::FLOAT32;
    bool is_const = false;   // initializer: lives in the weight cache
    bool is_input = false;
    int view_of = -1;        // storage shared with another value
    const void* const_ptr = nullptr;
    void* bound = nullptr;   // input read in place from the caller's device tensor
    int64_t offset = -1;     // arena offset (bytes)
    int def = -1, last = -1; // op index of definition and last use
};

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

struct TBNModel::Session::Impl {
    std::shared_ptr<ModelGraph> graph;
    TilingParams tiling;
    bool quant = false;
    QuantArithmetic arith = QuantArithmetic::F32;
    bool graph_replay = false;
    std::unordered_map<std::string, Tensor> inputs;

    // ---- caches that live as long as the Session ----
    std::unordered_map<std::string, Tensor> dev_init;          // uploaded initializers
    std::unordered_map<std::string, std::vector<float>> channel_scales;  // host copy of mean|w|
    std::unordered_map<std::string, Tensor> dev_scales;        // device per-channel scales
    std::unordered_map<std::string, bool> conv_already_binary;
    std::unordered_map<std::string, PackedWeights> packed;      // key: name + "#" + variant
    std::unordered_map<std::string, Tensor> conv_packed;        // conv-layout copies of `packed` entries
    std::unordered_map<std::string, Tensor> scaled_addends;     // beta * C of quantized Gemms
    std::unordered_map<std::string, Tensor> derived;            // depthwise +-1 weights, BatchNormalization folds
    std::unordered_map<std::string, Tensor> tbn_packed;         // fp4 weights of TBN-mode layers

    // ---- the compiled plan ----
    bool planned = false;
    bool plan_quant = false;
    QuantArithmetic plan_arith = QuantArithmetic::F32;
    std::map<std::string, Shape> plan_shapes;
    std::deque<Value> values;  // deque: references stay valid as values are added
    std::unordered_map<std::string, int> value_id;
    std::vector<Op> ops;
    Tensor arena;
    size_t launches = 0;
    hipStream_t replay_stream = nullptr;
    hipGraph_t hip_graph = nullptr;
    hipGraphExec_t hip_graph_exec = nullptr;
    int eager_runs = 0;
    bool replay_off = false;  // the plan needs an allocation that capture refuses

    ~Impl() { drop_graph(); if (replay_stream) (void)hipStreamDestroy(replay_stream); }

    void drop_graph() {
        if (hip_graph_exec) (void)hipGraphExecDestroy(hip_graph_exec);
        if (hip_graph) (void)hipGraphDestroy(hip_graph);
        hip_graph_exec = nullptr;
        hip_graph = nullptr;
    }

    // ---- weight helpers ------------------------------------------------------

    const Tensor& initializer(const std::string& name) const {
        auto it = graph->initializers.find(name);
        TBN_CHECK(it != graph->initializers.end(), RuntimeError, "initializer '" + name + "' not found");
        return it->second;
    }

    const Tensor& device_init(const std::string& name) {
        auto it = dev_init.find(name);
        if (it != dev_init.end()) return it->second;
        const Tensor& t = initializer(name);
        return dev_init.emplace(name, t.on_device() ? t : t.to_device(DeviceType::HIP)).first->second;
    }

    std::vector<float> host_floats(const std::string& name) const {
        return initializer(name).to_vector<float>();
    }

    // A constant [K, N] fp32 matrix stored once as [N, K]: every fp32 GEMM
    // kernel reads a column of op(B) as consecutive k then (16-byte loads
    // along k), and the product is the same.
    const float* transposed_init(const std::string& name, int64_t K, int64_t N) {
        const std::string key = name + "#T";
        auto it = dev_init.find(key);
        if (it == dev_init.end()) {
            const std::vector<float> b = host_floats(name);
            std::vector<float> t(b.size());
            for (int64_t k = 0; k < K; ++k)
                for (int64_t n = 0; n < N; ++n) t[n * K + k] = b[k * N + n];
            it = dev_init.emplace(key, Tensor(Shape{N, K}, DataType::FLOAT32, t.data(), DeviceType::HIP)).first;
        }
        return it->second.typed_data<float>();
    }

    // Per-channel mean|w| computed on the device with the Session's sequential
    // fp32 sum (model.hpp:383-395), plus the "already binary" test
    // (model.hpp:396-410) on the host copy of the weights.
    void conv_scales(const std::string& wname) {
        if (conv_already_binary.count(wname)) return;
        const Tensor& w = device_init(wname);
        const int64_t ch = w.shape().dims[0];
        const int64_t per = w.num_elements() / ch;
        Tensor s = Tensor::empty({ch}, DataType::FLOAT32, DeviceType::HIP);
        check_status(tbn_hip_channel_mean_abs(w.typed_data<float>(), ch, per, s.typed_data<float>(), cur_stream()),
                     "channel_mean_abs");
        std::vector<float> hs = s.to_vector<float>();
        const std::vector<float> hw = host_floats(wname);
        bool already = true;
        for (int64_t c = 0; c < ch && already; ++c) {
            const float scale = hs[c];
            int64_t near = 0;
            for (int64_t i = 0; i < per; ++i) {
                const float v = hw[c * per + i];
                const float expected = (v >= 0) ? scale : -scale;
                if (std::abs(v - expected) < 0.01f * scale || std::abs(v) < 0.01f) ++near;
            }
            if (near < per * 0.9f) already = false;
        }
        channel_scales[wname] = hs;
        dev_scales[wname] = s;
        conv_already_binary[wname] = already;
    }

    const PackedWeights& packed_binary(const std::string& wname, bool nk, int rule) {
        // rule: 0 = BINARY bytes, 1 = float w > 0, 2 = float w >= 0, 3 = TERNARY
        // values collapsed to signs as conv2d_ternary does (t < 0 -> -1, 0 and
        // +1 -> +1; conv2d.cpp:195-217)
        const std::string key = wname + "#b" + std::to_string(nk) + std::to_string(rule);
        auto it = packed.find(key);
        if (it != packed.end()) return it->second;
        if (rule == 3) {
            const Tensor& w = initializer(wname);
            const Tensor host = w.on_device() ? w.to_device(DeviceType::CPU) : w;
            Tensor bin(host.shape(), DataType::BINARY);
            for (int64_t i = 0; i < host.num_elements(); ++i)
                bin.typed_data<uint8_t>()[i] = host.typed_data<int8_t>()[i] < 0 ? 0 : 1;
            return packed.emplace(key, pack_binary_weights(bin.to_device(DeviceType::HIP), nk, false)).first->second;
        }
        return packed.emplace(key, pack_binary_weights(device_init(wname), nk, rule == 2)).first->second;
    }

    // fp4 weights of a TBN-mode conv (the TBN conv layout) or Gemm ([N_pad,
    // K_pad / 2] rows), made once per Session from the packed bits.
    const Tensor& tbn_conv_weights(const std::string& node, const PackedWeights& pw, const tbn_conv2d_desc& d) {
        const std::string key = node + "#tbnconv" + std::to_string(reinterpret_cast<uintptr_t>(&pw));
        auto it = tbn_packed.find(key);
        if (it != tbn_packed.end()) return it->second;
        int64_t bytes = 0;
        check_status(tbn_hip_tbn_conv_weights_bytes(&d, &bytes), ("Conv '" + node + "'").c_str());
        Tensor w4 = Tensor::empty({bytes}, DataType::UINT8, DeviceType::HIP);
        check_status(tbn_hip_pack_tbn_conv_weights(pw.bits.typed_data<uint8_t>(), pw.K_pad, pw.N_pad, &d,
                                                   w4.typed_data<uint8_t>(), cur_stream()),
                     ("Conv '" + node + "'").c_str());
        return tbn_packed.emplace(key, w4).first->second;
    }

    const Tensor& tbn_gemm_weights(const std::string& node, const PackedWeights& pw, bool fill) {
        const std::string key = node + "#tbngemm" + std::to_string(reinterpret_cast<uintptr_t>(&pw));
        auto it = tbn_packed.find(key);
        if (it != tbn_packed.end()) return it->second;
        Tensor w4 = Tensor::empty({pw.N_pad * pw.K_pad / 2}, DataType::UINT8, DeviceType::HIP);
        if (fill)
            check_status(tbn_hip_pack_f4_weights(pw.bits.typed_data<uint8_t>(), pw.K_pad, pw.N_pad,
                                                 w4.typed_data<uint8_t>(), cur_stream()),
                         ("Gemm '" + node + "'").c_str());
        return tbn_packed.emplace(key, w4).first->second;
    }

    // The packed-bits buffer of a quantized Gemm whose B is not an initializer
    // (filled by the op itself on every run).
    const PackedWeights& dynamic_binary(const std::string& node_name, int64_t K, int64_t N) {
        PackedWeights pw;
        pw.kind = PackedWeights::Kind::Binary;
        pw.K = K;
        pw.N = N;
        pw.K_pad = detail::ceil_to(K, 128);
        pw.N_pad = detail::ceil_to(N, 8);
        pw.bits = Tensor::empty({pw.N_pad * pw.K_pad / 8}, DataType::UINT8, DeviceType::HIP);
        return packed.insert_or_assign(node_name + "#dyn", std::move(pw)).first->second;
    }

    const PackedWeights& packed_ternary(const std::string& wname, bool nk) {
        const std::string key = wname + "#t" + std::to_string(nk);
        auto it = packed.find(key);
        if (it != packed.end()) return it->second;
        return packed.emplace(key, pack_ternary_weights(device_init(wname), nk)).first->second;
    }

    // The quantized Gemm's "already binary" test samples about 1000 values for
    // exact -1, 1, 0, 0.999, -0.999 (model.hpp:765-786).
    bool gemm_already_binary(const std::string& bname) {
        const std::vector<float> b = host_floats(bname);
        const int64_t n = static_cast<int64_t>(b.size());
        const int64_t step = std::max<int64_t>(1, n / 1000);
        for (int64_t i = 0; i < n; i += step) {
            const float v = b[i];
            if (v != -1.0f && v != 1.0f && v != 0.0f && v != 0.999f && v != -0.999f) return false;
        }
        return true;
    }

    // ---- compilation ---------------------------------------------------------------

    int new_value(const std::string& name, const Shape& shape, DataType dt) {
        Value v;
        v.name = name;
        v.shape = shape;
        v.dtype = dt;
        values.push_back(v);
        value_id[name] = static_cast<int>(values.size()) - 1;
        return value_id[name];
    }

    int lookup(const std::string& name, const std::string& node) {
        auto it = value_id.find(name);
        if (it != value_id.end()) return it->second;
        auto init = graph->initializers.find(name);
        TBN_CHECK(init != graph->initializers.end(), RuntimeError,
                  "node '" + node + "': input '" + name + "' not found");
        int id = new_value(name, init->second.shape(), init->second.dtype());
        values[id].is_const = true;
        values[id].const_ptr = device_init(name).data();
        return id;
    }

    const float* const_f32(int id) const { return static_cast<const float*>(values[id].const_ptr); }

    // Weights of a depthwise layer as fp32 on the device: the initializer
    // itself, or its exact +-1 / -1,0,+1 values when the layer is quantized
    // (`rule`: 0 BINARY bytes, 1 w > 0, 2 w >= 0, 3 TERNARY values).
    const float* depthwise_weights(const std::string& wname, int rule) {
        const std::string key = wname + "#dw" + std::to_string(rule);
        auto it = derived.find(key);
        if (it != derived.end()) return it->second.typed_data<float>();
        const Tensor& w = initializer(wname);
        const Tensor host = w.on_device() ? w.to_device(DeviceType::CPU) : w;
        const int64_t n = host.num_elements();
        std::vector<float> v(static_cast<size_t>(n));
        for (int64_t i = 0; i < n; ++i) {
            if (rule == 0) v[i] = host.typed_data<uint8_t>()[i] == 1 ? 1.0f : -1.0f;
            else if (rule == 3) v[i] = static_cast<float>(host.typed_data<int8_t>()[i]);
            else {
                const float x = host.typed_data<float>()[i];
                v[i] = (rule == 2 ? x >= 0.0f : x > 0.0f) ? 1.0f : -1.0f;
            }
        }
        Tensor d(host.shape(), DataType::FLOAT32, v.data(), DeviceType::HIP);
        return derived.emplace(key, d).first->second.typed_data<float>();
    }

    void lower_conv(const ModelNode& node) {
        TBN_CHECK(node.inputs.size() >= 2, InvalidArgumentError, "Conv expects at least 2 inputs");
        TBN_CHECK(node.outputs.size() == 1, InvalidArgumentError, "Conv expects 1 output");
        const int xi = lookup(node.inputs[0], node.name);
        const std::string& wname = node.inputs[1];
        TBN_CHECK(graph->initializers.count(wname), NotImplementedError,
                  "Conv '" + node.name + "': weights must be an initializer");
        const int wi = lookup(wname, node.name);
        const Shape xs = values[xi].shape;
        const Shape ws = values[wi].shape;
        TBN_CHECK(xs.rank() == 4, InvalidShapeError, "Conv input must be 4D (NCHW), got " + shape_to_string(xs));
        TBN_CHECK(ws.rank() == 4, InvalidShapeError, "Conv weights must be 4D, got " + shape_to_string(ws));
        const Conv2DParams p = conv_params(node, ws);
        // conv2d_grouped (conv2d.cpp:372-384) throws for groups > 1; here a
        // group of one input channel is the depthwise kernel and larger groups
        // run the dense kernels group by group.
        TBN_CHECK(p.groups >= 1 && ws.dims[0] % p.groups == 0, InvalidShapeError,
                  "Conv '" + node.name + "': output channels must be divisible by group");
        TBN_CHECK(xs.dims[1] == ws.dims[1] * p.groups, InvalidShapeError, "Conv '" + node.name + "': channel mismatch");
        Op op;
        op.node = node.name;
        op.in.push_back(xi);
        op.groups = p.groups;
        op.desc = tbn_conv2d_desc{xs.dims[0], xs.dims[1], xs.dims[2], xs.dims[3], ws.dims[0], ws.dims[2],
                                  ws.dims[3], p.stride_h, p.stride_w, p.pad_h, p.pad_w, p.dilation_h, p.dilation_w};
        const int64_t OH = (xs.dims[2] + 2 * p.pad_h - p.dilation_h * (ws.dims[2] - 1) - 1) / p.stride_h + 1;
        const int64_t OW = (xs.dims[3] + 2 * p.pad_w - p.dilation_w * (ws.dims[3] - 1) - 1) / p.stride_w + 1;
        TBN_CHECK(OH > 0 && OW > 0, InvalidShapeError, "Conv '" + node.name + "': invalid output dimensions");
        if (node.inputs.size() >= 3 && !node.inputs[2].empty()) {
            // any value of the graph, as the reference reads it (model.hpp:207-214)
            const int bi = lookup(node.inputs[2], node.name);
            TBN_CHECK(values[bi].shape.size() == ws.dims[0], InvalidShapeError,
                      "Conv '" + node.name + "': bias size must equal the output channels");
            if (values[bi].is_const) {
                op.bias = const_f32(bi);
                op.bias_name = node.inputs[2];
            } else {
                TBN_CHECK(values[bi].dtype == DataType::FLOAT32, InvalidArgumentError,
                          "Conv '" + node.name + "': bias must be FLOAT32");
                op.bias_value = bi;
                op.in.push_back(bi);
            }
        }
        op.weight_name = wname;
        const bool depthwise = p.groups > 1 && ws.dims[1] == 1;
        const DataType wt = values[wi].dtype;
        // TBN arithmetic for the convs the reference itself can run
        const bool tbn = arith == QuantArithmetic::TBN && p.groups == 1;
        int dw_rule = -1;  // depthwise weights: -1 fp32 as stored, else the depthwise_weights rule
        if (wt == DataType::BINARY) {
            op.kind = OpKind::ConvQuant;
            if (depthwise) dw_rule = 0;
            else op.pw = &packed_binary(wname, true, 0);
        } else if (wt == DataType::TERNARY) {
            op.kind = OpKind::ConvQuant;
            if (depthwise) dw_rule = 3;
            else op.pw = tbn ? &packed_binary(wname, true, 3) : &packed_ternary(wname, true);
        } else if (wt == DataType::FLOAT32 && quant && quantize_allowed(node)) {
            op.kind = OpKind::ConvQuant;
            conv_scales(wname);
            if (conv_already_binary[wname]) {
                // cached path: signs w >= 0, y = (acc + b) * s[m] (model.hpp:414-559)
                if (depthwise) dw_rule = 2;
                else op.pw = &packed_binary(wname, true, 2);
                op.scale = dev_scales[wname].typed_data<float>();
                op.scale_name = wname;
                op.flags |= TBN_EPI_BIAS_THEN_SCALE;
            } else {
                // quantize_to_binary(W) (w > 0) then conv2d_binary, no scale (model.hpp:560-564)
                if (depthwise) dw_rule = 1;
                else op.pw = &packed_binary(wname, true, 1);
            }
        } else {
            TBN_CHECK(wt == DataType::FLOAT32, InvalidArgumentError, "Conv '" + node.name + "': unsupported weight type");
            op.kind = OpKind::ConvF32;
            op.w = const_f32(wi);
        }
        if (depthwise) {
            op.kind = OpKind::ConvDepthwise;
            op.w = dw_rule < 0 ? const_f32(wi) : depthwise_weights(wname, dw_rule);
            op.out = new_value(node.outputs[0], Shape{xs.dims[0], ws.dims[0], OH, OW}, DataType::FLOAT32);
            ops.push_back(op);
            return;
        }
        if (tbn && op.kind == OpKind::ConvQuant) {
            // ternarized taps times the +-1 weights, then the reference's
            // bias / scale steps (model.hpp:482-557, conv2d.cpp:220-316)
            op.tbn = true;
            op.tbn_w = &tbn_conv_weights(node.name, *op.pw, op.desc);
            // the two-pass kernels' ternarized input: a workspace slot of the arena
            check_status(tbn_hip_tbn_conv_scratch_bytes(&op.desc, &op.tbn_scratch),
                         ("Conv '" + node.name + "'").c_str());
            if (op.tbn_scratch) op.workspace = new_value(node.name + "#t4", Shape{op.tbn_scratch}, DataType::UINT8);
            op.out = new_value(node.outputs[0], Shape{xs.dims[0], ws.dims[0], OH, OW}, DataType::FLOAT32);
            ops.push_back(op);
            return;
        }
        // the descriptor one group's dense conv sees
        tbn_conv2d_desc dg = op.desc;
        dg.c /= p.groups;
        dg.m /= p.groups;
        const int kind = op.pw && op.pw->kind == PackedWeights::Kind::Ternary ? TBN_WEIGHTS_TERNARY
                                                                              : TBN_WEIGHTS_BINARY;
        int64_t wbytes = 0;
        if (op.kind == OpKind::ConvQuant && dg.c >= 16 &&
            tbn_hip_conv_weights_bytes(kind, &dg, &wbytes) == TBN_SUCCESS) {
            // patch conv: conv-layout weights once per Session (per group),
            // then no allocation and no re-ordering per run
            const int64_t col_bytes = kind == TBN_WEIGHTS_BINARY ? op.pw->K_pad / 8 : op.pw->K_pad / 4;
            for (int64_t g = 0; g < p.groups; ++g) {
                const std::string key = wname + "#conv" + std::to_string(reinterpret_cast<uintptr_t>(op.pw)) + "g" +
                                        std::to_string(g) + "/" + std::to_string(p.groups);
                auto it = conv_packed.find(key);
                if (it == conv_packed.end()) {
                    Tensor cw = Tensor::empty({wbytes}, DataType::UINT8, DeviceType::HIP);
                    check_status(tbn_hip_pack_conv_weights(kind, op.pw->bits.typed_data<uint8_t>() + g * dg.m * col_bytes,
                                                           op.pw->K_pad, op.pw->N_pad - g * dg.m, &dg,
                                                           cw.typed_data<uint8_t>(), cur_stream()),
                                 ("Conv '" + node.name + "'").c_str());
                    it = conv_packed.emplace(key, cw).first;
                }
                op.group_conv_w.push_back(&it->second);
            }
            op.conv_w = op.group_conv_w[0];
        }
        if (p.groups > 1) {
            const int64_t ws_floats = detail::grouped_conv_workspace(op.desc, p.groups);
            if (ws_floats) op.workspace = new_value(node.name + "#groups", Shape{ws_floats}, DataType::FLOAT32);
        }
        op.out = new_value(node.outputs[0], Shape{xs.dims[0], ws.dims[0], OH, OW}, DataType::FLOAT32);
        ops.push_back(op);
    }

    // ONNX BatchNormalization in inference form (not in the reference):
    // y = (x - mean) / sqrt(var + epsilon) * scale + B over dim 1, as
    // y = x * k + t; folded into a preceding conv's epilogue by fold_batchnorm.
    void lower_batchnorm(const ModelNode& node) {
        TBN_CHECK(node.inputs.size() == 5 && !node.outputs.empty(), InvalidArgumentError,
                  "BatchNormalization expects 5 inputs");
        if (auto a = find_attr(node, "training_mode"); a && a->is_int())
            TBN_CHECK(a->as_int() == 0, NotImplementedError, "BatchNormalization '" + node.name + "': training mode");
        const int xi = lookup(node.inputs[0], node.name);
        const Shape xs = values[xi].shape;
        TBN_CHECK(xs.rank() >= 2, InvalidShapeError, "BatchNormalization input must be at least 2-D");
        for (int i = 1; i < 5; ++i)
            TBN_CHECK(graph->initializers.count(node.inputs[i]), NotImplementedError,
                      "BatchNormalization '" + node.name + "': parameters must be initializers");
        float eps = 1e-5f;
        if (auto a = find_attr(node, "epsilon"); a && a->is_float()) eps = a->as_float();
        std::vector<float> k, t;
        detail::batch_norm_affine(initializer(node.inputs[1]), initializer(node.inputs[2]),
                                  initializer(node.inputs[3]), initializer(node.inputs[4]), eps, xs.dims[1], k, t);
        Op op;
        op.kind = OpKind::ChannelAffine;
        op.node = node.name;
        op.in = {xi};
        op.bn_k = k;
        op.bn_t = t;
        op.scale = derived_floats(node.name + "#bn_k", k);
        op.bias = derived_floats(node.name + "#bn_t", t);
        int64_t hw = 1;
        for (size_t i = 2; i < xs.dims.size(); ++i) hw *= xs.dims[i];
        op.outer = xs.dims[0];
        op.inner = xs.dims[1];
        op.rest = hw;
        op.out = new_value(node.outputs[0], xs, DataType::FLOAT32);
        ops.push_back(op);
    }

    // Device copy of `v`, kept for the Session's lifetime.  An entry already
    // queued kernels may read is never replaced: other contents get a new key.
    const float* derived_floats(std::string key, const std::vector<float>& v) {
        for (;;) {
            auto it = derived.find(key);
            if (it == derived.end()) break;
            const Tensor& t = it->second;
            if (t.num_elements() == static_cast<int64_t>(v.size())) {
                const std::vector<float> have = t.to_vector<float>();
                if (std::memcmp(have.data(), v.data(), v.size() * sizeof(float)) == 0) return t.typed_data<float>();
            }
            key += "'";
        }
        Tensor d(Shape{static_cast<int64_t>(v.size())}, DataType::FLOAT32, v.data(), DeviceType::HIP);
        return derived.emplace(key, d).first->second.typed_data<float>();
    }

    void lower_gemm(const ModelNode& node, bool matmul) {
        TBN_CHECK(node.inputs.size() >= 2, InvalidArgumentError, "Gemm expects at least 2 inputs");
        TBN_CHECK(node.outputs.size() == 1, InvalidArgumentError, "Gemm expects 1 output");
        Op op;
        op.node = node.name;
        if (!matmul) {
            if (auto a = find_attr(node, "alpha"); a && a->is_float()) op.alpha = a->as_float();
            op.beta = 1.0f;
            if (auto a = find_attr(node, "beta"); a && a->is_float()) op.beta = a->as_float();
            if (auto a = find_attr(node, "transA"); a && a->is_int()) op.transA = a->as_int() != 0;
            if (auto a = find_attr(node, "transB"); a && a->is_int()) op.transB = a->as_int() != 0;
        }
        const int ai = lookup(node.inputs[0], node.name);
        const int bi = lookup(node.inputs[1], node.name);
        const Shape as = values[ai].shape;
        const Shape bs = values[bi].shape;
        if (as.rank() != 2 || bs.rank() != 2) {
            if (matmul) throw NotImplementedError("MatMul for non-2D tensors not implemented");
            throw InvalidShapeError("Gemm '" + node.name + "': inputs must be 2-D");
        }
        op.M = op.transA ? as.dims[1] : as.dims[0];
        op.K = op.transA ? as.dims[0] : as.dims[1];
        const int64_t Kb = op.transB ? bs.dims[1] : bs.dims[0];
        op.N = op.transB ? bs.dims[0] : bs.dims[1];
        TBN_CHECK(op.K == Kb, InvalidShapeError, "Gemm '" + node.name + "': inner dimensions differ");
        op.in = {ai};
        int ci = -1;
        if (!matmul && node.inputs.size() >= 3 && !node.inputs[2].empty()) {
            ci = lookup(node.inputs[2], node.name);
            const int64_t cn = values[ci].shape.size();
            op.cin_1d = values[ci].shape.rank() == 1 ? 1 : 0;
            TBN_CHECK(op.cin_1d ? cn == op.N : cn == op.M * op.N, InvalidShapeError,
                      "Gemm '" + node.name + "': C must be [N] or [M, N]");
        }
        const bool quantized = quant && quantize_allowed(node) && !matmul && values[bi].dtype == DataType::FLOAT32 &&
                               !op.transA && !op.transB;
        if (quantized) {
            op.kind = OpKind::GemmQuant;
            const std::string& bname = node.inputs[1];
            if (values[bi].is_const) {
                // already binary: signs w >= 0 (model.hpp:790-841); otherwise
                // quantize_to_binary (w > 0) (model.hpp:842-845); scale 1 either way.
                op.pw = &packed_binary(bname, false, gemm_already_binary(bname) ? 2 : 1);
            } else {
                // B computed or supplied at run time: the same test and packing
                // on the device on every run (TBN_SIGN_GEMM_SAMPLED).
                op.pw = &dynamic_binary(node.name, op.K, op.N);
                op.dyn_b = bi;
                op.in.push_back(bi);
            }
            // then result * alpha + beta * C (model.hpp:847-870)
            if (arith == QuantArithmetic::TBN) {
                // qlinear_matmul_binary_blocked_packed's ternarized product
                // (quantized_gemm_neon.cpp:249-309); the fp4 activation rows
                // go to a workspace slot of the arena
                op.tbn = true;
                op.tbn_w = &tbn_gemm_weights(node.name, *op.pw, op.dyn_b < 0);
                op.workspace = new_value(node.name + "#t4", Shape{op.M * (op.pw->K_pad / 2)}, DataType::UINT8);
            }
        } else {
            op.kind = OpKind::GemmF32;
            op.in.push_back(bi);
            TBN_CHECK(values[bi].dtype == DataType::FLOAT32 && values[ai].dtype == DataType::FLOAT32,
                      InvalidArgumentError, "gemm requires float32 inputs");
            if (values[bi].is_const && !op.transB) op.bt = transposed_init(node.inputs[1], op.K, op.N);
        }
        if (ci >= 0 && op.beta != 0.0f) {
            if (values[ci].is_const) op.cin = const_f32(ci);
            else { op.cin_value = ci; op.in.push_back(ci); }
        }
        op.out = new_value(node.outputs[0], Shape{op.M, op.N}, DataType::FLOAT32);
        ops.push_back(op);
    }

    void lower_unary(const ModelNode& node, OpKind kind) {
        TBN_CHECK(node.inputs.size() >= 1 && node.outputs.size() >= 1, InvalidArgumentError,
                  node.op_type + " expects 1 input and 1 output");
        const int xi = lookup(node.inputs[0], node.name);
        Op op;
        op.kind = kind;
        op.node = node.name;
        op.in = {xi};
        Shape out = values[xi].shape;
        if (kind == OpKind::MaxPool || kind == OpKind::AvgPool || kind == OpKind::GlobalAvgPool ||
            kind == OpKind::GlobalMaxPool) {
            TBN_CHECK(out.rank() == 4, InvalidShapeError, node.op_type + " input must be 4D (NCHW)");
        }
        if (kind == OpKind::MaxPool || kind == OpKind::AvgPool) {
            op.pool = pool_params(node, kind == OpKind::AvgPool);
            const auto& d = out.dims;
            const Pool2DParams& p = op.pool;
            int64_t hw[2];
            const std::string what = node.op_type + " '" + node.name + "'";
            if (kind == OpKind::MaxPool)
                check_status(tbn_hip_maxpool2d(nullptr, d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w, p.stride_h,
                                               p.stride_w, p.pad_h, p.pad_w, 1, 1, p.ceil_mode, nullptr, hw, nullptr),
                             what.c_str());
            else
                check_status(tbn_hip_avgpool2d(nullptr, d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w, p.stride_h,
                                               p.stride_w, p.pad_h, p.pad_w, 1, 1, 0, p.count_include_pad, nullptr,
                                               hw, nullptr),
                             what.c_str());
            out = Shape{d[0], d[1], hw[0], hw[1]};
        } else if (kind == OpKind::GlobalAvgPool || kind == OpKind::GlobalMaxPool) {
            out = Shape{out.dims[0], out.dims[1], 1, 1};
        } else if (kind == OpKind::TernaryAct) {
            op.scalar = 0.5f;
        }
        op.out = new_value(node.outputs[0], out, DataType::FLOAT32);
        ops.push_back(op);
    }

    void lower_view(const ModelNode& node, const Shape& shape) {
        const int xi = lookup(node.inputs[0], node.name);
        TBN_CHECK(shape.size() == values[xi].shape.size(), InvalidShapeError,
                  node.op_type + " '" + node.name + "' changes the element count");
        Op op;
        op.kind = OpKind::View;
        op.node = node.name;
        op.in = {xi};
        op.out = new_value(node.outputs[0], shape, values[xi].dtype);
        values[op.out].view_of = xi;
        ops.push_back(op);
    }

    void lower_add(const ModelNode& node) {
        TBN_CHECK(node.inputs.size() == 2, InvalidArgumentError, "Add expects 2 inputs");
        TBN_CHECK(node.outputs.size() == 1, InvalidArgumentError, "Add expects 1 output");
        int ai = lookup(node.inputs[0], node.name);
        int bi = lookup(node.inputs[1], node.name);
        if (values[ai].shape.rank() == 1 && values[bi].shape.rank() == 2) std::swap(ai, bi);
        Op op;
        op.kind = OpKind::Add;
        op.node = node.name;
        op.in = {ai, bi};
        detail::add_view(values[ai].shape, values[bi].shape, op.outer, op.inner, op.rest);
        op.out = new_value(node.outputs[0], values[ai].shape, DataType::FLOAT32);
        ops.push_back(op);
    }

    void lower_elementwise(const ModelNode& node, int elem_op) {
        TBN_CHECK(node.inputs.size() == 2 && node.outputs.size() == 1, InvalidArgumentError,
                  node.op_type + " expects 2 inputs and 1 output");
        const int ai = lookup(node.inputs[0], node.name);
        Op op;
        op.kind = OpKind::Elementwise;
        op.node = node.name;
        op.elem_op = elem_op;
        op.in = {ai};
        const bool have_rhs = value_id.count(node.inputs[1]) || graph->initializers.count(node.inputs[1]);
        if (have_rhs) {
            const int bi = lookup(node.inputs[1], node.name);
            op.rhs_n = values[bi].shape.size();
            TBN_CHECK(op.rhs_n > 0, InvalidShapeError, node.op_type + " right operand is empty");
            if (values[bi].is_const) op.rhs_const = const_f32(bi);
            else { op.rhs_value = bi; op.in.push_back(bi); }
        } else {
            TBN_CHECK(elem_op != TBN_OP_SUB, RuntimeError, "Sub rhs not found");
            auto a = find_attr(node, "value");
            op.scalar = a ? a->as_float() : 0.0f;
        }
        op.out = new_value(node.outputs[0], values[ai].shape, DataType::FLOAT32);
        ops.push_back(op);
    }

    void lower(const ModelNode& node) {
        const std::string& t = node.op_type;
        if (t == "Conv") return lower_conv(node);
        if (t == "BatchNormalization") return lower_batchnorm(node);
        if (t == "Gemm") return lower_gemm(node, false);
        if (t == "MatMul") return lower_gemm(node, true);
        if (t == "Add") return lower_add(node);
        if (t == "Relu") {
            // the reference turns Relu into a ternary activation (threshold 0.5)
            // when quantization is on and the input name matches (model.hpp:1144-1165)
            const bool ternary = quant && (node.inputs[0].find("conv2d_1") != std::string::npos ||
                                           node.inputs[0].find("conv2_out") != std::string::npos);
            return lower_unary(node, ternary ? OpKind::TernaryAct : OpKind::Relu);
        }
        if (t == "MaxPool") return lower_unary(node, OpKind::MaxPool);
        if (t == "AveragePool" || t == "AvgPool") return lower_unary(node, OpKind::AvgPool);
        if (t == "GlobalAveragePool" || t == "GlobalAvgPool") return lower_unary(node, OpKind::GlobalAvgPool);
        if (t == "GlobalMaxPool") return lower_unary(node, OpKind::GlobalMaxPool);
        if (t == "Flatten") {
            const int xi = lookup(node.inputs[0], node.name);
            int64_t axis = 1;
            if (auto a = find_attr(node, "axis"); a && a->is_int()) axis = a->as_int();
            const auto& d = values[xi].shape.dims;
            TBN_CHECK(axis >= 0 && axis <= static_cast<int64_t>(d.size()), InvalidArgumentError, "Flatten axis out of range");
            int64_t outer = 1, inner = 1;
            for (int64_t i = 0; i < axis; ++i) outer *= d[i];
            for (size_t i = axis; i < d.size(); ++i) inner *= d[i];
            return lower_view(node, Shape{outer, inner});
        }
        if (t == "Reshape") {
            const int xi = lookup(node.inputs[0], node.name);
            Shape s;
            if (node.inputs.size() >= 2) {
                auto it = graph->initializers.find(node.inputs[1]);
                TBN_CHECK(it != graph->initializers.end(), NotImplementedError,
                          "Reshape '" + node.name + "': the shape must be an initializer");
                const std::vector<int64_t> dims = it->second.to_vector<int64_t>();
                s.dims = dims;
            }
            int64_t known = 1;
            int unknown = -1;
            for (size_t i = 0; i < s.dims.size(); ++i) {
                if (s.dims[i] == -1) unknown = static_cast<int>(i);
                else known *= s.dims[i];
            }
            if (unknown >= 0) s.dims[unknown] = known ? values[xi].shape.size() / known : 0;
            return lower_view(node, s);
        }
        if (t == "Cast") return lower_view(node, values[lookup(node.inputs[0], node.name)].shape);
        if (t == "Sub") return lower_elementwise(node, TBN_OP_SUB);
        if (t == "Greater") return lower_elementwise(node, TBN_OP_GREATER);
        if (t == "Less") return lower_elementwise(node, TBN_OP_LESS);
        throw NotImplementedError("Operator '" + t + "' not implemented");
    }

    // ---- fusion -------------------------------------------------------------------

    std::vector<int> readers(int v) const {
        std::vector<int> r;
        for (size_t i = 0; i < ops.size(); ++i)
            if (!ops[i].dead && std::find(ops[i].in.begin(), ops[i].in.end(), v) != ops[i].in.end())
                r.push_back(static_cast<int>(i));
        return r;
    }

    bool is_output(int v) const {
        for (const auto& o : graph->outputs)
            if (value_id.count(o) && value_id.at(o) == v) return true;
        return false;
    }

    // The single op reading value v, or -1 when v has several readers, a view
    // reading it, or is a graph output.
    int sole_reader(int v) const {
        if (is_output(v)) return -1;
        auto r = readers(v);
        if (r.size() != 1) return -1;
        return r[0];
    }

    // Op `victim` is absorbed into op `host`: its output becomes host's output.
    void absorb(int host, int victim) {
        ops[victim].dead = true;
        const int old_out = ops[host].out;
        ops[host].out = ops[victim].out;
        (void)old_out;
    }

    // A BatchNormalization reading a conv's output that nothing else reads
    // becomes part of the conv's epilogue: with v = (acc + a) * s + b,
    // v * k + t = acc * (s*k) + (a*s*k + b*k + t), products formed in double
    // and rounded once.  The fp32 conv has no scale stage: its weights are
    // scaled instead (w * k per output channel).
    void fold_batchnorm() {
        for (size_t i = 0; i < ops.size(); ++i) {
            Op& bn = ops[i];
            if (bn.dead || bn.kind != OpKind::ChannelAffine) continue;
            const int p = producer(bn.in[0]);
            if (p < 0) continue;
            Op& c = ops[p];
            const bool conv = c.kind == OpKind::ConvF32 || c.kind == OpKind::ConvQuant || c.kind == OpKind::ConvDepthwise;
            if (!conv || c.residual >= 0 || c.bias_value >= 0 || (c.flags & (TBN_EPI_RELU | TBN_EPI_MAXPOOL2X2)) ||
                sole_reader(c.out) != static_cast<int>(i) || static_cast<int64_t>(bn.bn_k.size()) != c.desc.m)
                continue;
            const int64_t M = c.desc.m;
            const bool bts = (c.flags & TBN_EPI_BIAS_THEN_SCALE) != 0;
            const std::vector<float> b = c.bias ? host_floats(c.bias_name) : std::vector<float>(M, 0.0f);
            const std::vector<float> sc = c.scale ? channel_scales.at(c.scale_name) : std::vector<float>(M, 1.0f);
            std::vector<float> s2(M), b2(M);
            for (int64_t m = 0; m < M; ++m) {
                const double k = bn.bn_k[m], t = bn.bn_t[m], sm = sc[m], bm = b[m];
                s2[m] = static_cast<float>(sm * k);
                b2[m] = static_cast<float>((bts ? bm * sm * k : bm * k) + t);
            }
            if (c.kind == OpKind::ConvF32) {
                std::vector<float> w = host_floats(c.weight_name);
                const int64_t per = static_cast<int64_t>(w.size()) / M;
                for (int64_t m = 0; m < M; ++m)
                    for (int64_t j = 0; j < per; ++j)
                        w[m * per + j] = static_cast<float>(static_cast<double>(w[m * per + j]) * bn.bn_k[m]);
                c.w = derived_floats(c.node + "#bn_w", w);
            } else {
                c.scale = derived_floats(c.node + "#bn_s", s2);
                c.flags &= ~TBN_EPI_BIAS_THEN_SCALE;
            }
            c.bias = derived_floats(c.node + "#bn_b", b2);
            absorb(p, static_cast<int>(i));
        }
    }

    // For Add(conv_out, other) where `other` is produced after the conv but
    // from values that exist before it (a ResNet projection shortcut in
    // export order), move other's producer in front of the conv so the add
    // can be fused into the conv's epilogue.
    void hoist_residual_producers() {
        for (size_t a = 0; a < ops.size(); ++a) {
            if (ops[a].dead || ops[a].kind != OpKind::Add || ops[a].in.size() != 2) continue;
            for (int side = 0; side < 2; ++side) {
                const int i = producer(ops[a].in[side]);
                const int p = producer(ops[a].in[1 - side]);
                if (i < 0 || p < 0 || ops[i].kind != OpKind::ConvQuant || p < i || p > static_cast<int>(a)) continue;
                bool ready = true;
                for (int in : ops[p].in) {
                    const int q = producer(in);
                    if (q >= i) ready = false;
                }
                if (!ready) continue;
                Op moved = ops[p];
                ops.erase(ops.begin() + p);
                ops.insert(ops.begin() + i, moved);
                break;
            }
        }
    }

    void fuse() {
        fold_batchnorm();
        hoist_residual_producers();
        for (size_t i = 0; i < ops.size(); ++i) {
            Op& op = ops[i];
            if (op.dead) continue;
            const bool conv = op.kind == OpKind::ConvQuant || op.kind == OpKind::ConvF32 ||
                              op.kind == OpKind::ConvDepthwise;
            const bool gemm = op.kind == OpKind::GemmQuant || op.kind == OpKind::GemmF32;
            // residual Add (+Relu) into a quantized conv whose addend is ready
            if (((op.kind == OpKind::ConvQuant && op.groups == 1) || op.kind == OpKind::ConvDepthwise) &&
                !(op.flags & (TBN_EPI_RELU | TBN_EPI_MAXPOOL2X2))) {
                int r = sole_reader(op.out);
                if (r >= 0 && ops[r].kind == OpKind::Add) {
                    const int other = ops[r].in[0] == op.out ? ops[r].in[1] : ops[r].in[0];
                    const Value& ov = values[other];
                    const bool ready = ov.is_const || ov.is_input || producer(other) < static_cast<int>(i);
                    if (ops[r].in[0] != ops[r].in[1] && ov.shape == values[op.out].shape && ready &&
                        !ov.is_const) {
                        op.residual = other;
                        op.in.push_back(other);
                        absorb(static_cast<int>(i), r);
                    }
                }
            }
            // Relu into Conv / Gemm / Add
            if ((conv || gemm || op.kind == OpKind::Add || op.kind == OpKind::ChannelAffine) &&
                !(op.flags & TBN_EPI_MAXPOOL2X2)) {
                int r = sole_reader(op.out);
                if (r >= 0 && ops[r].kind == OpKind::Relu) {
                    op.flags |= TBN_EPI_RELU;
                    absorb(static_cast<int>(i), r);
                }
            }
            // 3x3/2 pad-1 floor MaxPool after the fp32 stem conv with its Relu
            // fused (the ResNet stem), when the library takes the shape
            if (op.kind == OpKind::ConvF32 && op.groups == 1 && op.residual < 0 && (op.flags & TBN_EPI_RELU) &&
                !(op.flags & TBN_EPI_MAXPOOL2X2)) {
                int r = sole_reader(op.out);
                if (r >= 0 && ops[r].kind == OpKind::MaxPool) {
                    const Pool2DParams& p = ops[r].pool;
                    if (p.kernel_h == 3 && p.kernel_w == 3 && p.stride_h == 2 && p.stride_w == 2 && p.pad_h == 1 &&
                        p.pad_w == 1 && p.dilation_h == 1 && p.dilation_w == 1 && !p.ceil_mode &&
                        tbn_hip_conv2d_f32_supported(&op.desc, op.flags | TBN_EPI_MAXPOOL3X3S2) == TBN_SUCCESS) {
                        op.flags |= TBN_EPI_MAXPOOL3X3S2;
                        absorb(static_cast<int>(i), r);
                    }
                }
            }
            // 2x2/2 floor MaxPool (with or without a Relu either side) into Conv;
            // a TBN conv fuses the pool only together with a Relu
            if (conv && op.residual < 0 && op.groups == 1 && op.kind != OpKind::ConvDepthwise) {
                int r = sole_reader(op.out);
                if (r >= 0 && ops[r].kind == OpKind::MaxPool) {
                    const Pool2DParams& p = ops[r].pool;
                    const Shape& s = values[op.out].shape;
                    int after = sole_reader(ops[r].out);
                    const bool relu_ok = !op.tbn || (op.flags & TBN_EPI_RELU) ||
                                         (after >= 0 && ops[after].kind == OpKind::Relu);
                    if (p.kernel_h == 2 && p.kernel_w == 2 && p.stride_h == 2 && p.stride_w == 2 && p.pad_h == 0 &&
                        p.pad_w == 0 && p.dilation_h == 1 && p.dilation_w == 1 && !p.ceil_mode && s.dims[2] >= 2 &&
                        s.dims[3] >= 2 && relu_ok) {
                        op.flags |= TBN_EPI_MAXPOOL2X2;
                        absorb(static_cast<int>(i), r);
                        int r2 = sole_reader(op.out);
                        if (r2 >= 0 && ops[r2].kind == OpKind::Relu && !(op.flags & TBN_EPI_RELU)) {
                            op.flags |= TBN_EPI_RELU;  // relu(max(x)) = max(relu(x))
                            absorb(static_cast<int>(i), r2);
                        }
                    }
                }
            }
        }
    }

    int producer(int v) const {
        for (size_t i = 0; i < ops.size(); ++i)
            if (!ops[i].dead && ops[i].out == v) return static_cast<int>(i);
        return -1;
    }

    // ---- fused projection pairs ---------------------------------------------------------

    int weights_kind(const Op& op) const {
        return op.pw->kind == PackedWeights::Kind::Binary ? TBN_WEIGHTS_BINARY : TBN_WEIGHTS_TERNARY;
    }

    // A prepacked quantized conv with a k x k kernel, pad (k - 1) / 2,
    // dilation 1, equal strides, one group, no pool, no run-time bias.
    bool pairable(const Op& op, int64_t k) const {
        const tbn_conv2d_desc& d = op.desc;
        const bool weights = op.tbn ? op.tbn_w != nullptr : (op.conv_w != nullptr && op.pw != nullptr);
        return !op.dead && !op.paired && op.kind == OpKind::ConvQuant && op.groups == 1 && weights &&
               op.bias_value < 0 && d.kh == k && d.kw == k && d.ph == (k - 1) / 2 && d.pw == (k - 1) / 2 &&
               d.dh == 1 && d.dw == 1 && d.sh == d.sw &&
               (op.flags & ~(TBN_EPI_RELU | TBN_EPI_BIAS_THEN_SCALE)) == 0;
    }

    // A ResNet downsampling block reads its input twice: the first 3x3 conv
    // (stride s, pad 1) and the 1x1 stride-s projection shortcut to the same
    // channel count.  When the library takes the pair
    // (tbn_hip_conv2d_f32_prepacked_pair, or tbn_hip_conv2d_tbn_prepacked_pair
    // in TBN arithmetic, mode 2) both run in the 3x3 conv's launch with the
    // bits of the two launches; the projection's output is then written at
    // the conv's position, which the memory plan takes as its definition.
    // Every reader of that output must come after the conv.
    void pair_projections() {
        for (size_t a = 0; a < ops.size(); ++a) {
            Op& conv = ops[a];
            if (!pairable(conv, 3)) continue;
            for (size_t p = 0; p < ops.size(); ++p) {
                Op& proj = ops[p];
                if (p == a || !pairable(proj, 1) || proj.residual >= 0 || proj.in[0] != conv.in[0] ||
                    proj.desc.m != conv.desc.m || proj.desc.sh != conv.desc.sh || proj.tbn != conv.tbn ||
                    (!conv.tbn && weights_kind(proj) != weights_kind(conv)))
                    continue;
                bool later = true;
                for (int r : readers(proj.out))
                    if (r <= static_cast<int>(a)) later = false;
                if (!later || is_output(proj.out)) continue;
                const int rc =
                    conv.tbn ? tbn_hip_conv2d_tbn_prepacked_pair(nullptr, &conv.desc, nullptr, nullptr, 1.0f, nullptr,
                                                                 nullptr, conv.flags, -0.1f, 0.1f, nullptr, nullptr,
                                                                 nullptr, 1.0f, nullptr, proj.flags, nullptr, 2, nullptr)
                             : tbn_hip_conv2d_f32_prepacked_pair(weights_kind(conv), nullptr, &conv.desc, nullptr,
                                                                 nullptr, 1.0f, nullptr, nullptr, conv.flags, nullptr,
                                                                 nullptr, nullptr, 1.0f, nullptr, proj.flags, nullptr,
                                                                 2, nullptr);
                if (rc != TBN_SUCCESS) {
                    (void)tbn_hip_last_error();  // not taken: the two convs run apart
                    continue;
                }
                conv.pair = static_cast<int>(p);
                proj.paired = true;
                break;
            }
        }
    }

    // ---- memory planning -------------------------------------------------------------

    int root(int v) const {
        while (values[v].view_of >= 0) v = values[v].view_of;
        return v;
    }

    void plan_memory() {
        const int nops = static_cast<int>(ops.size());
        for (auto& v : values) { v.def = -1; v.last = -1; v.offset = -1; }
        for (int i = 0; i < nops; ++i) {
            if (ops[i].dead) continue;
            const int o = root(ops[i].out);
            if (values[o].def < 0) values[o].def = i;
            values[o].last = std::max(values[o].last, i);
            for (int in : ops[i].in) values[root(in)].last = std::max(values[root(in)].last, i);
            if (ops[i].workspace >= 0) {
                values[ops[i].workspace].def = i;
                values[ops[i].workspace].last = i;
            }
        }
        // a paired projection's output is written in its conv's launch
        for (int i = 0; i < nops; ++i)
            if (!ops[i].dead && ops[i].pair >= 0) {
                Value& v = values[root(ops[ops[i].pair].out)];
                v.def = std::min(v.def, i);
            }
        for (const auto& name : graph->outputs) {
            auto it = value_id.find(name);
            TBN_CHECK(it != value_id.end(), RuntimeError, "Output '" + name + "' was not produced");
            values[root(it->second)].last = nops;  // live until the next run
        }
        for (auto& v : values)
            if (v.is_input) { v.def = -1; v.last = std::max(v.last, 0); }
        // greedy placement, largest first
        std::vector<int> order;
        for (size_t i = 0; i < values.size(); ++i) {
            const Value& v = values[i];
            if (v.is_const || v.view_of >= 0) continue;
            if (!v.is_input && v.def < 0) continue;  // never produced (dead)
            order.push_back(static_cast<int>(i));
        }
        auto bytes = [&](int i) { return round_up(values[i].shape.size() * element_size(values[i].dtype), 256); };
        std::sort(order.begin(), order.end(), [&](int a, int b) { return bytes(a) > bytes(b); });
        std::vector<int> placed;
        size_t total = 0;
        for (int i : order) {
            const size_t sz = std::max<size_t>(bytes(i), 256);
            const int d0 = values[i].def, d1 = values[i].last;
            std::vector<std::pair<size_t, size_t>> busy;
            for (int j : placed) {
                const int e0 = values[j].def, e1 = values[j].last;
                if (d0 <= e1 && e0 <= d1) busy.push_back({static_cast<size_t>(values[j].offset),
                                                          static_cast<size_t>(values[j].offset) + std::max<size_t>(bytes(j), 256)});
            }
            std::sort(busy.begin(), busy.end());
            size_t off = 0;
            for (auto& b : busy) {
                if (off + sz <= b.first) break;
                off = std::max(off, b.second);
            }
            values[i].offset = static_cast<int64_t>(off);
            total = std::max(total, off + sz);
            placed.push_back(i);
        }
        arena = Tensor::empty({static_cast<int64_t>(std::max<size_t>(total, 256))}, DataType::UINT8, DeviceType::HIP);
    }

    void* ptr(int v) {
        const Value& val = values[v];
        if (val.is_const) return const_cast<void*>(val.const_ptr);
        const int r = root(v);
        if (values[r].is_const) return const_cast<void*>(values[r].const_ptr);
        if (values[r].bound) return values[r].bound;
        return static_cast<uint8_t*>(arena.data()) + values[r].offset;
    }
    float* fp(int v) { return static_cast<float*>(ptr(v)); }

    void compile() {
        drop_graph();
        eager_runs = 0;
        replay_off = false;
        values.clear();
        value_id.clear();
        ops.clear();
        arena = Tensor();
        for (const auto& name : graph->inputs) {
            if (graph->initializers.count(name)) continue;
            auto it = inputs.find(name);
            TBN_CHECK(it != inputs.end(), InvalidArgumentError, "Input '" + name + "' not set");
            int id = new_value(name, it->second.shape(), it->second.dtype());
            values[id].is_input = true;
        }
        for (const auto& node : graph->nodes) lower(node);
        fuse();
        pair_projections();
        plan_memory();
        tune_convs();
        launches = 0;
        for (const auto& op : ops)
            if (!op.dead && !op.paired && op.kind != OpKind::View)
                launches += op.groups > 1 && op.kind != OpKind::ConvDepthwise ? op.groups * (op.desc.n == 1 ? 1 : 3) : 1;
        planned = true;
        plan_quant = quant;
        plan_arith = arith;
        plan_shapes.clear();
        for (auto& kv : inputs) plan_shapes[kv.first] = kv.second.shape();
    }

    // Times the conv tiles of every patch conv once per geometry (the library
    // keeps the winner for the process), so no run times, allocates or waits
    // for tile selection.  Skipped while the caller's stream captures: those
    // convs then use the library's static tile rule.
    void tune_convs() {
        const tbn_stream_t s = cur_stream();
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(static_cast<hipStream_t>(s), &st) != hipSuccess ||
            st != hipStreamCaptureStatusNone)
            return;
        for (auto& op : ops) {
            if (op.dead || op.paired || op.kind != OpKind::ConvQuant || op.groups > 1 || !op.conv_w) continue;
            if (op.pair >= 0) {
                const Op& pr = ops[op.pair];
                check_status(tbn_hip_conv2d_f32_prepacked_pair(
                                 weights_kind(op), fp(op.in[0]), &op.desc, op.conv_w->typed_data<uint8_t>(), op.scale,
                                 1.0f, bias_of(op), op.residual >= 0 ? fp(op.residual) : nullptr, op.flags, fp(op.out),
                                 pr.conv_w->typed_data<uint8_t>(), pr.scale, 1.0f, bias_of(pr), pr.flags, fp(pr.out),
                                 1, s),
                             ("tuning node '" + op.node + "' with '" + pr.node + "'").c_str());
                continue;
            }
            check_status(tbn_hip_conv2d_tune_prepacked(
                             op.pw->kind == PackedWeights::Kind::Binary ? TBN_WEIGHTS_BINARY : TBN_WEIGHTS_TERNARY,
                             fp(op.in[0]), &op.desc, op.conv_w->typed_data<uint8_t>(), op.scale, 1.0f, bias_of(op),
                             op.residual >= 0 ? fp(op.residual) : nullptr, op.flags, fp(op.out), s),
                         ("tuning node '" + op.node + "'").c_str());
        }
    }

    bool plan_valid() const {
        if (!planned || plan_quant != quant || plan_arith != arith) return false;
        if (plan_shapes.size() != inputs.size()) return false;
        for (auto& kv : inputs) {
            auto it = plan_shapes.find(kv.first);
            if (it == plan_shapes.end() || it->second != kv.second.shape()) return false;
        }
        return true;
    }

    // ---- execution ---------------------------------------------------------------------

    const float* bias_of(const Op& op) { return op.bias ? op.bias : (op.bias_value >= 0 ? fp(op.bias_value) : nullptr); }

    // A grouped conv with more than one input channel per group: one dense
    // conv per group on channel slices of the input and output.
    void launch_grouped(Op& op, tbn_stream_t s, const std::string& what) {
        const int64_t G = op.groups, Mg = op.desc.m / G;
        const int64_t w_per_group = Mg * (op.desc.c / G) * op.desc.kh * op.desc.kw;
        const bool ternary = op.pw && op.pw->kind == PackedWeights::Kind::Ternary;
        const int wkind = ternary ? TBN_WEIGHTS_TERNARY : TBN_WEIGHTS_BINARY;
        detail::run_grouped_conv(
            op.desc, G, fp(op.in[0]), fp(op.out), op.workspace >= 0 ? fp(op.workspace) : nullptr,
            [&](int64_t g, const float* xg, const tbn_conv2d_desc& dg, float* yg) {
                const float* sc = op.scale ? op.scale + g * Mg : nullptr;
                const float* bi = bias_of(op) ? bias_of(op) + g * Mg : nullptr;
                if (op.kind == OpKind::ConvF32) {
                    check_status(tbn_hip_conv2d_f32(xg, &dg, op.w + g * w_per_group, bi, op.flags, yg, s), what.c_str());
                } else if (!op.group_conv_w.empty()) {
                    check_status(tbn_hip_conv2d_f32_prepacked(wkind, xg, &dg, op.group_conv_w[g]->typed_data<uint8_t>(),
                                                              sc, 1.0f, bi, nullptr, op.flags, yg, s),
                                 what.c_str());
                } else {
                    const int64_t col_bytes = ternary ? op.pw->K_pad / 4 : op.pw->K_pad / 8;
                    check_status(tbn_hip_conv2d_f32_quantized(wkind, xg, &dg,
                                                              op.pw->bits.typed_data<uint8_t>() + g * Mg * col_bytes,
                                                              op.pw->K_pad, op.pw->N_pad - g * Mg, sc, 1.0f, bi,
                                                              nullptr, op.flags, yg, s),
                                 what.c_str());
                }
            },
            s);
    }

    void launch(Op& op, tbn_stream_t s) {
        const std::string what = "node '" + op.node + "'";
        switch (op.kind) {
            case OpKind::View:
                return;
            case OpKind::ConvF32:
                if (op.groups > 1) return launch_grouped(op, s, what);
                check_status(tbn_hip_conv2d_f32(fp(op.in[0]), &op.desc, op.w, bias_of(op), op.flags, fp(op.out), s),
                             what.c_str());
                return;
            case OpKind::ConvDepthwise:
                check_status(tbn_hip_conv2d_depthwise(fp(op.in[0]), &op.desc, op.w, op.scale, 1.0f, bias_of(op),
                                                      op.residual >= 0 ? fp(op.residual) : nullptr, op.flags,
                                                      fp(op.out), s),
                             what.c_str());
                return;
            case OpKind::ChannelAffine:
                check_status(tbn_hip_channel_affine(fp(op.in[0]), op.outer, op.inner, op.rest, op.scale, op.bias,
                                                    op.flags, fp(op.out), s),
                             what.c_str());
                return;
            case OpKind::ConvQuant:
                if (op.groups > 1) return launch_grouped(op, s, what);
                if (op.tbn && op.paired) return;  // written by its pair's launch
                if (op.tbn && op.pair >= 0) {
                    const Op& pr = ops[op.pair];
                    check_status(tbn_hip_conv2d_tbn_prepacked_pair(
                                     fp(op.in[0]), &op.desc, op.tbn_w->typed_data<uint8_t>(), op.scale, 1.0f,
                                     bias_of(op), op.residual >= 0 ? fp(op.residual) : nullptr, op.flags, -0.1f, 0.1f,
                                     fp(op.out), pr.tbn_w->typed_data<uint8_t>(), pr.scale, 1.0f, bias_of(pr),
                                     pr.flags, fp(pr.out), 0, s),
                                 (what + " with '" + pr.node + "'").c_str());
                    return;
                }
                if (op.tbn) {
                    check_status(tbn_hip_conv2d_tbn_prepacked(fp(op.in[0]), &op.desc, op.tbn_w->typed_data<uint8_t>(),
                                                              op.scale, 1.0f, bias_of(op),
                                                              op.residual >= 0 ? fp(op.residual) : nullptr, op.flags,
                                                              -0.1f, 0.1f,
                                                              op.workspace >= 0
                                                                  ? static_cast<uint8_t*>(ptr(op.workspace))
                                                                  : nullptr,
                                                              fp(op.out), s),
                                 what.c_str());
                    return;
                }
                if (op.paired) return;  // written by its pair's launch
                if (op.pair >= 0) {
                    const Op& pr = ops[op.pair];
                    check_status(tbn_hip_conv2d_f32_prepacked_pair(
                                     weights_kind(op), fp(op.in[0]), &op.desc, op.conv_w->typed_data<uint8_t>(),
                                     op.scale, 1.0f, bias_of(op), op.residual >= 0 ? fp(op.residual) : nullptr,
                                     op.flags, fp(op.out), pr.conv_w->typed_data<uint8_t>(), pr.scale, 1.0f,
                                     bias_of(pr), pr.flags, fp(pr.out), 0, s),
                                 (what + " with '" + pr.node + "'").c_str());
                    return;
                }
                if (op.conv_w) {
                    check_status(tbn_hip_conv2d_f32_prepacked(
                                     op.pw->kind == PackedWeights::Kind::Binary ? TBN_WEIGHTS_BINARY
                                                                                : TBN_WEIGHTS_TERNARY,
                                     fp(op.in[0]), &op.desc, op.conv_w->typed_data<uint8_t>(), op.scale, 1.0f,
                                     bias_of(op), op.residual >= 0 ? fp(op.residual) : nullptr, op.flags, fp(op.out),
                                     s),
                                 what.c_str());
                    return;
                }
                check_status(tbn_hip_conv2d_f32_quantized(
                                 op.pw->kind == PackedWeights::Kind::Binary ? TBN_WEIGHTS_BINARY : TBN_WEIGHTS_TERNARY,
                                 fp(op.in[0]), &op.desc, op.pw->bits.typed_data<uint8_t>(), op.pw->K_pad,
                                 op.pw->N_pad, op.scale, 1.0f, bias_of(op), op.residual >= 0 ? fp(op.residual) : nullptr,
                                 op.flags, fp(op.out), s),
                             what.c_str());
                return;
            case OpKind::GemmQuant: {
                if (op.dyn_b >= 0)
                    check_status(tbn_hip_quantize_pack_binary_f32(fp(op.dyn_b), op.K, op.N, TBN_LAYOUT_KN,
                                                                  TBN_SIGN_GEMM_SAMPLED, 0.0f, op.pw->K_pad,
                                                                  op.pw->N_pad,
                                                                  const_cast<uint8_t*>(op.pw->bits.typed_data<uint8_t>()),
                                                                  s),
                                 what.c_str());
                const float* cin = op.cin ? op.cin : (op.cin_value >= 0 ? fp(op.cin_value) : nullptr);
                if (op.tbn) {
                    uint8_t* w4 = const_cast<uint8_t*>(op.tbn_w->typed_data<uint8_t>());
                    if (op.dyn_b >= 0)
                        check_status(tbn_hip_pack_f4_weights(op.pw->bits.typed_data<uint8_t>(), op.pw->K_pad,
                                                             op.pw->N_pad, w4, s),
                                     what.c_str());
                    check_status(tbn_hip_gemm_tbn_prepacked(fp(op.in[0]), op.K, op.M, op.K, w4, op.pw->K_pad, op.N,
                                                            op.pw->N_pad, op.alpha, cin, op.cin_1d, op.beta, -0.1f,
                                                            0.1f, op.flags, static_cast<uint8_t*>(ptr(op.workspace)),
                                                            fp(op.out), op.N, s),
                                 what.c_str());
                    return;
                }
                check_status(tbn_hip_gemm_f32_quantized(
                                 op.pw->kind == PackedWeights::Kind::Binary ? TBN_WEIGHTS_BINARY : TBN_WEIGHTS_TERNARY,
                                 fp(op.in[0]), op.K, op.M, op.N, op.K, op.pw->bits.typed_data<uint8_t>(),
                                 op.pw->K_pad, op.pw->N_pad, nullptr, op.alpha, nullptr, cin, op.cin_1d, op.beta,
                                 op.flags, fp(op.out), op.N, s),
                             what.c_str());
                return;
            }
            case OpKind::GemmF32: {
                const float* cin = op.cin ? op.cin : (op.cin_value >= 0 ? fp(op.cin_value) : nullptr);
                check_status(tbn_hip_gemm_f32(fp(op.in[0]), op.bt ? op.bt : fp(op.in[1]), cin, op.cin_1d, op.M, op.K,
                                              op.N, op.alpha, cin ? op.beta : 0.0f, op.transA, op.bt ? 1 : op.transB,
                                              op.flags, fp(op.out), s),
                             what.c_str());
                return;
            }
            case OpKind::Add:
                check_status(tbn_hip_add(fp(op.in[0]), fp(op.in[1]), op.outer, op.inner, op.rest, 1, op.flags,
                                         fp(op.out), s),
                             what.c_str());
                return;
            case OpKind::Relu:
                check_status(tbn_hip_relu(fp(op.in[0]), values[op.out].shape.size(), fp(op.out), s), what.c_str());
                return;
            case OpKind::TernaryAct:
                check_status(tbn_hip_ternary_activation(fp(op.in[0]), values[op.out].shape.size(), op.scalar,
                                                        fp(op.out), s),
                             what.c_str());
                return;
            case OpKind::MaxPool: {
                const auto& d = values[op.in[0]].shape.dims;
                const Pool2DParams& p = op.pool;
                check_status(tbn_hip_maxpool2d(fp(op.in[0]), d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w,
                                               p.stride_h, p.stride_w, p.pad_h, p.pad_w, 1, 1, p.ceil_mode,
                                               fp(op.out), nullptr, s),
                             what.c_str());
                return;
            }
            case OpKind::AvgPool: {
                const auto& d = values[op.in[0]].shape.dims;
                const Pool2DParams& p = op.pool;
                check_status(tbn_hip_avgpool2d(fp(op.in[0]), d[0], d[1], d[2], d[3], p.kernel_h, p.kernel_w,
                                               p.stride_h, p.stride_w, p.pad_h, p.pad_w, 1, 1, 0,
                                               p.count_include_pad, fp(op.out), nullptr, s),
                             what.c_str());
                return;
            }
            case OpKind::GlobalAvgPool: {
                const auto& d = values[op.in[0]].shape.dims;
                check_status(tbn_hip_global_avgpool2d(fp(op.in[0]), d[0], d[1], d[2], d[3], fp(op.out), s),
                             what.c_str());
                return;
            }
            case OpKind::GlobalMaxPool: {
                const auto& d = values[op.in[0]].shape.dims;
                check_status(tbn_hip_global_maxpool2d(fp(op.in[0]), d[0], d[1], d[2], d[3], fp(op.out), s),
                             what.c_str());
                return;
            }
            case OpKind::Elementwise: {
                const float* rhs = op.rhs_const ? op.rhs_const : (op.rhs_value >= 0 ? fp(op.rhs_value) : nullptr);
                check_status(tbn_hip_elementwise(op.elem_op, fp(op.in[0]), values[op.out].shape.size(), rhs,
                                                 op.rhs_n, op.scalar, fp(op.out), s),
                             what.c_str());
                return;
            }
        }
    }

    // A device input of the planned dtype, 256-byte aligned like the arena,
    // that no graph output shares storage with is read in place by the ops
    // (no copy); the others are copied into the arena.  No op writes to its
    // inputs' storage (each op's output is placed apart from its live
    // inputs), so the caller's tensor is only read.  Returns whether any
    // binding changed since the last call.
    bool bind_inputs() {
        bool changed = false;
        for (auto& kv : inputs) {
            Value& v = values[root(value_id.at(kv.first))];
            const Tensor& t = kv.second;
            void* want = nullptr;
            if (t.on_device() && t.dtype() == v.dtype && t.data_size() == v.shape.size() * element_size(v.dtype) &&
                reinterpret_cast<uintptr_t>(t.data()) % 256 == 0) {
                want = const_cast<void*>(t.data());
                for (const auto& name : graph->outputs) {
                    auto it = value_id.find(name);
                    if (it != value_id.end() && &values[root(it->second)] == &v) want = nullptr;
                }
            }
            if (v.bound != want) changed = true;
            v.bound = want;
        }
        return changed;
    }

    void upload_inputs(tbn_stream_t s) {
        for (auto& kv : inputs) {
            const int id = value_id.at(kv.first);
            const Tensor& t = kv.second;
            if (values[root(id)].bound) continue;
            const Value& v = values[root(id)];
            TBN_CHECK(t.dtype() == v.dtype && t.data_size() == v.shape.size() * element_size(v.dtype),
                      InvalidArgumentError, "Input '" + kv.first + "' has the wrong data type");
            if (t.on_device()) {
                if (hipMemcpyAsync(ptr(id), t.data(), t.data_size(), hipMemcpyDeviceToDevice,
                                   static_cast<hipStream_t>(s)) != hipSuccess)
                    throw RuntimeError("input copy failed for '" + kv.first + "'");
            } else {
                if (hipMemcpyAsync(ptr(id), t.data(), t.data_size(), hipMemcpyHostToDevice,
                                   static_cast<hipStream_t>(s)) != hipSuccess)
                    throw RuntimeError("input upload failed for '" + kv.first + "'");
                if (hipStreamSynchronize(static_cast<hipStream_t>(s)) != hipSuccess)
                    throw RuntimeError("input upload failed for '" + kv.first + "'");
            }
        }
    }

    void run_ops(tbn_stream_t s) {
        for (auto& op : ops)
            if (!op.dead) launch(op, s);
    }

    void run() {
        size_t user_inputs = 0;
        for (const auto& name : graph->inputs)
            if (!graph->initializers.count(name)) ++user_inputs;
        TBN_CHECK(inputs.size() == user_inputs, InvalidArgumentError,
                  "Not all inputs provided (expected " + std::to_string(user_inputs) + ", got " +
                      std::to_string(inputs.size()) + ")");
        if (!plan_valid()) compile();
        tbn_stream_t s = cur_stream();
        // a replayed graph holds the input addresses it was recorded with
        if (bind_inputs()) drop_graph();
        if (!graph_replay) {
            upload_inputs(s);
            run_ops(s);
            return;
        }
        // HIP graph replay: the first run is eager (warms every cache), the
        // second records the ops, later runs replay them.  The caller's
        // stream is used directly; the null stream cannot be captured, so
        // with it the ops run on a private stream ordered after it by events.
        hipStream_t cs = static_cast<hipStream_t>(s);
        const bool own = cs == nullptr;
        if (own && !replay_stream) {
            if (hipStreamCreate(&replay_stream) != hipSuccess) throw RuntimeError("hipStreamCreate failed");
        }
        hipStream_t rs = own ? replay_stream : cs;
        hipEvent_t ev = nullptr;
        if (own) {
            if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
                throw RuntimeError("hipEventCreate failed");
            (void)hipEventRecord(ev, cs);
            (void)hipStreamWaitEvent(rs, ev, 0);
        }
        upload_inputs(rs);
        if (eager_runs < 1 || replay_off) {
            run_ops(rs);
            ++eager_runs;
        } else {
            if (!hip_graph_exec) {
                if (hipStreamBeginCapture(rs, hipStreamCaptureModeThreadLocal) != hipSuccess)
                    throw RuntimeError("hipStreamBeginCapture failed");
                bool refused = false;
                try {
                    run_ops(rs);
                } catch (const NotImplementedError&) {
                    // an op needs a split-K workspace, which is never
                    // allocated under capture: this plan runs eagerly
                    refused = true;
                } catch (...) {
                    hipGraph_t g = nullptr;
                    (void)hipStreamEndCapture(rs, &g);
                    if (g) (void)hipGraphDestroy(g);
                    throw;
                }
                if (refused) {
                    hipGraph_t g = nullptr;
                    (void)hipStreamEndCapture(rs, &g);
                    if (g) (void)hipGraphDestroy(g);
                    (void)hipGetLastError();
                    replay_off = true;
                    run_ops(rs);
                    ++eager_runs;
                    goto done;
                }
                if (hipStreamEndCapture(rs, &hip_graph) != hipSuccess) throw RuntimeError("hipStreamEndCapture failed");
                if (hipGraphInstantiate(&hip_graph_exec, hip_graph, nullptr, nullptr, 0) != hipSuccess)
                    throw RuntimeError("hipGraphInstantiate failed");
            }
            if (hipGraphLaunch(hip_graph_exec, rs) != hipSuccess) throw RuntimeError("hipGraphLaunch failed");
        }
    done:
        if (own) {
            // the null stream continues after the replay
            (void)hipEventRecord(ev, rs);
            (void)hipStreamWaitEvent(cs, ev, 0);
            (void)hipEventDestroy(ev);
        }
    }

    Tensor output_device(const std::string& name) {
        TBN_CHECK(planned, InvalidArgumentError, "Output '" + name + "' not available");
        TBN_CHECK(std::find(graph->outputs.begin(), graph->outputs.end(), name) != graph->outputs.end(),
                  InvalidArgumentError, "Output '" + name + "' not available");
        auto it = value_id.find(name);
        TBN_CHECK(it != value_id.end(), RuntimeError, "Output '" + name + "' was not produced");
        const Value& v = values[it->second];
        Tensor view = Tensor::wrap(v.shape, v.dtype, ptr(it->second), DeviceType::HIP);
        return view;
    }

    size_t bytes_held() const {
        size_t b = arena.data_size();
        for (auto& kv : dev_init) b += kv.second.data_size();
        for (auto& kv : packed) b += kv.second.bits.data_size();
        for (auto& kv : conv_packed) b += kv.second.data_size();
        for (auto& kv : tbn_packed) b += kv.second.data_size();
        for (auto& kv : dev_scales) b += kv.second.data_size();
        return b;
    }
};

// ===========================================================================
// Session public interface
// ===========================================================================

TBNModel::Session::Session(std::shared_ptr<ModelGraph> graph, TilingParams tiling) : impl_(new Impl()) {
    TBN_CHECK(graph != nullptr, InvalidArgumentError, "graph is null");
    impl_->graph = std::move(graph);
    impl_->tiling = tiling;
}

TBNModel::Session::~Session() = default;
TBNModel::Session::Session(Session&&) noexcept = default;
TBNModel::Session& TBNModel::Session::operator=(Session&&) noexcept = default;

void TBNModel::Session::set_quantization(bool enable) { impl_->quant = enable; }
bool TBNModel::Session::is_quantization_enabled() const { return impl_->quant; }
void TBNModel::Session::set_quant_arithmetic(QuantArithmetic a) { impl_->arith = a; }
QuantArithmetic TBNModel::Session::quant_arithmetic() const { return impl_->arith; }
void TBNModel::Session::set_tiling(const TilingParams& p) { impl_->tiling = p; }
const TilingParams& TBNModel::Session::get_tiling() const { return impl_->tiling; }

void TBNModel::Session::set_input(const std::string& name, const Tensor& tensor) {
    const auto& vi = impl_->graph->value_info;
    TBN_CHECK(vi.count(name) > 0, InvalidArgumentError, "Input '" + name + "' not found in model");
    TBN_CHECK(tensor.shape() == vi.at(name), InvalidShapeError, "Input shape mismatch for '" + name + "'");
    impl_->inputs[name] = tensor;
}

Tensor TBNModel::Session::get_input(const std::string& name) const {
    auto it = impl_->inputs.find(name);
    TBN_CHECK(it != impl_->inputs.end(), InvalidArgumentError, "Input '" + name + "' not set");
    return it->second;
}

void TBNModel::Session::run() { impl_->run(); }

Tensor TBNModel::Session::get_output(const std::string& name) const {
    return impl_->output_device(name).to_device(DeviceType::CPU);
}

Tensor TBNModel::Session::get_output_device(const std::string& name) const { return impl_->output_device(name); }

void TBNModel::Session::set_graph_replay(bool enable) {
    if (enable == impl_->graph_replay) return;
    impl_->graph_replay = enable;
    impl_->drop_graph();
    impl_->eager_runs = 0;
}

void TBNModel::Session::synchronize() const { device::synchronize(); }
size_t TBNModel::Session::planned_launches() const { return impl_->planned ? impl_->launches : 0; }
size_t TBNModel::Session::device_bytes() const { return impl_->bytes_held(); }

// ===========================================================================
// InferenceSession
// ===========================================================================

InferenceSession::InferenceSession(std::shared_ptr<TBNModel> model, const Options& options)
    : model_(std::move(model)), options_(options) {}

void InferenceSession::initialize() {
    TBN_CHECK(model_ != nullptr, InvalidArgumentError, "Model is null");
    model_->validate();
    session_ = std::make_unique<TBNModel::Session>(model_->create_session());
    session_->set_quantization(options_.use_quantization);
    initialized_ = true;
}

void InferenceSession::set_input(const std::string& name, const Tensor& tensor) {
    TBN_CHECK(initialized_, RuntimeError, "Session not initialized");
    TBN_CHECK(model_->has_input(name), InvalidArgumentError, "Input '" + name + "' not found in model");
    TBN_CHECK(tensor.shape() == model_->get_input_shape(name), InvalidShapeError,
              "Input shape mismatch for '" + name + "'");
    inputs_[name] = tensor;
}

Tensor InferenceSession::get_input(const std::string& name) const {
    auto it = inputs_.find(name);
    TBN_CHECK(it != inputs_.end(), InvalidArgumentError, "Input '" + name + "' not set");
    return it->second;
}

void InferenceSession::run() {
    TBN_CHECK(initialized_, RuntimeError, "Session not initialized");
    TBN_CHECK(inputs_.size() == model_->inputs().size(), InvalidArgumentError, "Not all inputs provided");
    const auto t0 = std::chrono::high_resolution_clock::now();
    for (const auto& kv : inputs_) session_->set_input(kv.first, kv.second);
    session_->run();
    outputs_.clear();
    for (const auto& name : model_->outputs()) outputs_[name] = session_->get_output(name);
    const auto t1 = std::chrono::high_resolution_clock::now();
    last_run_us_ = std::chrono::duration<double, std::micro>(t1 - t0).count();
    if (options_.enable_profiling)
        std::fprintf(stderr, "[tbn] Inference completed in %.1f us\n", last_run_us_);
}

Tensor InferenceSession::get_output(const std::string& name) const {
    auto it = outputs_.find(name);
    TBN_CHECK(it != outputs_.end(), InvalidArgumentError, "Output '" + name + "' not available");
    return it->second;
}

std::unique_ptr<InferenceSession> create_inference_session(std::shared_ptr<TBNModel> model,
                                                           const InferenceSession::Options& options) {
    auto s = std::make_unique<InferenceSession>(std::move(model), options);
    s->initialize();
    return s;
}

}  // namespace tbn
