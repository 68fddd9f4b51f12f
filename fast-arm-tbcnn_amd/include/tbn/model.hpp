// Graph model and device-resident Session of the tbn runtime.
//
// ModelNode / ModelGraph / AttributeValue / TBNModel keep the reference's
// shape (tbn-runtime/include/tbn/runtime/model.hpp:21-35,37-121,1318-1320;
// attribute.hpp:12-70).  TBNModel::Session keeps its interface
// (model.hpp:121-235: set_quantization, set_tiling, set_input, run,
// get_output) but executes differently: the first run() compiles the graph
// into a plan for the given input shapes -- weights uploaded, quantized and
// packed once, every activation given a slot in one device arena reused by
// liveness, Conv/Gemm/Add fused with a following Relu and Conv with a
// following 2x2 MaxPool -- and every run() then queues that plan on the
// current stream with no host round trip between ops.  Only set_input (host
// tensors are uploaded) and get_output (copied back) cross PCIe.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

#include "operators.hpp"
#include "tensor.hpp"

namespace tbn {

struct AttributeValue {
    using Value = std::variant<int64_t, float, std::string, Tensor, std::vector<int64_t>,
                               std::vector<float>, std::vector<std::string>>;
    Value value;

    AttributeValue() : value(int64_t(0)) {}
    AttributeValue(int64_t v) : value(v) {}
    AttributeValue(int v) : value(static_cast<int64_t>(v)) {}
    AttributeValue(float v) : value(v) {}
    AttributeValue(double v) : value(static_cast<float>(v)) {}
    AttributeValue(const std::string& v) : value(v) {}
    AttributeValue(const char* v) : value(std::string(v)) {}
    AttributeValue(const Tensor& v) : value(v) {}
    AttributeValue(const std::vector<int64_t>& v) : value(v) {}
    AttributeValue(const std::vector<float>& v) : value(v) {}
    AttributeValue(const std::vector<std::string>& v) : value(v) {}

    bool is_int() const { return std::holds_alternative<int64_t>(value); }
    bool is_float() const { return std::holds_alternative<float>(value); }
    bool is_string() const { return std::holds_alternative<std::string>(value); }
    bool is_tensor() const { return std::holds_alternative<Tensor>(value); }
    bool is_ints() const { return std::holds_alternative<std::vector<int64_t>>(value); }
    bool is_floats() const { return std::holds_alternative<std::vector<float>>(value); }
    bool is_strings() const { return std::holds_alternative<std::vector<std::string>>(value); }

    int64_t as_int() const { return std::get<int64_t>(value); }
    float as_float() const { return std::get<float>(value); }
    const std::string& as_string() const { return std::get<std::string>(value); }
    const Tensor& as_tensor() const { return std::get<Tensor>(value); }
    const std::vector<int64_t>& as_ints() const { return std::get<std::vector<int64_t>>(value); }
    const std::vector<float>& as_floats() const { return std::get<std::vector<float>>(value); }
    const std::vector<std::string>& as_strings() const { return std::get<std::vector<std::string>>(value); }

    int64_t as_int_or(int64_t d) const { return is_int() ? as_int() : d; }
    float as_float_or(float d) const { return is_float() ? as_float() : d; }
};

using NodeAttributes = std::unordered_map<std::string, AttributeValue>;

struct ModelNode {
    std::string name;
    std::string op_type;
    std::vector<std::string> inputs;
    std::vector<std::string> outputs;
    NodeAttributes attributes;
};

struct ModelGraph {
    std::vector<ModelNode> nodes;
    std::unordered_map<std::string, Tensor> initializers;
    std::unordered_map<std::string, Shape> value_info;
    std::vector<std::string> inputs;
    std::vector<std::string> outputs;
};

// Arithmetic of the quantized layers of a Session (the reference's
// conv2d_binary / conv2d_ternary convs, and with quantization enabled its
// auto-quantized convs and Gemms).
//   F32: fp32 activations times exact +-1 (times the per-channel scale where
//        the reference applies one), fp32 accumulation -- the float x binary
//        product (the default).
//   TBN: the reference's own arithmetic, bit for bit: activations ternarized
//        at +-0.1, integer products with the +-1 weights, float(C) then the
//        reference's bias / scale / alpha / beta steps (model.hpp:414-564,
//        763-870; conv2d.cpp:195-316).  Grouped and depthwise convs, which
//        the reference cannot run, keep F32.
enum class QuantArithmetic { F32, TBN };

class TBNModel {
public:
    TBNModel();
    explicit TBNModel(std::shared_ptr<ModelGraph> graph);

    const ModelGraph& graph() const { return *graph_; }
    ModelGraph& graph() { return *graph_; }
    std::shared_ptr<ModelGraph> graph_ptr() const { return graph_; }

    void set_producer(const std::string& name, const std::string& version) {
        producer_name_ = name;
        producer_version_ = version;
    }
    const std::string& producer_name() const { return producer_name_; }
    const std::string& producer_version() const { return producer_version_; }

    const std::vector<std::string>& inputs() const { return graph_->inputs; }
    const std::vector<std::string>& outputs() const { return graph_->outputs; }
    bool has_input(const std::string& name) const;
    bool has_output(const std::string& name) const;
    const Shape& get_input_shape(const std::string& name) const;
    const Shape& get_output_shape(const std::string& name) const;
    // model.hpp:88-121: inputs/outputs/nodes present, every name has a shape.
    void validate() const;

    class Session {
    public:
        Session(std::shared_ptr<ModelGraph> graph,
                TilingParams tiling = TilingParams::default_128x128());
        ~Session();
        Session(Session&&) noexcept;
        Session& operator=(Session&&) noexcept;
        Session(const Session&) = delete;
        Session& operator=(const Session&) = delete;

        void set_quantization(bool enable);
        bool is_quantization_enabled() const;
        // The arithmetic of the quantized layers (F32 by default).
        void set_quant_arithmetic(QuantArithmetic a);
        QuantArithmetic quant_arithmetic() const;
        void set_tiling(const TilingParams& p);
        const TilingParams& get_tiling() const;

        // Host or HIP tensor of the declared shape (model.hpp:176-182).
        void set_input(const std::string& name, const Tensor& tensor);
        Tensor get_input(const std::string& name) const;
        // Queues the whole graph on the current stream (model.hpp:190-228).
        void run();
        // Host copy of an output (waits for the device).
        Tensor get_output(const std::string& name) const;
        // The output's device tensor (valid until the next run(); no copy, no wait).
        Tensor get_output_device(const std::string& name) const;

        // Records the plan into a HIP graph on first use and replays it on
        // every run() (launch-bound graphs such as LeNet).  Needs a non-null
        // current stream.
        void set_graph_replay(bool enable);
        // Waits for the current stream.
        void synchronize() const;
        // Number of kernel launches per run() in the compiled plan (0 before run()).
        size_t planned_launches() const;
        // Device bytes held: packed/uploaded weights and the activation arena.
        size_t device_bytes() const;

    private:
        struct Impl;
        std::unique_ptr<Impl> impl_;
    };

    Session create_session(TilingParams tiling = TilingParams::default_128x128()) {
        return Session(graph_, tiling);
    }

private:
    std::shared_ptr<ModelGraph> graph_;
    std::string model_path_;
    std::string producer_name_;
    std::string producer_version_;
};

// Read an ONNX model (model.hpp:1328-1329 of the reference); the reader is in
// onnx_parser.hpp.
TBNModel load_model(const std::string& path);
TBNModel load_model_from_buffer(const void* data, size_t size);
const char* get_version();

}  // namespace tbn
