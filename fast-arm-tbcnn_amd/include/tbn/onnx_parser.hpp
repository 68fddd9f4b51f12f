// ONNX model reader of the tbn runtime (the reference's
// tbn-runtime/include/tbn/onnx_integration/onnx_parser.hpp:21-48 and
// src/onnx_integration/onnx_parser.cpp:67-366).
//
// The reference decodes ModelProto with libonnx + protobuf
// (onnx_parser.cpp:18-24) and leaves every tensor whose bytes live in an
// external data file as zeros (onnx_parser.cpp:218-236).  This reader decodes
// the protobuf wire format itself -- only the fields a ModelGraph keeps -- and
// reads external data from the file each tensor names, resolved against the
// model file's directory.  The graph it builds is the reference's: graph
// inputs, outputs and value_info shapes (a symbolic dimension becomes 1),
// initializers as host tensors, nodes with their attributes in file order
// (an unnamed node is called "<op_type>_<first output>").
//
// Differences from the reference, each an error the reference lets through:
//  * a tensor that holds no data although it has elements, raw data whose
//    size does not match its shape, and a data type the runtime has no
//    DataType for are InvalidModelError / NotImplementedError instead of a
//    zero-filled (or overrun) tensor;
//  * a graph input that also names an initializer is left out of the graph's
//    inputs (it is a constant with a default value, set by the initializer).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "model.hpp"

namespace tbn {

class OnnxParser {
public:
    OnnxParser();
    ~OnnxParser();
    OnnxParser(const OnnxParser&) = delete;
    OnnxParser& operator=(const OnnxParser&) = delete;

    // Reads and decodes a .onnx file; external data locations are relative
    // to its directory.  Throws InvalidModelError on a malformed file.
    void parse_from_file(const std::string& path);
    // Decodes a serialized ModelProto.  `base_dir` resolves external data
    // locations; with an empty `base_dir` a model that has external data is
    // rejected.
    void parse_from_buffer(const void* data, size_t size, const std::string& base_dir = "");

    // A fresh ModelGraph of the parsed model (initializer tensors are shared
    // between the graphs returned).
    std::shared_ptr<ModelGraph> get_graph();

    std::string get_producer_name() const;
    std::string get_producer_version() const;
    int64_t ir_version() const;
    // Opset version imported for `domain` ("" is the default ONNX domain), or
    // -1 when the model imports none.
    int64_t opset_version(const std::string& domain = "") const;
    // What was skipped while decoding (attribute and value types a ModelGraph
    // cannot hold), one message each; the reference logs these as warnings.
    const std::vector<std::string>& warnings() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// onnx_parser.cpp:345-366.
TBNModel load_onnx_model(const std::string& path);
TBNModel load_onnx_model_from_buffer(const void* data, size_t size, const std::string& base_dir = "");

}  // namespace tbn
