// ONNX ModelProto -> ModelGraph, decoding the protobuf wire format directly
// (the reference's tbn-runtime/src/onnx_integration/onnx_parser.cpp:67-366
// does this through libonnx).  Field numbers are those of onnx/onnx.proto
// (IR version 10); unknown fields are skipped by wire type, as protobuf does.
#include "tbn/onnx_parser.hpp"

#include <cstring>
#include <fstream>
#include <limits>
#include <map>
#include <utility>

#include "tbn/errors.hpp"

namespace tbn {

namespace {

// ---- protobuf wire format -------------------------------------------------------

enum Wire : int { kVarint = 0, kFixed64 = 1, kLen = 2, kFixed32 = 5 };

struct Field {
    uint32_t num = 0;
    int wire = 0;
    uint64_t v = 0;               // kVarint, kFixed64, kFixed32
    const uint8_t* p = nullptr;   // kLen
    size_t n = 0;
};

[[noreturn]] void malformed(const std::string& what) { throw InvalidModelError("malformed ONNX model: " + what); }

// Cursor over the bytes of one message.
class Reader {
public:
    Reader(const uint8_t* p, size_t n, const char* what) : p_(p), end_(p + n), what_(what) {}

    bool next(Field& f) {
        if (p_ == end_) return false;
        const uint64_t key = varint();
        f.num = static_cast<uint32_t>(key >> 3);
        f.wire = static_cast<int>(key & 7);
        if (f.num == 0 || (key >> 3) > 0x1FFFFFFF) fail("bad field number");
        switch (f.wire) {
            case kVarint: f.v = varint(); break;
            case kFixed64: need(8); std::memcpy(&f.v, p_, 8); p_ += 8; break;
            case kFixed32: {
                need(4);
                uint32_t w;
                std::memcpy(&w, p_, 4);
                f.v = w;
                p_ += 4;
                break;
            }
            case kLen: {
                const uint64_t n = varint();
                need(n);
                f.p = p_;
                f.n = static_cast<size_t>(n);
                p_ += n;
                break;
            }
            default: fail("unsupported wire type " + std::to_string(f.wire));
        }
        return true;
    }

    uint64_t varint() {
        uint64_t r = 0;
        for (int shift = 0; shift < 64; shift += 7) {
            need(1);
            const uint8_t c = *p_++;
            r |= static_cast<uint64_t>(c & 0x7F) << shift;
            if (!(c & 0x80)) return r;
        }
        fail("varint longer than 10 bytes");
    }

    bool done() const { return p_ == end_; }

private:
    void need(uint64_t n) const {
        if (n > static_cast<uint64_t>(end_ - p_)) fail("truncated");
    }
    [[noreturn]] void fail(const std::string& why) const { malformed(std::string(what_) + ": " + why); }

    const uint8_t* p_;
    const uint8_t* end_;
    const char* what_;
};

void expect(const Field& f, int wire, const char* what) {
    if (f.wire != wire)
        malformed(std::string(what) + ": field " + std::to_string(f.num) + " has wire type " +
                  std::to_string(f.wire));
}

std::string as_string(const Field& f, const char* what) {
    expect(f, kLen, what);
    return std::string(reinterpret_cast<const char*>(f.p), f.n);
}

int64_t as_int64(const Field& f, const char* what) {
    expect(f, kVarint, what);
    return static_cast<int64_t>(f.v);
}

// Repeated varint field, packed (one kLen record) or not (one record each).
template <class T>
void append_varints(const Field& f, std::vector<T>& out, const char* what) {
    if (f.wire == kVarint) {
        out.push_back(static_cast<T>(f.v));
        return;
    }
    expect(f, kLen, what);
    Reader r(f.p, f.n, what);
    while (!r.done()) out.push_back(static_cast<T>(r.varint()));
}

// Repeated fixed-width field (float: 4 bytes, double: 8 bytes), packed or not.
template <class T>
void append_fixed(const Field& f, std::vector<T>& out, const char* what) {
    constexpr int wire = sizeof(T) == 4 ? kFixed32 : kFixed64;
    if (f.wire == wire) {
        T v;
        if constexpr (sizeof(T) == 4) {
            const uint32_t w = static_cast<uint32_t>(f.v);
            std::memcpy(&v, &w, 4);
        } else {
            std::memcpy(&v, &f.v, 8);
        }
        out.push_back(v);
        return;
    }
    expect(f, kLen, what);
    if (f.n % sizeof(T)) malformed(std::string(what) + ": packed length not a multiple of the element size");
    if (f.n == 0) return;
    const size_t old = out.size();
    out.resize(old + f.n / sizeof(T));
    std::memcpy(out.data() + old, f.p, f.n);
}

// ---- ONNX messages ----------------------------------------------------------------

// TensorProto.DataType -> DataType and element size; false if unsupported.
bool map_dtype(int32_t t, DataType& dt) {
    switch (t) {
        case 1: dt = DataType::FLOAT32; return true;
        case 2: dt = DataType::UINT8; return true;
        case 3: dt = DataType::INT8; return true;
        case 4: dt = DataType::UINT16; return true;
        case 5: dt = DataType::INT16; return true;
        case 6: dt = DataType::INT32; return true;
        case 7: dt = DataType::INT64; return true;
        case 9: dt = DataType::BOOL; return true;
        case 10: dt = DataType::FLOAT16; return true;
        case 12: dt = DataType::UINT32; return true;
        case 13: dt = DataType::UINT64; return true;
        case 16: dt = DataType::BFLOAT16; return true;
        default: return false;
    }
}

struct TensorFields {
    std::string name;
    int32_t data_type = 0;
    std::vector<int64_t> dims;
    bool has_raw = false;
    const uint8_t* raw = nullptr;
    size_t raw_n = 0;
    std::vector<float> float_data;
    std::vector<int64_t> int32_data;  // varints: int32 values, or the bits of 8/16-bit types
    std::vector<int64_t> int64_data;
    std::vector<uint64_t> uint64_data;
    std::vector<std::pair<std::string, std::string>> external;
    int64_t data_location = 0;
    bool has_segment = false;
};

TensorFields read_tensor(const Field& outer) {
    static const char* what = "TensorProto";
    expect(outer, kLen, what);
    TensorFields t;
    Reader r(outer.p, outer.n, what);
    Field f;
    while (r.next(f)) {
        switch (f.num) {
            case 1: append_varints(f, t.dims, what); break;
            case 2: t.data_type = static_cast<int32_t>(as_int64(f, what)); break;
            case 3: t.has_segment = true; break;
            case 4: append_fixed(f, t.float_data, what); break;
            case 5: append_varints(f, t.int32_data, what); break;
            case 7: append_varints(f, t.int64_data, what); break;
            case 8: t.name = as_string(f, what); break;
            case 9:
                expect(f, kLen, what);
                t.has_raw = true;
                t.raw = f.p;
                t.raw_n = f.n;
                break;
            case 11: append_varints(f, t.uint64_data, what); break;
            case 13: {  // StringStringEntryProto {key = 1, value = 2}
                expect(f, kLen, what);
                std::string key, value;
                Reader e(f.p, f.n, "StringStringEntryProto");
                Field g;
                while (e.next(g)) {
                    if (g.num == 1) key = as_string(g, "StringStringEntryProto");
                    else if (g.num == 2) value = as_string(g, "StringStringEntryProto");
                }
                t.external.emplace_back(std::move(key), std::move(value));
                break;
            }
            case 14: t.data_location = as_int64(f, what); break;
            default: break;  // string_data, double_data, doc_string, metadata
        }
    }
    return t;
}

bool parse_decimal(const std::string& s, uint64_t& v) {
    if (s.empty() || s.size() > 19) return false;
    v = 0;
    for (char c : s) {
        if (c < '0' || c > '9') return false;
        v = v * 10 + static_cast<uint64_t>(c - '0');
    }
    return true;
}

// `location` must stay inside the model's directory: relative, no "..".
bool safe_relative_path(const std::string& loc) {
    if (loc.empty() || loc[0] == '/' || loc[0] == '\\' || loc.find(':') != std::string::npos) return false;
    size_t start = 0;
    while (start <= loc.size()) {
        size_t end = loc.find_first_of("/\\", start);
        if (end == std::string::npos) end = loc.size();
        if (loc.compare(start, end - start, "..") == 0 && end - start == 2) return false;
        start = end + 1;
    }
    return true;
}

// Where an external tensor's bytes are: the file (resolved against
// `base_dir`, which `location` may not leave) and the offset, after checking
// that the range holds exactly `bytes`.
struct ExternalRange {
    std::string path;
    uint64_t offset = 0;
};

ExternalRange external_range(const TensorFields& t, const std::string& base_dir, size_t bytes) {
    std::string location;
    uint64_t offset = 0, length = 0;
    bool has_length = false;
    for (const auto& [key, value] : t.external) {
        if (key == "location") location = value;
        else if (key == "offset") {
            if (!parse_decimal(value, offset)) malformed("tensor '" + t.name + "': external data offset '" + value + "'");
        } else if (key == "length") {
            if (!parse_decimal(value, length)) malformed("tensor '" + t.name + "': external data length '" + value + "'");
            has_length = true;
        }
    }
    TBN_CHECK(!location.empty(), InvalidModelError, "tensor '" + t.name + "': external data without a location");
    TBN_CHECK(safe_relative_path(location), InvalidModelError,
              "tensor '" + t.name + "': external data location '" + location +
                  "' must be a relative path inside the model's directory");
    TBN_CHECK(!base_dir.empty(), InvalidModelError,
              "tensor '" + t.name + "' keeps its data in '" + location +
                  "', but the model was read from a buffer without a base directory");
    const std::string path = base_dir + "/" + location;
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    TBN_CHECK(static_cast<bool>(in), InvalidModelError, "tensor '" + t.name + "': cannot open external data file " + path);
    const uint64_t file_size = static_cast<uint64_t>(in.tellg());
    TBN_CHECK(offset <= file_size, InvalidModelError, "tensor '" + t.name + "': external data offset past the end of " + path);
    if (!has_length) length = file_size - offset;
    TBN_CHECK(length <= file_size - offset, InvalidModelError,
              "tensor '" + t.name + "': external data range past the end of " + path);
    TBN_CHECK(length == bytes, InvalidModelError,
              "tensor '" + t.name + "': external data holds " + std::to_string(length) + " bytes, its shape needs " +
                  std::to_string(bytes));
    return {path, offset};
}

void read_external(const TensorFields& t, const ExternalRange& r, void* dst, size_t bytes) {
    std::ifstream in(r.path, std::ios::binary);
    in.seekg(static_cast<std::streamoff>(r.offset));
    in.read(static_cast<char*>(dst), static_cast<std::streamsize>(bytes));
    TBN_CHECK(static_cast<bool>(in), InvalidModelError, "tensor '" + t.name + "': short read from " + r.path);
}

// onnx_parser.cpp:196-239, with external data and size checks.  Every size is
// checked against the data present before the tensor is allocated, so a
// malformed shape cannot ask for more memory than the file backs.
Tensor make_tensor(const TensorFields& t, const std::string& base_dir) {
    DataType dt;
    TBN_CHECK(map_dtype(t.data_type, dt), NotImplementedError,
              "tensor '" + t.name + "': ONNX data type " + std::to_string(t.data_type) + " is not supported");
    TBN_CHECK(!t.has_segment, NotImplementedError, "tensor '" + t.name + "': segmented tensors are not supported");
    Shape shape;
    uint64_t numel = 1;
    for (int64_t d : t.dims) {
        TBN_CHECK(d >= 0, InvalidModelError, "tensor '" + t.name + "': negative dimension");
        TBN_CHECK(d == 0 || numel <= (uint64_t(1) << 48) / static_cast<uint64_t>(d), InvalidModelError,
                  "tensor '" + t.name + "': too many elements");
        numel *= static_cast<uint64_t>(d);
        shape.dims.push_back(d);
    }
    const size_t esize = element_size(dt);
    const size_t bytes = static_cast<size_t>(numel) * esize;
    const bool external = t.data_location == 1 || !t.external.empty();

    if (external) {
        if (bytes == 0) return Tensor(shape, dt);
        const ExternalRange range = external_range(t, base_dir, bytes);
        Tensor out(shape, dt);
        read_external(t, range, out.data(), bytes);
        return out;
    }
    if (t.has_raw) {
        TBN_CHECK(t.raw_n == bytes, InvalidModelError,
                  "tensor '" + t.name + "': raw_data holds " + std::to_string(t.raw_n) + " bytes, its shape needs " +
                      std::to_string(bytes));
        return Tensor(shape, dt, t.raw);
    }
    if (numel == 0) return Tensor(shape, dt);
    // typed fields: float_data (FLOAT), int64_data (INT64), uint64_data
    // (UINT32, UINT64), int32_data (INT32 and the 8/16-bit types, as their
    // value or bits)
    const char* field = dt == DataType::FLOAT32 ? "float_data"
                        : dt == DataType::INT64 ? "int64_data"
                        : (dt == DataType::UINT32 || dt == DataType::UINT64) ? "uint64_data"
                                                                             : "int32_data";
    const size_t count = dt == DataType::FLOAT32 ? t.float_data.size()
                         : dt == DataType::INT64 ? t.int64_data.size()
                         : (dt == DataType::UINT32 || dt == DataType::UINT64) ? t.uint64_data.size()
                                                                              : t.int32_data.size();
    TBN_CHECK(count == numel, InvalidModelError,
              "tensor '" + t.name + "': " + field + " holds " + std::to_string(count) + " values, its shape has " +
                  std::to_string(numel));
    Tensor out(shape, dt);
    auto* dst = static_cast<uint8_t*>(out.data());
    if (dt == DataType::FLOAT32) {
        std::memcpy(dst, t.float_data.data(), bytes);
    } else if (dt == DataType::INT64) {
        std::memcpy(dst, t.int64_data.data(), bytes);
    } else if (dt == DataType::UINT32 || dt == DataType::UINT64) {
        for (size_t i = 0; i < numel; ++i) {
            const uint64_t v = t.uint64_data[i];
            std::memcpy(dst + i * esize, &v, esize);  // little-endian: the low bytes
        }
    } else {
        for (size_t i = 0; i < numel; ++i) {
            const uint32_t v = static_cast<uint32_t>(t.int32_data[i]);
            std::memcpy(dst + i * esize, &v, esize);
        }
    }
    return out;
}

// ValueInfoProto -> (name, shape); onnx_parser.cpp:161-177 (symbolic dims -> 1).
std::pair<std::string, Shape> read_value_info(const Field& outer, std::vector<std::string>& warnings) {
    static const char* what = "ValueInfoProto";
    expect(outer, kLen, what);
    std::string name;
    Shape shape;
    bool tensor_type = false, has_type = false;
    Reader r(outer.p, outer.n, what);
    Field f;
    while (r.next(f)) {
        if (f.num == 1) name = as_string(f, what);
        if (f.num != 2) continue;
        has_type = true;
        expect(f, kLen, "TypeProto");
        Reader tr(f.p, f.n, "TypeProto");
        Field g;
        while (tr.next(g)) {
            if (g.num != 1) continue;  // tensor_type
            tensor_type = true;
            expect(g, kLen, "TypeProto.Tensor");
            Reader tt(g.p, g.n, "TypeProto.Tensor");
            Field h;
            while (tt.next(h)) {
                if (h.num != 2) continue;  // shape
                expect(h, kLen, "TensorShapeProto");
                Reader sr(h.p, h.n, "TensorShapeProto");
                Field d;
                while (sr.next(d)) {
                    if (d.num != 1) continue;
                    expect(d, kLen, "TensorShapeProto.Dimension");
                    Reader dr(d.p, d.n, "TensorShapeProto.Dimension");
                    Field e;
                    int64_t value = 1;
                    while (dr.next(e))
                        if (e.num == 1) value = as_int64(e, "TensorShapeProto.Dimension");
                    shape.dims.push_back(value);
                }
            }
        }
    }
    if (has_type && !tensor_type) warnings.push_back("value '" + name + "' is not a tensor; its shape is left empty");
    return {name, shape};
}

enum AttrType : int64_t {
    kAttrFloat = 1, kAttrInt = 2, kAttrString = 3, kAttrTensor = 4, kAttrGraph = 5,
    kAttrFloats = 6, kAttrInts = 7, kAttrStrings = 8
};

// onnx_parser.cpp:255-311.  Returns false for attribute types a ModelGraph
// cannot hold (graphs, tensor lists, type protos, sparse tensors).
bool read_attribute(const Field& outer, const std::string& base_dir, std::string& name, AttributeValue& value,
                    int64_t& type) {
    static const char* what = "AttributeProto";
    expect(outer, kLen, what);
    type = 0;
    float fval = 0;
    int64_t ival = 0;
    std::string sval;
    const Field* tfield = nullptr;
    Field tcopy;
    std::vector<float> floats;
    std::vector<int64_t> ints;
    std::vector<std::string> strings;
    bool has_f = false, has_i = false, has_s = false, has_t = false, has_other = false, ref = false;
    Reader r(outer.p, outer.n, what);
    Field f;
    while (r.next(f)) {
        switch (f.num) {
            case 1: name = as_string(f, what); break;
            case 2: {
                expect(f, kFixed32, what);
                const uint32_t w = static_cast<uint32_t>(f.v);
                std::memcpy(&fval, &w, 4);
                has_f = true;
                break;
            }
            case 3: ival = as_int64(f, what); has_i = true; break;
            case 4: sval = as_string(f, what); has_s = true; break;
            case 5: expect(f, kLen, what); tcopy = f; tfield = &tcopy; has_t = true; break;
            case 7: append_fixed(f, floats, what); break;
            case 8: append_varints(f, ints, what); break;
            case 9: strings.push_back(as_string(f, what)); break;
            case 20: type = as_int64(f, what); break;
            case 21: ref = true; break;
            case 6: case 10: case 11: case 14: case 15: case 22: case 23: has_other = true; break;
            default: break;
        }
    }
    if (ref) return false;  // a reference to an enclosing function's attribute
    if (type == 0) {  // IR versions before 0.0.2 carry no type: infer it from the field present
        if (has_f) type = kAttrFloat;
        else if (has_i) type = kAttrInt;
        else if (has_s) type = kAttrString;
        else if (has_t) type = kAttrTensor;
        else if (!floats.empty()) type = kAttrFloats;
        else if (!ints.empty()) type = kAttrInts;
        else if (!strings.empty()) type = kAttrStrings;
        else if (has_other) return false;
    }
    switch (type) {
        case kAttrFloat: value = AttributeValue(fval); return true;
        case kAttrInt: value = AttributeValue(ival); return true;
        case kAttrString: value = AttributeValue(sval); return true;
        case kAttrTensor:
            if (!tfield) malformed("attribute '" + name + "' of type TENSOR holds no tensor");
            value = AttributeValue(make_tensor(read_tensor(*tfield), base_dir));
            return true;
        case kAttrFloats: value = AttributeValue(floats); return true;
        case kAttrInts: value = AttributeValue(ints); return true;
        case kAttrStrings: value = AttributeValue(strings); return true;
        default: return false;
    }
}

// NodeProto; onnx_parser.cpp:241-313.
ModelNode read_node(const Field& outer, const std::string& base_dir, std::vector<std::string>& warnings) {
    static const char* what = "NodeProto";
    expect(outer, kLen, what);
    ModelNode node;
    std::string domain;
    Reader r(outer.p, outer.n, what);
    Field f;
    std::vector<Field> attrs;
    while (r.next(f)) {
        switch (f.num) {
            case 1: node.inputs.push_back(as_string(f, what)); break;
            case 2: node.outputs.push_back(as_string(f, what)); break;
            case 3: node.name = as_string(f, what); break;
            case 4: node.op_type = as_string(f, what); break;
            case 5: attrs.push_back(f); break;
            case 7: domain = as_string(f, what); break;
            default: break;
        }
    }
    if (node.name.empty()) node.name = node.op_type + "_" + (node.outputs.empty() ? std::string() : node.outputs[0]);
    for (const Field& a : attrs) {
        std::string name;
        AttributeValue value;
        int64_t type = 0;
        if (read_attribute(a, base_dir, name, value, type)) node.attributes[name] = std::move(value);
        else
            warnings.push_back("node '" + node.name + "': attribute '" + name + "' of type " + std::to_string(type) +
                               " skipped");
    }
    if (!domain.empty() && domain != "ai.onnx")
        warnings.push_back("node '" + node.name + "': operator domain '" + domain + "'");
    return node;
}

}  // namespace

// ---- OnnxParser ---------------------------------------------------------------------

struct OnnxParser::Impl {
    std::shared_ptr<ModelGraph> graph;
    std::string producer_name, producer_version;
    int64_t ir_version = 0;
    std::map<std::string, int64_t> opsets;
    std::vector<std::string> warnings;

    void decode_graph(const Field& outer, const std::string& base_dir) {
        static const char* what = "GraphProto";
        expect(outer, kLen, what);
        std::vector<Field> nodes, inits, inputs, outputs, infos;
        Reader r(outer.p, outer.n, what);
        Field f;
        while (r.next(f)) {
            switch (f.num) {
                case 1: nodes.push_back(f); break;
                case 5: inits.push_back(f); break;
                case 11: inputs.push_back(f); break;
                case 12: outputs.push_back(f); break;
                case 13: infos.push_back(f); break;
                case 15: warnings.push_back("sparse initializer skipped"); break;
                default: break;
            }
        }
        // Initializers first, so inputs that name one can be told apart.
        for (const Field& x : inits) {
            TensorFields t = read_tensor(x);
            TBN_CHECK(!t.name.empty(), InvalidModelError, "initializer without a name");
            graph->initializers[t.name] = make_tensor(t, base_dir);
        }
        for (const Field& x : inputs) {
            auto [name, shape] = read_value_info(x, warnings);
            if (graph->initializers.count(name)) continue;
            graph->inputs.push_back(name);
            graph->value_info[name] = shape;
        }
        for (const Field& x : outputs) {
            auto [name, shape] = read_value_info(x, warnings);
            graph->outputs.push_back(name);
            graph->value_info[name] = shape;
        }
        for (const Field& x : infos) {
            auto [name, shape] = read_value_info(x, warnings);
            graph->value_info[name] = shape;
        }
        for (const Field& x : nodes) graph->nodes.push_back(read_node(x, base_dir, warnings));
    }

    void decode(const uint8_t* p, size_t n, const std::string& base_dir) {
        graph = std::make_shared<ModelGraph>();
        producer_name.clear();
        producer_version.clear();
        ir_version = 0;
        opsets.clear();
        warnings.clear();
        static const char* what = "ModelProto";
        Reader r(p, n, what);
        Field f;
        bool has_graph = false;
        while (r.next(f)) {
            switch (f.num) {
                case 1: ir_version = as_int64(f, what); break;
                case 2: producer_name = as_string(f, what); break;
                case 3: producer_version = as_string(f, what); break;
                case 7: decode_graph(f, base_dir); has_graph = true; break;
                case 8: {
                    expect(f, kLen, "OperatorSetIdProto");
                    Reader o(f.p, f.n, "OperatorSetIdProto");
                    Field g;
                    std::string domain;
                    int64_t version = 0;
                    while (o.next(g)) {
                        if (g.num == 1) domain = as_string(g, "OperatorSetIdProto");
                        else if (g.num == 2) version = as_int64(g, "OperatorSetIdProto");
                    }
                    opsets[domain] = version;
                    break;
                }
                default: break;
            }
        }
        TBN_CHECK(has_graph, InvalidModelError, "ONNX model has no graph");
    }
};

OnnxParser::OnnxParser() : impl_(std::make_unique<Impl>()) {}
OnnxParser::~OnnxParser() = default;

void OnnxParser::parse_from_file(const std::string& path) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    TBN_CHECK(static_cast<bool>(in), InvalidModelError, "Failed to open ONNX file: " + path);
    const std::streamoff size = in.tellg();
    TBN_CHECK(size >= 0, InvalidModelError, "Failed to read ONNX file: " + path);
    std::vector<uint8_t> bytes(static_cast<size_t>(size));
    in.seekg(0);
    in.read(reinterpret_cast<char*>(bytes.data()), size);
    TBN_CHECK(static_cast<bool>(in), InvalidModelError, "Failed to read ONNX file: " + path);
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? std::string(".") : (slash == 0 ? std::string("/") : path.substr(0, slash));
    impl_->decode(bytes.data(), bytes.size(), dir);
}

void OnnxParser::parse_from_buffer(const void* data, size_t size, const std::string& base_dir) {
    TBN_CHECK(data != nullptr || size == 0, InvalidArgumentError, "parse_from_buffer: null data");
    impl_->decode(static_cast<const uint8_t*>(data), size, base_dir);
}

std::shared_ptr<ModelGraph> OnnxParser::get_graph() {
    TBN_CHECK(impl_->graph != nullptr, RuntimeError, "OnnxParser: no model parsed");
    return std::make_shared<ModelGraph>(*impl_->graph);
}

std::string OnnxParser::get_producer_name() const { return impl_->producer_name; }
std::string OnnxParser::get_producer_version() const { return impl_->producer_version; }
int64_t OnnxParser::ir_version() const { return impl_->ir_version; }

int64_t OnnxParser::opset_version(const std::string& domain) const {
    auto it = impl_->opsets.find(domain);
    if (it == impl_->opsets.end() && domain.empty()) it = impl_->opsets.find("ai.onnx");
    return it == impl_->opsets.end() ? -1 : it->second;
}

const std::vector<std::string>& OnnxParser::warnings() const { return impl_->warnings; }

TBNModel load_onnx_model(const std::string& path) {
    OnnxParser parser;
    parser.parse_from_file(path);
    TBNModel model(parser.get_graph());
    model.set_producer(parser.get_producer_name(), parser.get_producer_version());
    return model;
}

TBNModel load_onnx_model_from_buffer(const void* data, size_t size, const std::string& base_dir) {
    OnnxParser parser;
    parser.parse_from_buffer(data, size, base_dir);
    TBNModel model(parser.get_graph());
    model.set_producer(parser.get_producer_name(), parser.get_producer_version());
    return model;
}

}  // namespace tbn
