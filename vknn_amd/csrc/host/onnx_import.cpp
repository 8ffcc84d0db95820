// ONNX model import (reference include/vknn/graph.h:42 `Graph importOnnx(const std::string &)`,
// implemented there by src/import/onnx/onnx_parser.cpp:23-57 and the builder/parsers beside it).
//
// The protobuf wire format is decoded directly — there is no protobuf library in either build —
// by a cursor that checks every length and varint against the end of its buffer, so a truncated
// or corrupt file raises Error(InvalidArgument) instead of reading past the buffer. The graph that
// comes out is the one the reference's importer builds from the same file:
//   * ModelProto.graph (field 7) is the only field read; no graph -> InvalidArgument.
//   * Nodes keep their ONNX order until the final stable topological sort. op_type maps to OpType
//     by the reference's table (src/core/op.cpp:112-221): ReduceMean -> GlobalAvgPool, Upsample ->
//     Resize, the elementwise math ops -> Unary/Binary with their sub-op code, the ReduceX family ->
//     Reduce. An op with no mapping stays OpType::Unknown (a warning is printed) so the session
//     reports which op no backend runs.
//   * Unary parameters take the ONNX defaults (onnx_node_parser.h:267-283): LeakyRelu alpha 0.01
//     and Elu alpha 1.0 into actLo; HardSigmoid alpha 0.2 / beta 0.5 into actLo / actHi.
//   * Tensor names resolve in SSA order (onnx_graph_builder.h:158-222): a node input binds to the
//     latest earlier producer of that name, every node output gets a fresh TensorId carrying its
//     value_info shape, a declared graph output is re-pointed at the last producer of its name,
//     and a node without a name is called "<OpTypeName>_<index>".
//   * Initializers become host buffers: INT64 stays int64, every other element type is decoded
//     to fp32 (FLOAT, FLOAT16, DOUBLE, and the integer types by value). Weights stored outside the
//     model (data_location EXTERNAL) are read from the named file relative to the model's folder,
//     each file once. Initializers listed among the graph inputs are dropped from the inputs.
//   * Attribute tensors (Constant's "value") become Floats or Ints attributes that keep the
//     tensor's dims in Attr::shape.
// Where the reference would zero-fill a short raw_data or ignore an out-of-range external slice,
// this importer rejects the file (InvalidArgument) — a model with missing weight bytes is not run.
#include "vknn/graph.h"
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <unordered_map>

namespace vknn {

    namespace {

        [[noreturn]] void malformed(const std::string &what) { throw Error(Status::InvalidArgument, "malformed ONNX file: " + what); }

        // A bounds-checked protobuf cursor over [p, end).
        struct Wire {
            const uint8_t *p, *end;

            bool more() const { return p < end; }

            uint64_t varint() {
                uint64_t v = 0;
                for (int shift = 0; shift < 64; shift += 7) {
                    if (p >= end) malformed("varint runs past the end of its message");
                    const uint8_t b = *p++;
                    v |= (uint64_t) (b & 0x7f) << shift;
                    if (!(b & 0x80)) return v;
                }
                malformed("varint longer than 10 bytes");
            }
            const uint8_t *take(uint64_t n) {
                if (n > (uint64_t) (end - p)) malformed("field length runs past the end of its message");
                const uint8_t *q = p;
                p += n;
                return q;
            }
            uint32_t fixed32() {
                uint32_t v;
                std::memcpy(&v, take(4), 4);
                return v;
            }
            uint64_t fixed64() {
                uint64_t v;
                std::memcpy(&v, take(8), 8);
                return v;
            }
            Wire sub() {
                const uint64_t n = varint();
                const uint8_t *q = take(n);
                return Wire {q, q + n};
            }
            std::string text() {
                Wire s = sub();
                return std::string((const char *) s.p, (size_t) (s.end - s.p));
            }
            void skip(int wt) {
                switch (wt) {
                    case 0: varint(); break;
                    case 1: take(8); break;
                    case 2: sub(); break;
                    case 5: take(4); break;
                    default: malformed("unsupported wire type " + std::to_string(wt));
                }
            }
            // Next field tag; false at the end of the message.
            bool next(uint32_t &field, int &wt) {
                if (p >= end) return false;
                const uint64_t tag = varint();
                field              = (uint32_t) (tag >> 3);
                wt                 = (int) (tag & 7);
                if (field == 0) malformed("field number 0");
                return true;
            }
        };

        float bitsToFloat(uint32_t b) {
            float f;
            std::memcpy(&f, &b, 4);
            return f;
        }

        // A repeated scalar field arrives packed (wire type 2) or one value per tag.
        template <typename Read> void repeated(Wire &w, int wt, Read read) {
            if (wt == 2) {
                Wire s = w.sub();
                while (s.more()) read(s);
            } else {
                read(w);
            }
        }

        enum : int32_t {
            kFloat = 1, kUint8 = 2, kInt8 = 3, kUint16 = 4, kInt16 = 5, kInt32 = 6, kInt64 = 7, kBool = 9, kFloat16 = 10,
            kDouble = 11, kUint32 = 12, kUint64 = 13
        };

        // Graph-level dtype of a declared input/output (reference onnx_types.h:52-72).
        DType dtypeOfElem(int32_t el) {
            switch (el) {
                case kFloat16: return DType::Float16;
                case kInt64: return DType::Int64;
                case kInt32: return DType::Int32;
                case kInt8: return DType::Int8;
                case kUint8: case kBool: return DType::UInt8;
                default: return DType::Float32;
            }
        }

        // TensorProto: 1 dims, 2 data_type, 4 float_data, 5 int32_data, 7 int64_data, 8 name,
        // 9 raw_data, 10 double_data, 13 external_data {1 key, 2 value}, 14 data_location.
        struct TensorMsg {
            std::vector<int64_t> dims;
            int32_t              dtype = kFloat;
            std::string          name;
            const uint8_t       *raw   = nullptr;
            size_t               rawN  = 0;
            std::vector<float>   floats;
            std::vector<int32_t> int32s;
            std::vector<int64_t> int64s;
            std::vector<double>  doubles;
            bool                 external = false;
            std::string          location;
            int64_t              offset = 0, length = -1;

            int64_t elems() const {
                int64_t n = 1;
                for (int64_t d: dims) {
                    if (d < 0) malformed("tensor '" + name + "' has a negative dimension");
                    // no product may wrap: a wrapped count would pass the byte checks below while
                    // the shape still claims the huge size
                    if (d && n > (int64_t(1) << 40) / d) malformed("tensor '" + name + "' has more than 2^40 elements");
                    n *= d;
                }
                return n;
            }
        };

        TensorMsg readTensor(Wire w) {
            TensorMsg t;
            uint32_t  f;
            int       wt;
            while (w.next(f, wt)) {
                switch (f) {
                    case 1: repeated(w, wt, [&](Wire &s) { t.dims.push_back((int64_t) s.varint()); }); break;
                    case 2: t.dtype = (int32_t) w.varint(); break;
                    case 4: repeated(w, wt, [&](Wire &s) { t.floats.push_back(bitsToFloat(s.fixed32())); }); break;
                    case 5: repeated(w, wt, [&](Wire &s) { t.int32s.push_back((int32_t) s.varint()); }); break;
                    case 7: repeated(w, wt, [&](Wire &s) { t.int64s.push_back((int64_t) s.varint()); }); break;
                    case 8: t.name = w.text(); break;
                    case 9: {
                        Wire s = w.sub();
                        t.raw  = s.p;
                        t.rawN = (size_t) (s.end - s.p);
                        break;
                    }
                    case 10:
                        repeated(w, wt, [&](Wire &s) {
                            uint64_t b = s.fixed64();
                            double   d;
                            std::memcpy(&d, &b, 8);
                            t.doubles.push_back(d);
                        });
                        break;
                    case 13: {
                        Wire        e = w.sub();
                        std::string key, val;
                        uint32_t    ef;
                        int         ewt;
                        while (e.next(ef, ewt)) {
                            if (ef == 1 && ewt == 2) key = e.text();
                            else if (ef == 2 && ewt == 2) val = e.text();
                            else e.skip(ewt);
                        }
                        if (key == "location") t.location = val;
                        else if (key == "offset") t.offset = std::strtoll(val.c_str(), nullptr, 10);
                        else if (key == "length") t.length = std::strtoll(val.c_str(), nullptr, 10);
                        break;
                    }
                    case 14: t.external = w.varint() == 1; break;
                    default: w.skip(wt); break;
                }
            }
            return t;
        }

        size_t elemBytes(int32_t dt) {
            switch (dt) {
                case kFloat: case kInt32: case kUint32: return 4;
                case kFloat16: case kInt16: case kUint16: return 2;
                case kDouble: case kInt64: case kUint64: return 8;
                case kInt8: case kUint8: case kBool: return 1;
                default: return 0;
            }
        }

        // Element i of a little-endian raw buffer of ONNX type dt, as a double (exact for every
        // type here except 64-bit integers beyond 2^53, which only shape tensors hold and which
        // take the int64 path instead).
        double rawValue(const uint8_t *r, int32_t dt, int64_t i) {
            switch (dt) {
                case kFloat: { uint32_t b; std::memcpy(&b, r + 4 * i, 4); return bitsToFloat(b); }
                case kFloat16: { uint16_t h; std::memcpy(&h, r + 2 * i, 2); return halfToFloat(h); }
                case kDouble: { double d; std::memcpy(&d, r + 8 * i, 8); return d; }
                case kInt64: { int64_t v; std::memcpy(&v, r + 8 * i, 8); return (double) v; }
                case kUint64: { uint64_t v; std::memcpy(&v, r + 8 * i, 8); return (double) v; }
                case kInt32: { int32_t v; std::memcpy(&v, r + 4 * i, 4); return v; }
                case kUint32: { uint32_t v; std::memcpy(&v, r + 4 * i, 4); return v; }
                case kInt16: { int16_t v; std::memcpy(&v, r + 2 * i, 2); return v; }
                case kUint16: { uint16_t v; std::memcpy(&v, r + 2 * i, 2); return v; }
                case kInt8: return (int8_t) r[i];
                default: return r[i];
            }
        }

        // The tensor's n values decoded to fp32.
        std::vector<float> floatValues(const TensorMsg &t, int64_t n) {
            std::vector<float> v((size_t) n);
            if (t.raw) {
                const size_t eb = elemBytes(t.dtype);
                if (!eb) malformed("tensor '" + t.name + "' has unsupported element type " + std::to_string(t.dtype));
                if ((size_t) n > t.rawN / eb) malformed("tensor '" + t.name + "' holds fewer bytes than its dims need");
                for (int64_t i = 0; i < n; ++i) v[i] = (float) rawValue(t.raw, t.dtype, i);
                return v;
            }
            auto fill = [&](const auto &src) {
                if ((int64_t) src.size() < n) malformed("tensor '" + t.name + "' holds fewer values than its dims need");
                for (int64_t i = 0; i < n; ++i) v[i] = (float) src[i];
            };
            if (!t.floats.empty()) fill(t.floats);
            else if (!t.doubles.empty()) fill(t.doubles);
            else if (!t.int64s.empty()) fill(t.int64s);
            else if (t.dtype == kFloat16) {
                // FLOAT16 values in int32_data carry the half's bit pattern in the low 16 bits
                if ((int64_t) t.int32s.size() < n) malformed("tensor '" + t.name + "' holds fewer values than its dims need");
                for (int64_t i = 0; i < n; ++i) v[i] = halfToFloat((fp16_t) (t.int32s[i] & 0xffff));
            } else if (!t.int32s.empty()) fill(t.int32s);
            else if (n) malformed("tensor '" + t.name + "' has no data");
            return v;
        }

        std::vector<int64_t> int64Values(const TensorMsg &t, int64_t n) {
            std::vector<int64_t> v((size_t) n);
            if (t.raw) {
                if ((size_t) n > t.rawN / 8) malformed("tensor '" + t.name + "' holds fewer bytes than its dims need");
                std::memcpy(v.data(), t.raw, (size_t) n * 8);
            } else {
                if ((int64_t) t.int64s.size() < n) malformed("tensor '" + t.name + "' holds fewer values than its dims need");
                std::copy(t.int64s.begin(), t.int64s.begin() + n, v.begin());
            }
            return v;
        }

        // Attribute tensors: Floats/Ints with the dims kept (reference onnx_node_parser.h:96-158).
        // A dims-less tensor is treated as a scalar.
        void tensorAttr(const TensorMsg &t, Attr &a) {
            a.shape   = t.dims;
            int64_t n = t.dims.empty() ? 1 : t.elems();
            if (t.dims.empty() && !t.raw) n = (int64_t) std::max<size_t>({1, t.floats.size(), t.int64s.size(), t.int32s.size(), t.doubles.size()});
            if (t.dtype == kInt64 || (!t.raw && !t.int64s.empty())) {
                a.kind = Attr::Ints;
                a.ints = int64Values(t, n);
            } else {
                a.kind   = Attr::Floats;
                a.floats = floatValues(t, n);
            }
        }

        // AttributeProto: 1 name, 2 f, 3 i, 4 s, 5 t, 7 floats, 8 ints.
        void readAttr(Wire w, Attributes &out) {
            std::string name;
            Attr        a;
            uint32_t    f;
            int         wt;
            while (w.next(f, wt)) {
                switch (f) {
                    case 1: name = w.text(); break;
                    case 2: a.f = bitsToFloat(w.fixed32()); a.kind = Attr::Float; break;
                    case 3: a.i = (int64_t) w.varint(); a.kind = Attr::Int; break;
                    case 4: a.str = w.text(); a.kind = Attr::String; break;
                    case 5: tensorAttr(readTensor(w.sub()), a); break;
                    case 7: repeated(w, wt, [&](Wire &s) { a.floats.push_back(bitsToFloat(s.fixed32())); }); a.kind = Attr::Floats; break;
                    case 8: repeated(w, wt, [&](Wire &s) { a.ints.push_back((int64_t) s.varint()); }); a.kind = Attr::Ints; break;
                    default: w.skip(wt); break;
                }
            }
            out.map[name] = std::move(a);
        }

        // ValueInfoProto: 1 name, 2 type { 1 tensor_type { 1 elem_type, 2 shape { 1 dim { 1 dim_value,
        // 2 dim_param } } } }. A symbolic or missing dimension reads as -1.
        void readValueInfo(Wire w, std::string &name, Shape &shape, int32_t &elem) {
            uint32_t f;
            int      wt;
            while (w.next(f, wt)) {
                if (f == 1 && wt == 2) { name = w.text(); continue; }
                if (f != 2 || wt != 2) { w.skip(wt); continue; }
                Wire type = w.sub();
                while (type.next(f, wt)) {
                    if (f != 1 || wt != 2) { type.skip(wt); continue; }
                    Wire tt = type.sub();
                    while (tt.next(f, wt)) {
                        if (f == 1 && wt == 0) { elem = (int32_t) tt.varint(); continue; }
                        if (f != 2 || wt != 2) { tt.skip(wt); continue; }
                        Wire sh = tt.sub();
                        while (sh.next(f, wt)) {
                            if (f != 1 || wt != 2) { sh.skip(wt); continue; }
                            Wire    dim = sh.sub();
                            int64_t v   = -1;
                            while (dim.next(f, wt)) {
                                if (f == 1 && wt == 0) v = (int64_t) dim.varint();
                                else dim.skip(wt);
                            }
                            shape.push_back(v);
                        }
                    }
                }
            }
        }

        struct OpMap {
            OpType  type  = OpType::Unknown;
            int32_t subOp = 0;
        };

        // ONNX op_type -> OpType (+ sub-op code), the reference's table (src/core/op.cpp:112-221).
        OpMap mapOp(const std::string &s) {
            static const std::unordered_map<std::string, OpType> direct = {
                {"Conv", OpType::Conv}, {"ConvTranspose", OpType::ConvTranspose}, {"Clip", OpType::Clip}, {"Relu", OpType::Relu},
                {"Add", OpType::Add}, {"GlobalAveragePool", OpType::GlobalAvgPool}, {"ReduceMean", OpType::GlobalAvgPool},
                {"AveragePool", OpType::AvgPool}, {"MaxPool", OpType::MaxPool}, {"Gemm", OpType::Gemm}, {"MatMul", OpType::MatMul},
                {"Einsum", OpType::Einsum}, {"Reshape", OpType::Reshape}, {"Expand", OpType::Expand}, {"Tile", OpType::Tile},
                {"Squeeze", OpType::Squeeze}, {"Flatten", OpType::Flatten}, {"Softmax", OpType::Softmax},
                {"LayerNormalization", OpType::LayerNorm}, {"BatchNormalization", OpType::BatchNorm}, {"Concat", OpType::Concat},
                {"Pad", OpType::Pad}, {"Identity", OpType::Identity}, {"Constant", OpType::Constant}, {"Shape", OpType::Shape},
                {"Gather", OpType::Gather}, {"Unsqueeze", OpType::Unsqueeze}, {"PRelu", OpType::PRelu}, {"Resize", OpType::Resize},
                {"Upsample", OpType::Resize}, {"GridSample", OpType::GridSample}, {"Transpose", OpType::Transpose},
                {"Slice", OpType::Slice}, {"DepthToSpace", OpType::DepthToSpace}, {"Cast", OpType::Cast}, {"Split", OpType::Split},
                {"Where", OpType::Where}, {"Equal", OpType::Equal}, {"Greater", OpType::Greater},
                {"GreaterOrEqual", OpType::GreaterEqual}, {"GreaterEqual", OpType::GreaterEqual},
                {"ConstantOfShape", OpType::ConstantOfShape}, {"EyeLike", OpType::EyeLike}, {"ScatterND", OpType::ScatterND},
            };
            // ReduceType codes of the reference (Mean 0 .. L2 5); ReduceMean itself maps to GlobalAvgPool above.
            static const std::unordered_map<std::string, int32_t> reduce = {
                {"ReduceSum", 1}, {"ReduceMax", 2}, {"ReduceMin", 3}, {"ReduceProd", 4}, {"ReduceL2", 5}};
            using U = UnaryType;
            static const std::unordered_map<std::string, U> unary = {
                {"Sigmoid", U::Sigmoid}, {"Tanh", U::Tanh}, {"HardSwish", U::HardSwish}, {"HardSigmoid", U::HardSigmoid},
                {"LeakyRelu", U::LeakyRelu}, {"Elu", U::Elu}, {"Abs", U::Abs}, {"Neg", U::Neg}, {"Exp", U::Exp}, {"Log", U::Log},
                {"Sqrt", U::Sqrt}, {"Floor", U::Floor}, {"Ceil", U::Ceil}, {"Erf", U::Erf}, {"Cos", U::Cos}, {"Sin", U::Sin},
                {"Reciprocal", U::Reciprocal}, {"Softplus", U::Softplus}};
            using B = BinaryType;
            static const std::unordered_map<std::string, B> binary = {
                {"Mul", B::Mul}, {"Sub", B::Sub}, {"Div", B::Div}, {"Max", B::Max}, {"Min", B::Min}, {"Pow", B::Pow}};
            if (auto it = direct.find(s); it != direct.end()) return {it->second, 0};
            if (auto it = reduce.find(s); it != reduce.end()) return {OpType::Reduce, it->second};
            if (auto it = unary.find(s); it != unary.end()) return {OpType::Unary, (int32_t) it->second};
            if (auto it = binary.find(s); it != binary.end()) return {OpType::Binary, (int32_t) it->second};
            return {};
        }

        // NodeProto: 1 input, 2 output, 3 name, 4 op_type, 5 attribute.
        struct NodeMsg {
            Node                     node;
            std::vector<std::string> ins, outs;
        };

        NodeMsg readNode(Wire w) {
            NodeMsg     m;
            std::string opType;
            uint32_t    f;
            int         wt;
            while (w.next(f, wt)) {
                switch (f) {
                    case 1: m.ins.push_back(w.text()); break;
                    case 2: m.outs.push_back(w.text()); break;
                    case 3: m.node.name = w.text(); break;
                    case 4: opType = w.text(); break;
                    case 5: readAttr(w.sub(), m.node.attr); break;
                    default: w.skip(wt); break;
                }
            }
            Node     &n  = m.node;
            const OpMap op = mapOp(opType);
            n.type     = op.type;
            n.subOp    = op.subOp;
            if (n.type == OpType::Unary) {
                const UnaryType u = (UnaryType) n.subOp;
                if (u == UnaryType::LeakyRelu) n.actLo = n.attr.getf("alpha", 0.01f);
                else if (u == UnaryType::Elu) n.actLo = n.attr.getf("alpha", 1.0f);
                else if (u == UnaryType::HardSigmoid) {
                    n.actLo = n.attr.getf("alpha", 0.2f);
                    n.actHi = n.attr.getf("beta", 0.5f);
                }
            }
            if (n.type == OpType::Unknown) std::fprintf(stderr, "vknn: unknown ONNX op '%s' (node %s)\n", opType.c_str(), n.name.c_str());
            return m;
        }

        class Importer {
          public:
            Importer(Graph &g, std::string dir): g_(g), dir_(std::move(dir)) {}

            void graph(Wire w) {
                std::vector<TensorMsg>       inits;
                std::vector<NodeMsg>         nodes;
                std::map<std::string, Shape> hints;
                uint32_t                     f;
                int                          wt;
                while (w.next(f, wt)) {
                    if (wt != 2) { w.skip(wt); continue; }
                    switch (f) {
                        case 1: nodes.push_back(readNode(w.sub())); break;
                        case 5: inits.push_back(readTensor(w.sub())); break;
                        case 11: case 12: {
                            std::string name;
                            Shape       shape;
                            int32_t     elem = kFloat;
                            readValueInfo(w.sub(), name, shape, elem);
                            TensorId id = g_.findOrAdd(name);
                            g_.desc(id).shape = shape;
                            g_.desc(id).dtype = dtypeOfElem(elem);
                            if (f == 11) {
                                g_.desc(id).isInput = true;
                                g_.inputs.push_back(id);
                            } else {
                                g_.desc(id).isOutput = true;
                                g_.outputs.push_back(id);
                            }
                            break;
                        }
                        case 13: {
                            std::string name;
                            Shape       shape;
                            int32_t     elem = kFloat;
                            readValueInfo(w.sub(), name, shape, elem);
                            if (!name.empty() && !shape.empty()) hints[name] = shape;
                            break;
                        }
                        default: w.skip(wt); break;
                    }
                }
                std::unordered_map<std::string, TensorId> latest;
                for (TensorId id: g_.inputs) latest[g_.desc(id).name] = id;
                for (TensorMsg &t: inits) latest[t.name] = initializer(t);
                for (size_t i = 0; i < nodes.size(); ++i) {
                    Node &n = nodes[i].node;
                    for (const std::string &s: nodes[i].ins) {
                        if (s.empty()) { n.inputs.push_back(kNoTensor); continue; }
                        auto it = latest.find(s);
                        n.inputs.push_back(it != latest.end() ? it->second : g_.findOrAdd(s));
                    }
                    for (const std::string &s: nodes[i].outs) {
                        if (s.empty()) { n.outputs.push_back(kNoTensor); continue; }
                        TensorDesc d;
                        d.name = s;
                        if (auto h = hints.find(s); h != hints.end()) d.shape = h->second;
                        const TensorId id = g_.addTensor(std::move(d));
                        latest[s]         = id;
                        n.outputs.push_back(id);
                    }
                    if (n.name.empty()) n.name = std::string(opTypeName(n.type)) + "_" + std::to_string(i);
                    g_.nodes.push_back(std::move(n));
                }
                for (TensorId &o: g_.outputs) {
                    auto it = latest.find(g_.desc(o).name);
                    if (it == latest.end() || it->second == o) continue;
                    TensorDesc &last = g_.desc(it->second);
                    last.isOutput    = true;
                    last.shape       = g_.desc(o).shape;
                    last.dtype       = g_.desc(o).dtype;
                    o                = it->second;
                }
                std::vector<TensorId> real;
                for (TensorId id: g_.inputs)
                    if (!g_.isInitializer(id)) real.push_back(id);
                g_.inputs = std::move(real);
            }

          private:
            Graph                                                &g_;
            std::string                                           dir_;
            std::unordered_map<std::string, std::vector<uint8_t>> files_;

            // Point an EXTERNAL tensor's raw bytes at its slice of the data file.
            void resolveExternal(TensorMsg &t) {
                if (!t.external || t.raw) return;
                if (t.location.empty()) malformed("external tensor '" + t.name + "' has no location");
                const std::string path = dir_.empty() ? t.location : dir_ + "/" + t.location;
                auto              it   = files_.find(path);
                if (it == files_.end()) {
                    std::ifstream f(path, std::ios::binary);
                    if (!f) throw Error(Status::IoError, "cannot open external data file " + path + " (tensor '" + t.name + "')");
                    it = files_.emplace(path, std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>())).first;
                }
                const std::vector<uint8_t> &file = it->second;
                const int64_t len = t.length >= 0 ? t.length : (int64_t) file.size() - t.offset;
                // checked without adding: offset and length come from the file and may be near INT64_MAX
                if (t.offset < 0 || len < 0 || t.offset > (int64_t) file.size() || len > (int64_t) file.size() - t.offset)
                    malformed("external slice of tensor '" + t.name + "' lies outside " + path);
                t.raw  = file.data() + t.offset;
                t.rawN = (size_t) len;
            }

            TensorId initializer(TensorMsg &t) {
                resolveExternal(t);
                const TensorId id = g_.findOrAdd(t.name);
                TensorDesc    &d  = g_.desc(id);
                d.isInitializer   = true;
                d.shape           = t.dims;
                const int64_t n   = t.elems();
                HostBuffer    hb;
                if (t.dtype == kInt64) {
                    d.dtype = DType::Int64;
                    hb.resizeElems(n, DType::Int64);
                    std::vector<int64_t> v = int64Values(t, n);
                    if (n) std::memcpy(hb.i64(), v.data(), (size_t) n * 8);
                } else {
                    d.dtype = DType::Float32;
                    hb.resizeElems(n, DType::Float32);
                    std::vector<float> v = floatValues(t, n);
                    if (n) std::memcpy(hb.f32(), v.data(), (size_t) n * 4);
                }
                g_.initializers[id] = std::move(hb);
                return id;
            }
        };

    } // namespace

    Graph importOnnxBytes(const uint8_t *data, size_t size, const std::string &baseDir) {
        Graph    g;
        Wire     w {data, data + size};
        bool     found = false;
        uint32_t f;
        int      wt;
        while (w.next(f, wt)) {
            if (f == 7 && wt == 2) {
                Importer(g, baseDir).graph(w.sub());
                found = true;
            } else {
                w.skip(wt);
            }
        }
        if (!found) throw Error(Status::InvalidArgument, "no GraphProto in ONNX model");
        g.topoSort();
        return g;
    }

    Graph importOnnx(const std::string &path) {
        std::ifstream f(path, std::ios::binary);
        if (!f) throw Error(Status::IoError, "cannot open ONNX file: " + path);
        std::vector<uint8_t> buf((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
        const size_t         slash = path.find_last_of("/\\");
        return importOnnxBytes(buf.data(), buf.size(), slash == std::string::npos ? std::string() : path.substr(0, slash));
    }

} // namespace vknn
