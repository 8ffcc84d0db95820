// The ".vxm" model file: an optimized graph (after import and the standard passes) with its
// weights, so a reload skips parsing and passes. The byte layout is the reference's "VXM2" format
// (src/core/model_io.cpp:14-230), kept identical so files move between the two builds:
//
//   u32 magic 0x324d5856 ("VXM2", little endian)
//   u32 nTensors { str name | vec<i64> shape | u32 dtype | u32 format | u32 flags (1 in, 2 out, 4 init) }
//   u32 nNodes   { u32 type | str name | vec<i32> inputs | vec<i32> outputs | u32 fusedAct |
//                  f32 actLo | f32 actHi | i64 subOp | i64 fusedResidual | i64 fusedBias |
//                  u32 nAttr { str key | u32 kind | i64 i | f32 f | vec<i64> ints | vec<f32> floats | str s } }
//   vec<i32> graph inputs | vec<i32> graph outputs
//   u32 nInit    { i64 tensor id | vec<u8> bytes }
// where str = u32 length + bytes and vec<T> = u32 count + count * sizeof(T) bytes. Enumerator
// values (OpType, DType, TensorFormat, ActType, Attr::Kind) are the reference's.
//
// Reading is done from one in-memory copy of the file with a bounds check on every field, and
// the loaded graph is validated (tensor ids in range, initializer sizes match their shapes), so
// a truncated or corrupt file is rejected instead of producing a half-filled graph.
#include "vknn/graph.h"
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>

namespace vknn {

    namespace {
        constexpr uint32_t kVxm2 = 0x324d5856u;

        struct Out {
            std::vector<uint8_t> b;
            void raw(const void *p, size_t n) {
                const uint8_t *c = (const uint8_t *) p;
                b.insert(b.end(), c, c + n);
            }
            void u32(uint32_t v) { raw(&v, 4); }
            void i64(int64_t v) { raw(&v, 8); }
            void f32(float v) { raw(&v, 4); }
            void str(const std::string &s) {
                u32((uint32_t) s.size());
                raw(s.data(), s.size());
            }
            template <typename T> void vec(const std::vector<T> &v) {
                u32((uint32_t) v.size());
                raw(v.data(), v.size() * sizeof(T));
            }
        };

        struct In {
            const uint8_t *p;
            size_t         n, off = 0;
            bool           ok = true;
            bool take(void *dst, size_t k) {
                if (!ok || k > n - off) return ok = false;
                std::memcpy(dst, p + off, k);
                off += k;
                return true;
            }
            uint32_t u32() {
                uint32_t v = 0;
                take(&v, 4);
                return v;
            }
            int64_t i64() {
                int64_t v = 0;
                take(&v, 8);
                return v;
            }
            float f32() {
                float v = 0;
                take(&v, 4);
                return v;
            }
            std::string str() {
                uint32_t k = u32();
                if (!ok || k > n - off) {
                    ok = false;
                    return {};
                }
                std::string s((const char *) p + off, k);
                off += k;
                return s;
            }
            template <typename T> std::vector<T> vec() {
                uint32_t k = u32();
                if (!ok || (size_t) k > (n - off) / sizeof(T)) {
                    ok = false;
                    return {};
                }
                std::vector<T> v(k);
                take(v.data(), (size_t) k * sizeof(T));
                return v;
            }
        };

        bool validId(const Graph &g, int64_t id, bool allowNone) {
            return (allowNone && id == kNoTensor) || (id >= 0 && id < (int64_t) g.tensors.size());
        }
    } // namespace

    std::vector<uint8_t> serializeGraphBin(const Graph &g) {
        Out w;
        w.u32(kVxm2);
        w.u32((uint32_t) g.tensors.size());
        for (const TensorDesc &t: g.tensors) {
            w.str(t.name);
            w.vec(t.shape);
            w.u32((uint32_t) t.dtype);
            w.u32((uint32_t) t.format);
            w.u32((t.isInput ? 1u : 0u) | (t.isOutput ? 2u : 0u) | (t.isInitializer ? 4u : 0u));
        }
        w.u32((uint32_t) g.nodes.size());
        for (const Node &nd: g.nodes) {
            w.u32((uint32_t) nd.type);
            w.str(nd.name);
            w.vec(nd.inputs);
            w.vec(nd.outputs);
            w.u32((uint32_t) nd.fusedAct);
            w.f32(nd.actLo);
            w.f32(nd.actHi);
            w.i64(nd.subOp);
            w.i64(nd.fusedResidual);
            w.i64(nd.fusedBias);
            w.u32((uint32_t) nd.attr.map.size());
            for (const auto &kv: nd.attr.map) {
                w.str(kv.first);
                w.u32((uint32_t) kv.second.kind);
                w.i64(kv.second.i);
                w.f32(kv.second.f);
                w.vec(kv.second.ints);
                w.vec(kv.second.floats);
                w.str(kv.second.str);
            }
        }
        w.vec(g.inputs);
        w.vec(g.outputs);
        w.u32((uint32_t) g.initializers.size());
        for (const auto &kv: g.initializers) {
            w.i64(kv.first);
            w.vec(kv.second.bytes);
        }
        return std::move(w.b);
    }

    bool parseGraphBin(Graph &out, const uint8_t *data, size_t size, std::string *why) {
        auto bad = [&](const std::string &m) {
            if (why) *why = m;
            return false;
        };
        In r {data, size};
        if (r.u32() != kVxm2 || !r.ok) return bad("bad magic (not a VXM2 file)");
        Graph    g;
        uint32_t nt = r.u32();
        if (!r.ok || nt > size / 20) return bad("tensor count out of range");
        g.tensors.resize(nt);
        for (uint32_t i = 0; i < nt && r.ok; ++i) {
            TensorDesc &t = g.tensors[i];
            t.name        = r.str();
            t.shape       = r.vec<int64_t>();
            uint32_t dt = r.u32(), fmt = r.u32(), fl = r.u32();
            if (dt > (uint32_t) DType::Int64) return bad("tensor " + t.name + ": unknown dtype");
            t.dtype         = (DType) dt;
            t.format        = (TensorFormat) fmt;
            t.isInput       = fl & 1;
            t.isOutput      = fl & 2;
            t.isInitializer = fl & 4;
            if (!t.name.empty()) g.tensorByName[t.name] = (TensorId) i;
        }
        uint32_t nn = r.u32();
        if (!r.ok || nn > size / 40) return bad("node count out of range");
        g.nodes.resize(nn);
        for (uint32_t i = 0; i < nn && r.ok; ++i) {
            Node &nd         = g.nodes[i];
            nd.type          = (OpType) r.u32();
            nd.name          = r.str();
            nd.inputs        = r.vec<TensorId>();
            nd.outputs       = r.vec<TensorId>();
            nd.fusedAct      = (ActType) r.u32();
            nd.actLo         = r.f32();
            nd.actHi         = r.f32();
            nd.subOp         = (int32_t) r.i64();
            nd.fusedResidual = (TensorId) r.i64();
            nd.fusedBias     = (TensorId) r.i64();
            uint32_t na      = r.u32();
            for (uint32_t a = 0; a < na && r.ok; ++a) {
                std::string k = r.str();
                Attr        at;
                at.kind   = (Attr::Kind) r.u32();
                at.i      = r.i64();
                at.f      = r.f32();
                at.ints   = r.vec<int64_t>();
                at.floats = r.vec<float>();
                at.str    = r.str();
                nd.attr.map[k] = std::move(at);
            }
        }
        g.inputs    = r.vec<TensorId>();
        g.outputs   = r.vec<TensorId>();
        uint32_t ni = r.u32();
        for (uint32_t i = 0; i < ni && r.ok; ++i) {
            int64_t    id = r.i64();
            HostBuffer hb;
            hb.bytes = r.vec<uint8_t>();
            if (r.ok && !validId(g, id, false)) return bad("initializer for unknown tensor id " + std::to_string(id));
            g.initializers[(TensorId) id] = std::move(hb);
        }
        if (!r.ok) return bad("truncated file");
        // structural checks: every id refers to a tensor, initializers hold their shape's bytes
        for (const Node &nd: g.nodes) {
            for (TensorId t: nd.inputs)
                if (!validId(g, t, true)) return bad("node " + nd.name + ": input id out of range");
            for (TensorId t: nd.outputs)
                if (!validId(g, t, false)) return bad("node " + nd.name + ": output id out of range");
            if (!validId(g, nd.fusedResidual, true) || !validId(g, nd.fusedBias, true)) return bad("node " + nd.name + ": fused id out of range");
        }
        for (TensorId t: g.inputs)
            if (!validId(g, t, false)) return bad("graph input id out of range");
        for (TensorId t: g.outputs)
            if (!validId(g, t, false)) return bad("graph output id out of range");
        for (const auto &kv: g.initializers) {
            const TensorDesc &t = g.tensors[kv.first];
            int64_t           e = 1;
            for (int64_t d: t.shape) e *= d;
            if (!t.shape.empty() && (size_t) e * dtypeSize(t.dtype) != kv.second.bytes.size())
                return bad("initializer " + t.name + ": " + std::to_string(kv.second.bytes.size()) + " bytes for its shape");
        }
        out = std::move(g);
        return true;
    }

    bool saveGraphBin(const Graph &g, const std::string &path) {
        std::vector<uint8_t> b = serializeGraphBin(g);
        std::ofstream        f(path, std::ios::binary | std::ios::trunc);
        if (!f) return false;
        f.write((const char *) b.data(), (std::streamsize) b.size());
        return (bool) f;
    }

    bool loadGraphBin(Graph &g, const std::string &path, std::string *why) {
        std::ifstream f(path, std::ios::binary);
        if (!f) {
            if (why) *why = "cannot open " + path;
            return false;
        }
        std::vector<uint8_t> b((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
        return parseGraphBin(g, b.data(), b.size(), why);
    }

} // namespace vknn
