// A complete, deterministic text form of a Graph — every tensor the nodes or the graph reference
// (id, name, shape, dtype, role), every initializer (byte count and FNV-1a hash of its bytes) and
// every node (type, name, sub-op, fused fields, inputs, outputs, attributes with floats as bit
// patterns). Two graphs print the same text exactly when an importer built the same graph, so
// comparing texts checks an import node for node. Uses only the Graph API, and so compiles against
// this build's headers and the reference's alike.
#pragma once
#include "vknn/graph.h"
#include <cstdio>
#include <cstring>
#include <string>

namespace vknn_text {

    inline std::string hexf(float f) {
        uint32_t b;
        std::memcpy(&b, &f, 4);
        char s[16];
        std::snprintf(s, sizeof s, "%08x", b);
        return s;
    }

    inline std::string shape(const vknn::Shape &s) {
        std::string o = "[";
        for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
        return o + "]";
    }

    inline std::string tensor(const vknn::Graph &g, vknn::TensorId t) {
        if (t == vknn::kNoTensor) return "-";
        return "#" + std::to_string(t) + ":" + g.tensors[t].name;
    }

    inline std::string graph(const vknn::Graph &g) {
        std::string o;
        for (size_t t = 0; t < g.tensors.size(); ++t) {
            const auto &d = g.tensors[t];
            o += "tensor #" + std::to_string(t) + " " + d.name + " " + shape(d.shape) + " dtype=" + std::to_string((int) d.dtype) +
                 " in=" + std::to_string((int) d.isInput) + " out=" + std::to_string((int) d.isOutput) + " init=" + std::to_string((int) d.isInitializer) + "\n";
        }
        for (auto t: g.inputs) o += "input " + tensor(g, t) + "\n";
        for (auto t: g.outputs) o += "output " + tensor(g, t) + "\n";
        for (const auto &kv: g.initializers) {
            uint64_t h = 1469598103934665603ull;
            for (uint8_t c: kv.second.bytes) h = (h ^ c) * 1099511628211ull;
            char hs[24];
            std::snprintf(hs, sizeof hs, "%016llx", (unsigned long long) h);
            o += "init " + tensor(g, kv.first) + " bytes=" + std::to_string(kv.second.bytes.size()) + " fnv=" + hs + "\n";
        }
        for (const auto &n: g.nodes) {
            o += "node " + std::string(vknn::opTypeName(n.type)) + " '" + n.name + "' sub=" + std::to_string(n.subOp) + " act=" +
                 std::to_string((int) n.fusedAct) + " lo=" + hexf(n.actLo) + " hi=" + hexf(n.actHi) + " res=" + tensor(g, n.fusedResidual) +
                 " bias=" + tensor(g, n.fusedBias) + " in=";
            for (auto t: n.inputs) o += tensor(g, t) + ";";
            o += " out=";
            for (auto t: n.outputs) o += tensor(g, t) + ";";
            for (const auto &kv: n.attr.map) {
                const auto &a = kv.second;
                o += " " + kv.first + "(" + std::to_string((int) a.kind) + ")=i" + std::to_string(a.i) + ",f" + hexf(a.f) + ",s'" + a.str + "',ints";
                for (auto v: a.ints) o += ":" + std::to_string(v);
                o += ",floats";
                for (auto v: a.floats) o += ":" + hexf(v);
                o += ",shape" + shape(a.shape);
            }
            o += "\n";
        }
        return o;
    }

} // namespace vknn_text
