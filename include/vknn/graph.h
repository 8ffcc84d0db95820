// The graph IR (backend-agnostic; every tensor is logically NCHW). Mirrors the reference's
// Graph (include/vknn/graph.h:11-41): tensors indexed by TensorId, topologically ordered nodes,
// name lookup, graph inputs/outputs and initializer host data keyed by tensor id.
#pragma once
#include "vknn/types.h"
#include <map>
#include <string>
#include <vector>

namespace vknn {

    class Graph {
      public:
        std::vector<TensorDesc>         tensors;
        std::vector<Node>               nodes;
        std::map<std::string, TensorId> tensorByName;
        std::vector<TensorId>           inputs;
        std::vector<TensorId>           outputs;
        std::map<TensorId, HostBuffer>  initializers;

        TensorId findOrAdd(const std::string &name);
        TensorId find(const std::string &name) const;
        TensorId addTensor(TensorDesc d);
        bool     isInitializer(TensorId id) const { return initializers.count(id) > 0; }

        const TensorDesc &desc(TensorId id) const { return tensors[id]; }
        TensorDesc       &desc(TensorId id) { return tensors[id]; }

        // Stable topological sort of nodes by tensor dependencies. Throws on a cycle.
        void        topoSort();
        std::string dump() const;
    };

    // ONNX import (reference include/vknn/graph.h:42): the graph of an ONNX model file as the
    // reference's importer builds it, before any pass. Weights stored outside the model are read
    // relative to the model's folder. Throws Error(IoError) for an unreadable file and
    // Error(InvalidArgument) for a malformed one.
    Graph importOnnx(const std::string &path);
    // The same from an in-memory ModelProto; `baseDir` resolves external weight files.
    Graph importOnnxBytes(const uint8_t *data, size_t size, const std::string &baseDir = "");

    // The ".vxm" model file (reference include/vknn/graph.h:46-47, src/core/model_io.cpp): an
    // optimized graph with its weights in the reference's VXM2 byte layout. load returns false on
    // a missing, foreign, truncated or inconsistent file and then says why in `why`.
    bool                 saveGraphBin(const Graph &g, const std::string &path);
    bool                 loadGraphBin(Graph &g, const std::string &path, std::string *why = nullptr);
    std::vector<uint8_t> serializeGraphBin(const Graph &g);
    bool                 parseGraphBin(Graph &g, const uint8_t *data, size_t size, std::string *why = nullptr);

} // namespace vknn
