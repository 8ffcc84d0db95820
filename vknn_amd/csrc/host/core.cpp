// Core support of the vknn host library: Graph helpers (name lookup, stable topological sort),
// op names, the backend registry, config string helpers and the profiler. Behaviour follows the
// reference's src/core/graph.cpp:9-110, backend_registry.cpp:1-25, config.cpp:19-60 and
// profiler.cpp:30-116.
#include "vknn/backend.h"
#include "vknn/config.h"
#include "vknn/graph.h"
#include <algorithm>
#include <cstdio>
#include <sstream>
#include <unordered_map>

namespace vknn {

    TensorId Graph::find(const std::string &name) const {
        auto it = tensorByName.find(name);
        return it == tensorByName.end() ? kNoTensor : it->second;
    }

    TensorId Graph::findOrAdd(const std::string &name) {
        TensorId id = find(name);
        if (id != kNoTensor) return id;
        TensorDesc d;
        d.name = name;
        return addTensor(std::move(d));
    }

    TensorId Graph::addTensor(TensorDesc d) {
        TensorId id = (TensorId) tensors.size();
        if (!d.name.empty()) tensorByName[d.name] = id;
        tensors.push_back(std::move(d));
        return id;
    }

    // Kahn's algorithm; among ready nodes the lowest original index goes first (stable).
    void Graph::topoSort() {
        const int                     n = (int) nodes.size();
        std::unordered_map<int, int>  producer;
        for (int i = 0; i < n; ++i)
            for (TensorId o: nodes[i].outputs)
                if (o != kNoTensor) producer[o] = i;
        std::vector<std::vector<int>> succ(n);
        std::vector<int>              indeg(n, 0);
        for (int i = 0; i < n; ++i) {
            std::vector<int> preds;
            for (TensorId t: nodes[i].inputs) {
                auto it = producer.find(t);
                if (it != producer.end() && it->second != i) preds.push_back(it->second);
            }
            std::sort(preds.begin(), preds.end());
            preds.erase(std::unique(preds.begin(), preds.end()), preds.end());
            for (int p: preds) {
                succ[p].push_back(i);
                ++indeg[i];
            }
        }
        std::vector<int> ready;
        for (int i = 0; i < n; ++i)
            if (!indeg[i]) ready.push_back(i);
        std::vector<Node> out;
        out.reserve(n);
        while (!ready.empty()) {
            auto it = std::min_element(ready.begin(), ready.end());
            int  i  = *it;
            ready.erase(it);
            out.push_back(nodes[i]);
            for (int s: succ[i])
                if (--indeg[s] == 0) ready.push_back(s);
        }
        if ((int) out.size() != n) throw Error(Status::InvalidArgument, "graph has a cycle");
        nodes = std::move(out);
    }

    std::string Graph::dump() const {
        std::ostringstream os;
        for (const Node &nd: nodes) {
            os << opTypeName(nd.type) << " '" << nd.name << "' in=";
            for (TensorId t: nd.inputs) os << t << (t >= 0 ? shapeStr(tensors[t].shape) : "") << " ";
            os << "out=";
            for (TensorId t: nd.outputs) os << t << (t >= 0 ? shapeStr(tensors[t].shape) : "") << " ";
            os << "act=" << (int) nd.fusedAct << " res=" << nd.fusedResidual << "\n";
        }
        return os.str();
    }

    const char *opTypeName(OpType t) {
        static const char *names[] = {
            "Unknown", "Conv", "ConvTranspose", "Clip", "Relu", "Add", "GlobalAveragePool", "AveragePool", "MaxPool", "Gemm", "MatMul",
            "Einsum", "Reshape", "Expand", "Tile", "Squeeze", "Flatten", "Softmax", "LayerNormalization", "BatchNormalization", "Concat", "Pad",
            "Identity", "Constant", "Shape", "Gather", "Unsqueeze", "Unary", "Binary", "PRelu", "Resize", "GridSample",
            "Transpose", "Slice", "Reduce", "DepthToSpace", "Cast", "Split", "Where", "Equal", "Greater", "GreaterEqual",
            "ConstantOfShape", "EyeLike", "ScatterND", "FusedSE", "FusedDwPw", "FusedPointwise", "ConvertLayout", "ConvertDtype"};
        int i = (int) t;
        return (i >= 0 && i < (int) (sizeof(names) / sizeof(names[0]))) ? names[i] : "?";
    }

    // ---------------------------------------------------------------- registry
    BackendRegistry &BackendRegistry::instance() {
        static BackendRegistry r;
        return r;
    }
    void BackendRegistry::registerBackend(BackendKind k, Factory f) { factories_[k] = std::move(f); }
    bool BackendRegistry::has(BackendKind k) const { return factories_.count(k) > 0; }
    std::unique_ptr<Backend> BackendRegistry::create(BackendKind k) const {
        auto it = factories_.find(k);
        return it == factories_.end() ? nullptr : it->second();
    }

    // ---------------------------------------------------------------- config strings
    static std::string lower(std::string s) {
        for (auto &c: s) c = (char) std::tolower((unsigned char) c);
        return s;
    }
    const char *backendName(BackendKind k) {
        switch (k) {
            case BackendKind::Vulkan: return "Vulkan";
            case BackendKind::Cpu: return "CPU";
            case BackendKind::Hip: return "HIP";
        }
        return "?";
    }
    BackendKind backendFromStr(const std::string &s) {
        std::string l = lower(s);
        if (l == "vulkan" || l == "gpu") return BackendKind::Vulkan;
        if (l == "hip" || l == "rocm") return BackendKind::Hip;
        return BackendKind::Cpu;
    }
    Precision precisionFromStr(const std::string &s) {
        std::string l = lower(s);
        if (l == "normal" || l == "mixed") return Precision::Normal;
        if (l == "high" || l == "fp32") return Precision::High;
        return Precision::Low;
    }
    Mode winogradFromStr(const std::string &s) {
        std::string l = lower(s);
        return l == "on" ? Mode::On : (l == "off" ? Mode::Off : Mode::Auto);
    }
    Mode tuningFromStr(const std::string &s) {
        std::string l = lower(s);
        return l == "off" ? Mode::NoTune : (l == "thorough" ? Mode::Thorough : Mode::Fast);
    }

    // ---------------------------------------------------------------- profiler
    double Profiler::totalCpuMs() const {
        double s = 0;
        for (auto &r: records_) s += r.cpuMs;
        return s;
    }
    double Profiler::totalGpuMs() const {
        double s = 0;
        for (auto &r: records_)
            if (r.gpuMs > 0) s += r.gpuMs;
        return s;
    }
    void Profiler::printTable() const {
        std::vector<OpRecord> v = records_;
        std::sort(v.begin(), v.end(), [](const OpRecord &a, const OpRecord &b) { return a.gpuMs > b.gpuMs; });
        std::printf("%-32s %-14s %-6s %10s %10s\n", "op", "type", "be", "gpu_ms", "TFLOP/s");
        for (auto &r: v)
            std::printf("%-32s %-14s %-6s %10.4f %10.2f\n", r.name.c_str(), opTypeName(r.type), r.backend.c_str(), r.gpuMs,
                        r.gpuMs > 0 ? r.flops / (r.gpuMs * 1e9) : 0.0);
    }
    std::string Profiler::toJson() const {
        std::ostringstream os;
        os << "[";
        for (size_t i = 0; i < records_.size(); ++i) {
            const OpRecord &r = records_[i];
            os << (i ? "," : "") << "{\"name\":\"" << r.name << "\",\"type\":\"" << opTypeName(r.type) << "\",\"backend\":\""
               << r.backend << "\",\"cpu_ms\":" << r.cpuMs << ",\"gpu_ms\":" << r.gpuMs << ",\"flops\":" << r.flops
               << ",\"bytes\":" << r.bytesIO << "}";
        }
        os << "]";
        return os.str();
    }

} // namespace vknn
