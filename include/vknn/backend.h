// The pluggable-backend contract: ExecContext, Segment, Backend, BackendRegistry and the
// self-registration macro, plus the per-op profiler records. Mirrors the reference's
// backend_class.h:15-47, segment.h:12-23, backend_registry.h:12-32, exec_context.h:13-21,
// op_record.h:10-15 and profiler_class.h:10-38.
#pragma once
#include "vknn/config.h"
#include "vknn/graph.h"
#include "vknn/rt_tensor.h"
#include <array>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace vknn {

    struct OpRecord {
        std::string             name;
        OpType                  type = OpType::Unknown;
        std::string             backend;
        double                  cpuMs    = 0.0;
        double                  gpuMs    = -1.0;
        std::array<uint32_t, 3> dispatch = {0, 0, 0};
        int64_t                 bytesIO  = 0;
        bool                    fellBack = false;
        double                  flops    = 0.0; // algorithmic FLOPs of the op (HIP backend fills it)
    };

    class Profiler {
      public:
        void setEnabled(bool e) { enabled_ = e; }
        bool enabled() const { return enabled_; }
        void clear() { records_.clear(); }
        void add(const OpRecord &r) {
            if (enabled_) records_.push_back(r);
        }
        const std::vector<OpRecord> &records() const { return records_; }
        std::vector<OpRecord>       &records() { return records_; }
        void                         printTable() const;
        std::string                  toJson() const;
        double                       totalCpuMs() const;
        double                       totalGpuMs() const;

      private:
        bool                  enabled_ = false;
        std::vector<OpRecord> records_;
    };

    struct ExecContext {
        std::vector<RtTensor> *pool     = nullptr;
        const Graph           *graph    = nullptr;
        const Config          *config   = nullptr;
        Profiler              *profiler = nullptr;
        RtTensor              &t(TensorId id) { return (*pool)[id]; }
    };

    class Backend;

    class Segment {
      public:
        virtual ~Segment()                 = default;
        virtual void run(ExecContext &ctx) = 0;
        Backend     *backend               = nullptr;
        bool         isFallback            = false;
        std::vector<int>      nodeIdx;
        std::vector<TensorId> boundaryInputs;
        std::vector<TensorId> boundaryOutputs;
    };

    class Backend {
      public:
        virtual ~Backend()                                   = default;
        virtual BackendKind kind() const                     = 0;
        virtual const char *name() const                     = 0;
        virtual bool        available() const                = 0;
        virtual void        configure(const Config &) {}
        virtual bool        supports(OpType t, DType dt) const = 0;
        virtual bool        supportsNode(const Graph &, const Node &nd, DType dt) const { return supports(nd.type, dt); }
        virtual void        toHost(RtTensor &, ExecContext &) {}
        virtual void        toDevice(RtTensor &, ExecContext &) {}
        virtual std::unique_ptr<Segment> compileSegment(const std::vector<int> &nodeIdx, Graph &g, const Config &cfg) = 0;
        virtual void        finalize() {}
    };

    class BackendRegistry {
      public:
        using Factory = std::function<std::unique_ptr<Backend>()>;
        static BackendRegistry  &instance();
        void                     registerBackend(BackendKind k, Factory f);
        bool                     has(BackendKind k) const;
        std::unique_ptr<Backend> create(BackendKind k) const;

      private:
        std::map<BackendKind, Factory> factories_;
    };

    struct BackendRegistrar {
        BackendRegistrar(BackendKind k, BackendRegistry::Factory f) { BackendRegistry::instance().registerBackend(k, std::move(f)); }
    };

#define VKNN_REGISTER_BACKEND(KIND, TYPE)                                                                   \
    static ::vknn::BackendRegistrar _vx_backend_reg_##TYPE(KIND, []() -> std::unique_ptr<::vknn::Backend> { \
        return std::unique_ptr<::vknn::Backend>(new TYPE());                                                \
    })

} // namespace vknn
