// Session: owns the planned graph, the chosen backend(s) and the tensor pool. Mirrors the
// reference Session (session_class.h:18-85) and IOTensor (io_tensor.h:15-31): create from an
// in-memory graph, run with named host tensors.
#pragma once
#include "vknn/backend.h"
#include "vknn/passes.h"
#include <memory>
#include <string>
#include <vector>

namespace vknn {

    struct IOTensor {
        std::string          name;
        Shape                shape;
        DType                dtype        = DType::Float32;
        int                  dmaBufFd     = -1;
        TensorFormat         dmaBufFormat = TensorFormat::NCHW;
        DType                dmaBufDtype  = DType::Float32;
        std::vector<uint8_t> data;
        float               *f32() { return reinterpret_cast<float *>(data.data()); }
        const float         *f32() const { return reinterpret_cast<const float *>(data.data()); }
    };

    struct IOInfo {
        std::string  name;
        Shape        shape;
        DType        dtype        = DType::Float32;
        int64_t      elems        = 0;
        int64_t      deviceBytes  = 0;
        TensorFormat deviceFormat = TensorFormat::NCHW;
        DType        deviceDtype  = DType::Float32;
    };

    class Session {
      public:
        ~Session();
        // Build from an already-imported graph (the entry point the reference's tests use). The
        // standard passes run first; `passOpt` overrides the default pass options.
        static std::unique_ptr<Session> create(Graph &&g, const Config &cfg);
        static std::unique_ptr<Session> create(Graph &&g, const Config &cfg, const PassOptions &passOpt);
        // Import an ONNX model (importOnnx) and build a session from it; an empty cfg.cacheFile
        // becomes "<model path without extension>.cache" (reference session.cpp:123-131).
        static std::unique_ptr<Session> createFromOnnx(const std::string &path, const Config &cfg);
        // Load a pre-optimized ".vxm" graph: the passes are already applied and do not run again.
        // An empty cfg.cacheFile becomes "<model path without extension>.cache" (reference
        // session.cpp:133-155). Throws Error(RuntimeError) when the file cannot be loaded.
        static std::unique_ptr<Session> createFromVxm(const std::string &path, const Config &cfg);
        // Write the planned (post-pass) graph and its weights as ".vxm" (reference session.cpp:157-159).
        // Needs the host weights, so it fails once they were released (cfg.freeWeightsAfterUpload).
        bool saveOptimized(const std::string &path) const;

        Status run(const std::vector<IOTensor> &inputs, std::vector<IOTensor> &outputs);
        Status run(const std::vector<std::vector<float>> &inputData, std::vector<IOTensor> &outputs);
        std::vector<float> infer(const std::vector<float> &input);

        std::vector<IOInfo> inputInfo() const;
        std::vector<IOInfo> outputInfo() const;

        const Graph  &graph() const { return graph_; }
        const Config &config() const { return cfg_; }
        Profiler     &profiler() { return profiler_; }
        std::vector<BackendKind> nodeBackends() const;
        const RtTensor          *tensor(const std::string &name) const;

        // Direct access to the runtime pool and segments, used by the C API to bind device-resident
        // inputs and to run segments without host round trips.
        std::vector<RtTensor>                 &pool() { return pool_; }
        std::vector<std::unique_ptr<Segment>> &segments() { return segments_; }
        Status                                 runSegments();
        // Message of the exception behind the last non-Ok status of run()/runSegments().
        const std::string                     &lastError() const { return lastError_; }

      private:
        Session() = default;
        void plan(const PassOptions &opt);

        Graph    graph_;
        Config   cfg_;
        bool     graphOptimized_ = false; // loaded from .vxm: passes already baked in
        bool     weightsReleased_ = false;
        Profiler profiler_;
        std::vector<std::unique_ptr<Backend>> backends_;
        std::map<BackendKind, Backend *>      byKind_;
        std::vector<int>                      nodeBackendIdx_;
        std::vector<std::unique_ptr<Segment>> segments_;
        std::vector<RtTensor>                 pool_;
        std::string                           lastError_;
    };

} // namespace vknn
