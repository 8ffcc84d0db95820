// TEST INFRASTRUCTURE — a minimal host backend registered as BackendKind::Cpu, so tests can build
// sessions whose graphs alternate between HIP and host segments (HIP -> CPU -> HIP) and check the
// session's boundary transfers (Session::runSegments, Backend::toHost, the HIP segment's staging
// uploads) the way the reference's CPU fallback exercises them (src/core/session.cpp partitioning
// into per-backend segments, src/backend/cpu/cpu_backend.cpp). It is never part of the product:
// libvknn.so ships no CPU backend, and this library is loaded only by tests, which call
// vknn_test_cpu_backend_register() before creating a session with the option cpu_fallback=1.
//
// Ops (fp32 NCHW host tensors, plain loops): Unary (every UnaryType, parameters in actLo/actHi as
// the importer stores them), Relu, Clip (bounds from initializer inputs or min/max attributes),
// Add and Binary (same shapes), GlobalAvgPool. The math follows the ONNX operator definitions.
#include "vknn/backend.h"
#include <algorithm>
#include <cmath>
#include <cstring>

namespace {

    using namespace vknn;

    float unary(UnaryType u, float x, float a, float b) {
        switch (u) {
            case UnaryType::Sigmoid: return 1.f / (1.f + std::exp(-x));
            case UnaryType::Tanh: return std::tanh(x);
            case UnaryType::HardSwish: return x * std::min(std::max(x + 3.f, 0.f), 6.f) / 6.f;
            case UnaryType::HardSigmoid: return std::min(std::max(a * x + b, 0.f), 1.f);
            case UnaryType::LeakyRelu: return x >= 0.f ? x : a * x;
            case UnaryType::Elu: return x >= 0.f ? x : a * (std::exp(x) - 1.f);
            case UnaryType::Abs: return std::fabs(x);
            case UnaryType::Neg: return -x;
            case UnaryType::Exp: return std::exp(x);
            case UnaryType::Log: return std::log(x);
            case UnaryType::Sqrt: return std::sqrt(x);
            case UnaryType::Floor: return std::floor(x);
            case UnaryType::Ceil: return std::ceil(x);
            case UnaryType::Relu: return std::max(x, 0.f);
            case UnaryType::SiLU: return x / (1.f + std::exp(-x));
            case UnaryType::Erf: return std::erf(x);
            case UnaryType::Cos: return std::cos(x);
            case UnaryType::Sin: return std::sin(x);
            case UnaryType::Reciprocal: return 1.f / x;
            case UnaryType::Softplus: return std::log1p(std::exp(x));
            default: throw Error(Status::Unsupported, "test CPU backend: unary op");
        }
    }

    float binary(BinaryType t, float x, float y) {
        switch (t) {
            case BinaryType::Mul: return x * y;
            case BinaryType::Sub: return x - y;
            case BinaryType::Div: return x / y;
            case BinaryType::Max: return std::max(x, y);
            case BinaryType::Min: return std::min(x, y);
            case BinaryType::Pow: return std::pow(x, y);
            case BinaryType::Add: return x + y;
            default: throw Error(Status::Unsupported, "test CPU backend: binary op");
        }
    }

    class TestCpuSegment: public Segment {
      public:
        TestCpuSegment(const Graph &g): g_(g) {}

        void run(ExecContext &ctx) override {
            for (int i: nodeIdx) {
                const Node &nd = g_.nodes[i];
                RtTensor   &y  = ctx.t(nd.outputs[0]);
                y.shape        = g_.desc(nd.outputs[0]).shape;
                y.dtype        = DType::Float32;
                y.allocHost();
                y.deviceValid = false;
                float        *yo = y.host.f32();
                const int64_t n  = y.elems();
                const float  *a  = in(ctx, nd.inputs[0]);
                switch (nd.type) {
                    case OpType::Unary:
                        for (int64_t k = 0; k < n; ++k) yo[k] = unary((UnaryType) nd.subOp, a[k], nd.actLo, nd.actHi);
                        break;
                    case OpType::Relu:
                        for (int64_t k = 0; k < n; ++k) yo[k] = std::max(a[k], 0.f);
                        break;
                    case OpType::Clip: {
                        float lo = -INFINITY, hi = INFINITY;
                        if (nd.inputs.size() > 1 && nd.inputs[1] != kNoTensor) lo = in(ctx, nd.inputs[1])[0];
                        if (nd.inputs.size() > 2 && nd.inputs[2] != kNoTensor) hi = in(ctx, nd.inputs[2])[0];
                        lo = nd.attr.getf("min", lo);
                        hi = nd.attr.getf("max", hi);
                        for (int64_t k = 0; k < n; ++k) yo[k] = std::min(std::max(a[k], lo), hi);
                        break;
                    }
                    case OpType::Add: case OpType::Binary: {
                        const float *b = in(ctx, nd.inputs[1]);
                        const BinaryType t = nd.type == OpType::Add ? BinaryType::Add : (BinaryType) nd.subOp;
                        for (int64_t k = 0; k < n; ++k) yo[k] = binary(t, a[k], b[k]);
                        break;
                    }
                    case OpType::GlobalAvgPool: {
                        const Shape &s  = g_.desc(nd.inputs[0]).shape;
                        const int64_t hw = s[2] * s[3];
                        for (int64_t p = 0; p < s[0] * s[1]; ++p) {
                            double acc = 0;
                            for (int64_t k = 0; k < hw; ++k) acc += a[p * hw + k];
                            yo[p] = (float) (acc / (double) hw);
                        }
                        break;
                    }
                    default: throw Error(Status::Unsupported, std::string("test CPU backend: ") + opTypeName(nd.type));
                }
            }
        }

      private:
        const Graph &g_;

        const float *in(ExecContext &ctx, TensorId t) {
            if (g_.isInitializer(t)) return g_.initializers.at(t).f32();
            RtTensor &r = ctx.t(t);
            if (!r.hostValid) throw Error(Status::RuntimeError, "test CPU backend: input without host data: " + g_.desc(t).name);
            return r.host.f32();
        }
    };

    class TestCpuBackend: public Backend {
      public:
        BackendKind kind() const override { return BackendKind::Cpu; }
        const char *name() const override { return "CPU(test)"; }
        bool        available() const override { return true; }
        bool        supports(OpType t, DType) const override {
            return t == OpType::Unary || t == OpType::Relu || t == OpType::Clip || t == OpType::Add || t == OpType::Binary ||
                   t == OpType::GlobalAvgPool;
        }
        bool supportsNode(const Graph &g, const Node &nd, DType dt) const override {
            if (!supports(nd.type, dt) || nd.fusedAct != ActType::None || nd.fusedResidual != kNoTensor) return false;
            if (nd.type == OpType::Add || nd.type == OpType::Binary)
                return nd.inputs.size() == 2 && g.desc(nd.inputs[0]).shape == g.desc(nd.inputs[1]).shape;
            return true;
        }
        std::unique_ptr<Segment> compileSegment(const std::vector<int> &, Graph &g, const Config &) override {
            return std::unique_ptr<Segment>(new TestCpuSegment(g));
        }
    };

} // namespace

extern "C" __attribute__((visibility("default"))) int vknn_test_cpu_backend_register(void) {
    BackendRegistry::instance().registerBackend(BackendKind::Cpu, []() -> std::unique_ptr<Backend> { return std::unique_ptr<Backend>(new TestCpuBackend()); });
    return 0;
}
