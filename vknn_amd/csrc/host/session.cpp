// Session planner and runner. Same contract as the reference Session (src/core/session.cpp):
// plan = standard passes -> topological order -> backends in priority order (cfg.backend, then
// cfg.fallback, then CPU only when allowCpuFallback) -> per-node assignment to the first backend
// whose supportsNode accepts it (else Unsupported) -> maximal same-backend runs become segments ->
// boundary input/output sets -> host weights released. run = bind host inputs, run segments in
// order, bring graph outputs to the host.
#include "vknn/runtime.h"
#include "vknn/session.h"
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <set>
#include <string>

namespace vknn {

    Session::~Session() {
        segments_.clear();
        pool_.clear();
        backends_.clear();
    }

    std::unique_ptr<Session> Session::create(Graph &&g, const Config &cfg) {
        PassOptions opt;
        opt.fuseDwPw          = cfg.fuseDwPw;
        opt.fuseSqueezeExcite = cfg.fuseSqueezeExcite;
        const char *auto_se   = std::getenv("VKNN_HIP_AUTO_SE");
        if (cfg.backend == BackendKind::Hip && cfg.hipAutoSE && !(auto_se && std::string(auto_se) == "0")) opt.fuseSqueezeExcite = true;
        const char *auto_dwpw = std::getenv("VKNN_HIP_AUTO_DWPW");
        if (cfg.backend == BackendKind::Hip && cfg.hipAutoDwPw && !(auto_dwpw && std::string(auto_dwpw) == "0")) opt.fuseDwPw = true;
        return create(std::move(g), cfg, opt);
    }

    std::unique_ptr<Session> Session::create(Graph &&g, const Config &cfg, const PassOptions &opt) {
        std::unique_ptr<Session> s(new Session());
        s->graph_ = std::move(g);
        s->cfg_   = cfg;
        s->plan(opt);
        return s;
    }

    std::unique_ptr<Session> Session::createFromOnnx(const std::string &path, const Config &cfg) {
        Config c = cfg;
        if (c.cacheFile.empty()) c.cacheFile = Runtime::defaultCacheFile(path);
        return create(importOnnx(path), c);
    }

    std::unique_ptr<Session> Session::createFromVxm(const std::string &path, const Config &cfg) {
        Graph       g;
        std::string why;
        if (!loadGraphBin(g, path, &why)) throw Error(Status::RuntimeError, "failed to load .vxm " + path + ": " + why);
        std::unique_ptr<Session> s(new Session());
        s->graph_          = std::move(g);
        s->cfg_            = cfg;
        s->graphOptimized_ = true;
        if (s->cfg_.cacheFile.empty()) {
            const size_t slash = path.find_last_of("/\\"), dot = path.find_last_of('.');
            const bool   ext   = dot != std::string::npos && (slash == std::string::npos || dot > slash);
            s->cfg_.cacheFile  = (ext ? path.substr(0, dot) : path) + ".cache";
        }
        s->plan(PassOptions {});
        return s;
    }

    bool Session::saveOptimized(const std::string &path) const {
        if (weightsReleased_) return false;
        return saveGraphBin(graph_, path);
    }

    void Session::plan(const PassOptions &opt) {
        if (!graphOptimized_) runStandardPasses(graph_, opt);
        graph_.topoSort();

        std::vector<BackendKind> order = {cfg_.backend};
        for (BackendKind k: cfg_.fallback) order.push_back(k);
        if (cfg_.allowCpuFallback) order.push_back(BackendKind::Cpu);
        std::set<BackendKind> seen;
        for (BackendKind k: order) {
            if (!seen.insert(k).second || !BackendRegistry::instance().has(k)) continue;
            auto b = BackendRegistry::instance().create(k);
            if (!b || !b->available()) continue;
            byKind_[k] = b.get();
            backends_.push_back(std::move(b));
        }
        if (backends_.empty()) throw Error(Status::RuntimeError, std::string("no usable backend (requested ") + backendName(cfg_.backend) + ")");

        pool_.resize(graph_.tensors.size());
        for (size_t i = 0; i < pool_.size(); ++i) {
            pool_[i].id    = (TensorId) i;
            pool_[i].shape = graph_.tensors[i].shape;
            pool_[i].dtype = graph_.tensors[i].dtype;
        }

        for (auto &b: backends_) b->configure(cfg_);
        nodeBackendIdx_.assign(graph_.nodes.size(), -1);
        for (size_t n = 0; n < graph_.nodes.size(); ++n) {
            const Node &nd = graph_.nodes[n];
            for (size_t bi = 0; bi < backends_.size(); ++bi)
                if (backends_[bi]->supportsNode(graph_, nd, DType::Float32)) {
                    nodeBackendIdx_[n] = (int) bi;
                    break;
                }
            if (nodeBackendIdx_[n] < 0)
                throw Error(Status::Unsupported, std::string("no backend supports op ") + opTypeName(nd.type) + " (" + nd.name + ")");
        }

        // maximal runs of consecutive nodes on the same backend
        std::vector<std::vector<int>> runs;
        for (size_t n = 0; n < graph_.nodes.size(); ++n) {
            if (runs.empty() || nodeBackendIdx_[runs.back().back()] != nodeBackendIdx_[n]) runs.emplace_back();
            runs.back().push_back((int) n);
        }
        for (auto &r: runs) {
            Backend *be = backends_[nodeBackendIdx_[r[0]]].get();
            std::set<TensorId> produced, consumed;
            for (int i: r) {
                for (TensorId t: graph_.nodes[i].outputs)
                    if (t != kNoTensor) produced.insert(t);
                for (TensorId t: graph_.nodes[i].inputs)
                    if (t != kNoTensor && !graph_.isInitializer(t)) consumed.insert(t);
            }
            std::vector<TensorId> bin, bout;
            for (TensorId t: consumed)
                if (!produced.count(t)) bin.push_back(t);
            std::set<TensorId> usedOutside(graph_.outputs.begin(), graph_.outputs.end());
            for (size_t n = 0; n < graph_.nodes.size(); ++n) {
                if (std::find(r.begin(), r.end(), (int) n) != r.end()) continue;
                for (TensorId t: graph_.nodes[n].inputs) usedOutside.insert(t);
            }
            for (TensorId t: produced)
                if (usedOutside.count(t)) bout.push_back(t);
            // the boundary sets are attached once compileSegment returns; the segment reads them
            // when it first runs (staging buffers are sized then)
            auto seg = be->compileSegment(r, graph_, cfg_);
            seg->backend         = be;
            seg->nodeIdx         = r;
            seg->boundaryInputs  = bin;
            seg->boundaryOutputs = bout;
            seg->isFallback      = be->kind() != cfg_.backend;
            segments_.push_back(std::move(seg));
        }
        for (auto &b: backends_) b->finalize();
        if (cfg_.freeWeightsAfterUpload) {
            std::set<TensorId> keep;
            for (const Node &nd: graph_.nodes)
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor && graph_.isInitializer(t) && numElements(graph_.desc(t).shape) <= 4) keep.insert(t);
            for (auto it = graph_.initializers.begin(); it != graph_.initializers.end();) {
                if (keep.count(it->first)) ++it;
                else it = graph_.initializers.erase(it);
            }
            weightsReleased_ = true;
        }
        profiler_.setEnabled(cfg_.profile);
    }

    Status Session::runSegments() {
        try {
            ExecContext ctx;
            ctx.pool     = &pool_;
            ctx.graph    = &graph_;
            ctx.config   = &cfg_;
            ctx.profiler = &profiler_;
            for (auto &seg: segments_) {
                for (TensorId t: seg->boundaryInputs) {
                    RtTensor &rt = pool_[t];
                    if (!rt.hostValid && rt.deviceValid) {
                        for (auto &b: backends_) b->toHost(rt, ctx);
                    }
                }
                seg->run(ctx);
            }
        } catch (const Error &e) {
            lastError_ = e.what();
            return e.status();
        } catch (const std::exception &e) {
            lastError_ = e.what();
            return Status::RuntimeError;
        }
        return Status::Ok;
    }

    Status Session::run(const std::vector<IOTensor> &inputs, std::vector<IOTensor> &outputs) {
        try {
            // dma-buf bindings hold for one run: clear the last run's, then take this run's inputs
            // and the outputs the caller pre-filled with a name and an fd (reference
            // session_class.h:34-37)
            for (TensorId t: graph_.inputs) pool_[t].dmaBufFd = -1;
            for (TensorId t: graph_.outputs) pool_[t].dmaBufFd = -1;
            for (const IOTensor &io: outputs) {
                if (io.dmaBufFd < 0) continue;
                TensorId id = kNoTensor;
                for (TensorId t: graph_.outputs)
                    if (graph_.desc(t).name == io.name || (outputs.size() == 1 && graph_.outputs.size() == 1)) id = t;
                if (id == kNoTensor) throw Error(Status::NotFound, "no graph output named " + io.name);
                pool_[id].dmaBufFd     = io.dmaBufFd;
                pool_[id].dmaBufFormat = io.dmaBufFormat;
                pool_[id].dmaBufDtype  = io.dmaBufDtype;
            }
            for (const IOTensor &io: inputs) {
                TensorId id = graph_.find(io.name);
                if (id == kNoTensor && inputs.size() == 1 && graph_.inputs.size() == 1) id = graph_.inputs[0];
                if (id == kNoTensor) throw Error(Status::NotFound, "no graph input named " + io.name);
                RtTensor &rt = pool_[id];
                rt.shape     = graph_.desc(id).shape;
                if (io.dmaBufFd >= 0) {
                    rt.dmaBufFd     = io.dmaBufFd;
                    rt.dmaBufFormat = io.dmaBufFormat;
                    rt.dmaBufDtype  = io.dmaBufDtype;
                    rt.hostValid    = false;
                    rt.deviceValid  = false;
                    continue;
                }
                if (io.dtype != DType::Float32) throw Error(Status::InvalidArgument, "inputs must be fp32");
                if ((int64_t) io.data.size() != numElements(graph_.desc(id).shape) * 4)
                    throw Error(Status::InvalidArgument, "input " + io.name + " has " + std::to_string(io.data.size() / 4) + " values, expected " +
                                                             std::to_string(numElements(graph_.desc(id).shape)));
                rt.dtype = DType::Float32;
                rt.host.bytes = io.data;
                rt.hostValid   = true;
                rt.deviceValid = false;
            }
            Status st = runSegments();
            if (st != Status::Ok) return st;
            ExecContext ctx;
            ctx.pool   = &pool_;
            ctx.graph  = &graph_;
            ctx.config = &cfg_;
            outputs.clear();
            for (TensorId t: graph_.outputs) {
                RtTensor &rt = pool_[t];
                if (rt.dmaBufFd >= 0) { // written into the caller's buffer; no host data
                    IOTensor o;
                    o.name         = graph_.desc(t).name;
                    o.shape        = graph_.desc(t).shape;
                    o.dmaBufFd     = rt.dmaBufFd;
                    o.dmaBufFormat = rt.dmaBufFormat;
                    o.dmaBufDtype  = rt.dmaBufDtype;
                    outputs.push_back(std::move(o));
                    continue;
                }
                if (!rt.hostValid)
                    for (auto &b: backends_) {
                        b->toHost(rt, ctx);
                        if (rt.hostValid) break;
                    }
                IOTensor o;
                o.name  = graph_.desc(t).name;
                o.shape = graph_.desc(t).shape;
                o.dtype = DType::Float32;
                o.data  = rt.host.bytes;
                outputs.push_back(std::move(o));
            }
        } catch (const Error &e) {
            lastError_ = e.what();
            return e.status();
        } catch (const std::exception &e) {
            lastError_ = e.what();
            return Status::RuntimeError;
        }
        return Status::Ok;
    }

    Status Session::run(const std::vector<std::vector<float>> &inputData, std::vector<IOTensor> &outputs) {
        if (inputData.size() != graph_.inputs.size()) return Status::InvalidArgument;
        std::vector<IOTensor> ins;
        for (size_t i = 0; i < inputData.size(); ++i) {
            IOTensor io;
            io.name  = graph_.desc(graph_.inputs[i]).name;
            io.shape = graph_.desc(graph_.inputs[i]).shape;
            io.data.resize(inputData[i].size() * 4);
            std::memcpy(io.data.data(), inputData[i].data(), io.data.size());
            ins.push_back(std::move(io));
        }
        return run(ins, outputs);
    }

    std::vector<float> Session::infer(const std::vector<float> &input) {
        std::vector<IOTensor> outs;
        if (run(std::vector<std::vector<float>> {input}, outs) != Status::Ok || outs.empty()) return {};
        const float *p = outs[0].f32();
        return std::vector<float>(p, p + numElements(outs[0].shape));
    }

    std::vector<IOInfo> Session::inputInfo() const {
        std::vector<IOInfo> v;
        for (TensorId t: graph_.inputs) {
            IOInfo i;
            i.name         = graph_.desc(t).name;
            i.shape        = graph_.desc(t).shape;
            i.elems        = numElements(i.shape);
            i.deviceFormat = TensorFormat::NC4HW4;
            i.deviceDtype  = DType::Float16;
            i.deviceBytes  = formatElems(TensorFormat::NC4HW4, NCHW::from(i.shape)) * 2;
            v.push_back(i);
        }
        return v;
    }

    std::vector<IOInfo> Session::outputInfo() const {
        std::vector<IOInfo> v;
        for (TensorId t: graph_.outputs) {
            IOInfo i;
            i.name         = graph_.desc(t).name;
            i.shape        = graph_.desc(t).shape;
            i.elems        = numElements(i.shape);
            i.deviceFormat = TensorFormat::NC4HW4;
            i.deviceDtype  = DType::Float16;
            i.deviceBytes  = formatElems(TensorFormat::NC4HW4, NCHW::from(i.shape)) * 2;
            v.push_back(i);
        }
        return v;
    }

    std::vector<BackendKind> Session::nodeBackends() const {
        std::vector<BackendKind> v;
        for (int bi: nodeBackendIdx_) v.push_back(backends_[bi]->kind());
        return v;
    }

    const RtTensor *Session::tensor(const std::string &name) const {
        TensorId id = graph_.find(name);
        return id == kNoTensor ? nullptr : &pool_[id];
    }

} // namespace vknn
