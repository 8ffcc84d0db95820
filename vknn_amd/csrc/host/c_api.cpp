// C ABI over Session + the HIP backend (declared in include/vknn_c.h).
#include "vknn_c.h"
#include "hip_backend.h"
#include "tune_cache.h"
#include "model_zoo.h"
#include "graph_text.h"
#include "vknn/session.h"
#include <cstring>
#include <algorithm>
#include <cstdlib>
#include <sstream>
#include <string>

using namespace vknn;

namespace {
    thread_local std::string g_err;

    int fail(const std::string &m) {
        g_err = m;
        return 1;
    }

    void copyOut(const std::string &s, char *buf, int64_t cap) {
        if (!buf || cap <= 0) return;
        size_t n = std::min<size_t>((size_t) cap - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }

    struct Opts {
        Config cfg;
        bool   passes = true; // vknn_model_save_vxm: "passes=0" writes the graph as built
        Opts(const char *s) {
            cfg.backend = BackendKind::Hip;
            std::string str = s ? s : "";
            std::stringstream ss(str);
            std::string item;
            while (std::getline(ss, item, ';')) {
                auto eq = item.find('=');
                if (eq == std::string::npos) continue;
                std::string k = item.substr(0, eq), v = item.substr(eq + 1);
                if (k == "winograd") cfg.setHint(Hint::Winograd, winogradFromStr(v));
                else if (k == "tuning") cfg.setHint(Hint::Tuning, tuningFromStr(v));
                else if (k == "graphs") cfg.hipGraphs = v != "0";
                else if (k == "branches") cfg.hipBranches = v != "0";
                else if (k == "profile") cfg.profile = v != "0";
                else if (k == "profile_reps") cfg.profileReps = std::max(1, std::atoi(v.c_str()));
                else if (k == "fuse_dwpw") cfg.fuseDwPw = v != "0";
                else if (k == "fuse_se") cfg.fuseSqueezeExcite = v != "0";
                else if (k == "hip_auto_se") cfg.hipAutoSE = v != "0";
                else if (k == "hip_auto_dwpw") cfg.hipAutoDwPw = v != "0";
                else if (k == "cache_file") cfg.cacheFile = v;
                else if (k == "passes") passes = v != "0";
                else if (k == "cpu_fallback") cfg.allowCpuFallback = v != "0";
                else if (k == "keep_weights") cfg.freeWeightsAfterUpload = v == "0";
                else if (k == "cache_mode") cfg.cacheMode = v == "off" ? CacheMode::Off : v == "tune" ? CacheMode::Tune : CacheMode::Full;
            }
            // setHint resizes the hint table with zeros; keep unset knobs at their defaults.
            if (cfg.hints.size() > (size_t) Hint::Tuning && !std::strstr(str.c_str(), "tuning=")) cfg.setHint(Hint::Tuning, Mode::Fast);
        }
    };
} // namespace

struct vknn_session_s {
    std::unique_ptr<Session> sess;
    std::string              model;
};

static hipbe::HipSegment *onlySegment(vknn_session s) {
    auto &segs = s->sess->segments();
    if (segs.size() != 1) throw Error(Status::Unsupported, "device I/O needs the whole graph in one HIP segment");
    auto *h = dynamic_cast<hipbe::HipSegment *>(segs[0].get());
    if (!h) throw Error(Status::Unsupported, "segment is not a HIP segment");
    return h;
}

extern "C" {

const char *vknn_last_error(void) { return g_err.c_str(); }

int vknn_model_io(const char *model, int64_t batch, int64_t *in_shape4, int64_t *out_elems, int32_t *n_out, int32_t max_out) {
    try {
        if (!model || !in_shape4 || !n_out || (max_out > 0 && !out_elems)) return fail("model_io: null argument");
        std::vector<int64_t> in, out;
        if (!vknn_zoo::io_shapes(model, batch, in, out)) return fail(std::string("unknown model ") + model);
        for (int i = 0; i < 4; ++i) in_shape4[i] = in[i];
        *n_out = (int32_t) out.size();
        for (int i = 0; i < (int) out.size() && i < max_out; ++i) out_elems[i] = out[i];
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

double vknn_model_flops(const char *model) {
    try {
        return vknn_zoo::conv_flops_per_image(model);
    } catch (const std::exception &e) {
        fail(e.what());
        return 0.0;
    }
}

int vknn_session_create_model(const char *model, int64_t batch, uint64_t seed, const char *options, vknn_session *out) {
    try {
        Graph g = vknn_zoo::build(model, batch, seed);
        if (g.nodes.empty()) return fail(std::string("unknown model ") + model);
        Opts o(options);
        std::unique_ptr<vknn_session_s> s(new vknn_session_s());
        s->model = model;
        s->sess  = Session::create(std::move(g), o.cfg);
        *out     = s.release();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_destroy(vknn_session s) {
    try {
        delete s;
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_run_host(vknn_session s, const float *x, int64_t nx, float *y, int64_t ny) {
    try {
        std::vector<float> in(x, x + nx);
        std::vector<IOTensor> outs;
        Status st = s->sess->run(std::vector<std::vector<float>> {in}, outs);
        if (st != Status::Ok) return fail(std::string("run failed: ") + statusStr(st) + ": " + s->sess->lastError());
        int64_t off = 0;
        for (auto &o: outs) {
            int64_t n = numElements(o.shape);
            if (off + n > ny) return fail("output buffer too small");
            std::memcpy(y + off, o.f32(), (size_t) n * 4);
            off += n;
        }
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_run_dmabuf(vknn_session s, int32_t in_fd, int32_t in_fmt, int32_t in_f16, int32_t out_fd, int32_t out_fmt, int32_t out_f16,
                            float *y, int64_t ny) {
    try {
        if (!s) return fail("run_dmabuf: null session");
        auto layout = [](int32_t f) {
            if (f < 0 || f > 3) throw Error(Status::InvalidArgument, "dma-buf layout must be 0 NCHW, 1 NHWC, 2 NC4HW4 or 3 device-native");
            return (TensorFormat) f;
        };
        const Graph &g = s->sess->graph();
        if (g.inputs.size() != 1 || g.outputs.empty()) return fail("run_dmabuf: the model must have one input");
        std::vector<IOTensor> ins(1), outs;
        ins[0].name  = g.desc(g.inputs[0]).name;
        ins[0].shape = g.desc(g.inputs[0]).shape;
        if (in_fd >= 0) {
            ins[0].dmaBufFd     = in_fd;
            ins[0].dmaBufFormat = layout(in_fmt);
            ins[0].dmaBufDtype  = in_f16 ? DType::Float16 : DType::Float32;
        } else {
            return fail("run_dmabuf: no input fd");
        }
        if (out_fd >= 0) {
            IOTensor o;
            o.name         = g.desc(g.outputs[0]).name;
            o.dmaBufFd     = out_fd;
            o.dmaBufFormat = layout(out_fmt);
            o.dmaBufDtype  = out_f16 ? DType::Float16 : DType::Float32;
            outs.push_back(o);
        }
        Status st = s->sess->run(ins, outs);
        if (st != Status::Ok) return fail(std::string("run failed: ") + statusStr(st) + ": " + s->sess->lastError());
        int64_t off = 0;
        for (auto &o: outs) {
            if (o.dmaBufFd >= 0) continue;
            int64_t n = numElements(o.shape);
            if (!y || off + n > ny) return fail("output buffer too small");
            std::memcpy(y + off, o.f32(), (size_t) n * 4);
            off += n;
        }
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_bind_device_input(vknn_session s, const float *dev_x) {
    try {
        auto *seg = onlySegment(s);
        seg->bindDeviceInput(s->sess->graph().inputs[0], dev_x);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_bind_device_input_as(vknn_session s, const void *dev_x, int32_t fmt, int32_t f16) {
    try {
        auto *seg = onlySegment(s);
        seg->bindDeviceInputAs(s->sess->graph().inputs[0], dev_x, fmt, f16 != 0);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_run_device(vknn_session s) {
    try {
        if (!s) return fail("run_device: null session");
        Status st = s->sess->runSegments();
        return st == Status::Ok ? 0 : fail(std::string("run failed: ") + statusStr(st) + ": " + s->sess->lastError());
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_sync(vknn_session s) {
    try {
        hipbe::check(vkhip_stream_sync(onlySegment(s)->stream()), "sync");
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

const float *vknn_session_device_output(vknn_session s, int32_t k) {
    try {
        return onlySegment(s)->deviceOutput(s->sess->graph().outputs.at(k));
    } catch (const std::exception &e) {
        fail(e.what());
        return nullptr;
    }
}

int vknn_session_read_outputs(vknn_session s, float *y, int64_t ny) {
    try {
        auto   *seg = onlySegment(s);
        int64_t off = 0;
        for (TensorId t: s->sess->graph().outputs) {
            int64_t n = numElements(s->sess->graph().desc(t).shape);
            if (off + n > ny) return fail("output buffer too small");
            seg->download(t, y + off);
            off += n;
        }
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

void *vknn_session_stream(vknn_session s) {
    try {
        return onlySegment(s)->stream();
    } catch (const std::exception &e) {
        fail(e.what());
        return nullptr;
    }
}

int vknn_session_profile_json(vknn_session s, char *buf, int64_t cap) {
    try {
        copyOut(s->sess->profiler().toJson(), buf, cap);
        s->sess->profiler().clear();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_describe(vknn_session s, char *buf, int64_t cap) {
    try {
        std::string d;
        for (auto &seg: s->sess->segments())
            if (auto *h = dynamic_cast<hipbe::HipSegment *>(seg.get())) d += h->describe();
        copyOut(d, buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_segments(vknn_session s, char *buf, int64_t cap) {
    try {
        if (!s) return fail("segments: null session");
        std::string d;
        for (auto &seg: s->sess->segments()) {
            d += std::string(seg->backend ? seg->backend->name() : "?") + " nodes=" + std::to_string(seg->nodeIdx.size()) + " in=";
            for (TensorId t: seg->boundaryInputs) d += s->sess->graph().desc(t).name + ",";
            d += " out=";
            for (TensorId t: seg->boundaryOutputs) d += s->sess->graph().desc(t).name + ",";
            d += "\n";
        }
        copyOut(d, buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_count_ops(vknn_session s, const char *op) {
    try {
        int n = 0;
        for (const Node &nd: s->sess->graph().nodes)
            if (std::string(opTypeName(nd.type)) == op) ++n;
        return n;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

static std::string nodeList(const Graph &g) {
    std::string d;
    for (const Node &nd: g.nodes)
        d += std::string(opTypeName(nd.type)) + " " + nd.name + " act=" + std::to_string((int) nd.fusedAct) +
             " res=" + std::to_string(nd.fusedResidual != kNoTensor ? 1 : 0) + " out=" + shapeStr(g.desc(nd.outputs[0]).shape) + "\n";
    return d;
}

static Graph optimizedZooGraph(const char *model, int64_t batch, uint64_t seed, const char *options) {
    Graph g = vknn_zoo::build(model, batch, seed);
    if (g.nodes.empty()) throw Error(Status::InvalidArgument, std::string("unknown model ") + model);
    Opts o(options);
    if (!o.passes) return g;
    PassOptions po;
    po.batch             = batch;
    po.fuseDwPw          = o.cfg.fuseDwPw;
    po.fuseSqueezeExcite = o.cfg.fuseSqueezeExcite;
    runStandardPasses(g, po);
    g.topoSort();
    return g;
}

int vknn_graph_after_passes(const char *model, int64_t batch, const char *options, char *buf, int64_t cap) {
    try {
        copyOut(nodeList(optimizedZooGraph(model, batch, 1, options)), buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_model_save_vxm(const char *model, int64_t batch, uint64_t seed, const char *options, const char *path) {
    try {
        if (!path) return fail("save_vxm: null path");
        if (!saveGraphBin(optimizedZooGraph(model, batch, seed, options), path)) return fail(std::string("cannot write ") + path);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_vxm_describe(const char *path, char *buf, int64_t cap) {
    try {
        Graph       g;
        std::string why;
        if (!path || !loadGraphBin(g, path, &why)) return fail(std::string("failed to load .vxm ") + (path ? path : "(null)") + ": " + why);
        copyOut(nodeList(g), buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_create_vxm(const char *path, const char *options, vknn_session *out) {
    try {
        if (!path || !out) return fail("create_vxm: null argument");
        Opts o(options);
        std::unique_ptr<vknn_session_s> s(new vknn_session_s());
        s->model = path;
        s->sess  = Session::createFromVxm(path, o.cfg);
        *out     = s.release();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_onnx_describe(const char *path, char *buf, int64_t cap) {
    try {
        if (!path) return fail("onnx_describe: null path");
        copyOut(vknn_text::graph(importOnnx(path)), buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_onnx_after_passes(const char *path, const char *options, char *buf, int64_t cap) {
    try {
        if (!path) return fail("onnx_after_passes: null path");
        Graph g = importOnnx(path);
        Opts  o(options);
        PassOptions po;
        po.fuseDwPw          = o.cfg.fuseDwPw;
        po.fuseSqueezeExcite = o.cfg.fuseSqueezeExcite;
        runStandardPasses(g, po);
        g.topoSort();
        copyOut(nodeList(g), buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_create_onnx(const char *path, const char *options, vknn_session *out) {
    try {
        if (!path || !out) return fail("create_onnx: null argument");
        Opts o(options);
        std::unique_ptr<vknn_session_s> s(new vknn_session_s());
        s->model = path;
        s->sess  = Session::createFromOnnx(path, o.cfg);
        *out     = s.release();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_session_save_optimized(vknn_session s, const char *path) {
    try {
        if (!s || !path) return fail("save_optimized: null argument");
        if (!s->sess->saveOptimized(path)) return fail(std::string("cannot save the optimized graph to ") + path + " (host weights released: create the session with keep_weights=1)");
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_tune_cache_load(const char *path) {
    try {
        return path ? hipbe::TuneCache::instance().load(path, true) : 0;
    } catch (const std::exception &e) {
        fail(e.what());
        return 0;
    }
}

int vknn_tune_cache_save(const char *path) {
    try {
        if (!path || hipbe::TuneCache::instance().save(path)) return fail(std::string("cannot write cache file ") + (path ? path : "(null)"));
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_tune_cache_put(const char *key, int32_t value) {
    try {
        if (!key) return fail("tune cache: null key");
        hipbe::TuneCache::instance().put(key, value);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_tune_cache_get(const char *key, int32_t *value) {
    try {
        int32_t v = 0;
        if (!key || !hipbe::TuneCache::instance().get(key, v)) return 1;
        if (value) *value = v;
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_tune_cache_clear(void) {
    try {
        hipbe::TuneCache::instance().clear();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_tune_cache_stats(int64_t *entries, int64_t *hits, int64_t *misses) {
    try {
        auto &c = hipbe::TuneCache::instance();
        if (entries) *entries = (int64_t) c.size();
        if (hits) *hits = c.hits();
        if (misses) *misses = c.misses();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_weight_cache_stats(int64_t *entries, int64_t *hits, int64_t *misses) {
    try {
        auto &c = hipbe::TuneCache::instance();
        if (entries) *entries = (int64_t) c.weightCount();
        if (hits) *hits = c.weightHits();
        if (misses) *misses = c.weightMisses();
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

int vknn_tune_cache_gpu_tag(char *buf, int64_t cap) {
    try {
        copyOut(hipbe::gpuTag(), buf, cap);
        return 0;
    } catch (const std::exception &e) {
        return fail(e.what());
    }
}

} // extern "C"
