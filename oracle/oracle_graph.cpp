// TEST INFRASTRUCTURE — whole-graph CPU oracle. Executes a zoo graph node by node with the C
// restatements in oracle.c, reproducing what the reference CPU backend computes after its standard
// passes (src/import/run_standard_passes.cpp:5-75):
//   * BatchNorm after a single-consumer Conv is folded into the conv weights first
//     (fold_batchnorm.cpp:57-78), so the conv sums the folded weights exactly as the reference does;
//   * Mul(x, HardSigmoid(x)) / Mul(x, Sigmoid(x)) with a single-use gate is evaluated as the fused
//     HardSwish / SiLU formula (fuse_swish.cpp:63-90, cpu_backend.cpp:55-66), as the reference
//     CPU backend does after fuseSwish;
//   * Relu/Clip/Add fusions are arithmetic no-ops (same float operations in the same order), so
//     those nodes execute literally.
// Not product code: only tests/, the smoke check and bench.py's CPU baseline load it.
#include "oracle.h"
#include "model_zoo.h"
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#define ORACLE_API extern "C" __attribute__((visibility("default")))

using namespace vknn;

namespace {

    struct T {
        std::vector<float>   v;
        std::vector<int64_t> s; // shape
    };

    std::vector<int64_t> ints(const Node &n, const char *k, std::vector<int64_t> d) {
        const auto &v = n.attr.getints(k);
        return v.empty() ? d : v;
    }

    std::string g_err;

    int run_graph(Graph &g, const float *x, int64_t nx, float *y, int64_t ny, float *trace = nullptr) {
        std::map<TensorId, T> vals;
        for (auto &kv: g.initializers) {
            const HostBuffer &hb = kv.second;
            T                 t;
            t.v.assign(hb.f32(), hb.f32() + hb.bytes.size() / 4);
            t.s        = g.desc(kv.first).shape;
            vals[kv.first] = std::move(t);
        }
        TensorId in = g.inputs[0];
        T        xi;
        xi.s = g.desc(in).shape;
        xi.v.assign(x, x + nx);
        if ((int64_t) xi.v.size() != numElements(xi.s)) {
            g_err = "input size mismatch";
            return 1;
        }
        vals[in] = std::move(xi);

        // use counts (node inputs only, as the reference passes count them)
        std::map<TensorId, int> uses;
        std::map<TensorId, int> producer;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            for (TensorId t: g.nodes[i].inputs) uses[t]++;
            for (TensorId t: g.nodes[i].outputs) producer[t] = (int) i;
        }
        // BN fold (restated): fold into a private copy of the conv weights/bias
        std::map<int, std::pair<std::vector<float>, std::vector<float>>> folded; // conv node -> (w, b)
        std::map<int, bool>                                              bnFolded;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &bn = g.nodes[i];
            if (bn.type != OpType::BatchNorm) continue;
            auto it = producer.find(bn.inputs[0]);
            if (it == producer.end() || g.nodes[it->second].type != OpType::Conv || uses[bn.inputs[0]] != 1) continue;
            const Node &cv   = g.nodes[it->second];
            const T    &W    = vals[cv.inputs[1]];
            int64_t     cout = W.s[0], per = (int64_t) W.v.size() / cout;
            std::vector<float> w = W.v, b((size_t) cout, 0.f);
            if (cv.inputs.size() > 2 && cv.inputs[2] != kNoTensor) b = vals[cv.inputs[2]].v;
            oracle_fold_bn(w.data(), b.data(), cout, per, vals[bn.inputs[1]].v.data(), vals[bn.inputs[2]].v.data(),
                           vals[bn.inputs[3]].v.data(), vals[bn.inputs[4]].v.data(), bn.attr.getf("epsilon", 1e-5f));
            folded[it->second] = {w, b};
            bnFolded[(int) i]  = true;
        }

        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &nd = g.nodes[i];
            auto        X  = [&](int k) -> T & { return vals[nd.inputs[k]]; };
            T           out;
            switch (nd.type) {
                case OpType::Conv: {
                    const T &x0 = X(0);
                    const T &W  = X(1);
                    std::vector<float> wv = W.v, bv;
                    const float       *bp = nullptr;
                    if (folded.count((int) i)) {
                        wv = folded[(int) i].first;
                        bv = folded[(int) i].second;
                        bp = bv.data();
                    } else if (nd.inputs.size() > 2 && nd.inputs[2] != kNoTensor) {
                        bp = X(2).v.data();
                    }
                    auto    st = ints(nd, "strides", {1, 1}), pad = ints(nd, "pads", {0, 0, 0, 0}), dil = ints(nd, "dilations", {1, 1});
                    int64_t grp = nd.attr.geti("group", 1);
                    int64_t OH, OW;
                    oracle_conv_out_hw(x0.s[2], x0.s[3], W.s[2], W.s[3], st.data(), pad.data(), dil.data(), &OH, &OW);
                    out.s = {x0.s[0], W.s[0], OH, OW};
                    out.v.resize((size_t) numElements(out.s));
                    oracle_conv2d(x0.v.data(), x0.s[0], x0.s[1], x0.s[2], x0.s[3], wv.data(), W.s[0], W.s[2], W.s[3], bp, st.data(), pad.data(),
                                  dil.data(), grp, nullptr, 0, 0, 0, out.v.data());
                    break;
                }
                case OpType::BatchNorm: {
                    if (bnFolded.count((int) i)) {
                        out = X(0);
                        break;
                    }
                    // standalone BN: src/backend/cpu/ops/batchnorm.cpp (a = g/sqrt(v+eps), b = beta - mean*a)
                    const T &x0 = X(0);
                    out         = x0;
                    int64_t C = x0.s[1], hw = (int64_t) x0.v.size() / (x0.s[0] * C);
                    for (int64_t n = 0; n < x0.s[0]; ++n)
                        for (int64_t c = 0; c < C; ++c) {
                            float a = X(1).v[c] / std::sqrt(X(4).v[c] + nd.attr.getf("epsilon", 1e-5f));
                            float b = X(2).v[c] - X(3).v[c] * a;
                            for (int64_t p = 0; p < hw; ++p) out.v[(n * C + c) * hw + p] = x0.v[(n * C + c) * hw + p] * a + b;
                        }
                    break;
                }
                case OpType::Relu: {
                    out = X(0);
                    oracle_unary(X(0).v.data(), out.v.data(), (int64_t) out.v.size(), 13, 0, 0);
                    break;
                }
                case OpType::Clip: {
                    float lo = -INFINITY, hi = INFINITY;
                    if (nd.inputs.size() > 1 && nd.inputs[1] != kNoTensor) lo = X(1).v[0];
                    if (nd.inputs.size() > 2 && nd.inputs[2] != kNoTensor) hi = X(2).v[0];
                    out = X(0);
                    oracle_unary(X(0).v.data(), out.v.data(), (int64_t) out.v.size(), -1, lo, hi);
                    break;
                }
                case OpType::Unary: {
                    out = X(0);
                    oracle_unary(X(0).v.data(), out.v.data(), (int64_t) out.v.size(), nd.subOp, nd.actLo, nd.actHi);
                    break;
                }
                case OpType::Binary: {
                    // swish restatement: Mul(x, gate(x)) with a single-use gate -> fused formula
                    if ((BinaryType) nd.subOp == BinaryType::Mul) {
                        int handled = 0;
                        for (int e = 0; e < 2 && !handled; ++e) {
                            auto pit = producer.find(nd.inputs[e]);
                            if (pit == producer.end()) continue;
                            const Node &gate = g.nodes[pit->second];
                            if (gate.type != OpType::Unary || gate.inputs[0] != nd.inputs[1 - e] || uses[nd.inputs[e]] != 1) continue;
                            UnaryType su = (UnaryType) gate.subOp;
                            if (su != UnaryType::HardSigmoid && su != UnaryType::Sigmoid) continue;
                            out = X(1 - e);
                            oracle_apply_act(out.v.data(), (int64_t) out.v.size(), su == UnaryType::HardSigmoid ? 4 : 5, 0, 0);
                            handled = 1;
                        }
                        if (handled) break;
                    }
                    const T &a = X(0), &b = X(1);
                    if (a.s == b.s) {
                        out.s = a.s;
                        out.v.resize(a.v.size());
                        oracle_binary(a.v.data(), b.v.data(), out.v.data(), (int64_t) a.v.size(), nd.subOp);
                    } else {
                        const T &big = a.v.size() >= b.v.size() ? a : b, &sm = a.v.size() >= b.v.size() ? b : a;
                        out.s = big.s;
                        out.v.resize(big.v.size());
                        oracle_mul_channel(big.v.data(), sm.v.data(), out.v.data(), big.s[0], big.s[1], big.s[2] * big.s[3]);
                    }
                    break;
                }
                case OpType::Add: {
                    out.s = X(0).s;
                    out.v.resize(X(0).v.size());
                    oracle_add(X(0).v.data(), X(1).v.data(), out.v.data(), (int64_t) out.v.size(), 0, 0, 0);
                    break;
                }
                case OpType::GlobalAvgPool: {
                    const T &x0 = X(0);
                    out.s       = {x0.s[0], x0.s[1], 1, 1};
                    out.v.resize((size_t) (x0.s[0] * x0.s[1]));
                    oracle_global_avg_pool(x0.v.data(), out.v.data(), x0.s[0], x0.s[1], x0.s[2] * x0.s[3]);
                    break;
                }
                case OpType::MaxPool: {
                    const T &x0 = X(0);
                    auto     k = ints(nd, "kernel_shape", {1, 1}), st = ints(nd, "strides", {1, 1}), p = ints(nd, "pads", {0, 0, 0, 0});
                    int64_t  OH = (x0.s[2] + p[0] + p[2] - k[0]) / st[0] + 1, OW = (x0.s[3] + p[1] + p[3] - k[1]) / st[1] + 1;
                    out.s = {x0.s[0], x0.s[1], OH, OW};
                    out.v.resize((size_t) numElements(out.s));
                    oracle_maxpool(x0.v.data(), out.v.data(), x0.s[0], x0.s[1], x0.s[2], x0.s[3], k[0], k[1], st[0], st[1], p[0], p[1], OH, OW);
                    break;
                }
                case OpType::Flatten: {
                    out = X(0);
                    int64_t a = out.s[0];
                    out.s     = {a, (int64_t) out.v.size() / a};
                    break;
                }
                case OpType::Gemm: {
                    const T &a = X(0), &b = X(1);
                    int      tB = (int) nd.attr.geti("transB", 0);
                    int64_t  M = a.s[0], K = a.s[1], N = tB ? b.s[0] : b.s[1];
                    out.s = {M, N};
                    out.v.resize((size_t) (M * N));
                    oracle_gemm(a.v.data(), b.v.data(), nd.inputs.size() > 2 ? X(2).v.data() : nullptr, out.v.data(), M, K, N, tB,
                                nd.attr.getf("alpha", 1.f), nd.attr.getf("beta", 1.f), 0, 0, 0);
                    break;
                }
                case OpType::Concat: {
                    std::vector<const float *> xs;
                    std::vector<int64_t>       cs;
                    int64_t                    C = 0;
                    for (size_t k = 0; k < nd.inputs.size(); ++k) {
                        xs.push_back(X((int) k).v.data());
                        cs.push_back(X((int) k).s[1]);
                        C += X((int) k).s[1];
                    }
                    const T &x0 = X(0);
                    out.s       = {x0.s[0], C, x0.s[2], x0.s[3]};
                    out.v.resize((size_t) numElements(out.s));
                    oracle_concat_channels(xs.data(), cs.data(), (int) xs.size(), out.v.data(), x0.s[0], x0.s[2] * x0.s[3]);
                    break;
                }
                case OpType::Split: {
                    const T &x0 = X(0);
                    int64_t  nout = (int64_t) nd.outputs.size(), each = x0.s[1] / nout;
                    for (int64_t k = 0; k < nout; ++k) {
                        T o;
                        o.s = {x0.s[0], each, x0.s[2], x0.s[3]};
                        o.v.resize((size_t) numElements(o.s));
                        oracle_slice_channels(x0.v.data(), o.v.data(), x0.s[0], x0.s[1], k * each, each, x0.s[2] * x0.s[3]);
                        vals[nd.outputs[k]] = std::move(o);
                    }
                    continue;
                }
                case OpType::Resize: {
                    const T &x0 = X(0);
                    const T &sc = X(2);
                    out.s = {x0.s[0], x0.s[1], (int64_t) (x0.s[2] * sc.v[2]), (int64_t) (x0.s[3] * sc.v[3])};
                    out.v.resize((size_t) numElements(out.s));
                    int mode = nd.attr.gets("coordinate_transformation_mode", "half_pixel") == "asymmetric" ? 2 : 0;
                    oracle_resize_nearest(x0.v.data(), out.v.data(), x0.s[0] * x0.s[1], x0.s[2], x0.s[3], out.s[2], out.s[3], mode);
                    break;
                }
                default:
                    g_err = std::string("oracle: no op ") + std::to_string((int) nd.type);
                    return 1;
            }
            if (trace) {
                float m = 0.f;
                for (float v: out.v) m = std::fmax(m, std::fabs(v));
                trace[i] = m;
            }
            vals[nd.outputs[0]] = std::move(out);
        }
        int64_t off = 0;
        for (TensorId o: g.outputs) {
            const T &t = vals[o];
            if (off + (int64_t) t.v.size() > ny) {
                g_err = "output buffer too small";
                return 1;
            }
            std::memcpy(y + off, t.v.data(), t.v.size() * 4);
            off += (int64_t) t.v.size();
        }
        return 0;
    }

} // namespace

ORACLE_API const char *oracle_last_error(void) { return g_err.c_str(); }

ORACLE_API int oracle_model_run(const char *name, int64_t batch, uint64_t seed, const float *x, int64_t nx, float *y, int64_t ny) {
    Graph g = vknn_zoo::build(name, batch, seed);
    if (g.nodes.empty()) {
        g_err = std::string("unknown model ") + name;
        return 1;
    }
    return run_graph(g, x, nx, y, ny);
}

// Per-node max |output| (index = node order of the unfused zoo graph); for range diagnostics.
ORACLE_API int oracle_model_trace(const char *name, int64_t batch, uint64_t seed, const float *x, int64_t nx, float *y, int64_t ny,
                                  float *trace, int64_t ntrace) {
    Graph g = vknn_zoo::build(name, batch, seed);
    if ((int64_t) g.nodes.size() > ntrace) return 1;
    return run_graph(g, x, nx, y, ny, trace);
}

ORACLE_API int oracle_model_io(const char *name, int64_t batch, int64_t *in4, int64_t *out_elems, int32_t *n_out, int32_t max_out) {
    std::vector<int64_t> in, out;
    if (!vknn_zoo::io_shapes(name, batch, in, out)) return 1;
    for (int i = 0; i < 4; ++i) in4[i] = in[i];
    *n_out = (int32_t) out.size();
    for (int i = 0; i < (int) out.size() && i < max_out; ++i) out_elems[i] = out[i];
    return 0;
}

ORACLE_API double oracle_model_flops(const char *name) { return vknn_zoo::conv_flops_per_image(name); }
