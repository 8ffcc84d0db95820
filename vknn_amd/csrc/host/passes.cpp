// Graph passes that shape the conv-path nodes the HIP backend executes. Same rewrites and
// eligibility rules as the reference passes, implemented over a shared use-count helper:
//   foldConstantNodes  the Constant case of src/import/const_fold.cpp:33 with the value emitted as
//                      backend/cpu/ops/constant.cpp:8-38 does (dims kept, else a flat [n])
//   inferShapes        src/import/infer_shapes.cpp (rules for the conv-path op set)
//   foldBatchNorm      src/import/fold_batchnorm.cpp:5-131
//   fuseActivations    src/import/fuse_activations.cpp:5-125 (Relu6 only when lo==0 && hi==6)
//   fuseResidualAdd    src/import/fuse_residual_add.cpp:5-124 (1x1 s1 p0 g1 producer only)
//   fuseSwish          src/import/fuse_swish.cpp:5-99
//   fuseSqueezeExcite  src/import/fuse_squeeze_excite.cpp:5-95
//   fuseDwPw           src/import/fuse_dwpw.cpp:38-146
//   runStandardPasses  src/import/run_standard_passes.cpp:5-75 (conv-path subset, same order)
#include "vknn/passes.h"
#include <cmath>
#include <set>

namespace vknn {

    namespace {

        std::vector<int64_t> attrInts(const Node &n, const char *k, std::vector<int64_t> d) {
            const auto &v = n.attr.getints(k);
            return v.empty() ? d : v;
        }

        // Producer index and use count (node inputs + graph outputs) per tensor.
        struct Uses {
            std::vector<int> producer, count;
            explicit Uses(const Graph &g, bool countOutputs = true) {
                producer.assign(g.tensors.size(), -1);
                count.assign(g.tensors.size(), 0);
                for (size_t i = 0; i < g.nodes.size(); ++i) {
                    for (TensorId o: g.nodes[i].outputs)
                        if (o != kNoTensor) producer[o] = (int) i;
                    for (TensorId t: g.nodes[i].inputs)
                        if (t != kNoTensor) ++count[t];
                }
                if (countOutputs)
                    for (TensorId t: g.outputs)
                        if (t != kNoTensor) ++count[t];
            }
        };

        void dropNodes(Graph &g, const std::set<int> &drop) {
            if (drop.empty()) return;
            std::vector<Node> kept;
            kept.reserve(g.nodes.size());
            for (size_t i = 0; i < g.nodes.size(); ++i)
                if (!drop.count((int) i)) kept.push_back(std::move(g.nodes[i]));
            g.nodes = std::move(kept);
        }

        bool isPointwiseConv(const Graph &g, const Node &c) {
            if (c.type != OpType::Conv || c.attr.geti("group", 1) != 1) return false;
            const Shape &w = g.desc(c.inputs[1]).shape;
            if (w.size() != 4 || w[2] != 1 || w[3] != 1) return false;
            auto s = attrInts(c, "strides", {1, 1});
            auto p = attrInts(c, "pads", {0, 0, 0, 0});
            return s[0] == 1 && s[1] == 1 && p[0] == 0 && p[1] == 0 && p[2] == 0 && p[3] == 0;
        }

        TensorId biasOf(const Node &c) {
            if (c.inputs.size() > 2 && c.inputs[2] != c.fusedResidual) return c.inputs[2];
            return kNoTensor;
        }

    } // namespace

    void rewireTensor(Graph &g, TensorId from, TensorId to) {
        if (from == to || from == kNoTensor) return;
        for (Node &n: g.nodes) {
            for (TensorId &t: n.inputs)
                if (t == from) t = to;
            if (n.fusedResidual == from) n.fusedResidual = to;
        }
        for (TensorId &t: g.outputs)
            if (t == from) t = to;
    }

    // Constant nodes (ONNX import) become initializers, so the parameters they carry (Clip bounds,
    // Resize scales, Split sizes) are readable by the rules below and no backend runs them. The
    // value comes from the "value" tensor attribute, or value_float(s) / value_int(s).
    void foldConstantNodes(Graph &g) {
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &n = g.nodes[i];
            if (n.type != OpType::Constant || n.outputs.empty() || n.outputs[0] == kNoTensor) continue;
            const Attr *a = nullptr;
            for (const char *k: {"value", "value_floats", "value_ints", "value_float", "value_int"})
                if (auto it = n.attr.map.find(k); it != n.attr.map.end()) {
                    a = &it->second;
                    break;
                }
            if (!a) continue;
            const TensorId o = n.outputs[0];
            TensorDesc    &d = g.desc(o);
            HostBuffer     hb;
            const bool     ints = a->kind == Attr::Ints || a->kind == Attr::Int;
            std::vector<int64_t> iv = a->kind == Attr::Int ? std::vector<int64_t> {a->i} : a->ints;
            std::vector<float>   fv = a->kind == Attr::Float ? std::vector<float> {a->f} : a->floats;
            const size_t         cnt = ints ? iv.size() : fv.size();
            d.shape = !a->shape.empty() ? a->shape : Shape {(int64_t) cnt};
            if (ints) {
                d.dtype = DType::Int64;
                hb.resizeElems((int64_t) cnt, DType::Int64);
                for (size_t k = 0; k < cnt; ++k) hb.i64()[k] = iv[k];
            } else {
                d.dtype = DType::Float32;
                hb.resizeElems((int64_t) cnt, DType::Float32);
                for (size_t k = 0; k < cnt; ++k) hb.f32()[k] = fv[k];
            }
            d.isInitializer   = true;
            g.initializers[o] = std::move(hb);
            drop.insert((int) i);
        }
        dropNodes(g, drop);
    }

    void inferShapes(Graph &g, int64_t batch) {
        for (TensorId in: g.inputs)
            for (auto &d: g.desc(in).shape)
                if (d < 0) d = batch;
        auto SH = [&](TensorId id) -> Shape & { return g.desc(id).shape; };
        for (Node &nd: g.nodes) {
            if (nd.outputs.empty() || nd.inputs.empty()) continue;
            TensorId     o  = nd.outputs[0];
            const Shape &s0 = SH(nd.inputs[0]);
            switch (nd.type) {
                case OpType::Conv: {
                    if (s0.empty()) break;
                    const Shape &w = SH(nd.inputs[1]);
                    if (w.size() < 4) break;
                    NCHW x   = NCHW::from(s0);
                    auto st  = attrInts(nd, "strides", {1, 1});
                    auto pad = attrInts(nd, "pads", {0, 0, 0, 0});
                    auto dil = attrInts(nd, "dilations", {1, 1});
                    SH(o)    = {x.n, w[0], (x.h + pad[0] + pad[2] - (dil[0] * (w[2] - 1) + 1)) / st[0] + 1,
                                (x.w + pad[1] + pad[3] - (dil[1] * (w[3] - 1) + 1)) / st[1] + 1};
                    break;
                }
                case OpType::FusedDwPw: {
                    if (s0.empty()) break;
                    const Shape &dw = SH(nd.inputs[1]);
                    const Shape &pw = SH(nd.inputs[3]);
                    NCHW x   = NCHW::from(s0);
                    auto st  = attrInts(nd, "strides", {1, 1});
                    auto pad = attrInts(nd, "pads", {0, 0, 0, 0});
                    auto dil = attrInts(nd, "dilations", {1, 1});
                    SH(o)    = {x.n, pw[0], (x.h + pad[0] + pad[2] - (dil[0] * (dw[2] - 1) + 1)) / st[0] + 1,
                                (x.w + pad[1] + pad[3] - (dil[1] * (dw[3] - 1) + 1)) / st[1] + 1};
                    break;
                }
                case OpType::FusedSE: {
                    if (s0.empty()) break;
                    NCHW x = NCHW::from(s0);
                    SH(o)  = {x.n, x.c, 1, 1};
                    break;
                }
                case OpType::Clip: case OpType::Relu: case OpType::BatchNorm: case OpType::Identity: case OpType::Unary:
                case OpType::FusedPointwise:
                    SH(o) = s0;
                    break;
                case OpType::Add: case OpType::Binary: {
                    if (nd.inputs.size() < 2) break;
                    const Shape &a = s0, &b = SH(nd.inputs[1]);
                    size_t rank = std::max(a.size(), b.size());
                    Shape  out(rank, 1);
                    for (size_t i = 0; i < rank; ++i) {
                        int64_t da = i + a.size() >= rank ? a[i + a.size() - rank] : 1;
                        int64_t db = i + b.size() >= rank ? b[i + b.size() - rank] : 1;
                        out[i]     = std::max(da, db);
                    }
                    SH(o) = out;
                    break;
                }
                case OpType::GlobalAvgPool: {
                    if (s0.empty()) break;
                    NCHW x = NCHW::from(s0);
                    SH(o)  = {x.n, x.c, 1, 1};
                    break;
                }
                case OpType::MaxPool: case OpType::AvgPool: {
                    if (s0.empty()) break;
                    NCHW x  = NCHW::from(s0);
                    auto k  = attrInts(nd, "kernel_shape", {1, 1});
                    auto st = attrInts(nd, "strides", {1, 1});
                    auto p  = attrInts(nd, "pads", {0, 0, 0, 0});
                    SH(o)   = {x.n, x.c, (x.h + p[0] + p[2] - k[0]) / st[0] + 1, (x.w + p[1] + p[3] - k[1]) / st[1] + 1};
                    break;
                }
                case OpType::Flatten: {
                    if (s0.empty()) break;
                    int64_t axis = nd.attr.geti("axis", 1);
                    if (axis < 0) axis += (int64_t) s0.size();
                    int64_t a = 1, b = 1;
                    for (int64_t i = 0; i < (int64_t) s0.size(); ++i) (i < axis ? a : b) *= s0[i];
                    SH(o) = {a, b};
                    break;
                }
                case OpType::Gemm: {
                    if (s0.size() < 2) break;
                    const Shape &w = SH(nd.inputs[1]);
                    int64_t M = nd.attr.geti("transA", 0) ? s0[1] : s0[0];
                    int64_t N = nd.attr.geti("transB", 0) ? w[0] : w[1];
                    SH(o)     = {M, N};
                    break;
                }
                case OpType::Concat: {
                    if (s0.empty()) break;
                    int64_t axis = nd.attr.geti("axis", 0);
                    if (axis < 0) axis += (int64_t) s0.size();
                    Shape out = s0;
                    out[axis] = 0;
                    for (TensorId t: nd.inputs) out[axis] += SH(t)[axis];
                    SH(o) = out;
                    break;
                }
                case OpType::Split: {
                    if (s0.empty()) break;
                    int64_t axis = nd.attr.geti("axis", 0);
                    if (axis < 0) axis += (int64_t) s0.size();
                    std::vector<int64_t> sp = nd.attr.getints("split");
                    if (sp.empty() && nd.inputs.size() > 1 && nd.inputs[1] != kNoTensor && g.isInitializer(nd.inputs[1]) &&
                        g.desc(nd.inputs[1]).dtype == DType::Int64) {
                        const HostBuffer &hb = g.initializers[nd.inputs[1]];
                        sp.assign(hb.i64(), hb.i64() + hb.bytes.size() / 8);
                    }
                    if (sp.empty())
                        for (size_t k = 0; k < nd.outputs.size(); ++k) sp.push_back(s0[axis] / (int64_t) nd.outputs.size());
                    for (size_t k = 0; k < nd.outputs.size() && k < sp.size(); ++k) {
                        if (nd.outputs[k] == kNoTensor) continue;
                        Shape os = s0;
                        os[axis] = sp[k];
                        SH(nd.outputs[k]) = os;
                    }
                    break;
                }
                case OpType::Resize: {
                    if (s0.size() != 4) break;
                    Shape s = s0;
                    auto  initF = [&](size_t idx) -> const HostBuffer * {
                        if (idx >= nd.inputs.size() || nd.inputs[idx] == kNoTensor) return nullptr;
                        auto it = g.initializers.find(nd.inputs[idx]);
                        return it == g.initializers.end() ? nullptr : &it->second;
                    };
                    if (const HostBuffer *sz = initF(3); sz && sz->bytes.size() == 4 * 8) {
                        for (int k = 0; k < 4; ++k) s[k] = sz->i64()[k];
                    } else if (const HostBuffer *sc = initF(2); sc && sc->bytes.size() == 4 * 4) {
                        for (int k = 0; k < 4; ++k) s[k] = (int64_t) (s0[k] * sc->f32()[k]);
                    }
                    SH(o) = s;
                    break;
                }
                default:
                    break;
            }
        }
    }

    void eliminateIdentity(Graph &g) {
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            if (g.nodes[i].type != OpType::Identity) continue;
            rewireTensor(g, g.nodes[i].outputs[0], g.nodes[i].inputs[0]);
            drop.insert((int) i);
        }
        dropNodes(g, drop);
    }

    void eliminateDeadNodes(Graph &g) {
        for (bool changed = true; changed;) {
            changed = false;
            Uses          u(g);
            std::set<int> drop;
            for (size_t i = 0; i < g.nodes.size(); ++i) {
                bool live = false;
                for (TensorId o: g.nodes[i].outputs) live = live || (o != kNoTensor && u.count[o] > 0);
                if (!live) drop.insert((int) i);
            }
            changed = !drop.empty();
            dropNodes(g, drop);
        }
    }

    void foldBatchNorm(Graph &g) {
        Uses          u(g, false);
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &bn = g.nodes[i];
            if (bn.type != OpType::BatchNorm) continue;
            int pi = u.producer[bn.inputs[0]];
            if (pi < 0 || g.nodes[pi].type != OpType::Conv || u.count[g.nodes[pi].outputs[0]] != 1) continue;
            Node        &conv  = g.nodes[pi];
            const float *gamma = g.initializers[bn.inputs[1]].f32();
            const float *beta  = g.initializers[bn.inputs[2]].f32();
            const float *mean  = g.initializers[bn.inputs[3]].f32();
            const float *var   = g.initializers[bn.inputs[4]].f32();
            const float  eps   = bn.attr.getf("epsilon", 1e-5f);
            const int64_t cout = g.desc(conv.inputs[1]).shape[0];
            const int64_t per  = numElements(g.desc(conv.inputs[1]).shape) / cout;
            float        *w    = g.initializers[conv.inputs[1]].f32();
            TensorId      bid  = (conv.inputs.size() > 2 && conv.inputs[2] != kNoTensor) ? conv.inputs[2] : kNoTensor;
            if (bid == kNoTensor) {
                TensorDesc d;
                d.name          = conv.name + "_bias";
                d.shape         = {cout};
                d.isInitializer = true;
                bid             = g.addTensor(d);
                g.initializers[bid].resizeElems(cout, DType::Float32);
                if (conv.inputs.size() < 3) conv.inputs.resize(3, kNoTensor);
                conv.inputs[2] = bid;
            }
            float *b = g.initializers[bid].f32();
            for (int64_t oc = 0; oc < cout; ++oc) {
                float a = gamma[oc] / std::sqrt(var[oc] + eps);
                for (int64_t k = 0; k < per; ++k) w[oc * per + k] *= a;
                b[oc] = (b[oc] - mean[oc]) * a + beta[oc];
            }
            TensorId bnOut = bn.outputs[0], convOut = conv.outputs[0];
            for (Node &n: g.nodes)
                for (TensorId &t: n.inputs)
                    if (t == bnOut) t = convOut;
            for (TensorId &t: g.outputs)
                if (t == bnOut) t = convOut;
            drop.insert((int) i);
        }
        dropNodes(g, drop);
    }

    void fuseActivations(Graph &g) {
        Uses          u(g);
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &act = g.nodes[i];
            if (act.type != OpType::Clip && act.type != OpType::Relu) continue;
            int pi = u.producer[act.inputs[0]];
            if (pi < 0) continue;
            Node &prod = g.nodes[pi];
            if (prod.type != OpType::Conv && prod.type != OpType::Gemm && prod.type != OpType::Add) continue;
            if (prod.fusedAct != ActType::None || u.count[prod.outputs[0]] != 1) continue;
            if (act.type == OpType::Relu) {
                prod.fusedAct = ActType::Relu;
            } else {
                float lo = 0.f, hi = 6.f;
                if (act.inputs.size() > 1 && act.inputs[1] != kNoTensor && g.isInitializer(act.inputs[1])) lo = g.initializers[act.inputs[1]].f32()[0];
                if (act.inputs.size() > 2 && act.inputs[2] != kNoTensor && g.isInitializer(act.inputs[2])) hi = g.initializers[act.inputs[2]].f32()[0];
                if (act.attr.has("min")) lo = act.attr.getf("min", lo);
                if (act.attr.has("max")) hi = act.attr.getf("max", hi);
                prod.fusedAct = (lo == 0.f && hi == 6.f) ? ActType::Relu6 : ActType::Clip;
                prod.actLo    = lo;
                prod.actHi    = hi;
            }
            TensorId from = act.outputs[0], to = prod.outputs[0];
            for (Node &n: g.nodes)
                for (TensorId &t: n.inputs)
                    if (t == from) t = to;
            for (TensorId &t: g.outputs)
                if (t == from) t = to;
            drop.insert((int) i);
        }
        dropNodes(g, drop);
    }

    void fuseResidualAdd(Graph &g) {
        Uses          u(g);
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &add = g.nodes[i];
            if (add.type != OpType::Add || add.inputs.size() != 2) continue;
            int      ci = -1;
            TensorId residual = kNoTensor;
            for (int e = 0; e < 2 && ci < 0; ++e) {
                int p = u.producer[add.inputs[e]];
                if (p >= 0 && g.nodes[p].fusedResidual == kNoTensor && isPointwiseConv(g, g.nodes[p])) {
                    ci       = p;
                    residual = add.inputs[1 - e];
                }
            }
            if (ci < 0 || u.count[g.nodes[ci].outputs[0]] != 1) continue;
            Node &conv         = g.nodes[ci];
            conv.fusedResidual = residual;
            conv.inputs.push_back(residual);
            if (conv.fusedAct == ActType::None) {
                conv.fusedAct = add.fusedAct;
                conv.actLo    = add.actLo;
                conv.actHi    = add.actHi;
            }
            TensorId from = add.outputs[0], to = conv.outputs[0];
            for (Node &n: g.nodes)
                for (TensorId &t: n.inputs)
                    if (t == from) t = to;
            for (TensorId &t: g.outputs)
                if (t == from) t = to;
            drop.insert((int) i);
        }
        dropNodes(g, drop);
    }

    void fuseSwish(Graph &g) {
        Uses          u(g, false);
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            Node &M = g.nodes[i];
            if (M.type != OpType::Binary || (BinaryType) M.subOp != BinaryType::Mul || M.inputs.size() != 2) continue;
            int      gate = -1;
            TensorId x    = kNoTensor;
            for (int e = 0; e < 2 && gate < 0; ++e) {
                int pc = u.producer[M.inputs[e]];
                if (pc < 0 || g.nodes[pc].type != OpType::Unary) continue;
                UnaryType su = (UnaryType) g.nodes[pc].subOp;
                if ((su == UnaryType::HardSigmoid || su == UnaryType::Sigmoid) && g.nodes[pc].inputs[0] == M.inputs[1 - e]) {
                    gate = pc;
                    x    = M.inputs[1 - e];
                }
            }
            if (gate < 0 || u.count[g.nodes[gate].outputs[0]] != 1) continue;
            ActType act = (UnaryType) g.nodes[gate].subOp == UnaryType::HardSigmoid ? ActType::HardSwish : ActType::SiLU;
            int     px  = u.producer[x];
            bool    toProducer = px >= 0 && (g.nodes[px].type == OpType::Conv || g.nodes[px].type == OpType::Gemm) &&
                              g.nodes[px].fusedAct == ActType::None && u.count[x] == 2;
            if (toProducer) {
                g.nodes[px].fusedAct = act;
                rewireTensor(g, M.outputs[0], x);
                drop.insert((int) i);
            } else {
                M.type   = OpType::Unary;
                M.subOp  = (int32_t) (act == ActType::HardSwish ? UnaryType::HardSwish : UnaryType::SiLU);
                M.inputs = {x};
            }
            drop.insert(gate);
        }
        dropNodes(g, drop);
    }

    void fuseSqueezeExcite(Graph &g) {
        Uses          u(g, false);
        std::set<int> drop;
        auto single = [&](TensorId t) { return t != kNoTensor && u.count[t] == 1; };
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            Node &hs = g.nodes[i];
            if (hs.type != OpType::Unary || (UnaryType) hs.subOp != UnaryType::HardSigmoid) continue;
            int p2 = u.producer[hs.inputs[0]];
            if (p2 < 0 || g.nodes[p2].type != OpType::Conv || !single(g.nodes[p2].outputs[0])) continue;
            int p1 = u.producer[g.nodes[p2].inputs[0]];
            if (p1 < 0 || g.nodes[p1].type != OpType::Conv || !single(g.nodes[p1].outputs[0])) continue;
            if (g.nodes[p1].fusedAct != ActType::Relu) continue;
            int pg = u.producer[g.nodes[p1].inputs[0]];
            if (pg < 0 || g.nodes[pg].type != OpType::GlobalAvgPool) continue;
            const Node &c1 = g.nodes[p1], &c2 = g.nodes[p2];
            Node        se;
            se.type    = OpType::FusedSE;
            se.name    = c1.name + "#se";
            se.inputs  = {c1.inputs[0], c1.inputs[1], biasOf(c1), c2.inputs[1], biasOf(c2)};
            se.outputs = {hs.outputs[0]};
            se.actLo   = hs.actLo;
            se.actHi   = hs.actHi;
            g.nodes[i] = se;
            drop.insert(p1);
            drop.insert(p2);
        }
        dropNodes(g, drop);
    }

    void fuseDwPw(Graph &g) {
        Uses          u(g, false);
        std::set<int> drop;
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            const Node &P = g.nodes[i];
            if (!isPointwiseConv(g, P)) continue;
            int di = u.producer[P.inputs[0]];
            if (di < 0 || g.nodes[di].type != OpType::Conv) continue;
            const Node &D = g.nodes[di];
            if (u.count[D.outputs[0]] != 1) continue;
            const Shape &dw = g.desc(D.inputs[1]).shape;
            NCHW         dx = NCHW::from(g.desc(D.inputs[0]).shape);
            if (!(D.attr.geti("group", 1) == dx.c && dw.size() == 4 && dw[1] == 1)) continue;
            if (D.fusedAct != ActType::None && D.fusedAct != ActType::Relu && D.fusedAct != ActType::Relu6) continue;
            Node f;
            f.type   = OpType::FusedDwPw;
            f.name   = D.name + "#dwpw";
            f.inputs = {D.inputs[0], D.inputs[1], biasOf(D), P.inputs[1], biasOf(P)};
            if (P.fusedResidual != kNoTensor) {
                f.inputs.push_back(P.fusedResidual);
                f.fusedResidual = P.fusedResidual;
            }
            f.outputs  = {P.outputs[0]};
            f.attr     = D.attr;
            f.subOp    = (int32_t) D.fusedAct;
            f.fusedAct = P.fusedAct;
            f.actLo    = P.actLo;
            f.actHi    = P.actHi;
            g.nodes[i] = f;
            drop.insert(di);
        }
        dropNodes(g, drop);
    }

    void runStandardPasses(Graph &g, const PassOptions &opt) {
        foldConstantNodes(g);
        inferShapes(g, opt.batch);
        eliminateIdentity(g);
        foldBatchNorm(g);
        fuseActivations(g);
        fuseResidualAdd(g);
        if (opt.fuseSwish) fuseSwish(g);
        if (opt.fuseSqueezeExcite) fuseSqueezeExcite(g);
        if (opt.fuseDwPw) fuseDwPw(g);
        eliminateDeadNodes(g);
        inferShapes(g, opt.batch);
    }

} // namespace vknn
