// The HIP backend: vknn::Backend + Segment implementations that run the fused fp16 conv path on
// MI355X through the vkhip C ABI only (no HIP headers here). Behaviour mirrors the reference's
// Vulkan backend for this path:
//   capability gate        src/backend/vulkan/vk_backend.cpp:173-434 (supportsNode; FusedDwPw E<=1024,
//                          FusedSE C<=1024 Cr<=256; High precision declined)
//   segment                vk_backend.cpp:716-1458 (device buffers per activation, boundary pack
//                          of host NCHW fp32 into NC4HW4 fp16, one in-order queue, boundary unpack,
//                          optional per-op timing into the profiler)
//   conv op                src/backend/vulkan/ops/conv.cpp:342-553 (kernel classification,
//                          weight prepack, per-shape autotune with the 3% Winograd margin)
//   other ops              ops/fused_dwpw.cpp, ops/fused_se.cpp, ops/add.cpp, ops/binary.cpp
// MI355X-specific: the launch sequence of a segment is captured once into a HIP graph and replayed.
#include "hip_backend.h"
#include "tune_cache.h"
#include "vkhip.h"
#include "vknn/profiler.h"
#include <algorithm>
#include <functional>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <sys/stat.h>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <sstream>

namespace vknn {

    struct DeviceStorage {
        void  *ptr   = nullptr;
        size_t bytes = 0;
        bool   owned = true;
        ~DeviceStorage() {
            if (owned && ptr) vkhip_free(ptr);
        }
    };

    namespace hipbe {

        void check(int rc, const std::string &what) {
            if (rc) throw Error(Status::RuntimeError, what + ": " + vkhip_last_error());
        }

        DevBuf::DevBuf(size_t n): bytes(n) { check(vkhip_malloc(&ptr, std::max<size_t>(n, 256)), "device allocation"); }
        DevBuf::~DevBuf() {
            if (ptr) vkhip_free(ptr);
        }

        // A conv workspace, zeroed: split-K plans that reduce in the kernel (VKHIP_CONV_SPLITK_LAST)
        // keep arrival counters in it that must start at zero (each call leaves them zero).
        std::shared_ptr<DevBuf> workspace(size_t bytes) {
            if (!bytes) return nullptr;
            auto b = std::make_shared<DevBuf>(bytes);
            check(vkhip_fill_zero(b->ptr, bytes, nullptr), "workspace fill");
            return b;
        }

        std::shared_ptr<DevBuf> upload(const void *host, size_t bytes) {
            auto b = std::make_shared<DevBuf>(bytes);
            check(vkhip_memcpy_h2d(b->ptr, host, bytes, nullptr), "weight upload");
            return b;
        }

        static std::vector<int64_t> attrInts(const Node &n, const char *k, std::vector<int64_t> d) {
            const auto &v = n.attr.getints(k);
            return v.empty() ? d : v;
        }

        // Plans a stem conv + max pool may take: thin tile 45 (conv_thin_pool_kernel, the 7x7 stride-2
        // stem); VKNN_HIP_FUSE_POOL=1 adds the 64-row stem tiles (stem_pool_kernel, slower than the
        // two launches on the ResNet-50 stem: kept for other stems).
        static std::vector<int> poolTiles() {
            const char *e = std::getenv("VKNN_HIP_FUSE_POOL");
            if (e && std::string(e) == "1") return {45, 21, 22};
            return {45};
        }

        static const float *initF32(const Graph &g, TensorId id) {
            if (id == kNoTensor) return nullptr;
            auto it = g.initializers.find(id);
            if (it == g.initializers.end()) throw Error(Status::Unsupported, "HIP backend needs constant weights (tensor " + g.desc(id).name + ")");
            return it->second.f32();
        }

        static TensorId biasOf(const Node &c) {
            if (c.inputs.size() > 2 && c.inputs[2] != c.fusedResidual) return c.inputs[2];
            return kNoTensor;
        }

        size_t nc4Bytes(const Shape &s) { return (size_t) formatElems(TensorFormat::NC4HW4, NCHW::from(s)) * 2; }

        // The descriptor of a dense conv node as it runs on its own (no residual, no folds).
        static vkhip_conv_desc convDescOf(const Graph &g, const Node &node) {
            vkhip_conv_desc d {};
            NCHW         x  = NCHW::from(g.desc(node.inputs[0]).shape);
            NCHW         y  = NCHW::from(g.desc(node.outputs[0]).shape);
            const Shape &ws = g.desc(node.inputs[1]).shape;
            auto st = attrInts(node, "strides", {1, 1}), pad = attrInts(node, "pads", {0, 0, 0, 0}), dil = attrInts(node, "dilations", {1, 1});
            d.N = (int) x.n; d.Cin = (int) x.c; d.H = (int) x.h; d.W = (int) x.w;
            d.Cout = (int) ws[0]; d.OH = (int) y.h; d.OW = (int) y.w;
            d.KH = (int) ws[2]; d.KW = (int) ws[3]; d.SH = (int) st[0]; d.SW = (int) st[1];
            d.PT = (int) pad[0]; d.PL = (int) pad[1]; d.DH = (int) dil[0]; d.DW = (int) dil[1];
            d.group = (int) node.attr.geti("group", 1);
            d.act = (int) node.fusedAct; d.act_lo = node.actLo; d.act_hi = node.actHi;
            return d;
        }

        // ------------------------------------------------------------ conv autotune cache
        // Keyed by the conv geometry under the per-GPU tag; the chosen (algo, tile, ksplit) lives in
        // the process-wide TuneCache, which Config::cacheFile persists across processes (the
        // reference's tune table: ops/conv.cpp:195-238 keys, vk_backend.cpp:30-150 storage).
        static std::string keyOf(const vkhip_conv_desc &d, int mode) {
            std::string k = gpuTag() + "/conv";
            for (int v: {d.N, d.Cin, d.H, d.W, d.Cout, d.OH, d.OW, d.KH, d.KW, d.SH, d.SW, d.PT, d.PL, d.DH, d.DW, d.group, d.has_res, mode})
                k += "_" + std::to_string(v);
            if (d.in_scale) k += "_xs";
            return k;
        }
        // (algo, tile, ksplit) <-> one i32 table value: algo in bits 0-7, tile+1 in 8-15, ksplit in 16-23
        static int32_t encodePick(const std::array<int32_t, 3> &p) { return (p[0] & 0xff) | (((p[1] + 1) & 0xff) << 8) | ((p[2] & 0xff) << 16); }
        static std::array<int32_t, 3> decodePick(int32_t v) { return {v & 0xff, ((v >> 8) & 0xff) - 1, (v >> 16) & 0xff}; }

        // In-graph plan refinement (HipSegment::refinePlans) is on unless VKNN_HIP_REFINE=0.
        static bool refineEnabled() {
            const char *e = std::getenv("VKNN_HIP_REFINE");
            return !(e && e[0] == '0');
        }

        // ------------------------------------------------------------ conv
        struct ConvOp: HipOp {
            vkhip_conv_desc         d {};
            vkhip_conv_plan         plan {};
            std::shared_ptr<DevBuf> blob, ws;
            TensorId                in = kNoTensor, out = kNoTensor, res = kNoTensor;
            // Set by the segment before prepare when a channel-broadcast Mul (the squeeze-excite
            // scale) is folded into this conv: the conv reads the Mul's unscaled operand `scaledIn`
            // and multiplies it by `xscale` ([N,C,1,1]) on the way into the GEMM.
            TensorId                scaledIn = kNoTensor, xscale = kNoTensor;
            // Set by the segment when the 3x3 stride-2 max pool that is this conv's only reader is
            // fused into it (a first-layer conv): the conv writes the pooled tensor `poolOut` and
            // its own output never exists in memory.
            TensorId                poolOut = kNoTensor;
            vkhip_pool_desc         pd {};
            // Set by the segment before prepare when the hard-sigmoid that is this conv's only reader
            // is folded into its epilogue (the squeeze-excite gate after the second FC): the conv
            // writes `actOut` with activation `foldAct` (lo, hi) instead of its own output.
            TensorId                actOut = kNoTensor;
            int                     foldAct = 0;
            float                   foldLo = 0.f, foldHi = 0.f;
            // Set by the segment before prepare when the Add that is this conv's only reader (the
            // conv already applies its own activation) is folded into its epilogue: the conv writes
            // the Add's output `addOut` = act(conv + bias) + `postRes` (a residual after the
            // activation, has_res 2).
            TensorId                addOut = kNoTensor, postRes = kNoTensor;
            // Set by the segment after prepare when the global average pool of a squeeze-excite
            // that reads this depthwise conv's output is folded into it: the conv also writes the
            // per-(plane, row tile) sums of its output into `gapPart` (gapR partials per plane).
            std::shared_ptr<DevBuf> gapPart;
            int                     gapR = 0;
            // Set by the segment before prepare when the conv reads or writes a view (a slice of an
            // in-place concat or split): the plan is then a GEMM or split-K one (no Winograd).
            bool                    viewIO = false;
            bool                    cacheWeights = false; // keep the prepacked blob in the cache file
            // The tuner's near-ties for the in-graph refinement (HipSegment::refinePlans), each with
            // its packed blob and workspace; [0] is the tuner's pick. Empty unless this op was tuned.
            struct Cand {
                vkhip_conv_plan         p {};
                std::shared_ptr<DevBuf> blob, ws;
                std::vector<uint8_t>    host; // kept for the cache file's weight section
                std::string             wkey;
            };
            std::vector<Cand> nearTies;
            std::string       tuneKey;

            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                cacheWeights   = env.config->cachesWeights() && !env.config->cacheFile.empty();
                in             = scaledIn != kNoTensor ? scaledIn : node.inputs[0];
                out            = actOut != kNoTensor ? actOut : addOut != kNoTensor ? addOut : node.outputs[0];
                res            = postRes != kNoTensor ? postRes : node.fusedResidual;
                NCHW         x  = NCHW::from(g.desc(in).shape);
                NCHW         y  = NCHW::from(g.desc(out).shape);
                const Shape &ws_ = g.desc(node.inputs[1]).shape;
                auto st  = attrInts(node, "strides", {1, 1});
                auto pad = attrInts(node, "pads", {0, 0, 0, 0});
                auto dil = attrInts(node, "dilations", {1, 1});
                d.N = (int) x.n; d.Cin = (int) x.c; d.H = (int) x.h; d.W = (int) x.w;
                d.Cout = (int) ws_[0]; d.OH = (int) y.h; d.OW = (int) y.w;
                d.KH = (int) ws_[2]; d.KW = (int) ws_[3]; d.SH = (int) st[0]; d.SW = (int) st[1];
                d.PT = (int) pad[0]; d.PL = (int) pad[1]; d.DH = (int) dil[0]; d.DW = (int) dil[1];
                d.group = (int) node.attr.geti("group", 1);
                d.act = (int) node.fusedAct; d.act_lo = node.actLo; d.act_hi = node.actHi;
                if (actOut != kNoTensor) d.act = foldAct, d.act_lo = foldLo, d.act_hi = foldHi;
                d.has_res = postRes != kNoTensor ? 2 : res != kNoTensor ? 1 : 0;
                d.in_scale = xscale != kNoTensor;
                kind  = d.group > 1 ? "dwconv" : "conv";
                flops = 2.0 * d.N * d.Cout * (double) (d.Cin / d.group) * d.KH * d.KW * d.OH * d.OW;
                bytes = (int64_t) (nc4Bytes(g.desc(in).shape) + nc4Bytes(g.desc(out).shape) * (d.has_res ? 2 : 1)) +
                        (int64_t) d.Cout * (d.Cin / d.group) * d.KH * d.KW * 2;
                const float *w = initF32(g, node.inputs[1]);
                const float *b = initF32(g, biasOf(node));
                if (poolOut != kNoTensor) {
                    // the fused stem + pool kernel: the thin tile, or (opt-in) the 64-row stem tiles
                    bool ok = false;
                    for (int t: poolTiles())
                        if (!ok && vkhip_conv_plan_make(&d, VKHIP_CONV_GEMM, t, 0, &plan) == VKHIP_OK && vkhip_conv_maxpool_supported(&d, &plan, &pd)) ok = true;
                    if (!ok) throw Error(Status::RuntimeError, "conv + max pool fusion planned for an unsupported shape: " + name);
                    bytes = (int64_t) (nc4Bytes(g.desc(in).shape) + nc4Bytes(g.desc(poolOut).shape)) + (int64_t) d.Cout * d.Cin * d.KH * d.KW * 2;
                    build(w, b);
                    return;
                }
                choosePlan(env, w, b);
            }

            // Cache key of the prepacked blob: the node, its conv signature and plan, the blob layout
            // version (VKHIP_PACK_FORMAT) and a hash of the source weights and bias (a changed model,
            // plan or packer never takes a stale blob). The
            // reference keys its blobs by model tag + node + role (vk_op_common.h uploadCached).
            std::string weightKey(const float *w, const float *b) const { return weightKey(w, b, plan); }
            std::string weightKey(const float *w, const float *b, const vkhip_conv_plan &pl) const {
                uint64_t h = 1469598103934665603ull; // FNV-1a, 64 bit, over the fp32 bytes
                auto mix = [&](const float *p, size_t n) {
                    const uint8_t *c = reinterpret_cast<const uint8_t *>(p);
                    for (size_t i = 0; i < n * 4; ++i) h = (h ^ c[i]) * 1099511628211ull;
                };
                mix(w, (size_t) d.Cout * (d.Cin / d.group) * d.KH * d.KW);
                if (b) mix(b, (size_t) d.Cout);
                char tail[96];
                std::snprintf(tail, sizeof tail, "#p%d_%d_%d#f%d#%016llx", pl.algo, pl.tile, pl.ksplit, VKHIP_PACK_FORMAT,
                              (unsigned long long) h);
                return gpuTag() + "/w/" + name + keyOf(d, 0).substr(gpuTag().size()) + tail;
            }

            void build(const float *w, const float *b) {
                // a view conv runs GEMM or split-K plans only (no Winograd transforms over views)
                if (viewIO && plan.algo == VKHIP_CONV_WINOGRAD) check(vkhip_conv_plan_make(&d, VKHIP_CONV_GEMM, -1, 0, &plan), "conv plan");
                // warm start: the prepacked blob from the cache file's weight section (CacheMode::Full
                // with a cache file, reference uploadCached); packed and retained on a miss
                std::vector<uint8_t> host;
                std::string          wkey;
                if (cacheWeights) {
                    wkey = weightKey(w, b);
                    if (!TuneCache::instance().getWeights(wkey, plan.weight_bytes, host)) host.clear();
                }
                if (host.empty()) {
                    host.resize(plan.weight_bytes);
                    check(vkhip_conv_pack_weights(&d, &plan, w, b, host.data()), "conv weight pack");
                    if (cacheWeights) TuneCache::instance().putWeights(wkey, host);
                }
                blob = upload(host.data(), host.size());
                ws   = workspace(plan.workspace_bytes);
            }

            void choosePlan(SegEnv &env, const float *w, const float *b) {
                const Config &cfg    = *env.config;
                const int     tuning = cfg.hint(Hint::Tuning, (int) Mode::Fast);
                const int     wino   = cfg.hint(Hint::Winograd, (int) Mode::Auto);
                const bool dw = d.group > 1;
                if (dw && (tuning == (int) Mode::NoTune || !env.tunable)) {
                    check(vkhip_conv_plan_make(&d, VKHIP_CONV_DEPTHWISE, -1, 0, &plan), "conv plan");
                    build(w, b);
                    return;
                }
                vkhip_conv_plan tmp;
                const bool wino_ok = !dw && !viewIO && vkhip_conv_plan_make(&d, VKHIP_CONV_WINOGRAD, -1, 0, &tmp) == VKHIP_OK && d.Cin >= 32 && d.Cout >= 32;
                if (wino == (int) Mode::On && wino_ok) {
                    check(vkhip_conv_plan_make(&d, VKHIP_CONV_WINOGRAD, -1, 0, &plan), "conv plan");
                    build(w, b);
                    return;
                }
                if (tuning == (int) Mode::NoTune || !env.tunable) {
                    check(vkhip_conv_plan_make(&d, VKHIP_CONV_AUTO, -1, 0, &plan), "conv plan");
                    build(w, b);
                    return;
                }
                const std::string key = keyOf(d, tuning * 4 + wino) + (viewIO ? "_view" : "");
                tuneKey               = key;
                int32_t           cached = 0;
                if (TuneCache::instance().get(key, cached)) {
                    // an entry that no longer makes a plan (e.g. written by another build) is re-tuned
                    const auto c = decodePick(cached);
                    if (vkhip_conv_plan_make(&d, c[0], c[1], c[2], &plan) == VKHIP_OK) {
                        build(w, b);
                        return;
                    }
                }
                // Candidates: every GEMM tile, split-K for low-parallelism shapes, Winograd if eligible.
                std::vector<std::array<int32_t, 3>> cands;
                const int ntiles = dw ? 0 : vkhip_conv_tile_count();
                // VKNN_HIP_SKIP_TILES=a,b,...: tiles the tuner leaves out (A/B measurements)
                std::set<int> skipTiles;
                if (const char *st = std::getenv("VKNN_HIP_SKIP_TILES")) {
                    std::stringstream ss(st);
                    std::string       tok;
                    while (std::getline(ss, tok, ','))
                        if (!tok.empty()) skipTiles.insert(std::atoi(tok.c_str()));
                }
                for (int t = 0; t < ntiles; ++t)
                    if (!skipTiles.count(t)) cands.push_back({VKHIP_CONV_GEMM, t, 0});
                if (dw) // the depthwise kernel's rows per strip
                    // + 100 x strips per workgroup, 900: persistent plane groups (VKNN_HIP_DW_PIPE=0: one strip only)
                    for (int rt: {4, 7, 14, 204, 207, 404, 407, 907, 914})
                        if (rt < 100 || !(std::getenv("VKNN_HIP_DW_PIPE") && std::getenv("VKNN_HIP_DW_PIPE")[0] == '0'))
                            cands.push_back({VKHIP_CONV_DEPTHWISE, rt, 0});
                vkhip_conv_plan base;
                check(vkhip_conv_plan_make(&d, VKHIP_CONV_AUTO, -1, 0, &base), "conv plan");
                int64_t pixels = (int64_t) d.N * d.OH * d.OW;
                // Split-K when the direct grid cannot fill the device (fewer than ~2 workgroups per CU
                // with the big tiles) and the reduction is deep enough to split.
                const int64_t kdepth = (int64_t) d.KH * d.KW * ((d.Cin + 3) / 4) * 4;
                if (!dw && (pixels <= 4096 || base.algo == VKHIP_CONV_SPLITK || (pixels * (int64_t) d.Cout <= (int64_t) 512 * 128 * 256 && kdepth >= 512))) {
                    for (int t: {3, 6, 1, 8, 10, 14, 16, 17, 18, 20, 26})
                        for (int ks: {2, 3, 4, 8, 16})
                            for (int alg: {VKHIP_CONV_SPLITK, VKHIP_CONV_SPLITK_LAST}) cands.push_back({alg, t, ks});
                }
                if (tuning != (int) Mode::Thorough) {
                    // Fast: the heuristic pick, the tiles that win somewhere on the config shapes, and
                    // the split-K set.
                    std::vector<std::array<int32_t, 3>> keep;
                    for (auto &c: cands)
                        if (c[0] == VKHIP_CONV_SPLITK || c[0] == VKHIP_CONV_SPLITK_LAST || c[0] == VKHIP_CONV_DEPTHWISE || c[1] == base.tile || c[1] == 0 || c[1] == 1 || c[1] == 3 || c[1] == 5 ||
                            c[1] == 7 || c[1] >= 8)
                            keep.push_back(c);
                    cands = keep;
                }
                double                 best = 1e30, bestDirect = 1e30;
                std::array<int32_t, 3> pick = {base.algo, base.tile, base.ksplit};
                // Candidates run as the network runs them (with the residual read when the conv has
                // one) on rotating buffer sets whose total exceeds the GPU's 256 MB last-level
                // cache, so memory-bound layers are timed from HBM like in a full forward pass
                // rather than from cache-resident repeats of one input.
                const size_t xbytes = nc4Bytes({d.N, d.Cin, d.H, d.W}), ybytes = nc4Bytes({d.N, d.Cout, d.OH, d.OW});
                const size_t set_bytes = xbytes + ybytes * (d.has_res ? 2 : 1);
                const int    nset      = (int) std::min<size_t>(6, std::max<size_t>(1, ((size_t) 640 << 20) / std::max<size_t>(set_bytes, 1) + 1));
                std::vector<TuneSet> sets;
                for (int k = 0; k < nset; ++k) {
                    TuneSet t;
                    t.x = std::make_shared<DevBuf>(xbytes);
                    t.y = std::make_shared<DevBuf>(ybytes);
                    check(vkhip_fill_zero(t.x->ptr, xbytes, nullptr), "tune fill");
                    check(vkhip_fill_zero(t.y->ptr, ybytes, nullptr), "tune fill");
                    if (d.has_res) {
                        t.r = std::make_shared<DevBuf>(ybytes);
                        check(vkhip_fill_zero(t.r->ptr, ybytes, nullptr), "tune fill");
                    }
                    if (d.in_scale) {
                        t.s = std::make_shared<DevBuf>(nc4Bytes({d.N, d.Cin, 1, 1}));
                        check(vkhip_fill_zero(t.s->ptr, t.s->bytes, nullptr), "tune fill");
                    }
                    sets.push_back(t);
                }
                // two rounds: every candidate briefly, then the four fastest again with more
                // repetitions, so near-ties are decided on a steadier measurement
                std::vector<std::pair<double, std::array<int32_t, 3>>> timed;
                for (auto &c: cands) {
                    vkhip_conv_plan p;
                    if (vkhip_conv_plan_make(&d, c[0], c[1], c[2], &p)) continue;
                    timed.push_back({timePlan(p, w, b, sets, 2), {p.algo, p.tile, p.ksplit}});
                }
                std::sort(timed.begin(), timed.end(), [](const auto &x, const auto &y) { return x.first < y.first; });
                for (size_t i = 0; i < timed.size() && i < 4; ++i) {
                    vkhip_conv_plan p;
                    const auto &c = timed[i].second;
                    if (vkhip_conv_plan_make(&d, c[0], c[1], c[2], &p)) continue;
                    const double ms = std::min(timed[i].first, timePlan(p, w, b, sets, 6));
                    if (ms < best) {
                        best = ms;
                        pick = c;
                    }
                }
                bestDirect = best;
                if (wino_ok && wino != (int) Mode::Off) {
                    // the position GEMMs on the heuristic tile and on the register-/DMA-fed tiles
                    double bestWino = 1e30;
                    std::array<int32_t, 3> wpick {};
                    for (int t: {-1, 8, 10, 14, 12, 16}) {
                        vkhip_conv_plan p;
                        if (vkhip_conv_plan_make(&d, VKHIP_CONV_WINOGRAD, t, 0, &p)) continue;
                        double ms = timePlan(p, w, b, sets, 6);
                        if (ms < bestWino) {
                            bestWino = ms;
                            wpick    = {p.algo, p.tile, p.ksplit};
                        }
                    }
                    // Winograd must win by 3% (reference ops/conv.cpp:16 kWinoMargin) so timing noise
                    // cannot flip a near-tie between kernels that round differently.
                    if (bestWino < bestDirect * 0.97) pick = wpick;
                }
                TuneCache::instance().put(key, encodePick(pick));
                check(vkhip_conv_plan_make(&d, pick[0], pick[1], pick[2], &plan), "conv plan");
                build(w, b);
                if (refineEnabled() && !viewIO) {
                    // near-ties (within 12% of the pick on the isolated shape), at most three
                    std::vector<std::array<int32_t, 3>> alts;
                    for (auto &t: timed)
                        if (t.second != pick && t.first <= best * 1.12 && alts.size() < 3) alts.push_back(t.second);
                    if (!alts.empty()) {
                        nearTies.push_back({plan, blob, ws, {}, {}});
                        for (auto &c: alts) {
                            Cand k;
                            if (vkhip_conv_plan_make(&d, c[0], c[1], c[2], &k.p)) continue;
                            k.host.resize(k.p.weight_bytes);
                            if (vkhip_conv_pack_weights(&d, &k.p, w, b, k.host.data())) continue;
                            k.blob = upload(k.host.data(), k.host.size());
                            k.ws   = workspace(k.p.workspace_bytes);
                            if (cacheWeights) k.wkey = weightKey(w, b, k.p);
                            else k.host.clear();
                            nearTies.push_back(std::move(k));
                        }
                        if (nearTies.size() < 2) nearTies.clear();
                    }
                }
            }

            std::string planKey() const override { return tuneKey; }
            int  candidates() const override { return gapPart || poolOut != kNoTensor ? 0 : (int) nearTies.size(); }
            void useCandidate(int j) override {
                plan = nearTies[j].p;
                blob = nearTies[j].blob;
                ws   = nearTies[j].ws;
            }
            void commitCandidate(int j) override {
                if (nearTies.empty()) return;
                useCandidate(j);
                if (j > 0) {
                    TuneCache::instance().put(tuneKey, encodePick({plan.algo, plan.tile, plan.ksplit}));
                    if (cacheWeights && !nearTies[j].host.empty()) TuneCache::instance().putWeights(nearTies[j].wkey, nearTies[j].host);
                }
                nearTies.clear();
            }

            struct TuneSet {
                std::shared_ptr<DevBuf> x, y, r, s;
            };

            // min over reps timings of 6 back-to-back launches, each on the next buffer set
            double timePlan(const vkhip_conv_plan &p, const float *w, const float *b, const std::vector<TuneSet> &sets, int reps) {
                std::vector<uint8_t> host(p.weight_bytes);
                if (vkhip_conv_pack_weights(&d, &p, w, b, host.data())) return 1e30;
                auto   bl  = upload(host.data(), host.size());
                auto   wsb = workspace(p.workspace_bytes);
                size_t k   = 0;
                auto   run = [&]() {
                    const TuneSet &t = sets[k++ % sets.size()];
                    return forward(p, t.x->ptr, t.s ? t.s->ptr : nullptr, bl->ptr, t.r ? t.r->ptr : nullptr, t.y->ptr, wsb ? wsb->ptr : nullptr, nullptr);
                };
                vkhip_event_t e0, e1;
                check(vkhip_event_create(&e0), "event");
                check(vkhip_event_create(&e1), "event");
                double best = 1e30;
                if (run() == VKHIP_OK) {
                    for (int r = 0; r < reps; ++r) {
                        vkhip_event_record(e0, nullptr);
                        for (int i = 0; i < 6; ++i) run();
                        vkhip_event_record(e1, nullptr);
                        vkhip_event_sync(e1);
                        float ms = 0;
                        vkhip_event_elapsed_ms(e0, e1, &ms);
                        best = std::min(best, (double) ms);
                    }
                }
                check(vkhip_stream_sync(nullptr), "tune sync");
                vkhip_event_destroy(e0);
                vkhip_event_destroy(e1);
                return best;
            }

            int forward(const vkhip_conv_plan &p, const void *x, const void *xs, const void *bl, const void *r, void *y, void *w, vkhip_stream_t s) {
                return d.in_scale ? vkhip_conv_forward_scaled(&d, &p, x, xs, bl, r, y, w, s) : vkhip_conv_forward(&d, &p, x, bl, r, y, w, s);
            }

            void record(SegEnv &env, vkhip_stream_t s) override {
                if (poolOut != kNoTensor) {
                    check(vkhip_conv_maxpool_forward(&d, &plan, &pd, env.dev(in), blob->ptr, env.dev(poolOut), s), "conv + max pool " + name);
                    return;
                }
                if (gapPart) {
                    check(vkhip_conv_forward_pooled(&d, &plan, env.dev(in), blob->ptr, res != kNoTensor ? env.dev(res) : nullptr, env.dev(out),
                                                    gapPart->ptr, s),
                          "conv + pool sums " + name);
                    return;
                }
                if (viewIO) {
                    if (res != kNoTensor)
                        check(vkhip_conv_forward_view_res(&d, &plan, env.dev(in), env.pstride(in), blob->ptr, env.dev(res), env.dev(out), env.pstride(out),
                                                          ws ? ws->ptr : nullptr, s),
                              "conv " + name);
                    else
                        check(vkhip_conv_forward_view(&d, &plan, env.dev(in), env.pstride(in), blob->ptr, env.dev(out), env.pstride(out),
                                                      ws ? ws->ptr : nullptr, s),
                              "conv " + name);
                    return;
                }
                check(forward(plan, env.dev(in), xscale != kNoTensor ? env.dev(xscale) : nullptr, blob->ptr,
                              res != kNoTensor ? env.dev(res) : nullptr, env.dev(out), ws ? ws->ptr : nullptr, s),
                      "conv " + name);
            }

            std::string describe() const override {
                static const char *algos[] = {"auto", "gemm", "splitk", "winograd", "depthwise", "splitk_last"};
                return std::string(algos[plan.algo]) + " tile=" + std::to_string(plan.tile) + " ksplit=" + std::to_string(plan.ksplit) +
                       (d.in_scale ? " +input scale" : "") + (poolOut != kNoTensor ? " +max pool" : "") + (gapPart ? " +pool sums" : "") + " kernel=" +
                       (poolOut != kNoTensor ? std::string(plan.tile == 45 ? "conv_thin_pool_kernel" : "stem_pool_kernel") : std::string(vkhip_conv_plan_kernel(&plan)));
            }
        };

        // ------------------------------------------------------------ fused dw + pw
        struct DwPwOp: HipOp {
            vkhip_dwpw_desc         d {};
            std::shared_ptr<DevBuf> blob, mid;
            TensorId                in, out, res = kNoTensor;
            // Either the fused kernel, or the depthwise and projection convs back to back on the
            // tuned single-op kernels with the E-channel intermediate in HBM: the fused kernel
            // keeps that intermediate on chip but its depthwise stage is slower than the tiled
            // depthwise kernel, so prepare() times both on the real shape and keeps the faster.
            bool                    split = false;
            ConvOp                  dwc, pwc;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                in  = node.inputs[0];
                out = node.outputs[0];
                res = node.fusedResidual;
                NCHW x = NCHW::from(g.desc(in).shape), y = NCHW::from(g.desc(out).shape);
                const Shape &dws = g.desc(node.inputs[1]).shape;
                auto st = attrInts(node, "strides", {1, 1}), pad = attrInts(node, "pads", {0, 0, 0, 0}), dil = attrInts(node, "dilations", {1, 1});
                vkhip_conv_desc &c = d.dw;
                c.N = (int) x.n; c.Cin = (int) x.c; c.H = (int) x.h; c.W = (int) x.w; c.Cout = (int) x.c; c.OH = (int) y.h; c.OW = (int) y.w;
                c.KH = (int) dws[2]; c.KW = (int) dws[3]; c.SH = (int) st[0]; c.SW = (int) st[1]; c.PT = (int) pad[0]; c.PL = (int) pad[1];
                c.DH = (int) dil[0]; c.DW = (int) dil[1]; c.group = (int) x.c; c.act = node.subOp; c.act_lo = 0; c.act_hi = 6;
                d.Cout = (int) y.c; d.act = (int) node.fusedAct; d.act_lo = node.actLo; d.act_hi = node.actHi; d.has_res = res != kNoTensor;
                if (!vkhip_dwpw_supported(&d)) throw Error(Status::Unsupported, "FusedDwPw shape not supported: " + name);
                const float *dw_w = initF32(g, node.inputs[1]), *dw_b = initF32(g, node.inputs[2]);
                const float *pw_w = initF32(g, node.inputs[3]), *pw_b = initF32(g, node.inputs[4]);
                std::vector<uint8_t> host(vkhip_dwpw_weight_bytes(&d));
                check(vkhip_dwpw_pack_weights(&d, dw_w, dw_b, pw_w, pw_b, host.data()), "dwpw pack");
                blob  = upload(host.data(), host.size());
                kind  = "dwpw";
                flops = 2.0 * c.N * c.OH * c.OW * ((double) c.Cin * c.KH * c.KW + (double) c.Cin * d.Cout);
                bytes = (int64_t) (nc4Bytes(g.desc(in).shape) + nc4Bytes(g.desc(out).shape) * (d.has_res ? 2 : 1));

                // the split alternative: depthwise conv (+ its activation), then the 1x1 projection
                // (+ residual + activation), both planned like standalone convs
                dwc.d = c;
                dwc.d.has_res = 0;
                pwc.d = vkhip_conv_desc {};
                pwc.d.N = c.N; pwc.d.Cin = c.Cin; pwc.d.H = c.OH; pwc.d.W = c.OW; pwc.d.Cout = d.Cout; pwc.d.OH = c.OH; pwc.d.OW = c.OW;
                pwc.d.KH = 1; pwc.d.KW = 1; pwc.d.SH = 1; pwc.d.SW = 1; pwc.d.DH = 1; pwc.d.DW = 1; pwc.d.group = 1;
                pwc.d.act = d.act; pwc.d.act_lo = d.act_lo; pwc.d.act_hi = d.act_hi; pwc.d.has_res = d.has_res;
                if (!env.tunable) return; // untuned sessions keep the fused kernel
                dwc.choosePlan(env, dw_w, dw_b);
                pwc.choosePlan(env, pw_w, pw_b);
                mid = std::make_shared<DevBuf>(nc4Bytes({c.N, c.Cin, c.OH, c.OW}));
                std::string key = gpuTag() + "/dwpw";
                for (int v: {c.N, c.Cin, c.H, c.W, c.OH, c.OW, c.KH, c.KW, c.SH, c.SW, c.PT, c.PL, d.Cout, d.has_res})
                    key += "_" + std::to_string(v);
                int32_t cached = 0;
                if (TuneCache::instance().get(key, cached)) {
                    split = cached != 0;
                    if (!split) mid.reset();
                    return;
                }
                auto xb = std::make_shared<DevBuf>(nc4Bytes({c.N, c.Cin, c.H, c.W}));
                auto yb = std::make_shared<DevBuf>(nc4Bytes({c.N, d.Cout, c.OH, c.OW}));
                auto rb = d.has_res ? std::make_shared<DevBuf>(nc4Bytes({c.N, d.Cout, c.OH, c.OW})) : nullptr;
                check(vkhip_fill_zero(xb->ptr, xb->bytes, nullptr), "dwpw tune fill");
                if (rb) check(vkhip_fill_zero(rb->ptr, rb->bytes, nullptr), "dwpw tune fill");
                auto timeIt = [&](bool sp) {
                    vkhip_event_t e0, e1;
                    check(vkhip_event_create(&e0), "event");
                    check(vkhip_event_create(&e1), "event");
                    double best = 1e30;
                    for (int r = 0; r < 4; ++r) {
                        vkhip_event_record(e0, nullptr);
                        for (int k = 0; k < 3; ++k) launch(sp, xb->ptr, rb ? rb->ptr : nullptr, yb->ptr, nullptr);
                        vkhip_event_record(e1, nullptr);
                        vkhip_event_sync(e1);
                        float ms = 0;
                        vkhip_event_elapsed_ms(e0, e1, &ms);
                        if (r > 0) best = std::min(best, (double) ms); // first round warms up
                    }
                    vkhip_event_destroy(e0);
                    vkhip_event_destroy(e1);
                    return best;
                };
                split = timeIt(true) < timeIt(false);
                TuneCache::instance().put(key, split ? 1 : 0);
                if (!split) mid.reset();
            }
            void launch(bool sp, const void *x, const void *r, void *y, vkhip_stream_t s) {
                if (!sp) {
                    check(vkhip_dwpw_forward(&d, x, blob->ptr, r, y, s), "dwpw " + name);
                    return;
                }
                check(vkhip_conv_forward(&dwc.d, &dwc.plan, x, dwc.blob->ptr, nullptr, mid->ptr, dwc.ws ? dwc.ws->ptr : nullptr, s), "dwpw dw " + name);
                check(vkhip_conv_forward(&pwc.d, &pwc.plan, mid->ptr, pwc.blob->ptr, r, y, pwc.ws ? pwc.ws->ptr : nullptr, s), "dwpw pw " + name);
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                launch(split, env.dev(in), res != kNoTensor ? env.dev(res) : nullptr, env.dev(out), s);
            }
            std::string describe() const override { return split ? "split: dw + 1x1" : "fused kernel"; }
        };

        // ------------------------------------------------------------ fused SE middle
        struct SeOp: HipOp {
            std::shared_ptr<DevBuf> blob, ws;
            TensorId                in, out;
            int64_t                 N, C, Cr;
            float                   alpha, beta;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                in  = node.inputs[0];
                out = node.outputs[0];
                NCHW x = NCHW::from(g.desc(in).shape);
                N = x.n; C = x.c; Cr = g.desc(node.inputs[1]).shape[0];
                alpha = node.actLo; beta = node.actHi;
                std::vector<uint8_t> host(vkhip_se_weight_bytes(C, Cr));
                check(vkhip_se_pack_weights(C, Cr, initF32(g, node.inputs[1]), initF32(g, node.inputs[2]), initF32(g, node.inputs[3]),
                                            initF32(g, node.inputs[4]), host.data()),
                      "se pack");
                blob  = upload(host.data(), host.size());
                ws    = workspace(vkhip_se_workspace_bytes(N, Cr));
                kind  = "se";
                flops = 4.0 * N * C * Cr;
                bytes = (int64_t) (host.size() + (size_t) N * ((C + 3) / 4 * 4) * 2 * 2);
            }
            // set by the segment when the average pool before this op is folded into the depthwise
            // conv that feeds it: the squeeze input comes from that conv's partial sums
            std::shared_ptr<DevBuf> part;
            int                     R  = 0;
            int64_t                 HW = 0;
            void record(SegEnv &env, vkhip_stream_t s) override {
                if (part) check(vkhip_fused_se_pooled(part->ptr, R, HW, blob->ptr, env.dev(out), N, C, Cr, alpha, beta, ws->ptr, s), "fused_se " + name);
                else check(vkhip_fused_se(env.dev(in), blob->ptr, env.dev(out), N, C, Cr, alpha, beta, ws->ptr, s), "fused_se " + name);
            }
            std::string describe() const override { return part ? "pool folded into the depthwise conv" : ""; }
        };

        // ------------------------------------------------------------ Gemm (FC head) as a 1x1 conv
        struct GemmOp: HipOp {
            std::unique_ptr<ConvOp> conv;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g  = *env.graph;
                const Shape &as = g.desc(node.inputs[0]).shape;
                const Shape &bs = g.desc(node.inputs[1]).shape;
                if (as.size() != 2 || node.attr.geti("transA", 0)) throw Error(Status::Unsupported, "Gemm: only A [M,K] without transA");
                const int64_t M = as[0], K = as[1];
                const bool    tB = node.attr.geti("transB", 0) != 0;
                const int64_t Nn = tB ? bs[0] : bs[1];
                const float   alpha = node.attr.getf("alpha", 1.f), beta = node.attr.getf("beta", 1.f);
                const float  *B     = initF32(g, node.inputs[1]);
                const float  *Cv    = node.inputs.size() > 2 ? initF32(g, node.inputs[2]) : nullptr;
                if (Cv && numElements(g.desc(node.inputs[2]).shape) != Nn) throw Error(Status::Unsupported, "Gemm: C must be [N]");
                std::vector<float> w((size_t) (Nn * K)), b((size_t) Nn, 0.f);
                for (int64_t n = 0; n < Nn; ++n) {
                    for (int64_t k = 0; k < K; ++k) w[n * K + k] = alpha * (tB ? B[n * K + k] : B[k * Nn + n]);
                    if (Cv) b[n] = beta * Cv[n];
                }
                conv        = std::make_unique<ConvOp>();
                conv->name  = name;
                conv->in    = in  = node.inputs[0];
                conv->out   = out = node.outputs[0];
                vkhip_conv_desc &d = conv->d;
                d.N = (int) M; d.Cin = (int) K; d.H = d.W = 1; d.Cout = (int) Nn; d.OH = d.OW = 1; d.KH = d.KW = 1;
                d.SH = d.SW = d.DH = d.DW = 1; d.group = 1; d.act = (int) node.fusedAct; d.act_lo = node.actLo; d.act_hi = node.actHi;
                kind  = "gemm";
                flops = 2.0 * M * K * Nn;
                bytes = (M * K + M * Nn + K * Nn) * 2;
                // the skinny-GEMM kernel (weights read once, K split over the waves of a workgroup)
                // or the conv GEMM path; tuned sessions time both and keep the faster
                rows = M; depth = K; cols = Nn;
                act = d.act; lo = d.act_lo; hi = d.act_hi;
                std::vector<uint8_t> host(vkhip_fc_weight_bytes(K, Nn));
                check(vkhip_fc_pack_weights(K, Nn, w.data(), 1, b.data(), 1.f, 1.f, host.data()), "fc pack");
                fcblob = upload(host.data(), host.size());
                if (!env.tunable || env.config->hint(Hint::Tuning, (int) Mode::Fast) == (int) Mode::NoTune) return;
                conv->choosePlan(env, w.data(), b.data());
                std::string key = gpuTag() + "/gemm";
                for (int64_t v: {M, K, Nn, (int64_t) d.act}) key += "_" + std::to_string(v);
                int32_t cached = 0;
                if (TuneCache::instance().get(key, cached)) {
                    useConv = cached != 0;
                } else {
                    auto xb = std::make_shared<DevBuf>(nc4Bytes({M, K, 1, 1}));
                    auto yb = std::make_shared<DevBuf>(nc4Bytes({M, Nn, 1, 1}));
                    check(vkhip_fill_zero(xb->ptr, xb->bytes, nullptr), "gemm tune fill");
                    auto timeIt = [&](bool cv) {
                        vkhip_event_t e0, e1;
                        check(vkhip_event_create(&e0), "event");
                        check(vkhip_event_create(&e1), "event");
                        double best = 1e30;
                        for (int r = 0; r < 4; ++r) {
                            vkhip_event_record(e0, nullptr);
                            for (int k = 0; k < 5; ++k) launch(cv, xb->ptr, yb->ptr, nullptr);
                            vkhip_event_record(e1, nullptr);
                            vkhip_event_sync(e1);
                            float ms = 0;
                            vkhip_event_elapsed_ms(e0, e1, &ms);
                            if (r > 0) best = std::min(best, (double) ms);
                        }
                        vkhip_event_destroy(e0);
                        vkhip_event_destroy(e1);
                        return best;
                    };
                    useConv = timeIt(true) < timeIt(false);
                    TuneCache::instance().put(key, useConv ? 1 : 0);
                }
                if (!useConv) conv.reset();
            }
            void launch(bool cv, const void *x, void *y, vkhip_stream_t s) {
                if (cv) {
                    check(vkhip_conv_forward(&conv->d, &conv->plan, x, conv->blob->ptr, nullptr, y, conv->ws ? conv->ws->ptr : nullptr, s), "gemm " + name);
                    return;
                }
                check(vkhip_fc(x, fcblob->ptr, y, rows, depth, cols, act, lo, hi, s), "fc " + name);
            }
            void record(SegEnv &env, vkhip_stream_t s) override { launch(useConv, env.dev(conv ? conv->in : in), env.dev(conv ? conv->out : out), s); }
            std::string describe() const override { return useConv ? conv->describe() : "fc kernel"; }

            std::shared_ptr<DevBuf> fcblob;
            bool                    useConv = false;
            int64_t                 rows = 0, depth = 0, cols = 0;
            int                     act  = 0;
            float                   lo = 0, hi = 0;
            TensorId                in = kNoTensor, out = kNoTensor;
        };

        // ------------------------------------------------------------ element-wise & data movement
        struct AddOp: HipOp {
            TensorId a, b, out;
            int64_t  n;
            int      act;
            float    lo, hi;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                a = node.inputs[0]; b = node.inputs[1]; out = node.outputs[0];
                if (g.desc(a).shape != g.desc(b).shape) throw Error(Status::Unsupported, "Add: only same-shape operands");
                n = (int64_t) nc4Bytes(g.desc(out).shape) / 2;
                act = (int) node.fusedAct; lo = node.actLo; hi = node.actHi;
                kind = "add";
                bytes = n * 6;
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                const int64_t pa = env.pstride(a), pb = env.pstride(b), py = env.pstride(out);
                if (pa || pb || py) {
                    const NCHW x = NCHW::from(env.graph->desc(out).shape);
                    check(vkhip_add_view(env.dev(a), pa, env.dev(b), pb, env.dev(out), py, x.n, x.c, x.h * x.w, act, lo, hi, s), "add " + name);
                    return;
                }
                check(vkhip_add(env.dev(a), env.dev(b), env.dev(out), n, act, lo, hi, s), "add " + name);
            }
        };

        struct BinaryOp: HipOp {
            TensorId a, b, out;
            int64_t  n = 0, N = 0, C = 0, HW = 0;
            int      op;
            bool     bcast = false;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                a = node.inputs[0]; b = node.inputs[1]; out = node.outputs[0];
                op = node.subOp;
                Shape sa = g.desc(a).shape, sb = g.desc(b).shape;
                if (sa == sb) {
                    n = (int64_t) nc4Bytes(sa) / 2;
                } else if ((BinaryType) op == BinaryType::Mul && sa.size() == 4 && sb.size() == 4 && sa[0] == sb[0] && sa[1] == sb[1] &&
                           (sb[2] * sb[3] == 1 || sa[2] * sa[3] == 1)) {
                    if (sa[2] * sa[3] == 1) std::swap(a, b), std::swap(sa, sb);
                    bcast = true;
                    N = sa[0]; C = sa[1]; HW = sa[2] * sa[3];
                } else {
                    throw Error(Status::Unsupported, "Binary: only same-shape or Mul with [N,C,1,1] broadcast");
                }
                kind = bcast ? "scale" : "binary";
                bytes = (int64_t) nc4Bytes(g.desc(out).shape) * (bcast ? 2 : 3);
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                if (bcast) check(vkhip_channel_scale(env.dev(a), env.dev(b), env.dev(out), N, C, HW, s), "scale " + name);
                else check(vkhip_binary(env.dev(a), env.dev(b), env.dev(out), n, op, s), "binary " + name);
            }
        };

        struct UnaryOp: HipOp {
            TensorId in, out;
            int64_t  n;
            int      op;
            float    p0, p1;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                in = node.inputs[0]; out = node.outputs[0];
                n  = (int64_t) nc4Bytes(g.desc(out).shape) / 2;
                if (node.type == OpType::Relu) {
                    op = (int) UnaryType::Relu; p0 = p1 = 0;
                } else if (node.type == OpType::Clip) {
                    op = -1; p0 = -INFINITY; p1 = INFINITY;
                    if (node.inputs.size() > 1 && node.inputs[1] != kNoTensor) p0 = initF32(g, node.inputs[1])[0];
                    if (node.inputs.size() > 2 && node.inputs[2] != kNoTensor) p1 = initF32(g, node.inputs[2])[0];
                    if (node.attr.has("min")) p0 = node.attr.getf("min", p0);
                    if (node.attr.has("max")) p1 = node.attr.getf("max", p1);
                } else {
                    op = node.subOp; p0 = node.actLo; p1 = node.actHi;
                }
                kind = "unary";
                bytes = n * 4;
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                check(vkhip_unary(env.dev(in), env.dev(out), n, op, p0, p1, s), "unary " + name);
            }
        };

        struct GapOp: HipOp {
            TensorId in, out;
            NCHW     x;
            void prepare(const Node &node, SegEnv &env) override {
                in = node.inputs[0]; out = node.outputs[0];
                x = NCHW::from(env.graph->desc(in).shape);
                kind = "gap";
                bytes = (int64_t) nc4Bytes(env.graph->desc(in).shape);
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                check(vkhip_global_avg_pool(env.dev(in), env.dev(out), x.n, x.c, x.h, x.w, s), "gap " + name);
            }
        };

        struct MaxPoolOp: HipOp {
            TensorId        in, out;
            vkhip_pool_desc d {};
            void prepare(const Node &node, SegEnv &env) override {
                in = node.inputs[0]; out = node.outputs[0];
                NCHW x = NCHW::from(env.graph->desc(in).shape), y = NCHW::from(env.graph->desc(out).shape);
                auto k = attrInts(node, "kernel_shape", {1, 1}), st = attrInts(node, "strides", {1, 1}), p = attrInts(node, "pads", {0, 0, 0, 0});
                auto dl = attrInts(node, "dilations", {1, 1});
                if (node.attr.geti("ceil_mode", 0) || dl[0] != 1 || dl[1] != 1)
                    throw Error(Status::Unsupported, "MaxPool: ceil_mode/dilation");
                d.N = (int) x.n; d.C = (int) x.c; d.H = (int) x.h; d.W = (int) x.w; d.OH = (int) y.h; d.OW = (int) y.w;
                d.KH = (int) k[0]; d.KW = (int) k[1]; d.SH = (int) st[0]; d.SW = (int) st[1]; d.PT = (int) p[0]; d.PL = (int) p[1];
                kind = "maxpool";
                bytes = (int64_t) (nc4Bytes(env.graph->desc(in).shape) + nc4Bytes(env.graph->desc(out).shape) * (1 + chain.size()));
            }
            // Set by the segment before prepare: the same-size pools that follow this one in a
            // chain (each the only pool reading the previous output, the SPPF block); their outputs
            // come from this op's single launch (vkhip_maxpool_chain).
            std::vector<TensorId> chain;
            void record(SegEnv &env, vkhip_stream_t s) override {
                if (chain.empty()) {
                    check(vkhip_maxpool_view(&d, env.dev(in), env.pstride(in), env.dev(out), env.pstride(out), s), "maxpool " + name);
                    return;
                }
                void   *ys[4] = {env.dev(out)};
                int64_t ps[4] = {env.pstride(out)};
                for (size_t k = 0; k < chain.size(); ++k) ys[k + 1] = env.dev(chain[k]), ps[k + 1] = env.pstride(chain[k]);
                check(vkhip_maxpool_chain(&d, env.dev(in), env.pstride(in), ys, ps, (int32_t) (1 + chain.size()), s), "maxpool chain " + name);
            }
            std::string describe() const override { return chain.empty() ? "" : "+" + std::to_string(chain.size()) + " chained pools in one launch"; }
        };

        struct ConcatOp: HipOp {
            std::vector<TensorId> ins;
            std::vector<int64_t>  cs;
            TensorId              out;
            int64_t               N, HW;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                ins = node.inputs; out = node.outputs[0];
                const Shape &os = g.desc(out).shape;
                int64_t axis = node.attr.geti("axis", 0);
                if (axis < 0) axis += (int64_t) os.size();
                if (os.size() != 4 || axis != 1) throw Error(Status::Unsupported, "Concat: only 4-D channel concat");
                for (TensorId t: ins) cs.push_back(g.desc(t).shape[1]);
                N = os[0]; HW = os[2] * os[3];
                kind = "concat";
                bytes = (int64_t) nc4Bytes(os) * 2;
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                std::vector<const void *> xs;
                for (TensorId t: ins) xs.push_back(env.dev(t));
                check(vkhip_concat_channels(xs.data(), cs.data(), (int) xs.size(), env.dev(out), N, HW, s), "concat " + name);
            }
        };

        struct SplitOp: HipOp {
            TensorId              in;
            std::vector<TensorId> outs;
            std::vector<int64_t>  c0s, cs;
            int64_t               N, Cx, HW;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                in = node.inputs[0]; outs = node.outputs;
                const Shape &is = g.desc(in).shape;
                int64_t axis = node.attr.geti("axis", 0);
                if (axis < 0) axis += (int64_t) is.size();
                if (is.size() != 4 || axis != 1) throw Error(Status::Unsupported, "Split: only 4-D channel split");
                N = is[0]; Cx = is[1]; HW = is[2] * is[3];
                int64_t c0 = 0;
                for (TensorId t: outs) {
                    int64_t c = t == kNoTensor ? 0 : g.desc(t).shape[1];
                    c0s.push_back(c0); cs.push_back(c);
                    c0 += c;
                }
                kind = "split";
                bytes = (int64_t) nc4Bytes(is) * 2;
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                for (size_t i = 0; i < outs.size(); ++i)
                    if (outs[i] != kNoTensor) check(vkhip_slice_channels(env.dev(in), env.dev(outs[i]), N, Cx, c0s[i], cs[i], HW, s), "split " + name);
            }
        };

        // The resize kernel reads x[floor(d / s)] for an integer upscale s. The reference's nearest
        // rule (round_prefer_floor of the source coordinate, cpu/ops/resize.cpp:30-87) gives the same
        // index under half_pixel and pytorch_half_pixel coordinates ((d + 0.5) / s - 0.5 stays within
        // 0.5 - 0.5/s of floor(d / s)), under asymmetric ones only up to s = 2 (d / s = k + 2/3 rounds
        // up at s = 3), and under align_corners only for s = 1.
        static bool resizeFloorExact(const Node &nd, int64_t h, int64_t w, int64_t oh, int64_t ow) {
            if (nd.attr.gets("mode", "nearest") != "nearest" || h <= 0 || w <= 0 || oh % h || ow % w) return false;
            const std::string c = nd.attr.gets("coordinate_transformation_mode", "half_pixel");
            const int64_t     s = std::max(oh / h, ow / w);
            if (c == "half_pixel" || c == "pytorch_half_pixel") return true;
            if (c == "asymmetric") return s <= 2;
            return s == 1;
        }

        struct ResizeOp: HipOp {
            TensorId in, out;
            NCHW     x, y;
            void prepare(const Node &node, SegEnv &env) override {
                in = node.inputs[0]; out = node.outputs[0];
                x = NCHW::from(env.graph->desc(in).shape); y = NCHW::from(env.graph->desc(out).shape);
                if (!resizeFloorExact(node, x.h, x.w, y.h, y.w))
                    throw Error(Status::Unsupported, "Resize: only nearest integer upscales whose source index is floor(d / factor)");
                kind = "resize";
                bytes = (int64_t) (nc4Bytes(env.graph->desc(in).shape) + nc4Bytes(env.graph->desc(out).shape));
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                check(vkhip_resize_nearest_view(env.dev(in), env.pstride(in), env.dev(out), env.pstride(out), x.n, x.c, x.h, x.w, y.h, y.w, s),
                      "resize " + name);
            }
        };

        // Metadata-only ops: the output aliases the input buffer (no launch).
        struct AliasOp: HipOp {
            void prepare(const Node &, SegEnv &) override { kind = "alias"; }
            void record(SegEnv &, vkhip_stream_t) override {}
        };

        // A node folded into a conv (a channel-broadcast Mul into the conv that consumes it,
        // ConvOp::xscale; a max pool into the conv it reads, ConvOp::poolOut): no launch.
        struct FoldedMulOp: HipOp {
            std::string into, what = "scale";
            void        prepare(const Node &, SegEnv &) override { kind = "folded"; }
            void        record(SegEnv &, vkhip_stream_t) override {}
            std::string describe() const override { return what + (what.find(':') != std::string::npos ? " " : " folded into ") + into; }
        };

        // ------------------------------------------------------------ two stride-2 stem convs
        // A 3x3 stride-2 conv over at most 4 channels and the 3x3 stride-2 conv that is its only
        // reader (the YOLOv8n stem, 3 -> 16 -> 32) as one op at the second conv's place: one
        // launch of vkhip_conv3x3s2_pair_forward, the intermediate never in HBM. The weights are
        // the thin tiles' blobs; no plan search (one kernel).
        struct Stem2Op: HipOp {
            const Node             *na = nullptr; // the first conv (this op is prepared with the second)
            const Node             *nc = nullptr; // optional 1x1 tail: the second conv's only reader
            vkhip_conv_desc         d1 {}, d2 {}, d3 {};
            vkhip_conv_plan         p1 {}, p2 {}, p3 {};
            std::shared_ptr<DevBuf> blob1, blob2, blob3;
            TensorId                in = kNoTensor, out = kNoTensor;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                d1 = convDescOf(g, *na);
                d2 = convDescOf(g, node);
                if (nc) d3 = convDescOf(g, *nc);
                in = na->inputs[0];
                out = nc ? nc->outputs[0] : node.outputs[0];
                check(vkhip_conv3x3s2_pair_plan(&d1, &d2, nc ? &d3 : nullptr, &p1, &p2, &p3), "stem pair plan " + name);
                std::vector<uint8_t> h1(p1.weight_bytes), h2(p2.weight_bytes), h3(nc ? p3.weight_bytes : 0);
                check(vkhip_conv_pack_weights(&d1, &p1, initF32(g, na->inputs[1]), initF32(g, biasOf(*na)), h1.data()), "stem pair pack");
                check(vkhip_conv_pack_weights(&d2, &p2, initF32(g, node.inputs[1]), initF32(g, biasOf(node)), h2.data()), "stem pair pack");
                if (nc) check(vkhip_conv_pack_weights(&d3, &p3, initF32(g, nc->inputs[1]), initF32(g, biasOf(*nc)), h3.data()), "stem pair pack");
                blob1 = upload(h1.data(), h1.size());
                blob2 = upload(h2.data(), h2.size());
                if (nc) blob3 = upload(h3.data(), h3.size());
                kind  = "conv";
                flops = 2.0 * d1.N * d1.Cout * d1.Cin * 9 * d1.OH * d1.OW + 2.0 * d2.N * d2.Cout * d2.Cin * 9 * d2.OH * d2.OW +
                        (nc ? 2.0 * d3.N * d3.Cout * d3.Cin * d3.OH * d3.OW : 0.0);
                bytes = (int64_t) (nc4Bytes(g.desc(in).shape) + nc4Bytes(g.desc(out).shape)) +
                        (int64_t) (d1.Cout * d1.Cin + d2.Cout * d2.Cin) * 9 * 2 + (nc ? (int64_t) d3.Cout * d3.Cin * 2 : 0);
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                check(vkhip_conv3x3s2_pair_forward(&d1, &d2, nc ? &d3 : nullptr, env.dev(in), blob1->ptr, blob2->ptr, nc ? blob3->ptr : nullptr,
                                                   env.dev(out), env.pstride(out), s),
                      "stem pair " + name);
            }
            std::string describe() const override {
                return "fused with " + na->name + (nc ? " and the 1x1 " + nc->name + " after it" : std::string()) + " kernel=conv_stem2_kernel";
            }
        };

        // ------------------------------------------------------------ stem + first depthwise block
        // A 3x3 stride-2 stem conv over at most 4 channels and the FusedDwPw block that is its only
        // reader (residual: the stem's output), the MobileNetV3 stem and first block, as one op at
        // the block's place: vkhip_stem_dwpw_forward, both 16-channel tensors in LDS.
        struct StemDwPwOp: HipOp {
            const Node             *na = nullptr; // the stem conv (this op is prepared with the block)
            vkhip_conv_desc         ds {}, dd {}, dp {};
            vkhip_conv_plan         ps {}, pd {}, pp {};
            std::shared_ptr<DevBuf> blobs, blobd, blobp;
            TensorId                in = kNoTensor, out = kNoTensor;
            // the block's three descriptors from the stem's and the FusedDwPw node's
            static bool descs(const Graph &g, const Node &stem, const Node &blk, vkhip_conv_desc &s, vkhip_conv_desc &d, vkhip_conv_desc &p) {
                s = convDescOf(g, stem);
                NCHW x = NCHW::from(g.desc(blk.inputs[0]).shape), y = NCHW::from(g.desc(blk.outputs[0]).shape);
                const Shape &dws = g.desc(blk.inputs[1]).shape, &pws = g.desc(blk.inputs[3]).shape;
                if (dws.size() != 4 || pws.size() < 2 || pws[0] != y.c) return false;
                auto st = attrInts(blk, "strides", {1, 1}), pad = attrInts(blk, "pads", {0, 0, 0, 0}), dil = attrInts(blk, "dilations", {1, 1});
                d = vkhip_conv_desc {};
                d.N = (int) x.n; d.Cin = d.Cout = d.group = (int) x.c; d.H = (int) x.h; d.W = (int) x.w; d.OH = (int) y.h; d.OW = (int) y.w;
                d.KH = (int) dws[2]; d.KW = (int) dws[3]; d.SH = (int) st[0]; d.SW = (int) st[1]; d.PT = (int) pad[0]; d.PL = (int) pad[1];
                d.DH = (int) dil[0]; d.DW = (int) dil[1]; d.act = blk.subOp; d.act_lo = 0; d.act_hi = 6;
                if (pad.size() != 4 || pad[2] != pad[0] || pad[3] != pad[1]) return false;
                p = vkhip_conv_desc {};
                p.N = (int) y.n; p.Cin = (int) x.c; p.H = p.OH = (int) y.h; p.W = p.OW = (int) y.w; p.Cout = (int) y.c;
                p.KH = p.KW = p.SH = p.SW = p.DH = p.DW = p.group = 1;
                p.act = (int) blk.fusedAct; p.act_lo = blk.actLo; p.act_hi = blk.actHi; p.has_res = blk.fusedResidual != kNoTensor;
                return true;
            }
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                if (!descs(g, *na, node, ds, dd, dp)) throw Error(Status::Unsupported, "stem + block shapes: " + name);
                in  = na->inputs[0];
                out = node.outputs[0];
                check(vkhip_stem_dwpw_plan(&ds, &dd, &dp, &ps, &pd, &pp), "stem block plan " + name);
                vkhip_conv_desc ep = dp;
                ep.has_res = 0;
                std::vector<uint8_t> hs(ps.weight_bytes), hd(pd.weight_bytes), hp(pp.weight_bytes);
                check(vkhip_conv_pack_weights(&ds, &ps, initF32(g, na->inputs[1]), initF32(g, biasOf(*na)), hs.data()), "stem block pack");
                check(vkhip_conv_pack_weights(&dd, &pd, initF32(g, node.inputs[1]), initF32(g, node.inputs[2]), hd.data()), "stem block pack");
                check(vkhip_conv_pack_weights(&ep, &pp, initF32(g, node.inputs[3]), initF32(g, node.inputs[4]), hp.data()), "stem block pack");
                blobs = upload(hs.data(), hs.size());
                blobd = upload(hd.data(), hd.size());
                blobp = upload(hp.data(), hp.size());
                kind  = "conv";
                flops = 2.0 * ds.N * ds.OH * ds.OW * ((double) ds.Cout * ds.Cin * 9 + (double) dd.Cin * 9 + (double) dp.Cout * dp.Cin);
                bytes = (int64_t) (nc4Bytes(g.desc(in).shape) + nc4Bytes(g.desc(out).shape));
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                check(vkhip_stem_dwpw_forward(&ds, &dd, &dp, env.dev(in), blobs->ptr, blobd->ptr, blobp->ptr, env.dev(out), env.pstride(out), s),
                      "stem block " + name);
            }
            std::string describe() const override { return "fused with " + na->name + " kernel=conv_stem_dwpw_kernel"; }
        };

        // ------------------------------------------------------------ two 3x3 stride-1 convs
        // A 3x3 conv over 9-16 channels and the 3x3 conv that is its only reader, with the Add of
        // the first conv's input after the second's activation when there is one (the YOLOv8
        // bottleneck), as one op at the second conv's place: vkhip_conv3x3_pair_forward, the
        // intermediate in LDS, the shortcut taken from the input band.
        struct PairOp: HipOp {
            const Node             *na = nullptr; // the first conv (this op is prepared with the second)
            TensorId                addOut = kNoTensor; // the folded Add's output, when there is one
            vkhip_conv_desc         d1 {}, d2 {};
            vkhip_conv_plan         p1 {}, p2 {};
            std::shared_ptr<DevBuf> blob1, blob2;
            TensorId                in = kNoTensor, out = kNoTensor;
            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                d1 = convDescOf(g, *na);
                d2 = convDescOf(g, node);
                if (addOut != kNoTensor) d2.has_res = 2;
                in  = na->inputs[0];
                out = addOut != kNoTensor ? addOut : node.outputs[0];
                check(vkhip_conv3x3_pair_plan(&d1, &d2, &p1, &p2), "conv pair plan " + name);
                vkhip_conv_desc e2 = d2;
                e2.has_res = 0;
                std::vector<uint8_t> h1(p1.weight_bytes), h2(p2.weight_bytes);
                check(vkhip_conv_pack_weights(&d1, &p1, initF32(g, na->inputs[1]), initF32(g, biasOf(*na)), h1.data()), "conv pair pack");
                check(vkhip_conv_pack_weights(&e2, &p2, initF32(g, node.inputs[1]), initF32(g, biasOf(node)), h2.data()), "conv pair pack");
                blob1 = upload(h1.data(), h1.size());
                blob2 = upload(h2.data(), h2.size());
                kind  = "conv";
                flops = 2.0 * 9 * d1.N * d1.OH * d1.OW * ((double) d1.Cout * d1.Cin + (double) d2.Cout * d2.Cin);
                bytes = (int64_t) (nc4Bytes(g.desc(in).shape) + nc4Bytes(g.desc(out).shape)) + (int64_t) (d1.Cout * d1.Cin + d2.Cout * d2.Cin) * 9 * 2;
            }
            void record(SegEnv &env, vkhip_stream_t s) override {
                check(vkhip_conv3x3_pair_forward(&d1, &d2, env.dev(in), env.pstride(in), blob1->ptr, blob2->ptr, env.dev(out), env.pstride(out), s),
                      "conv pair " + name);
            }
            std::string describe() const override {
                return "fused with " + na->name + (addOut != kNoTensor ? " (+ its input after the activation)" : "") + " kernel=conv_pair_kernel";
            }
        };

        // ------------------------------------------------------------ fused 3x3 + 1x1
        // A 3x3 conv whose only reader is a 1x1 conv (a bottleneck's middle conv and its expansion)
        // as one op at the 1x1's place in the order (its residual, e.g. a projection shortcut, may be
        // computed between the two). Either the fused kernel (vkhip_convpw_forward: the 3x3 output
        // stays in registers) or the two convs on their own tuned plans with the intermediate in
        // HBM; prepare() plans both convs like standalone ones, times the fused kernel against them
        // on rotating buffer sets larger than the last-level cache, and keeps the faster (the
        // choice is kept in the tune table).
        struct ConvPwOp: HipOp {
            const Node             *n3 = nullptr; // the 3x3 node (this op is prepared with the 1x1 node)
            const Node             *n4 = nullptr; // optional: a 1x1 reading the pair's output (the chain)
            ConvOp                  c3, c1, c4;
            vkhip_convpw_desc       pd {};
            vkhip_convpw2_desc      pd2 {};
            vkhip_conv_plan         plan {}, plan2 {};
            std::shared_ptr<DevBuf> blob, blob2;
            // 0: fused pair (then c4 on its own), 1: split (c3, c1, c4), 2: the chained kernel
            int                     mode = 1;

            void prepare(const Node &node, SegEnv &env) override {
                const Graph &g = *env.graph;
                c3.name = n3->name;
                c1.name = node.name;
                c3.prepare(*n3, env);
                c1.prepare(node, env);
                if (n4) {
                    c4.name = n4->name;
                    c4.prepare(*n4, env);
                }
                kind  = "convpw";
                flops = c3.flops + c1.flops + (n4 ? c4.flops : 0);
                bytes = c3.bytes + c1.bytes + (n4 ? c4.bytes : 0);
                pd.conv = c3.d;
                pd.Cout = c1.d.Cout; pd.act = c1.d.act; pd.act_lo = c1.d.act_lo; pd.act_hi = c1.d.act_hi; pd.has_res = c1.d.has_res;
                if (!env.tunable || vkhip_convpw_plan(&pd, &plan) != VKHIP_OK) return;
                std::vector<float> w1(initF32(g, node.inputs[1]), initF32(g, node.inputs[1]) + (size_t) pd.Cout * pd.conv.Cout);
                std::vector<uint8_t> host(plan.weight_bytes), host2;
                check(vkhip_convpw_pack_weights(&pd, &plan, initF32(g, n3->inputs[1]), initF32(g, biasOf(*n3)), w1.data(), initF32(g, biasOf(node)),
                                                host.data()),
                      "convpw pack");
                bool chain = false;
                if (n4) {
                    pd2.pw = pd;
                    pd2.Cout3 = c4.d.Cout; pd2.act3 = c4.d.act; pd2.act3_lo = c4.d.act_lo; pd2.act3_hi = c4.d.act_hi;
                    if (vkhip_convpw2_plan(&pd2, &plan2) == VKHIP_OK) {
                        host2.resize(plan2.weight_bytes);
                        check(vkhip_convpw2_pack_weights(&pd2, &plan2, initF32(g, n3->inputs[1]), initF32(g, biasOf(*n3)), w1.data(),
                                                         initF32(g, biasOf(node)), initF32(g, n4->inputs[1]), initF32(g, biasOf(*n4)), host2.data()),
                              "convpw2 pack");
                        chain = true;
                    }
                }
                std::string key = gpuTag() + (n4 ? "/convpw2" : "/convpw");
                for (int v: {pd.conv.N, pd.conv.Cin, pd.conv.H, pd.conv.W, pd.conv.Cout, pd.conv.SH, pd.Cout, pd.has_res, c3.plan.tile, c1.plan.tile,
                             n4 ? c4.d.Cout : 0, n4 ? c4.plan.tile : 0})
                    key += "_" + std::to_string(v);
                int32_t cached = 0;
                if (!TuneCache::instance().get(key, cached) || (cached == 2 && !chain)) {
                    blob = upload(host.data(), host.size());
                    if (chain) blob2 = upload(host2.data(), host2.size());
                    const double ts = timeRuns(1), tf = timeRuns(0), tc = chain ? timeRuns(2) : 1e30;
                    cached = ts <= std::min(tf, tc) ? 1 : (tc < tf ? 2 : 0);
                    TuneCache::instance().put(key, cached);
                }
                mode = cached;
                if (mode != 0) blob.reset();
                if (mode != 2) blob2.reset();
                if (mode == 1) return;
                if (mode == 0 && !blob) blob = upload(host.data(), host.size());
                if (mode == 2 && !blob2) blob2 = upload(host2.data(), host2.size());
                const vkhip_conv_desc &c = pd.conv;
                bytes = (int64_t) (nc4Bytes({c.N, c.Cin, c.H, c.W}) + nc4Bytes({c.N, pd.Cout, c.OH, c.OW}) * (pd.has_res ? 2 : 1)) +
                        (int64_t) c.Cout * (c.Cin * 9 + pd.Cout) * 2;
                if (n4) bytes += mode == 2 ? (int64_t) nc4Bytes({c.N, c4.d.Cout, c.OH, c.OW}) + (int64_t) c4.d.Cout * pd.Cout * 2 : c4.bytes;
            }

            // Rotating buffer sets (input, intermediate, residual, output, chained output) whose total
            // exceeds the 256 MB last-level cache, so every alternative is timed from HBM as in a
            // forward pass.
            struct Set {
                std::shared_ptr<DevBuf> x, m, r, y, y2;
            };
            std::vector<Set> sets_;
            void makeSets() {
                if (!sets_.empty()) return;
                const vkhip_conv_desc &c = pd.conv;
                const size_t xb = nc4Bytes({c.N, c.Cin, c.H, c.W}), mb = nc4Bytes({c.N, c.Cout, c.OH, c.OW}), yb = nc4Bytes({c.N, pd.Cout, c.OH, c.OW});
                const size_t y2b = n4 ? nc4Bytes({c.N, c4.d.Cout, c.OH, c.OW}) : 0;
                const size_t one = xb + mb + yb * (pd.has_res ? 2 : 1) + y2b;
                const int    n   = (int) std::min<size_t>(6, std::max<size_t>(1, ((size_t) 640 << 20) / std::max<size_t>(one, 1) + 1));
                for (int k = 0; k < n; ++k) {
                    Set t;
                    t.x = std::make_shared<DevBuf>(xb);
                    t.m = std::make_shared<DevBuf>(mb);
                    t.y = std::make_shared<DevBuf>(yb);
                    if (n4) t.y2 = std::make_shared<DevBuf>(y2b);
                    check(vkhip_fill_zero(t.x->ptr, xb, nullptr), "convpw tune fill");
                    if (pd.has_res) {
                        t.r = std::make_shared<DevBuf>(yb);
                        check(vkhip_fill_zero(t.r->ptr, yb, nullptr), "convpw tune fill");
                    }
                    sets_.push_back(t);
                }
            }
            void launch(int m, const void *x, const void *mid, const void *r, void *y, void *y2, vkhip_stream_t s) {
                if (m == 2) {
                    check(vkhip_convpw2_forward(&pd2, &plan2, x, blob2->ptr, r, y, y2, s), "convpw2 " + name);
                    return;
                }
                if (m == 0) check(vkhip_convpw_forward(&pd, &plan, x, blob->ptr, r, y, s), "convpw " + name);
                else {
                    check(c3.forward(c3.plan, x, nullptr, c3.blob->ptr, nullptr, (void *) mid, c3.ws ? c3.ws->ptr : nullptr, s), "convpw 3x3 " + name);
                    check(c1.forward(c1.plan, mid, nullptr, c1.blob->ptr, r, y, c1.ws ? c1.ws->ptr : nullptr, s), "convpw 1x1 " + name);
                }
                if (n4) check(c4.forward(c4.plan, y, nullptr, c4.blob->ptr, nullptr, y2, c4.ws ? c4.ws->ptr : nullptr, s), "convpw chained 1x1 " + name);
            }
            double timeRuns(int m) {
                makeSets();
                vkhip_event_t e0, e1;
                check(vkhip_event_create(&e0), "event");
                check(vkhip_event_create(&e1), "event");
                double best = 1e30;
                size_t k    = 0;
                for (int r = 0; r < 5; ++r) {
                    vkhip_event_record(e0, nullptr);
                    for (int i = 0; i < 6; ++i) {
                        const Set &t = sets_[k++ % sets_.size()];
                        launch(m, t.x->ptr, t.m->ptr, t.r ? t.r->ptr : nullptr, t.y->ptr, t.y2 ? t.y2->ptr : nullptr, nullptr);
                    }
                    vkhip_event_record(e1, nullptr);
                    vkhip_event_sync(e1);
                    float ms = 0;
                    vkhip_event_elapsed_ms(e0, e1, &ms);
                    if (r > 0) best = std::min(best, (double) ms); // the first round warms up
                }
                vkhip_event_destroy(e0);
                vkhip_event_destroy(e1);
                return best;
            }

            void record(SegEnv &env, vkhip_stream_t s) override {
                launch(mode, env.dev(c3.in), env.dev(c3.out), c1.res != kNoTensor ? env.dev(c1.res) : nullptr, env.dev(c1.out),
                       n4 ? env.dev(c4.out) : nullptr, s);
            }
            std::string describe() const override {
                const std::string chained = n4 ? " then 1x1 " + c4.name + " (" + c4.describe() + ")" : "";
                if (mode == 1) return "split: " + c3.name + " (" + c3.describe() + ") then 1x1 " + c1.describe() + chained;
                if (mode == 2) return "fused 3x3 + 1x1 + 1x1 (" + c3.name + " in registers, " + c4.name + " chained) kernel=conv_halo_pw_kernel";
                return "fused 3x3 + 1x1 (" + c3.name + " in registers) kernel=conv_halo_pw_kernel" + chained;
            }
        };

        // 3x3 + 1x1 pairs (ConvPwOp): a 3x3 conv of the segment whose output only a 1x1 stride-1
        // conv of the segment reads, with shapes the fused kernel may take (vkhip_convpw_plan; the
        // timing in ConvPwOp decides). Returns 1x1 node -> 3x3 node. `skip`: nodes already fused or
        // folded into another op.
        static void planPwPairs(const Graph &g, const std::vector<int> &idx, const std::set<int> &skip, std::map<int, int> &pw) {
            std::set<int>           inSeg(idx.begin(), idx.end());
            std::map<TensorId, int> readers, producer;
            for (size_t i = 0; i < g.nodes.size(); ++i) {
                const Node &nd = g.nodes[i];
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor) ++readers[t];
                if (nd.fusedResidual != kNoTensor) ++readers[nd.fusedResidual];
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor) producer[t] = (int) i;
            }
            for (TensorId t: g.outputs) readers[t] += 1000;
            auto convDesc = [&](const Node &c, vkhip_conv_desc &d) {
                if (c.type != OpType::Conv || c.inputs.size() < 2 || !g.isInitializer(c.inputs[1]) || c.outputs.empty()) return false;
                const Shape &ws = g.desc(c.inputs[1]).shape;
                if (ws.size() != 4 || g.desc(c.inputs[0]).shape.size() != 4) return false;
                NCHW x = NCHW::from(g.desc(c.inputs[0]).shape), y = NCHW::from(g.desc(c.outputs[0]).shape);
                auto st = attrInts(c, "strides", {1, 1}), pad = attrInts(c, "pads", {0, 0, 0, 0}), dl = attrInts(c, "dilations", {1, 1});
                if (pad[2] != pad[0] || pad[3] != pad[1]) return false;
                d = vkhip_conv_desc {};
                d.N = (int) x.n; d.Cin = (int) x.c; d.H = (int) x.h; d.W = (int) x.w; d.Cout = (int) ws[0]; d.OH = (int) y.h; d.OW = (int) y.w;
                d.KH = (int) ws[2]; d.KW = (int) ws[3]; d.SH = (int) st[0]; d.SW = (int) st[1]; d.PT = (int) pad[0]; d.PL = (int) pad[1];
                d.DH = (int) dl[0]; d.DW = (int) dl[1]; d.group = (int) c.attr.geti("group", 1); d.act = (int) c.fusedAct;
                d.act_lo = c.actLo; d.act_hi = c.actHi; d.has_res = c.fusedResidual != kNoTensor;
                return true;
            };
            for (int b: idx) {
                const Node     &n1 = g.nodes[b];
                vkhip_conv_desc d1, d3;
                if (skip.count(b) || !convDesc(n1, d1) || d1.KH != 1 || d1.KW != 1 || d1.SH != 1 || d1.SW != 1 || d1.PT != 0 || d1.PL != 0 || d1.group != 1)
                    continue;
                const TensorId t  = n1.inputs[0];
                auto           pit = producer.find(t);
                if (pit == producer.end() || !inSeg.count(pit->second) || skip.count(pit->second) || readers[t] != 1) continue;
                const Node &n3 = g.nodes[pit->second];
                if (!convDesc(n3, d3) || d3.KH != 3 || d3.has_res || d3.Cout != d1.Cin || n1.fusedResidual == t) continue;
                vkhip_convpw_desc pd {};
                pd.conv = d3;
                pd.Cout = d1.Cout; pd.act = d1.act; pd.act_lo = d1.act_lo; pd.act_hi = d1.act_hi; pd.has_res = d1.has_res;
                vkhip_conv_plan plan;
                if (vkhip_convpw_plan(&pd, &plan) != VKHIP_OK) continue;
                pw[b] = pit->second;
            }
        }

        // Stem + pool fusion: a MaxPool 3x3 stride 2 pad 1 whose input is the output of a conv of the
        // same segment that nothing else reads, and that conv a first layer the fused kernel takes
        // (vkhip_conv_maxpool_supported on its stem plan). Returns conv node -> pool node.
        static void planPoolFolds(const Graph &g, const std::vector<int> &idx, std::map<int, int> &convPool) {
            std::set<int>           inSeg(idx.begin(), idx.end());
            std::map<TensorId, int> readers, producer;
            for (size_t i = 0; i < g.nodes.size(); ++i) {
                const Node &nd = g.nodes[i];
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor) ++readers[t];
                if (nd.fusedResidual != kNoTensor) ++readers[nd.fusedResidual];
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor) producer[t] = (int) i;
            }
            for (TensorId t: g.outputs) readers[t] += 1000;
            for (int i: idx) {
                const Node &p = g.nodes[i];
                if (p.type != OpType::MaxPool || p.inputs.empty()) continue;
                auto k = attrInts(p, "kernel_shape", {1, 1}), st = attrInts(p, "strides", {1, 1}), pad = attrInts(p, "pads", {0, 0, 0, 0});
                auto dl = attrInts(p, "dilations", {1, 1});
                if (k[0] != 3 || k[1] != 3 || st[0] != 2 || st[1] != 2 || pad[0] != 1 || pad[1] != 1 || pad[2] != 1 || pad[3] != 1 ||
                    p.attr.geti("ceil_mode", 0) || dl[0] != 1 || dl[1] != 1)
                    continue;
                const TensorId t = p.inputs[0];
                auto           pit = producer.find(t);
                if (pit == producer.end() || !inSeg.count(pit->second) || readers[t] != 1) continue;
                const Node &c = g.nodes[pit->second];
                if (c.type != OpType::Conv || c.fusedResidual != kNoTensor || c.inputs.size() < 2 || !g.isInitializer(c.inputs[1])) continue;
                const Shape &ws = g.desc(c.inputs[1]).shape;
                NCHW         x = NCHW::from(g.desc(c.inputs[0]).shape), y = NCHW::from(g.desc(t).shape), z = NCHW::from(g.desc(p.outputs[0]).shape);
                auto cst = attrInts(c, "strides", {1, 1}), cpad = attrInts(c, "pads", {0, 0, 0, 0}), cdl = attrInts(c, "dilations", {1, 1});
                if (ws.size() != 4) continue;
                vkhip_conv_desc d {};
                d.N = (int) x.n; d.Cin = (int) x.c; d.H = (int) x.h; d.W = (int) x.w; d.Cout = (int) ws[0]; d.OH = (int) y.h; d.OW = (int) y.w;
                d.KH = (int) ws[2]; d.KW = (int) ws[3]; d.SH = (int) cst[0]; d.SW = (int) cst[1]; d.PT = (int) cpad[0]; d.PL = (int) cpad[1];
                d.DH = (int) cdl[0]; d.DW = (int) cdl[1]; d.group = (int) c.attr.geti("group", 1); d.act = (int) c.fusedAct;
                if (cpad[2] != cpad[0] || cpad[3] != cpad[1]) continue;
                vkhip_pool_desc pd {};
                pd.N = (int) y.n; pd.C = (int) y.c; pd.H = (int) y.h; pd.W = (int) y.w; pd.OH = (int) z.h; pd.OW = (int) z.w;
                pd.KH = pd.KW = 3; pd.SH = pd.SW = 2; pd.PT = pd.PL = 1;
                vkhip_conv_plan plan;
                bool            ok = false;
                for (int tile: poolTiles())
                    if (!ok && vkhip_conv_plan_make(&d, VKHIP_CONV_GEMM, tile, 0, &plan) == VKHIP_OK && vkhip_conv_maxpool_supported(&d, &plan, &pd)) ok = true;
                if (ok) convPool[pit->second] = i;
            }
        }

        // Squeeze-excite scale folding: y = Mul(h, s) with s of shape [N,C,1,1] (the SE branch output)
        // whose only reader is a dense 1x1 stride-1 pad-0 conv of the same segment becomes that conv's
        // input scale, so h*s is never written (the reference runs the Mul as its own Binary op,
        // ops/binary.cpp:32-43; the product is rounded to fp16 exactly as that op's store does).
        // Returns conv node -> (h, s) and the set of folded Mul nodes.
        // Activation folds: a HardSigmoid unary whose input is the output of a 1x1 stride-1 dense conv
        // of this segment with no activation of its own, read by nothing else, runs in that conv's
        // epilogue (the squeeze-excite gate after its second FC when the SE is not fused): the conv
        // writes the unary's output with VKHIP_ACT_HARDSIGMOID (lo = alpha, hi = beta, computed on
        // the fp32 sum, where the separate unary reads the conv's fp16 output).
        static void planActFolds(const Graph &g, const std::vector<int> &idx, const std::set<int> &skip, std::map<int, int> &convOf) {
            std::set<int>           inSeg(idx.begin(), idx.end());
            std::map<TensorId, int> readers, producer;
            for (size_t i = 0; i < g.nodes.size(); ++i) {
                const Node &nd = g.nodes[i];
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor) ++readers[t];
                if (nd.fusedResidual != kNoTensor) ++readers[nd.fusedResidual];
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor) producer[t] = (int) i;
            }
            for (TensorId t: g.outputs) readers[t] += 1000; // a graph output is never folded away
            for (int u: idx) {
                const Node &un = g.nodes[u];
                if (un.type != OpType::Unary || (UnaryType) un.subOp != UnaryType::HardSigmoid || un.inputs.empty() || un.outputs.empty()) continue;
                const TensorId t = un.inputs[0];
                auto           pit = producer.find(t);
                if (pit == producer.end() || !inSeg.count(pit->second) || skip.count(pit->second) || readers[t] != 1) continue;
                const Node &c = g.nodes[pit->second];
                if (c.type != OpType::Conv || c.fusedAct != ActType::None || c.inputs.size() < 2 || !g.isInitializer(c.inputs[1])) continue;
                const Shape &w = g.desc(c.inputs[1]).shape;
                auto st = attrInts(c, "strides", {1, 1}), pad = attrInts(c, "pads", {0, 0, 0, 0});
                if (w.size() != 4 || w[2] != 1 || w[3] != 1 || c.attr.geti("group", 1) != 1 || st[0] != 1 || st[1] != 1 || pad[0] || pad[1] ||
                    pad[2] || pad[3])
                    continue;
                convOf[u] = pit->second;
            }
        }

        // Adds that fold into the conv producing one operand as a residual after its activation
        // (y = act(conv + bias) + r, the YOLOv8 bottleneck shortcut): an Add without activation of
        // two same-shape tensors, one written by a dense conv of this segment that nothing else
        // reads; the other operand r is produced before that conv in the segment order (or comes
        // from outside the segment), so it exists when the conv runs. Views are checked by the
        // caller. convOf: Add node -> conv node.
        static void planResFolds(const Graph &g, const std::vector<int> &idx, const std::set<int> &skip, std::map<int, std::pair<int, TensorId>> &convOf) {
            std::map<int, int>      pos;
            for (size_t k = 0; k < idx.size(); ++k) pos[idx[k]] = (int) k;
            std::map<TensorId, int> readers, producer;
            for (size_t i = 0; i < g.nodes.size(); ++i) {
                const Node &nd = g.nodes[i];
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor) ++readers[t];
                if (nd.fusedResidual != kNoTensor) ++readers[nd.fusedResidual];
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor) producer[t] = (int) i;
            }
            for (TensorId t: g.outputs) readers[t] += 1000; // a graph output is never folded away
            std::set<int> taken;
            for (int u: idx) {
                const Node &ad = g.nodes[u];
                if (ad.type != OpType::Add || ad.inputs.size() != 2 || ad.outputs.empty() || ad.fusedAct != ActType::None || skip.count(u)) continue;
                if (ad.inputs[0] == ad.inputs[1] || g.desc(ad.inputs[0]).shape != g.desc(ad.inputs[1]).shape || g.desc(ad.inputs[0]).shape.size() != 4) continue;
                for (int e = 0; e < 2; ++e) {
                    const TensorId t = ad.inputs[e], r = ad.inputs[1 - e];
                    auto           pit = producer.find(t);
                    if (pit == producer.end() || !pos.count(pit->second) || skip.count(pit->second) || taken.count(pit->second) || readers[t] != 1) continue;
                    const Node &c = g.nodes[pit->second];
                    if (c.type != OpType::Conv || c.fusedResidual != kNoTensor || c.attr.geti("group", 1) != 1 || c.inputs.size() < 2 ||
                        !g.isInitializer(c.inputs[1]) || g.desc(c.inputs[1]).shape.size() != 4 || r == c.inputs[0])
                        continue;
                    auto rp = producer.find(r);
                    if (rp != producer.end() && pos.count(rp->second) && pos[rp->second] >= pos[pit->second]) continue;
                    convOf[u] = {pit->second, r};
                    taken.insert(pit->second);
                    break;
                }
            }
        }

        static void planScaleFolds(const Graph &g, const std::vector<int> &idx, std::map<int, std::pair<TensorId, TensorId>> &conv,
                                   std::set<int> &muls) {
            std::set<int>           inSeg(idx.begin(), idx.end());
            std::map<TensorId, int> readers;
            for (const Node &nd: g.nodes) {
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor) ++readers[t];
                if (nd.fusedResidual != kNoTensor && std::find(nd.inputs.begin(), nd.inputs.end(), nd.fusedResidual) == nd.inputs.end())
                    ++readers[nd.fusedResidual];
            }
            for (TensorId t: g.outputs) readers[t] += 1000; // a graph output is never folded away
            for (int i: idx) {
                const Node &m = g.nodes[i];
                if (m.type != OpType::Binary || m.subOp != (int) BinaryType::Mul || m.inputs.size() != 2) continue;
                TensorId     h = m.inputs[0], sc = m.inputs[1];
                const Shape &sh = g.desc(h).shape, &ss = g.desc(sc).shape;
                if (g.isInitializer(h) || g.isInitializer(sc) || sh.size() != 4 || ss.size() != 4) continue;
                const Shape *ph = &sh, *ps = &ss;
                if (sh[2] * sh[3] == 1 && ss[2] * ss[3] != 1) std::swap(h, sc), std::swap(ph, ps);
                if ((*ph)[0] != (*ps)[0] || (*ph)[1] != (*ps)[1] || (*ps)[2] * (*ps)[3] != 1 || (*ph)[2] * (*ph)[3] == 1) continue;
                const TensorId t = m.outputs[0];
                if (readers[t] != 1) continue;
                for (int j: idx) {
                    const Node &c = g.nodes[j];
                    if (c.type != OpType::Conv || c.inputs.empty() || c.inputs[0] != t || c.fusedResidual == t) continue;
                    const Shape &w = g.desc(c.inputs[1]).shape;
                    auto st = attrInts(c, "strides", {1, 1}), pad = attrInts(c, "pads", {0, 0, 0, 0});
                    if (c.attr.geti("group", 1) != 1 || w.size() != 4 || w[2] != 1 || w[3] != 1 || st[0] != 1 || st[1] != 1 ||
                        pad[0] != 0 || pad[1] != 0 || pad[2] != 0 || pad[3] != 0 || !inSeg.count(j))
                        break;
                    vkhip_conv_desc d {};
                    NCHW x = NCHW::from(sh);
                    d.N = (int) x.n; d.Cin = (int) x.c; d.H = d.OH = (int) x.h; d.W = d.OW = (int) x.w; d.Cout = (int) w[0];
                    d.KH = d.KW = d.SH = d.SW = d.DH = d.DW = d.group = 1; d.in_scale = 1;
                    vkhip_conv_plan p;
                    if (vkhip_conv_plan_make(&d, VKHIP_CONV_GEMM, -1, 0, &p) != VKHIP_OK) break; // shape the scaled kernel does not take
                    conv[j] = {h, sc};
                    muls.insert(i);
                    break;
                }
            }
        }

        static bool isAliasOp(const Graph &g, const Node &nd) {
            // ConvertLayout (reference ops/convert_layout.cpp) changes only the physical layout of
            // the same logical NCHW tensor; this backend keeps every activation NC4HW4 fp16, so
            // in a HIP segment it is the identity (vkhip_convert_layout serves boundary callers).
            if (nd.type == OpType::Identity || nd.type == OpType::ConvertLayout) return true;
            if (nd.type == OpType::Flatten || nd.type == OpType::Reshape || nd.type == OpType::Squeeze || nd.type == OpType::Unsqueeze) {
                // [N,C,1,1] <-> [N,C]: the NC4HW4 bytes are identical.
                NCHW a = NCHW::from(g.desc(nd.inputs[0]).shape), b = NCHW::from(g.desc(nd.outputs[0]).shape);
                return a.n == b.n && a.c == b.c && a.h * a.w == 1 && b.h * b.w == 1;
            }
            return false;
        }

        std::unique_ptr<HipOp> makeOp(const Graph &g, const Node &nd) {
            if (isAliasOp(g, nd)) return std::make_unique<AliasOp>();
            switch (nd.type) {
                case OpType::Conv: return std::make_unique<ConvOp>();
                case OpType::FusedDwPw: return std::make_unique<DwPwOp>();
                case OpType::FusedSE: return std::make_unique<SeOp>();
                case OpType::Gemm: return std::make_unique<GemmOp>();
                case OpType::Add: return std::make_unique<AddOp>();
                case OpType::Binary: return std::make_unique<BinaryOp>();
                case OpType::Unary: case OpType::Relu: case OpType::Clip: return std::make_unique<UnaryOp>();
                case OpType::GlobalAvgPool: return std::make_unique<GapOp>();
                case OpType::MaxPool: return std::make_unique<MaxPoolOp>();
                case OpType::Concat: return std::make_unique<ConcatOp>();
                case OpType::Split: return std::make_unique<SplitOp>();
                case OpType::Resize: return std::make_unique<ResizeOp>();
                default: return nullptr;
            }
        }

        // ------------------------------------------------------------ segment
        HipSegment::HipSegment(const std::vector<int> &idx, Graph &g, const Config &cfg): g_(g), cfg_(cfg) {
            nodeIdx = idx;
            check(vkhip_stream_create(&stream_), "stream");
            env_.graph   = &g;
            env_.config  = &cfg;
            env_.tunable = true;
            env_.seg     = this;
            const char *mk = std::getenv("VKNN_HIP_OP_MARKERS");
            markers_       = mk && std::strcmp(mk, "1") == 0;
            // Tensors this segment touches, in first-use order.
            std::set<TensorId> produced;
            for (int i: idx) {
                const Node &nd = g.nodes[i];
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor) produced.insert(t);
            }
            for (int i: idx) {
                const Node &nd = g.nodes[i];
                if (isAliasOp(g, nd)) alias_[nd.outputs[0]] = resolve(nd.inputs[0]);
            }
            std::map<int, std::pair<TensorId, TensorId>> scaled;
            std::set<int>                                folded;
            // VKNN_HIP_FOLD_SCALE=0 keeps every Mul as its own launch (A/B measurements)
            const char *fold_env = std::getenv("VKNN_HIP_FOLD_SCALE");
            if (!fold_env || std::string(fold_env) != "0") planScaleFolds(g, idx, scaled, folded);
            std::map<int, std::string> foldedInto;
            for (auto &kv: scaled)
                for (int m: folded)
                    if (g.nodes[m].outputs[0] == g.nodes[kv.first].inputs[0]) foldedInto[m] = g.nodes[kv.first].name;
            // A stem conv and its max pool as one kernel (poolTiles); VKNN_HIP_FUSE_POOL=0 keeps the
            // two launches (A/B).
            std::map<int, int> convPool;
            std::set<int>      pools;
            const char        *pool_env = std::getenv("VKNN_HIP_FUSE_POOL");
            if (!pool_env || std::string(pool_env) != "0") planPoolFolds(g, idx, convPool);
            for (auto &kv: convPool) {
                pools.insert(kv.second);
                foldedInto[kv.second] = g.nodes[kv.first].name;
            }
            // Squeeze-excite pool folding: a GlobalAveragePool whose input is a depthwise conv of this
            // segment and whose output only a FusedSE of this segment reads. The conv (once its
            // plan is known) also leaves the pool sums, and the FusedSE forms its input from them,
            // so the pool neither launches nor re-reads the conv output. VKNN_HIP_FOLD_GAP=0 keeps it.
            std::map<int, int> gapConv; // GAP node -> depthwise conv node
            std::map<int, int> seGap;   // FusedSE node -> GAP node
            {
                const char *gap_env = std::getenv("VKNN_HIP_FOLD_GAP");
                if (!gap_env || std::string(gap_env) != "0") {
                    std::set<int>           inSeg(idx.begin(), idx.end());
                    std::map<TensorId, int> producer;
                    std::map<TensorId, std::vector<int>> readers;
                    for (size_t i = 0; i < g.nodes.size(); ++i) {
                        for (TensorId t: g.nodes[i].inputs)
                            if (t != kNoTensor) readers[t].push_back((int) i);
                        if (g.nodes[i].fusedResidual != kNoTensor) readers[g.nodes[i].fusedResidual].push_back((int) i);
                        for (TensorId t: g.nodes[i].outputs)
                            if (t != kNoTensor) producer[t] = (int) i;
                    }
                    std::set<TensorId> gout(g.outputs.begin(), g.outputs.end());
                    for (int i: idx) {
                        const Node &p = g.nodes[i];
                        if (p.type != OpType::GlobalAvgPool || p.inputs.empty() || gout.count(p.outputs[0])) continue;
                        auto pit = producer.find(p.inputs[0]);
                        if (pit == producer.end() || !inSeg.count(pit->second) || folded.count(pit->second)) continue;
                        const Node &c = g.nodes[pit->second];
                        if (c.type != OpType::Conv || c.attr.geti("group", 1) <= 1 || scaled.count(pit->second) || convPool.count(pit->second)) continue;
                        const auto &rd = readers[p.outputs[0]];
                        if (rd.size() != 1 || !inSeg.count(rd[0]) || g.nodes[rd[0]].type != OpType::FusedSE || g.nodes[rd[0]].inputs[0] != p.outputs[0])
                            continue;
                        gapConv[i]   = pit->second;
                        seGap[rd[0]] = i;
                    }
                }
            }
            std::map<int, ConvOp *> convOps;       // node -> its ConvOp (pool-fold candidates)
            std::map<int, std::shared_ptr<DevBuf>> gapParts; // folded GAP node -> partial sums
            std::map<int, int>      gapR;
            std::map<int, size_t>   opPos; // node -> index of its op
            // In-place concat / split (planViews); VKNN_HIP_VIEWS=0 keeps their copies (A/B).
            {
                std::set<int> noWrite, noRead;
                // a conv + pool kernel reads a dense input and writes the pool's output densely
                for (auto &kv: convPool) noWrite.insert(kv.first), noWrite.insert(kv.second), noRead.insert(kv.first);
                for (auto &kv: scaled) noRead.insert(kv.first);
                for (int m: folded) noRead.insert(m), noWrite.insert(m);
                for (auto &kv: gapConv) noWrite.insert(kv.second);
                const char *views_env = std::getenv("VKNN_HIP_VIEWS");
                if (!views_env || std::string(views_env) != "0") planViews(idx, noWrite, noRead);
            }
            // 3x3 + 1x1 pairs (ConvPwOp) among the convs no other fold or view touches;
            // VKNN_HIP_FUSE_PW=0 keeps every conv on its own (A/B).
            std::map<int, int> pwPairs; // 1x1 node -> 3x3 node
            std::set<int>      pwFolded; // 3x3 nodes of the pairs
            std::map<int, int> pwChain;  // 1x1 node of a pair -> the 1x1 chained after it
            std::set<int>      pwChained;
            {
                const char *pw_env = std::getenv("VKNN_HIP_FUSE_PW");
                if (!pw_env || std::string(pw_env) != "0") {
                    std::set<int> skip(folded.begin(), folded.end());
                    for (auto &kv: scaled) skip.insert(kv.first);
                    for (auto &kv: convPool) skip.insert(kv.first), skip.insert(kv.second);
                    for (auto &kv: gapConv) skip.insert(kv.first), skip.insert(kv.second);
                    std::map<int, int> cand;
                    planPwPairs(g, idx, skip, cand);
                    for (auto &kv: cand) {
                        const Node &n1 = g.nodes[kv.first], &n3 = g.nodes[kv.second];
                        bool view = false;
                        for (TensorId t: {n3.inputs[0], n3.outputs[0], n1.outputs[0], n1.fusedResidual})
                            if (t != kNoTensor && (place_.count(resolve(t)) || pstride(t) > 0)) view = true;
                        if (view) continue;
                        pwPairs[kv.first] = kv.second;
                        pwFolded.insert(kv.second);
                    }
                    // chains: a 1x1 stride-1 conv of at most 64 outputs, no residual, reading a pair's
                    // output (the next bottleneck's reduction) runs inside the pair's op
                    std::set<int> inSeg(idx.begin(), idx.end());
                    for (auto &kv: pwPairs) {
                        const TensorId t = g.nodes[kv.first].outputs[0];
                        for (int r: idx) {
                            const Node &nr = g.nodes[r];
                            if (r == kv.first || skip.count(r) || pwPairs.count(r) || pwFolded.count(r) || pwChained.count(r)) continue;
                            if (nr.type != OpType::Conv || nr.inputs.size() < 2 || nr.inputs[0] != t || nr.fusedResidual != kNoTensor ||
                                !g.isInitializer(nr.inputs[1]) || nr.outputs.empty())
                                continue;
                            const Shape &ws = g.desc(nr.inputs[1]).shape;
                            auto st = attrInts(nr, "strides", {1, 1}), pad = attrInts(nr, "pads", {0, 0, 0, 0});
                            if (ws.size() != 4 || ws[2] != 1 || ws[3] != 1 || ws[0] > 64 || st[0] != 1 || st[1] != 1 || pad[0] || pad[1] || pad[2] ||
                                pad[3] || nr.attr.geti("group", 1) != 1)
                                continue;
                            if (place_.count(resolve(nr.outputs[0])) || pstride(nr.outputs[0]) > 0) continue;
                            pwChain[kv.first] = r;
                            pwChained.insert(r);
                            break;
                        }
                    }
                }
            }
            // Hard-sigmoid folds into the producing conv (planActFolds); VKNN_HIP_FOLD_ACT=0 keeps the
            // unary launches (A/B).
            std::map<int, int> actFold; // HardSigmoid node -> conv node
            std::map<int, int> actConv; // conv node -> HardSigmoid node
            {
                const char *act_env = std::getenv("VKNN_HIP_FOLD_ACT");
                if (!act_env || std::string(act_env) != "0") {
                    std::set<int> skip(folded.begin(), folded.end());
                    for (auto &kv: scaled) skip.insert(kv.first);
                    for (auto &kv: convPool) skip.insert(kv.first), skip.insert(kv.second);
                    for (auto &kv: gapConv) skip.insert(kv.second);
                    for (auto &kv: pwPairs) skip.insert(kv.first);
                    skip.insert(pwFolded.begin(), pwFolded.end());
                    skip.insert(pwChained.begin(), pwChained.end());
                    planActFolds(g, idx, skip, actFold);
                    for (auto it = actFold.begin(); it != actFold.end();) {
                        // a conv that writes or reads a view keeps its own output
                        const Node &c = g.nodes[it->second];
                        if (pstride(c.inputs[0]) > 0 || pstride(g.nodes[it->first].outputs[0]) > 0 || place_.count(resolve(c.outputs[0])))
                            it = actFold.erase(it);
                        else ++it;
                    }
                    for (auto &kv: actFold) actConv[kv.second] = kv.first;
                }
            }
            // Adds after an activated conv fold into its epilogue (planResFolds); VKNN_HIP_FOLD_ADD=0
            // keeps the add launches (A/B).
            std::map<int, std::pair<int, TensorId>> addFold; // Add node -> (conv node, residual)
            std::map<int, int>                      addConv; // conv node -> Add node
            {
                const char *add_env = std::getenv("VKNN_HIP_FOLD_ADD");
                if (!add_env || std::string(add_env) != "0") {
                    std::set<int> skip(folded.begin(), folded.end());
                    for (auto &kv: scaled) skip.insert(kv.first);
                    for (auto &kv: convPool) skip.insert(kv.first), skip.insert(kv.second);
                    for (auto &kv: gapConv) skip.insert(kv.second);
                    for (auto &kv: pwPairs) skip.insert(kv.first);
                    skip.insert(pwFolded.begin(), pwFolded.end());
                    skip.insert(pwChained.begin(), pwChained.end());
                    for (auto &kv: actConv) skip.insert(kv.first);
                    for (int i: idx)
                        if (viewCats_.count(i) || viewSplits_.count(i)) skip.insert(i);
                    planResFolds(g, idx, skip, addFold);
                    // the residual is read at the output's plane stride: both dense, or both slices
                    // of tensors with the same channel blocks per image
                    auto eff = [&](TensorId t) { return pstride(t) > 0 ? pstride(t) : (g.desc(t).shape[1] + 3) / 4; };
                    for (auto it = addFold.begin(); it != addFold.end();) {
                        const TensorId o = g.nodes[it->first].outputs[0], r = it->second.second;
                        if (eff(o) != eff(r) || (pstride(o) > 0) != (pstride(r) > 0)) it = addFold.erase(it);
                        else ++it;
                    }
                    for (auto &kv: addFold) addConv[kv.second.first] = kv.first;
                }
            }
            // Chains of same-size max pools (the SPPF block: each pool the only pool reading the
            // previous one's output) as one launch at the first pool's place. VKNN_HIP_POOL_CHAIN=0
            // keeps one launch per pool (A/B).
            std::map<int, std::vector<int>> poolChain; // first pool -> the pools it also computes
            std::set<int>                   poolChained;
            {
                const char *pc_env = std::getenv("VKNN_HIP_POOL_CHAIN");
                if (!pc_env || std::string(pc_env) != "0") {
                    std::set<int> inSeg(idx.begin(), idx.end());
                    std::map<TensorId, std::vector<int>> readers;
                    for (int i: idx)
                        for (TensorId t: g.nodes[i].inputs)
                            if (t != kNoTensor) readers[t].push_back(i);
                    auto samePool = [&](const Node &m) {
                        if (m.type != OpType::MaxPool || m.inputs.empty() || m.outputs.empty() || pools.count(&m - &g.nodes[0])) return false;
                        auto k = attrInts(m, "kernel_shape", {1, 1}), st = attrInts(m, "strides", {1, 1}), p = attrInts(m, "pads", {0, 0, 0, 0});
                        auto dl = attrInts(m, "dilations", {1, 1});
                        if (m.attr.geti("ceil_mode", 0) || dl[0] != 1 || dl[1] != 1 || k[0] != k[1] || (k[0] != 3 && k[0] != 5) || st[0] != 1 || st[1] != 1 ||
                            p[0] != k[0] / 2 || p[1] != k[0] / 2 || p[2] != k[0] / 2 || p[3] != k[0] / 2)
                            return false;
                        const Shape &xs = g.desc(m.inputs[0]).shape;
                        return xs.size() == 4 && xs == g.desc(m.outputs[0]).shape && (size_t) (xs[2] + k[0] - 1) * (2 * xs[3] + k[0] - 1) * 8 <= 64 * 1024;
                    };
                    for (int i: idx) {
                        if (poolChained.count(i) || !samePool(g.nodes[i])) continue;
                        std::vector<int> ch;
                        int              cur = i;
                        while (ch.size() < 3) {
                            int nxt = -1;
                            for (int r: readers[g.nodes[cur].outputs[0]])
                                if (nxt < 0 && inSeg.count(r) && !poolChained.count(r) && r != i && samePool(g.nodes[r]) &&
                                    attrInts(g.nodes[r], "kernel_shape", {1, 1}) == attrInts(g.nodes[i], "kernel_shape", {1, 1}))
                                    nxt = r;
                            if (nxt < 0) break;
                            ch.push_back(nxt);
                            cur = nxt;
                        }
                        if (ch.empty()) continue;
                        poolChain[i] = ch;
                        poolChained.insert(ch.begin(), ch.end());
                    }
                }
            }
            // Two stride-2 stem convs as one op (Stem2Op): the second conv -> the first, which is
            // folded. VKNN_HIP_FUSE_STEM2=0 keeps the two launches (A/B).
            std::map<int, int> stem2Of;   // second conv node -> first conv node
            std::map<int, int> stem2Tail; // second conv node -> its 1x1 tail conv
            std::set<int>      stem2Folded; // first convs and tails
            {
                const char *st2_env = std::getenv("VKNN_HIP_FUSE_STEM2");
                if (!st2_env || std::string(st2_env) != "0") {
                    std::set<int> skip(folded.begin(), folded.end());
                    for (auto &kv: scaled) skip.insert(kv.first);
                    for (auto &kv: convPool) skip.insert(kv.first), skip.insert(kv.second);
                    for (auto &kv: gapConv) skip.insert(kv.second);
                    for (auto &kv: pwPairs) skip.insert(kv.first);
                    skip.insert(pwFolded.begin(), pwFolded.end());
                    skip.insert(pwChained.begin(), pwChained.end());
                    for (auto &kv: actConv) skip.insert(kv.first);
                    for (auto &kv: addConv) skip.insert(kv.first);
                    std::map<TensorId, int> readers, producer;
                    for (size_t i = 0; i < g.nodes.size(); ++i) {
                        for (TensorId t: g.nodes[i].inputs)
                            if (t != kNoTensor) ++readers[t];
                        if (g.nodes[i].fusedResidual != kNoTensor) ++readers[g.nodes[i].fusedResidual];
                        for (TensorId t: g.nodes[i].outputs)
                            if (t != kNoTensor) producer[t] = (int) i;
                    }
                    for (TensorId t: g.outputs) readers[t] += 1000;
                    std::set<int> inSeg(idx.begin(), idx.end());
                    auto dense = [&](const Node &c) {
                        return c.type == OpType::Conv && c.inputs.size() >= 2 && g.isInitializer(c.inputs[1]) && c.fusedResidual == kNoTensor &&
                               g.desc(c.inputs[1]).shape.size() == 4 && !c.outputs.empty();
                    };
                    for (int b: idx) {
                        const Node &nb = g.nodes[b];
                        if (skip.count(b) || !dense(nb)) continue;
                        const TensorId t = nb.inputs[0];
                        auto           pa = producer.find(t);
                        if (pa == producer.end() || !inSeg.count(pa->second) || skip.count(pa->second) || stem2Folded.count(pa->second) ||
                            stem2Of.count(pa->second) || readers[t] != 1)
                            continue;
                        const Node &na = g.nodes[pa->second];
                        if (!dense(na) || place_.count(resolve(t)) || pstride(t) > 0 || pstride(na.inputs[0]) > 0 || place_.count(resolve(na.inputs[0])))
                            continue;
                        vkhip_conv_desc d1 = convDescOf(g, na), d2 = convDescOf(g, nb);
                        vkhip_conv_plan q1, q2, q3;
                        if (vkhip_conv3x3s2_pair_plan(&d1, &d2, nullptr, &q1, &q2, &q3) != VKHIP_OK) continue;
                        stem2Of[b] = pa->second;
                        stem2Folded.insert(pa->second);
                        // the 1x1 conv that is the second conv's only reader runs as the kernel's tail
                        const TensorId t2 = nb.outputs[0];
                        if (readers[t2] != 1 || place_.count(resolve(t2)) || pstride(t2) > 0) continue;
                        for (int c: idx) {
                            const Node &ncn = g.nodes[c];
                            if (skip.count(c) || !dense(ncn) || ncn.inputs[0] != t2) continue;
                            vkhip_conv_desc d3 = convDescOf(g, ncn);
                            if (vkhip_conv3x3s2_pair_plan(&d1, &d2, &d3, &q1, &q2, &q3) != VKHIP_OK) break;
                            stem2Tail[b] = c;
                            stem2Folded.insert(c);
                            break;
                        }
                    }
                }
            }
            // Two 3x3 stride-1 convs over 9-16 channels (+ the Add of the first one's input) as one
            // op (PairOp): second conv -> first; VKNN_HIP_FUSE_PAIR=0 keeps them apart (A/B). At 32
            // channels the halo tiles the tuner picks for the two convs are as fast as the pair.
            std::map<int, int> pairOf; // second conv -> first conv
            std::set<int>      pairFolded;
            {
                const char *pr_env = std::getenv("VKNN_HIP_FUSE_PAIR");
                if (!pr_env || std::string(pr_env) != "0") {
                    std::set<int> skip(folded.begin(), folded.end());
                    for (auto &kv: scaled) skip.insert(kv.first);
                    for (auto &kv: convPool) skip.insert(kv.first), skip.insert(kv.second);
                    for (auto &kv: gapConv) skip.insert(kv.second);
                    for (auto &kv: pwPairs) skip.insert(kv.first);
                    skip.insert(pwFolded.begin(), pwFolded.end());
                    skip.insert(pwChained.begin(), pwChained.end());
                    for (auto &kv: actConv) skip.insert(kv.first);
                    skip.insert(stem2Folded.begin(), stem2Folded.end());
                    for (auto &kv: stem2Of) skip.insert(kv.first);
                    std::map<TensorId, int> readers, producer;
                    for (size_t i = 0; i < g.nodes.size(); ++i) {
                        for (TensorId t: g.nodes[i].inputs)
                            if (t != kNoTensor) ++readers[t];
                        if (g.nodes[i].fusedResidual != kNoTensor) ++readers[g.nodes[i].fusedResidual];
                        for (TensorId t: g.nodes[i].outputs)
                            if (t != kNoTensor) producer[t] = (int) i;
                    }
                    for (TensorId t: g.outputs) readers[t] += 1000;
                    std::set<int> inSeg(idx.begin(), idx.end());
                    for (int b: idx) {
                        const Node &nb = g.nodes[b];
                        if (skip.count(b) || nb.type != OpType::Conv || nb.inputs.size() < 2 || !g.isInitializer(nb.inputs[1]) ||
                            nb.fusedResidual != kNoTensor || g.desc(nb.inputs[1]).shape.size() != 4)
                            continue;
                        const TensorId t = nb.inputs[0];
                        auto           pa = producer.find(t);
                        if (pa == producer.end() || !inSeg.count(pa->second) || skip.count(pa->second) || pairFolded.count(pa->second) ||
                            pairOf.count(pa->second) || readers[t] != 1 || addConv.count(pa->second))
                            continue;
                        const Node &na = g.nodes[pa->second];
                        if (na.type != OpType::Conv || na.inputs.size() < 2 || !g.isInitializer(na.inputs[1]) || na.fusedResidual != kNoTensor ||
                            g.desc(na.inputs[1]).shape.size() != 4 || place_.count(resolve(t)) || pstride(t) > 0)
                            continue;
                        vkhip_conv_desc d1 = convDescOf(g, na), d2 = convDescOf(g, nb);
                        if (d1.Cin > 16) continue;
                        // a folded Add: only the one whose residual is the pair's input
                        auto ad = addConv.find(b);
                        if (ad != addConv.end()) {
                            if (addFold[ad->second].second != na.inputs[0]) continue;
                            d2.has_res = 2;
                        }
                        vkhip_conv_plan q1, q2;
                        if (vkhip_conv3x3_pair_plan(&d1, &d2, &q1, &q2) != VKHIP_OK) continue;
                        pairOf[b] = pa->second;
                        pairFolded.insert(pa->second);
                    }
                }
            }
            // A stem conv and the FusedDwPw block that reads it (StemDwPwOp): block -> stem, which
            // is folded. VKNN_HIP_FUSE_STEM_BLOCK=0 keeps the two ops (A/B).
            std::map<int, int> sdOf;
            std::set<int>      sdFolded;
            {
                const char *sd_env = std::getenv("VKNN_HIP_FUSE_STEM_BLOCK");
                if (!sd_env || std::string(sd_env) != "0") {
                    std::set<int> skip(folded.begin(), folded.end());
                    for (auto &kv: scaled) skip.insert(kv.first);
                    for (auto &kv: convPool) skip.insert(kv.first), skip.insert(kv.second);
                    for (auto &kv: gapConv) skip.insert(kv.second);
                    for (auto &kv: pwPairs) skip.insert(kv.first);
                    skip.insert(pwFolded.begin(), pwFolded.end());
                    skip.insert(pwChained.begin(), pwChained.end());
                    for (auto &kv: actConv) skip.insert(kv.first);
                    for (auto &kv: addConv) skip.insert(kv.first);
                    skip.insert(stem2Folded.begin(), stem2Folded.end());
                    for (auto &kv: stem2Of) skip.insert(kv.first);
                    skip.insert(pairFolded.begin(), pairFolded.end());
                    for (auto &kv: pairOf) skip.insert(kv.first);
                    std::map<TensorId, int> readers, producer;
                    for (size_t i = 0; i < g.nodes.size(); ++i) {
                        for (TensorId t: g.nodes[i].inputs)
                            if (t != kNoTensor) ++readers[t];
                        if (g.nodes[i].fusedResidual != kNoTensor) ++readers[g.nodes[i].fusedResidual];
                        for (TensorId t: g.nodes[i].outputs)
                            if (t != kNoTensor) producer[t] = (int) i;
                    }
                    for (TensorId t: g.outputs) readers[t] += 1000;
                    std::set<int> inSeg(idx.begin(), idx.end());
                    for (int b: idx) {
                        const Node &nb = g.nodes[b];
                        if (skip.count(b) || nb.type != OpType::FusedDwPw || nb.inputs.size() < 5 || nb.outputs.empty()) continue;
                        bool inits = true; // weights given, biases given or absent
                        for (int k = 1; k < 5; ++k) inits = inits && (nb.inputs[k] != kNoTensor ? g.isInitializer(nb.inputs[k]) : (k & 1) == 0);
                        const TensorId t = nb.inputs[0];
                        auto           pa = producer.find(t);
                        const bool     res = nb.fusedResidual != kNoTensor;
                        // the block is the stem output's only reader (it lists the residual as an input too)
                        int own = res ? 1 : 0;
                        for (TensorId u: nb.inputs) own += u == t;
                        if (!inits || (res && nb.fusedResidual != t) || pa == producer.end() || !inSeg.count(pa->second) || skip.count(pa->second) ||
                            readers[t] != own)
                            continue;
                        const Node &na = g.nodes[pa->second];
                        if (na.type != OpType::Conv || na.inputs.size() < 2 || !g.isInitializer(na.inputs[1]) || na.fusedResidual != kNoTensor ||
                            g.desc(na.inputs[1]).shape.size() != 4 || place_.count(resolve(t)) || pstride(t) > 0 || pstride(na.inputs[0]) > 0 ||
                            place_.count(resolve(na.inputs[0])))
                            continue;
                        vkhip_conv_desc ds, dd, dp;
                        vkhip_conv_plan q1, q2, q3;
                        if (!StemDwPwOp::descs(g, na, nb, ds, dd, dp) || vkhip_stem_dwpw_plan(&ds, &dd, &dp, &q1, &q2, &q3) != VKHIP_OK) continue;
                        sdOf[b] = pa->second;
                        sdFolded.insert(pa->second);
                    }
                }
            }
            // Device buffers: one NC4HW4 fp16 buffer per activation (aliases share their source's;
            // a tensor placed in another one by planViews has none of its own).
            for (int i: idx) {
                const Node &nd = g.nodes[i];
                if (isAliasOp(g, nd)) continue;
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor && !g.isInitializer(t) && !produced.count(t) && !bufs_.count(t)) bufs_[t] = std::make_shared<DevBuf>(nc4Bytes(g.desc(t).shape));
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor && !bufs_.count(t) && !place_.count(t)) bufs_[t] = std::make_shared<DevBuf>(nc4Bytes(g.desc(t).shape));
            }
            std::vector<std::vector<TensorId>> ins, outs;
            for (int i: idx) {
                const Node &nd = g.nodes[i];
                std::unique_ptr<HipOp> op;
                auto gc = gapConv.find(i);
                if (gc != gapConv.end() && convOps.count(gc->second)) {
                    ConvOp   *c = convOps[gc->second];
                    const int R = vkhip_conv_pool_parts(&c->d, &c->plan);
                    if (R > 0) {
                        c->gapR    = R;
                        c->gapPart = std::make_shared<DevBuf>((size_t) c->d.N * ((c->d.Cout + 3) / 4) * R * 16);
                        gapParts[i] = c->gapPart;
                        gapR[i]     = R;
                        auto f  = std::make_unique<FoldedMulOp>();
                        f->into = c->name;
                        f->what = "global average pool";
                        op      = std::move(f);
                    }
                }
                const bool inPlace = viewCats_.count(i) || viewSplits_.count(i);
                if (inPlace) {
                    auto f  = std::make_unique<FoldedMulOp>();
                    f->what = nd.type == OpType::Concat ? "concat in place: its inputs are written into" : "split in place: its outputs are views of";
                    f->into = g.desc(nd.type == OpType::Concat ? nd.outputs[0] : nd.inputs[0]).name;
                    op      = std::move(f);
                } else if (op) {
                } else if (folded.count(i) || pools.count(i)) {
                    auto f  = std::make_unique<FoldedMulOp>();
                    f->into = foldedInto[i];
                    if (pools.count(i)) f->what = "max pool";
                    op      = std::move(f);
                } else if (actFold.count(i)) {
                    auto f  = std::make_unique<FoldedMulOp>();
                    f->what = "hard-sigmoid";
                    f->into = g.nodes[actFold[i]].name;
                    op      = std::move(f);
                } else if (pairFolded.count(i)) {
                    auto f = std::make_unique<FoldedMulOp>();
                    f->what = "3x3 conv: runs with the 3x3 conv that reads it,";
                    for (auto &kv: pairOf)
                        if (kv.second == i) f->into = g.nodes[kv.first].name;
                    op = std::move(f);
                } else if (pairOf.count(i)) {
                    auto c = std::make_unique<PairOp>();
                    c->na  = &g.nodes[pairOf[i]];
                    auto ad = addConv.find(i);
                    if (ad != addConv.end()) c->addOut = g.nodes[ad->second].outputs[0];
                    op = std::move(c);
                } else if (poolChained.count(i)) {
                    auto f  = std::make_unique<FoldedMulOp>();
                    f->what = "max pool: computed in the launch of the chain's first pool,";
                    for (auto &kv: poolChain)
                        for (int m: kv.second)
                            if (m == i) f->into = g.nodes[kv.first].name;
                    op = std::move(f);
                } else if (sdFolded.count(i)) {
                    auto f  = std::make_unique<FoldedMulOp>();
                    f->what = "stem conv: runs with the depthwise block that reads it,";
                    for (auto &kv: sdOf)
                        if (kv.second == i) f->into = g.nodes[kv.first].name;
                    op = std::move(f);
                } else if (sdOf.count(i)) {
                    auto c = std::make_unique<StemDwPwOp>();
                    c->na  = &g.nodes[sdOf[i]];
                    op     = std::move(c);
                } else if (stem2Folded.count(i)) {
                    auto f = std::make_unique<FoldedMulOp>();
                    f->what = "3x3 stride-2 conv: runs with the stride-2 conv that reads it,";
                    for (auto &kv: stem2Of)
                        if (kv.second == i) f->into = g.nodes[kv.first].name;
                    for (auto &kv: stem2Tail)
                        if (kv.second == i) f->what = "1x1 conv: runs as the tail of the stride-2 pair,", f->into = g.nodes[kv.first].name;
                    op = std::move(f);
                } else if (stem2Of.count(i)) {
                    auto c = std::make_unique<Stem2Op>();
                    c->na  = &g.nodes[stem2Of[i]];
                    if (stem2Tail.count(i)) c->nc = &g.nodes[stem2Tail[i]];
                    op = std::move(c);
                } else if (addFold.count(i)) {
                    auto f  = std::make_unique<FoldedMulOp>();
                    f->what = "add (a residual after the activation)";
                    f->into = g.nodes[addFold[i].first].name;
                    op      = std::move(f);
                } else if (pwFolded.count(i)) {
                    auto f = std::make_unique<FoldedMulOp>();
                    f->what = "3x3 conv: runs with the 1x1 conv that reads it,";
                    for (auto &kv: pwPairs)
                        if (kv.second == i) f->into = g.nodes[kv.first].name;
                    op = std::move(f);
                } else if (pwChained.count(i)) {
                    auto f = std::make_unique<FoldedMulOp>();
                    f->what = "1x1 conv: runs with the 3x3 + 1x1 pair whose output it reads,";
                    for (auto &kv: pwChain)
                        if (kv.second == i) f->into = g.nodes[kv.first].name;
                    op = std::move(f);
                } else if (pwPairs.count(i)) {
                    auto c = std::make_unique<ConvPwOp>();
                    c->n3  = &g.nodes[pwPairs[i]];
                    if (pwChain.count(i)) c->n4 = &g.nodes[pwChain[i]];
                    op     = std::move(c);
                } else op = makeOp(g, nd);
                if (!op) throw Error(Status::Unsupported, std::string("HIP backend has no kernel for ") + opTypeName(nd.type) + " (" + nd.name + ")");
                auto sit = scaled.find(i);
                if (sit != scaled.end()) {
                    auto *c     = static_cast<ConvOp *>(op.get());
                    c->scaledIn = sit->second.first;
                    c->xscale   = sit->second.second;
                }
                auto ait = actConv.find(i);
                if (ait != actConv.end()) {
                    auto       *c  = static_cast<ConvOp *>(op.get());
                    const Node &un = g.nodes[ait->second];
                    c->actOut      = un.outputs[0];
                    c->foldAct     = VKHIP_ACT_HARDSIGMOID;
                    c->foldLo      = un.actLo;
                    c->foldHi      = un.actHi;
                }
                auto pcit = poolChain.find(i);
                if (pcit != poolChain.end()) {
                    auto *m = static_cast<MaxPoolOp *>(op.get());
                    for (int c: pcit->second) m->chain.push_back(g.nodes[c].outputs[0]);
                }
                auto dit = pairOf.count(i) ? addConv.end() : addConv.find(i); // a pair op takes its Add itself
                if (dit != addConv.end()) {
                    auto *c    = static_cast<ConvOp *>(op.get());
                    c->addOut  = g.nodes[dit->second].outputs[0];
                    c->postRes = addFold[dit->second].second;
                }
                auto pit = convPool.find(i);
                if (pit != convPool.end()) {
                    auto       *c  = static_cast<ConvOp *>(op.get());
                    const Node &pn = g.nodes[pit->second];
                    NCHW        y  = NCHW::from(g.desc(pn.inputs[0]).shape), z = NCHW::from(g.desc(pn.outputs[0]).shape);
                    c->poolOut     = pn.outputs[0];
                    c->pd.N = (int) y.n; c->pd.C = (int) y.c; c->pd.H = (int) y.h; c->pd.W = (int) y.w; c->pd.OH = (int) z.h; c->pd.OW = (int) z.w;
                    c->pd.KH = c->pd.KW = 3; c->pd.SH = c->pd.SW = 2; c->pd.PT = c->pd.PL = 1;
                }
                op->name = nd.name;
                op->type = nd.type;
                const bool gapFolded = gapParts.count(i) > 0;
                const bool pwOp = pwPairs.count(i) || pwFolded.count(i) || pwChained.count(i) || stem2Of.count(i) || stem2Folded.count(i) ||
                                  pairOf.count(i) || pairFolded.count(i) || sdOf.count(i) || sdFolded.count(i);
                if (nd.type == OpType::Conv && !inPlace && !gapFolded && !folded.count(i) && !pools.count(i) && !pwOp) {
                    bool v = false;
                    for (TensorId t: {nd.inputs[0], nd.outputs[0]}) v = v || pstride(t) > 0;
                    if (dit != addConv.end()) v = v || pstride(g.nodes[dit->second].outputs[0]) > 0;
                    static_cast<ConvOp *>(op.get())->viewIO = v;
                }
                if (!gapFolded) op->prepare(nd, env_);
                else op->kind = "folded";
                if (gapConv.size() && nd.type == OpType::Conv && !pwOp) convOps[i] = static_cast<ConvOp *>(op.get());
                auto sg = seGap.find(i);
                if (sg != seGap.end() && gapParts.count(sg->second)) {
                    auto       *se = static_cast<SeOp *>(op.get());
                    const Node &gn = g.nodes[sg->second];
                    NCHW        x  = NCHW::from(g.desc(gn.inputs[0]).shape);
                    se->part = gapParts[sg->second];
                    se->R    = gapR[sg->second];
                    se->HW   = x.h * x.w;
                }
                opPos[i] = ops_.size();
                ops_.push_back(std::move(op));
                // data the op's launches read and write (alias and folded ops launch nothing)
                std::vector<TensorId> in, out;
                if (inPlace) {
                    // no launch, but the dependency chain runs through it (readers of the concat
                    // output wait for the writers of its slices)
                    for (TensorId t: nd.inputs)
                        if (t != kNoTensor) in.push_back(resolve(t));
                    for (TensorId t: nd.outputs)
                        if (t != kNoTensor) out.push_back(resolve(t));
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (gapFolded) {
                    // the pool's output stands for the sums the conv's launch writes
                    outs[opPos[gapConv[i]]].push_back(resolve(nd.outputs[0]));
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (folded.count(i) || pools.count(i) || pwFolded.count(i) || pwChained.count(i) || actFold.count(i) || addFold.count(i) ||
                    stem2Folded.count(i) || poolChained.count(i) || pairFolded.count(i) || sdFolded.count(i)) {
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (pairOf.count(i)) {
                    // the pair reads the first conv's input and writes the second's output (or the Add's)
                    in.push_back(resolve(g.nodes[pairOf[i]].inputs[0]));
                    auto ad = addConv.find(i);
                    out.push_back(resolve(ad != addConv.end() ? g.nodes[ad->second].outputs[0] : nd.outputs[0]));
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (sdOf.count(i)) {
                    // the op reads the stem's input and writes the block's output
                    in.push_back(resolve(g.nodes[sdOf[i]].inputs[0]));
                    out.push_back(resolve(nd.outputs[0]));
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (stem2Of.count(i)) {
                    // the pair reads the first conv's input and writes the second's output (or its tail's)
                    in.push_back(resolve(g.nodes[stem2Of[i]].inputs[0]));
                    out.push_back(resolve(stem2Tail.count(i) ? g.nodes[stem2Tail[i]].outputs[0] : nd.outputs[0]));
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (pwPairs.count(i)) {
                    // the pair reads the 3x3's input (and the 1x1's residual) and writes the 1x1's output
                    in.push_back(resolve(g.nodes[pwPairs[i]].inputs[0]));
                    if (nd.fusedResidual != kNoTensor) in.push_back(resolve(nd.fusedResidual));
                    out.push_back(resolve(nd.outputs[0]));
                    if (pwChain.count(i)) out.push_back(resolve(g.nodes[pwChain[i]].outputs[0]));
                    ins.push_back(in);
                    outs.push_back(out);
                    continue;
                }
                if (!isAliasOp(g, nd)) {
                    if (sit != scaled.end()) {
                        in.push_back(resolve(sit->second.first));
                        in.push_back(resolve(sit->second.second));
                    }
                    for (size_t k = sit != scaled.end() ? 1 : 0; k < nd.inputs.size(); ++k) {
                        TensorId t = nd.inputs[k];
                        if (t != kNoTensor && !g.isInitializer(t)) in.push_back(resolve(t));
                    }
                    if (nd.fusedResidual != kNoTensor) in.push_back(resolve(nd.fusedResidual));
                    if (dit != addConv.end()) in.push_back(resolve(addFold[dit->second].second));
                    if (pcit != poolChain.end())
                        for (int c: pcit->second) out.push_back(resolve(g.nodes[c].outputs[0]));
                    if (pit != convPool.end()) out.push_back(resolve(g.nodes[pit->second].outputs[0]));
                    else if (ait != actConv.end()) out.push_back(resolve(g.nodes[ait->second].outputs[0]));
                    else if (dit != addConv.end()) out.push_back(resolve(g.nodes[dit->second].outputs[0]));
                    else
                        for (TensorId t: nd.outputs)
                            if (t != kNoTensor) out.push_back(resolve(t));
                }
                ins.push_back(in);
                outs.push_back(out);
            }
            check(vkhip_stream_sync(nullptr), "prepare sync");
            if (cfg.hipBranches) planStreams(ins, outs);
            if (refineEnabled() && !markers_) refinePlans();
        }

        // In-graph plan refinement. The autotuner times each conv alone on rotating cold buffers;
        // inside the forward pass its input was just written by the op before it and partly sits in
        // the last-level cache, which can reorder near-ties. Every op with near-tie candidates is
        // timed here in the segment's own op order (one in-order stream, events around each op,
        // the whole pass queued behind a short device sleep so the kernels run back to back), each
        // pass switching all such ops to their j-th candidate at once (ops are timed independently
        // of each other's choice). Three passes per candidate; an op keeps an alternative only if
        // its best time beats the tuner's pick by more than 2%.
        void HipSegment::refinePlans() {
            // a pick is changed only for a tune-table key no other op of the segment uses (another op
            // with the same key took the tuner's pick from the table and keeps it)
            std::map<std::string, int> keyUses;
            for (auto &op: ops_)
                if (!op->planKey().empty()) ++keyUses[op->planKey()];
            std::vector<int> ks;
            int              nc = 0;
            for (size_t k = 0; k < ops_.size(); ++k)
                if (ops_[k]->candidates() > 1 && keyUses[ops_[k]->planKey()] == 1) {
                    ks.push_back((int) k);
                    nc = std::max(nc, ops_[k]->candidates());
                } else ops_[k]->commitCandidate(0); // keeps its pick, frees the alternatives
            if (ks.empty()) return;
            for (TensorId t: boundaryInputs)
                if (!extIn_.count(t) && !staging_.count(t)) {
                    staging_[t] = std::make_shared<DevBuf>((size_t) numElements(g_.desc(t).shape) * 4);
                    check(vkhip_fill_zero(staging_[t]->ptr, staging_[t]->bytes, stream_), "refine fill");
                }
            for (TensorId t: boundaryOutputs)
                if (!outStaging_.count(t)) outStaging_[t] = std::make_shared<DevBuf>((size_t) numElements(g_.desc(t).shape) * 4);
            while (events_.size() < 2 * ops_.size()) {
                vkhip_event_t e;
                check(vkhip_event_create(&e), "event");
                events_.push_back(e);
            }
            std::vector<std::vector<double>> us(ks.size(), std::vector<double>(nc, 1e30));
            for (int rep = 0; rep < 4; ++rep)
                for (int j = 0; j < nc; ++j) {
                    for (int k: ks) ops_[k]->useCandidate(std::min(j, ops_[k]->candidates() - 1));
                    check(vkhip_gpu_sleep(3000, stream_), "refine sleep");
                    recordAll(true);
                    check(vkhip_stream_sync(stream_), "refine sync");
                    if (rep == 0) continue; // the first pass of each candidate warms it up
                    for (size_t i = 0; i < ks.size(); ++i) {
                        if (j >= ops_[ks[i]]->candidates()) continue;
                        float ms = 0;
                        check(vkhip_event_elapsed_ms(events_[2 * ks[i]], events_[2 * ks[i] + 1], &ms), "event time");
                        us[i][j] = std::min(us[i][j], (double) ms * 1e3);
                    }
                }
            for (size_t i = 0; i < ks.size(); ++i) {
                int best = 0;
                for (int j = 1; j < ops_[ks[i]]->candidates(); ++j)
                    if (us[i][j] < us[i][0] * 0.98 && us[i][j] < us[i][best]) best = j;
                ops_[ks[i]]->commitCandidate(best);
            }
        }

        // Two-stream list schedule over the recorded op order. Every activation has its own buffer
        // and is written by one op, so only read-after-write dependencies order ops. An op goes on
        // the main stream when it consumes the output of the op last placed there (the common
        // chain); an op that does not (a branch that only needs older tensors, such as a residual
        // block's projection shortcut) goes on the side stream, so the two overlap. Dependencies
        // that cross streams become event waits, and the side stream is joined back into the main
        // one before the boundary outputs are unpacked. The same sequence is what the HIP graph
        // captures (the first event wait forks the side stream into the capture).
        static constexpr double kSideMinUs = 4.0;

        void HipSegment::planStreams(const std::vector<std::vector<TensorId>> &ins, const std::vector<std::vector<TensorId>> &outs) {
            const int            n = (int) ops_.size();
            std::map<TensorId, int> producer; // tensor -> op index
            for (int k = 0; k < n; ++k)
                for (TensorId t: outs[k]) producer[t] = k;
            opStream_.assign(n, 0);
            opWaits_.assign(n, {});
            opSignals_.assign(n, 0);
            int tail[2]      = {-1, -1};  // last op placed on each stream (-1: the pack / nothing)
            int waited[2][2] = {{-2, -2}, {-2, -2}}; // waited[s][o]: latest op of stream o that s waited for
            bool any_side    = false;
            for (int k = 0; k < n; ++k) {
                if (ins[k].empty() && outs[k].empty()) continue; // alias: nothing launched
                std::vector<int> deps;
                for (TensorId t: ins[k]) {
                    auto it = producer.find(t);
                    deps.push_back(it != producer.end() && it->second < k ? it->second : -1);
                }
                const bool on_main_tail = tail[0] < 0 || std::find(deps.begin(), deps.end(), tail[0]) != deps.end();
                const bool on_side_tail = tail[1] >= 0 && std::find(deps.begin(), deps.end(), tail[1]) != deps.end();
                // Only ops long enough to gain from overlap go to the side stream: each cross-stream
                // wait costs a few microseconds of dependency latency in the graph, which small ops
                // (batch 1) do not recover. Estimated time at 6 TB/s or 1.5 PFLOP/s.
                const double est_us     = std::max((double) ops_[k]->bytes / 6e6, ops_[k]->flops / 1.5e9);
                const bool   worth      = est_us >= kSideMinUs;
                const int    st         = on_main_tail ? 0 : (on_side_tail || (!deps.empty() && worth) ? 1 : 0);
                opStream_[k]            = st;
                any_side |= st == 1;
                for (int d: deps) {
                    const int ds = d < 0 ? 0 : opStream_[d];
                    if (ds == st) continue;
                    if (d <= waited[st][ds]) continue; // an earlier wait already covers it
                    waited[st][ds] = d;
                    opWaits_[k].push_back(d);
                    if (d >= 0) opSignals_[d] = 1;
                }
                tail[st] = k;
            }
            useSide_ = any_side;
            if (!useSide_) return;
            check(vkhip_stream_create(&side_), "side stream");
            opEvents_.assign(n, nullptr);
            for (int k = 0; k < n; ++k)
                if (opSignals_[k]) check(vkhip_event_create(&opEvents_[k]), "event");
            check(vkhip_event_create(&packEvent_), "event");
            check(vkhip_event_create(&joinEvent_), "event");
        }

        HipSegment::~HipSegment() {
            if (graph_) vkhip_graph_destroy(graph_);
            for (auto &e: events_) vkhip_event_destroy(e);
            if (side_) {
                vkhip_stream_sync(side_);
                vkhip_stream_destroy(side_);
            }
            for (auto &e: opEvents_)
                if (e) vkhip_event_destroy(e);
            if (packEvent_) vkhip_event_destroy(packEvent_);
            if (joinEvent_) vkhip_event_destroy(joinEvent_);
            if (stream_) {
                vkhip_stream_sync(stream_);
                vkhip_stream_destroy(stream_);
            }
            for (auto &kv: dma_) vkhip_dmabuf_release(kv.second.h);
        }

        void *HipSegment::importDmaBuf(TensorId t, int fd, size_t bytes) {
            struct stat st {};
            const uint64_t id = ::fstat(fd, &st) == 0 ? ((uint64_t) st.st_dev << 40) ^ (uint64_t) st.st_ino : 0;
            DmaImport &imp = dma_[t];
            if (imp.h && imp.bytes == bytes && (id ? imp.id == id : imp.fd == fd)) return imp.ptr;
            if (imp.h) {
                check(vkhip_stream_sync(stream_), "sync");
                dropGraph(); // a captured graph holds the old address
                vkhip_dmabuf_release(imp.h);
                imp = DmaImport {};
            }
            vkhip_dmabuf h   = nullptr;
            void        *ptr = nullptr;
            check(vkhip_dmabuf_import(fd, bytes, &h, &ptr), "dma-buf import of " + g_.desc(t).name);
            imp = DmaImport {id, fd, bytes, h, ptr};
            return ptr;
        }

        // Layout code of the boundary converter for a declared dma-buf format; Auto means the
        // device-native NC4HW4 fp16.
        static std::pair<int, bool> dmaLayout(const RtTensor &rt) {
            if (rt.dmaBufFormat == TensorFormat::Auto) return {2, true};
            if (rt.dmaBufFormat != TensorFormat::NCHW && rt.dmaBufFormat != TensorFormat::NHWC && rt.dmaBufFormat != TensorFormat::NC4HW4)
                throw Error(Status::InvalidArgument, "dma-buf layout must be NCHW, NHWC, NC4HW4 or Auto");
            if (rt.dmaBufDtype != DType::Float32 && rt.dmaBufDtype != DType::Float16)
                throw Error(Status::InvalidArgument, "dma-buf dtype must be fp32 or fp16");
            return {(int) rt.dmaBufFormat, rt.dmaBufDtype == DType::Float16};
        }

        static size_t dmaBytes(const Shape &s, std::pair<int, bool> fmt) {
            NCHW         x = NCHW::from(s);
            const size_t c = fmt.first == 2 ? (size_t) (x.c + 3) / 4 * 4 : (size_t) x.c;
            return (size_t) x.n * c * x.h * x.w * (fmt.second ? 2 : 4);
        }

        // Bind (or unbind) this run's dma-buf inputs and outputs (reference vk_backend.cpp:1218-1318):
        // an input fd becomes the source of the boundary pack, converted from its declared layout;
        // an output fd receives the boundary tensor in its declared layout instead of the host path.
        void HipSegment::bindDmaBufs(ExecContext &ctx) {
            for (TensorId t: boundaryInputs) {
                const RtTensor &rt = ctx.t(t);
                if (rt.dmaBufFd >= 0) {
                    const auto fmt = dmaLayout(rt);
                    void      *ptr = importDmaBuf(t, rt.dmaBufFd, dmaBytes(g_.desc(t).shape, fmt));
                    bindDeviceInputAs(t, ptr, fmt.first, fmt.second);
                    dmaIn_.insert(t);
                } else if (dmaIn_.count(t)) {
                    extIn_.erase(t);
                    extFmt_.erase(t);
                    dmaIn_.erase(t);
                    dropGraph();
                }
            }
            for (TensorId t: boundaryOutputs) {
                const RtTensor &rt = ctx.t(t);
                if (rt.dmaBufFd >= 0) {
                    const auto fmt = dmaLayout(rt);
                    void      *ptr = importDmaBuf(t, rt.dmaBufFd, dmaBytes(g_.desc(t).shape, fmt));
                    auto       it  = extOut_.find(t);
                    if (it == extOut_.end() || it->second.first != ptr || it->second.second != fmt) {
                        extOut_[t] = {ptr, fmt};
                        dropGraph();
                    }
                } else if (extOut_.erase(t)) {
                    dropGraph();
                }
            }
        }

        // In-place channel concat and split (no counterpart in the reference, which copies: ops/concat.cpp,
        // ops/split.cpp). NC4HW4 stores each image as consecutive 4-channel planes, so a channel slice
        // that starts on a 4-channel boundary is a view: the same buffer at a plane offset, with the
        // wider tensor's planes per image as its stride. A Concat whose inputs are all such slices
        // is planned so every producer writes straight into its slice of the concat's buffer, and a
        // Split so its outputs are views of its input; neither launches anything. Every op that
        // writes or reads such a view must take plane strides (the conv GEMM and split-K kernels,
        // add, max pool, resize); a concat or split whose tensors meet any other op keeps its copy.
        void HipSegment::planViews(const std::vector<int> &idx, const std::set<int> &noWrite, const std::set<int> &noRead) {
            const Graph &g = g_;
            std::set<int> inSeg(idx.begin(), idx.end());
            std::map<TensorId, int>              producer;
            std::map<TensorId, std::vector<int>> readers;
            for (size_t i = 0; i < g.nodes.size(); ++i) {
                const Node &nd = g.nodes[i];
                for (TensorId t: nd.inputs)
                    if (t != kNoTensor) readers[t].push_back((int) i);
                if (nd.fusedResidual != kNoTensor && std::find(nd.inputs.begin(), nd.inputs.end(), nd.fusedResidual) == nd.inputs.end())
                    readers[nd.fusedResidual].push_back((int) i);
                for (TensorId t: nd.outputs)
                    if (t != kNoTensor) producer[t] = (int) i;
            }
            std::set<TensorId> gout(g.outputs.begin(), g.outputs.end());
            auto is4d = [&](TensorId t) { return g.desc(t).shape.size() == 4; };
            auto chan = [&](TensorId t) { return g.desc(t).shape[1]; };
            auto axis1 = [&](const Node &nd) {
                int64_t ax = nd.attr.geti("axis", 0);
                return ax == 1 || ax == -3;
            };
            // candidates: channel concats / splits whose slices all start on a 4-channel boundary
            std::set<int> cats, splits;
            for (int i: idx) {
                const Node &nd = g.nodes[i];
                if (nd.outputs.empty() || nd.outputs[0] == kNoTensor || !is4d(nd.outputs[0])) continue;
                if (nd.type == OpType::Concat && axis1(nd) && nd.inputs.size() >= 2) {
                    bool ok = true;
                    for (size_t k = 0; k + 1 < nd.inputs.size(); ++k) ok = ok && nd.inputs[k] != kNoTensor && chan(nd.inputs[k]) % 4 == 0;
                    if (ok) cats.insert(i);
                }
                if (nd.type == OpType::Split && axis1(nd) && nd.inputs.size() >= 1 && is4d(nd.inputs[0])) {
                    bool ok = true;
                    for (size_t k = 0; k + 1 < nd.outputs.size(); ++k) ok = ok && (nd.outputs[k] == kNoTensor || chan(nd.outputs[k]) % 4 == 0);
                    if (ok) splits.insert(i);
                }
            }
            auto weightsCin = [&](const Node &nd) { return g.desc(nd.inputs[1]).shape.size() == 4 ? g.desc(nd.inputs[1]).shape[1] : 0; };
            auto canWrite = [&](int p, const std::set<int> &cs) {
                const Node &nd = g.nodes[p];
                if (noWrite.count(p)) return false;
                switch (nd.type) {
                    case OpType::Conv: return nd.attr.geti("group", 1) == 1 && nd.fusedResidual == kNoTensor && weightsCin(nd) > 4;
                    case OpType::Add: return nd.inputs.size() == 2 && g.desc(nd.inputs[0]).shape == g.desc(nd.inputs[1]).shape;
                    case OpType::MaxPool: case OpType::Resize: return true;
                    case OpType::Concat: return cs.count(p) > 0; // an in-place concat inside another one
                    default: return false;
                }
            };
            auto canRead = [&](int c, TensorId t, const std::set<int> &cs, const std::set<int> &ss) {
                const Node &nd = g.nodes[c];
                if (!inSeg.count(c) || noRead.count(c)) return false;
                switch (nd.type) {
                    case OpType::Conv:
                        return nd.attr.geti("group", 1) == 1 && nd.inputs[0] == t && nd.fusedResidual != t && weightsCin(nd) > 4 &&
                               std::count(nd.inputs.begin(), nd.inputs.end(), t) == 1;
                    case OpType::Add: return nd.inputs.size() == 2 && g.desc(nd.inputs[0]).shape == g.desc(nd.inputs[1]).shape;
                    case OpType::MaxPool: case OpType::Resize: return true;
                    case OpType::Concat: return cs.count(c) > 0;
                    case OpType::Split: return ss.count(c) > 0;
                    default: return false;
                }
            };
            for (int round = 0; round < 64; ++round) {
                place_.clear();
                std::set<int> badCat, badSplit;
                for (int i: splits) {
                    const Node &nd = g.nodes[i];
                    int64_t     c0 = 0;
                    for (TensorId t: nd.outputs) {
                        if (t != kNoTensor) place_[t] = {nd.inputs[0], c0 / 4};
                        c0 += t == kNoTensor ? 0 : chan(t);
                    }
                }
                std::set<TensorId> fromCat; // tensors placed by a concat
                for (int i: cats) {
                    const Node &nd = g.nodes[i];
                    int64_t     off = 0;
                    for (TensorId t0: nd.inputs) {
                        TensorId t = t0;
                        int64_t  o = off;
                        while (place_.count(t) && !fromCat.count(t)) { // climb from a split output to the split input
                            o -= place_[t].off;
                            t = place_[t].parent;
                        }
                        auto it = place_.find(t);
                        const bool clash = (it != place_.end() && (it->second.parent != nd.outputs[0] || it->second.off != o)) || alias_.count(t);
                        if (o < 0 || clash || !producer.count(t) || !inSeg.count(producer[t]) || gout.count(t)) {
                            badCat.insert(i);
                            break;
                        }
                        place_[t] = {nd.outputs[0], o};
                        fromCat.insert(t);
                        off += chan(t0) / 4;
                    }
                }
                // every tensor that lives in another one: written by a view-capable op, read only by
                // view-capable ops of this segment, not a graph output
                for (auto &kv: place_) {
                    const TensorId t = kv.first;
                    int            owner = -1; // the concat or split that made it a view
                    for (int i: cats)
                        if (g.nodes[i].outputs[0] == kv.second.parent && fromCat.count(t)) owner = i;
                    const bool splitOut = !fromCat.count(t);
                    if (splitOut)
                        for (int i: splits)
                            if (std::find(g.nodes[i].outputs.begin(), g.nodes[i].outputs.end(), t) != g.nodes[i].outputs.end()) owner = i;
                    bool ok = !gout.count(t) && !alias_.count(t);
                    if (!splitOut) ok = ok && producer.count(t) && canWrite(producer[t], cats);
                    for (int c: readers[t]) ok = ok && canRead(c, t, cats, splits);
                    if (!ok && owner >= 0) (splitOut ? badSplit : badCat).insert(owner);
                }
                // a concat output that is itself placed must come from an in-place concat (checked
                // above); a split input may be a view itself (nested offsets add up in dev())
                if (badCat.empty() && badSplit.empty()) break;
                for (int i: badCat) cats.erase(i);
                for (int i: badSplit) splits.erase(i);
            }
            viewCats_   = cats;
            viewSplits_ = splits;
        }

        TensorId HipSegment::resolve(TensorId t) const {
            auto it = alias_.find(t);
            while (it != alias_.end()) {
                t  = it->second;
                it = alias_.find(t);
            }
            return t;
        }

        void *HipSegment::dev(TensorId t) {
            t       = resolve(t);
            auto pl = place_.find(t);
            if (pl != place_.end()) {
                const Shape &sh = g_.desc(t).shape;
                return static_cast<char *>(dev(pl->second.parent)) + pl->second.off * sh[2] * sh[3] * 8;
            }
            auto it = bufs_.find(t);
            if (it == bufs_.end()) throw Error(Status::RuntimeError, "no device buffer for tensor " + std::to_string(t));
            return it->second->ptr;
        }

        int64_t HipSegment::pstride(TensorId t) const {
            t = resolve(t);
            if (!place_.count(t)) return 0;
            while (place_.count(t)) t = place_.at(t).parent;
            return (g_.desc(t).shape[1] + 3) / 4;
        }

        void   *SegEnv::dev(TensorId t) { return seg->dev(t); }
        int64_t SegEnv::pstride(TensorId t) { return seg->pstride(t); }

        void HipSegment::bindDeviceInput(TensorId t, const float *devNchw) {
            if (extIn_[t] != devNchw || extFmt_.count(t)) {
                extIn_[t] = devNchw;
                extFmt_.erase(t);
                dropGraph();
            }
        }

        void HipSegment::bindDeviceInputAs(TensorId t, const void *dev, int fmt, bool f16) {
            if (fmt < 0 || fmt > 2) throw Error(Status::InvalidArgument, "declared input layout must be 0 (NCHW), 1 (NHWC) or 2 (NC4HW4)");
            const auto decl = std::make_pair(fmt, f16);
            auto       it   = extFmt_.find(t);
            if (extIn_[t] != dev || it == extFmt_.end() || it->second != decl) {
                extIn_[t]  = (const float *) dev;
                extFmt_[t] = decl;
                dropGraph();
            }
        }

        void HipSegment::dropGraph() {
            if (graph_) vkhip_graph_destroy(graph_);
            graph_  = nullptr;
            replay_ = 0;
        }

        // Everything the segment does on the device for one run: boundary packs, ops, boundary unpacks.
        void HipSegment::recordAll(bool timed) {
            for (TensorId t: boundaryInputs) {
                const Shape &s = g_.desc(t).shape;
                NCHW         x = NCHW::from(s);
                const float *src = extIn_.count(t) ? extIn_[t] : (const float *) staging_[t]->ptr;
                auto         fit = extFmt_.find(t);
                if (fit != extFmt_.end())
                    check(vkhip_boundary_convert(src, fit->second.first, fit->second.second ? 1 : 0, dev(t), 2, 1, x.n, x.c, x.h, x.w, stream_),
                          "boundary convert");
                else check(vkhip_pack_nchw_f32(src, dev(t), x.n, x.c, x.h, x.w, stream_), "pack");
            }
            if (timed || !useSide_ || markers_) {
                // one in-order stream (profiling times each op between its own two events; trace
                // markers need the launches in plan order)
                for (size_t k = 0; k < ops_.size(); ++k) {
                    if (markers_) check(vkhip_dispatch_marker((int32_t) k, stream_), "marker");
                    if (timed) vkhip_event_record(events_[2 * k], stream_);
                    for (int r = 0; r < (timed ? cfg_.profileReps : 1); ++r) ops_[k]->record(env_, stream_);
                    if (timed) vkhip_event_record(events_[2 * k + 1], stream_);
                }
            } else {
                check(vkhip_event_record(packEvent_, stream_), "event");
                for (size_t k = 0; k < ops_.size(); ++k) {
                    vkhip_stream_t s = opStream_[k] ? side_ : stream_;
                    for (int d: opWaits_[k]) check(vkhip_stream_wait_event(s, d < 0 ? packEvent_ : opEvents_[d]), "stream wait");
                    ops_[k]->record(env_, s);
                    if (opSignals_[k]) check(vkhip_event_record(opEvents_[k], s), "event");
                }
                // join: everything on the side stream completes before the main stream goes on
                check(vkhip_event_record(joinEvent_, side_), "event");
                check(vkhip_stream_wait_event(stream_, joinEvent_), "stream wait");
            }
            // host-bound outputs leave through one multi-tensor unpack (one launch for up to 8)
            std::vector<const void *> usrc;
            std::vector<float *>      udst;
            std::vector<int64_t>      ushape;
            for (TensorId t: boundaryOutputs) {
                NCHW y  = NCHW::from(g_.desc(t).shape);
                auto xo = extOut_.find(t);
                if (xo != extOut_.end())
                    check(vkhip_boundary_convert(dev(t), 2, 1, xo->second.first, xo->second.second.first, xo->second.second.second ? 1 : 0, y.n,
                                                 y.c, y.h, y.w, stream_),
                          "boundary convert (dma-buf output)");
                else {
                    usrc.push_back(dev(t));
                    udst.push_back((float *) outStaging_[t]->ptr);
                    for (int64_t v: {y.n, y.c, y.h, y.w}) ushape.push_back(v);
                }
            }
            if (!usrc.empty())
                check(vkhip_unpack_nchw_f32_multi(usrc.data(), udst.data(), ushape.data(), (int32_t) usrc.size(), stream_), "unpack");
        }

        void HipSegment::launch(bool profile) {
            // staging buffers for boundary tensors
            for (TensorId t: boundaryInputs)
                if (!extIn_.count(t) && !staging_.count(t)) staging_[t] = std::make_shared<DevBuf>((size_t) numElements(g_.desc(t).shape) * 4);
            for (TensorId t: boundaryOutputs)
                if (!outStaging_.count(t)) outStaging_[t] = std::make_shared<DevBuf>((size_t) numElements(g_.desc(t).shape) * 4);
            if (profile) {
                while (events_.size() < 2 * ops_.size()) {
                    vkhip_event_t e;
                    check(vkhip_event_create(&e), "event");
                    events_.push_back(e);
                }
                recordAll(true);
                return;
            }
            if (!cfg_.hipGraphs) {
                recordAll(false);
                return;
            }
            // First run executes eagerly; the second captures the identical sequence into a graph.
            if (!graph_ && replay_ == 0) {
                recordAll(false);
                replay_ = 1;
                return;
            }
            if (!graph_) {
                check(vkhip_graph_begin(stream_), "graph capture");
                try {
                    recordAll(false);
                } catch (...) {
                    // end the capture so the stream leaves capture mode, drop the partial graph,
                    // and start over eagerly on the next run
                    vkhip_graph_t partial = nullptr;
                    if (vkhip_graph_end(stream_, &partial) == VKHIP_OK && partial) vkhip_graph_destroy(partial);
                    replay_ = 0;
                    throw;
                }
                check(vkhip_graph_end(stream_, &graph_), "graph capture");
            }
            check(vkhip_graph_launch(graph_, stream_), "graph launch");
        }

        void HipSegment::run(ExecContext &ctx) {
            const bool profile = ctx.profiler && ctx.profiler->enabled();
            auto       t0      = std::chrono::high_resolution_clock::now();
            bindDmaBufs(ctx);
            for (TensorId t: boundaryInputs) {
                RtTensor &rt = ctx.t(t);
                if (extIn_.count(t)) continue;
                if (!rt.hostValid) throw Error(Status::RuntimeError, "boundary input without host data: " + g_.desc(t).name);
                if (!staging_.count(t)) staging_[t] = std::make_shared<DevBuf>((size_t) numElements(g_.desc(t).shape) * 4);
                check(vkhip_memcpy_h2d(staging_[t]->ptr, rt.host.f32(), (size_t) rt.elems() * 4, stream_), "input upload");
            }
            launch(profile);
            // a dma-buf output is complete when the run returns: the caller reads the buffer next
            if (!extOut_.empty()) check(vkhip_stream_sync(stream_), "sync (dma-buf output)");
            for (TensorId t: boundaryOutputs) {
                RtTensor &rt = ctx.t(t);
                rt.shape       = g_.desc(t).shape;
                rt.deviceValid = true;
                rt.hostValid   = false;
                rt.deviceFormat = TensorFormat::NC4HW4;
                rt.deviceDtype  = DType::Float16;
            }
            if (profile) {
                check(vkhip_stream_sync(stream_), "profile sync");
                auto t1 = std::chrono::high_resolution_clock::now();
                for (size_t k = 0; k < ops_.size(); ++k) {
                    OpRecord r;
                    r.name    = ops_[k]->name;
                    r.type    = ops_[k]->type;
                    r.backend = "HIP";
                    float ms  = 0;
                    vkhip_event_elapsed_ms(events_[2 * k], events_[2 * k + 1], &ms);
                    r.gpuMs   = ms / cfg_.profileReps;
                    r.flops   = ops_[k]->flops;
                    r.bytesIO = ops_[k]->bytes;
                    r.cpuMs   = std::chrono::duration<double, std::milli>(t1 - t0).count() / (double) ops_.size();
                    ctx.profiler->add(r);
                }
            }
        }

        void HipSegment::download(TensorId t, float *dst) {
            check(vkhip_stream_sync(stream_), "sync");
            auto it = outStaging_.find(t);
            if (it == outStaging_.end()) throw Error(Status::RuntimeError, "not a boundary output of this segment");
            check(vkhip_memcpy_d2h(dst, it->second->ptr, (size_t) numElements(g_.desc(t).shape) * 4, stream_), "output download");
        }

        std::string HipSegment::describe() const {
            std::string s;
            for (size_t k = 0; k < ops_.size(); ++k) {
                s += ops_[k]->name + " [" + ops_[k]->kind + "] " + ops_[k]->describe();
                if (useSide_ && opStream_[k] == 1 && !markers_) s += " (side stream)";
                char fb[64];
                std::snprintf(fb, sizeof fb, " {flops=%.6g bytes=%lld}", ops_[k]->flops, (long long) ops_[k]->bytes);
                s += fb;
                s += "\n";
            }
            return s;
        }

        // ------------------------------------------------------------ backend
        bool HipBackend::available() const { return vkhip_available() == 1; }

        void HipBackend::configure(const Config &cfg) {
            disabled_ = cfg.disableVkOps;
            high_     = cfg.precision == Precision::High;
        }

        bool HipBackend::supports(OpType t, DType) const {
            if (high_) return false; // fp32 storage tier is not part of this backend
            if (!disabled_.empty() && disabled_.find(opTypeName(t)) != std::string::npos) return false;
            switch (t) {
                case OpType::Conv: case OpType::FusedDwPw: case OpType::FusedSE: case OpType::Gemm: case OpType::Add: case OpType::Binary:
                case OpType::Unary: case OpType::Relu: case OpType::Clip: case OpType::GlobalAvgPool: case OpType::MaxPool:
                case OpType::Concat: case OpType::Split: case OpType::Resize: case OpType::Flatten: case OpType::Reshape:
                case OpType::Identity: case OpType::Squeeze: case OpType::Unsqueeze: case OpType::ConvertLayout:
                    return true;
                default: return false;
            }
        }

        bool HipBackend::supportsNode(const Graph &g, const Node &nd, DType dt) const {
            if (!supports(nd.type, dt)) return false;
            for (TensorId t: nd.inputs)
                if (t != kNoTensor && !g.isInitializer(t) && g.desc(t).shape.empty()) return false;
            switch (nd.type) {
                case OpType::Conv: {
                    if (nd.inputs.size() < 2 || !g.isInitializer(nd.inputs[1])) return false;
                    const Shape &w = g.desc(nd.inputs[1]).shape;
                    NCHW         x = NCHW::from(g.desc(nd.inputs[0]).shape);
                    int64_t      grp = nd.attr.geti("group", 1);
                    return w.size() == 4 && (grp == 1 || (grp == x.c && w[0] == x.c && w[1] == 1));
                }
                case OpType::FusedDwPw: return g.desc(nd.inputs[0]).shape.size() == 4 && g.desc(nd.inputs[0]).shape[1] <= 1024;
                case OpType::FusedSE: {
                    const Shape &f = g.desc(nd.inputs[0]).shape, &w1 = g.desc(nd.inputs[1]).shape;
                    return f.size() == 4 && f[1] <= 1024 && !w1.empty() && w1[0] <= 256;
                }
                case OpType::Gemm: return nd.inputs.size() >= 2 && g.isInitializer(nd.inputs[1]) && !nd.attr.geti("transA", 0);
                case OpType::Add: return nd.inputs.size() == 2 && g.desc(nd.inputs[0]).shape == g.desc(nd.inputs[1]).shape;
                case OpType::Binary: {
                    if (nd.inputs.size() != 2) return false;
                    const Shape &a = g.desc(nd.inputs[0]).shape, &b = g.desc(nd.inputs[1]).shape;
                    if (a == b) return nd.subOp >= 0 && nd.subOp != (int) BinaryType::Pow;
                    return nd.subOp == (int) BinaryType::Mul && a.size() == 4 && b.size() == 4 && a[0] == b[0] && a[1] == b[1] &&
                           (a[2] * a[3] == 1 || b[2] * b[3] == 1);
                }
                case OpType::Unary: {
                    UnaryType u = (UnaryType) nd.subOp;
                    return u == UnaryType::Sigmoid || u == UnaryType::HardSwish || u == UnaryType::HardSigmoid || u == UnaryType::Relu || u == UnaryType::SiLU;
                }
                case OpType::Clip:
                    for (size_t i = 1; i < nd.inputs.size() && i < 3; ++i)
                        if (nd.inputs[i] != kNoTensor && !g.isInitializer(nd.inputs[i])) return false;
                    return true;
                case OpType::Flatten: case OpType::Reshape: case OpType::Squeeze: case OpType::Unsqueeze: return isAliasOp(g, nd);
                case OpType::Concat: return g.desc(nd.outputs[0]).shape.size() == 4 && (nd.attr.geti("axis", 0) == 1 || nd.attr.geti("axis", 0) == -3);
                case OpType::Split: return g.desc(nd.inputs[0]).shape.size() == 4 && (nd.attr.geti("axis", 0) == 1 || nd.attr.geti("axis", 0) == -3);
                case OpType::Resize: {
                    const Shape &i = g.desc(nd.inputs[0]).shape, &o = g.desc(nd.outputs[0]).shape;
                    return i.size() == 4 && o.size() == 4 && i[0] == o[0] && i[1] == o[1] && resizeFloorExact(nd, i[2], i[3], o[2], o[3]);
                }
                default: return true;
            }
        }

        std::unique_ptr<Segment> HipBackend::compileSegment(const std::vector<int> &idx, Graph &g, const Config &cfg) {
            // warm start: the tune table of the unified cache file (reference vk_backend.cpp:440-509)
            if (cfg.cachesTuning() && !cfg.cacheFile.empty()) {
                cacheFile_ = cfg.cacheFile;
                TuneCache::instance().load(cacheFile_, cfg.cachesWeights());
            }
            auto s     = std::make_unique<HipSegment>(idx, g, cfg);
            s->backend = this;
            segs_.push_back(s.get());
            return s;
        }

        // Writes the tune table back when it changed (reference saveCaches, vk_backend.cpp:510-545;
        // an unchanged warm session leaves the file untouched).
        void HipBackend::finalize() {
            if (!cacheFile_.empty() && TuneCache::instance().save(cacheFile_))
                throw Error(Status::RuntimeError, "cannot write cache file " + cacheFile_);
        }

        void HipBackend::toHost(RtTensor &rt, ExecContext &) {
            if (rt.hostValid) return;
            for (HipSegment *s: segs_)
                if (s->ownsOutput(rt.id)) {
                    rt.host.resizeElems(rt.elems(), DType::Float32);
                    rt.dtype = DType::Float32;
                    s->download(rt.id, rt.host.f32());
                    rt.hostValid = true;
                    return;
                }
            throw Error(Status::RuntimeError, "tensor has no host data and no HIP segment owns it");
        }

        const float *HipSegment::deviceOutput(TensorId t) const {
            auto it = outStaging_.find(t);
            return it == outStaging_.end() ? nullptr : (const float *) it->second->ptr;
        }

        bool HipSegment::ownsOutput(TensorId t) const { return outStaging_.count(t) > 0; }

    } // namespace hipbe

    using hipbe::HipBackend;
    VKNN_REGISTER_BACKEND(BackendKind::Hip, HipBackend);

} // namespace vknn
