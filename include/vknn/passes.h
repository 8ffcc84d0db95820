// Graph passes on the NCHW IR that produce the fused conv nodes the HIP kernels execute. Mirrors the
// reference pass declarations (src/import/passes.h:6-49) for the conv path: shape inference, BN
// folding, activation / residual / swish fusion, the SE and depthwise+project fusions, identity
// elimination, and the standard pipeline.
#pragma once
#include "vknn/graph.h"

namespace vknn {

    void foldConstantNodes(Graph &g);
    void inferShapes(Graph &g, int64_t batch = 1);
    void eliminateIdentity(Graph &g);
    void eliminateDeadNodes(Graph &g);
    void foldBatchNorm(Graph &g);
    void fuseActivations(Graph &g);
    void fuseResidualAdd(Graph &g);
    void fuseSwish(Graph &g);
    void fuseSqueezeExcite(Graph &g);
    void fuseDwPw(Graph &g);
    void rewireTensor(Graph &g, TensorId from, TensorId to);

    struct PassOptions {
        int64_t batch               = 1;
        bool    fuseSwish           = true;
        bool    fuseSqueezeExcite   = false;
        bool    fuseDwPw            = false;
        bool    fusePointwiseChains = true; // accepted for source compatibility; the HIP epilogues fuse instead
        bool    dumpBig             = false;
    };

    void runStandardPasses(Graph &g, const PassOptions &opt = {});

} // namespace vknn
