// Programmatic graphs for the benchmark configurations of the fused conv path, written only against
// the vknn graph API (Graph / TensorDesc / Node / Attr / HostBuffer), so the same source builds
// against this repository's headers and against the reference's own headers.
//
// Weights come from an in-repo PRNG (splitmix64 + Box-Muller), so every build on every machine
// produces the same graph for the same (name, batch, seed).
#pragma once
#include "vknn/graph.h"
#include <cstdint>
#include <string>
#include <vector>

namespace vknn_zoo {

    // Names: "conv3x3_bn_relu" (config 0), "mnv2_block" (config 1), "resnet50" (config 2),
    // "mobilenetv3_large" (config 3), "yolov8n" (config 4), plus small test graphs
    // "conv_tiny", "resnet_tiny", "mnv3_tiny", "yolo_tiny" with the same op mix at small sizes.
    vknn::Graph build(const std::string &name, int64_t batch, uint64_t seed);
    // Input and output shapes of a named model (for buffer sizing).
    bool io_shapes(const std::string &name, int64_t batch, std::vector<int64_t> &in, std::vector<int64_t> &out);
    // Algorithmic conv FLOPs per image of a named model (2*Cout*Cin/g*KH*KW*OH*OW summed, FC included).
    double conv_flops_per_image(const std::string &name);

    // Deterministic generator used for weights (and available to tests for inputs).
    struct Rng {
        uint64_t state;
        explicit Rng(uint64_t seed): state(seed * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull) {}
        uint64_t next() {
            uint64_t z = (state += 0x9E3779B97F4A7C15ull);
            z          = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z          = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            return z ^ (z >> 31);
        }
        // uniform in [0, 1) with 24 random bits
        float uniform() { return (float) (next() >> 40) * (1.0f / 16777216.0f); }
        float uniform(float lo, float hi) { return lo + (hi - lo) * uniform(); }
        // standard normal, Box-Muller on two uniforms in (0, 1]
        float normal();
    };

} // namespace vknn_zoo
