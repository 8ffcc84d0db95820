// Runtime configuration. Mirrors the reference Config (config_struct.h:13-94), BackendKind
// (backend_kind.h:7), Precision (precision.h:11), Hint/Mode (hint.h:8-26) and CacheMode
// (cache_mode.h:10). BackendKind gains one enumerator, Hip, for the MI355X backend; the existing
// values keep their numbers.
#pragma once
#include "vknn/types.h"
#include <string>
#include <vector>

namespace vknn {

    enum class BackendKind { Vulkan = 0, Cpu = 1, Hip = 2 };
    const char *backendName(BackendKind k);
    // "vulkan"/"gpu" -> Vulkan, "hip"/"rocm" -> Hip, anything else -> Cpu (reference config.cpp:19-25
    // maps unknown strings to CPU; "hip" is the one new spelling).
    BackendKind backendFromStr(const std::string &s);

    enum class Precision { Low = 0, Normal = 1, High = 2 };
    Precision precisionFromStr(const std::string &s);

    enum class CacheMode { Off = 0, Tune = 1, Full = 2 };

    enum class Hint { Winograd = 0, Tuning = 1, WinogradVariant = 2, WinogradUnit = 3, DirectConv3x3 = 4 };
    enum class Mode {
        Auto = 0, On = 1, Off = 2,
        NoTune = 0, Fast = 1, Thorough = 2,
        TiledGemm = 0, Fused = 1, FusedSplit = 2, FullyFused = 3, SubgroupGemm = 4,
        F23 = 0, F43 = 4,
        DirectAuto = 0, RegisterTiled = 1, LdsHalo = 2,
    };
    Mode winogradFromStr(const std::string &s);
    Mode tuningFromStr(const std::string &s);

    struct Config {
        BackendKind              backend          = BackendKind::Hip;
        std::vector<BackendKind> fallback         = {};
        // The HIP build ships no CPU backend: a node the HIP backend cannot run is an Unsupported
        // error, never a silent host fallback. A host backend registered by the caller (the
        // tests' oracle/test_cpu_backend.cpp) takes such nodes only when this is set.
        bool                     allowCpuFallback = false;

        Precision precision = Precision::Low;

        std::string cacheFile;
        std::string cacheDir  = "";
        CacheMode   cacheMode = CacheMode::Full;
        bool        cachesPipeline() const { return cacheMode != CacheMode::Off; }
        bool        cachesTuning() const { return cacheMode != CacheMode::Off; }
        bool        cachesWeights() const { return cacheMode == CacheMode::Full; }

        bool        freeWeightsAfterUpload = true;
        int         maxSubmitNodes         = 500;
        bool        noFlatOps              = false;
        bool        timing                 = false;
        bool        debugSegments          = false;
        std::string disableVkOps;
        std::string dumpTensors;
        std::string fp32Tensors;
        bool        profile      = false;
        int         verbosity    = 1;
        bool        layerDump    = false;
        std::string layerDumpDir = "";

        // HIP backend: capture each segment's launch sequence into a HIP graph after the first run
        // and replay it (the analogue of the reference's pre-recorded command buffer).
        bool hipGraphs = true;
        // HIP backend: issue a node whose inputs do not depend on the node recorded just before it
        // (e.g. a residual block's projection shortcut) on a second stream, joined back by events,
        // so independent branches of a segment overlap. false keeps one in-order stream.
        bool hipBranches = true;
        // HIP backend, profiling only: launches per op between its two timing events (the op's
        // time is their average; amortizes the event overhead on short kernels).
        int profileReps = 1;
        // Fusion passes the reference exposes only as compiler flags (passes.h:33-40).
        bool fuseDwPw          = false;
        bool fuseSqueezeExcite = false;
        // HIP backend: run the squeeze-excite fusion (fuseSqueezeExcite) even when it is off, since
        // on this backend the fused op (pool folded into the depthwise conv, two FC launches) is
        // faster than the pool, two 1x1 convs and the gate (MobileNetV3-Large b128: 1.073 ->
        // 1.016 ms). The fused op keeps FC1's output in fp32 where the unfused chain rounds it to
        // fp16, so results differ within the fp16 parity tolerance. Option key "hip_auto_se";
        // VKNN_HIP_AUTO_SE=0 also turns it off.
        bool hipAutoSE = true;
        // HIP backend: likewise the depthwise + pointwise fusion (fuseDwPw) even when it is off; the
        // backend then times the fused kernel against the two convs per op and keeps the faster
        // (MobileNetV2 block b128 0.166 -> 0.142 ms, MobileNetV3-Large b128 1.018 -> 1.006 ms).
        // Option key "hip_auto_dwpw"; VKNN_HIP_AUTO_DWPW=0 also turns it off.
        bool hipAutoDwPw = true;

        std::vector<int> hints;
        void setHint(Hint h, int value) {
            if ((int) h >= (int) hints.size()) hints.resize((int) h + 1, 0);
            hints[(int) h] = value;
        }
        void setHint(Hint h, Mode v) { setHint(h, (int) v); }
        int  hint(Hint h, int dflt = 0) const { return (int) h < (int) hints.size() ? hints[(int) h] : dflt; }
    };

} // namespace vknn
