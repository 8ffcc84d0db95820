// Top-level facade (reference include/vknn/runtime.h:10-35): load a model file with its unified
// cache file: a pre-optimized ".vxm" model, or any other path as an ONNX model.
#pragma once
#include "vknn/session.h"
#include <memory>
#include <string>

namespace vknn {

    class Runtime {
      public:
        // `cacheFile` empty -> "<model path without extension>.cache" next to the model.
        static std::unique_ptr<Session> load(const std::string &path, const Config &cfg = {}, const std::string &cacheFile = "") {
            Config c    = cfg;
            c.cacheFile = cacheFile.empty() ? defaultCacheFile(path) : cacheFile;
            const bool vxm = path.size() >= 4 && path.compare(path.size() - 4, 4, ".vxm") == 0;
            return vxm ? Session::createFromVxm(path, c) : Session::createFromOnnx(path, c);
        }
        static std::string defaultCacheFile(const std::string &modelPath) {
            const size_t slash = modelPath.find_last_of("/\\"), dot = modelPath.find_last_of('.');
            const bool   ext   = dot != std::string::npos && (slash == std::string::npos || dot > slash);
            return (ext ? modelPath.substr(0, dot) : modelPath) + ".cache";
        }
    };

} // namespace vknn
