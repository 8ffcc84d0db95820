// Persistent autotune table in the reference's unified cache-file container.
//
// File layout (reference src/backend/vulkan/vk_backend.cpp:445-545 for the container, :30-126 for
// the weight/tune section):
//   "VKNNCAC1" | u32 pipeLen | pipe bytes | u32 wLen | w bytes
//   w = u32 nWeights {u32 klen | key | u32 nfloats | floats}  u32 nTune {u32 klen | key | i32 val}
// The HIP backend has no pipeline cache (its code objects live in libvkhip.so), so it writes
// pipeLen = 0 (a foreign pipeline section is kept verbatim so a rewrite does not drop it). The
// weight section holds the prepacked conv blobs (the bytes vkhip_conv_pack_weights writes, stored
// as ceil(bytes / 4) floats) when the file is loaded with keepWeights (CacheMode::Full, as the
// reference's WeightCache retains them only then); the tune table is always kept. Keys are
// namespaced by a per-GPU tag ("<tag>/<signature>"), like the reference's gpuTag, so entries from
// other devices never apply.
#pragma once
#include <atomic>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace vknn {
    namespace hipbe {

        class TuneCache {
          public:
            static TuneCache &instance();

            // Merge the tune entries of `path` (once per path; absent or unrecognised files are
            // ignored, as in the reference). Returns the number of entries read.
            int  load(const std::string &path, bool keepWeights = false);
            // Write the table to `path` unless the bytes equal what the file already holds.
            // Returns 0 on success (written or unchanged), -1 when the file cannot be written.
            int  save(const std::string &path);
            bool get(const std::string &key, int32_t &val);
            void put(const std::string &key, int32_t val);
            void clear();
            size_t size();
            // Lookups that found / did not find an entry since the last clear().
            int64_t hits() const { return hits_.load(); }
            int64_t misses() const { return misses_.load(); }

            // Prepacked weight blobs. getWeights succeeds only for a blob of exactly `bytes` bytes.
            bool   getWeights(const std::string &key, size_t bytes, std::vector<uint8_t> &out);
            void   putWeights(const std::string &key, const std::vector<uint8_t> &blob);
            size_t weightCount();
            int64_t weightHits() const { return wHits_.load(); }
            int64_t weightMisses() const { return wMisses_.load(); }

            // Parse a container's tune entries (and its pipeline bytes, and its weight blobs when
            // `weights` is given) without touching the table.
            static bool parse(const std::vector<uint8_t> &bytes, std::map<std::string, int32_t> &tune, std::vector<char> *pipe,
                              std::map<std::string, std::vector<uint8_t>> *weights = nullptr);

          private:
            std::vector<uint8_t> serialize(); // caller holds mu_
            std::mutex                          mu_;
            std::map<std::string, int32_t>      tune_;
            std::map<std::string, bool>         loaded_, wloaded_;
            std::map<std::string, std::vector<uint8_t>> weights_;
            std::atomic<int64_t>                wHits_ {0}, wMisses_ {0};
            std::map<std::string, std::vector<uint8_t>> fileBytes_;
            std::vector<char>                   pipe_;
            std::atomic<int64_t>                hits_ {0}, misses_ {0};
        };

        // The per-GPU key namespace: "hip-<arch>-<CUs>cu".
        std::string gpuTag();

    } // namespace hipbe
} // namespace vknn
