// Persistent autotune table (declared in tune_cache.h).
#include "tune_cache.h"
#include "vkhip.h"
#include <cstring>
#include <fstream>
#include <iterator>

namespace vknn {
    namespace hipbe {

        TuneCache &TuneCache::instance() {
            static TuneCache c;
            return c;
        }

        static void wr32(std::vector<uint8_t> &out, uint32_t v) {
            const uint8_t *b = (const uint8_t *) &v;
            out.insert(out.end(), b, b + 4);
        }

        bool TuneCache::parse(const std::vector<uint8_t> &bytes, std::map<std::string, int32_t> &tune, std::vector<char> *pipe,
                              std::map<std::string, std::vector<uint8_t>> *weights) {
            const uint8_t *p = bytes.data();
            const size_t   n = bytes.size();
            if (n < 8 || std::memcmp(p, "VKNNCAC1", 8) != 0) return false;
            size_t off  = 8;
            auto   rd32 = [&](uint32_t &v) {
                if (off + 4 > n) return false;
                std::memcpy(&v, p + off, 4);
                off += 4;
                return true;
            };
            uint32_t pl = 0;
            if (!rd32(pl) || off + pl > n) return false;
            if (pipe) pipe->assign((const char *) p + off, (const char *) p + off + pl);
            off += pl;
            uint32_t wl = 0;
            if (!rd32(wl) || off + wl > n) return true; // container without a weight section
            const size_t end = off + wl;
            auto rdIn = [&](uint32_t &v) { return off + 4 <= end && rd32(v); };
            uint32_t nw = 0;
            if (!rdIn(nw)) return true;
            for (uint32_t i = 0; i < nw; ++i) { // prepacked weight blobs: kept when asked for, else skipped
                uint32_t kl = 0, nf = 0;
                if (!rdIn(kl) || off + kl > end) return true;
                std::string k((const char *) p + off, kl);
                off += kl;
                if (!rdIn(nf) || off + (size_t) nf * 4 > end) return true;
                if (weights) (*weights)[k].assign(p + off, p + off + (size_t) nf * 4);
                off += (size_t) nf * 4;
            }
            uint32_t nt = 0;
            if (!rdIn(nt)) return true;
            for (uint32_t i = 0; i < nt; ++i) {
                uint32_t kl = 0;
                if (!rdIn(kl) || off + kl + 4 > end) return true; // truncated tail: keep what was read
                std::string k((const char *) p + off, kl);
                off += kl;
                int32_t v = 0;
                std::memcpy(&v, p + off, 4);
                off += 4;
                tune[k] = v;
            }
            return true;
        }

        std::vector<uint8_t> TuneCache::serialize() {
            std::vector<uint8_t> w;
            wr32(w, (uint32_t) weights_.size());
            for (auto &kv: weights_) { // blobs as whole floats (zero padded to 4 bytes)
                wr32(w, (uint32_t) kv.first.size());
                w.insert(w.end(), kv.first.begin(), kv.first.end());
                const size_t nf = (kv.second.size() + 3) / 4;
                wr32(w, (uint32_t) nf);
                w.insert(w.end(), kv.second.begin(), kv.second.end());
                w.insert(w.end(), nf * 4 - kv.second.size(), 0);
            }
            wr32(w, (uint32_t) tune_.size());
            for (auto &kv: tune_) {
                wr32(w, (uint32_t) kv.first.size());
                w.insert(w.end(), kv.first.begin(), kv.first.end());
                wr32(w, (uint32_t) kv.second);
            }
            std::vector<uint8_t> out = {'V', 'K', 'N', 'N', 'C', 'A', 'C', '1'};
            wr32(out, (uint32_t) pipe_.size());
            out.insert(out.end(), pipe_.begin(), pipe_.end());
            wr32(out, (uint32_t) w.size());
            out.insert(out.end(), w.begin(), w.end());
            return out;
        }

        int TuneCache::load(const std::string &path, bool keepWeights) {
            std::lock_guard<std::mutex> lk(mu_);
            if (path.empty() || (loaded_[path] && (!keepWeights || wloaded_[path]))) return 0;
            const bool first = !loaded_[path];
            loaded_[path]    = true;
            if (keepWeights) wloaded_[path] = true;
            std::ifstream f(path, std::ios::binary);
            if (!f) return 0;
            std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
            std::map<std::string, int32_t> t;
            std::vector<char>              pipe;
            std::map<std::string, std::vector<uint8_t>> w;
            // the weight section is carried along even when this session does not use it (tune-only
            // mode), so that writing the table back never drops another session's blobs
            if (!parse(bytes, t, &pipe, &w)) return 0; // unrecognised -> regenerate
            for (auto &kv: w) weights_.insert(kv); // blobs packed in this process take precedence
            if (!first) return 0;                 // a later load that only adds the weights
            fileBytes_[path] = bytes;
            if (pipe_.empty()) pipe_ = pipe;
            for (auto &kv: t) tune_.insert(kv); // entries tuned in this process take precedence
            return (int) t.size();
        }

        bool TuneCache::getWeights(const std::string &key, size_t bytes, std::vector<uint8_t> &out) {
            std::lock_guard<std::mutex> lk(mu_);
            auto it = weights_.find(key);
            // stored as whole floats: the blob is the first `bytes` of a (bytes + 3) / 4 float run
            if (it == weights_.end() || (it->second.size() != bytes && it->second.size() != (bytes + 3) / 4 * 4)) {
                ++wMisses_;
                return false;
            }
            ++wHits_;
            out.assign(it->second.begin(), it->second.begin() + bytes);
            return true;
        }

        void TuneCache::putWeights(const std::string &key, const std::vector<uint8_t> &blob) {
            std::lock_guard<std::mutex> lk(mu_);
            weights_[key] = blob;
        }

        size_t TuneCache::weightCount() {
            std::lock_guard<std::mutex> lk(mu_);
            return weights_.size();
        }

        int TuneCache::save(const std::string &path) {
            std::lock_guard<std::mutex> lk(mu_);
            if (path.empty()) return 0;
            std::vector<uint8_t> out = serialize();
            auto it = fileBytes_.find(path);
            if (it != fileBytes_.end() && it->second == out) return 0; // unchanged: leave the file alone
            std::ofstream f(path, std::ios::binary | std::ios::trunc);
            if (!f) return -1;
            f.write((const char *) out.data(), (std::streamsize) out.size());
            if (!f) return -1;
            fileBytes_[path] = out;
            return 0;
        }

        bool TuneCache::get(const std::string &key, int32_t &val) {
            std::lock_guard<std::mutex> lk(mu_);
            auto it = tune_.find(key);
            if (it == tune_.end()) {
                ++misses_;
                return false;
            }
            ++hits_;
            val = it->second;
            return true;
        }

        void TuneCache::put(const std::string &key, int32_t val) {
            std::lock_guard<std::mutex> lk(mu_);
            tune_[key] = val;
        }

        void TuneCache::clear() {
            std::lock_guard<std::mutex> lk(mu_);
            tune_.clear();
            weights_.clear();
            loaded_.clear();
            wloaded_.clear();
            wHits_ = wMisses_ = 0;
            fileBytes_.clear();
            pipe_.clear();
            hits_ = misses_ = 0;
        }

        size_t TuneCache::size() {
            std::lock_guard<std::mutex> lk(mu_);
            return tune_.size();
        }

        static std::string makeGpuTag() {
            char name[128] = {0};
            int  cus = 0, clk = 0;
            size_t hbm = 0;
            if (vkhip_device_info(name, sizeof(name), &cus, &clk, &hbm)) return "hip-unknown";
            // name is "<marketing name> (<gcnArchName>)"; keep the arch up to its feature suffix
            std::string n(name), arch = n;
            size_t      lp = n.find('(');
            if (lp != std::string::npos) arch = n.substr(lp + 1);
            arch = arch.substr(0, arch.find_first_of(":)"));
            return "hip-" + arch + "-" + std::to_string(cus) + "cu";
        }

        std::string gpuTag() {
            static const std::string tag = makeGpuTag();
            return tag;
        }

    } // namespace hipbe
} // namespace vknn
