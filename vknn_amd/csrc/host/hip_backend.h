// HIP backend classes (internal header of the vknn host library).
#pragma once
#include "vkhip.h"
#include "vknn/backend.h"
#include <map>
#include <set>
#include <memory>
#include <string>
#include <vector>

namespace vknn {
    namespace hipbe {

        void check(int rc, const std::string &what);

        // RAII device allocation through the vkhip ABI.
        struct DevBuf {
            void  *ptr   = nullptr;
            size_t bytes = 0;
            explicit DevBuf(size_t n);
            ~DevBuf();
            DevBuf(const DevBuf &)            = delete;
            DevBuf &operator=(const DevBuf &) = delete;
        };
        std::shared_ptr<DevBuf> upload(const void *host, size_t bytes);
        size_t                  nc4Bytes(const Shape &s);

        class HipSegment;

        struct SegEnv {
            const Graph  *graph   = nullptr;
            const Config *config  = nullptr;
            bool          tunable = true;
            HipSegment   *seg     = nullptr;
            void         *dev(TensorId t);
            // channel blocks per image of the buffer t lives in when t is a view into a wider
            // tensor (a slice of an in-place channel concat or split), 0 when t is dense
            int64_t       pstride(TensorId t);
        };

        // One HIP operator: prepare = classify + prepack/upload weights (+ autotune); record =
        // append its launches to the segment's stream.
        struct HipOp {
            virtual ~HipOp()                                  = default;
            virtual void        prepare(const Node &, SegEnv &) = 0;
            virtual void        record(SegEnv &, vkhip_stream_t) = 0;
            virtual std::string describe() const { return ""; }
            // In-graph plan refinement: alternative plans of the op (0 or 1: nothing to refine),
            // switching to one of them, and keeping one (which also records it as the op's pick).
            virtual int  candidates() const { return 0; }
            virtual void useCandidate(int) {}
            virtual void commitCandidate(int) {}
            virtual std::string planKey() const { return {}; } // tune-table key of the op's plan ("" if none)
            std::string         name, kind;
            OpType              type  = OpType::Unknown;
            double              flops = 0;
            int64_t             bytes = 0;
        };

        class HipSegment: public Segment {
          public:
            HipSegment(const std::vector<int> &idx, Graph &g, const Config &cfg);
            ~HipSegment() override;
            void        run(ExecContext &ctx) override;
            void       *dev(TensorId t);
            int64_t     pstride(TensorId t) const;
            // Read a boundary input straight from device memory (NCHW fp32) instead of host data.
            void        bindDeviceInput(TensorId t, const float *devNchw);
            // Same, from a declared layout (0 NCHW, 1 NHWC, 2 NC4HW4) and dtype (fp16 or fp32),
            // converted by the boundary converter (fp32 -> fp16 rounds to nearest even), as the
            // reference does for a declared-format dma-buf input.
            void        bindDeviceInputAs(TensorId t, const void *dev, int fmt, bool f16);
            // Copy a boundary output (already unpacked to NCHW fp32 on the device) to the host.
            void        download(TensorId t, float *dst);
            const float *deviceOutput(TensorId t) const;
            bool        ownsOutput(TensorId t) const;
            vkhip_stream_t stream() const { return stream_; }
            std::string describe() const;
            const std::vector<std::unique_ptr<HipOp>> &ops() const { return ops_; }

          private:
            TensorId resolve(TensorId t) const;
            void     planStreams(const std::vector<std::vector<TensorId>> &ins, const std::vector<std::vector<TensorId>> &outs);
            void     refinePlans();
            void     recordAll(bool timed);
            void     launch(bool profile);
            void     dropGraph();
            // dma-buf boundaries (IOTensor.dmaBufFd): import the fd of tensor t, reusing the last
            // import while the same buffer and size come back; returns the device address
            void    *importDmaBuf(TensorId t, int fd, size_t bytes);
            void     bindDmaBufs(ExecContext &ctx);

            Graph                                         &g_;
            const Config                                  &cfg_;
            SegEnv                                         env_;
            vkhip_stream_t                                 stream_ = nullptr;
            vkhip_graph_t                                  graph_  = nullptr;
            int                                            replay_ = 0;
            std::vector<std::unique_ptr<HipOp>>            ops_;
            std::map<TensorId, std::shared_ptr<DevBuf>>    bufs_, staging_, outStaging_;
            std::map<TensorId, TensorId>                   alias_;
            // In-place channel concat / split: tensor -> (the tensor it lives in, its first channel
            // block there); only the outermost tensor of a chain owns a buffer.
            struct Place {
                TensorId parent;
                int64_t  off;
            };
            std::map<TensorId, Place>                      place_;
            void planViews(const std::vector<int> &idx, const std::set<int> &noWrite, const std::set<int> &noRead);
            std::set<int>                                  viewCats_, viewSplits_; // concat / split nodes done in place
            std::map<TensorId, const float *>              extIn_;
            std::map<TensorId, std::pair<int, bool>>       extFmt_; // declared (layout, fp16) of a bound input
            struct DmaImport {
                uint64_t     id    = 0; // st_dev:st_ino of the fd's file, or 0
                int          fd    = -1;
                size_t       bytes = 0;
                vkhip_dmabuf h     = nullptr;
                void        *ptr   = nullptr;
            };
            std::map<TensorId, DmaImport>                  dma_;
            std::set<TensorId>                             dmaIn_;  // inputs bound to an imported dma-buf
            std::map<TensorId, std::pair<void *, std::pair<int, bool>>> extOut_; // outputs written to a dma-buf
            std::vector<vkhip_event_t>                     events_;
            // Two-stream schedule (see planStreams): per op its stream (0 main, 1 side), the ops
            // whose completion events it waits for (-1 = the boundary pack), and whether its own
            // completion event is needed.
            vkhip_stream_t                                 side_ = nullptr;
            std::vector<int>                               opStream_;
            std::vector<std::vector<int>>                  opWaits_;
            std::vector<char>                              opSignals_;
            std::vector<vkhip_event_t>                     opEvents_;
            vkhip_event_t                                  packEvent_ = nullptr, joinEvent_ = nullptr;
            bool                                           useSide_ = false;
            // VKNN_HIP_OP_MARKERS=1: an empty marker dispatch before every op, all ops on one
            // stream, so a kernel trace splits into per-op launches (vknn_amd/prof_summary.py layers)
            bool                                           markers_ = false;
        };

        class HipBackend: public Backend {
          public:
            BackendKind kind() const override { return BackendKind::Hip; }
            const char *name() const override { return "HIP"; }
            bool        available() const override;
            void        configure(const Config &cfg) override;
            bool        supports(OpType t, DType dt) const override;
            bool        supportsNode(const Graph &g, const Node &nd, DType dt) const override;
            void        toHost(RtTensor &rt, ExecContext &ctx) override;
            std::unique_ptr<Segment> compileSegment(const std::vector<int> &idx, Graph &g, const Config &cfg) override;
            void        finalize() override;

          private:
            std::string               disabled_;
            bool                      high_ = false;
            std::vector<HipSegment *> segs_;
            std::string               cacheFile_;
        };

    } // namespace hipbe
} // namespace vknn
