// Core value types of the vknn API, restated for the HIP build: status/error, shapes, tensor ids,
// element types and the host fp16 codec, tensor formats, activation/op codes, attributes, the IR
// node and the tensor descriptor. Names, enumerator values and field meanings follow the reference
// headers so code written against vknn compiles unchanged:
//   status.h:5-37, error.h:9-20, shape.h:7-31, tensor_id.h:5-8, dtype.h:9-157,
//   tensor_format_enum.h:6-30, act_type.h:8, op_type.h:9-62, unary_type.h:11-33,
//   binary_type.h:8, attr.h:8-20, attributes.h:9-38, node.h:13-33, tensor_desc.h:9-26,
//   host_buffer.h:9-27, nchw.h:11-58.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace vknn {

    // ------------------------------------------------------------------ status / error
    enum class Status { Ok = 0, InvalidArgument, Unsupported, NotFound, RuntimeError, DeviceLost, IoError };

    inline const char *statusStr(Status s) {
        static const char *names[] = {"Ok", "InvalidArgument", "Unsupported", "NotFound", "RuntimeError", "DeviceLost", "IoError"};
        int i = (int) s;
        return (i >= 0 && i < 7) ? names[i] : "?";
    }

    class Error: public std::runtime_error {
      public:
        Error(Status s, const std::string &msg): std::runtime_error(std::string(statusStr(s)) + ": " + msg), status_(s) {}
        Status status() const { return status_; }

      private:
        Status status_;
    };

    // ------------------------------------------------------------------ shapes / ids
    using Shape = std::vector<int64_t>;

    inline int64_t numElements(const Shape &s) {
        if (s.empty()) return 0;
        int64_t n = 1;
        for (int64_t d: s) n *= d;
        return n;
    }
    inline std::string shapeStr(const Shape &s) {
        std::string r = "[";
        for (size_t i = 0; i < s.size(); ++i) r += (i ? "," : "") + std::to_string(s[i]);
        return r + "]";
    }

    using TensorId               = int32_t;
    constexpr TensorId kNoTensor = -1;

    // ------------------------------------------------------------------ element types
    enum class DType : uint8_t { Float32 = 0, Float16 = 1, Int32 = 2, Int8 = 3, UInt8 = 4, Int64 = 5 };

    inline size_t dtypeSize(DType d) {
        switch (d) {
            case DType::Float32: case DType::Int32: return 4;
            case DType::Float16: return 2;
            case DType::Int8: case DType::UInt8: return 1;
            case DType::Int64: return 8;
        }
        return 0;
    }
    inline const char *dtypeStr(DType d) {
        switch (d) {
            case DType::Float32: return "f32";
            case DType::Float16: return "f16";
            case DType::Int32: return "i32";
            case DType::Int8: return "i8";
            case DType::UInt8: return "u8";
            case DType::Int64: return "i64";
        }
        return "?";
    }

    // Host half codec with the exact rounding of the reference's boundary codec (dtype.h:121-157):
    // the 13 dropped mantissa bits round half-away-from-zero on the magnitude (carry may ripple into
    // the exponent, 65520 -> inf); subnormal results round the same way on the shifted-out bit; any
    // exponent below -24 flushes to signed zero; NaN keeps only the quiet bit (payload dropped).
    // The GPU pack kernel implements the same integer recipe so packing is bit-exact.
    using fp16_t = uint16_t;

    inline float halfToFloat(fp16_t h) {
        uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
        uint32_t e    = (h >> 10) & 0x1Fu;
        uint32_t m    = h & 0x3FFu;
        uint32_t bits;
        if (e == 0x1F) {
            bits = sign | 0x7F800000u | (m << 13);
        } else if (e != 0) {
            bits = sign | ((e + 112u) << 23) | (m << 13);
        } else if (m == 0) {
            bits = sign;
        } else {
            // subnormal: normalise the mantissa (value = m * 2^-24)
            int shift = 0;
            while (!(m & 0x400u)) { m <<= 1; ++shift; }
            bits = sign | ((uint32_t) (113 - shift) << 23) | ((m & 0x3FFu) << 13);
        }
        float out;
        std::memcpy(&out, &bits, 4);
        return out;
    }

    inline void halfToFloatBulk(const fp16_t *src, float *dst, int64_t n) {
        for (int64_t i = 0; i < n; ++i) dst[i] = halfToFloat(src[i]);
    }

    inline fp16_t floatToHalf(float v) {
        uint32_t bits;
        std::memcpy(&bits, &v, 4);
        const uint32_t sign = (bits >> 16) & 0x8000u;
        const uint32_t fexp = (bits >> 23) & 0xFFu;
        const uint32_t man  = bits & 0x7FFFFFu;
        if (fexp == 0xFF) return (fp16_t) (sign | 0x7C00u | (man ? 0x200u : 0u));
        const int32_t e = (int32_t) fexp - 112; // rebias 127 -> 15
        if (e >= 31) return (fp16_t) (sign | 0x7C00u);
        if (e > 0) {
            uint32_t h = sign | ((uint32_t) e << 10) | (man >> 13);
            return (fp16_t) (h + ((man >> 12) & 1u));
        }
        if (e < -10) return (fp16_t) sign;
        const uint32_t full = man | 0x800000u;
        const uint32_t sh   = (uint32_t) (14 - e);
        return (fp16_t) (sign | ((full >> sh) + ((full >> (sh - 1)) & 1u)));
    }

    // ------------------------------------------------------------------ layouts
    enum class TensorFormat : uint8_t { NCHW = 0, NHWC = 1, NC4HW4 = 2, Auto = 3, Unknown = 255 };

    inline const char *formatStr(TensorFormat f) {
        switch (f) {
            case TensorFormat::NCHW: return "NCHW";
            case TensorFormat::NHWC: return "NHWC";
            case TensorFormat::NC4HW4: return "NC4HW4";
            case TensorFormat::Auto: return "Auto";
            default: return "?";
        }
    }

    // Shape viewed as NCHW. Rank > 4 folds the leading dims into N; rank 3 is (N,C,L,1); rank 2 is
    // (N,C,1,1); rank 1 is (1,C,1,1).
    struct NCHW {
        int64_t n = 1, c = 1, h = 1, w = 1;
        static NCHW from(const Shape &s) {
            NCHW r;
            const size_t k = s.size();
            if (k >= 4) {
                r.w = s[k - 1];
                r.h = s[k - 2];
                r.c = s[k - 3];
                r.n = 1;
                for (size_t i = 0; i + 3 < k; ++i) r.n *= s[i];
            } else if (k == 3) {
                r.n = s[0]; r.c = s[1]; r.h = s[2];
            } else if (k == 2) {
                r.n = s[0]; r.c = s[1];
            } else if (k == 1) {
                r.c = s[0];
            }
            return r;
        }
        int64_t elems() const { return n * c * h * w; }
    };

    inline int64_t cBlocks(int64_t c) { return (c + 3) / 4; }

    inline int64_t formatElems(TensorFormat fmt, const NCHW &x) {
        return fmt == TensorFormat::NC4HW4 ? x.n * cBlocks(x.c) * 4 * x.h * x.w : x.elems();
    }

    // ------------------------------------------------------------------ op codes
    enum class ActType : int32_t { None = 0, Relu = 1, Relu6 = 2, Clip = 3, HardSwish = 4, SiLU = 5 };

    enum class OpType {
        Unknown = 0, Conv, ConvTranspose, Clip, Relu, Add, GlobalAvgPool, AvgPool, MaxPool, Gemm, MatMul, Einsum,
        Reshape, Expand, Tile, Squeeze, Flatten, Softmax, LayerNorm, BatchNorm, Concat, Pad, Identity, Constant,
        Shape, Gather, Unsqueeze, Unary, Binary, PRelu, Resize, GridSample, Transpose, Slice, Reduce, DepthToSpace,
        Cast, Split, Where, Equal, Greater, GreaterEqual, ConstantOfShape, EyeLike, ScatterND, FusedSE, FusedDwPw,
        FusedPointwise, ConvertLayout, ConvertDtype,
    };
    const char *opTypeName(OpType t);

    enum class UnaryType : int32_t {
        Invalid = -1, Sigmoid = 0, Tanh = 1, HardSwish = 2, HardSigmoid = 3, LeakyRelu = 4, Elu = 5, Abs = 6,
        Neg = 7, Exp = 8, Log = 9, Sqrt = 10, Floor = 11, Ceil = 12, Relu = 13, SiLU = 14, Erf = 15, Cos = 16,
        Sin = 17, Reciprocal = 18, Softplus = 19
    };
    enum class BinaryType : int32_t { Invalid = -1, Mul = 0, Sub = 1, Div = 2, Max = 3, Min = 4, Pow = 5, Add = 6 };

    // ------------------------------------------------------------------ attributes / node
    struct Attr {
        enum Kind { None, Int, Float, Ints, Floats, String } kind = None;
        int64_t              i = 0;
        float                f = 0;
        std::vector<int64_t> ints;
        std::vector<float>   floats;
        std::string          str;
        std::vector<int64_t> shape;
    };

    struct Attributes {
        std::map<std::string, Attr> map;
        bool    has(const std::string &k) const { return map.count(k) > 0; }
        int64_t geti(const std::string &k, int64_t d = 0) const {
            auto it = map.find(k);
            return it == map.end() ? d : it->second.i;
        }
        float getf(const std::string &k, float d = 0) const {
            auto it = map.find(k);
            return it == map.end() ? d : it->second.f;
        }
        const std::vector<int64_t> &getints(const std::string &k) const {
            static const std::vector<int64_t> none;
            auto it = map.find(k);
            return it == map.end() ? none : it->second.ints;
        }
        const std::vector<float> &getfloats(const std::string &k) const {
            static const std::vector<float> none;
            auto it = map.find(k);
            return it == map.end() ? none : it->second.floats;
        }
        std::string gets(const std::string &k, const std::string &d = "") const {
            auto it = map.find(k);
            return it == map.end() ? d : it->second.str;
        }
    };

    struct Node {
        OpType                type = OpType::Unknown;
        std::string           name;
        std::vector<TensorId> inputs;
        std::vector<TensorId> outputs;
        Attributes            attr;
        ActType               fusedAct = ActType::None;
        float                 actLo = 0, actHi = 0;
        int32_t               subOp         = 0;
        TensorId              fusedResidual = kNoTensor;
        TensorId              fusedBias     = kNoTensor;
    };

    struct TensorDesc {
        std::string  name;
        Shape        shape;
        DType        dtype         = DType::Float32;
        TensorFormat format        = TensorFormat::NCHW;
        bool         isInput       = false;
        bool         isOutput      = false;
        bool         isInitializer = false;
        bool         gpuFlat       = false;
        bool         storeFp32     = false;
    };

    struct HostBuffer {
        std::vector<uint8_t> bytes;
        void           resizeElems(int64_t n, DType dt) { bytes.assign((size_t) n * dtypeSize(dt), 0); }
        float         *f32() { return reinterpret_cast<float *>(bytes.data()); }
        const float   *f32() const { return reinterpret_cast<const float *>(bytes.data()); }
        int64_t       *i64() { return reinterpret_cast<int64_t *>(bytes.data()); }
        const int64_t *i64() const { return reinterpret_cast<const int64_t *>(bytes.data()); }
    };

} // namespace vknn
