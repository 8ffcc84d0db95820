// Runtime tensor: host NCHW fp32 data and/or a backend-owned device copy with validity flags.
// Mirrors the reference RtTensor (rt_tensor.h:15-43); DeviceStorage stays an opaque type that the
// one linked device backend defines (device_storage.h:8).
#pragma once
#include "vknn/types.h"
#include <memory>

namespace vknn {

    struct DeviceStorage;

    struct RtTensor {
        TensorId id    = kNoTensor;
        Shape    shape;
        DType    dtype = DType::Float32;

        HostBuffer host;
        bool       hostValid = false;

        std::shared_ptr<DeviceStorage> device;
        TensorFormat                   deviceFormat = TensorFormat::Unknown;
        DType                          deviceDtype  = DType::Float32;
        bool                           deviceValid  = false;
        int                            dmaBufFd     = -1;
        TensorFormat                   dmaBufFormat = TensorFormat::NCHW;
        DType                          dmaBufDtype  = DType::Float32;

        int64_t elems() const { return numElements(shape); }
        void    allocHost() {
            host.resizeElems(elems(), dtype);
            hostValid = true;
        }
    };

} // namespace vknn
