// Forwarding header: TensorDesc/HostBuffer live in types.h, RtTensor in rt_tensor.h.
#pragma once
#include "vknn/types.h"
#include "vknn/rt_tensor.h"
