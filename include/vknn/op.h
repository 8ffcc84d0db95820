// Umbrella for the op-graph value types (reference include/vknn/op.h).
#pragma once
#include "vknn/types.h"
