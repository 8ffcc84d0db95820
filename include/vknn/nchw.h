// Forwarding header kept so code that includes the reference header name compiles unchanged.
#pragma once
#include "vknn/types.h"
