// Instantiations of conv_halo_pw_kernel (a 3x3 conv fused with the 1x1 conv that reads it) for the
// two mid widths it serves: 64 channels (wave tile 64 x 64, workgroup 64 x 256 pixels) and 128
// channels (wave tile 128 x 32, workgroup 128 x 128); the 1x1 runs in chunks of 32 output channels
// (64-row chunks need more registers than two waves per SIMD allow and spill).
#include "conv_kernels.h"

namespace vkhip {

    template <int FM, int FN, int MC, int NBI0, int... NBIS>
    static PwKernelFn pick_pw(int nbi) {
        if (nbi <= NBI0) return conv_halo_pw_kernel<FM, FN, 4, 1, 2, NBI0, false, MC>;
        if constexpr (sizeof...(NBIS) > 0) return pick_pw<FM, FN, MC, NBIS...>(nbi);
        return nullptr;
    }

    PwKernelFn pw_tile_kernel(int cmid, int nbi) {
        if (cmid == 64) return pick_pw<2, 2, 1, 1, 2, 3, 4, 5, 6, 8, 10, 12, 15>(nbi);
        if (cmid == 128) return pick_pw<4, 1, 1, 1, 2, 3, 4, 5, 6, 8, 10>(nbi);
        return nullptr;
    }

} // namespace vkhip
