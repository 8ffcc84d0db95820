// Instantiations of conv_halo_pw_kernel (a 3x3 conv fused with the 1x1 conv that reads it) for 64
// mid channels (wave tile 64 x 64, workgroup 64 x 256 pixels); the 1x1 runs in chunks of 32 output
// channels (64-row chunks need more registers than two waves per SIMD allow and spill), with or
// without a chained second 1x1 of up to 64 output channels (MR fragments).
#include "conv_kernels.h"

namespace vkhip {

    // the instantiation for band size nbi (the smallest NBI that holds it) and its LDS bytes
    template <int FM, int FN, int MC, int MR, int NBI0, int... NBIS>
    static PwKernelFn pick_pw(int nbi, int *lds) {
        if (nbi <= NBI0) {
            if (lds) *lds = halo_lds_bytes<FM, 1, 4, 1, 2, NBI0>();
            return conv_halo_pw_kernel<FM, FN, 4, 1, 2, NBI0, false, MC, MR>;
        }
        if constexpr (sizeof...(NBIS) > 0) return pick_pw<FM, FN, MC, MR, NBIS...>(nbi, lds);
        return nullptr;
    }

    // mr: 32-row fragments of a chained second 1x1 (0: none; 1 or 2 with 64 mid channels)
    PwKernelFn pw_tile_kernel(int cmid, int nbi, int mr, int *lds) {
        if (cmid == 64 && mr == 0) return pick_pw<2, 2, 1, 0, 1, 2, 3, 4, 5, 6, 8, 10, 12, 15>(nbi, lds);
        if (cmid == 64 && mr == 1) return pick_pw<2, 2, 1, 1, 4, 5, 6, 8, 10, 12, 15>(nbi, lds);
        if (cmid == 64 && mr == 2) return pick_pw<2, 2, 1, 2, 4, 5, 6, 8, 10, 12, 15>(nbi, lds);
        return nullptr;
    }

} // namespace vkhip
