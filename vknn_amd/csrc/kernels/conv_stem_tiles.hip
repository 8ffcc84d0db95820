// Tile instantiations of conv_stem_kernel (tiles 21-23: 3x3/7x7 over at most 4 input channels).
#include "conv_kernels.h"

namespace vkhip {

    template <int K, int FM, int FN, int WM, int WN, int NBI0, int... NBIS>
    static GemmKernelFn pick_stem(int nbi) {
        if (nbi <= NBI0) return conv_stem_kernel<K, FM, FN, WM, WN, NBI0>;
        if constexpr (sizeof...(NBIS) > 0) return pick_stem<K, FM, FN, WM, WN, NBIS...>(nbi);
        return nullptr;
    }

    // bmode carries the kernel size (3 or 7)
    GemmKernelFn stem_tile_kernel(int tile, int bmode, int nbi) {
        switch (tile) {
            case 21: return bmode == 7 ? pick_stem<7, 2, 2, 1, 4, 8, 16, 24, 32, 48>(nbi) : pick_stem<3, 2, 2, 1, 4, 4, 8, 16, 24, 32, 48>(nbi);
            case 22: return bmode == 7 ? pick_stem<7, 2, 1, 1, 4, 8, 16, 24, 32, 48>(nbi) : pick_stem<3, 2, 1, 1, 4, 4, 8, 16, 24, 32, 48>(nbi);
            case 23: return bmode == 7 ? pick_stem<7, 1, 2, 1, 4, 8, 16, 24, 32, 48>(nbi) : pick_stem<3, 1, 2, 1, 4, 4, 8, 16, 24, 32, 48>(nbi);
        }
        return nullptr;
    }

} // namespace vkhip
