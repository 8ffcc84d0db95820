// Tile instantiations of conv_halo_kernel (tiles 17-20, 26, 27, 32-35: 3x3 with the input band staged once).
#include "conv_kernels.h"

namespace vkhip {

    // the smallest band-size instantiation (NBIS ascending) that holds nbi chunks per slot
    // nbi < 0: odd input width (the ODD variant), |nbi| chunks
    template <int FM, int FN, int WM, int WN, int KK, int NS, int NBI0, int... NBIS>
    static GemmKernelFn pick_halo(int nbi) {
        const bool odd = nbi < 0;
        const int  n   = odd ? -nbi : nbi;
        if (n <= NBI0) return odd ? conv_halo_kernel<FM, FN, WM, WN, KK, NS, NBI0, true> : conv_halo_kernel<FM, FN, WM, WN, KK, NS, NBI0>;
        if constexpr (sizeof...(NBIS) > 0) return pick_halo<FM, FN, WM, WN, KK, NS, NBIS...>(nbi);
        return nullptr;
    }
    GemmKernelFn halo_tile_kernel(int tile, int nbi) {
        switch (tile) {
            case 17: return pick_halo<2, 2, 2, 2, 1, 3, 1, 2, 3, 4>(nbi);
            case 18: return pick_halo<2, 2, 1, 4, 1, 2, 1, 2, 3, 4, 5, 6, 8, 10, 12, 15>(nbi);
            case 19: return pick_halo<2, 4, 2, 2, 1, 2, 2, 3, 4, 5, 6, 8, 10>(nbi);
            case 20: return pick_halo<2, 1, 1, 4, 1, 1, 1, 2, 3, 4, 5, 6, 8, 10, 12, 16>(nbi);
            case 26: return pick_halo<2, 1, 1, 4, 1, 2, 1, 2, 3, 4, 5, 6, 8>(nbi);
            case 27: return pick_halo<2, 2, 1, 4, 1, 1, 2, 4, 6, 8, 10, 12, 15>(nbi);
            case 32: return pick_halo<1, 2, 1, 4, 1, 2, 1, 2, 3, 4, 5, 6, 8, 10, 12, 15>(nbi);
            case 33: return pick_halo<1, 1, 1, 4, 1, 2, 1, 2, 3, 4, 5, 6, 8>(nbi);
            case 34: return pick_halo<1, 2, 1, 4, 1, 1, 2, 4, 6, 8, 10, 12, 16>(nbi);
            case 35: return pick_halo<1, 1, 1, 4, 1, 1, 2, 4, 6, 8, 10>(nbi);
        }
        return nullptr;
    }

} // namespace vkhip
