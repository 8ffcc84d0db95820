// Tile instantiations of conv_bd_kernel (tiles 8-10: B fragments loaded straight into registers).
#include "conv_kernels.h"

namespace vkhip {

    template <int FM, int FN, int WM, int WN, int D>
    static GemmKernelFn pick_bd(int bmode) {
        switch (bmode) {
            case BMODE_1X1: return conv_bd_kernel<FM, FN, WM, WN, BMODE_1X1, D>;
            case BMODE_ALIGNED: return conv_bd_kernel<FM, FN, WM, WN, BMODE_ALIGNED, D>;
            default: return conv_bd_kernel<FM, FN, WM, WN, BMODE_GENERAL, D>;
        }
    }


    GemmKernelFn bd_tile_kernel(int tile, int bmode) {
        switch (tile) {
            case 8: return pick_bd<4, 2, 1, 4, 1>(bmode);
            case 9: return pick_bd<2, 2, 2, 2, 1>(bmode);
            case 10: return pick_bd<2, 2, 1, 4, 1>(bmode);
        }
        return nullptr;
    }

} // namespace vkhip
