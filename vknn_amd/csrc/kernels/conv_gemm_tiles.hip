// Tile instantiations of conv_gemm_kernel (tiles 0-7: A and B staged through LDS).
#include "conv_kernels.h"

namespace vkhip {

    template <int BM, int BN, int WM, int WN>
    static GemmKernelFn pick_bmode(int bmode) {
        switch (bmode) {
            case BMODE_1X1: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_1X1>;
            case BMODE_ALIGNED: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_ALIGNED>;
            case BMODE_1X1_P16: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_1X1_P16>;
            case BMODE_ALIGNED_P16: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_ALIGNED_P16>;
            default: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_GENERAL>;
        }
    }

    GemmKernelFn gemm_tile_kernel(int tile, int bmode) {
        switch (tile) {
            case 0: return pick_bmode<128, 128, 2, 2>(bmode);
            case 1: return pick_bmode<64, 128, 2, 2>(bmode);
            case 2: return pick_bmode<128, 64, 2, 2>(bmode);
            case 3: return pick_bmode<64, 64, 2, 2>(bmode);
            case 4: return pick_bmode<256, 128, 2, 2>(bmode);
            case 5: return pick_bmode<128, 256, 2, 2>(bmode);
            case 6: return pick_bmode<32, 128, 1, 4>(bmode);
            case 7: return pick_bmode<64, 256, 1, 4>(bmode);
        }
        return nullptr;
    }

} // namespace vkhip
