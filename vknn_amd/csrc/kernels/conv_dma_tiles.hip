// Tile instantiations of conv_dma_kernel (tiles 11-16, 24, 25, 28-31, and 46-49 with the LDS-staged epilogue: dense B operands via LDS DMA) and of its
// persistent variant conv_dma_persist_kernel (tiles 36-42).
#include "conv_kernels.h"

namespace vkhip {

    // conv_dma_kernel with its LDS ring cut to the number of K stages one split runs (fewer stages
    // need no deeper ring; the smaller LDS footprint lets more workgroups share a CU).
    template <int FM, int FN, int NS, int WM, int WN, int PS = 8, bool XS = false>
    static GemmKernelFn pick_dma_ps(int steps) {
        if constexpr (NS > 1) {
            if (steps < NS) return pick_dma_ps<FM, FN, NS - 1, WM, WN, PS, XS>(steps);
        }
        return conv_dma_kernel<FM, FN, NS, WM, WN, PS, XS>;
    }
    // bmode 2 = stride-2 columns (16 bytes per B column)
    template <int FM, int FN, int NS, int WM, int WN>
    static GemmKernelFn pick_dma(int steps, int bmode) {
        constexpr int lds16 = NS * (32 * FM * WM + 2 * 32 * FN * WN) * kBK * 2; // LDS of the 16-byte-column variant
        if (bmode == 2) {
            if constexpr (lds16 <= 160 * 1024) return pick_dma_ps<FM, FN, NS, WM, WN, 16>(steps);
            else return nullptr;
        }
        return pick_dma_ps<FM, FN, NS, WM, WN, 8>(steps);
    }

    // LDS-staged epilogue variants (the ring cut to the step count like pick_dma_ps, but never
    // below what the epilogue's BM / 4 rows of 1040 bytes need)
    template <int FM, int FN, int NS, int WM, int WN, int PS = 8>
    static GemmKernelFn pick_le_ps(int steps) {
        constexpr int STG = (32 * FM * WM + 32 * FN * WN * PS / 8) * kBK * 2;
        if constexpr (NS > 1 && (NS - 1) * STG >= (32 * FM * WM / 4) * 1040) {
            if (steps < NS) return pick_le_ps<FM, FN, NS - 1, WM, WN, PS>(steps);
        }
        return conv_dma_kernel<FM, FN, NS, WM, WN, PS, false, true>;
    }
    template <int FM, int FN, int NS, int WM, int WN>
    static GemmKernelFn pick_le(int steps, int bmode) {
        constexpr int lds16 = NS * (32 * FM * WM + 2 * 32 * FN * WN) * kBK * 2;
        if (bmode == 2) {
            if constexpr (lds16 <= 160 * 1024) return pick_le_ps<FM, FN, NS, WM, WN, 16>(steps);
            else return nullptr;
        }
        return pick_le_ps<FM, FN, NS, WM, WN, 8>(steps);
    }

    // persistent variants (the ring spans tiles, so it is never cut to the step count)
    template <int FM, int FN, int NS, int WM, int WN>
    static GemmKernelFn pick_pers(int bmode) {
        constexpr int lds16 = NS * ((32 * FM * WM + 2 * 32 * FN * WN) * kBK * 2 + 1024) + 1024; // ring + bias slices + spare
        if (bmode == 2) {
            if constexpr (lds16 <= 160 * 1024) return conv_dma_persist_kernel<FM, FN, NS, WM, WN, 16>;
            else return nullptr;
        }
        return conv_dma_persist_kernel<FM, FN, NS, WM, WN, 8>;
    }

    // the smallest band-size instantiation (NBIS ascending) that holds nbi chunks per slot
    // nbi < 0: odd input width (the ODD variant), |nbi| chunks
    // xs: the input-scale variant (only the tiles that win on squeeze-excite projections)
    GemmKernelFn dma_tile_kernel(int tile, int bmode, int steps, bool xs) {
        if (xs) {
            if (bmode == 2) return nullptr;
            switch (tile) {
                case 14: return pick_dma_ps<2, 2, 2, 2, 2, 8, true>(steps);
                case 16: return pick_dma_ps<2, 2, 4, 2, 2, 8, true>(steps);
                case 24: return pick_dma_ps<1, 2, 2, 2, 2, 8, true>(steps);
                case 25: return pick_dma_ps<2, 2, 2, 1, 4, 8, true>(steps);
            }
            return nullptr;
        }
        switch (tile) {
            case 11: return pick_dma<4, 4, 2, 2, 2>(steps, bmode);
            case 12: return pick_dma<4, 2, 2, 2, 4>(steps, bmode);
            case 13: return pick_dma<2, 4, 2, 4, 2>(steps, bmode);
            case 14: return pick_dma<2, 2, 2, 2, 2>(steps, bmode);
            case 15: return pick_dma<2, 2, 2, 4, 2>(steps, bmode);
            case 16: return pick_dma<2, 2, 4, 2, 2>(steps, bmode);
            case 24: return pick_dma<1, 2, 2, 2, 2>(steps, bmode);
            case 25: return pick_dma<2, 2, 2, 1, 4>(steps, bmode);
            case 28: return pick_dma<1, 2, 3, 2, 2>(steps, bmode);
            case 29: return pick_dma<2, 2, 3, 2, 2>(steps, bmode);
            case 30: return pick_dma<2, 2, 3, 1, 4>(steps, bmode);
            case 31: return pick_dma<1, 2, 4, 2, 2>(steps, bmode);
            case 36: return pick_pers<2, 2, 2, 2, 2>(bmode);
            case 37: return pick_pers<2, 2, 3, 2, 2>(bmode);
            case 38: return pick_pers<1, 2, 2, 2, 2>(bmode);
            case 39: return pick_pers<1, 2, 4, 2, 2>(bmode);
            case 40: return pick_pers<2, 2, 2, 1, 4>(bmode);
            case 41: return pick_pers<2, 2, 2, 4, 2>(bmode);
            case 42: return pick_pers<2, 2, 4, 2, 2>(bmode);
            case 46: return pick_le<2, 2, 2, 2, 2>(steps, bmode);
            case 47: return pick_le<1, 2, 2, 2, 2>(steps, bmode);
            case 48: return pick_le<2, 2, 3, 2, 2>(steps, bmode);
            case 49: return pick_le<1, 2, 4, 2, 2>(steps, bmode);
        }
        return nullptr;
    }

} // namespace vkhip
