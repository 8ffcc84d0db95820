// The first two convs of a YOLOv8-style backbone in one kernel: a 3x3 stride-2 conv over at most 4
// input channels to 9-16 channels, then a 3x3 stride-2 conv to at most 32 channels (YOLOv8n:
// 3 -> 16 at 640x640, 16 -> 32 at 320x320). Run as two launches, the 16-channel intermediate
// (half the input's pixels, four times its channel slots) goes to HBM and comes back; both
// launches stream at a fraction of HBM bandwidth with a launch ramp each. Here:
//   * one persistent workgroup per CU slot walks items of 2 output rows x 64 output columns
//     (XCD-contiguous item ranges, so the input rows adjacent items share come from L2);
//   * the item's input band (11 rows x 290 columns of the input's 4-channel slot) is copied
//     global->LDS by buffer-load-to-LDS;
//   * the first conv computes the 5 x 144 intermediate pixels the second conv's stride-2 window
//     needs (9 column tiles of 16; 129 are used) and leaves them in LDS as fp16, rounded like
//     the separate conv's store, with positions outside the intermediate image set to zero (the
//     second conv's padding);
//   * the second conv reads that tile, adds bias and activation and stores 8-byte NC4HW4 slots, or,
//     with a 1x1 tail conv (the next layer when it is the second conv's only reader), leaves its
//     tile in LDS for the tail, which stores instead.
// Both convs use v_mfma_f32_16x16x32_f16 with their weights in registers, in the thin kernel's
// fragment layout (the blobs vkhip_conv_pack_weights writes for thin tiles 43 / 44).
// Reference semantics: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) twice.
#include "conv_kernels.h"

#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

namespace vkhip {

    struct Stem2Args {
        const uint2  *x;
        uint2        *y;
        const half_t *wa, *wb, *wc; // thin-kernel fragment layout [m_frag][step][lane][8 halves]
        const float  *ba, *bb, *bc; // [16], [MTB*16], [MTC*16]
        int           N, H, W;        // input
        int           HA, WA;         // first conv's output
        int           HB, WB;         // second conv's output
        int           cbx, cbm, cbo;  // channel slots: input, intermediate, output (of the second conv)
        int           cbc;            // output slots of the 1x1 tail (y is then its output)
        int           x_pstride, y_pstride;
        unsigned      x_bytes, y_bytes;
        int           acta, actb, actc;
        float         loa, hia, lob, hib, loc, hic;
    };

    namespace stem2 {
        constexpr int OR   = 2;             // output rows per item
        constexpr int OCW  = 64;            // output columns per item
        constexpr int IR   = 2 * OR + 1;    // intermediate rows (stride-2 window over OR rows)
        constexpr int IT   = 9;             // 16-pixel column tiles of the intermediate (2*OCW+1 = 129 used)
        constexpr int ICW  = IT * 16;
        constexpr int BR   = 2 * IR + 1;    // input band rows
        constexpr int BC   = 2 * ICW + 2;   // input band columns (even: whole pixel pairs)
        constexpr int BPPR = BC / 2;
        constexpr int CBM  = 4;             // intermediate slots (9-16 channels)
    } // namespace stem2

    template <int ACT>
    __device__ __forceinline__ float stem2_act(float v, int act, float lo, float hi) {
        return apply_act(v, ACT >= 0 ? ACT : act, lo, hi);
    }

    // MTC > 0: a 1x1 conv over the second conv's output (MTC 16-channel fragments) runs as a tail:
    // the second conv's tile goes to LDS instead of HBM and y is the 1x1's output.
    template <int MTB, int ACTA, int ACTB, int MTC>
    __global__ __launch_bounds__(256, 2) void conv_stem2_kernel(Stem2Args a) {
        using namespace stem2;
        constexpr int NSA   = 2;                      // first conv: 9 taps x 4 channels in 2 32-deep steps
        constexpr int NSB   = (9 * CBM * 4 + 31) / 32; // second conv: 5 steps
        constexpr int TP    = BR * BPPR;               // pixel pairs of the band (one slot)
        constexpr int NI    = (TP + 63) / 64;
        constexpr int NBW   = (NI + 3) / 4;
        constexpr int BAND  = NBW * 4 * 1024;
        constexpr int INTER = CBM * IR * ICW * 8;
        constexpr int CTILE = MTC ? MTB * 4 * OR * OCW * 8 : 0; // the second conv's tile for the tail
        static_assert(BAND + INTER + CTILE <= 80 * 1024, "two workgroups per CU at least");
        __shared__ __attribute__((aligned(16))) unsigned char sm[BAND + INTER + CTILE];
        unsigned char *band  = sm;
        unsigned char *inter = sm + BAND;
        unsigned char *ctile = sm + BAND + INTER;

        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int rblk = (a.HB + OR - 1) / OR, cblk = (a.WB + OCW - 1) / OCW;
        const int items = a.N * rblk * cblk;
        constexpr unsigned kInvalid = 0x80000000u;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);

        half8 wfa[1][NSA], wfb[MTB][NSB], wfc[MTC ? MTC : 1][1];
        {
            const half8 *pa = reinterpret_cast<const half8 *>(a.wa);
            const half8 *pb = reinterpret_cast<const half8 *>(a.wb);
#pragma unroll
            for (int j = 0; j < NSA; ++j) wfa[0][j] = pa[j * 64 + lane];
#pragma unroll
            for (int m = 0; m < MTB; ++m)
#pragma unroll
                for (int j = 0; j < NSB; ++j) wfb[m][j] = pb[(m * NSB + j) * 64 + lane];
            if constexpr (MTC > 0) {
                const half8 *pc = reinterpret_cast<const half8 *>(a.wc);
#pragma unroll
                for (int m = 0; m < MTC; ++m) wfc[m][0] = pc[m * 64 + lane];
            }
        }
        // per (step, half): offset of the lane's (tap, slot) from the window origin, -1 = zero pad.
        // First conv over the band: 4 channels per tap (k = tap*4 + c); second over the
        // intermediate tile: 16 channels per tap (k = tap*16 + slot*4 + c).
        int aoff[NSA][2], boff[NSB][2];
#pragma unroll
        for (int j = 0; j < NSA; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int tap = (32 * j + 8 * (lane >> 4) + 4 * q) / 4;
                aoff[j][q]    = tap < 9 ? (tap / 3) * BC + tap % 3 : -1;
            }
#pragma unroll
        for (int j = 0; j < NSB; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int k   = 32 * j + 8 * (lane >> 4) + 4 * q;
                const int tap = k / 16, slot = (k % 16) / 4;
                boff[j][q]    = tap < 9 ? (slot * IR + tap / 3) * ICW + tap % 3 : -1;
            }

        // tail (1x1 over MTB*16 channels in one 32-deep step): the lane's slots 8(l/16)/4 + q of the tile
        int coff[1][2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int slot = 2 * (lane >> 4) + q;
            coff[0][q]     = slot < MTB * 4 ? slot * OR * OCW : -1;
        }
        auto mma = [&](const unsigned char *src, const auto &off, const auto &wf, int base, auto &acc) __attribute__((always_inline)) {
            constexpr int NS = sizeof(off) / sizeof(off[0]);
            constexpr int MT = sizeof(acc) / sizeof(acc[0]);
            // acc holds the biases on entry; absent taps (off < 0) read the window origin and are
            // masked after the read (no branches)
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                u32x2 v[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int   o = off[j][q] < 0 ? 0 : off[j][q];
                    const u32x2 t = *reinterpret_cast<const u32x2 *>(src + (base + o) * 8);
                    v[q]          = off[j][q] >= 0 ? t : u32x2 {0u, 0u};
                }
                const half8 bf = __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y));
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[m][j], bf, acc[m], 0, 0, 0);
            }
        };
        const int g = lane >> 4, px = lane & 15;
        // the lane's biases (rows 4g..4g+3 of each 16-channel fragment), which seed the accumulators
        float4v bsa[1], bsb[MTB], bsc[MTC ? MTC : 1];
        bsa[0] = *reinterpret_cast<const float4v *>(a.ba + g * 4);
#pragma unroll
        for (int m = 0; m < MTB; ++m) bsb[m] = *reinterpret_cast<const float4v *>(a.bb + (m * 4 + g) * 4);
#pragma unroll
        for (int m = 0; m < (MTC ? MTC : 1); ++m) bsc[m] = MTC ? *reinterpret_cast<const float4v *>(a.bc + (m * 4 + g) * 4) : float4v {};

        // items: XCD-contiguous ranges (workgroup b runs on XCD b % 8)
        const int G = gridDim.x;
        const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3;
        const int gx  = (G >> 3) + ((G & 7) > xcd ? 1 : 0);
        const int pxc = xcd * (G >> 3) + min(xcd, G & 7);
        const int i0  = (int) ((long long) items * pxc / G) + lb;
        const int i1  = (int) ((long long) items * (pxc + gx) / G);
        for (int it = i0; it < i1; it += gx) {
            const int cb = it % cblk, rest = it / cblk;
            const int ox0 = cb * OCW, oy0 = (rest % rblk) * OR, n = rest / rblk;
            // band row r, column c <-> input (4 oy0 - 3 + r, 4 ox0 - 4 + c)
            const int iy0 = 4 * oy0 - 3, ix0 = 4 * ox0 - 4;
#pragma unroll
            for (int r = 0; r < NBW; ++r) {
                const int i   = r * 4 + wave;
                const int p   = i * 64 + lane;
                const int pc  = p % BPPR, row = p / BPPR;
                const int iy  = iy0 + row, ix = ix0 + 2 * pc;
                const bool ok = p < TP && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                const unsigned off = ok ? (unsigned) (((n * a.x_pstride * a.H + iy) * a.W + ix) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (band + i * 1024), 16, off, 0, 0, 0);
            }
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // this wave's copies (and last item's stores) done
            __asm__ volatile("s_barrier" ::: "memory");        // every wave's copies landed
            // first conv: intermediate pixel (r, c) <-> first-conv output (2 oy0 - 1 + r, 2 ox0 - 1 + c),
            // its window at band row 2r, column 2c + 1
            // two units per pass, so their LDS reads and MFMAs overlap
            auto first_unit = [&](int u) __attribute__((always_inline)) {
                const int r = u / IT, c = (u % IT) * 16 + px;
                float4v   acc[1] = {bsa[0]};
                mma(band, aoff, wfa, 2 * r * BC + 2 * c + 1, acc);
                const int  iy = 2 * oy0 - 1 + r, ix = 2 * ox0 - 1 + c;
                const bool in = ((unsigned) iy < (unsigned) a.HA) & ((unsigned) ix < (unsigned) a.WA) & (g < a.cbm);
                float4v    v  = acc[0];
                v.x = stem2_act<ACTA>(v.x, a.acta, a.loa, a.hia);
                v.y = stem2_act<ACTA>(v.y, a.acta, a.loa, a.hia);
                v.z = stem2_act<ACTA>(v.z, a.acta, a.loa, a.hia);
                v.w = stem2_act<ACTA>(v.w, a.acta, a.loa, a.hia);
                *reinterpret_cast<u32x2 *>(inter + ((g * IR + r) * ICW + c) * 8) = in ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0u, 0u};
            };
            // (past the end, the second unit repeats the last one: the same values to the same place)
            for (int u = wave; u < IR * IT; u += 8) {
                first_unit(u);
                first_unit(min(u + 4, IR * IT - 1));
            }
            __syncthreads(); // the intermediate tile is complete
            // second conv: output (oy0 + orow, ox0 + c), window at intermediate row 2 orow, column 2c
#pragma unroll 1
            for (int u = wave; u < OR * (OCW / 16); u += 4) {
                const int orow = u / (OCW / 16), c = (u % (OCW / 16)) * 16 + px;
                float4v   acc[MTB];
#pragma unroll
                for (int m = 0; m < MTB; ++m) acc[m] = bsb[m];
                mma(inter, boff, wfb, 2 * orow * ICW + 2 * c, acc);
                const int  oy = oy0 + orow, ox = ox0 + c;
                const bool pok = oy < a.HB && ox < a.WB;
#pragma unroll
                for (int m = 0; m < MTB; ++m) {
                    const int ocb = m * 4 + g;
                    float4v   v   = acc[m];
                    v.x = stem2_act<ACTB>(v.x, a.actb, a.lob, a.hib);
                    v.y = stem2_act<ACTB>(v.y, a.actb, a.lob, a.hib);
                    v.z = stem2_act<ACTB>(v.z, a.actb, a.lob, a.hib);
                    v.w = stem2_act<ACTB>(v.w, a.actb, a.lob, a.hib);
                    if constexpr (MTC > 0) {
                        // to the tail's tile (channel slots past the output's are zero)
                        *reinterpret_cast<u32x2 *>(ctile + ((ocb * OR + orow) * OCW + c) * 8) =
                            ocb < a.cbo ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0u, 0u};
                    } else {
                        const unsigned off = pok && ocb < a.cbo ? (unsigned) ((((n * a.y_pstride + ocb) * a.HB + oy) * a.WB + ox) * 8) : kInvalid;
                        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, off, 0, kStreamStore);
                    }
                }
            }
            if constexpr (MTC > 0) {
                __syncthreads(); // the second conv's tile is complete
                // 1x1 tail: output (oy0 + orow, ox0 + c) from the tile's pixel (orow, c)
#pragma unroll 1
                for (int u = wave; u < OR * (OCW / 16); u += 4) {
                    const int orow = u / (OCW / 16), c = (u % (OCW / 16)) * 16 + px;
                    float4v   acc[MTC];
#pragma unroll
                    for (int m = 0; m < MTC; ++m) acc[m] = bsc[m];
                    mma(ctile, coff, wfc, orow * OCW + c, acc);
                    const int  oy = oy0 + orow, ox = ox0 + c;
                    const bool pok = oy < a.HB && ox < a.WB;
#pragma unroll
                    for (int m = 0; m < MTC; ++m) {
                        const int ocb = m * 4 + g;
                        float4v   v   = acc[m];
                        v.x = stem2_act<ACTB>(v.x, a.actc, a.loc, a.hic);
                        v.y = stem2_act<ACTB>(v.y, a.actc, a.loc, a.hic);
                        v.z = stem2_act<ACTB>(v.z, a.actc, a.loc, a.hic);
                        v.w = stem2_act<ACTB>(v.w, a.actc, a.loc, a.hic);
                        const unsigned off = pok && ocb < a.cbc ? (unsigned) ((((n * a.y_pstride + ocb) * a.HB + oy) * a.WB + ox) * 8) : kInvalid;
                        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, off, 0, kStreamStore);
                    }
                }
            }
            __syncthreads(); // band and intermediate tile free for the next item
        }
    }

    typedef void (*Stem2KernelFn)(Stem2Args);

    // kernel for MTB / MTC (0: no tail); one compile-time activation when all the convs share it
    template <int MTB, int MTC>
    static Stem2KernelFn stem2_pick(int acta, int actb, int actc) {
        if (acta == actb && (MTC == 0 || actc == acta)) {
            switch (acta) {
                case VKHIP_ACT_RELU: return conv_stem2_kernel<MTB, VKHIP_ACT_RELU, VKHIP_ACT_RELU, MTC>;
                case VKHIP_ACT_SILU: return conv_stem2_kernel<MTB, VKHIP_ACT_SILU, VKHIP_ACT_SILU, MTC>;
                case VKHIP_ACT_HARDSWISH: return conv_stem2_kernel<MTB, VKHIP_ACT_HARDSWISH, VKHIP_ACT_HARDSWISH, MTC>;
                default: break;
            }
        }
        return conv_stem2_kernel<MTB, -1, -1, MTC>; // activations chosen at run time
    }

} // namespace vkhip

using namespace vkhip;

static bool stem2_conv_ok(const vkhip_conv_desc *c) {
    return c->group == 1 && c->KH == 3 && c->KW == 3 && c->SH == 2 && c->SW == 2 && c->PT == 1 && c->PL == 1 && c->DH == 1 && c->DW == 1 &&
           !c->in_scale && !c->has_res && c->N > 0 && c->H > 0 && c->W > 0 && c->OH == (c->H - 1) / 2 + 1 && c->OW == (c->W - 1) / 2 + 1;
}

extern "C" {

int vkhip_conv3x3s2_pair_plan(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, const vkhip_conv_desc *c3, vkhip_conv_plan *p1,
                              vkhip_conv_plan *p2, vkhip_conv_plan *p3) {
    if (!c1 || !c2 || !p1 || !p2 || (c3 && !p3)) return set_error(VKHIP_ERR_INVALID, "conv3x3s2_pair_plan: null argument");
    if (!stem2_conv_ok(c1) || !stem2_conv_ok(c2))
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3s2_pair: two dense 3x3 stride-2 pad-1 convs, no residual or input scale");
    if (c2->N != c1->N || c2->Cin != c1->Cout || c2->H != c1->OH || c2->W != c1->OW)
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3s2_pair: the second conv reads the first's output");
    if (c1->Cin > 4 || c1->Cout < 9 || c1->Cout > 16 || c2->Cout > 32 || c1->W % 2)
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3s2_pair: at most 4 input channels, 9-16 between, at most 32 out, an even input width");
    if (c3 && (c3->group != 1 || c3->KH != 1 || c3->KW != 1 || c3->SH != 1 || c3->SW != 1 || c3->PT || c3->PL || c3->DH != 1 || c3->DW != 1 ||
               c3->in_scale || c3->has_res || c3->N != c2->N || c3->Cin != c2->Cout || c3->H != c2->OH || c3->W != c2->OW || c3->OH != c3->H ||
               c3->OW != c3->W || c3->Cout > 32 || c3->Cout <= 0))
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3s2_pair: the tail is a dense 1x1 conv over the second conv's output, at most 32 out");
    if ((int64_t) c1->N * c1->H * c1->W * 8 >= (1LL << 31) || (int64_t) c2->N * ceil_div(std::max(c2->Cout, c3 ? c3->Cout : 0), 4) * c2->OH * c2->OW * 8 >= (1LL << 31))
        return set_error(VKHIP_ERR_INVALID, "conv3x3s2_pair: tensor >= 2 GiB");
    // the blobs are the thin tiles' (16 or 32 output rows). The second conv's own thin plan would
    // need an even width, which the fused kernel does not (its input never leaves LDS, and the
    // blob layout does not depend on the width); the same for the tail.
    vkhip_conv_desc e2 = *c2;
    e2.W += e2.W & 1;
    int rc = vkhip_conv_plan_make(c1, VKHIP_CONV_GEMM, 43, 0, p1);
    if (!rc) rc = vkhip_conv_plan_make(&e2, VKHIP_CONV_GEMM, c2->Cout <= 16 ? 43 : 44, 0, p2);
    if (!rc && c3) {
        vkhip_conv_desc e3 = *c3;
        e3.W += e3.W & 1;
        e3.OW = e3.W;
        rc = vkhip_conv_plan_make(&e3, VKHIP_CONV_GEMM, c3->Cout <= 16 ? 43 : 44, 0, p3);
    }
    return rc;
}

int vkhip_conv3x3s2_pair_forward(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, const vkhip_conv_desc *c3, const void *x, const void *blob1,
                                 const void *blob2, const void *blob3, void *y, int64_t y_pstride, vkhip_stream_t s) {
    if (!c1 || !c2 || !x || !blob1 || !blob2 || !y || (c3 && !blob3)) return set_error(VKHIP_ERR_INVALID, "conv3x3s2_pair_forward: null argument");
    vkhip_conv_plan p1, p2, p3;
    int rc = vkhip_conv3x3s2_pair_plan(c1, c2, c3, &p1, &p2, &p3);
    if (rc) return rc;
    const int     cbo = (int) ceil_div(c2->Cout, 4), cby = c3 ? (int) ceil_div(c3->Cout, 4) : cbo;
    const int64_t yps = y_pstride > 0 ? y_pstride : cby;
    if (yps < cby) return set_error(VKHIP_ERR_INVALID, "conv3x3s2_pair_forward: plane stride below the channel blocks");
    const int64_t oplane = (int64_t) c2->OH * c2->OW * 8;
    if ((int64_t) c2->N * yps * oplane >= (1LL << 31)) return set_error(VKHIP_ERR_INVALID, "conv3x3s2_pair_forward: view >= 2 GiB");
    const int mtb = c2->Cout <= 16 ? 1 : 2, mtc = !c3 ? 0 : c3->Cout <= 16 ? 1 : 2;
    Stem2Args a;
    std::memset(&a, 0, sizeof(a));
    a.x  = (const uint2 *) x;
    a.y  = (uint2 *) y;
    // blob: bias [Coutp] fp32 at 0, weights at align256(Coutp * 4) (Coutp = 16 or 32)
    a.ba = (const float *) blob1;
    a.bb = (const float *) blob2;
    a.bc = (const float *) blob3;
    a.wa = (const half_t *) ((const char *) blob1 + 256);
    a.wb = (const half_t *) ((const char *) blob2 + 256);
    a.wc = blob3 ? (const half_t *) ((const char *) blob3 + 256) : nullptr;
    a.N = c1->N; a.H = c1->H; a.W = c1->W;
    a.HA = c1->OH; a.WA = c1->OW; a.HB = c2->OH; a.WB = c2->OW;
    a.cbx = 1; a.cbm = (int) ceil_div(c1->Cout, 4); a.cbo = cbo; a.cbc = c3 ? cby : 0;
    a.x_pstride = 1; a.y_pstride = (int) yps;
    a.x_bytes = (unsigned) ((int64_t) c1->N * c1->H * c1->W * 8);
    a.y_bytes = (unsigned) (((int64_t) (c2->N - 1) * yps + cby) * oplane);
    a.acta = c1->act; a.loa = c1->act_lo; a.hia = c1->act_hi;
    a.actb = c2->act; a.lob = c2->act_lo; a.hib = c2->act_hi;
    if (c3) a.actc = c3->act, a.loc = c3->act_lo, a.hic = c3->act_hi;
    const int actc = c3 ? c3->act : c1->act;
    Stem2KernelFn fn = mtb == 1 ? (mtc == 0 ? stem2_pick<1, 0>(c1->act, c2->act, actc) : mtc == 1 ? stem2_pick<1, 1>(c1->act, c2->act, actc)
                                                                                             : stem2_pick<1, 2>(c1->act, c2->act, actc))
                                : (mtc == 0 ? stem2_pick<2, 0>(c1->act, c2->act, actc) : mtc == 1 ? stem2_pick<2, 1>(c1->act, c2->act, actc)
                                                                                             : stem2_pick<2, 2>(c1->act, c2->act, actc));
    const int64_t items = (int64_t) c2->N * ceil_div(c2->OH, stem2::OR) * ceil_div(c2->OW, stem2::OCW);
    // as many workgroups as the device holds at once, at most one per item
    static std::mutex                                mu;
    static std::vector<std::pair<const void *, int>> occ;
    int per_cu = 0, cus = 256;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (auto &e: occ)
            if (e.first == (const void *) fn) per_cu = e.second;
        if (!per_cu) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *) fn, 256, 0) != hipSuccess || per_cu <= 0) per_cu = 1;
            occ.emplace_back((const void *) fn, per_cu);
        }
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    }
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>((int64_t) cus * per_cu, items));
    fn<<<dim3((unsigned) grid), 256, 0, resolve_stream(s)>>>(a);
    return check_launch("conv3x3s2_pair");
}

} // extern "C"
