// A MobileNetV3 stem and its first block in one kernel: a 3x3 stride-2 conv over at most 4 input
// channels to 9-16 channels, a 3x3 stride-1 depthwise conv over those channels, and the 1x1
// projection back to at most 16 channels with the stem's output as the residual (MobileNetV3-Large:
// 3 -> 16 hard-swish at 224x224, dw 3x3 ReLU, 16 -> 16 + x). Run as separate launches, the
// 16-channel tensors at 112x112 go through HBM several times; here they stay in LDS:
//   * one persistent workgroup per CU slot walks items of 4 output rows x up to 64 columns (the
//     width split evenly), XCD-contiguous item ranges;
//   * the stem's input band (13 rows of the input's 4-channel slot) arrives in LDS by
//     buffer-load-to-LDS, double-buffered: the next item's copies run under this item's work;
//   * the stem computes the 6-row tile the depthwise window needs (16x16x32 MFMA, weights in
//     registers) into LDS as fp16, zero outside the image (the depthwise conv's padding), rounded
//     like the separate conv's store;
//   * the depthwise conv runs on MFMA too, as a 3x3 conv over 16 channels whose weight matrix is
//     zero off the diagonal (built in registers from the depthwise blob); its tile goes to LDS as fp16;
//   * the projection (one 32-deep MFMA step per 16 pixels) adds the stem's pixel from LDS as the
//     residual and its activation, and stores 8-byte NC4HW4 slots.
// The kernel is bound by instruction issue, not HBM: biases seed the accumulators, phases are
// branch-free and take two 16-pixel units per pass so LDS reads and MFMAs overlap.
// Reference semantics: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) for the stem, FusedDwPw
// (src/backend/cpu/ops/fused_dwpw.cpp:10-87) for the block.
#include "conv_kernels.h"

#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

namespace vkhip {

    struct StemDwPwArgs {
        const uint2  *x;
        uint2        *y;
        const half_t *wa, *wp; // thin-kernel fragment layout (stem: 3x3 over 1 slot; projection: 1x1 over 4 slots)
        const float  *ba, *bd, *bp;
        const uint2  *wd; // depthwise weights [slot][tap] x 4 channels fp16
        int           N, H, W;  // input
        int           ocw;      // output columns per item
        int           OH, OW;   // stem / block output
        int           cbm, cbo; // channel slots: stem output, projection output
        int           y_pstride;
        unsigned      x_bytes, y_bytes;
        int           acta, actd, actp, res;
        float         loa, hia, lod, hid, lop, hip;
    };

    namespace sdp {
        constexpr int OR   = 4;           // output rows per item
        constexpr int MAXW = 64;          // output columns per item, at most (a.ocw: the image width split evenly)
        constexpr int IR   = OR + 2;      // stem rows the depthwise window needs
        constexpr int MSW  = MAXW + 2;    // stem columns, at most
        constexpr int BR   = 2 * IR + 1;  // input band rows
        constexpr int MBPR = MSW + 1;     // band pixel pairs per row, at most (2 * MSW + 2 columns)
        constexpr int CB   = 4;           // channel slots of the block (9-16 channels)
    } // namespace sdp

    // Hard-swish as v * relu6(v + 3) times the fp32 reciprocal of 6 (within one fp32 ulp of the
    // quotient, well inside the fp16 rounding that follows; 4 instructions instead of a divide).
    template <int ACT>
    __device__ __forceinline__ float sdp_act(float v, int act, float lo, float hi) {
        if constexpr (ACT == VKHIP_ACT_HARDSWISH) return v * fminf(fmaxf(v + 3.f, 0.f), 6.f) * (1.f / 6.f);
        return apply_act(v, ACT >= 0 ? ACT : act, lo, hi);
    }

    // v / d for 0 <= v < 2^12 and 1 <= d <= 128, with r = 1/d in fp32: v/d is at least 1/(2d)
    // away from the next integer (v + 1/2 over d), far more than the product's rounding error.
    __device__ __forceinline__ int fdiv(int v, float r) { return (int) (((float) v + 0.5f) * r); }

    // A workgroup barrier over LDS writes only: the next item's band copies stay in flight
    // (__syncthreads would wait for them too).
    __device__ __forceinline__ void sdp_lds_barrier() {
        __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0); vmcnt, expcnt untouched
        __asm__ volatile("s_barrier" ::: "memory");
    }

    // Items of OR output rows x a.ocw columns; all tiles are indexed by flat pixel number, so the
    // 16-pixel MFMA columns and the depthwise lanes run across row ends without padding columns.
    // The band is double-buffered: the next item's copies are issued before this item's stem.
    template <int ACTA, int ACTD, int ACTP>
    __global__ __launch_bounds__(256, 2) void conv_stem_dwpw_kernel(StemDwPwArgs a) {
        using namespace sdp;
        constexpr int NSA  = 2; // stem: 9 taps x 4 channels in 2 32-deep steps
        constexpr int NI   = (BR * MBPR + 63) / 64;
        constexpr int NBW  = (NI + 3) / 4;
        constexpr int BAND = NI * 1024;
        constexpr int STEM = CB * IR * MSW * 8;
        constexpr int DWT  = CB * OR * MAXW * 8;
        constexpr int DWTO = STEM;       // the depthwise tile's offset from the stem tile
        constexpr int DUMPO = STEM + DWT; // 64 lanes x 8 bytes for the writes of lanes past a tile
        static_assert(2 * BAND + STEM + DWT + 512 <= 160 * 1024 / 3, "three workgroups per CU");
        __shared__ __attribute__((aligned(16))) unsigned char sm[2 * BAND + STEM + DWT + 512];
        unsigned char *stem = sm + 2 * BAND;
        unsigned char *dwt  = sm + 2 * BAND + STEM;

        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int ocw  = a.ocw, sw = ocw + 2, bc = 2 * sw + 2, bppr = sw + 1;
        const int tp   = BR * bppr;         // band pixel pairs
        const int sp   = IR * sw;           // stem tile pixels per slot
        const int op   = OR * ocw;          // output pixels per slot
        const float rsw = 1.f / (float) sw, rocw = 1.f / (float) ocw, rbppr = 1.f / (float) bppr;
        const int rblk = (a.OH + OR - 1) / OR, cblk = (a.OW + ocw - 1) / ocw;
        const int items = a.N * rblk * cblk;
        constexpr unsigned kInvalid = 0x80000000u;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);

        half8 wfa[NSA], wfp;
        {
            const half8 *pa = reinterpret_cast<const half8 *>(a.wa);
#pragma unroll
            for (int j = 0; j < NSA; ++j) wfa[j] = pa[j * 64 + lane];
            wfp = reinterpret_cast<const half8 *>(a.wp)[lane];
        }
        const int g = lane >> 4, px = lane & 15;
        // stem B operand: k = tap*4 + c; the lane's two 4-channel halves are taps 8j + 2g + q
        int  aoff[NSA][2];
        bool aval[NSA][2];
#pragma unroll
        for (int j = 0; j < NSA; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int tap = 8 * j + 2 * g + q;
                aval[j][q]    = tap < 9;
                aoff[j][q]    = tap < 9 ? (tap / 3) * bc + tap % 3 : 0;
            }
        // projection B operand: k = slot*4 + c over the depthwise tile's 4 slots (k >= 16: zero)
        const bool pval[2] = {2 * g < CB, 2 * g + 1 < CB};
        const int  poff[2] = {pval[0] ? (2 * g) * op : 0, pval[1] ? (2 * g + 1) * op : 0};
        // depthwise on MFMA: a 3x3 conv over 16 channels whose weights are zero off the diagonal,
        // k = tap*16 + channel in 5 32-deep steps. The lane's A fragment (row l%16, k = 32j + 8(l/16)
        // + e) holds the one tap weight of channel l%16 when that channel is among its 8 k.
        constexpr int NSD = 5;
        half8 wfd[NSD];
        {
            const int     m  = lane & 15;
            const half_t *wd = reinterpret_cast<const half_t *>(a.wd);
#pragma unroll
            for (int j = 0; j < NSD; ++j) {
                const int k0 = 32 * j + 8 * g, tap = k0 / 16, c0 = k0 % 16;
                half8     f  = {};
                const bool hit = tap < 9 && m >= c0 && m < c0 + 8 && m / 4 < a.cbm;
                const half_t w = hit ? wd[((m / 4) * 9 + tap) * 4 + m % 4] : (half_t) 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = c0 + e == m ? w : (half_t) 0.f;
                wfd[j] = f;
            }
        }
        // the lane's B halves: taps 2j + g/2, slots 2(g%2) + q of the stem tile
        int  doff[NSD][2];
        bool dval[NSD][2];
#pragma unroll
        for (int j = 0; j < NSD; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int tap = 2 * j + (g >> 1);
                dval[j][q]    = tap < 9;
                doff[j][q]    = tap < 9 ? (2 * (g & 1) + q) * sp + (tap / 3) * sw + tap % 3 : 0;
            }
        const float4v bsd = *reinterpret_cast<const float4v *>(a.bd + g * 4);
        const float4v bsa = *reinterpret_cast<const float4v *>(a.ba + g * 4);
        const float4v bsp = *reinterpret_cast<const float4v *>(a.bp + g * 4);

        // items: XCD-contiguous ranges (workgroup b runs on XCD b % 8)
        const int G = gridDim.x;
        const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3;
        const int gx  = (G >> 3) + ((G & 7) > xcd ? 1 : 0);
        const int pxc = xcd * (G >> 3) + min(xcd, G & 7);
        const int i0  = (int) ((long long) items * pxc / G) + lb;
        const int i1  = (int) ((long long) items * (pxc + gx) / G);
        // band row r, column c of item it <-> input (2 oy0 - 3 + r, 2 ox0 - 4 + c)
        auto copy_band = [&](int it, unsigned char *band) __attribute__((always_inline)) {
            const int cb = it % cblk, rest = it / cblk;
            const int ox0 = cb * ocw, oy0 = (rest % rblk) * OR, n = rest / rblk;
            const int iy0 = 2 * oy0 - 3, ix0 = 2 * ox0 - 4;
#pragma unroll
            for (int r = 0; r < NBW; ++r) {
                const int i   = r * 4 + wave;
                if (i >= NI) break; // wave-uniform
                const int p   = i * 64 + lane;
                const int row = fdiv(p, rbppr), pc = p - row * bppr;
                const int iy  = iy0 + row, ix = ix0 + 2 * pc;
                const bool ok = p < tp && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                const unsigned off = ok ? (unsigned) (((n * a.H + iy) * a.W + ix) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (band + i * 1024), 16, off, 0, 0, 0);
            }
        };
        if (i0 < i1) copy_band(i0, sm);
        int buf = 0;
        for (int it = i0; it < i1; it += gx, buf ^= 1) {
            const int cb = it % cblk, rest = it / cblk;
            const int ox0 = cb * ocw, oy0 = (rest % rblk) * OR, n = rest / rblk;
            unsigned char *band = sm + buf * BAND;
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // this wave's copies (and last item's stores) done
            __asm__ volatile("s_barrier" ::: "memory");        // every wave's copies landed; the other band is free
            if (it + gx < i1) copy_band(it + gx, sm + (buf ^ 1) * BAND);
            // Each phase takes two 16-pixel units per wave and pass, branch-free (reads of absent taps
            // are masked after the read; lanes past the tile write to the dump slot), so the two
            // units' LDS reads and MFMAs overlap.
            // stem: tile pixel q = r * sw + c <-> stem output (oy0 - 1 + r, ox0 - 1 + c), window at band row 2r, column 2c + 1
            auto stem_unit = [&](int u, float4v &acc, int &q, int &r, int &c) __attribute__((always_inline)) {
                q = u * 16 + px;
                r = fdiv(q, rsw);
                c = q - r * sw;
                const int base = 2 * r * bc + 2 * c + 1;
                acc = bsa; // the bias seeds the accumulator
#pragma unroll
                for (int j = 0; j < NSA; ++j) {
                    u32x2 v[2];
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const u32x2 t = *reinterpret_cast<const u32x2 *>(band + (base + aoff[j][q2]) * 8);
                        v[q2]         = aval[j][q2] ? t : u32x2 {0u, 0u};
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wfa[j], __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y)), acc, 0, 0, 0);
                }
            };
            auto stem_store = [&](float4v acc, int q, int r, int c) __attribute__((always_inline)) {
                const int  iy = oy0 - 1 + r, ix = ox0 - 1 + c;
                const bool in = ((unsigned) iy < (unsigned) a.OH) & ((unsigned) ix < (unsigned) a.OW) & (g < a.cbm); // no branches
                float4v    v  = acc;
                v.x = sdp_act<ACTA>(v.x, a.acta, a.loa, a.hia);
                v.y = sdp_act<ACTA>(v.y, a.acta, a.loa, a.hia);
                v.z = sdp_act<ACTA>(v.z, a.acta, a.loa, a.hia);
                v.w = sdp_act<ACTA>(v.w, a.acta, a.loa, a.hia);
                const int w = q < sp ? (g * sp + q) * 8 : DUMPO + lane * 8;
                *reinterpret_cast<u32x2 *>(stem + w) = in ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0u, 0u};
            };
            for (int u = wave; u * 16 < sp; u += 8) {
                float4v acc0, acc1;
                int     q0, r0, c0, q1, r1, c1;
                stem_unit(u, acc0, q0, r0, c0);
                stem_unit(u + 4, acc1, q1, r1, c1);
                stem_store(acc0, q0, r0, c0);
                stem_store(acc1, q1, r1, c1);
            }
            sdp_lds_barrier(); // the stem tile is complete
            // depthwise: output pixel p = orow * ocw + c, window at stem row orow, column c
            auto dw_unit = [&](int u, float4v &acc, int &p) __attribute__((always_inline)) {
                p = u * 16 + px;
                const int orow = fdiv(p, rocw), c = p - orow * ocw;
                const int base = orow * sw + c;
                acc = bsd;
#pragma unroll
                for (int j = 0; j < NSD; ++j) {
                    u32x2 v[2];
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const u32x2 t = *reinterpret_cast<const u32x2 *>(stem + (base + doff[j][q2]) * 8);
                        v[q2]         = dval[j][q2] ? t : u32x2 {0u, 0u};
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wfd[j], __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y)), acc, 0, 0, 0);
                }
            };
            auto dw_store = [&](float4v acc, int p) __attribute__((always_inline)) {
                float4v v = acc;
                v.x = sdp_act<ACTD>(v.x, a.actd, a.lod, a.hid);
                v.y = sdp_act<ACTD>(v.y, a.actd, a.lod, a.hid);
                v.z = sdp_act<ACTD>(v.z, a.actd, a.lod, a.hid);
                v.w = sdp_act<ACTD>(v.w, a.actd, a.lod, a.hid);
                const int w = p < op ? DWTO + (g * op + p) * 8 : DUMPO + lane * 8;
                *reinterpret_cast<u32x2 *>(stem + w) = g < a.cbm ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0u, 0u};
            };
            for (int u = wave; u * 16 < op; u += 8) {
                float4v acc0, acc1;
                int     p0, p1;
                dw_unit(u, acc0, p0);
                dw_unit(u + 4, acc1, p1);
                dw_store(acc0, p0);
                dw_store(acc1, p1);
            }
            sdp_lds_barrier(); // the depthwise tile is complete
            // projection: output pixel p from the depthwise tile, residual from the stem tile
            auto pw_unit = [&](int u) __attribute__((always_inline)) {
                const int p = u * 16 + px, orow = fdiv(p, rocw), c = p - orow * ocw;
                u32x2     v[2];
#pragma unroll
                for (int q2 = 0; q2 < 2; ++q2) {
                    const u32x2 t = *reinterpret_cast<const u32x2 *>(dwt + (poff[q2] + p) * 8);
                    v[q2]         = pval[q2] ? t : u32x2 {0u, 0u};
                }
                const u32x2 rv  = *reinterpret_cast<const u32x2 *>(stem + (g * sp + (orow + 1) * sw + c + 1) * 8);
                float4v     acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wfp, __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y)), bsp, 0, 0, 0);
                const int  oy = oy0 + orow, ox = ox0 + c;
                const bool pok = (p < op) & (oy < a.OH) & (ox < a.OW) & (g < a.cbo);
                float4v    o   = acc;
                if (a.res) o += h4_to_f4(__builtin_bit_cast(half4, rv));
                o.x = sdp_act<ACTP>(o.x, a.actp, a.lop, a.hip);
                o.y = sdp_act<ACTP>(o.y, a.actp, a.lop, a.hip);
                o.z = sdp_act<ACTP>(o.z, a.actp, a.lop, a.hip);
                o.w = sdp_act<ACTP>(o.w, a.actp, a.lop, a.hip);
                const unsigned off = pok ? (unsigned) ((((n * a.y_pstride + g) * a.OH + oy) * a.OW + ox) * 8) : kInvalid;
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(o)), yrs, off, 0, kStreamStore);
            };
            for (int u = wave; u * 16 < op; u += 8) {
                pw_unit(u);
                pw_unit(u + 4);
            }
            // no barrier here: the next item's stem and depthwise writes follow barriers that every
            // wave reaches after its projection, and its band was filled while this item ran
        }
    }

    typedef void (*StemDwPwKernelFn)(StemDwPwArgs);

    // the MobileNetV3 combination (hard-swish stem, ReLU depthwise, linear projection) at compile
    // time, every other one with activations chosen at run time
    static StemDwPwKernelFn stem_dwpw_pick(int acta, int actd, int actp) {
        if (acta == VKHIP_ACT_HARDSWISH && actd == VKHIP_ACT_RELU && actp == VKHIP_ACT_NONE)
            return conv_stem_dwpw_kernel<VKHIP_ACT_HARDSWISH, VKHIP_ACT_RELU, VKHIP_ACT_NONE>;
        return conv_stem_dwpw_kernel<-1, -1, -1>;
    }

} // namespace vkhip

using namespace vkhip;

extern "C" {

int vkhip_stem_dwpw_plan(const vkhip_conv_desc *cs, const vkhip_conv_desc *cd, const vkhip_conv_desc *cp, vkhip_conv_plan *ps, vkhip_conv_plan *pd,
                         vkhip_conv_plan *pp) {
    if (!cs || !cd || !cp || !ps || !pd || !pp) return set_error(VKHIP_ERR_INVALID, "stem_dwpw_plan: null argument");
    const bool stem_ok = cs->group == 1 && cs->KH == 3 && cs->KW == 3 && cs->SH == 2 && cs->SW == 2 && cs->PT == 1 && cs->PL == 1 && cs->DH == 1 &&
                         cs->DW == 1 && !cs->in_scale && !cs->has_res && cs->N > 0 && cs->Cin <= 4 && cs->Cin > 0 && cs->Cout >= 9 && cs->Cout <= 16 &&
                         cs->W % 2 == 0 && cs->OH == (cs->H - 1) / 2 + 1 && cs->OW == (cs->W - 1) / 2 + 1;
    const bool dw_ok = cd->group == cs->Cout && cd->Cin == cs->Cout && cd->Cout == cs->Cout && cd->KH == 3 && cd->KW == 3 && cd->SH == 1 &&
                       cd->SW == 1 && cd->PT == 1 && cd->PL == 1 && cd->DH == 1 && cd->DW == 1 && !cd->has_res && !cd->in_scale && cd->N == cs->N &&
                       cd->H == cs->OH && cd->W == cs->OW && cd->OH == cd->H && cd->OW == cd->W;
    const bool pw_ok = cp->group == 1 && cp->KH == 1 && cp->KW == 1 && cp->SH == 1 && cp->SW == 1 && !cp->PT && !cp->PL && cp->DH == 1 && cp->DW == 1 &&
                       !cp->in_scale && cp->N == cs->N && cp->Cin == cs->Cout && cp->H == cs->OH && cp->W == cs->OW && cp->OH == cp->H &&
                       cp->OW == cp->W && cp->Cout > 0 && cp->Cout <= 16 && (cp->has_res == 0 || (cp->has_res == 1 && cp->Cout == cs->Cout));
    if (!stem_ok || !dw_ok || !pw_ok)
        return set_error(VKHIP_ERR_UNSUPPORTED, "stem_dwpw: a 3x3 stride-2 stem over at most 4 channels to 9-16 (even input width), a 3x3 stride-1 "
                         "depthwise conv over them and a 1x1 projection to at most 16 channels (residual: the stem's output)");
    if ((int64_t) cs->N * cs->H * cs->W * 8 >= (1LL << 31) || (int64_t) cs->N * 4 * cs->OH * cs->OW * 8 >= (1LL << 31))
        return set_error(VKHIP_ERR_INVALID, "stem_dwpw: tensor >= 2 GiB");
    // stem and projection blobs: thin tile 43 (16 output rows); the depthwise blob: the depthwise packer
    vkhip_conv_desc e = *cp;
    e.W += e.W & 1;
    e.OW = e.W;
    e.has_res = 0;
    int rc = vkhip_conv_plan_make(cs, VKHIP_CONV_GEMM, 43, 0, ps);
    if (!rc) rc = vkhip_conv_plan_make(cd, VKHIP_CONV_DEPTHWISE, -1, 0, pd);
    if (!rc) rc = vkhip_conv_plan_make(&e, VKHIP_CONV_GEMM, 43, 0, pp);
    return rc;
}

int vkhip_stem_dwpw_forward(const vkhip_conv_desc *cs, const vkhip_conv_desc *cd, const vkhip_conv_desc *cp, const void *x, const void *blob_s,
                            const void *blob_d, const void *blob_p, void *y, int64_t y_pstride, vkhip_stream_t s) {
    if (!cs || !cd || !cp || !x || !blob_s || !blob_d || !blob_p || !y) return set_error(VKHIP_ERR_INVALID, "stem_dwpw_forward: null argument");
    vkhip_conv_plan ps, pd, pp;
    int rc = vkhip_stem_dwpw_plan(cs, cd, cp, &ps, &pd, &pp);
    if (rc) return rc;
    const int     cbo = (int) ceil_div(cp->Cout, 4);
    const int64_t yps = y_pstride > 0 ? y_pstride : cbo;
    if (yps < cbo) return set_error(VKHIP_ERR_INVALID, "stem_dwpw_forward: plane stride below the channel blocks");
    const int64_t oplane = (int64_t) cs->OH * cs->OW * 8;
    if ((int64_t) cs->N * yps * oplane >= (1LL << 31)) return set_error(VKHIP_ERR_INVALID, "stem_dwpw_forward: view >= 2 GiB");
    StemDwPwArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x  = (const uint2 *) x;
    a.y  = (uint2 *) y;
    // thin blobs: bias [16] fp32 at 0, weights at 256; depthwise blob: bias [Cb*4] at 0, weights at align256(Cb * 16)
    a.ba = (const float *) blob_s;
    a.wa = (const half_t *) ((const char *) blob_s + 256);
    a.bp = (const float *) blob_p;
    a.wp = (const half_t *) ((const char *) blob_p + 256);
    a.bd = (const float *) blob_d;
    a.wd = (const uint2 *) ((const char *) blob_d + 256); // align256(4 slots * 16 bytes)
    a.N = cs->N; a.H = cs->H; a.W = cs->W; a.OH = cs->OH; a.OW = cs->OW;
    a.cbm = (int) ceil_div(cs->Cout, 4); a.cbo = cbo; a.y_pstride = (int) yps;
    a.x_bytes = (unsigned) ((int64_t) cs->N * cs->H * cs->W * 8);
    a.y_bytes = (unsigned) (((int64_t) (cs->N - 1) * yps + cbo) * oplane);
    a.acta = cs->act; a.loa = cs->act_lo; a.hia = cs->act_hi;
    a.actd = cd->act; a.lod = cd->act_lo; a.hid = cd->act_hi;
    a.actp = cp->act; a.lop = cp->act_lo; a.hip = cp->act_hi;
    a.res  = cp->has_res;
    StemDwPwKernelFn fn = stem_dwpw_pick(cs->act, cd->act, cp->act);
    const int cblk = (int) ceil_div(cs->OW, sdp::MAXW);
    a.ocw = (int) ceil_div(cs->OW, cblk);
    const int64_t items = (int64_t) cs->N * ceil_div(cs->OH, sdp::OR) * cblk;
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
    return check_launch("stem_dwpw");
}

} // extern "C"
