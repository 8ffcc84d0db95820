// A MobileNetV3 stem and its first block in one kernel: a 3x3 stride-2 conv over at most 4 input
// channels to 9-16 channels, a 3x3 stride-1 depthwise conv over those channels, and the 1x1
// projection back to at most 16 channels with the stem's output as the residual (MobileNetV3-Large:
// 3 -> 16 hard-swish at 224x224, dw 3x3 ReLU, 16 -> 16 + x). Run as three launches (stem, dw,
// 1x1), the 16-channel tensors at 112x112 go through HBM five times; here they stay in LDS:
//   * one persistent workgroup per CU slot walks items of 2 output rows x 64 columns
//     (XCD-contiguous item ranges);
//   * the stem's input band (9 rows x 162 columns of the input's 4-channel slot) arrives in LDS by
//     buffer-load-to-LDS; the stem computes the 4 x 80 pixels the depthwise window needs
//     (16x16x32 MFMA, weights in registers) into LDS as fp16, zero outside the image (the
//     depthwise conv's padding), rounded like the separate conv's store;
//   * the depthwise conv (VALU, fp32 sums of fp16 taps) writes its 2 x 64 tile to LDS as fp16;
//   * the projection (one 32-deep MFMA step per 16 pixels) adds bias, the stem's pixel from LDS as
//     the residual, and its activation, and stores 8-byte NC4HW4 slots.
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
        int           OH, OW;   // stem / block output
        int           cbm, cbo; // channel slots: stem output, projection output
        int           y_pstride;
        unsigned      x_bytes, y_bytes;
        int           acta, actd, actp, res;
        float         loa, hia, lod, hid, lop, hip;
    };

    namespace sdp {
        constexpr int OR   = 2;          // output rows per item
        constexpr int OCW  = 64;         // output columns per item
        constexpr int IR   = OR + 2;     // stem rows the depthwise window needs
        constexpr int IT   = 5;          // 16-pixel column tiles of the stem tile (66 of 80 used)
        constexpr int ICW  = IT * 16;
        constexpr int BR   = 2 * IR + 1; // input band rows
        constexpr int BC   = 2 * ICW + 2; // input band columns (even: whole pixel pairs)
        constexpr int BPPR = BC / 2;
        constexpr int CB   = 4;          // channel slots of the block (9-16 channels)
    } // namespace sdp

    template <int ACT>
    __device__ __forceinline__ float sdp_act(float v, int act, float lo, float hi) {
        return apply_act(v, ACT >= 0 ? ACT : act, lo, hi);
    }

    template <int ACTA, int ACTD, int ACTP>
    __global__ __launch_bounds__(256, 2) void conv_stem_dwpw_kernel(StemDwPwArgs a) {
        using namespace sdp;
        constexpr int NSA   = 2; // stem: 9 taps x 4 channels in 2 32-deep steps
        constexpr int TP    = BR * BPPR;
        constexpr int NI    = (TP + 63) / 64;
        constexpr int NBW   = (NI + 3) / 4;
        constexpr int BAND  = NBW * 4 * 1024;
        constexpr int STEM  = CB * IR * ICW * 8;
        constexpr int DWT   = CB * OR * OCW * 8;
        static_assert(CB * OR * OCW == 2 * 256, "the depthwise loop: two pixels per thread");
        __shared__ __attribute__((aligned(16))) unsigned char sm[BAND + STEM + DWT];
        unsigned char *band = sm;
        unsigned char *stem = sm + BAND;
        unsigned char *dwt  = sm + BAND + STEM;

        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int rblk = (a.OH + OR - 1) / OR, cblk = (a.OW + OCW - 1) / OCW;
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
        int aoff[NSA][2];
#pragma unroll
        for (int j = 0; j < NSA; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int tap = 8 * j + 2 * g + q;
                aoff[j][q]    = tap < 9 ? (tap / 3) * BC + tap % 3 : -1;
            }
        // projection B operand: k = slot*4 + c over the depthwise tile's 4 slots (k >= 16: zero)
        const int poff[2] = {2 * g < CB ? (2 * g) * OR * OCW : -1, 2 * g + 1 < CB ? (2 * g + 1) * OR * OCW : -1};
        // depthwise: wave w computes slot w, its lanes consecutive pixels (conflict-free LDS rows)
        const int dslot = wave;
        float4v   dww[9];
        {
            const uint2 *w = a.wd + dslot * 9;
#pragma unroll
            for (int t = 0; t < 9; ++t) dww[t] = dslot < a.cbm ? h4_to_f4(u2_as_h4(w[t])) : float4v {0.f, 0.f, 0.f, 0.f}; // the blob holds cbm slots
        }
        const float4v dwb = *reinterpret_cast<const float4v *>(a.bd + dslot * 4);

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
            // band row r, column c <-> input (2 oy0 - 3 + r, 2 ox0 - 4 + c)
            const int iy0 = 2 * oy0 - 3, ix0 = 2 * ox0 - 4;
#pragma unroll
            for (int r = 0; r < NBW; ++r) {
                const int i   = r * 4 + wave;
                const int p   = i * 64 + lane;
                const int pc  = p % BPPR, row = p / BPPR;
                const int iy  = iy0 + row, ix = ix0 + 2 * pc;
                const bool ok = p < TP && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                const unsigned off = ok ? (unsigned) (((n * a.H + iy) * a.W + ix) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (band + i * 1024), 16, off, 0, 0, 0);
            }
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // this wave's copies (and last item's stores) done
            __asm__ volatile("s_barrier" ::: "memory");        // every wave's copies landed
            // stem: tile pixel (r, c) <-> stem output (oy0 - 1 + r, ox0 - 1 + c), window at band row 2r, column 2c + 1
            for (int u = wave; u < IR * IT; u += 4) {
                const int r = u / IT, c = (u % IT) * 16 + px;
                float4v   acc = {0.f, 0.f, 0.f, 0.f};
                const int base = 2 * r * BC + 2 * c + 1;
#pragma unroll
                for (int j = 0; j < NSA; ++j) {
                    u32x2 v[2];
#pragma unroll
                    for (int q = 0; q < 2; ++q) v[q] = aoff[j][q] >= 0 ? *reinterpret_cast<const u32x2 *>(band + (base + aoff[j][q]) * 8) : u32x2 {0u, 0u};
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wfa[j], __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y)), acc, 0, 0, 0);
                }
                const int  iy = oy0 - 1 + r, ix = ox0 - 1 + c;
                const bool in = iy >= 0 && iy < a.OH && ix >= 0 && ix < a.OW && g < a.cbm;
                float4v    v  = acc + *reinterpret_cast<const float4v *>(a.ba + g * 4);
                v.x = sdp_act<ACTA>(v.x, a.acta, a.loa, a.hia);
                v.y = sdp_act<ACTA>(v.y, a.acta, a.loa, a.hia);
                v.z = sdp_act<ACTA>(v.z, a.acta, a.loa, a.hia);
                v.w = sdp_act<ACTA>(v.w, a.acta, a.loa, a.hia);
                *reinterpret_cast<u32x2 *>(stem + ((g * IR + r) * ICW + c) * 8) = in ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0u, 0u};
            }
            __syncthreads(); // the stem tile is complete
            // depthwise: output (oy0 + orow, ox0 + c) of slot dslot, window at stem row orow, column c
#pragma unroll
            for (int k = 0; k < CB * OR * OCW / 256; ++k) {
                const int pix = lane + k * 64; // 0 .. OR*OCW-1
                const int orow = pix / OCW, c = pix % OCW;
                const unsigned char *s = stem + ((dslot * IR + orow) * ICW + c) * 8;
                float4v acc = dwb;
#pragma unroll
                for (int t = 0; t < 9; ++t) acc += dww[t] * h4_to_f4(__builtin_bit_cast(half4, *reinterpret_cast<const u32x2 *>(s + ((t / 3) * ICW + t % 3) * 8)));
                acc.x = sdp_act<ACTD>(acc.x, a.actd, a.lod, a.hid);
                acc.y = sdp_act<ACTD>(acc.y, a.actd, a.lod, a.hid);
                acc.z = sdp_act<ACTD>(acc.z, a.actd, a.lod, a.hid);
                acc.w = sdp_act<ACTD>(acc.w, a.actd, a.lod, a.hid);
                *reinterpret_cast<u32x2 *>(dwt + ((dslot * OR + orow) * OCW + c) * 8) = dslot < a.cbm ? __builtin_bit_cast(u32x2, f4_to_h4(acc)) : u32x2 {0u, 0u};
            }
            __syncthreads(); // the depthwise tile is complete
            // projection: output (oy0 + orow, ox0 + c) from the depthwise tile's pixel, residual from the stem tile
#pragma unroll 1
            for (int u = wave; u < OR * (OCW / 16); u += 4) {
                const int orow = u / (OCW / 16), c = (u % (OCW / 16)) * 16 + px;
                u32x2     v[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) v[q] = poff[q] >= 0 ? *reinterpret_cast<const u32x2 *>(dwt + (poff[q] + orow * OCW + c) * 8) : u32x2 {0u, 0u};
                float4v acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wfp, __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y)),
                                                                     float4v {0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                const int  oy = oy0 + orow, ox = ox0 + c;
                const bool pok = oy < a.OH && ox < a.OW;
                float4v    o   = acc + *reinterpret_cast<const float4v *>(a.bp + g * 4);
                if (a.res) o += h4_to_f4(__builtin_bit_cast(half4, *reinterpret_cast<const u32x2 *>(stem + ((g * IR + orow + 1) * ICW + c + 1) * 8)));
                o.x = sdp_act<ACTP>(o.x, a.actp, a.lop, a.hip);
                o.y = sdp_act<ACTP>(o.y, a.actp, a.lop, a.hip);
                o.z = sdp_act<ACTP>(o.z, a.actp, a.lop, a.hip);
                o.w = sdp_act<ACTP>(o.w, a.actp, a.lop, a.hip);
                const unsigned off = pok && g < a.cbo ? (unsigned) ((((n * a.y_pstride + g) * a.OH + oy) * a.OW + ox) * 8) : kInvalid;
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(o)), yrs, off, 0, kStreamStore);
            }
            // no barrier here: the next item's band copies overwrite only the band (last read before
            // the stem tile's barrier), and its stem and depthwise writes follow barriers that every
            // wave reaches after its projection
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
    const int64_t items = (int64_t) cs->N * ceil_div(cs->OH, sdp::OR) * ceil_div(cs->OW, sdp::OCW);
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
