// Two 3x3 stride-1 pad-1 convs in a row over at most 32 channels, in one kernel: the YOLOv8
// bottleneck (cv1 -> cv2, optionally + its input: the shortcut) and the C2f head pairs. Run as
// two thin-kernel launches, the first conv writes its whole output to HBM and the second reads
// it back with a third of the rows twice (plus the residual once more); at 160x160 and 80x80
// both launches are short enough that launch and pipeline-fill latency dominate. Here:
//   * one persistent workgroup per CU slot walks work items of 4 output rows x 64 columns (items
//     in XCD-contiguous ranges, so the input rows vertically adjacent items share come from L2);
//   * the item's input band (8 rows x 82 columns, every channel slot) is copied global->LDS by
//     buffer-load-to-LDS; the first conv computes its output over the 6 x 80 pixels the second
//     conv's 3x3 window needs (16-pixel MFMA column tiles; positions outside the image are set
//     to zero, the second conv's padding) and leaves it in LDS as fp16, rounded exactly like the
//     separate conv's fp16 store;
//   * the second conv reads that tile from LDS, adds bias, activation and (shortcut) the input
//     pixel from the band after the activation, and stores 8-byte NC4HW4 slots;
//   * both convs use v_mfma_f32_16x16x32_f16 with their weights in registers (the thin kernel's
//     fragment layout and packed blob).
// Several workgroups share a CU (the band is single-buffered), so one's copies overlap another's
// math.
// Reference semantics: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) twice, then Add
// (src/backend/cpu/ops/add.cpp) for the shortcut.
#include "conv_kernels.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace vkhip {

    struct PairArgs {
        const uint2  *x;
        uint2        *y;
        const half_t *w1, *w2; // thin-kernel fragment layout [m_frag][step][lane][8 halves]
        const float  *b1, *b2; // [MT*16]
        int           N, H, W, Cb;
        int           x_pstride, y_pstride;
        unsigned      x_bytes, y_bytes;
        int           act1, act2;
        float         lo1, hi1, lo2, hi2;
        int           res; // 1: y = act2(conv2) + x
    };

    namespace pair {
        constexpr int OR   = 4;            // output rows per item (one per wave)
        constexpr int OCW  = 64;           // output columns per item
        constexpr int IR   = OR + 2;       // rows of the intermediate tile
        constexpr int IT   = 5;            // 16-pixel column tiles of the intermediate tile
        constexpr int ICW  = IT * 16;      // its columns (OCW + 2 needed)
        constexpr int BR   = OR + 4;       // band rows
        constexpr int BC   = ICW + 2;      // band columns (even: whole pixel pairs)
        constexpr int BPPR = BC / 2;       // pixel pairs per band row
    } // namespace pair

    template <int ACT>
    __device__ __forceinline__ float pair_act(float v, int act, float lo, float hi) {
        return apply_act(v, ACT >= 0 ? ACT : act, lo, hi);
    }

    template <int CB, int ACT1, int ACT2>
    __global__ __launch_bounds__(256, 2) void conv_pair_kernel(PairArgs a) {
        using namespace pair;
        constexpr int MT     = CB / 4;                 // 16-channel fragments (both convs)
        constexpr int CIN4   = CB * 4;
        constexpr int NSTEPS = (9 * CIN4 + 31) / 32;   // 32-deep MFMA steps
        constexpr int TP     = CB * BR * BPPR;         // pixel pairs of one band
        constexpr int NI     = (TP + 63) / 64;         // 1 KB copies of one band
        constexpr int NBW    = (NI + 3) / 4;           // copies per wave
        constexpr int BAND   = NBW * 4 * 1024;
        constexpr int INTER  = CB * IR * ICW * 8;      // intermediate tile bytes
        static_assert(CB == 4 || CB == 8, "16 or 32 channels");
        static_assert(BAND + INTER <= 80 * 1024, "two workgroups per CU");
        __shared__ __attribute__((aligned(16))) unsigned char sm[BAND + INTER];
        unsigned char *band  = sm;
        unsigned char *inter = sm + BAND;

        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int H = a.H, W = a.W;
        const int rblk = (H + OR - 1) / OR, cblk = (W + OCW - 1) / OCW;
        const int items = a.N * rblk * cblk;
        constexpr unsigned kInvalid = 0x80000000u;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);

        half8 wf1[MT][NSTEPS], wf2[MT][NSTEPS];
        {
            const half8 *p1 = reinterpret_cast<const half8 *>(a.w1);
            const half8 *p2 = reinterpret_cast<const half8 *>(a.w2);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int j = 0; j < NSTEPS; ++j) {
                    wf1[m][j] = p1[(m * NSTEPS + j) * 64 + lane];
                    wf2[m][j] = p2[(m * NSTEPS + j) * 64 + lane];
                }
        }
        // per (step, half): the pixel offset of this lane's 4-channel slot and tap relative to the
        // output pixel's window origin, in band (b) and intermediate (i) coordinates; -1 = zero pad
        int boff[NSTEPS][2], ioff[NSTEPS][2];
#pragma unroll
        for (int j = 0; j < NSTEPS; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if constexpr (CB == 8) {
                    // 32 channels: step j is tap j, the lane's slot 2(l/16) + q; written so that
                    // the tap part is a constant (an LDS instruction offset, not a register)
                    const int slot = 2 * (lane >> 4) + q;
                    boff[j][q]     = slot * BR * BC + (j / 3) * BC + j % 3;
                    ioff[j][q]     = slot * IR * ICW + (j / 3) * ICW + j % 3;
                } else {
                    const int k   = 32 * j + 8 * (lane >> 4) + 4 * q;
                    const int tap = k / CIN4, slot = (k % CIN4) / 4;
                    boff[j][q]    = tap < 9 ? (slot * BR + tap / 3) * BC + tap % 3 : -1;
                    ioff[j][q]    = tap < 9 ? (slot * IR + tap / 3) * ICW + tap % 3 : -1;
                }
            }

        auto item_pos = [&](int it, int &n, int &oy0, int &ox0) __attribute__((always_inline)) {
            const int cb = it % cblk, rest = it / cblk;
            ox0 = cb * OCW;
            oy0 = (rest % rblk) * OR;
            n   = rest / rblk;
        };
        // band row r, column c <-> input (oy0 - 2 + r, ox0 - 2 + c)
        auto issue_band = [&](int n, int oy0, int ox0) __attribute__((always_inline)) {
#pragma unroll
            for (int r = 0; r < NBW; ++r) {
                const int i   = r * 4 + wave;
                const int p   = i * 64 + lane;
                const int pc  = p % BPPR, rs = p / BPPR;
                const int row = rs % BR, slot = rs / BR;
                const int iy  = oy0 - 2 + row, ix = ox0 - 2 + 2 * pc;
                const bool ok = p < TP && slot < a.Cb && iy >= 0 && iy < H && ix >= 0 && ix < W;
                const unsigned off = ok ? (unsigned) ((((n * a.x_pstride + slot) * H + iy) * W + ix) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (band + i * 1024), 16, off, 0, 0, 0);
            }
        };
        auto mma = [&](const unsigned char *src, const int (&off)[NSTEPS][2], const half8 (&wf)[MT][NSTEPS], int base, float4v (&acc)[MT])
            __attribute__((always_inline)) {
            // acc holds the biases on entry; absent taps (off < 0) read the window origin and are
            // masked after the read (no branches)
#pragma unroll
            for (int j = 0; j < NSTEPS; ++j) {
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
        float4v bs1[MT], bs2[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            bs1[m] = *reinterpret_cast<const float4v *>(a.b1 + (m * 4 + g) * 4);
            bs2[m] = *reinterpret_cast<const float4v *>(a.b2 + (m * 4 + g) * 4);
        }

        // items: XCD-contiguous ranges (workgroup b runs on XCD b % 8)
        const int G = gridDim.x;
        const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3;
        const int gx  = (G >> 3) + ((G & 7) > xcd ? 1 : 0);
        const int pxc = xcd * (G >> 3) + min(xcd, G & 7);
        const int i0  = (int) ((long long) items * pxc / G) + lb;
        const int i1  = (int) ((long long) items * (pxc + gx) / G);
        for (int it = i0; it < i1; it += gx) {
            int n, oy0, ox0;
            item_pos(it, n, oy0, ox0);
            issue_band(n, oy0, ox0);
            // every copy of this wave (and every store of the previous item) complete, then all waves'
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
            __asm__ volatile("s_barrier" ::: "memory");
            // first conv over the 6 x 80 intermediate tile: (row, column tile) units dealt to the waves
            // two units per pass, so their LDS reads and MFMAs overlap (past the end, the second
            // unit repeats the last one: the same values to the same place)
            auto first_unit = [&](int u) __attribute__((always_inline)) {
                const int r = u / IT, t = u % IT;
                const int c = t * 16 + px;                       // intermediate column
                float4v   acc[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] = bs1[m];
                mma(band, boff, wf1, r * BC + c, acc);
                const int  iy = oy0 - 1 + r, ix = ox0 - 1 + c;
                const bool in = ((unsigned) iy < (unsigned) H) & ((unsigned) ix < (unsigned) W);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const int ocb = m * 4 + g;
                    float4v   v   = acc[m];
                    v.x = pair_act<ACT1>(v.x, a.act1, a.lo1, a.hi1);
                    v.y = pair_act<ACT1>(v.y, a.act1, a.lo1, a.hi1);
                    v.z = pair_act<ACT1>(v.z, a.act1, a.lo1, a.hi1);
                    v.w = pair_act<ACT1>(v.w, a.act1, a.lo1, a.hi1);
                    // outside the image: the second conv's zero padding; channel slots past Cb: zero
                    const u32x2 h = in & (ocb < a.Cb) ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0u, 0u};
                    *reinterpret_cast<u32x2 *>(inter + ((ocb * IR + r) * ICW + c) * 8) = h;
                }
            };
            if constexpr (CB == 8) {
                for (int u = wave; u < IR * IT; u += 4) first_unit(u);
            } else {
                for (int u = wave; u < IR * IT; u += 8) {
                    first_unit(u);
                    first_unit(min(u + 4, IR * IT - 1));
                }
            }
            __syncthreads(); // the intermediate tile is complete
            // second conv: output row oy0 + wave, 4 column tiles
            const int oy = oy0 + wave;
#pragma unroll 1
            for (int t = 0; t < OCW / 16; ++t) {
                const int c = t * 16 + px; // output column within the item
                float4v   acc[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] = bs2[m];
                mma(inter, ioff, wf2, wave * ICW + c, acc);
                const int  ox  = ox0 + c;
                const bool pok = (oy < H) & (ox < W);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const int ocb = m * 4 + g;
                    float4v   v   = acc[m];
                    v.x = pair_act<ACT2>(v.x, a.act2, a.lo2, a.hi2);
                    v.y = pair_act<ACT2>(v.y, a.act2, a.lo2, a.hi2);
                    v.z = pair_act<ACT2>(v.z, a.act2, a.lo2, a.hi2);
                    v.w = pair_act<ACT2>(v.w, a.act2, a.lo2, a.hi2);
                    if (a.res) v += h4_to_f4(__builtin_bit_cast(half4, *reinterpret_cast<const u32x2 *>(band + ((ocb * BR + wave + 2) * BC + c + 2) * 8)));
                    const unsigned off = pok && ocb < a.Cb ? (unsigned) ((((n * a.y_pstride + ocb) * H + oy) * W + ox) * 8) : kInvalid;
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, off, 0, kStreamStore);
                }
            }
            __syncthreads(); // band and intermediate tile free for the next item
        }
    }

    typedef void (*PairKernelFn)(PairArgs);

    template <int CB>
    static PairKernelFn pair_pick(int act1, int act2) {
        if (act1 == act2) {
            switch (act1) {
                case VKHIP_ACT_NONE: return conv_pair_kernel<CB, VKHIP_ACT_NONE, VKHIP_ACT_NONE>;
                case VKHIP_ACT_RELU: return conv_pair_kernel<CB, VKHIP_ACT_RELU, VKHIP_ACT_RELU>;
                case VKHIP_ACT_SILU: return conv_pair_kernel<CB, VKHIP_ACT_SILU, VKHIP_ACT_SILU>;
                default: break;
            }
        }
        return conv_pair_kernel<CB, -1, -1>; // activations chosen at run time
    }

} // namespace vkhip

using namespace vkhip;

static bool pair_conv_ok(const vkhip_conv_desc *c) {
    return c->group == 1 && c->KH == 3 && c->KW == 3 && c->SH == 1 && c->SW == 1 && c->PT == 1 && c->PL == 1 && c->DH == 1 && c->DW == 1 &&
           c->OH == c->H && c->OW == c->W && !c->in_scale && c->N > 0 && c->H > 0 && c->W > 0;
}

// channel slots of the pair kernel for C channels (the thin kernel's rounding), or 0
static int pair_cb(int C) {
    const int cb = thin_cinb(ceil_div(C, 4));
    return C > 0 && C <= 32 && (cb == 4 || cb == 8) ? cb : 0;
}

extern "C" {

int vkhip_conv3x3_pair_plan(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, vkhip_conv_plan *p1, vkhip_conv_plan *p2) {
    if (!c1 || !c2 || !p1 || !p2) return set_error(VKHIP_ERR_INVALID, "conv3x3_pair_plan: null argument");
    if (!pair_conv_ok(c1) || !pair_conv_ok(c2) || c1->has_res || (c2->has_res != 0 && c2->has_res != 2))
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3_pair: two dense 3x3 stride-1 pad-1 convs, no input scale, the second with has_res 0 or 2");
    if (c2->N != c1->N || c2->H != c1->H || c2->W != c1->W || c2->Cin != c1->Cout || c1->Cout != c1->Cin || c2->Cout != c1->Cin)
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3_pair: the second conv reads the first's output and every channel count is equal");
    const int cb = pair_cb(c1->Cin);
    if (!cb || c1->W % 2) return set_error(VKHIP_ERR_UNSUPPORTED, "conv3x3_pair: 9-32 channels and an even width");
    if ((int64_t) c1->N * ceil_div(c1->Cin, 4) * c1->H * c1->W * 8 >= (1LL << 31)) return set_error(VKHIP_ERR_INVALID, "conv3x3_pair: tensor >= 2 GiB");
    // the blobs are the thin tiles' (16 or 32 output rows)
    const int tile = cb == 4 ? 43 : 44;
    vkhip_conv_desc d1 = *c1, d2 = *c2;
    d2.has_res = 0;
    int rc = vkhip_conv_plan_make(&d1, VKHIP_CONV_GEMM, tile, 0, p1);
    if (!rc) rc = vkhip_conv_plan_make(&d2, VKHIP_CONV_GEMM, tile, 0, p2);
    return rc;
}

int vkhip_conv3x3_pair_forward(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, const void *x, int64_t x_pstride, const void *blob1,
                               const void *blob2, void *y, int64_t y_pstride, vkhip_stream_t s) {
    if (!c1 || !c2 || !x || !blob1 || !blob2 || !y) return set_error(VKHIP_ERR_INVALID, "conv3x3_pair_forward: null argument");
    vkhip_conv_plan p1, p2;
    int rc = vkhip_conv3x3_pair_plan(c1, c2, &p1, &p2);
    if (rc) return rc;
    const int cb = pair_cb(c1->Cin), Cb = (int) ceil_div(c1->Cin, 4);
    const int64_t xps = x_pstride > 0 ? x_pstride : Cb, yps = y_pstride > 0 ? y_pstride : Cb;
    if (xps < Cb || yps < Cb) return set_error(VKHIP_ERR_INVALID, "conv3x3_pair_forward: plane stride below the channel blocks");
    const int64_t plane = (int64_t) c1->H * c1->W * 8;
    if ((int64_t) c1->N * std::max(xps, yps) * plane >= (1LL << 31)) return set_error(VKHIP_ERR_INVALID, "conv3x3_pair_forward: view >= 2 GiB");
    PairArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = (const uint2 *) x;
    a.y = (uint2 *) y;
    // blob: bias [Coutp] fp32 at 0, weights at align256(Coutp * 4) (Coutp = the tile's 16 or 32 rows)
    const size_t wofs = ((size_t) cb * 4 * 4 + 255) & ~(size_t) 255;
    a.b1 = (const float *) blob1;
    a.b2 = (const float *) blob2;
    a.w1 = (const half_t *) ((const char *) blob1 + wofs);
    a.w2 = (const half_t *) ((const char *) blob2 + wofs);
    a.N = c1->N; a.H = c1->H; a.W = c1->W; a.Cb = Cb;
    a.x_pstride = (int) xps; a.y_pstride = (int) yps;
    a.x_bytes = (unsigned) (((int64_t) (c1->N - 1) * xps + Cb) * plane);
    a.y_bytes = (unsigned) (((int64_t) (c1->N - 1) * yps + Cb) * plane);
    a.act1 = c1->act; a.lo1 = c1->act_lo; a.hi1 = c1->act_hi;
    a.act2 = c2->act; a.lo2 = c2->act_lo; a.hi2 = c2->act_hi;
    a.res  = c2->has_res == 2;
    PairKernelFn fn = cb == 4 ? pair_pick<4>(c1->act, c2->act) : pair_pick<8>(c1->act, c2->act);
    const int64_t items = (int64_t) c1->N * ceil_div(c1->H, pair::OR) * ceil_div(c1->W, pair::OCW);
    // as many workgroups as the device holds at once, at most one per item
    static std::mutex                               mu;
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
    return check_launch("conv3x3_pair");
}

} // extern "C"
