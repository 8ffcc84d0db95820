// Thin-channel direct convolution for gfx950: 3x3 (pad 1) or 1x1 (pad 0) convs, stride 1 or 2,
// over at most 32 input and 64 output channels (the first layers of YOLOv8n and the MobileNet
// stems: 3->16, 16->32, 16->16, 32->32 at 160x160 and above), and 7x7 pad-3 convs over at most 4
// input channels (the ResNet stem, 3->64 at stride 2). The implicit-GEMM tiles waste most
// of a 32-row MFMA tile and a whole LDS stage per workgroup on such layers, and the tiles are too
// short to overlap one workgroup's load latency with another's stores, so they run at ~0.1-0.25
// of HBM. Here:
//   * MFMA v_mfma_f32_16x16x32_f16 (M = 16 output channels, N = 16 output pixels of one row,
//     K = 32 values of (tap, channel)), so a 16-channel conv wastes nothing; the whole reduction
//     of the output channel blocks is at most 28 fragments held in registers (the weights are
//     loaded once per workgroup);
//   * one persistent workgroup per CU slot walks work items of 4 output rows x 64 columns; the
//     input bands of the next NBUF-1 items (rows (4-1)*S + K, 64*S + K + 1 columns, every channel
//     slot) are copied global->LDS by buffer-load-to-LDS while the current item computes from
//     another buffer of an NBUF-deep ring, and the current item's stores are issued after those
//     copies, so a wait for a band never waits for the stores issued after it;
//   * the accumulator layout of the 16x16 MFMA (lane l: pixel l%16, channels 4(l/16)..+3) is one
//     NC4HW4 slot of one pixel, so every store is one 8-byte write of 4 channels;
//   * RES (3x3 stride 1 only): a residual of the output's shape and plane stride is copied into the
//     same ring buffer as the item's input band (one 4 x 64 tile per output channel slot), so it
//     arrives under the band's wait, and is added before (has_res 1) or after (has_res 2) the
//     activation.
// Reference semantics: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) — bias, activation, fp16 store.
#include "conv_kernels.h"

namespace vkhip {

    namespace thin {
        constexpr int OR  = 4;  // output rows per work item (one per wave)
        constexpr int OCW = 64; // output columns per work item (4 pixel tiles of 16)
        template <int K, int S>
        struct Band {
            static constexpr int PAD  = K / 2;
            static constexpr int COFF = (PAD + 1) & ~1;                     // band column of input column ox0*S (even start, >= PAD)
            static constexpr int ROWS = (OR - 1) * S + K;
            static constexpr int COLS = ((OCW - 1) * S + K + (COFF - PAD) + 1) & ~1; // even: whole pixel pairs
            static constexpr int PPR  = COLS / 2;                           // pixel pairs per band row
        };
    } // namespace thin

    // LDS bytes of one band buffer of the thin kernel (input band only)
    template <int CINB, int K, int S>
    constexpr int thin_band_bytes() {
        using B = thin::Band<K, S>;
        return ((CINB * B::ROWS * B::PPR + 63) / 64 + 3) / 4 * 4 * 1024;
    }
    // 1 KB copies per wave of one item's residual tile (MT*4 slots x 4 rows x 64 pixels, 8 bytes each)
    template <int MT, bool RES>
    constexpr int thin_res_copies() {
        return RES ? MT * 2 : 0;
    }

    template <int CINB, int MT, int K, int S, int NBUF, bool RES>
    __global__ __launch_bounds__(256, 2) void conv_thin_kernel(GemmArgs a) {
        using B = thin::Band<K, S>;
        constexpr int OR = thin::OR, OCW = thin::OCW;
        constexpr int CIN4   = CINB * 4;
        constexpr int NSTEPS = (K * K * CIN4 + 31) / 32;   // 32-deep MFMA steps
        constexpr int TP     = CINB * B::ROWS * B::PPR;    // pixel pairs of one band
        constexpr int NI     = (TP + 63) / 64;             // 1 KB copies of one band
        constexpr int NBW    = (NI + 3) / 4;               // copies per wave (the surplus ones copy zeros)
        constexpr int NRW    = thin_res_copies<MT, RES>(); // residual copies per wave
        constexpr int RBASE  = NBW * 4 * 1024;             // residual tile's offset in a ring buffer
        constexpr int BAND   = (NBW + NRW) * 4 * 1024;     // LDS bytes of one ring buffer
        static_assert(RBASE == thin_band_bytes<CINB, K, S>() && (NBUF == 2 || NBUF == 3), "band ring");
        static_assert(!RES || (K == 3 && S == 1), "residual: 3x3 stride 1 only");
        static_assert(NBUF * BAND <= 160 * 1024, "band ring fits LDS");
        static_assert(MT * NSTEPS <= 28, "weights fit the register budget");
        __shared__ __attribute__((aligned(16))) unsigned char sm[NBUF * BAND];

        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int OH = a.OHW / a.OW, OW = a.OW, H = a.H, W = a.W;
        const int N      = a.P / a.OHW;
        const int rblk   = (OH + OR - 1) / OR, cblk = (OW + OCW - 1) / OCW;
        const int items  = N * rblk * cblk;
        constexpr unsigned kInvalid = 0x80000000u;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc((void *) (RES ? a.res : a.y), (short) 0, RES ? (int) a.y_bytes : 0, 0x00020000);

        // weights: fragment (m, j) of lane l holds rows m*16 + l%16, reduction values 32j + 8(l/16) .. +7
        half8 wf[MT][NSTEPS];
        {
            const half8 *wp = reinterpret_cast<const half8 *>(a.w);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int j = 0; j < NSTEPS; ++j) wf[m][j] = wp[(m * NSTEPS + j) * 64 + lane];
        }
        // the lane's biases (rows 4(l/16)..+3 of each fragment), which seed the accumulators; held
        // in registers, since a load in the tile loop could not move above the buffer stores
        float4v bsv[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) bsv[m] = *reinterpret_cast<const float4v *>(a.bias + (m * 4 + (lane >> 4)) * 4);
        // per (step, half): the LDS pixel offset of this lane's 4-channel slot relative to the
        // output pixel's band position, or -1 for a zero pad of the reduction (tap >= K*K)
        int boff[NSTEPS][2];
#pragma unroll
        for (int j = 0; j < NSTEPS; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int k   = 32 * j + 8 * (lane >> 4) + 4 * q;
                const int tap = k / CIN4, slot = (k % CIN4) / 4;
                boff[j][q]    = tap < K * K ? (slot * B::ROWS + tap / K) * B::COLS + tap % K - B::PAD + B::COFF : -1;
            }

        auto item_pos = [&](int it, int &n, int &oy0, int &ox0) __attribute__((always_inline)) {
            const int cb = it % cblk, rest = it / cblk;
            ox0 = cb * OCW;
            oy0 = (rest % rblk) * OR;
            n   = rest / rblk;
        };
        auto issue_band = [&](int it, int buf) __attribute__((always_inline)) {
            int n, oy0, ox0;
            item_pos(it, n, oy0, ox0);
            const int iy0 = oy0 * S - B::PAD, ix0 = ox0 * S - B::COFF;
            unsigned char *dst = sm + buf * BAND;
#pragma unroll
            for (int r = 0; r < NBW; ++r) {
                const int i   = r * 4 + wave;
                const int p   = i * 64 + lane;
                const int pc  = p % B::PPR, rs = p / B::PPR;
                const int row = rs % B::ROWS, slot = rs / B::ROWS;
                const int iy  = iy0 + row, ix = ix0 + 2 * pc;
                const bool ok = p < TP && slot < a.Cinb && iy >= 0 && iy < H && ix >= 0 && ix < W;
                const unsigned off = ok ? (unsigned) ((((n * a.x_pstride + slot) * H + iy) * W + ix) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (dst + i * 1024), 16, off, 0, 0, 0);
            }
            // residual tile: [slot][row][64 pixels], two pixels per lane and copy
#pragma unroll
            for (int r = 0; r < NRW; ++r) {
                const int i    = r * 4 + wave;
                const int p    = i * 64 + lane;
                const int pc   = p % (OCW / 2), rs = p / (OCW / 2);
                const int row  = rs % OR, slot = rs / OR;
                const int oy   = oy0 + row, ox = ox0 + 2 * pc;
                const bool ok  = slot < a.Coutb && oy < a.OHW / a.OW && ox < a.OW;
                const unsigned off = ok ? (unsigned) ((((n * a.y_pstride + slot) * (a.OHW / a.OW) + oy) * a.OW + ox) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rrs, (__attribute__((address_space(3))) void *) (dst + RBASE + i * 1024), 16, off, 0, 0, 0);
            }
        };

        auto finish = [&](int it, int buf, auto act_c) __attribute__((always_inline)) {
            constexpr int ACT = decltype(act_c)::value;
            int n, oy0, ox0;
            item_pos(it, n, oy0, ox0);
            const unsigned char *band = sm + buf * BAND;
            const int oy  = oy0 + wave;
            const int g   = lane >> 4;
#pragma unroll
            for (int t = 0; t < OCW / 16; ++t) {
                const int ox   = ox0 + t * 16 + (lane & 15);
                const int base = wave * S * B::COLS + (t * 16 + (lane & 15)) * S;
                float4v   acc[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] = bsv[m];
#pragma unroll
                for (int j = 0; j < NSTEPS; ++j) {
                    u32x2 v[2];
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        // a zero pad of the reduction reads the window origin and is masked after
                        // the read (no branch)
                        const int   o = boff[j][q] < 0 ? 0 : boff[j][q];
                        const u32x2 t = *reinterpret_cast<const u32x2 *>(band + (base + o) * 8);
                        v[q]          = boff[j][q] >= 0 ? t : u32x2 {0u, 0u};
                    }
                    const half8 bf = __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y));
#pragma unroll
                    for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[m][j], bf, acc[m], 0, 0, 0);
                }
                const bool pok = oy < OH && ox < OW;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const int ocb = m * 4 + g;
                    const int oc  = ocb * 4;
                    float4v   v   = acc[m];
                    float4v   r   = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (RES) {
                        r = h4_to_f4(__builtin_bit_cast(half4, *reinterpret_cast<const u32x2 *>(band + RBASE + ((ocb * OR + wave) * OCW + t * 16 + (lane & 15)) * 8)));
                        if (a.has_res != 2) v += r;
                    }
                    v.x = apply_act(v.x, ACT, a.lo, a.hi);
                    v.y = apply_act(v.y, ACT, a.lo, a.hi);
                    v.z = apply_act(v.z, ACT, a.lo, a.hi);
                    v.w = apply_act(v.w, ACT, a.lo, a.hi);
                    if (RES && a.has_res == 2) v += r;
                    if (oc + 0 >= a.Cout) v.x = 0.f;
                    if (oc + 1 >= a.Cout) v.y = 0.f;
                    if (oc + 2 >= a.Cout) v.z = 0.f;
                    if (oc + 3 >= a.Cout) v.w = 0.f;
                    const unsigned off = pok && ocb < a.Coutb ? (unsigned) ((((n * a.y_pstride + ocb) * OH + oy) * OW + ox) * 8) : kInvalid;
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, off, 0, kStreamStore);
                }
            }
        };
        auto compute_store = [&](int it, int buf) __attribute__((always_inline)) {
            using std::integral_constant;
            switch (a.act) {
                case VKHIP_ACT_RELU: finish(it, buf, integral_constant<int, VKHIP_ACT_RELU> {}); break;
                case VKHIP_ACT_RELU6: finish(it, buf, integral_constant<int, VKHIP_ACT_RELU6> {}); break;
                case VKHIP_ACT_CLIP: finish(it, buf, integral_constant<int, VKHIP_ACT_CLIP> {}); break;
                case VKHIP_ACT_HARDSWISH: finish(it, buf, integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
                case VKHIP_ACT_SILU: finish(it, buf, integral_constant<int, VKHIP_ACT_SILU> {}); break;
                case VKHIP_ACT_HARDSIGMOID: finish(it, buf, integral_constant<int, VKHIP_ACT_HARDSIGMOID> {}); break;
                default: finish(it, buf, integral_constant<int, VKHIP_ACT_NONE> {}); break;
            }
        };

        // stores per wave per item: every (pixel tile, fragment) store is issued, out-of-range ones
        // with an offset the buffer drops, so the count is fixed
        constexpr int kStores = (OCW / 16) * MT;
        constexpr int kCopies = NBW + NRW; // copies per wave per item
        static_assert((NBUF - 1) * kStores + kCopies <= 63, "stores and copies in flight fit the counter");
        // vmcnt(n) with n a compile-time constant (the counter retires in issue order)
        auto wait_for = [](auto n_c) __attribute__((always_inline)) {
            constexpr int n = decltype(n_c)::value;
            __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
        };
        using std::integral_constant;
        // Item order. Workgroup b runs on XCD b % 8 (ids are dealt to the 8 XCDs round-robin).
        // a.item_order 1: the items are cut into 8 contiguous ranges, one per XCD, which that XCD's
        // workgroups walk in order, so items a workgroup's XCD runs at the same time are neighbours
        // and the input rows two vertically adjacent items share are read from that XCD's L2 once;
        // 0: one strided walk over all items.
        const int G = gridDim.x;
        const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3;
        // XCD x holds gx workgroups, px of them on the XCDs before it; its range is its share
        const int gx  = a.item_order ? (G >> 3) + ((G & 7) > xcd ? 1 : 0) : G;
        const int px  = xcd * (G >> 3) + min(xcd, G & 7);
        const int i0  = a.item_order ? (int) ((long long) items * px / G) + lb : blockIdx.x;
        const int i1  = a.item_order ? (int) ((long long) items * (px + gx) / G) : items;
        auto item_at = [&](int k) __attribute__((always_inline)) { return i0 + k * gx < i1 ? i0 + k * gx : -1; };
        int buf = 0;
#pragma unroll
        for (int d = 0; d < NBUF - 1; ++d)
            if (item_at(d) >= 0) issue_band(item_at(d), d);
        for (int k = 0; item_at(k) >= 0; ++k) {
            const int it = item_at(k);
            // Wait for this item's band. Issued after it, and allowed to stay in flight: the stores
            // of the (at most NBUF - 1) items computed since, and the band of the next item when
            // NBUF = 3 and that item exists.
            const bool more = NBUF == 3 && item_at(k + 1) >= 0;
            if constexpr (NBUF == 2) {
                if (k == 0) wait_for(integral_constant<int, 0> {});
                else wait_for(integral_constant<int, kStores> {});
            } else {
                if (k == 0) {
                    if (more) wait_for(integral_constant<int, kCopies> {});
                    else wait_for(integral_constant<int, 0> {});
                } else if (k == 1) {
                    if (more) wait_for(integral_constant<int, kCopies + kStores> {});
                    else wait_for(integral_constant<int, kStores> {});
                } else {
                    if (more) wait_for(integral_constant<int, kCopies + 2 * kStores> {});
                    else wait_for(integral_constant<int, 2 * kStores> {});
                }
            }
            __asm__ volatile("s_barrier" ::: "memory"); // all copies of the band landed; the oldest buffer is free
            const int nxt = item_at(k + NBUF - 1);
            if (nxt >= 0) issue_band(nxt, buf == 0 ? NBUF - 1 : buf - 1);
            compute_store(it, buf);
            buf = buf + 1 == NBUF ? 0 : buf + 1;
        }
    }

    // ring depth: three buffers (two items ahead) when they leave room for two workgroups per CU
    template <int CB, int K, int S, int MT, bool RES>
    constexpr int thin_nbuf() {
        return 3 * (thin_band_bytes<CB, K, S>() + thin_res_copies<MT, RES>() * 4 * 1024) <= 80 * 1024 ? 3 : 2;
    }

    template <int CB, int MT_>
    static GemmKernelFn thin_pick_ks(int k, int s, bool res) {
        if constexpr (MT_ * ((9 * CB * 4 + 31) / 32) <= 20) {
            if (k == 3 && s == 1)
                return res ? conv_thin_kernel<CB, MT_, 3, 1, thin_nbuf<CB, 3, 1, MT_, true>(), true>
                           : conv_thin_kernel<CB, MT_, 3, 1, thin_nbuf<CB, 3, 1, MT_, false>(), false>;
            if (res) return nullptr;
            if (k == 3 && s == 2) return conv_thin_kernel<CB, MT_, 3, 2, thin_nbuf<CB, 3, 2, MT_, false>(), false>;
        }
        if (res) return nullptr;
        if constexpr (CB == 1) {
            if (k == 7 && s == 2) return conv_thin_kernel<CB, MT_, 7, 2, thin_nbuf<CB, 7, 2, MT_, false>(), false>;
        }
        if (k == 1 && s == 1) return conv_thin_kernel<CB, MT_, 1, 1, thin_nbuf<CB, 1, 1, MT_, false>(), false>;
        return nullptr;
    }
    template <int CB>
    static GemmKernelFn thin_pick_mt(int mt, int k, int s, bool res) {
        if (mt == 1) return thin_pick_ks<CB, 1>(k, s, res);
        if (mt == 2) return thin_pick_ks<CB, 2>(k, s, res);
        if (mt == 4) return thin_pick_ks<CB, 4>(k, s, res);
        return nullptr;
    }
    // kernel for a thin plan: cinb input slots (rounded up to 1, 2, 4 or 8), mt 16-channel output
    // fragments (1, 2 or 4), with a residual (3x3 stride 1 only) or without
    GemmKernelFn thin_kernel_for(int cinb, int mt, int k, int s, bool res) {
        switch (thin_cinb(cinb)) {
            case 1: return thin_pick_mt<1>(mt, k, s, res);
            case 2: return thin_pick_mt<2>(mt, k, s, res);
            case 4: return thin_pick_mt<4>(mt, k, s, res);
            case 8: return thin_pick_mt<8>(mt, k, s, res);
        }
        return nullptr;
    }

} // namespace vkhip
