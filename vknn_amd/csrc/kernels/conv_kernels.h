// Implicit-GEMM convolution kernels for gfx950 (device templates shared by the tile instantiation
// files conv_*_tiles.hip and the host code in conv.hip).
//
// Convolution on gfx950: one implicit-GEMM kernel on fp16 MFMA (v_mfma_f32_32x32x16_f16, fp32
// accumulation) serves every dense conv of the path — 1x1 pointwise (stride 1 or 2), 3x3 s1/s2,
// 7x7 stems — plus the 16 batched GEMMs of Winograd F(2x2,3x3) and split-K for deep layers with
// few output pixels. Depthwise convs run on a bandwidth kernel without MFMA.
//
// GEMM view (per image batch, all images flattened into the pixel axis):
//   rows    m = output channel        (MFMA "M"; a lane's 4 consecutive rows = one NC4HW4 block,
//                                      so every epilogue store is one 8-byte fp16x4 write)
//   columns p = (n, oy, ox)           (MFMA "N")
//   reduction k = slot*4 + lane, slot = tap*Cinb + cb, tap = ky*KW + kx
// A = packed weights fp16 in [m_tile][k_stage][BM][64] order (host prepack, zero padded); B = input pixels gathered on
// the fly from NC4HW4 fp16 (8 bytes per (pixel, slot)), zero outside the image.
//
// Reference semantics followed: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) for the convolution,
// residual and activation order; ops/conv.cpp:104-141 + shaders/wino_*_fp16.comp for the
// Winograd F(2,3) matrices (G, B^T, A^T) and the fp16 storage of V and M; the split-K reduce
// (shaders/conv1x1_reduce_fp16.comp) for partial sums + bias + residual + activation.
#pragma once
#include "common.h"
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>


namespace vkhip {

    // ------------------------------------------------------------------ kernel arguments
    struct GemmArgs {
        const uint2  *x;    // NC4HW4 fp16, 8-byte (4-channel) vectors
        const half_t *w;    // tiled [m_tile][k_stage][BM][64]
        const float  *bias; // [Coutp]
        const uint2  *res;
        uint2        *y;
        float4v      *part; // split-K partials [ksplit][Coutb][P]
        int           Cinb, H, W, HW;
        int           Coutb, Cout, OW, OHW;
        int           KW, SH, SW, PT, PL, DH, DW;
        int           P, Kslots, nsteps, steps_per_split;
        int           Pv, OHWp; // GEMM columns and columns per image: P and OH*OW, or with one padding
                                // column per image when the dense-B kernel needs an even count
        int           act;
        float         lo, hi;
        int           has_res, omode, m_tiles;         // has_res: 1 residual added before the activation, 2 after it
        int           n_tiles;                         // column tiles (persistent kernels walk m_tiles x n_tiles)
        long long     x_bstride, w_bstride, y_bstride; // batch (blockIdx.z) strides: uint2 / half / uint2
        unsigned      x_bytes;                         // bytes of one batch slice of x (< 2 GiB)
        unsigned      y_bytes;                         // bytes of one batch slice of y (< 2 GiB)
        const uint2  *xs;                              // input channel scale [N][Cinb] x 4 fp16 (in_scale)
        unsigned      xs_bytes;                        // bytes of xs
        int           x_pstride, y_pstride;            // channel blocks per image of the buffers x / y point into
                                                       // (Cinb / Coutb, or more for a view into a wider tensor)
        int          *cnt;                             // split-K: per-tile arrival counters when the last
                                                       // workgroup of a tile sums the partials (else null)
        int           item_order;                      // conv_thin_kernel: 1 XCD-contiguous item ranges, 0 strided
    };

    enum { OMODE_EPILOGUE = 0, OMODE_RAW = 1, OMODE_PARTIAL = 2 };
    // B gather modes. *_P16 variants load two adjacent output pixels of one channel slot with a
    // single 16-byte load (the vector memory pipe costs the same per instruction for 8 or 16
    // bytes); they need every pixel pair to be adjacent in memory at every tap (unit stride, even
    // row width / even image size).
    enum { BMODE_1X1 = 0, BMODE_ALIGNED = 1, BMODE_GENERAL = 2, BMODE_1X1_P16 = 3, BMODE_ALIGNED_P16 = 4 };

    constexpr int kThreads = 256; // 4 wave64s per workgroup
    constexpr int kBK      = 64;  // reduction halves per LDS stage (16 channel slots)
    constexpr int kAStride = 72;  // LDS row stride of the A tile in halves (64 + 8 pad = 144 bytes)

    // 16-byte global load from an 8-byte aligned address (two adjacent NC4HW4 pixels).
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned int u32x4_a8 __attribute__((ext_vector_type(4), aligned(8)));
    __device__ __forceinline__ u32x4 u32x4_make(unsigned a, unsigned b, unsigned c, unsigned d) { return u32x4 {a, b, c, d}; }

    // Spread consecutive workgroup ids (dispatched round-robin over the 8 XCDs) so that runs of
    // consecutive logical tiles land on one XCD and share its L2.
    __device__ __forceinline__ int xcd_remap(int bid, int nwg) {
        const int xcd = bid & 7, local = bid >> 3, q = nwg >> 3, r = nwg & 7;
        return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
    }


    // Instruction-interleaving hints for one 16-K step: after each MFMA, place a share of the LDS
    // reads (next step's fragments), LDS writes (next stage's tile) and global loads (the stage
    // after), so the wave keeps the matrix core busy while those are in flight.
    enum { SG_MFMA = 0x008, SG_VALU = 0x002, SG_VMEM_READ = 0x020, SG_DS_READ = 0x100, SG_DS_WRITE = 0x200 };
    template <int I, int NM, int NR, int NW, int NV>
    struct Interleave {
        static __device__ __forceinline__ void apply() {
            if constexpr (I < NM) {
                constexpr int r = NR * (I + 1) / NM - NR * I / NM;
                constexpr int w = NW * (I + 1) / NM - NW * I / NM;
                constexpr int v = NV * (I + 1) / NM - NV * I / NM;
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
                if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(SG_DS_READ, r, 0);
                if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, w, 0);
                if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(SG_VMEM_READ, v, 0);
                Interleave<I + 1, NM, NR, NW, NV>::apply();
            }
        }
    };

    // ------------------------------------------------------------------ in-kernel split-K reduction
    // The split-K workgroups of one output tile (blockIdx.x, splits blockIdx.y) store their fp32
    // partial tiles agent-coherent (MODE 4: written through to the device coherence point, so no
    // cache write-back is needed before counting in), wait for those stores, and count in on the
    // tile's counter; the workgroup that arrives last resets the counter (each launch leaves every
    // counter at zero) and returns true. `flag`: a word of the kernel's LDS that no wave reads or
    // writes any more (the broadcast of the outcome).
    constexpr int kCoherent = 16; // buffer cache policy: sc1 (agent scope)

    __device__ __forceinline__ bool splitk_last_arrival(const GemmArgs &a, volatile int *flag) {
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // vmcnt(0): this wave's partial stores are complete
        __syncthreads();
        if (threadIdx.x == 0) {
            int      *c    = a.cnt + blockIdx.x;
            const int old  = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == (int) gridDim.y - 1;
            if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last;
        }
        __syncthreads();
        return *flag != 0;
    }

    // acc := the sum of the tile's partials over splits 0, 1, ..., in that order (this workgroup's
    // own split from its registers, the others read agent-coherent), so the result does not depend
    // on which workgroup arrived last.
    template <int FM, int FN>
    __device__ __forceinline__ void splitk_gather(const GemmArgs &a, float16v (&acc)[FM][FN], int mw0, int nw0, int split, int lane) {
        constexpr unsigned kInvalid = 0x80000000u;
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc((void *) a.part, (short) 0, 0x7FFFFFFF, 0x00020000);
        const int      lrow = lane & 31, lk = lane >> 5;
        const unsigned sstride = (unsigned) a.Coutb * (unsigned) a.P * 16u;
        unsigned       off[FN][FM][4];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int  px  = nw0 + j * 32 + lrow;
            const int  pn  = px / a.OHWp;
            const int  pr  = px - pn * a.OHWp;
            const bool pok = (px < a.Pv) & (pr < a.OHW);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int ocb = (mw0 + i * 32 + qq * 8 + lk * 4) >> 2;
                    off[j][i][qq] = (pok & (ocb < a.Coutb)) ? (unsigned) ((ocb * a.P + pn * a.OHW + pr) * 16) : kInvalid;
                }
        }
        float16v sum[FM][FN];
        const int ks = (int) gridDim.y;
        for (int s = 0; s < ks; ++s) {
            float16v p[FM][FN];
            if (s == split) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) p[i][j] = acc[i][j];
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) {
                            const unsigned o = off[j][i][qq] == kInvalid ? kInvalid : off[j][i][qq] + (unsigned) s * sstride;
                            const float4v  v = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(prs, o, 0, kCoherent));
#pragma unroll
                            for (int r = 0; r < 4; ++r) p[i][j][qq * 4 + r] = v[r];
                        }
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) sum[i][j] = s == 0 ? p[i][j] : sum[i][j] + p[i][j];
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = sum[i][j];
    }

    template <int BM, int BN, int WM, int WN, int BMODE_>
    __global__ __launch_bounds__(kThreads) void conv_gemm_kernel(GemmArgs a) {
        constexpr bool P16   = BMODE_ >= BMODE_1X1_P16;
        constexpr int  BMODE = BMODE_ == BMODE_1X1_P16 ? BMODE_1X1 : (BMODE_ == BMODE_ALIGNED_P16 ? BMODE_ALIGNED : BMODE_);
        constexpr int TM = BM / WM, TN = BN / WN; // wave tile
        constexpr int FM = TM / 32, FN = TN / 32; // 32x32 MFMA fragments per wave
        static_assert(WM * WN == 4, "4 waves");
        static_assert(FM >= 1 && FN >= 1, "wave tile >= 32x32");
        constexpr int ACHUNK  = BM * kBK / 8;            // 16-byte chunks in one A stage
        constexpr int ALOADS  = ACHUNK / kThreads;
        constexpr int QN      = BN / 2;                  // pixel pairs in the tile
        constexpr int BITEMS  = 8 * QN / kThreads;       // (slot pair, pixel pair) items per thread
        constexpr int SPSTEP  = kThreads / QN;           // slot-pair stride between a thread's items
        static_assert(ALOADS >= 1 && ACHUNK % kThreads == 0, "A tile");
        static_assert(BITEMS >= 1 && kThreads % QN == 0, "B tile");

        __shared__ u32x4 As[2][BM * kAStride / 8];
        __shared__ u32x4 Bs[2][8 * BN]; // [slot pair][pixel] x (8 channels, fp16)

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = tid >> 6;
        const int wm0  = (wave / WN) * TM;
        const int wn0  = (wave % WN) * TN;

        const int lin    = xcd_remap(blockIdx.x, gridDim.x);
        const int m_tile = lin % a.m_tiles;
        const int n_tile = lin / a.m_tiles;
        const int m0     = m_tile * BM;
        const int n0     = n_tile * BN;
        const int split  = blockIdx.y;
        const int bz     = blockIdx.z;

        const uint2  *X  = a.x + bz * a.x_bstride;
        const half_t *Wt = a.w + bz * a.w_bstride + (long long) m_tile * a.nsteps * (BM * kBK);

        // ---- this thread's pixel pair (fixed for the whole K loop)
        const int q   = tid % QN;
        // slot pair of this thread; wave-uniform when a wave covers one slot pair (QN >= 64)
        const int sp0 = QN >= 64 ? __builtin_amdgcn_readfirstlane(tid / QN) : tid / QN;
        int       pv[2], piy[2], pix[2], pbyte[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int p = n0 + 2 * q + i;
            pv[i]       = p < a.P;
            const int pp = pv[i] ? p : 0;
            const int n  = pp / a.OHW;
            const int r  = pp - n * a.OHW;
            const int oy = r / a.OW;
            const int ox = r - oy * a.OW;
            piy[i]       = oy * a.SH - a.PT;
            pix[i]       = ox * a.SW - a.PL;
            // byte offset of (n, channel block 0, iy0, ix0); x slices are < 2 GiB
            pbyte[i] = (n * a.x_pstride * a.HW + piy[i] * a.W + pix[i]) * 8;
        }

        const int ks_begin = split * a.steps_per_split;
        const int ks_end   = min(a.nsteps, ks_begin + a.steps_per_split);

        // Two register prefetch sets: stage ks+3 is loaded while stage ks computes and is written
        // to LDS at the start of stage ks+2 (1.75 stages of lead time for L2/HBM latency).
        u32x4 areg[2][ALOADS];
        u32x4 b0[2][BITEMS], b1[2][BITEMS]; // per item: slot e=0 / e=1, each {pixel 0 (8 B), pixel 1 (8 B)}
        unsigned bfix[2];                      // P16: per (item, slot) 4 bits {pixel0 ok, pixel1 ok, shift right, shift left}

        // B gathers go through a raw buffer resource: an offset at or past num_records returns zero
        // in hardware, so padding taps, K tails and pixels past P need no branch.
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) X, (short) 0, (int) a.x_bytes, 0x00020000);
        constexpr unsigned kInvalid = 0x80000000u;
        const int          xmax16   = (int) a.x_bytes - 16;

        // weights of this M tile only: prefetches past the last stage read zeros, not other tiles
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *) Wt, (short) 0, ks_end * (BM * kBK * 2), 0x00020000);
        const int kslots = min(a.Kslots, ks_end * 16); // slots past this split read zeros
        const int hw8 = a.HW * 8;

        auto load_tiles = [&](int ks, auto set_c) __attribute__((always_inline)) {
            constexpr int S = decltype(set_c)::value;
            const int wsoff = ks * (BM * kBK * 2);
            unsigned  fixbits = 0;
#pragma unroll
            for (int i = 0; i < ALOADS; ++i) areg[S][i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, (tid + i * kThreads) * 16, wsoff, 0);
#pragma unroll
            for (int j = 0; j < BITEMS; ++j) {
                const int sp   = sp0 + j * SPSTEP; // slot pair within the stage (0..7), wave-uniform
                const int slot = ks * 16 + 2 * sp;  // first slot of the pair
                unsigned  off[2][2];                // [slot e][pixel i], byte offsets or kInvalid
                int       p16o[2];                  // P16: pixel 0 byte offset per slot
                bool      p16ok[2][2];              // P16: [slot e][pixel i] validity
                if (BMODE == BMODE_1X1) {
                    const int s0 = slot * hw8;
                    p16o[0] = pbyte[0] + s0;
                    p16o[1] = pbyte[0] + s0 + hw8;
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        p16ok[0][i] = (pv[i] != 0) & (slot < kslots);
                        p16ok[1][i] = (pv[i] != 0) & (slot + 1 < kslots);
                        off[0][i] = ((pv[i] != 0) & (slot < kslots)) ? (unsigned) (pbyte[i] + s0) : kInvalid;
                        off[1][i] = ((pv[i] != 0) & (slot + 1 < kslots)) ? (unsigned) (pbyte[i] + s0 + hw8) : kInvalid;
                    }
                } else if (BMODE == BMODE_ALIGNED) {
                    // Cinb % 8 == 0: the 8 slots of each half stage share one tap (all scalar).
                    const int half = ks * 16 + (sp >> 2) * 8;
                    const int tap  = half / a.Cinb;
                    const int cb   = half - tap * a.Cinb + 2 * (sp & 3);
                    const int ky   = tap / a.KW;
                    const int kx   = tap - ky * a.KW;
                    const int dy = ky * a.DH, dx = kx * a.DW;
                    const int soff = cb * hw8 + (dy * a.W + dx) * 8;
                    const bool kin = slot < kslots;
                    p16o[0] = pbyte[0] + soff;
                    p16o[1] = pbyte[0] + soff + hw8;
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const bool ok = kin & (pv[i] != 0) & ((unsigned) (piy[i] + dy) < (unsigned) a.H) & ((unsigned) (pix[i] + dx) < (unsigned) a.W);
                        p16ok[0][i] = ok;
                        p16ok[1][i] = ok;
                        off[0][i] = ok ? (unsigned) (pbyte[i] + soff) : kInvalid;
                        off[1][i] = ok ? (unsigned) (pbyte[i] + soff + hw8) : kInvalid;
                    }
                } else {
                    p16o[0] = p16o[1] = 0;
                    p16ok[0][0] = p16ok[0][1] = p16ok[1][0] = p16ok[1][1] = false;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int g   = slot + e;
                        const int tap = g / a.Cinb;
                        const int cb  = g - tap * a.Cinb;
                        const int ky  = tap / a.KW;
                        const int kx  = tap - ky * a.KW;
                        const int dy = ky * a.DH, dx = kx * a.DW;
                        const int soff = cb * hw8 + (dy * a.W + dx) * 8;
#pragma unroll
                        for (int i = 0; i < 2; ++i) {
                            const bool ok = (g < kslots) & (pv[i] != 0) & ((unsigned) (piy[i] + dy) < (unsigned) a.H) & ((unsigned) (pix[i] + dx) < (unsigned) a.W);
                            off[e][i]     = ok ? (unsigned) (pbyte[i] + soff) : kInvalid;
                        }
                    }
                }
                if constexpr (P16) {
                    // off[e][0] holds pixel 0's byte offset even when pixel 0 is padding (the pair is
                    // adjacent in memory); load 16 bytes from there, clamped into the tensor.
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int  o0 = p16o[e];
                        const bool ok0 = p16ok[e][0], ok1 = p16ok[e][1];
                        const int  ol = o0 < 0 ? 0 : (o0 > xmax16 ? xmax16 : o0);
                        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, (ok0 | ok1) ? (unsigned) ol : kInvalid, 0, 0);
                        if (e == 0) b0[S][j] = v;
                        else b1[S][j] = v;
                        const unsigned bits = (ok0 ? 1u : 0u) | (ok1 ? 2u : 0u) | (o0 < 0 ? 4u : 0u) | (o0 > xmax16 ? 8u : 0u);
                        fixbits |= bits << (4 * (2 * j + e));
                    }
                } else {
                    const u32x2 v00 = __builtin_amdgcn_raw_buffer_load_b64(xrs, off[0][0], 0, 0);
                    const u32x2 v01 = __builtin_amdgcn_raw_buffer_load_b64(xrs, off[0][1], 0, 0);
                    const u32x2 v10 = __builtin_amdgcn_raw_buffer_load_b64(xrs, off[1][0], 0, 0);
                    const u32x2 v11 = __builtin_amdgcn_raw_buffer_load_b64(xrs, off[1][1], 0, 0);
                    b0[S][j] = u32x4_make(v00.x, v00.y, v01.x, v01.y);
                    b1[S][j] = u32x4_make(v10.x, v10.y, v11.x, v11.y);
                }
            }
            bfix[S] = fixbits;
        };

        auto store_tiles = [&](int buf, auto set_c) __attribute__((always_inline)) {
            constexpr int S = decltype(set_c)::value;
#pragma unroll
            for (int i = 0; i < ALOADS; ++i) {
                const int c = tid + i * kThreads, row = c >> 3, col = c & 7;
                As[buf][row * (kAStride / 8) + col] = areg[S][i];
            }
            if constexpr (P16) {
                const unsigned fb = bfix[S];
#pragma unroll
                for (int j = 0; j < BITEMS; ++j)
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const unsigned bits = fb >> (4 * (2 * j + e));
                        u32x4          v    = e == 0 ? b0[S][j] : b1[S][j];
                        if (bits & 4u) v = u32x4_make(0u, 0u, v.x, v.y);  // pair began 8 bytes before the tensor
                        if (bits & 8u) v = u32x4_make(v.z, v.w, 0u, 0u);  // pair ended 8 bytes past the tensor
                        if (!(bits & 1u)) v.x = v.y = 0u;                  // pixel 0 is padding
                        if (!(bits & 2u)) v.z = v.w = 0u;                  // pixel 1 is padding
                        if (e == 0) b0[S][j] = v;
                        else b1[S][j] = v;
                    }
            }
#pragma unroll
            for (int j = 0; j < BITEMS; ++j) {
                const int sp = sp0 + j * SPSTEP;
                // pixel 0 gets {slot e=0 lanes, slot e=1 lanes}, pixel 1 likewise
                Bs[buf][sp * BN + 2 * q]     = u32x4_make(b0[S][j].x, b0[S][j].y, b1[S][j].x, b1[S][j].y);
                Bs[buf][sp * BN + 2 * q + 1] = u32x4_make(b0[S][j].z, b0[S][j].w, b1[S][j].z, b1[S][j].w);
            }
        };

        float16v acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        const int lrow = lane & 31; // A row / B column inside a 32x32 fragment
        const int lk   = lane >> 5; // which 8-wide K group of the 16-wide MFMA step

        // Fragment double buffer: the next 16-K step's A/B fragments are read from LDS while the
        // current step's MFMAs run.
        half8 fa[2][FM], fb[2][FN];
        auto read_frags = [&](int buf, int kk, int fbuf) __attribute__((always_inline)) {
            const half_t *Ab = reinterpret_cast<const half_t *>(As[buf]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
                fa[fbuf][i] = *reinterpret_cast<const half8 *>(Ab + (wm0 + i * 32 + lrow) * kAStride + kk * 16 + lk * 8);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                fb[fbuf][j] = *reinterpret_cast<const half8 *>(&Bs[buf][(kk * 2 + lk) * BN + wn0 + j * 32 + lrow]);
        };

        // Stage pipeline (LDS double buffer, two register prefetch sets):
        //   step 0 of stage ks : write the set holding stage ks+1 into the idle LDS buffer;
        //   step 1             : issue the global loads of stage ks+3 into that (now free) set;
        //   steps 0..3         : read the next 16-K fragments while the current MFMAs run;
        //   end                : barrier, read the first fragments of stage ks+1.
        // The stage loop runs in pairs (register sets are compile-time indices); a trailing odd
        // stage and all prefetches past ks_end read zeros, so they add nothing to the sums.
        constexpr int NM = FM * FN, NR = FM + FN, NW = ALOADS + 2 * BITEMS, NV = ALOADS + 4 * BITEMS;
        auto mfmas = [&](int fbuf) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[fbuf][i], fb[fbuf][j], acc[i][j], 0, 0, 0);
        };
        auto stage = [&](int ks, int buf, auto set_c) __attribute__((always_inline)) {
            read_frags(buf, 1, 1);
            store_tiles(buf ^ 1, set_c);
            mfmas(0);
            Interleave<0, NM, NR, NW, 0>::apply();
            __builtin_amdgcn_sched_barrier(0);
            read_frags(buf, 2, 0);
            load_tiles(ks + 3, set_c);
            mfmas(1);
            Interleave<0, NM, NR, 0, NV>::apply();
            __builtin_amdgcn_sched_barrier(0);
            read_frags(buf, 3, 1);
            mfmas(0);
            Interleave<0, NM, NR, 0, 0>::apply();
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
            __syncthreads();
            read_frags(buf ^ 1, 0, 0);
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        if (ks_begin < ks_end) {
            load_tiles(ks_begin, S0 {});
            store_tiles(0, S0 {});
            __syncthreads();
            load_tiles(ks_begin + 1, S1 {});
            load_tiles(ks_begin + 2, S0 {});
            read_frags(0, 0, 0);
            for (int ks = ks_begin; ks < ks_end; ks += 2) {
                stage(ks, 0, S1 {});
                stage(ks + 1, 1, S0 {});
            }
        }

        // ---- epilogue. D layout of a 32x32 fragment: lane l holds column l%32, register r holds
        // row 8*(r/4) + 4*(l/32) + r%4, so registers 4q..4q+3 are one 4-channel block.
        // Pass 1 issues every bias / residual load of the tile, pass 2 computes and stores; rows or
        // pixels outside the tensor get an out-of-range offset, so their loads read zero and their
        // stores are dropped by the buffer unit.
        unsigned yoff[FN][FM][4];
        auto offsets = [&](bool partial) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int  px  = n0 + wn0 + j * 32 + lrow;
                const bool pok = px < a.P;
                const int  pn  = px / a.OHW;
                const int  pr  = px - pn * a.OHW;
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int  ocb = (m0 + wm0 + i * 32 + qq * 8 + lk * 4) >> 2;
                        const bool ok  = pok & (ocb < a.Coutb);
                        if (partial) yoff[j][i][qq] = ok ? (unsigned) (((split * a.Coutb + ocb) * a.P + px) * 16) : kInvalid;
                        else yoff[j][i][qq] = ok ? (unsigned) (((pn * a.y_pstride + ocb) * a.OHW + pr) * 8) : kInvalid;
                    }
            }
        };
        offsets(a.omode == OMODE_PARTIAL);
        bool epi = a.omode == OMODE_EPILOGUE;
        if (a.omode == OMODE_PARTIAL) {
            const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc((void *) a.part, (short) 0, 0x7FFFFFFF, 0x00020000);
            auto store = [&](auto aux_c) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) {
                            float4v v = {acc[i][j][qq * 4 + 0], acc[i][j][qq * 4 + 1], acc[i][j][qq * 4 + 2], acc[i][j][qq * 4 + 3]};
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs, yoff[j][i][qq], 0, decltype(aux_c)::value);
                        }
            };
            if (!a.cnt) {
                store(std::integral_constant<int, 0> {});
                return;
            }
            store(std::integral_constant<int, kCoherent> {});
            if (!splitk_last_arrival(a, reinterpret_cast<volatile int *>(&Bs[0][0]))) return;
            // the workgroup that arrived last finishes the tile from the summed partials
            splitk_gather<FM, FN>(a, acc, m0 + wm0, n0 + wn0, split, lane);
            offsets(false);
            epi = true;
        }
        {
            uint2 *Y = a.y + bz * a.y_bstride;
            const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) Y, (short) 0, (int) a.y_bytes, 0x00020000);
            float4v     bia[FM][4];
            u32x2       rv[FN][FM][4];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int oc = m0 + wm0 + i * 32 + qq * 8 + lk * 4;
                    bia[i][qq]   = epi ? *reinterpret_cast<const float4v *>(a.bias + oc) : float4v {0.f, 0.f, 0.f, 0.f};
                }
            if (epi && a.has_res) {
                const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc((void *) (a.res + bz * a.y_bstride), (short) 0, (int) a.y_bytes, 0x00020000);
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) rv[j][i][qq] = __builtin_amdgcn_raw_buffer_load_b64(rrs, yoff[j][i][qq], 0, kStreamLoad);
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) rv[j][i][qq] = u32x2 {0u, 0u};
            }
            auto finish = [&](auto act_c) __attribute__((always_inline)) {
                constexpr int ACT = decltype(act_c)::value;
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) {
                            const int oc = m0 + wm0 + i * 32 + qq * 8 + lk * 4;
                            float4v   v  = {acc[i][j][qq * 4 + 0], acc[i][j][qq * 4 + 1], acc[i][j][qq * 4 + 2], acc[i][j][qq * 4 + 3]};
                            v += bia[i][qq];
                            const float4v r = h4_to_f4(__builtin_bit_cast(half4, rv[j][i][qq]));
                            if (a.has_res != 2) v += r;
                            v.x = apply_act(v.x, ACT, a.lo, a.hi);
                            v.y = apply_act(v.y, ACT, a.lo, a.hi);
                            v.z = apply_act(v.z, ACT, a.lo, a.hi);
                            v.w = apply_act(v.w, ACT, a.lo, a.hi);
                            if (a.has_res == 2) v += r;
                            if (oc + 0 >= a.Cout) v.x = 0.f;
                            if (oc + 1 >= a.Cout) v.y = 0.f;
                            if (oc + 2 >= a.Cout) v.z = 0.f;
                            if (oc + 3 >= a.Cout) v.w = 0.f;
                            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, yoff[j][i][qq], 0, kStreamStore);
                        }
            };
            switch (epi ? a.act : 0) {
                case VKHIP_ACT_RELU: finish(std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
                case VKHIP_ACT_RELU6: finish(std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
                case VKHIP_ACT_CLIP: finish(std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
                case VKHIP_ACT_HARDSWISH: finish(std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
                case VKHIP_ACT_SILU: finish(std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
                case VKHIP_ACT_HARDSIGMOID: finish(std::integral_constant<int, VKHIP_ACT_HARDSIGMOID> {}); break;
                default: finish(std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
            }
        }
    }

    // ------------------------------------------------------------------ B-direct GEMM kernel
    // Second main loop for the same implicit GEMM, built to cut LDS traffic per MFMA:
    //   * A (weights) is prepacked on the host in MFMA fragment order ([m_tile][stage][kk][m_frag]
    //     [lane][8 halves]) and copied global -> LDS by the buffer unit itself (buffer_load ... lds,
    //     16 bytes per lane), three stages deep; no VGPR staging, no ds_write;
    //   * B (activation pixels) never touches LDS: every lane gathers the two NC4HW4 slots of its own
    //     fragment column straight into the MFMA operand registers, one stage ahead;
    //   * each wave owns a (32*FM) x (32*FN) block; the 4 waves tile the workgroup WM x WN.
    // LDS reads per 16-K step and wave are FM fragments (the A operand) for FM*FN MFMAs.
    // Epilogue shared by the register-tile kernels: the D layout of a 32x32 fragment puts output
    // column l%32 in lane l and rows 8*(r/4) + 4*(l/32) + r%4 in register r, so registers 4q..4q+3
    // are one NC4HW4 channel block and each store is one 8-byte write. One fragment column j at a
    // time: its residual loads and offsets are the only extra registers live next to the sums.
    // Rows or pixels outside the tensor get an out-of-range offset (loads read zero, stores drop).
    // Schedule of one 16-K step: NM MFMAs; the next step's NR LDS reads go out between the first
    // half of them, the NV register moves that assemble B fragments between the last quarter (so
    // the moves find their reads complete instead of stalling the MFMA issue).
    // NG global (LDS-DMA) loads, when given, go out one per MFMA from the first one on.
    template <int I, int NM, int NR, int NV, int NG = 0>
    struct StepSchedule {
        static __device__ __forceinline__ void apply() {
            if constexpr (I < NM) {
                constexpr int H = NM / 2 > 0 ? NM / 2 : 1;
                constexpr int Q = NM - (3 * NM) / 4 > 0 ? NM - (3 * NM) / 4 : 1;
                constexpr int r = I < H ? NR * (I + 1) / H - NR * I / H : 0;
                constexpr int J = I - (NM - Q);
                constexpr int v = J >= 0 ? NV * (J + 1) / Q - NV * J / Q : 0;
                constexpr int gl = NG * (I + 1) / NM - NG * I / NM;
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
                if constexpr (gl > 0) __builtin_amdgcn_sched_group_barrier(SG_VMEM_READ, gl, 0);
                if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(SG_DS_READ, r, 0);
                if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(SG_VALU, v, 0);
                StepSchedule<I + 1, NM, NR, NV, NG>::apply();
            }
        }
    };

    template <int FM, int FN>
    __device__ __forceinline__ void gemm_epilogue(const GemmArgs &a, float16v (&acc)[FM][FN], int mw0, int nw0, int split, int bz,
                                                  int lane, volatile int *flag = nullptr) {
        constexpr unsigned kInvalid = 0x80000000u;
        const int  lrow = lane & 31;
        const int  lk   = lane >> 5;
        uint2     *Y    = a.y + bz * a.y_bstride;
        // Offsets and residual loads: all fragment columns up front when that is at most 32
        // registers of loads (the latency is paid once), one column at a time otherwise, the
        // next column's loads issued before this column's stores. Every load of the epilogue
        // goes out before the stores it could queue behind: the vector memory counter retires in
        // order, so waiting for a load issued after a store also waits for that store.
        // MODE (compile time, so the element loop has no branches): 0 split-K partials (fp32, raw),
        // 1 raw fp16 (Winograd M), 2 bias + act, 3 bias + residual + act, 4 split-K partials stored
        // agent-coherent (write-through, for the in-kernel reduction).
        constexpr int JG = FM * FN <= 8 ? FN : 1; // fragment columns per group
        constexpr int NG = FN / JG;
        auto finish = [&](auto mode_c, auto act_c) __attribute__((always_inline)) {
            constexpr int MODE = decltype(mode_c)::value;
            constexpr int ACT  = decltype(act_c)::value;
            constexpr bool PARTIAL = MODE == 0 || MODE == 4;
            const __amdgpu_buffer_rsrc_t yrs = PARTIAL ? __builtin_amdgcn_make_buffer_rsrc((void *) a.part, (short) 0, 0x7FFFFFFF, 0x00020000)
                                                       : __builtin_amdgcn_make_buffer_rsrc((void *) Y, (short) 0, (int) a.y_bytes, 0x00020000);
            const __amdgpu_buffer_rsrc_t rrs =
                __builtin_amdgcn_make_buffer_rsrc((void *) (MODE == 3 ? a.res + bz * a.y_bstride : Y), (short) 0, (int) a.y_bytes, 0x00020000);
            float4v bv[FM][4];
            if constexpr (MODE == 2 || MODE == 3) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) bv[i][qq] = *reinterpret_cast<const float4v *>(a.bias + mw0 + i * 32 + qq * 8 + lk * 4);
            }
            unsigned yoff[NG > 1 ? 2 : 1][JG][FM][4];
            u32x2    rv[NG > 1 ? 2 : 1][JG][FM][4];
            auto prep = [&](int j0, int b) __attribute__((always_inline)) {
#pragma unroll
                for (int jj = 0; jj < JG; ++jj) {
                    const int  px  = nw0 + (j0 + jj) * 32 + lrow;
                    const int  pn  = px / a.OHWp;
                    const int  pr  = px - pn * a.OHWp;
                    const bool pok = (px < a.Pv) & (pr < a.OHW);
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) {
                            const int  ocb = (mw0 + i * 32 + qq * 8 + lk * 4) >> 2;
                            const bool ok  = pok & (ocb < a.Coutb);
                            if constexpr (PARTIAL)
                                yoff[b][jj][i][qq] = ok ? (unsigned) (((split * a.Coutb + ocb) * a.P + pn * a.OHW + pr) * 16) : kInvalid;
                            else yoff[b][jj][i][qq] = ok ? (unsigned) (((pn * a.y_pstride + ocb) * a.OHW + pr) * 8) : kInvalid;
                            if constexpr (MODE == 3) rv[b][jj][i][qq] = __builtin_amdgcn_raw_buffer_load_b64(rrs, yoff[b][jj][i][qq], 0, kStreamLoad);
                        }
                }
            };
            prep(0, 0);
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const int j0 = g * JG, b = g & 1;
                if (g + 1 < NG) prep(j0 + JG, b ^ 1);
#pragma unroll
                for (int jj = 0; jj < JG; ++jj)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) {
                            const int j  = j0 + jj;
                            const int oc = mw0 + i * 32 + qq * 8 + lk * 4;
                            float4v   v  = {acc[i][j][qq * 4 + 0], acc[i][j][qq * 4 + 1], acc[i][j][qq * 4 + 2], acc[i][j][qq * 4 + 3]};
                            if constexpr (PARTIAL) {
                                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), yrs, yoff[b][jj][i][qq], 0,
                                                                       MODE == 4 ? kCoherent : kStreamStore);
                                continue;
                            }
                            if constexpr (MODE == 2 || MODE == 3) v += bv[i][qq];
                            float4v r = {0.f, 0.f, 0.f, 0.f};
                            if constexpr (MODE == 3) r = h4_to_f4(__builtin_bit_cast(half4, rv[b][jj][i][qq]));
                            if (MODE == 3 && a.has_res != 2) v += r;
                            v.x = apply_act(v.x, ACT, a.lo, a.hi);
                            v.y = apply_act(v.y, ACT, a.lo, a.hi);
                            v.z = apply_act(v.z, ACT, a.lo, a.hi);
                            v.w = apply_act(v.w, ACT, a.lo, a.hi);
                            if (MODE == 3 && a.has_res == 2) v += r;
                            if (oc + 0 >= a.Cout) v.x = 0.f;
                            if (oc + 1 >= a.Cout) v.y = 0.f;
                            if (oc + 2 >= a.Cout) v.z = 0.f;
                            if (oc + 3 >= a.Cout) v.w = 0.f;
                            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, yoff[b][jj][i][qq], 0, kStreamStore);
                        }
            }
        };
        using I = std::integral_constant<int, 0>;
        if (a.omode == OMODE_PARTIAL) {
            if (!a.cnt) return finish(I {}, I {});
            finish(std::integral_constant<int, 4> {}, I {});
            if (!splitk_last_arrival(a, flag)) return;
            splitk_gather<FM, FN>(a, acc, mw0, nw0, split, lane);
            // the workgroup that arrived last finishes the tile from the summed partials
        } else if (a.omode == OMODE_RAW) return finish(std::integral_constant<int, 1> {}, I {});
        auto with_act = [&](auto mode_c) __attribute__((always_inline)) {
            switch (a.act) {
                case VKHIP_ACT_RELU: finish(mode_c, std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
                case VKHIP_ACT_RELU6: finish(mode_c, std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
                case VKHIP_ACT_CLIP: finish(mode_c, std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
                case VKHIP_ACT_HARDSWISH: finish(mode_c, std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
                case VKHIP_ACT_SILU: finish(mode_c, std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
                case VKHIP_ACT_HARDSIGMOID: finish(mode_c, std::integral_constant<int, VKHIP_ACT_HARDSIGMOID> {}); break;
                default: finish(mode_c, std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
            }
        };
        if (a.has_res) with_act(std::integral_constant<int, 3> {});
        else with_act(std::integral_constant<int, 2> {});
    }

    template <int I, int N, typename F>
    __device__ __forceinline__ void static_for(F &&f) {
        if constexpr (I < N) {
            f(std::integral_constant<int, I> {});
            static_for<I + 1, N>(f);
        }
    }

    // D = prefetch distance in stages: stage ks+D is issued while stage ks computes (D+1 register
    // sets for B, D+2 LDS buffers for A).
    template <int FM, int FN, int WM, int WN, int BMODE, int D>
    __global__ __launch_bounds__(kThreads, (16 * FM * FN + 16 * FN * (D + 1) + 4 * FM + 40 <= 256) ? 2 : 1) void conv_bd_kernel(GemmArgs a) {
        static_assert(WM * WN == 4, "4 waves");
        static_assert(BMODE == BMODE_1X1 || BMODE == BMODE_ALIGNED || BMODE == BMODE_GENERAL, "B mode");
        constexpr int BM     = WM * 32 * FM;
        constexpr int MF     = BM / 32;            // m fragments per tile
        constexpr int ASTAGE = BM * kBK * 2;       // bytes of one A stage
        constexpr int NA     = ASTAGE / (kThreads * 16); // LDS DMA instructions per thread and stage
        constexpr int NB     = 4 * FN * 2;         // B loads per lane and stage
        constexpr int NBUF   = D + 2;
        static_assert(NA >= 1 && ASTAGE % (kThreads * 16) == 0, "A stage");
        __shared__ __attribute__((aligned(16))) unsigned char As[NBUF][ASTAGE];

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wmi  = wave / WN;
        const int wni  = wave % WN;

        const int lin    = xcd_remap(blockIdx.x, gridDim.x);
        const int m_tile = lin % a.m_tiles;
        const int n_tile = lin / a.m_tiles;
        const int m0     = m_tile * BM;
        const int n0     = n_tile * (WN * 32 * FN);
        const int split  = blockIdx.y;
        const int bz     = blockIdx.z;
        const int wm0    = wmi * 32 * FM;
        const int wn0    = wni * 32 * FN;

        const uint2         *X  = a.x + bz * a.x_bstride;
        const unsigned char *Wt = reinterpret_cast<const unsigned char *>(a.w + bz * a.w_bstride) + (long long) m_tile * a.nsteps * ASTAGE;

        const int ks_begin = split * a.steps_per_split;
        const int ks_end   = min(a.nsteps, ks_begin + a.steps_per_split);

        // Buffer resources. Range checks apply to the per-lane offset; every guard (padding tap,
        // pixel past P, K tail, stage past ks_end) therefore lives in the VGPR offset, while the
        // wave-uniform part of each address (channel slot, tap shift, stage) goes in the SGPR
        // offset. The activation resource is rebased by `lead` bytes so per-lane pixel offsets,
        // which include the top/left padding shift, are never negative.
        const int lead = (a.PT * a.W + a.PL) * 8;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) ((const char *) X - lead), (short) 0,
                                                                             (int) a.x_bytes + lead, 0x00020000);
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *) Wt, (short) 0, ks_end * ASTAGE, 0x00020000);
        constexpr unsigned kInvalid = 0x80000000u;
        const int hw8    = a.HW * 8;
        const int kslots = min(a.Kslots, ks_end * 16);
        const int g      = lane >> 5; // which pair of slots of a 16-K step this lane supplies

        // this lane's fragment columns (output pixels): offset of (n, slot 2g, iy0, ix0) and, for
        // the shared-tap gather, the set of taps that land inside the image
        unsigned pbase[FN];
        unsigned tapok[FN];
        int      piy[FN], pix[FN];
        bool     pv[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int p  = n0 + wn0 + 32 * j + (lane & 31);
            pv[j]        = p < a.P;
            const int pp = pv[j] ? p : 0;
            const int n  = pp / a.OHW;
            const int r  = pp - n * a.OHW;
            const int oy = r / a.OW;
            const int ox = r - oy * a.OW;
            piy[j]       = oy * a.SH - a.PT;
            pix[j]       = ox * a.SW - a.PL;
            pbase[j]     = (unsigned) ((n * a.x_pstride * a.HW + piy[j] * a.W + pix[j]) * 8 + lead + 2 * g * hw8);
            tapok[j]     = 0;
            if constexpr (BMODE == BMODE_ALIGNED) {
                for (int t = 0; t < a.Kslots / a.Cinb; ++t) {
                    const int ky = t / a.KW, kx = t - (t / a.KW) * a.KW;
                    const bool ok = pv[j] & ((unsigned) (piy[j] + ky * a.DH) < (unsigned) a.H) & ((unsigned) (pix[j] + kx * a.DW) < (unsigned) a.W);
                    tapok[j] |= (ok ? 1u : 0u) << t;
                }
            }
            if (!pv[j]) pbase[j] = kInvalid;
        }

        u32x2 breg[D + 1][4][FN][2];

        auto issue_a = [&](int ks) __attribute__((always_inline)) {
            unsigned char *dst = As[ks % NBUF];
#pragma unroll
            for (int r = 0; r < NA; ++r) {
                const int chunk = (r * 4 + wave) * 1024; // wave-uniform LDS base of this 1 KB piece
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *) (dst + chunk), 16,
                                                         (unsigned) (chunk + lane * 16) + (unsigned) (ks * ASTAGE), 0, 0, 0);
            }
        };
        auto issue_b = [&](int ks, auto set_c) __attribute__((always_inline)) {
            constexpr int S = decltype(set_c)::value;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int s0 = ks * 16 + kk * 4; // first slot of this 16-K step (wave-uniform)
                if constexpr (BMODE == BMODE_1X1) {
                    const unsigned so = (unsigned) (s0 * hw8);
                    if (s0 + 4 <= kslots) {
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
                            breg[S][kk][j][0] = __builtin_amdgcn_raw_buffer_load_b64(xrs, pbase[j], so, 0);
                            breg[S][kk][j][1] = __builtin_amdgcn_raw_buffer_load_b64(xrs, pbase[j], so + hw8, 0);
                        }
                    } else { // K tail: slots past Kslots read zero
                        const bool k0 = s0 + 2 * g < kslots, k1 = s0 + 2 * g + 1 < kslots;
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
                            breg[S][kk][j][0] = __builtin_amdgcn_raw_buffer_load_b64(xrs, k0 ? pbase[j] : kInvalid, so, 0);
                            breg[S][kk][j][1] = __builtin_amdgcn_raw_buffer_load_b64(xrs, k1 ? pbase[j] : kInvalid, so + hw8, 0);
                        }
                    }
                } else if constexpr (BMODE == BMODE_ALIGNED) {
                    // Cinb % 4 == 0: the 4 slots of the step share one tap
                    const int tap = s0 / a.Cinb;
                    const int cb  = s0 - tap * a.Cinb;
                    const int ky  = tap / a.KW;
                    const int kx  = tap - ky * a.KW;
                    const unsigned so = (unsigned) (cb * hw8 + (ky * a.DH * a.W + kx * a.DW) * 8);
                    const bool kin = s0 < kslots;
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const unsigned vo = (kin && ((tapok[j] >> tap) & 1u)) ? pbase[j] : kInvalid;
                        breg[S][kk][j][0] = __builtin_amdgcn_raw_buffer_load_b64(xrs, vo, so, 0);
                        breg[S][kk][j][1] = __builtin_amdgcn_raw_buffer_load_b64(xrs, vo, so + hw8, 0);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int slot = s0 + 2 * g + e;
                        const int tap  = slot / a.Cinb;
                        const int cb   = slot - tap * a.Cinb;
                        const int ky   = tap / a.KW;
                        const int kx   = tap - ky * a.KW;
                        const int dy = ky * a.DH, dx = kx * a.DW;
                        const int o  = (cb - 2 * g) * hw8 + (dy * a.W + dx) * 8;
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
                            const bool ok = (slot < kslots) & pv[j] & ((unsigned) (piy[j] + dy) < (unsigned) a.H) & ((unsigned) (pix[j] + dx) < (unsigned) a.W);
                            breg[S][kk][j][e] = __builtin_amdgcn_raw_buffer_load_b64(xrs, ok ? pbase[j] + (unsigned) o : kInvalid, 0, 0);
                        }
                    }
                }
            }
        };

        float16v acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        // vmcnt wait immediate (gfx9 encoding: vmcnt[3:0] | expcnt[6:4]=7 | lgkmcnt[11:8]=15 | vmcnt[5:4] at [15:14])
        constexpr int kAhead     = D * (NA + NB) < 63 ? D * (NA + NB) : 63; // loads that may stay in flight
        constexpr int kWaitStage = (kAhead & 15) | (7 << 4) | (15 << 8) | ((kAhead >> 4) << 14);
        constexpr int kWaitAll   = (7 << 4) | (15 << 8);

        // A fragments are double buffered: step kk+1's LDS reads are in flight while step kk's
        // MFMAs issue.
        auto compute = [&](int ks, auto set_c) __attribute__((always_inline)) {
            constexpr int S = decltype(set_c)::value;
            const unsigned char *Ab = As[ks % NBUF] + ((wmi * FM) * 64 + lane) * 16;
            half8 fa[2][FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[0][i] = *reinterpret_cast<const half8 *>(Ab + i * 1024);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                if (kk < 3) {
#pragma unroll
                    for (int i = 0; i < FM; ++i) fa[(kk + 1) & 1][i] = *reinterpret_cast<const half8 *>(Ab + ((kk + 1) * MF + i) * 1024);
                }
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const u32x4 bv = u32x4_make(breg[S][kk][j][0].x, breg[S][kk][j][0].y, breg[S][kk][j][1].x, breg[S][kk][j][1].y);
                    const half8 fb = __builtin_bit_cast(half8, bv);
#pragma unroll
                    for (int i = 0; i < FM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk & 1][i], fb, acc[i][j], 0, 0, 0);
                }
                if (kk < 3) Interleave<0, FM * FN, FM, 0, 0>::apply();
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // Stage ks: issue stage ks+1 (A into LDS buffer (ks+1)%3, B into the other register set),
        // wait until stage ks has landed, barrier (every wave's share of A is in LDS and every wave
        // is done with stage ks-1, so the next issue may reuse buffer (ks+2)%3 = (ks-1)%3), compute.
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        // The loop runs whole groups of D+1 stages (register sets are compile-time indices) and has a
        // single exit, so the accumulators stay in place; the last < D+1 stages run after it. Each
        // stage issues stage ks+D (A into LDS buffer (ks+D)%(D+2), B into the set freed by stage
        // ks-1), waits until stage ks has landed, then barriers: every wave's share of A is in LDS
        // and every wave is done with stage ks-1, whose buffer the next issue reuses. Issues past
        // ks_end read zeros (out-of-range buffer offsets) into idle buffers.
        if (ks_begin < ks_end) {
            static_for<0, D>([&](auto p) {
                issue_a(ks_begin + p.value);
                issue_b(ks_begin + p.value, p);
            });
            int ks = ks_begin;
            for (; ks + (D + 1) <= ks_end; ks += D + 1) {
                static_for<0, D + 1>([&](auto p) {
                    constexpr int P = decltype(p)::value;
                    issue_a(ks + P + D);
                    issue_b(ks + P + D, std::integral_constant<int, (P + D) % (D + 1)> {});
                    __builtin_amdgcn_s_waitcnt(kWaitStage);
                    __asm__ volatile("s_barrier" ::: "memory");
                    compute(ks + P, p);
                });
            }
            static_for<0, D>([&](auto p) {
                if (ks + p.value < ks_end) {
                    __builtin_amdgcn_s_waitcnt(kWaitAll);
                    __asm__ volatile("s_barrier" ::: "memory");
                    compute(ks + p.value, p);
                }
            });
        }

        gemm_epilogue<FM, FN>(a, acc, m0 + wm0, n0 + wn0, split, bz, lane, reinterpret_cast<volatile int *>(&As[0][0]));
    }

    // ------------------------------------------------------------------ LDS-staged epilogue
    // Epilogue of a BM x 128 tile through LDS, for dense NC4HW4 outputs with an even pixel count
    // per image: the residual tile reaches LDS by buffer-load-to-LDS, one 1 KB row (128 pixels of
    // one channel block) per copy; each lane finishes its accumulators in place there (bias,
    // residual, activation, fp16); then whole rows leave as 16-byte stores. Against the register
    // epilogue (one 8-byte load and one 8-byte store per lane per 4-channel fragment quarter) it
    // issues half the vector-memory instructions, each moving a contiguous kilobyte. `sm` must hold
    // BM / 4 rows of 1040 bytes; the caller has finished reading it.
    template <int FM, int FN, int BM, int BN, int NW>
    __device__ __forceinline__ void gemm_epilogue_lds(const GemmArgs &a, float16v (&acc)[FM][FN], unsigned char *sm, int m0, int n0, int wm0,
                                                      int wn0, int wave, int lane) {
        static_assert(BN == 128, "one copy per channel-block row");
        constexpr int      RS = BN * 8 + 16; // row stride, padded so the two half-waves of an 8-byte access use other banks
        constexpr int      ROWS = BM / 4;
        constexpr unsigned kInvalid = 0x80000000u;
        const int          lrow = lane & 31, lk = lane >> 5;
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rrs =
            __builtin_amdgcn_make_buffer_rsrc((void *) (a.has_res ? a.res : a.y), (short) 0, a.has_res ? (int) a.y_bytes : 0, 0x00020000);
        // this lane's pixel pair of every row
        const int  px  = n0 + 2 * lane;
        const int  pn  = px / a.OHWp;
        const int  pr  = px - pn * a.OHWp;
        const bool pok = px < a.Pv && pr < a.OHW;
        auto goff = [&](int r) __attribute__((always_inline)) {
            const int ocb = (m0 >> 2) + r;
            return pok && ocb < a.Coutb ? (unsigned) (((pn * a.y_pstride + ocb) * a.OHW + pr) * 8) : kInvalid;
        };
        __syncthreads(); // every wave is done with the ring
        if (a.has_res) {
#pragma unroll
            for (int r = wave; r < ROWS; r += NW) {
#if defined(__HIP_DEVICE_COMPILE__) // `sm` is a generic pointer here: the host pass rejects its cast to the LDS space
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rrs, (__attribute__((address_space(3))) void *) (sm + r * RS), 16, goff(r), 0, 0, kStreamLoad);
#endif
            }
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        }
        __syncthreads();
        auto finish = [&](auto act_c) __attribute__((always_inline)) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int     rl = (wm0 + i * 32 + qq * 8 + lk * 4) >> 2;
                    const int     oc = m0 + rl * 4;
                    const float4v bv = *reinterpret_cast<const float4v *>(a.bias + oc);
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        u32x2  *e = reinterpret_cast<u32x2 *>(sm + rl * RS + (wn0 + j * 32 + lrow) * 8);
                        float4v v = {acc[i][j][qq * 4 + 0], acc[i][j][qq * 4 + 1], acc[i][j][qq * 4 + 2], acc[i][j][qq * 4 + 3]};
                        v += bv;
                        float4v r = {0.f, 0.f, 0.f, 0.f};
                        if (a.has_res) r = h4_to_f4(__builtin_bit_cast(half4, *e));
                        if (a.has_res != 2) v += r;
                        v.x = apply_act(v.x, ACT, a.lo, a.hi);
                        v.y = apply_act(v.y, ACT, a.lo, a.hi);
                        v.z = apply_act(v.z, ACT, a.lo, a.hi);
                        v.w = apply_act(v.w, ACT, a.lo, a.hi);
                        if (a.has_res == 2) v += r;
                        if (oc + 0 >= a.Cout) v.x = 0.f;
                        if (oc + 1 >= a.Cout) v.y = 0.f;
                        if (oc + 2 >= a.Cout) v.z = 0.f;
                        if (oc + 3 >= a.Cout) v.w = 0.f;
                        *e = __builtin_bit_cast(u32x2, f4_to_h4(v));
                    }
                }
        };
        switch (a.act) {
            case VKHIP_ACT_RELU: finish(std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
            case VKHIP_ACT_RELU6: finish(std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
            case VKHIP_ACT_CLIP: finish(std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
            case VKHIP_ACT_HARDSWISH: finish(std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
            case VKHIP_ACT_SILU: finish(std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
            case VKHIP_ACT_HARDSIGMOID: finish(std::integral_constant<int, VKHIP_ACT_HARDSIGMOID> {}); break;
            default: finish(std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
        }
        __syncthreads();
#pragma unroll
        for (int r = wave; r < ROWS; r += NW)
            __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4 *>(sm + r * RS + lane * 16), yrs, goff(r), 0, kStreamStore);
    }

    // ------------------------------------------------------------------ LDS-DMA GEMM kernel
    // Third main loop, for dense B operands: 1x1 stride-1 convs over images with an even pixel
    // count, and the Winograd position GEMMs. Both operands reach LDS through the buffer unit
    // (buffer_load ... lds, 16 bytes per lane) with no VGPR staging:
    //   A  prepacked weights in MFMA fragment order ([m_tile][stage][kk][m_frag][lane][8 halves]);
    //   B  [slot][pixel] stage of 16 NC4HW4 channel slots x BN pixels, one lane per pixel pair of
    //      one slot (a pair never straddles two images because the pixel count per image is even).
    // Four waves in a 2x2 grid, each owning a (32FM) x (32FN) block; with FM = FN = 4 the
    // workgroup tile is 256 x 256, which keeps the operand bytes per MFMA (and so the address-unit
    // and LDS traffic) low enough for the matrix cores. Two LDS stages: stage ks+1 streams in while
    // stage ks computes (one barrier per stage). A fragments read with ds_read_b128, B fragments
    // with two ds_read_b64 (slots 2g and 2g+1 of the lane's pixel), both double buffered across
    // the 16-K steps.
    // PS = 16: stride-2 1x1 convs. Each lane copies one output pixel's input pixel (2oy, 2ox)
    // together with its right neighbour (16 bytes, the neighbour unused), so B columns sit 16 bytes
    // apart in LDS.
    // XS: the input is scaled per (image, channel) first (a squeeze-excite scale folded into the
    // conv that consumes it). Each stage then also copies the scale slice of its 64 K values for
    // up to 8 consecutive images (lane l: image l/8, halves (l%8)*8..+7) into 1 KB after the B
    // stage, and every B fragment is multiplied by the scales of its column's image before the
    // MFMA (fp16 products, rounded like the separate Mul's fp16 store).
    // LE: the LDS-staged epilogue (gemm_epilogue_lds; GEMM epilogue mode, BN = 128, even pixel
    // count per image).
    template <int FM, int FN, int NS, int WM, int WN, int PS = 8, bool XS = false, bool LE = false>
    __global__ __launch_bounds__(64 * WM * WN, 1) void conv_dma_kernel(GemmArgs a) {
        constexpr int NW     = WM * WN; // waves
        constexpr int BM     = 32 * FM * WM;
        constexpr int BN     = 32 * FN * WN;
        constexpr int MF     = BM / 32;
        constexpr int ASTAGE = BM * kBK * 2;
        constexpr int BSTAGE = BN * kBK * 2 * PS / 8;
        constexpr int NA     = ASTAGE / (NW * 1024);
        constexpr int NB     = BSTAGE / (NW * 1024);
        static_assert(NA >= 1 && NB >= 1 && ASTAGE % (NW * 1024) == 0 && BSTAGE % (NW * 1024) == 0, "stage split");
        constexpr int BPB    = BN * PS / 1024; // 1 KB pixel blocks per slot row of the B stage
        constexpr int SSTAGE = XS ? 1024 : 0;  // scale slice of the stage
        constexpr int STAGE  = ASTAGE + BSTAGE + SSTAGE;
        static_assert(!XS || PS == 8, "input scale on dense stride-1 columns only");
        __shared__ __attribute__((aligned(16))) unsigned char sm[NS * STAGE + (XS ? 1024 : 0)]; // + spare for the idle scale copies

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wmi  = wave / WN;
        const int wni  = wave % WN;

        const int lin    = xcd_remap(blockIdx.x, gridDim.x);
        const int m_tile = lin % a.m_tiles;
        const int n_tile = lin / a.m_tiles;
        const int m0     = m_tile * BM;
        const int n0     = n_tile * BN;
        const int split  = blockIdx.y;
        const int bz     = blockIdx.z;
        const int wm0    = wmi * 32 * FM;
        const int wn0    = wni * 32 * FN;

        const uint2         *X  = a.x + bz * a.x_bstride;
        const unsigned char *Wt = reinterpret_cast<const unsigned char *>(a.w + bz * a.w_bstride) + (long long) m_tile * a.nsteps * ASTAGE;
        const int ks_begin = split * a.steps_per_split;
        const int ks_end   = min(a.nsteps, ks_begin + a.steps_per_split);
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) X, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *) Wt, (short) 0, ks_end * ASTAGE, 0x00020000);
        constexpr unsigned kInvalid = 0x80000000u;
        const int hw8 = a.HW * 8;

        // B copy: instruction r of this wave fills 1 KB chunk c = r*NW + wave of the stage, i.e.
        // slot c / BPB, pixels (c % BPB)*128 + 2*lane (+1). Per-lane pixel bases are fixed.
        unsigned pbase[BPB];
#pragma unroll
        for (int pb = 0; pb < BPB; ++pb) {
            // virtual columns: OHWp per image (the padding column of an odd image reads the next
            // 8 bytes, whatever they hold; its outputs are never stored)
            if constexpr (PS == 8) {
                const int p = n0 + pb * 128 + 2 * lane;
                const int n = p / a.OHWp;
                pbase[pb]   = p < a.Pv ? (unsigned) ((n * a.x_pstride * a.HW + (p - n * a.OHWp)) * 8) : kInvalid;
            } else {
                const int p  = n0 + pb * 64 + lane;
                const int n  = p / a.OHW;
                const int r  = p - n * a.OHW;
                const int oy = r / a.OW;
                pbase[pb]    = p < a.P ? (unsigned) ((n * a.x_pstride * a.HW + (a.SH * oy) * a.W + a.SW * (r - oy * a.OW)) * 8) : kInvalid;
            }
        }
        // XS: images n_first .. n_first+7 of the scale table; lane l copies image n_first + l/8
        const int      n_first = n0 / a.OHWp;
        const unsigned xs_row  = (unsigned) a.Cinb * 8u;
        const int      img     = n_first + (lane >> 3);
        const unsigned sbase   = XS && img * a.OHWp < a.Pv ? (unsigned) img * xs_row : kInvalid;
        const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc((void *) (XS ? a.xs : a.x), (short) 0, XS ? (int) a.xs_bytes : 0, 0x00020000);
        auto issue = [&](int ks, int buf) __attribute__((always_inline)) {
            unsigned char *dst = sm + buf * STAGE;
#pragma unroll
            for (int r = 0; r < NA; ++r) {
                const int chunk = (r * NW + wave) * 1024;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *) (dst + chunk), 16,
                                                         (unsigned) (chunk + lane * 16) + (unsigned) (ks * ASTAGE), 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < NB; ++r) {
                const int c    = r * NW + wave;
                const int slot = ks * 16 + c / BPB; // wave-uniform
                const unsigned vo = slot < a.Kslots ? pbase[c % BPB] : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (dst + ASTAGE + c * 1024), 16, vo,
                                                         (unsigned) (slot * hw8), 0, 0);
            }
            if constexpr (XS) {
                // every wave issues one copy so the per-wave copy counts (the vmcnt waits) stay
                // equal; waves other than 0 copy nothing into the spare block
                const int  k0  = ks * kBK + (lane & 7) * 8;
                const bool ok  = wave == 0 && sbase != kInvalid && k0 < a.Kslots * 4;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (__attribute__((address_space(3))) void *) (wave == 0 ? dst + ASTAGE + BSTAGE : sm + NS * STAGE),
                                                         16, ok ? sbase + (unsigned) (k0 * 2) : kInvalid, 0, 0, 0);
            }
        };

        float16v acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        const int g = lane >> 5;
        // XS: byte offset of each fragment column's image row in the stage's scale slice
        int simg[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int p = n0 + wn0 + 32 * j + (lane & 31);
            simg[j]     = (p < a.Pv ? p / a.OHWp - n_first : 0) * (kBK * 2) + g * 16;
        }
        auto compute = [&](int buf, int next_ks, int next_buf) __attribute__((always_inline)) {
            const unsigned char *Ab = sm + buf * STAGE + ((wmi * FM) * 64 + lane) * 16;
            const unsigned char *Bb = sm + buf * STAGE + ASTAGE + (2 * g * BN + wn0 + (lane & 31)) * PS;
            const unsigned char *Sb = sm + buf * STAGE + ASTAGE + BSTAGE;
            half8 fa[2][FM], fb[2][FN];
            auto rd = [&](int kk, int d) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const u32x2 lo = *reinterpret_cast<const u32x2 *>(Bb + (kk * 4 * BN + 32 * j) * PS);
                    const u32x2 hi = *reinterpret_cast<const u32x2 *>(Bb + ((kk * 4 + 1) * BN + 32 * j) * PS);
                    fb[d][j] = __builtin_bit_cast(half8, u32x4_make(lo.x, lo.y, hi.x, hi.y));
                    // halves (kk*4 + 2g)*4 .. +8 of the column's image: slots 2g, 2g+1 of step kk
                    if constexpr (XS) fb[d][j] *= *reinterpret_cast<const half8 *>(Sb + simg[j] + kk * 32);
                }
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[d][i] = *reinterpret_cast<const half8 *>(Ab + (kk * MF + i) * 1024);
            };
            // Each 16-K step issues its MFMAs with the next step's LDS reads interleaved between
            // them (the scheduler would otherwise reuse one fragment register and wait on every read).
            rd(0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // the copies of a later stage go out between the first step's MFMAs
                if (kk == 0 && next_ks >= 0) issue(next_ks, next_buf);
                if (kk < 3) rd(kk + 1, (kk + 1) & 1);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk & 1][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
                if (kk == 0) StepSchedule<0, FM * FN, FM + (XS ? 3 : 2) * FN, (XS ? 8 : 4) * FN, NA + NB + (XS ? 1 : 0)>::apply();
                else if (kk < 3) StepSchedule<0, FM * FN, FM + (XS ? 3 : 2) * FN, (XS ? 8 : 4) * FN>::apply();
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // NS LDS stages, prefetch distance NS-1: stage ks waits for its own copies (the NS-2 later
        // stages may stay in flight), barriers (all waves' copies landed; all waves done with
        // stage ks-1, whose buffer the next issue refills), issues stage ks+NS-1, computes.
        constexpr int NPW    = NA + NB + (XS ? 1 : 0); // copies per wave per stage
        constexpr int kAhead = NS < 2 ? 0 : ((NS - 2) * NPW < 63 ? (NS - 2) * NPW : 63);
        constexpr int kWait  = (kAhead & 15) | (7 << 4) | (15 << 8) | ((kAhead >> 4) << 14);
        if constexpr (NS == 1) {
            // one stage (GEMMs with a single K stage per split): copy, wait, compute; no LDS ring,
            // so several workgroups fit on a CU and overlap each other's copies and epilogues
            for (int ks = ks_begin; ks < ks_end; ++ks) {
                if (ks > ks_begin) __asm__ volatile("s_barrier" ::: "memory");
                issue(ks, 0);
                __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
                __asm__ volatile("s_barrier" ::: "memory");
                compute(0, -1, 0);
            }
        } else if (ks_begin < ks_end) {
#pragma unroll
            for (int d = 0; d < NS - 1; ++d)
                if (ks_begin + d < ks_end) issue(ks_begin + d, d);
            for (int ks = ks_begin; ks < ks_end; ++ks) {
                const int rel = ks - ks_begin;
                if (ks + NS - 2 < ks_end) __builtin_amdgcn_s_waitcnt(kWait);
                else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // tail: nothing later in flight
                __asm__ volatile("s_barrier" ::: "memory");
                compute(rel % NS, ks + NS - 1 < ks_end ? ks + NS - 1 : -1, (rel + NS - 1) % NS);
            }
        }
        static_assert(!LE || NS * STAGE >= (BM / 4) * 1040, "the LDS-staged epilogue fits the ring");
        if constexpr (LE) {
            unsigned char *smg = sm;
            gemm_epilogue_lds<FM, FN, BM, BN, NW>(a, acc, smg, m0, n0, wm0, wn0, wave, lane);
        }
        else gemm_epilogue<FM, FN>(a, acc, m0 + wm0, n0 + wn0, split, bz, lane, reinterpret_cast<volatile int *>(sm));
    }

    // ------------------------------------------------------------------ persistent LDS-DMA GEMM kernel
    // conv_dma_kernel's operands, stage layout and 16-K step, with the copies and the math split
    // over two groups of waves, run by one workgroup per CU that walks a strided list of tiles.
    // Why: in conv_dma_kernel every wave both copies its share of each K stage and stores its
    // epilogue, and the vector-memory counter retires in issue order, so a wave that waits for its
    // next copies also waits for every store it issued before them; and all workgroups of a launch
    // start together, so the whole GPU loads, then stores, in lockstep. Measured on 1x1 layers with
    // a residual, the load phase and the epilogue phase add up instead of overlapping. Here:
    //   * NP = 4 producer waves only copy: each issues its quarter of every K stage's A and B
    //     chunks (buffer-load-to-LDS) into an NS-stage ring, NS-1 stages ahead, across tile
    //     boundaries, and waits only for its own copies; with the stage's copies it also copies
    //     the tile's bias slice into the stage that holds the tile's last K step;
    //   * the WM x WN consumer waves only compute and store: at the first K stage of a tile they
    //     load its residual into registers (hidden behind the tile's MFMAs), run the 16-K steps
    //     from LDS, then apply bias (from LDS), residual and activation and store. Their counter
    //     holds only residual loads and stores, so the epilogue of tile t never waits for copies
    //     and the producers keep streaming tile t+1 meanwhile.
    // One s_barrier per K stage pairs the two groups: before it the producers wait for stage s's
    // copies and the consumers finish stage s-1; after it the consumers read stage s and the
    // producers refill stage s-1's buffer.
    // Tile order: at step it, XCD x runs tiles (it*8 + x)*per + 0..per-1 (per = gridDim.x / 8;
    // workgroup ids are dealt to the XCDs round-robin), so the tiles an XCD runs at once are
    // consecutive and share their B columns (tile % m_tiles is the M tile) in its L2.
    // GEMM epilogue mode only (no split-K partials, no Winograd positions).
    constexpr int kProducers = 4;
    template <int FM, int FN, int NS, int WM, int WN, int PS = 8>
    __global__ __launch_bounds__(64 * (WM * WN + kProducers), 1) void conv_dma_persist_kernel(GemmArgs a) {
        constexpr int NC     = WM * WN;       // consumer waves
        constexpr int NP     = kProducers;
        constexpr int BM     = 32 * FM * WM;
        constexpr int BN     = 32 * FN * WN;
        constexpr int MF     = BM / 32;
        constexpr int ASTAGE = BM * kBK * 2;
        constexpr int BSTAGE = BN * kBK * 2 * PS / 8;
        constexpr int NA     = ASTAGE / (NP * 1024);  // A chunks per producer per stage
        constexpr int NB     = BSTAGE / (NP * 1024);  // B chunks per producer per stage
        static_assert(NS >= 2 && NA >= 1 && NB >= 1 && ASTAGE % (NP * 1024) == 0 && BSTAGE % (NP * 1024) == 0, "stage split");
        static_assert(BM * 4 <= 1024, "bias slice fits one 1 KB copy");
        constexpr int BPB    = BN * PS / 1024;
        constexpr int STAGE  = ASTAGE + BSTAGE + 1024; // + the bias slice
        constexpr int NPP    = NA + NB + 1;            // copies per producer per stage (one bias copy each; 3 of them idle)
        static_assert((NS - 1) * NPP <= 63, "copies in flight fit the counter");
        __shared__ __attribute__((aligned(16))) unsigned char sm[NS * STAGE + 1024]; // + a spare block for idle bias copies

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

        const int ntiles = a.m_tiles * a.n_tiles;
        const int per    = gridDim.x >> 3;
        const int first  = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
        const int ntw    = first < ntiles ? (ntiles - first + 8 * per - 1) / (8 * per) : 0; // tiles of this workgroup
        const int nst    = a.nsteps;
        const int S      = ntw * nst;                                                          // K stages of this workgroup
        if (S == 0) return;
        auto tile_of = [&](int it) { return first + it * 8 * per; };
        constexpr unsigned kInvalid = 0x80000000u;

        if (wave >= NC) {
            // ---------------- producer
            const int pw = wave - NC;
            const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
            const __amdgpu_buffer_rsrc_t wrs =
                __builtin_amdgcn_make_buffer_rsrc((void *) a.w, (short) 0, a.m_tiles * nst * ASTAGE, 0x00020000);
            const __amdgpu_buffer_rsrc_t brs =
                __builtin_amdgcn_make_buffer_rsrc((void *) a.bias, (short) 0, a.m_tiles * BM * 4, 0x00020000);
            const int hw8 = a.HW * 8;
            int       i_it = 0, i_ks = 0, m_tile = 0;
            unsigned  pbase[BPB];
            auto set_issue_tile = [&](int it) __attribute__((always_inline)) {
                const int t  = tile_of(it);
                m_tile       = t % a.m_tiles;
                const int n0 = (t / a.m_tiles) * BN;
#pragma unroll
                for (int pb = 0; pb < BPB; ++pb) {
                    if constexpr (PS == 8) {
                        const int p = n0 + pb * 128 + 2 * lane;
                        const int n = p / a.OHWp;
                        pbase[pb]   = p < a.Pv ? (unsigned) ((n * a.x_pstride * a.HW + (p - n * a.OHWp)) * 8) : kInvalid;
                    } else {
                        const int p  = n0 + pb * 64 + lane;
                        const int n  = p / a.OHW;
                        const int r  = p - n * a.OHW;
                        const int oy = r / a.OW;
                        pbase[pb]    = p < a.P ? (unsigned) ((n * a.x_pstride * a.HW + (a.SH * oy) * a.W + a.SW * (r - oy * a.OW)) * 8) : kInvalid;
                    }
                }
            };
            auto issue = [&](int buf) __attribute__((always_inline)) {
                unsigned char *dst = sm + buf * STAGE;
                const unsigned wofs = (unsigned) ((m_tile * nst + i_ks) * ASTAGE);
#pragma unroll
                for (int r = 0; r < NA; ++r) {
                    const int chunk = (r * NP + pw) * 1024;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *) (dst + chunk), 16,
                                                             (unsigned) (chunk + lane * 16) + wofs, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < NB; ++r) {
                    const int c    = r * NP + pw;
                    const int slot = i_ks * 16 + c / BPB; // wave-uniform
                    const unsigned vo = slot < a.Kslots ? pbase[c % BPB] : kInvalid;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (dst + ASTAGE + c * 1024), 16, vo,
                                                             (unsigned) (slot * hw8), 0, 0);
                }
                // producer 0 copies the tile's bias into the stage of its last K step; the others
                // copy nothing into the spare block, so every producer's copy count stays NPP
                const bool bias_here = pw == 0 && i_ks == nst - 1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (__attribute__((address_space(3))) void *) (bias_here ? dst + ASTAGE + BSTAGE : sm + NS * STAGE),
                                                         16, bias_here && lane * 16 < BM * 4 ? (unsigned) (m_tile * BM * 4 + lane * 16) : kInvalid, 0, 0, 0);
                if (++i_ks == nst) {
                    i_ks = 0;
                    if (++i_it < ntw) set_issue_tile(i_it);
                }
            };
            set_issue_tile(0);
#pragma unroll
            for (int d = 0; d < NS - 1; ++d)
                if (d < S) issue(d);
            constexpr int kAhead = (NS - 2) * NPP;
            int buf = 0;
            for (int s = 0; s < S; ++s) {
                if (s + NS - 2 < S) __builtin_amdgcn_s_waitcnt((kAhead & 15) | (7 << 4) | (15 << 8) | ((kAhead >> 4) << 14));
                else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
                __asm__ volatile("s_barrier" ::: "memory");
                const int nb = buf == 0 ? NS - 1 : buf - 1; // (s + NS - 1) % NS
                if (s + NS - 1 < S) issue(nb);
                buf = buf + 1 == NS ? 0 : buf + 1;
            }
            return;
        }

        // ---------------- consumer
        const int wmi  = wave / WN;
        const int wni  = wave % WN;
        const int wm0  = wmi * 32 * FM;
        const int wn0  = wni * 32 * FN;
        const int lrow = lane & 31;
        const int lk   = lane >> 5;
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rrs =
            __builtin_amdgcn_make_buffer_rsrc((void *) (a.has_res ? a.res : a.y), (short) 0, a.has_res ? (int) a.y_bytes : 0, 0x00020000);

        float16v acc[FM][FN];
        u32x2    rv[FN][FM][4];
        // byte offset of output (j, i, qq) of this lane in y (and the residual), or kInvalid
        auto out_offset = [&](int t, int j, int i, int qq) __attribute__((always_inline)) {
            const int  px  = (t / a.m_tiles) * BN + wn0 + j * 32 + lrow;
            const int  pn  = px / a.OHWp;
            const int  pr  = px - pn * a.OHWp;
            const int  ocb = ((t % a.m_tiles) * BM + wm0 + i * 32 + qq * 8 + lk * 4) >> 2;
            return ((px < a.Pv) & (pr < a.OHW) & (ocb < a.Coutb)) ? (unsigned) (((pn * a.y_pstride + ocb) * a.OHW + pr) * 8) : kInvalid;
        };
        auto prefetch_residual = [&](int t) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) rv[j][i][qq] = a.has_res ? __builtin_amdgcn_raw_buffer_load_b64(rrs, out_offset(t, j, i, qq), 0, kStreamLoad)
                                                                            : u32x2 {0u, 0u};
        };
        auto store_tile = [&](int t, const unsigned char *bias_lds, auto act_c) __attribute__((always_inline)) {
            constexpr int ACT = decltype(act_c)::value;
            const int     mw0 = (t % a.m_tiles) * BM + wm0;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const float4v bv = *reinterpret_cast<const float4v *>(bias_lds + (wm0 + i * 32 + qq * 8 + lk * 4) * 4);
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const int oc = mw0 + i * 32 + qq * 8 + lk * 4;
                        float4v   v  = {acc[i][j][qq * 4 + 0], acc[i][j][qq * 4 + 1], acc[i][j][qq * 4 + 2], acc[i][j][qq * 4 + 3]};
                        v += bv;
                        const float4v r = h4_to_f4(__builtin_bit_cast(half4, rv[j][i][qq]));
                        if (a.has_res != 2) v += r;
                        v.x = apply_act(v.x, ACT, a.lo, a.hi);
                        v.y = apply_act(v.y, ACT, a.lo, a.hi);
                        v.z = apply_act(v.z, ACT, a.lo, a.hi);
                        v.w = apply_act(v.w, ACT, a.lo, a.hi);
                        if (a.has_res == 2) v += r;
                        if (oc + 0 >= a.Cout) v.x = 0.f;
                        if (oc + 1 >= a.Cout) v.y = 0.f;
                        if (oc + 2 >= a.Cout) v.z = 0.f;
                        if (oc + 3 >= a.Cout) v.w = 0.f;
                        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), yrs, out_offset(t, j, i, qq), 0, kStreamStore);
                    }
                }
        };
        auto epilogue = [&](int t, const unsigned char *bias_lds) __attribute__((always_inline)) {
            using std::integral_constant;
            switch (a.act) {
                case VKHIP_ACT_RELU: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_RELU> {}); break;
                case VKHIP_ACT_RELU6: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_RELU6> {}); break;
                case VKHIP_ACT_CLIP: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_CLIP> {}); break;
                case VKHIP_ACT_HARDSWISH: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
                case VKHIP_ACT_SILU: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_SILU> {}); break;
                case VKHIP_ACT_HARDSIGMOID: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_HARDSIGMOID> {}); break;
                default: store_tile(t, bias_lds, integral_constant<int, VKHIP_ACT_NONE> {}); break;
            }
        };

        const int g = lane >> 5;
        auto compute = [&](int buf) __attribute__((always_inline)) {
            const unsigned char *Ab = sm + buf * STAGE + ((wmi * FM) * 64 + lane) * 16;
            const unsigned char *Bb = sm + buf * STAGE + ASTAGE + (2 * g * BN + wn0 + (lane & 31)) * PS;
            half8 fa[2][FM], fb[2][FN];
            auto rd = [&](int kk, int d) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const u32x2 lo = *reinterpret_cast<const u32x2 *>(Bb + (kk * 4 * BN + 32 * j) * PS);
                    const u32x2 hi = *reinterpret_cast<const u32x2 *>(Bb + ((kk * 4 + 1) * BN + 32 * j) * PS);
                    fb[d][j] = __builtin_bit_cast(half8, u32x4_make(lo.x, lo.y, hi.x, hi.y));
                }
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[d][i] = *reinterpret_cast<const half8 *>(Ab + (kk * MF + i) * 1024);
            };
            rd(0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                if (kk < 3) rd(kk + 1, (kk + 1) & 1);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk & 1][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
                if (kk < 3) StepSchedule<0, FM * FN, FM + 2 * FN, 4 * FN>::apply();
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        int buf = 0;
        for (int it = 0; it < ntw; ++it) {
            const int t = tile_of(it);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
            int last = buf;
            for (int ks = 0; ks < nst; ++ks) {
                __asm__ volatile("s_barrier" ::: "memory");
                if (ks == 0) prefetch_residual(t);
                compute(buf);
                last = buf;
                buf  = buf + 1 == NS ? 0 : buf + 1;
            }
            // the bias slice rides in the tile's last stage, which no copy overwrites before the
            // next barrier
            epilogue(t, sm + last * STAGE + ASTAGE + BSTAGE);
        }
    }

    // ------------------------------------------------------------------ 3x3 halo-tile GEMM kernel
    // Direct 3x3 pad-1 convolution, stride 1 or 2 (Cin a multiple of 16*KK, even input width W),
    // that reads each input pixel once per workgroup instead of once per tap: the workgroup's BN
    // consecutive output pixels (row-major over n, oy, ox, free to cross image boundaries) need a
    // band of input rows (rows S*oy - 1 .. S*oy + 1 of each output row oy);
    // per channel slot the band is copied global->LDS by buffer-load-to-LDS, 16 bytes (a pixel pair)
    // per lane, into rows of W + 2 pixels (W + 3 for odd W): W data pixels then zero pixels, so the left
    // neighbour of column 0 is the previous row's last zero pixel (for the first band row: the
    // previous slot's zero tail, or a zero guard before slot 0) and the right neighbour of
    // column W-1 is the first one. Each image contributes H + 2 band rows (its zero rows above and
    // below), so the band row of (n, iy) is (n - n_first)(H + 2) + iy + 1 - S*oy_first. Rows outside
    // the image, pad pairs and lanes past the band get an out-of-range offset and write zeros.
    // The 9 taps of a 16-channel K step then read their B fragments from the same band at a
    // shift of (ky - 1)(W + 2) + (kx - 1) pixels. A (weights) arrives by LDS DMA too, prepacked as
    // [m_tile][stage][tap][kk][m_frag][lane][8 halves].
    //   FM x FN fragments per wave, WM x WN waves; KK 16-channel K steps per LDS stage; NS stages
    //   in the ring; NBI 1 KB DMA chunks per channel slot of the band (rows * (W + 2) / 2 lanes).
    //   ODD: odd input width. Band rows are then W + 3 pixels (pairs stay 16-byte aligned) and the
    //   pair that holds pixel W-1 also copies the next image row's first pixel into column W, the
    //   right pad; the B fragments of the right-hand taps are zeroed in registers for the output
    //   columns whose right neighbour is that pad.
    // LDS bytes of a halo workgroup: NS ring stages plus the spare 1 KB that surplus A copies fill
    template <int FM, int WM, int WN, int KK, int NS, int NBI>
    __host__ __device__ constexpr int halo_lds_bytes() {
        return NS * (9 * KK * FM * WM * 1024 + 32 + 4 * KK * NBI * 1024) + ((9 * KK * FM * WM) % (WM * WN) ? 1024 : 0);
    }

    // The halo kernel's main loop (everything before its epilogue): the workgroup (m_tile, n0)
    // accumulates its BM x BN tile over K stages ks_begin .. ks_end of split `split` into acc,
    // with the ring in `sm` (halo_lds_bytes).
    template <int FM, int FN, int WM, int WN, int KK, int NS, int NBI, bool ODD>
    __device__ __forceinline__ void halo_mainloop(const GemmArgs &a, unsigned char *sm, float16v (&acc)[FM][FN], int tid, int lane, int wave,
                                                  int m_tile, int n0, int split) {
        constexpr int NW     = WM * WN;
        constexpr int BM     = 32 * FM * WM;
        constexpr int BN     = 32 * FN * WN;
        constexpr int MF     = BM / 32;
        constexpr int SLOTS  = 4 * KK;                 // channel slots per stage
        constexpr int SS     = NBI * 1024;             // LDS bytes per slot of the band
        constexpr int ASTAGE = 9 * KK * MF * 1024;     // A bytes per stage
        constexpr int BOFF   = ASTAGE + 32;            // band start (32 zero guard bytes before it)
        constexpr int STAGE  = BOFF + SLOTS * SS;
        constexpr int NA     = ASTAGE / 1024;          // 1 KB A chunks per stage
        constexpr int NB     = SLOTS * NBI;            // 1 KB band chunks per stage
        // every wave issues the same number of copies per stage (the vmcnt waits count them): A
        // chunks are rounded up to a multiple of the wave count, the surplus ones copy zeros into
        // a spare 1 KB after the ring
        constexpr int NAW = (NA + NW - 1) / NW;
        constexpr int SPARE = NA % NW ? 1024 : 0;
        static_assert(NS * STAGE + SPARE <= 160 * 1024, "LDS budget");
        static_assert(NS * STAGE + SPARE == halo_lds_bytes<FM, WM, WN, KK, NS, NBI>(), "LDS size");
        static_assert(NB % NW == 0, "band copies per wave");
        const int wmi = wave / WN;
        const int wni = wave % WN;
        const int wn0 = wni * 32 * FN;

        const int W   = a.W, H = a.H, HW = a.HW, OW = a.OW, OHW = a.OHW, S = a.SH;
        const int RS  = (W + 3) & ~1; // band row stride in pixels: W data + 1 or 2 zero pads (even)
        const int PW  = RS >> 1;      // pixel pairs per band row
        const int nf  = n0 / OHW;
        const int iyf = S * ((n0 - nf * OHW) / OW); // input row of the first pixel's centre tap
        const int NI  = a.P / OHW;
        // band rows of this workgroup: up to the row below its last pixel's centre row; lanes past
        // them copy zeros, so the last 8 bytes of every slot are zero (the left neighbour of the
        // next slot's first pixel)
        const int pl    = min(a.P, n0 + BN) - 1;
        const int nl    = pl / OHW;
        const int nrows = (nl - nf) * (H + 2) + S * ((pl - nl * OHW) / OW) + 1 - iyf + 2;

        const unsigned char *Wt = reinterpret_cast<const unsigned char *>(a.w) + (long long) m_tile * a.nsteps * ASTAGE;
        const int ks_begin = split * a.steps_per_split;
        const int ks_end   = min(a.nsteps, ks_begin + a.steps_per_split);
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *) Wt, (short) 0, ks_end * ASTAGE, 0x00020000);
        constexpr unsigned kInvalid = 0x80000000u;

        // zero guards in front of every stage's band (never written by the copies)
        if (tid < NS * 2) *reinterpret_cast<u32x4 *>(&sm[(tid >> 1) * STAGE + ASTAGE + (tid & 1) * 16]) = u32x4 {0u, 0u, 0u, 0u};

        // Band copy chunks: chunk c = r*NW + wave of the stage covers slot c / NBI, lanes
        // (c % NBI)*64 + lane of that slot's band; the per-lane source offsets repeat for every slot.
        constexpr int NBW = NB / NW; // band chunks per wave per stage
        unsigned bsrc[NBI];
#pragma unroll
        for (int i = 0; i < NBI; ++i) {
            const int k    = i * 64 + lane;
            const int vrow = k / PW;
            const int pc   = k - vrow * PW;
            const int vabs = vrow + iyf;
            const int n    = nf + vabs / (H + 2);
            const int iy   = vabs % (H + 2) - 1;
            const bool ok  = 2 * pc < W && iy >= 0 && iy < H && n < NI && vrow < nrows;
            bsrc[i]        = ok ? (unsigned) (((n * a.x_pstride) * HW + iy * W + 2 * pc) * 8) : kInvalid;
        }
        const unsigned hw8 = (unsigned) HW * 8u;
        auto issue = [&](int ks, int buf) __attribute__((always_inline)) {
            unsigned char *dst = sm + buf * STAGE;
#pragma unroll
            for (int r = 0; r < NAW; ++r) {
                const int  c    = r * NW + wave;
                const bool real = NA % NW == 0 || c < NA;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *) (real ? dst + c * 1024 : sm + NS * STAGE), 16,
                                                         real ? (unsigned) (c * 1024 + lane * 16) + (unsigned) (ks * ASTAGE) : kInvalid, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < NBW; ++r) {
                const int c  = r * NW + wave;
                const int sl = c / NBI;
                const unsigned vo = bsrc[c % NBI]; // (a local: the host pass rejects the array element as a builtin operand)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (dst + BOFF + sl * SS + (c % NBI) * 1024),
                                                         16, vo, (unsigned) (ks * SLOTS + sl) * hw8, 0, 0);
            }
        };

        // B fragment pixel of each fragment column: LDS pixel index of the centre tap.
        const int g = lane >> 5;
        int       qb[FN];
        bool      redge[FN] = {}; // right neighbour is column W (not zero when W is odd)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int p = n0 + wn0 + 32 * j + (lane & 31);
            int       q = W + 3; // any interior position: columns past P read the band harmlessly
            if (p < a.P) {
                const int n  = p / OHW;
                const int r  = p - n * OHW;
                const int oy = r / OW;
                q            = ((n - nf) * (H + 2) + S * oy + 1 - iyf) * RS + S * (r - oy * OW);
                if constexpr (ODD) redge[j] = S * (r - oy * OW) + 1 == W;
            }
            qb[j] = BOFF + (2 * g) * SS + q * 8;
        }
        int tapoff[9];
#pragma unroll
        for (int t = 0; t < 9; ++t) tapoff[t] = ((t / 3 - 1) * RS + (t % 3 - 1)) * 8;

#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        auto compute = [&](int buf, int next_ks, int next_buf) __attribute__((always_inline)) {
            const unsigned char *S  = sm + buf * STAGE;
            const unsigned char *Ab = S + ((wmi * FM) * 64 + lane) * 16;
            half8 fa[2][FM], fb[2][FN];
            // step s = kk * 9 + tap
            auto rd = [&](int s, int d) __attribute__((always_inline)) {
                const int kk = s / 9, t = s % 9;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const unsigned char *bp = S + qb[j] + tapoff[t] + kk * 4 * SS;
                    u32x2 lo = *reinterpret_cast<const u32x2 *>(bp);
                    u32x2 hi = *reinterpret_cast<const u32x2 *>(bp + SS);
                    if constexpr (ODD) {
                        if (t % 3 == 2) {
                            lo = redge[j] ? u32x2 {0u, 0u} : lo;
                            hi = redge[j] ? u32x2 {0u, 0u} : hi;
                        }
                    }
                    fb[d][j] = __builtin_bit_cast(half8, u32x4_make(lo.x, lo.y, hi.x, hi.y));
                }
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[d][i] = *reinterpret_cast<const half8 *>(Ab + ((t * KK + kk) * MF + i) * 1024);
            };
            rd(0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 9 * KK; ++s) {
                if (s == 0 && next_ks >= 0) issue(next_ks, next_buf);
                if (s + 1 < 9 * KK) rd(s + 1, (s + 1) & 1);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
                if (s == 0) StepSchedule<0, FM * FN, FM + 2 * FN, 4 * FN, NAW + NBW>::apply();
                else if (s + 1 < 9 * KK) StepSchedule<0, FM * FN, FM + 2 * FN, 4 * FN>::apply();
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        constexpr int NPW    = NAW + NBW; // copies per wave per stage
        constexpr int kAhead = NS < 2 ? 0 : ((NS - 2) * NPW < 63 ? (NS - 2) * NPW : 63);
        constexpr int kWait  = (kAhead & 15) | (7 << 4) | (15 << 8) | ((kAhead >> 4) << 14);
        __syncthreads(); // guards written
        if constexpr (NS == 1) {
            // one LDS stage: copy, wait, compute (the workgroups sharing a CU overlap each other)
            for (int ks = ks_begin; ks < ks_end; ++ks) {
                if (ks > ks_begin) __asm__ volatile("s_barrier" ::: "memory");
                issue(ks, 0);
                __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
                __asm__ volatile("s_barrier" ::: "memory");
                compute(0, -1, 0);
            }
        } else if (ks_begin < ks_end) {
#pragma unroll
            for (int d = 0; d < NS - 1; ++d)
                if (ks_begin + d < ks_end) issue(ks_begin + d, d);
            for (int ks = ks_begin; ks < ks_end; ++ks) {
                const int rel = ks - ks_begin;
                if (ks + NS - 2 < ks_end) __builtin_amdgcn_s_waitcnt(kWait);
                else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
                __asm__ volatile("s_barrier" ::: "memory");
                compute(rel % NS, ks + NS - 1 < ks_end ? ks + NS - 1 : -1, (rel + NS - 1) % NS);
            }
        }
    }

    template <int FM, int FN, int WM, int WN, int KK, int NS, int NBI, bool ODD = false>
    __global__ __launch_bounds__(64 * WM * WN, 1) void conv_halo_kernel(GemmArgs a) {
        constexpr int BM = 32 * FM * WM;
        constexpr int BN = 32 * FN * WN;
        __shared__ __attribute__((aligned(16))) unsigned char sm[halo_lds_bytes<FM, WM, WN, KK, NS, NBI>()];
        const int tid    = threadIdx.x;
        const int lane   = tid & 63;
        const int wave   = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int lin    = xcd_remap(blockIdx.x, gridDim.x);
        const int m_tile = lin % a.m_tiles;
        const int n0     = (lin / a.m_tiles) * BN;
        const int split  = blockIdx.y;
        float16v  acc[FM][FN];
        halo_mainloop<FM, FN, WM, WN, KK, NS, NBI, ODD>(a, sm, acc, tid, lane, wave, m_tile, n0, split);
        gemm_epilogue<FM, FN>(a, acc, m_tile * BM + (wave / WN) * 32 * FM, n0 + (wave % WN) * 32 * FN, split, 0, lane,
                              reinterpret_cast<volatile int *>(sm));
    }

    // ------------------------------------------------------------------ fused 3x3 -> 1x1 kernel
    // A 3x3 conv (the halo main loop above, with the workgroup's M tile covering all BM = Cmid of
    // its output channels: one wave row, WM = 1) followed by a 1x1 conv over those Cmid channels
    // (a bottleneck's 3x3 then its 1x1 expansion), without the Cmid-channel intermediate leaving
    // the registers. After the 3x3 main loop each wave holds all Cmid channels of its 32*FN pixels
    // as fp32 MFMA results: acc[i][j][8h + t] is channel i*32 + (2h + t/4)*8 + 4g + t%4 (g = lane /
    // 32) of pixel column j. Bias, activation and the fp16 rounding the separate conv's store
    // applies turn them in place into the B operand of the 1x1: the 8 values of (i, h) are exactly
    // one 16-deep K step of lane group g, so the 1x1 weights are prepacked with their K order
    // permuted to match ([32-row fragment][step s = 2i + h][lane][8 halves], lane = g*32 + row%32,
    // entry t = channel i*32 + (2h + t/4)*8 + 4g + t%4). The 1x1 then runs in chunks of 32*MC
    // output channels: the chunk's weight fragments are loaded straight from global memory (they
    // stay in L2; every wave reads the same ones) one chunk ahead, so they are in flight before the
    // previous chunk's epilogue stores, and each chunk ends in the shared epilogue (bias, residual,
    // activation, fp16 store) with the 1x1's arguments.
    struct PwArgs {
        const half_t *w;       // prepacked 1x1 weights, nchunks * MC fragments of 2*FM KB
        int           nchunks; // ceil(Cout / (32 * MC))
        GemmArgs      e;       // the 1x1's epilogue: bias, res, y, Cout / Coutb, P, OHW, act, ...
        // An optional second 1x1 (MR > 0) over the first one's output (the next bottleneck's
        // reduction), accumulated chunk by chunk: w3 [MR fragments][2 * nchunks steps][64][8 halves]
        // (K order permuted like w, chunk c being fragment c), its bias [32 * MR], output y3.
        const half_t *w3;
        const float  *bias3;
        uint2        *y3;
        int           Cout3, Coutb3, act3;
        float         lo3, hi3;
        unsigned      y3_bytes;
    };

    template <int FM, int FN, int WN, int KK, int NS, int NBI, bool ODD, int MC, int MR = 0>
    __global__ __launch_bounds__(64 * WN, 2) void conv_halo_pw_kernel(GemmArgs a, PwArgs p) {
        static_assert(MR == 0 || MC == 1, "the chained 1x1 takes 32-row chunks");
        constexpr int BN = 32 * FN * WN;
        constexpr int KS = 2 * FM; // 16-deep K steps of the 1x1
        __shared__ __attribute__((aligned(16))) unsigned char sm[halo_lds_bytes<FM, 1, WN, KK, NS, NBI>()];
        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int n0   = xcd_remap(blockIdx.x, gridDim.x) * BN; // m_tiles == 1
        const int wn0  = wave * 32 * FN;
        float16v  acc[FM][FN];
        halo_mainloop<FM, FN, 1, WN, KK, NS, NBI, ODD>(a, sm, acc, tid, lane, wave, 0, n0, 0);

        // the 3x3's epilogue without its store: bias, activation, fp16 -> the 1x1's B fragments
        const int g = lane >> 5;
        half8     bm[FM][2][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float4v b0 = *reinterpret_cast<const float4v *>(a.bias + i * 32 + (2 * h) * 8 + g * 4);
                const float4v b1 = *reinterpret_cast<const float4v *>(a.bias + i * 32 + (2 * h + 1) * 8 + g * 4);
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    float4v lo = {acc[i][j][8 * h + 0], acc[i][j][8 * h + 1], acc[i][j][8 * h + 2], acc[i][j][8 * h + 3]};
                    float4v hi = {acc[i][j][8 * h + 4], acc[i][j][8 * h + 5], acc[i][j][8 * h + 6], acc[i][j][8 * h + 7]};
                    lo += b0;
                    hi += b1;
                    if (a.act == VKHIP_ACT_RELU) { // the bottleneck case, without the activation switch
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            lo[e] = fmaxf(lo[e], 0.f);
                            hi[e] = fmaxf(hi[e], 0.f);
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            lo[e] = apply_act(lo[e], a.act, a.lo, a.hi);
                            hi[e] = apply_act(hi[e], a.act, a.lo, a.hi);
                        }
                    }
                    const half4 l4 = f4_to_h4(lo), h4 = f4_to_h4(hi);
                    bm[i][h][j] = half8 {l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
                }
            }

        // The 1x1 in chunks of 32*MC output channels, software-pipelined one chunk deep: the next
        // chunk's weight fragments and residual values are loaded before this chunk's MFMAs and
        // stores (the vector memory counter retires in order, so they never wait behind the stores).
        const GemmArgs &e = p.e;
        constexpr unsigned kInvalid = 0x80000000u;
        // The 1x1 weights and bias (and the chained 1x1's) are staged in the idle ring once per
        // workgroup, 1 KB copy units dealt round-robin to the waves, while the mid epilogue runs;
        // every wave then reads its fragments from LDS. Layout: W2 [chunk][step][lane] x 16 bytes,
        // bias [nchunks * 32 * MC] fp32, W3 [fragment][step][lane] x 16 bytes, bias3 [32 * MR] fp32.
        const int NW2 = p.nchunks * MC * KS;              // KB of W2
        const int NB  = (p.nchunks * MC * 32 * 4 + 1023) / 1024;
        const int NW3 = MR > 0 ? MR * 2 * p.nchunks : 0;
        const int NB3 = MR > 0 ? 1 : 0;
        const int OB = NW2 * 1024, OW3 = OB + NB * 1024, OB3 = OW3 + NW3 * 1024;
        {
            __syncthreads(); // every wave is done with the ring
            const __amdgpu_buffer_rsrc_t r2 = __builtin_amdgcn_make_buffer_rsrc((void *) p.w, (short) 0, NW2 * 1024, 0x00020000);
            const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void *) e.bias, (short) 0, p.nchunks * MC * 32 * 4, 0x00020000);
            const __amdgpu_buffer_rsrc_t r3 = __builtin_amdgcn_make_buffer_rsrc((void *) (MR > 0 ? p.w3 : p.w), (short) 0, NW3 * 1024, 0x00020000);
            const __amdgpu_buffer_rsrc_t rb3 = __builtin_amdgcn_make_buffer_rsrc((void *) (MR > 0 ? p.bias3 : e.bias), (short) 0, MR * 32 * 4, 0x00020000);
            const int units = NW2 + NB + NW3 + NB3;
            for (int u = wave; u < units; u += WN) {
                __amdgpu_buffer_rsrc_t rs = r2;
                int                    k  = u;
                if (u >= NW2 + NB + NW3) rs = rb3, k = u - NW2 - NB - NW3;
                else if (u >= NW2 + NB) rs = r3, k = u - NW2 - NB;
                else if (u >= NW2) rs = rb, k = u - NW2;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *) (sm + u * 1024), 16, (unsigned) (k * 1024 + lane * 16), 0, 0, 0);
            }
        }
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) e.y, (short) 0, (int) e.y_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc((void *) (e.has_res ? e.res : e.y), (short) 0, (int) e.y_bytes, 0x00020000);
        // per fragment column: the output pixel's byte offset at channel block 0 (or invalid)
        unsigned pbase[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int px = n0 + wn0 + 32 * j + (lane & 31);
            const int pn = px / e.OHW, pr = px - pn * e.OHW;
            pbase[j]     = px < e.P ? (unsigned) ((pn * e.y_pstride * e.OHW + pr) * 8) : kInvalid;
        }
        // output offset of (chunk c, fragment mi, column j, row group qq): block ocb = 8(c*MC + mi) + 2qq + g
        auto yoff = [&](int c, int mi, int j, int qq) __attribute__((always_inline)) {
            const int ocb = 8 * (c * MC + mi) + 2 * qq + g;
            return pbase[j] != kInvalid && ocb < e.Coutb ? pbase[j] + (unsigned) (ocb * e.OHW * 8) : kInvalid;
        };
        u32x2 rn[MC][FN][4];
        auto  load = [&](int c) __attribute__((always_inline)) { // the residual of chunk c
            if (e.has_res) {
#pragma unroll
                for (int mi = 0; mi < MC; ++mi)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) rn[mi][j][qq] = __builtin_amdgcn_raw_buffer_load_b64(rrs, yoff(c, mi, j, qq), 0, kStreamLoad);
            }
        };
        load(0);
        constexpr int MRX = MR > 0 ? MR : 1;
        float16v      acc3[MRX][FN];
        if constexpr (MR > 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc3[m][j][r] = 0.f;
        }
        // the staged weights have landed (the residual loads issued after them may stay in flight)
        if (e.has_res) __builtin_amdgcn_s_waitcnt((MC * FN * 4) | (7 << 4) | (15 << 8));
        else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __syncthreads();
        for (int c = 0; c < p.nchunks; ++c) {
            u32x2 rc[MC][FN][4];
#pragma unroll
            for (int mi = 0; mi < MC; ++mi)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) rc[mi][j][qq] = rn[mi][j][qq];
            if (c + 1 < p.nchunks) load(c + 1);
            float16v acc2[MC][FN];
#pragma unroll
            for (int mi = 0; mi < MC; ++mi)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc2[mi][j][r] = 0.f;
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int mi = 0; mi < MC; ++mi) {
                    const half8 af = *reinterpret_cast<const half8 *>(sm + (((c * MC + mi) * KS + s) * 64 + lane) * 16);
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc2[mi][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bm[s / 2][s % 2][j], acc2[mi][j], 0, 0, 0);
                }
            // epilogue: bias, residual, activation (compile-time), zero past Cout, fp16 store
            half4 o16[4][FN]; // the stored fp16 values: the chained 1x1's B operand
            auto epi = [&](auto act_c) __attribute__((always_inline)) {
                constexpr int ACT = decltype(act_c)::value;
#pragma unroll
                for (int mi = 0; mi < MC; ++mi)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int     oc = 32 * (c * MC + mi) + 8 * qq + 4 * g;
                        const float4v bv = *reinterpret_cast<const float4v *>(sm + OB + oc * 4);
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
                            float4v v = {acc2[mi][j][qq * 4 + 0], acc2[mi][j][qq * 4 + 1], acc2[mi][j][qq * 4 + 2], acc2[mi][j][qq * 4 + 3]};
                            v += bv;
                            if (e.has_res) v += h4_to_f4(__builtin_bit_cast(half4, rc[mi][j][qq]));
#pragma unroll
                            for (int t = 0; t < 4; ++t) v[t] = oc + t < e.Cout ? apply_act(v[t], ACT, e.lo, e.hi) : 0.f;
                            const half4 o = f4_to_h4(v);
                            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o), yrs, yoff(c, mi, j, qq), 0, kStreamStore);
                            if constexpr (MR > 0) o16[qq][j] = o;
                        }
                    }
            };
            switch (e.act) {
                case VKHIP_ACT_RELU: epi(std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
                case VKHIP_ACT_RELU6: epi(std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
                case VKHIP_ACT_CLIP: epi(std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
                case VKHIP_ACT_HARDSWISH: epi(std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
                case VKHIP_ACT_SILU: epi(std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
                default: epi(std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
            }
            // the chained 1x1: this chunk's 32 output channels are its K steps 2c, 2c + 1 (the
            // stored values of row groups 2h, 2h + 1 form the B fragment of step 2c + h)
            if constexpr (MR > 0) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const half4 lo = o16[2 * h][j], hi = o16[2 * h + 1][j];
                        const half8 b8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                        for (int m = 0; m < MR; ++m) {
                            const half8 wf = *reinterpret_cast<const half8 *>(sm + OW3 + ((m * 2 * p.nchunks + 2 * c + h) * 64 + lane) * 16);
                            acc3[m][j]     = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, b8, acc3[m][j], 0, 0, 0);
                        }
                    }
            }
        }
        if constexpr (MR > 0) {
            // the chained 1x1's epilogue: bias, activation, fp16 store into y3
            const __amdgpu_buffer_rsrc_t y3rs = __builtin_amdgcn_make_buffer_rsrc((void *) p.y3, (short) 0, (int) p.y3_bytes, 0x00020000);
            auto epi3 = [&](auto act_c) __attribute__((always_inline)) {
                constexpr int ACT = decltype(act_c)::value;
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int     oc = 32 * m + 8 * qq + 4 * g;
                        const float4v bv = *reinterpret_cast<const float4v *>(sm + OB3 + oc * 4);
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
                            float4v v = {acc3[m][j][qq * 4 + 0], acc3[m][j][qq * 4 + 1], acc3[m][j][qq * 4 + 2], acc3[m][j][qq * 4 + 3]};
                            v += bv;
#pragma unroll
                            for (int t = 0; t < 4; ++t) v[t] = oc + t < p.Cout3 ? apply_act(v[t], ACT, p.lo3, p.hi3) : 0.f;
                            const int      px  = n0 + wn0 + 32 * j + (lane & 31);
                            const int      pn  = px / e.OHW, pr = px - pn * e.OHW;
                            const int      ocb = oc >> 2;
                            const unsigned off = px < e.P && ocb < p.Coutb3 ? (unsigned) (((pn * p.Coutb3 + ocb) * e.OHW + pr) * 8) : kInvalid;
                            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f4_to_h4(v)), y3rs, off, 0, kStreamStore);
                        }
                    }
            };
            switch (p.act3) {
                case VKHIP_ACT_RELU: epi3(std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
                case VKHIP_ACT_RELU6: epi3(std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
                case VKHIP_ACT_CLIP: epi3(std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
                case VKHIP_ACT_HARDSWISH: epi3(std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
                case VKHIP_ACT_SILU: epi3(std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
                default: epi3(std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
            }
        }
    }

    // ------------------------------------------------------------------ stem kernel (Cin <= 4)
    // KxK convolution (K = 3 or 7, stride 1 or 2, pad K/2) over at most 4 input channels, i.e. the
    // first layer of a CNN on an RGB image. The whole reduction is KxK taps x 4 channels, so one
    // 16-deep MFMA K step holds 4 taps (lanes 0-31 taps 4s and 4s+1, lanes 32-63 taps 4s+2 and
    // 4s+3, 4 channels each; taps past K*K have zero weights) and all KT = ceil(K*K/4) steps fit
    // one LDS stage: the workgroup copies its input band (one channel slot) and the prepacked
    // weights [m_tile][step][m_frag][lane][8 halves] once, waits, and runs every step from LDS.
    // Band layout as in the halo kernel with rows of W + K - 1 pixels (W data, K - 1 zeros that
    // serve as the right pad of this row and the left pad of the next) and H + K - 1 band rows per
    // image (K/2 zero rows above and below).
    template <int K, int FM, int FN, int WM, int WN, int NBI>
    __global__ __launch_bounds__(64 * WM * WN) void conv_stem_kernel(GemmArgs a) {
        constexpr int NW     = WM * WN;
        constexpr int BM     = 32 * FM * WM;
        constexpr int BN     = 32 * FN * WN;
        constexpr int MF     = BM / 32;
        constexpr int KT     = (K * K + 3) / 4; // 16-deep K steps
        constexpr int KH2    = K / 2;
        constexpr int NA     = KT * MF;         // 1 KB A chunks
        constexpr int BOFF   = NA * 1024 + 32;  // band start (32 zero guard bytes before it)
        constexpr int NC     = NA + NBI;        // chunks per workgroup
        constexpr int NCW    = (NC + NW - 1) / NW;
        constexpr int SPARE  = BOFF + NBI * 1024;
        static_assert(SPARE + 1024 <= 160 * 1024, "LDS budget");
        __shared__ __attribute__((aligned(16))) unsigned char sm[SPARE + 1024];

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wmi  = wave / WN;
        const int wni  = wave % WN;
        const int lin    = xcd_remap(blockIdx.x, gridDim.x);
        const int m_tile = lin % a.m_tiles;
        const int n0     = (lin / a.m_tiles) * BN;
        const int m0     = m_tile * BM;
        const int wm0    = wmi * 32 * FM;
        const int wn0    = wni * 32 * FN;

        const int W = a.W, H = a.H, OW = a.OW, OHW = a.OHW, S = a.SH;
        const int RS  = W + K - 1;  // band row stride in pixels (even: W even, K odd)
        const int VR  = H + K - 1;  // band rows per image
        const int nf  = n0 / OHW;
        const int iyf = S * ((n0 - nf * OHW) / OW);
        const int NI  = a.P / OHW;
        const int pl  = min(a.P, n0 + BN) - 1;
        const int nl  = pl / OHW;
        const int nrows = (nl - nf) * VR + S * ((pl - nl * OHW) / OW) + 2 * KH2 + 1 - iyf;

        const unsigned char *Wt = reinterpret_cast<const unsigned char *>(a.w) + (long long) m_tile * NA * 1024;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *) Wt, (short) 0, NA * 1024, 0x00020000);
        constexpr unsigned kInvalid = 0x80000000u;
        if (tid < 2) *reinterpret_cast<u32x4 *>(&sm[NA * 1024 + tid * 16]) = u32x4 {0u, 0u, 0u, 0u};

        // copies: chunk c = r*NW + wave; chunks < NA are weights, then NBI band chunks, the rest
        // (every wave issues the same count) copy zeros into the spare KB
#pragma unroll
        for (int r = 0; r < NCW; ++r) {
            const int c = r * NW + wave;
            if (c < NA) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *) (sm + c * 1024), 16,
                                                         (unsigned) (c * 1024 + lane * 16), 0, 0, 0);
            } else {
                const int  k    = (c - NA) * 64 + lane;
                const int  vrow = k / (RS >> 1);
                const int  pc   = k - vrow * (RS >> 1);
                const int  vabs = vrow + iyf;
                const int  n    = nf + vabs / VR;
                const int  iy   = vabs % VR - KH2;
                const bool ok   = c < NC && 2 * pc < W && iy >= 0 && iy < H && n < NI && vrow < nrows;
                const unsigned vo = ok ? (unsigned) ((n * a.HW + iy * W + 2 * pc) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (c < NC ? sm + BOFF + (c - NA) * 1024 : sm + SPARE),
                                                         16, vo, 0, 0, 0);
            }
        }

        // per lane: centre pixel of each fragment column, and the two tap offsets of every step
        const int g = lane >> 5;
        int       qb[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int p = n0 + wn0 + 32 * j + (lane & 31);
            int       q = KH2 * RS + KH2; // any interior position for columns past P
            if (p < a.P) {
                const int n  = p / OHW;
                const int rr = p - n * OHW;
                const int oy = rr / OW;
                q            = ((n - nf) * VR + S * oy + KH2 - iyf) * RS + S * (rr - oy * OW);
            }
            qb[j] = BOFF + q * 8;
        }
        int toff[KT][2];
#pragma unroll
        for (int s = 0; s < KT; ++s)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int t = 4 * s + 2 * g + h;
                toff[s][h]  = t < K * K ? ((t / K - KH2) * RS + (t % K - KH2)) * 8 : 0;
            }

        float16v acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __syncthreads();
        const unsigned char *Ab = sm + ((wmi * FM) * 64 + lane) * 16;
        half8 fa[2][FM], fb[2][FN];
        auto rd = [&](int s, int d) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const u32x2 lo = *reinterpret_cast<const u32x2 *>(sm + qb[j] + toff[s][0]);
                const u32x2 hi = *reinterpret_cast<const u32x2 *>(sm + qb[j] + toff[s][1]);
                fb[d][j] = __builtin_bit_cast(half8, u32x4_make(lo.x, lo.y, hi.x, hi.y));
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[d][i] = *reinterpret_cast<const half8 *>(Ab + (s * MF + i) * 1024);
        };
        rd(0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KT; ++s) {
            if (s + 1 < KT) rd(s + 1, (s + 1) & 1);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
            if (s + 1 < KT) StepSchedule<0, FM * FN, FM + 2 * FN, 4 * FN>::apply();
            __builtin_amdgcn_sched_barrier(0);
        }
        gemm_epilogue<FM, FN>(a, acc, m0 + wm0, n0 + wn0, 0, 0, lane);
    }

    // ------------------------------------------------------------------ host side: tiles & plans
    // kind 0: conv_gemm_kernel (A and B staged through LDS), WM x WN waves over a BM x BN tile.
    // kind 1: conv_bd_kernel (A via LDS DMA, B straight into registers), waves of (32FM) x (32FN).
    // kind 2: conv_dma_kernel (A and B via LDS DMA; dense B only: 1x1 s1 with an even pixel count
    //         per image, Winograd GEMMs with an even tile count), 2x2 waves of (32FM) x (32FN).
    // kind 3: conv_halo_kernel (3x3 pad-1, stride 1 or 2: input band staged once in LDS for all 9
    //         taps), KK 16-channel K steps per LDS stage.
    // kind 4: conv_stem_kernel (3x3 or 7x7, stride 1 or 2, pad K/2, at most 4 input channels).
    // kind 5: conv_thin_kernel (3x3 pad 1 or 1x1, stride 1 or 2, at most 32 input channels and BM
    //         output channels, FM = BM / 16 fragments; weights in registers).
    // PERS (kind 2 only): the persistent variant (conv_dma_persist_kernel), gridDim = resident
    // workgroups, each walking a strided list of tiles.
    // LE (kind 2 only): the LDS-staged epilogue (gemm_epilogue_lds).
    struct TileCfg {
        int BM, BN, WM, WN, kind, FM, FN, KK, PERS, LE;
    };
    static const TileCfg kTiles[] = {
        {128, 128, 2, 2, 0, 0, 0}, // 0
        {64, 128, 2, 2, 0, 0, 0},  // 1
        {128, 64, 2, 2, 0, 0, 0},  // 2
        {64, 64, 2, 2, 0, 0, 0},   // 3
        {256, 128, 2, 2, 0, 0, 0}, // 4
        {128, 256, 2, 2, 0, 0, 0}, // 5
        {32, 128, 1, 4, 0, 0, 0},  // 6
        {64, 256, 1, 4, 0, 0, 0},  // 7
        {128, 256, 1, 4, 1, 4, 2}, // 8
        {128, 128, 2, 2, 1, 2, 2}, // 9
        {64, 256, 1, 4, 1, 2, 2},  // 10
        {256, 256, 2, 2, 2, 4, 4}, // 11
        {256, 256, 2, 4, 2, 4, 2}, // 12 (8 waves)
        {256, 256, 4, 2, 2, 2, 4}, // 13 (8 waves)
        {128, 128, 2, 2, 2, 2, 2}, // 14
        {256, 128, 4, 2, 2, 2, 2}, // 15 (8 waves)
        {128, 128, 2, 2, 2, 2, 2},    // 16 (4-stage LDS ring)
        {128, 128, 2, 2, 3, 2, 2, 1}, // 17 (3-stage ring)
        {64, 256, 1, 4, 3, 2, 2, 1},  // 18 (2-stage ring, two workgroups per CU)
        {128, 256, 2, 2, 3, 2, 4, 1}, // 19 (2-stage ring)
        {64, 128, 1, 4, 3, 2, 1, 1},  // 20 (one stage, several workgroups per CU)
        {64, 256, 1, 4, 4, 2, 2},     // 21 stem
        {64, 128, 1, 4, 4, 2, 1},     // 22 stem
        {32, 256, 1, 4, 4, 1, 2},     // 23 stem (few output channels)
        {64, 128, 2, 2, 2, 1, 2},     // 24
        {64, 256, 1, 4, 2, 2, 2},     // 25
        {64, 128, 1, 4, 3, 2, 1, 1},  // 26 halo (2-stage ring, two workgroups per CU for small bands)
        {64, 256, 1, 4, 3, 2, 2, 1},  // 27 halo (one stage: workgroups overlap each other instead of a ring)
        {64, 128, 2, 2, 2, 1, 2},     // 28 tile 24 with a 3-stage ring (two K stages in flight)
        {128, 128, 2, 2, 2, 2, 2},    // 29 tile 14 with a 3-stage ring
        {64, 256, 1, 4, 2, 2, 2},     // 30 tile 25 with a 3-stage ring
        {64, 128, 2, 2, 2, 1, 2},     // 31 tile 24 with a 4-stage ring
        {32, 256, 1, 4, 3, 1, 2, 1},  // 32 halo for few output channels (2-stage ring)
        {32, 128, 1, 4, 3, 1, 1, 1},  // 33 halo for few output channels, small bands (2-stage ring)
        {32, 256, 1, 4, 3, 1, 2, 1},  // 34 tile 32 with one stage (single-stage reductions: more workgroups per CU)
        {32, 128, 1, 4, 3, 1, 1, 1},  // 35 tile 33 with one stage
        {128, 128, 2, 2, 2, 2, 2, 0, 1}, // 36 persistent tile 14 (2-stage ring)
        {128, 128, 2, 2, 2, 2, 2, 0, 1}, // 37 persistent tile 14, 3-stage ring
        {64, 128, 2, 2, 2, 1, 2, 0, 1},  // 38 persistent tile 24 (2-stage ring)
        {64, 128, 2, 2, 2, 1, 2, 0, 1},  // 39 persistent tile 24, 4-stage ring
        {64, 256, 1, 4, 2, 2, 2, 0, 1},  // 40 persistent tile 25 (2-stage ring)
        {256, 128, 4, 2, 2, 2, 2, 0, 1}, // 41 persistent tile 15 (8 waves, 2-stage ring)
        {128, 128, 2, 2, 2, 2, 2, 0, 1}, // 42 persistent tile 14, 4-stage ring
        {16, 256, 1, 4, 5, 1, 0, 0},     // 43 thin conv, 16 output channels (conv_thin_kernel)
        {32, 256, 1, 4, 5, 2, 0, 0},     // 44 thin conv, 32 output channels
        {64, 256, 1, 4, 5, 4, 0, 0},     // 45 thin conv, 64 output channels
        {128, 128, 2, 2, 2, 2, 2, 0, 0, 1}, // 46 tile 14 with the LDS-staged epilogue
        {64, 128, 2, 2, 2, 1, 2, 0, 0, 1},  // 47 tile 24 with the LDS-staged epilogue
        {128, 128, 2, 2, 2, 2, 2, 0, 0, 1}, // 48 tile 29 (3-stage ring) with the LDS-staged epilogue
        {64, 128, 2, 2, 2, 1, 2, 0, 0, 1},  // 49 tile 31 (4-stage ring) with the LDS-staged epilogue
    };
    constexpr int kNumTiles = 50;
    constexpr int kHaloMaxNBI[kNumTiles] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 4, 15, 10, 16, 48, 48, 48, 0, 0, 8, 15, 0, 0, 0, 0, 15, 8, 16, 10,
                                            0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    typedef void (*GemmKernelFn)(GemmArgs);

    // Kernel selectors, one per tile family (each defined in its own translation unit so the
    // template instantiations compile in parallel). bmode / steps / nbi as in gemm_kernel_for.
    GemmKernelFn gemm_tile_kernel(int tile, int bmode);
    // conv_thin_kernel for cinb input slots (rounded up to 1, 2, 4 or 8), mt 16-channel output
    // fragments, a k x k kernel and stride s (nullptr if not instantiated)
    GemmKernelFn thin_kernel_for(int cinb, int mt, int k, int s, bool res);
    // the 7x7 stride-2 stem on thin tile 45 with its 3x3 stride-2 max pool in one kernel (conv_thin_pool.hip)
    bool thin_pool_ok(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p);
    int  thin_pool_launch(const vkhip_conv_desc *d, const vkhip_pool_desc *p, const void *x, const void *blob, void *y, vkhip_stream_t s);
    inline int thin_cinb(int64_t cinb) { return cinb <= 1 ? 1 : cinb <= 2 ? 2 : cinb <= 4 ? 4 : 8; }
    GemmKernelFn bd_tile_kernel(int tile, int bmode);
    GemmKernelFn dma_tile_kernel(int tile, int bmode, int steps, bool xs);
    GemmKernelFn halo_tile_kernel(int tile, int nbi);
    typedef void (*PwKernelFn)(GemmArgs, PwArgs);
    // the fused 3x3 -> 1x1 kernel for a mid width (64 or 128) and band size, or null
    PwKernelFn pw_tile_kernel(int cmid, int nbi, int mr, int *lds);
    // stem conv + 3x3/s2 max pool (stem_pool.hip): FM = 2 (64 output channels), WM = 1, WN waves
    // over FN fragments each, so BN = 32 FN WN GEMM columns = up to BN / OW conv rows; LDS holds the
    // conv tile (16 channel blocks x BN columns) plus a spare KB. Two configurations: 0 = 8 waves x
    // 4 fragments (1024 columns, one workgroup per CU), 1 = 4 waves x 3 fragments (384 columns,
    // three workgroups per CU). Arguments: conv args, pooled output, POH, POW, pooled rows per
    // workgroup, band chunks.
    constexpr int kSP0FN = 4, kSP0WN = 8, kSP1FN = 3, kSP1WN = 4;
    constexpr int stem_pool_bn(int fn, int wn) { return 32 * fn * wn; }
    constexpr int stem_pool_lds(int fn, int wn) { return 16 * stem_pool_bn(fn, wn) * 8 + 1024; }
    typedef void (*StemPoolFn)(GemmArgs, uint2 *, int, int, int, int);
    StemPoolFn stem_pool_kernel_for(int K, int cfg);
    GemmKernelFn stem_tile_kernel(int tile, int bmode, int nbi);

} // namespace vkhip
