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
// A = packed weights [Coutp][Kp] fp16 (host prepack, zero padded); B = input pixels gathered on
// the fly from NC4HW4 fp16 (8 bytes per (pixel, slot)), zero outside the image.
//
// Reference semantics followed: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) for the convolution,
// residual and activation order; ops/conv.cpp:104-141 + shaders/wino_*_fp16.comp for the
// Winograd F(2,3) matrices (G, B^T, A^T) and the fp16 storage of V and M; the split-K reduce
// (shaders/conv1x1_reduce_fp16.comp) for partial sums + bias + residual + activation.
#include "common.h"
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace vkhip {

    // ------------------------------------------------------------------ kernel arguments
    struct GemmArgs {
        const uint2  *x;    // NC4HW4 fp16, 8-byte (4-channel) vectors
        const half_t *w;    // [Coutp][Kp]
        const float  *bias; // [Coutp]
        const uint2  *res;
        uint2        *y;
        float4v      *part; // split-K partials [ksplit][Coutb][P]
        int           Cinb, H, W, HW;
        int           Coutb, Cout, OW, OHW;
        int           KW, SH, SW, PT, PL, DH, DW;
        int           P, Kslots, Kp, nsteps, steps_per_split;
        int           act;
        float         lo, hi;
        int           has_res, omode, m_tiles;
        long long     x_bstride, w_bstride, y_bstride; // batch (blockIdx.z) strides: uint2 / half / uint2
    };

    enum { OMODE_EPILOGUE = 0, OMODE_RAW = 1, OMODE_PARTIAL = 2 };
    enum { BMODE_1X1 = 0, BMODE_ALIGNED = 1, BMODE_GENERAL = 2 };

    constexpr int kThreads = 256; // 4 wave64s per workgroup
    constexpr int kAStride = 40;  // LDS row stride of the A tile in halves (32 + 8 pad, 80 bytes)

    template <int BM, int BN, int WM, int WN, int BMODE>
    __global__ __launch_bounds__(kThreads) void conv_gemm_kernel(GemmArgs a) {
        constexpr int TM = BM / WM, TN = BN / WN; // wave tile
        constexpr int FM = TM / 32, FN = TN / 32; // 32x32 MFMA fragments per wave
        static_assert(WM * WN == 4, "4 waves");
        static_assert(FM >= 1 && FN >= 1, "wave tile >= 32x32");
        constexpr int SPT     = 8 * BN / kThreads;       // B slots loaded per thread per K step
        constexpr int SSTRIDE = kThreads / BN;           // slot stride between a thread's loads
        constexpr int ACHUNK  = BM * 4;                  // 16-byte chunks in an A tile
        constexpr int ALOADS  = (ACHUNK + kThreads - 1) / kThreads;
        static_assert(SPT >= 1 && kThreads % BN == 0, "BN must divide 256");

        __shared__ __attribute__((aligned(16))) half_t As[2][BM * kAStride];
        __shared__ __attribute__((aligned(16))) uint4  Bs[2][4 * BN];

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = tid >> 6;
        const int wm0  = (wave / WN) * TM;
        const int wn0  = (wave % WN) * TN;

        const int bid    = blockIdx.x;
        const int m_tile = bid % a.m_tiles;
        const int n_tile = bid / a.m_tiles;
        const int m0     = m_tile * BM;
        const int n0     = n_tile * BN;
        const int split  = blockIdx.y;
        const int bz     = blockIdx.z;

        const uint2  *X  = a.x + bz * a.x_bstride;
        const half_t *Wt = a.w + bz * a.w_bstride;

        // ---- this thread's B pixel (fixed for the whole K loop)
        const int  pl     = tid % BN;
        const int  sbase  = tid / BN;
        const int  p      = n0 + pl;
        const bool pvalid = p < a.P;
        int        n = 0, iy0 = 0, ix0 = 0;
        {
            int pp = pvalid ? p : 0;
            n      = pp / a.OHW;
            int r  = pp - n * a.OHW;
            int oy = r / a.OW;
            int ox = r - oy * a.OW;
            iy0    = oy * a.SH - a.PT;
            ix0    = ox * a.SW - a.PL;
        }
        const long long xbase   = (long long) n * a.Cinb * a.HW;
        const int       pix_off = iy0 * a.W + ix0; // 1x1 mode: always inside the image

        const int ks_begin = split * a.steps_per_split;
        const int ks_end   = min(a.nsteps, ks_begin + a.steps_per_split);

        uint4 areg[ALOADS];
        uint2 breg[SPT];

        auto load_tiles = [&](int ks) {
#pragma unroll
            for (int i = 0; i < ALOADS; ++i) {
                int c = tid + i * kThreads;
                if (ACHUNK % kThreads == 0 || c < ACHUNK) {
                    int row = c >> 2, col8 = c & 3;
                    areg[i] = *reinterpret_cast<const uint4 *>(Wt + (long long) (m0 + row) * a.Kp + ks * 32 + col8 * 8);
                }
            }
            if (BMODE == BMODE_ALIGNED) {
                // Cinb % 8 == 0: all 8 slots of this step share one tap (uniform across the block).
                int tap = (ks * 8) / a.Cinb;
                int cb0 = ks * 8 - tap * a.Cinb;
                int ky  = tap / a.KW;
                int kx  = tap - ky * a.KW;
                int iy  = iy0 + ky * a.DH;
                int ix  = ix0 + kx * a.DW;
                bool ok = pvalid && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                const uint2 *src = X + xbase + (long long) cb0 * a.HW + iy * a.W + ix;
#pragma unroll
                for (int j = 0; j < SPT; ++j) {
                    int s   = sbase + j * SSTRIDE;
                    breg[j] = ok ? src[(long long) s * a.HW] : make_uint2(0u, 0u);
                }
            } else {
#pragma unroll
                for (int j = 0; j < SPT; ++j) {
                    int  g  = ks * 8 + sbase + j * SSTRIDE;
                    bool ok = pvalid && g < a.Kslots;
                    long long off = 0;
                    if (BMODE == BMODE_1X1) {
                        off = xbase + (long long) g * a.HW + pix_off;
                    } else {
                        int tap = g / a.Cinb;
                        int cb  = g - tap * a.Cinb;
                        int ky  = tap / a.KW;
                        int kx  = tap - ky * a.KW;
                        int iy  = iy0 + ky * a.DH;
                        int ix  = ix0 + kx * a.DW;
                        ok      = ok && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                        off     = xbase + (long long) cb * a.HW + iy * a.W + ix;
                    }
                    breg[j] = ok ? X[off] : make_uint2(0u, 0u);
                }
            }
        };

        auto store_tiles = [&](int buf) {
#pragma unroll
            for (int i = 0; i < ALOADS; ++i) {
                int c = tid + i * kThreads;
                if (ACHUNK % kThreads == 0 || c < ACHUNK) {
                    int row = c >> 2, col8 = c & 3;
                    *reinterpret_cast<uint4 *>(&As[buf][row * kAStride + col8 * 8]) = areg[i];
                }
            }
#pragma unroll
            for (int j = 0; j < SPT; ++j) {
                int s = sbase + j * SSTRIDE;
                reinterpret_cast<uint2 *>(&Bs[buf][(s >> 1) * BN + pl])[s & 1] = breg[j];
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

        if (ks_begin < ks_end) {
            load_tiles(ks_begin);
            store_tiles(0);
            __syncthreads();
            for (int ks = ks_begin; ks < ks_end; ++ks) {
                const int  buf  = (ks - ks_begin) & 1;
                const bool more = ks + 1 < ks_end;
                if (more) load_tiles(ks + 1);
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    half8 af[FM], bf[FN];
#pragma unroll
                    for (int i = 0; i < FM; ++i)
                        af[i] = *reinterpret_cast<const half8 *>(&As[buf][(wm0 + i * 32 + lrow) * kAStride + kk * 16 + lk * 8]);
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        bf[j] = *reinterpret_cast<const half8 *>(&Bs[buf][(kk * 2 + lk) * BN + wn0 + j * 32 + lrow]);
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int j = 0; j < FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
                if (more) store_tiles(buf ^ 1);
                __syncthreads();
            }
        }

        // ---- epilogue. D layout of a 32x32 fragment: lane l holds column l%32, register r holds
        // row 8*(r/4) + 4*(l/32) + r%4, so registers 4q..4q+3 are one 4-channel block.
        uint2   *Y  = a.y + bz * a.y_bstride;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int px = n0 + wn0 + j * 32 + lrow;
            if (px >= a.P) continue;
            const int pn = px / a.OHW;
            const int pr = px - pn * a.OHW;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int oc  = m0 + wm0 + i * 32 + q * 8 + lk * 4;
                    const int ocb = oc >> 2;
                    if (ocb >= a.Coutb) continue;
                    float4v v;
                    v.x = acc[i][j][q * 4 + 0];
                    v.y = acc[i][j][q * 4 + 1];
                    v.z = acc[i][j][q * 4 + 2];
                    v.w = acc[i][j][q * 4 + 3];
                    if (a.omode == OMODE_PARTIAL) {
                        a.part[((long long) split * a.Coutb + ocb) * a.P + px] = v;
                        continue;
                    }
                    const long long yi = ((long long) pn * a.Coutb + ocb) * a.OHW + pr;
                    if (a.omode == OMODE_EPILOGUE) {
                        float4v b = *reinterpret_cast<const float4v *>(a.bias + oc);
                        v += b;
                        if (a.has_res) v += h4_to_f4(u2_as_h4(a.res[yi]));
                        v.x = apply_act(v.x, a.act, a.lo, a.hi);
                        v.y = apply_act(v.y, a.act, a.lo, a.hi);
                        v.z = apply_act(v.z, a.act, a.lo, a.hi);
                        v.w = apply_act(v.w, a.act, a.lo, a.hi);
                    }
                    if (oc + 0 >= a.Cout) v.x = 0.f;
                    if (oc + 1 >= a.Cout) v.y = 0.f;
                    if (oc + 2 >= a.Cout) v.z = 0.f;
                    if (oc + 3 >= a.Cout) v.w = 0.f;
                    Y[yi] = h4_as_u2(f4_to_h4(v));
                }
            }
        }
    }

    // Split-K reduce: y = act(sum_s part[s] + bias (+res)).
    __global__ void splitk_reduce_kernel(const float4v *part, const float *bias, const uint2 *res, uint2 *y, int ksplit,
                                         int Coutb, int Cout, int P, int OHW, int act, float lo, float hi, int has_res) {
        long long idx   = (long long) blockIdx.x * blockDim.x + threadIdx.x;
        long long total = (long long) Coutb * P;
        if (idx >= total) return;
        int     ocb = (int) (idx / P);
        int     px  = (int) (idx - (long long) ocb * P);
        float4v v   = *reinterpret_cast<const float4v *>(bias + ocb * 4);
        for (int s = 0; s < ksplit; ++s) v += part[((long long) s * Coutb + ocb) * P + px];
        int       pn = px / OHW, pr = px - pn * OHW;
        long long yi = ((long long) pn * Coutb + ocb) * OHW + pr;
        if (has_res) v += h4_to_f4(u2_as_h4(res[yi]));
        v.x = apply_act(v.x, act, lo, hi);
        v.y = apply_act(v.y, act, lo, hi);
        v.z = apply_act(v.z, act, lo, hi);
        v.w = apply_act(v.w, act, lo, hi);
        int oc = ocb * 4;
        if (oc + 0 >= Cout) v.x = 0.f;
        if (oc + 1 >= Cout) v.y = 0.f;
        if (oc + 2 >= Cout) v.z = 0.f;
        if (oc + 3 >= Cout) v.w = 0.f;
        y[yi] = h4_as_u2(f4_to_h4(v));
    }

    // ------------------------------------------------------------------ Winograd F(2x2,3x3)
    // V = B^T d B per 4x4 input tile (pad 1), B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]].
    // V is laid out [pos][Cinb][nT] x 4 channels, i.e. 16 NC4HW4 planes of nT "pixels".
    __global__ void wino_input_kernel(const uint2 *x, uint2 *V, int Cinb, int H, int W, int nTH, int nTW, int nT) {
        long long idx = (long long) blockIdx.x * blockDim.x + threadIdx.x;
        if (idx >= (long long) Cinb * nT) return;
        int cb = (int) (idx / nT);
        int t  = (int) (idx - (long long) cb * nT);
        int per = nTH * nTW;
        int n  = t / per;
        int tr = t - n * per;
        int th = tr / nTW, tw = tr - (tr / nTW) * nTW;
        const uint2 *src = x + ((long long) n * Cinb + cb) * H * W;
        float4v d[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int iy = 2 * th - 1 + i;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int ix = 2 * tw - 1 + j;
                bool ok = iy >= 0 && iy < H && ix >= 0 && ix < W;
                d[i][j] = ok ? h4_to_f4(u2_as_h4(src[iy * W + ix])) : float4v {0.f, 0.f, 0.f, 0.f};
            }
        }
        float4v tm[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            tm[0][j] = d[0][j] - d[2][j];
            tm[1][j] = d[1][j] + d[2][j];
            tm[2][j] = d[2][j] - d[1][j];
            tm[3][j] = d[1][j] - d[3][j];
        }
        const long long plane = (long long) Cinb * nT;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4v v0 = tm[i][0] - tm[i][2];
            float4v v1 = tm[i][1] + tm[i][2];
            float4v v2 = tm[i][2] - tm[i][1];
            float4v v3 = tm[i][1] - tm[i][3];
            V[(i * 4 + 0) * plane + idx] = h4_as_u2(f4_to_h4(v0));
            V[(i * 4 + 1) * plane + idx] = h4_as_u2(f4_to_h4(v1));
            V[(i * 4 + 2) * plane + idx] = h4_as_u2(f4_to_h4(v2));
            V[(i * 4 + 3) * plane + idx] = h4_as_u2(f4_to_h4(v3));
        }
    }

    // Y = A^T M A (A^T = [[1,1,1,0],[0,1,-1,-1]]) + bias, activation, scatter into NC4HW4 fp16.
    __global__ void wino_output_kernel(const uint2 *M, const float *bias, uint2 *y, int Coutb, int Cout, int OH, int OW,
                                       int nTH, int nTW, int nT, int act, float lo, float hi) {
        long long idx = (long long) blockIdx.x * blockDim.x + threadIdx.x;
        if (idx >= (long long) Coutb * nT) return;
        int ocb = (int) (idx / nT);
        int t   = (int) (idx - (long long) ocb * nT);
        int per = nTH * nTW;
        int n   = t / per;
        int tr  = t - n * per;
        int th  = tr / nTW, tw = tr - (tr / nTW) * nTW;
        const long long plane = (long long) Coutb * nT;
        float4v m[4][4];
#pragma unroll
        for (int pos = 0; pos < 16; ++pos) m[pos / 4][pos % 4] = h4_to_f4(u2_as_h4(M[pos * plane + idx]));
        float4v s[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[0][j] = m[0][j] + m[1][j] + m[2][j];
            s[1][j] = m[1][j] - m[2][j] - m[3][j];
        }
        float4v b = *reinterpret_cast<const float4v *>(bias + ocb * 4);
        uint2  *dst = y + ((long long) n * Coutb + ocb) * OH * OW;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float4v o[2];
            o[0] = s[i][0] + s[i][1] + s[i][2] + b;
            o[1] = s[i][1] - s[i][2] - s[i][3] + b;
            int oy = 2 * th + i;
            if (oy >= OH) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                int ox = 2 * tw + j;
                if (ox >= OW) continue;
                float4v v = o[j];
                v.x = apply_act(v.x, act, lo, hi);
                v.y = apply_act(v.y, act, lo, hi);
                v.z = apply_act(v.z, act, lo, hi);
                v.w = apply_act(v.w, act, lo, hi);
                int oc = ocb * 4;
                if (oc + 0 >= Cout) v.x = 0.f;
                if (oc + 1 >= Cout) v.y = 0.f;
                if (oc + 2 >= Cout) v.z = 0.f;
                if (oc + 3 >= Cout) v.w = 0.f;
                dst[oy * OW + ox] = h4_as_u2(f4_to_h4(v));
            }
        }
    }

    // ------------------------------------------------------------------ depthwise
    // Thread = (n, cb, oy, OXT consecutive ox) of one 4-channel block; fp32 weights [Cb][KH][KW][4]
    // and bias [Cb*4]. Reference semantics: ConvCpu with group == C (conv.cpp:40-80).
    struct DwArgs {
        const uint2 *x;
        const float *w;
        const float *bias;
        const uint2 *res;
        uint2       *y;
        int          N, Cb, C, H, W, OH, OW, KH, KW, SH, SW, PT, PL, DH, DW;
        int          act;
        float        lo, hi;
        int          has_res;
    };

    template <int KH, int KW, int S, int OXT>
    __global__ __launch_bounds__(256) void dwconv_kernel(DwArgs a) {
        const int kh = KH > 0 ? KH : a.KH;
        const int kw = KW > 0 ? KW : a.KW;
        const int sh = S > 0 ? S : a.SH;
        const int sw = S > 0 ? S : a.SW;
        const int dh = KH > 0 ? 1 : a.DH;
        const int dw = KH > 0 ? 1 : a.DW;
        int       oxc = (a.OW + OXT - 1) / OXT;
        long long idx = (long long) blockIdx.x * blockDim.x + threadIdx.x;
        long long total = (long long) a.N * a.Cb * a.OH * oxc;
        if (idx >= total) return;
        int xc = (int) (idx % oxc);
        long long t = idx / oxc;
        int oy = (int) (t % a.OH);
        t /= a.OH;
        int cb = (int) (t % a.Cb);
        int n  = (int) (t / a.Cb);
        int ox0 = xc * OXT;
        float4v b = *reinterpret_cast<const float4v *>(a.bias + cb * 4);
        float4v acc[OXT];
#pragma unroll
        for (int o = 0; o < OXT; ++o) acc[o] = b;
        const uint2 *src = a.x + ((long long) n * a.Cb + cb) * a.H * a.W;
        const float4v *wv = reinterpret_cast<const float4v *>(a.w) + (long long) cb * kh * kw;
        const int iy0 = oy * sh - a.PT;
        const int ix0 = ox0 * sw - a.PL;
        for (int ky = 0; ky < kh; ++ky) {
            int iy = iy0 + ky * dh;
            if (iy < 0 || iy >= a.H) continue;
            const uint2 *row = src + (long long) iy * a.W;
            if constexpr (KH > 0) {
                // fixed-size kernel, unit dilation: load the row segment once, reuse across OXT outputs
                constexpr int SEG = (OXT - 1) * (S > 0 ? S : 1) + (KW > 0 ? KW : 1);
                float4v seg[SEG];
#pragma unroll
                for (int c = 0; c < SEG; ++c) {
                    int ix = ix0 + c;
                    seg[c] = (ix >= 0 && ix < a.W) ? h4_to_f4(u2_as_h4(row[ix])) : float4v {0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int kx = 0; kx < KW; ++kx) {
                    float4v wk = wv[ky * KW + kx];
#pragma unroll
                    for (int o = 0; o < OXT; ++o) acc[o] += seg[o * S + kx] * wk;
                }
            } else {
                for (int kx = 0; kx < kw; ++kx) {
                    float4v wk = wv[ky * kw + kx];
#pragma unroll
                    for (int o = 0; o < OXT; ++o) {
                        int ix = ix0 + o * sw + kx * dw;
                        if (ix >= 0 && ix < a.W) acc[o] += h4_to_f4(u2_as_h4(row[ix])) * wk;
                    }
                }
            }
        }
        uint2 *dst = a.y + ((long long) n * a.Cb + cb) * a.OH * a.OW + (long long) oy * a.OW;
        const uint2 *rsrc = a.has_res ? a.res + ((long long) n * a.Cb + cb) * a.OH * a.OW + (long long) oy * a.OW : nullptr;
#pragma unroll
        for (int o = 0; o < OXT; ++o) {
            int ox = ox0 + o;
            if (ox >= a.OW) break;
            float4v v = acc[o];
            if (rsrc) v += h4_to_f4(u2_as_h4(rsrc[ox]));
            v.x = apply_act(v.x, a.act, a.lo, a.hi);
            v.y = apply_act(v.y, a.act, a.lo, a.hi);
            v.z = apply_act(v.z, a.act, a.lo, a.hi);
            v.w = apply_act(v.w, a.act, a.lo, a.hi);
            int c = cb * 4;
            if (c + 0 >= a.C) v.x = 0.f;
            if (c + 1 >= a.C) v.y = 0.f;
            if (c + 2 >= a.C) v.z = 0.f;
            if (c + 3 >= a.C) v.w = 0.f;
            dst[ox] = h4_as_u2(f4_to_h4(v));
        }
    }

    // ------------------------------------------------------------------ host side: tiles & plans
    struct TileCfg {
        int BM, BN, WM, WN;
    };
    static const TileCfg kTiles[] = {
        {128, 128, 2, 2}, // 0
        {64, 128, 2, 2},  // 1
        {128, 64, 2, 2},  // 2
        {64, 64, 2, 2},   // 3
        {256, 128, 2, 2}, // 4
        {128, 256, 2, 2}, // 5
        {32, 128, 1, 4},  // 6
        {64, 256, 1, 4},  // 7
    };
    constexpr int kNumTiles = 8;

    typedef void (*GemmKernelFn)(GemmArgs);

    template <int BM, int BN, int WM, int WN>
    static GemmKernelFn pick_bmode(int bmode) {
        switch (bmode) {
            case BMODE_1X1: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_1X1>;
            case BMODE_ALIGNED: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_ALIGNED>;
            default: return conv_gemm_kernel<BM, BN, WM, WN, BMODE_GENERAL>;
        }
    }

    static GemmKernelFn gemm_kernel_for(int tile, int bmode) {
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

    struct ConvGeom {
        int64_t Cinb, Coutb, Kslots, Kp, nsteps, Coutp, P, m_tiles, n_tiles;
        int     bmode;
    };

    static bool is_depthwise(const vkhip_conv_desc *d) { return d->group > 1; }

    static bool wino_eligible(const vkhip_conv_desc *d) {
        return d->group == 1 && d->KH == 3 && d->KW == 3 && d->SH == 1 && d->SW == 1 && d->PT == 1 && d->PL == 1 &&
               d->DH == 1 && d->DW == 1 && d->OH == d->H && d->OW == d->W;
    }

    // GEMM geometry for the direct implicit-GEMM path (or one Winograd position GEMM).
    static ConvGeom gemm_geom(const vkhip_conv_desc *d, int tile, bool wino) {
        ConvGeom g;
        const TileCfg &t = kTiles[tile];
        g.Cinb  = ceil_div(d->Cin, 4);
        g.Coutb = ceil_div(d->Cout, 4);
        if (wino) {
            int64_t nT = (int64_t) d->N * ceil_div(d->OH, 2) * ceil_div(d->OW, 2);
            g.Kslots   = g.Cinb;
            g.P        = nT;
            g.bmode    = BMODE_1X1;
        } else {
            g.Kslots = (int64_t) d->KH * d->KW * g.Cinb;
            g.P      = (int64_t) d->N * d->OH * d->OW;
            bool one = d->KH == 1 && d->KW == 1 && d->PT == 0 && d->PL == 0;
            g.bmode  = one ? BMODE_1X1 : (g.Cinb % 8 == 0 ? BMODE_ALIGNED : BMODE_GENERAL);
        }
        g.Kp      = round_up(g.Kslots * 4, 32);
        g.nsteps  = g.Kp / 32;
        g.m_tiles = ceil_div(g.Coutb * 4, t.BM);
        g.Coutp   = g.m_tiles * t.BM;
        g.n_tiles = ceil_div(g.P, t.BN);
        return g;
    }

    static int default_tile(const vkhip_conv_desc *d, bool wino) {
        // Largest tile (by area) whose M extent is not mostly empty and that still yields >= 2
        // workgroups per CU (256 CUs); otherwise the smallest tile that fits the channel count.
        const int order[] = {4, 5, 0, 7, 2, 1, 3, 6};
        int64_t   cout4   = ceil_div(d->Cout, 4) * 4;
        int64_t   mcap    = std::max<int64_t>(32, round_up(cout4, 32));
        for (int t: order) {
            const TileCfg &c = kTiles[t];
            if (c.BM > mcap) continue;
            ConvGeom g   = gemm_geom(d, t, wino);
            int64_t  wgs = g.m_tiles * g.n_tiles * (wino ? 16 : 1);
            if (wgs >= 512) return t;
        }
        return mcap <= 32 ? 6 : 3;
    }

    static size_t align256(size_t v) { return (v + 255) & ~(size_t) 255; }

} // namespace vkhip

using namespace vkhip;

extern "C" {

int vkhip_conv_tile_count(void) { return kNumTiles; }

int vkhip_conv_plan_make(const vkhip_conv_desc *d, int32_t algo, int32_t tile, int32_t ksplit, vkhip_conv_plan *plan) {
    if (!d || !plan) return set_error(VKHIP_ERR_INVALID, "conv_plan_make: null argument");
    if (d->N <= 0 || d->Cin <= 0 || d->H <= 0 || d->W <= 0 || d->Cout <= 0 || d->OH <= 0 || d->OW <= 0 || d->KH <= 0 ||
        d->KW <= 0 || d->SH <= 0 || d->SW <= 0 || d->DH <= 0 || d->DW <= 0 || d->PT < 0 || d->PL < 0)
        return set_error(VKHIP_ERR_INVALID, "conv_plan_make: bad geometry");
    if ((d->OH - 1) * d->SH - d->PT + (d->KH - 1) * d->DH < 0 || (d->OW - 1) * d->SW - d->PL + (d->KW - 1) * d->DW < 0)
        return set_error(VKHIP_ERR_INVALID, "conv_plan_make: output does not overlap the input");
    if ((int64_t) d->N * d->OH * d->OW >= (1LL << 31) || (int64_t) d->N * ceil_div(d->Cin, 4) * d->H * d->W >= (1LL << 40))
        return set_error(VKHIP_ERR_INVALID, "conv_plan_make: tensor too large");
    std::memset(plan, 0, sizeof(*plan));
    const bool dw = is_depthwise(d);
    if (dw) {
        if (d->group != d->Cin || d->group != d->Cout)
            return set_error(VKHIP_ERR_UNSUPPORTED, "grouped conv with group=%d (Cin=%d Cout=%d) is not depthwise", d->group, d->Cin, d->Cout);
        if (algo != VKHIP_CONV_AUTO && algo != VKHIP_CONV_DEPTHWISE)
            return set_error(VKHIP_ERR_INVALID, "depthwise conv only runs the depthwise algorithm");
        int64_t Cb         = ceil_div(d->Cin, 4);
        plan->algo         = VKHIP_CONV_DEPTHWISE;
        plan->weight_bytes = align256((size_t) Cb * 4 * 4) + (size_t) Cb * d->KH * d->KW * 16;
        return VKHIP_OK;
    }
    if (d->group != 1) return set_error(VKHIP_ERR_UNSUPPORTED, "grouped conv");
    if (algo == VKHIP_CONV_DEPTHWISE) return set_error(VKHIP_ERR_INVALID, "depthwise algorithm on a dense conv");
    if (algo == VKHIP_CONV_WINOGRAD && !wino_eligible(d))
        return set_error(VKHIP_ERR_INVALID, "Winograd F(2,3) needs 3x3 stride 1 pad 1 dilation 1");
    if (algo == VKHIP_CONV_AUTO) {
        ConvGeom g   = gemm_geom(d, 3, false);
        int64_t  wgs = g.m_tiles * g.n_tiles;
        algo         = (wgs < 256 && g.nsteps >= 16) ? VKHIP_CONV_SPLITK : VKHIP_CONV_GEMM;
    }
    const bool wino = algo == VKHIP_CONV_WINOGRAD;
    if (tile < 0) tile = (algo == VKHIP_CONV_SPLITK) ? (ceil_div(d->Cout, 4) * 4 <= 32 ? 6 : 3) : default_tile(d, wino);
    if (tile >= kNumTiles) return set_error(VKHIP_ERR_INVALID, "tile index %d out of range", tile);
    ConvGeom g = gemm_geom(d, tile, wino);
    plan->algo = algo;
    plan->tile = tile;
    size_t wb  = (size_t) g.Coutp * g.Kp * 2;
    plan->weight_bytes = align256((size_t) g.Coutp * 4) + wb * (wino ? 16 : 1);
    if (algo == VKHIP_CONV_SPLITK) {
        int64_t wgs = g.m_tiles * g.n_tiles;
        if (ksplit <= 0) {
            ksplit = (int) std::min<int64_t>({(int64_t) 16, std::max<int64_t>(2, ceil_div(512, wgs)), g.nsteps});
        }
        if (ksplit < 1) ksplit = 1;
        if (ksplit > g.nsteps) ksplit = (int) g.nsteps;
        plan->ksplit          = ksplit;
        plan->workspace_bytes = (size_t) ksplit * g.Coutb * g.P * 16;
    } else if (wino) {
        int64_t nT            = g.P;
        plan->workspace_bytes = align256((size_t) 16 * g.Cinb * nT * 8) + (size_t) 16 * g.Coutb * nT * 8;
    }
    return VKHIP_OK;
}

int vkhip_conv_pack_weights(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const float *w, const float *bias, void *blob) {
    if (!d || !plan || !w || !blob) return set_error(VKHIP_ERR_INVALID, "conv_pack_weights: null argument");
    std::memset(blob, 0, plan->weight_bytes);
    if (plan->algo == VKHIP_CONV_DEPTHWISE) {
        int64_t Cb = ceil_div(d->Cin, 4);
        float  *b  = (float *) blob;
        float  *wp = (float *) ((char *) blob + align256((size_t) Cb * 16));
        for (int c = 0; c < d->Cin; ++c) {
            if (bias) b[c] = bias[c];
            for (int ky = 0; ky < d->KH; ++ky)
                for (int kx = 0; kx < d->KW; ++kx)
                    wp[(((int64_t) (c / 4) * d->KH + ky) * d->KW + kx) * 4 + c % 4] = w[((int64_t) c * d->KH + ky) * d->KW + kx];
        }
        return VKHIP_OK;
    }
    const bool wino = plan->algo == VKHIP_CONV_WINOGRAD;
    ConvGeom   g    = gemm_geom(d, plan->tile, wino);
    float     *b    = (float *) blob;
    half_t    *wp   = (half_t *) ((char *) blob + align256((size_t) g.Coutp * 4));
    if (bias)
        for (int oc = 0; oc < d->Cout; ++oc) b[oc] = bias[oc];
    if (!wino) {
        for (int oc = 0; oc < d->Cout; ++oc)
            for (int ic = 0; ic < d->Cin; ++ic)
                for (int ky = 0; ky < d->KH; ++ky)
                    for (int kx = 0; kx < d->KW; ++kx) {
                        int64_t slot = ((int64_t) ky * d->KW + kx) * g.Cinb + ic / 4;
                        wp[(int64_t) oc * g.Kp + slot * 4 + ic % 4] = (half_t) w[(((int64_t) oc * d->Cin + ic) * d->KH + ky) * d->KW + kx];
                    }
        return VKHIP_OK;
    }
    // U = G g G^T, G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]] (reference ops/conv.cpp:117-141)
    static const float G[4][3] = {{1.f, 0.f, 0.f}, {0.5f, 0.5f, 0.5f}, {0.5f, -0.5f, 0.5f}, {0.f, 0.f, 1.f}};
    const int64_t      plane = g.Coutp * g.Kp;
    for (int oc = 0; oc < d->Cout; ++oc)
        for (int ic = 0; ic < d->Cin; ++ic) {
            const float *k = w + ((int64_t) oc * d->Cin + ic) * 9;
            float        Gg[4][3];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 3; ++j) Gg[i][j] = G[i][0] * k[j] + G[i][1] * k[3 + j] + G[i][2] * k[6 + j];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) {
                    float u = Gg[i][0] * G[j][0] + Gg[i][1] * G[j][1] + Gg[i][2] * G[j][2];
                    wp[(i * 4 + j) * plane + (int64_t) oc * g.Kp + ic] = (half_t) u;
                }
        }
    return VKHIP_OK;
}

int vkhip_conv_forward(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                       void *y, void *workspace, vkhip_stream_t s) {
    if (!d || !plan || !x || !blob || !y) return set_error(VKHIP_ERR_INVALID, "conv_forward: null argument");
    if (d->has_res && !res) return set_error(VKHIP_ERR_INVALID, "conv_forward: has_res without a residual tensor");
    if (plan->workspace_bytes && !workspace) return set_error(VKHIP_ERR_INVALID, "conv_forward: plan needs a workspace");
    hipStream_t st = resolve_stream(s);

    if (plan->algo == VKHIP_CONV_DEPTHWISE) {
        DwArgs a;
        int64_t Cb = ceil_div(d->Cin, 4);
        a.x = (const uint2 *) x;
        a.bias = (const float *) blob;
        a.w = (const float *) ((const char *) blob + align256((size_t) Cb * 16));
        a.res = (const uint2 *) res;
        a.y = (uint2 *) y;
        a.N = d->N; a.Cb = (int) Cb; a.C = d->Cin; a.H = d->H; a.W = d->W; a.OH = d->OH; a.OW = d->OW;
        a.KH = d->KH; a.KW = d->KW; a.SH = d->SH; a.SW = d->SW; a.PT = d->PT; a.PL = d->PL; a.DH = d->DH; a.DW = d->DW;
        a.act = d->act; a.lo = d->act_lo; a.hi = d->act_hi; a.has_res = d->has_res;
        constexpr int OXT = 4;
        int64_t total = (int64_t) d->N * Cb * d->OH * ceil_div(d->OW, OXT);
        dim3 grid((unsigned) ceil_div(total, 256));
        bool unit = d->DH == 1 && d->DW == 1 && d->SH == d->SW;
        if (unit && d->KH == 3 && d->KW == 3 && d->SH == 1) dwconv_kernel<3, 3, 1, OXT><<<grid, 256, 0, st>>>(a);
        else if (unit && d->KH == 3 && d->KW == 3 && d->SH == 2) dwconv_kernel<3, 3, 2, OXT><<<grid, 256, 0, st>>>(a);
        else if (unit && d->KH == 5 && d->KW == 5 && d->SH == 1) dwconv_kernel<5, 5, 1, OXT><<<grid, 256, 0, st>>>(a);
        else if (unit && d->KH == 5 && d->KW == 5 && d->SH == 2) dwconv_kernel<5, 5, 2, OXT><<<grid, 256, 0, st>>>(a);
        else dwconv_kernel<0, 0, 0, OXT><<<grid, 256, 0, st>>>(a);
        return check_launch("dwconv");
    }

    const bool wino = plan->algo == VKHIP_CONV_WINOGRAD;
    if (plan->tile < 0 || plan->tile >= kNumTiles) return set_error(VKHIP_ERR_INVALID, "conv_forward: bad tile");
    ConvGeom       g = gemm_geom(d, plan->tile, wino);
    const TileCfg &t = kTiles[plan->tile];

    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.w      = (const half_t *) ((const char *) blob + align256((size_t) g.Coutp * 4));
    a.bias   = (const float *) blob;
    a.Cinb   = (int) g.Cinb;
    a.Coutb  = (int) g.Coutb;
    a.Cout   = d->Cout;
    a.P      = (int) g.P;
    a.Kslots = (int) g.Kslots;
    a.Kp     = (int) g.Kp;
    a.nsteps = (int) g.nsteps;
    a.steps_per_split = (int) g.nsteps;
    a.act    = d->act;
    a.lo     = d->act_lo;
    a.hi     = d->act_hi;
    a.m_tiles = (int) g.m_tiles;
    GemmKernelFn fn = gemm_kernel_for(plan->tile, g.bmode);

    if (wino) {
        const int nTH = (int) ceil_div(d->OH, 2), nTW = (int) ceil_div(d->OW, 2);
        const int nT  = (int) g.P;
        uint2    *V   = (uint2 *) workspace;
        uint2    *M   = (uint2 *) ((char *) workspace + align256((size_t) 16 * g.Cinb * nT * 8));
        int64_t   nin = g.Cinb * nT;
        wino_input_kernel<<<dim3((unsigned) ceil_div(nin, 256)), 256, 0, st>>>((const uint2 *) x, V, (int) g.Cinb, d->H, d->W, nTH, nTW, nT);
        int rc = check_launch("wino_input");
        if (rc) return rc;
        a.x = V;
        a.y = M;
        a.H = 1; a.W = nT; a.HW = nT;
        a.OW = nT; a.OHW = nT;
        a.KW = 1; a.SH = 1; a.SW = 1; a.DH = 1; a.DW = 1;
        a.omode     = OMODE_RAW;
        a.x_bstride = (long long) g.Cinb * nT;
        a.w_bstride = (long long) g.Coutp * g.Kp;
        a.y_bstride = (long long) g.Coutb * nT;
        dim3 grid((unsigned) (g.m_tiles * g.n_tiles), 1, 16);
        fn<<<grid, kThreads, 0, st>>>(a);
        if ((rc = check_launch("wino_gemm"))) return rc;
        int64_t nout = g.Coutb * nT;
        wino_output_kernel<<<dim3((unsigned) ceil_div(nout, 256)), 256, 0, st>>>(M, a.bias, (uint2 *) y, (int) g.Coutb, d->Cout, d->OH, d->OW,
                                                                               nTH, nTW, nT, d->act, d->act_lo, d->act_hi);
        return check_launch("wino_output");
    }

    a.x  = (const uint2 *) x;
    a.y  = (uint2 *) y;
    a.res = (const uint2 *) res;
    a.has_res = d->has_res;
    a.H  = d->H; a.W = d->W; a.HW = d->H * d->W;
    a.OW = d->OW; a.OHW = d->OH * d->OW;
    a.KW = d->KW; a.SH = d->SH; a.SW = d->SW; a.PT = d->PT; a.PL = d->PL; a.DH = d->DH; a.DW = d->DW;
    if (plan->algo == VKHIP_CONV_SPLITK) {
        int ks = plan->ksplit;
        a.steps_per_split = (int) ceil_div(g.nsteps, ks);
        ks = (int) ceil_div(g.nsteps, a.steps_per_split);
        a.omode = OMODE_PARTIAL;
        a.part  = (float4v *) workspace;
        dim3 grid((unsigned) (g.m_tiles * g.n_tiles), (unsigned) ks, 1);
        fn<<<grid, kThreads, 0, st>>>(a);
        int rc = check_launch("conv_gemm_splitk");
        if (rc) return rc;
        int64_t total = g.Coutb * g.P;
        splitk_reduce_kernel<<<dim3((unsigned) ceil_div(total, 256)), 256, 0, st>>>(
            (const float4v *) workspace, a.bias, a.res, a.y, ks, (int) g.Coutb, d->Cout, (int) g.P, a.OHW, d->act, d->act_lo,
            d->act_hi, d->has_res);
        return check_launch("splitk_reduce");
    }
    a.omode = OMODE_EPILOGUE;
    dim3 grid((unsigned) (g.m_tiles * g.n_tiles), 1, 1);
    fn<<<grid, kThreads, 0, st>>>(a);
    return check_launch("conv_gemm");
}

} // extern "C"
