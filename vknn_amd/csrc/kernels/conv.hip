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
#include "conv_kernels.h"
#include <mutex>
#include <numeric>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>

namespace vkhip {

    // Split-K reduce: y = act(sum_s part[s] + bias (+res)).
    __global__ void splitk_reduce_kernel(const float4v *part, const float *bias, const uint2 *res, uint2 *y, int ksplit,
                                         int Coutb, int Cout, int P, int OHW, int act, float lo, float hi, int has_res, int ypst) {
        long long idx   = (long long) blockIdx.x * blockDim.x + threadIdx.x;
        long long total = (long long) Coutb * P;
        if (idx >= total) return;
        int     ocb = (int) (idx / P);
        int     px  = (int) (idx - (long long) ocb * P);
        float4v v   = *reinterpret_cast<const float4v *>(bias + ocb * 4);
        for (int s = 0; s < ksplit; ++s) v += part[((long long) s * Coutb + ocb) * P + px];
        int       pn = px / OHW, pr = px - pn * OHW;
        long long yi = ((long long) pn * ypst + ocb) * OHW + pr; // the residual shares y's plane stride
        float4v   r  = {0.f, 0.f, 0.f, 0.f};
        if (has_res) r = h4_to_f4(u2_as_h4(res[yi]));
        if (has_res != 2) v += r;
        v.x = apply_act(v.x, act, lo, hi);
        v.y = apply_act(v.y, act, lo, hi);
        v.z = apply_act(v.z, act, lo, hi);
        v.w = apply_act(v.w, act, lo, hi);
        if (has_res == 2) v += r;
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
        // each tile row as two 16-byte loads of pixel pairs (8-byte aligned); pairs that cross the
        // image's left or right edge fall back to single pixels with the outside one zero
        const int c0 = 2 * tw - 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int iy = 2 * th - 1 + i;
            if (iy < 0 || iy >= H) {
#pragma unroll
                for (int j = 0; j < 4; ++j) d[i][j] = float4v {0.f, 0.f, 0.f, 0.f};
                continue;
            }
            const uint2 *row = src + (long long) iy * W;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = c0 + 2 * h;
                uint2     p0 = {0u, 0u}, p1 = {0u, 0u};
                if (c >= 0 && c + 1 < W) {
                    const u32x4 q = *reinterpret_cast<const u32x4_a8 *>(row + c);
                    p0 = uint2 {q.x, q.y};
                    p1 = uint2 {q.z, q.w};
                } else {
                    if (c >= 0 && c < W) p0 = row[c];
                    if (c + 1 >= 0 && c + 1 < W) p1 = row[c + 1];
                }
                d[i][2 * h]     = h4_to_f4(u2_as_h4(p0));
                d[i][2 * h + 1] = h4_to_f4(u2_as_h4(p1));
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
    // res: the fused residual (same layout as y) or null; added after the bias, before the
    // activation, like every conv epilogue.
    __global__ void wino_output_kernel(const uint2 *M, const float *bias, const uint2 *res, uint2 *y, int Coutb, int Cout, int OH, int OW,
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
        uint2       *dst  = y + ((long long) n * Coutb + ocb) * OH * OW;
        const uint2 *rsrc = res ? res + ((long long) n * Coutb + ocb) * OH * OW : nullptr;
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
                if (rsrc) v += h4_to_f4(u2_as_h4(rsrc[oy * OW + ox]));
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
    // Thread = (n, cb, oy, OXT consecutive ox) of one 4-channel block; fp16 weights [Cb][KH][KW][4]
    // and bias [Cb*4]. Reference semantics: ConvCpu with group == C (conv.cpp:40-80).
    struct DwArgs {
        const uint2 *x;
        const half4 *w;    // fp16 weights [Cb][KH][KW] x 4 channels
        const float *bias;
        const uint2 *res;
        uint2       *y;
        int          N, Cb, C, H, W, OH, OW, KH, KW, SH, SW, PT, PL, DH, DW;
        int          act;
        float        lo, hi;
        int          has_res;
        float4v     *pool; // dwconv_lds_kernel: per-(plane, row tile) sums of the stored outputs, or null
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
        const half4 *wv = a.w + (long long) cb * kh * kw;
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
                    float4v wk = h4_to_f4(wv[ky * KW + kx]);
#pragma unroll
                    for (int o = 0; o < OXT; ++o) acc[o] += seg[o * S + kx] * wk;
                }
            } else {
                for (int kx = 0; kx < kw; ++kx) {
                    float4v wk = h4_to_f4(wv[ky * kw + kx]);
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

    // LDS-tiled depthwise conv for fixed KHxKW / stride with unit dilation. A workgroup owns PP
    // consecutive (n, channel block) planes x RT output rows x the full output width: it copies
    // the input rows those outputs need into LDS once (zero halo for padding, 16-byte loads where
    // rows are 16-byte aligned). Each thread then owns one output column of one plane and computes
    // its RT outputs as a vertical strip: the plane's KHxKW weights stay in registers, and every
    // input row is read from LDS once and added into all the outputs whose window covers it
    // (fp16 taps feed fp32 FMAs through v_fma_mix). HBM traffic is one read of the input (plus the
    // KH - S halo rows per strip) and one coalesced write of the output.
    struct DwTile {
        int PP, IR, IWp, PLA; // planes per WG, LDS rows per plane, LDS row pitch (pixels), LDS column of ix=0
        int PS;               // LDS plane pitch (pixels): IR * IWp padded so consecutive planes start on different banks
        int row_tiles, plane_groups;
        int RPW, rt_groups;   // row tiles per workgroup (> 1: software-pipelined strips), workgroups per plane group
        unsigned mHW, mW;     // ceil(2^32 / (H*W)), ceil(2^32 / W): n / d = umulhi(n, m) for n * d < 2^32 (0: divide)
    };

    // MODE 0: one strip per workgroup. MODE 1: RPW consecutive strips of the same planes per
    // workgroup, the next strip's input prefetched into registers. MODE 2 (one strip covers the
    // plane): a persistent workgroup walks plane groups pg, pg + gridDim.x, ...; the next group's
    // input (one contiguous range) is loaded into registers while the current group computes, and
    // the host sizes the grid so that gridDim.x * PP is a multiple of Cb: every thread keeps the
    // same channel block, so its weights are loaded once.
    template <int KH, int KW, int S, int RT, int MODE>
    __global__ __launch_bounds__(256) void dwconv_lds_kernel(DwArgs a, DwTile t) {
        extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
        constexpr int IR = (RT - 1) * S + KH; // input rows of one strip
        uint2 *tile = reinterpret_cast<uint2 *>(dsm); // [PP][PS: IR x IWp + padding]
        const int tid = threadIdx.x;
        const int rtg = MODE == 2 ? 0 : blockIdx.x % t.rt_groups;
        int       pg  = MODE == 2 ? blockIdx.x : blockIdx.x / t.rt_groups;
        const int NCb = a.N * a.Cb;
        int       p0  = pg * t.PP;
        int       np  = min(t.PP, NCb - p0);
        const int IWp = t.IWp, PLA = t.PLA;

        // The thread's output column and plane; its weights and bias are loaded first so their
        // latency overlaps the input copy.
        const int OW = a.OW;
        const int ox = tid % OW;
        const int pl = tid / OW;
        int       p  = p0 + min(pl, np - 1);
        const int cb = MODE == 2 ? (p0 + min(pl, t.PP - 1)) % a.Cb : p % a.Cb;
        // weights stored and held as fp16 (the storage precision of every GPU weight on this path):
        // half the registers of fp32, and v_fma_mix takes fp16 x fp16 products into the fp32 sums
        half4 w[KH * KW];
#pragma unroll
        for (int k = 0; k < KH * KW; ++k) w[k] = a.w[(long long) cb * KH * KW + k];
        const float4v b0 = *reinterpret_cast<const float4v *>(a.bias + cb * 4);
        // the same weights as channel-wise column pairs for v_dot2_f32_f16 (see strip)
        half2v wp2[KH][KW / 2 > 0 ? KW / 2 : 1][4];
#pragma unroll
        for (int ky = 0; ky < KH; ++ky)
#pragma unroll
            for (int q = 0; q < KW / 2; ++q) {
                const half4 w0 = w[ky * KW + 2 * q], w1 = w[ky * KW + 2 * q + 1];
                wp2[ky][q][0] = half2v {w0.x, w1.x};
                wp2[ky][q][1] = half2v {w0.y, w1.y};
                wp2[ky][q][2] = half2v {w0.z, w1.z};
                wp2[ky][q][3] = half2v {w0.w, w1.w};
            }

        const int W = a.W, H = a.H;
        // input strip of row tile rt -> LDS
        auto load_tile = [&](const int rt) __attribute__((always_inline)) {
        const int iy0 = rt * RT * S - a.PT;
        if (t.row_tiles == 1) {
            // One strip covers every output row, so the workgroup's planes are one contiguous range
            // of the input (np * H * W pixels from plane p0): zero the LDS tile, then copy the range
            // linearly — fully coalesced, all of a thread's loads in flight at once — and drop each
            // pixel at its padded tile position (row iy + PT, column ix + PLA).
            const int tile_units = np * t.PS;
            for (int i = tid; i < tile_units; i += 256) tile[i] = uint2 {0u, 0u};
            __syncthreads();
            constexpr int U    = 16;
            const int     HW   = H * W;
            const int     tot  = np * HW;
            const uint2  *base = a.x + (long long) p0 * HW;
            for (int b0 = tid; b0 < tot; b0 += 256 * U) {
                uint2 v[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int e = b0 + u * 256;
                    v[u]        = e < tot ? base[e] : uint2 {0u, 0u};
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int e = b0 + u * 256;
                    if (e >= tot) break;
                    // e / HW and pix / W by multiply-high (exact: e * HW and pix * W stay below 2^32)
                    const int pl = t.mHW ? (int) __umulhi((unsigned) e, t.mHW) : e / HW, pix = e - pl * HW;
                    const int iy = t.mW ? (int) __umulhi((unsigned) pix, t.mW) : pix / W, ix = pix - iy * W;
                    tile[pl * t.PS + (iy + a.PT) * IWp + ix + PLA] = v[u];
                }
            }
        } else {
            // input rows -> LDS: each thread keeps one column and steps down the rows (plane-major),
            // U rows per round with all U loads issued before any LDS write, so a round costs one
            // memory latency instead of U (most tiles need a single round)
            const bool v16 = (W % 2 == 0) && (PLA % 2 == 0);
            {
                constexpr int U = 16;
                const int cols  = v16 ? IWp / 2 : IWp; // 16- or 8-byte units per LDS row
                const int rpp   = 256 / cols;
                const int col   = tid % cols;
                const int ix    = (v16 ? 2 * col : col) - PLA;
                const bool cok  = ix >= 0 && ix < W;
                const int rows  = np * IR;
                const int r2    = tid / cols;
                if (r2 < rpp) {
                    auto copy = [&](auto vec_c) __attribute__((always_inline)) {
                        using T = decltype(vec_c);
                        for (int base = r2; base < rows; base += U * rpp) {
                            T v[U];
    #pragma unroll
                            for (int u = 0; u < U; ++u) {
                                const int  row = base + u * rpp;
                                const int  pl  = row / IR, r = row - pl * IR; // IR is a compile-time constant
                                const int  iy  = iy0 + r;
                                const bool ok  = row < rows && cok && (unsigned) iy < (unsigned) H;
                                v[u] = T {};
                                if (ok) v[u] = *reinterpret_cast<const T *>(a.x + ((long long) (p0 + pl) * H + iy) * W + ix);
                            }
    #pragma unroll
                            for (int u = 0; u < U; ++u) {
                                const int row = base + u * rpp;
                                const int pl = row / IR, r = row - pl * IR;
                                if (row < rows) *reinterpret_cast<T *>(tile + pl * t.PS + r * IWp + (v16 ? 2 * col : col)) = v[u];
                            }
                        }
                    };
                    if (v16) copy(u32x4 {});
                    else copy(u32x2 {});
                }
            }
        }
        };

        // strip of row tile rt from LDS: RT outputs per thread, activation, store, pool partials
        auto strip = [&](const int rt) __attribute__((always_inline)) {
        const int oy0 = rt * RT;

        const bool live = pl < np && (MODE != 2 || pl < t.PP);
        float4v acc[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) acc[r] = b0;
        const uint2 *src = tile + min(pl, np - 1) * t.PS + ox * S + (PLA - a.PL);
        // Taps in column pairs (kx, kx+1) go through v_dot2_f32_f16: one instruction adds both
        // fp16 x fp16 products of one channel into its fp32 sum, half the FMAs of the strip. A
        // pair's two taps of one channel are packed once per input row and reused by every output
        // row whose window covers the row; an odd last column stays a mixed-precision FMA.
#pragma unroll
        for (int ir = 0; ir < IR; ++ir) {
            half4 tap[KW];
#pragma unroll
            for (int kx = 0; kx < KW; ++kx) tap[kx] = u2_as_h4(src[ir * IWp + kx]);
            half2v tp[KW / 2][4];
#pragma unroll
            for (int q = 0; q < KW / 2; ++q) {
                tp[q][0] = half2v {tap[2 * q].x, tap[2 * q + 1].x};
                tp[q][1] = half2v {tap[2 * q].y, tap[2 * q + 1].y};
                tp[q][2] = half2v {tap[2 * q].z, tap[2 * q + 1].z};
                tp[q][3] = half2v {tap[2 * q].w, tap[2 * q + 1].w};
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int ky = ir - r * S;
                if (ky < 0 || ky >= KH) continue;
#pragma unroll
                for (int q = 0; q < KW / 2; ++q) {
                    acc[r].x = __builtin_amdgcn_fdot2(tp[q][0], wp2[ky][q][0], acc[r].x, false);
                    acc[r].y = __builtin_amdgcn_fdot2(tp[q][1], wp2[ky][q][1], acc[r].y, false);
                    acc[r].z = __builtin_amdgcn_fdot2(tp[q][2], wp2[ky][q][2], acc[r].z, false);
                    acc[r].w = __builtin_amdgcn_fdot2(tp[q][3], wp2[ky][q][3], acc[r].w, false);
                }
                if constexpr (KW % 2) {
                    const half4 wv = w[ky * KW + KW - 1];
                    const half4 tv = tap[KW - 1];
                    acc[r].x = __builtin_fmaf((float) tv.x, (float) wv.x, acc[r].x);
                    acc[r].y = __builtin_fmaf((float) tv.y, (float) wv.y, acc[r].y);
                    acc[r].z = __builtin_fmaf((float) tv.z, (float) wv.z, acc[r].z);
                    acc[r].w = __builtin_fmaf((float) tv.w, (float) wv.w, acc[r].w);
                }
            }
        }
        const int       nrows = live ? min(RT, a.OH - oy0) : 0;
        const long long yb    = ((long long) p * a.OH + oy0) * OW + ox;
        const int       c     = cb * 4;
        float4v         psum  = {0.f, 0.f, 0.f, 0.f}; // this column's share of the plane sum (pool)
        // uniform conditions, tested once: a channel count that is not a multiple of 4 (padding
        // channels of the last block are stored as zeros) and the pool sums
        const bool ragged = (a.C & 3) != 0, pooled = a.pool != nullptr;
        auto finish = [&](auto act_c) __attribute__((always_inline)) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                if (r >= nrows) break;
                float4v v = acc[r];
                if (a.has_res) v += h4_to_f4(u2_as_h4(a.res[yb + (long long) r * OW]));
                v.x = apply_act(v.x, ACT, a.lo, a.hi);
                v.y = apply_act(v.y, ACT, a.lo, a.hi);
                v.z = apply_act(v.z, ACT, a.lo, a.hi);
                v.w = apply_act(v.w, ACT, a.lo, a.hi);
                if (ragged) {
                    if (c + 0 >= a.C) v.x = 0.f;
                    if (c + 1 >= a.C) v.y = 0.f;
                    if (c + 2 >= a.C) v.z = 0.f;
                    if (c + 3 >= a.C) v.w = 0.f;
                }
                const half4 h = f4_to_h4(v);
                a.y[yb + (long long) r * OW] = h4_as_u2(h);
                if (pooled) {
                    // fp16 value x 1 + fp32 sum: one mixed-precision fma per channel, the same
                    // single rounding as converting and adding
                    psum.x = __builtin_fmaf((float) h.x, 1.f, psum.x);
                    psum.y = __builtin_fmaf((float) h.y, 1.f, psum.y);
                    psum.z = __builtin_fmaf((float) h.z, 1.f, psum.z);
                    psum.w = __builtin_fmaf((float) h.w, 1.f, psum.w);
                }
            }
        };
        switch (a.act) {
            case VKHIP_ACT_RELU: finish(std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
            case VKHIP_ACT_RELU6: finish(std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
            case VKHIP_ACT_CLIP: finish(std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
            case VKHIP_ACT_HARDSWISH: finish(std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
            case VKHIP_ACT_SILU: finish(std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
            default: finish(std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
        }
        if (a.pool) {
            // the global-average-pool numerator of a following squeeze-excite, without reading the
            // output back: sum of the fp16 values just stored, per plane of this row tile (columns
            // in order, then the host-visible partials per row tile in order: deterministic)
            __syncthreads(); // every wave is done with the input tile
            // MODE 2 keeps the tile's zero halo across groups: its reduction area follows the tile
            float4v *red = reinterpret_cast<float4v *>(dsm + (MODE == 2 ? ((t.PP * t.PS * 8 + 15) & ~15) : 0));
            red[tid] = psum;
            __syncthreads();
            if (tid < np) {
                float4v sum = {0.f, 0.f, 0.f, 0.f};
                for (int k = 0; k < OW; ++k) sum += red[tid * OW + k];
                a.pool[(long long) (p0 + tid) * t.row_tiles + rt] = sum;
            }
        }
        };

        if constexpr (MODE == 2) {
            // persistent plane groups (row_tiles == 1): the halo of the tile is zeroed once and
            // only the data positions are rewritten per group
            constexpr int UP  = 16; // pixels per thread of one group's input (host: PP * H * W <= 4096)
            const int     HW  = H * W;
            for (int i = tid; i < t.PP * t.PS; i += 256) tile[i] = uint2 {0u, 0u};
            uint2 v[UP];
            auto fetch = [&](const int g) __attribute__((always_inline)) {
                const int    q0   = g * t.PP;
                const int    tot  = min(t.PP, NCb - q0) * HW;
                const uint2 *base = a.x + (long long) q0 * HW;
#pragma unroll
                for (int u = 0; u < UP; ++u) {
                    const int e = tid + u * 256;
                    v[u]        = e < tot ? base[e] : uint2 {0u, 0u};
                }
            };
            if (pg < t.plane_groups) fetch(pg);
            for (bool first = true; pg < t.plane_groups; pg += gridDim.x, first = false) {
                p0 = pg * t.PP;
                np = min(t.PP, NCb - p0);
                p  = p0 + min(pl, np - 1);
                __syncthreads(); // the previous group's strip is done with the tile (first: the halo is zero)
                const int tot = np * HW;
#pragma unroll
                for (int u = 0; u < UP; ++u) {
                    const int e = tid + u * 256;
                    if (e >= tot) break;
                    const int pq = t.mHW ? (int) __umulhi((unsigned) e, t.mHW) : e / HW, pix = e - pq * HW;
                    const int iy = t.mW ? (int) __umulhi((unsigned) pix, t.mW) : pix / W, ix = pix - iy * W;
                    tile[pq * t.PS + (iy + a.PT) * IWp + ix + PLA] = v[u];
                }
                __syncthreads();
                if (pg + (int) gridDim.x < t.plane_groups) fetch(pg + gridDim.x);
                strip(0);
                (void) first;
            }
        } else if constexpr (MODE == 1) {
            const int rt_first = rtg * t.RPW;
            const int rt_end   = min(rt_first + t.RPW, t.row_tiles);
            // Several strips per workgroup, software-pipelined: the global loads of strip k + 1 are
            // issued into registers before strip k is computed from LDS, so their latency hides
            // behind the FMAs. The host selects this only when one round of PF loads of 16 bytes
            // per thread covers a strip (W even, np * IR <= PF * rows per round).
            constexpr int PF   = 8;
            const int     cols = IWp / 2, rpp = 256 / cols;
            const int     col = tid % cols, r2 = tid / cols;
            const int     ix  = 2 * col - PLA;
            const bool    cok = ix >= 0 && ix < W && r2 < rpp;
            const int     rows = np * IR;
            u32x4         v[PF];
            auto fetch = [&](const int rt) __attribute__((always_inline)) {
                const int iy0 = rt * RT * S - a.PT;
#pragma unroll
                for (int u = 0; u < PF; ++u) {
                    const int  row = r2 + u * rpp;
                    const int  pl = row / IR, r = row - pl * IR;
                    const int  iy = iy0 + r;
                    const bool ok = row < rows && cok && (unsigned) iy < (unsigned) H;
                    v[u] = u32x4 {0u, 0u, 0u, 0u};
                    if (ok) v[u] = *reinterpret_cast<const u32x4 *>(a.x + ((long long) (p0 + pl) * H + iy) * W + ix);
                }
            };
            fetch(rt_first);
            for (int rt = rt_first; rt < rt_end; ++rt) {
                if (rt > rt_first) __syncthreads(); // the previous strip's LDS reads are done
                if (r2 < rpp) {
#pragma unroll
                    for (int u = 0; u < PF; ++u) {
                        const int row = r2 + u * rpp;
                        const int pl = row / IR, r = row - pl * IR;
                        if (row < rows) *reinterpret_cast<u32x4 *>(tile + pl * t.PS + r * IWp + 2 * col) = v[u];
                    }
                }
                __syncthreads();
                if (rt + 1 < rt_end) fetch(rt + 1);
                strip(rt);
            }
        } else {
            // one strip per workgroup (the host launches this variant only with RPW == 1)
            load_tile(rtg);
            __syncthreads();
            strip(rtg);
        }
    }

    // Tile geometry for dwconv_lds_kernel: as many planes as fill 256 threads with one output
    // column each; RT output rows per strip.
    static bool dw_tile(const vkhip_conv_desc *d, int64_t NCb, int RT, int RPW, DwTile &t) {
        const int S = d->SH;
        if (d->OW > 256) return false;
        t.PLA = (d->PL + 1) & ~1;
        const int need_w = std::max<int>((d->OW - 1) * S + d->KW - d->PL + t.PLA, t.PLA + d->W);
        t.IWp = (need_w + 1) & ~1;
        if (t.IWp > 256) return false;
        t.IR = (RT - 1) * S + d->KH;
        t.PP = (int) std::max<int64_t>(1, std::min<int64_t>(NCb, 256 / d->OW));
        // plane pitch: the lanes of one plane read about OW * S consecutive 8-byte units, so a pitch
        // of that many units modulo the 32 units of the 64 banks puts the next plane's lanes on the
        // banks right after them
        const int want = ((d->OW * S + 1) & ~1) % 32; // even: rows of a plane stay 16-byte aligned
        t.PS = t.IR * t.IWp;
        while (t.PS % 32 != want) ++t.PS;
        while (t.PP > 1 && (size_t) t.PP * t.PS * 8 > 48 * 1024) --t.PP;
        if ((size_t) t.PP * t.PS * 8 > 48 * 1024) return false;
        const uint64_t HW = (uint64_t) d->H * d->W;
        const uint64_t span = (uint64_t) t.PP * HW; // largest dividend of the plane split
        t.mHW = HW > 1 && span * HW < (1ULL << 32) ? (unsigned) (((1ULL << 32) + HW - 1) / HW) : 0u;
        t.mW  = d->W > 1 && HW * (uint64_t) d->W < (1ULL << 32) ? (unsigned) (((1ULL << 32) + d->W - 1) / d->W) : 0u;
        t.row_tiles    = (int) ceil_div(d->OH, RT);
        t.plane_groups = (int) ceil_div(NCb, t.PP);
        // pipelined strips: W even (16-byte loads) and one round of 8 loads per thread per strip
        t.RPW = std::max(1, std::min(RPW, t.row_tiles));
        if (t.RPW > 1 && (d->W % 2 != 0 || t.PP * t.IR > 8 * (256 / (t.IWp / 2)))) t.RPW = 1;
        t.rt_groups = (int) ceil_div(t.row_tiles, t.RPW);
        return true;
    }

    // Persistent plane groups (depthwise tiles 9xx): one strip covers the plane and one group's
    // input fits 16 pixels per thread.
    static bool dw_persist_ok(const vkhip_conv_desc *d, const DwTile &t) {
        return t.row_tiles == 1 && (int64_t) t.PP * d->H * d->W <= 16 * 256;
    }
    // Grid of the persistent depthwise kernel: every workgroup walks groups g, g + G, ... and keeps
    // its threads' channel blocks only if G * PP is a multiple of Cb, so G is a multiple of
    // q = Cb / gcd(PP, Cb), as many as the device holds at once (at least q); or one workgroup per
    // group when that many fit at once anyway.
    static unsigned dw_persist_grid(const vkhip_conv_desc *d, const DwTile &t, size_t sm) {
        static std::mutex mu;
        static int        cus = 0;
        {
            std::lock_guard<std::mutex> lock(mu);
            if (!cus) {
                int dev = 0;
                if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
                    cus = 256;
            }
        }
        // resident workgroups of 256 threads: 3 per CU by registers for the 3x3 kernels with up to 7
        // rows per strip (<= 168 VGPRs), 2 for the others (<= 232), fewer if the LDS holds fewer
        const int     by_regs = d->KH == 3 && t.IR <= 9 + 6 ? 3 : 2;
        const int64_t per_cu  = std::max<int64_t>(1, std::min<int64_t>(by_regs, (160 * 1024) / std::max<size_t>(sm, 1)));
        const int64_t res    = per_cu * cus;
        if (t.plane_groups <= res) return (unsigned) t.plane_groups;
        const int64_t Cb = ceil_div(d->Cin, 4);
        const int64_t q  = Cb / std::gcd((int64_t) t.PP, Cb);
        return (unsigned) std::max<int64_t>(q, res / q * q);
    }

    // ------------------------------------------------------------------ host side: plans

    // the kernel of tile `tile` (kTiles), by family
    static GemmKernelFn gemm_kernel_for(int tile, int bmode, int steps, int nbi = 0, bool xs = false) {
        if (tile < 0 || tile >= kNumTiles) return nullptr;
        switch (kTiles[tile].kind) {
            case 0: return gemm_tile_kernel(tile, bmode);
            case 1: return bd_tile_kernel(tile, bmode);
            case 2: return dma_tile_kernel(tile, bmode, steps, xs);
            case 3: return halo_tile_kernel(tile, nbi);
            case 4: return stem_tile_kernel(tile, bmode, nbi);
        }
        return nullptr;
    }

    struct ConvGeom {
        int64_t Cinb, Coutb, Kslots, Kp, nsteps, Coutp, P, m_tiles, n_tiles;
        int64_t Pv, HWp; // GEMM columns and columns per image (see GemmArgs::Pv)
        int     bmode;
    };

    static bool is_depthwise(const vkhip_conv_desc *d) { return d->group > 1; }

    // conv_dma_kernel copies B as pixel pairs of one channel slot: the GEMM columns must be dense
    // NC4HW4 pixels (1x1, stride 1, no padding, or a Winograd V plane); an odd pixel count per
    // image gets one padding column per image (gemm_geom).
    static bool dma_eligible(const vkhip_conv_desc *d, bool wino) {
        if (wino) return true;
        const int S = d->SH;
        return d->KH == 1 && d->KW == 1 && (S == 1 || S == 2) && d->SW == S && d->PT == 0 && d->PL == 0 && d->OH == (d->H - 1) / S + 1 &&
               d->OW == (d->W - 1) / S + 1;
    }

    // conv_halo_kernel: 3x3, stride 1 or 2 (both axes), pad 1, dilation 1, output (H - 1)/S + 1,
    // Cin a multiple of the stage's 16*KK channels (odd input widths take the ODD variant).
    static bool halo_shape_ok(const vkhip_conv_desc *d, const TileCfg &t) {
        const int S = d->SH;
        return d->group == 1 && d->KH == 3 && d->KW == 3 && (S == 1 || S == 2) && d->SW == S && d->PT == 1 && d->PL == 1 &&
               d->DH == 1 && d->DW == 1 && d->OH == (d->H - 1) / S + 1 && d->OW == (d->W - 1) / S + 1 && d->Cin % (16 * t.KK) == 0;
    }

    // 1 KB copy chunks per channel slot of the largest input band any workgroup of a halo tile
    // needs: band rows run from the row above the first output pixel's row to the row below the
    // last one's, with two extra (zero) rows per image boundary crossed; W/2 + 1 pixel pairs a row.
    static int halo_nbi(const vkhip_conv_desc *d, const TileCfg &t) {
        const int64_t OHW = (int64_t) d->OH * d->OW, P = (int64_t) d->N * OHW, PW = ((d->W + 3) & ~1) / 2, S = d->SH;
        int64_t       rows = 0;
        for (int64_t p0 = 0; p0 < P; p0 += t.BN) {
            const int64_t p1 = std::min(P, p0 + t.BN) - 1;
            const int64_t nf = p0 / OHW, oyf = (p0 % OHW) / d->OW;
            const int64_t nl = p1 / OHW, oyl = (p1 % OHW) / d->OW;
            rows = std::max(rows, (nl - nf) * (d->H + 2) + S * (oyl - oyf) + 1 + 2);
        }
        int nbi = (int) ceil_div(rows * PW, 64);
        const int nw = t.WM * t.WN;
        while ((4 * t.KK * nbi) % nw) ++nbi;
        return nbi;
    }

    // conv_stem_kernel: at most 4 input channels, square 3x3 or 7x7 kernel, stride 1 or 2 (both
    // axes), pad K/2, dilation 1, even input width.
    static bool stem_shape_ok(const vkhip_conv_desc *d) {
        const int K = d->KH, S = d->SH;
        return d->group == 1 && d->Cin <= 4 && (K == 3 || K == 7) && d->KW == K && (S == 1 || S == 2) && d->SW == S &&
               d->PT == K / 2 && d->PL == K / 2 && d->DH == 1 && d->DW == 1 && d->OH == (d->H + 2 * (K / 2) - K) / S + 1 &&
               d->OW == (d->W + 2 * (K / 2) - K) / S + 1 && d->W % 2 == 0;
    }

    // 1 KB copy chunks of the largest input band a stem workgroup needs (rows of W + K - 1 pixels,
    // H + K - 1 band rows per image).
    static int stem_nbi(const vkhip_conv_desc *d, const TileCfg &t) {
        const int64_t OHW = (int64_t) d->OH * d->OW, P = (int64_t) d->N * OHW, S = d->SH, K = d->KH;
        const int64_t RS = d->W + K - 1, VR = d->H + K - 1;
        int64_t       rows = 0;
        for (int64_t p0 = 0; p0 < P; p0 += t.BN) {
            const int64_t p1 = std::min(P, p0 + t.BN) - 1;
            const int64_t nf = p0 / OHW, oyf = (p0 % OHW) / d->OW;
            const int64_t nl = p1 / OHW, oyl = (p1 % OHW) / d->OW;
            rows = std::max(rows, (nl - nf) * VR + S * (oyl - oyf) + 2 * (K / 2) + 1);
        }
        return (int) ceil_div(rows * (RS / 2), 64);
    }

    // conv_thin_kernel: 3x3 pad 1 (stride 1 or 2), 1x1 pad 0 stride 1 or 7x7 pad 3 stride 2 over at most
    // 4 channels; dilation 1, Cin <= 32, Cout
    // within the tile's BM, even input width (the band copies whole pixel pairs), no input scale, a
    // residual only on 3x3 stride 1, and an instantiated kernel (its weights fit the register budget)
    static bool thin_shape_ok(const vkhip_conv_desc *d, const TileCfg &t, int algo) {
        const int K = d->KH, S = d->SH;
        if (algo != VKHIP_CONV_GEMM || d->group != 1 || d->in_scale || d->Cin > 32 || d->Cout > t.BM) return false;
        if (d->KW != K || d->SW != S || d->DH != 1 || d->DW != 1 || d->W % 2) return false;
        if (!((K == 3 && d->PT == 1 && d->PL == 1 && (S == 1 || S == 2)) || (K == 1 && d->PT == 0 && d->PL == 0 && S == 1) ||
              (K == 7 && d->PT == 3 && d->PL == 3 && S == 2 && d->Cin <= 4)))
            return false;
        if (d->OH != (d->H + 2 * d->PT - K) / S + 1 || d->OW != (d->W + 2 * d->PL - K) / S + 1) return false;
        return thin_kernel_for((int) ceil_div(d->Cin, 4), t.FM, K, S, d->has_res != 0) != nullptr;
    }

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
            g.bmode    = (t.kind == 0 && nT % 2 == 0) ? BMODE_1X1_P16 : BMODE_1X1;
        } else {
            g.Kslots = (int64_t) d->KH * d->KW * g.Cinb;
            g.P      = (int64_t) d->N * d->OH * d->OW;
            const bool one  = d->KH == 1 && d->KW == 1 && d->PT == 0 && d->PL == 0;
            const bool unit = d->SW == 1 && d->DW == 1;
            if (t.kind == 1) g.bmode = one ? BMODE_1X1 : ((g.Cinb % 4 == 0 && d->KH * d->KW <= 32) ? BMODE_ALIGNED : BMODE_GENERAL);
            else if (one) g.bmode = (d->SH == 1 && d->SW == 1 && (d->OH * d->OW) % 2 == 0) ? BMODE_1X1_P16 : BMODE_1X1;
            else if (g.Cinb % 8 == 0) g.bmode = (unit && d->OW % 2 == 0) ? BMODE_ALIGNED_P16 : BMODE_ALIGNED;
            else g.bmode = BMODE_GENERAL;
        }
        g.Kp      = round_up(g.Kslots * 4, kBK);
        g.nsteps  = g.Kp / kBK;
        if (t.kind == 4) { // all K*K taps x 4 channels in one stage of ceil(K*K/4) 16-deep steps
            g.Kp     = ceil_div((int64_t) d->KH * d->KW, 4) * 16;
            g.nsteps = 1;
            g.bmode  = d->KH;
        }
        if (t.kind == 5) { // (tap, channel) over the rounded slot count, 32-deep MFMA steps
            g.nsteps = ceil_div((int64_t) d->KH * d->KW * thin_cinb(g.Cinb) * 4, 32);
            g.Kp     = g.nsteps * 32;
        }
        if (t.kind == 3) { // 9 taps x Cin, stages of 16*KK channels (all 9 taps each)
            g.Kp     = 9 * (int64_t) d->Cin;
            g.nsteps = d->Cin / (16 * t.KK);
        }
        g.m_tiles = ceil_div(g.Coutb * 4, t.BM);
        g.Coutp   = g.m_tiles * t.BM;
        g.HWp     = wino ? g.P : (int64_t) d->OH * d->OW;
        if (t.kind == 2 && !wino && d->SH == 2) g.bmode = 2; // stride-2 columns: one pixel per lane, no pairing
        else if (t.kind == 2) g.HWp += g.HWp & 1;
        g.Pv      = wino ? g.HWp : (int64_t) d->N * g.HWp;
        g.n_tiles = ceil_div(g.Pv, t.BN);
        return g;
    }

    // Position of weight (oc, k) in the tiled layout [m_tile][k_stage][BM][64]: one K stage of one
    // M tile is a contiguous BM*64-half block, read linearly by the kernel.
    // kind 1 tiles store each stage in MFMA A-fragment order instead: [kk (16-K step)][m fragment]
    // [lane][8 halves], lane = (k%16)/8*32 + row%32, so the LDS image is the global image.
    static inline int64_t tiled_index(const ConvGeom &g, const TileCfg &t, int64_t oc, int64_t k) {
        const int     BM   = t.BM;
        const int64_t base = ((oc / BM) * g.nsteps + k / kBK) * (int64_t) (BM * kBK);
        if (t.kind == 0) return base + (oc % BM) * kBK + k % kBK; // kinds 1 and 2: fragment order
        if (t.kind == 5) {
            // [m_frag][step][lane][8 halves], lane = (kt%32)/8 * 16 + oc%16, kt = tap*4*cinb' + c
            const int64_t tap = (k / 4) / g.Cinb, c = ((k / 4) % g.Cinb) * 4 + k % 4;
            const int64_t kt  = tap * thin_cinb(g.Cinb) * 4 + c;
            return (((oc / 16) * g.nsteps + kt / 32) * 64 + ((kt % 32) / 8) * 16 + oc % 16) * 8 + kt % 8;
        }
        if (t.kind == 4) {
            // [m_tile][step][m_frag][lane][8 halves]; Cinb = 1, so k = tap*4 + c and step = tap/4
            const int64_t tap = k / 4, kr = (tap % 4) * 4 + k % 4, r = oc % BM;
            const int64_t l = (kr / 8) * 32 + r % 32;
            return (oc / BM) * g.Kp * BM + (((tap / 4) * (BM / 32) + r / 32) * 64 + l) * 8 + kr % 8;
        }
        if (t.kind == 3) {
            // [m_tile][stage][tap][kk][m_frag][lane][8 halves]; k = (tap*Cinb + cb)*4 + c%4
            const int64_t tap = (k / 4) / g.Cinb, c = ((k / 4) % g.Cinb) * 4 + k % 4;
            const int64_t SK = 16 * t.KK, stage = c / SK, kk = (c % SK) / 16, kr = c % 16, r = oc % BM;
            const int64_t l = (kr / 8) * 32 + r % 32;
            const int64_t hb = ((oc / BM) * g.nsteps + stage) * (int64_t) (9 * SK * BM);
            return hb + (((tap * t.KK + kk) * (BM / 32) + r / 32) * 64 + l) * 8 + kr % 8;
        }
        const int64_t r = oc % BM, kr = k % kBK;
        const int64_t kk = kr / 16, l = ((kr % 16) / 8) * 32 + r % 32;
        return base + ((kk * (BM / 32) + r / 32) * 64 + l) * 8 + kr % 8;
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

    // Grid of a persistent kernel: the workgroups the device holds at once (occupancy of this
    // kernel x CUs), a multiple of 8 (its tile order deals tiles to the 8 XCDs), and no more than
    // the tiles need.
    static unsigned persist_grid(GemmKernelFn fn, int threads, int64_t ntiles) {
        static std::mutex                   mu;
        static std::vector<std::pair<const void *, int>> occ;
        static int                          cus = 0;
        int                                 n   = 0;
        {
            std::lock_guard<std::mutex> lock(mu);
            if (!cus) {
                int dev = 0;
                if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                    cus <= 0)
                    cus = 256;
            }
            for (auto &e: occ)
                if (e.first == (const void *) fn) n = e.second;
            if (!n) {
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *) fn, threads, 0) != hipSuccess || n <= 0) n = 1;
                occ.emplace_back((const void *) fn, n);
            }
        }
        int64_t g = std::max<int64_t>(8, ((int64_t) cus * n) / 8 * 8);
        return (unsigned) std::min<int64_t>(g, round_up(ntiles, 8));
    }

    // Scratch of the allocation-free forward entry point: one copy per GPU (a __device__ array
    // lives in every device's memory at its own address). Host code never passes the array's name
    // to a kernel: it is only a host-side handle, so the per-device address comes from
    // hipGetSymbolAddress, taken once per device with that device current.
    static __device__ __align__(256) unsigned char scratch[VKHIP_NOALLOC_SCRATCH_BYTES];
    // Arrival counters of its in-kernel split-K reductions (VKHIP_CONV_SPLITK_LAST), apart from the
    // scratch that other calls overwrite: zero when the module loads, and every call leaves them zero.
    static __device__ __align__(256) int scratch_counters[VKHIP_NOALLOC_MAX_TILES];
    constexpr int kMaxDevices = 64;

    static int scratch_ptr(void **out, int **counters) {
        static std::mutex mu;
        static void      *ptrs[kMaxDevices] = {};
        static void      *cptrs[kMaxDevices] = {};
        int               dev             = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
            return set_error(VKHIP_ERR_RUNTIME, "conv_forward_noalloc: no current device");
        std::lock_guard<std::mutex> lock(mu);
        if (!ptrs[dev]) {
            void      *p = nullptr, *c = nullptr;
            hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (rc == hipSuccess) rc = hipGetSymbolAddress(&c, HIP_SYMBOL(scratch_counters));
            if (rc != hipSuccess || !p || !c)
                return set_error(VKHIP_ERR_RUNTIME, "conv_forward_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                                 hipGetErrorString(rc));
            ptrs[dev]  = p;
            cptrs[dev] = c;
        }
        *out      = ptrs[dev];
        *counters = (int *) cptrs[dev];
        return VKHIP_OK;
    }

} // namespace vkhip

using namespace vkhip;

extern "C" {

int vkhip_conv_tile_count(void) { return kNumTiles; }

const char *vkhip_conv_plan_kernel(const vkhip_conv_plan *plan) {
    static const char *kinds[] = {"conv_gemm_kernel", "conv_bd_kernel", "conv_dma_kernel", "conv_halo_kernel", "conv_stem_kernel", "conv_thin_kernel"};
    if (!plan) return "?";
    if (plan->algo == VKHIP_CONV_GEMM && plan->tile >= 0 && plan->tile < kNumTiles && kTiles[plan->tile].PERS) return "conv_dma_persist_kernel";
    if (plan->algo == VKHIP_CONV_DEPTHWISE) return "dwconv_lds_kernel";
    if (plan->tile < 0 || plan->tile >= kNumTiles) return "?";
    if (plan->algo == VKHIP_CONV_WINOGRAD) return "wino_input_kernel+conv_gemm_kernel+wino_output_kernel";
    return kinds[kTiles[plan->tile].kind];
}

int vkhip_conv_plan_make(const vkhip_conv_desc *d, int32_t algo, int32_t tile, int32_t ksplit, vkhip_conv_plan *plan) {
    if (!d || !plan) return set_error(VKHIP_ERR_INVALID, "conv_plan_make: null argument");
    if (d->N <= 0 || d->Cin <= 0 || d->H <= 0 || d->W <= 0 || d->Cout <= 0 || d->OH <= 0 || d->OW <= 0 || d->KH <= 0 ||
        d->KW <= 0 || d->SH <= 0 || d->SW <= 0 || d->DH <= 0 || d->DW <= 0 || d->PT < 0 || d->PL < 0)
        return set_error(VKHIP_ERR_INVALID, "conv_plan_make: bad geometry");
    if ((d->OH - 1) * d->SH - d->PT + (d->KH - 1) * d->DH < 0 || (d->OW - 1) * d->SW - d->PL + (d->KW - 1) * d->DW < 0)
        return set_error(VKHIP_ERR_INVALID, "conv_plan_make: output does not overlap the input");
    // the GEMM gathers address the input through a buffer resource with 31-bit byte offsets
    if ((int64_t) d->N * d->OH * d->OW >= (1LL << 31) || (int64_t) d->N * ceil_div(d->Cin, 4) * d->H * d->W * 8 >= (1LL << 31) ||
        (int64_t) d->N * ceil_div(d->Cout, 4) * d->OH * d->OW * 8 >= (1LL << 31) ||
        (int64_t) 16 * d->N * ceil_div(std::max(d->Cin, d->Cout), 4) * ceil_div(d->OH, 2) * ceil_div(d->OW, 2) * 8 >= (1LL << 31))
        return set_error(VKHIP_ERR_INVALID, "conv_plan_make: input tensor >= 2 GiB (split the batch)");
    if (d->has_res < 0 || d->has_res > 2) return set_error(VKHIP_ERR_INVALID, "conv_plan_make: has_res is 0, 1 or 2");
    std::memset(plan, 0, sizeof(*plan));
    const bool dw = is_depthwise(d);
    if (dw && d->has_res == 2) return set_error(VKHIP_ERR_UNSUPPORTED, "depthwise conv: no residual after the activation");
    if (dw) {
        if (d->group != d->Cin || d->group != d->Cout)
            return set_error(VKHIP_ERR_UNSUPPORTED, "grouped conv with group=%d (Cin=%d Cout=%d) is not depthwise", d->group, d->Cin, d->Cout);
        if (algo != VKHIP_CONV_AUTO && algo != VKHIP_CONV_DEPTHWISE)
            return set_error(VKHIP_ERR_INVALID, "depthwise conv only runs the depthwise algorithm");
        // tile = rows per strip (4, 7 or 14) + 100 x strips per workgroup (2 or 4: pipelined strips)
        if (tile > 0 && ((tile % 100 != 4 && tile % 100 != 7 && tile % 100 != 14) || (tile / 100 != 0 && tile / 100 != 2 && tile / 100 != 4 && tile / 100 != 9)))
            return set_error(VKHIP_ERR_INVALID, "depthwise tile %d: rows per strip 4, 7 or 14, plus 100 x 2 or 4 strips per workgroup, or 900 "
                             "(persistent plane groups) (0 or -1: by shape)", tile);
        if (tile >= 900) {
            DwTile t;
            const bool unit = d->DH == 1 && d->DW == 1 && d->SH == d->SW && d->KH == d->KW && (d->KH == 3 || d->KH == 5) && (d->SH == 1 || d->SH == 2);
            if (!unit || !dw_tile(d, (int64_t) d->N * ceil_div(d->Cin, 4), tile % 100, 1, t) || !dw_persist_ok(d, t))
                return set_error(VKHIP_ERR_UNSUPPORTED, "depthwise tile %d: persistent plane groups need one strip per plane and at most 4096 "
                                 "input pixels per group", tile);
        }
        int64_t Cb         = ceil_div(d->Cin, 4);
        plan->algo         = VKHIP_CONV_DEPTHWISE;
        plan->tile         = tile > 0 ? tile : 0;
        plan->weight_bytes = align256((size_t) Cb * 4 * 4) + (size_t) Cb * d->KH * d->KW * 8;
        return VKHIP_OK;
    }
    if (d->group != 1) return set_error(VKHIP_ERR_UNSUPPORTED, "grouped conv");
    if (algo == VKHIP_CONV_DEPTHWISE) return set_error(VKHIP_ERR_INVALID, "depthwise algorithm on a dense conv");
    if (d->in_scale) {
        // the scale rides on the dense-B (LDS-DMA) kernel: 1x1, stride 1, no padding, no split-K
        if (d->KH != 1 || d->KW != 1 || d->SH != 1 || d->SW != 1 || d->PT != 0 || d->PL != 0 || d->OH != d->H || d->OW != d->W)
            return set_error(VKHIP_ERR_UNSUPPORTED, "input scale needs a 1x1 stride-1 pad-0 conv");
        if (algo == VKHIP_CONV_AUTO) algo = VKHIP_CONV_GEMM;
        if (algo != VKHIP_CONV_GEMM) return set_error(VKHIP_ERR_UNSUPPORTED, "input scale runs the GEMM algorithm only");
        if (tile < 0) tile = 14;
        if (tile >= kNumTiles || kTiles[tile].kind != 2 || !dma_tile_kernel(tile, 0, 1, true))
            return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d has no input-scale variant", tile);
        // a workgroup's columns may cover at most 8 images (the scale slice of a stage)
        const int64_t hwp = (int64_t) d->OH * d->OW + ((int64_t) d->OH * d->OW & 1);
        if (ceil_div(kTiles[tile].BN - 1, hwp) > 7)
            return set_error(VKHIP_ERR_UNSUPPORTED, "input scale: tile %d spans more than 8 images of %lld pixels", tile, (long long) hwp);
    }
    if (algo == VKHIP_CONV_WINOGRAD && !wino_eligible(d))
        return set_error(VKHIP_ERR_INVALID, "Winograd F(2,3) needs 3x3 stride 1 pad 1 dilation 1");
    if (algo < VKHIP_CONV_AUTO || algo > VKHIP_CONV_SPLITK_LAST) return set_error(VKHIP_ERR_INVALID, "unknown conv algorithm %d", algo);
    if (algo == VKHIP_CONV_AUTO) {
        ConvGeom g   = gemm_geom(d, 3, false);
        int64_t  wgs = g.m_tiles * g.n_tiles;
        algo         = (wgs < 256 && g.nsteps >= 16) ? VKHIP_CONV_SPLITK : VKHIP_CONV_GEMM;
    }
    const bool wino  = algo == VKHIP_CONV_WINOGRAD;
    const bool split = algo == VKHIP_CONV_SPLITK || algo == VKHIP_CONV_SPLITK_LAST;
    if (tile < 0) tile = split ? (ceil_div(d->Cout, 4) * 4 <= 32 ? 6 : 3) : default_tile(d, wino);
    if (tile >= kNumTiles) return set_error(VKHIP_ERR_INVALID, "tile index %d out of range", tile);
    if (algo == VKHIP_CONV_SPLITK_LAST && (kTiles[tile].kind > 3 || kTiles[tile].PERS || kTiles[tile].LE))
        return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d has no in-kernel split-K reduction (gather, B-direct, LDS-DMA and halo tiles only)", tile);
    if (d->has_res == 2 && (wino || kTiles[tile].kind == 4))
        return set_error(VKHIP_ERR_UNSUPPORTED, "a residual after the activation runs on GEMM / split-K plans of the gather, B-direct, LDS-DMA, "
                         "halo and thin tiles only");
    if (kTiles[tile].kind == 3 && (wino || !halo_shape_ok(d, kTiles[tile]) || halo_nbi(d, kTiles[tile]) > kHaloMaxNBI[tile]))
        return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d needs a 3x3 stride-1/2 pad-1 conv with Cin %% %d == 0 and a band that fits LDS", tile,
                         16 * kTiles[tile].KK);
    if (kTiles[tile].kind == 4 && (wino || !stem_shape_ok(d) || stem_nbi(d, kTiles[tile]) > kHaloMaxNBI[tile]))
        return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d needs a 3x3/7x7 stride-1/2 pad-K/2 conv over at most 4 channels with even W", tile);
    if (kTiles[tile].kind == 2 && dma_eligible(d, wino) && !gemm_kernel_for(tile, gemm_geom(d, tile, wino).bmode, 1))
        return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d has no stride-2 variant (LDS)", tile);
    if (kTiles[tile].kind == 2 && !dma_eligible(d, wino))
        return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d needs a dense B operand (1x1 stride 1 with an even pixel count, or Winograd)", tile);
    if (kTiles[tile].kind == 5 && !thin_shape_ok(d, kTiles[tile], algo))
        return set_error(VKHIP_ERR_UNSUPPORTED, "thin tile %d needs a plain GEMM plan of a 3x3 pad-1 or 1x1 conv, stride 1 or 2 (1x1: stride 1), "
                         "Cin <= 32, Cout <= %d, even input width, a residual only on 3x3 stride 1", tile, kTiles[tile].BM);
    if (kTiles[tile].LE && (algo != VKHIP_CONV_GEMM || d->in_scale || ((int64_t) d->OH * d->OW) % 2))
        return set_error(VKHIP_ERR_UNSUPPORTED, "tile %d (LDS-staged epilogue) runs plain GEMM plans of an even pixel count per image only", tile);
    if (kTiles[tile].PERS && (algo != VKHIP_CONV_GEMM || d->in_scale))
        return set_error(VKHIP_ERR_UNSUPPORTED, "persistent tile %d runs plain GEMM plans only (no split-K, Winograd or input scale)", tile);
    ConvGeom g = gemm_geom(d, tile, wino);
    plan->algo = algo;
    plan->tile = tile;
    size_t wb  = (size_t) g.Coutp * g.Kp * 2;
    plan->weight_bytes = align256((size_t) g.Coutp * 4) + wb * (wino ? 16 : 1);
    if (split) {
        int64_t wgs = g.m_tiles * g.n_tiles;
        if (ksplit <= 0) {
            ksplit = (int) std::min<int64_t>({(int64_t) 16, std::max<int64_t>(2, ceil_div(512, wgs)), g.nsteps});
        }
        if (ksplit < 1) ksplit = 1;
        if (ksplit > g.nsteps) ksplit = (int) g.nsteps;
        while (ksplit > 1 && (int64_t) ksplit * g.Coutb * g.P * 16 >= (1LL << 31)) --ksplit;
        plan->ksplit          = ksplit;
        plan->workspace_bytes = (size_t) ksplit * g.Coutb * g.P * 16;
        // SPLITK_LAST: one arrival counter per output tile after the partials
        if (algo == VKHIP_CONV_SPLITK_LAST) plan->workspace_bytes = align256(plan->workspace_bytes) + (size_t) wgs * 4;
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
        half_t *wp = (half_t *) ((char *) blob + align256((size_t) Cb * 16));
        for (int c = 0; c < d->Cin; ++c) {
            if (bias) b[c] = bias[c];
            for (int ky = 0; ky < d->KH; ++ky)
                for (int kx = 0; kx < d->KW; ++kx)
                    wp[(((int64_t) (c / 4) * d->KH + ky) * d->KW + kx) * 4 + c % 4] = ref_half(w[((int64_t) c * d->KH + ky) * d->KW + kx]);
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
                        wp[tiled_index(g, kTiles[plan->tile], oc, slot * 4 + ic % 4)] = ref_half(w[(((int64_t) oc * d->Cin + ic) * d->KH + ky) * d->KW + kx]);
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
                    wp[(i * 4 + j) * plane + tiled_index(g, kTiles[plan->tile], oc, ic)] = ref_half(u);
                }
        }
    return VKHIP_OK;
}

} // extern "C"

// ---------------------------------------------------------------- stem conv + max pool
namespace vkhip {
    // Pooled rows per workgroup and band chunks of the fused stem + pool kernel, or false when the
    // pair does not fit it: a stem-kernel plan with 64-row tiles (one M tile: Cout <= 64), no
    // residual, a 3x3 stride-2 pad-1 pool over exactly the conv output, and a band that fits LDS
    // next to the weights.
    // Configuration: the 1024-column workgroups (several pooled rows per tile, so the recomputed
    // shared conv row costs least), else the 384-column ones.
    static bool stem_pool_geom(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p, int &PR, int &NBI, int &cfg) {
        if (!d || !plan || !p) return false;
        if (plan->algo != VKHIP_CONV_GEMM || plan->tile < 0 || plan->tile >= kNumTiles) return false;
        const TileCfg &t = kTiles[plan->tile];
        if (t.kind != 4 || t.BM != 64 || d->Cout > 64 || d->has_res || d->in_scale || !stem_shape_ok(d)) return false;
        if (p->N != d->N || p->C != d->Cout || p->H != d->OH || p->W != d->OW || p->KH != 3 || p->KW != 3 || p->SH != 2 || p->SW != 2 ||
            p->PT != 1 || p->PL != 1 || p->OH != (d->OH - 1) / 2 + 1 || p->OW != (d->OW - 1) / 2 + 1)
            return false;
        const int K = d->KH, S = d->SH, RS = d->W + K - 1, KT = (K * K + 3) / 4;
        for (cfg = 0; cfg < 2; ++cfg) {
            const int bn = cfg == 0 ? stem_pool_bn(kSP0FN, kSP0WN) : stem_pool_bn(kSP1FN, kSP1WN);
            const int lds = cfg == 0 ? stem_pool_lds(kSP0FN, kSP0WN) : stem_pool_lds(kSP1FN, kSP1WN);
            PR = (bn / d->OW - 1) / 2;
            if (PR < 1) continue;
            const int R = 2 * PR + 1, VRB = S * (R - 1) + K;
            NBI = (int) ceil_div((int64_t) VRB * (RS / 2), 64);
            if ((KT * 2 + NBI) * 1024 + 32 <= lds - 1024) return true;
        }
        return false;
    }
} // namespace vkhip

extern "C" {

int vkhip_conv_maxpool_supported(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p) {
    int PR, NBI, cfg;
    return thin_pool_ok(d, plan, p) || stem_pool_geom(d, plan, p, PR, NBI, cfg) ? 1 : 0;
}

int vkhip_conv_maxpool_forward(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p, const void *x, const void *blob,
                               void *y, vkhip_stream_t s) {
    if (!d || !plan || !p || !x || !blob || !y) return set_error(VKHIP_ERR_INVALID, "conv_maxpool: null argument");
    if (thin_pool_ok(d, plan, p)) return thin_pool_launch(d, p, x, blob, y, s);
    int PR = 0, NBI = 0, cfg = 0;
    if (!stem_pool_geom(d, plan, p, PR, NBI, cfg)) return set_error(VKHIP_ERR_UNSUPPORTED, "conv_maxpool: shape or plan not supported");
    StemPoolFn fn = stem_pool_kernel_for(d->KH, cfg);
    if (!fn) return set_error(VKHIP_ERR_UNSUPPORTED, "conv_maxpool: kernel size");
    ConvGeom g = gemm_geom(d, plan->tile, false);
    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.w      = (const half_t *) ((const char *) blob + align256((size_t) g.Coutp * 4));
    a.bias   = (const float *) blob;
    a.Cinb   = (int) g.Cinb;
    a.Coutb  = (int) g.Coutb;
    a.Cout   = d->Cout;
    a.act    = d->act;
    a.lo     = d->act_lo;
    a.hi     = d->act_hi;
    a.x      = (const uint2 *) x;
    a.x_bytes = (unsigned) ((int64_t) d->N * g.Cinb * d->H * d->W * 8);
    a.H  = d->H; a.W = d->W; a.HW = d->H * d->W;
    a.OW = d->OW; a.OHW = d->OH * d->OW;
    a.SH = d->SH; a.SW = d->SW; a.PT = d->PT; a.PL = d->PL;
    const int groups = (int) ceil_div(p->OH, PR);
    fn<<<dim3((unsigned) (d->N * groups)), 64 * (cfg == 0 ? kSP0WN : kSP1WN), 0, resolve_stream(s)>>>(a, (uint2 *) y, p->OH, p->OW, PR, NBI);
    return check_launch("stem_pool");
}

} // extern "C"

// The forward pass of every conv algorithm; xs is the input scale of an in_scale plan (or null).
// x_pstride / y_pstride: channel blocks per image of the buffers x and y point into (0: dense, i.e.
// ceil(Cin/4) / ceil(Cout/4)); larger for views into a wider tensor (a channel slice of a concat).
static int conv_forward_impl(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *xs, const void *blob,
                             const void *res, void *y, void *workspace, vkhip_stream_t s, void *pool = nullptr, int64_t x_pstride = 0,
                             int64_t y_pstride = 0, int stages = 7, int *counters = nullptr) {
    if (!d || !plan || !x || !blob || !y) return set_error(VKHIP_ERR_INVALID, "conv_forward: null argument");
    const int64_t cinb = ceil_div(d->Cin, 4), coutb = ceil_div(d->Cout, 4);
    const int64_t xps = x_pstride > 0 ? x_pstride : cinb, yps = y_pstride > 0 ? y_pstride : coutb;
    const bool    dense = xps == cinb && yps == coutb;
    if (xps < cinb || yps < coutb) return set_error(VKHIP_ERR_INVALID, "conv_forward: plane stride below the channel blocks");
    if (!dense && (plan->algo == VKHIP_CONV_WINOGRAD || plan->algo == VKHIP_CONV_DEPTHWISE || d->in_scale ||
                   (plan->tile >= 0 && plan->tile < kNumTiles && kTiles[plan->tile].kind == 4)))
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv_forward_view: views need a GEMM or split-K plan (not the stem tiles), no input scale");
    if (d->has_res < 0 || d->has_res > 2) return set_error(VKHIP_ERR_INVALID, "conv_forward: has_res is 0, 1 or 2");
    if (d->has_res == 2 && (plan->algo == VKHIP_CONV_WINOGRAD || plan->algo == VKHIP_CONV_DEPTHWISE ||
                            (plan->tile >= 0 && plan->tile < kNumTiles && kTiles[plan->tile].kind == 4)))
        return set_error(VKHIP_ERR_UNSUPPORTED, "conv_forward: a residual after the activation needs a GEMM or split-K plan (not the stem tiles)");
    if ((int64_t) d->N * std::max(xps * d->H * d->W, yps * d->OH * d->OW) * 8 >= (1LL << 31))
        return set_error(VKHIP_ERR_INVALID, "conv_forward: view >= 2 GiB");
    if (d->has_res && !res) return set_error(VKHIP_ERR_INVALID, "conv_forward: has_res without a residual tensor");
    if (plan->workspace_bytes && !workspace) return set_error(VKHIP_ERR_INVALID, "conv_forward: plan needs a workspace");
    hipStream_t st = resolve_stream(s);

    if (plan->algo == VKHIP_CONV_DEPTHWISE) {
        DwArgs a;
        int64_t Cb = ceil_div(d->Cin, 4);
        a.x = (const uint2 *) x;
        a.bias = (const float *) blob;
        a.w = (const half4 *) ((const char *) blob + align256((size_t) Cb * 16));
        a.res = (const uint2 *) res;
        a.y = (uint2 *) y;
        a.N = d->N; a.Cb = (int) Cb; a.C = d->Cin; a.H = d->H; a.W = d->W; a.OH = d->OH; a.OW = d->OW;
        a.KH = d->KH; a.KW = d->KW; a.SH = d->SH; a.SW = d->SW; a.PT = d->PT; a.PL = d->PL; a.DH = d->DH; a.DW = d->DW;
        a.act = d->act; a.lo = d->act_lo; a.hi = d->act_hi; a.has_res = d->has_res;
        a.pool = (float4v *) pool;
        bool unit = d->DH == 1 && d->DW == 1 && d->SH == d->SW;
        DwTile t;
        const int RT = plan->tile > 0 ? plan->tile % 100 : (d->OH % 7 == 0 ? 7 : 4);
        if (unit && d->KH == d->KW && (d->KH == 3 || d->KH == 5) && (d->SH == 1 || d->SH == 2) &&
            dw_tile(d, (int64_t) d->N * Cb, RT, std::max(1, plan->tile / 100), t)) {
            const bool   pers = plan->tile >= 900;
            const size_t tile_bytes = (size_t) t.PP * t.PS * 8;
            // the pool reduction reuses the tile, or (persistent groups: the halo must survive) follows it
            const size_t sm = pers ? ((tile_bytes + 15) & ~(size_t) 15) + (pool ? 256 * 16 : 0) : std::max<size_t>(tile_bytes, pool ? 256 * 16 : 0);
            dim3 g2((unsigned) ((int64_t) t.rt_groups * t.plane_groups));
            if (pers) {
                if (!dw_persist_ok(d, t)) return set_error(VKHIP_ERR_INVALID, "conv_forward: depthwise tile %d does not fit this shape", plan->tile);
                g2 = dim3(dw_persist_grid(d, t, sm));
            }
#define VKHIP_DW_LAUNCH(K, S_)                                                                                 \
    (pers ? (RT == 14 ? dwconv_lds_kernel<K, K, S_, 14, 2><<<g2, 256, sm, st>>>(a, t)                                          \
                      : RT == 7 ? dwconv_lds_kernel<K, K, S_, 7, 2><<<g2, 256, sm, st>>>(a, t)                                  \
                                : dwconv_lds_kernel<K, K, S_, 4, 2><<<g2, 256, sm, st>>>(a, t))                                 \
     : t.RPW > 1 ? (RT == 14 ? dwconv_lds_kernel<K, K, S_, 14, 1><<<g2, 256, sm, st>>>(a, t)                                    \
                             : RT == 7 ? dwconv_lds_kernel<K, K, S_, 7, 1><<<g2, 256, sm, st>>>(a, t)                           \
                                       : dwconv_lds_kernel<K, K, S_, 4, 1><<<g2, 256, sm, st>>>(a, t))                          \
                 : (RT == 14 ? dwconv_lds_kernel<K, K, S_, 14, 0><<<g2, 256, sm, st>>>(a, t)                                    \
                             : RT == 7 ? dwconv_lds_kernel<K, K, S_, 7, 0><<<g2, 256, sm, st>>>(a, t)                           \
                                       : dwconv_lds_kernel<K, K, S_, 4, 0><<<g2, 256, sm, st>>>(a, t)))
            if (d->KH == 3 && d->SH == 1) VKHIP_DW_LAUNCH(3, 1);
            else if (d->KH == 3) VKHIP_DW_LAUNCH(3, 2);
            else if (d->SH == 1) VKHIP_DW_LAUNCH(5, 1);
            else VKHIP_DW_LAUNCH(5, 2);
#undef VKHIP_DW_LAUNCH
            return check_launch("dwconv_lds");
        }
        if (pool) return set_error(VKHIP_ERR_UNSUPPORTED, "conv_forward_pooled: the plan does not run the tiled depthwise kernel");
        constexpr int OXT = 4;
        int64_t total = (int64_t) d->N * Cb * d->OH * ceil_div(d->OW, OXT);
        dim3 grid((unsigned) ceil_div(total, 256));
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
    a.x_pstride = (int) g.Cinb;
    a.y_pstride = (int) g.Coutb;
    a.Pv     = (int) g.Pv;
    a.OHWp   = (int) g.HWp;
    a.Kslots = (int) g.Kslots;
    a.nsteps = (int) g.nsteps;
    a.steps_per_split = (int) g.nsteps;
    a.act    = d->act;
    a.lo     = d->act_lo;
    a.hi     = d->act_hi;
    a.m_tiles = (int) g.m_tiles;
    const bool split       = plan->algo == VKHIP_CONV_SPLITK || plan->algo == VKHIP_CONV_SPLITK_LAST;
    const int  split_steps = split ? (int) ceil_div(g.nsteps, plan->ksplit) : (int) g.nsteps;
    GemmKernelFn fn = gemm_kernel_for(plan->tile, g.bmode, split_steps,
                                      t.kind == 3 ? halo_nbi(d, t) * (d->W % 2 ? -1 : 1) : (t.kind == 4 ? stem_nbi(d, t) : 0), d->in_scale != 0);
    if (!fn && t.kind != 5) return set_error(VKHIP_ERR_INVALID, "conv_forward: no kernel for tile %d", plan->tile);

    if (wino) {
        const int nTH = (int) ceil_div(d->OH, 2), nTW = (int) ceil_div(d->OW, 2);
        const int nT  = (int) g.P;
        uint2    *V   = (uint2 *) workspace;
        uint2    *M   = (uint2 *) ((char *) workspace + align256((size_t) 16 * g.Cinb * nT * 8));
        int64_t   nin = g.Cinb * nT;
        int rc = 0;
        if (stages & 1) {
            wino_input_kernel<<<dim3((unsigned) ceil_div(nin, 256)), 256, 0, st>>>((const uint2 *) x, V, (int) g.Cinb, d->H, d->W, nTH, nTW, nT);
            if ((rc = check_launch("wino_input"))) return rc;
        }
        a.x = V;
        a.x_bytes = (unsigned) (g.Cinb * nT * 8);
        a.y_bytes = (unsigned) (g.Coutb * nT * 8);
        a.y = M;
        a.H = 1; a.W = nT; a.HW = nT;
        a.OW = nT; a.OHW = nT;
        a.KW = 1; a.SH = 1; a.SW = 1; a.DH = 1; a.DW = 1;
        a.omode     = OMODE_RAW;
        a.x_bstride = (long long) g.Cinb * nT;
        a.w_bstride = (long long) g.Coutp * g.Kp;
        a.y_bstride = (long long) g.Coutb * nT;
        dim3 grid((unsigned) (g.m_tiles * g.n_tiles), 1, 16);
        if (stages & 2) {
            fn<<<grid, 64 * t.WM * t.WN, 0, st>>>(a);
            if ((rc = check_launch("wino_gemm"))) return rc;
        }
        if (!(stages & 4)) return VKHIP_OK;
        int64_t nout = g.Coutb * nT;
        wino_output_kernel<<<dim3((unsigned) ceil_div(nout, 256)), 256, 0, st>>>(M, a.bias, d->has_res ? (const uint2 *) res : nullptr, (uint2 *) y,
                                                                               (int) g.Coutb, d->Cout, d->OH, d->OW,
                                                                               nTH, nTW, nT, d->act, d->act_lo, d->act_hi);
        return check_launch("wino_output");
    }

    a.x  = (const uint2 *) x;
    a.xs = (const uint2 *) xs;
    a.xs_bytes = (unsigned) ((int64_t) d->N * g.Cinb * 8);
    a.x_bytes = (unsigned) (((int64_t) (d->N - 1) * xps + g.Cinb) * d->H * d->W * 8);
    a.y_bytes = (unsigned) (((int64_t) (d->N - 1) * yps + g.Coutb) * d->OH * d->OW * 8);
    a.x_pstride = (int) xps;
    a.y_pstride = (int) yps;
    a.y  = (uint2 *) y;
    a.res = (const uint2 *) res;
    a.has_res = d->has_res;
    a.H  = d->H; a.W = d->W; a.HW = d->H * d->W;
    a.OW = d->OW; a.OHW = d->OH * d->OW;
    a.KW = d->KW; a.SH = d->SH; a.SW = d->SW; a.PT = d->PT; a.PL = d->PL; a.DH = d->DH; a.DW = d->DW;
    if (split) {
        int ks = plan->ksplit;
        a.steps_per_split = (int) ceil_div(g.nsteps, ks);
        ks = (int) ceil_div(g.nsteps, a.steps_per_split);
        a.omode = OMODE_PARTIAL;
        a.part  = (float4v *) workspace;
        if (plan->algo == VKHIP_CONV_SPLITK_LAST) {
            // the last workgroup of each tile sums the partials: counters after them, zero between calls
            a.cnt = counters ? counters : (int *) ((char *) workspace + align256((size_t) plan->ksplit * g.Coutb * g.P * 16));
        }
        dim3 grid((unsigned) (g.m_tiles * g.n_tiles), (unsigned) ks, 1);
        fn<<<grid, 64 * t.WM * t.WN, 0, st>>>(a);
        int rc = check_launch("conv_gemm_splitk");
        if (rc || plan->algo == VKHIP_CONV_SPLITK_LAST) return rc;
        int64_t total = g.Coutb * g.P;
        splitk_reduce_kernel<<<dim3((unsigned) ceil_div(total, 256)), 256, 0, st>>>(
            (const float4v *) workspace, a.bias, a.res, a.y, ks, (int) g.Coutb, d->Cout, (int) g.P, a.OHW, d->act, d->act_lo,
            d->act_hi, d->has_res, (int) yps);
        return check_launch("splitk_reduce");
    }
    a.omode   = OMODE_EPILOGUE;
    a.n_tiles = (int) g.n_tiles;
    if (t.kind == 5) {
        GemmKernelFn tf = thin_kernel_for((int) g.Cinb, t.FM, d->KH, d->SH, d->has_res != 0);
        if (!tf) return set_error(VKHIP_ERR_INVALID, "conv_forward: no thin kernel for this shape");
        const int64_t items = (int64_t) d->N * ceil_div(d->OH, 4) * ceil_div(d->OW, 64);
        // as many workgroups as the device holds at once: the items are short, so concurrency,
        // not the per-workgroup pipeline, hides most of the load latency (measured: one or two
        // workgroups per CU run 1.2-2x slower than full occupancy)
        dim3 grid((unsigned) std::min<int64_t>(persist_grid(tf, 256, items), items), 1, 1);
        // XCD-contiguous item ranges on 3x3 stride 1, where vertically adjacent items share a third
        // of their input rows (16x16 3x3 at 160x160, b16: 12.3 -> 11.4 us); the strided walk
        // elsewhere (stride 2 and 1x1 bands barely overlap, and there it measured 1-3% faster).
        // VKHIP_THIN_ORDER=0: the strided walk everywhere (A/B).
        static const bool xcd_order = !(std::getenv("VKHIP_THIN_ORDER") && std::getenv("VKHIP_THIN_ORDER")[0] == '0');
        a.item_order = xcd_order && d->KH == 3 && d->SH == 1;
        tf<<<grid, 256, 0, st>>>(a);
        return check_launch("conv_thin");
    }
    if (t.PERS) {
        const int threads = 64 * (t.WM * t.WN + kProducers);
        dim3      grid(persist_grid(fn, threads, g.m_tiles * g.n_tiles), 1, 1);
        fn<<<grid, threads, 0, st>>>(a);
        return check_launch("conv_gemm_persist");
    }
    dim3 grid((unsigned) (g.m_tiles * g.n_tiles), 1, 1);
    fn<<<grid, 64 * t.WM * t.WN, 0, st>>>(a);
    return check_launch("conv_gemm");
}

extern "C" {

int vkhip_conv_forward(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                       void *y, void *workspace, vkhip_stream_t s) {
    if (d && d->in_scale) return set_error(VKHIP_ERR_INVALID, "conv_forward: an in_scale plan runs through vkhip_conv_forward_scaled");
    return conv_forward_impl(d, plan, x, nullptr, blob, res, y, workspace, s);
}

int vkhip_conv_forward_stages(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                              void *y, void *workspace, int stages, vkhip_stream_t s) {
    if (!plan || stages < 1 || stages > 7) return set_error(VKHIP_ERR_INVALID, "conv_forward_stages: stages is a mask of 1..7");
    if (plan->algo != VKHIP_CONV_WINOGRAD && stages != 7)
        return set_error(VKHIP_ERR_INVALID, "conv_forward_stages: only a Winograd plan runs part of its stages");
    if (d && d->in_scale) return set_error(VKHIP_ERR_INVALID, "conv_forward_stages: no input-scale plans");
    return conv_forward_impl(d, plan, x, nullptr, blob, res, y, workspace, s, nullptr, 0, 0, stages);
}

int vkhip_conv_forward_view(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, int64_t x_pstride, const void *blob, void *y,
                            int64_t y_pstride, void *workspace, vkhip_stream_t s) {
    if (d && d->in_scale) return set_error(VKHIP_ERR_INVALID, "conv_forward_view: no input-scale plans");
    if (d && d->has_res) return set_error(VKHIP_ERR_INVALID, "conv_forward_view: a residual conv runs vkhip_conv_forward_view_res");
    return conv_forward_impl(d, plan, x, nullptr, blob, nullptr, y, workspace, s, nullptr, x_pstride, y_pstride);
}

int vkhip_conv_forward_view_res(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, int64_t x_pstride, const void *blob,
                                const void *res, void *y, int64_t y_pstride, void *workspace, vkhip_stream_t s) {
    if (d && d->in_scale) return set_error(VKHIP_ERR_INVALID, "conv_forward_view_res: no input-scale plans");
    return conv_forward_impl(d, plan, x, nullptr, blob, res, y, workspace, s, nullptr, x_pstride, y_pstride);
}

int vkhip_conv_pool_parts(const vkhip_conv_desc *d, const vkhip_conv_plan *plan) {
    if (!d || !plan || plan->algo != VKHIP_CONV_DEPTHWISE || d->in_scale) return 0;
    const bool unit = d->DH == 1 && d->DW == 1 && d->SH == d->SW;
    const int  RT   = plan->tile > 0 ? plan->tile % 100 : (d->OH % 7 == 0 ? 7 : 4);
    DwTile     t;
    if (!(unit && d->KH == d->KW && (d->KH == 3 || d->KH == 5) && (d->SH == 1 || d->SH == 2) &&
          dw_tile(d, (int64_t) d->N * ceil_div(d->Cin, 4), RT, std::max(1, plan->tile / 100), t)))
        return 0;
    return t.row_tiles;
}

int vkhip_conv_forward_pooled(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                              void *y, void *pool, vkhip_stream_t s) {
    if (!pool || vkhip_conv_pool_parts(d, plan) <= 0) return set_error(VKHIP_ERR_UNSUPPORTED, "conv_forward_pooled: needs a tiled depthwise plan and a pool buffer");
    return conv_forward_impl(d, plan, x, nullptr, blob, res, y, nullptr, s, pool);
}

int vkhip_conv_forward_scaled(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *xs, const void *blob,
                              const void *res, void *y, void *workspace, vkhip_stream_t s) {
    if (!d || !xs || !d->in_scale) return set_error(VKHIP_ERR_INVALID, "conv_forward_scaled: needs an in_scale plan and a scale tensor");
    return conv_forward_impl(d, plan, x, xs, blob, res, y, workspace, s);
}

int vkhip_conv_forward_noalloc(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob,
                               const void *res, void *y, vkhip_stream_t s) {
    if (!d || !plan) return set_error(VKHIP_ERR_INVALID, "conv_forward_noalloc: null argument");
    // The scratch is a fixed array next to other module globals: size it from the descriptor, not
    // from the caller's plan, so a plan made for another shape cannot make a kernel write past it.
    vkhip_conv_plan fresh;
    if (vkhip_conv_plan_make(d, plan->algo, plan->tile, plan->ksplit, &fresh) != VKHIP_OK)
        return set_error(VKHIP_ERR_INVALID, "conv_forward_noalloc: the plan does not fit the descriptor");
    if (fresh.workspace_bytes != plan->workspace_bytes || fresh.weight_bytes != plan->weight_bytes)
        return set_error(VKHIP_ERR_INVALID, "conv_forward_noalloc: the plan's sizes (workspace %zu, weights %zu) differ from the "
                         "descriptor's (%zu, %zu)", plan->workspace_bytes, plan->weight_bytes, fresh.workspace_bytes, fresh.weight_bytes);
    if (plan->workspace_bytes > VKHIP_NOALLOC_SCRATCH_BYTES)
        return set_error(VKHIP_ERR_INVALID, "conv_forward_noalloc: the plan needs %zu bytes of workspace, more than the %zu-byte scratch",
                         plan->workspace_bytes, (size_t) VKHIP_NOALLOC_SCRATCH_BYTES);
    if (plan->algo == VKHIP_CONV_SPLITK_LAST) {
        const ConvGeom g = gemm_geom(d, plan->tile, false);
        if (g.m_tiles * g.n_tiles > VKHIP_NOALLOC_MAX_TILES)
            return set_error(VKHIP_ERR_INVALID, "conv_forward_noalloc: the plan has %lld output tiles, more than the %d arrival counters",
                             (long long) (g.m_tiles * g.n_tiles), VKHIP_NOALLOC_MAX_TILES);
    }
    void *ws  = nullptr;
    int  *cnt = nullptr;
    if (plan->workspace_bytes) {
        int rc = vkhip_init();
        if (rc) return rc;
        if ((rc = scratch_ptr(&ws, &cnt))) return rc;
    }
    if (d->in_scale) return set_error(VKHIP_ERR_INVALID, "conv_forward: an in_scale plan runs through vkhip_conv_forward_scaled");
    return conv_forward_impl(d, plan, x, nullptr, blob, res, y, ws, s, nullptr, 0, 0, 7, cnt);
}

} // extern "C"

// ---------------------------------------------------------------------- fused 3x3 + 1x1
namespace vkhip {

    // The fused kernel's tile for a mid width: its halo geometry (the 3x3 weights are packed like
    // the halo tile with the same BM and KK, which fixes the A layout) and the 1x1 chunking.
    struct PwTile {
        int     halo_tile; // kTiles entry whose A layout the 3x3 weights use (BM = mid width, KK = 1)
        TileCfg t;         // the fused workgroup: BM = mid width, WM = 1, WN = 4
        int     MC;        // 32-row 1x1 fragments per chunk
    };
    static bool pw_tile(int cmid, PwTile &p) {
        if (cmid != 64) return false;
        p = {18, {64, 256, 1, 4, 3, 2, 2, 1}, 1};
        return true;
    }
    static constexpr int kPwMaxNBI64 = 15;

    // 1x1 parts of the blob, after the 3x3 plan's weight bytes: bias [nchunks * 32 * MC] fp32, then
    // the weights [nchunks * MC fragments][2 * FM steps][64 lanes][8 halves]
    struct PwLayout {
        size_t  w3_bytes, off_b1, off_w1, bytes;
        int64_t nchunks, frags, steps;
    };
    static PwLayout pw_layout(const vkhip_convpw_desc *d, const PwTile &pt, size_t w3_bytes) {
        PwLayout L;
        L.w3_bytes = w3_bytes;
        L.nchunks  = ceil_div(d->Cout, 32 * pt.MC);
        L.frags    = L.nchunks * pt.MC;
        L.steps    = 2 * (d->conv.Cout / 32);
        L.off_b1   = align256(w3_bytes);
        L.off_w1   = L.off_b1 + align256((size_t) L.frags * 32 * 4);
        L.bytes    = L.off_w1 + (size_t) L.frags * L.steps * 1024;
        return L;
    }

    static int pw_check(const vkhip_convpw_desc *d, PwTile &pt, vkhip_conv_plan &p3) {
        if (!d) return set_error(VKHIP_ERR_INVALID, "convpw: null descriptor");
        const vkhip_conv_desc &c = d->conv;
        if (!pw_tile(c.Cout, pt)) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw: mid width %d (64 only)", c.Cout);
        if (c.has_res || c.in_scale || c.N <= 0 || d->Cout <= 0 || c.W % 2) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw: 3x3 with a residual, an input scale or odd width");
        if (!halo_shape_ok(&c, pt.t)) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw: not a halo-tile 3x3 (pad 1, stride 1/2, Cin %% 16 == 0)");
        const int nbi = halo_nbi(&c, pt.t);
        int       lds = 0;
        if (nbi > kPwMaxNBI64 || !pw_tile_kernel(c.Cout, nbi, 0, &lds))
            return set_error(VKHIP_ERR_UNSUPPORTED, "convpw: input band too large for LDS");
        // the 1x1 weights and bias are staged in the kernel's LDS ring
        const int64_t nch = ceil_div(d->Cout, 32 * pt.MC);
        if ((nch * pt.MC * 2 * (c.Cout / 32) + ceil_div(nch * pt.MC * 32 * 4, 1024)) * 1024 > lds)
            return set_error(VKHIP_ERR_UNSUPPORTED, "convpw: 1x1 weights do not fit the kernel's LDS");
        const int64_t P = (int64_t) c.N * c.OH * c.OW;
        if (P * ceil_div(std::max(c.Cin, d->Cout), 4) * 8 >= (1LL << 31) || (int64_t) c.N * ceil_div(c.Cin, 4) * c.H * c.W * 8 >= (1LL << 31))
            return set_error(VKHIP_ERR_UNSUPPORTED, "convpw: tensor >= 2 GiB");
        // the 3x3 part is packed like a GEMM plan of the halo tile with the same A layout (the band
        // limit that tile's own kernels have does not apply: the fused kernel checked its own above)
        const ConvGeom g = gemm_geom(&c, pt.halo_tile, false);
        std::memset(&p3, 0, sizeof(p3));
        p3.algo         = VKHIP_CONV_GEMM;
        p3.tile         = pt.halo_tile;
        p3.weight_bytes = align256((size_t) g.Coutp * 4) + (size_t) g.Coutp * g.Kp * 2;
        return VKHIP_OK;
    }

    // The chained second 1x1 (vkhip_convpw2_*): after the pair's blob, its bias [32 * MR] fp32 and
    // weights [MR fragments][2 * nchunks steps][64][8 halves].
    struct PwChain {
        PwLayout pair;
        int      MR;
        size_t   off_b2, off_w2, bytes;
    };
    static int pw_chain(const vkhip_convpw2_desc *d, const PwTile &pt, const vkhip_conv_plan &p3, PwChain &ch) {
        if (d->pw.conv.Cout != 64 || pt.MC != 1 || d->Cout3 <= 0 || d->Cout3 > 64)
            return set_error(VKHIP_ERR_UNSUPPORTED, "convpw2: the chained 1x1 needs 64 mid channels and at most 64 outputs");
        ch.pair = pw_layout(&d->pw, pt, p3.weight_bytes);
        ch.MR   = (int) ceil_div(d->Cout3, 32);
        int lds = 0;
        if (!pw_tile_kernel(64, halo_nbi(&d->pw.conv, pt.t), ch.MR, &lds)) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw2: no chained kernel for this band");
        const int64_t kb = ch.pair.frags * ch.pair.steps + ceil_div(ch.pair.frags * 32 * 4, 1024) + ch.MR * 2 * ch.pair.nchunks + 1;
        if (kb * 1024 > lds) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw2: weights do not fit the kernel's LDS");
        ch.off_b2 = align256(ch.pair.bytes);
        ch.off_w2 = ch.off_b2 + align256((size_t) ch.MR * 32 * 4);
        ch.bytes  = ch.off_w2 + (size_t) ch.MR * 2 * ch.pair.nchunks * 1024;
        return VKHIP_OK;
    }

    static int convpw_forward_impl(const vkhip_convpw_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                                   void *y, const vkhip_convpw2_desc *d2, void *y2, vkhip_stream_t s) {
        if (!plan || !x || !blob || !y) return set_error(VKHIP_ERR_INVALID, "convpw_forward: null argument");
        PwTile          pt;
        vkhip_conv_plan p3;
        int rc = pw_check(d, pt, p3);
        if (rc) return rc;
        const PwLayout L = pw_layout(d, pt, p3.weight_bytes);
        PwChain        ch {};
        if (d2 && (rc = pw_chain(d2, pt, p3, ch))) return rc;
        if (plan->weight_bytes != (d2 ? ch.bytes : L.bytes)) return set_error(VKHIP_ERR_INVALID, "convpw_forward: plan does not match the descriptor");
        if (d->has_res && !res) return set_error(VKHIP_ERR_INVALID, "convpw_forward: has_res without a residual tensor");
        if (d->has_res > 1) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw_forward: the residual is added before the activation only");
        const vkhip_conv_desc &c = d->conv;
        const int              nbi = halo_nbi(&c, pt.t);
        PwKernelFn             fn  = pw_tile_kernel(c.Cout, nbi, d2 ? ch.MR : 0, nullptr);
        if (!fn) return set_error(VKHIP_ERR_UNSUPPORTED, "convpw_forward: no kernel for band %d", nbi);
        ConvGeom g = gemm_geom(&c, pt.halo_tile, false);
        GemmArgs a;
        std::memset(&a, 0, sizeof(a));
        a.x = (const uint2 *) x;
        a.w = (const half_t *) ((const char *) blob + align256((size_t) g.Coutp * 4));
        a.bias = (const float *) blob;
        a.Cinb = (int) g.Cinb; a.Coutb = (int) g.Coutb; a.Cout = c.Cout;
        a.P = (int) g.P; a.Pv = (int) g.Pv; a.OHWp = (int) g.HWp;
        a.Kslots = (int) g.Kslots; a.nsteps = (int) g.nsteps; a.steps_per_split = (int) g.nsteps;
        a.act = c.act; a.lo = c.act_lo; a.hi = c.act_hi;
        a.m_tiles = 1;
        a.x_pstride = (int) g.Cinb; a.y_pstride = (int) g.Coutb;
        a.x_bytes = (unsigned) ((int64_t) c.N * g.Cinb * c.H * c.W * 8);
        a.H = c.H; a.W = c.W; a.HW = c.H * c.W; a.OW = c.OW; a.OHW = c.OH * c.OW;
        a.KW = c.KW; a.SH = c.SH; a.SW = c.SW; a.PT = c.PT; a.PL = c.PL; a.DH = c.DH; a.DW = c.DW;
        a.omode = OMODE_EPILOGUE;
        PwArgs p;
        std::memset(&p, 0, sizeof(p));
        p.w       = (const half_t *) ((const char *) blob + L.off_w1);
        p.nchunks = (int) L.nchunks;
        GemmArgs &e = p.e;
        const int64_t Coutb = ceil_div(d->Cout, 4), OHW = (int64_t) c.OH * c.OW;
        e.bias = (const float *) ((const char *) blob + L.off_b1);
        e.res = (const uint2 *) res; e.has_res = d->has_res;
        e.y = (uint2 *) y;
        e.Cout = d->Cout; e.Coutb = (int) Coutb;
        e.P = (int) g.P; e.Pv = (int) g.P; e.OHW = (int) OHW; e.OHWp = (int) OHW; e.OW = c.OW;
        e.y_pstride = (int) Coutb;
        e.y_bytes = (unsigned) ((int64_t) c.N * Coutb * OHW * 8);
        e.act = d->act; e.lo = d->act_lo; e.hi = d->act_hi;
        e.omode = OMODE_EPILOGUE;
        e.m_tiles = 1;
        if (d2) {
            p.w3     = (const half_t *) ((const char *) blob + ch.off_w2);
            p.bias3  = (const float *) ((const char *) blob + ch.off_b2);
            p.y3     = (uint2 *) y2;
            p.Cout3  = d2->Cout3;
            p.Coutb3 = (int) ceil_div(d2->Cout3, 4);
            p.act3   = d2->act3; p.lo3 = d2->act3_lo; p.hi3 = d2->act3_hi;
            p.y3_bytes = (unsigned) ((int64_t) c.N * p.Coutb3 * OHW * 8);
        }
        const unsigned grid = (unsigned) ceil_div(g.P, pt.t.BN);
        fn<<<dim3(grid), 64 * pt.t.WN, 0, resolve_stream(s)>>>(a, p);
        return check_launch(d2 ? "convpw2" : "convpw");
    }

} // namespace vkhip

extern "C" {

int vkhip_convpw_plan(const vkhip_convpw_desc *d, vkhip_conv_plan *plan) {
    if (!plan) return set_error(VKHIP_ERR_INVALID, "convpw_plan: null plan");
    PwTile          pt;
    vkhip_conv_plan p3;
    int rc = pw_check(d, pt, p3);
    if (rc) return rc;
    *plan              = p3;
    plan->weight_bytes = pw_layout(d, pt, p3.weight_bytes).bytes;
    plan->workspace_bytes = 0;
    return VKHIP_OK;
}

int vkhip_convpw_pack_weights(const vkhip_convpw_desc *d, const vkhip_conv_plan *plan, const float *w3, const float *b3, const float *w1,
                              const float *b1, void *blob) {
    if (!plan || !w3 || !w1 || !blob) return set_error(VKHIP_ERR_INVALID, "convpw_pack: null argument");
    PwTile          pt;
    vkhip_conv_plan p3;
    int rc = pw_check(d, pt, p3);
    if (rc) return rc;
    const PwLayout L = pw_layout(d, pt, p3.weight_bytes);
    if (plan->weight_bytes != L.bytes) return set_error(VKHIP_ERR_INVALID, "convpw_pack: plan does not match the descriptor");
    std::memset(blob, 0, L.bytes);
    if ((rc = vkhip_conv_pack_weights(&d->conv, &p3, w3, b3, blob))) return rc;
    float  *bias = (float *) ((char *) blob + L.off_b1);
    half_t *wp   = (half_t *) ((char *) blob + L.off_w1);
    const int Cmid = d->conv.Cout;
    if (b1)
        for (int m = 0; m < d->Cout; ++m) bias[m] = b1[m];
    // fragment f, step s = 2i + h, lane l = g*32 + row%32, entry t: channel i*32 + (2h + t/4)*8 + 4g + t%4
    for (int64_t f = 0; f < L.frags; ++f)
        for (int64_t s = 0; s < L.steps; ++s)
            for (int l = 0; l < 64; ++l)
                for (int t = 0; t < 8; ++t) {
                    const int64_t m = f * 32 + (l & 31);
                    const int     i = (int) (s / 2), h = (int) (s % 2), g = l >> 5;
                    const int     ch = i * 32 + (2 * h + t / 4) * 8 + 4 * g + t % 4;
                    if (m < d->Cout) wp[((f * L.steps + s) * 64 + l) * 8 + t] = ref_half(w1[m * Cmid + ch]);
                }
    return VKHIP_OK;
}

int vkhip_convpw_forward(const vkhip_convpw_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res, void *y,
                         vkhip_stream_t s) {
    return convpw_forward_impl(d, plan, x, blob, res, y, nullptr, nullptr, s);
}

int vkhip_convpw2_plan(const vkhip_convpw2_desc *d, vkhip_conv_plan *plan) {
    if (!d || !plan) return set_error(VKHIP_ERR_INVALID, "convpw2_plan: null argument");
    PwTile          pt;
    vkhip_conv_plan p3;
    int rc = pw_check(&d->pw, pt, p3);
    if (rc) return rc;
    PwChain ch;
    if ((rc = pw_chain(d, pt, p3, ch))) return rc;
    *plan                 = p3;
    plan->weight_bytes    = ch.bytes;
    plan->workspace_bytes = 0;
    return VKHIP_OK;
}

int vkhip_convpw2_pack_weights(const vkhip_convpw2_desc *d, const vkhip_conv_plan *plan, const float *w3, const float *b3, const float *w1,
                               const float *b1, const float *w2, const float *b2, void *blob) {
    if (!d || !plan || !w2 || !blob) return set_error(VKHIP_ERR_INVALID, "convpw2_pack: null argument");
    PwTile          pt;
    vkhip_conv_plan p3;
    int rc = pw_check(&d->pw, pt, p3);
    if (rc) return rc;
    PwChain ch;
    if ((rc = pw_chain(d, pt, p3, ch))) return rc;
    if (plan->weight_bytes != ch.bytes) return set_error(VKHIP_ERR_INVALID, "convpw2_pack: plan does not match the descriptor");
    vkhip_conv_plan pp = *plan;
    pp.weight_bytes    = ch.pair.bytes;
    if ((rc = vkhip_convpw_pack_weights(&d->pw, &pp, w3, b3, w1, b1, blob))) return rc;
    std::memset((char *) blob + ch.pair.bytes, 0, ch.bytes - ch.pair.bytes);
    float  *bias = (float *) ((char *) blob + ch.off_b2);
    half_t *wp   = (half_t *) ((char *) blob + ch.off_w2);
    const int K2 = d->pw.Cout; // the chained 1x1 reads the pair's output channels
    if (b2)
        for (int m = 0; m < d->Cout3; ++m) bias[m] = b2[m];
    // fragment m, step s = 2c + h (chunk c of the pair's output), lane l = g*32 + row%32, entry t:
    // channel c*32 + (2h + t/4)*8 + 4g + t%4 (the order the pair's stored chunk holds them in)
    for (int m = 0; m < ch.MR; ++m)
        for (int64_t st = 0; st < 2 * ch.pair.nchunks; ++st)
            for (int l = 0; l < 64; ++l)
                for (int t = 0; t < 8; ++t) {
                    const int64_t row = m * 32 + (l & 31);
                    const int     c = (int) (st / 2), h = (int) (st % 2), g = l >> 5;
                    const int     k = c * 32 + (2 * h + t / 4) * 8 + 4 * g + t % 4;
                    if (row < d->Cout3 && k < K2) wp[((m * 2 * ch.pair.nchunks + st) * 64 + l) * 8 + t] = ref_half(w2[row * K2 + k]);
                }
    return VKHIP_OK;
}

int vkhip_convpw2_forward(const vkhip_convpw2_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res, void *y,
                          void *y2, vkhip_stream_t s) {
    if (!d || !y2) return set_error(VKHIP_ERR_INVALID, "convpw2_forward: null argument");
    return convpw_forward_impl(&d->pw, plan, x, blob, res, y, d, y2, s);
}

} // extern "C"
