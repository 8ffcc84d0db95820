// Fused depthwise + 1x1 project on gfx950 (reference FusedDwPw: src/backend/cpu/ops/fused_dwpw.cpp
// :10-87, shaders/fused_dwpw_fp16.comp). One workgroup owns BN consecutive output pixels and all E
// expanded channels:
//   phase 1  depthwise KHxKW + bias + dw activation for E channels x BN pixels, written to LDS as
//            fp16 in the MFMA B-operand layout (the E-channel intermediate never touches HBM);
//   phase 2  the 1x1 projection as MFMA 32x32x16 GEMMs (A = packed pw weights streamed from L2,
//            B = the LDS tile), then bias (+ residual) + activation and the fp16 NC4HW4 store.
// Also hosts the fully-connected helper (a 1x1 conv over [N,K,1,1]).
#include "common.h"
#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace vkhip {

    struct DwPwArgs {
        const uint2  *x;
        const float  *dw_b;  // [Eb*4]
        const float  *dw_w;  // [Eb][KH][KW][4]
        const float  *pw_b;  // [Coutp]
        const half_t *pw_w;  // [Coutp][Kp]
        const uint2  *res;
        uint2        *y;
        int           N, E, Eb, Ebp, H, W, OH, OW, KH, KW, SH, SW, PT, PL, DH, DW;
        int           dw_act;
        int           Cout, Coutb, m_frags, Kp, P;
        int           act;
        float         lo, hi;
        int           has_res;
    };

    template <int BN>
    __global__ __launch_bounds__(256) void dwpw_kernel(DwPwArgs a) {
        extern __shared__ uint4 lds[]; // [Ebp/2 slot pairs][BN] x 16 bytes
        const int tid = threadIdx.x;
        const int n0  = blockIdx.x * BN;

        // ---- phase 1: depthwise into LDS
        const int items = a.Ebp * BN;
        for (int it = tid; it < items; it += 256) {
            const int cb = it / BN;
            const int pl = it - cb * BN;
            const int p  = n0 + pl;
            float4v   v  = {0.f, 0.f, 0.f, 0.f};
            if (cb < a.Eb && p < a.P) {
                int n  = p / (a.OH * a.OW);
                int r  = p - n * a.OH * a.OW;
                int oy = r / a.OW;
                int ox = r - oy * a.OW;
                v      = *reinterpret_cast<const float4v *>(a.dw_b + cb * 4);
                const uint2   *src = a.x + ((long long) n * a.Eb + cb) * a.H * a.W;
                const float4v *wv  = reinterpret_cast<const float4v *>(a.dw_w) + (long long) cb * a.KH * a.KW;
                for (int ky = 0; ky < a.KH; ++ky) {
                    int iy = oy * a.SH - a.PT + ky * a.DH;
                    if (iy < 0 || iy >= a.H) continue;
                    for (int kx = 0; kx < a.KW; ++kx) {
                        int ix = ox * a.SW - a.PL + kx * a.DW;
                        if (ix < 0 || ix >= a.W) continue;
                        v += h4_to_f4(u2_as_h4(src[iy * a.W + ix])) * wv[ky * a.KW + kx];
                    }
                }
                v.x = apply_act(v.x, a.dw_act, 0.f, 6.f);
                v.y = apply_act(v.y, a.dw_act, 0.f, 6.f);
                v.z = apply_act(v.z, a.dw_act, 0.f, 6.f);
                v.w = apply_act(v.w, a.dw_act, 0.f, 6.f);
                int c = cb * 4;
                if (c + 0 >= a.E) v.x = 0.f;
                if (c + 1 >= a.E) v.y = 0.f;
                if (c + 2 >= a.E) v.z = 0.f;
                if (c + 3 >= a.E) v.w = 0.f;
            }
            reinterpret_cast<uint2 *>(&lds[(cb >> 1) * BN + pl])[cb & 1] = h4_as_u2(f4_to_h4(v));
        }
        __syncthreads();

        // ---- phase 2: projection GEMM, work = m_frags x (BN/32) fragments spread over 4 waves
        const int lane = tid & 63, wave = tid >> 6;
        const int lrow = lane & 31, lk = lane >> 5;
        constexpr int NF = BN / 32;
        const int nwork = a.m_frags * NF;
        const int ksteps = a.Kp / 16;
        for (int wk = wave; wk < nwork; wk += 4) {
            const int mf = wk / NF, nf = wk - (wk / NF) * NF;
            float16v  acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = 0.f;
            const half_t *wrow = a.pw_w + (long long) (mf * 32 + lrow) * a.Kp + lk * 8;
            for (int k = 0; k < ksteps; ++k) {
                half8 af = *reinterpret_cast<const half8 *>(wrow + k * 16);
                half8 bf = *reinterpret_cast<const half8 *>(&lds[(k * 2 + lk) * BN + nf * 32 + lrow]);
                acc      = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
            }
            const int px = n0 + nf * 32 + lrow;
            if (px >= a.P) continue;
            const int OHW = a.OH * a.OW;
            const int pn = px / OHW, pr = px - pn * OHW;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int oc  = mf * 32 + q * 8 + lk * 4;
                const int ocb = oc >> 2;
                if (ocb >= a.Coutb) continue;
                float4v v = {acc[q * 4 + 0], acc[q * 4 + 1], acc[q * 4 + 2], acc[q * 4 + 3]};
                v += *reinterpret_cast<const float4v *>(a.pw_b + oc);
                const long long yi = ((long long) pn * a.Coutb + ocb) * OHW + pr;
                if (a.has_res) v += h4_to_f4(u2_as_h4(a.res[yi]));
                v.x = apply_act(v.x, a.act, a.lo, a.hi);
                v.y = apply_act(v.y, a.act, a.lo, a.hi);
                v.z = apply_act(v.z, a.act, a.lo, a.hi);
                v.w = apply_act(v.w, a.act, a.lo, a.hi);
                if (oc + 0 >= a.Cout) v.x = 0.f;
                if (oc + 1 >= a.Cout) v.y = 0.f;
                if (oc + 2 >= a.Cout) v.z = 0.f;
                if (oc + 3 >= a.Cout) v.w = 0.f;
                a.y[yi] = h4_as_u2(f4_to_h4(v));
            }
        }
    }

    // Strip-tiled fused dw + pw: a workgroup owns RT whole output rows of one image (BN = RT * OW
    // pixels, contiguous in every NC4HW4 plane) and walks the E expanded channels in chunks of CB
    // channel blocks (CB/4 16-deep MFMA K steps; CB * OW <= 256, so each thread owns one
    // (channel block, output column) of a chunk — two when OW > 64):
    //   1. the chunk's input rows ((RT-1)*S + K of them, zero columns left and right) and the
    //      chunk's slice of the packed projection weights are copied into LDS, each thread issuing
    //      all of its loads before its first LDS write, so a chunk costs one memory latency and
    //      every input pixel is read from L2 once per workgroup; the thread's depthwise weights go
    //      to registers as fp16;
    //   2. the thread walks the IR input rows of its column once, K taps per row, adding each into
    //      the RT output rows it feeds (RT independent fp32 accumulators, v_fma_mix with fp16
    //      operands), then applies bias and the dw activation and stores the RT outputs as fp16
    //      into an LDS chunk laid out as MFMA B fragments (16-byte channel-block pairs per pixel);
    //   3. each wave accumulates the projection of its 32-pixel fragments over the chunk's K steps
    //      with v_mfma_f32_32x32x16_f16, A and B from LDS.
    // The E-channel intermediate lives only in LDS. After the last chunk the epilogue adds bias (+
    // residual), applies the activation and stores fp16 NC4HW4.
    //   K: kernel size (3 or 5, square), S: stride (1 or 2), MF: 32-row output fragments (Cout <=
    //   32 * MF <= 64), RT: output rows per strip (BN = RT * OW <= 256, two pixel fragments per wave).
    struct DwStrip {
        int BN, IWp, PLA, NF, CB;
    };

    // LDS of one chunk: [A: MF*32 rows x CB/2 16-byte k groups | dw weights: CB x K*K float4 |
    // dw bias: CB float4][B chunk: CB/2 pairs x NF*32 pixels x 16 B][input: CB planes x IR rows x
    // IWp x 8 B]
    __host__ __device__ inline size_t dwpw_strip_a_bytes(int MF, int K, const DwStrip &t) {
        return (size_t) MF * 32 * t.CB * 8 + (size_t) t.CB * K * K * 16 + (size_t) t.CB * 16;
    }
    __host__ __device__ inline size_t dwpw_strip_lds(int MF, int K, int IR, const DwStrip &t) {
        return dwpw_strip_a_bytes(MF, K, t) + (size_t) t.CB / 2 * t.NF * 32 * 16 + (size_t) t.CB * IR * t.IWp * 8;
    }


    template <int K, int S, int MF, int RT>
    __global__ __launch_bounds__(256, (K == 3 && MF == 1 && RT <= 4) ? 4 : (K == 3 && RT <= 4) ? 3 : 2) void dwpw_strip_kernel(DwPwArgs a, DwStrip t) {
        constexpr int IR  = (RT - 1) * S + K;
        constexpr int NFW = 2;
        extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
        const size_t ab = dwpw_strip_a_bytes(MF, K, t);
        uint4 *asm_ = reinterpret_cast<uint4 *>(dsm);                                              // [MF*32][CB/2], weights, bias
        uint4 *bch  = reinterpret_cast<uint4 *>(dsm + ab);                                         // [CB/2][NF*32]
        uint2 *stg  = reinterpret_cast<uint2 *>(dsm + ab + (size_t) t.CB / 2 * t.NF * 32 * 16);    // [CB][IR][IWp]
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int row_tiles = (a.OH + RT - 1) / RT;
        const int n     = blockIdx.x / row_tiles;
        const int oy0   = (blockIdx.x - n * row_tiles) * RT;
        const int nrows = min(RT, a.OH - oy0);
        const int npx   = nrows * a.OW;
        const int iy0   = oy0 * S - a.PT;
        const int OHW = a.OH * a.OW, HW = a.H * a.W;
        const int BNF = t.NF * 32, CB = t.CB, KG = CB / 2;
        const int IWp = t.IWp;
        const int items = CB * a.OW;

        // input copy geometry: each thread keeps one column and steps down rows (plane-major)
        const int  rpp  = 256 / IWp;
        const int  ccol = tid % IWp;
        const int  crow = tid / IWp;
        const int  cix  = ccol - t.PLA;
        const bool cok  = (unsigned) cix < (unsigned) a.W && crow < rpp;

        float16v acc[MF][NFW];
#pragma unroll
        for (int m = 0; m < MF; ++m)
#pragma unroll
            for (int f = 0; f < NFW; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[m][f][r] = 0.f;

        const int chunks = (a.Ebp + CB - 1) / CB;
        const int rows   = CB * IR;                 // input rows of a chunk
        const int na     = MF * 32 * KG, nw = CB * K * K, n16 = na + nw + CB; // 16-byte units
        // 1. a chunk's data goes global -> registers -> LDS with a batch of loads in flight per
        //    thread before its LDS writes (other workgroups on the CU compute meanwhile): input rows
        //    (8-byte units; each thread keeps one column and steps down the rows), then the
        //    projection weights, depthwise weights and bias (16-byte units, contiguous in LDS)
        for (int ch = 0; ch < chunks; ++ch) {
            const int cb0 = ch * CB;
            {
                constexpr int U = 6;
                for (int base = crow; base < rows; base += U * rpp) {
                    uint2 v[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int row = base + u * rpp;
                        const int pl = row / IR, r = row - pl * IR; // IR is a compile-time constant
                        const int cb = cb0 + pl, iy = iy0 + r;
                        v[u] = uint2 {0u, 0u};
                        if (row < rows && cok && cb < a.Eb && (unsigned) iy < (unsigned) a.H)
                            v[u] = a.x[((long long) n * a.Eb + cb) * HW + (long long) iy * a.W + cix];
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int row = base + u * rpp;
                        if (row < rows && crow < rpp) stg[row * IWp + ccol] = v[u];
                    }
                }
            }
            for (int i = tid; i < n16; i += 256) {
                const uint4 *src = nullptr;
                if (i < na) {
                    const int row = i / KG, k0 = cb0 * 4 + (i - row * KG) * 8;
                    if (k0 < a.Kp) src = reinterpret_cast<const uint4 *>(a.pw_w + (long long) row * a.Kp + k0);
                } else if (i < na + nw) {
                    if (cb0 + (i - na) / (K * K) < a.Eb) src = reinterpret_cast<const uint4 *>(a.dw_w) + (long long) cb0 * K * K + (i - na);
                } else if (cb0 + (i - na - nw) < a.Eb) {
                    src = reinterpret_cast<const uint4 *>(a.dw_b) + cb0 + (i - na - nw);
                }
                asm_[i] = src ? *src : uint4 {0u, 0u, 0u, 0u};
            }
            __syncthreads();
            const float4v *wsm = reinterpret_cast<const float4v *>(asm_ + na);
            const float4v *bsm = wsm + nw;
            // 2. depthwise for this thread's (channel block, column) items
            for (int it = tid; it < items; it += 256) {
                const int cbl = it / a.OW;
                const int ox  = it - cbl * a.OW;
                const int cb  = cb0 + cbl;
                uint2    *dst = reinterpret_cast<uint2 *>(&bch[(cbl >> 1) * BNF + ox]) + (cbl & 1);
                if (cb >= a.Eb) {
#pragma unroll
                    for (int r = 0; r < RT; ++r)
                        if (r < nrows) dst[2 * r * a.OW] = uint2 {0u, 0u};
                    continue;
                }
                half4 w[K * K];
#pragma unroll
                for (int k = 0; k < K * K; ++k) w[k] = f4_to_h4(wsm[cbl * K * K + k]);
                const float4v b = bsm[cbl];
                float4v acc4[RT];
#pragma unroll
                for (int r = 0; r < RT; ++r) acc4[r] = b;
                const uint2 *src = stg + cbl * IR * IWp + ox * S + (t.PLA - a.PL);
#pragma unroll
                for (int ir = 0; ir < IR; ++ir) {
                    half4 tap[K];
#pragma unroll
                    for (int kx = 0; kx < K; ++kx) tap[kx] = u2_as_h4(src[ir * IWp + kx]);
#pragma unroll
                    for (int r = 0; r < RT; ++r) {
                        const int ky = ir - r * S;
                        if (ky < 0 || ky >= K) continue;
#pragma unroll
                        for (int kx = 0; kx < K; ++kx) {
                            const half4 wv = w[ky * K + kx];
                            acc4[r].x = __builtin_fmaf((float) tap[kx].x, (float) wv.x, acc4[r].x);
                            acc4[r].y = __builtin_fmaf((float) tap[kx].y, (float) wv.y, acc4[r].y);
                            acc4[r].z = __builtin_fmaf((float) tap[kx].z, (float) wv.z, acc4[r].z);
                            acc4[r].w = __builtin_fmaf((float) tap[kx].w, (float) wv.w, acc4[r].w);
                        }
                    }
                }
                const int c = cb * 4;
                auto finish = [&](auto act_c) __attribute__((always_inline)) {
                    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
                    for (int r = 0; r < RT; ++r) {
                        if (r >= nrows) break;
                        float4v v = acc4[r];
                        v.x = apply_act(v.x, ACT, 0.f, 6.f);
                        v.y = apply_act(v.y, ACT, 0.f, 6.f);
                        v.z = apply_act(v.z, ACT, 0.f, 6.f);
                        v.w = apply_act(v.w, ACT, 0.f, 6.f);
                        if (c + 0 >= a.E) v.x = 0.f;
                        if (c + 1 >= a.E) v.y = 0.f;
                        if (c + 2 >= a.E) v.z = 0.f;
                        if (c + 3 >= a.E) v.w = 0.f;
                        dst[2 * r * a.OW] = h4_as_u2(f4_to_h4(v));
                    }
                };
                if (a.dw_act == VKHIP_ACT_RELU) finish(std::integral_constant<int, VKHIP_ACT_RELU> {});
                else if (a.dw_act == VKHIP_ACT_RELU6) finish(std::integral_constant<int, VKHIP_ACT_RELU6> {});
                else finish(std::integral_constant<int, VKHIP_ACT_NONE> {});
            }
            // pixels past the strip's last row (fragment padding) read as zero
            for (int i = tid; i < KG * BNF; i += 256)
                if (i % BNF >= npx) bch[i] = uint4 {0u, 0u, 0u, 0u};
            __syncthreads();
            // 3. projection: the chunk's K steps for every fragment of this wave
            for (int ks = 0; ks < CB / 4; ++ks) {
                const int kg = ks * 2 + (lane >> 5);
#pragma unroll
                for (int f = 0; f < NFW; ++f) {
                    const int fr = wave + 4 * f;
                    if (fr >= t.NF) break;
                    const half8 bf = *reinterpret_cast<const half8 *>(&bch[kg * BNF + fr * 32 + (lane & 31)]);
#pragma unroll
                    for (int m = 0; m < MF; ++m) {
                        const half8 af = *reinterpret_cast<const half8 *>(&asm_[(m * 32 + (lane & 31)) * KG + kg]);
                        acc[m][f]      = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[m][f], 0, 0, 0);
                    }
                }
            }
            __syncthreads(); // the next chunk overwrites every LDS region
        }

        // epilogue: bias (+ residual) + activation, fp16 NC4HW4 store
        const int lk = lane >> 5;
#pragma unroll
        for (int f = 0; f < NFW; ++f) {
            const int fr = wave + 4 * f;
            if (fr >= t.NF) break;
            const int px = fr * 32 + (lane & 31);
            if (px >= npx) continue;
            const long long pix = (long long) oy0 * a.OW + px; // within the image's plane
#pragma unroll
            for (int m = 0; m < MF; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int oc  = m * 32 + q * 8 + lk * 4;
                    const int ocb = oc >> 2;
                    if (ocb >= a.Coutb) continue;
                    float4v v = {acc[m][f][q * 4 + 0], acc[m][f][q * 4 + 1], acc[m][f][q * 4 + 2], acc[m][f][q * 4 + 3]};
                    v += *reinterpret_cast<const float4v *>(a.pw_b + oc);
                    const long long yi = ((long long) n * a.Coutb + ocb) * OHW + pix;
                    if (a.has_res) v += h4_to_f4(u2_as_h4(a.res[yi]));
                    v.x = apply_act(v.x, a.act, a.lo, a.hi);
                    v.y = apply_act(v.y, a.act, a.lo, a.hi);
                    v.z = apply_act(v.z, a.act, a.lo, a.hi);
                    v.w = apply_act(v.w, a.act, a.lo, a.hi);
                    if (oc + 0 >= a.Cout) v.x = 0.f;
                    if (oc + 1 >= a.Cout) v.y = 0.f;
                    if (oc + 2 >= a.Cout) v.z = 0.f;
                    if (oc + 3 >= a.Cout) v.w = 0.f;
                    a.y[yi] = h4_as_u2(f4_to_h4(v));
                }
        }
    }

    // Ring-staged fused dw + pw (even input width). Same work split and arithmetic as the strip
    // kernel — a workgroup owns SR output rows of one image (SR = RG row groups of RTT rows, BN =
    // SR * OW pixels) and walks the E expanded channels in chunks of CB channel blocks — but every
    // chunk's operands reach LDS by buffer-load-to-LDS (16 bytes per lane, no VGPR staging) into a
    // ring of NS stages, so chunk ch + NS - 1 streams in while chunk ch computes:
    //   stage = [input band: CB planes x IR rows x IWp pixels, pixel pairs copied whole (input
    //            column ix at LDS column ix + PLA, PLA even, zero pads from out-of-range lanes)]
    //           [projection weights MF*32 x CB/2 16-byte k groups][dw weights CB x K*K, fp16 x 4]
    //           [dw bias CB float4], T KB, copied in 1 KB units dealt round-robin to the 4
    //           waves (lanes past the data copy zeros);
    //   dw       thread item (channel block, row group, column): RTT outputs from (RTT-1)*S + K
    //            band rows, fp16 taps and weights into fp32 sums, bias + dw activation, fp16 into
    //            the B chunk (MFMA fragment layout, 16-byte channel-block pairs per pixel);
    //   project  v_mfma_f32_32x32x16_f16 over the chunk's CB/4 K steps, A from the stage.
    // Units of channel blocks at or past Eb (and projection k past Kp) copy zeros, so padded
    // channels contribute exact zeros. Two barriers per chunk; the band is read from L2/HBM once.
    struct DwRing {
        int         SR, RG, IR, IWp, PLA, NF, CB; // strip rows, row groups, band rows, LDS row pitch (pixels), LDS column of ix=0, pixel fragments, blocks per chunk
        int         NCI, T, na, nw;               // input KB per stage, KB per stage, A / dw-weight 16-byte units
        int         x_bytes, blob_bytes, off_dwb, off_dww, off_pww;
        const void *blob;
    };

    __device__ __forceinline__ void wait_vm_upto(int n) {
        // s_waitcnt takes an immediate: vmcnt(n), expcnt and lgkmcnt left at their maxima
        switch (n) {
            case 0: __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8)); break;
            case 1: __builtin_amdgcn_s_waitcnt(1 | (7 << 4) | (15 << 8)); break;
            case 2: __builtin_amdgcn_s_waitcnt(2 | (7 << 4) | (15 << 8)); break;
            case 3: __builtin_amdgcn_s_waitcnt(3 | (7 << 4) | (15 << 8)); break;
            case 4: __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8)); break;
            case 5: __builtin_amdgcn_s_waitcnt(5 | (7 << 4) | (15 << 8)); break;
            case 6: __builtin_amdgcn_s_waitcnt(6 | (7 << 4) | (15 << 8)); break;
            case 7: __builtin_amdgcn_s_waitcnt(7 | (7 << 4) | (15 << 8)); break;
            default: __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8)); break;
        }
    }

    // copies per wave per stage: stages of at most 16 KB for the 3x3 single-fragment kernels (the
    // register budget of four waves per SIMD), 24 KB otherwise
    __host__ __device__ constexpr int ring_rmax(int K, int MF) { return K == 3 && MF == 1 ? 4 : 6; }

    template <int K, int S, int MF, int RTT, int NS>
    __global__ __launch_bounds__(256, (K == 3 && MF == 1) ? 4 : 2) void dwpw_ring_kernel(DwPwArgs a, DwRing t) {
        constexpr int IRT = (RTT - 1) * S + K; // band rows one item reads
        constexpr int NFW = 2;
        constexpr unsigned kInvalid = 0x80000000u;
        extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
        const int STAGE = t.T * 1024;
        uint4    *bch   = reinterpret_cast<uint4 *>(dsm + NS * STAGE); // [CB/2][NF*32]
        const int tid = threadIdx.x, lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int RW   = (t.T - wave + 3) / 4; // copies this wave issues per stage (units wave, wave + 4, ...)
        const int row_tiles = (a.OH + t.SR - 1) / t.SR;
        const int n     = blockIdx.x / row_tiles;
        const int oy0   = (blockIdx.x - n * row_tiles) * t.SR;
        const int nrows = min(t.SR, a.OH - oy0);
        const int npx   = nrows * a.OW;
        const int iy0   = oy0 * S - a.PT;
        const int HW = a.H * a.W, OHW = a.OH * a.OW;
        const int CB = t.CB, KG = CB / 2, BNF = t.NF * 32, IWp = t.IWp, PW = IWp >> 1;
        const int chunks = (a.Ebp + CB - 1) / CB;
        const int ni = CB * t.IR * PW; // input units of a stage

        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, t.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc((void *) t.blob, (short) 0, t.blob_bytes, 0x00020000);

        // per-lane copy plan, one word per copy: the source offset at chunk 0 (16-byte aligned) with
        // bit 0 set when the unit is real for Eb / CB + 1 chunks instead of Eb / CB (its channel
        // block within the chunk is below Eb % CB), or kInvalid for a unit that is always zero
        // (padding, rows and columns outside the image, lanes past the data). The per-chunk
        // advance depends only on the unit's region.
        constexpr int RMAX = ring_rmax(K, MF);
        unsigned      plan[RMAX];
        const int rmd = a.Eb % CB;
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int c    = r * 4 + wave;
            unsigned  base = kInvalid;
            int       key  = 0; // the unit's channel block within the chunk
            if (r < RW) {
                if (c < t.NCI) {
                    const int u = c * 64 + lane;
                    if (u < ni) {
                        const int pl = u / (t.IR * PW), rem = u - pl * (t.IR * PW);
                        const int rr = rem / PW, j = rem - rr * PW;
                        const int iy = iy0 + rr, ix = 2 * j - t.PLA;
                        if ((unsigned) iy < (unsigned) a.H && ix >= 0 && ix < a.W) {
                            base = (unsigned) ((((long long) n * a.Eb + pl) * HW + (long long) iy * a.W + ix) * 8);
                            key  = pl;
                        }
                    }
                } else {
                    const int ua = (c - t.NCI) * 64 + lane;
                    if (ua < t.na) {
                        const int row = ua / KG, kg = ua - row * KG;
                        base = (unsigned) (t.off_pww + (row * a.Kp + kg * 8) * 2);
                        key  = 2 * kg;
                    } else if (ua < t.na + t.nw) {
                        const int uw = ua - t.na; // fp16 weights, two taps per unit
                        base = (unsigned) (t.off_dww + uw * 16);
                        key  = (2 * uw) / (K * K);
                    } else if (ua < t.na + t.nw + CB) {
                        const int ub = ua - t.na - t.nw;
                        base = (unsigned) (t.off_dwb + ub * 16);
                        key  = ub;
                    }
                }
            }
            plan[r] = base == kInvalid ? kInvalid : base | (key < rmd ? 1u : 0u);
        }
        const int      q0   = a.Eb / CB;
        const unsigned xinc = (unsigned) CB * (unsigned) HW * 8u;
        auto issue = [&](int ch, int buf) __attribute__((always_inline)) {
            unsigned char *dst = dsm + buf * STAGE;
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                if (r >= RW) break;
                const int      c    = r * 4 + wave;
                const unsigned p    = plan[r];
                const bool     real = !(p & kInvalid) && ch < q0 + (int) (p & 1u);
                if (c < t.NCI) {
                    const unsigned vo = real ? (p & ~1u) + (unsigned) ch * xinc : kInvalid;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (dst + c * 1024), 16, vo, 0, 0, 0);
                } else {
                    const int      ua  = (c - t.NCI) * 64 + lane;
                    const unsigned inc = ua < t.na ? (unsigned) CB * 8u : ua < t.na + t.nw ? (unsigned) (CB * K * K * 8) : (unsigned) CB * 16u;
                    const unsigned vo  = real ? (p & ~1u) + (unsigned) ch * inc : kInvalid;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (__attribute__((address_space(3))) void *) (dst + c * 1024), 16, vo, 0, 0, 0);
                }
            }
        };

        float16v acc[MF][NFW];
#pragma unroll
        for (int m = 0; m < MF; ++m)
#pragma unroll
            for (int f = 0; f < NFW; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[m][f][r] = 0.f;

        // fragment columns past the strip's pixels read as zero (never written by the dw phase)
        for (int i = tid; i < KG * BNF; i += 256)
            if (i % BNF >= npx) bch[i] = uint4 {0u, 0u, 0u, 0u};

#pragma unroll
        for (int d = 0; d < NS - 1; ++d)
            if (d < chunks) issue(d, d);

        // this thread's dw items (channel block, row group, column): it = tid and tid + 256,
        // as LDS offsets: band pixel of the first tap, B-chunk half4 slot, weights, bias
        int  isrc[2], idst[2], iw[2], ib[2], irw[2];
        bool iok[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int it  = tid + 256 * k;
            const int cbl = it / (t.RG * a.OW);
            const int rem = it - cbl * (t.RG * a.OW);
            const int rg  = rem / a.OW, ox = rem - rg * a.OW;
            const int r0  = rg * RTT;
            iok[k]  = cbl < CB && r0 < nrows;
            isrc[k] = (cbl * t.IR + r0 * S) * IWp + ox * S + (t.PLA - a.PL);
            idst[k] = ((cbl >> 1) * BNF + r0 * a.OW + ox) * 2 + (cbl & 1);
            iw[k]   = cbl * K * K;
            ib[k]   = cbl;
            irw[k]  = nrows - r0;
        }

        const bool two_items = CB * t.RG * a.OW > 256;
        for (int ch = 0; ch < chunks; ++ch) {
            const int buf = ch % NS;
            wait_vm_upto(min(NS - 2, chunks - 1 - ch) * RW);
            __builtin_amdgcn_s_waitcnt(0xC07F); // and this wave's LDS writes
            __asm__ volatile("s_barrier" ::: "memory");
            if (ch + NS - 1 < chunks) issue(ch + NS - 1, (ch + NS - 1) % NS);

            // LDS is accessed through ext-vector types only: the compiler then keeps the copies
            // in flight across these accesses instead of waiting for them
            const unsigned char *stg  = dsm + buf * STAGE;
            const half8         *asm_ = reinterpret_cast<const half8 *>(stg + t.NCI * 1024);
            const half4         *wsm  = reinterpret_cast<const half4 *>(asm_ + t.na);
            const float4v       *bsm  = reinterpret_cast<const float4v *>(wsm + 2 * t.nw);
            const half4         *inp  = reinterpret_cast<const half4 *>(stg);
            half4               *bh   = reinterpret_cast<half4 *>(bch);
            auto item = [&](const int k) __attribute__((always_inline)) {
                if (!iok[k]) return;
                half4 w[K * K];
#pragma unroll
                for (int q = 0; q < K * K; ++q) w[q] = wsm[iw[k] + q];
                const float4v b = bsm[ib[k]];
                float4v       acc4[RTT];
#pragma unroll
                for (int r = 0; r < RTT; ++r) acc4[r] = b;
                const half4 *src = inp + isrc[k];
#pragma unroll
                for (int ir = 0; ir < IRT; ++ir) {
                    half4 tap[K];
#pragma unroll
                    for (int kx = 0; kx < K; ++kx) tap[kx] = src[ir * IWp + kx];
#pragma unroll
                    for (int r = 0; r < RTT; ++r) {
                        const int ky = ir - r * S;
                        if (ky < 0 || ky >= K) continue;
#pragma unroll
                        for (int kx = 0; kx < K; ++kx) {
                            const half4 wv = w[ky * K + kx];
                            acc4[r].x = __builtin_fmaf((float) tap[kx].x, (float) wv.x, acc4[r].x);
                            acc4[r].y = __builtin_fmaf((float) tap[kx].y, (float) wv.y, acc4[r].y);
                            acc4[r].z = __builtin_fmaf((float) tap[kx].z, (float) wv.z, acc4[r].z);
                            acc4[r].w = __builtin_fmaf((float) tap[kx].w, (float) wv.w, acc4[r].w);
                        }
                    }
                }
                const int c   = (ch * CB + ib[k]) * 4;
                half4    *dst = bh + idst[k];
                // channels past E are zeroed; only the chunk holding E's last block needs the test
                auto finish = [&](auto act_c, auto mask_c) __attribute__((always_inline)) {
                    constexpr int  ACT  = decltype(act_c)::value;
                    constexpr bool MASK = decltype(mask_c)::value;
#pragma unroll
                    for (int r = 0; r < RTT; ++r) {
                        if (r >= irw[k]) break;
                        float4v v = acc4[r];
                        v.x = apply_act(v.x, ACT, 0.f, 6.f);
                        v.y = apply_act(v.y, ACT, 0.f, 6.f);
                        v.z = apply_act(v.z, ACT, 0.f, 6.f);
                        v.w = apply_act(v.w, ACT, 0.f, 6.f);
                        if (MASK) {
                            if (c + 0 >= a.E) v.x = 0.f;
                            if (c + 1 >= a.E) v.y = 0.f;
                            if (c + 2 >= a.E) v.z = 0.f;
                            if (c + 3 >= a.E) v.w = 0.f;
                        }
                        dst[2 * r * a.OW] = f4_to_h4(v);
                    }
                };
                using yes = std::true_type;
                using no  = std::false_type;
                const bool tail = (ch + 1) * CB * 4 > a.E;
                if (a.dw_act == VKHIP_ACT_RELU) {
                    if (tail) finish(std::integral_constant<int, VKHIP_ACT_RELU> {}, yes {});
                    else finish(std::integral_constant<int, VKHIP_ACT_RELU> {}, no {});
                } else if (a.dw_act == VKHIP_ACT_RELU6) {
                    if (tail) finish(std::integral_constant<int, VKHIP_ACT_RELU6> {}, yes {});
                    else finish(std::integral_constant<int, VKHIP_ACT_RELU6> {}, no {});
                } else {
                    if (tail) finish(std::integral_constant<int, VKHIP_ACT_NONE> {}, yes {});
                    else finish(std::integral_constant<int, VKHIP_ACT_NONE> {}, no {});
                }
            };
            item(0);
            if (two_items) item(1); // a uniform branch: the two items are not interleaved
            __builtin_amdgcn_s_waitcnt(0xC07F); // B chunk written (LDS), copies left in flight
            __asm__ volatile("s_barrier" ::: "memory");
            for (int ks = 0; ks < CB / 4; ++ks) {
                const int kg = ks * 2 + (lane >> 5);
#pragma unroll
                for (int f = 0; f < NFW; ++f) {
                    const int fr = wave + 4 * f;
                    if (fr >= t.NF) break;
                    const half8 bf = *reinterpret_cast<const half8 *>(&bch[kg * BNF + fr * 32 + (lane & 31)]);
#pragma unroll
                    for (int m = 0; m < MF; ++m) {
                        const half8 af = *reinterpret_cast<const half8 *>(&asm_[(m * 32 + (lane & 31)) * KG + kg]);
                        acc[m][f]      = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[m][f], 0, 0, 0);
                    }
                }
            }
        }

        // epilogue: bias (+ residual) + activation, fp16 NC4HW4 store
        const int lk = lane >> 5;
#pragma unroll
        for (int f = 0; f < NFW; ++f) {
            const int fr = wave + 4 * f;
            if (fr >= t.NF) break;
            const int px = fr * 32 + (lane & 31);
            if (px >= npx) continue;
            const long long pix = (long long) oy0 * a.OW + px;
#pragma unroll
            for (int m = 0; m < MF; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int oc  = m * 32 + q * 8 + lk * 4;
                    const int ocb = oc >> 2;
                    if (ocb >= a.Coutb) continue;
                    float4v v = {acc[m][f][q * 4 + 0], acc[m][f][q * 4 + 1], acc[m][f][q * 4 + 2], acc[m][f][q * 4 + 3]};
                    v += *reinterpret_cast<const float4v *>(a.pw_b + oc);
                    const long long yi = ((long long) n * a.Coutb + ocb) * OHW + pix;
                    if (a.has_res) v += h4_to_f4(u2_as_h4(a.res[yi]));
                    v.x = apply_act(v.x, a.act, a.lo, a.hi);
                    v.y = apply_act(v.y, a.act, a.lo, a.hi);
                    v.z = apply_act(v.z, a.act, a.lo, a.hi);
                    v.w = apply_act(v.w, a.act, a.lo, a.hi);
                    if (oc + 0 >= a.Cout) v.x = 0.f;
                    if (oc + 1 >= a.Cout) v.y = 0.f;
                    if (oc + 2 >= a.Cout) v.z = 0.f;
                    if (oc + 3 >= a.Cout) v.w = 0.f;
                    a.y[yi] = h4_as_u2(f4_to_h4(v));
                }
        }
    }

    struct DwPwGeom {
        int64_t Eb, Ebp, Kp, Coutb, Coutp, m_frags;
        size_t  off_dwb, off_dww, off_dwh, off_pwb, off_pww, bytes;
        int     BN;
    };

    static size_t a256(size_t v) { return (v + 255) & ~(size_t) 255; }


    typedef void (*GemmStripFn)(DwPwArgs, DwStrip);
    constexpr int kStripRT[] = {14, 8, 7, 4, 2}; // rows per strip the kernel is built for
    template <int K, int S, int MF>
    static GemmStripFn strip_rt(int rt) {
        switch (rt) {
            case 14: return dwpw_strip_kernel<K, S, MF, 14>;
            case 8: return dwpw_strip_kernel<K, S, MF, 8>;
            case 7: return dwpw_strip_kernel<K, S, MF, 7>;
            case 4: return dwpw_strip_kernel<K, S, MF, 4>;
            case 2: return dwpw_strip_kernel<K, S, MF, 2>;
        }
        return nullptr;
    }
    static GemmStripFn dwpw_strip_fn(int K, int S, int mf, int rt) {
        if (mf != 1 && mf != 2) return nullptr;
        if (K == 3) {
            if (S == 1) return mf == 1 ? strip_rt<3, 1, 1>(rt) : strip_rt<3, 1, 2>(rt);
            return mf == 1 ? strip_rt<3, 2, 1>(rt) : strip_rt<3, 2, 2>(rt);
        }
        if (S == 1) return mf == 1 ? strip_rt<5, 1, 1>(rt) : strip_rt<5, 1, 2>(rt);
        return mf == 1 ? strip_rt<5, 2, 1>(rt) : strip_rt<5, 2, 2>(rt);
    }

    // The strip kernel takes square 3x3 / 5x5 kernels at stride 1 or 2 without dilation, up to 64
    // output channels and rows of at most 128 pixels. Rows per strip: the largest built RT with
    // RT * OW <= 256 (and no more than the output has, unless none fits); channel blocks per chunk:
    // the largest multiple of 4 with CB * OW <= 256 (at least 4), at most the padded channel count,
    // halved until the chunk fits 64 KB of LDS (room for a second workgroup per CU).
    static bool dwpw_strip_fits(const vkhip_dwpw_desc *d, const DwPwGeom &g, DwStrip &t, int &RT) {
        const vkhip_conv_desc &c = d->dw;
        if (c.KH != c.KW || (c.KH != 3 && c.KH != 5) || c.SH != c.SW || (c.SH != 1 && c.SH != 2) || c.DH != 1 || c.DW != 1) return false;
        if (g.m_frags > 2 || c.PL < 0 || c.PT < 0 || c.OW > 128) return false;
        RT = 0;
        for (int rt: kStripRT)
            if (rt * c.OW <= 256 && (rt <= c.OH || RT == 0)) {
                RT = rt;
                if (rt <= c.OH) break;
            }
        if (!RT) return false;
        t.BN  = RT * c.OW;
        t.NF  = (int) ceil_div(t.BN, 32);
        if (t.NF > 8) return false;
        t.PLA = c.PL;
        t.IWp = std::max((c.OW - 1) * c.SW + c.KW, c.W + c.PL);
        if (t.IWp > 256) return false;
        t.CB = (int) std::max<int64_t>(4, (256 / c.OW) / 4 * 4);
        t.CB = (int) std::min<int64_t>(t.CB, g.Ebp);
        const int IR = (RT - 1) * c.SH + c.KH;
        auto fits = [&]() { return dwpw_strip_lds((int) g.m_frags, c.KH, IR, t) <= 64 * 1024; };
        while (t.CB > 4 && !fits()) t.CB -= 4;
        if (t.CB % 4) return false;
        return fits();
    }

    typedef void (*RingFn)(DwPwArgs, DwRing);
    template <int K, int S, int MF, int NS>
    static RingFn ring_rtt(int rtt) {
        switch (rtt) {
            case 4: return dwpw_ring_kernel<K, S, MF, 4, NS>;
            case 2: return dwpw_ring_kernel<K, S, MF, 2, NS>;
            case 1: return dwpw_ring_kernel<K, S, MF, 1, NS>;
        }
        return nullptr;
    }
    template <int NS>
    static RingFn ring_fn_ns(int K, int S, int mf, int rtt) {
        if (K == 3) {
            if (S == 1) return mf == 1 ? ring_rtt<3, 1, 1, NS>(rtt) : ring_rtt<3, 1, 2, NS>(rtt);
            return mf == 1 ? ring_rtt<3, 2, 1, NS>(rtt) : ring_rtt<3, 2, 2, NS>(rtt);
        }
        if (S == 1) return mf == 1 ? ring_rtt<5, 1, 1, NS>(rtt) : ring_rtt<5, 1, 2, NS>(rtt);
        return mf == 1 ? ring_rtt<5, 2, 1, NS>(rtt) : ring_rtt<5, 2, 2, NS>(rtt);
    }

    // LDS bytes of the ring kernel: NS stages of T KB plus the B chunk
    static size_t dwpw_ring_lds(const DwRing &t, int NS) { return (size_t) NS * t.T * 1024 + (size_t) t.CB / 2 * t.NF * 32 * 16; }

    // Ring-kernel geometry: square 3x3 / 5x5, stride 1 or 2, no dilation, Cout <= 64, even input
    // width, 32-bit buffer offsets. Strip: RTT rows per item (4, else 2, else 1) and RG row groups,
    // SR = RG * RTT rows with SR * OW <= 256 and no more rows than the output needs; CB the largest
    // multiple of 4 (at least 4) with CB * RG * OW <= 256. Smaller strips are tried until a stage
    // fits ring_rmax KB per wave and the workgroup 64 KB of LDS.
    static bool dwpw_ring_fits(const vkhip_dwpw_desc *d, const DwPwGeom &g, int NS, DwRing &t, int &RTT) {
        const vkhip_conv_desc &c = d->dw;
        if (c.KH != c.KW || (c.KH != 3 && c.KH != 5) || c.SH != c.SW || (c.SH != 1 && c.SH != 2) || c.DH != 1 || c.DW != 1) return false;
        if (g.m_frags > 2 || c.PL < 0 || c.PT < 0 || c.W % 2 || c.OW > 256) return false;
        if ((int64_t) c.N * g.Eb * c.H * c.W * 8 >= (1LL << 31) || g.bytes >= (1ULL << 31)) return false;
        const int K = c.KH, S = c.SH, OW = c.OW;
        t.PLA = (c.PL + 1) & ~1;
        t.IWp = std::max(t.PLA + c.W, (OW - 1) * S + K - c.PL + t.PLA);
        t.IWp = (t.IWp + 1) & ~1;
        const int SRmax = std::min(c.OH, 256 / OW);
        if (SRmax < 1) return false;
        for (int rtt: {4, 2, 1}) {
            if (rtt > SRmax && rtt > 1) continue;
            for (int rg = (SRmax + rtt - 1) / rtt; rg >= 1; --rg) {
                if (rg * rtt * OW > 256) continue;
                t.RG = rg;
                t.SR = rg * rtt;
                t.NF = (int) ceil_div((int64_t) t.SR * OW, 32);
                if (t.NF > 8) continue;
                t.CB = std::max(4, 256 / (rg * OW) / 4 * 4);
                t.CB = (int) std::min<int64_t>(t.CB, g.Ebp);
                t.IR  = (t.SR - 1) * S + K;
                t.na  = (int) g.m_frags * 32 * t.CB / 2;
                t.nw  = t.CB * K * K / 2;
                t.NCI = (int) ceil_div((int64_t) t.CB * t.IR * (t.IWp / 2), 64);
                const int nca = (int) ceil_div(t.na + t.nw + t.CB, 64);
                t.T = t.NCI + nca;
                if (t.T > 4 * ring_rmax(K, (int) g.m_frags) || dwpw_ring_lds(t, NS) > 64 * 1024) continue;
                RTT = rtt;
                return true;
            }
        }
        return false;
    }

    static DwPwGeom dwpw_geom(const vkhip_dwpw_desc *d) {
        DwPwGeom g;
        g.Eb      = ceil_div(d->dw.Cin, 4);
        g.Ebp     = round_up(g.Eb, 8);
        g.Kp      = g.Ebp * 4;
        g.Coutb   = ceil_div(d->Cout, 4);
        g.m_frags = ceil_div(g.Coutb * 4, 32);
        g.Coutp   = g.m_frags * 32;
        g.off_pwb = 0;
        g.off_dwb = a256((size_t) g.Coutp * 4);
        g.off_dww = g.off_dwb + a256((size_t) g.Eb * 16);
        g.off_dwh = g.off_dww + a256((size_t) g.Eb * d->dw.KH * d->dw.KW * 16);
        g.off_pww = g.off_dwh + a256((size_t) g.Eb * d->dw.KH * d->dw.KW * 8);
        g.bytes   = g.off_pww + (size_t) g.Coutp * g.Kp * 2;
        g.BN      = (g.Ebp * 64 * 8 <= 65536) ? 64 : 32;
        return g;
    }


    // y[n][m] = act(b[m] + sum_k x[n][k] w[m][k]) for a small batch N: one workgroup computes a
    // 16 (m) x 16*NF (n) tile with v_mfma_f32_16x16x16f16; its 8 waves take interleaved 32-deep K
    // chunks and reduce their partial tiles through LDS. Fragments go straight from global memory
    // to registers, all U chunks of a wave issued before the first MFMA: weights are read once, x
    // (N*K fp16, small) is served from L2. Lane l of a 16x16x16 MFMA holds A[l%16][4(l/16)..+3],
    // B[4(l/16)..+3][l%16] and D rows 4(l/16)..+3 of column l%16. Within a 32-deep chunk lane
    // group q loads the 8 contiguous k at 8q..8q+7 of its row/column and feeds the low four to one
    // MFMA and the high four to the next: the same permutation of k on A and B, so the sum is the
    // same. X16: x rows are 16-byte aligned (round_up(K,4) % 8 == 0) and loaded 16 bytes at once.
    // PART: x is not given; each 4-channel block of it is the global average pool of a depthwise
    // output, fp16(sum of R fp32 partial sums [N][Kb][R] / HW) (what the pool kernel computes and
    // stores), formed while loading.
    struct FcArgs {
        const uint2   *x;
        const half_t  *w;
        const float   *b;
        uint2         *y;
        int            N, Kb, Kp, M, Mb, act;
        float          lo, hi;
        const float4v *part;
        int            R;
        float          hw;
    };

    template <int NF, bool X16, bool PART>
    __device__ __forceinline__ void fc_tile(const FcArgs &f_, int m0, int n0, float4v (*red)[NF][64]) {
        constexpr int U = 8;
        const FcArgs &A = f_;
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const int r = lane & 15, q = lane >> 4;
        const half_t *wrow = A.w + (size_t) (m0 + r) * A.Kp + 8 * q;
        const uint2  *xrow[NF];
        bool          nok[NF];
        for (int f = 0; f < NF; ++f) {
            const int n = n0 + f * 16 + r;
            nok[f]      = n < A.N;
            xrow[f]     = A.x + (size_t) (nok[f] ? n : 0) * A.Kb + 2 * q;
        }
        float4v acc[NF];
        for (int f = 0; f < NF; ++f) acc[f] = float4v {0.f, 0.f, 0.f, 0.f};
        const int chunks = A.Kp >> 5;
        for (int c0 = wave; c0 < chunks; c0 += 8 * U) {
            half8 a[U], bv[U][NF];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 8 * u;
                a[u]        = half8 {0, 0, 0, 0, 0, 0, 0, 0};
                if (c < chunks) a[u] = *(const half8 *) (wrow + c * 32);
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    const int kb = c * 8 + 2 * q; // first 4-element block of this lane's 8
                    half4     lo4 = {0, 0, 0, 0}, hi4 = {0, 0, 0, 0};
                    if (PART) {
                        const int n = n0 + f * 16 + r;
                        auto pooled = [&](int k) __attribute__((always_inline)) {
                            const float4v *q = A.part + ((long long) n * A.Kb + k) * A.R;
                            float4v        s4 = {0.f, 0.f, 0.f, 0.f};
                            for (int i = 0; i < A.R; ++i) s4 += q[i];
                            return f4_to_h4(s4 / A.hw);
                        };
                        if (c < chunks && nok[f] && kb < A.Kb) lo4 = pooled(kb);
                        if (c < chunks && nok[f] && kb + 1 < A.Kb) hi4 = pooled(kb + 1);
                    } else if (c < chunks && nok[f]) {
                        if (X16) {
                            if (kb < A.Kb) {
                                const uint4 v = *(const uint4 *) (xrow[f] + c * 8);
                                lo4 = u2_as_h4(uint2 {v.x, v.y});
                                hi4 = u2_as_h4(uint2 {v.z, v.w});
                            }
                        } else {
                            if (kb < A.Kb) lo4 = u2_as_h4(xrow[f][c * 8]);
                            if (kb + 1 < A.Kb) hi4 = u2_as_h4(xrow[f][c * 8 + 1]);
                        }
                    }
                    bv[u][f] = half8 {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    const half4 alo = {a[u][0], a[u][1], a[u][2], a[u][3]}, ahi = {a[u][4], a[u][5], a[u][6], a[u][7]};
                    const half4 blo = {bv[u][f][0], bv[u][f][1], bv[u][f][2], bv[u][f][3]};
                    const half4 bhi = {bv[u][f][4], bv[u][f][5], bv[u][f][6], bv[u][f][7]};
                    acc[f] = __builtin_amdgcn_mfma_f32_16x16x16f16(alo, blo, acc[f], 0, 0, 0);
                    acc[f] = __builtin_amdgcn_mfma_f32_16x16x16f16(ahi, bhi, acc[f], 0, 0, 0);
                }
        }
        for (int f = 0; f < NF; ++f) red[wave][f][lane] = acc[f];
        __syncthreads();
        if (threadIdx.x < NF * 64) {
            const int f = threadIdx.x >> 6;
            float4v   v = red[0][f][lane];
            for (int k = 1; k < 8; ++k) v += red[k][f][lane];
            const int n  = n0 + f * 16 + r;
            const int mb = (m0 >> 2) + q; // output channel block: rows m0+4q .. +3
            if (n < A.N && mb < A.Mb) {
                float4v o;
                for (int j = 0; j < 4; ++j) {
                    const int m = mb * 4 + j;
                    o[j]        = m < A.M ? apply_act(v[j] + A.b[m], A.act, A.lo, A.hi) : 0.f;
                }
                A.y[(size_t) n * A.Mb + mb] = h4_as_u2(f4_to_h4(o));
            }
        }
    }

    template <int NF, bool X16, bool PART = false>
    __global__ __launch_bounds__(512) void fc_kernel(FcArgs f) {
        __shared__ float4v red[8][NF][64];
        fc_tile<NF, X16, PART>(f, blockIdx.x * 16, blockIdx.y * (16 * NF), red);
    }

} // namespace vkhip

using namespace vkhip;

extern "C" {

int vkhip_dwpw_supported(const vkhip_dwpw_desc *d) {
    if (!d) return 0;
    const vkhip_conv_desc &c = d->dw;
    if (c.group != c.Cin || c.Cout != c.Cin || c.Cin <= 0 || c.Cin > 1024) return 0;
    if (d->Cout <= 0 || c.N <= 0 || c.OH <= 0 || c.OW <= 0) return 0;
    if (c.act != VKHIP_ACT_NONE && c.act != VKHIP_ACT_RELU && c.act != VKHIP_ACT_RELU6) return 0;
    if ((int64_t) c.N * c.OH * c.OW >= (1LL << 31)) return 0;
    return 1;
}

size_t vkhip_dwpw_weight_bytes(const vkhip_dwpw_desc *d) { return d ? dwpw_geom(d).bytes : 0; }

int vkhip_dwpw_pack_weights(const vkhip_dwpw_desc *d, const float *dw_w, const float *dw_b, const float *pw_w, const float *pw_b, void *blob) {
    if (!d || !dw_w || !pw_w || !blob) return set_error(VKHIP_ERR_INVALID, "dwpw_pack: null argument");
    if (!vkhip_dwpw_supported(d)) return set_error(VKHIP_ERR_UNSUPPORTED, "dwpw_pack: unsupported descriptor");
    DwPwGeom g = dwpw_geom(d);
    std::memset(blob, 0, g.bytes);
    char  *base = (char *) blob;
    float *pwb = (float *) (base + g.off_pwb), *dwb = (float *) (base + g.off_dwb), *dww = (float *) (base + g.off_dww);
    half_t *pww = (half_t *) (base + g.off_pww), *dwh = (half_t *) (base + g.off_dwh);
    const int E = d->dw.Cin, KH = d->dw.KH, KW = d->dw.KW;
    for (int c = 0; c < E; ++c) {
        if (dw_b) dwb[c] = dw_b[c];
        for (int ky = 0; ky < KH; ++ky)
            for (int kx = 0; kx < KW; ++kx) {
                const int64_t i = (((int64_t) (c / 4) * KH + ky) * KW + kx) * 4 + c % 4;
                dww[i] = dw_w[((int64_t) c * KH + ky) * KW + kx];
                dwh[i] = ref_half(dww[i]);
            }
    }
    for (int oc = 0; oc < d->Cout; ++oc) {
        if (pw_b) pwb[oc] = pw_b[oc];
        for (int e = 0; e < E; ++e) pww[(int64_t) oc * g.Kp + e] = ref_half(pw_w[(int64_t) oc * E + e]);
    }
    return VKHIP_OK;
}

int vkhip_dwpw_forward(const vkhip_dwpw_desc *d, const void *x, const void *blob, const void *res, void *y, vkhip_stream_t s) {
    if (!d || !x || !blob || !y) return set_error(VKHIP_ERR_INVALID, "dwpw_forward: null argument");
    if (!vkhip_dwpw_supported(d)) return set_error(VKHIP_ERR_UNSUPPORTED, "dwpw_forward: unsupported descriptor");
    if (d->has_res && !res) return set_error(VKHIP_ERR_INVALID, "dwpw_forward: has_res without residual");
    if (d->has_res > 1) return set_error(VKHIP_ERR_UNSUPPORTED, "dwpw_forward: the residual is added before the activation only");
    DwPwGeom g = dwpw_geom(d);
    const vkhip_conv_desc &c = d->dw;
    DwPwArgs a;
    const char *base = (const char *) blob;
    a.x = (const uint2 *) x;
    a.dw_b = (const float *) (base + g.off_dwb);
    a.dw_w = (const float *) (base + g.off_dww);
    a.pw_b = (const float *) (base + g.off_pwb);
    a.pw_w = (const half_t *) (base + g.off_pww);
    a.res = (const uint2 *) res;
    a.y = (uint2 *) y;
    a.N = c.N; a.E = c.Cin; a.Eb = (int) g.Eb; a.Ebp = (int) g.Ebp; a.H = c.H; a.W = c.W; a.OH = c.OH; a.OW = c.OW;
    a.KH = c.KH; a.KW = c.KW; a.SH = c.SH; a.SW = c.SW; a.PT = c.PT; a.PL = c.PL; a.DH = c.DH; a.DW = c.DW;
    a.dw_act = c.act;
    a.Cout = d->Cout; a.Coutb = (int) g.Coutb; a.m_frags = (int) g.m_frags; a.Kp = (int) g.Kp;
    a.P = c.N * c.OH * c.OW;
    a.act = d->act; a.lo = d->act_lo; a.hi = d->act_hi; a.has_res = d->has_res;
    DwStrip t;
    int     RT = 0;
    // VKHIP_DWPW_STRIP=0 keeps the untiled kernel (A/B measurements)
    const char *strip_env = std::getenv("VKHIP_DWPW_STRIP");
    const bool  strip_on  = !(strip_env && strip_env[0] == '0');
    // VKHIP_DWPW_RING=0 keeps the strip kernel (A/B measurements). Two LDS stages: measured
    // faster than three on every shape, since the third stage costs a workgroup per CU.
    const char *ring_env = std::getenv("VKHIP_DWPW_RING");
    const bool  ring_on  = !(ring_env && ring_env[0] == '0');
    constexpr int kRingNS = 2;
    DwRing rt;
    int    RTT = 0;
    if (ring_on && dwpw_ring_fits(d, g, kRingNS, rt, RTT)) {
        rt.x_bytes    = (int) (c.N * g.Eb * c.H * c.W * 8);
        rt.blob_bytes = (int) g.bytes;
        rt.off_dwb    = (int) g.off_dwb;
        rt.off_dww    = (int) g.off_dwh;
        rt.off_pww    = (int) g.off_pww;
        rt.blob       = blob;
        RingFn fn     = ring_fn_ns<kRingNS>(c.KH, c.SH, (int) g.m_frags, RTT);
        if (fn) {
            dim3 grid((unsigned) (c.N * ceil_div(c.OH, rt.SR)));
            fn<<<grid, 256, dwpw_ring_lds(rt, kRingNS), resolve_stream(s)>>>(a, rt);
            return check_launch("dwpw_ring");
        }
    }
    if (strip_on && dwpw_strip_fits(d, g, t, RT)) {
        const size_t sm = dwpw_strip_lds((int) g.m_frags, c.KH, (RT - 1) * c.SH + c.KH, t);
        dim3         grid((unsigned) (c.N * ceil_div(c.OH, RT)));
        hipStream_t  st = resolve_stream(s);
        GemmStripFn  fn = dwpw_strip_fn(c.KH, c.SH, (int) g.m_frags, RT);
        if (fn) {
            fn<<<grid, 256, sm, st>>>(a, t);
            return check_launch("dwpw_strip");
        }
    }
    size_t sm = (size_t) g.Ebp / 2 * g.BN * 16;
    dim3   grid((unsigned) ceil_div(a.P, g.BN));
    if (g.BN == 64) dwpw_kernel<64><<<grid, 256, sm, resolve_stream(s)>>>(a);
    else dwpw_kernel<32><<<grid, 256, sm, resolve_stream(s)>>>(a);
    return check_launch("dwpw");
}

// ---------------------------------------------------------------- fully connected (skinny GEMM)
// Blob: fp16 W[Mp][Kp] (rows padded to Mp = M rounded up to 16, K to Kp = K rounded up to 32,
// zeros in the padding) followed by fp32 b[Mp].
static void fc_geom(int64_t K, int64_t M, int64_t &Kp, int64_t &Mp) {
    Kp = round_up(K, 32);
    Mp = round_up(M, 16);
}

size_t vkhip_fc_weight_bytes(int64_t K, int64_t M) {
    if (K <= 0 || M <= 0) return 0;
    int64_t Kp, Mp;
    fc_geom(K, M, Kp, Mp);
    return (size_t) (Mp * Kp * 2 + Mp * 4);
}

int vkhip_fc_pack_weights(int64_t K, int64_t M, const float *w, int32_t transB, const float *b, float alpha, float beta, void *blob) {
    if (!w || !blob || K <= 0 || M <= 0) return set_error(VKHIP_ERR_INVALID, "fc_pack: bad arguments");
    int64_t Kp, Mp;
    fc_geom(K, M, Kp, Mp);
    std::memset(blob, 0, vkhip_fc_weight_bytes(K, M));
    half_t *wp = (half_t *) blob;
    float  *bp = (float *) ((char *) blob + Mp * Kp * 2);
    // Gemm B is [K][M] unless transB ([M][K]); alpha scales it and beta the bias, in fp32 before
    // the fp16 conversion (reference cpu/ops/gemm.cpp applies them to the fp32 product).
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t k = 0; k < K; ++k) wp[m * Kp + k] = ref_half(alpha * (transB ? w[m * K + k] : w[k * M + m]));
        bp[m] = b ? beta * b[m] : 0.f;
    }
    return VKHIP_OK;
}

static FcArgs fc_args(const void *x, const float4v *part, int R, int HW, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act,
                      float lo, float hi) {
    int64_t Kp, Mp;
    fc_geom(K, M, Kp, Mp);
    FcArgs f;
    f.x    = (const uint2 *) x;
    f.w    = (const half_t *) blob;
    f.b    = (const float *) ((const char *) blob + Mp * Kp * 2);
    f.y    = (uint2 *) y;
    f.N    = (int) N;
    f.Kb   = (int) (round_up(K, 4) / 4);
    f.Kp   = (int) Kp;
    f.M    = (int) M;
    f.Mb   = (int) (round_up(M, 4) / 4);
    f.act  = act;
    f.lo   = lo;
    f.hi   = hi;
    f.part = part;
    f.R    = R;
    f.hw   = (float) HW;
    return f;
}

// fc launcher: x as fp16 rows, or (part != null) as the pooled partial sums described at fc_kernel
static int fc_launch(const void *x, const float4v *part, int R, int HW, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act,
                     float lo, float hi, vkhip_stream_t s) {
    if ((!x && !part) || !blob || !y || N <= 0 || K <= 0 || M <= 0) return set_error(VKHIP_ERR_INVALID, "fc: bad arguments");
    if (N * round_up(K, 4) >= (1LL << 31) || N * round_up(M, 4) >= (1LL << 31)) return set_error(VKHIP_ERR_UNSUPPORTED, "fc: tensor too large");
    int64_t Kp, Mp;
    fc_geom(K, M, Kp, Mp);
    const int Kb = (int) (round_up(K, 4) / 4);
    // n tiles of 16 while the grid is small (more workgroups pulling weights), else 32
    const bool nf1 = (Mp / 16) * ceil_div(N, 16) <= 512;
    dim3       grid((unsigned) (Mp / 16), (unsigned) ceil_div(N, nf1 ? 16 : 32));
    hipStream_t st = resolve_stream(s);
    const FcArgs f = fc_args(x, part, R, HW, blob, y, N, K, M, act, lo, hi);
    if (part) {
        if (nf1) fc_kernel<1, false, true><<<grid, 512, 0, st>>>(f);
        else fc_kernel<2, false, true><<<grid, 512, 0, st>>>(f);
    } else if (nf1) {
        if (Kb % 2 == 0) fc_kernel<1, true><<<grid, 512, 0, st>>>(f);
        else fc_kernel<1, false><<<grid, 512, 0, st>>>(f);
    } else {
        if (Kb % 2 == 0) fc_kernel<2, true><<<grid, 512, 0, st>>>(f);
        else fc_kernel<2, false><<<grid, 512, 0, st>>>(f);
    }
    return check_launch("fc");
}

int vkhip_fc(const void *x, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act, float lo, float hi, vkhip_stream_t s) {
    if (!x) return set_error(VKHIP_ERR_INVALID, "fc: bad arguments");
    return fc_launch(x, nullptr, 0, 1, blob, y, N, K, M, act, lo, hi, s);
}

int vkhip_fc_pooled(const void *part, int32_t R, int64_t HW, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act, float lo,
                    float hi, vkhip_stream_t s) {
    if (!part || R <= 0 || HW <= 0 || HW >= (1LL << 24)) return set_error(VKHIP_ERR_INVALID, "fc_pooled: bad arguments");
    return fc_launch(nullptr, (const float4v *) part, R, (int) HW, blob, y, N, K, M, act, lo, hi, s);
}

// ---------------------------------------------------------------- squeeze-excite middle
// The blob is the fc blob of W1 (K = C, M = Cr) at offset 0 and that of W2 (K = Cr, M = C) at a
// 256-byte aligned offset. The workspace holds the fp16 hidden layer [N][ceil(Cr/4)] x 4.
static size_t se_w2_offset(int64_t C, int64_t Cr) { return (vkhip_fc_weight_bytes(C, Cr) + 255) & ~(size_t) 255; }

size_t vkhip_se_weight_bytes(int64_t C, int64_t Cr) { return C > 0 && Cr > 0 ? se_w2_offset(C, Cr) + vkhip_fc_weight_bytes(Cr, C) : 0; }

size_t vkhip_se_workspace_bytes(int64_t N, int64_t Cr) { return N > 0 && Cr > 0 ? (size_t) (N * round_up(Cr, 4) * 2) : 0; }

int vkhip_se_pack_weights(int64_t C, int64_t Cr, const float *w1, const float *b1, const float *w2, const float *b2, void *blob) {
    if (!w1 || !w2 || !blob || C <= 0 || Cr <= 0) return set_error(VKHIP_ERR_INVALID, "se_pack: bad arguments");
    std::memset(blob, 0, vkhip_se_weight_bytes(C, Cr));
    int rc = vkhip_fc_pack_weights(C, Cr, w1, 1, b1, 1.f, 1.f, blob);
    if (rc) return rc;
    return vkhip_fc_pack_weights(Cr, C, w2, 1, b2, 1.f, 1.f, (char *) blob + se_w2_offset(C, Cr));
}

// x (avg, fp16 rows) or part (the pooled partial sums): FC1 + ReLU into the workspace, then FC2 +
// hard-sigmoid into y, as two fc launches.
static int se_launch(const void *avg, const float4v *part, int R, int64_t HW, const void *blob, void *y, int64_t N, int64_t C, int64_t Cr,
                     float alpha, float beta, void *workspace, vkhip_stream_t s) {
    int rc = fc_launch(avg, part, R, (int) HW, blob, workspace, N, C, Cr, VKHIP_ACT_RELU, 0.f, 0.f, s);
    if (rc) return rc;
    return fc_launch(workspace, nullptr, 0, 1, (const char *) blob + se_w2_offset(C, Cr), y, N, Cr, C, VKHIP_ACT_HARDSIGMOID, alpha, beta, s);
}

int vkhip_fused_se(const void *avg, const void *blob, void *y, int64_t N, int64_t C, int64_t Cr, float alpha, float beta, void *workspace,
                   vkhip_stream_t s) {
    if (!avg || !blob || !y || !workspace || N <= 0 || C <= 0 || Cr <= 0) return set_error(VKHIP_ERR_INVALID, "fused_se: bad arguments");
    return se_launch(avg, nullptr, 0, 1, blob, y, N, C, Cr, alpha, beta, workspace, s);
}

int vkhip_fused_se_pooled(const void *part, int32_t R, int64_t HW, const void *blob, void *y, int64_t N, int64_t C, int64_t Cr, float alpha,
                          float beta, void *workspace, vkhip_stream_t s) {
    if (!part || R <= 0 || HW <= 0 || HW >= (1LL << 24) || !blob || !y || !workspace || N <= 0 || C <= 0 || Cr <= 0)
        return set_error(VKHIP_ERR_INVALID, "fused_se_pooled: bad arguments");
    return se_launch(nullptr, (const float4v *) part, R, HW, blob, y, N, C, Cr, alpha, beta, workspace, s);
}

} // extern "C"
