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

    struct DwPwGeom {
        int64_t Eb, Ebp, Kp, Coutb, Coutp, m_frags;
        size_t  off_dwb, off_dww, off_pwb, off_pww, bytes;
        int     BN;
    };

    static size_t a256(size_t v) { return (v + 255) & ~(size_t) 255; }

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
        g.off_pww = g.off_dww + a256((size_t) g.Eb * d->dw.KH * d->dw.KW * 16);
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
    template <int NF, bool X16>
    __global__ __launch_bounds__(512) void fc_kernel(const uint2 *x, const half_t *w, const float *b, uint2 *y, int N, int Kb,
                                                     int Kp, int M, int Mb, int act, float lo, float hi) {
        constexpr int U = 8;
        __shared__ float4v red[8][NF][64];
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const int r = lane & 15, q = lane >> 4;
        const int m0 = blockIdx.x * 16, n0 = blockIdx.y * (16 * NF);
        const half_t *wrow = w + (size_t) (m0 + r) * Kp + 8 * q;
        const uint2  *xrow[NF];
        bool          nok[NF];
        for (int f = 0; f < NF; ++f) {
            const int n = n0 + f * 16 + r;
            nok[f]      = n < N;
            xrow[f]     = x + (size_t) (nok[f] ? n : 0) * Kb + 2 * q;
        }
        float4v acc[NF];
        for (int f = 0; f < NF; ++f) acc[f] = float4v {0.f, 0.f, 0.f, 0.f};
        const int chunks = Kp >> 5;
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
                    if (c < chunks && nok[f]) {
                        if (X16) {
                            if (kb < Kb) {
                                const uint4 v = *(const uint4 *) (xrow[f] + c * 8);
                                lo4 = u2_as_h4(uint2 {v.x, v.y});
                                hi4 = u2_as_h4(uint2 {v.z, v.w});
                            }
                        } else {
                            if (kb < Kb) lo4 = u2_as_h4(xrow[f][c * 8]);
                            if (kb + 1 < Kb) hi4 = u2_as_h4(xrow[f][c * 8 + 1]);
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
        if (threadIdx.x >= NF * 64) return;
        const int f = threadIdx.x >> 6;
        float4v   v = red[0][f][lane];
        for (int k = 1; k < 8; ++k) v += red[k][f][lane];
        const int n  = n0 + f * 16 + r;
        const int mb = (m0 >> 2) + q; // output channel block: rows m0+4q .. +3
        if (n >= N || mb >= Mb) return;
        float4v o;
        for (int j = 0; j < 4; ++j) {
            const int m = mb * 4 + j;
            o[j]        = m < M ? apply_act(v[j] + b[m], act, lo, hi) : 0.f;
        }
        y[(size_t) n * Mb + mb] = h4_as_u2(f4_to_h4(o));
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
    half_t *pww = (half_t *) (base + g.off_pww);
    const int E = d->dw.Cin, KH = d->dw.KH, KW = d->dw.KW;
    for (int c = 0; c < E; ++c) {
        if (dw_b) dwb[c] = dw_b[c];
        for (int ky = 0; ky < KH; ++ky)
            for (int kx = 0; kx < KW; ++kx) dww[(((int64_t) (c / 4) * KH + ky) * KW + kx) * 4 + c % 4] = dw_w[((int64_t) c * KH + ky) * KW + kx];
    }
    for (int oc = 0; oc < d->Cout; ++oc) {
        if (pw_b) pwb[oc] = pw_b[oc];
        for (int e = 0; e < E; ++e) pww[(int64_t) oc * g.Kp + e] = (half_t) pw_w[(int64_t) oc * E + e];
    }
    return VKHIP_OK;
}

int vkhip_dwpw_forward(const vkhip_dwpw_desc *d, const void *x, const void *blob, const void *res, void *y, vkhip_stream_t s) {
    if (!d || !x || !blob || !y) return set_error(VKHIP_ERR_INVALID, "dwpw_forward: null argument");
    if (!vkhip_dwpw_supported(d)) return set_error(VKHIP_ERR_UNSUPPORTED, "dwpw_forward: unsupported descriptor");
    if (d->has_res && !res) return set_error(VKHIP_ERR_INVALID, "dwpw_forward: has_res without residual");
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
        for (int64_t k = 0; k < K; ++k) wp[m * Kp + k] = (half_t) (alpha * (transB ? w[m * K + k] : w[k * M + m]));
        bp[m] = b ? beta * b[m] : 0.f;
    }
    return VKHIP_OK;
}

int vkhip_fc(const void *x, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act, float lo, float hi, vkhip_stream_t s) {
    if (!x || !blob || !y || N <= 0 || K <= 0 || M <= 0) return set_error(VKHIP_ERR_INVALID, "fc: bad arguments");
    if (N * round_up(K, 4) >= (1LL << 31) || N * round_up(M, 4) >= (1LL << 31)) return set_error(VKHIP_ERR_UNSUPPORTED, "fc: tensor too large");
    int64_t Kp, Mp;
    fc_geom(K, M, Kp, Mp);
    const half_t *wp = (const half_t *) blob;
    const float  *bp = (const float *) ((const char *) blob + Mp * Kp * 2);
    const int Kb = (int) (round_up(K, 4) / 4), Mb = (int) (round_up(M, 4) / 4);
    // n tiles of 16 while the grid is small (more workgroups pulling weights), else 32
    const bool nf1 = (Mp / 16) * ceil_div(N, 16) <= 512;
    dim3       grid((unsigned) (Mp / 16), (unsigned) ceil_div(N, nf1 ? 16 : 32));
    hipStream_t st = resolve_stream(s);
    const uint2 *xx = (const uint2 *) x;
    uint2       *yy = (uint2 *) y;
    if (nf1) {
        if (Kb % 2 == 0) fc_kernel<1, true><<<grid, 512, 0, st>>>(xx, wp, bp, yy, (int) N, Kb, (int) Kp, (int) M, Mb, act, lo, hi);
        else fc_kernel<1, false><<<grid, 512, 0, st>>>(xx, wp, bp, yy, (int) N, Kb, (int) Kp, (int) M, Mb, act, lo, hi);
    } else {
        if (Kb % 2 == 0) fc_kernel<2, true><<<grid, 512, 0, st>>>(xx, wp, bp, yy, (int) N, Kb, (int) Kp, (int) M, Mb, act, lo, hi);
        else fc_kernel<2, false><<<grid, 512, 0, st>>>(xx, wp, bp, yy, (int) N, Kb, (int) Kp, (int) M, Mb, act, lo, hi);
    }
    return check_launch("fc");
}

} // extern "C"
