/*
 * TEST INFRASTRUCTURE — CPU oracle of the fused fp16 convolution path (see oracle.h).
 * Each function restates one reference CPU routine with the same loop order and accumulator
 * types; the citation above each function names the file:lines it follows.
 * Build: gcc -O2 -std=c99 (no -ffast-math, no FMA: x86-64 baseline has none, as in the reference
 * build) so the float arithmetic matches the reference CPU backend bit for bit.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* include/vknn/dtype.h:121-157 */
uint16_t oracle_float_to_half(float v) {
    uint32_t f;
    memcpy(&f, &v, 4);
    uint32_t sign = (f >> 16) & 0x8000u;
    int32_t  e    = (int32_t) ((f >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = f & 0x7FFFFFu;
    if (((f >> 23) & 0xFFu) == 0xFFu) return (uint16_t) (sign | 0x7C00u | (mant ? 0x200u : 0u));
    if (e >= 0x1F) return (uint16_t) (sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t) sign;
        mant |= 0x800000u;
        uint32_t shift = (uint32_t) (14 - e);
        uint32_t half  = mant >> shift;
        if ((mant >> (shift - 1)) & 1u) half += 1;
        return (uint16_t) (sign | half);
    }
    uint16_t out = (uint16_t) (sign | ((uint32_t) e << 10) | (mant >> 13));
    if (mant & 0x1000u) out += 1;
    return out;
}

/* include/vknn/dtype.h:60-92 */
float oracle_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    uint32_t e    = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t f;
    if (e == 0) {
        if (mant == 0) {
            f = sign;
        } else {
            e = 127 - 15 + 1;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                --e;
            }
            mant &= 0x3FFu;
            f = sign | (e << 23) | (mant << 13);
        }
    } else if (e == 0x1F) {
        f = sign | 0x7F800000u | (mant << 13);
    } else {
        f = sign | ((e - 15 + 127) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

void oracle_float_to_half_n(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_float_to_half(src[i]);
}
/* IEEE-754 binary32 -> binary16, round to nearest, ties to even (not the reference host codec:
 * this is what the reference's GLSL float16_t conversion does on the boundary converter). */
uint16_t oracle_float_to_half_rne(float v) {
    uint32_t x;
    memcpy(&x, &v, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ex   = (x >> 23) & 0xFFu;
    uint32_t       m    = x & 0x7FFFFFu;
    if (ex == 0xFFu) return (uint16_t) (sign | 0x7C00u | (m ? 0x200u | (m >> 13) : 0u)); /* inf / quiet NaN */
    const int e = (int) ex - 127 + 15;
    if (e >= 31) return (uint16_t) (sign | 0x7C00u);                                    /* overflow */
    if (e <= 0) {                                                                         /* subnormal or zero */
        if (e < -10) return (uint16_t) sign;
        m |= 0x800000u;                      /* implicit bit */
        const int      shift = 14 - e;       /* 24-bit significand -> 10-bit field at exponent -14 */
        const uint32_t half  = 1u << (shift - 1);
        uint32_t       q     = m >> shift;
        const uint32_t rem   = m & ((1u << shift) - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q; /* may carry into the smallest normal */
        return (uint16_t) (sign | q);
    }
    uint32_t       q   = ((uint32_t) e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q; /* carry may reach the exponent, even inf */
    return (uint16_t) (sign | q);
}

static int64_t oracle_layout_offset(int fmt, int64_t n, int64_t c, int64_t h, int64_t w, int64_t C, int64_t H, int64_t W) {
    if (fmt == 1) return ((n * H + h) * W + w) * C + c;
    if (fmt == 2) return (((n * ((C + 3) / 4) + c / 4) * H + h) * W + w) * 4 + c % 4;
    return ((n * C + c) * H + h) * W + w;
}

void oracle_boundary_convert(const void *src, int src_fmt, int src_f16, void *dst, int dst_fmt, int dst_f16, int64_t N, int64_t C,
                             int64_t H, int64_t W) {
    const int64_t Cd = dst_fmt == 2 ? (C + 3) / 4 * 4 : C; /* destination channel extent incl. padding */
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < Cd; ++c)
            for (int64_t h = 0; h < H; ++h)
                for (int64_t w = 0; w < W; ++w) {
                    const int64_t di = dst_fmt == 2 ? oracle_layout_offset(2, n, c, h, w, C, H, W) : oracle_layout_offset(dst_fmt, n, c, h, w, C, H, W);
                    float         v  = 0.f;
                    uint16_t      hv = 0;
                    if (c < C) {
                        const int64_t si = oracle_layout_offset(src_fmt, n, c, h, w, C, H, W);
                        if (src_f16) {
                            hv = ((const uint16_t *) src)[si];
                            v  = oracle_half_to_float(hv);
                        } else {
                            v = ((const float *) src)[si];
                        }
                    }
                    if (dst_f16) ((uint16_t *) dst)[di] = c < C ? (src_f16 ? hv : oracle_float_to_half_rne(v)) : 0;
                    else ((float *) dst)[di] = v;
                }
}

void oracle_half_to_float_n(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_half_to_float(src[i]);
}

/* src/backend/vulkan/vk_backend.cpp:576-611 (fp16 NC4HW4 pack: gather 4 channels, zero lanes
 * past C, floatToHalf each) */
void oracle_pack_nc4hw4(const float *src, uint16_t *dst, int64_t N, int64_t C, int64_t H, int64_t W) {
    int64_t Cb = (C + 3) / 4;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t cb = 0; cb < Cb; ++cb)
            for (int64_t h = 0; h < H; ++h)
                for (int64_t w = 0; w < W; ++w) {
                    int64_t base = ((((n * Cb + cb) * H + h) * W) + w) * 4;
                    float   t[4] = {0, 0, 0, 0};
                    for (int l = 0; l < 4; ++l) {
                        int64_t c = cb * 4 + l;
                        if (c < C) t[l] = src[((n * C + c) * H + h) * W + w];
                    }
                    for (int l = 0; l < 4; ++l) dst[base + l] = oracle_float_to_half(t[l]);
                }
}

/* src/backend/vulkan/vk_backend.cpp:652-673 */
void oracle_unpack_nc4hw4(const uint16_t *src, float *dst, int64_t N, int64_t C, int64_t H, int64_t W) {
    int64_t Cb = (C + 3) / 4;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < C; ++c)
            for (int64_t h = 0; h < H; ++h)
                for (int64_t w = 0; w < W; ++w) {
                    int64_t cb = c / 4, l = c % 4;
                    int64_t s  = ((((n * Cb + cb) * H + h) * W) + w) * 4 + l;
                    dst[((n * C + c) * H + h) * W + w] = oracle_half_to_float(src[s]);
                }
}

/* src/backend/cpu/cpu_backend.cpp:33-72 */
void oracle_apply_act(float *p, int64_t n, int act, float lo, float hi) {
    switch (act) {
        case 1:
            for (int64_t i = 0; i < n; ++i) p[i] = p[i] > 0 ? p[i] : 0;
            break;
        case 2:
            for (int64_t i = 0; i < n; ++i) {
                float v = p[i];
                p[i]    = v < 0 ? 0 : (v > 6 ? 6 : v);
            }
            break;
        case 3:
            for (int64_t i = 0; i < n; ++i) {
                float v = p[i];
                p[i]    = v < lo ? lo : (v > hi ? hi : v);
            }
            break;
        case 4:
            for (int64_t i = 0; i < n; ++i) {
                float v = p[i];
                float c = v + 3.f;
                c       = c > 0.f ? c : 0.f; /* std::max(v+3, 0) */
                c       = c < 6.f ? c : 6.f; /* std::min(., 6) */
                p[i]    = v * c / 6.f;
            }
            break;
        case 5:
            for (int64_t i = 0; i < n; ++i) p[i] = p[i] / (1.f + expf(-p[i]));
            break;
        default:
            break;
    }
}

void oracle_conv_out_hw(int64_t H, int64_t W, int64_t KH, int64_t KW, const int64_t st[2], const int64_t pads[4],
                        const int64_t dil[2], int64_t *OH, int64_t *OW) {
    *OH = (H + pads[0] + pads[2] - (dil[0] * (KH - 1) + 1)) / st[0] + 1;
    *OW = (W + pads[1] + pads[3] - (dil[1] * (KW - 1) + 1)) / st[1] + 1;
}

/* src/backend/cpu/ops/conv.cpp:9-92: n -> oc -> oy -> ox; acc = bias; ic -> ky -> kx with
 * bounds-continue; then y += residual over the whole tensor; then applyAct. */
void oracle_conv2d(const float *x, int64_t N, int64_t C, int64_t H, int64_t W, const float *w, int64_t Cout, int64_t KH,
                   int64_t KW, const float *bias, const int64_t st[2], const int64_t pads[4], const int64_t dil[2],
                   int64_t group, const float *res, int act, float lo, float hi, float *y) {
    int64_t OH, OW;
    oracle_conv_out_hw(H, W, KH, KW, st, pads, dil, &OH, &OW);
    int64_t inCg  = C / group;
    int64_t outCg = Cout / group;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t oc = 0; oc < Cout; ++oc) {
            int64_t g       = oc / outCg;
            int64_t icStart = g * inCg;
            float   b       = bias ? bias[oc] : 0.f;
            for (int64_t oy = 0; oy < OH; ++oy)
                for (int64_t ox = 0; ox < OW; ++ox) {
                    float   acc = b;
                    int64_t iy0 = oy * st[0] - pads[0];
                    int64_t ix0 = ox * st[1] - pads[1];
                    for (int64_t ic = 0; ic < inCg; ++ic) {
                        const float *xch = x + ((n * C + (icStart + ic)) * H) * W;
                        const float *wch = w + ((oc * inCg + ic) * KH) * KW;
                        for (int64_t ky = 0; ky < KH; ++ky) {
                            int64_t iy = iy0 + ky * dil[0];
                            if (iy < 0 || iy >= H) continue;
                            for (int64_t kx = 0; kx < KW; ++kx) {
                                int64_t ix = ix0 + kx * dil[1];
                                if (ix < 0 || ix >= W) continue;
                                acc += xch[iy * W + ix] * wch[ky * KW + kx];
                            }
                        }
                    }
                    y[((n * Cout + oc) * OH + oy) * OW + ox] = acc;
                }
        }
    int64_t total = N * Cout * OH * OW;
    if (res)
        for (int64_t i = 0; i < total; ++i) y[i] += res[i];
    oracle_apply_act(y, total, act, lo, hi);
}

/* src/backend/cpu/ops/fused_dwpw.cpp:10-87: per image, depthwise into a scratch [E][OH*OW],
 * dw act with bounds 0/6, then project (acc = pb; += pw*dw over e; + res) and one final act. */
void oracle_fused_dwpw(const float *x, int64_t N, int64_t E, int64_t H, int64_t W, const float *dw_w, int64_t KH, int64_t KW,
                       const float *dw_b, const float *pw_w, int64_t Cout, const float *pw_b, const int64_t st[2],
                       const int64_t pad[4], const int64_t dil[2], int dw_act, const float *res, int act, float lo, float hi,
                       float *y) {
    int64_t OH, OW;
    oracle_conv_out_hw(H, W, KH, KW, st, pad, dil, &OH, &OW);
    float *dwOut = (float *) malloc((size_t) (E * OH * OW) * sizeof(float));
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t e = 0; e < E; ++e)
            for (int64_t oy = 0; oy < OH; ++oy)
                for (int64_t ox = 0; ox < OW; ++ox) {
                    float acc = dw_b ? dw_b[e] : 0.f;
                    for (int64_t ky = 0; ky < KH; ++ky) {
                        int64_t iy = oy * st[0] - pad[0] + ky * dil[0];
                        if (iy < 0 || iy >= H) continue;
                        for (int64_t kx = 0; kx < KW; ++kx) {
                            int64_t ix = ox * st[1] - pad[1] + kx * dil[1];
                            if (ix < 0 || ix >= W) continue;
                            acc += x[((n * E + e) * H + iy) * W + ix] * dw_w[(e * KH + ky) * KW + kx];
                        }
                    }
                    dwOut[(e * OH + oy) * OW + ox] = acc;
                }
        oracle_apply_act(dwOut, E * OH * OW, dw_act, 0, 6);
        for (int64_t c = 0; c < Cout; ++c)
            for (int64_t p = 0; p < OH * OW; ++p) {
                float acc = pw_b ? pw_b[c] : 0.f;
                for (int64_t e = 0; e < E; ++e) acc += pw_w[c * E + e] * dwOut[e * OH * OW + p];
                int64_t oi = (n * Cout + c) * OH * OW + p;
                if (res) acc += res[oi];
                y[oi] = acc;
            }
    }
    free(dwOut);
    oracle_apply_act(y, N * Cout * OH * OW, act, lo, hi);
}

/* src/backend/cpu/ops/fused_se.cpp:9-47 */
void oracle_fused_se(const float *avg, int64_t N, int64_t C, const float *w1, int64_t Cr, const float *b1, const float *w2,
                     const float *b2, float a, float b, float *y) {
    float *s1 = (float *) malloc((size_t) Cr * sizeof(float));
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t j = 0; j < Cr; ++j) {
            double s = b1 ? b1[j] : 0.0;
            for (int64_t c = 0; c < C; ++c) s += (double) w1[j * C + c] * avg[n * C + c];
            s1[j] = s > 0 ? (float) s : 0.f;
        }
        for (int64_t k = 0; k < C; ++k) {
            double s = b2 ? b2[k] : 0.0;
            for (int64_t j = 0; j < Cr; ++j) s += (double) w2[k * Cr + j] * s1[j];
            float v = a * (float) s + b;
            v       = v > 0.f ? v : 0.f; /* std::max(., 0) */
            y[n * C + k] = v < 1.f ? v : 1.f;
        }
    }
    free(s1);
}

/* src/backend/cpu/ops/add.cpp:67-86 */
void oracle_add(const float *a, const float *b, float *y, int64_t n, int act, float lo, float hi) {
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
    oracle_apply_act(y, n, act, lo, hi);
}

/* src/backend/cpu/ops/binary.cpp: Mul with a [N,C,1,1] operand broadcast over H*W */
void oracle_mul_channel(const float *x, const float *s, float *y, int64_t N, int64_t C, int64_t HW) {
    for (int64_t nc = 0; nc < N * C; ++nc)
        for (int64_t p = 0; p < HW; ++p) y[nc * HW + p] = x[nc * HW + p] * s[nc];
}

/* src/backend/cpu/ops/binary.cpp (same-shape path; BinaryType codes) */
void oracle_binary(const float *a, const float *b, float *y, int64_t n, int op) {
    for (int64_t i = 0; i < n; ++i) {
        float u = a[i], v = b[i];
        switch (op) {
            case 0: y[i] = u * v; break;
            case 1: y[i] = u - v; break;
            case 2: y[i] = u / v; break;
            case 3: y[i] = u > v ? u : v; break;
            case 4: y[i] = u < v ? u : v; break;
            case 5: y[i] = powf(u, v); break;
            default: y[i] = u + v; break;
        }
    }
}

/* src/backend/cpu/ops/unary.cpp:9-58 (subset on the conv path), relu.cpp, clip.cpp */
void oracle_unary(const float *x, float *y, int64_t n, int op, float p0, float p1) {
    for (int64_t i = 0; i < n; ++i) {
        float v = x[i], r = v;
        switch (op) {
            case -1: r = v < p0 ? p0 : (v > p1 ? p1 : v); break;
            case 0: r = 1.f / (1.f + expf(-v)); break;
            case 2: {
                float c = v + 3.f;
                c       = c > 0.f ? c : 0.f;
                c       = c < 6.f ? c : 6.f;
                r       = v * c / 6.f;
                break;
            }
            case 3: {
                float t = p0 * v + p1;
                t       = t > 0.f ? t : 0.f;
                r       = t < 1.f ? t : 1.f;
                break;
            }
            case 13: r = v > 0 ? v : 0; break;
            case 14: r = v / (1.f + expf(-v)); break;
            default: break;
        }
        y[i] = r;
    }
}

/* src/backend/cpu/ops/global_avg_pool.cpp:7-28 */
void oracle_global_avg_pool(const float *x, float *y, int64_t N, int64_t C, int64_t HW) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < C; ++c) {
            const float *p = x + (n * C + c) * HW;
            double       s = 0;
            for (int64_t i = 0; i < HW; ++i) s += p[i];
            y[n * C + c] = (float) (s / HW);
        }
}

/* src/backend/cpu/ops/maxpool.cpp:7-55 */
void oracle_maxpool(const float *x, float *y, int64_t N, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t SH,
                    int64_t SW, int64_t PT, int64_t PL, int64_t OH, int64_t OW) {
    for (int64_t nc = 0; nc < N * C; ++nc) {
        const float *xc = x + nc * H * W;
        for (int64_t oy = 0; oy < OH; ++oy)
            for (int64_t ox = 0; ox < OW; ++ox) {
                float m = -INFINITY;
                for (int64_t ky = 0; ky < KH; ++ky) {
                    int64_t iy = oy * SH - PT + ky;
                    if (iy < 0 || iy >= H) continue;
                    for (int64_t kx = 0; kx < KW; ++kx) {
                        int64_t ix = ox * SW - PL + kx;
                        if (ix < 0 || ix >= W) continue;
                        float v = xc[iy * W + ix];
                        m       = (m < v) ? v : m; /* std::max(m, v) */
                    }
                }
                y[(nc * OH + oy) * OW + ox] = m;
            }
    }
}

/* src/backend/cpu/ops/gemm.cpp:11-60 (scalar path: acc over k, *alpha, + beta*c[n], act) */
void oracle_gemm(const float *a, const float *b, const float *c, float *y, int64_t M, int64_t K, int64_t N, int transB,
                 float alpha, float beta, int act, float lo, float hi) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0;
            for (int64_t k = 0; k < K; ++k) {
                float av = a[m * K + k];
                float bv = transB ? b[n * K + k] : b[k * N + n];
                acc += av * bv;
            }
            acc *= alpha;
            if (c) acc += beta * c[n];
            y[m * N + n] = acc;
        }
    oracle_apply_act(y, M * N, act, lo, hi);
}

/* src/backend/cpu/ops/concat.cpp (axis 1) */
void oracle_concat_channels(const float *const *xs, const int64_t *cs, int count, float *y, int64_t N, int64_t HW) {
    int64_t Cy = 0;
    for (int i = 0; i < count; ++i) Cy += cs[i];
    for (int64_t n = 0; n < N; ++n) {
        int64_t c0 = 0;
        for (int i = 0; i < count; ++i) {
            memcpy(y + (n * Cy + c0) * HW, xs[i] + n * cs[i] * HW, (size_t) (cs[i] * HW) * sizeof(float));
            c0 += cs[i];
        }
    }
}

/* src/backend/cpu/ops/split.cpp (axis 1, one output) */
void oracle_slice_channels(const float *x, float *y, int64_t N, int64_t Cx, int64_t c0, int64_t C, int64_t HW) {
    for (int64_t n = 0; n < N; ++n) memcpy(y + n * C * HW, x + (n * Cx + c0) * HW, (size_t) (C * HW) * sizeof(float));
}

/* src/backend/cpu/ops/resize.cpp:30-45 (srcCoord: scale = out/in as float; half_pixel (0) or
 * asymmetric (2)) and :75-87 (nearest = round_prefer_floor, clamped) */
static float resize_src(int d, int outS, int inS, int coordMode) {
    float scale = (float) outS / (float) inS;
    if (coordMode == 2) return (float) d / scale;
    return ((float) d + 0.5f) / scale - 0.5f;
}
void oracle_resize_nearest(const float *x, float *y, int64_t NC, int64_t H, int64_t W, int64_t OH, int64_t OW, int coordMode) {
    for (int64_t nc = 0; nc < NC; ++nc) {
        const float *xc = x + nc * H * W;
        float       *yc = y + nc * OH * OW;
        for (int oy = 0; oy < (int) OH; ++oy) {
            float fy = resize_src(oy, (int) OH, (int) H, coordMode);
            for (int ox = 0; ox < (int) OW; ++ox) {
                float fx = resize_src(ox, (int) OW, (int) W, coordMode);
                int   iy = (int) floorf(fy);
                if (fy - iy > 0.5f) iy++;
                int ix = (int) floorf(fx);
                if (fx - ix > 0.5f) ix++;
                iy = iy < 0 ? 0 : (iy > (int) H - 1 ? (int) H - 1 : iy);
                ix = ix < 0 ? 0 : (ix > (int) W - 1 ? (int) W - 1 : ix);
                yc[oy * OW + ox] = xc[iy * W + ix];
            }
        }
    }
}

/* src/import/fold_batchnorm.cpp:57-78 */
void oracle_fold_bn(float *w, float *b, int64_t Cout, int64_t perOC, const float *gamma, const float *beta, const float *mean,
                    const float *var, float eps) {
    for (int64_t oc = 0; oc < Cout; ++oc) {
        float a = gamma[oc] / sqrtf(var[oc] + eps);
        for (int64_t k = 0; k < perOC; ++k) w[oc * perOC + k] *= a;
        b[oc] = (b[oc] - mean[oc]) * a + beta[oc];
    }
}
