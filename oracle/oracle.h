/*
 * TEST INFRASTRUCTURE — the CPU oracle of the fused fp16 convolution path.
 *
 * A plain-C restatement of the reference's CPU backend arithmetic for this path, with the same
 * loop nests and the same fp32 (or, where the reference uses it, double) accumulation order, so a
 * build with the same compiler flags reproduces the reference CPU results bit for bit. It is the
 * parity checker for the HIP kernels and the timed CPU baseline; nothing in the product links or
 * calls it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   codec, pack/unpack     exhaustive rounding-boundary sweep vs oracle/_ref + golden edge table +
 *                          closed forms (exactly representable values round-trip, RNE disagreement set)
 *   conv2d                 oracle/_ref single-op graphs (bit-exact) + golden fixtures + torch
 *                          conv2d textbook cross-check + brute-force on tiny inputs
 *   fused_dwpw, fused_se   oracle/_ref single-node graphs (bit-exact) + golden fixtures + the
 *                          composition identity (dwpw == conv(dw) -> conv(pw))
 *   add/mul/unary/act/gap/ oracle/_ref single-op graphs + closed forms
 *   maxpool/gemm/concat/
 *   resize/bn_fold
 *   boundary_convert       numpy: astype(float16) (IEEE round-to-nearest-even) and
 *                          reshape/transpose constructions of NHWC and NC4HW4
 */
#ifndef VKNN_ORACLE_H
#define VKNN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/vknn/dtype.h:121-157 / :60-92 */
uint16_t oracle_float_to_half(float v);
float    oracle_half_to_float(uint16_t h);
void     oracle_float_to_half_n(const float *src, uint16_t *dst, int64_t n);
void     oracle_half_to_float_n(const uint16_t *src, float *dst, int64_t n);
/* fp32 -> fp16 with IEEE round-to-nearest-even (the GPU boundary converter's rounding,
 * shaders/boundary_convert.comp, as opposed to the host codec above). */
uint16_t oracle_float_to_half_rne(float v);
/* shaders/boundary_convert.comp:20-58 (also shaders/convert_layout.comp for the same-type case):
 * fmt 0 NCHW, 1 NHWC, 2 NC4HW4; *_f16 selects fp16 (uint16 bits) or fp32 storage. One destination
 * element at a time, NC4HW4 padding lanes 0. */
void     oracle_boundary_convert(const void *src, int src_fmt, int src_f16, void *dst, int dst_fmt, int dst_f16, int64_t N, int64_t C,
                                 int64_t H, int64_t W);

/* src/backend/vulkan/vk_backend.cpp:576-611 (fp16 NC4HW4 pack) and :652-673 (unpack) */
void oracle_pack_nc4hw4(const float *src, uint16_t *dst, int64_t N, int64_t C, int64_t H, int64_t W);
void oracle_unpack_nc4hw4(const uint16_t *src, float *dst, int64_t N, int64_t C, int64_t H, int64_t W);

/* src/backend/cpu/cpu_backend.cpp:33-72 (act codes = vknn ActType) */
void oracle_apply_act(float *p, int64_t n, int act, float lo, float hi);

/* src/backend/cpu/ops/conv.cpp:9-92. w: [Cout][Cin/group][KH][KW]; pads = {top,left,bottom,right};
 * bias, res may be NULL. y: [N][Cout][OH][OW] with the ONNX output-size rule. */
void oracle_conv2d(const float *x, int64_t N, int64_t C, int64_t H, int64_t W, const float *w, int64_t Cout, int64_t KH,
                   int64_t KW, const float *bias, const int64_t strides[2], const int64_t pads[4], const int64_t dil[2],
                   int64_t group, const float *res, int act, float lo, float hi, float *y);
void oracle_conv_out_hw(int64_t H, int64_t W, int64_t KH, int64_t KW, const int64_t strides[2], const int64_t pads[4],
                        const int64_t dil[2], int64_t *OH, int64_t *OW);

/* src/backend/cpu/ops/fused_dwpw.cpp:10-87. dw_w [E][1][KH][KW]; pw_w [Cout][E]. */
void oracle_fused_dwpw(const float *x, int64_t N, int64_t E, int64_t H, int64_t W, const float *dw_w, int64_t KH, int64_t KW,
                       const float *dw_b, const float *pw_w, int64_t Cout, const float *pw_b, const int64_t strides[2],
                       const int64_t pads[4], const int64_t dil[2], int dw_act, const float *res, int act, float lo, float hi,
                       float *y);

/* src/backend/cpu/ops/fused_se.cpp:9-47 (double accumulation). avg [N][C]; w1 [Cr][C]; w2 [C][Cr]. */
void oracle_fused_se(const float *avg, int64_t N, int64_t C, const float *w1, int64_t Cr, const float *b1, const float *w2,
                     const float *b2, float alpha, float beta, float *y);

/* src/backend/cpu/ops/add.cpp:67-86 (same-shape path + fused act) */
void oracle_add(const float *a, const float *b, float *y, int64_t n, int act, float lo, float hi);
/* src/backend/cpu/ops/binary.cpp (Mul, channel broadcast s[N][C] over [N][C][HW]) */
void oracle_mul_channel(const float *x, const float *s, float *y, int64_t N, int64_t C, int64_t HW);
void oracle_binary(const float *a, const float *b, float *y, int64_t n, int op);
/* src/backend/cpu/ops/unary.cpp (UnaryType codes; HardSigmoid alpha/beta in p0/p1) and
 * src/backend/cpu/ops/relu.cpp, clip.cpp (op -1 = clip to [p0,p1]) */
void oracle_unary(const float *x, float *y, int64_t n, int op, float p0, float p1);
/* src/backend/cpu/ops/global_avg_pool.cpp:7-28 (double accumulation) */
void oracle_global_avg_pool(const float *x, float *y, int64_t N, int64_t C, int64_t HW);
/* src/backend/cpu/ops/maxpool.cpp:7-55 */
void oracle_maxpool(const float *x, float *y, int64_t N, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t SH,
                    int64_t SW, int64_t PT, int64_t PL, int64_t OH, int64_t OW);
/* src/backend/cpu/ops/gemm.cpp:11-60. a [M][K]; b [K][N] or [N][K] (transB); c [N] or NULL. */
void oracle_gemm(const float *a, const float *b, const float *c, float *y, int64_t M, int64_t K, int64_t N, int transB,
                 float alpha, float beta, int act, float lo, float hi);
/* src/backend/cpu/ops/concat.cpp (axis 1), split.cpp (axis 1), resize.cpp (nearest; coordMode 0 half_pixel, 2 asymmetric) */
void oracle_concat_channels(const float *const *xs, const int64_t *cs, int count, float *y, int64_t N, int64_t HW);
void oracle_slice_channels(const float *x, float *y, int64_t N, int64_t Cx, int64_t c0, int64_t C, int64_t HW);
void oracle_resize_nearest(const float *x, float *y, int64_t NC, int64_t H, int64_t W, int64_t OH, int64_t OW, int coordMode);
/* src/import/fold_batchnorm.cpp:57-78: w[oc][*] *= a; b = (b - mean)*a + beta, a = gamma/sqrt(var+eps) */
void oracle_fold_bn(float *w, float *b, int64_t Cout, int64_t perOC, const float *gamma, const float *beta, const float *mean,
                    const float *var, float eps);

#ifdef __cplusplus
}
#endif
#endif
