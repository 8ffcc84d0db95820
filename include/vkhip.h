/*
 * vkhip — the C-ABI seam between the vknn host code (C++) and the MI355X (gfx950) HIP kernels of
 * the fused fp16 convolution path. Plain pointers, sizes and POD descriptors; every entry point
 * returns an int status (0 = ok) and never throws. vkhip_last_error() holds the last message.
 *
 * It replaces, for the HIP backend, the reference's Vulkan device runtime and per-op dispatch:
 *   - device/buffers/streams/events/graphs  <- src/backend/vulkan/vk_context.cpp, vk_buffer.cpp,
 *                                              vk_command.cpp (submitAndWait, timestamp queries)
 *   - conv launchers                         <- src/backend/vulkan/ops/conv.cpp:491-553 (record):
 *                                              conv1x1 / split-K / conv1x1_s2 / direct / Winograd
 *   - weight prepack                         <- src/backend/vulkan/ops/conv.cpp:364-437 (prepare)
 *   - depthwise, fused dw+pw, fused SE       <- ops/conv.cpp:535-552, ops/fused_dwpw.cpp:42-111,
 *                                              ops/fused_se.cpp:134-163
 *   - pack / unpack                          <- src/backend/vulkan/vk_backend.cpp:558-696
 *   - add, channel-broadcast mul             <- ops/add.cpp:21-41, ops/binary.cpp:32-43
 *
 * Activation tensors on the device are NC4HW4 fp16: element (n,c,h,w) sits at
 * (((n*Cb + c/4)*H + h)*W + w)*4 + c%4 with Cb = ceil(C/4); lanes with c >= C hold +0.
 * Arithmetic is fp32; every fp16 activation store rounds to nearest even.
 */
#ifndef VKHIP_H
#define VKHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
#define VKHIP_OK 0
#define VKHIP_ERR_INVALID 1     /* bad argument / shape the kernel does not take */
#define VKHIP_ERR_UNSUPPORTED 2 /* valid request this build does not implement */
#define VKHIP_ERR_RUNTIME 3     /* HIP runtime error */
#define VKHIP_ERR_NODEVICE 4    /* no usable gfx950 device */

typedef void *vkhip_stream_t; /* hipStream_t; NULL = the library's own default stream */
typedef void *vkhip_event_t;  /* hipEvent_t */
typedef void *vkhip_graph_t;  /* hipGraphExec_t */

/* ---------------------------------------------------------------- runtime */
int         vkhip_init(void);      /* select device 0, create the default stream */
int         vkhip_available(void); /* 1 when a gfx950 device is present and usable */
int         vkhip_device_info(char *name, int name_len, int *cu_count, int *clock_khz, size_t *hbm_bytes);
const char *vkhip_last_error(void);
const char *vkhip_build_info(void);

int vkhip_malloc(void **p, size_t bytes);
int vkhip_free(void *p);

/* dma-buf interop (the reference's zero-copy I/O: IOTensor.dmaBufFd bound as the boundary buffer,
 * src/backend/vulkan/vk_backend.cpp:1218-1318, src/core/ion.cpp).
 *   import: map a caller's dma-buf fd (`bytes` long) into device memory; the caller keeps fd (the
 *           runtime imports a duplicate). *dev_ptr addresses the buffer until release.
 *   export: a dma-buf fd for `bytes` of device memory from vkhip_malloc (page-aligned size); the
 *           caller closes it. */
typedef struct vkhip_dmabuf_s *vkhip_dmabuf;
int vkhip_dmabuf_import(int fd, size_t bytes, vkhip_dmabuf *out, void **dev_ptr);
int vkhip_dmabuf_release(vkhip_dmabuf h);
int vkhip_dmabuf_export(const void *dev_ptr, size_t bytes, int *fd);
int vkhip_memcpy_h2d(void *dst, const void *src, size_t bytes, vkhip_stream_t s);
int vkhip_memcpy_d2h(void *dst, const void *src, size_t bytes, vkhip_stream_t s);
int vkhip_memcpy_d2d(void *dst, const void *src, size_t bytes, vkhip_stream_t s);
/* Zero `bytes` with a fill kernel (safe inside a captured graph, unlike a memset node). */
int vkhip_fill_zero(void *p, size_t bytes, vkhip_stream_t s);
/* Hold stream s for about `us` microseconds (0 .. 100000) with a one-wave kernel that sleeps and
 * exits: the host can enqueue a timed sequence behind it, so the kernels then run back to back.
 * For measurements (the plan refinement); no counterpart in the reference. */
int vkhip_gpu_sleep(int32_t us, vkhip_stream_t s);

int vkhip_stream_create(vkhip_stream_t *s);
int vkhip_stream_destroy(vkhip_stream_t s);
int vkhip_stream_sync(vkhip_stream_t s);
int vkhip_device_sync(void);

int vkhip_event_create(vkhip_event_t *e);
int vkhip_event_destroy(vkhip_event_t e);
int vkhip_event_record(vkhip_event_t e, vkhip_stream_t s);
int vkhip_event_sync(vkhip_event_t e);
/* Work issued to s after this call waits for e's last record (also inside graph capture, where it
 * forks/joins a second stream into the captured graph). */
int vkhip_stream_wait_event(vkhip_stream_t s, vkhip_event_t e);
int vkhip_event_elapsed_ms(vkhip_event_t start, vkhip_event_t stop, float *ms);

/* Stream capture into an executable graph (the analogue of a pre-recorded command buffer). */
int vkhip_graph_begin(vkhip_stream_t s);
int vkhip_graph_end(vkhip_stream_t s, vkhip_graph_t *g);
int vkhip_graph_launch(vkhip_graph_t g, vkhip_stream_t s);
int vkhip_graph_destroy(vkhip_graph_t g);

/* ---------------------------------------------------------------- activations */
#define VKHIP_ACT_NONE 0
#define VKHIP_ACT_RELU 1
#define VKHIP_ACT_RELU6 2
#define VKHIP_ACT_CLIP 3
#define VKHIP_ACT_HARDSWISH 4
#define VKHIP_ACT_SILU 5
#define VKHIP_ACT_HARDSIGMOID 6 /* clamp(lo*v + hi, 0, 1): the squeeze-excite gate (alpha = lo, beta = hi) */

/* ---------------------------------------------------------------- pack / unpack
 * NCHW fp32 (host or device memory the kernel can read) <-> NC4HW4 fp16 on the device.
 * The fp32->fp16 rounding is bit-identical to the reference host codec floatToHalf
 * (include/vknn/dtype.h:121-157: half-away-from-zero on the dropped bits, NaN -> sign|0x7E00,
 * overflow -> inf, underflow below 2^-25 -> 0), so a device pack equals the reference host pack
 * (vk_backend.cpp:576-611) bit for bit. Unpack is exact. */
int vkhip_pack_nchw_f32(const float *src, void *dst, int64_t N, int64_t C, int64_t H, int64_t W, vkhip_stream_t s);
int vkhip_unpack_nchw_f32(const void *src, float *dst, int64_t N, int64_t C, int64_t H, int64_t W, vkhip_stream_t s);
/* vkhip_unpack_nchw_f32 over `count` tensors (shapes: N, C, H, W per tensor), the ones whose H*W is
 * a multiple of 4 (and whose destination is 16-byte aligned) in one launch per 8: a segment's
 * several outputs (a detector's heads) leave in one dispatch. Same bits as one call per tensor.
 * No reference counterpart: the reference downloads each output on its own (vk_backend.cpp). */
int vkhip_unpack_nchw_f32_multi(const void *const *srcs, float *const *dsts, const int64_t *shapes, int32_t count, vkhip_stream_t s);
/* Profiling aid, no counterpart in the reference: enqueue one empty single-wave dispatch
 * (dispatch_marker_kernel) so that a kernel trace can be cut into the launches of each operator.
 * The vknn session records one before every operator when VKNN_HIP_OP_MARKERS=1. */
int vkhip_dispatch_marker(int32_t id, vkhip_stream_t s);
/* Flat (row-major) variants: a straight element-wise convert (vk_backend.cpp:559-575, 637-651). */
int vkhip_pack_flat_f32(const float *src, void *dst, int64_t n, vkhip_stream_t s);
int vkhip_unpack_flat_f32(const void *src, float *dst, int64_t n, vkhip_stream_t s);
/* NC4HW4 <-> flat row-major NCHW of one element type (elem_bytes 2: fp16, 4: fp32), a pure copy;
 * dir 0: NC4HW4 -> flat, 1: flat -> NC4HW4 (padding lanes of the last channel block written 0).
 * Replaces ops/convert_layout.cpp + shaders/convert_layout.comp:1-33 (node.subOp = dir). */
int vkhip_convert_layout(const void *src, void *dst, int64_t N, int64_t C, int64_t H, int64_t W, int32_t dir, int32_t elem_bytes,
                         vkhip_stream_t s);
/* Layout + dtype conversion between declared boundary formats, one destination element per
 * thread: fmt 0 NCHW, 1 NHWC, 2 NC4HW4 (padding lanes written 0); f16 = 1 for fp16 storage, 0 for
 * fp32. fp32 -> fp16 rounds to nearest even (unlike the host codec above), fp16 -> fp32 is exact.
 * Replaces ops/boundary_convert.{h,cpp} + shaders/boundary_convert.comp:1-58. */
int vkhip_boundary_convert(const void *src, int32_t src_fmt, int32_t src_f16, void *dst, int32_t dst_fmt, int32_t dst_f16, int64_t N,
                           int64_t C, int64_t H, int64_t W, vkhip_stream_t s);

/* ---------------------------------------------------------------- convolution
 * One descriptor covers dense (group 1) and depthwise (group == Cin == Cout) 2-D convolution
 * with a fused epilogue y = act(conv(x) + bias (+ residual)). OH/OW are the caller's (ONNX rule
 * OH = (H + pad_top + pad_bottom - (DH*(KH-1)+1))/SH + 1); only pad_top/pad_left matter. */
typedef struct vkhip_conv_desc {
    int32_t N, Cin, H, W;
    int32_t Cout, OH, OW;
    int32_t KH, KW, SH, SW, PT, PL, DH, DW;
    int32_t group;
    int32_t act;
    float   act_lo, act_hi;
    int32_t has_res; /* 1: a residual tensor of the output's shape is added before the activation
                      * (the reference's fused residual, FuseResidualAdd); 2: after it, y = act(conv
                      * + bias) + res (a standalone Add after an activated conv, e.g. the YOLOv8
                      * bottleneck shortcut; GEMM / split-K plans, not Winograd, depthwise or the
                      * stem tiles) */
    int32_t in_scale; /* 1: the input is first multiplied by a per-(image, input channel) scale
                       * (vkhip_conv_forward_scaled; dense 1x1 stride-1 pad-0 convs only) */
} vkhip_conv_desc;

/* Algorithms. GEMM is the implicit-GEMM MFMA kernel (any KHxKW/stride/pad/dilation, group 1);
 * SPLITK splits its reduction over `ksplit` workgroups and reduces fp32 partials in a second pass;
 * WINOGRAD is F(2x2,3x3) (3x3 s1 p1 d1 only): input transform, 16 batched MFMA GEMMs, output
 * transform; DEPTHWISE is the bandwidth kernel for group == C. SPLITK_LAST is SPLITK without the
 * second pass: the workgroup that finishes a tile's partials last sums them (in split order, so
 * the result does not depend on arrival order) and runs the epilogue. Its workspace holds the
 * partials, then at align256(ksplit * 16 * ceil(Cout/4) * N*OH*OW) one int arrival counter per
 * output tile: they must be zero before a workspace's first SPLITK_LAST call, and every call
 * leaves them zero (so calls that share a workspace must not overlap in time). The reference's
 * split-K (src/backend/vulkan/ops/conv.cpp:51-65,440-447) always runs a reduce dispatch. */
#define VKHIP_CONV_AUTO 0
#define VKHIP_CONV_GEMM 1
#define VKHIP_CONV_SPLITK 2
#define VKHIP_CONV_WINOGRAD 3
#define VKHIP_CONV_DEPTHWISE 4
#define VKHIP_CONV_SPLITK_LAST 5

typedef struct vkhip_conv_plan {
    int32_t algo;            /* one of VKHIP_CONV_* (never AUTO once planned) */
    int32_t tile;            /* GEMM tile configuration index (see vkhip_conv_tile_count) */
    int32_t ksplit;          /* split-K parts (SPLITK only) */
    int32_t reserved;
    size_t  weight_bytes;    /* size of the packed weight blob */
    size_t  workspace_bytes; /* device scratch the forward call needs (0 = none) */
} vkhip_conv_plan;

/* Fill `plan` for `algo` (AUTO picks by shape heuristics). `tile` < 0 picks the default tile; for
 * a depthwise conv `tile` is the number of output rows per strip of the row-tiled kernel (4, 7 or
 * 14; 0 or < 0: chosen by shape). */
int vkhip_conv_plan_make(const vkhip_conv_desc *d, int32_t algo, int32_t tile, int32_t ksplit, vkhip_conv_plan *plan);
int vkhip_conv_tile_count(void);
/* Name of the kernel family a plan launches (e.g. "conv_dma_kernel"; Winograd names its three
 * kernels joined by '+'), as a profiler shows it; for reports, no reference counterpart. */
const char *vkhip_conv_plan_kernel(const vkhip_conv_plan *plan);
/* Version of the prepacked blob layouts vkhip_conv_pack_weights (and the fused-op packers) write:
 * raised whenever any layout or the weight rounding changes. Caches of packed blobs keep it in their keys, so a blob packed
 * by another build is never taken (no counterpart in the reference, whose blobs are keyed by node
 * and role only, vk_op_common.h). */
#define VKHIP_PACK_FORMAT 5
/* Host-side prepack: fp32 OIHW weights [Cout][Cin/group][KH][KW] and optional fp32 bias[Cout]
 * into the blob the plan's kernel reads (bias stays fp32; weights become fp16, RNE). */
int vkhip_conv_pack_weights(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const float *w, const float *bias, void *blob);
/* y = act(conv(x) + bias (+ res)). x, y, res: NC4HW4 fp16 device tensors. */
int vkhip_conv_forward(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob,
                       const void *res, void *y, void *workspace, vkhip_stream_t s);
/* y = act(conv(x * xs) + bias (+ res)) for a plan made with d->in_scale = 1: xs is the
 * [N][C][1][1] channel scale as an NC4HW4 fp16 device tensor (N rows of ceil(Cin/4)*4 halves, the
 * output of a squeeze-excite branch). The product x * xs is rounded to fp16 before the
 * convolution, exactly like a separate channel-broadcast Mul (ops/binary.cpp:32-43) writing fp16,
 * so the result equals Mul followed by the conv; the scaled tensor itself never reaches memory. */
int vkhip_conv_forward_scaled(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *xs,
                              const void *blob, const void *res, void *y, void *workspace, vkhip_stream_t s);

/* vkhip_conv_forward running only some stages of a Winograd plan, for timing each kernel on its
 * own: `stages` is a mask, 1 = input transform (x -> V in the workspace), 2 = the 16 batched
 * GEMMs (V -> M), 4 = output transform (M -> y, with bias, residual and activation); 7 runs the
 * whole conv and is the only mask other plans accept. Stages read what earlier calls left in the
 * workspace. No counterpart in the reference (its Winograd records the three dispatches together,
 * src/backend/vulkan/ops/conv.cpp; for reports and tests only). */
int vkhip_conv_forward_stages(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                              void *y, void *workspace, int stages, vkhip_stream_t s);

/* vkhip_conv_forward without a workspace argument and without any allocation: the split-K
 * partials or Winograd V/M planes go to a fixed device-resident scratch array of
 * VKHIP_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. No counterpart in the
 * reference; it exists for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Plans whose workspace_bytes
 * exceed the maximum are rejected with VKHIP_ERR_INVALID. Every call on one GPU shares that GPU's
 * scratch, which keeps the last call's contents: calls that overlap in time on one GPU (two
 * streams, or two host threads) race and must be serialised by the caller. */
#define VKHIP_NOALLOC_SCRATCH_BYTES ((size_t) 64 << 20)
/* SPLITK_LAST plans keep their arrival counters in a separate device array of this many ints per
 * GPU (zero at load, left zero by every call); plans with more output tiles are rejected. */
#define VKHIP_NOALLOC_MAX_TILES 16384
/* Depthwise conv that also leaves, for a following global average pool, the sum of its stored fp16
 * outputs per (plane, row tile): pool is [N*ceil(C/4)][R] x 4 fp32, R = vkhip_conv_pool_parts
 * (0: the plan's kernel cannot; then use vkhip_conv_forward and vkhip_global_avg_pool). y is
 * exactly what vkhip_conv_forward writes. No counterpart in the reference (its GlobalAveragePool
 * re-reads the conv output, cpu/ops/global_avg_pool.cpp:7-28). */
int vkhip_conv_pool_parts(const vkhip_conv_desc *d, const vkhip_conv_plan *plan);
int vkhip_conv_forward_pooled(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res,
                              void *y, void *pool, vkhip_stream_t s);

/* vkhip_conv_forward on views: x and y may point into wider NC4HW4 tensors, `x_pstride` /
 * `y_pstride` channel blocks (4-channel planes) per image apart instead of ceil(Cin/4) /
 * ceil(Cout/4) (0 = dense). This lets a conv read a channel slice of a tensor (a Split output) and
 * write straight into its slice of a channel Concat, so neither is copied. GEMM and split-K plans
 * only (not the stem tiles, Winograd or depthwise), no residual, no input scale. No counterpart in
 * the reference, whose Concat and Split copy (ops/concat.cpp, ops/split.cpp). */
int vkhip_conv_forward_view(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, int64_t x_pstride, const void *blob,
                            void *y, int64_t y_pstride, void *workspace, vkhip_stream_t s);

/* vkhip_conv_forward_view for a conv with a residual (has_res 1 or 2): `res` is read with y's
 * layout, i.e. `y_pstride` channel blocks per image (a slice of the same concat as y, as in a
 * YOLOv8 C2f block, or a dense tensor when y is dense). The reference has no view entry points:
 * its Add (src/backend/cpu/ops/add.cpp) after the conv and its in-place concat are what this
 * call replaces. */
int vkhip_conv_forward_view_res(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, int64_t x_pstride, const void *blob,
                                const void *res, void *y, int64_t y_pstride, void *workspace, vkhip_stream_t s);

/* ---------------------------------------------------------------- two 3x3 convs in one kernel
 * y = act2(conv2(act1(conv1(x)) rounded to fp16)) (+ x when c2->has_res == 2: the residual is the
 * pair's input, added after act2), for two dense 3x3 stride-1 pad-1 convs with 9-32 channels in,
 * between and out (all equal) and an even width: the YOLOv8 bottleneck (cv1, cv2 and its
 * shortcut) and the C2f head pairs. The intermediate tensor stays in LDS. Weights: each conv's
 * blob packed by vkhip_conv_pack_weights with the plan vkhip_conv3x3_pair_plan returns for it
 * (c2's plan is made with has_res 0). x and y may be views (plane strides as in
 * vkhip_conv_forward_view; 0 = dense). No reference counterpart: the reference runs the two
 * ConvCpu calls (src/backend/cpu/ops/conv.cpp:9-92) and its Add (src/backend/cpu/ops/add.cpp). */
int vkhip_conv3x3_pair_plan(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, vkhip_conv_plan *p1, vkhip_conv_plan *p2);
int vkhip_conv3x3_pair_forward(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, const void *x, int64_t x_pstride, const void *blob1,
                               const void *blob2, void *y, int64_t y_pstride, vkhip_stream_t s);

/* ---------------------------------------------------------------- two stride-2 stem convs in one kernel
 * y = act2(conv2(act1(conv1(x)) rounded to fp16)) for two dense 3x3 stride-2 pad-1 convs, the first
 * over at most 4 input channels to 9-16 channels, the second to at most 32 (the YOLOv8n stem,
 * 3 -> 16 -> 32), with an even input width; the intermediate tensor stays in LDS. With c3 (else
 * NULL): a dense 1x1 conv over the second conv's output (at most 32 out, the next layer when it is
 * the second conv's only reader) runs in the same kernel, y is its output and the second conv's
 * output stays in LDS too. x is a dense NC4HW4 tensor; y may be a view (`y_pstride` channel blocks
 * per image; 0 = dense). Weights: each conv's blob packed by vkhip_conv_pack_weights with the plan
 * vkhip_conv3x3s2_pair_plan returns for it. No reference counterpart: the reference runs the
 * ConvCpu calls one by one (src/backend/cpu/ops/conv.cpp:9-92). */
int vkhip_conv3x3s2_pair_plan(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, const vkhip_conv_desc *c3, vkhip_conv_plan *p1,
                              vkhip_conv_plan *p2, vkhip_conv_plan *p3);
int vkhip_conv3x3s2_pair_forward(const vkhip_conv_desc *c1, const vkhip_conv_desc *c2, const vkhip_conv_desc *c3, const void *x, const void *blob1,
                                 const void *blob2, const void *blob3, void *y, int64_t y_pstride, vkhip_stream_t s);

/* ---------------------------------------------------------------- a stem and its first block in one kernel
 * y = actp(Wp * rnd(actd(dw3x3(s))) + bp [+ s]) with s = rnd(acta(conv3x3s2(x))): a dense 3x3
 * stride-2 pad-1 conv over at most 4 input channels to 9-16 channels (cs), a 3x3 stride-1 pad-1
 * depthwise conv over them (cd) and a dense 1x1 projection to at most 16 channels (cp; has_res 1:
 * the residual is the stem's output, Cout equal to the stem's). The MobileNetV3 stem and first
 * inverted-residual block (3 -> 16 -> dw 16 -> 16 + x); both 16-channel tensors stay in LDS. x is
 * a dense NC4HW4 tensor with an even width; y may be a view (`y_pstride` channel blocks per image;
 * 0 = dense). Weights: each conv's blob packed by vkhip_conv_pack_weights with the plan
 * vkhip_stem_dwpw_plan returns for it. No reference counterpart: the reference runs ConvCpu
 * (src/backend/cpu/ops/conv.cpp:9-92) and then FusedDwPw (src/backend/cpu/ops/fused_dwpw.cpp:10-87). */
int vkhip_stem_dwpw_plan(const vkhip_conv_desc *cs, const vkhip_conv_desc *cd, const vkhip_conv_desc *cp, vkhip_conv_plan *ps,
                         vkhip_conv_plan *pd, vkhip_conv_plan *pp);
int vkhip_stem_dwpw_forward(const vkhip_conv_desc *cs, const vkhip_conv_desc *cd, const vkhip_conv_desc *cp, const void *x, const void *blob_s,
                            const void *blob_d, const void *blob_p, void *y, int64_t y_pstride, vkhip_stream_t s);

int vkhip_conv_forward_noalloc(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob,
                               const void *res, void *y, vkhip_stream_t s);

/* ---------------------------------------------------------------- fused depthwise + 1x1 project
 * Reference FusedDwPw (src/backend/cpu/ops/fused_dwpw.cpp:10-87): t = dw_act(dwconv(x) + dw_b)
 * with dw_act in {None, Relu, Relu6}; y = act(W_pw t + pw_b (+ res)). The E-channel intermediate
 * stays on chip. The descriptor's Cin/Cout/act describe the dw stage (Cout == Cin == E). */
typedef struct vkhip_dwpw_desc {
    vkhip_conv_desc dw;
    int32_t         Cout;
    int32_t         act;
    float           act_lo, act_hi;
    int32_t         has_res;
} vkhip_dwpw_desc;
int    vkhip_dwpw_supported(const vkhip_dwpw_desc *d);
size_t vkhip_dwpw_weight_bytes(const vkhip_dwpw_desc *d);
int    vkhip_dwpw_pack_weights(const vkhip_dwpw_desc *d, const float *dw_w, const float *dw_b, const float *pw_w,
                               const float *pw_b, void *blob);
int    vkhip_dwpw_forward(const vkhip_dwpw_desc *d, const void *x, const void *blob, const void *res, void *y, vkhip_stream_t s);

/* ---------------------------------------------------------------- fused 3x3 + 1x1
 * A bottleneck's 3x3 conv and the 1x1 conv that is the only reader of its output, as one kernel:
 * t = conv.act(conv3x3(x) + b3) rounded to fp16 as the 3x3's own store would round it, then
 * y = act(W1 t + b1 (+ res)). The reference runs them as two Conv nodes (ConvCpu,
 * src/backend/cpu/ops/conv.cpp:9-92, each with its fused epilogue); the intermediate never reaches
 * memory here. No reference counterpart as an entry point. conv: the 3x3 (pad 1, stride 1 or 2,
 * even W, Cin a multiple of 16, Cout = the mid width 64, has_res = 0); Cout, act and
 * has_res: the 1x1 (stride 1, no padding). */
typedef struct vkhip_convpw_desc {
    vkhip_conv_desc conv;
    int32_t         Cout;
    int32_t         act;
    float           act_lo, act_hi;
    int32_t         has_res;
} vkhip_convpw_desc;
/* VKHIP_ERR_UNSUPPORTED when no fused kernel fits the shapes; weight_bytes = the whole blob. */
int vkhip_convpw_plan(const vkhip_convpw_desc *d, vkhip_conv_plan *plan);
/* w3 [Cmid][Cin][3][3], w1 [Cout][Cmid] fp32 (rounded to fp16, RNE), biases fp32 or null. */
int vkhip_convpw_pack_weights(const vkhip_convpw_desc *d, const vkhip_conv_plan *plan, const float *w3, const float *b3, const float *w1,
                              const float *b1, void *blob);
int vkhip_convpw_forward(const vkhip_convpw_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res, void *y,
                         vkhip_stream_t s);
/* The pair above chained with a second 1x1 that reads the pair's output (the next bottleneck's
 * reduction): y2 = act3(W2 y + b2), accumulated chunk by chunk from the fp16 values the pair stores
 * to y, so y is written once and not read back. 64 mid channels and Cout3 <= 64 only; y is still
 * written in full (the next block's residual). No reference counterpart (three Conv nodes there). */
typedef struct vkhip_convpw2_desc {
    vkhip_convpw_desc pw;
    int32_t           Cout3;
    int32_t           act3;
    float             act3_lo, act3_hi;
} vkhip_convpw2_desc;
int vkhip_convpw2_plan(const vkhip_convpw2_desc *d, vkhip_conv_plan *plan);
/* w2 [Cout3][pw.Cout] fp32, b2 [Cout3] or null; the rest as vkhip_convpw_pack_weights. */
int vkhip_convpw2_pack_weights(const vkhip_convpw2_desc *d, const vkhip_conv_plan *plan, const float *w3, const float *b3, const float *w1,
                               const float *b1, const float *w2, const float *b2, void *blob);
int vkhip_convpw2_forward(const vkhip_convpw2_desc *d, const vkhip_conv_plan *plan, const void *x, const void *blob, const void *res, void *y,
                          void *y2, vkhip_stream_t s);

/* ---------------------------------------------------------------- squeeze-excite + pooling
 * Global average pool: x [N,C,H,W] -> y [N,C,1,1] (both NC4HW4 fp16; fp32 accumulation). */
int vkhip_global_avg_pool(const void *x, void *y, int64_t N, int64_t C, int64_t H, int64_t W, vkhip_stream_t s);
/* Fused SE middle (reference FusedSE, src/backend/cpu/ops/fused_se.cpp:9-47):
 * s = clamp(alpha*(W2 relu(W1 avg + b1) + b2) + beta, 0, 1). avg/y: NC4HW4 fp16 [N,C,1,1].
 * Two skinny-GEMM launches over the whole batch (the vkhip_fc kernel): relu(W1 avg + b1) into the
 * workspace ([N,Cr,1,1] fp16, vkhip_se_workspace_bytes), then the gated W2 product into y. w1 is
 * [Cr][C], w2 [C][Cr] (fp32, rounded to fp16 by the pack); the blob holds both fc blobs. */
size_t vkhip_se_weight_bytes(int64_t C, int64_t Cr);
size_t vkhip_se_workspace_bytes(int64_t N, int64_t Cr);
int    vkhip_se_pack_weights(int64_t C, int64_t Cr, const float *w1, const float *b1, const float *w2, const float *b2, void *blob);
int    vkhip_fused_se(const void *avg, const void *blob, void *y, int64_t N, int64_t C, int64_t Cr, float alpha, float beta,
                      void *workspace, vkhip_stream_t s);
/* vkhip_fused_se whose avg is not in memory: the squeeze input is formed from the R fp32 partial
 * sums per (image, 4-channel block) that vkhip_conv_forward_pooled left ([N][ceil(C/4)][R] x 4
 * floats), as fp16(sum / HW), the value vkhip_global_avg_pool would have stored. Folds the
 * reference's GlobalAveragePool (cpu/ops/global_avg_pool.cpp) into the depthwise conv before it
 * and the first FC after it; no counterpart of its own in the reference. */
int    vkhip_fused_se_pooled(const void *part, int32_t R, int64_t HW, const void *blob, void *y, int64_t N, int64_t C, int64_t Cr,
                             float alpha, float beta, void *workspace, vkhip_stream_t s);
/* y = x * scale[n,c] (channel broadcast; reference Binary Mul BCAST, ops/binary.cpp:32-43). */
int vkhip_channel_scale(const void *x, const void *scale, void *y, int64_t N, int64_t C, int64_t HW, vkhip_stream_t s);

/* ---------------------------------------------------------------- element-wise
 * y = act(a + b) over `n` packed fp16 elements (reference Add same-shape path, add.cpp:67-86). */
int vkhip_add(const void *a, const void *b, void *y, int64_t n, int32_t act, float lo, float hi, vkhip_stream_t s);
/* vkhip_add over views (plane strides per image as in vkhip_conv_forward_view; 0 = dense) of
 * N x C x HW NC4HW4 tensors. */
int vkhip_add_view(const void *a, int64_t a_pstride, const void *b, int64_t b_pstride, void *y, int64_t y_pstride, int64_t N, int64_t C,
                   int64_t HW, int32_t act, float lo, float hi, vkhip_stream_t s);
/* y = op(x) on `n` packed fp16 elements; op is a vknn UnaryType code (Sigmoid 0, HardSwish 2,
 * HardSigmoid 3 with alpha/beta in p0/p1, Relu 13, SiLU 14) or, with unary = -1, a clip to [p0,p1]. */
int vkhip_unary(const void *x, void *y, int64_t n, int32_t unary, float p0, float p1, vkhip_stream_t s);
/* Element-wise binary on equal shapes (BinaryType code: Mul 0, Sub 1, Div 2, Max 3, Min 4, Add 6). */
int vkhip_binary(const void *a, const void *b, void *y, int64_t n, int32_t op, vkhip_stream_t s);

/* ---------------------------------------------------------------- whole-network data movement */
typedef struct vkhip_pool_desc {
    int32_t N, C, H, W, OH, OW, KH, KW, SH, SW, PT, PL;
} vkhip_pool_desc;
int vkhip_maxpool(const vkhip_pool_desc *d, const void *x, void *y, vkhip_stream_t s);
/* vkhip_maxpool over views (plane strides per image; 0 = dense). */
int vkhip_maxpool_view(const vkhip_pool_desc *d, const void *x, int64_t x_pstride, void *y, int64_t y_pstride, vkhip_stream_t s);
/* `count` (1-4) same-size max pools in a chain, one launch: ys[0] = pool(x), ys[k] = pool(ys[k-1])
 * for a KxK (K = 3 or 5) stride-1 pad-K/2 pool whose plane fits LDS (the SPPF block of a detector
 * neck); every output may be a view (y_pstrides[k]; 0 = dense). Bit-identical to `count`
 * vkhip_maxpool_view calls. No reference counterpart: the reference runs its MaxPool
 * (src/backend/cpu/ops/maxpool.cpp) once per node. */
int vkhip_maxpool_chain(const vkhip_pool_desc *d, const void *x, int64_t x_pstride, void *const *ys, const int64_t *y_pstrides, int32_t count,
                        vkhip_stream_t s);
/* A first-layer conv (at most 4 input channels, 3x3 or 7x7, stride 1 or 2, pad K/2, <= 64 output
 * channels, no residual) followed by a 3x3 stride-2 pad-1 max pool over its output, in one
 * kernel: y = maxpool(act(conv(x) + bias)), bit-identical to vkhip_conv_forward then
 * vkhip_maxpool, without the conv output in memory. The plan must be a stem-kernel plan with
 * 64-row tiles (vkhip_conv_plan_make with tile 21 or 22), or the 64-output thin plan (tile 45) for a
 * 7x7 stride-2 pad-3 conv over an even input width (the ResNet stem), and its packed blob. No
 * counterpart in the reference, which runs the two as separate ops (ops/conv.cpp, ops/pool.cpp). */
int vkhip_conv_maxpool_supported(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p);
int vkhip_conv_maxpool_forward(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p, const void *x, const void *blob,
                               void *y, vkhip_stream_t s);
/* Fully connected y[N,M] = act(x[N,K] W^T + b): x/y are [N,C,1,1] NC4HW4 fp16 tensors.
 * Blob: fp16 W[Mp][Kp] followed by fp32 b[Mp], Mp = M rounded up to 16, Kp = K rounded up to 32,
 * zero padded (vkhip_fc_weight_bytes). One skinny-GEMM kernel: 16 x 16/32 output tiles, K split
 * over 8 waves. */
size_t vkhip_fc_weight_bytes(int64_t K, int64_t M);
int    vkhip_fc_pack_weights(int64_t K, int64_t M, const float *w, int32_t transB, const float *b, float alpha, float beta, void *blob);
int    vkhip_fc(const void *x, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act, float lo, float hi,
                vkhip_stream_t s);
/* vkhip_fc with x formed from pooled partial sums as in vkhip_fused_se_pooled (K channels, R
 * partials per 4-channel block, HW pixels per plane). */
int    vkhip_fc_pooled(const void *part, int32_t R, int64_t HW, const void *blob, void *y, int64_t N, int64_t K, int64_t M, int32_t act,
                       float lo, float hi, vkhip_stream_t s);
/* Channel concat of `count` NC4HW4 inputs (any channel counts) into y. */
int vkhip_concat_channels(const void *const *xs, const int64_t *cs, int32_t count, void *y, int64_t N, int64_t HW,
                          vkhip_stream_t s);
/* Channel slice [c0, c0+C) of x (Cx channels) into y (C channels). */
int vkhip_slice_channels(const void *x, void *y, int64_t N, int64_t Cx, int64_t c0, int64_t C, int64_t HW, vkhip_stream_t s);
/* Nearest-neighbour resize: y[oy,ox] = x[floor(oy*H/OH), floor(ox*W/OW)]. For integer upscale
 * factors this is the reference's nearest (round_prefer_floor, src/backend/cpu/ops/resize.cpp:30-87)
 * under half_pixel and pytorch_half_pixel coordinates, and under asymmetric ones up to 2x. */
int vkhip_resize_nearest(const void *x, void *y, int64_t N, int64_t C, int64_t H, int64_t W, int64_t OH, int64_t OW,
                         vkhip_stream_t s);
/* vkhip_resize_nearest over views (plane strides per image; 0 = dense). */
int vkhip_resize_nearest_view(const void *x, int64_t x_pstride, void *y, int64_t y_pstride, int64_t N, int64_t C, int64_t H, int64_t W,
                              int64_t OH, int64_t OW, vkhip_stream_t s);

#ifdef __cplusplus
}
#endif
#endif /* VKHIP_H */
