/*
 * vknn_c — a C ABI over the vknn Session with the HIP backend, for callers that cannot use the
 * C++ API (Python ctypes in the tests and the benchmark). The reference has no C API; its public
 * surface is the C++ Session/Model (include/vknn/session_class.h:18-85, model_class.h:14-54).
 * These entry points wrap exactly that: build a graph (here: a named model from the built-in
 * zoo), Session::create with BackendKind::Hip, run.
 *
 * Options string: ';'-separated key=value pairs, all optional:
 *   winograd=auto|on|off   tuning=off|fast|thorough   graphs=0|1   profile=0|1
 *   fuse_dwpw=0|1          fuse_se=0|1
 */
#ifndef VKNN_C_H
#define VKNN_C_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vknn_session_s *vknn_session;

const char *vknn_last_error(void);

/* Input shape (4 dims) and the number of outputs / their element counts of a zoo model. */
int vknn_model_io(const char *model, int64_t batch, int64_t *in_shape4, int64_t *out_elems, int32_t *n_out, int32_t max_out);
/* Algorithmic conv + FC FLOPs per image of a zoo model. */
double vknn_model_flops(const char *model);

int vknn_session_create_model(const char *model, int64_t batch, uint64_t seed, const char *options, vknn_session *out);
int vknn_session_destroy(vknn_session s);
/* Host path: x (NCHW fp32) in, all outputs (NCHW fp32, concatenated in graph order) out. */
int vknn_session_run_host(vknn_session s, const float *x, int64_t nx, float *y, int64_t ny);
/* Zero-copy run (reference IOTensor.dmaBufFd, io_tensor.h:10-23, Session::run output bindings,
 * session_class.h:34-37): the single input is read from the dma-buf `in_fd`, converted from its
 * declared layout (0 NCHW, 1 NHWC, 2 NC4HW4, 3 device-native = NC4HW4 fp16) and dtype (in_f16);
 * with out_fd >= 0 the first output is written into that dma-buf in its declared layout, and the
 * run returns once it is there; other outputs (or all, with out_fd < 0) land in y as fp32 NCHW.
 * Imports are cached while the same buffer comes back. */
int vknn_session_run_dmabuf(vknn_session s, int32_t in_fd, int32_t in_fmt, int32_t in_f16, int32_t out_fd, int32_t out_fmt, int32_t out_f16,
                            float *y, int64_t ny);
/* Device path: the input is read from device memory (NCHW fp32, e.g. from vkhip_malloc); the run
 * is enqueued on the session stream and returns without waiting. */
int vknn_session_bind_device_input(vknn_session s, const float *dev_x);
/* Same, from a declared layout (0 NCHW, 1 NHWC, 2 NC4HW4) and element type (f16 = 1: fp16,
 * 0: fp32), converted on the device by vkhip_boundary_convert (fp32 -> fp16 rounds to nearest
 * even), like the reference's declared-format dma-buf input (vk_backend.cpp:1218-1318). */
int vknn_session_bind_device_input_as(vknn_session s, const void *dev_x, int32_t fmt, int32_t f16);
int vknn_session_run_device(vknn_session s);
int vknn_session_sync(vknn_session s);
/* Device pointer of output k (NCHW fp32, valid after a run completes). */
const float *vknn_session_device_output(vknn_session s, int32_t k);
int vknn_session_read_outputs(vknn_session s, float *y, int64_t ny);
void *vknn_session_stream(vknn_session s);
/* Per-op profile of the last profiled run (JSON array) and the per-op kernel plan (text). */
int vknn_session_profile_json(vknn_session s, char *buf, int64_t cap);
int vknn_session_describe(vknn_session s, char *buf, int64_t cap);
/* The session's segments in run order, one line each: "<backend> nodes=<n> in=<names,> out=<names,>". */
int vknn_session_segments(vknn_session s, char *buf, int64_t cap);
/* Number of nodes of one op type (e.g. "Conv", "FusedDwPw") in the session's planned graph. */
int vknn_session_count_ops(vknn_session s, const char *op_type_name);
/* Host only (no device needed): run the standard passes on a zoo model and write the resulting
 * node list, one node per line: "<OpType> <name> act=<ActType> res=<0|1> out=<shape>". */
int vknn_graph_after_passes(const char *model, int64_t batch, const char *options, char *buf, int64_t cap);

/* The ".vxm" model file (reference VXM2 layout, src/core/model_io.cpp; Session::createFromVxm and
 * saveOptimized, src/core/session.cpp:133-159).
 *   save_vxm: build a zoo model, run the standard passes (options: fuse_dwpw, fuse_se; passes=0
 *             skips them) and write the graph with its weights; host only.
 *   vxm_describe: load a .vxm and write its node list in the vknn_graph_after_passes format; host only.
 *   session_create_vxm: plan a session from a .vxm (passes are not re-run); an empty cache_file
 *             option means "<path without extension>.cache", as in the reference.
 *   session_save_optimized: write a session's planned graph; needs "keep_weights=1" at creation. */
int vknn_model_save_vxm(const char *model, int64_t batch, uint64_t seed, const char *options, const char *path);
int vknn_vxm_describe(const char *path, char *buf, int64_t cap);
int vknn_session_create_vxm(const char *path, const char *options, vknn_session *out);
int vknn_session_save_optimized(vknn_session s, const char *path);

/* ONNX models (reference include/vknn/graph.h:42 importOnnx, src/core/session.cpp:123-131
 * Session::createFromOnnx).
 *   onnx_describe: import a model and write the graph as imported (before any pass) in full:
 *             tensors, inputs, outputs, initializer hashes, nodes with attributes; host only.
 *   onnx_after_passes: the node list after the standard passes (vknn_graph_after_passes format);
 *             options fuse_dwpw, fuse_se; host only.
 *   session_create_onnx: import and plan a session; an empty cache_file option means
 *             "<path without extension>.cache", as in the reference. */
int vknn_onnx_describe(const char *path, char *buf, int64_t cap);
int vknn_onnx_after_passes(const char *path, const char *options, char *buf, int64_t cap);
int vknn_session_create_onnx(const char *path, const char *options, vknn_session *out);

/* Persistent autotune table (the tune section of the reference's unified cache file "VKNNCAC1",
 * src/backend/vulkan/vk_backend.cpp:30-150 and :440-545). A session created with the option
 * "cache_file=<path>" (and cache_mode tune or full, the default full) merges the file's table
 * before compiling and writes it back afterwards when it changed. These calls reach the same
 * process-wide table directly; none needs a device.
 *   load: merge a file's entries (once per path), returns the number of tune entries read (0 if
 *         absent/unknown); its prepacked weight blobs are kept too, as with CacheMode::Full
 *   save: write the table and the weight blobs (untouched when the bytes are unchanged);
 *   get: 0 found, 1 absent; weight_cache_stats: blobs held, and lookups that found / missed one */
int vknn_tune_cache_load(const char *path);
int vknn_tune_cache_save(const char *path);
int vknn_tune_cache_put(const char *key, int32_t value);
int vknn_tune_cache_get(const char *key, int32_t *value);
int vknn_tune_cache_clear(void);
int vknn_tune_cache_stats(int64_t *entries, int64_t *hits, int64_t *misses);
int vknn_weight_cache_stats(int64_t *entries, int64_t *hits, int64_t *misses);
/* The key namespace of this device ("hip-<arch>-<CUs>cu"); needs the device. */
int vknn_tune_cache_gpu_tag(char *buf, int64_t cap);

#ifdef __cplusplus
}
#endif
#endif
