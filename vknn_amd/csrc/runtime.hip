// The device-runtime half of the vkhip C ABI: device selection, buffers, copies, streams, events
// and stream-captured graphs. Replaces the reference's Vulkan runtime layer
// (src/backend/vulkan/vk_context.cpp, vk_buffer.cpp, vk_command.cpp) for the HIP backend.
#include "kernels/common.h"
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unistd.h>

namespace vkhip {

    static thread_local char g_err[1024] = "";
    static hipStream_t       g_stream    = nullptr;
    static int               g_inited    = 0; // 0 = not tried, 1 = ok, -1 = failed
    static std::mutex        g_init_mu;

    int set_error(int code, const char *fmt, ...) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(g_err, sizeof(g_err), fmt, ap);
        va_end(ap);
        return code;
    }

    int check_launch(const char *what) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(VKHIP_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
        return VKHIP_OK;
    }

    hipStream_t resolve_stream(vkhip_stream_t s) { return s ? (hipStream_t) s : g_stream; }

    static int hip_check(hipError_t e, const char *what) {
        if (e != hipSuccess) return set_error(VKHIP_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(e));
        return VKHIP_OK;
    }

    // Byte-fill kernel: 16-byte stores over the aligned body, bytes for the tail.
    __global__ void fill_zero_kernel(uint8_t *p, size_t bytes) {
        size_t n16 = bytes / 16;
        size_t i   = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
        size_t st  = (size_t) gridDim.x * blockDim.x;
        uint4  z   = make_uint4(0, 0, 0, 0);
        for (size_t k = i; k < n16; k += st) reinterpret_cast<uint4 *>(p)[k] = z;
        for (size_t k = n16 * 16 + i; k < bytes; k += st) p[k] = 0;
    }

    // Holds the stream for about `iters` x 3.4 us (s_sleep 127 = 127 x 64 clocks at ~2.4 GHz),
    // then exits: a bounded wait, never a spin on memory.
    __global__ void sleep_kernel(int iters) {
        for (int i = 0; i < iters; ++i) __builtin_amdgcn_s_sleep(127);
    }

} // namespace vkhip

using namespace vkhip;

extern "C" {

int vkhip_init(void) {
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_inited == 1) return VKHIP_OK;
    if (g_inited == -1) return VKHIP_ERR_NODEVICE;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        g_inited = -1;
        return set_error(VKHIP_ERR_NODEVICE, "no HIP device");
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        g_inited = -1;
        return set_error(VKHIP_ERR_NODEVICE, "hipGetDeviceProperties failed");
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_inited = -1;
        return set_error(VKHIP_ERR_NODEVICE, "device 0 is %s; this build targets gfx950 only", prop.gcnArchName);
    }
    if (hipSetDevice(0) != hipSuccess) {
        g_inited = -1;
        return set_error(VKHIP_ERR_NODEVICE, "hipSetDevice(0) failed");
    }
    if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
        g_inited = -1;
        return set_error(VKHIP_ERR_RUNTIME, "hipStreamCreate failed");
    }
    g_inited = 1;
    return VKHIP_OK;
}

int vkhip_available(void) { return vkhip_init() == VKHIP_OK ? 1 : 0; }

int vkhip_device_info(char *name, int name_len, int *cu_count, int *clock_khz, size_t *hbm_bytes) {
    int rc = vkhip_init();
    if (rc) return rc;
    hipDeviceProp_t prop;
    if ((rc = hip_check(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties"))) return rc;
    if (name && name_len > 0) snprintf(name, (size_t) name_len, "%s (%s)", prop.name, prop.gcnArchName);
    if (cu_count) *cu_count = prop.multiProcessorCount;
    if (clock_khz) *clock_khz = prop.clockRate;
    if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
    return VKHIP_OK;
}

const char *vkhip_last_error(void) { return g_err; }

const char *vkhip_build_info(void) { return "vkhip gfx950 (hipcc " __VERSION__ ")"; }

int vkhip_malloc(void **p, size_t bytes) {
    int rc = vkhip_init();
    if (rc) return rc;
    if (!p) return set_error(VKHIP_ERR_INVALID, "vkhip_malloc: null out pointer");
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    return hip_check(hipMalloc(p, bytes), "hipMalloc");
}

int vkhip_free(void *p) {
    if (!p) return VKHIP_OK;
    return hip_check(hipFree(p), "hipFree");
}

// ------------------------------------------------------------------ dma-buf interop
struct vkhip_dmabuf_s {
    hipExternalMemory_t mem = nullptr;
    void               *ptr = nullptr;
};

int vkhip_dmabuf_import(int fd, size_t bytes, vkhip_dmabuf *out, void **dev_ptr) {
    int rc = vkhip_init();
    if (rc) return rc;
    if (fd < 0 || !bytes || !out || !dev_ptr) return set_error(VKHIP_ERR_INVALID, "dmabuf_import: bad arguments");
    *out     = nullptr;
    *dev_ptr = nullptr;
    // the runtime may take the descriptor it imports: give it a duplicate, the caller keeps fd
    const int dup_fd = ::dup(fd);
    if (dup_fd < 0) return set_error(VKHIP_ERR_INVALID, "dmabuf_import: dup failed");
    hipExternalMemoryHandleDesc hd {};
    hd.type      = hipExternalMemoryHandleTypeOpaqueFd;
    hd.handle.fd = dup_fd;
    hd.size      = bytes;
    hipExternalMemory_t mem = nullptr;
    if (hipImportExternalMemory(&mem, &hd) != hipSuccess) {
        ::close(dup_fd);
        (void) hipGetLastError();
        return set_error(VKHIP_ERR_RUNTIME, "dmabuf_import: hipImportExternalMemory failed");
    }
    hipExternalMemoryBufferDesc bd {};
    bd.offset = 0;
    bd.size   = bytes;
    void *p   = nullptr;
    if (hipExternalMemoryGetMappedBuffer(&p, mem, &bd) != hipSuccess) {
        (void) hipGetLastError();
        hipDestroyExternalMemory(mem);
        return set_error(VKHIP_ERR_RUNTIME, "dmabuf_import: hipExternalMemoryGetMappedBuffer failed");
    }
    *out     = new vkhip_dmabuf_s {mem, p};
    *dev_ptr = p;
    return VKHIP_OK;
}

int vkhip_dmabuf_release(vkhip_dmabuf h) {
    if (!h) return VKHIP_OK;
    int rc = VKHIP_OK;
    if (h->ptr && hipFree(h->ptr) != hipSuccess) rc = set_error(VKHIP_ERR_RUNTIME, "dmabuf_release: hipFree of the mapping failed");
    if (h->mem && hipDestroyExternalMemory(h->mem) != hipSuccess) rc = set_error(VKHIP_ERR_RUNTIME, "dmabuf_release: hipDestroyExternalMemory failed");
    delete h;
    return rc;
}

int vkhip_dmabuf_export(const void *dev_ptr, size_t bytes, int *fd) {
    if (!dev_ptr || !bytes || !fd) return set_error(VKHIP_ERR_INVALID, "dmabuf_export: bad arguments");
    *fd = -1;
    int h = -1;
    if (hipMemGetHandleForAddressRange(&h, (hipDeviceptr_t) dev_ptr, bytes, hipMemRangeHandleTypeDmaBufFd, 0) != hipSuccess || h < 0) {
        (void) hipGetLastError();
        return set_error(VKHIP_ERR_RUNTIME, "dmabuf_export: hipMemGetHandleForAddressRange failed");
    }
    *fd = h;
    return VKHIP_OK;
}

int vkhip_memcpy_h2d(void *dst, const void *src, size_t bytes, vkhip_stream_t s) {
    if (!bytes) return VKHIP_OK;
    int rc = hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, resolve_stream(s)), "hipMemcpy H2D");
    if (rc) return rc;
    return hip_check(hipStreamSynchronize(resolve_stream(s)), "hipStreamSynchronize");
}

int vkhip_memcpy_d2h(void *dst, const void *src, size_t bytes, vkhip_stream_t s) {
    if (!bytes) return VKHIP_OK;
    int rc = hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, resolve_stream(s)), "hipMemcpy D2H");
    if (rc) return rc;
    return hip_check(hipStreamSynchronize(resolve_stream(s)), "hipStreamSynchronize");
}

int vkhip_memcpy_d2d(void *dst, const void *src, size_t bytes, vkhip_stream_t s) {
    if (!bytes) return VKHIP_OK;
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, resolve_stream(s)), "hipMemcpy D2D");
}

int vkhip_fill_zero(void *p, size_t bytes, vkhip_stream_t s) {
    if (!bytes) return VKHIP_OK;
    if (!p) return set_error(VKHIP_ERR_INVALID, "vkhip_fill_zero: null pointer");
    if (((uintptr_t) p) % 16) return set_error(VKHIP_ERR_INVALID, "vkhip_fill_zero: pointer not 16-byte aligned");
    size_t  n16    = bytes / 16 + 1;
    int64_t blocks = ceil_div((int64_t) n16, 256);
    if (blocks > 4096) blocks = 4096;
    fill_zero_kernel<<<dim3((unsigned) blocks), dim3(256), 0, resolve_stream(s)>>>((uint8_t *) p, bytes);
    return check_launch("fill_zero");
}

int vkhip_gpu_sleep(int32_t us, vkhip_stream_t s) {
    if (us < 0 || us > 100000) return set_error(VKHIP_ERR_INVALID, "vkhip_gpu_sleep: 0 .. 100000 us");
    sleep_kernel<<<dim3(1), dim3(64), 0, resolve_stream(s)>>>((us + 2) / 3);
    return check_launch("gpu_sleep");
}

int vkhip_stream_create(vkhip_stream_t *s) {
    int rc = vkhip_init();
    if (rc) return rc;
    hipStream_t st;
    if ((rc = hip_check(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate"))) return rc;
    *s = (vkhip_stream_t) st;
    return VKHIP_OK;
}

int vkhip_stream_destroy(vkhip_stream_t s) { return s ? hip_check(hipStreamDestroy((hipStream_t) s), "hipStreamDestroy") : VKHIP_OK; }

int vkhip_stream_sync(vkhip_stream_t s) { return hip_check(hipStreamSynchronize(resolve_stream(s)), "hipStreamSynchronize"); }

int vkhip_device_sync(void) { return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int vkhip_event_create(vkhip_event_t *e) {
    int rc = vkhip_init();
    if (rc) return rc;
    hipEvent_t ev;
    if ((rc = hip_check(hipEventCreate(&ev), "hipEventCreate"))) return rc;
    *e = (vkhip_event_t) ev;
    return VKHIP_OK;
}

int vkhip_event_destroy(vkhip_event_t e) { return e ? hip_check(hipEventDestroy((hipEvent_t) e), "hipEventDestroy") : VKHIP_OK; }

int vkhip_event_record(vkhip_event_t e, vkhip_stream_t s) { return hip_check(hipEventRecord((hipEvent_t) e, resolve_stream(s)), "hipEventRecord"); }

int vkhip_stream_wait_event(vkhip_stream_t s, vkhip_event_t e) {
    return hip_check(hipStreamWaitEvent(resolve_stream(s), (hipEvent_t) e, 0), "hipStreamWaitEvent");
}

int vkhip_event_sync(vkhip_event_t e) { return hip_check(hipEventSynchronize((hipEvent_t) e), "hipEventSynchronize"); }

int vkhip_event_elapsed_ms(vkhip_event_t a, vkhip_event_t b, float *ms) {
    return hip_check(hipEventElapsedTime(ms, (hipEvent_t) a, (hipEvent_t) b), "hipEventElapsedTime");
}

int vkhip_graph_begin(vkhip_stream_t s) {
    return hip_check(hipStreamBeginCapture(resolve_stream(s), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

int vkhip_graph_end(vkhip_stream_t s, vkhip_graph_t *g) {
    hipGraph_t graph = nullptr;
    int        rc    = hip_check(hipStreamEndCapture(resolve_stream(s), &graph), "hipStreamEndCapture");
    if (rc) return rc;
    hipGraphExec_t exec = nullptr;
    rc                  = hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void) hipGraphDestroy(graph);
    if (rc) return rc;
    *g = (vkhip_graph_t) exec;
    return VKHIP_OK;
}

int vkhip_graph_launch(vkhip_graph_t g, vkhip_stream_t s) { return hip_check(hipGraphLaunch((hipGraphExec_t) g, resolve_stream(s)), "hipGraphLaunch"); }

int vkhip_graph_destroy(vkhip_graph_t g) { return g ? hip_check(hipGraphExecDestroy((hipGraphExec_t) g), "hipGraphExecDestroy") : VKHIP_OK; }

} // extern "C"
