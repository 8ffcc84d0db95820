"""Zero-copy dma-buf I/O (vknn_session_run_dmabuf; reference IOTensor.dmaBufFd bound as the
boundary GPU buffer, src/backend/vulkan/vk_backend.cpp:1218-1318). The dma-bufs are device
allocations exported with vkhip_dmabuf_export (hipMemGetHandleForAddressRange), the form a camera
or another GPU client hands over; the session imports each fd (hipImportExternalMemory), reads
the input from it in its declared layout and writes the output into the output fd.

The input values are fp16-representable, so the declared-format converter (fp32 -> fp16 rounds to
nearest even) and the host pack (the reference host codec) store the same halves, and every
zero-copy result must equal the host path bit for bit."""
import ctypes

import numpy as np
import pytest

import vknn_amd as V

pytestmark = pytest.mark.gpu
ALIGN = 2 << 20


def _export(buf):
    fd = ctypes.c_int(-1)
    if V.vkhip().vkhip_dmabuf_export(buf.ptr, buf.nbytes, ctypes.byref(fd)):
        pytest.skip("dma-buf export unavailable here: " + V.vkhip().vkhip_last_error().decode(errors='replace'))
    return fd.value


def _nc4(x):
    n, c, h, w = x.shape
    cp = (c + 3) // 4 * 4
    p = np.zeros((n, cp, h, w), x.dtype)
    p[:, :c] = x
    return np.ascontiguousarray(p.reshape(n, cp // 4, 4, h, w).transpose(0, 1, 3, 4, 2))


@pytest.mark.parametrize("model,batch", [("resnet_tiny", 2), ("mnv3_tiny", 2)])
def test_dmabuf_io_matches_host_path(gpu, model, batch):
    import os
    s = V.Session(model, batch, seed=3)
    n_in, n_out = int(np.prod(s.in_shape)), sum(s.out_elems)
    x = np.random.default_rng(8).standard_normal(s.in_shape).astype(np.float16).astype(np.float32)
    ref = s.run(x)
    inb, outb = V.DeviceBuffer(ALIGN * ((n_in * 4) // ALIGN + 1)), V.DeviceBuffer(ALIGN * ((n_out * 4) // ALIGN + 1))
    in_fd, out_fd = _export(inb), _export(outb)
    try:
        lib = V.vknn()
        cases = [
            ("nchw f32 in/out", x, 0, 0, 0, 0, lambda y: y, np.float32),
            ("nhwc f16 in", x.transpose(0, 2, 3, 1).astype(np.float16), 1, 1, 0, 0, lambda y: y, np.float32),
            ("device-native in", _nc4(x.astype(np.float16)), 3, 1, 0, 0, lambda y: y, np.float32),
            ("nchw f16 out", x, 0, 0, 0, 1, lambda y: y.astype(np.float16), np.float16),
        ]
        for what, xin, ifmt, if16, ofmt, of16, conv, odt in cases:
            print(f"{model}: {what}", flush=True)
            inb.upload(np.ascontiguousarray(xin))
            outb.zero()
            y = np.zeros(n_out, np.float32)
            for _ in range(2):  # the second run reuses the cached imports (and a captured graph)
                rc = lib.vknn_session_run_dmabuf(s.h, in_fd, ifmt, if16, out_fd, ofmt, of16, y.ctypes.data, y.size)
                assert rc == 0, lib.vknn_last_error().decode(errors='replace')
                got = outb.download(odt, s.out_elems[0])
                want = conv(ref[:s.out_elems[0]])
                assert np.array_equal(got.view(np.uint16 if odt == np.float16 else np.uint32),
                                      np.asarray(want, odt).view(np.uint16 if odt == np.float16 else np.uint32)), what
        # back to the host path on the same session
        assert np.array_equal(s.run(x), ref)
    finally:
        os.close(in_fd)
        os.close(out_fd)
        s.close()
        inb.close()
        outb.close()
