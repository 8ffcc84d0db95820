"""The ".vxm" model file (reference src/core/model_io.cpp, VXM2 layout; Session::createFromVxm /
saveOptimized, src/core/session.cpp:133-159).

The layout is pinned against the reference's own writer and reader, compiled from its sources
into oracle/_ref/libvknn_ref.so: the same graph written by both is byte-identical, and a file
written here is read and re-written unchanged by the reference. GPU tests check that a session
planned from a .vxm computes exactly what the session built from the model does."""
import ctypes
import struct

import numpy as np
import pytest

import oracle_lib as O
import vknn_amd as V

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference sources absent)")

MODELS = [("conv3x3_bn_relu", 1, ""), ("mnv2_block", 2, ""), ("resnet_tiny", 2, ""), ("mnv3_tiny", 1, "fuse_se=1;fuse_dwpw=1"),
          ("yolo_tiny", 1, ""), ("resnet50", 1, "")]


def ref_api():
    r = O.ref()
    r.ref_save_vxm.restype = ctypes.c_int
    r.ref_save_vxm.argtypes = [ctypes.c_char_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_char_p]
    r.ref_vxm_resave.restype = ctypes.c_int
    r.ref_vxm_resave.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
    return r


def save(model, batch, path, options="", seed=5):
    lib = V.vknn()
    assert lib.vknn_model_save_vxm(model.encode(), batch, seed, options.encode(), str(path).encode()) == 0, lib.vknn_last_error()


def describe(path):
    lib = V.vknn()
    buf = ctypes.create_string_buffer(1 << 20)
    rc = lib.vknn_vxm_describe(str(path).encode(), buf, len(buf))
    return (buf.value.decode() if rc == 0 else None), lib.vknn_last_error().decode(errors='replace')


@needs_ref
@pytest.mark.parametrize("model,batch,opts", MODELS)
def test_writer_matches_reference_writer(tmp_path, model, batch, opts):
    """The zoo graph as built, written by this build and by the reference: identical bytes."""
    ours, theirs = tmp_path / "ours.vxm", tmp_path / "ref.vxm"
    save(model, batch, ours, "passes=0")
    assert ref_api().ref_save_vxm(model.encode(), batch, 5, 0, str(theirs).encode()) == 0
    assert ours.read_bytes() == theirs.read_bytes()


@needs_ref
@pytest.mark.parametrize("model,batch,opts", MODELS)
def test_reference_reads_optimized_file_unchanged(tmp_path, model, batch, opts):
    """A post-pass graph written here (fused activations, residuals, dw+pw / SE nodes) is read by
    the reference's loader and written back byte for byte."""
    ours, back = tmp_path / "ours.vxm", tmp_path / "back.vxm"
    save(model, batch, ours, opts)
    assert ref_api().ref_vxm_resave(str(ours).encode(), str(back).encode()) == 0
    assert back.read_bytes() == ours.read_bytes()


@needs_ref
@pytest.mark.parametrize("model,batch", [("resnet_tiny", 2), ("mnv3_tiny", 1), ("yolo_tiny", 1)])
def test_reads_reference_optimized_file(tmp_path, model, batch):
    """A file the reference session wrote after its own passes loads here."""
    theirs = tmp_path / "ref_opt.vxm"
    assert ref_api().ref_save_vxm(model.encode(), batch, 5, 1, str(theirs).encode()) == 0
    text, err = describe(theirs)
    assert text is not None, err
    assert len(text.splitlines()) > 3


@pytest.mark.parametrize("model,batch,opts", MODELS)
def test_optimized_file_holds_the_planned_graph(tmp_path, model, batch, opts):
    f = tmp_path / "m.vxm"
    save(model, batch, f, opts)
    text, err = describe(f)
    assert text == V.graph_after_passes(model, batch, opts), err


def test_header_layout(tmp_path):
    """Magic "VXM2", then the tensor table: u32 count, then per tensor str name, vec<i64> shape,
    u32 dtype, u32 format, u32 flags."""
    f = tmp_path / "c.vxm"
    save("conv3x3_bn_relu", 1, f, "passes=0")
    b = f.read_bytes()
    assert b[:4] == b"VXM2"
    nt, = struct.unpack_from("<I", b, 4)
    assert nt > 2
    off = 8
    kl, = struct.unpack_from("<I", b, off)
    name = b[off + 4:off + 4 + kl].decode()
    off += 4 + kl
    nd, = struct.unpack_from("<I", b, off)
    dims = struct.unpack_from(f"<{nd}q", b, off + 4)
    off += 4 + 8 * nd
    dtype, fmt, flags = struct.unpack_from("<III", b, off)
    # the first tensor of the config-0 graph is its NCHW fp32 input
    assert name and dims == (1, 64, 56, 56) and (dtype, fmt, flags) == (0, 0, 1)


def test_rejects_truncated_and_foreign_files(tmp_path):
    f = tmp_path / "r.vxm"
    save("resnet_tiny", 1, f, "")
    b = f.read_bytes()
    cut = tmp_path / "cut.vxm"
    for n in sorted({0, 3, 4, 8, 50, len(b) // 3, len(b) // 2, len(b) - 9, len(b) - 1}):
        cut.write_bytes(b[:n])
        text, err = describe(cut)
        assert text is None and ("truncated" in err or "magic" in err or "out of range" in err), (n, err)
    cut.write_bytes(b"VXM1" + b[4:])
    assert describe(cut)[0] is None and "magic" in describe(cut)[1]
    assert describe(tmp_path / "absent.vxm")[0] is None


def test_rejects_inconsistent_initializer(tmp_path):
    """An initializer whose byte count disagrees with its tensor's shape is refused."""
    f = tmp_path / "c.vxm"
    save("conv3x3_bn_relu", 1, f, "passes=0")
    b = bytearray(f.read_bytes())
    # The initializer table ends the file ({i64 id, u32 len, len bytes} per entry), so the last
    # blob is the L bytes after the u32 at len(b) - L - 4 that reads L. Shorten it by 4 bytes.
    tail = len(b)
    for L in range(4, tail):
        pos = tail - L - 4
        if pos < 0:
            break
        if struct.unpack_from("<I", b, pos)[0] == L and L % 4 == 0 and L >= 16:
            break
    else:
        pytest.fail("no initializer blob found")
    struct.pack_into("<I", b, pos, L - 4)
    del b[-4:]
    bad = tmp_path / "bad.vxm"
    bad.write_bytes(bytes(b))
    text, err = describe(bad)
    assert text is None and "bytes for its shape" in err, err


@pytest.mark.gpu
@pytest.mark.parametrize("model,batch,opts", [("resnet_tiny", 2, ""), ("mnv3_tiny", 2, "fuse_se=1;fuse_dwpw=1"), ("yolo_tiny", 1, "")])
def test_session_from_vxm_matches_model_session(tmp_path, model, batch, opts):
    """Same graph, same (shared in-process) tune table -> same plans -> identical outputs; and the
    session's own saveOptimized writes the same file."""
    V.require_gpu()
    f = tmp_path / "m.vxm"
    save(model, batch, f, opts, seed=11)
    s1 = V.Session(model, batch, seed=11, options=opts + ";keep_weights=1")
    s2 = V.Session.from_vxm(f, model, batch, options=opts)
    x = np.random.default_rng(3).standard_normal(int(np.prod(s1.in_shape))).astype(np.float32)
    y1, y2 = s1.run(x), s2.run(x)
    assert s1.describe() == s2.describe()
    np.testing.assert_array_equal(y1, y2)
    g = tmp_path / "saved.vxm"
    s1.save_optimized(g)
    assert g.read_bytes() == f.read_bytes()
    with pytest.raises(V.VkhipError, match="keep_weights"):
        s2.save_optimized(tmp_path / "no.vxm")
