"""The persistent autotune table: the reference's unified cache-file container ("VKNNCAC1",
src/backend/vulkan/vk_backend.cpp:440-545) with its weight/tune section (vk_backend.cpp:30-126).
CPU tests drive the table through include/vknn_c.h; the GPU test checks that a second session
on the same cache file takes every plan from the file instead of timing candidates."""
import ctypes
import struct

import numpy as np

import pytest

import vknn_amd as V


def container(pipe=b"", weights=(), tune=()):
    """A cache file laid out as the reference writes it."""
    w = struct.pack("<I", len(weights))
    for k, floats in weights:
        w += struct.pack("<I", len(k)) + k + struct.pack("<I", len(floats)) + struct.pack(f"<{len(floats)}f", *floats)
    w += struct.pack("<I", len(tune))
    for k, v in tune:
        w += struct.pack("<I", len(k)) + k + struct.pack("<i", v)
    return b"VKNNCAC1" + struct.pack("<I", len(pipe)) + pipe + struct.pack("<I", len(w)) + w


@pytest.fixture
def lib():
    lib = V.vknn()
    lib.vknn_tune_cache_clear()
    yield lib
    lib.vknn_tune_cache_clear()


def get(lib, key):
    v = ctypes.c_int32()
    rc = lib.vknn_tune_cache_get(key, ctypes.byref(v))
    return v.value if rc == 0 else None


def test_reads_reference_layout(lib, tmp_path):
    """A reference-written file: pipeline bytes and prepacked weights are skipped, tune entries
    (negative values included) are read."""
    f = tmp_path / "m.cache"
    f.write_bytes(container(b"PIPELINE-BLOB", [(b"w0", [1.0, 2.0, 3.0])], [(b"gpu/convls_1", 128), (b"gpu/wino_2", -1)]))
    assert lib.vknn_tune_cache_load(str(f).encode()) == 2
    assert get(lib, b"gpu/convls_1") == 128
    assert get(lib, b"gpu/wino_2") == -1
    assert get(lib, b"gpu/absent") is None
    n, h, m = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    lib.vknn_tune_cache_stats(ctypes.byref(n), ctypes.byref(h), ctypes.byref(m))
    assert (n.value, h.value, m.value) == (2, 2, 1)
    lib.vknn_weight_cache_stats(ctypes.byref(n), None, None)
    assert n.value == 1  # the prepacked blob is retained (CacheMode::Full)


def test_weight_section_roundtrip(lib, tmp_path):
    """Prepacked weight blobs survive a load and a rewrite byte for byte, next to the tune table
    and a foreign pipeline section; keys come out sorted, as the reference's std::map writes them."""
    src = container(b"PIPE", [(b"hip/w/conv_9#b", [0.5, -2.0]), (b"hip/w/conv_1#a", [1.0, 2.0, 3.0])], [(b"t", 7)])
    f, g = tmp_path / "a.cache", tmp_path / "b.cache"
    f.write_bytes(src)
    assert lib.vknn_tune_cache_load(str(f).encode()) == 1
    n = ctypes.c_int64()
    lib.vknn_weight_cache_stats(ctypes.byref(n), None, None)
    assert n.value == 2
    assert lib.vknn_tune_cache_save(str(g).encode()) == 0
    assert g.read_bytes() == container(b"PIPE", [(b"hip/w/conv_1#a", [1.0, 2.0, 3.0]), (b"hip/w/conv_9#b", [0.5, -2.0])], [(b"t", 7)])


def test_truncated_weight_section_keeps_nothing_past_the_cut(lib, tmp_path):
    """A weight blob cut short (section length fixed so the container parses) ends the section:
    the complete blob before it is kept, the tune table after it is not reached."""
    full = container(b"", [(b"w0", [1.0]), (b"w1", [2.0, 3.0])], [(b"t", 1)])
    body = full[:-(4 + 1 + 4 + 4 + 4)]  # drop the tune table and the last float of w1
    wl = len(body) - 16
    body = body[:12] + struct.pack("<I", wl) + body[16:]
    f = tmp_path / "w.cache"
    f.write_bytes(body)
    assert lib.vknn_tune_cache_load(str(f).encode()) == 0
    n = ctypes.c_int64()
    lib.vknn_weight_cache_stats(ctypes.byref(n), None, None)
    assert n.value == 1 and get(lib, b"t") is None


def test_save_roundtrip_and_unchanged_file_untouched(lib, tmp_path):
    f = tmp_path / "rt.cache"
    assert lib.vknn_tune_cache_put(b"hip-gfx950-256cu/conv_64_256_14_14", 0x031201) == 0
    assert lib.vknn_tune_cache_put(b"hip-gfx950-256cu/dwpw_1", 1) == 0
    assert lib.vknn_tune_cache_save(str(f).encode()) == 0
    data = f.read_bytes()
    # the HIP table writes no pipeline bytes and no weights; keys in sorted order
    assert data == container(b"", [], [(b"hip-gfx950-256cu/conv_64_256_14_14", 0x031201), (b"hip-gfx950-256cu/dwpw_1", 1)])
    lib.vknn_tune_cache_clear()
    assert lib.vknn_tune_cache_load(str(f).encode()) == 2
    assert get(lib, b"hip-gfx950-256cu/conv_64_256_14_14") == 0x031201
    # unchanged table: the file is not rewritten (mtime and bytes stay)
    before = f.stat().st_mtime_ns
    f.chmod(0o444)
    try:
        assert lib.vknn_tune_cache_save(str(f).encode()) == 0
    finally:
        f.chmod(0o644)
    assert f.stat().st_mtime_ns == before and f.read_bytes() == data


def test_rewrite_keeps_foreign_pipeline_section(lib, tmp_path):
    f = tmp_path / "p.cache"
    f.write_bytes(container(b"PIPE", [], [(b"a", 1)]))
    assert lib.vknn_tune_cache_load(str(f).encode()) == 1
    lib.vknn_tune_cache_put(b"b", 2)
    assert lib.vknn_tune_cache_save(str(f).encode()) == 0
    assert f.read_bytes() == container(b"PIPE", [], [(b"a", 1), (b"b", 2)])


@pytest.mark.parametrize("blob", [b"", b"NOTACACHE", b"VKNNCAC1\xff\xff\xff\xff", container()[:-3]])
def test_unrecognised_or_truncated_files_are_ignored(lib, tmp_path, blob):
    f = tmp_path / "bad.cache"
    f.write_bytes(blob)
    assert lib.vknn_tune_cache_load(str(f).encode()) == 0
    assert get(lib, b"a") is None


def test_truncated_tune_tail_keeps_complete_entries(lib, tmp_path):
    full = container(b"", [], [(b"a", 1), (b"bb", 2)])
    # cut inside the second entry but fix the section length so the container itself parses
    body = full[:-3]
    wlen_off = 8 + 4 + 0
    wl = len(body) - (wlen_off + 4)
    body = body[:wlen_off] + struct.pack("<I", wl) + body[wlen_off + 4:]
    f = tmp_path / "t.cache"
    f.write_bytes(body)
    assert lib.vknn_tune_cache_load(str(f).encode()) == 1
    assert get(lib, b"a") == 1 and get(lib, b"bb") is None


def test_missing_file_and_unwritable_path(lib, tmp_path):
    assert lib.vknn_tune_cache_load(str(tmp_path / "none.cache").encode()) == 0
    lib.vknn_tune_cache_put(b"k", 3)
    assert lib.vknn_tune_cache_save(str(tmp_path / "no_dir" / "x.cache").encode()) != 0
    assert b"cannot write cache file" in lib.vknn_last_error()


@pytest.mark.gpu
def test_warm_start_takes_plans_from_cache_file(lib, tmp_path):
    """Cold session: tunes and writes the file. After clearing the in-process table, a second
    session on the same file reads every plan back (no lookup misses) and plans identically."""
    V.require_gpu()
    f = tmp_path / "resnet.cache"
    opts = f"cache_file={f};tuning=fast"
    s1 = V.Session("resnet50", 2, seed=3, options=opts)
    plan1 = s1.describe()
    del s1
    data = f.read_bytes()
    assert data.startswith(b"VKNNCAC1")
    tag = ctypes.create_string_buffer(128)
    lib.vknn_tune_cache_gpu_tag(tag, 128)
    assert tag.value.startswith(b"hip-gfx950")
    assert tag.value + b"/conv_" in data
    n = ctypes.c_int64()
    lib.vknn_tune_cache_stats(ctypes.byref(n), None, None)
    entries = n.value
    assert entries > 10
    lib.vknn_tune_cache_clear()
    s2 = V.Session("resnet50", 2, seed=3, options=opts)
    h, m = ctypes.c_int64(), ctypes.c_int64()
    lib.vknn_tune_cache_stats(ctypes.byref(n), ctypes.byref(h), ctypes.byref(m))
    assert m.value == 0 and h.value > 10 and n.value == entries
    assert s2.describe() == plan1
    del s2
    assert f.read_bytes() == data  # unchanged table: file untouched


@pytest.mark.gpu
def test_warm_start_takes_prepacked_weights_from_cache_file(lib, tmp_path):
    """CacheMode::Full (the default) with a cache file keeps every conv's prepacked blob in the
    file's weight section. A warm session packs nothing: every blob comes from the file, and the
    outputs are bit-identical. A model with other weights (another seed) finds no blob of its own."""
    V.require_gpu()
    f = tmp_path / "w.cache"
    opts = f"cache_file={f}"
    s1 = V.Session("resnet_tiny", 2, seed=3, options=opts)
    x = np.random.default_rng(0).standard_normal(s1.in_shape).astype(np.float32)
    y1 = s1.run(x)
    convs = s1.count_ops("Conv")
    del s1
    n, h, m = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    lib.vknn_weight_cache_stats(ctypes.byref(n), None, None)
    assert n.value >= convs > 0
    lib.vknn_tune_cache_clear()
    s2 = V.Session("resnet_tiny", 2, seed=3, options=opts)
    lib.vknn_weight_cache_stats(ctypes.byref(n), ctypes.byref(h), ctypes.byref(m))
    assert m.value == 0 and h.value == convs
    np.testing.assert_array_equal(s2.run(x), y1)
    del s2
    lib.vknn_tune_cache_clear()
    s3 = V.Session("resnet_tiny", 2, seed=4, options=opts)
    lib.vknn_weight_cache_stats(ctypes.byref(n), ctypes.byref(h), ctypes.byref(m))
    assert h.value == 0 and m.value == convs
    del s3
    lib.vknn_tune_cache_clear()
    s4 = V.Session("resnet_tiny", 2, seed=3, options=opts + ";cache_mode=tune")
    lib.vknn_weight_cache_stats(ctypes.byref(n), ctypes.byref(h), ctypes.byref(m))
    assert h.value == 0 and m.value == 0  # Tune mode neither reads nor keeps blobs
    np.testing.assert_array_equal(s4.run(x), y1)
    del s4
    # blobs written under another pack-format version (the key's #f<version># field) are not taken
    import re
    data = f.read_bytes()
    vers = set(re.findall(rb"#f(\d+)#", data))
    assert len(vers) == 1, vers
    ver = vers.pop()
    other = str((int(ver) + 1) % (10 ** len(ver))).zfill(len(ver)).encode()
    f.write_bytes(data.replace(b"#f" + ver + b"#", b"#f" + other + b"#"))
    lib.vknn_tune_cache_clear()
    s5 = V.Session("resnet_tiny", 2, seed=3, options=opts)
    lib.vknn_weight_cache_stats(ctypes.byref(n), ctypes.byref(h), ctypes.byref(m))
    assert h.value == 0 and m.value == convs
    np.testing.assert_array_equal(s5.run(x), y1)
