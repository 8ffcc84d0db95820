"""The persistent autotune table: the reference's unified cache-file container ("VKNNCAC1",
src/backend/vulkan/vk_backend.cpp:440-545) with its weight/tune section (vk_backend.cpp:30-126).
CPU tests drive the table through include/vknn_c.h; the GPU test checks that a second session
on the same cache file takes every plan from the file instead of timing candidates."""
import ctypes
import struct

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
