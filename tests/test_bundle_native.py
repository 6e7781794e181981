"""The native a100-native-io/v1 reader (g950_bundle_*, host code, no GPU).

It must accept every held bundle, decode the same records as the Python
reader, and refuse corrupted images with the reference reader's reason
(a100c/runtime/bundle.c:111-339; the rejection checks of
a100c/tests/test_runtime_smoke.py:111-124).  The two readers are independent
implementations of the same ordered rule list, so the tests hold them to the
same verdict on every single-field corruption of the held images, and pin the
reasons the reference's own smoke test provokes.
"""
import ctypes
import struct
import subprocess

import numpy as np
import pytest

from compiler_amd import bundle as bmod
from compiler_amd import runtime as rt
from tests._fixtures import GOLDEN, INDEX

EXEC = rt.PKG / "lib" / "g950_exec"


def py_reason(image):
    try:
        bmod.parse(image)
    except bmod.BundleRejected as e:
        return e.reason
    return None


@pytest.mark.parametrize("case", sorted(INDEX))
def test_native_open_decodes_like_python(case):
    lib = rt.load_library()
    path = GOLDEN / case / "bundle.bin"
    assert rt.bundle_check(path.read_bytes()) is None
    b = ctypes.c_void_p()
    reason = ctypes.c_int(-1)
    assert lib.g950_bundle_open(str(path).encode(), 0, ctypes.byref(b), ctypes.byref(reason)) == 0
    try:
        ref = bmod.read(GOLDEN / case)
        assert lib.g950_bundle_count(b, 0) == len(ref.storages)
        assert lib.g950_bundle_count(b, 1) == len(ref.views)
        assert lib.g950_bundle_count(b, 2) == len(ref.scalars)
        assert lib.g950_bundle_count(b, 3) == len(ref.relocations)
        for i, rv in enumerate(ref.views):
            v = rt.View()
            assert lib.g950_bundle_view(b, i, ctypes.byref(v)) == 0
            assert v.dtype == rv.dtype and v.ndim == len(rv.shape) and bool(v.flags & 1) == rv.output
            assert tuple(v.shape[k] for k in range(v.ndim)) == tuple(rv.shape)
            assert tuple(v.strides[k] for k in range(v.ndim)) == tuple(rv.strides)
            assert v.data - v.storage == rv.offset
            assert v.storage_size == ref.storages[rv.storage][1]
            # the view's bytes over the mapping equal the Python reader's array
            n = int(np.prod(rv.shape)) if rv.shape else 1
            if n and all(s > 0 for s in rv.strides):
                arr = ref.array(rv)
                span = (ctypes.c_ubyte * (v.storage_size - rv.offset)).from_address(v.data)
                mine = np.ndarray(rv.shape, dtype=arr.dtype, buffer=span, strides=rv.strides)
                assert np.array_equal(mine, arr, equal_nan=True)
        for i, rs in enumerate(ref.scalars):
            s = rt.Scalar()
            assert lib.g950_bundle_scalar(b, i, ctypes.byref(s)) == 0
            assert (s.dtype, s.size, s.bits) == (rs.dtype, rs.size, rs.bits)
    finally:
        assert lib.g950_bundle_close(b) == 0


@pytest.mark.parametrize("case", ["softmax97-float32-t1", "attention-bfloat16-t1", "matmul-tail-float16-t1"])
def test_every_metadata_field_corruption_same_verdict(case):
    """Flip every metadata byte three ways: both readers agree on each image."""
    img = bytearray((GOLDEN / case / "bundle.bin").read_bytes())
    ref = bmod.parse(img)
    meta_end = min(off for off, _ in ref.storages)
    checked = rejected = 0
    for pos in range(meta_end):
        for mutate in (lambda b: b ^ 0xFF, lambda b: (b + 1) & 0xFF, lambda b: 0x80):
            bad = bytearray(img)
            bad[pos] = mutate(bad[pos])
            if bad == img:
                continue
            p, n = py_reason(bad), rt.bundle_check(bad)
            assert p == n, f"byte {pos}: python {p} native {n}"
            checked += 1
            rejected += p is not None
    assert checked > 3 * meta_end - 10 and rejected > meta_end // 2
    # truncations at every length
    for cut in range(0, len(img), max(1, len(img) // 97)):
        assert py_reason(img[:cut]) == rt.bundle_check(img[:cut])


def _synthetic(reloc=None, table_output=False):
    """A two-view image: an int64 pointer table of 2 entries and a float32
    target of 4 elements, plus optional relocation record."""
    nrel = 1 if reloc else 0
    meta = 32 + 2 * 16 + 2 * (24 + 16) + 0 + 24 * nrel
    s0 = (meta + 63) // 64 * 64
    s1 = s0 + 64
    img = bytearray(s1 + 64)
    struct.pack_into("<8s6I", img, 0, b"A100IO01", 1, 2, 2, 0, nrel, 0)
    struct.pack_into("<QQ", img, 32, s0, 16)
    struct.pack_into("<QQ", img, 48, s1, 16)
    cur = 64
    struct.pack_into("<IIIIq", img, cur, 0, rt.DT_INT64, 1, 1 if table_output else 0, 0)
    struct.pack_into("<qq", img, cur + 24, 2, 8)
    cur += 40
    struct.pack_into("<IIIIq", img, cur, 1, rt.DT_F32, 1, 0, 0)
    struct.pack_into("<qq", img, cur + 24, 4, 4)
    cur += 40
    if reloc:
        struct.pack_into("<IIQq", img, cur, *reloc)
    return img


@pytest.mark.parametrize("reloc,table_output,reason", [
    ((0, 1, 1, 4), False, None),
    ((0, 1, 2, 0), False, "reloc-entry"),          # slot 2 of a 2-entry table
    ((0, 1, 1, 17), False, "reloc-offset"),        # past the 16-byte target
    ((0, 1, 2**61, 0), False, "reloc-entry"),      # entry*8 would wrap
    ((0, 2, 0, 0), False, "reloc-view"),
    ((1, 0, 0, 0), False, "reloc-table-width"),    # float32 table
    ((0, 1, 0, 0), True, "reloc-table-output"),
])
def test_relocation_rules(reloc, table_output, reason):
    img = _synthetic(reloc, table_output)
    assert py_reason(img) == reason
    assert rt.bundle_check(img) == reason


def test_reference_smoke_corruptions():
    """test_runtime_smoke.py:111-124 corrupts a view's i64 offset field and a
    relocation's entry field; both must be refused with those reasons."""
    img = bytearray((GOLDEN / "softmax97-float32-t1" / "bundle.bin").read_bytes())
    struct.pack_into("<q", img, 32 + 2 * 16 + 16, 1 << 40)
    assert rt.bundle_check(img) == "view-offset" == py_reason(img)
    img = _synthetic((0, 1, 1, 0))
    struct.pack_into("<Q", img, 64 + 80 + 8, 1 << 20)
    assert rt.bundle_check(img) == "reloc-entry" == py_reason(img)


def test_reason_names_match_reference_table():
    lib = rt.load_library()
    names = [lib.g950_bundle_reason(i).decode() for i in range(1, 26)]
    assert names == ["open", "size", "magic", "version", "reserved", "map", "storage-bounds",
                     "count-bounds", "alloc", "view-truncated", "view-storage", "view-dtype",
                     "view-offset", "view-dim", "view-reach", "view-flags", "scalar-truncated",
                     "scalar-width", "reloc-truncated", "reloc-view", "reloc-table-width",
                     "reloc-table-output", "reloc-entry", "reloc-offset", "storage-overlaps-metadata"]
    assert lib.g950_bundle_reason(0) == b"unknown" and lib.g950_bundle_reason(26) == b"unknown"


def test_exec_cli_rejects_before_touching_a_device(tmp_path):
    """g950_exec refuses a corrupted bundle with the reason and exit 3, and a
    bad command line with exit 2, before any GPU call; the file is untouched."""
    img = bytearray((GOLDEN / "softmax97-float32-t1" / "bundle.bin").read_bytes())
    struct.pack_into("<I", img, 8, 7)
    p = tmp_path / "bundle.bin"
    p.write_bytes(bytes(img))
    r = subprocess.run([str(EXEC), "--bundle", str(tmp_path), "--op", "softmax_kernel"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 3 and '"reason":"version"' in r.stdout
    assert p.read_bytes() == bytes(img)
    r = subprocess.run([str(EXEC), "--bundle", str(p), "--op", "no_such_kernel"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
    r = subprocess.run([str(EXEC), "--bundle", str(p), "--op", "softmax", "--repeats", "0"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
