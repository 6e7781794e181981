"""a100-native-io/v1 reader: every held fixture parses, names resolve, and
corrupted images are rejected before anything is returned (the rejection
behaviour a100c/tests/test_runtime_smoke.py:111-124 asks of the native reader)."""
import struct

import pytest

from compiler_amd import bundle as bmod
from tests._fixtures import GOLDEN, INDEX


@pytest.mark.parametrize("case", sorted(INDEX))
def test_fixture_parses(case):
    b = bmod.read(GOLDEN / case)
    assert b.views and all(v.name for v in b.views)
    assert any(v.output for v in b.views)
    for v in b.views:
        arr = b.array(v)
        assert arr.shape == tuple(v.shape)


def _image():
    return bytearray((GOLDEN / "softmax97-float32-t1" / "bundle.bin").read_bytes())


def test_rejects_bad_magic():
    img = _image()
    img[0:8] = b"XXXXXXXX"
    with pytest.raises(bmod.BundleRejected) as e:
        bmod.parse(img)
    assert e.value.reason == "magic"


def test_rejects_bad_version_and_reserved():
    img = _image()
    struct.pack_into("<I", img, 8, 2)
    with pytest.raises(bmod.BundleRejected) as e:
        bmod.parse(img)
    assert e.value.reason == "version"
    img = _image()
    struct.pack_into("<I", img, 28, 1)
    with pytest.raises(bmod.BundleRejected) as e:
        bmod.parse(img)
    assert e.value.reason == "reserved"


def test_rejects_truncation_and_view_reach():
    img = _image()
    with pytest.raises(bmod.BundleRejected):
        bmod.parse(img[:40])
    # first view's shape[0] (after header 32 B + 2 storage rows 32 B + view head 24 B)
    img = _image()
    off = 32 + 2 * 16 + 24
    (rows,) = struct.unpack_from("<q", img, off)
    struct.pack_into("<q", img, off, rows + 1)
    with pytest.raises(bmod.BundleRejected) as e:
        bmod.parse(img)
    assert e.value.reason == "view-reach"


def test_rejects_bad_dtype_and_flags():
    img = _image()
    off = 32 + 2 * 16
    struct.pack_into("<I", img, off + 4, 99)
    with pytest.raises(bmod.BundleRejected) as e:
        bmod.parse(img)
    assert e.value.reason == "view-dtype"
    img = _image()
    struct.pack_into("<I", img, off + 12, 6)
    with pytest.raises(bmod.BundleRejected) as e:
        bmod.parse(img)
    assert e.value.reason == "view-flags"


def test_scalar_decode():
    b = bmod.read(GOLDEN / "attention-bfloat16-t1")
    assert b.scalar("N_CTX") == 32 and b.scalar("H") == 4
    assert abs(b.scalar("scale") - 0.125) < 1e-7
