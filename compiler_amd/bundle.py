"""Reader for the ``a100-native-io/v1`` argument image.

The image format is the reference's host<->native boundary
(writer: a100_support/native_io.py:49-126; reader: a100c/runtime/bundle.c:10-19,
111-339).  Layout, little-endian:

  header   32 B : magic "A100IO01", u32 version=1, u32 nstorage, u32 nviews,
                  u32 nscalars, u32 nrelocations, u32 reserved=0
  storage  16 B each : u64 file offset, u64 size
  view          : u32 storage, u32 dtype, u32 ndim, u32 flags(bit0=output),
                  i64 offset, ndim*i64 shape, ndim*i64 byte strides
  scalar   16 B : u32 dtype, u32 size, u64 bits
  reloc    24 B : u32 table view, u32 target view, u64 entry, i64 byte_offset

Views and scalars are in sorted argument-name order; the names themselves live
in the companion ``bundle.json``.  The whole image is validated before
anything is returned, and a violation raises ``BundleRejected`` carrying the
same reason names the reference reader reports (bundle.c:59-88).
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

MAGIC = b"A100IO01"
HEADER = struct.Struct("<8s6I")
STORAGE = struct.Struct("<QQ")
VIEW = struct.Struct("<IIIIq")
SCALAR = struct.Struct("<IIQ")
RELOCATION = struct.Struct("<IIQq")

# dtype codes of the format (a100c/runtime/a100rt.h:58-72)
DTYPE_CODES = {
    "bool": 1, "int8": 2, "uint8": 3, "int16": 4, "uint16": 5, "int32": 6,
    "uint32": 7, "int64": 8, "uint64": 9, "float16": 10, "bfloat16": 11,
    "float32": 12, "float64": 13,
}
DTYPE_NAMES = {code: name for name, code in DTYPE_CODES.items()}
ITEMSIZE = {1: 1, 2: 1, 3: 1, 4: 2, 5: 2, 6: 4, 7: 4, 8: 8, 9: 8, 10: 2, 11: 2, 12: 4, 13: 8}
# numpy storage type per code; bf16 is carried as its uint16 bits
NUMPY_STORAGE = {1: np.bool_, 2: np.int8, 3: np.uint8, 4: np.int16, 5: np.uint16,
                 6: np.int32, 7: np.uint32, 8: np.int64, 9: np.uint64,
                 10: np.float16, 11: np.uint16, 12: np.float32, 13: np.float64}


class BundleRejected(ValueError):
    """The image violates a100-native-io/v1; ``reason`` names the rule."""

    def __init__(self, reason: str, detail: str = ""):
        super().__init__(f"bundle rejected: {reason}" + (f" ({detail})" if detail else ""))
        self.reason = reason


@dataclass
class ViewRecord:
    storage: int
    dtype: int
    shape: tuple
    strides: tuple  # bytes
    offset: int
    output: bool
    name: str | None = None


@dataclass
class ScalarRecord:
    dtype: int
    size: int
    bits: int
    name: str | None = None

    def value(self):
        """Decode the raw little-endian bits to a Python number."""
        raw = self.bits.to_bytes(8, "little")[: self.size]
        return np.frombuffer(raw, dtype=NUMPY_STORAGE[self.dtype])[0].item()


@dataclass
class Bundle:
    image: bytearray
    storages: list  # (offset, size)
    views: list
    scalars: list
    relocations: list
    names: dict = field(default_factory=dict)

    def view(self, name: str) -> ViewRecord:
        for v in self.views:
            if v.name == name:
                return v
        raise KeyError(name)

    def scalar(self, name: str):
        for s in self.scalars:
            if s.name == name:
                return s.value()
        raise KeyError(name)

    def array(self, name_or_view) -> np.ndarray:
        """A numpy view of one argument over the image (bf16 as uint16 bits)."""
        v = self.view(name_or_view) if isinstance(name_or_view, str) else name_or_view
        off, _size = self.storages[v.storage]
        return np.ndarray(v.shape, dtype=NUMPY_STORAGE[v.dtype], buffer=self.image,
                          offset=off + v.offset, strides=v.strides)


def _reach(shape, strides, itemsize):
    """(lowest, highest+1) byte touched relative to the view base."""
    if any(s == 0 for s in shape):
        return 0, 0
    lo = sum(st * (n - 1) for n, st in zip(shape, strides) if st < 0)
    hi = sum(st * (n - 1) for n, st in zip(shape, strides) if st > 0)
    return lo, hi + itemsize


def parse(image: bytes | bytearray, names: dict | None = None) -> Bundle:
    """Validate and decode a whole image (mirrors a100c/runtime/bundle.c:111-339).

    The checks run in the reference reader's order, so the first rule an image
    breaks is the reason reported (the native reader, ``g950_bundle_check``,
    follows the same order and the tests hold the two to the same verdicts)."""
    image = bytearray(image)
    size = len(image)
    if size < HEADER.size:
        raise BundleRejected("size")
    magic, version, nstorage, nviews, nscalars, nreloc, reserved = HEADER.unpack_from(image, 0)
    if magic != MAGIC:
        raise BundleRejected("magic")
    if version != 1:
        raise BundleRejected("version")
    if reserved != 0:
        raise BundleRejected("reserved")
    cursor = HEADER.size
    if nstorage * STORAGE.size > size - cursor:
        raise BundleRejected("storage-bounds", "storage table")
    storages = []
    for i in range(nstorage):
        off, ln = STORAGE.unpack_from(image, cursor + i * STORAGE.size)
        if off > size or ln > size - off:
            raise BundleRejected("storage-bounds", f"storage {i}")
        storages.append((off, ln))
    if nviews > size // 24 or nscalars > size // 16 or nreloc > size // 24:
        raise BundleRejected("count-bounds")
    cursor += nstorage * STORAGE.size
    views = []
    for i in range(nviews):
        if cursor + VIEW.size > size:
            raise BundleRejected("view-truncated")
        storage, dtype, ndim, flags, offset = VIEW.unpack_from(image, cursor)
        if storage >= nstorage:
            raise BundleRejected("view-storage", f"view {i}")
        if dtype not in ITEMSIZE:
            raise BundleRejected("view-dtype", f"view {i}")
        if flags & ~1:
            raise BundleRejected("view-flags", f"view {i}")
        cursor += VIEW.size
        if 16 * ndim > size - cursor:
            raise BundleRejected("view-truncated")
        s_off, s_len = storages[storage]
        if offset < 0 or offset > s_len:
            raise BundleRejected("view-offset", f"view {i}")
        dims = struct.unpack_from("<" + "q" * (2 * ndim), image, cursor)
        cursor += 16 * ndim
        shape, strides = tuple(dims[:ndim]), tuple(dims[ndim:])
        if any(n < 0 for n in shape):
            raise BundleRejected("view-dim", f"view {i}")
        lo, hi = _reach(shape, strides, ITEMSIZE[dtype])
        if offset + lo < 0 or offset + hi > s_len:
            raise BundleRejected("view-reach", f"view {i}")
        views.append(ViewRecord(storage, dtype, shape, strides, offset, bool(flags & 1)))
    if SCALAR.size * nscalars > size - cursor:
        raise BundleRejected("scalar-truncated")
    scalars = []
    for i in range(nscalars):
        dtype, width, bits = SCALAR.unpack_from(image, cursor)
        cursor += SCALAR.size
        if dtype not in ITEMSIZE or width != ITEMSIZE[dtype]:
            raise BundleRejected("scalar-width", f"scalar {i}")
        scalars.append(ScalarRecord(dtype, width, bits))
    if RELOCATION.size * nreloc > size - cursor:
        raise BundleRejected("reloc-truncated")
    metadata_end = cursor + RELOCATION.size * nreloc
    for i, (off, _ln) in enumerate(storages):
        if off < metadata_end:
            raise BundleRejected("storage-overlaps-metadata", f"storage {i}")
    relocations = []
    for i in range(nreloc):
        table, target, entry, byte_offset = RELOCATION.unpack_from(image, cursor)
        cursor += RELOCATION.size
        if table >= nviews or target >= nviews:
            raise BundleRejected("reloc-view")
        t, d = views[table], views[target]
        if t.dtype not in (8, 9):
            raise BundleRejected("reloc-table-width")
        if t.output:
            raise BundleRejected("reloc-table-output")
        if entry > (2**64 - 1) // 8 or t.offset + entry * 8 + 8 > storages[t.storage][1]:
            raise BundleRejected("reloc-entry")
        if byte_offset < 0 or byte_offset > storages[d.storage][1] - d.offset:
            raise BundleRejected("reloc-offset")
        relocations.append((table, target, entry, byte_offset))
    bundle = Bundle(image, storages, views, scalars, relocations)
    if names:
        for rec, name in zip(views, names.get("view_order", [])):
            rec.name = name
        for rec, name in zip(scalars, names.get("scalar_order", [])):
            rec.name = name
    return bundle


def read(directory_or_bin) -> Bundle:
    """Read ``bundle.bin`` (+ ``bundle.json`` names when present)."""
    path = Path(directory_or_bin)
    bin_path = path / "bundle.bin" if path.is_dir() else path
    json_path = bin_path.with_name("bundle.json")
    names = json.loads(json_path.read_text()) if json_path.exists() else None
    return parse(bin_path.read_bytes(), names)
