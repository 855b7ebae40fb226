"""The `.tirs` tensor bundle: the one file format tabicl-anywhere uses for weights, fitted caches and test vectors.

Layout (`src/store.rs:1-11`):

    bytes 0..8    magic "TIRSBNDL"
    bytes 8..16   u64 little-endian: length of the index in bytes
    index         utf-8 text, one line per tensor:  name dtype offset nbytes dim0 dim1 ...
    data          each tensor starts on a 64-byte boundary (offset counts from the start of the file)

Reading follows `Bundle::from_source` (`src/store.rs:317-351`): the index must be at most 64 MiB and every line's
shape must account for exactly its stored bytes. Writing follows `BundleWriter::create_on` (`src/store.rs:430-461`):
the data area starts after a 64-byte-rounded index sized from a 10^15 offset guess, tensors in the order given.
float16 tensors widen to float32 exactly when read as floats (`Bundle::read_f32_at`, `src/store.rs:381-398`).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

MAGIC = b"TIRSBNDL"
MAX_INDEX = 64 << 20

_DTYPES = {
    "float32": np.dtype("<f4"),
    "int32": np.dtype("<i4"),
    "float16": np.dtype("<f2"),
    "uint8": np.dtype("u1"),
    "int8": np.dtype("i1"),
    "float64": np.dtype("<f8"),
    "int64": np.dtype("<i8"),
}


class BundleError(ValueError):
    """A damaged or foreign bundle (the reference's `io::ErrorKind::InvalidData`)."""


@dataclass
class Entry:
    name: str
    dtype: str
    offset: int
    nbytes: int
    dims: tuple

    def __len__(self) -> int:
        n = 1
        for v in self.dims:
            n *= v
        return n


class Bundle:
    """A bundle held in memory (bytes) or read from a path."""

    def __init__(self, data: bytes | bytearray | memoryview):
        self.data = memoryview(data)
        if len(self.data) < 16 or bytes(self.data[:8]) != MAGIC:
            raise BundleError("not a tabicl-anywhere bundle")
        (index_len,) = struct.unpack("<Q", self.data[8:16])
        if index_len > MAX_INDEX:
            raise BundleError(f"bundle index claims {index_len} bytes; the file is damaged")
        if 16 + index_len > len(self.data):
            raise BundleError("read past the end of the bundle bytes")
        text = bytes(self.data[16:16 + index_len]).decode("utf-8")
        self.entries: list[Entry] = []
        self.by_name: dict[str, int] = {}
        for line in text.splitlines():
            p = line.split(" ")
            if len(p) < 4:
                raise BundleError(f"short index line: {line}")
            name, dtype = p[0], p[1]
            try:
                offset, nbytes = int(p[2]), int(p[3])
                dims = tuple(int(s) for s in p[4:])
            except ValueError as exc:
                raise BundleError(f"{line}: {exc}") from None
            if dtype not in _DTYPES:
                raise BundleError(f"{line}: unknown tensor type")
            count = 1
            for v in dims:
                count *= v
            if count * _DTYPES[dtype].itemsize != nbytes:
                raise BundleError(f"{line}: shape and length disagree; the file is damaged")
            self.by_name[name] = len(self.entries)
            self.entries.append(Entry(name, dtype, offset, nbytes, dims))

    @classmethod
    def open(cls, path) -> "Bundle":
        with open(path, "rb") as f:
            return cls(f.read())

    def has(self, name: str) -> bool:
        return name in self.by_name

    def entry(self, name: str) -> Entry:
        try:
            return self.entries[self.by_name[name]]
        except KeyError:
            raise BundleError(f"bundle has no tensor named {name}") from None

    def raw(self, name: str) -> np.ndarray:
        """The stored bytes of `name` as a uint8 array (a view: no copy)."""
        e = self.entry(name)
        if e.offset + e.nbytes > len(self.data):
            raise BundleError(f"{name}: read past the end")
        return np.frombuffer(self.data, dtype=np.uint8, count=e.nbytes, offset=e.offset)

    def array(self, name: str) -> np.ndarray:
        """The tensor in its stored type and shape."""
        e = self.entry(name)
        a = self.raw(name).view(_DTYPES[e.dtype])
        return a.reshape(e.dims) if e.dims else a

    def f32s(self, name: str) -> np.ndarray:
        """The tensor as float32 (float16 widened exactly), flat, as `Bundle::f32s`."""
        e = self.entry(name)
        if e.dtype not in ("float32", "float16"):
            raise BundleError(f"{name}: wanted float32, have {e.dtype}")
        return np.ascontiguousarray(self.array(name).astype(np.float32).reshape(-1))

    def i32s(self, name: str) -> np.ndarray:
        e = self.entry(name)
        if e.dtype != "int32":
            raise BundleError(f"{name}: is {e.dtype}, wanted int32")
        return np.ascontiguousarray(self.array(name).reshape(-1))

    def f64s(self, name: str) -> np.ndarray:
        return np.ascontiguousarray(self.raw(name).view("<f8"))

    def bytes(self, name: str) -> bytes:
        return self.raw(name).tobytes()


def join_parts(manifest_path) -> "Bundle":
    """A bundle stored as numbered parts beside a JSON manifest (`{"bytes": total, "parts": [{"file", "bytes"}]}`),
    joined in order, as the reference ships its 16-bit weights (`store::join_parts`, `src/store.rs:269-280`). Every
    part must have exactly its listed size, and the parts must add up to the total."""
    import json
    import os

    with open(manifest_path) as f:
        man = json.load(f)
    here = os.path.dirname(os.path.abspath(manifest_path))
    out = bytearray()
    for part in man["parts"]:
        name = part["file"]
        if os.path.basename(name) != name:
            raise BundleError(f"part {name}: parts must sit beside their manifest")
        with open(os.path.join(here, name), "rb") as f:
            data = f.read()
        if len(data) != int(part["bytes"]):
            raise BundleError(f"{name} is {len(data)} bytes, the parts list says {part['bytes']}")
        out += data
    if len(out) != int(man["bytes"]):
        raise BundleError(f"the parts hold {len(out)} bytes, the manifest says {man['bytes']}")
    return Bundle(bytes(out))


def _line(name: str, dtype: str, off: int, nb: int, dims) -> str:
    return " ".join([name, dtype, str(off), str(nb)] + [str(v) for v in dims]) + "\n"


def layout(tensors):
    """Offsets for `tensors` (a list of `(name, dtype, dims)`) exactly as `BundleWriter::create_on` places them:
    returns `(index_text, entries, total_bytes)`."""
    for name, dtype, _ in tensors:
        if not name or " " in name or "\n" in name:
            raise ValueError(f"tensor name '{name}' is empty or has a space or line break")
        if dtype not in _DTYPES:
            raise ValueError(f"unknown tensor type {dtype}")
    sizes = []
    for _, dtype, dims in tensors:
        n = 1
        for v in dims:
            n *= v
        sizes.append(n * _DTYPES[dtype].itemsize)
    guess = sum(len(_line(n, d, 10 ** 15, nb, dims)) for (n, d, dims), nb in zip(tensors, sizes))
    pos = -(-(guess + 16) // 64) * 64
    index = ""
    entries = []
    for (n, d, dims), nb in zip(tensors, sizes):
        index += _line(n, d, pos, nb, dims)
        entries.append(Entry(n, d, pos, nb, tuple(dims)))
        pos = -(-(pos + nb) // 64) * 64
    return index, entries, pos


def write(path_or_none, tensors: dict) -> bytes:
    """Write a bundle of numpy arrays (`name -> array`, in order); returns the bytes, and writes them to
    `path_or_none` if given."""
    dt_name = {v: k for k, v in _DTYPES.items()}
    specs = []
    arrays = []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        if a.dtype == np.dtype("float32"):
            a = a.astype("<f4")
        key = np.dtype(a.dtype).newbyteorder("<") if a.dtype.itemsize > 1 else a.dtype
        dtype = dt_name.get(np.dtype(key))
        if dtype is None:
            raise ValueError(f"{name}: unsupported dtype {a.dtype}")
        specs.append((name, dtype, list(a.shape)))
        arrays.append(a)
    index, entries, total = layout(specs)
    out = bytearray(total)
    idx = index.encode("utf-8")
    out[0:8] = MAGIC
    out[8:16] = struct.pack("<Q", len(idx))
    out[16:16 + len(idx)] = idx
    for e, a in zip(entries, arrays):
        out[e.offset:e.offset + e.nbytes] = a.tobytes()
    if path_or_none is not None:
        with open(path_or_none, "wb") as f:
            f.write(out)
    return bytes(out)
