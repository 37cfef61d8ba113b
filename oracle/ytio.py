"""CPU restatement of YTensor's .yt file format — TEST INFRASTRUCTURE ONLY.

Only tests/ may use this module: it writes checkpoints for the loader tests and
reads files back to check the product's writer. It is pinned against the
reference's own yt::io::YTensorIO (compiled into oracle/_ref by `make ref`):
files written here are byte-identical to the reference's for the same tensors,
and the reference-written fixtures under tests/golden read back to their
recorded arrays (tests/test_ytio.py).

Format, little-endian (src/ytensor_io.inl):
  header   "YTENSORF" | u8 version (0) | str metadata           writeHeader 487-506
  record   str name | str typeName | i32 typeSize | str tensorType |
           u64 nbytes + i32 dims[] | str compressMethod | u64 size | payload
                                                                close() 367-399
  index    u64 offset of each record | u32 count               writeIndex 561-578
  str = u32 length + bytes (string2data 24-32); array2data (templates.inl:5-14)
  zlib: deflateInit2(level -1, Z_DEFLATED, 15, 8, Z_FILTERED) over the whole
  payload in one call (compressData, templates.inl:17-46); read with
  inflateInit2(15 + 32) (decompressData 147-250).
"""
from __future__ import annotations

import struct
import zlib

import numpy as np

MAGIC = b"YTENSORF"
VERSION = 0

# reference typeName -> numpy dtype (bfloat16 kept as its uint16 bits)
NP = {"float32": np.float32, "float64": np.float64, "float16": np.float16, "bfloat16": np.uint16,
      "int8": np.int8, "int16": np.int16, "int32": np.int32, "int64": np.int64, "uint8": np.uint8,
      "uint16": np.uint16, "uint32": np.uint32, "uint64": np.uint64, "bool": np.bool_}


def _str(b: str) -> bytes:
    e = b.encode()
    return struct.pack("<I", len(e)) + e


def encode(tensors, compress: str = "", metadata: str = "") -> bytes:
    """tensors: [(name, typeName, shape, bytes-like payload)] -> file bytes."""
    out = bytearray(MAGIC + struct.pack("<B", VERSION) + _str(metadata))
    offsets = []
    for name, tname, shape, data in tensors:
        raw = bytes(data)
        tsize = np.dtype(NP[tname]).itemsize
        if compress == "zlib" and raw:
            co = zlib.compressobj(-1, zlib.DEFLATED, 15, 8, zlib.Z_FILTERED)
            payload = co.compress(raw) + co.flush()
        else:
            payload = raw
        offsets.append(len(out))
        out += _str(name) + _str(tname) + struct.pack("<i", tsize) + _str("dense")
        out += struct.pack("<Q", 4 * len(shape)) + struct.pack(f"<{len(shape)}i", *shape)
        out += _str(compress if compress == "zlib" else "") + struct.pack("<Q", len(payload)) + payload
    out += struct.pack(f"<{len(offsets)}Q", *offsets) + struct.pack("<I", len(offsets))
    return bytes(out)


def write(path: str, arrays: dict, compress: str = "", types: dict | None = None) -> None:
    """arrays: name -> numpy array (bf16 as uint16 bits with types[name] = "bfloat16")."""
    types = types or {}
    rev = {np.dtype(v): k for k, v in NP.items() if k not in ("bfloat16", "uint16")}
    rev[np.dtype(np.uint16)] = "uint16"
    items = []
    for name, a in arrays.items():
        a = np.ascontiguousarray(a)
        tname = types.get(name, rev[a.dtype])
        items.append((name, tname, list(a.shape), a.tobytes()))
    with open(path, "wb") as f:
        f.write(encode(items, compress))


def read(path: str) -> tuple[str, list[dict]]:
    """-> (metadata, [{name, typeName, typeSize, tensorType, shape, compress, payload, data}])
    with data the decoded numpy array (None for non-dense records)."""
    b = open(path, "rb").read()
    if b[:8] != MAGIC:
        raise ValueError("bad magic")
    pos = 9
    (n,) = struct.unpack_from("<I", b, pos)
    meta = b[pos + 4:pos + 4 + n].decode()
    (count,) = struct.unpack_from("<I", b, len(b) - 4)
    offs = struct.unpack_from(f"<{count}Q", b, len(b) - 4 - 8 * count)
    recs = []
    for o in offs:
        p = o

        def s():
            nonlocal p
            (ln,) = struct.unpack_from("<I", b, p)
            v = b[p + 4:p + 4 + ln].decode()
            p += 4 + ln
            return v
        name, tname = s(), s()
        (tsize,) = struct.unpack_from("<i", b, p)
        p += 4
        ttype = s()
        (sb,) = struct.unpack_from("<Q", b, p)
        p += 8
        shape = list(struct.unpack_from(f"<{sb // 4}i", b, p))
        p += sb
        comp = s()
        (cs,) = struct.unpack_from("<Q", b, p)
        p += 8
        payload = b[p:p + cs]
        raw = zlib.decompress(payload) if comp == "zlib" and payload else payload
        data = None
        if ttype == "dense" and tname in NP:
            data = np.frombuffer(raw, dtype=NP[tname]).reshape(shape).copy()
        recs.append(dict(name=name, typeName=tname, typeSize=tsize, tensorType=ttype, shape=shape, compress=comp,
                         payload=payload, data=data))
    return meta, recs
