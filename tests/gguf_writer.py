"""A GGUF v3 writer for tests, written from the published file layout
(ggml's gguf.md): little-endian header {magic "GGUF", version u32,
tensor_count u64, kv_count u64}, the key/values {key: u64 length + UTF-8,
value type u32, value}, the tensor infos {name, n_dims u32, dims u64[n_dims],
type u32, offset u64 (relative to the data section)}, zero padding to the
alignment, then each tensor's bytes at its offset (offsets aligned too).

It shares no code with the library's reader, so a file written here and read
there checks both against the layout, not against each other's mistakes.
"""
from __future__ import annotations

import struct
from typing import Any, List, Optional, Sequence, Tuple

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
         I64: "<q", F64: "<d"}
# bytes per block and elements per block of the tensor types used here
TYPE_BLOCK = {0: (4, 1), 1: (2, 1), 8: (34, 32), 12: (144, 256), 13: (176, 256), 14: (210, 256), 30: (2, 1)}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v: Any) -> bytes:
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_PACK[t], v)


class GGUFWriter:
    def __init__(self, alignment: Optional[int] = None, version: int = 3):
        self.kvs: List[Tuple[str, int, Any]] = []
        self.tensors: List[Tuple[str, Tuple[int, ...], int, bytes]] = []
        self.version = version
        self.alignment = alignment or 32
        if alignment is not None:
            self.kv("general.alignment", U32, alignment)

    def kv(self, key: str, t: int, value: Any) -> "GGUFWriter":
        self.kvs.append((key, t, value))
        return self

    def array(self, key: str, et: int, items: Sequence) -> "GGUFWriter":
        return self.kv(key, ARR, (et, list(items)))

    def tensor(self, name: str, dims: Sequence[int], t: int, data) -> "GGUFWriter":
        raw = np.ascontiguousarray(data).tobytes() if not isinstance(data, (bytes, bytearray)) else bytes(data)
        n = int(np.prod(dims))
        bb, be = TYPE_BLOCK[t]
        assert n % be == 0 and len(raw) == n // be * bb, f"{name}: {len(raw)} bytes for {n} elements of type {t}"
        self.tensors.append((name, tuple(int(d) for d in dims), t, raw))
        return self

    def layout(self) -> Tuple[bytes, List[int], int]:
        """(header bytes, tensor offsets, data offset)."""
        a = self.alignment
        head = struct.pack("<IIQQ", 0x46554747, self.version, len(self.tensors), len(self.kvs))
        for k, t, v in self.kvs:
            head += _str(k) + struct.pack("<I", t) + _value(t, v)
        offs, off = [], 0
        for name, dims, t, raw in self.tensors:
            offs.append(off)
            off = (off + len(raw) + a - 1) // a * a
        for (name, dims, t, raw), o in zip(self.tensors, offs):
            head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", t, o)
        data_off = (len(head) + a - 1) // a * a
        return head, offs, data_off

    def to_bytes(self) -> bytes:
        head, offs, data_off = self.layout()
        out = bytearray(head)
        out += b"\0" * (data_off - len(head))
        for (name, dims, t, raw), o in zip(self.tensors, offs):
            out += b"\0" * (data_off + o - len(out))
            out += raw
        return bytes(out)

    def write(self, path: str) -> str:
        with open(path, "wb") as f:
            f.write(self.to_bytes())
        return path
