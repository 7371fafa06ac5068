"""Minimal GGUF v2/v3 writer for the tests: the layout the reader parses (include/hymoe.h, hy_gguf_open) --
"GGUF", u32 version, u64 tensor count, u64 key/value count, the key/value pairs, the tensor table, padding to the
alignment, then each tensor's bytes at an aligned offset.  Values are given as (type id, value)."""
import struct
from typing import Iterable, List, Sequence, Tuple

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STR:
        return _str(v)
    if t == ARR:
        at, items = v
        out = struct.pack("<IQ", at, len(items))
        return out + b"".join(_value(at, x) for x in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kv: Sequence[Tuple[str, int, object]], tensors: Sequence[Tuple[str, int, Sequence[int], bytes]],
               alignment: int = 32, version: int = 3, magic: bytes = b"GGUF") -> bytes:
    """kv: (key, type, value) -- arrays as (ARR, (element type, [items])); tensors: (name, ggml type, ne, data)."""
    head = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets: List[int] = []
    off = 0
    for name, gt, ne, data in tensors:
        offsets.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, gt, ne, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
        head += struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    body = bytearray()
    for (name, gt, ne, data), o in zip(tensors, offsets):
        body += b"\0" * (o - len(body)) + data
    return bytes(head) + b"\0" * pad + bytes(body)


def write_gguf(path, kv: Iterable, tensors: Iterable, **kw) -> None:
    with open(path, "wb") as f:
        f.write(gguf_bytes(list(kv), list(tensors), **kw))
