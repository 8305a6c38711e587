"""A small GGUF v3 writer for the loader tests (test infrastructure).

Writes the container the reference loader reads (qw35-server/src/loader/
tensors.rs:23-121, cursor.rs, metadata.rs:206-288): magic, version, counts,
metadata key/values, tensor infos (name, ndim, dims, type, offset relative to
the data section), padding to the alignment, then the tensor data, each
tensor at an aligned offset.
"""
from __future__ import annotations

import struct

GGUF_MAGIC = 0x46554747

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        item_type, items = v
        return struct.pack("<IQ", item_type, len(items)) + b"".join(_value(item_type, x) for x in items)
    raise ValueError(t)


def build(kv: list[tuple[str, int, object]], tensors: list[tuple[str, tuple, int, bytes]],
          alignment: int = 32, version: int = 3, magic: int = GGUF_MAGIC) -> tuple[bytes, list[dict]]:
    """kv: (key, type, value); tensors: (name, dims, type_id, data bytes).
    Returns (image, [{name, dims, type_id, abs_offset, bytes}])."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(kv))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    rel = []
    off = 0
    for _, _, _, data in tensors:
        off = -(-off // alignment) * alignment
        rel.append(off)
        off += len(data)
    for (name, dims, type_id, _), r in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", type_id, r)
    data_pos = -(-len(head) // alignment) * alignment
    image = bytearray(head + b"\0" * (data_pos - len(head)))
    for (_, _, _, data), r in zip(tensors, rel):
        end = data_pos + r
        image += b"\0" * (end - len(image))
        image += data
    info = [{"name": n, "dims": tuple(d), "type_id": t, "abs_offset": data_pos + r, "bytes": len(b)}
            for (n, d, t, b), r in zip(tensors, rel)]
    return bytes(image), info
