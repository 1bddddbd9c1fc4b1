"""Test infrastructure: GGUF version 3 files written byte by byte from the format's description (little-endian; a header
of magic, version, tensor count, metadata count; the metadata entries (key string, value type, value); the tensor
infos (name, n_dims, dims innermost first, ggml type, offset from the data section); padding to the alignment; the
data section). Used to make the files the reader is tested on - valid ones and every kind of broken one."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
          F64: "<d"}
# ggml type id -> (values a block, bytes a block), for the types used here
BLOCK = {0: (1, 4), 12: (256, 144), 16: (256, 66), 18: (256, 98), 19: (256, 50), 29: (256, 56), 30: (1, 2),
         40: (64, 36), 43: (32, 33)}


def s(x):
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def value(t, v, item=None):
    """a value's bytes after its key: type, then the value (for an array: element type, count, elements)"""
    out = struct.pack("<I", t)
    if t == STR:
        return out + s(v)
    if t == ARR:
        out += struct.pack("<IQ", item, len(v))
        for x in v:
            out += s(x) if item == STR else struct.pack(SCALAR[item], x)
        return out
    return out + struct.pack(SCALAR[t], v)


def tensor_bytes(type_, dims):
    values, nbytes = BLOCK[type_]
    n = 1
    for d in dims:
        n *= d
    assert n % values == 0
    return n // values * nbytes


def model(tensors, kv=(), align=None, magic=b"GGUF", version=3, data=None):
    """a whole file: tensors a list of (name, type, dims, payload bytes or None, offset or None); kv a list of
    (key, type, value[, item]). offsets default to consecutive, each aligned; payloads default to a pattern"""
    kvs = list(kv)
    if align is not None:
        kvs = [("general.alignment", U32, align)] + kvs
    a = align or 32
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for e in kvs:
        head += s(e[0]) + value(e[1], e[2], e[3] if len(e) > 3 else None)
    infos, blobs, at = b"", [], 0
    for name, type_, dims, payload, offset in tensors:
        if payload is None:  # (a given payload may be any length: the broken files' own)
            payload = bytes((i * 7 + len(name)) & 255 for i in range(tensor_bytes(type_, dims)))
        off = at if offset is None else offset
        infos += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", type_, off)
        blobs.append((off, payload))
        at = (max(at, off + len(payload)) + a - 1) // a * a
    body = head + infos
    body += b"\0" * ((-len(body)) % a)
    base = len(body)
    blob = bytearray()
    for off, payload in blobs:
        if len(blob) < off + len(payload):
            blob += b"\0" * (off + len(payload) - len(blob))
        blob[off:off + len(payload)] = payload
    return (body + bytes(blob)) if data is None else (body + data), base
