"""GGUF model files through the library's reader (include/osmos/model/gguf.h: gguf_create and friends), and expert
slices of a model's tensors on the device for the lane layer (libosmos_amd.layer.LaneLayer).

A model's metadata and tensor places come from gguf_create (the reference's reader's checks: src/model/gguf.c); a
tensor's bytes are read from its file in place (numpy.memmap over [offset, offset + bytes)) and copied to the device
as they are - GGUF rows of whole blocks, the layout every kernel here reads. An expert tensor (llama.cpp's
`blk.N.ffn_{gate,up,down}_exps.weight`: dims [cols, rows, n_exp]) is n_exp matrices back to back, `bytes / n_exp` apart:
exactly what OsmosLaneLayer's gate / up / down with *_bytes take.
"""
import ctypes

import numpy as np

from . import capi

VALUE_SIZE = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
ARRAY_DTYPE = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
               7: np.uint8, 10: np.uint64, 11: np.int64, 12: np.float64}
STRING, ARRAY = 8, 9


class GgufError(ValueError):
    pass


class Model:
    """an open model (gguf_create, or gguf_header with header_only); close() or a with-block frees it"""

    def __init__(self, path, header_only=False):
        L = capi.lib()
        err = ctypes.create_string_buffer(capi.GGUF_ERR)
        fn = L.gguf_header if header_only else L.gguf_create
        self._g = fn(path.encode(), err)
        if not self._g:
            raise GgufError(err.value.decode(errors="replace"))
        g = self._g.contents
        self.paths = [g.paths[i].decode() for i in range(g.n_files)]
        self.sizes = [int(g.sizes[i]) for i in range(g.n_files)]
        self.tensors = {}
        for i in range(g.n_tensors):
            t = g.tensors[i]
            self.tensors[t.name.decode()] = {"type": int(t.type), "dims": [int(t.dims[d]) for d in range(t.n_dims)],
                                            "file": int(t.file), "offset": int(t.offset), "bytes": int(t.bytes)}
        self.kv = {}
        for i in range(g.n_kv):
            k = g.kv[i]
            self.kv[k.key.decode()] = _value(k)

    def close(self):
        if self._g:
            capi.lib().gguf_destroy(self._g)
            self._g = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def raw(self, name):
        """the tensor's bytes, in place (a read-only memmap of its file's range)"""
        t = self.tensors[name]
        return np.memmap(self.paths[t["file"]], dtype=np.uint8, mode="r", offset=t["offset"], shape=(t["bytes"],))

    def experts(self, name, torch, device="cuda"):
        """an expert tensor (dims [cols, rows, n_exp]) on the device as (n_exp, bytes an expert) uint8, with its type,
        rows and cols"""
        t = self.tensors[name]
        if len(t["dims"]) != 3:
            raise GgufError("%s: not an expert tensor (dims %s)" % (name, t["dims"]))
        cols, rows, n_exp = t["dims"]
        host = np.asarray(self.raw(name)).reshape(n_exp, -1)
        dev = torch.empty(host.shape, dtype=torch.uint8, device=device)
        dev.copy_(torch.from_numpy(np.array(host, copy=True)))  # (the map is read-only: a host copy, then the device)
        return dev, t["type"], rows, cols


def _value(k):
    if k.type == STRING:
        return k.v.s.decode(errors="replace") if k.v.s else ""
    if k.type == ARRAY:
        if k.item == STRING:
            arr = ctypes.cast(k.v.items, ctypes.POINTER(ctypes.c_char_p))
            return [arr[i].decode(errors="replace") for i in range(k.n)]
        dt = ARRAY_DTYPE[k.item]
        n = int(k.n)
        if n == 0:
            return np.zeros(0, dt)
        buf = (ctypes.c_uint8 * (n * np.dtype(dt).itemsize)).from_address(k.v.items)
        return np.frombuffer(bytes(buf), dtype=dt)
    if k.type in (1, 3, 5, 11):
        return int(k.v.i)
    if k.type in (6, 12):
        return float(k.v.f)
    if k.type == 7:
        return bool(k.v.u)
    return int(k.v.u)
