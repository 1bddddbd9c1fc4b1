"""A routed MoE layer over the lane's int8 contract, for Python callers: the experts' three tensors resident on the
device, one call of the C ABI's osmos_lane_layer a step (include/osmos_mi355x.h). The workspace is allocated (zeroed) once per
token count and reused; nothing here computes - every step is the library's kernels on the given stream.
"""
import ctypes
import math

from . import capi


class LaneLayer:
    def __init__(self, type_gu, type_down, dim, ff, n_exp, k, gate, up, down, lim=math.inf):
        """gate / up / down: uint8 device tensors [n_exp, bytes an expert] in GGUF row layout"""
        import torch
        self.torch = torch
        self.tensors = (gate, up, down)
        self.desc = capi.OsmosLaneLayer(type_gu, type_down, dim, ff, n_exp, k, lim, gate.data_ptr(), up.data_ptr(),
                                        down.data_ptr(), gate[0].numel(), up[0].numel(), down[0].numel())
        self.dim, self.k = dim, k
        self._ws = {}

    def workspace(self, n_tok):
        if n_tok not in self._ws:
            nbytes = capi.lib().osmos_lane_workspace(ctypes.byref(self.desc), n_tok)
            ws = self.torch.zeros(nbytes + 256, dtype=self.torch.uint8, device="cuda")
            off = (-ws.data_ptr()) % 256
            self._ws[n_tok] = (ws, ws.data_ptr() + off, nbytes)
        return self._ws[n_tok]

    def forward(self, x, ids, w, add, out, stream=None):
        """x [n_tok, dim] f32, ids [n_tok, k] int32, w [n_tok, k] f32, add / out [n_tok, dim] f32 (device tensors)"""
        n_tok = x.shape[0]
        _, ws, nbytes = self.workspace(n_tok)
        ok = capi.lib().osmos_lane_layer(ctypes.byref(self.desc), capi.addr(x), n_tok, capi.addr(ids), capi.addr(w),
                                         capi.addr(add), capi.addr(out), ctypes.c_void_p(ws), nbytes, stream)
        if not ok:
            raise RuntimeError("osmos_lane_layer refused")
        return out
