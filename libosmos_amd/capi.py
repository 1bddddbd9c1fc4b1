"""ctypes bindings of libosmos_mi355x.so's C ABI (the declarations in include/osmos/gpu/*.h, include/osmos/model/gguf.h
and include/osmos_mi355x.h), argument for argument: pointers are device addresses (a torch tensor's data_ptr() or a
hipMalloc'd address), `stream` a hipStream_t (torch.cuda.current_stream().cuda_stream) or None for the default.

the library is never replaced by anything else: if libosmos_mi355x.so is missing, lib() raises - there is no CPU
fallback on the product path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libosmos_mi355x.so")

P = ctypes.c_void_p
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
F32 = ctypes.c_float
B = ctypes.c_bool

# name -> (restype, argtypes); the exact C signatures
SIGS = {
    "q8_round": (B, [P, U32, U32, U32, P, P, P]),
    "q8_group_tok": (B, [U32, P, P, P, P, U32, U32, U32, U32, P, P, P, U32, P]),
    "q8_gate_up": (B, [U32, P, P, P, P, P, P, U32, U32, U32, U32, P, P, P, F32, P, U32, P]),
    "mv_run": (B, [U32, P, U32, U32, P, U32, P, P]),
    "mv_group": (B, [U32, P, U32, U32, U32, P, U32, U32, P, P]),
    "mv_group_tok": (B, [U32, P, P, P, U32, U32, U32, U32, P, U32, P, U32, P]),
    "mv_strided": (B, [U32, P, U32, U32, P, U32, U32, P, U32, P]),
    "quant_known": (B, [U32]),
    "mmq_known": (B, [U32]),
    "mmq_x8_rows": (B, [P, U32, P, U32, U32, P, P, P, P]),
    "mmq_group": (B, [U32, P, P, U32, U32, U32, U32, P, P, P, P, P, P, U32, P]),
    "q4x_route": (B, [P, U32, U32, U32, P, P, P, P]),
    "q4x_expert_bounds": (None, [U32, U32, P]),
    "q4x_expert_tiles": (B, [P, U32, U32, U32, U32, U32, P, P]),
    "q4x_moe_sum": (B, [P, P, P, U32, U32, U32, P, P, P, P]),
    "q4x_swiglu_rows": (B, [P, P, U32, P, U32, P, P, P]),
    "q4x_swiglu": (B, [P, P, U64, P, P, P]),
    "q4x_spin": (B, [U32, P]),
    "ops_wait": (B, [P, U32, P]),
    "osmos_wait_limit": (None, [U64]),
    "ops_copy_rows": (B, [P, P, P, U32, U32, P]),
    "mm_known": (B, [U32]),
    "mm_fits": (B, [U32, U32, U32]),
    "mm_col_tiles": (U32, [U32, U32]),
    "mm_x16": (B, [P, U32, U32, U32, P, P, P]),
    "mm_x16_rows": (B, [P, U32, P, U32, U32, P, P, P]),
    "mm_run": (B, [U32, P, U32, U32, P, U32, P, U32, P]),
    "mm_group": (B, [U32, P, P, U32, U32, U32, U32, P, P, U32, P, P, U32, P]),
    "ops_swiglu_lane": (B, [P, P, U32, F32, P, U32, P, P]),
    "ops_gather_rows": (B, [P, P, P, U32, U32, P]),
    "ops_gather_sum_add": (B, [P, P, P, U32, U32, U32, P, P]),
    "osmos_lane_tables": (B, [P, U32, U32, U32, P, P, P, P, P, P, P, P, P, P, P]),
    "quant_dequant": (B, [U32, P, U64, P, P]),
    "quant_dequant_f16": (B, [U32, P, U64, P, P]),
    "quant_repack_q5k": (B, [P, U32, U32, P, P]),
}



class OsmosLaneLayer(ctypes.Structure):
    """include/osmos_mi355x.h's OsmosLaneLayer"""
    _fields_ = [("type_gu", U32), ("type_down", U32), ("dim", U32), ("ff", U32), ("n_exp", U32), ("k", U32),
                ("lim", F32), ("gate", P), ("up", P), ("down", P), ("gate_bytes", U64), ("up_bytes", U64),
                ("down_bytes", U64)]


class Q4xExpertTiles(ctypes.Structure):
    """include/osmos/gpu/q4x_ops.h's Q4xExpertTiles"""
    _fields_ = [("base", P * 3), ("bytes", U64 * 3), ("tab", P * 3), ("ptr", P * 3), ("cnt", P), ("gidx", P),
                ("hidx", P), ("xg", P), ("yg", P), ("xd", P), ("yd", P), ("where", P), ("off", P)]


class Q4xX16(ctypes.Structure):
    """include/osmos/gpu/q4x_ops.h's Q4xX16"""
    _fields_ = [("x16", P), ("overflow", P), ("cols", U32), ("row0", U32)]


class Q4xExpertBounds(ctypes.Structure):
    _fields_ = [("first", U32 * 4), ("count", U32 * 4), ("entries", U32), ("slots", U32)]


SIGS.update({
    "osmos_lane_workspace": (U64, [ctypes.POINTER(OsmosLaneLayer), U32]),
    "osmos_lane_layer": (B, [ctypes.POINTER(OsmosLaneLayer), P, U32, P, P, P, P, P, U64, P]),
    "osmos_lane_layer_noalloc": (B, [ctypes.POINTER(OsmosLaneLayer), P, U32, P, P, P, P, P]),
    "osmos_lane_gate_up": (B, [ctypes.POINTER(OsmosLaneLayer), P, U32, P, P, P, P]),
    "osmos_lane_down": (B, [ctypes.POINTER(OsmosLaneLayer), P, U32, P, P, P, P]),
    "osmos_lane_group": (B, [U32, P, P, P, U32, U32, U32, U32, P, P, P, U32, P]),
})



# include/osmos/gpu/quant.h
QUANT_Q5_K = 13
QUANT_Q5_KR = 0x100 | QUANT_Q5_K
QUANT_Q5_KR_BYTES_A_BLOCK = 180


def quant_q5kr_bytes(rows, cols):
    return rows * (cols // 256) * QUANT_Q5_KR_BYTES_A_BLOCK


# include/osmos/model/gguf.h (host memory: the GGUF reader touches no GPU)
GGUF_ERR = 256
GGUF_MAX_DIMS = 4


class GgufValue(ctypes.Union):
    _fields_ = [("u", ctypes.c_uint64), ("i", ctypes.c_int64), ("f", ctypes.c_double), ("s", ctypes.c_char_p),
                ("items", P)]


class GgufKv(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("type", ctypes.c_int), ("item", ctypes.c_int), ("n", U64), ("v", GgufValue)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", U32), ("n_dims", U32), ("dims", U64 * GGUF_MAX_DIMS),
                ("file", ctypes.c_int), ("offset", U64), ("bytes", U64)]


class Gguf(ctypes.Structure):
    _fields_ = [("n_files", ctypes.c_int), ("paths", ctypes.POINTER(ctypes.c_char_p)), ("sizes", ctypes.POINTER(U64)),
                ("kv", ctypes.POINTER(GgufKv)), ("n_kv", ctypes.c_size_t), ("tensors", ctypes.POINTER(GgufTensor)),
                ("n_tensors", ctypes.c_size_t)]


SIGS.update({
    "gguf_create": (ctypes.POINTER(Gguf), [ctypes.c_char_p, ctypes.c_char_p]),
    "gguf_header": (ctypes.POINTER(Gguf), [ctypes.c_char_p, ctypes.c_char_p]),
    "gguf_destroy": (None, [ctypes.POINTER(Gguf)]),
    "gguf_tensor": (ctypes.POINTER(GgufTensor), [ctypes.POINTER(Gguf), ctypes.c_char_p]),
    "gguf_kv": (ctypes.POINTER(GgufKv), [ctypes.POINTER(Gguf), ctypes.c_char_p]),
    "gguf_bytes": (U64, [U32, U64]),
    "gguf_int": (B, [ctypes.POINTER(GgufKv), ctypes.c_size_t, ctypes.POINTER(ctypes.c_int64)]),
})



# include/osmos/cpu/lane.h (host threads: the lane's CPU half touches no GPU)
CPU_LANE_FAILED = 0x80000000


class CpuLaneExpert(ctypes.Structure):
    _fields_ = [("gate", P), ("up", P), ("down", P), ("row0", U32), ("cnt", U32)]


class CpuLaneJob(ctypes.Structure):
    _fields_ = [("type_gu", U32), ("type_down", U32), ("dim", U32), ("ff", U32), ("lim", F32), ("x", P),
                ("scale", P), ("n_rows", U32), ("e", ctypes.POINTER(CpuLaneExpert)), ("n_e", U32), ("y", P),
                ("seq", P), ("value", U32)]


SIGS.update({
    "cpu_lane_create": (P, [ctypes.c_int, P, U32, U32, U32]),
    "cpu_lane_destroy": (None, [P]),
    "cpu_lane_submit": (B, [P, ctypes.POINTER(CpuLaneJob)]),
    "cpu_lane_wait": (B, [P]),
})

_lib = None


class MissingLibrary(RuntimeError):
    pass


def lib():
    """the loaded library (built by `python -m libosmos_amd.build` or __graft_entry__.build())"""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MissingLibrary("%s is not built: run python -m libosmos_amd.build (no fallback exists)" % LIB_PATH)
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGS.items():
            if hasattr(h, name):
                f = getattr(h, name)
                f.restype, f.argtypes = res, args
        _lib = h
    return _lib


def addr(t):
    """a tensor's device address (None for None)"""
    return None if t is None else ctypes.c_void_p(t.data_ptr())
