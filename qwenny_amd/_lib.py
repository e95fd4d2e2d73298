"""ctypes bindings of libqwenny_hip.so (include/qwenny_hip.h). Loading fails loudly when the library is missing: there
is no CPU fallback for any product."""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QWENNY_HIP_LIB") or os.path.join(HERE, "libqwenny_hip.so")  # QWENNY_HIP_LIB: another build (tuning)

P, S, I, U64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64


class QuantC(ctypes.Structure):
    """qh_quant (checkpoint.rs:21-31 Quant)"""

    _fields_ = [("bits", ctypes.c_int32), ("group", ctypes.c_int32), ("rows", S), ("cols", S), ("q", P),
                ("scales", P), ("offsets", P)]


class MatDesc(ctypes.Structure):
    """qh_mat_desc"""

    _fields_ = [("wt", ctypes.c_int32), ("rows", S), ("cols", S), ("valid", S), ("code_bytes", S),
                ("scale_bytes", S), ("zero_bytes", S), ("per_channel", ctypes.c_int32)]


class LoraC(ctypes.Structure):
    """qh_lora (the reference's lora_add / lora_silu arguments)"""

    _fields_ = [("xa", P), ("split", ctypes.c_int32), ("m_cols", ctypes.c_int32), ("b_f16", P),
                ("rank", ctypes.c_int32), ("tab", P), ("tok_slot", P), ("slot_scale", P)]


# name -> (restype, argtypes); every symbol include/qwenny_hip.h declares
SIGNATURES = {
    "qh_last_error": (ctypes.c_char_p, []),
    "qh_quant_from_packed": (I, [P, S, S, S, I, I, P, P, S, S, P, P, ctypes.POINTER(QuantC)]),
    "qh_quant_zero_points": (I, [ctypes.POINTER(QuantC), P]),
    "qh_quant_row_into": (I, [ctypes.POINTER(QuantC), S, P]),
    "qh_row_order": (I, [S, I, P]),
    "qh_packed_sizes": (I, [I, S, S, ctypes.POINTER(S), ctypes.POINTER(S), ctypes.POINTER(S)]),
    "qh_pack_quant": (I, [ctypes.POINTER(QuantC), P, P, S, I, P, P, P]),
    "qh_unpack_row": (I, [I, S, S, P, P, P, S, P, P, P]),
    "qh_pack_dense_int8": (I, [P, S, S, P, S, P, P]),
    "qh_open": (I, [I, ctypes.POINTER(P)]),
    "qh_close": (None, [P]),
    "qh_mat_upload": (I, [P, I, S, S, P, P, P, S, ctypes.POINTER(P)]),
    "qh_mat_quant": (I, [P, ctypes.POINTER(QuantC), I, ctypes.POINTER(P)]),
    "qh_mat_quant_rows": (I, [P, ctypes.POINTER(QuantC), P, P, S, S, ctypes.POINTER(P)]),
    "qh_mat_dense_int8": (I, [P, P, S, S, I, ctypes.POINTER(P)]),
    "qh_mat_dense": (I, [P, P, S, S, I, ctypes.POINTER(P)]),
    "qh_quant_to_bf16": (I, [ctypes.POINTER(QuantC), P]),
    "qh_dequant": (I, [P, P, P, P, S, S, S, I, I, S, S, P, I]),
    "qh_diag_read": (I, [P, P, S, S, I, P]),
    "qh_graph_begin": (I, [P]),
    "qh_graph_end": (I, [P, ctypes.POINTER(P)]),
    "qh_graph_launch": (I, [P, P]),
    "qh_graph_free": (None, [P]),
    "qh_sum_parts": (I, [P, P, I, S, S, P]),
    "qh_add_rmsnorm": (I, [P, P, P, I, S, S, P, P, ctypes.c_float]),
    "qh_lora_add": (I, [P, P, I, I, P, I, S, P, P, P, S, P, S]),
    "qh_lora_silu": (I, [P, P, I, I, P, I, S, P, P, P, S, P, S, P]),
    "qh_pack_dense_bf16": (I, [P, S, S, P, S, P]),
    "qh_unpack_row_bf16": (I, [S, S, P, S, P]),
    "qh_mat_free": (None, [P]),
    "qh_mat_describe": (I, [P, ctypes.POINTER(MatDesc)]),
    "qh_mat_download": (I, [P, P, P, P]),
    "qh_mat_split": (I, [P, P, S]),
    "qh_mat_kernel": (I, [P, P, S, I, I]),
    "qh_part_len": (S, [P, P, S, S]),
    "qh_gemm": (I, [P, P, P, P, S, S, P, S, P, I, P, I]),
    "qh_gemm_noalloc": (I, [P, P, P, P, S, S, P, S, P, I, P, I]),
    "qh_gemm_lora": (I, [P, P, P, P, S, S, P, I, I, ctypes.POINTER(LoraC)]),
    "qh_put_block": (I, [P, P, P, ctypes.POINTER(QuantC), P, S, P]),
}

_lib = None


class QhError(RuntimeError):
    """A libqwenny_hip call returned an error status."""

    def __init__(self, code, msg):
        super().__init__(f"{msg} (status {code})")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `python qwenny_amd/build.py` (no CPU fallback exists)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(handle, name)
            f.restype = res
            f.argtypes = args
        _lib = handle
    return _lib


def check(rc):
    """Raise QhError for a negative status; return it otherwise."""
    if rc is not None and rc < 0:
        raise QhError(rc, lib().qh_last_error().decode())
    return rc
