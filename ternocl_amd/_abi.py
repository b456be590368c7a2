"""ctypes signatures of the C ABI (include/ternocl_amd.h).

``SYMBOLS`` lists every exported entry point; tests check that the header
declares exactly these and that the built library exports all of them.
"""
from __future__ import annotations

import ctypes as C

P = C.c_void_p


class GemvTile(C.Structure):
    """ternocl_gemv_tile (include/ternocl_amd.h)."""
    _fields_ = [("engine", C.c_int), ("waves", C.c_int), ("cols_per_lane", C.c_int),
                ("groups_per_wave", C.c_int), ("col_lanes", C.c_int), ("k_slices", C.c_int)]

I = C.c_int
Z = C.c_size_t

# name -> (restype, argtypes)
SYMBOLS: dict[str, tuple] = {
    "ternocl_status_string": (C.c_char_p, [I]),
    "ternocl_last_error": (C.c_char_p, []),
    "ternocl_version": (C.c_char_p, []),
    "ternocl_int2_gemm_ws_bytes": (Z, [I, I, I]),
    "ternocl_workspace_zero": (I, [P, Z, P]),
    "ternocl_int2_fp16_upcvt_gemm": (I, [I, P, P, P, P, P, P, I, I, I, I, I, P, Z, P]),
    "ternocl_int2_fp16_upcvt_gemm_ex": (I, [I, P, P, P, P, P, P, I, I, I, I, I, P, Z,
                                            C.POINTER(GemvTile), P]),
    "ternocl_int2_dequant": (I, [I, P, P, P, I, I, P]),
    "ternocl_int2_gemv_decode": (I, [I, I, P, P, I, I, P]),
    "ternocl_int2_gemv_stream_probe": (I, [I, P, P, P, I, I, I, P]),
    "ternocl_bitcos_fwht_gemm_ws": (I, [I, P, P, I, I, P, P, P, I, P, P, P, I, I, I, I, I, P, Z, P]),
    "ternocl_stream_read_probe": (I, [P, Z, P, P]),
    "ternocl_ldsa": (I, [I]),
    "ternocl_quant_a": (I, [I, P, P, P, I, I, P]),
    "ternocl_int2_int8_gemm": (I, [I, P, P, P, P, P, P, P, P, I, I, I, I, I, P]),
    "ternocl_int2_int8_gemm_ws": (I, [I, P, P, P, P, P, P, P, P, I, I, I, I, I, P, Z, P]),
    "ternocl_int2_int8_gemm_ws_bytes": (Z, [I, I, I]),
    "ternocl_int2_s8_decode": (I, [P, P, I, I, P]),
    "ternocl_bitcos_fp16_upcvt_gemm": (I, [I, P, P, P, P, I, P, P, P, I, I, I, I, I, P]),
    "ternocl_bitcos_fp16_upcvt_gemm_ws": (I, [I, P, P, P, P, I, P, P, P, I, I, I, I, I, P, Z, P]),
    "ternocl_bitcos_gemv_ws_bytes": (Z, [I, I]),
    "ternocl_bitcos_gemm_mt_ws_bytes": (Z, [I, I]),
    "ternocl_bitcos_fp16_upcvt_gemm_mt": (I, [I, P, P, P, P, I, P, P, P, I, I, I, I, I, P, Z, P]),
    "ternocl_bitcos_to_int2": (I, [P, P, I, P, I, I, P]),
    "ternocl_bitcos_slice_ranks": (I, [P, P, I, I, I, P]),
    "ternocl_bitcos_pick_ls": (I, [I, I, I]),
    "ternocl_bitcos_dequant": (I, [I, P, P, P, I, I, P]),
    "ternocl_int2_pack": (I, [P, P, I, I]),
    "ternocl_int2_unpack": (I, [P, P, I, I]),
    "ternocl_bitcos_pack_words": (Z, [P, I, I]),
    "ternocl_bitcos_pack": (I, [P, I, I, P, Z]),
    "ternocl_bitcos_unpack": (I, [P, Z, I, I, P]),
    "ternocl_bitcos_slice_ranks_host": (I, [P, I, I, I, P]),
    "ternocl_hadamard_fwht": (I, [I, P, P, P, I, I, I, I, P]),
    "ternocl_moe_tile_rows": (I, []),
    "ternocl_int2_moe_route": (I, [P, P, P, P, I, I, P]),
    "ternocl_int2_moe_gather": (I, [I, P, P, P, I, I, I, P]),
    "ternocl_int2_moe_gemm": (I, [I, P, P, P, I, P, P, P, P, I, I, I, I, I, I, P]),
    "ternocl_int2_moe_combine": (I, [I, P, P, P, P, I, I, I, P]),
    "ternocl_int2_moe_prefill_ws_bytes": (Z, [I, I, I, I, I]),
    "ternocl_int2_moe_prefill": (I, [I, P, P, P, I, I, I, I, I, P, P, P, P, P, P, P, P, Z, P]),
    "ternocl_int2_moe_prefill_int8_ws_bytes": (Z, [I, I, I, I, I]),
    "ternocl_int2_moe_prefill_int8": (I, [I, P, P, P, I, I, I, I, I, P, P, P, P, P, P, P, P, Z, P]),
    "ternocl_int2_moe_decode_ws_bytes": (Z, [I, I, I, I]),
    "ternocl_int2_moe_decode": (I, [I, P, P, P, I, I, I, I, I, P, P, P, P, P, P, P, P, Z, P]),
    "ternocl_int2_moe_decode_noalloc": (I, [I, P, P, P, I, I, I, I, I, P, P, P, P, P, P, P, P]),
}


def declare(lib: C.CDLL) -> None:
    for name, (res, args) in SYMBOLS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
