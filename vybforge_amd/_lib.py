"""ctypes binding of libvybdq.so (the C-ABI in include/vybdq.h).

The library is loaded from this package directory only (built in-tree by
``python -m vybforge_amd.build``). There is no fallback: if the library is missing or
does not export the declared entry points, importing this module raises.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvybdq.so")

# return codes / enums (include/vybdq.h)
OK = 0
ERR_ARG, ERR_SHAPE, ERR_ALIGN, ERR_HIP, ERR_WORKSPACE = -1, -2, -3, -4, -5
F32, F16, BF16, F64 = 0, 1, 2, 3
Q4_GGML, Q4_INTERLEAVED = 0, 1
EXL3_MCG = 1
MOE_NOALLOC_MAX_BYTES = 64 * 1024 * 1024  # VYBDQ_MOE_NOALLOC_MAX_BYTES
PB_GEMV, PB_GEMM, PB_GEMM_XH = 0x100, 0x200, 0x300
PB_MOE, PB_EXL3DQ, PB_EXL3INV = 0x400, 0x500, 0x600
PB_EXL3HGEN, PB_EXL3HGEN32 = 0x700, 0x701
PB_EXL3HAD1, PB_EXL3HAD132 = 0x800, 0x801
PB_EXL3HAD2, PB_EXL3HAD232 = 0x900, 0x901
PB_EXL3CVT32 = 0xA00

_u64, _i64, _int, _u32 = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32

# name -> argtypes (restype int unless listed in _RESTYPE)
SIGNATURES = {
    "vybdq_abi_version": [],
    "vybdq_last_error": [],
    "vybdq_dequant_q4_0": [_u64, _u64, _i64, _int, _int, _u64],
    "vybdq_dequant_q8_0": [_u64, _u64, _i64, _int, _u64],
    "vybdq_dequant": [_int, _u64, _u64, _i64, _int, _u64],
    "vybdq_gemv": [_int, _u64, _u64, _u64, _i64, _i64, _i64, _int, _int, _u64, _u64],
    "vybdq_gemv_q4_0": [_u64, _u64, _u64, _i64, _i64, _i64, _int, _int, _u64, _int, _u64],
    "vybdq_gemv_q8_0": [_u64, _u64, _u64, _i64, _i64, _i64, _int, _int, _u64, _u64],
    "vybdq_gemv_q4_0_seg3": [_u64, _i64, _int, _int,
                             _u64, _u64, _i64, _int,
                             _u64, _u64, _i64, _int,
                             _u64, _u64, _i64, _int, _u64],
    "vybdq_gemv_seg3": [_int, _u64, _i64, _i64, _int,
                        _u64, _u64, _i64, _int, _u64,
                        _u64, _u64, _i64, _int, _u64,
                        _u64, _u64, _i64, _int, _u64, _u64],
    "vybdq_quant_q8_act": [_u64, _u64, _u64, _i64, _i64, _int, _u64],
    "vybdq_gemv_xq8": [_int, _u64, _u64, _u64, _u64, _i64, _i64, _int, _u64, _u64],
    "vybdq_gemv_xq8_seg3": [_int, _u64, _u64, _i64,
                            _u64, _u64, _i64, _int, _u64,
                            _u64, _u64, _i64, _int, _u64,
                            _u64, _u64, _i64, _int, _u64, _u64],
    "vybdq_gguf_open": [ctypes.c_char_p],
    "vybdq_gguf_close": [_i64],
    "vybdq_gguf_info": [_i64, _int],
    "vybdq_gguf_find_tensor": [_i64, ctypes.c_char_p],
    "vybdq_gguf_find_kv": [_i64, ctypes.c_char_p],
    "vybdq_gguf_tensor_name": [_i64, _i64, ctypes.c_char_p, _i64],
    "vybdq_gguf_tensor_field": [_i64, _i64, _int],
    "vybdq_gguf_kv_key": [_i64, _i64, ctypes.c_char_p, _i64],
    "vybdq_gguf_kv_field": [_i64, _i64, _int],
    "vybdq_gguf_kv_float": [_i64, _i64],
    "vybdq_gguf_kv_string": [_i64, _i64, ctypes.c_char_p, _i64],
    "vybdq_gguf_read_tensor": [_i64, _i64, _int, ctypes.c_void_p, _i64],
    "vybdq_gguf_slab_offset": [_i64, _i64, _i64],
    "vybdq_gguf_slab_bytes": [_i64, _i64],
    "vybdq_gguf_load_slab": [_i64, _u64, _i64, _i64, _int, _u64],
    "vybdq_st_open": [ctypes.c_char_p],
    "vybdq_st_close": [_i64],
    "vybdq_st_info": [_i64, _int],
    "vybdq_st_find": [_i64, ctypes.c_char_p],
    "vybdq_st_tensor_name": [_i64, _i64, ctypes.c_char_p, _i64],
    "vybdq_st_tensor_dtype": [_i64, _i64, ctypes.c_char_p, _i64],
    "vybdq_st_tensor_field": [_i64, _i64, _int],
    "vybdq_st_meta": [_i64, ctypes.c_char_p, ctypes.c_char_p, _i64],
    "vybdq_st_meta_key": [_i64, _i64, ctypes.c_char_p, _i64],
    "vybdq_st_read": [_i64, _i64, ctypes.c_void_p, _i64],
    "vybdq_st_upload": [_i64, _i64, _u64, _i64, _u64],
    "vybdq_st_index_open": [ctypes.c_char_p],
    "vybdq_st_index_close": [_i64],
    "vybdq_st_index_count": [_i64],
    "vybdq_st_index_entry": [_i64, _i64, ctypes.c_char_p, _i64, ctypes.c_char_p, _i64],
    "vybdq_st_index_shard": [_i64, ctypes.c_char_p, ctypes.c_char_p, _i64],
    "vybdq_router_logits": [_u64, _int, _u64, _int, _u64, _int, _i64, _i64, _i64, _u64],
    "vybdq_rmsnorm_q8": [_u64, _u64, _u64, _u64, _u64, _u64, _i64, _i64, ctypes.c_double, _int, _int, _u64],
    "vybdq_swiglu_q8": [_u64, _u64, _u64, _u64, _u64, _i64, _int, _int, _u64],
    "vybdq_chain_workspace_size": [_int],
    "vybdq_gemv_chain": [_int, _u64, _int, _i64, _i64, _u64, _u64],
    "vybdq_chain_status": [_u64],
    "vybdq_exl3_decode_tiles": [_u64, _u64, _i64, _i64, _int, _int, _u64],
    "vybdq_dequant_exl3": [_u64, _u64, _u64, _u64, _i64, _i64, _int, _int, _u64],
    "vybdq_exl3_workspace_size": [_i64, _i64, _i64],
    "vybdq_exl3_gemm": [_u64, _u64, _u64, _u64, _u64, _i64, _i64, _i64, _int, _int, _int, _u64, _i64, _u64],
    "vybdq_gemm": [_int, _u64, _u64, _u64, _i64, _i64, _i64, _int, _int, _i64, _u64, _u64],
    "vybdq_gemm_workspace_size": [_int, _i64, _i64, _i64],
    "vybdq_gemm_ws": [_int, _u64, _u64, _u64, _i64, _i64, _i64, _int, _int, _i64, _u64, _u64, _i64, _u64],
    "vybdq_gemm_q8_0_i8_workspace_size": [_i64, _i64, _i64],
    "vybdq_gemm_q8_0_i8": [_u64, _u64, _u64, _u64, _i64, _i64, _i64, _int, _i64, _u64, _u64, _i64, _u64],
    "vybdq_launch_pblock": [_int, _u64, _u64],
    "vybdq_launch_pblock_grid": [_int, _u64, _u32, _u32, _u64],
    "vybdq_exl3_deq_map": [_u64, _u64, _u64, _int, _u64],
    "vybdq_pblock_status": [],
    "vybdq_moe_route": [_u64, _int, _u64, _u64, _u64, _i64, _i64, _i64, ctypes.c_double, _u64],
    "vybdq_moe_workspace_size": [_i64, _i64, _i64, _i64, _i64],
    "vybdq_moe_forward": [_int, _u64, _int, _u64, _int, _u64, _u64, _u64, _u64, _u64, _u64, _u64, _u64, _int,
                          _u64, _u64, _i64, _i64, _i64, _i64, _i64, ctypes.c_double, ctypes.c_double, _u64,
                          _i64, _u64],
    "vybdq_moe_forward_noalloc": [_int, _u64, _int, _u64, _int, _u64, _u64, _u64, _u64, _u64, _u64, _u64, _u64,
                                  _int, _u64, _u64, _i64, _i64, _i64, _i64, _i64, ctypes.c_double,
                                  ctypes.c_double, _u64],
    "vybdq_moe_exl3_workspace_size": [_i64, _i64, _i64, _i64, _i64],
    "vybdq_moe_forward_exl3": [_u64, _int, _u64, _int, _u64, _u64, _u64, _u64, _u64, _u64, _int, _u64, _u64,
                               _i64, _i64, _i64, _i64, _i64, ctypes.c_double, ctypes.c_double, _u64, _i64, _u64],
}
_RESTYPE = {"vybdq_last_error": ctypes.c_char_p, "vybdq_chain_workspace_size": ctypes.c_int64,
            "vybdq_exl3_workspace_size": ctypes.c_int64, "vybdq_moe_workspace_size": ctypes.c_int64,
            "vybdq_moe_exl3_workspace_size": ctypes.c_int64,
            "vybdq_gemm_workspace_size": ctypes.c_int64, "vybdq_gemm_q8_0_i8_workspace_size": ctypes.c_int64,
            "vybdq_gguf_kv_float": ctypes.c_double}
for _n in ("vybdq_gguf_open", "vybdq_gguf_info", "vybdq_gguf_find_tensor", "vybdq_gguf_find_kv",
           "vybdq_gguf_tensor_name", "vybdq_gguf_tensor_field", "vybdq_gguf_kv_key", "vybdq_gguf_kv_field",
           "vybdq_gguf_kv_string", "vybdq_gguf_read_tensor", "vybdq_gguf_slab_offset", "vybdq_gguf_slab_bytes",
           "vybdq_st_open", "vybdq_st_info", "vybdq_st_find", "vybdq_st_tensor_name", "vybdq_st_tensor_dtype",
           "vybdq_st_tensor_field", "vybdq_st_meta", "vybdq_st_meta_key", "vybdq_st_read", "vybdq_st_upload",
           "vybdq_st_index_open", "vybdq_st_index_count", "vybdq_st_index_entry", "vybdq_st_index_shard"):
    _RESTYPE[_n] = ctypes.c_int64


class VybdqError(RuntimeError):
    def __init__(self, code, where, msg):
        super().__init__(f"{where} failed with code {code}: {msg}")
        self.code = code


def _load():
    # PyTorch ROCm wheels carry their own libamdhip64. Loading torch first lets this library
    # bind to that same runtime; loading this library first would put two HIP runtimes in one
    # process, and torch streams/pointers would not be valid in ours.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libvybdq.so is not built ({LIB_PATH}); run python -m vybforge_amd.build")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the export is missing
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    return lib


lib = _load()


def last_error():
    return lib.vybdq_last_error().decode()


def call(name, *args):
    """Call an entry point; raise VybdqError on a nonzero return code."""
    rc = getattr(lib, name)(*args)
    if rc != OK:
        raise VybdqError(rc, name, last_error())
    return rc
