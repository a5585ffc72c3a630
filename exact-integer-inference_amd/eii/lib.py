"""ctypes binding of libeii.so (include/eii.h).

The library is loaded from the package directory, where build.py puts it.  There is no
fallback: a missing or unloadable library raises immediately.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_HERE, "libeii.so")
HOSTCHECK_PATH = os.path.join(_HERE, "libeii_hostcheck.so")

EII_OK, EII_E_IO, EII_E_DEVICE, EII_E_BOUND, EII_E_ARG = 0, 2, 3, 4, 5
KERNEL_KINDS = ("embed", "rmsnorm", "gemm_qkv", "rope", "attention", "gemm_o", "gemm_gate_up", "silu_gate",
                "gemm_down", "gemm_head")

vp, i32, i64p, i32p = C.c_void_p, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int32)


class EIIError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libeii status {code}: {msg}")
        self.code = code


TRACE_SITES = ("norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope", "attn_ctx", "resid_mid",
               "norm2_out", "gate_proj", "up_proj", "mlp_gated",
               "norm1_U", "norm1_z", "attn_score", "attn_prob", "o_res", "norm2_U", "norm2_z", "silu_gate",
               "down_res")


class eii_trace(C.Structure):
    _fields_ = [(n, vp) for n in TRACE_SITES]


# name -> (restype, argtypes); every entry point include/eii.h declares
SIGNATURES = {
    "eii_last_error": (C.c_char_p, []),
    "eii_model_load": (i32, [C.c_char_p, i32, C.POINTER(vp)]),
    "eii_model_free": (None, [vp]),
    "eii_model_set_rope": (i32, [vp, i64p, i64p, i32]),
    "eii_model_rope_rows": (i32, [vp]),
    "eii_model_formats": (i32, [vp, i32, i64p, i64p]),
    "eii_model_set_graphs": (i32, [vp, i32]),
    "eii_forward": (i32, [vp, vp, i32, i32, vp, vp, vp, vp, vp]),
    "eii_forward_packed": (i32, [vp, vp, i32p, i32, vp, vp, vp, vp, vp]),
    "eii_check": (i32, [vp, vp]),
    "eii_kv_create": (i32, [vp, i32, i32, C.POINTER(vp)]),
    "eii_kv_free": (None, [vp]),
    "eii_kv_length": (i32, [vp]),
    "eii_kv_reset": (i32, [vp]),
    "eii_kv_append": (i32, [vp, vp, vp, i32, vp, vp]),
    "eii_argmax": (i32, [vp, i32, i32, vp, vp]),
    "eii_profile_begin": (i32, [vp, i32]),
    "eii_profile_end": (i32, [vp, vp, C.POINTER(C.c_double), i32p]),
    "eii_block": (i32, [vp, i32, vp, i32, i32, C.POINTER(eii_trace), vp]),
    "eii_embed": (i32, [vp, vp, i32, vp, vp]),
    "eii_final": (i32, [vp, vp, i32, vp, vp]),
    "eii_weight_colsum": (i32, [vp, i32, i32, vp, vp]),
    "eii_gemm_i8": (i32, [vp, i32, vp, i32, i32, i32, vp, vp]),
    "eii_gemm_i8_ws": (i32, [vp, i32, vp, vp, i32, i32, i32, vp, vp]),
    "eii_gemm_i8_ws_noalloc": (i32, [vp, i32, vp, vp, i32, i32, i32, vp, vp]),
    "eii_linear": (i32, [vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "eii_rmsnorm": (i32, [vp, i32, vp, i32, i32, i32, vp, vp]),
    "eii_attention": (i32, [vp, vp, i32, i32, vp, i32, i32, i32, i32, i32, vp, vp]),
    "eii_rope": (i32, [vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp]),
    "eii_silu_gate": (i32, [vp, vp, i32, vp, i32, i32, i32, i32, vp, vp]),
}

_lib = None


def load():
    """The loaded libeii.so with typed entry points (raises if it is absent)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EIIError(EII_E_IO, f"{LIB_PATH} is missing: build it with "
                                     "`python exact-integer-inference_amd/build.py`")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc):
    if rc != EII_OK:
        raise EIIError(rc, load().eii_last_error().decode())
    return rc


def load_hostcheck():
    """Host build of the kernels' integer helpers (eii_int.h) and index maps (index_maps.h), for CPU tests."""
    lib = C.CDLL(HOSTCHECK_PATH)
    for n in ("eii_host_rs", "eii_host_sat", "eii_host_norm_U", "eii_host_attn_prob",
              "eii_host_div_floor_q20"):
        getattr(lib, n).restype = C.c_int64
    lib.eii_host_rs.argtypes = [C.c_int64, i32]
    lib.eii_host_sat.argtypes = [C.c_int64, i32]
    lib.eii_host_norm_U.argtypes = [C.c_int64, C.c_int64, C.c_int64]
    lib.eii_host_attn_prob.argtypes = [C.c_int64, C.c_int64]
    lib.eii_host_div_floor_q20.argtypes = [C.c_int64, C.c_int64]
    lib.eii_host_limb_dot.restype = C.c_int64
    lib.eii_host_limb_dot.argtypes = [vp, vp, i32, i32]
    # CPU model of the kernels' index maps (index_maps.h)
    lib.eii_host_gemm_model.restype = C.c_int64
    lib.eii_host_gemm_model.argtypes = [i32, i32, i32, i32, i32, i32, C.c_uint64, i32, vp]
    lib.eii_host_attn_model.restype = C.c_int64
    lib.eii_host_attn_model.argtypes = [C.c_uint64, i32]
    lib.eii_host_attn_digits.restype = C.c_int64
    lib.eii_host_attn_digits.argtypes = [C.c_uint64, i32]
    lib.eii_host_wfrag_model.restype = C.c_int64
    lib.eii_host_wfrag_model.argtypes = [i32, i32]
    return lib
