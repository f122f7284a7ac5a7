"""ctypes binding of libv7g.so (the HIP/gfx950 library; C ABI in include/v7g_lib.h).

The library must have been built (``v7multiplikator_amd.build.build_library()``
or ``__graft_entry__.build()``); there is no fallback path: a missing library
raises at first use.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libv7g.so")

V7G_OK = 0
V7G_ERR_NULL = 1
V7G_ERR_SHAPE = 2
V7G_ERR_ALIGN = 3
V7G_ERR_HIP = 4
V7G_ERR_NO_TABLES = 5
V7G_ERR_ADDRESS = 6
V7G_ERR_ALIAS = 7

_vp = ctypes.c_void_p
_i = ctypes.c_int
_ll = ctypes.c_longlong
_f = ctypes.c_float

# Plain-C (sysv) entries and their signatures.  The ms_abi drop-in entries
# (v7s_*, v7d_quantize) are exported too but are meant for v7_lib.h-style hosts;
# the C++ loadtest calls them.
SIGNATURES = {
    "v7g_init": (_i, []),
    "v7g_set_stream": (None, [_vp]),
    "v7g_get_stream": (_vp, []),
    "v7g_sync": (_i, []),
    "v7g_time_next_call": (_i, [_vp, _vp]),
    "v7g_set_pointer_checks": (None, [_i]),
    "v7g_get_pointer_checks": (_i, []),
    "v7g_check_pointer": (_i, [_vp]),
    "v7g_set_rms_eps": (None, [_f]),
    "v7g_get_rms_eps": (_f, []),
    "v7g_get_last_error": (_i, []),
    "v7g_clear_last_error": (None, []),
    "v7g_error_string": (ctypes.c_char_p, [_i]),
    "v7g_get_rope_tables": (_i, [_vp, _vp, _vp, _vp]),
    "v7g_rope_init": (_i, [_i, _f, _i]),
    "v7g_build_rope_tables": (_i, [_vp, _vp, _i, _i, _f]),
    "v7g_build_rope_tables_llama3": (_i, [_vp, _vp, _i, _i, _f, _f, _f, _f, _i]),
    "v7g_rope_init_llama3": (_i, [_i, _f, _i, _f, _f, _f, _i]),
    "v7g_set_rope_config": (_i, [_i, _f, _f, _f, _f, _i]),
    "v7g_get_rope_config": (_i, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "v7g_clear_rope_config": (None, []),
    "v7g_arith_selfcheck": (_i, [_vp]),
    "v7g_arith_selfcheck_noalloc": (_i, [_vp, _i]),
    "v7g_fused_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f]),
    "v7g_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f]),
    "v7g_rmsnorm_quantize": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _f]),
    "v7g_add_rmsnorm_quantize": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f]),
    "v7g_add_inplace": (_i, [_vp, _vp, _ll]),
    "v7g_rmsnorm_rope_heads": (_i, [_vp, _i, _ll, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _f]),
    "v7g_qk_rmsnorm_rope": (_i, [_vp, _ll, _i, _vp, _vp, _ll, _i, _vp, _i, _i, _vp, _vp, _vp, _i, _i, _i, _f]),
    "v7g_qk_rmsnorm_rope_kv": (_i, [_vp, _ll, _i, _vp, _vp, _ll, _i, _vp, _i, _i, _vp, _vp, _vp, _i, _i, _i, _f,
                                    _vp, _ll, _i]),
    "v7g_kv_pack_f16": (_i, [_vp, _ll, _vp, _ll, _i, _i]),
    "v7g_kv_pack_f16_kv": (_i, [_vp, _ll, _vp, _ll, _vp, _vp, _ll, _i, _i]),
    "v7g_rope_only_heads": (_i, [_vp, _i, _ll, _i, _i, _vp, _vp, _vp, _i, _i, _i]),
    "v7g_qkv_rope_stage": (_i, [_vp]),
    "v7g_swiglu_f32": (_i, [_vp, _vp, _vp, _ll]),
    "v7g_swiglu_q8": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "v7g_quantize_q8": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "v7g_embedding_gather_q8": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i]),
}

# ms_abi drop-in entries (reference names; not callable through ctypes on Linux).
DROP_IN = [
    "v7s_fused_add_rmsnorm",
    "v7s_rmsnorm",
    "v7s_rmsnorm_quantize",
    "v7s_add_inplace",
    "v7s_rmsnorm_rope_heads",
    "v7s_qk_fork_heads",
    "v7d_quantize",
    "v7s_embedding_row",
    "v7s_swiglu_row",
    "v7s_swiglu_quantize_row",
    "v7s_rope_init",
    "v7s_kv_pack_f16",
    "v7s_rope_only_heads",
]


class QkvSide(ctypes.Structure):
    """v7g_qkv_side (include/v7g_lib.h)."""
    _fields_ = [("buf", _vp), ("token_stride", _ll), ("n_heads", _i), ("norm_weight", _vp), ("bias", _vp),
                ("cache", _vp), ("cache_stride", _ll), ("keep_f32", _i)]


class QkvStage(ctypes.Structure):
    """v7g_qkv_stage (include/v7g_lib.h)."""
    _fields_ = [("q", QkvSide), ("k", QkvSide), ("v", QkvSide), ("n_tokens", _i), ("head_dim", _i),
                ("cos_table", _vp), ("sin_table", _vp), ("positions", _vp), ("pos0", _i), ("rope_max_dim", _i),
                ("table_rows", _i), ("eps", _f)]

_lib = None


class V7GError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what}: v7g error {code} ({error_string(code)})")


def load():
    """Returns the loaded library; raises if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: the HIP library has not been built "
                "(run `python -c 'import __graft_entry__ as g; g.build()'`)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def error_string(code: int) -> str:
    s = load().v7g_error_string(int(code))
    return s.decode() if s else "?"


def check(rc: int, what: str) -> None:
    if rc != V7G_OK:
        load().v7g_clear_last_error()
        raise V7GError(rc, what)
