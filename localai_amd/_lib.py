"""ctypes binding of liblocalai_hip.so (the C ABI declared in include/localai_hip.h).

The library is built in-tree by ``python -m localai_amd.build`` (or
``__graft_entry__.build()``). Loading fails loudly: there is no CPU fallback
anywhere in this package.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / 'liblocalai_hip.so'

STATUS = {0: 'OK', 1: 'EARG', 2: 'ETYPE', 3: 'EHIP', 4: 'ENOMEM', 5: 'ESTATE'}

_c_int, _c_i64, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
_u8p, _f32p = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_float)

# name -> (restype, argtypes); mirrors include/localai_hip.h
SIGNATURES = {
    'localai_hip_version': (_c_int, []),
    'localai_hip_init': (_c_int, [_c_int]),
    'localai_hip_last_error': (ctypes.c_char_p, []),
    'localai_hip_last_status': (_c_int, []),
    'localai_hip_block_layout': (_c_int, [_c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    'localai_hip_dequant': (_c_int, [_c_int, _vp, _c_i64, _vp, _vp]),
    'localai_hip_f32_matvec': (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    'localai_hip_ggml_matvec': (_c_int, [_c_int, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    'localai_hip_qmat_create': (_c_int, [_c_int, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp,
                                         ctypes.POINTER(_vp)]),
    'localai_hip_qmat_destroy': (_c_int, [_vp]),
    'localai_hip_qmat_device_bytes': (_c_i64, [_vp]),
    'localai_hip_qmat_unpack': (_c_int, [_vp, _vp, _vp]),
    'localai_hip_qmat_dequant': (_c_int, [_vp, _c_i64, _vp, _vp]),
    'localai_hip_matvec': (_c_int, [_vp, _c_i64, _vp, _vp, _c_int, _vp]),
    'localai_hip_matvec_many': (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp]),
    'localai_hip_matmul_workspace_size': (_c_i64, [_vp, _c_i64]),
    'localai_hip_matmul': (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_int, _vp, _c_i64, _vp]),
    'localai_hip_zaya_router': (_c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _c_i64, _vp, _vp, _c_i64, _vp,
                                         _vp, _c_i64, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    'localai_hip_zaya_scale': (_c_int, [_vp, _vp, _c_i64, _vp, _vp, _vp]),
    'localai_hip_moe_workspace_size': (_c_i64, [_c_i64, _c_i64, _c_int, _c_i64, _c_i64]),
    'localai_hip_moe_table_offsets': (_c_int, [_c_i64, _c_i64, _c_int, _c_i64, _c_i64, _vp]),
    'localai_hip_moe_experts1': (_c_int, [_vp, _c_i64, _vp, _vp, _c_int, _vp, _vp, ctypes.c_int32, _vp, _vp, _c_i64,
                                          _vp]),
    'localai_hip_moe_forward': (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_int, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _c_i64, _vp]),
    'localai_hip_moe_expert_gemm': (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_int, _vp, _c_i64, _c_int, _vp]),
    'localai_hip_static_workspace_bytes': (_c_i64, []),
    'localai_hip_moe_forward_static': (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_int, _vp, _vp, _vp, _vp,
                                                _vp, _vp]),
    'localai_hip_moe_error': (_c_int, [_vp, _c_i64, _c_i64, _vp]),
    'localai_hip_stream_read': (_c_int, [_vp, _c_i64, _vp, _vp]),
    'localai_hip_layer_workspace_size': (_c_i64, [_c_i64, _c_i64]),
    'localai_hip_layer_chain': (_c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _c_int, _c_int,
                                         _vp, _vp, _vp, _vp, _vp, _c_i64, _vp]),
    'localai_hip_layer_chain_mode': (_c_int, [_c_int]),
    'localai_hip_layer_error': (_c_int, [_vp, _vp]),
    'localai_hip_attention_workspace_size': (_c_i64, [_c_i64, _c_int, _c_int, _c_int]),
    'localai_hip_attention_decode': (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int,
                                              _c_i64, _vp, _vp, _vp, _c_i64, _vp]),
    'localai_hip_delta_net_step': (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    'localai_hip_debug_fused_wait': (_c_int, [_c_int, _c_int]),
    'localai_hip_register_host': (_c_int, [_vp, ctypes.c_size_t]),
    'localai_hip_unregister_host': (_c_int, [_vp]),
    'localai_hip_cache_entries': (_c_i64, []),
    'localai_hip_cache_clear': (_c_int, []),
}
for _n in ('q8_0', 'q4_0', 'q4k', 'q5k', 'q6k'):
    SIGNATURES[f'localai_{_n}_matvec'] = (None, [_u8p, _f32p, _f32p, _c_int, _c_int, _c_int])
    SIGNATURES[f'localai_{_n}_matmul'] = (None, [_u8p, _f32p, _f32p, _c_int, _c_int, _c_int, _c_int])


class HipError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f'{STATUS.get(status, status)}: {message}')
        self.status = status


_LIB = None
_LOCK = threading.Lock()


def load():
    """Load the library (once). Raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f'{LIB_PATH} is missing: run `python -m localai_amd.build`')
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _LIB = lib
    return _LIB


def check(status):
    if status != 0:
        msg = load().localai_hip_last_error().decode(errors='replace')
        raise HipError(status, msg)
    return status
