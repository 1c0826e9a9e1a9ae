"""questwend_amd -- QuestWend's MoE expert hot path on one AMD Instinct MI355X.

The product is the C-ABI library ``libqwmoe.so`` (declared in
``include/qwmoe.h``): router top-k, GGML_OP_MUL_MAT_ID over Q4_K expert slot
pools, SwiGLU, the gate-weighted combine (+ shared expert), the verify head
with greedy MTP acceptance, and the GPU LRU slot pool with its slab fetch.
This module is the thin ctypes binding over that ABI that tests, the
benchmark and Python callers use; it holds no compute of its own and raises
if the library was not built (there is no CPU fallback).
"""
import ctypes
import os

__all__ = ["lib", "QwmError", "QwmTensor", "MoeLayer", "PoolDesc", "PoolSig", "PoolSigDesc", "PoolStats", "tensor",
           "check",
           "TYPE_F32", "TYPE_Q8_0", "TYPE_Q4_K", "TYPE_Q5_K", "TYPE_Q6_K", "TYPE_I32", "FETCH_MEMCPY", "FETCH_GATHER"]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqwmoe.so")

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_I32 = 0, 8, 12, 13, 14, 26
FETCH_MEMCPY, FETCH_GATHER = 0, 1
NOALLOC_SCRATCH_BYTES = 4 << 20        # QWM_NOALLOC_SCRATCH_BYTES
_TYPE_SIZE = {TYPE_F32: (4, 1), TYPE_I32: (4, 1), TYPE_Q8_0: (34, 32), TYPE_Q4_K: (144, 256), TYPE_Q5_K: (176, 256),
              TYPE_Q6_K: (210, 256)}

OK, ERR_UNSUPPORTED, ERR_ARG, ERR_WORKSPACE, ERR_HIP, ERR_NO_VICTIM, ERR_STATE, ERR_IO = 0, -1, -2, -3, -4, -5, -6, -7
ERR_NOMEM, ERR_INTERNAL = -8, -9

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t


class QwmError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libqwmoe error {code}: {msg}")
        self.code = code


class QwmTensor(ctypes.Structure):
    """struct qwm_tensor (mirrors ggml_tensor's type/ne/nb/data)."""
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                ("data", ctypes.c_void_p)]


class MoeLayer(ctypes.Structure):
    """struct qwm_moe_layer."""
    _fields_ = [("gate_pool", QwmTensor), ("up_pool", QwmTensor), ("down_pool", QwmTensor),
                ("router", QwmTensor), ("sh_gate", QwmTensor), ("sh_up", QwmTensor), ("sh_down", QwmTensor),
                ("sh_gate_inp", QwmTensor), ("n_expert_used", ctypes.c_int32), ("norm_weights", ctypes.c_int32),
                ("weights_scale", ctypes.c_float), ("gating_func", ctypes.c_int32), ("exp_probs_b", QwmTensor)]


class PoolDesc(ctypes.Structure):
    """struct qwm_pool_desc."""
    _fields_ = [("n_layer", ctypes.c_int32), ("n_expert", ctypes.c_int32), ("n_slots", ctypes.c_int32 * 3),
                ("pool_data", ctypes.c_void_p * 3), ("slab_bytes", ctypes.c_size_t * 3),
                ("host_slabs", ctypes.c_void_p * 3), ("protect_active", ctypes.c_int32),
                ("indexed", ctypes.c_int32), ("fetch_mode", ctypes.c_int32)]


class PoolSig(ctypes.Structure):
    """struct qwm_pool_sig: one signature pool (role, type, ne0, ne1)."""
    _fields_ = [("role", ctypes.c_int32), ("type", ctypes.c_int32), ("ne0", ctypes.c_int64), ("ne1", ctypes.c_int64),
                ("slab_bytes", ctypes.c_size_t), ("n_layers", ctypes.c_int32), ("n_slots", ctypes.c_int32),
                ("pool_data", ctypes.c_void_p)]


class PoolSigDesc(ctypes.Structure):
    """struct qwm_pool_sig_desc."""
    _fields_ = [("n_layer", ctypes.c_int32), ("n_expert", ctypes.c_int32), ("n_pools", ctypes.c_int32),
                ("pools", ctypes.POINTER(PoolSig)), ("layer_pool", ctypes.c_void_p),
                ("host_slabs", ctypes.c_void_p * 3), ("protect_active", ctypes.c_int32),
                ("indexed", ctypes.c_int32), ("fetch_mode", ctypes.c_int32)]


class PoolStats(ctypes.Structure):
    _fields_ = [("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64), ("evictions", ctypes.c_uint64),
                ("fetch_bytes", ctypes.c_uint64), ("fetches", ctypes.c_uint64), ("clock", ctypes.c_uint64)]


_lib = None


class GgufTensor(ctypes.Structure):
    """struct qwm_gguf_tensor."""
    _fields_ = [("type", ctypes.c_int32), ("n_dims", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


def lib():
    """Loads libqwmoe.so (built in-tree by __graft_entry__.build()); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB_PATH)
    T = ctypes.POINTER(QwmTensor)
    sig = {
        "qwm_tensor_init": (None, [T, _I32, _I64, _I64, _I64, _P]),
        "qwm_version": (ctypes.c_char_p, []),
        "qwm_last_error": (ctypes.c_char_p, []),
        "qwm_workspace_init": (ctypes.c_int, [_P, _SZ, _P]),
        "qwm_mul_mat_id_workspace_size": (_SZ, [T, T, T]),
        "qwm_mul_mat_id": (ctypes.c_int, [T, T, T, T, _P, _SZ, _P]),
        "qwm_swiglu": (ctypes.c_int, [T, T, T, _P]),
        "qwm_mul_mat_id_swiglu_workspace_size": (_SZ, [T, T, T, T]),
        "qwm_mul_mat_id_swiglu": (ctypes.c_int, [T, T, T, T, T, _P, _SZ, _P]),
        "qwm_moe_workspace_size": (_SZ, [ctypes.POINTER(MoeLayer), _I64]),
        "qwm_moe_route": (ctypes.c_int, [ctypes.POINTER(MoeLayer), T, T, T, T, _P, _SZ, _P]),
        "qwm_moe_experts": (ctypes.c_int, [ctypes.POINTER(MoeLayer), T, T, T, T, T, T, T, _P, _SZ, _P]),
        "qwm_moe_block_resident": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _I32, _P, _I64, T, T, T, T, T, T,
                                                  _P, _SZ, _P]),
        "qwm_moe_decode_workspace_size": (_SZ, [ctypes.POINTER(MoeLayer), _I32, _I64]),
        "qwm_moe_decode": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _I32, _P, _I64, T, _P, _SZ, _P]),
        "qwm_moe_decode_sel": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _I32, _P, _I64, T, _P, _P, _P, _P, _SZ, _P]),
        "qwm_pool_resident_bits": (ctypes.c_int, [_P, _I32, _P]),
        "qwm_pool_touch": (ctypes.c_int, [_P, _I32, _P, _I32]),
        "qwm_pool_capacity": (ctypes.c_int, [_P, _I32]),
        "qwm_pool_quota_of": (ctypes.c_int, [_P, _I32]),
        "qwm_pool_quotas_active": (ctypes.c_int, [_P]),
        "qwm_pool_set_quotas": (ctypes.c_int, [_P, _I32]),
        "qwm_pool_plan_slices": (ctypes.c_int, [_P, _I32, _P, _I32, _I32, _I32, _P, _P, _P]),
        "qwm_moe_cached_batch_workspace_size": (_SZ, [ctypes.POINTER(MoeLayer), _I64, _I32]),
        "qwm_moe_cached_batch": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _P, _I32, T, T, T, T, _I32, _P, _P, _P, _P,
                                                _SZ, _P]),
        "qwm_verify_workspace_size": (_SZ, [T, _I64]),
        "qwm_verify_accept": (ctypes.c_int, [T, T, _P, ctypes.c_float, _P, _P, _P, _SZ, _P]),
        "qwm_verify_step_workspace_size": (_SZ, [ctypes.POINTER(MoeLayer), T, _I64]),
        "qwm_verify_step": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _I32, _P, _I64, T, T, T, T, T, T, T,
                                           _P, ctypes.c_float, _P, _P, _P, _SZ, _P]),
        "qwm_verify_step_noalloc": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _I32, _P, _I64, T, T, T, T, T, T, T,
                                                   _P, ctypes.c_float, _P, _P, _P]),
        "qwm_pool_create": (ctypes.c_int, [ctypes.POINTER(PoolDesc), _P, ctypes.POINTER(_P)]),
        "qwm_pool_destroy": (None, [_P]),
        "qwm_pool_create_sig": (ctypes.c_int, [ctypes.POINTER(PoolSigDesc), _P, ctypes.POINTER(_P)]),
        "qwm_pool_plan_sigs": (ctypes.c_int, [_I32, _I32, T, ctypes.c_uint64, _I32, ctypes.POINTER(PoolSig), _I32, _P,
                                              _P, _P]),
        "qwm_pool_layer_pool": (ctypes.c_int, [_P, _I32, _I32]),
        "qwm_pool_ensure": (ctypes.c_int, [_P, _I32, _P, _I32, _P, _P, _P]),
        "qwm_pool_wait": (ctypes.c_int, [_P, _P]),
        "qwm_pool_get_stats": (ctypes.c_int, [_P, ctypes.POINTER(PoolStats)]),
        "qwm_pool_slot_of_row": (ctypes.c_int, [_P, _I32, _I32, _P]),
        "qwm_pool_slots": (ctypes.c_int, [_P, _I32, _P, _P]),
        "qwm_pool_attach_file": (ctypes.c_int, [_P, _I32, _I32, ctypes.c_char_p, ctypes.c_uint64]),
        "qwm_pool_set_io": (ctypes.c_int, [_P, _I32, _I32]),
        "qwm_pool_rebalance": (ctypes.c_int, [_P, _I32, _I64, _P, _P]),
        "qwm_pool_clear_counts": (ctypes.c_int, [_P]),
        "qwm_moe_cached_workspace_size": (_SZ, [ctypes.POINTER(MoeLayer), _I64]),
        "qwm_moe_cached_step": (ctypes.c_int, [ctypes.POINTER(MoeLayer), _P, _I32, T, T, T, T, _P, _P, _SZ, _P]),
        "qwm_gguf_find_tensor": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]),
        "qwm_pool_attach_gguf": (ctypes.c_int, [_P, ctypes.c_char_p, _I32]),
        "qwm_pool_save_profile": (ctypes.c_int, [_P, ctypes.c_char_p]),
        "qwm_pool_load_profile": (ctypes.c_int, [_P, ctypes.c_char_p, _P]),
        "qwm_slab_fetch_async": (ctypes.c_int, [_P, _SZ, _I32, _P, _P, _P]),
        "qwm_quantize": (ctypes.c_int, [_I32, _P, _P, _I64, _P]),
        "qwm_profile_start": (ctypes.c_int, [ctypes.c_char_p, _I32]),
        "qwm_profile_stop": (ctypes.c_int, [_P, _I32]),
        "qwm_set_spin_limit": (ctypes.c_int, [ctypes.c_uint32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc):
    if rc != OK:
        raise QwmError(rc, lib().qwm_last_error().decode(errors="replace"))
    return rc


def tensor(type_, ne0, ne1=1, ne2=1, data=None):
    """A contiguous qwm_tensor; `data` is a device pointer (int) or a torch tensor."""
    t = QwmTensor()
    if data is not None and hasattr(data, "data_ptr"):
        data = data.data_ptr()
    ts, bl = _TYPE_SIZE[type_]
    if ne0 % bl:
        raise ValueError(f"ne0={ne0} is not a multiple of the block size {bl}")
    t.type = type_
    t.ne[0], t.ne[1], t.ne[2], t.ne[3] = ne0, ne1, ne2, 1
    t.nb[0] = ts
    t.nb[1] = ts * (ne0 // bl)
    t.nb[2] = t.nb[1] * ne1
    t.nb[3] = t.nb[2] * ne2
    t.data = data
    return t


def row_bytes(type_, ne0):
    ts, bl = _TYPE_SIZE[type_]
    return ts * (ne0 // bl)
