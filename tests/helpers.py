"""Shared test plumbing: ctypes handles on the oracle (test infrastructure)
and on the reference leaf build, seeded input generation, ggml block sizes."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_LEAF_SO = os.path.join(ROOT, "oracle", "_ref", "libggml_leaf.so")
REF_LRU_SO = os.path.join(ROOT, "oracle", "_ref", "libggml_lru.so")

P = ctypes.c_void_p
I64 = ctypes.c_int64
F32 = ctypes.c_float

# ggml_type values and block sizes (ggml.h:390-420, ggml-common.h)
GGML_F32, GGML_Q8_0, GGML_Q4_K, GGML_Q8_K, GGML_I32 = 0, 8, 12, 15, 26
Q4K_BYTES, Q8K_BYTES, Q80_BYTES = 144, 292, 34


def ptr(a):
    return a.ctypes.data_as(P)


def ref_available():
    return os.path.exists(REF_LEAF_SO) and os.path.exists(REF_LRU_SO)


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle/liboracle.so missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(ORACLE_SO)
        for name in ["qwo_vec_dot_q4_K_q8_K", "qwo_vec_dot_q8_0_q8_0", "qwo_vec_dot_q6_K_q8_K", "qwo_vec_dot_q5_K_q8_K", "qwo_vec_dot_f32",
                     "qwo_v_expf", "qwo_v_silu", "qwo_fp16_to_fp32"]:
            getattr(lib, name).restype = F32
        lib.qwo_v_expf.argtypes = [F32]
        lib.qwo_v_silu.argtypes = [F32]
        lib.qwo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.qwo_fp32_to_fp16.argtypes = [F32]
        lib.qwo_fp32_to_fp16.restype = ctypes.c_uint16
        lib.qwo_row_bytes.restype = ctypes.c_size_t
        lib.qwo_row_bytes.argtypes = [ctypes.c_int, I64]
        lib.qwo_pool_new.restype = P
        lib.qwo_pool_new.argtypes = [ctypes.c_int, ctypes.c_int, P, ctypes.c_int]
        lib.qwo_pool_free.argtypes = [P]
        lib.qwo_pool_new_sig.restype = P
        lib.qwo_pool_new_sig.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, ctypes.c_int]
        lib.qwo_pool_layer_pool.argtypes = [P, ctypes.c_int, ctypes.c_int]
        lib.qwo_pool_plan_sigs.argtypes = [ctypes.c_int, ctypes.c_int, P, ctypes.c_uint64, ctypes.c_int, P,
                                           ctypes.c_int, P, P]
        lib.qwo_pool_ensure.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, P, P, P, P]
        lib.qwo_pool_stats.argtypes = [P, P]
        lib.qwo_pool_clock.argtypes = [P]
        lib.qwo_pool_clock.restype = ctypes.c_uint64
        lib.qwo_pool_slot_of_row.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
        lib.qwo_pool_slots.argtypes = [P, ctypes.c_int, P, P]
        lib.qwo_pool_resident.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.qwo_pool_touch.argtypes = [P, ctypes.c_int, P, ctypes.c_int]
        lib.qwo_pool_capacity.argtypes = [P, ctypes.c_int]
        lib.qwo_pool_quota_of.argtypes = [P, ctypes.c_int]
        lib.qwo_pool_set_quotas.argtypes = [P, ctypes.c_int]
        lib.qwo_pool_quotas_active.argtypes = [P]
        lib.qwo_pool_plan_slices.argtypes = [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P]
        lib.qwo_pool_save_profile.argtypes = [P, ctypes.c_char_p, ctypes.c_int]
        lib.qwo_pool_rebalance.argtypes = [P, ctypes.c_int, I64, P]
        lib.qwo_pool_clear_counts.argtypes = [P]
        lib.qwo_pool_load_profile.argtypes = [P, ctypes.c_char_p, P]
        lib.qwo_route.argtypes = [I64, I64, I64, P, P, P, ctypes.c_int, ctypes.c_int, F32, P, P, P, P, P]
        lib.qwo_route_ex.argtypes = [I64, I64, I64, P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, F32,
                                     P, P, P, P, P]
        lib.qwo_expf.argtypes = [F32]
        lib.qwo_expf.restype = F32
        lib.qwo_sigmoid.argtypes = [F32]
        lib.qwo_sigmoid.restype = F32
        lib.qwo_mul_mat_id.argtypes = [ctypes.c_int, P, I64, I64, I64, P, I64, I64, P, I64, P]
        lib.qwo_mul_mat.argtypes = [ctypes.c_int, P, I64, I64, P, I64, P]
        lib.qwo_rms_norm.argtypes = [I64, P, F32, P, P]
        lib.qwo_lm_head_argmax.argtypes = [P, I64, I64, P, I64, P, P, P]
        lib.qwo_accept.argtypes = [P, P, ctypes.c_int, P]
        _oracle = lib
    return _oracle


_ref = None


def ref():
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(REF_LEAF_SO)
        for name in ["qwr_vec_dot_q4_K_q8_K", "qwr_vec_dot_q8_0_q8_0", "qwr_vec_dot_q6_K_q8_K", "qwr_vec_dot_q5_K_q8_K", "qwr_vec_dot_f32",
                     "qwr_sum"]:
            getattr(lib, name).restype = F32
        lib.qwr_argmax.restype = ctypes.c_int
        _ref = lib
    return _ref


_lru = None


def ref_lru():
    global _lru
    if _lru is None:
        lib = ctypes.CDLL(REF_LRU_SO)
        lib.qwr_lru_new.restype = P
        lib.qwr_lru_new.argtypes = [ctypes.c_int]
        lib.qwr_lru_free.argtypes = [P]
        lib.qwr_lru_rebuild.argtypes = [P, ctypes.c_int, P, P]
        lib.qwr_lru_occupy_or_touch.argtypes = [P, ctypes.c_int, ctypes.c_uint64]
        lib.qwr_lru_release.argtypes = [P, ctypes.c_int]
        lib.qwr_lru_pick.argtypes = [P, P]
        _lru = lib
    return _lru


# ---------------------------------------------------------------- inputs --

def normal(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def quantize_q4_K(w):
    """Rows of w (f32 [..., K]) -> Q4_K bytes, via the oracle (bit-identical
    to ggml's quantize_row_q4_K_ref)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    K = w.shape[-1]
    rows = w.size // K
    out = np.zeros(rows * (K // 256) * Q4K_BYTES, np.uint8)
    oracle().qwo_quantize_q4_K(ptr(w), ptr(out), I64(rows), I64(K))
    return out


def quantize_q8_0_model(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros(w.size // 32 * Q80_BYTES, np.uint8)
    oracle().qwo_quantize_q8_0_ref(ptr(w), ptr(out), I64(w.size))
    return out


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


Q6K_BYTES = 210
GGML_Q6_K = 14


def random_q6_K(rng, rows, K, d=2e-3):
    """rows x K weights as random Q6_K blocks (ggml-common.h block_q6_K: ql
    [128], qh [64], int8 scales [16], fp16 d): every 6-bit value and every
    int8 scale occurs; d around `d`.  A valid block needs no quantizer."""
    nb = rows * (K // 256)
    b = np.zeros((nb, Q6K_BYTES), np.uint8)
    b[:, :192] = rng.integers(0, 256, (nb, 192), dtype=np.uint8)
    b[:, 192:208] = rng.integers(-128, 128, (nb, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
    b[:, 208:210] = (np.abs(rng.standard_normal(nb)) * d + d / 8).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


Q5K_BYTES = 176
GGML_Q5_K = 13


def random_q5_K(rng, rows, K, d=2e-3):
    """rows x K weights as random Q5_K blocks (ggml-common.h block_q5_K: fp16
    d, fp16 dmin, 12 packed 6-bit scale/min bytes, qh [32], qs [128]): every
    5-bit value, scale and min occurs; d and dmin around `d`."""
    nb = rows * (K // 256)
    b = np.zeros((nb, Q5K_BYTES), np.uint8)
    b[:, 0:2] = (np.abs(rng.standard_normal(nb)) * d + d / 8).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = (np.abs(rng.standard_normal(nb)) * d / 4).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 4:] = rng.integers(0, 256, (nb, Q5K_BYTES - 4), dtype=np.uint8)
    return b.reshape(-1)
