"""Pins the oracle against committed vectors of the reference's own CPU kernels
(tests/golden/ref_vectors.npz, written by tests/golden/make_golden.py from the
ggml sources and core/gpu_lru_index.h compiled by oracle/Makefile).  Runs
without the reference build: this is the oracle's pin where the reference
tree is absent."""
import ctypes
import os

import numpy as np
import pytest

from tests.helpers import I64, Q4K_BYTES, Q8K_BYTES, Q80_BYTES, oracle, ptr

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def f32bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_q4_K_quantizer(g):
    x = g["q4k_x"]
    q = np.zeros(x.shape[0] * Q4K_BYTES, np.uint8)
    oracle().qwo_quantize_q4_K(ptr(x), ptr(q), I64(x.shape[0]), I64(256))
    assert np.array_equal(q, g["q4k_q"])


def test_q8_K_quantizer(g):
    x = g["q8k_x"]
    q = np.zeros(x.shape[0] * Q8K_BYTES, np.uint8)
    oracle().qwo_quantize_q8_K(ptr(x), ptr(q), I64(x.size))
    assert np.array_equal(q, g["q8k_q"])


def test_q8_0_quantizers(g):
    x = g["q80_x"]
    for fn, key in [(oracle().qwo_quantize_q8_0_x86, "q80_x86"), (oracle().qwo_quantize_q8_0_ref, "q80_ref")]:
        q = np.zeros(x.shape[0] * Q80_BYTES, np.uint8)
        fn(ptr(x), ptr(q), I64(x.size))
        assert np.array_equal(q, g[key]), key


@pytest.mark.parametrize("K", [768, 2048])
def test_q4_K_q8_K_dot(g, K):
    w, a = g[f"dq4k{K}_w"], g[f"dq4k{K}_a"]
    rb, ab = K // 256 * Q4K_BYTES, K // 256 * Q8K_BYTES
    s = np.array([oracle().qwo_vec_dot_q4_K_q8_K(K, ptr(w[i * rb:]), ptr(a[i * ab:])) for i in range(6)], np.float32)
    assert np.array_equal(f32bits(s), g[f"dq4k{K}_s"])


def test_q8_0_q8_0_dot(g):
    K = 2048
    w, a = g["dq80_w"], g["dq80_a"]
    rb = K // 32 * Q80_BYTES
    s = np.array([oracle().qwo_vec_dot_q8_0_q8_0(K, ptr(w[i * rb:]), ptr(a[i * rb:])) for i in range(4)], np.float32)
    assert np.array_equal(f32bits(s), g["dq80_s"])


def test_vec_dot_f32(g):
    o, s = 0, []
    for n in g["vdf_n"]:
        for _ in range(2):
            u = np.ascontiguousarray(g["vdf_u"][o:o + n])
            v = np.ascontiguousarray(g["vdf_v"][o:o + n])
            s.append(oracle().qwo_vec_dot_f32(int(n), ptr(u), ptr(v)))
            o += n
    assert np.array_equal(f32bits(np.array(s, np.float32)), g["vdf_s"])


def test_simd_expf_silu(g):
    e = np.array([oracle().qwo_v_expf(float(v)) for v in g["exp_x"]], np.float32)
    si = np.array([oracle().qwo_v_silu(float(v)) for v in g["exp_x"]], np.float32)
    assert np.array_equal(f32bits(e), g["exp_y"])
    assert np.array_equal(f32bits(si), g["silu_y"])


@pytest.mark.parametrize("E", [128, 512, 100])
def test_soft_max(g, E):
    x = g[f"sm{E}_x"]
    p = np.zeros_like(x)
    for r in range(x.shape[0]):
        oracle().qwo_soft_max_row(E, ptr(x[r]), ptr(p[r]))
    assert np.array_equal(f32bits(p), g[f"sm{E}_y"])


def test_swiglu(g):
    y = np.zeros(100, np.float32)
    oracle().qwo_swiglu(100, ptr(y), ptr(g["swiglu_g"]), ptr(g["swiglu_u"]))
    assert np.array_equal(f32bits(y), g["swiglu_y"])


def test_argmax_last_index(g):
    got = [oracle().qwo_argmax(8, ptr(np.ascontiguousarray(r))) for r in g["argmax_x"]]
    assert got == g["argmax_i"].tolist()


def test_slot_pool_trace(g):
    n_layer, n_expert = (int(v) for v in g["pool_shape"])
    slots = g["pool_slots"]
    h = oracle().qwo_pool_new(n_layer, n_expert, ptr(slots), 0)
    try:
        o = 0
        for layer, n in zip(g["pool_layers"], g["pool_lens"]):
            ids = np.ascontiguousarray(g["pool_ids"][o:o + n])
            out = np.zeros((3, n), np.int32)
            log = np.zeros(4 * 3 * n, np.int32)
            nf = ctypes.c_int()
            rc = oracle().qwo_pool_ensure(h, int(layer), ptr(ids), int(n), ptr(out[0]), ptr(out[1]), ptr(out[2]),
                                          ptr(log), ctypes.byref(nf))
            assert rc == 0
            assert np.array_equal(out, g["pool_out"][:, o:o + n])
            o += n
    finally:
        oracle().qwo_pool_free(h)
