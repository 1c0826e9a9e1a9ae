"""Pins the oracle (oracle/qwm_oracle.cpp) bit-for-bit against the reference's
own leaf kernels, compiled from the unmodified ggml sources by oracle/Makefile
(oracle/_ref/libggml_leaf.so).  CPU only."""
import ctypes

import numpy as np
import pytest

from tests.helpers import (I64, Q4K_BYTES, Q8K_BYTES, Q80_BYTES, bits, oracle, ptr, ref)

pytestmark = pytest.mark.ref


def _q4k(fn, x):
    out = np.zeros(x.size // 256 * Q4K_BYTES, np.uint8)
    fn(ptr(x), ptr(out), I64(x.size))
    return out


@pytest.mark.parametrize("scale", [0.02, 1.0, 1e-3, 30.0])
def test_q4_K_quantizer_bytes(scale):
    rng = np.random.default_rng(int(scale * 1000) + 3)
    x = (rng.standard_normal((1500, 256)) * scale).astype(np.float32)
    x[::7] = np.abs(x[::7])          # all-positive blocks (min clamps to 0)
    x[3::11] = 0                     # all-zero blocks
    x[5::13, :100] = 0               # partially zero blocks
    x[9::17, 32:64] = x[9::17, 32:33]  # constant sub-block
    a = np.zeros(1500 * Q4K_BYTES, np.uint8)
    oracle().qwo_quantize_q4_K(ptr(x), ptr(a), I64(1500), I64(256))
    b = _q4k(ref().qwr_quantize_q4_K, x)
    assert np.array_equal(a, b)


def test_q4_K_dequant_matches_reference():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(64 * 256) * 0.02).astype(np.float32)
    q = _q4k(ref().qwr_quantize_q4_K, x)
    ya = np.zeros_like(x)
    yb = np.zeros_like(x)
    oracle().qwo_dequantize_q4_K(ptr(q), ptr(ya), I64(x.size))
    ref().qwr_dequantize_q4_K(ptr(q), ptr(yb), I64(x.size))
    assert np.array_equal(bits(ya), bits(yb))


@pytest.mark.parametrize("scale", [1.0, 1e-4, 300.0])
def test_q8_K_activation_quantizer(scale):
    rng = np.random.default_rng(17)
    x = (rng.standard_normal(128 * 256) * scale).astype(np.float32)
    x[:256] = 0                       # zero block
    x[256:512] = -np.abs(x[256:512])  # negative max
    a = np.zeros(128 * Q8K_BYTES, np.uint8)
    b = np.zeros_like(a)
    c = np.zeros_like(a)
    oracle().qwo_quantize_q8_K(ptr(x), ptr(a), I64(x.size))
    ref().qwr_quantize_q8_K(ptr(x), ptr(b), I64(x.size))
    ref().qwr_quantize_q8_K_ref(ptr(x), ptr(c), I64(x.size))
    assert np.array_equal(a, b) and np.array_equal(b, c)


def test_q8_0_quantizers():
    rng = np.random.default_rng(19)
    x = rng.standard_normal(512 * 32).astype(np.float32)
    x[:32] = 0
    x[32:64] = np.arange(32) - 15.5   # exact .5 ties after scaling
    for ofn, rfn in [(oracle().qwo_quantize_q8_0_x86, ref().qwr_quantize_q8_0),
                     (oracle().qwo_quantize_q8_0_ref, ref().qwr_quantize_q8_0_ref)]:
        a = np.zeros(512 * Q80_BYTES, np.uint8)
        b = np.zeros_like(a)
        ofn(ptr(x), ptr(a), I64(x.size))
        rfn(ptr(x), ptr(b), I64(x.size))
        assert np.array_equal(a, b)


@pytest.mark.parametrize("K", [256, 768, 2048])
def test_vec_dot_q4_K_q8_K_bits(K):
    rng = np.random.default_rng(K)
    w = (rng.standard_normal((200, K)) * 0.02).astype(np.float32)
    q = _q4k(ref().qwr_quantize_q4_K, w)
    x = rng.standard_normal((200, K)).astype(np.float32)
    y = np.zeros(200 * (K // 256) * Q8K_BYTES, np.uint8)
    ref().qwr_quantize_q8_K(ptr(x), ptr(y), I64(x.size))
    rb = K // 256 * Q4K_BYTES
    yb = K // 256 * Q8K_BYTES
    for i in range(200):
        a = oracle().qwo_vec_dot_q4_K_q8_K(K, ptr(q[i * rb:]), ptr(y[i * yb:]))
        b = ref().qwr_vec_dot_q4_K_q8_K(K, ptr(q[i * rb:]), ptr(y[i * yb:]))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


def test_vec_dot_q8_0_q8_0_bits():
    rng = np.random.default_rng(23)
    K = 2048
    w = rng.standard_normal((200, K)).astype(np.float32)
    x = rng.standard_normal((200, K)).astype(np.float32)
    wq = np.zeros(200 * K // 32 * Q80_BYTES, np.uint8)
    xq = np.zeros_like(wq)
    ref().qwr_quantize_q8_0_ref(ptr(w), ptr(wq), I64(w.size))
    ref().qwr_quantize_q8_0(ptr(x), ptr(xq), I64(x.size))
    rb = K // 32 * Q80_BYTES
    for i in range(200):
        a = oracle().qwo_vec_dot_q8_0_q8_0(K, ptr(wq[i * rb:]), ptr(xq[i * rb:]))
        b = ref().qwr_vec_dot_q8_0_q8_0(K, ptr(wq[i * rb:]), ptr(xq[i * rb:]))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


@pytest.mark.parametrize("n", [1, 7, 8, 10, 16, 23, 64, 100, 777, 2048])
def test_vec_dot_f32_bits(n):
    rng = np.random.default_rng(n)
    for _ in range(100):
        u = rng.standard_normal(n).astype(np.float32)
        v = rng.standard_normal(n).astype(np.float32)
        a = oracle().qwo_vec_dot_f32(n, ptr(u), ptr(v))
        b = ref().qwr_vec_dot_f32(n, ptr(u), ptr(v))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


@pytest.mark.parametrize("E,T", [(128, 2), (128, 4), (512, 3), (512, 8), (100, 5)])
def test_router_logits_bits_every_token_count(E, T):
    """Router mul_mat f32 at T >= 2: ggml-cpu computes vec_dot_f32 per (row,
    column) (ggml-cpu.c:1165-1244; llamafile is compiled out of the
    reference's build and tiled/ takes no f32 weights), so each logit equals
    the reference's own vec_dot_f32 on that row and column, bit for bit."""
    H = 2048
    rng = np.random.default_rng(E * 10 + T)
    Wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    k = 8
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    logits = np.zeros((T, E), np.float32)
    assert oracle().qwo_route(I64(E), I64(H), I64(T), ptr(Wr), ptr(x), None, k, 1, 1.0,
                              ptr(ids), ptr(w), ptr(logits), None, None) == 0
    want = np.array([[ref().qwr_vec_dot_f32(H, ptr(Wr[e]), ptr(x[t])) for e in range(E)] for t in range(T)],
                    np.float32)
    assert np.array_equal(bits(logits), bits(want))


def test_simd_expf_silu_bits():
    rng = np.random.default_rng(29)
    xs = np.concatenate([rng.uniform(-110, 92, 4096), rng.standard_normal(4096) * 4,
                         np.array([0.0, -0.0, 88.7, -103.9, 1e-30, -1e-30] + [0.0] * 10)]).astype(np.float32)
    ea = np.array([oracle().qwo_v_expf(float(v)) for v in xs], np.float32)
    sa = np.array([oracle().qwo_v_silu(float(v)) for v in xs], np.float32)
    eb = np.zeros_like(xs)
    sb = np.zeros_like(xs)
    for i in range(0, xs.size, 16):
        ref().qwr_v_expf16(ptr(xs[i:]), ptr(eb[i:]))
        ref().qwr_v_silu16(ptr(xs[i:]), ptr(sb[i:]))
    assert np.array_equal(bits(ea), bits(eb))
    assert np.array_equal(bits(sa), bits(sb))


@pytest.mark.parametrize("E", [128, 512, 100])
def test_soft_max_row_bits(E):
    rng = np.random.default_rng(E)
    for _ in range(50):
        logits = (rng.standard_normal(E) * 0.9).astype(np.float32)
        pa = np.zeros(E, np.float32)
        pb = np.zeros(E, np.float32)
        oracle().qwo_soft_max_row(E, ptr(logits), ptr(pa))
        ref().qwr_soft_max_row(E, ptr(logits), ptr(pb))
        assert np.array_equal(bits(pa), bits(pb))


@pytest.mark.parametrize("n", [768, 512, 100])
def test_swiglu_bits(n):
    rng = np.random.default_rng(n + 1)
    g = (rng.standard_normal(n) * 3).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    ya = np.zeros(n, np.float32)
    yb = np.zeros(n, np.float32)
    oracle().qwo_swiglu(n, ptr(ya), ptr(g), ptr(u))
    ref().qwr_swiglu(n, ptr(yb), ptr(g), ptr(u))
    assert np.array_equal(bits(ya), bits(yb))


def test_argmax_last_index_on_ties():
    x = np.array([1.0, 3.0, 2.0, 3.0, -1.0, 3.0, 0.5], np.float32)
    assert oracle().qwo_argmax(x.size, ptr(x)) == ref().qwr_argmax(x.size, ptr(x)) == 5
    rng = np.random.default_rng(31)
    for _ in range(50):
        v = rng.integers(-3, 4, 1000).astype(np.float32)
        assert oracle().qwo_argmax(v.size, ptr(v)) == ref().qwr_argmax(v.size, ptr(v))


@pytest.mark.parametrize("K", [256, 768, 2048])
def test_vec_dot_q6_K_q8_K_bits(K):
    """The oracle's Q6_K dot equals the reference's x86 kernel bit for bit,
    over random blocks with every 6-bit value and int8 scale, against Q8_K
    activations from the reference quantizer (including +-127 saturation)."""
    from tests.helpers import Q6K_BYTES, random_q6_K
    rng = np.random.default_rng(K + 6)
    q = random_q6_K(rng, 200, K)
    x = rng.standard_normal((200, K)).astype(np.float32)
    x[::7, ::13] *= 50.0
    y = np.zeros(200 * (K // 256) * Q8K_BYTES, np.uint8)
    ref().qwr_quantize_q8_K(ptr(x), ptr(y), I64(x.size))
    rb, yb = K // 256 * Q6K_BYTES, K // 256 * Q8K_BYTES
    for i in range(200):
        a = oracle().qwo_vec_dot_q6_K_q8_K(K, ptr(q[i * rb:]), ptr(y[i * yb:]))
        b = ref().qwr_vec_dot_q6_K_q8_K(K, ptr(q[i * rb:]), ptr(y[i * yb:]))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), i


def test_q6_K_dequant_matches_reference_and_dot():
    """dequantize_row_q6_K equals the reference's; the oracle's dot equals the
    float64 dot of the dequantized row with the dequantized Q8_K row to fp32
    rounding (a closed form independent of the lane order)."""
    from tests.helpers import Q6K_BYTES, random_q6_K
    rng = np.random.default_rng(66)
    K = 1024
    q = random_q6_K(rng, 50, K)
    a = np.zeros(50 * K, np.float32)
    b = np.zeros_like(a)
    oracle().qwo_dequantize_q6_K(ptr(q), ptr(a), I64(a.size))
    ref().qwr_dequantize_q6_K(ptr(q), ptr(b), I64(b.size))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    x = rng.standard_normal((50, K)).astype(np.float32)
    y = np.zeros(50 * (K // 256) * Q8K_BYTES, np.uint8)
    ref().qwr_quantize_q8_K(ptr(x), ptr(y), I64(x.size))
    yb = y.reshape(50, K // 256, Q8K_BYTES)
    yd = yb[:, :, :4].copy().view(np.float32)[:, :, 0]
    yq = yb[:, :, 4:260].view(np.int8).astype(np.float64) * yd[:, :, None]
    for i in range(50):
        exact = float(np.dot(a[i * K:(i + 1) * K].astype(np.float64), yq[i].reshape(-1)))
        got = oracle().qwo_vec_dot_q6_K_q8_K(K, ptr(q[i * K // 256 * Q6K_BYTES:]), ptr(y[i * (K // 256) * Q8K_BYTES:]))
        assert abs(got - exact) <= 1e-5 * np.abs(a[i * K:(i + 1) * K] * yq[i].reshape(-1)).sum() + 1e-6


@pytest.mark.parametrize("K", [256, 1024, 2048])
def test_vec_dot_q5_K_q8_K_bits(K):
    """The oracle's Q5_K dot (eight lanes plus the fused scalar mins sum)
    equals the reference's x86 kernel bit for bit over random blocks."""
    from tests.helpers import Q5K_BYTES, random_q5_K
    rng = np.random.default_rng(K + 5)
    q = random_q5_K(rng, 200, K)
    x = rng.standard_normal((200, K)).astype(np.float32)
    x[::5, ::11] *= 40.0
    y = np.zeros(200 * (K // 256) * Q8K_BYTES, np.uint8)
    ref().qwr_quantize_q8_K(ptr(x), ptr(y), I64(x.size))
    rb, yb = K // 256 * Q5K_BYTES, K // 256 * Q8K_BYTES
    for i in range(200):
        a = oracle().qwo_vec_dot_q5_K_q8_K(K, ptr(q[i * rb:]), ptr(y[i * yb:]))
        b = ref().qwr_vec_dot_q5_K_q8_K(K, ptr(q[i * rb:]), ptr(y[i * yb:]))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), i
