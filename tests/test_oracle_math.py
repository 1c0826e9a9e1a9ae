"""Pins the parts of the oracle that the reference leaf build does not cover
(routing, mul_mat_id indexing, the MoE block graph, the verify head, the slot
pool) against what the mathematics fixes: fp64 textbook forms, exact integer
block sums, closed-form special cases, invariants, brute force on tiny
inputs, and the reference's own known-answer slot-victim cases.  CPU only."""
import ctypes

import numpy as np
import pytest

from tests.helpers import (GGML_Q4_K, GGML_Q8_0, I64, F32, Q4K_BYTES, Q8K_BYTES, bits, oracle, ptr,
                           quantize_q4_K, quantize_q8_0_model, ref_available, ref_lru)


def dequant_q4k(q, K):
    out = np.zeros(q.size // Q4K_BYTES * 256, np.float32)
    oracle().qwo_dequantize_q4_K(ptr(q), ptr(out), I64(out.size))
    return out.reshape(-1, K).astype(np.float64)


def dequant_q8k(x):
    """f32 rows -> Q8_K -> dequantized fp64 (d * q)."""
    K = x.shape[-1]
    q = np.zeros(x.size // 256 * Q8K_BYTES, np.uint8)
    oracle().qwo_quantize_q8_K(ptr(np.ascontiguousarray(x)), ptr(q), I64(x.size))
    blocks = q.reshape(-1, Q8K_BYTES)
    d = blocks[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
    qs = blocks[:, 4:260].view(np.int8).astype(np.float64)
    bsums = blocks[:, 260:292].copy().view(np.int16)
    assert np.array_equal(bsums, blocks[:, 4:260].view(np.int8).reshape(-1, 16, 16).sum(-1))
    return (qs * d[:, None]).reshape(x.shape[:-1] + (K,))


# ------------------------------------------------------------ formats --

def test_fp16_conversion_matches_ieee():
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(20000) * 0.05, rng.uniform(-6.5e4, 6.5e4, 2000),
                        [6.1e-5, 6.0e-8, 3.0e-8, 1e-9, 65504, 65519, 0.0]]).astype(np.float32)
    got = np.array([oracle().qwo_fp32_to_fp16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, v.astype(np.float16).view(np.uint16))
    h = np.arange(0, 0x7c00, 7, dtype=np.uint16)
    back = np.array([oracle().qwo_fp16_to_fp32(int(x)) for x in h], np.float32)
    assert np.array_equal(back, h.view(np.float16).astype(np.float32))


def test_q8_K_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    deq = dequant_q8k(x)
    amax = np.abs(x).max(-1, keepdims=True)
    assert np.all(np.abs(deq - x) <= amax / 127 * 0.5 + 1e-6)
    # the element of largest magnitude maps to -127 * sign(max) * -1 exactly
    i = np.abs(x).argmax(-1)
    assert np.allclose(deq[np.arange(16), i], x[np.arange(16), i], rtol=1e-6)


def test_q4_K_dequant_error_bound():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((32, 2048)) * 0.02).astype(np.float32)
    deq = dequant_q4k(quantize_q4_K(w), 2048)
    err = np.abs(deq - w).reshape(32, -1, 32).max(-1)
    span = (w.reshape(32, -1, 32).max(-1) - np.minimum(w.reshape(32, -1, 32).min(-1), 0))
    # within one 4-bit step of the sub-block range (the 6-bit scale/min
    # requantization costs up to ~0.3 step on top of the 0.5 step rounding)
    assert np.all(err <= span / 15 * 0.9)
    assert np.sqrt(((deq - w) ** 2).mean()) / w.std() < 0.08


# ---------------------------------------------------------------- dots --

@pytest.mark.parametrize("K", [256, 768, 2048])
def test_q4_K_dot_is_exact_blockwise(K):
    """The oracle's Q4_K x Q8_K dot equals the fp64 dot of the dequantized
    operands up to the fp32 rounding of the per-block accumulation."""
    rng = np.random.default_rng(K + 7)
    w = (rng.standard_normal((64, K)) * 0.02).astype(np.float32)
    q = quantize_q4_K(w)
    x = rng.standard_normal((64, K)).astype(np.float32)
    xq = np.zeros(64 * K // 256 * Q8K_BYTES, np.uint8)
    oracle().qwo_quantize_q8_K(ptr(x), ptr(xq), I64(x.size))
    exact = (dequant_q4k(q, K) * dequant_q8k(x)).sum(-1)
    rb, yb = K // 256 * Q4K_BYTES, K // 256 * Q8K_BYTES
    got = np.array([oracle().qwo_vec_dot_q4_K_q8_K(K, ptr(q[i * rb:]), ptr(xq[i * yb:])) for i in range(64)])
    scale = np.abs(dequant_q4k(q, K)).sum(-1) * np.abs(dequant_q8k(x)).max(-1)
    assert np.all(np.abs(got - exact) <= 1e-6 * scale + 1e-7)


# ------------------------------------------------------------- routing --

def route(Wr, x, k, norm=1, scale=1.0, rm=None):
    E, H = Wr.shape
    T = x.shape[0]
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    lg = np.zeros((T, E), np.float32)
    pr = np.zeros((T, E), np.float32)
    mg = np.zeros(T, np.float32)
    rc = oracle().qwo_route(I64(E), I64(H), I64(T), ptr(Wr), ptr(x),
                            ptr(rm) if rm is not None else None, k, norm, F32(scale),
                            ptr(ids), ptr(w), ptr(lg), ptr(pr), ptr(mg))
    assert rc == 0
    return ids, w, lg, pr, mg


@pytest.mark.parametrize("E,k,T", [(128, 8, 1), (128, 8, 4), (512, 10, 4), (4, 2, 3)])
def test_route_against_fp64(E, k, T):
    rng = np.random.default_rng(E * 10 + T)
    H = 2048 if E > 4 else 256
    Wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, w, lg, pr, mg = route(Wr, x, k)
    l64 = x.astype(np.float64) @ Wr.astype(np.float64).T
    assert np.allclose(lg, l64, rtol=0, atol=1e-5 * np.abs(l64).max())
    p64 = np.exp(l64 - l64.max(-1, keepdims=True))
    p64 /= p64.sum(-1, keepdims=True)
    assert np.allclose(pr, p64, rtol=2e-6, atol=1e-9)
    for t in range(T):
        order = np.argsort(-p64[t], kind="stable")[:k]
        if mg[t] > 1e-5:
            assert list(ids[t]) == list(order)
        assert len(set(ids[t])) == k and ids[t].min() >= 0 and ids[t].max() < E
        assert np.all(np.diff(pr[t][ids[t]]) <= 0)             # descending
        assert abs(w[t].astype(np.float64).sum() - 1.0) < 1e-6  # normalized
        ref_w = p64[t][order] / p64[t][order].sum()
        assert np.allclose(w[t], ref_w, rtol=2e-6)


def route_ex(Wr, x, k, gating, bias=None, rm=None, norm=1):
    E, H = Wr.shape
    T = x.shape[0]
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    pr = np.zeros((T, E), np.float32)
    lg = np.zeros((T, E), np.float32)
    assert oracle().qwo_route_ex(I64(E), I64(H), I64(T), ptr(Wr), ptr(x), ptr(rm) if rm is not None else None,
                                 ptr(bias) if bias is not None else None, gating, k, norm, F32(1.0),
                                 ptr(ids), ptr(w), ptr(lg), ptr(pr), None) == 0
    return ids, w, lg, pr


def test_route_sigmoid_and_bias_known_answer():
    """Sigmoid gating with an exp_probs_b bias, by hand (runtime.cpp:2701-2728):
    the bias reorders the ranking but the weights stay the selected experts'
    own sigmoid probabilities, renormalized.  E = 4, top-2, identity router."""
    Wr = np.eye(4, 256, dtype=np.float32)
    x = np.zeros((1, 256), np.float32)
    x[0, :4] = [2.0, 1.0, 0.0, -1.0]
    bias = np.array([0.0, 0.0, 0.5, 0.0], np.float32)
    ids, w, _, pr = route_ex(Wr, x, 2, gating=2, bias=bias)
    s = 1.0 / (1.0 + np.exp(-np.array([2.0, 1.0, 0.0, -1.0])))
    # ranks: 0.881, 0.731, 0.5 + 0.5 = 1.0, 0.269 -> experts 2 then 0
    assert list(ids[0]) == [2, 0]
    assert np.allclose(pr[0], s, rtol=1e-6)
    assert np.allclose(w[0], np.array([s[2], s[0]]) / (s[2] + s[0]), rtol=1e-6)
    # without the bias: experts 0 then 1
    ids, w, _, _ = route_ex(Wr, x, 2, gating=2)
    assert list(ids[0]) == [0, 1]
    assert np.allclose(w[0], np.array([s[0], s[1]]) / (s[0] + s[1]), rtol=1e-6)
    # the mask is applied again after the bias: a masked expert never wins
    rm = np.zeros((1, 4), np.float32)
    rm[0, 2] = -np.inf
    ids, _, _, _ = route_ex(Wr, x, 2, gating=2, bias=bias, rm=rm)
    assert 2 not in list(ids[0])
    # soft_max gating with the same bias: probabilities e^l / sum, rank + bias
    ids, w, _, pr = route_ex(Wr, x, 2, gating=1, bias=np.array([0.0, 0.0, 0.9, 0.0], np.float32))
    e = np.exp(np.array([2.0, 1.0, 0.0, -1.0]) - 2.0)
    p = e / e.sum()
    assert np.allclose(pr[0], p, rtol=1e-6)
    assert list(ids[0]) == [2, 0]                     # 0.087 + 0.9 > 0.644 > 0.237
    assert np.allclose(w[0], np.array([p[2], p[0]]) / (p[2] + p[0]), rtol=1e-6)


@pytest.mark.parametrize("E,k,T", [(128, 8, 4), (512, 10, 2)])
def test_route_sigmoid_bias_against_fp64(E, k, T):
    rng = np.random.default_rng(E + k)
    H = 2048
    Wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    ids, w, lg, pr = route_ex(Wr, x, k, gating=2, bias=bias)
    l64 = x.astype(np.float64) @ Wr.astype(np.float64).T
    p64 = 1.0 / (1.0 + np.exp(-l64))
    assert np.allclose(pr, p64, rtol=2e-6)
    rank = p64 + bias
    for t in range(T):
        order = np.argsort(-rank[t], kind="stable")
        if rank[t][order[k - 1]] - rank[t][order[k]] > 1e-5:
            assert sorted(ids[t]) == sorted(order[:k])
        assert np.allclose(w[t], p64[t][ids[t]] / p64[t][ids[t]].sum(), rtol=2e-6)


def test_route_mask_scale_and_no_norm():
    rng = np.random.default_rng(4)
    E, H, k = 128, 256, 8
    Wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, H)).astype(np.float32)
    rm = np.zeros((2, E), np.float32)
    rm[:, :64] = -np.inf                       # mask half the experts
    ids, w, _, pr, _ = route(Wr, x, k, norm=0, scale=2.5, rm=rm)
    assert ids.min() >= 64
    assert np.allclose(w, pr[np.arange(2)[:, None], ids] * 2.5)
    assert np.all(pr[:, :64] == 0)


def test_route_tiny_brute_force():
    """E=4, top-2 with hand-made logits: softmax by hand, ties resolved by
    std::sort (recorded: lower index first for this input)."""
    Wr = np.eye(4, 256, dtype=np.float32)
    x = np.zeros((1, 256), np.float32)
    x[0, :4] = [0.5, 2.0, -1.0, 1.0]
    ids, w, _, pr, _ = route(Wr, x, 2)
    e = np.exp(np.array([0.5, 2.0, -1.0, 1.0]) - 2.0)
    assert list(ids[0]) == [1, 3]
    assert np.allclose(pr[0], e / e.sum(), rtol=1e-6)
    assert np.allclose(w[0], np.array([e[1], e[3]]) / (e[1] + e[3]), rtol=1e-6)


# ----------------------------------------------------------- mul_mat_id --

@pytest.mark.parametrize("wtype", [GGML_Q4_K, GGML_Q8_0])
def test_mul_mat_id_indexing(wtype):
    """c[:, e, t] = as[:, :, ids[e,t]] . b[:, e % ne11, t]; checked with fp64
    dequantized operands, including broadcast of b (ne11 = 1) and repeated
    experts.  A transposed or mis-indexed operand fails by orders of magnitude."""
    rng = np.random.default_rng(wtype)
    K, N, S, k, T = 512, 48, 6, 3, 2
    w = (rng.standard_normal((S, N, K)) * 0.02).astype(np.float32)
    if wtype == GGML_Q4_K:
        q = quantize_q4_K(w)
        deq = dequant_q4k(q, K).reshape(S, N, K)
        xq = lambda v: dequant_q8k(v)
    else:
        q = quantize_q8_0_model(w)
        blocks = q.reshape(-1, 34)
        d = blocks[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
        deq = (blocks[:, 2:].view(np.int8).astype(np.float64) * d[:, None]).reshape(S, N, K)
        def xq(v):
            out = np.zeros(v.size // 32 * 34, np.uint8)
            oracle().qwo_quantize_q8_0_x86(ptr(np.ascontiguousarray(v)), ptr(out), I64(v.size))
            bl = out.reshape(-1, 34)
            dd = bl[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
            return (bl[:, 2:].view(np.int8).astype(np.float64) * dd[:, None]).reshape(v.shape)
    ids = np.array([[5, 0, 5], [2, 3, 1]], np.int32)
    for ne11 in [1, k]:
        b = rng.standard_normal((T, ne11, K)).astype(np.float32)
        dst = np.zeros((T, k, N), np.float32)
        assert oracle().qwo_mul_mat_id(wtype, ptr(q), I64(K), I64(N), I64(S), ptr(b), I64(ne11), I64(T),
                                       ptr(ids), I64(k), ptr(dst)) == 0
        bq = xq(b)
        for t in range(T):
            for e in range(k):
                exact = deq[ids[t, e]] @ bq[t, e % ne11]
                assert np.allclose(dst[t, e], exact, rtol=1e-5, atol=1e-5 * np.abs(exact).max())
    bad = ids.copy()
    bad[0, 0] = S
    assert oracle().qwo_mul_mat_id(wtype, ptr(q), I64(K), I64(N), I64(S), ptr(b), I64(ne11), I64(T),
                                   ptr(bad), I64(k), ptr(dst)) == -1


# ------------------------------------------------------------- verify --

def _silu64(v):
    return v / (1.0 + np.exp(-v))


def _block_fp64(case, x, slots, w, plant=None):
    """The MoE block as an fp64 textbook composition of pinned parts: Q4_K
    weights dequantized, Q8_K of x and of the SwiGLU activations (the
    quantizer is pinned against the reference's own), gate and up dots,
    silu(gate) * up, the down dot, the weighted sum over the k experts, and
    the shared expert times sigmoid(g . x).  `plant` swaps in one plausible
    mistake, to show the bound catches it."""
    T, H, N, k = x.shape[0], case.H, case.N, case.k
    gate = dequant_q4k(case.gate_q, H).reshape(case.S, N, H)
    up = dequant_q4k(case.up_q, H).reshape(case.S, N, H)
    down = dequant_q4k(case.down_q, N).reshape(case.S, H, N)
    xq = dequant_q8k(x)
    out = np.zeros((T, H))
    gates = np.zeros((T, k, N))
    ups = np.zeros((T, k, N))
    for t in range(T):
        for j in range(k):
            e = slots[t, j]
            if plant == "slot":
                e = (e + 1) % case.S
            g = gate[e] @ xq[t]
            u = up[e] @ xq[t]
            gates[t, j], ups[t, j] = g, u
            act = _silu64(u) * g if plant == "swap" else _silu64(g) * u
            aq = dequant_q8k(act.astype(np.float32)[None, :])[0]
            wd = down[e].reshape(N, H).T if plant == "transpose" else down[e]   # the slab read as [N][H]
            dn = wd @ aq
            out[t] += (1.0 if plant == "weights" else w[t, j]) * dn
        if case.shared and plant != "no_shared":
            sg = dequant_q4k(case.shg_q, H) @ xq[t]
            su = dequant_q4k(case.shu_q, H) @ xq[t]
            sa = dequant_q8k((_silu64(sg) * su).astype(np.float32)[None, :])[0]
            sh = dequant_q4k(case.shd_q, case.N_sh) @ sa
            z = case.sh_inp.astype(np.float64) @ x[t].astype(np.float64)
            out[t] += sh / (1.0 + np.exp(-z))
    return out, gates, ups


@pytest.mark.parametrize("T,shared", [(1, False), (3, True)])
def test_moe_block_against_fp64(T, shared):
    """The oracle's block graph (qwo_moe_block: gate/up MUL_MAT_ID, SwiGLU, down
    MUL_MAT_ID, the k-weighted combine, the gated shared expert) against the
    fp64 composition above, with the router's ids and weights (pinned by the
    routing tests).  The gap is the oracle's fp32 roundings (~1e-7); a slot off
    by one, gate and up swapped, a transposed down matrix, unweighted experts
    or a dropped shared expert each miss by more than 1e-2."""
    from tests.moe_case import MoeCase, QwoMoeArgs
    case = MoeCase(seed=40 + T, H=512, N=256, E=16, k=4, S=16, shared=shared, N_sh=256)
    x = case.rng.standard_normal((T, case.H)).astype(np.float32)
    ids, w, _, _ = case.route(x)
    slots = ids.astype(np.int32)
    exp64, g64, u64 = _block_fp64(case, x, slots, w)
    got = case.block(x, slots, w).astype(np.float64)
    err = np.linalg.norm(got - exp64) / np.linalg.norm(exp64)
    assert err < 1e-5, err
    # the intermediates the oracle exposes: gate and up rows of every (token, expert)
    gate = np.zeros((T, case.k, case.N), np.float32)
    up = np.zeros_like(gate)
    a = QwoMoeArgs()
    a.H, a.N, a.k, a.T = case.H, case.N, case.k, T
    a.weight_type = case.ggml_type
    a.gate_pool, a.up_pool, a.down_pool = case.gate_q.ctypes.data, case.up_q.ctypes.data, case.down_q.ctypes.data
    a.n_slots = case.S
    a.slot_g = a.slot_u = a.slot_d = slots.ctypes.data
    a.weights = w.ctypes.data
    a.x = x.ctypes.data
    out = np.zeros((T, case.H), np.float32)
    a.out = out.ctypes.data
    a.gate_out, a.up_out = gate.ctypes.data, up.ctypes.data
    assert oracle().qwo_moe_block(ctypes.byref(a)) == 0
    assert np.abs(gate - g64).max() <= 1e-5 * np.abs(g64).max()
    assert np.abs(up - u64).max() <= 1e-5 * np.abs(u64).max()
    for plant in ("slot", "swap", "transpose", "weights") + (("no_shared",) if shared else ()):
        bad, _, _ = _block_fp64(case, x, slots, w, plant)
        assert np.linalg.norm(got - bad) / np.linalg.norm(bad) > 1e-2, plant


def test_rms_norm_and_accept():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    y = np.zeros_like(x)
    oracle().qwo_rms_norm(I64(2048), ptr(x), F32(1e-6), None, ptr(y))
    exp = x / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6)
    assert np.allclose(y, exp, rtol=1e-6)
    xn = ctypes.c_int32()
    for vA, drafts, a in [([5, 6, 7, 8], [5, 6, 7], 3), ([5, 6, 7, 8], [5, 9, 7], 1),
                          ([5, 6, 7, 8], [4, 6, 7], 0), ([1, 2, 3, 4], [1, 2, 9], 2)]:
        va = np.array(vA, np.int32)
        dr = np.array(drafts, np.int32)
        assert oracle().qwo_accept(ptr(va), ptr(dr), 3, ctypes.byref(xn)) == a
        assert xn.value == vA[a]


def test_lm_head_argmax_small():
    rng = np.random.default_rng(10)
    H, V, T = 256, 1000, 3
    W = (rng.standard_normal((V, H)) / np.sqrt(H)).astype(np.float32)
    Wq = quantize_q8_0_model(W)
    h = rng.standard_normal((T, H)).astype(np.float32)
    vA = np.zeros(T, np.int32)
    logits = np.zeros((T, V), np.float32)
    mg = np.zeros(T, np.float32)
    assert oracle().qwo_lm_head_argmax(ptr(Wq), I64(H), I64(V), ptr(h), I64(T), ptr(vA), ptr(logits), ptr(mg)) == 0
    exact = h.astype(np.float64) @ W.astype(np.float64).T
    assert np.allclose(logits, exact, atol=0.05)     # Q8_0 quantization error only
    for t in range(T):
        assert vA[t] == np.flatnonzero(logits[t] == logits[t].max())[-1]


# ----------------------------------------------------------- slot pool --

class Pool:
    def __init__(self, n_layer, n_expert, slots, protect=0):
        s = np.array(slots, np.int32)
        self.h = oracle().qwo_pool_new(n_layer, n_expert, ptr(s), protect)
        self.slots = slots

    def ensure(self, layer, ids):
        ids = np.array(ids, np.int32)
        out = np.zeros((3, ids.size), np.int32)
        log = np.zeros(4 * 3 * max(1, ids.size), np.int32)
        nf = ctypes.c_int()
        rc = oracle().qwo_pool_ensure(self.h, layer, ptr(ids), ids.size, ptr(out[0]), ptr(out[1]), ptr(out[2]),
                                      ptr(log), ctypes.byref(nf))
        return rc, out, log[:4 * nf.value].reshape(-1, 4)

    def slots_of(self, role):
        n = self.slots[role]
        k = np.zeros(n, np.int32)
        c = np.zeros(n, np.uint64)
        oracle().qwo_pool_slots(self.h, role, ptr(k), ptr(c))
        return k, c

    def __del__(self):
        oracle().qwo_pool_free(self.h)


def test_pool_known_answers():
    p = Pool(2, 8, [4, 4, 4])
    rc, out, log = p.ensure(0, [3, 1])
    # cold pool: lowest free slots, gate->up->down per id, clock 1..6
    assert rc == 0 and out.tolist() == [[0, 1], [0, 1], [0, 1]]
    assert log.tolist() == [[0, 0, 3, 0], [1, 0, 3, 0], [2, 0, 3, 0], [0, 0, 1, 1], [1, 0, 1, 1], [2, 0, 1, 1]]
    k, c = p.slots_of(0)
    assert k.tolist() == [3, 1, -1, -1] and c.tolist() == [1, 4, 0, 0]
    rc, out, log = p.ensure(1, [3, 3])       # same expert id, other layer: new key; repeat is a hit
    assert out[:, 0].tolist() == [2, 2, 2] and out[:, 1].tolist() == [2, 2, 2] and len(log) == 3
    rc, out, log = p.ensure(0, [5, 6])       # pool full at slot 3 then LRU: slot 0 (clock 1) is oldest
    assert out[:, 0].tolist() == [3, 3, 3] and out[:, 1].tolist() == [0, 0, 0]
    rc, out, log = p.ensure(0, [1])          # hit
    assert out[:, 0].tolist() == [1, 1, 1] and len(log) == 0


def test_pool_protection_and_exhaustion():
    p = Pool(1, 16, [2, 2, 2], protect=1)
    assert p.ensure(0, [0, 1])[0] == 0
    rc, _, _ = p.ensure(0, [0, 1, 2])        # both slots hold protected ids
    assert rc == -1
    q = Pool(1, 16, [2, 2, 2], protect=0)    # default reference mode: no protection
    assert q.ensure(0, [0, 1])[0] == 0
    rc, out, _ = q.ensure(0, [0, 1, 2])
    assert rc == 0 and out[0].tolist() == [0, 1, 0]   # expert 2 evicts the LRU slot (expert 0)


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_pool_victims_match_reference_lru_index(seed):
    """Randomized Zipf traces: every victim the oracle chooses equals the
    reference GpuLruIndex::pick over the same occupancy and clocks."""
    rng = np.random.default_rng(seed)
    n_layer, n_expert, slots = 3, 64, [40, 37, 45]
    p = Pool(n_layer, n_expert, slots)
    lru = ref_lru()
    idx = [lru.qwr_lru_new(s) for s in slots]
    for r in range(3):
        keys = np.full(slots[r], -1, np.int32)
        clocks = np.zeros(slots[r], np.uint64)
        assert lru.qwr_lru_rebuild(idx[r], slots[r], ptr(keys), ptr(clocks)) == 0
    pop = 1.0 / np.arange(1, n_expert + 1) ** 1.1
    pop /= pop.sum()
    for step in range(300):
        layer = int(rng.integers(0, n_layer))
        T = int(rng.integers(1, 5))
        ids = np.concatenate([rng.choice(n_expert, 8, replace=False, p=pop) for _ in range(T)]).astype(np.int32)
        before = [p.slots_of(r) for r in range(3)]
        rc, out, log = p.ensure(layer, ids)
        assert rc == 0
        # replay decisions on the reference index, role by role in call order
        keys = [before[r][0].copy() for r in range(3)]
        clocks = [before[r][1].copy() for r in range(3)]
        clock = int(max(c.max() for _, c in before))
        fetched = {(int(a), int(b), int(c)): int(d) for a, b, c, d in log}
        for i, e in enumerate(ids):
            key = layer * n_expert + int(e)
            for r in range(3):
                clock += 1
                slot = int(out[r, i])
                if keys[r][slot] != key:
                    victim = lru.qwr_lru_pick(idx[r], None)
                    assert victim == slot
                    if keys[r][slot] >= 0:
                        assert lru.qwr_lru_release(idx[r], slot) == 0
                    keys[r][slot] = key
                assert lru.qwr_lru_occupy_or_touch(idx[r], slot, clock) == 0
                clocks[r][slot] = clock
        for r in range(3):
            k_after, c_after = p.slots_of(r)
            assert np.array_equal(k_after, keys[r]) and np.array_equal(c_after, clocks[r])
    for h in idx:
        lru.qwr_lru_free(h)
