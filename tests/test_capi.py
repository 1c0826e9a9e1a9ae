"""CPU checks of the C ABI: libqwmoe.so loads without a GPU, exports every
function include/qwmoe.h declares, rejects malformed arguments before any
device work, and its slot pool takes the same decisions as the oracle's
restatement of ExpertCache (decision-only pools need no GPU)."""
import ctypes
import os
import re

import numpy as np
import pytest

import questwend_amd as qa
from tests.helpers import ROOT, oracle, ptr


def header_functions():
    src = open(os.path.join(ROOT, "include", "qwmoe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(qwm_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    names = header_functions()
    assert len(names) >= 20
    lib = ctypes.CDLL(qa.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert qa.lib().qwm_version().startswith(b"qwmoe")


def test_tensor_init_matches_python_helper():
    t = qa.QwmTensor()
    qa.lib().qwm_tensor_init(ctypes.byref(t), qa.TYPE_Q4_K, 2048, 768, 128, None)
    u = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 128)
    assert list(t.ne) == list(u.ne) and list(t.nb) == list(u.nb)
    assert t.nb[1] == 1152 and t.nb[2] == 884736


def test_argument_validation_without_gpu():
    L = qa.lib()
    a = qa.tensor(qa.TYPE_Q4_K, 256, 4, 2)
    b = qa.tensor(qa.TYPE_F32, 512, 1, 1)      # K mismatch (ggml.c:3428)
    ids = qa.tensor(qa.TYPE_I32, 2, 1, 1)
    assert L.qwm_mul_mat_id(a, b, ids, qa.tensor(qa.TYPE_F32, 4, 2, 1), None, 0, None) == qa.ERR_ARG
    assert b"ne[0]" in L.qwm_last_error()
    b = qa.tensor(qa.TYPE_F32, 256, 1, 1)
    ids_bad = qa.tensor(qa.TYPE_I32, 3, 2, 1)   # ids->ne[1] != b->ne[2]
    assert L.qwm_mul_mat_id(a, b, ids_bad, None, None, 0, None) == qa.ERR_ARG
    assert L.qwm_mul_mat_id(a, b, ids, qa.tensor(qa.TYPE_F32, 4, 2, 1), None, 0, None) == qa.ERR_WORKSPACE
    wide = qa.tensor(qa.TYPE_F32, 256, 1, 9)    # 9 columns, N 4: not the grouped GEMM's shape (N % 64), so GEMV chunks
    i9 = qa.tensor(qa.TYPE_I32, 2, 9, 1)
    assert L.qwm_mul_mat_id_workspace_size(a, wide, i9) > 0
    assert L.qwm_mul_mat_id(a, wide, i9, None, None, 0, None) == qa.ERR_ARG          # dst NULL
    a64 = qa.tensor(qa.TYPE_Q4_K, 2048, 512, 8)
    b64 = qa.tensor(qa.TYPE_F32, 2048, 1, 64)
    i64 = qa.tensor(qa.TYPE_I32, 4, 64, 1)
    assert L.qwm_mul_mat_id_workspace_size(a64, b64, i64) > 0
    assert L.qwm_mul_mat_id(a64, b64, i64, qa.tensor(qa.TYPE_F32, 512, 4, 64), None, 0, None) == qa.ERR_WORKSPACE
    # other types: GEMV launches over column chunks, whose workspace holds one chunk
    assert 0 < L.qwm_mul_mat_id_workspace_size(qa.tensor(qa.TYPE_Q6_K, 2048, 512, 8), b64, i64) < \
        L.qwm_mul_mat_id_workspace_size(a64, b64, i64)
    # sizes cover either path: the grouped GEMM, or the GEMV chunks that unaligned weights fall back to
    q80 = qa.tensor(qa.TYPE_Q8_0, 2048, 512, 8)
    assert L.qwm_mul_mat_id_workspace_size(q80, b64, i64) >= L.qwm_mul_mat_id_workspace_size(a64, b64, i64) > 0
    i200 = qa.tensor(qa.TYPE_I32, 200, 64, 1)     # more ids per column than the pair table holds
    assert L.qwm_mul_mat_id_workspace_size(qa.tensor(qa.TYPE_Q6_K, 2048, 512, 256), b64, i200) == 0
    # the gate/up/SwiGLU call: up must match gate in type and shape; act is [N, n_ids, T]
    act64 = qa.tensor(qa.TYPE_F32, 512, 4, 64)
    # covers the grouped pass and the split path (gate and up in the workspace) that unaligned weights take
    assert L.qwm_mul_mat_id_swiglu_workspace_size(a64, a64, b64, i64) == \
        2 * 512 * 4 * 64 * 4 + L.qwm_mul_mat_id_workspace_size(a64, b64, i64)
    for up in (qa.tensor(qa.TYPE_Q4_K, 2048, 512, 4), qa.tensor(qa.TYPE_Q8_0, 2048, 512, 8)):
        assert L.qwm_mul_mat_id_swiglu_workspace_size(a64, up, b64, i64) == 0
        assert L.qwm_mul_mat_id_swiglu(a64, up, b64, i64, act64, None, 0, None) == qa.ERR_ARG
    assert L.qwm_mul_mat_id_swiglu(a64, a64, b64, i64, qa.tensor(qa.TYPE_F32, 512, 4, 32), None, 0, None) == qa.ERR_ARG
    assert L.qwm_mul_mat_id_swiglu(a64, a64, b64, i64, act64, None, 0, None) == qa.ERR_WORKSPACE
    b4 = qa.tensor(qa.TYPE_F32, 2048, 1, 4)     # 4 columns: two GEMV calls and the SwiGLU pass, gate/up in the workspace
    i4 = qa.tensor(qa.TYPE_I32, 4, 4, 1)
    assert L.qwm_mul_mat_id_swiglu_workspace_size(a64, a64, b4, i4) == \
        2 * 512 * 4 * 4 * 4 + L.qwm_mul_mat_id_workspace_size(a64, b4, i4)
    lay = qa.MoeLayer()
    lay.router = qa.tensor(qa.TYPE_F32, 2048, 128)
    lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 4)
    lay.up_pool = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 4)
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, 768, 2048, 4)
    lay.n_expert_used = 8
    assert L.qwm_moe_workspace_size(lay, 4) > 0
    assert L.qwm_moe_workspace_size(lay, 9) == 0
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, 512, 2048, 4)   # down K != gate N
    assert L.qwm_moe_workspace_size(lay, 1) == 0
    lm = qa.tensor(qa.TYPE_Q4_K, 2048, 1000)
    assert L.qwm_verify_workspace_size(lm, 4) == 0          # lm_head must be Q8_0
    assert L.qwm_verify_workspace_size(qa.tensor(qa.TYPE_Q8_0, 2048, 151936), 4) > 0


def test_wide_hidden_sizes_without_gpu():
    """Hidden sizes 3072 and 4096 (Qwen3-235B-A22B: 4096, FFN 1536) are taken by
    the MoE layer, MUL_MAT_ID and verify-head entry points; other sizes above
    2048 are refused (workspace size 0)."""
    L = qa.lib()
    for H, ok in ((4096, True), (3072, True), (2304, False), (5120, False)):
        lay = qa.MoeLayer()
        lay.router = qa.tensor(qa.TYPE_F32, H, 128)
        lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, H, 1536, 4)
        lay.up_pool = qa.tensor(qa.TYPE_Q4_K, H, 1536, 4)
        lay.down_pool = qa.tensor(qa.TYPE_Q4_K, 1536, H, 4)
        lay.n_expert_used = 8
        assert (L.qwm_moe_workspace_size(lay, 4) > 0) == ok, H
        b = qa.tensor(qa.TYPE_F32, H, 1, 4)
        ids = qa.tensor(qa.TYPE_I32, 8, 4)
        for t in (qa.TYPE_Q4_K, qa.TYPE_Q5_K, qa.TYPE_Q6_K, qa.TYPE_Q8_0):
            assert (L.qwm_mul_mat_id_workspace_size(qa.tensor(t, H, 1536, 16), b, ids) > 0) == ok, (H, t)
    # prefill-sized batches at K 4096 take the grouped GEMM (Q4_K, Q8_0) or the GEMV chunks (Q6_K): both sized
    b64 = qa.tensor(qa.TYPE_F32, 4096, 1, 64)
    i64 = qa.tensor(qa.TYPE_I32, 8, 64)
    sz = {t: L.qwm_mul_mat_id_workspace_size(qa.tensor(t, 4096, 1536, 128), b64, i64)
          for t in (qa.TYPE_Q4_K, qa.TYPE_Q8_0, qa.TYPE_Q6_K)}
    assert all(v > 0 for v in sz.values()) and sz[qa.TYPE_Q8_0] >= sz[qa.TYPE_Q4_K] > sz[qa.TYPE_Q6_K], sz
    # the verify head takes 3072 and 4096 for up to 4 tokens
    for H in (3072, 4096):
        lm = qa.tensor(qa.TYPE_Q8_0, H, 151936)
        assert L.qwm_verify_workspace_size(lm, 4) > 0 and L.qwm_verify_workspace_size(lm, 5) == 0
    assert L.qwm_verify_workspace_size(qa.tensor(qa.TYPE_Q8_0, 2560, 1000), 1) == 0
    # the fused verify step stays at hidden size 2048 (it returns 0, the per-op path serves 4096)
    lay = qa.MoeLayer()
    lay.router = qa.tensor(qa.TYPE_F32, 4096, 128)
    lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, 4096, 1536, 4)
    lay.up_pool = qa.tensor(qa.TYPE_Q4_K, 4096, 1536, 4)
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, 1536, 4096, 4)
    lay.n_expert_used = 8
    assert L.qwm_verify_step_workspace_size(lay, qa.tensor(qa.TYPE_Q8_0, 4096, 151936), 4) == 0


def test_block_resident_rejects_short_tensors_without_gpu():
    """qwm_moe_block_resident checks out/resid columns and the ids/weights
    outputs' type, shape and stride before any device work (a tensor with
    too few columns would otherwise be written past its end)."""
    L = qa.lib()
    lay = qa.MoeLayer()
    lay.router = qa.tensor(qa.TYPE_F32, 2048, 128, 1, 0x10000)
    lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 4, 0x10000)
    lay.up_pool = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 4, 0x10000)
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, 768, 2048, 4, 0x10000)
    lay.n_expert_used = 8
    T = 4
    fake = 0x20000
    x = qa.tensor(qa.TYPE_F32, 2048, T, 1, fake)
    ids = qa.tensor(qa.TYPE_I32, 8, T, 1, fake)
    w = qa.tensor(qa.TYPE_F32, 8, T, 1, fake)

    def call(out, resid=None, ids_out=None, w_out=None):
        return L.qwm_moe_block_resident(lay, 0, ctypes.c_void_p(fake), 128, x, None, resid, out, ids_out, w_out,
                                        ctypes.c_void_p(fake), 1, None)

    good = qa.tensor(qa.TYPE_F32, 2048, T, 1, fake)
    assert call(good) == qa.ERR_WORKSPACE                    # every argument accepted; the workspace is too small
    assert call(qa.tensor(qa.TYPE_F32, 2048, T - 1, 1, fake)) == qa.ERR_ARG
    assert call(good, resid=qa.tensor(qa.TYPE_F32, 2048, 1, 1, fake)) == qa.ERR_ARG
    assert call(good, ids_out=qa.tensor(qa.TYPE_I32, 8, T - 1, 1, fake)) == qa.ERR_ARG
    assert call(good, ids_out=qa.tensor(qa.TYPE_F32, 8, T, 1, fake)) == qa.ERR_ARG      # wrong type
    assert call(good, w_out=qa.tensor(qa.TYPE_F32, 4, T, 1, fake)) == qa.ERR_ARG
    assert call(good, ids_out=ids, w_out=w) == qa.ERR_WORKSPACE


def test_gating_and_bias_checks_without_gpu():
    L = qa.lib()
    lay = qa.MoeLayer()
    lay.router = qa.tensor(qa.TYPE_F32, 2048, 128, 1, 0x10000)
    lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 4, 0x10000)
    lay.up_pool = qa.tensor(qa.TYPE_Q4_K, 2048, 768, 4, 0x10000)
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, 768, 2048, 4, 0x10000)
    lay.n_expert_used = 8
    for g in (0, 1, 2):
        lay.gating_func = g
        assert L.qwm_moe_workspace_size(lay, 4) > 0
    lay.gating_func = 3                                    # core/model.cpp:754-756 refuses it too
    assert L.qwm_moe_workspace_size(lay, 4) == 0
    lay.gating_func = 2
    lay.exp_probs_b = qa.tensor(qa.TYPE_F32, 128, 1, 1, 0x20000)
    assert L.qwm_moe_workspace_size(lay, 4) > 0
    lay.exp_probs_b = qa.tensor(qa.TYPE_F32, 64, 1, 1, 0x20000)    # not [E]
    assert L.qwm_moe_workspace_size(lay, 4) == 0
    lay.exp_probs_b = qa.tensor(qa.TYPE_I32, 128, 1, 1, 0x20000)
    assert L.qwm_moe_workspace_size(lay, 4) == 0


class GpuPool:
    """Decision-only libqwmoe pool (no host slabs, so no copies, no GPU)."""

    def __init__(self, n_layer, n_expert, slots, protect=0, indexed=0):
        d = qa.PoolDesc()
        d.n_layer, d.n_expert = n_layer, n_expert
        for r in range(3):
            d.n_slots[r] = slots[r]
            d.slab_bytes[r] = 0
        d.protect_active, d.indexed = protect, indexed
        h = ctypes.c_void_p()
        qa.check(qa.lib().qwm_pool_create(ctypes.byref(d), None, ctypes.byref(h)))
        self.h, self.slots = h, slots

    def ensure(self, layer, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((3, ids.size), np.int32)
        rc = qa.lib().qwm_pool_ensure(self.h, layer, ptr(ids), ids.size, ptr(out[0]), ptr(out[1]), ptr(out[2]))
        return rc, out

    def state(self, role):
        k = np.zeros(self.slots[role], np.int32)
        c = np.zeros(self.slots[role], np.uint64)
        qa.check(qa.lib().qwm_pool_slots(self.h, role, ptr(k), ptr(c)))
        return k, c

    def __del__(self):
        if getattr(self, "h", None):
            qa.lib().qwm_pool_destroy(self.h)


class OraclePool:
    def __init__(self, n_layer, n_expert, slots, protect=0):
        s = np.array(slots, np.int32)
        self.h = oracle().qwo_pool_new(n_layer, n_expert, ptr(s), protect)
        self.slots = slots

    def ensure(self, layer, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((3, ids.size), np.int32)
        nf = ctypes.c_int()
        rc = oracle().qwo_pool_ensure(self.h, layer, ptr(ids), ids.size, ptr(out[0]), ptr(out[1]), ptr(out[2]),
                                      None, ctypes.byref(nf))
        return rc, out

    def state(self, role):
        k = np.zeros(self.slots[role], np.int32)
        c = np.zeros(self.slots[role], np.uint64)
        oracle().qwo_pool_slots(self.h, role, ptr(k), ptr(c))
        return k, c

    def __del__(self):
        oracle().qwo_pool_free(self.h)


@pytest.mark.parametrize("indexed", [0, 1])
@pytest.mark.parametrize("protect", [0, 1])
def test_pool_matches_oracle_on_zipf_traces(indexed, protect):
    rng = np.random.default_rng(17 + indexed + 2 * protect)
    n_layer, n_expert, slots = 4, 128, [90, 77, 101]
    g = GpuPool(n_layer, n_expert, slots, protect, indexed)
    o = OraclePool(n_layer, n_expert, slots, protect)
    pop = 1.0 / np.arange(1, n_expert + 1) ** 1.1
    pop /= pop.sum()
    perm = rng.permutation(n_expert)
    for step in range(400):
        layer = int(rng.integers(0, n_layer))
        T = int(rng.integers(1, 5))
        ids = np.concatenate([perm[rng.choice(n_expert, 8, replace=False, p=pop)] for _ in range(T)])
        rg, sg = g.ensure(layer, ids)
        ro, so = o.ensure(layer, ids)
        assert rg == ro
        if rg == 0:
            assert np.array_equal(sg, so)
    for r in range(3):
        kg, cg = g.state(r)
        ko, co = o.state(r)
        assert np.array_equal(kg, ko) and np.array_equal(cg, co)
    st = qa.PoolStats()
    qa.check(qa.lib().qwm_pool_get_stats(g.h, ctypes.byref(st)))
    hmo = np.zeros(3, np.uint64)
    oracle().qwo_pool_stats(o.h, ptr(hmo))
    assert (st.hits, st.misses, st.evictions) == tuple(int(v) for v in hmo)
    row_g = np.zeros(n_expert, np.int32)
    row_o = np.zeros(n_expert, np.int32)
    for r in range(3):
        for layer in range(n_layer):
            qa.check(qa.lib().qwm_pool_slot_of_row(g.h, r, layer, ptr(row_g)))
            oracle().qwo_pool_slot_of_row(o.h, r, layer, ptr(row_o))
            assert np.array_equal(row_g, row_o)


@pytest.mark.parametrize("indexed", [0, 1])
def test_pool_touch_and_residency_match_oracle(indexed):
    """The fast path's bookkeeping (runtime.cpp:6155-6176): residency bitmaps
    equal ExpertCache::resident for all three roles, and touches of the
    selected experts (GATE, UP, DOWN per expert, non-resident ones left
    alone) leave the pool in the oracle's state, interleaved with ensure
    calls on a Zipf trace."""
    rng = np.random.default_rng(31 + indexed)
    n_layer, n_expert, slots = 3, 96, [40, 33, 47]
    g = GpuPool(n_layer, n_expert, slots, 0, indexed)
    o = OraclePool(n_layer, n_expert, slots, 0)
    pop = 1.0 / np.arange(1, n_expert + 1) ** 1.1
    pop /= pop.sum()
    words = (n_expert + 31) // 32
    for step in range(300):
        layer = int(rng.integers(0, n_layer))
        ids = rng.choice(n_expert, 8, replace=False, p=pop).astype(np.int32)
        if step % 3:
            rg, _ = g.ensure(layer, ids)
            ro, _ = o.ensure(layer, ids)
            assert rg == ro == 0
        else:
            qa.check(qa.lib().qwm_pool_touch(g.h, layer, ptr(ids), ids.size))
            oracle().qwo_pool_touch(o.h, layer, ptr(ids), ids.size)
        bits = np.zeros(words, np.uint32)
        qa.check(qa.lib().qwm_pool_resident_bits(g.h, layer, ptr(bits)))
        want = [all(oracle().qwo_pool_resident(o.h, r, layer, e) for r in range(3)) for e in range(n_expert)]
        got = [bool((bits[e >> 5] >> (e & 31)) & 1) for e in range(n_expert)]
        assert got == want
    for r in range(3):
        kg, cg = g.state(r)
        ko, co = o.state(r)
        assert np.array_equal(kg, ko) and np.array_equal(cg, co)
    st = qa.PoolStats()
    qa.check(qa.lib().qwm_pool_get_stats(g.h, ctypes.byref(st)))
    hmo = np.zeros(3, np.uint64)
    oracle().qwo_pool_stats(o.h, ptr(hmo))
    assert (st.hits, st.misses, st.evictions) == tuple(int(v) for v in hmo)


def test_pool_touch_known_answer():
    """One layer, 4 experts, 2 slots per role: ensure [0, 1], then touch
    [1, 3]: expert 1 gets clock + 1 (gate), + 2 (up), + 3 (down); expert 3 is
    not resident and is left alone."""
    g = GpuPool(1, 4, [2, 2, 2])
    rc, _ = g.ensure(0, np.array([0, 1], np.int32))
    assert rc == 0
    st = qa.PoolStats()
    qa.check(qa.lib().qwm_pool_get_stats(g.h, ctypes.byref(st)))
    c0, h0 = st.clock, st.hits
    ids = np.array([1, 3], np.int32)
    qa.check(qa.lib().qwm_pool_touch(g.h, 0, ptr(ids), 2))
    for r in range(3):
        keys, clk = g.state(r)
        assert clk[list(keys).index(1)] == c0 + 1 + r
    qa.check(qa.lib().qwm_pool_get_stats(g.h, ctypes.byref(st)))
    assert st.clock == c0 + 3 and st.hits == h0 + 3
    bits = np.zeros(1, np.uint32)
    qa.check(qa.lib().qwm_pool_resident_bits(g.h, 0, ptr(bits)))
    assert bits[0] == 0b0011
    assert qa.lib().qwm_pool_touch(g.h, 0, ptr(np.array([4], np.int32)), 1) == qa.ERR_ARG


def plan(h, layer, sel, T, n_used, max_slice, oracle_side=False):
    sel = np.ascontiguousarray(sel, np.int32)
    slices = np.zeros(2 * T, np.int32)
    uni = ctypes.c_int32()
    if oracle_side:
        ns = oracle().qwo_pool_plan_slices(h, layer, ptr(sel), T, n_used, max_slice, ptr(slices), ctypes.byref(uni))
    else:
        n = ctypes.c_int32()
        qa.check(qa.lib().qwm_pool_plan_slices(h, layer, ptr(sel), T, n_used, max_slice, ptr(slices),
                                               ctypes.byref(n), ctypes.byref(uni)))
        ns = n.value
    return [tuple(slices[2 * i:2 * i + 2]) for i in range(ns)], uni.value


def test_plan_slices_known_answer():
    """plan_slices (runtime.cpp:4639-4687), by hand: 12 slots per role, no
    quotas: cap = max(2, 12 - 8) = 4 distinct experts per slice; the batch
    union (5) exceeds quota_of - 8 = 4, so quotas end off."""
    g = GpuPool(1, 16, [12, 12, 12])
    sel = [0, 1,  2, 3,  0, 4,  4, 5]
    got, uni = plan(g.h, 0, sel, 4, 2, 0)
    assert got == [(0, 2), (2, 2)] and uni == 6
    assert qa.lib().qwm_pool_quotas_active(g.h) == 0
    assert qa.lib().qwm_pool_capacity(g.h, 0) == 12 and qa.lib().qwm_pool_quota_of(g.h, 0) == 12
    got, _ = plan(g.h, 0, sel, 4, 2, 1)                 # max_slice 1: one token per slice
    assert got == [(0, 1), (1, 1), (2, 1), (3, 1)]
    got, _ = plan(g.h, 0, [0, 1, 0, 1, 1, 0], 3, 2, 0)   # union 2 <= 4: quotas on, one slice
    assert got == [(0, 3)] and qa.lib().qwm_pool_quotas_active(g.h) == 1


@pytest.mark.parametrize("indexed", [0, 1])
def test_plan_slices_match_oracle(indexed):
    """Slices, union and quota mode equal the oracle's over Zipf batches of
    1..300 tokens, before and after a quota rebalance (which makes capacity
    and quota_of per layer), with and without a slice length cap."""
    rng = np.random.default_rng(41 + indexed)
    n_layer, E, k, slots = 3, 64, 4, [40, 36, 44]
    g = GpuPool(n_layer, E, slots, 0, indexed)
    o = OraclePool(n_layer, E, slots, 0)
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    pop /= pop.sum()
    for step in range(120):
        layer = int(rng.integers(0, n_layer))
        T = int(rng.integers(1, 300))
        sel = np.concatenate([rng.choice(E, k, replace=False, p=pop) for _ in range(T)]).astype(np.int32)
        max_slice = int(rng.choice([0, 0, 7, 64]))
        a = plan(g.h, layer, sel, T, k, max_slice)
        b = plan(o.h, layer, sel, T, k, max_slice, oracle_side=True)
        assert a == b, (step, a, b)
        assert qa.lib().qwm_pool_quotas_active(g.h) == oracle().qwo_pool_quotas_active(o.h)
        for l in range(n_layer):
            assert qa.lib().qwm_pool_capacity(g.h, l) == oracle().qwo_pool_capacity(o.h, l)
            assert qa.lib().qwm_pool_quota_of(g.h, l) == oracle().qwo_pool_quota_of(o.h, l)
        for s0, ln in a[0]:                                # each slice's union fits the capacity it was cut for
            assert ln >= 1
        # feed the pools a decode-like step, and now and then rebalance
        ids = rng.choice(E, k, replace=False, p=pop).astype(np.int32)
        assert g.ensure(layer, ids)[0] == o.ensure(layer, ids)[0] == 0
        if step == 60:
            q = np.zeros(n_layer, np.int32)
            qa.check(qa.lib().qwm_pool_rebalance(g.h, k, 0, ptr(q), None))
            qo = np.zeros(n_layer, np.int32)
            assert oracle().qwo_pool_rebalance(o.h, k, 0, ptr(qo)) >= 0
            assert np.array_equal(q, qo)


def test_pool_exhaustion_is_reported_and_consistent():
    g = GpuPool(1, 16, [2, 2, 2], protect=1)
    assert g.ensure(0, [0, 1])[0] == 0
    rc, _ = g.ensure(0, [0, 1, 2])
    assert rc == qa.ERR_NO_VICTIM
    assert b"No unprotected GPU cache victim" in qa.lib().qwm_last_error()
    k, _ = g.state(0)
    assert sorted(k.tolist()) == [0, 1]          # nothing was evicted or published
    assert g.ensure(0, [16])[0] == qa.ERR_ARG    # expert id out of range


def test_pool_attach_file_checks_without_gpu(tmp_path):
    """The file tier's set-up errors, on a pool whose device memory is never
    touched: a missing file is an I/O error, a file shorter than offset +
    n_expert * slab_bytes an argument error (both with the path in the
    message), as are a role without a device pool and bad reader settings."""
    L = qa.lib()
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = 2, 8
    for r in range(3):
        d.n_slots[r] = 4
        d.pool_data[r] = 4096 if r < 2 else None        # never dereferenced here
        d.slab_bytes[r] = 1000
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), None, ctypes.byref(h)))
    try:
        missing = str(tmp_path / "none.bin").encode()
        assert L.qwm_pool_attach_file(h, 0, 0, missing, 0) == qa.ERR_IO
        assert missing in L.qwm_last_error()
        short = tmp_path / "short.bin"
        short.write_bytes(b"\0" * (100 + 8 * 1000 - 1))
        assert L.qwm_pool_attach_file(h, 0, 1, str(short).encode(), 100) == qa.ERR_ARG
        assert b"shorter" in L.qwm_last_error()
        short.write_bytes(b"\0" * (100 + 8 * 1000))
        assert L.qwm_pool_attach_file(h, 0, 1, str(short).encode(), 100) == qa.OK
        assert L.qwm_pool_attach_file(h, 1, 1, str(short).encode(), 100) == qa.OK
        assert L.qwm_pool_attach_file(h, 2, 0, str(short).encode(), 0) == qa.ERR_ARG     # no device pool
        assert L.qwm_pool_attach_file(h, 3, 0, str(short).encode(), 0) == qa.ERR_ARG     # no such role
        assert L.qwm_pool_attach_file(h, 0, 2, str(short).encode(), 0) == qa.ERR_ARG     # no such layer
        assert L.qwm_pool_set_io(h, 0, 0) == qa.ERR_ARG
        assert L.qwm_pool_set_io(h, 65, 0) == qa.ERR_ARG
        assert L.qwm_pool_set_io(h, 4, -1) == qa.ERR_ARG
        assert L.qwm_pool_set_io(h, 4, 3) == qa.OK
    finally:
        L.qwm_pool_destroy(h)


def oracle_profile_text(o):
    buf = ctypes.create_string_buffer(1 << 20)
    n = oracle().qwo_pool_save_profile(o.h, buf, len(buf))
    assert n >= 0
    return buf.value


def load_profile(g, path):
    n = ctypes.c_int64(-1)
    qa.check(qa.lib().qwm_pool_load_profile(g.h, str(path).encode(), ctypes.byref(n)))
    return n.value


@pytest.mark.parametrize("indexed", [0, 1])
def test_pool_profile_roundtrip_matches_oracle(tmp_path, indexed):
    """save_profile after a Zipf trace writes the oracle's text byte for byte;
    load_prefetch of it into fresh, smaller pools installs the same experts
    into the same slots with the same clocks, counting nothing."""
    rng = np.random.default_rng(23)
    n_layer, n_expert, slots = 3, 64, [40, 33, 47]
    g = GpuPool(n_layer, n_expert, slots, 0, indexed)
    o = OraclePool(n_layer, n_expert, slots)
    pop = 1.0 / np.arange(1, n_expert + 1) ** 1.1
    pop /= pop.sum()
    perm = rng.permutation(n_expert)
    for step in range(150):
        layer = int(rng.integers(0, n_layer))
        ids = np.concatenate([perm[rng.choice(n_expert, 6, replace=False, p=pop)] for _ in range(4)])
        assert g.ensure(layer, ids)[0] == o.ensure(layer, ids)[0] == 0
    path = tmp_path / "cache.profile"
    qa.check(qa.lib().qwm_pool_save_profile(g.h, str(path).encode()))
    text = path.read_bytes()
    assert text == oracle_profile_text(o)
    assert text.startswith(b"QWENEXPCACHE 1\n3 64\n")

    small = [20, 9, 31]
    g2 = GpuPool(n_layer, n_expert, small, 0, indexed)
    o2 = OraclePool(n_layer, n_expert, small)
    n_g = load_profile(g2, path)
    n_o = oracle().qwo_pool_load_profile(o2.h, text, None)
    assert n_g == n_o == sum(small)
    for r in range(3):
        kg, cg = g2.state(r)
        ko, co = o2.state(r)
        assert np.array_equal(kg, ko) and np.array_equal(cg, co)
    st = qa.PoolStats()
    qa.check(qa.lib().qwm_pool_get_stats(g2.h, ctypes.byref(st)))
    assert (st.hits, st.misses, st.evictions) == (0, 0, 0) and st.clock == sum(small)
    # a second load finds every pool full: nothing more is installed
    assert load_profile(g2, path) == 0


def test_pool_profile_known_answer(tmp_path):
    """A hand-made profile, 1 layer x 4 experts, 2 slots per role: per role the
    two largest counts win, the larger into the lower slot; entries out of
    range are ignored; equal counts keep the file's order; the clock runs
    over the installs in count order across roles."""
    path = tmp_path / "p.txt"
    path.write_text("QWENEXPCACHE 1\n1 4\n"
                    "0 0 0 5\n0 0 1 9\n0 0 2 7\n0 0 3 1\n"     # gate: 1 (9), 2 (7)
                    "1 0 3 4\n1 0 0 4\n1 0 1 2\n"              # up: 3 and 0 tie at 4: file order
                    "2 0 2 8\n2 1 0 99\n3 0 0 99\n2 0 9 99\n")  # down: 2 only; the rest out of range
    g = GpuPool(1, 4, [2, 2, 2])
    assert load_profile(g, path) == 5
    # count order: gate 1 (9), down 2 (8), gate 2 (7), up 3 (4), up 0 (4)
    assert [g.state(r)[0].tolist() for r in range(3)] == [[1, 2], [3, 0], [2, -1]]
    assert [g.state(r)[1].tolist() for r in range(3)] == [[1, 3], [4, 5], [2, 0]]
    o = OraclePool(1, 4, [2, 2, 2])
    assert oracle().qwo_pool_load_profile(o.h, path.read_bytes(), None) == 5
    for r in range(3):
        assert np.array_equal(g.state(r)[0], o.state(r)[0]) and np.array_equal(g.state(r)[1], o.state(r)[1])


@pytest.mark.parametrize("text", [None, b"QWENEXPCACHE 2\n1 4\n0 0 1 9\n", b"QWENEXPCACHE 1\n2 4\n0 0 1 9\n",
                                  b"QWENEXPCACHE 1\n1 5\n0 0 1 9\n", b"garbage\n"])
def test_pool_profile_cold_start(tmp_path, text):
    """A missing profile, another version or another pool shape installs
    nothing and is not an error (the reference's cold start)."""
    path = tmp_path / "p.txt"
    if text is not None:
        path.write_bytes(text)
    g = GpuPool(1, 4, [2, 2, 2])
    assert load_profile(g, path) == 0
    assert all((g.state(r)[0] == -1).all() for r in range(3))


def rebalance(g, n_used, budget):
    q = np.zeros(g.n_layer, np.int32)
    n = ctypes.c_int64(-1)
    rc = qa.lib().qwm_pool_rebalance(g.h, n_used, budget, ptr(q), ctypes.byref(n))
    return rc, q, n.value


@pytest.mark.parametrize("indexed,protect", [(0, 0), (1, 0), (1, 1)])
def test_pool_rebalance_matches_oracle(indexed, protect):
    """compute_quota + rebalance after a trace whose layers route with
    different spreads, then more ensure calls under the quotas: quotas,
    filled experts, every call's slots and the final pool state equal the
    oracle's (the indexed mode falls back to the scan once quotas are on)."""
    rng = np.random.default_rng(31 + indexed + 2 * protect)
    n_layer, n_expert, slots, n_used = 4, 64, [60, 50, 70], 6
    g = GpuPool(n_layer, n_expert, slots, protect, indexed)
    g.n_layer = n_layer
    o = OraclePool(n_layer, n_expert, slots, protect)
    pops = []
    for l in range(n_layer):                       # layer l: Zipf skew 0.6 .. 1.5
        p = 1.0 / np.arange(1, n_expert + 1) ** (0.6 + 0.3 * l)
        pops.append((rng.permutation(n_expert), p / p.sum()))

    def trace(steps):
        for _ in range(steps):
            l = int(rng.integers(0, n_layer))
            perm, p = pops[l]
            ids = np.concatenate([perm[rng.choice(n_expert, n_used, replace=False, p=p)] for _ in range(2)])
            rg, sg = g.ensure(l, ids)
            ro, so = o.ensure(l, ids)
            assert rg == ro
            if rg == 0:
                assert np.array_equal(sg, so)

    trace(120)
    rc, qg, ng = rebalance(g, n_used, 1000)
    qo = np.zeros(n_layer, np.int32)
    no = oracle().qwo_pool_rebalance(o.h, n_used, 1000, ptr(qo))
    assert rc == qa.OK and np.array_equal(qg, qo) and ng == no, (qg, qo, ng, no)
    assert qg.sum() <= min(slots) and (qg >= n_used).all()
    for r in range(3):
        assert all(np.array_equal(a, b) for a, b in zip(g.state(r), o.state(r)))
    trace(120)
    for r in range(3):
        assert all(np.array_equal(a, b) for a, b in zip(g.state(r), o.state(r)))


def test_pool_quota_known_answer():
    """2 layers x 4 experts, 5 slots per role, n_used 2.  Counts (summed over
    the roles) 10, 9, 8 for layer 0's experts 0-2 and 7, 1 for layer 1's
    experts 0-1: the floor gives each layer 2 (4 slots), the greedy gives
    layer 0's third entry the last slot: quotas [3, 2].  All five experts are
    already resident, so nothing is filled.  Then a miss of layer 1 (at its
    quota) recycles layer 1's least recently used slot, although the global
    LRU slot belongs to layer 0."""
    g = GpuPool(2, 4, [5, 5, 5])
    g.n_layer = 2
    for e, n in [(0, 10), (1, 9), (2, 8)]:
        for _ in range(n):
            assert g.ensure(0, [e])[0] == 0
    assert g.ensure(1, [1])[0] == 0
    for _ in range(7):
        assert g.ensure(1, [0])[0] == 0
    rc, q, n = rebalance(g, 2, 100)
    assert rc == qa.OK and q.tolist() == [3, 2] and n == 0
    keys_before = g.state(0)[0].copy()
    slot_l1e1 = int(np.nonzero(keys_before == 4 + 1)[0][0])
    rc, slots = g.ensure(1, [2])
    assert rc == 0 and slots[0][0] == slot_l1e1          # layer 1's LRU slot, not layer 0's
    k = g.state(0)[0]
    assert sorted(k.tolist()) == [0, 1, 2, 4, 6]
