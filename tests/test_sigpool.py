"""CPU checks of the signature pools (ExpertCache's constructor,
expert_cache.cpp:225-296): signature discovery and sizing by hand, and the
pool's decisions over several pools per role -- a Q4_K_M-like layout whose
down tensors are Q6_K on some layers and Q4_K on the others -- against the
oracle's restatement on traces with ensure, touch, plan_slices, rebalance
and profiles (decision-only pools need no GPU)."""
import ctypes

import numpy as np
import pytest

import questwend_amd as qa
from tests.helpers import oracle, ptr

H, N = 512, 256
Q4K = (qa.TYPE_Q4_K, H, N, (H // 256) * 144 * N)           # gate/up [512, 256]: 73728 bytes per expert
Q4K_DOWN = (qa.TYPE_Q4_K, N, H, (N // 256) * 144 * H)      # down [256, 512] Q4_K: 73728
Q6K_DOWN = (qa.TYPE_Q6_K, N, H, (N // 256) * 210 * H)      # down [256, 512] Q6_K: 107520


def expert_tensors(n_layer, n_expert, q6_layers):
    """The expert tensors per (role, layer), role-major, as qwm_tensor."""
    ts = (qa.QwmTensor * (3 * n_layer))()
    for r in range(3):
        for l in range(n_layer):
            typ, ne0, ne1, slab = Q4K if r < 2 else (Q6K_DOWN if l in q6_layers else Q4K_DOWN)
            t = ts[r * n_layer + l]
            t.type = typ
            t.ne[0], t.ne[1], t.ne[2], t.ne[3] = ne0, ne1, n_expert, 1
            t.nb[2] = slab
    return ts


def plan_sigs(n_layer, n_expert, q6_layers, vram, n_used, max_sigs=8):
    ts = expert_tensors(n_layer, n_expert, q6_layers)
    sigs = (qa.PoolSig * max_sigs)()
    ns = ctypes.c_int32()
    lp = np.zeros(3 * n_layer, np.int32)
    frac = ctypes.c_double()
    rc = qa.lib().qwm_pool_plan_sigs(n_layer, n_expert, ts, vram, n_used, sigs, max_sigs, ctypes.byref(ns), ptr(lp),
                                     ctypes.byref(frac))
    return rc, [sigs[i] for i in range(ns.value)], lp, frac.value


def oracle_plan_sigs(n_layer, n_expert, q6_layers, vram, n_used, max_sigs=8):
    t = np.zeros((3 * n_layer, 4), np.int64)
    for r in range(3):
        for l in range(n_layer):
            typ, ne0, ne1, slab = Q4K if r < 2 else (Q6K_DOWN if l in q6_layers else Q4K_DOWN)
            t[r * n_layer + l] = (typ, ne0, ne1, slab)
    out = np.zeros((max_sigs, 7), np.int64)
    lp = np.zeros(3 * n_layer, np.int32)
    frac = ctypes.c_double()
    ns = oracle().qwo_pool_plan_sigs(n_layer, n_expert, ptr(t), vram, n_used, ptr(out), max_sigs, ptr(lp),
                                     ctypes.byref(frac))
    return ns, out[:max(ns, 0)], lp, frac.value


# 4 layers x 8 experts, down Q6_K on layers 0 and 3: the bytes of every
# expert tensor are 4*8*73728 (gate) + 4*8*73728 (up) + 2*8*107520 (Q6_K
# down) + 2*8*73728 (Q4_K down) = 7,618,560.
TOTAL = 7618560


@pytest.mark.parametrize("vram,slots,frac", [
    (TOTAL // 2, [16, 16, 8, 8], 0.5),            # half of every pool: 32 * 0.5, 16 * 0.5
    (TOTAL // 4, [8, 8, 4, 4], 0.25),
    (TOTAL, [32, 32, 16, 16], 1.0),               # everything fits
    (3 * TOTAL, [32, 32, 16, 16], 1.0),           # frac is cut to 1
    (TOTAL * 3 // 10, [9, 9, 4, 4], 0.3),         # (int)(0.3 * 32) = 9, (int)(0.3 * 16) = 4
])
def test_plan_sigs_known_answer(vram, slots, frac):
    """Signatures in first-seen order over roles then layers: gate Q4_K (4
    layers), up Q4_K (4), down Q6_K (first at layer 0; layers 0 and 3), down
    Q4_K (layers 1 and 2); each pool gets (int)(frac * n_layers * n_expert)
    slots."""
    rc, sigs, lp, f = plan_sigs(4, 8, {0, 3}, vram, 2)
    assert rc == qa.OK
    assert [(s.role, s.type, s.ne0, s.ne1, s.slab_bytes, s.n_layers) for s in sigs] == [
        (0, qa.TYPE_Q4_K, H, N, 73728, 4), (1, qa.TYPE_Q4_K, H, N, 73728, 4),
        (2, qa.TYPE_Q6_K, N, H, 107520, 2), (2, qa.TYPE_Q4_K, N, H, 73728, 2)]
    assert lp.tolist() == [0, 0, 0, 0, 1, 1, 1, 1, 2, 3, 3, 2]
    assert [s.n_slots for s in sigs] == slots
    assert f == pytest.approx(frac, rel=1e-12)
    ns, osig, olp, of = oracle_plan_sigs(4, 8, {0, 3}, vram, 2)
    assert ns == 4 and np.array_equal(olp, lp) and of == f
    assert osig[:, 6].tolist() == slots


def test_plan_sigs_refuses_pools_of_n_used_slots():
    """A pool sized to n_used slots or fewer is refused (the reference
    throws "GPU pool cannot fit transient workspace plus retained
    experts"): at frac 0.25 the down pools get 4 slots, fine for n_used 3,
    refused for n_used 4; at a tiny budget every pool is raised to n_used and
    refused."""
    assert plan_sigs(4, 8, {0, 3}, TOTAL // 4, 3)[0] == qa.OK
    assert plan_sigs(4, 8, {0, 3}, TOTAL // 4, 4)[0] == qa.ERR_ARG
    assert "n_used" in qa.lib().qwm_last_error().decode()
    assert oracle_plan_sigs(4, 8, {0, 3}, TOTAL // 4, 4)[0] == -1
    assert plan_sigs(4, 8, {0, 3}, 1000, 2)[0] == qa.ERR_ARG
    assert plan_sigs(4, 8, {0, 3}, TOTAL, 2, max_sigs=3)[0] == qa.ERR_ARG
    assert oracle_plan_sigs(4, 8, {0, 3}, TOTAL, 2, max_sigs=3)[0] == -2
    assert plan_sigs(4, 8, set(), TOTAL, 2)[1].__len__() == 3          # uniform file: one pool per role


class SigPool:
    """Decision-only signature pool, product side and oracle side."""

    def __init__(self, n_layer, n_expert, pool_slots, pool_role, layer_pool, protect=0, indexed=0):
        n = len(pool_slots)
        self.sig = (qa.PoolSig * n)()
        for i in range(n):
            self.sig[i].role, self.sig[i].n_slots = pool_role[i], pool_slots[i]
        self.lp = np.ascontiguousarray(layer_pool, np.int32)
        d = qa.PoolSigDesc()
        d.n_layer, d.n_expert, d.n_pools = n_layer, n_expert, n
        d.pools = ctypes.cast(self.sig, ctypes.POINTER(qa.PoolSig))
        d.layer_pool = self.lp.ctypes.data
        d.protect_active, d.indexed = protect, indexed
        h = ctypes.c_void_p()
        qa.check(qa.lib().qwm_pool_create_sig(ctypes.byref(d), None, ctypes.byref(h)))
        self.h = h
        self.o = oracle().qwo_pool_new_sig(n_layer, n_expert, n, ptr(np.array(pool_slots, np.int32)),
                                           ptr(np.array(pool_role, np.int32)), ptr(self.lp), protect)
        assert self.o
        self.slots, self.n_layer, self.n_expert = pool_slots, n_layer, n_expert

    def ensure(self, layer, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        g = np.zeros((3, ids.size), np.int32)
        o = np.zeros((3, ids.size), np.int32)
        rg = qa.lib().qwm_pool_ensure(self.h, layer, ptr(ids), ids.size, ptr(g[0]), ptr(g[1]), ptr(g[2]))
        nf = ctypes.c_int()
        ro = oracle().qwo_pool_ensure(self.o, layer, ptr(ids), ids.size, ptr(o[0]), ptr(o[1]), ptr(o[2]), None,
                                      ctypes.byref(nf))
        assert (rg == 0) == (ro == 0)
        if rg == 0:
            assert np.array_equal(g, o)
        return rg, g

    def check_equal(self):
        for i, S in enumerate(self.slots):
            kg, cg = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            ko, co = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            qa.check(qa.lib().qwm_pool_slots(self.h, i, ptr(kg), ptr(cg)))
            oracle().qwo_pool_slots(self.o, i, ptr(ko), ptr(co))
            assert np.array_equal(kg, ko) and np.array_equal(cg, co), f"pool {i}"
        rg, ro = np.zeros(self.n_expert, np.int32), np.zeros(self.n_expert, np.int32)
        for r in range(3):
            for l in range(self.n_layer):
                qa.check(qa.lib().qwm_pool_slot_of_row(self.h, r, l, ptr(rg)))
                oracle().qwo_pool_slot_of_row(self.o, r, l, ptr(ro))
                assert np.array_equal(rg, ro), f"slot_of role {r} layer {l}"
        for l in range(self.n_layer):
            assert qa.lib().qwm_pool_capacity(self.h, l) == oracle().qwo_pool_capacity(self.o, l)
            assert qa.lib().qwm_pool_quota_of(self.h, l) == oracle().qwo_pool_quota_of(self.o, l)
        st = qa.PoolStats()
        qa.check(qa.lib().qwm_pool_get_stats(self.h, ctypes.byref(st)))
        hmo = np.zeros(3, np.uint64)
        oracle().qwo_pool_stats(self.o, ptr(hmo))
        assert (st.hits, st.misses, st.evictions) == tuple(int(v) for v in hmo)
        assert st.clock == oracle().qwo_pool_clock(self.o)

    def close(self):
        qa.lib().qwm_pool_destroy(self.h)
        oracle().qwo_pool_free(self.o)


def test_sig_pool_known_answer():
    """2 layers x 4 experts; gate and up pools of 3 slots shared by both
    layers; down pool A (2 slots) for layer 0, B (2 slots) for layer 1.
    ensure(0, [0, 1]) takes clocks 1..6 (gate, up, down per id), ensure(1,
    [0]) 7..9 (key 4 in gate slot 2, up slot 2, B slot 0).  ensure(0, [2])
    evicts key 0 from gate slot 0 (clock 1), up slot 0 (clock 2) and A slot
    0 (clock 3) -- B, another pool, keeps layer 1's expert in slot 0 and its
    free slot 1."""
    p = SigPool(2, 4, [3, 3, 2, 2], [0, 1, 2, 2], [0, 0, 1, 1, 2, 3])
    try:
        assert p.ensure(0, [0, 1])[0] == 0
        rc, s = p.ensure(1, [0])
        assert rc == 0 and s[:, 0].tolist() == [2, 2, 0]
        rc, s = p.ensure(0, [2])
        assert rc == 0 and s[:, 0].tolist() == [0, 0, 0]
        keys = []
        for i, S in enumerate([3, 3, 2, 2]):
            k, c = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            qa.check(qa.lib().qwm_pool_slots(p.h, i, ptr(k), ptr(c)))
            keys.append(k.tolist())
        assert keys == [[2, 1, 4], [2, 1, 4], [2, 1], [4, -1]]
        bits = np.zeros(1, np.uint32)
        qa.check(qa.lib().qwm_pool_resident_bits(p.h, 0, ptr(bits)))
        assert bits[0] == 0b0110
        qa.check(qa.lib().qwm_pool_resident_bits(p.h, 1, ptr(bits)))
        assert bits[0] == 0b0001
        assert [qa.lib().qwm_pool_capacity(p.h, l) for l in range(2)] == [2, 2]
        assert [qa.lib().qwm_pool_layer_pool(p.h, r, l) for r in range(3) for l in range(2)] == [0, 0, 1, 1, 2, 3]
        p.check_equal()
    finally:
        p.close()


def profile_text(p, tmp_path, name):
    path = tmp_path / name
    qa.check(qa.lib().qwm_pool_save_profile(p.h, str(path).encode()))
    buf = ctypes.create_string_buffer(1 << 20)
    n = oracle().qwo_pool_save_profile(p.o, buf, len(buf))
    assert n >= 0
    return path, path.read_bytes(), buf.value


@pytest.mark.parametrize("indexed,protect", [(0, 0), (1, 0), (1, 1)])
def test_sig_pool_matches_oracle_on_traces(tmp_path, indexed, protect):
    """Q4_K_M-like layout, 6 layers x 64 experts, down Q6_K on layers 0, 4
    and 5: signatures and pool sizes from qwm_pool_plan_sigs at 30% of the
    expert bytes, then Zipf traces of ensure calls (2 tokens x 6 experts)
    interleaved with touches and plan_slices, a rebalance, more traces under
    the quotas, a profile save, and the profile loaded into fresh pools:
    every call's slots, every pool's keys and clocks, every (role, layer)'s
    slot_of row, capacity, quota_of, the stats and the profile text equal
    the oracle's."""
    n_layer, E, n_used = 6, 64, 6
    q6 = {0, 4, 5}
    total = 2 * n_layer * E * 73728 + len(q6) * E * 107520 + (n_layer - len(q6)) * E * 73728
    rc, sigs, lp, _ = plan_sigs(n_layer, E, q6, int(total * 0.3), n_used)
    assert rc == qa.OK and len(sigs) == 4
    slots, roles = [s.n_slots for s in sigs], [s.role for s in sigs]
    rng = np.random.default_rng(5 + indexed + 2 * protect)
    pops = []
    for l in range(n_layer):
        pz = 1.0 / np.arange(1, E + 1) ** (0.7 + 0.15 * l)
        pops.append((rng.permutation(E), pz / pz.sum()))
    p = SigPool(n_layer, E, slots, roles, lp, protect, indexed)

    def trace(steps):
        for step in range(steps):
            l = int(rng.integers(0, n_layer))
            perm, pz = pops[l]
            sel = np.stack([perm[rng.choice(E, n_used, replace=False, p=pz)] for _ in range(2)]).astype(np.int32)
            if step % 5 == 4:
                ids = np.ascontiguousarray(sel[0])
                qa.check(qa.lib().qwm_pool_touch(p.h, l, ptr(ids), ids.size))
                oracle().qwo_pool_touch(p.o, l, ptr(ids), ids.size)
                continue
            if step % 7 == 6:
                flat = np.ascontiguousarray(sel.ravel())
                sl_g, sl_o = np.zeros(4, np.int32), np.zeros(4, np.int32)
                ng, ug, uo = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
                qa.check(qa.lib().qwm_pool_plan_slices(p.h, l, ptr(flat), 2, n_used, 0, ptr(sl_g), ctypes.byref(ng),
                                                       ctypes.byref(ug)))
                no = oracle().qwo_pool_plan_slices(p.o, l, ptr(flat), 2, n_used, 0, ptr(sl_o), ctypes.byref(uo))
                assert (ng.value, ug.value) == (no, uo.value) and np.array_equal(sl_g, sl_o)
                assert qa.lib().qwm_pool_quotas_active(p.h) == oracle().qwo_pool_quotas_active(p.o)
            assert p.ensure(l, sel.ravel())[0] == 0

    try:
        trace(300)
        p.check_equal()
        qg, qo = np.zeros(n_layer, np.int32), np.zeros(n_layer, np.int32)
        nfill = ctypes.c_int64()
        qa.check(qa.lib().qwm_pool_rebalance(p.h, n_used, 40, ptr(qg), ctypes.byref(nfill)))
        no = oracle().qwo_pool_rebalance(p.o, n_used, 40, ptr(qo))
        assert np.array_equal(qg, qo) and nfill.value == no
        # a layer's quota fits the smallest of its three pools' shares
        assert (qg >= n_used).all()
        p.check_equal()
        trace(200)
        p.check_equal()
        path, text_g, text_o = profile_text(p, tmp_path, "sig.prof")
        assert text_g == text_o
        q = SigPool(n_layer, E, slots, roles, lp, protect, indexed)
        try:
            ng = ctypes.c_int64()
            qa.check(qa.lib().qwm_pool_load_profile(q.h, str(path).encode(), ctypes.byref(ng)))
            no = oracle().qwo_pool_load_profile(q.o, text_o, None)
            assert ng.value == no > 0
            q.check_equal()
        finally:
            q.close()
    finally:
        p.close()


def test_sig_pool_rebalance_takes_per_pool():
    """compute_quota's take (expert_cache.cpp:529-540) per pool: layer 0's
    down pool has 3 slots, layer 1's 10, the gate and up pools 12 each.
    With n_used 2, counts on layer 0's experts 0-3 and on layer 1's 5 and 6
    only, the floor gives
    each layer 2; the greedy gives layer 0 one more (its down pool then has
    none left) and layer 1 nothing (its first n_used entries are paid for by
    the floor and it has no others): quotas [3, 2]."""
    p = SigPool(2, 8, [12, 12, 3, 10], [0, 1, 2, 2], [0, 0, 1, 1, 2, 3])
    try:
        for e, n in [(0, 9), (1, 8), (2, 7), (3, 6)]:
            for _ in range(n):
                assert p.ensure(0, [e])[0] == 0
        for _ in range(2):
            assert p.ensure(1, [5, 6])[0] == 0
        q = np.zeros(2, np.int32)
        nf = ctypes.c_int64()
        qa.check(qa.lib().qwm_pool_rebalance(p.h, 2, 0, ptr(q), ctypes.byref(nf)))
        qo = np.zeros(2, np.int32)
        oracle().qwo_pool_rebalance(p.o, 2, 0, ptr(qo))
        assert q.tolist() == [3, 2] and qo.tolist() == [3, 2]
        assert qa.lib().qwm_pool_capacity(p.h, 0) == 3 and qa.lib().qwm_pool_capacity(p.h, 1) == 2
        p.check_equal()
    finally:
        p.close()


def test_sig_pool_create_checks():
    """qwm_pool_create_sig refuses routings it cannot serve: fewer than three
    pools, a (role, layer) routed to a pool of another role or out of range,
    a role outside 0..2, a pool without slots."""
    def create(slots, roles, lp, n_layer=2):
        sig = (qa.PoolSig * len(slots))()
        for i in range(len(slots)):
            sig[i].role, sig[i].n_slots = roles[i], slots[i]
        lpa = np.ascontiguousarray(lp, np.int32)
        d = qa.PoolSigDesc()
        d.n_layer, d.n_expert, d.n_pools = n_layer, 4, len(slots)
        d.pools = ctypes.cast(sig, ctypes.POINTER(qa.PoolSig))
        d.layer_pool = lpa.ctypes.data
        h = ctypes.c_void_p()
        rc = qa.lib().qwm_pool_create_sig(ctypes.byref(d), None, ctypes.byref(h))
        if rc == qa.OK:
            qa.lib().qwm_pool_destroy(h)
        return rc

    assert create([3, 3, 2, 2], [0, 1, 2, 2], [0, 0, 1, 1, 2, 3]) == qa.OK
    assert create([3, 3], [0, 1], [0, 0, 1, 1, 1, 1]) == qa.ERR_ARG
    assert create([3, 3, 2, 2], [0, 1, 2, 2], [0, 0, 1, 1, 2, 1]) == qa.ERR_ARG      # down -> up's pool
    assert "another role" in qa.lib().qwm_last_error().decode()
    assert create([3, 3, 2, 2], [0, 1, 2, 2], [0, 0, 1, 1, 2, 4]) == qa.ERR_ARG      # out of range
    assert create([3, 3, 2], [0, 1, 3], [0, 0, 1, 1, 2, 2]) == qa.ERR_ARG
    assert create([3, 0, 2], [0, 1, 2], [0, 0, 1, 1, 2, 2]) == qa.ERR_ARG
    assert not oracle().qwo_pool_new_sig(2, 4, 4, ptr(np.array([3, 3, 2, 2], np.int32)),
                                         ptr(np.array([0, 1, 2, 2], np.int32)),
                                         ptr(np.array([0, 0, 1, 1, 2, 1], np.int32)), 0)
