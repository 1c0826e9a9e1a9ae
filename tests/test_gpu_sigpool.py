"""GPU parity of signature pools (expert_cache.cpp:225-296) on a Q4_K_M-like
layout: three layers whose down tensors are Q6_K (layers 0 and 2) and Q4_K
(layer 1), gate/up Q4_K, pools planned by qwm_pool_plan_sigs at 60% of the
expert bytes -- one gate and one up pool shared by the three layers, one
down pool per down type.  A Zipf trace of qwm_moe_cached_step calls and one
qwm_moe_cached_batch call per layer run through the pools: routed ids and
every output equal the oracle's (bit for bit for the cached step), every
pool's keys and clocks equal the oracle's signature pool, and every occupied
slot of every pool holds its key's slab (misses fetched per (role, layer)
into the pool of that (role, layer), by copies or by the gather kernel)."""
import ctypes

import numpy as np
import pytest

from tests.helpers import bits, oracle, ptr
from tests.moe_case import MoeCase, rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from tests.test_gpu_pool import pinned, workspace, zipf_mask  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()
    return torch.device("cuda:0")


@pytest.mark.parametrize("fetch", [qa.FETCH_MEMCPY, qa.FETCH_GATHER])
def test_sig_pools_q4km_layout(dev, fetch):
    H, N, E, k, T, n_layer, steps = 512, 256, 32, 4, 4, 3, 18
    downs = ["q6_K", "same", "q6_K"]
    cases = [MoeCase(seed=90 + l, H=H, N=N, E=E, k=k, S=E, shared=True, N_sh=N, down=downs[l])
             for l in range(n_layer)]
    L = qa.lib()
    # signatures and pool sizes from the expert tensors' descriptors
    ts = (qa.QwmTensor * (3 * n_layer))()
    for l, c in enumerate(cases):
        for r, (typ, ne0, ne1, arr) in enumerate([(c.qa_type, H, N, c.gate_q), (c.qa_type, H, N, c.up_q),
                                                  (c.down_qa, N, H, c.down_q)]):
            ts[r * n_layer + l] = qa.tensor(typ, ne0, ne1, E, 0)
            assert ts[r * n_layer + l].nb[2] * E == arr.nbytes
    total = sum(ts[i].nb[2] * E for i in range(3 * n_layer))
    sigs = (qa.PoolSig * 8)()
    ns = ctypes.c_int32()
    lp = np.zeros(3 * n_layer, np.int32)
    qa.check(L.qwm_pool_plan_sigs(n_layer, E, ts, int(total * 0.6), k, sigs, 8, ctypes.byref(ns), ptr(lp), None))
    assert ns.value == 4 and lp.tolist() == [0, 0, 0, 1, 1, 1, 2, 3, 2]
    # 57, 57, 38 and 19 slots: every pool holds a 4-token step's 16 experts
    assert [sigs[i].n_slots for i in range(4)] == [57, 57, 38, 19]
    pools = [torch.full((sigs[i].n_slots * sigs[i].slab_bytes,), 0xA5, dtype=torch.uint8, device="cuda")
             for i in range(ns.value)]
    for i in range(ns.value):
        sigs[i].pool_data = pools[i].data_ptr()
    print("pools:", [(sigs[i].role, sigs[i].type, sigs[i].n_slots, sigs[i].slab_bytes) for i in range(ns.value)],
          flush=True)
    host = [[pinned(c.gate_q), pinned(c.up_q), pinned(c.down_q)] for c in cases]
    host_ptrs = [(ctypes.c_void_p * n_layer)(*[host[l][r].data_ptr() for l in range(n_layer)]) for r in range(3)]
    d = qa.PoolSigDesc()
    d.n_layer, d.n_expert, d.n_pools = n_layer, E, ns.value
    d.pools = ctypes.cast(sigs, ctypes.POINTER(qa.PoolSig))
    d.layer_pool = lp.ctypes.data
    for r in range(3):
        d.host_slabs[r] = ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = fetch
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create_sig(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    slots = [sigs[i].n_slots for i in range(ns.value)]
    o = oracle().qwo_pool_new_sig(n_layer, E, ns.value, ptr(np.array(slots, np.int32)),
                                  ptr(np.array([sigs[i].role for i in range(ns.value)], np.int32)), ptr(lp), 0)
    layers = []
    for l, c in enumerate(cases):
        c.upload(torch)
        lay = c.layer
        pg, pu, pd = (int(lp[r * n_layer + l]) for r in range(3))
        lay.gate_pool = qa.tensor(c.qa_type, H, N, slots[pg], pools[pg])
        lay.up_pool = qa.tensor(c.qa_type, H, N, slots[pu], pools[pu])
        lay.down_pool = qa.tensor(c.down_qa, N, H, slots[pd], pools[pd])
        layers.append(lay)
    rng = np.random.default_rng(29 + fetch)
    perms = [rng.permutation(E) for _ in range(n_layer)]
    ws = workspace(max(L.qwm_moe_cached_workspace_size(lay, T) for lay in layers))

    def oracle_ensure(l, flat):
        so = np.zeros((3, flat.size), np.int32)
        nf = ctypes.c_int()
        assert oracle().qwo_pool_ensure(o, l, ptr(flat), flat.size, ptr(so[0]), ptr(so[1]), ptr(so[2]), None,
                                        ctypes.byref(nf)) == 0

    def check_pools():
        for i in range(ns.value):
            S, slab = slots[i], sigs[i].slab_bytes
            kg, cg = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            ko, co = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            qa.check(L.qwm_pool_slots(h, i, ptr(kg), ptr(cg)))
            oracle().qwo_pool_slots(o, i, ptr(ko), ptr(co))
            assert np.array_equal(kg, ko) and np.array_equal(cg, co), f"pool {i}: state differs"
            got = pools[i].cpu().numpy().reshape(S, slab)
            r = sigs[i].role
            for s_, key in enumerate(kg):
                if key >= 0:
                    l, e = divmod(int(key), E)
                    src = host[l][r].numpy().reshape(E, slab)
                    assert np.array_equal(got[s_], src[e]), f"pool {i} slot {s_} (layer {l}, expert {e})"

    try:
        # the cached step, layer by layer
        for step in range(steps):
            l = step % n_layer
            x = rng.standard_normal((T, H)).astype(np.float32)
            mask = zipf_mask(rng, perms[l], k, T)
            ids, w, _, _ = cases[l].route(x, mask)
            dx, drm = torch.from_numpy(x).cuda(), torch.from_numpy(mask).cuda()
            out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
            hids = np.zeros(T * k, np.int32)
            print(f"sig pools fetch={fetch}: cached step {step}, layer {l}", flush=True)
            qa.check(L.qwm_moe_cached_step(layers[l], h, l, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                                           qa.tensor(qa.TYPE_F32, E, T, 1, drm), None,
                                           qa.tensor(qa.TYPE_F32, H, T, 1, out), ptr(hids), ws.data_ptr(), ws.numel(),
                                           None))
            assert np.array_equal(hids.reshape(T, k), ids), f"step {step}: routed ids differ"
            oracle_ensure(l, np.ascontiguousarray(ids.ravel()))
            got = out.cpu().numpy()
            exp = cases[l].block(x, ids, w)
            assert np.array_equal(bits(got), bits(exp)), f"step {step}: rel err {rel_err(got, exp):.3e}"
        check_pools()
        st = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(h, ctypes.byref(st)))
        assert st.evictions > 0
        # one batch per layer through the same pools
        Tb = 24
        for l in range(n_layer):
            x = rng.standard_normal((Tb, H)).astype(np.float32)
            resid = rng.standard_normal((Tb, H)).astype(np.float32)
            mask = zipf_mask(rng, perms[l], k, Tb)
            ids, w, _, _ = cases[l].route(x, mask)
            exp = cases[l].block(x, ids, w) + resid
            flat = np.ascontiguousarray(ids.ravel())
            sl_o = np.zeros(2 * Tb, np.int32)
            nso = oracle().qwo_pool_plan_slices(o, l, ptr(flat), Tb, k, 0, ptr(sl_o), None)
            for i in range(nso):
                t0, ln = sl_o[2 * i], sl_o[2 * i + 1]
                oracle_ensure(l, np.ascontiguousarray(flat[t0 * k:(t0 + ln) * k]))
            dx, dr, drm = (torch.from_numpy(a).cuda() for a in (x, resid, mask))
            out = torch.full((Tb, H), float("nan"), dtype=torch.float32, device="cuda")
            wsb = workspace(L.qwm_moe_cached_batch_workspace_size(layers[l], Tb, 0))
            hids = np.zeros(Tb * k, np.int32)
            hsl = np.zeros(2 * Tb, np.int32)
            nsl = ctypes.c_int32()
            print(f"sig pools fetch={fetch}: batch of {Tb} on layer {l}", flush=True)
            qa.check(L.qwm_moe_cached_batch(layers[l], h, l, qa.tensor(qa.TYPE_F32, H, Tb, 1, dx),
                                            qa.tensor(qa.TYPE_F32, E, Tb, 1, drm),
                                            qa.tensor(qa.TYPE_F32, H, Tb, 1, dr), qa.tensor(qa.TYPE_F32, H, Tb, 1, out),
                                            0, ptr(hids), ptr(hsl), ctypes.byref(nsl), wsb.data_ptr(), wsb.numel(),
                                            None))
            torch.cuda.synchronize()
            assert np.array_equal(hids.reshape(Tb, k), ids)
            assert [tuple(hsl[2 * i:2 * i + 2]) for i in range(nsl.value)] == \
                [tuple(sl_o[2 * i:2 * i + 2]) for i in range(nso)]
            got = out.cpu().numpy()
            err = rel_err(got, exp)
            print(f"  slices {nsl.value}, rel err {err:.3e}", flush=True)
            assert np.isfinite(got).all() and err < 1e-5
            if max(hsl[2 * i + 1] for i in range(nsl.value)) <= 8:
                assert np.array_equal(bits(got), bits(exp))
        check_pools()
    finally:
        L.qwm_pool_destroy(h)
        oracle().qwo_pool_free(o)


def test_cached_step_rejects_a_pool_of_another_layer(dev):
    """The layer's down_pool must be the pool of (down, layer): the Q4_K
    layer's descriptor handed to a Q6_K layer's index is refused before any
    work (its slab stride is not that pool's)."""
    H, N, E, k = 512, 256, 16, 4
    c0 = MoeCase(seed=3, H=H, N=N, E=E, k=k, S=E, down="q6_K")
    c1 = MoeCase(seed=4, H=H, N=N, E=E, k=k, S=E)
    ts = (qa.QwmTensor * 6)()
    for l, c in enumerate([c0, c1]):
        ts[0 + l] = qa.tensor(c.qa_type, H, N, E, 0)
        ts[2 + l] = qa.tensor(c.qa_type, H, N, E, 0)
        ts[4 + l] = qa.tensor(c.down_qa, N, H, E, 0)
    L = qa.lib()
    sigs = (qa.PoolSig * 4)()
    ns = ctypes.c_int32()
    lp = np.zeros(6, np.int32)
    qa.check(L.qwm_pool_plan_sigs(2, E, ts, 1 << 40, k, sigs, 4, ctypes.byref(ns), ptr(lp), None))
    assert ns.value == 4 and lp.tolist() == [0, 0, 1, 1, 2, 3] and [sigs[i].n_slots for i in range(4)] == [32, 32, 16, 16]
    pools = [torch.zeros(sigs[i].n_slots * sigs[i].slab_bytes, dtype=torch.uint8, device="cuda") for i in range(4)]
    for i in range(4):
        sigs[i].pool_data = pools[i].data_ptr()
    d = qa.PoolSigDesc()
    d.n_layer, d.n_expert, d.n_pools = 2, E, 4
    d.pools = ctypes.cast(sigs, ctypes.POINTER(qa.PoolSig))
    d.layer_pool = lp.ctypes.data
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create_sig(ctypes.byref(d), None, ctypes.byref(h)))
    try:
        c1.upload(torch)
        lay = c1.layer
        lay.gate_pool = qa.tensor(c1.qa_type, H, N, sigs[0].n_slots, pools[0])     # shared by both layers: 2E slots
        lay.up_pool = qa.tensor(c1.qa_type, H, N, sigs[1].n_slots, pools[1])
        lay.down_pool = qa.tensor(c1.down_qa, N, H, sigs[3].n_slots, pools[3])
        x = torch.zeros((1, H), dtype=torch.float32, device="cuda")
        out = torch.zeros_like(x)
        ws = workspace(L.qwm_moe_cached_workspace_size(lay, 1))
        xt, ot = qa.tensor(qa.TYPE_F32, H, 1, 1, x), qa.tensor(qa.TYPE_F32, H, 1, 1, out)
        assert L.qwm_moe_cached_step(lay, h, 0, xt, None, None, ot, None, ws.data_ptr(), ws.numel(), None) == qa.ERR_ARG
        assert "down_pool" in L.qwm_last_error().decode()
        qa.check(L.qwm_moe_cached_step(lay, h, 1, xt, None, None, ot, None, ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
    finally:
        L.qwm_pool_destroy(h)
