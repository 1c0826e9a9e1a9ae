"""GPU miss fill through the slot pool: the cached decode loop of the
reference (route on the device, ids read back, ExpertCache::ensure on the
host, misses copied into pool slots from pinned host slabs, then the experts
run on slot ids), checked step by step against the oracle: the routed ids
bit-exact, the slot sequences of every role bit-exact against the oracle
pool, the copied slabs byte-identical to their host sources, and the MoE
block's output within 1e-3 of the oracle block over the full expert table.
Two layers share one pool per role, each token's experts are Zipf(1.1)
draws forced through the route mask, and the pool holds fewer slots than a
layer has experts (but more than one step selects), so misses evict experts
of both layers."""
import ctypes

import numpy as np
import pytest

from tests.gguf_file import GGML_Q4_K, T_STR, write_gguf
from tests.helpers import bits, oracle, ptr
from tests.moe_case import MoeCase, rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402

pytestmark = pytest.mark.gpu
FETCH = {"memcpy": qa.FETCH_MEMCPY, "gather": qa.FETCH_GATHER}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()
    return torch.device("cuda:0")


def workspace(nbytes):
    ws = torch.empty(max(256, (nbytes + 255) // 256 * 256), dtype=torch.uint8, device="cuda")
    qa.check(qa.lib().qwm_workspace_init(ws.data_ptr(), ws.numel(), None))
    return ws


def pinned(a):
    t = torch.empty(a.nbytes, dtype=torch.uint8, pin_memory=True)
    t.numpy()[:] = np.ascontiguousarray(a).view(np.uint8).ravel()
    return t


def zipf_mask(rng, perm, k, T, skew=1.1, bias=16.0):
    """Route mask that makes each token select k experts drawn without
    replacement from Zipf(skew) popularity over the permutation `perm`: +bias
    on the drawn experts' logits (the routing weights stay the softmax of
    their own logits, the bias cancels in the normalization)."""
    E = perm.size
    p = 1.0 / np.arange(1, E + 1) ** skew
    p /= p.sum()
    m = np.zeros((T, E), np.float32)
    for t in range(T):
        m[t, perm[rng.choice(E, k, replace=False, p=p)]] = bias
    return m


def write_slab_file(path, host, head=4133):
    """Every (layer, role) slab array of `host` ([layer][role] tensors) in one
    file behind a `head`-byte header (offsets not aligned to anything), as a
    model file holds its expert tensors; returns offsets [layer][role]."""
    offs, pos = [], head
    with open(path, "wb") as f:
        f.write(b"\x5a" * head)
        for row in host:
            offs.append([])
            for t in row:
                b = t.numpy().tobytes()
                offs[-1].append(pos)
                f.write(b)
                f.write(b"\x00" * 37)
                pos += len(b) + 37
    return offs


@pytest.mark.parametrize("wtype,protect,indexed,fetch", [("q4_K", 0, 0, "memcpy"), ("q4_K", 0, 0, "gather"),
                                                          ("q4_K", 1, 1, "gather"), ("q8_0", 0, 1, "memcpy"),
                                                          ("q8_0", 1, 0, "gather"), ("q4_K", 0, 1, "file"),
                                                          ("q8_0", 1, 0, "file"), ("q4_K", 1, 0, "file_gather")])
def test_pool_miss_fill_decode(dev, tmp_path, wtype, protect, indexed, fetch):
    """Decode steps over two layers sharing a pool smaller than the routed
    experts (Zipf popularity), misses filled from pinned host slabs (per-slab
    copies or one gather launch per call) or from a file through the reader
    threads and a 5-slab staging ring (then per-slab copies, or gather
    launches from the staging): slot sequences equal the oracle's, every
    occupied slot holds its slab byte for byte, and every MoE output matches
    the oracle."""
    H, N, E, k, T, S, n_layer, steps = 512, 256, 64, 4, 4, 20, 2, 24
    cases = [MoeCase(seed=40 + l, H=H, N=N, E=E, k=k, S=E, shared=True, N_sh=N, wtype=wtype) for l in range(n_layer)]
    rng = np.random.default_rng(9)
    perms = [rng.permutation(E) for _ in range(n_layer)]
    L = qa.lib()
    slab = [c.gate_q.nbytes // E for c in cases[:1]][0]
    assert cases[0].down_q.nbytes // E == slab

    # device pools of S slots per role, shared by both layers
    pool_t = [torch.full((S * slab,), 0xA5, dtype=torch.uint8, device="cuda") for _ in range(3)]
    host = [[pinned(c.gate_q), pinned(c.up_q), pinned(c.down_q)] for c in cases]   # [layer][role]
    host_ptrs = [(ctypes.c_void_p * n_layer)(*[host[l][r].data_ptr() for l in range(n_layer)]) for r in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = n_layer, E
    for r in range(3):
        d.n_slots[r] = S
        d.pool_data[r] = pool_t[r].data_ptr()
        d.slab_bytes[r] = slab
        d.host_slabs[r] = None if fetch.startswith("file") else ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.protect_active, d.indexed = protect, indexed
    d.fetch_mode = FETCH[{"file": "memcpy", "file_gather": "gather"}.get(fetch, fetch)]
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    if fetch.startswith("file"):
        path = str(tmp_path / "slabs.bin")
        offs = write_slab_file(path, host)
        for l in range(n_layer):
            for r in range(3):
                qa.check(L.qwm_pool_attach_file(h, r, l, path.encode(), offs[l][r]))
        qa.check(L.qwm_pool_set_io(h, 4, 5))
    o = oracle().qwo_pool_new(n_layer, E, ptr(np.array([S, S, S], np.int32)), protect)

    layers = []
    for c in cases:
        c.upload(torch)
        lay = c.layer
        lay.gate_pool = qa.tensor(c.qa_type, H, N, S, pool_t[0])
        lay.up_pool = qa.tensor(c.qa_type, H, N, S, pool_t[1])
        lay.down_pool = qa.tensor(c.qa_type, N, H, S, pool_t[2])
        layers.append(lay)
    ws = workspace(L.qwm_moe_workspace_size(layers[0], T))
    n_miss = 0
    try:
        for step in range(steps):
            l = step % n_layer
            c, lay = cases[l], layers[l]
            x = rng.standard_normal((T, H)).astype(np.float32)
            mask = zipf_mask(rng, perms[l], k, T)
            ids, w, _, _ = c.route(x, mask)
            dx = torch.from_numpy(x).cuda()
            drm = torch.from_numpy(mask).cuda()
            gids = torch.zeros((T, k), dtype=torch.int32, device="cuda")
            gw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
            xt = qa.tensor(qa.TYPE_F32, H, T, 1, dx)
            qa.check(L.qwm_moe_route(lay, xt, qa.tensor(qa.TYPE_F32, E, T, 1, drm), qa.tensor(qa.TYPE_I32, k, T, 1, gids),
                                     qa.tensor(qa.TYPE_F32, k, T, 1, gw), ws.data_ptr(), ws.numel(), None))
            hids = gids.cpu().numpy()          # the reference's D2H read of the ids (synchronous)
            assert np.array_equal(hids, ids), f"step {step}: routed ids differ"
            assert np.array_equal(bits(gw.cpu().numpy()), bits(w))

            flat = np.ascontiguousarray(hids.ravel())
            sl = np.zeros((3, flat.size), np.int32)
            qa.check(L.qwm_pool_ensure(h, l, ptr(flat), flat.size, ptr(sl[0]), ptr(sl[1]), ptr(sl[2])))
            so = np.zeros((3, flat.size), np.int32)
            nf = ctypes.c_int()
            assert oracle().qwo_pool_ensure(o, l, ptr(flat), flat.size, ptr(so[0]), ptr(so[1]), ptr(so[2]),
                                            None, ctypes.byref(nf)) == 0
            assert np.array_equal(sl, so), f"step {step}: slot sequences differ"

            dsl = torch.from_numpy(sl).cuda()
            qa.check(L.qwm_pool_wait(h, None))
            out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
            st = [qa.tensor(qa.TYPE_I32, k, T, 1, dsl[r]) for r in range(3)]
            qa.check(L.qwm_moe_experts(lay, xt, st[0], st[1], st[2], qa.tensor(qa.TYPE_F32, k, T, 1, gw), None,
                                       qa.tensor(qa.TYPE_F32, H, T, 1, out), ws.data_ptr(), ws.numel(), None))
            exp = c.block(x, ids, w)           # every expert resident: slot = expert id
            got = out.cpu().numpy()
            err = rel_err(got, exp)
            assert np.array_equal(bits(got), bits(exp)), f"step {step}: rel err {err:.3e}"
        torch.cuda.synchronize()

        # every occupied slot holds its key's host slab, byte for byte
        for r in range(3):
            keys = np.zeros(S, np.int32)
            qa.check(L.qwm_pool_slots(h, r, ptr(keys), None))
            dev_bytes = pool_t[r].cpu().numpy().reshape(S, slab)
            for s, key in enumerate(keys):
                if key < 0:
                    continue
                lyr, e = divmod(int(key), E)
                src = host[lyr][r].numpy().reshape(E, slab)[e]
                assert np.array_equal(dev_bytes[s], src), f"role {r} slot {s} key {key}"
        stt = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(h, ctypes.byref(stt)))
        hmo = np.zeros(3, np.uint64)
        oracle().qwo_pool_stats(o, ptr(hmo))
        assert (stt.hits, stt.misses, stt.evictions) == tuple(int(v) for v in hmo)
        assert stt.fetches == stt.misses and stt.fetch_bytes == stt.misses * slab
        n_miss = stt.misses
        print(f"pool {wtype} protect={protect} indexed={indexed} fetch={fetch}: hits {stt.hits} misses {stt.misses} "
              f"evictions {stt.evictions}")
        assert stt.evictions > 0, "the trace should overflow the pool"
    finally:
        L.qwm_pool_destroy(h)
        oracle().qwo_pool_free(o)
    assert n_miss > 0


def test_slab_fetch_async_event(dev):
    """One slab copy on a side stream, ordered by its done event."""
    L = qa.lib()
    slab, S = 589824, 3
    src = pinned(np.random.default_rng(2).integers(0, 256, slab, dtype=np.uint8))
    pool = torch.zeros(S * slab, dtype=torch.uint8, device="cuda")
    copy = torch.cuda.Stream()
    ev = torch.cuda.Event()
    ev.record(copy)                       # creates the event
    qa.check(L.qwm_slab_fetch_async(ctypes.c_void_p(pool.data_ptr()), slab, 2, ctypes.c_void_p(src.data_ptr()),
                                    ctypes.c_void_p(copy.cuda_stream), ctypes.c_void_p(ev.cuda_event)))
    torch.cuda.current_stream().wait_event(ev)
    got = pool.cpu().numpy().reshape(S, slab)
    assert np.array_equal(got[2], src.numpy())
    assert not got[:2].any()


def small_pool(n_slots, slab, host_t, fetch, copy, n_layer=1, n_expert=16):
    pool_t = [torch.zeros(n_slots * slab, dtype=torch.uint8, device="cuda") for _ in range(3)]
    ptrs = [(ctypes.c_void_p * n_layer)(*[host_t[r][l].data_ptr() for l in range(n_layer)]) for r in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = n_layer, n_expert
    for r in range(3):
        d.n_slots[r] = n_slots
        d.pool_data[r] = pool_t[r].data_ptr()
        d.slab_bytes[r] = slab
        d.host_slabs[r] = ctypes.cast(ptrs[r], ctypes.c_void_p)
    d.fetch_mode = FETCH[fetch]
    h = ctypes.c_void_p()
    rc = qa.lib().qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h))
    return rc, h, pool_t, ptrs


@pytest.mark.parametrize("fetch", ["memcpy", "gather"])
def test_pool_refill_within_call(dev, fetch):
    """More distinct experts in one call than slots: a slot installed early in
    the call is evicted and refilled later in the same call, and must end up
    holding the later expert's slab (the copies of one call land in order)."""
    slab, S, E = 4096 + 16 * 37, 6, 16
    rng = np.random.default_rng(5)
    host_t = [[pinned(rng.integers(0, 256, E * slab, dtype=np.uint8))] for _ in range(3)]
    copy = torch.cuda.Stream()
    rc, h, pool_t, _keep = small_pool(S, slab, host_t, fetch, copy, n_expert=E)
    qa.check(rc)
    L = qa.lib()
    try:
        for ids in ([0, 1, 2, 3, 4, 5, 6, 7, 8, 9], [9, 3, 12, 13, 14, 15, 0, 1], [2, 2, 5, 11]):
            ids = np.array(ids, np.int32)
            sl = np.zeros((3, ids.size), np.int32)
            qa.check(L.qwm_pool_ensure(h, 0, ptr(ids), ids.size, ptr(sl[0]), ptr(sl[1]), ptr(sl[2])))
            qa.check(L.qwm_pool_wait(h, None))
            torch.cuda.synchronize()
            for r in range(3):
                keys = np.zeros(S, np.int32)
                qa.check(L.qwm_pool_slots(h, r, ptr(keys), None))
                got = pool_t[r].cpu().numpy().reshape(S, slab)
                src = host_t[r][0].numpy().reshape(E, slab)
                for s_, key in enumerate(keys):
                    assert key >= 0 and np.array_equal(got[s_], src[key]), (fetch, r, s_, key)
    finally:
        L.qwm_pool_destroy(h)


def test_pool_gather_needs_pinned_slabs(dev):
    """GATHER reads host slabs from the GPU: pageable memory is refused at create."""
    slab, S, E = 4096, 4, 16
    pageable = [[torch.zeros(E * slab, dtype=torch.uint8)] for _ in range(3)]
    rc, h, _, _keep = small_pool(S, slab, pageable, "gather", torch.cuda.Stream(), n_expert=E)
    assert rc == qa.ERR_ARG and not h.value
    assert b"pinned" in qa.lib().qwm_last_error()
    rc, h, _, _keep = small_pool(S, slab + 8, [[pinned(np.zeros(E * (slab + 8), np.uint8))] for _ in range(3)],
                                 "gather", torch.cuda.Stream(), n_expert=E)
    assert rc == qa.ERR_ARG and not h.value


@pytest.mark.parametrize("mode", ["memcpy", "gather"])
def test_pool_file_read_failure_unpublishes(dev, tmp_path, mode):
    """A file tier whose file was cut short after attach: the call returns
    QWM_ERR_IO naming the failed slab, the miss that failed and every later
    miss of the call are not resident afterwards (no key points at an unfilled
    slot), the earlier ones are and hold their slabs; once the file is whole
    again the same call fills every slot byte for byte."""
    L = qa.lib()
    E, S, slab = 8, 4, 8192
    rng = np.random.default_rng(5)
    host = [[torch.from_numpy(rng.integers(0, 256, E * slab, dtype=np.uint8)) for _ in range(3)]]
    path = tmp_path / "slabs.bin"
    offs = write_slab_file(str(path), host)
    whole = path.read_bytes()
    pool_t = [torch.zeros(S * slab, dtype=torch.uint8, device="cuda") for _ in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = 1, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
    d.fetch_mode = FETCH[mode]
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    try:
        for r in range(3):
            qa.check(L.qwm_pool_attach_file(h, r, 0, str(path).encode(), offs[0][r]))
        qa.check(L.qwm_pool_set_io(h, 3, 2))
        path.write_bytes(whole[:offs[0][0] + 6 * slab + 100])   # role 0 up to expert 5 only; roles 1, 2 gone
        ids = np.array([1, 5, 2], np.int32)
        out = np.zeros((3, 3), np.int32)
        rc = L.qwm_pool_ensure(h, 0, ptr(ids), 3, ptr(out[0]), ptr(out[1]), ptr(out[2]))
        assert rc == qa.ERR_IO
        assert b"end of file" in L.qwm_last_error()
        qa.check(L.qwm_pool_wait(h, None))
        torch.cuda.synchronize()
        resident = []
        for r in range(3):
            keys = np.zeros(S, np.int32)
            qa.check(L.qwm_pool_slots(h, r, ptr(keys), None))
            resident.append(sorted(int(k) for k in keys if k >= 0))
            row = np.zeros(E, np.int32)
            qa.check(L.qwm_pool_slot_of_row(h, r, 0, ptr(row)))
            assert sorted(int(e) for e in np.nonzero(row)[0]) == [e for e in resident[-1] if row[e] != 0]
        assert resident == [[1], [], []], resident         # misses in order: (1, gate) read, (1, up) failed
        st = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(h, ctypes.byref(st)))
        assert st.fetches == 1 and st.fetch_bytes == slab
        keys = np.zeros(S, np.int32)
        qa.check(L.qwm_pool_slots(h, 0, ptr(keys), None))
        s1 = int(np.nonzero(keys == 1)[0][0])
        assert np.array_equal(pool_t[0].cpu().numpy()[s1 * slab:(s1 + 1) * slab],
                              host[0][0].numpy()[slab:2 * slab])

        path.write_bytes(whole)
        rc = L.qwm_pool_ensure(h, 0, ptr(ids), 3, ptr(out[0]), ptr(out[1]), ptr(out[2]))
        assert rc == qa.OK, L.qwm_last_error()
        qa.check(L.qwm_pool_wait(h, None))
        torch.cuda.synchronize()
        for r in range(3):
            dev_bytes = pool_t[r].cpu().numpy().reshape(S, slab)
            src = host[0][r].numpy().reshape(E, slab)
            for i, e in enumerate(ids):
                assert np.array_equal(dev_bytes[out[r, i]], src[e]), f"role {r} expert {e}"
    finally:
        L.qwm_pool_destroy(h)


@pytest.mark.parametrize("mode", ["memcpy", "gather", "file", "gguf"])
def test_pool_profile_prefetch_fills_slabs(dev, tmp_path, mode):
    """load_prefetch over two layers: the installed slots hold their experts'
    slabs byte for byte once qwm_pool_wait has ordered the copies, whichever
    way the slabs arrive (per-slab copies, gather, file tier, or the file tier
    over the expert tensors of a GGUF model file)."""
    L = qa.lib()
    n_layer, E, S, slab = 2, 8, 3, 4608          # Q4_K [256, 32] per expert
    rng = np.random.default_rng(8)
    host = [[pinned(rng.integers(0, 256, E * slab, dtype=np.uint8)) for _ in range(3)] for _ in range(n_layer)]
    host_ptrs = [(ctypes.c_void_p * n_layer)(*[host[l][r].data_ptr() for l in range(n_layer)]) for r in range(3)]
    pool_t = [torch.zeros(S * slab, dtype=torch.uint8, device="cuda") for _ in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = n_layer, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
        d.host_slabs[r] = None if mode in ("file", "gguf") else ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = FETCH["memcpy" if mode == "memcpy" else "gather"]
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    try:
        if mode == "file":
            path = str(tmp_path / "slabs.bin")
            offs = write_slab_file(path, host)
            for l in range(n_layer):
                for r in range(3):
                    qa.check(L.qwm_pool_attach_file(h, r, l, path.encode(), offs[l][r]))
        if mode == "gguf":
            path = str(tmp_path / "model.gguf")
            ne = {"gate": [256, 32, E], "up": [256, 32, E], "down": [256, 32, E]}
            ts = [(f"blk.{5 + l}.ffn_{role}_exps.weight", GGML_Q4_K, ne[role], host[l][r].numpy().tobytes())
                  for l in range(n_layer) for r, role in enumerate(("gate", "up", "down"))]
            write_gguf(path, [("general.architecture", T_STR, "qwen3moe")], ts, alignment=64)
            qa.check(L.qwm_pool_attach_gguf(h, path.encode(), 5))
        lines = [f"{r} {l} {e} {int(c)}" for r in range(3) for l in range(n_layer) for e in range(E)
                 for c in [rng.integers(1, 1000)]]
        prof = tmp_path / "cache.profile"
        prof.write_text(f"QWENEXPCACHE 1\n{n_layer} {E}\n" + "\n".join(lines) + "\n")
        n = ctypes.c_int64()
        qa.check(L.qwm_pool_load_profile(h, str(prof).encode(), ctypes.byref(n)))
        assert n.value == 3 * S
        qa.check(L.qwm_pool_wait(h, None))
        torch.cuda.synchronize()
        for r in range(3):
            keys = np.zeros(S, np.int32)
            qa.check(L.qwm_pool_slots(h, r, ptr(keys), None))
            dev_bytes = pool_t[r].cpu().numpy().reshape(S, slab)
            for s, key in enumerate(keys):
                lyr, e = divmod(int(key), E)
                assert np.array_equal(dev_bytes[s], host[lyr][r].numpy().reshape(E, slab)[e]), f"role {r} slot {s}"
    finally:
        L.qwm_pool_destroy(h)


@pytest.mark.parametrize("fetch", ["memcpy", "gather"])
def test_moe_cached_step_matches_oracle(dev, fetch):
    """qwm_moe_cached_step (route, ids read back, ensure, slots up, wait,
    experts in one call) over a Zipf trace on two layers sharing a pool that
    overflows: routed ids equal the oracle's, the pool ends in the oracle
    pool's state (keys and clocks), and every output matches the oracle block
    with every expert resident, bit for bit."""
    H, N, E, k, T, S, n_layer, steps = 512, 256, 64, 4, 4, 20, 2, 16
    cases = [MoeCase(seed=70 + l, H=H, N=N, E=E, k=k, S=E, shared=True, N_sh=N) for l in range(n_layer)]
    rng = np.random.default_rng(13)
    perms = [rng.permutation(E) for _ in range(n_layer)]
    L = qa.lib()
    slab = cases[0].gate_q.nbytes // E
    pool_t = [torch.full((S * slab,), 0x5A, dtype=torch.uint8, device="cuda") for _ in range(3)]
    host = [[pinned(c.gate_q), pinned(c.up_q), pinned(c.down_q)] for c in cases]
    host_ptrs = [(ctypes.c_void_p * n_layer)(*[host[l][r].data_ptr() for l in range(n_layer)]) for r in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = n_layer, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
        d.host_slabs[r] = ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = FETCH[fetch]
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    o = oracle().qwo_pool_new(n_layer, E, ptr(np.array([S, S, S], np.int32)), 0)
    layers = []
    for c in cases:
        c.upload(torch)
        lay = c.layer
        lay.gate_pool = qa.tensor(c.qa_type, H, N, S, pool_t[0])
        lay.up_pool = qa.tensor(c.qa_type, H, N, S, pool_t[1])
        lay.down_pool = qa.tensor(c.qa_type, N, H, S, pool_t[2])
        layers.append(lay)
    ws = workspace(L.qwm_moe_cached_workspace_size(layers[0], T))
    try:
        for step in range(steps):
            l = step % n_layer
            x = rng.standard_normal((T, H)).astype(np.float32)
            mask = zipf_mask(rng, perms[l], k, T)
            ids, w, _, _ = cases[l].route(x, mask)
            dx, drm = torch.from_numpy(x).cuda(), torch.from_numpy(mask).cuda()
            out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
            hids = np.zeros(T * k, np.int32)
            qa.check(L.qwm_moe_cached_step(layers[l], h, l, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                                           qa.tensor(qa.TYPE_F32, E, T, 1, drm), None,
                                           qa.tensor(qa.TYPE_F32, H, T, 1, out), ptr(hids), ws.data_ptr(), ws.numel(),
                                           None))
            assert np.array_equal(hids.reshape(T, k), ids), f"step {step}: routed ids differ"
            so = np.zeros((3, T * k), np.int32)
            flat = np.ascontiguousarray(ids.ravel())
            nf = ctypes.c_int()
            assert oracle().qwo_pool_ensure(o, l, ptr(flat), flat.size, ptr(so[0]), ptr(so[1]), ptr(so[2]), None,
                                            ctypes.byref(nf)) == 0
            got = out.cpu().numpy()
            exp = cases[l].block(x, ids, w)
            assert np.array_equal(bits(got), bits(exp)), f"step {step}: rel err {rel_err(got, exp):.3e}"
        for r in range(3):
            kg, cg = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            ko, co = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            qa.check(L.qwm_pool_slots(h, r, ptr(kg), ptr(cg)))
            oracle().qwo_pool_slots(o, r, ptr(ko), ptr(co))
            assert np.array_equal(kg, ko) and np.array_equal(cg, co)
        st = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(h, ctypes.byref(st)))
        assert st.evictions > 0
    finally:
        L.qwm_pool_destroy(h)
        oracle().qwo_pool_free(o)


@pytest.mark.parametrize("mode", ["memcpy", "gather"])
def test_pool_rebalance_fills_slabs(dev, mode):
    """qwm_pool_rebalance's reshape installs fetch their slabs like misses:
    after counts on two layers (ensure calls) and a rebalance that moves the
    pool towards the hotter layer, every occupied slot holds its slab."""
    L = qa.lib()
    n_layer, E, S, slab = 2, 16, 6, 4608
    rng = np.random.default_rng(12)
    host = [[pinned(rng.integers(0, 256, E * slab, dtype=np.uint8)) for _ in range(3)] for _ in range(n_layer)]
    host_ptrs = [(ctypes.c_void_p * n_layer)(*[host[l][r].data_ptr() for l in range(n_layer)]) for r in range(3)]
    pool_t = [torch.zeros(S * slab, dtype=torch.uint8, device="cuda") for _ in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = n_layer, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
        d.host_slabs[r] = ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = FETCH[mode]
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    try:
        out = np.zeros((3, 2), np.int32)
        for step in range(30):                       # layer 1 hot over many experts, layer 0 over two
            l = 1 if step % 3 else 0
            ids = rng.choice(E, 2, replace=False).astype(np.int32) if l else np.array([0, 1], np.int32)
            qa.check(L.qwm_pool_ensure(h, l, ptr(ids), 2, ptr(out[0]), ptr(out[1]), ptr(out[2])))
        q = np.zeros(n_layer, np.int32)
        n = ctypes.c_int64()
        qa.check(L.qwm_pool_rebalance(h, 1, 100, ptr(q), ctypes.byref(n)))
        qa.check(L.qwm_pool_wait(h, None))
        torch.cuda.synchronize()
        assert q.sum() == S and q[1] > q[0]
        for r in range(3):
            keys = np.zeros(S, np.int32)
            qa.check(L.qwm_pool_slots(h, r, ptr(keys), None))
            dev_bytes = pool_t[r].cpu().numpy().reshape(S, slab)
            for s, key in enumerate(keys):
                if key >= 0:
                    lyr, e = divmod(int(key), E)
                    assert np.array_equal(dev_bytes[s], host[lyr][r].numpy().reshape(E, slab)[e]), (r, s, key)
    finally:
        L.qwm_pool_destroy(h)
