"""GPU parity at the workloads' own shapes, against the oracle:

  * verify step (qwm_verify_step): one Qwen3-30B-A3B-shape block (H 2048, 128
    experts, FFN 768, top-8) with all 128 experts resident, T = 4, followed
    by the Q8_0 lm_head 2048 x 151936, argmax and greedy accept;
  * decode (qwm_moe_decode): 48 stacked blocks of that shape, 1 token, two
    decode steps;
  * miss fill (qwm_moe_cached_step): a Qwen3-Next-shape layer (512 experts
    + shared, FFN 512, top-10) through a 128-slot pool per role, Zipf(1.1)
    popularity, 24 verify steps of 4 tokens, per-slab copies and the gather
    kernel;
  * prefill (qwm_mul_mat_id): 512 columns x top-10 over 512 experts, the
    gate/up shape (K 2048, N 512) and the down shape (K 512, N 2048).

Expert and lm_head weights are drawn on the device (N(0, 0.02), and
N(0, 1/2048) for the lm_head) and quantized by qwm_quantize, whose bytes
equal ggml's quantizers (tests/test_gpu_quant.py); the oracle reads the same
bytes back on the host.  Slot tables are distinct random permutations per
role (and per layer), so a role or layer mix-up cannot pass."""
import ctypes

import numpy as np
import pytest

from tests.helpers import F32, GGML_Q4_K, I64, bits, oracle, ptr
from tests.moe_case import QwoMoeArgs, rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from tests.test_gpu_pool import pinned, zipf_mask  # noqa: E402
from tests.test_gpu_verify import oracle_verify  # noqa: E402

pytestmark = pytest.mark.gpu
H = 2048


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


def gpu_weights(type_, n, seed, scale):
    """n weights N(0, scale^2) drawn on the device, quantized there."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    bs, bl = {qa.TYPE_Q4_K: (144, 256), qa.TYPE_Q8_0: (34, 32)}[type_]
    out = torch.empty(n // bl * bs, dtype=torch.uint8, device="cuda")
    chunk = 1 << 26
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        x = torch.randn(m, generator=g, device="cuda") * scale
        qa.check(qa.lib().qwm_quantize(type_, x.data_ptr(), out.data_ptr() + i // bl * bs, m, None))
    torch.cuda.synchronize()
    return out


class Block:
    """One MoE layer's weights: device tensors and their host bytes."""

    def __init__(self, seed, E, N, k, S, shared=False):
        self.E, self.N, self.k, self.S, self.shared = E, N, k, S, shared
        rng = np.random.default_rng(seed)
        self.router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        self.d_router = torch.from_numpy(self.router).cuda()
        if shared:
            self.d_sh = [gpu_weights(qa.TYPE_Q4_K, N * H, seed * 10 + r, 0.02) for r in range(3)]
            self.sh = [t.cpu().numpy() for t in self.d_sh]
            self.sh_inp = (rng.standard_normal(H) * 0.02).astype(np.float32)
            self.d_sh_inp = torch.from_numpy(self.sh_inp).cuda()
        self.rng = rng

    def layer(self, pools):
        L = qa.MoeLayer()
        L.gate_pool = qa.tensor(qa.TYPE_Q4_K, H, self.N, self.S, pools[0])
        L.up_pool = qa.tensor(qa.TYPE_Q4_K, H, self.N, self.S, pools[1])
        L.down_pool = qa.tensor(qa.TYPE_Q4_K, self.N, H, self.S, pools[2])
        L.router = qa.tensor(qa.TYPE_F32, H, self.E, 1, self.d_router)
        if self.shared:
            L.sh_gate = qa.tensor(qa.TYPE_Q4_K, H, self.N, 1, self.d_sh[0])
            L.sh_up = qa.tensor(qa.TYPE_Q4_K, H, self.N, 1, self.d_sh[1])
            L.sh_down = qa.tensor(qa.TYPE_Q4_K, self.N, H, 1, self.d_sh[2])
            L.sh_gate_inp = qa.tensor(qa.TYPE_F32, H, 1, 1, self.d_sh_inp)
        L.n_expert_used = self.k
        L.norm_weights = 1
        L.weights_scale = 1.0
        return L

    def route(self, x, rm=None):
        T = x.shape[0]
        ids = np.zeros((T, self.k), np.int32)
        w = np.zeros((T, self.k), np.float32)
        mg = np.zeros(T, np.float32)
        assert oracle().qwo_route(I64(self.E), I64(H), I64(T), ptr(self.router), ptr(x),
                                  ptr(rm) if rm is not None else None, self.k, 1, F32(1.0),
                                  ptr(ids), ptr(w), None, None, ptr(mg)) == 0
        return ids, w, mg

    def block(self, x, host_pools, n_slots, slots, w):
        """Oracle block over host pools [3] with per-role slot ids slots[3][T][k]."""
        T = x.shape[0]
        out = np.zeros((T, H), np.float32)
        a = QwoMoeArgs()
        a.H, a.N, a.k, a.T = H, self.N, self.k, T
        a.weight_type = a.down_type = GGML_Q4_K
        a.gate_pool, a.up_pool, a.down_pool = (p.ctypes.data for p in host_pools)
        a.n_slots = n_slots
        sl = [np.ascontiguousarray(s, np.int32) for s in slots]
        a.slot_g, a.slot_u, a.slot_d = (s.ctypes.data for s in sl)
        w = np.ascontiguousarray(w, np.float32)
        a.weights = w.ctypes.data
        x = np.ascontiguousarray(x)
        a.x = x.ctypes.data
        if self.shared:
            a.sh_gate, a.sh_up, a.sh_down = (t.ctypes.data for t in self.sh)
            a.N_sh = self.N
            a.sh_gate_inp = self.sh_inp.ctypes.data
        a.out = out.ctypes.data
        assert oracle().qwo_moe_block(ctypes.byref(a)) == 0
        return out


def resident_pools(E, N, seed):
    """All E experts of a layer, one slab per slot: device pools and host bytes."""
    d = [gpu_weights(qa.TYPE_Q4_K, E * N * H, seed + r, 0.02) for r in range(3)]
    return d, [t.cpu().numpy() for t in d]


def test_config_verify_step_full_vocab(dev):
    E, N, k, T, V = 128, 768, 8, 4, 151936
    blk = Block(501, E, N, k, E)
    d_pools, h_pools = resident_pools(E, N, 510)
    perms = [blk.rng.permutation(E).astype(np.int32) for _ in range(3)]      # expert -> slot, per role
    layer = blk.layer(d_pools)
    d_lm = gpu_weights(qa.TYPE_Q8_0, V * H, 520, 1.0 / np.sqrt(H))
    Wq = d_lm.cpu().numpy()
    lm_t = qa.tensor(qa.TYPE_Q8_0, H, V, 1, d_lm)
    table = np.concatenate(perms).astype(np.int32)
    dtab = torch.from_numpy(table).cuda()
    norm_w = (1.0 + 0.1 * blk.rng.standard_normal(H)).astype(np.float32)
    dn = torch.from_numpy(norm_w).cuda()
    L = qa.lib()
    ws = workspace(L.qwm_verify_step_workspace_size(layer, lm_t, T))
    for rep in range(2):
        x = blk.rng.standard_normal((T, H)).astype(np.float32)
        ids, w, _ = blk.route(x)
        out_ref = blk.block(x, h_pools, E, [perms[r][ids] for r in range(3)], w) + x
        vA0, _, _, _ = oracle_verify(Wq, H, V, out_ref, norm_w, 1e-6, np.zeros(T - 1, np.int32))
        drafts = np.where(blk.rng.random(T - 1) < 0.7, vA0[:T - 1], blk.rng.integers(0, V, T - 1)).astype(np.int32)
        vA, a, xn, margins = oracle_verify(Wq, H, V, out_ref, norm_w, 1e-6, drafts)
        dx = torch.from_numpy(x).cuda()
        ddr = torch.from_numpy(drafts).cuda()
        out = torch.zeros((T, H), device="cuda")
        gi = torch.zeros((T, k), dtype=torch.int32, device="cuda")
        gw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
        r = torch.zeros(T + 2, dtype=torch.int32, device="cuda")
        xt = qa.tensor(qa.TYPE_F32, H, T, 1, dx)
        print(f"verify step full vocab: rep {rep}", flush=True)
        qa.check(L.qwm_verify_step(layer, 0, dtab.data_ptr(), E, xt, None, xt, qa.tensor(qa.TYPE_F32, H, T, 1, out),
                                   qa.tensor(qa.TYPE_I32, k, T, 1, gi), qa.tensor(qa.TYPE_F32, k, T, 1, gw), lm_t,
                                   dn.data_ptr(), 1e-6, ddr.data_ptr(), r.data_ptr(), ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        rr = r.cpu().numpy()
        print(f"  result {rr.tolist()} oracle vA {vA.tolist()} a={a} x_new={xn} margins {margins.tolist()}", flush=True)
        assert rr[T] >= 0, "device-side wait timed out"
        assert np.array_equal(gi.cpu().numpy(), ids) and np.array_equal(bits(gw.cpu().numpy()), bits(w))
        assert np.array_equal(bits(out.cpu().numpy()), bits(out_ref)), "block output not bit-exact"
        clear = margins > 1e-3
        assert np.array_equal(rr[:T][clear], vA[clear])
        if clear.all():
            assert (rr[T], rr[T + 1]) == (a, xn)


def test_config_decode_48_layers(dev):
    """48 blocks share one 128-slab pool per role; each (layer, role) maps the
    layer's experts onto it through its own random permutation, and each
    layer has its own router."""
    E, N, k, n_layers = 128, 768, 8, 48
    d_pools, h_pools = resident_pools(E, N, 600)
    blks = [Block(700 + l, E, N, k, E) for l in range(n_layers)]
    rng = np.random.default_rng(17)
    perms = rng.permuted(np.tile(np.arange(E, dtype=np.int32), (n_layers, 3, 1)), axis=2)   # [layer][role][expert]
    tables = np.ascontiguousarray(perms.transpose(1, 0, 2).reshape(3, n_layers * E)).astype(np.int32)
    layers = (qa.MoeLayer * n_layers)()
    for l, b in enumerate(blks):
        layers[l] = b.layer(d_pools)
    L = qa.lib()
    dtab = torch.from_numpy(tables).cuda()
    ws = workspace(L.qwm_moe_decode_workspace_size(layers, n_layers, 1))
    for tok in range(2):
        x0 = rng.standard_normal((1, H)).astype(np.float32)
        x = x0.copy()
        for l, b in enumerate(blks):
            ids, w, _ = b.route(x)
            x = b.block(x, h_pools, E, [perms[l, r][ids] for r in range(3)], w) + x
        dx = torch.from_numpy(x0).cuda()
        print(f"decode 48 layers: token {tok}", flush=True)
        qa.check(L.qwm_moe_decode(layers, n_layers, dtab.data_ptr(), n_layers * E, qa.tensor(qa.TYPE_F32, H, 1, 1, dx),
                                  ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        got = dx.cpu().numpy()
        print(f"  rel err {rel_err(got, x):.3e}", flush=True)
        assert np.array_equal(bits(got), bits(x)), "48-layer decode not bit-exact"


@pytest.mark.parametrize("fetch", ["memcpy", "gather"])
def test_config_missfill_zipf(dev, fetch):
    E, N, k, T, S, steps = 512, 512, 10, 4, 128, 24
    blk = Block(800, E, N, k, S, shared=True)
    d_all, h_all = resident_pools(E, N, 810)             # the host tier: every expert's slabs
    slab = h_all[0].size // E
    host = [pinned(h) for h in h_all]
    del d_all
    host_ptrs = [(ctypes.c_void_p * 1)(host[r].data_ptr()) for r in range(3)]
    pool_t = [torch.full((S * slab,), 0xA5, dtype=torch.uint8, device="cuda") for _ in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = 1, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
        d.host_slabs[r] = ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = {"memcpy": qa.FETCH_MEMCPY, "gather": qa.FETCH_GATHER}[fetch]
    L = qa.lib()
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    o = oracle().qwo_pool_new(1, E, ptr(np.array([S, S, S], np.int32)), 0)
    layer = blk.layer(pool_t)
    ws = workspace(L.qwm_moe_cached_workspace_size(layer, T))
    perm = blk.rng.permutation(E)
    try:
        for step in range(steps):
            x = blk.rng.standard_normal((T, H)).astype(np.float32)
            mask = zipf_mask(blk.rng, perm, k, T)
            ids, w, _ = blk.route(x, mask)
            dx, drm = torch.from_numpy(x).cuda(), torch.from_numpy(mask).cuda()
            out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
            hids = np.zeros(T * k, np.int32)
            print(f"miss fill {fetch}: step {step}", flush=True)
            qa.check(L.qwm_moe_cached_step(layer, h, 0, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                                           qa.tensor(qa.TYPE_F32, E, T, 1, drm), None,
                                           qa.tensor(qa.TYPE_F32, H, T, 1, out), ptr(hids), ws.data_ptr(), ws.numel(),
                                           None))
            assert np.array_equal(hids.reshape(T, k), ids), f"step {step}: routed ids differ"
            so = np.zeros((3, T * k), np.int32)
            flat = np.ascontiguousarray(ids.ravel())
            nf = ctypes.c_int()
            assert oracle().qwo_pool_ensure(o, 0, ptr(flat), flat.size, ptr(so[0]), ptr(so[1]), ptr(so[2]), None,
                                            ctypes.byref(nf)) == 0
            got = out.cpu().numpy()
            exp = blk.block(x, h_all, E, [ids, ids, ids], w)    # every expert from the host tier
            err = rel_err(got, exp)
            assert np.array_equal(bits(got), bits(exp)), f"step {step}: rel err {err:.3e}"
        st = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(h, ctypes.byref(st)))
        print(f"  hits {st.hits} misses {st.misses} evictions {st.evictions}", flush=True)
        assert st.evictions > 0
        torch.cuda.synchronize()
        for r in range(3):
            kg, cg = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            ko, co = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            qa.check(L.qwm_pool_slots(h, r, ptr(kg), ptr(cg)))
            oracle().qwo_pool_slots(o, r, ptr(ko), ptr(co))
            assert np.array_equal(kg, ko) and np.array_equal(cg, co), f"role {r}: pool state differs from the oracle's"
            dev_bytes = pool_t[r].cpu().numpy().reshape(S, slab)
            src = h_all[r].reshape(E, slab)
            for s, key in enumerate(kg):
                if key >= 0:
                    assert np.array_equal(dev_bytes[s], src[key]), f"role {r} slot {s} does not hold expert {key}"
    finally:
        L.qwm_pool_destroy(h)
        oracle().qwo_pool_free(o)


@pytest.mark.parametrize("K,N", [(2048, 512), (512, 2048)])
def test_config_prefill_mul_mat_id(dev, K, N):
    """512 columns, 10 distinct experts each out of 512 (Zipf(1.1) popularity
    over a permutation, so some experts take many columns and some none);
    gate/up broadcast one input column (ne11 = 1), down reads one input per
    pair (ne11 = 10)."""
    E, T, n_ids = 512, 512, 10
    ne11 = 1 if K == 2048 else n_ids
    d_as = gpu_weights(qa.TYPE_Q4_K, E * N * K, 900 + K, 0.02)
    h_as = d_as.cpu().numpy()
    rng = np.random.default_rng(K)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    perm = rng.permutation(E)
    ids = np.stack([perm[rng.choice(E, n_ids, replace=False, p=p)] for _ in range(T)]).astype(np.int32)
    b = rng.standard_normal((T, ne11, K)).astype(np.float32)
    exp = np.zeros((T, n_ids, N), np.float32)
    assert oracle().qwo_mul_mat_id(GGML_Q4_K, ptr(h_as), I64(K), I64(N), I64(E), ptr(b), I64(ne11), I64(T),
                                   ptr(ids), I64(n_ids), ptr(exp)) == 0
    db, dids = torch.from_numpy(b).cuda(), torch.from_numpy(ids).cuda()
    dst = torch.full((T, n_ids, N), float("nan"), dtype=torch.float32, device="cuda")
    tas = qa.tensor(qa.TYPE_Q4_K, K, N, E, d_as)
    tb = qa.tensor(qa.TYPE_F32, K, ne11, T, db)
    tids = qa.tensor(qa.TYPE_I32, n_ids, T, 1, dids)
    L = qa.lib()
    ws = workspace(L.qwm_mul_mat_id_workspace_size(tas, tb, tids))
    for rep in range(2):                      # the grouping counters re-arm themselves
        print(f"prefill mul_mat_id K={K} N={N}: call {rep}", flush=True)
        qa.check(L.qwm_mul_mat_id(tas, tb, tids, qa.tensor(qa.TYPE_F32, N, n_ids, T, dst), ws.data_ptr(),
                                  ws.numel(), None))
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        err = rel_err(got, exp)
        worst = max(rel_err(got[t], exp[t]) for t in range(T))
        print(f"  rel err {err:.3e}, worst column {worst:.3e}, experts used {np.unique(ids).size}", flush=True)
        assert np.isfinite(got).all() and err < 1e-3 and worst < 1e-3


def test_config_batch_through_pool(dev):
    """A 64-token batch through the Qwen3-Next-shape layer (512 experts +
    shared, FFN 512, top-10) and a 128-slot pool per role
    (qwm_moe_cached_batch): Zipf(1.1) routing makes the batch's union exceed
    the pool, so plan_slices cuts it into several slices; ids bit-exact,
    slices and final pool state equal to the oracle's, output within 1e-5 of
    the oracle block over the full expert table."""
    E, N, k, T, S = 512, 512, 10, 64, 128
    blk = Block(880, E, N, k, S, shared=True)
    d_all, h_all = resident_pools(E, N, 890)
    slab = h_all[0].size // E
    host = [pinned(hh) for hh in h_all]
    del d_all
    host_ptrs = [(ctypes.c_void_p * 1)(host[r].data_ptr()) for r in range(3)]
    pool_t = [torch.full((S * slab,), 0xA5, dtype=torch.uint8, device="cuda") for _ in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = 1, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
        d.host_slabs[r] = ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = qa.FETCH_GATHER
    L = qa.lib()
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    o = oracle().qwo_pool_new(1, E, ptr(np.array([S, S, S], np.int32)), 0)
    layer = blk.layer(pool_t)
    try:
        x = blk.rng.standard_normal((T, H)).astype(np.float32)
        resid = blk.rng.standard_normal((T, H)).astype(np.float32)
        mask = zipf_mask(blk.rng, blk.rng.permutation(E), k, T)
        ids, w, _ = blk.route(x, mask)
        exp = blk.block(x, h_all, E, [ids, ids, ids], w) + resid
        flat = np.ascontiguousarray(ids.ravel())
        sl_o = np.zeros(2 * T, np.int32)
        ns_o = oracle().qwo_pool_plan_slices(o, 0, ptr(flat), T, k, 0, ptr(sl_o), None)
        nf = ctypes.c_int()
        for i in range(ns_o):
            t0, ln = sl_o[2 * i], sl_o[2 * i + 1]
            sub = np.ascontiguousarray(flat[t0 * k:(t0 + ln) * k])
            s3 = np.zeros((3, sub.size), np.int32)
            assert oracle().qwo_pool_ensure(o, 0, ptr(sub), sub.size, ptr(s3[0]), ptr(s3[1]), ptr(s3[2]), None,
                                            ctypes.byref(nf)) == 0
        dx, dr, drm = torch.from_numpy(x).cuda(), torch.from_numpy(resid).cuda(), torch.from_numpy(mask).cuda()
        out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
        ws = workspace(L.qwm_moe_cached_batch_workspace_size(layer, T, 0))
        hids = np.zeros(T * k, np.int32)
        hsl = np.zeros(2 * T, np.int32)
        nsl = ctypes.c_int32()
        print(f"batch through the pool: T={T}, oracle slices {ns_o}", flush=True)
        qa.check(L.qwm_moe_cached_batch(layer, h, 0, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                                        qa.tensor(qa.TYPE_F32, E, T, 1, drm), qa.tensor(qa.TYPE_F32, H, T, 1, dr),
                                        qa.tensor(qa.TYPE_F32, H, T, 1, out), 0, ptr(hids), ptr(hsl),
                                        ctypes.byref(nsl), ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        slices = [tuple(hsl[2 * i:2 * i + 2]) for i in range(nsl.value)]
        got = out.cpu().numpy()
        print(f"  slices {slices}, rel err {rel_err(got, exp):.3e}", flush=True)
        assert np.array_equal(hids.reshape(T, k), ids)
        assert slices == [tuple(sl_o[2 * i:2 * i + 2]) for i in range(ns_o)] and len(slices) >= 2
        assert np.isfinite(got).all() and rel_err(got, exp) < 1e-5
        for r in range(3):
            kg, cg = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            ko, co = np.zeros(S, np.int32), np.zeros(S, np.uint64)
            qa.check(L.qwm_pool_slots(h, r, ptr(kg), ptr(cg)))
            oracle().qwo_pool_slots(o, r, ptr(ko), ptr(co))
            assert np.array_equal(kg, ko) and np.array_equal(cg, co), f"role {r}: pool state differs"
    finally:
        L.qwm_pool_destroy(h)
        oracle().qwo_pool_free(o)
