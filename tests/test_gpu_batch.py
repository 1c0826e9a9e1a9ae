"""GPU parity of a batched MoE layer through the slot pool
(qwm_moe_cached_batch: decode_cached_batch's router, plan_slices /
ensure_slice and seg B, runtime.cpp:4509-4572, 4639-4698) against the
oracle: routed ids bit-exact, slices equal to the oracle's plan, the pool's
slot keys and clocks equal to the oracle pool's after the same per-slice
ensure calls, every occupied slot holding its slab, and the layer's output
against the oracle block over the full expert table (bit-exact for slices of
at most 8 tokens; within 1e-5 where a slice takes the grouped GEMM)."""
import ctypes

import numpy as np
import pytest

from tests.helpers import bits, oracle, ptr
from tests.moe_case import MoeCase, rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from tests.test_gpu_pool import pinned, zipf_mask  # noqa: E402

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("T,max_slice,shared,fetch,S,H,E", [(40, 0, True, qa.FETCH_GATHER, 20, 512, 64),
                                                            (40, 0, False, qa.FETCH_MEMCPY, 20, 512, 64),
                                                            (30, 6, True, qa.FETCH_GATHER, 20, 512, 64),
                                                            (5, 0, True, qa.FETCH_MEMCPY, 20, 512, 64),
                                                            (40, 0, True, qa.FETCH_GATHER, 64, 512, 64),
                                                            (24, 0, True, qa.FETCH_GATHER, 20, 4096, 32)])
def test_cached_batch_matches_oracle(dev, T, max_slice, shared, fetch, S, H, E):
    """S = 64 slots hold every expert: one slice of 40 tokens, whose gate and up
    slots agree, so it runs the fused gate/up/SwiGLU pass.  H = 4096: the
    slices' MUL_MAT_IDs run as GEMV chunks (the grouped GEMM holds K <= 2048)."""
    N, k = 256, 4
    case = MoeCase(seed=71 + T, H=H, N=N, E=E, k=k, S=E, shared=shared, N_sh=N)
    rng = np.random.default_rng(T + max_slice)
    slab = case.gate_q.nbytes // E
    host = [pinned(case.gate_q), pinned(case.up_q), pinned(case.down_q)]
    host_ptrs = [(ctypes.c_void_p * 1)(host[r].data_ptr()) for r in range(3)]
    pool_t = [torch.full((S * slab,), 0xA5, dtype=torch.uint8, device="cuda") for _ in range(3)]
    d = qa.PoolDesc()
    d.n_layer, d.n_expert = 1, E
    for r in range(3):
        d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = S, pool_t[r].data_ptr(), slab
        d.host_slabs[r] = ctypes.cast(host_ptrs[r], ctypes.c_void_p)
    d.fetch_mode = fetch
    L = qa.lib()
    copy = torch.cuda.Stream()
    h = ctypes.c_void_p()
    qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(h)))
    o = oracle().qwo_pool_new(1, E, ptr(np.array([S, S, S], np.int32)), 0)
    case.upload(torch)
    lay = case.layer
    lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, H, N, S, pool_t[0])
    lay.up_pool = qa.tensor(qa.TYPE_Q4_K, H, N, S, pool_t[1])
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, N, H, S, pool_t[2])
    try:
        for rep in range(2):
            x = rng.standard_normal((T, H)).astype(np.float32)
            resid = rng.standard_normal((T, H)).astype(np.float32)
            mask = zipf_mask(rng, rng.permutation(E), k, T)
            ids, w, _, _ = case.route(x, mask)
            exp = case.block(x, ids, w) + resid
            # the oracle's plan and per-slice ensure calls
            flat = np.ascontiguousarray(ids.ravel())
            sl_o = np.zeros(2 * T, np.int32)
            ns_o = oracle().qwo_pool_plan_slices(o, 0, ptr(flat), T, k, max_slice, ptr(sl_o), None)
            so = np.zeros((3, flat.size), np.int32)
            nf = ctypes.c_int()
            for i in range(ns_o):
                t0, ln = sl_o[2 * i], sl_o[2 * i + 1]
                sub = np.ascontiguousarray(flat[t0 * k:(t0 + ln) * k])
                s3 = np.zeros((3, sub.size), np.int32)
                assert oracle().qwo_pool_ensure(o, 0, ptr(sub), sub.size, ptr(s3[0]), ptr(s3[1]), ptr(s3[2]), None,
                                                ctypes.byref(nf)) == 0
            dx, dr = torch.from_numpy(x).cuda(), torch.from_numpy(resid).cuda()
            drm = torch.from_numpy(mask).cuda()
            out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
            ws = workspace(L.qwm_moe_cached_batch_workspace_size(lay, T, max_slice))
            hids = np.zeros(T * k, np.int32)
            hsl = np.zeros(2 * T, np.int32)
            nsl = ctypes.c_int32()
            print(f"cached batch T={T} max_slice={max_slice} shared={shared} S={S} H={H}: rep {rep}", flush=True)
            qa.check(L.qwm_profile_start(b"prefill_gemm_gu", 64))
            qa.check(L.qwm_moe_cached_batch(lay, h, 0, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                                            qa.tensor(qa.TYPE_F32, E, T, 1, drm), qa.tensor(qa.TYPE_F32, H, T, 1, dr),
                                            qa.tensor(qa.TYPE_F32, H, T, 1, out), max_slice, ptr(hids), ptr(hsl),
                                            ctypes.byref(nsl), ws.data_ptr(), ws.numel(), None))
            torch.cuda.synchronize()
            durs = np.zeros(64, np.float32)
            n_fused = L.qwm_profile_stop(durs.ctypes.data, 64)
            slices = [tuple(hsl[2 * i:2 * i + 2]) for i in range(nsl.value)]
            if S == E:
                assert n_fused == sum(1 for _, ln in slices if ln > 8) >= 1, "the fused gate/up pass did not run"
            print(f"  slices {slices}", flush=True)
            assert np.array_equal(hids.reshape(T, k), ids), "routed ids differ"
            assert slices == [tuple(sl_o[2 * i:2 * i + 2]) for i in range(ns_o)], "slices differ from the oracle's"
            got = out.cpu().numpy()
            err = rel_err(got, exp)
            print(f"  rel err {err:.3e}", flush=True)
            assert np.isfinite(got).all() and err < 1e-5
            if max(ln for _, ln in slices) <= 8:
                assert np.array_equal(bits(got), bits(exp)), "GEMV-width slices must be bit-exact"
            for r in range(3):
                kg, cg = np.zeros(S, np.int32), np.zeros(S, np.uint64)
                ko, co = np.zeros(S, np.int32), np.zeros(S, np.uint64)
                qa.check(L.qwm_pool_slots(h, r, ptr(kg), ptr(cg)))
                oracle().qwo_pool_slots(o, r, ptr(ko), ptr(co))
                assert np.array_equal(kg, ko) and np.array_equal(cg, co), f"role {r}: pool state differs"
                dev_bytes = pool_t[r].cpu().numpy().reshape(S, slab)
                src = host[r].numpy().reshape(E, slab)
                for s_, key in enumerate(kg):
                    if key >= 0:
                        assert np.array_equal(dev_bytes[s_], src[key]), f"role {r} slot {s_}"
        if T >= 40 and S < E:
            assert nsl.value >= 2, "the batch should need several slices"
    finally:
        L.qwm_pool_destroy(h)
        oracle().qwo_pool_free(o)
