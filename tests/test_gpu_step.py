"""GPU parity of the fused verify step (qwm_verify_step: the MoE block and the
verify head in one persistent launch) against the oracle, and bit-for-bit
against the same step through the per-op entry points
(qwm_moe_block_resident + qwm_verify_accept).  Several consecutive steps run
on one workspace, so the launch's self-resetting barriers and tickets are
exercised across calls."""
import numpy as np
import pytest

from tests.helpers import bits, quantize_q8_0_model
from tests.moe_case import MoeCase, rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from tests.test_gpu_verify import oracle_verify  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3
V = 16384


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def lm_head(dev):
    rng = np.random.default_rng(77)
    W = (rng.standard_normal((V, 2048)) / np.sqrt(2048)).astype(np.float32)
    Wq = quantize_q8_0_model(W)
    return Wq, torch.from_numpy(Wq).cuda()


def workspace(nbytes):
    ws = torch.empty(max(256, (nbytes + 255) // 256 * 256), dtype=torch.uint8, device="cuda")
    qa.check(qa.lib().qwm_workspace_init(ws.data_ptr(), ws.numel(), None))
    return ws


def slot_tables(case, ids):
    """Selected experts -> pool slots (first-occurrence order), same for the 3 roles."""
    uniq = list(dict.fromkeys(int(e) for e in ids.ravel()))
    assert len(uniq) <= case.S
    table = np.zeros(case.E, np.int32)
    for s, e in enumerate(uniq):
        table[e] = s
    return np.tile(table, 3), table[ids]


@pytest.mark.parametrize("cfg", [
    dict(T=4, E=128, k=8, N=768),
    dict(T=1, E=128, k=8, N=768),
    dict(T=8, E=128, k=8, N=768),
    dict(T=4, E=512, k=10, N=512, shared=True),
    dict(T=2, E=512, k=10, N=512, shared=True, sh_gate=False),
    dict(T=4, E=128, k=8, N=768, down="q6_K"),                  # Q6_K down slabs (Q4_K_M last layers)
    dict(T=3, E=512, k=10, N=512, shared=True, down="q6_K"),
    dict(T=4, E=512, k=10, N=512, shared=True, gating=2, bias=0.05),   # sigmoid routing + exp_probs_b
    dict(T=2, E=128, k=8, N=768, bias=0.004),                           # soft_max + exp_probs_b
])
def test_fused_step(dev, lm_head, cfg):
    T = cfg.pop("T")
    Wq, dW = lm_head
    case = MoeCase(seed=1000 + T + cfg["E"], S=T * cfg["k"], **cfg)
    case.upload(torch)
    L = qa.lib()
    layer = case.layer
    lm_t = qa.tensor(qa.TYPE_Q8_0, 2048, V, 1, dW)
    ws_step = workspace(L.qwm_verify_step_workspace_size(layer, lm_t, T))
    ws_moe = workspace(L.qwm_moe_workspace_size(layer, T))
    ws_v = workspace(L.qwm_verify_workspace_size(lm_t, T))
    norm_w = (1.0 + 0.1 * case.rng.standard_normal(2048)).astype(np.float32)
    dn = torch.from_numpy(norm_w).cuda()
    for rep in range(3):
        x = case.rng.standard_normal((T, case.H)).astype(np.float32)
        ids, w, mg, _ = case.route(x)
        table, slots = slot_tables(case, ids)
        out_ref = case.block(x, slots, w) + x
        vA0, _, _, _ = oracle_verify(Wq, 2048, V, out_ref, norm_w, 1e-6, np.zeros(max(T - 1, 1), np.int32))
        keep = case.rng.random(max(T - 1, 1)) < 0.7
        drafts = np.where(keep, vA0[:max(T - 1, 1)], case.rng.integers(0, V, max(T - 1, 1))).astype(np.int32)
        vA, a, xn, margins = oracle_verify(Wq, 2048, V, out_ref, norm_w, 1e-6, drafts)

        dx = torch.from_numpy(x).cuda()
        dtab = torch.from_numpy(table).cuda()
        ddr = torch.from_numpy(drafts).cuda()
        xt = qa.tensor(qa.TYPE_F32, case.H, T, 1, dx)
        res = {}
        for path in ("ops", "step"):
            out = torch.zeros((T, case.H), device="cuda")
            gi = torch.zeros((T, case.k), dtype=torch.int32, device="cuda")
            gw = torch.zeros((T, case.k), dtype=torch.float32, device="cuda")
            r = torch.zeros(T + 2, dtype=torch.int32, device="cuda")
            ot = qa.tensor(qa.TYPE_F32, case.H, T, 1, out)
            it = qa.tensor(qa.TYPE_I32, case.k, T, 1, gi)
            wt = qa.tensor(qa.TYPE_F32, case.k, T, 1, gw)
            if path == "ops":
                qa.check(L.qwm_moe_block_resident(layer, 0, dtab.data_ptr(), case.E, xt, None, xt, ot, it, wt,
                                                  ws_moe.data_ptr(), ws_moe.numel(), None))
                qa.check(L.qwm_verify_accept(lm_t, ot, dn.data_ptr(), 1e-6, ddr.data_ptr(), r.data_ptr(),
                                             ws_v.data_ptr(), ws_v.numel(), None))
            else:
                qa.check(L.qwm_verify_step(layer, 0, dtab.data_ptr(), case.E, xt, None, xt, ot, it, wt, lm_t,
                                           dn.data_ptr(), 1e-6, ddr.data_ptr(), r.data_ptr(),
                                           ws_step.data_ptr(), ws_step.numel(), None))
            torch.cuda.synchronize()
            res[path] = (out.cpu().numpy(), gi.cpu().numpy(), gw.cpu().numpy(), r.cpu().numpy())
        out_b, ids_b, w_b, r_b = res["step"]
        out_a, ids_a, w_a, r_a = res["ops"]
        print(f"T={T} {cfg} rep {rep}: step result {r_b.tolist()} ops {r_a.tolist()} oracle vA {vA.tolist()} "
              f"a={a} rel err {rel_err(out_b, out_ref):.2e} min margin {float(np.min(margins)):.3e}", flush=True)
        assert r_b[T] >= 0, "device-side barrier timeout"
        assert np.array_equal(ids_b, ids) and np.array_equal(bits(w_b), bits(w))
        assert rel_err(out_b, out_ref) < TOL
        assert np.array_equal(bits(out_b), bits(out_ref)), "block output not bit-exact"
        assert np.array_equal(bits(out_b), bits(out_a)), "fused step and per-op path differ"
        assert np.array_equal(r_b, r_a)
        clear = margins > 1e-3
        assert np.array_equal(r_b[:T][clear], vA[clear])
        if clear.all():
            assert (r_b[T], r_b[T + 1]) == (a, xn)


def test_out_of_range_slots_are_clamped(dev, lm_head):
    """Slot tables with ids outside [0, S) -- -1, S + 3, -5 for the experts a
    token selects -- run without reading outside the pools: the per-op
    resident path and the fused step give bit for bit what the same tables
    give with those ids clamped to 0, S - 1 and 0."""
    T = 2
    Wq, dW = lm_head
    case = MoeCase(seed=4242, E=128, k=8, N=768, S=T * 8)
    case.upload(torch)
    L = qa.lib()
    layer = case.layer
    lm_t = qa.tensor(qa.TYPE_Q8_0, 2048, V, 1, dW)
    ws_step = workspace(L.qwm_verify_step_workspace_size(layer, lm_t, T))
    ws_moe = workspace(L.qwm_moe_workspace_size(layer, T))
    norm_w = np.ones(2048, np.float32)
    dn = torch.from_numpy(norm_w).cuda()
    x = case.rng.standard_normal((T, case.H)).astype(np.float32)
    ids, _, _, _ = case.route(x)
    table, _ = slot_tables(case, ids)
    e0, e1 = int(ids[0, 0]), int(ids[1, 1])
    bad = table.copy()
    bad[0 * case.E + e0], bad[1 * case.E + e0], bad[2 * case.E + e1] = -1, case.S + 3, -5
    clamped = table.copy()
    clamped[0 * case.E + e0], clamped[1 * case.E + e0], clamped[2 * case.E + e1] = 0, case.S - 1, 0
    dx = torch.from_numpy(x).cuda()
    ddr = torch.zeros(T - 1, dtype=torch.int32, device="cuda")
    xt = qa.tensor(qa.TYPE_F32, case.H, T, 1, dx)
    res = {}
    for name, tab in (("bad", bad), ("clamped", clamped)):
        dtab = torch.from_numpy(tab).cuda()
        for path in ("ops", "step"):
            out = torch.zeros((T, case.H), device="cuda")
            r = torch.zeros(T + 2, dtype=torch.int32, device="cuda")
            ot = qa.tensor(qa.TYPE_F32, case.H, T, 1, out)
            print(f"clamp test: table {name}, path {path}", flush=True)
            if path == "ops":
                qa.check(L.qwm_moe_block_resident(layer, 0, dtab.data_ptr(), case.E, xt, None, xt, ot, None, None,
                                                  ws_moe.data_ptr(), ws_moe.numel(), None))
            else:
                qa.check(L.qwm_verify_step(layer, 0, dtab.data_ptr(), case.E, xt, None, xt, ot, None, None, lm_t,
                                           dn.data_ptr(), 1e-6, ddr.data_ptr(), r.data_ptr(), ws_step.data_ptr(),
                                           ws_step.numel(), None))
            torch.cuda.synchronize()
            res[name, path] = out.cpu().numpy()
    for path in ("ops", "step"):
        assert np.isfinite(res["bad", path]).all()
        assert np.array_equal(bits(res["bad", path]), bits(res["clamped", path])), path
