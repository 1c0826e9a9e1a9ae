"""GPU check of qwm_verify_step_noalloc (the fused verify step with its scratch
in a static device array instead of a caller workspace) against
qwm_verify_step on a workspace: outputs, routed ids and weights, and the
accept result bit for bit, on two calls in a row whose second is smaller
(fewer tokens, so the array keeps the first call's larger contents)."""
import numpy as np
import pytest

from tests.helpers import bits, quantize_q8_0_model
from tests.moe_case import MoeCase

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402

pytestmark = pytest.mark.gpu
V = 16384


def _workspace(nbytes):
    ws = torch.empty(max(256, (nbytes + 255) // 256 * 256), dtype=torch.uint8, device="cuda")
    qa.check(qa.lib().qwm_workspace_init(ws.data_ptr(), ws.numel(), None))
    return ws


def test_noalloc_step_matches_workspace_step():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L = qa.lib()
    rng = np.random.default_rng(91)
    Wq = quantize_q8_0_model((rng.standard_normal((V, 2048)) / np.sqrt(2048)).astype(np.float32))
    dW = torch.from_numpy(Wq).cuda()
    lm_t = qa.tensor(qa.TYPE_Q8_0, 2048, V, 1, dW)
    case = MoeCase(seed=4242, S=32, E=128, k=8, N=768)
    case.upload(torch)
    layer = case.layer
    table = np.tile(np.arange(case.E, dtype=np.int32) % case.S, 3)       # expert e lives in slot e % 32
    dtab = torch.from_numpy(table).cuda()
    for T in (4, 2):                                 # the second call is the smaller one
        print(f"noalloc step: T={T}", flush=True)
        x = case.rng.standard_normal((T, case.H)).astype(np.float32)
        ids, w, _, _ = case.route(x)
        drafts = case.rng.integers(0, V, max(T - 1, 1)).astype(np.int32)
        dx = torch.from_numpy(x).cuda()
        ddr = torch.from_numpy(drafts).cuda()
        xt = qa.tensor(qa.TYPE_F32, case.H, T, 1, dx)
        ws = _workspace(L.qwm_verify_step_workspace_size(layer, lm_t, T))
        assert ws.numel() <= qa.NOALLOC_SCRATCH_BYTES
        res = {}
        for path in ("workspace", "noalloc"):
            out = torch.zeros((T, case.H), device="cuda")
            gi = torch.zeros((T, case.k), dtype=torch.int32, device="cuda")
            gw = torch.zeros((T, case.k), dtype=torch.float32, device="cuda")
            r = torch.zeros(T + 2, dtype=torch.int32, device="cuda")
            ot = qa.tensor(qa.TYPE_F32, case.H, T, 1, out)
            it = qa.tensor(qa.TYPE_I32, case.k, T, 1, gi)
            wt = qa.tensor(qa.TYPE_F32, case.k, T, 1, gw)
            if path == "workspace":
                qa.check(L.qwm_verify_step(layer, 0, dtab.data_ptr(), case.E, xt, None, xt, ot, it, wt, lm_t, None,
                                           1e-6, ddr.data_ptr(), r.data_ptr(), ws.data_ptr(), ws.numel(), None))
            else:
                qa.check(L.qwm_verify_step_noalloc(layer, 0, dtab.data_ptr(), case.E, xt, None, xt, ot, it, wt, lm_t,
                                                   None, 1e-6, ddr.data_ptr(), r.data_ptr(), None))
            torch.cuda.synchronize()
            res[path] = (out.cpu().numpy(), gi.cpu().numpy(), gw.cpu().numpy(), r.cpu().numpy())
        oa, ia, wa, ra = res["workspace"]
        ob, ib, wb, rb = res["noalloc"]
        print(f"  workspace result {ra.tolist()} noalloc result {rb.tolist()}", flush=True)
        assert ra[T] >= 0 and rb[T] >= 0, "device-side wait timed out"
        assert np.array_equal(ia, ids) and np.array_equal(ib, ids), "routed ids differ from the oracle"
        assert np.array_equal(bits(wb), bits(w))
        assert np.array_equal(bits(ob), bits(oa)), "block output differs between the two entry points"
        assert np.array_equal(rb, ra), "accept result differs between the two entry points"
