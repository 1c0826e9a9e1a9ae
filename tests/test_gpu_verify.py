"""GPU parity of the verify head (rms_norm -> Q8_0 lm_head -> argmax) and the
greedy MTP acceptance against the oracle.  vA, the accepted count and the
next token must be identical; a differing argmax is only tolerated where the
oracle's top-2 logit margin is below 1e-5 (a near-tie that no fp32 summation
order can settle), and the test reports the margins it saw."""
import ctypes

import numpy as np
import pytest

from tests.helpers import F32, I64, oracle, ptr, quantize_q8_0_model

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402

pytestmark = pytest.mark.gpu
NEAR_TIE = 1e-5


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()
    return torch.device("cuda:0")


def oracle_verify(Wq, H, V, x, norm_w, eps, drafts):
    T = x.shape[0]
    h = np.zeros_like(x)
    for t in range(T):
        oracle().qwo_rms_norm(I64(H), ptr(x[t]), F32(eps), ptr(norm_w) if norm_w is not None else None, ptr(h[t]))
    vA = np.zeros(T, np.int32)
    mg = np.zeros(T, np.float32)
    assert oracle().qwo_lm_head_argmax(ptr(Wq), I64(H), I64(V), ptr(h), I64(T), ptr(vA), None, ptr(mg)) == 0
    xn = ctypes.c_int32()
    a = oracle().qwo_accept(ptr(vA), ptr(drafts), T - 1, ctypes.byref(xn)) if T > 1 else 0
    return vA, a, (xn.value if T > 1 else int(vA[0])), mg


def gpu_verify(dW, H, V, x, norm_w, eps, drafts):
    T = x.shape[0]
    lm = qa.tensor(qa.TYPE_Q8_0, H, V, 1, dW)
    need = qa.lib().qwm_verify_workspace_size(lm, T)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    dx = torch.from_numpy(x).cuda()
    dn = torch.from_numpy(norm_w).cuda() if norm_w is not None else None
    dd = torch.from_numpy(drafts).cuda() if T > 1 else None
    res = torch.zeros(T + 2, dtype=torch.int32, device="cuda")
    qa.check(qa.lib().qwm_verify_accept(lm, qa.tensor(qa.TYPE_F32, H, T, 1, dx), dn.data_ptr() if dn is not None else None,
                                        eps, dd.data_ptr() if dd is not None else None, res.data_ptr(), ws.data_ptr(),
                                        ws.numel(), None))
    torch.cuda.synchronize()
    r = res.cpu().numpy()
    return r[:T], int(r[T]), int(r[T + 1])


def check_case(vA, a, xn, gvA, ga, gxn, mg):
    for t in range(len(vA)):
        if gvA[t] != vA[t]:
            assert mg[t] < NEAR_TIE, f"argmax differs at t={t} with margin {mg[t]}"
            return False
    assert (ga, gxn) == (a, xn)
    return True


@pytest.mark.parametrize("H,V,T", [(2048, 32768, 4), (2048, 4096, 1), (2048, 8192, 8), (2048, 1000, 2),
                                   (4096, 16384, 4), (4096, 3000, 1), (3072, 8192, 3)])
def test_verify_accept_parity(dev, H, V, T):
    """Hidden sizes 3072 and 4096 (up to 4 tokens) beside 2048."""
    rng = np.random.default_rng(V + T)
    W = (rng.standard_normal((V, H)) / np.sqrt(H)).astype(np.float32)
    Wq = quantize_q8_0_model(W)
    dW = torch.from_numpy(Wq).cuda()
    norm_w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    margins = []
    for rep in range(6):
        x = (rng.standard_normal((T, H)) * (1 + rep)).astype(np.float32)
        nw = norm_w if rep % 2 else None
        vA0, _, _, _ = oracle_verify(Wq, H, V, x, nw, 1e-6, np.zeros(max(T - 1, 1), np.int32))
        # drafts: accept the first `rep % T` tokens, then a mismatch
        drafts = vA0[: max(T - 1, 1)].copy()
        if T > 1 and rep % T < T - 1:
            drafts[rep % T] = (drafts[rep % T] + 1) % V
        vA, a, xn, mg = oracle_verify(Wq, H, V, x, nw, 1e-6, drafts)
        gvA, ga, gxn = gpu_verify(dW, H, V, x, nw, 1e-6, drafts)
        margins.extend(mg.tolist())
        check_case(vA, a, xn, gvA, ga, gxn, mg)
        if T > 1:
            assert a == (rep % T if rep % T < T - 1 else T - 1)
    print(f"verify H={H} V={V} T={T}: min top-2 margin {min(margins):.3e}")


def test_verify_full_vocab(dev):
    """The workload's lm_head (Q8_0 2048 x 151936), one 4-token verify batch."""
    H, V, T = 2048, 151936, 4
    g = torch.Generator(device="cuda").manual_seed(7)
    Wf = torch.randn((V, H), generator=g, device="cuda") / np.sqrt(H)
    W = Wf.cpu().numpy()
    del Wf
    Wq = quantize_q8_0_model(W)
    del W
    dW = torch.from_numpy(Wq).cuda()
    rng = np.random.default_rng(3)
    x = rng.standard_normal((T, H)).astype(np.float32)
    vA0, _, _, _ = oracle_verify(Wq, H, V, x, None, 1e-6, np.zeros(T - 1, np.int32))
    drafts = vA0[: T - 1].copy()
    drafts[2] = (drafts[2] + 5) % V          # accept 2 drafts
    vA, a, xn, mg = oracle_verify(Wq, H, V, x, None, 1e-6, drafts)
    gvA, ga, gxn = gpu_verify(dW, H, V, x, None, 1e-6, drafts)
    print(f"full vocab: vA {vA.tolist()} gpu {gvA.tolist()} a={a}/{ga} margins {mg.tolist()}")
    assert check_case(vA, a, xn, gvA, ga, gxn, mg)
    assert a == 2 and xn == vA[2]
