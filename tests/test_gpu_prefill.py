"""GPU parity of GGML_OP_MUL_MAT_ID on prefill-sized batches (more than 8
columns: the expert-grouped GEMM on int8 MFMA, Q4_K and Q8_0 weights) against
the oracle's ggml-CPU restatement, on Qwen3-Next-like shapes (gate/up: K 2048,
N 512; down: K 512, N 2048), with skewed expert popularity, experts left
without columns, column counts that are not multiples of the 16-column tile,
and two calls in a row on one workspace (the grouping counters re-arm
themselves); Q8_0 weights off 16-byte alignment take the GEMV chunks, bit for
bit against the oracle."""
import numpy as np
import pytest

from tests.helpers import GGML_Q4_K, GGML_Q8_0, I64, bits, oracle, ptr, quantize_q4_K, quantize_q8_0_model
from tests.moe_case import rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3


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


def zipf_ids(rng, T, n_ids, n_as, skew):
    """Distinct experts per column; popularity ~ rank^-skew (skew 0: uniform)."""
    p = 1.0 / np.arange(1, n_as + 1) ** skew
    p /= p.sum()
    perm = rng.permutation(n_as)
    return np.stack([perm[rng.choice(n_as, n_ids, replace=False, p=p)] for _ in range(T)]).astype(np.int32)


QTYPE = {GGML_Q4_K: qa.TYPE_Q4_K, GGML_Q8_0: qa.TYPE_Q8_0}


def run_case(rng, K, N, n_as, n_ids, ne11, T, skew, ws=None, q=None, wtype=GGML_Q4_K, offset=0):
    """offset: bytes the weights sit past a 256-byte boundary on the device."""
    w = None
    if q is None:
        w = (rng.standard_normal((n_as, N, K)) * 0.02).astype(np.float32)
        q = quantize_q4_K(w) if wtype == GGML_Q4_K else quantize_q8_0_model(w)
    b = rng.standard_normal((T, ne11, K)).astype(np.float32)
    ids = zipf_ids(rng, T, n_ids, n_as, skew)
    exp = np.zeros((T, n_ids, N), np.float32)
    assert oracle().qwo_mul_mat_id(wtype, ptr(q), I64(K), I64(N), I64(n_as), ptr(b), I64(ne11), I64(T),
                                   ptr(ids), I64(n_ids), ptr(exp)) == 0
    das = torch.zeros(q.size + 256, dtype=torch.uint8, device="cuda")[offset:offset + q.size]
    das.copy_(torch.from_numpy(q))
    db = torch.from_numpy(b).cuda()
    dids = torch.from_numpy(ids).cuda()
    dst = torch.full((T, n_ids, N), float("nan"), dtype=torch.float32, device="cuda")
    tas = qa.tensor(QTYPE[wtype], K, N, n_as, das)
    tb = qa.tensor(qa.TYPE_F32, K, ne11, T, db)
    tids = qa.tensor(qa.TYPE_I32, n_ids, T, 1, dids)
    need = qa.lib().qwm_mul_mat_id_workspace_size(tas, tb, tids)
    assert need > 0
    if ws is None or ws.numel() < need:
        ws = workspace(need)
    qa.check(qa.lib().qwm_mul_mat_id(tas, tb, tids, qa.tensor(qa.TYPE_F32, N, n_ids, T, dst), ws.data_ptr(),
                                     ws.numel(), None))
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    return got, exp, ids, ws, q


@pytest.mark.parametrize("wtype", [GGML_Q4_K, GGML_Q8_0])
@pytest.mark.parametrize("K,N,n_as,n_ids,ne11,T,skew", [
    (2048, 512, 64, 8, 1, 64, 0.0),      # gate/up shape, uniform
    (2048, 512, 64, 8, 1, 40, 1.1),      # Zipf(1.1): uneven groups, experts without columns
    (512, 2048, 64, 8, 8, 48, 0.5),      # down shape: one b row per (column, slot)
    (768, 2048, 32, 4, 4, 24, 0.0),      # K = 3 blocks
    (256, 64, 16, 2, 1, 9, 0.0),         # smallest: K one block, one row tile
    (4096, 256, 16, 8, 1, 24, 0.0),      # hidden 4096 (Qwen3-235B-A22B gate/up): one workgroup per CU
    (3072, 128, 16, 4, 1, 20, 0.5),      # hidden 3072: two workgroups per CU
])
def test_prefill_mul_mat_id(dev, wtype, K, N, n_as, n_ids, ne11, T, skew):
    rng = np.random.default_rng(K + N + T)
    got, exp, ids, _, _ = run_case(rng, K, N, n_as, n_ids, ne11, T, skew, wtype=wtype)
    counts = np.bincount(ids.ravel(), minlength=n_as)
    err = rel_err(got, exp)
    print(f"prefill type={wtype} K={K} N={N} T={T} skew={skew}: rel err {err:.3e}; columns per expert max {counts.max()} "
          f"empty experts {int((counts == 0).sum())}")
    assert np.isfinite(got).all(), "some outputs were not written"
    assert err < TOL
    for t in range(T):
        for e in range(n_ids):
            assert rel_err(got[t, e], exp[t, e]) < TOL


def test_prefill_repeat_on_one_workspace(dev):
    """Calls of different shapes on one workspace (a layer's gate/up and its
    down projection lay the workspace out differently): no state may carry
    over from one call to the next."""
    rng = np.random.default_rng(3)
    L = qa.lib()
    ids_t = qa.tensor(qa.TYPE_I32, 6, 30, 1)
    big = max(L.qwm_mul_mat_id_workspace_size(qa.tensor(qa.TYPE_Q4_K, 512, 2048, 32), qa.tensor(qa.TYPE_F32, 512, 6, 30), ids_t),
              L.qwm_mul_mat_id_workspace_size(qa.tensor(qa.TYPE_Q4_K, 2048, 512, 32), qa.tensor(qa.TYPE_F32, 2048, 1, 30), ids_t))
    ws = workspace(big)
    got1, exp1, _, ws, q = run_case(rng, 2048, 512, 32, 6, 1, 30, 1.1, ws=ws)
    got2, exp2, _, _, _ = run_case(rng, 512, 2048, 32, 6, 6, 30, 0.0, ws=ws)
    got3, exp3, _, _, _ = run_case(rng, 2048, 512, 32, 6, 1, 30, 0.0, ws=ws, q=q)
    for g, e in ((got1, exp1), (got2, exp2), (got3, exp3)):
        assert np.isfinite(g).all() and rel_err(g, e) < TOL


def test_prefill_q80_unaligned_weights_take_the_gemv_chunks(dev):
    """Q8_0 weights 4 bytes past a 16-byte boundary: the grouped GEMM needs
    16-byte aligned pieces, so the call runs the GEMV chunks, whose results
    are ggml's bit for bit; the same weights aligned take the GEMM (1e-3)."""
    rng = np.random.default_rng(5)
    q = quantize_q8_0_model((rng.standard_normal((16, 128, 512)) * 0.02).astype(np.float32))
    got, exp, _, _, _ = run_case(rng, 512, 128, 16, 4, 1, 20, 0.0, q=q, wtype=GGML_Q8_0, offset=4)
    np.testing.assert_array_equal(bits(got), bits(exp))
    got2, exp2, _, _, _ = run_case(rng, 512, 128, 16, 4, 1, 20, 0.0, q=q, wtype=GGML_Q8_0, offset=0)
    assert np.isfinite(got2).all() and rel_err(got2, exp2) < TOL
