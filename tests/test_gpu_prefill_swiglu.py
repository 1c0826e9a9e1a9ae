"""GPU parity of qwm_mul_mat_id_swiglu: act = swiglu_split(MUL_MAT_ID(gate),
MUL_MAT_ID(up)), the first half of build_segB (core/runtime.cpp:4539-4541).

Two bars.  Against the oracle's ggml-CPU restatement (qwo_mul_mat_id of gate
and of up, then qwo_swiglu per row) within the prefill GEMM's 1e-3.  Against
the GPU's own separate path (two qwm_mul_mat_id calls, then SwiGLU of those
outputs) bit for bit: the fused pass runs the same dots in the same order and
the same SwiGLU expressions.  Shapes: Qwen3-Next's gate/up (K 2048, N 512,
512 experts, top-10, 512 tokens) at full size, skewed and ragged groups on
smaller pools, Q8_0 weights, the T <= 8 path (separate calls inside), and two
calls in a row on one workspace."""
import numpy as np
import pytest

from tests.helpers import GGML_Q4_K, GGML_Q8_0, I64, oracle, ptr, quantize_q4_K, quantize_q8_0_model
from tests.moe_case import rel_err
from tests.test_gpu_prefill import workspace, zipf_ids

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3
QTYPE = {GGML_Q4_K: qa.TYPE_Q4_K, GGML_Q8_0: qa.TYPE_Q8_0}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()
    return torch.device("cuda:0")


def gpu_case(qg, qu, b, ids, K, N, n_as, gtype=GGML_Q4_K, ws=None):
    """Fused act and the separate path's gate, up (GPU), all as numpy."""
    L = qa.lib()
    T, ne11, _ = b.shape
    n_ids = ids.shape[1]
    dg, du = (q if torch.is_tensor(q) else torch.from_numpy(q).cuda() for q in (qg, qu))
    db = torch.from_numpy(b).cuda()
    dids = torch.from_numpy(ids).cuda()
    tg = qa.tensor(QTYPE[gtype], K, N, n_as, dg)
    tu = qa.tensor(QTYPE[gtype], K, N, n_as, du)
    tb = qa.tensor(qa.TYPE_F32, K, ne11, T, db)
    tids = qa.tensor(qa.TYPE_I32, n_ids, T, 1, dids)
    need = max(L.qwm_mul_mat_id_swiglu_workspace_size(tg, tu, tb, tids), L.qwm_mul_mat_id_workspace_size(tg, tb, tids))
    assert need > 0, L.qwm_last_error()
    if ws is None or ws.numel() < need:
        ws = workspace(need)
    act = torch.full((T, n_ids, N), float("nan"), dtype=torch.float32, device="cuda")
    qa.check(L.qwm_mul_mat_id_swiglu(tg, tu, tb, tids, qa.tensor(qa.TYPE_F32, N, n_ids, T, act), ws.data_ptr(),
                                     ws.numel(), None))
    torch.cuda.synchronize()
    act_np = act.cpu().numpy()
    sep = []
    for t in (tg, tu):
        dst = torch.full((T, n_ids, N), float("nan"), dtype=torch.float32, device="cuda")
        qa.check(L.qwm_mul_mat_id(t, tb, tids, qa.tensor(qa.TYPE_F32, N, n_ids, T, dst), ws.data_ptr(), ws.numel(),
                                  None))
        torch.cuda.synchronize()
        sep.append(dst.cpu().numpy())
    return act_np, sep[0], sep[1], ws


def swiglu_rows(g, u):
    """The oracle's ggml_vec_swiglu_f32 over each row of N."""
    N = g.shape[-1]
    g2 = np.ascontiguousarray(g.reshape(-1, N))
    u2 = np.ascontiguousarray(u.reshape(-1, N))
    y = np.empty_like(g2)
    for r in range(g2.shape[0]):
        oracle().qwo_swiglu(int(N), ptr(y[r]), ptr(g2[r]), ptr(u2[r]))
    return y.reshape(g.shape)


def oracle_act(gtype, qg, qu, b, ids, K, N, n_as):
    T, ne11, _ = b.shape
    n_ids = ids.shape[1]
    out = []
    for q in (qg, qu):
        exp = np.zeros((T, n_ids, N), np.float32)
        assert oracle().qwo_mul_mat_id(gtype, ptr(q), I64(K), I64(N), I64(n_as), ptr(b), I64(ne11), I64(T), ptr(ids),
                                       I64(n_ids), ptr(exp)) == 0
        out.append(exp)
    return swiglu_rows(out[0], out[1])


@pytest.mark.parametrize("gtype,K,N,n_as,n_ids,T,skew", [
    (GGML_Q4_K, 2048, 512, 64, 10, 64, 0.0),    # Qwen3-Next gate/up rows, uniform
    (GGML_Q4_K, 2048, 512, 64, 10, 40, 1.1),    # Zipf(1.1): uneven groups, experts without columns
    (GGML_Q4_K, 768, 128, 32, 4, 24, 0.0),      # K = 3 blocks, ragged 16-column tiles
    (GGML_Q4_K, 256, 64, 16, 2, 9, 0.0),        # smallest prefill: one block, one row tile
    (GGML_Q4_K, 2048, 512, 64, 10, 5, 0.0),     # T <= 8: the GEMV path, separate calls
    (GGML_Q8_0, 512, 256, 16, 4, 20, 0.0),      # Q8_0 past 8 columns: the grouped pass
    (GGML_Q8_0, 2048, 512, 64, 10, 64, 1.1),    # Q8_0 at the gate/up shape, Zipf(1.1)
    (GGML_Q4_K, 4096, 256, 16, 8, 24, 0.0),     # hidden 4096 (Qwen3-235B-A22B): K of 16 blocks
    (GGML_Q8_0, 3072, 128, 16, 4, 20, 0.5),     # hidden 3072
])
def test_swiglu_matches_oracle_and_separate_calls(dev, gtype, K, N, n_as, n_ids, T, skew):
    rng = np.random.default_rng(K + N + T + gtype)
    quant = quantize_q4_K if gtype == GGML_Q4_K else quantize_q8_0_model
    qg = quant((rng.standard_normal((n_as, N, K)) * 0.02).astype(np.float32))
    qu = quant((rng.standard_normal((n_as, N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, 1, K)).astype(np.float32)
    ids = zipf_ids(rng, T, n_ids, n_as, skew)
    act, g, u, _ = gpu_case(qg, qu, b, ids, K, N, n_as, gtype)
    assert np.isfinite(act).all(), "some outputs were not written"
    np.testing.assert_array_equal(act.view(np.uint32), swiglu_rows(g, u).view(np.uint32))
    exp = oracle_act(gtype, qg, qu, b, ids, K, N, n_as)
    err = rel_err(act, exp)
    print(f"swiglu type={gtype} K={K} N={N} T={T} skew={skew}: rel err vs oracle {err:.3e}")
    assert err < TOL


def random_q4k(n_as, N, K, seed):
    """Q4_K pools of random bytes with finite scales (d, dmin in [2^-10, 2^-8]):
    every such block is a valid Q4_K block, and the pools cost no CPU
    quantization at 512 experts."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = n_as * N * (K // 256)
    q = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device="cuda", generator=g)
    sc = (torch.rand((nb, 2), device="cuda", generator=g) * 3 + 1) * 2.0 ** -10
    q[:, :4] = sc.to(torch.float16).view(torch.uint8).reshape(nb, 4)
    return q.reshape(-1)


def test_swiglu_qwen3_next_full_size(dev):
    """512 experts x 512 rows x 2048, top-10 of 512 tokens (Zipf 0.8 routing),
    then 100 tokens on the same workspace: fused equals separate bit for bit."""
    K, N, n_as, n_ids = 2048, 512, 512, 10
    rng = np.random.default_rng(11)
    qg = random_q4k(n_as, N, K, 1)
    qu = random_q4k(n_as, N, K, 2)
    ws = None
    for T in (512, 100):
        b = rng.standard_normal((T, 1, K)).astype(np.float32)
        ids = zipf_ids(rng, T, n_ids, n_as, 0.8)
        act, g, u, ws = gpu_case(qg, qu, b, ids, K, N, n_as, ws=ws)
        assert np.isfinite(act).all()
        np.testing.assert_array_equal(act.view(np.uint32), swiglu_rows(g, u).view(np.uint32))
        print(f"qwen3-next T={T}: fused == separate over {act.size} outputs")



@pytest.mark.parametrize("N,rows", [(512, 37), (200, 9), (7, 3)])
def test_swiglu_node_matches_oracle(dev, N, rows):
    """qwm_swiglu (the GGML_GLU_OP_SWIGLU node alone): bit for bit against the
    oracle's ggml_vec_swiglu_f32 per row, 16-wide chunks and the scalar tail
    (N 200 and 7 have one), also with act written over gate."""
    rng = np.random.default_rng(N + rows)
    g = (rng.standard_normal((rows, N)) * 4).astype(np.float32)
    u = rng.standard_normal((rows, N)).astype(np.float32)
    exp = swiglu_rows(g, u)
    L = qa.lib()
    dg, du = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    act = torch.full((rows, N), float("nan"), dtype=torch.float32, device="cuda")
    tg, tu = qa.tensor(qa.TYPE_F32, N, rows, 1, dg), qa.tensor(qa.TYPE_F32, N, rows, 1, du)
    qa.check(L.qwm_swiglu(tg, tu, qa.tensor(qa.TYPE_F32, N, rows, 1, act), None))
    qa.check(L.qwm_swiglu(tg, tu, tg, None))                       # in place over gate
    torch.cuda.synchronize()
    np.testing.assert_array_equal(act.cpu().numpy().view(np.uint32), exp.view(np.uint32))
    np.testing.assert_array_equal(dg.cpu().numpy().view(np.uint32), exp.view(np.uint32))
    assert L.qwm_swiglu(tg, qa.tensor(qa.TYPE_F32, N, rows + 1, 1, du), tg, None) == qa.ERR_ARG
