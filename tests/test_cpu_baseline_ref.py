"""The CPU baselines that bench.py times beside the GPU (oracle/_ref, built
from the reference's own ggml-CPU kernels) compute the same results as the
oracle: the MoE block (decode and miss-fill baselines) and MUL_MAT_ID (the
prefill baseline).  CPU only; needs oracle/_ref."""
import ctypes

import numpy as np
import pytest

from tests.helpers import GGML_Q4_K, I64, oracle, ptr, quantize_q4_K, ref
from tests.moe_case import MoeCase, rel_err

pytestmark = pytest.mark.ref
P = ctypes.c_void_p


class BlockArgs(ctypes.Structure):
    _fields_ = [("H", ctypes.c_int64), ("N", ctypes.c_int64), ("E", ctypes.c_int64), ("k", ctypes.c_int64),
                ("T", ctypes.c_int64), ("router", P), ("rm", P), ("gate", P), ("up", P), ("down", P),
                ("sh_gate", P), ("sh_up", P), ("sh_down", P), ("sh_inp", P), ("x", P), ("out", P), ("ids", P),
                ("n_threads", ctypes.c_int)]


def cpu_block(c, x, rm=None):
    T = x.shape[0]
    a = BlockArgs()
    a.H, a.N, a.E, a.k, a.T = c.H, c.N, c.E, c.k, T
    a.router, a.rm = c.router.ctypes.data, (rm.ctypes.data if rm is not None else None)
    a.gate, a.up, a.down = c.gate_q.ctypes.data, c.up_q.ctypes.data, c.down_q.ctypes.data
    if c.shared:
        a.sh_gate, a.sh_up, a.sh_down = c.shg_q.ctypes.data, c.shu_q.ctypes.data, c.shd_q.ctypes.data
        a.sh_inp = c.sh_inp.ctypes.data if c.sh_inp is not None else None
    out = np.zeros((T, c.H), np.float32)
    ids = np.zeros((T, c.k), np.int32)
    a.x, a.out, a.ids, a.n_threads = x.ctypes.data, out.ctypes.data, ids.ctypes.data, 4
    lib = ref()
    lib.qwr_cpu_moe_block.argtypes = [ctypes.POINTER(BlockArgs)]
    assert lib.qwr_cpu_moe_block(ctypes.byref(a)) == 0
    return out, ids


@pytest.mark.parametrize("T,shared,mask", [(1, False, False), (1, True, True), (4, True, True), (4, False, False)])
def test_cpu_moe_block_matches_oracle(T, shared, mask):
    c = MoeCase(seed=21 + T, H=512, N=256, E=16, k=4, S=16, shared=shared, N_sh=256)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, c.H)).astype(np.float32)
    rm = (rng.standard_normal((T, c.E)) * 0.5).astype(np.float32) if mask else None
    got, ids = cpu_block(c, x, rm)
    eids, w, _, _ = c.route(x, rm)
    assert np.array_equal(ids, eids)
    exp = c.block(x, eids, w) + x
    assert rel_err(got, exp) < 1e-5


def test_cpu_mul_mat_id_matches_oracle():
    rng = np.random.default_rng(4)
    K, N, n_as, n_ids, ne11, T = 512, 64, 8, 3, 1, 20
    q = quantize_q4_K((rng.standard_normal((n_as, N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, ne11, K)).astype(np.float32)
    ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
    got = np.zeros((T, n_ids, N), np.float32)
    lib = ref()
    lib.qwr_cpu_mul_mat_id.argtypes = [P, I64, I64, I64, P, I64, I64, P, I64, P, ctypes.c_int]
    assert lib.qwr_cpu_mul_mat_id(ptr(q), K, N, n_as, ptr(b), ne11, T, ptr(ids), n_ids, ptr(got), 4) == 0
    exp = np.zeros_like(got)
    assert oracle().qwo_mul_mat_id(GGML_Q4_K, ptr(q), I64(K), I64(N), I64(n_as), ptr(b), I64(ne11), I64(T),
                                   ptr(ids), I64(n_ids), ptr(exp)) == 0
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
