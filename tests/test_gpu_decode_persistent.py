"""GPU parity of the persistent decode loop (qwm_moe_decode / _sel at one
token and hidden size 2048 run every layer in one launch per group of 16
layers, qwm_decode.hip) against the oracle applied layer by layer and
against the per-op kernels (qwm_moe_block_resident one layer at a time), bit
for bit: 1, 3 and 17 layers (two launches) of the Qwen3-30B-A3B shape over
one shared pool per role with per-layer permuted slot tables; two
Qwen3-Next-shape layers (512 experts, shared expert, top-10) with sigmoid
gating and a ranking bias on one and a Q6_K down pool on the other; the
selection record and the miss flag; HIP graph replay; and the bounded waits'
give-up path forced by a spin limit of 0 (a = -1 from the fused step, bit 1
of the decode miss flag; every kernel exits, and the next call on the same
workspace is bit-exact)."""
import ctypes

import numpy as np
import pytest

from tests.helpers import bits
from tests.moe_case import MoeCase, rel_err

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from tests.test_gpu_configs import H, Block, resident_pools, workspace  # noqa: E402
from tests.test_gpu_verify import oracle_verify  # noqa: E402

pytestmark = pytest.mark.gpu
E, N, K = 128, 768, 8
DEFAULT_SPIN = 1 << 21


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def pools(dev):
    return resident_pools(E, N, 900)


def stack(n_layers, seed, d_pools):
    blks = [Block(seed + l, E, N, K, E) for l in range(n_layers)]
    rng = np.random.default_rng(seed)
    perms = rng.permuted(np.tile(np.arange(E, dtype=np.int32), (n_layers, 3, 1)), axis=2)   # [layer][role][expert]
    tables = np.ascontiguousarray(perms.transpose(1, 0, 2).reshape(3, n_layers * E)).astype(np.int32)
    layers = (qa.MoeLayer * n_layers)()
    for l, b in enumerate(blks):
        layers[l] = b.layer(d_pools)
    return blks, perms, tables, layers, rng


def oracle_chain(blks, perms, h_pools, x0):
    x, ids_all = x0.copy(), []
    for l, b in enumerate(blks):
        ids, w, _ = b.route(x)
        ids_all.append(ids)
        x = b.block(x, h_pools, E, [perms[l, r][ids] for r in range(3)], w) + x
    return x, ids_all


def per_op_chain(layers, n_layers, dtab, stride, x0):
    L = qa.lib()
    ws = workspace(L.qwm_moe_workspace_size(layers[0], 1))
    a = torch.from_numpy(x0).cuda()
    for l in range(n_layers):
        b = torch.zeros_like(a)
        ta, tb = qa.tensor(qa.TYPE_F32, H, 1, 1, a), qa.tensor(qa.TYPE_F32, H, 1, 1, b)
        qa.check(L.qwm_moe_block_resident(layers[l], l, dtab.data_ptr(), stride, ta, None, ta, tb, None, None,
                                          ws.data_ptr(), ws.numel(), None))
        a = b
    torch.cuda.synchronize()
    return a.cpu().numpy()


@pytest.mark.parametrize("n_layers", [1, 3, 17])
def test_persistent_decode_bit_exact(dev, pools, n_layers):
    d_pools, h_pools = pools
    blks, perms, tables, layers, rng = stack(n_layers, 910 + n_layers, d_pools)
    L = qa.lib()
    dtab = torch.from_numpy(tables).cuda()
    ws = workspace(L.qwm_moe_decode_workspace_size(layers, n_layers, 1))
    for tok in range(2):
        x0 = rng.standard_normal((1, H)).astype(np.float32)
        exp, _ = oracle_chain(blks, perms, h_pools, x0)
        dx = torch.from_numpy(x0).cuda()
        print(f"persistent decode {n_layers} layers: token {tok}", flush=True)
        qa.check(L.qwm_moe_decode(layers, n_layers, dtab.data_ptr(), n_layers * E, qa.tensor(qa.TYPE_F32, H, 1, 1, dx),
                                  ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        got = dx.cpu().numpy()
        print(f"  rel err {rel_err(got, exp):.3e}", flush=True)
        assert np.array_equal(bits(got), bits(exp)), "persistent decode differs from the oracle"
        if tok == 0:
            per_op = per_op_chain(layers, n_layers, dtab, n_layers * E, x0)
            assert np.array_equal(bits(got), bits(per_op)), "persistent decode differs from the per-op kernels"


def test_persistent_decode_qwen3next_layers(dev):
    """Two Qwen3-Next-shape layers through their own 40-slot pools (several
    experts per slot): layer 0 with sigmoid gating and an exp_probs_b
    ranking bias, layer 1 with Q6_K down slabs (routed and shared)."""
    cases = [MoeCase(seed=950, H=H, N=512, E=512, k=10, S=40, shared=True, N_sh=512, gating=2, bias=0.05),
             MoeCase(seed=951, H=H, N=512, E=512, k=10, S=40, shared=True, N_sh=512, down="q6_K")]
    rng = np.random.default_rng(952)
    maps = [(rng.permutation(512) % 40).astype(np.int32) for _ in cases]   # expert -> slot, all roles
    tables = np.zeros((3, 2 * 512), np.int32)
    for l in range(2):
        tables[:, l * 512:(l + 1) * 512] = maps[l]
    layers = (qa.MoeLayer * 2)()
    for l, c in enumerate(cases):
        layers[l] = c.upload(torch)
    L = qa.lib()
    dtab = torch.from_numpy(tables).cuda()
    ws = workspace(L.qwm_moe_decode_workspace_size(layers, 2, 1))
    for tok in range(2):
        x0 = rng.standard_normal((1, H)).astype(np.float32)
        x = x0.copy()
        for l, c in enumerate(cases):
            ids, w, _, _ = c.route(x)
            x = c.block(x, maps[l][ids], w) + x
        dx = torch.from_numpy(x0).cuda()
        print(f"persistent decode, Qwen3-Next layers: token {tok}", flush=True)
        qa.check(L.qwm_moe_decode(layers, 2, dtab.data_ptr(), 2 * 512, qa.tensor(qa.TYPE_F32, H, 1, 1, dx),
                                  ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        got = dx.cpu().numpy()
        print(f"  rel err {rel_err(got, x):.3e}", flush=True)
        assert np.array_equal(bits(got), bits(x))


def test_persistent_decode_sel_and_graph(dev, pools):
    """The selection record and the miss flag on the persistent path, then
    the call captured in a HIP graph and replayed three times with eager
    work between the replays, each replay bit-exact."""
    d_pools, h_pools = pools
    n_layers = 3
    blks, perms, tables, layers, rng = stack(n_layers, 970, d_pools)
    L = qa.lib()
    dtab = torch.from_numpy(tables).cuda()
    ws = workspace(L.qwm_moe_decode_workspace_size(layers, n_layers, 1))
    words = (E + 31) // 32
    x0 = rng.standard_normal((1, H)).astype(np.float32)
    exp, ids_ref = oracle_chain(blks, perms, h_pools, x0)

    def run(bitmap, x_in):
        dx = torch.from_numpy(x_in).cuda()
        dids = torch.full((n_layers, 1, K), -7, dtype=torch.int32, device="cuda")
        dbits = torch.from_numpy(bitmap.view(np.int32)).cuda()
        flag = torch.full((1,), 5, dtype=torch.int32, device="cuda")
        qa.check(L.qwm_moe_decode_sel(layers, n_layers, dtab.data_ptr(), n_layers * E,
                                      qa.tensor(qa.TYPE_F32, H, 1, 1, dx), dids.data_ptr(), dbits.data_ptr(),
                                      flag.data_ptr(), ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        return dx.cpu().numpy(), dids.cpu().numpy(), int(flag.cpu().numpy()[0])

    full = np.full((n_layers, words), 0xFFFFFFFF, np.uint32)
    got, gids, flag = run(full, x0)
    assert flag == 0 and np.array_equal(bits(got), bits(exp))
    for l in range(n_layers):
        assert np.array_equal(gids[l], ids_ref[l]), f"layer {l}: recorded ids differ"
    miss = full.copy()
    e1 = int(ids_ref[1][0, 0])
    miss[1, e1 >> 5] &= np.uint32(~(1 << (e1 & 31)) & 0xFFFFFFFF)
    assert run(miss, x0)[2] == 1
    used = set(int(e) for i in ids_ref for e in i.ravel())
    eu = next(e for e in range(E) if e not in used)
    other = full.copy()
    other[2, eu >> 5] &= np.uint32(~(1 << (eu & 31)) & 0xFFFFFFFF)
    assert run(other, x0)[2] == 0

    # graph replay
    wsg = workspace(L.qwm_moe_decode_workspace_size(layers, n_layers, 1))
    gx = torch.zeros((1, H), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qa.check(L.qwm_moe_decode(layers, n_layers, dtab.data_ptr(), n_layers * E, qa.tensor(qa.TYPE_F32, H, 1, 1, gx),
                                  wsg.data_ptr(), wsg.numel(), torch.cuda.current_stream().cuda_stream))
    for rep in range(3):
        xi = rng.standard_normal((1, H)).astype(np.float32)
        eager = run(full, xi)[0]
        gx.copy_(torch.from_numpy(xi).cuda())
        graph.replay()
        torch.cuda.synchronize()
        print(f"persistent decode graph replay {rep}", flush=True)
        assert np.array_equal(bits(gx.cpu().numpy()), bits(eager)), f"replay {rep} differs from the eager call"


def test_spin_limit_zero_gives_up_and_recovers(dev, pools):
    """A spin limit of 0 makes the persistent launches' waits give up: the
    fused step reports a = x_new = -1, the decode sets bit 1 of its miss
    flag, and every kernel exits.  Back at the default bound, the next call
    on the same workspace is bit-exact."""
    d_pools, h_pools = pools
    L = qa.lib()
    T, V = 4, 16384
    blk = Block(980, E, N, K, E)
    perms = [blk.rng.permutation(E).astype(np.int32) for _ in range(3)]
    layer = blk.layer(d_pools)
    rng = np.random.default_rng(981)
    Wd = (rng.standard_normal((V, H)) / np.sqrt(H)).astype(np.float32)
    from tests.helpers import quantize_q8_0_model
    Wq = quantize_q8_0_model(Wd)
    dW = torch.from_numpy(Wq).cuda()
    lm_t = qa.tensor(qa.TYPE_Q8_0, H, V, 1, dW)
    dtab = torch.from_numpy(np.concatenate(perms).astype(np.int32)).cuda()
    norm_w = np.ones(H, np.float32)
    dn = torch.from_numpy(norm_w).cuda()
    ws = workspace(L.qwm_verify_step_workspace_size(layer, lm_t, T))
    x = blk.rng.standard_normal((T, H)).astype(np.float32)
    ids, w, _ = blk.route(x)
    out_ref = blk.block(x, h_pools, E, [perms[r][ids] for r in range(3)], w) + x
    drafts = np.zeros(T - 1, np.int32)
    vA, a_ref, xn_ref, margins = oracle_verify(Wq, H, V, out_ref, norm_w, 1e-6, drafts)
    dx = torch.from_numpy(x).cuda()
    ddr = torch.from_numpy(drafts).cuda()
    xt = qa.tensor(qa.TYPE_F32, H, T, 1, dx)

    def step():
        out = torch.zeros((T, H), device="cuda")
        r = torch.zeros(T + 2, dtype=torch.int32, device="cuda")
        qa.check(L.qwm_verify_step(layer, 0, dtab.data_ptr(), E, xt, None, xt, qa.tensor(qa.TYPE_F32, H, T, 1, out),
                                   None, None, lm_t, dn.data_ptr(), 1e-6, ddr.data_ptr(), r.data_ptr(), ws.data_ptr(),
                                   ws.numel(), None))
        torch.cuda.synchronize()
        return out.cpu().numpy(), r.cpu().numpy()

    blks, dperms, tables, layers, drng = stack(3, 985, d_pools)
    dtab3 = torch.from_numpy(tables).cuda()
    wsd = workspace(L.qwm_moe_decode_workspace_size(layers, 3, 1))
    x0 = drng.standard_normal((1, H)).astype(np.float32)
    dexp, _ = oracle_chain(blks, dperms, h_pools, x0)

    def decode():
        dxx = torch.from_numpy(x0).cuda()
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        full = torch.full((3, (E + 31) // 32), -1, dtype=torch.int32, device="cuda")
        qa.check(L.qwm_moe_decode_sel(layers, 3, dtab3.data_ptr(), 3 * E, qa.tensor(qa.TYPE_F32, H, 1, 1, dxx), None,
                                      full.data_ptr(), flag.data_ptr(), wsd.data_ptr(), wsd.numel(), None))
        torch.cuda.synchronize()
        return dxx.cpu().numpy(), int(flag.cpu().numpy()[0])

    try:
        qa.check(L.qwm_set_spin_limit(0))
        print("spin limit 0: fused step", flush=True)
        _, r0 = step()
        assert r0[T] == -1 and r0[T + 1] == -1, r0
        print("spin limit 0: decode", flush=True)
        _, f0 = decode()
        assert f0 & 2, f0
    finally:
        qa.check(L.qwm_set_spin_limit(DEFAULT_SPIN))
    print("default spin limit: fused step and decode again", flush=True)
    out1, r1 = step()
    assert r1[T] >= 0
    assert np.array_equal(bits(out1), bits(out_ref)), "the step after a give-up is not bit-exact"
    clear = margins > 1e-3
    assert np.array_equal(r1[:T][clear], vA[clear])
    x1, f1 = decode()
    assert f1 == 0 and np.array_equal(bits(x1), bits(dexp)), "the decode after a give-up is not bit-exact"
