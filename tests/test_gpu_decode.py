"""GPU parity of the decode loop over stacked MoE blocks (qwm_moe_decode:
x = x + MoE_l(x) for every layer, slots remapped on the device from per-layer
tables) against the oracle applied layer by layer (bit for bit, Q4_K and Q8_0
slabs), and bit for bit against the same layers through
qwm_moe_block_resident one call at a time."""
import numpy as np
import pytest

from tests.moe_case import MoeCase, rel_err

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


@pytest.mark.parametrize("T,n_layers,wtype,H,N", [(1, 4, "q4_K", 512, 256), (4, 5, "q4_K", 512, 256),
                                                  (2, 3, "q8_0", 512, 256),
                                                  (1, 2, "q4_K", 4096, 512), (3, 2, "q8_0", 3072, 256)])
def test_decode_layers(dev, T, n_layers, wtype, H, N):
    """Hidden sizes 3072 and 4096 take the per-layer launches (the persistent
    decode is built for 2048)."""
    E, k = 16, 4
    cases = [MoeCase(seed=100 + l, H=H, N=N, E=E, k=k, S=E, wtype=wtype) for l in range(n_layers)]
    rng = np.random.default_rng(7)
    perms = [rng.permutation(E).astype(np.int32) for _ in range(n_layers)]   # expert -> slot, per layer
    tables = np.zeros((3, n_layers * E), np.int32)
    for l in range(n_layers):
        tables[:, l * E:(l + 1) * E] = perms[l]
    layers = (qa.MoeLayer * n_layers)()
    for l, c in enumerate(cases):
        layers[l] = c.upload(torch)
    x0 = rng.standard_normal((T, H)).astype(np.float32)

    # oracle, layer by layer
    x = x0.copy()
    for l, c in enumerate(cases):
        ids, w, _, _ = c.route(x)
        x = c.block(x, perms[l][ids], w) + x
    exp = x

    dtab = torch.from_numpy(tables).cuda()
    L = qa.lib()
    dx = torch.from_numpy(x0).cuda()
    ws = workspace(L.qwm_moe_decode_workspace_size(layers, n_layers, T))
    qa.check(L.qwm_moe_decode(layers, n_layers, dtab.data_ptr(), n_layers * E, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                              ws.data_ptr(), ws.numel(), None))
    # the same layers one block at a time
    wsb = workspace(L.qwm_moe_workspace_size(layers[0], T))
    a = torch.from_numpy(x0).cuda()
    for l in range(n_layers):
        b = torch.zeros_like(a)
        ta, tb = qa.tensor(qa.TYPE_F32, H, T, 1, a), qa.tensor(qa.TYPE_F32, H, T, 1, b)
        qa.check(L.qwm_moe_block_resident(layers[l], l, dtab.data_ptr(), n_layers * E, ta, None, ta, tb, None, None,
                                          wsb.data_ptr(), wsb.numel(), None))
        a = b
    torch.cuda.synchronize()
    got = dx.cpu().numpy()
    err = rel_err(got, exp)
    print(f"decode T={T} layers={n_layers} {wtype} H={H}: rel err {err:.3e}")
    assert err < TOL
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), f"{wtype} decode loop not bit-exact"
    assert np.array_equal(got.view(np.uint32), a.cpu().numpy().view(np.uint32)), "loop and per-block calls differ"


def test_decode_rejects_mixed_shapes(dev):
    a = MoeCase(seed=1, H=512, N=256, E=16, k=4, S=16)
    b = MoeCase(seed=2, H=512, N=512, E=16, k=4, S=16)
    layers = (qa.MoeLayer * 2)()
    layers[0] = a.upload(torch)
    layers[1] = b.upload(torch)
    assert qa.lib().qwm_moe_decode_workspace_size(layers, 2, 1) == 0


@pytest.mark.parametrize("T,n_layers", [(1, 3), (4, 4)])
def test_decode_graph_replay(dev, T, n_layers):
    """The decode loop captured into a HIP graph (through torch.cuda.graph)
    and replayed three times, with eager work and synchronizations between
    the replays: every replay equals the eager loop on the same input bit for
    bit (the kernels re-arm their own counters; the loop records no memset)."""
    H, N, E, k = 512, 256, 16, 4
    cases = [MoeCase(seed=300 + l, H=H, N=N, E=E, k=k, S=E) for l in range(n_layers)]
    rng = np.random.default_rng(11)
    tables = np.zeros((3, n_layers * E), np.int32)
    for l in range(n_layers):
        tables[:, l * E:(l + 1) * E] = rng.permutation(E).astype(np.int32)
    layers = (qa.MoeLayer * n_layers)()
    for l, c in enumerate(cases):
        layers[l] = c.upload(torch)
    L = qa.lib()
    dtab = torch.from_numpy(tables).cuda()
    nbytes = L.qwm_moe_decode_workspace_size(layers, n_layers, T)
    ws_e, ws_g = workspace(nbytes), workspace(nbytes)
    xs = [rng.standard_normal((T, H)).astype(np.float32) for _ in range(3)]

    def eager(x0):
        dx = torch.from_numpy(x0).cuda()
        qa.check(L.qwm_moe_decode(layers, n_layers, dtab.data_ptr(), n_layers * E, qa.tensor(qa.TYPE_F32, H, T, 1, dx),
                                  ws_e.data_ptr(), ws_e.numel(), None))
        torch.cuda.synchronize()
        return dx.cpu().numpy()

    gx = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qa.check(L.qwm_moe_decode(layers, n_layers, dtab.data_ptr(), n_layers * E, qa.tensor(qa.TYPE_F32, H, T, 1, gx),
                                  ws_g.data_ptr(), ws_g.numel(), torch.cuda.current_stream().cuda_stream))
    for rep, x0 in enumerate(xs):
        exp = eager(x0)
        gx.copy_(torch.from_numpy(x0).cuda())
        graph.replay()
        torch.cuda.synchronize()
        got = gx.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), f"replay {rep} differs from the eager loop"


@pytest.mark.parametrize("T", [1, 2])
def test_decode_sel_record_and_miss_flag(dev, T):
    """qwm_moe_decode_sel keeps every layer's selected experts (the fast
    path's sel_all, runtime.cpp:2759-2766) and raises the miss flag exactly
    when a selected expert's residency bit is clear (6155-6166): all bits set
    -> flag 0, ids equal to the oracle's layer by layer and x bit-exact; the
    bit of one expert that layer 1 selects cleared -> flag 1; the bit of an
    expert no layer selects cleared -> flag 0."""
    H, N, E, k, n_layers = 512, 256, 40, 4, 3
    cases = [MoeCase(seed=500 + l, H=H, N=N, E=E, k=k, S=E) for l in range(n_layers)]
    rng = np.random.default_rng(23 + T)
    perms = [rng.permutation(E).astype(np.int32) for _ in range(n_layers)]
    tables = np.zeros((3, n_layers * E), np.int32)
    for l in range(n_layers):
        tables[:, l * E:(l + 1) * E] = perms[l]
    layers = (qa.MoeLayer * n_layers)()
    for l, c in enumerate(cases):
        layers[l] = c.upload(torch)
    x0 = rng.standard_normal((T, H)).astype(np.float32)
    x = x0.copy()
    ids_ref = []
    for l, c in enumerate(cases):
        ids, w, _, _ = c.route(x)
        ids_ref.append(ids)
        x = c.block(x, perms[l][ids], w) + x
    L = qa.lib()
    dtab = torch.from_numpy(tables).cuda()
    ws = workspace(L.qwm_moe_decode_workspace_size(layers, n_layers, T))
    words = (E + 31) // 32
    used = set(int(e) for i in ids_ref for e in i.ravel())
    unused = [e for e in range(E) if e not in used]
    assert unused

    def run(bits):
        dx = torch.from_numpy(x0).cuda()
        dids = torch.full((n_layers, T, k), -7, dtype=torch.int32, device="cuda")
        dbits = torch.from_numpy(bits.view(np.int32)).cuda()
        flag = torch.full((1,), 5, dtype=torch.int32, device="cuda")
        qa.check(L.qwm_moe_decode_sel(layers, n_layers, dtab.data_ptr(), n_layers * E,
                                      qa.tensor(qa.TYPE_F32, H, T, 1, dx), dids.data_ptr(), dbits.data_ptr(),
                                      flag.data_ptr(), ws.data_ptr(), ws.numel(), None))
        torch.cuda.synchronize()
        return dx.cpu().numpy(), dids.cpu().numpy(), int(flag.cpu().numpy()[0])

    full = np.zeros((n_layers, words), np.uint32)
    for l in range(n_layers):
        for e in range(E):
            full[l, e >> 5] |= np.uint32(1 << (e & 31))
    got, gids, flag = run(full)
    print(f"decode_sel T={T}: flag {flag}", flush=True)
    assert flag == 0
    for l in range(n_layers):
        assert np.array_equal(gids[l], ids_ref[l]), f"layer {l}: recorded ids differ"
    assert np.array_equal(got.view(np.uint32), x.view(np.uint32))
    miss = full.copy()
    e1 = int(ids_ref[1][0, 0])
    miss[1, e1 >> 5] &= np.uint32(~(1 << (e1 & 31)) & 0xFFFFFFFF)
    _, gids, flag = run(miss)
    assert flag == 1 and np.array_equal(gids[1], ids_ref[1])
    other = full.copy()
    eu = unused[0]
    other[2, eu >> 5] &= np.uint32(~(1 << (eu & 31)) & 0xFFFFFFFF)
    _, _, flag = run(other)
    assert flag == 0
