"""The GGUF tensor index (qwm_gguf_find_tensor, qwm_pool_attach_gguf) on
files written by tests/gguf_file.py: offsets, shapes, types and sizes of the
tensors, every key/value type skipped correctly, the alignment key honoured,
and malformed files refused.  CPU only."""
import ctypes

import numpy as np
import pytest

import questwend_amd as qa
from tests.gguf_file import (GGML_F32, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, T_ARR, T_BOOL, T_F32, T_F64, T_I8, T_I16,
                             T_I32, T_I64, T_STR, T_U8, T_U16, T_U32, T_U64, write_gguf)

KVS = [("general.architecture", T_STR, "qwen3moe"), ("a.u8", T_U8, 7), ("a.i8", T_I8, -7), ("a.u16", T_U16, 700),
       ("a.i16", T_I16, -700), ("a.u32", T_U32, 70000), ("a.i32", T_I32, -70000), ("a.f32", T_F32, 0.5),
       ("a.bool", T_BOOL, True), ("a.u64", T_U64, 1 << 40), ("a.i64", T_I64, -(1 << 40)), ("a.f64", T_F64, 0.25),
       ("a.arr_u32", T_ARR, (T_U32, [1, 2, 3])), ("tokenizer.tokens", T_ARR, (T_STR, ["a", "bc", "", "def"])),
       ("a.empty", T_ARR, (T_I16, []))]


def find(path, name):
    t = qa.GgufTensor()
    rc = qa.lib().qwm_gguf_find_tensor(str(path).encode(), name.encode(), ctypes.byref(t))
    return rc, t


def expert_tensors(rng, n_block, E, K, N, gtype=GGML_Q4_K):
    per = {GGML_Q4_K: K // 256 * 144, GGML_Q6_K: K // 256 * 210, GGML_Q8_0: K // 32 * 34}[gtype]
    out = []
    for b in range(n_block):
        for role in ("gate", "up", "down"):
            kk, nn = (K, N) if role != "down" else (N, K)
            row = {GGML_Q4_K: kk // 256 * 144, GGML_Q6_K: kk // 256 * 210, GGML_Q8_0: kk // 32 * 34}[gtype]
            data = rng.integers(0, 256, E * nn * row, dtype=np.uint8).tobytes()
            out.append((f"blk.{b}.ffn_{role}_exps.weight", gtype, [kk, nn, E], data))
    assert per > 0
    return out


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_find_tensor_offsets_shapes_sizes(tmp_path, alignment):
    rng = np.random.default_rng(3)
    ts = [("token_embd.weight", GGML_Q8_0, [512, 10], rng.integers(0, 256, 10 * 16 * 34, dtype=np.uint8).tobytes()),
          ("output_norm.weight", GGML_F32, [512], rng.integers(0, 256, 2048, dtype=np.uint8).tobytes()),
          ("blk.0.attn_v.weight", GGML_Q6_K, [512, 64], rng.integers(0, 256, 64 * 2 * 210, dtype=np.uint8).tobytes())]
    ts += expert_tensors(rng, 2, 4, 512, 256)
    path = tmp_path / "m.gguf"
    offs = write_gguf(str(path), KVS, ts, alignment)
    blob = path.read_bytes()
    for name, gtype, ne, data in ts:
        rc, t = find(path, name)
        assert rc == qa.OK, qa.lib().qwm_last_error()
        assert t.offset == offs[name] and t.offset % (alignment or 32) == 0
        assert (t.type, t.n_dims) == (gtype, len(ne))
        assert list(t.ne) == list(ne) + [1] * (4 - len(ne))
        assert t.nbytes == len(data)
        assert blob[t.offset:t.offset + t.nbytes] == data


def test_find_tensor_errors(tmp_path):
    rng = np.random.default_rng(4)
    ts = expert_tensors(rng, 1, 2, 256, 256)
    good = tmp_path / "good.gguf"
    write_gguf(str(good), KVS, ts)
    blob = good.read_bytes()
    L = qa.lib()
    assert find(tmp_path / "missing.gguf", ts[0][0])[0] == qa.ERR_IO
    assert find(good, "blk.7.ffn_gate_exps.weight")[0] == qa.ERR_ARG
    assert b"no tensor blk.7" in L.qwm_last_error()
    cases = {"magic.gguf": b"GGUX" + blob[4:], "v1.gguf": blob[:4] + (1).to_bytes(4, "little") + blob[8:],
             "cut.gguf": blob[:200]}
    for name, data in cases.items():
        (tmp_path / name).write_bytes(data)
        assert find(tmp_path / name, ts[0][0])[0] == qa.ERR_ARG, name
    nested = tmp_path / "nested.gguf"
    write_gguf(str(nested), [("x", T_ARR, (T_ARR, []))], ts)
    assert find(nested, ts[0][0])[0] == qa.ERR_ARG
    odd = tmp_path / "odd.gguf"
    write_gguf(str(odd), KVS, ts, alignment=48)
    assert find(odd, ts[0][0])[0] == qa.ERR_ARG
    assert b"power-of-two" in L.qwm_last_error()


def test_pool_attach_gguf_checks_shapes(tmp_path):
    """qwm_pool_attach_gguf takes blk.<first_block + l> for the pool's layers
    and refuses tensors that do not hold n_expert slabs of slab_bytes."""
    rng = np.random.default_rng(5)
    E, K, N = 4, 512, 256
    path = tmp_path / "m.gguf"
    write_gguf(str(path), KVS, expert_tensors(rng, 3, E, K, N))
    L = qa.lib()

    def pool(n_layer, n_expert, slab):
        d = qa.PoolDesc()
        d.n_layer, d.n_expert = n_layer, n_expert
        for r in range(3):
            d.n_slots[r], d.pool_data[r], d.slab_bytes[r] = 2, 4096, slab   # device memory never touched
        h = ctypes.c_void_p()
        qa.check(L.qwm_pool_create(ctypes.byref(d), None, ctypes.byref(h)))
        return h

    slab = N * K // 256 * 144
    for n_layer, first, n_expert, sl, want in [(2, 1, E, slab, qa.OK), (3, 0, E, slab, qa.OK),
                                               (2, 2, E, slab, qa.ERR_ARG), (1, 0, E + 1, slab, qa.ERR_ARG),
                                               (1, 0, E, slab + 16, qa.ERR_ARG)]:
        h = pool(n_layer, n_expert, sl)
        try:
            assert L.qwm_pool_attach_gguf(h, str(path).encode(), first) == want, (n_layer, first, n_expert, sl)
        finally:
            L.qwm_pool_destroy(h)
