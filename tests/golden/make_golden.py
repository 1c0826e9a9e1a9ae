"""Writes tests/golden/ref_vectors.npz: input/output vectors of the reference's
own CPU kernels for this path, so the oracle can be pinned where the
reference build (oracle/_ref, compiled from the unmodified ggml sources and
core/gpu_lru_index.h by oracle/Makefile) is not available.

Run from the repository root after `make -C oracle all ref`:
    python tests/golden/make_golden.py

Every array is plain numeric data (numpy .npz, no pickles).  Float results are
stored as their bit patterns (uint32) so the test can demand bit equality.
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.helpers import (I64, Q4K_BYTES, Q8K_BYTES, Q80_BYTES, oracle, ptr, ref, ref_available,  # noqa: E402
                           ref_lru)

OUT = os.path.join(HERE, "ref_vectors.npz")


def f32bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def main():
    if not ref_available():
        raise SystemExit("oracle/_ref is not built (make -C oracle ref)")
    R = ref()
    rng = np.random.default_rng(20260901)
    g = {}

    # Q4_K quantizer (ggml-quants.c:1458-1528): four scales plus edge blocks
    x = np.concatenate([rng.standard_normal((8, 256)) * s for s in (0.02, 1.0, 1e-3, 30.0)]).astype(np.float32)
    x[0] = 0                                   # all-zero block
    x[1] = np.abs(x[1])                        # all-positive block (min clamps to 0)
    x[2, 32:64] = x[2, 32]                     # constant sub-block
    x[3, :100] = 0                             # partially zero block
    q = np.zeros(x.shape[0] * Q4K_BYTES, np.uint8)
    R.qwr_quantize_q4_K(ptr(x), ptr(q), I64(x.size))
    g["q4k_x"], g["q4k_q"] = x, q

    # Q8_K activation quantizer (ggml-quants.c:2769-2806 via arch/x86/quants.c:505)
    x = (rng.standard_normal((6, 256)) * np.array([1.0, 1e-4, 300.0, 1.0, 1.0, 1.0])[:, None]).astype(np.float32)
    x[3] = 0
    x[4] = -np.abs(x[4])                       # negative max
    x[5, 7] = x[5, 9] = -50.0                  # first of two equal |max| wins
    q = np.zeros(6 * Q8K_BYTES, np.uint8)
    R.qwr_quantize_q8_K(ptr(x), ptr(q), I64(x.size))
    g["q8k_x"], g["q8k_q"] = x, q

    # Q8_0 quantizers: x86 activation path (arch/x86/quants.c:302-345) and the
    # model-file reference (ggml-quants.c:276-300)
    x = rng.standard_normal((16, 32)).astype(np.float32)
    x[0] = 0
    x[1] = np.arange(32) - 15.5                # .5 ties after scaling
    qa = np.zeros(16 * Q80_BYTES, np.uint8)
    qr = np.zeros_like(qa)
    R.qwr_quantize_q8_0(ptr(x), ptr(qa), I64(x.size))
    R.qwr_quantize_q8_0_ref(ptr(x), ptr(qr), I64(x.size))
    g["q80_x"], g["q80_x86"], g["q80_ref"] = x, qa, qr

    # Q4_K x Q8_K dot (arch/x86/quants.c:2102-2170), K = 768 and 2048
    for K in (768, 2048):
        w = (rng.standard_normal((6, K)) * 0.02).astype(np.float32)
        a = rng.standard_normal((6, K)).astype(np.float32)
        wq = np.zeros(6 * K // 256 * Q4K_BYTES, np.uint8)
        aq = np.zeros(6 * K // 256 * Q8K_BYTES, np.uint8)
        R.qwr_quantize_q4_K(ptr(w), ptr(wq), I64(w.size))
        R.qwr_quantize_q8_K(ptr(a), ptr(aq), I64(a.size))
        rb, ab = K // 256 * Q4K_BYTES, K // 256 * Q8K_BYTES
        s = np.array([R.qwr_vec_dot_q4_K_q8_K(K, ptr(wq[i * rb:]), ptr(aq[i * ab:])) for i in range(6)], np.float32)
        g[f"dq4k{K}_w"], g[f"dq4k{K}_a"], g[f"dq4k{K}_s"] = wq, aq, f32bits(s)

    # Q8_0 x Q8_0 dot (the lm_head path), K = 2048
    K = 2048
    w = rng.standard_normal((4, K)).astype(np.float32)
    a = rng.standard_normal((4, K)).astype(np.float32)
    wq = np.zeros(4 * K // 32 * Q80_BYTES, np.uint8)
    aq = np.zeros_like(wq)
    R.qwr_quantize_q8_0_ref(ptr(w), ptr(wq), I64(w.size))
    R.qwr_quantize_q8_0(ptr(a), ptr(aq), I64(a.size))
    rb = K // 32 * Q80_BYTES
    s = np.array([R.qwr_vec_dot_q8_0_q8_0(K, ptr(wq[i * rb:]), ptr(aq[i * rb:])) for i in range(4)], np.float32)
    g["dq80_w"], g["dq80_a"], g["dq80_s"] = wq, aq, f32bits(s)

    # ggml_vec_dot_f32 (vec.cpp:11-135): every tail shape
    ns = np.array([1, 7, 8, 10, 16, 23, 64, 100, 777, 2048], np.int64)
    us, vs, ss = [], [], []
    for n in ns:
        for _ in range(2):
            u = rng.standard_normal(n).astype(np.float32)
            v = rng.standard_normal(n).astype(np.float32)
            us.append(u)
            vs.append(v)
            ss.append(R.qwr_vec_dot_f32(int(n), ptr(u), ptr(v)))
    g["vdf_n"], g["vdf_u"], g["vdf_v"] = ns, np.concatenate(us), np.concatenate(vs)
    g["vdf_s"] = f32bits(np.array(ss, np.float32))

    # ggml_v_expf / ggml_v_silu (vec.h:1191-1226), 16 lanes at a time
    xs = np.concatenate([rng.uniform(-110, 92, 224), rng.standard_normal(16) * 4,
                         np.array([0.0, -0.0, 88.7, -103.9, 1e-30, -1e-30] + [0.0] * 10)]).astype(np.float32)
    e = np.zeros_like(xs)
    si = np.zeros_like(xs)
    for i in range(0, xs.size, 16):
        R.qwr_v_expf16(ptr(xs[i:]), ptr(e[i:]))
        R.qwr_v_silu16(ptr(xs[i:]), ptr(si[i:]))
    g["exp_x"], g["exp_y"], g["silu_y"] = xs, f32bits(e), f32bits(si)

    # soft_max rows (ops.cpp:5813-5920) for E = 128, 512 and a ragged 100
    for E in (128, 512, 100):
        lg = (rng.standard_normal((3, E)) * 0.9).astype(np.float32)
        p = np.zeros_like(lg)
        for r in range(3):
            R.qwr_soft_max_row(E, ptr(lg[r]), ptr(p[r]))
        g[f"sm{E}_x"], g[f"sm{E}_y"] = lg, f32bits(p)

    # swiglu (vec.cpp:417-445), ragged length
    gt = (rng.standard_normal(100) * 3).astype(np.float32)
    up = rng.standard_normal(100).astype(np.float32)
    y = np.zeros(100, np.float32)
    R.qwr_swiglu(100, ptr(y), ptr(gt), ptr(up))
    g["swiglu_g"], g["swiglu_u"], g["swiglu_y"] = gt, up, f32bits(y)

    # argmax keeps the last maximum (vec.h:1618-1626)
    xa = np.array([[1.0, 3.0, 2.0, 3.0, -1.0, 3.0, 0.5, 0.0],
                   [5.0, 5.0, 5.0, 5.0, 5.0, 5.0, 5.0, 5.0],
                   [-2.0, -1.0, -3.0, -1.0, -4.0, -5.0, -6.0, -7.0]], np.float32)
    g["argmax_x"] = xa
    g["argmax_i"] = np.array([R.qwr_argmax(8, ptr(r)) for r in xa], np.int32)

    # slot pool: a Zipf trace through ensure(); every victim the oracle takes is
    # checked against the reference GpuLruIndex::pick before it is recorded
    g.update(pool_trace(rng))
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(g)} arrays)")


def pool_trace(rng):
    n_layer, n_expert, slots = 2, 32, np.array([12, 11, 13], np.int32)
    O = oracle()
    h = O.qwo_pool_new(n_layer, n_expert, ptr(slots), 0)
    lru = ref_lru()
    idx = [lru.qwr_lru_new(int(s)) for s in slots]
    for r in range(3):
        keys = np.full(slots[r], -1, np.int32)
        clocks = np.zeros(slots[r], np.uint64)
        assert lru.qwr_lru_rebuild(idx[r], int(slots[r]), ptr(keys), ptr(clocks)) == 0
    pop = 1.0 / np.arange(1, n_expert + 1) ** 1.1
    pop /= pop.sum()
    layers, lens, all_ids, all_out = [], [], [], []
    state = [(np.full(s, -1, np.int32), np.zeros(s, np.uint64)) for s in slots]
    clock = 0
    for _ in range(60):
        layer = int(rng.integers(0, n_layer))
        T = int(rng.integers(1, 4))
        ids = np.concatenate([rng.choice(n_expert, 4, replace=False, p=pop) for _ in range(T)]).astype(np.int32)
        out = np.zeros((3, ids.size), np.int32)
        log = np.zeros(4 * 3 * ids.size, np.int32)
        nf = ctypes.c_int()
        rc = O.qwo_pool_ensure(h, layer, ptr(ids), ids.size, ptr(out[0]), ptr(out[1]), ptr(out[2]), ptr(log),
                               ctypes.byref(nf))
        assert rc == 0
        for i, e in enumerate(ids):
            key = layer * n_expert + int(e)
            for r in range(3):
                clock += 1
                slot = int(out[r, i])
                keys, clocks = state[r]
                if keys[slot] != key:
                    assert lru.qwr_lru_pick(idx[r], None) == slot
                    if keys[slot] >= 0:
                        assert lru.qwr_lru_release(idx[r], slot) == 0
                    keys[slot] = key
                clocks[slot] = clock
                assert lru.qwr_lru_occupy_or_touch(idx[r], slot, ctypes.c_uint64(clock)) == 0
        layers.append(layer)
        lens.append(ids.size)
        all_ids.append(ids)
        all_out.append(out)
    O.qwo_pool_free(h)
    for i in idx:
        lru.qwr_lru_free(i)
    return {"pool_shape": np.array([n_layer, n_expert], np.int32), "pool_slots": slots,
            "pool_layers": np.array(layers, np.int32), "pool_lens": np.array(lens, np.int32),
            "pool_ids": np.concatenate(all_ids), "pool_out": np.concatenate(all_out, axis=1)}


if __name__ == "__main__":
    main()
