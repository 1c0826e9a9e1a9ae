"""Benchmark of the MoE verify step on one MI355X.

Workload (the metric's configuration): one Qwen3-30B-A3B-shape MoE block
(hidden 2048, 128 experts, FFN 768, top-8, Q4_K experts quantized from
N(0, 0.02), f32 router N(0, 0.02)) run as an MTP verify batch of 4 tokens
(x ~ N(0, 1)), followed by the verify head: rms_norm, a Q8_0 lm_head
2048 x 151936 (quantized from N(0, 1/sqrt(2048))), argmax and the greedy
acceptance against seeded drafts.  All experts are resident in the slot
pools (slot = expert id, remapped on the device).  A step is one verify
batch; inputs for every step are resident in HBM before timing starts.

Prints one JSON line: tokens/s (4 tokens per step), the roofline of the
dominant kernel (the lm_head GEMV, HBM-bound), measured with HIP events
around its launches inside the timed region, and the CPU baseline: the
same step through the reference's own ggml-CPU kernels on this host.
"""
import argparse
import ctypes
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE tokens/s + achieved HBM GB/s (% of 8 TB/s), Q4_K verify, 1×MI355X"
HBM_PEAK_GBS = 8000.0
H, N, E, K_USED, T, V = 2048, 768, 128, 8, 4, 151936
Q4K_ROW_GU = H // 256 * 144          # 1152 B
Q4K_ROW_D = N // 256 * 144           # 432 B
SLAB = N * Q4K_ROW_GU                # 884,736 B per role per expert
LM_ROW = H // 32 * 34                # 2176 B
QK_K_ = 256
CAL_BYTES = 256 << 20                # calibration copy for the PMC byte counters
TRAFFIC_SUMMARY = {"step": os.path.join(ROOT, "profiles", "verify_step_T4_traffic.json"),
                   "ops": os.path.join(ROOT, "profiles", "verify_ops_T4_traffic.json"),
                   "prefill": os.path.join(ROOT, "profiles", "prefill_T512_traffic.json")}


def measured_traffic(path, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the calibration kernel),
    or None."""
    try:
        with open(TRAFFIC_SUMMARY[path]) as f:
            return float(json.load(f)["kernels"][kernel]["traffic_bytes"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="default: 200 (verify), 256 (decode48)")
    ap.add_argument("--warmup", type=int, default=None, help="default: 20 (verify), 10 (decode48)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bounded CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--accept-rate", type=float, default=0.7, help="probability that a draft equals the target")
    ap.add_argument("--path", choices=["step", "ops"], default="step",
                    help="step: the fused verify step (one launch); ops: qwm_moe_block_resident + qwm_verify_accept")
    ap.add_argument("--workload", choices=["verify", "decode48", "prefill", "missfill"], default="verify",
                    help="verify: the metric's MTP verify step; decode48: 1-token decode through 48 stacked "
                         "MoE blocks (qwm_moe_decode, HIP graph); prefill: 512 tokens through one "
                         "Qwen3-Next-shape layer's MUL_MAT_IDs (expert-grouped MFMA GEMM); missfill: T=4 verify "
                         "batches through one Qwen3-Next-shape layer with a 128-slot LRU pool, misses copied "
                         "from pinned host memory")
    ap.add_argument("--popularity", choices=["sampled", "offset"], default="sampled",
                    help="missfill: sampled = each token's top-10 drawn from Zipf(1.1) and forced through the route "
                         "mask; offset = a fixed log-popularity logit offset (nearly every lookup then hits)")
    ap.add_argument("--fetch", choices=["gather", "memcpy", "file"], default="gather",
                    help="missfill: how misses reach the pool (the other mode is run too and reported beside)")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"decode48": 256, "prefill": 50, "missfill": 400}.get(args.workload, 200)
    if args.warmup is None:
        args.warmup = {"decode48": 10, "prefill": 5, "missfill": 200}.get(args.workload, 20)
    return args


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (the library has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import questwend_amd as qa

    if args.workload == "decode48":
        bench_decode(args, torch, qa)
        return
    if args.workload == "prefill":
        bench_prefill(args, torch, qa)
        return
    if args.workload == "missfill":
        bench_missfill(args, torch, qa)
        return
    L = qa.lib()
    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    stream = torch.cuda.current_stream().cuda_stream

    # ------------------------------------------------------------ weights --
    pools = [torch.empty(E * SLAB, dtype=torch.uint8, device=dev) for _ in range(3)]
    tmp = torch.empty(N * H, dtype=torch.float32, device=dev)
    for r in range(3):
        for e in range(E):
            tmp.normal_(0.0, 0.02)
            qa.check(L.qwm_quantize(qa.TYPE_Q4_K, tmp.data_ptr(), pools[r].data_ptr() + e * SLAB, N * H, stream))
    router = (torch.randn((E, H), device=dev) * 0.02).contiguous()
    lm_f = torch.empty(V * H, dtype=torch.float32, device=dev).normal_(0.0, 1.0 / np.sqrt(H))
    lm = torch.empty(V * LM_ROW, dtype=torch.uint8, device=dev)
    qa.check(L.qwm_quantize(qa.TYPE_Q8_0, lm_f.data_ptr(), lm.data_ptr(), V * H, stream))
    del lm_f, tmp
    tables = torch.arange(E, dtype=torch.int32, device=dev).repeat(3).contiguous()   # slot = expert id

    layer = qa.MoeLayer()
    layer.gate_pool = qa.tensor(qa.TYPE_Q4_K, H, N, E, pools[0])
    layer.up_pool = qa.tensor(qa.TYPE_Q4_K, H, N, E, pools[1])
    layer.down_pool = qa.tensor(qa.TYPE_Q4_K, N, H, E, pools[2])
    layer.router = qa.tensor(qa.TYPE_F32, H, E, 1, router)
    layer.n_expert_used, layer.norm_weights, layer.weights_scale = K_USED, 1, 1.0
    lm_t = qa.tensor(qa.TYPE_Q8_0, H, V, 1, lm)

    n_all = args.warmup + args.steps
    xs = torch.randn((n_all, T, H), device=dev)
    hs = torch.empty((n_all, T, H), device=dev)
    ids = torch.zeros((n_all, T, K_USED), dtype=torch.int32, device=dev)
    wts = torch.zeros((n_all, T, K_USED), dtype=torch.float32, device=dev)
    res = torch.zeros((n_all, T + 2), dtype=torch.int32, device=dev)
    drafts = torch.zeros((n_all, T - 1), dtype=torch.int32, device=dev)
    ws_moe = torch.empty(L.qwm_moe_workspace_size(layer, T), dtype=torch.uint8, device=dev)
    ws_v = torch.empty(L.qwm_verify_workspace_size(lm_t, T), dtype=torch.uint8, device=dev)
    ws_s = torch.empty(L.qwm_verify_step_workspace_size(layer, lm_t, T), dtype=torch.uint8, device=dev)
    for w in (ws_moe, ws_v, ws_s):
        qa.check(L.qwm_workspace_init(w.data_ptr(), w.numel(), stream))

    def step(s):
        x_t = qa.tensor(qa.TYPE_F32, H, T, 1, xs[s])
        h_t = qa.tensor(qa.TYPE_F32, H, T, 1, hs[s])
        i_t = qa.tensor(qa.TYPE_I32, K_USED, T, 1, ids[s])
        w_t = qa.tensor(qa.TYPE_F32, K_USED, T, 1, wts[s])
        if args.path == "step":
            qa.check(L.qwm_verify_step(layer, 0, tables.data_ptr(), E, x_t, None, x_t, h_t, i_t, w_t, lm_t,
                                       None, 1e-6, drafts[s].data_ptr(), res[s].data_ptr(),
                                       ws_s.data_ptr(), ws_s.numel(), stream))
            return
        qa.check(L.qwm_moe_block_resident(layer, 0, tables.data_ptr(), E, x_t, None, x_t, h_t, i_t, w_t,
                                          ws_moe.data_ptr(), ws_moe.numel(), stream))
        qa.check(L.qwm_verify_accept(lm_t, h_t, None, 1e-6, drafts[s].data_ptr(), res[s].data_ptr(),
                                     ws_v.data_ptr(), ws_v.numel(), stream))

    # seeded drafts: one untimed pass finds each step's targets; a draft equals
    # its target with probability accept-rate (so a in {0..3} all occur)
    for s in range(n_all):
        step(s)
    torch.cuda.synchronize()
    target = res[:, :T - 1].clone()
    rng = np.random.default_rng(args.seed)
    keep = torch.from_numpy(rng.random((n_all, T - 1)) < args.accept_rate).to(dev)
    rnd = torch.from_numpy(rng.integers(0, V, (n_all, T - 1)).astype(np.int32)).to(dev)
    drafts.copy_(torch.where(keep, target, rnd))

    # ------------------------------------------------------------- timed --
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
    main_kernel = "step" if args.path == "step" else "lm_head"
    qa.check(L.qwm_profile_start(main_kernel.encode(), args.steps))
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for s in range(args.warmup, n_all):
        step(s)
    ev1.record()
    torch.cuda.synchronize()
    elapsed_ms = ev0.elapsed_time(ev1)
    lm_ms = np.zeros(args.steps, np.float32)
    n_lm = L.qwm_profile_stop(lm_ms.ctypes.data, args.steps)
    ms_step = elapsed_ms / args.steps
    tokens_per_s = T * args.steps / (elapsed_ms / 1e3)
    r = res[args.warmup:].cpu().numpy()
    accepted = r[:, T]
    acc_tok_s = float((accepted + 1).sum()) / (elapsed_ms / 1e3)

    # secondary kernels of the per-op path (untimed pass, same steps)
    kern = {}
    for name in (["route", "gate_up", "down"] if args.path == "ops" else []):
        qa.check(L.qwm_profile_start(name.encode(), args.steps))
        for s in range(args.warmup, n_all):
            step(s)
        torch.cuda.synchronize()
        d = np.zeros(args.steps, np.float32)
        n = L.qwm_profile_stop(d.ctypes.data, args.steps)
        kern[name] = float(d[:n].mean() * 1e3) if n else None

    # a plain streaming kernel of known size (torch.neg: reads and writes
    # 256 MiB, a kernel name of its own): under rocprofv3 --pmc its FETCH_SIZE
    # and WRITE_SIZE give the counters' scale
    cal_src = torch.full((CAL_BYTES // 4,), 1.0, dtype=torch.float32, device=dev)
    cal_dst = torch.empty_like(cal_src)
    for _ in range(3):
        torch.neg(cal_src, out=cal_dst)
    torch.cuda.synchronize()
    del cal_src, cal_dst

    # algorithmic bytes
    ids_np = ids[args.warmup:].cpu().numpy()
    uniq = np.array([len(np.unique(i)) for i in ids_np])
    lm_bytes = V * LM_ROW + T * (H + H // 32 * 4)
    step_bytes = uniq * 3 * SLAB + E * H * 4 + 2 * T * H * 4 + V * LM_ROW
    lm_avg_ms = float(lm_ms[:n_lm].mean())
    main_bytes = float(step_bytes.mean()) if args.path == "step" else lm_bytes
    lm_gbs = main_bytes / (lm_avg_ms * 1e-3) / 1e9
    gu_bytes = float(uniq.mean()) * 2 * SLAB
    dn_bytes = float(uniq.mean()) * SLAB
    for name, b in [("gate_up", gu_bytes), ("down", dn_bytes)]:
        if kern.get(name):
            kern[name + "_gbs"] = b / (kern[name] * 1e-6) / 1e9

    out = {
        "metric": METRIC, "value": tokens_per_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "MTP verify T=4 (1+3 drafts) through one Qwen3-30B-A3B-shape MoE block "
                               "(H 2048, 128 experts resident, FFN 768, top-8, Q4_K) + rms_norm + Q8_0 lm_head "
                               "2048x151936 argmax + greedy accept",
                   "tokens_per_step": T, "experts_per_step_mean": float(uniq.mean())},
        "roofline": {"bound": "hbm",
                     "kernel": ("step (MoE block + verify head, one launch)" if args.path == "step"
                                else "lm_head (Q8_0 GEMV + argmax)"),
                     "achieved": lm_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": lm_gbs / HBM_PEAK_GBS,
                     "traffic": measured_traffic(args.path, main_kernel),
                     "traffic_source": os.path.relpath(TRAFFIC_SUMMARY[args.path], ROOT),
                     "bytes_per_launch": main_bytes, "avg_launch_us": lm_avg_ms * 1e3, "launches_timed": int(n_lm)},
        "path": args.path,
        "step_hbm_gbs": float(step_bytes.mean()) / (ms_step * 1e-3) / 1e9,
        "step_bytes_mean": float(step_bytes.mean()),
        "accepted_tokens_per_s": acc_tok_s,
        "accept_histogram": np.bincount(accepted, minlength=T).tolist(),
        "kernels_us": kern,
    }

    # --------------------------------------------------------- CPU baseline --
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args, torch, pools, router, lm, xs, drafts, ids, res)
    print(json.dumps(out))


def bench_decode(args, torch, qa, n_layers=48):
    """1-token decode through 48 stacked Qwen3-30B-A3B-shape MoE blocks
    (attention omitted), every expert resident (slot = expert id through
    device tables, ~17 GB of Q4_K), a new N(0, 1) input each step; one step
    is one qwm_moe_decode call, replayed from a HIP graph."""
    L = qa.lib()
    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    stream = torch.cuda.current_stream().cuda_stream
    T1 = 1
    pools, routers = [], []
    tmp = torch.empty(N * H, dtype=torch.float32, device=dev)
    layers = (qa.MoeLayer * n_layers)()
    for l in range(n_layers):
        pl = [torch.empty(E * SLAB, dtype=torch.uint8, device=dev) for _ in range(3)]
        for r in range(3):
            for e in range(E):
                tmp.normal_(0.0, 0.02)
                qa.check(L.qwm_quantize(qa.TYPE_Q4_K, tmp.data_ptr(), pl[r].data_ptr() + e * SLAB, N * H, stream))
        rt = (torch.randn((E, H), device=dev) * 0.02).contiguous()
        pools.append(pl)
        routers.append(rt)
        layers[l].gate_pool = qa.tensor(qa.TYPE_Q4_K, H, N, E, pl[0])
        layers[l].up_pool = qa.tensor(qa.TYPE_Q4_K, H, N, E, pl[1])
        layers[l].down_pool = qa.tensor(qa.TYPE_Q4_K, N, H, E, pl[2])
        layers[l].router = qa.tensor(qa.TYPE_F32, H, E, 1, rt)
        layers[l].n_expert_used, layers[l].norm_weights, layers[l].weights_scale = K_USED, 1, 1.0
        if l % 8 == 7:
            torch.cuda.synchronize()
            print(f"decode48: {l + 1} layers quantized", file=sys.stderr, flush=True)
    del tmp
    tables = torch.arange(E, dtype=torch.int32, device=dev).repeat(3, n_layers).contiguous()   # [3][layer * E + e]
    ws = torch.empty(L.qwm_moe_decode_workspace_size(layers, n_layers, T1), dtype=torch.uint8, device=dev)
    qa.check(L.qwm_workspace_init(ws.data_ptr(), ws.numel(), stream))
    n_all = args.warmup + args.steps
    xs = torch.randn((n_all, T1, H), device=dev)
    xw = torch.empty((T1, H), device=dev)
    xt = qa.tensor(qa.TYPE_F32, H, T1, 1, xw)

    def decode(st):
        qa.check(L.qwm_moe_decode(layers, n_layers, tables.data_ptr(), n_layers * E, xt, ws.data_ptr(), ws.numel(), st))

    def timed(replay):
        for s in range(args.warmup):
            xw.copy_(xs[s])
            replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for s in range(args.warmup, n_all):
            xw.copy_(xs[s])
            replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    ms_direct = timed(lambda: decode(torch.cuda.current_stream().cuda_stream))
    graph = torch.cuda.CUDAGraph()
    xw.copy_(xs[0])
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        decode(torch.cuda.current_stream().cuda_stream)
    ms_graph = timed(graph.replay)
    ms = min(ms_direct, ms_graph)
    # the same 48 layers through the per-op kernels (qwm_moe_block_resident per
    # layer: route, gate/up, down launches), replayed from a HIP graph on the
    # same box, as the comparison for the persistent launches
    wsb = torch.empty(L.qwm_moe_workspace_size(layers[0], T1), dtype=torch.uint8, device=dev)
    qa.check(L.qwm_workspace_init(wsb.data_ptr(), wsb.numel(), stream))
    xb = torch.empty((T1, H), device=dev)
    tb = qa.tensor(qa.TYPE_F32, H, T1, 1, xb)

    def per_op(st):
        for l in range(n_layers):
            src, dst = (xt, tb) if l % 2 == 0 else (tb, xt)
            qa.check(L.qwm_moe_block_resident(layers[l], l, tables.data_ptr(), n_layers * E, src, None, src, dst,
                                              None, None, wsb.data_ptr(), wsb.numel(), st))
    g_op = torch.cuda.CUDAGraph()
    xw.copy_(xs[0])
    torch.cuda.synchronize()
    with torch.cuda.graph(g_op):
        per_op(torch.cuda.current_stream().cuda_stream)
    ms_per_op = timed(g_op.replay)
    step_bytes = n_layers * (K_USED * 3 * SLAB + E * H * 4 + 2 * T1 * H * 4)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        lib = ref_cpu_lib()
        if lib is None:
            cpu = NO_REF
        else:
            # the GPU's output for the first input after every prefix of the layers,
            # as the parity check of the sample
            gpu_x = []
            for nl in range(1, n_layers + 1):
                xw.copy_(xs[0])
                qa.check(L.qwm_moe_decode(layers, nl, tables.data_ptr(), n_layers * E, xt, ws.data_ptr(), ws.numel(),
                                          torch.cuda.current_stream().cuda_stream))
                gpu_x.append(xw.cpu().numpy()[0].copy())
            host = [[p.cpu().numpy() for p in pl] for pl in pools]
            rts = [rt.cpu().numpy() for rt in routers]
            x_np = xs.cpu().numpy()
            a = BlockArgs()
            a.H, a.N, a.E, a.k, a.T, a.n_threads = H, N, E, K_USED, T1, CPU_THREADS
            ids = np.zeros((T1, K_USED), np.int32)
            out = np.zeros((T1, H), np.float32)
            a.ids, a.out = ids.ctypes.data, out.ctypes.data
            res = {}

            def token(i):
                x = np.ascontiguousarray(x_np[i % n_all])
                for l in range(n_layers):
                    a.router, a.gate, a.up, a.down = (rts[l].ctypes.data, host[l][0].ctypes.data,
                                                      host[l][1].ctypes.data, host[l][2].ctypes.data)
                    a.x = x.ctypes.data
                    lib.qwr_cpu_moe_block(ctypes.byref(a))
                    if i == 0:
                        res.setdefault("layers", []).append((x.copy(), out.copy(), ids.copy()))
                    x = out.copy()

            n, secs = timed_sample(token, args.cpu_seconds)
            errs = [rel_err(c[1][0], g) for c, g in zip(res["layers"], gpu_x)]
            first_off = next((l + 1 for l, e_ in enumerate(errs) if e_ > 1e-3), None)
            # every block on the CPU's own input: the single-layer parity, free of the chain's divergence
            wsb = torch.empty(L.qwm_moe_workspace_size(layers[0], T1), dtype=torch.uint8, device=dev)
            qa.check(L.qwm_workspace_init(wsb.data_ptr(), wsb.numel(), stream))
            blk_err, ids_same = [], 0
            for l, (xin, xout, cids) in enumerate(res["layers"]):
                din = torch.from_numpy(xin).to(dev)
                dout = torch.empty_like(din)
                gids = torch.empty((T1, K_USED), dtype=torch.int32, device=dev)
                tin = qa.tensor(qa.TYPE_F32, H, T1, 1, din)
                qa.check(L.qwm_moe_block_resident(layers[l], l, tables.data_ptr(), n_layers * E, tin, None, tin,
                                                  qa.tensor(qa.TYPE_F32, H, T1, 1, dout),
                                                  qa.tensor(qa.TYPE_I32, K_USED, T1, 1, gids), None,
                                                  wsb.data_ptr(), wsb.numel(), stream))
                blk_err.append(rel_err(dout.cpu().numpy() - xin, xout - xin))
                ids_same += int(np.array_equal(gids.cpu().numpy(), cids))
            cpu = {"value": n / secs, "unit": "tokens/s", "cores": CPU_THREADS, "kind": "reference",
                   "sample": f"{n} decode tokens ({secs:.1f} s) through the same 48 blocks with the reference's "
                             f"ggml-CPU kernels (x86-64 AVX-512 build, {CPU_THREADS} OpenMP threads)",
                   "ms_per_token": 1e3 * secs / n,
                   "parity_first_token": {
                       "per_block_on_cpu_input": {"max_rel_err_moe": max(blk_err), "median_rel_err_moe": float(np.median(blk_err)),
                                                  "layers_with_identical_ids": f"{ids_same}/{n_layers}"},
                       "chained_rel_err_per_layer": [float(f"{e_:.3g}") for e_ in errs],
                       "chain_first_layer_above_1e-3": first_off}}
    print(json.dumps({
        "metric": "MoE decode tokens/s + achieved HBM GB/s (% of 8 TB/s), 48 stacked Q4_K blocks, 1xMI355X",
        "value": T1 / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "1-token decode through 48 stacked Qwen3-30B-A3B-shape MoE blocks (H 2048, 128 experts "
                               "resident per layer, FFN 768, top-8, Q4_K; attention omitted), new N(0,1) input per step",
                   "graph": ms_graph <= ms_direct, "ms_direct": ms_direct, "ms_graph": ms_graph,
                   "ms_per_op_kernels_graph": ms_per_op},
        "roofline": {"bound": "hbm", "kernel": "whole step (3 persistent k_decode launches of 16 layers)", "achieved": gbs,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                     "bytes_per_launch": step_bytes},
        "cpu_baseline": cpu,
    }))


def bench_prefill(args, torch, qa, T_pf=512, E_pf=512, k_pf=10, N_pf=512):
    """A 512-token prefill chunk through one Qwen3-Next-shape MoE layer's
    expert GEMMs (hidden 2048, 512 experts, FFN 512, top-10, Q4_K from
    N(0, 0.02)): act = swiglu(mul_mat_id(gate, x, ids), mul_mat_id(up, x, ids)),
    down = mul_mat_id(down, act, ids).  ids are each token's top-10 of random
    router logits.  The timed step is qwm_mul_mat_id_swiglu (one grouped
    int8-MFMA pass over gate and up that writes act) and qwm_mul_mat_id for
    down; the same step through three separate qwm_mul_mat_id calls and a
    torch SwiGLU is timed beside it for comparison."""
    L = qa.lib()
    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    stream = torch.cuda.current_stream().cuda_stream
    slab = N_pf * H // QK_K_ * 144
    pools = [torch.empty(E_pf * slab, dtype=torch.uint8, device=dev) for _ in range(3)]
    tmp = torch.empty(N_pf * H, dtype=torch.float32, device=dev)
    for r in range(3):
        for e in range(E_pf):
            tmp.normal_(0.0, 0.02)
            qa.check(L.qwm_quantize(qa.TYPE_Q4_K, tmp.data_ptr(), pools[r].data_ptr() + e * slab, N_pf * H, stream))
    del tmp
    x = torch.randn((T_pf, 1, H), device=dev)
    ids = torch.topk(torch.randn((T_pf, E_pf), device=dev), k_pf, dim=1).indices.to(torch.int32).contiguous()
    gate = torch.empty((T_pf, k_pf, N_pf), device=dev)
    up = torch.empty_like(gate)
    act = torch.empty_like(gate)
    down = torch.empty((T_pf, k_pf, H), device=dev)
    t_g = qa.tensor(qa.TYPE_Q4_K, H, N_pf, E_pf, pools[0])
    t_u = qa.tensor(qa.TYPE_Q4_K, H, N_pf, E_pf, pools[1])
    t_d = qa.tensor(qa.TYPE_Q4_K, N_pf, H, E_pf, pools[2])
    t_x = qa.tensor(qa.TYPE_F32, H, 1, T_pf, x)
    t_ids = qa.tensor(qa.TYPE_I32, k_pf, T_pf, 1, ids)
    t_act = qa.tensor(qa.TYPE_F32, N_pf, k_pf, T_pf, act)
    need = max(L.qwm_mul_mat_id_swiglu_workspace_size(t_g, t_u, t_x, t_ids),
               L.qwm_mul_mat_id_workspace_size(t_g, t_x, t_ids), L.qwm_mul_mat_id_workspace_size(t_d, t_act, t_ids))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    qa.check(L.qwm_workspace_init(ws.data_ptr(), ws.numel(), stream))

    def gemm(t_as, t_b, out, st):
        qa.check(L.qwm_mul_mat_id(t_as, t_b, t_ids, qa.tensor(qa.TYPE_F32, out.shape[2], k_pf, T_pf, out),
                                  ws.data_ptr(), ws.numel(), st))

    def step():
        st = torch.cuda.current_stream().cuda_stream
        qa.check(L.qwm_mul_mat_id_swiglu(t_g, t_u, t_x, t_ids, t_act, ws.data_ptr(), ws.numel(), st))
        gemm(t_d, t_act, down, st)

    def step_separate():
        st = torch.cuda.current_stream().cuda_stream
        gemm(t_u, t_x, up, st)
        gemm(t_g, t_x, gate, st)
        torch.mul(torch.nn.functional.silu(gate), up, out=act)
        gemm(t_d, t_act, down, st)

    def timed(fn, launches):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        qa.check(L.qwm_profile_start(b"prefill_gemm*", launches * args.steps))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        g = np.zeros(launches * args.steps, np.float32)
        n = L.qwm_profile_stop(g.ctypes.data, launches * args.steps)
        return e0.elapsed_time(e1) / args.steps, (g[:n].reshape(-1, launches) if n == launches * args.steps else None)

    ms_sep, g_sep = timed(step_separate, 3)
    down_sep = down.clone()
    ms, g_ms = timed(step, 2)
    # the PMC byte counters' scale (as in the verify bench): torch.neg over 256 MiB
    cal_src = torch.full((CAL_BYTES // 4,), 1.0, dtype=torch.float32, device=dev)
    cal_dst = torch.empty_like(cal_src)
    for _ in range(3):
        torch.neg(cal_src, out=cal_dst)
    torch.cuda.synchronize()
    del cal_src, cal_dst
    act_fused = act.clone()
    torch.mul(torch.nn.functional.silu(gate), up, out=act)     # the separate path's act, same x and ids
    act_diff = float((act_fused - act).abs().max())
    down_diff = float((down - down_sep).abs().max())
    cpu = None
    if not args.no_cpu:
        lib = ref_cpu_lib()
        if lib is None:
            cpu = NO_REF
        else:
            hq = [p.cpu().numpy() for p in pools]
            xh = x.cpu().numpy()
            ih = ids.cpu().numpy()
            gd = down.cpu().numpy()
            hg = np.zeros((T_pf, k_pf, N_pf), np.float32)
            hu = np.zeros_like(hg)
            hd = np.zeros((T_pf, k_pf, H), np.float32)
            P_ = lambda arr: arr.ctypes.data

            def cpu_step(i):
                lib.qwr_cpu_mul_mat_id(P_(hq[1]), H, N_pf, E_pf, P_(xh), 1, T_pf, P_(ih), k_pf, P_(hu), CPU_THREADS)
                lib.qwr_cpu_mul_mat_id(P_(hq[0]), H, N_pf, E_pf, P_(xh), 1, T_pf, P_(ih), k_pf, P_(hg), CPU_THREADS)
                ha = np.ascontiguousarray((hg / (1.0 + np.exp(-hg)) * hu).astype(np.float32))
                lib.qwr_cpu_mul_mat_id(P_(hq[2]), N_pf, H, E_pf, P_(ha), k_pf, T_pf, P_(ih), k_pf, P_(hd), CPU_THREADS)

            n, secs = timed_sample(cpu_step, args.cpu_seconds)
            cpu = {"value": T_pf * n / secs, "unit": "tokens/s", "cores": CPU_THREADS, "kind": "reference",
                   "sample": f"{n} prefill steps ({secs:.1f} s): the same three MUL_MAT_IDs through the reference's "
                             f"ggml-CPU vec_dot kernels ({CPU_THREADS} OpenMP threads; ggml's tiled AVX-512 VNNI "
                             f"kernel for experts with >= 8 columns is not built here); down output against the "
                             f"GPU's: rel err {rel_err(hd, gd):.2e}",
                   "ms_per_step": 1e3 * secs / n}
    used = len(np.unique(ids.cpu().numpy()))
    w_bytes = 3 * used * slab
    flops = 2.0 * T_pf * k_pf * (2 * N_pf * H + H * N_pf)
    gemm_ms = float(g_ms.sum(1).mean()) if g_ms is not None else ms
    # the fused gate/up launch: both matrices' used slabs, x read, act written
    gu_bytes = 2 * used * slab + 4 * T_pf * H + 4 * T_pf * k_pf * N_pf
    gu_ms = float(g_ms[:, 0].mean()) if g_ms is not None else ms
    gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    step_gbs = (w_bytes + 4 * T_pf * H + 2 * 4 * T_pf * k_pf * N_pf + 4 * T_pf * k_pf * H) / (gemm_ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "MoE prefill tokens/s (expert GEMMs of one Qwen3-Next-shape layer), 1xMI355X",
        "value": T_pf / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "512-token prefill chunk, one Qwen3-Next-shape MoE layer (H 2048, 512 experts, FFN 512, "
                               "top-10, Q4_K): gate+up+SwiGLU in one expert-grouped int8 MFMA pass, then down",
                   "experts_used": used, "gemm_ms_per_step": gemm_ms,
                   "gemm_ms_each": g_ms.mean(0).tolist() if g_ms is not None else None,
                   "gemm_GBps_step": step_gbs,
                   "separate": {"ms_per_step": ms_sep, "tokens_per_s": T_pf / (ms_sep * 1e-3),
                                "gemm_ms_each": g_sep.mean(0).tolist() if g_sep is not None else None,
                                "act_max_abs_diff_vs_torch_silu": act_diff, "down_max_abs_diff": down_diff}},
        "roofline": {"bound": "hbm", "kernel": "k_pf_gemm<8, gate/up> (1 of 2 launches per step)", "achieved": gbs,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": measured_traffic("prefill", "gate_up"),
                     "traffic_source": os.path.relpath(TRAFFIC_SUMMARY["prefill"], ROOT),
                     "bytes_per_launch": gu_bytes},
        "mfma": {"tops": flops / (gemm_ms * 1e-3) / 1e12, "peak_int8_tops": 5000.0,
                 "frac": flops / (gemm_ms * 1e-3) / 5e15},
        "cpu_baseline": cpu,
    }))


def bench_missfill(args, torch, qa, E_n=512, N_n=512, k_n=10, S_n=128, skew=1.1):
    """MTP verify batches (T = 4, new N(0, 1) inputs each step) through one
    Qwen3-Next-shape MoE layer (hidden 2048, 512 experts + a shared expert,
    FFN 512, top-10, Q4_K from N(0, 0.02)) whose experts live in pinned host
    memory, with a GPU slot pool of 128 experts per role.  Zipf(1.1)
    popularity over a seeded expert permutation enters through the route
    mask: "sampled" (default) draws each token's 10 experts from Zipf(1.1)
    and forces them with a +16 mask bias (the routing weights stay the
    softmax of their own logits); "offset" adds fixed offsets log(p_e), under
    which the router keeps choosing about the same 110 experts and the pool
    nearly never misses.  A step is the reference's cached path: route on the
    device, the ids read back (synchronous), the pool's LRU decisions on the
    host with misses copied by hipMemcpyAsync on a side stream, the slot ids
    uploaded, the compute stream waiting for the copies, then the experts on
    slot ids.  Warmup steps bring the pool to its steady state before
    timing."""
    L = qa.lib()
    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    stream = torch.cuda.current_stream().cuda_stream
    slab = N_n * H // QK_K_ * 144
    host = []
    tmp = torch.empty(N_n * H, dtype=torch.float32, device=dev)
    stage = torch.empty(E_n * slab, dtype=torch.uint8, device=dev)
    for r in range(3):
        for e in range(E_n):
            tmp.normal_(0.0, 0.02)
            qa.check(L.qwm_quantize(qa.TYPE_Q4_K, tmp.data_ptr(), stage.data_ptr() + e * slab, N_n * H, stream))
        hr = torch.empty(E_n * slab, dtype=torch.uint8, pin_memory=True)
        hr.copy_(stage)
        host.append(hr)
    sh = []
    for r in range(3):
        q = torch.empty(slab, dtype=torch.uint8, device=dev)
        tmp.normal_(0.0, 0.02)
        qa.check(L.qwm_quantize(qa.TYPE_Q4_K, tmp.data_ptr(), q.data_ptr(), N_n * H, stream))
        sh.append(q)
    del tmp, stage
    router = (torch.randn((E_n, H), device=dev) * 0.02).contiguous()
    sh_inp = (torch.randn(H, device=dev) * 0.02).contiguous()
    pools = [torch.empty(S_n * slab, dtype=torch.uint8, device=dev) for _ in range(3)]
    lay = qa.MoeLayer()
    lay.gate_pool = qa.tensor(qa.TYPE_Q4_K, H, N_n, S_n, pools[0])
    lay.up_pool = qa.tensor(qa.TYPE_Q4_K, H, N_n, S_n, pools[1])
    lay.down_pool = qa.tensor(qa.TYPE_Q4_K, N_n, H, S_n, pools[2])
    lay.router = qa.tensor(qa.TYPE_F32, H, E_n, 1, router)
    lay.sh_gate = qa.tensor(qa.TYPE_Q4_K, H, N_n, 1, sh[0])
    lay.sh_up = qa.tensor(qa.TYPE_Q4_K, H, N_n, 1, sh[1])
    lay.sh_down = qa.tensor(qa.TYPE_Q4_K, N_n, H, 1, sh[2])
    lay.sh_gate_inp = qa.tensor(qa.TYPE_F32, H, 1, 1, sh_inp)
    lay.n_expert_used, lay.norm_weights, lay.weights_scale = k_n, 1, 1.0

    n_all = args.warmup + args.steps
    mrng = np.random.default_rng(args.seed)
    perm = mrng.permutation(E_n)
    if args.popularity == "offset":
        rank = np.empty(E_n, np.float64)
        rank[perm] = np.arange(1, E_n + 1)
        rm = torch.from_numpy(np.tile((-skew * np.log(rank)).astype(np.float32), (n_all, T, 1))).to(dev)
    else:
        p = 1.0 / np.arange(1, E_n + 1) ** skew
        p /= p.sum()
        m = np.zeros((n_all, T, E_n), np.float32)
        for s in range(n_all):
            for t in range(T):
                m[s, t, perm[mrng.choice(E_n, k_n, replace=False, p=p)]] = 16.0
        rm = torch.from_numpy(m).to(dev)
    copy = torch.cuda.Stream()
    host_ptrs = [(ctypes.c_void_p * 1)(host[r].data_ptr()) for r in range(3)]
    xs = torch.randn((n_all, T, H), device=dev)
    ws = torch.empty(L.qwm_moe_workspace_size(lay, T), dtype=torch.uint8, device=dev)
    qa.check(L.qwm_workspace_init(ws.data_ptr(), ws.numel(), stream))
    gids = torch.empty((T, k_n), dtype=torch.int32, device=dev)
    gw = torch.empty((T, k_n), dtype=torch.float32, device=dev)
    hid = torch.empty(T * k_n, dtype=torch.int32, pin_memory=True)
    hsl = torch.empty((3, T * k_n), dtype=torch.int32, pin_memory=True)
    dsl = torch.empty((3, T * k_n), dtype=torch.int32, device=dev)
    out = torch.empty((T, H), device=dev)
    t_rms = [qa.tensor(qa.TYPE_F32, E_n, T, 1, rm[s]) for s in range(n_all)]
    t_ids, t_w = qa.tensor(qa.TYPE_I32, k_n, T, 1, gids), qa.tensor(qa.TYPE_F32, k_n, T, 1, gw)
    t_sl = [qa.tensor(qa.TYPE_I32, k_n, T, 1, dsl[r]) for r in range(3)]
    t_out = qa.tensor(qa.TYPE_F32, H, T, 1, out)
    t_xs = [qa.tensor(qa.TYPE_F32, H, T, 1, xs[s]) for s in range(n_all)]
    cur = torch.cuda.current_stream()
    n_ids = T * k_n
    hs = [hsl[r].data_ptr() for r in range(3)]

    def run_mode(fetch):
        """A fresh pool with the given fetch mode over the same inputs.  "file":
        the slabs come from a file (the three roles' expert arrays back to
        back), read by the pool's reader threads; the file was just written,
        so its pages are in the host's page cache (no device I/O is timed), and
        the staged slabs reach the pool by slab-gather launches."""
        d = qa.PoolDesc()
        d.n_layer, d.n_expert = 1, E_n
        for r in range(3):
            d.n_slots[r] = S_n
            d.pool_data[r] = pools[r].data_ptr()
            d.slab_bytes[r] = slab
            d.host_slabs[r] = None if fetch == "file" else ctypes.cast(host_ptrs[r], ctypes.c_void_p)
        d.fetch_mode = qa.FETCH_MEMCPY if fetch == "memcpy" else qa.FETCH_GATHER   # file: gathers from the staging
        pool = ctypes.c_void_p()
        qa.check(L.qwm_pool_create(ctypes.byref(d), ctypes.c_void_p(copy.cuda_stream), ctypes.byref(pool)))
        if fetch == "file":
            fd, path = tempfile.mkstemp(prefix="qwm_slabs_", suffix=".bin")
            with os.fdopen(fd, "wb") as f:
                for r in range(3):
                    f.write(host[r].numpy().tobytes())
            try:
                for r in range(3):
                    qa.check(L.qwm_pool_attach_file(pool, r, 0, path.encode(), r * E_n * slab))
            finally:
                os.unlink(path)   # the pool holds its descriptor
            qa.check(L.qwm_pool_set_io(pool, 8, 0))

        def step(s, ev=None, unions=None):
            if ev is not None:
                ev[0].record(cur)
            qa.check(L.qwm_moe_route(lay, t_xs[s], t_rms[s], t_ids, t_w, ws.data_ptr(), ws.numel(), stream))
            if ev is not None:
                ev[1].record(cur)
            hid.copy_(gids.view(-1), non_blocking=True)
            cur.synchronize()
            if unions is not None:
                unions.append(len(np.unique(hid.numpy())))
            if ev is not None:
                ev[2].record(copy)
            qa.check(L.qwm_pool_ensure(pool, 0, hid.data_ptr(), n_ids, hs[0], hs[1], hs[2]))
            if ev is not None:
                ev[3].record(copy)
            dsl.copy_(hsl, non_blocking=True)
            qa.check(L.qwm_pool_wait(pool, stream))
            if ev is not None:
                ev[4].record(cur)
            qa.check(L.qwm_moe_experts(lay, t_xs[s], t_sl[0], t_sl[1], t_sl[2], t_w, None, t_out, ws.data_ptr(),
                                       ws.numel(), stream))
            if ev is not None:
                ev[5].record(cur)

        for s in range(args.warmup):
            step(s)
        torch.cuda.synchronize()
        st0 = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(pool, ctypes.byref(st0)))
        # timed run: whole-loop events only
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for s in range(args.warmup, n_all):
            step(s)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        st1 = qa.PoolStats()
        qa.check(L.qwm_pool_get_stats(pool, ctypes.byref(st1)))
        # breakdown run over the same inputs again (the pool keeps evolving)
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(args.steps)]
        unions = []
        for i, s in enumerate(range(args.warmup, n_all)):
            step(s, evs[i], unions)
        torch.cuda.synchronize()
        rt = np.array([[ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2]), ev[2].elapsed_time(ev[3]),
                        ev[3].elapsed_time(ev[4]), ev[4].elapsed_time(ev[5])] for ev in evs])
        L.qwm_pool_destroy(pool)
        lookups = (st1.hits + st1.misses) - (st0.hits + st0.misses)
        misses = st1.misses - st0.misses
        miss_bytes = (st1.fetch_bytes - st0.fetch_bytes) / args.steps
        copy_ms = rt[:, 2]
        return {"ms": ms, "rt": rt, "union": float(np.mean(unions)),
                "pool": {"hit_rate": 1.0 - misses / max(lookups, 1), "misses_per_step": misses / args.steps / 3,
                         "miss_bytes_per_step": miss_bytes, "evictions": int(st1.evictions - st0.evictions)},
                "breakdown_ms_median": {"route": float(np.median(rt[:, 0])),
                                        "ids_readback": float(np.median(rt[:, 1])),
                                        "ensure_and_copies": float(np.median(rt[:, 2])),
                                        "copies_to_experts_start": float(np.median(rt[:, 3])),
                                        "experts": float(np.median(rt[:, 4]))},
                "host_link_GBs": (miss_bytes * args.steps) / max(float(copy_ms.sum()) * 1e-3, 1e-9) / 1e9}

    cpu = None
    if not args.no_cpu:
        lib = ref_cpu_lib()
        if lib is None:
            cpu = NO_REF
        else:
            # every expert in host memory (the pinned slabs), the shared expert and router copied back
            hs_np = [h.numpy() for h in host]
            sh_np = [q.cpu().numpy() for q in sh]
            rt_np = router.cpu().numpy()
            si_np = sh_inp.cpu().numpy()
            rm_np = rm.cpu().numpy()
            x_np = xs.cpu().numpy()
            a = BlockArgs()
            a.H, a.N, a.E, a.k, a.T, a.n_threads = H, N_n, E_n, k_n, T, CPU_THREADS
            a.router, a.gate, a.up, a.down = rt_np.ctypes.data, hs_np[0].ctypes.data, hs_np[1].ctypes.data, hs_np[2].ctypes.data
            a.sh_gate, a.sh_up, a.sh_down, a.sh_inp = (sh_np[0].ctypes.data, sh_np[1].ctypes.data, sh_np[2].ctypes.data,
                                                       si_np.ctypes.data)
            ids_c = np.zeros((T, k_n), np.int32)
            out_c = np.zeros((T, H), np.float32)
            a.ids, a.out = ids_c.ctypes.data, out_c.ctypes.data

            def cpu_step(i):
                s_ = args.warmup + i % args.steps
                xi = np.ascontiguousarray(x_np[s_])
                ri = np.ascontiguousarray(rm_np[s_])
                a.x, a.rm = xi.ctypes.data, ri.ctypes.data
                lib.qwr_cpu_moe_block(ctypes.byref(a))

            n, secs = timed_sample(cpu_step, args.cpu_seconds)
            cpu = {"value": T * n / secs, "unit": "tokens/s", "cores": CPU_THREADS, "kind": "reference",
                   "sample": f"{n} verify steps ({secs:.1f} s) of the same inputs through the reference's ggml-CPU "
                             f"kernels with every expert in host memory ({CPU_THREADS} OpenMP threads)",
                   "ms_per_step": 1e3 * secs / n}
    others = {m: run_mode(m) for m in ("gather", "memcpy", "file") if m != args.fetch}
    res = run_mode(args.fetch)
    rt = res["rt"]
    kern_ms = float(np.median(rt[:, 0]) + np.median(rt[:, 4]))
    step_bytes = 3 * slab * res["union"] + E_n * H * 4 + 3 * slab + 2 * T * H * 4
    gbs = step_bytes / (kern_ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "MoE verify tokens/s with LRU slot-pool miss fills, one Qwen3-Next-shape layer, 1xMI355X",
        "value": T / (res["ms"] * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": res["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "MTP verify T=4 through one Qwen3-Next-shape MoE layer (H 2048, 512 experts + shared, "
                               "FFN 512, top-10, Q4_K) with a 128-slot LRU pool per role, experts in pinned host "
                               "memory, Zipf(1.1) popularity through the route mask",
                   "pool_slots": S_n, "skew": skew, "popularity": args.popularity, "fetch": args.fetch,
                   "distinct_experts_per_step": res["union"]},
        "pool": res["pool"],
        "breakdown_ms_median": res["breakdown_ms_median"],
        "host_link": {"achieved_GBs": res["host_link_GBs"], "peak_GBs": 64.0},
        "other_fetch": {m: {"ms_per_step": o["ms"], "tokens_per_s": T / (o["ms"] * 1e-3),
                            "host_link_GBs": o["host_link_GBs"], "hit_rate": o["pool"]["hit_rate"],
                            "breakdown_ms_median": o["breakdown_ms_median"]} for m, o in others.items()},
        "roofline": {"bound": "hbm", "kernel": "route + experts (selected slabs, router, shared expert)",
                     "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "bytes_per_launch": step_bytes},
        "cpu_baseline": cpu,
    }))


class StepArgs(ctypes.Structure):
    _fields_ = [("H", ctypes.c_int64), ("N", ctypes.c_int64), ("E", ctypes.c_int64), ("k", ctypes.c_int64),
                ("T", ctypes.c_int64), ("V", ctypes.c_int64), ("router", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("up", ctypes.c_void_p), ("down", ctypes.c_void_p), ("lm_head", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("drafts", ctypes.c_void_p), ("ids", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("vA", ctypes.c_void_p), ("accepted", ctypes.c_void_p), ("n_threads", ctypes.c_int)]


class BlockArgs(ctypes.Structure):
    """qwr_block_args of oracle/ref_harness/cpu_step.cpp."""
    _fields_ = [("H", ctypes.c_int64), ("N", ctypes.c_int64), ("E", ctypes.c_int64), ("k", ctypes.c_int64),
                ("T", ctypes.c_int64), ("router", ctypes.c_void_p), ("rm", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("up", ctypes.c_void_p), ("down", ctypes.c_void_p), ("sh_gate", ctypes.c_void_p),
                ("sh_up", ctypes.c_void_p), ("sh_down", ctypes.c_void_p), ("sh_inp", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("out", ctypes.c_void_p), ("ids", ctypes.c_void_p), ("n_threads", ctypes.c_int)]


def ref_cpu_lib():
    """The reference's ggml-CPU kernels with the step/block harness (oracle/_ref), or None."""
    so = os.path.join(ROOT, "oracle", "_ref", "libggml_leaf.so")
    if not os.path.exists(so):
        return None
    lib = ctypes.CDLL(so)
    lib.qwr_cpu_verify_step.argtypes = [ctypes.POINTER(StepArgs)]
    lib.qwr_cpu_moe_block.argtypes = [ctypes.POINTER(BlockArgs)]
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.qwr_cpu_mul_mat_id.argtypes = [P, I, I, I, P, I, I, P, I, P, ctypes.c_int]
    return lib


def timed_sample(fn, seconds, max_runs=100000):
    """One untimed warm-up call, then calls until `seconds` are spent; returns (runs, seconds)."""
    fn(0)
    n, t_total = 0, 0.0
    while t_total < seconds and n < max_runs:
        t0 = time.perf_counter()
        fn(n + 1)
        t_total += time.perf_counter() - t0
        n += 1
    return n, t_total


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


NO_REF = {"value": None, "unit": "tokens/s", "cores": 0, "kind": "reference", "sample": "oracle/_ref not built"}
CPU_THREADS = 16


def cpu_baseline(args, torch, pools, router, lm, xs, drafts, ids_gpu, res_gpu):
    """The same verify steps through the reference's own ggml-CPU kernels
    (oracle/_ref, compiled from the reference sources), timed on this host."""
    so = os.path.join(ROOT, "oracle", "_ref", "libggml_leaf.so")
    if not os.path.exists(so):
        return {"value": None, "unit": "tokens/s", "cores": 0, "kind": "reference", "sample": "oracle/_ref not built"}
    lib = ctypes.CDLL(so)
    lib.qwr_cpu_verify_step.argtypes = [ctypes.POINTER(StepArgs)]
    g, u, d = (p.cpu().numpy() for p in pools)
    rt = router.cpu().numpy()
    lmh = lm.cpu().numpy()
    threads = min(16, os.cpu_count() or 1)
    x_np = xs.cpu().numpy()
    dr = drafts.cpu().numpy()
    ids_ref = ids_gpu.cpu().numpy()
    res_ref = res_gpu.cpu().numpy()
    a = StepArgs()
    a.H, a.N, a.E, a.k, a.T, a.V = H, N, E, K_USED, T, V
    a.router, a.gate, a.up, a.down, a.lm_head = rt.ctypes.data, g.ctypes.data, u.ctypes.data, d.ctypes.data, lmh.ctypes.data
    a.n_threads = threads
    ids = np.zeros((T, K_USED), np.int32)
    out = np.zeros((T, H), np.float32)
    vA = np.zeros(T, np.int32)
    acc = ctypes.c_int32()
    a.ids, a.out, a.vA, a.accepted = ids.ctypes.data, out.ctypes.data, vA.ctypes.data, ctypes.addressof(acc)
    s0 = args.warmup
    # one untimed warm-up step, then the timed steps (cycling over the bench's
    # step inputs) until the time budget is spent
    n_run, steps, agree, t_total = 0, 0, 0, 0.0
    while True:
        s = s0 + n_run % args.steps
        xi = np.ascontiguousarray(x_np[s])
        di = np.ascontiguousarray(dr[s])
        a.x, a.drafts = xi.ctypes.data, di.ctypes.data
        t0 = time.perf_counter()
        lib.qwr_cpu_verify_step(ctypes.byref(a))
        dt = time.perf_counter() - t0
        if n_run > 0:
            t_total += dt
            steps += 1
        n_run += 1
        agree += int(np.array_equal(np.sort(ids, 1), np.sort(ids_ref[s], 1)) and np.array_equal(vA, res_ref[s][:T]))
        if t_total >= args.cpu_seconds or steps >= 20000:
            break
    return {"value": T * steps / t_total, "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"{steps} verify steps ({t_total:.1f} s) of the same workload through the reference's "
                      f"ggml-CPU kernels (x86-64 AVX-512 build, {threads} OpenMP threads); "
                      f"{agree}/{n_run} steps gave the GPU's expert ids and argmaxes",
            "ms_per_step": 1e3 * t_total / steps}


if __name__ == "__main__":
    main()
