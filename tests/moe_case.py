"""Seeded synthetic MoE layers for the parity tests: weights quantized on the
CPU by the oracle (bit-identical to ggml's quantize_q4_K / quantize_q8_0), uploaded with
torch, and the matching oracle results.  Shapes follow the workloads:
Qwen3-30B-A3B (H 2048, 128 experts, FFN 768, top-8) and Qwen3-Next
(H 2048, 512 experts + shared, FFN 512, top-10); the slot pools hold a few
slots so that fixtures stay small, with selected experts mapped to slots."""
import ctypes

import numpy as np

import questwend_amd as qa
from tests.helpers import (GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_Q8_0, I64, F32, oracle, ptr, quantize_q4_K,
                           quantize_q8_0_model, random_q5_K, random_q6_K)


class QwoMoeArgs(ctypes.Structure):
    _fields_ = [("H", ctypes.c_int64), ("N", ctypes.c_int64), ("k", ctypes.c_int64), ("T", ctypes.c_int64),
                ("weight_type", ctypes.c_int), ("gate_pool", ctypes.c_void_p), ("up_pool", ctypes.c_void_p),
                ("down_pool", ctypes.c_void_p), ("n_slots", ctypes.c_int64), ("slot_g", ctypes.c_void_p),
                ("slot_u", ctypes.c_void_p), ("slot_d", ctypes.c_void_p), ("weights", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("sh_gate", ctypes.c_void_p), ("sh_up", ctypes.c_void_p),
                ("sh_down", ctypes.c_void_p), ("N_sh", ctypes.c_int64), ("sh_gate_inp", ctypes.c_void_p),
                ("out", ctypes.c_void_p), ("gate_out", ctypes.c_void_p), ("up_out", ctypes.c_void_p),
                ("act_out", ctypes.c_void_p), ("experts_out", ctypes.c_void_p), ("down_type", ctypes.c_int)]


class MoeCase:
    def __init__(self, seed, H=2048, N=768, E=128, k=8, S=16, shared=False, N_sh=512, sh_gate=True, wtype="q4_K",
                 down="same", gating=1, bias=0.0):
        """wtype: "q4_K" or "q8_0" expert slabs (the model-file quantizers), or
        "q5_K" (random valid blocks);
        down="q6_K": random Q6_K down slabs (routed and shared) beside Q4_K
        gate/up, as Q4_K_M model files store some layers;
        gating: 1 soft_max, 2 sigmoid routing; bias > 0: an exp_probs_b
        ranking bias drawn N(0, bias^2)."""
        rng = np.random.default_rng(seed)
        assert wtype in ("q4_K", "q8_0", "q5_K") and down in ("same", "q6_K")
        self.wtype = wtype
        self.ggml_type = {"q4_K": GGML_Q4_K, "q8_0": GGML_Q8_0, "q5_K": GGML_Q5_K}[wtype]
        self.qa_type = {"q4_K": qa.TYPE_Q4_K, "q8_0": qa.TYPE_Q8_0, "q5_K": qa.TYPE_Q5_K}[wtype]
        if wtype == "q5_K":        # random valid blocks (every 5-bit value, scale and min occurs)
            def quantize(w):
                return random_q5_K(rng, int(np.prod(w.shape[:-1])), w.shape[-1], 1e-4)
        else:
            quantize = quantize_q4_K if wtype == "q4_K" else quantize_q8_0_model
        self.H, self.N, self.E, self.k, self.S = H, N, E, k, S
        self.shared, self.N_sh, self.has_sh_gate = shared, N_sh, sh_gate
        self.router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        self.gating = gating
        self.bias = (rng.standard_normal(E) * bias).astype(np.float32) if bias > 0 else None
        self.gate_q = quantize((rng.standard_normal((S, N, H)) * 0.02).astype(np.float32))
        self.up_q = quantize((rng.standard_normal((S, N, H)) * 0.02).astype(np.float32))
        self.down_q = quantize((rng.standard_normal((S, H, N)) * 0.02).astype(np.float32))
        self.down_ggml, self.down_qa = self.ggml_type, self.qa_type
        if down == "q6_K":
            self.down_q = random_q6_K(rng, S * H, N, 1e-4)
            self.down_ggml, self.down_qa = GGML_Q6_K, qa.TYPE_Q6_K
        if shared:
            self.shg_q = quantize((rng.standard_normal((N_sh, H)) * 0.02).astype(np.float32))
            self.shu_q = quantize((rng.standard_normal((N_sh, H)) * 0.02).astype(np.float32))
            self.shd_q = quantize((rng.standard_normal((H, N_sh)) * 0.02).astype(np.float32))
            if down == "q6_K":
                self.shd_q = random_q6_K(rng, H, N_sh, 1e-4)
            self.sh_inp = (rng.standard_normal(H) * 0.02).astype(np.float32) if sh_gate else None
        self.rng = rng

    # ---------------------------------------------------------------- oracle --
    def route(self, x, rm=None):
        T = x.shape[0]
        ids = np.zeros((T, self.k), np.int32)
        w = np.zeros((T, self.k), np.float32)
        mg = np.zeros(T, np.float32)
        lg = np.zeros((T, self.E), np.float32)
        assert oracle().qwo_route_ex(I64(self.E), I64(self.H), I64(T), ptr(self.router), ptr(x),
                                     ptr(rm) if rm is not None else None,
                                     ptr(self.bias) if self.bias is not None else None, self.gating, self.k, 1,
                                     F32(1.0), ptr(ids), ptr(w), ptr(lg), None, ptr(mg)) == 0
        return ids, w, mg, lg

    def block(self, x, slots, weights):
        """Oracle MoE block with the given slot ids (same for the 3 roles)."""
        T = x.shape[0]
        out = np.zeros((T, self.H), np.float32)
        a = QwoMoeArgs()
        a.H, a.N, a.k, a.T = self.H, self.N, self.k, T
        a.weight_type = self.ggml_type
        a.down_type = self.down_ggml
        a.gate_pool, a.up_pool, a.down_pool = self.gate_q.ctypes.data, self.up_q.ctypes.data, self.down_q.ctypes.data
        a.n_slots = self.S
        slots = np.ascontiguousarray(slots, np.int32)
        a.slot_g = a.slot_u = a.slot_d = slots.ctypes.data
        weights = np.ascontiguousarray(weights, np.float32)
        a.weights = weights.ctypes.data
        a.x = x.ctypes.data
        if self.shared:
            a.sh_gate, a.sh_up, a.sh_down = self.shg_q.ctypes.data, self.shu_q.ctypes.data, self.shd_q.ctypes.data
            a.N_sh = self.N_sh
            a.sh_gate_inp = self.sh_inp.ctypes.data if self.sh_inp is not None else None
        a.out = out.ctypes.data
        assert oracle().qwo_moe_block(ctypes.byref(a)) == 0
        return out

    # ------------------------------------------------------------------- GPU --
    def upload(self, torch):
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        self.d_router = dev(self.router)
        self.d_gate, self.d_up, self.d_down = dev(self.gate_q), dev(self.up_q), dev(self.down_q)
        L = qa.MoeLayer()
        L.gate_pool = qa.tensor(self.qa_type, self.H, self.N, self.S, self.d_gate)
        L.up_pool = qa.tensor(self.qa_type, self.H, self.N, self.S, self.d_up)
        L.down_pool = qa.tensor(self.down_qa, self.N, self.H, self.S, self.d_down)
        L.router = qa.tensor(qa.TYPE_F32, self.H, self.E, 1, self.d_router)
        if self.shared:
            self.d_shg, self.d_shu, self.d_shd = dev(self.shg_q), dev(self.shu_q), dev(self.shd_q)
            L.sh_gate = qa.tensor(self.qa_type, self.H, self.N_sh, 1, self.d_shg)
            L.sh_up = qa.tensor(self.qa_type, self.H, self.N_sh, 1, self.d_shu)
            L.sh_down = qa.tensor(self.down_qa, self.N_sh, self.H, 1, self.d_shd)
            if self.sh_inp is not None:
                self.d_shinp = dev(self.sh_inp)
                L.sh_gate_inp = qa.tensor(qa.TYPE_F32, self.H, 1, 1, self.d_shinp)
        L.n_expert_used = self.k
        L.norm_weights = 1
        L.weights_scale = 1.0
        L.gating_func = self.gating
        if self.bias is not None:
            self.d_bias = dev(self.bias)
            L.exp_probs_b = qa.tensor(qa.TYPE_F32, self.E, 1, 1, self.d_bias)
        self.layer = L
        return L


def rel_err(got, exp):
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    return float(np.linalg.norm(got - exp) / max(np.linalg.norm(exp), 1e-30))
