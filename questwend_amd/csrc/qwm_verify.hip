// qwm_verify.hip -- the MTP verify head on gfx950: rms_norm + x86 Q8_0
// activation quantization, the Q8_0 lm_head GEMV with a fused running argmax,
// and the greedy acceptance check.
//
// lm_head rows are 2176 bytes (64 blocks of 34 bytes); lane b of a wave owns
// block b of the row.  A 34-byte block starts on a 4-byte boundary for even b
// and 2 bytes past one for odd b, so each lane loads the 9 aligned dwords
// covering its block and shifts the quant bytes into place; the weight bytes
// of a row are therefore read by 64 lanes in one coalesced sweep.
#include "qwm_device.h"
#include "qwm_internal.h"

namespace qwm {

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int VH_MAX_T = MAX_T;
constexpr int LM_ROWS_PER_WAVE = 16;
constexpr int LM_STEPS = 4;          // rows whose loads are in flight together

// h = rms_norm(x) * norm_w (ggml-cpu/ops.cpp:4120-4160: sum of float squares
// in double, mean rounded to float, scale = 1/sqrtf(mean + eps)), then the x86
// Q8_0 quantizer (ggml-cpu/arch/x86/quants.c:302-345): d = amax/127 stored as
// fp16, q = round-half-even(h * 127/amax).  One block of 256 threads per token.
__global__ void __launch_bounds__(256) k_vhead_prep(const float * __restrict__ x, const float * __restrict__ norm_w,
                                                     float eps, int H, int8_t * __restrict__ hq, float * __restrict__ hd) {
    __shared__ double part[4];
    __shared__ float s_scale;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float * xt = x + (size_t)t * H;
    double acc = 0.0;
    for (int i = tid; i < H; i += 256) {
        const float v = xt[i];
        acc += (double)(v * v);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (tid == 0) {
        const double sum = (part[0] + part[1]) + (part[2] + part[3]);
        const float mean = (float)(sum / (double)H);
        s_scale = 1.0f / sqrtf(mean + eps);
    }
    __syncthreads();
    const float scale = s_scale;
    // one 32-value block per 32 lanes (a half wave)
    const int half = lane >> 5, l = lane & 31;
    for (int b = wave * 2 + half; b < H / QK8_0; b += 8) {
        const int i = b * QK8_0 + l;
        float v = xt[i] * scale;
        if (norm_w) v = v * norm_w[i];
        float amax = __builtin_fabsf(v);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, WAVE));
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        hq[(size_t)t * H + i] = (int8_t)(int)__builtin_rintf(v * id);
        if (l == 0) hd[(size_t)t * (H / QK8_0) + b] = fp16_to_f32(f32_to_fp16(d));
    }
}

// logits[t][r] = sum_b d_w(r,b) * d_h(t,b) * sum_32 q_w * q_h; keeps, per token,
// the running maximum (ties: larger row index, ggml-cpu/vec.h:1618-1626).
template <int NT>
__global__ void __launch_bounds__(256) k_lmhead_argmax(const uint8_t * __restrict__ W, int H, int V,
                                                        const int8_t * __restrict__ hq, const float * __restrict__ hd,
                                                        float * __restrict__ pv, int32_t * __restrict__ pi) {
    __shared__ float s_v[4][NT];
    __shared__ int32_t s_i[4][NT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nblk = H / QK8_0;                 // 64 for H = 2048
    const size_t row_bytes = (size_t)nblk * 34;
    const bool act = lane < nblk;
    // activations of every token for this lane's block
    uint32_t aq[NT][8];
    float ad[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (act) {
            const uint4 * q = reinterpret_cast<const uint4 *>(hq + (size_t)t * H + lane * QK8_0);
            const uint4 q0 = q[0], q1 = q[1];
            aq[t][0] = q0.x; aq[t][1] = q0.y; aq[t][2] = q0.z; aq[t][3] = q0.w;
            aq[t][4] = q1.x; aq[t][5] = q1.y; aq[t][6] = q1.z; aq[t][7] = q1.w;
            ad[t] = hd[(size_t)t * nblk + lane];
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) aq[t][i] = 0;
            ad[t] = 0.f;
        }
    }
    float best[NT];
    int besti[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { best[t] = -__builtin_inff(); besti[t] = -1; }

    const int r_begin = (blockIdx.x * 4 + wave) * LM_ROWS_PER_WAVE;
    const size_t off = (size_t)(lane * 34) & ~(size_t)3;
    const int shift = (lane & 1) ? 32 : 16;     // bit offset of the quants in the 9-dword window
    for (int r0 = r_begin; r0 < min(r_begin + LM_ROWS_PER_WAVE, V); r0 += LM_STEPS) {
        uint32_t win[LM_STEPS][9];
#pragma unroll
        for (int s = 0; s < LM_STEPS; ++s) {
            const int r = r0 + s;
            if (act && r < V) {
                const uint32_t * p = reinterpret_cast<const uint32_t *>(W + (size_t)r * row_bytes + off);
                const u32x4_a4 v0 = *reinterpret_cast<const u32x4_a4 *>(p);
                const u32x4_a4 v1 = *reinterpret_cast<const u32x4_a4 *>(p + 4);
                win[s][0] = v0.x; win[s][1] = v0.y; win[s][2] = v0.z; win[s][3] = v0.w;
                win[s][4] = v1.x; win[s][5] = v1.y; win[s][6] = v1.z; win[s][7] = v1.w;
                win[s][8] = p[8];
            } else {
#pragma unroll
                for (int i = 0; i < 9; ++i) win[s][i] = 0;
            }
        }
#pragma unroll
        for (int s = 0; s < LM_STEPS; ++s) {
            const int r = r0 + s;
            const uint16_t dbits = (lane & 1) ? (uint16_t)(win[s][0] >> 16) : (uint16_t)(win[s][0] & 0xffff);
            const float dw = fp16_to_f32(dbits);
            uint32_t wq[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint64_t pair = ((uint64_t)win[s][i + 1] << 32) | win[s][i];
                wq[i] = (uint32_t)(pair >> shift);
            }
            float lg[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                int isum = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) isum = dot4(wq[i], aq[t][i], isum);
                lg[t] = act ? (dw * ad[t]) * (float)isum : 0.f;
                lg[t] = group_sum<64>(lg[t]);
                if (r < V && (lg[t] > best[t] || (lg[t] == best[t] && r > besti[t]))) { best[t] = lg[t]; besti[t] = r; }
            }
        }
    }
    if (lane == 0)
        for (int t = 0; t < NT; ++t) { s_v[wave][t] = best[t]; s_i[wave][t] = besti[t]; }
    __syncthreads();
    if (threadIdx.x < NT) {
        const int t = threadIdx.x;
        float v = s_v[0][t];
        int i = s_i[0][t];
        for (int w = 1; w < 4; ++w)
            if (s_v[w][t] > v || (s_v[w][t] == v && s_i[w][t] > i)) { v = s_v[w][t]; i = s_i[w][t]; }
        pv[(size_t)blockIdx.x * NT + t] = v;
        pi[(size_t)blockIdx.x * NT + t] = i;
    }
}

// vA[t] = argmax over the per-block partials; then the accept rule of
// core/runtime.cpp:3648-3652.  One block, one wave per token.
__global__ void __launch_bounds__(512) k_accept(const float * __restrict__ pv, const int32_t * __restrict__ pi,
                                                 int n_wg, int NT, const int32_t * __restrict__ drafts, int32_t * __restrict__ result) {
    __shared__ int32_t vA[VH_MAX_T];
    const int lane = threadIdx.x & 63, t = threadIdx.x >> 6;
    if (t < NT) {
        float v = -__builtin_inff();
        int idx = -1;
        for (int b = lane; b < n_wg; b += 64) {
            const float ov = pv[(size_t)b * NT + t];
            const int oi = pi[(size_t)b * NT + t];
            if (ov > v || (ov == v && oi > idx)) { v = ov; idx = oi; }
        }
        wave_argmax_last(v, idx);
        if (lane == 0) vA[t] = idx < 0 ? 0 : idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int a = 0;
        while (a < NT - 1 && vA[a] == drafts[a]) ++a;
        for (int i = 0; i < NT; ++i) result[i] = vA[i];
        result[NT] = a;
        result[NT + 1] = vA[a];
    }
}

bool verify_plan(const qwm_tensor * lm_head, int64_t T, VerifyPlan & p, std::string & why) {
    p.H = lm_head->ne[0];
    p.V = lm_head->ne[1];
    p.T = T;
    if (lm_head->type != T_Q8_0) { why = "lm_head must be Q8_0"; return false; }
    if (p.H % QK8_0 || p.H / QK8_0 > 64) { why = "lm_head: H must be a multiple of 32, <= 2048"; return false; }
    if (T < 1 || T > VH_MAX_T) { why = "verify batch must hold 1..8 tokens"; return false; }
    p.n_wg = (int)((p.V + 4 * LM_ROWS_PER_WAVE - 1) / (4 * LM_ROWS_PER_WAVE));
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    p.counters = take(256);
    p.hq = take((size_t)T * p.H + sizeof(float) * T * (p.H / QK8_0));
    p.partial_v = take(sizeof(float) * p.n_wg * T);
    p.partial_i = take(sizeof(int32_t) * p.n_wg * T);
    p.total = o;
    return true;
}

int launch_verify(const uint8_t * lm_head, const float * x, const float * norm_w, float eps,
                  const int32_t * drafts, int32_t * result, const VerifyPlan & p, uint8_t * ws, hipStream_t s) {
    int8_t * hq = reinterpret_cast<int8_t *>(ws + p.hq);
    float * hd = reinterpret_cast<float *>(ws + p.hq + align_up((size_t)p.T * p.H, 16));
    float * pv = reinterpret_cast<float *>(ws + p.partial_v);
    int32_t * pi = reinterpret_cast<int32_t *>(ws + p.partial_i);
    QWM_TIMED("vhead_prep", s, k_vhead_prep<<<dim3((unsigned)p.T), 256, 0, s>>>(x, norm_w, eps, (int)p.H, hq, hd));
    const dim3 grid((unsigned)p.n_wg);
    prof_begin("lm_head", s);
    switch (p.T) {
        case 1: k_lmhead_argmax<1><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        case 2: k_lmhead_argmax<2><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        case 3: k_lmhead_argmax<3><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        case 4: k_lmhead_argmax<4><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        case 5: k_lmhead_argmax<5><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        case 6: k_lmhead_argmax<6><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        case 7: k_lmhead_argmax<7><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
        default: k_lmhead_argmax<8><<<grid, 256, 0, s>>>(lm_head, (int)p.H, (int)p.V, hq, hd, pv, pi); break;
    }
    prof_end("lm_head", s);
    QWM_TIMED("accept", s, k_accept<<<1, 512, 0, s>>>(pv, pi, p.n_wg, (int)p.T, drafts, result));
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
