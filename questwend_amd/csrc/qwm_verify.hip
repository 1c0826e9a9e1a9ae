// qwm_verify.hip -- the MTP verify head on gfx950 in one kernel: rms_norm +
// x86 Q8_0 activation quantization, the Q8_0 lm_head GEMV with a running
// argmax, and (in the last block to finish) the cross-block argmax and the
// greedy acceptance check.
//
// Work split: a fixed grid of a few blocks per CU; block g owns a contiguous
// slice of vocabulary rows and its four waves stream it in steps of 4*RPS
// rows.  A row of the Q8_0 lm_head is 64 blocks of 34 bytes (2176 bytes);
// each lane owns BPL consecutive blocks (BPL = 2: 68 bytes, dword aligned;
// BPL = 1: the 9 aligned dwords around its block), so 64/BPL lanes cover a
// row and one wave step covers BPL rows.  Every lane keeps its blocks' Q8_0
// activations of all tokens in registers; the per-row sum over lanes is a
// DPP reduction within 16-lane rows plus four lane reads.  Weight loads run
// PF steps ahead of the arithmetic.
#include "qwm_device.h"
#include "qwm_internal.h"

namespace qwm {

constexpr int VH_MAX_T = MAX_T;
constexpr int VH_PF = 3;            // weight buffers: two steps stay in flight while one is consumed

struct VerifyArgs {
    const uint8_t * W; int H, V;
    const float * x; const float * norm_w; float eps;
    const int32_t * drafts; int32_t * result;
    float * pv; int32_t * pi; int32_t * counter;
};

template <int BPL> struct Win { static constexpr int N = BPL == 1 ? 9 : 17 * BPL / 2; };

// Loads the dword-aligned window holding this lane's BPL blocks of `row`
// (always in bounds: callers clamp the row and the lane's block group).
template <int BPL>
QWM_DEV void load_window(uint32_t (&w)[Win<BPL>::N], const uint8_t * row, int j) {
    constexpr int NW = Win<BPL>::N;
    const uint32_t * p = reinterpret_cast<const uint32_t *>(row + ((size_t)(34 * BPL * j) & ~(size_t)3));
    typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
#pragma unroll
    for (int i = 0; i + 4 <= NW; i += 4) {
        const u32x4_a4 v = *reinterpret_cast<const u32x4_a4 *>(p + i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
#pragma unroll
    for (int i = NW & ~3; i < NW; ++i) w[i] = p[i];
}

// Quant dwords and scale of block b (0 <= b < BPL) of the window.
template <int BPL>
QWM_DEV void block_from_window(const uint32_t (&w)[Win<BPL>::N], int b, int odd, uint32_t (&q)[8], float & d) {
    if (BPL == 1) {
        const int sh = odd ? 32 : 16;
        d = fp16_to_f32(odd ? (uint16_t)(w[0] >> 16) : (uint16_t)(w[0] & 0xffff));
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = (uint32_t)((((uint64_t)w[i + 1] << 32) | w[i]) >> sh);
    } else {
        // block b starts at byte 34*b of a dword-aligned window
        const int o = 34 * b;
        const int dw = o >> 2;
        if ((o & 3) == 0) {
            d = fp16_to_f32((uint16_t)(w[dw] & 0xffff));
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = __builtin_amdgcn_alignbit(w[dw + i + 1], w[dw + i], 16);
        } else {
            d = fp16_to_f32((uint16_t)(w[dw] >> 16));
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = w[dw + 1 + i];
        }
    }
}

template <int NT, int BPL>
__global__ void __launch_bounds__(256) k_verify_head(VerifyArgs a) {
    constexpr int LPR = 64 / BPL;     // lanes per row
    constexpr int RPS = BPL;          // rows per wave step
    constexpr int NW = Win<BPL>::N;
    __shared__ double s_part[4][NT];
    __shared__ float s_scale[NT];
    __shared__ float s_bv[4][NT];
    __shared__ int32_t s_bi[4][NT];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane % LPR, rsub = lane / LPR;
    const int H = a.H, V = a.V, nblk = H / QK8_0;
    const size_t row_bytes = (size_t)nblk * 34;
    const bool lane_ok = BPL * j < nblk;
    const int jc = lane_ok ? j : (nblk / BPL - 1);        // clamped block group (H < 2048)

    const int64_t rb = (int64_t)blockIdx.x * V / gridDim.x, re = (int64_t)(blockIdx.x + 1) * V / gridDim.x;
    const int n_steps = (int)((re - rb + 4 * RPS - 1) / (4 * RPS));
    auto row_ptr = [&](int s) {
        int64_t r = rb + (int64_t)s * 4 * RPS + wave * RPS + rsub;
        r = r < re ? r : re - 1;                              // clamped: loads stay in bounds
        return a.W + r * row_bytes;
    };

    // weight loads for the first steps go out before the activation work
    uint32_t win[VH_PF][NW];
#pragma unroll
    for (int p = 0; p < VH_PF; ++p) load_window<BPL>(win[p], row_ptr(p), jc);

    // ---- h = rms_norm(x) * norm_w (ggml-cpu/ops.cpp:4120-4160), then the x86
    // Q8_0 quantizer (ggml-cpu/arch/x86/quants.c:302-345) for this lane's blocks
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        double acc = 0.0;
        for (int i = tid; i < H; i += 256) {
            const float v = a.x[(size_t)t * H + i];
            acc += (double)(v * v);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
        if (lane == 0) s_part[wave][t] = acc;
    }
    __syncthreads();
    if (tid < NT) {
        const double sum = (s_part[0][tid] + s_part[1][tid]) + (s_part[2][tid] + s_part[3][tid]);
        const float mean = (float)(sum / (double)H);
        s_scale[tid] = 1.0f / sqrtf(mean + a.eps);
    }
    __syncthreads();
    // one (token, block) per thread: quantize into LDS, shared by the 4 waves
    __shared__ uint4 s_q[NT][64][2];
    __shared__ float s_d[NT][64];
#pragma unroll 1
    for (int tb = tid; tb < NT * nblk; tb += 256) {
        const int t = tb / nblk, blk = tb % nblk;
        const float sc = s_scale[t];
        const float4 * src = reinterpret_cast<const float4 *>(a.x + (size_t)t * H + blk * QK8_0);
        float y[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = src[i];
            y[4 * i + 0] = v.x * sc; y[4 * i + 1] = v.y * sc; y[4 * i + 2] = v.z * sc; y[4 * i + 3] = v.w * sc;
        }
        if (a.norm_w) {
            const float4 * nw = reinterpret_cast<const float4 *>(a.norm_w + blk * QK8_0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 g = nw[i];
                y[4 * i + 0] = y[4 * i + 0] * g.x; y[4 * i + 1] = y[4 * i + 1] * g.y;
                y[4 * i + 2] = y[4 * i + 2] * g.z; y[4 * i + 3] = y[4 * i + 3] * g.w;
            }
        }
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, __builtin_fabsf(y[i]));
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        uint32_t pk[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t packed = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) packed |= (uint32_t)((int)__builtin_rintf(y[4 * i + k] * id) & 0xff) << (8 * k);
            pk[i] = packed;
        }
        s_q[t][blk][0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        s_q[t][blk][1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        s_d[t][blk] = fp16_to_f32(f32_to_fp16(d));
    }
    __syncthreads();
    uint32_t aq[NT][BPL][8];
    float ad[NT][BPL];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int b = 0; b < BPL; ++b) {
            const int blk = min(BPL * j + b, nblk - 1);
            const uint4 q0 = s_q[t][blk][0], q1 = s_q[t][blk][1];
            aq[t][b][0] = q0.x; aq[t][b][1] = q0.y; aq[t][b][2] = q0.z; aq[t][b][3] = q0.w;
            aq[t][b][4] = q1.x; aq[t][b][5] = q1.y; aq[t][b][6] = q1.z; aq[t][b][7] = q1.w;
            ad[t][b] = s_d[t][blk];
        }

    // running argmax per token; every wave scans its rows in increasing order,
    // so ">=" keeps the last maximum (ggml-cpu/vec.h:1618-1626)
    float best[NT];
    int32_t besti[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { best[t] = -__builtin_inff(); besti[t] = -1; }

    const int odd = (34 * BPL * jc) & 2;   // BPL == 1: block starts 2 bytes into its window
    auto consume = [&](const uint32_t (&w)[NW], int s) {
        float part[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) part[t] = 0.f;
#pragma unroll
        for (int b = 0; b < BPL; ++b) {
            uint32_t q[8];
            float dw;
            block_from_window<BPL>(w, b, odd, q, dw);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                int isum = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) isum = dot4(q[i], aq[t][b][i], isum);
                part[t] = __builtin_fmaf(dw * ad[t][b], (float)isum, part[t]);
            }
        }
        const int64_t r0 = rb + (int64_t)s * 4 * RPS + wave * RPS;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float v = row16_sum(lane_ok ? part[t] : 0.f);
#pragma unroll
            for (int rr = 0; rr < RPS; ++rr) {
                float tot = readlane_f(v, rr * LPR);
#pragma unroll
                for (int g = 1; g < LPR / 16; ++g) tot += readlane_f(v, rr * LPR + 16 * g);
                const int64_t r = r0 + rr;
                const bool take = (r < re) & (tot >= best[t]);
                best[t] = take ? tot : best[t];
                besti[t] = take ? (int32_t)r : besti[t];
            }
        }
    };

    int s = 0;
    for (; s + VH_PF <= n_steps; s += VH_PF) {
#pragma unroll
        for (int p = 0; p < VH_PF; ++p) {
            consume(win[p], s + p);
            load_window<BPL>(win[p], row_ptr(min(s + p + VH_PF, n_steps - 1)), jc);
        }
    }
#pragma unroll
    for (int p = 0; p < VH_PF; ++p)
        if (s + p < n_steps) consume(win[p], s + p);

    // ---- block argmax -> partials; the last block reduces them and accepts
    if (lane == 0)
#pragma unroll
        for (int t = 0; t < NT; ++t) { s_bv[wave][t] = best[t]; s_bi[wave][t] = besti[t]; }
    __syncthreads();
    if (tid < NT) {
        float v = s_bv[0][tid];
        int i = s_bi[0][tid];
        for (int w = 1; w < 4; ++w)
            if (s_bv[w][tid] > v || (s_bv[w][tid] == v && s_bi[w][tid] > i)) { v = s_bv[w][tid]; i = s_bi[w][tid]; }
        a.pv[(size_t)blockIdx.x * NT + tid] = v;
        a.pi[(size_t)blockIdx.x * NT + tid] = i;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(a.counter, 1) == (int)gridDim.x - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    __shared__ int32_t vA[NT];
    for (int t = wave; t < NT; t += 4) {
        float v = -__builtin_inff();
        int idx = -1;
        for (int g = lane; g < (int)gridDim.x; g += 64) {
            const float ov = __builtin_nontemporal_load(a.pv + (size_t)g * NT + t);
            const int oi = __builtin_nontemporal_load(a.pi + (size_t)g * NT + t);
            if (ov > v || (ov == v && oi > idx)) { v = ov; idx = oi; }
        }
        wave_argmax_last(v, idx);
        if (lane == 0) vA[t] = idx < 0 ? 0 : idx;
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        while (acc < NT - 1 && vA[acc] == a.drafts[acc]) ++acc;   // runtime.cpp:3648-3652
        for (int i = 0; i < NT; ++i) a.result[i] = vA[i];
        a.result[NT] = acc;
        a.result[NT + 1] = vA[acc];
        *a.counter = 0;
    }
}

static int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
    }
    return cus;
}

bool verify_plan(const qwm_tensor * lm_head, int64_t T, VerifyPlan & p, std::string & why) {
    p.H = lm_head->ne[0];
    p.V = lm_head->ne[1];
    p.T = T;
    if (lm_head->type != T_Q8_0) { why = "lm_head must be Q8_0"; return false; }
    if (p.H % 64 || p.H / QK8_0 > 64) { why = "lm_head: H must be a multiple of 64, <= 2048"; return false; }
    if (T < 1 || T > VH_MAX_T) { why = "verify batch must hold 1..8 tokens"; return false; }
    if (p.V < 1 || p.V > (1LL << 30)) { why = "lm_head: vocabulary size out of range"; return false; }
    p.n_wg = (int)std::min<int64_t>(2 * 256, (p.V + 7) / 8);
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    p.counters = take(256);
    p.hq = 0;
    p.partial_v = take(sizeof(float) * p.n_wg * T);
    p.partial_i = take(sizeof(int32_t) * p.n_wg * T);
    p.total = o;
    return true;
}

template <int NT>
static void launch_nt(const VerifyArgs & a, int n_wg, hipStream_t s) {
    if (NT <= 4) k_verify_head<NT, 2><<<dim3((unsigned)n_wg), 256, 0, s>>>(a);
    else k_verify_head<NT, 1><<<dim3((unsigned)n_wg), 256, 0, s>>>(a);
}

int launch_verify(const uint8_t * lm_head, const float * x, const float * norm_w, float eps,
                  const int32_t * drafts, int32_t * result, const VerifyPlan & p, uint8_t * ws, hipStream_t s) {
    VerifyArgs a;
    a.W = lm_head; a.H = (int)p.H; a.V = (int)p.V;
    a.x = x; a.norm_w = norm_w; a.eps = eps;
    a.drafts = drafts; a.result = result;
    a.pv = reinterpret_cast<float *>(ws + p.partial_v);
    a.pi = reinterpret_cast<int32_t *>(ws + p.partial_i);
    a.counter = reinterpret_cast<int32_t *>(ws + p.counters);
    const int n_wg = std::min(p.n_wg, 2 * device_cus());
    prof_begin("lm_head", s);
    switch (p.T) {
        case 1: launch_nt<1>(a, n_wg, s); break;
        case 2: launch_nt<2>(a, n_wg, s); break;
        case 3: launch_nt<3>(a, n_wg, s); break;
        case 4: launch_nt<4>(a, n_wg, s); break;
        case 5: launch_nt<5>(a, n_wg, s); break;
        case 6: launch_nt<6>(a, n_wg, s); break;
        case 7: launch_nt<7>(a, n_wg, s); break;
        default: launch_nt<8>(a, n_wg, s); break;
    }
    prof_end("lm_head", s);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
