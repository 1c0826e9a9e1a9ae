// qwm_quant.hip -- the model-file quantizers on the GPU: Q4_K
// (quantize_row_q4_K_ref with its make_qkx2_quants search, ggml-quants.c:
// 799-870, 1458-1528) and Q8_0 (quantize_row_q8_0_ref, ggml-quants.c:276-300).
// They produce the bytes ggml's CPU quantizer produces (same operation order,
// with fused multiply-adds exactly where gcc fuses them on x86-64), so large
// synthetic expert slabs and lm_heads can be made on the device.  One thread
// per 256-value block (Q4_K) or per 32-value block (Q8_0).
#include "qwm_device.h"
#include "qwm_internal.h"

namespace qwm {

__device__ float make_qkx2_quants_dev(const float * x, const float * weights, uint8_t * L, float * the_min,
                                      uint8_t * Laux) {
    constexpr int n = 32, nmax = 15, nstep = 20;
    constexpr float rmin = -1.f, rdelta = 0.1f;
    float vmin = x[0], vmax = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < vmin) vmin = x[i];
        if (x[i] > vmax) vmax = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x = __builtin_fmaf(w, x[i], sum_x);
    }
    if (vmin > 0) vmin = 0;
    if (vmax == vmin) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -vmin;
        return 0.f;
    }
    float iscale = nmax / (vmax - vmin);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        const int l = nearest_int_mul(iscale, x[i] - vmin);
        L[i] = (uint8_t)max(0, min(nmax, l));
        float diff = __builtin_fmaf(scale, (float)L[i], vmin) - x[i];
        diff = diff * diff;
        best_error = __builtin_fmaf(weights[i], diff, best_error);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = __builtin_fmaf(rdelta, (float)is, rmin) + nmax;
        iscale = iscale / (vmax - vmin);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int_mul(iscale, x[i] - vmin);
            l = max(0, min(nmax, l));
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            const float wl = w * l;
            sum_l = sum_l + wl;
            sum_l2 = __builtin_fmaf(wl, (float)l, sum_l2);
            sum_xl = __builtin_fmaf(wl, x[i], sum_xl);
        }
        const float D = __builtin_fmaf(sum_w, sum_l2, -(sum_l * sum_l));
        if (D > 0) {
            float this_scale = __builtin_fmaf(-sum_x, sum_l, sum_w * sum_xl) / D;
            float this_min = __builtin_fmaf(sum_l2, sum_x, -(sum_l * sum_xl)) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = __builtin_fmaf(this_scale, (float)Laux[i], this_min) - x[i];
                diff = diff * diff;
                cur_error = __builtin_fmaf(weights[i], diff, cur_error);
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                vmin = this_min;
            }
        }
    }
    *the_min = -vmin;
    return scale;
}

__global__ void __launch_bounds__(128) k_quantize_q4K(const float * __restrict__ src, uint8_t * __restrict__ dst,
                                                       int64_t n_blocks) {
    const int64_t ib = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (ib >= n_blocks) return;
    const float * x = src + ib * QK_K;
    block_q4_K * y = reinterpret_cast<block_q4_K *>(dst) + ib;
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 = sum_x2 + x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + __builtin_fabsf(x[32 * j + l]);
        scales[j] = make_qkx2_quants_dev(x + 32 * j, weights, L + 32 * j, &mins[j], Laux);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t sc[12] = {0};
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nearest_int_mul(inv_scale, scales[j]);
        uint8_t lm = (uint8_t)nearest_int_mul(inv_min, mins[j]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        if (j < 4) { sc[j] = ls; sc[j + 4] = lm; }
        else {
            sc[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4);
            sc[j - 4] |= ((ls >> 4) << 6);
            sc[j - 0] |= ((lm >> 4) << 6);
        }
    }
    const uint16_t dh = f32_to_fp16(max_scale / 63.f), mh = f32_to_fp16(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        int s, m;
        q4k_scale_min(j, sc, s, m);
        const float d = fp16_to_f32(dh) * s;
        if (!d) continue;
        const float dm = fp16_to_f32(mh) * m;
        for (int ii = 0; ii < 32; ++ii) {
            const float v = (x[32 * j + ii] + dm) / d;
            int l = (int)(__float_as_uint(v + 12582912.f) & 0x007fffffu) - 0x00400000;
            L[32 * j + ii] = (uint8_t)max(0, min(15, l));
        }
    }
    y->d = dh;
    y->dmin = mh;
    for (int j = 0; j < 12; ++j) y->scales[j] = sc[j];
    for (int j = 0; j < QK_K; j += 64)
        for (int l = 0; l < 32; ++l) y->qs[j / 2 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
}

__global__ void __launch_bounds__(256) k_quantize_q8_0(const float * __restrict__ src, uint8_t * __restrict__ dst,
                                                        int64_t n_blocks) {
    const int64_t ib = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (ib >= n_blocks) return;
    const float * x = src + ib * QK8_0;
    float amax = 0.f;
    for (int j = 0; j < QK8_0; ++j) amax = fmaxf(amax, __builtin_fabsf(x[j]));
    const float d = amax / 127.f;
    const float id = d ? 1.0f / d : 0.0f;
    uint8_t * y = dst + ib * 34;
    const uint16_t dh = f32_to_fp16(d);
    y[0] = (uint8_t)(dh & 0xff);
    y[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < QK8_0; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

int launch_quantize(int32_t type, const float * src, void * dst, int64_t n, hipStream_t s) {
    if (type == T_Q4_K) {
        const int64_t nb = n / QK_K;
        if (nb) k_quantize_q4K<<<dim3((unsigned)((nb + 127) / 128)), 128, 0, s>>>(src, (uint8_t *)dst, nb);
    } else {
        const int64_t nb = n / QK8_0;
        if (nb) k_quantize_q8_0<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, s>>>(src, (uint8_t *)dst, nb);
    }
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
