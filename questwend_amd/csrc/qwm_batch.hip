// qwm_batch.hip -- the element-wise tail of a batched MoE layer (the seg B of
// decode_cached_batch, core/runtime.cpp:4534-4572) for token counts past the
// decode/verify kernels': SwiGLU over [rows][n], the weighted sum of the
// experts in k order with the shared expert and the residual, and the shared
// expert's sigmoid gate per token.  The GEMMs themselves are MUL_MAT_ID
// launches (qwm_mul_mat_id); these kernels are HBM-bound single passes.
#include "qwm_device.h"
#include "qwm_internal.h"

namespace qwm {

// ggml_swiglu_split on the CPU (ops.cpp:3331-3385, vec.cpp:417-445, AVX-512):
// act = silu(g) * u per element, silu = x / (1 + v_expf(-x)) over the 16-wide
// chunks of each row of n and x / (1 + expf(-x)) (libm) on its scalar tail.
__global__ void __launch_bounds__(256) k_swiglu_rows(const float * g, const float * u, float * act, int n,
                                                     int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int c = (int)(i % n);
    const float x = g[i];
    act[i] = (c < n - (n & 15)) ? v_silu(x) * u[i] : x / (1.0f + libm_expf(-x)) * u[i];
}

// out[t][h] = ((ex[t][0][h] * w[t][0] + ex[t][1][h] * w[t][1]) + ...)
//             (+ sh[t][h] (* shg[t])) (+ resid[t][h])
// build_segB's ggml_mul then left-to-right ggml_add chain (runtime.cpp:
// 4544-4550), the shared expert's ggml_mul by its gate and ggml_add
// (4553-4561), and the residual add (4568).  One thread per output.
__global__ void __launch_bounds__(256) k_combine_batch(const float * ex, const float * w, const float * sh,
                                                       const float * shg, const float * resid, float * out, int H,
                                                       int k, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int64_t t = i / H;
    const int h = (int)(i % H);
    const float * e = ex + (size_t)t * k * H + h;
    const float * wt = w + (size_t)t * k;
    float acc = e[0] * wt[0];
    for (int j = 1; j < k; ++j) acc = acc + e[(size_t)j * H] * wt[j];
    if (sh) {
        float v = sh[i];
        if (shg) v = v * shg[t];
        acc = acc + v;
    }
    if (resid) acc = acc + resid[i];
    out[i] = acc;
}

// The shared expert's gate: sigmoid(gw . x_t) per token (ggml_mul_mat with an
// f32 [H, 1] weight runs ggml_vec_dot_f32 per column, vec.cpp:11-135 AVX-512
// order; then unary-ops.cpp:31-33).  One wave per token; lane L accumulates
// the elements 64 s + L, then (L, L ^ 32), (L, L ^ 16) and the 16-lane tree.
__global__ void __launch_bounds__(256) k_sh_gate(const float * gw, const float * x, float * shg, int H, int T) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;                                    // uniform per wave
    const float * xr = x + (size_t)t * H;
    float acc = 0.f;
    for (int s = 0; s < H / 64; ++s) acc = __builtin_fmaf(gw[64 * s + lane], xr[64 * s + lane], acc);
    acc += lane_xor32_f(acc);
    acc += lane_xor16_f(acc);
    acc = tree16_dpp(acc);
    if (lane == 0) shg[t] = libm_sigmoid(acc);
}

int launch_swiglu_rows(const float * g, const float * u, float * act, int n, int64_t rows, hipStream_t s) {
    const int64_t total = (int64_t)n * rows;
    if (total <= 0) return QWM_OK;
    k_swiglu_rows<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s>>>(g, u, act, n, total);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

int launch_combine_batch(const float * ex, const float * w, const float * sh, const float * shg, const float * resid,
                         float * out, int H, int k, int64_t T, hipStream_t s) {
    const int64_t total = (int64_t)H * T;
    if (total <= 0) return QWM_OK;
    k_combine_batch<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s>>>(ex, w, sh, shg, resid, out, H, k,
                                                                                 total);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

int launch_sh_gate(const float * gw, const float * x, float * shg, int H, int T, hipStream_t s) {
    if (T <= 0) return QWM_OK;
    k_sh_gate<<<dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s>>>(gw, x, shg, H, T);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
