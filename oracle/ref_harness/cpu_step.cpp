// One MoE verify step on the CPU through the reference's own ggml-CPU leaf
// kernels (compiled from the unmodified sources into oracle/_ref), for the
// CPU baseline that bench.py reports beside the GPU.  Test/benchmark
// infrastructure only.
//
// The orchestration restates the reference graph (core/runtime.cpp:
// build_router 3785, route_experts 2693-2734, build_segB 4534-4572, verify
// head 5014-5046, accept 3648-3652) and ggml-cpu's MUL_MAT_ID strategy
// (ggml-cpu.c:1554-1734: quantize the activations once, group the routed
// columns by expert, then every thread takes rows of the expert's matrix and
// dots them with each column).  Threads: OpenMP, like ggml's default build.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "ggml-common.h"
#include "ggml-quants.h"
#include "vec.h"

#define QWR_API extern "C" __attribute__((visibility("default")))

extern "C" {
void ggml_vec_dot_q4_K_q8_K(int n, float * s, size_t bs, const void * vx, size_t bx, const void * vy, size_t by, int nrc);
void ggml_vec_dot_q8_0_q8_0(int n, float * s, size_t bs, const void * vx, size_t bx, const void * vy, size_t by, int nrc);
void quantize_row_q8_0(const float * x, void * y, int64_t k);
void quantize_row_q8_K(const float * x, void * y, int64_t k);
}

struct qwr_step_args {
    int64_t H, N, E, k, T, V;
    const float * router;                 // [E][H]
    const uint8_t * gate; const uint8_t * up; const uint8_t * down;   // Q4_K slabs, slot = expert id
    const uint8_t * lm_head;              // Q8_0 [V][H]
    const float * x;                      // [T][H]
    const int32_t * drafts;               // [T-1]
    int32_t * ids; float * out; int32_t * vA; int32_t * accepted;
    int n_threads;
};

QWR_API int qwr_cpu_verify_step(const qwr_step_args * a) {
    const int64_t H = a->H, N = a->N, E = a->E, k = a->k, T = a->T, V = a->V;
    const int nt = a->n_threads;
    const size_t gu_row = (size_t)(H / QK_K) * sizeof(block_q4_K), dn_row = (size_t)(N / QK_K) * sizeof(block_q4_K);
    // router + softmax + top-k + normalized weights
    std::vector<float> logits((size_t)(T * E)), probs((size_t)(T * E)), w((size_t)(T * k));
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t e = 0; e < E; ++e)
        for (int64_t t = 0; t < T; ++t)
            ggml_vec_dot_f32((int)H, &logits[(size_t)(t * E + e)], 0, a->router + e * H, 0, a->x + t * H, 0, 1);
    for (int64_t t = 0; t < T; ++t) {
        float mx = -INFINITY;
        ggml_vec_max_f32((int)E, &mx, &logits[(size_t)(t * E)]);
        ggml_float sum = ggml_vec_soft_max_f32((int)E, &probs[(size_t)(t * E)], &logits[(size_t)(t * E)], mx);
        ggml_vec_scale_f32((int)E, &probs[(size_t)(t * E)], (float)(1.0 / sum));
        std::vector<int32_t> idx((size_t)E);
        for (int64_t e = 0; e < E; ++e) idx[(size_t)e] = (int32_t)e;
        const float * p = &probs[(size_t)(t * E)];
        std::sort(idx.begin(), idx.end(), [p](int32_t l, int32_t r) { return p[l] > p[r]; });
        float s = 0.f;
        for (int64_t j = 0; j < k; ++j) { a->ids[t * k + j] = idx[(size_t)j]; w[(size_t)(t * k + j)] = p[idx[(size_t)j]]; }
        ggml_vec_sum_f32((int)k, &s, &w[(size_t)(t * k)]);
        s = std::max(s, 6.103515625e-5f);
        for (int64_t j = 0; j < k; ++j) w[(size_t)(t * k + j)] /= s;
    }
    // activations -> Q8_K
    std::vector<block_q8_K> xq((size_t)(T * H / QK_K));
    for (int64_t t = 0; t < T; ++t) quantize_row_q8_K(a->x + t * H, &xq[(size_t)(t * H / QK_K)], H);
    // group the (token, slot) pairs by expert
    std::vector<std::vector<int64_t>> by_expert((size_t)E);
    std::vector<int64_t> order;
    for (int64_t p = 0; p < T * k; ++p) {
        const int32_t e = a->ids[p];
        if (by_expert[(size_t)e].empty()) order.push_back(e);
        by_expert[(size_t)e].push_back(p);
    }
    std::vector<float> gate((size_t)(T * k * N)), upv((size_t)(T * k * N)), act((size_t)(T * k * N));
    for (int64_t e : order) {
        const auto & pairs = by_expert[(size_t)e];
        const uint8_t * G = a->gate + (size_t)e * N * gu_row;
        const uint8_t * U = a->up + (size_t)e * N * gu_row;
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t r = 0; r < N; ++r)
            for (int64_t p : pairs) {
                const block_q8_K * col = &xq[(size_t)((p / k) * H / QK_K)];
                ggml_vec_dot_q4_K_q8_K((int)H, &gate[(size_t)(p * N + r)], 0, G + r * gu_row, 0, col, 0, 1);
                ggml_vec_dot_q4_K_q8_K((int)H, &upv[(size_t)(p * N + r)], 0, U + r * gu_row, 0, col, 0, 1);
            }
    }
    for (int64_t p = 0; p < T * k; ++p)
        ggml_vec_swiglu_f32((int)N, &act[(size_t)(p * N)], &gate[(size_t)(p * N)], &upv[(size_t)(p * N)]);
    std::vector<block_q8_K> aq((size_t)(T * k * N / QK_K));
    for (int64_t p = 0; p < T * k; ++p) quantize_row_q8_K(&act[(size_t)(p * N)], &aq[(size_t)(p * N / QK_K)], N);
    std::vector<float> ex((size_t)(T * k * H));
    for (int64_t e : order) {
        const auto & pairs = by_expert[(size_t)e];
        const uint8_t * D = a->down + (size_t)e * H * dn_row;
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t r = 0; r < H; ++r)
            for (int64_t p : pairs)
                ggml_vec_dot_q4_K_q8_K((int)N, &ex[(size_t)(p * H + r)], 0, D + r * dn_row, 0, &aq[(size_t)(p * N / QK_K)], 0, 1);
    }
    // combine + residual, verify head
    std::vector<block_q8_0> hq((size_t)(T * H / QK8_0));
    for (int64_t t = 0; t < T; ++t) {
        float * o = a->out + t * H;
        for (int64_t h = 0; h < H; ++h) {
            float s = ex[(size_t)((t * k) * H + h)] * w[(size_t)(t * k)];
            for (int64_t j = 1; j < k; ++j) s += ex[(size_t)((t * k + j) * H + h)] * w[(size_t)(t * k + j)];
            o[h] = s + a->x[t * H + h];
        }
        ggml_float ss = 0.0;
        for (int64_t h = 0; h < H; ++h) ss += (ggml_float)(o[h] * o[h]);
        const float scale = 1.0f / sqrtf((float)(ss / H) + 1e-6f);
        std::vector<float> hn((size_t)H);
        for (int64_t h = 0; h < H; ++h) hn[(size_t)h] = o[h] * scale;
        quantize_row_q8_0(hn.data(), &hq[(size_t)(t * H / QK8_0)], H);
    }
    const size_t lm_row = (size_t)(H / QK8_0) * sizeof(block_q8_0);
    std::vector<float> lg((size_t)(T * V));
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < V; ++r)
        for (int64_t t = 0; t < T; ++t)
            ggml_vec_dot_q8_0_q8_0((int)H, &lg[(size_t)(t * V + r)], 0, a->lm_head + r * lm_row, 0,
                                   &hq[(size_t)(t * H / QK8_0)], 0, 1);
    for (int64_t t = 0; t < T; ++t) {
        int v = 0;
        ggml_vec_argmax_f32((int)V, &v, &lg[(size_t)(t * V)]);
        a->vA[t] = v;
    }
    int acc = 0;
    while (acc < T - 1 && a->vA[acc] == a->drafts[acc]) ++acc;
    *a->accepted = acc;
    return 0;
}

// One MoE block, x + MoE(x), for the decode, miss-fill and prefill baselines:
// router (+ route mask), soft_max, top-k, normalized weights; gate/up/down
// through MUL_MAT_ID's strategy as above; SwiGLU; the combine in the graph's
// order (T == 1: vec_dot_f32 over the k expert outputs, runtime.cpp:3815-3817;
// T > 1: product then the left-to-right add chain, 4544-4550); the shared
// expert with its sigmoid gate (3820-3828, 4553-4561); the residual.
struct qwr_block_args {
    int64_t H, N, E, k, T;
    const float * router;                 // [E][H]
    const float * rm;                     // [T][E] or null
    const uint8_t * gate; const uint8_t * up; const uint8_t * down;   // Q4_K, slot = expert id
    const uint8_t * sh_gate; const uint8_t * sh_up; const uint8_t * sh_down;   // or null
    const float * sh_inp;                 // [H] or null
    const float * x;                      // [T][H]
    float * out;                          // [T][H]
    int32_t * ids;                        // [T][k]
    int n_threads;
};

static void ffn_rows(const uint8_t * W, size_t row, int64_t rows, int64_t K, const block_q8_K * xq, float * y, int nt) {
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < rows; ++r) ggml_vec_dot_q4_K_q8_K((int)K, &y[r], 0, W + (size_t)r * row, 0, xq, 0, 1);
}

QWR_API int qwr_cpu_moe_block(const qwr_block_args * a) {
    const int64_t H = a->H, N = a->N, E = a->E, k = a->k, T = a->T;
    const int nt = a->n_threads;
    const size_t gu_row = (size_t)(H / QK_K) * sizeof(block_q4_K), dn_row = (size_t)(N / QK_K) * sizeof(block_q4_K);
    std::vector<float> logits((size_t)(T * E)), probs((size_t)(T * E)), w((size_t)(T * k));
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t e = 0; e < E; ++e)
        for (int64_t t = 0; t < T; ++t) {
            float v;
            ggml_vec_dot_f32((int)H, &v, 0, a->router + e * H, 0, a->x + t * H, 0, 1);
            logits[(size_t)(t * E + e)] = a->rm ? v + a->rm[t * E + e] : v;
        }
    for (int64_t t = 0; t < T; ++t) {
        float mx = -INFINITY;
        ggml_vec_max_f32((int)E, &mx, &logits[(size_t)(t * E)]);
        ggml_float sum = ggml_vec_soft_max_f32((int)E, &probs[(size_t)(t * E)], &logits[(size_t)(t * E)], mx);
        ggml_vec_scale_f32((int)E, &probs[(size_t)(t * E)], (float)(1.0 / sum));
        std::vector<int32_t> idx((size_t)E);
        for (int64_t e = 0; e < E; ++e) idx[(size_t)e] = (int32_t)e;
        const float * p = &probs[(size_t)(t * E)];
        std::sort(idx.begin(), idx.end(), [p](int32_t l, int32_t r) { return p[l] > p[r]; });   // ggml_argsort_top_k
        float s = 0.f;
        for (int64_t j = 0; j < k; ++j) { a->ids[t * k + j] = idx[(size_t)j]; w[(size_t)(t * k + j)] = p[idx[(size_t)j]]; }
        ggml_vec_sum_f32((int)k, &s, &w[(size_t)(t * k)]);
        s = std::max(s, 6.103515625e-5f);
        for (int64_t j = 0; j < k; ++j) w[(size_t)(t * k + j)] /= s;
    }
    std::vector<block_q8_K> xq((size_t)(T * H / QK_K));
    for (int64_t t = 0; t < T; ++t) quantize_row_q8_K(a->x + t * H, &xq[(size_t)(t * H / QK_K)], H);
    std::vector<std::vector<int64_t>> by_expert((size_t)E);
    std::vector<int64_t> order;
    for (int64_t p = 0; p < T * k; ++p) {
        const int32_t e = a->ids[p];
        if (by_expert[(size_t)e].empty()) order.push_back(e);
        by_expert[(size_t)e].push_back(p);
    }
    std::vector<float> gate((size_t)(T * k * N)), upv((size_t)(T * k * N)), act((size_t)(T * k * N));
    for (int64_t e : order) {
        const auto & pairs = by_expert[(size_t)e];
        const uint8_t * G = a->gate + (size_t)e * N * gu_row;
        const uint8_t * U = a->up + (size_t)e * N * gu_row;
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t r = 0; r < N; ++r)
            for (int64_t p : pairs) {
                const block_q8_K * col = &xq[(size_t)((p / k) * H / QK_K)];
                ggml_vec_dot_q4_K_q8_K((int)H, &gate[(size_t)(p * N + r)], 0, G + r * gu_row, 0, col, 0, 1);
                ggml_vec_dot_q4_K_q8_K((int)H, &upv[(size_t)(p * N + r)], 0, U + r * gu_row, 0, col, 0, 1);
            }
    }
    for (int64_t p = 0; p < T * k; ++p)
        ggml_vec_swiglu_f32((int)N, &act[(size_t)(p * N)], &gate[(size_t)(p * N)], &upv[(size_t)(p * N)]);
    std::vector<block_q8_K> aq((size_t)(T * k * N / QK_K));
    for (int64_t p = 0; p < T * k; ++p) quantize_row_q8_K(&act[(size_t)(p * N)], &aq[(size_t)(p * N / QK_K)], N);
    std::vector<float> ex((size_t)(T * k * H));
    for (int64_t e : order) {
        const auto & pairs = by_expert[(size_t)e];
        const uint8_t * D = a->down + (size_t)e * H * dn_row;
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t r = 0; r < H; ++r)
            for (int64_t p : pairs)
                ggml_vec_dot_q4_K_q8_K((int)N, &ex[(size_t)(p * H + r)], 0, D + r * dn_row, 0, &aq[(size_t)(p * N / QK_K)], 0, 1);
    }
    // shared expert
    std::vector<float> sh((size_t)(T * H), 0.f), shg((size_t)T, 1.f);
    if (a->sh_gate) {
        std::vector<float> g((size_t)N), u((size_t)N), s((size_t)N);
        std::vector<block_q8_K> sq((size_t)(N / QK_K));
        for (int64_t t = 0; t < T; ++t) {
            ffn_rows(a->sh_gate, gu_row, N, H, &xq[(size_t)(t * H / QK_K)], g.data(), nt);
            ffn_rows(a->sh_up, gu_row, N, H, &xq[(size_t)(t * H / QK_K)], u.data(), nt);
            ggml_vec_swiglu_f32((int)N, s.data(), g.data(), u.data());
            quantize_row_q8_K(s.data(), sq.data(), N);
            ffn_rows(a->sh_down, dn_row, H, N, sq.data(), &sh[(size_t)(t * H)], nt);
            if (a->sh_inp) {
                float l;
                ggml_vec_dot_f32((int)H, &l, 0, a->sh_inp, 0, a->x + t * H, 0, 1);
                shg[(size_t)t] = 1.f / (1.f + expf(-l));
            }
        }
    }
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < H; ++h) {
            float s;
            if (T == 1) {
                float ev[64];
                for (int64_t j = 0; j < k; ++j) ev[j] = ex[(size_t)(j * H + h)];
                ggml_vec_dot_f32((int)k, &s, 0, ev, 0, w.data(), 0, 1);
            } else {
                s = ex[(size_t)((t * k) * H + h)] * w[(size_t)(t * k)];
                for (int64_t j = 1; j < k; ++j) s += ex[(size_t)((t * k + j) * H + h)] * w[(size_t)(t * k + j)];
            }
            if (a->sh_gate) s += sh[(size_t)(t * H + h)] * shg[(size_t)t];
            a->out[t * H + h] = s + a->x[t * H + h];
        }
    return 0;
}

// GGML_OP_MUL_MAT_ID over Q4_K (ggml-cpu.c:1554-1734 without the tiled
// AVX-512 VNNI kernel of experts with >= 8 columns): every column of b to
// Q8_K once, the (column, slot) pairs grouped by expert, every thread takes
// rows of the expert's matrix and dots them with each of its columns.
QWR_API int qwr_cpu_mul_mat_id(const uint8_t * as, int64_t K, int64_t N, int64_t n_as, const float * b, int64_t ne11,
                               int64_t T, const int32_t * ids, int64_t n_ids, float * dst, int n_threads) {
    const size_t row = (size_t)(K / QK_K) * sizeof(block_q4_K);
    std::vector<block_q8_K> bq((size_t)(T * ne11 * K / QK_K));
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t c = 0; c < T * ne11; ++c) quantize_row_q8_K(b + c * K, &bq[(size_t)(c * K / QK_K)], K);
    std::vector<std::vector<int64_t>> by_expert((size_t)n_as);
    for (int64_t p = 0; p < T * n_ids; ++p) {
        const int32_t e = ids[p];
        if (e < 0 || e >= n_as) return -1;
        by_expert[(size_t)e].push_back(p);
    }
    for (int64_t e = 0; e < n_as; ++e) {
        const auto & pairs = by_expert[(size_t)e];
        if (pairs.empty()) continue;
        const uint8_t * W = as + (size_t)e * N * row;
#pragma omp parallel for num_threads(n_threads) schedule(static)
        for (int64_t r = 0; r < N; ++r)
            for (int64_t p : pairs) {
                const int64_t t = p / n_ids, c = (p % n_ids) % ne11;
                ggml_vec_dot_q4_K_q8_K((int)K, &dst[(size_t)(p * N + r)], 0, W + r * row, 0,
                                       &bq[(size_t)((t * ne11 + c) * K / QK_K)], 0, 1);
            }
    }
    return 0;
}
