// C entry points over the reference ggml vector helpers (ggml/src/ggml-cpu/vec.h
// inline functions and vec.cpp), compiled against the unmodified reference
// sources by oracle/Makefile into oracle/_ref/.  Test infrastructure only.
#include "vec.h"

#define QWR_API extern "C" __attribute__((visibility("default")))

// ggml_v_expf / ggml_v_silu (vec.h:1191-1226), 16 lanes at a time.
QWR_API void qwr_v_expf16(const float * x, float * y) { _mm512_storeu_ps(y, ggml_v_expf(_mm512_loadu_ps(x))); }
QWR_API void qwr_v_silu16(const float * x, float * y) { _mm512_storeu_ps(y, ggml_v_silu(_mm512_loadu_ps(x))); }
// ggml_vec_soft_max_f32 (vec.cpp:531) followed by the 1/sum scaling of
// ggml_compute_forward_soft_max_f32 (ops.cpp:5899-5900).
QWR_API void qwr_soft_max_row(int n, const float * x, float * y) {
    float max = -INFINITY;
    ggml_vec_max_f32(n, &max, x);
    ggml_float sum = ggml_vec_soft_max_f32(n, y, x, max);
    sum = 1.0 / sum;
    ggml_vec_scale_f32(n, y, sum);
}
QWR_API void qwr_swiglu(int n, float * y, const float * gate, const float * up) { ggml_vec_swiglu_f32(n, y, gate, up); }
QWR_API void qwr_silu(int n, float * y, const float * x) { ggml_vec_silu_f32(n, y, x); }
QWR_API int qwr_argmax(int n, const float * x) { int v = 0; ggml_vec_argmax_f32(n, &v, x); return v; }
QWR_API float qwr_sum(int n, const float * x) { float s; ggml_vec_sum_f32(n, &s, x); return s; }
