/* C entry points over the reference ggml leaf kernels, compiled together with
 * the unmodified reference sources by oracle/Makefile into oracle/_ref/.
 * Test infrastructure only: it pins the restatement in oracle/qwm_oracle.cpp.
 * Reference symbols wrapped:
 *   quantize_row_q4_K_ref, quantize_row_q8_K_ref, quantize_row_q8_0_ref,
 *   dequantize_row_q4_K, dequantize_row_q6_K (ggml/src/ggml-quants.c)
 *   quantize_row_q8_0, quantize_row_q8_K, ggml_vec_dot_q4_K_q8_K,
 *   ggml_vec_dot_q5_K_q8_K, ggml_vec_dot_q6_K_q8_K, ggml_vec_dot_q8_0_q8_0
 *                                 (ggml/src/ggml-cpu/arch/x86/quants.c)
 *   ggml_vec_dot_f32              (ggml/src/ggml-cpu/vec.cpp)           */
#include "ggml-common.h"
#include "ggml-quants.h"
#include <stddef.h>
#include <stdint.h>

#define QWR_API __attribute__((visibility("default")))

void ggml_vec_dot_f32(int n, float * s, size_t bs, const float * x, size_t bx, const float * y, size_t by, int nrc);
void ggml_vec_dot_q4_K_q8_K(int n, float * s, size_t bs, const void * vx, size_t bx, const void * vy, size_t by, int nrc);
void ggml_vec_dot_q8_0_q8_0(int n, float * s, size_t bs, const void * vx, size_t bx, const void * vy, size_t by, int nrc);
void ggml_vec_dot_q6_K_q8_K(int n, float * s, size_t bs, const void * vx, size_t bx, const void * vy, size_t by, int nrc);
void ggml_vec_dot_q5_K_q8_K(int n, float * s, size_t bs, const void * vx, size_t bx, const void * vy, size_t by, int nrc);
void quantize_row_q8_0(const float * x, void * y, int64_t k);
void quantize_row_q8_K(const float * x, void * y, int64_t k);

QWR_API void qwr_quantize_q4_K(const float * x, void * y, int64_t k) { quantize_row_q4_K_ref(x, (block_q4_K *) y, k); }
QWR_API void qwr_dequantize_q4_K(const void * x, float * y, int64_t k) { dequantize_row_q4_K((const block_q4_K *) x, y, k); }
QWR_API void qwr_quantize_q8_K_ref(const float * x, void * y, int64_t k) { quantize_row_q8_K_ref(x, (block_q8_K *) y, k); }
QWR_API void qwr_quantize_q8_K(const float * x, void * y, int64_t k) { quantize_row_q8_K(x, y, k); }
QWR_API void qwr_quantize_q8_0_ref(const float * x, void * y, int64_t k) { quantize_row_q8_0_ref(x, (block_q8_0 *) y, k); }
QWR_API void qwr_quantize_q8_0(const float * x, void * y, int64_t k) { quantize_row_q8_0(x, y, k); }
QWR_API float qwr_vec_dot_q4_K_q8_K(int n, const void * x, const void * y) { float s; ggml_vec_dot_q4_K_q8_K(n, &s, 0, x, 0, y, 0, 1); return s; }
QWR_API float qwr_vec_dot_q5_K_q8_K(int n, const void * x, const void * y) { float s; ggml_vec_dot_q5_K_q8_K(n, &s, 0, x, 0, y, 0, 1); return s; }
QWR_API float qwr_vec_dot_q6_K_q8_K(int n, const void * x, const void * y) { float s; ggml_vec_dot_q6_K_q8_K(n, &s, 0, x, 0, y, 0, 1); return s; }
QWR_API void qwr_dequantize_q6_K(const void * x, float * y, int64_t k) { dequantize_row_q6_K((const block_q6_K *) x, y, k); }
QWR_API float qwr_vec_dot_q8_0_q8_0(int n, const void * x, const void * y) { float s; ggml_vec_dot_q8_0_q8_0(n, &s, 0, x, 0, y, 0, 1); return s; }
QWR_API float qwr_vec_dot_f32(int n, const float * x, const float * y) { float s; ggml_vec_dot_f32(n, &s, 0, x, 0, y, 0, 1); return s; }
