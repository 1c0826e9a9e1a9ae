// qwm_oracle.cpp -- CPU restatement of the MoE expert path of QuestWend's
// vendored ggml CPU backend (x86-64, AVX-512 build), used ONLY as test
// infrastructure: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg load it to check results.  Nothing in questwend_amd/ links or calls it.
//
// Every function cites the reference file:line whose behaviour it restates
// (paths relative to the QuestWend tree; ggml = third_party/ggml/src).
// Floating-point order is restated where the reference fixes it with SIMD
// intrinsics (fused multiply-adds, lane layouts, horizontal-add trees); this
// file is compiled with -ffp-contract=off so that only the explicit fmaf()
// calls below fuse.
//
// Pinning (see tests/test_oracle_*.py):
//   * Q4_K/Q8_K/Q8_0 quantizers, vec_dot_{q4_K_q8_K,q8_0_q8_0,f32}, the SIMD
//     expf/silu/softmax/swiglu leaves are compared bit-for-bit with the
//     reference leaf sources compiled by oracle/Makefile into oracle/_ref/.
//   * Integer block dots are checked against exact int64 arithmetic and the
//     dequantized fp64 dot; softmax/top-k/combine against fp64 textbook forms.
//   * The slot pool is checked against the reference GpuLruIndex header and the
//     reference test's linear_scan known answers.
//   * The f32 router mul_mat runs vec_dot_f32 per (row, column) at every
//     column count, as the reference's ggml-cpu build does (GGML_LLAMAFILE is
//     off there, ggml/CMakeLists.txt:113-114,197, so ggml-cpu.c:1300 is
//     compiled out, and tiled/tiled.cpp:605-640 takes no f32 weights).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <functional>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <thread>
#include <string>
#include <unordered_map>
#include <vector>

#define QWO_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;

// ggml block layouts (ggml-common.h:251-256, 325-338, 369-376).
struct block_q4_K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; };
struct block_q8_K { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; };
struct block_q8_0 { uint16_t d; int8_t qs[QK8_0]; };
struct block_q6_K { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; };
struct block_q5_K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[QK_K / 8]; uint8_t qs[QK_K / 2]; };
static_assert(sizeof(block_q5_K) == 176, "q5_K");
static_assert(sizeof(block_q6_K) == 210, "q6_K");
static_assert(sizeof(block_q4_K) == 144, "q4_K");
static_assert(sizeof(block_q8_K) == 292, "q8_K");
static_assert(sizeof(block_q8_0) == 34, "q8_0");

// ggml_type values (ggml.h:390-420).
constexpr int T_F32 = 0, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15;

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// IEEE binary16 <-> binary32, round-to-nearest-even.  Same results as
// ggml-impl.h:396-446 (software) and F16C (_cvtss_sh(x,0)) for finite inputs.
inline float fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        const float v = std::ldexp((float)man, -24);  // subnormal, exact
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112) << 23) | (man << 13));
}
inline uint16_t fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00);  // rounds to inf
    if (ax < 0x38800000u) {                                   // fp16 subnormal / zero
        // value = ax_float; fp16 subnormal unit is 2^-24
        const float v = u2f(ax) * 16777216.0f;                // exact scaling by 2^24
        const float r = std::nearbyint(v);                    // RNE (default rounding mode)
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t m = ax + 0xc8000000u;       // rebias exponent (127-15) << 23
    m += 0x0fff + ((m >> 13) & 1);       // round to nearest even
    return (uint16_t)(sign | (m >> 13));
}

// ggml-quants.c:621-626
inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i; std::memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}
// nearest_int(a*b) as gcc compiles it once inlined: the product and the
// magic-number add fuse into one fma (checked against the compiled
// reference's Q8_K and Q4_K bytes).
inline int nearest_int_mul(float a, float b) {
    float val = fmaf(a, b, 12582912.f);
    int i; std::memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

// ---------------------------------------------------------------- Q4_K ----

// ggml-quants.c:799-870 (make_qkx2_quants).  The fmaf() calls are where gcc
// -O3 -march=x86-64-v4 (GNU dialect, fp-contract=fast) contracts the
// reference's multiply-adds; tests compare the bytes with the compiled
// reference to keep this honest.
float make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L,
                       float * the_min, uint8_t * Laux, float rmin, float rdelta, int nstep, bool use_mad) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        float w = weights[i];
        sum_w += w;
        sum_x = fmaf(w, x[i], sum_x);
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int_mul(iscale, x[i] - min);
        L[i] = (uint8_t)std::max(0, std::min(nmax, l));
        float diff = fmaf(scale, (float)L[i], min) - x[i];
        diff = use_mad ? std::fabs(diff) : diff * diff;
        float w = weights[i];
        best_error = fmaf(w, diff, best_error);
    }
    if (nstep < 1) { *the_min = -min; return scale; }
    for (int is = 0; is <= nstep; ++is) {
        iscale = fmaf(rdelta, (float)is, rmin) + nmax;
        iscale = iscale / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int_mul(iscale, x[i] - min);
            l = std::max(0, std::min(nmax, l));
            Laux[i] = (uint8_t)l;
            float w = weights[i];
            sum_l = sum_l + w * l;          // w*l has three uses: not fused
            sum_l2 = fmaf(w * l, (float)l, sum_l2);
            sum_xl = fmaf(w * l, x[i], sum_xl);
        }
        float D = fmaf(sum_w, sum_l2, -(sum_l * sum_l));
        if (D > 0) {
            float this_scale = fmaf(-sum_x, sum_l, sum_w * sum_xl) / D;   // gcc fuses the second product here
            float this_min = fmaf(sum_l2, sum_x, -(sum_l * sum_xl)) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = fmaf(this_scale, (float)Laux[i], this_min) - x[i];
                diff = use_mad ? std::fabs(diff) : diff * diff;
                float w = weights[i];
                cur_error = fmaf(w, diff, cur_error);
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

// ggml-quants.c:871-878
inline void get_scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

// ggml-quants.c:1458-1528 (quantize_row_q4_K_ref; quantize_q4_K without an
// importance matrix calls it row by row).
void quantize_row_q4_K(const float * x, block_q4_K * y, int64_t k) {
    const int nb = (int)(k / QK_K);
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int i = 0; i < nb; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            // gcc vectorizes this loop: unfused products added in order.
            for (int l = 0; l < 32; ++l) sum_x2 = sum_x2 + x[32 * j + l] * x[32 * j + l];
            float av_x = std::sqrt(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20, false);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        std::memset(y[i].scales, 0, 12);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)nearest_int_mul(inv_scale, scales[j]);
            uint8_t lm = (uint8_t)nearest_int_mul(inv_min, mins[j]);
            ls = std::min<uint8_t>(63, ls);
            lm = std::min<uint8_t>(63, lm);
            if (j < 4) { y[i].scales[j] = ls; y[i].scales[j + 4] = lm; }
            else {
                y[i].scales[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4);
                y[i].scales[j - 4] |= ((ls >> 4) << 6);
                y[i].scales[j - 0] |= ((lm >> 4) << 6);
            }
        }
        y[i].d = fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = fp32_to_fp16(max_min / 63.f);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = fp16_to_fp32(y[i].d) * sc;
            if (!d) continue;
            const float dm = fp16_to_fp32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                l = std::max(0, std::min(15, l));
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        uint8_t * q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += QK_K;
    }
}

// ggml-quants.c:1530-1552
void dequantize_row_q4_K(const block_q4_K * x, float * y, int64_t k) {
    const int nb = (int)(k / QK_K);
    for (int i = 0; i < nb; i++) {
        const uint8_t * q = x[i].qs;
        const float d = fp16_to_fp32(x[i].d), min = fp16_to_fp32(x[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = min * m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32; is += 2;
        }
    }
}

// ---------------------------------------------------------------- Q8_K ----

// ggml-quants.c:2769-2806 (x86 quantize_row_q8_K forwards here,
// ggml-cpu/arch/x86/quants.c:505-507).
void quantize_row_q8_K(const float * x, block_q8_K * y, int64_t k) {
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; ++j) {
            float ax = std::fabs(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        if (!amax) {
            y[i].d = 0;
            std::memset(y[i].qs, 0, QK_K);
            std::memset(y[i].bsums, 0, sizeof(y[i].bsums));
            x += QK_K;
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; ++j) {
            int v = nearest_int_mul(iscale, x[j]);
            y[i].qs[j] = (int8_t)std::min(127, v);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1 / iscale;
        x += QK_K;
    }
}

// ---------------------------------------------------------------- Q8_0 ----

// ggml-quants.c:276-300: the model-file quantizer (round half away from zero,
// multiplier 1/d).  Used for the lm_head weights.
void quantize_row_q8_0_ref(const float * x, block_q8_0 * y, int64_t k) {
    const int nb = (int)(k / QK8_0);
    for (int i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = std::max(amax, std::fabs(x[i * QK8_0 + j]));
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = fp32_to_fp16(d);
        for (int j = 0; j < QK8_0; ++j) y[i].qs[j] = (int8_t)std::round(x[i * QK8_0 + j] * id);
    }
}

// ggml-cpu/arch/x86/quants.c:302-345: the activation quantizer on x86
// (multiplier 127/amax, round half to even).  AVX-512 builds take this AVX2
// branch too.
void quantize_row_q8_0_x86(const float * x, block_q8_0 * y, int64_t k) {
    const int nb = (int)(k / QK8_0);
    for (int i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = std::max(amax, std::fabs(x[i * QK8_0 + j]));
        const float d = amax / 127.f;
        y[i].d = fp32_to_fp16(d);
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        for (int j = 0; j < QK8_0; ++j) y[i].qs[j] = (int8_t)(int)std::nearbyint(x[i * QK8_0 + j] * id);
    }
}

// ------------------------------------------------------ horizontal sums ----

// hsum_float_8 (ggml-cpu/arch/x86/quants.c:43-49): lanes (i, i+4), then
// (i, i+2), then (0, 1).
inline float hsum8(const float a[8]) {
    float r[4];
    for (int i = 0; i < 4; ++i) r[i] = a[i + 4] + a[i];
    const float s0 = r[0] + r[2], s1 = r[1] + r[3];
    return s0 + s1;
}
// 4-lane tail of vec_dot_q4_K_q8_K (quants.c:2181-2182).
inline float hsum4(const float a[4]) {
    const float s0 = a[0] + a[2], s1 = a[1] + a[3];
    return s0 + s1;
}
// _mm512_reduce_add_ps as emitted by gcc: halving tree over 8, 4, 2, 1.
inline float reduce16(const float a[16]) {
    float t8[8], t4[4];
    for (int i = 0; i < 8; ++i) t8[i] = a[i + 8] + a[i];
    for (int i = 0; i < 4; ++i) t4[i] = t8[i + 4] + t8[i];
    const float t2a = t4[0] + t4[2], t2b = t4[1] + t4[3];
    return t2a + t2b;
}

// ----------------------------------------------------------------- dots ----

// ggml-cpu/arch/x86/quants.c:2102-2183 (AVX2 branch): integer sums per
// 4-byte lane group, per-block fused multiply-add into 8 float lanes plus a
// 4-lane min accumulator.
float vec_dot_q4_K_q8_K(int n, const block_q4_K * x, const block_q8_K * y) {
    const int nb = n / QK_K;
    float acc[8] = {0}, acc_m[4] = {0};
    for (int i = 0; i < nb; ++i) {
        const float d = y[i].d * fp16_to_fp32(x[i].d);
        const float dmin = -y[i].d * fp16_to_fp32(x[i].dmin);
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        int32_t q8s[8];
        for (int j = 0; j < 8; ++j) q8s[j] = (int16_t)(y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        for (int l = 0; l < 4; ++l) {
            const int32_t prod = mn[2 * l] * q8s[2 * l] + mn[2 * l + 1] * q8s[2 * l + 1];
            acc_m[l] = fmaf(dmin, (float)prod, acc_m[l]);
        }
        int32_t sumi[8] = {0};
        const uint8_t * q4 = x[i].qs;
        const int8_t * q8 = y[i].qs;
        for (int j = 0; j < 4; ++j) {
            for (int m = 0; m < 8; ++m) {
                int32_t lo = 0, hi = 0;
                for (int e = 4 * m; e < 4 * m + 4; ++e) {
                    lo += (q4[e] & 0xF) * q8[e];
                    hi += (q4[e] >> 4) * q8[32 + e];
                }
                sumi[m] += sc[2 * j] * lo + sc[2 * j + 1] * hi;
            }
            q4 += 32; q8 += 64;
        }
        for (int m = 0; m < 8; ++m) acc[m] = fmaf(d, (float)sumi[m], acc[m]);
    }
    return hsum8(acc) + hsum4(acc_m);
}

// Q5_K (ggml-common.h:340-356): the Q4_K header and nibble layout plus a
// fifth bit per value, bit 2j (low nibbles of 32-byte group j) or 2j + 1
// (high nibbles) of qh[l] for the group's byte l.
inline int q5_value(const block_q5_K & b, int e) {
    const int j = e / 64, h = (e % 64) / 32, l = e % 32;
    const uint8_t q = b.qs[32 * j + l];
    return (h ? q >> 4 : q & 15) | (((b.qh[l] >> (2 * j + h)) & 1) << 4);
}

// ggml_vec_dot_q5_K_q8_K, x86 AVX2 branch (ggml-cpu/arch/x86/quants.c:
// 1958-2046): scales and mins unpacked as for Q4_K; eight int32 lanes per
// block, lane m = sum over the eight 32-value sub-blocks s of scale[s] times
// the dot of sub-block values 4m..4m+3; acc[m] = fma(y.d * fp16(x.d),
// (float)lane, acc[m]); the mins go to one float per row:
// summs += (-y.d * fp16(x.dmin)) * (sum_j min[j] * (bsums[2j] + bsums[2j+1])),
// a statement gcc contracts into a fused multiply-add (-ffp-contract=fast,
// the GNU C default); result hsum8(acc) + summs.
float vec_dot_q5_K_q8_K(int n, const block_q5_K * x, const block_q8_K * y) {
    float acc[8] = {0};
    float summs = 0.f;
    for (int i = 0; i < n / QK_K; ++i) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        const float d = y[i].d * fp16_to_fp32(x[i].d);
        const float dmin = -y[i].d * fp16_to_fp32(x[i].dmin);
        int32_t msum = 0;
        for (int j = 0; j < 8; ++j) msum += mn[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        summs = fmaf(dmin, (float)msum, summs);
        for (int m = 0; m < 8; ++m) {
            int32_t lane = 0;
            for (int s = 0; s < 8; ++s) {
                int32_t t = 0;
                for (int e = 32 * s + 4 * m; e < 32 * s + 4 * m + 4; ++e) t += q5_value(x[i], e) * y[i].qs[e];
                lane += sc[s] * t;
            }
            acc[m] = fmaf(d, (float)lane, acc[m]);
        }
    }
    return hsum8(acc) + summs;
}

// The 6-bit value of element e (0..255) of a Q6_K block, 0..63
// (ggml-quants.c:1940-1970 before its -32): element 128j + 32k + l takes the
// low (k < 2) or high (k >= 2) nibble of ql[64j + 32(k & 1) + l] and bits
// 2k, 2k+1 of qh[32j + l] as its top two bits.
inline int q6_value(const block_q6_K & b, int e) {
    const int j = e / 128, k = (e % 128) / 32, l = e % 32;
    const uint8_t q = b.ql[64 * j + 32 * (k & 1) + l];
    return ((k < 2 ? q & 15 : q >> 4) | (((b.qh[32 * j + l] >> (2 * k)) & 3) << 4));
}

// dequantize_row_q6_K (ggml-quants.c:1940-1970): d * scale[e / 16] * (q - 32).
void dequantize_row_q6_K(const block_q6_K * x, float * y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const float d = fp16_to_fp32(x[i].d);
        for (int e = 0; e < QK_K; ++e) y[i * QK_K + e] = d * x[i].scales[e / 16] * (q6_value(x[i], e) - 32);
    }
}

// ggml_vec_dot_q6_K_q8_K, x86 AVX2 branch (ggml-cpu/arch/x86/quants.c:
// 2490-2566): eight int32 lanes per block, lane m gathering, over the eight
// 32-value chunks c, scale[2c + (m >= 4)] times the dot of chunk values
// 4m..4m+3 (6-bit values without the -32), minus 32 * (bsums[2m] * scale[2m]
// + bsums[2m+1] * scale[2m+1]); then acc[m] = fma(y.d * fp16(x.d),
// (float)lane, acc[m]) block after block and hsum8.
float vec_dot_q6_K_q8_K(int n, const block_q6_K * x, const block_q8_K * y) {
    float acc[8] = {0};
    for (int i = 0; i < n / QK_K; ++i) {
        const float d = y[i].d * fp16_to_fp32(x[i].d);
        int32_t lane[8] = {0};
        for (int c = 0; c < 8; ++c)
            for (int m = 0; m < 8; ++m) {
                int32_t s = 0;
                for (int e = 32 * c + 4 * m; e < 32 * c + 4 * m + 4; ++e) s += q6_value(x[i], e) * y[i].qs[e];
                lane[m] += x[i].scales[2 * c + (m >= 4)] * s;
            }
        for (int m = 0; m < 8; ++m) {
            lane[m] -= 32 * (y[i].bsums[2 * m] * x[i].scales[2 * m] + y[i].bsums[2 * m + 1] * x[i].scales[2 * m + 1]);
            acc[m] = fmaf(d, (float)lane[m], acc[m]);
        }
    }
    return hsum8(acc);
}

// ggml-cpu/arch/x86/quants.c:1372-1402 (AVX2 branch, taken by the AVX-512
// build too).
float vec_dot_q8_0_q8_0(int n, const block_q8_0 * x, const block_q8_0 * y) {
    const int nb = n / QK8_0;
    float acc[8] = {0};
    for (int ib = 0; ib < nb; ++ib) {
        const float d = fp16_to_fp32(x[ib].d) * fp16_to_fp32(y[ib].d);
        for (int m = 0; m < 8; ++m) {
            int32_t s = 0;
            for (int e = 4 * m; e < 4 * m + 4; ++e) s += x[ib].qs[e] * y[ib].qs[e];
            acc[m] = fmaf(d, (float)s, acc[m]);
        }
    }
    return hsum8(acc);
}

// ggml-cpu/vec.cpp:11-135 with the AVX-512 mapping of simd-mappings.h:454-499:
// 4 accumulators x 16 lanes, fused multiply-add over 64-wide steps, reduce
// (0+2, 1+3, 0+1) then the 16-lane tree, then the scalar tail
// `sumf += x[i]*y[i]`.  gcc -O3 vectorizes that tail: 16- and then one
// 8-element group take unfused products added in order, the last < 8
// elements are contracted to fused multiply-adds.
float vec_dot_f32(int n, const float * x, const float * y) {
    const int np = n & ~63;
    float sum[4][16] = {{0}};
    for (int i = 0; i < np; i += 64)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 16; ++l)
                sum[j][l] = fmaf(x[i + 16 * j + l], y[i + 16 * j + l], sum[j][l]);
    for (int l = 0; l < 16; ++l) { sum[0][l] = sum[0][l] + sum[2][l]; sum[1][l] = sum[1][l] + sum[3][l]; }
    for (int l = 0; l < 16; ++l) sum[0][l] = sum[0][l] + sum[1][l];
    float sumf = reduce16(sum[0]);
    int i = np;
    for (; n - i >= 16; i += 16)
        for (int l = 0; l < 16; ++l) sumf = sumf + x[i + l] * y[i + l];
    if (n - i >= 8) {
        for (int l = 0; l < 8; ++l) sumf = sumf + x[i + l] * y[i + l];
        i += 8;
    }
    for (; i < n; ++i) sumf = fmaf(x[i], y[i], sumf);
    return sumf;
}

// ------------------------------------------------------------ SIMD math ----

// ggml-cpu/vec.h:1191-1216 (ggml_v_expf, AVX-512): exp via 2^n * poly(b),
// restated lane-wise with the same fused multiply-adds.
float v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    const bool d = std::fabs(n) > 192.0f;
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u, fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                         u, fmaf(0x1.ffffecp-1f, b, 1.0f));
    if (d) return n <= 0.0f ? 0.0f : INFINITY;
    return std::ldexp(j, (int)n);   // _mm512_scalef_ps(j, n); n is integral here
}

// ggml-cpu/vec.h:1219-1226
float v_silu(float x) {
    const float neg_x = 0.0f - x;
    const float e = v_expf(neg_x);
    return x / (1.0f + e);
}

// ggml-cpu/vec.h:1065-1067 (scalar tail)
float silu_scalar(float x) { return x / (1.0f + std::exp(-x)); }

// ggml-cpu/vec.cpp:417-445: 16-lane body, scalar libm tail.
void vec_swiglu(int n, float * y, const float * x, const float * g) {
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int l = 0; l < 16; ++l) y[i + l] = v_silu(x[i + l]) * g[i + l];
    for (; i < n; ++i) y[i] = silu_scalar(x[i]) * g[i];
}
// ggml-cpu/vec.cpp:380-415
void vec_silu(int n, float * y, const float * x) {
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int l = 0; l < 16; ++l) y[i + l] = v_silu(x[i + l]);
    for (; i < n; ++i) y[i] = silu_scalar(x[i]);
}

// ggml-cpu/ops.cpp:5813-5920 + vec.cpp:531-600 (AVX-512): row max, 16-wide
// v_expf chunks summed with the 16-lane tree into a double, libm tail,
// then multiply by (float)(1/sum).
void soft_max_row(int n, const float * x, float * y) {
    float max = -INFINITY;
    for (int i = 0; i < n; ++i) max = std::max(max, x[i]);
    double sum = 0;
    int i = 0;
    for (; i + 15 < n; i += 16) {
        float v[16];
        for (int l = 0; l < 16; ++l) { v[l] = v_expf(x[i + l] - max); y[i + l] = v[l]; }
        sum += (double)reduce16(v);
    }
    for (; i < n; ++i) { const float v = std::exp(x[i] - max); sum += (double)v; y[i] = v; }
    sum = 1.0 / sum;
    const float s = (float)sum;
    for (int k = 0; k < n; ++k) y[k] *= s;
}

// ggml-cpu/ops.cpp:8706-8756 (descending argsort with std::sort and a strict
// ">" comparator; ggml_argsort_top_k keeps the first k, ggml.c:5462-5478).
void argsort_desc(int n, const float * x, int32_t * idx) {
    for (int j = 0; j < n; ++j) idx[j] = j;
    std::sort(idx, idx + n, [x](int32_t a, int32_t b) { return x[a] > x[b]; });
}

// ggml-cpu/vec.h:1618-1626: the last index among equal maxima wins.
int argmax_last(int n, const float * x) {
    float max = -INFINITY;
    int idx = 0;
    for (int i = 0; i < n; ++i) {
        max = (max > x[i]) ? max : x[i];
        if (max == x[i]) idx = i;
    }
    return idx;
}

// ------------------------------------------------------------ mat-vec ops ----

size_t row_bytes(int type, int64_t k) {
    switch (type) {
        case T_F32: return (size_t)k * 4;
        case T_Q8_0: return (size_t)(k / QK8_0) * sizeof(block_q8_0);
        case T_Q4_K: return (size_t)(k / QK_K) * sizeof(block_q4_K);
        case T_Q6_K: return (size_t)(k / QK_K) * sizeof(block_q6_K);
        case T_Q5_K: return (size_t)(k / QK_K) * sizeof(block_q5_K);
        case T_Q8_K: return (size_t)(k / QK_K) * sizeof(block_q8_K);
    }
    throw std::invalid_argument("unsupported ggml type");
}
// type_traits_cpu[type].vec_dot_type (ggml-cpu.c:216-320)
int vec_dot_type(int type) {
    switch (type) {
        case T_Q4_K: return T_Q8_K;
        case T_Q6_K: return T_Q8_K;
        case T_Q5_K: return T_Q8_K;
        case T_Q8_0: return T_Q8_0;
        case T_F32: return T_F32;
    }
    throw std::invalid_argument("unsupported weight type");
}
void from_float(int vtype, const float * x, void * y, int64_t k) {
    switch (vtype) {
        case T_Q8_K: quantize_row_q8_K(x, (block_q8_K *)y, k); return;
        case T_Q8_0: quantize_row_q8_0_x86(x, (block_q8_0 *)y, k); return;
        case T_F32: std::memcpy(y, x, (size_t)k * 4); return;
    }
}
float dot_row(int type, int k, const void * w, const void * xq) {
    switch (type) {
        case T_Q4_K: return vec_dot_q4_K_q8_K(k, (const block_q4_K *)w, (const block_q8_K *)xq);
        case T_Q6_K: return vec_dot_q6_K_q8_K(k, (const block_q6_K *)w, (const block_q8_K *)xq);
        case T_Q5_K: return vec_dot_q5_K_q8_K(k, (const block_q5_K *)w, (const block_q8_K *)xq);
        case T_Q8_0: return vec_dot_q8_0_q8_0(k, (const block_q8_0 *)w, (const block_q8_0 *)xq);
        case T_F32: return vec_dot_f32(k, (const float *)w, (const float *)xq);
    }
    throw std::invalid_argument("unsupported weight type");
}

// Runs fn(i) for i in [0, n) over the host's threads when n is large.  Every
// output element is computed by one call in its own fixed order, so the split
// changes nothing but the wall time of large fixtures.
void parallel_for(int64_t n, const std::function<void(int64_t)> & fn) {
    const int64_t nt = std::max<int64_t>(1, std::min<int64_t>(n / 16, (int64_t)std::thread::hardware_concurrency()));
    if (nt <= 1) { for (int64_t i = 0; i < n; ++i) fn(i); return; }
    std::vector<std::thread> pool;
    for (int64_t w = 0; w < nt; ++w)
        pool.emplace_back([&, w]() { for (int64_t i = w; i < n; i += nt) fn(i); });
    for (auto & th : pool) th.join();
}

// ggml-cpu.c:1554-1734: quantize every column of b to the weight's
// vec_dot_type, then dst[:, e, t] = as[:, :, ids[e,t]] . b[:, e % ne11, t].
// (The tiled path that ggml takes for experts with >= 8 routed columns sums
// blocks in another order; within a block the integer sums are identical.)
void mul_mat_id(int type, const void * as, int64_t K, int64_t N, int64_t n_as,
                const float * b, int64_t ne11, int64_t T,
                const int32_t * ids, int64_t n_ids, float * dst) {
    const int vt = vec_dot_type(type);
    const size_t qrow = row_bytes(vt, K);
    std::vector<uint8_t> bq((size_t)(ne11 * T) * qrow);
    for (int64_t t = 0; t < T; ++t)
        for (int64_t i = 0; i < ne11; ++i)
            from_float(vt, b + (t * ne11 + i) * K, bq.data() + (size_t)(t * ne11 + i) * qrow, K);
    const size_t wrow = row_bytes(type, K);
    for (int64_t i = 0; i < T * n_ids; ++i)
        if (ids[i] < 0 || ids[i] >= n_as) throw std::out_of_range("mul_mat_id: expert id out of range");
    parallel_for(T * n_ids, [&](int64_t i) {
        const int64_t t = i / n_ids, e = i % n_ids;
        const uint8_t * slab = (const uint8_t *)as + (size_t)ids[i] * N * wrow;
        const uint8_t * col = bq.data() + (size_t)(t * ne11 + e % ne11) * qrow;
        float * out = dst + i * N;
        for (int64_t r = 0; r < N; ++r) out[r] = dot_row(type, (int)K, slab + (size_t)r * wrow, col);
    });
}

// Dense mul_mat (ggml-cpu.c:1165-1244 one_chunk, 1257-1470): vec_dot per
// (row, column) for every type on this path, f32 included, at any column
// count: the reference builds ggml-cpu without llamafile (the branch at
// ggml-cpu.c:1300 is compiled out) and its tiled path takes only K-quant and
// IQ weights (tiled/tiled.cpp:605-640).
void mul_mat(int type, const void * w, int64_t K, int64_t N, const float * x, int64_t T, float * dst) {
    const size_t wrow = row_bytes(type, K);
    if (type == T_F32) {
        for (int64_t t = 0; t < T; ++t)
            for (int64_t r = 0; r < N; ++r) {
                const float * wr = (const float *)((const uint8_t *)w + (size_t)r * wrow);
                dst[t * N + r] = vec_dot_f32((int)K, wr, x + t * K);
            }
        return;
    }
    const int vt = vec_dot_type(type);
    const size_t qrow = row_bytes(vt, K);
    std::vector<uint8_t> xq((size_t)T * qrow);
    for (int64_t t = 0; t < T; ++t) from_float(vt, x + t * K, xq.data() + (size_t)t * qrow, K);
    parallel_for((N + 255) / 256, [&](int64_t c) {
        for (int64_t r = 256 * c; r < std::min<int64_t>(N, 256 * (c + 1)); ++r)
            for (int64_t t = 0; t < T; ++t)
                dst[t * N + r] = dot_row(type, (int)K, (const uint8_t *)w + (size_t)r * wrow, xq.data() + (size_t)t * qrow);
    });
}

}  // namespace

// ====================================================================
// C ABI of the oracle (ctypes from tests/, smoke() and bench.py only)
// ====================================================================

QWO_API uint16_t qwo_fp32_to_fp16(float f) { return fp32_to_fp16(f); }
QWO_API float qwo_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
// Rows are independent (ggml's quantize_q4_K loops over them); they are split
// over threads here only to keep large test fixtures quick to build.
QWO_API void qwo_quantize_q4_K(const float * x, void * y, int64_t nrow, int64_t k) {
    const int64_t nt = std::max<int64_t>(1, std::min<int64_t>(nrow / 64, (int64_t)std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (int64_t w = 0; w < nt; ++w)
        pool.emplace_back([=]() {
            for (int64_t r = w; r < nrow; r += nt) quantize_row_q4_K(x + r * k, (block_q4_K *)y + r * (k / QK_K), k);
        });
    for (auto & th : pool) th.join();
}
QWO_API void qwo_dequantize_q4_K(const void * x, float * y, int64_t k) { dequantize_row_q4_K((const block_q4_K *)x, y, k); }
QWO_API void qwo_quantize_q8_K(const float * x, void * y, int64_t k) { quantize_row_q8_K(x, (block_q8_K *)y, k); }
QWO_API void qwo_quantize_q8_0_ref(const float * x, void * y, int64_t k) { quantize_row_q8_0_ref(x, (block_q8_0 *)y, k); }
QWO_API void qwo_quantize_q8_0_x86(const float * x, void * y, int64_t k) { quantize_row_q8_0_x86(x, (block_q8_0 *)y, k); }
QWO_API float qwo_vec_dot_q4_K_q8_K(int n, const void * x, const void * y) { return vec_dot_q4_K_q8_K(n, (const block_q4_K *)x, (const block_q8_K *)y); }
QWO_API float qwo_vec_dot_q5_K_q8_K(int n, const void * x, const void * y) { return vec_dot_q5_K_q8_K(n, (const block_q5_K *)x, (const block_q8_K *)y); }
QWO_API float qwo_vec_dot_q6_K_q8_K(int n, const void * x, const void * y) { return vec_dot_q6_K_q8_K(n, (const block_q6_K *)x, (const block_q8_K *)y); }
QWO_API void qwo_dequantize_q6_K(const void * x, float * y, int64_t k) { dequantize_row_q6_K((const block_q6_K *)x, y, k); }
QWO_API float qwo_vec_dot_q8_0_q8_0(int n, const void * x, const void * y) { return vec_dot_q8_0_q8_0(n, (const block_q8_0 *)x, (const block_q8_0 *)y); }
QWO_API float qwo_vec_dot_f32(int n, const float * x, const float * y) { return vec_dot_f32(n, x, y); }
QWO_API float qwo_v_expf(float x) { return v_expf(x); }
QWO_API float qwo_v_silu(float x) { return v_silu(x); }
QWO_API void qwo_swiglu(int n, float * y, const float * gate, const float * up) { vec_swiglu(n, y, gate, up); }
QWO_API void qwo_soft_max_row(int n, const float * x, float * y) { soft_max_row(n, x, y); }
QWO_API void qwo_argsort_desc(int n, const float * x, int32_t * idx) { argsort_desc(n, x, idx); }
QWO_API int qwo_argmax(int n, const float * x) { return argmax_last(n, x); }
QWO_API size_t qwo_row_bytes(int type, int64_t k) { return row_bytes(type, k); }

QWO_API int qwo_mul_mat_id(int type, const void * as, int64_t K, int64_t N, int64_t n_as,
                           const float * b, int64_t ne11, int64_t T, const int32_t * ids, int64_t n_ids, float * dst) {
    try { mul_mat_id(type, as, K, N, n_as, b, ne11, T, ids, n_ids, dst); return 0; }
    catch (...) { return -1; }
}
QWO_API int qwo_mul_mat(int type, const void * w, int64_t K, int64_t N, const float * x, int64_t T, float * dst) {
    try { mul_mat(type, w, K, N, x, T, dst); return 0; }
    catch (...) { return -1; }
}

// core/runtime.cpp:2693-2734 (route_experts) after the router mul_mat
// (build_router 3785-3798 / build_segB router 4515-4519):
//   logits = W_r . x (+ rm);
//   probs = soft_max(logits), or sigmoid(logits) when gating_func == 2
//     (hparams.gating_sigmoid(), core/model.h:160; ggml-cpu unary-ops.cpp:31-33:
//     1 / (1 + expf(-x)) with the C library's expf);
//   rank = probs; with exp_probs_b: rank = probs + bias, then + rm again;
//   sel = argsort_top_k(rank);  w = probs[sel];
//   if norm: w /= clamp(sum(w), 6.103515625e-5, inf); if scale not in {0, 1}: w *= scale.
// Outputs: ids [T][k] (token-major, k order), weights [T][k]; optional
// logits/probs [T][E] and the rank margin (rank[k-1] - rank[k]) per token.
QWO_API int qwo_route_ex(int64_t E, int64_t H, int64_t T, const float * Wr, const float * x, const float * rm,
                         const float * bias, int gating_func, int k, int norm, float scale, int32_t * ids,
                         float * weights, float * logits_out, float * probs_out, float * margin_out) {
    try {
        if (k < 1 || k > E || k > 512) return -1;
        std::vector<float> logits((size_t)(E * T)), probs((size_t)(E * T)), rank((size_t)E);
        mul_mat(T_F32, Wr, H, E, x, T, logits.data());
        for (int64_t t = 0; t < T; ++t) {
            float * lt = logits.data() + t * E;
            if (rm) for (int64_t e = 0; e < E; ++e) lt[e] = lt[e] + rm[t * E + e];
            float * pt = probs.data() + t * E;
            if (gating_func == 2)
                for (int64_t e = 0; e < E; ++e) pt[e] = 1.0f / (1.0f + expf(-lt[e]));
            else
                soft_max_row((int)E, lt, pt);
            for (int64_t e = 0; e < E; ++e) {
                rank[e] = pt[e];
                if (bias) {
                    rank[e] = rank[e] + bias[e];
                    if (rm) rank[e] = rank[e] + rm[t * E + e];
                }
            }
            std::vector<int32_t> idx((size_t)E);
            argsort_desc((int)E, rank.data(), idx.data());
            float w[512];
            for (int j = 0; j < k; ++j) { ids[t * k + j] = idx[j]; w[j] = pt[idx[j]]; }
            if (margin_out) margin_out[t] = (k < E) ? rank[idx[k - 1]] - rank[idx[k]] : INFINITY;
            if (norm) {
                double s = 0.0;
                for (int j = 0; j < k; ++j) s += (double)w[j];
                float ws = (float)s;
                ws = std::max(std::min(ws, INFINITY), 6.103515625e-5f);
                for (int j = 0; j < k; ++j) w[j] = w[j] / ws;
            }
            if (scale != 0.0f && scale != 1.0f)
                for (int j = 0; j < k; ++j) w[j] = w[j] * scale;
            for (int j = 0; j < k; ++j) weights[t * k + j] = w[j];
        }
        if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);
        if (probs_out) std::memcpy(probs_out, probs.data(), probs.size() * 4);
        return 0;
    } catch (...) { return -1; }
}
QWO_API int qwo_route(int64_t E, int64_t H, int64_t T, const float * Wr, const float * x, const float * rm,
                      int k, int norm, float scale, int32_t * ids, float * weights,
                      float * logits_out, float * probs_out, float * margin_out) {
    return qwo_route_ex(E, H, T, Wr, x, rm, nullptr, 1, k, norm, scale, ids, weights, logits_out, probs_out, margin_out);
}

// The C library's expf and the sigmoid built on it (ggml-cpu unary-ops.cpp:31-33).
QWO_API float qwo_expf(float x) { return expf(x); }
QWO_API float qwo_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// One MoE FFN block over the slot pools: core/runtime.cpp:3801-3830
// (build_moe_cached, T=1) and 4534-4572 (build_segB, T>1).
//   up = mul_mat_id(up_pool, x, slot_u); gate = mul_mat_id(gate_pool, x, slot_g)
//   act = swiglu_split(gate, up); experts = mul_mat_id(down_pool, act, slot_d)
//   T == 1: out = mul_mat(cont(transpose(experts)), w)  -- vec_dot_f32, n = k
//   T >  1: out = ((e0*w0 + e1*w1) + e2*w2) + ...       -- ggml_mul, ggml_add chain
//   shared expert (if sh_gate): sh = down_sh(silu(gate_sh x) * up_sh x)
//     [ * sigmoid(gate_inp_sh . x) ];  out += sh
// Pools are [K, N, n_slots] Q4_K (or Q8_0) slabs; slot ids are [T][k].
// Optional intermediates: gate/up/act [T][k][N], experts [T][k][H].
struct qwo_moe_args {
    int64_t H, N, k, T;
    int weight_type;
    const void * gate_pool; const void * up_pool; const void * down_pool; int64_t n_slots;
    const int32_t * slot_g; const int32_t * slot_u; const int32_t * slot_d;
    const float * weights;          // [T][k]
    const float * x;                // [T][H]
    const void * sh_gate; const void * sh_up; const void * sh_down; int64_t N_sh;  // optional
    const float * sh_gate_inp;      // optional f32 [H]
    float * out;                    // [T][H]
    float * gate_out; float * up_out; float * act_out; float * experts_out;  // optional
    int down_type;                  // type of the down pool; 0: weight_type (Q4_K_M files store some as Q6_K)
};

QWO_API int qwo_moe_block(const qwo_moe_args * a) {
    try {
        const int64_t H = a->H, N = a->N, k = a->k, T = a->T;
        std::vector<float> gate((size_t)(T * k * N)), up((size_t)(T * k * N)), act((size_t)(T * k * N));
        std::vector<float> ex((size_t)(T * k * H));
        mul_mat_id(a->weight_type, a->up_pool, H, N, a->n_slots, a->x, 1, T, a->slot_u, k, up.data());
        mul_mat_id(a->weight_type, a->gate_pool, H, N, a->n_slots, a->x, 1, T, a->slot_g, k, gate.data());
        for (int64_t r = 0; r < T * k; ++r) vec_swiglu((int)N, act.data() + r * N, gate.data() + r * N, up.data() + r * N);
        mul_mat_id(a->down_type ? a->down_type : a->weight_type, a->down_pool, N, H, a->n_slots, act.data(), k, T,
                   a->slot_d, k, ex.data());
        for (int64_t t = 0; t < T; ++t) {
            float * o = a->out + t * H;
            const float * w = a->weights + t * k;
            if (T == 1) {
                std::vector<float> col((size_t)k);
                for (int64_t h = 0; h < H; ++h) {
                    for (int64_t j = 0; j < k; ++j) col[j] = ex[(t * k + j) * H + h];
                    o[h] = vec_dot_f32((int)k, col.data(), w);
                }
            } else {
                for (int64_t h = 0; h < H; ++h) {
                    float s = ex[(t * k + 0) * H + h] * w[0];
                    for (int64_t j = 1; j < k; ++j) s = s + ex[(t * k + j) * H + h] * w[j];
                    o[h] = s;
                }
            }
        }
        if (a->sh_gate) {
            const int64_t Ns = a->N_sh;
            std::vector<float> g((size_t)(T * Ns)), u((size_t)(T * Ns)), s((size_t)(T * Ns)), sh((size_t)(T * H));
            mul_mat(a->weight_type, a->sh_gate, H, Ns, a->x, T, g.data());
            mul_mat(a->weight_type, a->sh_up, H, Ns, a->x, T, u.data());
            for (int64_t t = 0; t < T; ++t) {
                vec_silu((int)Ns, s.data() + t * Ns, g.data() + t * Ns);
                for (int64_t i = 0; i < Ns; ++i) s[t * Ns + i] = s[t * Ns + i] * u[t * Ns + i];
            }
            mul_mat(a->down_type ? a->down_type : a->weight_type, a->sh_down, Ns, H, s.data(), T, sh.data());
            for (int64_t t = 0; t < T; ++t) {
                float gsc = 1.0f;
                if (a->sh_gate_inp) {
                    const float z = vec_dot_f32((int)H, a->sh_gate_inp, a->x + t * H);
                    gsc = 1.f / (1.f + std::exp(-z));   // ggml-cpu/unary-ops.cpp:31 (libm expf)
                }
                for (int64_t h = 0; h < H; ++h) {
                    const float v = a->sh_gate_inp ? sh[t * H + h] * gsc : sh[t * H + h];
                    a->out[t * H + h] = a->out[t * H + h] + v;
                }
            }
        }
        if (a->gate_out) std::memcpy(a->gate_out, gate.data(), gate.size() * 4);
        if (a->up_out) std::memcpy(a->up_out, up.data(), up.size() * 4);
        if (a->act_out) std::memcpy(a->act_out, act.data(), act.size() * 4);
        if (a->experts_out) std::memcpy(a->experts_out, ex.data(), ex.size() * 4);
        return 0;
    } catch (...) { return -1; }
}

// Verify head (core/runtime.cpp:5014-5046): h = rms_norm(resid + moe) * norm_w
// (ggml-cpu/ops.cpp:4120-4160: double sum of float squares, scale =
// 1/sqrtf(mean + eps)); logits = Q8_0 lm_head . h; vA[t] = argmax (last index
// on ties).  Accept (runtime.cpp:3648-3652): a = longest prefix with
// vA[j] == drafts[j] (j < K); x_new = vA[a].
QWO_API void qwo_rms_norm(int64_t H, const float * x, float eps, const float * norm_w, float * y) {
    double sum = 0.0;
    for (int64_t i = 0; i < H; ++i) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)H);
    const float scale = 1.0f / std::sqrt(mean + eps);
    for (int64_t i = 0; i < H; ++i) y[i] = x[i] * scale;
    if (norm_w) for (int64_t i = 0; i < H; ++i) y[i] = y[i] * norm_w[i];
}

QWO_API int qwo_lm_head_argmax(const void * w_q8_0, int64_t H, int64_t V, const float * h, int64_t T,
                               int32_t * vA, float * logits_out, float * margin_out) {
    try {
        std::vector<float> logits((size_t)(V * T));
        mul_mat(T_Q8_0, w_q8_0, H, V, h, T, logits.data());
        for (int64_t t = 0; t < T; ++t) {
            const float * lt = logits.data() + t * V;
            vA[t] = argmax_last((int)V, lt);
            if (margin_out) {
                float best = -INFINITY, second = -INFINITY;
                for (int64_t v = 0; v < V; ++v) {
                    if (lt[v] > best) { second = best; best = lt[v]; }
                    else if (lt[v] > second) second = lt[v];
                }
                margin_out[t] = best - second;
            }
        }
        if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);
        return 0;
    } catch (...) { return -1; }
}

QWO_API int qwo_accept(const int32_t * vA, const int32_t * drafts, int K, int32_t * x_new) {
    int a = 0;
    while (a < K && vA[a] == drafts[a]) ++a;
    *x_new = vA[a];
    return a;
}

// ====================================================================
// Slot pool: the RAM-tier decisions of core/expert_cache.cpp (ensure
// 1615-1645, slot_for 1465-1479, install 1173-1180, pick_victim 1129-1170
// with activation scores off, release_victim/drop_slot 1067-1088,
// publish/record hooks gpu_lru_pool_hooks.h:11-79).  Signature pools
// (225-296): one pool per (role, type, ne0, ne1), every (role, layer)
// routed to one of them; one clock shared by all pools; per id the roles go
// gate, up, down.  qwo_pool_new makes the three-pool case (pool r serves
// role r of every layer).  Victim: the lowest free slot, else the minimum
// clock among unprotected occupied slots (strict <, so the lowest slot wins
// ties and a UINT64_MAX clock never wins).  Protection
// (ActiveExpertGuard, expert_cache.cpp:46-59) only exists when the demand
// table is allocated, i.e. under the TinyLFU admission mode; `protect`
// selects it.
// ====================================================================
struct qwo_pool {
    int n_layer, n_expert;
    bool protect;
    uint64_t clock = 0;
    uint64_t hits = 0, misses = 0, evictions = 0;
    struct Pool {
        int role = 0;
        int n_slots = 0;
        std::vector<int> slot2key;
        std::vector<uint64_t> clk;
        std::unordered_map<int, int> key2slot;
        std::vector<int32_t> slot_of;
        std::vector<int> occ;
        std::unordered_map<int, uint64_t> count;
        std::vector<int> quota;         // per layer, after a rebalance
    };
    std::vector<Pool> pools;
    std::vector<int> lp[3];             // pool index of (role, layer)
    std::vector<uint8_t> active;
    bool quota_on = false;
    int n_used = 0;
    Pool & P(int r, int l) { return pools[(size_t)lp[r][(size_t)l]]; }
    const Pool & P(int r, int l) const { return pools[(size_t)lp[r][(size_t)l]]; }
};

// pick_victim (expert_cache.cpp:1129-1170, activation scores off): the lowest
// free slot; else, without quotas, the minimum clock among unprotected
// occupied slots; with quotas (after a rebalance) a layer at or over its
// quota takes from its own slots and any other layer from layers over their
// quotas, and if that finds nothing, the global minimum clock.
static int qwo_pick(const qwo_pool * p, const qwo_pool::Pool & R, int layer) {
    const bool self = p->quota_on && R.quota[(size_t)layer] >= 0 && R.occ[(size_t)layer] >= R.quota[(size_t)layer];
    int victim = -1;
    uint64_t best = UINT64_MAX;
    for (int s = 0; s < R.n_slots; ++s) {
        const int ks = R.slot2key[(size_t)s];
        if (ks < 0) return s;
        if (p->protect && p->active[(size_t)ks]) continue;
        if (p->quota_on) {
            const int kl = ks / p->n_expert;
            if (self) { if (kl != layer) continue; }
            else if (R.occ[(size_t)kl] <= R.quota[(size_t)kl]) continue;
        }
        if (R.clk[(size_t)s] < best) { best = R.clk[(size_t)s]; victim = s; }
    }
    if (victim >= 0 || !p->quota_on) return victim;
    for (int s = 0; s < R.n_slots; ++s) {
        const int ks = R.slot2key[(size_t)s];
        if (p->protect && ks >= 0 && p->active[(size_t)ks]) continue;
        if (R.clk[(size_t)s] < best) { best = R.clk[(size_t)s]; victim = s; }
    }
    return victim;
}

// install (expert_cache.cpp:1173-1180): pick, drop, publish with clock + 1.
static int qwo_install(qwo_pool * p, qwo_pool::Pool & R, int key, int layer) {
    const int victim = qwo_pick(p, R, layer);
    if (victim < 0) return -1;
    const int old = R.slot2key[(size_t)victim];
    if (old >= 0) {
        R.occ[(size_t)(old / p->n_expert)]--;
        R.slot_of[(size_t)old] = 0;
        R.key2slot.erase(old);
        R.slot2key[(size_t)victim] = -1;
        p->evictions++;
    }
    R.key2slot.emplace(key, victim);
    R.slot2key[(size_t)victim] = key;
    R.occ[(size_t)layer]++;
    R.slot_of[(size_t)key] = victim;
    p->clock += 1;
    R.clk[(size_t)victim] = p->clock;
    return victim;
}

// Signature pools: pool_slots [n_pools], pool_role [n_pools], layer_pool
// [3 * n_layer] (role-major).  Returns NULL when a (role, layer) names a
// pool out of range or of another role.
QWO_API qwo_pool * qwo_pool_new_sig(int n_layer, int n_expert, int n_pools, const int32_t * pool_slots,
                                    const int32_t * pool_role, const int32_t * layer_pool, int protect) {
    auto * p = new qwo_pool();
    p->n_layer = n_layer; p->n_expert = n_expert; p->protect = protect != 0;
    p->pools.resize((size_t)n_pools);
    for (int i = 0; i < n_pools; ++i) {
        auto & R = p->pools[(size_t)i];
        R.role = pool_role[i];
        R.n_slots = pool_slots[i];
        R.slot2key.assign((size_t)R.n_slots, -1);
        R.clk.assign((size_t)R.n_slots, 0);
        R.slot_of.assign((size_t)n_layer * n_expert, 0);
        R.occ.assign((size_t)n_layer, 0);
        R.quota.assign((size_t)n_layer, -1);
    }
    for (int r = 0; r < 3; ++r) {
        p->lp[r].assign(layer_pool + (size_t)r * n_layer, layer_pool + (size_t)(r + 1) * n_layer);
        for (int l = 0; l < n_layer; ++l) {
            const int i = p->lp[r][(size_t)l];
            if (i < 0 || i >= n_pools || p->pools[(size_t)i].role != r) { delete p; return nullptr; }
        }
    }
    if (p->protect) p->active.assign((size_t)n_layer * n_expert, 0);
    return p;
}
QWO_API qwo_pool * qwo_pool_new(int n_layer, int n_expert, const int32_t * n_slots, int protect) {
    const int32_t roles[3] = {0, 1, 2};
    std::vector<int32_t> lp((size_t)3 * n_layer);
    for (int r = 0; r < 3; ++r)
        for (int l = 0; l < n_layer; ++l) lp[(size_t)r * n_layer + l] = r;
    return qwo_pool_new_sig(n_layer, n_expert, 3, n_slots, roles, lp.data(), protect);
}
QWO_API void qwo_pool_free(qwo_pool * p) { delete p; }
QWO_API int qwo_pool_layer_pool(const qwo_pool * p, int role, int layer) { return p->lp[role][(size_t)layer]; }

// Signature discovery and sizing (expert_cache.cpp:225-287): for roles in
// order and layers in order, the expert tensor's (type, ne0, ne1) finds its
// signature (the first with the same role, type and shape) or opens a new
// one; each signature counts its layers.  frac = vram / sum(slab * n_layers *
// n_expert), at most 1 (1 when the sum is 0); a pool gets (int)(frac * cap)
// slots, cap = n_layers * n_expert, raised to n_used and cut to cap; a pool
// of n_used slots or fewer is refused (the reference throws: with the
// transient workspace off it must hold more than n_used).  tensors: per
// (role, layer), role-major, {type, ne0, ne1, slab}.  sigs_out: per signature
// {role, type, ne0, ne1, slab, n_layers, n_slots}, at most max_sigs.
// Returns the signature count, -1 when a pool is too small, -2 when
// max_sigs is exceeded.
QWO_API int qwo_pool_plan_sigs(int n_layer, int n_expert, const int64_t * tensors, uint64_t vram, int n_used,
                               int64_t * sigs_out, int max_sigs, int32_t * layer_pool, double * frac_out) {
    int ns = 0;
    for (int r = 0; r < 3; ++r)
        for (int l = 0; l < n_layer; ++l) {
            const int64_t * t = tensors + 4 * ((size_t)r * n_layer + l);
            int idx = -1;
            for (int s = 0; s < ns; ++s) {
                const int64_t * g = sigs_out + 7 * s;
                if (g[0] == r && g[1] == t[0] && g[2] == t[1] && g[3] == t[2]) { idx = s; break; }
            }
            if (idx < 0) {
                if (ns >= max_sigs) return -2;
                idx = ns++;
                int64_t * g = sigs_out + 7 * idx;
                g[0] = r; g[1] = t[0]; g[2] = t[1]; g[3] = t[2]; g[4] = t[3]; g[5] = 0; g[6] = 0;
            }
            sigs_out[7 * idx + 5]++;
            layer_pool[(size_t)r * n_layer + l] = idx;
        }
    uint64_t total = 0;
    for (int s = 0; s < ns; ++s) total += (uint64_t)sigs_out[7 * s + 4] * (uint64_t)sigs_out[7 * s + 5] * (uint64_t)n_expert;
    double frac = total ? (double)vram / (double)total : 1.0;
    if (frac > 1.0) frac = 1.0;
    if (frac_out) *frac_out = frac;
    for (int s = 0; s < ns; ++s) {
        const int cap = (int)sigs_out[7 * s + 5] * n_expert;
        int n = (int)(frac * cap);
        if (n < n_used) n = n_used;
        if (n > cap) n = cap;
        if (n <= n_used) return -1;
        sigs_out[7 * s + 6] = n;
    }
    return ns;
}

// Returns 0, or -1 when no unprotected victim exists ("No unprotected GPU
// cache victim").  fetch_log (optional, 4 ints per fetch: role, layer,
// expert, slot) records the slab copies in order; *n_fetch gets their count.
QWO_API int qwo_pool_ensure(qwo_pool * p, int layer, const int32_t * ids, int n,
                            int32_t * slot_g, int32_t * slot_u, int32_t * slot_d,
                            int32_t * fetch_log, int * n_fetch) {
    int nf = 0;
    std::vector<size_t> changed;
    if (p->protect)
        for (int i = 0; i < n; ++i) {
            const size_t key = (size_t)layer * p->n_expert + ids[i];
            if (!p->active[key]) { p->active[key] = 1; changed.push_back(key); }
        }
    int32_t * outs[3] = {slot_g, slot_u, slot_d};
    int rc = 0;
    for (int i = 0; i < n && rc == 0; ++i) {
        const int e = ids[i];
        const int key = layer * p->n_expert + e;
        for (int r = 0; r < 3; ++r) {
            auto & R = p->P(r, layer);
            R.count[key]++;
            auto it = R.key2slot.find(key);
            if (it != R.key2slot.end()) {
                p->hits++;
                p->clock += 1;
                R.clk[(size_t)it->second] = p->clock;
                outs[r][i] = it->second;
                continue;
            }
            p->misses++;
            const int victim = qwo_install(p, R, key, layer);
            if (victim < 0) { rc = -1; break; }
            if (fetch_log) {
                fetch_log[4 * nf + 0] = r; fetch_log[4 * nf + 1] = layer;
                fetch_log[4 * nf + 2] = e; fetch_log[4 * nf + 3] = victim;
            }
            ++nf;
            outs[r][i] = victim;
        }
    }
    for (size_t key : changed) p->active[key] = 0;
    if (n_fetch) *n_fetch = nf;
    return rc;
}
// ExpertCache::save_profile (expert_cache.cpp:1485-1500) as text into buf
// (cap bytes): "QWENEXPCACHE 1", "n_layer n_expert", then "role layer expert
// count" for every counted key, pools in order, keys ascending within a pool
// (the reference walks each pool's count map in hash order; the loader below
// reads any order).  Returns the text length, or -1 if it does not fit.
QWO_API int qwo_pool_save_profile(const qwo_pool * p, char * buf, int cap) {
    std::string s = "QWENEXPCACHE 1\n" + std::to_string(p->n_layer) + " " + std::to_string(p->n_expert) + "\n";
    for (const auto & R : p->pools) {
        std::vector<std::pair<int, uint64_t>> kv(R.count.begin(), R.count.end());
        std::sort(kv.begin(), kv.end());
        for (const auto & c : kv)
            s += std::to_string(R.role) + " " + std::to_string(c.first / p->n_expert) + " " +
                 std::to_string(c.first % p->n_expert) + " " + std::to_string(c.second) + "\n";
    }
    if ((int)s.size() + 1 > cap) return -1;
    std::memcpy(buf, s.c_str(), s.size() + 1);
    return (int)s.size();
}

// ExpertCache::load_prefetch (expert_cache.cpp:1502-1538) from profile text:
// a header other than "QWENEXPCACHE 1" with this pool's n_layer and n_expert
// is a cold start (nothing installed, returns 0).  Entries with role, layer
// and expert in range are ordered by count, largest first (a stable order:
// equal counts keep the text's order, where the reference's std::sort leaves
// it unspecified); each is installed -- lowest free slot, drop-free, clock +
// 1, uncounted -- unless the pool of its (role, layer) is full or the key is
// resident.  fetch_log as in qwo_pool_ensure.  Returns the number of installs.
QWO_API int qwo_pool_load_profile(qwo_pool * p, const char * text, int32_t * fetch_log) {
    int ver = 0, nl = 0, ne = 0, used = 0;
    if (std::sscanf(text, "QWENEXPCACHE %d%n", &ver, &used) != 1 || ver != 1) return 0;
    text += used;
    if (std::sscanf(text, "%d %d%n", &nl, &ne, &used) != 2 || nl != p->n_layer || ne != p->n_expert) return 0;
    text += used;
    struct Ent { int r, l, e; unsigned long long c; };
    std::vector<Ent> ents;
    Ent en;
    while (std::sscanf(text, "%d %d %d %llu%n", &en.r, &en.l, &en.e, &en.c, &used) == 4) {
        text += used;
        if (en.r >= 0 && en.r < 3 && en.l >= 0 && en.l < p->n_layer && en.e >= 0 && en.e < p->n_expert) ents.push_back(en);
    }
    std::stable_sort(ents.begin(), ents.end(), [](const Ent & a, const Ent & b) { return a.c > b.c; });
    int n = 0;
    for (const Ent & x : ents) {
        auto & R = p->P(x.r, x.l);
        if ((int)R.key2slot.size() >= R.n_slots) continue;
        const int key = x.l * p->n_expert + x.e;
        if (R.key2slot.count(key)) continue;
        int slot = 0;
        while (R.slot2key[(size_t)slot] >= 0) ++slot;
        if (fetch_log) {
            fetch_log[4 * n + 0] = x.r; fetch_log[4 * n + 1] = x.l;
            fetch_log[4 * n + 2] = x.e; fetch_log[4 * n + 3] = slot;
        }
        R.key2slot.emplace(key, slot);
        R.slot2key[(size_t)slot] = key;
        R.occ[(size_t)x.l]++;
        R.slot_of[(size_t)key] = slot;
        p->clock += 1;
        R.clk[(size_t)slot] = p->clock;
        ++n;
    }
    return n;
}

// ExpertCache::compute_quota + rebalance (expert_cache.cpp:509-625): per-key
// counts summed over the pools, entries ordered by (count, key) descending;
// a layer takes one slot in each of the pools of its three roles, while all
// three have one left; floor: each layer up to n_used; then one more per
// entry beyond its layer's first n_used (quota < n_expert) while its pools
// have slots.  The same quota goes to each of a layer's pools; quotas on;
// then up to fill_budget experts, hottest first within each layer's quota,
// installed in every role that lacks them.  quota_out [n_layer] (optional).
// Returns the experts filled, or -1 when an install finds no victim.
QWO_API int qwo_pool_rebalance(qwo_pool * p, int n_used, int64_t fill_budget, int32_t * quota_out) {
    const int L = p->n_layer, E = p->n_expert;
    std::unordered_map<int, uint64_t> cnt;
    for (const auto & R : p->pools)
        for (const auto & kv : R.count) cnt[kv.first] += kv.second;
    std::vector<std::pair<uint64_t, int>> ents;
    for (const auto & kv : cnt) ents.emplace_back(kv.second, kv.first);
    std::sort(ents.begin(), ents.end(), std::greater<std::pair<uint64_t, int>>());
    std::vector<int> quota((size_t)L, 0);
    if (!cnt.empty()) {
        std::vector<int64_t> rem(p->pools.size());
        for (size_t i = 0; i < p->pools.size(); ++i) rem[i] = p->pools[i].n_slots;
        auto take = [&](int l) {
            for (int r = 0; r < 3; ++r)
                if (rem[(size_t)p->lp[r][(size_t)l]] <= 0) return false;
            for (int r = 0; r < 3; ++r) rem[(size_t)p->lp[r][(size_t)l]]--;
            return true;
        };
        for (int l = 0; l < L; ++l)
            while (quota[(size_t)l] < n_used && take(l)) quota[(size_t)l]++;
        std::vector<int> seen((size_t)L, 0);
        for (const auto & e : ents) {
            const int l = e.second / E;
            if (seen[(size_t)l]++ < n_used) continue;
            if (quota[(size_t)l] >= E) continue;
            if (!take(l)) continue;
            quota[(size_t)l]++;
        }
    }
    for (int l = 0; l < L; ++l)
        for (int r = 0; r < 3; ++r) p->P(r, l).quota[(size_t)l] = quota[(size_t)l];
    p->quota_on = true;
    p->n_used = n_used;
    if (quota_out) for (int l = 0; l < L; ++l) quota_out[l] = quota[(size_t)l];
    std::vector<int> seen((size_t)L, 0);
    int filled = 0;
    for (const auto & e : ents) {
        if (filled >= fill_budget) break;
        const int key = e.second, l = key / E;
        if (seen[(size_t)l] >= quota[(size_t)l]) continue;
        seen[(size_t)l]++;
        bool all = true;
        for (int r = 0; r < 3; ++r) all = all && p->P(r, l).key2slot.count(key);
        if (all) continue;
        for (int r = 0; r < 3; ++r) {
            auto & R = p->P(r, l);
            if (!R.key2slot.count(key) && qwo_install(p, R, key, l) < 0) return -1;
        }
        ++filled;
    }
    return filled;
}
QWO_API void qwo_pool_clear_counts(qwo_pool * p) { for (auto & R : p->pools) R.count.clear(); }

QWO_API void qwo_pool_stats(const qwo_pool * p, uint64_t * out3) {
    out3[0] = p->hits; out3[1] = p->misses; out3[2] = p->evictions;
}
QWO_API uint64_t qwo_pool_clock(const qwo_pool * p) { return p->clock; }
QWO_API void qwo_pool_slot_of_row(const qwo_pool * p, int role, int layer, int32_t * out) {
    std::memcpy(out, p->P(role, layer).slot_of.data() + (size_t)layer * p->n_expert, (size_t)p->n_expert * 4);
}
// ExpertCache::resident (expert_cache.cpp:1442-1446) and ::touch (1453-1463):
// a resident key counts one access, its slot takes clock + 1, the hit counter
// grows; the decode fast path touches GATE, UP, DOWN per selected expert
// (runtime.cpp:6170-6176).
QWO_API int qwo_pool_resident(const qwo_pool * p, int role, int layer, int expert) {
    return p->P(role, layer).key2slot.count(layer * p->n_expert + expert) ? 1 : 0;
}
QWO_API void qwo_pool_touch(qwo_pool * p, int layer, const int32_t * ids, int n) {
    for (int i = 0; i < n; ++i) {
        const int key = layer * p->n_expert + ids[i];
        for (int r = 0; r < 3; ++r) {
            auto & R = p->P(r, layer);
            auto it = R.key2slot.find(key);
            if (it == R.key2slot.end()) continue;
            R.count[key]++;
            p->clock += 1;
            R.clk[(size_t)it->second] = p->clock;
            p->hits++;
        }
    }
}
// ExpertCache::capacity (expert_cache.cpp:478-491) and ::quota_of (493-501),
// over the pools of the layer's three roles.
QWO_API int qwo_pool_capacity(const qwo_pool * p, int layer) {
    int m = INT32_MAX;
    for (int r = 0; r < 3; ++r) {
        const auto & R = p->P(r, layer);
        const int q = R.quota[(size_t)layer];
        m = std::min(m, p->quota_on && q >= 0 ? std::max(q, p->n_used) : R.n_slots);
    }
    return m;
}
QWO_API int qwo_pool_quota_of(const qwo_pool * p, int layer) {
    int m = INT32_MAX;
    for (int r = 0; r < 3; ++r) {
        const auto & R = p->P(r, layer);
        m = std::min(m, R.quota[(size_t)layer] >= 0 ? R.quota[(size_t)layer] : R.n_slots);
    }
    return m;
}
QWO_API void qwo_pool_set_quotas(qwo_pool * p, int on) { p->quota_on = on != 0; }
QWO_API int qwo_pool_quotas_active(const qwo_pool * p) { return p->quota_on ? 1 : 0; }

// decode_cached_batch's plan_slices (core/runtime.cpp:4639-4687): pass 1 the
// layer's union over the batch, quotas on iff it fits quota_of - 8; pass 2
// token slices whose union stays within max(n_used, capacity - 8) and whose
// length stays within max_slice (0: 1024).  slices: (t0, len) pairs.
QWO_API int qwo_pool_plan_slices(qwo_pool * p, int layer, const int32_t * sel, int T, int n_used, int max_slice,
                                 int32_t * slices, int32_t * union_out) {
    const int E = p->n_expert;
    if (max_slice == 0) max_slice = 1024;
    std::vector<uint8_t> seen((size_t)E, 0);
    int uni = 0;
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < n_used; ++j) {
            const int e = sel[(size_t)t * n_used + j];
            if (!seen[(size_t)e]) { seen[(size_t)e] = 1; ++uni; }
        }
    p->quota_on = uni <= qwo_pool_quota_of(p, layer) - 8;
    const int cap = std::max(n_used, qwo_pool_capacity(p, layer) - 8);
    std::fill(seen.begin(), seen.end(), 0);
    int ns = 0, distinct = 0, t0 = 0;
    for (int t = 0; t < T; ++t) {
        int nnew = 0;
        for (int j = 0; j < n_used; ++j) {
            const int e = sel[(size_t)t * n_used + j];
            if (!seen[(size_t)e]) { seen[(size_t)e] = 1; ++nnew; }
        }
        if ((distinct + nnew > cap || t - t0 >= max_slice) && t > t0) {
            slices[2 * ns] = t0; slices[2 * ns + 1] = t - t0; ++ns;
            std::fill(seen.begin(), seen.end(), 0);
            distinct = 0; nnew = 0;
            for (int j = 0; j < n_used; ++j) {
                const int e = sel[(size_t)t * n_used + j];
                if (!seen[(size_t)e]) { seen[(size_t)e] = 1; ++nnew; }
            }
            t0 = t;
        }
        distinct += nnew;
    }
    slices[2 * ns] = t0; slices[2 * ns + 1] = T - t0; ++ns;
    if (union_out) *union_out = uni;
    return ns;
}

// Per-slot key and clock of pool `pool` (for qwo_pool_new, the role).
QWO_API void qwo_pool_slots(const qwo_pool * p, int pool, int32_t * slot2key, uint64_t * clk) {
    const auto & R = p->pools[(size_t)pool];
    for (int s = 0; s < R.n_slots; ++s) { slot2key[s] = R.slot2key[(size_t)s]; clk[s] = R.clk[(size_t)s]; }
}
