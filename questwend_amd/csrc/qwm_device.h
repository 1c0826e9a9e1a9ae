// qwm_device.h -- device-side building blocks for the gfx950 MoE expert path:
// ggml block layouts, the CPU backend's exact scalar conventions (fp16
// rounding, the magic-number nearest_int, the AVX-512 expf polynomial) and
// wave64 reductions.  Every kernel source includes this header; all of them
// are compiled with -ffp-contract=off, so a fused multiply-add appears only
// where it is written (__builtin_fmaf), exactly where ggml-CPU fuses.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "qwm_expf.h"

#define QWM_DEV __device__ __forceinline__

namespace qwm {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int WAVE = 64;

// ggml-common.h:325-338 (144 B) and 251-256 (34 B).
struct block_q4_K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; };
struct block_q8_0 { uint16_t d; int8_t qs[QK8_0]; };
static_assert(sizeof(block_q4_K) == 144, "block_q4_K");
static_assert(sizeof(block_q8_0) == 34, "block_q8_0");

// ---------------------------------------------------------------- scalars --

QWM_DEV float fp16_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
QWM_DEV uint16_t f32_to_fp16(float f) { return __half_as_ushort(__float2half_rn(f)); }

// nearest_int(a*b) of ggml-quants.c:621-626 as gcc -O3 emits it on x86-64
// with FMA: the product and the 1.5*2^23 magic add fuse into one fma.
QWM_DEV int nearest_int_mul(float a, float b) {
    const float v = __builtin_fmaf(a, b, 12582912.f);
    return (int)(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

// ggml_v_expf (ggml-cpu/vec.h:1191-1216, AVX-512 lane): 2^n * poly(b).
QWM_DEV float v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = __builtin_fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, __builtin_fmaf(-n, 0x1.62e4p-1f, x));
    const float u = b * b;
    const float j = __builtin_fmaf(
        __builtin_fmaf(__builtin_fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                       __builtin_fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
        u, __builtin_fmaf(0x1.ffffecp-1f, b, 1.0f));
    if (__builtin_fabsf(n) > 192.0f) return n <= 0.0f ? 0.0f : __builtin_inff();
    return __builtin_ldexpf(j, (int)n);
}

// ggml_v_silu (ggml-cpu/vec.h:1219-1226)
QWM_DEV float v_silu(float x) { return x / (1.0f + v_expf(0.0f - x)); }

// Q4_K 6-bit scale/min of sub-block j (ggml-quants.c:871-878).
QWM_DEV void q4k_scale_min(int j, const uint8_t * q, int & d, int & m) {
    if (j < 4) { d = q[j] & 63; m = q[j + 4] & 63; }
    else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}
// Same, from the three scale dwords held in registers (bytes 4..15 of the
// block header): s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
// Branch-free: lanes of one wave take different j.
QWM_DEV void q4k_scale_min_reg(int j, uint32_t s0, uint32_t s1, uint32_t s2, int & d, int & m) {
    const int b = (j & 3) * 8;
    const uint32_t a0 = s0 >> b, a1 = s1 >> b, q8 = (s2 >> b) & 0xff;   // scales[j], [j+4], [j+8]
    const int dl = (int)(a0 & 63), ml = (int)(a1 & 63);
    const int dh = (int)((q8 & 0xF) | ((a0 >> 6 & 3) << 4));           // j >= 4: scales[j+4] & 15 | scales[j-4] >> 6
    const int mh = (int)((q8 >> 4) | ((a1 >> 6 & 3) << 4));
    d = j < 4 ? dl : dh;
    m = j < 4 ? ml : mh;
}

QWM_DEV int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// --------------------------------------------------------- wave reductions --

template <int WIDTH>
QWM_DEV float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
template <int WIDTH>
QWM_DEV int group_sum_i(int v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
template <int WIDTH>
QWM_DEV float group_max(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// DPP lane moves (no LDS round trip).  Controls: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
QWM_DEV float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Every lane of each 16-lane row receives the sum over that row.
QWM_DEV float row16_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return v;
}
// Value of lane ^ 16 / lane ^ 32 without LDS: the gfx950 permlane swaps
// exchange rows 0<->1, 2<->3 (16-lane rows) or the two wave halves.
QWM_DEV uint32_t lane_xor16(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
}
QWM_DEV uint32_t lane_xor32(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
}
QWM_DEV float lane_xor16_f(float v) { return __uint_as_float(lane_xor16(__float_as_uint(v))); }
QWM_DEV float lane_xor32_f(float v) { return __uint_as_float(lane_xor32(__float_as_uint(v))); }
template <int CTRL>
QWM_DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }

// Sum over aligned groups of W lanes (16, 32 or 64), available in every lane
// of the group.  Quad butterflies, then rotations by 4 and 8 inside the
// 16-lane row, then the permlane swaps.  The grouping of the additions differs
// between the four quads of a row, so lanes may differ in the last bit: use
// one lane's result.
template <int W>
QWM_DEV float lane_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
    if (W >= 32) v += lane_xor16_f(v);
    if (W >= 64) v += lane_xor32_f(v);
    return v;
}
template <int W>
QWM_DEV int lane_sum_i(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    v += dpp_i<0x124>(v);
    v += dpp_i<0x128>(v);
    if (W >= 32) v += (int)lane_xor16((uint32_t)v);
    if (W >= 64) v += (int)lane_xor32((uint32_t)v);
    return v;
}
// Wave maximum (exact: every lane gets the same value).
QWM_DEV float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    v = fmaxf(v, lane_xor16_f(v));
    return fmaxf(v, lane_xor32_f(v));
}
// _mm512_reduce_add_ps's halving tree (pairs i+8, i+4, i+2, i+1) within each
// 16-lane row, bit-identical in every lane: after the rotation by 8 the row
// has period 8, so the rotation by 4 pairs lane i with i^4 (mod 8), and so on.
QWM_DEV float tree16_dpp(float v) {
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x122>(v);
    v += dpp_f<0x121>(v);
    return v;
}

// Sum over aligned groups of W lanes (16, 32 or 64): the wave halves, then
// the 16-lane row pairs, then the row's halving tree.  Every lane of a group
// holds the same bits, and wave_sum_scatter8 forms the same sums.
template <int W>
QWM_DEV float halves_sum(float v) {
    if (W >= 64) v += lane_xor32_f(v);
    if (W >= 32) v += lane_xor16_f(v);
    return tree16_dpp(v);
}

// Pairwise sums that scatter two operands over the result: swap_add32 leaves
// a[l] + a[l + 32] in lanes 0-31 and b[l - 32] + b[l] in lanes 32-63;
// swap_add16 leaves the 16-lane rows [a0 + a1, b0 + b1, a2 + a3, b2 + b3].
QWM_DEV float swap_add32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
QWM_DEV float swap_add16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wave sums of the eight values a[0..3] and b[0..3] in six swaps instead of
// twenty-four: every lane of 16-lane row q receives sa = sum(a[scatter_row(q)])
// and sb = sum(b[scatter_row(q)]), bit-identical to halves_sum<64>.
QWM_DEV int scatter_row(int q) { return ((q & 1) << 1) | (q >> 1); }
QWM_DEV void wave_sum_scatter8(const float (&a)[4], const float (&b)[4], float & sa, float & sb) {
    const float a01 = swap_add32(a[0], a[1]), a23 = swap_add32(a[2], a[3]);
    const float b01 = swap_add32(b[0], b[1]), b23 = swap_add32(b[2], b[3]);
    sa = tree16_dpp(swap_add16(a01, a23));
    sb = tree16_dpp(swap_add16(b01, b23));
}

QWM_DEV float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// The 16-lane halving tree of _mm512_reduce_add_ps (gcc: lanes i+8, i+4, i+2,
// i+1).  An xor butterfly produces the same sums in every lane of the group.
QWM_DEV float tree16(float v) {
    v += __shfl_xor(v, 8, WAVE);
    v += __shfl_xor(v, 4, WAVE);
    v += __shfl_xor(v, 2, WAVE);
    v += __shfl_xor(v, 1, WAVE);
    return v;
}

// ------------------------------------------------ cross-workgroup hand-off --
// Some kernels let their last workgroup to finish (ticket == gridDim - 1)
// consume what the others wrote.  A __threadfence() there would write back
// and invalidate the issuing XCD's whole L2 once per workgroup, stalling every
// wave that streams through it, so the hand-off data is written and read with
// agent-scope atomic accesses instead (coherent across the XCDs' L2s with no
// cache maintenance) and each wave drains its own writes before the ticket.
template <typename T>
QWM_DEV void st_agent(T * p, T v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <typename T>
QWM_DEV T ld_agent(const T * p) { return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Every thread of the n participating workgroups calls this after its
// st_agent writes; true in all threads of the last one to arrive, which also
// re-arms the counter for the next launch.
QWM_DEV bool last_workgroup(int32_t * counter, int n) {
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);               // this wave's writes have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const int ticket = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = ticket == n - 1;
        if (s_last) st_agent(counter, 0);
    }
    __syncthreads();
    return s_last;
}
QWM_DEV bool last_workgroup(int32_t * counter) {
    return last_workgroup(counter, (int)(gridDim.x * gridDim.y * gridDim.z));
}

// Dataflow hand-off between workgroups of one launch.  signal_count: after
// this workgroup's agent-scope writes have completed, count one completion.
// wait_count: until `target` completions are counted (thread 0 polls; the
// spin is bounded, a timeout sets *err and lets the workgroup go on).
QWM_DEV void signal_count(int32_t * c) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The polling wave sleeps 64 cycles between reads: without the sleep the
// first hand-off of an isolated fused step released 3-4 us earlier, but back
// to back the 512 pollers' reads slowed the step by 0.5 us and the decode
// loop by 2%.
QWM_DEV void wait_count(const int32_t * c, int32_t target, int32_t * err, uint32_t limit) {
    if (threadIdx.x == 0) {
        uint32_t spins = 0;
        while (ld_agent(c) < target) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > limit) { st_agent(err, 1); break; }
        }
    }
    __syncthreads();
}

// Orders LDS traffic between the lanes of one wave (no workgroup barrier).
QWM_DEV void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-wide best (v, i) under "larger v, then smaller i" (a total order, so
// the rotation all-reduce is exact); every lane receives the winner.
QWM_DEV void wave_best_first(float & v, int & i) {
#define QWM_BEST_STEP(MOVE_F, MOVE_I)                                     \
    {                                                                     \
        const float ov = MOVE_F;                                          \
        const int oi = MOVE_I;                                            \
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }            \
    }
    QWM_BEST_STEP(dpp_f<0xB1>(v), dpp_i<0xB1>(i))
    QWM_BEST_STEP(dpp_f<0x4E>(v), dpp_i<0x4E>(i))
    QWM_BEST_STEP(dpp_f<0x124>(v), dpp_i<0x124>(i))
    QWM_BEST_STEP(dpp_f<0x128>(v), dpp_i<0x128>(i))
    QWM_BEST_STEP(lane_xor16_f(v), (int)lane_xor16((uint32_t)i))
    QWM_BEST_STEP(lane_xor32_f(v), (int)lane_xor32((uint32_t)i))
#undef QWM_BEST_STEP
}

// Argmax over a wave where ties take the larger index (ggml-cpu/vec.h:1618-1626
// keeps the last maximum); NaN never wins.
QWM_DEV void wave_argmax_last(float & v, int & idx) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, WAVE);
        const int oi = __shfl_xor(idx, o, WAVE);
        if (ov > v || (ov == v && oi > idx)) { v = ov; idx = oi; }
    }
}

}  // namespace qwm
