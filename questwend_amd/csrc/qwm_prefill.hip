// qwm_prefill.hip -- GGML_OP_MUL_MAT_ID for prefill-sized batches (T > 8
// columns) over Q4_K expert slabs: the (column, expert) pairs are grouped by
// expert and each group runs as a GEMM on the matrix cores.
//
// Numerics follow ggml's CPU path for Q4_K: b is quantized to Q8_K exactly as
// quantize_row_q8_K (ggml-quants.c:2769-2806), every 32-element sub-block dot
// is an exact int32 (v_mfma_i32_16x16x32_i8 on the unpacked nibbles), the
// 6-bit sub-block scales and mins are applied in integers, and only the
// per-256 block scaling is floating point (fp32, in block order).
//
// Tile: a workgroup owns 64 weight rows x 16 columns of one expert; each of
// its 4 waves owns 16 rows.  With the columns as the MFMA's A side and the
// weight rows as its B side, lane l holds row l % 16 for both its loads and
// its outputs (columns 4 (l / 16) .. +3), so a lane's scales are those of one
// row.  The 16 columns' Q8_K data sit in LDS for the whole K.
#include <hip/hip_runtime.h>

#include "qwm_internal.h"
#include "qwm_q4k.h"
#include "qwm_q80.h"

namespace qwm {

constexpr int PF_TOK = 16;     // columns per tile
constexpr int PF_ROWS = 64;    // weight rows per tile
constexpr int PF_MAXK = 4096;  // longest K held in LDS (3072 and 4096 above 2048)
constexpr int PF_MAX_AS = 4096;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // 16-byte pieces (plain vector loads and stores)

struct PfArgs {
    const float * b; size_t b_nb1, b_nb2;     // bytes
    const int32_t * ids; size_t ids_nb1;      // bytes
    const uint8_t * as; size_t slab, row_bytes;
    const uint8_t * as2;                      // GU: the up matrix (same type, shape and slabs as `as`)
    int K, N, ne11, T, n_ids, n_as;
    int q8;                                   // weights Q8_0 (b quantized to Q8_0), else Q4_K (b to Q8_K)
    int8_t * qs; float * d; int32_t * bs;     // quantized rows of b [T * ne11]: values, scales (K/32 per
                                              // row), Q8_K sums of 16 (Q4_K only)
    int4 * items;                             // per column tile: expert, first column, columns, 0
    int32_t * perm; int32_t * total; int32_t * err;
    float * dst; size_t dst_nb1, dst_nb2;
};

constexpr int PF_PREP_THREADS = 1024;

// The expert of pair p (column t = p / n_ids, id slot p % n_ids), or -1 past
// the last pair; an id outside [0, n_as) sets `bad` and reads expert 0.
__device__ inline int pf_pair_expert(const PfArgs & a, int p, int P, bool & bad) {
    if (p >= P) return -1;
    const int t = p / a.n_ids, e = p % a.n_ids;
    const int v = *reinterpret_cast<const int32_t *>(reinterpret_cast<const uint8_t *>(a.ids) + t * a.ids_nb1 + e * 4);
    if (v < 0 || v >= a.n_as) { bad = true; return 0; }
    return v;
}

// The grouping, in one workgroup: the expert histogram of this call's pairs
// (in LDS), its exclusive scan, the column-tile table (the tiles of expert e
// are consecutive: first column, columns) and the pairs placed in their
// expert's group through per-expert cursors in LDS.  Inside a group the order
// is whatever the LDS atomics give: a column's result does not depend on its
// position.  The first KB * UN * G pairs' experts are read once and kept in
// registers for both passes (all of a 512-token chunk's top-10); further pairs
// are read in batches of UN * G, each requested before it touches LDS, so the
// loads overlap.  Nothing carries over between calls, so calls of any shape
// may share a workspace.
__device__ void pf_group(const PfArgs & a) {
    constexpr int G = PF_PREP_THREADS, NW = G / 64, PER = PF_MAX_AS / G, UN = 4, KB = 2;
    __shared__ int32_t s_c[PF_MAX_AS];
    __shared__ int32_t s_wsum[2][NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int P = a.T * a.n_ids;
    bool bad = false;
    int keep[KB][UN];                              // pair (kb UN + j) G + tid
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < UN; ++j) keep[kb][j] = pf_pair_expert(a, (kb * UN + j) * G + tid, P, bad);
    for (int e = tid; e < a.n_as; e += G) s_c[e] = 0;
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < UN; ++j)
            if (keep[kb][j] >= 0) atomicAdd(&s_c[keep[kb][j]], 1);
    for (int p0 = KB * UN * G; p0 < P; p0 += G * UN) {
        int v[UN];
#pragma unroll
        for (int j = 0; j < UN; ++j) v[j] = pf_pair_expert(a, p0 + j * G + tid, P, bad);
#pragma unroll
        for (int j = 0; j < UN; ++j)
            if (v[j] >= 0) atomicAdd(&s_c[v[j]], 1);
    }
    if (bad) st_agent(a.err, 1);
    __syncthreads();
    int c[PER], cs = 0, is = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int e = PER * tid + q;
        c[q] = e < a.n_as ? s_c[e] : 0;
        cs += c[q];
        is += (c[q] + PF_TOK - 1) / PF_TOK;
    }
    int cx = cs, ix = is;    // inclusive scans over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int cy = __shfl_up(cx, o, 64), iy = __shfl_up(ix, o, 64);
        if (lane >= o) { cx += cy; ix += iy; }
    }
    if (lane == 63) { s_wsum[0][wave] = cx; s_wsum[1][wave] = ix; }
    __syncthreads();
    int cb = cx - cs, ib = ix - is;
    for (int w = 0; w < wave; ++w) { cb += s_wsum[0][w]; ib += s_wsum[1][w]; }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int e = PER * tid + q;
        if (e < a.n_as) {
            for (int ct = 0; ct * PF_TOK < c[q]; ++ct)
                a.items[ib + ct] = make_int4(e, cb + ct * PF_TOK, min(PF_TOK, c[q] - ct * PF_TOK), 0);
            s_c[e] = cb;     // this thread's own entries: the cursor starts at the group's first column
        }
        cb += c[q];
        ib += (c[q] + PF_TOK - 1) / PF_TOK;
    }
    if (tid == G - 1) *a.total = ib;
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < UN; ++j)
            if (keep[kb][j] >= 0) a.perm[atomicAdd(&s_c[keep[kb][j]], 1)] = (kb * UN + j) * G + tid;
    for (int p0 = KB * UN * G; p0 < P; p0 += G * UN) {
        int v[UN];
#pragma unroll
        for (int j = 0; j < UN; ++j) v[j] = pf_pair_expert(a, p0 + j * G + tid, P, bad);
#pragma unroll
        for (int j = 0; j < UN; ++j)
            if (v[j] >= 0) a.perm[atomicAdd(&s_c[v[j]], 1)] = p0 + j * G + tid;
    }
}

// One launch before the GEMM: workgroup 0 groups the pairs by expert while the
// others quantize b's columns (one 256-block per wave): Q8_K for Q4_K weights
// (quantize_row_q8_K), ggml's x86 Q8_0 quantizer for Q8_0 weights.
__global__ void __launch_bounds__(PF_PREP_THREADS) k_pf_prep(PfArgs a) {
    if (blockIdx.x == 0) {
        pf_group(a);
        return;
    }
    constexpr int NW = PF_PREP_THREADS / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rows = a.T * a.ne11, nb = a.K / QK_K;
    for (int jb = (blockIdx.x - 1) * NW + wave; jb < rows * nb; jb += (gridDim.x - 1) * NW) {
        const int row = jb / nb, b = jb % nb;
        const int t = row / a.ne11, i = row % a.ne11;
        const float * src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(a.b) + t * a.b_nb2 + i * a.b_nb1);
        if (a.q8)
            quantize_q80_256(src + b * QK_K, a.qs + (size_t)row * a.K + b * QK_K, a.d + (size_t)row * (a.K / 32) + b * 8,
                             lane);
        else
            quantize_block_q8K(src + b * QK_K, a.qs + (size_t)row * a.K + b * QK_K, a.d + (size_t)row * (a.K / 32) + b,
                               a.bs + (size_t)row * (a.K / 16) + b * 16, lane);
    }
}

// The grouped GEMM.  Units are (16-column tile of one expert, row tile of 64
// weight rows); a workgroup owns 64 rows x 16 columns at a time, 16 rows per
// wave, and runs a contiguous range of units (see the loop head).
// GU: the same tile of the up matrix (a.as2) streams beside the gate rows
// (a.as), and each output is ggml_swiglu_split's silu(gate) * up (the
// vectorized silu on the rows' 16-wide chunks, libm expf on the tail, as
// k_swiglu_rows): the dots are those of two separate calls bit for bit.
// Q8: Q8_0 weights (34-byte blocks of 32: fp16 d and int8 values), each block's
// exact int32 dot on one MFMA and d_w d_x sumi in fp32; the activations are
// Q8_0 (ggml's vec_dot_type for Q8_0).
// Three workgroups per CU for Q4_K (LDS 47 KB each at K 2048; 168 VGPRs), two
// where that budget spills (gate/up with 1, 6 or 7 blocks per row) and for Q8_0
// (64 KB of LDS at K 2048); two at K 3072 (66-73 KB) and one at K 4096
// (84-91 KB: the 16 activation rows alone take 66 KB).
template <int NB, bool GU, bool Q8>
constexpr int pf_occupancy() {
    return NB > 12 ? 1 : NB > 8 ? 2 : (Q8 || (GU && (NB == 1 || NB >= 6 && NB != 8))) ? 2 : 3;
}

template <int NB, bool GU, bool Q8>
__global__ void __launch_bounds__(256, (pf_occupancy<NB, GU, Q8>())) k_pf_gemm(PfArgs a) {
    constexpr int K = NB * QK_K;
    // a step is the wave's 16 rows x 256 weights: PPR 16-byte pieces per row (one
    // 144-byte Q4_K block, or eight 34-byte Q8_0 blocks), SP pieces, NL loads per lane
    constexpr int PPR = Q8 ? 17 : 9, SROW = 16 * PPR, SP = 16 * PPR, NL = (SP + 63) / 64;
    // rows padded by 8 bytes: the operand reads (16 columns x 4 k-slices x 8 B)
    // are then free of bank conflicts (measured on gfx950: none with 8, some with
    // 16 or 32, many with no padding); the rows are 8-byte aligned
    constexpr int QP = K + 8;
    constexpr int NS = GU ? 2 : 1;                      // weight streams
    __shared__ __align__(16) int8_t s_q[PF_TOK][QP];   // the columns' quantized values
    __shared__ __align__(16) float s_d[Q8 ? NB * 8 : NB][PF_TOK];   // their scales (per 32 or per 256)
    // the sums of the 32 Q8_K values of each sub-block, [sub-block][column]: integers below 2^12 in
    // magnitude, held as floats for the mins' f32 MFMA (A[column][sub-block] at lane column + 16 k)
    __shared__ __align__(16) float s_bsf[Q8 ? 1 : NB * 8][PF_TOK];
    __shared__ __align__(16) uint8_t s_w[4][16 * SROW];  // each wave's staging of one step's weights
    __shared__ int32_t s_pair[PF_TOK];                  // each column's Q8_K row of b, -1: none
    __shared__ int64_t s_out[PF_TOK];                   // byte offset of each column's output row in dst, -1: none
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Persistent: the grid is the resident workgroup count W, and workgroup w takes
    // the units u in [w U / W, (w + 1) U / W) of the U = column tiles x row tiles
    // (column-tile-major), so every workgroup streams within one unit of the same
    // weight bytes.  A run of units inside one column tile is a segment: its
    // columns are staged once and its row tiles stream in turn.
    const int RT = a.N / PF_ROWS;
    const int U = *a.total * RT;
    const int u_end = (int)((int64_t)(blockIdx.x + 1) * U / gridDim.x);
    for (int u = (int)((int64_t)blockIdx.x * U / gridDim.x); u < u_end;) {
        const int4 desc = a.items[u / RT];
        const int e = desc.x, c0 = desc.y, nc = desc.z;
        const int rt0 = u % RT, rt1 = min(RT, rt0 + (u_end - u));
        u += rt1 - rt0;
        __syncthreads();                                     // the previous segment's column tables are read
        const int rl = lane & 15, kq = lane >> 4;           // B side: row rl, k-slice kq; outputs: columns 4 kq .. +3
        int row = rt0 * PF_ROWS + wave * 16 + rl;           // the lane's output row
        // A step's weights (the wave's 16 rows x SROW bytes) are loaded as whole
        // 16-byte pieces: piece p = lane + 64 i (i < NL, p < SP) is piece p % PPR of
        // row p / PPR's step, so one load covers several rows' steps in full (the
        // 8-byte slices each lane needs for the MFMA would touch 16 lines for 32 bytes
        // per load, which holds the stream near half the HBM rate).  Piece p goes to
        // byte 16 p of the wave's LDS buffer, which then holds the 16 rows' steps in
        // block layout.  The first PF steps are requested before the columns are staged.
        // wave-uniform bases (scalar registers) and 32-bit lane offsets: a segment stays
        // inside one expert's slab, below 2 GiB (checked at launch)
        const int wave_u = __builtin_amdgcn_readfirstlane(wave);
        const uint8_t * wbase[NS];
        wbase[0] = a.as + (size_t)e * a.slab + (size_t)(rt0 * PF_ROWS + wave_u * 16) * a.row_bytes;
        if constexpr (GU) wbase[1] = a.as2 + (size_t)e * a.slab + (size_t)(rt0 * PF_ROWS + wave_u * 16) * a.row_bytes;
        uint32_t poff[NL];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int pc = min(lane + 64 * i, SP - 1);        // lanes past the last piece: an in-bounds address, never loaded
            poff[i] = (uint32_t)(pc / PPR) * (uint32_t)a.row_bytes + (uint32_t)(pc % PPR) * 16u;
        }
        // ring depth: steps in flight per stream, a divisor of NB (every group of PF steps is
        // then whole); 3 waves per SIMD leave room for one step of each stream beside the other
        // (deeper rings spill at that budget)
        constexpr int PF = (GU || NB <= 2) ? 1 : (NB % 2 == 0 ? 2 : 1);
        u32x4 wr[NL][NS][PF];                               // the ring: a step's pieces per lane
        // step st: the st % NB-th 256 weights of row tile rt0 + st / NB
        auto load_s = [&](int q, int p, int st) {
            const uint32_t o = (uint32_t)(st / NB) * (uint32_t)(PF_ROWS * a.row_bytes) + (uint32_t)(st % NB) * (uint32_t)SROW;
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                if (SP % 64 != 0 && i == NL - 1) {
                    // the last load's lanes past the step's pieces stay idle (their values are never staged)
                    u32x4 t = __builtin_nondeterministic_value(wr[i][q][p]);
                    if (lane < SP - 64 * (NL - 1)) t = *reinterpret_cast<const u32x4 *>(wbase[q] + (poff[i] + o));
                    wr[i][q][p] = t;
                } else {
                    wr[i][q][p] = *reinterpret_cast<const u32x4 *>(wbase[q] + (poff[i] + o));
                }
            }
        };
#pragma unroll
        for (int p = 0; p < PF; ++p)
#pragma unroll
            for (int q = 0; q < NS; ++q) load_s(q, p, p);     // PF <= NB: inside the first row tile
        // the tile's columns: Q8_K rows of b into LDS (zeros past nc)
        // (pair p = t n_ids + slot: column t of b, row slot % ne11 of it; output row (slot, t))
        if (tid < PF_TOK) {
            const int p = tid < nc ? a.perm[c0 + tid] : -1;
            const int t = p / a.n_ids, sl = p % a.n_ids;
            s_pair[tid] = p >= 0 ? t * a.ne11 + sl % a.ne11 : -1;      // the Q8_K row of b
            s_out[tid] = p >= 0 ? (int64_t)t * (int64_t)a.dst_nb2 + (int64_t)sl * (int64_t)a.dst_nb1 : (int64_t)-1;
        }
        __syncthreads();
#pragma unroll
        for (int v = tid; v < PF_TOK * (K / 16); v += 256) {
            const int c = v / (K / 16), o = v % (K / 16);
            const int src = s_pair[c];
            uint4 w = make_uint4(0, 0, 0, 0);
            if (src >= 0) w = reinterpret_cast<const uint4 *>(a.qs + (size_t)src * K)[o];
            uint2 * dq = reinterpret_cast<uint2 *>(&s_q[c][16 * o]);
            dq[0] = make_uint2(w.x, w.y);
            dq[1] = make_uint2(w.z, w.w);
        }
#pragma unroll
        for (int v = tid; v < PF_TOK * NB * 8; v += 256) {
            const int c = v / (NB * 8), j = v % (NB * 8);
            const int src = s_pair[c];
            if constexpr (Q8) {
                s_d[j][c] = src >= 0 ? a.d[(size_t)src * (K / 32) + j] : 0.f;
            } else {
                int sm = 0;
                float dd = 0.f;
                if (src >= 0) {
                    const int2 bs = reinterpret_cast<const int2 *>(a.bs + (size_t)src * (K / 16))[j];
                    sm = bs.x + bs.y;
                    if ((j & 7) == 0) dd = a.d[(size_t)src * (K / 32) + j / 8];
                }
                s_bsf[j][c] = (float)sm;
                if ((j & 7) == 0) s_d[j / 8][c] = dd;
            }
        }
        __syncthreads();

        // the ring over the (row tile, block) sequence: groups of PF steps, slots
        // static inside a group; the bound is a runtime count, so the groups stay
        // a loop and only one group's values are live at a time.  Step s is block
        // s % NB of row tile rt0 + s / NB.
        const int nsteps = (rt1 - rt0) * NB;
        uint8_t * wbuf = s_w[wave];
        // one block of one weight row against the tile's 16 columns.  The sub-block
        // dots are exact int32 (one int8 MFMA each, issued back to back into their
        // own accumulators) and the 6-bit scales multiply them in 24-bit integer
        // multiply-adds (|dot| <= 32 * 15 * 128 < 2^17, the block's sum below 2^23):
        // each step of that sum goes through an empty asm, so the compiler keeps it
        // a chain of v_mad_i32_i24 instead of regrouping it into multiplies and
        // three-way adds.  The scales are unpacked four to a register (scales 4..7:
        // the low nibbles of bytes 8..11 and bits 6..7 of bytes 0..3).  The mins term
        // sum_j min_j * bsum_j (|product| < 2^18, every partial sum < 2^24) runs as
        // two f32 MFMAs (16x16x4): each value and partial sum is an integer that
        // fp32 holds exactly, so the result is the integer sum in any order.
        auto block_dot = [&](int b, const uint4 hd, const uint2 (&qq)[4], float (&facc)[4], float (&facc_m)[4]) {
            // mins: B[k][row] = the row's min of sub-block k (k = kq, then kq + 4), A[column][k] = bsum
            const int sh = 8 * kq;
            const uint32_t a1 = hd.z >> sh, q8 = (hd.w >> sh) & 0xff;
            const float mn_lo = (float)(int)(a1 & 63);
            const float mn_hi = (float)(int)((q8 >> 4) | ((a1 >> 6 & 3) << 4));
            v4f mins = {0.f, 0.f, 0.f, 0.f};
            mins = __builtin_amdgcn_mfma_f32_16x16x4f32(s_bsf[b * 8 + kq][rl], mn_lo, mins, 0, 0, 0);
            mins = __builtin_amdgcn_mfma_f32_16x16x4f32(s_bsf[b * 8 + 4 + kq][rl], mn_hi, mins, 0, 0, 0);
            const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);   // scales 4..7, one a byte
            int acc[4] = {0, 0, 0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {                 // two groups of 4 sub-blocks
                v4i dj[4];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * h + jj;
                    const uint2 raw = qq[j >> 1];
                    const uint32_t m4 = 0x0F0F0F0Fu;
                    const uint32_t w0 = (j & 1) ? (raw.x >> 4) & m4 : raw.x & m4;
                    const uint32_t w1 = (j & 1) ? (raw.y >> 4) & m4 : raw.y & m4;
                    const long bw = (long)(((uint64_t)w1 << 32) | w0);
                    // A side: column rl's 8 activations of sub-block j (elements 32 j ..), k-slice kq
                    const uint2 xv = *reinterpret_cast<const uint2 *>(&s_q[rl][b * QK_K + 32 * j + 8 * kq]);
                    const long ax = (long)(((uint64_t)xv.y << 32) | xv.x);
                    const v4i z = {0, 0, 0, 0};
                    dj[jj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
                }
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int scj = h == 0 ? (int)((hd.y >> (8 * jj)) & 63) : (int)((sc_hi >> (8 * jj)) & 0xff);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        acc[r] = __mul24(scj, dj[jj][r]) + acc[r];
                        if (4 * h + jj < 7) asm("" : "+v"(acc[r]));
                    }
                }
            }
            const float dw = fp16_to_f32((uint16_t)(hd.x & 0xffff)), dmw = fp16_to_f32((uint16_t)(hd.x >> 16));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dx = s_d[b][4 * kq + r];
                facc[r] = __builtin_fmaf(dx * dw, (float)acc[r], facc[r]);
                facc_m[r] = __builtin_fmaf(-dx * dmw, mins[r], facc_m[r]);
            }
        };
        // Q8_0: the step's 8 blocks of one weight row (w = its 272 staged bytes, dword
        // aligned).  Block j is d (fp16) at 34 j and 32 int8 values after it; lane kq's
        // 8 values start at 34 j + 2 + 8 kq, dword aligned for odd j and 2 bytes off for
        // even j (three dwords read and realigned).  sumi is exact (32 products of
        // |v| <= 128); the scaling is fma(d_w d_x, sumi, acc) per block, in block order.
        auto q80_step_dot = [&](int b, const uint8_t * w, float (&facc)[4]) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int o = 34 * j + 2 + 8 * kq;
                uint32_t w0, w1, dbits;
                if (j & 1) {
                    const uint32_t * v = reinterpret_cast<const uint32_t *>(w + o);
                    w0 = v[0];
                    w1 = v[1];
                    dbits = *reinterpret_cast<const uint32_t *>(w + 34 * j - 2) >> 16;
                } else {
                    const uint32_t * v = reinterpret_cast<const uint32_t *>(w + o - 2);
                    const uint32_t d0 = v[0], d1 = v[1], d2 = v[2];
                    w0 = __builtin_amdgcn_alignbit(d1, d0, 16);
                    w1 = __builtin_amdgcn_alignbit(d2, d1, 16);
                    dbits = *reinterpret_cast<const uint32_t *>(w + 34 * j) & 0xffff;
                }
                const long bw = (long)(((uint64_t)w1 << 32) | w0);
                const uint2 xv = *reinterpret_cast<const uint2 *>(&s_q[rl][b * QK_K + 32 * j + 8 * kq]);
                const long ax = (long)(((uint64_t)xv.y << 32) | xv.x);
                const v4i z = {0, 0, 0, 0};
                const v4i dj = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
                const float dw = fp16_to_f32((uint16_t)dbits);
                const float4 dx = *reinterpret_cast<const float4 *>(&s_d[b * 8 + j][4 * kq]);
                facc[0] = __builtin_fmaf(dw * dx.x, (float)dj[0], facc[0]);
                facc[1] = __builtin_fmaf(dw * dx.y, (float)dj[1], facc[1]);
                facc[2] = __builtin_fmaf(dw * dx.z, (float)dj[2], facc[2]);
                facc[3] = __builtin_fmaf(dw * dx.w, (float)dj[3], facc[3]);
            }
        };
        float facc[NS][4], facc_m[NS][4];
#pragma unroll
        for (int q = 0; q < NS; ++q)
#pragma unroll
            for (int r = 0; r < 4; ++r) { facc[q][r] = 0.f; facc_m[q][r] = 0.f; }
#pragma unroll 1
        for (int b0 = 0; b0 < nsteps; b0 += PF)
#pragma unroll
        for (int pslot = 0; pslot < PF; ++pslot) {
            const int st = b0 + pslot;
            if constexpr (NB % PF != 0) {
                if (st >= nsteps) break;
            }
            const int b = st % NB;
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                // the slot's pieces into the wave's buffer, then the slot is refilled (always: the
                // tail re-reads the last block) and the lane reads its row's block in MFMA layout.
                // A wave's LDS operations run in order, so the buffer needs no barrier between
                // steps or between the gate and up streams.
                u32x4 * wb4 = reinterpret_cast<u32x4 *>(wbuf);
#pragma unroll
                for (int i = 0; i < NL; ++i)
                    if (64 * (i + 1) <= SP || lane < SP - 64 * i) wb4[lane + 64 * i] = wr[i][q][pslot];
                load_s(q, pslot, min(st + PF, nsteps - 1));
                __builtin_amdgcn_wave_barrier();
                if constexpr (Q8) {
                    q80_step_dot(b, wbuf + rl * SROW, facc[q]);
                } else {
                    const uint4 hd = *reinterpret_cast<const uint4 *>(wbuf + rl * SROW);
                    uint2 qq[4];
#pragma unroll
                    for (int jp = 0; jp < 4; ++jp)
                        qq[jp] = *reinterpret_cast<const uint2 *>(wbuf + rl * SROW + 16 + 32 * jp + 8 * kq);
                    __builtin_amdgcn_wave_barrier();
                    block_dot(b, hd, qq, facc[q], facc_m[q]);
                }
            }
            if (b == NB - 1) {                          // the row tile is done: its outputs, then the next tile
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t off = s_out[4 * kq + r];
                    if (off >= 0) {
                        float * o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.dst) + off);
                        const float gv = facc[0][r] + facc_m[0][r];
                        if constexpr (GU) {
                            const float uv = facc[NS - 1][r] + facc_m[NS - 1][r];
                            o[row] = (row < a.N - (a.N & 15)) ? v_silu(gv) * uv : gv / (1.0f + libm_expf(-gv)) * uv;
                        } else {
                            o[row] = gv;
                        }
                    }
#pragma unroll
                    for (int q = 0; q < NS; ++q) { facc[q][r] = 0.f; facc_m[q][r] = 0.f; }
                }
                row += PF_ROWS;
            }
        }
    }
}

size_t prefill_workspace(int64_t K, int64_t N, int64_t n_as, int64_t T, int64_t ne11, int64_t n_ids) {
    const int64_t rows = T * ne11, P = T * n_ids;
    const int64_t max_tiles = P / PF_TOK + n_as;                     // column tiles
    size_t o = 0;
    auto take = [&](size_t bytes) { o = align_up(o + bytes, 256); };
    take((size_t)rows * K);
    take(sizeof(float) * rows * (K / 32));                           // scales: per 32 (Q8_0) or per 256 (Q8_K)
    take(sizeof(int32_t) * rows * (K / 16));
    take(sizeof(int4) * max_tiles);
    take(sizeof(int32_t) * P);                                        // perm
    take(256);                                                        // total, err
    return o;
}

// bytes per 256 weights of a row: a Q4_K block, or eight Q8_0 blocks
static int64_t pf_bytes_per_256(int32_t wtype) { return wtype == T_Q8_0 ? 272 : 144; }

bool prefill_supported(int32_t wtype, int64_t K, int64_t N, int64_t n_as, const void * as, std::string & why) {
    if (wtype != T_Q4_K && wtype != T_Q8_0) { why = "prefill mul_mat_id: Q4_K or Q8_0 weights only"; return false; }
    if (K % QK_K || (K > 2048 && K != 3072 && K != 4096)) {
        why = "prefill mul_mat_id: K must be a multiple of 256 up to 2048, or 3072 or 4096";
        return false;
    }
    if (N % PF_ROWS) { why = "prefill mul_mat_id: N must be a multiple of 64"; return false; }
    if (n_as > PF_MAX_AS) { why = "prefill mul_mat_id: more than 4096 experts"; return false; }
    if ((uint64_t)N * (uint64_t)(K / QK_K) * (uint64_t)pf_bytes_per_256(wtype) >= (1ull << 31)) {
        why = "prefill mul_mat_id: expert slab of 2 GiB or more";
        return false;
    }
    if ((uintptr_t)as % 16) { why = "prefill mul_mat_id: weights must be 16-byte aligned"; return false; }
    return true;
}

// The persistent GEMM's grid: the workgroups one launch keeps resident (the
// occupancy query per kernel and device, done once).
template <int NB, bool GU, bool Q8>
static int launch_gemm(const PfArgs & a, hipStream_t s) {
    static int grid[64] = {};
    int dev = 0;
    QWM_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(QWM_ERR_UNSUPPORTED, "prefill mul_mat_id: device index past 63");
    if (!grid[dev]) {
        int per_cu = 0, cus = 0;
        QWM_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_pf_gemm<NB, GU, Q8>, 256, 0));
        QWM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        grid[dev] = std::max(1, per_cu) * std::max(1, cus);
    }
    k_pf_gemm<NB, GU, Q8><<<dim3((unsigned)grid[dev]), 256, 0, s>>>(a);
    return QWM_OK;
}

int launch_prefill(const MmidArgs & m, uint8_t * ws, hipStream_t s, const uint8_t * up) {
    std::string why;
    if (!prefill_supported(m.wtype, m.K, m.N, m.n_as, m.as, why) || (up && !prefill_supported(m.wtype, m.K, m.N, m.n_as, up, why)))
        return fail(QWM_ERR_UNSUPPORTED, why);
    const int64_t rows = m.T * m.ne11, P = m.T * m.n_ids;
    const int64_t max_tiles = P / PF_TOK + m.n_as;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    PfArgs a;
    a.b = m.b; a.b_nb1 = m.b_nb1; a.b_nb2 = m.b_nb2; a.ids = m.ids; a.ids_nb1 = m.ids_nb1;
    a.as = m.as; a.slab = m.slab; a.row_bytes = (size_t)((m.K / QK_K) * pf_bytes_per_256(m.wtype));
    a.as2 = up;
    a.q8 = m.wtype == T_Q8_0;
    a.K = (int)m.K; a.N = (int)m.N; a.ne11 = (int)m.ne11; a.T = (int)m.T; a.n_ids = (int)m.n_ids; a.n_as = (int)m.n_as;
    a.qs = reinterpret_cast<int8_t *>(ws + take((size_t)rows * m.K));
    a.d = reinterpret_cast<float *>(ws + take(sizeof(float) * rows * (m.K / 32)));
    a.bs = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * rows * (m.K / 16)));
    a.items = reinterpret_cast<int4 *>(ws + take(sizeof(int4) * max_tiles));
    a.perm = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * P));
    a.total = reinterpret_cast<int32_t *>(ws + take(256));
    a.err = a.total + 1;
    a.dst = m.dst; a.dst_nb1 = m.dst_nb1; a.dst_nb2 = m.dst_nb2;
    const int64_t nblk = rows * (m.K / QK_K);
    const int64_t nw = PF_PREP_THREADS / 64;
    const unsigned prep_grid = 1 + (unsigned)std::max<int64_t>(1, std::min<int64_t>(512, (nblk + nw - 1) / nw));
    QWM_TIMED("prefill_prep", s, k_pf_prep<<<prep_grid, PF_PREP_THREADS, 0, s>>>(a));
    const char * label = up ? "prefill_gemm_gu" : "prefill_gemm";
    prof_begin(label, s);
    int rc = QWM_OK;
    const bool q8 = a.q8 != 0;
#define QWM_PF_CASE(NBV)                                                                                            \
    case NBV:                                                                                                       \
        rc = q8 ? (up ? launch_gemm<NBV, true, true>(a, s) : launch_gemm<NBV, false, true>(a, s))                   \
                : (up ? launch_gemm<NBV, true, false>(a, s) : launch_gemm<NBV, false, false>(a, s));                \
        break;
    switch (m.K / QK_K) {
        QWM_PF_CASE(1) QWM_PF_CASE(2) QWM_PF_CASE(3) QWM_PF_CASE(4) QWM_PF_CASE(5) QWM_PF_CASE(6) QWM_PF_CASE(7)
        QWM_PF_CASE(8) QWM_PF_CASE(12)
        default: QWM_PF_CASE(16)
    }
#undef QWM_PF_CASE
    if (rc != QWM_OK) return rc;
    prof_end(label, s);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
