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

namespace qwm {

constexpr int PF_TOK = 16;     // columns per tile
constexpr int PF_ROWS = 64;    // weight rows per tile
constexpr int PF_RT = 4;       // row tiles per work item (the columns stay in LDS across them)
constexpr int PF_MAXK = 2048;  // longest K held in LDS
constexpr int PF_MAX_AS = 4096;

typedef int v4i __attribute__((ext_vector_type(4)));

struct PfArgs {
    const float * b; size_t b_nb1, b_nb2;     // bytes
    const int32_t * ids; size_t ids_nb1;      // bytes
    const uint8_t * as; size_t slab, row_bytes;
    int K, N, ne11, T, n_ids, n_as;
    int8_t * qs; float * d; int32_t * bs;     // Q8_K rows of b: [T * ne11]
    int32_t * cnt_copy; int32_t * off; int32_t * fill; int32_t * item_off;
    int4 * items;                             // per work item: expert, first column, columns, first row tile
    int32_t * perm; int32_t * eid; int32_t * total; int32_t * err;
    float * dst; size_t dst_nb1, dst_nb2;
};

// Q8_K of b's columns (one 256-block per wave) and each pair's expert.
__global__ void __launch_bounds__(256) k_pf_prep(PfArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rows = a.T * a.ne11, nb = a.K / QK_K;
    for (int jb = blockIdx.x * 4 + wave; jb < rows * nb; jb += gridDim.x * 4) {
        const int row = jb / nb, b = jb % nb;
        const int t = row / a.ne11, i = row % a.ne11;
        const float * src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(a.b) + t * a.b_nb2 + i * a.b_nb1);
        quantize_block_q8K(src + b * QK_K, a.qs + (size_t)row * a.K + b * QK_K, a.d + (size_t)row * nb + b,
                           a.bs + (size_t)row * (a.K / 16) + b * 16, lane);
    }
    const int P = a.T * a.n_ids;
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < P; p += gridDim.x * blockDim.x) {
        const int t = p / a.n_ids, e = p % a.n_ids;
        int v = *reinterpret_cast<const int32_t *>(reinterpret_cast<const uint8_t *>(a.ids) + t * a.ids_nb1 + e * 4);
        if (v < 0 || v >= a.n_as) { st_agent(a.err, 1); v = 0; }
        a.eid[p] = v;
    }
}

// One workgroup: the expert histogram (in LDS, from this call's pairs), group
// offsets (its exclusive scan) and the tile table (tiles of expert e are items
// item_off[e] .. item_off[e + 1] - 1).  Nothing carries over between calls,
// so calls of any shape may share a workspace.
__global__ void __launch_bounds__(1024) k_pf_scan(PfArgs a) {
    __shared__ int32_t s_c[PF_MAX_AS], s_i[PF_MAX_AS];
    __shared__ int32_t s_wsum[2][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rt = (a.N / PF_ROWS + PF_RT - 1) / PF_RT;    // row chunks per column tile
    for (int e = tid; e < a.n_as; e += 1024) s_c[e] = 0;
    __syncthreads();
    const int P = a.T * a.n_ids;
    for (int p = tid; p < P; p += 1024) atomicAdd(&s_c[a.eid[p]], 1);
    __syncthreads();
    for (int e = tid; e < a.n_as; e += 1024) {
        const int c = s_c[e];
        s_i[e] = (c + PF_TOK - 1) / PF_TOK * rt;
        a.cnt_copy[e] = c;
        a.fill[e] = 0;
    }
    __syncthreads();
    // exclusive scans of s_c and s_i over n_as <= 4096 entries, 4 per thread
    int c4[4], i4[4], cs = 0, is = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = 4 * tid + q;
        c4[q] = e < a.n_as ? s_c[e] : 0;
        i4[q] = e < a.n_as ? s_i[e] : 0;
        cs += c4[q];
        is += i4[q];
    }
    int cx = cs, ix = is;    // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int cy = __shfl_up(cx, o, 64), iy = __shfl_up(ix, o, 64);
        if (lane >= o) { cx += cy; ix += iy; }
    }
    if (lane == 63) { s_wsum[0][wave] = cx; s_wsum[1][wave] = ix; }
    __syncthreads();
    int cb = 0, ib = 0;
    for (int w = 0; w < wave; ++w) { cb += s_wsum[0][w]; ib += s_wsum[1][w]; }
    cb += cx - cs;
    ib += ix - is;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = 4 * tid + q;
        if (e < a.n_as) {
            a.off[e] = cb;
            a.item_off[e] = ib;
            for (int it = 0; it < i4[q]; ++it) {
                const int ct = it / rt;
                a.items[ib + it] = make_int4(e, cb + ct * PF_TOK, min(PF_TOK, c4[q] - ct * PF_TOK), (it % rt) * PF_RT);
            }
        }
        cb += c4[q];
        ib += i4[q];
    }
    if (tid == 1023) { a.off[a.n_as] = cb; a.item_off[a.n_as] = ib; *a.total = ib; }
}

// Pairs into their expert's group (any order inside a group: each column's
// result does not depend on its position).
__global__ void __launch_bounds__(256) k_pf_scatter(PfArgs a) {
    const int P = a.T * a.n_ids;
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < P; p += gridDim.x * blockDim.x) {
        const int e = a.eid[p];
        const int pos = a.off[e] + __hip_atomic_fetch_add(a.fill + e, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.perm[pos] = p;
    }
}

// The grouped GEMM.  Item it = (expert, 16-column tile, up to PF_RT row tiles
// of 64): the columns are staged in LDS once, the row tiles run in turn.
template <int NB>
__global__ void __launch_bounds__(256) k_pf_gemm(PfArgs a) {
    constexpr int K = NB * QK_K;
    // rows padded by 16 bytes: an operand read (16 columns x 4 k-slices x 8 B)
    // then covers all 64 banks once per half wave instead of one bank group
    constexpr int QP = K + 16;
    __shared__ __align__(16) int8_t s_q[PF_TOK][QP];
    __shared__ float s_d[NB][PF_TOK];
    __shared__ __align__(16) int16_t s_q8s[PF_TOK][NB * 8 + 2];   // sums of the 32 Q8_K values of each sub-block
    __shared__ int32_t s_pair[PF_TOK];
    const int it = blockIdx.x;
    if (it >= *a.total) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int4 desc = a.items[it];
    const int e = desc.x, c0 = desc.y, nc = desc.z;
    const int rt0 = desc.w, rt1 = min(rt0 + PF_RT, a.N / PF_ROWS);
    const int rl = lane & 15, kq = lane >> 4;           // B side: row rl, k-slice kq; outputs: columns 4 kq .. +3
    int row = rt0 * PF_ROWS + wave * 16 + rl;
    const uint8_t * wrow = a.as + (size_t)e * a.slab + (size_t)row * a.row_bytes;
    // weights of block b: header (16 B) and the lane's 8 bytes of each 32-byte qs group;
    // the first PF blocks are requested before the columns (they do not depend on them)
    constexpr int PF = NB < 4 ? NB : 4;
    uint4 hd_r[PF];
    uint2 qq_r[PF][4];
    auto load_w = [&](int b, uint4 & hd, uint2 (&qq)[4]) {
        const uint8_t * blk = wrow + (size_t)b * 144;
        hd = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qq[jp] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * jp + 8 * kq);
    };
#pragma unroll
    for (int p = 0; p < PF; ++p) load_w(p, hd_r[p], qq_r[p]);      // PF <= NB: blocks of the first row tile
    // the tile's columns: Q8_K rows of b into LDS (zeros past nc)
    if (tid < PF_TOK) s_pair[tid] = tid < nc ? a.perm[c0 + tid] : -1;
    __syncthreads();
    for (int v = tid; v < PF_TOK * (K / 16); v += 256) {
        const int c = v / (K / 16), o = v % (K / 16);
        const int p = s_pair[c];
        uint4 w = make_uint4(0, 0, 0, 0);
        if (p >= 0) {
            const int row = (p / a.n_ids) * a.ne11 + (p % a.n_ids) % a.ne11;
            w = reinterpret_cast<const uint4 *>(a.qs + (size_t)row * K)[o];
        }
        reinterpret_cast<uint4 *>(&s_q[c][0])[o] = w;
    }
    for (int v = tid; v < PF_TOK * NB * 8; v += 256) {
        const int c = v / (NB * 8), j = v % (NB * 8);
        const int p = s_pair[c];
        int16_t s = 0;
        float dd = 0.f;
        if (p >= 0) {
            const int row = (p / a.n_ids) * a.ne11 + (p % a.n_ids) % a.ne11;
            const int32_t * bs = a.bs + (size_t)row * (K / 16);
            s = (int16_t)(bs[2 * j] + bs[2 * j + 1]);
            if ((j & 7) == 0) dd = a.d[(size_t)row * NB + j / 8];
        }
        s_q8s[c][j] = s;
        if ((j & 7) == 0) s_d[j / 8][c] = dd;
    }
    __syncthreads();

    // the ring over the (row tile, block) sequence: groups of PF steps, slots
    // static inside a group; the bound is a runtime count, so the groups stay
    // a loop and only one group's values are live at a time.  Step s is block
    // s % NB of row tile rt0 + s / NB.
    const int nbr = a.K / QK_K;
    const int nsteps = (rt1 - rt0) * nbr;
    auto load_s = [&](int st, uint4 & hd, uint2 (&qq)[4]) {
        const uint8_t * blk = wrow + (size_t)(st / nbr) * PF_ROWS * a.row_bytes + (size_t)(st % nbr) * 144;
        hd = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qq[jp] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * jp + 8 * kq);
    };
    float facc[4] = {0.f, 0.f, 0.f, 0.f}, facc_m[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int b0 = 0; b0 < nsteps; b0 += PF)
#pragma unroll
    for (int pslot = 0; pslot < PF; ++pslot) {
        const int st = b0 + pslot;
        if (st >= nsteps) break;
        const int b = st % nbr;
        const uint4 hd = hd_r[pslot];
        uint2 qq[4];
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qq[jp] = qq_r[pslot][jp];
        if (st + PF < nsteps) load_s(st + PF, hd_r[pslot], qq_r[pslot]);
        int sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) q4k_scale_min_reg(j, hd.y, hd.z, hd.w, sc[j], mn[j]);
        int acc[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint2 raw = qq[j >> 1];
            const uint32_t m4 = 0x0F0F0F0Fu;
            const uint32_t w0 = (j & 1) ? (raw.x >> 4) & m4 : raw.x & m4;
            const uint32_t w1 = (j & 1) ? (raw.y >> 4) & m4 : raw.y & m4;
            const long bw = (long)(((uint64_t)w1 << 32) | w0);
            // A side: column rl's 8 activations of sub-block j (elements 32 j ..), k-slice kq
            const int8_t * xs = &s_q[rl][b * QK_K + 32 * j + 8 * kq];
            const uint2 xv = *reinterpret_cast<const uint2 *>(xs);
            const long ax = (long)(((uint64_t)xv.y << 32) | xv.x);
            v4i dj = {0, 0, 0, 0};
            dj = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, dj, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += sc[j] * dj[r];
        }
        const float dw = fp16_to_f32((uint16_t)(hd.x & 0xffff)), dmw = fp16_to_f32((uint16_t)(hd.x >> 16));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int c = 4 * kq + r;
            int mins = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) mins += __mul24(mn[j], (int)s_q8s[c][b * 8 + j]);
            const float dx = s_d[b][c];
            facc[r] = __builtin_fmaf(dx * dw, (float)acc[r], facc[r]);
            facc_m[r] = __builtin_fmaf(-dx * dmw, (float)mins, facc_m[r]);
        }
        if (b == nbr - 1) {                          // the row tile is done: its outputs, then the next tile
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = 4 * kq + r;
                const int p = s_pair[c];
                if (p >= 0) {
                    float * o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.dst) + (p / a.n_ids) * a.dst_nb2 +
                                                          (p % a.n_ids) * a.dst_nb1);
                    o[row] = facc[r] + facc_m[r];
                }
                facc[r] = 0.f;
                facc_m[r] = 0.f;
            }
            row += PF_ROWS;
        }
    }
}

size_t prefill_workspace(int64_t K, int64_t N, int64_t n_as, int64_t T, int64_t ne11, int64_t n_ids) {
    const int64_t rows = T * ne11, P = T * n_ids;
    const int64_t max_items = (P / PF_TOK + n_as) * ((N / PF_ROWS + PF_RT - 1) / PF_RT);
    size_t o = 0;
    auto take = [&](size_t bytes) { o = align_up(o + bytes, 256); };
    take((size_t)rows * K);
    take(sizeof(float) * rows * (K / QK_K));
    take(sizeof(int32_t) * rows * (K / 16));
    for (int i = 0; i < 4; ++i) take(sizeof(int32_t) * (n_as + 1));   // cnt_copy, off, fill, item_off
    take(sizeof(int4) * max_items);
    take(sizeof(int32_t) * P);                                        // perm
    take(sizeof(int32_t) * P);                                        // eid
    take(256);                                                        // total, err
    return o;
}

bool prefill_supported(int64_t K, int64_t N, int64_t n_as, std::string & why) {
    if (K % QK_K || K > PF_MAXK) { why = "prefill mul_mat_id: K must be a multiple of 256, <= 2048"; return false; }
    if (N % PF_ROWS) { why = "prefill mul_mat_id: N must be a multiple of 64"; return false; }
    if (n_as > PF_MAX_AS) { why = "prefill mul_mat_id: more than 4096 experts"; return false; }
    return true;
}

int launch_prefill(const MmidArgs & m, uint8_t * ws, hipStream_t s) {
    if (m.wtype != T_Q4_K) return fail(QWM_ERR_UNSUPPORTED, "prefill mul_mat_id: Q4_K weights only");
    std::string why;
    if (!prefill_supported(m.K, m.N, m.n_as, why)) return fail(QWM_ERR_UNSUPPORTED, why);
    const int64_t rows = m.T * m.ne11, P = m.T * m.n_ids;
    const int64_t max_items = (P / PF_TOK + m.n_as) * ((m.N / PF_ROWS + PF_RT - 1) / PF_RT);
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    PfArgs a;
    a.b = m.b; a.b_nb1 = m.b_nb1; a.b_nb2 = m.b_nb2; a.ids = m.ids; a.ids_nb1 = m.ids_nb1;
    a.as = m.as; a.slab = m.slab; a.row_bytes = (size_t)(m.K / QK_K) * 144;
    a.K = (int)m.K; a.N = (int)m.N; a.ne11 = (int)m.ne11; a.T = (int)m.T; a.n_ids = (int)m.n_ids; a.n_as = (int)m.n_as;
    a.qs = reinterpret_cast<int8_t *>(ws + take((size_t)rows * m.K));
    a.d = reinterpret_cast<float *>(ws + take(sizeof(float) * rows * (m.K / QK_K)));
    a.bs = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * rows * (m.K / 16)));
    a.cnt_copy = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * (m.n_as + 1)));
    a.off = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * (m.n_as + 1)));
    a.fill = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * (m.n_as + 1)));
    a.item_off = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * (m.n_as + 1)));
    a.items = reinterpret_cast<int4 *>(ws + take(sizeof(int4) * max_items));
    a.perm = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * P));
    a.eid = reinterpret_cast<int32_t *>(ws + take(sizeof(int32_t) * P));
    a.total = reinterpret_cast<int32_t *>(ws + take(256));
    a.err = a.total + 1;
    a.dst = m.dst; a.dst_nb1 = m.dst_nb1; a.dst_nb2 = m.dst_nb2;
    const int64_t nblk = rows * (m.K / QK_K);
    const unsigned prep_grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(1024, std::max((nblk + 3) / 4, (P + 255) / 256)));
    QWM_TIMED("prefill_prep", s, k_pf_prep<<<prep_grid, 256, 0, s>>>(a));
    k_pf_scan<<<1, 1024, 0, s>>>(a);
    k_pf_scatter<<<(unsigned)std::max<int64_t>(1, std::min<int64_t>(1024, (P + 255) / 256)), 256, 0, s>>>(a);
    const dim3 grid((unsigned)max_items);
    prof_begin("prefill_gemm", s);
    switch (m.K / QK_K) {
        case 1: k_pf_gemm<1><<<grid, 256, 0, s>>>(a); break;
        case 2: k_pf_gemm<2><<<grid, 256, 0, s>>>(a); break;
        case 3: k_pf_gemm<3><<<grid, 256, 0, s>>>(a); break;
        case 4: k_pf_gemm<4><<<grid, 256, 0, s>>>(a); break;
        case 5: k_pf_gemm<5><<<grid, 256, 0, s>>>(a); break;
        case 6: k_pf_gemm<6><<<grid, 256, 0, s>>>(a); break;
        case 7: k_pf_gemm<7><<<grid, 256, 0, s>>>(a); break;
        default: k_pf_gemm<8><<<grid, 256, 0, s>>>(a); break;
    }
    prof_end("prefill_gemm", s);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
