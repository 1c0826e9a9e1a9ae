/*
 * qwmoe.h -- C ABI of libqwmoe, the MI355X (gfx950) implementation of
 * QuestWend's MoE expert hot path: router top-k, GGML_OP_MUL_MAT_ID over
 * Q4_K / Q8_0 expert slot pools, SwiGLU, the gate-weighted combine (+ shared
 * expert), the verify head (rms_norm -> Q8_0 lm_head -> argmax) with greedy
 * MTP acceptance, the GPU LRU slot pool and its slab fetch.
 *
 * Conventions
 *  - Tensors use ggml's layout: ne[0] is the contiguous dimension, nb[] are
 *    byte strides, `type` is a ggml_type value (ggml.h:390-420).  Data
 *    pointers are device pointers unless a comment says host.
 *  - Every entry point returns QWM_OK (0) or a negative QWM_ERR_* code and
 *    never throws (each body runs behind an exception barrier); size queries
 *    return 0 instead.  qwm_last_error() describes the last failure of the
 *    calling thread.  The slot pool's calls take every allocation before
 *    their first change to the pool, so a QWM_ERR_NOMEM leaves it as it was.
 *    QWM_ERR_UNSUPPORTED means "shape/type not handled here": the caller
 *    keeps its own fallback, as ggml's supports_op contract expects.
 *  - The library allocates no device memory on the hot path.  Scratch comes
 *    from a caller-owned workspace sized by qwm_*_workspace_size() and zeroed
 *    once with qwm_workspace_init() (it keeps self-resetting counters).
 *    The counters' places depend on the call's shape: before a workspace
 *    serves calls of another shape (T, layer shape), initialize it again.
 *    (qwm_mul_mat_id keeps no state between calls.)
 *  - Work is enqueued on the given hipStream_t (passed as void*); calls are
 *    asynchronous unless stated otherwise.  Calls that share a workspace must
 *    be ordered on one stream.
 *  - Numerics follow ggml's CPU backend on x86-64 (AVX-512 build): activations
 *    entering Q4_K dots are quantized to Q8_K, those entering Q8_0 dots with
 *    the x86 Q8_0 quantizer, so every 32/256-element block sum is the same
 *    integer; router logits, softmax and the weight normalization reproduce
 *    the CPU's floating-point order.
 */
#ifndef QWMOE_H
#define QWMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWM_OK               0
#define QWM_ERR_UNSUPPORTED (-1)
#define QWM_ERR_ARG         (-2)
#define QWM_ERR_WORKSPACE   (-3)
#define QWM_ERR_HIP         (-4)
#define QWM_ERR_NO_VICTIM   (-5)
#define QWM_ERR_STATE       (-6)
#define QWM_ERR_IO          (-7)
#define QWM_ERR_NOMEM       (-8)   /* host memory ran out (std::bad_alloc inside the library) */
#define QWM_ERR_INTERNAL    (-9)   /* any other C++ exception inside the library */

/* ggml_type values used on this path (ggml.h:390-420) */
#define QWM_TYPE_F32   0
#define QWM_TYPE_Q8_0  8
#define QWM_TYPE_Q4_K 12
#define QWM_TYPE_Q5_K 13
#define QWM_TYPE_Q6_K 14
#define QWM_TYPE_I32  26

/* Mirrors the data-carrying part of struct ggml_tensor (ggml.h). */
typedef struct qwm_tensor {
    int32_t type;
    int64_t ne[4];
    size_t  nb[4];
    void *  data;
} qwm_tensor;

/* Fills ne/nb for a contiguous tensor of the given type (nb[0] = block size). */
void qwm_tensor_init(qwm_tensor * t, int32_t type, int64_t ne0, int64_t ne1, int64_t ne2, void * data);

const char * qwm_version(void);
const char * qwm_last_error(void);

/* Zero-fills a workspace (a fill kernel, no hipMemsetAsync; safe to capture). */
int qwm_workspace_init(void * workspace, size_t bytes, void * stream);

/* ---------------------------------------------------------------- ops ---- */

/* GGML_OP_MUL_MAT_ID (ggml.c:3398-3440; CPU: ggml-cpu.c:1554-1734):
 *   dst[:, e, t] = as[:, :, ids[e, t]] . b[:, e % ne11(b), t]
 * as: Q4_K, Q5_K, Q6_K or Q8_0 [K, N, n_as]; b: f32 [K, ne11, T]; ids: i32
 * [n_ids, T]; dst: f32 [N, n_ids, T].  Supported: K a multiple of 256 up
 * to 2048, or 3072 or 4096; Q5_K data 16-byte aligned, Q6_K and Q8_0 4-byte
 * aligned.
 *   T <= 8: one GEMV launch, n_ids * T <= 128.
 *   T > 8, Q4_K or Q8_0 with N % 64 == 0 and 16-byte aligned data: the
 *   grouped int8-MFMA GEMM (prefill), n_ids * T <= 2^22.
 *   T > 8, otherwise: GEMV launches over column chunks, n_ids <= 128.
 * The workspace size covers either T > 8 path. */
size_t qwm_mul_mat_id_workspace_size(const qwm_tensor * as, const qwm_tensor * b, const qwm_tensor * ids);
int qwm_mul_mat_id(const qwm_tensor * as, const qwm_tensor * b, const qwm_tensor * ids, qwm_tensor * dst,
                   void * workspace, size_t ws_bytes, void * stream);

/* GGML_GLU_OP_SWIGLU in split form (ggml_swiglu_split, ggml.c:3082; CPU
 * ggml_compute_forward_swiglu_f32, ops.cpp:3331-3385): act = silu(gate) * up
 * per row of ne[0] elements, ggml_vec_swiglu_f32's vectorized silu on the
 * 16-wide chunks and libm expf on the tail.  gate, up, act: contiguous f32 of
 * one shape; act may alias gate or up.  No workspace. */
int qwm_swiglu(const qwm_tensor * gate, const qwm_tensor * up, qwm_tensor * act, void * stream);

/* The expert FFN's first half in one call: act = ggml_swiglu_split(
 * MUL_MAT_ID(gate, b, ids), MUL_MAT_ID(up, b, ids)), the two MUL_MAT_ID nodes
 * and the GGML_GLU_OP_SWIGLU node of build_segB (core/runtime.cpp:4539-4541;
 * ops.cpp:3331-3385).  gate and up: same type, shape and strides, each as
 * qwm_mul_mat_id's `as`; act: contiguous f32 [N, n_ids, T].  Where
 * qwm_mul_mat_id takes the grouped GEMM, one grouped pass streams the gate
 * and up rows of each tile side by side and writes act (no gate/up
 * intermediates in HBM; the activations are quantized once).  Otherwise two
 * qwm_mul_mat_id calls into the workspace and an element-wise pass; the
 * workspace size covers both.  Either way act equals, bit for bit, SwiGLU
 * applied to what two qwm_mul_mat_id calls return. */
size_t qwm_mul_mat_id_swiglu_workspace_size(const qwm_tensor * gate, const qwm_tensor * up, const qwm_tensor * b,
                                            const qwm_tensor * ids);
int qwm_mul_mat_id_swiglu(const qwm_tensor * gate, const qwm_tensor * up, const qwm_tensor * b, const qwm_tensor * ids,
                          qwm_tensor * act, void * workspace, size_t ws_bytes, void * stream);

/* --------------------------------------------------- the MoE FFN block --- */

/* One MoE layer's weights: slot pools in ggml layout (gate/up [H, N, S],
 * down [N, H, S]), the f32 router [H, E], and an optional shared expert
 * (data == NULL when absent): gate/up [H, N_sh], down [N_sh, H], and the
 * optional f32 shared gate row [H, 1].  gate/up are Q4_K, Q5_K or Q8_0 and
 * down the same type (or Q6_K beside Q4_K/Q5_K, as K-quant "_M" files have
 * it); the shared expert's types match the pools'.  N is a multiple of 256
 * up to 2048; H too, or 3072 or 4096 (the fused verify step and the
 * persistent decode take 2048 only). */
typedef struct qwm_moe_layer {
    qwm_tensor gate_pool, up_pool, down_pool;
    qwm_tensor router;
    qwm_tensor sh_gate, sh_up, sh_down, sh_gate_inp;
    int32_t n_expert_used;      /* k */
    int32_t norm_weights;       /* hparams.expert_weights_norm */
    float   weights_scale;      /* hparams.expert_weights_scale (0 or 1: none) */
    int32_t gating_func;        /* hparams.expert_gating_func: 2 = sigmoid; 0 or 1 = soft_max */
    qwm_tensor exp_probs_b;     /* optional f32 [E] ranking bias (blk.N.exp_probs_b.bias); data NULL: none */
} qwm_moe_layer;

/* Router (core/runtime.cpp:2693-2734 after the router mul_mat 3785-3798):
 *   logits = router . x (+ rm);  probs = soft_max(logits) (gating_func 2: sigmoid);
 *   rank = probs (+ exp_probs_b, then + rm again);
 *   ids = top-k(rank) [k, T];    w = probs[ids] (/ clamp(sum, 6.1035e-5) if norm)
 * x: f32 [H, T]; rm: optional f32 [E, T] added to the logits; ids_out: i32
 * [k, T]; w_out: f32 [k, T].  The top-k keeps the lower expert index on exact
 * rank ties (std::sort leaves their order unspecified).  T <= 8.
 * Activation tensors (x, out, resid) must be 16-byte aligned. */
size_t qwm_moe_workspace_size(const qwm_moe_layer * layer, int64_t T);
int qwm_moe_route(const qwm_moe_layer * layer, const qwm_tensor * x, const qwm_tensor * rm,
                  qwm_tensor * ids_out, qwm_tensor * w_out, void * workspace, size_t ws_bytes, void * stream);

/* Expert FFN over the slot pools (build_moe_cached, runtime.cpp:3801-3830,
 * and build_segB, 4534-4572):
 *   up = mul_mat_id(up_pool, x, slot_u); gate = mul_mat_id(gate_pool, x, slot_g)
 *   act = swiglu(gate, up); experts = mul_mat_id(down_pool, act, slot_d)
 *   T == 1: out = cont(transpose(experts)) . w     (k-ordered fused sum)
 *   T >  1: out = e0*w0 + e1*w1 + ... left to right
 *   + shared expert: out += down_sh(silu(gate_sh x) * up_sh x) [* sigmoid(g_inp . x)]
 *   if resid != NULL: out += resid (the block's residual add).
 * Must follow qwm_moe_route on the same workspace (it reuses the quantized x
 * and the expert schedule).  slot_*: i32 [k, T] device slot ids; weights: f32
 * [k, T]; out: f32 [H, T]. */
int qwm_moe_experts(const qwm_moe_layer * layer, const qwm_tensor * x, const qwm_tensor * slot_g,
                    const qwm_tensor * slot_u, const qwm_tensor * slot_d, const qwm_tensor * weights,
                    const qwm_tensor * resid, qwm_tensor * out, void * workspace, size_t ws_bytes, void * stream);

/* Route + experts with the in-graph slot remap of the fast decode path
 * (runtime.cpp:2759-2787): slot = slot_of[role][layer * E + id] read on the
 * device from `slot_tables` (i32 [E * n_layer, 3], role-major: gate, up,
 * down).  No host round trip; the pools must hold every selected expert.
 * Slot ids (here, in qwm_moe_experts' slot tensors and in the other
 * resident paths) are not checked against the pools: the kernels clamp an
 * id outside [0, S) into the pool, so a bad id computes with a wrong slab
 * but never reads outside the pool tensor.  The cached paths take their ids
 * from the pool, which are always in range. */
int qwm_moe_block_resident(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                           int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm,
                           const qwm_tensor * resid, qwm_tensor * out, qwm_tensor * ids_out, qwm_tensor * w_out,
                           void * workspace, size_t ws_bytes, void * stream);

/* Decode through stacked MoE blocks (the per-layer segment B of
 * decode_cached, runtime.cpp:5064-5888, with every expert resident and the
 * in-graph slot remap of 2759-2787): for l = 0 .. n_layers-1,
 *   x = x + MoE_l(x)     (qwm_moe_block_resident with layer index l)
 * x: f32 [H, T] in/out.  The layers share one shape.  slot_tables as for
 * qwm_moe_block_resident, with table_stride >= n_layers * E.  Nothing waits
 * for the host between layers; the call can be captured in a HIP graph (its
 * only copy, for odd n_layers, is a device-to-device memcpy). */
size_t qwm_moe_decode_workspace_size(const qwm_moe_layer * layers, int32_t n_layers, int64_t T);
int qwm_moe_decode(const qwm_moe_layer * layers, int32_t n_layers, const int32_t * slot_tables, int64_t table_stride,
                   qwm_tensor * x, void * workspace, size_t ws_bytes, void * stream);

/* qwm_moe_decode with the record of the optimistic single-graph decode
 * (decode_cached_fast: the selection kept per layer, runtime.cpp:2759-2766;
 * residency verified after the run, 6155-6166, and the selected experts
 * touched, 6170-6176):
 *   ids_all: device i32 [k, T, n_layers] or NULL: every layer's selected
 *     experts (the runtime's sel_all);
 *   resident_bits: device u32 [n_layers][ceil(E / 32)] or NULL: bit e of
 *     layer l set when expert e of layer l is resident in all three role
 *     pools (qwm_pool_resident_bits);
 *   miss_flag: device i32, cleared by the call and set to 1 when a selected
 *     expert's bit is clear.  Such a layer read the slot-0 sentinel of its
 *     slot table, so x is then invalid: the reference restores its state and
 *     runs the token through the cached path (decode_cached); with the flag
 *     clear, the caller touches the selected experts (qwm_pool_touch).
 * Graph-capturable like qwm_moe_decode (the flag is cleared by a kernel). */
int qwm_moe_decode_sel(const qwm_moe_layer * layers, int32_t n_layers, const int32_t * slot_tables,
                       int64_t table_stride, qwm_tensor * x, int32_t * ids_all, const uint32_t * resident_bits,
                       int32_t * miss_flag, void * workspace, size_t ws_bytes, void * stream);

/* -------------------------------------------------- verify + acceptance --- */

/* Verify head + greedy acceptance (runtime.cpp:5014-5046 and 3648-3652):
 *   h = rms_norm(x, eps) * norm_w;  logits = lm_head . h (Q8_0 [H, V]);
 *   vA[t] = argmax(logits[:, t])  (last index among equal maxima)
 *   a = longest prefix with vA[j] == drafts[j], j < n_draft;  x_new = vA[a]
 * x: f32 [H, T]; norm_w: optional f32 [H]; drafts: device i32 [n_draft]
 * (n_draft = T - 1); result: device i32 [T + 2] = vA[0..T-1], a, x_new.
 * Supported: H in {512, 1024, 1536, 2048} with 1 <= T <= 8, H in {3072, 4096}
 * with 1 <= T <= 4; x and norm_w 16-byte
 * aligned, lm_head 4-byte aligned with contiguous rows. */
size_t qwm_verify_workspace_size(const qwm_tensor * lm_head, int64_t T);
int qwm_verify_accept(const qwm_tensor * lm_head, const qwm_tensor * x, const float * norm_w, float eps,
                      const int32_t * drafts, int32_t * result, void * workspace, size_t ws_bytes, void * stream);

/* ------------------------------------------------- the fused verify step --- */

/* One MTP verify step in a single launch: qwm_moe_block_resident followed by
 * qwm_verify_accept on the block's output (runtime.cpp:2759-2787 for the
 * in-graph slot remap, 3801-3830 / 4534-4572 for the block, 5014-5046 and
 * 3648-3652 for the head), with the same numerics.  The kernel is persistent:
 * a grid of exactly the workgroups the GPU holds at once, handing data to each
 * other through the workspace, so the launch occupies the whole GPU until it
 * ends (work on other streams delays it).
 *   out = MoE(x) (+ resid);  h = rms_norm(out) * norm_w;  vA = argmax(lm_head . h)
 *   result: device i32 [T + 2] = vA[0..T-1], a, x_new; a = -1 reports a
 *   device-side synchronization timeout (results invalid).
 * Supported: Q4_K pools, hidden size 2048, FFN width 512, 768, 1024 or 2048
 * (a shared expert of the same width), <= 512 experts, lm_head Q8_0 [2048, V]
 * with V >= 8192, T <= 8.  out must not overlap x or resid.  ids_out,
 * w_out and norm_w may be NULL.  QWM_ERR_UNSUPPORTED: use the two calls. */
size_t qwm_verify_step_workspace_size(const qwm_moe_layer * layer, const qwm_tensor * lm_head, int64_t T);
int qwm_verify_step(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                    int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm, const qwm_tensor * resid,
                    qwm_tensor * out, qwm_tensor * ids_out, qwm_tensor * w_out, const qwm_tensor * lm_head,
                    const float * norm_w, float eps, const int32_t * drafts, int32_t * result,
                    void * workspace, size_t ws_bytes, void * stream);

/* qwm_verify_step without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * step's scratch is a static device array of QWM_NOALLOC_SCRATCH_BYTES that
 * each GPU holds until the process ends; every supported shape of
 * qwm_verify_step fits (a larger need returns QWM_ERR_UNSUPPORTED).  Each
 * call clears the part it uses with a fill kernel before the step (so the
 * call can be captured).  All calls on one GPU share that array: calls that
 * overlap on one GPU (other streams, other threads) race.  The device address
 * is looked up on the first call per device.  Allocates nothing. */
#define QWM_NOALLOC_SCRATCH_BYTES (4u << 20)
int qwm_verify_step_noalloc(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                            int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm, const qwm_tensor * resid,
                            qwm_tensor * out, qwm_tensor * ids_out, qwm_tensor * w_out, const qwm_tensor * lm_head,
                            const float * norm_w, float eps, const int32_t * drafts, int32_t * result, void * stream);

/* ------------------------------------------------------- quantization --- */

/* Model-file quantization on the device, as ggml_quantize_chunk does it
 * without an importance matrix: Q4_K = quantize_row_q4_K_ref
 * (ggml-quants.c:1458-1528), Q8_0 = quantize_row_q8_0_ref (276-300).
 * src: f32 [n] (n a multiple of the block length); dst: n / block * bytes. */
int qwm_quantize(int32_t type, const float * src, void * dst, int64_t n, void * stream);

/* -------------------------------------------------------- measurement --- */

/* Brackets each of the next `max_launches` launches of one kernel with a
 * hipEvent pair on the stream it runs on.  Kernel names: "route",
 * "gate_up", "down" (with the combine), "lm_head", "step" (the fused verify
 * step), "decode" (the persistent decode), "mul_mat_id_prep", "mul_mat_id",
 * "prefill_prep", "prefill_gemm" (the prefill GEMM), "prefill_gemm_gu" (its
 * gate/up/SwiGLU form).  A name ending in '*' matches every kernel name that
 * starts with the text before it.  Owner thread only. */
int qwm_profile_start(const char * kernel, int32_t max_launches);
/* Waits for the recorded events, writes each launch's duration in ms and
 * returns how many launches were timed (stops the profiling). */
int qwm_profile_stop(float * durations_ms, int32_t capacity);

/* The bound of every wait inside the persistent launches (the fused verify
 * step, the persistent decode loop), in polls of the waiting wave (a read of
 * the counter and a 64-cycle sleep each); default 2^21.  A wait that runs out lets its workgroup go on, and the call
 * reports it: the verify result's a and x_new are -1, the decode miss flag
 * gets bit 1 (value 2).  The launches re-arm their counters either way, so
 * the next call on the same workspace is unaffected.  A small bound (0 gives
 * up after one read) forces that path, for tests of it.  Calls launched
 * afterwards use the new bound. */
int qwm_set_spin_limit(uint32_t polls);

/* ---------------------------------------------------------- slot pool --- */

/* ExpertCache's RAM-tier decisions (core/expert_cache.cpp: ensure 1615-1645,
 * slot_for 1465-1479, install 1173-1180, pick_victim 1129-1170, drop
 * 1067-1088; hooks core/gpu_lru_pool_hooks.h): one pool per role over all
 * layers, one global clock, lowest free slot first, else the least recently
 * used unprotected slot.  Misses are copied from pinned host slabs with
 * hipMemcpyAsync on the pool's copy stream; the compute stream is made to
 * wait for them (qwm_pool_wait).  Host-side, owner thread only. */
typedef struct qwm_pool qwm_pool;

typedef struct qwm_pool_desc {
    int32_t n_layer, n_expert;
    int32_t n_slots[3];          /* per role: gate, up, down */
    void *  pool_data[3];        /* device base of each role's [K, N, n_slots] tensor */
    size_t  slab_bytes[3];       /* nb[2] of each role */
    const void * const * host_slabs[3]; /* per role: host_slabs[r][layer] = pinned [K, N, n_expert] source; may be NULL */
    int32_t protect_active;      /* 1: ActiveExpertGuard protection (TinyLFU mode); 0: reference default */
    int32_t indexed;             /* 1: O(1) indexed LRU (QWEN_GPU_LRU_INDEX=1); 0: linear scan */
    int32_t fetch_mode;          /* QWM_FETCH_MEMCPY or QWM_FETCH_GATHER */
} qwm_pool_desc;

/* How misses reach the pool (the bytes are the same either way):
 * MEMCPY: one hipMemcpyAsync per missed slab on the copy stream, as the
 *   reference's fetch_slab; host slabs may be pageable (then the copies are
 *   synchronous).
 * GATHER: one kernel per qwm_pool_ensure call on the copy stream pulls every
 *   missed slab of the call over the host link (about twice the rate of
 *   per-slab copies for 576 KiB slabs).  Host slabs must be pinned
 *   (hipHostMalloc) and, like pool_data, 16-byte aligned; slab_bytes a
 *   multiple of 16; at most 32767 slots per role.  qwm_pool_create checks
 *   these. */
#define QWM_FETCH_MEMCPY 0
#define QWM_FETCH_GATHER 1

typedef struct qwm_pool_stats {
    uint64_t hits, misses, evictions, fetch_bytes, fetches;
    uint64_t clock;
} qwm_pool_stats;

int qwm_pool_create(const qwm_pool_desc * desc, void * copy_stream, qwm_pool ** out);
void qwm_pool_destroy(qwm_pool * pool);

/* Signature pools (ExpertCache's constructor, expert_cache.cpp:225-296): one
 * pool per (role, type, ne0, ne1) of the expert tensors, so that a file whose
 * ffn_down_exps is Q6_K on some layers and Q4_K on others keeps each in a
 * pool of its own slab size.  Every (role, layer) is routed to one pool; a
 * pool holds the keys (layer * n_expert + expert) of all the layers routed
 * to it; one clock and one quota per layer serve every pool.  A pool made
 * by qwm_pool_create is the case of three pools, pool r serving role r of
 * every layer. */
typedef struct qwm_pool_sig {
    int32_t role;                /* 0 gate, 1 up, 2 down */
    int32_t type;                /* ggml type of the expert tensors */
    int64_t ne0, ne1;            /* their first two dimensions */
    size_t  slab_bytes;          /* their nb[2] */
    int32_t n_layers;            /* layers routed to this pool */
    int32_t n_slots;
    void *  pool_data;           /* device [ne0, ne1, n_slots]: set by the caller before qwm_pool_create_sig */
} qwm_pool_sig;

/* Signature discovery and sizing (expert_cache.cpp:225-287).  experts: the
 * expert tensors per (role, layer), role-major (experts[r * n_layer + l];
 * type, ne[0..2] and nb[2] are read; ne[2] must be n_expert).  For roles in
 * order and layers in order, a tensor joins the first signature with its
 * role, type, ne0 and ne1, or opens a new one (sigs[], in that order, at most
 * max_sigs); layer_pool[r * n_layer + l] receives the index.  Sizing: frac =
 * vram_bytes / sum(slab_bytes * n_layers * n_expert), at most 1; a pool gets
 * (int)(frac * n_layers * n_expert) slots, at least n_used and at most that
 * cap.  A pool left with n_used slots or fewer is refused (QWM_ERR_ARG), as
 * the reference refuses it.  *frac_out (may be NULL): frac.  pool_data is
 * left NULL. */
int qwm_pool_plan_sigs(int32_t n_layer, int32_t n_expert, const qwm_tensor * experts, uint64_t vram_bytes,
                       int32_t n_used, qwm_pool_sig * sigs, int32_t max_sigs, int32_t * n_sigs,
                       int32_t * layer_pool, double * frac_out);

typedef struct qwm_pool_sig_desc {
    int32_t n_layer, n_expert;
    int32_t n_pools;
    const qwm_pool_sig * pools;  /* [n_pools]: role, n_slots, pool_data and slab_bytes are used */
    const int32_t * layer_pool;  /* [3 * n_layer], role-major: the pool of (role, layer), of that role */
    const void * const * host_slabs[3]; /* as in qwm_pool_desc */
    int32_t protect_active, indexed, fetch_mode; /* as in qwm_pool_desc */
} qwm_pool_sig_desc;
int qwm_pool_create_sig(const qwm_pool_sig_desc * desc, void * copy_stream, qwm_pool ** out);
/* The pool index of (role, layer) (0..n_pools-1), or a QWM_ERR_* code. */
int qwm_pool_layer_pool(const qwm_pool * pool, int32_t role, int32_t layer);
/* ids: host i32 [n] (token-major); slot_*: host i32 [n].  Issues the slab
 * copies for misses on the copy stream.  QWM_ERR_NO_VICTIM leaves the pool
 * consistent (the failing role is not published; the misses before it are
 * fetched).  The copies overwrite the victims' slots without waiting for
 * other streams: the caller makes sure that no kernel still reads them (in
 * the decode loop the synchronous read-back of the routed ids that precedes
 * this call does). */
int qwm_pool_ensure(qwm_pool * pool, int32_t layer, const int32_t * ids, int32_t n,
                    int32_t * slot_gate, int32_t * slot_up, int32_t * slot_down);
/* Makes `stream` wait for every slab copy issued so far (hipStreamWaitEvent). */
int qwm_pool_wait(qwm_pool * pool, void * stream);
int qwm_pool_get_stats(const qwm_pool * pool, qwm_pool_stats * out);
/* Dense expert -> slot row of (role, layer), 0 for non-resident experts
 * (ExpertCache::slot_of_row, expert_cache.cpp:1448-1451); host i32 [n_expert].
 * The slots index the pool of (role, layer). */
int qwm_pool_slot_of_row(const qwm_pool * pool, int32_t role, int32_t layer, int32_t * out);
/* Per-slot key (layer * n_expert + expert, -1 free) and clock of pool
 * `pool_index` (for a pool made by qwm_pool_create, the role). */
int qwm_pool_slots(const qwm_pool * pool, int32_t pool_index, int32_t * keys, uint64_t * clocks);
/* ExpertCache::resident for all three roles (expert_cache.cpp:1442-1446), as
 * a bitmap: bit e of bits[e / 32] set when expert e of `layer` is resident
 * in the gate, up and down pools; host u32 [ceil(n_expert / 32)]. */
int qwm_pool_resident_bits(const qwm_pool * pool, int32_t layer, uint32_t * bits);
/* ExpertCache::touch (expert_cache.cpp:1453-1463) of GATE, UP, DOWN for each
 * of ids[0..n) in order (runtime.cpp:6170-6176): a resident key counts one
 * access, its slot takes clock + 1 and the hit counter grows; a key that is
 * not resident is left alone. */
int qwm_pool_touch(qwm_pool * pool, int32_t layer, const int32_t * ids, int32_t n);

/* One layer of the cached decode path (decode_cached, runtime.cpp:5292-5341)
 * in one call: qwm_moe_route, the routed ids read back to the host
 * (synchronizes `stream`, as the reference's D2H read does),
 * qwm_pool_ensure(pool, layer_index, ...) with the misses copied on the
 * pool's copy stream, the slot ids uploaded, qwm_pool_wait(pool, stream),
 * then qwm_moe_experts on the slot ids (resid may be NULL).  ids_host
 * (i32 [T * k], may be NULL) receives the routed ids.  The layer's pools are
 * the device tensors of the pools of (role, layer_index): same base, nb[2]
 * equal to their slab bytes and ne[2] at least their slots (QWM_ERR_ARG
 * otherwise).  Not capturable into a graph (host round trip).
 * Pool errors (QWM_ERR_NO_VICTIM, QWM_ERR_IO) are returned before the
 * experts run. */
size_t qwm_moe_cached_workspace_size(const qwm_moe_layer * layer, int64_t T);
int qwm_moe_cached_step(const qwm_moe_layer * layer, qwm_pool * pool, int32_t layer_index, const qwm_tensor * x,
                        const qwm_tensor * rm, const qwm_tensor * resid, qwm_tensor * out, int32_t * ids_host,
                        void * workspace, size_t ws_bytes, void * stream);

/* ExpertCache::capacity (expert_cache.cpp:478-491): the fewest slots the
 * layer may hold in any role before recycling its own (its quota, at least
 * n_used, while quotas are on; else the pool size).  quota_of (493-501): the
 * layer's quota (the pool size where none was computed).  set_quotas /
 * quotas_active: ExpertCache::set_quotas / quotas_active (expert_cache.h:
 * 154-162).  Return values >= 0, or a QWM_ERR_* code. */
int qwm_pool_capacity(const qwm_pool * pool, int32_t layer);
int qwm_pool_quota_of(const qwm_pool * pool, int32_t layer);
int qwm_pool_quotas_active(const qwm_pool * pool);
int qwm_pool_set_quotas(qwm_pool * pool, int32_t on);
/* decode_cached_batch's plan_slices (runtime.cpp:4639-4687) for the routed
 * ids sel (host i32 [T * n_used], token-major) of one layer: quotas switched
 * on when the batch's expert union fits quota_of(layer) - 8 and off
 * otherwise (left so: save qwm_pool_quotas_active() before a batch and
 * restore it after, as the reference's QuotaScope does); then slices
 * (t0, len) of consecutive tokens, cut where the slice's union would pass
 * max(n_used, capacity(layer) - 8) or its length max_slice (0: 1024, the
 * QWEN_SEGB_SLICE default).  slices: host i32 [2 * T]; *union_out (may be
 * NULL) receives the batch's union size. */
int qwm_pool_plan_slices(qwm_pool * pool, int32_t layer, const int32_t * sel, int32_t T, int32_t n_used,
                         int32_t max_slice, int32_t * slices, int32_t * n_slices, int32_t * union_out);

/* A batch of 1..QWM_BATCH_MAX_T tokens through one MoE layer on the slot pool
 * (decode_cached_batch's router, plan_slices / ensure_slice and seg B,
 * runtime.cpp:4509-4572, 4639-4698):
 *   the router for every token (qwm_moe_route's numerics, eight tokens per
 *   launch); the routed ids read back (synchronizes `stream`); the slices
 *   planned on the pool (qwm_pool_plan_slices, which sets the quota mode);
 *   per slice: qwm_pool_ensure (after the previous slice's kernels finish,
 *   so that no victim is still being read), the slot ids uploaded,
 *   qwm_pool_wait, then up/gate MUL_MAT_ID, SwiGLU, down MUL_MAT_ID, the
 *   weighted sum in k order (ggml_mul then a left-to-right ggml_add chain),
 *   the shared expert times its sigmoid gate, and resid (may be NULL).
 * x, resid, out: f32 [H, T] (out must not overlap x); rm: optional f32
 * [E, T].  ids_host (host i32 [k * T]), slices_host (host i32 [2 * T]) and
 * n_slices may be NULL.  The layer's pools are the pools of (role,
 * layer_index), checked as in qwm_moe_cached_step.
 * Slices of more than 8 tokens run the grouped MUL_MAT_ID GEMM (Q4_K) or GEMV
 * launches over column chunks (other types).  Not capturable. */
#define QWM_BATCH_MAX_T 4096
size_t qwm_moe_cached_batch_workspace_size(const qwm_moe_layer * layer, int64_t T, int32_t max_slice);
int qwm_moe_cached_batch(const qwm_moe_layer * layer, qwm_pool * pool, int32_t layer_index, const qwm_tensor * x,
                         const qwm_tensor * rm, const qwm_tensor * resid, qwm_tensor * out, int32_t max_slice,
                         int32_t * ids_host, int32_t * slices_host, int32_t * n_slices, void * workspace,
                         size_t ws_bytes, void * stream);

/* Cache profiles (ExpertCache::save_profile / load_prefetch,
 * expert_cache.cpp:1485-1538), in the reference's text format:
 * "QWENEXPCACHE 1", "n_layer n_expert", then "role layer expert count" per
 * key that ensure has counted (roles in order, keys ascending here).
 * load: a missing or incompatible profile installs nothing and returns
 * QWM_OK (cold start); otherwise entries in range, largest count first (equal
 * counts in file order), are installed into free slots until their role's
 * pool is full, skipping resident keys, their slabs fetched as misses are
 * (qwm_pool_wait orders them).  *n_installed (may be NULL) gets the count. */
int qwm_pool_save_profile(const qwm_pool * pool, const char * path);
int qwm_pool_load_profile(qwm_pool * pool, const char * path, int64_t * n_installed);

/* Per-layer quotas (ExpertCache::compute_quota / rebalance,
 * expert_cache.cpp:509-625): one quota per layer from the access counts
 * summed over the roles -- every layer first gets up to n_used experts (the
 * model's n_expert_used) while every role's pool has slots left, then the
 * counts, largest first (ties: larger key first), each give their layer one
 * more while slots remain.  From then on a miss of a layer at or over its
 * quota recycles one of that layer's slots, any other miss takes a slot from
 * a layer over its quota (least recently used first; none: the global LRU),
 * and the indexed mode's shortcut is off.  Then the hottest experts inside
 * each layer's quota are installed, all three roles, up to fill_budget
 * experts (*n_filled, may be NULL).  quota_out: host i32 [n_layer], may be NULL.
 * clear_counts: ExpertCache::clear_counts. */
int qwm_pool_rebalance(qwm_pool * pool, int32_t n_used, int64_t fill_budget, int32_t * quota_out,
                       int64_t * n_filled);
int qwm_pool_clear_counts(qwm_pool * pool);

/* File tier (ExpertCache::fetch_parallel's file path, expert_cache.cpp:
 * 1194-1440, with its persistent readers, expert_io_workers.h): misses of
 * (role, layer) are read from `path` at offset + expert * slab_bytes instead
 * of host_slabs.  At the end of each qwm_pool_ensure call, reader threads
 * pread the call's missed slabs into a pinned staging ring and each slab is
 * copied to its slot on the copy stream as soon as its read is complete, in
 * the order of the misses (so qwm_pool_ensure returns after the reads; the
 * copies complete asynchronously, as with the other fetch modes).  A failed
 * read returns QWM_ERR_IO and un-publishes that miss and the later ones of
 * the call (their experts are not resident afterwards).  The file must hold
 * offset + n_expert * slab_bytes bytes (QWM_ERR_ARG otherwise); the pool
 * keeps the descriptor open until qwm_pool_destroy or the next attach of the
 * same (role, layer). */
int qwm_pool_attach_file(qwm_pool * pool, int32_t role, int32_t layer, const char * path, uint64_t offset);
/* GGUF model files (Model::tensor_file_offset, core/model.cpp:454-458 and
 * 636-677): a tensor's ggml type, shape and absolute file offset (the data
 * section, the end of the tensor infos rounded up to general.alignment, plus
 * the tensor's offset).  nbytes = 0 for a type not sized here (sized: F32,
 * F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K..Q6_K).  QWM_ERR_IO: the
 * file cannot be opened; QWM_ERR_ARG: not GGUF v2/v3, malformed, or no such
 * tensor. */
typedef struct qwm_gguf_tensor {
    int32_t type, n_dims;
    int64_t ne[4];
    uint64_t offset, nbytes;
} qwm_gguf_tensor;
int qwm_gguf_find_tensor(const char * path, const char * name, qwm_gguf_tensor * out);
/* Attaches blk.<first_block + l>.ffn_{gate,up,down}_exps.weight (the names of
 * expert_cache.cpp:88-93) of a GGUF file to the file tier, for every layer l
 * of the pool; each must hold n_expert slabs of the role's slab_bytes
 * (QWM_ERR_ARG otherwise, naming the tensor). */
int qwm_pool_attach_gguf(qwm_pool * pool, const char * path, int32_t first_block);
/* Reader threads (1..64, default 8) and staging slabs (0: as many as fit in
 * 64 MiB, the reference's batch size) of the file tier. */
int qwm_pool_set_io(qwm_pool * pool, int32_t n_threads, int32_t staging_slabs);

/* One slab copy: pool_data + slot * slab_bytes <- pinned_src (async H2D on
 * copy_stream), then records done_event (a hipEvent_t, may be NULL)
 * (ExpertCache::fetch_slab RAM tier, expert_cache.cpp:706-717). */
int qwm_slab_fetch_async(void * pool_data, size_t slab_bytes, int32_t slot, const void * pinned_src,
                         void * copy_stream, void * done_event);

#ifdef __cplusplus
}
#endif

#endif /* QWMOE_H */
