// qwm_verify.hip -- launcher of the stand-alone verify head (the device code
// is in qwm_vhead.h, shared with the fused verify step).
#include "qwm_internal.h"
#include "qwm_vhead.h"

namespace qwm {

template <int NT, int NS, int PF>
__global__ void __launch_bounds__(256) k_verify_head(VerifyArgs a) {
    __shared__ __align__(16) uint8_t smem[VhSmem<NT, NS>::bytes];
    // hidden sizes above 2048: the first tiles after the prep (their windows
    // and the prep's inputs do not fit the registers together)
    verify_body<NT, NS, PF, (NS > 4 ? VH_LATE : VH_EARLY)>(a, blockIdx.x, gridDim.x, smem);
}

static int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
    }
    return cus;
}

bool verify_plan(const qwm_tensor * lm_head, int64_t T, VerifyPlan & p, std::string & why) {
    p.H = lm_head->ne[0];
    p.V = lm_head->ne[1];
    p.T = T;
    if (lm_head->type != T_Q8_0) { why = "lm_head must be Q8_0"; return false; }
    if (p.H % 512 || (p.H > 2048 && p.H != 3072 && p.H != 4096)) {
        why = "lm_head: H must be 512, 1024, 1536, 2048, 3072 or 4096";
        return false;
    }
    if (T < 1 || T > VH_MAX_T) { why = "verify batch must hold 1..8 tokens"; return false; }
    if (p.H > 2048 && T > 4) { why = "lm_head: hidden sizes 3072 and 4096 take 1..4 tokens"; return false; }
    if (p.V < 1 || p.V > (1LL << 30)) { why = "lm_head: vocabulary size out of range"; return false; }
    p.n_wg = (int)std::min<int64_t>(2 * 256, (p.V + 7) / 8);
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    p.counters = take(256);
    p.hq = 0;
    p.partial_v = take(sizeof(float) * p.n_wg * T);
    p.partial_i = take(sizeof(int32_t) * p.n_wg * T);
    p.total = o;
    return true;
}

// Hidden sizes 3072 and 4096 (6 and 8 block sets per lane) run at one tile in
// flight and up to 4 tokens: the lane's windows and activations then fill its
// registers.
template <int NT>
static void launch_nt(const VerifyArgs & a, int n_wg, hipStream_t s) {
    constexpr int PF = NT <= 4 ? 2 : 1;
    const dim3 grid((unsigned)n_wg);
    switch (a.H) {
        case 512: k_verify_head<NT, 1, PF><<<grid, 256, 0, s>>>(a); break;
        case 1024: k_verify_head<NT, 2, PF><<<grid, 256, 0, s>>>(a); break;
        case 1536: k_verify_head<NT, 3, PF><<<grid, 256, 0, s>>>(a); break;
        case 3072:
            if constexpr (NT <= 4) k_verify_head<NT, 6, 1><<<grid, 256, 0, s>>>(a);
            break;
        case 4096:
            if constexpr (NT <= 4) k_verify_head<NT, 8, 1><<<grid, 256, 0, s>>>(a);
            break;
        default: k_verify_head<NT, 4, PF><<<grid, 256, 0, s>>>(a); break;
    }
}

int launch_verify(const uint8_t * lm_head, const float * x, const float * norm_w, float eps,
                  const int32_t * drafts, int32_t * result, const VerifyPlan & p, uint8_t * ws, hipStream_t s) {
    VerifyArgs a;
    a.W = lm_head; a.H = (int)p.H; a.V = (int)p.V;
    a.x = x; a.norm_w = norm_w; a.eps = eps;
    a.drafts = drafts; a.result = result;
    a.pv = reinterpret_cast<float *>(ws + p.partial_v);
    a.pi = reinterpret_cast<int32_t *>(ws + p.partial_i);
    a.counter = reinterpret_cast<int32_t *>(ws + p.counters);
    const int n_wg = std::min(p.n_wg, 2 * device_cus());
    prof_begin("lm_head", s);
    switch (p.T) {
        case 1: launch_nt<1>(a, n_wg, s); break;
        case 2: launch_nt<2>(a, n_wg, s); break;
        case 3: launch_nt<3>(a, n_wg, s); break;
        case 4: launch_nt<4>(a, n_wg, s); break;
        case 5: launch_nt<5>(a, n_wg, s); break;
        case 6: launch_nt<6>(a, n_wg, s); break;
        case 7: launch_nt<7>(a, n_wg, s); break;
        default: launch_nt<8>(a, n_wg, s); break;
    }
    prof_end("lm_head", s);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
