// qwm_step_hi.hip -- the fused verify step's instantiations for T = 6, 7
// (qwm_step_kernel.h), compiled beside qwm_step.hip.
#include "qwm_step_kernel.h"

namespace qwm {

int launch_step_hi(StepArgs & a, int T, int nb_d, hipStream_t s) {
    return T == 6 ? launch_step_nt<6>(a, nb_d, s) : launch_step_nt<7>(a, nb_d, s);
}

}  // namespace qwm
