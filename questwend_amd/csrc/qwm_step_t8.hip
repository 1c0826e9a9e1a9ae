// qwm_step_t8.hip -- the fused verify step's instantiations for T = 8
// (qwm_step_kernel.h), compiled beside qwm_step.hip.
#include "qwm_step_kernel.h"

namespace qwm {

int launch_step_t8(StepArgs & a, int nb_d, hipStream_t s) { return launch_step_nt<8>(a, nb_d, s); }

}  // namespace qwm
