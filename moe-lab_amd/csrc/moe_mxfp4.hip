// MXFP4 expert kernels for gfx950 (E2M1 codes, one E8M0 scale per 32 weights).
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

int run_mxfp4_slots(const ExpertsArgs&) { return MOE_ERR_DTYPE; }
int run_mxfp4_grouped(const ExpertsArgs&) { return MOE_ERR_DTYPE; }

}  // namespace moe
