// Race-check instantiations of the main kernel (see debug_sync in
// fa3_bwd_main_kernel.h), in a translation unit of their own so that they
// build beside the fast ones.
#include "fa3_bwd_main_kernel.h"

namespace fa3 {

void launch_race_check(const FusedArgs& a, int head_dim, bool causal, bool bf16,
                       hipStream_t stream) {
    if (head_dim == 128) launch_dd<128, true>(a, causal, bf16, stream);
    else launch_dd<64, true>(a, causal, bf16, stream);
}

}  // namespace fa3
