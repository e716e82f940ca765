/*
 * shaobo_fa3_components.h -- per-stage entry points of libshaobo_fa3_bwd.so
 * (reference: include/shaobo_fa3_components.h:10-58).
 */
#ifndef SHAOBO_FA3_COMPONENTS_H_
#define SHAOBO_FA3_COMPONENTS_H_

#include "shaobo_fa3_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Delta preprocess (reference src/dot_do_o_kernel.cpp:78-125).
 *   delta[r]            = sum_d dout[r, d] * out[r, d]        (fp32, rows = B*Hq*S)
 *   packed_sidecar[r*3] = {row_max_log2, row_inv_sum, delta[r]}
 * LSE mode (params->softmax_aux_mode == LSE): row_max_log2 = aux0[r] * log2 e,
 * row_inv_sum = 1; SMAX_SSUM mode: row_max_log2 = aux0[r] * scale * log2 e,
 * row_inv_sum = 1 / aux1[r] (0 when aux1[r] == 0).  softmax_scale is taken
 * as given (no default substitution), as in the reference.
 * Returns UNSUPPORTED for unsupported shape/dtype/layout/aux mode and
 * INVALID_VALUE for a missing pointer. */
int shaobo_fa3_bwd_dot_do_o(const void* dout,
                            const void* out,
                            const void* softmax_aux0,
                            const void* softmax_aux1,
                            void* delta,
                            void* packed_sidecar,
                            const ShaoboFa3Params* params);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SHAOBO_FA3_COMPONENTS_H_ */
