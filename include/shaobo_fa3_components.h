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

/* Fused backward from the packed sidecar (reference
 * include/shaobo_fa3_components.h:47-58, src/fused_bwd_kernel.cpp:1673-1764):
 * P = exp2(s * scale * log2 e - max_log2) * inv_sum, dS = P (dP - delta);
 * dq, dk, dv fp16 BHSD.  softmax_scale is taken as given.  Accepts fp16 BHSD,
 * Dqk == Dv in {64, 128}, causal 0/1, Sq == Sk with Sq % 128 == 0, Hq a
 * multiple of Hkv (UNSUPPORTED otherwise); INVALID_VALUE for a null pointer
 * or a workspace shorter than shaobo_fa3_bwd_fused5_workspace_bytes()
 * (0 for an unsupported shape). */
size_t shaobo_fa3_bwd_fused5_workspace_bytes(const ShaoboFa3Params* params);

int shaobo_fa3_bwd_fused5(const void* dout,
                          const void* q,
                          const void* k,
                          const void* v,
                          const void* packed_sidecar,
                          void* dq,
                          void* dk,
                          void* dv,
                          const ShaoboFa3Params* params);

/* dK / dV only (reference include/shaobo_fa3_components.h:10-22,
 * src/dkv_kernel.cpp:1288-1421); dk, dv written as fp32 [B, H, S, D].
 *   dkv_path 5 (canonical): the packed sidecar of shaobo_fa3_bwd_dot_do_o in
 *     params->reserved_ptr[3]; out, aux0, aux1 and dq unused.  One query head
 *     per KV head, causal, Sq == Sk, Sq % 128 == 0, fp16 BHSD, D in {64, 128}.
 *     No workspace: the workspace-bytes query returns 0.
 *   dkv_path 1 (naive correctness path): recomputes the forward softmax and
 *     delta from Q, K, V, dO in fp32 (out, aux0, aux1, dq unused) through a
 *     workspace of (2 B H S^2 + 3 B H S) floats, which the workspace-bytes
 *     query returns.  One query head per KV head, Sq == Sk (any length),
 *     either causal flag, fp16 BHSD, no dropout, D in {64, 128}.
 * Other shapes and other dkv_path values are UNSUPPORTED. */
size_t shaobo_fa3_bwd_dkv_workspace_bytes(const ShaoboFa3Params* params);

int shaobo_fa3_bwd_dkv(const void* dout,
                       const void* q,
                       const void* k,
                       const void* v,
                       const void* out,
                       const void* softmax_aux0,
                       const void* softmax_aux1,
                       void* dq,
                       void* dk,
                       void* dv,
                       const ShaoboFa3Params* params);

/* dQ only (reference include/shaobo_fa3_components.h:24-36,
 * src/dq_kernel.cpp:1486-1625); dq written as fp32 [B, Hq, S, D]; out, dk,
 * dv unused.
 *   dq_path 6 (canonical): aux0 = raw row max, aux1 = row sum (SMAX_SSUM
 *     convention), delta in params->reserved_ptr[0]; shapes as for
 *     shaobo_fa3_bwd_dkv's canonical path; no workspace.
 *   dq_path 1 (naive correctness path): as dkv_path 1 (aux0 / aux1 unused),
 *     with the same workspace size.
 * Other shapes and other dq_path values are UNSUPPORTED. */
size_t shaobo_fa3_bwd_dq_workspace_bytes(const ShaoboFa3Params* params);

int shaobo_fa3_bwd_dq(const void* dout,
                      const void* q,
                      const void* k,
                      const void* v,
                      const void* out,
                      const void* softmax_aux0,
                      const void* softmax_aux1,
                      void* dq,
                      void* dk,
                      void* dv,
                      const ShaoboFa3Params* params);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SHAOBO_FA3_COMPONENTS_H_ */
