/*
 * shaobo_fa3_api.h -- public C ABI of the MI355X (gfx950) FlashAttention-3
 * backward library `libshaobo_fa3_bwd.so`.
 *
 * Drop-in boundary: every declaration below keeps the name, argument order,
 * argument meaning, enum values and struct byte layout of the reference ABI
 * (reference: include/shaobo_fa3_api.h:11-147), so a caller built against the
 * reference header links against this library unchanged.  Field offsets are
 * pinned with static_assert in flash-attention3_amd/csrc/fa3_bwd_api.cpp.
 *
 * Tensor convention (all device pointers, contiguous BHSD):
 *   q, out, dout, dq : fp16 [batch, num_heads_q,  seqlen, head_dim]
 *   k, v, dk, dv     : fp16 [batch, num_heads_kv, seqlen, head_dim]
 *   softmax_lse      : fp32 [batch, num_heads_q, seqlen], natural log of
 *                      sum_j exp(softmax_scale * q.k_j)  (Tri Dao convention)
 *   softmax_d        : fp32 [batch, num_heads_q, seqlen] = rowsum(dout * out)
 * The library allocates nothing: the caller owns every buffer including the
 * workspace sized by shaobo_fa3_bwd_v2_workspace_bytes().  All launches go to
 * the null stream and are asynchronous unless params->sync_after_launch == 1.
 */
#ifndef SHAOBO_FA3_API_H_
#define SHAOBO_FA3_API_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference: include/shaobo_fa3_api.h:11 */
#define SHAOBO_FA3_API_VERSION 2u

/* Status codes (reference: include/shaobo_fa3_api.h:13-19). */
typedef enum ShaoboFa3Status {
    SHAOBO_FA3_STATUS_SUCCESS = 0,
    SHAOBO_FA3_STATUS_INVALID_VALUE = 1,
    SHAOBO_FA3_STATUS_UNSUPPORTED = 2,
    SHAOBO_FA3_STATUS_NOT_IMPLEMENTED = 3,
    SHAOBO_FA3_STATUS_HIP_ERROR = 4
} ShaoboFa3Status;

/* Element types (reference: include/shaobo_fa3_api.h:21-25). */
typedef enum ShaoboFa3DType {
    SHAOBO_FA3_DTYPE_FP16 = 0,
    SHAOBO_FA3_DTYPE_BF16 = 1,
    SHAOBO_FA3_DTYPE_FP8 = 2
} ShaoboFa3DType;

/* Tensor layouts (reference: include/shaobo_fa3_api.h:27-30). */
typedef enum ShaoboFa3Layout {
    SHAOBO_FA3_LAYOUT_BHSD = 0,
    SHAOBO_FA3_LAYOUT_BSHD = 1
} ShaoboFa3Layout;

/* Softmax auxiliary input convention (reference: include/shaobo_fa3_api.h:32-35).
 * SMAX_SSUM: aux0 = raw row max of q.k (unscaled), aux1 = row sum of
 *            exp2((s - max) * scale * log2 e).  LSE: aux0 = natural-log LSE. */
typedef enum ShaoboFa3SoftmaxAuxMode {
    SHAOBO_FA3_SOFTMAX_AUX_SMAX_SSUM = 0,
    SHAOBO_FA3_SOFTMAX_AUX_LSE = 1
} ShaoboFa3SoftmaxAuxMode;

/* Capability feature bits (reference: include/shaobo_fa3_api.h:37-51). */
typedef uint64_t ShaoboFa3BwdFeatureMask;

#define SHAOBO_FA3_BWD_FEATURE_FIXED_LENGTH (UINT64_C(1) << 0)
#define SHAOBO_FA3_BWD_FEATURE_VARLEN (UINT64_C(1) << 1)
#define SHAOBO_FA3_BWD_FEATURE_FP16 (UINT64_C(1) << 2)
#define SHAOBO_FA3_BWD_FEATURE_BF16 (UINT64_C(1) << 3)
#define SHAOBO_FA3_BWD_FEATURE_CAUSAL (UINT64_C(1) << 4)
#define SHAOBO_FA3_BWD_FEATURE_LOCAL_WINDOW (UINT64_C(1) << 5)
#define SHAOBO_FA3_BWD_FEATURE_GQA (UINT64_C(1) << 6)
#define SHAOBO_FA3_BWD_FEATURE_SOFTCAP (UINT64_C(1) << 7)
#define SHAOBO_FA3_BWD_FEATURE_DETERMINISTIC (UINT64_C(1) << 8)
#define SHAOBO_FA3_BWD_FEATURE_SOFTMAX_LSE (UINT64_C(1) << 9)
#define SHAOBO_FA3_BWD_FEATURE_BSHD (UINT64_C(1) << 10)
#define SHAOBO_FA3_BWD_FEATURE_BHSD (UINT64_C(1) << 11)
#define SHAOBO_FA3_BWD_FEATURE_FULL_ATTENTION (UINT64_C(1) << 12)

/* Backward launch parameters.  Versioned by struct_size; field order and
 * types are the reference's (include/shaobo_fa3_api.h:53-99), sizeof == 296
 * on x86-64 SysV.  Always start from shaobo_fa3_params_init(). */
typedef struct ShaoboFa3Params {
    uint32_t struct_size;

    int32_t batch;
    int32_t seqlen_q;
    int32_t seqlen_k;
    int32_t num_heads_q;
    int32_t num_heads_kv;
    int32_t head_dim_qk;
    int32_t head_dim_v;

    int32_t causal;            /* 0 or 1; causal = bottom-right aligned, Sq == Sk */
    int32_t window_left;       /* -1 = unbounded */
    int32_t window_right;      /* -1 = unbounded */
    float softmax_scale;       /* used when softmax_scale_is_set == 1 */
    float dropout_p;           /* must be 0 */

    int32_t dtype;             /* ShaoboFa3DType */
    int32_t layout;            /* ShaoboFa3Layout */
    int32_t softmax_aux_mode;  /* ShaoboFa3SoftmaxAuxMode */
    int32_t dkv_path;          /* legacy component selector, ignored by v2 */
    int32_t dq_path;           /* legacy component selector, ignored by v2 */
    int32_t block_threads;     /* legacy, ignored */
    int32_t sync_after_launch; /* 1: hipDeviceSynchronize before returning */

    const int32_t* cu_seqlens_q; /* varlen: must be NULL */
    const int32_t* cu_seqlens_k; /* varlen: must be NULL */
    int32_t max_seqlen_q;        /* 0 or seqlen_q */
    int32_t max_seqlen_k;        /* 0 or seqlen_k */

    void* workspace;             /* caller-owned device scratch */
    size_t workspace_bytes;

    int32_t reserved_i32[16];
    void* reserved_ptr[8];

    /* Tri Dao FA3 backward tail (appended; older callers are told apart by
     * struct_size). */
    const int32_t* seqused_q;    /* must be NULL */
    const int32_t* seqused_k;    /* must be NULL */
    int64_t total_q;             /* 0 or batch * seqlen_q */
    int64_t total_k;             /* 0 or batch * seqlen_k */
    float softcap;               /* must be 0 */
    int32_t deterministic;       /* 0 or 1 */
    int32_t sm_margin;           /* must be 0 */
    int32_t softmax_scale_is_set;/* 0: scale = 1/sqrt(head_dim_qk) */
} ShaoboFa3Params;

/* Capability report (reference: include/shaobo_fa3_api.h:101-109). */
typedef struct ShaoboFa3BwdCapabilities {
    uint32_t struct_size;
    uint32_t api_version;
    ShaoboFa3BwdFeatureMask feature_mask;
    int32_t min_head_dim;
    int32_t max_head_dim;
    int32_t head_dim_alignment;
    int32_t sequence_alignment;
} ShaoboFa3BwdCapabilities;

/* Zero the struct, then set struct_size, window -1/-1, FP16, BHSD, LSE.
 * Replaces reference src/shaobo_fa3_bwd_api.cpp:160-171. */
void shaobo_fa3_params_init(ShaoboFa3Params* params);

/* Fill *capabilities (caller sets struct_size first).  Returns
 * INVALID_VALUE on NULL or a short struct.
 * Replaces reference src/shaobo_fa3_bwd_api.cpp:173-193. */
int shaobo_fa3_bwd_get_capabilities(ShaoboFa3BwdCapabilities* capabilities);

/* Check params only (no pointers, no launch): SUCCESS, INVALID_VALUE or
 * UNSUPPORTED.  Replaces reference src/shaobo_fa3_bwd_api.cpp:195-198. */
int shaobo_fa3_bwd_v2_validate(const ShaoboFa3Params* params);

/* Device workspace the v2 entry needs; 0 when params are invalid or
 * unsupported.  Replaces reference src/shaobo_fa3_bwd_api.cpp:200-204. */
size_t shaobo_fa3_bwd_v2_workspace_bytes(const ShaoboFa3Params* params);

/* Tri Dao FA3-style backward.  softmax_lse is the natural-log LSE from the
 * forward pass.  softmax_d is optional (NULL: kept in the workspace) and
 * receives rowsum(dout * out) in fp32.  dq, dk, dv are fully overwritten.
 * Replaces reference src/shaobo_fa3_bwd_api.cpp:206-260. */
int shaobo_fa3_bwd_v2(const void* dout,
                      const void* q,
                      const void* k,
                      const void* v,
                      const void* out,
                      const void* softmax_lse,
                      void* dq,
                      void* dk,
                      void* dv,
                      void* softmax_d,
                      const ShaoboFa3Params* params);

/* Static string for a status code ("success", "invalid_value", ...).
 * Declared by the reference at include/shaobo_fa3_api.h:133. */
const char* shaobo_fa3_status_string(int status);

/* Legacy two-auxiliary entry (reference include/shaobo_fa3_api.h:135-147).
 * softmax_aux_mode selects SMAX_SSUM (aux0 = raw max, aux1 = sum) or LSE
 * (aux0 = natural LSE, aux1 unused).  Same outputs as v2 (fp16 dq/dk/dv). */
size_t shaobo_fa3_bwd_workspace_bytes(const ShaoboFa3Params* params);

int shaobo_fa3_bwd(const void* dout,
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

#endif  /* SHAOBO_FA3_API_H_ */
