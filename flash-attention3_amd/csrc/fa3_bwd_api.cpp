// C ABI of libshaobo_fa3_bwd.so: parameter validation, capability report,
// workspace sizing and the v2 / legacy / component entry points.
//
// Behavioural contract (reference src/shaobo_fa3_bwd_api.cpp):
//   * validate before any dispatch; INVALID_VALUE for malformed input,
//     UNSUPPORTED for well-formed requests outside the capability set
//     (:70-120), null tensors / short workspace -> INVALID_VALUE (:221-231);
//   * default scale 1/sqrt(head_dim_qk) when softmax_scale_is_set == 0
//     (:241-243); softmax_d optional (:234-236);
//   * all work on the null stream, asynchronous unless sync_after_launch
//     (:254-259); HIP launch failures -> HIP_ERROR.
// Extension over the reference: head_dim 64 is accepted besides 128.
#include "shaobo_fa3_api.h"
#include "shaobo_fa3_components.h"
#include "shaobo_fa3_ext.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstring>
#include <limits>

#include "fa3_bwd_internal.h"

namespace fa3 {
hipError_t launch_device(hipStream_t stream, int* dev) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    hipDevice_t sd = -1;
    if (stream != nullptr) {
        e = hipStreamGetDevice(stream, &sd);
        if (e != hipSuccess) return e;
    }
    const int d = launch_device_of(cur, stream != nullptr, (int)sd);
    if (d < 0) return hipErrorInvalidDevice;
    *dev = d;
    return hipSuccess;
}
}  // namespace fa3

// The struct layout is part of the ABI: pin it (reference header order,
// x86-64 SysV offsets).
static_assert(offsetof(ShaoboFa3Params, struct_size) == 0, "abi");
static_assert(offsetof(ShaoboFa3Params, batch) == 4, "abi");
static_assert(offsetof(ShaoboFa3Params, causal) == 32, "abi");
static_assert(offsetof(ShaoboFa3Params, softmax_scale) == 44, "abi");
static_assert(offsetof(ShaoboFa3Params, dtype) == 52, "abi");
static_assert(offsetof(ShaoboFa3Params, sync_after_launch) == 76, "abi");
static_assert(offsetof(ShaoboFa3Params, cu_seqlens_q) == 80, "abi");
static_assert(offsetof(ShaoboFa3Params, cu_seqlens_k) == 88, "abi");
static_assert(offsetof(ShaoboFa3Params, max_seqlen_q) == 96, "abi");
static_assert(offsetof(ShaoboFa3Params, workspace) == 104, "abi");
static_assert(offsetof(ShaoboFa3Params, workspace_bytes) == 112, "abi");
static_assert(offsetof(ShaoboFa3Params, reserved_i32) == 120, "abi");
static_assert(offsetof(ShaoboFa3Params, reserved_ptr) == 184, "abi");
static_assert(offsetof(ShaoboFa3Params, seqused_q) == 248, "abi");
static_assert(offsetof(ShaoboFa3Params, total_q) == 264, "abi");
static_assert(offsetof(ShaoboFa3Params, softcap) == 280, "abi");
static_assert(offsetof(ShaoboFa3Params, deterministic) == 284, "abi");
static_assert(offsetof(ShaoboFa3Params, sm_margin) == 288, "abi");
static_assert(offsetof(ShaoboFa3Params, softmax_scale_is_set) == 292, "abi");
static_assert(sizeof(ShaoboFa3Params) == 296, "abi");
static_assert(sizeof(ShaoboFa3BwdCapabilities) == 32, "abi");

namespace {

constexpr int kSequenceAlignment = 128;
constexpr int kMinHeadDim = 64;
constexpr int kMaxHeadDim = 128;

bool is_flag(int32_t v) { return v == 0 || v == 1; }

// Causal forces window_right = 0; windows at least as long as the sequence
// are the same as unbounded (reference :53-68).
bool window_is_full(const ShaoboFa3Params* p) {
    int left = p->window_left >= p->seqlen_k - 1 ? -1 : p->window_left;
    int right = p->window_right >= p->seqlen_q - 1 ? -1 : p->window_right;
    if (p->causal) right = 0;
    return left < 0 && (p->causal ? right == 0 : right < 0);
}

bool head_dim_supported(int d) { return d == 64 || d == 128; }

int validate(const ShaoboFa3Params* p) {
    if (p == nullptr || p->struct_size < sizeof(ShaoboFa3Params)) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    const bool dims_ok = p->batch > 0 && p->seqlen_q > 0 && p->seqlen_k > 0 &&
                         p->num_heads_q > 0 && p->num_heads_kv > 0 &&
                         p->num_heads_q % p->num_heads_kv == 0;
    const bool flags_ok = is_flag(p->causal) && is_flag(p->deterministic) &&
                          is_flag(p->sync_after_launch) && is_flag(p->softmax_scale_is_set);
    const bool scale_ok = p->softmax_scale_is_set == 0 ||
                          (std::isfinite(p->softmax_scale) && p->softmax_scale >= 0.0f);
    const bool softcap_ok = std::isfinite(p->softcap) && p->softcap >= 0.0f;
    const bool dropout_ok = std::isfinite(p->dropout_p) && p->dropout_p >= 0.0f &&
                            p->dropout_p < 1.0f;
    if (!dims_ok || !flags_ok || !scale_ok || !softcap_ok || !dropout_ok) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }

    const int64_t total_q = (int64_t)p->batch * p->seqlen_q;
    const int64_t total_k = (int64_t)p->batch * p->seqlen_k;
    const bool fixed_length =
        p->cu_seqlens_q == nullptr && p->cu_seqlens_k == nullptr && p->seqused_q == nullptr &&
        p->seqused_k == nullptr && (p->max_seqlen_q == 0 || p->max_seqlen_q == p->seqlen_q) &&
        (p->max_seqlen_k == 0 || p->max_seqlen_k == p->seqlen_k) &&
        (p->total_q == 0 || p->total_q == total_q) && (p->total_k == 0 || p->total_k == total_k);
    // Extensions over the reference: bf16 and BSHD (its capability bits
    // exist, its kernels reject them), head_dim 64.
    const bool dtype_ok = p->dtype == SHAOBO_FA3_DTYPE_FP16 || p->dtype == SHAOBO_FA3_DTYPE_BF16;
    const bool layout_ok =
        p->layout == SHAOBO_FA3_LAYOUT_BHSD || p->layout == SHAOBO_FA3_LAYOUT_BSHD;
    if (!fixed_length || !dtype_ok || !layout_ok || !head_dim_supported(p->head_dim_qk) ||
        p->head_dim_v != p->head_dim_qk || p->seqlen_q != p->seqlen_k ||
        p->seqlen_q % kSequenceAlignment != 0 || p->dropout_p != 0.0f || p->softcap != 0.0f ||
        p->sm_margin != 0 || !window_is_full(p)) {
        return SHAOBO_FA3_STATUS_UNSUPPORTED;
    }
    return SHAOBO_FA3_STATUS_SUCCESS;
}

fa3::BwdProblem problem_of(const ShaoboFa3Params* p) {
    fa3::BwdProblem pr;
    pr.batch = p->batch;
    pr.seqlen = p->seqlen_q;
    pr.heads_q = p->num_heads_q;
    pr.heads_kv = p->num_heads_kv;
    pr.head_dim = p->head_dim_qk;
    pr.causal = p->causal != 0;
    pr.deterministic = p->deterministic != 0;
    pr.bf16 = p->dtype == SHAOBO_FA3_DTYPE_BF16;
    pr.bshd = p->layout == SHAOBO_FA3_LAYOUT_BSHD;
    pr.scale = p->softmax_scale_is_set ? p->softmax_scale
                                       : 1.0f / std::sqrt((float)p->head_dim_qk);
    return pr;
}

// sync_after_launch: the whole device for the null stream (reference
// behaviour), the caller's stream otherwise.  When the launch used the split
// plan, the synchronised call also reads the workspace's error word: a split
// wait that gave up wrote the launch's epoch there, and the call reports a
// HIP error instead of returning wrong gradients as success.  On a caller's
// stream the word is read by a copy queued on that stream, so the one
// stream synchronisation covers it (no other stream is waited for).
int finish(hipError_t err, const ShaoboFa3Params* p, hipStream_t stream = nullptr,
           const void* err_word = nullptr, unsigned long long epoch = 0) {
    if (err != hipSuccess) return SHAOBO_FA3_STATUS_HIP_ERROR;
    if (!p->sync_after_launch) return SHAOBO_FA3_STATUS_SUCCESS;
    unsigned long long word = 0;
    if (stream == nullptr) {
        if (hipDeviceSynchronize() != hipSuccess) return SHAOBO_FA3_STATUS_HIP_ERROR;
        if (err_word != nullptr &&
            hipMemcpy(&word, err_word, sizeof(word), hipMemcpyDeviceToHost) != hipSuccess) {
            return SHAOBO_FA3_STATUS_HIP_ERROR;
        }
    } else {
        if (err_word != nullptr && hipMemcpyAsync(&word, err_word, sizeof(word),
                                                  hipMemcpyDeviceToHost, stream) != hipSuccess) {
            return SHAOBO_FA3_STATUS_HIP_ERROR;
        }
        if (hipStreamSynchronize(stream) != hipSuccess) return SHAOBO_FA3_STATUS_HIP_ERROR;
    }
    if (err_word != nullptr && word == epoch) return SHAOBO_FA3_STATUS_HIP_ERROR;
    return SHAOBO_FA3_STATUS_SUCCESS;
}

// Device of the launches on `stream`: SUCCESS, INVALID_VALUE for a stream
// of another device than the current one (the library's per-device arrays
// are looked up with the launch device current), HIP_ERROR when the runtime
// fails.
int resolve_device(hipStream_t stream, int* dev) {
    const hipError_t e = fa3::launch_device(stream, dev);
    if (e == hipErrorInvalidDevice) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    return e == hipSuccess ? SHAOBO_FA3_STATUS_SUCCESS : SHAOBO_FA3_STATUS_HIP_ERROR;
}

// Options of the extension entries: the launch stream; no_alloc: the
// library's static scratch array instead of the caller's workspace, whose
// fields are then ignored; events: three hipEvent_t recorded around the two
// kernels (or null); stages: which of the two kernels to launch (bit 0 the
// preprocess, bit 1 the main kernel).
struct RunOpts {
    hipStream_t stream = nullptr;
    bool no_alloc = false;
    void* const* events = nullptr;
    int stages = 3;
};

// Shared body of v2, the legacy entry and the extension entries.
int run_backward(const void* dout, const void* q, const void* k, const void* v, const void* out,
                 const void* aux0, const void* aux1, bool aux_is_lse, void* dq, void* dk,
                 void* dv, void* softmax_d, const ShaoboFa3Params* params,
                 const RunOpts& opt = RunOpts{}) {
    const hipStream_t stream = opt.stream;
    const int status = validate(params);
    if (status != SHAOBO_FA3_STATUS_SUCCESS) return status;
    if (dout == nullptr || q == nullptr || k == nullptr || v == nullptr || out == nullptr ||
        aux0 == nullptr || (!aux_is_lse && aux1 == nullptr) || dq == nullptr || dk == nullptr ||
        dv == nullptr) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    fa3::BwdProblem pr = problem_of(params);
    fa3::WorkspacePlan plan = fa3::plan_workspace(pr);
    void* workspace = params->workspace;
    if (opt.no_alloc) {
        // the head-split plan's per-query-head dK / dV need not fit the
        // scratch array: then the plan with one dKV job per KV head
        if (plan.ok && plan.hs_chunks > 0 && plan.total > fa3::kNoAllocScratchBytes) {
            pr.no_head_split = true;
            plan = fa3::plan_workspace(pr);
        }
        // shapes whose workspace exceeds the scratch array are refused
        // before any HIP call
        if (!plan.ok || plan.total > fa3::kNoAllocScratchBytes) {
            return SHAOBO_FA3_STATUS_INVALID_VALUE;
        }
    } else if (!plan.ok || workspace == nullptr || params->workspace_bytes < plan.total) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    int device = -1;
    const int dev_status = resolve_device(stream, &device);
    if (dev_status != SHAOBO_FA3_STATUS_SUCCESS) return dev_status;
    if (opt.no_alloc && fa3::noalloc_scratch(device, &workspace) != hipSuccess) {
        return SHAOBO_FA3_STATUS_HIP_ERROR;
    }
    fa3::BwdTensors t;
    t.device = device;
    t.dout = dout;
    t.q = q;
    t.k = k;
    t.v = v;
    t.out = out;
    t.aux0 = static_cast<const float*>(aux0);
    t.aux1 = static_cast<const float*>(aux1);
    t.aux_is_lse = aux_is_lse;
    t.dq = dq;
    t.dk = dk;
    t.dv = dv;
    t.delta = static_cast<float*>(softmax_d);
    t.stream = stream;
    if (opt.events != nullptr) {
        for (int i = 0; i < 3; ++i) t.events[i] = static_cast<hipEvent_t>(opt.events[i]);
    }
    t.stages = opt.stages;
    unsigned long long epoch = 0;
    const hipError_t err = fa3::launch_backward(pr, t, workspace, &epoch);
    const char* ws = static_cast<const char*>(workspace);
    // the error word belongs to the main kernel's split waits
    const bool split = plan.bal_m > 0 && (opt.stages & 2);
    return finish(err, params, stream, split ? ws + plan.err_off : nullptr, epoch);
}

// Workspace of v2 and of the legacy entry (the same whatever the aux mode).
size_t workspace_bytes_of(const ShaoboFa3Params* params) {
    if (validate(params) != SHAOBO_FA3_STATUS_SUCCESS) return 0;
    const fa3::WorkspacePlan plan = fa3::plan_workspace(problem_of(params));
    return plan.ok ? plan.total : 0;
}

// ---- component entries ----
// Reference path ids (include/dkv_contract.h:7-8, include/dq_contract.h:7-8).
constexpr int kDkvPathCanonical = 5;
constexpr int kDqPathCanonical = 6;
constexpr int kPathReferenceCorrectness = 1;  // naive path of both components

// Shape / dtype / layout acceptance shared by the dKV and dQ components
// (reference valid_dkv_shape / valid_dq_shape, src/dkv_kernel.cpp:50-57,
// src/dq_kernel.cpp:63-70) and their canonical paths (:59-67, :81-89):
// one query head per KV head, causal, Sq == Sk, whole 128-row tiles.
bool component_shape_ok(const ShaoboFa3Params* p) {
    return p->batch > 0 && p->seqlen_q > 0 && p->seqlen_k > 0 && p->num_heads_q > 0 &&
           head_dim_supported(p->head_dim_qk) && p->head_dim_v == p->head_dim_qk &&
           p->dtype == SHAOBO_FA3_DTYPE_FP16 && p->layout == SHAOBO_FA3_LAYOUT_BHSD &&
           p->seqlen_k == p->seqlen_q && p->seqlen_q % kSequenceAlignment == 0 &&
           p->num_heads_kv == p->num_heads_q && p->causal == 1;
}

// Acceptance of the naive path 1 (reference valid_reference_shape,
// src/dkv_kernel.cpp:69-75, src/dq_kernel.cpp:72-78): fp16 BHSD, Sq == Sk,
// one query head per KV head, no dropout; any sequence length and causal
// flag.  The reference builds D = 128 only; D = 64 is accepted here too.
bool naive_shape_ok(const ShaoboFa3Params* p) {
    return p->batch > 0 && p->seqlen_q > 0 && p->seqlen_k > 0 && p->num_heads_q > 0 &&
           head_dim_supported(p->head_dim_qk) && p->head_dim_v == p->head_dim_qk &&
           p->dtype == SHAOBO_FA3_DTYPE_FP16 && p->layout == SHAOBO_FA3_LAYOUT_BHSD &&
           p->seqlen_k == p->seqlen_q && p->num_heads_kv == p->num_heads_q &&
           p->dropout_p == 0.0f;
}

// Workspace of path 1 (reference reference_workspace_bytes,
// src/dkv_kernel.cpp:77-86): (2 B H S^2 + 3 B H S) fp32; 0 for other shapes.
size_t naive_workspace(const ShaoboFa3Params* p) {
    if (!naive_shape_ok(p)) return 0;
    fa3::BwdProblem pr;
    pr.batch = p->batch;
    pr.seqlen = p->seqlen_q;
    pr.heads_q = p->num_heads_q;
    pr.heads_kv = p->num_heads_kv;
    pr.head_dim = p->head_dim_qk;
    return fa3::naive_workspace_bytes(pr);
}

// Path 1 of either component (reference src/dkv_kernel.cpp:1320-1372,
// src/dq_kernel.cpp:1562-1625): role 1 writes fp32 dK / dV, role 2 fp32 dQ.
int run_naive(const void* dout, const void* q, const void* k, const void* v, void* dq,
              void* dk, void* dv, const ShaoboFa3Params* params, int role) {
    if (!naive_shape_ok(params)) return SHAOBO_FA3_STATUS_UNSUPPORTED;
    const bool outs = role == 1 ? (dk != nullptr && dv != nullptr) : dq != nullptr;
    if (dout == nullptr || q == nullptr || k == nullptr || v == nullptr || !outs ||
        params->workspace == nullptr) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    const size_t need = naive_workspace(params);
    if (need == 0 || params->workspace_bytes < need) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    fa3::BwdProblem pr;
    pr.batch = params->batch;
    pr.seqlen = params->seqlen_q;
    pr.heads_q = params->num_heads_q;
    pr.heads_kv = params->num_heads_kv;
    pr.head_dim = params->head_dim_qk;
    pr.causal = params->causal != 0;
    pr.scale = params->softmax_scale;
    fa3::BwdTensors t;
    t.dout = dout;
    t.q = q;
    t.k = k;
    t.v = v;
    t.dq = dq;
    t.dk = dk;
    t.dv = dv;
    return finish(fa3::launch_naive(pr, t, params->workspace, role), params);
}

// fused5 acceptance (reference src/fused_bwd_kernel.cpp:1682-1693): fp16 BHSD,
// Dqk == Dv (64 or 128 here; the reference builds D = 128 only), causal flag,
// Sq == Sk in whole 128-row tiles, Hq a multiple of Hkv.
bool fused5_shape_ok(const ShaoboFa3Params* p) {
    return p->batch > 0 && p->seqlen_q > 0 && p->num_heads_q > 0 &&
           p->dtype == SHAOBO_FA3_DTYPE_FP16 && p->layout == SHAOBO_FA3_LAYOUT_BHSD &&
           head_dim_supported(p->head_dim_qk) && p->head_dim_v == p->head_dim_qk &&
           is_flag(p->causal) && p->seqlen_q == p->seqlen_k &&
           p->seqlen_q % kSequenceAlignment == 0 && p->num_heads_kv > 0 &&
           p->num_heads_q % p->num_heads_kv == 0;
}

// Problem of a component entry: the scale is taken as given (the reference
// components do not substitute the default).
fa3::BwdProblem component_problem(const ShaoboFa3Params* p, bool out_f32) {
    fa3::BwdProblem pr;
    pr.batch = p->batch;
    pr.seqlen = p->seqlen_q;
    pr.heads_q = p->num_heads_q;
    pr.heads_kv = p->num_heads_kv;
    pr.head_dim = p->head_dim_qk;
    pr.causal = p->causal != 0;
    pr.deterministic = true;
    pr.scale = p->softmax_scale;
    pr.out_f32 = out_f32;
    return pr;
}

// fused5: rows from the packed sidecar
size_t component_workspace(const fa3::BwdProblem& pr) {
    const fa3::WorkspacePlan plan = fa3::plan_workspace(pr);
    return plan.ok ? plan.total : 0;
}

}  // namespace

extern "C" {

void shaobo_fa3_params_init(ShaoboFa3Params* params) {
    if (params == nullptr) return;
    std::memset(params, 0, sizeof(*params));
    params->struct_size = sizeof(*params);
    params->window_left = -1;
    params->window_right = -1;
    params->dtype = SHAOBO_FA3_DTYPE_FP16;
    params->layout = SHAOBO_FA3_LAYOUT_BHSD;
    params->softmax_aux_mode = SHAOBO_FA3_SOFTMAX_AUX_LSE;
}

int shaobo_fa3_bwd_get_capabilities(ShaoboFa3BwdCapabilities* caps) {
    if (caps == nullptr || caps->struct_size < sizeof(ShaoboFa3BwdCapabilities)) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    caps->api_version = SHAOBO_FA3_API_VERSION;
    caps->feature_mask = SHAOBO_FA3_BWD_FEATURE_FIXED_LENGTH | SHAOBO_FA3_BWD_FEATURE_FP16 |
                         SHAOBO_FA3_BWD_FEATURE_BF16 | SHAOBO_FA3_BWD_FEATURE_CAUSAL |
                         SHAOBO_FA3_BWD_FEATURE_GQA | SHAOBO_FA3_BWD_FEATURE_DETERMINISTIC |
                         SHAOBO_FA3_BWD_FEATURE_SOFTMAX_LSE | SHAOBO_FA3_BWD_FEATURE_BSHD |
                         SHAOBO_FA3_BWD_FEATURE_BHSD | SHAOBO_FA3_BWD_FEATURE_FULL_ATTENTION;
    caps->min_head_dim = kMinHeadDim;
    caps->max_head_dim = kMaxHeadDim;
    caps->head_dim_alignment = kMinHeadDim;
    caps->sequence_alignment = kSequenceAlignment;
    return SHAOBO_FA3_STATUS_SUCCESS;
}

int shaobo_fa3_bwd_v2_validate(const ShaoboFa3Params* params) { return validate(params); }

size_t shaobo_fa3_bwd_v2_workspace_bytes(const ShaoboFa3Params* params) {
    return workspace_bytes_of(params);
}

int shaobo_fa3_bwd_v2(const void* dout, const void* q, const void* k, const void* v,
                      const void* out, const void* softmax_lse, void* dq, void* dk, void* dv,
                      void* softmax_d, const ShaoboFa3Params* params) {
    return run_backward(dout, q, k, v, out, softmax_lse, nullptr, true, dq, dk, dv, softmax_d,
                        params);
}

int shaobo_fa3_bwd_v2_on_stream(const void* dout, const void* q, const void* k, const void* v,
                                const void* out, const void* softmax_lse, void* dq, void* dk,
                                void* dv, void* softmax_d, const ShaoboFa3Params* params,
                                void* stream) {
    RunOpts opt;
    opt.stream = static_cast<hipStream_t>(stream);
    return run_backward(dout, q, k, v, out, softmax_lse, nullptr, true, dq, dk, dv, softmax_d,
                        params, opt);
}

void shaobo_fa3_ext_set_split_spin_limit(int polls) { fa3::set_split_spin_limit(polls); }

void shaobo_fa3_ext_set_race_check(int on) { fa3::set_debug_kernels(on != 0); }

int shaobo_fa3_ext_bwd_v2_no_alloc(const void* dout, const void* q, const void* k, const void* v,
                                   const void* out, const void* softmax_lse, void* dq, void* dk,
                                   void* dv, void* softmax_d, const ShaoboFa3Params* params,
                                   void* stream) {
    RunOpts opt;
    opt.stream = static_cast<hipStream_t>(stream);
    opt.no_alloc = true;
    return run_backward(dout, q, k, v, out, softmax_lse, nullptr, true, dq, dk, dv, softmax_d,
                        params, opt);
}

int shaobo_fa3_ext_bwd_v2_timed(const void* dout, const void* q, const void* k, const void* v,
                                const void* out, const void* softmax_lse, void* dq, void* dk,
                                void* dv, void* softmax_d, const ShaoboFa3Params* params,
                                void* stream, void* const* events) {
    RunOpts opt;
    opt.stream = static_cast<hipStream_t>(stream);
    opt.events = events;
    return run_backward(dout, q, k, v, out, softmax_lse, nullptr, true, dq, dk, dv, softmax_d,
                        params, opt);
}

int shaobo_fa3_ext_bwd_v2_stages(const void* dout, const void* q, const void* k, const void* v,
                                 const void* out, const void* softmax_lse, void* dq, void* dk,
                                 void* dv, void* softmax_d, const ShaoboFa3Params* params,
                                 void* stream, int stages) {
    if (stages < 1 || stages > 3) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    RunOpts opt;
    opt.stream = static_cast<hipStream_t>(stream);
    opt.stages = stages;
    return run_backward(dout, q, k, v, out, softmax_lse, nullptr, true, dq, dk, dv, softmax_d,
                        params, opt);
}

int shaobo_fa3_ext_split_status(const void* workspace, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int device = -1;
    const int dev_status = resolve_device(s, &device);
    if (dev_status != SHAOBO_FA3_STATUS_SUCCESS) return dev_status;
    const char* base = static_cast<const char*>(workspace);
    if (base == nullptr) {
        void* p = nullptr;
        if (fa3::noalloc_scratch(device, &p) != hipSuccess) return SHAOBO_FA3_STATUS_HIP_ERROR;
        base = static_cast<const char*>(p);
    }
    void* word_ptr = const_cast<char*>(base + fa3::kErrWordOffset);
    unsigned long long word = 0;
    if (hipMemcpyAsync(&word, word_ptr, sizeof(word), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        return SHAOBO_FA3_STATUS_HIP_ERROR;
    }
    if (!fa3::epoch_issued(word)) return SHAOBO_FA3_STATUS_SUCCESS;
    // reported once: the word goes back to 0 (no launch uses epoch 0)
    if (hipMemsetAsync(word_ptr, 0, sizeof(word), s) != hipSuccess) {
        return SHAOBO_FA3_STATUS_HIP_ERROR;
    }
    (void)hipStreamSynchronize(s);
    return SHAOBO_FA3_STATUS_HIP_ERROR;
}

int shaobo_fa3_ext_split_error_count(void* stream, unsigned long long* count) {
    if (count == nullptr) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int device = -1;
    const int dev_status = resolve_device(s, &device);
    if (dev_status != SHAOBO_FA3_STATUS_SUCCESS) return dev_status;
    unsigned long long* counter = nullptr;
    if (fa3::split_giveup_count(device, &counter) != hipSuccess) {
        return SHAOBO_FA3_STATUS_HIP_ERROR;
    }
    unsigned long long n = 0;
    if (hipMemcpyAsync(&n, counter, sizeof(n), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        return SHAOBO_FA3_STATUS_HIP_ERROR;
    }
    *count = n;
    return SHAOBO_FA3_STATUS_SUCCESS;
}

const char* shaobo_fa3_status_string(int status) {
    switch (status) {
        case SHAOBO_FA3_STATUS_SUCCESS: return "success";
        case SHAOBO_FA3_STATUS_INVALID_VALUE: return "invalid_value";
        case SHAOBO_FA3_STATUS_UNSUPPORTED: return "unsupported";
        case SHAOBO_FA3_STATUS_NOT_IMPLEMENTED: return "not_implemented";
        case SHAOBO_FA3_STATUS_HIP_ERROR: return "hip_error";
        default: return "unknown";
    }
}

size_t shaobo_fa3_bwd_workspace_bytes(const ShaoboFa3Params* params) {
    if (params == nullptr) return 0;
    return workspace_bytes_of(params);
}

int shaobo_fa3_bwd(const void* dout, const void* q, const void* k, const void* v,
                   const void* out, const void* softmax_aux0, const void* softmax_aux1, void* dq,
                   void* dk, void* dv, const ShaoboFa3Params* params) {
    if (params == nullptr) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    const int mode = params->softmax_aux_mode;
    if (mode != SHAOBO_FA3_SOFTMAX_AUX_LSE && mode != SHAOBO_FA3_SOFTMAX_AUX_SMAX_SSUM) {
        return validate(params) == SHAOBO_FA3_STATUS_SUCCESS ? SHAOBO_FA3_STATUS_UNSUPPORTED
                                                              : validate(params);
    }
    return run_backward(dout, q, k, v, out, softmax_aux0, softmax_aux1,
                        mode == SHAOBO_FA3_SOFTMAX_AUX_LSE, dq, dk, dv, nullptr, params);
}

// ---- component entries (include/shaobo_fa3_components.h) ----

int shaobo_fa3_bwd_dot_do_o(const void* dout, const void* out, const void* softmax_aux0,
                            const void* softmax_aux1, void* delta, void* packed_sidecar,
                            const ShaoboFa3Params* params) {
    // Same acceptance as the reference component (src/dot_do_o_kernel.cpp:65-94):
    // shape/dtype/layout/aux-mode checks only, then pointer checks.
    if (params == nullptr || params->batch <= 0 || params->seqlen_q <= 0 ||
        params->num_heads_q <= 0 || !head_dim_supported(params->head_dim_qk) ||
        params->head_dim_v != params->head_dim_qk || params->dtype != SHAOBO_FA3_DTYPE_FP16 ||
        params->layout != SHAOBO_FA3_LAYOUT_BHSD ||
        (params->softmax_aux_mode != SHAOBO_FA3_SOFTMAX_AUX_SMAX_SSUM &&
         params->softmax_aux_mode != SHAOBO_FA3_SOFTMAX_AUX_LSE)) {
        return SHAOBO_FA3_STATUS_UNSUPPORTED;
    }
    const bool lse = params->softmax_aux_mode == SHAOBO_FA3_SOFTMAX_AUX_LSE;
    if (dout == nullptr || out == nullptr || softmax_aux0 == nullptr ||
        (!lse && softmax_aux1 == nullptr) || delta == nullptr || packed_sidecar == nullptr) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    fa3::BwdProblem pr;
    pr.batch = params->batch;
    pr.seqlen = params->seqlen_q;
    pr.heads_q = params->num_heads_q;
    pr.heads_kv = params->num_heads_q;
    pr.head_dim = params->head_dim_qk;
    pr.scale = params->softmax_scale;
    fa3::BwdTensors t;
    t.dout = dout;
    t.out = out;
    t.aux0 = static_cast<const float*>(softmax_aux0);
    t.aux1 = static_cast<const float*>(softmax_aux1);
    t.aux_is_lse = lse;
    t.delta = static_cast<float*>(delta);
    t.packed = static_cast<float*>(packed_sidecar);
    return finish(fa3::launch_preprocess(pr, t, nullptr, nullptr), params);
}

size_t shaobo_fa3_bwd_fused5_workspace_bytes(const ShaoboFa3Params* params) {
    if (params == nullptr || !fused5_shape_ok(params)) return 0;
    return component_workspace(component_problem(params, false));
}

int shaobo_fa3_bwd_fused5(const void* dout, const void* q, const void* k, const void* v,
                          const void* packed_sidecar, void* dq, void* dk, void* dv,
                          const ShaoboFa3Params* params) {
    if (params == nullptr || dout == nullptr || q == nullptr || k == nullptr || v == nullptr ||
        packed_sidecar == nullptr || dq == nullptr || dk == nullptr || dv == nullptr) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    if (!fused5_shape_ok(params)) return SHAOBO_FA3_STATUS_UNSUPPORTED;
    fa3::BwdTensors t;
    t.dout = dout;
    t.q = q;
    t.k = k;
    t.v = v;
    t.packed_in = static_cast<const float*>(packed_sidecar);
    t.dq = dq;
    t.dk = dk;
    t.dv = dv;
    const fa3::BwdProblem pr = component_problem(params, false);
    const fa3::WorkspacePlan plan = fa3::plan_workspace(pr);
    if (!plan.ok || params->workspace == nullptr || params->workspace_bytes < plan.total) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    const int dev_status = resolve_device(nullptr, &t.device);
    if (dev_status != SHAOBO_FA3_STATUS_SUCCESS) return dev_status;
    unsigned long long epoch = 0;
    const hipError_t err = fa3::launch_backward(pr, t, params->workspace, &epoch);
    const char* ws = static_cast<const char*>(params->workspace);
    return finish(err, params, nullptr, plan.bal_m > 0 ? ws + plan.err_off : nullptr, epoch);
}

size_t shaobo_fa3_bwd_dkv_workspace_bytes(const ShaoboFa3Params* params) {
    // the canonical path reads the sidecar directly and needs none
    if (params == nullptr || params->dkv_path != kPathReferenceCorrectness) return 0;
    return naive_workspace(params);
}

int shaobo_fa3_bwd_dkv(const void* dout, const void* q, const void* k, const void* v,
                       const void* out, const void* softmax_aux0, const void* softmax_aux1,
                       void* dq, void* dk, void* dv, const ShaoboFa3Params* params) {
    (void)out;
    (void)softmax_aux0;
    (void)softmax_aux1;
    (void)dq;
    if (params == nullptr) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    if (params->dkv_path == kPathReferenceCorrectness) {
        return run_naive(dout, q, k, v, nullptr, dk, dv, params, 1);
    }
    if (params->dkv_path != kDkvPathCanonical || !component_shape_ok(params)) {
        return SHAOBO_FA3_STATUS_UNSUPPORTED;
    }
    if (dout == nullptr || q == nullptr || k == nullptr || v == nullptr || dk == nullptr ||
        dv == nullptr || params->reserved_ptr[3] == nullptr) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    fa3::BwdTensors t;
    t.dout = dout;
    t.q = q;
    t.k = k;
    t.v = v;
    t.packed_in = static_cast<const float*>(params->reserved_ptr[3]);
    t.dk = dk;
    t.dv = dv;
    return finish(fa3::launch_component(component_problem(params, true), t, 1), params);
}

size_t shaobo_fa3_bwd_dq_workspace_bytes(const ShaoboFa3Params* params) {
    // the canonical path reads max / sum / delta directly and needs none
    if (params == nullptr || params->dq_path != kPathReferenceCorrectness) return 0;
    return naive_workspace(params);
}

int shaobo_fa3_bwd_dq(const void* dout, const void* q, const void* k, const void* v,
                      const void* out, const void* softmax_aux0, const void* softmax_aux1,
                      void* dq, void* dk, void* dv, const ShaoboFa3Params* params) {
    (void)out;
    (void)dk;
    (void)dv;
    if (params == nullptr) return SHAOBO_FA3_STATUS_INVALID_VALUE;
    if (params->dq_path == kPathReferenceCorrectness) {
        return run_naive(dout, q, k, v, dq, nullptr, nullptr, params, 2);
    }
    if (params->dq_path != kDqPathCanonical || !component_shape_ok(params)) {
        return SHAOBO_FA3_STATUS_UNSUPPORTED;
    }
    if (dout == nullptr || q == nullptr || k == nullptr || v == nullptr ||
        softmax_aux0 == nullptr || softmax_aux1 == nullptr || dq == nullptr ||
        params->reserved_ptr[0] == nullptr) {
        return SHAOBO_FA3_STATUS_INVALID_VALUE;
    }
    fa3::BwdTensors t;
    t.dout = dout;
    t.q = q;
    t.k = k;
    t.v = v;
    t.aux0 = static_cast<const float*>(softmax_aux0);
    t.aux1 = static_cast<const float*>(softmax_aux1);
    t.delta_in = static_cast<const float*>(params->reserved_ptr[0]);
    t.dq = dq;
    return finish(fa3::launch_component(component_problem(params, true), t, 2), params);
}

}  // extern "C"
