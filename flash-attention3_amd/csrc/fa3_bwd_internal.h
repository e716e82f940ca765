// Host-side launch interface between the C ABI layer (fa3_bwd_api.cpp) and
// the HIP kernels.  Nothing here is exported from the shared library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "shaobo_fa3_ext.h"

namespace fa3 {

// Keys owned by one workgroup of the main kernel, and query rows it consumes
// per pipeline step.  The main kernel tiles both sequence axes by 64.
constexpr int kTileN = 64;
constexpr int kTileM = 64;

// Job queues of the persistent main kernel: one counter per XCD (workgroup
// id % 8), each on its own 128-byte line of the workspace, and an exit
// count; zeroed by the preprocess pass that runs before the main kernel
// (and by the main kernel's last workgroup as it leaves).
constexpr int kQueues = 8;
constexpr int kQueueStride = 32;  // 32-bit words between counters
constexpr int kQueueExitWord = 16;  // the launch's exit count, on queue 0's line
constexpr size_t kQueueBytes = (size_t)kQueues * kQueueStride * 4;

// The device that a launch on a stream runs on: the current device, for the
// null stream or a stream of the current device; -1 for a stream of another
// device (the library's per-device arrays -- the no-allocation scratch, the
// give-up count -- are looked up with the current device, so such a launch
// is refused rather than handed another GPU's addresses).
inline int launch_device_of(int current, bool has_stream, int stream_device) {
    return !has_stream || stream_device == current ? current : -1;
}

// Division by a launch-invariant divisor d (1 <= d < 2^31) of 0 <= n < 2^31
// as a multiply-high, an add and a shift (Granlund-Montgomery round-up
// method): with s = ceil(log2 d) and mul = floor(2^32 (2^s - d) / d) + 1,
// n / d = (mulhi(n, mul) + n) >> s.  The host computes mul and s once per
// launch; in the kernels the operands are wave-uniform, so a quotient costs
// three scalar instructions instead of a ~30-instruction division sequence
// that all 8 waves of a workgroup would run on the CU's one scalar unit.
struct FastDiv {
    uint32_t mul = 1;
    uint32_t shr = 0;
    int d = 1;
};

inline FastDiv make_fastdiv(int d) {
    FastDiv f;
    if (d < 1) d = 1;  // unused divisor slot
    f.d = d;
    uint32_t s = 0;
    while (s < 31 && (1u << s) < (uint32_t)d) ++s;
    f.shr = s;
    f.mul = (uint32_t)(((uint64_t)1 << 32) * (((uint64_t)1 << s) - (uint64_t)d) / (uint64_t)d + 1);
    return f;
}

__host__ __device__ inline int fdiv(const FastDiv& f, int n) {
    const uint32_t hi = (uint32_t)(((uint64_t)(uint32_t)n * f.mul) >> 32);
    return (int)((hi + (uint32_t)n) >> f.shr);
}

// Everything a backward launch needs, already validated and resolved
// (default scale applied, aux mode folded into the lse2 preprocessing).
struct BwdProblem {
    int batch = 0;
    int seqlen = 0;     // Sq == Sk
    int heads_q = 0;
    int heads_kv = 0;
    int head_dim = 0;   // Dqk == Dv, 64 or 128
    bool causal = false;
    bool deterministic = false;
    float scale = 0.f;  // softmax scale
    bool out_f32 = false;  // outputs fp32 (component entries) instead of fp16
    bool bf16 = false;     // 16-bit tensors are bf16 (fp16 otherwise)
    bool bshd = false;     // tensors are [B, S, H, D] (BHSD otherwise); rows stay [B, Hq, S]
    bool no_head_split = false;  // GQA: one dKV job per KV head, whatever the shape
};

struct BwdTensors {
    const void* dout = nullptr;
    const void* q = nullptr;
    const void* k = nullptr;
    const void* v = nullptr;
    const void* out = nullptr;
    const float* aux0 = nullptr;   // LSE (natural log) or raw row max
    const float* aux1 = nullptr;   // row sum (SMAX_SSUM mode) or nullptr
    bool aux_is_lse = true;
    void* dq = nullptr;
    void* dk = nullptr;
    void* dv = nullptr;
    float* delta = nullptr;        // fp32 rows (softmax_d); may be null
    float* packed = nullptr;       // optional [rows][3] sidecar
    // Row statistics given instead of computed from O (component entries):
    // a packed [max_log2, inv_sum, delta] sidecar (fused5, dK/dV), or
    // delta_in together with the raw max / sum pair in aux0 / aux1 (dQ).
    const float* packed_in = nullptr;
    const float* delta_in = nullptr;
    // Stream of every launch (null: the legacy default stream, as in the
    // reference ABI; the stream entry points pass the caller's) and its
    // device, which is the current device (launch_device).
    hipStream_t stream = nullptr;
    int device = -1;
    // Optional events recorded on `stream` before the preprocess, before the
    // main kernel and after it (null: not recorded).
    hipEvent_t events[3] = {nullptr, nullptr, nullptr};
    // Kernels to launch: bit 0 the preprocess (or row statistics), bit 1 the
    // main kernel, which then reads what an earlier preprocess of the same
    // workspace left there.
    int stages = 3;
};

// Device workspace of the v2 / legacy / fused5 entries (regions 256-B
// aligned):
//   * the error word (one 64-bit word), set to the launch's epoch by a split
//     wait that gives up;
//   * -lse2 and -delta rows, written by the preprocess pass;
//   * split plan only (bal_m > 0): two 64-bit synchronisation words per
//     split job of each role, and the fp32 partial sums of one piece per
//     split job (dKV jobs, then dQ jobs).
struct WorkspacePlan {
    size_t err_off = 0;
    size_t nlse2_off = 0;
    size_t ndelta_off = 0;
    size_t queue_off = 0;   // kQueueBytes of job-queue counters
    int bal_m = 0;          // > 0: split plan with M = bal_m
    int n_split = 0;        // split jobs per role
    size_t sync_off = 0;
    size_t pkv_off = 0;     // dKV pieces' partial sums
    size_t pq_off = 0;      // dQ pieces' partial sums
    int hs_chunks = 0;        // > 0: head-split default plan (GQA, few groups)
    size_t hsd_off = 0;       // its fp32 dK contributions [B][Hkv hs_chunks][S][D], then dV's
    size_t total = 0;
    bool ok = false;        // false: the sizes overflow size_t / the kernel's offsets
};

WorkspacePlan plan_workspace(const BwdProblem& p);

// Launches the backward on t.stream: the delta / lse2 preprocess (or the
// packed sidecar's fold), then the main kernel.  *epoch receives the value
// the launch's split waits compare with (and write into the error word when
// they give up).
hipError_t launch_backward(const BwdProblem& p, const BwdTensors& t, void* workspace,
                           unsigned long long* epoch);

// Delta preprocess: delta into t.delta, -lse2 and -delta into the given rows;
// any of the three may be null.  Alone, it is the component entry
// shaobo_fa3_bwd_dot_do_o.  queue (optional): the main kernel's job-queue
// counters, zeroed.
hipError_t launch_preprocess(const BwdProblem& p, const BwdTensors& t, float* nlse2,
                             float* ndelta, unsigned int* queue = nullptr);

// -lse2 and -delta rows from the packed sidecar t.packed_in; queue as above.
hipError_t launch_rowstats(const BwdProblem& p, const BwdTensors& t, float* nlse2,
                           float* ndelta, unsigned int* queue = nullptr);

// Workspace-free single-role components (causal, heads_q == heads_kv, fp32
// outputs when p.out_f32): role 1 writes dK / dV from t.packed_in, role 2
// writes dQ from aux0 (raw max), aux1 (sum) and t.delta_in.
hipError_t launch_component(const BwdProblem& p, const BwdTensors& t, int role);

// Naive fp32 correctness path of the dK/dV (role 1) and dQ (role 2)
// components (dkv_path / dq_path 1): fp16 BHSD, one query head per KV head,
// fp32 outputs, through the reference's S^2-sized workspace of
// naive_workspace_bytes(p) bytes (0: the sizes overflow).
size_t naive_workspace_bytes(const BwdProblem& p);
hipError_t launch_naive(const BwdProblem& p, const BwdTensors& t, void* workspace, int role);

// Polls a split wait makes before it gives up (test hook; default 1 << 24).
void set_split_spin_limit(int polls);

// Race-check instantiations of the main kernel for the launches that follow
// (test hook; see shaobo_fa3_ext_set_race_check).
void set_debug_kernels(bool on);

// Device of the launches on `stream` (null: the legacy default stream of
// the current device).  The library's per-device arrays (the no-allocation
// scratch, the give-up count) are looked up with that device current, so a
// stream of another device than the current one is refused
// (hipErrorInvalidDevice).
hipError_t launch_device(hipStream_t stream, int* dev);

// Workspace of the no-allocation entry: a static device array of
// kNoAllocScratchBytes per GPU.  noalloc_scratch returns its device address
// on device dev, which must be current (looked up once per device, then
// cached).
constexpr size_t kNoAllocScratchBytes = SHAOBO_FA3_EXT_SCRATCH_BYTES;
hipError_t noalloc_scratch(int dev, void** ptr);

// Device address of device dev's count of split waits that gave up (a
// 64-bit counter the kernels increment; dev must be current).
hipError_t split_giveup_count(int dev, unsigned long long** ptr);

// Whether `word` is an epoch one of this process's launches used: an error
// word holding one was written by a split wait that gave up (garbage in an
// uninitialised workspace practically never falls in that range).
bool epoch_issued(unsigned long long word);

// Byte offset of the error word in every v2 / legacy / fused5 workspace.
constexpr size_t kErrWordOffset = 0;

}  // namespace fa3
