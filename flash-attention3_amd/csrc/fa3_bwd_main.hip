// Main FA3 backward kernel for gfx950: the fast instantiations and the host
// side (job map, split plan, workspace plan, launch).  The kernels and their
// device helpers are in fa3_bwd_main_kernel.h.
#include "fa3_bwd_main_kernel.h"
#include "fa3_job_map.h"
#include "fa3_split_plan.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <memory>
#include <mutex>
#include <random>
#include <vector>

namespace fa3 {
namespace {



FusedArgs base_args(const BwdProblem& p, const BwdTensors& t) {
    FusedArgs a{};
    a.q = (const _Float16*)t.q;
    a.k = (const _Float16*)t.k;
    a.v = (const _Float16*)t.v;
    a.dout = (const _Float16*)t.dout;
    a.dq = t.dq;
    a.dk = t.dk;
    a.dv = t.dv;
    a.out_f32 = p.out_f32 ? 1 : 0;
    a.q_rs = p.bshd ? p.heads_q * p.head_dim : p.head_dim;
    a.q_hs = p.bshd ? p.head_dim : p.seqlen * p.head_dim;
    a.kv_rs = p.bshd ? p.heads_kv * p.head_dim : p.head_dim;
    a.kv_hs = p.bshd ? p.head_dim : p.seqlen * p.head_dim;
    a.seqlen = p.seqlen;
    a.heads_q = p.heads_q;
    a.heads_kv = p.heads_kv;
    a.group = p.heads_q / p.heads_kv;
    a.div_hq = make_fastdiv(p.heads_q);
    a.div_hkv = make_fastdiv(p.heads_kv);
    a.div_group = make_fastdiv(a.group);
    a.div_g1 = make_fastdiv(a.group + 1);
    a.n_groups = p.batch * p.heads_kv;
    a.scale_log2 = p.scale * kLog2e;
    a.scale = p.scale;
    a.spin_limit = 1;
    return a;
}


std::atomic<int> g_spin_limit{1 << 24};
std::atomic<bool> g_debug_kernels{false};

// Compute units of device `dev` (cached per device); 0 if unknown.
int cu_count(int dev) {
    static std::mutex mu;
    static int cache[64] = {};
    if (dev < 0 || dev >= 64) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cache[dev] = n;
    }
    return cache[dev];
}

// Epochs: a process-wide counter started at a random 64-bit value, so a
// word left in a workspace by an earlier launch (of this or another
// process) practically never equals the current launch's epoch.  The
// launches of this process have used the epochs [g_epoch0, g_epoch) (0
// skipped), which lets the host tell an error word written by one of them
// from whatever an uninitialised workspace holds.
unsigned long long epoch_seed() {
    std::random_device rd;
    unsigned long long x = ((unsigned long long)rd() << 32) ^ rd();
    x ^= (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count();
    return x | 1;
}
const unsigned long long g_epoch0 = epoch_seed();
std::atomic<unsigned long long> g_epoch{g_epoch0};

unsigned long long next_epoch() {
    unsigned long long e;
    do e = g_epoch.fetch_add(1, std::memory_order_relaxed);
    while (e == 0);
    return e;
}

// size_t arithmetic that reports overflow instead of wrapping
struct Checked {
    size_t v = 0;
    bool ok = true;
    Checked add(size_t x) const {
        Checked r = *this;
        r.ok = ok && !__builtin_add_overflow(v, x, &r.v);
        return r;
    }
    Checked mul(size_t x) const {
        Checked r = *this;
        r.ok = ok && !__builtin_mul_overflow(v, x, &r.v);
        return r;
    }
    Checked align() const { return add(255).and_mask(); }
    Checked and_mask() const {
        Checked r = *this;
        r.v &= ~(size_t)255;
        return r;
    }
};

}  // namespace

void set_split_spin_limit(int polls) { g_spin_limit.store(polls < 0 ? 0 : polls); }

void set_debug_kernels(bool on) { g_debug_kernels.store(on); }

bool epoch_issued(unsigned long long word) {
    return word != 0 && word - g_epoch0 < g_epoch.load(std::memory_order_relaxed) - g_epoch0;
}

// Workspace of the no-allocation entry.  Each GPU holds its own copy of the
// array; in host code `scratch` is only a handle for the runtime, never a
// device address, so the kernels receive the address hipGetSymbolAddress
// reports for the launch's device.  Nothing in it needs clearing between
// calls: the split words are tagged with each launch's epoch, and everything
// else is written before it is read within a call.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
// Split waits that gave up on this GPU since the library was loaded (the
// kernels count them; shaobo_fa3_ext_split_error_count reads them).
static __device__ unsigned long long split_giveups[1];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_symbol_mu;
void* g_scratch_ptr[kMaxDevices] = {};
void* g_giveups_ptr[kMaxDevices] = {};

// Device address of a __device__ array on device dev, looked up once per
// device with that device current (the caller's launches run on it).
hipError_t symbol_address(int dev, const void* symbol, void* (&cache)[kMaxDevices], void** ptr) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_symbol_mu);
    if (cache[dev] == nullptr) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != dev) return hipErrorInvalidDevice;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, symbol);
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        cache[dev] = p;
    }
    *ptr = cache[dev];
    return hipSuccess;
}
}  // namespace

hipError_t noalloc_scratch(int dev, void** ptr) {
    return symbol_address(dev, HIP_SYMBOL(scratch), g_scratch_ptr, ptr);
}

hipError_t split_giveup_count(int dev, unsigned long long** ptr) {
    void* p = nullptr;
    const hipError_t e = symbol_address(dev, HIP_SYMBOL(split_giveups), g_giveups_ptr, &p);
    *ptr = static_cast<unsigned long long*>(p);
    return e;
}

// The split plan runs its workgroups in one round: past one job per CU the
// default plan (one job per workgroup, or the persistent queues from 512
// jobs on) measured faster for every shape tried -- 384 jobs: B1 H12 S1024
// D128 -18 %, B1 H6 S2048 D64 -24 %; 512 jobs: B1 H8 S2048 D128 -4.8 %,
// B1 H2 S8192 D64 -10.6 %, B1 H16 S1024 D64 +0.3 %.
constexpr long long kSplitMaxJobs = 256;
static_assert(kSplitMaxJobs <= kMaxSplitWgs, "one descriptor per split-plan workgroup");

// Head-split plan choice.  Work in dKV steps (a dQ step ~0.75 of one); a
// CU's share = all steps / kHeadSplitCus (an MI355X's CU count: the plan,
// and so the workspace size, depends on the shape only).  The merged plan
// takes max(share, G QT) -- its longest job, G heads' query tiles against
// key tile 0 -- and chunks of G / f heads take max(share, G QT / f), times
// 1 + kHeadSplitPerChunk f (the fp32 contributions' traffic and the extra
// prologues), plus kHeadSplitFixed for the reduction launch.  The plan picks
// the f with the least estimate, if it is below kHeadSplitGain x the merged
// plan's: near the boundary the estimate's error exceeds the gain (B2 Hq16
// Hkv4 S2048 D128 causal: estimated -3 %, measured +9 %).  Measured (D 128
// causal): 32 chunks at B1 Hq32 Hkv1 S4096 run each step of the share ~12 %
// slower than the merged plan runs a full machine's; 8 chunks there take
// the backward from 1 596 to 532 us, 2 chunks at B4 from 2 099 to 1 982.
constexpr int kHeadSplitCus = 256;
constexpr double kHeadSplitPerChunk = 0.004;
constexpr double kHeadSplitFixed = 8.0;
constexpr double kHeadSplitGain = 0.92;
constexpr int kHeadSplitMaxChunks = 64;

// The chunk count f (a divisor of G, >= 2) of the head-split plan for this
// shape, or 0 for the merged plan.  (G QT > share needs QT + 1 < 2 x 256 /
// (1.75 B Hkv) causal, QT < 256 / (1.75 B Hkv) full: the plan never meets a
// sequence long enough to strain the reduction's 32-bit indices.)
int head_split_chunks(const BwdProblem& p, int qt) {
    const int group = p.heads_kv > 0 ? p.heads_q / p.heads_kv : 0;
    if (group < 2 || qt <= 0 || p.out_f32 || p.no_head_split) return 0;
    const double steps = p.causal ? 0.5 * qt * (qt + 1.0) : (double)qt * qt;
    const double share = (double)p.batch * p.heads_q * steps * 1.75 / kHeadSplitCus;
    const double merged = std::max(share, (double)group * qt);
    int best = 0;
    double best_t = kHeadSplitGain * merged;
    // beyond 64 chunks the chunks' own cost (+26 %) outweighs any split
    for (int f = 2; f <= std::min(group, kHeadSplitMaxChunks); ++f) {
        if (group % f != 0) continue;
        const double t = std::max(share, (double)(group / f) * qt) * (1.0 + kHeadSplitPerChunk * f) +
                         kHeadSplitFixed;
        if (t < best_t) {
            best_t = t;
            best = f;
        }
    }
    return best;
}

WorkspacePlan plan_workspace(const BwdProblem& p) {
    WorkspacePlan w;
    if (p.batch <= 0 || p.heads_q <= 0 || p.seqlen <= 0 || p.head_dim <= 0) return w;
    const Checked rows = Checked{(size_t)p.batch}.mul((size_t)p.heads_q).mul((size_t)p.seqlen);
    Checked at{256};  // the error word's region
    w.err_off = kErrWordOffset;
    w.nlse2_off = at.v;
    at = at.add(rows.mul(sizeof(float)).v).align();
    w.ndelta_off = at.v;
    at = at.add(rows.mul(sizeof(float)).v).align();
    w.queue_off = at.v;
    at = at.add(kQueueBytes).align();
    if (!rows.ok) return w;
    // Split plan for causal shapes with one query head per KV head and few
    // jobs (at most one per CU of an MI355X): see bwd_main_kernel.
    const int qt = p.seqlen / kTileM;
    const long long jobs = 2LL * p.batch * p.heads_q * qt;
    if (p.causal && p.heads_q == p.heads_kv && qt >= 4 && qt % 2 == 0 && jobs <= kSplitMaxJobs) {
        w.bal_m = qt / 2;  // <= kMaxBalM since jobs <= kSplitMaxJobs
        w.n_split = p.batch * p.heads_q * w.bal_m;
        const size_t kv_piece = (size_t)4 * 2 * (p.head_dim / 64) * 4096;
        const size_t q_piece = (size_t)4 * (p.head_dim / 64) * 4096;
        w.sync_off = at.v;
        at = at.add((size_t)w.n_split * 4 * sizeof(unsigned long long)).align();
        w.pkv_off = at.v;
        at = at.add((size_t)w.n_split * kv_piece).align();
        w.pq_off = at.v;
        at = at.add((size_t)w.n_split * q_piece).align();
        // the kernel addresses the partial sums with 32-bit buffer offsets
        if (w.pq_off - w.pkv_off > 0xFFFFFFFFull || at.v - w.pq_off > 0xFFFFFFFFull) return w;
    }
    // Head-split default plan for GQA: when one dKV job (G heads' query
    // tiles against one key tile) is much longer than a CU's share of the
    // work, it alone sets the kernel's length (MQA at batch 1), so each dKV
    // job runs for a chunk of the heads and the chunks' fp32 contributions
    // are summed afterwards.
    if (w.bal_m == 0) {
        w.hs_chunks = head_split_chunks(p, qt);
        if (w.hs_chunks > 0) {
            w.hsd_off = at.v;
            const Checked parts = Checked{(size_t)p.batch}
                                      .mul((size_t)p.heads_kv)
                                      .mul((size_t)w.hs_chunks)
                                      .mul((size_t)p.seqlen)
                                      .mul((size_t)p.head_dim);
            at = at.add(parts.mul(sizeof(float) * 2).v).align();
            if (!parts.ok) return w;
        }
    }
    if (!at.ok || !rows.ok || rows.v > (size_t)INT32_MAX) return w;
    w.total = at.v;
    w.ok = true;
    return w;
}

hipError_t launch_component(const BwdProblem& p, const BwdTensors& t, int role) {
    FusedArgs a = base_args(p, t);
    a.packed = t.packed_in;
    a.smax = t.aux0;
    a.ssum = t.aux1;
    a.delta = t.delta_in;
    a.jobs_per_group = p.seqlen / kTileN;
    set_job_map(a);
    const dim3 grid(a.n_groups * a.jobs_per_group);
    if (p.head_dim == 128) {
        if (role == 1) hipLaunchKernelGGL((bwd_component_kernel<128, 1>), grid, dim3(kThreads), 0, t.stream, a);
        else hipLaunchKernelGGL((bwd_component_kernel<128, 2>), grid, dim3(kThreads), 0, t.stream, a);
    } else {
        if (role == 1) hipLaunchKernelGGL((bwd_component_kernel<64, 1>), grid, dim3(kThreads), 0, t.stream, a);
        else hipLaunchKernelGGL((bwd_component_kernel<64, 2>), grid, dim3(kThreads), 0, t.stream, a);
    }
    return hipGetLastError();
}

#ifdef FA3_TIMELINE
namespace {
unsigned long long* g_timeline = nullptr;
}
// Timeline build only (no product entry point): the device buffer that the
// main-kernel launches that follow fill with per-workgroup timestamps (null:
// none).  At least 2^21 + 32 x workgroups 64-bit words, zeroed by the caller.
extern "C" __attribute__((visibility("default"))) void fa3_timeline_set(void* buffer) {
    g_timeline = static_cast<unsigned long long*>(buffer);
}
#endif

hipError_t launch_backward(const BwdProblem& p, const BwdTensors& t, void* workspace,
                           unsigned long long* epoch) {
    const WorkspacePlan plan = plan_workspace(p);
    if (!plan.ok) return hipErrorInvalidValue;
    char* ws = static_cast<char*>(workspace);
    FusedArgs a = base_args(p, t);
    float* nlse2 = reinterpret_cast<float*>(ws + plan.nlse2_off);
    float* ndelta = reinterpret_cast<float*>(ws + plan.ndelta_off);
    auto mark = [&](int i) {
        return t.events[i] != nullptr ? hipEventRecord(t.events[i], t.stream) : hipSuccess;
    };
    hipError_t err = mark(0);
    if (err != hipSuccess) return err;
    unsigned int* queue = reinterpret_cast<unsigned int*>(ws + plan.queue_off);
    if (t.stages & 1) {
        err = t.packed_in != nullptr ? launch_rowstats(p, t, nlse2, ndelta, queue)
                                     : launch_preprocess(p, t, nlse2, ndelta, queue);
    }
    if (err == hipSuccess) err = mark(1);
    if (err != hipSuccess) return err;
    if (!(t.stages & 2)) return mark(2);
    a.nlse2 = nlse2;
    a.ndelta = ndelta;
    const int group = p.heads_q / p.heads_kv;
    // per key tile / query tile: one dKV job (head split: one per chunk of
    // G / chunks query heads) and G dQ jobs
    a.jobs_per_group = (p.seqlen / kTileN) * ((plan.hs_chunks > 0 ? plan.hs_chunks : 1) + group);
    if (plan.hs_chunks > 0) {
        a.part_dk = reinterpret_cast<float*>(ws + plan.hsd_off);
        a.part_dv = a.part_dk + (size_t)p.batch * p.heads_kv * plan.hs_chunks * p.seqlen * p.head_dim;
        a.hs_chunks = plan.hs_chunks;
        a.hs_heads = group / plan.hs_chunks;
        a.div_chunks = make_fastdiv(plan.hs_chunks);
    }
    const int cus = cu_count(t.device) & ~7;
    {
        // the longest job (a dKV job: its G, or G / chunks, heads' query
        // tiles) against a CU's share, in dKV steps (a dQ step ~0.75)
        const int qt = p.seqlen / kTileN;
        const double steps = p.causal ? 0.5 * qt * (qt + 1.0) : (double)qt * qt;
        const double share = (double)p.batch * p.heads_q * steps * 1.75 / std::max(cus, 8);
        const int heads = plan.hs_chunks > 0 ? group / plan.hs_chunks : group;
        set_job_map(a, (double)heads * qt, share, std::max(cus, 8));
    }
    a.n_jobs = a.n_groups * a.jobs_per_group;
    a.queue = queue;
    // persistent default plan once there are more than two jobs per CU: one
    // workgroup per CU (a multiple of 8, the XCD count) pulls jobs from the
    // queues, so no CU waits for the in-order dispatch of new workgroups.
    // At exactly two per CU the hardware's dispatch of one job per
    // workgroup measured faster (512 jobs: B1 H16 S1024 D128 -9.8 %, B1 H8
    // S2048 D64 -11.2 %, B1 H16 S1024 D64 full -19.3 %, B1 H4 S4096 D128
    // -1.1 %); from 576 jobs on the queues win (B1 H9 S2048 D128: +7.6 %
    // without them), and below 512 too (384 jobs: +6 to +16 % with them).
    a.persist = plan.bal_m == 0 && cus >= 8 && a.n_jobs > 2 * cus ? cus : 0;
    a.epoch = next_epoch();
    if (epoch != nullptr) *epoch = a.epoch;
    a.err = reinterpret_cast<unsigned long long*>(ws + plan.err_off);
    err = split_giveup_count(t.device, &a.giveups);
    if (err != hipSuccess) return err;
    a.spin_limit = g_spin_limit.load();
#ifdef FA3_TIMELINE
    a.tl = g_timeline;
#endif
    a.bal_m = plan.bal_m;
    if (plan.bal_m > 0) {
        a.n_split = plan.n_split;
        a.sync = reinterpret_cast<unsigned long long*>(ws + plan.sync_off);
        a.part_kv = reinterpret_cast<float*>(ws + plan.pkv_off);
        a.part_q = reinterpret_cast<float*>(ws + plan.pq_off);
        a.part_kv_bytes = (uint32_t)(plan.pq_off - plan.pkv_off);
        a.part_q_bytes = (uint32_t)(plan.total - plan.pq_off);
        // each workgroup's descriptor: its job id's kind x = pos mod M (pos
        // as the job map deals it), group, head-piece length and short job
        const int M = plan.bal_m;
        if (a.n_jobs > kMaxSplitWgs || a.n_groups > 64) return hipErrorInvalidValue;
        const SplitPlan& sp = split_plan(M);
        for (int id = 0; id < a.n_jobs; ++id) {
            int g = 0, pos = 0;
            job_of(a, id, g, pos);
            const int kind = pos / M, x = pos % M;
            const int len = kind == 1 || kind == 2 ? sp.head_kv[x] : sp.head_q[x];
            const int s = sp.shrt[kind][x];
            const int sfield = s < 0 ? kNoShort : sp.after[kind][x] ? kShortAfter + s : s;
            a.split_desc[id] = split_desc(kind, x, g, len, sfield);
        }
    }
    if (g_debug_kernels.load()) launch_race_check(a, p.head_dim, p.causal, p.bf16, t.stream);
    else if (p.head_dim == 128) launch_dd<128, false>(a, p.causal, p.bf16, t.stream);
    else launch_dd<64, false>(a, p.causal, p.bf16, t.stream);
    err = hipGetLastError();
    if (err == hipSuccess && plan.hs_chunks > 0) {
        const dim3 rg((unsigned)((p.seqlen * (p.head_dim / 4) + 255) / 256),
                      (unsigned)(p.batch * p.heads_kv));
        _Float16* dk = static_cast<_Float16*>(t.dk);
        _Float16* dv = static_cast<_Float16*>(t.dv);
        auto reduce = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, rg, dim3(256), 0, t.stream, a.part_dk, a.part_dv, dk, dv,
                               p.heads_kv, plan.hs_chunks, p.seqlen, a.kv_rs, a.kv_hs);
        };
        if (p.head_dim == 128)
            reduce(p.bf16 ? gqa_reduce_kernel<128, true> : gqa_reduce_kernel<128, false>);
        else
            reduce(p.bf16 ? gqa_reduce_kernel<64, true> : gqa_reduce_kernel<64, false>);
        err = hipGetLastError();
    }
    return err == hipSuccess ? mark(2) : err;
}

}  // namespace fa3
