// Main FA3 backward kernel for gfx950 (replaces the reference's fused 5-GEMM
// kernel and its dQ / GQA-dKV reductions: src/fused_bwd_kernel.cpp:1362-1671,
// src/fused_bwd_dq_reduce.cpp:27-109, and the legacy dKV / dQ kernels
// src/dkv_kernel.cpp:957-1085, src/dq_kernel.cpp:794-953).  It runs after the
// delta preprocess (fa3_bwd_preprocess.hip), which supplies per query row
// -lse2 = -LSE * log2(e) and -delta = -rowsum(dO * O); the component kernels
// at the end of this file read the reference's row statistics directly
// instead.
//
// Two job roles; each output element has one writer:
//
//  * dKV role -- owns a 64-key tile of one KV head; streams every 64-row query
//    tile that can see it (causal: from the diagonal on) of every query head
//    in its GQA group, accumulating dK^T and dV^T in fp32 registers:
//        S = Q K^T, dP = dO V^T, P = exp2(S c - lse2), dS = P (dP - delta),
//        dV^T += dO^T P, dK^T += Q^T dS                 (4 GEMMs per tile)
//  * dQ role -- owns a 64-row query tile of one query head; streams the key
//    tiles it sees, recomputing S^T and dP^T, and accumulates dQ^T:
//        S^T = K Q^T, dP^T = V dO^T, dS^T, dQ^T += K^T dS^T (3 GEMMs per tile)
//
// The softmax scale is folded out of dS and applied once to dK and dQ.  The
// score waves' resident operand (K in the dKV role, Q in the dQ role) is
// multiplied by c = scale * log2(e) in LDS as it lands (fp32 product,
// rounded once to the operand type) and -lse2 seeds the S accumulators, so
// the MFMAs leave S c - lse2 and P costs one exp2 per element (kScaled).
// When c > 1 (scale > ln 2) K c or Q c could overflow fp16: those launches,
// the split plan and the component kernels use the unscaled instantiations,
// which apply c in the loop.
//
// A workgroup runs one job with 8 waves, two per SIMD, specialised:
//   score waves 0..3: S and dP of 16 rows x 64 columns of the step's tile
//            pair (v_mfma_f32_16x16x32_f16; -delta seeds the dP
//            accumulators), then P and dS in fp16 into LDS;
//   gradient waves 4..7: the output products (v_mfma_f32_32x32x16_f16) over
//            the P / dS written one step earlier, each wave a share of the
//            (matrix, 32-wide D slice) pairs; the streamed tile's transposed
//            operand (ds_read_b64_tr_b16) is read one step ahead and carried
//            in registers.
// In step j the score waves make P / dS of tile j + 1 while the gradient
// waves consume those of tile j, so P / dS are double-buffered and one
// barrier per step suffices; both loops pass the same barriers, and the
// compiler allocates registers for the larger of the two, not their sum.
// Every global read of the loop is a direct-to-LDS load (global_load_lds)
// into one of three stages, issued two steps ahead (by all 8 waves at head
// dim 128, by the gradient waves at 64): a stage holds a streamed tile pair
// and, in the dKV role, its 64 rows' statistics.  The issue pattern
// is the same every step (a finished stream re-loads its last tile into a
// free stage), so every wait is a constant count.
//
// Split plan (causal, one query head per KV head, at most 256 jobs; see
// bwd_main_kernel): long jobs are cut in two pieces run by different
// workgroups.  Each piece counts its arrival; the first to arrive stores its
// fp32 partial sums with device-coherent stores and marks them done, the
// second waits for that mark, adds them to its own and writes the output.
// fp32 addition of two terms is commutative, so the result does not depend
// on which piece finished first.
//
// This header holds the kernels and their device helpers; it is compiled
// into fa3_bwd_main.hip (the fast instantiations and the host side) and
// fa3_bwd_main_debug.hip (the race-check instantiations, see debug_sync),
// so that the two halves build in parallel.
#pragma once

#include <type_traits>

#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"
#include "fa3_split_plan.h"

namespace fa3 {

constexpr int kMaxSplitWgs = 256;  // its workgroups: one per job, at most one per CU

// Split-plan workgroup descriptor (one 32-bit word per workgroup, built on
// the host): bits 0..1 the workgroup's kind (see bwd_main_kernel), 2..8 x,
// 9..14 the (batch, head) group, 15..23 the head-piece length of the split
// job it works on (tiles; a length covering the whole job leaves it
// unsplit), 24..31 the short dQ job (query tile < M) that the workgroup
// runs before its piece (kind 0: between its whole dKV job and its dQ
// remainder), kShortAfter + that tile for a short job run after the piece
// (tiles < 127 only), or kNoShort.  The split plan has at most 256 jobs and
// S / 64 >= 4, so M <= 64, groups <= 32 and lengths <= 128 fit (the fields
// would hold 512 jobs).
constexpr int kNoShort = 255;
constexpr int kShortAfter = 128;
__host__ __device__ constexpr uint32_t split_desc(int kind, int x, int g, int len, int shrt) {
    return (uint32_t)kind | ((uint32_t)x << 2) | ((uint32_t)g << 9) | ((uint32_t)len << 15) |
           ((uint32_t)shrt << 24);
}

struct FusedArgs {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    const _Float16* dout;
    // Row statistics, by row-source mode kRows of the role templates:
    // 0: -lse2 (lse2 = LSE log2 e) and -delta arrays written by a preprocess pass;
    // 1: the packed sidecar [max_log2, inv_sum, delta] per row (dKV only);
    // 2: raw row max, row sum and delta arrays (dQ only).
    const float* nlse2;  // [B*Hq*S], -lse2
    const float* ndelta; // [B*Hq*S], -delta
    const float* packed; // [B*Hq*S][3]
    const float* smax;   // [B*Hq*S]
    const float* ssum;
    const float* delta;
    void* dq;          // fp16 / bf16 (the inputs' type), or fp32 when out_f32
    void* dk;
    void* dv;
    int out_f32;
    // element strides of one sequence row and one head in the q-side (Q, O,
    // dO, dQ) and kv-side (K, V, dK, dV) tensors: BHSD (D, S D) or BSHD
    // (H D, D); a batch is H S D elements in both layouts
    int q_rs, q_hs, kv_rs, kv_hs;
    int seqlen;
    int heads_q;
    int heads_kv;
    int group;  // heads_q / heads_kv
    // divisors of the kernels' index arithmetic (FastDiv: magic multipliers
    // computed once on the host)
    FastDiv div_hq, div_hkv, div_group, div_g1;  // heads_q, heads_kv, group, group + 1
    // job map: n_groups (batch, kv head) groups of jobs_per_group jobs; with
    // xcd_parts > 0 each group is split into xcd_parts interleaved parts
    // ("virtual groups"), and XCD x runs the xcd_vgroups consecutive ones
    // from x xcd_vgroups on (so a group's parts share as few XCDs as they
    // can), one after another (xcd_interleave 0; map_radix = the part's
    // length) or position by position across them (xcd_interleave 1;
    // map_radix = xcd_vgroups).  Without parts that divide a group evenly
    // (xcd_parts 0), ids run group by group, or position by position across
    // all groups (xcd_interleave 1).
    int n_groups;
    int jobs_per_group;
    int xcd_parts;
    int map_radix;
    int xcd_interleave;
    int xcd_vgroups;
    int xcd_mode;  // xcd_parts | xcd_interleave << 8: job_of reads both in one load
    FastDiv div_parts, div_radix, div_jpg, div_groups;  // xcd_parts, map_radix, jobs_per_group, n_groups
    // Persistent default plan (persist > 0): the grid has persist workgroups
    // (a multiple of 8, one per CU).  Job ids of the map above are dealt to
    // queues by id % 8 (the XCD the hardware would have sent them to);
    // workgroup w runs id w first, then pops k = 0, 1, .. from queue w % 8
    // (a counter in the workspace, zeroed by the preprocess) and runs id
    // w % 8 + 8 (k + persist / 8), until the id reaches n_jobs.
    int persist;
    int n_jobs;
    unsigned int* queue;
    float scale_log2;
    float scale;
    // split plan (bal_m > 0, causal and one query head per KV head): see
    // bwd_main_kernel.  Synchronisation words and partial sums live in the
    // workspace.
    int bal_m;
    // one descriptor per workgroup (split_desc): a workgroup reads its own
    // word and the arguments its units' set-up needs in one batch of scalar
    // loads, so its first tile loads go out after one argument round trip
    uint32_t split_desc[kMaxSplitWgs];
    // Split-job synchronisation (see split_arrive / split_end): per split job
    // an arrival word and a ready word, compared with this launch's epoch, so
    // nothing needs clearing between launches.  dKV jobs first, then dQ jobs.
    unsigned long long epoch;
    unsigned long long* sync;
    unsigned long long* err;  // set to epoch when a split wait gives up
    unsigned long long* giveups;  // this GPU's count of split waits that gave up
    int spin_limit;
    int n_split;              // split jobs per role
    float* part_kv;    // [job][wave][register / 4][lane][4] fp32, first piece's sums
    float* part_q;
    uint32_t part_kv_bytes;
    uint32_t part_q_bytes;
    // Head-split default plan (GQA with few groups): each dKV job covers
    // hs_heads = G / hs_chunks query heads (chunk c: heads c hs_heads ..) and
    // writes its fp32 dK / dV contribution to part_dk / part_dv
    // [B][Hkv hs_chunks][S][D]; a reduce launch sums each KV head's
    // hs_chunks contributions (gqa_reduce_kernel).
    float* part_dk;
    float* part_dv;
    int hs_chunks;
    int hs_heads;
    FastDiv div_chunks;
#ifdef FA3_TIMELINE
    unsigned long long* tl;  // per-workgroup timestamps (timeline build only, below)
#endif
};

namespace {

// Timeline build (-DFA3_TIMELINE, lib/libshaobo_fa3_bwd_timeline.so; the
// product build compiles none of this): per workgroup, words 64 blockIdx.x ..
// hold [0] its entry time, [29] its split descriptor, [30] HW_ID, [31]
// XCC_ID; unit u < 4 of the workgroup stamps word (1 << 21) + 32 blockIdx.x +
// 8 u + s with s = 0 unit start, 7 resident tiles landed, 1 loop start,
// 2 last step done, 3 unit end (its stores complete), 4 first piece
// published, 5 second piece past its wait, 6 partial sums added.  The stamps
// are s_memrealtime (100 MHz) values written by the first gradient wave.
#ifdef FA3_TIMELINE
template <typename A>
__device__ __forceinline__ void tl_unit(const A& a, int u, int s) {
    if (a.tl != nullptr && threadIdx.x == 4 * kWave && u < 4)
        a.tl[(1u << 21) + (size_t)blockIdx.x * 32 + u * 8 + s] = __builtin_amdgcn_s_memrealtime();
}
#define FA3_TL(u, s) tl_unit(a, u, s)
#define FA3_TL_DRAIN() wait_vm_lgkm0<0>()
#else
#define FA3_TL(u, s) ((void)0)
#define FA3_TL_DRAIN() ((void)0)
#endif


// The kernel arguments where the launch put them, in the kernel-argument
// segment (constant address space, scalar loads).  The persistent job loop
// reads a job's set-up values (the divisors of the job map) through this
// pointer after an empty asm, so that the compiler re-reads them per job
// instead of holding them in scalar registers across both roles' code.
typedef __attribute__((address_space(4))) const FusedArgs KArgs;
__device__ __forceinline__ KArgs& kargs() {
    return *(KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
}
// a divisor read from the argument segment
__host__ __device__ __forceinline__ int fdiv(__attribute__((address_space(4))) const FastDiv& f, int n) {
    return fdiv(FastDiv{f.mul, f.shr, f.d}, n);
}

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kStages = 3;

template <int D>
struct Cfg {
    static constexpr int kTileBytes = 64 * D * 2;           // one [64][D] fp16 tile
    static constexpr int kRowsBytes = 1024;  // row statistics of 64 rows (768 B used)
    static constexpr int kStageBytes = 2 * kTileBytes + kRowsBytes;
    static constexpr int kKs = D / 32;                      // 16x16x32 k-steps over D
    static constexpr int kDB = D / 32;                      // 32-wide slices of D
    static constexpr int kChunks = D / 8;                   // 16-byte chunks per row
    static constexpr int kLoadsPerTile = kTileBytes / (kWaves * 1024);  // per lane, 8 loaders
    // Who issues the streamed tiles' loads: at D 64 the 4 gradient waves
    // (their MFMAs wait for the score waves' anyway, and the score waves are
    // the step's critical path: P5 -9 %); at D 128 all 8 waves (a gradient
    // wave with twice the loads and the larger transposed reads becomes the
    // critical path: P3 +7 %).
    static constexpr bool kGradLoads = D == 64;
    static constexpr int kLoaders = kGradLoads ? 4 : 8;
    static constexpr int kNld = kTileBytes / (kLoaders * 1024);  // tile loads per loader
    // direct-to-LDS loads per loading wave and stage: dKV Q, dO, rows; dQ K, V
    static constexpr int kDmaKv = 2 * kNld + 1;
    static constexpr int kDmaQ = 2 * kNld;
    static constexpr int kPdsBytes = 64 * 64 * 2;           // one [64][64] fp16 tile
    static constexpr int kPdsOff = kStages * kStageBytes;   // P / dS double buffer
    static constexpr int kFlagOff = kPdsOff + 2 * 2 * kPdsBytes;  // split-plan flag word
    static constexpr int kBytes = kFlagOff + 256;
    static_assert(kLoadsPerTile >= 1, "tile covers all waves");
    static_assert(kStageBytes % 512 == 0 && kPdsOff % 512 == 0, "bank-aligned tiles");
    static_assert(2 * kTileBytes <= 2 * 2 * kPdsBytes, "prologue staging fits the P / dS area");
    static_assert(kBytes <= 160 * 1024, "LDS budget");
};

// s_waitcnt vmcnt(N) lgkmcnt(0): all but the last N vector-memory loads have
// landed and this wave's LDS accesses are done.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that the compiler may not move memory accesses across.
__device__ __forceinline__ void barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
}

// 16-bit operands travel as f16x8 bits whatever their type; kBf16 selects
// the bf16 instruction.
template <bool kBf16>
__device__ __forceinline__ f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    if constexpr (kBf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <bool kBf16>
__device__ __forceinline__ f32x16 mfma_32x32x16t(f16x8 a, f16x8 b, f32x16 c) {
    if constexpr (kBf16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return mfma_32x32x16(a, b, c);
}
// fp32 -> the 16-bit operand type (round to nearest even), as f16 bits
template <bool kBf16>
__device__ __forceinline__ _Float16 to16(float x) {
    if constexpr (kBf16) return __builtin_bit_cast(_Float16, (__bf16)x);
    else return (_Float16)x;
}

// Direct-to-LDS copy of a row-major [64][D] fp16 tile into a swizzled LDS
// tile, shared by loaders (waves) of N 1 KiB blocks each.  Lane `lane` of
// loader `ld` moves the 16-byte chunk that belongs at LDS byte
// blk * 1024 + lane * 16 (blk = ld * N + j); its source byte offset within the
// global tile is precomputed once.
// Row order of the tiles the score waves hold as B operands (the dKV job's
// K / V, the dQ job's Q / dO): LDS row 16 b + i holds sequence row b + 4 i of
// the tile, so score block b's 16 columns are rows b, b + 4, .., b + 60 (the
// order that makes their P / dS stores conflict-free, see pds_off4).
__device__ __forceinline__ int perm_row(int r) { return (r >> 4) + 4 * (r & 15); }

// kPerm: LDS row r receives source row perm_row(r).
template <int D, int N = Cfg<D>::kLoadsPerTile, bool kPerm = false>
__device__ __forceinline__ void tile_load_offsets(uint32_t (&off)[N], int ld, int lane,
                                                  int row_stride) {
    using C = Cfg<D>;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const int id = (ld * N + j) * 64 + lane;  // physical chunk
        const int row = id / C::kChunks;
        const int phys = id % C::kChunks;
        int sw;
        if constexpr (C::kChunks == 16) sw = ((row & 3) << 2) | ((row >> 2) & 3);
        else sw = swz128(row);
        const int logical = (phys ^ sw) & (C::kChunks - 1);
        const int src = kPerm ? perm_row(row) : row;
        off[j] = (uint32_t)((src * row_stride + logical * 8) * 2);
    }
}

template <int N>
__device__ __forceinline__ void load_tile_async(FA3_LDS char* tile, const _Float16* src,
                                                const uint32_t (&off)[N], int ld) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
        __builtin_amdgcn_global_load_lds((const void*)((const char*)src + off[j]),
                                         (FA3_LDS void*)(tile + (ld * N + j) * 1024), 16, 0, 0);
    }
}

// Direct-to-LDS copy of the statistics of the 64 query rows row0 .. of a
// streamed tile by the 4 gradient waves, loader t moving rows 16 t .. 16 t +
// 15 (one load each; one dword per active lane):
//   kRows 0: -lse2 -> rows[32 t .. 32 t + 16), -delta -> rows[32 t + 16 ..
//            32 t + 32) (lanes 0..31);
//   kRows 1: packed[3 (row0 + 16 t) ..] -> rows[48 t .. 48 t + 48), i.e. the
//            [row][3] layout of all 64 rows (lanes 0..47).
template <int kRows>
__device__ __forceinline__ void load_rows4_async(FA3_LDS char* rows, const FusedArgs& a,
                                                 size_t row0, int t, int lane) {
    if constexpr (kRows == 0) {
        const float* src = (lane < 16 ? a.nlse2 : a.ndelta) + row0 + 16 * t + (lane & 15);
        if (lane < 32)
            __builtin_amdgcn_global_load_lds((const void*)src, (FA3_LDS void*)(rows + 128 * t), 4,
                                             0, 0);
    } else {
        static_assert(kRows == 1, "per-step rows of the dKV role");
        if (lane < 48)
            __builtin_amdgcn_global_load_lds((const void*)(a.packed + 3 * (row0 + 16 * t) + lane),
                                             (FA3_LDS void*)(rows + 192 * t), 4, 0, 0);
    }
}

// Direct-to-LDS copy of the row statistics of 64 query rows starting at row0;
// every wave issues exactly one load (one dword per active lane).
//   kRows 0: -lse2 -> rows[0..64), -delta -> rows[64..128); wave w, lanes 0..15.
//   kRows 1: packed[3 row0 .. 3 row0 + 192) -> rows[0..192) ([row][3]);
//            wave w, lanes 0..23 move dwords 24 w .. 24 w + 23.
//   kRows 2: max -> rows[0..64), sum -> rows[64..128), delta -> rows[128..192);
//            wave w, lanes 0..23 move entries 24 w .. 24 w + 23 of that list.
template <int kRows>
__device__ __forceinline__ void load_rows_async(FA3_LDS char* rows, const FusedArgs& a,
                                                size_t row0, int w, int lane) {
    if constexpr (kRows == 0) {
        const float* src = (w < 4 ? a.nlse2 : a.ndelta) + row0 + 16 * (w & 3) + lane;
        FA3_LDS char* dst = rows + 256 * (w >> 2) + 64 * (w & 3);
        if (lane < 16)
            __builtin_amdgcn_global_load_lds((const void*)src, (FA3_LDS void*)dst, 4, 0, 0);
    } else {
        const int i = 24 * w + lane;
        const float* src;
        if constexpr (kRows == 1) {
            src = a.packed + 3 * row0 + i;
        } else {
            const int arr = i >> 6;
            src = (arr == 0 ? a.smax : arr == 1 ? a.ssum : a.delta) + row0 + (i & 63);
        }
        if (lane < 24)
            __builtin_amdgcn_global_load_lds((const void*)src, (FA3_LDS void*)(rows + 96 * w), 4,
                                             0, 0);
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// the 16-bit operand type (f16 bits) -> fp32
template <bool kBf16>
__device__ __forceinline__ float from16(_Float16 x) {
    if constexpr (kBf16) return (float)__builtin_bit_cast(__bf16, x);
    else return (float)x;
}

// Multiplies by c (fp32 product, one rounding to the tile's type) the chunks
// of a tile that loader ld's load_tile_async copied into LDS: each lane reads
// back exactly the 16 bytes its own direct-to-LDS load wrote, so this wave's
// vmcnt wait for those loads orders it and no barrier is needed.  The
// caller's lgkmcnt wait and barrier publish the result.
template <bool kBf16, int N>
__device__ __forceinline__ void scale_own_chunks(FA3_LDS char* tile, int ld, int lane, float c) {
    f16x8 v[N];
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = lds_read_b128(tile, (ld * N + j) * 1024 + lane * 16);
#pragma unroll
    for (int j = 0; j < N; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = to16<kBf16>(from16<kBf16>(v[j][e]) * c);
        lds_write_b128(tile, (ld * N + j) * 1024 + lane * 16, v[j]);
    }
}

// threadIdx.x as a value the compiler cannot hoist out of a loop: in the
// persistent kernel's job loop, per-lane values derived from it (load
// offsets and the like) are then recomputed per job instead of being held in
// registers across both roles' code.
__device__ __forceinline__ int opaque_tid() {
    int tid = threadIdx.x;
    __asm__ volatile("" : "+v"(tid));
    return tid;
}

// Wave issue priority, pinned in program order.  A score wave runs its LDS
// reads and S / dP MFMAs at raised priority: its MFMAs then win the SIMD's
// matrix unit over the gradient wave's, so its softmax and P / dS writes
// (VALU, LDS) run beside the gradient wave's MFMAs instead of after them.
template <int kPrio>
__device__ __forceinline__ void set_prio() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(kPrio);
    __builtin_amdgcn_sched_barrier(0);
}

// A operand (32 x 16: m = D column, k = tile row) of a phase-2 product, read
// transposed from a swizzled [64][D] tile: lane l gets column 32 db + l % 32,
// rows 16 ks + 8 (l / 32) + t, t = 0..7 (two reads of 4 rows).
// swap (wave-uniform): rows 16 ks + 8 (l / 32) + 4 .. + 7 first, then + 0 ..
// + 3 -- the operand's two halves exchanged (see pds_off4).
template <int D>
__device__ __forceinline__ f16x8 tile_read_t(const FA3_LDS char* tile, int db, int ks, int lane,
                                             bool swap = false) {
    const int g = lane >> 4, r = lane & 15;
    const int col = 32 * db + 16 * (g & 1) + 4 * (r & 3);
    const int row = 16 * ks + 8 * (g >> 1) + (r >> 2);
    const uint32_t lo = tile_off<D>(row, col >> 3) + (col & 7) * 2;
    const uint32_t hi = tile_off<D>(row + 4, col >> 3) + (col & 7) * 2;
    return concat4(lds_read_tr4(tile, swap ? hi : lo), lds_read_tr4(tile, swap ? lo : hi));
}

// P / dS tile [64 rows][64 columns], 16-bit, 8 chunks of 16 B (8 columns) per
// row: P^T / dS^T of the dKV job (rows = keys, columns = query rows), dS of
// the dQ job (rows = query rows, columns = keys).  Chunk c of row r sits at
// r * 128 + (c ^ pds_swz(r)) * 16, its two 8-byte halves exchanged when r >=
// 32.  A score wave stores 4 columns (8 B) of rows b + 4 i, i = lane % 16
// (perm_row): pds_swz is a bijection on those rows' bits 2..4 and bit 5 picks
// the half, so the 16 lanes a ds_write_b64 serves together (16 k .. 16 k + 15,
// one 128-byte bank period) hit 16 distinct 8-byte slots.  The gradient waves'
// ds_read_b128 of rows 32 blk + l % 32 (served in groups of 16 lanes chosen by
// lane bit 5 and the parity of lane bits 2..4) stay conflict-free too; for
// blk = 1 the operand holds its two 4-column halves exchanged, and the A
// operand of the same product is exchanged to match (swap_halves, or
// tile_read_t's swap).
__device__ __forceinline__ int pds_swz(int r) { return ((r >> 2) & 7) ^ ((r >> 1) & 1); }
__device__ __forceinline__ uint32_t pds_chunk(int r, int c) {
    return (uint32_t)(r * 128 + ((c ^ pds_swz(r)) & 7) * 16);
}
// byte offset of columns 4 q .. 4 q + 3 of row r
__device__ __forceinline__ uint32_t pds_off4(int r, int q) {
    return pds_chunk(r, q >> 1) + (((q & 1) ^ (r >> 5)) & 1) * 8;
}
// (two 64-bit register moves)
__device__ __forceinline__ f16x8 swap_halves(f16x8 x) {
    typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
    const u64x2 v = __builtin_bit_cast(u64x2, x);
    unsigned long long lo, hi;
    __asm__("v_mov_b64 %0, %1" : "=v"(lo) : "v"(v[1]));
    __asm__("v_mov_b64 %0, %1" : "=v"(hi) : "v"(v[0]));
    return __builtin_bit_cast(f16x8, u64x2{lo, hi});
}
// Element offset of sequence row s of head h in batch b.
template <int D, typename A>
__device__ __forceinline__ size_t q_elem(const A& a, int b, int h, int s) {
    return (size_t)b * a.heads_q * a.seqlen * D + (size_t)h * a.q_hs + (size_t)s * a.q_rs;
}
template <int D, typename A>
__device__ __forceinline__ size_t kv_elem(const A& a, int b, int h, int s) {
    return (size_t)b * a.heads_kv * a.seqlen * D + (size_t)h * a.kv_hs + (size_t)s * a.kv_rs;
}

// ----------------------------------------------------------------------------
// Outputs
// ----------------------------------------------------------------------------
// 16 bytes of a final output (dQ, dK, dV), written with the non-temporal
// policy: nothing in this launch reads them again, so they stream out
// instead of sitting dirty in L2 until the kernel's end-of-launch writeback.
__device__ __forceinline__ void store_out(_Float16* p, f16x8 x) {
    __builtin_nontemporal_store(x, (f16x8*)p);
}

// Four consecutive output elements (element offset `off`): the inputs'
// 16-bit type, or fp32.
template <bool kBf16, typename A>
__device__ __forceinline__ void store4(const A& a, void* base, size_t off, f32x4 v) {
    if (a.out_f32) {
        *(f32x4*)((float*)base + off) = v;
    } else {
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = to16<kBf16>(v[e]);
        *(f16x4*)((_Float16*)base + off) = o;
    }
}

// (matrix, D slice) pair u of dKV gradient wave t, as pu = 2 slice + matrix
// (matrix 0: dV from dO and P, 1: dK from Q and dS).  Waves 0, 1 own dV and
// waves 2, 3 own dK, each for D / 64 consecutive 32-wide slices, so a wave
// reads only one of the P / dS tiles.
template <int D>
__device__ __forceinline__ int dkv_pair(int t, int u) {
    return 2 * ((D / 64) * (t & 1) + u) + (t >> 1);
}

// Output staging tiles of the epilogues, 16-bit, [rows][32] (64-byte rows,
// 4 chunks of 16 B) or [rows][64] (128-byte rows, 8 chunks): byte offset of
// half `hf` (8 bytes) of chunk c of row r.  A gradient wave writes one half
// of one chunk for 16 consecutive rows per ds_write_b64 lane group (one
// 128-byte bank period): the chunk XOR (row bits 1..2, or 0..2) and the half
// flip (row bit 3) put those 16 writes on distinct 8-byte slots.  The
// read-back (ds_read_b128 of whole chunks, rows with bit 3 uniform per
// instruction) stays conflict-free and swaps the halves of rows with bit 3
// set back (stage_fix).
__device__ __forceinline__ uint32_t stage64_chunk(int r, int c) {  // 16-byte aligned
    return (uint32_t)(r * 64 + ((c ^ (r >> 1)) & 3) * 16);
}
__device__ __forceinline__ uint32_t stage128_chunk(int r, int c) {  // 16-byte aligned
    return (uint32_t)(r * 128 + ((c ^ r) & 7) * 16);
}
__device__ __forceinline__ uint32_t stage64_off(int r, int c, int hf) {
    return stage64_chunk(r, c) + ((hf ^ (r >> 3)) & 1) * 8;
}
__device__ __forceinline__ uint32_t stage128_off(int r, int c, int hf) {
    return stage128_chunk(r, c) + ((hf ^ (r >> 3)) & 1) * 8;
}
__device__ __forceinline__ f16x8 stage_fix(f16x8 x, int r) {
    return (r & 8) ? __builtin_shufflevector(x, x, 4, 5, 6, 7, 0, 1, 2, 3) : x;
}
// Row of read-back instruction j, lane `lane`, of a 64-byte-row staging
// tile: lanes 4 i .. 4 i + 3 read the 4 chunks of one row; row bit 3 = j & 1.
__device__ __forceinline__ int stage64_row(int j, int lane) {
    return ((lane >> 2) & 7) | ((j & 1) << 3) | (((lane >> 5) & 1) << 4) | ((j >> 1) << 5);
}

// The head-split plan's fp32 dK / dV contributions [B][Hkv chunks][S][D], as
// seen by store_dkv (its fp32 path): one "KV head" per chunk, rows of D.
template <int D>
struct PartView {
    float* dk;
    float* dv;
    float scale;
    int seqlen;
    int heads_kv;  // Hkv x chunks
    size_t kv_hs;  // seqlen * D
    static constexpr int out_f32 = 1;
    static constexpr int kv_rs = D;
};

// dV^T / dK^T accumulators of gradient wave t (pairs dkv_pair(t, u)) to dV /
// dK of KV head hkv of batch b, keys kbase ..; lane: key 32 kb + l32,
// d = 32 slice + 8 (i / 4) + 4 h + i % 4.  The wave's pairs share one matrix
// and cover D columns d0 .. d0 + 32 kPpw of all 64 keys; 16-bit outputs are
// transposed through the wave's own 8 KiB (D 64: 4 KiB) of `stage` so that
// every global store writes whole 128-byte (D 64: 64-byte) row segments.
template <int D, bool kBf16, typename A>
__device__ __forceinline__ void store_dkv(const A& a, int b, int hkv, int kbase, int t, int lane,
                                          const f32x16 (&acc)[D / 64][2], FA3_LDS char* stage) {
    constexpr int kPpw = D / 64;
    const int l32 = lane & 31, h = lane >> 5;
    const size_t base = kv_elem<D>(a, b, hkv, kbase);
    if (!a.out_f32) {
        const float mul = (t >> 1) == 0 ? 1.f : a.scale;
        _Float16* outp = (_Float16*)((t >> 1) == 0 ? a.dv : a.dk);
        const int d0 = 32 * kPpw * (t & 1);
        FA3_LDS char* st = stage + t * (64 * 64 * kPpw);
#pragma unroll
        for (int u = 0; u < kPpw; ++u)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4) {
                    f16x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = to16<kBf16>(acc[u][kb][4 * a4 + e] * mul);
                    const int key = 32 * kb + l32;
                    const uint32_t off =
                        D == 128 ? stage128_off(key, 4 * u + a4, h) : stage64_off(key, a4, h);
                    lds_write_b64(st, off, v);
                }
        // the wave reads back only what it wrote: its LDS accesses complete in order
#pragma unroll
        for (int j = 0; j < 8 * kPpw / 2; ++j) {
            int key, c;
            if constexpr (D == 128) {
                key = 8 * j + ((lane >> 2) & 7);
                c = (lane & 3) | ((lane >> 5) << 2);
            } else {
                key = stage64_row(j, lane);
                c = lane & 3;
            }
            const f16x8 x = stage_fix(
                lds_read_b128(st, D == 128 ? stage128_chunk(key, c) : stage64_chunk(key, c)), key);
            store_out(outp + base + (size_t)key * a.kv_rs + d0 + 8 * c, x);
        }
        return;
    }
#pragma unroll
    for (int u = 0; u < kPpw; ++u) {
        const int pu = dkv_pair<D>(t, u);
        const float mul = (pu & 1) == 0 ? 1.f : a.scale;
        void* outp = (pu & 1) == 0 ? a.dv : a.dk;
        const size_t off0 = base + 32 * (pu >> 1) + 4 * h;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[u][kb][4 * a4 + e] * mul;
                store4<kBf16>(a, outp, off0 + (size_t)(32 * kb + l32) * a.kv_rs + 8 * a4, v);
            }
        }
    }
}

// dQ^T accumulators of gradient wave t to the dQ tile at element `base`;
// lane: row 32 rb + l32, d = 32 db + 8 (i / 4) + 4 h + i % 4.  16-bit
// outputs go through the wave's 4 KiB (D 64: 2 KiB) of `stage`, so every
// global store writes whole 64-byte row segments.
template <int D, bool kBf16, typename A>
__device__ __forceinline__ void store_dq(const A& a, size_t base, int t, int lane,
                                         const f32x16 (&acc)[D / 64], FA3_LDS char* stage) {
    constexpr int kRb = D / 64;
    const int db = D == 128 ? t : t >> 1;
    const int rb0 = D == 128 ? 0 : t & 1;
    const int l32 = lane & 31, h = lane >> 5;
    if (!a.out_f32) {
        FA3_LDS char* st = stage + t * (32 * kRb * 64);
#pragma unroll
        for (int r = 0; r < kRb; ++r)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f16x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = to16<kBf16>(acc[r][4 * a4 + e] * a.scale);
                lds_write_b64(st, stage64_off(32 * r + l32, a4, h), v);
            }
        _Float16* outp = (_Float16*)a.dq + base + 32 * db;
#pragma unroll
        for (int j = 0; j < 2 * kRb; ++j) {
            const int r = stage64_row(j, lane), c = lane & 3;  // r: row within the wave's block
            const f16x8 x = stage_fix(lds_read_b128(st, stage64_chunk(r, c)), r);
            store_out(outp + (size_t)(32 * rb0 + r) * a.q_rs + 8 * c, x);
        }
        return;
    }
    const size_t off0 = base + 32 * db + 4 * h;
#pragma unroll
    for (int r = 0; r < kRb; ++r) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[r][4 * a4 + e] * a.scale;
            store4<kBf16>(a, a.dq, off0 + (size_t)(32 * (rb0 + r) + l32) * a.q_rs + 8 * a4, v);
        }
    }
}

// Partial sums of split jobs travel between workgroups (possibly on
// different XCDs, whose L2 caches are not coherent with each other) through
// 16-byte buffer loads and stores with the sc1 cache policy -- the policy
// this chip's agent-scope atomic loads and stores use, coherent device-wide
// by itself -- so no cache-wide writeback / invalidate (which would also
// evict the tiles every CU of the XCD is streaming) is needed.  A wave's
// accumulators go out as [register / 4][lane][4]: one instruction moves 1 KiB
// of consecutive bytes.
constexpr int kCachePolicySc1 = 16;
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer access on gfx9

__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, kBufferWord3);
}

// Stores / adds the N accumulator blocks of one wave at byte offset base.
template <int N>
__device__ __forceinline__ void put_partials(__amdgpu_buffer_rsrc_t r, uint32_t base,
                                             const f32x16* acc, int lane) {
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = {acc[n][4 * g], acc[n][4 * g + 1], acc[n][4 * g + 2], acc[n][4 * g + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r,
                                                   base + ((n * 4 + g) * 64 + lane) * 16, 0,
                                                   kCachePolicySc1);
        }
}
template <int N>
__device__ __forceinline__ void add_partials(__amdgpu_buffer_rsrc_t r, uint32_t base, f32x16* acc,
                                             int lane) {
    f32x4 v[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            v[n][g] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           r, base + ((n * 4 + g) * 64 + lane) * 16, 0, kCachePolicySc1));
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[n][4 * g + e] += v[n][g][e];
}

// The two pieces of split job j meet through two 64-bit words, sync[2 j]
// (arrival) and sync[2 j + 1] (ready), compared with this launch's epoch: a
// value unique to the launch (nonzero), so a word never written by it reads
// as "not yet" and no clearing pass is needed; the words are left cleared at
// the end of every job, so a replayed launch that reuses its epoch (graph
// capture) finds them cleared too.
//
// split_arrive (thread 0, right after the score waves' last barrier, while
// the gradient waves run the last products): swaps the epoch into the arrival
// word.  The piece that reads back the epoch arrived second; it then waits
// for the ready word at once (a bounded spin), so that wait overlaps the
// gradient waves' last products instead of following them, and clears both
// words without waiting for those stores (nobody reads the words again in
// this launch).  *flag: 0 first, 1 second.
// split_end (every wave, after its last pipeline step; the gradient waves
// pass put_own storing their partial sums, the score waves a no-op): the
// first piece stores its partial sums, waits until its stores have
// completed (s_waitcnt vmcnt(0) covers stores on gfx9) and swaps the epoch
// into the ready word; it writes nothing else.  The second piece, past the
// barrier that follows its wait, adds the first piece's partial sums and
// writes the output.  The output is piece 0 + piece 1 either way (a
// two-term fp32 sum is the same in either order), so the result does not
// depend on which piece finishes first.
//
// The wait cannot block for long -- the first piece has left its loop and
// only stores after arriving -- but it is bounded all the same.  A wait that
// gives up swaps a marker (the epoch with bit 63 flipped) into the ready
// word; of the give-up and the first piece's publish, whichever comes later
// reads the other's value back and clears the word, so it never stays equal
// to the epoch (a replay would take that for published partial sums).  If
// the give-up reads back the epoch, the partial sums were published in time
// and nothing failed.  Otherwise it writes the epoch into the workspace's
// error word, which the host reports as a HIP error when it synchronises,
// and counts it in this GPU's give-up count, which asynchronous callers can
// query: a timed-out sum is never silent.
//
// Ordering: every cross-workgroup access (words and partial sums) is an
// agent-scope access with the sc1 policy, coherent at the device level; the
// writer's data stores complete before its ready swap is issued, and the
// reader issues its data loads only after it has observed the ready word
// (its wait and a workgroup barrier come in between).
__device__ __forceinline__ unsigned long long giveup_marker(unsigned long long epoch) {
    return epoch ^ (1ull << 63);
}

template <typename A>
__device__ __forceinline__ void split_arrive(const A& a, int job, FA3_LDS int* flag) {
    if (threadIdx.x == 0) {
        unsigned long long* arrival = a.sync + 2 * job;
        unsigned long long* ready = arrival + 1;
        const unsigned long long old =
            __hip_atomic_exchange(arrival, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool second = old == a.epoch;
        if (second) {
            bool seen = false;
            for (int i = 0; i < a.spin_limit; ++i) {
                if (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    a.epoch) {
                    seen = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (!seen) {
                seen = __hip_atomic_exchange(ready, giveup_marker(a.epoch), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
                if (!seen) {
                    __hip_atomic_store(a.err, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_fetch_add(a.giveups, 1ull, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            // leave the words cleared, so that a replay of the same launch (a
            // captured graph keeps the epoch) starts from "nobody arrived";
            // after a give-up the first piece's publish clears the ready word
            __hip_atomic_store(arrival, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (seen) __hip_atomic_store(ready, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *flag = second ? 1 : 0;
    }
}

template <typename A, typename PutOwn>
__device__ __forceinline__ bool split_end(const A& a, int job, FA3_LDS int* flag,
                                          PutOwn&& put_own) {
    wait_vm_lgkm0<63>();  // lgkmcnt(0): the flag's LDS store is done
    barrier();
    if (*flag != 0) return true;
    put_own();
    wait_vm_lgkm0<0>();
    barrier();
    if (threadIdx.x == 0) {
        unsigned long long* ready = a.sync + 2 * job + 1;
        if (__hip_atomic_exchange(ready, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            giveup_marker(a.epoch))
            __hip_atomic_store(ready, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return false;
}

// ----------------------------------------------------------------------------
// Race-check instantiations (kDebug): the same arithmetic in the same order,
// with the pipeline's concurrency taken out, so that a race in the fast
// kernel shows up as a bitwise difference between the two (tests compare
// them).  Every unit starts on an LDS filled with 0xFF bytes (a NaN in
// fp16, bf16 and fp32), so a read of LDS that the unit has not written
// turns its outputs into NaN; and after each LDS phase of a pipeline step
// (the score waves' operand reads and P / dS stores, the gradient waves'
// transposed reads and products) every wave waits for all of its memory
// operations and meets the others at a barrier.  Both roles pass the same
// number of these barriers per step and in their prologues.
// ----------------------------------------------------------------------------
template <bool kDebug>
__device__ __forceinline__ void debug_sync() {
    if constexpr (kDebug) {
        wait_vm_lgkm0<0>();
        barrier();
    }
}

template <int D, bool kDebug>
__device__ __forceinline__ void debug_poison(FA3_LDS char* smem) {
    if constexpr (kDebug) {
        debug_sync<true>();  // every wave is done with what the LDS holds
        const f16x8 nan = __builtin_bit_cast(f16x8, u32x4{~0u, ~0u, ~0u, ~0u});
        static_assert(Cfg<D>::kBytes % 16 == 0, "whole 16-byte chunks");
        for (int i = threadIdx.x * 16; i < Cfg<D>::kBytes; i += kThreads * 16)
            lds_write_b128(smem, i, nan);
        debug_sync<true>();
    }
}

// ----------------------------------------------------------------------------
// dKV role
// ----------------------------------------------------------------------------
// Key tile kt of KV head hkv in batch b.  Streams query tiles [qa, qb) of
// every query head of the group (kHeadSplit: of the hs_heads query heads from
// hr on, the outputs being their fp32 contribution, chunk pc of part_dk /
// part_dv).  slot < 0:
// the job is whole and writes dK / dV; otherwise the unit is piece slot & 1
// of split job slot >> 1 and the pieces' partial sums meet in split_end.
template <int D, bool kCausal, bool kBf16, int kRows = 0, bool kLateIssue = false,
          bool kScaled = true, bool kDebug = false, bool kHeadSplit = false, typename DA>
__device__ __forceinline__ void dkv_role(const FusedArgs& a, const DA& d, int b, int hkv, int kt, int qa, int qb,
                                         int slot,
                         FA3_LDS char* smem, int tlu = 0, int hr = 0, int pc = 0) {
    static_assert(kRows == 0 || kRows == 1, "dKV rows come as -lse2/-delta or packed");
    using C = Cfg<D>;
    const int tid = opaque_tid();
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = w & 3;
    const int l16 = lane & 15, g4 = lane >> 4, l32 = lane & 31, h = lane >> 5;

    const int S = d.seqlen;
    const int QT = S / 64;
    const int group = d.group;
    const int kbase = kt * 64;
    const int n_it = (kHeadSplit ? d.hs_heads : group) * (qb - qa);

    // loader index of this wave when it loads (see Cfg::kGradLoads)
    const int ldr = C::kGradLoads ? t : w;
    const bool loads = !C::kGradLoads || w >= 4;
    FA3_LDS char* pds0 = smem + C::kPdsOff;
    // this key tile's K (times c when kScaled, below) and V are staged in the
    // P / dS area; their loads go out before the rest of the set-up
    uint32_t ld_off[C::kNld], kv_off[C::kLoadsPerTile];
    tile_load_offsets<D, C::kLoadsPerTile, true>(kv_off, w, lane, d.kv_rs);
    {
        const size_t k0 = kv_elem<D>(d, b, hkv, kbase);
        load_tile_async(pds0, d.k + k0, kv_off, w);
        load_tile_async(pds0 + C::kTileBytes, d.v + k0, kv_off, w);
    }
    __builtin_amdgcn_sched_barrier(0);
    tile_load_offsets<D, C::kNld>(ld_off, ldr, lane, d.q_rs);

    // Cursor of the next query tile to load; a finished stream keeps
    // re-loading its last tile (into a stage nobody reads), so every step
    // issues the same loads.  (The cursor keeps running element and
    // statistics-row offsets, so a step's issue is a few adds.)
    int ld_qt = qa, ld_left = n_it;
    const int h0 = kHeadSplit ? hr : hkv * group;
    size_t ld_e = q_elem<D>(d, b, h0, qa * 64);                  // Q / dO element
    size_t ld_row = ((size_t)b * d.heads_q + h0) * S + qa * 64;  // statistics row
    const size_t step_e = (size_t)64 * d.q_rs;
    const size_t wrap_e = (size_t)d.q_hs - (size_t)(qb - qa - 1) * step_e;  // next head, tile qa
    const size_t wrap_row = (size_t)S - (size_t)(qb - qa - 1) * 64;
    auto issue = [&](FA3_LDS char* st) {  // loading waves
        load_tile_async(st, a.q + ld_e, ld_off, ldr);
        load_tile_async(st + C::kTileBytes, a.dout + ld_e, ld_off, ldr);
        if constexpr (C::kGradLoads)
            load_rows4_async<kRows>(st + 2 * C::kTileBytes, a, ld_row, t, lane);
        else
            load_rows_async<kRows>(st + 2 * C::kTileBytes, a, ld_row, w, lane);
        if (--ld_left > 0) {
            if (++ld_qt == qb) {
                ld_qt = qa;
                ld_e += wrap_e;
                ld_row += wrap_row;
            } else {
                ld_e += step_e;
                ld_row += 64;
            }
        }
    };
    // Step barrier: the loading waves' loads of the next tile have landed
    // (only the latest issue may be in flight) and every wave's LDS accesses
    // are done.
    auto top = [&]() {
        if (loads) wait_vm_lgkm0<C::kDmaKv>();
        else wait_vm_lgkm0<0>();
        barrier();
    };

    FA3_LDS char* st_ld = smem;                     // stage of tile j (refilled in step j)
    FA3_LDS char* st_1 = smem + C::kStageBytes;      // stage of tile j + 1
    FA3_LDS char* st_2 = smem + 2 * C::kStageBytes;  // stage of tile j + 2
    auto rotate = [&]() {
        FA3_LDS char* x = st_ld;
        st_ld = st_1;
        st_1 = st_2;
        st_2 = x;
    };
    FA3_LDS int* flag = (FA3_LDS int*)(smem + C::kFlagOff);
    FA3_LDS char* pds1 = pds0 + 2 * C::kPdsBytes;
    auto prologue_loads = [&]() {
        // K and V are on their way (issued at the top); the stages follow
        if (loads) {
            issue(st_ld);
            issue(st_1);
            issue(st_2);
        }
        if constexpr (kScaled) {
            // this wave's K loads have landed once only the later ones (V,
            // the three stages) may be in flight
            if (loads) wait_vm_lgkm0<C::kLoadsPerTile + 3 * C::kDmaKv>();
            else wait_vm_lgkm0<C::kLoadsPerTile>();
            scale_own_chunks<kBf16, C::kLoadsPerTile>(pds0, w, lane, a.scale_log2);
        }
        // wait for K and V only: the score waves copy them into registers
        // while the first streamed tile lands (the prologues wait for it)
        if (loads) wait_vm_lgkm0<3 * C::kDmaKv>();
        else wait_vm_lgkm0<0>();
        barrier();
    };

    if (w < 4) {
        // ---- score waves: S, dP, P, dS of query rows 16 t .. +16 and all 64
        // keys (four 16-key blocks kb: keys kb + 4 l16, perm_row); P^T and
        // dS^T go to LDS.
        // B operands: LDS row 16 kb + l16 (key kb + 4 l16), D chunk p1_chunk(s, g4)
        f16x8 kf[4][C::kKs], vf[4][C::kKs];
        f32x4 sacc[4], pacc[4];  // rows 16 t + 4 g4 + i, keys kb + 4 l16
        int sm_qt = qa;          // query tile of the next softmax
        auto next_masked = [&]() {
            const bool m = kCausal && sm_qt == kt;
            if (++sm_qt == qb) sm_qt = qa;
            return m;
        };
        // S = Q K^T and dP - delta = dO V^T - delta, then P and dS, written
        // transposed ([key][row]) into the P / dS buffer
        auto score = [&](bool masked, const FA3_LDS char* st, FA3_LDS char* pds,
                         FA3_LDS char* ld, bool do_issue) {
            f16x8 aq[C::kKs], ad[C::kKs];
            set_prio<3>();
#pragma unroll
            for (int s = 0; s < C::kKs; ++s) {
                const uint32_t off = tile_off<D>(16 * t + l16, p1_chunk<D>(s, g4));
                aq[s] = lds_read_b128(st, off);
                ad[s] = lds_read_b128(st + C::kTileBytes, off);
            }
            f32x4 nl2, ndl;  // -lse2 and -delta of rows 16 t + 4 g4 + i
            if constexpr (kRows == 0) {
                // -lse2 / -delta of rows 16 t .. in the layout of the loaders
                const FA3_LDS char* r =
                    st + 2 * C::kTileBytes +
                    (C::kGradLoads ? 128 * t + 16 * g4 : (16 * t + 4 * g4) * 4);
                nl2 = *(const FA3_LDS f32x4*)r;
                ndl = *(const FA3_LDS f32x4*)(r + (C::kGradLoads ? 64 : 256));
            } else {
                // [row][max_log2, inv_sum, delta]: exp2(x - m) * inv = exp2(x - (m - log2 inv))
                const FA3_LDS f32x4* r =
                    (const FA3_LDS f32x4*)(st + 2 * C::kTileBytes + (16 * t + 4 * g4) * 12);
                const f32x4 r0 = r[0], r1 = r[1], r2 = r[2];
                const float f[12] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1],
                                     r1[2], r1[3], r2[0], r2[1], r2[2], r2[3]};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    nl2[i] = __log2f(f[3 * i + 1]) - f[3 * i];
                    ndl[i] = -f[3 * i + 2];
                }
            }
            // all operand reads in flight before the first MFMA: the waits
            // then count down instead of draining the LDS queue per k-step.
            // kLateIssue (split plan): this wave's loads of the tile after
            // next go out behind them (P3 -1 %); otherwise right after the
            // barrier (step), which suits the default plan's longer loads
            // (more L2 misses; P4 +0.6 % the other way)
            __builtin_amdgcn_sched_barrier(0);
            if (!C::kGradLoads && kLateIssue && do_issue) issue(ld);
            __builtin_amdgcn_sched_barrier(0);
            debug_sync<kDebug>();
#pragma unroll
            for (int s = 0; s < C::kKs; ++s) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    sacc[kb] = mfma_16x16x32<kBf16>(aq[s], kf[kb][s],
                                                    s != 0 ? sacc[kb] : kScaled ? nl2 : f32x4{});
                    pacc[kb] = mfma_16x16x32<kBf16>(ad[s], vf[kb][s], s == 0 ? ndl : pacc[kb]);
                }
            }
            set_prio<0>();
            // sacc = S c - lse2 (kScaled: K c, -lse2 seed), else S
            float p[16], ds[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int kb = e >> 2, i = e & 3;
                p[e] = fast_exp2(kScaled ? sacc[kb][i] : sacc[kb][i] * a.scale_log2 + nl2[i]);
                ds[e] = p[e] * pacc[kb][i];
            }
            if (masked) {  // causal diagonal tile: keys after the row see nothing
                __asm__ volatile("" ::: "memory");  // keep this a branch
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    if ((e >> 2) + 4 * l16 > 16 * t + 4 * g4 + (e & 3)) {
                        p[e] = 0.f;
                        ds[e] = 0.f;
                    }
                }
            }
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                f16x4 pv, dv;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pv[i] = to16<kBf16>(p[4 * kb + i]);
                    dv[i] = to16<kBf16>(ds[4 * kb + i]);
                }
                const uint32_t off = pds_off4(kb + 4 * l16, 4 * t + g4);
                lds_write_b64(pds, off, pv);
                lds_write_b64(pds + C::kPdsBytes, off, dv);
            }
            debug_sync<kDebug>();
        };
        // The LDS regions a step touches are passed as restrict pointers, so
        // the compiler can tell that its reads do not depend on the
        // direct-to-LDS loads into other regions and adds no wait for them.
        auto prologue = [&](FA3_LDS char* __restrict__ s0, FA3_LDS char* __restrict__ pa) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int s = 0; s < C::kKs; ++s) {
                    const uint32_t off = tile_off<D>(16 * kb + l16, p1_chunk<D>(s, g4));
                    kf[kb][s] = lds_read_b128(pa, off);
                    vf[kb][s] = lds_read_b128(pa + C::kTileBytes, off);
                }
            if constexpr (C::kGradLoads) wait_vm_lgkm0<0>();  // K / V reads done before P / dS overwrite them
            else wait_vm_lgkm0<2 * C::kDmaKv>();
            barrier();
            score(next_masked(), s0, pa, pa, false);
        };
        auto step = [&](FA3_LDS char* __restrict__ ld, const FA3_LDS char* __restrict__ s1,
                        FA3_LDS char* __restrict__ pwr) {
            top();
            if constexpr (!C::kGradLoads && !kLateIssue) issue(ld);
            __builtin_amdgcn_sched_barrier(0);
            score(next_masked(), s1, pwr, ld, true);
            __builtin_amdgcn_sched_barrier(0);
        };
        FA3_TL(tlu, 0);
        prologue_loads();
        FA3_TL(tlu, 7);
        prologue(st_ld, pds0);
        FA3_TL(tlu, 1);
        int j = 0;
        for (; j + 2 < n_it; j += 2) {
            step(st_ld, st_1, pds1);
            rotate();
            step(st_ld, st_1, pds0);
            rotate();
        }
        if (j + 1 < n_it) step(st_ld, st_1, pds1);
        top();  // matches the gradient waves' last phase
        if (slot >= 0) {
            split_arrive(d, slot >> 1, flag);
            split_end(d, slot >> 1, flag, [] {});
        }
    } else {
        // ---- gradient waves: dV^T and dK^T for D slice(s); wave t owns the
        // (matrix, slice) pairs dkv_pair(t, 0 .. kPpw - 1) over all 64 keys
        // (two 32-key blocks)
        constexpr int kPpw = C::kDB / 2;
        f32x16 acc[kPpw][2];
#pragma unroll
        for (int u = 0; u < kPpw; ++u) {
            acc[u][0] = f32x16{};
            acc[u][1] = f32x16{};
        }
        // A operands (X^T, X = dO or Q) of a tile: [pair][k-step]
        f16x8 xa[kPpw][4], xb[kPpw][4];
        auto read_xt = [&](const FA3_LDS char* st, f16x8 (&xt)[kPpw][4]) {
#pragma unroll
            for (int u = 0; u < kPpw; ++u) {
                const int pu = dkv_pair<D>(t, u);
                const FA3_LDS char* x = st + ((pu & 1) == 0 ? C::kTileBytes : 0);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) xt[u][ks] = tile_read_t<D>(x, pu >> 1, ks, lane);
            }
        };
        // X^T P (or dS) with P / dS read as B operands, keys 32 kb + l32;
        // the wave's pairs share their matrix, hence their B operands.  All B
        // operands of the step are read before the first MFMA, so one LDS
        // round trip covers them all.
        const uint32_t mat = (t >> 1) * C::kPdsBytes;  // P or dS
        auto grad = [&](const f16x8 (&xt)[kPpw][4], const FA3_LDS char* pds) {
            f16x8 bp[4][2];
            const FA3_LDS char* m = pds + mat;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    bp[ks][kb] = lds_read_b128(m, pds_chunk(32 * kb + l32, 2 * ks + h));
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
            set_prio<0>();  // raised for the step's LDS reads (see step)
            // key block 1's operands arrive with their halves exchanged
            // (pds_off4): its products take the A operands exchanged too,
            // copied while block 0's products run
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int u = 0; u < kPpw; ++u)
                        acc[u][kb] = mfma_32x32x16t<kBf16>(kb ? swap_halves(xt[u][ks]) : xt[u][ks],
                                                           bp[ks][kb], acc[u][kb]);
        };
        auto prologue = [&](const FA3_LDS char* __restrict__ s0) {
            wait_vm_lgkm0<2 * C::kDmaKv>();  // the first tile has landed
            barrier();
            read_xt(s0, xa);
            debug_sync<kDebug>();  // the score waves' first operand reads
            debug_sync<kDebug>();  // and P / dS stores
        };
        auto step = [&](FA3_LDS char* __restrict__ ld, const FA3_LDS char* __restrict__ s1,
                        const FA3_LDS char* __restrict__ prd, const f16x8 (&xcur)[kPpw][4],
                        f16x8 (&xnext)[kPpw][4]) {
            top();
            issue(ld);
            __builtin_amdgcn_sched_barrier(0);
            // next tile's operands first: the LDS reads run while the score
            // waves' (higher priority) MFMAs hold the matrix unit, and this
            // wave's MFMAs overlap their softmax instead.  The reads go out at
            // priority 2 (below the score waves' MFMA phase, above their
            // softmax), so they are not held back behind the softmax (P3 -1 %).
            set_prio<2>();
            read_xt(s1, xnext);
            debug_sync<kDebug>();
            grad(xcur, prd);
            debug_sync<kDebug>();
            __builtin_amdgcn_sched_barrier(0);
        };
        auto last = [&](const f16x8 (&xcur)[kPpw][4], const FA3_LDS char* __restrict__ prd) {
            top();
            grad(xcur, prd);
        };
        FA3_TL(tlu, 0);
        prologue_loads();
        FA3_TL(tlu, 7);
        prologue(st_ld);
        FA3_TL(tlu, 1);
        int j = 0;
        for (; j + 2 < n_it; j += 2) {
            step(st_ld, st_1, pds0, xa, xb);
            rotate();
            step(st_ld, st_1, pds1, xb, xa);
            rotate();
        }
        if (j + 1 < n_it) {
            step(st_ld, st_1, pds0, xa, xb);
            last(xb, pds1);
        } else {
            last(xa, pds0);
        }
        FA3_TL(tlu, 2);
        // st_1 is free now: nobody reads it any more, and only the latest
        // issue (into st_ld, or st_2 after a rotate) may still be landing, so
        // it stages the outputs
        if (kHeadSplit) {
            const PartView<D> pv{a.part_dk, a.part_dv, a.scale, d.seqlen,
                                 d.heads_kv * d.hs_chunks, (size_t)d.seqlen * D};
            store_dkv<D, kBf16>(pv, b, pc, kbase, t, lane, acc, st_1);
            FA3_TL_DRAIN();
            FA3_TL(tlu, 3);
            return;
        }
        if (slot < 0) {
            store_dkv<D, kBf16>(d, b, hkv, kbase, t, lane, acc, st_1);
            FA3_TL_DRAIN();
            FA3_TL(tlu, 3);
            return;
        }
        // partial sums of the first piece: [job][wave][2 kPpw accumulator blocks]
        constexpr int kBlk = 2 * kPpw;
        const __amdgpu_buffer_rsrc_t pr = partial_rsrc(d.part_kv, d.part_kv_bytes);
        const uint32_t part = (uint32_t)((slot >> 1) * 4 + t) * (kBlk * 4096);
        f32x16* flat = &acc[0][0];
        if (split_end(d, slot >> 1, flag, [&] { put_partials<kBlk>(pr, part, flat, lane); })) {
            FA3_TL(tlu, 5);
            add_partials<kBlk>(pr, part, flat, lane);
            FA3_TL(tlu, 6);
            store_dkv<D, kBf16>(d, b, hkv, kbase, t, lane, acc, st_1);
        } else {
            FA3_TL(tlu, 4);
        }
        FA3_TL_DRAIN();
        FA3_TL(tlu, 3);
    }
}

// ----------------------------------------------------------------------------
// dQ role
// ----------------------------------------------------------------------------
// Query tile qt of query head hq (KV head hkv) in batch b.  Streams key
// tiles [ka, kb) (the causal diagonal, key tile qt, is masked).  slot: as
// for dkv_role.
template <int D, bool kCausal, bool kBf16, int kRows = 0, bool kLateIssue = false,
          bool kScaled = true, bool kDebug = false, typename DA>
__device__ __forceinline__ void dq_role(const FusedArgs& a, const DA& d, int b, int hq, int hkv, int qt, int ka,
                                        int kb, int slot,
                        FA3_LDS char* smem, int tlu = 0) {
    static_assert(kRows == 0 || kRows == 2, "dQ rows come as -lse2/-delta or max/sum/delta");
    using C = Cfg<D>;
    const int tid = opaque_tid();
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = w & 3;
    const int l16 = lane & 15, g4 = lane >> 4, l32 = lane & 31, h = lane >> 5;

    const int S = d.seqlen;
    const int QT = S / 64;
    const int group = d.group;
    const size_t row0 = ((size_t)b * d.heads_q + hq) * S + qt * 64;  // statistics row
    const size_t q0 = q_elem<D>(d, b, hq, qt * 64);  // this tile's Q / dO / dQ elements
    const int n_kt = kb - ka;

    const int ldr = C::kGradLoads ? t : w;  // as in dkv_role
    const bool loads = !C::kGradLoads || w >= 4;
    FA3_LDS char* ds0 = smem + C::kPdsOff;
    // this query tile's Q (times c when kScaled, below) and dO are staged in
    // the dS area, its -lse2 and -delta in the (otherwise unused) rows slot
    // of stage 0; these loads go out before the rest of the set-up
    uint32_t ld_off[C::kNld], q_off[C::kLoadsPerTile];
    tile_load_offsets<D, C::kLoadsPerTile, true>(q_off, w, lane, d.q_rs);
    load_tile_async(ds0, a.q + q0, q_off, w);
    load_tile_async(ds0 + C::kTileBytes, a.dout + q0, q_off, w);
    load_rows_async<kRows>(smem + 2 * C::kTileBytes, a, row0, w, lane);
    __builtin_amdgcn_sched_barrier(0);
    tile_load_offsets<D, C::kNld>(ld_off, ldr, lane, d.kv_rs);
    const _Float16* kh = d.k + kv_elem<D>(d, b, hkv, 0);
    const _Float16* vh = d.v + kv_elem<D>(d, b, hkv, 0);
    int ld_kt = ka;
    size_t ld_e = (size_t)ka * 64 * d.kv_rs;
    const size_t step_e = (size_t)64 * d.kv_rs;
    auto issue = [&](FA3_LDS char* st) {  // loading waves
        load_tile_async(st, kh + ld_e, ld_off, ldr);
        load_tile_async(st + C::kTileBytes, vh + ld_e, ld_off, ldr);
        if (ld_kt + 1 < kb) {
            ++ld_kt;
            ld_e += step_e;
        }
    };
    auto top = [&]() {
        if (loads) wait_vm_lgkm0<C::kDmaQ>();
        else wait_vm_lgkm0<0>();
        barrier();
    };

    FA3_LDS char* st_ld = smem;
    FA3_LDS char* st_1 = smem + C::kStageBytes;
    FA3_LDS char* st_2 = smem + 2 * C::kStageBytes;
    auto rotate = [&]() {
        FA3_LDS char* x = st_ld;
        st_ld = st_1;
        st_1 = st_2;
        st_2 = x;
    };
    FA3_LDS int* flag = (FA3_LDS int*)(smem + C::kFlagOff);
    FA3_LDS char* ds1 = ds0 + 2 * C::kPdsBytes;
    auto prologue_loads = [&]() {
        // Q, dO and the rows are on their way (issued at the top)
        if (loads) {  // as in dkv_role: Q, dO and the rows first
            issue(st_ld);
            issue(st_1);
            issue(st_2);
        }
        if constexpr (kScaled) {
            // this wave's Q loads have landed once only the later ones (dO,
            // the rows' one load, the three stages) may be in flight
            if (loads) wait_vm_lgkm0<C::kLoadsPerTile + 1 + 3 * C::kDmaQ>();
            else wait_vm_lgkm0<C::kLoadsPerTile + 1>();
            scale_own_chunks<kBf16, C::kLoadsPerTile>(ds0, w, lane, a.scale_log2);
        }
        if (loads) wait_vm_lgkm0<3 * C::kDmaQ>();
        else wait_vm_lgkm0<0>();
        barrier();
    };

    if (w < 4) {
        // ---- score waves: S^T, dP^T, dS^T of keys 16 t .. +16 of each key
        // tile and all 64 query rows (four 16-row blocks rb: rows rb + 4 l16,
        // perm_row); dS goes to LDS.
        // B operands: LDS row 16 rb + l16 (query row rb + 4 l16), D chunk p1_chunk(s, g4)
        f16x8 qf[4][C::kKs], df[4][C::kKs];
        f32x4 nl2[4];            // -lse2 of row rb + 4 l16, the S^T accumulators' start
        f32x4 ndl[4];            // -delta of row rb + 4 l16, the dP^T accumulators' start
        f32x4 sacc[4], pacc[4];  // keys 16 t + 4 g4 + i, rows rb + 4 l16
        auto score = [&](bool masked, const FA3_LDS char* st, FA3_LDS char* ds,
                         FA3_LDS char* ld, bool do_issue) {
            f16x8 ak[C::kKs], av[C::kKs];
            set_prio<3>();
#pragma unroll
            for (int s = 0; s < C::kKs; ++s) {
                const uint32_t off = tile_off<D>(16 * t + l16, p1_chunk<D>(s, g4));
                ak[s] = lds_read_b128(st, off);
                av[s] = lds_read_b128(st + C::kTileBytes, off);
            }
            __builtin_amdgcn_sched_barrier(0);  // as in dkv_role
            if (!C::kGradLoads && kLateIssue && do_issue) issue(ld);
            __builtin_amdgcn_sched_barrier(0);
            debug_sync<kDebug>();
#pragma unroll
            for (int s = 0; s < C::kKs; ++s) {
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    sacc[rb] = mfma_16x16x32<kBf16>(ak[s], qf[rb][s],
                                                    s != 0 ? sacc[rb] : kScaled ? nl2[rb] : f32x4{});
                    pacc[rb] = mfma_16x16x32<kBf16>(av[s], df[rb][s], s == 0 ? ndl[rb] : pacc[rb]);
                }
            }
            set_prio<0>();
            // sacc = S^T c - lse2 (kScaled: Q c, -lse2 seed), else S^T
            float p[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int rb = e >> 2, i = e & 3;
                const float x = kScaled ? sacc[rb][i] : sacc[rb][i] * a.scale_log2 + nl2[rb][0];
                p[e] = fast_exp2(x) * pacc[rb][i];
            }
            if (masked) {  // causal diagonal tile
                __asm__ volatile("" ::: "memory");  // keep this a branch
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (16 * t + 4 * g4 + (e & 3) > (e >> 2) + 4 * l16) p[e] = 0.f;
            }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                f16x4 dv;
#pragma unroll
                for (int i = 0; i < 4; ++i) dv[i] = to16<kBf16>(p[4 * rb + i]);
                lds_write_b64(ds, pds_off4(rb + 4 * l16, 4 * t + g4), dv);
            }
            debug_sync<kDebug>();
        };
        auto prologue = [&](FA3_LDS char* __restrict__ s0, FA3_LDS char* __restrict__ pa) {
            const FA3_LDS float* rows = (const FA3_LDS float*)(s0 + 2 * C::kTileBytes);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int r = rb + 4 * l16;  // query row, held at LDS row 16 rb + l16
#pragma unroll
                for (int s = 0; s < C::kKs; ++s) {
                    const uint32_t off = tile_off<D>(16 * rb + l16, p1_chunk<D>(s, g4));
                    qf[rb][s] = lds_read_b128(pa, off);
                    df[rb][s] = lds_read_b128(pa + C::kTileBytes, off);
                }
                float nl, n;
                if constexpr (kRows == 0) {
                    nl = rows[r];
                    n = rows[64 + r];
                } else {  // exp2((x - max) c) / sum = exp2(x c - (max c + log2 sum))
                    nl = -(rows[r] * a.scale_log2 + __log2f(rows[64 + r]));
                    n = -rows[128 + r];
                }
                nl2[rb] = f32x4{nl, nl, nl, nl};
                ndl[rb] = f32x4{n, n, n, n};
            }
            if constexpr (C::kGradLoads) wait_vm_lgkm0<0>();  // Q / dO reads done before dS overwrites them
            else wait_vm_lgkm0<2 * C::kDmaQ>();
            barrier();
            score(kCausal && ka == qt, s0, pa, pa, false);
        };
        // step j computes the dS of key tile ka + j + 1
        auto step = [&](bool masked, FA3_LDS char* __restrict__ ld,
                        const FA3_LDS char* __restrict__ s1, FA3_LDS char* __restrict__ pwr) {
            top();
            if constexpr (!C::kGradLoads && !kLateIssue) issue(ld);
            __builtin_amdgcn_sched_barrier(0);
            score(masked, s1, pwr, ld, true);
            __builtin_amdgcn_sched_barrier(0);
        };
        FA3_TL(tlu, 0);
        prologue_loads();
        FA3_TL(tlu, 7);
        prologue(st_ld, ds0);
        FA3_TL(tlu, 1);
        int j = 0;
        for (; j + 2 < n_kt; j += 2) {
            step(kCausal && ka + j + 1 == qt, st_ld, st_1, ds1);
            rotate();
            step(kCausal && ka + j + 2 == qt, st_ld, st_1, ds0);
            rotate();
        }
        if (j + 1 < n_kt) step(kCausal && ka + j + 1 == qt, st_ld, st_1, ds1);
        top();  // matches the gradient waves' last phase
        if (slot >= 0) {
            split_arrive(d, d.n_split + (slot >> 1), flag);
            split_end(d, d.n_split + (slot >> 1), flag, [] {});
        }
    } else {
        // ---- gradient waves: dQ^T slice(s) over query rows; D = 128: slice
        // t, both 32-row blocks; D = 64: slice t / 2, row block t % 2
        constexpr int kRb = C::kDB / 2;  // 32-row blocks per wave
        const int db = C::kDB == 4 ? t : t >> 1;
        const int rb0 = C::kDB == 4 ? 0 : t & 1;
        f32x16 acc[kRb];
#pragma unroll
        for (int r = 0; r < kRb; ++r) acc[r] = f32x16{};
        f16x8 xa[4], xb[4];  // K^T of a key tile, per k-step
        // row block 1's dS operands arrive with their halves exchanged
        // (pds_off4): at D 64 the wave's only block is rb0 and its K^T
        // operands are read exchanged; at D 128 block 1 takes swap_halves
        const bool swap_read = kRb == 1 && rb0 == 1;
        auto read_xt = [&](const FA3_LDS char* st, f16x8 (&xt)[4]) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) xt[ks] = tile_read_t<D>(st, db, ks, lane, swap_read);
        };
        auto grad = [&](const f16x8 (&xt)[4], const FA3_LDS char* ds) {
            f16x8 bd[4][kRb];  // all B operands first: one LDS round trip
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < kRb; ++r)
                    bd[ks][r] = lds_read_b128(ds, pds_chunk(32 * (rb0 + r) + l32, 2 * ks + h));
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
            set_prio<0>();  // as in dkv_role
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < kRb; ++r)
                    acc[r] = mfma_32x32x16t<kBf16>(kRb == 2 && r == 1 ? swap_halves(xt[ks]) : xt[ks],
                                                   bd[ks][r], acc[r]);
        };
        auto prologue = [&](const FA3_LDS char* __restrict__ s0) {
            wait_vm_lgkm0<2 * C::kDmaQ>();
            barrier();
            read_xt(s0, xa);
            debug_sync<kDebug>();  // as in dkv_role
            debug_sync<kDebug>();
        };
        auto step = [&](FA3_LDS char* __restrict__ ld, const FA3_LDS char* __restrict__ s1,
                        const FA3_LDS char* __restrict__ prd, const f16x8 (&xcur)[4],
                        f16x8 (&xnext)[4]) {
            top();
            issue(ld);
            __builtin_amdgcn_sched_barrier(0);
            // as in dkv_role
            set_prio<2>();
            read_xt(s1, xnext);
            debug_sync<kDebug>();
            grad(xcur, prd);
            debug_sync<kDebug>();
            __builtin_amdgcn_sched_barrier(0);
        };
        auto last = [&](const f16x8 (&xcur)[4], const FA3_LDS char* __restrict__ prd) {
            top();
            grad(xcur, prd);
        };
        FA3_TL(tlu, 0);
        prologue_loads();
        FA3_TL(tlu, 7);
        prologue(st_ld);
        FA3_TL(tlu, 1);
        int j = 0;
        for (; j + 2 < n_kt; j += 2) {
            step(st_ld, st_1, ds0, xa, xb);
            rotate();
            step(st_ld, st_1, ds1, xb, xa);
            rotate();
        }
        if (j + 1 < n_kt) {
            step(st_ld, st_1, ds0, xa, xb);
            last(xb, ds1);
        } else {
            last(xa, ds0);
        }
        FA3_TL(tlu, 2);
        // st_1 is free now (see dkv_role) and stages the outputs
        if (slot < 0) {
            store_dq<D, kBf16>(d, q0, t, lane, acc, st_1);
            FA3_TL_DRAIN();
            FA3_TL(tlu, 3);
            return;
        }
        // partial sums of the first piece: [job][wave][kRb accumulator blocks]
        const __amdgpu_buffer_rsrc_t pr = partial_rsrc(d.part_q, d.part_q_bytes);
        const uint32_t part = (uint32_t)((slot >> 1) * 4 + t) * (kRb * 4096);
        if (split_end(d, d.n_split + (slot >> 1), flag,
                      [&] { put_partials<kRb>(pr, part, acc, lane); })) {
            FA3_TL(tlu, 5);
            add_partials<kRb>(pr, part, acc, lane);
            FA3_TL(tlu, 6);
            store_dq<D, kBf16>(d, q0, t, lane, acc, st_1);
        } else {
            FA3_TL(tlu, 4);
        }
        FA3_TL_DRAIN();
        FA3_TL(tlu, 3);
    }
}

// Between two units of one workgroup (split plan, persistent default plan):
// every wave's LDS accesses are done and every load of the first unit has
// landed, but the gradient waves' output stores -- the last kStores
// vector-memory operations they issued -- may still be in flight: the
// vector-memory operations of a wave complete in issue order, so
// vmcnt(kStores) covers every load before them.  kStores is at most the
// number of stores the first unit's epilogue issues (store_dkv: 4 (D / 64),
// store_dq: 2 (D / 64), more with fp32 outputs).  The score waves wait for
// everything (their only stores are the split words and the queue pop).
template <int kStores>
__device__ __forceinline__ void unit_gap() {
    if (threadIdx.x >= 4 * kWave) wait_vm_lgkm0<kStores>();
    else wait_vm_lgkm0<0>();
    barrier();
}

// Job id -> (group, position in the group); see the job map below.
template <typename A>
__host__ __device__ __forceinline__ void job_of(const A& a, int id, int& g, int& pos) {
    const int mode = a.xcd_mode;
    const int parts = mode & 255;
    const bool interleave = (mode >> 8) != 0;
    if (parts > 0) {
        const int xcd = id & 7;
        const int n = id >> 3;
        const int hi = fdiv(a.div_radix, n), lo = n - hi * a.map_radix;
        // j: the virtual group among this XCD's, k: the position in its part
        const int j = interleave ? lo : hi, k = interleave ? hi : lo;
        const int v = xcd * a.xcd_vgroups + j;  // virtual group = (group, part)
        g = fdiv(a.div_parts, v);
        pos = v - g * parts + parts * k;
    } else if (interleave) {
        pos = fdiv(a.div_groups, id);
        g = id - pos * a.n_groups;
    } else {
        g = fdiv(a.div_jpg, id);
        pos = id - g * a.jobs_per_group;
    }
}

// Job map.  Jobs are grouped by (batch, kv head) -- a group's dKV jobs and
// the dQ jobs of its query heads touch only that head's Q, dO, K, V.  The
// hardware deals consecutive workgroup ids round-robin to the 8 XCDs; when
// the shape allows, block id -> (xcd, position) is arranged so that each XCD
// runs whole parts of groups, keeping a head's tiles in one L2.
//
// Default plan: the order of a group's jobs is longest first, so that the
// short jobs come last and even out the workgroups' finishing times (list
// scheduling).  Non-causal, or G > 1: positions p < QT are the dKV jobs of
// key tiles p, then p = QT + G L + r the dQ job of query head r at query
// tile QT - 1 - L -- a dKV job streams G heads' tiles and a dQ step is ~0.75
// of a dKV step, so every dKV job is at least as long as any dQ job but the
// causal tail (A/B against the level order below: P4 -2.2 to -2.8 %, P5
// -0.7 to -1.0 %, B2 Hq32 Hkv8 S4096 full -6.2 %).  Causal with G = 1 (the
// kOrder 1 instantiations): level L holds the dKV job of key tile L (p =
// 2 L) and the dQ job of query tile QT - 1 - L (p = 2 L + 1), two lists of
// the same slope merged (the role order measured +0.8 to +1.7 % there, B1
// H16 S8192 D128, and a runtime choice inside one instantiation +0.8 %).
//
// Head-split default plan (part_dk set; GQA with so few groups that one dKV
// job, G QT steps, would outlast the average workgroup): the dKV jobs come
// hs_chunks per key tile, p = hs_chunks L + c for key tile L and chunk c of
// hs_heads query heads, each writing the chunk's fp32 contribution to dK /
// dV; gqa_reduce_kernel then sums the hs_chunks contributions of each KV
// head in chunk order (deterministic).
//
// Split plan (bal_m = M = QT / 2 > 0; causal, G = 1, few jobs): the causal
// jobs run 1 .. QT steps, so one long job would set the kernel's length.
// The long jobs (dKV key tiles x < M, dQ query tiles M + x) are cut into a
// head piece and a remainder, and the short jobs are spread over the
// workgroups that have time for them.  Each workgroup has a descriptor
// (split_desc) with its kind, x, group, head length and short job (a
// whole dQ job of query tile < M, if the plan places one there):
//   kind 0:  dKV key tile M + x (whole), the short job, then the remainder
//            of dQ query tile M + x (key tiles len .. M + x);
//   kind 1:  the short job, then the remainder of dKV key tile x (query
//            tiles x + len .. QT - 1);
//   kind 2:  the short job, then the head piece of dKV key tile x (len
//            tiles);
//   kind 3:  the short job, then the head piece of dQ query tile M + x
//            (len tiles).
// The host picks the head lengths and the short jobs' places from a cost
// model of the steps, prologues and epilogues, so that the workgroups
// finish together (a length covering the whole job leaves it unsplit).
//
// kSplit selects the split plan (a separate instantiation: its units issue
// their loads at a different point of the step, see dkv_role's score).
// kScaled: the score waves' resident operands are multiplied by scale_log2
// (default plan, launches with scale_log2 <= 1).  The split plan keeps them
// unscaled: its units are short (8 to 32 steps), and the scaling in each
// unit's prologue cost about what its steps save (P3 +0.5 %).
// kDebug selects the race-check instantiation (see debug_sync).  kAfter: a
// split plan that places short jobs after pieces (only such plans run the
// code for them).  kOrder: the default plan's job order (see the job map) --
// 0 dKV jobs first, 1 level by level (causal, G = 1), 2 dKV jobs first, one
// per query head (head split).
template <int D, bool kCausal, bool kBf16, bool kSplit, bool kScaled, bool kDebug = false,
          bool kAfter = false, int kOrder = 0>
__global__ __launch_bounds__(kThreads, 1) void bwd_main_kernel(FusedArgs a) {
    static_assert(kCausal || !kSplit, "the split plan is causal");
    static_assert(kSplit || !kAfter, "short jobs after pieces are a split-plan placement");
    static_assert(!kSplit || kOrder == 0, "the job orders are default-plan orders");
    static_assert(!(kScaled && kSplit), "the split plan runs unscaled");
    __shared__ __attribute__((aligned(1024))) char smem_raw[Cfg<D>::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;
#ifdef FA3_TIMELINE
    if (a.tl != nullptr && threadIdx.x == 0) {
        unsigned long long* p = a.tl + (size_t)blockIdx.x * 64;
        p[0] = __builtin_amdgcn_s_memrealtime();
        p[30] = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID
        p[31] = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // XCC_ID
    }
#endif
    const int group = a.group;
    const int QT = a.seqlen / 64;
    int g, pos;
    if constexpr (kSplit) {
        // the workgroup's descriptor and every argument the units' set-up
        // reads before its first loads, requested together: without the asm
        // the compiler issues them branch by branch, one dependent round
        // trip each (P3: ~1.6 us from entry to the first load)
        const uint32_t desc = a.split_desc[blockIdx.x];
        __asm__ volatile("" ::"s"(desc), "s"(a.div_hkv.mul), "s"(a.div_hkv.shr), "s"(a.heads_kv),
                         "s"(a.heads_q), "s"(a.group), "s"(a.bal_m), "s"(a.seqlen), "s"(a.q_rs),
                         "s"(a.q_hs), "s"(a.kv_rs), "s"(a.kv_hs), "s"(a.q), "s"(a.k), "s"(a.v),
                         "s"(a.dout), "s"(a.nlse2), "s"(a.ndelta));
        const int kind = desc & 3, x = (desc >> 2) & 127, len = (desc >> 15) & 511;
#ifdef FA3_TIMELINE
        if (a.tl != nullptr && threadIdx.x == 0) a.tl[(size_t)blockIdx.x * 64 + 29] = desc;
#endif
        // (a plan with short jobs after pieces runs the kAfter instantiation)
        const int sfield = desc >> 24;
        const bool after = kAfter && sfield != kNoShort && sfield >= kShortAfter;
        const int shrt =
            kAfter && sfield != kNoShort ? sfield & (kShortAfter - 1) : sfield;
        g = (desc >> 9) & 63;
        // G = 1: group g is query head g (and KV head g) of batch b
        const int b = fdiv(a.div_hkv, g), h = g - b * a.heads_kv;
        const int M = a.bal_m;
        const int job0 = g * M;
        if (kind == 0) {
            // dKV key tile M + x whole, the short dQ job (query tile shrt,
            // whole) if placed before, then the remainder of dQ query tile M + x
            const int nq = M + x + 1, lq = len;
            debug_poison<D, kDebug>(smem);
            dkv_role<D, kCausal, kBf16, 0, true, false, kDebug>(a, a, b, h, M + x, M + x, QT, -1,
                                                                smem, 0);
            if (shrt != kNoShort && !after) {
                unit_gap<4 * (D / 64)>();
                debug_poison<D, kDebug>(smem);
                dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(a, a, b, h, h, shrt, 0,
                                                                   shrt + 1, -1, smem, 1);
            }
            if (lq < nq) {
                if (shrt != kNoShort && !after) unit_gap<2 * (D / 64)>();
                else unit_gap<4 * (D / 64)>();
                debug_poison<D, kDebug>(smem);
                dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(
                    a, a, b, h, h, M + x, lq, nq, 2 * (job0 + x) + 1, smem,
                    (shrt != kNoShort && !after) ? 2 : 1);
            }
        } else if (kind == 1) {
            // the short dQ job (query tile shrt, whole) if placed before, then the
            // remainder of dKV key tile x
            const int nkv = QT - x, lkv = len;
            if (shrt != kNoShort && !after) {
                debug_poison<D, kDebug>(smem);
                dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(a, a, b, h, h, shrt, 0,
                                                                   shrt + 1, -1, smem, 0);
                if (lkv < nkv) unit_gap<2 * (D / 64)>();
            }
            if (lkv < nkv) {
                debug_poison<D, kDebug>(smem);
                dkv_role<D, kCausal, kBf16, 0, true, false, kDebug>(
                    a, a, b, h, x, x + lkv, QT, 2 * (job0 + x) + 1, smem,
                    (shrt != kNoShort && !after) ? 1 : 0);
            }
        } else if (kind == 2) {
            // the short dQ job if placed before, then the head piece (or all) of dKV
            // key tile x
            const int nkv = QT - x, lkv = len;
            if (shrt != kNoShort && !after) {
                debug_poison<D, kDebug>(smem);
                dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(a, a, b, h, h, shrt, 0,
                                                                   shrt + 1, -1, smem, 0);
                unit_gap<2 * (D / 64)>();
            }
            debug_poison<D, kDebug>(smem);
            dkv_role<D, kCausal, kBf16, 0, true, false, kDebug>(
                a, a, b, h, x, x, x + min(lkv, nkv), lkv < nkv ? 2 * (job0 + x) : -1, smem,
                (shrt != kNoShort && !after) ? 1 : 0);
        } else {
            // the short dQ job (query tile shrt, whole) if placed before, then the
            // head piece (or all) of dQ query tile M + x
            const int nq = M + x + 1, lq = len;
            if (shrt != kNoShort && !after) {
                debug_poison<D, kDebug>(smem);
                dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(a, a, b, h, h, shrt, 0,
                                                                   shrt + 1, -1, smem, 0);
                unit_gap<2 * (D / 64)>();
            }
            debug_poison<D, kDebug>(smem);
            dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(
                a, a, b, h, h, M + x, 0, min(lq, nq), lq < nq ? 2 * (job0 + x) : -1, smem,
                (shrt != kNoShort && !after) ? 1 : 0);
        }
        // a short job placed after the piece (kAfter instantiations only):
        // it fills the time a piece that published first would wait for its
        // partner's add.  Everything it needs is decoded again from the
        // descriptor and read again from the arguments (the empty asm), so
        // that nothing but the descriptor is held in scalar registers across
        // the piece.  The gap waits as after a dQ unit: that leaves fewer
        // stores in flight than a gap after a dKV unit allows, so it is safe
        // after either.
        if constexpr (kAfter) {
            uint32_t dd = desc;
            __asm__ volatile("" : "+s"(dd));
            const int sa = dd >> 24;
            if (sa != kNoShort && sa >= kShortAfter) {
                KArgs* ap = &kargs();
                __asm__ volatile("" : "+s"(ap));
                const int ga = (dd >> 9) & 63;
                const int ba = fdiv(ap->div_hkv, ga), ha = ga - ba * ap->heads_kv;
                const int st = sa - kShortAfter;
                unit_gap<2 * (D / 64)>();
                debug_poison<D, kDebug>(smem);
                dq_role<D, kCausal, kBf16, 0, true, false, kDebug>(a, a, ba, ha, ha, st, 0, st + 1,
                                                                   -1, smem, 3);
            }
        }
        return;
    }
    // d: the argument segment, for the job's set-up (divisors); the roles
    // read the rest from a
    // timeline build: the unit slot of the workgroup's job (the first three
    // jobs, then the latest one in slot 3); the product build stamps nothing
#ifdef FA3_TIMELINE
    int tl_job = 0;
#define FA3_TL_JOB (tl_job < 3 ? tl_job : 3)
#else
#define FA3_TL_JOB 0
#endif
    auto run = [&](KArgs& d, int id) {
        job_of(d, id, g, pos);
        // the job's level (key tile of a dKV job; a dQ job's query tile is
        // QT - 1 - level) and slot (0: dKV, r > 0: dQ of query head r - 1)
        int level, slot, hl = 0;  // hl: the dKV job's chunk of query heads (kOrder 2)
        if constexpr (kOrder == 1) {
            level = fdiv(d.div_g1, pos);
            slot = pos - level * (group + 1);
        } else {
            // dKV jobs first: QT of them (kOrder 2: hs_chunks per level, one
            // per chunk of query heads), then G dQ jobs per level
            const int n_dkv = kOrder == 2 ? d.hs_chunks * QT : QT;
            if (pos < n_dkv) {
                if constexpr (kOrder == 2) {
                    level = fdiv(d.div_chunks, pos);
                    hl = pos - level * d.hs_chunks;
                } else {
                    level = pos;
                }
                slot = 0;
            } else {
                const int r = pos - n_dkv;
                level = fdiv(d.div_group, r);
                slot = 1 + r - level * group;
            }
        }
        const int b = fdiv(d.div_hkv, g), hkv = g - b * a.heads_kv;
        debug_poison<D, kDebug>(smem);
        if (slot == 0) {
            dkv_role<D, kCausal, kBf16, 0, false, kScaled, kDebug, kOrder == 2>(
                a, d, b, hkv, level, kCausal ? level : 0, QT, -1, smem, FA3_TL_JOB,
                kOrder == 2 ? hkv * group + hl * d.hs_heads : 0,
                kOrder == 2 ? hkv * d.hs_chunks + hl : 0);
        } else {
            const int qt = QT - 1 - level;
            dq_role<D, kCausal, kBf16, 0, false, kScaled, kDebug>(
                a, d, b, hkv * group + slot - 1, hkv, qt, 0, kCausal ? qt + 1 : QT, -1, smem,
                FA3_TL_JOB);
        }
    };
#undef FA3_TL_JOB
    // Persistent plan: thread 0 (a score wave, done with the job before the
    // gradient waves' last products and epilogue) pops the next id while
    // they finish, and passes it on through LDS; the gap's barrier
    // publishes it.  Otherwise (persist == 0) the workgroup runs its one job.
    // Queue q holds the ids q + 8 (k + persist / 8), k = 0, 1, .. below
    // n_jobs (its first persist / 8 ids are the static first jobs of the
    // workgroups q, q + 8, ..).  A workgroup drains its own XCD's queue,
    // then steals from the others in turn (the XCDs do not run at one speed:
    // 7 % apart at P4, 17 % at P5 without stealing), and leaves when every
    // queue is dry.  Every id below n_jobs is popped once.  The last
    // workgroup to leave (the exit count, kept on queue 0's line) puts all
    // counters back to 0, so the queues are clean for the next launch even
    // without the preprocess's clearing.
    const int n_static = a.persist >> 3;
    int qcur = blockIdx.x & 7;  // thread 0: the queue being drained
    FA3_LDS int* next = (FA3_LDS int*)(smem + Cfg<D>::kFlagOff + 64);
    int id = blockIdx.x;
    for (;;) {
        KArgs* ap = &kargs();
        __asm__ volatile("" : "+s"(ap));
        run(*ap, id);
#ifdef FA3_TIMELINE
        ++tl_job;
#endif
        if (a.persist == 0) return;
        if (threadIdx.x == 0) {
            int nid = -1;
            for (int tries = 0; tries < kQueues && nid < 0; ++tries) {
                const unsigned int k = __hip_atomic_fetch_add(a.queue + kQueueStride * qcur, 1u,
                                                              __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
                const long long cand = qcur + 8 * ((long long)k + n_static);
                if (cand < a.n_jobs) nid = (int)cand;
                else qcur = (qcur + 1) & 7;
            }
            *next = nid;
        }
        unit_gap<2 * (D / 64)>();
        id = *next;
        if (id < 0) break;
    }
    if (threadIdx.x == 0) {
        // every pop of this workgroup has returned before its exit counts
        unsigned int* exits = a.queue + kQueueExitWord;
        if (__hip_atomic_fetch_add(exits, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (unsigned int)a.persist - 1) {
            for (int q = 0; q < kQueues; ++q)
                __hip_atomic_store(a.queue + kQueueStride * q, 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(exits, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Single-role grids of the dK/dV and dQ components (causal, one query head
// per KV head, fp32 outputs): one job per key tile (kRole 1, row statistics
// from the packed sidecar) or per query tile (kRole 2, from max / sum /
// delta), longest first.  No workspace: the statistics are folded in LDS.
// The operands stay unscaled (any softmax scale; these entries are not the
// fast path).
template <int D, int kRole>
__global__ __launch_bounds__(kThreads, 1) void bwd_component_kernel(FusedArgs a) {
    __shared__ __attribute__((aligned(1024))) char smem_raw[Cfg<D>::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;
    int g, pos;
    job_of(a, blockIdx.x, g, pos);
    // one query head per KV head: group g is head h of batch b
    const int b = fdiv(a.div_hkv, g), h = g - b * a.heads_kv;
    const int QT = a.seqlen / 64;
    if constexpr (kRole == 1) {
        dkv_role<D, true, false, 1, false, false>(a, a, b, h, pos, pos, QT, -1, smem);
    } else {
        const int qt = QT - 1 - pos;
        dq_role<D, true, false, 2, false, false>(a, a, b, h, h, qt, 0, qt + 1, -1, smem);
    }
}

// Head-split plan: dK / dV of KV head hkv = the sum, in chunk order, of the
// fp32 contributions part[b][hkv chunks + c][:][:] of its chunks of query
// heads, rounded once to the outputs' type.  Block (x, bh): 1024 elements of
// KV head bh = b Hkv + hkv, four per thread.  HBM-bound: reads `chunks` fp32
// values per 16-bit value written, for dK and dV.
template <int D, bool kBf16>
__global__ __launch_bounds__(256) void gqa_reduce_kernel(
    const float* __restrict__ part_dk, const float* __restrict__ part_dv, _Float16* __restrict__ dk,
    _Float16* __restrict__ dv, int heads_kv, int chunks, int seqlen, int kv_rs, int kv_hs) {
    const int i = blockIdx.x * 256 + threadIdx.x;  // 4-element chunk of the head
    if (i >= seqlen * (D / 4)) return;
    const int bh = blockIdx.y;
    const int b = bh / heads_kv, hkv = bh - b * heads_kv;
    const int sq = i / (D / 4), c = i % (D / 4);
    const size_t head = (size_t)seqlen * D;
    const size_t src = (size_t)bh * chunks * head + 4 * (size_t)i;
    f32x4 sk = *(const f32x4*)(part_dk + src), sv = *(const f32x4*)(part_dv + src);
    for (int r = 1; r < chunks; ++r) {
        sk += *(const f32x4*)(part_dk + src + r * head);
        sv += *(const f32x4*)(part_dv + src + r * head);
    }
    const size_t dst = (size_t)b * heads_kv * head + (size_t)hkv * kv_hs + (size_t)sq * kv_rs + 4 * c;
    f16x4 ok, ov;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        ok[e] = to16<kBf16>(sk[e]);
        ov[e] = to16<kBf16>(sv[e]);
    }
    *(f16x4*)(dk + dst) = ok;
    *(f16x4*)(dv + dst) = ov;
}

// Instantiation of the main kernel for a launch: head dim, causal, 16-bit
// type, split plan, scaled resident operands, race check.
template <int D, bool kDebug>
void launch_dd(const FusedArgs& a, bool causal, bool bf16, hipStream_t stream) {
    const dim3 grid(a.persist > 0 ? a.persist : a.n_groups * a.jobs_per_group);
    const dim3 block(kThreads);
    const bool split = a.bal_m > 0;  // causal only (plan_workspace)
    // the split plan's instantiation with the code for short jobs after
    // pieces, when the plan places one there
    bool after = false;
    for (int i = 0; split && i < a.n_jobs; ++i) {
        const int sf = (int)(a.split_desc[i] >> 24);
        after = after || (sf != kNoShort && sf >= kShortAfter);
    }
    // K c / Q c cannot overflow fp16 when c <= 1
    const bool scaled = a.scale_log2 <= 1.f;
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, stream, a); };
    // the default plan's job order: 2 head split (the plan set part_dk), 1
    // level by level (causal, G = 1), else 0
    const int order = a.part_dk != nullptr ? 2 : causal && a.group == 1 ? 1 : 0;
    auto dflt = [&](auto bf, auto cz) {
        constexpr bool kB = decltype(bf)::value, kC = decltype(cz)::value;
        auto pick = [&](auto ord) {
            constexpr int kO = decltype(ord)::value;
            go(scaled ? bwd_main_kernel<D, kC, kB, false, true, kDebug, false, kO>
                      : bwd_main_kernel<D, kC, kB, false, false, kDebug, false, kO>);
        };
        if (order == 2) pick(std::integral_constant<int, 2>{});
        else if constexpr (kC) {
            if (order == 1) pick(std::integral_constant<int, 1>{});
            else pick(std::integral_constant<int, 0>{});
        } else {
            pick(std::integral_constant<int, 0>{});
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (split) {
        if (bf16) go(after ? bwd_main_kernel<D, true, true, true, false, kDebug, true>
                           : bwd_main_kernel<D, true, true, true, false, kDebug, false>);
        else go(after ? bwd_main_kernel<D, true, false, true, false, kDebug, true>
                      : bwd_main_kernel<D, true, false, true, false, kDebug, false>);
    } else if (bf16) {
        if (causal) dflt(T{}, T{});
        else dflt(T{}, F{});
    } else {
        if (causal) dflt(F{}, T{});
        else dflt(F{}, F{});
    }
}

}  // namespace

// The race-check instantiations (fa3_bwd_main_debug.hip).
void launch_race_check(const FusedArgs& a, int head_dim, bool causal, bool bf16,
                       hipStream_t stream);

}  // namespace fa3
