// Main FA3 backward kernel for gfx950 (replaces the reference's fused 5-GEMM
// kernel and its dQ / GQA-dKV reductions: src/fused_bwd_kernel.cpp:1362-1671,
// src/fused_bwd_dq_reduce.cpp:27-109, and the legacy dKV / dQ kernels
// src/dkv_kernel.cpp:957-1085, src/dq_kernel.cpp:794-953).
//
// Two job roles; every output element has one writer:
//
//  * dKV job -- owns a 64-key tile of one KV head; streams every 64-row query
//    tile that can see it (causal: from the diagonal on) of every query head
//    of its GQA group:
//        S = Q K^T, dP = dO V^T, P = exp2(S c - lse2), dS = P (dP - delta),
//        dV^T += dO^T P, dK^T += Q^T dS                  (4 GEMMs per tile)
//  * dQ job -- owns a 64-row query tile of one query head; streams the key
//    tiles it sees, recomputing S^T and dP^T:
//        dQ^T += K^T dS^T                                (3 GEMMs per tile)
//
// The softmax scale is folded out of dS and applied once to dK and dQ.
//
// A workgroup is 4 waves, one per SIMD, and every wave runs the whole chain
// for its share of the step's tile pair, so P and dS never leave registers:
//  * dKV: wave w owns query rows 16 w .. 16 w + 15 of the streamed tile.  It
//    forms S and dP of those rows against all 64 keys with
//    v_mfma_f32_16x16x32 (K and V held in registers as B operands), then
//    P and dS; v_permlane16_swap turns their 16x16 accumulator layout into
//    the 32x32x16 operand layout (keys x its 16 rows), and the wave adds its
//    rows' share of dV^T and dK^T (64 keys x D) with v_mfma_f32_32x32x16,
//    the streamed tile's transposed operand read with ds_read_b64_tr_b16.
//    Each wave thus holds a partial dK / dV over its rows; the job's
//    epilogue adds the four partials through LDS.
//  * dQ: wave w owns keys 16 w .. 16 w + 15 of the streamed key tile; Q and
//    dO of the job's 64 rows are held in registers as B operands; its dS^T
//    feeds dQ^T (D x 64 rows) over its 16 keys, and the epilogue adds the
//    four partials.
// Every global read of the loop is a direct-to-LDS load (global_load_lds)
// into one of three stages, issued two steps ahead.  The issue pattern is
// the same every step (a finished stream re-loads its last tile into a stage
// nobody reads), so every wait is a constant count.
//
// Row statistics: with the natural-log LSE input (v2), lse2 = LSE log2 e and
// delta = rowsum(dO * O) are formed in the kernel -- the dKV job streams O
// beside Q and dO, the dQ job loads its own O tile and also writes delta
// (softmax_d) -- so a backward is one launch.  The other sources (a
// preprocess pass's lse2 / -delta arrays, the reference's packed sidecar,
// raw max / sum / delta arrays) serve the legacy and component entries.
//
// Split plan (causal, one query head per KV head, few jobs): long jobs are
// cut in two pieces run by different workgroups; see bwd_main_kernel.
#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"

#include <atomic>
#include <chrono>
#include <random>
#include <type_traits>

namespace fa3 {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxBalM = 128;  // split plan: at most 512 jobs, so M = QT / 2 <= 128

// Row-statistics source of a role (template parameter kRows).
enum : int {
    kRowsArrays = 0,  // lse2 and -delta arrays written by a preprocess pass
    kRowsPacked = 1,  // packed sidecar [max_log2, inv_sum, delta] (dKV only)
    kRowsMaxSum = 2,  // raw row max, row sum and delta arrays (dQ only)
    kRowsInline = 3,  // natural-log LSE; delta = rowsum(dO * O) formed here
};

struct MainArgs {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    const _Float16* dout;
    const _Float16* out;   // O (kRowsInline)
    const float* lse;      // natural-log LSE [B*Hq*S] (kRowsInline)
    const float* lse2;     // [B*Hq*S] (kRowsArrays)
    const float* ndelta;   // [B*Hq*S], -delta (kRowsArrays)
    const float* packed;   // [B*Hq*S][3] (kRowsPacked)
    const float* smax;     // (kRowsMaxSum)
    const float* ssum;
    const float* delta_in;
    float* delta_out;      // softmax_d written by the dQ jobs (kRowsInline; may be null)
    void* dq;              // the inputs' 16-bit type, or fp32 when out_f32
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
    // job map: n_groups (batch, kv head) groups of jobs_per_group jobs; with
    // xcd_parts > 0 each group is split into xcd_parts interleaved parts of
    // part_len jobs and whole parts are pinned to one XCD.
    int n_groups;
    int jobs_per_group;
    int xcd_parts;
    int part_len;
    float scale_log2;
    float scale;
    // split plan (bal_m > 0): head-piece lengths (tiles) of the long jobs,
    // x in [0, bal_m): dKV job of key tile x and dQ job of query tile bal_m +
    // x; a length covering the whole job means that job is not split.
    int bal_m;
    uint16_t head_kv[kMaxBalM];
    uint16_t head_q[kMaxBalM];
    // Split-job synchronisation (see split_arrive / split_end): per split job
    // an arrival word and a ready word, compared with this launch's epoch, so
    // nothing needs clearing between launches.  dKV jobs first, then dQ jobs.
    unsigned long long epoch;
    unsigned long long* sync;
    unsigned long long* err;  // set to epoch when a split wait gives up
    int spin_limit;
    int n_split;              // split jobs per role
    float* part_kv;           // [job][wave][tile][4][lane][4] fp32
    float* part_q;
    uint32_t part_kv_bytes;
    uint32_t part_q_bytes;
};

// MainArgs as seen in the kernel-argument segment (constant address space).
typedef __attribute__((address_space(4))) const MainArgs KernArgs;

template <int D>
struct Cfg {
    static constexpr int kTileBytes = 64 * D * 2;  // one [64][D] 16-bit tile
    static constexpr int kRowsBytes = 1024;        // statistics of 64 rows (768 B used)
    // stage: tiles A, B, C (dKV: Q, dO, O; dQ: K, V) and the rows block
    static constexpr int kStageBytes = 3 * kTileBytes + kRowsBytes;
    static constexpr int kRowsOff = 3 * kTileBytes;
    static constexpr int kStages = 3;
    static constexpr int kKs = D / 32;       // 16x16x32 k-steps over D = 32-wide D blocks
    static constexpr int kChunks = D / 8;    // 16-byte chunks per row
    static constexpr int kLd = kTileBytes / (kWaves * 1024);  // 1 KiB loads per wave and tile
    static constexpr int kTiles = 2 * kKs;   // 32x32 accumulator tiles per 64 x D matrix
    static constexpr int kOwn = kTiles / 4;  // tiles a wave owns in the epilogue
    // dKV P / dS operand exchange, 4 KiB per wave: at D 128 in the stage's
    // O rows (see dkv_role), at D 64 in an area of its own
    static constexpr int kXchgOff = kStages * kStageBytes;
    static constexpr int kXchgBytes = D == 128 ? 0 : 4 * 4096;
    static constexpr int kFlagOff = kXchgOff + kXchgBytes;   // split flag (one int)
    static constexpr int kDeltaOff = kFlagOff + 256;         // delta partials, 256 B per wave
    static constexpr int kBytes = kDeltaOff + 1024;
    static_assert(kStageBytes % 512 == 0, "bank-aligned stages");
    static_assert(kBytes <= 160 * 1024, "LDS budget");
    // epilogue reduction: 4 source waves x kTiles tiles x 4 KiB
    static_assert(4 * kTiles * 4096 <= kStages * kStageBytes, "reduction fits the stages");
};

// s_waitcnt vmcnt(N) lgkmcnt(0): all but the last N vector-memory operations
// have completed and this wave's LDS accesses are done.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

// s_waitcnt vmcnt(N): all but the last N vector-memory operations have
// completed (LDS accesses are not waited for).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(N): all but this wave's last N LDS operations have
// completed (LDS operations of a wave complete in issue order).
template <int N>
__device__ __forceinline__ void wait_lgkm() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(0x3F | (0x7 << 4) | (N << 8) | (0x3 << 14));
}

// Scheduling patterns for the current region (between sched_barriers):
// kM MFMAs, each followed by a share of the region's VALU work (and, for
// sched_interleave, kR memory instructions spread over the first MFMAs), so
// that one wave keeps its matrix unit busy while its VALU runs the softmax.
template <int kM, int kR>
__device__ __forceinline__ void sched_interleave() {
#pragma unroll
    for (int i = 0; i < kM; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (i < kR) __builtin_amdgcn_sched_group_barrier(0x180 | 0x010, 1, 0);  // DS read / VMEM
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
}
template <int kM>
__device__ __forceinline__ void sched_interleave_valu() {
#pragma unroll
    for (int i = 0; i < kM; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
    }
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
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    if constexpr (kBf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <bool kBf16>
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    if constexpr (kBf16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Two fp32 values rounded to the 16-bit operand type, packed in one dword
// (low half = a).
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (kBf16) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        const bf16x2 v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        const f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
}

// fp32 -> the 16-bit output type (round to nearest even), as f16 bits
template <bool kBf16>
__device__ __forceinline__ _Float16 to16(float x) {
    if constexpr (kBf16) return __builtin_bit_cast(_Float16, (__bf16)x);
    else return (_Float16)x;
}

// 16x16 accumulator blocks c0 (columns j 0..15 of a 32-column block) and c1
// (columns 16..31), rows 4 (l / 16) + i, into the operand of a 32x32x16 MFMA
// whose lane l holds column l % 32 and rows 8 (l / 32) .. + 7 of the same 16
// rows.  v_permlane16_swap exchanges the odd 16-lane rows of its first
// operand with the even rows of its second, which moves each lane's missing
// four rows into place; no other data movement is needed.
template <bool kBf16>
__device__ __forceinline__ f16x8 c16_to_op32(f32x4 c0, f32x4 c1) {
    uint32_t a0 = pack2<kBf16>(c0[0], c0[1]), a1 = pack2<kBf16>(c0[2], c0[3]);
    uint32_t b0 = pack2<kBf16>(c1[0], c1[1]), b1 = pack2<kBf16>(c1[2], c1[3]);
    const auto s0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
    const auto s1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
    const u32x4 r = {s0[0], s1[0], s0[1], s1[1]};
    return __builtin_bit_cast(f16x8, r);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// threadIdx.x behind an empty asm: values a role derives from it (lane
// offsets, addresses) are then its own, so the compiler neither shares them
// with the other role of a two-unit workgroup nor keeps them live across
// both, which would push a role past the register file.
__device__ __forceinline__ int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Direct-to-LDS copy of a row-major [64][D] tile into a swizzled LDS tile,
// shared by the 4 waves (kLd 1 KiB blocks each).  Lane `lane` of wave `ld`
// moves the 16-byte chunk that belongs at LDS byte blk * 1024 + lane * 16
// (blk = ld * kLd + j); its source byte offset within the global tile is
// precomputed once.
template <int D>
__device__ __forceinline__ void tile_load_offsets(uint32_t (&off)[Cfg<D>::kLd], int ld, int lane,
                                                  int row_stride) {
    using C = Cfg<D>;
#pragma unroll
    for (int j = 0; j < C::kLd; ++j) {
        const int id = (ld * C::kLd + j) * 64 + lane;  // physical chunk
        const int row = id / C::kChunks;
        const int phys = id % C::kChunks;
        int sw;
        if constexpr (C::kChunks == 16) sw = ((row & 3) << 2) | ((row >> 2) & 3);
        else sw = swz128(row);
        const int logical = (phys ^ sw) & (C::kChunks - 1);
        off[j] = (uint32_t)((row * row_stride + logical * 8) * 2);
    }
}

template <int D>
__device__ __forceinline__ void load_tile_async(FA3_LDS char* tile, const _Float16* src,
                                                const uint32_t (&off)[Cfg<D>::kLd], int ld) {
#pragma unroll
    for (int j = 0; j < Cfg<D>::kLd; ++j) {
        __builtin_amdgcn_global_load_lds((const void*)((const char*)src + off[j]),
                                         (FA3_LDS void*)(tile + (ld * Cfg<D>::kLd + j) * 1024), 16,
                                         0, 0);
    }
}

// Direct-to-LDS copy of the statistics of the 64 query rows row0 .. of a
// tile; wave w moves rows 16 w .. 16 w + 15 with one load (one dword per
// active lane).  Layout in the rows block, by source:
//   kRowsInline: LSE[r] at 4 r;
//   kRowsArrays: lse2[r] at 128 (r / 16) + 4 (r % 16), -delta[r] 64 B after;
//   kRowsPacked: packed[r][0..2] at 12 r;
//   kRowsMaxSum: max[r] at 4 r, sum[r] at 256 + 4 r, delta[r] at 512 + 4 r
//                (wave w moves entries 48 w .. 48 w + 47 of that list).
template <int kRows, typename A>
__device__ __forceinline__ void load_rows_async(FA3_LDS char* rows, const A& a, size_t row0,
                                                int w, int lane) {
    if constexpr (kRows == kRowsInline) {
        if (lane < 16)
            __builtin_amdgcn_global_load_lds((const void*)(a.lse + row0 + 16 * w + lane),
                                             (FA3_LDS void*)(rows + 64 * w), 4, 0, 0);
    } else if constexpr (kRows == kRowsArrays) {
        const float* src = (lane < 16 ? a.lse2 : a.ndelta) + row0 + 16 * w + (lane & 15);
        if (lane < 32)
            __builtin_amdgcn_global_load_lds((const void*)src, (FA3_LDS void*)(rows + 128 * w), 4,
                                             0, 0);
    } else if constexpr (kRows == kRowsPacked) {
        if (lane < 48)
            __builtin_amdgcn_global_load_lds((const void*)(a.packed + 3 * (row0 + 16 * w) + lane),
                                             (FA3_LDS void*)(rows + 192 * w), 4, 0, 0);
    } else {
        static_assert(kRows == kRowsMaxSum, "row source");
        const int i = 48 * w + lane;
        const int arr = i >> 6;
        const float* src = (arr == 0 ? a.smax : arr == 1 ? a.ssum : a.delta_in) + row0 + (i & 63);
        if (lane < 48)
            __builtin_amdgcn_global_load_lds((const void*)src, (FA3_LDS void*)(rows + 192 * w), 4,
                                             0, 0);
    }
}

// Operand of a 32x32x16 product (32 x 16: lane l holds column 32 db + l % 32,
// rows 16 ks + 8 (l / 32) + t, t = 0..7) read transposed from a swizzled
// [64][D] tile (two reads of 4 rows).
template <int D>
__device__ __forceinline__ f16x8 tile_read_t(const FA3_LDS char* tile, int db, int ks, int lane) {
    const int g = lane >> 4, r = lane & 15;
    const int col = 32 * db + 16 * (g & 1) + 4 * (r & 3);
    const int row = 16 * ks + 8 * (g >> 1) + (r >> 2);
    const uint32_t lo = tile_off<D>(row, col >> 3) + (col & 7) * 2;
    const uint32_t hi = tile_off<D>(row + 4, col >> 3) + (col & 7) * 2;
    return concat4(lds_read_tr4(tile, lo), lds_read_tr4(tile, hi));
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
// Epilogue: four waves' partial sums -> one
// ----------------------------------------------------------------------------
// Accumulator tile u (of kTiles = 2 kKs 32x32 tiles: u = 2 nb + mb, 32-wide D
// block nb, 32-wide block mb of the job's keys / rows) belongs to wave u % 4
// after the reduction.  Every wave writes the tiles it does not own into LDS
// slot (u, source wave) as [4][64 lanes][4] fp32, so each access is one
// conflict-free 16-byte chunk per lane; the owner adds the three other
// waves' copies of its tiles.
template <int D>
__device__ __forceinline__ uint32_t red_off(int u, int src, int g, int lane) {
    return (uint32_t)((((u * 4 + src) * 4 + g) * 64 + lane) * 16);
}

// acc[u] for every tile; on return own[j] holds the full sum of tile 4 j + w.
template <int D>
__device__ __forceinline__ void reduce_tiles(const f32x16 (&acc)[Cfg<D>::kTiles],
                                             f32x16 (&own)[Cfg<D>::kOwn], FA3_LDS char* red, int w,
                                             int lane) {
    using C = Cfg<D>;
#pragma unroll
    for (int u = 0; u < C::kTiles; ++u) {
        if ((u & 3) == w) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = {acc[u][4 * g], acc[u][4 * g + 1], acc[u][4 * g + 2], acc[u][4 * g + 3]};
            *(FA3_LDS f32x4*)(red + red_off<D>(u, w, g, lane)) = v;
        }
    }
#pragma unroll
    for (int j = 0; j < C::kOwn; ++j) {
        // tile 4 j + w (the loop over u keeps register indexing static)
#pragma unroll
        for (int u = 0; u < C::kTiles; ++u)
            if (u == 4 * j + w) own[j] = acc[u];
    }
    wait_vm_lgkm0<0>();
    barrier();
#pragma unroll
    for (int j = 0; j < C::kOwn; ++j) {
        const int u = 4 * j + w;
#pragma unroll
        for (int s = 1; s < 4; ++s) {
            const int src = (w + s) & 3;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v = *(const FA3_LDS f32x4*)(red + red_off<D>(u, src, g, lane));
#pragma unroll
                for (int e = 0; e < 4; ++e) own[j][4 * g + e] += v[e];
            }
        }
    }
}

// Two waves (w and partner) hold partial sums of the same N tiles; tile t
// goes to the wave whose `sel` equals t % 2.  Each writes the N / 2 tiles it
// gives away into LDS slot (writer, t) as [4][64 lanes][4] fp32 -- one
// conflict-free 16-byte chunk per lane and access -- and adds the partner's
// copies of the tiles it keeps: on return own[j] holds tile 2 j + sel.
template <int N>
__device__ __forceinline__ void reduce_pair(const f32x16 (&acc)[N], f32x16 (&own)[N / 2],
                                            FA3_LDS char* red, int w, int partner, int sel,
                                            int lane) {
    auto slot = [&](int x, int t, int g) {
        return (uint32_t)((((x * N + t) * 4 + g) * 64 + lane) * 16);
    };
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const f32x16& give = sel ? acc[2 * j] : acc[2 * j + 1];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = {give[4 * g], give[4 * g + 1], give[4 * g + 2], give[4 * g + 3]};
            *(FA3_LDS f32x4*)(red + slot(w, 2 * j + (sel ^ 1), g)) = v;
        }
        own[j] = sel ? acc[2 * j + 1] : acc[2 * j];
    }
    wait_vm_lgkm0<0>();
    barrier();
#pragma unroll
    for (int j = 0; j < N / 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = *(const FA3_LDS f32x4*)(red + slot(partner, 2 * j + sel, g));
#pragma unroll
            for (int e = 0; e < 4; ++e) own[j][4 * g + e] += v[e];
        }
}

// Byte offset of 16-byte chunk c (of 4) of row r in a [32][32] 16-bit
// staging tile (64-byte rows, chunks XOR-swizzled by r / 4): 32 rows x 8 bytes
// written with ds_write_b64 and 16 rows x 4 chunks read with ds_read_b128 are
// both bank-conflict free.
__device__ __forceinline__ uint32_t row64_off(int r, int c) {
    return (uint32_t)(r * 64 + ((c ^ (r >> 2)) & 3) * 16);
}

// Stores owned tile `t` (lane: column n = 32 mb + l % 32 of the job's keys /
// rows = output row, D = 32 nb + 8 (i / 4) + 4 h + i % 4) times `mul` to the
// output rows starting at element `base` (row stride `rs`).  16-bit outputs
// are transposed through the wave's 2 KiB of `stage` so that each global
// store writes 16 bytes of one row.
template <bool kBf16, typename A>
__device__ __forceinline__ void store_tile(const A& a, void* outp, size_t base, int rs,
                                           int mb, int nb, const f32x16& t, float mul,
                                           FA3_LDS char* stage, int lane) {
    const int l32 = lane & 31, h = lane >> 5;
    if (a.out_f32) {
        float* o = (float*)outp + base + (size_t)(32 * mb + l32) * rs + 32 * nb + 4 * h;
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            const f32x4 v = {t[4 * a4] * mul, t[4 * a4 + 1] * mul, t[4 * a4 + 2] * mul,
                             t[4 * a4 + 3] * mul};
            *(f32x4*)(o + 8 * a4) = v;
        }
        return;
    }
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
        f16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = to16<kBf16>(t[4 * a4 + e] * mul);
        lds_write_b64(stage, row64_off(l32, a4) + 8 * h, v);
    }
    // the wave reads back only what it wrote: its LDS accesses complete in order
    _Float16* o = (_Float16*)outp + base + 32 * nb;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = 16 * j + (lane >> 2), c = lane & 3;
        const f16x8 x = lds_read_b128(stage, row64_off(r, c));
        *(f16x8*)(o + (size_t)(32 * mb + r) * rs + 8 * c) = x;
    }
}

// ----------------------------------------------------------------------------
// Split jobs
// ----------------------------------------------------------------------------
// Partial sums of split jobs travel between workgroups (possibly on
// different XCDs, whose L2 caches are not coherent with each other) through
// 16-byte buffer loads and stores with the sc1 cache policy -- the policy
// this chip's agent-scope atomic loads and stores use, coherent device-wide
// by itself -- so no cache-wide writeback / invalidate (which would also
// evict the tiles every CU of the XCD is streaming) is needed.
constexpr int kCachePolicySc1 = 16;
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer access on gfx9

__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, kBufferWord3);
}

template <int N>
__device__ __forceinline__ void put_partials(__amdgpu_buffer_rsrc_t r, uint32_t base,
                                             const f32x16 (&acc)[N], int lane) {
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
__device__ __forceinline__ void add_partials(__amdgpu_buffer_rsrc_t r, uint32_t base,
                                             f32x16 (&acc)[N], int lane) {
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
// as "not yet" and no clearing pass is needed; the second piece clears both
// words once it has seen the ready word, so a replayed launch that reuses
// its epoch (graph capture) finds them cleared too.
//
// split_arrive: thread 0 swaps the epoch into the arrival word.  The piece
// that reads back the epoch arrived second; the other arrived first.
// split_end: the first piece stores its (reduced) partial sums, waits until
// its stores have completed (s_waitcnt vmcnt(0) covers stores on gfx9) and
// writes the epoch into the ready word; it writes nothing else.  The second
// piece waits for the ready word (one thread, a bounded spin) and then adds
// the first piece's partial sums and writes the output.  The output is piece
// 0 + piece 1 either way (a two-term fp32 sum is the same in either order),
// so the result does not depend on which piece finishes first.  The wait
// cannot block for long -- the first piece has left its loop and only
// stores after arriving -- but it is bounded all the same; a wait that gives
// up writes the epoch into the error word, which the host reports as a HIP
// error when it synchronises, so a timed-out sum is never silent.
//
// Ordering: every cross-workgroup access (words and partial sums) is an
// agent-scope access with the sc1 policy, coherent at the device level; the
// writer's data stores complete before its ready store is issued, and the
// reader issues its data loads only after it has observed the ready word
// (its wait and a workgroup barrier come in between).
template <typename A>
__device__ __forceinline__ void split_arrive(const A& a, int job, FA3_LDS int* flag) {
    if (threadIdx.x == 0) {
        const unsigned long long old = __hip_atomic_exchange(
            a.sync + 2 * job, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == a.epoch ? 1 : 0;
    }
}

template <typename A, typename PutOwn>
__device__ __forceinline__ bool split_end(const A& a, int job, FA3_LDS int* flag,
                                          PutOwn&& put_own) {
    wait_vm_lgkm0<0>();
    barrier();
    const int second = *flag;
    if (!second) {
        put_own();
        wait_vm_lgkm0<0>();
        barrier();
        if (threadIdx.x == 0)
            __hip_atomic_store(a.sync + 2 * job + 1, a.epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    if (threadIdx.x == 0) {
        bool seen = false;
        for (int i = 0; i < a.spin_limit; ++i) {
            if (__hip_atomic_load(a.sync + 2 * job + 1, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) == a.epoch) {
                seen = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!seen)
            __hip_atomic_store(a.err, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Nobody reads the words again in this launch (the first piece wrote
        // its last one before the ready word was seen): leave them cleared, so
        // that a replay of the same launch (a captured graph keeps the epoch)
        // starts from "nobody arrived".
        __hip_atomic_store(a.sync + 2 * job, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.sync + 2 * job + 1, 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vm_lgkm0<0>();
    barrier();
    return true;
}

// ----------------------------------------------------------------------------
// dKV role
// ----------------------------------------------------------------------------
// Waves pair up: wave w forms S, dP, P and dS of query rows 16 w .. 16 w + 15
// against all 64 keys, and accumulates dV^T and dK^T for D half c = w % 2
// (all 64 keys) over the rows of its pair p = w / 2 (rows 32 p .. 32 p +
// 31).  The pair swaps the P / dS operands of its rows through LDS once per
// step: written into the rows of the stage's O tile that the wave itself
// read for delta (D 128: exactly 4 KiB), or into a separate area (D 64).
// The two pairs then hold partial sums over their rows, added in the
// epilogue.
//
// Streams query tiles [qa, qb) of every query head of the group.  slot < 0:
// the job is whole and writes dK / dV; otherwise the unit is a piece of
// split job `slot` and the pieces' partial sums meet in split_end.
template <int D, bool kCausal, bool kBf16, int kRows, typename A>
__device__ void dkv_role(const A& a, int bkv, int kt, int qa, int qb, int slot,
                         FA3_LDS char* smem) {
    static_assert(kRows == kRowsArrays || kRows == kRowsPacked || kRows == kRowsInline,
                  "dKV rows come as arrays, packed or inline");
    using C = Cfg<D>;
    constexpr int T = C::kTileBytes;
    constexpr int kKs = C::kKs;
    constexpr int kNh = kKs / 2;  // 32-wide D blocks per half
    constexpr bool kO = kRows == kRowsInline;  // O streamed for delta
    const int tid = opaque_tid();
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pw = w ^ 1;                 // pair partner
    const int ch = w & 1, pr = w >> 1;    // D half, row pair
    const int l16 = lane & 15, g4 = lane >> 4;

    const int S = a.seqlen;
    const int group = a.heads_q / a.heads_kv;
    const int b = bkv / a.heads_kv;
    const int hkv = bkv % a.heads_kv;
    const int kbase = kt * 64;
    const int n_it = group * (qb - qa);

    uint32_t q_off[C::kLd], kv_off[C::kLd];
    tile_load_offsets<D>(q_off, w, lane, a.q_rs);
    tile_load_offsets<D>(kv_off, w, lane, a.kv_rs);

    // Cursor of the next query tile to load; a finished stream keeps
    // re-loading its last tile (into a stage nobody reads), so every step
    // issues the same loads.
    int ld_qt = qa, ld_left = n_it;
    const int h0 = hkv * group;
    size_t ld_e = q_elem<D>(a, b, h0, qa * 64);                  // Q / dO / O element
    size_t ld_row = ((size_t)b * a.heads_q + h0) * S + qa * 64;  // statistics row
    const size_t step_e = (size_t)64 * a.q_rs;
    const size_t wrap_e = (size_t)a.q_hs - (size_t)(qb - qa - 1) * step_e;  // next head, tile qa
    const size_t wrap_row = (size_t)S - (size_t)(qb - qa - 1) * 64;
    // part 0: Q, part 1: dO, part 2: O (kO) and the rows, then the cursor
    // moves on; a step spreads its parts over its MFMAs
    auto issue_part = [&](FA3_LDS char* st, int part) {
        if (part == 0) {
            load_tile_async<D>(st, a.q + ld_e, q_off, w);
            return;
        }
        if (part == 1) {
            load_tile_async<D>(st + T, a.dout + ld_e, q_off, w);
            return;
        }
        if constexpr (kO) load_tile_async<D>(st + 2 * T, a.out + ld_e, q_off, w);
        load_rows_async<kRows>(st + C::kRowsOff, a, ld_row, w, lane);
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
    constexpr int kDma = (kO ? 3 : 2) * C::kLd + 1;  // loads per wave and stage

    FA3_LDS char* st0 = smem;
    FA3_LDS char* st1 = smem + C::kStageBytes;
    FA3_LDS char* st2 = smem + 2 * C::kStageBytes;
    FA3_LDS int* flag = (FA3_LDS int*)(smem + C::kFlagOff);

    // ---- prologue: K and V of this key tile, staged in stage 2, become the
    // B operands of S and dP (lane: key 16 kb + l16, D chunk p1_chunk(s, g4))
    f16x8 kf[4][kKs], vf[4][kKs];
    {
        const size_t k0 = kv_elem<D>(a, b, hkv, kbase);
        load_tile_async<D>(st2, a.k + k0, kv_off, w);
        load_tile_async<D>(st2 + T, a.v + k0, kv_off, w);
        for (int part = 0; part < 3; ++part) issue_part(st0, part);
        for (int part = 0; part < 3; ++part) issue_part(st1, part);
        wait_vm_lgkm0<2 * kDma>();
        barrier();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int s = 0; s < kKs; ++s) {
                const uint32_t off = tile_off<D>(16 * kb + l16, p1_chunk<D>(s, g4));
                kf[kb][s] = lds_read_b128(st2, off);
                vf[kb][s] = lds_read_b128(st2 + T, off);
            }
        wait_vm_lgkm0<63>();  // K / V read before stage 2 takes tile 2
    }

    // dV^T / dK^T partials over the pair's rows for D half ch: tile t = 2 n +
    // mb (D block ch kNh + n, key block mb); lane: key 32 mb + l % 32,
    // D 32 (ch kNh + n) + 8 (i / 4) + 4 h + i % 4
    f32x16 accv[2 * kNh], acck[2 * kNh];
#pragma unroll
    for (int t = 0; t < 2 * kNh; ++t) {
        accv[t] = f32x16{};
        acck[t] = f32x16{};
    }

    // P / dS operand exchange area of wave x: 4 KiB ([matrix][mb][lane] f16x8)
    auto xchg = [&](FA3_LDS char* st, int x) -> FA3_LDS char* {
        if constexpr (D == 128) return st + 2 * T + x * 4096;  // the O rows wave x read
        else return smem + C::kXchgOff + x * 4096;
    };

    // The operands a wave reads for its own rows of a tile, prefetched during
    // the previous step: the A operands of S and dP (rows 16 w + l16, D chunks
    // p1_chunk(s, g4)) and the rows' statistics, turned into lse2 and -delta
    // of rows 16 w + 4 g4 + i (the S / dP accumulator rows).  With inline rows,
    // delta comes from O's matching chunks: the four lanes of a row add their
    // parts through 256 bytes of LDS, which also moves the sums to the
    // accumulators' layout, in the order (g0 + g1) + (g2 + g3).  The wave's rows were loaded by
    // its own direct-to-LDS loads, so its own s_waitcnt is all they need.
    f16x8 aq[kKs], ad[kKs], ao[kKs];
    f32x4 l2, nd, rs0, rs1, rs2;
    FA3_LDS char* dslot = smem + C::kDeltaOff + 256 * w;
    // LDS reads issued by read_own, in order
    constexpr int kOwnReads = (kO ? 3 : 2) * kKs + (kRows == kRowsPacked ? 3 : kRows == kRowsArrays ? 2 : 1);
    auto read_own = [&](const FA3_LDS char* st) {
#pragma unroll
        for (int s = 0; s < kKs; ++s) {
            const uint32_t off = tile_off<D>(16 * w + l16, p1_chunk<D>(s, g4));
            aq[s] = lds_read_b128(st, off);
            ad[s] = lds_read_b128(st + T, off);
            if constexpr (kO) ao[s] = lds_read_b128(st + 2 * T, off);
        }
        const FA3_LDS char* rows = st + C::kRowsOff;
        if constexpr (kRows == kRowsInline) {
            rs0 = *(const FA3_LDS f32x4*)(rows + (16 * w + 4 * g4) * 4);
        } else if constexpr (kRows == kRowsArrays) {
            rs0 = *(const FA3_LDS f32x4*)(rows + 128 * w + 16 * g4);
            rs1 = *(const FA3_LDS f32x4*)(rows + 128 * w + 16 * g4 + 64);
        } else {
            const FA3_LDS f32x4* r = (const FA3_LDS f32x4*)(rows + (16 * w + 4 * g4) * 12);
            rs0 = r[0];
            rs1 = r[1];
            rs2 = r[2];
        }
    };
    auto finish_own = [&]() {
        if constexpr (kRows == kRowsInline) {
#pragma unroll
            for (int i = 0; i < 4; ++i) l2[i] = rs0[i] * kLog2e;
            float drow = 0.f;
#pragma unroll
            for (int s = 0; s < kKs; ++s) drow = dot8<kBf16>(ad[s], ao[s], drow);
            // partial of row l16 from lane group g4 -> slot [row][g4]; each
            // lane then adds the four partials of rows 4 g4 + i
            *(FA3_LDS float*)(dslot + 16 * l16 + 4 * g4) = drow;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 q = *(const FA3_LDS f32x4*)(dslot + 16 * (4 * g4 + i));
                nd[i] = (q[0] + q[1]) + (q[2] + q[3]);
            }
        } else if constexpr (kRows == kRowsArrays) {
            l2 = rs0;
            nd = rs1;
        } else {
            // [row][max_log2, inv_sum, delta]: exp2(x - m) * inv = exp2(x - (m - log2 inv))
            const float f[12] = {rs0[0], rs0[1], rs0[2], rs0[3], rs1[0], rs1[1],
                                 rs1[2], rs1[3], rs2[0], rs2[1], rs2[2], rs2[3]};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                l2[i] = f[3 * i] - __log2f(f[3 * i + 1]);
                nd[i] = -f[3 * i + 2];
            }
        }
    };
    // nd holds +delta from the inline path until the step uses it; the sign is
    // applied where the dP accumulators are seeded
    constexpr float kNdSign = kRows == kRowsInline ? -1.f : 1.f;

    // Phase A of one tile (rows 16 w .. 16 w + 15 of stage st), in groups
    // whose MFMAs and VALU work the scheduler interleaves (sched_group_barrier):
    //   G0: S and dP of key blocks 0, 1 (4 accumulator chains) beside the
    //       transposed reads of the own-row gradient operands and the first
    //       loads of tile j + 2;
    //   G1: S and dP of key blocks 2, 3 beside the softmax of blocks 0, 1 and
    //       their P / dS operands (key block mb 0, also written for the
    //       partner);
    //   G2: the own rows' dV^T / dK^T for mb 0 beside the softmax of blocks
    //       2, 3 and the operands of mb 1;
    //   G3: the own rows' dV^T / dK^T for mb 1, the rest of the loads.
    auto phase_a = [&](FA3_LDS char* __restrict__ st, const FA3_LDS char* __restrict__ nxt1,
                       FA3_LDS char* __restrict__ nxt2, bool prefetch, auto masked_c) {
        constexpr bool kMasked = decltype(masked_c)::value;
        const FA3_LDS char* tq = st;
        const FA3_LDS char* tdo = st + T;
        f32x4 sacc[4], pacc[4], p[4], ds[4];
        f16x8 bo[kNh], bq[kNh], ap[2], as[2];
        FA3_LDS char* mine = xchg(st, w);
        const f32x4 ndl = nd * kNdSign;  // -delta of the accumulator rows
        auto mfma_s_dp = [&](int kb0) {
#pragma unroll
            for (int s = 0; s < kKs; ++s)
#pragma unroll
                for (int kb = kb0; kb < kb0 + 2; ++kb) {
                    sacc[kb] = mfma16<kBf16>(aq[s], kf[kb][s], s == 0 ? f32x4{} : sacc[kb]);
                    pacc[kb] = mfma16<kBf16>(ad[s], vf[kb][s], s == 0 ? ndl : pacc[kb]);
                }
        };
        // P = exp2(S c - lse2), dS = P (dP - delta) of key block kb; on the
        // causal diagonal tile the keys after a row see nothing
        auto softmax = [&](int kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = fast_exp2(sacc[kb][i] * a.scale_log2 - l2[i]);
                if constexpr (kMasked) {
                    if (16 * kb + l16 > 16 * w + 4 * g4 + i) x = 0.f;
                }
                p[kb][i] = x;
                ds[kb][i] = x * pacc[kb][i];
            }
        };
        // operands of the gradient products (keys 32 mb + l % 32, rows 8 h + t
        // of the wave's 16) and their copy for the partner
        auto operands = [&](int mb) {
            ap[mb] = c16_to_op32<kBf16>(p[2 * mb], p[2 * mb + 1]);
            as[mb] = c16_to_op32<kBf16>(ds[2 * mb], ds[2 * mb + 1]);
            lds_write_b128(mine, (0 * 2 + mb) * 1024 + lane * 16, ap[mb]);
            lds_write_b128(mine, (1 * 2 + mb) * 1024 + lane * 16, as[mb]);
        };
        auto own_grad = [&](int mb) {
#pragma unroll
            for (int n = 0; n < kNh; ++n) {
                accv[2 * n + mb] = mfma32<kBf16>(bo[n], ap[mb], accv[2 * n + mb]);
                acck[2 * n + mb] = mfma32<kBf16>(bq[n], as[mb], acck[2 * n + mb]);
            }
        };
        // G0
        mfma_s_dp(0);
#pragma unroll
        for (int n = 0; n < kNh; ++n) {
            bo[n] = tile_read_t<D>(tdo, ch * kNh + n, w, lane);
            bq[n] = tile_read_t<D>(tq, ch * kNh + n, w, lane);
        }
        issue_part(nxt2, 0);
        sched_interleave<4 * kKs, 2 * kNh + C::kLd>();
        __builtin_amdgcn_sched_barrier(0);
        // G1
        mfma_s_dp(2);
        softmax(0);
        softmax(1);
        operands(0);
        sched_interleave_valu<4 * kKs>();
        __builtin_amdgcn_sched_barrier(0);
        // G2
        own_grad(0);
        softmax(2);
        softmax(3);
        operands(1);
        sched_interleave_valu<2 * kNh>();
        __builtin_amdgcn_sched_barrier(0);
        // G3 (and the prefetch of tile j + 1's own rows: its loads were issued
        // a step ago; only tile j + 2's may still be in flight)
        own_grad(1);
        issue_part(nxt2, 1);
        issue_part(nxt2, 2);
        if (prefetch) {
            wait_vm<kDma>();
            read_own(nxt1);
        }
    };

    // Phase B: the partner's rows (its P / dS operands and the matching
    // transposed operands of this wave's D half); while they are read, the
    // next tile's prefetched rows become lse2 / delta.
    auto phase_b = [&](const FA3_LDS char* __restrict__ st, bool prefetch) {
        const FA3_LDS char* theirs = xchg(const_cast<FA3_LDS char*>(st), pw);
        f16x8 bo[kNh], bq[kNh], ap[2], as[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            ap[mb] = lds_read_b128(theirs, (0 * 2 + mb) * 1024 + lane * 16);
            as[mb] = lds_read_b128(theirs, (1 * 2 + mb) * 1024 + lane * 16);
        }
#pragma unroll
        for (int n = 0; n < kNh; ++n) {
            bo[n] = tile_read_t<D>(st + T, ch * kNh + n, pw, lane);
            bq[n] = tile_read_t<D>(st, ch * kNh + n, pw, lane);
        }
        if (prefetch) finish_own();
#pragma unroll
        for (int n = 0; n < kNh; ++n)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                accv[2 * n + mb] = mfma32<kBf16>(bo[n], ap[mb], accv[2 * n + mb]);
                acck[2 * n + mb] = mfma32<kBf16>(bq[n], as[mb], acck[2 * n + mb]);
            }
    };

    // ---- main loop: tile j lives in stage j % 3; tile j + 2 goes into the
    // stage of tile j - 1 once every wave has passed this step's first
    // barrier.  One step per iteration over rotating stage pointers (addresses
    // are then formed from one runtime base instead of one set per stage).
    int sm_qt = qa;  // query tile of the next step
    FA3_LDS char* cur = st0;
    FA3_LDS char* nx1 = st1;
    FA3_LDS char* nx2 = st2;
    wait_vm<kDma>();  // tile 0 (only tile 1 may be in flight)
    read_own(cur);
    finish_own();
    for (int j = 0; j < n_it; ++j) {
        barrier();  // every wave is done with tile j - 1: its stage takes tile j + 2
        const bool masked = kCausal && sm_qt == kt;
        if (++sm_qt == qb) sm_qt = qa;
        const bool prefetch = j + 1 < n_it;
        if (masked) phase_a(cur, nx1, nx2, prefetch, std::true_type{});
        else phase_a(cur, nx1, nx2, prefetch, std::false_type{});
        // the exchange writes are done (the prefetch reads issued after them
        // may still be in flight)
        if (prefetch) wait_lgkm<kOwnReads>();
        else wait_lgkm<0>();
        barrier();
        phase_b(cur, prefetch);
        FA3_LDS char* x = cur;
        cur = nx1;
        nx1 = nx2;
        nx2 = x;
    }

    // ---- epilogue: the stages are free once the re-loads have landed; the
    // two pairs' partials meet (wave w and w ^ 2 share a D half; row pair pr
    // keeps key block mb = pr)
    wait_vm_lgkm0<0>();
    barrier();
    f32x16 ownv[kNh], ownk[kNh];
    reduce_pair<2 * kNh>(accv, ownv, smem, w, w ^ 2, pr, lane);
    barrier();
    reduce_pair<2 * kNh>(acck, ownk, smem, w, w ^ 2, pr, lane);
    if (slot >= 0) {
        split_arrive(a, slot, flag);
        const __amdgpu_buffer_rsrc_t prs = partial_rsrc(a.part_kv, a.part_kv_bytes);
        const uint32_t base = (uint32_t)(slot * 4 + w) * (2 * kNh * 4096);
        if (!split_end(a, slot, flag, [&] {
                put_partials<kNh>(prs, base, ownv, lane);
                put_partials<kNh>(prs, base + kNh * 4096, ownk, lane);
            }))
            return;
        add_partials<kNh>(prs, base, ownv, lane);
        add_partials<kNh>(prs, base + kNh * 4096, ownk, lane);
    }
    barrier();  // the reduction slots are free again: stage the stores there
    const size_t obase = kv_elem<D>(a, b, hkv, kbase);
    FA3_LDS char* stg = smem + w * 4096;
#pragma unroll
    for (int n = 0; n < kNh; ++n) {
        const int nb = ch * kNh + n;
        store_tile<kBf16>(a, a.dv, obase, a.kv_rs, pr, nb, ownv[n], 1.f, stg, lane);
        store_tile<kBf16>(a, a.dk, obase, a.kv_rs, pr, nb, ownk[n], a.scale, stg + 2048, lane);
    }
}

// ----------------------------------------------------------------------------
// dQ role
// ----------------------------------------------------------------------------
// Streams key tiles [ka, kb) (the causal diagonal, key tile qt, is masked).
// slot: as for dkv_role.  Writes delta (softmax_d) for its rows when it
// forms it (kRowsInline) and is the job's only or first piece.
template <int D, bool kCausal, bool kBf16, int kRows, typename A>
__device__ void dq_role(const A& a, int bhq, int qt, int ka, int kb, int slot,
                        bool write_delta, FA3_LDS char* smem) {
    static_assert(kRows == kRowsArrays || kRows == kRowsMaxSum || kRows == kRowsInline,
                  "dQ rows come as arrays, max / sum / delta or inline");
    using C = Cfg<D>;
    constexpr int T = C::kTileBytes;
    constexpr int kKs = C::kKs;
    const int tid = opaque_tid();
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g4 = lane >> 4;

    const int S = a.seqlen;
    const int group = a.heads_q / a.heads_kv;
    const int b = bhq / a.heads_q;
    const int hq = bhq - b * a.heads_q;
    const int hkv = hq / group;
    const size_t row0 = (size_t)bhq * S + qt * 64;  // statistics row
    const size_t q0 = q_elem<D>(a, b, hq, qt * 64);  // this tile's Q / dO / O / dQ elements
    const int n_kt = kb - ka;

    uint32_t kv_off[C::kLd], q_off[C::kLd];
    tile_load_offsets<D>(kv_off, w, lane, a.kv_rs);
    tile_load_offsets<D>(q_off, w, lane, a.q_rs);
    const _Float16* kh = a.k + kv_elem<D>(a, b, hkv, 0);
    const _Float16* vh = a.v + kv_elem<D>(a, b, hkv, 0);
    int ld_kt = ka;
    size_t ld_e = (size_t)ka * 64 * a.kv_rs;
    const size_t step_e = (size_t)64 * a.kv_rs;
    // part 0: K, part 1: V, then the cursor moves on
    auto issue_part = [&](FA3_LDS char* st, int part) {
        if (part == 0) {
            load_tile_async<D>(st, kh + ld_e, kv_off, w);
            return;
        }
        load_tile_async<D>(st + T, vh + ld_e, kv_off, w);
        if (ld_kt + 1 < kb) {
            ++ld_kt;
            ld_e += step_e;
        }
    };
    constexpr int kDma = 2 * C::kLd;

    FA3_LDS char* st0 = smem;
    FA3_LDS char* st1 = smem + C::kStageBytes;
    FA3_LDS char* st2 = smem + 2 * C::kStageBytes;
    FA3_LDS int* flag = (FA3_LDS int*)(smem + C::kFlagOff);

    // ---- prologue: this query tile's Q, dO (and O) and row statistics,
    // staged in stage 2, become B operands (lane: row 16 rb + l16, D chunk
    // p1_chunk(s, g4)) and per-lane row values
    f16x8 qf[4][kKs], df[4][kKs];
    float l2[4], dlt[4];  // lse2 and delta of row 16 rb + l16
    {
        load_tile_async<D>(st2, a.q + q0, q_off, w);
        load_tile_async<D>(st2 + T, a.dout + q0, q_off, w);
        if constexpr (kRows == kRowsInline) load_tile_async<D>(st2 + 2 * T, a.out + q0, q_off, w);
        load_rows_async<kRows>(st2 + C::kRowsOff, a, row0, w, lane);
        for (int part = 0; part < 2; ++part) issue_part(st0, part);
        for (int part = 0; part < 2; ++part) issue_part(st1, part);
        wait_vm_lgkm0<2 * kDma>();
        barrier();
        const FA3_LDS char* rows = st2 + C::kRowsOff;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int r = 16 * rb + l16;
            float drow = 0.f;
#pragma unroll
            for (int s = 0; s < kKs; ++s) {
                const uint32_t off = tile_off<D>(r, p1_chunk<D>(s, g4));
                qf[rb][s] = lds_read_b128(st2, off);
                df[rb][s] = lds_read_b128(st2 + T, off);
                if constexpr (kRows == kRowsInline)
                    drow = dot8<kBf16>(df[rb][s], lds_read_b128(st2 + 2 * T, off), drow);
            }
            if constexpr (kRows == kRowsInline) {
                drow += __shfl_xor(drow, 16);
                drow += __shfl_xor(drow, 32);
                dlt[rb] = drow;
                l2[rb] = ((const FA3_LDS float*)rows)[r] * kLog2e;
            } else if constexpr (kRows == kRowsArrays) {
                l2[rb] = *(const FA3_LDS float*)(rows + 128 * rb + 4 * l16);
                dlt[rb] = -*(const FA3_LDS float*)(rows + 128 * rb + 64 + 4 * l16);
            } else {  // exp2((x - max) c) / sum = exp2(x c - (max c + log2 sum))
                const FA3_LDS float* rf = (const FA3_LDS float*)rows;
                l2[rb] = rf[r] * a.scale_log2 + __log2f(rf[64 + r]);
                dlt[rb] = rf[128 + r];
            }
        }
        if constexpr (kRows == kRowsInline) {
            // softmax_d: wave w writes rows 16 w .. 16 w + 15 (one writer per row)
            if (write_delta && a.delta_out != nullptr && lane < 16) {
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    if (rb == w) a.delta_out[row0 + 16 * rb + l16] = dlt[rb];
            }
        }
    }

    // dQ^T partial over this wave's keys: tile u = 2 nb + mb (D block nb, row
    // block mb); lane: row 32 mb + l % 32, D 32 nb + 8 (i / 4) + 4 h + i % 4
    f32x16 accq[C::kTiles];
#pragma unroll
    for (int u = 0; u < C::kTiles; ++u) accq[u] = f32x16{};

    // The A operands of S^T and dP^T for the wave's own keys of a tile (keys
    // 16 w + l16, D chunks p1_chunk(s, g4)), prefetched one step ahead.  The
    // wave reads only rows it loaded itself, so the loop has no barrier: each
    // wave's s_waitcnt orders its own loads and reads.
    f16x8 ak[kKs], av[kKs];
    auto read_own = [&](const FA3_LDS char* st) {
#pragma unroll
        for (int s = 0; s < kKs; ++s) {
            const uint32_t off = tile_off<D>(16 * w + l16, p1_chunk<D>(s, g4));
            ak[s] = lds_read_b128(st, off);
            av[s] = lds_read_b128(st + T, off);
        }
    };

    // One key tile (stage st), in groups whose MFMAs and VALU work the
    // scheduler interleaves:
    //   G0: S^T and dP^T of row blocks 0, 1 beside the K^T operand reads of
    //       dQ^T and the first loads of tile j + 2;
    //   G1: row blocks 2, 3 beside the softmax of blocks 0, 1 and their dS^T
    //       operand (row block mb 0);
    //   G2: dQ^T of mb 0 beside the softmax of blocks 2, 3;
    //   G3: dQ^T of mb 1 and the rest of the loads.
    auto compute = [&](const FA3_LDS char* __restrict__ st, const FA3_LDS char* __restrict__ nxt1,
                       FA3_LDS char* __restrict__ nxt2, bool prefetch, auto masked_c) {
        constexpr bool kMasked = decltype(masked_c)::value;
        const FA3_LDS char* tk = st;
        f32x4 sacc[4], pacc[4], ds[4];
        f16x8 bk[kKs], as[2];
        auto mfma_s_dp = [&](int rb0) {
#pragma unroll
            for (int s = 0; s < kKs; ++s)
#pragma unroll
                for (int rb = rb0; rb < rb0 + 2; ++rb) {
                    const float nd = -dlt[rb];
                    sacc[rb] = mfma16<kBf16>(ak[s], qf[rb][s], s == 0 ? f32x4{} : sacc[rb]);
                    pacc[rb] = mfma16<kBf16>(av[s], df[rb][s],
                                             s == 0 ? f32x4{nd, nd, nd, nd} : pacc[rb]);
                }
        };
        auto softmax = [&](int rb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = fast_exp2(sacc[rb][i] * a.scale_log2 - l2[rb]) * pacc[rb][i];
                if constexpr (kMasked) {
                    if (16 * w + 4 * g4 + i > 16 * rb + l16) x = 0.f;
                }
                ds[rb][i] = x;
            }
        };
        // dQ^T += K^T dS^T for row block mb (dS^T operand: rows 32 mb + l % 32,
        // the wave's keys 8 h + t)
        auto grad = [&](int mb) {
#pragma unroll
            for (int nb = 0; nb < kKs; ++nb)
                accq[2 * nb + mb] = mfma32<kBf16>(bk[nb], as[mb], accq[2 * nb + mb]);
        };
        // G0
        mfma_s_dp(0);
        // K^T operands of dQ^T: D block nb, keys 16 w + 8 h + t
#pragma unroll
        for (int nb = 0; nb < kKs; ++nb) bk[nb] = tile_read_t<D>(tk, nb, w, lane);
        issue_part(nxt2, 0);
        sched_interleave<4 * kKs, kKs + C::kLd>();
        __builtin_amdgcn_sched_barrier(0);
        // G1
        mfma_s_dp(2);
        softmax(0);
        softmax(1);
        as[0] = c16_to_op32<kBf16>(ds[0], ds[1]);
        sched_interleave_valu<4 * kKs>();
        __builtin_amdgcn_sched_barrier(0);
        // G2 (and the prefetch of tile j + 1's own keys: its loads were issued
        // a step ago; only tile j + 2's first part may still be in flight)
        grad(0);
        softmax(2);
        softmax(3);
        as[1] = c16_to_op32<kBf16>(ds[2], ds[3]);
        if (prefetch) {
            wait_vm<C::kLd>();
            read_own(nxt1);
        }
        sched_interleave_valu<kKs>();
        __builtin_amdgcn_sched_barrier(0);
        // G3
        grad(1);
        issue_part(nxt2, 1);
    };

    int cur_kt = ka;
    FA3_LDS char* cur = st0;
    FA3_LDS char* nx1 = st1;
    FA3_LDS char* nx2 = st2;
    // the prologue's barrier let every wave finish reading stage 2 (this
    // tile's Q, dO, O) before any wave loads into it
    wait_vm_lgkm0<63>();
    barrier();
    wait_vm<kDma>();  // key tile 0 (only tile 1 may be in flight)
    read_own(cur);
    for (int j = 0; j < n_kt; ++j) {
        const bool masked = kCausal && cur_kt == qt;
        ++cur_kt;
        const bool prefetch = j + 1 < n_kt;
        if (masked) compute(cur, nx1, nx2, prefetch, std::true_type{});
        else compute(cur, nx1, nx2, prefetch, std::false_type{});
        FA3_LDS char* x = cur;
        cur = nx1;
        nx1 = nx2;
        nx2 = x;
    }

    wait_vm_lgkm0<0>();
    barrier();
    f32x16 own[C::kOwn];
    reduce_tiles<D>(accq, own, smem, w, lane);
    if (slot >= 0) {
        split_arrive(a, a.n_split + slot, flag);
        const __amdgpu_buffer_rsrc_t pr = partial_rsrc(a.part_q, a.part_q_bytes);
        const uint32_t base = (uint32_t)(slot * 4 + w) * (C::kOwn * 4096);
        if (!split_end(a, a.n_split + slot, flag, [&] { put_partials<C::kOwn>(pr, base, own, lane); }))
            return;
        add_partials<C::kOwn>(pr, base, own, lane);
    }
    barrier();
    FA3_LDS char* stg = smem + w * 4096;
#pragma unroll
    for (int jj = 0; jj < C::kOwn; ++jj) {
        const int u = 4 * jj + w, nb = u >> 1, mb = u & 1;
        store_tile<kBf16>(a, a.dq, q0, a.q_rs, mb, nb, own[jj], a.scale, stg, lane);
    }
}

// Block id -> (group, position in the group); see the job map below.
__device__ __forceinline__ void job_of(const MainArgs& a, int& g, int& pos) {
    const int id = blockIdx.x;
    if (a.xcd_parts > 0) {
        const int xcd = id & 7;
        const int n = id >> 3;
        const int v = xcd + 8 * (n / a.part_len);  // virtual group = (group, part)
        g = v / a.xcd_parts;
        pos = v % a.xcd_parts + a.xcd_parts * (n % a.part_len);
    } else {
        g = id / a.jobs_per_group;
        pos = id % a.jobs_per_group;
    }
}

// Job map.  Jobs are grouped by (batch, kv head) -- a group's dKV jobs and
// the dQ jobs of its query heads touch only that head's Q, dO, O, K, V.  The
// hardware deals consecutive workgroup ids round-robin to the 8 XCDs; when
// the shape allows, block id -> (xcd, position) is arranged so that each XCD
// runs whole parts of groups, keeping a head's tiles in one L2.
//
// Default plan: within a group, position p = (level L, slot r) with G + 1
// slots per level: slot 0 is the dKV job of key tile L, slot r > 0 the dQ
// job of query head r - 1 at query tile QT - 1 - L, so the dispatch order is
// longest first (causal).
//
// Split plan (bal_m = M = QT / 2 > 0; causal, G = 1, few jobs): the causal
// jobs run 1 .. QT steps, so one long job would set the kernel's length.
// The long jobs (dKV key tiles x < M, dQ query tiles M + x) are cut into a
// head piece of head_kv[x] / head_q[x] tiles and a remainder, and each
// remainder shares a workgroup with a short job of the other role
// (x = p mod M):
//   p in [0, M):    dKV key tile M + x (whole), then the remainder of dQ
//                   query tile M + x (key tiles head_q[x] .. M + x);
//   p in [M, 2M):   dQ query tile x (whole), then the remainder of dKV key
//                   tile x (query tiles x + head_kv[x] .. QT - 1);
//   p in [2M, 3M):  head piece of dKV key tile x;
//   p in [3M, 4M):  head piece of dQ query tile M + x.
// The host picks the head lengths from a cost model of the steps, prologues
// and epilogues so that the workgroups finish together (a length covering
// the whole job leaves it unsplit).
// Workgroups per CU: at head dim 64 two fit (registers <= 256 per wave, LDS
// <= 80 KiB), so each SIMD runs two waves that hide each other's latencies.
template <int D>
constexpr int kBlocksPerCu = D == 64 ? 2 : 1;

template <int D, bool kCausal, bool kBf16, int kRows>
__global__ __launch_bounds__(kThreads, kBlocksPerCu<D>) void bwd_main_kernel(MainArgs a) {
    __shared__ __attribute__((aligned(1024))) char smem_raw[Cfg<D>::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;
    int g, pos;
    job_of(a, g, pos);
    const int group = a.heads_q / a.heads_kv;
    const int QT = a.seqlen / 64;
    // This workgroup's units, run in order: role (0 dKV, 1 dQ), the job's
    // head (dKV: KV head b * Hkv + h; dQ: query head b * Hq + h), its tile,
    // the streamed range [lo, hi), the split slot (-1: whole job) and whether
    // a dQ unit writes delta.  One call site per role keeps the code (and its
    // register allocation) to one copy of each.
    int n_units = 1;
    int role[2], head[2], tile[2], lo[2], hi[2], slot[2];
    bool wdelta[2] = {true, true};
    if (kCausal && a.bal_m > 0) {
        // G = 1: group g is query head g (and KV head g)
        const int M = a.bal_m;
        const int job0 = g * M;
        if (pos < M) {
            // dKV key tile M + x whole, then the remainder of dQ query tile M + x
            const int x = pos, nq = M + x + 1, lq = a.head_q[x];
            role[0] = 0, tile[0] = M + x, lo[0] = M + x, hi[0] = QT, slot[0] = -1;
            role[1] = 1, tile[1] = M + x, lo[1] = lq, hi[1] = nq, slot[1] = job0 + x;
            wdelta[1] = false;
            n_units = lq < nq ? 2 : 1;
        } else if (pos < 2 * M) {
            // dQ query tile x whole, then the remainder of dKV key tile x
            const int x = pos - M, nkv = QT - x, lkv = a.head_kv[x];
            role[0] = 1, tile[0] = x, lo[0] = 0, hi[0] = x + 1, slot[0] = -1;
            role[1] = 0, tile[1] = x, lo[1] = x + lkv, hi[1] = QT, slot[1] = job0 + x;
            n_units = lkv < nkv ? 2 : 1;
        } else if (pos < 3 * M) {
            // head piece (or all) of dKV key tile x
            const int x = pos - 2 * M, nkv = QT - x, lkv = a.head_kv[x];
            role[0] = 0, tile[0] = x, lo[0] = x, hi[0] = x + min(lkv, nkv);
            slot[0] = lkv < nkv ? job0 + x : -1;
        } else {
            // head piece (or all) of dQ query tile M + x
            const int x = pos - 3 * M, nq = M + x + 1, lq = a.head_q[x];
            role[0] = 1, tile[0] = M + x, lo[0] = 0, hi[0] = min(lq, nq);
            slot[0] = lq < nq ? job0 + x : -1;
        }
        head[0] = head[1] = g;
    } else {
        const int level = pos / (group + 1);
        const int r = pos % (group + 1);
        slot[0] = -1;
        if (r == 0) {
            role[0] = 0, head[0] = g, tile[0] = level, lo[0] = kCausal ? level : 0, hi[0] = QT;
        } else {
            const int b = g / a.heads_kv, hkv = g % a.heads_kv;
            const int qt = QT - 1 - level;
            role[0] = 1, head[0] = b * a.heads_q + hkv * group + r - 1, tile[0] = qt;
            lo[0] = 0, hi[0] = kCausal ? qt + 1 : QT;
        }
    }
    for (int u = 0; u < n_units; ++u) {
        const int ru = __builtin_amdgcn_readfirstlane(u == 0 ? role[0] : role[1]);
        const int hu = __builtin_amdgcn_readfirstlane(u == 0 ? head[0] : head[1]);
        const int tu = __builtin_amdgcn_readfirstlane(u == 0 ? tile[0] : tile[1]);
        const int lu = __builtin_amdgcn_readfirstlane(u == 0 ? lo[0] : lo[1]);
        const int hiu = __builtin_amdgcn_readfirstlane(u == 0 ? hi[0] : hi[1]);
        const int su = __builtin_amdgcn_readfirstlane(u == 0 ? slot[0] : slot[1]);
        const bool wd = u == 0 ? wdelta[0] : wdelta[1];
        if (u > 0) {
            wait_vm_lgkm0<0>();
            barrier();
        }
        // the arguments through an opaque pointer into the kernel-argument
        // segment: each role loads the fields it uses itself instead of all
        // of them living in SGPRs throughout
        const KernArgs* ap = (const KernArgs*)__builtin_amdgcn_kernarg_segment_ptr();
        asm volatile("" : "+s"(ap));
        if (ru == 0) dkv_role<D, kCausal, kBf16, kRows>(*ap, hu, tu, lu, hiu, su, smem);
        else dq_role<D, kCausal, kBf16, kRows>(*ap, hu, tu, lu, hiu, su, wd, smem);
    }
}

// Single-role grids of the dK/dV and dQ components (causal, one query head
// per KV head, fp16 inputs, fp32 outputs): one job per key tile (kRole 1,
// row statistics from the packed sidecar) or per query tile (kRole 2, from
// max / sum / delta), longest first.  No workspace: the statistics are folded
// in registers.
template <int D, int kRole>
__global__ __launch_bounds__(kThreads, 1) void bwd_component_kernel(MainArgs a) {
    __shared__ __attribute__((aligned(1024))) char smem_raw[Cfg<D>::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;
    int g, pos;
    job_of(a, g, pos);
    const int QT = a.seqlen / 64;
    if constexpr (kRole == 1) {
        dkv_role<D, true, false, kRowsPacked>(a, g, pos, pos, QT, -1, smem);
    } else {
        const int qt = QT - 1 - pos;
        dq_role<D, true, false, kRowsMaxSum>(a, g, qt, 0, qt + 1, -1, false, smem);
    }
}


// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------
template <int D, bool kCausal, bool kBf16>
void launch_rows(const MainArgs& a, bool inline_rows, dim3 grid, hipStream_t stream) {
    if (inline_rows)
        hipLaunchKernelGGL((bwd_main_kernel<D, kCausal, kBf16, kRowsInline>), grid, dim3(kThreads),
                           0, stream, a);
    else
        hipLaunchKernelGGL((bwd_main_kernel<D, kCausal, kBf16, kRowsArrays>), grid, dim3(kThreads),
                           0, stream, a);
}

template <int D>
void launch_d(const MainArgs& a, bool causal, bool bf16, bool inline_rows, hipStream_t stream) {
    const dim3 grid(a.n_groups * a.jobs_per_group);
    if (bf16) {
        if (causal) launch_rows<D, true, true>(a, inline_rows, grid, stream);
        else launch_rows<D, false, true>(a, inline_rows, grid, stream);
    } else {
        if (causal) launch_rows<D, true, false>(a, inline_rows, grid, stream);
        else launch_rows<D, false, false>(a, inline_rows, grid, stream);
    }
}

// XCD-aware job map: n_groups groups of jobs_per_group jobs.
void set_job_map(MainArgs& a) {
    int gcd8 = 8;
    while (a.n_groups % gcd8 != 0) gcd8 >>= 1;
    const int parts = 8 / gcd8;  // smallest split with n_groups * parts % 8 == 0
    const bool fits = a.jobs_per_group % parts == 0;
    a.xcd_parts = fits ? parts : 0;
    a.part_len = fits ? a.jobs_per_group / parts : 0;
}

// Head-piece lengths of the split plan.  Workgroup times in units of one dKV
// step: a dQ step costs kQ, a unit's prologue kPro, its epilogue kWholeKv /
// kWholeQ for a whole job; of a split job, the piece that arrives first
// spends kPub* (storing its partial sums) and the second, after waiting for
// them, kAdd* (adding them and writing the output); kEntry at kernel entry
// and kGap between two units.  For each x the pair of workgroups sharing a
// job is balanced: the head length minimises the later of the two finishing
// times.
void split_heads(int M, uint16_t* head_kv, uint16_t* head_q) {
    constexpr double kQ = 0.75, kPro = 1.5, kEntry = 0.5, kGap = 0.3;
    constexpr double kWholeKv = 1.5, kWholeQ = 1.0;
    constexpr double kPubKv = 1.5, kAddKv = 2.0, kPubQ = 1.0, kAddQ = 1.3;
    // a, b: the two workgroups' times up to the end of their last steps
    auto pair_end = [](double a, double b, double pub, double add) {
        const double first = a < b ? a : b, second = a < b ? b : a;
        return (second > first + pub ? second : first + pub) + add;
    };
    const int QT = 2 * M;
    for (int x = 0; x < M; ++x) {
        // dKV key tile x (QT - x tiles): head piece alone, remainder after
        // the whole dQ job of query tile x
        int best = QT - x;
        double best_t = 1e30;
        for (int L = 1; L <= QT - x; ++L) {
            const int r = QT - x - L;
            const double c = kEntry + kPro + L;
            const double b = kEntry + kPro + (x + 1) * kQ + kWholeQ;
            const double t = r > 0 ? pair_end(c, b + kGap + kPro + r, kPubKv, kAddKv)
                                   : (c + kWholeKv > b ? c + kWholeKv : b);
            if (t < best_t) {
                best_t = t;
                best = L;
            }
        }
        head_kv[x] = (uint16_t)best;
        // dQ query tile M + x (M + x + 1 tiles): head piece alone, remainder
        // after the whole dKV job of key tile M + x (M - x tiles)
        best = M + x + 1;
        best_t = 1e30;
        for (int L = 1; L <= M + x + 1; ++L) {
            const int r = M + x + 1 - L;
            const double d = kEntry + kPro + L * kQ;
            const double av = kEntry + kPro + (M - x) + kWholeKv;
            const double t = r > 0 ? pair_end(d, av + kGap + kPro + r * kQ, kPubQ, kAddQ)
                                   : (d + kWholeQ > av ? d + kWholeQ : av);
            if (t < best_t) {
                best_t = t;
                best = L;
            }
        }
        head_q[x] = (uint16_t)best;
    }
}

MainArgs base_args(const BwdProblem& p, const BwdTensors& t) {
    MainArgs a{};
    a.q = (const _Float16*)t.q;
    a.k = (const _Float16*)t.k;
    a.v = (const _Float16*)t.v;
    a.dout = (const _Float16*)t.dout;
    a.out = (const _Float16*)t.out;
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
    a.n_groups = p.batch * p.heads_kv;
    a.scale_log2 = p.scale * kLog2e;
    a.scale = p.scale;
    a.spin_limit = 1;
    return a;
}

std::atomic<int> g_spin_limit{1 << 24};

// Epochs: a process-wide counter started at a random 64-bit value, so a
// word left in a workspace by an earlier launch (of this or another
// process) practically never equals the current launch's epoch.
unsigned long long next_epoch() {
    static std::atomic<unsigned long long> counter{[] {
        std::random_device rd;
        unsigned long long x = ((unsigned long long)rd() << 32) ^ rd();
        x ^= (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count();
        return x | 1;
    }()};
    unsigned long long e;
    do e = counter.fetch_add(1, std::memory_order_relaxed);
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

WorkspacePlan plan_workspace(const BwdProblem& p, bool inline_rows) {
    WorkspacePlan w;
    w.inline_rows = inline_rows;
    if (p.batch <= 0 || p.heads_q <= 0 || p.seqlen <= 0 || p.head_dim <= 0) return w;
    const Checked rows = Checked{(size_t)p.batch}.mul((size_t)p.heads_q).mul((size_t)p.seqlen);
    Checked at{256};  // the error word's region
    w.err_off = 0;
    if (!inline_rows) {
        w.lse2_off = at.v;
        at = at.add(rows.mul(sizeof(float)).v).align();
        w.ndelta_off = at.v;
        at = at.add(rows.mul(sizeof(float)).v).align();
        if (!rows.ok) return w;
    }
    // Split plan for causal shapes with one query head per KV head and few
    // jobs (at most two per CU of an MI355X): see bwd_main_kernel.
    const int qt = p.seqlen / kTileM;
    const long long jobs = 2LL * p.batch * p.heads_q * qt;
    if (p.causal && p.heads_q == p.heads_kv && qt >= 4 && qt % 2 == 0 && jobs <= 512) {
        w.bal_m = qt / 2;  // <= kMaxBalM since jobs <= 512
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
    if (!at.ok || !rows.ok || rows.v > (size_t)INT32_MAX) return w;
    w.total = at.v;
    w.ok = true;
    return w;
}

hipError_t launch_component(const BwdProblem& p, const BwdTensors& t, int role) {
    MainArgs a = base_args(p, t);
    a.packed = t.packed_in;
    a.smax = t.aux0;
    a.ssum = t.aux1;
    a.delta_in = t.delta_in;
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

hipError_t launch_backward(const BwdProblem& p, const BwdTensors& t, void* workspace,
                           unsigned long long* epoch) {
    const bool inline_rows = t.aux_is_lse && t.packed_in == nullptr;
    const WorkspacePlan plan = plan_workspace(p, inline_rows);
    if (!plan.ok) return hipErrorInvalidValue;
    char* ws = static_cast<char*>(workspace);
    MainArgs a = base_args(p, t);
    if (inline_rows) {
        a.lse = t.aux0;
        a.delta_out = t.delta;
    } else {
        float* lse2 = reinterpret_cast<float*>(ws + plan.lse2_off);
        float* ndelta = reinterpret_cast<float*>(ws + plan.ndelta_off);
        const hipError_t err = t.packed_in != nullptr ? launch_rowstats(p, t, lse2, ndelta)
                                                      : launch_preprocess(p, t, lse2, ndelta);
        if (err != hipSuccess) return err;
        a.lse2 = lse2;
        a.ndelta = ndelta;
    }
    const int group = p.heads_q / p.heads_kv;
    a.jobs_per_group = (p.seqlen / kTileN) * (1 + group);
    set_job_map(a);
    a.epoch = next_epoch();
    if (epoch != nullptr) *epoch = a.epoch;
    a.err = reinterpret_cast<unsigned long long*>(ws + plan.err_off);
    a.spin_limit = g_spin_limit.load();
    a.bal_m = plan.bal_m;
    if (plan.bal_m > 0) {
        a.n_split = plan.n_split;
        a.sync = reinterpret_cast<unsigned long long*>(ws + plan.sync_off);
        a.part_kv = reinterpret_cast<float*>(ws + plan.pkv_off);
        a.part_q = reinterpret_cast<float*>(ws + plan.pq_off);
        a.part_kv_bytes = (uint32_t)(plan.pq_off - plan.pkv_off);
        a.part_q_bytes = (uint32_t)(plan.total - plan.pq_off);
        split_heads(plan.bal_m, a.head_kv, a.head_q);
    }
    if (p.head_dim == 128) launch_d<128>(a, p.causal, p.bf16, inline_rows, t.stream);
    else launch_d<64>(a, p.causal, p.bf16, inline_rows, t.stream);
    return hipGetLastError();
}

}  // namespace fa3
