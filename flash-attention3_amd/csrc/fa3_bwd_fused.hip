// Main FA3 backward kernel for gfx950 (replaces the reference's fused 5-GEMM
// kernel and its dQ / GQA-dKV reductions: src/fused_bwd_kernel.cpp:1362-1671,
// src/fused_bwd_dq_reduce.cpp:27-109, and the legacy dKV / dQ kernels
// src/dkv_kernel.cpp:957-1085, src/dq_kernel.cpp:794-953).  It runs after the
// delta preprocess (fa3_bwd_preprocess.hip), which supplies per query row
// delta = rowsum(dO * O) and lse2 = LSE * log2(e).
//
// Two workgroup roles share one grid, and no workgroup ever adds into memory
// another one writes (no atomics, no partial buffers, bitwise deterministic):
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
// The softmax scale is folded out of dS and applied once to dK and dQ.
//
// Wave layout: 4 waves, wave w = (w & 1, w >> 1) = (key half, query half) in
// the dKV role and (query half, key half) in the dQ role; each wave works on
// a 32 x 32 score block with v_mfma_f32_32x32x16_f16.  The two waves that
// share an output block add their partials through LDS once at the end.
//
// Pipeline: streamed tiles live in four LDS buffers filled by direct-to-LDS
// loads (global_load_lds_dwordx4) issued three tiles ahead; iteration `it`
// runs the softmax of tile it (VALU) beside S/dP of tile it+1 (MFMA), then
// the dV/dK (or dQ) MFMAs of tile it.  Waits use explicit vmcnt values so the
// loads of the following tile stay in flight across the barrier.
#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"

namespace fa3 {
namespace {

struct FusedArgs {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    const _Float16* dout;
    const float* lse2;   // [B*Hq*S]
    const float* delta;  // [B*Hq*S]
    _Float16* dq;
    _Float16* dk;
    _Float16* dv;
    int seqlen;
    int heads_q;
    int heads_kv;
    int batch;
    // job map: n_groups (batch, kv head) groups of jobs_per_group jobs; with
    // xcd_parts > 0 each group is split into xcd_parts interleaved parts of
    // part_len jobs and whole parts are pinned to one XCD.
    int n_groups;
    int jobs_per_group;
    int xcd_parts;
    int part_len;
    float scale_log2;
    float scale;
};

constexpr int kNBuf = 4;

template <int D>
struct Cfg {
    static constexpr int kTileBytes = 64 * D * 2;          // one [64][D] fp16 tile
    static constexpr int kKSteps = D / 16;                 // MFMA k-steps over D
    static constexpr int kMB = D / 32;                     // 32-row blocks of D
    static constexpr int kChunks = D / 8;                  // 16-byte chunks per row
    static constexpr int kLoadsPerWave = kTileBytes / 1024 / 4;
    // dKV role buffer: Q tile, dO tile, lse2[64], delta[64]
    static constexpr int kKvRows = 2 * kTileBytes;
    static constexpr int kKvBuf = kKvRows + 2 * 64 * 4;
    // dQ role buffer: K tile, V tile
    static constexpr int kQBuf = 2 * kTileBytes;
    static constexpr int kBytes = kNBuf * (kKvBuf > kQBuf ? kKvBuf : kQBuf);
    // final cross-wave exchange: 2 waves x kMB x 16 x 64 floats
    static_assert(2 * kMB * 16 * 64 * 4 <= kBytes, "exchange fits in the buffers");
};

// s_waitcnt vmcnt(N) leaving the LDS and export counters alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Direct-to-LDS copy of a row-major [64][D] fp16 tile into a swizzled LDS
// tile.  Lane `lane` of wave `wave` moves the 16-byte chunk that belongs at
// LDS byte blk * 1024 + lane * 16 (blk = wave * kLoadsPerWave + j); its
// source byte offset within the global tile is precomputed once.
template <int D>
__device__ __forceinline__ void tile_load_offsets(uint32_t (&off)[Cfg<D>::kLoadsPerWave],
                                                  int wave, int lane) {
    using C = Cfg<D>;
#pragma unroll
    for (int j = 0; j < C::kLoadsPerWave; ++j) {
        const int id = (wave * C::kLoadsPerWave + j) * 64 + lane;  // physical chunk
        const int row = id / C::kChunks;
        const int phys = id % C::kChunks;
        int sw;
        if constexpr (C::kChunks == 16) sw = ((row & 3) << 2) | ((row >> 2) & 3);
        else sw = swz128(row);
        const int logical = (phys ^ sw) & (C::kChunks - 1);
        off[j] = (uint32_t)((row * D + logical * 8) * 2);
    }
}

template <int D>
__device__ __forceinline__ void load_tile_async(FA3_LDS char* tile, const _Float16* src,
                                                const uint32_t (&off)[Cfg<D>::kLoadsPerWave],
                                                int wave) {
    using C = Cfg<D>;
#pragma unroll
    for (int j = 0; j < C::kLoadsPerWave; ++j) {
        __builtin_amdgcn_global_load_lds((const void*)((const char*)src + off[j]),
                                         (FA3_LDS void*)(tile + (wave * C::kLoadsPerWave + j) * 1024),
                                         16, 0, 0);
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ----------------------------------------------------------------------------
// dKV role
// ----------------------------------------------------------------------------
template <int D, bool kCausal>
__device__ void dkv_role(const FusedArgs& a, int bkv, int kt, FA3_LDS char* smem) {
    using C = Cfg<D>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wk = w & 1, wq = w >> 1;
    const int l32 = lane & 31, h = lane >> 5, g = lane >> 4, r16 = lane & 15;

    const int S = a.seqlen;
    const int QT = S / 64;
    const int group = a.heads_q / a.heads_kv;
    const int b = bkv / a.heads_kv;
    const int hkv = bkv % a.heads_kv;
    const int kbase = kt * 64;

    const _Float16* kp = a.k + ((size_t)bkv * S + kbase) * D;
    const _Float16* vp = a.v + ((size_t)bkv * S + kbase) * D;
    f16x8 kf[C::kKSteps], vf[C::kKSteps];
#pragma unroll
    for (int s = 0; s < C::kKSteps; ++s) {
        kf[s] = *(const f16x8*)(kp + (32 * wk + l32) * D + 16 * s + 8 * h);
        vf[s] = *(const f16x8*)(vp + (32 * wk + l32) * D + 16 * s + 8 * h);
    }
    f32x16 dkt[C::kMB], dvt[C::kMB];
#pragma unroll
    for (int mb = 0; mb < C::kMB; ++mb) {
        dkt[mb] = f32x16{};
        dvt[mb] = f32x16{};
    }

    const int qt0 = kCausal ? kt : 0;
    const int per_head = QT - qt0;
    const int n_it = group * per_head;
    uint32_t ld_off[C::kLoadsPerWave];
    tile_load_offsets<D>(ld_off, w, lane);

    // Tiles are issued in order; (issue_bhq, issue_qt) is the next one.
    int issue_bhq = b * a.heads_q + hkv * group;
    int issue_qt = qt0;
    auto issue_next = [&](int slot) {
        const size_t row0 = (size_t)issue_bhq * S + issue_qt * 64;
        FA3_LDS char* nb = smem + slot * C::kKvBuf;
        load_tile_async<D>(nb, a.q + row0 * D, ld_off, w);
        load_tile_async<D>(nb + C::kTileBytes, a.dout + row0 * D, ld_off, w);
        if (w == 0) {
            __builtin_amdgcn_global_load_lds((const void*)(a.lse2 + row0 + lane),
                                             (FA3_LDS void*)(nb + C::kKvRows), 4, 0, 0);
        } else if (w == 1) {
            __builtin_amdgcn_global_load_lds((const void*)(a.delta + row0 + lane),
                                             (FA3_LDS void*)(nb + C::kKvRows + 256), 4, 0, 0);
        }
        if (++issue_qt == QT) {
            issue_qt = qt0;
            ++issue_bhq;
        }
    };
    // vmcnt allowing `tiles` tiles of this wave's loads to stay in flight
    auto wait_tiles = [&](int tiles) {
        if (w < 2) {
            if (tiles >= 2) wait_vmcnt<2 * (2 * C::kLoadsPerWave + 1)>();
            else if (tiles == 1) wait_vmcnt<2 * C::kLoadsPerWave + 1>();
            else wait_vmcnt<0>();
        } else {
            if (tiles >= 2) wait_vmcnt<2 * (2 * C::kLoadsPerWave)>();
            else if (tiles == 1) wait_vmcnt<2 * C::kLoadsPerWave>();
            else wait_vmcnt<0>();
        }
    };

    // S = Q K^T, dP = dO V^T (wave: q rows 32wq.., keys 32wk..)
    auto stage_a = [&](FA3_LDS char* buf, f32x16& sacc, f32x16& pacc) {
        sacc = f32x16{};
        pacc = f32x16{};
#pragma unroll
        for (int s = 0; s < C::kKSteps; ++s) {
            const uint32_t off = tile_off<D>(32 * wq + l32, 2 * s + h);
            sacc = mfma_32x32x16(lds_read_b128(buf, off), kf[s], sacc);
            pacc = mfma_32x32x16(lds_read_b128(buf + C::kTileBytes, off), vf[s], pacc);
        }
    };
    // P and dS; lane holds key 32wk + l32, q = 32wq + 8(i/4) + 4h + i%4.
    auto stage_b = [&](auto masked, const f32x16& sacc, const f32x16& pacc,
                       const FA3_LDS char* buf, f16x8 (&pb)[2], f16x8 (&dsb)[2]) {
        const FA3_LDS float* rows = (const FA3_LDS float*)(buf + C::kKvRows);
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            const f32x4 l2 = *(const FA3_LDS f32x4*)(rows + 32 * wq + 8 * a4 + 4 * h);
            const f32x4 dl = *(const FA3_LDS f32x4*)(rows + 64 + 32 * wq + 8 * a4 + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 4 * a4 + e;
                float p = fast_exp2(sacc[i] * a.scale_log2 - l2[e]);
                if constexpr (decltype(masked)::value) {
                    if (32 * wk + l32 > 32 * wq + 8 * a4 + 4 * h + e) p = 0.f;
                }
                pb[i >> 3][i & 7] = (_Float16)p;
                dsb[i >> 3][i & 7] = (_Float16)(p * (pacc[i] - dl[e]));
            }
        }
    };
    // dV^T += dO^T P, dK^T += Q^T dS; A operands by transposed reads with
    // q = 16ks + 8u + 4h + j matching the C-register order of P / dS.
    auto stage_c = [&](FA3_LDS char* buf, const f16x8 (&pb)[2], const f16x8 (&dsb)[2]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int mb = 0; mb < C::kMB; ++mb) {
                f16x4 ao[2], aq[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int row = 32 * wq + 16 * ks + 8 * u + 4 * h + (r16 >> 2);
                    const int col = 32 * mb + 16 * (g & 1) + 4 * (r16 & 3);
                    const uint32_t off = tile_off<D>(row, col >> 3) + (col & 7) * 2;
                    ao[u] = lds_read_tr4(buf + C::kTileBytes, off);
                    aq[u] = lds_read_tr4(buf, off);
                }
                dvt[mb] = mfma_32x32x16(concat4(ao[0], ao[1]), pb[ks], dvt[mb]);
                dkt[mb] = mfma_32x32x16(concat4(aq[0], aq[1]), dsb[ks], dkt[mb]);
            }
        }
    };
    // One pipeline step on tile `it`: softmax of it, S/dP of it+1, dV/dK of
    // it.  The last step computes S/dP on a stale buffer and drops them, so
    // every step has the same straight-line body.
    auto step = [&](auto masked, int it, f32x16& sacc, f32x16& pacc) {
        const int slot = it & (kNBuf - 1);
        if (it + 1 < n_it) {
            wait_tiles(it + 2 < n_it ? 1 : 0);  // tile it+1 landed everywhere
            __builtin_amdgcn_s_barrier();        // and tile it-1's buffer is free
            if (it + 3 < n_it) issue_next((it + 3) & (kNBuf - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
        f16x8 pb[2], dsb[2];
        FA3_LDS char* buf = smem + slot * C::kKvBuf;
        stage_b(masked, sacc, pacc, buf, pb, dsb);
        stage_a(smem + ((slot + 1) & (kNBuf - 1)) * C::kKvBuf, sacc, pacc);
        stage_c(buf, pb, dsb);
        __builtin_amdgcn_sched_barrier(0);
    };

    // prologue: up to three tiles in flight, S/dP of tile 0
    const int pre = n_it < 3 ? n_it : 3;
    for (int i = 0; i < pre; ++i) issue_next(i);
    wait_tiles(pre - 1);
    __builtin_amdgcn_s_barrier();
    f32x16 sacc, pacc;
    stage_a(smem, sacc, pacc);

    // The causal diagonal is the first query tile of every head in the group.
    int it = 0;
    for (int gi = 0; gi < group; ++gi) {
        if (kCausal) step(std::true_type{}, it, sacc, pacc);
        else step(std::false_type{}, it, sacc, pacc);
        ++it;
        for (int j = 1; j < per_head; ++j, ++it) step(std::false_type{}, it, sacc, pacc);
    }

    // Combine the two query-half partials; lane: key 32wk + l32,
    // d = 32mb + 8(i/4) + 4h + i%4.
    FA3_LDS float* xch = (FA3_LDS float*)smem + wk * (C::kMB * 16 * 64);
    _Float16* dkp = a.dk + ((size_t)bkv * S + kbase + 32 * wk + l32) * D;
    _Float16* dvp = a.dv + ((size_t)bkv * S + kbase + 32 * wk + l32) * D;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        f32x16* acc = pass == 0 ? dvt : dkt;
        const float mul = pass == 0 ? 1.f : a.scale;
        _Float16* outp = pass == 0 ? dvp : dkp;
        __syncthreads();
        if (wq == 1) {
#pragma unroll
            for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) xch[(mb * 16 + i) * 64 + lane] = acc[mb][i];
        }
        __syncthreads();
        if (wq == 0) {
#pragma unroll
            for (int mb = 0; mb < C::kMB; ++mb) {
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4) {
                    f16x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * a4 + e;
                        o[e] = (_Float16)((acc[mb][i] + xch[(mb * 16 + i) * 64 + lane]) * mul);
                    }
                    *(f16x4*)(outp + 32 * mb + 8 * a4 + 4 * h) = o;
                }
            }
        }
    }
}

// ----------------------------------------------------------------------------
// dQ role
// ----------------------------------------------------------------------------
template <int D, bool kCausal>
__device__ void dq_role(const FusedArgs& a, int bhq, int qt, FA3_LDS char* smem) {
    using C = Cfg<D>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = w & 1, wk = w >> 1;
    const int l32 = lane & 31, h = lane >> 5, g = lane >> 4, r16 = lane & 15;

    const int S = a.seqlen;
    const int QT = S / 64;
    const int group = a.heads_q / a.heads_kv;
    const int b = bhq / a.heads_q;
    const int bkv = b * a.heads_kv + (bhq % a.heads_q) / group;
    const int qbase = qt * 64;
    const size_t row = (size_t)bhq * S + qbase + 32 * wq + l32;

    // B operands of S^T = K Q^T and dP^T = V dO^T: q = row, d = 16s + 8h + t
    f16x8 qf[C::kKSteps], df[C::kKSteps];
#pragma unroll
    for (int s = 0; s < C::kKSteps; ++s) {
        qf[s] = *(const f16x8*)(a.q + row * D + 16 * s + 8 * h);
        df[s] = *(const f16x8*)(a.dout + row * D + 16 * s + 8 * h);
    }
    const float l2 = a.lse2[row];
    const float delta_row = a.delta[row];

    f32x16 dqt[C::kMB];
#pragma unroll
    for (int mb = 0; mb < C::kMB; ++mb) dqt[mb] = f32x16{};

    const int n_kt = kCausal ? qt + 1 : QT;
    const _Float16* kh = a.k + (size_t)bkv * S * D;
    const _Float16* vh = a.v + (size_t)bkv * S * D;
    uint32_t ld_off[C::kLoadsPerWave];
    tile_load_offsets<D>(ld_off, w, lane);
    int issue_kt = 0;
    auto issue_next = [&](int slot) {
        FA3_LDS char* nb = smem + slot * C::kQBuf;
        load_tile_async<D>(nb, kh + (size_t)issue_kt * 64 * D, ld_off, w);
        load_tile_async<D>(nb + C::kTileBytes, vh + (size_t)issue_kt * 64 * D, ld_off, w);
        ++issue_kt;
    };
    auto wait_tiles = [&](int tiles) {
        if (tiles >= 2) wait_vmcnt<2 * (2 * C::kLoadsPerWave)>();
        else if (tiles == 1) wait_vmcnt<2 * C::kLoadsPerWave>();
        else wait_vmcnt<0>();
    };
    // S^T, dP^T: lane holds q = 32wq + l32, key = 32wk + 8(i/4) + 4h + i%4
    auto stage_a = [&](FA3_LDS char* buf, f32x16& sacc, f32x16& pacc) {
        sacc = f32x16{};
        pacc = f32x16{};
#pragma unroll
        for (int s = 0; s < C::kKSteps; ++s) {
            const uint32_t off = tile_off<D>(32 * wk + l32, 2 * s + h);
            sacc = mfma_32x32x16(lds_read_b128(buf, off), qf[s], sacc);
            pacc = mfma_32x32x16(lds_read_b128(buf + C::kTileBytes, off), df[s], pacc);
        }
    };
    auto stage_b = [&](auto masked, const f32x16& sacc, const f32x16& pacc, f16x8 (&dsb)[2]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float p = fast_exp2(sacc[i] * a.scale_log2 - l2);
            if constexpr (decltype(masked)::value) {
                if (32 * wk + 8 * (i >> 2) + 4 * h + (i & 3) > 32 * wq + l32) p = 0.f;
            }
            dsb[i >> 3][i & 7] = (_Float16)(p * (pacc[i] - delta_row));
        }
    };
    // dQ^T += K^T dS^T; A = K^T by transposed reads, key order matching dsb
    auto stage_c = [&](FA3_LDS char* buf, const f16x8 (&dsb)[2]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int mb = 0; mb < C::kMB; ++mb) {
                f16x4 ak[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int krow = 32 * wk + 16 * ks + 8 * u + 4 * h + (r16 >> 2);
                    const int col = 32 * mb + 16 * (g & 1) + 4 * (r16 & 3);
                    ak[u] = lds_read_tr4(buf, tile_off<D>(krow, col >> 3) + (col & 7) * 2);
                }
                dqt[mb] = mfma_32x32x16(concat4(ak[0], ak[1]), dsb[ks], dqt[mb]);
            }
        }
    };

    auto step = [&](auto masked, int kt, f32x16& sacc, f32x16& pacc) {
        const int slot = kt & (kNBuf - 1);
        if (kt + 1 < n_kt) {
            wait_tiles(kt + 2 < n_kt ? 1 : 0);
            __builtin_amdgcn_s_barrier();
            if (kt + 3 < n_kt) issue_next((kt + 3) & (kNBuf - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
        f16x8 dsb[2];
        stage_b(masked, sacc, pacc, dsb);
        stage_a(smem + ((slot + 1) & (kNBuf - 1)) * C::kQBuf, sacc, pacc);
        stage_c(smem + slot * C::kQBuf, dsb);
        __builtin_amdgcn_sched_barrier(0);
    };

    const int pre = n_kt < 3 ? n_kt : 3;
    for (int i = 0; i < pre; ++i) issue_next(i);
    wait_tiles(pre - 1);
    __builtin_amdgcn_s_barrier();
    f32x16 sacc, pacc;
    stage_a(smem, sacc, pacc);
    // key tiles before the last are below the causal diagonal
    for (int kt = 0; kt + 1 < n_kt; ++kt) step(std::false_type{}, kt, sacc, pacc);
    if (kCausal) step(std::true_type{}, n_kt - 1, sacc, pacc);
    else step(std::false_type{}, n_kt - 1, sacc, pacc);

    // Combine the two key-half partials; lane: q = 32wq + l32,
    // d = 32mb + 8(i/4) + 4h + i%4.
    FA3_LDS float* xch = (FA3_LDS float*)smem + wq * (C::kMB * 16 * 64);
    __syncthreads();
    if (wk == 1) {
#pragma unroll
        for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) xch[(mb * 16 + i) * 64 + lane] = dqt[mb][i];
    }
    __syncthreads();
    if (wk == 0) {
        _Float16* dqp = a.dq + row * D;
#pragma unroll
        for (int mb = 0; mb < C::kMB; ++mb) {
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f16x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * a4 + e;
                    o[e] = (_Float16)((dqt[mb][i] + xch[(mb * 16 + i) * 64 + lane]) * a.scale);
                }
                *(f16x4*)(dqp + 32 * mb + 8 * a4 + 4 * h) = o;
            }
        }
    }
}

// Job map.  Jobs are grouped by (batch, kv head) -- a group's dKV jobs and
// the dQ jobs of its query heads touch only that head's Q, dO, K, V.  Within
// a group, position p = (level L, slot r) with G + 1 slots per level: slot 0
// is the dKV job of key tile L, slot r > 0 the dQ job of query head r - 1 at
// query tile QT - 1 - L, so the dispatch order is longest first (causal).
// The hardware deals consecutive workgroup ids round-robin to the 8 XCDs;
// when the shape allows, block id -> (xcd, position) is arranged so that each
// XCD runs whole parts of groups, keeping a head's tiles in one L2.
template <int D, bool kCausal>
__global__ __launch_bounds__(256, 1) void bwd_fused_kernel(FusedArgs a) {
    __shared__ __attribute__((aligned(1024))) char smem_raw[Cfg<D>::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;
    const int id = blockIdx.x;
    int g, pos;
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
    const int group = a.heads_q / a.heads_kv;
    const int QT = a.seqlen / 64;
    const int level = pos / (group + 1);
    const int slot = pos % (group + 1);
    if (slot == 0) {
        dkv_role<D, kCausal>(a, g, level, smem);
    } else {
        const int b = g / a.heads_kv, hkv = g % a.heads_kv;
        dq_role<D, kCausal>(a, b * a.heads_q + hkv * group + slot - 1, QT - 1 - level, smem);
    }
}

template <int D>
void launch_d(const FusedArgs& a, bool causal) {
    const dim3 grid(a.n_groups * a.jobs_per_group);
    if (causal) hipLaunchKernelGGL((bwd_fused_kernel<D, true>), grid, dim3(256), 0, 0, a);
    else hipLaunchKernelGGL((bwd_fused_kernel<D, false>), grid, dim3(256), 0, 0, a);
}

}  // namespace

hipError_t launch_backward(const BwdProblem& p, const BwdTensors& t, void* workspace) {
    auto mark = [&](int i) {
        if (t.stage_events[i] != nullptr) (void)hipEventRecord(t.stage_events[i], 0);
    };
    const WorkspacePlan plan = plan_workspace(p);
    char* ws = static_cast<char*>(workspace);
    float* lse2 = reinterpret_cast<float*>(ws + plan.lse2_off);
    BwdTensors pre = t;
    if (pre.delta == nullptr) pre.delta = reinterpret_cast<float*>(ws + plan.delta_off);

    mark(0);
    hipError_t err = launch_preprocess(p, pre, lse2, nullptr);
    if (err != hipSuccess) return err;
    mark(1);

    FusedArgs a;
    a.q = (const _Float16*)t.q;
    a.k = (const _Float16*)t.k;
    a.v = (const _Float16*)t.v;
    a.dout = (const _Float16*)t.dout;
    a.lse2 = lse2;
    a.delta = pre.delta;
    a.dq = (_Float16*)t.dq;
    a.dk = (_Float16*)t.dk;
    a.dv = (_Float16*)t.dv;
    a.seqlen = p.seqlen;
    a.heads_q = p.heads_q;
    a.heads_kv = p.heads_kv;
    a.batch = p.batch;
    a.n_groups = p.batch * p.heads_kv;
    a.jobs_per_group = (p.seqlen / kTileN) * (1 + p.heads_q / p.heads_kv);
    {
        int gcd8 = 8;
        while (a.n_groups % gcd8 != 0) gcd8 >>= 1;
        const int parts = 8 / gcd8;  // smallest split with n_groups * parts % 8 == 0
        const bool fits = a.jobs_per_group % parts == 0;
        a.xcd_parts = fits ? parts : 0;
        a.part_len = fits ? a.jobs_per_group / parts : 0;
    }
    a.scale_log2 = p.scale * kLog2e;
    a.scale = p.scale;
    if (p.head_dim == 128) launch_d<128>(a, p.causal);
    else launch_d<64>(a, p.causal);
    err = hipGetLastError();
    mark(2);
    mark(3);
    return err;
}

WorkspacePlan plan_workspace(const BwdProblem& p) {
    WorkspacePlan w;
    const size_t rows = (size_t)p.batch * p.heads_q * p.seqlen;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    w.lse2_off = 0;
    w.delta_off = align(rows * sizeof(float));
    w.total = align(w.delta_off + rows * sizeof(float));
    w.ok = true;
    return w;
}

}  // namespace fa3
