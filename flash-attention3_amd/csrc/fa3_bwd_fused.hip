// The FA3 backward for gfx950 in one launch (replaces the reference's
// delta preprocess + fused 5-GEMM kernel + dQ / dKV reductions:
// src/dot_do_o_kernel.cpp:26-63, src/fused_bwd_kernel.cpp:1362-1671,
// src/fused_bwd_dq_reduce.cpp:27-109, and the legacy dKV / dQ kernels
// src/dkv_kernel.cpp:957-1085, src/dq_kernel.cpp:794-953).
//
// Two workgroup roles share the grid, so no workgroup ever adds into memory
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
// Both roles compute delta = rowsum(dO * O) themselves from the tiles they
// load (same fp32 operation order in both, so the values agree bitwise); the
// dQ role also writes it to softmax_d.  lse2 = LSE * log2(e) (or, for the
// legacy max/sum input, max * scale * log2(e) + log2(sum)).  The softmax scale
// is folded out of dS and applied once to dK and dQ.
//
// Wave layout: 4 waves, wave w = (w & 1, w >> 1) = (key half, query half) in
// the dKV role and (query half, key half) in the dQ role; each wave works on
// a 32 x 32 score block with v_mfma_f32_32x32x16_f16.  The two waves that
// share an output block add their partials through LDS once at the end.
// Streamed tiles are double-buffered in LDS and filled with direct-to-LDS
// loads (global_load_lds_dwordx4) one tile ahead of use.
#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"

namespace fa3 {
namespace {

struct FusedArgs {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    const _Float16* dout;
    const _Float16* out;
    const float* aux0;
    const float* aux1;
    _Float16* dq;
    _Float16* dk;
    _Float16* dv;
    float* delta_out;  // may be null
    int seqlen;
    int heads_q;
    int heads_kv;
    int batch;
    int n_kv_jobs;
    int n_q_jobs;
    float scale_log2;
    float scale;
};

template <int D>
struct Cfg {
    static constexpr int kTileBytes = 64 * D * 2;          // one [64][D] fp16 tile
    static constexpr int kKSteps = D / 16;                 // MFMA k-steps over D
    static constexpr int kMB = D / 32;                     // 32-row blocks of D
    static constexpr int kChunks = D / 8;                  // 16-byte chunks per row
    static constexpr int kLoadsPerWave = kTileBytes / 1024 / 4;
    // dKV role: per buffer Q, dO, O tiles; then wave-private delta/lse2 rows.
    static constexpr int kKvBuf = 3 * kTileBytes;
    static constexpr int kKvPriv = 2 * kKvBuf;
    static constexpr int kKvBytes = kKvPriv + 4 * 2 * 32 * 4;
    // dQ role: per buffer K, V tiles.
    static constexpr int kQBuf = 2 * kTileBytes;
    static constexpr int kQBytes = 2 * kQBuf;
    static constexpr int kBytes = kKvBytes > kQBytes ? kKvBytes : kQBytes;
    // final cross-wave exchange: 2 waves x kMB x 16 x 64 floats
    static_assert(2 * kMB * 16 * 64 * 4 <= 2 * kTileBytes, "exchange fits in the tiles");
};

// Direct-to-LDS copy of rows [row0, row0 + 64) of a row-major [*, D] fp16
// tensor into a swizzled [64][D] LDS tile; every wave moves kLoadsPerWave KB.
template <int D>
__device__ __forceinline__ void load_tile_async(FA3_LDS char* tile, const _Float16* src, int wave,
                                                int lane) {
    using C = Cfg<D>;
#pragma unroll
    for (int j = 0; j < C::kLoadsPerWave; ++j) {
        const int blk = wave * C::kLoadsPerWave + j;       // 1 KB block of the tile
        const int id = blk * 64 + lane;                    // physical 16-byte chunk
        const int row = id / C::kChunks;
        const int phys = id % C::kChunks;
        int sw;
        if constexpr (C::kChunks == 16) sw = ((row & 3) << 2) | ((row >> 2) & 3);
        else sw = swz128(row);
        const int logical = (phys ^ sw) & (C::kChunks - 1);
        __builtin_amdgcn_global_load_lds((const void*)(src + row * D + logical * 8),
                                         (FA3_LDS void*)(tile + blk * 1024), 16, 0, 0);
    }
}

__device__ __forceinline__ float fdot8(f16x8 a, f16x8 b, float acc) {
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        acc = __builtin_amdgcn_fdot2(f16x2{a[t], a[t + 1]}, f16x2{b[t], b[t + 1]}, acc, false);
    }
    return acc;
}

template <bool kLse>
__device__ __forceinline__ float lse2_of(const FusedArgs& a, size_t row) {
    if constexpr (kLse) {
        return a.aux0[row] * kLog2e;
    } else {
        return a.aux0[row] * a.scale_log2 + __builtin_amdgcn_logf(a.aux1[row]);
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ----------------------------------------------------------------------------
// dKV role
// ----------------------------------------------------------------------------
template <int D, bool kCausal, bool kLse>
__device__ void dkv_role(const FusedArgs& a, int job, FA3_LDS char* smem) {
    using C = Cfg<D>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wk = w & 1, wq = w >> 1;
    const int l32 = lane & 31, h = lane >> 5, g = lane >> 4, r16 = lane & 15;

    const int S = a.seqlen;
    const int QT = S / 64;
    const int kv_total = a.batch * a.heads_kv;
    const int kt = job / kv_total;   // longest (causal) first
    const int bkv = job % kv_total;
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
    const int bhq0 = b * a.heads_q + hkv * group;
    auto tile_of = [&](int it, int& bhq, int& qt) {
        bhq = bhq0 + it / per_head;
        qt = qt0 + it % per_head;
    };
    FA3_LDS float* priv = (FA3_LDS float*)(smem + C::kKvPriv) + w * 64;

    // prologue: tile 0 in flight, its softmax row statistic in a register
    int bhq, qt;
    tile_of(0, bhq, qt);
    {
        const size_t base = ((size_t)bhq * S + qt * 64) * D;
        load_tile_async<D>(smem, a.q + base, w, lane);
        load_tile_async<D>(smem + C::kTileBytes, a.dout + base, w, lane);
        load_tile_async<D>(smem + 2 * C::kTileBytes, a.out + base, w, lane);
    }
    float l2_cur = lse2_of<kLse>(a, (size_t)bhq * S + qt * 64 + 32 * wq + l32);

    for (int it = 0; it < n_it; ++it) {
        const int cur_qt = qt;
        FA3_LDS char* buf = smem + (it & 1) * C::kKvBuf;
        __syncthreads();  // tile `it` landed; buffer (it+1)&1 no longer read
        float l2_next = 0.f;
        if (it + 1 < n_it) {
            tile_of(it + 1, bhq, qt);
            const size_t base = ((size_t)bhq * S + qt * 64) * D;
            FA3_LDS char* nbuf = smem + ((it + 1) & 1) * C::kKvBuf;
            load_tile_async<D>(nbuf, a.q + base, w, lane);
            load_tile_async<D>(nbuf + C::kTileBytes, a.dout + base, w, lane);
            load_tile_async<D>(nbuf + 2 * C::kTileBytes, a.out + base, w, lane);
            l2_next = lse2_of<kLse>(a, (size_t)bhq * S + qt * 64 + 32 * wq + l32);
        }

        // S = Q K^T, dP = dO V^T (wave: q rows 32wq.., keys 32wk..), and the
        // lane's half of delta for row 32wq + l32 from the same dO fragments.
        f32x16 sacc = f32x16{}, pacc = f32x16{};
        float dpart = 0.f;
#pragma unroll
        for (int s = 0; s < C::kKSteps; ++s) {
            const uint32_t off = tile_off<D>(32 * wq + l32, 2 * s + h);
            const f16x8 qa = lds_read_b128(buf, off);
            const f16x8 da = lds_read_b128(buf + C::kTileBytes, off);
            const f16x8 oa = lds_read_b128(buf + 2 * C::kTileBytes, off);
            sacc = mfma_32x32x16(qa, kf[s], sacc);
            pacc = mfma_32x32x16(da, vf[s], pacc);
            dpart = fdot8(da, oa, dpart);
        }
        const float delta_row = dpart + __shfl_xor(dpart, 32);
        // wave-private broadcast of (delta, lse2) for the wave's 32 rows
        if (h == 0) {
            priv[l32] = delta_row;
            priv[32 + l32] = l2_cur;
        }
        __builtin_amdgcn_wave_barrier();

        // P, dS: lane holds key 32wk + l32, q = 32wq + 8(i/4) + 4h + i%4
        const bool diag = kCausal && (cur_qt == kt);
        f16x8 pb[2], dsb[2];
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            const f32x4 dl = *(const FA3_LDS f32x4*)(priv + 8 * a4 + 4 * h);
            const f32x4 l2 = *(const FA3_LDS f32x4*)(priv + 32 + 8 * a4 + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 4 * a4 + e;
                float p = fast_exp2(sacc[i] * a.scale_log2 - l2[e]);
                if (diag && (32 * wk + l32 > 32 * wq + 8 * a4 + 4 * h + e)) p = 0.f;
                pb[i >> 3][i & 7] = (_Float16)p;
                dsb[i >> 3][i & 7] = (_Float16)(p * (pacc[i] - dl[e]));
            }
        }

        // dV^T += dO^T P, dK^T += Q^T dS; A operands by transposed reads with
        // q = 16ks + 8u + 4h + j matching the C-register order of P / dS.
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
        l2_cur = l2_next;
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
template <int D, bool kCausal, bool kLse>
__device__ void dq_role(const FusedArgs& a, int job, FA3_LDS char* smem) {
    using C = Cfg<D>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = w & 1, wk = w >> 1;
    const int l32 = lane & 31, h = lane >> 5, g = lane >> 4, r16 = lane & 15;

    const int S = a.seqlen;
    const int QT = S / 64;
    const int q_total = a.batch * a.heads_q;
    const int qt = QT - 1 - job / q_total;  // longest (causal) first
    const int bhq = job % q_total;
    const int group = a.heads_q / a.heads_kv;
    const int b = bhq / a.heads_q;
    const int bkv = b * a.heads_kv + (bhq % a.heads_q) / group;
    const int qbase = qt * 64;
    const size_t row = (size_t)bhq * S + qbase + 32 * wq + l32;

    // B operands of S^T = K Q^T and dP^T = V dO^T: q = row, d = 16s + 8h + t;
    // delta for the row from the same dO fragments and O.
    f16x8 qf[C::kKSteps], df[C::kKSteps];
    float dpart = 0.f;
#pragma unroll
    for (int s = 0; s < C::kKSteps; ++s) {
        qf[s] = *(const f16x8*)(a.q + row * D + 16 * s + 8 * h);
        df[s] = *(const f16x8*)(a.dout + row * D + 16 * s + 8 * h);
        const f16x8 of = *(const f16x8*)(a.out + row * D + 16 * s + 8 * h);
        dpart = fdot8(df[s], of, dpart);
    }
    const float delta_row = dpart + __shfl_xor(dpart, 32);
    const float l2 = lse2_of<kLse>(a, row);
    if (a.delta_out != nullptr && wk == 0 && h == 0) a.delta_out[row] = delta_row;

    f32x16 dqt[C::kMB];
#pragma unroll
    for (int mb = 0; mb < C::kMB; ++mb) dqt[mb] = f32x16{};

    const int n_kt = kCausal ? qt + 1 : QT;
    const _Float16* kh = a.k + (size_t)bkv * S * D;
    const _Float16* vh = a.v + (size_t)bkv * S * D;
    load_tile_async<D>(smem, kh, w, lane);
    load_tile_async<D>(smem + C::kTileBytes, vh, w, lane);

    for (int kt = 0; kt < n_kt; ++kt) {
        FA3_LDS char* buf = smem + (kt & 1) * C::kQBuf;
        __syncthreads();
        if (kt + 1 < n_kt) {
            FA3_LDS char* nbuf = smem + ((kt + 1) & 1) * C::kQBuf;
            load_tile_async<D>(nbuf, kh + (size_t)(kt + 1) * 64 * D, w, lane);
            load_tile_async<D>(nbuf + C::kTileBytes, vh + (size_t)(kt + 1) * 64 * D, w, lane);
        }
        // S^T, dP^T: lane holds q = 32wq + l32, key = 32wk + 8(i/4) + 4h + i%4
        f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
        for (int s = 0; s < C::kKSteps; ++s) {
            const uint32_t off = tile_off<D>(32 * wk + l32, 2 * s + h);
            sacc = mfma_32x32x16(lds_read_b128(buf, off), qf[s], sacc);
            pacc = mfma_32x32x16(lds_read_b128(buf + C::kTileBytes, off), df[s], pacc);
        }
        const bool diag = kCausal && (kt == qt);
        f16x8 dsb[2];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float p = fast_exp2(sacc[i] * a.scale_log2 - l2);
            if (diag && (32 * wk + 8 * (i >> 2) + 4 * h + (i & 3) > 32 * wq + l32)) p = 0.f;
            dsb[i >> 3][i & 7] = (_Float16)(p * (pacc[i] - delta_row));
        }
        // dQ^T += K^T dS^T; A = K^T by transposed reads, key order matching dsb
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
    }

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

// Grid: the two roles interleaved, each in longest-first order, so the
// dispatcher starts the longest jobs first.
template <int D, bool kCausal, bool kLse>
__global__ __launch_bounds__(256, 1) void bwd_fused_kernel(FusedArgs a) {
    __shared__ __attribute__((aligned(1024))) char smem_raw[Cfg<D>::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;
    const int id = blockIdx.x;
    const int both = a.n_kv_jobs < a.n_q_jobs ? a.n_kv_jobs : a.n_q_jobs;
    bool kv;
    int job;
    if (id < 2 * both) {
        kv = (id & 1) == 0;
        job = id >> 1;
    } else {
        kv = a.n_kv_jobs > a.n_q_jobs;
        job = both + (id - 2 * both);
    }
    if (kv) dkv_role<D, kCausal, kLse>(a, job, smem);
    else dq_role<D, kCausal, kLse>(a, job, smem);
}

template <int D, bool kCausal, bool kLse>
void launch_t(const FusedArgs& a) {
    hipLaunchKernelGGL((bwd_fused_kernel<D, kCausal, kLse>), dim3(a.n_kv_jobs + a.n_q_jobs),
                       dim3(256), 0, 0, a);
}

template <int D>
void launch_d(const FusedArgs& a, bool causal, bool lse) {
    if (causal) {
        if (lse) launch_t<D, true, true>(a);
        else launch_t<D, true, false>(a);
    } else {
        if (lse) launch_t<D, false, true>(a);
        else launch_t<D, false, false>(a);
    }
}

}  // namespace

hipError_t launch_backward(const BwdProblem& p, const BwdTensors& t, void* workspace) {
    (void)workspace;
    auto mark = [&](int i) {
        if (t.stage_events[i] != nullptr) (void)hipEventRecord(t.stage_events[i], 0);
    };
    FusedArgs a;
    a.q = (const _Float16*)t.q;
    a.k = (const _Float16*)t.k;
    a.v = (const _Float16*)t.v;
    a.dout = (const _Float16*)t.dout;
    a.out = (const _Float16*)t.out;
    a.aux0 = t.aux0;
    a.aux1 = t.aux1;
    a.dq = (_Float16*)t.dq;
    a.dk = (_Float16*)t.dk;
    a.dv = (_Float16*)t.dv;
    a.delta_out = t.delta;
    a.seqlen = p.seqlen;
    a.heads_q = p.heads_q;
    a.heads_kv = p.heads_kv;
    a.batch = p.batch;
    a.n_kv_jobs = (p.seqlen / kTileN) * p.batch * p.heads_kv;
    a.n_q_jobs = (p.seqlen / kTileM) * p.batch * p.heads_q;
    a.scale_log2 = p.scale * kLog2e;
    a.scale = p.scale;
    mark(0);
    mark(1);
    if (p.head_dim == 128) launch_d<128>(a, p.causal, t.aux_is_lse);
    else launch_d<64>(a, p.causal, t.aux_is_lse);
    const hipError_t err = hipGetLastError();
    mark(2);
    mark(3);
    return err;
}

WorkspacePlan plan_workspace(const BwdProblem& p) {
    (void)p;
    WorkspacePlan w;
    w.total = 256;  // reserved; the single-launch path keeps no state in it
    w.ok = true;
    return w;
}

}  // namespace fa3
