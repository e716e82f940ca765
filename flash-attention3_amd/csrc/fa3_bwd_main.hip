// Main FA3 backward kernel for gfx950 (replaces the reference's fused 5-GEMM
// kernel src/fused_bwd_kernel.cpp:1362-1671 and the legacy dKV / dQ kernels
// src/dkv_kernel.cpp:957-1085, src/dq_kernel.cpp:794-953) plus the dQ
// finalize pass (replaces src/fused_bwd_dq_reduce.cpp:27-67).
//
// Work decomposition: one workgroup (4 waves) owns a 64-key tile of one KV
// head and streams every 64-row query tile that can see it (causal: from the
// diagonal tile on), for every query head of its GQA group.  dK/dV stay in
// fp32 registers for the whole sweep, so GQA needs no reduction pass.
// Wave w = (wk = w & 1, wq = w >> 1) owns keys [32wk, 32wk + 32) of the tile
// and query rows [32wq, 32wq + 32) of each query tile.  Per query tile:
//   S    = Q K^T              (MFMA, A = Q rows from LDS, B = K from VGPRs)
//   dP   = dO V^T             (MFMA, A = dO rows from LDS, B = V from VGPRs)
//   P    = exp2(S * scale * log2e - lse2),  dS = P * (dP - delta)
//   dV^T += dO^T P            (A = dO^T via ds_read_b64_tr_b16, B = P in VGPRs)
//   dK^T += Q^T dS            (A = Q^T  via ds_read_b64_tr_b16, B = dS in VGPRs)
//   dS^T -> LDS; dQ = dS K    (A = dS via transposed read, B = K^T in VGPRs)
//   dQ is added into an fp32 accumulator with global atomics, or (the
//   deterministic mode) stored as a per-key-tile partial and summed in order.
// The softmax scale is folded out of dS: dK and dQ are scaled once at the end.
#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"

namespace fa3 {
namespace {

struct MainArgs {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    const _Float16* dout;
    const float* lse2;
    const float* delta;
    float* dq_acc;
    _Float16* dk;
    _Float16* dv;
    int seqlen;
    int heads_q;
    int heads_kv;
    int kv_heads_total;  // batch * heads_kv
    int num_ktiles;
    float scale_log2;
    float scale;
};

// LDS map (bytes): Q tile, dO tile, dS^T tile, lse2[64], delta[64].
template <int D>
struct Lds {
    static constexpr int kTile = kTileM * D * 2;
    static constexpr int kQ = 0;
    static constexpr int kDO = kTile;
    static constexpr int kDS = 2 * kTile;
    static constexpr int kLse = kDS + kTileN * kTileM * 2;
    static constexpr int kDelta = kLse + kTileM * 4;
    static constexpr int kBytes = kDelta + kTileM * 4;
    // The final dK/dV cross-wave reduction reuses [0, 2 * kTile).
    static_assert(2 * kTile >= 2 * 32 * D * 4, "dK/dV exchange must fit in the Q/dO tiles");
};

template <int D, bool kCausal, bool kDeterministic>
__global__ __launch_bounds__(256, 1) void bwd_main_kernel(MainArgs a) {
    constexpr int kKSteps = D / 16;   // MFMA k-steps over the head dim
    constexpr int kMB = D / 32;       // 32-wide head-dim blocks (dK^T/dV^T rows)
    constexpr int kNB5 = D / 64;      // head-dim blocks per wave in dQ = dS K
    constexpr int kChunks = D / 8;    // 16-byte chunks per tile row
    using L = Lds<D>;
    __shared__ __attribute__((aligned(16))) char smem_raw[L::kBytes];
    FA3_LDS char* smem = (FA3_LDS char*)smem_raw;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int wk = w & 1;
    const int wq = w >> 1;
    const int l32 = lane & 31;
    const int h = lane >> 5;
    const int g = lane >> 4;
    const int r16 = lane & 15;

    // Longest work first: all heads' k-tile 0 before any k-tile 1 (causal
    // k-tile z sees S - 64 z query rows).
    const int kt = blockIdx.x / a.kv_heads_total;
    const int bkv = blockIdx.x % a.kv_heads_total;
    const int group = a.heads_q / a.heads_kv;
    const int b = bkv / a.heads_kv;
    const int hkv = bkv % a.heads_kv;
    const int S = a.seqlen;
    const int kbase = kt * kTileN;

    const _Float16* kp = a.k + ((size_t)bkv * S + kbase) * D;
    const _Float16* vp = a.v + ((size_t)bkv * S + kbase) * D;

    // B operands of S = Q K^T and dP = dO V^T: key 32wk + l32, d = 16s + 8h + t.
    f16x8 kf[kKSteps], vf[kKSteps];
#pragma unroll
    for (int s = 0; s < kKSteps; ++s) {
        kf[s] = *(const f16x8*)(kp + (32 * wk + l32) * D + 16 * s + 8 * h);
        vf[s] = *(const f16x8*)(vp + (32 * wk + l32) * D + 16 * s + 8 * h);
    }
    // B operand of dQ = dS K: d = (D/2) wk + 32 nb + l32, key = 16 ks + 8h + t.
    f16x8 ktf[kNB5][4];
#pragma unroll
    for (int nb = 0; nb < kNB5; ++nb) {
        const int d = (D / 2) * wk + 32 * nb + l32;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            f16x8 t;
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = kp[(16 * ks + 8 * h + j) * D + d];
            ktf[nb][ks] = t;
        }
    }

    f32x16 dkt[kMB], dvt[kMB];
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
        dkt[mb] = f32x16{};
        dvt[mb] = f32x16{};
    }

    const int qt_begin = kCausal ? kt : 0;
    const int qt_end = S / kTileM;

    for (int gi = 0; gi < group; ++gi) {
        const int bhq = b * a.heads_q + hkv * group + gi;
        const _Float16* qh = a.q + (size_t)bhq * S * D;
        const _Float16* doh = a.dout + (size_t)bhq * S * D;
        const float* lse2h = a.lse2 + (size_t)bhq * S;
        const float* deltah = a.delta + (size_t)bhq * S;

        for (int qt = qt_begin; qt < qt_end; ++qt) {
            const int qbase = qt * kTileM;
            // ---- stage the query tile (Q, dO, lse2, delta) into LDS ----
            __syncthreads();
#pragma unroll
            for (int j = 0; j < kTileM * kChunks / 256; ++j) {
                const int id = tid + 256 * j;
                const int row = id / kChunks;
                const int c = id % kChunks;
                const f16x8 qv = *(const f16x8*)(qh + (size_t)(qbase + row) * D + c * 8);
                const f16x8 dv = *(const f16x8*)(doh + (size_t)(qbase + row) * D + c * 8);
                lds_write_b128(smem + L::kQ, tile_off<D>(row, c), qv);
                lds_write_b128(smem + L::kDO, tile_off<D>(row, c), dv);
            }
            if (tid < 64) {
                ((FA3_LDS float*)(smem + L::kLse))[tid] = lse2h[qbase + tid];
            } else if (tid < 128) {
                ((FA3_LDS float*)(smem + L::kDelta))[tid - 64] = deltah[qbase + tid - 64];
            }
            __syncthreads();

            // ---- S = Q K^T and dP = dO V^T (32 q x 32 keys per wave) ----
            f32x16 sacc = f32x16{};
            f32x16 pacc = f32x16{};
#pragma unroll
            for (int s = 0; s < kKSteps; ++s) {
                const uint32_t off = tile_off<D>(32 * wq + l32, 2 * s + h);
                const f16x8 qa = lds_read_b128(smem + L::kQ, off);
                const f16x8 da = lds_read_b128(smem + L::kDO, off);
                sacc = mfma_32x32x16(qa, kf[s], sacc);
                pacc = mfma_32x32x16(da, vf[s], pacc);
            }

            // ---- P and dS; lane holds key 32wk + l32, q = 32wq + 8(i/4) + 4h + i%4 ----
            const FA3_LDS f32x4* lse4 = (const FA3_LDS f32x4*)(smem + L::kLse);
            const FA3_LDS f32x4* del4 = (const FA3_LDS f32x4*)(smem + L::kDelta);
            const bool diag = kCausal && (qt == kt);
            f16x8 pb[2], dsb[2];
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const f32x4 l2 = lse4[(32 * wq + 8 * a4 + 4 * h) / 4];
                const f32x4 dl = del4[(32 * wq + 8 * a4 + 4 * h) / 4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * a4 + e;
                    float p = exp2f(sacc[i] * a.scale_log2 - l2[e]);
                    if (diag) {
                        const int qloc = 32 * wq + 8 * a4 + 4 * h + e;
                        const int kloc = 32 * wk + l32;
                        if (kloc > qloc) p = 0.f;
                    }
                    const float ds = p * (pacc[i] - dl[e]);
                    pb[i / 8][i % 8] = (_Float16)p;
                    dsb[i / 8][i % 8] = (_Float16)ds;
                }
            }

            // ---- dS^T -> LDS ([key][q], 8-byte writes of 4 consecutive q) ----
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f16x4 v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = dsb[a4 / 2][(a4 % 2) * 4 + e];
                lds_write_b64(smem + L::kDS, dst_off(32 * wk + l32, 4 * wq + a4) + 8 * h, v4);
            }

            // ---- dV^T += dO^T P,  dK^T += Q^T dS ----
            // A operand (m = d = 32mb + l32, k = q = 16ks + 8u + 4h + j) by
            // transposed reads: lane r16 points at row (r16 >> 2) of the 4-row
            // block, column 32mb + 16(g&1) + 4(r16&3).
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int mb = 0; mb < kMB; ++mb) {
                    f16x4 ao[2], aq[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int row = 32 * wq + 16 * ks + 8 * u + 4 * h + (r16 >> 2);
                        const int col = 32 * mb + 16 * (g & 1) + 4 * (r16 & 3);
                        const uint32_t off = tile_off<D>(row, col >> 3) + (col & 7) * 2;
                        ao[u] = lds_read_tr4(smem + L::kDO, off);
                        aq[u] = lds_read_tr4(smem + L::kQ, off);
                    }
                    dvt[mb] = mfma_32x32x16(concat4(ao[0], ao[1]), pb[ks], dvt[mb]);
                    dkt[mb] = mfma_32x32x16(concat4(aq[0], aq[1]), dsb[ks], dkt[mb]);
                }
            }

            __syncthreads();  // dS^T of all four waves visible

            // ---- dQ = dS K: q rows 32wq + .., d = (D/2) wk + 32 nb + .. ----
            f32x16 dqacc[kNB5];
#pragma unroll
            for (int nb = 0; nb < kNB5; ++nb) dqacc[nb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                f16x4 rr[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int key = 16 * ks + 8 * h + 4 * u + (r16 >> 2);
                    const int col = 32 * wq + 16 * (g & 1) + 4 * (r16 & 3);
                    rr[u] = lds_read_tr4(smem + L::kDS, dst_off(key, col >> 3) + (col & 7) * 2);
                }
                const f16x8 dsa = concat4(rr[0], rr[1]);
#pragma unroll
                for (int nb = 0; nb < kNB5; ++nb) dqacc[nb] = mfma_32x32x16(dsa, ktf[nb][ks], dqacc[nb]);
            }

            // lane: d = (D/2) wk + 32 nb + l32, q = 32wq + 8(i/4) + 4h + i%4
            float* dst;
            if constexpr (kDeterministic) {
                dst = a.dq_acc + (((size_t)bhq * a.num_ktiles + kt) * S + qbase) * D;
            } else {
                dst = a.dq_acc + ((size_t)bhq * S + qbase) * D;
            }
#pragma unroll
            for (int nb = 0; nb < kNB5; ++nb) {
                const int d = (D / 2) * wk + 32 * nb + l32;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int qrow = 32 * wq + 8 * (i / 4) + 4 * h + (i % 4);
                    if constexpr (kDeterministic) {
                        dst[(size_t)qrow * D + d] = dqacc[nb][i];
                    } else {
                        atomicAdd(dst + (size_t)qrow * D + d, dqacc[nb][i]);
                    }
                }
            }
        }
    }

    // ---- combine the two query-half partials of each key half, write dK/dV ----
    // dV^T/dK^T lane layout: key = 32wk + l32, d = 32mb + 8(i/4) + 4h + i%4.
    FA3_LDS float* xch = (FA3_LDS float*)smem + wk * (kMB * 16 * 64);
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
            for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) xch[(mb * 16 + i) * 64 + lane] = acc[mb][i];
        }
        __syncthreads();
        if (wq == 0) {
#pragma unroll
            for (int mb = 0; mb < kMB; ++mb) {
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

// dQ finalize: dq = fp16(scale * acc)  (atomic mode), or the ordered sum of
// the per-key-tile partials that can be non-zero (deterministic mode; causal
// row q only has partials from key tiles 0 .. q / 64).
template <bool kDeterministic>
__global__ __launch_bounds__(256) void dq_finalize_kernel(const float* __restrict__ acc,
                                                          _Float16* __restrict__ dq,
                                                          size_t elems, int seqlen, int head_dim,
                                                          int num_ktiles, int causal, float scale) {
    const size_t i8 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i8 >= elems) return;
    f32x4 s0, s1;
    if constexpr (!kDeterministic) {
        s0 = *(const f32x4*)(acc + i8);
        s1 = *(const f32x4*)(acc + i8 + 4);
    } else {
        const size_t per_head = (size_t)seqlen * head_dim;
        const size_t bh = i8 / per_head;
        const size_t inner = i8 % per_head;
        const int row = (int)(inner / head_dim);
        const int last = causal ? row / kTileN : num_ktiles - 1;
        s0 = f32x4{};
        s1 = f32x4{};
        const float* p = acc + bh * num_ktiles * per_head + inner;
        for (int t = 0; t <= last; ++t) {
            s0 += *(const f32x4*)(p + (size_t)t * per_head);
            s1 += *(const f32x4*)(p + (size_t)t * per_head + 4);
        }
    }
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        o[e] = (_Float16)(s0[e] * scale);
        o[4 + e] = (_Float16)(s1[e] * scale);
    }
    *(f16x8*)(dq + i8) = o;
}

template <int D, bool kCausal, bool kDet>
void launch_main_t(const MainArgs& args, int blocks) {
    hipLaunchKernelGGL((bwd_main_kernel<D, kCausal, kDet>), dim3(blocks), dim3(256), 0, 0, args);
}

template <int D>
void launch_main_d(const MainArgs& args, int blocks, bool causal, bool det) {
    if (causal) {
        if (det) launch_main_t<D, true, true>(args, blocks);
        else launch_main_t<D, true, false>(args, blocks);
    } else {
        if (det) launch_main_t<D, false, true>(args, blocks);
        else launch_main_t<D, false, false>(args, blocks);
    }
}

}  // namespace

hipError_t launch_backward(const BwdProblem& p, const BwdTensors& t, void* workspace) {
    const WorkspacePlan plan = plan_workspace(p);
    if (!plan.ok || workspace == nullptr) return hipErrorInvalidValue;
    char* ws = (char*)workspace;
    float* dq_acc = (float*)(ws + plan.dq_acc_off);
    float* lse2 = (float*)(ws + plan.lse2_off);

    auto mark = [&](int i) {
        if (t.stage_events[i] != nullptr) (void)hipEventRecord(t.stage_events[i], 0);
    };
    // Atomic mode clears the accumulator rows in the preprocess pass; the
    // deterministic partials are fully overwritten where they are read.
    mark(0);
    hipError_t err = launch_preprocess(p, t, lse2, p.deterministic ? nullptr : dq_acc);
    if (err != hipSuccess) return err;

    MainArgs a;
    a.q = (const _Float16*)t.q;
    a.k = (const _Float16*)t.k;
    a.v = (const _Float16*)t.v;
    a.dout = (const _Float16*)t.dout;
    a.lse2 = lse2;
    a.delta = t.delta;
    a.dq_acc = dq_acc;
    a.dk = (_Float16*)t.dk;
    a.dv = (_Float16*)t.dv;
    a.seqlen = p.seqlen;
    a.heads_q = p.heads_q;
    a.heads_kv = p.heads_kv;
    a.kv_heads_total = p.batch * p.heads_kv;
    a.num_ktiles = p.seqlen / kTileN;
    a.scale_log2 = p.scale * kLog2e;
    a.scale = p.scale;
    const int blocks = a.num_ktiles * a.kv_heads_total;
    mark(1);
    if (p.head_dim == 128) launch_main_d<128>(a, blocks, p.causal, p.deterministic);
    else launch_main_d<64>(a, blocks, p.causal, p.deterministic);
    err = hipGetLastError();
    if (err != hipSuccess) return err;

    const size_t elems = (size_t)p.batch * p.heads_q * p.seqlen * p.head_dim;
    const int fblocks = (int)((elems / 8 + 255) / 256);
    mark(2);
    if (p.deterministic) {
        hipLaunchKernelGGL((dq_finalize_kernel<true>), dim3(fblocks), dim3(256), 0, 0, dq_acc,
                           (_Float16*)t.dq, elems, p.seqlen, p.head_dim, a.num_ktiles,
                           p.causal ? 1 : 0, p.scale);
    } else {
        hipLaunchKernelGGL((dq_finalize_kernel<false>), dim3(fblocks), dim3(256), 0, 0, dq_acc,
                           (_Float16*)t.dq, elems, p.seqlen, p.head_dim, a.num_ktiles,
                           p.causal ? 1 : 0, p.scale);
    }
    err = hipGetLastError();
    mark(3);
    return err;
}

WorkspacePlan plan_workspace(const BwdProblem& p) {
    WorkspacePlan w;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t rows = (size_t)p.batch * p.heads_q * p.seqlen;
    const size_t elems = rows * (size_t)p.head_dim;
    const size_t ktiles = (size_t)p.seqlen / kTileN;
    w.dq_acc_off = 0;
    w.dq_acc_bytes = (p.deterministic ? elems * ktiles : elems) * sizeof(float);
    w.lse2_off = align(w.dq_acc_off + w.dq_acc_bytes);
    w.delta_off = align(w.lse2_off + rows * sizeof(float));
    w.total = align(w.delta_off + rows * sizeof(float));
    w.ok = true;
    return w;
}

}  // namespace fa3
