// Delta preprocess of the FA3 backward (replaces reference
// src/dot_do_o_kernel.cpp:26-63 `dot_do_o_kernel`).
//
// Per query row r of [B, Hq, S]:
//   delta[r] = sum_d fp32(dO[r, d]) * fp32(O[r, d])          (fp32)
//   lse2[r]  = LSE[r] * log2(e)                                 (LSE input)
//            = max[r] * scale * log2(e) + log2(sum[r])          (SMAX_SSUM)
// so that P = exp2(s * scale * log2(e) - lse2[r]).  The main kernel takes
// -lse2[r] (nlse2) and -delta[r] (ndelta), which seed its S and dP
// accumulators so that they end at S c - lse2 and dP - delta.  Each output
// is optional (null pointer: not written).
// Optionally also writes the reference's packed sidecar
// [row_max_log2, row_inv_sum, delta] (reference src/dot_do_o_kernel.cpp:49-61).
//
// HBM-bound: D / 8 lanes per row, each with one 16-byte load of dO and one of
// O (so every load of the launch is in flight at once), an in-register dot and
// a butterfly over the row's lanes (row_delta).
#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"

namespace fa3 {
namespace {

// Zeroes the main kernel's job-queue counters and exit count (block 0, one
// lane per word; agent-scope stores, as the words are used by agent-scope
// atomics).
__device__ __forceinline__ void clear_queues(unsigned int* queue) {
    if (queue != nullptr && blockIdx.x == 0 && threadIdx.x <= kQueues)
        __hip_atomic_store(queue + (threadIdx.x < kQueues ? kQueueStride * threadIdx.x
                                                           : kQueueExitWord),
                           0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Rows are [B, Hq, S]; O / dO element strides of one sequence row (q_rs) and
// one head (q_hs) cover BHSD and BSHD; kBf16: O / dO are bf16.
template <int D, bool kLse, bool kBf16>
__global__ __launch_bounds__(256) void preprocess_kernel(
    const _Float16* __restrict__ dout, const _Float16* __restrict__ out,
    const float* __restrict__ aux0, const float* __restrict__ aux1,
    float* __restrict__ delta, float* __restrict__ nlse2, float* __restrict__ ndelta,
    float* __restrict__ packed, unsigned int* __restrict__ queue, int rows,
    float scale_log2, int heads_q, int seqlen, int q_rs, int q_hs) {
    clear_queues(queue);
    constexpr int kLanesPerRow = D / 8;
    constexpr int kRowsPerBlock = 256 / kLanesPerRow;
    const int sub = threadIdx.x % kLanesPerRow;
    const int row = blockIdx.x * kRowsPerBlock + threadIdx.x / kLanesPerRow;
    if (row >= rows) return;  // rows % kRowsPerBlock may be non-zero only at the tail

    // The row's statistics are loaded by every lane of the row, beside its
    // O / dO loads, so the kernel waits out one memory round trip, not two.
    const float a0 = aux0[row];
    const float a1 = kLse ? 0.f : aux1[row];
    size_t elem;
    if (q_rs == D && q_hs == seqlen * D) {
        elem = (size_t)row * D;  // BHSD: O / dO rows in the order of the statistics rows
    } else {
        const int hs = heads_q * seqlen;
        const int b = row / hs, rem = row - b * hs, h = rem / seqlen, sq = rem - h * seqlen;
        elem = (size_t)b * hs * D + (size_t)h * q_hs + (size_t)sq * q_rs;
    }
    const float acc = row_delta<D, kBf16>(dout, out, elem, sub);

    if (sub == 0) {
        float l2, max_log2, inv_sum;
        if constexpr (kLse) {
            l2 = a0 * kLog2e;
            max_log2 = l2;
            inv_sum = 1.f;
        } else {
            const float s = a1;
            max_log2 = a0 * scale_log2;
            inv_sum = s != 0.f ? 1.f / s : 0.f;
            l2 = max_log2 + log2f(s);
        }
        if (delta != nullptr) delta[row] = acc;
        if (nlse2 != nullptr) nlse2[row] = -l2;
        if (ndelta != nullptr) ndelta[row] = -acc;
        if (packed != nullptr) {
            packed[(size_t)row * 3 + 0] = max_log2;
            packed[(size_t)row * 3 + 1] = inv_sum;
            packed[(size_t)row * 3 + 2] = acc;
        }
    }
}

template <int D>
hipError_t launch_pre_d(const BwdProblem& p, const BwdTensors& t, float* nlse2, float* ndelta,
                        unsigned int* queue) {
    constexpr int kRowsPerBlock = 256 / (D / 8);
    const int rows = p.batch * p.heads_q * p.seqlen;
    const int blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    const float scale_log2 = p.scale * kLog2e;
    const int q_rs = p.bshd ? p.heads_q * D : D;
    const int q_hs = p.bshd ? D : p.seqlen * D;
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, t.stream, (const _Float16*)t.dout,
                           (const _Float16*)t.out, t.aux0, t.aux1, t.delta, nlse2, ndelta,
                           t.packed, queue, rows, scale_log2, p.heads_q, p.seqlen,
                           q_rs, q_hs);
    };
    if (t.aux_is_lse) {
        if (p.bf16) go(preprocess_kernel<D, true, true>);
        else go(preprocess_kernel<D, true, false>);
    } else {
        if (p.bf16) go(preprocess_kernel<D, false, true>);
        else go(preprocess_kernel<D, false, false>);
    }
    return hipGetLastError();
}

// Row statistics from the packed sidecar [max_log2, inv_sum, delta]
// (reference src/dot_do_o_kernel.cpp:49-61) for the fused5 entry:
// -lse2 = log2(inv_sum) - max_log2, since exp2(x - m) * inv = exp2(x - (m -
// log2 inv)), and -delta.
__global__ __launch_bounds__(256) void rowstats_kernel(const float* __restrict__ packed,
                                                       float* __restrict__ nlse2,
                                                       float* __restrict__ ndelta,
                                                       unsigned int* __restrict__ queue, int rows) {
    clear_queues(queue);
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    nlse2[r] = log2f(packed[(size_t)r * 3 + 1]) - packed[(size_t)r * 3];
    ndelta[r] = -packed[(size_t)r * 3 + 2];
}

}  // namespace

hipError_t launch_rowstats(const BwdProblem& p, const BwdTensors& t, float* nlse2, float* ndelta,
                           unsigned int* queue) {
    const int rows = p.batch * p.heads_q * p.seqlen;
    hipLaunchKernelGGL(rowstats_kernel, dim3((rows + 255) / 256), dim3(256), 0, t.stream,
                       t.packed_in, nlse2, ndelta, queue, rows);
    return hipGetLastError();
}

hipError_t launch_preprocess(const BwdProblem& p, const BwdTensors& t, float* nlse2,
                             float* ndelta, unsigned int* queue) {
    if (p.head_dim == 128) return launch_pre_d<128>(p, t, nlse2, ndelta, queue);
    if (p.head_dim == 64) return launch_pre_d<64>(p, t, nlse2, ndelta, queue);
    return hipErrorInvalidValue;
}

}  // namespace fa3
