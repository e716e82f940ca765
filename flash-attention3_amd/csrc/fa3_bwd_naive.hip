// Naive fp32 backward of the dK/dV and dQ components' correctness path
// (dkv_path / dq_path 1; replaces the reference's fa3_bwd_dkv_ref_* and
// fa3_bwd_dq_ref_* kernels, src/dkv_kernel.cpp:1086-1266 and
// src/dq_kernel.cpp:955-1129, dispatched at src/dkv_kernel.cpp:1319-1383 and
// src/dq_kernel.cpp:1562-1625).
//
// It ignores O and the forward's row statistics and recomputes everything
// from Q, K, V, dO in fp32 (fp16 inputs, BHSD, one query head per KV head),
// through the reference's S^2-sized workspace, laid out as the reference
// lays it out (fp32, consecutive):
//   prob [rows][S]   P = softmax(Q K^T scale), 0 where causally masked
//   dp   [rows][S]   dP = dO V^T, 0 where masked
//   row_max [rows]   max_k (q . k) scale over the visible keys
//   row_sum [rows]   sum_k exp((q . k) scale - row_max)
//   delta [rows]     sum_d dO[d] (P V)[d]   (O recomputed in fp32)
// and then
//   dK[k][d] = sum_q P[q][k] (dP[q][k] - delta[q]) scale Q[q][d]
//   dV[k][d] = sum_q P[q][k] dO[q][d]
//   dQ[q][d] = sum_k P[q][k] (dP[q][k] - delta[q]) scale K[k][d]
// written as fp32.  Correctness-oriented: one workgroup per query row for
// the workspace, one thread per output element.
#include "fa3_bwd_device.h"
#include "fa3_bwd_internal.h"

namespace fa3 {
namespace {

constexpr int kRowThreads = 256;
constexpr int kMaxD = 128;

// Block-wide reduction of one float over kRowThreads threads (max or sum).
template <bool kMax>
__device__ __forceinline__ float block_reduce(float x, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float y = __shfl_xor(x, off, 64);
        x = kMax ? fmaxf(x, y) : x + y;
    }
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();  // red is free (its last readers are done)
    if (lane == 0) red[w] = x;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kRowThreads / 64; ++i) r = kMax ? fmaxf(r, red[i]) : r + red[i];
    return r;
}

// One query row per workgroup: prob, dp, row_max, row_sum, delta.
__global__ __launch_bounds__(kRowThreads) void naive_rows_kernel(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k,
    const _Float16* __restrict__ v, const _Float16* __restrict__ dout, float* __restrict__ prob,
    float* __restrict__ dp, float* __restrict__ row_max, float* __restrict__ row_sum,
    float* __restrict__ delta, int seqlen, int dim, int causal, float scale) {
    __shared__ float qrow[kMaxD], dorow_f[kMaxD], red[kRowThreads / 64];
    __shared__ float part[kRowThreads];
    const size_t row = blockIdx.x;  // (b * heads + h) * seqlen + s
    const int s = (int)(row % seqlen);
    const size_t head = row / seqlen;
    const _Float16* kh = k + head * seqlen * dim;
    const _Float16* vh = v + head * seqlen * dim;
    const _Float16* dorow = dout + row * dim;
    float* p = prob + row * seqlen;
    float* dpr = dp + row * seqlen;
    const int tid = threadIdx.x;
    for (int d = tid; d < dim; d += kRowThreads) {
        qrow[d] = (float)q[row * dim + d];
        dorow_f[d] = (float)dorow[d];
    }
    __syncthreads();
    const int visible = causal ? s + 1 : seqlen;  // keys 0 .. visible - 1
    // scaled scores into prob, and dP
    float mx = -3.4028234663852886e38f;
    for (int j = tid; j < seqlen; j += kRowThreads) {
        float sc = 0.f, dpv = 0.f;
        if (j < visible) {
            for (int d = 0; d < dim; ++d) {
                sc += qrow[d] * (float)kh[(size_t)j * dim + d];
                dpv += dorow_f[d] * (float)vh[(size_t)j * dim + d];
            }
            sc *= scale;
            mx = fmaxf(mx, sc);
        }
        p[j] = sc;
        dpr[j] = dpv;
    }
    mx = block_reduce<true>(mx, red);
    float sum = 0.f;
    for (int j = tid; j < seqlen; j += kRowThreads) {
        const float e = j < visible ? expf(p[j] - mx) : 0.f;
        p[j] = e;
        sum += e;
    }
    sum = block_reduce<false>(sum, red);
    const float inv = sum != 0.f ? 1.f / sum : 0.f;
    for (int j = tid; j < seqlen; j += kRowThreads) p[j] *= inv;
    __syncthreads();  // every thread's prob entries are written
    // O = P V in fp32: thread pair (d, half) sums half of the keys
    const int d = tid % kMaxD, half = tid / kMaxD;
    float o = 0.f;
    if (d < dim) {
        for (int j = half; j < visible; j += 2) o += p[j] * (float)vh[(size_t)j * dim + d];
    }
    part[tid] = o;
    __syncthreads();
    float dl = 0.f;
    if (tid < dim) dl = dorow_f[tid] * (part[tid] + part[tid + kMaxD]);
    dl = block_reduce<false>(dl, red);
    if (tid == 0) {
        row_max[row] = mx;
        row_sum[row] = sum;
        delta[row] = dl;
    }
}

// dK / dV of key j of one head: thread d of workgroup (head, j).
__global__ void naive_dkv_kernel(const _Float16* __restrict__ q, const _Float16* __restrict__ dout,
                                 const float* __restrict__ prob, const float* __restrict__ dp,
                                 const float* __restrict__ delta, float* __restrict__ dk,
                                 float* __restrict__ dv, int seqlen, int dim, int causal,
                                 float scale) {
    const size_t key_row = blockIdx.x;  // (b * heads + h) * seqlen + j
    const int j = (int)(key_row % seqlen);
    const size_t head = key_row / seqlen;
    const int d = threadIdx.x;
    if (d >= dim) return;
    float ak = 0.f, av = 0.f;
    for (int s = causal ? j : 0; s < seqlen; ++s) {
        const size_t row = head * seqlen + s;
        const size_t pair = row * seqlen + j;
        const float pv = prob[pair];
        av += pv * (float)dout[row * dim + d];
        ak += pv * (dp[pair] - delta[row]) * scale * (float)q[row * dim + d];
    }
    dk[key_row * dim + d] = ak;
    dv[key_row * dim + d] = av;
}

// dQ of query row s of one head: thread d of workgroup (head, s).
__global__ void naive_dq_kernel(const _Float16* __restrict__ k, const float* __restrict__ prob,
                                const float* __restrict__ dp, const float* __restrict__ delta,
                                float* __restrict__ dq, int seqlen, int dim, int causal,
                                float scale) {
    const size_t row = blockIdx.x;
    const int s = (int)(row % seqlen);
    const size_t head = row / seqlen;
    const int d = threadIdx.x;
    if (d >= dim) return;
    const float dl = delta[row];
    float acc = 0.f;
    const int visible = causal ? s + 1 : seqlen;
    for (int j = 0; j < visible; ++j) {
        const size_t pair = row * seqlen + j;
        acc += prob[pair] * (dp[pair] - dl) * scale * (float)k[(head * seqlen + j) * dim + d];
    }
    dq[row * dim + d] = acc;
}

}  // namespace

size_t naive_workspace_bytes(const BwdProblem& p) {
    if (p.batch <= 0 || p.heads_q <= 0 || p.seqlen <= 0) return 0;
    size_t rows = 0, pairs = 0, n = 0, bytes = 0;
    // rows <= 2^31 - 1: the row kernel's grid
    if (__builtin_mul_overflow((size_t)p.batch, (size_t)p.heads_q, &rows) ||
        __builtin_mul_overflow(rows, (size_t)p.seqlen, &rows) || rows > 0x7FFFFFFFu ||
        __builtin_mul_overflow(rows, (size_t)p.seqlen, &pairs) ||
        __builtin_mul_overflow(pairs, (size_t)2, &n) || __builtin_add_overflow(n, 3 * rows, &n) ||
        __builtin_mul_overflow(n, sizeof(float), &bytes)) {
        return 0;
    }
    return bytes;
}

hipError_t launch_naive(const BwdProblem& p, const BwdTensors& t, void* workspace, int role) {
    if (p.head_dim > kMaxD) return hipErrorInvalidValue;
    const size_t rows = (size_t)p.batch * p.heads_q * p.seqlen;
    const size_t pairs = rows * p.seqlen;
    float* prob = static_cast<float*>(workspace);
    float* dp = prob + pairs;
    float* row_max = dp + pairs;
    float* row_sum = row_max + rows;
    float* delta = row_sum + rows;
    const auto* q = static_cast<const _Float16*>(t.q);
    const auto* k = static_cast<const _Float16*>(t.k);
    const auto* v = static_cast<const _Float16*>(t.v);
    const auto* dout = static_cast<const _Float16*>(t.dout);
    hipLaunchKernelGGL(naive_rows_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0, t.stream, q,
                       k, v, dout, prob, dp, row_max, row_sum, delta, p.seqlen, p.head_dim,
                       p.causal ? 1 : 0, p.scale);
    if (role == 1) {
        hipLaunchKernelGGL(naive_dkv_kernel, dim3((unsigned)rows), dim3(p.head_dim), 0, t.stream,
                           q, dout, prob, dp, delta, static_cast<float*>(t.dk),
                           static_cast<float*>(t.dv), p.seqlen, p.head_dim, p.causal ? 1 : 0,
                           p.scale);
    } else {
        hipLaunchKernelGGL(naive_dq_kernel, dim3((unsigned)rows), dim3(p.head_dim), 0, t.stream, k,
                           prob, dp, delta, static_cast<float*>(t.dq), p.seqlen, p.head_dim,
                           p.causal ? 1 : 0, p.scale);
    }
    return hipGetLastError();
}

}  // namespace fa3
