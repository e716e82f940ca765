// The CPU oracle (oracle/fa3_bwd_oracle.cpp) on small shapes under the
// sanitizers (built by tests/sanitize/Makefile): MHA and GQA, causal and not,
// fp16 and bf16, uneven row blocks, several threads -- ASan / UBSan for
// memory errors and undefined behaviour, TSan for data races between the
// worker threads.  Results are checked for finiteness only; their values
// are pinned by the oracle's own tests.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

extern "C" {
void fa3o_randn_fmt(uint16_t* out, size_t n, uint64_t seed, int fmt);
void fa3o_forward_fmt(const uint16_t* q16, const uint16_t* k16, const uint16_t* v16, int B,
                      int Hq, int Hkv, int S, int D, int causal, float scale, int bkv_begin,
                      int bkv_end, uint16_t* out16, float* smax, float* ssum, float* lse,
                      int threads, int fmt);
void fa3o_backward_fmt(const uint16_t* q16, const uint16_t* k16, const uint16_t* v16,
                       const uint16_t* out16, const uint16_t* dout16, const float* smax,
                       const float* ssum, int B, int Hq, int Hkv, int S, int D, int causal,
                       float scale, int bkv_begin, int bkv_end, float* delta, float* dq,
                       float* dk, float* dv, int threads, int fmt);
}

int main() {
    struct Case { int B, Hq, Hkv, S, D, causal, fmt, threads; };
    const Case cases[] = {{1, 1, 1, 64, 32, 1, 0, 4}, {2, 4, 2, 100, 16, 0, 0, 8},
                          {1, 2, 1, 70, 64, 1, 1, 3}, {1, 3, 3, 33, 8, 0, 1, 16}};
    int bad = 0;
    for (const Case& c : cases) {
        const size_t qn = (size_t)c.B * c.Hq * c.S * c.D, kn = (size_t)c.B * c.Hkv * c.S * c.D;
        const size_t rows = (size_t)c.B * c.Hq * c.S;
        std::vector<uint16_t> q(qn), k(kn), v(kn), dout(qn), out(qn);
        fa3o_randn_fmt(q.data(), qn, 1, c.fmt);
        fa3o_randn_fmt(k.data(), kn, 2, c.fmt);
        fa3o_randn_fmt(v.data(), kn, 3, c.fmt);
        fa3o_randn_fmt(dout.data(), qn, 4, c.fmt);
        std::vector<float> smax(rows), ssum(rows), lse(rows), delta(rows), dq(qn), dk(kn), dv(kn);
        const float scale = 1.f / std::sqrt((float)c.D);
        fa3o_forward_fmt(q.data(), k.data(), v.data(), c.B, c.Hq, c.Hkv, c.S, c.D, c.causal,
                         scale, 0, c.B * c.Hkv, out.data(), smax.data(), ssum.data(), lse.data(),
                         c.threads, c.fmt);
        fa3o_backward_fmt(q.data(), k.data(), v.data(), out.data(), dout.data(), smax.data(),
                          ssum.data(), c.B, c.Hq, c.Hkv, c.S, c.D, c.causal, scale, 0,
                          c.B * c.Hkv, delta.data(), dq.data(), dk.data(), dv.data(), c.threads,
                          c.fmt);
        for (float x : dq) bad += !std::isfinite(x);
        for (float x : dk) bad += !std::isfinite(x);
        for (float x : dv) bad += !std::isfinite(x);
        for (float x : delta) bad += !std::isfinite(x);
    }
    std::printf("oracle_run: %d non-finite values\n", bad);
    return bad == 0 ? 0 : 1;
}
