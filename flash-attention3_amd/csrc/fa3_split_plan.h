// Host-side planner of the main kernel's split plan (plain C++, no HIP):
// included by fa3_bwd_main.hip, and by tests/sanitize/split_plan_check.cpp,
// which checks its invariants on the CPU.
#pragma once

#include <algorithm>
#include <memory>
#include <mutex>
#include <vector>

namespace fa3 {

constexpr int kMaxBalM = 128;  // split plan: at most 512 jobs, so M = QT / 2 <= 128

// The split plan's head-piece lengths and short-job places.  Workgroup
// times in units of one dKV step, measured on MI355X at B1 H4 S2048 D128
// (per-workgroup timestamps): a dQ step costs 0.73, a unit's prologue (loads
// + first score phase) 2.5, its epilogue 2.0 (dKV) / 0.8 (dQ) for a whole
// job; of a split job, the piece that arrives first spends kPub (storing its
// partial sums) and the second, after waiting for them, kAdd (adding them
// and writing the output); 0.65 at kernel entry and between two units.
// Pairs of workgroups share a split job: dKV pair x (kinds 2 and 1) and dQ
// pair x (kinds 3 and 0).  The short dQ jobs (query tiles s < M, s + 1
// tiles each) go first on the kind-1 workgroup of a dKV pair or on the
// kind-3 workgroup of a dQ pair, one per pair at most: longest first, each
// to the pair where the plan's latest finishing time grows least.  Each
// pair's head length minimises the later of its two finishing times.
struct SplitPlan {
    int head_kv[kMaxBalM], head_q[kMaxBalM];
    int short_kv[kMaxBalM], short_q[kMaxBalM];  // short dQ tile or -1
};

namespace plan_model {
constexpr double kQ = 0.73, kPro = 2.5, kEntry = 0.65, kGap = 0.65;
constexpr double kWholeKv = 2.0, kWholeQ = 0.8;
constexpr double kPubKv = 2.6, kAddKv = 2.8, kPubQ = 1.6, kAddQ = 1.8;
// a, b: the two workgroups' times up to the end of their last steps
inline double pair_end(double a, double b, double pub, double add) {
    const double first = a < b ? a : b, second = a < b ? b : a;
    return (second > first + pub ? second : first + pub) + add;
}
// time before a workgroup's split piece starts: kernel entry, or a whole
// short dQ job of s + 1 tiles and the gap after it
inline double start_after(int s) { return s < 0 ? kEntry : kEntry + kPro + s * kQ + kWholeQ + kGap; }
// dKV pair x (QT - x tiles), short job s on the remainder's workgroup:
// the finishing time and the best head length
inline double kv_pair(int QT, int x, int s, int* head) {
    double best_t = 1e30;
    *head = QT - x;
    for (int L = 1; L <= QT - x; ++L) {
        const int r = QT - x - L;
        const double c = kEntry + kPro + (L - 1);
        const double t = r > 0 ? pair_end(c, start_after(s) + kPro + (r - 1), kPubKv, kAddKv)
                               : std::max(c + kWholeKv, s < 0 ? 0.0 : start_after(s) - kGap);
        if (t < best_t) {
            best_t = t;
            *head = L;
        }
    }
    return best_t;
}
// dQ pair x (query tile M + x, M + x + 1 tiles), short job s on the head
// piece's workgroup; the remainder follows the whole dKV job of key tile
// M + x (M - x tiles)
inline double q_pair(int M, int x, int s, int* head) {
    double best_t = 1e30;
    *head = M + x + 1;
    const double av = kEntry + kPro + (M - x - 1) + kWholeKv;
    for (int L = 1; L <= M + x + 1; ++L) {
        const int r = M + x + 1 - L;
        const double d = start_after(s) + kPro + (L - 1) * kQ;
        const double t = r > 0 ? pair_end(d, av + kGap + kPro + (r - 1) * kQ, kPubQ, kAddQ)
                               : std::max(d + kWholeQ, av);
        if (t < best_t) {
            best_t = t;
            *head = L;
        }
    }
    return best_t;
}
}  // namespace plan_model

// Plans are cached per M (the plan depends on M alone).
inline const SplitPlan& split_plan(int M) {
    using namespace plan_model;
    static std::mutex mu;
    static std::unique_ptr<SplitPlan> cache[kMaxBalM + 1];
    std::lock_guard<std::mutex> lock(mu);
    if (cache[M]) return *cache[M];
    auto plan = std::make_unique<SplitPlan>();
    const int QT = 2 * M, P = 2 * M;  // pairs: dKV 0 .. M - 1, then dQ M .. 2M - 1
    // end[p][s + 1]: pair p's finishing time with short job s (-1: none)
    std::vector<double> end((size_t)P * (M + 1));
    int h = 0;
    for (int p = 0; p < P; ++p)
        for (int s = -1; s < M; ++s)
            end[(size_t)p * (M + 1) + s + 1] = p < M ? kv_pair(QT, p, s, &h) : q_pair(M, p - M, s, &h);
    std::vector<int> shrt(P, -1);
    std::vector<double> cur(P);
    for (int p = 0; p < P; ++p) cur[p] = end[(size_t)p * (M + 1)];
    for (int s = M - 1; s >= 0; --s) {
        // the plan's latest time without pair p: the largest or the second largest
        int i1 = -1, i2 = -1;
        for (int p = 0; p < P; ++p) {
            if (i1 < 0 || cur[p] > cur[i1]) {
                i2 = i1;
                i1 = p;
            } else if (i2 < 0 || cur[p] > cur[i2]) {
                i2 = p;
            }
        }
        int best_p = -1;
        double best_t = 1e30;
        for (int p = 0; p < P; ++p) {
            if (shrt[p] >= 0) continue;
            const double rest = p == i1 ? (i2 >= 0 ? cur[i2] : 0.0) : cur[i1];
            const double t = std::max(rest, end[(size_t)p * (M + 1) + s + 1]);
            if (t < best_t) {
                best_t = t;
                best_p = p;
            }
        }
        shrt[best_p] = s;
        cur[best_p] = end[(size_t)best_p * (M + 1) + s + 1];
    }
    for (int x = 0; x < M; ++x) {
        plan->short_kv[x] = shrt[x];
        plan->short_q[x] = shrt[M + x];
        kv_pair(QT, x, shrt[x], &plan->head_kv[x]);
        q_pair(M, x, shrt[M + x], &plan->head_q[x]);
    }
    cache[M] = std::move(plan);
    return *cache[M];
}

}  // namespace fa3
