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
// tiles each) go, one per workgroup at most, before a workgroup's piece of
// the split job (kinds 1, 2, 3) or between kind 0's whole dKV job and its
// dQ remainder: longest first, each to the workgroup where the plan's latest
// finishing time grows least.  Each pair's head length minimises the later
// of its two finishing times.  The planner also runs the same greedy
// restricted to kinds 1 and 3 and keeps the shorter of the two plans.
struct SplitPlan {
    int head_kv[kMaxBalM], head_q[kMaxBalM];
    int shrt[4][kMaxBalM];  // [kind][x]: the short dQ tile that workgroup runs, or -1
    double makespan;        // modelled, in dKV steps
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
// dKV pair x (QT - x tiles), short jobs sh before the head piece (kind 2)
// and sr before the remainder (kind 1): the finishing time and the best
// head length
inline double kv_pair(int QT, int x, int sh, int sr, int* head) {
    double best_t = 1e30;
    *head = QT - x;
    for (int L = 1; L <= QT - x; ++L) {
        const int r = QT - x - L;
        const double c = start_after(sh) + kPro + (L - 1);
        const double t = r > 0 ? pair_end(c, start_after(sr) + kPro + (r - 1), kPubKv, kAddKv)
                               : std::max(c + kWholeKv, sr < 0 ? 0.0 : start_after(sr) - kGap);
        if (t < best_t) {
            best_t = t;
            *head = L;
        }
    }
    return best_t;
}
// dQ pair x (query tile M + x, M + x + 1 tiles), short job sh before the
// head piece (kind 3); kind 0 runs the whole dKV job of key tile M + x
// (M - x tiles), then short job sr, then the remainder
inline double q_pair(int M, int x, int sh, int sr, int* head) {
    double best_t = 1e30;
    *head = M + x + 1;
    double av = kEntry + kPro + (M - x - 1) + kWholeKv;
    if (sr >= 0) av += kGap + kPro + sr * kQ + kWholeQ;
    for (int L = 1; L <= M + x + 1; ++L) {
        const int r = M + x + 1 - L;
        const double d = start_after(sh) + kPro + (L - 1) * kQ;
        const double t = r > 0 ? pair_end(d, av + kGap + kPro + (r - 1) * kQ, kPubQ, kAddQ)
                               : std::max(d + kWholeQ, av);
        if (t < best_t) {
            best_t = t;
            *head = L;
        }
    }
    return best_t;
}
// pair p (dKV pairs 0 .. M - 1, then dQ pairs) with shorts on its head-piece
// and its remainder workgroup
inline double pair_time(int M, int p, int sh, int sr, int* head) {
    return p < M ? kv_pair(2 * M, p, sh, sr, head) : q_pair(M, p - M, sh, sr, head);
}
// Greedy placement of the short jobs (sides: 0 the head piece's workgroup,
// 1 the remainder's; all_sides false: kind 1 and kind 3 only)
inline void place_shorts(int M, bool all_sides, SplitPlan* plan) {
    const int P = 2 * M;
    std::vector<int> sh(P, -1), sr(P, -1);
    std::vector<double> cur(P);
    int h = 0;
    for (int p = 0; p < P; ++p) cur[p] = pair_time(M, p, -1, -1, &h);
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
        int best_p = -1, best_side = 0;
        double best_t = 1e30, best_pt = 0;
        for (int p = 0; p < P; ++p) {
            const double rest = p == i1 ? (i2 >= 0 ? cur[i2] : 0.0) : cur[i1];
            for (int side = 0; side < 2; ++side) {
                // kind 1 is the dKV remainder's side, kind 3 the dQ head's
                if (!all_sides && side != (p < M ? 1 : 0)) continue;
                if ((side == 0 ? sh[p] : sr[p]) >= 0) continue;
                const double pt = side == 0 ? pair_time(M, p, s, sr[p], &h) : pair_time(M, p, sh[p], s, &h);
                const double t = std::max(rest, pt);
                if (t < best_t) {
                    best_t = t;
                    best_pt = pt;
                    best_p = p;
                    best_side = side;
                }
            }
        }
        (best_side == 0 ? sh : sr)[best_p] = s;
        cur[best_p] = best_pt;
    }
    plan->makespan = 0;
    for (int x = 0; x < M; ++x) {
        plan->shrt[2][x] = sh[x];
        plan->shrt[1][x] = sr[x];
        plan->shrt[3][x] = sh[M + x];
        plan->shrt[0][x] = sr[M + x];
        plan->makespan = std::max(plan->makespan, kv_pair(2 * M, x, sh[x], sr[x], &plan->head_kv[x]));
        plan->makespan = std::max(plan->makespan, q_pair(M, x, sh[M + x], sr[M + x], &plan->head_q[x]));
    }
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
    auto two = std::make_unique<SplitPlan>();
    place_shorts(M, true, plan.get());
    place_shorts(M, false, two.get());
    cache[M] = two->makespan < plan->makespan ? std::move(two) : std::move(plan);
    return *cache[M];
}

}  // namespace fa3
