// Host-side planner of the main kernel's split plan (plain C++, no HIP):
// included by fa3_bwd_main.hip, and by tests/sanitize/split_plan_check.cpp,
// which checks its invariants on the CPU.
#pragma once

#include <algorithm>
#include <memory>
#include <mutex>
#include <vector>

namespace fa3 {

constexpr int kMaxBalM = 128;  // M = QT / 2 of a split plan (at most 256 jobs: M <= 64)

// The split plan's head-piece lengths and short-job places.  Workgroup
// times in units of one dKV step, measured on MI355X at B1 H4 S2048 D128
// (per-workgroup timestamps): a dQ step costs 0.73, a unit's prologue (loads
// + first score phase) 2.5, its epilogue 2.0 (dKV) / 0.8 (dQ) for a whole
// job; of a split job, the piece that arrives first spends kPub (storing its
// partial sums) and the second, after waiting for them, kAdd (adding them
// and writing the output); 0.65 at kernel entry and between two units.
// Pairs of workgroups share a split job: dKV pair x (kinds 2 and 1) and dQ
// pair x (kinds 3 and 0).  The short dQ jobs (query tiles s < M, s + 1
// tiles each) go, one per workgroup at most, before or after a workgroup's
// piece of the split job (kinds 1, 2, 3), or after kind 0's whole dKV job
// (before its dQ remainder) or at its end.  A short job after a piece
// fills the time the piece that publishes first would otherwise spend
// idle while its partner adds the partial sums.  Placement is greedy,
// longest first, each to the workgroup and position where the plan's
// latest finishing time grows least.  Each pair's head length minimises
// the later of its two finishing times.  The planner runs the greedy with
// and without the kinds 0 and 2 and with and without the positions after a
// piece, and keeps the first plan of the shortest makespan (the positions
// after a piece only when they shorten it).
struct SplitPlan {
    int head_kv[kMaxBalM], head_q[kMaxBalM];
    int shrt[4][kMaxBalM];    // [kind][x]: the short dQ tile that workgroup runs, or -1
    bool after[4][kMaxBalM];  // ... after its piece (else before it)
    double makespan;          // modelled, in dKV steps
};

namespace plan_model {
constexpr double kQ = 0.73, kPro = 2.5, kEntry = 0.65, kGap = 0.65;
constexpr double kWholeKv = 2.0, kWholeQ = 0.8;
constexpr double kPubKv = 2.6, kAddKv = 2.8, kPubQ = 1.6, kAddQ = 1.8;
// a workgroup's short job: its query tile s (-1: none) and its position
struct Side {
    int s = -1;
    bool after = false;
};
// a whole short dQ job of s + 1 tiles after the gap that precedes it
inline double short_time(int s) { return kGap + kPro + s * kQ + kWholeQ; }
// time before a workgroup's piece starts: kernel entry, and a short job run
// before the piece with the gap after it
inline double start_of(Side sd) {
    return sd.s >= 0 && !sd.after ? kEntry + kPro + sd.s * kQ + kWholeQ + kGap : kEntry;
}
// time a short job run after the piece adds
inline double tail_of(Side sd) { return sd.s >= 0 && sd.after ? short_time(sd.s) : 0.0; }
// the two workgroups' finishing times when their split pieces' last steps
// end at a (head) and b (remainder): the one that ends first publishes,
// the other waits for it and adds
inline double pair_finish(double a, double b, double pub, double add, Side ha, Side hb) {
    const double first = a < b ? a : b, second = a < b ? b : a;
    const double fe = first + pub, se = (second > fe ? second : fe) + add;
    const double ea = a < b ? fe : se, eb = a < b ? se : fe;
    return std::max(ea + tail_of(ha), eb + tail_of(hb));
}
// dKV pair x (QT - x tiles): the head piece on kind 2 (its short h), the
// remainder on kind 1 (short r); the later finishing time and the best head
// length
inline double kv_pair(int QT, int x, Side h, Side r, int* head) {
    double best_t = 1e30;
    *head = QT - x;
    for (int L = 1; L <= QT - x; ++L) {
        const int rr = QT - x - L;
        const double c = start_of(h) + kPro + (L - 1);
        // unsplit: kind 1 runs its short job alone, if it has one
        const double t =
            rr > 0 ? pair_finish(c, start_of(r) + kPro + (rr - 1), kPubKv, kAddKv, h, r)
                   : std::max(c + kWholeKv + tail_of(h),
                              r.s < 0 ? 0.0 : kEntry + kPro + r.s * kQ + kWholeQ);
        if (t < best_t) {
            best_t = t;
            *head = L;
        }
    }
    return best_t;
}
// dQ pair x (query tile M + x, M + x + 1 tiles): the head piece on kind 3
// (short h); kind 0 runs the whole dKV job of key tile M + x (M - x tiles),
// then its short r if placed before, then the remainder, then r if after
inline double q_pair(int M, int x, Side h, Side r, int* head) {
    double best_t = 1e30;
    *head = M + x + 1;
    double av = kEntry + kPro + (M - x - 1) + kWholeKv;
    if (r.s >= 0 && !r.after) av += short_time(r.s);
    for (int L = 1; L <= M + x + 1; ++L) {
        const int rr = M + x + 1 - L;
        const double d = start_of(h) + kPro + (L - 1) * kQ;
        const double t =
            rr > 0 ? pair_finish(d, av + kGap + kPro + (rr - 1) * kQ, kPubQ, kAddQ, h, r)
                   : std::max(d + kWholeQ + tail_of(h), av + tail_of(r));
        if (t < best_t) {
            best_t = t;
            *head = L;
        }
    }
    return best_t;
}
// pair p (dKV pairs 0 .. M - 1, then dQ pairs) with shorts on its head-piece
// and its remainder workgroup
inline double pair_time(int M, int p, Side h, Side r, int* head) {
    return p < M ? kv_pair(2 * M, p, h, r, head) : q_pair(M, p - M, h, r, head);
}
// Greedy placement of the short jobs (sides: 0 the head piece's workgroup,
// 1 the remainder's; all_sides false: kind 1 and kind 3 only; allow_after:
// also after the piece -- not for s = 127, which the descriptor could not
// tell from "no short" in that position)
inline void place_shorts(int M, bool all_sides, bool allow_after, SplitPlan* plan) {
    const int P = 2 * M;
    std::vector<Side> sh(P), sr(P);
    std::vector<double> cur(P);
    int h = 0;
    for (int p = 0; p < P; ++p) cur[p] = pair_time(M, p, sh[p], sr[p], &h);
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
        bool best_after = false;
        double best_t = 1e30, best_pt = 0;
        for (int p = 0; p < P; ++p) {
            const double rest = p == i1 ? (i2 >= 0 ? cur[i2] : 0.0) : cur[i1];
            for (int side = 0; side < 2; ++side) {
                // kind 1 is the dKV remainder's side, kind 3 the dQ head's
                if (!all_sides && side != (p < M ? 1 : 0)) continue;
                if ((side == 0 ? sh[p] : sr[p]).s >= 0) continue;
                for (int af = 0; af < (allow_after && s < 127 ? 2 : 1); ++af) {
                    Side hs = sh[p], rs = sr[p];
                    (side == 0 ? hs : rs) = Side{s, af != 0};
                    const double pt = pair_time(M, p, hs, rs, &h);
                    const double t = std::max(rest, pt);
                    if (t < best_t) {
                        best_t = t;
                        best_pt = pt;
                        best_p = p;
                        best_side = side;
                        best_after = af != 0;
                    }
                }
            }
        }
        (best_side == 0 ? sh : sr)[best_p] = Side{s, best_after};
        cur[best_p] = best_pt;
    }
    plan->makespan = 0;
    for (int x = 0; x < M; ++x) {
        const Side sides[4] = {sr[M + x], sr[x], sh[x], sh[M + x]};  // kinds 0 .. 3
        for (int k = 0; k < 4; ++k) {
            plan->shrt[k][x] = sides[k].s;
            plan->after[k][x] = sides[k].s >= 0 && sides[k].after;
        }
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
    std::unique_ptr<SplitPlan> best;
    for (int v = 0; v < 4; ++v) {
        auto plan = std::make_unique<SplitPlan>();
        place_shorts(M, (v & 1) == 0, v >= 2, plan.get());
        if (!best || plan->makespan < best->makespan - 1e-9) best = std::move(plan);
    }
    cache[M] = std::move(best);
    return *cache[M];
}

}  // namespace fa3
