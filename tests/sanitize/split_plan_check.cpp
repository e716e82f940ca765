// CPU check of the split plan's planner (flash-attention3_amd/csrc/fa3_split_plan.h),
// built under ASan + UBSan: for every M the kernel can receive (2 .. 128),
//   * each short dQ job (query tiles 0 .. M - 1) is placed exactly once, on
//     one of the four workgroup kinds of a pair, before or after its piece
//     (after only below tile 127, which the descriptor could not tell from
//     "no short" in that position);
//   * every head length lies in 1 .. the job's tile count (the kernel's
//     descriptor holds it in 9 bits);
//   * the plan's recorded makespan is its modelled finishing time, and it
//     is no later than that of the fixed pairing the planner replaced (dKV
//     pair x runs short job x on its remainder's workgroup, dQ pairs none),
//     each pair at its best head length under the same model.
// Exit status 0 when all hold.
#include <cmath>
#include <cstdio>
#include <vector>

#include "fa3_split_plan.h"

int main() {
    using namespace fa3;
    int bad = 0;
    for (int M = 2; M <= kMaxBalM; ++M) {
        const SplitPlan& p = split_plan(M);
        const int QT = 2 * M;
        std::vector<int> seen(M, 0);
        double planned = 0, fixed = 0;
        int h = 0;
        using plan_model::Side;
        for (int x = 0; x < M; ++x) {
            for (int k = 0; k < 4; ++k) {
                const int s = p.shrt[k][x];
                if (s >= M || s < -1) ++bad;
                else if (s >= 0) ++seen[s];
                if (p.after[k][x] && (s < 0 || s >= 127)) ++bad;
            }
            const auto side = [&](int k) { return Side{p.shrt[k][x], p.after[k][x]}; };
            if (p.head_kv[x] < 1 || p.head_kv[x] > QT - x || p.head_kv[x] > 511) ++bad;
            if (p.head_q[x] < 1 || p.head_q[x] > M + x + 1 || p.head_q[x] > 511) ++bad;
            planned = std::max(planned, plan_model::kv_pair(QT, x, side(2), side(1), &h));
            if (h != p.head_kv[x]) ++bad;
            planned = std::max(planned, plan_model::q_pair(M, x, side(3), side(0), &h));
            if (h != p.head_q[x]) ++bad;
            fixed = std::max(fixed, plan_model::kv_pair(QT, x, Side{}, Side{x, false}, &h));
            fixed = std::max(fixed, plan_model::q_pair(M, x, Side{}, Side{}, &h));
        }
        for (int s = 0; s < M; ++s)
            if (seen[s] != 1) ++bad;
        if (std::fabs(planned - p.makespan) > 1e-9) ++bad;
        if (planned > fixed + 1e-9) ++bad;
        if (M == 8 || M == 16 || bad)
            std::printf("M=%d modelled %.2f (fixed pairing %.2f) problems so far %d\n", M, planned,
                        fixed, bad);
    }
    std::printf("%s\n", bad ? "FAIL" : "ok");
    return bad ? 1 : 0;
}
