// Checks the main kernel's job map (set_job_map in
// flash-attention3_amd/csrc/fa3_job_map.h, job_of in fa3_bwd_main_kernel.h)
// on the host, over group counts 1..80 and group sizes of every plan (split
// plan 2 QT, default G = 1 2 QT, GQA QT (1 + G), head split QT (f + G)), with
// the groups one after another and interleaved:
//   * every id below n_groups x jobs_per_group runs exactly one (group,
//     position), and every (group, position) has an id;
//   * with XCD-aligned parts, every id of one (group, part) lands on one XCD
//     (id mod 8), and an XCD's parts are consecutive;
//   * interleaved, each XCD deals its parts' jobs in non-decreasing rank
//     within the part (position / parts: a part holds positions part,
//     part + parts, ..), and without parts the whole id sequence deals
//     non-decreasing positions, so the longest jobs of all groups come
//     first.
// Exit status 1 on any violation.  Built as HIP host code (no device pass).
#include <cstdio>
#include <vector>

#include "fa3_job_map.h"

int main() {
    int fails = 0;
    long long cases = 0;
    std::vector<int> jpgs;
    for (int qt : {2, 4, 6, 10, 16, 30, 32, 50, 64}) {
        jpgs.push_back(2 * qt);
        for (int g : {2, 3, 4, 8}) jpgs.push_back(qt * (1 + g));
        jpgs.push_back(qt * (2 + 8));
    }
    for (int ng = 1; ng <= 80; ++ng) {
        for (int jpg : jpgs) {
            for (int mode = 0; mode < 2; ++mode) {
                fa3::FusedArgs a{};
                a.n_groups = ng;
                a.jobs_per_group = jpg;
                // mode 1: few jobs per CU, so the map interleaves
                if (mode == 0) fa3::set_job_map(a);
                else fa3::set_job_map(a, 1.0, 1.0, 1 << 20);
                if (a.xcd_interleave != mode) {
                    std::printf("interleave flag %d, want %d (groups %d, jpg %d)\n",
                                a.xcd_interleave, mode, ng, jpg);
                    ++fails;
                    continue;
                }
                const int n = ng * jpg;
                std::vector<int> seen((size_t)n, -1), xcd_of_vg;
                const int parts = a.xcd_parts;
                if (parts > 0) xcd_of_vg.assign((size_t)ng * parts, -1);
                std::vector<int> last_rank(9, -1);
                const int fails_before = fails;
                for (int id = 0; id < n; ++id) {
                    int g = -1, pos = -1;
                    fa3::job_of(a, id, g, pos);
                    ++cases;
                    if (g < 0 || g >= ng || pos < 0 || pos >= jpg) {
                        std::printf("id %d -> (%d, %d) out of range (groups %d, jpg %d)\n", id, g,
                                    pos, ng, jpg);
                        ++fails;
                        break;
                    }
                    int& s = seen[(size_t)g * jpg + pos];
                    if (s >= 0) {
                        std::printf("(%d, %d) from ids %d and %d (groups %d, jpg %d)\n", g, pos, s,
                                    id, ng, jpg);
                        ++fails;
                        break;
                    }
                    s = id;
                    const int lane = parts > 0 ? id & 7 : 8;
                    if (parts > 0) {
                        const int vg = g * parts + pos % parts;
                        int& x = xcd_of_vg[(size_t)vg];
                        if (x < 0) x = id & 7;
                        if (x != (id & 7)) {
                            std::printf("part %d of group %d on XCDs %d and %d (groups %d, jpg %d)\n",
                                        pos % parts, g, x, id & 7, ng, jpg);
                            ++fails;
                            break;
                        }
                    }
                    if (mode == 1) {
                        const int rank = parts > 0 ? pos / parts : pos;
                        if (rank < last_rank[lane]) {
                            std::printf("rank %d after %d on lane %d (groups %d, jpg %d)\n",
                                        rank, last_rank[lane], lane, ng, jpg);
                            ++fails;
                            break;
                        }
                        last_rank[lane] = rank;
                    }
                }
                if (parts > 0 && fails == fails_before) {
                    // an XCD's parts are consecutive virtual groups
                    for (size_t v = 1; v < xcd_of_vg.size(); ++v) {
                        if (xcd_of_vg[v] < xcd_of_vg[v - 1]) {
                            std::printf("virtual group %zu on XCD %d after XCD %d (groups %d, jpg %d)\n",
                                        v, xcd_of_vg[v], xcd_of_vg[v - 1], ng, jpg);
                            ++fails;
                            break;
                        }
                    }
                }
                if (fails > 20) return 1;
            }
        }
    }
    std::printf("job map: %lld ids checked, %d failures\n", cases, fails);
    return fails == 0 ? 0 : 1;
}
