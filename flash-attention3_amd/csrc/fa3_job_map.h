// XCD-aware job map of the main kernel's default plan and of the split
// plan's descriptors: which (group, position) each workgroup id runs (job_of
// in fa3_bwd_main_kernel.h reads the fields set here).  Host code.
#pragma once

#include "fa3_bwd_main_kernel.h"

namespace fa3 {

// An XCD runs its K virtual groups one after another, or position by
// position across them (longest jobs of all of them first).  Run one after
// another, the last group's longest job starts when about share / K of a
// CU's share of the work is left, and may set the kernel's end; one group at
// a time keeps the XCD's L2 on fewer heads.  The map interleaves with at
// most kInterleaveJobsPerCu jobs per CU, or when the longest job is at least
// kInterleaveTail x share / K (all in dKV steps) and the XCD's virtual
// groups belong to at most kInterleaveSpan groups.  Measured: B1 H9 S2048
// D128 causal -20.7 % (2.25 jobs per CU), B1 Hq28 Hkv7 S4096 -20.2 % (8.75,
// longest 256 against share / K 57), B1 H19 S4096 -4.3 % (9.5; 64 against
// 14; 3 groups per XCD); interleaving P4 (20 per CU; 256 against 455) left
// its time unchanged and raised its L2 misses 1.9x, B1 H36 S4096 (18; 64
// against 57) +6.9 %, B2 H24 S2048 D64 (12; 32 against 29) +1.3 %, P5 (32;
// 128 against 896) +6.5 %, B8 H16 S1024 D128 (16; 16 against 7.4, but 16
// groups per XCD) +20 %, B4 H32 S1024 +20 %.
inline constexpr int kInterleaveJobsPerCu = 8;
inline constexpr double kInterleaveTail = 2.0;
inline constexpr int kInterleaveSpan = 4;

// XCD-aware job map: n_groups groups of jobs_per_group jobs.  longest:
// the longest job, share: a CU's share of the work (both in dKV steps),
// cus: the CU count -- for the interleave choice above (the defaults: one
// group after another).
inline void set_job_map(FusedArgs& a, double longest = 0.0, double share = 1.0, int cus = 0) {
    int gcd8 = 8;
    while (a.n_groups % gcd8 != 0) gcd8 >>= 1;
    const int parts = 8 / gcd8;  // smallest split with n_groups * parts % 8 == 0
    const bool fits = a.jobs_per_group % parts == 0;
    a.xcd_parts = fits ? parts : 0;
    a.xcd_vgroups = fits ? a.n_groups * parts / 8 : 0;
    const long long jobs = (long long)a.n_groups * a.jobs_per_group;
    // the groups an XCD's virtual groups belong to (one more where its
    // first part is not a group's first)
    const int span = fits ? (a.xcd_vgroups + parts - 1) / parts : a.n_groups;
    const bool interleave =
        jobs <= (long long)kInterleaveJobsPerCu * cus ||
        (span <= kInterleaveSpan && longest * a.xcd_vgroups >= kInterleaveTail * share);
    a.xcd_interleave = interleave ? 1 : 0;
    a.xcd_mode = a.xcd_parts | a.xcd_interleave << 8;
    a.map_radix = !fits ? 0 : interleave ? a.xcd_vgroups : a.jobs_per_group / parts;
    a.div_parts = make_fastdiv(a.xcd_parts);
    a.div_radix = make_fastdiv(a.map_radix);
    a.div_jpg = make_fastdiv(a.jobs_per_group);
    a.div_groups = make_fastdiv(a.n_groups);
}

}  // namespace fa3
