// Checks the stream-device rule of the stream-taking entries
// (fa3::launch_device_of in flash-attention3_amd/csrc/fa3_bwd_internal.h),
// under UBSan: the null stream and a stream of the current device launch on
// the current device; a stream of any other device is refused (-1), for
// every pair of device ordinals 0..15.  This branch needs two GPUs to reach
// through the C ABI, so it is checked here.  Exit status 1 on any mismatch.
#include <cstdio>

#include "fa3_bwd_internal.h"

int main() {
    int bad = 0;
    for (int cur = 0; cur < 16; ++cur) {
        if (fa3::launch_device_of(cur, false, -1) != cur) ++bad;
        for (int sd = 0; sd < 16; ++sd) {
            const int want = sd == cur ? cur : -1;
            if (fa3::launch_device_of(cur, true, sd) != want) {
                std::printf("current %d stream device %d -> %d (want %d)\n", cur, sd,
                            fa3::launch_device_of(cur, true, sd), want);
                ++bad;
            }
        }
    }
    std::printf("%s\n", bad ? "FAIL" : "ok");
    return bad ? 1 : 0;
}
