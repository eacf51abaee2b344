// Host-side check of the persistent launch schedule (q4k_launch.hpp): for
// every shape, each row group is assigned to exactly one (work-group, round),
// work-group b's first row group is b, and no work-group takes more rounds
// than the launch sizes its result buffer for. Built with hipcc and run by tests/test_native_sched.py; with no
// device visible, device_cus() reports 256.
#include "../../modgrad_amd/csrc/q4k_launch.hpp"

#include <cstdio>
#include <vector>

int main() {
    long checked = 0;
    for (long groups = 1; groups <= 12000; groups += (groups < 1200 ? 1 : 37)) {
        for (int occ = 1; occ <= 3; ++occ) {
            const mgq::PersistPlan p = mgq::persistent_plan(groups, occ);
            const int G = (int)p.grid;
            std::vector<int> hits(groups, 0);
            for (int b = 0; b < G; ++b) {
                // the GEMV issues its first stage before computing the
                // schedule, assuming work-group b's first row group is b
                if (mgq::sched_group(p.sch, b, G, 0) != b) {
                    std::printf("FAIL groups=%ld occ=%d b=%d first group %d\n", groups, occ, b,
                                mgq::sched_group(p.sch, b, G, 0));
                    return 1;
                }
                const int c = mgq::sched_count(p.sch, b, G, (int)groups);
                if (c > p.rounds || c < 1) {
                    std::printf("FAIL groups=%ld occ=%d b=%d count=%d rounds=%ld\n", groups, occ, b,
                                c, p.rounds);
                    return 1;
                }
                for (int j = 0; j < c; ++j) {
                    const int g = mgq::sched_group(p.sch, b, G, j);
                    if (g < 0 || g >= groups) {
                        std::printf("FAIL groups=%ld occ=%d b=%d j=%d group=%d\n", groups, occ, b,
                                    j, g);
                        return 1;
                    }
                    ++hits[g];
                }
            }
            for (long g = 0; g < groups; ++g)
                if (hits[g] != 1) {
                    std::printf("FAIL groups=%ld occ=%d group %ld hit %d times\n", groups, occ, g,
                                hits[g]);
                    return 1;
                }
            ++checked;
        }
    }
    std::printf("ok %ld schedules\n", checked);
    return 0;
}
