// Line-oriented driver for the host-only capacity policy in
// vauss_amd/csrc/vs_capacity.h, used by tests/test_capacity_policy.py.
//   rec W H SLOT REQUIRED SPLATS LIMIT  -> "<changed 0|1> <hint at SPLATS or -1>"
//   hint W H SLOT SPLATS LIMIT          -> "<hint or -1>"
//   bucket RATIO                        -> "<bucket index>"
//   quantile Q R1 R2 ... Rn             -> "<upper edge of the bucket holding quantile Q>"
#include <cstdio>
#include <iostream>
#include <sstream>
#include <string>

#include "../vauss_amd/csrc/vs_capacity.h"

int main() {
    vs::CapacityTable table;
    std::string line;
    while (std::getline(std::cin, line)) {
        std::istringstream in(line);
        std::string op;
        if (!(in >> op)) continue;
        if (op == "rec") {
            uint32_t w, h, slot, splats;
            size_t req, limit;
            in >> w >> h >> slot >> req >> splats >> limit;
            const vs::CapacityKey k{w, h, slot};
            const bool changed = table.record(k, req, splats, limit);
            size_t out = 0;
            const bool have = table.hint(k, splats, limit, out);
            std::printf("%d %lld\n", changed ? 1 : 0, have ? (long long)out : -1LL);
        } else if (op == "hint") {
            uint32_t w, h, slot, splats;
            size_t limit;
            in >> w >> h >> slot >> splats >> limit;
            size_t out = 0;
            const bool have = table.hint(vs::CapacityKey{w, h, slot}, splats, limit, out);
            std::printf("%lld\n", have ? (long long)out : -1LL);
        } else if (op == "bucket") {
            double r;
            in >> r;
            std::printf("%d\n", vs::RatioHistogram::bucket(r));
        } else if (op == "quantile") {
            double q, r;
            in >> q;
            vs::RatioHistogram hist;
            while (in >> r) hist.push(r);
            std::printf("%.17g\n", hist.quantile(q));
        } else {
            std::printf("error\n");
        }
        std::fflush(stdout);
    }
    return 0;
}
