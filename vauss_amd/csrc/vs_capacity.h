// vs_capacity.h -- host-side intersection capacity hints for lagged training
// renders (no device code).
//
// Restates the policy of crates/splat-train-render/src/render.rs:38-223: one
// hint per (image size, count slot); a window of 200 renders ends by sizing
// the hint to the window's p99 intersections per splat (log-spaced histogram,
// 8 buckets per octave) with 25 % headroom, never below the window's largest
// render plus 5 %; before the first full window the hint grows at once to
// 1.5x a requirement within 30 % of it, after it only on an overflow, to just
// cover it.  A hint measured at S splats scales linearly to N >= S splats.
#pragma once
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <map>
#include <tuple>

namespace vs {

constexpr uint32_t CAPACITY_WINDOW = 200;
constexpr double CAPACITY_QUANTILE = 0.99;
constexpr double QUANTILE_HEADROOM = 1.25;
constexpr int RATIO_BUCKETS = 160;

// Intersections per splat, 8 buckets per octave from 2^-10 to 2^10.
struct RatioHistogram {
    uint32_t n[RATIO_BUCKETS] = {};
    static int bucket(double ratio) {
        const double b = std::floor(std::log2(std::max(ratio, 1e-9)) * 8.0) + 80.0;
        return (int)std::min<double>(std::max<double>(b, 0.0), RATIO_BUCKETS - 1);
    }
    void push(double ratio) { ++n[bucket(ratio)]; }
    // Upper edge of the bucket holding quantile q.
    double quantile(double q) const {
        uint64_t total = 0;
        for (uint32_t c : n) total += c;
        const uint64_t rank = (uint64_t)std::max(1.0, std::ceil((double)total * q));
        uint64_t seen = 0;
        for (int i = 0; i < RATIO_BUCKETS; ++i) {
            seen += n[i];
            if (seen >= rank) return std::pow(2.0, (i - 80.0 + 1.0) / 8.0);
        }
        return std::pow(2.0, (RATIO_BUCKETS - 80.0) / 8.0);
    }
};

inline size_t div_ceil(size_t a, size_t b) { return a / b + (a % b != 0); }
// A capacity covering a seen requirement, with 5 % for growth between windows.
inline size_t covering_max(size_t required, size_t limit) {
    return std::max<size_t>(std::min(required + div_ceil(required, 20), limit), 1);
}
inline size_t capacity_with_headroom(size_t required, size_t limit) {
    return std::max<size_t>(std::min(required + div_ceil(required, 2), limit), 1);
}

struct Capacity {
    size_t isects = 0;
    uint32_t splats = 0;            // the splat count the hint was measured at
    uint32_t window_len = 0;
    size_t window_max = 0;
    uint64_t window_sum = 0;
    uint32_t window_over = 0;
    RatioHistogram ratios;
    bool settled = false;
    size_t for_splats(uint32_t total_splats, size_t limit) const {
        const unsigned __int128 grown = (unsigned __int128)isects * std::max(total_splats, splats) /
                                        std::max<uint32_t>(splats, 1u);
        return std::max<size_t>((size_t)std::min<unsigned __int128>(grown, limit), 1);
    }
};

using CapacityKey = std::tuple<uint32_t, uint32_t, uint32_t>;   // image width, height, count slot

class CapacityTable {
public:
    // The hint for `total_splats`, or false when nothing was recorded at this key.
    bool hint(const CapacityKey& k, uint32_t total_splats, size_t limit, size_t& out) const {
        auto it = table_.find(k);
        if (it == table_.end()) return false;
        out = it->second.for_splats(total_splats, limit);
        return true;
    }
    // record_capacity (render.rs:118-191).  Returns true when the hint changed.
    bool record(const CapacityKey& k, size_t required, uint32_t splats, size_t limit) {
        if (table_.size() >= 32 && table_.find(k) == table_.end()) table_.clear();
        const size_t desired = capacity_with_headroom(required, limit);
        auto it = table_.find(k);
        if (it == table_.end()) {
            Capacity c;
            c.isects = desired;
            c.splats = splats;
            it = table_.emplace(k, c).first;
        }
        Capacity& e = it->second;
        bool changed = false;
        const size_t current = e.for_splats(splats, limit);
        e.window_len += 1;
        e.window_max = std::max(e.window_max, required);
        e.window_sum += required;
        e.ratios.push((double)required / (double)std::max<uint32_t>(splats, 1u));
        if (required > current) e.window_over += 1;
        size_t grow_to = 0;
        if (!e.settled) {
            if (required + div_ceil(required, 10) * 3 > current) grow_to = desired;
        } else if (required > current) {
            grow_to = covering_max(required, limit);
        }
        if (grow_to) {
            e.isects = std::max(grow_to, current);
            e.splats = splats;
            changed = true;
        }
        if (e.window_len >= CAPACITY_WINDOW) {
            const double ratio = e.ratios.quantile(CAPACITY_QUANTILE) * QUANTILE_HEADROOM;
            const size_t by_ratio = (size_t)std::ceil((double)splats * ratio);
            const size_t target = std::min(std::max<size_t>(std::max(by_ratio, covering_max(e.window_max, limit)), 1), limit);
            const size_t cur = e.for_splats(splats, limit);
            if (target > cur || target < cur - cur / 4) {
                e.isects = target;
                e.splats = splats;
                changed = true;
            }
            e.window_len = 0;
            e.window_max = 0;
            e.window_sum = 0;
            e.window_over = 0;
            e.ratios = RatioHistogram{};
            e.settled = true;
        }
        return changed;
    }
    const Capacity* find(const CapacityKey& k) const {
        auto it = table_.find(k);
        return it == table_.end() ? nullptr : &it->second;
    }

private:
    std::map<CapacityKey, Capacity> table_;
};

} // namespace vs
