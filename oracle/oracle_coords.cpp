// oracle_coords.cpp -- TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// downsample_coords restated from the reference (session.cpp:168-233).  This
// file is compiled with -ffp-contract=off: the reference's build of
// session.cpp uses no FMA instructions (GGML_NATIVE OFF, no -march), so its
// double arithmetic rounds after every operation, and so does this.

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <random>
#include <set>
#include <vector>

namespace {

// session.cpp:122-127, each field zero-extended, aliasing included.
uint64_t cell_key(int32_t b, int32_t x, int32_t y, int32_t z) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(b)) << 48) |
           (static_cast<uint64_t>(static_cast<uint32_t>(x)) << 32) |
           (static_cast<uint64_t>(static_cast<uint32_t>(y)) << 16) |
           static_cast<uint64_t>(static_cast<uint32_t>(z) & 0xffffu);
}

}  // namespace

int64_t orc_downsample_coords(const int32_t *coords, int64_t n, int64_t max_coords, int32_t factor,
                              uint32_t seed, int32_t *out) {
    // session.cpp:173-174: small sets are returned as they are.
    if (n <= max_coords) {
        std::copy(coords, coords + n * 4, out);
        return n;
    }
    // :176-184 bounding box of (x, y, z).
    int32_t lo[3], hi[3];
    for (int a = 0; a < 3; ++a) lo[a] = hi[a] = coords[1 + a];
    for (int64_t i = 1; i < n; ++i)
        for (int a = 0; a < 3; ++a) {
            lo[a] = std::min(lo[a], coords[i * 4 + 1 + a]);
            hi[a] = std::max(hi[a], coords[i * 4 + 1 + a]);
        }
    // :185-195 the centred target range per axis.
    double target[3], tmin[3];
    int32_t tmin_i[3], tmax_i[3];
    for (int a = 0; a < 3; ++a) {
        const double original = static_cast<double>(hi[a] - lo[a] + 1);
        target[a] = original / static_cast<double>(factor);
        const double offset = (original - target[a]) * 0.5;
        tmin[a] = static_cast<double>(lo[a]) + offset;
        const double tmax = tmin[a] + target[a] - 1.0;
        tmin_i[a] = static_cast<int32_t>(tmin[a]);
        tmax_i[a] = static_cast<int32_t>(tmax);
    }
    // :197-216 map, round half up, clamp; keep first occurrences.
    std::vector<int32_t> unique;
    std::set<uint64_t> seen;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t *p = coords + i * 4;
        int32_t m[4] = {p[0], 0, 0, 0};
        for (int a = 0; a < 3; ++a) {
            const double denom = static_cast<double>(hi[a] - lo[a]);
            const double normalized = denom > 0.0 ? (static_cast<double>(p[a + 1]) - lo[a]) / denom : 0.0;
            const double value = normalized * (target[a] - 1.0) + tmin[a];
            int64_t r = static_cast<int64_t>(std::floor(value + 0.5));
            r = std::max<int64_t>(r, tmin_i[a]);
            r = std::min<int64_t>(r, tmax_i[a]);
            m[a + 1] = static_cast<int32_t>(r);
        }
        if (seen.insert(cell_key(m[0], m[1], m[2], m[3])).second) unique.insert(unique.end(), m, m + 4);
    }
    const int64_t un = static_cast<int64_t>(unique.size() / 4);
    if (un <= max_coords) {
        std::copy(unique.begin(), unique.end(), out);
        return un;
    }
    // :217-229 the sample: the first max_coords of a std::shuffle under
    // std::mt19937(seed).
    std::mt19937 rng(seed);
    std::vector<size_t> order(static_cast<size_t>(un));
    std::iota(order.begin(), order.end(), size_t(0));
    std::shuffle(order.begin(), order.end(), rng);
    for (int64_t j = 0; j < max_coords; ++j)
        std::copy(unique.begin() + static_cast<ptrdiff_t>(order[static_cast<size_t>(j)] * 4),
                  unique.begin() + static_cast<ptrdiff_t>(order[static_cast<size_t>(j)] * 4 + 4), out + j * 4);
    return max_coords;
}

uint32_t orc_mt19937_draw(uint32_t seed, int64_t k) {
    // The k-th output (1-based) of std::mt19937(seed), to pin the generator.
    std::mt19937 rng(seed);
    uint32_t v = 0;
    for (int64_t i = 0; i < k; ++i) v = static_cast<uint32_t>(rng());
    return v;
}
