// oracle.cpp -- TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// A plain C++ restatement of the reference's CPU algorithms for the sparse
// voxel path.  It is the checker for the HIP library and the timed CPU
// baseline; it is never linked into, loaded by or called from the product.
// Every function cites the reference lines it restates.

#include "oracle.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <map>
#include <set>
#include <thread>
#include <tuple>
#include <vector>

namespace {

using Key4 = std::tuple<int32_t, int32_t, int32_t, int32_t>;  // (b, x, y, z)

inline void offset_delta(int o, int *dx, int *dy, int *dz) {
    // sparse_ops.cpp:132 -- o = (dx+1)*9 + (dy+1)*3 + (dz+1)
    *dx = o / 9 - 1;
    *dy = (o / 3) % 3 - 1;
    *dz = o % 3 - 1;
}

inline bool add_fits(int32_t v, int d, int32_t *out) {
    const int64_t s = static_cast<int64_t>(v) + d;
    if (s < INT32_MIN || s > INT32_MAX) return false;
    *out = static_cast<int32_t>(s);
    return true;
}

template <class F>
void parallel_rows(int64_t n, int threads, F &&fn) {
    if (threads <= 1 || n < 64) {
        fn(int64_t(0), n);
        return;
    }
    std::vector<std::thread> pool;
    const int64_t chunk = (n + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        const int64_t lo = t * chunk, hi = std::min<int64_t>(n, lo + chunk);
        if (lo >= hi) break;
        pool.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto &th : pool) th.join();
}

int default_threads() {
    const unsigned h = std::thread::hardware_concurrency();
    return h == 0 ? 1 : static_cast<int>(std::min(h, 16u));
}

// Build the ordered (b,x,y,z) -> first-row index.  std::map::emplace keeps
// the first occurrence, as sparse_ops.cpp:119-124 does.
std::map<Key4, int32_t> ordered_index(const int32_t *coords, int64_t n) {
    std::map<Key4, int32_t> idx;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t *c = coords + i * 4;
        idx.emplace(Key4{c[0], c[1], c[2], c[3]}, static_cast<int32_t>(i));
    }
    return idx;
}

void fill_kmap(const std::map<Key4, int32_t> &idx, int64_t n, int32_t missing,
               int32_t *kmap) {
    // sparse_ops.cpp:126-140: every row starts at the sentinel; only rows that
    // own a key (first occurrence) get their 27 lookups filled.
    std::fill(kmap, kmap + 27 * n, missing);
    for (const auto &[key, row] : idx) {
        const auto [b, x, y, z] = key;
        for (int o = 0; o < 27; ++o) {
            int dx, dy, dz;
            offset_delta(o, &dx, &dy, &dz);
            int32_t nx, ny, nz;
            if (!add_fits(x, dx, &nx) || !add_fits(y, dy, &ny) || !add_fits(z, dz, &nz))
                continue;
            auto it = idx.find(Key4{b, nx, ny, nz});
            if (it != idx.end()) kmap[static_cast<int64_t>(row) * 27 + o] = it->second;
        }
    }
}

inline float silu_f(float v) { return v / (1.0f + std::exp(-v)); }

}  // namespace

extern "C" {

int orc_kmap_subm3(const int32_t *coords, int64_t n, int32_t missing, int32_t *kmap) {
    if (n <= 0) return 0;
    fill_kmap(ordered_index(coords, n), n, missing, kmap);
    return 1;
}

int64_t orc_coarsen2(const int32_t *coords, int64_t n, int32_t *coarse_coords,
                     int32_t *fine_to_coarse, int32_t *children, float *inv_count) {
    // sparse_ops.cpp:53-104.  Coarse key uses C++ truncating division; rows
    // are the lexicographic rank of the unique coarse keys.
    if (n <= 0) return -1;
    std::map<Key4, int32_t> coarse;
    auto ckey = [&](int64_t i) {
        const int32_t *c = coords + i * 4;
        return Key4{c[0], c[1] / 2, c[2] / 2, c[3] / 2};
    };
    for (int64_t i = 0; i < n; ++i) coarse.emplace(ckey(i), 0);
    int32_t id = 0;
    for (auto &[k, v] : coarse) {
        v = id;
        coarse_coords[id * 4 + 0] = std::get<0>(k);
        coarse_coords[id * 4 + 1] = std::get<1>(k);
        coarse_coords[id * 4 + 2] = std::get<2>(k);
        coarse_coords[id * 4 + 3] = std::get<3>(k);
        ++id;
    }
    const int64_t nc = id;
    std::vector<int32_t> cnt(static_cast<size_t>(nc), 0);
    std::fill(children, children + 8 * nc, static_cast<int32_t>(n));
    for (int64_t i = 0; i < n; ++i) {
        const int32_t c = coarse.at(ckey(i));
        fine_to_coarse[i] = c;
        const int slot = cnt[static_cast<size_t>(c)]++;
        if (slot < 8) children[static_cast<int64_t>(c) * 8 + slot] = static_cast<int32_t>(i);
    }
    for (int64_t c = 0; c < nc; ++c)
        inv_count[c] = 1.0f / static_cast<float>(cnt[static_cast<size_t>(c)] + 1);
    return nc;
}

int orc_subdivide2(const int32_t *parents, int64_t count, int32_t *child_coords,
                   int32_t *neighbors) {
    // sparse_ops.cpp:272-404, with an ordered map in place of the dense /
    // unordered parent index (the lookups answer the same questions).
    if (!parents || count <= 0 || count > INT32_MAX / 8) return 0;
    std::map<Key4, int32_t> pidx;
    for (int64_t p = 0; p < count; ++p) {
        const int32_t *c = parents + p * 4;
        if (!pidx.emplace(Key4{c[0], c[1], c[2], c[3]}, static_cast<int32_t>(p)).second)
            return 0;  // duplicate parent (:327, :329-332)
        for (int ch = 0; ch < 8; ++ch) {
            int32_t *o = child_coords + (p * 8 + ch) * 4;
            o[0] = c[0];
            o[1] = static_cast<int32_t>(static_cast<uint32_t>(c[1]) * 2u + (ch >> 2));
            o[2] = static_cast<int32_t>(static_cast<uint32_t>(c[2]) * 2u + ((ch >> 1) & 1));
            o[3] = static_cast<int32_t>(static_cast<uint32_t>(c[3]) * 2u + (ch & 1));
        }
    }
    // Children exist for every parent, so a child neighbour exists iff its
    // parent-grid cell exists: child (2p+bits)+d lives in parent
    // p + floor((bits+d)/2) at child slot (bits+d) mod 2 (:346-365).
    std::fill(neighbors, neighbors + count * 8 * 27, -1);
    for (int64_t p = 0; p < count; ++p) {
        const int32_t *c = parents + p * 4;
        for (int ch = 0; ch < 8; ++ch) {
            const int bits[3] = {ch >> 2, (ch >> 1) & 1, ch & 1};
            for (int o = 0; o < 27; ++o) {
                int d[3];
                offset_delta(o, &d[0], &d[1], &d[2]);
                int pd[3], tb[3];
                for (int a = 0; a < 3; ++a) {
                    const int v = bits[a] + d[a];
                    pd[a] = v < 0 ? -1 : (v > 1 ? 1 : 0);
                    tb[a] = v - 2 * pd[a];
                }
                int32_t px, py, pz;
                if (!add_fits(c[1], pd[0], &px) || !add_fits(c[2], pd[1], &py) ||
                    !add_fits(c[3], pd[2], &pz))
                    continue;
                auto it = pidx.find(Key4{c[0], px, py, pz});
                if (it == pidx.end()) continue;
                neighbors[(p * 8 + ch) * 27 + o] = it->second * 8 + tb[0] * 4 + tb[1] * 2 + tb[2];
            }
        }
    }
    return 1;
}

void orc_conv_subm(const float *x, int64_t n_in, int32_t cin, const int32_t *kmap,
                   int64_t n_out, int32_t kvol, const float *w, int32_t layout,
                   int32_t cout, const float *bias, float *y) {
    parallel_rows(n_out, default_threads(), [&](int64_t lo, int64_t hi) {
        std::vector<double> acc(static_cast<size_t>(cout));
        for (int64_t i = lo; i < hi; ++i) {
            for (int co = 0; co < cout; ++co) acc[co] = bias ? bias[co] : 0.0;
            for (int o = 0; o < kvol; ++o) {
                const int64_t j = kmap ? kmap[i * kvol + o] : i;
                if (j < 0 || j >= n_in) continue;  // missing neighbour -> zero row
                const float *xr = x + j * cin;
                for (int co = 0; co < cout; ++co) {
                    const float *wr = layout == 0
                                          ? w + (static_cast<int64_t>(co) * kvol + o) * cin
                                          : w + (static_cast<int64_t>(o) * cout + co) * cin;
                    // Four float64 partial sums (independent chains; the order
                    // is fixed, so results are deterministic).
                    double s[4] = {0.0, 0.0, 0.0, 0.0};
                    int ci = 0;
                    for (; ci + 4 <= cin; ci += 4)
                        for (int u = 0; u < 4; ++u)
                            s[u] += static_cast<double>(wr[ci + u]) * static_cast<double>(xr[ci + u]);
                    for (; ci < cin; ++ci) s[0] += static_cast<double>(wr[ci]) * static_cast<double>(xr[ci]);
                    acc[co] += (s[0] + s[1]) + (s[2] + s[3]);
                }
            }
            for (int co = 0; co < cout; ++co) y[i * cout + co] = static_cast<float>(acc[co]);
        }
    });
}

void orc_layernorm(const float *x, int64_t n, int32_t c, float eps, const float *w,
                   const float *b, float *y) {
    for (int64_t i = 0; i < n; ++i) {
        const float *r = x + i * c;
        double mean = 0.0;
        for (int k = 0; k < c; ++k) mean += r[k];
        mean /= c;
        double var = 0.0;
        for (int k = 0; k < c; ++k) var += (r[k] - mean) * (r[k] - mean);
        var /= c;
        const double rstd = 1.0 / std::sqrt(var + static_cast<double>(eps));
        for (int k = 0; k < c; ++k) {
            double v = (r[k] - mean) * rstd;
            if (w) v *= w[k];
            if (b) v += b[k];
            y[i * c + k] = static_cast<float>(v);
        }
    }
}

void orc_groupnorm(const float *x, int64_t n, int32_t c, int32_t groups, float eps,
                   const float *w, const float *b, float *y) {
    const int cg = c / groups;
    for (int g = 0; g < groups; ++g) {
        double s = 0.0;
        for (int64_t i = 0; i < n; ++i)
            for (int k = g * cg; k < (g + 1) * cg; ++k) s += x[i * c + k];
        const double cnt = static_cast<double>(n) * cg;
        const double mean = s / cnt;
        double v = 0.0;
        for (int64_t i = 0; i < n; ++i)
            for (int k = g * cg; k < (g + 1) * cg; ++k) {
                const double d = x[i * c + k] - mean;
                v += d * d;
            }
        const double rstd = 1.0 / std::sqrt(v / cnt + static_cast<double>(eps));
        for (int64_t i = 0; i < n; ++i)
            for (int k = g * cg; k < (g + 1) * cg; ++k) {
                double t = (x[i * c + k] - mean) * rstd;
                if (w) t *= w[k];
                if (b) t += b[k];
                y[i * c + k] = static_cast<float>(t);
            }
    }
}

void orc_silu(const float *x, int64_t count, float *y) {
    for (int64_t i = 0; i < count; ++i) y[i] = silu_f(x[i]);
}

void orc_modulate(const float *h, int64_t n, int32_t c, const float *scale,
                  const float *shift, float *y) {
    for (int64_t i = 0; i < n; ++i)
        for (int k = 0; k < c; ++k) {
            const float v = h[i * c + k];
            y[i * c + k] = (v * scale[k] + v) + shift[k];
        }
}

void orc_add(const float *a, const float *b, int64_t count, float *y) {
    for (int64_t i = 0; i < count; ++i) y[i] = a[i] + b[i];
}

void orc_downsample_mean(const float *x, int64_t nf, int32_t c, const int32_t *children,
                         const float *inv_count, int64_t nc, float *y) {
    for (int64_t r = 0; r < nc; ++r)
        for (int k = 0; k < c; ++k) {
            float s = 0.0f;
            for (int j = 0; j < 8; ++j) {
                const int32_t i = children[r * 8 + j];
                if (i >= 0 && i < nf) s += x[static_cast<int64_t>(i) * c + k];
            }
            y[r * c + k] = s * inv_count[r];
        }
}

void orc_upsample_nearest(const float *coarse, int64_t nc, int32_t c,
                          const int32_t *fine_to_coarse, int64_t nf, float *y) {
    for (int64_t i = 0; i < nf; ++i) {
        const int32_t r = fine_to_coarse[i];
        for (int k = 0; k < c; ++k)
            y[i * c + k] = (r >= 0 && r < nc) ? coarse[static_cast<int64_t>(r) * c + k] : 0.0f;
    }
}

void orc_repeat_children(const float *x, int64_t p, int32_t c, float *y) {
    for (int64_t i = 0; i < p; ++i)
        for (int j = 0; j < 8; ++j)
            std::memcpy(y + (i * 8 + j) * c, x + i * c, sizeof(float) * c);
}

int64_t orc_occupancy_coords(const float *occ, int32_t res, int32_t *out) {
    int64_t n = 0;
    for (int x = 0; x < res; ++x)
        for (int y = 0; y < res; ++y)
            for (int z = 0; z < res; ++z)
                if (occ[(static_cast<int64_t>(x) * res + y) * res + z] > 0.0f) {
                    out[n * 4 + 0] = 0;
                    out[n * 4 + 1] = x;
                    out[n * 4 + 2] = y;
                    out[n * 4 + 3] = z;
                    ++n;
                }
    return n;
}

int64_t orc_prune_surface(const int32_t *coords, int64_t n, int32_t *out) {
    // A voxel is kept when any of its 27 neighbourhood cells is empty.  Cells
    // are identified by the packed key of session.cpp:122-127 (b<<48 | x<<32
    // | y<<16 | z&0xffff, each field zero-extended), aliasing included.
    auto key = [](int32_t b, int32_t x, int32_t y, int32_t z) {
        return (static_cast<uint64_t>(static_cast<uint32_t>(b)) << 48) |
               (static_cast<uint64_t>(static_cast<uint32_t>(x)) << 32) |
               (static_cast<uint64_t>(static_cast<uint32_t>(y)) << 16) |
               static_cast<uint64_t>(static_cast<uint32_t>(z) & 0xffffu);
    };
    std::set<uint64_t> occ;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t *c = coords + i * 4;
        occ.insert(key(c[0], c[1], c[2], c[3]));
    }
    int64_t m = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t *c = coords + i * 4;
        bool surface = false;
        for (int o = 0; o < 27 && !surface; ++o) {
            int dx, dy, dz;
            offset_delta(o, &dx, &dy, &dz);
            if (!occ.count(key(c[0], c[1] + dx, c[2] + dy, c[3] + dz))) surface = true;
        }
        if (surface) {
            std::memcpy(out + m * 4, c, sizeof(int32_t) * 4);
            ++m;
        }
    }
    return m;
}

// --------------------------------------------------------------------------
// CPU baseline: im2col gather + FP32 GEMM (GGML CPU op decomposition).
// --------------------------------------------------------------------------
typedef float v8f __attribute__((vector_size(32)));

static inline v8f load8(const float *p) {
    v8f v;
    std::memcpy(&v, p, sizeof(v));
    return v;
}
static inline float hsum8(v8f v) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

void orc_conv_im2col_gemm_f32(const float *x, int64_t n_in, int32_t cin,
                              const int32_t *kmap, int64_t n_out, const float *w,
                              int32_t cout, const float *bias, float *y,
                              int32_t threads) {
    const int64_t K = 27LL * cin;
    const int64_t K8 = K & ~int64_t(7);
    constexpr int64_t RB = 16;  // im2col rows gathered per block
    if (threads <= 0) threads = default_threads();
    // Blocks of RB rows are dealt round-robin style so every thread streams W.
    const int64_t nblocks = (n_out + RB - 1) / RB;
    parallel_rows(nblocks, threads, [&](int64_t blo, int64_t bhi) {
        std::vector<float> a(static_cast<size_t>(RB * K));
        for (int64_t blk = blo; blk < bhi; ++blk) {
            const int64_t r0 = blk * RB, rows = std::min<int64_t>(RB, n_out - r0);
            // get_rows from the (n_in + 1)-row table whose last row is zero.
            for (int64_t r = 0; r < rows; ++r)
                for (int o = 0; o < 27; ++o) {
                    const int64_t j = kmap[(r0 + r) * 27 + o];
                    float *dst = a.data() + r * K + static_cast<int64_t>(o) * cin;
                    if (j >= 0 && j < n_in)
                        std::memcpy(dst, x + j * cin, sizeof(float) * cin);
                    else
                        std::memset(dst, 0, sizeof(float) * cin);
                }
            // GEMM: 2 rows x 4 output channels per register block.
            for (int64_t r = 0; r < rows; r += 2) {
                const bool two = r + 1 < rows;
                const float *a0 = a.data() + r * K;
                const float *a1 = two ? a0 + K : a0;
                for (int co = 0; co < cout; co += 4) {
                    const int nc4 = std::min(4, cout - co);
                    const float *wr[4];
                    for (int q = 0; q < 4; ++q) wr[q] = w + static_cast<int64_t>(co + std::min(q, nc4 - 1)) * K;
                    v8f s0[4] = {}, s1[4] = {};
                    for (int64_t k = 0; k < K8; k += 8) {
                        const v8f x0 = load8(a0 + k), x1 = load8(a1 + k);
                        for (int q = 0; q < 4; ++q) {
                            const v8f wv = load8(wr[q] + k);
                            s0[q] += x0 * wv;
                            s1[q] += x1 * wv;
                        }
                    }
                    for (int q = 0; q < nc4; ++q) {
                        float t0 = hsum8(s0[q]), t1 = hsum8(s1[q]);
                        for (int64_t k = K8; k < K; ++k) {
                            t0 += a0[k] * wr[q][k];
                            t1 += a1[k] * wr[q][k];
                        }
                        const float bb = bias ? bias[co + q] : 0.0f;
                        y[(r0 + r) * cout + co + q] = t0 + bb;
                        if (two) y[(r0 + r + 1) * cout + co + q] = t1 + bb;
                    }
                }
            }
        }
    });
}

void orc_round_bf16(const float *x, int64_t count, float *y) {
    for (int64_t i = 0; i < count; ++i) {
        uint32_t u;
        std::memcpy(&u, &x[i], 4);
        if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
            u |= 0x00400000u;  // quiet NaN, keep the payload's top bits
        } else {
            u += 0x7fffu + ((u >> 16) & 1u);
        }
        u &= 0xffff0000u;
        std::memcpy(&y[i], &u, 4);
    }
}

}  // extern "C"
