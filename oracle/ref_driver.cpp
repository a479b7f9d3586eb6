// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A C entry layer over the reference's own sparse_ops.cpp, compiled from
// /root/reference/src/objects_runtime by oracle/Makefile into
// oracle/_ref/libref_sparse_ops.so.  It lets the tests and the fixture writer
// call the reference's SlatTables::build and MeshSubdivideTables::build
// directly.  The reference source is compiled where it lies; nothing of it is
// copied here.
#include "sparse_ops.hpp"

#include <cstring>

extern "C" {

// SlatTables::build (sparse_ops.hpp:36).  Output capacities: conv_fine 27n,
// fine_to_coarse n, conv_coarse 27n, coarse_children 8n, coarse_inv_count n.
// Returns nc, or -1 when build() returns false.
int64_t ref_slat_tables(const int32_t *coords, int64_t n, int32_t channels,
                        int32_t *conv_fine, int32_t *fine_to_coarse,
                        int32_t *conv_coarse, int32_t *coarse_children,
                        float *coarse_inv_count) {
    sam3d::SlatTables tb;
    if (!tb.build(coords, n, channels)) return -1;
    std::memcpy(conv_fine, tb.conv_fine.data(), tb.conv_fine.size() * sizeof(int32_t));
    std::memcpy(fine_to_coarse, tb.fine_to_coarse.data(), tb.fine_to_coarse.size() * sizeof(int32_t));
    std::memcpy(conv_coarse, tb.conv_coarse.data(), tb.conv_coarse.size() * sizeof(int32_t));
    std::memcpy(coarse_children, tb.coarse_children.data(), tb.coarse_children.size() * sizeof(int32_t));
    std::memcpy(coarse_inv_count, tb.coarse_inv_count.data(), tb.coarse_inv_count.size() * sizeof(float));
    return tb.nc;
}

// MeshSubdivideTables::build (sparse_ops.hpp:77).  Returns 1 on success, 0 when
// build() returns false.
int ref_mesh_subdivide(const int32_t *parents, int64_t count, int32_t *child_coords,
                       int32_t *neighbors) {
    sam3d::MeshSubdivideTables t;
    if (!t.build(parents, count)) return 0;
    std::memcpy(child_coords, t.child_coords.data(), t.child_coords.size() * sizeof(int32_t));
    std::memcpy(neighbors, t.neighbors.data(), t.neighbors.size() * sizeof(int32_t));
    return 1;
}

}  // extern "C"
