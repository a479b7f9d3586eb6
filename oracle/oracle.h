/*
 * oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the sam3d.cpp sparse-voxel path, used as the parity
 * checker by tests/, by __graft_entry__.smoke() and by the bench's
 * cpu_baseline leg.  Nothing in the product (sam3d.cpp_amd/) links, loads or
 * calls this library.  Each function names the reference lines it restates.
 *
 * Conventions (same as the reference):
 *   coords   int32 [n][4] = (b, x, y, z)
 *   kmap     int32 [n][27], offset o = (dx+1)*9 + (dy+1)*3 + (dz+1)
 *   features row-major [rows][C] float32
 *   a kmap entry outside [0, n_in) is a missing neighbour (zero contribution)
 */
#ifndef S3DX_ORACLE_H
#define S3DX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* sparse_ops.cpp:117-142 (build_conv over the fine index of :119-124). */
int orc_kmap_subm3(const int32_t *coords, int64_t n, int32_t missing, int32_t *kmap);

/* sparse_ops.cpp:53-104 + :142.  coarse_coords cap n*4, children cap 8n,
 * inv_count cap n.  Returns nc (>0) or -1 for n <= 0. */
int64_t orc_coarsen2(const int32_t *coords, int64_t n, int32_t *coarse_coords,
                     int32_t *fine_to_coarse, int32_t *children, float *inv_count);

/* sparse_ops.cpp:272-404.  Returns 1 on success, 0 on rejection (count <= 0,
 * count > INT32_MAX/8, duplicate parent). */
int orc_subdivide2(const int32_t *parents, int64_t count, int32_t *child_coords,
                   int32_t *neighbors);

/* Sparse conv y[i] = bias + sum_o W_o x[kmap[i][o]], accumulated in double.
 * layout 0: W [cout][kvol][cin] (slat_flow_graph.cpp:112-130 with the
 *           converter's (Cout, 27*Cin) rows, gguf_schema.py:326-334)
 * layout 1: W [kvol][cout][cin] (mesh_decoder_graph.cpp:81-103,
 *           convert_sam3d_to_gguf.py:486-492)
 * kvol 1 with kmap == NULL is the identity map (a linear layer). */
void orc_conv_subm(const float *x, int64_t n_in, int32_t cin, const int32_t *kmap,
                   int64_t n_out, int32_t kvol, const float *w, int32_t layout,
                   int32_t cout, const float *bias, float *y);

/* ggml_norm over each row + optional affine (graph_builder.cpp:56-62). */
void orc_layernorm(const float *x, int64_t n, int32_t c, float eps, const float *w,
                   const float *b, float *y);
/* sparse_group_norm (mesh_decoder_graph.cpp:16-30): statistics over every row
 * and the C/groups channels of a group, then affine. */
void orc_groupnorm(const float *x, int64_t n, int32_t c, int32_t groups, float eps,
                   const float *w, const float *b, float *y);
/* ggml_silu, in place allowed. */
void orc_silu(const float *x, int64_t count, float *y);
/* modulate (slat_flow_graph.cpp:55-59): h*scale + h + shift, per channel. */
void orc_modulate(const float *h, int64_t n, int32_t c, const float *scale,
                  const float *shift, float *y);
/* y = a + b elementwise. */
void orc_add(const float *a, const float *b, int64_t count, float *y);
/* downsample (slat_flow_graph.cpp:159-183): sum of the 8 gathered children
 * (sentinel rows are zero) times coarse_inv_count. */
void orc_downsample_mean(const float *x, int64_t nf, int32_t c, const int32_t *children,
                         const float *inv_count, int64_t nc, float *y);
/* upsample (slat_flow_graph.cpp:186-190): y[i] = coarse[fine_to_coarse[i]]. */
void orc_upsample_nearest(const float *coarse, int64_t nc, int32_t c,
                          const int32_t *fine_to_coarse, int64_t nf, float *y);
/* repeat_children (mesh_decoder_graph.cpp:32-38): y[p*8+j] = x[p]. */
void orc_repeat_children(const float *x, int64_t p, int32_t c, float *y);

/* session.cpp:1437-1441: occupancy logits [64][64][64] (x-major) > 0 ->
 * coords (0,x,y,z); returns count, out cap 64^3*4. */
int64_t orc_occupancy_coords(const float *occ, int32_t res, int32_t *out);
/* session.cpp:133-163 prune_surface_coords(max_neighbor_axes_dist=1). */
int64_t orc_prune_surface(const int32_t *coords, int64_t n, int32_t *out);
/* session.cpp:168-233 downsample_coords (oracle_coords.cpp); out cap
 * min(n, max_coords) rows; returns the row count. */
int64_t orc_downsample_coords(const int32_t *coords, int64_t n, int64_t max_coords, int32_t factor,
                              uint32_t seed, int32_t *out);
/* k-th output (1-based) of std::mt19937(seed). */
uint32_t orc_mt19937_draw(uint32_t seed, int64_t k);

/* CPU baseline: the GGML CPU decomposition of the SLat conv
 * (slat_flow_graph.cpp:116-130): concat a zero row, get_rows im2col into
 * [n_out][27*cin], then an FP32 GEMM against W [cout][27*cin] plus bias,
 * split over output rows on `threads` threads.  Accumulates in float. */
void orc_conv_im2col_gemm_f32(const float *x, int64_t n_in, int32_t cin,
                              const int32_t *kmap, int64_t n_out, const float *w,
                              int32_t cout, const float *bias, float *y,
                              int32_t threads);

/* Round float32 to bfloat16 (nearest-even) and back, elementwise. */
void orc_round_bf16(const float *x, int64_t count, float *y);

#ifdef __cplusplus
}
#endif
#endif
