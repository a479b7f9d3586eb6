/*
 * s3dx_sparse.h -- C ABI of the MI355X (gfx950) sparse-voxel convolution path
 * of the sam3d.cpp Objects runtime (SLat flow sparse blocks and the mesh
 * decoder's sparse upsample stack).
 *
 * Conventions (mirroring include/sam3d.h:20-41 and src/error.hpp:15-22 of the
 * reference):
 *   - every fallible call returns s3dx_status and takes a caller-owned error
 *     buffer (error, error_capacity); success clears it, failure truncates and
 *     NUL-terminates the message; NULL,0 discards diagnostics, NULL,nonzero is
 *     S3DX_INVALID_ARGUMENT;
 *   - no exception, public struct layout or global last-error crosses the ABI;
 *   - every data pointer is a caller-owned DEVICE buffer unless the parameter
 *     says "host";
 *   - work is enqueued on the caller's stream (a hipStream_t, NULL = the
 *     default stream); calls that must report a data-dependent result to the
 *     host (a row count, a rejected input) synchronize that stream and say so;
 *   - distinct streams/requests may be used concurrently; one workspace must
 *     not be shared by calls in flight at the same time.
 *
 * Data layouts (as in the reference):
 *   coords   int32 [n][4] = (b, x, y, z), 16-byte aligned
 *   kmap     int32 [n][27], offset o = (dx+1)*9 + (dy+1)*3 + (dz+1)
 *            (sparse_ops.cpp:132); any entry outside [0, n_in) is a missing
 *            neighbour and contributes zero, which covers both the SLat
 *            sentinel n (sparse_ops.cpp:128) and the mesh sentinel -1
 *            (sparse_ops.cpp:367)
 *   features row-major [rows][C] (ggml (C, N), graph_builder.hpp:3-7),
 *            float32 or bfloat16
 */
#ifndef S3DX_SPARSE_H
#define S3DX_SPARSE_H

#include <stdint.h>

#define S3DX_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef uint32_t s3dx_status;
#define S3DX_OK UINT32_C(0)
#define S3DX_INVALID_ARGUMENT UINT32_C(1)
#define S3DX_OUT_OF_MEMORY UINT32_C(2)
#define S3DX_INTERNAL_ERROR UINT32_C(3)

typedef void *s3dx_stream; /* hipStream_t */
typedef void *s3dx_event;  /* hipEvent_t */

/* element types */
#define S3DX_F32 0
#define S3DX_BF16 1

/* source weight layouts accepted by s3dx_conv_set_weights (float32, host) */
#define S3DX_WEIGHT_SLAT 0 /* [Cout][kvol][Cin]: the converter's (Cout, 27*Cin) rows,
                              scripts/objects/gguf_schema.py:326-334 */
#define S3DX_WEIGHT_MESH 1 /* [kvol][Cout][Cin]: packed ne{Cin*Cout, 27},
                              scripts/objects/convert_sam3d_to_gguf.py:486-492 */

#define S3DX_ABI_VERSION UINT32_C(1)
S3DX_API uint32_t s3dx_abi_version(void);

/* ------------------------------------------------------------------------
 * Device plumbing: the Backend seam of the reference
 * (src/objects_runtime/backend.hpp:16-58: alloc, set_input_*, run,
 * get_tensor_*), reduced to what a caller of this library needs.
 * ---------------------------------------------------------------------- */
S3DX_API s3dx_status s3dx_device_info(int32_t *device_count, char *name, uint64_t name_capacity,
                                      char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_malloc(void **out, uint64_t bytes, char *error, uint64_t error_capacity);
S3DX_API void s3dx_free(void *ptr);
/* Copies enqueue on `stream` and then synchronize it (set_input_* / get_tensor_*). */
S3DX_API s3dx_status s3dx_memcpy_h2d(void *dst, const void *host_src, uint64_t bytes,
                                     s3dx_stream stream, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_memcpy_d2h(void *host_dst, const void *src, uint64_t bytes,
                                     s3dx_stream stream, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_stream_create(s3dx_stream *out, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_stream_destroy(s3dx_stream stream, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_stream_synchronize(s3dx_stream stream, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_event_create(s3dx_event *out, char *error, uint64_t error_capacity);
/* An event for timing only (no counterpart in the reference; for benchmarks):
 * recording it skips the system-scope memory fence, whose cache write-back and
 * invalidation would otherwise land between the timed launches.  Not for
 * making device writes visible to the host. */
S3DX_API s3dx_status s3dx_timing_event_create(s3dx_event *out, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_event_destroy(s3dx_event event, char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_event_record(s3dx_event event, s3dx_stream stream, char *error,
                                       uint64_t error_capacity);
/* Waits for `stop`, then writes the milliseconds between the two events. */
S3DX_API s3dx_status s3dx_event_elapsed_ms(s3dx_event start, s3dx_event stop, float *ms,
                                           char *error, uint64_t error_capacity);

/* ------------------------------------------------------------------------
 * Kernel maps (the host table builders of sparse_ops.{hpp,cpp}, on device)
 * ---------------------------------------------------------------------- */

/* Workspace bytes for s3dx_kmap_subm3 on n voxels (host query). */
S3DX_API s3dx_status s3dx_kmap_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                              uint64_t error_capacity);

/* Submanifold 3x3x3 neighbour table.  Replaces build_conv
 * (sparse_ops.cpp:117-142) for the fine and coarse SLat maps (missing_value
 * = n) and the mesh neighbour rows (missing_value = -1).  kmap[i][o] is the
 * row of the FIRST voxel with coordinates coords[i] + delta(o), or
 * missing_value; rows of later duplicates of a coordinate stay entirely
 * missing_value (sparse_ops.cpp:120-141).  Byte-identical to the reference.
 * Requires 0 < n <= INT32_MAX / 27.  Asynchronous on `stream`, two
 * launches.  The workspace needs no clearing: every build tags the words it
 * writes with a fresh per-call tag, and a word is used only when its row's
 * input coordinates are the ones looked up, so the map is byte-identical to
 * the reference whatever the workspace holds on entry (zeros, an earlier
 * build's table, or arbitrary bytes); one workspace serves any sequence of
 * builds on one stream. */
S3DX_API s3dx_status s3dx_kmap_subm3(const int32_t *coords, int64_t n, int32_t missing_value,
                                     int32_t *kmap, void *workspace, uint64_t workspace_bytes,
                                     s3dx_stream stream, char *error, uint64_t error_capacity);

/* s3dx_kmap_subm3 without a workspace and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  The table lives in a static device array of the library
 * (18 MiB + 256 bytes on each GPU it runs on, held until the process ends),
 * so n is limited to 262144 voxels (S3DX_INVALID_ARGUMENT above that).  Same
 * kernels and results as s3dx_kmap_subm3 (per-call tags, rows checked
 * against the input coordinates, no clearing pass: the array starts zeroed
 * and keeps the last call's table).  All calls on one GPU share that array:
 * calls that overlap in time on one GPU (different streams, threads) race
 * and must be serialized by the caller. */
S3DX_API s3dx_status s3dx_kmap_subm3_static(const int32_t *coords, int64_t n, int32_t missing_value,
                                            int32_t *kmap, s3dx_stream stream, char *error,
                                            uint64_t error_capacity);

/* Workspace bytes for s3dx_coarsen2 on n fine voxels (host query). */
S3DX_API s3dx_status s3dx_coarsen2_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                                  uint64_t error_capacity);

/* 2x OR-pool of the SLat downsample tables (sparse_ops.cpp:53-104).  Coarse
 * keys are (b, x/2, y/2, z/2) with C++ truncating division; coarse rows are
 * their lexicographic rank.  Outputs (capacities for nc <= n):
 *   coarse_coords   int32 [n][4]   (first nc rows written)
 *   fine_to_coarse  int32 [n]
 *   coarse_children int32 [8n]     (first 8*nc written; c*8+j = j-th smallest
 *                                   fine row of coarse row c, sentinel n)
 *   coarse_inv_count float [n]     (1/(count+1), the scatter-mean quirk)
 *   *nc_out         host int64
 * The coarse kernel map is s3dx_kmap_subm3(coarse_coords, nc, nc, ...)
 * (sparse_ops.cpp:142).  Sets of batch 0 in [0, 128)^3 with at most eight
 * rows per coarse cell take a window (a bitmap of the coarse cells ranked by
 * a scan, no sort) and synchronize `stream` once, to return nc; any other set
 * is sorted (O(n log n) for any int32 coordinates and bounding box) after
 * that synchronization and synchronizes once more. */
S3DX_API s3dx_status s3dx_coarsen2(const int32_t *coords, int64_t n, int32_t *coarse_coords,
                                   int32_t *fine_to_coarse, int32_t *coarse_children,
                                   float *coarse_inv_count, int64_t *nc_out, void *workspace,
                                   uint64_t workspace_bytes, s3dx_stream stream, char *error,
                                   uint64_t error_capacity);

/* Workspace bytes for s3dx_subdivide2 on `parent_count` parents (host query). */
S3DX_API s3dx_status s3dx_subdivide2_workspace_size(int64_t parent_count, uint64_t *bytes,
                                                    char *error, uint64_t error_capacity);

/* Exact 2x subdivide + child neighbour table, replacing
 * MeshSubdivideTables::build (sparse_ops.cpp:272-404).  child_coords
 * [8p][4]: row p*8 + (bx*4 + by*2 + bz) = (b, 2x+bx, 2y+by, 2z+bz), z fastest.
 * child_kmap [8p][27] (may be NULL): neighbour rows, -1 when missing.
 * Rejects p <= 0, p > INT32_MAX/8 and duplicate parents with
 * S3DX_INVALID_ARGUMENT (the reference returns false).  Synchronizes
 * `stream` to check for duplicates. */
S3DX_API s3dx_status s3dx_subdivide2(const int32_t *parent_coords, int64_t parent_count,
                                     int32_t *child_coords, int32_t *child_kmap, void *workspace,
                                     uint64_t workspace_bytes, s3dx_stream stream, char *error,
                                     uint64_t error_capacity);

/* ------------------------------------------------------------------------
 * Occupancy -> coordinates (the step before the SLat stage,
 * src/objects_runtime/session.cpp).  Each keeps the reference's row order and
 * synchronizes `stream` once to read the row count.  Cells are told apart by
 * the reference's coordinate_key (session.cpp:122-127), overlapping fields
 * and all, so every int32 input gives the reference's rows.
 * ---------------------------------------------------------------------- */

S3DX_API s3dx_status s3dx_occupancy_workspace_size(int32_t nx, int32_t ny, int32_t nz, uint64_t *bytes,
                                                   char *error, uint64_t error_capacity);
/* Threshold of the decoder's occupancy: every cell with occupancy > 0, in
 * x-major order (flat = (x*ny + y)*nz + z), as rows (0, x, y, z)
 * (session.cpp:1437-1441).  occupancy: device float32 [nx][ny][nz];
 * coords: device int32 [nx*ny*nz][4] capacity; *count: rows written. */
S3DX_API s3dx_status s3dx_occupancy_coords(const float *occupancy, int32_t nx, int32_t ny, int32_t nz,
                                           int32_t *coords, int64_t *count, void *workspace,
                                           uint64_t workspace_bytes, s3dx_stream stream, char *error,
                                           uint64_t error_capacity);

S3DX_API s3dx_status s3dx_prune_surface_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                                       uint64_t error_capacity);
/* prune_surface_coords (session.cpp:133-163): the rows with at least one
 * empty cell in their 3x3x3 neighbourhood (same b), in input order.
 * surface: int32 [n][4] capacity.  Requires 0 < n <= INT32_MAX / 27. */
S3DX_API s3dx_status s3dx_prune_surface(const int32_t *coords, int64_t n, int32_t *surface,
                                        int64_t *count, void *workspace, uint64_t workspace_bytes,
                                        s3dx_stream stream, char *error, uint64_t error_capacity);

S3DX_API s3dx_status s3dx_downsample_coords_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                                           uint64_t error_capacity);
/* downsample_coords (session.cpp:168-233; the pipeline calls it with
 * max_coords 42000, factor 2, seed 42): n <= max_coords returns the rows
 * unchanged; otherwise each axis is mapped onto a centred range of 1/factor
 * the bounding box (double precision, rounded half up, clamped), duplicates
 * dropped keeping first occurrences, and more than max_coords survivors are
 * sampled by std::shuffle under std::mt19937(seed), as the reference does.
 * out: int32 [min(n, max_coords)][4] capacity. */
S3DX_API s3dx_status s3dx_downsample_coords(const int32_t *coords, int64_t n, int64_t max_coords,
                                            int32_t factor, uint32_t seed, int32_t *out, int64_t *count,
                                            void *workspace, uint64_t workspace_bytes, s3dx_stream stream,
                                            char *error, uint64_t error_capacity);

/* ------------------------------------------------------------------------
 * Sparse convolution layer: the SLat `conv` lambda + gb_linear
 * (slat_flow_graph.cpp:105-155, graph_builder.cpp:44-54) and the mesh
 * `convolution` lambda (mesh_decoder_graph.cpp:81-103), as one
 * gather-GEMM kernel with fused prologue/epilogue.  kvol 1 with a NULL kmap is
 * a linear layer (1x1 skip, 96->101 head, build_mesh_output_layer
 * mesh_decoder_graph.cpp:134-140).
 *
 * Per output row i:  v = bias + sum_o W_o . in(kmap[i][o])
 *   in(j)   = x[j]                               (default)
 *           = x[j >> 3] + slot_offset[j & 7]     (gather_parent: repeat_children
 *                                                 mesh_decoder_graph.cpp:32-38)
 *           then silu(in*pre_scale + pre_shift)  (input affine+SiLU: GroupNorm
 *                                                 apply + ggml_silu; missing
 *                                                 rows stay zero)
 * The parent repeat alone costs nothing (the gather reads row j >> 3).  Slot
 * offsets and the affine + SiLU run once per source element, in a row pass
 * before the gather, into a buffer the layer object owns and grows on demand
 * (rows: 8 * n_in with slot offsets, else n_in), rounded to the conv's dtype
 * as a stored tensor would be.  Runs of one such layer object on different
 * streams must not overlap: they share that buffer.
 *   v -> LayerNorm over Cout (eps, optional affine), optional modulate
 *        v*scale + v + shift (slat_flow_graph.cpp:55-59) -> optional SiLU
 *        -> optional + residual[i] -> y[i]
 * All of it in float32, rounded once to y's dtype.  When the output tile
 * cannot span the row (Cout above 256, or not whole 32-column blocks) the
 * LayerNorm runs as a second pass over the conv's float32 output, kept in
 * another buffer the layer owns (n_out * Cout * 4 bytes, same rules).
 * Arithmetic: float32 inputs use FP32 MFMA/VALU; bfloat16 inputs use BF16 MFMA;
 * both accumulate in float32.  Deterministic (no atomics on outputs).
 * ---------------------------------------------------------------------- */
typedef struct s3dx_conv s3dx_conv;

/* dtype: S3DX_F32 or S3DX_BF16 (the input feature type and the arithmetic). */
S3DX_API s3dx_status s3dx_conv_create(int32_t cin, int32_t cout, int32_t kvol, int32_t dtype,
                                      s3dx_conv **out, char *error, uint64_t error_capacity);
S3DX_API void s3dx_conv_free(s3dx_conv *conv);
/* host float32 weights in `layout` and optional host bias [cout]; packed once
 * into the device layout the kernel reads. */
S3DX_API s3dx_status s3dx_conv_set_weights(s3dx_conv *conv, const float *host_weight,
                                           int32_t layout, const float *host_bias,
                                           char *error, uint64_t error_capacity);
/* repeat_children of the input; host slot_offset [8][cin] float32 may be NULL. */
S3DX_API s3dx_status s3dx_conv_set_gather_parent(s3dx_conv *conv, int32_t enable,
                                                 const float *host_slot_offset, char *error,
                                                 uint64_t error_capacity);
/* Input affine + SiLU; DEVICE scale/shift [cin] float32, read at run time
 * (s3dx_groupnorm_stats writes them).  NULL,NULL disables. */
S3DX_API s3dx_status s3dx_conv_set_input_affine_silu(s3dx_conv *conv, const float *scale,
                                                     const float *shift, char *error,
                                                     uint64_t error_capacity);
/* Fused epilogue LayerNorm (enable 0/1), host affine weight/bias [cout] and
 * host modulate scale/shift [cout], each may be NULL. */
S3DX_API s3dx_status s3dx_conv_set_layernorm(s3dx_conv *conv, int32_t enable, float eps,
                                             const float *host_weight, const float *host_bias,
                                             const float *host_mod_scale,
                                             const float *host_mod_shift, char *error,
                                             uint64_t error_capacity);
/* Per-forward modulate of the fused LayerNorm, h*scale + h + shift
 * (slat_flow_graph.cpp:55-59): DEVICE scale/shift [cout] float32, caller-owned,
 * read when s3dx_conv_run runs.  In the SLat res_block they are the two halves
 * of emb_layers(silu(t_emb)), recomputed on the device for each of the flow's
 * forwards (slat_flow_graph.cpp:238-243, 257), so a caller updates the buffers
 * and runs again without touching the layer.  Takes precedence over host
 * modulate arrays given to s3dx_conv_set_layernorm; NULL,NULL returns to
 * those.  Requires the LayerNorm epilogue to be enabled; disabling it clears
 * this setting. */
S3DX_API s3dx_status s3dx_conv_set_modulate(s3dx_conv *conv, const float *scale, const float *shift,
                                            char *error, uint64_t error_capacity);
S3DX_API s3dx_status s3dx_conv_set_silu(s3dx_conv *conv, int32_t enable, char *error,
                                        uint64_t error_capacity);
/* Residual at parent resolution (enable 0/1): the residual passed to
 * s3dx_conv_run holds ceil(n_out / 8) rows and output row i adds residual row
 * i >> 3, i.e. repeat_children of a per-parent tensor.  The mesh block's skip
 * (mesh_decoder_graph.cpp:125-131) is a 1x1 conv of repeat_children(x), which
 * equals repeat_children of the 1x1 conv of x: run the skip on the parents
 * and let the block's second conv add it this way. */
S3DX_API s3dx_status s3dx_conv_set_residual_parent(s3dx_conv *conv, int32_t enable, char *error,
                                                   uint64_t error_capacity);
/* Input dtype of the layer's x: its own dtype (the default), or S3DX_BF16
 * for an S3DX_F32 layer.  No counterpart as a call: the reference's graph
 * feeds F32 tensors throughout; this lets a BF16 producer feed an FP32 layer
 * (the mesh head, mesh_decoder_graph.cpp:134-140) without a separate
 * conversion pass.  The rows are exact in FP32: 1x1 layers read them in
 * the kernel (with Cin 32, 64, 96 or 128 and Cout <= 128 on BF16 MFMAs,
 * the FP32 weights split into three BF16 terms, at FP32 accuracy), others
 * widen them once into the layer's buffer (same rule as the transforms).
 * Not combinable with input transforms. */
S3DX_API s3dx_status s3dx_conv_set_input_dtype(s3dx_conv *conv, int32_t dtype, char *error,
                                               uint64_t error_capacity);
/* Runs the layer.  x [n_in or n_in parents][cin] in the layer's input dtype; kmap
 * [n_out][kvol] (NULL only for kvol 1, where output row i reads input row i,
 * so n_out may not exceed the input rows); residual [n_out][cout] in y_dtype
 * or NULL; y [n_out][cout] in y_dtype.  Asynchronous on `stream`.  Launches
 * in stream-K runs (see s3dx_conv_run_planned; FP32 layers of Cin >= 256 as
 * well) keep their partial tiles in another buffer the layer owns (up to
 * 64 MiB): as with the transform buffer, runs of one layer object on
 * different streams must not overlap. */
S3DX_API s3dx_status s3dx_conv_run(const s3dx_conv *conv, const void *x, int64_t n_in,
                                   const int32_t *kmap, int64_t n_out, const void *residual,
                                   void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                   uint64_t error_capacity);
/* Gather plans.  No counterpart in the reference, whose GGML graph gathers
 * im2col rows afresh in every forward (slat_flow_graph.cpp:116-130).  A plan
 * holds, for each 64-row tile of a kernel map, the distinct source rows its
 * 27 offsets name and the table the halo-staged kernel gathers them by --
 * work that otherwise opens every such launch.  It depends only on the map
 * and on how `conv` reads its input (n_in rows, parent rows or transformed
 * rows), so build it once per map (as the reference builds its tables once
 * per sample, session.cpp:1563-1566) and pass it to every
 * s3dx_conv_run_planned over that map by layers set up alike (e.g. both
 * convs of a res_block).  The caller keeps kmap unchanged while the plan is
 * in use.  create enqueues the build on `stream` and picks the records' tile
 * height from `conv`: 128 output rows when its halo kernel's 128-row tiles
 * fill the GPU's compute units in one pass (runs then use an 8-wave kernel
 * on those tiles; 18 KiB of device memory per 128 rows), else 64 rows (7
 * KiB per 64 rows); free releases it. */
typedef struct s3dx_gather_plan s3dx_gather_plan;
S3DX_API s3dx_status s3dx_gather_plan_create(const s3dx_conv *conv, int64_t n_in, const int32_t *kmap,
                                             int64_t n_out, s3dx_stream stream, s3dx_gather_plan **out,
                                             char *error, uint64_t error_capacity);
S3DX_API void s3dx_gather_plan_free(s3dx_gather_plan *plan);
/* Rebuilds `plan` in place for another map (e.g. the next sample's), with no
 * allocation: n_out may be at most the n_out the plan was created for
 * (S3DX_INVALID_ARGUMENT otherwise).  Enqueued on `stream`; runs still
 * queued on another stream that read the old plan must be ordered before it. */
S3DX_API s3dx_status s3dx_gather_plan_rebuild(s3dx_gather_plan *plan, const s3dx_conv *conv, int64_t n_in,
                                              const int32_t *kmap, int64_t n_out, s3dx_stream stream,
                                              char *error, uint64_t error_capacity);
/* s3dx_kmap_subm3 followed by s3dx_gather_plan_rebuild(plan, conv, n, kmap,
 * n) in one pass: the kernel map of coords into kmap (byte-identical to
 * s3dx_kmap_subm3, same workspace and guarantees) and, from the same
 * lookups, the map's gather plan for `conv`'s source rows -- two launches
 * instead of three, and the map is not read back.  No counterpart as a call:
 * the reference builds its tables on the host once per sample
 * (session.cpp:1563-1566) and gathers im2col rows afresh in every forward.
 * For layers that gather the map's own rows (not s3dx_conv_set_gather_parent);
 * n at most the rows the plan was created for. */
S3DX_API s3dx_status s3dx_kmap_subm3_planned(const int32_t *coords, int64_t n, int32_t missing_value,
                                             int32_t *kmap, s3dx_gather_plan *plan, const s3dx_conv *conv,
                                             void *workspace, uint64_t workspace_bytes, s3dx_stream stream,
                                             char *error, uint64_t error_capacity);
/* s3dx_conv_run with a gather plan built for the same kmap, n_out and source
 * rows (S3DX_INVALID_ARGUMENT when the sizes or the source setup differ).
 * Results are bit-identical to s3dx_conv_run, except for layers of at least
 * 512 input channels whose 128-row tiles outnumber the CUs (e.g. 1024 -> 1024
 * on 5,086 rows): with a 128-row plan those run in stream-K runs, equal runs
 * of (tile, 64-channel chunk) units one per CU, and a tile split between
 * runs adds its pieces in a fixed order, so results are deterministic but
 * rounded differently from the unplanned run (within BF16 rounding).
 * Launches that do not use the halo kernel ignore the plan. */
S3DX_API s3dx_status s3dx_conv_run_planned(const s3dx_conv *conv, const s3dx_gather_plan *plan, const void *x,
                                           int64_t n_in, const int32_t *kmap, int64_t n_out, const void *residual,
                                           void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                           uint64_t error_capacity);
/* Describes, as one line of text, the kernel variant s3dx_conv_run launches
 * for n_in input and n_out output rows (buffers assumed 16-byte aligned,
 * output in the layer's dtype, no residual: a BF16 1x1 layer's "linear pipe"
 * kernel takes only those), e.g. "mfma tiling=11 split-k rows=128 cols=128
 * kc=128 xf=0 ln=fused grid=221x1".  Host only, no device work.  No counterpart in the reference
 * (whose conv is a fixed GGML graph); it exists for tests and benchmarks. */
S3DX_API s3dx_status s3dx_conv_plan(const s3dx_conv *conv, int64_t n_in, int64_t n_out, char *plan,
                                    uint64_t plan_capacity, char *error, uint64_t error_capacity);
/* The same for s3dx_conv_run_planned with `gather_plan`: the kernel it
 * launches, with " plan=64" or " plan=128" appended when that kernel reads
 * the plan.  No counterpart in the reference. */
S3DX_API s3dx_status s3dx_conv_plan_planned(const s3dx_conv *conv, const s3dx_gather_plan *gather_plan,
                                            int64_t n_in, int64_t n_out, char *plan, uint64_t plan_capacity,
                                            char *error, uint64_t error_capacity);

/* ------------------------------------------------------------------------
 * Standalone row ops (graph_builder.cpp:56-62, mesh_decoder_graph.cpp:16-30,
 * slat_flow_graph.cpp:157-190).  x and y may alias where noted.
 * ---------------------------------------------------------------------- */

/* y = [silu]( modulate( LayerNorm_rows(x, eps) * w + b ) ); w, b, mod_scale,
 * mod_shift are device [c] float32 or NULL.  x/y dtype F32 or BF16; x == y
 * allowed. */
S3DX_API s3dx_status s3dx_layernorm_rows(const void *x, int32_t x_dtype, int64_t n, int32_t c,
                                         float eps, const float *w, const float *b,
                                         const float *mod_scale, const float *mod_shift,
                                         int32_t silu, void *y, int32_t y_dtype,
                                         s3dx_stream stream, char *error,
                                         uint64_t error_capacity);

/* Workspace bytes for s3dx_groupnorm_stats (host query). */
S3DX_API s3dx_status s3dx_groupnorm_workspace_size(int64_t n, int32_t c, int32_t groups,
                                                   uint64_t *bytes, char *error,
                                                   uint64_t error_capacity);
/* SparseGroupNorm statistics over all n rows (eps, groups | c): writes the
 * per-channel affine scale[c] = gamma*rstd, shift[c] = beta - mean*gamma*rstd
 * (device float32 [c]) that s3dx_conv_set_input_affine_silu or
 * s3dx_affine_rows consume.  gamma/beta device [c] or NULL.  Two-pass,
 * deterministic. */
S3DX_API s3dx_status s3dx_groupnorm_stats(const void *x, int32_t x_dtype, int64_t n, int32_t c,
                                          int32_t groups, float eps, const float *gamma,
                                          const float *beta, float *scale, float *shift,
                                          void *workspace, uint64_t workspace_bytes,
                                          s3dx_stream stream, char *error,
                                          uint64_t error_capacity);
/* y = [silu](x*scale + shift) per channel; x == y allowed. */
S3DX_API s3dx_status s3dx_affine_rows(const void *x, int32_t x_dtype, int64_t n, int32_t c,
                                      const float *scale, const float *shift, int32_t silu,
                                      void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                      uint64_t error_capacity);

/* SLat downsample (slat_flow_graph.cpp:159-183): y[r] = inv_count[r] *
 * sum_j x[children[r*8+j]], entries outside [0, nf) contribute zero. */
S3DX_API s3dx_status s3dx_downsample_mean(const void *x, int32_t dtype, int64_t nf, int32_t c,
                                          const int32_t *children, const float *inv_count,
                                          int64_t nc, void *y, s3dx_stream stream, char *error,
                                          uint64_t error_capacity);
/* SLat upsample (slat_flow_graph.cpp:186-190): y[i] = coarse[fine_to_coarse[i]]. */
S3DX_API s3dx_status s3dx_upsample_nearest(const void *coarse, int32_t dtype, int64_t nc,
                                           int32_t c, const int32_t *fine_to_coarse, int64_t nf,
                                           void *y, s3dx_stream stream, char *error,
                                           uint64_t error_capacity);
/* Row concatenation along channels (ggml_concat of the SLat out blocks,
 * slat_flow_graph.cpp:443, 477), optionally through a row index:
 * y[i] = [a[r][0..ca), b[r][0..cb)] with r = rows[i] (rows NULL: r = i),
 * zero rows for r outside [0, n_src).  With rows = fine_to_coarse it is
 * out_blocks.0's concat + nearest upsample (:443-444) in one pass.  A copy,
 * bit-exact; y [n][ca + cb] must not overlap a or b. */
S3DX_API s3dx_status s3dx_concat_rows(const void *a, int32_t ca, const void *b, int32_t cb, int32_t dtype,
                                      int64_t n_src, const int32_t *rows, int64_t n, void *y,
                                      s3dx_stream stream, char *error, uint64_t error_capacity);
/* dtype conversion F32 <-> BF16 (round to nearest even), count elements. */
S3DX_API s3dx_status s3dx_convert(const void *x, int32_t x_dtype, int64_t count, void *y,
                                  int32_t y_dtype, s3dx_stream stream, char *error,
                                  uint64_t error_capacity);

#ifdef __cplusplus
}
#endif
#endif
