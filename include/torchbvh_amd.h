/*
 * torchbvh_amd C ABI — BVH build and exact k-NN for 2-D/3-D fp32 point clouds
 * on AMD Instinct MI355X (gfx950).
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as `void*`; a null stream means the legacy default stream).  The
 * library never allocates device memory: callers query a workspace size, pass
 * a device buffer of at least that many bytes, and own every output buffer.
 * All launches are asynchronous on `stream`; no entry point synchronises the
 * host.  Entry points are reentrant; calls that share one workspace buffer on
 * overlapping streams race, exactly as two kernels writing one buffer would.
 *
 * Return value: TBVH_OK (0) on success, otherwise an error code, with a
 * human-readable message available from tbvh_last_error() on the calling
 * thread.
 *
 * Layouts (identical to the reference's handle payload):
 *   points          [B, N, D] fp32 (batched) or [T, D] packed (ragged)
 *   node_aabbs      [B, nr, 2D] fp32, row = (lo_0..lo_{D-1}, hi_0..hi_{D-1}),
 *                   real nodes of the implicit tree in level order
 *   sorted_indices  [B, N] int64, per-cloud (local) original point index of
 *                   each Morton-ordered leaf
 *   scene_min/max   [B, D] fp32
 *   left/right_child_mem, mem_to_leaf   [nr] int32 (ragged: packed per cloud)
 *   order           [B, M] int64 local query indices in Morton order
 *   out_indices     [B, M, K] int64 local point indices, ascending by
 *                   (squared distance, index)
 *   out_distances   [B, M, K] fp32 squared distances
 */
#ifndef TORCHBVH_AMD_H
#define TORCHBVH_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TBVH_OK = 0,
    TBVH_ERR_INVALID_ARGUMENT = 1,
    TBVH_ERR_WORKSPACE_TOO_SMALL = 2,
    TBVH_ERR_HIP = 3,
};

/* ABI version of this header; bumped on any signature change. */
#define TBVH_ABI_VERSION 2
int tbvh_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* tbvh_last_error(void);

/* ---- implicit-tree closed forms (host only; no GPU work) -------------------
 * Replace implicit_tree.cuh:55-68 (`virtual_leaves`, `real_node_count`,
 * `leaf_level`) for sizing outputs on the host.  n >= 1 and n <= INT32_MAX. */
int     tbvh_leaf_level(int64_t n);
int64_t tbvh_virtual_leaves(int64_t n);
int64_t tbvh_real_node_count(int64_t n);

/* ---- batched build ----------------------------------------------------------
 * Replaces `build_bvh_batched_cooperative` (torchbvh/csrc/bindings.cpp:155-157,
 * torchbvh/csrc/bvh_build.cu:679-721): per-cloud AABB, 30-bit (3-D) or 32-bit
 * (2-D) Morton codes, stable key/value sort, implicit-tree node AABBs and the
 * traversal arrays, for B clouds of N points.  Requires B >= 1, N >= 1,
 * B*N <= INT32_MAX, D in {2,3}.  `left_child_mem`, `right_child_mem` and
 * `mem_to_leaf` are [nr] (shared by all clouds, as in the reference). */
int tbvh_build_workspace_size(int64_t B, int64_t N, int D, size_t* bytes);
int tbvh_build(const float* points, int64_t B, int64_t N, int D,
               float* node_aabbs, int64_t* sorted_indices,
               float* scene_min, float* scene_max,
               int32_t* left_child_mem, int32_t* right_child_mem,
               int32_t* mem_to_leaf,
               void* workspace, size_t workspace_bytes, void* stream);

/* ---- ragged build -------------------------------------------------------------
 * Replaces the per-segment Python loop of `_build_bvh_ragged`
 * (torchbvh/_query.py:68-85), which calls the batched build once per cloud,
 * with one segmented launch sequence.  `offsets` is a device int64 [B+1]
 * array (0 = offsets[0] < offsets[1] < ... < offsets[B] = total).  Outputs
 * are the per-cloud results concatenated: node_aabbs [sum nr_b, 2D],
 * sorted_indices [total] (local indices), scene_min/max [B, D], the three
 * traversal arrays [sum nr_b], and node_offsets [B+1] int64 (device) giving
 * each cloud's first node row.  `total_nodes` = sum of real_node_count(n_b)
 * (the caller sizes the outputs with it).  Offsets are validated by the
 * caller; the library trusts them. */
int tbvh_build_ragged_workspace_size(int64_t B, int64_t total, int D,
                                     size_t* bytes);
int tbvh_build_ragged(const float* points, const int64_t* offsets,
                      int64_t B, int64_t total, int D,
                      float* node_aabbs, int64_t* sorted_indices,
                      float* scene_min, float* scene_max,
                      int32_t* left_child_mem, int32_t* right_child_mem,
                      int32_t* mem_to_leaf, int64_t* node_offsets,
                      int64_t total_nodes,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---- build + acceleration structure in one call ------------------------------
 * No counterpart in the reference (it has no acceleration structure).  Same
 * outputs as tbvh_build / tbvh_build_ragged and, in the same launch sequence,
 * the k-NN acceleration structure that tbvh_accel_build(_ragged) would build
 * from them (sized by tbvh_accel_size, 256-byte aligned); it reuses the sort's
 * keys and the tree passes' point reads instead of recomputing them.  Every
 * cloud must hold at most 2^28 points.  Same workspace size as the plain
 * builds. */
int tbvh_build_with_accel(const float* points, int64_t B, int64_t N, int D,
                          float* node_aabbs, int64_t* sorted_indices,
                          float* scene_min, float* scene_max,
                          int32_t* left_child_mem, int32_t* right_child_mem,
                          int32_t* mem_to_leaf, void* accel,
                          void* workspace, size_t workspace_bytes, void* stream);
int tbvh_build_ragged_with_accel(const float* points, const int64_t* offsets,
                                 int64_t B, int64_t total, int D,
                                 float* node_aabbs, int64_t* sorted_indices,
                                 float* scene_min, float* scene_max,
                                 int32_t* left_child_mem, int32_t* right_child_mem,
                                 int32_t* mem_to_leaf, int64_t* node_offsets,
                                 int64_t total_nodes, void* accel,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* ---- build + acceleration structure without any allocation -------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tbvh_build_with_accel with its workspace taken from a
 * library-owned device array of TBVH_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends) instead of a caller buffer.  Outputs and their
 * layout are those of tbvh_build_with_accel, bit for bit.  Fails with
 * TBVH_ERR_WORKSPACE_TOO_SMALL when tbvh_build_workspace_size(B, N, D)
 * exceeds the array (about 3.9M points in total).  `stream` must belong to
 * the calling thread's current device.  Calls no allocator.  Every call on
 * one GPU uses that GPU's one array, so calls that overlap on one GPU
 * (other streams, other host threads) race; calls in order on one stream
 * do not. */
#define TBVH_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int tbvh_build_with_accel_noalloc(const float* points, int64_t B, int64_t N, int D,
                                  float* node_aabbs, int64_t* sorted_indices,
                                  float* scene_min, float* scene_max,
                                  int32_t* left_child_mem, int32_t* right_child_mem,
                                  int32_t* mem_to_leaf, void* accel, void* stream);

/* ---- primitive build ----------------------------------------------------------
 * Replaces `build_primitive_bvh_batched` (torchbvh/csrc/bindings.cpp:159-160,
 * torchbvh/csrc/bvh_build.cu:60-93, 757-821; used by `_ray.py:195`):
 * `primitives` is [B, F, V, D] float32, (V, D) = (2, 2) segments or (3, 3)
 * triangles.  Leaves are the primitives' vertex boxes; each cloud's bounds
 * are the min / max of those boxes' corners; the Morton codes are of the
 * centres (vertex sum / V) against those bounds.  Outputs as tbvh_build,
 * with F in place of N.  The sort is stable (the reference's is not: the
 * orders agree wherever centre codes are distinct). */
int tbvh_build_primitives_workspace_size(int64_t B, int64_t F, int V, int D, size_t* bytes);
int tbvh_build_primitives(const float* primitives, int64_t B, int64_t F, int V, int D,
                          float* node_aabbs, int64_t* sorted_indices,
                          float* scene_min, float* scene_max,
                          int32_t* left_child_mem, int32_t* right_child_mem,
                          int32_t* mem_to_leaf,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- point ordering -----------------------------------------------------------
 * Replaces `morton_sort_points_batched` (torchbvh/csrc/bindings.cpp:194,
 * torchbvh/csrc/bvh_build.cu:723-740; used by `_fps.py:112, 190`): each
 * cloud's bounds, 30/32-bit Morton codes against them and the stable order,
 * `sorted_indices` [B, N] int64 (cloud-local).  The bounds are the points'
 * plain min / max (the reference's points.min(1) / max(1), :731-732), not
 * the build's +-1e30-seeded ones, so the order equals tbvh_build's
 * `sorted_indices` except for a cloud lying entirely beyond +-1e30 on an
 * axis.  NaN coordinates are outside the contract (torch's min/max
 * propagate NaN, the reduction here skips it). */
int tbvh_morton_sort_points_workspace_size(int64_t B, int64_t N, int D, size_t* bytes);
int tbvh_morton_sort_points(const float* points, int64_t B, int64_t N, int D,
                            int64_t* sorted_indices,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ---- query ordering -----------------------------------------------------------
 * Replaces `morton_sort_queries_narrow` (torchbvh/csrc/morton_sort.cu:212-287):
 * Morton codes of the queries against the BVH's scene bounds, stable sort,
 * int64 order [B, M].  M may be 0 (nothing is launched). */
int tbvh_sort_queries_workspace_size(int64_t B, int64_t M, int D,
                                     size_t* bytes);
int tbvh_sort_queries(const float* queries, int64_t B, int64_t M, int D,
                      const float* scene_min, const float* scene_max,
                      int64_t* order,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Ragged form: queries [total_q, D] packed by `query_offsets` (device int64
 * [B+1]); `order` [total_q] receives local query indices per cloud.  Replaces
 * the per-segment calls made by `_query_knn_ragged` (torchbvh/_query.py:347-360). */
int tbvh_sort_queries_ragged_workspace_size(int64_t B, int64_t total_q, int D,
                                            size_t* bytes);
int tbvh_sort_queries_ragged(const float* queries, const int64_t* query_offsets,
                             int64_t B, int64_t total_q, int D,
                             const float* scene_min, const float* scene_max,
                             int64_t* order,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/* ---- k-NN with neighbour rows (fused gather) ------------------------------------------
 * No entry-point counterpart: the reference gathers source_points[indices]
 * in Python after the k-NN call (torchbvh/_query.py:169-174, 203-215,
 * 362-366).  These run tbvh_knn_accel / tbvh_knn_accel_ragged and also write,
 * for result row r and neighbour j, the source row of that neighbour:
 * out_positions[(r * k + j) * source_cols + c].  `source_points` has the
 * points' layout ([B, num_leaves, source_cols] batched, packed rows with
 * point_offsets ragged), float32. */
int tbvh_knn_accel_positions(const void* accel, const float* queries, const int64_t* order,
                             int64_t B, int64_t M, int64_t num_leaves, int D, int k,
                             const float* source_points, int source_cols,
                             int64_t* out_indices, float* out_distances, float* out_positions,
                             void* stream);
/* tbvh_knn_accel_grid with the neighbour rows of tbvh_knn_accel_positions
 * (the same workspace; results and rows the same as
 * tbvh_knn_accel_positions'). */
int tbvh_knn_accel_grid_positions(const void* accel, const float* node_aabbs,
                                  int64_t num_real_nodes, const float* queries,
                                  const int64_t* order, int64_t B, int64_t M,
                                  int64_t num_leaves, int D, int k,
                                  const float* source_points, int source_cols,
                                  int64_t* out_indices, float* out_distances,
                                  float* out_positions, void* workspace,
                                  size_t workspace_bytes, void* stream);
int tbvh_knn_accel_ragged_positions(const void* accel, const int64_t* point_offsets,
                                    int64_t total_points, const float* queries,
                                    const int64_t* query_offsets, const int64_t* order,
                                    int64_t B, int64_t total_q, int D, int k,
                                    const float* source_points, int source_cols,
                                    int64_t* out_indices, float* out_distances,
                                    float* out_positions, void* stream);

/* ---- traversal schedule ----------------------------------------------------------------
 * No counterpart in the reference (`query_knn` there orders queries with the
 * full sort above, `_query.py:142,241`).  The order only schedules the
 * traversal — k-NN results do not depend on it — so these key each query
 * on the Hilbert index of its Morton-grid cell (1024 cells per axis in 3-D,
 * 65536 in 2-D; J. Skilling, AIP Conf. Proc. 707, 2004) and sort on its top
 * 16 bits only (stable: ties keep ascending query index), two radix passes
 * instead of four.  Same arguments and workspace sizes as
 * tbvh_sort_queries / tbvh_sort_queries_ragged. */
int tbvh_schedule_queries(const float* queries, int64_t B, int64_t M, int D,
                          const float* scene_min, const float* scene_max,
                          int64_t* order,
                          void* workspace, size_t workspace_bytes, void* stream);
int tbvh_schedule_queries_ragged(const float* queries, const int64_t* query_offsets,
                                 int64_t B, int64_t total_q, int D,
                                 const float* scene_min, const float* scene_max,
                                 int64_t* order,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* ---- routed query ordering -------------------------------------------------------------
 * Replaces `morton_sort_routed_queries_batched` (torchbvh/csrc/bindings.cpp:196,
 * morton_sort.cu:82-120, 288-329; used by `_conditional.py:164`): every query
 * [b, m] has a route (bool as one byte; true selects the first of two BVHs)
 * and is encoded against that route's bounds; `order` [B, M] int64 is the
 * stable order of the composite key (route << code_bits | code), i.e. each
 * cloud's false-route queries in Morton order, then its true-route queries. */
int tbvh_sort_routed_queries_workspace_size(int64_t B, int64_t M, int D,
                                            size_t* bytes);
int tbvh_sort_routed_queries(const float* queries, const uint8_t* routes,
                             int64_t B, int64_t M, int D,
                             const float* true_min, const float* true_max,
                             const float* false_min, const float* false_max,
                             int64_t* order,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ---- diagnostic: Morton codes ------------------------------------------------------
 * No counterpart in the reference's FFI (its codes stay inside
 * `narrow_morton_sort_batched`, bvh_build.cu:551-600, and
 * `morton_sort_queries_narrow_impl`, morton_sort.cu:212-262).  Exposes the
 * library's Morton kernel so parity tests can compare codes bit for bit:
 * codes [B*M] u32 of rows [B, M, D] against per-cloud bounds [B, D].  Uses the
 * query-ordering workspace size. */
int tbvh_morton_codes(const float* rows, int64_t B, int64_t M, int D,
                      const float* scene_min, const float* scene_max,
                      uint32_t* codes,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---- exact k-NN ------------------------------------------------------------------
 * Replaces `query_knn_batched_cached_bounds` and
 * `query_knn_batched_cached_bounds_ordered` (torchbvh/csrc/knn_query.cu:419-446,
 * dispatch and checks :350-417).  `order` may be NULL (queries are launched in
 * input order).  k in {4, 8, 16, 32}; num_leaves >= k.  Results are the k
 * smallest (squared distance, index) pairs in lexicographic order, so exact
 * distance ties resolve to the lower point index.  The traversal makes the
 * reference's visits in the reference's order, so it also returns the
 * reference's rows where they depend on that order (points with a NaN
 * coordinate, which no node box bounds). */
int tbvh_knn(const float* node_aabbs, const int64_t* sorted_indices,
             const float* queries, const int64_t* order,
             int64_t B, int64_t M, int64_t num_leaves, int64_t num_real_nodes,
             int D, int k,
             int64_t* out_indices, float* out_distances, void* stream);

/* Spatial-output form.  Replaces `query_knn_batched_cached_bounds_spatial`
 * (torchbvh/csrc/bindings.cpp:199, knn_query.cu:448-461, used by
 * `_mls.py:169`): same search, but output row [b, m] holds the result of
 * query order[b, m] (the launch order, which is the Morton order the MLS
 * kernels consume) instead of query m.  `order` is required. */
int tbvh_knn_spatial(const float* node_aabbs, const int64_t* sorted_indices,
                     const float* queries, const int64_t* order,
                     int64_t B, int64_t M, int64_t num_leaves, int64_t num_real_nodes,
                     int D, int k,
                     int64_t* out_indices, float* out_distances, void* stream);

/* Ragged form over the packed outputs of tbvh_build_ragged.  point_offsets,
 * node_offsets and query_offsets are device int64 [B+1]; `order` (local query
 * indices from tbvh_sort_queries_ragged) may be NULL.  Every cloud must hold
 * at least k points (checked by the caller).  Output rows follow the packed
 * query rows; indices are local to each cloud. */
int tbvh_knn_ragged(const float* node_aabbs, const int64_t* sorted_indices,
                    const int64_t* point_offsets, const int64_t* node_offsets,
                    const float* queries, const int64_t* query_offsets,
                    const int64_t* order,
                    int64_t B, int64_t total_q, int D, int k,
                    int64_t* out_indices, float* out_distances, void* stream);

/* ---- k-NN acceleration structure ------------------------------------------------
 * No counterpart in the reference: its traversal walks the implicit tree
 * directly (torchbvh/csrc/knn_query.cu:47-154).  Built from a finished BVH
 * (the points plus tbvh_build's / tbvh_build_ragged's outputs), an accel
 * buffer holds a radix tree over the same Morton order with exact child
 * boxes, parent links and leaf buckets of up to 6 (3-D) or 8 (2-D) points;
 * tbvh_knn_accel(_ragged) returns exactly what tbvh_knn(_ragged) returns for
 * the same BVH while visiting about ten times fewer nodes.  Clouds may hold
 * at most 2^28 points.
 *   accel bytes   : tbvh_accel_size(B, total_points, D)
 *   workspace     : tbvh_accel_workspace_size(B, total_points, D)
 * For the batched form total_points = B * N.  tbvh_accel_build_from_tree
 * needs only the BVH's node_aabbs and sorted_indices (a caller of the
 * reference's query bindings holds nothing else; num_real_nodes must be
 * real_node_count(N)): the leaf rows are the points in Morton order and the
 * root box gives the build's bounds, so it writes the same bytes as
 * tbvh_accel_build.  That holds only for the point BVH the build writes, so
 * it also checks the tensors on the device and stores into the device word
 * *defects 0 when they are one (leaf rows degenerate boxes, lo and hi
 * bitwise equal; every internal row the fminf/fmaxf merge of its children,
 * a copy of the left child where the right one is virtual; leaf codes
 * non-decreasing; sorted indices in [0, N)) and 1 otherwise (a primitive
 * BVH, edited boxes, another Morton order): the accel is then not to be
 * used, and tbvh_knn answers for those tensors.
 * Precondition of tbvh_knn_accel*: `accel` (256-byte aligned, else
 * TBVH_ERR_INVALID_ARGUMENT) holds what one of these builders (or
 * tbvh_build*_with_accel) wrote for the same clouds.  Its child and parent
 * links are followed as stored; refs outside a cloud are skipped (no read
 * leaves the cloud's rows), but links corrupted into a cycle would keep
 * the traversal running without end, so an accel must never be modified or
 * taken from another BVH (the Python layer records which node_aabbs each
 * accel it builds belongs to and refuses any other pairing). */
int tbvh_accel_size(int64_t B, int64_t total_points, int D, size_t* bytes);
int tbvh_accel_workspace_size(int64_t B, int64_t total_points, int D, size_t* bytes);
int tbvh_accel_build(const float* points, const int64_t* sorted_indices,
                     const float* node_aabbs, const float* scene_min,
                     const float* scene_max, int64_t B, int64_t N, int D,
                     void* accel, void* workspace, size_t workspace_bytes,
                     void* stream);
int tbvh_accel_build_from_tree(const float* node_aabbs, const int64_t* sorted_indices,
                               int64_t B, int64_t N, int64_t num_real_nodes, int D,
                               void* accel, uint32_t* defects,
                               void* workspace, size_t workspace_bytes, void* stream);
int tbvh_accel_build_ragged(const float* points, const int64_t* offsets,
                            const int64_t* sorted_indices, const float* node_aabbs,
                            const float* scene_min, const float* scene_max,
                            int64_t B, int64_t total, int D,
                            void* accel, void* workspace, size_t workspace_bytes,
                            void* stream);
int tbvh_knn_accel(const void* accel, const float* queries, const int64_t* order,
                   int64_t B, int64_t M, int64_t num_leaves, int D, int k,
                   int64_t* out_indices, float* out_distances, void* stream);
/* Spatial-output form of tbvh_knn_accel (see tbvh_knn_spatial). */
int tbvh_knn_accel_spatial(const void* accel, const float* queries, const int64_t* order,
                           int64_t B, int64_t M, int64_t num_leaves, int D, int k,
                           int64_t* out_indices, float* out_distances, void* stream);
/* tbvh_knn_accel with a workspace, for the same bindings
 * (`query_knn_batched_cached_bounds(_ordered)`, torchbvh/csrc/bindings.cpp:
 * 197-198, knn_query.cu:419-446): the same results, found by a cell-block
 * search first.  The accel's points are cut into Morton cells against each
 * cloud's root box (row 0 of its node_aabbs, num_real_nodes rows per cloud,
 * which must be real_node_count(num_leaves)); each query scans the 3^D
 * cells around its own and keeps that result when its k-th distance lies
 * inside the block's margin (then no point outside can enter the list);
 * the others, and every query of a cloud that is not near-uniform (a long
 * empty run of cells, a non-finite point, cells out of the points' order),
 * run the accel traversal seeded with that k-th distance.  Workspace:
 * tbvh_knn_accel_grid_workspace_size (0 for clouds too small for a grid
 * or of 2^24 points or more: then this is tbvh_knn_accel); a null
 * workspace also runs tbvh_knn_accel. */
int tbvh_knn_accel_grid_workspace_size(int64_t B, int64_t M, int64_t num_leaves, int D, int k,
                                       size_t* bytes);
int tbvh_knn_accel_grid(const void* accel, const float* node_aabbs, int64_t num_real_nodes,
                        const float* queries, const int64_t* order,
                        int64_t B, int64_t M, int64_t num_leaves, int D, int k,
                        int64_t* out_indices, float* out_distances,
                        void* workspace, size_t workspace_bytes, void* stream);
/* Spatial-output form of tbvh_knn_accel_grid, for the binding
 * `query_knn_batched_cached_bounds_spatial` (torchbvh/csrc/bindings.cpp:
 * 199, knn_query.cu:448-461): results in launch (order) position, the same
 * as tbvh_knn_accel_spatial's; the same workspace; `order` required. */
int tbvh_knn_accel_grid_spatial(const void* accel, const float* node_aabbs,
                                int64_t num_real_nodes, const float* queries,
                                const int64_t* order, int64_t B, int64_t M,
                                int64_t num_leaves, int D, int k,
                                int64_t* out_indices, float* out_distances,
                                void* workspace, size_t workspace_bytes, void* stream);
int tbvh_knn_accel_ragged(const void* accel, const int64_t* point_offsets,
                          int64_t total_points, const float* queries,
                          const int64_t* query_offsets, const int64_t* order,
                          int64_t B, int64_t total_q, int D, int k,
                          int64_t* out_indices, float* out_distances, void* stream);

/* ---- routed k-NN (spatial output) --------------------------------------------------
 * Replaces `query_knn_routed_batched_cached_bounds_spatial`
 * (torchbvh/csrc/bindings.cpp:200, knn_query.cu:183-327, 463-539; used by `_conditional.py:181`):
 * query [b, order[b, m]] searches the true-route tree if routes[b, query] is
 * non-zero, else the false-route tree, whose indices are reported after the
 * true cloud's (+ true_num_leaves); output row [b, m] (launch order).  Both
 * clouds need at least k points.  Same candidate rule as tbvh_knn. */
int tbvh_knn_routed_spatial(const float* true_node_aabbs, const int64_t* true_sorted_indices,
                            const float* false_node_aabbs, const int64_t* false_sorted_indices,
                            const float* queries, const uint8_t* routes, const int64_t* order,
                            int64_t B, int64_t M,
                            int64_t true_num_leaves, int64_t true_num_real_nodes,
                            int64_t false_num_leaves, int64_t false_num_real_nodes,
                            int D, int k,
                            int64_t* out_indices, float* out_distances, void* stream);
/* Same over the two clouds' acceleration structures (no counterpart in the
 * reference; identical results). */
int tbvh_knn_accel_routed_spatial(const void* true_accel, const void* false_accel,
                                  const float* queries, const uint8_t* routes,
                                  const int64_t* order, int64_t B, int64_t M,
                                  int64_t true_num_leaves, int64_t false_num_leaves,
                                  int D, int k,
                                  int64_t* out_indices, float* out_distances, void* stream);
/* Cell-block form of tbvh_knn_accel_routed_spatial, for the same binding
 * (no counterpart in the reference; identical results): each query first
 * searches the block of grid cells around it in its route's structure (as
 * tbvh_knn_accel_grid does, against that structure's root box, row 0 of
 * its node_aabbs per cloud), and the queries the block cannot decide run
 * the routed accel traversal.  Workspace:
 * tbvh_knn_accel_routed_grid_workspace_size (0 where either cloud is too
 * small for a grid, or of 2^24 points or more: then this is
 * tbvh_knn_accel_routed_spatial); a null workspace also runs that. */
int tbvh_knn_accel_routed_grid_workspace_size(int64_t B, int64_t M, int64_t true_num_leaves,
                                              int64_t false_num_leaves, int D, int k, size_t* bytes);
int tbvh_knn_accel_routed_grid_spatial(const void* true_accel, const float* true_node_aabbs,
                                       int64_t true_num_real_nodes, const void* false_accel,
                                       const float* false_node_aabbs, int64_t false_num_real_nodes,
                                       const float* queries, const uint8_t* routes,
                                       const int64_t* order, int64_t B, int64_t M,
                                       int64_t true_num_leaves, int64_t false_num_leaves,
                                       int D, int k, int64_t* out_indices, float* out_distances,
                                       void* workspace, size_t workspace_bytes, void* stream);

/* ---- displaced-query interpolation --------------------------------------------------
 * Replaces the neighbour gather and rank loop of `interpolate_displaced`
 * (torchbvh/_multihead.py:123-144): values (B, N, H, C), indices, weights
 * and exact (B, N, H, k; indices local to the cloud, weights already
 * normalised, exact non-zero where the neighbour is an exact hit), out
 * (B, N, H, C).  out[b, n, h, c] = sum over ranks j in order of
 * values[b, indices[.., j], h, c] * weights[.., j], or, where any exact[.., j]
 * is set, the sum of those neighbours' values divided by their count; each
 * step rounds the product and the sum separately, as the reference's tensor
 * operations do.  An index outside [0, N) contributes zero. */
int tbvh_interpolate_neighbors(const float* values, const int64_t* indices, const float* weights,
                               const uint8_t* exact, int64_t B, int64_t N, int64_t H, int64_t C, int k,
                               float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHBVH_AMD_H */
