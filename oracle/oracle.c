/*
 * oracle.c — CPU restatement of the reference's BVH build + exact k-NN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped.  The product (torchbvh_amd) never
 * links, loads or calls it.
 *
 * Each function cites the reference code it restates (paths relative to the
 * reference repository).  Deliberate, documented differences from the
 * reference, shared with the HIP path:
 *   - Morton normalisation uses IEEE fp32 division (the reference is compiled
 *     with --use_fast_math; its approximate divide cannot be reproduced).
 *   - k-NN ties: results are the k smallest (distance, index) pairs in
 *     lexicographic order (the reference keeps DFS order among equal
 *     distances, which its own docs leave unspecified).
 *   - k = 32 is accepted in addition to 4, 8, 16.
 * Build: see oracle/build_oracle.py (gcc -O2 -ffp-contract=off -fopenmp).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------
 * Implicit tree closed forms — torchbvh/csrc/implicit_tree.cuh:26-127
 * ---------------------------------------------------------------------- */
static int flog2(uint32_t x) { return 31 - __builtin_clz(x); }
static int clog2(uint32_t x) { return x <= 1 ? 0 : flog2(x - 1) + 1; }

int orc_leaf_level(int n) { return clog2((uint32_t)n); }                  /* :55-58 */
int orc_virtual_leaves(int n) { return (1 << orc_leaf_level(n)) - n; }     /* :50-53 */
int orc_real_node_count(int n) {                                           /* :55-58 */
    return 2 * n - 1 + __builtin_popcount((uint32_t)orc_virtual_leaves(n));
}
static int level_of(int i) { return flog2((uint32_t)i + 1u); }             /* :74-76 */
static int virtual_nodes_above(int n, int level) {                         /* :64-68 */
    const int L = orc_leaf_level(n);
    const int shift = L - level + 1;
    const uint32_t lvl = shift >= 32 ? 0u : ((uint32_t)orc_virtual_leaves(n) >> shift);
    return (int)(2u * lvl) - __builtin_popcount(lvl);
}
static int real_nodes_at_level(int n, int level) {                         /* :86-89 */
    const int L = orc_leaf_level(n);
    return (1 << level) - (orc_virtual_leaves(n) >> (L - level));
}
int orc_memory_index(int n, int i) { return i - virtual_nodes_above(n, level_of(i)); } /* :91-94 */
int orc_is_virtual(int n, int i) {                                         /* :96-100 */
    const int level = level_of(i);
    return i - ((1 << level) - 1) >= real_nodes_at_level(n, level);
}

/* ------------------------------------------------------------------------
 * Morton codes — torchbvh/csrc/morton.cuh:19-68 (IEEE division)
 * ---------------------------------------------------------------------- */
static float clamp01(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }
static float normalize_axis(float x, float lo, float hi) {
    const float extent = hi - lo;
    if (extent <= 0.0f) return 0.0f;
    return clamp01((x - lo) / extent);
}
static uint32_t quantize(float x, uint32_t bins) {
    const float scaled = clamp01(x) * (float)bins;
    const uint32_t q = (uint32_t)scaled;
    return q >= bins ? bins - 1u : q;
}
uint32_t orc_split3(uint32_t x) {
    x &= 0x3ffu;
    x = (x | (x << 16)) & 0x030000ffu;
    x = (x | (x << 8)) & 0x0300f00fu;
    x = (x | (x << 4)) & 0x030c30c3u;
    x = (x | (x << 2)) & 0x09249249u;
    return x;
}
uint32_t orc_split2(uint32_t x) {
    x &= 0xffffu;
    x = (x | (x << 8)) & 0x00ff00ffu;
    x = (x | (x << 4)) & 0x0f0f0f0fu;
    x = (x | (x << 2)) & 0x33333333u;
    x = (x | (x << 1)) & 0x55555555u;
    return x;
}
uint32_t orc_morton(const float* p, int D, const float* lo, const float* hi) {
    if (D == 3) {
        return orc_split3(quantize(normalize_axis(p[0], lo[0], hi[0]), 1024u)) |
               (orc_split3(quantize(normalize_axis(p[1], lo[1], hi[1]), 1024u)) << 1) |
               (orc_split3(quantize(normalize_axis(p[2], lo[2], hi[2]), 1024u)) << 2);
    }
    return orc_split2(quantize(normalize_axis(p[0], lo[0], hi[0]), 65536u)) |
           (orc_split2(quantize(normalize_axis(p[1], lo[1], hi[1]), 65536u)) << 1);
}
void orc_morton_codes(const float* pts, int64_t n, int D, const float* lo, const float* hi,
                      uint32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_morton(pts + i * D, D, lo, hi);
}

/* ------------------------------------------------------------------------
 * Hilbert index of integer cells, b bits per axis (no reference
 * counterpart: this library's traversal schedule).  Skilling, "Programming
 * the Hilbert curve", AIP Conf. Proc. 707 (2004): the axes-to-transpose
 * transform (undo excess work, Gray encode), then the transposed bits read
 * level by level from the top, axis 0 first within a level.
 * ---------------------------------------------------------------------- */
uint32_t orc_hilbert_cell(const uint32_t* cell, int D, int b) {
    uint32_t x[3] = {0u, 0u, 0u};
    for (int d = 0; d < D; ++d) x[d] = cell[d];
    for (uint32_t q = 1u << (b - 1); q > 1u; q >>= 1) {
        const uint32_t m = q - 1u;
        for (int i = 0; i < D; ++i) {
            if (x[i] & q) {
                x[0] ^= m;
            } else {
                const uint32_t t = (x[0] ^ x[i]) & m;
                x[0] ^= t;
                x[i] ^= t;
            }
        }
    }
    for (int i = 1; i < D; ++i) x[i] ^= x[i - 1];
    uint32_t t = 0u;
    for (uint32_t q = 1u << (b - 1); q > 1u; q >>= 1)
        if (x[D - 1] & q) t ^= q - 1u;
    for (int i = 0; i < D; ++i) x[i] ^= t;
    uint32_t h = 0u;
    for (int j = b - 1; j >= 0; --j)
        for (int i = 0; i < D; ++i) h = (h << 1) | ((x[i] >> j) & 1u);
    return h;
}
void orc_hilbert_cells(const uint32_t* cells, int64_t n, int D, int b, uint32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_hilbert_cell(cells + i * D, D, b);
}
/* The same cells as the Morton codes (1024 per axis in 3-D, 65536 in 2-D). */
void orc_hilbert_codes(const float* pts, int64_t n, int D, const float* lo, const float* hi,
                       uint32_t* out) {
    const int b = D == 3 ? 10 : 16;
    for (int64_t i = 0; i < n; ++i) {
        uint32_t c[3];
        for (int d = 0; d < D; ++d) c[d] = quantize(normalize_axis(pts[i * D + d], lo[d], hi[d]), 1u << b);
        out[i] = orc_hilbert_cell(c, D, b);
    }
}

/* ------------------------------------------------------------------------
 * Bounds — torchbvh/csrc/bvh_build.cu:453-494 (fminf/fmaxf from +-1e30)
 * ---------------------------------------------------------------------- */
void orc_bounds(const float* pts, int64_t n, int D, float* lo, float* hi) {
    for (int d = 0; d < D; ++d) {
        float a = 1.0e30f, b = -1.0e30f;
        for (int64_t i = 0; i < n; ++i) {
            a = fminf(a, pts[i * D + d]);
            b = fmaxf(b, pts[i * D + d]);
        }
        lo[d] = a;
        hi[d] = b;
    }
}

/* ------------------------------------------------------------------------
 * Stable argsort by u32 key — the contract of the reference's
 * cub::DeviceSegmentedRadixSort::SortPairs over iota values
 * (bvh_build.cu:551-600, morton_sort.cu:212-262): ascending key, equal keys
 * in ascending original index.  Bottom-up merge sort.
 * ---------------------------------------------------------------------- */
void orc_stable_argsort(const uint32_t* keys, int64_t n, int64_t* perm) {
    int64_t* tmp = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n > 0 ? n : 1));
    for (int64_t i = 0; i < n; ++i) perm[i] = i;
    int64_t* src = perm;
    int64_t* dst = tmp;
    for (int64_t w = 1; w < n; w *= 2) {
        for (int64_t lo = 0; lo < n; lo += 2 * w) {
            int64_t mid = lo + w < n ? lo + w : n;
            int64_t hi = lo + 2 * w < n ? lo + 2 * w : n;
            int64_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) dst[o++] = keys[src[b]] < keys[src[a]] ? src[b++] : src[a++];
            while (a < mid) dst[o++] = src[a++];
            while (b < hi) dst[o++] = src[b++];
        }
        int64_t* t = src; src = dst; dst = t;
    }
    if (src != perm) memcpy(perm, src, sizeof(int64_t) * (size_t)n);
    free(tmp);
}

/* ------------------------------------------------------------------------
 * Build — torchbvh/csrc/bvh_build.cu:679-721 (entry), :238-359 (node
 * AABBs: leaf = point box; parent = min/max of real children; a parent
 * whose right child is virtual copies its left child), :361-398
 * (traversal arrays).  One cloud of n points.
 * ---------------------------------------------------------------------- */
/* Node AABBs and traversal arrays over `sorted` leaves whose boxes are
 * leaf_boxes[sorted[j]] (2D floats each, by original index). */
static void build_nodes(const float* leaf_boxes, int n, int D, const int64_t* sorted, float* node_aabbs,
                        int32_t* left, int32_t* right, int32_t* leaf) {
    const int L = orc_leaf_level(n);
    const int W = 2 * D;
    const int first_leaf = (1 << L) - 1;
    for (int level = L; level >= 0; --level) {
        const int first = (1 << level) - 1;
        const int real = real_nodes_at_level(n, level);
        for (int j = 0; j < real; ++j) {
            const int i = first + j;
            float* box = node_aabbs + (int64_t)orc_memory_index(n, i) * W;
            const int row = orc_memory_index(n, i);
            if (level == L) {
                memcpy(box, leaf_boxes + sorted[i - first_leaf] * W, sizeof(float) * (size_t)W);
                left[row] = -1;
                right[row] = -1;
                leaf[row] = i - first_leaf;
            } else {
                const int lc = 2 * i + 1, rc = 2 * i + 2;
                const float* a = node_aabbs + (int64_t)orc_memory_index(n, lc) * W;
                if (orc_is_virtual(n, rc)) {
                    memcpy(box, a, sizeof(float) * (size_t)W);
                    right[row] = -1;
                } else {
                    const float* b = node_aabbs + (int64_t)orc_memory_index(n, rc) * W;
                    for (int d = 0; d < D; ++d) {
                        box[d] = fminf(a[d], b[d]);
                        box[D + d] = fmaxf(a[D + d], b[D + d]);
                    }
                    right[row] = orc_memory_index(n, rc);
                }
                left[row] = orc_memory_index(n, lc);
                leaf[row] = -1;
            }
        }
    }
}

void orc_build(const float* pts, int n, int D, float* node_aabbs, int64_t* sorted,
               float* scene_lo, float* scene_hi, int32_t* left, int32_t* right, int32_t* leaf) {
    orc_bounds(pts, n, D, scene_lo, scene_hi);
    uint32_t* codes = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    orc_morton_codes(pts, n, D, scene_lo, scene_hi, codes);
    orc_stable_argsort(codes, n, sorted);
    free(codes);
    /* leaf = the point's degenerate box */
    float* boxes = (float*)malloc(sizeof(float) * (size_t)n * 2 * D);
    for (int j = 0; j < n; ++j)
        for (int d = 0; d < D; ++d) boxes[(int64_t)j * 2 * D + d] = boxes[(int64_t)j * 2 * D + D + d] = pts[(int64_t)j * D + d];
    build_nodes(boxes, n, D, sorted, node_aabbs, left, right, leaf);
    free(boxes);
}

/* ------------------------------------------------------------------------
 * Primitive build — torchbvh/csrc/bvh_build.cu:61-93 (per primitive: vertex
 * min/max box and centre = sequential vertex sum / V), :789-791 (scene
 * bounds = min of the boxes' lower corners, max of their upper corners),
 * :793-800 (Morton codes of the centres, sorted; here stably, ties by
 * primitive index), :801-811 (node AABBs with the primitive boxes as
 * leaves).  One sample of n primitives of V vertices in D dimensions.
 * ---------------------------------------------------------------------- */
void orc_build_primitives(const float* prims, int n, int V, int D, float* node_aabbs, int64_t* sorted,
                          float* scene_lo, float* scene_hi, int32_t* left, int32_t* right, int32_t* leaf,
                          float* centers_out) {
    const int W = 2 * D;
    float* boxes = (float*)malloc(sizeof(float) * (size_t)n * W);
    for (int d = 0; d < D; ++d) { scene_lo[d] = INFINITY; scene_hi[d] = -INFINITY; }
    for (int j = 0; j < n; ++j) {
        const float* p = prims + (int64_t)j * V * D;
        for (int d = 0; d < D; ++d) {
            float lo = p[d], hi = p[d], sum = p[d];
            for (int v = 1; v < V; ++v) {
                const float x = p[v * D + d];
                lo = fminf(lo, x);
                hi = fmaxf(hi, x);
                sum += x;
            }
            centers_out[(int64_t)j * D + d] = sum / (float)V;
            boxes[(int64_t)j * W + d] = lo;
            boxes[(int64_t)j * W + D + d] = hi;
            scene_lo[d] = fminf(scene_lo[d], lo);
            scene_hi[d] = fmaxf(scene_hi[d], hi);
        }
    }
    uint32_t* codes = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    orc_morton_codes(centers_out, n, D, scene_lo, scene_hi, codes);
    orc_stable_argsort(codes, n, sorted);
    free(codes);
    build_nodes(boxes, n, D, sorted, node_aabbs, left, right, leaf);
    free(boxes);
}

/* ------------------------------------------------------------------------
 * Distances — torchbvh/csrc/geometry.cuh:3-18:
 *   delta_d = max(lo - q, max(0, q - hi)),  dist = sum delta_d^2
 * with the FMA contraction of `dist += delta * delta`:
 *   fma(d2, d2, fma(d1, d1, d0 * d0)).
 * ---------------------------------------------------------------------- */
static float box_dist(const float* q, const float* box, int D) {
    float s = 0.0f;
    for (int d = 0; d < D; ++d) {
        const float delta = fmaxf(box[d] - q[d], fmaxf(0.0f, q[d] - box[D + d]));
        s = d == 0 ? delta * delta : fmaf(delta, delta, s);
    }
    return s;
}
static float point_dist(const float* q, const float* p, int D) {
    float s = 0.0f;
    for (int d = 0; d < D; ++d) {
        const float delta = fmaxf(p[d] - q[d], fmaxf(0.0f, q[d] - p[d]));
        s = d == 0 ? delta * delta : fmaf(delta, delta, s);
    }
    return s;
}
float orc_point_dist(const float* q, const float* p, int D) { return point_dist(q, p, D); }

/* Ascending list of K (dist, idx); empty slots are (FLT_MAX, -1)
 * (knn_query.cu:13, :80-86).  Accept a candidate iff dist < FLT_MAX and
 * (dist, idx) < the last entry lexicographically. */
static void list_init(float* dist, int64_t* idx, int K) {
    for (int i = 0; i < K; ++i) { dist[i] = FLT_MAX; idx[i] = -1; }
}
static int lex_less(float da, int64_t ia, float db, int64_t ib) {
    return da < db || (da == db && (uint32_t)ia < (uint32_t)ib);
}
static void list_insert(float* dist, int64_t* idx, int K, float d, int64_t i) {
    if (!(d < FLT_MAX) || !lex_less(d, i, dist[K - 1], idx[K - 1])) return;
    int at = K - 1;
    while (at > 0 && lex_less(d, i, dist[at - 1], idx[at - 1])) {
        dist[at] = dist[at - 1];
        idx[at] = idx[at - 1];
        --at;
    }
    dist[at] = d;
    idx[at] = i;
}

/* Brute force over all n points (the reference tests' oracle,
 * tests/test_knn.py:10-12, with the lexicographic tie rule). */
void orc_knn_brute(const float* pts, int64_t n, const float* qs, int64_t m, int D, int K,
                   int64_t* out_idx, float* out_dist) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t qi = 0; qi < m; ++qi) {
        float* dist = out_dist + qi * K;
        int64_t* idx = out_idx + qi * K;
        list_init(dist, idx, K);
        const float* q = qs + qi * D;
        for (int64_t j = 0; j < n; ++j) {
            const float d = point_dist(q, pts + j * D, D);
            if (d <= dist[K - 1]) list_insert(dist, idx, K, d, j);
        }
    }
}

/* Branch-and-bound over the built tree — restates the traversal of
 * torchbvh/csrc/knn_query.cu:47-154 (root distance first; both real
 * children evaluated, near first with ties to the left; far child pushed
 * with its cached distance if <= the k-th distance; popped nodes re-tested)
 * with the lexicographic list above. */
void orc_knn_bvh(const float* node_aabbs, const int64_t* sorted, int n, const float* qs,
                 int64_t m, int D, int K, int64_t* out_idx, float* out_dist) {
    const int L = orc_leaf_level(n);
    const int first_leaf = (1 << L) - 1;
    const int W = 2 * D;
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t qi = 0; qi < m; ++qi) {
        float* dist = out_dist + qi * K;
        int64_t* idx = out_idx + qi * K;
        list_init(dist, idx, K);
        const float* q = qs + qi * D;
        int stack_node[64];
        float stack_dist[64];
        int sp = 0;
        int node = 0;
        float nd = box_dist(q, node_aabbs, D);
        for (;;) {
            const float worst = dist[K - 1];
            int descended = 0;
            if (nd <= worst) {
                if (node >= first_leaf) {
                    list_insert(dist, idx, K, nd, sorted[node - first_leaf]);
                } else {
                    const int lc = 2 * node + 1, rc = 2 * node + 2;
                    const int rreal = !orc_is_virtual(n, rc);
                    const float ld = box_dist(q, node_aabbs + (int64_t)orc_memory_index(n, lc) * W, D);
                    const float rd = rreal
                        ? box_dist(q, node_aabbs + (int64_t)orc_memory_index(n, rc) * W, D)
                        : FLT_MAX;
                    const int left_near = ld <= rd;
                    const int near = left_near ? lc : rc, far = left_near ? rc : lc;
                    const float near_d = left_near ? ld : rd, far_d = left_near ? rd : ld;
                    const int far_real = left_near ? rreal : 1;
                    const int near_real = left_near ? 1 : rreal;
                    if (far_real && far_d <= worst) {
                        stack_node[sp] = far;
                        stack_dist[sp] = far_d;
                        ++sp;
                    }
                    if (near_real && near_d <= worst) {
                        node = near;
                        nd = near_d;
                        descended = 1;
                    }
                }
            }
            if (descended) continue;
            if (sp == 0) break;
            --sp;
            node = stack_node[sp];
            nd = stack_dist[sp];
        }
    }
}

/* Fused-chain distance of every (query row, returned index) pair: lets tests
 * check that each returned distance is exactly the distance of the returned
 * point (negative indices give FLT_MAX, the empty-slot value). */
void orc_pair_distances(const float* pts, const float* qs, const int64_t* idx, int64_t m,
                        int D, int K, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        for (int j = 0; j < K; ++j) {
            const int64_t i = idx[r * K + j];
            out[r * K + j] = i < 0 ? FLT_MAX : point_dist(qs + r * D, pts + i * D, D);
        }
    }
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int t) {
#ifdef _OPENMP
    if (t > 0) omp_set_num_threads(t);
#else
    (void)t;
#endif
}
