/* CPU restatement of the reference FPS path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
 * load this library, and only as the checker or the timed CPU baseline.  The
 * product path (ns_fps_amd) never links, loads or calls it.
 *
 * All entry points are plain C over flat arrays so ctypes can call them.
 * Status: 0 = ok, negative = invalid argument.
 */
#ifndef NSFPS_ORACLE_H
#define NSFPS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Work census of one FPS run under the reference's candidate rule
 * (src/yuezu_fps.cpp:560-597 cube of cells -> buckets; every point of every
 * candidate bucket is updated, src/yuezu_fps.cpp:495-513).  "leaves" counts
 * the reference's 16-point MortonBlocks (src/yuezu_fps.h:20-22, 122-140). */
typedef struct {
  uint64_t iterations;      /* loop iterations that performed an update */
  uint64_t cand_cells;      /* in-grid cube cells summed over iterations */
  uint64_t cand_points;     /* points of candidate buckets, summed */
  uint64_t cand_leaves;     /* 16-point leaves of candidate buckets, summed */
  uint64_t first_pass_points;
  uint64_t first_pass_leaves;
  uint64_t audit_violations; /* points outside the candidates whose distance
                                would have lowered their cache (audit mode) */
} orc_census;

/* make_range derived fields (src/yuezu_fps.cpp:136-161 and :7-40).
 * luts gets the x, y and z LUTs concatenated; returns the entry count or -1. */
int orc_range(const float *bounds6, const uint32_t *blocks3, float *inv_bs3,
              float *block_size3, uint32_t *bits3, uint32_t *luts,
              uint32_t lut_cap);

/* compute_bbox bounds (src/yuezu_fps.cpp:648-670), +/- BOUNDARY_EPS. */
int orc_bbox(const float *xyz, uint64_t n, float *bounds6);

/* Cell indices (ix,iy,iz per point) and Morton code per point
 * (src/yuezu_fps.cpp:170-199). */
int orc_cell_code(const float *xyz, uint64_t n, const float *bounds6,
                  const uint32_t *blocks3, uint32_t *cells3, uint32_t *codes);

/* Logical layout: bucket (= code % total_blocks) per point, and the logical
 * order (original indices sorted stably by bucket; src/yuezu_fps.cpp:277-283,
 * 411-416, 431-438). */
int orc_layout(const float *xyz, uint64_t n, const float *bounds6,
               const uint32_t *blocks3, uint32_t *bucket, uint32_t *order);

/* FPS under the reference rule.  bounds6 == NULL selects compute_bbox.
 * out receives up to m original indices; *out_len the count (early stop when
 * the maximum min-distance is <= 0).  census may be NULL.  audit != 0 also
 * runs the full update check each iteration (O(N) per iteration). */
int orc_fps(const float *xyz, uint64_t n, uint64_t m, const float *bounds6,
            const uint32_t *blocks3, int32_t *out, uint64_t *out_len,
            orc_census *census, int audit);

/* Per-iteration record of the same run: selected maximum, candidate points
 * and candidate 16-point leaves (entry 0: the first full pass).  Arrays hold
 * m entries; cand_leaves may be NULL. */
int orc_fps_trace(const float *xyz, uint64_t n, uint64_t m,
                  const float *bounds6, const uint32_t *blocks3, int32_t *out,
                  uint64_t *out_len, float *max_dist, uint32_t *cand_points,
                  uint32_t *cand_leaves);

/* Naive O(N*M) FPS (eval/src_cpu/compare_cpu_test.cpp:10-57 shape):
 * start at row 0, cache initialised to FLT_MAX, full update every iteration,
 * stop when the maximum is <= 0.  tie_mode 0: ties go to the lowest original
 * index.  tie_mode 1: ties go to the lowest logical key (bucket, index) of
 * the given range (bounds6 == NULL -> compute_bbox).  max_iters limits the
 * number of loop iterations (0 = no limit) so a bounded sample can be timed. */
int orc_fps_naive(const float *xyz, uint64_t n, uint64_t m,
                  const float *bounds6, const uint32_t *blocks3, int tie_mode,
                  int32_t *out, uint64_t *out_len, uint64_t max_iters);

/* The naive FPS with ties to the lowest original index, each iteration's
 * update and argmax split over `threads` OpenMP threads (0 = the OpenMP
 * default): every thread scans a contiguous range in index order and the
 * range maxima merge by (larger distance, then lower index), which is the
 * leftmost maximum of the whole scan.  The all-cores CPU baseline. */
int orc_fps_naive_mt(const float *xyz, uint64_t n, uint64_t m, int32_t *out,
                     uint64_t *out_len, uint64_t max_iters, int threads);

/* OpenMP threads orc_fps_naive_mt uses for threads = 0. */
int orc_max_threads(void);

/* Grouping after sampling (no counterpart in the reference; PointNet++'s
 * query_ball_point on the FPS distance).  orc_gather_points: out[i] =
 * xyz[idx[i]]; returns 1 if an index lies outside [0, n) (nothing written
 * for it).  orc_ball_query: row j of out (m x nsample) holds the first
 * nsample indices i, in input order, with sqdist(p_i, c_j) < r2; fewer hits
 * repeat the first hit, none gives zeros. */
int orc_gather_points(const float *xyz, uint64_t n, const int32_t *idx, uint64_t m,
                      float *out);
int orc_ball_query(const float *xyz, uint64_t n, const float *centers, uint64_t m,
                   float r2, uint32_t nsample, int32_t *out);

#ifdef __cplusplus
}
#endif

#endif
