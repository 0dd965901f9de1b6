/* CPU restatement of the reference FPS path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker: tests/, __graft_entry__.smoke() and bench.py's
 * CPU-baseline leg load it; the product (ns_fps_amd) never does.
 *
 * It restates src/yuezu_fps.cpp (the reference) in plain C without its data
 * structures: the result depends only on the cell of each point, the input
 * order and the fp32 arithmetic, because every level of the reference's max
 * tree keeps the leftmost maximum (strict '>' from -1: src/yuezu_fps.cpp:257,
 * :339, :365), so the selected point is the leftmost maximum in logical order
 * (bucket ascending, then original index ascending).  Buckets replace the
 * 16-point MortonBlocks and a binary tournament tree replaces the 16-ary
 * CacheBlock tree; neither changes the result.
 *
 * Build with -ffp-contract=off: the squared distance must be
 * fl(fl(fl(dx*dx) + fl(dy*dy)) + fl(dz*dz)), no FMA.
 *
 * Parity pinning (see tests/test_oracle.py): golden vectors written by the
 * reference compiled from its own sources (oracle/_ref), closed-form LUTs,
 * hand-made known answers, and brute-force equivalence with the naive FPS.
 */
#include "nsfps_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define ORC_BOUNDARY_EPS 1e-6f /* src/yuezu_fps.h:43-45 */
#define ORC_LEAF 16u           /* MORTON_BLOCK_SIZE, src/yuezu_fps.h:20-22 */

typedef struct {
  float mn[3], mx[3];
  uint32_t blocks[3];
  float inv_bs[3];
  float bsize[3];
  uint32_t bits[3];
  uint32_t *lut[3];
  uint64_t total;
} orc_rng;

/* _calc_bits, src/yuezu_fps.cpp:45-50 */
static uint32_t calc_bits(uint32_t blocks) {
  uint32_t bits = 0;
  while (bits < 32 && (1u << bits) < blocks)
    ++bits;
  return bits ? bits : 1;
}

/* _compute_bit_positions (src/yuezu_fps.cpp:69-97) fused with
 * _generate_morton_lut (:52-66): the first min(bits) rounds interleave
 * x, y, z; each later round takes x, then y, then z where still present. */
static int build_luts(orc_rng *r) {
  uint32_t pos[3][32];
  uint32_t cnt[3] = {0, 0, 0};
  uint32_t bit = 0;
  uint32_t common = r->bits[0], maxb = r->bits[0];
  for (int a = 1; a < 3; ++a) {
    if (r->bits[a] < common) common = r->bits[a];
    if (r->bits[a] > maxb) maxb = r->bits[a];
  }
  for (uint32_t i = 0; i < common; ++i)
    for (int a = 0; a < 3; ++a)
      pos[a][cnt[a]++] = bit++;
  for (uint32_t i = common; i < maxb; ++i)
    for (int a = 0; a < 3; ++a)
      if (i < r->bits[a])
        pos[a][cnt[a]++] = bit++;
  for (int a = 0; a < 3; ++a) {
    uint32_t count = 1u << r->bits[a];
    r->lut[a] = (uint32_t *)malloc(sizeof(uint32_t) * count);
    if (!r->lut[a]) return -1;
    for (uint32_t v = 0; v < count; ++v) {
      uint32_t code = 0;
      for (uint32_t k = 0; k < r->bits[a]; ++k)
        if (v & (1u << k))
          code |= 1u << pos[a][k];
      r->lut[a][v] = code;
    }
  }
  return 0;
}

/* make_range, src/yuezu_fps.cpp:136-161; block_size_*, :7-11 */
static int rng_init(orc_rng *r, const float *b6, const uint32_t *blocks3) {
  memset(r, 0, sizeof(*r));
  for (int a = 0; a < 3; ++a) {
    if (blocks3[a] == 0 || blocks3[a] > (1u << 20)) return -1;
    r->mn[a] = b6[2 * a];
    r->mx[a] = b6[2 * a + 1];
    r->blocks[a] = blocks3[a];
    r->bsize[a] = (r->mx[a] - r->mn[a]) / (float)blocks3[a];
    r->inv_bs[a] = 1.0f / ((r->mx[a] - r->mn[a]) / (float)blocks3[a]);
    r->bits[a] = calc_bits(blocks3[a]);
  }
  if (r->bits[0] + r->bits[1] + r->bits[2] > 32) return -1;
  r->total = (uint64_t)blocks3[0] * blocks3[1] * blocks3[2];
  return build_luts(r);
}

static void rng_free(orc_rng *r) {
  for (int a = 0; a < 3; ++a) free(r->lut[a]);
}

/* std::min(v, hi) and std::max(lo, v) exactly as <algorithm> defines them. */
static inline float std_min(float a, float b) { return (b < a) ? b : a; }
static inline float std_max(float a, float b) { return (a < b) ? b : a; }

/* Point3D::compute_block_indices, src/yuezu_fps.cpp:170-193 */
static inline uint32_t cell_axis(const orc_rng *r, int a, float v) {
  float c = std_max(r->mn[a], std_min(v, r->mx[a] - ORC_BOUNDARY_EPS));
  uint32_t i = (uint32_t)((c - r->mn[a]) * r->inv_bs[a]);
  return i < r->blocks[a] - 1 ? i : r->blocks[a] - 1;
}

static inline uint32_t code_of(const orc_rng *r, uint32_t ix, uint32_t iy,
                               uint32_t iz) {
  return r->lut[0][ix] | r->lut[1][iy] | r->lut[2][iz];
}

/* squared_distance, src/yuezu_fps.cpp:205-209 (no contraction) */
static inline float sqdist(float px, float py, float pz, float qx, float qy,
                           float qz) {
  float dx = px - qx, dy = py - qy, dz = pz - qz;
  return dx * dx + dy * dy + dz * dz;
}

int orc_range(const float *bounds6, const uint32_t *blocks3, float *inv_bs3,
              float *block_size3, uint32_t *bits3, uint32_t *luts,
              uint32_t lut_cap) {
  orc_rng r;
  if (rng_init(&r, bounds6, blocks3)) { rng_free(&r); return -1; }
  uint64_t total = 0;
  for (int a = 0; a < 3; ++a) {
    inv_bs3[a] = r.inv_bs[a];
    block_size3[a] = r.bsize[a];
    bits3[a] = r.bits[a];
    total += 1ull << r.bits[a];
  }
  if (total > lut_cap) { rng_free(&r); return -1; }
  uint64_t o = 0;
  for (int a = 0; a < 3; ++a)
    for (uint32_t v = 0; v < (1u << r.bits[a]); ++v)
      luts[o++] = r.lut[a][v];
  rng_free(&r);
  return (int)total;
}

/* compute_bbox, src/yuezu_fps.cpp:648-670 (empty cloud -> [0,1]^3) */
int orc_bbox(const float *xyz, uint64_t n, float *b6) {
  if (n == 0) {
    b6[0] = 0; b6[1] = 1; b6[2] = 0; b6[3] = 1; b6[4] = 0; b6[5] = 1;
    return 0;
  }
  float mn[3] = {xyz[0], xyz[1], xyz[2]}, mx[3] = {xyz[0], xyz[1], xyz[2]};
  for (uint64_t i = 0; i < n; ++i)
    for (int a = 0; a < 3; ++a) {
      mn[a] = std_min(mn[a], xyz[3 * i + a]);
      mx[a] = std_max(mx[a], xyz[3 * i + a]);
    }
  for (int a = 0; a < 3; ++a) {
    b6[2 * a] = mn[a] - ORC_BOUNDARY_EPS;
    b6[2 * a + 1] = mx[a] + ORC_BOUNDARY_EPS;
  }
  return 0;
}

int orc_cell_code(const float *xyz, uint64_t n, const float *bounds6,
                  const uint32_t *blocks3, uint32_t *cells3, uint32_t *codes) {
  orc_rng r;
  if (rng_init(&r, bounds6, blocks3)) { rng_free(&r); return -1; }
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t c[3];
    for (int a = 0; a < 3; ++a) c[a] = cell_axis(&r, a, xyz[3 * i + a]);
    cells3[3 * i] = c[0];
    cells3[3 * i + 1] = c[1];
    cells3[3 * i + 2] = c[2];
    codes[i] = code_of(&r, c[0], c[1], c[2]);
  }
  rng_free(&r);
  return 0;
}

/* Stable counting sort by bucket (= code % total_blocks,
 * src/yuezu_fps.cpp:411-416).  start has total+1 entries. */
static int make_layout(const orc_rng *r, const float *xyz, uint64_t n,
                       uint32_t *bucket, uint32_t *order, uint64_t *start) {
  memset(start, 0, sizeof(uint64_t) * (r->total + 1));
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t ix = cell_axis(r, 0, xyz[3 * i]);
    uint32_t iy = cell_axis(r, 1, xyz[3 * i + 1]);
    uint32_t iz = cell_axis(r, 2, xyz[3 * i + 2]);
    uint32_t b = (uint32_t)(code_of(r, ix, iy, iz) % r->total);
    bucket[i] = b;
    start[b + 1]++;
  }
  for (uint64_t b = 0; b < r->total; ++b) start[b + 1] += start[b];
  uint64_t *fill = (uint64_t *)malloc(sizeof(uint64_t) * r->total);
  if (!fill) return -1;
  memcpy(fill, start, sizeof(uint64_t) * r->total);
  for (uint64_t i = 0; i < n; ++i) order[fill[bucket[i]]++] = (uint32_t)i;
  free(fill);
  return 0;
}

int orc_layout(const float *xyz, uint64_t n, const float *bounds6,
               const uint32_t *blocks3, uint32_t *bucket, uint32_t *order) {
  orc_rng r;
  if (rng_init(&r, bounds6, blocks3)) { rng_free(&r); return -1; }
  uint64_t *start = (uint64_t *)malloc(sizeof(uint64_t) * (r.total + 1));
  int rc = start ? make_layout(&r, xyz, n, bucket, order, start) : -1;
  free(start);
  rng_free(&r);
  return rc;
}

/* Tournament tree over buckets: node = (value, logical position); the larger
 * value wins, equal values go to the smaller position (leftmost). */
typedef struct {
  float v;
  uint32_t pos;
} orc_key;

static inline orc_key key_better(orc_key a, orc_key b) {
  if (b.v > a.v || (b.v == a.v && b.pos < a.pos)) return b;
  return a;
}

typedef struct {
  orc_rng r;
  uint64_t n;
  uint32_t *order; /* logical position -> original index */
  uint64_t *start; /* bucket -> first logical position */
  float *X, *Y, *Z, *C;
  orc_key *tree;
  uint64_t P;
  uint32_t *stamp; /* bucket -> last iteration it was a candidate (audit) */
} orc_state;

static void st_free(orc_state *s) {
  free(s->order); free(s->start); free(s->X); free(s->Y); free(s->Z);
  free(s->C); free(s->tree); free(s->stamp);
  rng_free(&s->r);
}

/* Leftmost maximum of one bucket (MortonBlock::update_distance's max,
 * src/yuezu_fps.cpp:245-264, over the whole bucket). */
static orc_key bucket_max(const orc_state *s, uint64_t b) {
  orc_key k = {-1.0f, UINT32_MAX};
  for (uint64_t i = s->start[b]; i < s->start[b + 1]; ++i)
    if (s->C[i] > k.v) { k.v = s->C[i]; k.pos = (uint32_t)i; }
  return k;
}

static void tree_set(orc_state *s, uint64_t b, orc_key k) {
  uint64_t i = s->P + b;
  s->tree[i] = k;
  for (i >>= 1; i >= 1; i >>= 1)
    s->tree[i] = key_better(s->tree[2 * i], s->tree[2 * i + 1]);
}

static void update_bucket(orc_state *s, uint64_t b, float qx, float qy,
                          float qz) {
  for (uint64_t i = s->start[b]; i < s->start[b + 1]; ++i) {
    float d = sqdist(s->X[i], s->Y[i], s->Z[i], qx, qy, qz);
    if (d < s->C[i]) s->C[i] = d;
  }
  tree_set(s, b, bucket_max(s, b));
}

/* Cube half-widths of get_morton_codes_in_range (src/yuezu_fps.cpp:564-570):
 * n = (int)ceil(sqrtf(D) / block_size).  Values at or beyond the grid size
 * cover the whole grid; they are clamped there (the reference aborts in
 * vector::reserve when the cube is astronomically large). */
static inline int cube_half(float D, float bsize, uint32_t blocks) {
  if (D < 0.0f) D = 0.0f;
  float rad = sqrtf(D);
  float f = ceilf(rad / bsize);
  if (!(f < (float)blocks)) return (int)blocks;
  return (int)f;
}

static int fps_core(const float *xyz, uint64_t n, uint64_t m,
                    const float *bounds6, const uint32_t *blocks3,
                    int32_t *out, uint64_t *out_len, orc_census *census,
                    int audit, float *max_dist, uint32_t *cand_trace,
                    uint32_t *leaf_trace) {
  *out_len = 0;
  if (census) memset(census, 0, sizeof(*census));
  if (n == 0 || m == 0) return 0; /* src/yuezu_fps.cpp:678-680 */
  if (n > 0x7fffffffull) return -2;
  if (m >= n) {                   /* src/yuezu_fps.cpp:681-688 */
    for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)i;
    *out_len = n;
    return 0;
  }
  float bb[6];
  if (!bounds6) { orc_bbox(xyz, n, bb); bounds6 = bb; }
  orc_state s;
  memset(&s, 0, sizeof(s));
  if (rng_init(&s.r, bounds6, blocks3)) { st_free(&s); return -1; }
  s.n = n;
  uint64_t T = s.r.total;
  uint32_t *bucket = (uint32_t *)malloc(sizeof(uint32_t) * n);
  s.order = (uint32_t *)malloc(sizeof(uint32_t) * n);
  s.start = (uint64_t *)malloc(sizeof(uint64_t) * (T + 1));
  s.X = (float *)malloc(sizeof(float) * n);
  s.Y = (float *)malloc(sizeof(float) * n);
  s.Z = (float *)malloc(sizeof(float) * n);
  s.C = (float *)malloc(sizeof(float) * n);
  for (s.P = 1; s.P < T; s.P <<= 1) {}
  s.tree = (orc_key *)malloc(sizeof(orc_key) * 2 * s.P);
  s.stamp = (uint32_t *)calloc(T, sizeof(uint32_t));
  if (!bucket || !s.order || !s.start || !s.X || !s.Y || !s.Z || !s.C ||
      !s.tree || !s.stamp || make_layout(&s.r, xyz, n, bucket, s.order, s.start)) {
    free(bucket);
    st_free(&s);
    return -3;
  }
  free(bucket);
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t o = s.order[i];
    s.X[i] = xyz[3 * o];
    s.Y[i] = xyz[3 * o + 1];
    s.Z[i] = xyz[3 * o + 2];
    s.C[i] = FLT_MAX; /* src/yuezu_fps.cpp:215-217, :223 */
  }
  for (uint64_t i = 0; i < 2 * s.P; ++i) {
    s.tree[i].v = -1.0f;
    s.tree[i].pos = UINT32_MAX;
  }
  /* First pass against row 0 (src/yuezu_fps.cpp:696-697, :431-438). */
  const float fx = xyz[0], fy = xyz[1], fz = xyz[2];
  for (uint64_t b = 0; b < T; ++b) {
    for (uint64_t i = s.start[b]; i < s.start[b + 1]; ++i) {
      float d = sqdist(s.X[i], s.Y[i], s.Z[i], fx, fy, fz);
      if (d < s.C[i]) s.C[i] = d;
    }
    s.tree[s.P + b] = bucket_max(&s, b);
    if (census) {
      uint64_t c = s.start[b + 1] - s.start[b];
      census->first_pass_points += c;
      census->first_pass_leaves += (c + ORC_LEAF - 1) / ORC_LEAF;
    }
  }
  for (uint64_t i = s.P - 1; i >= 1; --i)
    s.tree[i] = key_better(s.tree[2 * i], s.tree[2 * i + 1]);

  out[0] = 0;
  uint64_t len = 1;
  if (max_dist) max_dist[0] = INFINITY;
  if (cand_trace) cand_trace[0] = (uint32_t)n;
  if (leaf_trace) {
    uint64_t l0 = 0;
    for (uint64_t b = 0; b < T; ++b) l0 += (s.start[b + 1] - s.start[b] + ORC_LEAF - 1) / ORC_LEAF;
    leaf_trace[0] = (uint32_t)l0;
  }
  for (uint64_t it = 1; it < m; ++it) {
    orc_key top = s.tree[1];
    float D = top.v < 0.0f ? 0.0f : top.v;
    if (D <= 0.0f) break; /* src/yuezu_fps.cpp:705-706 */
    uint64_t p = top.pos;
    out[len++] = (int32_t)s.order[p];
    if (max_dist) max_dist[it] = D;
    const float qx = s.X[p], qy = s.Y[p], qz = s.Z[p];
    /* get_morton_codes_in_range, src/yuezu_fps.cpp:560-597 */
    int h[3];
    uint32_t qc[3];
    const float q3[3] = {qx, qy, qz};
    for (int a = 0; a < 3; ++a) {
      h[a] = cube_half(D, s.r.bsize[a], s.r.blocks[a]);
      qc[a] = cell_axis(&s.r, a, q3[a]);
    }
    int lo[3], hi[3];
    for (int a = 0; a < 3; ++a) {
      lo[a] = (int)qc[a] - h[a] < 0 ? 0 : (int)qc[a] - h[a];
      hi[a] = (int)qc[a] + h[a] > (int)s.r.blocks[a] - 1 ? (int)s.r.blocks[a] - 1
                                                          : (int)qc[a] + h[a];
    }
    uint64_t cand_pts = 0, cand_lv = 0;
    for (int bz = lo[2]; bz <= hi[2]; ++bz)
      for (int by = lo[1]; by <= hi[1]; ++by)
        for (int bx = lo[0]; bx <= hi[0]; ++bx) {
          uint64_t b = code_of(&s.r, (uint32_t)bx, (uint32_t)by, (uint32_t)bz) % T;
          uint64_t c = s.start[b + 1] - s.start[b];
          cand_pts += c;
          cand_lv += (c + ORC_LEAF - 1) / ORC_LEAF;
          if (census) {
            census->cand_cells++;
            census->cand_points += c;
            census->cand_leaves += (c + ORC_LEAF - 1) / ORC_LEAF;
          }
          if (audit) s.stamp[b] = (uint32_t)it;
          if (c) update_bucket(&s, b, qx, qy, qz);
        }
    if (census) census->iterations++;
    if (cand_trace) cand_trace[it] = (uint32_t)(cand_pts > UINT32_MAX ? UINT32_MAX : cand_pts);
    if (leaf_trace) leaf_trace[it] = (uint32_t)(cand_lv > UINT32_MAX ? UINT32_MAX : cand_lv);
    if (audit && census) {
      for (uint64_t b = 0; b < T; ++b) {
        if (s.stamp[b] == (uint32_t)it) continue;
        for (uint64_t i = s.start[b]; i < s.start[b + 1]; ++i)
          if (sqdist(s.X[i], s.Y[i], s.Z[i], qx, qy, qz) < s.C[i])
            census->audit_violations++;
      }
    }
  }
  *out_len = len;
  st_free(&s);
  return 0;
}

int orc_fps(const float *xyz, uint64_t n, uint64_t m, const float *bounds6,
            const uint32_t *blocks3, int32_t *out, uint64_t *out_len,
            orc_census *census, int audit) {
  return fps_core(xyz, n, m, bounds6, blocks3, out, out_len, census, audit,
                  NULL, NULL, NULL);
}

int orc_fps_trace(const float *xyz, uint64_t n, uint64_t m,
                  const float *bounds6, const uint32_t *blocks3, int32_t *out,
                  uint64_t *out_len, float *max_dist, uint32_t *cand_points,
                  uint32_t *cand_leaves) {
  return fps_core(xyz, n, m, bounds6, blocks3, out, out_len, NULL, 0, max_dist,
                  cand_points, cand_leaves);
}

int orc_fps_naive(const float *xyz, uint64_t n, uint64_t m,
                  const float *bounds6, const uint32_t *blocks3, int tie_mode,
                  int32_t *out, uint64_t *out_len, uint64_t max_iters) {
  *out_len = 0;
  if (n == 0 || m == 0) return 0;
  if (n > 0x7fffffffull) return -2;
  if (m >= n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)i;
    *out_len = n;
    return 0;
  }
  uint32_t *scan = (uint32_t *)malloc(sizeof(uint32_t) * n); /* argmax order */
  float *C = (float *)malloc(sizeof(float) * n);
  if (!scan || !C) { free(scan); free(C); return -3; }
  if (tie_mode == 1) {
    float bb[6];
    if (!bounds6) { orc_bbox(xyz, n, bb); bounds6 = bb; }
    orc_rng r;
    uint32_t *bucket = (uint32_t *)malloc(sizeof(uint32_t) * n);
    uint64_t *start = NULL;
    int rc = rng_init(&r, bounds6, blocks3);
    if (!rc) {
      start = (uint64_t *)malloc(sizeof(uint64_t) * (r.total + 1));
      rc = (bucket && start) ? make_layout(&r, xyz, n, bucket, scan, start) : -3;
    }
    free(bucket); free(start); rng_free(&r);
    if (rc) { free(scan); free(C); return rc; }
  } else {
    for (uint64_t i = 0; i < n; ++i) scan[i] = (uint32_t)i;
  }
  for (uint64_t i = 0; i < n; ++i) C[i] = FLT_MAX;
  out[0] = 0;
  uint64_t len = 1, last = 0;
  for (uint64_t it = 1; it < m; ++it) {
    if (max_iters && it > max_iters) break;
    const float qx = xyz[3 * last], qy = xyz[3 * last + 1], qz = xyz[3 * last + 2];
    for (uint64_t j = 0; j < n; ++j) {
      float d = sqdist(xyz[3 * j], xyz[3 * j + 1], xyz[3 * j + 2], qx, qy, qz);
      if (d < C[j]) C[j] = d;
    }
    float best = -1.0f;
    uint64_t bi = 0;
    for (uint64_t k = 0; k < n; ++k) {
      uint32_t j = scan[k];
      if (C[j] > best) { best = C[j]; bi = j; }
    }
    if (best <= 0.0f) break;
    out[len++] = (int32_t)bi;
    last = bi;
  }
  *out_len = len;
  free(scan);
  free(C);
  return 0;
}

int orc_max_threads(void) { return omp_get_max_threads(); }

int orc_fps_naive_mt(const float *xyz, uint64_t n, uint64_t m, int32_t *out,
                     uint64_t *out_len, uint64_t max_iters, int threads) {
  *out_len = 0;
  if (n == 0 || m == 0) return 0;
  if (n > 0x7fffffffull) return -2;
  if (m >= n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)i;
    *out_len = n;
    return 0;
  }
  float *C = (float *)malloc(sizeof(float) * n);
  if (!C) return -3;
  const int nt = threads > 0 ? threads : omp_get_max_threads();
  for (uint64_t i = 0; i < n; ++i) C[i] = FLT_MAX;
  out[0] = 0;
  uint64_t len = 1, last = 0;
  for (uint64_t it = 1; it < m; ++it) {
    if (max_iters && it > max_iters) break;
    const float qx = xyz[3 * last], qy = xyz[3 * last + 1], qz = xyz[3 * last + 2];
    float gbest = -1.0f;
    int64_t gbi = 0;
#pragma omp parallel num_threads(nt)
    {
      float best = -1.0f;
      int64_t bi = 0;
#pragma omp for schedule(static) nowait
      for (int64_t j = 0; j < (int64_t)n; ++j) {
        const float d = sqdist(xyz[3 * j], xyz[3 * j + 1], xyz[3 * j + 2], qx, qy, qz);
        if (d < C[j]) C[j] = d;
        if (C[j] > best) {
          best = C[j];
          bi = j;
        }
      }
#pragma omp critical
      {
        if (best > gbest || (best == gbest && bi < gbi)) {
          gbest = best;
          gbi = bi;
        }
      }
    }
    if (gbest <= 0.0f) break;
    out[len++] = (int32_t)gbi;
    last = (uint64_t)gbi;
  }
  *out_len = len;
  free(C);
  return 0;
}

/* ---- grouping after sampling: a literal scan per center ------------------ */

int orc_gather_points(const float *xyz, uint64_t n, const int32_t *idx, uint64_t m,
                      float *out) {
  int bad = 0;
  for (uint64_t i = 0; i < m; ++i) {
    if (idx[i] < 0 || (uint64_t)idx[i] >= n) {
      bad = 1;
      continue;
    }
    for (int a = 0; a < 3; ++a) out[3 * i + a] = xyz[3 * (uint64_t)idx[i] + a];
  }
  return bad;
}

int orc_ball_query(const float *xyz, uint64_t n, const float *centers, uint64_t m,
                   float r2, uint32_t nsample, int32_t *out) {
  for (uint64_t j = 0; j < m; ++j) {
    int32_t *row = out + j * nsample;
    uint32_t cnt = 0;
    for (uint32_t k = 0; k < nsample; ++k) row[k] = 0;
    for (uint64_t i = 0; i < n && cnt < nsample; ++i) {
      const float *p = xyz + 3 * i, *c = centers + 3 * j;
      float dx = p[0] - c[0], dy = p[1] - c[1], dz = p[2] - c[2];
      float s = dx * dx + dy * dy;
      float d2 = s + dz * dz;
      if (d2 < r2) {
        if (cnt == 0)
          for (uint32_t k = 0; k < nsample; ++k) row[k] = (int32_t)i;
        row[cnt++] = (int32_t)i;
      }
    }
  }
  return 0;
}
