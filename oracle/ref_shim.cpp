// C entry points over the reference's own C++ library, compiled together with
// src/yuezu_fps.cpp from the reference tree by oracle/Makefile into
// oracle/_ref/.  This file is ours; the reference sources are compiled where
// they lie and never copied.  The built library is a checker and a CPU
// baseline only: tests and the benchmark's CPU leg load it, nothing else does.
//
// Entry points mirror the reference surface:
//   ref_fps          -> yuezu_fps()       (src/yuezu_fps.h:211-212)
//   ref_fps_bbox     -> compute_bbox() + yuezu_fps()   (src/yuezu_fps.cpp:648-670)
//   ref_range        -> make_range()      (src/yuezu_fps.cpp:136-161)
//   ref_cell_code    -> Point3D::compute_morton_code() (src/yuezu_fps.cpp:195-199)
#include "yuezu_fps.h"

#include <cstdint>
#include <cstring>
#include <vector>

static std::vector<Point3D> to_points(const float *xyz, uint64_t n) {
  std::vector<Point3D> pts;
  pts.reserve(n);
  for (uint64_t i = 0; i < n; ++i)
    pts.emplace_back(xyz[3 * i], xyz[3 * i + 1], xyz[3 * i + 2], (size_t)i);
  return pts;
}

extern "C" {

int ref_fps(const float *xyz, uint64_t n, uint64_t m, const float *bounds6,
            const uint32_t *blocks3, int64_t *out, uint64_t *out_len) {
  std::vector<Point3D> pts = to_points(xyz, n);
  SpaceRange r = make_range(bounds6[0], bounds6[1], bounds6[2], bounds6[3],
                            bounds6[4], bounds6[5], blocks3[0], blocks3[1],
                            blocks3[2]);
  std::vector<size_t> idx = yuezu_fps(pts, m, r);
  for (size_t i = 0; i < idx.size(); ++i)
    out[i] = (int64_t)idx[i];
  *out_len = idx.size();
  return 0;
}

int ref_fps_bbox(const float *xyz, uint64_t n, uint64_t m,
                 const uint32_t *blocks3, int64_t *out, uint64_t *out_len) {
  std::vector<Point3D> pts = to_points(xyz, n);
  SpaceRange r = compute_bbox(pts, blocks3[0], blocks3[1], blocks3[2]);
  std::vector<size_t> idx = yuezu_fps(pts, m, r);
  for (size_t i = 0; i < idx.size(); ++i)
    out[i] = (int64_t)idx[i];
  *out_len = idx.size();
  return 0;
}

// Derived range fields: inv_bs[3], block_size[3], bits[3], then the three
// LUTs concatenated into luts (capacity lut_cap entries).  Returns the number
// of LUT entries written, or -1 if lut_cap is too small.
int ref_range(const float *bounds6, const uint32_t *blocks3, float *inv_bs3,
              float *block_size3, uint32_t *bits3, uint32_t *luts,
              uint32_t lut_cap) {
  SpaceRange r = make_range(bounds6[0], bounds6[1], bounds6[2], bounds6[3],
                            bounds6[4], bounds6[5], blocks3[0], blocks3[1],
                            blocks3[2]);
  inv_bs3[0] = r.inv_bs_x;
  inv_bs3[1] = r.inv_bs_y;
  inv_bs3[2] = r.inv_bs_z;
  block_size3[0] = r.block_size_x();
  block_size3[1] = r.block_size_y();
  block_size3[2] = r.block_size_z();
  bits3[0] = r.x_bits();
  bits3[1] = r.y_bits();
  bits3[2] = r.z_bits();
  size_t total = r.x_lut_.size() + r.y_lut_.size() + r.z_lut_.size();
  if (total > lut_cap)
    return -1;
  size_t o = 0;
  for (uint32_t v : r.x_lut_) luts[o++] = v;
  for (uint32_t v : r.y_lut_) luts[o++] = v;
  for (uint32_t v : r.z_lut_) luts[o++] = v;
  return (int)total;
}

// Cell indices and Morton code per point (before the "% total_blocks" of the
// bucket table).  cells3 gets ix, iy, iz per point.
int ref_cell_code(const float *xyz, uint64_t n, const float *bounds6,
                  const uint32_t *blocks3, uint32_t *cells3, uint32_t *codes) {
  SpaceRange r = make_range(bounds6[0], bounds6[1], bounds6[2], bounds6[3],
                            bounds6[4], bounds6[5], blocks3[0], blocks3[1],
                            blocks3[2]);
  for (uint64_t i = 0; i < n; ++i) {
    Point3D p(xyz[3 * i], xyz[3 * i + 1], xyz[3 * i + 2], (size_t)i);
    auto c = p.compute_block_indices(r);
    cells3[3 * i] = std::get<0>(c);
    cells3[3 * i + 1] = std::get<1>(c);
    cells3[3 * i + 2] = std::get<2>(c);
    codes[i] = p.compute_morton_code(r);
  }
  return 0;
}

// compute_bbox bounds (min_x,max_x,min_y,max_y,min_z,max_z) after the +/-eps.
int ref_bbox(const float *xyz, uint64_t n, float *bounds6) {
  std::vector<Point3D> pts = to_points(xyz, n);
  SpaceRange r = compute_bbox(pts, 16, 16, 16);
  bounds6[0] = r.min_x; bounds6[1] = r.max_x;
  bounds6[2] = r.min_y; bounds6[3] = r.max_y;
  bounds6[4] = r.min_z; bounds6[5] = r.max_z;
  return 0;
}

} // extern "C"
