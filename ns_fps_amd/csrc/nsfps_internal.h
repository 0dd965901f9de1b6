// Internal types shared by the host library (nsfps_host.cpp) and the HIP
// kernels (nsfps_kernels.hip).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsfps {

// Points per leaf: one wave64 holds one leaf, one point per lane.
constexpr uint32_t kLeaf = 64;
// Fan-out of the max tree above the leaves (one wave reduces one node).
constexpr uint32_t kFan = 64;
// Sub-cell Morton bits (3 per axis) used to order points physically inside a
// cell so that leaf bounding boxes are tight; results do not depend on it.
constexpr uint32_t kFineBits = 9;
// Largest number of level-1 tree nodes the single-workgroup loop keeps in LDS.
constexpr uint32_t kMaxL1 = 8192;
// Cube cells enumerated per chunk by the single-workgroup loop.
constexpr uint32_t kCellChunk = 1024;

// Range values the kernels need, all derived on the host exactly as the
// reference derives them (src/yuezu_fps.cpp:7-11, 136-161, 170-193).
struct RangeDev {
  float mn[3];
  float hiclamp[3];  // max - BOUNDARY_EPS (fp32)
  float inv_bs[3];
  float bsize[3];
  uint32_t blocks[3];
  uint32_t lut_off[3];  // offsets of the x/y/z LUTs in CloudDev::lut
  uint32_t T;           // total blocks = number of buckets
  uint32_t bijective;   // 1 when bucket <-> cell is one-to-one
};

// Everything one cloud's kernels touch.  Device pointers; passed by value to
// single-cloud kernels and as an array to the batched loop.
struct CloudDev {
  uint32_t n;        // points
  uint32_t m;        // samples requested (1 <= m < n)
  uint32_t nleaves;
  uint32_t nl1;      // level-1 tree nodes = ceil(nleaves / kFan)
  uint32_t phys0;    // physical slot of input row 0 (the first sample)
  uint32_t pad_;
  RangeDev r;
  const uint32_t *lut;
  const float *X, *Y, *Z;
  float *C;                  // min squared distance per physical slot
  const uint32_t *RANK;      // logical rank per physical slot
  const uint32_t *ORIG;      // input row per physical slot
  const uint32_t *cell_leaf; // T + 1 entries: first leaf of each bucket
  const float4 *leaf_lo;     // bbox min xyz, w = first physical slot (bits)
  const float4 *leaf_hi;     // bbox max xyz, w = point count (bits)
  const uint32_t *leaf_cell; // ix | iy << 10 | iz << 20
  uint64_t *leaf_key;        // max key of the leaf
  uint32_t *leaf_win;        // physical slot holding that key
  uint64_t *l1_key;
  uint32_t *l1_win;
  uint64_t *root_key;        // 1 entry
  uint32_t *root_win;        // 1 entry
  uint32_t *iter;            // samples emitted so far (1 entry)
  uint32_t *done;            // set once sampling finished (1 entry)
  uint32_t *counter;         // arrival counter of the grid-wide step
  int32_t *out;              // m entries
};

// Argmax key: larger min-distance wins, equal distances go to the smaller
// logical rank (the reference's leftmost-maximum rule).
__host__ __device__ inline uint64_t make_key(float d, uint32_t rank) {
  union { float f; uint32_t u; } c;
  c.f = d;
  return ((uint64_t)c.u << 32) | (uint64_t)(~rank);
}

__host__ __device__ inline float key_dist(uint64_t k) {
  union { float f; uint32_t u; } c;
  c.u = (uint32_t)(k >> 32);
  return c.f;
}

}  // namespace nsfps
