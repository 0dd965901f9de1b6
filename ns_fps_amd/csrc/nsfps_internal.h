// Internal types shared by the host library (nsfps_host.cpp) and the HIP
// kernels (nsfps_build.hip, nsfps_sample.hip).  Not part of the C ABI.
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
// Level-1 nodes the tree engine's single-workgroup loop can hold (level 2 then
// fits one wave); the runs engine has no such limit.
constexpr uint32_t kMaxL1 = 4096;
// Threads of the single-workgroup loop (one cube cell per thread per chunk):
// 512 by default, 1024 selectable.
constexpr uint32_t kLateThreads = 512;
// Candidate leaves flattened into LDS per round.
constexpr uint32_t kCandCap = 1024;
// Dynamic LDS budget of the single-workgroup loop (gfx950: 160 KiB per CU).
constexpr uint32_t kLdsBudget = 160 * 1024 - 1024;
constexpr uint32_t kNone = 0xffffffffu;
// Speculative-run engine: list entries (one per thread of the run kernel; also
// the most picks one run can accept), bins per key histogram, histograms per
// round (one from the update pass, then two refinement passes).
constexpr uint32_t kListCap = 1024;
// workgroups per level-1 node in the split update pass
constexpr uint32_t kUpdateSplit = 4;
constexpr uint32_t kHistBins = 4096;
constexpr uint32_t kHists = 3;
constexpr uint32_t kRefinePasses = 2;  // refinement passes when they are launched

// Cells one bucket can hold: codes run below 2^(bits x + bits y + bits z) < 8T.
constexpr uint32_t kMaxAlias = 8;
// Cell that lies outside every cube clipped to a grid whose cells share
// buckets (such a grid has an axis of at most 1023 blocks): pads alias lists.
constexpr uint32_t kNoCell = 0x3fffffffu;

// Cube half-width thresholds kept per axis (half-widths up to this many are
// found by comparisons; larger ones by the reference's arithmetic).
constexpr uint32_t kCubeThr = 8;

// Range values the kernels need, all derived on the host exactly as the
// reference derives them (src/yuezu_fps.cpp:7-11, 136-161, 170-193).
struct RangeDev {
  float mn[3];
  float hiclamp[3];  // max - BOUNDARY_EPS (fp32)
  float inv_bs[3];
  float bsize[3];
  uint32_t blocks[3];
  uint32_t lut_off[3];  // offsets of the x/y/z LUTs in the concatenated LUT
  uint32_t lut_total;
  uint32_t T;           // total blocks = number of buckets
  uint32_t bijective;   // 1 when bucket <-> cell is one-to-one
  // Cells of one bucket: the valid cells among the codes b, b + T, b + 2T, ...
  // below 2^cbits.  na bounds their number (1 when one-to-one, at most
  // kMaxAlias); cmask[a] holds axis a's bits of a code.
  uint32_t na;
  uint32_t cbits;
  uint32_t cmask[3];
  // cube half-width thresholds: half-width >= k + 1 exactly when D >= cube_thr[a][k]
  float cube_thr[3][kCubeThr];
};

// Byte offsets inside the dynamic LDS of the single-workgroup loop; kNone
// marks an optional region that did not fit.
struct LdsPlan {
  uint32_t l1k, l1p;      // level-1 keys (u64) and winner positions (float4)
  uint32_t l1lo, l1hi;    // level-1 bounding boxes (float4), optional
  uint32_t l2k, l2p;      // level-2 (<= 64 nodes)
  uint32_t lut;           // concatenated Morton LUTs (u32)
  uint32_t ctab;          // cell table (uint2, T + 1), optional
  uint32_t cand;          // kCandCap x 3 u32: leaf, first slot, count
  uint32_t slot;          // u32 per level-1 node: staging slot or kNone
  uint32_t m1, dl1;       // dirty level-1 bitmask / list
  uint32_t m2;            // dirty level-2 bitmask (64 bits)
  uint32_t cm;            // per staging slot: 64-bit mask of candidate children
  uint32_t sk, sp;        // staging: dcap x 64 keys (u64) / positions (float4)
  uint32_t dcap;          // staging slots (level-1 nodes per fast iteration)
  uint32_t total;         // bytes
};

// State of the speculative-run engine of one cloud, carried between the
// kernels of a round and from one round to the next.
struct RunState {
  uint64_t kref0;     // every key is <= kref0 when the update pass runs
  uint64_t bkey;      // list threshold chosen by the selection
  uint32_t s0;        // bin shift of the update pass's key histogram
  uint32_t s0_next;   // bin shift proposed for the next round
  uint32_t npicks;    // picks of the last run (applied by the next update pass)
  uint32_t nlist;     // list entries gathered this round
  uint32_t rounds;    // rounds that ran (statistics)
  uint32_t err;       // set if a list overflowed (internal error)
  uint32_t forced;    // rounds whose threshold was forced for want of refinement passes
  uint32_t pad;
};

// Everything one cloud's kernels touch.  Device pointers; passed by value to
// the grid-wide step and as an array to the single-workgroup loop.
struct CloudDev {
  uint32_t n;        // points
  uint32_t m;        // samples requested (2 <= m < n)
  uint32_t nslots;   // physical slots (n, or T * cap when padded)
  uint32_t nleaves;
  uint32_t nl1;      // level-1 tree nodes = ceil(nleaves / kFan)
  uint32_t phys0;    // physical slot of input row 0 (the first sample)
  uint32_t padded;   // 1: slot = bucket * cap + j, leaf = bucket * lpc + k
  uint32_t lpc;      // leaves per bucket when padded
  uint32_t mixed;    // 1: leaf l holds slots 64 l .. 64 l + 63 of the logical order,
                     // which may belong to several buckets (runs engine, one cell
                     // per bucket); 0: a leaf holds points of one bucket
  uint32_t pad0;
  RangeDev r;
  LdsPlan lds;
  const uint32_t *lut;
  float4 *P4;                 // x, y, z, min squared distance per slot
  const uint2 *RO;            // logical rank, input row per slot
  const uint32_t *R;          // logical rank per slot (RO's x apart: the passes over many
                              // points need the rank alone)
  const uint2 *cell_info;     // T + 1 entries: first slot, first leaf
  const float4 *leaf_lo;      // bbox min xyz, w = first slot (bits)
  const float4 *leaf_hi;      // bbox max xyz, w = point count (bits)
  const uint2 *leaf_sc;       // first slot, point count (leaf_lo.w / leaf_hi.w packed)
  const uint32_t *leaf_cell;  // ix | iy << 10 | iz << 20
  const uint32_t *leaf_al;    // r.na per leaf: the cells of its bucket, kNoCell-padded
  const uint2 *leaf_cbox;     // lo / hi corners of the cells of the leaf's points (10 bits
                              // per axis; lo > hi on some axis: no points)
  uint64_t *leaf_key;         // max key of the leaf
  float4 *leaf_pos;           // x, y, z, input row (bits) of that key
  uint64_t *l1_key;
  uint64_t *l1_part;  // split update pass: each node's key is the largest of its
                      // kUpdateSplit parts (l1_key then zero; otherwise parts zero)
  float4 *l1_pos;
  const float4 *l1_lo;        // level-1 bounding boxes
  const float4 *l1_hi;
  const uint2 *l1_cbox;       // level-1 nodes: lo / hi corners over the cells of their
                              // leaves' buckets (lo > hi on some axis: no points)
  uint64_t *root_key;         // 1 entry
  float4 *root_pos;           // 1 entry
  uint32_t *iter;             // samples emitted so far (1 entry)
  uint32_t *done;             // set once sampling finished (1 entry)
  uint32_t *counter;          // arrival counter of the grid-wide step
  int32_t *out;               // m entries
  uint64_t *prof;             // loop phase clocks / counters, or null
  // speculative-run engine
  RunState *rs;
  uint32_t *hist;             // kHists x kHistBins
  float4 *pick_p;             // kListCap: x, y, z, D of each pick of a run
  uint2 *pick_c;              // kListCap: cube lo / hi cells, 11 bits per axis with guard bits
                              // (lo, hi | guards: the run kernel's box-test form)
  float4 *list_p;             // kListCap: x, y, z, min distance
  uint2 *list_r;              // kListCap: logical rank, input row
  uint32_t *list_c;           // kListCap: cell (10 bits per axis)
  uint32_t *list_al;          // kListCap x r.na: the cells of each entry's bucket
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
