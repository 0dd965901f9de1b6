// Speculative-run sampling engine (gfx950).
//
// Keys (min-distance bits << 32 | ~logical rank) only ever decrease.  Take a
// threshold key B and the list of every point whose key is >= B: a point
// outside the list stays below B for the rest of the sampling, so while the
// list's maximum is >= B it is the global maximum, i.e. the reference's next
// sample (src/yuezu_fps.cpp:703-722).  The run kernel holds the list in one
// workgroup (one entry per thread) and takes samples from it one after
// another, applying each sample's cube update (src/yuezu_fps.cpp:560-597) to
// the list alone, until the list maximum drops below B or sampling ends.
//
// A grid-wide pass then applies every sample of the run to every point.
// min() of exact fp32 distances commutes, so each point ends with the same
// bits as after the reference's one-by-one updates.  The same pass rebuilds
// the leaf and level-1 keys and histograms the keys for the next threshold.
// Only the keys: the samples come from the list, so the winners' positions
// (leaf_pos, l1_pos, which the tree engine keeps) are not maintained.
//
// One round, in stream order:
//   k_update     picks -> points, leaf and level-1 keys, key histogram
//   k_refine x2  finer histograms inside the crossing bin, only when needed
//   k_gather     threshold B (<= kListCap keys above it), list of those points
//   k_run        samples from the list
// The first round's only pick is input row 0 with a cube covering the whole
// grid: the reference's first full pass (src/yuezu_fps.cpp:431-438).
//
// The cube test compares cell coordinates.  Where cells share buckets (block
// counts that are not powers of two: the Morton code is taken modulo the
// block count, src/yuezu_fps.cpp:413, 592) a point is updated when the cube
// holds any cell of its bucket, so every kernel tests each cell of a bucket
// (the ALIAS variants).
#include <hip/hip_runtime.h>

#include "nsfps_device.h"
#include "nsfps_launch.h"

namespace nsfps {

constexpr uint32_t kPassThreads = 1024;  // grid-wide passes: one level-1 node per workgroup
constexpr uint32_t kPassWaves = kPassThreads / 64;
constexpr uint32_t kLeavesPerWave = kFan / kPassWaves;
constexpr uint32_t kMaxShift = 52;  // kHistBins << 52 covers the whole u64 key range
constexpr uint32_t kSparseGroups = 128;  // workgroups per cloud of the refinement and gather passes
constexpr uint32_t kGatherNodes = 16;    // nodes per list-range claim of the gather pass
constexpr uint32_t kGatherHold = 4;      // hot leaves per wave whose points stay in registers

// Work counters of the grid-wide passes (profile words, summed over rounds):
// leaves whose points the update pass reads and those points, and the same
// for the gather pass.
enum : uint32_t { kCtUpLeaves = 24, kCtUpPoints, kCtGaLeaves, kCtGaPoints };
// The update pass's phase clocks (s_memrealtime ticks summed over the
// workgroups that update a node): run state, node and picks; the leaves; the
// node key and the histogram's flush; and those workgroups.
enum : uint32_t { kUpTPicks = 32, kUpTLeaves, kUpTFlush, kUpGroups };
// Finer update-pass clocks: the first reads, clearing the histogram, finding
// the touched leaves, and their points' reads (parts of the two above); the
// gather pass's: the selection's replay, the leaf records, the held points
// and the list range's claim, the writes; and its workgroups.
enum : uint32_t {
  kUpTLoad = 40, kUpTZero, kUpTHits, kUpTPts,
  kGaTSel = 44, kGaTLeaf, kGaTClaim, kGaTWrite, kGaGroups,
  // per update workgroup, over its waves: the latest and the summed times
  // from the picks' barrier to the points' arrival and to the leaf loop's end
  kUpWPtsMax = 49, kUpWPtsSum, kUpWLoopMax, kUpWLoopSum,
  // leaves the update pass reads because a pick touches them, and their points
  kCtUpHitLeaves = 53, kCtUpHitPoints,
  // per update workgroup, over its waves: the latest and the summed times of
  // finding the touched leaves
  kUpWHitsMax = 55, kUpWHitsSum,
  // keys inside the update pass's histogram window (summed over rounds), and
  // the list entries gathered
  kGaWinKeys = 57, kGaListed, kGaWinMax
};

__device__ __forceinline__ uint32_t pack_cell(uint32_t x, uint32_t y, uint32_t z) {
  return x | (y << 10) | (z << 20);
}

// Squared distance from q to the nearest point of the box lo..hi, in the
// operation order of sqdist.  Rounding is monotonic, so it never exceeds
// sqdist of q and a point in the box: when it is >= every distance of the
// box's points, q lowers none of them (a point is lowered by a strictly
// smaller distance).  NaN when q has a NaN coordinate.
__device__ __forceinline__ float box_bound(float qx, float qy, float qz, float lx, float ly,
                                           float lz, float hx, float hy, float hz) {
  const float qv[3] = {qx, qy, qz}, lv[3] = {lx, ly, lz}, hv[3] = {hx, hy, hz};
  float g[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const float below = lv[a] - qv[a], above = qv[a] - hv[a];
    const float gg = below > above ? below : above;
    g[a] = gg > 0.f ? gg : 0.f;
  }
  return (g[0] * g[0] + g[1] * g[1]) + g[2] * g[2];
}

// Cell inside a cube given as packed lo / hi corners.
__device__ __forceinline__ bool cell_in(uint32_t cell, uint2 cube) {
  const uint32_t x = cell & 1023u, y = (cell >> 10) & 1023u, z = cell >> 20;
  // & rather than &&: straight-line compares, no branch per axis
  return (x >= (cube.x & 1023u)) & (x <= (cube.y & 1023u)) & (y >= ((cube.x >> 10) & 1023u)) &
         (y <= ((cube.y >> 10) & 1023u)) & (z >= (cube.x >> 20)) & (z <= (cube.y >> 20));
}

// Cells packed 11 bits per axis (x | y << 11 | z << 22): bits 10 and 21 stay
// clear and act as guards, so lo <= c <= hi on all three axes takes two
// subtractions.  cg = pack11(c) | kGuards, c11 = pack11(c), hig = pack11(hi) |
// kGuards.  Per axis, cg - lo keeps its guard bit (or, for z, does not borrow)
// exactly when c >= lo, and hig - c11 likewise when c <= hi.
constexpr uint32_t kGuards = (1u << 10) | (1u << 21);

__device__ __forceinline__ uint32_t pack11(uint32_t c10) {
  return (c10 & 1023u) | (((c10 >> 10) & 1023u) << 11) | ((c10 >> 20) << 22);
}

__device__ __forceinline__ uint32_t in_box11(uint32_t cg, uint32_t c11, uint32_t lo,
                                             uint32_t hig) {
  uint32_t t1, t2;
  const bool b1 = __builtin_usub_overflow(cg, lo, &t1);
  const bool b2 = __builtin_usub_overflow(hig, c11, &t2);
  return (uint32_t)(((t1 & t2 & kGuards) == kGuards) & !b1 & !b2);
}

// Level-1 node g's key: the largest of l1_key and the node's parts (in a call
// whose update pass is split, l1_key is zero and the parts hold the largest
// keys of the node's quarters; otherwise the parts are zero).  In the split
// update pass a workgroup reads its siblings' parts while they may write
// them: the parts are read and written as relaxed agent-scope atomics (each
// 64-bit word whole, no order needed: either value of a part bounds its
// quarter's points, distances only falling).
__device__ __forceinline__ uint64_t node_key(const CloudDev &c, uint32_t g) {
  NSFPS_GLOBAL uint64_t *const pp = gptr(c.l1_part) + (size_t)g * kUpdateSplit;
  uint64_t k = gptr(c.l1_key)[g];
#pragma unroll
  for (uint32_t s = 0; s < kUpdateSplit; ++s) {
    const uint64_t v = __hip_atomic_load(pp + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    k = v > k ? v : k;
  }
  return k;
}

// Cube overlapping the cell range [lo, hi] (packed corners).
__device__ __forceinline__ bool cube_overlaps(uint2 cube, uint32_t lo, uint32_t hi) {
  bool ok = true;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const uint32_t s = 10u * a;
    ok &= ((cube.x >> s) & 1023u) <= ((hi >> s) & 1023u);
    ok &= ((cube.y >> s) & 1023u) >= ((lo >> s) & 1023u);
  }
  return ok;
}

// Histogram window of a selection pass: kHistBins bins of 2^S keys each, bin
// 0 ending at kref.  Lowest key inside the window:
__device__ __forceinline__ uint64_t window_lo(uint64_t kref, uint32_t S) {
  if (S >= kMaxShift) return 0;
  const uint64_t w = ((uint64_t)kHistBins << S) - 1;
  return kref >= w ? kref - w : 0;
}

__device__ __forceinline__ uint32_t key_bin(uint64_t key, uint64_t kref, uint32_t S) {
  if (key > kref) return kNone;
  const uint64_t b = (kref - key) >> S;
  return b < kHistBins ? (uint32_t)b : kNone;
}

// The key histograms (kHists of kHistBins each): the update pass counts
// histogram 0, the refinement passes histograms 1 and 2.
__device__ __forceinline__ NSFPS_GLOBAL uint32_t *hist_set(const CloudDev &c) {
  return gptr(c.hist);
}

// Threshold selection, replayed identically by every workgroup that needs it.
// A histogram over window (kref, S) gives the first bin where the cumulative
// count exceeds the free capacity; the bins before it are taken.  If they
// fill less than half of it, that crossing bin is histogrammed again 12 bits
// finer by the next refinement pass.  The update pass counts one window below
// kref0 (shift s0, set from the previous round's key span).  A window that
// holds fewer keys than the list takes all of them: the run is shorter, and
// the next round's window, sized from this round's span, is 4x wider.  When
// nothing fits (more than kListCap keys share the finest bin) or the window is
// empty, the threshold is the maximum key.
struct Sel {
  uint64_t kref;
  uint64_t bkey;     // resolved threshold
  uint32_t S;
  uint32_t cap;      // capacity left
  uint32_t total;    // entries taken so far
  uint32_t state;    // 0: refinement pass `pass` needed, 1: resolved, 2: use the maximum key
  uint32_t pass;
  uint32_t win;      // keys inside the update pass's histogram window
};

struct Step {
  uint32_t tot;     // keys in the window
  uint32_t bs;      // crossing bin, kNone when tot <= cap
  uint32_t before;  // keys in the bins before it
};

// Block-wide, all kPassThreads threads; sc holds kPassWaves + 2 words of LDS.
// h: this thread's four bins of the histogram.
__device__ Step hist_step(uint4 h, uint32_t cap, uint32_t *sc) {
  const uint32_t tid = threadIdx.x;
  uint32_t tot;
  const uint32_t pre = block_excl_scan<kPassWaves>(h.x + h.y + h.z + h.w, sc, &tot);
  const uint32_t bins[4] = {h.x, h.y, h.z, h.w};
  uint32_t c = pre;
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    if (c <= cap && c + bins[j] > cap) {  // exactly one bin crosses
      sc[kPassWaves] = 4 * tid + j;
      sc[kPassWaves + 1] = c;
    }
    c += bins[j];
  }
  __syncthreads();
  Step st;
  st.tot = tot;
  st.bs = tot <= cap ? kNone : sc[kPassWaves];
  st.before = tot <= cap ? 0u : sc[kPassWaves + 1];
  __syncthreads();
  return st;
}
__device__ Step hist_step(const uint32_t *H, uint32_t cap, uint32_t *sc) {
  return hist_step(gptr(reinterpret_cast<const uint4 *>(H))[threadIdx.x], cap, sc);
}

// Replays the selection from the update pass's histograms and the first
// `avail - 1` refinement histograms; `passes` refinement passes run this
// round, so the threshold is forced at step `passes` (forced is set when that
// rule, not the histograms, ended the selection with a list under a quarter
// full).  h0: this thread's bins of the update pass's histogram, when the
// caller read them already.
__device__ Sel sel_replay(const CloudDev &c, uint32_t avail, uint32_t passes, uint32_t *sc,
                          bool *forced = nullptr, const uint4 *h0 = nullptr) {
  const NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
  Sel s;
  s.kref = rs.kref0;
  s.bkey = 0;
  s.S = rs.s0;
  s.cap = kListCap;
  s.total = 0;
  s.state = 0;
  s.pass = 0;
  const uint32_t *H0 = c.hist;
  Step st = h0 ? hist_step(*h0, s.cap, sc) : hist_step(H0, s.cap, sc);
  s.win = st.tot;
  for (uint32_t p = 0;; ++p) {
    if (st.bs == kNone) {  // the whole window fits
      s.total += st.tot;
      s.bkey = window_lo(s.kref, s.S);
      s.state = s.total ? 1u : 2u;
      return s;
    }
    s.total += st.before;
    if (st.before >= s.cap / 2 || s.S == 0 || p == passes) {
      // forced, and the list under a quarter full: refinement would have paid
      if (forced) *forced = st.before < s.cap / 2 && s.S != 0 && s.total < kListCap / 4;
      s.bkey = s.kref - ((uint64_t)st.bs << s.S) + 1;  // keys above bin bs
      s.state = s.total ? 1u : 2u;
      return s;
    }
    s.cap -= st.before;
    s.kref -= (uint64_t)st.bs << s.S;
    s.S = s.S >= 12 ? s.S - 12 : 0;
    if (p + 1 >= avail) {
      s.pass = p + 1;
      return s;
    }
    st = hist_step(H0 + (1 + p) * kHistBins, s.cap, sc);
  }
}

__device__ __forceinline__ const NSFPS_GLOBAL RunState &rstate(const CloudDev &c) {
  return *gptr(c.rs);
}

// ------------------------------------------------------------ update pass

// Applies the picks of the last run to the points of level-1 node blockIdx.x,
// rewrites the keys of the touched leaves and of the node, and counts the keys
// inside the histogram window.  A pick takes part in a node only when its
// cube overlaps the node's cells and it may lower one of the node's points:
// its least squared distance to the node's box (box_bound) is below the
// largest distance of those points, which the node's key holds (the
// reference's cube rule, src/yuezu_fps.cpp:560-597, also visits points no
// pick lowers; skipping them changes no distance).  Leaves no pick touches
// whose key lies below the window keep their key and are not read.  A leaf
// keeps its key too when no pick lowers the point that holds it (keys only
// decrease), so its maximum is searched only otherwise.  Reads that do not depend on each other are
// issued together: the wave's leaf records with the run state and the node's
// record, a pick's cube with its position, and the points of every leaf of
// the wave that needs reading.  PROF: counts the leaves and points it reads.
// ALIAS: cells share buckets, and a pick touches a leaf when its cube holds
// any cell of the leaf's bucket (src/yuezu_fps.cpp:573-597 updates every point
// of every bucket of the cube's cells); nodes are screened by the corners of
// those cells.  LB: a pick also takes part in a leaf only if its distance
// bound to the leaf's box is below the leaf key's distance (the node test
// again, per leaf).  SPLIT: the node's leaves are split over SPLIT
// workgroups, each storing the largest key of its leaves as one of the
// node's parts (node_key reads the node's key back as the largest part).
// MIXED: a leaf is a run of 64 slots of the logical order and may hold
// several buckets (one cell each); a pick touches the leaf when its cube
// overlaps the leaf's cell box, and lowers a point only when the point's own
// cell lies in the cube (the reference's rule, point by point).
template <bool PROF, bool ALIAS, bool LB, uint32_t SPLIT, bool MIXED>
__global__ __launch_bounds__(kPassThreads, 2) __attribute__((amdgpu_num_sgpr(60))) void k_update(
    const CloudDev *__restrict__ clouds) {
  static_assert(!(ALIAS && MIXED), "leaves of several buckets need one cell per bucket");
  __shared__ uint32_t s_hist[kHistBins];
  __shared__ float4 s_pp[kListCap];
  __shared__ uint2 s_pc[kListCap];  // the picks' cube corners: pack11(lo), pack11(hi) | kGuards
  __shared__ uint64_t s_lk[kFan];
  __shared__ uint32_t s_np;
  __shared__ uint32_t s_ct[4];  // PROF: leaves and points read by the workgroup, and of them touched
  __shared__ uint32_t s_wt[PROF ? 3 * kPassWaves : 1];  // PROF: per-wave clocks
  const CloudDev &c = clouds[blockIdx.y];
  // SPLIT workgroups per node: this one takes leaves sub * kFan / SPLIT ..
  constexpr uint32_t kLPW = kLeavesPerWave / SPLIT;  // leaves per wave
  static_assert(kLPW >= 1 && kLPW * SPLIT == kLeavesPerWave, "whole leaves per wave");
  const uint32_t g = blockIdx.x / SPLIT, sub = blockIdx.x % SPLIT;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint64_t ut0 = PROF ? __builtin_amdgcn_s_memrealtime() : 0;
  // this wave's leaves: lane k < kLPW holds leaf leaf0 + k's record
  const uint32_t leaf0 = g * kFan + sub * (kFan / SPLIT) + wave * kLPW;
  uint64_t mkey = 0;
  uint32_t mcell = 0, mst = 0, mcnt = 0;
  uint32_t mchi = 0;  // MIXED: the leaf's cell box is mcell .. mchi
  // LB (leaf bounds): the leaf's box of points (an absent leaf's stays empty)
  constexpr bool lbound = LB;
  float4 mlo = make_float4(0.f, 0.f, 0.f, 0.f), mhi = mlo;
  if (lane < kLPW && leaf0 + lane < c.nleaves) {
    mkey = gptr(c.leaf_key)[leaf0 + lane];
    if (MIXED) {
      const uint2 cb = gptr(c.leaf_cbox)[leaf0 + lane];
      mcell = cb.x;
      mchi = cb.y;
    } else {
      mcell = gptr(c.leaf_cell)[leaf0 + lane];
    }
    const uint2 sc = gptr(c.leaf_sc)[leaf0 + lane];
    mst = sc.x;
    mcnt = sc.y;
    if (lbound) {
      mlo = gptr(c.leaf_lo)[leaf0 + lane];
      mhi = gptr(c.leaf_hi)[leaf0 + lane];
    }
  }
  const NSFPS_GLOBAL RunState &rs = rstate(c);
  const uint32_t done = *gptr(c.done);
  const uint32_t npicks = min(rs.npicks, kListCap);
  const uint64_t kref = rs.kref0;
  const uint32_t S = rs.s0;
  const uint32_t gn = g < c.nl1 ? g : 0u;  // read unconditionally, used only if g < nl1
  // split: a sibling workgroup may have written its part already; either value
  // bounds this workgroup's points (distances only fall)
  const uint64_t nkey = SPLIT == 1 ? gptr(c.l1_key)[gn] : node_key(c, gn);
  uint32_t clo, chi;
  uint64_t uta = 0, utb = 0, utc = 0, utd = 0;
  // the node's box of points (x > its hi x: no points)
  const float4 nlo = gptr(c.l1_lo)[gn], nhi = gptr(c.l1_hi)[gn];
  // the cells of this wave's leaves' buckets: lane i < kLPW * na
  // holds word i of the wave's stretch of leaf_al
  const uint32_t na = ALIAS ? c.r.na : 1u;
  uint32_t mal = kNoCell;
  if (ALIAS) {
    const uint2 cb = gptr(c.l1_cbox)[gn];
    if (lane < kLPW * na && leaf0 + lane / na < c.nleaves)
      mal = gptr(c.leaf_al)[(size_t)leaf0 * na + lane];
    pin_sgpr(done, npicks, kref, S, nkey, cb.x, cb.y, nlo.x, nlo.y, nlo.z, nhi.x, nhi.y,
             nhi.z);
    if (g >= c.nl1 || done || cb.x == kNone) return;  // finished, or no points
    if (PROF) uta = __builtin_amdgcn_s_memrealtime();
    clo = cb.x;
    chi = cb.y;
  } else {
    // the run state and the node's record are read together, ahead of the exit
    pin_sgpr(done, npicks, kref, S, nkey, nlo.x, nlo.y, nlo.z, nhi.x, nhi.y, nhi.z);
    if (g >= c.nl1 || done || nlo.x > nhi.x) return;  // finished, or no points
    if (PROF) uta = __builtin_amdgcn_s_memrealtime();
    clo = pack_cell(cell_axis(c.r, 0, nlo.x), cell_axis(c.r, 1, nlo.y), cell_axis(c.r, 2, nlo.z));
    chi = pack_cell(cell_axis(c.r, 0, nhi.x), cell_axis(c.r, 1, nhi.y), cell_axis(c.r, 2, nhi.z));
  }
  const uint64_t wlo = window_lo(kref, S);
  // the node's cell range in the picks' box-test form
  const uint32_t clo11 = pack11(clo), chi11g = pack11(chi) | kGuards;
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) s_hist[j] = 0;
  if (tid == 0) s_np = 0;
  if (PROF && tid < 4) s_ct[tid] = 0;
  __syncthreads();
  if (PROF) utb = __builtin_amdgcn_s_memrealtime();
  for (uint32_t i = tid; i < npicks; i += kPassThreads) {
    const uint2 cb = gptr(c.pick_c)[i];
    const float4 pp = gptr(c.pick_p)[i];
    const float px = pp.x, py = pp.y, pz = pp.z;
    const uint32_t c0 = cb.x, c1 = cb.y;
    pin_vgpr(c0, c1, px, py, pz);  // both reads in flight together
    // the cube overlaps the node's cells (cube lo <= node hi and node lo <=
    // cube hi on every axis: the guard test of in_box11 crosswise), and the
    // pick may lower one of its points (the node key holds their largest
    // distance)
    if (in_box11(c1, c0, clo11, chi11g) &&
        !(box_bound(px, py, pz, nlo.x, nlo.y, nlo.z, nhi.x, nhi.y, nhi.z) >=
          __uint_as_float((uint32_t)(nkey >> 32)))) {
      const uint32_t k = atomicAdd(&s_np, 1u);
      s_pp[k] = make_float4(px, py, pz, 0.f);
      s_pc[k] = make_uint2(c0, c1);
    }
  }
  __syncthreads();
  const uint32_t nsel = s_np;
  const uint64_t ut1 = PROF ? __builtin_amdgcn_s_memrealtime() : 0;
  if (nsel == 0 && nkey < wlo) return;  // nothing changes, nothing to count
  // which leaves a pick touches (hm: the first 64 picks whose cube holds the
  // leaf's cell), and which must be read
  uint32_t c11[kLPW], st[kLPW], cnt[kLPW];
  uint32_t ch11g[MIXED ? kLPW : 1];  // MIXED: pack11 of the leaf's cell box hi, with guards
  uint64_t okey[kLPW], hm[kLPW];
  bool hit[kLPW], need[kLPW];
  // pick i's cube (its s_pc record) holds (a cell of the bucket of) leaf k.
  // Testing the leaf's box against the pick as the node's is tested costs
  // more here than the reads it saves on points that fill their cells.
  const auto touches_pick = [&](uint32_t k, uint2 cube) -> bool {
    uint32_t in;
    if (MIXED) {  // the cube overlaps the leaf's cell box (in_box11 crosswise)
      in = in_box11(cube.y, cube.x, c11[k], ch11g[MIXED ? k : 0]);
    } else if (!ALIAS) {
      in = in_box11(c11[k] | kGuards, c11[k], cube.x, cube.y);
    } else if (na == 2) {
      const uint32_t a0 = pack11(rdlane(mal, 2 * k)), a1 = pack11(rdlane(mal, 2 * k + 1));
      in = in_box11(a0 | kGuards, a0, cube.x, cube.y) | in_box11(a1 | kGuards, a1, cube.x, cube.y);
    } else {
      in = 0;
      for (uint32_t a = 0; a < na; ++a) {
        const uint32_t a0 = pack11(rdlane(mal, k * na + a));
        in |= in_box11(a0 | kGuards, a0, cube.x, cube.y);
      }
    }
    return in != 0;
  };
  const auto touches = [&](uint32_t k, uint32_t i) -> bool { return touches_pick(k, s_pc[i]); };
  // the first 64 picks' cubes, lane i holding pick i's, read once for the
  // four leaves (past nsel: stale LDS, masked out)
  const uint2 pc0 = s_pc[lane];
  const bool in0 = lane < nsel;
  const float4 pp0 = lbound ? s_pp[lane] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (uint32_t k = 0; k < kLPW; ++k) {
    c11[k] = pack11(rdlane(mcell, k));
    if (MIXED) ch11g[MIXED ? k : 0] = pack11(rdlane(mchi, k)) | kGuards;
    st[k] = rdlane(mst, k);
    cnt[k] = rdlane(mcnt, k);
    okey[k] = ((uint64_t)rdlane((uint32_t)(mkey >> 32), k) << 32) | rdlane((uint32_t)mkey, k);
    // with leaf bounds, a pick takes part in leaf k only if its squared
    // distance to the leaf's box (in sqdist's operation order, so never above
    // a point's distance) is below the leaf key's distance, the largest of
    // its points: otherwise it lowers none of them
    const float lmax = __uint_as_float((uint32_t)(okey[k] >> 32));
    const float4 blo = make_float4(__uint_as_float(rdlane(__float_as_uint(mlo.x), k)),
                                   __uint_as_float(rdlane(__float_as_uint(mlo.y), k)),
                                   __uint_as_float(rdlane(__float_as_uint(mlo.z), k)), 0.f);
    const float4 bhi = make_float4(__uint_as_float(rdlane(__float_as_uint(mhi.x), k)),
                                   __uint_as_float(rdlane(__float_as_uint(mhi.y), k)),
                                   __uint_as_float(rdlane(__float_as_uint(mhi.z), k)), 0.f);
    const auto may_lower = [&](float4 q) -> bool {
      return !lbound ||
             !(box_bound(q.x, q.y, q.z, blo.x, blo.y, blo.z, bhi.x, bhi.y, bhi.z) >= lmax);
    };
    hm[k] = __ballot((uint32_t)in0 & (uint32_t)touches_pick(k, pc0) & (uint32_t)may_lower(pp0));
    bool h = hm[k] != 0;
    for (uint32_t cb = 64; cb < nsel && !h; cb += 64)
      h = __ballot((cb + lane < nsel) && touches(k, cb + lane) && may_lower(s_pp[cb + lane])) != 0;
    hit[k] = h;
    need[k] = leaf0 + k < c.nleaves && (h || okey[k] >= wlo);
  }
  if (PROF) {
    utc = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) s_wt[2 * kPassWaves + wave] = (uint32_t)(utc - ut1);
  }
  if (PROF && lane == 0) {
    uint32_t nl = 0, npt = 0, nh = 0, nhp = 0;
#pragma unroll
    for (uint32_t k = 0; k < kLPW; ++k) {
      nl += need[k] ? 1u : 0u;
      npt += need[k] ? cnt[k] : 0u;
      nh += need[k] && hit[k] ? 1u : 0u;
      nhp += need[k] && hit[k] ? cnt[k] : 0u;
    }
    if (nl) {
      atomicAdd(&s_ct[0], nl);
      atomicAdd(&s_ct[1], npt);
      atomicAdd(&s_ct[2], nh);
      atomicAdd(&s_ct[3], nhp);
    }
  }
  float4 p[kLPW];
  uint32_t rk[kLPW];  // logical ranks
  // every lane loads, without a branch, so that the four leaves' loads are in
  // flight together; a lane without a point of a needed leaf reads slot 0
  // (one line for the whole wave) and its values are never used: every use
  // below is guarded by lane < cnt
#pragma unroll
  for (uint32_t k = 0; k < kLPW; ++k) {
    const uint32_t idx = need[k] && lane < cnt[k] ? st[k] + lane : 0u;
    p[k] = gptr(c.P4)[idx];
    rk[k] = gptr(c.R)[idx];
  }
  if (PROF) {  // wait for the points (profiled build only)
#pragma unroll
    for (uint32_t k = 0; k < kLPW; ++k) pin_vgpr(p[k].x, rk[k]);
    utd = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) s_wt[wave] = (uint32_t)(utd - ut1);
  }
  // each leaf's stores are issued as soon as it is worked out, so that they
  // overlap the next leaves' work (deferring them all to the end measured
  // 0.23 ms slower per call on the 1M uniform cube)
#pragma unroll
  for (uint32_t k = 0; k < kLPW; ++k) {
    const uint32_t li = wave * kLPW + k;
    uint64_t key = 0;
    if (leaf0 + k < c.nleaves) {
      // unchanged unless the point holding the key is lowered below
      key = okey[k];
      if (need[k]) {
        const bool act = lane < cnt[k];
        const uint32_t lo = ~rk[k];
        float d = p[k].w;
        if (hit[k]) {
          // MIXED: this point's own cell (pack11), the cell its bucket is
          uint32_t pc11 = 0;
          if (MIXED)
            pc11 = pack11(pack_cell(cell_axis(c.r, 0, p[k].x), cell_axis(c.r, 1, p[k].y),
                                    cell_axis(c.r, 2, p[k].z)));
          for (uint32_t cb = 0; cb < nsel; cb += 64) {
            uint64_t m = cb == 0 ? hm[k] : __ballot((cb + lane < nsel) & touches(k, cb + lane));
            while (m) {
              const uint32_t j = (uint32_t)__ffsll((long long)m) - 1;
              m &= m - 1;
              const float4 q = s_pp[cb + j];
              const float dd = sqdist(p[k].x, p[k].y, p[k].z, q.x, q.y, q.z);
              if (MIXED) {
                const uint2 qc = s_pc[cb + j];
                d = in_box11(pc11 | kGuards, pc11, qc.x, qc.y) && dd < d ? dd : d;
              } else {
                d = dd < d ? dd : d;
              }
            }
          }
          const bool lowered = act && d < p[k].w;
          if (lowered) ((NSFPS_GLOBAL float *)gptr(c.P4 + st[k] + lane))[3] = d;
          if (__ballot(lowered && lo == (uint32_t)okey[k])) {
            const uint32_t hi = act ? __float_as_uint(d) : 0u;
            uint32_t mh;
            const uint32_t wl = key_winner(hi, lo, act, mh);
            key = ((uint64_t)mh << 32) | rdlane(lo, wl);  // the leaf has points: wl < 64
            if (lane == 0) gptr(c.leaf_key)[leaf0 + k] = key;
          }
        }
        if (act) {
          const uint32_t hi = __float_as_uint(d);
          const uint32_t b = key_bin(((uint64_t)hi << 32) | lo, kref, S);
          if (b != kNone) atomicAdd(&s_hist[b], 1u);
        }
      }
    }
    if (lane == 0) s_lk[li] = key;
  }
  if (PROF && lane == 0) s_wt[kPassWaves + wave] = (uint32_t)(__builtin_amdgcn_s_memrealtime() - ut1);
  __syncthreads();
  const uint64_t ut2 = PROF ? __builtin_amdgcn_s_memrealtime() : 0;
  if (wave == 0 && SPLIT == 1) {
    const uint64_t k = s_lk[lane];
    uint32_t mh;
    const uint32_t wl = key_winner((uint32_t)(k >> 32), (uint32_t)k, true, mh);
    if (lane == 0) gptr(c.l1_key)[g] = ((uint64_t)mh << 32) | (uint32_t)s_lk[wl];
  } else if (wave == 0) {
    // this quarter's largest key (keys are unique: the rank is their low word)
    const uint64_t part = wave_max_u64(lane < kFan / SPLIT ? s_lk[lane] : 0ull);
    if (lane == 0)
      __hip_atomic_store(gptr(c.l1_part) + (size_t)g * SPLIT + sub, part, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  NSFPS_GLOBAL uint32_t *H = hist_set(c);
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) {
    const uint32_t v = s_hist[j];
    if (v) atomicAdd(&H[j], v);
  }
  if (PROF && tid == 0) {
    const uint64_t ut3 = __builtin_amdgcn_s_memrealtime();
    unsigned long long *pw = (unsigned long long *)gptr(c.prof);
    atomicAdd(pw + kUpTPicks, (unsigned long long)(ut1 - ut0));
    atomicAdd(pw + kUpTLeaves, (unsigned long long)(ut2 - ut1));
    atomicAdd(pw + kUpTFlush, (unsigned long long)(ut3 - ut2));
    atomicAdd(pw + kUpGroups, 1ull);
    atomicAdd(pw + kUpTLoad, (unsigned long long)(uta - ut0));
    atomicAdd(pw + kUpTZero, (unsigned long long)(utb - uta));
    atomicAdd(pw + kUpTHits, (unsigned long long)(utc - ut1));
    atomicAdd(pw + kUpTPts, (unsigned long long)(utd - utc));
    uint32_t pmax = 0, psum = 0, lmax = 0, lsum = 0, hmax = 0, hsum = 0;
    for (uint32_t w = 0; w < kPassWaves; ++w) {
      hmax = max(hmax, s_wt[2 * kPassWaves + w]);
      hsum += s_wt[2 * kPassWaves + w];
      pmax = max(pmax, s_wt[w]);
      psum += s_wt[w];
      lmax = max(lmax, s_wt[kPassWaves + w]);
      lsum += s_wt[kPassWaves + w];
    }
    atomicAdd(pw + kUpWPtsMax, (unsigned long long)pmax);
    atomicAdd(pw + kUpWPtsSum, (unsigned long long)psum);
    atomicAdd(pw + kUpWLoopMax, (unsigned long long)lmax);
    atomicAdd(pw + kUpWLoopSum, (unsigned long long)lsum);
    atomicAdd(pw + kUpWHitsMax, (unsigned long long)hmax);
    atomicAdd(pw + kUpWHitsSum, (unsigned long long)hsum);
    atomicAdd(pw + kCtUpLeaves, (unsigned long long)s_ct[0]);
    atomicAdd(pw + kCtUpPoints, (unsigned long long)s_ct[1]);
    atomicAdd(pw + kCtUpHitLeaves, (unsigned long long)s_ct[2]);
    atomicAdd(pw + kCtUpHitPoints, (unsigned long long)s_ct[3]);
  }
}

// ------------------------------------------------------- refinement passes

// Refinement pass `pass` (1 or 2): counts the keys inside the window the
// selection replayed from the earlier histograms asks for; does nothing when
// the threshold is already resolved.  Few workgroups, each striding over the
// level-1 nodes: the pass is usually skipped, and then costs little more than
// its launch.
__global__ __launch_bounds__(kPassThreads) void k_refine(const CloudDev *__restrict__ clouds,
                                                         uint32_t pass, uint32_t passes) {
  __shared__ uint32_t s_hist[kHistBins];
  __shared__ uint32_t s_sc[kPassWaves + 2];
  const CloudDev &c = clouds[blockIdx.y];
  if (blockIdx.x >= c.nl1 || *gptr(c.done)) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const Sel s = sel_replay(c, pass, passes, s_sc);
  if (s.state != 0 || s.pass != pass) return;
  const uint64_t wlo = window_lo(s.kref, s.S);
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) s_hist[j] = 0;
  __syncthreads();
  for (uint32_t g = blockIdx.x; g < c.nl1; g += gridDim.x) {
    if (node_key(c, g) < wlo) continue;
    for (uint32_t k = 0; k < kLeavesPerWave; ++k) {
      const uint32_t leaf = g * kFan + wave * kLeavesPerWave + k;
      if (leaf >= c.nleaves || gptr(c.leaf_key)[leaf] < wlo) continue;
      const uint2 sc = gptr(c.leaf_sc)[leaf];
      const uint32_t st = sc.x, cnt = sc.y;
      if (lane < cnt) {
        const float d = ((const NSFPS_GLOBAL float *)gptr(c.P4 + st + lane))[3];
        const uint32_t rank = gptr(c.R)[st + lane];
        const uint32_t b = key_bin(((uint64_t)__float_as_uint(d) << 32) | ~rank, s.kref, s.S);
        if (b != kNone) atomicAdd(&s_hist[b], 1u);
      }
    }
  }
  __syncthreads();
  NSFPS_GLOBAL uint32_t *H = hist_set(c) + pass * kHistBins;
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) {
    const uint32_t v = s_hist[j];
    if (v) atomicAdd(&H[j], v);
  }
}

// ------------------------------------------------------------- gather pass

__device__ __forceinline__ uint32_t bit_length(uint64_t v) { return v ? 64u - __clzll(v) : 0u; }

// Resolves the threshold from the histograms and appends every point whose key
// is >= it to the list.  When no threshold below the maximum fits the list
// (more than kListCap keys inside the finest bin), the threshold is the
// maximum key itself: a run of one sample.  Few workgroups, each striding over
// the level-1 nodes; most nodes hold no key above the threshold.  PROF: counts
// the hot leaves whose points it reads and those points.  An entry's cell is
// its point's own (where its cube is centred when it becomes a sample).
// ALIAS (cells share buckets): the entry also carries the cells of its
// bucket.
template <bool PROF, bool ALIAS>
__global__ __launch_bounds__(kPassThreads) void k_gather(const CloudDev *__restrict__ clouds,
                                                         uint32_t passes) {
  __shared__ uint32_t s_sc[kPassWaves + 2];
  __shared__ uint64_t s_wk[kPassWaves];
  const CloudDev &c = clouds[blockIdx.y];
  const uint64_t gt0 = PROF ? __builtin_amdgcn_s_memrealtime() : 0;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  // Reads that depend on nothing read before them go out together with the
  // run state: the update pass's histogram bins and the first node chunk's
  // leaf records.
  const uint4 h0 = gptr(reinterpret_cast<const uint4 *>(c.hist))[tid];
  const auto leaf_of = [&](uint32_t c0, uint32_t &gq) {
    gq = c0 + (lane / kLeavesPerWave) * gridDim.x;
    return gq * kFan + wave * kLeavesPerWave + lane % kLeavesPerWave;
  };
  uint64_t lkey = 0;
  uint32_t lst = 0, lcnt = 0;
  const auto read_leaf = [&](uint32_t c0) {
    uint32_t gq;
    const uint32_t lf = leaf_of(c0, gq);
    lkey = 0;
    lst = lcnt = 0;
    if (gq < c.nl1 && lf < c.nleaves) {
      lkey = gptr(c.leaf_key)[lf];
      const uint2 sc = gptr(c.leaf_sc)[lf];
      lst = sc.x;
      lcnt = sc.y;
    }
  };
  read_leaf(blockIdx.x);
  if (blockIdx.x >= c.nl1 || *gptr(c.done)) return;
  NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
  uint64_t gt1 = 0, gt2 = 0, gt3 = 0;
  bool forced = false;
  const Sel s = sel_replay(c, passes + 1, passes, s_sc, &forced, &h0);
  uint64_t bkey = s.bkey;
  if (s.state == 2) {
    uint64_t best = 0;
    for (uint32_t j = tid; j < c.nl1; j += kPassThreads) {
      const uint64_t k = node_key(c, j);
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) s_wk[wave] = best;
    __syncthreads();
    best = 0;
    for (uint32_t w = 0; w < kPassWaves; ++w) best = s_wk[w] > best ? s_wk[w] : best;
    bkey = best;
  }
  if (PROF) gt1 = __builtin_amdgcn_s_memrealtime();
  if (blockIdx.x == 0 && tid == 0) {
    rs.bkey = bkey;
    // the first rounds start from windows over the whole key range and are
    // forced as a rule; later forced rounds ask for refinement passes
    rs.forced += forced && rs.rounds >= 2 ? 1u : 0u;
    // next round: fine bins of about 1/2048 of this round's key span
    uint32_t nx = bit_length(rs.kref0 - bkey + 1);
    nx = nx > 11u ? nx - 11u : 0u;
    rs.s0_next = nx < kMaxShift ? nx : kMaxShift;
  }
  // Nodes in chunks of kGatherNodes; lane l of a wave holds leaf l % 4 of the
  // wave's four leaves of node l / 4 of the chunk, so one read brings in all
  // its leaf records.  The points of the first kGatherHold hot leaves stay in
  // registers, the others are read again for writing; the workgroup takes one
  // range of the list per chunk (one global atomic).
  static_assert(kGatherNodes * kLeavesPerWave == 64, "one leaf record per lane");
  __shared__ uint32_t s_cnt, s_base;
  for (uint32_t c0 = blockIdx.x; c0 < c.nl1; c0 += kGatherNodes * gridDim.x) {
    if (c0 != blockIdx.x) read_leaf(c0);
    uint32_t gq;
    const uint32_t lf = leaf_of(c0, gq);
    const bool hot = lcnt != 0 && lkey >= bkey;  // an empty or absent leaf has key 0
    if (PROF) {
      pin_vgpr(lst, lcnt, (uint32_t)hot);
      if (!gt2) gt2 = __builtin_amdgcn_s_memrealtime();
    }
    if (tid == 0) s_cnt = 0;
    uint64_t rest = __ballot(hot);
    if (PROF) {
      const uint64_t hp = __ballot(hot);
      const uint32_t pts = rdlane(wave_incl_scan(hot ? lcnt : 0u), 63);
      if (lane == 0 && hp) {
        atomicAdd((unsigned long long *)gptr(c.prof) + kCtGaLeaves,
                  (unsigned long long)__popcll(hp));
        atomicAdd((unsigned long long *)gptr(c.prof) + kCtGaPoints, (unsigned long long)pts);
      }
    }
    float4 hp[kGatherHold];
    uint2 hr[kGatherHold];
    uint32_t hn[kGatherHold], hal[kGatherHold];
    uint64_t htk[kGatherHold];
    const uint32_t na = ALIAS ? c.r.na : 1u;
    // the held leaves' points: every lane loads, without a branch, so that
    // the loads are in flight together; a lane past the leaf's points, or of
    // a wave with fewer hot leaves, reads slot 0 and its values go unused
    // (hn[u] = 0 when there is no leaf)
#pragma unroll
    for (uint32_t u = 0; u < kGatherHold; ++u) {
      const bool have = rest != 0;
      const uint32_t j = have ? (uint32_t)__builtin_ctzll(rest) : 0u;
      rest &= rest - 1;
      const uint32_t st = rdlane(lst, j), cnt = have ? rdlane(lcnt, j) : 0u;
      hn[u] = cnt;
      const uint32_t idx = lane < cnt ? st + lane : 0u;
      hp[u] = gptr(c.P4)[idx];
      hr[u] = gptr(c.RO)[idx];
      hal[u] = kNoCell;  // lane a < na: cell a of the held leaf's bucket
      if (ALIAS && have && lane < na) hal[u] = gptr(c.leaf_al)[(size_t)rdlane(lf, j) * na + lane];
    }
    uint32_t mine = 0;
#pragma unroll
    for (uint32_t u = 0; u < kGatherHold; ++u) {
      htk[u] = __ballot(lane < hn[u] &&
                        (((uint64_t)__float_as_uint(hp[u].w) << 32) | ~hr[u].x) >= bkey);
      mine += (uint32_t)__popcll(htk[u]);
    }
    const uint64_t later = rest;  // hot leaves beyond the first kGatherHold: counted now,
    while (rest) {                // read again to be written
      const uint32_t j = (uint32_t)__builtin_ctzll(rest);
      rest &= rest - 1;
      const uint32_t st = rdlane(lst, j), cnt = rdlane(lcnt, j);
      bool take = false;
      if (lane < cnt) {
        const float d = ((const NSFPS_GLOBAL float *)gptr(c.P4 + st + lane))[3];
        take = (((uint64_t)__float_as_uint(d) << 32) | ~gptr(c.R)[st + lane]) >= bkey;
      }
      mine += (uint32_t)__popcll(__ballot(take));
    }
    __syncthreads();  // s_cnt is zero
    uint32_t base = 0;
    if (lane == 0 && mine) base = atomicAdd(&s_cnt, mine);
    __syncthreads();
    if (tid == 0) s_base = s_cnt ? atomicAdd(&rs.nlist, s_cnt) : 0u;
    __syncthreads();
    base = s_base + rdlane(base, 0);
    if (PROF && !gt3) gt3 = __builtin_amdgcn_s_memrealtime();
    // the list's pointers in vector registers: a pointer loaded again from
    // the arguments after a store would first wait for the store
    NSFPS_GLOBAL float4 *const LP = vgpr_ptr(gptr(c.list_p));
    NSFPS_GLOBAL uint2 *const LR = vgpr_ptr(gptr(c.list_r));
    NSFPS_GLOBAL uint32_t *const LC = vgpr_ptr(gptr(c.list_c));
    // arguments by value: a reference into hp / hr would make those arrays
    // memory (the compiler then keeps them in LDS)
    const auto put = [&](float4 p, uint2 ro, uint32_t al, uint64_t m) {
      if ((m >> lane) & 1u) {
        const uint32_t i = base + lanes_below(m);
        if (i < kListCap) {
          LP[i] = p;
          LR[i] = ro;
          // the point's own cell (its bucket's, when buckets have one cell;
          // a leaf may hold several buckets)
          LC[i] = pack_cell(cell_axis(c.r, 0, p.x), cell_axis(c.r, 1, p.y), cell_axis(c.r, 2, p.z));
          if (ALIAS)
            for (uint32_t a = 0; a < na; ++a) gptr(c.list_al)[(size_t)i * na + a] = rdlane(al, a);
        } else {
          rs.err = 1;
        }
      }
      base += (uint32_t)__popcll(m);
    };
#pragma unroll
    for (uint32_t u = 0; u < kGatherHold; ++u) put(hp[u], hr[u], hal[u], htk[u]);
    rest = later;
    while (rest) {
      const uint32_t j = (uint32_t)__builtin_ctzll(rest);
      rest &= rest - 1;
      const uint32_t st = rdlane(lst, j), cnt = rdlane(lcnt, j);
      float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
      uint2 ro = make_uint2(0u, 0u);
      uint32_t al = kNoCell;
      if (lane < cnt) {
        p = gptr(c.P4)[st + lane];
        ro = gptr(c.RO)[st + lane];
      }
      if (ALIAS && lane < na) al = gptr(c.leaf_al)[(size_t)rdlane(lf, j) * na + lane];
      const bool take = lane < cnt && (((uint64_t)__float_as_uint(p.w) << 32) | ~ro.x) >= bkey;
      put(p, ro, al, __ballot(take));
    }
    __syncthreads();  // s_base is read before the next chunk's claim
  }
  if (PROF && tid == 0 && blockIdx.x == 0) {
    unsigned long long *pw = (unsigned long long *)gptr(c.prof);
    atomicAdd(pw + kGaWinKeys, (unsigned long long)s.win);
    atomicAdd(pw + kGaListed, (unsigned long long)s.total);
    atomicMax(pw + kGaWinMax, (unsigned long long)s.win);
  }
  if (PROF && tid == 0 && gt3) {  // the first chunk's clocks; the writes: every chunk's rest
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    unsigned long long *pw = (unsigned long long *)gptr(c.prof);
    atomicAdd(pw + kGaTSel, (unsigned long long)(gt1 - gt0));
    atomicAdd(pw + kGaTLeaf, (unsigned long long)(gt2 - gt1));
    atomicAdd(pw + kGaTClaim, (unsigned long long)(gt3 - gt2));
    atomicAdd(pw + kGaTWrite, (unsigned long long)(t - gt3));
    atomicAdd(pw + kGaGroups, 1ull);
  }
}

// ---------------------------------------------------------------- the run

// One workgroup per cloud, eight waves (two per SIMD: the kernel is bound by
// instruction latency, which the second wave hides); every thread holds
// kOwnSlots list entries.  The list sits in LDS sorted by coarse cell (x >> sx, y >> sy,
// z >> sz; at most kCells of them) with the first entry of every coarse cell,
// so the entries inside a cube are found by walking, for each coarse (y, z)
// row the cube spans, the entries of its x range.
//
// The threshold argument is applied once more inside the list: a hot
// threshold H leaves at most HOT entries at or above it (64, or 128 where the
// points fill many buckets), and those are resolved in parallel phases.  Rank the remaining hot copies by key; copy j
// is "lowered" when the cube of a higher-ranked copy contains it and brings
// its distance down.  Every copy ranked above the first lowered one is a
// sample, in rank order: all copies ranked above it are samples too, a copy
// lowered by one of them started below it, and the rest of the list is below
// H.  The copies that are not lowered go on being samples past a lowered copy
// j as long as they exceed K_j, j's key once every copy above it that is not
// lowered has been applied (j's key can only be lower when their turn
// comes).  So a phase takes those samples at once, applies their cubes to
// the remaining copies, and ranks again, until no copy is >= max(H, B).  Then the
// hot run's samples are applied to every list entry (a
// sample with a small cube is applied by its copy's lanes walking its rows of
// the cell index, one with a large cube by every thread to its own entries)
// and the next hot set is chosen.  The run ends when no entry is >= B.
constexpr uint32_t kRunThreads = 512;
constexpr uint32_t kRunWaves = kRunThreads / 64;
constexpr uint32_t kOwnSlots = kListCap / kRunThreads;
// A hot set holds at most HOT copies (64, or 128 when no cells share
// buckets).  Each copy has kLanes threads, each comparing it with kCmp other
// copies; masks over the copies (or their ranks) take kWords 64-bit words.
template <uint32_t HOT>
struct HotSet {
  static constexpr uint32_t kLanes = kRunThreads / HOT;  // threads per hot copy (and per sample)
  static constexpr uint32_t kCmp = HOT / kLanes;         // copies each of them compares against
  static constexpr uint32_t kWords = HOT / 64;
  static constexpr uint32_t kCmpMask = kCmp >= 32 ? 0xffffffffu : (1u << kCmp) - 1u;
  static_assert((kLanes == 4 || kLanes == 8 || kLanes == 16) && (HOT == 64 || HOT == 128) &&
                    kCmp <= 32 && kCmp % 8 == 0,
                "the run kernel layout");
};
constexpr uint32_t kHotMax = 128;
constexpr uint32_t kSelBins = 256;
constexpr uint32_t kCells = 4096;    // coarse cells of the list's cell index
// Copies >= the hot threshold left after a phase that justify another phase.
// A phase accepts at least the first-ranked copy, so a value of at least the
// hot set's size means one phase per hot set, the copies left over going back
// to the next selection: ranking
// them again in further phases measured slower (uniform cube 8.36 ms per call
// at 12, 8.26 at 32, 8.20 at 48, 8.09 at kHot; LiDAR scan 5.38 / 5.26 / 5.19 /
// 5.14 ms).  Measured again on the later kernels, further phases at 32 gain
// only where phases accept few samples (quickstart, about 20 of 64: 0.711
// against 0.732 ms) and lose elsewhere (uniform cube 8.02 against 7.70 ms,
// clustered cloud 73.5 against 69.8); allowing them only after a phase of at
// most 24 samples still cost the uniform cube 3 % and the clustered cloud 4 %.
constexpr uint32_t kPhaseMin = kHotMax;
// Cubes over more coarse rows, or with more list entries in one lane's rows,
// are applied by every thread to its own entries instead of walked.  Rows
// below 64 keep the walk's row arithmetic exact.  With a lane's rows walked
// as one list, 16 rows (two a lane) measured best: per call, uniform cube
// 7.73 ms at 16 rows and 7.88 at 24, LiDAR scan 4.49 and 4.50, clustered
// 71.0 and 73.4 (row by row at 24 rows: 7.94, 4.75, 69.3).
constexpr uint32_t kWalkRows = 16;
constexpr uint32_t kWalkLaneEntries = 16;
constexpr uint32_t kDenseWalkRows = 12;  // 128-copy sets on dense clouds
static_assert(kWalkRows <= 64, "the walk's row arithmetic");
// With hot sets of 128 copies a sample has 4 lanes: ROWS rows (16, or 12 for
// dense clouds) and 24 entries a lane.  Measured per call (rows / entries):
// uniform cube 7.21 ms at 16 / 16, 16 / 24 and 16 / 32, 7.26 at 12 / 24,
// 7.38 at 24 / 16, 8.47 at 8 / 16; clustered cloud 62.1, 61.6, 61.6, 60.5,
// 63.8 and 60.5 ms.  The rows' gain is the lane's row slots (3 against 4 in
// the walk's entry-to-row mapping): a limit of 12 rows read at run time, the
// slots still sized for 16, left the clustered cloud at 61.9 ms.
template <uint32_t HOT, uint32_t ROWS>
struct WalkLimits {
  static constexpr uint32_t kRows = ROWS;
  static constexpr uint32_t kLaneEntries = HOT == 128 ? 24 : kWalkLaneEntries;
  static_assert(kRows <= 64, "the walk's row arithmetic");
};
constexpr uint32_t kCellsPerThread = kCells / kRunThreads;
static_assert(kCellsPerThread % 4 == 0, "the cell scan reads whole uint4s");

// Phase clocks of the run kernel (s_memtime cycles of wave 0, summed over
// rounds into the cloud's profile words) when PROF is set.
enum : uint32_t {
  kRpLoad = 0, kRpSelect, kRpGather, kRpPhases, kRpApply, kRpTail, kRpBig, kRpRank,
  kRpPicks = 8, kRpRounds, kRpHotRounds, kRpPhaseCount, kRpWalk, kRpPublish,
  kRpRtLoad = 14,  // s_memrealtime ticks (100 MHz) from the kernel's start to the end of the load
  kRpRtTotal = 15, //   and to the kernel's end
  kRpWords = 16,
  // words kept past the first kRpWords (local words 16.., profile words
  // 28.., after the work counters of the passes): the wait at the barrier
  // after the walk, the pass over entries whose bucket has several cells,
  // and those entries summed over hot sets
  kRpWalkWait = 16, kRpAlias = 17, kRpAliasN = 18, kRpLocal = 19, kRpExtraAt = 28
};

// Cube corners of a sample: cell qc, half-widths h, clipped to the grid.
__device__ __forceinline__ void cube_corners(uint32_t qc, uint32_t h, uint32_t b0, uint32_t b1,
                                             uint32_t b2, uint32_t &lo_c, uint32_t &hi_c) {
  const uint32_t qcx = qc & 1023u, qcy = (qc >> 10) & 1023u, qcz = qc >> 20;
  const uint32_t g0 = h & 1023u, g1 = (h >> 10) & 1023u, g2 = h >> 20;
  lo_c = pack_cell(qcx > g0 ? qcx - g0 : 0u, qcy > g1 ? qcy - g1 : 0u, qcz > g2 ? qcz - g2 : 0u);
  hi_c = pack_cell(min(qcx + g0, b0 - 1), min(qcy + g1, b1 - 1), min(qcz + g2, b2 - 1));
}

// Cube half-width of a sample with distance D on axis a (src/yuezu_fps.cpp:
// 564-570), clipped to blocks - 1 (at or beyond the grid it selects the same
// cells).  The half-width is monotone in D: below the last of the range's
// thresholds it is the number of thresholds <= D (no square root or
// division); above it, the reference's arithmetic (correctly rounded sqrtf
// and division, as on the host that derived the thresholds).
__device__ __forceinline__ uint32_t half_axis(const RangeDev &r, int a, float D) {
  uint32_t h = 0;
#pragma unroll
  for (uint32_t k = 0; k < kCubeThr; ++k) h += D >= r.cube_thr[a][k] ? 1u : 0u;
  if (h == kCubeThr) h = min((uint32_t)cube_half(D, r.bsize[a], r.blocks[a]), r.blocks[a] - 1);
  return h;
}

// The three half-widths packed 10 bits per axis.
__device__ __forceinline__ uint32_t packed_halves(const RangeDev &r, float D) {
  return half_axis(r, 0, D) | (half_axis(r, 1, D) << 10) | (half_axis(r, 2, D) << 20);
}

// The first three thresholds of every axis, in scalar registers.  Below the
// third of every axis (half-widths of at most 2: the common case once cubes
// are small) the packed half-widths take two comparisons per axis.
struct SmallHalves {
  float t[3][3];
  __device__ __forceinline__ explicit SmallHalves(const RangeDev &r) {
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int k = 0; k < 3; ++k) t[a][k] = r.cube_thr[a][k];
  }
  __device__ __forceinline__ bool covers(float D) const {
    return D < t[0][2] && D < t[1][2] && D < t[2][2];
  }
  __device__ __forceinline__ uint32_t packed(float D) const {
    uint32_t h = 0;
#pragma unroll
    for (int a = 0; a < 3; ++a)
      h |= ((D >= t[a][0] ? 1u : 0u) + (D >= t[a][1] ? 1u : 0u)) << (10 * a);
    return h;
  }
};

// LDS slot of hot copy i.  Lane q of a copy's group compares against copies
// q * kCmp + u; the kLanes copies read together for one u sit side by side,
// so one read by a wave touches distinct banks.
template <uint32_t HOT>
__device__ __forceinline__ uint32_t hot_slot(uint32_t i) {
  return (i % HotSet<HOT>::kCmp) * HotSet<HOT>::kLanes + i / HotSet<HOT>::kCmp;
}

// Sum / minimum over the L lanes of a group (aligned lanes).
template <uint32_t L>
__device__ __forceinline__ uint32_t group_sum(uint32_t v) {
  v += dpp_mov<kDppQuad1032>(v);
  v += dpp_mov<kDppQuad2301>(v);
  if (L >= 8) v += dpp_mov<kDppHalfMirror>(v);  // lane i and 7 - i: the other quad
  if (L >= 16) v += dpp_mov<kDppMirror>(v);     // lane i and 15 - i: the other half
  return v;
}
template <uint32_t L>
__device__ __forceinline__ uint32_t group_min(uint32_t v) {
  v = min(v, dpp_mov<kDppQuad1032>(v));
  v = min(v, dpp_mov<kDppQuad2301>(v));
  if (L >= 8) v = min(v, dpp_mov<kDppHalfMirror>(v));
  if (L >= 16) v = min(v, dpp_mov<kDppMirror>(v));
  return v;
}

// Bin shift of a hot-threshold histogram whose kSelBins bins end at kref and
// cover every key down to bkey.
__device__ __forceinline__ uint32_t sel_shift(uint64_t kref, uint64_t bkey) {
  const uint32_t n = bit_length(kref - bkey);
  return n > 8u ? n - 8u : 0u;
}

// Counts this thread's live keys (>= bkey) into histogram H (window kref, S);
// every live key is <= kref.
__device__ __forceinline__ void hist_live(const float *d, const uint32_t *lo, uint64_t bkey,
                                          uint64_t kref, uint32_t S, uint32_t *H,
                                          NSFPS_GLOBAL uint32_t *err) {
#pragma unroll
  for (uint32_t s = 0; s < kOwnSlots; ++s) {
    const uint64_t key = ((uint64_t)__float_as_uint(d[s]) << 32) | lo[s];
    if (lo[s] != 0u && key >= bkey) {
      if (key <= kref) atomicAdd(&H[(uint32_t)((kref - key) >> S)], 1u);
      else *err = 3;  // cannot happen (kref bounds every live key)
    }
  }
}

// The run of one cloud by one workgroup of kRunThreads.  ALIAS: cells share
// buckets.  A sample then updates
// every entry whose bucket has a cell inside its cube (src/yuezu_fps.cpp:
// 573-597).  The walk finds entries by their own cell; the entries whose
// bucket has further cells are few and listed apart, and after each walk
// every one of them is tested against every sample of the hot set; the
// phases test every cell of a hot copy's bucket.  HOT: copies per hot set;
// ROWS: the walk's row limit.  WHOLE (clouds in few buckets): the list's
// cell box is taken at its load, and a large-cube sample whose cube holds it
// is applied to every entry with no cell test.
template <bool PROF, bool ALIAS, uint32_t HOT, uint32_t ROWS, bool WHOLE>
__device__ __forceinline__ void run_list(const CloudDev &c) {
  static_assert(!(WHOLE && ALIAS), "the list box is of the entries' own cells");
  // the alias pass holds one sample per lane
  static_assert(!ALIAS || HOT == 64, "shared buckets take hot sets of 64");
  constexpr uint32_t kHot = HOT, kCopyLanes = HotSet<HOT>::kLanes, kCmp = HotSet<HOT>::kCmp,
                     kWords = HotSet<HOT>::kWords;
  __shared__ uint4 s_pc[kListCap];      // sorted list: {x, y, z, pack11(cell)}
  __shared__ uint32_t s_dd[kListCap];   // its distances (bits)
  __shared__ uint2 s_rk[kListCap];      // its {~logical rank, input row}
  __shared__ uint4 s_hq[2][kHot];       // hot copies at hot_slot<HOT>(i), one buffer per phase parity:
                                        //   {pack11(cube lo), pack11(cube hi) | guards, ~rank,
                                        //   distance bits}; key 0 once taken
  __shared__ __align__(16) uint32_t s_rank[kHot];  // rank of each hot copy in the phase
  __shared__ unsigned long long s_lowm[2][kWords];  // bit r: the copy ranked r is lowered
  __shared__ unsigned long long s_lowc[2][kWords];  // bit j: hot copy j is lowered
  __shared__ unsigned long long s_kmax[2];  // the largest bound K_j of a lowered copy
  __shared__ uint4 s_hx[kHot];          // hot copies: {cell, pack11(cell) | guards, pack11(cell),
                                        //   half-widths}
  __shared__ uint4 s_hp[kHot];          // hot copies: {x, y, z, row}
  __shared__ uint4 s_rp[kHot];          // accepted hot copies at their slot: {x, y, z, row}
  __shared__ uint2 s_rc[kHot];          //   cube corners, pack11 (hi with guards)
  __shared__ __align__(16) uint32_t s_cell[kCells + 4];  // first entry of each coarse cell
  __shared__ uint32_t s_big[2 * kWords];                // samples with large cubes
  __shared__ uint32_t s_bigw[WHOLE ? 2 * kWords : 1];  // WHOLE: those whose cube holds the list box
  __shared__ __align__(16) uint32_t s_sel[3][kSelBins];  // hot-threshold histograms, rotating
  __shared__ uint32_t s_nhot;
  __shared__ unsigned long long s_kmr;   // largest key of a hot copy left unaccepted
  __shared__ uint32_t s_wn[2 * kRunWaves];  // wave sums of the two cell-count scans
  __shared__ uint32_t s_wr[2][kRunWaves][2];
  __shared__ uint32_t s_geo[4];  // coarse cell shifts (x | y << 8 | z << 16), ncx, ncy
  // ALIAS: the cells of each entry's bucket (pack11, kNoCell-padded, at the
  // entry's sorted position), the sorted positions of the entries whose
  // bucket has several cells, the hot copies' positions, and the hot set's
  // samples by output order: cube corners (pack11; hi with guards) and x, y, z
  __shared__ uint32_t s_al[ALIAS ? kListCap * kMaxAlias : 1];
  // ALIAS: a second coarse cell index, of records {x, y, z, pack11(cell)} of
  // the entries' other cells (the cells of their bucket besides their own)
  // and the entry each belongs to, so that the walk reaches an entry through
  // any cell of its bucket; entries whose records do not fit go to a pass
  // over every sample of the hot set (s_alist)
  __shared__ __align__(16) uint32_t s_xc[ALIAS ? kCells + 4 : 4];
  __shared__ uint4 s_xp[ALIAS ? kListCap : 1];
  __shared__ uint32_t s_xe[ALIAS ? kListCap : 1];
  __shared__ uint32_t s_nx;
  __shared__ uint32_t s_alist[ALIAS ? kListCap : 1];
  __shared__ uint32_t s_nal;
  __shared__ uint32_t s_hpos[kHot];
  // WHOLE: the list's cell box, per axis the largest cell and 1023 - the smallest
  __shared__ uint32_t s_lb[WHOLE ? 6 : 1];
  __shared__ uint2 s_sbox[ALIAS ? kHot : 1];
  __shared__ float4 s_spos[ALIAS ? kHot : 1];
  const uint64_t rt0 = PROF ? __builtin_amdgcn_s_memrealtime() : 0;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
  // every input of the run is read at once: the done flag, the run state and
  // the whole list buffer (entries at or beyond the list length are stale
  // and ignored)
  const uint32_t done_in = *gptr(c.done);
  const uint32_t nlist = min(rs.nlist, kListCap);
  const uint64_t bkey = rs.bkey, kref0 = rs.kref0;
  float4 P[kOwnSlots];
  uint2 R[kOwnSlots];
  uint32_t C[kOwnSlots];
  const uint32_t na = ALIAS ? c.r.na : 1u;
  uint32_t AL[ALIAS ? kOwnSlots : 1][kMaxAlias];
#pragma unroll
  for (uint32_t s = 0; s < kOwnSlots; ++s) {
    const uint32_t i = s * kRunThreads + tid;
    P[s] = gptr(c.list_p)[i];
    R[s] = gptr(c.list_r)[i];
    C[s] = gptr(c.list_c)[i];
    if (ALIAS) {
#pragma unroll
      for (uint32_t a = 0; a < kMaxAlias; ++a)
        AL[s][a] = a < na && i < nlist ? gptr(c.list_al)[(size_t)i * na + a] : kNoCell;
    }
  }
  uint64_t pf[kRpLocal] = {}, tl = 0;
  if (PROF) tl = __builtin_amdgcn_s_memtime();
#define NSFPS_RMARK(ph)                                  \
  do {                                                   \
    if (PROF) {                                          \
      const uint64_t t_ = __builtin_amdgcn_s_memtime();  \
      pf[ph] += t_ - tl;                                 \
      tl = t_;                                           \
    }                                                    \
  } while (0)
  const uint32_t b0 = c.r.blocks[0], b1 = c.r.blocks[1], b2 = c.r.blocks[2];
  // coarse cells (x >> sx, y >> sy, z >> sz), at most kCells of them: the
  // longest coarse axis is halved until they fit
  uint32_t sx = 0, sy = 0, sz = 0;
  while (true) {
    const uint32_t ex = ((b0 - 1) >> sx) + 1, ey = ((b1 - 1) >> sy) + 1, ez = ((b2 - 1) >> sz) + 1;
    if (ex * ey * ez <= kCells) break;
    if (ex >= ey && ex >= ez) ++sx;
    else if (ey >= ez) ++sy;
    else ++sz;
  }
  const uint32_t ncx = ((b0 - 1) >> sx) + 1, ncy = ((b1 - 1) >> sy) + 1;
  for (uint32_t j = tid; j < kCells + 4; j += kRunThreads) {
    s_cell[j] = 0;
    if (ALIAS) s_xc[j] = 0;
  }
  if (tid < kSelBins) {
    s_sel[0][tid] = 0;
    s_sel[1][tid] = 0;
  }
  if (tid < kHot) s_hq[0][tid] = make_uint4(0u, 0u, 0u, 0u);  // key 0: an unused slot
  if (WHOLE && tid < 6) s_lb[tid] = 0;
  if (tid == 0) {
    s_nhot = 0;
    if (ALIAS) {
      s_nal = 0;
      s_nx = 0;
    }
    s_geo[0] = sx | (sy << 8) | (sz << 16);
    s_geo[1] = ncx;
    s_geo[2] = ncy;
  }
  __syncthreads();
  if (done_in) return;  // uniform: the whole workgroup leaves

  // ---- list -> LDS in coarse-cell order (counting sort)
  {
    const auto coarse = [&](uint32_t c10) {
      return (((c10 >> 20) >> sz) * ncy + (((c10 >> 10) & 1023u) >> sy)) * ncx +
             ((c10 & 1023u) >> sx);
    };
    uint32_t G[kOwnSlots], K[kOwnSlots];
    // ALIAS: per entry, its other cells' number and whether their records
    // fit the second index, and each record's place among its coarse cell's
    uint32_t NO[ALIAS ? kOwnSlots : 1] = {};
    bool XI[ALIAS ? kOwnSlots : 1] = {};
    uint32_t XK[ALIAS ? kOwnSlots : 1][kMaxAlias];
#pragma unroll
    for (uint32_t s = 0; s < kOwnSlots; ++s) {
      const uint32_t i = s * kRunThreads + tid;
      if (i < nlist) {
        G[s] = coarse(C[s]);
        K[s] = atomicAdd(&s_cell[G[s]], 1u);
        if (ALIAS) {
          uint32_t no = 0;
#pragma unroll
          for (uint32_t a = 0; a < kMaxAlias; ++a) no += AL[s][a] != kNoCell && AL[s][a] != C[s];
          NO[s] = no;
          if (no && atomicAdd(&s_nx, no) + no <= kListCap) {
            XI[s] = true;
#pragma unroll
            for (uint32_t a = 0; a < kMaxAlias; ++a)
              if (AL[s][a] != kNoCell && AL[s][a] != C[s]) XK[s][a] = atomicAdd(&s_xc[coarse(AL[s][a])], 1u);
          }
        }
      }
    }
    __syncthreads();
    {  // exclusive scan of the cell counts, kCellsPerThread consecutive cells per thread
      constexpr uint32_t kV = kCellsPerThread / 4;
      uint4 v[kV];
      uint32_t sum = 0;
#pragma unroll
      for (uint32_t j = 0; j < kV; ++j) {
        v[j] = reinterpret_cast<const uint4 *>(s_cell)[kV * tid + j];
        sum += v[j].x + v[j].y + v[j].z + v[j].w;
      }
      uint32_t tot;
      uint32_t pre = block_excl_scan<kRunWaves>(sum, s_wn, &tot);
#pragma unroll
      for (uint32_t j = 0; j < kV; ++j) {
        const uint4 o = make_uint4(pre, pre + v[j].x, pre + v[j].x + v[j].y,
                                   pre + v[j].x + v[j].y + v[j].z);
        pre += v[j].x + v[j].y + v[j].z + v[j].w;
        reinterpret_cast<uint4 *>(s_cell)[kV * tid + j] = o;
      }
      if (tid == 0) s_cell[kCells] = tot;
      if (ALIAS) {  // the second index's counts, the same way (its own wave sums)
        uint32_t sum2 = 0;
#pragma unroll
        for (uint32_t j = 0; j < kV; ++j) {
          v[j] = reinterpret_cast<const uint4 *>(s_xc)[kV * tid + j];
          sum2 += v[j].x + v[j].y + v[j].z + v[j].w;
        }
        uint32_t tot2;
        uint32_t pre2 = block_excl_scan<kRunWaves>(sum2, s_wn + kRunWaves, &tot2);
#pragma unroll
        for (uint32_t j = 0; j < kV; ++j) {
          const uint4 o = make_uint4(pre2, pre2 + v[j].x, pre2 + v[j].x + v[j].y,
                                     pre2 + v[j].x + v[j].y + v[j].z);
          pre2 += v[j].x + v[j].y + v[j].z + v[j].w;
          reinterpret_cast<uint4 *>(s_xc)[kV * tid + j] = o;
        }
        if (tid == 0) s_xc[kCells] = tot2;
      }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t s = 0; s < kOwnSlots; ++s) {
      const uint32_t i = s * kRunThreads + tid;
      if (i < nlist) {
        const uint32_t pos = s_cell[G[s]] + K[s];
        s_pc[pos] = make_uint4(__float_as_uint(P[s].x), __float_as_uint(P[s].y),
                               __float_as_uint(P[s].z), pack11(C[s]));
        s_dd[pos] = __float_as_uint(P[s].w);
        s_rk[pos] = make_uint2(~R[s].x, R[s].y);
        if (ALIAS) {
          // the bucket's cells (pack11), and the records of the other cells
          // in the second index, or the entry in the pass's list
#pragma unroll
          for (uint32_t a = 0; a < kMaxAlias; ++a) {
            s_al[pos * kMaxAlias + a] = pack11(AL[s][a]);
            if (XI[s] && AL[s][a] != kNoCell && AL[s][a] != C[s]) {
              const uint32_t dst = s_xc[coarse(AL[s][a])] + XK[s][a];
              s_xp[dst] = make_uint4(__float_as_uint(P[s].x), __float_as_uint(P[s].y),
                                     __float_as_uint(P[s].z), pack11(AL[s][a]));
              s_xe[dst] = pos;
            }
          }
          if (NO[s] && !XI[s]) s_alist[atomicAdd(&s_nal, 1u)] = pos;
        }
      }
    }
    __syncthreads();
  }
  // owned entries: sorted entry s * kRunThreads + tid; an empty slot has
  // distance 0 and key 0 and is never live
  float x[kOwnSlots], y[kOwnSlots], z[kOwnSlots], d[kOwnSlots];
  // own cells in pack11 form (the box tests of samples with large cubes) and
  // 10 bits per axis (a sample's cube centre)
  uint32_t lo[kOwnSlots], row[kOwnSlots], cc[kOwnSlots], c11[kOwnSlots];
#pragma unroll
  for (uint32_t s = 0; s < kOwnSlots; ++s) {
    const uint32_t i = s * kRunThreads + tid;
    uint4 e0 = make_uint4(0u, 0u, 0u, 0u);
    uint2 e1 = make_uint2(0u, 0u);
    uint32_t e2 = 0;
    if (i < nlist) {
      e0 = s_pc[i];
      e1 = s_rk[i];
      e2 = s_dd[i];
    }
    x[s] = __uint_as_float(e0.x);
    y[s] = __uint_as_float(e0.y);
    z[s] = __uint_as_float(e0.z);
    d[s] = __uint_as_float(e2);
    lo[s] = e1.x;
    row[s] = e1.y;
    c11[s] = e0.w;
    cc[s] = (e0.w & 1023u) | (((e0.w >> 11) & 1023u) << 10) | ((e0.w >> 22) << 20);
  }
  if (WHOLE) {  // the list's cell box (every entry's cell lies in it)
    uint32_t bmax[3] = {0u, 0u, 0u}, bmin[3] = {0u, 0u, 0u};  // bmin: 1023 - the smallest
#pragma unroll
    for (uint32_t s = 0; s < kOwnSlots; ++s) {
      if (s * kRunThreads + tid < nlist) {
#pragma unroll
        for (uint32_t a = 0; a < 3; ++a) {
          const uint32_t v = (cc[s] >> (10 * a)) & 1023u;
          bmax[a] = max(bmax[a], v);
          bmin[a] = max(bmin[a], 1023u - v);
        }
      }
    }
#pragma unroll
    for (uint32_t a = 0; a < 3; ++a) {
      bmax[a] = wave_max_u32(bmax[a]);
      bmin[a] = wave_max_u32(bmin[a]);
    }
    if (lane == 0) {
#pragma unroll
      for (uint32_t a = 0; a < 3; ++a) {
        atomicMax(&s_lb[a], bmax[a]);
        atomicMax(&s_lb[3 + a], bmin[a]);
      }
    }
  }
  uint32_t it = *gptr(c.iter);
  const uint32_t m = c.m;
  NSFPS_GLOBAL int32_t *const out = gptr(c.out);
  NSFPS_GLOBAL float4 *const pick_p = gptr(c.pick_p);
  NSFPS_GLOBAL uint2 *const pick_c = gptr(c.pick_c);
  NSFPS_GLOBAL uint32_t *const err = &rs.err;
  uint32_t np = 0;
  bool done = false;
  // The first hot set's histogram: every key is <= kref0 (keys only decrease).
  // Later ones are counted right after each hot set's walk.
  uint64_t kref = kref0 > bkey ? kref0 : bkey;
  uint32_t S = sel_shift(kref, bkey);
  hist_live(d, lo, bkey, kref, S, s_sel[0], err);
  __syncthreads();
  // WHOLE: the list box's corners in pack11 form (an empty list leaves them
  // crossed, and no cube then holds them both)
  uint32_t lb_lo = 0, lb_hi = 0;
  if (WHOLE) {
    lb_lo = pack11(pack_cell(1023u - s_lb[3], 1023u - s_lb[4], 1023u - s_lb[5]));
    lb_hi = pack11(pack_cell(s_lb[0], s_lb[1], s_lb[2]));
  }
  // coarse grid, kept in vector registers (the scalar file is full in the walk)
  const uint32_t gsh = s_geo[0], gx = s_geo[1], gy = s_geo[2];
  const uint32_t gsx = gsh & 255u, gsy = (gsh >> 8) & 255u, gsz = gsh >> 16;
  NSFPS_RMARK(kRpLoad);
  if (PROF) pf[kRpRtLoad] = __builtin_amdgcn_s_memrealtime() - rt0;
  while (true) {
    uint64_t key[kOwnSlots];
    bool live[kOwnSlots];
#pragma unroll
    for (uint32_t s = 0; s < kOwnSlots; ++s) {
      key[s] = ((uint64_t)__float_as_uint(d[s]) << 32) | lo[s];
      live[s] = lo[s] != 0u && key[s] >= bkey;
    }
    // ---- hot threshold.  Histogram 0 (window kref, S) holds every live key;
    // windows of kSelBins bins are refined 8 bits at a time; buffer i % 3 of
    // step i was zeroed a step (or a hot set) before, and every wave scans it
    // itself: one barrier per refinement step.
    uint64_t hth = bkey;
    uint32_t nlive = 0;
    {
      uint64_t wref = kref;
      uint32_t wS = S, cap = kHot;
      for (uint32_t step = 0;; ++step) {
        const uint4 hv = reinterpret_cast<const uint4 *>(s_sel[step % 3])[lane];
        const uint32_t tot = hv.x + hv.y + hv.z + hv.w;
        const uint32_t incl = wave_incl_scan(tot);
        if (step == 0) {
          nlive = rdlane(incl, 63);
          if (nlive <= kHot) break;  // every live entry is hot (or none is left)
        }
        const uint64_t over = __ballot(incl > cap);  // running totals only grow
        if (!over) {  // cannot happen (a refined window holds more than cap keys)
          *err = 4;
          nlive = 0;
          break;
        }
        const uint32_t c0 = incl - tot, c1 = c0 + hv.x, c2 = c1 + hv.y, c3 = c2 + hv.z;
        const uint32_t jj = c1 > cap ? 0u : c2 > cap ? 1u : c3 > cap ? 2u : 3u;
        const uint32_t bf = c1 > cap ? c0 : c2 > cap ? c1 : c3 > cap ? c2 : c3;
        const uint32_t L = (uint32_t)__builtin_ctzll(over);
        const uint32_t bs = 4 * L + rdlane(jj, L), before = rdlane(bf, L);
        if (before >= cap / 2 || wS == 0) {
          hth = wref - ((uint64_t)bs << wS) + 1;
          break;
        }
        wref -= (uint64_t)bs << wS;
        cap -= before;
        wS = wS >= 8u ? wS - 8u : 0u;
        uint32_t *H = s_sel[(step + 1) % 3];
#pragma unroll
        for (uint32_t s = 0; s < kOwnSlots; ++s) {
          if (live[s] && key[s] <= wref) {
            const uint64_t bb = (wref - key[s]) >> wS;
            if (bb < kSelBins) atomicAdd(&H[(uint32_t)bb], 1u);
          }
        }
        if (tid < kSelBins) s_sel[(step + 2) % 3][tid] = 0;
        __syncthreads();
      }
      hth = hth > bkey ? hth : bkey;
    }
    if (nlive == 0) break;  // every key is below B: the run ends
    NSFPS_RMARK(kRpSelect);
    // ---- hot copies -> LDS, placed by an LDS counter; then one wave computes
    // every copy's cube (one pass over the cube code rather than one per wave
    // holding a hot entry).  Unused slots were cleared during the previous
    // hot set's walk (key 0).
    {
      uint64_t bal[kOwnSlots];
      uint32_t tot = 0;
#pragma unroll
      for (uint32_t s = 0; s < kOwnSlots; ++s) {
        bal[s] = __ballot(live[s] && key[s] >= hth);
        tot += (uint32_t)__popcll(bal[s]);
      }
      uint32_t base = 0;
      if (lane == 0 && tot) base = atomicAdd(&s_nhot, tot);
      base = rdlane(base, 0);
      // raw copies: {cell, ~rank, distance} and {x, y, z, row}
#pragma unroll
      for (uint32_t s = 0; s < kOwnSlots; ++s) {
        const uint32_t hi = base + lanes_below(bal[s]);
        base += (uint32_t)__popcll(bal[s]);
        if ((bal[s] >> lane) & 1u) {
          if (hi < kHot) {
            s_hx[hi] = make_uint4(cc[s], lo[s], __float_as_uint(d[s]), 0u);
            s_hp[hi] = make_uint4(__float_as_uint(x[s]), __float_as_uint(y[s]),
                                  __float_as_uint(z[s]), row[s]);
            if (ALIAS) s_hpos[hi] = s * kRunThreads + tid;
          } else {  // cannot happen (at most kHot keys are >= the hot threshold)
            *err = 2;
          }
        }
      }
      if (tid < 2 * kWords) s_big[tid] = 0;
      if (WHOLE && tid < 2 * kWords) s_bigw[WHOLE ? tid : 0] = 0;
      if (tid == 0) {
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) {
          s_lowm[0][w] = 0;
          s_lowc[0][w] = 0;
        }
        s_kmax[0] = 0;
        s_kmr = 0;
      }
      __syncthreads();
      if (tid < min(s_nhot, kHot)) {  // the first kHot / 64 waves, a copy a lane
        const uint4 hx = s_hx[tid];
        const float D = __uint_as_float(hx.z);
        const SmallHalves sh(c.r);
        uint32_t h;
        if (sh.covers(D)) h = sh.packed(D);
        else h = packed_halves(c.r, D);
        uint32_t lo_c, hi_c;
        cube_corners(hx.x, h, b0, b1, b2, lo_c, hi_c);
        s_hq[0][hot_slot<HOT>(tid)] = make_uint4(pack11(lo_c), pack11(hi_c) | kGuards, hx.y, hx.z);
        s_hx[tid] = make_uint4(hx.x, pack11(hx.x) | kGuards, pack11(hx.x), h);
      }
      __syncthreads();
    }
    NSFPS_RMARK(kRpGather);
    // ---- phases: thread (j, q) works for hot copy j against copies
    // kCmp q .. kCmp q + kCmp - 1.  A copy's group keeps what the walk needs
    // once the copy is accepted: its sample index and cube.
    const uint32_t hj = tid / kCopyLanes, hq = tid % kCopyLanes;
    const uint32_t room = m - it;  // samples left (>= 1)
    // Per phase, two barriers: after the ranks (the accepted prefix is known),
    // and after the next buffer of hot copies is written.
    uint32_t npk = 0, stop = 0, ph = 0;
    bool my_acc = false;
    uint64_t my_key = 0;  // the copy's key at the last phase (0: none, or accepted)
    uint32_t my_out = 0, my_qc = 0, my_hh = 0;
    // ALIAS: the cells of copy j's bucket (pack11; kNoCell's packing never
    // lies in a clipped box).  Unused slots read some entry's cells: they
    // have key 0 and are never compared.
    uint32_t ja[kMaxAlias];
    if (ALIAS) {
      const uint32_t pj = s_hpos[hj] & (kListCap - 1u);
#pragma unroll
      for (uint32_t a = 0; a < kMaxAlias; ++a)
        ja[a] = a < na ? s_al[pj * kMaxAlias + a] : pack11(kNoCell);
    }
    // 1 when (a cell of the bucket of) copy j lies in the box of pack11
    // corners lo, hig; two cells per bucket (grids near powers of two) take
    // two tests, more take all kMaxAlias (padding never lies in a box)
    const bool na2 = na == 2;
    const auto j_in = [&](uint32_t cg, uint32_t c11, uint32_t lo, uint32_t hig) -> uint32_t {
      if (!ALIAS) return in_box11(cg, c11, lo, hig);
      uint32_t r = in_box11(ja[0] | kGuards, ja[0], lo, hig) | in_box11(ja[1] | kGuards, ja[1], lo, hig);
      if (!na2) {
#pragma unroll
        for (uint32_t a = 2; a < kMaxAlias; ++a) r |= in_box11(ja[a] | kGuards, ja[a], lo, hig);
      }
      return r;
    };
    while (true) {
      const uint4 me = s_hq[ph][hot_slot<HOT>(hj)];
      const uint4 mx = s_hx[hj];
      const uint64_t mkey = ((uint64_t)me.w << 32) | me.z;
      my_key = mkey;
      const bool remj = mkey != 0;  // copies taken earlier, and unused slots, have key 0
      // bit u of cand: copy kCmp q + u is remaining, ranked above j, and its
      // cube holds j.  The kCmp copies of this lane are read 8 at a time, all
      // loads of a chunk issued before any use.
      uint32_t cnt = 0, cand = 0;
#pragma unroll
      for (uint32_t c0 = 0; c0 < kCmp; c0 += 8) {
        uint4 og[8];
#pragma unroll
        for (uint32_t v = 0; v < 8; ++v) og[v] = s_hq[ph][kCopyLanes * (c0 + v) + hq];  // copy kCmp hq + c0 + v
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t v = 0; v < 8; ++v) {
          const uint32_t gt = (uint32_t)((((uint64_t)og[v].w << 32) | og[v].z) > mkey);
          cnt += gt;
          cand |= (gt & j_in(mx.y, mx.z, og[v].x, og[v].y)) << (c0 + v);
        }
      }
      uint32_t low = 0;
      if (cand) {  // rare: the exact distance decides
        const uint4 pj = s_hp[hj];
        for (uint32_t cm = cand; cm; cm &= cm - 1) {
          const uint32_t u = (uint32_t)__builtin_ctz(cm);
          const uint4 pi = s_hp[hq * kCmp + u];
          const float dd = sqdist(__uint_as_float(pj.x), __uint_as_float(pj.y),
                                  __uint_as_float(pj.z), __uint_as_float(pi.x),
                                  __uint_as_float(pi.y), __uint_as_float(pi.z));
          low |= dd < __uint_as_float(me.w) ? 1u : 0u;
        }
      }
      const uint32_t rank = group_sum<kCopyLanes>(cnt);
      const bool lowered = group_sum<kCopyLanes>(low) != 0;
      const bool rep = remj && hq == 0;
      const bool ge = mkey >= hth;
      if (rep) s_rank[hj] = rank;
      if (hq == 0 && !remj) s_rank[hj] = kHot;  // never accepted
      if (rep && lowered) {
        atomicOr(&s_lowm[ph][rank >> 6], 1ull << (rank & 63u));
        atomicOr(&s_lowc[ph][hj >> 6], 1ull << (hj & 63u));
      }
      const uint32_t wge = (uint32_t)__popcll(__ballot(rep && ge));
      const uint32_t wnz = (uint32_t)__popcll(__ballot(rep && ge && me.w != 0u));
      if (lane == 0) {
        s_wr[ph][wave][0] = wge;
        s_wr[ph][wave][1] = wnz;
      }
      if (tid == 0) {
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) {
          s_lowm[ph ^ 1][w] = 0;
          s_lowc[ph ^ 1][w] = 0;
        }
        s_kmax[ph ^ 1] = 0;
      }
      __syncthreads();
      NSFPS_RMARK(kRpRank);
      // copies >= the hot threshold with distance > 0 are ranks 0 .. nnz - 1
      unsigned long long lowm[kWords], lowany = 0;
#pragma unroll
      for (uint32_t w = 0; w < kWords; ++w) {
        lowm[w] = s_lowm[ph][w];
        lowany |= lowm[w];
      }
      uint32_t nge = 0, nnz = 0;
#pragma unroll
      for (uint32_t w = 0; w < kRunWaves; ++w) {
        nge += s_wr[ph][w][0];
        nnz += s_wr[ph][w][1];
      }
      // A lowered copy j bounds the samples of the phase by K_j, its key once
      // every copy above it that is not lowered is a sample (more samples
      // only lower it further): ranks at or below K_j wait for the next phase.
      uint32_t sstop = kHot;
      if (lowany) {
        if (remj && lowered) {  // the whole group of a lowered copy
          const uint32_t lb = hq * kCmp;  // this lane's copies' bits
          const uint32_t lowc = (uint32_t)(s_lowc[ph][lb >> 6] >> (lb & 63u));
          uint32_t nk = me.w;
          uint32_t nm = cand & ~lowc & HotSet<HOT>::kCmpMask;
          if (nm) {
            const uint4 pj = s_hp[hj];
            for (; nm; nm &= nm - 1) {
              const uint32_t u = (uint32_t)__builtin_ctz(nm);
              const uint4 pi = s_hp[hq * kCmp + u];
              const float dd = sqdist(__uint_as_float(pj.x), __uint_as_float(pj.y),
                                      __uint_as_float(pj.z), __uint_as_float(pi.x),
                                      __uint_as_float(pi.y), __uint_as_float(pi.z));
              nk = min(nk, __float_as_uint(dd));  // non-negative floats order like their bits
            }
          }
          const uint64_t K = ((uint64_t)group_min<kCopyLanes>(nk) << 32) | me.z;
          if (hq == 0) atomicMax(&s_kmax[ph], (unsigned long long)K);
        }
        __syncthreads();
        // the first rank at or below some K_j: the least number of copies
        // above a K_j is the number above the largest, which every wave
        // counts over the copies itself
        const unsigned long long kmax = s_kmax[ph];
        sstop = 0;
#pragma unroll
        for (uint32_t t = 0; t < kHot / 64; ++t) {
          const uint4 o = s_hq[ph][64 * t + lane];
          sstop += (uint32_t)__popcll(__ballot((((uint64_t)o.w << 32) | o.z) > kmax));
        }
      }
      // the samples: copies not lowered, ranked below min(stop, nnz), the
      // first room - npk of them, in rank order
      const uint32_t seff = min(sstop, nnz);
      uint64_t accr[kWords];  // by rank
      uint32_t P = 0;
#pragma unroll
      for (uint32_t w = 0; w < kWords; ++w) {
        const uint32_t r0 = 64 * w;
        const uint64_t f = seff >= r0 + 64 ? ~0ull : seff > r0 ? (1ull << (seff - r0)) - 1ull : 0ull;
        accr[w] = f & ~lowm[w];
        P += (uint32_t)__popcll(accr[w]);
      }
      while (P > room - npk) {  // the last samples of the call: the highest ranks go
#pragma unroll
        for (int w = (int)kWords - 1; w >= 0; --w) {
          if (accr[w]) {
            accr[w] &= ~(1ull << (63 - __clzll(accr[w])));
            break;
          }
        }
        --P;
      }
      // ranks below r among the accepted, and whether r is accepted
      const auto acc_below = [&](uint32_t r) -> uint32_t {
        uint32_t b = 0;
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) {
          const uint32_t r0 = 64 * w;
          b += r >= r0 + 64 ? (uint32_t)__popcll(accr[w])
               : r > r0     ? (uint32_t)__popcll(accr[w] & ((1ull << (r - r0)) - 1ull))
                            : 0u;
        }
        return b;
      };
      const auto acc_has = [&](uint32_t r) -> bool {
        return (accr[(r >> 6) & (kWords - 1u)] >> (r & 63u)) & 1u;
      };
      if (P == 0) {  // rank 0: below the hot threshold, or distance 0
        stop = (nge == 0) ? 1u : 2u;
        break;
      }
      const bool acc = remj && rank < kHot && acc_has(rank);
      if (acc) {
        my_acc = true;
        my_key = 0;
        my_out = npk + acc_below(rank);
        my_qc = mx.x;
        my_hh = mx.w;
      }
      npk += P;
      if (npk >= room) {  // the last sample needs no update
        stop = 2;
        break;
      }
      if (P >= nnz && nnz < nge) {  // the next copy has distance 0: src/yuezu_fps.cpp:705-706
        stop = 2;
        break;
      }
      // few copies left: they go back to the next selection (always so at
      // kPhaseMin = kHot, at most kHot copies being >= the hot threshold)
      if (kPhaseMin >= kHot || nge - P < kPhaseMin) {
        stop = P >= nge ? 1u : 0u;
        break;
      }
      // the accepted cubes on the remaining copies
      const bool remj2 = remj && !acc;
      uint32_t mnb = 0xffffffffu;
      if (remj2) {
        uint32_t rk[kCmp];
#pragma unroll
        for (uint32_t v = 0; v < kCmp / 4; ++v) {
          const uint4 r4 = reinterpret_cast<const uint4 *>(s_rank)[hq * (kCmp / 4) + v];
          rk[4 * v] = r4.x;
          rk[4 * v + 1] = r4.y;
          rk[4 * v + 2] = r4.z;
          rk[4 * v + 3] = r4.w;
        }
        uint32_t cand2 = 0;
#pragma unroll
        for (uint32_t u = 0; u < kCmp; ++u) {
          const uint4 o = s_hq[ph][kCopyLanes * u + hq];
          cand2 |= ((rk[u] < kHot ? (uint32_t)acc_has(rk[u]) : 0u) & j_in(mx.y, mx.z, o.x, o.y)) << u;
        }
        if (cand2) {  // rare: the exact distances
          const uint4 pj = s_hp[hj];
          while (cand2) {
            const uint32_t u = (uint32_t)__builtin_ctz(cand2);
            cand2 &= cand2 - 1;
            const uint4 pi = s_hp[hq * kCmp + u];
            const float dd = sqdist(__uint_as_float(pj.x), __uint_as_float(pj.y),
                                    __uint_as_float(pj.z), __uint_as_float(pi.x),
                                    __uint_as_float(pi.y), __uint_as_float(pi.z));
            mnb = min(mnb, __float_as_uint(dd));  // non-negative floats order like their bits
          }
        }
      }
      mnb = group_min<kCopyLanes>(mnb);
      // the next buffer: accepted copies get key 0, lowered ones new cubes
      if (hq == 0) {
        uint4 nv = me;
        if (acc) {
          nv.z = 0u;
          nv.w = 0u;
        } else if (remj && mnb < me.w) {
          const uint32_t h = packed_halves(c.r, __uint_as_float(mnb));
          uint32_t lo_c, hi_c;
          cube_corners(mx.x, h, b0, b1, b2, lo_c, hi_c);
          nv = make_uint4(pack11(lo_c), pack11(hi_c) | kGuards, me.z, mnb);
          s_hx[hj].w = h;
        }
        s_hq[ph ^ 1][hot_slot<HOT>(hj)] = nv;
      }
      __syncthreads();
      ph ^= 1;
      NSFPS_RMARK(kRpPhases);
      if (PROF) pf[kRpPhaseCount] += 1;
    }
    NSFPS_RMARK(kRpPhases);
    // ---- the hot run's samples -> global memory and every list entry.
    // The group of an accepted copy walks the coarse rows its cube spans,
    // min-ing distances into LDS.  A cube over more than kWalkRows rows, or a
    // lane meeting more than kWalkLaneEntries entries in its rows, flags the
    // sample instead; flagged samples are applied below by every thread to its
    // own entries (applying a sample twice changes nothing).  Meanwhile the
    // next hot set's copy buffer and first histogram are cleared, and the
    // largest key of a copy left unaccepted bounds the next histogram.
    {
      const uint32_t q = hq;
      if (tid < kHot) s_hq[0][tid] = make_uint4(0u, 0u, 0u, 0u);
      if (tid < kSelBins) s_sel[0][tid] = 0;
      if (q == 0 && my_key != 0) atomicMax(&s_kmr, (unsigned long long)my_key);
      if (my_acc) {
        const uint4 rp = s_hp[hj];
        const uint32_t qc = my_qc, hh = my_hh;
        uint32_t lo_c, hi_c;
        cube_corners(qc, hh, b0, b1, b2, lo_c, hi_c);
        const uint32_t lo11 = pack11(lo_c), hi11g = pack11(hi_c) | kGuards;
        if (q == 0) {
          out[it + my_out] = (int32_t)rp.w;
          pick_p[np + my_out] = make_float4(__uint_as_float(rp.x), __uint_as_float(rp.y),
                                            __uint_as_float(rp.z), 0.f);
          pick_c[np + my_out] = make_uint2(lo11, hi11g);
          s_rp[hj] = rp;
          s_rc[hj] = make_uint2(lo11, hi11g);
          if (ALIAS) {
            s_sbox[my_out] = make_uint2(lo11, hi11g);
            s_spos[my_out] = make_float4(__uint_as_float(rp.x), __uint_as_float(rp.y),
                                         __uint_as_float(rp.z), 0.f);
          }
        }
        const uint32_t x0 = (lo_c & 1023u) >> gsx, x1 = (hi_c & 1023u) >> gsx;
        const uint32_t y0 = ((lo_c >> 10) & 1023u) >> gsy, y1 = ((hi_c >> 10) & 1023u) >> gsy;
        const uint32_t z0 = (lo_c >> 20) >> gsz, z1 = (hi_c >> 20) >> gsz;
        const uint32_t ny = y1 - y0 + 1, nrows = ny * (z1 - z0 + 1);
        bool big = nrows > WalkLimits<HOT, ROWS>::kRows;
        if (!big) {
          // row rr = rz * ny + ry; rz = floor((rr + 0.5) / ny) holds with an
          // approximate reciprocal: rr < 64 leaves a margin of 0.5 / ny
          const float rny = __builtin_amdgcn_rcpf((float)ny);
          const float px = __uint_as_float(rp.x), py = __uint_as_float(rp.y),
                      pz = __uint_as_float(rp.z);
          // four entries per step, their reads in flight together (a short
          // last step repeats an entry: min is idempotent); one 16-byte read
          // each, and the min is unconditional (a no-op outside the cube), so
          // the cell is not read ahead of the coordinates
          const auto walk4 = [&](const uint32_t(&ee)[4]) {
            uint4 pe[4];
#pragma unroll
            for (uint32_t t = 0; t < 4; ++t) pe[t] = s_pc[ee[t]];
#pragma unroll
            for (uint32_t t = 0; t < 4; ++t) {
              const uint32_t dt =
                  __float_as_uint(sqdist(__uint_as_float(pe[t].x), __uint_as_float(pe[t].y),
                                         __uint_as_float(pe[t].z), px, py, pz));
              // non-negative floats order like their bits
              atomicMin(&s_dd[ee[t]],
                        in_box11(pe[t].w | kGuards, pe[t].w, lo11, hi11g) ? dt : 0xffffffffu);
            }
          };
          if (!ALIAS) {
            // the lane's rows (rr = q, q + kCopyLanes, ...): their entry
            // ranges read up front (one LDS wait; a lane with fewer rows reads
            // row 0's again and counts it empty), then their entries walked
            // as one list.  Per call, against row by row (whose last step in
            // each row mostly repeats): uniform cube 2.6 % and LiDAR scan
            // 5.5 % faster, clustered cloud (full rows) 2.5 % slower.
            constexpr uint32_t kLaneRows = (WalkLimits<HOT, ROWS>::kRows + kCopyLanes - 1) / kCopyLanes;
            uint32_t rs[kLaneRows], rn[kLaneRows], ne = 0;
#pragma unroll
            for (uint32_t t = 0; t < kLaneRows; ++t) {
              const bool ok = q + t * kCopyLanes < nrows;
              const uint32_t rr = ok ? q + t * kCopyLanes : 0u;
              const uint32_t rz = (uint32_t)(((float)rr + 0.5f) * rny), ry = rr - rz * ny;
              const uint32_t rw = ((z0 + rz) * gy + y0 + ry) * gx;
              const uint32_t e0 = s_cell[rw + x0], e1 = s_cell[rw + x1 + 1];
              rs[t] = e0;
              rn[t] = ok ? e1 - e0 : 0u;
              ne += rn[t];
            }
            // more entries than the lane's budget: the sample is flagged (the
            // same samples as a row-by-row test: running totals only grow)
            if (ne > WalkLimits<HOT, ROWS>::kLaneEntries) {
              big = true;
            } else {
              for (uint32_t f = 0; f < ne; f += 4) {
                uint32_t ee[4];
#pragma unroll
                for (uint32_t t = 0; t < 4; ++t) {  // list position -> entry
                  const uint32_t ff = f + t < ne ? f + t : ne - 1;
                  uint32_t e = rs[0] + ff, acc = rn[0];
#pragma unroll
                  for (uint32_t u = 1; u < kLaneRows; ++u) {
                    e = ff >= acc ? rs[u] + (ff - acc) : e;
                    acc += rn[u];
                  }
                  ee[t] = e;
                }
                walk4(ee);
              }
            }
          } else {
            // shared buckets: row by row, each row's entries and then the
            // other-cell records of its coarse cells (the budget counts both)
            uint32_t budget = kWalkLaneEntries;
            for (uint32_t rr = q; rr < nrows; rr += kCopyLanes) {
              const uint32_t rz = (uint32_t)(((float)rr + 0.5f) * rny), ry = rr - rz * ny;
              const uint32_t rw = ((z0 + rz) * gy + y0 + ry) * gx;
              const uint32_t e0 = s_cell[rw + x0], e1 = s_cell[rw + x1 + 1];
              const uint32_t f0 = s_xc[rw + x0], f1 = s_xc[rw + x1 + 1];
              if (e1 - e0 + (f1 - f0) > budget) {
                big = true;
                break;
              }
              budget -= e1 - e0 + (f1 - f0);
              for (uint32_t e = e0; e < e1; e += 4) {
                uint32_t ee[4];
#pragma unroll
                for (uint32_t t = 0; t < 4; ++t) ee[t] = e + t < e1 ? e + t : e1 - 1;
                walk4(ee);
              }
              for (uint32_t f = f0; f < f1; ++f) {
                const uint4 pa = s_xp[f];
                const uint32_t ea = s_xe[f];
                const uint32_t da =
                    __float_as_uint(sqdist(__uint_as_float(pa.x), __uint_as_float(pa.y),
                                           __uint_as_float(pa.z), px, py, pz));
                atomicMin(&s_dd[ea], in_box11(pa.w | kGuards, pa.w, lo11, hi11g) ? da : 0xffffffffu);
              }
            }
          }
        }
        if (big) {
          // WHOLE: a cube holding the list box holds every entry's cell
          const bool all = WHOLE && (in_box11(lb_lo | kGuards, lb_lo, lo11, hi11g) &
                                     in_box11(lb_hi | kGuards, lb_hi, lo11, hi11g)) != 0;
          if (all) atomicOr(&s_bigw[WHOLE ? hj >> 5 : 0], 1u << (hj & 31u));
          else atomicOr(&s_big[hj >> 5], 1u << (hj & 31u));
        }
      }
      NSFPS_RMARK(kRpWalk);
      __syncthreads();  // the walks' updates are in LDS
      NSFPS_RMARK(kRpWalkWait);
      if (ALIAS) {
        // the entries whose other cells did not fit the second index (the
        // walk reached them by their own cell alone), against every sample
        // of the hot set: a thread per entry; lane k of every wave holds
        // sample k's cube corners, which the loop reads lane by lane (the
        // walk is done, so the thread owns the entry's distance)
        const uint32_t nal = uniform(s_nal), nk = uniform(npk);
        const uint2 bx = s_sbox[lane < nk ? lane : 0u];
        if (PROF) pf[kRpAliasN] += nal;
        for (uint32_t ia = tid; ia < nal; ia += kRunThreads) {
          const uint32_t pe = s_alist[ia];
          const uint4 pp = s_pc[pe];
          uint32_t dm = s_dd[pe];
          // sample k's cube holds another cell of the bucket (rare): its distance
          const auto take = [&](uint32_t k) {
            const float4 q = s_spos[k];
            const float dd = sqdist(__uint_as_float(pp.x), __uint_as_float(pp.y),
                                    __uint_as_float(pp.z), q.x, q.y, q.z);
            dm = min(dm, __float_as_uint(dd));  // non-negative floats order like their bits
          };
          // every cell of the bucket (its own again: min is idempotent)
          uint32_t eo[kMaxAlias];
#pragma unroll
          for (uint32_t a = 0; a < kMaxAlias; ++a)
            eo[a] = a < na ? s_al[pe * kMaxAlias + a] : pack11(kNoCell);
          for (uint32_t k = 0; k < nk; ++k) {
            const uint32_t lo = rdlane(bx.x, k), hig = rdlane(bx.y, k);
            uint32_t in = 0;
#pragma unroll
            for (uint32_t a = 0; a < kMaxAlias; ++a)
              in |= in_box11(eo[a] | kGuards, eo[a], lo, hig);
            if (in) take(k);
          }
          s_dd[pe] = dm;
        }
        __syncthreads();
        NSFPS_RMARK(kRpAlias);
      }
#pragma unroll
      for (uint32_t s = 0; s < kOwnSlots; ++s)
        if (s * kRunThreads + tid < nlist) d[s] = __uint_as_float(s_dd[s * kRunThreads + tid]);
      NSFPS_RMARK(kRpApply);
      uint64_t bigm[kWords], bigw[kWords], bany = 0;
#pragma unroll
      for (uint32_t w = 0; w < kWords; ++w) {
        bigm[w] = ((uint64_t)uniform(s_big[2 * w + 1]) << 32) | uniform(s_big[2 * w]);
        bigw[w] = WHOLE ? ((uint64_t)uniform(s_bigw[WHOLE ? 2 * w + 1 : 0]) << 32) |
                              uniform(s_bigw[WHOLE ? 2 * w : 0])
                        : 0ull;
        bany |= bigm[w] | bigw[w];
      }
      if (bany) {
        // branch-free (the distance is always computed, the box test masks
        // it), two samples a trip so that their LDS reads overlap; a lone
        // last sample is applied twice (min is idempotent)
        const auto take = [&](const uint4 a0, const uint2 bx) {
#pragma unroll
          for (uint32_t s = 0; s < kOwnSlots; ++s) {
            uint32_t in = in_box11(c11[s] | kGuards, c11[s], bx.x, bx.y);
            if (ALIAS) {  // every cell of the bucket (the own cell among them)
              const uint32_t i = s * kRunThreads + tid;
              for (uint32_t a = 0; a < na; ++a) {
                const uint32_t e = s_al[i * kMaxAlias + a];
                in |= in_box11(e | kGuards, e, bx.x, bx.y);
              }
            }
            const float dd = sqdist(x[s], y[s], z[s], __uint_as_float(a0.x),
                                    __uint_as_float(a0.y), __uint_as_float(a0.z));
            // non-negative floats order like their bits; outside the cube the
            // distance becomes all ones, which never wins
            d[s] = __uint_as_float(min(__float_as_uint(d[s]), __float_as_uint(dd) | (in - 1u)));
          }
        };
        // WHOLE: a sample whose cube holds the list box holds every entry's
        // cell, and takes the distances with no cell test
        const auto take_all = [&](const uint4 a0) {
#pragma unroll
          for (uint32_t s = 0; s < kOwnSlots; ++s) {
            const float dd = sqdist(x[s], y[s], z[s], __uint_as_float(a0.x),
                                    __uint_as_float(a0.y), __uint_as_float(a0.z));
            d[s] = __uint_as_float(min(__float_as_uint(d[s]), __float_as_uint(dd)));
          }
        };
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) {
          uint64_t bm = bigw[w];
          while (WHOLE && bm) {
            const uint32_t ka = 64 * w + (uint32_t)__builtin_ctzll(bm);
            bm &= bm - 1;
            const uint32_t kc = bm ? 64 * w + (uint32_t)__builtin_ctzll(bm) : ka;
            bm &= bm - 1;
            const uint4 a0 = s_rp[ka], a1 = s_rp[kc];
            take_all(a0);
            take_all(a1);
          }
          bm = bigm[w];
          while (bm) {
            const uint32_t ka = 64 * w + (uint32_t)__builtin_ctzll(bm);
            bm &= bm - 1;
            const uint32_t kc = bm ? 64 * w + (uint32_t)__builtin_ctzll(bm) : ka;
            bm &= bm - 1;
            const uint4 a0 = s_rp[ka], a1 = s_rp[kc];
            const uint2 b0 = s_rc[ka], b1 = s_rc[kc];
            take(a0, b0);
            take(a1, b1);
          }
        }
#pragma unroll
        for (uint32_t s = 0; s < kOwnSlots; ++s)
          if (s * kRunThreads + tid < nlist) s_dd[s * kRunThreads + tid] = __float_as_uint(d[s]);
      }
      NSFPS_RMARK(kRpBig);
    }
    it += npk;
    np += npk;
    if (PROF) pf[kRpHotRounds] += 1;
    if (stop == 2) {
      done = true;
      break;
    }
    if (hth == bkey && stop == 1) break;  // every live entry was hot: all below B now
    // ---- the next hot set's first histogram.  Live keys are below the hot
    // threshold, or belong to a copy left unaccepted (at most its last key).
    {
      const uint64_t kmr = s_kmr;
      kref = hth > bkey ? hth - 1 : bkey;
      kref = kmr > kref ? kmr : kref;
      S = sel_shift(kref, bkey);
      hist_live(d, lo, bkey, kref, S, s_sel[0], err);
      if (tid < kSelBins) s_sel[1][tid] = 0;
      if (tid == 0) s_nhot = 0;
      __syncthreads();
    }
    NSFPS_RMARK(kRpPublish);
  }
  if (tid == 0) {
    *gptr(c.iter) = it;
    rs.npicks = np;
    rs.kref0 = bkey - 1;  // every key is below the threshold now
    rs.s0 = rs.s0_next;
    rs.nlist = 0;
    rs.rounds += 1;
    if (done) *gptr(c.done) = 1;
  }
  // the histograms this round's selection read are cleared for the next
  // round's update pass (16-byte stores: three a thread)
  NSFPS_GLOBAL uint4 *const hz = reinterpret_cast<NSFPS_GLOBAL uint4 *>(hist_set(c));
  for (uint32_t j = tid; j < kHists * kHistBins / 4; j += kRunThreads) hz[j] = make_uint4(0u, 0u, 0u, 0u);
  if (PROF && tid == 0) {
    NSFPS_RMARK(kRpTail);
    pf[kRpPicks] = np;
    pf[kRpRounds] = 1;
    pf[kRpRtTotal] = __builtin_amdgcn_s_memrealtime() - rt0;
    NSFPS_GLOBAL uint64_t *pw = gptr(c.prof);
    for (uint32_t i = 0; i < kRpWords; ++i) pw[i] += pf[i];
    for (uint32_t i = kRpWords; i < kRpLocal; ++i) pw[kRpExtraAt + i - kRpWords] += pf[i];
  }
#undef NSFPS_RMARK
}

template <bool PROF, bool ALIAS, uint32_t HOT, uint32_t ROWS, bool WHOLE>
__global__ __launch_bounds__(kRunThreads) void k_run(const CloudDev *__restrict__ clouds) {
  run_list<PROF, ALIAS, HOT, ROWS, WHOLE>(clouds[blockIdx.x]);
}


// ------------------------------------------------------------------ setup

// First round: the only pick is input row 0 (the first sample) with a cube
// over the whole grid.
__global__ __launch_bounds__(kPassThreads) void k_runs_init(const CloudDev *__restrict__ clouds,
                                                           bool split) {
  const CloudDev &c = clouds[blockIdx.x];
  const uint32_t tid = threadIdx.x;
  // split: each node's key moves into its first part (the other parts and
  // l1_key zero); otherwise the parts are zero
  for (uint32_t i = tid; i < c.nl1; i += kPassThreads) {
    NSFPS_GLOBAL uint64_t *const pp = gptr(c.l1_part) + (size_t)i * kUpdateSplit;
    const uint64_t k = gptr(c.l1_key)[i];
    for (uint32_t s = 0; s < kUpdateSplit; ++s) pp[s] = split && s == 0 ? k : 0ull;
    if (split) gptr(c.l1_key)[i] = 0;
  }
  if (tid == 0) {
    NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
    rs.kref0 = ~0ull;
    rs.bkey = 0;
    rs.s0 = kMaxShift;
    rs.s0_next = kMaxShift;
    rs.npicks = 1;
    rs.nlist = 0;
    rs.rounds = 0;
    rs.err = 0;
    rs.forced = 0;
    const float4 p0 = *gptr(c.root_pos);
    gptr(c.pick_p)[0] = make_float4(p0.x, p0.y, p0.z, INFINITY);
    gptr(c.pick_c)[0] = make_uint2(
        0u, pack11(pack_cell(c.r.blocks[0] - 1, c.r.blocks[1] - 1, c.r.blocks[2] - 1)) | kGuards);
    gptr(c.out)[0] = 0;
    *gptr(c.iter) = 1;
    *gptr(c.done) = c.m <= 1 ? 1u : 0u;
  }
  for (uint32_t j = tid; j < kHists * kHistBins; j += kPassThreads) gptr(c.hist)[j] = 0;
}

// ---------------------------------------------------------------- launchers

// The variants a call without profiling may launch.
hipError_t preload_runs_kernels() {
  constexpr uint32_t S = kUpdateSplit;
  return func_attributes(
      k_runs_init, k_refine, k_gather<false, false>, k_gather<false, true>,
      k_run<false, false, 64, kWalkRows, false>, k_run<false, false, 64, kWalkRows, true>,
      k_run<false, false, 128, kWalkRows, false>, k_run<false, false, 128, kDenseWalkRows, false>,
      k_run<false, true, 64, kWalkRows, false>, k_update<false, false, false, 1, false>, k_update<false, false, false, S, false>,
      k_update<false, false, true, 1, false>, k_update<false, false, true, S, false>,
      k_update<false, true, false, 1, false>, k_update<false, true, false, S, false>,
      k_update<false, true, true, 1, false>, k_update<false, true, true, S, false>,
      k_update<false, false, false, 1, true>, k_update<false, false, false, S, true>,
      k_update<false, false, true, 1, true>, k_update<false, false, true, S, true>);
}

hipError_t launch_runs_init(const CloudDev *d_clouds, uint32_t nclouds, bool split,
                            hipStream_t st) {
  k_runs_init<<<nclouds, kPassThreads, 0, st>>>(d_clouds, split);
  return hipGetLastError();
}

// The classic round's update, gather and run kernels of one variant; hot:
// the run kernel's hot-set size where cells do not share buckets (64 or 128);
// dense: 128-copy sets walk at most kDenseWalkRows rows.
template <bool PROF, bool ALIAS, bool LB, uint32_t SPLIT, bool MIXED>
void launch_classic(const CloudDev *d_clouds, uint32_t nclouds, dim3 grid, dim3 sparse,
                    uint32_t passes, uint32_t hot, bool dense, bool whole, hipStream_t st) {
  k_update<PROF, ALIAS, LB, SPLIT, MIXED>
      <<<dim3(grid.x * SPLIT, grid.y), kPassThreads, 0, st>>>(d_clouds);
  for (uint32_t p = 1; p <= passes; ++p)
    k_refine<<<sparse, kPassThreads, 0, st>>>(d_clouds, p, passes);
  k_gather<PROF, ALIAS><<<sparse, kPassThreads, 0, st>>>(d_clouds, passes);
  if (!ALIAS && hot == 128 && dense)
    k_run<PROF, false, 128, kDenseWalkRows, false><<<nclouds, kRunThreads, 0, st>>>(d_clouds);
  else if (!ALIAS && hot == 128)
    k_run<PROF, false, 128, kWalkRows, false><<<nclouds, kRunThreads, 0, st>>>(d_clouds);
  else if (!ALIAS && whole)
    k_run<PROF, false, 64, kWalkRows, true><<<nclouds, kRunThreads, 0, st>>>(d_clouds);
  else
    k_run<PROF, ALIAS, 64, kWalkRows, false><<<nclouds, kRunThreads, 0, st>>>(d_clouds);
}

hipError_t launch_rounds(const CloudDev *d_clouds, uint32_t nclouds, uint32_t max_nl1,
                         uint32_t rounds, uint32_t passes, bool profile, bool alias,
                         bool leaf_bound, bool split, bool mixed, uint32_t hot, bool dense,
                         bool whole, hipStream_t st) {
  if (alias && mixed) return hipErrorInvalidValue;  // leaves of several buckets: one cell each
  if (hot != 64 && hot != 128) return hipErrorInvalidValue;
  const dim3 grid(max_nl1, nclouds);
  const dim3 sparse(max_nl1 < kSparseGroups ? max_nl1 : kSparseGroups, nclouds);
  using Launch = void (*)(const CloudDev *, uint32_t, dim3, dim3, uint32_t, uint32_t, bool, bool,
                          hipStream_t);
  constexpr uint32_t S = kUpdateSplit;
  // [profile][cells: one per leaf, shared buckets, several per leaf][leaf_bound][split]
  static constexpr Launch kClassic[2][3][2][2] = {
      {{{launch_classic<false, false, false, 1, false>, launch_classic<false, false, false, S, false>},
        {launch_classic<false, false, true, 1, false>, launch_classic<false, false, true, S, false>}},
       {{launch_classic<false, true, false, 1, false>, launch_classic<false, true, false, S, false>},
        {launch_classic<false, true, true, 1, false>, launch_classic<false, true, true, S, false>}},
       {{launch_classic<false, false, false, 1, true>, launch_classic<false, false, false, S, true>},
        {launch_classic<false, false, true, 1, true>, launch_classic<false, false, true, S, true>}}},
      {{{launch_classic<true, false, false, 1, false>, launch_classic<true, false, false, S, false>},
        {launch_classic<true, false, true, 1, false>, launch_classic<true, false, true, S, false>}},
       {{launch_classic<true, true, false, 1, false>, launch_classic<true, true, false, S, false>},
        {launch_classic<true, true, true, 1, false>, launch_classic<true, true, true, S, false>}},
       {{launch_classic<true, false, false, 1, true>, launch_classic<true, false, false, S, true>},
        {launch_classic<true, false, true, 1, true>, launch_classic<true, false, true, S, true>}}}};
  const Launch classic = kClassic[profile][alias ? 1 : mixed ? 2 : 0][leaf_bound][split];
  for (uint32_t r = 0; r < rounds; ++r)
    classic(d_clouds, nclouds, grid, sparse, passes, hot, dense, whole, st);
  return hipGetLastError();
}

}  // namespace nsfps
