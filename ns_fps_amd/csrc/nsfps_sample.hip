// Sampling loop on the device (gfx950).
//
// Iteration i (src/yuezu_fps.cpp:703-722): take the maximum key (min-distance
// bits << 32 | ~logical rank) -- the reference's leftmost maximum in logical
// order -- stop if its distance is <= 0, emit its input row, and update every
// point of every bucket inside the cube of cells around it
// (src/yuezu_fps.cpp:560-597).  A leaf (<= 64 points of one bucket) or a whole
// level-1 node (64 leaves) is skipped only when the lower bound of the squared
// distance over its bounding box is >= its maximum key distance: then no point
// in it can change (exact, same fp32 operation order).
//
// Two kernels:
//  * k_wide_update / k_wide_root: one iteration over the whole device (every
//    workgroup owns level-1 nodes; a second launch reduces them to the root).
//    Used for the first iterations, while the cube covers much of the grid.
//  * k_late_loop: all remaining iterations of a cloud in one workgroup that
//    never returns to the host.  Level-1/level-2 keys and the winners'
//    coordinates live in LDS.  In the common case an iteration costs one
//    dependent global round trip: candidate leaf data and the sibling leaves
//    of every touched level-1 node are loaded together, merged in LDS, and the
//    dirty tree path is re-reduced there by one wave.
#include <hip/hip_runtime.h>

#include "nsfps_device.h"
#include "nsfps_launch.h"

namespace nsfps {

// Leaves are processed in rounds with their descriptors spread over lanes:
// lane u (< U) of a wave holds leaf u's index, slots, key and box; each leaf's
// wave-uniform values are read back with readlane when the wave works on it.

__device__ __forceinline__ uint32_t rl(uint32_t v, int u) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, u);
}
__device__ __forceinline__ uint64_t rl64(uint64_t v, int u) {
  return ((uint64_t)rl((uint32_t)(v >> 32), u) << 32) | rl((uint32_t)v, u);
}

// Leaf descriptor held by one lane.
struct LeafLane {
  uint32_t leaf;
  bool valid;
  uint64_t key;   // current key of the leaf
  float4 pos;     // current winner (x, y, z, input row bits)
  float4 lo, hi;  // box; lo.w = first slot, hi.w = count (bits)
};

__device__ __forceinline__ void load_leaf(const CloudDev &c, LeafLane &L, bool with_box) {
  L.key = 0;
  L.pos = make_float4(0.f, 0.f, 0.f, 0.f);
  L.lo = make_float4(INFINITY, 0.f, 0.f, 0.f);
  L.hi = make_float4(-INFINITY, 0.f, 0.f, 0.f);
  if (L.valid) {
    L.key = gptr(c.leaf_key)[L.leaf];
    L.pos = gptr(c.leaf_pos)[L.leaf];
    if (with_box) {
      L.lo = gptr(c.leaf_lo)[L.leaf];
      L.hi = gptr(c.leaf_hi)[L.leaf];
    }
  }
}

// Min-update and new keys of the U leaves described by lanes 0..U-1, whose
// points are loaded in p/ro (lane < count).  Leaves not in gomask are left
// alone.  On return lane u holds leaf u's key and winner (new or unchanged) and
// whether they changed; changed leaves are stored.  The U reductions are
// independent straight-line chains, so their latencies overlap.
template <int U>
__device__ __forceinline__ void round_compute(const CloudDev &c, const LeafLane &L, uint64_t gomask,
                                              const float4 *p, const uint2 *ro, float qx, float qy,
                                              float qz, uint64_t &nk, float4 &np, bool &ch) {
  const uint32_t lane = lane_id();
  uint32_t hiv[U], lov[U];
  bool act[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t cnt = ((gomask >> u) & 1) ? rl(__float_as_uint(L.hi.w), u) : 0u;
    act[u] = lane < cnt;
    const float d = sqdist(p[u].x, p[u].y, p[u].z, qx, qy, qz);
    float cc = p[u].w;
    if (act[u] && d < cc) {
      cc = d;
      ((NSFPS_GLOBAL float *)gptr(c.P4 + rl(__float_as_uint(L.lo.w), u) + lane))[3] = d;
    }
    hiv[u] = act[u] ? __float_as_uint(cc) : 0u;
    lov[u] = ~ro[u].x;
  }
  uint32_t m[U];
#pragma unroll
  for (int u = 0; u < U; ++u) m[u] = wave_max_u32(act[u] ? hiv[u] : 0u);
  uint64_t t[U];
  bool tie = false;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    t[u] = __ballot(act[u] && hiv[u] == m[u]);
    tie = tie || __popcll(t[u]) > 1;
  }
  if (tie) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (__popcll(t[u]) > 1) {
        const bool cand = act[u] && hiv[u] == m[u];
        const uint32_t l = wave_max_u32(cand ? lov[u] : 0u);
        t[u] = __ballot(cand && lov[u] == l);
      }
    }
  }
  nk = L.key;
  np = L.pos;
  ch = false;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!((gomask >> u) & 1) || !t[u]) continue;
    const uint32_t wl = (uint32_t)__ffsll((long long)t[u]) - 1;
    const uint64_t key = ((uint64_t)m[u] << 32) | rdlane(lov[u], wl);
    if (key == rl64(L.key, u)) continue;
    const float4 pos = make_float4(__uint_as_float(rdlane(__float_as_uint(p[u].x), wl)),
                                   __uint_as_float(rdlane(__float_as_uint(p[u].y), wl)),
                                   __uint_as_float(rdlane(__float_as_uint(p[u].z), wl)),
                                   __uint_as_float(rdlane(ro[u].y, wl)));
    if (lane == 0) {
      const uint32_t leaf = rl(L.leaf, u);
      gptr(c.leaf_key)[leaf] = key;
      gptr(c.leaf_pos)[leaf] = pos;
    }
    if (lane == (uint32_t)u) {
      nk = key;
      np = pos;
      ch = true;
    }
  }
}

// Round with the box test before the point loads (the points of a skipped
// leaf are never read).  L must hold the box of candidate leaves.
template <int U>
__device__ __forceinline__ void round_two_stage(const CloudDev &c, const LeafLane &L, bool cand,
                                                float qx, float qy, float qz, uint64_t &nk,
                                                float4 &np, bool &ch) {
  const uint32_t lane = lane_id();
  const bool go = L.valid && cand && box_lb(qx, qy, qz, L.lo, L.hi) < key_dist(L.key);
  const uint64_t gomask = __ballot(go);
  nk = L.key;
  np = L.pos;
  ch = false;
  if (!gomask) return;
  float4 p[U];
  uint2 ro[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    p[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    ro[u] = make_uint2(0u, 0u);
    if ((gomask >> u) & 1) {
      const uint32_t st = rl(__float_as_uint(L.lo.w), u), cn = rl(__float_as_uint(L.hi.w), u);
      if (lane < cn) {
        p[u] = gptr(c.P4)[st + lane];
        ro[u] = gptr(c.RO)[st + lane];
      }
    }
  }
  round_compute<U>(c, L, gomask, p, ro, qx, qy, qz, nk, np, ch);
}

__device__ __forceinline__ bool in_cube(const Cube &cb, uint32_t cell) {
  int cx = cell & 1023, cy = (cell >> 10) & 1023, cz = cell >> 20;
  return cx >= cb.lo[0] && cx <= cb.hi[0] && cy >= cb.lo[1] && cy <= cb.hi[1] && cz >= cb.lo[2] &&
         cz <= cb.hi[2];
}

// Sample and query point of the current iteration: the first sample is input
// row 0 (src/yuezu_fps.cpp:696) with an unbounded cube (the full first pass,
// src/yuezu_fps.cpp:431-438); later ones are the tree root.
struct Query {
  float x, y, z, D;
  uint32_t orig;
};

__device__ __forceinline__ Query make_query(uint32_t it, uint64_t rk, float4 rp) {
  Query q;
  q.x = rp.x;
  q.y = rp.y;
  q.z = rp.z;
  if (it == 0) {
    q.D = INFINITY;
    q.orig = 0;
  } else {
    q.D = key_dist(rk);
    q.orig = __float_as_uint(rp.w);
  }
  return q;
}

// One iteration over the whole device, in two launches so that kernel
// boundaries order the memory traffic (no device-scope fences):
//  * k_wide_update: every workgroup owns level-1 nodes (64 leaves each),
//    updates the candidate leaves among them and rewrites the node;
//  * k_wide_root: one workgroup emits the sample, reduces the level-1 nodes
//    to the root and advances the iteration.
// The candidate test compares cell coordinates, so the host runs these only
// when bucket <-> cell is one-to-one.
__global__ __launch_bounds__(1024) void k_wide_update(CloudDev c) {
  __shared__ uint64_t s_key[64];
  __shared__ float4 s_pos[64];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (*gptr(c.done)) return;
  const uint32_t it = *gptr(c.iter);
  if (it + 1 >= c.m) return;  // the last sample needs no update
  const Query q = make_query(it, *gptr(c.root_key), *gptr(c.root_pos));
  const Cube cb = make_cube(c.r, q.D, q.x, q.y, q.z);
  for (uint32_t g = blockIdx.x; g < c.nl1; g += gridDim.x) {
    // lanes 0..3 of wave w describe leaves g*64 + u*16 + w
    LeafLane L;
    L.leaf = g * kFan + lane * 16 + wave;
    L.valid = lane < 4 && L.leaf < c.nleaves;
    const bool cand = L.valid && in_cube(cb, gptr(c.leaf_cell)[L.leaf]);
    load_leaf(c, L, cand);
    uint64_t nk;
    float4 np;
    bool ch;
    round_two_stage<4>(c, L, cand, q.x, q.y, q.z, nk, np, ch);
    if (lane < 4) {
      s_key[lane * 16 + wave] = nk;
      s_pos[lane * 16 + wave] = np;
    }
    __syncthreads();
    if (wave == 0) {
      const uint64_t k = s_key[lane];
      uint32_t mh;
      const uint32_t wl = key_winner((uint32_t)(k >> 32), (uint32_t)k, true, mh);
      if (lane == 0) {
        gptr(c.l1_key)[g] = ((uint64_t)mh << 32) | (uint32_t)s_key[wl];
        gptr(c.l1_pos)[g] = s_pos[wl];
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(1024) void k_wide_root(CloudDev c) {
  __shared__ uint64_t s_key[16];
  __shared__ uint32_t s_idx[16];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (*gptr(c.done)) return;
  const uint32_t it = *gptr(c.iter);
  const Query q = make_query(it, *gptr(c.root_key), *gptr(c.root_pos));
  if (it + 1 >= c.m) {
    if (tid == 0) {
      gptr(c.out)[it] = (int32_t)q.orig;
      *gptr(c.iter) = it + 1;
      *gptr(c.done) = 1;
    }
    return;
  }
  uint64_t best = 0;
  uint32_t bj = 0;
  for (uint32_t j = tid; j < c.nl1; j += 1024) {
    uint64_t k = gptr(c.l1_key)[j];
    if (k > best) {
      best = k;
      bj = j;
    }
  }
  uint64_t km = wave_max_u64(best);
  uint32_t wl = argmax_lane(best, km, true);
  uint32_t wj = rdlane(bj, wl);
  if (lane == 0) {
    s_key[wave] = km;
    s_idx[wave] = wj;
  }
  __syncthreads();
  if (wave == 0) {
    uint64_t k = lane < 16 ? s_key[lane] : 0ull;
    uint64_t kk = wave_max_u64(k);
    uint32_t l2 = argmax_lane(k, kk, lane < 16);
    if (lane == 0) {
      gptr(c.out)[it] = (int32_t)q.orig;
      *gptr(c.root_key) = kk;
      *gptr(c.root_pos) = gptr(c.l1_pos)[s_idx[l2]];
      *gptr(c.iter) = it + 1;
      if (!(key_dist(kk) > 0.0f)) *gptr(c.done) = 1;
    }
  }
}

// ----------------------------------------------------- single-workgroup loop

constexpr int kU = 8;                        // leaves per wave per round
constexpr int kSib = 2;                      // sibling nodes prefetched per wave
constexpr uint32_t kSmallDirty = 6;          // up to this many dirty nodes: one wave

struct Lds {
  uint64_t *l1k;
  float4 *l1p;
  float4 *l1lo, *l1hi;  // null when absent
  uint64_t *l2k;
  float4 *l2p;
  uint32_t *lut;
  uint2 *ctab;             // null when the cell table stays in global memory
  uint32_t *cl, *cs, *cn;  // candidate leaf / first slot / slot count
  uint32_t *slot;          // staging slot of a dirty level-1 node
  uint32_t *m1, *dl1, *m2;
  uint32_t *cm;            // per staging slot: 64-bit mask of candidate children
  uint64_t *sk;
  float4 *sp;
};

__device__ __forceinline__ Lds carve(unsigned char *base, const LdsPlan &pl) {
  Lds s;
  s.l1k = (uint64_t *)(base + pl.l1k);
  s.l1p = (float4 *)(base + pl.l1p);
  s.l1lo = pl.l1lo == kNone ? nullptr : (float4 *)(base + pl.l1lo);
  s.l1hi = pl.l1hi == kNone ? nullptr : (float4 *)(base + pl.l1hi);
  s.l2k = (uint64_t *)(base + pl.l2k);
  s.l2p = (float4 *)(base + pl.l2p);
  s.lut = (uint32_t *)(base + pl.lut);
  s.ctab = pl.ctab == kNone ? nullptr : (uint2 *)(base + pl.ctab);
  s.cl = (uint32_t *)(base + pl.cand);
  s.cs = s.cl + kCandCap;
  s.cn = s.cs + kCandCap;
  s.slot = (uint32_t *)(base + pl.slot);
  s.m1 = (uint32_t *)(base + pl.m1);
  s.dl1 = (uint32_t *)(base + pl.dl1);
  s.m2 = (uint32_t *)(base + pl.m2);
  s.cm = (uint32_t *)(base + pl.cm);
  s.sk = (uint64_t *)(base + pl.sk);
  s.sp = (float4 *)(base + pl.sp);
  return s;
}

// First marker of level-1 node g appends it to the dirty list and gives it a
// staging slot (when one is left).
__device__ __forceinline__ void mark_dirty(const Lds &s, uint32_t *count, uint32_t dcap,
                                           uint32_t g) {
  const uint32_t bit = 1u << (g & 31);
  const uint32_t old = atomicOr(&s.m1[g >> 5], bit);
  if (!(old & bit)) {
    const uint32_t i = atomicAdd(count, 1u);
    s.dl1[i] = g;
    if (i < dcap) s.slot[g] = i;
  }
}

// Candidate leaves of one cell: leaf range, slot range (table mode).
struct CellLeaves {
  uint32_t la, lb;  // leaves [la, lb)
  uint32_t ps, pe;  // slots [ps, pe) (table mode)
};

__device__ __forceinline__ CellLeaves cell_leaves(const CloudDev &c, const Lds &s, uint32_t b) {
  CellLeaves r;
  if (c.padded) {
    r.la = b * c.lpc;
    r.lb = r.la + c.lpc;
    r.ps = r.pe = 0;
  } else {
    uint2 i0, i1;
    if (s.ctab) {
      i0 = s.ctab[b];
      i1 = s.ctab[b + 1];
    } else {
      i0 = gptr(c.cell_info)[b];
      i1 = gptr(c.cell_info)[b + 1];
    }
    r.la = i0.y;
    r.lb = i1.y;
    r.ps = i0.x;
    r.pe = i1.x;
  }
  return r;
}

__device__ __forceinline__ bool node_pruned(const Lds &s, uint32_t g, float qx, float qy,
                                            float qz) {
  if (!s.l1lo) return false;
  return !(box_lb(qx, qy, qz, s.l1lo[g], s.l1hi[g]) < key_dist(s.l1k[g]));
}

// Level-1 node g from 64 (key, winner) entries, one per lane; clears the
// node's dirty state.
__device__ __forceinline__ void reduce_l1(const Lds &s, uint32_t g, uint64_t k, float4 pos,
                                          bool v) {
  const uint32_t lane = lane_id();
  uint32_t mh;
  const uint32_t wl = key_winner((uint32_t)(k >> 32), (uint32_t)k, v, mh);
  const uint32_t lo = rdlane((uint32_t)k, wl);
  const float4 wp = shfl_f4(pos, wl);
  if (lane == 0) {
    s.l1k[g] = ((uint64_t)mh << 32) | lo;
    s.l1p[g] = wp;
    s.m1[g >> 5] = 0;  // every node of the word is in the dirty list
    s.slot[g] = kNone;
  }
}

// Level-2 node h, by one wave.
__device__ __forceinline__ void reduce_l2(const Lds &s, uint32_t h, uint32_t nl1) {
  const uint32_t lane = lane_id();
  const uint32_t j = h * kFan + lane;
  const bool v = j < nl1;
  const uint64_t k = v ? s.l1k[j] : 0ull;
  uint32_t mh;
  const uint32_t wl = key_winner((uint32_t)(k >> 32), (uint32_t)k, v, mh);
  const uint32_t lo = rdlane((uint32_t)k, wl);
  if (lane == 0) {
    s.l2k[h] = ((uint64_t)mh << 32) | lo;
    s.l2p[h] = s.l1p[h * kFan + wl];
  }
}

__device__ __forceinline__ void reduce_root(const Lds &s, uint32_t nl2, uint64_t *rk, float4 *rp) {
  const uint32_t lane = lane_id();
  const bool v = lane < nl2;
  const uint64_t k = v ? s.l2k[lane] : 0ull;
  uint32_t mh;
  const uint32_t wl = key_winner((uint32_t)(k >> 32), (uint32_t)k, v, mh);
  const uint32_t lo = rdlane((uint32_t)k, wl);
  if (lane == 0) {
    *rk = ((uint64_t)mh << 32) | lo;
    *rp = s.l2p[wl];
  }
}

// Level 2 (the nodes flagged in l2mask) and the root, by one wave.
__device__ __forceinline__ void reduce_top(const Lds &s, uint64_t l2mask, uint32_t nl1,
                                           uint32_t nl2, uint64_t *rk, float4 *rp) {
  while (l2mask) {
    const uint32_t h = (uint32_t)__ffsll((long long)l2mask) - 1;
    l2mask &= l2mask - 1;
    reduce_l2(s, h, nl1);
  }
  reduce_root(s, nl2, rk, rp);
}

// Phase clock (s_memtime cycles, thread 0, barrier to barrier) and work
// counters of the single-workgroup loop, kept when PROF is set.
enum : uint32_t {
  kPfTop = 0, kPfEnum, kPfFlatten, kPfA, kPfB, kPfC, kPfRebuild, kPfL2, kPfRoot,
  kPfIters = 16, kPfFast, kPfCells, kPfLeaves, kPfDirty, kPfRealtime, kPfCount = 24
};

template <bool PROF, uint32_t NT>
__global__ __launch_bounds__(NT) void k_late_loop(const CloudDev *__restrict__ clouds) {
  constexpr uint32_t kLW = NT / 64;      // waves
  constexpr uint32_t kRound = kLW * kU;  // leaves per round
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ uint32_t s_scan[2][kLW];
  __shared__ uint32_t s_n1;
  __shared__ uint64_t s_rk;
  __shared__ float4 s_rp;
  __shared__ uint64_t s_prof[kPfCount];
  const CloudDev &c = clouds[blockIdx.x];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (*gptr(c.done)) return;
  uint64_t t_last = 0, t_real0 = 0;
  if (PROF) {
    if (tid < kPfCount) s_prof[tid] = 0;
    t_last = __builtin_amdgcn_s_memtime();
    t_real0 = __builtin_amdgcn_s_memrealtime();
  }
#define NSFPS_MARK(ph)                                   \
  do {                                                   \
    if (PROF && tid == 0) {                              \
      uint64_t t_ = __builtin_amdgcn_s_memtime();        \
      s_prof[ph] += t_ - t_last;                         \
      t_last = t_;                                       \
    }                                                    \
  } while (0)
#define NSFPS_COUNT(ctr, v)                              \
  do {                                                   \
    if (PROF && tid == 0) s_prof[ctr] += (v);            \
  } while (0)
  const uint32_t nl1 = c.nl1;
  const uint32_t nl2 = (nl1 + kFan - 1) / kFan;
  const Lds s = carve(lds_raw, c.lds);
  const uint32_t dcap = c.lds.dcap;
  uint32_t it = *gptr(c.iter);
  uint32_t scan_parity = 0;

  for (uint32_t j = tid; j < nl1; j += NT) {
    s.l1k[j] = gptr(c.l1_key)[j];
    s.l1p[j] = gptr(c.l1_pos)[j];
    s.slot[j] = kNone;
    if (s.l1lo) {
      s.l1lo[j] = gptr(c.l1_lo)[j];
      s.l1hi[j] = gptr(c.l1_hi)[j];
    }
  }
  for (uint32_t j = tid; j < (nl1 + 31) / 32; j += NT) s.m1[j] = 0;
  for (uint32_t j = tid; j < 2 * dcap; j += NT) s.cm[j] = 0;
  for (uint32_t j = tid; j < c.r.lut_total; j += NT) s.lut[j] = gptr(c.lut)[j];
  if (s.ctab)
    for (uint32_t j = tid; j <= c.r.T; j += NT) s.ctab[j] = gptr(c.cell_info)[j];
  if (tid < 2) s.m2[tid] = 0;
  if (tid == 0) {
    s_n1 = 0;
    s_rk = *gptr(c.root_key);
    s_rp = *gptr(c.root_pos);
  }
  __syncthreads();
  for (uint32_t h = wave; h < nl2; h += kLW) reduce_l2(s, h, nl1);
  __syncthreads();

  while (true) {
    const Query q = make_query(it, s_rk, s_rp);
    if (it != 0 && !(q.D > 0.0f)) break;  // src/yuezu_fps.cpp:705-706
    if (it >= c.m) break;
    if (tid == 0) gptr(c.out)[it] = (int32_t)q.orig;
    ++it;
    if (it >= c.m) break;  // the last sample needs no update
    const Cube cb = make_cube(c.r, q.D, q.x, q.y, q.z);
    const uint32_t ex = (uint32_t)(cb.hi[0] - cb.lo[0] + 1);
    const uint32_t ey = (uint32_t)(cb.hi[1] - cb.lo[1] + 1);
    const uint32_t ez = (uint32_t)(cb.hi[2] - cb.lo[2] + 1);
    const uint32_t ncell = ex * ey * ez;
    NSFPS_MARK(kPfTop);
    NSFPS_COUNT(kPfIters, 1);
    NSFPS_COUNT(kPfCells, ncell);
    bool fast = false;
    for (uint32_t cbase = 0; cbase < ncell; cbase += NT) {
      // ---- enumerate this chunk's cells: unpruned leaves, dirty nodes
      const uint32_t t = cbase + tid;
      CellLeaves cl{0, 0, 0, 0};
      uint32_t cnt = 0;
      if (t < ncell) {
        const uint32_t ix = t % ex, iy = (t / ex) % ey, iz = t / (ex * ey);
        const uint32_t code = cell_code(c.r, s.lut, (uint32_t)cb.lo[0] + ix,
                                        (uint32_t)cb.lo[1] + iy, (uint32_t)cb.lo[2] + iz);
        const bool rep = c.r.bijective || bucket_first_in_cube(c.r, s.lut, code, cb);
        if (rep) cl = cell_leaves(c, s, c.r.bijective ? code : code % c.r.T);
        for (uint32_t g = cl.la / kFan; cl.la < cl.lb && g <= (cl.lb - 1) / kFan; ++g) {
          if (node_pruned(s, g, q.x, q.y, q.z)) continue;
          cnt += min(cl.lb, (g + 1) * kFan) - max(cl.la, g * kFan);
          mark_dirty(s, &s_n1, dcap, g);
        }
      }
      uint32_t total;
      const uint32_t off = block_excl_scan<kLW>(cnt, s_scan[scan_parity], &total);
      scan_parity ^= 1u;
      fast = (ncell <= NT) && total <= kCandCap && s_n1 <= dcap;
      NSFPS_MARK(kPfEnum);
      NSFPS_COUNT(kPfLeaves, total);
      // ---- flatten (all of it on the fast path, kCandCap per round otherwise)
      for (uint32_t rb = 0; rb < total; rb += kCandCap) {
        if (cnt) {
          uint32_t k = off;
          for (uint32_t g = cl.la / kFan; g <= (cl.lb - 1) / kFan; ++g) {
            const uint32_t a = max(cl.la, g * kFan), e = min(cl.lb, (g + 1) * kFan);
            if (node_pruned(s, g, q.x, q.y, q.z)) continue;
            uint64_t cmask = 0;
            for (uint32_t l = a; l < e; ++l, ++k) {
              if (k < rb || k >= rb + kCandCap) continue;
              uint32_t st, sc;
              if (c.padded) {
                st = l * kLeaf;
                sc = kLeaf;
              } else {
                st = cl.ps + (l - cl.la) * kLeaf;
                sc = min(kLeaf, cl.pe - st);
              }
              s.cl[k - rb] = l;
              s.cs[k - rb] = st;
              s.cn[k - rb] = sc;
              cmask |= 1ull << (l % kFan);
            }
            if (fast && cmask) {
              const uint32_t sl = s.slot[g];
              if ((uint32_t)cmask) atomicOr(&s.cm[2 * sl], (uint32_t)cmask);
              if (cmask >> 32) atomicOr(&s.cm[2 * sl + 1], (uint32_t)(cmask >> 32));
            }
          }
        }
        __syncthreads();
        NSFPS_MARK(kPfFlatten);
        const uint32_t nr = min(kCandCap, total - rb);
        if (fast) {
          // ---- phase A: candidates (lane-distributed, kU per wave per round)
          // with the sibling leaves of every dirty node loaded in round 0;
          // every staging entry is written once: by its candidate leaf, or by
          // the sibling load for the other children
          const uint32_t nd = s_n1;
          for (uint32_t jb = 0; jb < nr; jb += kRound) {
            const uint32_t j = jb + wave * kU + lane;
            LeafLane L;
            L.valid = lane < (uint32_t)kU && j < nr;
            L.leaf = L.valid ? s.cl[j] : 0u;
            const uint32_t ms = L.valid ? s.cs[j] : 0u, mn = L.valid ? s.cn[j] : 0u;
            load_leaf(c, L, true);
            const uint64_t vmask = __ballot(L.valid);
            float4 p[kU];
            uint2 ro[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
              p[u] = make_float4(0.f, 0.f, 0.f, 0.f);
              ro[u] = make_uint2(0u, 0u);
              if ((vmask >> u) & 1) {
                const uint32_t st = rl(ms, u), cn = rl(mn, u);
                if (lane < cn) {
                  p[u] = gptr(c.P4)[st + lane];
                  ro[u] = gptr(c.RO)[st + lane];
                }
              }
            }
            uint64_t sib_k[kSib];
            float4 sib_p[kSib];
            if (jb == 0) {
#pragma unroll
              for (int r = 0; r < kSib; ++r) {
                const uint32_t sl = wave + kLW * (uint32_t)r;
                const uint32_t jj = sl < nd ? s.dl1[sl] * kFan + lane : kNone;
                const bool ld = jj < c.nleaves;
                sib_k[r] = ld ? gptr(c.leaf_key)[jj] : 0ull;
                sib_p[r] = ld ? gptr(c.leaf_pos)[jj] : make_float4(0.f, 0.f, 0.f, 0.f);
              }
            }
            const bool go = L.valid && box_lb(q.x, q.y, q.z, L.lo, L.hi) < key_dist(L.key);
            uint64_t nk;
            float4 np;
            bool ch;
            round_compute<kU>(c, L, __ballot(go), p, ro, q.x, q.y, q.z, nk, np, ch);
            if (L.valid) {
              const uint32_t e = s.slot[L.leaf / kFan] * kFan + (L.leaf % kFan);
              s.sk[e] = nk;
              s.sp[e] = np;
            }
            if (jb == 0) {
#pragma unroll
              for (int r = 0; r < kSib; ++r) {
                const uint32_t sl = wave + kLW * (uint32_t)r;
                if (sl < nd) {
                  const uint64_t cm = ((uint64_t)s.cm[2 * sl + 1] << 32) | s.cm[2 * sl];
                  if (!((cm >> lane) & 1)) {
                    s.sk[sl * kFan + lane] = sib_k[r];
                    s.sp[sl * kFan + lane] = sib_p[r];
                  }
                }
              }
            }
          }
          for (uint32_t sl = wave + kLW * kSib; sl < nd; sl += kLW) {
            const uint32_t jj = s.dl1[sl] * kFan + lane;
            const uint64_t cm = ((uint64_t)s.cm[2 * sl + 1] << 32) | s.cm[2 * sl];
            if (!((cm >> lane) & 1)) {
              const bool ld = jj < c.nleaves;
              s.sk[sl * kFan + lane] = ld ? gptr(c.leaf_key)[jj] : 0ull;
              s.sp[sl * kFan + lane] = ld ? gptr(c.leaf_pos)[jj] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
          }
          __syncthreads();
          NSFPS_MARK(kPfA);
          NSFPS_COUNT(kPfFast, 1);
          NSFPS_COUNT(kPfDirty, nd);
          // ---- phase C: the dirty level-1 nodes from staging, then level 2
          // and the root; by wave 0 alone when few nodes are dirty
          if (nd <= kSmallDirty) {
            if (wave == 0) {
              uint64_t l2mask = 0;
              for (uint32_t sl = 0; sl < nd; ++sl) {
                const uint32_t g = s.dl1[sl];
                reduce_l1(s, g, s.sk[sl * kFan + lane], s.sp[sl * kFan + lane],
                          g * kFan + lane < c.nleaves);
                l2mask |= 1ull << (g / kFan);
              }
              if (lane < 2 * nd) s.cm[lane] = 0;
              reduce_top(s, l2mask, nl1, nl2, &s_rk, &s_rp);
              if (lane == 0) s_n1 = 0;
            }
          } else {
            for (uint32_t sl = wave; sl < nd; sl += kLW) {
              const uint32_t g = s.dl1[sl];
              reduce_l1(s, g, s.sk[sl * kFan + lane], s.sp[sl * kFan + lane],
                        g * kFan + lane < c.nleaves);
              if (lane == 0) {
                atomicOr(&s.m2[(g / kFan) >> 5], 1u << ((g / kFan) & 31));
                s.cm[2 * sl] = 0;
                s.cm[2 * sl + 1] = 0;
              }
            }
            __syncthreads();
            if (wave == 0) {
              reduce_top(s, ((uint64_t)s.m2[1] << 32) | s.m2[0], nl1, nl2, &s_rk, &s_rp);
              if (lane == 0) {
                s.m2[0] = 0;
                s.m2[1] = 0;
                s_n1 = 0;
              }
            }
          }
          NSFPS_MARK(kPfC);
        } else {
          for (uint32_t jb = 0; jb < nr; jb += kRound) {
            const uint32_t j = jb + wave * kU + lane;
            LeafLane L;
            L.valid = lane < (uint32_t)kU && j < nr;
            L.leaf = L.valid ? s.cl[j] : 0u;
            load_leaf(c, L, true);
            uint64_t nk;
            float4 np;
            bool ch;
            round_two_stage<kU>(c, L, L.valid, q.x, q.y, q.z, nk, np, ch);
          }
        }
        __syncthreads();
      }
    }
    if (!fast) {
      // rebuild every dirty level-1 node from the leaf records, then level 2
      // and the root
      const uint32_t n1 = s_n1;
      for (uint32_t x = wave; x < n1; x += kLW) {
        const uint32_t g = s.dl1[x];
        const uint32_t j = g * kFan + lane;
        const bool v = j < c.nleaves;
        const uint64_t k = v ? gptr(c.leaf_key)[j] : 0ull;
        const float4 pp = v ? gptr(c.leaf_pos)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        reduce_l1(s, g, k, pp, v);
        if (lane == 0) atomicOr(&s.m2[(g / kFan) >> 5], 1u << ((g / kFan) & 31));
      }
      for (uint32_t j = tid; j < 2 * dcap; j += NT) s.cm[j] = 0;
      __syncthreads();
      NSFPS_MARK(kPfRebuild);
      if (wave == 0) {
        reduce_top(s, ((uint64_t)s.m2[1] << 32) | s.m2[0], nl1, nl2, &s_rk, &s_rp);
        if (lane == 0) {
          s.m2[0] = 0;
          s.m2[1] = 0;
          s_n1 = 0;
        }
      }
      __syncthreads();
      NSFPS_MARK(kPfRoot);
    }
  }
  if (tid == 0) {
    *gptr(c.iter) = it;
    *gptr(c.done) = 1;
  }
  if (PROF) {
    __syncthreads();
    if (tid == 0) s_prof[kPfRealtime] = __builtin_amdgcn_s_memrealtime() - t_real0;
    __syncthreads();
    if (tid < kPfCount && c.prof) gptr(c.prof)[tid] = s_prof[tid];
  }
#undef NSFPS_MARK
#undef NSFPS_COUNT
}

// ---------------------------------------------------------------- launchers

hipError_t launch_wide_steps(const CloudDev &c, uint32_t steps, uint32_t grid, hipStream_t st) {
  for (uint32_t s = 0; s < steps; ++s) {
    k_wide_update<<<grid, 1024, 0, st>>>(c);
    k_wide_root<<<1, 1024, 0, st>>>(c);
  }
  return hipGetLastError();
}

template <bool PROF, uint32_t NT>
static hipError_t launch_late_t(const CloudDev *d_clouds, uint32_t nclouds, uint32_t lds_bytes,
                                hipStream_t st) {
  hipError_t e = hipFuncSetAttribute((const void *)k_late_loop<PROF, NT>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
  if (e != hipSuccess) return e;
  k_late_loop<PROF, NT><<<nclouds, NT, lds_bytes, st>>>(d_clouds);
  return hipGetLastError();
}

hipError_t launch_late_loop(const CloudDev *d_clouds, uint32_t nclouds, uint32_t lds_bytes,
                            bool profile, uint32_t threads, hipStream_t st) {
  if (threads == 1024)
    return profile ? launch_late_t<true, 1024>(d_clouds, nclouds, lds_bytes, st)
                   : launch_late_t<false, 1024>(d_clouds, nclouds, lds_bytes, st);
  return profile ? launch_late_t<true, 512>(d_clouds, nclouds, lds_bytes, st)
                 : launch_late_t<false, 512>(d_clouds, nclouds, lds_bytes, st);
}

}  // namespace nsfps
