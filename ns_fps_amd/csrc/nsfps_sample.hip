// Sampling loop on the device (gfx950).
//
// Iteration i (src/yuezu_fps.cpp:703-722): take the maximum key (min-distance
// bits << 32 | ~logical rank) -- the reference's leftmost maximum in logical
// order -- stop if its distance is <= 0, emit its input row, and update every
// point of every bucket inside the cube of cells around it
// (src/yuezu_fps.cpp:560-597).  A leaf (64 points of one bucket) or a whole
// level-1 node (64 leaves) is skipped only when the lower bound of the squared
// distance over its bounding box is >= its maximum key distance: then no point
// in it can change (exact, same fp32 operation order).
//
// Two kernels:
//  * k_wide_step: one iteration over the whole device (every workgroup owns
//    level-1 nodes; the last workgroup to arrive reduces to the root).  Used
//    for the first iterations, while the cube covers much of the grid.
//  * k_late_loop: all remaining iterations of a cloud in one 1024-thread
//    workgroup that never returns to the host.  Level-1/level-2 keys and the
//    winners' coordinates live in LDS.  In the common case one iteration costs
//    one dependent global round trip: candidate leaf data and the sibling
//    leaves of every touched level-1 node are loaded together, merged in LDS,
//    and the dirty tree path is re-reduced there.
#include <hip/hip_runtime.h>

#include "nsfps_device.h"
#include "nsfps_launch.h"

namespace nsfps {

// Leaves are processed in rounds with their metadata spread over lanes:
// lane u (< U) of a wave holds leaf u's index, slots and key; each leaf's
// wave-uniform values are read back with readlane when the wave works on it.

__device__ __forceinline__ uint32_t rl(uint32_t v, int u) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, u);
}
__device__ __forceinline__ uint64_t rl64(uint64_t v, int u) {
  return ((uint64_t)rl((uint32_t)(v >> 32), u) << 32) | rl((uint32_t)v, u);
}

// Min-update of one leaf whose points are loaded (lane < cnt holds p/ro).
// Returns true when the leaf's key changed; then key/pos are the new key and
// winner (wave-uniform) and both are stored for the leaf.
__device__ __forceinline__ bool update_leaf(const CloudDev &c, uint32_t leaf, uint32_t start,
                                            uint32_t cnt, float4 p, uint2 ro, float qx, float qy,
                                            float qz, uint64_t oldkey, uint64_t &key,
                                            float4 &pos) {
  const uint32_t lane = lane_id();
  const bool act = lane < cnt;
  uint64_t k = 0;
  if (act) {
    float d = sqdist(p.x, p.y, p.z, qx, qy, qz);
    float cc = p.w;
    if (d < cc) {
      cc = d;
      ((NSFPS_GLOBAL float *)gptr(c.P4 + start + lane))[3] = d;
    }
    k = make_key(cc, ro.x);
    p.w = __uint_as_float(ro.y);
  }
  uint64_t km = wave_max_u64(k);
  if (km == oldkey) return false;
  uint32_t wl = argmax_lane(k, km, act);
  pos = shfl_f4(p, wl);
  key = km;
  if (lane == 0) {
    gptr(c.leaf_key)[leaf] = km;
    gptr(c.leaf_pos)[leaf] = pos;
  }
  return true;
}

// Round with the box test before the point loads.  Lane u < U: leaf ml,
// exists (mv), inside the cube (mc).  On return lane u holds leaf u's current
// key and winner (mk/mp) and whether they changed.
template <int U>
__device__ __forceinline__ void round_two_stage(const CloudDev &c, uint32_t ml, bool mv, bool mc,
                                                float qx, float qy, float qz, uint64_t &mk,
                                                float4 &mp, bool &changed) {
  const uint32_t lane = lane_id();
  float4 lo = make_float4(INFINITY, 0.f, 0.f, 0.f), hi = make_float4(-INFINITY, 0.f, 0.f, 0.f);
  mk = 0;
  mp = make_float4(0.f, 0.f, 0.f, 0.f);
  changed = false;
  if (mv) {
    mk = gptr(c.leaf_key)[ml];
    mp = gptr(c.leaf_pos)[ml];
    if (mc) {
      lo = gptr(c.leaf_lo)[ml];
      hi = gptr(c.leaf_hi)[ml];
    }
  }
  const bool go = mv && mc && box_lb(qx, qy, qz, lo, hi) < key_dist(mk);
  const uint64_t gomask = __ballot(go);
  if (!gomask) return;
  float4 p[U];
  uint2 ro[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    p[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    ro[u] = make_uint2(0u, 0u);
    if ((gomask >> u) & 1) {
      uint32_t st = rl(__float_as_uint(lo.w), u), cn = rl(__float_as_uint(hi.w), u);
      if (lane < cn) {
        p[u] = gptr(c.P4)[st + lane];
        ro[u] = gptr(c.RO)[st + lane];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!((gomask >> u) & 1)) continue;
    uint32_t st = rl(__float_as_uint(lo.w), u), cn = rl(__float_as_uint(hi.w), u);
    uint64_t nk;
    float4 np;
    if (update_leaf(c, rl(ml, u), st, cn, p[u], ro[u], qx, qy, qz, rl64(mk, u), nk, np)) {
      if (lane == (uint32_t)u) {
        mk = nk;
        mp = np;
        changed = true;
      }
    }
  }
}

// Round with the point loads issued together with the metadata (one round
// trip).  Lane u < U: leaf ml (valid mv), slots [ms, ms + mn) to load; the
// leaf's own count masks the update.  On return lane u holds the new key and
// winner of leaf u when it changed.
template <int U>
__device__ __forceinline__ void round_speculative(const CloudDev &c, uint32_t ml, uint32_t ms,
                                                  uint32_t mn, bool mv, float qx, float qy,
                                                  float qz, uint64_t &nk_out, float4 &np_out,
                                                  bool &changed) {
  const uint32_t lane = lane_id();
  float4 lo = make_float4(INFINITY, 0.f, 0.f, 0.f), hi = make_float4(-INFINITY, 0.f, 0.f, 0.f);
  uint64_t mk = 0;
  changed = false;
  const uint64_t vmask = __ballot(mv);
  if (mv) {
    mk = gptr(c.leaf_key)[ml];
    lo = gptr(c.leaf_lo)[ml];
    hi = gptr(c.leaf_hi)[ml];
  }
  float4 p[U];
  uint2 ro[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    p[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    ro[u] = make_uint2(0u, 0u);
    if ((vmask >> u) & 1) {
      uint32_t st = rl(ms, u), cn = rl(mn, u);
      if (lane < cn) {
        p[u] = gptr(c.P4)[st + lane];
        ro[u] = gptr(c.RO)[st + lane];
      }
    }
  }
  const bool go = mv && box_lb(qx, qy, qz, lo, hi) < key_dist(mk);
  const uint64_t gomask = __ballot(go);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!((gomask >> u) & 1)) continue;
    uint32_t st = rl(__float_as_uint(lo.w), u), cn = rl(__float_as_uint(hi.w), u);
    uint64_t nk;
    float4 np;
    if (update_leaf(c, rl(ml, u), st, cn, p[u], ro[u], qx, qy, qz, rl64(mk, u), nk, np)) {
      if (lane == (uint32_t)u) {
        nk_out = nk;
        np_out = np;
        changed = true;
      }
    }
  }
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
    const uint32_t u = lane;
    const uint32_t ml = g * kFan + u * 16 + wave;
    const bool mv = u < 4 && ml < c.nleaves;
    const bool mc = mv && in_cube(cb, gptr(c.leaf_cell)[ml]);
    uint64_t mk;
    float4 mp;
    bool changed;
    round_two_stage<4>(c, ml, mv, mc, q.x, q.y, q.z, mk, mp, changed);
    if (u < 4) {
      s_key[u * 16 + wave] = mk;
      s_pos[u * 16 + wave] = mp;
    }
    __syncthreads();
    if (wave == 0) {
      uint64_t k = s_key[lane];
      uint64_t km = wave_max_u64(k);
      uint32_t wl = argmax_lane(k, km, true);
      if (lane == 0) {
        gptr(c.l1_key)[g] = km;
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

constexpr uint32_t kLateWaves = kLateThreads / 64;
constexpr int kU = 8;                                 // leaves per wave per round
constexpr uint32_t kRound = kLateWaves * kU;          // leaves per round
constexpr int kSib = 4;                               // sibling nodes prefetched per wave

struct Lds {
  uint64_t *l1k;
  float4 *l1p;
  float4 *l1lo, *l1hi;  // null when absent
  uint64_t *l2k;
  float4 *l2p;
  uint32_t *lut;
  uint2 *ctab;          // null when the cell table stays in global memory
  uint32_t *cl, *cs, *cn;  // candidate leaf / first slot / slot count
  uint32_t *slot;
  uint32_t *m1, *dl1, *m2, *dl2;
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
  s.dl2 = (uint32_t *)(base + pl.dl2);
  s.sk = (uint64_t *)(base + pl.sk);
  s.sp = (float4 *)(base + pl.sp);
  return s;
}

// Block-wide exclusive scan of one value per thread (kLateThreads threads)
// with a single barrier: every wave reads all wave totals.  Consecutive calls
// must alternate wsum buffers (kLateWaves entries each).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *total) {
  const uint32_t lane = lane_id(), wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (uint32_t w = 0; w < kLateWaves; ++w) {
    uint32_t t = wsum[w];
    before += w < wave ? t : 0u;
    all += t;
  }
  *total = all;
  return x - v + before;
}

// First marker of node g appends it to the dirty list.
__device__ __forceinline__ void mark_dirty(uint32_t *mask, uint32_t *list, uint32_t *count,
                                           uint32_t g) {
  uint32_t bit = 1u << (g & 31);
  uint32_t old = atomicOr(&mask[g >> 5], bit);
  if (!(old & bit)) list[atomicAdd(count, 1u)] = g;
}

// Candidate leaves of one cell: leaf range, slot range (table mode).
struct CellLeaves {
  uint32_t la, lb;      // leaves [la, lb)
  uint32_t ps, pe;      // slots [ps, pe) (table mode)
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

// Reduces level-1 node g from 64 (key, pos) entries held one per lane.
__device__ __forceinline__ void finish_l1(const Lds &s, uint32_t *n2, uint32_t g, uint64_t k,
                                          float4 p, bool v) {
  const uint32_t lane = lane_id();
  uint64_t km = wave_max_u64(k);
  uint32_t wl = argmax_lane(k, km, v);
  float4 wp = shfl_f4(p, wl);
  if (lane == 0) {
    s.l1k[g] = km;
    s.l1p[g] = wp;
    s.m1[g >> 5] = 0;  // every node of the word is in the dirty list
    s.slot[g] = kNone;
    mark_dirty(s.m2, s.dl2, n2, g / kFan);
  }
}

// Phase clock (s_memtime cycles, thread 0, barrier to barrier) and work
// counters of the single-workgroup loop, kept when PROF is set.
enum : uint32_t {
  kPfTop = 0, kPfEnum, kPfFlatten, kPfA, kPfB, kPfC, kPfRebuild, kPfL2, kPfRoot,
  kPfIters = 16, kPfFast, kPfCells, kPfLeaves, kPfDirty, kPfRealtime, kPfCount = 24
};

template <bool PROF>
__global__ __launch_bounds__(kLateThreads) void k_late_loop(const CloudDev *__restrict__ clouds) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ uint32_t s_scan[2][kLateWaves];
  uint32_t scan_parity = 0;
  __shared__ uint32_t s_n1, s_n2;
  __shared__ uint64_t s_rk;
  __shared__ float4 s_rp;
  const CloudDev &c = clouds[blockIdx.x];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (*gptr(c.done)) return;
  __shared__ uint64_t s_prof[kPfCount];
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

  for (uint32_t j = tid; j < nl1; j += kLateThreads) {
    s.l1k[j] = gptr(c.l1_key)[j];
    s.l1p[j] = gptr(c.l1_pos)[j];
    s.slot[j] = kNone;
    if (s.l1lo) {
      s.l1lo[j] = gptr(c.l1_lo)[j];
      s.l1hi[j] = gptr(c.l1_hi)[j];
    }
  }
  for (uint32_t j = tid; j < (nl1 + 31) / 32; j += kLateThreads) s.m1[j] = 0;
  for (uint32_t j = tid; j < c.r.lut_total; j += kLateThreads) s.lut[j] = gptr(c.lut)[j];
  if (s.ctab)
    for (uint32_t j = tid; j <= c.r.T; j += kLateThreads) s.ctab[j] = gptr(c.cell_info)[j];
  if (tid < 2) s.m2[tid] = 0;
  if (tid == 0) {
    s_n1 = 0;
    s_n2 = 0;
    s_rk = *gptr(c.root_key);
    s_rp = *gptr(c.root_pos);
  }
  __syncthreads();
  for (uint32_t h = wave; h < nl2; h += kLateWaves) {
    uint32_t j = h * kFan + lane;
    bool v = j < nl1;
    uint64_t k = v ? s.l1k[j] : 0ull;
    uint64_t km = wave_max_u64(k);
    uint32_t wl = argmax_lane(k, km, v);
    if (lane == 0) {
      s.l2k[h] = km;
      s.l2p[h] = s.l1p[h * kFan + wl];
    }
  }
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
    bool fast = false;
    NSFPS_MARK(kPfTop);
    NSFPS_COUNT(kPfIters, 1);
    NSFPS_COUNT(kPfCells, ncell);
    for (uint32_t cbase = 0; cbase < ncell; cbase += kLateThreads) {
      // ---- enumerate this chunk's cells: unpruned leaves, dirty nodes
      const uint32_t t = cbase + tid;
      CellLeaves cl{0, 0, 0, 0};
      uint32_t cnt = 0;
      if (t < ncell) {
        uint32_t ix = t % ex, iy = (t / ex) % ey, iz = t / (ex * ey);
        uint32_t b = bucket_of(c.r, s.lut, (uint32_t)cb.lo[0] + ix, (uint32_t)cb.lo[1] + iy,
                               (uint32_t)cb.lo[2] + iz);
        cl = cell_leaves(c, s, b);
        for (uint32_t g = cl.la / kFan; cl.la < cl.lb && g <= (cl.lb - 1) / kFan; ++g) {
          uint32_t a = max(cl.la, g * kFan), e = min(cl.lb, (g + 1) * kFan);
          if (node_pruned(s, g, q.x, q.y, q.z)) continue;
          cnt += e - a;
          mark_dirty(s.m1, s.dl1, &s_n1, g);
        }
      }
      uint32_t total;
      const uint32_t off = block_excl_scan(cnt, s_scan[scan_parity], &total);
      scan_parity ^= 1u;
      fast = (ncell <= kLateThreads) && total <= kCandCap && s_n1 <= dcap;
      NSFPS_MARK(kPfEnum);
      NSFPS_COUNT(kPfLeaves, total);
      // ---- flatten (all of it on the fast path, kCandCap per round otherwise)
      for (uint32_t rb = 0; rb < total; rb += kCandCap) {
        if (cnt) {
          uint32_t k = off;
          for (uint32_t g = cl.la / kFan; g <= (cl.lb - 1) / kFan; ++g) {
            uint32_t a = max(cl.la, g * kFan), e = min(cl.lb, (g + 1) * kFan);
            if (node_pruned(s, g, q.x, q.y, q.z)) continue;
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
            }
          }
        }
        if (fast && tid < s_n1) s.slot[s.dl1[tid]] = tid;
        __syncthreads();
        NSFPS_MARK(kPfFlatten);
        const uint32_t nr = min(kCandCap, total - rb);
        if (fast) {
          // ---- phase A: round 0 of the candidates and the sibling leaves of
          // every dirty node, loaded together
          const uint32_t nd = s_n1;
          uint32_t j = wave * kU + lane;
          bool mv = lane < (uint32_t)kU && j < nr;
          uint32_t ml = mv ? s.cl[j] : 0u, ms = mv ? s.cs[j] : 0u, mn = mv ? s.cn[j] : 0u;
          uint64_t sib_k[kSib];
          float4 sib_p[kSib];
#pragma unroll
          for (int r = 0; r < kSib; ++r) {
            uint32_t sl = wave + kLateWaves * (uint32_t)r;
            sib_k[r] = 0;
            sib_p[r] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sl < nd) {
              uint32_t jj = s.dl1[sl] * kFan + lane;
              if (jj < c.nleaves) {
                sib_k[r] = gptr(c.leaf_key)[jj];
                sib_p[r] = gptr(c.leaf_pos)[jj];
              }
            }
          }
          uint64_t nk = 0;
          float4 np = make_float4(0.f, 0.f, 0.f, 0.f);
          bool ch = false;
          round_speculative<kU>(c, ml, ms, mn, mv, q.x, q.y, q.z, nk, np, ch);
          for (uint32_t sl = wave + kLateWaves * kSib; sl < nd; sl += kLateWaves) {
            uint32_t jj = s.dl1[sl] * kFan + lane;
            bool v = jj < c.nleaves;
            s.sk[sl * kFan + lane] = v ? gptr(c.leaf_key)[jj] : 0ull;
            s.sp[sl * kFan + lane] = v ? gptr(c.leaf_pos)[jj] : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int r = 0; r < kSib; ++r) {
            uint32_t sl = wave + kLateWaves * (uint32_t)r;
            if (sl < nd) {
              s.sk[sl * kFan + lane] = sib_k[r];
              s.sp[sl * kFan + lane] = sib_p[r];
            }
          }
          __syncthreads();
          NSFPS_MARK(kPfA);
          NSFPS_COUNT(kPfFast, 1);
          NSFPS_COUNT(kPfDirty, nd);
          // ---- phase B: updated candidates overwrite their staging entry;
          // remaining rounds
          if (ch) {
            uint32_t e = s.slot[ml / kFan] * kFan + (ml % kFan);
            s.sk[e] = nk;
            s.sp[e] = np;
          }
          for (uint32_t jb = kRound; jb < nr; jb += kRound) {
            j = jb + wave * kU + lane;
            mv = lane < (uint32_t)kU && j < nr;
            ml = mv ? s.cl[j] : 0u;
            ms = mv ? s.cs[j] : 0u;
            mn = mv ? s.cn[j] : 0u;
            round_speculative<kU>(c, ml, ms, mn, mv, q.x, q.y, q.z, nk, np, ch);
            if (ch) {
              uint32_t e = s.slot[ml / kFan] * kFan + (ml % kFan);
              s.sk[e] = nk;
              s.sp[e] = np;
            }
          }
          __syncthreads();
          NSFPS_MARK(kPfB);
          // ---- phase C: re-reduce the dirty level-1 nodes from staging
          for (uint32_t sl = wave; sl < nd; sl += kLateWaves) {
            uint32_t g = s.dl1[sl];
            uint32_t jj = g * kFan + lane;
            finish_l1(s, &s_n2, g, s.sk[sl * kFan + lane], s.sp[sl * kFan + lane],
                      jj < c.nleaves);
          }
        } else {
          for (uint32_t jb = 0; jb < nr; jb += kRound) {
            uint32_t j = jb + wave * kU + lane;
            bool mv = lane < (uint32_t)kU && j < nr;
            uint32_t ml = mv ? s.cl[j] : 0u;
            uint64_t mk;
            float4 mp;
            bool ch;
            round_two_stage<kU>(c, ml, mv, mv, q.x, q.y, q.z, mk, mp, ch);
          }
        }
        __syncthreads();
        NSFPS_MARK(kPfC);
      }
    }
    if (!fast) {
      // rebuild every dirty level-1 node from the leaf records
      const uint32_t n1 = s_n1;
      for (uint32_t x = wave; x < n1; x += kLateWaves) {
        uint32_t g = s.dl1[x];
        uint32_t j = g * kFan + lane;
        bool v = j < c.nleaves;
        uint64_t k = v ? gptr(c.leaf_key)[j] : 0ull;
        float4 p = v ? gptr(c.leaf_pos)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        finish_l1(s, &s_n2, g, k, p, v);
      }
    }
    __syncthreads();
    NSFPS_MARK(kPfRebuild);
    if (tid == 0) s_n1 = 0;
    // ---- level 2 and the root
    const uint32_t n2 = s_n2;
    for (uint32_t x = wave; x < n2; x += kLateWaves) {
      uint32_t h = s.dl2[x];
      uint32_t j = h * kFan + lane;
      bool v = j < nl1;
      uint64_t k = v ? s.l1k[j] : 0ull;
      uint64_t km = wave_max_u64(k);
      uint32_t wl = argmax_lane(k, km, v);
      if (lane == 0) {
        s.l2k[h] = km;
        s.l2p[h] = s.l1p[h * kFan + wl];
      }
    }
    __syncthreads();
    NSFPS_MARK(kPfL2);
    if (wave == 0) {
      bool v = lane < nl2;
      uint64_t k = v ? s.l2k[lane] : 0ull;
      uint64_t km = wave_max_u64(k);
      uint32_t wl = argmax_lane(k, km, v);
      if (lane == 0) {
        s_rk = km;
        s_rp = s.l2p[wl];
        s_n2 = 0;
        s.m2[0] = 0;
        s.m2[1] = 0;
      }
    }
    __syncthreads();
    NSFPS_MARK(kPfRoot);
  }
  if (tid == 0) {
    *gptr(c.iter) = it;
    *gptr(c.done) = 1;
  }
  if (PROF) {
    __syncthreads();
    if (tid == 0) s_prof[kPfRealtime] = __builtin_amdgcn_s_memrealtime() - t_real0;
    __syncthreads();
    if (tid < kPfCount && gptr(c.prof)) gptr(c.prof)[tid] = s_prof[tid];
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

hipError_t launch_late_loop(const CloudDev *d_clouds, uint32_t nclouds, uint32_t lds_bytes,
                            bool profile, hipStream_t st) {
  const void *fn = profile ? (const void *)k_late_loop<true> : (const void *)k_late_loop<false>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
  if (e != hipSuccess) return e;
  if (profile)
    k_late_loop<true><<<nclouds, kLateThreads, lds_bytes, st>>>(d_clouds);
  else
    k_late_loop<false><<<nclouds, kLateThreads, lds_bytes, st>>>(d_clouds);
  return hipGetLastError();
}

}  // namespace nsfps
