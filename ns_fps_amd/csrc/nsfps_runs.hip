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
//
// One round, in stream order:
//   k_update     picks -> points, leaf and level-1 keys, fine + coarse histograms
//   k_refine x2  finer histograms inside the crossing bin, only when needed
//   k_gather     threshold B (<= kListCap keys above it), list of those points
//   k_run        samples from the list
// The first round's only pick is input row 0 with a cube covering the whole
// grid: the reference's first full pass (src/yuezu_fps.cpp:431-438).
//
// The cube test compares cell coordinates, so the engine runs only when
// bucket <-> cell is one-to-one.
#include <hip/hip_runtime.h>

#include "nsfps_device.h"
#include "nsfps_launch.h"

namespace nsfps {

constexpr uint32_t kPassThreads = 1024;  // grid-wide passes: one level-1 node per workgroup
constexpr uint32_t kPassWaves = kPassThreads / 64;
constexpr uint32_t kLeavesPerWave = kFan / kPassWaves;
constexpr uint32_t kMaxShift = 52;  // kHistBins << 52 covers the whole u64 key range

__device__ __forceinline__ uint32_t pack_cell(uint32_t x, uint32_t y, uint32_t z) {
  return x | (y << 10) | (z << 20);
}

// Cell inside a cube given as packed lo / hi corners.
__device__ __forceinline__ bool cell_in(uint32_t cell, uint2 cube) {
  const uint32_t x = cell & 1023u, y = (cell >> 10) & 1023u, z = cell >> 20;
  return x >= (cube.x & 1023u) && x <= (cube.y & 1023u) && y >= ((cube.x >> 10) & 1023u) &&
         y <= ((cube.y >> 10) & 1023u) && z >= (cube.x >> 20) && z <= (cube.y >> 20);
}

// Cube overlapping the cell range [lo, hi] (packed corners).
__device__ __forceinline__ bool cube_overlaps(uint2 cube, uint32_t lo, uint32_t hi) {
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const uint32_t s = 10u * a;
    if (((cube.x >> s) & 1023u) > ((hi >> s) & 1023u)) return false;
    if (((cube.y >> s) & 1023u) < ((lo >> s) & 1023u)) return false;
  }
  return true;
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

// Threshold selection, replayed identically by every workgroup that needs it.
// A histogram over window (kref, S) gives the first bin where the cumulative
// count exceeds the free capacity; the bins before it are taken.  If they
// fill less than half of it, that crossing bin is histogrammed again 12 bits
// finer by the next refinement pass.  The update pass counts two windows
// below kref0: a fine one (shift s0) and a 4096x wider coarse one, used when
// the fine window holds under half a list.  When nothing fits (more than
// kListCap keys share the finest bin) the threshold is the maximum key.
struct Sel {
  uint64_t kref;
  uint64_t bkey;     // resolved threshold
  uint32_t S;
  uint32_t cap;      // capacity left
  uint32_t total;    // entries taken so far
  uint32_t state;    // 0: refinement pass `pass` needed, 1: resolved, 2: use the maximum key
  uint32_t pass;
};

struct Step {
  uint32_t tot;     // keys in the window
  uint32_t bs;      // crossing bin, kNone when tot <= cap
  uint32_t before;  // keys in the bins before it
};

// Block-wide, all kPassThreads threads; sc holds kPassWaves + 2 words of LDS.
__device__ Step hist_step(const uint32_t *H, uint32_t cap, uint32_t *sc) {
  const uint32_t tid = threadIdx.x;
  const uint4 h = gptr(reinterpret_cast<const uint4 *>(H))[tid];
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

__device__ __forceinline__ uint32_t coarse_shift(uint32_t s0) {
  return s0 + 12 < kMaxShift ? s0 + 12 : kMaxShift;
}

// Replays the selection from the update pass's histograms and the first
// `avail - 1` refinement histograms.
__device__ Sel sel_replay(const CloudDev &c, uint32_t avail, uint32_t *sc) {
  const NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
  Sel s;
  s.kref = rs.kref0;
  s.bkey = 0;
  s.S = rs.s0;
  s.cap = kListCap;
  s.total = 0;
  s.state = 0;
  s.pass = 0;
  Step st = hist_step(c.hist, s.cap, sc);
  if (st.bs == kNone && st.tot < kListCap / 2) {
    s.S = coarse_shift(s.S);
    st = hist_step(c.hist + kHistBins, s.cap, sc);
  }
  for (uint32_t p = 0;; ++p) {
    if (st.bs == kNone) {  // the whole window fits
      s.total += st.tot;
      s.bkey = window_lo(s.kref, s.S);
      s.state = s.total ? 1u : 2u;
      return s;
    }
    s.total += st.before;
    if (st.before >= s.cap / 2 || s.S == 0 || p == kRefinePasses) {
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
    st = hist_step(c.hist + (2 + p) * kHistBins, s.cap, sc);
  }
}

__device__ __forceinline__ const NSFPS_GLOBAL RunState &rstate(const CloudDev &c) {
  return *gptr(c.rs);
}

// ------------------------------------------------------------ update pass

// Applies the picks of the last run to the points of level-1 node blockIdx.x,
// rewrites the keys of the touched leaves and of the node, and counts the keys
// into the fine and the coarse histogram.
__global__ __launch_bounds__(kPassThreads) void k_update(const CloudDev *__restrict__ clouds) {
  __shared__ uint32_t s_hist[2][kHistBins];
  __shared__ float4 s_pp[kListCap];
  __shared__ uint2 s_pc[kListCap];
  __shared__ uint64_t s_lk[kFan];
  __shared__ float4 s_lp[kFan];
  __shared__ uint32_t s_np;
  const CloudDev &c = clouds[blockIdx.y];
  const uint32_t g = blockIdx.x;
  if (g >= c.nl1 || *gptr(c.done)) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const NSFPS_GLOBAL RunState &rs = rstate(c);
  const uint32_t npicks = min(rs.npicks, kListCap);
  const uint64_t kref = rs.kref0;
  const uint32_t S = rs.s0, S1 = coarse_shift(S);
  const uint64_t wlo = window_lo(kref, S1);
  const float4 nlo = gptr(c.l1_lo)[g], nhi = gptr(c.l1_hi)[g];
  if (nlo.x > nhi.x) return;  // no points
  const uint32_t clo = pack_cell(cell_axis(c.r, 0, nlo.x), cell_axis(c.r, 1, nlo.y),
                                 cell_axis(c.r, 2, nlo.z));
  const uint32_t chi = pack_cell(cell_axis(c.r, 0, nhi.x), cell_axis(c.r, 1, nhi.y),
                                 cell_axis(c.r, 2, nhi.z));
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) {
    s_hist[0][j] = 0;
    s_hist[1][j] = 0;
  }
  if (tid == 0) s_np = 0;
  __syncthreads();
  for (uint32_t i = tid; i < npicks; i += kPassThreads) {
    const uint2 cb = gptr(c.pick_c)[i];
    if (cube_overlaps(cb, clo, chi)) {
      const uint32_t k = atomicAdd(&s_np, 1u);
      s_pp[k] = gptr(c.pick_p)[i];
      s_pc[k] = cb;
    }
  }
  __syncthreads();
  const uint32_t nsel = s_np;
  if (nsel == 0 && gptr(c.l1_key)[g] < wlo) return;  // nothing changes, nothing to count
  for (uint32_t k = 0; k < kLeavesPerWave; ++k) {
    const uint32_t li = wave * kLeavesPerWave + k;
    const uint32_t leaf = g * kFan + li;
    uint64_t key = 0;
    float4 pos = make_float4(0.f, 0.f, 0.f, 0.f);
    if (leaf < c.nleaves) {
      const uint64_t okey = gptr(c.leaf_key)[leaf];
      const uint32_t cell = gptr(c.leaf_cell)[leaf];
      bool hit = false;
      for (uint32_t cb = 0; cb < nsel && !hit; cb += 64)
        hit = __ballot(cb + lane < nsel && cell_in(cell, s_pc[cb + lane])) != 0;
      if (!hit && okey < wlo) {
        key = okey;
        pos = gptr(c.leaf_pos)[leaf];
      } else {
        const uint32_t st = __float_as_uint(gptr(c.leaf_lo)[leaf].w);
        const uint32_t cnt = __float_as_uint(gptr(c.leaf_hi)[leaf].w);
        const bool act = lane < cnt;
        float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
        uint2 ro = make_uint2(0u, 0u);
        if (act) {
          p = gptr(c.P4)[st + lane];
          ro = gptr(c.RO)[st + lane];
        }
        float d = p.w;
        if (hit) {
          for (uint32_t cb = 0; cb < nsel; cb += 64) {
            uint64_t m = __ballot(cb + lane < nsel && cell_in(cell, s_pc[cb + lane]));
            while (m) {
              const uint32_t j = (uint32_t)__ffsll((long long)m) - 1;
              m &= m - 1;
              const float4 q = s_pp[cb + j];
              const float dd = sqdist(p.x, p.y, p.z, q.x, q.y, q.z);
              d = dd < d ? dd : d;
            }
          }
          if (act && d < p.w) ((NSFPS_GLOBAL float *)gptr(c.P4 + st + lane))[3] = d;
        }
        const uint32_t hi = act ? __float_as_uint(d) : 0u, lo = ~ro.x;
        uint32_t mh;
        const uint32_t wl = key_winner(hi, lo, act, mh);
        if (wl < 64) {
          key = ((uint64_t)mh << 32) | rdlane(lo, wl);
          pos = make_float4(__uint_as_float(rdlane(__float_as_uint(p.x), wl)),
                            __uint_as_float(rdlane(__float_as_uint(p.y), wl)),
                            __uint_as_float(rdlane(__float_as_uint(p.z), wl)),
                            __uint_as_float(rdlane(ro.y, wl)));
        }
        if (hit && lane == 0 && key != okey) {
          gptr(c.leaf_key)[leaf] = key;
          gptr(c.leaf_pos)[leaf] = pos;
        }
        if (act) {
          const uint64_t kk = ((uint64_t)hi << 32) | lo;
          const uint32_t b = key_bin(kk, kref, S), b1 = key_bin(kk, kref, S1);
          if (b != kNone) atomicAdd(&s_hist[0][b], 1u);
          if (b1 != kNone) atomicAdd(&s_hist[1][b1], 1u);
        }
      }
    }
    if (lane == 0) {
      s_lk[li] = key;
      s_lp[li] = pos;
    }
  }
  __syncthreads();
  if (wave == 0) {
    const uint64_t k = s_lk[lane];
    uint32_t mh;
    const uint32_t wl = key_winner((uint32_t)(k >> 32), (uint32_t)k, true, mh);
    if (lane == 0) {
      gptr(c.l1_key)[g] = ((uint64_t)mh << 32) | (uint32_t)s_lk[wl];
      gptr(c.l1_pos)[g] = s_lp[wl];
    }
  }
  NSFPS_GLOBAL uint32_t *H = gptr(c.hist);
  for (uint32_t j = tid; j < 2 * kHistBins; j += kPassThreads) {
    const uint32_t v = s_hist[j / kHistBins][j % kHistBins];
    if (v) atomicAdd(&H[j], v);
  }
}

// ------------------------------------------------------- refinement passes

// Refinement pass `pass` (1 or 2): counts the keys of node blockIdx.x inside
// the window the selection replayed from the earlier histograms asks for;
// does nothing when the threshold is already resolved.
__global__ __launch_bounds__(kPassThreads) void k_refine(const CloudDev *__restrict__ clouds,
                                                         uint32_t pass) {
  __shared__ uint32_t s_hist[kHistBins];
  __shared__ uint32_t s_sc[kPassWaves + 2];
  const CloudDev &c = clouds[blockIdx.y];
  const uint32_t g = blockIdx.x;
  if (g >= c.nl1 || *gptr(c.done)) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const Sel s = sel_replay(c, pass, s_sc);
  if (s.state != 0 || s.pass != pass) return;
  const uint64_t wlo = window_lo(s.kref, s.S);
  if (gptr(c.l1_key)[g] < wlo) return;
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) s_hist[j] = 0;
  __syncthreads();
  for (uint32_t k = 0; k < kLeavesPerWave; ++k) {
    const uint32_t leaf = g * kFan + wave * kLeavesPerWave + k;
    if (leaf >= c.nleaves || gptr(c.leaf_key)[leaf] < wlo) continue;
    const uint32_t st = __float_as_uint(gptr(c.leaf_lo)[leaf].w);
    const uint32_t cnt = __float_as_uint(gptr(c.leaf_hi)[leaf].w);
    if (lane < cnt) {
      const float d = ((const NSFPS_GLOBAL float *)gptr(c.P4 + st + lane))[3];
      const uint32_t rank = gptr(c.RO)[st + lane].x;
      const uint32_t b = key_bin(((uint64_t)__float_as_uint(d) << 32) | ~rank, s.kref, s.S);
      if (b != kNone) atomicAdd(&s_hist[b], 1u);
    }
  }
  __syncthreads();
  NSFPS_GLOBAL uint32_t *H = gptr(c.hist + (1 + pass) * kHistBins);
  for (uint32_t j = tid; j < kHistBins; j += kPassThreads) {
    const uint32_t v = s_hist[j];
    if (v) atomicAdd(&H[j], v);
  }
}

// ------------------------------------------------------------- gather pass

__device__ __forceinline__ uint32_t bit_length(uint64_t v) { return v ? 64u - __clzll(v) : 0u; }

// Resolves the threshold from the histograms and appends every point of node
// blockIdx.x whose key is >= it to the list.  When no threshold below the
// maximum fits the list (more than kListCap keys inside the finest bin), the
// threshold is the maximum key itself: a run of one sample.
__global__ __launch_bounds__(kPassThreads) void k_gather(const CloudDev *__restrict__ clouds) {
  __shared__ uint32_t s_sc[kPassWaves + 2];
  __shared__ uint64_t s_wk[kPassWaves];
  const CloudDev &c = clouds[blockIdx.y];
  const uint32_t g = blockIdx.x;
  if (g >= c.nl1 || *gptr(c.done)) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
  const Sel s = sel_replay(c, kRefinePasses + 1, s_sc);
  uint64_t bkey = s.bkey;
  if (s.state == 2) {
    uint64_t best = 0;
    for (uint32_t j = tid; j < c.nl1; j += kPassThreads) {
      const uint64_t k = gptr(c.l1_key)[j];
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) s_wk[wave] = best;
    __syncthreads();
    best = 0;
    for (uint32_t w = 0; w < kPassWaves; ++w) best = s_wk[w] > best ? s_wk[w] : best;
    bkey = best;
  }
  if (g == 0 && tid == 0) {
    rs.bkey = bkey;
    // next round: fine bins of about 1/2048 of this round's key span
    uint32_t nx = bit_length(rs.kref0 - bkey + 1);
    nx = nx > 11u ? nx - 11u : 0u;
    rs.s0_next = nx < kMaxShift ? nx : kMaxShift;
  }
  if (gptr(c.l1_key)[g] < bkey) return;
  for (uint32_t k = 0; k < kLeavesPerWave; ++k) {
    const uint32_t leaf = g * kFan + wave * kLeavesPerWave + k;
    if (leaf >= c.nleaves || gptr(c.leaf_key)[leaf] < bkey) continue;
    const uint32_t st = __float_as_uint(gptr(c.leaf_lo)[leaf].w);
    const uint32_t cnt = __float_as_uint(gptr(c.leaf_hi)[leaf].w);
    const uint32_t cell = gptr(c.leaf_cell)[leaf];
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
    uint2 ro = make_uint2(0u, 0u);
    if (lane < cnt) {
      p = gptr(c.P4)[st + lane];
      ro = gptr(c.RO)[st + lane];
    }
    const bool take =
        lane < cnt && (((uint64_t)__float_as_uint(p.w) << 32) | ~ro.x) >= bkey;
    const uint64_t m = __ballot(take);
    if (!m) continue;
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&rs.nlist, (uint32_t)__popcll(m));
    base = rdlane(base, 0);
    if (take) {
      const uint32_t i = base + lanes_below(m);
      if (i < kListCap) {
        gptr(c.list_p)[i] = p;
        gptr(c.list_r)[i] = ro;
        gptr(c.list_c)[i] = cell;
      } else {
        rs.err = 1;
      }
    }
  }
}

// ---------------------------------------------------------------- the run

// One workgroup per cloud, list entry tid in thread tid.  Per sample: every
// wave finds its maximum key, the winners meet in LDS (one barrier), every
// wave reads all of them and agrees on the block maximum.
__global__ __launch_bounds__(kListCap) void k_run(const CloudDev *__restrict__ clouds) {
  __shared__ float s_t[3][kCubeTab];
  __shared__ uint4 s_rec[2][kListCap / 64][2];
  const CloudDev &c = clouds[blockIdx.x];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  if (*gptr(c.done)) return;
  NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
#pragma unroll
  for (int a = 0; a < 3; ++a)
    for (uint32_t k = tid; k <= c.r.blocks[a]; k += kListCap) s_t[a][k] = gptr(c.cube_t)[a * kCubeTab + k];
  const uint32_t nlist = min(rs.nlist, kListCap);
  const uint64_t bkey = rs.bkey;
  const bool act = tid < nlist;
  float4 e = make_float4(0.f, 0.f, 0.f, 0.f);
  uint2 er = make_uint2(0u, 0u);
  uint32_t ec = 0;
  if (act) {
    e = gptr(c.list_p)[tid];
    er = gptr(c.list_r)[tid];
    ec = gptr(c.list_c)[tid];
  }
  const uint32_t ex = ec & 1023u, ey = (ec >> 10) & 1023u, ez = ec >> 20;
  const uint32_t lo = ~er.x;
  uint32_t h0 = rs.hc[0], h1 = rs.hc[1], h2 = rs.hc[2];
  const uint32_t b0 = c.r.blocks[0], b1 = c.r.blocks[1], b2 = c.r.blocks[2];
  uint32_t it = *gptr(c.iter);
  const uint32_t m = c.m;
  __syncthreads();
  float t0 = h0 ? s_t[0][h0] : 0.f, t1 = h1 ? s_t[1][h1] : 0.f, t2 = h2 ? s_t[2][h2] : 0.f;
  float d = e.w;
  uint32_t np = 0, par = 0;
  bool done = false, capped = false;
  while (true) {
    if (np == kListCap) {  // cannot happen (every pick is a distinct list entry); stay exact anyway
      capped = true;
      break;
    }
    const uint32_t hi = act ? __float_as_uint(d) : 0u;
    uint32_t mh;
    const uint32_t wl = key_winner(hi, lo, act, mh);
    if (lane == wl) {
      s_rec[par][wave][0] = make_uint4(hi, lo, __float_as_uint(e.x), __float_as_uint(e.y));
      s_rec[par][wave][1] = make_uint4(__float_as_uint(e.z), er.y, ec, 0u);
    } else if (wl == 64 && lane == 0) {
      s_rec[par][wave][0] = make_uint4(0u, 0u, 0u, 0u);
      s_rec[par][wave][1] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    uint4 r0 = make_uint4(0u, 0u, 0u, 0u), r1 = r0;
    if (lane < kListCap / 64) {
      r0 = s_rec[par][lane][0];
      r1 = s_rec[par][lane][1];
    }
    uint32_t bh;
    const uint32_t wv = key_winner(r0.x, r0.y, lane < kListCap / 64, bh);
    const uint32_t wlo = rdlane(r0.y, wv);
    const uint64_t wkey = ((uint64_t)bh << 32) | wlo;
    if (wkey < bkey || wkey == 0) break;  // not provably the global maximum
    if (bh == 0) {                        // maximum distance 0: src/yuezu_fps.cpp:705-706
      done = true;
      break;
    }
    if (tid == 0) gptr(c.out)[it] = (int32_t)rdlane(r1.y, wv);
    if (++it >= m) {
      done = true;
      break;
    }
    const float qx = __uint_as_float(rdlane(r0.z, wv)), qy = __uint_as_float(rdlane(r0.w, wv));
    const float qz = __uint_as_float(rdlane(r1.x, wv));
    const uint32_t qc = rdlane(r1.z, wv);
    const float D = __uint_as_float(bh);
    // half-widths never grow: step down through the threshold table
    while (h0 && D < t0) t0 = --h0 ? s_t[0][h0] : 0.f;
    while (h1 && D < t1) t1 = --h1 ? s_t[1][h1] : 0.f;
    while (h2 && D < t2) t2 = --h2 ? s_t[2][h2] : 0.f;
    const uint32_t qx_c = qc & 1023u, qy_c = (qc >> 10) & 1023u, qz_c = qc >> 20;
    if (tid == 0) {
      const uint32_t lo_c = pack_cell(qx_c > h0 ? qx_c - h0 : 0u, qy_c > h1 ? qy_c - h1 : 0u,
                                      qz_c > h2 ? qz_c - h2 : 0u);
      const uint32_t hi_c = pack_cell(min(qx_c + h0, b0 - 1), min(qy_c + h1, b1 - 1),
                                      min(qz_c + h2, b2 - 1));
      gptr(c.pick_p)[np] = make_float4(qx, qy, qz, D);
      gptr(c.pick_c)[np] = make_uint2(lo_c, hi_c);
    }
    ++np;
    const uint32_t ax = max(ex, qx_c) - min(ex, qx_c), ay = max(ey, qy_c) - min(ey, qy_c),
                   az = max(ez, qz_c) - min(ez, qz_c);
    if (act && ax <= h0 && ay <= h1 && az <= h2) {
      const float dd = sqdist(e.x, e.y, e.z, qx, qy, qz);
      d = dd < d ? dd : d;
    }
    par ^= 1u;
  }
  if (tid == 0) {
    *gptr(c.iter) = it;
    rs.npicks = np;
    rs.hc[0] = h0;
    rs.hc[1] = h1;
    rs.hc[2] = h2;
    rs.kref0 = capped ? ~0ull : bkey - 1;  // every key is below the threshold now
    rs.s0 = capped ? kMaxShift : rs.s0_next;
    rs.nlist = 0;
    rs.rounds += 1;
    if (done) *gptr(c.done) = 1;
  }
  for (uint32_t j = tid; j < kHists * kHistBins; j += kListCap) gptr(c.hist)[j] = 0;
}

// ------------------------------------------------------------------ setup

// First round: the only pick is input row 0 (the first sample) with a cube
// over the whole grid.
__global__ __launch_bounds__(kPassThreads) void k_runs_init(const CloudDev *__restrict__ clouds) {
  const CloudDev &c = clouds[blockIdx.x];
  const uint32_t tid = threadIdx.x;
  if (tid == 0) {
    NSFPS_GLOBAL RunState &rs = *gptr(c.rs);
    rs.kref0 = ~0ull;
    rs.bkey = 0;
    rs.s0 = kMaxShift;
    rs.s0_next = kMaxShift;
    rs.npicks = 1;
    rs.nlist = 0;
    rs.hc[0] = c.r.blocks[0];
    rs.hc[1] = c.r.blocks[1];
    rs.hc[2] = c.r.blocks[2];
    rs.rounds = 0;
    rs.err = 0;
    const float4 p0 = *gptr(c.root_pos);
    gptr(c.pick_p)[0] = make_float4(p0.x, p0.y, p0.z, INFINITY);
    gptr(c.pick_c)[0] =
        make_uint2(0u, pack_cell(c.r.blocks[0] - 1, c.r.blocks[1] - 1, c.r.blocks[2] - 1));
    gptr(c.out)[0] = 0;
    *gptr(c.iter) = 1;
    *gptr(c.done) = c.m <= 1 ? 1u : 0u;
  }
  for (uint32_t j = tid; j < kHists * kHistBins; j += kPassThreads) gptr(c.hist)[j] = 0;
}

// ---------------------------------------------------------------- launchers

hipError_t launch_runs_init(const CloudDev *d_clouds, uint32_t nclouds, hipStream_t st) {
  k_runs_init<<<nclouds, kPassThreads, 0, st>>>(d_clouds);
  return hipGetLastError();
}

hipError_t launch_rounds(const CloudDev *d_clouds, uint32_t nclouds, uint32_t max_nl1,
                         uint32_t rounds, hipStream_t st) {
  const dim3 grid(max_nl1, nclouds);
  for (uint32_t r = 0; r < rounds; ++r) {
    k_update<<<grid, kPassThreads, 0, st>>>(d_clouds);
    for (uint32_t p = 1; p <= kRefinePasses; ++p) k_refine<<<grid, kPassThreads, 0, st>>>(d_clouds, p);
    k_gather<<<grid, kPassThreads, 0, st>>>(d_clouds);
    k_run<<<nclouds, kListCap, 0, st>>>(d_clouds);
  }
  return hipGetLastError();
}

}  // namespace nsfps
