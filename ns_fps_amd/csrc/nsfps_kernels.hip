// HIP kernels of the FPS path for gfx950 (CDNA4, wave64).
//
// Build: per-point bucket key (reference cell rule), two stable LSD radix sorts
// (bucket order = the reference's logical order; then a sub-cell Morton order
// inside each bucket for tight leaf boxes), SoA gather, cell/leaf tables and
// leaf bounding boxes.
//
// Sampling: iteration i selects the maximum of a packed 64-bit key
// (min-distance bits << 32 | ~logical rank), which is the reference's
// leftmost maximum in logical order (src/yuezu_fps.cpp:245-261, 324-372),
// updates every point of every bucket inside the reference's cube of cells
// (src/yuezu_fps.cpp:560-597) -- skipping a leaf only when its bounding-box
// lower bound proves the update a no-op -- and re-reduces the dirty tree paths.
//
// All distance arithmetic is fp32 without contraction:
// d = fl(fl(fl(dx*dx) + fl(dy*dy)) + fl(dz*dz)), dx = fl(px - qx)
// (src/yuezu_fps.cpp:205-209).  sqrtf and '/' are correctly rounded.
#include <hip/hip_runtime.h>

#include <float.h>
#include <math.h>
#include <stdint.h>

#include "nsfps_internal.h"
#include "nsfps_launch.h"

#pragma clang fp contract(off)

namespace nsfps {

// ---------------------------------------------------------------------------
// Exact helpers shared by build and sampling
// ---------------------------------------------------------------------------

// std::min(v, hi) / std::max(lo, v) with <algorithm>'s comparison order.
__device__ __forceinline__ float std_min(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float std_max(float a, float b) { return (a < b) ? b : a; }

// Point3D::compute_block_indices, one axis (src/yuezu_fps.cpp:170-193).
__device__ __forceinline__ uint32_t cell_axis(const RangeDev &r, int a, float v) {
  float c = std_max(r.mn[a], std_min(v, r.hiclamp[a]));
  uint32_t i = (uint32_t)((c - r.mn[a]) * r.inv_bs[a]);
  return i < r.blocks[a] - 1 ? i : r.blocks[a] - 1;
}

__device__ __forceinline__ uint32_t bucket_of(const RangeDev &r, const uint32_t *lut,
                                              uint32_t ix, uint32_t iy, uint32_t iz) {
  uint32_t code = lut[r.lut_off[0] + ix] | lut[r.lut_off[1] + iy] | lut[r.lut_off[2] + iz];
  return r.bijective ? code : code % r.T;
}

// squared_distance (src/yuezu_fps.cpp:205-209), no FMA.
__device__ __forceinline__ float sqdist(float px, float py, float pz, float qx, float qy,
                                        float qz) {
  float dx = px - qx, dy = py - qy, dz = pz - qz;
  float s = dx * dx + dy * dy;
  return s + dz * dz;
}

// Lower bound of sqdist over a box, same operation order; monotone rounding
// makes it <= sqdist(p, q) for every p inside the box.
__device__ __forceinline__ float box_lb(float qx, float qy, float qz, float4 lo, float4 hi) {
  float gx = qx < lo.x ? lo.x - qx : (qx > hi.x ? qx - hi.x : 0.0f);
  float gy = qy < lo.y ? lo.y - qy : (qy > hi.y ? qy - hi.y : 0.0f);
  float gz = qz < lo.z ? lo.z - qz : (qz > hi.z ? qz - hi.z : 0.0f);
  float s = gx * gx + gy * gy;
  return s + gz * gz;
}

// Cube half-width of get_morton_codes_in_range (src/yuezu_fps.cpp:564-570):
// (int)ceil(sqrtf(D) / block_size), clamped to the grid size (any larger value
// covers the same cells).
__device__ __forceinline__ int cube_half(float D, float bs, uint32_t blocks) {
  float rad = sqrtf(D < 0.0f ? 0.0f : D);
  float f = ceilf(rad / bs);
  if (!(f < (float)blocks)) return (int)blocks;
  return (int)f;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint64_t o = __shfl_xor(k, off, 64);
    k = o > k ? o : k;
  }
  return k;
}

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// ---------------------------------------------------------------------------
// Build kernels
// ---------------------------------------------------------------------------

// Bucket (reference cell rule, % T) and sub-cell Morton code per input row;
// bucket populations by atomics; flags non-finite coordinates.
__global__ void k_cell_keys(const float *__restrict__ xyz, uint32_t n, RangeDev r,
                            const uint32_t *__restrict__ lut, uint32_t *__restrict__ bucket,
                            uint32_t *__restrict__ fine, uint32_t *__restrict__ counts,
                            uint32_t *__restrict__ bad) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v[3] = {xyz[3 * (size_t)i], xyz[3 * (size_t)i + 1], xyz[3 * (size_t)i + 2]};
  uint32_t c[3], f = 0;
  bool finite = true;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    finite = finite && isfinite(v[a]);
    c[a] = cell_axis(r, a, v[a]);
    // sub-cell position, 3 bits per axis (only orders points inside a cell)
    float cl = std_max(r.mn[a], std_min(v[a], r.hiclamp[a]));
    float t = (cl - r.mn[a]) * r.inv_bs[a] - (float)c[a];
    int s = (int)(t * 8.0f);
    s = s < 0 ? 0 : (s > 7 ? 7 : s);
    // interleave: bit k of s -> bit 3k + a
#pragma unroll
    for (int k = 0; k < 3; ++k) f |= (uint32_t)((s >> k) & 1) << (3 * k + a);
  }
  if (!finite) atomicOr(bad, 1u);
  uint32_t b = bucket_of(r, lut, c[0], c[1], c[2]);
  bucket[i] = b;
  fine[i] = f;
  atomicAdd(&counts[b], 1u);
}

// --- stable LSD radix sort (8-bit digits), keys/values u32 -----------------
constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;  // per wave: 16 rounds x 64 lanes
constexpr int kSortTile = kSortThreads * kSortRounds;  // 4096

__global__ __launch_bounds__(kSortThreads) void k_radix_hist(const uint32_t *__restrict__ keys,
                                                            uint32_t n, int shift,
                                                            uint32_t *__restrict__ hist,
                                                            uint32_t nblocks) {
  __shared__ uint32_t cnt[256];
  cnt[threadIdx.x] = 0;
  __syncthreads();
  size_t base = (size_t)blockIdx.x * kSortTile;
  for (int i = threadIdx.x; i < kSortTile; i += kSortThreads) {
    size_t e = base + i;
    if (e < n) atomicAdd(&cnt[(keys[e] >> shift) & 255u], 1u);
  }
  __syncthreads();
  hist[(size_t)threadIdx.x * nblocks + blockIdx.x] = cnt[threadIdx.x];
}

// Exclusive scan of len u32 in place by one 1024-thread workgroup; data[len]
// receives the total.
__global__ __launch_bounds__(1024) void k_scan_excl(uint32_t *__restrict__ data, uint32_t len) {
  __shared__ uint32_t wsum[16];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t per = (len + 1023) / 1024;
  uint32_t b = tid * per, e = b + per < len ? b + per : len;
  uint32_t s = 0;
  for (uint32_t i = b; i < e; ++i) s += data[i];
  // inclusive scan across the block
  uint32_t v = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t o = __shfl_up(v, off, 64);
    if (lane >= (uint32_t)off) v += o;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  if (wave == 0) {
    uint32_t w = lane < 16 ? wsum[lane] : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      uint32_t o = __shfl_up(w, off, 64);
      if (lane >= (uint32_t)off) w += o;
    }
    if (lane < 16) wsum[lane] = w;
  }
  __syncthreads();
  uint32_t run = v - s + (wave ? wsum[wave - 1] : 0);
  for (uint32_t i = b; i < e; ++i) {
    uint32_t t = data[i];
    data[i] = run;
    run += t;
  }
  if (tid == 1023) data[len] = wsum[15];
}

__global__ __launch_bounds__(kSortThreads) void k_radix_scatter(
    const uint32_t *__restrict__ kin, const uint32_t *__restrict__ vin, uint32_t *__restrict__ kout,
    uint32_t *__restrict__ vout, uint32_t n, int shift, const uint32_t *__restrict__ hist,
    uint32_t nblocks) {
  __shared__ uint32_t wcnt[kSortThreads / 64][256];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < (kSortThreads / 64) * 256; i += kSortThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  const size_t base = (size_t)blockIdx.x * kSortTile + (size_t)wave * (64 * kSortRounds);
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  uint32_t key[kSortRounds], val[kSortRounds], rnk[kSortRounds];
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    size_t e = base + (size_t)r * 64 + lane;
    bool valid = e < n;
    key[r] = valid ? kin[e] : 0u;
    val[r] = valid ? (vin ? vin[e] : (uint32_t)e) : 0u;
  }
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    size_t e = base + (size_t)r * 64 + lane;
    bool valid = e < n;
    uint32_t d = (key[r] >> shift) & 255u;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      uint64_t m = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? m : ~m;
    }
    uint32_t before = (uint32_t)__popcll(peers & lt);
    uint32_t baseq = valid ? wcnt[wave][d] : 0u;
    rnk[r] = baseq + before;
    // every lane has read its base before any leader writes (one wave, LDS
    // operations complete in order)
    __builtin_amdgcn_s_waitcnt(0xc07f);
    if (valid && before == 0) wcnt[wave][d] = baseq + (uint32_t)__popcll(peers);
    __builtin_amdgcn_s_waitcnt(0xc07f);
  }
  __syncthreads();
  // exclusive prefix over waves, per digit
  {
    uint32_t t = tid;  // 256 threads <-> 256 digits
    uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) {
      uint32_t c = wcnt[w][t];
      wcnt[w][t] = s;
      s += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    size_t e = base + (size_t)r * 64 + lane;
    if (e < n) {
      uint32_t d = (key[r] >> shift) & 255u;
      uint32_t pos = hist[(size_t)d * nblocks + blockIdx.x] + wcnt[wave][d] + rnk[r];
      kout[pos] = key[r];
      vout[pos] = val[r];
    }
  }
}

// Secondary key per logical position: bucket then sub-cell code; value =
// logical rank.
__global__ void k_key2(const uint32_t *__restrict__ lorig, const uint32_t *__restrict__ bucket,
                       const uint32_t *__restrict__ fine, uint32_t n, int fine_shift,
                       int fine_bits, uint32_t *__restrict__ key2) {
  uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  uint32_t o = lorig[p];
  uint32_t f = fine_bits > 0 ? (fine[o] >> fine_shift) : 0u;
  key2[p] = (bucket[o] << fine_bits) | f;
}

// SoA gather into physical order; C starts at FLT_MAX (src/yuezu_fps.cpp:215-223).
__global__ void k_gather(const uint32_t *__restrict__ prank, const uint32_t *__restrict__ lorig,
                         const float *__restrict__ xyz, uint32_t n, float *__restrict__ X,
                         float *__restrict__ Y, float *__restrict__ Z, float *__restrict__ C,
                         uint32_t *__restrict__ RANK, uint32_t *__restrict__ ORIG,
                         uint32_t *__restrict__ phys0) {
  uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  uint32_t rk = prank[p];
  uint32_t o = lorig[rk];
  X[p] = xyz[3 * (size_t)o];
  Y[p] = xyz[3 * (size_t)o + 1];
  Z[p] = xyz[3 * (size_t)o + 2];
  C[p] = FLT_MAX;
  RANK[p] = rk;
  ORIG[p] = o;
  if (o == 0) *phys0 = p;
}

__global__ void k_leaf_counts(const uint32_t *__restrict__ counts, uint32_t T,
                              uint32_t *__restrict__ lc) {
  uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= T) return;
  lc[b] = (counts[b] + kLeaf - 1) / kLeaf;
}

// Leaf descriptors: first slot, count and cell of every leaf of bucket b.
__global__ void k_leaf_desc(const uint32_t *__restrict__ cell_start,
                            const uint32_t *__restrict__ cell_leaf, uint32_t T, RangeDev r,
                            const float *__restrict__ X, const float *__restrict__ Y,
                            const float *__restrict__ Z, float4 *__restrict__ leaf_lo,
                            float4 *__restrict__ leaf_hi, uint32_t *__restrict__ leaf_cell) {
  uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= T) return;
  uint32_t s = cell_start[b], e = cell_start[b + 1];
  if (s == e) return;
  uint32_t l = cell_leaf[b];
  uint32_t cx = cell_axis(r, 0, X[s]), cy = cell_axis(r, 1, Y[s]), cz = cell_axis(r, 2, Z[s]);
  uint32_t packed = cx | (cy << 10) | (cz << 20);
  for (uint32_t p = s; p < e; p += kLeaf, ++l) {
    uint32_t cnt = e - p < kLeaf ? e - p : kLeaf;
    leaf_lo[l] = make_float4(0.f, 0.f, 0.f, __uint_as_float(p));
    leaf_hi[l] = make_float4(0.f, 0.f, 0.f, __uint_as_float(cnt));
    leaf_cell[l] = packed;
  }
}

// Leaf bounding boxes and initial keys (FLT_MAX, smallest rank in the leaf);
// one wave per leaf.
__global__ __launch_bounds__(256) void k_leaf_bbox(uint32_t nleaves, const float *__restrict__ X,
                                                   const float *__restrict__ Y,
                                                   const float *__restrict__ Z,
                                                   const uint32_t *__restrict__ RANK,
                                                   float4 *__restrict__ leaf_lo,
                                                   float4 *__restrict__ leaf_hi,
                                                   uint64_t *__restrict__ leaf_key,
                                                   uint32_t *__restrict__ leaf_win) {
  uint32_t leaf = blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t lane = lane_id();
  if (leaf >= nleaves) return;
  float4 lo = leaf_lo[leaf], hi = leaf_hi[leaf];
  uint32_t start = __float_as_uint(lo.w), cnt = __float_as_uint(hi.w);
  bool act = lane < cnt;
  uint32_t p = start + (act ? lane : 0);
  float x = X[p], y = Y[p], z = Z[p];
  float mnx = x, mny = y, mnz = z, mxx = x, mxy = y, mxz = z;
  uint64_t k = act ? make_key(FLT_MAX, RANK[p]) : 0ull;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mnx = fminf(mnx, __shfl_xor(mnx, off, 64));
    mny = fminf(mny, __shfl_xor(mny, off, 64));
    mnz = fminf(mnz, __shfl_xor(mnz, off, 64));
    mxx = fmaxf(mxx, __shfl_xor(mxx, off, 64));
    mxy = fmaxf(mxy, __shfl_xor(mxy, off, 64));
    mxz = fmaxf(mxz, __shfl_xor(mxz, off, 64));
  }
  uint64_t km = wave_max_u64(k);
  uint64_t who = __ballot(k == km && act);
  uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
  if (lane == 0) {
    leaf_lo[leaf] = make_float4(mnx, mny, mnz, lo.w);
    leaf_hi[leaf] = make_float4(mxx, mxy, mxz, hi.w);
    leaf_key[leaf] = km;
    leaf_win[leaf] = start + wl;
  }
}

// Level-1 keys from the initial leaf keys (one wave per node).
__global__ __launch_bounds__(256) void k_l1_init(uint32_t nleaves, uint32_t nl1,
                                                 const uint64_t *__restrict__ leaf_key,
                                                 const uint32_t *__restrict__ leaf_win,
                                                 uint64_t *__restrict__ l1_key,
                                                 uint32_t *__restrict__ l1_win) {
  uint32_t g = blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t lane = lane_id();
  if (g >= nl1) return;
  uint32_t j = g * kFan + lane;
  bool v = j < nleaves;
  uint64_t k = v ? leaf_key[j] : 0ull;
  uint32_t w = v ? leaf_win[j] : 0u;
  uint64_t km = wave_max_u64(k);
  uint64_t who = __ballot(k == km && v);
  uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
  uint32_t ww = __shfl(w, (int)wl, 64);
  if (lane == 0) {
    l1_key[g] = km;
    l1_win[g] = ww;
  }
}

__global__ void k_init_state(CloudDev c) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    *c.iter = 0;
    *c.done = 0;
    *c.counter = 0;
    *c.root_key = 0;
    *c.root_win = c.phys0;
  }
}

// ---------------------------------------------------------------------------
// Sampling
// ---------------------------------------------------------------------------

// Up to U leaves per wave in flight: bounding boxes and keys first, then the
// points of the leaves the lower bound cannot skip.  On return key[u]/win[u]
// hold each leaf's current key and winner; changed[u] is set when the leaf's
// points were updated.
// valid[u]: the leaf exists (its key is loaded); cand[u]: it is inside the
// cube and must be updated unless its lower bound proves the update a no-op.
template <int U>
__device__ __forceinline__ void process_leaves(const CloudDev &c, const uint32_t *leaf,
                                               const bool *valid, const bool *cand, float qx,
                                               float qy, float qz, uint64_t *key, uint32_t *win,
                                               bool *changed) {
  const uint32_t lane = lane_id();
  float4 lo[U], hi[U];
  bool go[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    changed[u] = false;
    key[u] = 0;
    win[u] = 0;
    lo[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    hi[u] = lo[u];
    if (valid[u]) {
      key[u] = c.leaf_key[leaf[u]];
      win[u] = c.leaf_win[leaf[u]];
      if (cand[u]) {
        lo[u] = c.leaf_lo[leaf[u]];
        hi[u] = c.leaf_hi[leaf[u]];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    go[u] = valid[u] && cand[u] && box_lb(qx, qy, qz, lo[u], hi[u]) < key_dist(key[u]);
  float px[U], py[U], pz[U], pc[U];
  uint32_t pr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    pc[u] = -1.0f;
    if (go[u]) {
      uint32_t start = __float_as_uint(lo[u].w), cnt = __float_as_uint(hi[u].w);
      if (lane < cnt) {
        uint32_t p = start + lane;
        px[u] = c.X[p];
        py[u] = c.Y[p];
        pz[u] = c.Z[p];
        pc[u] = c.C[p];
        pr[u] = c.RANK[p];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!go[u]) continue;
    uint32_t start = __float_as_uint(lo[u].w), cnt = __float_as_uint(hi[u].w);
    uint64_t k = 0;
    if (lane < cnt) {
      float d = sqdist(px[u], py[u], pz[u], qx, qy, qz);
      float cc = pc[u];
      if (d < cc) {
        cc = d;
        c.C[start + lane] = d;
      }
      k = make_key(cc, pr[u]);
    }
    uint64_t km = wave_max_u64(k);
    uint64_t who = __ballot(k == km && lane < cnt);
    uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
    changed[u] = true;
    key[u] = km;
    win[u] = start + wl;
    if (lane == 0) {
      c.leaf_key[leaf[u]] = km;
      c.leaf_win[leaf[u]] = start + wl;
    }
  }
}

struct Cube {
  int lo[3], hi[3];
};

__device__ __forceinline__ Cube make_cube(const RangeDev &r, float D, float qx, float qy,
                                          float qz) {
  Cube cb;
  float q[3] = {qx, qy, qz};
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    int h = cube_half(D, r.bsize[a], r.blocks[a]);
    int qc = (int)cell_axis(r, a, q[a]);
    int lo = qc - h, hi = qc + h;
    cb.lo[a] = lo < 0 ? 0 : lo;
    cb.hi[a] = hi > (int)r.blocks[a] - 1 ? (int)r.blocks[a] - 1 : hi;
  }
  return cb;
}

// One FPS iteration over the whole device: every workgroup owns level-1 nodes
// (64 leaves each), updates the candidate leaves among them and rewrites the
// node's key; the last workgroup to arrive reduces the level-1 keys to the
// root and advances the iteration.  Used while the cube is large.
__global__ __launch_bounds__(1024) void k_wide_step(CloudDev c) {
  __shared__ uint64_t s_key[64];
  __shared__ uint32_t s_win[64];
  __shared__ uint32_t s_last;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (*c.done) return;
  const uint32_t it = *c.iter;
  uint32_t w0;
  float D;
  if (it == 0) {
    w0 = c.phys0;
    D = INFINITY;
  } else {
    w0 = *c.root_win;
    D = key_dist(*c.root_key);
  }
  const float qx = c.X[w0], qy = c.Y[w0], qz = c.Z[w0];
  const bool update = it + 1 < c.m;
  if (blockIdx.x == 0 && tid == 0) c.out[it] = (int32_t)c.ORIG[w0];
  if (update) {
    const Cube cb = make_cube(c.r, D, qx, qy, qz);
    for (uint32_t g = blockIdx.x; g < c.nl1; g += gridDim.x) {
      // Candidate test by cell coordinates: valid only when bucket <-> cell
      // is one-to-one (the host runs this kernel only then).
      uint32_t leaf[4];
      bool valid[4], cand[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        leaf[u] = g * kFan + (uint32_t)u * 16 + wave;
        valid[u] = leaf[u] < c.nleaves;
        cand[u] = false;
        if (valid[u]) {
          uint32_t cell = c.leaf_cell[leaf[u]];
          int cx = cell & 1023, cy = (cell >> 10) & 1023, cz = cell >> 20;
          cand[u] = cx >= cb.lo[0] && cx <= cb.hi[0] && cy >= cb.lo[1] && cy <= cb.hi[1] &&
                    cz >= cb.lo[2] && cz <= cb.hi[2];
        }
      }
      uint64_t key[4];
      uint32_t win[4];
      bool changed[4];
      process_leaves<4>(c, leaf, valid, cand, qx, qy, qz, key, win, changed);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (lane == 0) {
          s_key[u * 16 + wave] = key[u];
          s_win[u * 16 + wave] = win[u];
        }
      }
      __syncthreads();
      if (wave == 0) {
        uint64_t k = s_key[lane];
        uint64_t km = wave_max_u64(k);
        uint64_t who = __ballot(k == km);
        uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
        if (lane == 0) {
          c.l1_key[g] = km;
          c.l1_win[g] = s_win[wl];
        }
      }
      __syncthreads();
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(c.counter, 1u) == gridDim.x - 1) ? 1u : 0u;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (!update) {
    if (tid == 0) {
      *c.iter = it + 1;
      *c.done = 1;
      *c.counter = 0;
    }
    return;
  }
  // root = max over level-1 keys
  uint64_t best = 0;
  uint32_t bw = 0;
  for (uint32_t j = tid; j < c.nl1; j += 1024) {
    uint64_t k = __hip_atomic_load(&c.l1_key[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k > best) {
      best = k;
      bw = __hip_atomic_load(&c.l1_win[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  uint64_t km = wave_max_u64(best);
  uint64_t who = __ballot(best == km);
  uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
  uint32_t wwin = __shfl(bw, (int)wl, 64);
  if (lane == 0) {
    s_key[wave] = km;
    s_win[wave] = wwin;
  }
  __syncthreads();
  if (wave == 0) {
    uint64_t k = lane < 16 ? s_key[lane] : 0ull;
    uint64_t kk = wave_max_u64(k);
    uint64_t wh = __ballot(k == kk && lane < 16);
    uint32_t l2 = (uint32_t)__ffsll((long long)wh) - 1;
    if (lane == 0) {
      *c.root_key = kk;
      *c.root_win = s_win[l2];
      *c.iter = it + 1;
      if (!(key_dist(kk) > 0.0f)) *c.done = 1;
      *c.counter = 0;
    }
  }
}

// LDS layout of the single-workgroup loop (dynamic shared memory).
struct LateLds {
  uint64_t *l1k;
  uint32_t *l1w;
  uint16_t *dl1;    // dirty level-1 list
  uint32_t *m1;     // dirty level-1 bitmask
  uint64_t *l2k;    // <= 128 level-2 nodes
  uint32_t *l2w;
  uint16_t *dl2;
  uint32_t *m2;
  uint32_t *cand;   // flattened candidate leaves of the current round
};

constexpr uint32_t kCandCap = 4096;
constexpr uint32_t kMaxL2 = kMaxL1 / kFan;  // 128

__host__ __device__ inline size_t late_lds_bytes(uint32_t nl1) {
  size_t b = 0;
  b += (size_t)nl1 * 8;                 // l1k
  b += (size_t)nl1 * 4;                 // l1w
  b += ((size_t)nl1 * 2 + 15) & ~15ull; // dl1
  b += (((size_t)nl1 + 31) / 32) * 4 + 16;
  b += kMaxL2 * 8 + kMaxL2 * 4 + kMaxL2 * 2 + 16 + 16;
  b += kCandCap * 4;
  return (b + 255) & ~255ull;
}

__device__ inline LateLds carve(unsigned char *base, uint32_t nl1) {
  LateLds s;
  size_t o = 0;
  s.l1k = (uint64_t *)(base + o);
  o += (size_t)nl1 * 8;
  s.l1w = (uint32_t *)(base + o);
  o += (size_t)nl1 * 4;
  s.dl1 = (uint16_t *)(base + o);
  o += ((size_t)nl1 * 2 + 15) & ~15ull;
  s.m1 = (uint32_t *)(base + o);
  o += (((size_t)nl1 + 31) / 32) * 4 + 16;
  s.l2k = (uint64_t *)(base + o);
  o += kMaxL2 * 8;
  s.l2w = (uint32_t *)(base + o);
  o += kMaxL2 * 4;
  s.dl2 = (uint16_t *)(base + o);
  o += kMaxL2 * 2 + 16;
  s.m2 = (uint32_t *)(base + o);
  o += 16;
  s.cand = (uint32_t *)(base + o);
  return s;
}

// Block-wide exclusive scan of one value per thread (1024 threads).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *total) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t o = __shfl_up(x, off, 64);
    if (lane >= (uint32_t)off) x += o;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    uint32_t w = lane < 16 ? wsum[lane] : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      uint32_t o = __shfl_up(w, off, 64);
      if (lane >= (uint32_t)off) w += o;
    }
    if (lane < 16) wsum[16 + lane] = w;
  }
  __syncthreads();
  *total = wsum[16 + 15];
  uint32_t r = x - v + (wave ? wsum[16 + wave - 1] : 0);
  __syncthreads();
  return r;
}

// Mark level-1 node g dirty (first marker appends it to the list).
__device__ __forceinline__ void mark_dirty(uint32_t *mask, uint16_t *list, uint32_t *count,
                                           uint32_t g) {
  uint32_t bit = 1u << (g & 31);
  uint32_t old = atomicOr(&mask[g >> 5], bit);
  if (!(old & bit)) {
    uint32_t i = atomicAdd(count, 1u);
    list[i] = (uint16_t)g;
  }
}

// The sampling loop of one cloud in one 1024-thread workgroup: upper tree
// levels live in LDS, the loop never returns to the host.  blockIdx.x selects
// the cloud (batched mode launches one workgroup per cloud).
__global__ __launch_bounds__(1024) void k_late_loop(const CloudDev *__restrict__ clouds) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ uint32_t s_scan[32];
  __shared__ uint32_t s_n1, s_n2;
  __shared__ uint64_t s_root_key;
  __shared__ uint32_t s_root_win;
  const CloudDev c = clouds[blockIdx.x];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (*c.done) return;
  const uint32_t nl1 = c.nl1;
  const uint32_t nl2 = (nl1 + kFan - 1) / kFan;
  LateLds s = carve(lds_raw, nl1);
  uint32_t it = *c.iter;
  // Load level 1 from the grid-wide phase (or build it here when starting at
  // iteration 0: it is rebuilt after the first full update anyway).
  for (uint32_t j = tid; j < nl1; j += 1024) {
    s.l1k[j] = c.l1_key[j];
    s.l1w[j] = c.l1_win[j];
  }
  for (uint32_t j = tid; j < (nl1 + 31) / 32; j += 1024) s.m1[j] = 0;
  if (tid < 4) s.m2[tid] = 0;
  if (tid == 0) {
    s_n1 = 0;
    s_n2 = 0;
    s_root_key = *c.root_key;
    s_root_win = *c.root_win;
  }
  __syncthreads();
  // level 2 from level 1
  for (uint32_t h = wave; h < nl2; h += 16) {
    uint32_t j = h * kFan + lane;
    uint64_t k = j < nl1 ? s.l1k[j] : 0ull;
    uint64_t km = wave_max_u64(k);
    uint64_t who = __ballot(k == km && j < nl1);
    uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
    if (lane == 0) {
      s.l2k[h] = km;
      s.l2w[h] = s.l1w[h * kFan + wl];
    }
  }
  __syncthreads();

  while (true) {
    uint32_t w0;
    float D;
    if (it == 0) {
      w0 = c.phys0;
      D = INFINITY;
    } else {
      uint64_t rk = s_root_key;
      w0 = s_root_win;
      D = key_dist(rk);
      if (!(D > 0.0f)) break;
    }
    if (it >= c.m) break;
    const float qx = c.X[w0], qy = c.Y[w0], qz = c.Z[w0];
    if (tid == 0) c.out[it] = (int32_t)c.ORIG[w0];
    ++it;
    if (it >= c.m) break;
    const Cube cb = make_cube(c.r, D, qx, qy, qz);
    const uint32_t ex = (uint32_t)(cb.hi[0] - cb.lo[0] + 1);
    const uint32_t ey = (uint32_t)(cb.hi[1] - cb.lo[1] + 1);
    const uint32_t ez = (uint32_t)(cb.hi[2] - cb.lo[2] + 1);
    const uint32_t ncell = ex * ey * ez;
    for (uint32_t cbase = 0; cbase < ncell; cbase += kCellChunk) {
      uint32_t t = cbase + tid;
      uint32_t l0 = 0, cnt = 0;
      if (t < ncell) {
        uint32_t ix = t % ex, iy = (t / ex) % ey, iz = t / (ex * ey);
        uint32_t b = bucket_of(c.r, c.lut, (uint32_t)cb.lo[0] + ix, (uint32_t)cb.lo[1] + iy,
                               (uint32_t)cb.lo[2] + iz);
        l0 = c.cell_leaf[b];
        cnt = c.cell_leaf[b + 1] - l0;
      }
      uint32_t total;
      uint32_t off = block_excl_scan(cnt, s_scan, &total);
      for (uint32_t rb = 0; rb < total; rb += kCandCap) {
        // flatten this thread's leaves that fall in [rb, rb + kCandCap)
        uint32_t a = off > rb ? off : rb;
        uint32_t e = off + cnt < rb + kCandCap ? off + cnt : rb + kCandCap;
        for (uint32_t k = a; k < e; ++k) s.cand[k - rb] = l0 + (k - off);
        __syncthreads();
        uint32_t nr = total - rb < kCandCap ? total - rb : kCandCap;
        for (uint32_t jb = 0; jb < nr; jb += 64) {
          uint32_t leaf[4];
          bool valid[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            uint32_t j = jb + wave * 4 + (uint32_t)u;
            valid[u] = j < nr;
            leaf[u] = valid[u] ? s.cand[j] : 0u;
          }
          uint64_t key[4];
          uint32_t win[4];
          bool changed[4];
          process_leaves<4>(c, leaf, valid, valid, qx, qy, qz, key, win, changed);
          if (lane == 0) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (changed[u]) mark_dirty(s.m1, s.dl1, &s_n1, leaf[u] / kFan);
          }
        }
        __syncthreads();
      }
    }
    // rebuild dirty level-1 nodes from the leaf keys
    const uint32_t n1 = s_n1;
    for (uint32_t x = wave; x < n1; x += 16) {
      uint32_t g = s.dl1[x];
      uint32_t j = g * kFan + lane;
      bool v = j < c.nleaves;
      uint64_t k = v ? c.leaf_key[j] : 0ull;
      uint32_t w = v ? c.leaf_win[j] : 0u;
      uint64_t km = wave_max_u64(k);
      uint64_t who = __ballot(k == km && v);
      uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
      uint32_t ww = __shfl(w, (int)wl, 64);
      if (lane == 0) {
        s.l1k[g] = km;
        s.l1w[g] = ww;
        s.m1[g >> 5] = 0;  // whole word: every bit in it is rebuilt this pass
        mark_dirty(s.m2, s.dl2, &s_n2, g / kFan);
      }
    }
    __syncthreads();
    if (tid == 0) s_n1 = 0;
    // m1 words were zeroed by whichever wave rebuilt a node in them; nodes in
    // the same word are all rebuilt in this pass, so no bit survives.
    const uint32_t n2 = s_n2;
    for (uint32_t x = wave; x < n2; x += 16) {
      uint32_t h = s.dl2[x];
      uint32_t j = h * kFan + lane;
      bool v = j < nl1;
      uint64_t k = v ? s.l1k[j] : 0ull;
      uint64_t km = wave_max_u64(k);
      uint64_t who = __ballot(k == km && v);
      uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
      if (lane == 0) {
        s.l2k[h] = km;
        s.l2w[h] = s.l1w[h * kFan + wl];
      }
    }
    __syncthreads();
    if (wave == 0) {
      uint64_t k0 = lane < nl2 ? s.l2k[lane] : 0ull;
      uint64_t k1 = lane + 64 < nl2 ? s.l2k[lane + 64] : 0ull;
      uint32_t i0 = lane, i1 = lane + 64;
      uint64_t k = k0;
      uint32_t ii = i0;
      if (k1 > k) {
        k = k1;
        ii = i1;
      }
      uint64_t km = wave_max_u64(k);
      uint64_t who = __ballot(k == km);
      uint32_t wl = (uint32_t)__ffsll((long long)who) - 1;
      uint32_t idx = __shfl(ii, (int)wl, 64);
      if (lane == 0) {
        s_root_key = km;
        s_root_win = s.l2w[idx];
        s_n2 = 0;
        s.m2[0] = 0;
        s.m2[1] = 0;
        s.m2[2] = 0;
        s.m2[3] = 0;
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    *c.iter = it;
    *c.done = 1;
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

hipError_t launch_cell_keys(const float *xyz, uint32_t n, const RangeDev &r, const uint32_t *lut,
                            uint32_t *bucket, uint32_t *fine, uint32_t *counts, uint32_t *bad,
                            hipStream_t st) {
  if (n == 0) return hipSuccess;
  k_cell_keys<<<cdiv(n, 256), 256, 0, st>>>(xyz, n, r, lut, bucket, fine, counts, bad);
  return hipGetLastError();
}

hipError_t launch_scan(uint32_t *data, uint32_t len, hipStream_t st) {
  k_scan_excl<<<1, 1024, 0, st>>>(data, len);
  return hipGetLastError();
}

uint32_t radix_hist_len(uint32_t n) { return 256u * cdiv(n, kSortTile) + 1; }

hipError_t launch_radix_sort(uint32_t *keys, uint32_t *vals, uint32_t *keys_tmp,
                             uint32_t *vals_tmp, uint32_t n, int key_bits, uint32_t *hist,
                             bool iota_values, uint32_t **keys_out, uint32_t **vals_out,
                             hipStream_t st) {
  uint32_t nb = cdiv(n, kSortTile);
  uint32_t *ka = keys, *va = vals, *kb = keys_tmp, *vb = vals_tmp;
  bool first = true;
  for (int shift = 0; shift < key_bits; shift += 8) {
    k_radix_hist<<<nb, kSortThreads, 0, st>>>(ka, n, shift, hist, nb);
    k_scan_excl<<<1, 1024, 0, st>>>(hist, 256u * nb);
    k_radix_scatter<<<nb, kSortThreads, 0, st>>>(ka, (first && iota_values) ? nullptr : va, kb,
                                                 vb, n, shift, hist, nb);
    first = false;
    uint32_t *t = ka;
    ka = kb;
    kb = t;
    t = va;
    va = vb;
    vb = t;
  }
  if (first && iota_values) {
    // zero passes (key_bits == 0): values are the identity
    return hipErrorInvalidValue;
  }
  *keys_out = ka;
  *vals_out = va;
  return hipGetLastError();
}

hipError_t launch_key2(const uint32_t *lorig, const uint32_t *bucket, const uint32_t *fine,
                       uint32_t n, int fine_shift, int fine_bits, uint32_t *key2,
                       hipStream_t st) {
  k_key2<<<cdiv(n, 256), 256, 0, st>>>(lorig, bucket, fine, n, fine_shift, fine_bits, key2);
  return hipGetLastError();
}

hipError_t launch_gather(const uint32_t *prank, const uint32_t *lorig, const float *xyz,
                         uint32_t n, float *X, float *Y, float *Z, float *C, uint32_t *RANK,
                         uint32_t *ORIG, uint32_t *phys0, hipStream_t st) {
  k_gather<<<cdiv(n, 256), 256, 0, st>>>(prank, lorig, xyz, n, X, Y, Z, C, RANK, ORIG, phys0);
  return hipGetLastError();
}

hipError_t launch_leaf_counts(const uint32_t *counts, uint32_t T, uint32_t *lc, hipStream_t st) {
  k_leaf_counts<<<cdiv(T, 256), 256, 0, st>>>(counts, T, lc);
  return hipGetLastError();
}

hipError_t launch_leaf_build(const uint32_t *cell_start, const uint32_t *cell_leaf, uint32_t T,
                             uint32_t nleaves, const RangeDev &r, const float *X, const float *Y,
                             const float *Z, const uint32_t *RANK, float4 *leaf_lo,
                             float4 *leaf_hi, uint32_t *leaf_cell, uint64_t *leaf_key,
                             uint32_t *leaf_win, hipStream_t st) {
  k_leaf_desc<<<cdiv(T, 256), 256, 0, st>>>(cell_start, cell_leaf, T, r, X, Y, Z, leaf_lo, leaf_hi,
                                            leaf_cell);
  if (nleaves)
    k_leaf_bbox<<<cdiv(nleaves, 4), 256, 0, st>>>(nleaves, X, Y, Z, RANK, leaf_lo, leaf_hi,
                                                  leaf_key, leaf_win);
  return hipGetLastError();
}

hipError_t launch_init_state(const CloudDev &c, hipStream_t st) {
  if (c.nl1)
    k_l1_init<<<cdiv(c.nl1, 4), 256, 0, st>>>(c.nleaves, c.nl1, c.leaf_key, c.leaf_win, c.l1_key,
                                              c.l1_win);
  k_init_state<<<1, 64, 0, st>>>(c);
  return hipGetLastError();
}

hipError_t launch_wide_steps(const CloudDev &c, uint32_t steps, uint32_t grid, hipStream_t st) {
  for (uint32_t s = 0; s < steps; ++s) {
    k_wide_step<<<grid, 1024, 0, st>>>(c);
  }
  return hipGetLastError();
}

size_t late_lds(uint32_t max_nl1) { return late_lds_bytes(max_nl1); }

hipError_t launch_late_loop(const CloudDev *d_clouds, uint32_t nclouds, uint32_t max_nl1,
                            hipStream_t st) {
  size_t lds = late_lds_bytes(max_nl1);
  hipError_t e = hipFuncSetAttribute((const void *)k_late_loop,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  k_late_loop<<<nclouds, 1024, lds, st>>>(d_clouds);
  return hipGetLastError();
}

}  // namespace nsfps
