// The step after sampling: gather of the sampled points and the ball query of
// set-abstraction grouping, on the FPS output (int32 indices).
//
// The reference stops at the indices; its callers' next step is PointNet++'s
// sample-and-group (Qi et al., "PointNet++", NeurIPS 2017, the
// query_ball_point operator): for each center, the first nsample point
// indices in input order whose squared distance is below radius^2, the rest
// of the row repeating the first one found, a row of zeros when none is.  The
// distance is the FPS distance, ((dx*dx + dy*dy) + dz*dz) with no
// contraction, so grouping agrees bit for bit with the sampler's geometry.
//
// Ball query.  Small clouds: one wave per center scans the points in input
// order, 64 a step; a ballot gives the step's hits in index order, their ranks
// place them, and the wave leaves once nsample are found.  Large clouds: a
// uniform grid with cells of at least 1.01 * radius per axis (at most 128 per
// axis) over the finite points' bounds; a stable sort by cell keeps each
// cell's points in index order; one wave per center collects the hits of the
// 27 cells around the center's cell (every point closer than the radius lies
// in one of them: the cell index is floor((v - min) * inv_cs) clamped to the
// grid, non-expansive, and rounding moves it by far less than the 1 % margin),
// each cell's hits forming an index-sorted run in LDS, then a 27-way merge of
// the runs emits the nsample smallest indices, which are the first hits in
// input order.  A center with more than kBqCap hits is handed to the scan.

#include <hip/hip_runtime.h>

#include "nsfps_device.h"
#include "nsfps_launch.h"

#include <algorithm>

namespace nsfps {

namespace {

constexpr uint32_t kGroupWaves = 4;  // centers per 256-thread workgroup
constexpr uint32_t kBqCap = 1024;    // hits one wave holds for a center (grid path)

__global__ __launch_bounds__(256) void k_gather_points(const float *__restrict__ xyz, uint32_t n,
                                                       const int32_t *__restrict__ idx,
                                                       uint32_t m, float *__restrict__ out,
                                                       uint32_t *__restrict__ bad) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const int32_t k = idx[i];
  if (k < 0 || (uint32_t)k >= n) {  // never read outside the cloud
    atomicOr(bad, 1u);
    out[3 * (size_t)i] = out[3 * (size_t)i + 1] = out[3 * (size_t)i + 2] = 0.f;
    return;
  }
  out[3 * (size_t)i] = xyz[3 * (size_t)k];
  out[3 * (size_t)i + 1] = xyz[3 * (size_t)k + 1];
  out[3 * (size_t)i + 2] = xyz[3 * (size_t)k + 2];
}

__global__ __launch_bounds__(256) void k_ball_query(const float *__restrict__ xyz, uint32_t n,
                                                    const float *__restrict__ centers,
                                                    const uint32_t *__restrict__ ids, uint32_t m,
                                                    float r2, uint32_t nsample,
                                                    int32_t *__restrict__ out) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t w = blockIdx.x * kGroupWaves + (threadIdx.x >> 6);
  if (w >= m) return;  // whole waves leave together
  const uint32_t j = ids ? ids[w] : w;  // ids: centers of this pass (all < the center count)
  const float cx = centers[3 * (size_t)j], cy = centers[3 * (size_t)j + 1],
              cz = centers[3 * (size_t)j + 2];
  int32_t *const row = out + (size_t)j * nsample;
  uint32_t cnt = 0, first = 0;
  for (uint32_t base = 0; base < n && cnt < nsample; base += 64) {
    const uint32_t i = base + lane;
    bool hit = false;
    if (i < n) {
      const float d2 = sqdist(xyz[3 * (size_t)i], xyz[3 * (size_t)i + 1], xyz[3 * (size_t)i + 2],
                              cx, cy, cz);
      hit = d2 < r2;
    }
    const uint64_t mask = __ballot(hit);
    if (mask) {
      if (cnt == 0) first = base + (uint32_t)__builtin_ctzll(mask);
      const uint32_t pos = cnt + lanes_below(mask);
      if (hit && pos < nsample) row[pos] = (int32_t)i;
      cnt += (uint32_t)__popcll(mask);
    }
  }
  const uint32_t filled = cnt < nsample ? cnt : nsample;
  const int32_t pad = cnt ? (int32_t)first : 0;
  for (uint32_t k = filled + lane; k < nsample; k += 64) row[k] = pad;
}

// ---- grid path

// bnd[0..2]: ord(min) per axis (start 0xffffffff), bnd[3..5]: ord(max) (start 0),
// over the finite points
__global__ __launch_bounds__(256) void k_bq_bounds(const float *__restrict__ xyz, uint32_t n,
                                                   uint32_t *__restrict__ bnd) {
  uint32_t lo[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, hi[3] = {0u, 0u, 0u};
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float x = xyz[3 * (size_t)i], y = xyz[3 * (size_t)i + 1], z = xyz[3 * (size_t)i + 2];
    if (isfinite(x) && isfinite(y) && isfinite(z)) {
      const uint32_t o[3] = {ord_of(x), ord_of(y), ord_of(z)};
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        lo[a] = min(lo[a], o[a]);
        hi[a] = max(hi[a], o[a]);
      }
    }
  }
  // one atomic per value and workgroup: the six addresses are shared by the
  // whole grid, and contended atomics on one address serialise
  __shared__ uint32_t s_b[4][6];
  const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const uint32_t l = wave_min_u32(lo[a]), h = wave_max_u32(hi[a]);
    if ((threadIdx.x & 63u) == 0) {
      s_b[wave][a] = l;
      s_b[wave][3 + a] = h;
    }
  }
  __syncthreads();
  if (threadIdx.x < 6) {
    const uint32_t a = threadIdx.x;
    uint32_t v = s_b[0][a];
    for (uint32_t w = 1; w < 4; ++w) v = a < 3 ? min(v, s_b[w][a]) : max(v, s_b[w][a]);
    if (a < 3) atomicMin(&bnd[a], v);
    else atomicMax(&bnd[a], v);
  }
}

__device__ __forceinline__ uint32_t bq_axis(const BqGrid &g, int a, float v) {
  float t = (v - g.mn[a]) * g.inv_cs[a];
  t = fminf(fmaxf(t, 0.f), (float)(g.dim[a] - 1));  // NaN -> 0
  return (uint32_t)t;
}

__global__ void k_bq_grid(const uint32_t *__restrict__ bnd, float radius,
                          BqGrid *__restrict__ g) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  uint32_t cells = 1;
  for (int a = 0; a < 3; ++a) {
    float lo = float_of(bnd[a]), hi = float_of(bnd[3 + a]);
    if (!(bnd[a] <= bnd[3 + a])) lo = hi = 0.f;  // no finite point
    const float ext = hi - lo;
    const float cs = fmaxf(radius * 1.01f, ext / (float)(kBqMaxDim - 1));
    uint32_t dim = 1;
    float inv = 0.f;
    if (cs > 0.f && isfinite(cs)) {
      const float q = fminf(ext / cs, (float)(kBqMaxDim - 1));
      dim = (uint32_t)q + 1;
      inv = 1.f / cs;
    }
    g->mn[a] = lo;
    g->inv_cs[a] = inv;
    g->dim[a] = dim;
    cells *= dim;
  }
  g->ncells = cells;
}

// key: the point's cell, or ncells for a point with a non-finite coordinate
__global__ __launch_bounds__(256) void k_bq_keys(const float *__restrict__ xyz, uint32_t n,
                                                 const BqGrid *__restrict__ gp,
                                                 uint32_t *__restrict__ keys) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const BqGrid g = *gp;
  const float x = xyz[3 * (size_t)i], y = xyz[3 * (size_t)i + 1], z = xyz[3 * (size_t)i + 2];
  keys[i] = (isfinite(x) && isfinite(y) && isfinite(z))
                ? (bq_axis(g, 2, z) * g.dim[1] + bq_axis(g, 1, y)) * g.dim[0] + bq_axis(g, 0, x)
                : g.ncells;
}

// cell ranges of the sorted keys (cstart/cend zeroed before) and the points
// in sorted order with their input index
__global__ __launch_bounds__(256) void k_bq_cells(const uint32_t *__restrict__ skeys,
                                                  const uint32_t *__restrict__ sidx, uint32_t n,
                                                  const float *__restrict__ xyz,
                                                  const BqGrid *__restrict__ gp,
                                                  uint32_t *__restrict__ cstart,
                                                  uint32_t *__restrict__ cend,
                                                  float4 *__restrict__ spts) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t k = skeys[i], r = sidx[i];
  spts[i] = make_float4(xyz[3 * (size_t)r], xyz[3 * (size_t)r + 1], xyz[3 * (size_t)r + 2],
                        __uint_as_float(r));
  if (k >= gp->ncells) return;  // non-finite points: never candidates
  if (i == 0 || skeys[i - 1] != k) cstart[k] = i;
  if (i == n - 1 || skeys[i + 1] != k) cend[k] = i + 1;
}

__global__ __launch_bounds__(256) void k_bq_query(const float4 *__restrict__ spts,
                                                  const BqGrid *__restrict__ gp,
                                                  const uint32_t *__restrict__ cstart,
                                                  const uint32_t *__restrict__ cend,
                                                  const float *__restrict__ centers, uint32_t m,
                                                  float r2, uint32_t nsample,
                                                  int32_t *__restrict__ out,
                                                  uint32_t *__restrict__ ovf_ids,
                                                  uint32_t *__restrict__ ovf_count) {
  __shared__ uint32_t s_hits[kGroupWaves][kBqCap];
  __shared__ uint32_t s_runs[kGroupWaves][32];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t j = blockIdx.x * kGroupWaves + wave;
  if (j >= m) return;  // waves are independent: no barrier below
  const BqGrid g = *gp;
  const float cx = centers[3 * (size_t)j], cy = centers[3 * (size_t)j + 1],
              cz = centers[3 * (size_t)j + 2];
  const int gx = (int)bq_axis(g, 0, cx), gy = (int)bq_axis(g, 1, cy), gz = (int)bq_axis(g, 2, cz);
  uint32_t *const hits = s_hits[wave];
  uint32_t *const runs = s_runs[wave];
  // the 27 cells' ranges, read at once: lane l < 27 takes cell offset
  // (l % 3 - 1, l / 3 % 3 - 1, l / 9 - 1)
  uint32_t cb = 0, ce = 0;
  if (lane < 27) {
    const int x = gx + (int)(lane % 3) - 1, y = gy + (int)(lane / 3 % 3) - 1,
              z = gz + (int)(lane / 9) - 1;
    if (x >= 0 && x < (int)g.dim[0] && y >= 0 && y < (int)g.dim[1] && z >= 0 &&
        z < (int)g.dim[2]) {
      const uint32_t cell = ((uint32_t)z * g.dim[1] + (uint32_t)y) * g.dim[0] + (uint32_t)x;
      cb = cstart[cell];
      ce = cend[cell];
    }
  }
  uint64_t cells = __ballot(cb < ce);
  uint32_t cnt = 0, nruns = 0;
  // one cell's candidates, already read: its hits, in index order, form a run
  const auto scan_cell = [&](const float4 &q, bool in) {
    if (lane == 0) runs[nruns] = cnt;
    ++nruns;
    const bool hit = in && sqdist(q.x, q.y, q.z, cx, cy, cz) < r2;
    const uint64_t mask = __ballot(hit);
    const uint32_t pos = cnt + lanes_below(mask);
    if (hit && pos < kBqCap) hits[pos] = __float_as_uint(q.w);
    cnt += (uint32_t)__popcll(mask);
  };
  if (__ballot(ce - cb > 64u) == 0) {
    // every cell fits one step: two cells a step, both reads in flight
    while (cells) {
      const uint32_t l1 = (uint32_t)__builtin_ctzll(cells);
      cells &= cells - 1;
      const bool two = cells != 0;
      const uint32_t l2 = two ? (uint32_t)__builtin_ctzll(cells) : l1;
      if (two) cells &= cells - 1;
      const uint32_t b1 = rdlane(cb, l1), e1 = rdlane(ce, l1), b2 = rdlane(cb, l2),
                     e2 = two ? rdlane(ce, l2) : b2;
      const uint32_t i1 = b1 + lane, i2 = b2 + lane;
      float4 q1 = make_float4(0.f, 0.f, 0.f, 0.f), q2 = q1;
      if (i1 < e1) q1 = spts[i1];
      if (i2 < e2) q2 = spts[i2];
      scan_cell(q1, i1 < e1);
      if (two) scan_cell(q2, i2 < e2);
    }
  }
  while (cells) {  // some cell holds more than 64 points: one cell at a time
    const uint32_t l = (uint32_t)__builtin_ctzll(cells);
    cells &= cells - 1;
    const uint32_t b = rdlane(cb, l), e = rdlane(ce, l);
    if (lane == 0) runs[nruns] = cnt;  // this cell's hits start a run
    ++nruns;
    for (uint32_t s = b; s < e; s += 64) {
      const uint32_t i = s + lane;
      bool hit = false;
      uint32_t idx = 0;
      if (i < e) {
        const float4 q = spts[i];
        hit = sqdist(q.x, q.y, q.z, cx, cy, cz) < r2;
        idx = __float_as_uint(q.w);
      }
      const uint64_t mask = __ballot(hit);
      const uint32_t pos = cnt + lanes_below(mask);
      if (hit && pos < kBqCap) hits[pos] = idx;
      cnt += (uint32_t)__popcll(mask);
    }
  }
  int32_t *const row = out + (size_t)j * nsample;
  if (cnt > kBqCap) {  // too many hits to hold: the ordered scan takes this center
    if (lane == 0) ovf_ids[atomicAdd(ovf_count, 1u)] = j;
    return;
  }
  if (lane == 0) runs[nruns] = cnt;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // 27-way merge: lane r < nruns holds the head of run r
  uint32_t head = 0, end = 0, val = 0xffffffffu;
  if (lane < nruns) {
    head = runs[lane];
    end = runs[lane + 1];
    val = head < end ? hits[head] : 0xffffffffu;
  }
  const uint32_t take = cnt < nsample ? cnt : nsample;
  uint32_t firstv = 0;
  for (uint32_t r = 0; r < take; ++r) {
    const uint32_t wmin = wave_min_u32(val);
    if (r == 0) firstv = wmin;
    if (lane == 0) row[r] = (int32_t)wmin;
    if (val == wmin) {  // one lane: indices are distinct
      ++head;
      val = head < end ? hits[head] : 0xffffffffu;
    }
  }
  const int32_t pad = cnt ? (int32_t)firstv : 0;
  for (uint32_t k = take + lane; k < nsample; k += 64) row[k] = pad;
}

}  // namespace

hipError_t preload_group_kernels() {
  return func_attributes(k_gather_points, k_ball_query, k_bq_bounds, k_bq_grid, k_bq_keys,
                         k_bq_cells, k_bq_query);
}

hipError_t launch_gather_points(const float *xyz, uint32_t n, const int32_t *idx, uint32_t m,
                                float *out, uint32_t *bad, hipStream_t st) {
  if (m == 0) return hipSuccess;
  k_gather_points<<<(m + 255) / 256, 256, 0, st>>>(xyz, n, idx, m, out, bad);
  return hipGetLastError();
}

hipError_t launch_ball_query(const float *xyz, uint32_t n, const float *centers,
                             const uint32_t *ids, uint32_t m, float r2, uint32_t nsample,
                             int32_t *out, hipStream_t st) {
  if (m == 0) return hipSuccess;
  k_ball_query<<<(m + kGroupWaves - 1) / kGroupWaves, 64 * kGroupWaves, 0, st>>>(
      xyz, n, centers, ids, m, r2, nsample, out);
  return hipGetLastError();
}

hipError_t launch_bq_grid_build(const float *xyz, uint32_t n, float radius, uint32_t *bnd,
                                BqGrid *grid, uint32_t *keys, hipStream_t st) {
  const uint32_t nb = std::min<uint32_t>((n + 255) / 256, 512);
  k_bq_bounds<<<nb, 256, 0, st>>>(xyz, n, bnd);  // 256 threads: four waves (s_b)
  k_bq_grid<<<1, 64, 0, st>>>(bnd, radius, grid);
  k_bq_keys<<<(n + 255) / 256, 256, 0, st>>>(xyz, n, grid, keys);
  return hipGetLastError();
}

hipError_t launch_bq_cells(const uint32_t *skeys, const uint32_t *sidx, uint32_t n,
                           const float *xyz, const BqGrid *grid, uint32_t *cstart, uint32_t *cend,
                           float4 *spts, hipStream_t st) {
  k_bq_cells<<<(n + 255) / 256, 256, 0, st>>>(skeys, sidx, n, xyz, grid, cstart, cend, spts);
  return hipGetLastError();
}

hipError_t launch_bq_query(const float4 *spts, const BqGrid *grid, const uint32_t *cstart,
                           const uint32_t *cend, const float *centers, uint32_t m, float r2,
                           uint32_t nsample, int32_t *out, uint32_t *ovf_ids,
                           uint32_t *ovf_count, hipStream_t st) {
  if (m == 0) return hipSuccess;
  k_bq_query<<<(m + kGroupWaves - 1) / kGroupWaves, 64 * kGroupWaves, 0, st>>>(
      spts, grid, cstart, cend, centers, m, r2, nsample, out, ovf_ids, ovf_count);
  return hipGetLastError();
}

}  // namespace nsfps
