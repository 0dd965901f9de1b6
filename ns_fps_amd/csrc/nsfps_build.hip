// Structure build on the device (gfx950): per-point bucket key with the
// reference's cell rule, two stable LSD radix sorts, SoA gather into physical
// slots, cell table, leaves with bounding boxes, level-1 tree nodes.
//
// Logical order (the reference's layout, src/yuezu_fps.cpp:277-283, 411-416,
// 431-438) = stable sort of the input rows by bucket; the logical rank of a
// point is its position in that order and breaks ties in the argmax.  The
// physical order additionally sorts each bucket by a sub-cell Morton code so
// that 64-point leaves are spatially tight; it never changes the result.
#include <hip/hip_runtime.h>

#include "nsfps_device.h"
#include "nsfps_launch.h"

namespace nsfps {

// Bucket and sub-cell code per input row; bucket populations; non-finite flag.
__device__ __forceinline__ uint32_t cell_keys_at(uint32_t i, const float *__restrict__ xyz, uint32_t n,
                                             const RangeDev &r, const uint32_t *__restrict__ lut,
                                             uint32_t *__restrict__ bucket,
                                             uint32_t *__restrict__ fine,
                                             uint32_t *__restrict__ counts,
                                             uint32_t *__restrict__ bad) {
  if (i >= n) return ~0u;
  float v[3] = {xyz[3 * (size_t)i], xyz[3 * (size_t)i + 1], xyz[3 * (size_t)i + 2]};
  uint32_t c[3], f = 0;
  bool finite = true;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    finite = finite && isfinite(v[a]);
    c[a] = cell_axis(r, a, v[a]);
    float cl = std_max(r.mn[a], std_min(v[a], r.hiclamp[a]));
    float t = (cl - r.mn[a]) * r.inv_bs[a] - (float)c[a];
    int s = (int)(t * 8.0f);
    s = s < 0 ? 0 : (s > 7 ? 7 : s);
#pragma unroll
    for (int k = 0; k < 3; ++k) f |= (uint32_t)((s >> k) & 1) << (3 * k + a);
  }
  if (!finite) atomicOr(bad, 1u);
  uint32_t b = bucket_of(r, lut, c[0], c[1], c[2]);
  bucket[i] = b;
  fine[i] = f;
  if (counts) atomicAdd(&counts[b], 1u);  // null: counted elsewhere
  return b;
}

// The same from a range in device memory (computed on the device from the
// points' bounds, before the host knows it).
__global__ void k_cell_keys_dr(const float *__restrict__ xyz, uint32_t n,
                               const RangeDev *__restrict__ rp, const uint32_t *__restrict__ lut,
                               uint32_t *__restrict__ bucket, uint32_t *__restrict__ fine,
                               uint32_t *__restrict__ counts, uint32_t *__restrict__ bad) {
  const RangeDev r = *rp;
  cell_keys_at(blockIdx.x * blockDim.x + threadIdx.x, xyz, n, r, lut, bucket, fine, counts, bad);
}

// --- compute_bbox on the device (src/yuezu_fps.cpp:643-670) ---------------
//
// The reference keeps a running (v < mn ? v : mn) and (mx < v ? v : mx) from
// point 0 and uses only min - BOUNDARY_EPS and max + BOUNDARY_EPS.  Minimum
// and maximum of finite values do not depend on the order (a zero's sign is
// the only order-dependent bit, and +-0 - 1e-6 and +-0 + 1e-6 do not keep
// it), so per-cloud atomics on order-preserving integers give the same
// bounds.  Non-finite points are skipped here; the cell-key pass flags them
// and the call is refused.

// ord_lo[3 b + a] / ord_hi[3 b + a]: ord_of(min) / ord_of(max) of axis a of
// cloud b over its finite points (ord_lo starts at 0xffffffff, ord_hi at 0).
// Grid (workgroups per cloud, clouds); the clouds lie one after another.
__global__ __launch_bounds__(256) void k_cloud_bounds(const float *__restrict__ xyz,
                                                      uint32_t n_per,
                                                      uint32_t *__restrict__ ord_lo,
                                                      uint32_t *__restrict__ ord_hi) {
  const uint32_t b = blockIdx.y;
  const float *const c = xyz + (size_t)b * n_per * 3;
  uint32_t lo[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, hi[3] = {0u, 0u, 0u};
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n_per; i += gridDim.x * blockDim.x) {
    const float v[3] = {c[3 * (size_t)i], c[3 * (size_t)i + 1], c[3 * (size_t)i + 2]};
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      if (!isfinite(v[a])) continue;
      const uint32_t o = ord_of(v[a]);
      lo[a] = lo[a] < o ? lo[a] : o;
      hi[a] = hi[a] > o ? hi[a] : o;
    }
  }
  // one atomic per value and workgroup (contended atomics on one address
  // serialise)
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
    if (a < 3) atomicMin(&ord_lo[3 * b + a], v);
    else atomicMax(&ord_hi[3 * b + a - 3], v);
  }
}

// The range of cloud blockIdx.x from its bounds: min - 1e-6 and max + 1e-6
// per axis (an axis without a finite point gets 0 +- 1e-6), then make_range's
// derivation (src/yuezu_fps.cpp:136-161) in the host's fp32 operations:
// block size (max - min) / blocks, inv_bs = 1 / block size, the clamp bound
// max - 1e-6, and the cube thresholds.  tmpl holds the fields that depend on
// the block counts alone.  out[b] gets the range, bounds[6 b ..] its min x,
// max x, min y, max y, min z, max z; with bd, bd[b].c.r gets it too.  One
// wave per cloud: lane 3 k + a searches threshold k of axis a.
__global__ __launch_bounds__(64) void k_range_of_bounds(const uint32_t *__restrict__ ord_lo,
                                                        const uint32_t *__restrict__ ord_hi,
                                                        RangeDev tmpl, RangeDev *__restrict__ out,
                                                        float *__restrict__ bounds,
                                                        BuildDev *__restrict__ bd) {
  const uint32_t b = blockIdx.x, lane = threadIdx.x;
  constexpr float kEps = 1e-6f;  // BOUNDARY_EPS, src/yuezu_fps.h:43-45
  float mn[3], mx[3], bs[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const uint32_t lo = ord_lo[3 * b + a], hi = ord_hi[3 * b + a];
    const bool any = lo <= hi;
    mn[a] = (any ? float_of(lo) : 0.f) - kEps;
    mx[a] = (any ? float_of(hi) : 0.f) + kEps;
    bs[a] = (mx[a] - mn[a]) / (float)tmpl.blocks[a];
  }
  __shared__ float s_thr[3][kCubeThr];
  if (lane < 3 * kCubeThr) {
    const uint32_t a = lane % 3, k = lane / 3;
    s_thr[a][k] = cube_threshold_dev(bs[a], tmpl.blocks[a], k + 1);
  }
  __syncthreads();
  if (lane != 0) return;
  RangeDev r = tmpl;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    r.mn[a] = mn[a];
    r.hiclamp[a] = mx[a] - kEps;
    r.bsize[a] = bs[a];
    r.inv_bs[a] = 1.0f / bs[a];
#pragma unroll
    for (uint32_t k = 0; k < kCubeThr; ++k) r.cube_thr[a][k] = s_thr[a][k];
    bounds[6 * b + 2 * a] = mn[a];
    bounds[6 * b + 2 * a + 1] = mx[a];
  }
  out[b] = r;
  if (bd) bd[b].c.r = r;
}

// Bucket populations from the buckets sorted: each bucket's points are one
// run; the run's first element adds -(its position) and its last element
// adds its position + 1, so every bucket takes at most two atomics, never
// contended (counts start at zero).
__global__ void k_seg_counts(const uint32_t *__restrict__ keys, uint32_t n,
                             uint32_t *__restrict__ counts) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t k = keys[i];
  uint32_t delta = 0;
  if (i == 0 || keys[i - 1] != k) delta -= i;
  if (i + 1 == n || keys[i + 1] != k) delta += i + 1;
  if (delta) atomicAdd(&counts[k], delta);
}

__global__ void k_cell_keys(const float *__restrict__ xyz, uint32_t n, RangeDev r,
                            const uint32_t *__restrict__ lut, uint32_t *__restrict__ bucket,
                            uint32_t *__restrict__ fine, uint32_t *__restrict__ counts,
                            uint32_t *__restrict__ bad) {
  cell_keys_at(blockIdx.x * blockDim.x + threadIdx.x, xyz, n, r, lut, bucket, fine, counts, bad);
}

// --- stable LSD radix sort (8-bit digits), u32 keys and values -------------
constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;                        // per wave: 16 x 64 keys
constexpr int kSortTile = kSortThreads * kSortRounds;  // 4096 keys per block

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
__device__ __forceinline__ void scan_excl_block(uint32_t *__restrict__ data, uint32_t len,
                                                uint32_t *wsum) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t per = (len + 1023) / 1024;
  uint32_t b = tid * per, e = b + per < len ? b + per : len;
  uint32_t s = 0;
  for (uint32_t i = b; i < e; ++i) s += data[i];
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

__global__ __launch_bounds__(1024) void k_scan_excl(uint32_t *__restrict__ data, uint32_t len) {
  __shared__ uint32_t wsum[16];
  scan_excl_block(data, len, wsum);
}

// Longer scans: chunks of kScanChunk values, four consecutive per thread.
// Pass 1 sums every chunk, k_scan_excl scans the sums, pass 2 rescans every
// chunk from its offset.
constexpr uint32_t kScanChunk = 4096;
constexpr uint32_t kScanSingleMax = 16384;  // one workgroup up to here

__device__ __forceinline__ uint4 scan_load4(const uint32_t *data, uint32_t len, uint32_t i) {
  return make_uint4(i < len ? data[i] : 0u, i + 1 < len ? data[i + 1] : 0u,
                    i + 2 < len ? data[i + 2] : 0u, i + 3 < len ? data[i + 3] : 0u);
}

__global__ __launch_bounds__(1024) void k_scan_sums(const uint32_t *__restrict__ data, uint32_t len,
                                                    uint32_t *__restrict__ sums) {
  __shared__ uint32_t wsum[16];
  const uint4 v = scan_load4(data, len, blockIdx.x * kScanChunk + threadIdx.x * 4);
  uint32_t tot;
  block_excl_scan<16>(v.x + v.y + v.z + v.w, wsum, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

__global__ __launch_bounds__(1024) void k_scan_apply(uint32_t *__restrict__ data, uint32_t len,
                                                     const uint32_t *__restrict__ sums) {
  __shared__ uint32_t wsum[16];
  const uint32_t i = blockIdx.x * kScanChunk + threadIdx.x * 4;
  const uint4 v = scan_load4(data, len, i);
  uint32_t tot;
  uint32_t run = sums[blockIdx.x] + block_excl_scan<16>(v.x + v.y + v.z + v.w, wsum, &tot);
  if (i < len) data[i] = run;
  run += v.x;
  if (i + 1 < len) data[i + 1] = run;
  run += v.y;
  if (i + 2 < len) data[i + 2] = run;
  run += v.z;
  if (i + 3 < len) data[i + 3] = run;
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) data[len] = sums[gridDim.x];
}

// Stable scatter of one digit pass.  Each wave ranks its 1024 keys in order
// (16 rounds of 64): lanes with the same digit are found with 8 ballots, the
// running per-digit count of the wave lives in LDS; waves are then offset by
// an exclusive prefix over waves.
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
    // all lanes read their base before a leader writes (in-order LDS, one wave)
    __builtin_amdgcn_s_waitcnt(0xc07f);
    if (valid && before == 0) wcnt[wave][d] = baseq + (uint32_t)__popcll(peers);
    __builtin_amdgcn_s_waitcnt(0xc07f);
  }
  __syncthreads();
  {
    uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) {
      uint32_t c = wcnt[w][tid];
      wcnt[w][tid] = s;
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

// The logical sort of clouds of at most kSegSortMax points, one 1024-thread
// workgroup per cloud: cloud s is bucket[s * n_per .., + n_per), sorted by
// bucket with rows in input order inside a bucket.  keys_out[s * n_per + p]
// gets (s << key_shift) | bucket and vals_out the row s * n_per + r: what
// the radix sort over (cloud, bucket) keys writes.  An element is packed as
// (bucket << 14) | r, 16 of them per lane in registers (lane l of wave w
// holds r = 1024 w + 64 i + l); each pass of 8 bucket bits ranks them with
// the ballots of k_radix_scatter (a wave's elements in order, the wave's
// running count per digit in LDS), offsets digit by digit and then wave by
// wave, and scatters into LDS, or into keys_out / vals_out after the last
// pass.  Three global passes over the 64 clouds of 16,384 points took 96 us.
constexpr uint32_t kSegSortMax = kSegSortMaxPoints;
constexpr int kSegWaves = 16, kSegRounds = 16;  // 16 waves x 16 rounds x 64 lanes
static_assert(kSegWaves * kSegRounds * 64 == (int)kSegSortMax, "one element per lane and round");

__global__ __launch_bounds__(1024) void k_seg_sort(const uint32_t *__restrict__ bucket,
                                                   uint32_t n_per, int bits, int key_shift,
                                                   uint32_t *__restrict__ keys_out,
                                                   uint32_t *__restrict__ vals_out) {
  __shared__ uint32_t s_el[kSegSortMax];
  __shared__ uint32_t wcnt[kSegWaves][256];
  __shared__ uint32_t wsum[kSegWaves];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const size_t base = (size_t)blockIdx.x * n_per;
  const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
  uint32_t el[kSegRounds];
#pragma unroll
  for (int r = 0; r < kSegRounds; ++r) {
    const uint32_t e = wave * (64u * kSegRounds) + 64u * r + lane;
    el[r] = e < n_per ? (bucket[base + e] << 14) | e : 0u;
  }
  for (int shift = 0; shift < bits; shift += 8) {
    for (uint32_t i = tid; i < kSegWaves * 256u; i += 1024u) (&wcnt[0][0])[i] = 0u;
    __syncthreads();
    uint32_t rnk[kSegRounds];
#pragma unroll
    for (int r = 0; r < kSegRounds; ++r) {
      const bool valid = wave * (64u * kSegRounds) + 64u * r + lane < n_per;
      const uint32_t d = (el[r] >> (14 + shift)) & 255u;
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t m = __ballot((d >> b) & 1u);
        peers &= ((d >> b) & 1u) ? m : ~m;
      }
      const uint32_t before = (uint32_t)__popcll(peers & lt);
      const uint32_t baseq = valid ? wcnt[wave][d] : 0u;
      rnk[r] = baseq + before;
      // all lanes read their base before a leader writes (in-order LDS, one wave)
      __builtin_amdgcn_s_waitcnt(0xc07f);
      if (valid && before == 0) wcnt[wave][d] = baseq + (uint32_t)__popcll(peers);
      __builtin_amdgcn_s_waitcnt(0xc07f);
    }
    __syncthreads();
    // digit d's first position, then each wave's within the digit
    uint32_t tot = 0;
    if (tid < 256u)
      for (int w = 0; w < kSegWaves; ++w) tot += wcnt[w][tid];
    uint32_t all;
    const uint32_t first = block_excl_scan<kSegWaves>(tot, wsum, &all);
    if (tid < 256u) {
      uint32_t at = first;
      for (int w = 0; w < kSegWaves; ++w) {
        const uint32_t c = wcnt[w][tid];
        wcnt[w][tid] = at;
        at += c;
      }
    }
    __syncthreads();
    const bool last = shift + 8 >= bits;
#pragma unroll
    for (int r = 0; r < kSegRounds; ++r) {
      if (wave * (64u * kSegRounds) + 64u * r + lane >= n_per) continue;
      const uint32_t pos = wcnt[wave][(el[r] >> (14 + shift)) & 255u] + rnk[r];
      if (last) {
        keys_out[base + pos] = ((uint32_t)blockIdx.x << key_shift) | (el[r] >> 14);
        vals_out[base + pos] = (uint32_t)base + (el[r] & 0x3fffu);
      } else {
        s_el[pos] = el[r];
      }
    }
    if (last) break;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kSegRounds; ++r) {
      const uint32_t e = wave * (64u * kSegRounds) + 64u * r + lane;
      el[r] = e < n_per ? s_el[e] : 0u;
    }
  }
}

// Sort key of the clouds of a call sorted together: cloud index above the
// bucket (every cloud has n_per points, stored one cloud after another).
__global__ void k_cloud_keys(const uint32_t *__restrict__ bucket, uint32_t total, uint32_t n_per,
                             int bucket_bits, uint32_t *__restrict__ key) {
  uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total) return;
  key[g] = bucket[g] | ((g / n_per) << bucket_bits);
}

// Secondary key per logical position: cloud (when clouds are sorted
// together, position p belongs to cloud p / n_per), bucket, then the sub-cell
// code.
__global__ void k_key2(const uint32_t *__restrict__ lorig, const uint32_t *__restrict__ bucket,
                       const uint32_t *__restrict__ fine, uint32_t n, uint32_t n_per,
                       int cloud_shift, int fine_shift, int fine_bits,
                       uint32_t *__restrict__ key2) {
  uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  uint32_t o = lorig[p];
  uint32_t f = fine_bits > 0 ? (fine[o] >> fine_shift) : 0u;
  key2[p] = ((p / n_per) << cloud_shift) | (bucket[o] << fine_bits) | f;
}

// Leaves per bucket, the largest bucket population and the total of leaves.
__device__ __forceinline__ void leaf_counts_block(uint32_t blk, const uint32_t *__restrict__ counts,
                                                  uint32_t T, uint32_t *__restrict__ lc,
                                                  uint32_t *__restrict__ maxocc,
                                                  uint32_t *__restrict__ total,
                                                  uint32_t *__restrict__ occupied, uint32_t *s_red) {
  // s_red[0]: leaves of the block, s_red[1]: its largest bucket, s_red[2]:
  // its buckets holding points (one global atomic each per block)
  if (threadIdx.x < 3) s_red[threadIdx.x] = 0;
  __syncthreads();
  uint32_t b = blk * blockDim.x + threadIdx.x;
  if (b < T) {
    uint32_t c = counts[b];
    lc[b] = (c + kLeaf - 1) / kLeaf;
    if (c) {
      atomicMax(&s_red[1], c);
      atomicAdd(&s_red[0], (c + kLeaf - 1) / kLeaf);
      atomicAdd(&s_red[2], 1u);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0 && s_red[0]) atomicAdd(total, s_red[0]);
  if (threadIdx.x == 1 && s_red[1]) atomicMax(maxocc, s_red[1]);
  if (threadIdx.x == 2 && s_red[2]) atomicAdd(occupied, s_red[2]);
}

__global__ __launch_bounds__(256) void k_leaf_counts(const uint32_t *__restrict__ counts,
                                                     uint32_t T, uint32_t *__restrict__ lc,
                                                     uint32_t *__restrict__ maxocc,
                                                     uint32_t *__restrict__ total,
                                                     uint32_t *__restrict__ occupied) {
  __shared__ uint32_t s_red[3];
  leaf_counts_block(blockIdx.x, counts, T, lc, maxocc, total, occupied, s_red);
}

__device__ __forceinline__ void cell_info_at(uint32_t b, const uint32_t *__restrict__ cell_start,
                                             const uint32_t *__restrict__ cell_leaf, uint32_t T,
                                             uint2 *__restrict__ info) {
  if (b > T) return;
  info[b] = make_uint2(cell_start[b], cell_leaf[b]);
}

// Gather into physical slots; min-distance starts at FLT_MAX
// (src/yuezu_fps.cpp:215-223).  Dense: slot = physical position p.  Padded:
// slot = bucket * cap + (p - first position of the bucket).
__device__ __forceinline__ void gather_at(uint32_t p, const uint32_t *__restrict__ prank,
                                          const uint32_t *__restrict__ lorig, uint32_t base,
                                          const uint32_t *__restrict__ bucket,
                                          const uint32_t *__restrict__ cell_start,
                                          const float *__restrict__ xyz, uint32_t n,
                                          uint32_t padded, uint32_t cap, float4 *__restrict__ P4,
                                          uint2 *__restrict__ RO, uint32_t *__restrict__ R,
                                          uint32_t *__restrict__ phys0) {
  if (p >= n) return;
  // ranks and rows come from sorts that may hold other clouds: this cloud's
  // start in them is base; no prank: the physical order is the logical one
  uint32_t rkg = prank ? prank[p] : base + p;
  uint32_t rk = rkg - base;
  uint32_t o = lorig[rkg] - base;
  uint32_t slot = p;
  if (padded) {
    uint32_t b = bucket[o];
    slot = b * cap + (p - cell_start[b]);
  }
  P4[slot] = make_float4(xyz[3 * (size_t)o], xyz[3 * (size_t)o + 1], xyz[3 * (size_t)o + 2],
                         FLT_MAX);
  RO[slot] = make_uint2(rk, o);
  R[slot] = rk;
  if (o == 0) *phys0 = slot;
}

__global__ void k_gather(const uint32_t *__restrict__ prank, const uint32_t *__restrict__ lorig,
                         uint32_t base, const uint32_t *__restrict__ bucket,
                         const uint32_t *__restrict__ cell_start,
                         const float *__restrict__ xyz, uint32_t n, uint32_t padded, uint32_t cap,
                         float4 *__restrict__ P4, uint2 *__restrict__ RO,
                         uint32_t *__restrict__ R, uint32_t *__restrict__ phys0) {
  gather_at(blockIdx.x * blockDim.x + threadIdx.x, prank, lorig, base, bucket, cell_start, xyz, n,
            padded, cap, P4, RO, R, phys0);
}

// Leaf descriptors (first slot, point count, cell) of every leaf of bucket b,
// and the cells of the bucket (r.na per leaf).
__device__ __forceinline__ void leaf_desc_at(uint32_t b, const uint32_t *__restrict__ cell_start,
                                             const uint32_t *__restrict__ cell_leaf, uint32_t T,
                                             uint32_t padded, uint32_t cap, uint32_t lpc,
                                             const RangeDev &r, const float4 *__restrict__ P4,
                                             float4 *__restrict__ leaf_lo,
                                             float4 *__restrict__ leaf_hi,
                                             uint32_t *__restrict__ leaf_cell,
                                             uint32_t *__restrict__ leaf_al,
                                             uint2 *__restrict__ leaf_sc) {
  if (b >= T) return;
  uint32_t s = cell_start[b], e = cell_start[b + 1];
  uint32_t cntb = e - s;
  uint32_t first = padded ? b * cap : s;
  uint32_t l = padded ? b * lpc : cell_leaf[b];
  uint32_t nl = padded ? lpc : (cntb + kLeaf - 1) / kLeaf;
  uint32_t packed = 0;
  if (cntb) {
    float4 p = P4[first];
    packed = cell_axis(r, 0, p.x) | (cell_axis(r, 1, p.y) << 10) | (cell_axis(r, 2, p.z) << 20);
  }
  uint32_t al[kMaxAlias];
  if (nl) bucket_cells(r, b, al);
  for (uint32_t k = 0; k < nl; ++k, ++l) {
    uint32_t off = k * kLeaf;
    uint32_t cnt = cntb > off ? (cntb - off < kLeaf ? cntb - off : kLeaf) : 0u;
    leaf_lo[l] = make_float4(0.f, 0.f, 0.f, __uint_as_float(first + off));
    leaf_hi[l] = make_float4(0.f, 0.f, 0.f, __uint_as_float(cnt));
    leaf_sc[l] = make_uint2(first + off, cnt);
    leaf_cell[l] = packed;
    for (uint32_t a = 0; a < r.na; ++a) leaf_al[(size_t)l * r.na + a] = al[a];
  }
}

// Mixed leaves (runs engine, one cell per bucket): leaf l holds the slots
// 64 l .. 64 l + 63 of the logical order, whichever buckets they belong to.
__device__ __forceinline__ void leaf_desc_mixed_at(uint32_t l, uint32_t n, uint32_t nleaves,
                                                   float4 *__restrict__ leaf_lo,
                                                   float4 *__restrict__ leaf_hi,
                                                   uint32_t *__restrict__ leaf_cell,
                                                   uint32_t *__restrict__ leaf_al,
                                                   uint2 *__restrict__ leaf_sc) {
  if (l >= nleaves) return;
  const uint32_t first = l * kLeaf;
  const uint32_t cnt = n - first < kLeaf ? n - first : kLeaf;
  leaf_lo[l] = make_float4(0.f, 0.f, 0.f, __uint_as_float(first));
  leaf_hi[l] = make_float4(0.f, 0.f, 0.f, __uint_as_float(cnt));
  leaf_sc[l] = make_uint2(first, cnt);
  leaf_cell[l] = 0;      // a leaf of several cells: its cell box is leaf_cbox
  leaf_al[l] = kNoCell;  // one cell per bucket (r.na == 1)
}

// One cloud's cell table and leaf descriptors in one launch: thread i
// writes cell i's table entry and the leaves of bucket i (with mixed leaves,
// leaf i).  Two launches before; the small clouds' build waits on each
// launch's host time.
__global__ void k_cells(const uint32_t *__restrict__ cell_start,
                        const uint32_t *__restrict__ cell_leaf, uint32_t T, uint32_t padded,
                        uint32_t cap, uint32_t lpc, uint32_t mixed, uint32_t n, uint32_t nleaves,
                        RangeDev r, const float4 *__restrict__ P4, uint2 *__restrict__ info,
                        float4 *__restrict__ leaf_lo, float4 *__restrict__ leaf_hi,
                        uint32_t *__restrict__ leaf_cell, uint32_t *__restrict__ leaf_al,
                        uint2 *__restrict__ leaf_sc) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  cell_info_at(i, cell_start, cell_leaf, T, info);
  if (mixed)
    leaf_desc_mixed_at(i, n, nleaves, leaf_lo, leaf_hi, leaf_cell, leaf_al, leaf_sc);
  else
    leaf_desc_at(i, cell_start, cell_leaf, T, padded, cap, lpc, r, P4, leaf_lo, leaf_hi, leaf_cell,
                 leaf_al, leaf_sc);
}

// Leaf bounding boxes, the corners of their points' cells, and initial keys
// (FLT_MAX with the smallest rank of the leaf); empty leaves get an empty box
// (its cell corners lo > hi) and key 0.  One wave per leaf.  cell_axis is
// monotone, so the cells of the box's corners bound every point's cell.
__device__ __forceinline__ void leaf_bbox_at(uint32_t leaf, uint32_t nleaves, const RangeDev &r,
                                             const float4 *__restrict__ P4,
                                             const uint2 *__restrict__ RO,
                                             float4 *__restrict__ leaf_lo,
                                             float4 *__restrict__ leaf_hi,
                                             uint2 *__restrict__ leaf_cbox,
                                             uint64_t *__restrict__ leaf_key,
                                             float4 *__restrict__ leaf_pos) {
  uint32_t lane = lane_id();
  if (leaf >= nleaves) return;
  float4 lo = leaf_lo[leaf], hi = leaf_hi[leaf];
  uint32_t start = __float_as_uint(lo.w), cnt = __float_as_uint(hi.w);
  bool act = lane < cnt;
  float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
  uint2 ro = make_uint2(0u, 0u);
  if (act) {
    p = P4[start + lane];
    ro = RO[start + lane];
  }
  float mnx = act ? p.x : INFINITY, mny = act ? p.y : INFINITY, mnz = act ? p.z : INFINITY;
  float mxx = act ? p.x : -INFINITY, mxy = act ? p.y : -INFINITY, mxz = act ? p.z : -INFINITY;
  uint64_t k = act ? make_key(FLT_MAX, ro.x) : 0ull;
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
  uint32_t wl = argmax_lane(k, km, act);
  if (lane == 0) {
    leaf_lo[leaf] = make_float4(mnx, mny, mnz, lo.w);
    leaf_hi[leaf] = make_float4(mxx, mxy, mxz, hi.w);
    leaf_cbox[leaf] =
        make_uint2(cell_axis(r, 0, mnx) | (cell_axis(r, 1, mny) << 10) | (cell_axis(r, 2, mnz) << 20),
                   cell_axis(r, 0, mxx) | (cell_axis(r, 1, mxy) << 10) | (cell_axis(r, 2, mxz) << 20));
    leaf_key[leaf] = km;
  }
  if (cnt == 0) {
    if (lane == 0) leaf_pos[leaf] = make_float4(0.f, 0.f, 0.f, 0.f);
  } else if (lane == wl) {
    leaf_pos[leaf] = make_float4(p.x, p.y, p.z, __uint_as_float(ro.y));
  }
}

__global__ __launch_bounds__(256) void k_leaf_bbox(uint32_t nleaves, RangeDev r,
                                                   const float4 *__restrict__ P4,
                                                   const uint2 *__restrict__ RO,
                                                   float4 *__restrict__ leaf_lo,
                                                   float4 *__restrict__ leaf_hi,
                                                   uint2 *__restrict__ leaf_cbox,
                                                   uint64_t *__restrict__ leaf_key,
                                                   float4 *__restrict__ leaf_pos) {
  leaf_bbox_at(blockIdx.x * 4 + (threadIdx.x >> 6), nleaves, r, P4, RO, leaf_lo, leaf_hi, leaf_cbox,
               leaf_key, leaf_pos);
}

// Level-1 nodes from the initial leaves: max key, its position, the union
// of the leaf boxes, and the corners of the cells of the leaves' buckets
// (leaves with points only; x = kNone when there are none).  One wave per
// node.
__device__ __forceinline__ void l1_init_at(uint32_t g, uint32_t nleaves, uint32_t nl1,
                                           const uint64_t *__restrict__ leaf_key,
                                           const float4 *__restrict__ leaf_pos,
                                           const float4 *__restrict__ leaf_lo,
                                           const float4 *__restrict__ leaf_hi,
                                           const uint32_t *__restrict__ leaf_al, uint32_t na,
                                           uint64_t *__restrict__ l1_key,
                                           float4 *__restrict__ l1_pos,
                                           float4 *__restrict__ l1_lo,
                                           float4 *__restrict__ l1_hi,
                                           uint2 *__restrict__ l1_cbox) {
  uint32_t lane = lane_id();
  if (g >= nl1) return;
  uint32_t j = g * kFan + lane;
  bool v = j < nleaves;
  uint32_t cmin[3] = {kNone, kNone, kNone}, cmax[3] = {0u, 0u, 0u};
  if (v && __float_as_uint(leaf_hi[j].w) != 0u) {
    for (uint32_t a = 0; a < na; ++a) {
      const uint32_t cl = leaf_al[(size_t)j * na + a];
      if (cl == kNoCell) continue;
      const uint32_t cx[3] = {cl & 1023u, (cl >> 10) & 1023u, cl >> 20};
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        cmin[d] = cx[d] < cmin[d] ? cx[d] : cmin[d];
        cmax[d] = cx[d] > cmax[d] ? cx[d] : cmax[d];
      }
    }
  }
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    cmin[d] = wave_min_u32(cmin[d]);
    cmax[d] = wave_max_u32(cmax[d]);
  }
  uint64_t k = v ? leaf_key[j] : 0ull;
  float4 lo = v ? leaf_lo[j] : make_float4(INFINITY, INFINITY, INFINITY, 0.f);
  float4 hi = v ? leaf_hi[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, 0.f);
  float mnx = lo.x, mny = lo.y, mnz = lo.z, mxx = hi.x, mxy = hi.y, mxz = hi.z;
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
  uint32_t wl = argmax_lane(k, km, v);
  if (lane == 0) {
    l1_key[g] = km;
    l1_pos[g] = leaf_pos[g * kFan + wl];
    l1_lo[g] = make_float4(mnx, mny, mnz, 0.f);
    l1_hi[g] = make_float4(mxx, mxy, mxz, 0.f);
    l1_cbox[g] = cmin[0] == kNone
                     ? make_uint2(kNone, 0u)
                     : make_uint2(cmin[0] | (cmin[1] << 10) | (cmin[2] << 20),
                                  cmax[0] | (cmax[1] << 10) | (cmax[2] << 20));
  }
}


__device__ __forceinline__ void init_state_of(const CloudDev &c, const uint32_t *phys0) {
  *c.iter = 0;
  *c.done = 0;
  *c.counter = 0;
  *c.root_key = 0;
  *c.root_pos = c.P4[*phys0];
}

__global__ void k_init_state(CloudDev c, const uint32_t *__restrict__ phys0) {
  if (threadIdx.x == 0 && blockIdx.x == 0) init_state_of(c, phys0);
}

// One cloud's level-1 nodes (a wave each), and its run state (block 0,
// thread 0: it reads none of the nodes).
__global__ __launch_bounds__(256) void k_l1_init_state(CloudDev c,
                                                       const uint32_t *__restrict__ phys0) {
  l1_init_at(blockIdx.x * 4 + (threadIdx.x >> 6), c.nleaves, c.nl1, c.leaf_key, c.leaf_pos,
             c.leaf_lo, c.leaf_hi, c.leaf_al, c.r.na, c.l1_key, c.l1_pos,
             const_cast<float4 *>(c.l1_lo), const_cast<float4 *>(c.l1_hi),
             const_cast<uint2 *>(c.l1_cbox));
  if (blockIdx.x == 0 && threadIdx.x == 0) init_state_of(c, phys0);
}

// Fills 32-bit words (clears flags, counters and tables with a kernel, not a
// memset node, so that the call path holds no hipMemsetAsync).
__global__ void k_fill_u32(uint32_t *__restrict__ p, uint32_t value, uint64_t words) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride)
    p[i] = value;
}

// ---------------------------------------------------------------- launchers


static inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

hipError_t launch_fill_u32(void *p, uint32_t value, uint64_t words, hipStream_t st) {
  if (words == 0) return hipSuccess;
  const uint64_t blocks = (words + 255) / 256;
  k_fill_u32<<<(uint32_t)(blocks < 4096 ? blocks : 4096), 256, 0, st>>>((uint32_t *)p, value, words);
  return hipGetLastError();
}

hipError_t launch_seg_counts(const uint32_t *keys, uint32_t n, uint32_t *counts, hipStream_t st) {
  if (n == 0) return hipSuccess;
  k_seg_counts<<<(n + 255) / 256, 256, 0, st>>>(keys, n, counts);
  return hipGetLastError();
}

hipError_t launch_cell_keys(const float *xyz, uint32_t n, const RangeDev &r, const uint32_t *lut,
                            uint32_t *bucket, uint32_t *fine, uint32_t *counts, uint32_t *bad,
                            hipStream_t st) {
  if (n == 0) return hipSuccess;
  k_cell_keys<<<cdiv(n, 256), 256, 0, st>>>(xyz, n, r, lut, bucket, fine, counts, bad);
  return hipGetLastError();
}

uint32_t scan_tmp_len(uint32_t len) { return cdiv(len, kScanChunk) + 1; }

hipError_t launch_cell_keys_dr(const float *xyz, uint32_t n, const RangeDev *d_range,
                               const uint32_t *lut, uint32_t *bucket, uint32_t *fine,
                               uint32_t *counts, uint32_t *bad, hipStream_t st) {
  if (n == 0) return hipSuccess;
  k_cell_keys_dr<<<cdiv(n, 256), 256, 0, st>>>(xyz, n, d_range, lut, bucket, fine, counts, bad);
  return hipGetLastError();
}

hipError_t launch_device_ranges(const float *xyz, uint32_t n_per, uint32_t nclouds,
                                const RangeDev &tmpl, uint32_t *ord, RangeDev *out,
                                float *bounds, BuildDev *bd, hipStream_t st) {
  if (nclouds == 0) return hipSuccess;
  const hipError_t e = launch_fill_u32(ord, 0xffffffffu, 3ull * nclouds, st);
  if (e != hipSuccess) return e;
  const hipError_t e2 = launch_fill_u32(ord + 3ull * nclouds, 0u, 3ull * nclouds, st);
  if (e2 != hipSuccess) return e2;
  // about 4 points per thread, at most 256 workgroups per cloud (64 points
  // per thread on one workgroup per 16,384-point cloud took 32 us for 64
  // clouds: a thread's loop is a chain of load latencies)
  const uint32_t per = n_per ? cdiv(n_per, 256 * 4) : 1;
  k_cloud_bounds<<<dim3(per < 256 ? per : 256, nclouds), 256, 0, st>>>(xyz, n_per, ord,
                                                                        ord + 3ull * nclouds);
  k_range_of_bounds<<<nclouds, 64, 0, st>>>(ord, ord + 3ull * nclouds, tmpl, out, bounds, bd);
  return hipGetLastError();
}

hipError_t launch_scan(uint32_t *data, uint32_t len, uint32_t *tmp, hipStream_t st) {
  if (len <= kScanSingleMax) {
    k_scan_excl<<<1, 1024, 0, st>>>(data, len);
  } else {
    const uint32_t nb = cdiv(len, kScanChunk);
    k_scan_sums<<<nb, 1024, 0, st>>>(data, len, tmp);
    k_scan_excl<<<1, 1024, 0, st>>>(tmp, nb);
    k_scan_apply<<<nb, 1024, 0, st>>>(data, len, tmp);
  }
  return hipGetLastError();
}

uint32_t radix_hist_len(uint32_t n) { return 256u * cdiv(n, kSortTile) + 1; }

hipError_t launch_radix_sort(uint32_t *keys, uint32_t *vals, uint32_t *keys_tmp,
                             uint32_t *vals_tmp, uint32_t n, int key_bits, uint32_t *hist,
                             uint32_t *scan_tmp, bool iota_values, uint32_t **keys_out,
                             uint32_t **vals_out, hipStream_t st) {
  if (key_bits <= 0) return hipErrorInvalidValue;
  uint32_t nb = cdiv(n, kSortTile);
  uint32_t *ka = keys, *va = vals, *kb = keys_tmp, *vb = vals_tmp;
  bool first = true;
  for (int shift = 0; shift < key_bits; shift += 8) {
    k_radix_hist<<<nb, kSortThreads, 0, st>>>(ka, n, shift, hist, nb);
    const hipError_t e = launch_scan(hist, 256u * nb, scan_tmp, st);
    if (e != hipSuccess) return e;
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
  *keys_out = ka;
  *vals_out = va;
  return hipGetLastError();
}

hipError_t launch_seg_sort(const uint32_t *bucket, uint32_t n_per, uint32_t nclouds,
                           int bucket_bits, uint32_t *keys_out, uint32_t *vals_out,
                           hipStream_t st) {
  // rows in 14 bits, bucket above them; the cloud index above the bucket in
  // the keys written
  if (n_per > kSegSortMax || bucket_bits <= 0 || bucket_bits > 18 || nclouds == 0)
    return hipErrorInvalidValue;
  k_seg_sort<<<nclouds, 1024, 0, st>>>(bucket, n_per, bucket_bits, bucket_bits, keys_out,
                                       vals_out);
  return hipGetLastError();
}

hipError_t launch_cloud_keys(const uint32_t *bucket, uint32_t total, uint32_t n_per,
                             int bucket_bits, uint32_t *key, hipStream_t st) {
  k_cloud_keys<<<cdiv(total, 256), 256, 0, st>>>(bucket, total, n_per, bucket_bits, key);
  return hipGetLastError();
}

hipError_t launch_key2(const uint32_t *lorig, const uint32_t *bucket, const uint32_t *fine,
                       uint32_t n, uint32_t n_per, int cloud_shift, int fine_shift, int fine_bits,
                       uint32_t *key2, hipStream_t st) {
  k_key2<<<cdiv(n, 256), 256, 0, st>>>(lorig, bucket, fine, n, n_per, cloud_shift, fine_shift,
                                       fine_bits, key2);
  return hipGetLastError();
}

hipError_t launch_leaf_counts(const uint32_t *counts, uint32_t T, uint32_t *lc, uint32_t *maxocc,
                              uint32_t *total, uint32_t *occupied, hipStream_t st) {
  k_leaf_counts<<<cdiv(T, 256), 256, 0, st>>>(counts, T, lc, maxocc, total, occupied);
  return hipGetLastError();
}

hipError_t launch_gather(const uint32_t *prank, const uint32_t *lorig, uint32_t base,
                         const uint32_t *bucket, const uint32_t *cell_start, const float *xyz,
                         uint32_t n, uint32_t padded, uint32_t cap, float4 *P4, uint2 *RO,
                         uint32_t *R, uint32_t *phys0, hipStream_t st) {
  k_gather<<<cdiv(n, 256), 256, 0, st>>>(prank, lorig, base, bucket, cell_start, xyz, n, padded,
                                         cap, P4, RO, R, phys0);
  return hipGetLastError();
}

hipError_t launch_leaf_build(const uint32_t *cell_start, const uint32_t *cell_leaf, uint32_t T,
                             uint32_t padded, uint32_t cap, uint32_t lpc, uint32_t mixed,
                             uint32_t n, uint32_t nleaves, const RangeDev &r, const float4 *P4,
                             const uint2 *RO, float4 *leaf_lo, float4 *leaf_hi,
                             uint32_t *leaf_cell, uint32_t *leaf_al, uint2 *leaf_sc,
                             uint2 *leaf_cbox, uint64_t *leaf_key, float4 *leaf_pos,
                             uint2 *cell_info, hipStream_t st) {
  // the cell table has T + 1 entries; mixed leaves are described one a thread
  const uint64_t cells = (uint64_t)T + 1, threads = mixed && nleaves > cells ? nleaves : cells;
  k_cells<<<cdiv(threads, 256), 256, 0, st>>>(cell_start, cell_leaf, T, padded, cap, lpc, mixed, n,
                                              nleaves, r, P4, cell_info, leaf_lo, leaf_hi,
                                              leaf_cell, leaf_al, leaf_sc);
  if (nleaves)
    k_leaf_bbox<<<cdiv(nleaves, 4), 256, 0, st>>>(nleaves, r, P4, RO, leaf_lo, leaf_hi, leaf_cbox,
                                                  leaf_key, leaf_pos);
  return hipGetLastError();
}

hipError_t launch_init_state(const CloudDev &c, const uint32_t *d_phys0, hipStream_t st) {
  if (c.nl1)
    k_l1_init_state<<<cdiv(c.nl1, 4), 256, 0, st>>>(c, d_phys0);
  else
    k_init_state<<<1, 64, 0, st>>>(c, d_phys0);
  return hipGetLastError();
}

// ---- the build steps of many clouds, one launch each (grid y = cloud) -----

// Cell keys of many clouds, the bucket populations counted in LDS: workgroup (x, cloud)
// takes points [x kCellChunk, (x + 1) kCellChunk) of its cloud and adds its
// nonzero bins to the cloud's counts, or stores every bin (WHOLE: one
// workgroup covers each cloud).  One device-scope atomic per point, 2^20
// of them for 64 clouds of 16,384 points, took 42 us.  Dynamic LDS: T words.
constexpr uint32_t kCellChunk = 16384;
template <bool WHOLE>
__global__ __launch_bounds__(1024) void kb_cell_keys_lds(const BuildDev *__restrict__ bd) {
  extern __shared__ uint32_t s_cnt[];
  const BuildDev &b = bd[blockIdx.y];
  for (uint32_t t = threadIdx.x; t < b.T; t += blockDim.x) s_cnt[t] = 0;
  __syncthreads();
  const uint32_t i0 = blockIdx.x * kCellChunk;
#pragma unroll 4
  for (uint32_t k = threadIdx.x; k < kCellChunk; k += blockDim.x) {
    const uint32_t bk = cell_keys_at(i0 + k, b.xyz, b.n, b.c.r, b.c.lut, b.bucket, b.fine,
                                     nullptr, b.small);
    if (bk < b.T) atomicAdd(&s_cnt[bk], 1u);
  }
  __syncthreads();
  for (uint32_t t = threadIdx.x; t < b.T; t += blockDim.x) {
    const uint32_t v = s_cnt[t];
    if (WHOLE) b.counts[t] = v;
    else if (v) atomicAdd(&b.counts[t], v);
  }
}

__global__ __launch_bounds__(256) void kb_leaf_counts(const BuildDev *__restrict__ bd) {
  __shared__ uint32_t s_red[3];
  const BuildDev &b = bd[blockIdx.y];
  if (blockIdx.x * blockDim.x >= b.T) return;  // the whole block: no barrier is split
  leaf_counts_block(blockIdx.x, b.counts, b.T, b.lc, b.small + 1, b.small + 3, b.small + 4, s_red);
}

// block 2i scans cloud i's bucket populations, block 2i + 1 its leaf counts
__global__ __launch_bounds__(1024) void kb_scans(const BuildDev *__restrict__ bd) {
  __shared__ uint32_t wsum[16];
  const BuildDev &b = bd[blockIdx.x >> 1];
  scan_excl_block((blockIdx.x & 1) ? b.lc : b.counts, b.T, wsum);
}

__global__ void kb_zero_slots(const BuildDev *__restrict__ bd) {
  const BuildDev &b = bd[blockIdx.y];
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (!b.c.padded || i >= b.c.nslots) return;
  b.c.P4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  const_cast<uint2 *>(b.c.RO)[i] = make_uint2(0u, 0u);
  const_cast<uint32_t *>(b.c.R)[i] = 0u;
}

__global__ void kb_gather(const BuildDev *__restrict__ bd) {
  const BuildDev &b = bd[blockIdx.y];
  gather_at(blockIdx.x * blockDim.x + threadIdx.x, b.prank, b.lorig, b.base, b.bucket, b.counts,
            b.xyz, b.n, b.c.padded, b.cap, b.c.P4, const_cast<uint2 *>(b.c.RO),
            const_cast<uint32_t *>(b.c.R), b.small + 2);
}

// thread i: cell i's table entry, and the leaves of bucket i (or, with mixed
// leaves, leaf i)
__global__ void kb_cells(const BuildDev *__restrict__ bd) {
  const BuildDev &b = bd[blockIdx.y];
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  cell_info_at(i, b.counts, b.lc, b.T, const_cast<uint2 *>(b.c.cell_info));
  if (b.c.mixed)
    leaf_desc_mixed_at(i, b.n, b.c.nleaves, const_cast<float4 *>(b.c.leaf_lo),
                       const_cast<float4 *>(b.c.leaf_hi), const_cast<uint32_t *>(b.c.leaf_cell),
                       const_cast<uint32_t *>(b.c.leaf_al), const_cast<uint2 *>(b.c.leaf_sc));
  else
    leaf_desc_at(i, b.counts, b.lc, b.T, b.c.padded, b.cap, b.c.lpc, b.c.r, b.c.P4,
                 const_cast<float4 *>(b.c.leaf_lo), const_cast<float4 *>(b.c.leaf_hi),
                 const_cast<uint32_t *>(b.c.leaf_cell), const_cast<uint32_t *>(b.c.leaf_al),
                 const_cast<uint2 *>(b.c.leaf_sc));
}

__global__ __launch_bounds__(256) void kb_leaf_bbox(const BuildDev *__restrict__ bd) {
  const BuildDev &b = bd[blockIdx.y];
  leaf_bbox_at(blockIdx.x * 4 + (threadIdx.x >> 6), b.c.nleaves, b.c.r, b.c.P4, b.c.RO,
               const_cast<float4 *>(b.c.leaf_lo), const_cast<float4 *>(b.c.leaf_hi),
               const_cast<uint2 *>(b.c.leaf_cbox), b.c.leaf_key, b.c.leaf_pos);
}

__global__ __launch_bounds__(256) void kb_l1_init(const BuildDev *__restrict__ bd) {
  const BuildDev &b = bd[blockIdx.y];
  const CloudDev &c = b.c;
  l1_init_at(blockIdx.x * 4 + (threadIdx.x >> 6), c.nleaves, c.nl1, c.leaf_key, c.leaf_pos,
             c.leaf_lo, c.leaf_hi, c.leaf_al, c.r.na, c.l1_key, c.l1_pos,
             const_cast<float4 *>(c.l1_lo), const_cast<float4 *>(c.l1_hi),
             const_cast<uint2 *>(c.l1_cbox));
}

__global__ void kb_init_state(const BuildDev *__restrict__ bd) {
  if (threadIdx.x == 0) init_state_of(bd[blockIdx.x].c, bd[blockIdx.x].small + 2);
}

hipError_t launch_build_first_many(const BuildDev *d_bd, uint32_t nclouds, uint32_t nmax,
                                   uint32_t tmax, hipStream_t st) {
  if (tmax + 1 > kScanSingleMax) return hipErrorInvalidValue;
  if (nmax) {
    // bucket populations in LDS (tmax <= kScanSingleMax words); clouds with
    // fewer points than one workgroup's chunk take their counts whole
    const uint32_t chunks = cdiv(nmax, kCellChunk);
    if (chunks == 1)
      kb_cell_keys_lds<true><<<dim3(1, nclouds), 1024, tmax * 4, st>>>(d_bd);
    else
      kb_cell_keys_lds<false><<<dim3(chunks, nclouds), 1024, tmax * 4, st>>>(d_bd);
  }
  kb_leaf_counts<<<dim3(cdiv(tmax, 256), nclouds), 256, 0, st>>>(d_bd);
  kb_scans<<<2 * nclouds, 1024, 0, st>>>(d_bd);
  return hipGetLastError();
}

hipError_t launch_build_rest_many(const BuildDev *d_bd, uint32_t nclouds, uint32_t nmax,
                                  uint32_t tmax, uint32_t slots_max, uint32_t leaves_max,
                                  uint32_t l1_max, hipStream_t st) {
  if (slots_max) kb_zero_slots<<<dim3(cdiv(slots_max, 256), nclouds), 256, 0, st>>>(d_bd);
  if (nmax) kb_gather<<<dim3(cdiv(nmax, 256), nclouds), 256, 0, st>>>(d_bd);
  const uint64_t cells_or_leaves = (uint64_t)tmax + 1 > leaves_max ? (uint64_t)tmax + 1 : leaves_max;
  kb_cells<<<dim3(cdiv(cells_or_leaves, 256), nclouds), 256, 0, st>>>(d_bd);
  if (leaves_max) kb_leaf_bbox<<<dim3(cdiv(leaves_max, 4), nclouds), 256, 0, st>>>(d_bd);
  if (l1_max) kb_l1_init<<<dim3(cdiv(l1_max, 4), nclouds), 256, 0, st>>>(d_bd);
  kb_init_state<<<nclouds, 64, 0, st>>>(d_bd);
  return hipGetLastError();
}

hipError_t preload_build_kernels() {
  return func_attributes(k_cell_keys_dr, k_cloud_bounds, k_range_of_bounds, k_seg_counts,
                         k_cell_keys, k_radix_hist, k_scan_excl, k_scan_sums, k_scan_apply,
                         k_radix_scatter, k_seg_sort, k_cloud_keys, k_key2, k_leaf_counts, k_cells,
                         k_gather, k_leaf_bbox, k_l1_init_state,
                         k_init_state, k_fill_u32, kb_cell_keys_lds<true>,
                         kb_cell_keys_lds<false>, kb_leaf_counts, kb_scans,
                         kb_zero_slots, kb_gather, kb_cells, kb_leaf_bbox, kb_l1_init,
                         kb_init_state);
}

}  // namespace nsfps
