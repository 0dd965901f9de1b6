// Device helpers shared by the build and sampling kernels.  Every fp32
// expression here is evaluated without contraction (the translation units are
// compiled with -ffp-contract=off and this header repeats the pragma).
#pragma once

#include <hip/hip_runtime.h>

#include <float.h>
#include <math.h>
#include <stdint.h>

#include "nsfps_internal.h"

#pragma clang fp contract(off)

// Global address space.  Pointers read from a struct are generic, and generic
// (flat) accesses also count against the LDS wait counter, so every LDS wait
// would also wait for outstanding HBM loads; device code therefore accesses
// global memory through gptr().
// (The host compilation pass of these device functions keeps generic pointers.)
#if defined(__HIP_DEVICE_COMPILE__)
#define NSFPS_GLOBAL __attribute__((address_space(1)))
#else
#define NSFPS_GLOBAL
#endif

namespace nsfps {

template <class T>
__device__ __forceinline__ NSFPS_GLOBAL T *gptr(T *p) {
  return (NSFPS_GLOBAL T *)p;
}
template <class T>
__device__ __forceinline__ const NSFPS_GLOBAL T *gptr(const T *p) {
  return (const NSFPS_GLOBAL T *)p;
}

// std::min(v, hi) / std::max(lo, v) with <algorithm>'s comparison order.
__device__ __forceinline__ float std_min(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float std_max(float a, float b) { return (a < b) ? b : a; }

// Point3D::compute_block_indices, one axis (src/yuezu_fps.cpp:170-193):
// clamp into [min, max - 1e-6], scale by the stored reciprocal, truncate,
// clamp to the last block.
// Makes wave-uniform values live in scalar registers at this point.  The
// compiler otherwise issues each kernel-argument or CloudDev field read at
// its first use, behind the branches before it, one memory round trip each;
// values named here are read together, ahead of the first branch.
template <typename T>
__device__ __forceinline__ void pin_sgpr1(T v) {
  asm volatile("" : : "s"(v));
}
template <typename... T>
__device__ __forceinline__ void pin_sgpr(T... v) {  // by value: every read precedes every asm
  (pin_sgpr1(v), ...);
}

// Per-lane values: the loads producing them complete here, so loads issued
// before this point overlap instead of being moved behind a later branch.
template <typename T>
__device__ __forceinline__ void pin_vgpr1(T v) {
  asm volatile("" : : "v"(v));
}
template <typename... T>
__device__ __forceinline__ void pin_vgpr(T... v) {
  (pin_vgpr1(v), ...);
}

// p held in vector registers from here on: the compiler cannot load it again
// from the kernel's arguments, a scalar load that after a vector store must
// wait for the store to complete.
template <typename T>
__device__ __forceinline__ T *vgpr_ptr(T *p) {
  const uint64_t u = (uint64_t)p;
  uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
  asm volatile("" : "+v"(lo), "+v"(hi));
  return (T *)(((uint64_t)hi << 32) | lo);
}

// The range values cell_axis reads, as arguments of pin_sgpr.
#define NSFPS_CELL_RANGE(r)                                                                   \
  (r).mn[0], (r).mn[1], (r).mn[2], (r).hiclamp[0], (r).hiclamp[1], (r).hiclamp[2],           \
      (r).inv_bs[0], (r).inv_bs[1], (r).inv_bs[2], (r).blocks[0], (r).blocks[1], (r).blocks[2]

__device__ __forceinline__ uint32_t cell_axis(const RangeDev &r, int a, float v) {
  float c = std_max(r.mn[a], std_min(v, r.hiclamp[a]));
  uint32_t i = (uint32_t)((c - r.mn[a]) * r.inv_bs[a]);
  return i < r.blocks[a] - 1 ? i : r.blocks[a] - 1;
}

// Bucket of a cell: LUT Morton code, % total_blocks (src/yuezu_fps.cpp:195-199,
// 411-416, 592).  The modulo is the identity when every axis has 2^k >= 2
// blocks.
__device__ __forceinline__ uint32_t bucket_of(const RangeDev &r, const uint32_t *lut, uint32_t ix,
                                              uint32_t iy, uint32_t iz) {
  uint32_t code = lut[r.lut_off[0] + ix] | lut[r.lut_off[1] + iy] | lut[r.lut_off[2] + iz];
  return r.bijective ? code : code % r.T;
}

// The bits of v at the set positions of mask, packed from bit 0 up.
__device__ __forceinline__ uint32_t extract_bits(uint32_t v, uint32_t mask) {
  uint32_t r = 0, k = 0;
  for (uint32_t m = mask; m; m &= m - 1, ++k) r |= ((v >> __builtin_ctz(m)) & 1u) << k;
  return r;
}

// The cells of bucket b, packed 10 bits per axis, kNoCell-padded to r.na
// entries: every code b + jT below 2^cbits whose axis values lie inside the
// grid (src/yuezu_fps.cpp:413, 592: a cell's bucket is its LUT Morton code
// modulo the block count).
__device__ __forceinline__ void bucket_cells(const RangeDev &r, uint32_t b, uint32_t *out) {
  uint32_t k = 0;
  const uint64_t codes = 1ull << r.cbits;
  for (uint64_t code = b; code < codes && k < r.na; code += r.T) {
    const uint32_t x = extract_bits((uint32_t)code, r.cmask[0]);
    const uint32_t y = extract_bits((uint32_t)code, r.cmask[1]);
    const uint32_t z = extract_bits((uint32_t)code, r.cmask[2]);
    if (x < r.blocks[0] && y < r.blocks[1] && z < r.blocks[2]) out[k++] = x | (y << 10) | (z << 20);
  }
  for (; k < r.na; ++k) out[k] = kNoCell;
}

// Morton code of a cell from the concatenated LUTs.
__device__ __forceinline__ uint32_t cell_code(const RangeDev &r, const uint32_t *lut, uint32_t ix,
                                              uint32_t iy, uint32_t iz) {
  return lut[r.lut_off[0] + ix] | lut[r.lut_off[1] + iy] | lut[r.lut_off[2] + iz];
}

// Axis value whose Morton bits are `part`: the LUT is increasing, so a binary
// search finds it; kNone when no value has exactly these bits.
__device__ __forceinline__ uint32_t lut_inverse(const uint32_t *lut, uint32_t size, uint32_t part) {
  uint32_t lo = 0, hi = size;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) / 2;
    if (lut[mid] < part) lo = mid + 1;
    else hi = mid;
  }
  return (lo < size && lut[lo] == part) ? lo : 0xffffffffu;
}

// squared_distance (src/yuezu_fps.cpp:205-209): ((dx*dx + dy*dy) + dz*dz).
__device__ __forceinline__ float sqdist(float px, float py, float pz, float qx, float qy,
                                        float qz) {
  float dx = px - qx, dy = py - qy, dz = pz - qz;
  float s = dx * dx + dy * dy;
  return s + dz * dz;
}

// Lower bound of sqdist over a box with the same operation order.  Rounding
// is monotone, so it never exceeds sqdist(p, q) for a p inside the box; an
// empty box (lo > hi) gives +inf.
__device__ __forceinline__ float box_lb(float qx, float qy, float qz, float4 lo, float4 hi) {
  if (lo.x > hi.x) return INFINITY;
  float gx = qx < lo.x ? lo.x - qx : (qx > hi.x ? qx - hi.x : 0.0f);
  float gy = qy < lo.y ? lo.y - qy : (qy > hi.y ? qy - hi.y : 0.0f);
  float gz = qz < lo.z ? lo.z - qz : (qz > hi.z ? qz - hi.z : 0.0f);
  float s = gx * gx + gy * gy;
  return s + gz * gz;
}

// Cube half-width of get_morton_codes_in_range (src/yuezu_fps.cpp:564-570):
// (int)ceil(sqrtf(D) / block_size), clamped to the grid size (larger values
// cover the same cells).
__device__ __forceinline__ int cube_half(float D, float bs, uint32_t blocks) {
  float rad = sqrtf(D < 0.0f ? 0.0f : D);
  float f = ceilf(rad / bs);
  if (!(f < (float)blocks)) return (int)blocks;
  return (int)f;
}

// Order-preserving map of floats to unsigned integers (finite values), and
// back: atomicMin / atomicMax on the integers give the floats' minimum and
// maximum in any order of arrival.
__device__ __forceinline__ uint32_t ord_of(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float float_of(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// Smallest D >= 0 whose clipped cube half-width, min(cube_half(D), blocks -
// 1), is at least k1 (INFINITY when none is): the half-width is monotone in D
// and non-negative floats order like their bit patterns, so a binary search
// over the bits finds it.  The host derives the same table with the same
// arithmetic (correctly rounded sqrtf and division).
__device__ __forceinline__ float cube_threshold_dev(float bs, uint32_t blocks, uint32_t k1) {
  if (k1 > blocks - 1) return INFINITY;
  uint32_t lo = 0, hi = 0x7f800000u;  // +inf: half-width blocks - 1 >= k1
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    const int h = cube_half(__uint_as_float(mid), bs, blocks);
    const uint32_t hc = (uint32_t)h < blocks - 1 ? (uint32_t)h : blocks - 1;
    if (hc >= k1) hi = mid;
    else lo = mid + 1;
  }
  return __uint_as_float(lo);
}

struct Cube {
  int lo[3], hi[3];
};

__device__ __forceinline__ Cube make_cube(const RangeDev &r, float D, float qx, float qy,
                                          float qz) {
  Cube cb;
  const float q[3] = {qx, qy, qz};
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

// When bucket = code % T is not one-to-one, several cells share a bucket.  A
// cube cell stands for its bucket only if no cell of the cube has a smaller
// code of the same bucket, so that every bucket of the cube is visited once
// (the reference visits each bucket of its code list once,
// src/yuezu_fps.cpp:573-597).
__device__ __forceinline__ bool bucket_first_in_cube(const RangeDev &r, const uint32_t *lut,
                                                     uint32_t code, const Cube &cb) {
  const uint32_t sz[3] = {r.lut_off[1] - r.lut_off[0], r.lut_off[2] - r.lut_off[1],
                          r.lut_total - r.lut_off[2]};
  for (uint32_t k = code % r.T; k < code; k += r.T) {
    bool inside = true;
    for (int a = 0; a < 3 && inside; ++a) {
      const uint32_t mask = lut[r.lut_off[a] + sz[a] - 1];
      const uint32_t v = lut_inverse(lut + r.lut_off[a], sz[a], k & mask);
      inside = v != 0xffffffffu && (int)v >= cb.lo[a] && (int)v <= cb.hi[a];
    }
    if (inside) return false;
  }
  return true;
}

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// ---- wave64 reductions on the VALU (DPP row permutes + readlane), no LDS

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_or0(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

// Pure DPP move (old value undefined): lets the compiler fold it into the
// consuming VALU op.  Only used with controls that read a valid lane for
// every lane (quad permutes, row mirrors), so bound_ctrl never applies.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

constexpr int kDppQuad1032 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuad2301 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppShr1 = 0x111, kDppShr2 = 0x112, kDppShr4 = 0x114, kDppShr8 = 0x118;

template <int CTRL>
__device__ __forceinline__ void max_step(uint32_t &hi, uint32_t &lo) {
  uint32_t oh = dpp<CTRL>(hi), ol = dpp<CTRL>(lo);
  bool take = oh > hi || (oh == hi && ol > lo);
  hi = take ? oh : hi;
  lo = take ? ol : lo;
}

__device__ __forceinline__ uint32_t rdlane(uint32_t v, uint32_t l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}

// Maximum of a u32 over each row of 16 lanes, in every lane of the row (all
// lanes must be active).
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, dpp_mov<kDppQuad1032>(v));
  v = max(v, dpp_mov<kDppQuad2301>(v));
  v = max(v, dpp_mov<kDppHalfMirror>(v));
  v = max(v, dpp_mov<kDppMirror>(v));
  return v;
}

// Maximum of a u32 over the 64 lanes (all lanes must be active); the result
// is wave-uniform: the four row maxima.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row_max_u32(v);
  return max(max(rdlane(v, 0), rdlane(v, 16)), max(rdlane(v, 32), rdlane(v, 48)));
}

// Scalar max of two wave-uniform values, kept on the scalar unit (a vector
// max here would put the result in a VGPR and every later test on it would
// be a vector compare feeding a branch).
__device__ __forceinline__ uint32_t smax_u32(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("s_max_u32 %0, %1, %2" : "=s"(r) : "s"(a), "s"(b) : "scc");
  return r;
}

// wave_max_u32 with the result in a scalar register.
__device__ __forceinline__ uint32_t wave_max_u32_s(uint32_t v) {
  v = row_max_u32(v);
  return smax_u32(smax_u32(rdlane(v, 0), rdlane(v, 16)), smax_u32(rdlane(v, 32), rdlane(v, 48)));
}

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

// Minimum of a u32 over the 64 lanes (all lanes must be active); wave-uniform.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_mov<kDppQuad1032>(v));
  v = min(v, dpp_mov<kDppQuad2301>(v));
  v = min(v, dpp_mov<kDppHalfMirror>(v));
  v = min(v, dpp_mov<kDppMirror>(v));
  return min(min(rdlane(v, 0), rdlane(v, 16)), min(rdlane(v, 32), rdlane(v, 48)));
}

// Lane holding the largest key (hi << 32 | lo) among active lanes, or 64 when
// none is active; mhi receives the largest hi.  Keys of active lanes are
// unique, so the winner is unique.  The common case reduces hi only; lo is
// reduced among the lanes tied on hi.
__device__ __forceinline__ uint32_t key_winner(uint32_t hi, uint32_t lo, bool act, uint32_t &mhi) {
  const uint32_t m = wave_max_u32(act ? hi : 0u);
  uint64_t t = __ballot(act && hi == m);
  if (__popcll(t) > 1) {
    const uint32_t l = wave_max_u32((act && hi == m) ? lo : 0u);
    t = __ballot(act && hi == m && lo == l);
  }
  mhi = m;
  return t ? (uint32_t)__ffsll((long long)t) - 1 : 64u;
}

// Maximum of a u64 over the 64 lanes (all lanes must be active); the result
// is wave-uniform.  Rows of 16 lanes by DPP, then the four row maxima.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
  uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
  max_step<kDppQuad1032>(hi, lo);
  max_step<kDppQuad2301>(hi, lo);
  max_step<kDppHalfMirror>(hi, lo);
  max_step<kDppMirror>(hi, lo);
  uint64_t best = ((uint64_t)rdlane(hi, 0) << 32) | rdlane(lo, 0);
#pragma unroll
  for (uint32_t r = 16; r < 64; r += 16) {
    uint64_t v = ((uint64_t)rdlane(hi, r) << 32) | rdlane(lo, r);
    best = v > best ? v : best;
  }
  return best;
}

// Inclusive prefix sum over the 64 lanes (all lanes active).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += dpp_or0<kDppShr1>(v);
  v += dpp_or0<kDppShr2>(v);
  v += dpp_or0<kDppShr4>(v);
  v += dpp_or0<kDppShr8>(v);
  const uint32_t t0 = rdlane(v, 15), t1 = rdlane(v, 31), t2 = rdlane(v, 47);
  const uint32_t row = lane_id() >> 4;
  v += (row >= 1 ? t0 : 0u) + (row >= 2 ? t1 : 0u) + (row >= 3 ? t2 : 0u);
  return v;
}

// Block-wide exclusive scan of one value per thread with a single barrier:
// every wave reads all wave totals.  Consecutive calls must alternate wsum
// buffers (kLW entries each) unless a barrier separates them.
template <uint32_t kLW>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *total) {
  const uint32_t lane = lane_id(), wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (uint32_t w = 0; w < kLW; ++w) {
    uint32_t t = wsum[w];
    before += w < wave ? t : 0u;
    all += t;
  }
  *total = all;
  return x - v + before;
}

// Lanes below this one whose bit is set in mask.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Lane holding the wave maximum (keys are unique among active lanes).
__device__ __forceinline__ uint32_t argmax_lane(uint64_t k, uint64_t km, bool active) {
  uint64_t who = __ballot(active && k == km);
  return who ? (uint32_t)__ffsll((long long)who) - 1 : 0u;
}

// Wave-uniform values moved to scalar registers.
__device__ __forceinline__ float uni(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ uint32_t uni(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint64_t uni(uint64_t v) {
  return ((uint64_t)uni((uint32_t)(v >> 32)) << 32) | uni((uint32_t)v);
}
__device__ __forceinline__ float4 uni(float4 v) {
  return make_float4(uni(v.x), uni(v.y), uni(v.z), uni(v.w));
}

// Value of lane src (wave-uniform src) for every lane.
__device__ __forceinline__ float4 shfl_f4(float4 v, uint32_t src) {
  return make_float4(__uint_as_float(rdlane(__float_as_uint(v.x), src)),
                     __uint_as_float(rdlane(__float_as_uint(v.y), src)),
                     __uint_as_float(rdlane(__float_as_uint(v.z), src)),
                     __uint_as_float(rdlane(__float_as_uint(v.w), src)));
}

}  // namespace nsfps
