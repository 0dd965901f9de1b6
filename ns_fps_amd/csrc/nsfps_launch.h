// Kernel launchers (defined in nsfps_build.hip, nsfps_sample.hip,
// nsfps_runs.hip and nsfps_group.hip; called by nsfps_host.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "nsfps_internal.h"

namespace nsfps {

// Loads the kernels of one translation unit on the current device.  The
// runtime loads a code object, and resolves a kernel in it, when the kernel
// is first used; done at device set-up, that work stays out of the first
// call's device time.
hipError_t preload_build_kernels();
hipError_t preload_runs_kernels();
hipError_t preload_group_kernels();

// hipFuncGetAttributes on every kernel given (it loads the kernel's code
// object and resolves the kernel); the first error is returned.
template <typename... K>
hipError_t func_attributes(K... kernels) {
  hipError_t e = hipSuccess;
  hipFuncAttributes a;
  ((e = e == hipSuccess ? hipFuncGetAttributes(&a, reinterpret_cast<const void *>(kernels)) : e),
   ...);
  return e;
}


// words 32-bit words at p set to value
hipError_t launch_fill_u32(void *p, uint32_t value, uint64_t words, hipStream_t st);

// build
// counts null: no bucket populations (launch_seg_counts gives them from the
// sorted buckets)
hipError_t launch_cell_keys(const float *xyz, uint32_t n, const RangeDev &r, const uint32_t *lut,
                            uint32_t *bucket, uint32_t *fine, uint32_t *counts, uint32_t *bad,
                            hipStream_t st);
// k_cell_keys with the range in device memory (d_range).
hipError_t launch_cell_keys_dr(const float *xyz, uint32_t n, const RangeDev *d_range,
                               const uint32_t *lut, uint32_t *bucket, uint32_t *fine,
                               uint32_t *counts, uint32_t *bad, hipStream_t st);
// bucket populations into zeroed counts from n sorted bucket keys
hipError_t launch_seg_counts(const uint32_t *keys, uint32_t n, uint32_t *counts, hipStream_t st);
// exclusive scan in place, data[len] = total; tmp holds scan_tmp_len(len) words
uint32_t scan_tmp_len(uint32_t len);
hipError_t launch_scan(uint32_t *data, uint32_t len, uint32_t *tmp, hipStream_t st);
uint32_t radix_hist_len(uint32_t n);
hipError_t launch_radix_sort(uint32_t *keys, uint32_t *vals, uint32_t *keys_tmp,
                             uint32_t *vals_tmp, uint32_t n, int key_bits, uint32_t *hist,
                             uint32_t *scan_tmp, bool iota_values, uint32_t **keys_out,
                             uint32_t **vals_out,
                             hipStream_t st);
// sort key (cloud << bucket_bits) | bucket of clouds of n_per points stored
// one after another
constexpr uint32_t kSegSortMaxPoints = 16384;
// The logical sort of nclouds clouds of n_per <= 16,384 points each (cloud
// s's buckets at bucket + s * n_per), one workgroup per cloud: the keys
// ((s << bucket_bits) | bucket) and rows the radix sort over (cloud, bucket)
// keys writes.  bucket_bits <= 18.
hipError_t launch_seg_sort(const uint32_t *bucket, uint32_t n_per, uint32_t nclouds,
                           int bucket_bits, uint32_t *keys_out, uint32_t *vals_out,
                           hipStream_t st);
hipError_t launch_cloud_keys(const uint32_t *bucket, uint32_t total, uint32_t n_per,
                             int bucket_bits, uint32_t *key, hipStream_t st);
hipError_t launch_key2(const uint32_t *lorig, const uint32_t *bucket, const uint32_t *fine,
                       uint32_t n, uint32_t n_per, int cloud_shift, int fine_shift, int fine_bits,
                       uint32_t *key2, hipStream_t st);
hipError_t launch_leaf_counts(const uint32_t *counts, uint32_t T, uint32_t *lc, uint32_t *maxocc,
                              uint32_t *total, uint32_t *occupied, hipStream_t st);
// prank / lorig may come from sorts holding other clouds too: ranks and rows
// of this cloud are base + 0 .. base + n - 1 (prank points at this cloud's part)
hipError_t launch_gather(const uint32_t *prank, const uint32_t *lorig, uint32_t base,
                         const uint32_t *bucket, const uint32_t *cell_start, const float *xyz,
                         uint32_t n, uint32_t padded, uint32_t cap, float4 *P4, uint2 *RO,
                         uint32_t *R, uint32_t *phys0, hipStream_t st);
// The cell table (cell_info, T + 1 entries) and the leaves: per bucket
// (padded or dense), or with mixed = 1 runs of 64 slots of the logical order;
// then their boxes, cell corners and initial keys.
hipError_t launch_leaf_build(const uint32_t *cell_start, const uint32_t *cell_leaf, uint32_t T,
                             uint32_t padded, uint32_t cap, uint32_t lpc, uint32_t mixed,
                             uint32_t n, uint32_t nleaves, const RangeDev &r, const float4 *P4,
                             const uint2 *RO, float4 *leaf_lo, float4 *leaf_hi,
                             uint32_t *leaf_cell, uint32_t *leaf_al, uint2 *leaf_sc,
                             uint2 *leaf_cbox, uint64_t *leaf_key, float4 *leaf_pos,
                             uint2 *cell_info, hipStream_t st);
hipError_t launch_init_state(const CloudDev &c, const uint32_t *d_phys0, hipStream_t st);

// The build of many clouds, each step one launch for all of them (grid y =
// cloud), when every cloud has at most kManyMaxBuckets buckets.  Parameters
// per cloud live in device memory.
// Words of build statistics per cloud (BuildDev::small), read back in one copy.
constexpr uint32_t kStatWords = 8;

struct BuildDev {
  CloudDev c;                // the cloud's buffers and sizes
  const float *xyz;          // input (device)
  uint32_t *bucket, *fine;   // per input row
  uint32_t *counts, *lc;     // per bucket, scanned to first slot / first leaf
  uint32_t *small;           // kStatWords: [0] non-finite flag, [1] largest bucket, [2] slot
                             // of row 0, [3] dense leaves, [4] buckets holding points
  const uint32_t *prank;     // the sorts: this cloud's part of the physical order (null: the
                             // logical order)
  const uint32_t *lorig;     //   and the logical order of all clouds sorted together
  uint32_t n, T, cap, base;  // cap: slots per bucket when padded; base: this cloud's
                             // first rank / row in the sorts
};
constexpr uint32_t kManyMaxBuckets = 16383;
// cell keys, bucket populations, leaf counts and both scans
hipError_t launch_build_first_many(const BuildDev *d_bd, uint32_t nclouds, uint32_t nmax,
                                   uint32_t tmax, hipStream_t st);
// slots, cell table, leaves, level-1 nodes, initial state
hipError_t launch_build_rest_many(const BuildDev *d_bd, uint32_t nclouds, uint32_t nmax,
                                  uint32_t tmax, uint32_t slots_max, uint32_t leaves_max,
                                  uint32_t l1_max, hipStream_t st);

// compute_bbox of nclouds clouds of n_per points stored one after another
// (xyz, device) and the ranges of those bounds: out[b] (tmpl's block-count
// fields, the bounds' fp32 fields), bounds[6 b ..] (min x, max x, min y,
// max y, min z, max z), and bd[b].c.r when bd is non-null.  ord: 6 nclouds
// words of workspace.
hipError_t launch_device_ranges(const float *xyz, uint32_t n_per, uint32_t nclouds,
                                const RangeDev &tmpl, uint32_t *ord, RangeDev *out,
                                float *bounds, BuildDev *bd, hipStream_t st);

// sampling
hipError_t launch_wide_steps(const CloudDev &c, uint32_t steps, uint32_t grid, hipStream_t st);
hipError_t launch_late_loop(const CloudDev *d_clouds, uint32_t nclouds, uint32_t lds_bytes,
                            bool profile, uint32_t threads, hipStream_t st);
constexpr uint32_t kProfWords = 64;

// speculative-run engine
// split: the rounds' update pass is split (node keys move into their parts)
hipError_t launch_runs_init(const CloudDev *d_clouds, uint32_t nclouds, bool split,
                            hipStream_t st);
// `rounds` rounds of update pass, refinement passes, gather pass and run.
// alias: some cloud's cells share buckets.  leaf_bound: the update pass also
// bounds each pick by each leaf's box; split: it takes kUpdateSplit
// workgroups per level-1 node; mixed: the clouds' leaves are runs of 64 slots
// that may hold several buckets (never with alias).  hot: the run kernel's
// hot-set size, 64 or 128 (with alias always 64); dense: with 128, the walk
// for clouds whose filled buckets hold many points; whole: with 64 and no
// alias, the run kernel that applies a large-cube sample holding the list's
// cell box with no cell test (for clouds in few buckets).
hipError_t launch_rounds(const CloudDev *d_clouds, uint32_t nclouds, uint32_t max_nl1,
                         uint32_t rounds, uint32_t passes, bool profile, bool alias,
                         bool leaf_bound, bool split, bool mixed, uint32_t hot, bool dense,
                         bool whole, hipStream_t st);

// grouping after sampling (nsfps_group.hip): out[i] = xyz[idx[i]] (bad gets 1
// for an index outside [0, n), whose row is zeroed); ball query rows of
// nsample indices by the ordered scan (ids: the centers to do, or null for
// 0 .. m - 1) or by the grid: build (bnd preset to 3 x 0xffffffff, 3 x 0),
// stable sort of keys by the caller, cells (cstart/cend zeroed, kBqMaxDim^3
// words each), query (centers with more than the hit capacity are listed in
// ovf_ids / ovf_count for the scan)
constexpr uint32_t kBqMaxDim = 128;
struct BqGrid {
  float mn[3];
  float inv_cs[3];
  uint32_t dim[3];
  uint32_t ncells;
};
hipError_t launch_gather_points(const float *xyz, uint32_t n, const int32_t *idx, uint32_t m,
                                float *out, uint32_t *bad, hipStream_t st);
hipError_t launch_ball_query(const float *xyz, uint32_t n, const float *centers,
                             const uint32_t *ids, uint32_t m, float r2, uint32_t nsample,
                             int32_t *out, hipStream_t st);
hipError_t launch_bq_grid_build(const float *xyz, uint32_t n, float radius, uint32_t *bnd,
                                BqGrid *grid, uint32_t *keys, hipStream_t st);
hipError_t launch_bq_cells(const uint32_t *skeys, const uint32_t *sidx, uint32_t n,
                           const float *xyz, const BqGrid *grid, uint32_t *cstart, uint32_t *cend,
                           float4 *spts, hipStream_t st);
hipError_t launch_bq_query(const float4 *spts, const BqGrid *grid, const uint32_t *cstart,
                           const uint32_t *cend, const float *centers, uint32_t m, float r2,
                           uint32_t nsample, int32_t *out, uint32_t *ovf_ids,
                           uint32_t *ovf_count, hipStream_t st);

}  // namespace nsfps
