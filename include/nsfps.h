/* nsfps -- MI355X-native farthest point sampling (NS-FPS semantics).
 *
 * C ABI of the drop-in boundary.  Plain pointers and sizes only; every entry
 * point returns an nsfps_status and, on failure, leaves a message readable with
 * nsfps_last_error() (thread-local).  The library never falls back to a CPU
 * path: without a usable HIP device, compute entry points fail with
 * NSFPS_EDEVICE.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   nsfps_range_derive   SpaceRange derived fields + make_range()
 *                        (src/yuezu_fps.h:56-83, src/yuezu_fps.cpp:7-161)
 *   nsfps_bbox           compute_bbox()          (src/yuezu_fps.cpp:643-670)
 *   nsfps_fps            yuezu_fps() behind fps_numpy()
 *                        (src/yuezu_fps.h:211-212, src/yuezu_fps.cpp:676-730,
 *                         yuezu_fps/yuezu_fps_pybind.cpp:67-86)
 *   nsfps_fps_bbox       fps_with_bbox()  (yuezu_fps/yuezu_fps_pybind.cpp:88-101)
 *   nsfps_fps_batched    no single counterpart: B independent yuezu_fps() calls
 *                        (the batched set-abstraction use of fps_numpy)
 *   nsfps_fps_device     yuezu_fps() on device-resident input (cf. the
 *                        reference GPU driver's FpsGPU::sample,
 *                        eval/src_gpu/yuezu_fps_gpu.h:90-126)
 *   nsfps_plan_create / _sample / _destroy
 *                        the reference GPU driver's FpsGPU::initialize /
 *                        sample and its teardown (eval/src_gpu/yuezu_fps_gpu.h:
 *                        90-126): build once, sample many times
 *   nsfps_gather_points, nsfps_ball_query (and _device)
 *                        no counterpart: the grouping step the reference's
 *                        callers run on its output (see their declarations)
 *   nsfps_fps_device_noalloc
 *                        no counterpart: nsfps_fps_device for callers that
 *                        cannot allocate device memory (see its declaration)
 */
#ifndef NSFPS_H
#define NSFPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  NSFPS_OK = 0,
  NSFPS_EINVAL = 1,      /* invalid argument (shape, range, non-finite input) */
  NSFPS_EDEVICE = 2,     /* HIP runtime / device failure, or no device */
  NSFPS_ENOMEM = 3,      /* device allocation failed */
  NSFPS_EUNSUPPORTED = 4 /* valid input outside what this build handles: more than
                            1024 blocks on an axis (cells are packed 10 bits per
                            axis), more than 2^31-1 points or samples, a cloud
                            needing more than 4096 level-1 nodes when the tree
                            engine is asked for (NSFPS_ENGINE=tree; the default
                            engine has no such limit), or a layout beyond the
                            allocation-free entry point's array */
} nsfps_status;

/* The nine primary SpaceRange fields (src/yuezu_fps.h:56-60).  Derived fields
 * are always recomputed from these, so a range edited field by field can never
 * carry stale derived values. */
typedef struct {
  float min_x, max_x;
  float min_y, max_y;
  float min_z, max_z;
  uint32_t x_blocks, y_blocks, z_blocks;
} nsfps_range;

/* Number of cube half-width thresholds per axis in nsfps_range_info. */
#define NSFPS_CUBE_THRESHOLDS 8

/* Derived SpaceRange values (src/yuezu_fps.cpp:7-40, 136-161). */
typedef struct {
  float inv_bs[3];     /* 1.0f / ((max - min) / (float)blocks) */
  float block_size[3]; /* (max - min) / blocks */
  uint32_t bits[3];    /* ceil(log2(blocks)), at least 1 */
  uint32_t total_bits;
  uint64_t total_blocks;
  /* cube_thr[a][k]: the smallest squared distance D >= 0 whose cube
   * half-width on axis a, min((int)ceilf(sqrtf(D) / block_size[a]),
   * blocks - 1) (get_morton_codes_in_range, src/yuezu_fps.cpp:564-570, cells
   * beyond the grid being clipped), is at least k + 1; INFINITY when it never
   * is.  The half-width is monotone in D, so it equals the number of
   * thresholds <= D below the last one. */
  float cube_thr[3][NSFPS_CUBE_THRESHOLDS];
} nsfps_range_info;

/* Per-call measurements of the last compute call on this thread. */
typedef struct {
  double build_ms;   /* device time: cell keys, sorts, leaves (hipEvents) */
  double sample_ms;  /* device time: the sampling loop (hipEvents) */
  double wide_ms;    /* part of sample_ms spent in grid-wide iterations */
  double late_ms;    /* the single-workgroup loop kernel alone, or all rounds of runs */
  double device_ms;  /* build_ms + sample_ms */
  double e2e_ms;     /* host wall time of the whole call incl. copies */
  uint64_t n_points;
  uint64_t n_clouds;
  uint64_t n_leaves;
  uint64_t wide_iters;  /* iterations run by the grid-wide kernel */
  uint64_t samples;     /* samples produced (sum over clouds) */
  uint32_t padded;      /* 1 when the single cloud used the padded cell layout */
  uint32_t lds_bytes;   /* dynamic LDS of the single-workgroup loop */
  uint64_t rounds;      /* speculative-run rounds (max over clouds; 0 for the tree loop) */
  uint32_t engine;      /* 1: speculative runs, 0: grid-wide steps + tree loop */
  uint32_t update_split; /* workgroups per level-1 node of the runs engine's update pass
                           (1, or 4 when the call has few level-1 nodes) */
  uint32_t mixed;       /* 1 when leaves were runs of 64 slots that may hold several buckets */
  uint32_t hot_set;     /* copies per hot set of the runs engine's run kernel (64 or 128;
                           0 for the tree loop) */
} nsfps_stats;

/* Library constants mirrored from src/yuezu_fps.h:19-50. */
#define NSFPS_DEFAULT_X_BLOCKS 16
#define NSFPS_DEFAULT_Y_BLOCKS 16
#define NSFPS_DEFAULT_Z_BLOCKS 16
#define NSFPS_MORTON_BLOCK_SIZE 16
#define NSFPS_CACHE_BLOCK_SIZE 16

const char *nsfps_last_error(void);
const char *nsfps_version(void);

/* Number of visible HIP devices (0 when none); never fails. */
int nsfps_device_count(void);

/* Prepares the current device for the library's calls: loads its kernels
 * (the runtime loads code on a kernel's first use), creates the stream and
 * events the host-buffer calls use, and makes one copy each way through a
 * pinned buffer (the runtime sets its copy path up on first use).  No
 * counterpart in the reference (a CPU library).  Optional: the first call on
 * a device does the same; calling this first keeps that one-time work (tens
 * of milliseconds, most of it the runtime's own start) out of the first
 * call.  NSFPS_EDEVICE when no device is visible. */
nsfps_status nsfps_init_device(void);

/* Derived fields and Morton LUTs of a range.  luts receives the x, y and z
 * LUTs back to back (2^bits[0] + 2^bits[1] + 2^bits[2] entries) when non-NULL
 * and lut_cap is large enough.  Replaces make_range()/make_uniform_range()'s
 * derivation (src/yuezu_fps.cpp:98-161). */
nsfps_status nsfps_range_derive(const nsfps_range *range, nsfps_range_info *info,
                                uint32_t *luts, uint64_t lut_cap);

/* compute_bbox(): exact fp32 bounds -/+ 1e-6 and the given block counts
 * (src/yuezu_fps.cpp:648-670).  n == 0 gives [0,1]^3 with 1x1x1 blocks. */
nsfps_status nsfps_bbox(const float *xyz, uint64_t n, uint32_t x_blocks,
                        uint32_t y_blocks, uint32_t z_blocks, nsfps_range *out);

/* compute_bbox of device-resident points (d_xyz, n x 3 float32) on the
 * device: the same bounds as nsfps_bbox over the finite points (minimum and
 * maximum do not depend on the order; +-0 differ only before the -/+ 1e-6),
 * and, when info is non-NULL, the range's derived fields as the sampling
 * calls derive them on the device (nsfps_range_derive gives the same bits on
 * the host).  This is the range nsfps_fps, nsfps_fps_bbox and the batched
 * calls use when they are given none.  stream: a hipStream_t (NULL = default
 * stream); the call returns after the stream work completes. */
nsfps_status nsfps_bbox_device(const float *d_xyz, uint64_t n, uint32_t x_blocks,
                               uint32_t y_blocks, uint32_t z_blocks, nsfps_range *out,
                               nsfps_range_info *info, void *stream);

/* FPS of one cloud.  xyz: host pointer, n x 3 float32, C order.  range == NULL
 * selects compute_bbox with the default 16^3 blocks.  out: host buffer of at
 * least n_samples int32 entries; *out_len receives the sample count (smaller
 * than n_samples when the maximum min-distance reaches 0).  Start index 0,
 * n_samples >= n returns 0..n-1, n == 0 or n_samples == 0 returns nothing. */
nsfps_status nsfps_fps(const float *xyz, uint64_t n, uint64_t n_samples,
                       const nsfps_range *range, int32_t *out, uint64_t *out_len);

/* fps_with_bbox(): compute_bbox with the given block counts, then FPS. */
nsfps_status nsfps_fps_bbox(const float *xyz, uint64_t n, uint64_t n_samples,
                            uint32_t x_blocks, uint32_t y_blocks,
                            uint32_t z_blocks, int32_t *out, uint64_t *out_len);

/* B independent clouds of n points each (xyz: B x n x 3, host).  ranges: B
 * ranges, or NULL for a per-cloud compute_bbox with blocks3 (NULL -> 16^3),
 * found on the device.  out: B x n_samples int32 (row b holds cloud b's
 * samples; entries past out_lens[b] are unspecified); out_lens: B.  The
 * reference samples one cloud per call (yuezu_fps, src/yuezu_fps.cpp:676-730,
 * with compute_bbox for range=None, yuezu_fps/yuezu_fps_pybind.cpp:74-76);
 * this is B such calls in one. */
nsfps_status nsfps_fps_batched(const float *xyz, uint64_t batch, uint64_t n,
                               uint64_t n_samples, const nsfps_range *ranges,
                               const uint32_t *blocks3, int32_t *out,
                               uint64_t *out_lens);

/* nsfps_fps_batched on device memory: d_xyz (B x n x 3 float32) and d_out
 * (B x n_samples int32, row b holding cloud b's samples) are device
 * pointers; ranges, blocks3 and out_lens are host memory as in
 * nsfps_fps_batched.  stream is a hipStream_t (NULL = default stream); the
 * call returns after the stream work completes. */
nsfps_status nsfps_fps_batched_device(const float *d_xyz, uint64_t batch, uint64_t n,
                                      uint64_t n_samples, const nsfps_range *ranges,
                                      const uint32_t *blocks3, int32_t *d_out,
                                      uint64_t *out_lens, void *stream);

/* FPS of one cloud whose points already live in device memory (d_xyz, n x 3
 * float32) writing device memory (d_out, n_samples int32).  stream is a
 * hipStream_t (NULL = default stream); the call returns after the stream work
 * completes.  range must be non-NULL. */
nsfps_status nsfps_fps_device(const float *d_xyz, uint64_t n, uint64_t n_samples,
                              const nsfps_range *range, int32_t *d_out,
                              uint64_t *out_len, void *stream);

/* nsfps_fps_device without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  The call's whole
 * workspace (cell keys, sorts, slots, leaves, tree and sampling state) lives
 * in a static device array of nsfps_noalloc_scratch_bytes() bytes (64 MiB)
 * per device, reserved on every device by the library's code object in each
 * process that loads the library, whether or not this call is used, and
 * held until the process ends.  A cloud whose layout needs more fails with
 * NSFPS_EUNSUPPORTED and a message giving both sizes: measured limits are
 * 450,736 points on a 32^3 grid, 460,416 on 16^3 and 428,160 on 64x64x16.
 * Same arguments, samples and guards as nsfps_fps_device; no hipMalloc,
 * hipFree, stream or event creation, and no memset nodes (fill kernels clear
 * what must start at zero).  Like every call here it cannot be captured into
 * a HIP graph (it reads results back between batches of rounds and waits for
 * the stream): on a capturing stream it returns NSFPS_EUNSUPPORTED before
 * enqueuing anything.  The array keeps the last call's contents; calls are
 * serialised by the library's lock, and a call on one device must not
 * overlap another use of that device's array (the library makes none).
 * Statistics report e2e_ms only (no device events). */
nsfps_status nsfps_fps_device_noalloc(const float *d_xyz, uint64_t n, uint64_t n_samples,
                                      const nsfps_range *range, int32_t *d_out,
                                      uint64_t *out_len, void *stream);
uint64_t nsfps_noalloc_scratch_bytes(void);

/* A cloud built once and sampled many times, the split of the reference GPU
 * driver's FpsGPU::initialize / FpsGPU::sample (eval/src_gpu/yuezu_fps_gpu.h:
 * 90-126).  nsfps_plan_create builds the structure of n points (xyz: host
 * pointer, or a device pointer when on_device != 0; read during the call
 * only) on the current device, in device memory the plan owns.
 * nsfps_plan_sample restores the points' min-distances and keys and runs the
 * sampling alone: the samples of nsfps_fps on the same points and range, for
 * any n_samples, written to device memory d_out (n_samples int32) on stream
 * (a hipStream_t, NULL = default stream); it returns after the stream work
 * completes and must be called with the plan's device current.  Calls on one
 * plan, or on several, are serialised by the library's lock.
 * nsfps_plan_destroy frees the plan (NULL is ignored). */
typedef struct nsfps_plan_s nsfps_plan;
nsfps_status nsfps_plan_create(const float *xyz, uint64_t n, const nsfps_range *range,
                               int on_device, nsfps_plan **plan);
nsfps_status nsfps_plan_sample(nsfps_plan *plan, uint64_t n_samples, int32_t *d_out,
                               uint64_t *out_len, void *stream);
void nsfps_plan_destroy(nsfps_plan *plan);

/* The step after sampling: set-abstraction grouping on the samples.  No
 * counterpart in the reference, which stops at the indices; the next step of
 * its callers is PointNet++'s sample-and-group (query_ball_point).
 *
 * nsfps_gather_points: out[i] = xyz[idx[i]], m x 3 float32.  An index outside
 * [0, n) fails with NSFPS_EINVAL (checked on the host for host pointers; the
 * device variant zeroes that row and reports it after the stream work).
 *
 * nsfps_ball_query: out is m x nsample int32; row j holds, in input order,
 * the first nsample indices i whose ((dx*dx + dy*dy) + dz*dz) to center j is
 * below radius*radius (float32, no contraction: the FPS distance); a row with
 * fewer hits repeats its first hit, a row with none is all zeros.  radius
 * must be finite and >= 0, nsample >= 1.
 *
 * The _device variants take device pointers and a hipStream_t (NULL = default
 * stream) and return after the stream work completes. */
nsfps_status nsfps_gather_points(const float *xyz, uint64_t n, const int32_t *idx, uint64_t m,
                                 float *out);
nsfps_status nsfps_gather_points_device(const float *d_xyz, uint64_t n, const int32_t *d_idx,
                                        uint64_t m, float *d_out, void *stream);
nsfps_status nsfps_ball_query(const float *xyz, uint64_t n, const float *centers, uint64_t m,
                              float radius, uint32_t nsample, int32_t *out);
nsfps_status nsfps_ball_query_device(const float *d_xyz, uint64_t n, const float *d_centers,
                                     uint64_t m, float radius, uint32_t nsample, int32_t *d_out,
                                     void *stream);

/* Measurements of the last compute call made on this thread. */
nsfps_status nsfps_get_stats(nsfps_stats *stats);

/* Phase clocks and work counters of the single-workgroup sampling loop of the
 * last call on this thread (cloud 0), recorded only when the environment
 * variable NSFPS_PROFILE is set (all zero otherwise).  Words 0-8: s_memtime
 * cycles spent between the loop's barriers (0 cube, 1 cell enumeration + scan,
 * 2 flatten, 3 fast phase A: candidate + sibling loads, 4 fast phase B,
 * 5 fast phase C / slow rounds, 6 slow level-1 rebuild, 7 level 2, 8 root);
 * 16 iterations, 17 fast iterations, 18 cube cells, 19 candidate leaves,
 * 20 dirty level-1 nodes on fast iterations, 21 elapsed s_memrealtime ticks
 * (100 MHz).  No counterpart in the reference (it has no instrumentation). */
nsfps_status nsfps_get_loop_profile(uint64_t *words, uint32_t nwords);

/* Releases the cached device workspace of the calling process, and the pinned
 * host buffer that host-buffer inputs are staged through. */
void nsfps_release_workspace(void);

#ifdef __cplusplus
}
#endif

#endif
