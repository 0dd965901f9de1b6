// Host library behind the C ABI (include/nsfps.h): range derivation,
// validation, device workspace, build orchestration and the sampling launch.
//
// Reference interfaces mirrored (paths relative to the reference tree):
//   range derivation   src/yuezu_fps.cpp:7-161
//   compute_bbox       src/yuezu_fps.cpp:643-670
//   yuezu_fps guards   src/yuezu_fps.cpp:676-688 (empty, n_samples >= N)
#include "nsfps.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include <unistd.h>

#include "nsfps_internal.h"
#include "nsfps_launch.h"

namespace nsfps {
namespace {

constexpr float kBoundaryEps = 1e-6f;  // BOUNDARY_EPS, src/yuezu_fps.h:43-45

thread_local std::string g_err;
thread_local nsfps_stats g_stats;
thread_local uint64_t g_prof[kProfWords];

nsfps_status fail(nsfps_status s, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return s;
}

// ----------------------------------------------------- failure injection
//
// NSFPS_INJECT=<kind>:<n> makes the n-th HIP operation of that kind in a
// call fail inside the library, without reaching the runtime: kind is alloc
// (device or pinned allocation, reported as out of memory), launch (a kernel
// launch or kernel load), copy (a memory copy), sync (a wait for a stream or
// event) or any.  Every entry point reads the variable when it starts, so
// each call gets its own countdown and a call after the variable is removed
// runs normally.  The error paths this reaches (status, message, the
// workspace left usable, the stream drained) are tested on the GPU.
enum InjectKind : int { kInjNone = 0, kInjAlloc, kInjLaunch, kInjCopy, kInjSync, kInjAny };
thread_local int g_inj_kind = kInjNone;
thread_local uint64_t g_inj_left = 0;

void arm_injection() {
  g_inj_kind = kInjNone;
  const char *e = getenv("NSFPS_INJECT");
  if (!e || !*e) return;
  static const char *const names[] = {"", "alloc", "launch", "copy", "sync", "any"};
  const char *colon = strchr(e, ':');
  const size_t len = colon ? (size_t)(colon - e) : strlen(e);
  for (int k = kInjAlloc; k <= kInjAny; ++k)
    if (strlen(names[k]) == len && strncmp(e, names[k], len) == 0) g_inj_kind = k;
  const unsigned long long n = colon ? strtoull(colon + 1, nullptr, 10) : 1ull;
  g_inj_left = n ? n : 1;
}

// The kind of HIP operation an expression performs, from its text.
int op_kind(const char *expr) {
  const auto starts = [&](const char *p) { return strncmp(expr, p, strlen(p)) == 0; };
  if (starts("hipMalloc") || starts("hipHostMalloc")) return kInjAlloc;
  if (starts("launch_") || starts("preload_")) return kInjLaunch;
  if (starts("hipMemcpy")) return kInjCopy;
  if (starts("hipStreamSynchronize") || starts("hipEventSynchronize")) return kInjSync;
  return kInjAny;  // other runtime calls fail only under "any"
}

// hipSuccess, or the injected failure when this operation is the one armed.
hipError_t injected(int kind) {
  if (g_inj_kind == kInjNone || (g_inj_kind != kInjAny && g_inj_kind != kind)) return hipSuccess;
  if (--g_inj_left) return hipSuccess;
  g_inj_kind = kInjNone;
  return kind == kInjAlloc ? hipErrorOutOfMemory : hipErrorLaunchFailure;
}

#define HIP_TRY(expr)                                                                        \
  do {                                                                                       \
    hipError_t e_ = g_inj_kind ? injected(op_kind(#expr)) : hipSuccess;                      \
    const bool inj_ = e_ != hipSuccess;                                                      \
    if (!inj_) {                                                                             \
      e_ = (expr);                                                                           \
    }                                                                                        \
    if (e_ != hipSuccess)                                                                    \
      return fail(e_ == hipErrorOutOfMemory ? NSFPS_ENOMEM : NSFPS_EDEVICE, "%s: %s (%s:%d)", \
                  #expr, inj_ ? "injected failure (NSFPS_INJECT)" : hipGetErrorString(e_),   \
                  __FILE__, __LINE__);                                                       \
  } while (0)

// ---------------------------------------------------------------- range ----

uint32_t calc_bits(uint32_t blocks) {  // _calc_bits, src/yuezu_fps.cpp:45-50
  uint32_t bits = 0;
  while (bits < 32 && (1u << bits) < blocks) ++bits;
  return bits ? bits : 1;
}

struct HostRange {
  nsfps_range prim;
  nsfps_range_info info;
  std::vector<uint32_t> lut[3];
  RangeDev dev;
};

nsfps_status check_range(const nsfps_range &r) {
  const float b[6] = {r.min_x, r.max_x, r.min_y, r.max_y, r.min_z, r.max_z};
  for (float v : b)
    if (!std::isfinite(v)) return fail(NSFPS_EINVAL, "range bounds must be finite");
  if (!(r.max_x > r.min_x) || !(r.max_y > r.min_y) || !(r.max_z > r.min_z))
    return fail(NSFPS_EINVAL, "range must satisfy max > min on every axis");
  const uint32_t bl[3] = {r.x_blocks, r.y_blocks, r.z_blocks};
  for (uint32_t v : bl) {
    if (v == 0) return fail(NSFPS_EINVAL, "block counts must be >= 1");
    if (v > 1024)
      return fail(NSFPS_EUNSUPPORTED,
                  "block counts above 1024 per axis are not supported (a cell's coordinates are "
                  "packed 10 bits per axis)");
  }
  return NSFPS_OK;
}

// Cube half-width of get_morton_codes_in_range on one axis (src/yuezu_fps.cpp:
// 564-570), (int)ceilf(sqrtf(D) / block_size), clipped to blocks - 1 (cells
// beyond the grid are skipped, :583-589).  IEEE fp32 on the host, exactly as
// the device's cube_half (correctly rounded sqrtf and division).
uint32_t cube_half_host(float D, float bs, uint32_t blocks) {
  const float rad = sqrtf(D < 0.0f ? 0.0f : D);
  const float f = ceilf(rad / bs);
  const uint32_t h = !(f < (float)blocks) ? blocks : (uint32_t)f;
  return h < blocks - 1 ? h : blocks - 1;
}

// Smallest D >= 0 whose half-width is at least k1 (INFINITY when none is).
// The half-width is monotone in D (sqrtf, division by a positive value and
// ceilf are monotone), and non-negative floats order like their bit
// patterns, so the answer is the first bit pattern where the predicate
// turns true.  It lies within a few ulps of (k1 - 1 ... k1) * bs squared:
// the walk starts at the estimate and steps one ulp at a time, checking the
// predicate on both sides of the boundary it stops at; a binary search over
// the bits settles the rare case the walk does not (the same answer: the
// predicate is monotone).
float cube_threshold(float bs, uint32_t blocks, uint32_t k1) {
  if (k1 > blocks - 1) return INFINITY;
  auto as_float = [](uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
  };
  auto as_bits = [](float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
  };
  auto at_least = [&](uint32_t u) { return cube_half_host(as_float(u), bs, blocks) >= k1; };
  const float est = ((float)(k1 - 1) * bs) * ((float)(k1 - 1) * bs);
  if (std::isfinite(est) && est >= 0.0f) {
    uint32_t u = as_bits(est);
    constexpr int kWalk = 64;
    bool found = false;
    if (at_least(u)) {
      for (int i = 0; i < kWalk; ++i) {
        if (u == 0 || !at_least(u - 1)) {
          found = true;
          break;
        }
        --u;
      }
    } else {
      for (int i = 0; i < kWalk && u < 0x7f800000u; ++i) {
        ++u;
        if (at_least(u)) {
          found = true;
          break;
        }
      }
    }
    if (found) return as_float(u);
  }
  uint32_t lo = 0, hi = 0x7f800000u;  // +inf: half-width blocks - 1 >= k1
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (at_least(mid)) hi = mid;
    else lo = mid + 1;
  }
  return as_float(lo);
}

// The make_range fields that depend on the block counts alone
// (src/yuezu_fps.cpp:45-97, 136-161): bits, Morton bit positions and LUTs,
// bucket count, and how many cells a bucket holds.
void derive_blocks(const uint32_t bl[3], HostRange &h) {
  uint32_t tb = 0;
  for (int a = 0; a < 3; ++a) {
    h.info.bits[a] = calc_bits(bl[a]);
    tb += h.info.bits[a];
  }
  h.info.total_bits = tb;
  h.info.total_blocks = (uint64_t)bl[0] * bl[1] * bl[2];
  // bit positions: min(bits) rounds of x,y,z, then x,y,z where present
  uint32_t common = std::min({h.info.bits[0], h.info.bits[1], h.info.bits[2]});
  uint32_t maxb = std::max({h.info.bits[0], h.info.bits[1], h.info.bits[2]});
  std::vector<uint32_t> pos[3];
  uint32_t bit = 0;
  for (uint32_t i = 0; i < common; ++i)
    for (int a = 0; a < 3; ++a) pos[a].push_back(bit++);
  for (uint32_t i = common; i < maxb; ++i)
    for (int a = 0; a < 3; ++a)
      if (i < h.info.bits[a]) pos[a].push_back(bit++);
  for (int a = 0; a < 3; ++a) {
    uint32_t count = 1u << h.info.bits[a];
    h.lut[a].assign(count, 0);
    for (uint32_t v = 0; v < count; ++v) {
      uint32_t code = 0;
      for (uint32_t k = 0; k < h.info.bits[a]; ++k)
        if (v & (1u << k)) code |= 1u << pos[a][k];
      h.lut[a][v] = code;
    }
  }
  RangeDev &d = h.dev;
  bool bij = true;
  uint32_t off = 0;
  for (int a = 0; a < 3; ++a) {
    d.blocks[a] = bl[a];
    d.lut_off[a] = off;
    off += 1u << h.info.bits[a];
    if (bl[a] != (1u << h.info.bits[a])) bij = false;  // not a power of two, or 1
  }
  d.lut_total = off;
  d.T = (uint32_t)h.info.total_blocks;
  d.bijective = bij ? 1u : 0u;
  // cells per bucket: codes b + jT below 2^cbits, so at most ceil(2^cbits / T)
  // (< 8: each axis has fewer than twice its blocks in codes, or exactly twice
  // for one block); counted exactly over the cells when there are few
  d.cbits = tb;
  for (int a = 0; a < 3; ++a) d.cmask[a] = h.lut[a].back();
  if (bij) {
    d.na = 1;
  } else {
    const uint64_t codes = 1ull << tb, T = h.info.total_blocks;
    uint32_t na = (uint32_t)std::min<uint64_t>((codes + T - 1) / T, kMaxAlias);
    if (T <= 65536) {
      std::vector<uint8_t> cnt(T, 0);
      uint32_t mx = 1;
      for (uint32_t z = 0; z < bl[2]; ++z)
        for (uint32_t y = 0; y < bl[1]; ++y)
          for (uint32_t x = 0; x < bl[0]; ++x) {
            const uint32_t code = h.lut[0][x] | h.lut[1][y] | h.lut[2][z];
            mx = std::max<uint32_t>(mx, ++cnt[code % T]);
          }
      na = std::min(na, mx);
    }
    d.na = na;
  }
}

// The fp32 fields of make_range (src/yuezu_fps.cpp:136-161): block size,
// inv_bs = 1.0f / ((max - min) / blocks), the clamp bound max - 1e-6, and
// the cube half-width thresholds.  The block counts are derived already.
void derive_floats(const nsfps_range &r, HostRange &h) {
  h.prim = r;
  const float mn[3] = {r.min_x, r.min_y, r.min_z};
  const float mx[3] = {r.max_x, r.max_y, r.max_z};
  RangeDev &d = h.dev;
  for (int a = 0; a < 3; ++a) {
    h.info.inv_bs[a] = 1.0f / ((mx[a] - mn[a]) / (float)d.blocks[a]);
    h.info.block_size[a] = (mx[a] - mn[a]) / (float)d.blocks[a];
    d.mn[a] = mn[a];
    d.hiclamp[a] = mx[a] - kBoundaryEps;
    d.inv_bs[a] = h.info.inv_bs[a];
    d.bsize[a] = h.info.block_size[a];
  }
  static_assert(kCubeThr == NSFPS_CUBE_THRESHOLDS, "threshold count");
  for (int a = 0; a < 3; ++a)
    for (uint32_t k = 0; k < kCubeThr; ++k) {
      const float t = cube_threshold(h.info.block_size[a], d.blocks[a], k + 1);
      h.info.cube_thr[a][k] = t;
      d.cube_thr[a][k] = t;
    }
}

// make_range derivation (src/yuezu_fps.cpp:136-161) plus the LUTs of
// _compute_bit_positions/_generate_morton_lut (:52-97).
void derive(const nsfps_range &r, HostRange &h) {
  const uint32_t bl[3] = {r.x_blocks, r.y_blocks, r.z_blocks};
  derive_blocks(bl, h);
  derive_floats(r, h);
}

// compute_bbox (src/yuezu_fps.cpp:648-670) keeps, per axis, the running
// (v < mn ? v : mn) and (mx < v ? v : mx) from point 0.  Here points
// [lo, hi) run through 24 independent lanes (eight points a step; lane k
// holds axis k % 3), every lane started from point 0 of the cloud, and the
// lanes are folded with the same selects.  Minimum and maximum of the finite
// values do not depend on the order, a NaN point 0 stays NaN and any later
// NaN is skipped, exactly as in the single running pass; so pieces of one
// cloud may run on different threads and fold in any order.
void bounds_piece(const float *xyz, uint64_t lo, uint64_t hi, const float *p0, float *mn3,
                  float *mx3) {
  constexpr int kL = 24;
  float mn[kL], mx[kL];
  for (int k = 0; k < kL; ++k) mn[k] = mx[k] = p0[k % 3];
  const float *p = xyz + 3 * lo;
  const uint64_t nf = 3 * (hi - lo);
  uint64_t j = 0;
  for (; j + kL <= nf; j += kL)
    for (int k = 0; k < kL; ++k) {
      const float v = p[j + k];
      mn[k] = v < mn[k] ? v : mn[k];
      mx[k] = mx[k] < v ? v : mx[k];
    }
  for (; j < nf; ++j) {
    const int k = (int)(j % 3);
    const float v = p[j];
    mn[k] = v < mn[k] ? v : mn[k];
    mx[k] = mx[k] < v ? v : mx[k];
  }
  for (int a = 0; a < 3; ++a) {
    float m = mn[a], M = mx[a];
    for (int k = a + 3; k < kL; k += 3) {
      m = mn[k] < m ? mn[k] : m;
      M = M < mx[k] ? mx[k] : M;
    }
    mn3[a] = m;
    mx3[a] = M;
  }
}

// Worker threads for host-side scans, started on first need and kept until
// the process ends (starting threads on every call cost about as much as the
// scan they split).  run() splits f(0 .. n - 1) statically between the caller
// (q % parts == 0) and every worker (q % parts == its id), and returns once
// each worker has checked in for that call.  Calls to run() are serialised.
// A process forked from the owner has none of its threads (and maybe a lock
// held at the fork): there run() works alone, touching no pool state.  The
// pool is never destroyed, so no thread is joined at exit.
class HostPool {
 public:
  HostPool() : pid_(getpid()) {}
  void run(uint64_t n, unsigned want, const std::function<void(uint64_t)> &f) {
    if (getpid() != pid_) {
      for (uint64_t q = 0; q < n; ++q) f(q);
      return;
    }
    std::lock_guard<std::mutex> one(run_mu_);
    std::unique_lock<std::mutex> l(m_);
    while (th_.size() + 1 < want) {
      try {  // a worker that cannot be started leaves its share to the others
        const unsigned id = (unsigned)th_.size() + 1;
        th_.emplace_back([this, id, g = gen_] { loop(id, g); });
      } catch (...) {
        break;
      }
    }
    const unsigned k = (unsigned)th_.size();
    job_ = &f;
    n_ = n;
    parts_ = k + 1;
    finished_ = 0;
    ++gen_;
    l.unlock();
    go_.notify_all();
    for (uint64_t q = 0; q < n; q += k + 1) f(q);
    l.lock();
    done_.wait(l, [&] { return finished_ == k; });
    job_ = nullptr;
  }

 private:
  void loop(unsigned id, uint64_t seen) {
    std::unique_lock<std::mutex> l(m_);
    for (;;) {
      go_.wait(l, [&] { return gen_ != seen; });
      seen = gen_;
      const std::function<void(uint64_t)> *f = job_;
      const uint64_t n = n_, step = parts_;
      l.unlock();
      for (uint64_t q = id; q < n; q += step) (*f)(q);
      l.lock();
      ++finished_;
      done_.notify_one();
    }
  }
  const pid_t pid_;
  std::mutex run_mu_, m_;
  std::condition_variable go_, done_;
  std::vector<std::thread> th_;
  const std::function<void(uint64_t)> *job_ = nullptr;
  uint64_t n_ = 0, parts_ = 1, gen_ = 0;
  unsigned finished_ = 0;
};

HostPool &host_pool() {
  static HostPool *const pool = new HostPool;  // never destroyed (see above)
  return *pool;
}

// compute_bbox of `count` clouds of n points each (ranges[b] gets cloud b's
// bounds +- 1e-6; block counts untouched).  Pieces of at least kPiece points
// are spread over up to 16 threads of the host pool when there is enough
// work.
void bboxes(const float *xyz, uint64_t count, uint64_t n, nsfps_range *ranges) {
  constexpr uint64_t kPiece = 1u << 16;
  const uint64_t per = n ? (n + kPiece - 1) / kPiece : 0;  // pieces per cloud
  const uint64_t pieces = count * per;
  std::vector<float> part(6 * std::max<uint64_t>(pieces, 1));
  auto run = [&](uint64_t q) {
    const uint64_t b = q / per, k = q % per;
    const float *c = xyz + b * n * 3;
    bounds_piece(c, k * kPiece, std::min(n, (k + 1) * kPiece), c, &part[6 * q], &part[6 * q + 3]);
  };
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const uint64_t nt = std::min<uint64_t>(hw, pieces);
  if (nt <= 1 || count * n < 4 * kPiece) {
    for (uint64_t q = 0; q < pieces; ++q) run(q);
  } else {
    host_pool().run(pieces, (unsigned)nt, run);
  }
  for (uint64_t b = 0; b < count; ++b) {
    nsfps_range &r = ranges[b];
    if (n == 0) {
      r.min_x = 0; r.max_x = 1; r.min_y = 0; r.max_y = 1; r.min_z = 0; r.max_z = 1;
      r.x_blocks = r.y_blocks = r.z_blocks = 1;
      continue;
    }
    float mn[3], mx[3];
    for (int a = 0; a < 3; ++a) {
      mn[a] = part[6 * b * per + a];
      mx[a] = part[6 * b * per + 3 + a];
      for (uint64_t k = 1; k < per; ++k) {
        const float lo = part[6 * (b * per + k) + a], hi = part[6 * (b * per + k) + 3 + a];
        mn[a] = lo < mn[a] ? lo : mn[a];
        mx[a] = mx[a] < hi ? hi : mx[a];
      }
    }
    r.min_x = mn[0] - kBoundaryEps; r.max_x = mx[0] + kBoundaryEps;
    r.min_y = mn[1] - kBoundaryEps; r.max_y = mx[1] + kBoundaryEps;
    r.min_z = mn[2] - kBoundaryEps; r.max_z = mx[2] + kBoundaryEps;
  }
}

void bbox_of(const float *xyz, uint64_t n, nsfps_range &r) { bboxes(xyz, 1, n, &r); }

// ------------------------------------------------------------ workspace ----

// Pinned host memory that host-buffer inputs pass through on their way to
// the device: allocated once, grown when a call needs more, kept until the
// process ends.  `done` is recorded after the last copy out of it.
struct PinStage {
  char *p = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
};

// Streams of one call's sampling rounds, at most.  The runtime gives a
// process 4 hardware queues by default: 4 streams of rounds (with the
// caller's own) shared them, and 64 clouds of 16,384 points took 3.0 ms per
// call against 1.8 with 2 or 3.
constexpr uint32_t kMaxStreams = 3;
struct Arena {
  char *base = nullptr;
  size_t cap = 0;
  hipStream_t stream = nullptr;
  // the other groups of a call's clouds during the sampling rounds, and the
  // events that order them after the build and before each status read
  hipStream_t stream2[kMaxStreams - 1] = {};
  hipEvent_t fork = nullptr, join[kMaxStreams - 1] = {};
  hipEvent_t ev[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  int device = -1;
  PinStage pin;
  char *rb = nullptr;  // pinned buffer of the small read-backs the host waits for
  size_t rb_cap = 0;
};

std::mutex g_mu;
Arena g_arena[16];

// Bump layout over an arena; a null base measures the size.
struct Bump {
  char *base;
  size_t off = 0;
  explicit Bump(char *b) : base(b) {}
  template <class T>
  T *take(size_t count) {
    off = (off + 255) & ~size_t(255);
    T *p = base ? reinterpret_cast<T *>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

// Once per device (the current one), before its first call: the library's
// kernels are loaded, so that loading them does not fall inside a call.
bool g_kernels_loaded[16];

nsfps_status prepare_device(int dev) {
  if (dev < 0 || dev >= 16) return fail(NSFPS_EDEVICE, "device ordinal %d out of range", dev);
  if (g_kernels_loaded[dev]) return NSFPS_OK;
  HIP_TRY(preload_build_kernels());
  HIP_TRY(preload_runs_kernels());
  HIP_TRY(preload_group_kernels());
  g_kernels_loaded[dev] = true;
  return NSFPS_OK;
}

nsfps_status arena_for_device(Arena **out) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return fail(NSFPS_EDEVICE, "no HIP device available (nsfps has no CPU path)");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= 16) return fail(NSFPS_EDEVICE, "device ordinal %d out of range", dev);
  nsfps_status rc = prepare_device(dev);
  if (rc) return rc;
  Arena &a = g_arena[dev];
  if (!a.stream) {
    HIP_TRY(hipStreamCreateWithFlags(&a.stream, hipStreamNonBlocking));
    for (auto &e : a.ev) HIP_TRY(hipEventCreate(&e));
    a.device = dev;
    // The runtime sets a copy path up on its first use in a process: the
    // first staged upload of 120 KB held the host 6-7.6 ms inside the first
    // call's build.  One copy each way of kWarm bytes here, through the
    // pinned read-back buffer, moves that into the device's set-up.  A
    // failure only leaves the set-up to the first call.
    constexpr size_t kWarm = size_t(256) << 10;
    if (!a.rb && hipHostMalloc(reinterpret_cast<void **>(&a.rb), kWarm, hipHostMallocDefault) ==
                     hipSuccess)
      a.rb_cap = kWarm;
    void *warm = nullptr;
    if (a.rb && a.rb_cap >= kWarm && hipMalloc(&warm, kWarm) == hipSuccess) {
      if (hipMemcpyAsync(warm, a.rb, kWarm, hipMemcpyHostToDevice, a.stream) == hipSuccess &&
          hipMemcpyAsync(a.rb, warm, kWarm, hipMemcpyDeviceToHost, a.stream) == hipSuccess)
        (void)hipStreamSynchronize(a.stream);
      (void)hipFree(warm);
    }
    (void)hipGetLastError();
  }
  *out = &a;
  return NSFPS_OK;
}

nsfps_status arena_reserve(Arena &a, size_t bytes) {
  if (bytes <= a.cap) return NSFPS_OK;
  if (a.base) {
    HIP_TRY(hipStreamSynchronize(a.stream));
    HIP_TRY(hipFree(a.base));
    a.base = nullptr;
    a.cap = 0;
  }
  size_t want = bytes + bytes / 8 + (1u << 20);
  const hipError_t inj = injected(kInjAlloc);
  hipError_t e = inj != hipSuccess ? inj : hipMalloc(&a.base, want);
  if (e != hipSuccess) {
    a.base = nullptr;
    return fail(NSFPS_ENOMEM, "hipMalloc(%zu) failed: %s", want,
                inj != hipSuccess ? "injected failure (NSFPS_INJECT)" : hipGetErrorString(e));
  }
  a.cap = want;
  return NSFPS_OK;
}

// Host-buffer inputs to the device through the arena's pinned stage, in
// chunks: the CPU copies a chunk into pinned memory and the DMA of each
// chunk overlaps the copy of the next.  A pageable source would instead be
// pinned by the runtime on every new buffer (measured on the MI355X box: the
// upload of a fresh 12.6 MB array cost 4.4 ms, of one whose pages the
// runtime had cached 0.37 ms; pinned, 0.23 ms).  Without pinned memory the
// copies are made from the source as it is.
struct HostUp {
  void *dst;
  const void *src;
  size_t bytes;
};

// Host copies of at least this many bytes are split over the host pool.
constexpr size_t kPoolBytes = size_t(4) << 20, kPoolDownBytes = size_t(256) << 10;

nsfps_status upload_host(const std::vector<HostUp> &ups, hipStream_t st) {
  size_t total = 0;
  for (const auto &u : ups) total += (u.bytes + 255) & ~size_t(255);
  if (total == 0) return NSFPS_OK;
  Arena *ap = nullptr;
  nsfps_status rc = arena_for_device(&ap);
  if (rc) return rc;
  PinStage &ps = ap->pin;
  if (ps.pending) {  // an earlier call's copies may still read the stage
    HIP_TRY(hipEventSynchronize(ps.done));
    ps.pending = false;
  }
  if (!ps.done) HIP_TRY(hipEventCreateWithFlags(&ps.done, hipEventDisableTiming));
  if (total > ps.cap) {
    if (ps.p) HIP_TRY(hipHostFree(ps.p));
    ps.p = nullptr;
    ps.cap = 0;
    const size_t want = total + total / 8 + (1u << 20);
    if (injected(kInjAlloc) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&ps.p), want, hipHostMallocDefault) != hipSuccess) {
      ps.p = nullptr;
      (void)hipGetLastError();
      for (const auto &u : ups)
        HIP_TRY(hipMemcpyAsync(u.dst, u.src, u.bytes, hipMemcpyHostToDevice, st));
      return NSFPS_OK;
    }
    ps.cap = want;
  }
  // Up to kPoolBytes: 2 MB chunks, each copied into the stage and its DMA
  // enqueued right after, so a transfer overlaps the next chunk's copy.
  // Above: the host pool's threads copy 1 MB slices into the stage (one
  // thread copies at about 20 GB/s, less than the link), then one DMA per
  // input.  A DMA per slice, enqueued by the workers, spread the transfers
  // out: each hipMemcpyAsync held its thread 20-190 us, and 12.6 MB took
  // 0.65 ms on the stream for 0.3 ms of transfers.
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (total < kPoolBytes || hw == 1) {
    constexpr size_t kChunk = size_t(2) << 20;
    size_t at = 0;
    for (const auto &u : ups) {
      for (size_t off = 0; off < u.bytes; off += kChunk) {
        const size_t n = std::min(kChunk, u.bytes - off);
        memcpy(ps.p + at + off, static_cast<const char *>(u.src) + off, n);
        HIP_TRY(hipMemcpyAsync(static_cast<char *>(u.dst) + off, ps.p + at + off, n,
                               hipMemcpyHostToDevice, st));
      }
      at += (u.bytes + 255) & ~size_t(255);
    }
  } else {
    constexpr size_t kSlice = size_t(1) << 20;
    struct Slice {
      char *stage;
      const char *src;
      size_t n;
    };
    std::vector<Slice> sl;
    size_t at = 0;
    for (const auto &u : ups) {
      for (size_t off = 0; off < u.bytes; off += kSlice)
        sl.push_back(Slice{ps.p + at + off, static_cast<const char *>(u.src) + off,
                           std::min(kSlice, u.bytes - off)});
      at += (u.bytes + 255) & ~size_t(255);
    }
    host_pool().run(sl.size(), (unsigned)std::min<size_t>(hw, sl.size()),
                    [&](uint64_t q) { memcpy(sl[q].stage, sl[q].src, sl[q].n); });
    at = 0;
    for (const auto &u : ups) {
      HIP_TRY(hipMemcpyAsync(u.dst, ps.p + at, u.bytes, hipMemcpyHostToDevice, st));
      at += (u.bytes + 255) & ~size_t(255);
    }
  }
  HIP_TRY(hipEventRecord(ps.done, st));
  ps.pending = true;
  return NSFPS_OK;
}

// A call's result from the device into the caller's buffer.  From
// kPoolBytes on it goes through the pinned stage (when one of that size
// exists): one DMA and a wait, then the host pool's threads copy it out.  The
// runtime's own copy into a fresh pageable array faults the array's pages in
// one by one: 0.53 ms for 1 MB, of which the transfer took 23 us.  Smaller
// results are copied directly; the caller waits for the stream either way.
nsfps_status download_host(void *dst, const void *src, size_t bytes, hipStream_t st) {
  Arena *ap = nullptr;
  nsfps_status rc = arena_for_device(&ap);
  if (rc) return rc;
  PinStage &ps = ap->pin;
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (bytes < kPoolDownBytes || hw == 1 || !ps.p || ps.cap < bytes) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
    return NSFPS_OK;
  }
  if (ps.pending) HIP_TRY(hipStreamWaitEvent(st, ps.done, 0));  // uploads read the stage first
  HIP_TRY(hipMemcpyAsync(ps.p, src, bytes, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  ps.pending = false;
  const size_t slice = std::max<size_t>(size_t(64) << 10, (bytes / hw + 4095) & ~size_t(4095));
  const uint64_t parts = (bytes + slice - 1) / slice;
  host_pool().run(parts, (unsigned)std::min<uint64_t>(hw, parts), [&](uint64_t q) {
    const size_t off = q * slice;
    memcpy(static_cast<char *>(dst) + off, ps.p + off, std::min(slice, bytes - off));
  });
  return NSFPS_OK;
}

// The allocation-free entry point's call: nothing may be allocated, so the
// read-backs below take their pinned buffer only if an earlier call made it.
bool g_call_no_alloc = false;

// A small read-back the host waits for (build stats, the clouds' statuses):
// one DMA into a pinned buffer kept per device, then the wait.  A pageable
// destination made the runtime stage the copy, and the host waited 15-40 us
// longer per read-back.  Without the buffer the copy is made directly.
nsfps_status readback(void *dst, const void *src, size_t bytes, hipStream_t st) {
  Arena *ap = nullptr;
  if (g_call_no_alloc) {  // the arena as it is: nothing is created or grown
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev >= 0 && dev < 16) ap = &g_arena[dev];
  } else {
    const nsfps_status rc = arena_for_device(&ap);
    if (rc) return rc;
  }
  if (ap && ap->rb_cap < bytes && !g_call_no_alloc) {
    if (ap->rb) HIP_TRY(hipHostFree(ap->rb));
    ap->rb = nullptr;
    ap->rb_cap = 0;
    const size_t want = std::max<size_t>(bytes, size_t(64) << 10);
    if (injected(kInjAlloc) == hipSuccess &&
        hipHostMalloc(reinterpret_cast<void **>(&ap->rb), want, hipHostMallocDefault) ==
            hipSuccess) {
      ap->rb_cap = want;
    } else {
      ap->rb = nullptr;
      (void)hipGetLastError();
    }
  }
  if (!ap || ap->rb_cap < bytes) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    return NSFPS_OK;
  }
  HIP_TRY(hipMemcpyAsync(ap->rb, src, bytes, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  std::memcpy(dst, ap->rb, bytes);
  return NSFPS_OK;
}

// ------------------------------------------------------------ one cloud ----

// Per-cloud words the host polls between batches of rounds, contiguous over
// the clouds of a call so that one copy reads them all.
struct CloudStatus {
  uint32_t done, iter;
  RunState rs;
};

struct CloudPlan {
  uint32_t n = 0, m = 0;
  HostRange rng;
  const float *d_xyz_in = nullptr;  // device input, or null to stage h_xyz
  const float *h_xyz = nullptr;
  int32_t *d_out_user = nullptr;  // the caller's device buffer for the samples, or null
  CloudDev dev{};
  uint32_t slots_ub = 0, leaves_ub = 0, l1_ub = 0;
  // build-time buffers
  float *d_xyz_stage = nullptr;
  uint32_t *d_lut = nullptr, *d_counts = nullptr, *d_lc = nullptr;
  uint32_t *d_small = nullptr;  // kStatWords: [0] non-finite flag, [1] max occupancy, [2] phys0,
                                //   [3] dense leaves, [4] occupied buckets
  uint32_t occupied = 0;        // buckets holding points
  uint2 *d_cell_info = nullptr;
  uint32_t *d_bucket = nullptr, *d_fine = nullptr;  // per point: bucket, sub-cell code
  uint64_t cap = 0;                // slots per bucket in the padded layout
  bool tree = false;               // sampled by the tree engine (its loop holds level 1 in LDS)
  // the range is compute_bbox of the points with rng's block counts, found on
  // the device by the build (rng holds the block-count fields until then)
  bool bbox_dev = false;
  std::vector<uint32_t> lut_host;  // source of an asynchronous copy: lives until the sync
};

struct Scratch {
  uint32_t *kA, *kB, *vA, *vB, *vC, *hist, *scan;
};

int key_bits_for(uint32_t T) {
  int b = 0;
  while (b < 32 && (1ull << b) < (uint64_t)T) ++b;
  return b;
}

// Padded layout (slot = bucket * cap + j) is used when the largest bucket
// rounded up to whole leaves, times the bucket count, stays within this many
// slots: cell -> leaf becomes arithmetic, no table lookup per iteration.
uint64_t padded_slot_limit(uint32_t n) { return std::max<uint64_t>(4ull * n, 65536ull); }

// Lays out the persistent buffers of one cloud (upper bounds: the padded /
// dense decision is made on the device data during the build).
void layout_cloud(Bump &bp, CloudPlan &p) {
  const uint32_t n = p.n, T = p.rng.dev.T;
  uint64_t slots = std::max<uint64_t>(n, padded_slot_limit(n));
  uint64_t leaves = std::max<uint64_t>(n / kLeaf + 1 + std::min<uint32_t>(T, n), slots / kLeaf);
  p.slots_ub = (uint32_t)slots;
  p.leaves_ub = (uint32_t)leaves;
  p.l1_ub = (uint32_t)((leaves + kFan - 1) / kFan);
  CloudDev &c = p.dev;
  p.d_lut = bp.take<uint32_t>(p.rng.dev.lut_total + 16);
  c.P4 = bp.take<float4>(slots);
  c.RO = bp.take<uint2>(slots);
  c.R = bp.take<uint32_t>(slots);
  p.d_lc = bp.take<uint32_t>((size_t)T + 1);
  p.d_cell_info = bp.take<uint2>((size_t)T + 1);
  c.cell_info = p.d_cell_info;
  c.leaf_lo = bp.take<float4>(leaves);
  c.leaf_hi = bp.take<float4>(leaves);
  c.leaf_sc = bp.take<uint2>(leaves);
  c.leaf_cell = bp.take<uint32_t>(leaves);
  c.leaf_al = bp.take<uint32_t>(leaves * p.rng.dev.na);
  c.leaf_cbox = bp.take<uint2>(leaves);
  c.leaf_key = bp.take<uint64_t>(leaves);
  c.leaf_pos = bp.take<float4>(leaves);
  c.l1_key = bp.take<uint64_t>(p.l1_ub);
  c.l1_part = bp.take<uint64_t>((size_t)p.l1_ub * kUpdateSplit);
  c.l1_pos = bp.take<float4>(p.l1_ub);
  c.l1_lo = bp.take<float4>(p.l1_ub);
  c.l1_hi = bp.take<float4>(p.l1_ub);
  c.l1_cbox = bp.take<uint2>(p.l1_ub);
  c.root_key = bp.take<uint64_t>(1);
  c.root_pos = bp.take<float4>(1);
  c.counter = bp.take<uint32_t>(1);
  c.prof = bp.take<uint64_t>(kProfWords);
  c.hist = bp.take<uint32_t>((size_t)kHists * kHistBins);
  c.pick_p = bp.take<float4>(kListCap);
  c.pick_c = bp.take<uint2>(kListCap);
  c.list_p = bp.take<float4>(kListCap);
  c.list_r = bp.take<uint2>(kListCap);
  c.list_c = bp.take<uint32_t>(kListCap);
  c.list_al = bp.take<uint32_t>((size_t)kListCap * p.rng.dev.na);
  c.lut = p.d_lut;
  c.n = n;
  c.m = p.m;
  c.r = p.rng.dev;
}

void layout_scratch(Bump &bp, uint32_t n, uint32_t tmax, Scratch &s) {
  s.kA = bp.take<uint32_t>(n);
  s.kB = bp.take<uint32_t>(n);
  s.vA = bp.take<uint32_t>(n);
  s.vB = bp.take<uint32_t>(n);
  s.vC = bp.take<uint32_t>(n);
  s.hist = bp.take<uint32_t>(radix_hist_len(n) + 16);
  s.scan = bp.take<uint32_t>(scan_tmp_len(std::max(radix_hist_len(n), tmax + 1)) + 16);
}

// LDS layout of the single-workgroup loop for one cloud: required regions,
// then the cell table (table mode) and level-1 boxes when they fit, then as
// many staging slots as the rest allows (at most 64).
LdsPlan plan_lds(const CloudDev &c) {
  LdsPlan pl{};
  uint32_t off = 0;
  auto take = [&](uint64_t bytes) {
    off = (off + 15u) & ~15u;
    uint32_t o = off;
    off += (uint32_t)bytes;
    return o;
  };
  const uint32_t nl1 = std::max<uint32_t>(c.nl1, 1);
  pl.l1k = take((uint64_t)nl1 * 8);
  pl.l1p = take((uint64_t)nl1 * 16);
  pl.l2k = take(64 * 8);
  pl.l2p = take(64 * 16);
  pl.lut = take((uint64_t)c.r.lut_total * 4);
  pl.cand = take((uint64_t)kCandCap * 12);
  pl.slot = take((uint64_t)nl1 * 4);
  pl.m1 = take(((nl1 + 31) / 32) * 4);
  pl.dl1 = take((uint64_t)nl1 * 4);
  pl.m2 = take(8);
  const uint32_t slot_bytes = kFan * (8 + 16) + 8;  // staging entries + candidate mask
  pl.ctab = kNone;
  if (!c.padded) {
    uint64_t need = ((uint64_t)c.r.T + 1) * 8;
    if (off + need + 16 + 8 * slot_bytes <= kLdsBudget) pl.ctab = take(need);
  }
  pl.l1lo = pl.l1hi = kNone;
  if (off + 2ull * nl1 * 16 + 32 + 4 * slot_bytes <= kLdsBudget) {
    pl.l1lo = take((uint64_t)nl1 * 16);
    pl.l1hi = take((uint64_t)nl1 * 16);
  }
  uint32_t room = kLdsBudget > off + 96 ? kLdsBudget - off - 96 : 0;
  pl.dcap = std::min<uint32_t>(64, room / slot_bytes);
  pl.cm = take((uint64_t)std::max<uint32_t>(pl.dcap, 1) * 8);
  pl.sk = take((uint64_t)pl.dcap * kFan * 8);
  pl.sp = take((uint64_t)pl.dcap * kFan * 16);
  pl.total = (off + 255u) & ~255u;
  return pl;
}

// Buffers of a call that every cloud gets a contiguous part of, so that one
// copy or fill serves all clouds: staged host input, bucket populations, the
// words read back after the first build phase ([0] non-finite flag, [1] the
// largest bucket, [2] the slot of input row 0, [3] dense leaves), per-point
// bucket and sub-cell codes.
struct CallBuffers {
  float *xyz_stage = nullptr;
  uint32_t *counts = nullptr, *small = nullptr, *bucket = nullptr, *fine = nullptr;
  // ranges found on the device: bounds as order-preserving integers (6 per
  // cloud), the ranges, and their bounds as floats (6 per cloud)
  uint32_t *ord = nullptr;
  RangeDev *drng = nullptr;
  float *dbounds = nullptr;
  BuildDev *bd = nullptr;  // per-cloud parameters of the many-cloud build steps
  int32_t *out = nullptr;  // every cloud's samples, m entries per cloud
  size_t n_total = 0, counts_total = 0;
};

void layout_call(Bump &bp, std::vector<CloudPlan> &plans, CallBuffers &cb) {
  size_t stage = 0;
  cb.n_total = cb.counts_total = 0;
  for (auto &p : plans) {
    if (p.h_xyz) stage += (size_t)p.n * 3;
    cb.n_total += p.n;
    cb.counts_total += (size_t)p.rng.dev.T + 1;
  }
  cb.xyz_stage = stage ? bp.take<float>(stage) : nullptr;
  cb.counts = bp.take<uint32_t>(cb.counts_total);
  // small, drng and dbounds one after another: the build reads them back
  // in one copy
  cb.small = bp.take<uint32_t>(kStatWords * plans.size());
  cb.drng = bp.take<RangeDev>(plans.size());
  cb.dbounds = bp.take<float>(6 * plans.size());
  cb.bucket = bp.take<uint32_t>(cb.n_total);
  cb.fine = bp.take<uint32_t>(cb.n_total);
  cb.bd = bp.take<BuildDev>(plans.size());
  cb.ord = bp.take<uint32_t>(6 * plans.size());
  // the clouds' outputs back to back, rows of m entries: one read-back
  size_t outs = 0;
  for (auto &p : plans) outs += p.m;
  cb.out = bp.take<int32_t>(outs);
  if (!bp.base) return;  // measuring: no buffer to hand out
  size_t o_stage = 0, o_n = 0, o_c = 0, o_out = 0;
  for (size_t i = 0; i < plans.size(); ++i) {
    CloudPlan &p = plans[i];
    if (p.h_xyz) {
      p.d_xyz_stage = cb.xyz_stage + o_stage;
      o_stage += (size_t)p.n * 3;
    }
    p.d_counts = cb.counts + o_c;
    o_c += (size_t)p.rng.dev.T + 1;
    p.d_small = cb.small + kStatWords * i;
    p.d_bucket = cb.bucket + o_n;
    p.d_fine = cb.fine + o_n;
    o_n += p.n;
    // the samples go to the caller's device buffer when there is one (no copy
    // after the sampling), else into the call's rows
    p.dev.out = p.d_out_user ? p.d_out_user : cb.out + o_out;
    o_out += p.m;
  }
}

// Clouds sorted together, cloud index above the bucket: every cloud has the
// same point count and the keys fit 32 bits with room for sub-cell bits.
bool sort_together(const std::vector<CloudPlan> &plans, int *cloud_bits, int *bucket_bits) {
  if (plans.size() < 2) return false;
  uint32_t tmax = 0;
  for (auto &p : plans) {
    if (p.n != plans[0].n) return false;
    tmax = std::max(tmax, p.rng.dev.T);
  }
  *cloud_bits = key_bits_for((uint32_t)plans.size());
  *bucket_bits = std::max(1, key_bits_for(tmax));
  return *cloud_bits + *bucket_bits <= 28 && (uint64_t)plans[0].n * plans.size() < (1ull << 31);
}

// Device build of the clouds of a call up to the initial trees.  The first
// phase (cell keys, bucket populations, their scans) runs for every cloud,
// then the stream is synchronised once and a few words per cloud decide each
// layout; then both sorts run (once for all clouds when they can be sorted
// together), and each cloud's slots, leaves and tree are built.
nsfps_status sort_logical(const uint32_t *bucket, uint32_t n_per, uint32_t nclouds,
                          int cloud_bits, int bucket_bits, const Scratch &s, hipStream_t st,
                          uint32_t **keys, uint32_t **lorig);

// sorted: the cloud is sorted by bucket here (its rows in *lorig, the sorted
// buckets in *keys) and the bucket populations are counted from that order,
// not by an atomic per point (contended where points crowd into few buckets).
nsfps_status build_phase1(CloudPlan &p, const CloudPlan *lut_of, const Scratch &s, hipStream_t st,
                          const RangeDev *d_range, bool sorted = false, uint32_t **keys = nullptr,
                          uint32_t **lorig = nullptr) {
  const uint32_t T = p.rng.dev.T;
  if (lut_of) {
    p.d_lut = lut_of->d_lut;  // the same bit positions: the same tables
    p.dev.lut = p.d_lut;
  } else {
    std::vector<uint32_t> &lut = p.lut_host;
    lut.clear();
    for (int a = 0; a < 3; ++a) lut.insert(lut.end(), p.rng.lut[a].begin(), p.rng.lut[a].end());
    HIP_TRY(hipMemcpyAsync(p.d_lut, lut.data(), lut.size() * 4, hipMemcpyHostToDevice, st));
  }
  const float *xyz = p.h_xyz ? p.d_xyz_stage : p.d_xyz_in;
  if (p.bbox_dev)  // the range is in device memory, found from the points' bounds
    HIP_TRY(launch_cell_keys_dr(xyz, p.n, d_range, p.d_lut, p.d_bucket, p.d_fine,
                                sorted ? nullptr : p.d_counts, p.d_small, st));
  else
    HIP_TRY(launch_cell_keys(xyz, p.n, p.rng.dev, p.d_lut, p.d_bucket, p.d_fine,
                             sorted ? nullptr : p.d_counts, p.d_small, st));
  if (sorted) {
    nsfps_status rc = sort_logical(p.d_bucket, p.n, 1, 0, std::max(1, key_bits_for(T)), s, st,
                                   keys, lorig);
    if (rc) return rc;
    HIP_TRY(launch_seg_counts(*keys, p.n, p.d_counts, st));
  }
  HIP_TRY(launch_leaf_counts(p.d_counts, T, p.d_lc, p.d_small + 1, p.d_small + 3, p.d_small + 4,
                             st));
  HIP_TRY(launch_scan(p.d_counts, T, s.scan, st));  // -> first dense position per bucket
  HIP_TRY(launch_scan(p.d_lc, T, s.scan, st));      // -> first leaf per bucket (dense)
  return NSFPS_OK;
}

// Leaves of the per-bucket layouts (a leaf holds points of one bucket):
// padded (slot = bucket * cap + j) when that stays within the slot limit,
// else dense.  hs: the words read back after the first build phase.
uint64_t bucket_leaves(const CloudPlan &p, const uint32_t *hs, bool *padded, uint64_t *cap) {
  const uint32_t n = p.n, T = p.rng.dev.T;
  const uint32_t maxocc = hs[1], dense_leaves = hs[3];
  *cap = (uint64_t)((maxocc + kLeaf - 1) / kLeaf) * kLeaf;
  const uint64_t padded_slots = *cap * T;
  *padded = getenv("NSFPS_NO_PADDED") == nullptr && *cap > 0 &&
            padded_slots <= padded_slot_limit(n) && padded_slots <= p.slots_ub;
  return *padded ? padded_slots / kLeaf : dense_leaves;
}

// Mixed leaves (runs of 64 slots of the logical order, possibly of several
// buckets) for every cloud of a call, or for none: when the runs engine
// samples them, every cloud's buckets have one cell, and the per-bucket
// layout would fill its leaves to less than a quarter on the whole (the
// update and gather passes work on whole leaves, so sparse buckets waste
// their lanes; a mixed leaf instead tests each point's cell against each
// pick's cube).  Measured on the MI355X (sampling pass per call, per-bucket
// against mixed): 64 clouds of 16,384 points on 16^3 blocks (leaves 10 %
// full) 2.52 -> 1.82 ms; the 1M-point uniform cube (50 %) 7.47 -> 8.10 ms
// and the 120,000-point scan (66 %) 3.67 -> 4.66 ms, where the wider cell
// boxes and the per-point test cost more than the lanes they fill.
// NSFPS_MIXED=0 never takes them; NSFPS_MIXED=1 whenever allowed.
bool mixed_wanted(const std::vector<CloudPlan> &plans, const uint32_t *hs) {
  const char *e = getenv("NSFPS_MIXED");
  if (e && atoi(e) == 0) return false;
  uint64_t leaves = 0, points = 0;
  for (size_t i = 0; i < plans.size(); ++i) {
    const CloudPlan &p = plans[i];
    if (p.tree || !p.rng.dev.bijective) return false;
    bool padded;
    uint64_t cap;
    leaves += bucket_leaves(p, hs + kStatWords * i, &padded, &cap);
    points += p.n;
  }
  if (e && atoi(e) == 1) return true;
  return leaves * kLeaf > 4 * points;
}

nsfps_status decide_layout(CloudPlan &p, const uint32_t *hs, bool mixed) {
  CloudDev &c = p.dev;
  const uint32_t n = p.n, T = p.rng.dev.T;
  if (hs[0]) return fail(NSFPS_EINVAL, "points must be finite");
  p.occupied = hs[4];
  bool padded;
  uint64_t cap;
  const uint64_t leaves = bucket_leaves(p, hs, &padded, &cap);
  padded = padded && !mixed;
  p.cap = padded ? cap : 0;
  c.padded = padded ? 1u : 0u;
  c.mixed = mixed ? 1u : 0u;
  c.lpc = padded ? (uint32_t)(cap / kLeaf) : 0u;
  c.nslots = padded ? (uint32_t)(cap * T) : n;
  c.nleaves = mixed ? (n + kLeaf - 1) / kLeaf : (uint32_t)leaves;
  if (c.nleaves > p.leaves_ub)
    return fail(NSFPS_EDEVICE, "internal: leaf count %u exceeds bound %u", c.nleaves, p.leaves_ub);
  c.nl1 = (c.nleaves + kFan - 1) / kFan;
  // the tree engine's single-workgroup loop keeps every level-1 node in LDS;
  // the runs engine has no such limit (level-1 nodes are its grid size)
  if (p.tree && c.nl1 > kMaxL1)
    return fail(NSFPS_EUNSUPPORTED,
                "cloud needs %u level-1 nodes, above the %u the tree engine (grids whose block "
                "counts are not all powers of two) holds",
                c.nl1, kMaxL1);
  return NSFPS_OK;
}

// The stable sorts of `total` points: nclouds clouds of n_per points stored
// one after another (nclouds = 1: one cloud).  Sort 1 by (cloud, bucket) gives
// the logical order (values: rows); with `physical`, sort 2 by (cloud, bucket,
// sub-cell) inside it gives the physical order (values: logical positions),
// which keeps the leaves of large buckets compact for box tests.  Without it
// (no result depends on the physical order) the physical order is the
// logical one and *prank is null.  Rows and positions count from the first cloud's start.
nsfps_status sort_logical(const uint32_t *bucket, uint32_t n_per, uint32_t nclouds,
                          int cloud_bits, int bucket_bits, const Scratch &s, hipStream_t st,
                          uint32_t **keys, uint32_t **lorig) {
  const uint32_t total = n_per * nclouds;
  // clouds of at most 16,384 points: one workgroup sorts each in LDS
  // (NSFPS_GLOBAL_SORT=1: always the radix sort over all clouds)
  if (n_per <= kSegSortMaxPoints && bucket_bits <= 18 && !getenv("NSFPS_GLOBAL_SORT")) {
    HIP_TRY(launch_seg_sort(bucket, n_per, nclouds, bucket_bits, s.kB, s.vB, st));
    *keys = s.kB;
    *lorig = s.vB;
    return NSFPS_OK;
  }
  if (nclouds == 1)
    HIP_TRY(hipMemcpyAsync(s.kA, bucket, (size_t)total * 4, hipMemcpyDeviceToDevice, st));
  else
    HIP_TRY(launch_cloud_keys(bucket, total, n_per, bucket_bits, s.kA, st));
  HIP_TRY(launch_radix_sort(s.kA, s.vA, s.kB, s.vB, total, cloud_bits + bucket_bits, s.hist,
                            s.scan, true, keys, lorig, st));
  return NSFPS_OK;
}

nsfps_status sort_physical(const uint32_t *bucket, const uint32_t *fine, uint32_t n_per,
                           uint32_t nclouds, int cloud_bits, int bucket_bits, const Scratch &s,
                           hipStream_t st, const uint32_t *keys, const uint32_t *lorig,
                           uint32_t **prank) {
  const uint32_t total = n_per * nclouds;
  const int fb = std::min<int>((int)kFineBits, 32 - bucket_bits - cloud_bits);
  const int fshift = (int)kFineBits - fb;
  uint32_t *k2 = (keys == s.kA) ? s.kB : s.kA;
  uint32_t *k2tmp = (k2 == s.kA) ? s.kB : s.kA;
  uint32_t *v2 = (lorig == s.vA) ? s.vB : s.vA;
  const int cloud_shift = std::min(bucket_bits + fb, 31);
  HIP_TRY(launch_key2(lorig, bucket, fine, total, n_per, cloud_shift, fshift, fb, k2, st));
  uint32_t *kdummy = nullptr;
  HIP_TRY(launch_radix_sort(k2, v2, k2tmp, s.vC, total, cloud_bits + bucket_bits + fb, s.hist,
                            s.scan, true, &kdummy, prank, st));
  return NSFPS_OK;
}

nsfps_status sort_points(const uint32_t *bucket, const uint32_t *fine, uint32_t n_per,
                         uint32_t nclouds, int cloud_bits, int bucket_bits, bool physical,
                         const Scratch &s, hipStream_t st, uint32_t **lorig, uint32_t **prank) {
  uint32_t *keys = nullptr;
  nsfps_status rc = sort_logical(bucket, n_per, nclouds, cloud_bits, bucket_bits, s, st, &keys,
                                 lorig);
  if (rc) return rc;
  *prank = nullptr;
  if (!physical) return NSFPS_OK;
  return sort_physical(bucket, fine, n_per, nclouds, cloud_bits, bucket_bits, s, st, keys,
                       *lorig, prank);
}

// Slots, cell table, leaves and tree of one cloud from the sorts: its
// physical order is prank[0 .. n), ranks and rows in prank / lorig count from
// base.
nsfps_status finish_cloud(CloudPlan &p, const uint32_t *lorig, const uint32_t *prank,
                          uint32_t base, hipStream_t st) {
  CloudDev &c = p.dev;
  const uint32_t n = p.n, T = p.rng.dev.T;
  const float *xyz = p.h_xyz ? p.d_xyz_stage : p.d_xyz_in;
  if (c.padded) {
    HIP_TRY(launch_fill_u32(c.P4, 0u, (uint64_t)c.nslots * 4, st));
    HIP_TRY(launch_fill_u32(const_cast<uint2 *>(c.RO), 0u, (uint64_t)c.nslots * 2, st));
    HIP_TRY(launch_fill_u32(const_cast<uint32_t *>(c.R), 0u, (uint64_t)c.nslots, st));
  }
  HIP_TRY(launch_gather(prank, lorig, base, p.d_bucket, p.d_counts, xyz, n, c.padded,
                        (uint32_t)p.cap, c.P4, const_cast<uint2 *>(c.RO), const_cast<uint32_t *>(c.R),
                        p.d_small + 2, st));
  HIP_TRY(launch_leaf_build(p.d_counts, p.d_lc, T, c.padded, (uint32_t)p.cap, c.lpc, c.mixed, n,
                            c.nleaves, p.rng.dev, c.P4, c.RO, const_cast<float4 *>(c.leaf_lo),
                            const_cast<float4 *>(c.leaf_hi), const_cast<uint32_t *>(c.leaf_cell),
                            const_cast<uint32_t *>(c.leaf_al), const_cast<uint2 *>(c.leaf_sc),
                            const_cast<uint2 *>(c.leaf_cbox), c.leaf_key, c.leaf_pos,
                            p.d_cell_info, st));
  HIP_TRY(launch_init_state(c, p.d_small + 2, st));
  c.lds = plan_lds(c);
  return NSFPS_OK;
}

// bd: host copies of the many-cloud build parameters, sources of
// asynchronous copies; the caller keeps them until the stream is synchronised.
nsfps_status build_clouds(std::vector<CloudPlan> &plans, const CallBuffers &cb, const Scratch &s,
                          std::vector<BuildDev> &bd, hipStream_t st) {
  const size_t nc = plans.size();
  // input: one copy when the clouds lie one after another in host memory
  bool one_copy = cb.xyz_stage != nullptr;
  for (size_t i = 0; i < nc && one_copy; ++i)
    one_copy = plans[i].h_xyz && (i == 0 || plans[i].h_xyz == plans[i - 1].h_xyz +
                                                                (size_t)plans[i - 1].n * 3);
  std::vector<HostUp> ups;
  if (one_copy) {
    ups.push_back({cb.xyz_stage, plans[0].h_xyz, (size_t)cb.n_total * 12});
  } else {
    for (auto &p : plans)
      if (p.h_xyz) ups.push_back({p.d_xyz_stage, p.h_xyz, (size_t)p.n * 12});
  }
  {
    const nsfps_status rc = upload_host(ups, st);
    if (rc) return rc;
  }
  HIP_TRY(launch_fill_u32(cb.counts, 0u, cb.counts_total, st));
  HIP_TRY(launch_fill_u32(cb.small, 0u, nc * kStatWords, st));
  // many clouds sorted together, of few buckets each: one launch per build
  // step for all of them
  uint32_t nmax = 0, tmax = 0;
  for (auto &p : plans) {
    nmax = std::max(nmax, p.n);
    tmax = std::max(tmax, p.rng.dev.T);
  }
  int cbits = 0, bbits = 0;
  const bool together = sort_together(plans, &cbits, &bbits);
  const bool many = together && tmax <= kManyMaxBuckets;
  bd.assign(many ? nc : 0, BuildDev{});
  // compute_bbox on the device for the clouds that ask for it: one launch
  // when they all do and lie one after another, else one per cloud.  With
  // d_bd each range also goes into the cloud's build parameters.
  const auto xyz_of = [&](size_t i) {
    return plans[i].h_xyz ? (const float *)plans[i].d_xyz_stage : plans[i].d_xyz_in;
  };
  bool any_dev = false, one_launch = true;
  for (size_t i = 0; i < nc; ++i) {
    any_dev = any_dev || plans[i].bbox_dev;
    one_launch = one_launch && plans[i].bbox_dev && plans[i].n == plans[0].n &&
                 xyz_of(i) == xyz_of(0) + i * (size_t)plans[0].n * 3;
  }
  const auto device_ranges = [&](BuildDev *d_bd) -> nsfps_status {
    if (one_launch) {
      HIP_TRY(launch_device_ranges(xyz_of(0), plans[0].n, (uint32_t)nc, plans[0].rng.dev, cb.ord,
                                   cb.drng, cb.dbounds, d_bd, st));
      return NSFPS_OK;
    }
    for (size_t i = 0; i < nc; ++i)
      if (plans[i].bbox_dev)
        HIP_TRY(launch_device_ranges(xyz_of(i), plans[i].n, 1, plans[i].rng.dev, cb.ord + 6 * i,
                                     cb.drng + i, cb.dbounds + 6 * i, d_bd ? d_bd + i : nullptr,
                                     st));
    return NSFPS_OK;
  };
  if (any_dev && !many) {
    const nsfps_status rc = device_ranges(nullptr);
    if (rc) return rc;
  }
  uint32_t *keys1 = nullptr, *lorig1 = nullptr;  // one cloud: its sort by bucket
  for (size_t i = 0; i < nc; ++i) {
    const CloudPlan *lut_of = nullptr;
    if (i > 0 && plans[i].rng.lut[0] == plans[0].rng.lut[0] &&
        plans[i].rng.lut[1] == plans[0].rng.lut[1] && plans[i].rng.lut[2] == plans[0].rng.lut[2])
      lut_of = &plans[0];
    if (many) {
      CloudPlan &p = plans[i];
      if (lut_of) {
        p.d_lut = lut_of->d_lut;
        p.dev.lut = p.d_lut;
      } else {
        std::vector<uint32_t> &lut = p.lut_host;
        lut.clear();
        for (int a = 0; a < 3; ++a)
          lut.insert(lut.end(), p.rng.lut[a].begin(), p.rng.lut[a].end());
        HIP_TRY(hipMemcpyAsync(p.d_lut, lut.data(), lut.size() * 4, hipMemcpyHostToDevice, st));
      }
      BuildDev &b = bd[i];
      b = BuildDev{};
      b.c = p.dev;
      b.xyz = p.h_xyz ? p.d_xyz_stage : p.d_xyz_in;
      b.bucket = p.d_bucket;
      b.fine = p.d_fine;
      b.counts = p.d_counts;
      b.lc = p.d_lc;
      b.small = p.d_small;
      b.n = p.n;
      b.T = p.rng.dev.T;
      continue;
    }
    // one cloud: sorted by bucket before the layout is decided (the sort's
    // scratch buffers then stay untouched until its finish)
    nsfps_status rc = build_phase1(plans[i], lut_of, s, st, cb.drng + i, nc == 1, &keys1, &lorig1);
    if (rc) return rc;
  }
  if (many) {
    HIP_TRY(hipMemcpyAsync(cb.bd, bd.data(), nc * sizeof(BuildDev), hipMemcpyHostToDevice, st));
    if (any_dev) {
      const nsfps_status rc = device_ranges(cb.bd);
      if (rc) return rc;
    }
    HIP_TRY(launch_build_first_many(cb.bd, (uint32_t)nc, nmax, tmax, st));
  }
  std::vector<uint32_t> hs(kStatWords * nc);
  std::vector<float> hb(any_dev ? 6 * nc : 0);
  std::vector<RangeDev> hr(any_dev ? nc : 0);
  {  // one read-back: the build stats, and the ranges found on the device
    const char *const at = reinterpret_cast<const char *>(cb.small);
    const size_t o_r = reinterpret_cast<const char *>(cb.drng) - at;
    const size_t o_b = reinterpret_cast<const char *>(cb.dbounds) - at;
    std::vector<char> rb(any_dev ? o_b + hb.size() * 4 : nc * kStatWords * 4);
    const nsfps_status rc = readback(rb.data(), at, rb.size(), st);
    if (rc) return rc;
    std::memcpy(hs.data(), rb.data(), nc * kStatWords * 4);
    if (any_dev) {
      std::memcpy(hr.data(), rb.data() + o_r, nc * sizeof(RangeDev));
      std::memcpy(hb.data(), rb.data() + o_b, hb.size() * 4);
    }
  }
  for (size_t i = 0; i < nc; ++i)
    if (hs[kStatWords * i]) return fail(NSFPS_EINVAL, "points must be finite");
  // the ranges found on the device: checked as a range given by the caller
  // would be, and kept for the rest of the build and the sampling
  for (size_t i = 0; i < nc && any_dev; ++i) {
    CloudPlan &p = plans[i];
    if (!p.bbox_dev) continue;
    const float *b6 = &hb[6 * i];
    nsfps_range prim{b6[0], b6[1], b6[2], b6[3], b6[4], b6[5], p.rng.dev.blocks[0],
                     p.rng.dev.blocks[1], p.rng.dev.blocks[2]};
    const nsfps_status rc = check_range(prim);
    if (rc) return rc;
    p.rng.prim = prim;
    p.rng.dev = hr[i];
    for (int a = 0; a < 3; ++a) {
      p.rng.info.inv_bs[a] = hr[i].inv_bs[a];
      p.rng.info.block_size[a] = hr[i].bsize[a];
      for (uint32_t k = 0; k < kCubeThr; ++k) p.rng.info.cube_thr[a][k] = hr[i].cube_thr[a][k];
    }
    p.dev.r = hr[i];
  }
  const bool mixed = mixed_wanted(plans, hs.data());
  for (size_t i = 0; i < nc; ++i) {
    nsfps_status rc = decide_layout(plans[i], &hs[kStatWords * i], mixed);
    if (rc) return rc;
  }
  // the sub-cell sort for the tree engine, and where a bucket can fill a
  // level-1 node (the update pass's node boxes then lie inside one cell)
  bool physical = false;
  for (size_t i = 0; i < nc; ++i)
    physical = physical || plans[i].tree || hs[kStatWords * i + 1] >= kFan * kLeaf;
  if (together) {
    uint32_t *lorig = nullptr, *prank = nullptr;
    nsfps_status rc = sort_points(cb.bucket, cb.fine, plans[0].n, (uint32_t)nc, cbits, bbits,
                                  physical, s, st, &lorig, &prank);
    if (rc) return rc;
    if (many) {
      uint32_t slots_max = 0, leaves_max = 0, l1_max = 0;
      for (size_t i = 0; i < nc; ++i) {
        CloudPlan &p = plans[i];
        BuildDev &b = bd[i];
        b.c = p.dev;
        b.cap = (uint32_t)p.cap;
        b.base = (uint32_t)(i * plans[0].n);
        b.prank = prank ? prank + b.base : nullptr;
        b.lorig = lorig;
        if (p.dev.padded) slots_max = std::max(slots_max, p.dev.nslots);
        leaves_max = std::max(leaves_max, p.dev.nleaves);
        l1_max = std::max(l1_max, p.dev.nl1);
        p.dev.lds = plan_lds(p.dev);
      }
      HIP_TRY(hipMemcpyAsync(cb.bd, bd.data(), nc * sizeof(BuildDev), hipMemcpyHostToDevice, st));
      HIP_TRY(launch_build_rest_many(cb.bd, (uint32_t)nc, nmax, tmax, slots_max, leaves_max,
                                     l1_max, st));
      return NSFPS_OK;
    }
    for (size_t i = 0; i < nc; ++i) {
      const uint32_t base = (uint32_t)(i * plans[0].n);
      rc = finish_cloud(plans[i], lorig, prank ? prank + base : nullptr, base, st);
      if (rc) return rc;
    }
  } else {
    for (auto &p : plans) {
      uint32_t *lorig = nullptr, *prank = nullptr;
      const int bbits = std::max(1, key_bits_for(p.rng.dev.T));
      nsfps_status rc = NSFPS_OK;
      if (nc == 1) {  // sorted by bucket already
        lorig = lorig1;
        if (physical)
          rc = sort_physical(p.d_bucket, p.d_fine, p.n, 1, 0, bbits, s, st, keys1, lorig, &prank);
      } else {
        rc = sort_points(p.d_bucket, p.d_fine, p.n, 1, 0, bbits, physical, s, st, &lorig, &prank);
      }
      if (rc) return rc;
      rc = finish_cloud(p, lorig, prank, 0, st);
      if (rc) return rc;
    }
  }
  return NSFPS_OK;
}

uint32_t wide_iters_for(const CloudPlan &p) {
  if (!p.rng.dev.bijective) return 0;
  const char *env = getenv("NSFPS_WIDE_ITERS");
  uint64_t e;
  if (env) {
    e = strtoull(env, nullptr, 10);
  } else {
    e = p.n / 4096;
    e = std::max<uint64_t>(e, 8);
    e = std::min<uint64_t>(e, 1024);
  }
  return (uint32_t)std::min<uint64_t>(e, p.m);
}

double ms_between(hipEvent_t a, hipEvent_t b) {
  float ms = 0;
  if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return -1.0;
  return ms;
}

// Speculative-run rounds until every cloud is done.  Rounds are enqueued in
// growing batches; a round of a finished cloud returns at once.  Between
// batches the host reads each cloud's done flag, sample count and list
// overflow flag.  Rounds run without refinement passes (the update pass's
// windows nearly always resolve the threshold) until a round had to force it
// and got a list under a quarter full; from the next batch on, every round
// gets kRefinePasses passes.
// The batches of rounds (size, refinement passes) the last call of a given
// shape enqueued, and the rounds it needed.  A call of the same shape enqueues
// those batches back to back, cut at that many rounds, with no status read in
// between, then goes on batch by batch if it is not finished; rounds enqueued
// after a cloud is done return at once.  The samples never depend on how
// rounds are batched.  Guarded by g_mu.
struct RoundSchedule {
  uint64_t shape[5] = {0, 0, 0, 0, 0};
  std::vector<std::pair<uint32_t, uint32_t>> batches;
  uint64_t rounds = 0;
};
RoundSchedule g_schedule;

// Rounds whose clouds all have at most this many points use the update pass
// that also bounds each pick by each leaf's box of points (the bound's extra
// work pays where cubes are large against the leaves: sparse clouds).
// Measured on the MI355X: 10,000-point quickstart 1.04 -> 0.99 ms per call,
// 120,000-point scan 4.55 -> 4.40; with it, the 1M-point uniform cube was
// 1.8 % slower (0.6 % on the later kernels).
constexpr uint32_t kLeafBoundMaxPoints = 262144;
// Larger clouds whose filled buckets hold more than this many points on
// average take it too: dense buckets fill several leaves each, and the bound
// spares the leaves of a cube's cells that no pick can lower.  8M-point
// clustered cloud (586 points a filled bucket) 61.25 against 61.79 ms per
// call; the 1M-point uniform cube (32) was 7.28 against 7.24 with it.
constexpr uint32_t kLeafBoundDensity = 64;
// Rounds with at most this many level-1 nodes over all clouds split each
// node's leaves over kUpdateSplit workgroups of the update pass (its work
// then spreads over that many more CUs; a node's key is the largest of the
// parts its workgroups write).  Measured per call: quickstart (3 nodes)
// 0.97 -> 0.82 ms, 240,000-point scan 4.45 -> 4.21, 524,288-point clustered
// cloud 7.45 -> 7.29 (at this bound; 7.45 at 128), 64 clouds of 16,384
// points (256 nodes) unchanged; the 1M-point uniform cube (512 nodes) 7.7 ->
// 12.3 with it.
constexpr uint32_t kSplitMaxNodes = 256;
// Clouds whose points fill at least this many buckets are sampled with hot
// sets of 128 copies.  The run's 1,024 list entries then average at most 4
// in a cube of 3 x 3 x 3 cells, so the copies of a hot set seldom lower one
// another and a set of 128 yields about twice the samples of a set of 64
// (a CPU model of the acceptance rule on the 1M-point uniform cube's lists:
// 84-118 samples against 53-63).  Where cubes hold many entries (clouds in
// few cells, coarse grids, or many samples per point), the 128-copy sets
// cost more than they yield.  Measured on the MI355X, 128 against 64
// copies per call: 1M-point uniform cube (32,768 buckets filled) 7.35
// against 7.69 ms, 8M-point clustered cloud (14,321) 62.4 against 70.6;
// quickstart (8) 0.91 against 0.70, 120,000-point scan (1,266) 4.09 against
// 3.90, 64 clouds of 16,384 points (about 2,530 each) 2.31 against 2.06.
constexpr uint32_t kHot128MinCells = 6912;
// Clouds whose points fill at most this many buckets take the run kernel that
// applies a large-cube sample whose cube holds the list's cell box without a
// cell test per entry.  The 10,000-point quickstart (8 buckets, every cube of
// a positive distance holding every point), per call on the MI355X: 0.65-0.66
// -> 0.62-0.63 ms (large-cube samples 4.5 k -> 3.2 k cycles a hot set).
constexpr uint32_t kWholeMaxCells = 8;
// Calls of at least this many clouds sample them in two halves on two
// streams: each round's run kernel takes one CU per cloud, and one half's
// update and gather passes then run on the other CUs beside the other half's
// run kernel (clouds are independent).  NSFPS_STREAMS=n asks for n groups
// (at most kMaxStreams).  64 clouds of 16,384 points, per call on the
// MI355X: one stream 1.94 ms, two 1.79-1.81, three 1.71-1.80.
constexpr uint32_t kTwoStreamMinClouds = 8;
constexpr uint32_t kStreamGroups = 2;

// The shape of a call's sampling passes: the update pass's workgroups per
// level-1 node and the run kernel's hot-set size (0 when the tree engine ran).
struct PassShape {
  uint32_t split = 0, hot = 0;
};

// ev_end (or null) is recorded after each batch's launches, before its status
// read-back; fin gets the clouds' statuses after the last batch.
nsfps_status run_rounds(std::vector<CloudPlan> &plans, const CloudDev *d_clouds,
                        const CloudStatus *d_status, hipStream_t st, bool profile,
                        uint64_t *rounds_out, PassShape *shape_out, hipEvent_t ev_end,
                        std::vector<CloudStatus> &fin) {
  uint32_t max_nl1 = 1;
  bool alias = false;  // some cloud's cells share buckets
  bool leaf_bound = true;  // every cloud small enough (or dense enough) for the leaf-box bound
  bool dense = true;       // every cloud's filled buckets hold more than kLeafBoundDensity points
  for (auto &p : plans) {
    max_nl1 = std::max(max_nl1, p.dev.nl1);
    alias = alias || !p.rng.dev.bijective;
    const bool d = (uint64_t)p.n > kLeafBoundDensity * std::max(1u, p.occupied);
    leaf_bound = leaf_bound && (p.n <= kLeafBoundMaxPoints || d);
    dense = dense && d;
  }
  if (const char *e = getenv("NSFPS_LEAF_BOUND")) leaf_bound = atoi(e) != 0;  // forced either way
  if (const char *e = getenv("NSFPS_DENSE_WALK")) dense = atoi(e) != 0;
  const uint32_t nc = (uint32_t)plans.size();
  const bool mixed = plans[0].dev.mixed != 0;  // the same for every cloud of a call
  const bool split = (uint64_t)nc * max_nl1 <= kSplitMaxNodes;
  // the run kernel's hot sets: 128 copies when every cloud's points fill at
  // least kHot128MinCells buckets (and no cells share buckets); NSFPS_HOT=64
  // or 128 forces either size
  bool wide = !alias;
  for (auto &p : plans) wide = wide && p.occupied >= kHot128MinCells;
  const char *hot_env = getenv("NSFPS_HOT");
  if (hot_env && atoi(hot_env) == 64) wide = false;
  if (hot_env && atoi(hot_env) == 128) wide = !alias;
  const uint32_t hot = wide ? 128u : 64u;
  // clouds in few buckets: their large cubes hold the whole list (a sample's
  // cube is checked against the list's cell box in the kernel, so this only
  // chooses the kernel); NSFPS_WHOLE=0 or 1 forces either
  bool whole = !alias && hot == 64;
  for (auto &p : plans) whole = whole && p.occupied <= kWholeMaxCells;
  if (const char *e = getenv("NSFPS_WHOLE")) whole = atoi(e) != 0 && !alias && hot == 64;
  shape_out->split = split ? kUpdateSplit : 1u;
  shape_out->hot = hot;
  const uint64_t shape[5] = {nc, plans[0].n, plans[0].m, plans[0].rng.dev.T, max_nl1};
  const bool replay = std::equal(shape, shape + 5, g_schedule.shape) && !profile;
  std::vector<std::pair<uint32_t, uint32_t>> used;
  HIP_TRY(launch_runs_init(d_clouds, nc, split, st));
  // two halves on two streams (kTwoStreamMinClouds); not for the
  // allocation-free entry point, which creates nothing
  uint32_t groups = nc >= kTwoStreamMinClouds && !profile && !g_call_no_alloc ? kStreamGroups : 1u;
  if (const char *e = getenv("NSFPS_STREAMS")) groups = g_call_no_alloc ? 1u : (uint32_t)std::max(1, atoi(e));
  groups = std::min({groups, nc, kMaxStreams});
  const bool two = groups > 1;
  hipStream_t sts[kMaxStreams] = {st};
  uint32_t g0[kMaxStreams + 1] = {}, gmax[kMaxStreams] = {};
  Arena *ap2 = nullptr;
  if (two) {
    const nsfps_status rc = arena_for_device(&ap2);
    if (rc) return rc;
    if (!ap2->fork) HIP_TRY(hipEventCreateWithFlags(&ap2->fork, hipEventDisableTiming));
    for (uint32_t k = 1; k < groups; ++k) {
      if (!ap2->stream2[k - 1]) {
        HIP_TRY(hipStreamCreateWithFlags(&ap2->stream2[k - 1], hipStreamNonBlocking));
        HIP_TRY(hipEventCreateWithFlags(&ap2->join[k - 1], hipEventDisableTiming));
      }
      sts[k] = ap2->stream2[k - 1];
    }
    // the other streams start after the build and the run state's set-up
    HIP_TRY(hipEventRecord(ap2->fork, st));
    for (uint32_t k = 1; k < groups; ++k) HIP_TRY(hipStreamWaitEvent(sts[k], ap2->fork, 0));
  }
  for (uint32_t k = 0; k <= groups; ++k) g0[k] = (uint32_t)((uint64_t)nc * k / groups);
  for (uint32_t k = 0; k < groups; ++k) {
    gmax[k] = 1;
    for (uint32_t i = g0[k]; i < g0[k + 1]; ++i) gmax[k] = std::max(gmax[k], plans[i].dev.nl1);
  }
  const auto enqueue = [&](uint32_t take, uint32_t np) -> hipError_t {
    if (!two)
      return launch_rounds(d_clouds, nc, max_nl1, take, np, profile, alias, leaf_bound, split,
                           mixed, hot, dense, whole, st);
    for (uint32_t k = 0; k < groups; ++k) {
      const hipError_t e = launch_rounds(d_clouds + g0[k], g0[k + 1] - g0[k], gmax[k], take, np,
                                         profile, alias, leaf_bound, split, mixed, hot, dense,
                                         whole, sts[k]);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  };
  std::vector<CloudStatus> pr(nc);
  uint64_t last_samples = 0, enqueued = 0;
  uint32_t batch = 4, stalled = 0, passes = 0;
  bool launched = false;  // rounds are in the queue and no status read has followed
  if (replay) {
    for (const auto &bp : g_schedule.batches) {
      const uint32_t take = (uint32_t)std::min<uint64_t>(bp.first, g_schedule.rounds - enqueued);
      if (take == 0) break;
      HIP_TRY(enqueue(take, bp.second));
      enqueued += take;
      used.emplace_back(take, bp.second);
      passes = bp.second;
      launched = true;
    }
  }
  while (true) {
    if (!launched) {
      HIP_TRY(enqueue(batch, passes));
      enqueued += batch;
      used.emplace_back(batch, passes);
    }
    launched = false;
    for (uint32_t k = 1; k < groups; ++k) {  // the statuses are read on st once every group's rounds are done
      HIP_TRY(hipEventRecord(ap2->join[k - 1], sts[k]));
      HIP_TRY(hipStreamWaitEvent(st, ap2->join[k - 1], 0));
    }
    if (ev_end) HIP_TRY(hipEventRecord(ev_end, st));
    {
      const nsfps_status rc = readback(pr.data(), d_status, nc * sizeof(CloudStatus), st);
      if (rc) return rc;
    }
    bool all = true;
    uint64_t samples = 0, rounds = 0;
    for (auto &q : pr) {
      if (q.rs.err) {
        // 1: list overflow, 2: hot-copy overflow, 3: a live key above the hot
        // histogram, 4: no crossing bin in a hot-threshold histogram
        static const char *const what[] = {"", "list overflow", "hot-copy overflow",
                                           "key above the hot histogram",
                                           "no crossing bin in the hot histogram"};
        return fail(NSFPS_EDEVICE, "internal: speculative run state: %s",
                    q.rs.err < 5 ? what[q.rs.err] : "unknown");
      }
      all = all && q.done;
      samples += q.iter;
      if (q.rs.forced) passes = kRefinePasses;
      rounds = std::max<uint64_t>(rounds, q.rs.rounds);
    }
    *rounds_out = rounds;
    if (all) {
      std::copy(shape, shape + 5, g_schedule.shape);
      g_schedule.batches = used;
      g_schedule.rounds = rounds;
      fin = pr;
      break;
    }
    // every round takes at least one sample of every unfinished cloud
    stalled = samples == last_samples ? stalled + 1 : 0;
    if (stalled >= 2) return fail(NSFPS_EDEVICE, "internal: sampling made no progress");
    last_samples = samples;
    batch = std::min<uint32_t>(batch * 2, 64);
  }
  (void)enqueued;
  return NSFPS_OK;
}

// Device memory and stream of one call: the cached per-device arena (grown on
// demand), a plan's own allocation, or the allocation-free entry point's
// static scratch array.  ev: five events timing the phases, or null.
struct Ws {
  char *base = nullptr;
  size_t cap = 0;
  hipStream_t st = nullptr;
  const hipEvent_t *ev = nullptr;
  bool st_used = false;  // work of the call was enqueued on st
};

// Where one call's buffers live: per cloud (layout_cloud), for the call
// (layout_call), the sorts' scratch, and the per-cloud descriptors and status
// words the sampling kernels read.
struct CallLayout {
  CallBuffers cb{};
  Scratch sc{};
  CloudDev *d_clouds = nullptr;
  CloudStatus *d_status = nullptr;
  uint32_t nsort = 0, tmax = 0;
};

// Lays the call out over bp (a null base measures it).
void layout_all(Bump &bp, std::vector<CloudPlan> &plans, CallLayout &L) {
  for (auto &p : plans) layout_cloud(bp, p);
  layout_call(bp, plans, L.cb);
  layout_scratch(bp, L.nsort, L.tmax, L.sc);
  L.d_clouds = bp.take<CloudDev>(plans.size());
  L.d_status = bp.take<CloudStatus>(plans.size());
  if (bp.base)
    for (size_t i = 0; i < plans.size(); ++i) {
      plans[i].dev.done = &L.d_status[i].done;
      plans[i].dev.iter = &L.d_status[i].iter;
      plans[i].dev.rs = &L.d_status[i].rs;
    }
}

// Bytes of layout_all for these clouds (and the sort sizes it uses).
size_t measure_call(std::vector<CloudPlan> &plans, CallLayout &L) {
  uint32_t nmax = 0, tmax = 0;
  for (auto &p : plans) {
    nmax = std::max(nmax, p.n);
    tmax = std::max(tmax, p.rng.dev.T);
  }
  // sorts run over one cloud, or over all clouds of a call at once
  const uint64_t all = (uint64_t)nmax * plans.size();
  L.nsort = all <= 0x7fffffffu ? (uint32_t)std::max<uint64_t>(nmax, all) : nmax;
  L.tmax = tmax;
  Bump meas(nullptr);
  layout_all(meas, plans, L);
  return meas.off + 4096;
}

// The engine: speculative runs (for every grid; where cells share buckets its
// kernels test every cell of a bucket), or the tree loop when
// NSFPS_ENGINE=tree asks.
bool choose_runs(std::vector<CloudPlan> &plans) {
  bool runs = true;
  const char *eng = getenv("NSFPS_ENGINE");
  if (eng && strcmp(eng, "tree") == 0) runs = false;
  for (auto &p : plans) p.tree = !runs;
  return runs;
}

// Samples the built clouds (descriptors in plans[i].dev): grid-wide steps for
// the first iterations of a single cloud on the tree engine, then its loop;
// or the speculative-run rounds.
// fin: the runs engine's final statuses (left empty by the tree engine)
nsfps_status sample_clouds(std::vector<CloudPlan> &plans, const CallLayout &L, const Ws &ws,
                           bool runs, uint64_t *rounds, uint64_t *wide_total,
                           PassShape *pass, std::vector<CloudStatus> &fin) {
  hipStream_t st = ws.st;
  std::vector<CloudDev> devs;
  uint32_t lds_bytes = 0;
  for (auto &p : plans) {
    devs.push_back(p.dev);
    lds_bytes = std::max(lds_bytes, p.dev.lds.total);
  }
  const bool profile = getenv("NSFPS_PROFILE") != nullptr;
  *rounds = 0;
  *wide_total = 0;
  *pass = PassShape{};
  if (runs) {
    if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[3], st));
    HIP_TRY(hipMemcpyAsync(L.d_clouds, devs.data(), devs.size() * sizeof(CloudDev),
                           hipMemcpyHostToDevice, st));
    if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[4], st));
    if (profile) HIP_TRY(launch_fill_u32(plans[0].dev.prof, 0u, kProfWords * 2, st));
    return run_rounds(plans, L.d_clouds, L.d_status, st, profile, rounds, pass,
                      ws.ev ? ws.ev[2] : nullptr, fin);
  }
  if (plans.size() == 1) {
    uint32_t e = wide_iters_for(plans[0]);
    *wide_total = e;
    if (e) HIP_TRY(launch_wide_steps(plans[0].dev, e, std::max<uint32_t>(1, plans[0].dev.nl1), st));
  }
  if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[3], st));
  HIP_TRY(hipMemcpyAsync(L.d_clouds, devs.data(), devs.size() * sizeof(CloudDev),
                         hipMemcpyHostToDevice, st));
  if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[4], st));
  if (profile) HIP_TRY(launch_fill_u32(plans[0].dev.prof, 0u, kProfWords * 2, st));
  const char *lt = getenv("NSFPS_LATE_THREADS");
  const uint32_t late_threads = (lt && atoi(lt) == 1024) ? 1024u : kLateThreads;
  HIP_TRY(launch_late_loop(L.d_clouds, (uint32_t)plans.size(), lds_bytes, profile, late_threads,
                           st));
  return NSFPS_OK;
}

// After sampling: lengths, the samples to the host (out_on_host) and the
// statistics of the call (t0: host time at its start).
// fin: the clouds' final statuses when the sampling read them back already
// (the runs engine's last batch), else empty.
nsfps_status finish_call(std::vector<CloudPlan> &plans, const CallLayout &L, const Ws &ws,
                         bool runs, uint64_t rounds, uint64_t wide_total, const PassShape &pass,
                         std::vector<CloudStatus> &fin, bool out_on_host,
                         int32_t *h_out, uint64_t out_stride, uint64_t *out_lens,
                         std::chrono::steady_clock::time_point t0) {
  hipStream_t st = ws.st;
  if (fin.size() != plans.size()) {
    if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[2], st));
    fin.assign(plans.size(), CloudStatus{});
    const nsfps_status rc = readback(fin.data(), L.d_status, fin.size() * sizeof(CloudStatus), st);
    if (rc) return rc;
  }
  uint64_t samples = 0, leaves = 0, points = 0;
  uint32_t maxlen = 0, lds_bytes = 0;
  for (size_t i = 0; i < plans.size(); ++i) {
    out_lens[i] = fin[i].iter;
    samples += fin[i].iter;
    maxlen = std::max(maxlen, fin[i].iter);
    leaves += plans[i].dev.nleaves;
    points += plans[i].n;
    lds_bytes = std::max(lds_bytes, plans[i].dev.lds.total);
  }
  if (out_on_host && maxlen) {
    if (plans.size() > 1 && out_stride == plans[0].m) {
      // rows of m entries on both sides: one copy (entries past a cloud's
      // length are left unspecified, as the interface says)
      const nsfps_status rc = download_host(h_out, L.cb.out, plans.size() * (size_t)out_stride * 4, st);
      if (rc) return rc;
    } else {
      for (size_t i = 0; i < plans.size(); ++i)
        if (fin[i].iter) {
          const nsfps_status rc =
              download_host(h_out + i * out_stride, plans[i].dev.out, (size_t)fin[i].iter * 4, st);
          if (rc) return rc;
        }
    }
  }
  if (getenv("NSFPS_PROFILE"))
    HIP_TRY(hipMemcpyAsync(g_prof, plans[0].dev.prof, sizeof(g_prof), hipMemcpyDeviceToHost, st));
  else
    memset(g_prof, 0, sizeof(g_prof));
  HIP_TRY(hipStreamSynchronize(st));
  auto t1 = std::chrono::steady_clock::now();
  nsfps_stats &S = g_stats;
  if (ws.ev) {
    S.build_ms = ms_between(ws.ev[0], ws.ev[1]);
    S.sample_ms = ms_between(ws.ev[1], ws.ev[2]);
    S.wide_ms = ms_between(ws.ev[1], ws.ev[3]);
    S.late_ms = ms_between(ws.ev[4], ws.ev[2]);
    S.device_ms = S.build_ms + S.sample_ms;
  }
  S.e2e_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
  S.n_points = points;
  S.n_clouds = plans.size();
  S.n_leaves = leaves;
  S.wide_iters = wide_total;
  S.samples = samples;
  S.padded = plans.size() == 1 ? plans[0].dev.padded : 0;
  S.mixed = plans[0].dev.mixed;
  S.lds_bytes = runs ? 0 : lds_bytes;
  S.rounds = rounds;
  S.engine = runs ? 1u : 0u;
  S.update_split = pass.split;
  S.hot_set = pass.hot;
  return NSFPS_OK;
}

// One call from start to end over workspace ws: layout, build, sampling,
// results.  ws.base == null takes the calling thread's device arena.
// A call that fails after enqueuing work waits for its stream before
// returning, so that no kernel of it still runs when the next call reuses the
// workspace (the wait's own status is ignored: the first error is reported).
nsfps_status run_clouds_once(std::vector<CloudPlan> &plans, Ws &ws, bool out_on_host,
                             int32_t *h_out, uint64_t out_stride, uint64_t *out_lens,
                             CallLayout &L);

nsfps_status run_clouds(std::vector<CloudPlan> &plans, Ws ws, bool out_on_host, int32_t *h_out,
                        uint64_t out_stride, uint64_t *out_lens) {
  CallLayout L;
  const nsfps_status rc = run_clouds_once(plans, ws, out_on_host, h_out, out_stride, out_lens, L);
  if (rc && ws.st_used) {
    (void)hipStreamSynchronize(ws.st);
    // a failed call may leave rounds of its second half queued
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 16)
      for (hipStream_t s2 : g_arena[dev].stream2)
        if (s2) (void)hipStreamSynchronize(s2);
  }
  return rc;
}

nsfps_status run_clouds_once(std::vector<CloudPlan> &plans, Ws &ws, bool out_on_host,
                             int32_t *h_out, uint64_t out_stride, uint64_t *out_lens,
                             CallLayout &L) {
  auto t0 = std::chrono::steady_clock::now();
  const size_t need = measure_call(plans, L);
  if (!ws.base) {
    Arena *ap = nullptr;
    nsfps_status rc = arena_for_device(&ap);
    if (rc) return rc;
    rc = arena_reserve(*ap, need);
    if (rc) return rc;
    ws.base = ap->base;
    ws.cap = ap->cap;
    if (!ws.st) ws.st = ap->stream;
    ws.ev = ap->ev;
  } else if (need > ws.cap) {
    return fail(NSFPS_EUNSUPPORTED,
                "the call needs %zu bytes of device workspace, more than the %zu available",
                need, ws.cap);
  }
  Bump bp(ws.base);
  layout_all(bp, plans, L);
  const bool runs = choose_runs(plans);
  hipStream_t st = ws.st;
  ws.st_used = true;
  if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[0], st));
  std::vector<BuildDev> bd_host;  // lives until the stream is synchronised below
  nsfps_status rc = build_clouds(plans, L.cb, L.sc, bd_host, st);
  if (rc) return rc;
  if (ws.ev) HIP_TRY(hipEventRecord(ws.ev[1], st));
  uint64_t rounds = 0, wide_total = 0;
  PassShape pass;
  std::vector<CloudStatus> fin;
  rc = sample_clouds(plans, L, ws, runs, &rounds, &wide_total, &pass, fin);
  if (rc) return rc;
  return finish_call(plans, L, ws, runs, rounds, wide_total, pass, fin, out_on_host, h_out,
                     out_stride, out_lens, t0);
}

// Guards of yuezu_fps (src/yuezu_fps.cpp:678-688) that need no device.
bool trivial(uint64_t n, uint64_t m, int32_t *out, uint64_t *len) {
  if (n == 0 || m == 0) {
    *len = 0;
    return true;
  }
  if (m >= n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)i;
    *len = n;
    return true;
  }
  if (m == 1) {
    out[0] = 0;
    *len = 1;
    return true;
  }
  return false;
}

void reset_stats() { memset(&g_stats, 0, sizeof(g_stats)); }

// A call on a caller's stream cannot be captured into a HIP graph: between
// batches of rounds it reads each cloud's status back and waits for the
// stream, and it returns after the stream work completes.  Refused before
// anything is enqueued, so the capture is left as it was.
nsfps_status check_not_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(st, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return fail(NSFPS_EUNSUPPORTED,
                "the stream is being captured into a HIP graph: the call cannot be captured (it "
                "reads each cloud's status back between batches of rounds and waits for the "
                "stream)");
  return NSFPS_OK;
}

// A cloud built once and sampled many times (nsfps_plan_*): its own device
// memory holds the call layout and a copy of the arrays sampling changes
// (the points' min-distances, the leaf keys and winners), taken after the
// build; each sampling restores them, re-derives the level-1 nodes and the
// sampling state, and runs the sampling pass alone.
struct PlanImpl {
  int device = -1;
  std::vector<CloudPlan> plans;  // one cloud
  CallLayout L;
  char *mem = nullptr;
  size_t cap = 0;
  float4 *p4_0 = nullptr;
  uint64_t *lk_0 = nullptr;
  float4 *lp_0 = nullptr;
  hipEvent_t ev[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  bool runs = true;
  PlanImpl() = default;
  PlanImpl(const PlanImpl &) = delete;
  PlanImpl &operator=(const PlanImpl &) = delete;
  // Frees the plan's device memory and events on its device (the caller
  // holds g_mu).
  ~PlanImpl() {
    int cur = -1;
    const bool other = hipGetDevice(&cur) == hipSuccess && device >= 0 && cur != device;
    if (other) (void)hipSetDevice(device);
    for (auto &e : ev)
      if (e) (void)hipEventDestroy(e);
    if (mem) (void)hipFree(mem);
    if (other) (void)hipSetDevice(cur);
  }
};

// The allocation-free entry point's workspace: one array per device, of
// kScratchBytes, held until the process ends.  Host code uses only the
// address hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = 64ull << 20;
__device__ __align__(256) char scratch[kScratchBytes];
void *g_scratch_ptr[16];

nsfps_status scratch_for_device(void **out) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= 16) return fail(NSFPS_EDEVICE, "device ordinal %d out of range", dev);
  const nsfps_status rc = prepare_device(dev);
  if (rc) return rc;
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(NSFPS_EDEVICE, "no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NSFPS_OK;
}

}  // namespace
}  // namespace nsfps

struct nsfps_plan_s {
  nsfps::PlanImpl impl;
};

using namespace nsfps;

namespace {

// No C++ exception crosses the C ABI: host allocation failures and any other
// exception become a status with a message.
template <class F>
nsfps_status guarded(F &&f) {
  try {
    arm_injection();
    return f();
  } catch (const std::bad_alloc &) {
    return fail(NSFPS_ENOMEM, "host allocation failed");
  } catch (const std::exception &e) {
    return fail(NSFPS_EDEVICE, "internal error: %s", e.what());
  } catch (...) {
    return fail(NSFPS_EDEVICE, "internal error");
  }
}

}  // namespace

extern "C" {

const char *nsfps_last_error(void) { return g_err.c_str(); }

const char *nsfps_version(void) { return "nsfps 0.1.0 (gfx950)"; }

nsfps_status nsfps_init_device(void) {
  return guarded([&]() -> nsfps_status {
    std::lock_guard<std::mutex> lk(g_mu);
    Arena *ap = nullptr;
    return arena_for_device(&ap);
  });
}

int nsfps_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

nsfps_status nsfps_range_derive(const nsfps_range *range, nsfps_range_info *info, uint32_t *luts,
                                uint64_t lut_cap) {
  return guarded([&]() -> nsfps_status {
    if (!range || !info) return fail(NSFPS_EINVAL, "range and info must be non-NULL");
    const uint32_t bl[3] = {range->x_blocks, range->y_blocks, range->z_blocks};
    for (uint32_t v : bl)
      if (v == 0 || v > (1u << 20)) return fail(NSFPS_EINVAL, "block counts must be in [1, 2^20]");
    HostRange h;
    derive(*range, h);
    *info = h.info;
    if (luts) {
      uint64_t need = h.lut[0].size() + h.lut[1].size() + h.lut[2].size();
      if (need > lut_cap) return fail(NSFPS_EINVAL, "lut buffer too small (%llu needed)",
                                      (unsigned long long)need);
      uint64_t o = 0;
      for (int a = 0; a < 3; ++a)
        for (uint32_t v : h.lut[a]) luts[o++] = v;
    }
    return NSFPS_OK;
  });
}

nsfps_status nsfps_bbox(const float *xyz, uint64_t n, uint32_t xb, uint32_t yb, uint32_t zb,
                        nsfps_range *out) {
  return guarded([&]() -> nsfps_status {
    if (!out || (n && !xyz)) return fail(NSFPS_EINVAL, "null pointer");
    bbox_of(xyz, n, *out);
    if (n) {
      out->x_blocks = xb;
      out->y_blocks = yb;
      out->z_blocks = zb;
    }
    return NSFPS_OK;
  });
}

namespace {

// The range of a call without one: compute_bbox of the points with these
// block counts (found on the device by the build).  Checks the block counts
// as check_range would, on placeholder bounds.
nsfps_status check_blocks(const uint32_t bl[3]) {
  const nsfps_range r{0.f, 1.f, 0.f, 1.f, 0.f, 1.f, bl[0], bl[1], bl[2]};
  return check_range(r);
}

// Clouds of one call, each with range[b] (or, range == null, compute_bbox
// of its points with block counts bl on the device).  The block-count part
// of the derivation is shared by clouds with the same counts.
nsfps_status plan_clouds(std::vector<CloudPlan> &plans, uint64_t n, uint64_t m,
                         const nsfps_range *ranges, const uint32_t bl[3]) {
  for (size_t b = 0; b < plans.size(); ++b) {
    CloudPlan &p = plans[b];
    p.n = (uint32_t)n;
    p.m = (uint32_t)m;
    const uint32_t mine[3] = {ranges ? ranges[b].x_blocks : bl[0],
                              ranges ? ranges[b].y_blocks : bl[1],
                              ranges ? ranges[b].z_blocks : bl[2]};
    const HostRange &prev = plans[b ? b - 1 : 0].rng;
    if (b > 0 && prev.dev.blocks[0] == mine[0] && prev.dev.blocks[1] == mine[1] &&
        prev.dev.blocks[2] == mine[2])
      p.rng = prev;  // the LUTs and the other block-count fields
    else
      derive_blocks(mine, p.rng);
    if (ranges) derive_floats(ranges[b], p.rng);
    p.bbox_dev = ranges == nullptr;
  }
  return NSFPS_OK;
}

// nsfps_fps / nsfps_fps_bbox: range, or (range == null) compute_bbox with
// block counts bl.
nsfps_status fps_host_common(const float *xyz, uint64_t n, uint64_t m, const nsfps_range *range,
                             const uint32_t bl[3], int32_t *out, uint64_t *out_len) {
  reset_stats();
  if (!out_len || (m && !out) || (n && !xyz)) return fail(NSFPS_EINVAL, "null pointer");
  if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
  if (!range && n == 0) {  // compute_bbox of no points: nothing to sample
    *out_len = 0;
    return NSFPS_OK;
  }
  nsfps_status rc = range ? check_range(*range) : check_blocks(bl);
  if (rc) return rc;
  if (trivial(n, m, out, out_len)) return NSFPS_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  std::vector<CloudPlan> plans(1);
  rc = plan_clouds(plans, n, m, range, bl);
  if (rc) return rc;
  plans[0].h_xyz = xyz;
  return run_clouds(plans, Ws{}, true, out, 0, out_len);
}

// Argument checks of the batched calls; *blocks gets the block counts of a
// call without ranges.
nsfps_status check_batched(const float *xyz, uint64_t batch, uint64_t n, uint64_t m,
                           const nsfps_range *ranges, const uint32_t *blocks3, const void *out,
                           const uint64_t *out_lens, uint32_t blocks[3]) {
  if (!out_lens || (m && !out) || (n && !xyz)) return fail(NSFPS_EINVAL, "null pointer");
  if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
  if (batch > 65535) return fail(NSFPS_EUNSUPPORTED, "at most 65535 clouds per call");
  if (m && batch * m > 0x7fffffffull)
    return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 samples per call");
  blocks[0] = blocks3 ? blocks3[0] : NSFPS_DEFAULT_X_BLOCKS;
  blocks[1] = blocks3 ? blocks3[1] : NSFPS_DEFAULT_Y_BLOCKS;
  blocks[2] = blocks3 ? blocks3[2] : NSFPS_DEFAULT_Z_BLOCKS;
  if (ranges) {
    for (uint64_t b = 0; b < batch; ++b) {
      const nsfps_status rc = check_range(ranges[b]);
      if (rc) return rc;
    }
  } else if (n) {
    const nsfps_status rc = check_blocks(blocks);
    if (rc) return rc;
  }
  return NSFPS_OK;
}

}  // namespace

nsfps_status nsfps_fps(const float *xyz, uint64_t n, uint64_t n_samples, const nsfps_range *range,
                       int32_t *out, uint64_t *out_len) {
  return guarded([&]() -> nsfps_status {
    const uint32_t bl[3] = {NSFPS_DEFAULT_X_BLOCKS, NSFPS_DEFAULT_Y_BLOCKS,
                            NSFPS_DEFAULT_Z_BLOCKS};
    return fps_host_common(xyz, n, n_samples, range, bl, out, out_len);
  });
}

nsfps_status nsfps_fps_bbox(const float *xyz, uint64_t n, uint64_t n_samples, uint32_t xb,
                            uint32_t yb, uint32_t zb, int32_t *out, uint64_t *out_len) {
  return guarded([&]() -> nsfps_status {
    const uint32_t bl[3] = {xb, yb, zb};
    return fps_host_common(xyz, n, n_samples, nullptr, bl, out, out_len);
  });
}

nsfps_status nsfps_fps_batched(const float *xyz, uint64_t batch, uint64_t n, uint64_t m,
                               const nsfps_range *ranges, const uint32_t *blocks3, int32_t *out,
                               uint64_t *out_lens) {
  return guarded([&]() -> nsfps_status {
    reset_stats();
    if (batch == 0) return NSFPS_OK;
    uint32_t bl[3];
    nsfps_status rc = check_batched(xyz, batch, n, m, ranges, blocks3, out, out_lens, bl);
    if (rc) return rc;
    // every cloud has n points and m samples: all are trivial, or none
    uint64_t len = 0;
    if (trivial(n, m, out, &len)) {
      for (uint64_t b = 0; b < batch; ++b) {
        if (b) trivial(n, m, out + b * m, &len);
        out_lens[b] = len;
      }
      return NSFPS_OK;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    std::vector<CloudPlan> plans(batch);
    rc = plan_clouds(plans, n, m, ranges, bl);
    if (rc) return rc;
    for (uint64_t b = 0; b < batch; ++b) plans[b].h_xyz = xyz + b * n * 3;
    return run_clouds(plans, Ws{}, true, out, m, out_lens);
  });
}

nsfps_status nsfps_fps_batched_device(const float *d_xyz, uint64_t batch, uint64_t n, uint64_t m,
                                      const nsfps_range *ranges, const uint32_t *blocks3,
                                      int32_t *d_out, uint64_t *out_lens, void *stream) {
  return guarded([&]() -> nsfps_status {
    reset_stats();
    if (batch == 0) return NSFPS_OK;
    uint32_t bl[3];
    nsfps_status rc = check_batched(d_xyz, batch, n, m, ranges, blocks3, d_out, out_lens, bl);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    hipStream_t st = (hipStream_t)stream;
    rc = check_not_capturing(st);
    if (rc) return rc;
    uint64_t len = 0;
    std::vector<int32_t> one((size_t)std::max<uint64_t>(std::min(n, m), 1));
    if (trivial(n, m, one.data(), &len)) {  // the same rows for every cloud
      for (uint64_t b = 0; b < batch; ++b) {
        out_lens[b] = len;
        if (len)
          HIP_TRY(hipMemcpyAsync(d_out + b * m, one.data(), len * 4, hipMemcpyHostToDevice, st));
      }
      HIP_TRY(hipStreamSynchronize(st));
      return NSFPS_OK;
    }
    std::vector<CloudPlan> plans(batch);
    rc = plan_clouds(plans, n, m, ranges, bl);
    if (rc) return rc;
    for (uint64_t b = 0; b < batch; ++b) {
      plans[b].d_xyz_in = d_xyz + b * n * 3;
      plans[b].d_out_user = d_out + b * m;  // row b of the caller's buffer
    }
    Ws ws;
    ws.st = st;
    return run_clouds(plans, ws, false, nullptr, 0, out_lens);
  });
}

nsfps_status nsfps_bbox_device(const float *d_xyz, uint64_t n, uint32_t xb, uint32_t yb,
                               uint32_t zb, nsfps_range *out, nsfps_range_info *info,
                               void *stream) {
  return guarded([&]() -> nsfps_status {
    if (!out || (n && !d_xyz)) return fail(NSFPS_EINVAL, "null pointer");
    if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
    const uint32_t bl[3] = {xb, yb, zb};
    HostRange h;
    if (n == 0) {  // compute_bbox of no points, as nsfps_bbox gives it
      bbox_of(d_xyz, 0, *out);
      derive(*out, h);
      if (info) *info = h.info;
      return NSFPS_OK;
    }
    nsfps_status rc = check_blocks(bl);
    if (rc) return rc;
    derive_blocks(bl, h);
    std::lock_guard<std::mutex> lk(g_mu);
    rc = check_not_capturing((hipStream_t)stream);
    if (rc) return rc;
    Arena *ap = nullptr;
    rc = arena_for_device(&ap);
    if (rc) return rc;
    Bump meas(nullptr);
    meas.take<uint32_t>(6);
    meas.take<RangeDev>(1);
    meas.take<float>(6);
    rc = arena_reserve(*ap, meas.off);
    if (rc) return rc;
    Bump bp(ap->base);
    uint32_t *ord = bp.take<uint32_t>(6);
    RangeDev *drng = bp.take<RangeDev>(1);
    float *dbounds = bp.take<float>(6);
    hipStream_t st = (hipStream_t)stream;
    HIP_TRY(launch_device_ranges(d_xyz, (uint32_t)n, 1, h.dev, ord, drng, dbounds, nullptr, st));
    float b6[6];
    RangeDev r;
    {  // one read-back: the range, then its bounds
      const size_t o_b = reinterpret_cast<char *>(dbounds) - reinterpret_cast<char *>(drng);
      std::vector<char> rb(o_b + sizeof(b6));
      HIP_TRY(hipMemcpyAsync(rb.data(), drng, rb.size(), hipMemcpyDeviceToHost, st));
      HIP_TRY(hipStreamSynchronize(st));
      std::memcpy(&r, rb.data(), sizeof(r));
      std::memcpy(b6, rb.data() + o_b, sizeof(b6));
    }
    *out = nsfps_range{b6[0], b6[1], b6[2], b6[3], b6[4], b6[5], xb, yb, zb};
    if (info) {
      for (int a = 0; a < 3; ++a) {
        h.info.inv_bs[a] = r.inv_bs[a];
        h.info.block_size[a] = r.bsize[a];
        for (uint32_t k = 0; k < kCubeThr; ++k) h.info.cube_thr[a][k] = r.cube_thr[a][k];
      }
      *info = h.info;
    }
    return NSFPS_OK;
  });
}

nsfps_status nsfps_fps_device(const float *d_xyz, uint64_t n, uint64_t m, const nsfps_range *range,
                              int32_t *d_out, uint64_t *out_len, void *stream) {
  return guarded([&]() -> nsfps_status {
    reset_stats();
    if (!range || !out_len || (m && !d_out) || (n && !d_xyz))
      return fail(NSFPS_EINVAL, "null pointer");
    if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
    nsfps_status rc = check_range(*range);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    hipStream_t st = (hipStream_t)stream;
    rc = check_not_capturing(st);
    if (rc) return rc;
    if (n == 0 || m == 0 || m >= n || m == 1) {
      std::vector<int32_t> tmp((size_t)std::min<uint64_t>(std::max<uint64_t>(n, 1), m ? m : 1));
      trivial(n, m, tmp.data(), out_len);
      if (*out_len) {
        HIP_TRY(hipMemcpyAsync(d_out, tmp.data(), *out_len * 4, hipMemcpyHostToDevice, st));
        HIP_TRY(hipStreamSynchronize(st));
      }
      return NSFPS_OK;
    }
    std::vector<CloudPlan> plans(1);
    CloudPlan &p = plans[0];
    p.n = (uint32_t)n;
    p.m = (uint32_t)m;
    derive(*range, p.rng);
    p.d_xyz_in = d_xyz;
    p.d_out_user = d_out;
    Ws ws;
    ws.st = st;
    return run_clouds(plans, ws, false, nullptr, 0, out_len);
  });
}

nsfps_status nsfps_fps_device_noalloc(const float *d_xyz, uint64_t n, uint64_t m,
                                      const nsfps_range *range, int32_t *d_out,
                                      uint64_t *out_len, void *stream) {
  return guarded([&]() -> nsfps_status {
    reset_stats();
    if (!range || !out_len || (m && !d_out) || (n && !d_xyz))
      return fail(NSFPS_EINVAL, "null pointer");
    if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
    nsfps_status rc = check_range(*range);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
      return fail(NSFPS_EDEVICE, "no HIP device available (nsfps has no CPU path)");
    hipStream_t st = (hipStream_t)stream;
    rc = check_not_capturing(st);
    if (rc) return rc;
    void *ws_base = nullptr;
    rc = scratch_for_device(&ws_base);
    if (rc) return rc;
    struct NoAlloc {  // for this call only, whichever way it returns
      NoAlloc() { g_call_no_alloc = true; }
      ~NoAlloc() { g_call_no_alloc = false; }
    } no_alloc;
    if (n == 0 || m == 0 || m >= n || m == 1) {
      int32_t first[1] = {0};
      std::vector<int32_t> tmp;
      const int32_t *src = first;
      if (m >= n) {
        tmp.resize((size_t)n);
        trivial(n, m, tmp.data(), out_len);
        src = tmp.data();
      } else {
        trivial(n, m, first, out_len);
      }
      if (*out_len) {
        HIP_TRY(hipMemcpyAsync(d_out, src, *out_len * 4, hipMemcpyHostToDevice, st));
        HIP_TRY(hipStreamSynchronize(st));
      }
      return NSFPS_OK;
    }
    std::vector<CloudPlan> plans(1);
    CloudPlan &p = plans[0];
    p.n = (uint32_t)n;
    p.m = (uint32_t)m;
    derive(*range, p.rng);
    p.d_xyz_in = d_xyz;
    p.d_out_user = d_out;
    Ws ws;
    ws.base = (char *)ws_base;
    ws.cap = kScratchBytes;
    ws.st = st;
    return run_clouds(plans, ws, false, nullptr, 0, out_len);
  });
}

uint64_t nsfps_noalloc_scratch_bytes(void) { return kScratchBytes; }

nsfps_status nsfps_plan_create(const float *xyz, uint64_t n, const nsfps_range *range,
                               int on_device, nsfps_plan **out) {
  return guarded([&]() -> nsfps_status {
    reset_stats();
    if (!out || !range || (n && !xyz)) return fail(NSFPS_EINVAL, "null pointer");
    *out = nullptr;
    if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
    nsfps_status rc = check_range(*range);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
      return fail(NSFPS_EDEVICE, "no HIP device available (nsfps has no CPU path)");
    auto plan = std::make_unique<nsfps_plan_s>();
    PlanImpl &P = plan->impl;
    HIP_TRY(hipGetDevice(&P.device));
    rc = prepare_device(P.device);
    if (rc) return rc;
    P.plans.resize(1);
    CloudPlan &p = P.plans[0];
    p.n = (uint32_t)n;
    p.m = 0;  // the sample count is given to each sampling
    derive(*range, p.rng);
    if (on_device) p.d_xyz_in = xyz;
    else p.h_xyz = xyz;
    // a cloud of at most one point needs no device structure
    if (n <= 1) {
      *out = plan.release();
      return NSFPS_OK;
    }
    const size_t need = measure_call(P.plans, P.L);
    Bump snap(nullptr);
    snap.off = need;
    const CloudPlan &pb = P.plans[0];
    snap.take<float4>(pb.slots_ub);
    snap.take<uint64_t>(pb.leaves_ub);
    snap.take<float4>(pb.leaves_ub);
    const size_t total = snap.off + 256;
    const hipError_t inj = injected(kInjAlloc);
    hipError_t e = inj != hipSuccess ? inj : hipMalloc(&P.mem, total);
    if (e != hipSuccess) {
      P.mem = nullptr;
      return fail(NSFPS_ENOMEM, "hipMalloc(%zu) failed: %s", total,
                  inj != hipSuccess ? "injected failure (NSFPS_INJECT)" : hipGetErrorString(e));
    }
    P.cap = total;
    for (auto &ev : P.ev) HIP_TRY(hipEventCreate(&ev));
    Bump bp(P.mem);
    layout_all(bp, P.plans, P.L);
    bp.off = need;
    P.p4_0 = bp.take<float4>(pb.slots_ub);
    P.lk_0 = bp.take<uint64_t>(pb.leaves_ub);
    P.lp_0 = bp.take<float4>(pb.leaves_ub);
    P.runs = choose_runs(P.plans);
    hipStream_t st = nullptr;
    std::vector<BuildDev> bd_host;
    rc = build_clouds(P.plans, P.L.cb, P.L.sc, bd_host, st);
    if (rc) return rc;
    const CloudDev &c = P.plans[0].dev;
    HIP_TRY(hipMemcpyAsync(P.p4_0, c.P4, (size_t)c.nslots * sizeof(float4),
                           hipMemcpyDeviceToDevice, st));
    HIP_TRY(hipMemcpyAsync(P.lk_0, c.leaf_key, (size_t)c.nleaves * 8, hipMemcpyDeviceToDevice, st));
    HIP_TRY(hipMemcpyAsync(P.lp_0, c.leaf_pos, (size_t)c.nleaves * sizeof(float4),
                           hipMemcpyDeviceToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));
    // the input is not read again
    P.plans[0].h_xyz = nullptr;
    P.plans[0].d_xyz_in = nullptr;
    *out = plan.release();
    return NSFPS_OK;
  });
}

nsfps_status nsfps_plan_sample(nsfps_plan *plan, uint64_t m, int32_t *d_out, uint64_t *out_len,
                               void *stream) {
  return guarded([&]() -> nsfps_status {
    reset_stats();
    if (!plan || !out_len || (m && !d_out)) return fail(NSFPS_EINVAL, "null pointer");
    PlanImpl &P = plan->impl;
    std::lock_guard<std::mutex> lk(g_mu);
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != P.device)
      return fail(NSFPS_EINVAL, "the plan was created on device %d, the current device is %d",
                  P.device, dev);
    hipStream_t st = (hipStream_t)stream;
    nsfps_status rc0 = check_not_capturing(st);
    if (rc0) return rc0;
    CloudPlan &p = P.plans[0];
    const uint64_t n = p.n;
    if (n == 0 || m == 0 || m >= n || m == 1) {
      int32_t first[1] = {0};
      std::vector<int32_t> tmp;
      const int32_t *src = first;
      if (m >= n) {
        tmp.resize((size_t)n);
        trivial(n, m, tmp.data(), out_len);
        src = tmp.data();
      } else {
        trivial(n, m, first, out_len);
      }
      if (*out_len) {
        HIP_TRY(hipMemcpyAsync(d_out, src, *out_len * 4, hipMemcpyHostToDevice, st));
        HIP_TRY(hipStreamSynchronize(st));
      }
      return NSFPS_OK;
    }
    if (m > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 samples");
    auto t0 = std::chrono::steady_clock::now();
    p.m = (uint32_t)m;
    p.dev.m = (uint32_t)m;
    p.dev.out = d_out;
    Ws ws;
    ws.base = P.mem;
    ws.cap = P.cap;
    ws.st = st;
    ws.ev = P.ev;
    CloudDev &c = p.dev;
    // the restore and the sampling; a failure after work was enqueued waits
    // for the stream before returning, as run_clouds does
    const auto body = [&]() -> nsfps_status {
      HIP_TRY(hipEventRecord(P.ev[0], st));
      HIP_TRY(hipMemcpyAsync(c.P4, P.p4_0, (size_t)c.nslots * sizeof(float4),
                             hipMemcpyDeviceToDevice, st));
      HIP_TRY(hipMemcpyAsync(c.leaf_key, P.lk_0, (size_t)c.nleaves * 8, hipMemcpyDeviceToDevice,
                             st));
      HIP_TRY(hipMemcpyAsync(c.leaf_pos, P.lp_0, (size_t)c.nleaves * sizeof(float4),
                             hipMemcpyDeviceToDevice, st));
      HIP_TRY(launch_init_state(c, p.d_small + 2, st));
      HIP_TRY(hipEventRecord(P.ev[1], st));
      uint64_t rounds = 0, wide_total = 0;
      PassShape pass;
      std::vector<CloudStatus> fin;
      const nsfps_status rc =
          sample_clouds(P.plans, P.L, ws, P.runs, &rounds, &wide_total, &pass, fin);
      if (rc) return rc;
      return finish_call(P.plans, P.L, ws, P.runs, rounds, wide_total, pass, fin, false,
                         nullptr, 0, out_len, t0);
    };
    const nsfps_status rc = body();
    if (rc) (void)hipStreamSynchronize(st);
    return rc;
  });
}

void nsfps_plan_destroy(nsfps_plan *plan) {
  if (!plan) return;
  std::lock_guard<std::mutex> lk(g_mu);
  delete plan;
}

nsfps_status nsfps_get_loop_profile(uint64_t *words, uint32_t nwords) {
  return guarded([&]() -> nsfps_status {
    if (!words) return fail(NSFPS_EINVAL, "null pointer");
    for (uint32_t i = 0; i < nwords; ++i) words[i] = i < kProfWords ? g_prof[i] : 0;
    return NSFPS_OK;
  });
}

// ------------------------------------------------------------ grouping ----

namespace {

nsfps_status check_group(uint64_t n, uint64_t m, uint64_t row) {
  if (n > 0x7fffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^31-1 points per cloud");
  if (m > 0xffffffffull) return fail(NSFPS_EUNSUPPORTED, "at most 2^32-1 centers or indices");
  if (row && m > ((uint64_t)1 << 40) / row) return fail(NSFPS_EUNSUPPORTED, "output too large");
  return NSFPS_OK;
}

nsfps_status check_ball(float radius, uint32_t nsample) {
  if (!std::isfinite(radius) || radius < 0.f)
    return fail(NSFPS_EINVAL, "radius must be finite and >= 0");
  if (nsample == 0) return fail(NSFPS_EINVAL, "nsample must be >= 1");
  return NSFPS_OK;
}

// Workspace bytes in front of the grouping calls' buffers (the bad-index flag).
constexpr size_t kGroupFlag = 256;

}  // namespace

nsfps_status nsfps_gather_points_device(const float *d_xyz, uint64_t n, const int32_t *d_idx,
                                        uint64_t m, float *d_out, void *stream) {
  return guarded([&]() -> nsfps_status {
    if (m == 0) return NSFPS_OK;
    if (!d_idx || !d_out || (n && !d_xyz)) return fail(NSFPS_EINVAL, "null pointer");
    nsfps_status rc = check_group(n, m, 0);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    rc = check_not_capturing((hipStream_t)stream);
    if (rc) return rc;
    Arena *ap = nullptr;
    rc = arena_for_device(&ap);
    if (rc) return rc;
    rc = arena_reserve(*ap, kGroupFlag);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    uint32_t *d_bad = (uint32_t *)ap->base;
    uint32_t bad = 0;
    HIP_TRY(hipMemsetAsync(d_bad, 0, 4, st));
    HIP_TRY(launch_gather_points(d_xyz, (uint32_t)n, d_idx, (uint32_t)m, d_out, d_bad, st));
    HIP_TRY(hipMemcpyAsync(&bad, d_bad, 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    if (bad) return fail(NSFPS_EINVAL, "an index lies outside [0, n)");
    return NSFPS_OK;
  });
}

nsfps_status nsfps_gather_points(const float *xyz, uint64_t n, const int32_t *idx, uint64_t m,
                                 float *out) {
  return guarded([&]() -> nsfps_status {
    if (m == 0) return NSFPS_OK;
    if (!idx || !out || (n && !xyz)) return fail(NSFPS_EINVAL, "null pointer");
    nsfps_status rc = check_group(n, m, 0);
    if (rc) return rc;
    for (uint64_t i = 0; i < m; ++i)
      if (idx[i] < 0 || (uint64_t)idx[i] >= n) return fail(NSFPS_EINVAL, "an index lies outside [0, n)");
    std::lock_guard<std::mutex> lk(g_mu);
    Arena *ap = nullptr;
    rc = arena_for_device(&ap);
    if (rc) return rc;
    const size_t o_x = kGroupFlag, o_i = o_x + ((n * 12 + 255) & ~(size_t)255),
                 o_o = o_i + ((m * 4 + 255) & ~(size_t)255), total = o_o + m * 12;
    rc = arena_reserve(*ap, total);
    if (rc) return rc;
    hipStream_t st = ap->stream;
    char *b = ap->base;
    if (n) HIP_TRY(hipMemcpyAsync(b + o_x, xyz, n * 12, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(b + o_i, idx, m * 4, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemsetAsync(b, 0, 4, st));
    HIP_TRY(launch_gather_points((const float *)(b + o_x), (uint32_t)n, (const int32_t *)(b + o_i),
                                 (uint32_t)m, (float *)(b + o_o), (uint32_t *)b, st));
    HIP_TRY(hipMemcpyAsync(out, b + o_o, m * 12, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    return NSFPS_OK;
  });
}

namespace {

// The ordered scan costs up to n * m distance tests; the grid's set-up (bounds,
// a sort of the points, 16 MB of cell ranges) pays from about 2^26 of them.
// NSFPS_BALL_QUERY=grid or =scan forces a path (diagnostics; results agree).
bool bq_use_grid(uint64_t n, uint64_t m) {
  const char *mode = getenv("NSFPS_BALL_QUERY");
  if (mode && strcmp(mode, "grid") == 0) return n > 0;
  if (mode && strcmp(mode, "scan") == 0) return false;
  return n > 8192 && n * m > ((uint64_t)1 << 26);
}

size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace bytes of the grid path for n points and m centers.
size_t bq_grid_bytes(uint64_t n, uint64_t m) {
  const size_t cells = (size_t)kBqMaxDim * kBqMaxDim * kBqMaxDim;
  const uint32_t hl = radix_hist_len((uint32_t)n);
  return 3 * 256 + 4 * up256(n * 4) + up256(((size_t)hl + 16) * 4) +
         up256(((size_t)scan_tmp_len(hl) + 16) * 4) + 2 * up256(cells * 4) + up256(n * 16) +
         up256(m * 4);
}

// Ball query of device buffers on stream st; ws: bq_grid_bytes(n, m) of
// workspace (unused for small clouds).
nsfps_status ball_query_on(hipStream_t st, const float *xyz, uint64_t n, const float *centers,
                           uint64_t m, float radius, uint32_t nsample, int32_t *out, char *ws) {
  const float r2 = radius * radius;
  if (n == 0 || !(r2 > 0.f)) {  // nothing lies closer than the radius: rows of zeros
    HIP_TRY(hipMemsetAsync(out, 0, (size_t)m * nsample * 4, st));
  } else if (!bq_use_grid(n, m)) {
    HIP_TRY(launch_ball_query(xyz, (uint32_t)n, centers, nullptr, (uint32_t)m, r2, nsample, out,
                              st));
  } else {
    const size_t cells = (size_t)kBqMaxDim * kBqMaxDim * kBqMaxDim;
    const uint32_t hl = radix_hist_len((uint32_t)n);
    char *b = ws;
    auto take = [&](size_t bytes) {
      char *p = b;
      b += up256(bytes);
      return p;
    };
    uint32_t *bnd = (uint32_t *)take(32);
    BqGrid *grid = (BqGrid *)take(sizeof(BqGrid));
    uint32_t *novf_d = (uint32_t *)take(4);
    uint32_t *keys = (uint32_t *)take(n * 4), *vals = (uint32_t *)take(n * 4);
    uint32_t *keys2 = (uint32_t *)take(n * 4), *vals2 = (uint32_t *)take(n * 4);
    uint32_t *hist = (uint32_t *)take(((size_t)hl + 16) * 4);
    uint32_t *scan = (uint32_t *)take(((size_t)scan_tmp_len(hl) + 16) * 4);
    uint32_t *cstart = (uint32_t *)take(cells * 4), *cend = (uint32_t *)take(cells * 4);
    float4 *spts = (float4 *)take(n * 16);
    uint32_t *ovf = (uint32_t *)take(m * 4);
    HIP_TRY(hipMemsetAsync(bnd, 0xff, 12, st));
    HIP_TRY(hipMemsetAsync(bnd + 3, 0, 12, st));
    HIP_TRY(hipMemsetAsync(novf_d, 0, 4, st));
    HIP_TRY(hipMemsetAsync(cstart, 0, cells * 4, st));
    HIP_TRY(hipMemsetAsync(cend, 0, cells * 4, st));
    HIP_TRY(launch_bq_grid_build(xyz, (uint32_t)n, radius, bnd, grid, keys, st));
    uint32_t *sk = nullptr, *sv = nullptr;
    HIP_TRY(launch_radix_sort(keys, vals, keys2, vals2, (uint32_t)n, 22, hist, scan, true, &sk,
                              &sv, st));
    HIP_TRY(launch_bq_cells(sk, sv, (uint32_t)n, xyz, grid, cstart, cend, spts, st));
    HIP_TRY(launch_bq_query(spts, grid, cstart, cend, centers, (uint32_t)m, r2, nsample, out, ovf,
                            novf_d, st));
    uint32_t novf = 0;
    HIP_TRY(hipMemcpyAsync(&novf, novf_d, 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    if (novf > m) return fail(NSFPS_EDEVICE, "internal: %u ball-query overflows for %llu centers",
                              novf, (unsigned long long)m);
    if (novf)
      HIP_TRY(launch_ball_query(xyz, (uint32_t)n, centers, ovf, novf, r2, nsample, out, st));
  }
  HIP_TRY(hipStreamSynchronize(st));
  return NSFPS_OK;
}

}  // namespace

nsfps_status nsfps_ball_query_device(const float *d_xyz, uint64_t n, const float *d_centers,
                                     uint64_t m, float radius, uint32_t nsample, int32_t *d_out,
                                     void *stream) {
  return guarded([&]() -> nsfps_status {
    nsfps_status rc = check_ball(radius, nsample);
    if (rc) return rc;
    if (m == 0) return NSFPS_OK;
    if (!d_centers || !d_out || (n && !d_xyz)) return fail(NSFPS_EINVAL, "null pointer");
    rc = check_group(n, m, nsample);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    rc = check_not_capturing((hipStream_t)stream);
    if (rc) return rc;
    Arena *ap = nullptr;
    rc = arena_for_device(&ap);
    if (rc) return rc;
    if (bq_use_grid(n, m)) {
      rc = arena_reserve(*ap, bq_grid_bytes(n, m));
      if (rc) return rc;
    }
    return ball_query_on((hipStream_t)stream, d_xyz, n, d_centers, m, radius, nsample, d_out,
                         ap->base);
  });
}

nsfps_status nsfps_ball_query(const float *xyz, uint64_t n, const float *centers, uint64_t m,
                              float radius, uint32_t nsample, int32_t *out) {
  return guarded([&]() -> nsfps_status {
    nsfps_status rc = check_ball(radius, nsample);
    if (rc) return rc;
    if (m == 0) return NSFPS_OK;
    if (!centers || !out || (n && !xyz)) return fail(NSFPS_EINVAL, "null pointer");
    rc = check_group(n, m, nsample);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    Arena *ap = nullptr;
    rc = arena_for_device(&ap);
    if (rc) return rc;
    const size_t o_x = 0, o_c = o_x + up256(n * 12), o_o = o_c + up256(m * 12),
                 o_w = o_o + up256(m * (size_t)nsample * 4);
    rc = arena_reserve(*ap, o_w + (bq_use_grid(n, m) ? bq_grid_bytes(n, m) : 0));
    if (rc) return rc;
    hipStream_t st = ap->stream;
    char *b = ap->base;
    if (n) HIP_TRY(hipMemcpyAsync(b + o_x, xyz, n * 12, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(b + o_c, centers, m * 12, hipMemcpyHostToDevice, st));
    rc = ball_query_on(st, (const float *)(b + o_x), n, (const float *)(b + o_c), m, radius, nsample,
                       (int32_t *)(b + o_o), b + o_w);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(out, b + o_o, m * (size_t)nsample * 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    return NSFPS_OK;
  });
}

nsfps_status nsfps_get_stats(nsfps_stats *stats) {
  return guarded([&]() -> nsfps_status {
    if (!stats) return fail(NSFPS_EINVAL, "null pointer");
    *stats = g_stats;
    return NSFPS_OK;
  });
}

void nsfps_release_workspace(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto &a : g_arena) {
    if (a.base) {
      (void)hipFree(a.base);
      a.base = nullptr;
      a.cap = 0;
    }
    if (a.pin.p) {
      if (a.pin.pending) (void)hipEventSynchronize(a.pin.done);
      (void)hipHostFree(a.pin.p);
      a.pin.p = nullptr;
      a.pin.cap = 0;
      a.pin.pending = false;
    }
    if (a.rb) {
      (void)hipHostFree(a.rb);
      a.rb = nullptr;
      a.rb_cap = 0;
    }
  }
}

}  // extern "C"
