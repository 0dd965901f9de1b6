// Python module `yuezu_fps_module`: the reference's Python surface
// (yuezu_fps/yuezu_fps_pybind.cpp:103-150) bound to the nsfps C ABI.
//
//   SpaceRange, make_range, make_uniform_range, fps, fps_with_bbox, the five
//   constants -- same names and argument meaning as the reference -- plus
//   fps_batched and last_stats.
//
// Differences that fix reference defects, not behaviour:
//   * input is converted with c_style|forcecast, so strided views and float64
//     arrays are read correctly (the reference indexes ptr[i*3+k] of whatever
//     buffer it gets, yuezu_fps/yuezu_fps_pybind.cpp:17-33);
//   * derived SpaceRange values are recomputed from the nine primary fields on
//     every use (the reference keeps stale fields after edits and leaves them
//     uninitialised for dict ranges, :36-64, :107-125);
//   * the result is int32 (the reference returns size_t, :83-85);
//   * both `sample_count` (the binding's keyword, :137) and `n_samples` (the
//     README's keyword, README.md:70) are accepted.
// Invalid input raises InputError, a subclass of both ValueError and
// RuntimeError (the reference raises RuntimeError, :21, :61); device failures
// raise RuntimeError.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "nsfps.h"

namespace py = pybind11;

namespace {

PyObject *g_input_error = nullptr;

struct SpaceRangePy {
  float min_x = 0, max_x = 0, min_y = 0, max_y = 0, min_z = 0, max_z = 0;
  uint32_t x_blocks = 0, y_blocks = 0, z_blocks = 0;

  nsfps_range prim() const {
    nsfps_range r;
    r.min_x = min_x; r.max_x = max_x;
    r.min_y = min_y; r.max_y = max_y;
    r.min_z = min_z; r.max_z = max_z;
    r.x_blocks = x_blocks; r.y_blocks = y_blocks; r.z_blocks = z_blocks;
    return r;
  }
  nsfps_range_info info() const {
    nsfps_range r = prim();
    nsfps_range_info i{};
    if (nsfps_range_derive(&r, &i, nullptr, 0) != NSFPS_OK) {
      PyErr_SetString(g_input_error, nsfps_last_error());
      throw py::error_already_set();
    }
    return i;
  }
  // block_size_*: (max - min) / blocks (src/yuezu_fps.cpp:7-11)
  float block_size_x() const { return (max_x - min_x) / (float)x_blocks; }
  float block_size_y() const { return (max_y - min_y) / (float)y_blocks; }
  float block_size_z() const { return (max_z - min_z) / (float)z_blocks; }
  uint32_t x_bits() const { return info().bits[0]; }
  uint32_t y_bits() const { return info().bits[1]; }
  uint32_t z_bits() const { return info().bits[2]; }
  uint32_t total_bits() const { return info().total_bits; }
  uint64_t total_blocks() const { return (uint64_t)x_blocks * y_blocks * z_blocks; }
  float inv_bs_x() const { return info().inv_bs[0]; }
  float inv_bs_y() const { return info().inv_bs[1]; }
  float inv_bs_z() const { return info().inv_bs[2]; }
};

[[noreturn]] void raise_status(nsfps_status s) {
  std::string msg = nsfps_last_error();
  if (s == NSFPS_EINVAL) {
    PyErr_SetString(g_input_error, msg.c_str());
    throw py::error_already_set();
  }
  throw std::runtime_error(msg.empty() ? std::string("nsfps failure") : msg);
}

[[noreturn]] void raise_input(const std::string &msg) {
  PyErr_SetString(g_input_error, msg.c_str());
  throw py::error_already_set();
}

SpaceRangePy make_range_py(float min_x, float max_x, float min_y, float max_y, float min_z,
                           float max_z, uint32_t xb, uint32_t yb, uint32_t zb) {
  SpaceRangePy r;
  r.min_x = min_x; r.max_x = max_x;
  r.min_y = min_y; r.max_y = max_y;
  r.min_z = min_z; r.max_z = max_z;
  r.x_blocks = xb; r.y_blocks = yb; r.z_blocks = zb;
  return r;
}

using FArray = py::array_t<float, py::array::c_style | py::array::forcecast>;

FArray as_points(py::handle obj) {
  FArray a = FArray::ensure(obj);
  if (!a) raise_input("points must be convertible to a float32 array");
  if (a.ndim() != 2 || a.shape(1) != 3) raise_input("Expected 2D array with shape (N, 3)");
  return a;
}

// parse_range: SpaceRange object or dict (yuezu_fps/yuezu_fps_pybind.cpp:36-64)
nsfps_range parse_range(py::handle obj) {
  if (py::isinstance<SpaceRangePy>(obj)) return obj.cast<SpaceRangePy>().prim();
  if (py::isinstance<py::dict>(obj)) {
    py::dict d = py::reinterpret_borrow<py::dict>(obj);
    const char *req[6] = {"min_x", "max_x", "min_y", "max_y", "min_z", "max_z"};
    float v[6];
    for (int i = 0; i < 6; ++i) {
      if (!d.contains(req[i]))
        raise_input("range must be a SpaceRange object or a dict with keys: min_x, max_x, "
                    "min_y, max_y, min_z, max_z");
      v[i] = d[req[i]].cast<float>();
    }
    auto get_blocks = [&](const char *k) -> uint32_t {
      return d.contains(k) ? d[k].cast<uint32_t>() : (uint32_t)NSFPS_DEFAULT_X_BLOCKS;
    };
    nsfps_range r;
    r.min_x = v[0]; r.max_x = v[1]; r.min_y = v[2]; r.max_y = v[3]; r.min_z = v[4]; r.max_z = v[5];
    r.x_blocks = get_blocks("x_blocks");
    r.y_blocks = get_blocks("y_blocks");
    r.z_blocks = get_blocks("z_blocks");
    return r;
  }
  raise_input("range must be a SpaceRange object or a dict with keys: min_x, max_x, min_y, "
              "max_y, min_z, max_z");
}

uint64_t resolve_count(py::object sample_count, py::object n_samples) {
  if (!sample_count.is_none() && !n_samples.is_none())
    raise_input("pass only one of sample_count / n_samples");
  py::object v = sample_count.is_none() ? n_samples : sample_count;
  if (v.is_none()) raise_input("sample_count (or n_samples) is required");
  long long c = v.cast<long long>();
  if (c < 0) raise_input("sample_count must be >= 0");
  return (uint64_t)c;
}

py::array_t<int32_t> finish(std::vector<int32_t> &buf, uint64_t len) {
  py::array_t<int32_t> out((py::ssize_t)len);
  if (len) std::memcpy(out.mutable_data(), buf.data(), len * 4);
  return out;
}

py::array_t<int32_t> fps_py(py::handle points, py::object sample_count, py::object range,
                            py::object n_samples) {
  FArray p = as_points(points);
  uint64_t m = resolve_count(sample_count, n_samples);
  uint64_t n = (uint64_t)p.shape(0);
  bool has_range = !range.is_none();
  nsfps_range r{};
  if (has_range) r = parse_range(range);
  std::vector<int32_t> buf((size_t)std::max<uint64_t>(std::min(m, n), 1));
  uint64_t len = 0;
  nsfps_status s;
  {
    py::gil_scoped_release nogil;
    s = nsfps_fps(p.data(), n, m, has_range ? &r : nullptr, buf.data(), &len);
  }
  if (s != NSFPS_OK) raise_status(s);
  return finish(buf, len);
}

py::array_t<int32_t> fps_with_bbox_py(py::handle points, py::object sample_count, uint32_t xb,
                                      uint32_t yb, uint32_t zb, py::object n_samples) {
  FArray p = as_points(points);
  uint64_t m = resolve_count(sample_count, n_samples);
  uint64_t n = (uint64_t)p.shape(0);
  std::vector<int32_t> buf((size_t)std::max<uint64_t>(std::min(m, n), 1));
  uint64_t len = 0;
  nsfps_status s;
  {
    py::gil_scoped_release nogil;
    s = nsfps_fps_bbox(p.data(), n, m, xb, yb, zb, buf.data(), &len);
  }
  if (s != NSFPS_OK) raise_status(s);
  return finish(buf, len);
}

// Batched FPS: points (B, N, 3); range None (per-cloud compute_bbox with the
// given blocks), one range for all clouds, or a sequence of B ranges.
// Returns (indices int32 (B, n_samples) padded with -1, lengths int64 (B,)).
py::tuple fps_batched_py(py::handle points, uint64_t n_samples, py::object range, uint32_t xb,
                         uint32_t yb, uint32_t zb) {
  FArray p = FArray::ensure(points);
  if (!p) raise_input("points must be convertible to a float32 array");
  if (p.ndim() != 3 || p.shape(2) != 3) raise_input("Expected 3D array with shape (B, N, 3)");
  uint64_t B = (uint64_t)p.shape(0), n = (uint64_t)p.shape(1);
  std::vector<nsfps_range> rs;
  if (!range.is_none()) {
    if (py::isinstance<SpaceRangePy>(range) || py::isinstance<py::dict>(range)) {
      rs.assign(B, parse_range(range));
    } else {
      py::sequence seq = range.cast<py::sequence>();
      if ((uint64_t)py::len(seq) != B) raise_input("need one range per cloud");
      for (auto item : seq) rs.push_back(parse_range(item));
    }
  }
  uint64_t cols = std::min<uint64_t>(n_samples, n);
  py::array_t<int32_t> out({(py::ssize_t)B, (py::ssize_t)cols});
  py::array_t<int64_t> lens((py::ssize_t)B);
  // rows of n_samples on both sides (n_samples <= n): the library writes the
  // result array itself; otherwise through a buffer of its row stride
  const bool direct = cols == n_samples && cols > 0;
  std::vector<int32_t> buf(
      direct ? 0 : (size_t)std::max<uint64_t>(B * std::max<uint64_t>(n_samples, 1), 1));
  std::vector<uint64_t> lv(B);
  uint32_t blocks[3] = {xb, yb, zb};
  int32_t *o = out.mutable_data();
  int32_t *dst = direct ? o : buf.data();
  nsfps_status s;
  {
    py::gil_scoped_release nogil;
    s = nsfps_fps_batched(p.data(), B, n, n_samples, rs.empty() ? nullptr : rs.data(), blocks,
                          dst, lv.data());
  }
  if (s != NSFPS_OK) raise_status(s);
  int64_t *l = lens.mutable_data();
  for (uint64_t b = 0; b < B; ++b) {
    l[b] = (int64_t)lv[b];
    if (direct) {
      for (uint64_t j = lv[b]; j < cols; ++j) o[b * cols + j] = -1;
    } else {
      for (uint64_t j = 0; j < cols; ++j) o[b * cols + j] = j < lv[b] ? buf[b * n_samples + j] : -1;
    }
  }
  return py::make_tuple(out, lens);
}

// The grouping step after sampling (no counterpart in the reference):
// gather_points(points (N, 3), idx (M,)) -> (M, 3) float32;
// ball_query(points (N, 3), centers (M, 3), radius, nsample) -> (M, nsample) int32.
py::array_t<float> gather_points_py(py::handle points, py::handle idx) {
  FArray p = as_points(points);
  auto ia = py::array_t<int32_t, py::array::c_style | py::array::forcecast>::ensure(idx);
  if (!ia) raise_input("indices must be convertible to an int32 array");
  if (ia.ndim() != 1) raise_input("indices must be one-dimensional");
  const uint64_t n = (uint64_t)p.shape(0), m = (uint64_t)ia.shape(0);
  py::array_t<float> out({(py::ssize_t)m, (py::ssize_t)3});
  nsfps_status s;
  {
    py::gil_scoped_release nogil;
    s = nsfps_gather_points(p.data(), n, ia.data(), m, out.mutable_data());
  }
  if (s != NSFPS_OK) raise_status(s);
  return out;
}

py::array_t<int32_t> ball_query_py(py::handle points, py::handle centers, float radius,
                                   uint32_t nsample) {
  FArray p = as_points(points);
  FArray c = as_points(centers);
  const uint64_t n = (uint64_t)p.shape(0), m = (uint64_t)c.shape(0);
  py::array_t<int32_t> out({(py::ssize_t)m, (py::ssize_t)nsample});
  nsfps_status s;
  {
    py::gil_scoped_release nogil;
    s = nsfps_ball_query(p.data(), n, c.data(), m, radius, nsample, out.mutable_data());
  }
  if (s != NSFPS_OK) raise_status(s);
  return out;
}

py::dict last_stats_py() {
  nsfps_stats s{};
  nsfps_get_stats(&s);
  py::dict d;
  d["build_ms"] = s.build_ms;
  d["sample_ms"] = s.sample_ms;
  d["wide_ms"] = s.wide_ms;
  d["late_ms"] = s.late_ms;
  d["padded"] = s.padded;
  d["lds_bytes"] = s.lds_bytes;
  d["device_ms"] = s.device_ms;
  d["e2e_ms"] = s.e2e_ms;
  d["n_points"] = s.n_points;
  d["n_clouds"] = s.n_clouds;
  d["n_leaves"] = s.n_leaves;
  d["wide_iters"] = s.wide_iters;
  d["samples"] = s.samples;
  d["rounds"] = s.rounds;
  d["engine"] = s.engine ? "runs" : "tree";
  d["update_split"] = s.update_split;
  d["mixed"] = s.mixed;
  d["hot_set"] = s.hot_set;
  return d;
}

}  // namespace

PYBIND11_MODULE(yuezu_fps_module, m) {
  m.doc() = "Farthest point sampling (NS-FPS semantics) on AMD MI355X";

  py::tuple bases = py::make_tuple(py::handle(PyExc_ValueError), py::handle(PyExc_RuntimeError));
  g_input_error = PyErr_NewException("yuezu_fps_module.InputError", bases.ptr(), nullptr);
  m.attr("InputError") = py::handle(g_input_error);

  py::class_<SpaceRangePy>(m, "SpaceRange")
      .def(py::init<>())
      .def_readwrite("min_x", &SpaceRangePy::min_x)
      .def_readwrite("max_x", &SpaceRangePy::max_x)
      .def_readwrite("min_y", &SpaceRangePy::min_y)
      .def_readwrite("max_y", &SpaceRangePy::max_y)
      .def_readwrite("min_z", &SpaceRangePy::min_z)
      .def_readwrite("max_z", &SpaceRangePy::max_z)
      .def_readwrite("x_blocks", &SpaceRangePy::x_blocks)
      .def_readwrite("y_blocks", &SpaceRangePy::y_blocks)
      .def_readwrite("z_blocks", &SpaceRangePy::z_blocks)
      .def("block_size_x", &SpaceRangePy::block_size_x)
      .def("block_size_y", &SpaceRangePy::block_size_y)
      .def("block_size_z", &SpaceRangePy::block_size_z)
      .def("x_bits", &SpaceRangePy::x_bits)
      .def("y_bits", &SpaceRangePy::y_bits)
      .def("z_bits", &SpaceRangePy::z_bits)
      .def("total_bits", &SpaceRangePy::total_bits)
      .def("total_blocks", &SpaceRangePy::total_blocks)
      .def_property_readonly("inv_bs_x", &SpaceRangePy::inv_bs_x)
      .def_property_readonly("inv_bs_y", &SpaceRangePy::inv_bs_y)
      .def_property_readonly("inv_bs_z", &SpaceRangePy::inv_bs_z)
      .def("__repr__", [](const SpaceRangePy &r) {
        char b[256];
        snprintf(b, sizeof(b), "SpaceRange([%g, %g] x [%g, %g] x [%g, %g], %ux%ux%u)", r.min_x,
                 r.max_x, r.min_y, r.max_y, r.min_z, r.max_z, r.x_blocks, r.y_blocks, r.z_blocks);
        return std::string(b);
      });

  m.def("make_range", &make_range_py, py::arg("min_x"), py::arg("max_x"), py::arg("min_y"),
        py::arg("max_y"), py::arg("min_z"), py::arg("max_z"), py::arg("x_blocks"),
        py::arg("y_blocks"), py::arg("z_blocks"));

  m.def(
      "make_uniform_range",
      [](float min_x, float max_x, float min_y, float max_y, float min_z, float max_z,
         uint32_t bpd) { return make_range_py(min_x, max_x, min_y, max_y, min_z, max_z, bpd, bpd, bpd); },
      py::arg("min_x"), py::arg("max_x"), py::arg("min_y"), py::arg("max_y"), py::arg("min_z"),
      py::arg("max_z"), py::arg("blocks_per_dim"));

  m.def("fps", &fps_py, py::arg("points"), py::arg("sample_count") = py::none(),
        py::arg("range") = py::none(), py::kw_only(), py::arg("n_samples") = py::none());

  m.def("fps_with_bbox", &fps_with_bbox_py, py::arg("points"),
        py::arg("sample_count") = py::none(), py::arg("x_blocks") = NSFPS_DEFAULT_X_BLOCKS,
        py::arg("y_blocks") = NSFPS_DEFAULT_Y_BLOCKS, py::arg("z_blocks") = NSFPS_DEFAULT_Z_BLOCKS,
        py::kw_only(), py::arg("n_samples") = py::none());

  m.def("fps_batched", &fps_batched_py, py::arg("points"), py::arg("n_samples"),
        py::arg("range") = py::none(), py::arg("x_blocks") = NSFPS_DEFAULT_X_BLOCKS,
        py::arg("y_blocks") = NSFPS_DEFAULT_Y_BLOCKS, py::arg("z_blocks") = NSFPS_DEFAULT_Z_BLOCKS);

  m.def("gather_points", &gather_points_py, py::arg("points"), py::arg("idx"));
  m.def("ball_query", &ball_query_py, py::arg("points"), py::arg("centers"), py::arg("radius"),
        py::arg("nsample"));
  m.def("last_stats", &last_stats_py);
  m.def("last_loop_profile", []() {
    std::vector<uint64_t> w(24, 0);
    nsfps_get_loop_profile(w.data(), (uint32_t)w.size());
    return w;
  });
  m.def("device_count", []() { return nsfps_device_count(); });

  m.attr("DEFAULT_X_BLOCKS") = NSFPS_DEFAULT_X_BLOCKS;
  m.attr("DEFAULT_Y_BLOCKS") = NSFPS_DEFAULT_Y_BLOCKS;
  m.attr("DEFAULT_Z_BLOCKS") = NSFPS_DEFAULT_Z_BLOCKS;
  m.attr("MORTON_BLOCK_SIZE") = NSFPS_MORTON_BLOCK_SIZE;
  m.attr("CACHE_BLOCK_SIZE") = NSFPS_CACHE_BLOCK_SIZE;
}
