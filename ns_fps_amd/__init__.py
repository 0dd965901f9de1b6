"""MI355X-native farthest point sampling with the NS-FPS (yuezu_fps) semantics.

* ``yuezu_fps.yuezu_fps_module`` -- the drop-in Python module under the
  reference's import path (SpaceRange, make_range, make_uniform_range, fps,
  fps_with_bbox, constants, plus fps_batched and the grouping step), built
  from csrc/ by ``python -m ns_fps_amd.build``.
* ``ns_fps_amd.capi`` -- ctypes binding of the C ABI (include/nsfps.h).
* ``ns_fps_amd.workloads`` -- seeded synthetic clouds of the benchmark.
* ``ns_fps_amd.kitti`` -- KITTI scan files: reader, z filter, bounds range
  and the reference drivers' sampling runs.

There is no CPU implementation: without the built HIP library and a device,
compute calls raise.
"""

__version__ = "0.1.0"
