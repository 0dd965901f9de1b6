"""The reference's import path for the FPS module.

``import yuezu_fps.yuezu_fps_module as yf`` loads the pybind11 module built
here from ns_fps_amd/csrc/yuezu_fps_pybind.cpp (``python -m ns_fps_amd.build``),
which calls the HIP library ns_fps_amd/libnsfps.so through its C ABI.
"""
