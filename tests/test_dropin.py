"""The module under the reference's own import path.

Reference callers do ``import yuezu_fps.yuezu_fps_module as yf`` (example.py:2,
semantickitti_example.py:3, README.md:45; the name comes from setup.py:6) and
call ``yf.make_range`` with keywords and ``yf.fps`` with ``n_samples=``/
``range=`` keywords (README.md:59-71) or positionally (test.py:118,
example.py:26).  These tests import the module by that name and make those
calls unchanged; on the GPU every form must return the reference's samples
(the golden vector of the README's 10,000-point, 16^3 call)."""

import importlib
import os

import numpy as np
import pytest

from conftest import GOLDEN_CASES, ROOT


def test_reference_import_path_loads_the_built_module():
    yf = importlib.import_module("yuezu_fps.yuezu_fps_module")
    # NSFPS_MODULE: another build of the module stands in (the sanitized run)
    want = os.path.dirname(os.environ.get("NSFPS_MODULE") or
                           os.path.join(ROOT, "yuezu_fps", "yuezu_fps_module"))
    assert os.path.dirname(os.path.abspath(yf.__file__)) == os.path.abspath(want)
    for name in ["SpaceRange", "make_range", "make_uniform_range", "fps", "fps_with_bbox",
                 "DEFAULT_X_BLOCKS", "DEFAULT_Y_BLOCKS", "DEFAULT_Z_BLOCKS",
                 "MORTON_BLOCK_SIZE", "CACHE_BLOCK_SIZE"]:
        assert hasattr(yf, name), name
    # the README's keyword spelling of make_range
    r = yf.make_range(min_x=-100, max_x=100, min_y=-100, max_y=100, min_z=-100, max_z=100,
                      x_blocks=16, y_blocks=16, z_blocks=16)
    assert (r.x_blocks, r.y_blocks, r.z_blocks) == (16, 16, 16)
    assert r.total_blocks() == 4096 and r.total_bits() == 12


def test_only_one_copy_of_the_bindings_is_built():
    """pybind11 registers SpaceRange once per process; a second module with the
    same types would fail to import beside the first."""
    stale = [f for f in os.listdir(os.path.join(ROOT, "ns_fps_amd"))
             if f.startswith("yuezu_fps_module")]
    assert stale == []


@pytest.mark.gpu
def test_readme_and_testpy_call_forms_give_the_reference_samples():
    import yuezu_fps.yuezu_fps_module as yf
    if yf.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    case = next(c for c in GOLDEN_CASES if c.name == "quickstart_full")
    points = case.points
    assert case.range == (-100.0, 100.0, -100.0, 100.0, -100.0, 100.0, 16, 16, 16)
    space_range = yf.make_range(min_x=-100, max_x=100, min_y=-100, max_y=100,
                                min_z=-100, max_z=100, x_blocks=16, y_blocks=16, z_blocks=16)
    forms = {
        "readme_keywords": lambda: yf.fps(points, n_samples=1000, range=space_range),
        "positional": lambda: yf.fps(points, 1000, space_range),
        "binding_keyword": lambda: yf.fps(points, sample_count=1000, range=space_range),
        "positional_range_call": lambda: yf.fps(
            points, 1000, yf.make_range(-100, 100, -100, 100, -100, 100, 16, 16, 16)),
        "dict_range": lambda: yf.fps(points, 1000, {"min_x": -100, "max_x": 100, "min_y": -100,
                                                    "max_y": 100, "min_z": -100, "max_z": 100,
                                                    "x_blocks": 16, "y_blocks": 16,
                                                    "z_blocks": 16}),
    }
    for name, call in forms.items():
        got = call()
        assert np.array_equal(got, case.expected), name
        # the README's next line indexes the points with the result
        assert points[got].shape == (1000, 3), name
