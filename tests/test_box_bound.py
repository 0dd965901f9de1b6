"""The update pass skips a pick for a level-1 node when the pick's squared
distance to the node's box of points is at least the node's largest point
distance (ns_fps_amd/csrc/nsfps_runs.hip, box_bound and k_update).  That skip
changes no result only if the bound, computed in fp32 in sqdist's operation
order, never exceeds the fp32 squared distance of a point inside the box: then
no point of the node has a smaller distance to the pick than its own, and a
point is lowered only by a strictly smaller one (src/yuezu_fps.cpp:234-265).

The tests restate both computations in NumPy float32 (no contraction: NumPy
rounds each operation) and check the inequality over random boxes and points,
points on the box's faces and corners, picks just outside and inside the box,
and magnitudes from 1e-30 to 1e30 (overflow to inf included).  A bound taken
from the box's centre and half-extent fails them."""

import numpy as np

F = np.float32


def sqdist(p, q):
    d = (p - q).astype(F)
    return ((d[..., 0] * d[..., 0] + d[..., 1] * d[..., 1]).astype(F) + d[..., 2] * d[..., 2]).astype(F)


def box_bound(q, lo, hi):
    below = (lo - q).astype(F)
    above = (q - hi).astype(F)
    g = np.where(below > above, below, above).astype(F)
    g = np.where(g > F(0), g, F(0)).astype(F)
    return ((g[..., 0] * g[..., 0] + g[..., 1] * g[..., 1]).astype(F) + g[..., 2] * g[..., 2]).astype(F)


def check(lo, hi, p, q):
    """p lies in [lo, hi]; the bound of q against the box is <= sqdist(p, q)."""
    assert np.all(p >= lo) and np.all(p <= hi)
    b = box_bound(q, lo, hi)
    d = sqdist(p, q)
    bad = b > d
    assert not bad.any(), (lo[bad][:3], hi[bad][:3], p[bad][:3], q[bad][:3], b[bad][:3], d[bad][:3])


def boxes_points(rs, n, scale):
    c = (rs.standard_normal((n, 3)) * scale).astype(F)
    e = np.abs(rs.standard_normal((n, 3)) * scale * rs.choice([1e-6, 1e-3, 1.0], (n, 1))).astype(F)
    lo = (c - e).astype(F)
    hi = (c + e).astype(F)
    hi = np.maximum(hi, lo)
    t = rs.random_sample((n, 3)).astype(F)
    p = (lo + t * (hi - lo)).astype(F)
    p = np.minimum(np.maximum(p, lo), hi)  # rounding can step outside by an ulp
    return lo, hi, p


def test_bound_never_exceeds_a_point_distance_random():
    rs = np.random.RandomState(11)
    for scale in [1e-30, 1e-6, 1.0, 80.0, 1e6, 1e30]:
        lo, hi, p = boxes_points(rs, 200000, scale)
        q = (rs.standard_normal((200000, 3)) * scale * 3).astype(F)
        check(lo, hi, p, q)


def test_bound_with_points_on_faces_and_corners():
    rs = np.random.RandomState(12)
    n = 200000
    lo, hi, _ = boxes_points(rs, n, 1.0)
    pick = rs.randint(0, 2, (n, 3)).astype(bool)
    p = np.where(pick, lo, hi).astype(F)  # corners
    q = (rs.standard_normal((n, 3)) * 2).astype(F)
    check(lo, hi, p, q)
    face = rs.randint(0, 3, n)
    t = rs.random_sample((n, 3)).astype(F)
    p = (lo + t * (hi - lo)).astype(F)
    p = np.minimum(np.maximum(p, lo), hi)
    on_lo = rs.randint(0, 2, (n, 1)) == 1
    p[np.arange(n), face] = np.where(on_lo, lo, hi)[np.arange(n), face]
    check(lo, hi, p, q)


def test_bound_with_picks_an_ulp_from_the_box():
    rs = np.random.RandomState(13)
    n = 200000
    lo, hi, p = boxes_points(rs, n, 1.0)
    side = rs.randint(0, 2, (n, 3)).astype(bool)
    edge = np.where(side, lo, hi).astype(F)
    towards = np.where(side, F(-np.inf), F(np.inf)).astype(F)
    q = np.nextafter(edge, towards).astype(F)  # one ulp outside each face
    check(lo, hi, p, q)
    q = np.nextafter(edge, -towards).astype(F)  # one ulp inside
    check(lo, hi, p, q)


def test_a_bound_from_centre_and_half_extent_would_fail():
    """The same property for a plausible wrong bound (centre / half-extent
    form): it exceeds some point's distance, so the checks above can tell."""
    rs = np.random.RandomState(14)
    n = 200000
    lo, hi, p = boxes_points(rs, n, 1.0)
    q = (rs.standard_normal((n, 3)) * 3).astype(F)
    c = ((lo + hi) * F(0.5)).astype(F)
    e = ((hi - lo) * F(0.5)).astype(F)
    g = (np.abs((q - c).astype(F)) - e).astype(F)
    g = np.where(g > F(0), g, F(0)).astype(F)
    wrong = ((g[:, 0] * g[:, 0] + g[:, 1] * g[:, 1]).astype(F) + g[:, 2] * g[:, 2]).astype(F)
    assert np.any(wrong > sqdist(p, q))
