"""Comparison helpers shared by the tests."""
import numpy as np


def to_np(t):
    return t.detach().cpu().numpy()


def bits_mismatch(a, b, nan_equal=False):
    """Indices where the binary32 bit patterns differ (optionally NaN == NaN)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    assert a.shape == b.shape, (a.shape, b.shape)
    diff = a.view(np.uint32) != b.view(np.uint32)
    if nan_equal:
        diff &= ~(np.isnan(a) & np.isnan(b))
    return np.flatnonzero(diff)


def assert_bits_equal(a, b, what="", nan_equal=False):
    bad = bits_mismatch(a, b, nan_equal)
    if bad.size:
        i = bad[:5]
        raise AssertionError(f"{what}: {bad.size}/{np.size(a)} values differ; first at {i.tolist()}: "
                             f"got {np.asarray(a).ravel()[i].tolist()} want {np.asarray(b).ravel()[i].tolist()}")


def ulp_dist(a, b):
    """|ULP| distance on the ordered binary32 line (signed zeros are 0 apart)."""
    def key(x):
        i = np.ascontiguousarray(x, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(key(a) - key(b))
