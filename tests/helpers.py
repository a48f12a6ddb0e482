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


def special_f32_blocks(n):
    """fp32 blocks of n elements for the quantizers' edge rules: a NaN element
    (x*id is NaN), all NaN, an Inf (amax = Inf, id = 0, Inf*0 = NaN), a tiny
    amax (127/amax overflows to Inf: positive elements give x*id = +Inf, zero
    elements 0*Inf = NaN), a subnormal amax, -Inf elements, values near
    FLT_MAX, a -NaN element, and an ordinary block.  NaNs are the default quiet
    NaN (0x7FC00000 / 0xFFC00000)."""
    t = np.linspace(-1.0, 1.0, n, dtype=np.float32)
    b = np.zeros((9, n), np.float32)
    b[0] = 3.0 * t; b[0, 5] = np.nan
    b[1, :] = np.nan
    b[2] = t; b[2, 9] = np.inf
    b[3] = np.float32(1e-38) * np.sign(t)                         # amax < 127/FLT_MAX: id = +Inf
    b[4] = np.float32(1e-45) * (np.arange(n) % 3 - 1).astype(np.float32)  # subnormal amax
    b[5, ::2] = -np.inf
    b[6] = np.float32(3.4e38) * t
    b[7, 3] = -np.nan
    b[8] = 2.5 * t
    return b.reshape(-1)
