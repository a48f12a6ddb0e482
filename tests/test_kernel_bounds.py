"""Host-side replay of the kernels' launch geometry and address arithmetic.

For every shape the GPU tests use (and edge shapes: one row, spare waves in the
last workgroup, K = 0, ragged tails) this recomputes, lane by lane, the byte
ranges each kernel reads and writes and checks they stay inside the tensors.
It mirrors the index formulas of bpd_substrate_amd/csrc/*.hip and the launch
choices of their launchers; a change there must be mirrored here.  No GPU.
"""
import numpy as np
import pytest

Q4K, Q8K, Q80 = 144, 292, 34


def lanes():
    return np.arange(64)


# ---------------------------------------------------------------- Q4_K x Q8_K GEMV

def span_rows_per_wave(rows):
    """span_rows_per_wave() in q4k.hip."""
    return 1 if rows <= 2048 else 2


def q4k_gemv_shape(rows, nb):
    """(kind, R, G, WPB) as launch_gemv_order() in q4k.hip picks it for 16-byte
    aligned weights (kind 2: k_q4k_q8k_gemv_span)."""
    if nb == 16:
        return (2, span_rows_per_wave(rows), 1, 4)
    if nb > 16:
        return (1, 2, 1, 4)
    return (1, 1, 1, 8) if rows <= 8192 else (0, 2, 2, 4)


def x_accesses(c):
    """(offset, bytes) of every Q8_K access load_x makes for chunk c (both element maps)."""
    return ((0, 4), (260 + 4 * c, 4), (4 + 32 * c, 16), (4 + 32 * c + 16, 16),
            (4 + 64 * (c >> 1) + 16 * (c & 1), 16), (4 + 64 * (c >> 1) + 16 * (c & 1) + 32, 16))


def q6x_accesses(c, order):
    """(offset, bytes) of every Q8_K access q6x_load_raw makes for lane group c."""
    if order == 0:
        g0, e0 = 2 * c, 32 * c
        g1, e1 = g0 + 1, e0 + 16
    else:
        h, p = c >> 2, c & 3
        g0, e0 = 8 * h + p, 128 * h + 16 * p
        g1, e1 = g0 + 4, e0 + 64
    return ((0, 4), (4 + e0, 16), (4 + e1, 16), (260 + 2 * g0, 2), (260 + 2 * g1, 2))


def check_wide(M, nb, row0, R, G):
    w_size, x_size = M * nb * Q4K, nb * Q8K
    l = lanes()
    q, c = l >> 3, l & 7
    for t0 in range(0, (nb + 7) >> 3, G):
        for g in range(G):
            b = (t0 + g) * 8 + q
            bb = np.where(b < nb, b, nb - 1)
            for r in range(R):
                base = min(row0 + r, M - 1) * nb * Q4K + bb * Q4K
                assert (base + 16 + 16 * c + 16).max() <= w_size and base.min() >= 0
                assert (base + 4 * (c & 3) + 4).max() <= w_size
            for off, size in x_accesses(c):
                assert np.max(bb * Q8K + off + size) <= x_size and np.min(bb * Q8K + off) >= 0


def check_span(M, nb, row0, R, joint=True):
    """span_issue / span_rows of Span<NB=nb, R, JOINT> in q4k.hip for the wave
    whose first row is row0 of an M-row matrix (joint: R consecutive rows as one
    span; otherwise R one-row spans of different matrices, here rows row0 of R
    matrices of M rows): the 16-byte pieces (clamped to the tensor), the slot of
    whole loads, the 4-lane mapping's LDS reads (block clamped to nb-1), the
    load count each pass waits for, and span_load_x's Q8_K reads."""
    w_size, x_size = M * nb * Q4K, nb * Q8K
    segs = 1 if joint else R
    seg_pieces = (R if joint else 1) * nb * 9
    seg_loads = (seg_pieces + 63) // 64
    loads = segs * seg_loads
    slot = loads * 64 * 16
    l = lanes()
    bl, c4 = l >> 2, l & 3
    for g in range(segs):
        np_ = min(R, M - row0) * nb * 9 if joint else nb * 9
        span = row0 * nb * Q4K
        for u in range(seg_loads):
            p = np.minimum(l + 64 * u, np_ - 1)
            assert (span + 16 * p).min() >= 0 and (span + 16 * p + 16).max() <= w_size
            assert (16 * (l + 64 * (g * seg_loads + u)) + 16).max() <= slot
    for r in range(R):
        for t in range((nb + 15) // 16):
            end = min(16 * t + 16, nb)
            need = ((r * nb + end) * 9 + 63) // 64 if joint else r * seg_loads + (end * 9 + 63) // 64
            assert need <= loads
            row_off = r * nb * Q4K if joint else r * seg_loads * 1024
            bb = np.minimum(16 * t + bl, nb - 1)
            blk = row_off + bb * Q4K
            # every piece the pass reads lies in a load it waited for
            assert ((blk + 144) <= need * 1024).all()
            assert (blk + 16).max() <= slot
            assert (blk + 16 + 16 * c4 + 16).max() <= slot and (blk + 80 + 16 * c4 + 16).max() <= slot
    for t in range((nb + 15) // 16):
        b = np.minimum(16 * t + bl, nb - 1)
        for c in (c4, c4 + 4):
            for off, size in x_accesses(c):
                assert np.max(b * Q8K + off + size) <= x_size and np.min(b * Q8K + off) >= 0


def check_four(M, nb, row0, R):
    w_size, x_size = M * nb * Q4K, nb * Q8K
    l = lanes()
    bl, c4 = l >> 2, l & 3
    chunk = 4 * (l >> 5) + c4
    assert chunk.max() < 8
    for t in range((nb + 15) >> 4):
        b = 16 * t + bl
        bb = np.minimum(b, nb - 1)
        off_a = np.minimum(16 * t + (bl & 7), nb - 1) * Q4K + 16 + 16 * chunk
        off_b = np.minimum(16 * t + 8 + (bl & 7), nb - 1) * Q4K + 16 + 16 * chunk
        for r in range(R):
            rb = min(row0 + r, M - 1) * nb * Q4K
            for off in (off_a, off_b):
                assert (rb + off + 16).max() <= w_size and (rb + off).min() >= 0
            assert (rb + bb * Q4K + 4 * c4 + 4).max() <= w_size
        for c in (c4, c4 + 4):
            for off, size in x_accesses(c):
                assert np.max(bb * Q8K + off + size) <= x_size and np.min(bb * Q8K + off) >= 0


@pytest.mark.parametrize("M,K", [(4096, 4096), (14336, 4096), (4096, 14336), (1024, 4096), (1, 256), (5, 512),
                                 (13, 2304), (9, 2304), (3, 0), (64, 1024), (77, 512), (6144, 4096), (28672, 4096),
                                 (8193, 4096), (17, 4352), (2, 14336)])
@pytest.mark.parametrize("force", [None, (0, 2, 2, 4), (1, 1, 1, 8), (1, 2, 1, 4), (1, 1, 1, 16), (2, 2, 1, 4),
                                   (2, 1, 1, 4)])
def test_q4k_q8k_gemv_in_bounds(M, K, force):
    nb = K // 256
    if nb == 0:
        return  # no block-group pass runs: the kernels read nothing and write y = +0.0
    if force is not None and force[0] == 2 and nb != 16:
        return  # the span kernel is instantiated for K = 4096 only
    kind, R, G, WPB = force or q4k_gemv_shape(M, nb)
    waves = (M + R - 1) // R
    grid = (waves + WPB - 1) // WPB
    for blk in sorted({0, grid - 1}):
        for wave in range(WPB):
            row0 = (blk * WPB + wave) * R
            if row0 >= M:
                continue
            if kind == 0:
                check_wide(M, nb, row0, R, G)
            elif kind == 1:
                check_four(M, nb, row0, R)
            else:
                check_span(M, nb, row0, R)
            for r in range(R):
                if row0 + r < M:
                    assert (row0 + r) * 4 + 4 <= M * 4


@pytest.mark.parametrize("Ms", [[4096, 1024, 1024], [4096, 1024, 1024, 13], [1], [7, 2048], [14336, 14336]])
def test_q4k_multi_span_in_bounds(Ms):
    """k_q4k_q8k_multi_span / k_q4k_fused_span at K = 4096: every wave of every
    matrix (waves past the last row read row 0 of a non-empty matrix)."""
    nb = 16
    R = span_rows_per_wave(sum(Ms))
    for M in Ms:
        for row0 in range(0, M, R):
            check_span(M, nb, row0, R)
        check_span(M, nb, 0, R)


@pytest.mark.parametrize("nb,R,M", [(56, 1, 1), (56, 1, 7), (56, 1, 4096), (16, 2, 16384), (16, 2, 28672),
                                    (16, 2, 16385)])
def test_q4k_fused_span_pass_buffer_in_bounds(nb, R, M):
    """k_q4k_fused_span<ORDER, NB, R, WPB, PB = true> (K = 14336 one row per wave; K = 4096
    from 16,384 rows, two rows per wave): the rows' pieces as loads, each pass's pieces
    copied into a 16-block buffer and read back there."""
    buf = 16 * Q4K
    for row0 in sorted({0, ((M - 1) // R) * R}):
        check_span(M, nb, row0, R)  # global reads and x reads are those of the slot form
        l = lanes()
        bl = l >> 2
        pieces = R * nb * 9
        covered = np.zeros(pieces, bool)
        for r in range(R):
            for t in range((nb + 15) // 16):
                p0, n = (r * nb + 16 * t) * 9, min(16, nb - 16 * t) * 9
                for u in range((pieces + 63) // 64):
                    q = l + 64 * u - p0
                    ok = (q >= 0) & (q < n)
                    assert (16 * q[ok] + 16 <= buf).all()
                    covered[(l + 64 * u)[ok & (l + 64 * u < pieces)]] = True
                bb = np.minimum(16 * t + bl, nb - 1) - 16 * t
                assert (bb >= 0).all() and ((bb * Q4K + 144) <= buf).all()
                assert ((bb * Q4K + 144) <= n * 16).all()  # only the pass's own pieces are read
        assert covered.all()


@pytest.mark.parametrize("M", [1, 5, 512, 14336])
def test_q4k_swiglu_span_in_bounds(M):
    """k_q4k_swiglu_span: row r of gate and of up as two one-row spans."""
    for row in sorted({0, M - 1, M // 2}):
        check_span(M, 16, row, 2, joint=False)


@pytest.mark.parametrize("M", [1, 7, 64, 14336])
def test_q6k_span_in_bounds(M):
    """k_q6k_q8k_gemv_span (K = 4096, two rows per wave): the span pieces (clamped to
    the tensor), each pass's 105 pieces in the 1,680-byte buffer, the 2-byte-aligned
    operand words read as whole aligned dwords inside the buffer, the Q8_K reads."""
    Q6, nb, R, buf = 210, 16, 2, 8 * 210 + 16
    w_size, x_size = M * nb * Q6, nb * Q8K
    pieces = R * nb * Q6 // 16
    loads = (pieces + 63) // 64
    l = lanes()
    q, c = l >> 3, l & 7
    for row0 in sorted({0, ((M - 1) // R) * R}):
        np_ = min(R, M - row0) * nb * Q6 // 16
        span = row0 * nb * Q6
        for u in range(loads):
            p = np.minimum(l + 64 * u, np_ - 1)
            assert (span + 16 * p).min() >= 0 and (span + 16 * p + 16).max() <= w_size
        covered = np.zeros(pieces, bool)
        for r in range(R):
            for t in range(nb // 8):
                p0, n = (r * nb + 8 * t) * Q6 // 16, 8 * Q6 // 16
                assert (r * nb + 8 * t) * Q6 % 16 == 0
                for u in range(loads):
                    if 64 * u + 63 < p0 or 64 * u >= p0 + n:
                        continue
                    k = l + 64 * u - p0
                    ok = (k >= 0) & (k < n)
                    slot = np.where(ok, k, n)            # lanes outside the pass: the spare slot n
                    assert (16 * slot + 16 <= buf).all()
                    covered[(l + 64 * u)[ok & (l + 64 * u < pieces)]] = True
        assert covered.all()
    blk = q * Q6
    for order in (0, 1):
        if order == 0:
            spans = [(blk + 16 * c, 4), (blk + 128 + 8 * c, 2)]
            groups = (2 * c, 2 * c + 1)
        else:
            h, pp = c >> 2, c & 3
            spans = [(blk + 64 * h + 16 * pp, 4), (blk + 128 + 32 * h + 16 * (pp & 1), 4)]
            groups = (8 * h + pp, 8 * h + pp + 4)
        for addr, nw in spans:
            assert ((addr & 3) % 2 == 0).all()
            assert (((addr & ~3) + 4 * (nw + 1)) <= buf).all()   # nw + 1 aligned dwords
            assert ((addr + 4 * nw) <= 8 * Q6).all()              # the words themselves lie in the pass
        for g in groups:
            assert ((blk + 192 + g + 1) <= 8 * Q6).all()
        assert ((blk + 210) <= 8 * Q6).all()
        for t in range(nb // 8):
            xb = (8 * t + q) * Q8K
            for off, size in x_accesses(c):
                assert np.max(xb + off + size) <= x_size
            for g in groups:
                assert np.max(xb + 260 + 2 * g + 2) <= x_size


@pytest.mark.parametrize("M", [1, 5, 8, 9, 17, 4096])
def test_q6k_span_long_in_bounds(M):
    """k_q6k_q8k_gemv_span_long (K = 14336, one row per wave, 8 waves per workgroup):
    the x records (thread t < 448 loads the Q8_K bytes of super-block t/8, lane group
    t%8 -- threads past them record 447's, clamped -- and stores one 20-dword record),
    the 735 pieces of a row (clamped at the last piece; spare waves read row M-1 and
    store nothing), each of the 7 passes' 105 pieces inside the 1,696-byte pass
    buffer (lanes outside the pass write the spare slot 105) and covered by the
    loads, and each pass's record read."""
    Q6, NB, WPB, buf = 210, 56, 8, 8 * 210 + 16
    pieces, loads = NB * Q6 // 16, (NB * Q6 // 16 + 63) // 64
    assert pieces * 16 == NB * Q6 and (pieces, loads) == (735, 12)
    XR, REC = NB * 8, 20
    assert XR <= 64 * WPB
    tid = np.arange(64 * WPB)
    rt = np.minimum(tid, XR - 1)
    for order in (0, 1):
        for off, size in q6x_accesses(rt & 7, order):
            assert np.max((rt >> 3) * Q8K + off + size) <= NB * Q8K and np.min(off) >= 0
            assert np.max(off + size) <= Q8K                  # inside the record's super-block
    st = tid[tid < XR]
    assert (st * REC + 18).max() < XR * REC and len(set((st * REC).tolist())) == XR
    grid = (M + WPB - 1) // WPB
    w_size = M * NB * Q6
    l = lanes()
    for blk in sorted({0, grid - 1}):
        for wave in range(WPB):
            row = blk * WPB + wave
            span = (row if row < M else M - 1) * NB * Q6
            for u in range(loads):
                p = np.minimum(l + 64 * u, pieces - 1)
                assert span + 16 * p.min() >= 0 and span + 16 * p.max() + 16 <= w_size
    covered = np.zeros(pieces, bool)
    for t in range(NB // 8):
        assert 8 * t * Q6 % 16 == 0
        p0, n = 8 * t * Q6 // 16, 8 * Q6 // 16
        for u in range(loads):
            if 64 * u + 63 < p0 or 64 * u >= p0 + n:
                continue
            k = l + 64 * u - p0
            ok = (k >= 0) & (k < n)
            assert (16 * np.where(ok, k, n) + 16 <= buf).all()
            covered[(l + 64 * u)[ok]] = True
        q, c = l >> 3, l & 7
        rec = ((8 * t + q) * 8 + c) * REC
        assert (rec + 18).max() < XR * REC and rec.min() >= 0
    assert covered.all()


# ---------------------------------------------------------------- dequant

@pytest.mark.parametrize("nb", [1, 7, 33, 65536, 4096])
def test_dequant_in_bounds(nb):
    grid = (nb + 3) // 4
    for blk in {0, grid - 1}:
        for wave in range(4):
            b = blk * 4 + wave
            if b >= nb:
                continue
            l = lanes()
            assert b * Q4K + 16 + 4 * 31 + 4 <= nb * Q4K
            assert (b * 256 + 4 * l + 4).max() <= nb * 256


# ---------------------------------------------------------------- Q8_0 tile-order GEMV

V_PITCH, V_SCP, V_ROWS = 1248, 12, 2
V_SLOT = V_ROWS * V_PITCH + 4 * V_ROWS * V_SCP * 4


def v_xpitch(nb):
    return nb // 4 + 4


def v_lds(nb, nw):
    return (32 * v_xpitch(nb) + nb) * 4 + nw * V_SLOT


def q8_wide_config(mw, mt, nb):
    """(NW, XR) of k_q8_0_gemv_V as launch_wide() in q8_0.hip picks it for a
    16-byte aligned W, or None."""
    if nb == 0 or nb % 32 != 0:
        return None
    waves = -(-mw // V_ROWS) * mt
    if waves < 256:
        return None
    xr = lambda nw: next((x for x in (4, 8, 16, 32) if nb * 8 <= x * 64 * nw), None)
    nw = 4
    XR = xr(nw)
    if XR is None:
        nw = 8
        XR = xr(nw)
    if XR is None or v_lds(nb, nw) > 160 * 1024:
        return None
    return nw, XR


def check_wide_q8(mw, mt, nb, w_size, x_size, out_size):
    """k_q8_0_gemv_V: lane l of wave w in workgroup g (rows row0 = 2(g*NW + w) ..)
    reads 16-byte piece f = min(l + 64k, 135) (k < 3, every lane) -- row f/68,
    bytes 1088c + 16(f%68) of that row (rows past mw re-read row mw-1) -- for
    chunks c < nb/32, and the first 16 bytes of row row0c for the steps past the
    last chunk; it writes piece f at (f/68)*1248 + 16(f%68) of the wave's slot
    (lanes with l + 64k < 136); the scale pass (lane j: r = j/32,
    bb = j%32) reads the 16-bit scale at r*1248 + 34bb and writes
    sc[(4r + bb%4)*12 + bb/4]; lane (row, L, q) reads the dwords at 34bb + oa and
    34bb + oa + 4 of its row's chunk (bb % 4 == 0, oa = (34q + 2 + 4L) & ~3), four
    x dwords at (4L + q)*(nb/4 + 4) + 8c + b16/4 and four products at
    (4row + q)*12 + b16/4; the activation is quant dword min(i, 8nb-1) and scale
    min(j, nb-1)."""
    NW, XR = q8_wide_config(mw, mt, nb)
    NT, bpr, nch, xp = 64 * NW, nb * Q80, nb // 32, v_xpitch(nb)
    l = np.arange(64)
    groups = -(-mw // (V_ROWS * NW))
    for g in sorted({0, groups - 1}):
        for w in range(NW):
            row0 = (g * NW + w) * V_ROWS
            row0c = min(row0, mw - 1)
            assert row0c * bpr + 16 <= w_size
            for k in range(3):
                f = np.minimum(l + 64 * k, 135)
                r, pc = f // 68, f % 68
                off = (np.minimum(row0 + r, mw - 1) - row0c) * bpr + 16 * pc
                for c in (0, nch - 1):
                    a = row0c * bpr + off + c * 1088
                    assert a.min() >= 0 and (a + 16).max() <= w_size
                fw = np.minimum(l + 64 * k, 135)[l + 64 * k < 136]
                assert ((fw // 68) * V_PITCH + 16 * (fw % 68) + 16).max() <= V_ROWS * V_PITCH
    r, bb = l // 32, l % 32
    assert (r * V_PITCH + 34 * bb + 2).max() <= V_ROWS * V_PITCH
    assert ((4 * r + bb % 4) * V_SCP + bb // 4).max() < 4 * V_ROWS * V_SCP
    assert (nch - 1) * 32 + bb.max() < nb
    q, L, rr = l & 3, (l >> 2) & 7, l >> 5
    oa = (34 * q + 2 + 4 * L) & ~3
    for bb in range(0, 32, 4):
        assert (34 * bb + oa + 8).max() <= V_PITCH
    for b16 in (0, 16):
        xi = (4 * L + q) * xp + 8 * (nch - 1) + b16 // 4
        assert (xi + 4).max() <= 32 * xp
        si = (4 * rr + q) * V_SCP + b16 // 4
        assert (si + 4).max() <= 4 * V_ROWS * V_SCP
    i = np.minimum(np.arange(XR * NT), nb * 8 - 1)
    jd = np.minimum(np.arange(-(-XR // 8) * NT), nb - 1)
    assert nb <= -(-XR // 8) * NT
    for tok in range(mt):
        assert tok * bpr + ((i >> 3) * Q80 + 2 + 4 * (i & 7) + 4).max() <= x_size
        assert tok * bpr + (jd * Q80 + 2).max() <= x_size
    st = np.arange(XR * NT)
    st = st[st < nb * 8]
    b = st >> 3
    assert ((4 * (st & 7) + (b & 3)) * xp + (b >> 2)).max() < 32 * xp
    # 16-byte alignment of every vector LDS access: slots, x rows, product rows
    assert ((32 * xp + nb) * 4) % 16 == 0 and V_SLOT % 16 == 0 and (V_ROWS * V_PITCH) % 16 == 0
    assert (xp * 4) % 16 == 0 and (V_SCP * 4) % 16 == 0 and (8 * (nch - 1) * 4) % 16 == 0
    assert (mt - 1) * mw * 4 + mw * 4 <= out_size
    assert v_lds(nb, NW) <= 160 * 1024


def q8_gemv_config(mw, mt, K):
    nb = K // 32
    waves = (mw + 7) // 8
    if nb == 0:
        return None
    if q8_wide_config(mw, mt, nb) is not None:
        return ("wide", 0, 0)
    if nb * 36 > 64 * 1024:
        return ("plain", 4, 1)
    if waves * mt >= 1024:
        return ("pipelined", 4, 16)
    if nb * 36 + 2 * 64 * 36 * 4 <= 64 * 1024:
        return ("producer", 5, 32)
    return ("pipelined", 2, 32)


def check_producer(mw, mt, nb, layout, w_size):
    """k_q8_0_gemv_TP: producer lane p of workgroup g reads block min(c*32 + p%32,
    nb-1) of row min(8g + p/32, mw-1) for chunks c < nch, bytes [blk, blk+34)
    (34-byte blocks: 8 dwords from blk+2 for odd b, from blk for even b, plus a
    16-bit word at blk or blk+32) or [blk, blk+36) (padded records)."""
    nch = (nb + 31) // 32
    groups = (mw + 7) // 8
    p = np.arange(256)
    for g in sorted({0, groups - 1}):
        row = np.minimum(8 * g + (p >> 5), mw - 1)
        for c in range(nch):
            b = np.minimum(c * 32 + (p & 31), nb - 1)
            if layout == 0:
                blk = row * nb * Q80 + b * Q80
                lo, hi = blk, blk + 34
            else:
                blk = b * mw * 64 + row * 64
                lo, hi = blk, blk + 36
            assert lo.min() >= 0 and hi.max() <= w_size
        # products: (row8 + L) * 36 + j inside the two 64 x 36 slots; consumer lane t reads t*36 .. +32
        assert ((p >> 5) * 8 + 7) .max() * 36 + 31 < 64 * 36
        orow = 8 * g + (np.arange(64) >> 3)
        assert ((orow[orow < mw]) * 4 + 4).max(initial=0) <= mw * 4


@pytest.mark.parametrize("mw,mt,K", [(14336, 1, 4096), (4096, 1, 14336), (4, 2, 128), (7, 5, 128), (9, 7, 128),
                                     (2048, 2, 2048), (1, 1, 32), (13, 3, 4128), (64, 4, 256), (6, 3, 96),
                                     (3, 1, 64), (17, 1, 32), (15, 1, 256), (23, 1, 256), (7, 1, 256),
                                     (8192, 2, 1024), (8200, 3, 8192), (2048, 1, 8192), (9000, 1, 2048),
                                     (14336, 4, 4096), (2056, 1, 16384), (8192, 1, 32768), (2048, 1, 32768),
                                     (4096, 4, 4096), (4096, 2, 14336), (512, 1, 8192),
                                     (4100, 1, 4096), (1024, 1, 14336), (2048, 1, 4096), (512, 1, 65536),
                                     (513, 1, 3072), (28672, 1, 4096), (4097, 3, 1024)])
def test_q8_0_gemv_T_in_bounds(mw, mt, K):
    cfg = q8_gemv_config(mw, mt, K)
    nb = K // 32
    bpr = nb * Q80
    w_size, x_size, out_size = mw * bpr, mt * bpr, mw * mt * 4
    if cfg is None:
        return
    kind, WPB, U = cfg
    if kind == "wide":
        check_wide_q8(mw, mt, nb, w_size, x_size, out_size)
        return
    if kind == "producer":
        check_producer(mw, mt, nb, 0, w_size)
        for tok in range(mt):
            assert tok * bpr + (nb - 1) * Q80 + 2 + 28 + 4 <= x_size
        return
    waves = (mw + 7) // 8
    grid = (waves + WPB - 1) // WPB if kind == "pipelined" else (waves + 3) // 4
    l = lanes()
    L = l & 7
    for blk in sorted({0, grid - 1}):
        for wave in range(WPB):
            row = (blk * WPB + wave) * 8 + (l >> 3)
            if kind == "plain":
                continue
            row0 = min((blk * WPB + wave) * 8, mw - 1)
            doff = (np.maximum(np.minimum(row, mw - 1), row0) - row0) * bpr
            assert doff.min() >= 0
            voff = doff + 2 + 4 * L
            for b0 in range(0, nb + 2 * U, U):
                for u in range(U):
                    b = min(b0 + u, nb - 1)
                    base = row0 * bpr + b * Q80
                    assert (base + voff + 4).max() <= w_size and (base + doff).min() >= 0
                    assert (base + doff + 2).max() <= w_size
            for tok in range(mt):
                assert tok * bpr + (nb - 1) * Q80 + 2 + 28 + 4 <= x_size
                ok = row < mw
                assert ((tok * mw + row[ok]) * 4 + 4).max(initial=0) <= out_size


# ---------------------------------------------------------------- Q8_0 S-order GEMM (MFMA)

@pytest.mark.parametrize("mw,mt,K", [(14336, 512, 4096), (4, 2, 128), (7, 5, 128), (130, 129, 4096 + 32),
                                     (1, 1, 32), (256, 256, 64), (300, 17, 224)])
def test_q8_0_gemm_S_in_bounds(mw, mt, K):
    nb = K // 32
    if nb == 0:
        return
    bpr = nb * Q80
    gx, gy = (mw + 127) // 128, (mt + 127) // 128
    t = np.arange(256)
    for bx in {0, gx - 1}:
        for by in {0, gy - 1}:
            m0, n0 = bx * 128, by * 128
            for b0 in range(0, nb + 4, 4):
                for i in range(2):
                    p = t + 256 * i
                    rr, u = p & 127, p >> 7
                    blk = np.minimum(b0 + u, nb - 1)
                    wa = np.minimum(m0 + rr, mw - 1) * bpr + blk * Q80
                    xa = np.minimum(n0 + rr, mt - 1) * bpr + blk * Q80
                    assert wa.min() >= 0 and (wa + 34).max() <= mw * bpr
                    assert xa.min() >= 0 and (xa + 34).max() <= mt * bpr
                    assert u.max() < 4 and rr.max() < 128


# ---------------------------------------------------------------- fused Q8_K quantization prologue

def fused_config(rows, nb):
    """(WPB, IT) of launch_qmatmul_q4k_fused_multi in q4k.hip."""
    return (4, 1) if nb <= 16 else (16, 1)


@pytest.mark.parametrize("rows", [1, 300, 8192, 8193, 14336, 28672])
def test_fused_quantization_covers_x_and_stays_in_bounds(rows):
    for nb in range(1, 65):  # fused_max_k() = 64 * 256
        WPB, IT = fused_config(rows, nb)
        assert IT * 4 * WPB >= nb, "some Q8_K block would never be quantized"
        tid = np.arange(64 * WPB)
        gq, li = tid >> 4, tid & 15
        for it in range(IT):
            b = np.minimum(it * 4 * WPB + gq, nb - 1)
            assert ((b * 256 + 16 * li + 16) <= nb * 256).all() and (b >= 0).all()
            bw = it * 4 * WPB + gq
            ok = bw < nb
            assert ((bw[ok] * 304 + 16 * li[ok] + 16) <= nb * 304).all()
            assert ((bw[ok] * 304 + 288 + 4) <= nb * 304).all()


# ---------------------------------------------------------------- Q8_0 S-order GEMM, coalesced staging

@pytest.mark.parametrize("mw,mt,K", [(14336, 512, 4096), (130, 129, 4096), (1, 1, 128), (300, 17, 384), (256, 256, 128),
                                     (7, 5, 14336), (225, 3, 256), (4096, 512, 14336), (4100, 512, 768)])
@pytest.mark.parametrize("RT", [4, 2, 1])
@pytest.mark.parametrize("CT", [2, 1])
def test_q8_0_gemm_SH_in_bounds(mw, mt, K, RT, CT):
    """k_q8_0_gemm_SH<RT, CT>: 32*RT weight rows x 128 tokens per workgroup of
    NT = 64*RT*(4/CT) threads (waves of 32 rows x 32*CT tokens), staged in
    h_passes passes of NT staging threads (a thread pair per weight row and per
    token); every staged row and part covered once."""
    assert K % 128 == 0  # the launcher's condition for this kernel
    nb = K // 32
    bpr = nb * Q80
    wcn = 4 // CT
    nt = 64 * RT * wcn
    passes = (64 * RT + 256 + nt - 1) // nt
    t_all = np.arange(passes * nt)
    stored = t_all[t_all < 64 * RT + 256]
    assert len(stored) == 64 * RT + 256 and len(set(stored.tolist())) == len(stored)
    t = np.minimum(t_all, 64 * RT + 255)
    p, wrow = t & 1, t < 64 * RT
    row = np.where(wrow, t >> 1, (t - 64 * RT) >> 1)
    assert row.max() < max(32 * RT, 128)
    rows = 32 * RT
    for bx in {0, (mw + rows - 1) // rows - 1}:
        for by in {0, (mt + 127) // 128 - 1}:
            m0, n0 = bx * rows, by * 128
            for b0 in range(0, nb, 4):
                r = np.where(wrow, np.minimum(m0 + row, mw - 1), np.minimum(n0 + row, mt - 1))
                size = np.where(wrow, mw * bpr, mt * bpr)
                src = r * bpr + (b0 + 2 * p) * Q80
                assert (src >= 0).all() and ((src + 4 * 16 + 4) <= size).all()
                assert ((b0 + 2 * p + 1) < nb).all()  # both staged blocks exist
    # LDS: staged rows inside qa / qb and da / db; the scale operand rows (lanes
    # 32-63: the zero rows 32*RT and 128, which the arrays hold as their last row)
    lane = np.arange(64)
    col, half = lane & 31, lane >> 5
    cover = np.zeros((32 * RT, 128), dtype=int)
    for wave in range(RT * wcn):
        wr, wc = wave // wcn, wave % wcn
        ra = wr * 32 + col
        za = np.where(half == 1, 32 * RT, ra)
        assert za.max() <= 32 * RT and ra.max() < 32 * RT
        for ct in range(CT):
            cb = wc * 32 * CT + ct * 32 + col
            assert cb.max() < 128 and np.where(half == 1, 128, cb).max() <= 128
            cover[wr * 32:(wr + 1) * 32, wc * 32 * CT + ct * 32:wc * 32 * CT + ct * 32 + 32] += 1
    assert (cover == 1).all()  # every (row, token) of the tile computed by one wave


def h_swz(row, b):
    return ((row >> 2) ^ (row >> 3) ^ (b >> 1)) & 1


def test_q8_0_gemm_SH_swizzle():
    """The quant halves' swizzle: the writer of blocks 2p, 2p+1 and the reader of
    block u agree, and 16 consecutive lanes' 16-byte operand reads (one block,
    rows r..r+15, one half) and 16 consecutive lanes' staging writes (rows
    r..r+7, both parts) fall in 16 different 16-byte groups modulo 256 bytes."""
    rows = np.arange(256)
    for p in (0, 1):
        assert (h_swz(rows, 2 * p) == h_swz(rows, 2 * p + 1)).all()
    for u in range(4):
        for half in (0, 1):
            for r0 in range(0, 256, 16):
                r = np.arange(r0, r0 + 16)
                byte = (u * 128 + r) * 32 + 16 * (half ^ h_swz(r, u))
                assert len(set((byte % 256) // 16)) == 16
    t = np.arange(512)
    p, row = t & 1, t >> 1
    for h in (0, 1):
        byte = (2 * p * 128 + row) * 32 + 16 * (h ^ h_swz(row, 2 * p))
        for g in range(0, 512, 16):
            assert len(set((byte[g:g + 16] % 256) // 16)) == 16


# ---------------------------------------------------------------- Q6_K

Q6K = 210


@pytest.mark.parametrize("nb", [1, 3, 5, 4096])
@pytest.mark.parametrize("order", [0, 1])
def test_dequant_q6k_in_bounds(nb, order):
    l = lanes()
    for b in {0, nb - 1}:
        base = b * Q6K
        if order == 0:
            spans = [(2 * l, 2), (128 + l, 1)]
        else:
            e0 = 4 * l
            h, r = e0 >> 7, e0 & 127
            quarter, idx = r >> 5, r & 31
            spans = [(64 * h + 32 * (quarter & 1) + idx, 4), (128 + 32 * h + idx, 4)]
        spans += [(192 + (l >> 2), 1), (np.full(64, 208), 2)]
        for off, size in spans:
            assert (base + off + size).max() <= nb * Q6K and (base + off).min() >= 0
            assert (off + size).max() <= Q6K          # never reads into the next block


@pytest.mark.parametrize("M,K", [(1, 256), (5, 512), (64, 4096), (17, 14336), (3, 2304), (3, 0)])
@pytest.mark.parametrize("order", [0, 1])
def test_q6k_gemv_in_bounds(M, K, order):
    nb = K // 256
    if nb == 0:
        return
    R, WPB = 2, 4
    waves = (M + R - 1) // R
    grid = (waves + WPB - 1) // WPB
    c = lanes() & 7
    if order == 0:
        w_spans = [(16 * c, 16), (128 + 8 * c, 8), (192 + 2 * c, 1), (192 + 2 * c + 1, 1), (np.full(64, 208), 2)]
        x_spans = [(4 + 32 * c + 4 * j, 4) for j in range(8)]
        groups = [2 * c, 2 * c + 1]
    else:
        h, p = c >> 2, c & 3
        e0 = 128 * h + 16 * p
        w_spans = [(64 * h + 16 * p, 16), (128 + 32 * h + 16 * (p & 1), 16), (192 + 8 * h + p, 1),
                   (192 + 8 * h + p + 4, 1), (np.full(64, 208), 2)]
        x_spans = [(4 + e0 + 4 * k, 4) for k in range(4)] + [(4 + e0 + 64 + 4 * k, 4) for k in range(4)]
        groups = [8 * h + p, 8 * h + p + 4]
    x_spans += [(260 + 2 * g, 2) for g in groups] + [(np.zeros(64, int), 4)]
    for off, size in w_spans:
        assert (off + size).max() <= Q6K
    for off, size in x_spans:
        assert (off + size).max() <= Q8K
    assert all(np.max(g) < 16 for g in groups)
    for blk in sorted({0, grid - 1}):
        for wave in range(WPB):
            row0 = (blk * WPB + wave) * R
            if row0 >= M:
                continue
            for r in range(R):
                assert min(row0 + r, M - 1) < M


@pytest.mark.parametrize("mw,mt,K", [(4096, 1, 14336), (14336, 1, 4096), (13, 3, 160), (8, 1, 32), (9, 2, 64), (7, 5, 128)])
def test_q8_pad64_gemv_in_bounds(mw, mt, K):
    """k_q8_0_gemv_T<.., 1> / k_q8_0_gemm_T<1>: W records (b, n) at (b*mw + n)*64."""
    cfg = q8_gemv_config(mw, mt, K)
    if cfg is None:
        return
    nb = K // 32
    w_size = nb * mw * 64
    kind, WPB, U = cfg
    if kind == "producer":
        check_producer(mw, mt, nb, 1, w_size)
        return
    waves = (mw + 7) // 8
    grid = (waves + WPB - 1) // WPB if kind == "pipelined" else (waves + 3) // 4
    l = lanes()
    L = l & 7
    for blk in sorted({0, grid - 1}):
        for wave in range(WPB):
            row = (blk * WPB + wave) * 8 + (l >> 3)
            row0 = min((blk * WPB + wave) * 8, mw - 1)
            doff = (np.maximum(np.minimum(row, mw - 1), row0) - row0) * 64
            voff = doff + 4 + 4 * L
            for b0 in range(0, nb + 2 * U, U):
                for u in range(U):
                    b = min(b0 + u, nb - 1)
                    base = row0 * 64 + b * mw * 64
                    assert (base + voff + 4).max() <= w_size and (base + doff).min() >= 0
                    assert (base + doff + 2).max() <= w_size


@pytest.mark.parametrize("N,K", [(1, 32), (7, 96), (300, 4096)])
def test_q8_pad64_conversion_in_bounds(N, K):
    nb = K // 32
    g = np.arange(((N * nb * 32 + 255) // 256) * 256)
    rec, e = g >> 5, g & 31
    live = rec < N * nb
    rec, e = rec[live], e[live]
    n, b = rec // nb, rec % nb
    assert ((rec * 32 + e) < N * K).all()
    o = (b * N + n) * 64
    assert ((o + 4 + e) < N * nb * 64).all() and ((o + 36 + np.minimum(e, 27)) < N * nb * 64).all()


# ---------------------------------------------------------------- bpd_qmm_q4k, qdot grid P

@pytest.mark.parametrize("M,N,K", [(3, 5, 256), (64, 64, 4096), (7, 300, 512), (1, 1, 256), (5, 257, 768)])
def test_qmm_q4k_in_bounds(M, N, K):
    """k_qmm_q4k: grid (ceil(N/256), ceil(M/4)); wave w dequantizes row min(r0+w, M-1),
    thread c reads B[k][min(c, N-1)], stores only c < N and rows < M; the NaN re-walk
    reads the same ranges."""
    nb = K // 256
    a_size, b_size = M * nb * Q4K, K * N
    l = lanes()
    j, dw = l >> 3, 4 * (l >> 3) + (l & 3)
    assert (16 + 4 * dw + 4).max() <= Q4K and (4 * l + 4).max() <= 256
    gx, gy = (N + 255) // 256, (M + 3) // 4
    for by in sorted({0, gy - 1}):
        r0 = by * 4
        for wave in range(4):
            arow = min(r0 + wave, M - 1) * nb * Q4K
            assert arow + (nb - 1) * Q4K + Q4K <= a_size
        for bx in sorted({0, gx - 1}):
            col = bx * 256 + np.arange(256)
            cc = np.minimum(col, N - 1)
            assert ((nb * 256 - 1) * N + cc).max() < b_size and cc.min() >= 0
            for r in range(4):
                if r0 + r < M:
                    assert ((r0 + r) * N + col[col < N]).max() < M * N
    # the NaN re-walk: qs byte 16 + 16j + (k & 15) of each block
    assert 16 + 16 * 7 + 15 < Q4K


@pytest.mark.parametrize("n_rows,M,K", [(14336, 1, 4096), (4096, 1, 14336), (37, 3, 224), (9, 2, 32),
                                        (17, 5, 4128), (1, 1, 64), (8, 1, 52416)])
def test_q8_0_qdot_P_in_bounds(n_rows, M, K):
    """k_q8_0_qdot_P<8, 4>: LDS = 40 nb bytes; lane (L = 4h + i) loads block 2*min(p, np-1)+h
    (<= nb-1) at +2+4i and +18+4i, its scale at +0; the odd tail block's dword L; spare
    rows and waves clamp to row n_rows-1."""
    nb, WPB = K // 32, 4
    np_ = nb // 2
    bpr = nb * Q80
    assert nb * 40 <= 64 * 1024
    l = lanes()
    L, i, h = l & 7, l & 3, (l & 7) >> 2
    assert (2 + 4 * i + 16 + 4).max() <= Q80 and (2 + 4 * L + 4).max() <= Q80
    if np_ > 0:
        assert 2 * (np_ - 1) + 1 <= nb - 1
    waves = (n_rows + 7) // 8
    grid = (waves + WPB - 1) // WPB
    for blk in sorted({0, grid - 1}):
        for wave in range(WPB):
            row = (blk * WPB + wave) * 8 + (l >> 3)
            row0 = min((blk * WPB + wave) * 8, n_rows - 1)
            doff = (np.maximum(np.minimum(row, n_rows - 1), row0) - row0) * bpr
            assert (row0 * bpr + doff).min() >= 0
            last = row0 * bpr + doff + (nb - 1) * Q80 + Q80
            assert last.max() <= n_rows * bpr
            assert ((M - 1) * n_rows + row[row < n_rows]).max(initial=0) < M * n_rows
    # the staged activation row: dword i of element group, i <= nb*8 - 1
    n = nb * 8
    assert ((n - 1) >> 3) * Q80 + 2 + 4 * ((n - 1) & 7) + 4 <= bpr


@pytest.mark.parametrize("M,K", [(16, 256), (16, 4096), (77, 512), (4096, 4096), (300, 256), (14336, 4096),
                                 (64, 2048), (1, 1536), (5, 14336), (3, 16384), (2, 16640), (16, 262144)])
def test_qmatmul_q4k_chain_in_bounds_and_barriers(M, K):
    """k_qmatmul_q4k_chain: chunk c holds sub-blocks 6c..6c+5; producer p loads sub-blocks
    min(6c + 2p + t, nsb - 1) of row min(row0+r, M-1) (header + 16-byte qs slice), reads x of
    elements 32 sb .. 32 sb + 31 and writes prod[c&1][8(2p+t) + g][r] only for sb < nsb;
    the consumer reads the chunk's first min(192, 32(nsb - 6c)) products, exactly what the
    producers wrote; consumer and producers each pass nch barriers (plus the x-staging one)."""
    nb, rows, ahead, sbc = K // 256, 64, 4, 6
    nsb = 8 * nb
    nch = -(-nsb // sbc)
    rowbytes = nb * Q4K
    for c in range(nch + ahead):
        written = set()
        for p in range(3):
            for t in range(2):
                sb = sbc * c + 2 * p + t
                sbl = min(sb, nsb - 1)
                assert (sbl >> 3) * Q4K + 16 + 16 * (sbl & 7) + 16 <= rowbytes
                if c < nch and sb < nsb:
                    assert 32 * sb + 31 < K
                    k4 = 8 * (2 * p + t)
                    assert k4 + 7 < 48
                    written.update(range(k4, k4 + 8))
        if c < nch:
            n4 = min(192, 32 * (nsb - sbc * c)) // 4
            assert set(range(n4)) <= written
    assert 96 * 1024 + (K * 4 if K <= 16384 else 0) <= 160 * 1024
    grid = (M + rows - 1) // rows
    for bx in sorted({0, grid - 1}):
        r = np.minimum(bx * rows + np.arange(rows), M - 1)
        assert (r * rowbytes + rowbytes).max() <= M * rowbytes
    producer_barriers = sum(1 for c0 in range(0, nch, ahead) for a in range(ahead) if c0 + a < nch)
    assert producer_barriers == nch


# ---------------------------------------------------------------- workgroup numbering and the decode step

def xcd_major(b, G):
    """bpdq_device.h xcd_major: hardware workgroup b of G -> its place in row order."""
    return (b & 7) * (G >> 3) + (b >> 3) if (G & 7) == 0 else b


@pytest.mark.parametrize("G", [1, 7, 8, 16, 257, 512, 1025, 1792, 3584])
def test_xcd_major_is_a_permutation_with_xcd_local_ranges(G):
    """Every workgroup gets one place in row order and every place one workgroup;
    when G % 8 == 0 each XCD (b % 8) owns one contiguous range of places."""
    b = np.arange(G)
    m = np.array([xcd_major(int(i), G) for i in b])
    assert sorted(m.tolist()) == list(range(G))
    if G % 8 == 0:
        for x in range(8):
            mine = np.sort(m[b % 8 == x])
            assert (np.diff(mine) == 1).all() and mine[0] == x * (G // 8)


def pv_tile(b, H, group, slices):
    """llama.hip pv_tile: workgroup b -> (head, column slice)."""
    hkv = H // group
    if (hkv * slices) % 8 == 0:
        i = b >> 3
        pair = (i // group) * 8 + (b & 7)
        return (pair % hkv) * group + i % group, pair // hkv
    return b % H, b // H


@pytest.mark.parametrize("H,HKV,D", [(32, 8, 128), (4, 2, 64), (4, 2, 128), (8, 2, 128), (16, 1, 64), (4, 4, 32),
                                     (16, 1, 32), (64, 8, 128), (2, 1, 256)])
@pytest.mark.parametrize("cols", [16, 32])
def test_pv_tile_covers_every_head_and_slice_once(H, HKV, D, cols):
    """k_attn_pv's grid of H * D/cols workgroups: each (head, slice) exactly once, and
    with the XCD numbering the heads that read one V slice share an XCD."""
    slices, group = D // cols, H // HKV
    seen = set()
    xcd = {}
    for b in range(H * slices):
        head, s = pv_tile(b, H, group, slices)
        assert 0 <= head < H and 0 <= s < slices
        seen.add((head, s))
        xcd.setdefault((head // group, s), set()).add(b % 8)
    assert len(seen) == H * slices
    if (HKV * slices) % 8 == 0:
        assert all(len(v) == 1 for v in xcd.values())


@pytest.mark.parametrize("n", [1, 63, 64, 65, 1023, 1024, 1100, 2049, 16384])
@pytest.mark.parametrize("cols", [16, 32])
def test_attn_pv_ring_and_loads_in_bounds(n, cols):
    """k_attn_pv<ROWS, COLS>: producer f = tid + 256k loads V row min(c*ROWS + f/C4, n-1),
    columns 4(f % C4).. of the slice, and writes ring slot rows 4(f % C4)..+3 at column
    f / C4; the chain lanes read ROWS floats of ring row tid."""
    rows = 128 if 1024 <= n <= 16384 else 64
    c4 = cols // 4
    ld = rows + 4
    per = rows * c4 // 256
    ahead = min(4096 // (rows * c4), 8)
    assert ahead in (4, 8) and per >= 1
    nch = (n + rows - 1) // rows
    f = np.arange(256)[:, None] + 256 * np.arange(per)[None, :]
    for c in sorted({0, nch - 1, nch - 1 + ahead}):  # the prefetch runs ahead of the last chunk
        r = np.minimum(c * rows + f // c4, n - 1)
        assert (r >= 0).all() and (r < n).all()
        assert (4 * (f % c4) + 3 < cols).all()
    slot_w = 4 * (f % c4) * ld + f // c4
    assert (slot_w + 3 * ld < cols * ld).all() and (f // c4 < rows).all()
    chain = np.arange(cols)
    assert (chain * ld + rows <= cols * ld).all()


@pytest.mark.parametrize("E,F", [(4096, 4096), (4096, 14336)])
def test_folded_norm_partials_fit_their_buffers(E, F):
    """The residual epilogues write one partial per workgroup: O (K = n_head*head_dim =
    n_embd, span rows per wave as launch_q4k_res picks them, 4 waves) and down (K = ff:
    56 blocks -> one row per wave, 8 waves; 16 -> as O).  The step reserves E/4 + 1
    doubles per set, and k_norm_q8k keeps 16 per lane in registers (1,024)."""
    def grid(M, K):
        if K // 256 == 56:
            return (M + 7) // 8
        R = span_rows_per_wave(M)
        return ((M + R - 1) // R + 3) // 4
    for K in (E, F):
        g = grid(E, K)
        assert g <= E // 4 + 1
        assert g <= 16 * 64
    # k_norm_q8k: wave b quantizes float4s b*64 .. b*64 + 63 of x and w
    assert (E // 256) * 64 * 4 == E


# ---------------------------------------------------------------- multi-token softmax and P.V

@pytest.mark.parametrize("T,kv_pos", [(1, 0), (3, 1100), (65, 0), (70, 100), (130, 0), (512, 0), (64, 448),
                                      (40, 4000)])
def test_mt_softmax_loads_cover_each_row_once(T, kv_pos):
    """k_mt_softmax (64-token blocks, 512 threads): thread p reads float4 p % 16 of every
    64-row chunk of tokens p / 16 and p / 16 + 32, in groups of 8 chunks; each (token,
    row below its count) is read, exponentiated and written once; reads stay inside
    the token's score row (ld = pad64(kv_pos + T)); the LDS e rows (pitch EP) hold the
    group's 64-row chunks and the chain lanes read whole chunks of their own row."""
    ld = (kv_pos + T + 63) // 64 * 64
    p = np.arange(512)
    jq = p & 15
    for tb in range(0, T, 64):
        nt = min(64, T - tb)
        n_hi = kv_pos + tb + nt
        nch = (n_hi + 63) // 64
        assert 64 * nch <= ld
        ng = (nch + 7) // 8
        ep = 64 * min(nch, 8) + 4
        assert 64 * ep * 4 <= 160 * 1024
        seen = np.zeros((nt, 64 * nch), dtype=int)
        for k in range(2):
            tt = (p >> 4) + 32 * k
            has = tt < nt
            nrow = kv_pos + tb + tt + 1
            for g in range(ng):
                for c in range(8):
                    cc = 8 * g + c
                    if cc >= nch:
                        continue
                    j = 64 * cc + 4 * jq
                    assert (j + 3 < ld).all()
                    lds = tt * ep + 64 * c + 4 * jq
                    assert (lds[has] + 3 < 64 * ep).all()
                    for i in range(4):
                        ok = has & (j + i < nrow)
                        np.add.at(seen, (tt[ok], j[ok] + i), 1)
        for t in range(nt):
            n = kv_pos + tb + t + 1
            assert (seen[t, :n] == 1).all() and (seen[t, n:] == 0).all()
        # chain: lane t reads 16 float4 per chunk of the group (and one re-read)
        for g in range(ng):
            gc = min(8, nch - 8 * g)
            lane = np.arange(64)
            assert (lane * ep + 64 * gc <= 64 * ep).all()


@pytest.mark.parametrize("T,kv_pos,S", [(1, 0, 64), (3, 1100, 2048), (65, 0, 256), (70, 100, 256), (512, 0, 512),
                                      (130, 0, 256), (448, 64, 512)])
@pytest.mark.parametrize("H,HKV,D", [(32, 8, 128), (4, 1, 128), (8, 2, 32)])
def test_mt_pv_staging_in_bounds(T, kv_pos, S, H, HKV, D):
    """k_mt_pv (512 threads, 64 columns per workgroup; workgroup p takes token block
    nb - 1 - p, then block p unless it is the same one): for each block, thread tid
    stages float4 f = tid + 512k (k < 2) of the chunk's weights (token min(f % 64,
    nt - 1), rows 4(f / 64)..+3, in the token's score row of ld = pad64(kv_pos + T)
    floats) and of V (row min(j0 + f / 16, n_hi - 1), columns min(4(f % 16), ncol -
    4)..+3 of the slice), stored transposed to [row][token] and as [row][column];
    lane (tg, cg) of wave (th, ch) reads its 4 tokens' float4 and 2 columns' float2 per
    row; every token of the batch is one block's, every (token, column) of a block
    one lane's, and a 32-column Q8_0 block one 16-lane row's."""
    ld = (kv_pos + T + 63) // 64 * 64
    row = HKV * D
    tid = np.arange(512)
    nb = (T + 63) // 64
    token_owner = np.zeros(T, dtype=int)
    blocks = []
    for p in range((nb + 1) // 2):
        heavy = nb - 1 - p
        blocks.append((heavy * 64, min(64, T - heavy * 64)))
        if p != heavy:
            assert T - p * 64 >= 64  # the lighter block is whole
            blocks.append((p * 64, 64))
    for tb, nt in blocks:
        token_owner[tb:tb + nt] += 1
        n_hi = kv_pos + tb + nt
        assert n_hi <= S
        nch = (n_hi + 63) // 64
        assert 64 * nch <= ld
        for d0 in range(0, D, 64):
            ncol = min(64, D - d0)
            assert ncol % 32 == 0
            for c in range(nch):
                j0 = 64 * c
                for k in range(2):
                    f = tid + 512 * k
                    tt = np.minimum(f & 63, nt - 1)
                    for h in (0, H - 1):
                        off = ((tb + tt) * H + h) * ld + j0 + 4 * (f >> 6)
                        assert (off + 3 < T * H * ld).all() and (j0 + 4 * (f >> 6) + 3 < ld).all()
                    j = np.minimum(j0 + (f >> 4), n_hi - 1)
                    col = np.minimum(4 * (f & 15), ncol - 4)
                    assert (j < S).all() and (col + 3 < ncol).all()
                    for kvh in (0, HKV - 1):
                        assert ((j * row + kvh * D + d0 + col + 3) < S * row).all()
                    r = 4 * (f >> 6)
                    assert ((r + 3) * 64 + (f & 63) < 64 * 64).all() and (f < 1024).all()
            ff = tid[:, None] + 512 * np.arange(2)[None, :]
            cells = ((4 * (ff >> 6))[..., None] + np.arange(4)) * 64 + (ff & 63)[..., None]
            assert np.array_equal(np.sort(cells.reshape(-1)), np.arange(64 * 64))
    assert (token_owner == 1).all()
    own = np.zeros((64, 64), dtype=int)
    for wave in range(8):
        th, ch = wave >> 1, wave & 1
        lane = np.arange(64)
        tw, cw = 16 * th + 4 * (lane >> 4), 32 * ch + 2 * (lane & 15)
        assert (63 * 32 + (cw + 1) // 2 < 2048).all() and (63 * 16 + (tw + 3) // 4 < 1024).all()
        # the 16 lanes of one tg hold one token's 32 columns 32ch .. 32ch + 31
        for g in range(4):
            cols = cw[lane >> 4 == g]
            assert np.array_equal(np.sort(np.concatenate([cols, cols + 1])), np.arange(32 * ch, 32 * ch + 32))
        for k in range(4):
            for i in range(2):
                np.add.at(own, (tw + k, cw + i), 1)
    assert (own == 1).all()


@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 8, 12])
def test_mt_scores_tile_waves_cover_every_head_and_token_once(G):
    """k_mt_scores_tile<TPW>: the host picks REPS token subsets (as many as fit G heads
    each into 8 waves, a power of two), TPW = 16 / REPS; wave w takes head w % G and
    subset w / G (REPS > 1) or heads w, w + 8, ... with all 16 tokens (REPS = 1)."""
    reps = 8 if 8 // G >= 8 else 4 if 8 // G >= 4 else 2 if 8 // G >= 2 else 1
    tpw = 16 // reps
    assert G * reps <= 8 or reps == 1
    seen = np.zeros((G, 16), dtype=int)
    for wave in range(8):
        sub = 0 if reps == 1 else wave // G
        if sub >= reps:
            continue
        h = wave if reps == 1 else wave % G
        while h < G:
            seen[h, tpw * sub:tpw * sub + tpw] += 1
            h += 8 if reps == 1 else G
    assert (seen == 1).all()


@pytest.mark.parametrize("nP,nT", [(112, 4), (224, 4), (64, 4), (96, 4), (250, 4), (1, 1), (5, 2), (8, 3), (448, 1)])
def test_q8_0_gemm_SH_tile_order(nP, nT):
    """sh_tile: workgroup b of nP * nT takes (panel, token tile) once each; with nP
    a multiple of 8, panel p runs on XCD p % 8 (b % 8) and its nT tiles sit within
    one run of 8 nT consecutive workgroups."""
    seen = set()
    for b in range(nP * nT):
        if nP % 8 == 0:
            g, r = divmod(b, 8 * nT)
            by, bx = r >> 3, 8 * g + (r & 7)
            assert b % 8 == bx % 8 and b // (8 * nT) == bx // 8
        else:
            bx, by = b % nP, b // nP
        assert 0 <= bx < nP and 0 <= by < nT
        seen.add((bx, by))
    assert len(seen) == nP * nT


# ---------------------------------------------------------------- the reference Python loader's dequant

@pytest.mark.parametrize("code,per,size", [(2, 32, 18), (10, 256, 84), (11, 256, 110), (12, 256, 144)])
@pytest.mark.parametrize("nb", [1, 3, 4099])
def test_dequant_gguf_py_in_bounds(code, per, size, nb):
    """k_dequant_py<TYPE>: thread t < n_quads = nb*per/4 reads only bytes of block
    t / (per/4) and writes float4 t; every output quad written once."""
    qpb = per // 4
    n_quads = nb * per // 4
    grid = (n_quads + 255) // 256 * 256
    t = np.arange(grid)
    t = t[t < n_quads]
    assert np.array_equal(t, np.arange(n_quads))
    b, e0 = t // qpb, (t % qpb) * 4
    assert b.max() < nb
    if code == 2:
        offs = [np.zeros_like(e0), np.ones_like(e0)] + [np.where(e < 16, 2 + e, 2 + e - 16) for e in
                                                        (e0, e0 + 1, e0 + 2, e0 + 3)]
    elif code == 10:
        offs = [np.full_like(e0, 80), np.full_like(e0, 83), e0 >> 4, 16 + (e0 >> 2)]
    elif code == 11:
        si = e0 >> 4
        offs = [np.full_like(e0, 108), np.full_like(e0, 109), 96 + (si & 7), 32 + (e0 >> 2), e0 >> 3]
    else:
        ii = e0 & 127
        j = np.where(e0 >= 128, 4, 0) + (ii >> 5)
        offs = [np.full_like(e0, 0), np.full_like(e0, 3), 4 + j, 4 + j + 4, 4 + np.maximum(j - 4, 0),
                16 + ii, 16 + ii + 3]
    for o in offs:
        assert o.min() >= 0 and o.max() < size
    assert ((b * size + max(o.max() for o in offs)) < nb * size).all()


@pytest.mark.parametrize("esize", [2, 4])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 4097])
def test_copy_f16_f32_in_bounds(esize, n):
    """k_copy_f16_f32: thread t handles elements 4t .. 4t+cnt-1, cnt = min(4, n - 4t);
    whole quads as one float4 store, the tail element by element; each element once."""
    t = np.arange((n + 3) // 4)
    cnt = np.minimum(4, n - 4 * t)
    assert (cnt >= 1).all()
    elems = np.concatenate([4 * tt + np.arange(c) for tt, c in zip(t, cnt)])
    assert np.array_equal(elems, np.arange(n))
    assert (elems * esize + esize - 1).max() < n * esize
