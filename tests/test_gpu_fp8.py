"""FP8 block-scaled GEMV on the MI355X against the CPU oracle.

Parity bar: decoders bit-exact on every code; exact-representable known
answers bit-exact; otherwise worst vector-scaled relative error < 1e-5 and
the same argmax (the reference GPU gate, tests/unit/test_cuda.c:103-192);
the batched path bit-identical to single calls (test_cuda.c:194-256).
"""
import ctypes
import sys

import numpy as np
import pytest

import common
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5

# Residency is keyed by host pointer (the reference contract): keep every
# uploaded array alive for the test, then reset the backend so a later
# array that reuses an address is never mistaken for a resident one.
_keep = []


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    _keep.clear()
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------- decoders
def test_decoders_bit_exact(gpu, dsv4):
    for which, ref in (("e4m3", oracle.dump_e4m3()), ("e8m0", oracle.dump_e8m0()),
                       ("e2m1", oracle.dump_e2m1())):
        dev = dsv4.dump(which)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(dev), nan), which
        assert common.bits_equal(dev[~nan], ref[~nan]), which


@pytest.mark.parametrize("e8m0", [127, 120, 134, 100, 150, 119])
def test_scaled_e4m3_decoder_bit_exact(gpu, dsv4, e8m0):
    """The matrix-core FP8 form decodes e4m3 codes into bf16 with the E8M0
    block scale folded in (v_cvt_scalef32_pk_bf16_fp8): all 256 codes times
    2^(e8m0 - 127) against the reference decoder's value times the scale
    (exact: 3 mantissa bits fit bf16's 7), NaN codes NaN."""
    L = dsv4.lib()
    dev = np.empty(256, np.float32)
    assert L.dsv4_gpu_dump_e4m3_scaled(dev.ctypes.data, e8m0) == 0
    ref = (oracle.dump_e4m3().astype(np.float64) * 2.0 ** (e8m0 - 127)).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(dev), nan)
    assert common.bits_equal(dev[~nan], ref[~nan])
    assert L.dsv4_gpu_dump_e4m3_scaled(dev.ctypes.data, 256) == -1


def test_fp4_byte_order_bit_exact(gpu, dsv4):
    dev = dsv4.dump("fp4_bytes").reshape(256, 2)
    tab = oracle.dump_e2m1()
    b = np.arange(256)
    assert common.bits_equal(dev[:, 0], tab[b & 15])      # even = low nibble
    assert common.bits_equal(dev[:, 1], tab[b >> 4])


# ------------------------------------------------------------ known answers
def _run(dsv4, W, S, x, f32s=False, blk_r=128, blk_c=128):
    L = dsv4.lib()
    _keep.extend([W, S])
    m = dsv4.qmat(W, S, blk_r=blk_r, blk_c=blk_c)
    rc = (L.dsv4_gpu_upload_f32s if f32s else L.dsv4_gpu_upload)(ctypes.byref(m))
    assert rc == 0
    assert L.dsv4_gpu_has(ctypes.byref(m)) == 1
    return dsv4.mmq(m, x), m


def test_known_answers(gpu, dsv4):
    """test_matmul.c:63-130, run on the device."""
    W = np.zeros((2, 128), np.uint8); W[0], W[1] = 0x38, 0x40
    y, _ = _run(dsv4, W, np.array([[128]], np.uint8), np.ones(128, np.float32))
    assert list(y) == [256.0, 512.0]
    W = np.full((256, 128), 0x38, np.uint8)
    y, _ = _run(dsv4, W, np.array([[127], [129]], np.uint8), np.ones(128, np.float32))
    assert y[0] == 128 and y[127] == 128 and y[128] == 512 and y[255] == 512
    W = np.full((1, 256), 0x38, np.uint8)
    y, _ = _run(dsv4, W, np.array([[127, 128]], np.uint8), np.ones(256, np.float32))
    assert y[0] == 384.0


def check_shape(dsv4, rows, cols, seed, f32s=True, continuous=False):
    W, Sf, Se, x = common.fp8_problem(seed, rows, cols, continuous=continuous)
    S = Sf if (f32s or continuous) else Se
    y, m = _run(dsv4, W, S, x, f32s=(f32s or continuous))
    want = oracle.matmul_fp8(x, W, S)
    err = common.vec_rel_err(y, want)
    say("fp8 %dx%d seed %d %s: worst rel %.3g" %
        (rows, cols, seed, "cont" if continuous else ("f32" if f32s else "e8m0"), err))
    assert err < TOL
    assert int(np.argmax(y)) == int(np.argmax(want))
    return y, want


def test_c1_4096(gpu, dsv4):
    check_shape(dsv4, 4096, 4096, 0, f32s=True)
    check_shape(dsv4, 4096, 4096, 0, f32s=False)
    check_shape(dsv4, 4096, 4096, 1, continuous=True)


@pytest.mark.parametrize("scales", ["f32", "e8m0"])
@pytest.mark.parametrize("rows,cols", [(1536, 7168), (576, 7168), (24576, 1536),
                                       (7168, 16384), (7168, 7168)])
def test_c2_trunk_shapes(gpu, dsv4, rows, cols, scales):
    """fp32 block scales (the configuration's) and E8M0 ones (the
    reference's), both on the default VALU form."""
    check_shape(dsv4, rows, cols, 0, f32s=scales == "f32")


@pytest.mark.parametrize("scales", ["f32", "e8m0"])
def test_c2_lm_head(gpu, dsv4, scales):
    check_shape(dsv4, 129280, 7168, 0, f32s=scales == "f32")


@pytest.mark.parametrize("rows,cols", [(1, 16), (3, 48), (130, 96), (257, 1040),
                                       (64, 100), (33, 20000), (5, 8)])
def test_ragged_and_generic_shapes(gpu, dsv4, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    W = common.fp8_codes(rng, (rows, cols))
    e = rng.integers(-8, -3, size=((rows + 127) // 128, (cols + 127) // 128))
    S = (127 + e).astype(np.uint8)
    x = rng.standard_normal(cols, dtype=np.float32)
    y, _ = _run(dsv4, W, S, x)
    assert common.vec_rel_err(y, oracle.matmul_fp8(x, W, S)) < TOL


def test_reference_gpu_gate(gpu, dsv4):
    """test_cuda.c:103-256: 4096x8192, LCG data, E8M0 scales 120..134."""
    rows, cols = 4096, 8192
    r = 20260820
    M = (1 << 32) - 1

    # vectorised LCG: x_{k} = a^k x_0 + c (a^k - 1)/(a - 1), all mod 2^32
    def lcg_fast(n):
        nonlocal r
        a, c = 1103515245, 12345
        ks = np.arange(1, n + 1, dtype=np.uint64)
        # powers of a mod 2^32 by repeated squaring over the bits of k
        ak = np.ones(n, np.uint64); cs = np.zeros(n, np.uint64)
        pa, pc = np.uint64(a), np.uint64(c)
        kk = ks.copy()
        while kk.any():
            bit = (kk & 1).astype(bool)
            # compose (ak, cs) with (pa, pc): x -> pa*x + pc applied after
            cs[bit] = (cs[bit] * pa + pc) & np.uint64(M)
            ak[bit] = (ak[bit] * pa) & np.uint64(M)
            pc = (pc * pa + pc) & np.uint64(M)
            pa = (pa * pa) & np.uint64(M)
            kk >>= np.uint64(1)
        out = ((ak * np.uint64(r)) + cs) & np.uint64(M)
        r = int(out[-1])
        return out.astype(np.uint32)
    xs = lcg_fast(cols)
    x = (((xs >> 16) & 0xFFFF).astype(np.int64) - 32768).astype(np.float32) * np.float32(1e-3)
    wb = ((lcg_fast(rows * cols) >> 16) & 0xFF).astype(np.uint8)
    wb = np.where((wb & 0x7F) == 0x7F, wb & 0xFE, wb).astype(np.uint8).reshape(rows, cols)
    ns = (rows // 128) * (cols // 128)
    S = (120 + ((lcg_fast(ns) >> 16) % 15)).astype(np.uint8).reshape(rows // 128, cols // 128)
    y, m = _run(dsv4, wb, S, x)
    want = oracle.matmul_fp8(x, wb, S)
    err = common.vec_rel_err(y, want)
    say("reference gate 4096x8192: worst rel %.3g" % err)
    assert err < TOL and int(np.argmax(y)) == int(np.argmax(want))
    NT = 8
    t = np.arange(NT)[:, None]
    i = np.arange(cols)[None, :]
    xn = np.sin(0.7 * (i + 1) + 3.1 * (t + 1)).astype(np.float32)
    yn = dsv4.mmq_n(m, xn)
    for k in range(NT):
        assert common.bits_equal(yn[k], dsv4.mmq(m, xn[k])), k
    assert common.bits_equal(dsv4.mmq_n(m, xn[:1])[0], dsv4.mmq(m, xn[0]))


@pytest.mark.parametrize("form", ["0", "1"])
@pytest.mark.parametrize("rows,cols,nt", [(300, 1536, 5), (129, 7168, 64), (40, 64, 3),
                                          (500, 2048, 13), (70, 16384, 2), (33, 4096, 9),
                                          (7168, 7168, 64), (77, 1040, 21), (16, 112, 6),
                                          (1000, 7168, 11), (257, 2096, 20), (64, 16, 4),
                                          (200, 4096, 33), (18, 3072, 7), (300, 1536, 48)])
def test_batched_bit_identical(gpu, dsv4, monkeypatch, rows, cols, nt, form):
    """E8M0 scales on both forms. The default VALU form's batched kernel runs
    the GEMV's chunk dots, scale FMAs and reduction tree per (row, token).
    The matrix-core form (DSV4_GPU_FP8_MX=1) runs the single-token chain per
    (row, token), whatever column of which tile a token takes (up to 64
    tokens, ragged row tiles, columns not a multiple of the 256-byte unit or
    of the 1024-column segment; nt 48 and 64 take the 8-wave workgroups, nt
    48 with a ragged last token group); cols not a multiple of 16 take the
    generic kernel either way. Every token's row equals the single-token
    GEMV's bits."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", form)
    W, Sf, Se, _ = common.fp8_problem(21, rows, cols)
    x = np.random.default_rng(22).standard_normal((nt, cols), dtype=np.float32)
    y1, m = _run(dsv4, W, Se, x[0])
    yn = dsv4.mmq_n(m, x)
    for t in range(nt):
        assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), t
    assert common.vec_rel_err(yn, oracle.matmul_fp8(x, W, Se)) < TOL


@pytest.mark.parametrize("wdt", ["fp8", "fp8_f32s"])
@pytest.mark.parametrize("nt", [1, 5, 16])
def test_host_staging_modes_keep_bits(gpu, dsv4, monkeypatch, nt, wdt):
    """Host-buffer calls stage zero-copy by default (the inputs pulled to the
    device through the pinned arena's device mapping, the output written by
    the last kernel straight into it) or through two DMA copies
    (DSV4_GPU_HOST_ZC=0): the same bits either way, single token and
    batched, within 1e-5 of the oracle."""
    rows, cols = 1536, 2048
    W, Sf, Se, _ = common.fp8_problem(61, rows, cols)
    S = Se if wdt == "fp8" else Sf
    x = np.random.default_rng(62).standard_normal((nt, cols), dtype=np.float32)
    _, m = _run(dsv4, W, S, x[0], f32s=wdt == "fp8_f32s")
    outs = {}
    for zc in ("1", "0", "1"):
        monkeypatch.setenv("DSV4_GPU_HOST_ZC", zc)
        y = dsv4.mmq_n(m, x) if nt > 1 else dsv4.mmq(m, x[0])[None]
        if zc in outs:
            assert common.bits_equal(y, outs[zc]), "zero-copy repeat"
        outs[zc] = y
    assert common.bits_equal(outs["1"], outs["0"])
    assert common.vec_rel_err(outs["1"], oracle.matmul_fp8(x, W, S)) < TOL


def _same_bits_or_nan(a, b):
    """NaN where the other is NaN (any payload), the same bits elsewhere."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and common.bits_equal(a[~nan], b[~nan])


@pytest.mark.parametrize("scales", ["e8m0", "f32"])
@pytest.mark.parametrize("slots", ["0", "16", "32", "64"])
def test_batched_matrix_core_f32_chains_keep_bits(gpu, dsv4, monkeypatch, slots, scales):
    """The batched kernel for columns a multiple of 64 (k_fp8_mfn) runs the
    GEMV's four fmaf chains per chunk on v_mfma_f32_16x16x4f32 and the rest
    of its arithmetic on the VALU. Against the single-token GEMV and the VALU
    batched kernel (DSV4_GPU_FP8_MFN=0), bit for bit, for every part size
    DSV4_GPU_MFN_L (0: the launcher's rule, which keeps small batches and
    small launches on the VALU kernel; a size a shape does not take falls
    back to the VALU kernel), both scale formats, 16 to 256 row slots (1024
    to 16384 columns, and 512 = 32 slots), 1 to 4 chunks per slot, ragged
    row tiles and token tiles, a token of signed zeros against zero codes of
    both signs, a token of subnormals, and a token with inf."""
    cases = ((300, 1536, 5), (129, 7168, 37), (70, 16384, 2), (33, 4096, 17), (18, 3072, 7),
             (16, 512, 3), (47, 1024, 19), (200, 2048, 64), (40, 6144, 4), (7168, 7168, 64),
             (24, 256, 5))
    for rows, cols, nt in cases:
        rng = np.random.default_rng(rows * 7 + cols + nt)
        W = common.fp8_codes(rng, (rows, cols))
        W[:, : cols // 8] = np.where(rng.random((rows, cols // 8)) < 0.5, 0x00, 0x80)
        Sf, Se = common.fp8_scales(rng, rows, cols)
        x = rng.standard_normal((nt, cols), dtype=np.float32)
        x[1, : cols // 8] = -0.0
        x[1, cols // 8:] = np.where(rng.random(cols - cols // 8) < 0.5, 0.0, -0.0)
        if nt > 2:
            x[2] = (rng.standard_normal(cols) * 1e-39).astype(np.float32)   # subnormal
        if nt > 3:
            x[3, 5] = np.inf
        S = Se if scales == "e8m0" else Sf
        _, m = _run(dsv4, W, S, x[0], f32s=scales == "f32")
        monkeypatch.setenv("DSV4_GPU_FP8_MFN", "0")
        ref = dsv4.mmq_n(m, x)
        monkeypatch.setenv("DSV4_GPU_FP8_MFN", "1")
        monkeypatch.setenv("DSV4_GPU_MFN_L", slots)
        say("fp8 mfn %dx%d nt %d L %s %s" % (rows, cols, nt, slots, scales))
        yn = dsv4.mmq_n(m, x)
        monkeypatch.delenv("DSV4_GPU_MFN_L")
        assert _same_bits_or_nan(yn, ref), (rows, cols, nt, slots)
        for t in range(nt):
            assert _same_bits_or_nan(yn[t], dsv4.mmq(m, x[t])), (rows, cols, t)
        fin = np.isfinite(x).all(axis=1)
        assert common.vec_rel_err(yn[fin], oracle.matmul_fp8(x[fin], W, S)) < TOL


@pytest.mark.parametrize("ntmax", ["1", "3", "5", "6", "7"])
def test_batched_token_tiles_keep_bits(gpu, dsv4, monkeypatch, ntmax):
    """DSV4_GPU_MXN_NT (column tiles of five tokens per workgroup, so how many
    passes over the weights a batch takes) only reshapes the batched launch:
    every setting gives each token the single-token GEMV's bits."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", "1")
    monkeypatch.setenv("DSV4_GPU_MXD", "0")          # the register-staged kernel
    monkeypatch.setenv("DSV4_GPU_MXN_NT", ntmax)
    for rows, cols, nt in ((300, 1536, 64), (129, 7168, 37), (70, 2096, 11)):
        W, Sf, Se, _ = common.fp8_problem(23, rows, cols)
        x = np.random.default_rng(24).standard_normal((nt, cols), dtype=np.float32)
        y1, m = _run(dsv4, W, Se, x[0])
        say("fp8 mxn %dx%d nt %d MXN_NT %s" % (rows, cols, nt, ntmax))
        yn = dsv4.mmq_n(m, x)
        for t in range(nt):
            assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), (ntmax, rows, t)


@pytest.mark.parametrize("xf", ["0", "1"])
@pytest.mark.parametrize("kp", ["0", "2", "4"])
def test_batched_segment_split_keeps_bits(gpu, dsv4, monkeypatch, kp, xf):
    """DSV4_GPU_MXK: with one column tile of at most five tokens per group,
    the batched kernel splits each tile's segments over KP waves (0: one
    wave), which meet in LDS in segment order; DSV4_GPU_MXKF: its x terms
    from the pre-split planes (0) or formed from the f32 rows in each
    workgroup (1). Every setting gives each token the single-token GEMV's
    bits: uniform and per-lane scales, ragged row tiles and segments, a last
    unit past the row's end, fewer segments than waves (taken by the one-wave
    form), one to four groups."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", "1")
    monkeypatch.setenv("DSV4_GPU_MXK", kp)
    monkeypatch.setenv("DSV4_GPU_MXKF", xf)
    cases = ((300, 1536, 2, 128, 128), (129, 7168, 5, 128, 128), (70, 2096, 4, 1, 32),
             (33, 16384, 9, 16, 64), (200, 1040, 3, 4, 48), (16, 512, 20, 128, 128),
             (40, 64, 3, 128, 128), (7168, 7168, 4, 128, 128))
    for rows, cols, nt, blk_r, blk_c in cases:
        rng = np.random.default_rng(rows + cols + nt)
        W = common.fp8_codes(rng, (rows, cols))
        S = (127 + rng.integers(-8, -3, size=((rows + blk_r - 1) // blk_r,
                                              (cols + blk_c - 1) // blk_c))).astype(np.uint8)
        x = rng.standard_normal((nt, cols), dtype=np.float32)
        say("fp8 mxk %dx%d nt %d blk %dx%d MXK %s MXKF %s" % (rows, cols, nt, blk_r, blk_c,
                                                              kp, xf))
        _, m = _run(dsv4, W, S, x[0], blk_r=blk_r, blk_c=blk_c)
        yn = dsv4.mmq_n(m, x)
        for t in range(nt):
            assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), (kp, rows, cols, t)
        assert common.vec_rel_err(yn, oracle.matmul_fp8(x, W, S, blk_r, blk_c)) < TOL


@pytest.mark.parametrize("mxd,mw,pl", [("0", "8", "0"), ("1", "8", "0"), ("1", "4", "0"),
                                        ("1", "8", "1"), ("1", "4", "1"), ("1", "2", "1")])
def test_batched_dma_staging_keeps_bits(gpu, dsv4, monkeypatch, mxd, mw, pl):
    """DSV4_GPU_MXD: the batched matrix-core kernel whose weight and x-term
    stages are copied into LDS by direct-to-LDS loads (uniform scales, groups
    of up to 20 tokens with DSV4_GPU_MXD_PL=0, else planar groups of up to
    16, one column tile per term; DSV4_GPU_MXD_MW: workgroups of 8 waves over
    128 rows, 4 over 64 or, planar, 2 over 32) against the register-staged
    one. Each gives each
    token the single-token GEMV's bits: row counts that leave part of a
    workgroup or a 16-row tile empty, a last unit past the row's end, one
    unit, a single segment and sixteen, groups of 1 to 20 tokens."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", "1")
    monkeypatch.setenv("DSV4_GPU_MXD", mxd)
    monkeypatch.setenv("DSV4_GPU_MXD_MW", mw)
    monkeypatch.setenv("DSV4_GPU_MXD_PL", pl)
    cases = ((7168, 7168, 64, 128, 128), (300, 1536, 64, 128, 128), (129, 7168, 37, 128, 128),
             (33, 16384, 21, 16, 64), (70, 2096, 41, 32, 64), (16, 512, 20, 128, 128),
             (40, 64, 3, 128, 128), (257, 1024, 7, 16, 128), (136, 3072, 61, 64, 192),
             (200, 2048, 16, 128, 128), (96, 4096, 48, 128, 128), (81, 1280, 17, 32, 128))
    for rows, cols, nt, blk_r, blk_c in cases:
        rng = np.random.default_rng(rows + cols + nt + 7)
        W = common.fp8_codes(rng, (rows, cols))
        S = (127 + rng.integers(-8, -3, size=((rows + blk_r - 1) // blk_r,
                                              (cols + blk_c - 1) // blk_c))).astype(np.uint8)
        x = rng.standard_normal((nt, cols), dtype=np.float32)
        say("fp8 mxd %dx%d nt %d blk %dx%d MXD %s MW %s PL %s"
            % (rows, cols, nt, blk_r, blk_c, mxd, mw, pl))
        _, m = _run(dsv4, W, S, x[0], blk_r=blk_r, blk_c=blk_c)
        yn = dsv4.mmq_n(m, x)
        for t in range(nt):
            assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), (mxd, rows, cols, t)
        assert common.vec_rel_err(yn, oracle.matmul_fp8(x, W, S, blk_r, blk_c)) < TOL


@pytest.mark.parametrize("form", ["0", "1"])
@pytest.mark.parametrize("blk_r,blk_c", [(1, 32), (16, 64), (128, 128), (4, 48), (256, 256)])
def test_matrix_core_form_blockings(gpu, dsv4, monkeypatch, blk_r, blk_c, form):
    """E8M0 scale grids other than 128 x 128 (a scale per lane piece in the
    matrix-core form, DSV4_GPU_FP8_MX=1; the default VALU form too): against
    the oracle, and batched bit-identical."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", form)
    rows, cols, nt = 300, 1536, 7
    rng = np.random.default_rng(blk_r * 1000 + blk_c)
    W = common.fp8_codes(rng, (rows, cols))
    S = (127 + rng.integers(-8, -3, size=((rows + blk_r - 1) // blk_r,
                                           (cols + blk_c - 1) // blk_c))).astype(np.uint8)
    x = rng.standard_normal((nt, cols), dtype=np.float32)
    y, m = _run(dsv4, W, S, x[0], blk_r=blk_r, blk_c=blk_c)
    assert common.vec_rel_err(y, oracle.matmul_fp8(x[0], W, S, blk_r, blk_c)) < TOL
    yn = dsv4.mmq_n(m, x)
    for t in range(nt):
        assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), t


@pytest.mark.parametrize("form", ["1", "0"])
def test_e8m0_forms(gpu, dsv4, monkeypatch, form):
    """DSV4_GPU_FP8_MX=1 (the matrix core for E8M0 scales) and =0 (the
    default VALU form for every matrix): each within the bar, each with its
    own batched kernel bit-identical per token."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", form)
    rows, cols, nt = 1000, 7168, 6
    W, Sf, Se, _ = common.fp8_problem(71, rows, cols)
    x = np.random.default_rng(72).standard_normal((nt, cols), dtype=np.float32)
    y, m = _run(dsv4, W, Se, x[0])
    want = oracle.matmul_fp8(x, W, Se)
    assert common.vec_rel_err(y, want[0]) < TOL
    yn = dsv4.mmq_n(m, x)
    for t in range(nt):
        assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), t
    assert common.vec_rel_err(yn, want) < TOL


@pytest.mark.parametrize("scales", ["f32", "e8m0"])
@pytest.mark.parametrize("rows,cols", [(7168, 7168), (1536, 1536), (300, 4096), (260, 16384),
                                       (4096, 8192), (1024, 4096)])
def test_launch_shape_keeps_bits(gpu, dsv4, monkeypatch, rows, cols, scales):
    """Rows per thread (DSV4_GPU_FP8_R), prefetch (DSV4_GPU_FP8_PF),
    workgroups per CU (DSV4_GPU_FP8_WPC) and x through LDS (DSV4_GPU_FP8_XL)
    only reshape the launch: every setting gives the default's bits, in both
    scale formats (the default shape itself depends on the format)."""
    W, Sf, Se, x = common.fp8_problem(51, rows, cols)
    S = Sf if scales == "f32" else Se
    y0, m = _run(dsv4, W, S, x, f32s=scales == "f32")
    assert common.vec_rel_err(y0, oracle.matmul_fp8(x, W, S)) < TOL
    for r, pf, wpc, xl in ((1, 0, 2, None), (4, 0, 2, None), (2, 1, 2, None), (2, 0, 1, None),
                           (4, 1, 8, None), (1, 1, 4, None), (1, 1, 2, 1), (2, 0, 2, 0),
                           (4, 1, 2, 1)):
        monkeypatch.setenv("DSV4_GPU_FP8_R", str(r))
        monkeypatch.setenv("DSV4_GPU_FP8_PF", str(pf))
        monkeypatch.setenv("DSV4_GPU_FP8_WPC", str(wpc))
        if xl is None:
            monkeypatch.delenv("DSV4_GPU_FP8_XL", raising=False)
        else:
            monkeypatch.setenv("DSV4_GPU_FP8_XL", str(xl))
        say("fp8 %dx%d R %d PF %d WPC %d XL %s" % (rows, cols, r, pf, wpc, xl))
        assert common.bits_equal(dsv4.mmq(m, x), y0), (r, pf, wpc, xl)


def test_row_range_views(gpu, dsv4):
    """The wo_a group slicing of attention() (dsv4_layer.c:321-334): every
    group is resident as a view and computes only its rows. A slice that
    starts inside a 128-row block (o_lora below 128) counts its scale rows
    from its own scale pointer, as the reference's kernel does
    (dsv4_matmul.c:293-318); a scale pointer off a grid row, or scale rows
    past the parent's grid, do not resolve."""
    groups, gr, gw = 8, 256, 1024
    rows = groups * gr
    W, Sf, Se, x = common.fp8_problem(31, rows, gw)
    L = dsv4.lib()
    _keep.extend([W, Se])
    full = dsv4.qmat(W, Se)
    assert L.dsv4_gpu_upload(ctypes.byref(full)) == 0
    yfull = dsv4.mmq(full, x)
    sc = gw // 128
    for g in range(groups):
        sl = dsv4.DSV4QMat(W.ctypes.data + g * gr * gw,
                           Se.ctypes.data + g * (gr // 128) * sc,
                           dsv4.WFP8, gr, gw, 128, 128)
        assert L.dsv4_gpu_has(ctypes.byref(sl)) == 1
        assert common.bits_equal(dsv4.mmq(sl, x), yfull[g * gr:(g + 1) * gr])
    # rows 64..127 with the grid's first scale row: the parent's own scales
    mid = dsv4.DSV4QMat(W.ctypes.data + 64 * gw, Se.ctypes.data, dsv4.WFP8, 64, gw, 128, 128)
    assert L.dsv4_gpu_has(ctypes.byref(mid)) == 1
    assert common.bits_equal(dsv4.mmq(mid, x), yfull[64:128])
    off = dsv4.DSV4QMat(W.ctypes.data + 64 * gw, Se.ctypes.data + 1, dsv4.WFP8, 64, gw, 128, 128)
    assert L.dsv4_gpu_has(ctypes.byref(off)) == 0          # scale pointer off a grid row
    past = dsv4.DSV4QMat(W.ctypes.data + (rows - 128) * gw,
                         Se.ctypes.data + (rows // 128) * sc, dsv4.WFP8, 128, gw, 128, 128)
    assert L.dsv4_gpu_has(ctypes.byref(past)) == 0         # scale rows past the grid
    other = np.zeros_like(W)
    assert L.dsv4_gpu_has(ctypes.byref(dsv4.qmat(other, Se))) == 0


def test_device_entry_point_matches_host_path(gpu, dsv4):
    import torch
    rows, cols = 7168, 7168
    W, Sf, Se, x = common.fp8_problem(41, rows, cols)
    y_host, _ = _run(dsv4, W, Sf, x, f32s=True)
    dev = torch.device("cuda:0")
    dW = torch.from_numpy(W).to(dev)
    dS = torch.from_numpy(Sf).to(dev)
    dx = torch.from_numpy(x).to(dev)
    dy = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    rc = dsv4.lib().dsv4_gpu_fp8_gemv_d(dy.data_ptr(), dx.data_ptr(), dW.data_ptr(),
                                        dS.data_ptr(), 1, rows, cols, st)
    assert rc == 0
    torch.cuda.synchronize()
    assert common.bits_equal(dy.cpu().numpy(), y_host)


@pytest.mark.parametrize("form", ["0", "1"])
def test_batched_device_entry_point(gpu, dsv4, monkeypatch, form):
    """dsv4_gpu_fp8_gemv_n_d: every token's row equals dsv4_gpu_fp8_gemv_d on
    that token, bit for bit (the k_mmq_fp8_n contract), on device buffers,
    on both forms."""
    import torch
    monkeypatch.setenv("DSV4_GPU_FP8_MX", form)
    rows, cols, nt = 1000, 7168, 11
    W, Sf, Se, _ = common.fp8_problem(61, rows, cols)
    x = np.random.default_rng(62).standard_normal((nt, cols), dtype=np.float32)
    dev = torch.device("cuda:0")
    dW, dS, dx = (torch.from_numpy(a).to(dev) for a in (W, Se, x))
    dy = torch.empty((nt, rows), dtype=torch.float32, device=dev)
    d1 = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    L = dsv4.lib()
    assert L.dsv4_gpu_fp8_gemv_n_d(dy.data_ptr(), dx.data_ptr(), dW.data_ptr(), dS.data_ptr(),
                                   0, rows, cols, nt, st) == 0
    torch.cuda.synchronize()
    yn = dy.cpu().numpy()
    for t in range(nt):
        assert L.dsv4_gpu_fp8_gemv_d(d1.data_ptr(), dx[t].data_ptr(), dW.data_ptr(),
                                     dS.data_ptr(), 0, rows, cols, st) == 0
        torch.cuda.synchronize()
        assert common.bits_equal(yn[t], d1.cpu().numpy()), t
    assert common.vec_rel_err(yn, oracle.matmul_fp8(x, W, Se)) < TOL
    assert L.dsv4_gpu_fp8_gemv_n_d(dy.data_ptr(), dx.data_ptr(), dW.data_ptr(), dS.data_ptr(),
                                   0, rows, cols, 65, st) == -1     # above DSV4_MAX_BATCH


@pytest.mark.parametrize("form", ["0", "1"])
def test_unaligned_device_operands_refused(gpu, dsv4, monkeypatch, form):
    """The arithmetic follows from the matrix alone: a device-buffer call
    whose x (or W) breaks the 16-byte alignment of the chunked forms is
    refused (-1) rather than sent to another kernel with other bits; the
    aligned call on the same values is unaffected."""
    import torch
    monkeypatch.setenv("DSV4_GPU_FP8_MX", form)
    rows, cols, nt = 256, 2048, 3
    W, Sf, Se, _ = common.fp8_problem(63, rows, cols)
    x = np.random.default_rng(64).standard_normal((nt, cols), dtype=np.float32)
    dev = torch.device("cuda:0")
    dW, dS = torch.from_numpy(W).to(dev), torch.from_numpy(Se).to(dev)
    xb = torch.zeros(nt * cols + 4, dtype=torch.float32, device=dev)
    xb[1:1 + nt * cols] = torch.from_numpy(x.reshape(-1)).to(dev)
    dy = torch.empty((nt, rows), dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    L = dsv4.lib()
    odd = xb.data_ptr() + 4                              # 4 bytes past 16-byte alignment
    assert L.dsv4_gpu_fp8_gemv_d(dy.data_ptr(), odd, dW.data_ptr(), dS.data_ptr(), 0,
                                 rows, cols, st) == -1
    assert L.dsv4_gpu_fp8_gemv_n_d(dy.data_ptr(), odd, dW.data_ptr(), dS.data_ptr(), 0,
                                   rows, cols, nt, st) == -1
    dx = torch.from_numpy(x).to(dev)
    assert L.dsv4_gpu_fp8_gemv_n_d(dy.data_ptr(), dx.data_ptr(), dW.data_ptr(),
                                   dS.data_ptr(), 0, rows, cols, nt, st) == 0
    torch.cuda.synchronize()
    assert common.vec_rel_err(dy.cpu().numpy(), oracle.matmul_fp8(x, W, Se)) < TOL


def test_upload_refusals(gpu, dsv4):
    L = dsv4.lib()
    W = np.zeros((4, 32), np.uint8)
    S = np.zeros((4, 1), np.uint8)
    mf32 = dsv4.DSV4QMat(W.ctypes.data, S.ctypes.data, dsv4.WF32, 4, 8, 1, 1)
    assert L.dsv4_gpu_upload(ctypes.byref(mf32)) == -1        # no f32 matrices on the device
    m4 = dsv4.DSV4QMat(W.ctypes.data, S.ctypes.data, dsv4.WFP4, 4, 64, 1, 16)
    assert L.dsv4_gpu_upload(ctypes.byref(m4)) == -1          # FP4 blocks narrower than 32
    m8 = dsv4.DSV4QMat(W.ctypes.data, S.ctypes.data, dsv4.WFP8, 4, 32, 0, 128)
    assert L.dsv4_gpu_upload(ctypes.byref(m8)) == -1          # no row blocking
    mnull = dsv4.DSV4QMat(None, None, dsv4.WFP8, 4, 32, 128, 128)
    assert L.dsv4_gpu_upload(ctypes.byref(mnull)) == -1
    huge = dsv4.DSV4QMat(W.ctypes.data, S.ctypes.data, dsv4.WFP8, 1 << 30, 1 << 30, 128, 128)
    assert L.dsv4_gpu_upload(ctypes.byref(huge)) == -1          # no room: recoverable
