"""GPU parity of the HIP kernels against the CPU oracle (through the C ABI).

Bars: dequantisation, RoPE and the synthetic generator are bit-exact; matvec,
attention and the elementwise ops are within 1e-4 max relative error per
element (relative to max(|ref|, 1e-3 * max|ref|), see helpers.rel_err) and
inside the float64 accumulation bound.
"""
import numpy as np
import pytest

from helpers import (F32, Q2_K, Q3_K, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0, Q8_K, QUANT_TYPES, GEOM, NAMES,
                     PACK_REGIONS, assert_close, assert_close_scaled, pack_host, random_matrix, rel_err,
                     scaled_err, zero_code_patch)

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _rf():
    import ramforge_amd as rf

    return rf


def _with_subnormal_scales(t, raw, rng):
    """Force some f16 scale fields into the subnormal range (the reference
    decodes them at half their IEEE value)."""
    qk, bs = GEOM[t]
    blocks = raw.reshape(-1, bs)
    offs = {Q8_0: [0], Q4_0: [0], Q5_0: [0], Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208], Q2_K: [80, 82],
            Q3_K: [108]}.get(t, [])
    for o in offs:
        sel = rng.random(len(blocks)) < 0.3
        sub = rng.integers(1, 1024, size=sel.sum()).astype(np.uint16)
        blocks[sel, o:o + 2] = sub.view(np.uint8).reshape(-1, 2)
    return blocks.reshape(-1)


# ------------------------------------------------------------- dequant

@pytest.mark.parametrize("t", QUANT_TYPES + [F32])
def test_dequant_rows_bit_exact(ctx, orc, t):
    rf = _rf()
    rng = np.random.default_rng(100 + t)
    in_dim = 512 if GEOM[t][0] == 256 else 96
    rows = 9
    raw = _with_subnormal_scales(t, random_matrix(t, rows, in_dim, rng), rng)
    w = ctx.array(raw)
    out = ctx.empty((rows, in_dim))
    rf.dequantize_rows(ctx, t, w, in_dim, 0, rows, out)
    got = out.numpy()
    if t == F32:
        ref = raw.view(np.float32).reshape(rows, in_dim)
    else:
        ref = orc.dequantize_rows(t, raw, in_dim, rows)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), NAMES[t]
    # a row range decodes the same rows
    out2 = ctx.empty((3, in_dim))
    rf.dequantize_rows(ctx, t, w, in_dim, 4, 3, out2)
    assert np.array_equal(out2.numpy().view(np.uint32), ref[4:7].view(np.uint32))
    for a in (w, out, out2):
        a.free()


def test_dequant_f16_bf16_rows(ctx, orc):
    rf = _rf()
    bits = np.arange(65536, dtype=np.uint16)
    for t in (1, 30):
        w = ctx.array(bits.view(np.uint8))
        out = ctx.empty((65536,))
        rf.dequantize_rows(ctx, t, w, 65536, 0, 1, out)
        ref = orc.dequantize_row(t, bits.view(np.uint8), 65536)
        assert np.array_equal(out.numpy().view(np.uint32), ref.view(np.uint32))
        w.free()
        out.free()


def test_dequant_validation(ctx):
    rf = _rf()
    w = ctx.array(np.zeros(34, np.uint8))
    out = ctx.empty((64,))
    with pytest.raises(rf.RamforgeError, match="row truncated"):
        rf.dequantize_rows(ctx, Q8_0, w, 64, 0, 1, out)
    with pytest.raises(rf.RamforgeError, match="not divisible"):
        rf.dequantize_rows(ctx, Q8_0, w, 31, 0, 1, out)
    # sizes computed from the shape must not wrap past the bounds check
    with pytest.raises(rf.RamforgeError, match="overflows"):
        rf.dequantize_rows(ctx, Q8_0, w, 1 << 40, 1 << 30, 1 << 30, out.ptr)
    with pytest.raises(rf.RamforgeError, match="overflows"):
        rf.dequantize_rows(ctx, Q8_0, w, 32, (1 << 64) - 2, 4, out.ptr)
    w.free()
    out.free()


def test_device_array_views_stay_in_their_buffer(ctx):
    with pytest.raises(ValueError, match="exceeds"):
        ctx.alloc(8, shape=(4,), dtype=np.float32)
    a = ctx.alloc(8, shape=(2,), dtype=np.float32)
    a.shape = (4,)
    with pytest.raises(ValueError, match="view"):
        a.numpy()
    a.free()


# -------------------------------------------------------------- matvec

def _check_matvec(ctx, orc, t, out_dim, in_dim, seed, row_start=0, row_count=None, threads=16, x_off=0, w_off=0):
    """x_off / w_off place x and the weights that many bytes past a 256-byte
    aligned allocation (the tiled kernels need 16-byte aligned x)."""
    rf = _rf()
    rng = np.random.default_rng(seed)
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    print(f"  matvec {NAMES[t]} out={out_dim} in={in_dim} rows={row_start}+{row_count} seed={seed} "
          f"x_off={x_off} w_off={w_off}", flush=True)
    w = ctx.array(np.concatenate([np.zeros(w_off, np.uint8), raw]))
    xd = ctx.array(np.concatenate([np.zeros(x_off, np.uint8), x.view(np.uint8)]))
    n = out_dim - row_start if row_count is None else row_count
    y = ctx.empty((n,))
    rf.matvec(ctx, t, w.ptr + w_off, (out_dim, in_dim), xd.ptr + x_off, y, row_start, row_count,
              w_bytes=raw.nbytes)
    got = y.numpy()
    if t == F32:
        ref = orc.backend_matvec_f32(raw.view(np.float32), in_dim, out_dim, x, threads, True)
        wdec = raw.view(np.float32).reshape(out_dim, in_dim)
    else:
        ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, threads)
        wdec = orc.dequantize_rows(t, raw, in_dim, out_dim)
    ref = ref[row_start:row_start + n]
    w64 = wdec[row_start:row_start + n].astype(np.float64)
    scale = np.abs(w64) @ np.abs(x.astype(np.float64))
    err = assert_close_scaled(got, ref, scale, TOL, what=f"{NAMES[t]} {out_dim}x{in_dim}")
    ref64 = w64 @ x.astype(np.float64)
    assert np.all(np.abs(got - ref64) <= scale * 64 * 2.0 ** -24), NAMES[t]
    print(f"    scaled rel err vs oracle {err:.2e}; plain rel err {rel_err(got, ref):.2e}; "
          f"oracle vs f64 {scaled_err(ref, ref64, scale):.2e}, gpu vs f64 {scaled_err(got, ref64, scale):.2e}",
          flush=True)
    for a in (w, xd, y):
        a.free()
    return err


@pytest.fixture(params=[2, 1, 0], ids=["wave", "stream", "oneshot"])
def kernel_mode(request):
    rf = _rf()
    old = rf.tune_matvec_kernel(-1)
    rf.tune_matvec_kernel(request.param)
    yield request.param
    rf.tune_matvec_kernel(old)


WAVE_SHAPES_32 = [(1, 64), (7, 128), (513, 4096), (130, 2048), (33, 4096), (4096, 4096), (6000, 1024), (7000, 4096),
                  (6200, 1088), (300, 9024), (64, 14336), (41, 16448)]
WAVE_SHAPES_256 = [(1, 512), (7, 1024), (513, 4096), (130, 2048), (4096, 4096), (6000, 1024), (7000, 4096),
                   (6200, 1536), (77, 1536), (300, 10240), (64, 14336), (41, 16384)]


WAVE_SHAPES_F32 = [(1, 32), (7, 96), (513, 4096), (4096, 4096), (6000, 1024), (300, 9024), (77, 16384)]


@pytest.mark.parametrize("t,out_dim,in_dim", [(t, o, n) for t in (Q8_0, Q4_0) for o, n in WAVE_SHAPES_32] +
                         [(t, o, n) for t in (Q4_K, Q6_K) for o, n in WAVE_SHAPES_256] +
                         [(F32, o, n) for o, n in WAVE_SHAPES_F32])
def test_matvec_wave_kernel_shapes(ctx, orc, t, out_dim, in_dim):
    """The wave-staged kernel (plain Q8_0 / Q4_0 / Q4_K / Q6_K rf_matvec):
    rows that leave wavefronts of a workgroup idle, four- and eight-wavefront
    workgroups and more than one row per wavefront (6000 rows), x held in
    registers (7000 and 6200 rows, the second with a partial step: 16
    blocks per step for Q8_0 / Q4_0, 4 super-blocks for Q4_K, 2 for Q6_K),
    partial steps with x read from LDS, and rows longer than one 8 KiB item
    (Q8_0 at 9024 and 14336 inputs, Q4_0 at 16448, Q6_K at 10240 and 14336:
    two chunks per row; Q4_K rows of more than 4096 inputs take the
    streaming kernel).  F32 rows take the per-wavefront F32 kernel: items of
    2048 floats, the last one partial (96, 9024), up to 8 per row (16384)."""
    rf = _rf()
    assert rf.tune_matvec_kernel(-1) == 2
    _check_matvec(ctx, orc, t, out_dim, in_dim, 1500 + out_dim + in_dim + t)


@pytest.mark.parametrize("t", [Q4_K, Q8_0])
@pytest.mark.parametrize("case", ["pinf", "both", "nan"])
def test_matvec_wave_nonfinite_x_in_registers(ctx, orc, t, case):
    """x holding infinities or a NaN on the wave-staged kernel's
    x-in-registers path (7000 rows): every row's kind (NaN, +inf, -inf)
    equals the oracle's.  Q4_K switches the eight-element shares that meet a
    non-finite x to the kind of the reference's terms."""
    rf = _rf()
    rng = np.random.default_rng(2250 + t)
    out_dim, in_dim = 7000, 1024
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    if case in ("pinf", "both"):
        x[70] = np.inf
    if case == "both":
        x[900] = -np.inf
    if case == "nan":
        x[513] = np.nan
    print(f"  wave kernel non-finite x {NAMES[t]} {case}", flush=True)
    w, xd, y = ctx.array(raw), ctx.array(x), ctx.empty((out_dim,))
    rf.matvec(ctx, t, w, (out_dim, in_dim), xd, y)
    got = y.numpy()
    with np.errstate(all="ignore"):
        ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, 16)
    for kind in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(kind(got), kind(ref)), (NAMES[t], case, kind.__name__)
    for a in (w, xd, y):
        a.free()


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q6_K])
def test_matvec_wave_kernel_offsets(ctx, orc, t):
    """Row ranges (the base moves by whole rows, still dword aligned), a
    weight base 4 bytes past an aligned allocation (the wave-staged kernel)
    and 2 bytes past (not dword aligned: the other kernels)."""
    for i, (rs, rc, w_off) in enumerate(((37, 100, 0), (0, None, 4), (5, 11, 2), (299, 1, 4))):
        _check_matvec(ctx, orc, t, 300, 4096, 1600 + i, row_start=rs, row_count=rc, w_off=w_off)


@pytest.mark.parametrize("t", QUANT_TYPES + [F32])
def test_matvec_small_shapes(ctx, orc, t, kernel_mode):
    qk = GEOM[t][0]
    shapes = [(67, 512), (1, 256), (130, 1024)] if qk == 256 else [(67, 96), (3, 32), (130, 1024), (33, 4096)]
    for i, (o, n) in enumerate(shapes):
        _check_matvec(ctx, orc, t, o, n, 200 + 10 * t + i)


@pytest.mark.parametrize("t", [Q4_0, Q6_K, Q8_0, F32])
def test_matvec_row_range_is_local(ctx, orc, t, kernel_mode):
    in_dim = 512
    _check_matvec(ctx, orc, t, 300, in_dim, 300 + t, row_start=128, row_count=77)
    _check_matvec(ctx, orc, t, 300, in_dim, 310 + t, row_start=299, row_count=None)


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K, F32])
def test_matvec_unaligned_pointers(ctx, orc, t, kernel_mode):
    # x 4 bytes off 16-byte alignment takes the rowwise kernel; weights 2 bytes
    # off take the one-shot tiled kernel (the streaming kernel needs 16 bytes)
    _check_matvec(ctx, orc, t, 70, 512, 350 + t, x_off=4)
    _check_matvec(ctx, orc, t, 70, 512, 360 + t, w_off=2)
    _check_matvec(ctx, orc, t, 70, 512, 370 + t, x_off=8, w_off=6, row_start=5, row_count=40)


# Formats whose codes are signed offsets (no min term): a zero code decodes to
# an exact 0 weight.
ZERO_CODE_TYPES = [Q8_0, Q4_0, Q5_0, Q6_K, Q3_K, Q8_K]


def _outlier_elems(t):
    return [5, 21] if GEOM[t][0] == 32 else list(range(5, 256, 16))


@pytest.mark.parametrize("t", ZERO_CODE_TYPES)
def test_matvec_zero_code_outliers(ctx, orc, t, kernel_mode):
    """Every 16-element unit of x holds one 1e4 element that meets a zero
    weight in every row; the row sums come from the 1e-3 elements.  The
    reference's terms (q * d) * x are exact there (a zero term adds
    nothing), and so are the kernels' signed-code products: the 1e-4 bar and
    the float64 bound hold.  A q + offset decode would lose the small terms
    against the 1e4 * offset it subtracts again."""
    rf = _rf()
    rng = np.random.default_rng(2100 + t)
    out_dim, in_dim = 300, 4096
    raw = zero_code_patch(t, random_matrix(t, out_dim, in_dim, rng), _outlier_elems(t))
    x = rng.normal(0, 1e-3, in_dim).astype(np.float32)
    x[5::16] = 1e4
    print(f"  zero-code outliers {NAMES[t]}", flush=True)
    w, xd, y = ctx.array(raw), ctx.array(x), ctx.empty((out_dim,))
    rf.matvec(ctx, t, w, (out_dim, in_dim), xd, y)
    got = y.numpy()
    ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, 16)
    wdec = orc.dequantize_rows(t, raw, in_dim, out_dim).astype(np.float64)
    scale = np.abs(wdec) @ np.abs(x.astype(np.float64))
    e = assert_close_scaled(got, ref, scale, TOL, what=f"{NAMES[t]} zero-code outliers")
    assert np.all(np.abs(got - wdec @ x.astype(np.float64)) <= scale * 64 * 2.0 ** -24)
    print(f"    scaled rel err {e:.2e}", flush=True)
    for a in (w, xd, y):
        a.free()


@pytest.mark.parametrize("t", QUANT_TYPES + [F32])
@pytest.mark.parametrize("case", ["pinf", "both", "nan"])
def test_matvec_nonfinite_x(ctx, orc, t, case, kernel_mode):
    """x holding infinities or a NaN through the GGUF-layout kernels: the
    kind of every row (NaN, +inf, -inf) equals the oracle's, i.e. the
    reference's terms (q * d) * x summed in order."""
    rf = _rf()
    rng = np.random.default_rng(2200 + t)
    out_dim, in_dim = 260, 2048
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    if case in ("pinf", "both"):
        x[70] = np.inf
    if case == "both":
        x[1500] = -np.inf
    if case == "nan":
        x[999] = np.nan
    w, xd, y = ctx.array(raw), ctx.array(x), ctx.empty((out_dim,))
    rf.matvec(ctx, t, w, (out_dim, in_dim), xd, y)
    got = y.numpy()
    with np.errstate(all="ignore"):
        if t == F32:
            ref = orc.backend_matvec_f32(raw.view(np.float32), in_dim, out_dim, x, 16, True)
        else:
            ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, 16)
    for kind in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(kind(got), kind(ref)), (NAMES[t], case, kind.__name__)
    for a in (w, xd, y):
        a.free()


PACKED = [Q8_0, Q4_0, Q4_K, Q6_K]
_pack_host = pack_host


@pytest.mark.parametrize("t", PACKED)
def test_pack_weights_layout_is_exact(ctx, t):
    rf = _rf()
    rng = np.random.default_rng(40 + t)
    for rows, in_dim in ((3, 256), (17, 4096), (5, 14336)):
        raw = random_matrix(t, rows, in_dim, rng)
        w = ctx.array(raw)
        p = ctx.empty((raw.nbytes,), np.uint8)
        rf.pack_weights(ctx, t, w, rows, in_dim, p)
        assert np.array_equal(p.numpy(), _pack_host(t, raw, rows, in_dim)), (NAMES[t], rows, in_dim)
        w.free()
        p.free()


def _digit_bound(wdec, x):
    """Documented bound of the digit-plane decode beyond f32 rounding: sum
    over 16-element units u of 2^(E_u - 31) sum_k |w_k|, with 2^E_u the power
    of two above the unit's largest |x| (E_u >= -96)."""
    units = np.abs(x.astype(np.float64)).reshape(-1, 16)
    _, e = np.frexp(units.max(axis=1))
    e = np.maximum(e, -96)
    wu = np.abs(wdec).reshape(wdec.shape[0], -1, 16).sum(axis=2)
    return wu @ np.ldexp(1.0, e - 31)


def _check_matvec_packed(ctx, orc, t, out_dim, in_dim, seed, row_start=0, row_count=None, x_off=0, patch=None,
                         xgen=None, digits=False, bar=True):
    rf = _rf()
    rng = np.random.default_rng(seed)
    raw = random_matrix(t, out_dim, in_dim, rng)
    if patch is not None:
        raw = patch(raw.copy(), rng)
    x = (rng.normal(0, 1, in_dim) if xgen is None else xgen(rng, in_dim)).astype(np.float32)
    print(f"  packed matvec {NAMES[t]} out={out_dim} in={in_dim} rows={row_start}+{row_count} seed={seed} "
          f"x_off={x_off}", flush=True)
    w = ctx.array(_pack_host(t, raw, out_dim, in_dim))
    xd = ctx.array(np.concatenate([np.zeros(x_off, np.uint8), x.view(np.uint8)]))
    n = out_dim - row_start if row_count is None else row_count
    y = ctx.empty((n,))
    rf.matvec_packed(ctx, t, w, (out_dim, in_dim), xd.ptr + x_off, y, row_start, row_count)
    got = y.numpy()
    ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, 16)[row_start:row_start + n]
    wdec = orc.dequantize_rows(t, raw, in_dim, out_dim)[row_start:row_start + n].astype(np.float64)
    scale = np.abs(wdec) @ np.abs(x.astype(np.float64))
    allowed = scale * 64 * 2.0 ** -24 + (_digit_bound(wdec, x) if digits else 0.0)
    dev = np.abs(got - wdec @ x.astype(np.float64))
    assert np.all(dev <= allowed), (NAMES[t], float(np.max(dev / np.maximum(allowed, 1e-300))))
    err = scaled_err(got, ref, scale)
    if bar:
        assert err <= TOL, f"packed {NAMES[t]} {out_dim}x{in_dim}: max scaled relative error {err:.3e} > {TOL:.1e}"
    print(f"    scaled rel err vs oracle {err:.2e}, float64 deviation {np.max(dev / allowed):.2f} of its bound",
          flush=True)
    for a in (w, xd, y):
        a.free()


@pytest.mark.parametrize("t", PACKED)
@pytest.mark.parametrize("out_dim,in_dim", [(1, 32), (67, 96), (3, 256), (130, 1024), (33, 2048), (70, 3072),
                                            (11, 3328), (257, 4096), (1000, 5120), (4096, 4096), (14336, 4096),
                                            (4096, 14336), (9, 16384), (5, 28672)])
def test_matvec_packed_shapes(ctx, orc, t, out_dim, in_dim):
    if in_dim % GEOM[t][0]:
        pytest.skip(f"{NAMES[t]} rows are whole {GEOM[t][0]}-element blocks")
    if not _rf().packed_supported(t, in_dim):
        # x of a row must fit the workgroup's LDS (64 KiB, or what the device allows)
        pytest.skip(f"in_dim {in_dim} exceeds this device's LDS for {NAMES[t]}")
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 1200 + t + in_dim % 977 + out_dim)


def _x_wide_range(rng, n):
    """x whose 16-element units span many magnitudes: per-element log-normal
    spread, whole units of zeros, of f32 subnormals and of values near 1e30."""
    x = rng.normal(0, 1, n) * np.exp(rng.normal(0, 4, n))
    u = x.reshape(-1, 16)
    u[3::29] = 0.0
    u[5::31] = rng.normal(0, 1, (len(u[5::31]), 16)) * 1e-40
    u[7::37] = rng.normal(0, 1, (len(u[7::37]), 16)) * 1e30
    u[9::41, 3] = 0.0
    return x


# Shapes whose wavefronts hold at least 24 KiB of codes on a 256-CU device,
# where Q8_0 and Q4_0 take x as int8 digit planes in digit mode 1 (Q8_0:
# 3 rows of 8192 codes per wavefront; Q4_0 12288 x 16384: 3 rows of 8192
# bytes per wavefront of 1024-thread workgroups); the others above use the
# float path unless digits are forced.
@pytest.mark.parametrize("digits_mode", [1], indirect=True, ids=["auto"])
@pytest.mark.parametrize("t,out_dim,in_dim", [(Q8_0, 6144, 8192), (Q4_0, 12288, 16384), (Q8_0, 28672, 8192)])
@pytest.mark.parametrize("xkind", ["normal", "wide"])
def test_matvec_packed_digit_planes(ctx, orc, digits_mode, t, out_dim, in_dim, xkind):
    if not _rf().packed_supported(t, in_dim):
        pytest.skip(f"in_dim {in_dim} exceeds this device's LDS for {NAMES[t]}")
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 1500 + t + out_dim % 97,
                         xgen=_x_wide_range if xkind == "wide" else None, digits=True)


@pytest.fixture
def digits_mode(request):
    """rf_tune_matvec_digits for the test: 0 float x, 2 digit planes on every
    packed Q8_0 / Q4_0 launch whose LDS holds them."""
    rf = _rf()
    old = rf.tune_matvec_digits(-1)
    assert rf.tune_matvec_digits(request.param) == request.param
    yield request.param
    rf.tune_matvec_digits(old)


@pytest.mark.parametrize("digits_mode", [2], indirect=True, ids=["forced"])
@pytest.mark.parametrize("t", [Q8_0, Q4_0])
@pytest.mark.parametrize("out_dim,in_dim", [(1, 32), (67, 96), (130, 1024), (257, 4096), (4096, 4096),
                                            (14336, 4096), (4096, 14336), (9, 16384)])
def test_matvec_packed_forced_digit_planes(ctx, orc, digits_mode, t, out_dim, in_dim):
    """The digit-plane decode on every shape (forced), against the oracle's
    bar and its documented bound: each x element is off by at most
    2^(E_u - 31), 2^E_u the power of two above its 16-element unit's largest
    |x|."""
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 1600 + t + out_dim, digits=True)
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 1650 + t + out_dim, xgen=_x_wide_range, digits=True)


@pytest.mark.parametrize("digits_mode", [2], indirect=True, ids=["forced"])
@pytest.mark.parametrize("t", [Q8_0, Q4_0])
def test_matvec_packed_digit_rows_and_unaligned_x(ctx, orc, digits_mode, t):
    _check_matvec_packed(ctx, orc, t, 300, 4096, 1700 + t, row_start=128, row_count=77, digits=True)
    _check_matvec_packed(ctx, orc, t, 50, 2048, 1720 + t, x_off=4, digits=True)


def _x_outlier_channels(rng, n):
    """Activations with outlier channels: normal x with every 64th element
    200-2000 times larger (the units holding one meet the codes of all
    rows, zeros included)."""
    x = rng.normal(0, 1, n)
    x[7::64] *= rng.uniform(200, 2000, len(x[7::64])) * rng.choice([-1, 1], len(x[7::64]))
    return x


def _x_adversarial(rng, n):
    """Every 16-element unit: one element of 1e4, fifteen of about 1e-3."""
    x = rng.normal(0, 1e-3, n)
    x[5::16] = 1e4
    return x


def _zero_codes_at(t, positions):
    """Patch: the codes of block elements `positions` are the zero weight."""
    return lambda raw, rng: zero_code_patch(t, raw, positions)


@pytest.mark.parametrize("digits_mode", [2, 0], indirect=True, ids=["digits", "float"])
@pytest.mark.parametrize("t", [Q8_0, Q4_0])
def test_matvec_packed_outlier_channels(ctx, orc, digits_mode, t):
    """Realistic activation outliers (200-2000x in one channel of 64): both
    decodes meet the 1e-4 bar."""
    _check_matvec_packed(ctx, orc, t, 2048, 4096, 1800 + t, xgen=_x_outlier_channels, digits=digits_mode == 2)


@pytest.mark.parametrize("digits_mode", [2, 0], indirect=True, ids=["digits", "float"])
@pytest.mark.parametrize("t", [Q8_0, Q4_0])
def test_matvec_packed_adversarial_units(ctx, orc, digits_mode, t):
    """The digit decode's worst case: every unit's 1e4 element meets a zero
    weight and the row sum is made of the 1e-3 elements, which keep about 6
    bits below their unit's 2^14.  The float decode meets the 1e-4 bar; the
    digit decode stays inside its documented bound (and is not expected to
    meet the bar: its deviation from the reference's arithmetic shows here,
    which is why mode 0 exists)."""
    _check_matvec_packed(ctx, orc, t, 512, 4096, 1900 + t, xgen=_x_adversarial, patch=_zero_codes_at(t, [5, 21]),
                         digits=digits_mode == 2, bar=digits_mode == 0)


@pytest.mark.parametrize("digits_mode", [2, 0], indirect=True, ids=["digits", "float"])
@pytest.mark.parametrize("t", PACKED)
@pytest.mark.parametrize("case", ["pinf", "ninf", "both", "nan"])
def test_matvec_packed_nonfinite_x(ctx, orc, digits_mode, t, case):
    """x holding infinities or a NaN: every row is non-finite, and which of
    NaN, +inf or -inf it is follows from the reference's terms (decoded
    weight times x: NaN for a zero weight at an infinity, or for infinite
    terms of both signs).  The kinds must equal the oracle's row for row."""
    rf = _rf()
    rng = np.random.default_rng(2000 + t)
    out_dim, in_dim = 700, 4096
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    if case in ("pinf", "both"):
        x[100] = np.inf
    if case in ("ninf", "both"):
        x[2049] = -np.inf
    if case == "nan":
        x[3000] = np.nan
    w = ctx.array(pack_host(t, raw, out_dim, in_dim))
    xd = ctx.array(x)
    y = ctx.empty((out_dim,))
    rf.matvec_packed(ctx, t, w, (out_dim, in_dim), xd, y)
    got = y.numpy()
    with np.errstate(all="ignore"):
        ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, 16)
    assert not np.isfinite(ref).any()
    for kind in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(kind(got), kind(ref)), (NAMES[t], case, kind.__name__)
    print(f"  {NAMES[t]} {case}: {np.isnan(ref).sum()} NaN, {np.isposinf(ref).sum()} +inf, "
          f"{np.isneginf(ref).sum()} -inf rows as the oracle", flush=True)
    for a in (w, xd, y):
        a.free()


@pytest.fixture
def inflight_mode(request):
    """rf_tune_packed_inflight for the test: 1 one-row-per-wavefront launches
    request their rows before staging x, 0 the two-step ring everywhere."""
    rf = _rf()
    old = rf.tune_packed_inflight(-1)
    assert rf.tune_packed_inflight(request.param) == request.param
    yield request.param
    rf.tune_packed_inflight(old)


@pytest.mark.parametrize("inflight_mode", [1, 0], indirect=True, ids=["inflight", "ring"])
@pytest.mark.parametrize("t", PACKED)
@pytest.mark.parametrize("out_dim,in_dim", [(4096, 4096), (1000, 4096), (2048, 4096), (2048, 2048), (3072, 2048)])
def test_matvec_packed_inflight_shapes(ctx, orc, inflight_mode, t, out_dim, in_dim):
    """in_dim 4096 launches with one row per wavefront (all requested before
    the x prologue) and with the ring, against the oracle; rows of 2048
    inputs (config 4's widths) take the ring in both modes."""
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 2300 + t + out_dim)
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 2310 + t + out_dim, row_start=7, row_count=out_dim - 20)


@pytest.mark.parametrize("inflight_mode", [1, 0], indirect=True, ids=["inflight", "ring"])
@pytest.mark.parametrize("t", PACKED)
@pytest.mark.parametrize("out_dim,in_dim", [(4096, 14336), (3000, 14336), (6144, 4096), (8000, 4096)])
def test_matvec_packed_model_shapes(ctx, orc, inflight_mode, t, out_dim, in_dim):
    """The 8B down-projection width (14336 inputs: four steps of a row) and
    Q/K/V-like row counts (several rows per wavefront), both launch modes."""
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 2400 + t + out_dim)
    _check_matvec_packed(ctx, orc, t, out_dim, in_dim, 2410 + t + out_dim, row_start=5, row_count=out_dim - 9)


@pytest.mark.parametrize("t", PACKED)
def test_matvec_packed_row_range_and_unaligned_x(ctx, orc, t):
    _check_matvec_packed(ctx, orc, t, 300, 4096, 1300 + t, row_start=128, row_count=77)
    _check_matvec_packed(ctx, orc, t, 300, 4096, 1310 + t, row_start=299)
    _check_matvec_packed(ctx, orc, t, 50, 2048, 1320 + t, x_off=4)


# byte offsets of the f16 super-scales of a block (Q4_K: d and dmin)
F16_SCALES = {Q8_0: [0], Q4_0: [0], Q4_K: [0, 2], Q6_K: [208]}


@pytest.mark.parametrize("t", PACKED)
def test_matvec_packed_subnormal_and_signed_scales(ctx, orc, t):
    """Every f16 block scale (and Q4_K min scale) an f16 subnormal (the
    reference decodes frac * 2^-25, half the IEEE value), +-0 or negative: the
    packed kernel's hardware f16 conversion plus its subnormal rule against
    the oracle.  With no normal scale in the matrix, a scale off by 2x would
    show at full size."""
    def patch(raw, rng):
        bs = GEOM[t][1]
        blocks = raw.reshape(-1, bs)
        for off in F16_SCALES[t]:
            sc = rng.integers(1, 0x400, len(blocks)).astype(np.uint16)
            sc[::3] |= 0x8000
            sc[1::7] = 0
            sc[2::11] = 0x8000
            blocks[:, off:off + 2] = sc.view(np.uint8).reshape(-1, 2)
        return raw

    _check_matvec_packed(ctx, orc, t, 96, 3072, 1400 + t, patch=patch)


def test_matvec_packed_validation(ctx):
    rf = _rf()
    w = ctx.array(np.zeros(34 * 4, np.uint8))
    x = ctx.array(np.zeros(256, np.float32))
    y = ctx.array(np.full(2, 7.0, np.float32))
    with pytest.raises(rf.RamforgeError, match="truncated"):
        rf.matvec_packed(ctx, Q8_0, w, (2, 128), x, y)
    with pytest.raises(rf.RamforgeError, match="not divisible"):
        rf.matvec_packed(ctx, Q8_0, w, (2, 100), x, y)
    with pytest.raises(rf.RamforgeError, match="exceeds out_dim"):
        rf.matvec_packed(ctx, Q8_0, w, (1, 128), x, y, 2)
    with pytest.raises(rf.RamforgeError, match="does not support"):
        rf.matvec_packed(ctx, Q5_K, w, (1, 256), x, y)
    with pytest.raises(rf.RamforgeError, match="overflows"):  # 2^40 rows of 2^40 elements
        rf.matvec_packed(ctx, Q8_0, w, (1 << 40, 1 << 40), x.ptr, y, 0, 1)
    assert y.numpy().tolist() == [7.0, 7.0]  # destination untouched
    assert not rf.packed_supported(Q8_0, 1 << 16) and rf.packed_supported(Q4_0, 14336)
    assert rf.packed_supported(Q8_0, 14336) and not rf.packed_supported(Q8_0, 100)
    assert rf.packed_supported(Q4_K, 14336) and not rf.packed_supported(Q4_K, 4000)
    assert rf.packed_supported(Q6_K, 4096) and not rf.packed_supported(Q5_K, 4096)
    for a in (w, x, y):
        a.free()


def test_capture_replay_matches_eager(ctx):
    """rf_capture_begin/end + rf_graph_replay: the recorded launches replay to
    the eager result; replays interleave with eager work."""
    rf = _rf()
    rng = np.random.default_rng(77)
    raw = random_matrix(Q8_0, 257, 4096, rng)
    w, p = ctx.array(raw), ctx.empty((raw.nbytes,), np.uint8)
    rf.pack_weights(ctx, Q8_0, w, 257, 4096, p)
    x = ctx.array(rng.normal(0, 1, 4096).astype(np.float32))
    y1, y2 = ctx.empty((257,)), ctx.empty((257,))
    rf.matvec(ctx, Q8_0, w, (257, 4096), x, y1)
    rf.matvec_packed(ctx, Q8_0, p, (257, 4096), x, y2)
    e1, e2 = y1.numpy(), y2.numpy()
    y1.upload(np.zeros(257, np.float32))
    y2.upload(np.zeros(257, np.float32))
    with ctx.capture() as cap:
        rf.matvec(ctx, Q8_0, w, (257, 4096), x, y1)
        rf.matvec_packed(ctx, Q8_0, p, (257, 4096), x, y2)
    g = cap.graph
    for _ in range(3):
        ms = g.replay(2)
        assert ms > 0
        assert np.array_equal(y1.numpy(), e1) and np.array_equal(y2.numpy(), e2)
        y1.upload(np.zeros(257, np.float32))
        rf.matvec(ctx, Q8_0, w, (257, 4096), x, y1)  # eager work between replays
    g.close()
    for a in (w, p, x, y1, y2):
        a.free()


def test_matvec_f32_any_length_and_wide_rows(ctx, orc):
    _check_matvec(ctx, orc, F32, 5, 100, 401)     # in_dim not a multiple of 32: rowwise kernel
    _check_matvec(ctx, orc, Q8_0, 40, 40960, 402)  # > 1024 units per row: rowwise kernel
    _check_matvec(ctx, orc, Q4_K, 20, 33792, 403)


BASELINE_SHAPES = [(Q8_0, 4096, 4096), (Q4_0, 14336, 4096), (Q4_0, 4096, 14336), (Q4_K, 14336, 4096),
                   (Q4_K, 4096, 14336), (Q6_K, 14336, 4096), (Q6_K, 4096, 14336), (F32, 4096, 4096),
                   (Q8_0, 14336, 4096), (Q8_0, 4096, 14336)]


@pytest.mark.parametrize("t,out_dim,in_dim", BASELINE_SHAPES)
def test_matvec_baseline_shapes(ctx, orc, t, out_dim, in_dim, kernel_mode):
    _check_matvec(ctx, orc, t, out_dim, in_dim, 500 + t + out_dim % 97)


def test_matvec_kats(ctx):
    """quant.rs:1914-2175 matvec known answers through the HIP path."""
    rf = _rf()
    from helpers import h16, q4_0_block, q8_0_block

    cases = [(Q4_0, q4_0_block(0x3C00, [0x99] * 16) * 2, 32, 1.0, 32.0),
             (Q8_0, q8_0_block(0x3C00, [1] * 32) * 2, 32, 2.0, 64.0),
             (Q4_K, (h16(0x3C00) + h16(0) + bytes([1] * 12) + bytes([0x11] * 128)) * 2, 256, 1.0, 256.0),
             (Q5_K, (h16(0x3C00) + h16(0) + bytes([1] * 12) + bytes(32) + bytes([0x11] * 128)) * 2, 256, 1.0,
              256.0),
             (Q8_K, (np.float32(1).tobytes() + bytes([1] * 256) + bytes(32)) * 2, 256, 1.0, 256.0)]
    for t, raw, n, xv, expect in cases:
        w = ctx.array(np.frombuffer(raw, np.uint8))
        x = ctx.array(np.full(n, xv, np.float32))
        y = ctx.empty((2,))
        rf.matvec(ctx, t, w, (2, n), x, y)
        assert np.allclose(y.numpy(), expect, atol=1e-3), NAMES[t]
        for a in (w, x, y):
            a.free()


def test_matvec_validation_keeps_destination(ctx):
    rf = _rf()
    w = ctx.array(np.zeros(3 * 34, np.uint8))
    x = ctx.array(np.ones(32, np.float32))
    y = ctx.array(np.full(3, 7.0, np.float32))
    with pytest.raises(rf.RamforgeError, match="not divisible"):
        rf.matvec(ctx, Q8_0, w, (3, 31), x, y)
    # x / y lengths first, as quant.rs:990-997 (DeviceArray capacities here);
    # the library's own check of the weight bytes through a raw address
    with pytest.raises(rf.RamforgeError, match="matvec shape mismatch"):
        rf.matvec(ctx, Q8_0, w, (4, 32), x, y)
    with pytest.raises(rf.RamforgeError, match="weight truncated"):
        rf.matvec(ctx, Q8_0, w, (4, 32), x, y.ptr)
    with pytest.raises(rf.RamforgeError, match="exceeds out_dim"):
        rf.matvec(ctx, Q8_0, w, (3, 32), x, y, row_start=4)
    with pytest.raises(rf.RamforgeError, match="exceeds out_dim"):
        rf.matvec(ctx, Q8_0, w, (3, 32), x, y, row_start=2, row_count=2)
    with pytest.raises(rf.RamforgeError, match="does not support"):
        rf.matvec(ctx, 3, w, (3, 32), x, y)
    wf = ctx.array(np.zeros(6, np.float32))
    with pytest.raises(rf.RamforgeError, match="arity mismatch"):
        rf.GpuBackend(ctx).matvec(wf, [3, 2], ctx.array(np.ones(2, np.float32)), ctx.array(np.ones(3, np.float32)))
    assert np.all(y.numpy() == 7.0)


def test_matvec_backend_dispatch(ctx, orc):
    """compute_dispatch::matvec_backend: ggml [in, out] tensors."""
    rf = _rf()
    rng = np.random.default_rng(77)
    backend = rf.GpuBackend(ctx)
    for t in (Q4_0, Q6_K, Q8_0, F32):
        in_dim, out_dim = 512, 129
        raw = random_matrix(t, out_dim, in_dim, rng)
        x = rng.normal(0, 1, in_dim).astype(np.float32)
        td = rf.GpuTensor(t, (in_dim, out_dim), ctx.array(raw))
        y = ctx.empty((out_dim,))
        rf.matvec_backend(backend, td, ctx.array(x), y)
        ref = orc.dispatch_matvec(t, raw.view(np.float32) if t == F32 else raw, in_dim, out_dim, x, 4)
        wdec = raw.view(np.float32).reshape(out_dim, in_dim) if t == F32 else orc.dequantize_rows(t, raw, in_dim,
                                                                                                  out_dim)
        assert_close_scaled(y.numpy(), ref, np.abs(wdec.astype(np.float64)) @ np.abs(x.astype(np.float64)), TOL)


# ----------------------------------------------------------- attention

def _attention_case(ctx, orc, hist, qh, kvh, hd, seed, rope_pos=None):
    rf = _rf()
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, qh * hd).astype(np.float32)
    kh = rng.normal(0, 1, max(hist, 1) * kvh * hd).astype(np.float32)[: hist * kvh * hd]
    vh = rng.normal(0, 1, max(hist, 1) * kvh * hd).astype(np.float32)[: hist * kvh * hd]
    kc = rng.normal(0, 1, kvh * hd).astype(np.float32)
    vc = rng.normal(0, 1, kvh * hd).astype(np.float32)
    print(f"  attention hist={hist} qh={qh} kvh={kvh} hd={hd} rope={rope_pos} seed={seed}", flush=True)
    dq, dkc = ctx.array(q), ctx.array(kc)
    if rope_pos is not None:
        rf.apply_rope(ctx, dq, dkc, rope_pos, hd, qh, kvh, 10000.0)
        q, kc = orc.rope(q, kc, rope_pos, hd, qh, kvh, 10000.0)
        assert np.array_equal(dq.numpy().view(np.uint32), q.view(np.uint32)), "RoPE not bit-exact"
        assert np.array_equal(dkc.numpy().view(np.uint32), kc.view(np.uint32)), "RoPE not bit-exact"
    dkh = ctx.array(kh if hist else np.zeros(1, np.float32))
    dvh = ctx.array(vh if hist else np.zeros(1, np.float32))
    dvc = ctx.array(vc)
    out = rf.attention_checked(ctx, dq, dkh, dvh, dkc, dvc, hist, qh, kvh, hd)
    got = out.numpy()
    ref = orc.attention(q, kh, vh, kc, vc, hist, qh, kvh, hd)
    # term magnitude of each output element: sum_p softmax_p |v_p| (float64)
    K = np.concatenate([kh.reshape(hist, kvh, hd), kc.reshape(1, kvh, hd)]).astype(np.float64)
    Vv = np.concatenate([vh.reshape(hist, kvh, hd), vc.reshape(1, kvh, hd)]).astype(np.float64)
    scale = np.zeros((qh, hd))
    for h in range(qh):
        g = h * kvh // qh
        s = K[:, g] @ q.reshape(qh, hd)[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        scale[h] = (p / p.sum()) @ np.abs(Vv[:, g])
    e = assert_close_scaled(got, ref, scale.reshape(-1), TOL, what=f"attention hist={hist}")
    print(f"    scaled rel err {e:.2e}, plain rel err {rel_err(got, ref):.2e}", flush=True)
    for a in (dq, dkc, dkh, dvh, dvc, out):
        a.free()


def test_attention_gqa_kat(ctx):
    rf = _rf()
    q = ctx.array(np.array([1.0, 0.0, 0.0, 1.0], np.float32))
    kc = ctx.array(np.array([1.0, 0.0], np.float32))
    vc = ctx.array(np.array([2.0, 3.0], np.float32))
    z = ctx.array(np.zeros(1, np.float32))
    out = rf.attention_checked(ctx, q, z, z, kc, vc, 0, 2, 1, 2)
    assert out.numpy().tolist() == [2.0, 3.0, 2.0, 3.0]


@pytest.mark.parametrize("hist,qh,kvh,hd", [(0, 4, 2, 8), (7, 6, 3, 10), (0, 32, 8, 128), (1, 32, 8, 128),
                                            (100, 32, 8, 128), (300, 32, 8, 64), (77, 8, 8, 128),
                                            (64, 16, 2, 128), (33, 4, 1, 256)])
def test_attention_shapes(ctx, orc, hist, qh, kvh, hd):
    _attention_case(ctx, orc, hist, qh, kvh, hd, 600 + hist + qh + hd)


@pytest.mark.parametrize("hist,qh,kvh", [(63, 32, 8), (64, 32, 8), (127, 32, 8), (511, 32, 8), (512, 32, 8),
                                         (1023, 32, 8), (1024, 32, 8), (1087, 32, 8), (300, 64, 8), (1100, 64, 8),
                                         (20000, 32, 8), (5000, 8, 1)])
def test_attention_chunk_tree(ctx, orc, hist, qh, kvh):
    """Contexts on both sides of each launch-regime boundary (64, 64 Sq, 128 Sq
    positions with Sq = min(256 / qh, 8) chunks per query head; 64-position
    chunks per KV head; longer chunks): one chunk with direct output, and
    split + merge with empty trailing chunks.  Each case runs twice and must
    give the same bits."""
    rf = _rf()
    _attention_case(ctx, orc, hist, qh, kvh, 128, 900 + hist + qh)
    rng = np.random.default_rng(hist)
    hd = 128
    arrs = [rng.normal(0, 1, n).astype(np.float32) for n in (qh * hd, max(hist, 1) * kvh * hd,
                                                           max(hist, 1) * kvh * hd, kvh * hd, kvh * hd)]
    dev = [ctx.array(x) for x in arrs]
    first = rf.attention_checked(ctx, *dev, hist, qh, kvh, hd).numpy()
    second = rf.attention_checked(ctx, *dev, hist, qh, kvh, hd).numpy()
    assert np.array_equal(first.view(np.uint32), second.view(np.uint32))
    for a in dev:
        a.free()


@pytest.mark.parametrize("mode", [0, 2], ids=["two-pass", "one-pass"])
@pytest.mark.parametrize("hist,qh,kvh,hd", [(0, 32, 8, 128), (63, 32, 8, 128), (127, 32, 8, 128),
                                            (1087, 32, 8, 128), (8191, 32, 8, 128), (5000, 8, 1, 128),
                                            (300, 64, 8, 64), (700, 16, 2, 256), (33, 4, 1, 256)])
def test_attention_kernel_modes(ctx, orc, mode, hist, qh, kvh, hd):
    """Both decode attention kernels on every launch regime (mode 2 runs the
    one-pass online-softmax kernel per KV head too, mode 0 the two-pass
    kernel per query head too), against the oracle."""
    rf = _rf()
    old = rf.tune_attention_kernel(-1)
    rf.tune_attention_kernel(mode)
    try:
        _attention_case(ctx, orc, hist, qh, kvh, hd, 1200 + hist + qh + hd, rope_pos=hist)
    finally:
        rf.tune_attention_kernel(old)


@pytest.mark.parametrize("ctx_len", [512, 2048, 8192])
def test_attention_baseline_config(ctx, orc, ctx_len):
    """32 q heads, 8 KV heads, hd 128, RoPE theta 1e4 at
    position hist = L - 1, so L positions are attended."""
    _attention_case(ctx, orc, ctx_len - 1, 32, 8, 128, 700 + ctx_len, rope_pos=ctx_len - 1)


def test_attention_validation(ctx):
    rf = _rf()
    z = ctx.array(np.zeros(64, np.float32))
    with pytest.raises(rf.RamforgeError, match="divisible"):
        rf.attention_checked(ctx, z, z, z, z, z, 0, 3, 2, 8)
    with pytest.raises(rf.RamforgeError, match="non-zero"):
        rf.attention_checked(ctx, z, z, z, z, z, 0, 0, 1, 8)


# --------------------------------------------------------- elementwise

def test_rope_bit_exact(ctx, orc):
    rf = _rf()
    rng = np.random.default_rng(801)
    for hd, qh, kvh in ((128, 32, 8), (64, 4, 4), (2, 1, 1)):
        for pos in (0, 1, 255, 8191):
            q = rng.normal(0, 1, qh * hd).astype(np.float32)
            k = rng.normal(0, 1, kvh * hd).astype(np.float32)
            dq, dk = ctx.array(q), ctx.array(k)
            rf.apply_rope(ctx, dq, dk, pos, hd, qh, kvh, 10000.0)
            rq, rk = orc.rope(q, k, pos, hd, qh, kvh, 10000.0)
            assert np.array_equal(dq.numpy().view(np.uint32), rq.view(np.uint32)), (hd, pos)
            assert np.array_equal(dk.numpy().view(np.uint32), rk.view(np.uint32)), (hd, pos)
            dq.free()
            dk.free()


def test_elementwise_ops(ctx, orc):
    rf = _rf()
    rng = np.random.default_rng(802)
    for n in (2, 4096, 14336):
        a = rng.normal(0, 2, n).astype(np.float32)
        b = rng.normal(1, 0.5, n).astype(np.float32)
        da, db, do = ctx.array(a), ctx.array(b), ctx.empty((n,))
        rf.rmsnorm(ctx, da, db, n, 1e-5, do)
        assert_close(do.numpy(), orc.rms_norm(a, b, 1e-5), 1e-5)
        rf.add(ctx, da, db, n, do)
        assert np.array_equal(do.numpy(), orc.add(a, b))
        rf.mul(ctx, da, db, n, do)
        assert np.array_equal(do.numpy(), orc.mul(a, b))
        dv = ctx.array(a)
        rf.bias_add(ctx, dv, db, n)  # in place, model_executor.rs:178-186
        assert np.array_equal(dv.numpy(), orc.add(a, b))
        dv.free()
        rf.silu(ctx, da, n, do)
        assert_close(do.numpy(), orc.silu(a), 1e-6)
        rf.swiglu(ctx, da, db, n, do)
        assert_close(do.numpy(), orc.swiglu(a, b), 1e-6)
        rf.softmax(ctx, da, n)
        assert_close(da.numpy(), orc.softmax(a), 1e-5)
        for x in (da, db, do):
            x.free()


def test_argmax_rules(ctx, orc):
    rf = _rf()
    rng = np.random.default_rng(803)
    big = rng.normal(0, 1, 128256).astype(np.float32)
    big[[5000, 90000]] = 10.0
    cases = [[1.0, 3.0, 3.0, 2.0], [float("nan"), 5.0, 6.0], [1.0, float("nan"), 6.0, 6.0], [float("-inf")] * 4,
             big, rng.normal(0, 1, 32000).astype(np.float32)]
    out = ctx.empty((1,), np.uint32)
    for c in cases:
        x = ctx.array(np.asarray(c, np.float32))
        rf.argmax(ctx, x, len(c), out)
        assert int(out.numpy()[0]) == orc.argmax(c)
        x.free()


@pytest.mark.parametrize("t", QUANT_TYPES + [F32])
def test_synth_matches_host_generator(ctx, orc, t):
    rf = _rf()
    bs = GEOM[t][1]
    for first, n, mul in ((0, 1000, 0.02 / 127), (123456, 777, 0.02)):
        d = ctx.empty((n * bs,), np.uint8)
        ctx.synth_blocks(t, 99 + t, first, n, mul, d)
        assert np.array_equal(d.numpy(), orc.synth_blocks(t, 99 + t, first, n, mul)), NAMES[t]
        d.free()


# --------------------------------------------------------------- ledger

def test_vram_ledger_semantics(ctx):
    rf = _rf()
    with rf.Context(0, vram_budget_bytes=1 << 20) as c:
        base = c.vram_used
        a = c.alloc(1000, "layer:0:attn_q.weight")
        assert c.charge("layer:0:attn_q.weight") == 1000 and c.vram_used == base + 1000
        with pytest.raises(rf.RamforgeError, match="already exists"):
            c.alloc(10, "layer:0:attn_q.weight")
        with pytest.raises(rf.RamforgeError, match="insufficient memory"):
            c.alloc(1 << 20, "layer:1:ffn_up.weight")
        assert c.vram_used == base + 1000  # the refused charge was rolled back
        c.rename_prefix("layer:0:", "cache:layer:0:")
        assert c.charge("cache:layer:0:attn_q.weight") == 1000 and c.charge("layer:0:attn_q.weight") is None
        a.charge = "cache:layer:0:attn_q.weight"
        a.free()
        assert c.vram_used == base and c.vram_peak >= base + 1000
        with pytest.raises(rf.RamforgeError, match="not found"):
            rf._lib.check(c.lib.rf_vram_release(c.handle, b"layer:9:nothing"))


def test_vram_rename_prefix_touches_only_its_prefix(ctx):
    """Renames act on exactly the charges that start with the prefix
    ("layer:1:" is not a prefix of "layer:10:"), refuse a rename onto an
    existing charge without changing anything, and keep each buffer freeable
    under its new name."""
    rf = _rf()
    with rf.Context(0, vram_budget_bytes=1 << 24) as c:
        base = c.vram_used
        names = ["layer:1:a", "layer:1:b", "layer:10:a", "layer:2:a", "cache:layer:3:a"]
        arrs = {n: c.alloc(100 + i, n) for i, n in enumerate(names)}
        c.rename_prefix("layer:1:", "cache:layer:1:")
        assert c.charge("cache:layer:1:a") == 100 and c.charge("cache:layer:1:b") == 101
        assert c.charge("layer:10:a") == 102 and c.charge("layer:1:a") is None
        with pytest.raises(rf.RamforgeError, match="already exists"):
            c.rename_prefix("cache:layer:3:", "cache:layer:1:")
        assert c.charge("cache:layer:3:a") == 104 and c.charge("cache:layer:1:a") == 100
        with pytest.raises(rf.RamforgeError, match="not found"):
            c.rename_prefix("layer:7:", "x:")
        c.rename_prefix("cache:layer:1:", "layer:5:")
        arrs["layer:1:a"].charge, arrs["layer:1:b"].charge = "layer:5:a", "layer:5:b"
        for a in arrs.values():
            a.free()
        assert c.vram_used == base
