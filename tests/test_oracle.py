"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

Each check is one of: a known-answer test of the reference's own test suite (cited), a golden
fixture written by the reference's own kernel code (tests/golden/, see make_vectors.py), or an
independent mathematical fact (brute-force nearest-value rounding, Sylvester Hadamard matrices,
Lloyd-Max optimality conditions by numerical integration, float64 attention).
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.golden import ref_harness as H
from tests.helpers import PUBLISHED_ERRORS, accuracy_inputs, gqa_attention_f64, relative_rms

GOLD = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


def gold(name):
    return np.load(f"{GOLD}/{name}.npz")


# ---------------------------------------------------------------------------------------------
# E4M3 (OCP FN)
# ---------------------------------------------------------------------------------------------
def e4m3_value_table():
    """Closed form of OCP E4M3FN: (-1)^s 2^(e-7)(1 + m/8), subnormals m 2^-9, S.1111.111 NaN."""
    vals = np.zeros(256, dtype=np.float64)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
            continue
        v = m * 2.0 ** -9 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8)
        vals[c] = -v if s else v
    return vals


def test_e4m3_decode_all_codes_closed_form():
    table = e4m3_value_table()
    for c in range(256):
        got = O.e4m3_to_f32(c)
        if np.isnan(table[c]):
            assert math.isnan(got)
        else:
            assert got == table[c], hex(c)
            assert math.copysign(1, got) == (-1 if c & 0x80 else 1)


def test_e4m3_reference_known_answers():
    # candle-core/src/accel/formats.rs:413-432
    for c in range(256):
        v = O.e4m3_to_f32(c)
        if math.isnan(v):
            continue
        back = O.f32_to_e4m3(v)
        if v == 0.0:
            assert back & 0x7F == 0
        else:
            assert back == c
    assert O.e4m3_to_f32(0x7E) == 448.0
    assert O.f32_to_e4m3(1000.0) == 0x7E
    assert O.f32_to_e4m3(-1000.0) == 0xFE
    assert O.e4m3_to_f32(0x01) == 0.001953125
    # candle-nn/tests/accel_rocm.rs:483-507
    known = [(0x00, 0.0), (0x80, -0.0), (0x01, 0.001953125), (0x81, -0.001953125),
             (0x07, 0.013671875), (0x08, 0.015625), (0x38, 1.0), (0xB8, -1.0), (0x40, 2.0),
             (0x78, 256.0), (0x7D, 416.0), (0x7E, 448.0), (0xFE, -448.0), (0x77, 240.0)]
    for c, v in known:
        got = O.e4m3_to_f32(c)
        assert got == v and math.copysign(1, got) == math.copysign(1, v), hex(c)
    assert math.isnan(O.e4m3_to_f32(0x7F)) and math.isnan(O.e4m3_to_f32(0xFF))


def brute_e4m3(x: np.ndarray) -> np.ndarray:
    """Nearest E4M3FN value, ties to the even code, saturation to +-448, NaN -> 0x7f|s."""
    pos = e4m3_value_table()[:0x7F]  # codes 0..0x7e ascending
    with np.errstate(invalid="ignore"):
        a = np.abs(x.astype(np.float64))
    s = (np.signbit(x).astype(np.uint8)) << 7
    i = np.clip(np.searchsorted(pos, a), 1, 0x7E)
    lo, hi = i - 1, i
    dl, dh = a - pos[lo], pos[hi] - a
    pick = np.where(dl < dh, lo, np.where(dh < dl, hi, np.where(lo % 2 == 0, lo, hi)))
    pick = np.where(a >= pos[0x7E], 0x7E, pick)
    out = (pick.astype(np.uint8) | s)
    return np.where(np.isnan(x), 0x7F | s, out).astype(np.uint8)


def test_e4m3_encode_matches_brute_force():
    # every f32 with the low 11 mantissa bits clear (2^21 patterns incl. both signs, inf, NaN)
    bits = (np.arange(1 << 21, dtype=np.uint64) << 11).astype(np.uint32)
    x = bits.view(np.float32)
    np.testing.assert_array_equal(O.e4m3_encode(x), brute_e4m3(x))
    # every midpoint between adjacent codes and its two f32 neighbours
    pos = e4m3_value_table()[:0x7F].astype(np.float32)
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, 1000), pos])
    near = np.concatenate([near, -near])
    np.testing.assert_array_equal(O.e4m3_encode(near), brute_e4m3(near))


def test_e4m3_encode_matches_torch_below_saturation():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-448, 448, 200000), rng.normal(0, 0.01, 200000)]).astype(np.float32)
    t = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = O.e4m3_encode(x)
    # torch keeps -0 for tiny negatives like the reference
    np.testing.assert_array_equal(ours, t)


# ---------------------------------------------------------------------------------------------
# E2M1, E8M0
# ---------------------------------------------------------------------------------------------
FP4 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_fp4_reference_known_answers():
    # candle-core/src/accel/formats.rs:446-458
    for c, v in enumerate(FP4):
        assert O.fp4_to_f32(c) == v
        assert O.fp4_to_f32(c | 8) == -v
        assert O.f32_to_fp4(v) == c
    assert O.f32_to_fp4(0.75) == 2
    assert O.f32_to_fp4(2.5) == 4
    assert O.f32_to_fp4(5.0) == 6
    assert O.f32_to_fp4(100.0) == 7


def test_fp4_encode_matches_brute_force():
    vals = np.array(FP4)
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-8, 8, 100000), (vals[:-1] + vals[1:]) / 2, vals,
                        -(vals[:-1] + vals[1:]) / 2]).astype(np.float32)
    x = np.concatenate([x, np.nextafter(x, 10), np.nextafter(x, -10)]).astype(np.float32)
    a = np.abs(x.astype(np.float64))
    i = np.clip(np.searchsorted(vals, a), 1, 7)
    lo, hi = i - 1, i
    dl, dh = a - vals[lo], vals[hi] - a
    pick = np.where(dl < dh, lo, np.where(dh < dl, hi, np.where(lo % 2 == 0, lo, hi)))
    pick = np.where(a >= 6.0, 7, pick)
    want = (pick | (np.signbit(x) * 8)).astype(np.uint8)
    np.testing.assert_array_equal(O.fp4_encode(x), want)


def test_mx_scale_known_answers():
    # candle-core/src/accel/formats.rs:460-465
    assert O.mx_scale_code(6.0, 2) == 127
    assert O.e8m0_to_f32(O.mx_scale_code(12.0, 2)) == 2.0
    assert O.mx_scale_code(0.0, 2) == 0
    # the OCP rule: scale = 2^(floor(log2 amax) - emax)
    for amax in [1e-3, 0.3, 1.0, 5.9, 6.0, 7.99, 1e6]:
        assert O.e8m0_to_f32(O.mx_scale_code(amax, 2)) == 2.0 ** (math.floor(math.log2(amax)) - 2)
    assert O.mx_scale_code(float("inf"), 2) == 0 and O.mx_scale_code(float("nan"), 2) == 0
    assert O.e8m0_to_f32(0) == 2.0 ** -127


# ---------------------------------------------------------------------------------------------
# layouts, bit streams
# ---------------------------------------------------------------------------------------------
def test_row_layouts():
    # candle-core/src/accel/formats.rs:467-477
    l = O.row_layout(O.TURBO_MSE, 3, 128)
    assert (l.code_words, l.aux_words, l.row_words) == (12, 0, 14)
    l = O.row_layout(O.TURBO_PROD, 4, 128)
    assert (l.code_words, l.aux_words, l.row_words) == (12, 4, 18)
    l = O.row_layout(O.MXFP4, 0, 64)
    assert (l.code_words, l.aux_words) == (8, 1)
    l = O.row_layout(O.NVFP4, 0, 128)
    assert (l.code_words, l.aux_words) == (16, 2)
    with pytest.raises(ValueError):
        O.row_layout(O.MXFP8, 0, 48)
    # the BASELINE formats at head_dim 128
    assert O.row_layout(O.FP8, 0, 128).row_words == 34
    assert O.row_layout(O.MXFP4, 0, 128).row_words == 19
    assert O.row_layout(O.TURBO_MSE, 4, 128).row_words == 18


def test_bit_stream():
    # candle-core/src/accel/formats.rs:496-504
    import ctypes
    w = (ctypes.c_uint32 * 4)()
    for j in range(40):
        O.lib().orc_put_bits(w, j * 3, 3, j % 8)
    O.lib().orc_get_bits.restype = ctypes.c_uint32
    for j in range(40):
        assert O.lib().orc_get_bits(w, ctypes.c_size_t(j * 3), 3) == j % 8


# ---------------------------------------------------------------------------------------------
# SplitMix64, rotations, codebooks
# ---------------------------------------------------------------------------------------------
def test_splitmix64_published_vector():
    # the published SplitMix64 output for seed 0 (Steele, Lea, Flood 2014; used by xoshiro seeding)
    assert O.splitmix_u64(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_box_muller_moments():
    x = O.normal(7, (400000,)).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.var() - 1) < 0.01
    assert abs((x ** 4).mean() - 3) < 0.05


def test_hadamard_rotation_structure():
    import scipy.linalg
    for d, seed in [(64, 7), (128, 42), (128, 44)]:
        m = O.rotation_matrix(d, O.ROT_HADAMARD, seed).astype(np.float64)
        signs = np.array([1.0 if (u & 1) == 0 else -1.0
                          for u in O.splitmix_u64(seed ^ 0x484144414D415244, d)])
        h = scipy.linalg.hadamard(d)
        np.testing.assert_allclose(m * math.sqrt(d), h * signs[None, :], rtol=1e-6)
        np.testing.assert_allclose(m @ m.T, np.eye(d), atol=1e-5)


def test_rotations_orthogonal():
    # candle-core/src/accel/turbo.rs:599-615
    for d, kind in [(64, O.ROT_HADAMARD), (48, O.ROT_DENSE), (16, O.ROT_NONE)]:
        m = O.rotation_matrix(d, kind, 7).astype(np.float64)
        np.testing.assert_allclose(m @ m.T, np.eye(d), atol=1e-4)


def seeded_gaussian_f64(seed: int, d: int) -> np.ndarray:
    """The d x d f64 normals of SplitMix64(seed) - Box-Muller from two uniforms
    ((u >> 11) + 0.5) / 2^53 per draw (turbo.rs:150-176) - computed here in numpy from the raw
    u64 stream."""
    u = np.array(O.splitmix_u64(seed, 2 * d * d), dtype=np.uint64)
    f = ((u >> np.uint64(11)).astype(np.float64) + 0.5) / float(1 << 53)
    u1, u2 = f[0::2], f[1::2]
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).reshape(d, d)


def gram_schmidt_by_qr(g: np.ndarray) -> np.ndarray:
    """The rows of g orthonormalised in order, from LAPACK's Householder QR of g^T: row i of the
    result spans rows 0..i of g and has a positive component along row i (the sign fixed by
    diag(R) > 0), which is what Gram-Schmidt of the rows in order computes."""
    qm, r = np.linalg.qr(g.T)
    return (qm * np.sign(np.diag(r))[None, :]).T


@pytest.mark.parametrize("d,seed", [(96, 42), (80, 44), (48, 7), (24, 0)])
def test_dense_rotation_is_gram_schmidt_of_seeded_normals(d, seed):
    """rotation_matrix(d, Dense, seed) (candle-core/src/accel/turbo.rs:204-230): the normals of
    SplitMix64(seed ^ "ROTATE!!") orthonormalised row by row. Pinned against an independent route
    (numpy's Box-Muller of the u64 stream, LAPACK QR) to within the f32 rounding of the entries;
    the transposed matrix, the unseeded stream or a lost row order each fail it."""
    m = O.rotation_matrix(d, O.ROT_DENSE, seed).astype(np.float64)
    want = gram_schmidt_by_qr(seeded_gaussian_f64(seed ^ 0x524F544154452121, d))
    np.testing.assert_allclose(m, want, rtol=0, atol=1e-6)
    assert np.abs(m.T - want).max() > 1e-2  # not symmetric: the orientation is pinned
    other = gram_schmidt_by_qr(seeded_gaussian_f64(seed, d))
    assert np.abs(m - other).max() > 1e-2
    flipped = gram_schmidt_by_qr(seeded_gaussian_f64(seed ^ 0x524F544154452121, d)[::-1])
    assert np.abs(m - flipped).max() > 1e-2


def test_rotation_resolve_known_answers(cq):
    """RotationKind::resolve (candle-core/src/accel/config.rs:131-138) and its test
    (config.rs:535-536): Auto.resolve(128) == Hadamard, Auto.resolve(96) == Dense; Hadamard at a
    head dim that is not a power of two is Dense. cqkv's DEFAULT is Auto for the TurboQuant
    formats and None for the others."""
    R = cq.resolve_rotation
    assert R(cq.TURBO4, cq.ROT_AUTO, 128) == cq.ROT_HADAMARD
    assert R(cq.TURBO4, cq.ROT_AUTO, 96) == cq.ROT_DENSE
    assert R(cq.FP8, cq.ROT_AUTO, 96) == cq.ROT_DENSE
    assert R(cq.FP8, cq.ROT_HADAMARD, 80) == cq.ROT_DENSE
    assert R(cq.FP8, cq.ROT_HADAMARD, 64) == cq.ROT_HADAMARD
    assert R(cq.TURBO4, cq.ROT_DEFAULT, 96) == cq.ROT_DENSE
    assert R(cq.TURBOPROD, cq.ROT_DEFAULT, 256) == cq.ROT_HADAMARD
    assert R(cq.FP8, cq.ROT_DEFAULT, 96) == cq.ROT_NONE
    assert R(cq.MXFP4, cq.ROT_DENSE, 128) == cq.ROT_DENSE
    assert R(cq.TURBO4, cq.ROT_NONE, 128) == cq.ROT_NONE
    with pytest.raises(cq.CqkvError):
        R(cq.FP8, 9, 128)


@pytest.mark.parametrize("d,kind,seed", [(96, 3, 42), (80, 3, 44), (256, 2, 42), (128, 2, 44),
                                         (64, 1, 0), (48, 4, 7)])
def test_library_rotation_matrix_equals_oracle(cq, d, kind, seed):
    """cqkv_rotation_matrix (the matrix a caller uploads as cqkv_side.rot) is the oracle's
    rotation_matrix bit for bit (cqkv kinds: 1 none, 2 Hadamard, 3 dense, 4 auto)."""
    okind = {1: O.ROT_NONE, 2: O.ROT_HADAMARD, 3: O.ROT_DENSE,
             4: O.ROT_HADAMARD if d & (d - 1) == 0 else O.ROT_DENSE}[kind]
    got = cq.rotation_matrix(d, kind, seed).numpy()
    np.testing.assert_array_equal(got, O.rotation_matrix(d, okind, seed))


def test_codebook_reference_bounds():
    # candle-core/src/accel/turbo.rs:584-597
    d = 128
    s = math.sqrt(d)
    c, _ = O.lloyd_max(d, 2)
    assert abs(c[2] * s - 0.4528) < 0.01 and abs(c[3] * s - 1.5104) < 0.02
    assert abs(c[0] + c[3]) < 1e-6
    c1, _ = O.lloyd_max(d, 1)
    assert abs(c1[1] * s - 0.7979) < 0.01


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_lloyd_max_conditions(bits):
    """Centroids are the conditional means of their cells under the density (1 - x^2)^((d-3)/2)
    on [-1, 1] (integrated independently with scipy), boundaries are the midpoints."""
    from scipy import integrate
    d = 128
    c, b = O.lloyd_max(d, bits)
    c = c.astype(np.float64)
    b64 = b.astype(np.float64)
    np.testing.assert_allclose(b64, (c[:-1] + c[1:]) / 2, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(c, -c[::-1], atol=0)
    expo = (d - 3) / 2
    f = lambda x: (1 - x * x) ** expo
    edges = np.concatenate([[-1.0], (c[:-1] + c[1:]) / 2, [1.0]])
    for i in range(len(c)):
        mass = integrate.quad(f, edges[i], edges[i + 1], epsabs=1e-14, limit=200)[0]
        mom = integrate.quad(lambda x: x * f(x), edges[i], edges[i + 1], epsabs=1e-14, limit=200)[0]
        # the reference integrates on a 2^16-point grid: cell boundaries snap to grid points,
        # which moves a centroid by up to ~one grid step h = 2 / 2^16; a wrong density
        # exponent or a dropped term moves them by ~1e-3
        assert abs(mom / mass - c[i]) < 2.0 / 65536, (i, mom / mass, c[i])


def test_codebook_close_to_gaussian_lloyd_max():
    # 16-level Lloyd-Max quantizer of N(0, 1) (Max 1960): for d = 128 the coordinates are close
    # to N(0, 1/d) with slightly lighter tails
    gauss = np.array([0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326])
    c, _ = O.lloyd_max(128, 4)
    np.testing.assert_allclose(c[8:] * math.sqrt(128), gauss, rtol=0.03)


# ---------------------------------------------------------------------------------------------
# row codecs against the reference's own kernel (golden fixtures)
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["fp8_d128", "fp8_d80", "mxfp4_d128", "mxfp4_d64", "nvfp4_d128",
                                  "nvfp4_d64", "mxfp8_d128", "mxfp8_d64"])
def test_quantize_rows_bit_exact_with_reference_kernel(name):
    g = gold(f"ref_quant_{name}")
    mode, bits = int(g["mode"]), int(g["bits"])
    got = O.quantize_rows(mode, bits, g["x"])
    np.testing.assert_array_equal(got, g["rows"])


def turbo_codes(rows: np.ndarray, bits: int, d: int) -> np.ndarray:
    """The b-bit codes of packed reference rows (LSB first across words)."""
    out = np.zeros(rows.shape[:-1] + (d,), dtype=np.int64)
    for j in range(d):
        for bit in range(bits):
            pos = bits * j + bit
            out[..., j] |= ((rows[..., pos // 32] >> (pos % 32)) & 1).astype(np.int64) << bit
    return out


@pytest.mark.parametrize("name,bits,d", [("turbo4_d128", 4, 128), ("turbo3_d128", 3, 128),
                                         ("turbo2_d64", 2, 64), ("turbo1_d64", 1, 64)])
def test_turbo_quantize_rows_vs_reference_kernel(name, bits, d):
    # the reference kernel sums the norm in a tree: codes may flip at a boundary (<= 0.1 %) and
    # the norm differs in the last bits (candle-core/tests/accel_kernels_host.rs:1000-1027);
    # TurboMse{1..4} (row layouts of formats.rs:224-242, b-bit codes packed LSB first)
    g = gold(f"ref_quant_{name}")
    got = O.quantize_rows(O.TURBO_MSE, bits, g["x"])
    want = g["rows"]
    l = O.row_layout(O.TURBO_MSE, bits, d)
    assert got.shape == want.shape == (want.shape[0], l.row_words)
    gn = got[:, l.code_words].view(np.float32)
    wn = want[:, l.code_words].view(np.float32)
    np.testing.assert_allclose(gn, wn, rtol=1e-5, atol=1e-6)
    gc, wc = turbo_codes(got, bits, d), turbo_codes(want, bits, d)
    assert (gc != wc).sum() <= max(1, got.shape[0] * d // 1000)
    assert (np.abs(gc - wc) <= 1).all()


@pytest.mark.parametrize("bits,d", [(3, 128), (2, 64)])
def test_prod_width_rows_match_reference_kernels(bits, d):
    """TurboProd{3} / {2} rows ((bits - 1)-bit codes, QJL signs, |r|) against the reference's
    pipeline (tq_quant, tq_resid, S r, tq_signs): codes equal, norms and |r| to 1e-5, signs but
    for <= 0.1 %."""
    g = gold("ref_prod_widths")
    y, want = g[f"x{bits}"], g[f"rows{bits}"]
    mine = O.quantize_rows_qjl(bits, y, O.qjl_matrix(d, 42))
    l = O.row_layout(O.TURBO_PROD, bits, d)
    cw, aw = l.code_words, l.aux_words
    np.testing.assert_array_equal(turbo_codes(mine, bits - 1, d), turbo_codes(want, bits - 1, d))
    for w in (cw + aw, cw + aw + 1):
        np.testing.assert_allclose(mine[..., w].view(np.float32), want[..., w].view(np.float32),
                                   rtol=1e-5)
    ms = np.unpackbits(mine[..., cw:cw + aw].copy().view(np.uint8))
    rs = np.unpackbits(want[..., cw:cw + aw].copy().view(np.uint8))
    assert (ms != rs).sum() <= max(1, ms.size // 1000)


@pytest.mark.parametrize("d", [128, 64])
def test_prod5_rows_match_reference_kernels(d):
    """TurboProd{5} rows (4-bit MSE codes, QJL signs, |r|) against the reference's pipeline:
    codes equal, norms and |r| to 1e-5, signs but for <= 0.1 %."""
    g = gold("ref_prod5")
    y, want = g[f"x_d{d}"], g[f"rows_d{d}"]
    mine = O.quantize_rows_qjl(5, y, O.qjl_matrix(d, 42))
    l = O.row_layout(O.TURBO_PROD, 5, d)
    cw, aw = l.code_words, l.aux_words
    assert l.code_bits == 4
    np.testing.assert_array_equal(turbo_codes(mine, 4, d), turbo_codes(want, 4, d))
    for w in (cw + aw, cw + aw + 1):
        np.testing.assert_allclose(mine[..., w].view(np.float32), want[..., w].view(np.float32),
                                   rtol=1e-5)
    ms = np.unpackbits(mine[..., cw:cw + aw].copy().view(np.uint8))
    rs = np.unpackbits(want[..., cw:cw + aw].copy().view(np.uint8))
    assert (ms != rs).sum() <= max(1, ms.size // 1000)


@pytest.mark.parametrize("vbits", [4, 3])
def test_prod5_decode_vs_reference_fused_kernel(vbits):
    """The reference's fused decode over TurboProd{5} keys and TurboMse{vbits} values equals
    float64 attention over the oracle's dequantized rows to 1e-5; the reference CPU path stays
    within 2e-2."""
    g = gold("ref_prod5")
    kd, vd, want = g["kd"], g[f"vd_mse{vbits}"], g[f"out_mse{vbits}"]
    q, _, _ = widths_inputs()
    B, Hq, Lq, D = q.shape
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42).astype(np.float64)
    pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44).astype(np.float64)
    s = O.qjl_matrix(D, 42)
    kx = O.dequantize_rows_qjl(5, D, kd, s).astype(np.float64) @ pk
    vx = O.dequantize_rows(O.TURBO_MSE, vbits, D, vd).astype(np.float64) @ pv
    scale = float(g["scale"])
    ex = np.zeros((B, Hq, Lq, D))
    for b in range(B):
        for h in range(Hq):
            sc = q[b, h].astype(np.float64) @ kx[b, h // 4].T * scale
            p = np.exp(sc - sc.max(1, keepdims=True))
            ex[b, h] = p @ vx[b, h // 4] / p.sum(1, keepdims=True)
    assert np.abs(ex - want).max() < 1e-5
    cpu = O.cache_attention(O.f32_to_bf16_bits(q), kd, vd, (O.TURBO_PROD, 5),
                            (O.TURBO_MSE, vbits), pk.astype(np.float32), pv.astype(np.float32),
                            kd.shape[2], scale, threads=8, qjl_k=s)
    assert np.abs(O.round_bf16(cpu) - want).max() < 2e-2


def widths_inputs():
    """The inputs of the ref_decode_widths fixture (tests/golden/make_vectors.py widths_case)."""
    B, Hq, Hkv, D, Lq, Lk = 2, 8, 2, 128, 2, 300
    q = O.round_bf16(O.normal(801, (B, Hq, Lq, D)))
    k = O.round_bf16(O.normal(802, (B, Hkv, Lk, D))).astype(np.float32)
    v = O.round_bf16(O.normal(803, (B, Hkv, Lk, D))).astype(np.float32)
    return q, k, v


WIDTH_DECODES = {"mse4_mse3": (O.TURBO_MSE, 4, 3), "prod3_mse2": (O.TURBO_PROD, 3, 2)}


@pytest.mark.parametrize("name", sorted(WIDTH_DECODES))
def test_width_decode_vs_reference_fused_kernel(name):
    """The reference's fused decode over TurboMse{4} keys + TurboMse{3} values and TurboProd{3}
    keys + TurboMse{2} values (tq_attn with a codebook table per side) equals float64 attention
    over the oracle's dequantized rows to 1e-5; the reference CPU path stays within 2e-2."""
    g = gold("ref_decode_widths")
    kmode, kbits, vbits = WIDTH_DECODES[name]
    kd, vd, want = g[f"kd_{name}"], g[f"vd_{name}"], g[f"out_{name}"]
    q, _, _ = widths_inputs()
    B, Hq, Lq, D = q.shape
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42).astype(np.float64)
    pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44).astype(np.float64)
    s = O.qjl_matrix(D, 42) if kmode == O.TURBO_PROD else None
    if kmode == O.TURBO_PROD:
        kq = O.dequantize_rows_qjl(kbits, D, kd, s)
    else:
        kq = O.dequantize_rows(kmode, kbits, D, kd)
    kx = kq.astype(np.float64) @ pk
    vx = O.dequantize_rows(O.TURBO_MSE, vbits, D, vd).astype(np.float64) @ pv
    scale = float(g["scale"])
    ex = np.zeros((B, Hq, Lq, D))
    for b in range(B):
        for h in range(Hq):
            sc = q[b, h].astype(np.float64) @ kx[b, h // 4].T * scale
            p = np.exp(sc - sc.max(1, keepdims=True))
            ex[b, h] = p @ vx[b, h // 4] / p.sum(1, keepdims=True)
    assert np.abs(ex - want).max() < 1e-5
    cpu = O.cache_attention(O.f32_to_bf16_bits(q), kd, vd, (kmode, kbits), (O.TURBO_MSE, vbits),
                            pk.astype(np.float32), pv.astype(np.float32), kd.shape[2], scale,
                            threads=8, qjl_k=s)
    assert np.abs(O.round_bf16(cpu) - want).max() < 2e-2


def test_fp8_row_properties():
    x = O.normal(5, (64, 128)) * np.float32(3)
    rows = O.quantize_rows(O.FP8, 0, x)
    s = rows[:, 32].view(np.float32)
    np.testing.assert_array_equal(s, (np.abs(x).max(1) / np.float32(448)).astype(np.float32))
    assert (rows[:, 33] == 0).all()
    codes = rows[:, :32].view(np.uint8).reshape(64, 128)
    table = e4m3_value_table()
    dec = table[codes] * s[:, None]
    # the largest element lands on +-448; every element within half an E4M3 step
    amax_pos = np.abs(x).argmax(1)
    assert ((codes[np.arange(64), amax_pos] & 0x7F) == 0x7E).all()
    rel = np.abs(dec - x) / np.maximum(np.abs(x), 2.0 ** -6 * s[:, None])
    assert rel.max() <= 2.0 ** -4 + 1e-6


def test_mxfp4_row_properties():
    x = O.normal(6, (64, 128))
    rows = O.quantize_rows(O.MXFP4, 0, x)
    dq = O.dequantize_rows(O.MXFP4, 0, 128, rows)
    for b in range(4):
        blk = x[:, 32 * b: 32 * b + 32]
        sc = (rows[:, 16] >> (8 * b)) & 0xFF
        amax = np.abs(blk).max(1)
        np.testing.assert_array_equal(sc, np.floor(np.log2(amax)).astype(int) - 2 + 127)
        # the block maximum / scale lies in [4, 8): it encodes to 4 or 6
        top = np.abs(dq[:, 32 * b: 32 * b + 32]).max(1) / 2.0 ** (sc.astype(float) - 127)
        assert np.isin(top, [4.0, 6.0]).all()
    assert (rows[:, 17].view(np.float32) == 1.0).all() and (rows[:, 18] == 0).all()


# ---------------------------------------------------------------------------------------------
# attention, masks, combine
# ---------------------------------------------------------------------------------------------
def test_key_ranges():
    # candle-core/src/accel/attention.rs:741-753
    assert O.key_range(0, 4, 4, -1, 0) == (0, 1)
    assert O.key_range(3, 4, 4, -1, 0) == (0, 4)
    assert O.key_range(0, 1, 10, -1, 0) == (0, 10)
    assert O.key_range(5, 8, 8, 2, 0) == (3, 6)
    assert O.key_range(1, 3, 7, -1, -1) == (0, 7)
    assert O.key_range(0, 4, 2, -1, 0) == (0, 0)


def attention_f64(q, k, v, scale, wl=-1, wr=-1, kv_lens=None, softcap=0.0, alibi=None):
    """Brute-force float64 attention; softcap and per-head ALiBi slopes as fa_logit
    (candle-core/kernels/flash_attn_impl.h:42-47): cap * tanh(s / cap), then - slope * |pos - j|."""
    b, hq, lq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros(q.shape)
    for bi in range(b):
        lk = k.shape[2] if kv_lens is None else int(kv_lens[bi])
        for h in range(hq):
            kk = k[bi, h // g, :lk].astype(np.float64)
            vv = v[bi, h // g, :lk].astype(np.float64)
            for i in range(lq):
                pos = i + lk - lq
                lo = max(pos - wl, 0) if wl >= 0 else 0
                hi = min(pos + wr + 1, lk) if wr >= 0 else lk
                lo = min(lo, lk)
                if lo >= hi:
                    continue
                s = kk[lo:hi] @ q[bi, h, i].astype(np.float64) * scale
                if softcap > 0:
                    s = softcap * np.tanh(s / softcap)
                if alibi is not None:
                    s = s - float(alibi[h]) * np.abs(pos - np.arange(lo, hi))
                p = np.exp(s - s.max())
                out[bi, h, i] = p @ vv[lo:hi] / p.sum()
    return out


@pytest.mark.parametrize("wl,wr", [(-1, -1), (-1, 0), (3, 0), (2, 1)])
def test_attention_unfused_vs_float64(wl, wr):
    q = O.normal(1, (2, 4, 5, 32))
    k = O.normal(2, (2, 2, 9, 32))
    v = O.normal(3, (2, 2, 9, 32))
    got = O.attention_unfused(q, k, v, 0.2, wl=wl, wr=wr)
    np.testing.assert_allclose(got, attention_f64(q, k, v, 0.2, wl, wr), atol=2e-6)


def test_attention_ragged_lengths_vs_float64():
    q = O.normal(11, (3, 4, 1, 16))
    k = O.normal(12, (3, 2, 40, 16))
    v = O.normal(13, (3, 2, 40, 16))
    lens = np.array([40, 1, 17], dtype=np.int32)
    got = O.attention_unfused(q, k, v, 0.25, kv_lens=lens)
    np.testing.assert_allclose(got, attention_f64(q, k, v, 0.25, kv_lens=lens), atol=2e-6)


@pytest.mark.parametrize("wl,wr", [(-1, -1), (-1, 0), (4, 1)])
def test_attention_softcap_alibi_vs_float64(wl, wr):
    q = O.normal(21, (2, 4, 6, 32)) * np.float32(2.0)
    k = O.normal(22, (2, 2, 11, 32))
    v = O.normal(23, (2, 2, 11, 32))
    slopes = np.array([0.0, 0.1, 0.35, 1.5], dtype=np.float32)
    got = O.attention_unfused(q, k, v, 0.4, softcap=3.0, wl=wl, wr=wr, alibi=slopes)
    want = attention_f64(q, k, v, 0.4, wl, wr, softcap=3.0, alibi=slopes)
    np.testing.assert_allclose(got, want, atol=2e-6)
    # a cap far above every score leaves the scores alone; zero slopes add nothing
    big = O.attention_unfused(q, k, v, 0.4, softcap=1e6, wl=wl, wr=wr, alibi=np.zeros(4, np.float32))
    np.testing.assert_allclose(big, O.attention_unfused(q, k, v, 0.4, wl=wl, wr=wr), atol=1e-6)


def oracle_fa_dense(q, k, v, scale, softcap, wl, wr, slopes_bh):
    """The oracle over (B, L, H, D) tensors with per-(batch, head) slopes, one sequence at a
    time (the oracle takes per-head slopes)."""
    out = np.zeros_like(q)
    for bi in range(q.shape[0]):
        qb = q[bi:bi + 1].transpose(0, 2, 1, 3)
        kb = k[bi:bi + 1].transpose(0, 2, 1, 3)
        vb = v[bi:bi + 1].transpose(0, 2, 1, 3)
        al = None if slopes_bh is None else slopes_bh[bi]
        o = O.attention_unfused(qb, kb, vb, scale, softcap=softcap, wl=wl, wr=wr, alibi=al)
        out[bi] = o[0].transpose(1, 0, 2)
    return out


def oracle_fa_varlen(q, k, v, cu_q, cu_k, scale, softcap, wl, wr, slopes):
    """The oracle over packed (total, H, D) sequences, one sequence at a time (the reference's
    own varlen invariant, candle-flash-attn/tests/api.rs:86-140)."""
    out = np.zeros_like(q)
    for bi in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[bi]), int(cu_q[bi + 1]), int(cu_k[bi]), int(cu_k[bi + 1])
        if qe == qs:
            continue
        o = oracle_fa_dense(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke], scale, softcap, wl,
                            wr, None if slopes is None else slopes[None])
        out[qs:qe] = o[0]
    return out


def test_attention_terms_vs_reference_tile_kernel_fixture():
    # soft-capping, per-(batch, head) ALiBi, windows and variable-length batches through the
    # reference's fa_tile_impl (tests/golden/make_vectors.py fa_case)
    g = gold("ref_fa_terms")
    dense = oracle_fa_dense(g["q"], g["k"], g["v"], 0.3, 2.5, 20, 2, g["slopes"])
    np.testing.assert_allclose(dense, g["dense"], atol=2e-5)
    var = oracle_fa_varlen(g["qv"], g["kv"], g["vv"], g["cu_q"], g["cu_k"], 0.25, 4.0, -1, 0,
                           g["slopes"][0])
    np.testing.assert_allclose(var, g["var"], atol=2e-5)


def test_attention_vs_reference_tq_attn_fixture():
    # the reference's tq_attng4_fp8 + tq_combine over FP8 rows vs the oracle's attention over the
    # dequantized rows (tolerance of candle-core/tests/accel_kernels_host.rs:1097-1313)
    g = gold("ref_attn_fp8")
    k = O.dequantize_rows(O.FP8, 0, 64, g["kd"])
    v = O.dequantize_rows(O.FP8, 0, 64, g["vd"])
    got = O.attention_unfused(g["q"], k, v, float(g["scale"]))
    np.testing.assert_allclose(got, g["out"], atol=3e-5, rtol=2e-4)


@pytest.mark.parametrize("name", ["turbo4", "mxfp4", "nvfp4", "mxfp8"])
def test_decode_dequantize_and_rotation_vs_reference_fused_kernel(name):
    """The reference's fused decode (tq_attng4 + tq_combine, then the value unrotation) over rows
    of each block / TurboQuant format with outlier channels, against the oracle's dequantizer,
    rotation matrices and f32 attention over the same rows (the reference's own tolerance for
    tq_attn, candle-core/tests/accel_kernels_host.rs:1097-1313): pins the oracle's per-format
    element decoding, block scales, codebook and (un)rotation to the reference kernel."""
    g = gold(f"ref_decode_{name}")
    mode, bits, d = int(g["mode"]), int(g["bits"]), g["q"].shape[-1]
    k = O.dequantize_rows(mode, bits, d, g["kd"])
    v = O.dequantize_rows(mode, bits, d, g["vd"])
    if mode == O.TURBO_MSE:
        k = O.unrotate_rows(O.rotation_matrix(d, O.ROT_HADAMARD, 42), k.reshape(-1, d)).reshape(k.shape)
        v = O.unrotate_rows(O.rotation_matrix(d, O.ROT_HADAMARD, 44), v.reshape(-1, d)).reshape(v.shape)
    got = O.attention_unfused(g["q"], k, v, float(g["scale"]))
    np.testing.assert_allclose(got, g["out"], atol=3e-5, rtol=2e-4)


def test_reference_cpu_path_deviates_from_its_fused_kernel_on_turbo4_outliers():
    """The reference's CPU path rounds the unrotated, dequantized cache to bf16 (keys_values,
    candle-nn/src/turbo_quant.rs:948-966) and its output to bf16; its fused kernel works on the
    f32 codebook values in the rotated domain. On outlier inputs the two differ by more than the
    2e-2 bar for TurboQuant-4 (and by less for the block formats): the reason the GPU decode is held
    to the fused kernel at 2e-2 / 2e-3 and to the CPU path within the CPU path's own deviation
    plus 2e-2."""
    from tests.helpers import oracle_decode
    import torch
    dev = {}
    for name in ("turbo4", "mxfp4", "nvfp4", "mxfp8"):
        g = gold(f"ref_decode_{name}")
        mode, kd = int(g["mode"]), g["kd"]
        cpu = oracle_decode(mode, torch.from_numpy(g["q"]), kd, g["vd"], kd.shape[2],
                            float(g["scale"]))
        dev[name] = float(np.abs(cpu - g["out"]).max())
    assert dev["turbo4"] > 2e-2
    assert max(dev["mxfp4"], dev["nvfp4"], dev["mxfp8"]) < 2e-2


def test_e4m3_threshold_table_reproduces_the_encoder():
    """The 126 code thresholds that the GPU sweep (test_gpu_e4m3_sweep.py) checks every f32 input
    of [0, 449] against: strictly increasing, the saturation code 126 reached at or below 448,
    and, on 2,000,000 random patterns of the range plus the patterns next to every threshold,
    equal to the oracle encoder (with -x giving 0x80 | code)."""
    from tests.helpers import E4M3_SWEEP_END, e4m3_thresholds
    thr = e4m3_thresholds()
    assert (np.diff(thr.astype(np.int64)) > 0).all()
    assert thr[-1].view(np.float32) <= 448.0
    rng = np.random.default_rng(12)
    u = np.concatenate([rng.integers(0, E4M3_SWEEP_END, 2_000_000),
                        thr.astype(np.int64), thr.astype(np.int64) - 1, [0, E4M3_SWEEP_END - 1]])
    u = u.astype(np.uint32)
    x = u.view(np.float32)
    want = np.searchsorted(thr, u, side="right").astype(np.uint8)
    np.testing.assert_array_equal(O.e4m3_encode(x), want)
    np.testing.assert_array_equal(O.e4m3_encode(-x), want | 0x80)


def test_fp4_threshold_table_reproduces_the_encoder():
    """The 7 E2M1 code thresholds of the GPU sweep: strictly increasing, and equal to the oracle
    encoder on 2,000,000 random non-NaN patterns (infinity included) and next to each threshold."""
    from tests.helpers import fp4_thresholds
    thr = fp4_thresholds()
    assert (np.diff(thr.astype(np.int64)) > 0).all()
    rng = np.random.default_rng(13)
    u = np.concatenate([rng.integers(0, 0x7F800001, 2_000_000), thr.astype(np.int64),
                        thr.astype(np.int64) - 1, [0, 0x7F800000]]).astype(np.uint32)
    x = u.view(np.float32)
    want = np.searchsorted(thr, u, side="right").astype(np.uint8)
    np.testing.assert_array_equal(O.fp4_encode(x), want)
    np.testing.assert_array_equal(O.fp4_encode(-x), want | 8)


def test_combine_bit_exact_with_reference_kernel():
    g = gold("ref_combine")
    np.testing.assert_array_equal(O.combine(g["part_o"], g["part_lse"]), g["o"])


def test_combine_of_key_splits_equals_full_attention():
    q = O.normal(21, (1, 2, 1, 16))
    k = O.normal(22, (1, 2, 60, 16))
    v = O.normal(23, (1, 2, 60, 16))
    full = O.attention_unfused(q, k, v, 0.3)[0, :, 0]
    cuts = [0, 7, 30, 30, 60]
    po, pl = [], []
    for a, b in zip(cuts[:-1], cuts[1:]):
        if a == b:
            po.append(np.zeros((2, 16), np.float32))
            pl.append(np.full(2, -np.inf, np.float32))
            continue
        o = O.attention_unfused(q, k[:, :, a:b], v[:, :, a:b], 0.3)[0, :, 0]
        s = np.einsum("hd,hkd->hk", q[0, :, 0].astype(np.float64), k[0, :, a:b].astype(np.float64)) * 0.3
        m = s.max(1)
        pl.append((m + np.log(np.exp(s - m[:, None]).sum(1))).astype(np.float32))
        po.append(o)
    np.testing.assert_allclose(O.combine(np.stack(po), np.stack(pl)), full, atol=2e-6)


def test_split_rules_known_answers():
    # candle-core/src/accel/attention.rs:799-807, 854-857
    assert O.split_count_grouped(8, 1, 8192, 60) == 64
    assert O.split_count_grouped(8, 1, 1000, 60) == 8
    assert O.split_count_grouped(64, 1, 2048, 16) == 16
    assert O.split_count_grouped(4096, 1, 2048, 16) == 1
    assert O.split_count_grouped(16, 4, 1024, 16) == 16
    assert O.split_count_grouped(16, 4, 8192, 16) == 64
    assert O.split_count_grouped(4096, 4, 2048, 16) == 1
    assert (O.row_group(16, 8), O.row_group(32, 2), O.row_group(12, 4), O.row_group(8, 8)) == (2, 8, 1, 1)


def test_cache_attention_fp8_matches_dequantized_bf16_path():
    """orc_cache_attention = dequantize -> bf16 -> unfused attention (turbo_quant.rs:948-990)."""
    b, hq, hkv, d, lk = 1, 4, 2, 64, 33
    kx = O.normal(31, (b, hkv, lk, d))
    vx = O.normal(32, (b, hkv, lk, d))
    q = O.normal(33, (b, hq, 1, d))
    qb = O.f32_to_bf16_bits(q)
    kr = O.quantize_rows(O.FP8, 0, kx)
    vr = O.quantize_rows(O.FP8, 0, vx)
    got = O.cache_attention(qb, kr, vr, (O.FP8, 0), (O.FP8, 0), None, None, lk, 0.125)
    kd = O.round_bf16(O.dequantize_rows(O.FP8, 0, d, kr))
    vd = O.round_bf16(O.dequantize_rows(O.FP8, 0, d, vr))
    want = attention_f64(O.bf16_bits_to_f32(qb), kd, vd, 0.125)
    np.testing.assert_allclose(got, want, atol=2e-6)


def test_turbo_cache_roundtrip_error_bound():
    # candle-core/src/accel/turbo.rs:621-656: relative mse of TurboMse-4 < 0.012 at d = 128
    d = 128
    x = O.normal(3, (64, d))
    pi = O.rotation_matrix(d, O.ROT_HADAMARD, 11)
    rows = O.quantize_rows(O.TURBO_MSE, 4, O.rotate_rows(pi, x))
    back = O.unrotate_rows(pi, O.dequantize_rows(O.TURBO_MSE, 4, d, rows))
    rel = ((back.astype(np.float64) - x) ** 2).sum() / (x.astype(np.float64) ** 2).sum()
    assert rel < 0.012


@pytest.mark.skipif(not H.available(), reason="reference harness not built (make -C oracle ref)")
@pytest.mark.parametrize("softcap,wl,wr", [(0.0, -1, 0), (1.5, -1, -1), (6.0, 9, 0)])
def test_live_reference_harness_fa_terms(softcap, wl, wr):
    q = O.normal(401, (2, 19, 4, 64)) * np.float32(1.5)
    k = O.normal(402, (2, 27, 1, 64))
    v = O.normal(403, (2, 27, 1, 64))
    slopes = np.array([[0.0, 0.2, 0.5, 1.0], [0.01, 0.02, 0.04, 0.08]], dtype=np.float32)
    want = H.fa(q, k, v, 0.2, softcap=softcap, wl=wl, wr=wr, alibi=slopes, alibi_bs=4)
    np.testing.assert_allclose(oracle_fa_dense(q, k, v, 0.2, softcap, wl, wr, slopes), want, atol=2e-5)


@pytest.mark.skipif(not H.available(), reason="reference harness not built (make -C oracle ref)")
def test_live_reference_harness_fp8_rows():
    x = O.normal(99, (23, 128))
    l = O.row_layout(O.FP8, 0, 128)
    want = H.tq_quant(x, O.FP8, 8, l.code_words, l.aux_words, l.row_words, H.tq_tab())
    np.testing.assert_array_equal(O.quantize_rows(O.FP8, 0, x), want)


# ---------------------------------------------------------------------------------------------
# rotary embeddings
# ---------------------------------------------------------------------------------------------
def rope_tables(rows: int, d: int, base: float = 10000.0):
    """cos / sin (rows, d/2) of the usual rotary angles p * base^(-2i/d), in f32."""
    inv = 1.0 / base ** (np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def test_rope_matches_rope_slow_bit_exact():
    """candle-nn/tests/ops.rs:248-270 (and :199-220 for rope_i): on the CPU the fast rope equals
    rope_slow bit for bit. rope_slow is x * cat(cos, cos) + rotate_half(x) * cat(sin, sin)
    (candle-nn/src/rotary_emb.rs:614-630); rope_i_slow reshapes to (.., d/2, 2)
    (rotary_emb.rs:305-324). Both are restated here with torch in f32, independently of the
    oracle's index arithmetic, and must agree with it exactly (random tables as in the test)."""
    import torch
    g = np.random.default_rng(299792458)
    b, h, t, d = 2, 5, 10, 16
    x = g.random((b, h, t, d), dtype=np.float32)
    cos = g.random((t, d // 2), dtype=np.float32)
    sin = g.random((t, d // 2), dtype=np.float32)
    xt, ct, st = torch.from_numpy(x), torch.from_numpy(cos), torch.from_numpy(sin)
    rot_half = torch.cat([-xt[..., d // 2:], xt[..., :d // 2]], -1)
    slow = xt * torch.cat([ct, ct], -1) + rot_half * torch.cat([st, st], -1)
    np.testing.assert_array_equal(O.rope(x, cos, sin, O.ROPE_HALVES, 0), slow.numpy())
    xr = xt.reshape(b, h, t, d // 2, 2)
    x0, x1 = xr[..., 0], xr[..., 1]
    c3, s3 = ct[:, :, None][..., 0], st[:, :, None][..., 0]
    slow_i = torch.stack([x0 * c3 - x1 * s3, x0 * s3 + x1 * c3], -1).reshape(b, h, t, d)
    np.testing.assert_array_equal(O.rope(x, cos, sin, O.ROPE_INTERLEAVED, 0), slow_i.numpy())
    # the two layouts differ (a swapped layout would pass neither identity above)
    assert not np.array_equal(O.rope(x, cos, sin, O.ROPE_HALVES, 0),
                              O.rope(x, cos, sin, O.ROPE_INTERLEAVED, 0))


@pytest.mark.parametrize("kind", [1, 2])
def test_rope_is_a_rotation_by_position(kind):
    """With real angle tables: each (pair) keeps its norm, rotating by -angle undoes it, and the
    score <rope(q, m), rope(k, n)> depends only on m - n (the defining property); float64 checks
    at f32 tolerance, so a wrong sign, pairing or table row fails them."""
    d, rows = 64, 40
    cos, sin = rope_tables(rows, d)
    g = np.random.default_rng(3)
    q = g.standard_normal((1, 1, 1, d)).astype(np.float32)
    k = g.standard_normal((1, 1, 1, d)).astype(np.float32)
    pairs = (lambda y: np.stack([y[..., :d // 2], y[..., d // 2:]], -1)) if kind == 1 else \
        (lambda y: np.stack([y[..., 0::2], y[..., 1::2]], -1))
    for p in (0, 7, 39):
        y = O.rope(q, cos, sin, kind, p)
        np.testing.assert_allclose(np.linalg.norm(pairs(y), axis=-1),
                                   np.linalg.norm(pairs(q), axis=-1), rtol=1e-6)
        back = O.rope(y, cos, -sin, kind, p)
        np.testing.assert_allclose(back, q, atol=1e-5)
    np.testing.assert_array_equal(O.rope(q, cos, sin, kind, 0), q)  # angle 0
    dots = [float((O.rope(q, cos, sin, kind, m).astype(np.float64) *
                   O.rope(k, cos, sin, kind, m - 5).astype(np.float64)).sum())
            for m in (5, 12, 30, 39)]
    np.testing.assert_allclose(dots, dots[0], rtol=1e-5, atol=1e-5)


def test_round_to_dtypes():
    x = np.array([1.0 + 2.0 ** -9, 1.0 + 3 * 2.0 ** -9, 65519.0, 1e-8], np.float32)
    np.testing.assert_array_equal(O.round_to(x, "bf16")[:3], [1.0, 1.0 + 2.0 ** -7, 65536.0])
    np.testing.assert_array_equal(O.round_to(x, "f16")[:2], [1.0 + 2.0 ** -9, 1.0 + 3 * 2.0 ** -9])
    assert np.isinf(O.round_to(np.float32(65520.0), "f16"))
    np.testing.assert_array_equal(O.round_to(x, "f32"), x)


# ---------------------------------------------------------------------------------------------
# per-tensor FP8 quantization (flash_attn_fp8)
# ---------------------------------------------------------------------------------------------
def test_fp8_tensor_quantize_semantics():
    """flash_attn.rs:882-887 through candle's affine (tensor.rs:3124, cpu_backend/mod.rs:313-315):
    the scale maps the largest magnitude to the E4M3 maximum 448; an all-zero tensor keeps
    scale 1; -0 becomes +0 (the `+ 0` of affine); every code is the nearest E4M3 value of
    x * f32(1 / f64(scale)) (brute force over the 127 positive finite codes)."""
    codes, s = O.fp8_quantize_tensor(np.zeros(10, np.float32))
    assert s == 1.0 and (codes == 0).all()
    g = np.random.default_rng(5)
    x = (g.standard_normal(4096) * 3).astype(np.float32)
    x[7] = -0.0
    x[9] = -x[np.argmax(np.abs(x))] * 1.0  # a second element at the maximum, negative
    codes, s = O.fp8_quantize_tensor(x)
    amax = np.abs(x).max()
    assert s == np.float32(amax / np.float32(448.0))
    assert codes[7] == 0x00
    assert codes[np.argmax(np.abs(x))] & 0x7F == 0x7E and codes[9] & 0x7F == 0x7E
    vals = np.array([e4m3_value_table()[c] for c in range(127)])  # positive finite codes
    mul = np.float32(1.0 / np.float64(s))
    q = (x * mul).astype(np.float64)
    for i in range(0, 4096, 37):
        d = np.abs(vals - abs(q[i]))
        best = np.flatnonzero(d == d.min())
        c = codes[i] & 0x7F
        assert c in best if len(best) == 1 else (c in best and c % 2 == 0), (i, q[i], c)
        if q[i] != 0:
            assert (codes[i] >> 7) == (1 if q[i] < 0 else 0)


def test_fp8_tensor_quantize_reciprocal_choice_only_matters_at_ties():
    """x times f32(1 / f64(scale)) (candle's affine) and the f32 quotient x / scale differ in
    the last f32 bit now and then, but an E4M3 code changes only where that bit crosses a
    rounding tie of the 3-bit mantissa: over 400 000 random elements the codes agree. The oracle
    follows the affine; a slip to the quotient would be immaterial at this bar."""
    g = np.random.default_rng(11)
    diff = quot = 0
    for _ in range(20):
        x = (g.standard_normal(20000) * g.uniform(0.1, 50)).astype(np.float32)
        codes, s = O.fp8_quantize_tensor(x)
        qa = (x * np.float32(1.0 / np.float64(s))).astype(np.float32)
        qb = (x / s).astype(np.float32)
        quot += int((qa != qb).sum())
        diff += int((O.e4m3_encode(qb) != codes).sum())
    assert quot > 0 and diff == 0


# ---------------------------------------------------------------------------------------------
# TurboProd (QJL) keys
# ---------------------------------------------------------------------------------------------
def prod_inputs():
    """The inputs of the ref_prod4 fixture (tests/golden/make_vectors.py prod_case)."""
    B, Hq, Hkv, D, Lq, Lk = 2, 8, 2, 128, 2, 300
    rng = np.random.default_rng(700)
    mask = rng.random((Hkv, D)) < 0.01
    q = O.round_bf16(O.normal(701, (B, Hq, Lq, D)))
    k = O.normal(702, (B, Hkv, Lk, D))
    v = O.normal(703, (B, Hkv, Lk, D))
    k = O.round_bf16(np.where(mask[None, :, None, :], k * 8, k)).astype(np.float32)
    v = O.round_bf16(np.where(mask[None, :, None, :], v * 8, v)).astype(np.float32)
    return q, k, v


def test_prod_rows_match_reference_kernels():
    """RowCodec::quantize_row of TurboProd{4} (3-bit codes, QJL sign bits of S r, rsc1 = |r|;
    turbo.rs:299-323) against the reference's GPU pipeline run on its host emulator (tq_quant,
    the tq_resid residual, the S r projection, tq_signs): codes equal, norms and |r| within
    rtol 1e-5 (their reduction orders differ), sign bits equal but for <= 0.1 % (a projection
    within rounding of zero)."""
    g = gold("ref_prod4")
    q, k, v = prod_inputs()
    D = 128
    s = O.qjl_matrix(D, 42)
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42)
    kx = O.rotate_rows(pk, k.reshape(-1, D)).reshape(k.shape)
    mine, ref = O.quantize_rows_qjl(4, kx, s), g["kd"]
    lay = O.row_layout(O.TURBO_PROD, 4, D)
    cw, aw = lay.code_words, lay.aux_words
    np.testing.assert_array_equal(mine[..., :cw], ref[..., :cw])
    for w in (cw + aw, cw + aw + 1):
        np.testing.assert_allclose(mine[..., w].view(np.float32), ref[..., w].view(np.float32),
                                   rtol=1e-5)
    ms = np.unpackbits(mine[..., cw:cw + aw].copy().view(np.uint8))
    rs = np.unpackbits(ref[..., cw:cw + aw].copy().view(np.uint8))
    assert (ms != rs).sum() <= ms.size // 1000


def test_prod_decode_vs_reference_fused_kernel():
    """The reference's fused decode over TurboProd keys (tq_attn with [q Pi^T, q Pi^T S^T],
    turbo_quant_impl.h:259-279, then the value unrotation) equals float64 attention over the
    oracle's dequantized rows (MSE part + QJL correction, turbo.rs:401-424) to 1e-5; the
    reference CPU path (dequantize, unrotate, bf16, unfused attention) stays within 2e-2."""
    g = gold("ref_prod4")
    q, _, _ = prod_inputs()
    B, Hq, Lq, D = q.shape
    s = O.qjl_matrix(D, 42)
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42).astype(np.float64)
    pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44).astype(np.float64)
    kd = O.dequantize_rows_qjl(4, D, g["kd"], s).astype(np.float64) @ pk
    vd = O.dequantize_rows(O.TURBO_MSE, 4, D, g["vd"]).astype(np.float64) @ pv
    scale = float(g["scale"])
    ex = np.zeros((B, Hq, Lq, D))
    for b in range(B):
        for h in range(Hq):
            sc = q[b, h].astype(np.float64) @ kd[b, h // 4].T * scale
            p = np.exp(sc - sc.max(1, keepdims=True))
            ex[b, h] = p @ vd[b, h // 4] / p.sum(1, keepdims=True)
    assert np.abs(ex - g["out"]).max() < 1e-5
    cpu = O.cache_attention(O.f32_to_bf16_bits(q), g["kd"], g["vd"], (O.TURBO_PROD, 4),
                            (O.TURBO_MSE, 4), pk.astype(np.float32), pv.astype(np.float32),
                            g["kd"].shape[2], scale, threads=8, qjl_k=s)
    assert np.abs(O.round_bf16(cpu) - g["out"]).max() < 2e-2


@pytest.mark.parametrize("qjl", [True, False])
def test_prod_inner_products_are_unbiased(qjl):
    """The reference's statistical test (turbo.rs:658-700) over 400 seeds of S: the TurboProd{2}
    estimate of x . y is unbiased (within 0.06 |x| |y|). Dropping the QJL correction (a planted
    mistake) leaves the 1-bit MSE estimate, shrunk by 2 / pi: it must fail."""
    d, n = 64, 400
    x = O.normal(5, (2, d))
    # correlated vectors (x . y ~ 0.9 |x| |y|), so the 2 / pi shrink of the planted mistake
    # stands well clear of the tolerance
    y, xx = x[0], (x[0] + 0.5 * x[1]).astype(np.float32)
    exact = float(xx @ y)
    mean = 0.0
    for seed in range(n):
        pi = O.rotation_matrix(d, O.ROT_HADAMARD, seed)
        rx = O.rotate_rows(pi, xx[None])[0]
        ry = O.rotate_rows(pi, y[None])[0]
        s = O.qjl_matrix(d, seed)
        rows = O.quantize_rows_qjl(2, rx[None], s)
        if qjl:
            back = O.dequantize_rows_qjl(2, d, rows, s)[0]
        else:
            back = O.dequantize_rows(O.TURBO_PROD, 2, d, rows)[0]
        mean += float(back @ ry) / n
    scale = float(np.sqrt((xx @ xx) * (y @ y)))
    if qjl:
        assert abs(mean - exact) < 0.06 * scale, (mean, exact)
    else:
        assert abs(mean - exact) > 0.06 * scale and \
            abs(mean - exact * 2 / np.pi) < 0.06 * scale, (mean, exact)


def test_qjl_matrix_is_standard_normal_from_its_seed():
    """S = SplitMix64((seed + 1) ^ "QJL_SKET") normals (turbo.rs:236-239): the stream of O.normal
    at that seed, moments of N(0, 1), distinct seeds give distinct matrices."""
    s = O.qjl_matrix(128, 42)
    np.testing.assert_array_equal(s.ravel(), O.normal((42 + 1) ^ 0x514A4C5F534B4554, (128 * 128,)))
    assert abs(s.mean()) < 0.02 and abs(s.var() - 1) < 0.03
    assert not np.array_equal(s, O.qjl_matrix(128, 43))


# ---------------------------------------------------------------------------------------------
# the reference's published attention-error table
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("kf,vf,want", PUBLISHED_ERRORS)
def test_published_attention_error_table_on_the_oracle(kf, vf, want):
    """The reference's own end-to-end accuracy table, recomputed on the oracle: its encoders,
    codebooks, Hadamard rotation (RotationKind::Auto at d = 128, keys seed s, values s + 2) and
    QJL stage, dequantized and unrotated in f32 (TurboKvCache::keys_values on the CPU) and
    attended in float64 against the exact attention of the f32 inputs. Each mean equals the
    published value to its three decimals; a mistake in a codebook, a rotation seed or the QJL
    correction moves these well past that."""
    d = 128
    errs = []
    for seed in range(6):
        k, v, q = accuracy_inputs(seed, d)

        def deq(fmt, x, s):
            pi = O.rotation_matrix(d, O.ROT_HADAMARD, s)
            y = O.rotate_rows(pi, x.reshape(-1, d))
            if fmt[0] == O.TURBO_PROD:
                sm = O.qjl_matrix(d, s)
                yd = O.dequantize_rows_qjl(fmt[1], d, O.quantize_rows_qjl(fmt[1], y, sm), sm)
            else:
                yd = O.dequantize_rows(fmt[0], fmt[1], d, O.quantize_rows(fmt[0], fmt[1], y))
            return O.unrotate_rows(pi, yd.reshape(-1, d)).reshape(x.shape)

        got = gqa_attention_f64(q, deq(kf, k, seed), deq(vf, v, seed + 2), d ** -0.5)
        errs.append(relative_rms(got, gqa_attention_f64(q, k, v, d ** -0.5)))
    assert abs(np.mean(errs) - want) <= 5e-4, (np.mean(errs), want)
