"""The C-ABI library on the CPU: it loads, exports every entry point include/cqkv.h declares,
its host-only functions agree with the oracle, and argument errors come back as status codes
(no GPU call is made by any of these)."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "cqkv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cqkv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(cq):
    names = declared_symbols()
    assert len(names) >= 14
    lib = ctypes.CDLL(cq.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(cq.EXPORTED) == names


def test_version(cq):
    assert cq.lib().cqkv_version().decode().startswith("cqkv")


def test_plane_sizes(cq):
    L = cq.lib()
    assert L.cqkv_codes_plane_bytes(cq.FP8, 128, 8192) == 8192 * 128
    assert L.cqkv_scales_plane_bytes(cq.FP8, 128, 8192) == 8192 * 4
    assert L.cqkv_codes_plane_bytes(cq.MXFP4, 128, 64) == 64 * 64
    assert L.cqkv_scales_plane_bytes(cq.MXFP4, 128, 64) == 64 * 4
    assert L.cqkv_scales_plane_bytes(cq.MXFP4, 64, 64) == 64 * 2
    assert L.cqkv_codes_plane_bytes(cq.TURBO4, 128, 32) == 32 * 64
    # head dims 1-256 (FA_MAX_HEAD_DIM); planes hold rows of 64, 128 or 256 elements
    assert L.cqkv_codes_plane_bytes(cq.FP8, 96, 32) == 32 * 128
    assert L.cqkv_codes_plane_bytes(cq.FP8, 80, 32) == 32 * 128
    assert L.cqkv_codes_plane_bytes(cq.FP8, 48, 32) == 32 * 64
    assert L.cqkv_codes_plane_bytes(cq.FP8, 256, 32) == 32 * 256
    assert L.cqkv_scales_plane_bytes(cq.MXFP4, 256, 32) == 32 * 8
    assert L.cqkv_scales_plane_bytes(cq.NVFP4, 80, 32) == 32 * 8 + 32 * 4
    assert L.cqkv_codes_plane_bytes(cq.FP8, 257, 32) == 0
    assert L.cqkv_codes_plane_bytes(cq.FP8, 0, 32) == 0
    # block formats need whole blocks (QuantFormat::validate, formats.rs:166-187)
    assert L.cqkv_codes_plane_bytes(cq.MXFP4, 80, 32) == 0
    assert L.cqkv_codes_plane_bytes(cq.MXFP8, 96, 32) == 32 * 128
    assert L.cqkv_codes_plane_bytes(cq.NVFP4, 72, 32) == 0
    assert L.cqkv_codes_plane_bytes(7, 128, 32) == 0
    # MXFP8: byte codes + E8M0 per 32; NVFP4: nibbles + E4M3 per 16, then an f32 per token
    assert L.cqkv_codes_plane_bytes(cq.MXFP8, 128, 64) == 64 * 128
    assert L.cqkv_scales_plane_bytes(cq.MXFP8, 128, 64) == 64 * 4
    assert L.cqkv_codes_plane_bytes(cq.NVFP4, 128, 64) == 64 * 64
    assert L.cqkv_scales_plane_bytes(cq.NVFP4, 128, 64) == 64 * 8 + 64 * 4
    assert L.cqkv_scales_plane_bytes(cq.NVFP4, 64, 64) == 64 * 4 + 64 * 4


def test_reference_row_words_known_answers(cq):
    """candle-core/src/accel/formats.rs:467-477: TurboMse{3} D=128 12 code words + rsc0, rsc1,
    TurboProd{4} D=128 12 + 4 aux + 2, MXFP4 D=64 8 code + 1 aux words, NVFP4 D=128 16 + 2
    (+ rsc0, rsc1); MXFP8 D=128 32 + 1 + 2 by the same rule (formats.rs:224-242). Widths outside
    TurboMse 1-4 / TurboProd 2-4, or a width for another format, give 0."""
    assert cq.reference_row_words(cq.TURBO4, 128, 3) == 12 + 2
    assert cq.reference_row_words(cq.TURBOPROD, 128, 4) == 12 + 4 + 2
    assert cq.reference_row_words(cq.TURBO4, 128, 1) == 4 + 2
    assert cq.reference_row_words(cq.TURBOPROD, 64, 2) == 2 + 2 + 2
    assert cq.reference_row_words(cq.TURBO4, 128, 5) == 0
    assert cq.reference_row_words(cq.TURBOPROD, 128, 1) == 0
    assert cq.reference_row_words(cq.TURBOPROD, 128, 5) == 16 + 4 + 2  # 4-bit MSE codes
    assert cq.reference_row_words(cq.TURBOPROD, 128, 6) == 0
    assert cq.reference_row_words(cq.FP8, 128, 4) == 0
    assert cq.reference_row_words(cq.MXFP4, 64) == 8 + 1 + 2
    assert cq.reference_row_words(cq.NVFP4, 128) == 16 + 2 + 2
    assert cq.reference_row_words(cq.MXFP8, 128) == 32 + 1 + 2
    assert cq.reference_row_words(cq.NVFP4, 64) == 8 + 1 + 2


@pytest.mark.parametrize("fmt,bits", [(5, 0), (2, 0), (0, 4), (3, 0), (4, 0), (0, 1), (0, 2),
                                      (0, 3), (1, 2), (1, 3), (1, 4)])
@pytest.mark.parametrize("d", [64, 128])
def test_reference_row_words_match_oracle_layout(cq, fmt, bits, d):
    # candle-core/src/accel/formats.rs:224-242, restated by the oracle
    cbits = bits if fmt in (0, 1) else 0
    assert cq.reference_row_words(fmt, d, cbits) == O.row_layout(fmt, bits, d).row_words


@pytest.mark.parametrize("d", [64, 128])
def test_turbo_codebook_identical_to_oracle(cq, d):
    c, b = cq.turbo_codebook(d, 4)
    oc, ob = O.lloyd_max(d, 4)
    np.testing.assert_array_equal(c, oc)
    np.testing.assert_array_equal(b, ob)


@pytest.mark.parametrize("d,seed", [(64, 7), (128, 42), (128, 44)])
def test_turbo_signs_match_oracle_rotation(cq, d, seed):
    s = cq.turbo_signs(d, seed)
    m = O.rotation_matrix(d, O.ROT_HADAMARD, seed)
    # row 0 of the Sylvester matrix is all +1: Pi[0][j] = sign_j / sqrt(d)
    np.testing.assert_array_equal(np.sign(m[0]), s)


def test_workspace_and_split_plan(cq):
    assert cq.decode_workspace_bytes(32, 32, 1, 128, 8) >= 8 * 1024 * 129 * 4
    assert cq.decode_workspace_bytes(0, 32, 1, 128, 8) == 0
    s = cq.decode_splits(32, 8, 8192)
    assert 1 <= s <= 256
    assert cq.decode_splits(1, 8, 512) >= 1
    # 4-bit formats run 4-wavefront workgroups: twice the workgroups, so at least as many splits
    for fmt in (cq.MXFP4, cq.TURBO4):
        assert cq.decode_splits(8, 8, 131072, fmt) >= cq.decode_splits(8, 8, 131072, cq.FP8)
    assert cq.decode_splits(64, 8, 32768, cq.MXFP4, ragged=True) >= 8  # pieces of <= 4096 keys


def test_argument_errors_are_status_codes(cq):
    L = cq.lib()
    x = (ctypes.c_int64 * 3)(1, 1, 1)
    assert L.cqkv_quant_append(None, None, 0, x, 1, 1, None, 0, None) == cq.ERR_ARG
    assert b"null cache side" in L.cqkv_last_error()
    side = cq.Side(cq.FP8, 0, 300, 8, 64, 0, 0, 0, 0, 1, 1)
    assert L.cqkv_quant_append(ctypes.byref(side), ctypes.c_void_p(1), 0, x, 1, 1, None, 0,
                               None) == cq.ERR_ARG
    assert b"head_dim 300" in L.cqkv_last_error()
    side = cq.Side(cq.MXFP4, 0, 80, 8, 64, 0, 0, 0, 0, 1, 1)
    assert L.cqkv_quant_append(ctypes.byref(side), ctypes.c_void_p(1), 0, x, 1, 1, None, 0,
                               None) == cq.ERR_ARG
    assert b"head_dim 80" in L.cqkv_last_error()
    # a dense rotation (TurboQuant at a head dim that is not a power of two) needs its matrix
    side = cq.Side(cq.TURBO4, 0, 96, 8, 64, 0, 0, 0, 42, 1, 1)
    assert L.cqkv_quant_append(ctypes.byref(side), ctypes.c_void_p(1), 0, x, 1, 1, None, 0,
                               None) == cq.ERR_ARG
    assert b"rotation matrix" in L.cqkv_last_error()
    side = cq.Side(cq.FP8, 0, 128, 8, 48, 0, 0, 0, 0, 1, 1)
    assert L.cqkv_quant_append(ctypes.byref(side), ctypes.c_void_p(1), 0, x, 1, 1, None, 0,
                               None) == cq.ERR_ARG
    assert b"multiple of 32" in L.cqkv_last_error()
    side = cq.Side(cq.FP8, 0, 128, 8, 64, 0, 0, 0, 0, 1, 1)
    # appending past the capacity is refused before any launch
    assert L.cqkv_quant_append(ctypes.byref(side), ctypes.c_void_p(1), 0, x, 1, 10, None, 60,
                               None) == cq.ERR_ARG
    assert b"exceed the capacity" in L.cqkv_last_error()
    # decode: a key side given twice, more (query, head) columns than 2^24, kv_len past the
    # capacity
    vs = cq.Side(cq.FP8, 1, 128, 8, 64, 0, 0, 0, 0, 1, 1)
    args = lambda k, v, hq, lq, kvlen, cap=0.0, bs=0: L.cqkv_decode_attention(
        ctypes.c_void_p(1), 0, x, ctypes.byref(k), ctypes.byref(v), 1, hq, lq, None, kvlen,
        0.1, -1, -1, cap, ctypes.c_void_p(1) if bs else None, bs, ctypes.c_void_p(1), 0, x, 0,
        None, 0, None)
    assert args(side, side, 8, 1, 10) == cq.ERR_ARG
    assert args(side, vs, 8 * 32, 1 << 20, 10) == cq.ERR_ARG
    assert args(side, vs, 8, 1, 65) == cq.ERR_ARG
    assert b"capacity" in L.cqkv_last_error()
    # score terms: a finite, non-negative soft cap; ALiBi slopes per head or per (batch, head)
    assert args(side, vs, 8, 1, 10, cap=-1.0) == cq.ERR_ARG
    assert b"softcap" in L.cqkv_last_error()
    assert args(side, vs, 8, 1, 10, cap=float("inf")) == cq.ERR_ARG
    assert args(side, vs, 8, 1, 10, bs=3) == cq.ERR_ARG
    assert b"alibi" in L.cqkv_last_error()


def test_flash_attn_ext_argument_errors(cq):
    """Soft-capping, ALiBi and variable-length arguments are checked before any launch."""
    L = cq.lib()
    x = (ctypes.c_int64 * 3)(8192, 256, 128)
    one = ctypes.c_void_p(256)

    def call(softcap=0.0, alibi=None, alibi_bs=0, cu_q=None, cu_k=None, tq=0, tk=0, kc=None,
             vc=None, hq=8, batch=2, dtype=0, kvd=None, d=128, kp=one, ks=x, ql=16):
        kvd = dtype if kvd is None else kvd
        return L.cqkv_flash_attn_ext(one, x, kp, ks, one, x, one, x, dtype, kvd, batch, ql, 16,
                                     hq, 2, d, 0.1, -1, 0, softcap, alibi, alibi_bs, cu_q, cu_k,
                                     tq, tk, kc, vc, 0, None, 0, None)
    # K / V rows must be 16-byte aligned (the kernels' 16-byte row loads) for bf16 / f16, rows of
    # whole 4-element pieces for f32 queries; head dims multiples of 8 up to 256
    assert call(kp=ctypes.c_void_p(258)) == cq.ERR_ARG
    assert b"16-byte aligned" in L.cqkv_last_error()
    assert call(ks=(ctypes.c_int64 * 3)(8192, 260, 128)) == cq.ERR_ARG
    assert call(ks=(ctypes.c_int64 * 3)(8192, 260, 128), ql=64) == cq.ERR_ARG
    assert call(dtype=2, kp=ctypes.c_void_p(260)) == cq.ERR_ARG  # f32 rows: 16-byte pieces
    assert b"aligned" in L.cqkv_last_error()
    assert call(dtype=2, kvd=0, kp=ctypes.c_void_p(252)) == cq.ERR_ARG  # bf16 rows: 8-byte pieces
    assert call(dtype=2, kvd=1, ks=(ctypes.c_int64 * 3)(8192, 258, 128)) == cq.ERR_ARG
    # the reference's dtype pairs only (kv_dtype_supported): no f16 / bf16 mix, no f32 K / V
    # under half queries, no E4M3 here (cqkv_flash_attn_fp8 takes it), no unknown ids
    for dt, kvd in ((0, 1), (1, 0), (0, 2), (1, 2), (2, 3), (3, 3), (-1, -1)):
        assert call(dtype=dt, kvd=kvd) == cq.ERR_ARG, (dt, kvd)
        assert b"dtype" in L.cqkv_last_error()
    assert call(d=100) == cq.ERR_ARG
    assert call(d=264) == cq.ERR_ARG
    assert b"head_dim" in L.cqkv_last_error()
    assert call(softcap=-1.0) == cq.ERR_ARG
    assert b"softcap" in L.cqkv_last_error()
    assert call(softcap=float("nan")) == cq.ERR_ARG
    assert call(alibi=one, alibi_bs=3) == cq.ERR_ARG
    assert b"alibi slopes" in L.cqkv_last_error()
    assert call(cu_q=one) == cq.ERR_ARG
    assert b"cu_seqlens" in L.cqkv_last_error()
    assert call(cu_q=one, cu_k=one, tq=0, tk=5) == cq.ERR_ARG
    assert b"total_q" in L.cqkv_last_error()
    side = cq.Side(cq.FP8, 0, 128, 2, 64, 0, 0, 0, 0, 1, 1)
    vside = cq.Side(cq.FP8, 1, 128, 2, 64, 0, 0, 0, 0, 1, 1)
    assert call(cu_q=one, cu_k=one, tq=5, tk=5, kc=ctypes.byref(side),
                vc=ctypes.byref(vside)) == cq.ERR_ARG
    assert b"dense batches only" in L.cqkv_last_error()
    # the workspace query: the MFMA prefill's V^T copy (bf16, head dim 128, > 16 queries) or the
    # plain kernel's split partials
    vt = L.cqkv_flash_attn_workspace_bytes(0, 2, 4096, 4096, 32, 8, 128, 0)
    assert vt >= 2 * 8 * 128 * 4096 * 2
    assert L.cqkv_flash_attn_workspace_bytes(1, 2, 1, 8192, 32, 8, 128, 0) > 0  # f16 decode splits
    assert L.cqkv_flash_attn_workspace_bytes(0, 2, 4096, 4096, 32, 7, 128, 0) == 0


def test_empty_inputs(cq):
    """No query rows (batch or q_len 0) are an empty output, as the reference's accelerated
    attention returns (candle-core/src/rocm_backend/accel.rs:87, 197, 481): the calls return
    before any launch and take null q / out / K / V; negative sizes stay errors, and the paged
    forms check their blocks first (no keys is still an error there, flash_attn.rs:682)."""
    L = cq.lib()
    x = (ctypes.c_int64 * 3)(8192, 256, 128)
    one = ctypes.c_void_p(256)

    def dense(batch, ql, kvl, q=None, k=None, dtype=0, kvd=None):
        kvd = dtype if kvd is None else kvd
        return L.cqkv_flash_attn_ext(q, x, k, x, k, x, q, x, dtype, kvd, batch, ql, kvl, 8, 2,
                                     128, 0.1, -1, 0, 0.0, None, 0, None, None, 0, 0, None, None,
                                     0, None, 0, None)
    for dt in (0, 1, 2):
        assert dense(0, 16, 16, dtype=dt) == cq.OK
        assert dense(2, 0, 16, dtype=dt, k=one) == cq.OK  # K / V rows (for a cache append)
        assert dense(2, 0, 16, dtype=dt) == cq.ERR_ARG
        assert dense(0, 0, 0, dtype=dt) == cq.OK
    assert dense(-1, 16, 16) == cq.ERR_ARG
    assert dense(2, -1, 16) == cq.ERR_ARG
    assert dense(2, 16, -1) == cq.ERR_ARG
    assert dense(2, 16, 16) == cq.ERR_ARG  # rows to write: q / out must be given
    assert b"null" in L.cqkv_last_error()
    assert dense(2, 0, 16, dtype=0, kvd=1, k=one) == cq.ERR_ARG  # dtype pairs are still checked
    assert L.cqkv_flash_attn_workspace_bytes(0, 2, 0, 16, 8, 2, 128, 0) == 0
    assert L.cqkv_flash_attn_workspace_bytes(0, 2, 16, 0, 8, 2, 128, 0) == 0

    def fp8(batch, ql, kvl, dtype=0):
        return L.cqkv_flash_attn_fp8(None, x, None, x, None, x, None, x, dtype, batch, ql, kvl,
                                     8, 8, 128, 0.1, -1, 0, 1.0, 1.0, None, None, None, 0, None)
    for dt in (0, 1, 2):
        assert fp8(0, 16, 16, dt) == cq.OK
        assert fp8(1, 0, 16, dt) == cq.OK
    assert fp8(1, 16, 0) == cq.ERR_ARG  # zero rows to write need q / out
    assert fp8(1, -1, 16) == cq.ERR_ARG

    k0 = cq.Side(cq.FP8, 0, 128, 8, 64, 0, 0, 0, 0, 1, 1)
    v0 = cq.Side(cq.FP8, 1, 128, 8, 64, 0, 0, 0, 0, 1, 1)
    xs = (ctypes.c_int64 * 3)(1, 1, 1)

    def decode(batch, ql, kvl=10):
        return L.cqkv_decode_attention(None, 0, xs, ctypes.byref(k0), ctypes.byref(v0), batch, 8,
                                       ql, None, kvl, 0.1, -1, -1, 0.0, None, 0, None, 0, xs, 0,
                                       None, 0, None)
    assert decode(0, 1) == cq.OK
    assert decode(1, 0) == cq.OK
    assert decode(1, 0, kvl=65) == cq.ERR_ARG  # kv_len above the capacity
    assert decode(-1, 1) == cq.ERR_ARG
    assert decode(1, 1) == cq.ERR_ARG

    def paged(rows, batch, ql):
        arr = (cq.KvBlock * 1)()
        arr[0].k, arr[0].v, arr[0].rows = ctypes.pointer(k0), ctypes.pointer(v0), rows
        return L.cqkv_decode_attention_paged(None, 0, xs, arr, 1, batch, 8, ql, 0.1, -1, -1, 0.0,
                                             None, 0, None, 0, xs, None, 0, None)
    assert paged(10, 0, 1) == cq.OK
    assert paged(10, 1, 0) == cq.OK
    assert paged(0, 1, 0) == cq.ERR_ARG
    assert b"no keys" in L.cqkv_last_error()

    def plain_blocks(rows, batch, ql):
        arr = (cq.PlainBlock * 1)()
        arr[0].k = arr[0].v = one
        arr[0].rows = rows
        for i, s in enumerate((8192, 128, 128)):
            arr[0].k_strides[i] = arr[0].v_strides[i] = s
        return L.cqkv_flash_attn_blocks(None, x, arr, 1, 0, 0, batch, 8, ql, 2, 128, 0.1, -1, 0,
                                        0.0, None, 0, None, x, None, 0, None)
    assert plain_blocks(10, 0, 16) == cq.OK
    assert plain_blocks(10, 2, 0) == cq.OK
    assert plain_blocks(0, 2, 0) == cq.ERR_ARG
    assert b"no keys" in L.cqkv_last_error()
    assert plain_blocks(10, 2, 16) == cq.ERR_ARG


def test_paged_argument_errors_and_workspace(cq):
    """cqkv_decode_attention_paged validates its blocks like the reference's check_blocks
    (candle-nn/src/flash_attn.rs:650-686) before any launch, and sizes its scratch."""
    L = cq.lib()
    x = (ctypes.c_int64 * 3)(1, 1, 1)
    k0 = cq.Side(cq.FP8, 0, 128, 8, 64, 0, 0, 0, 0, 1, 1)
    v0 = cq.Side(cq.FP8, 1, 128, 8, 64, 0, 0, 0, 0, 1, 1)
    k1 = cq.Side(cq.FP8, 0, 128, 8, 128, 0, 0, 0, 0, 1, 1)
    v1 = cq.Side(cq.FP8, 1, 128, 8, 128, 0, 0, 0, 0, 1, 1)
    kx = cq.Side(cq.MXFP4, 0, 128, 8, 64, 0, 0, 0, 0, 1, 1)

    def blocks(*bl):
        arr = (cq.KvBlock * len(bl))()
        for i, (k, v, r) in enumerate(bl):
            arr[i].k, arr[i].v, arr[i].rows = ctypes.pointer(k), ctypes.pointer(v), r
        return arr

    def call(arr, n, hq=8, lq=1):
        return L.cqkv_decode_attention_paged(ctypes.c_void_p(1), 0, x, arr, n, 1, hq, lq, 0.1,
                                             -1, -1, 0.0, None, 0, ctypes.c_void_p(1), 0, x, None,
                                             0, None)
    assert call(None, 0) == cq.ERR_ARG
    assert b"no blocks" in L.cqkv_last_error()
    assert call(blocks((k0, v0, 65)), 1) == cq.ERR_ARG  # rows above the capacity
    assert b"capacities" in L.cqkv_last_error()
    assert call(blocks((k0, v0, 0), (k1, v1, 0)), 2) == cq.ERR_ARG
    assert b"no keys" in L.cqkv_last_error()
    assert call(blocks((k0, v0, 10), (kx, v1, 10)), 2) == cq.ERR_ARG  # another format
    assert b"differs from block 0" in L.cqkv_last_error()
    assert call(blocks((k0, k0, 10)), 1) == cq.ERR_ARG  # a key side in the value slot
    assert call(blocks((k0, v0, 10)), 1, hq=8 * 32, lq=1 << 20) == cq.ERR_ARG  # 2^25 columns
    # scratch: the block table, the partials of the segments and the rotation buffers
    one = L.cqkv_decode_paged_workspace_bytes(blocks((k0, v0, 10)), 1, 1, 8, 1)
    many = L.cqkv_decode_paged_workspace_bytes(blocks((k1, v1, 128), (k1, v1, 128)), 2, 1, 8, 1)
    assert 0 < one < many
    assert L.cqkv_decode_paged_workspace_bytes(blocks((k0, v0, 65)), 1, 1, 8, 1) == 0


def test_gpu_entry_points_refuse_cpu_tensors(cq):
    torch = pytest.importorskip("torch")
    side = cq.CacheSide(cq.FP8, False, 1, 1, 64, 32, torch.zeros(1, dtype=torch.uint8),
                        torch.zeros(1, dtype=torch.uint8))
    with pytest.raises(cq.CqkvError):
        cq.quant_append(side, torch.zeros(1, 1, 1, 64))


def test_rope_quant_append_argument_errors(cq):
    """The fused RoPE + append checks its sides, kinds and positions before any launch."""
    L = cq.lib()
    x = (ctypes.c_int64 * 3)(1, 128, 128)
    one = ctypes.c_void_p(1)
    k = cq.Side(cq.FP8, 0, 128, 2, 64, 0, 0, 0, 0, 1, 1)
    v = cq.Side(cq.FP8, 1, 128, 2, 64, 0, 0, 0, 0, 1, 1)
    vm = cq.Side(cq.MXFP4, 1, 128, 2, 96, 0, 0, 0, 0, 1, 1)  # another format is fine, capacity not
    vr = cq.Side(cq.FP8, 1, 128, 2, 64, 7, 0, 0, 0, 1, 1)  # no rotation 7

    def call(ks=k, vs=v, kind=1, tokens=4, position=0, rows=100, hq=8, positions=None, cos=one):
        return L.cqkv_rope_quant_append(ctypes.byref(ks), ctypes.byref(vs), one, x, one, x, one,
                                        x, 0, 2, tokens, hq, cos, one, rows, kind, positions,
                                        position, one, x, None)
    assert call(kind=0) == cq.ERR_ARG
    assert b"rope kind" in L.cqkv_last_error()
    assert call(vs=vm) == cq.ERR_ARG
    assert b"capacity" in L.cqkv_last_error()
    assert call(vs=vr) == cq.ERR_ARG
    assert b"rotation" in L.cqkv_last_error()
    assert call(ks=v, vs=k) == cq.ERR_ARG
    assert call(hq=5) == cq.ERR_ARG
    assert call(position=62) == cq.ERR_ARG
    assert b"capacity" in L.cqkv_last_error()
    assert call(position=10, rows=12) == cq.ERR_ARG
    assert b"cos / sin rows" in L.cqkv_last_error()
    assert call(cos=None) == cq.ERR_ARG
    assert call(tokens=0) == cq.OK  # nothing to do, nothing launched
    # more blocks than one launch's 2^32 threads along x (device positions: no capacity check)
    big = ctypes.c_void_p(16)
    assert call(tokens=2_000_000_000, hq=2000, rows=100, positions=big) == cq.ERR_ARG
    assert b"exceed one launch" in L.cqkv_last_error()


def test_fp8_attention_argument_errors(cq):
    L = cq.lib()
    one = ctypes.c_void_p(8)
    x = (ctypes.c_int64 * 3)(8, 1024, 128)
    odd = (ctypes.c_int64 * 3)(8, 1028, 130)

    def attn(ks=x, hd=128, kd=1.0, dtype=0, ws=None, wsb=0):
        return L.cqkv_flash_attn_fp8(one, x, one, ks, one, x, one, x, dtype, 1, 16, 16, 8, 8, hd,
                                     0.1, -1, 0, kd, 1.0, None, None, ws, wsb, None)
    assert attn(hd=260) == cq.ERR_ARG  # head dims: multiples of 8 up to 256
    assert attn(hd=100) == cq.ERR_ARG
    assert attn(dtype=3) == cq.ERR_ARG  # bf16 / f16 / f32 queries
    assert attn(ws=one, wsb=16) == cq.ERR_WORKSPACE  # a workspace below the query's size
    assert L.cqkv_flash_attn_fp8_workspace_bytes(0, 1, 16, 16, 8, 8, 128) > 0
    assert L.cqkv_flash_attn_fp8_workspace_bytes(3, 1, 16, 16, 8, 8, 128) == 0
    # f32 queries read the codes directly: only the attention's own split partials
    f32_ws = L.cqkv_flash_attn_fp8_workspace_bytes(2, 1, 1, 8192, 32, 8, 128)
    assert f32_ws == L.cqkv_flash_attn_workspace_bytes(2, 1, 1, 8192, 32, 8, 128, 0) > 0
    assert f32_ws < L.cqkv_flash_attn_fp8_workspace_bytes(0, 1, 1, 8192, 32, 8, 128)
    assert attn(ks=odd) == cq.ERR_ARG
    assert b"multiples of 8" in L.cqkv_last_error()
    assert attn(kd=float("nan")) == cq.ERR_ARG

    def attn2(kv_len=16, hq=8, hkv=8):
        return L.cqkv_flash_attn_fp8(one, x, one, x, one, x, one, x, 0, 1, 16, kv_len, hq, hkv,
                                     128, 0.1, -1, 0, 1.0, 1.0, None, None, None, 0, None)
    assert attn2(kv_len=(1 << 23) + 1) == cq.ERR_ARG  # before any scratch or launch
    assert attn2(hq=6, hkv=4) == cq.ERR_ARG
    assert L.cqkv_hadamard_rows(one, 0, 1 << 27, 128, 128, 1, one, 128, None) == cq.ERR_ARG
    assert L.cqkv_hadamard_rows(one, 0, 4, 64, 128, 1, one, 128, None) == cq.ERR_ARG
    assert L.cqkv_hadamard_rows(one, 0, 4, 96, 96, 1, one, 96, None) == cq.ERR_ARG
    assert L.cqkv_fp8_quantize_tensor(one, 7, 16, one, one, None) == cq.ERR_ARG
    assert L.cqkv_fp8_quantize_tensor(None, 0, 16, one, one, None) == cq.ERR_ARG
    assert L.cqkv_fp8_quantize_tensor(one, 0, -1, one, one, None) == cq.ERR_ARG


def test_side_copy_argument_errors(cq):
    """Cache growth copies only between sides of one format, kind, shape and rotation, and only
    tokens both capacities hold; nothing is launched for zero tokens."""
    L = cq.lib()
    src = cq.Side(cq.MXFP4, 0, 128, 8, 64, 0, 0, 0, 42, 1, 1)

    def copy(dst, tokens=40, batch=2):
        return L.cqkv_side_copy(ctypes.byref(dst), ctypes.byref(src), batch, tokens, None)
    assert copy(cq.Side(cq.FP8, 0, 128, 8, 128, 0, 0, 0, 42, 1, 1)) == cq.ERR_ARG
    assert b"format" in L.cqkv_last_error()
    assert copy(cq.Side(cq.MXFP4, 1, 128, 8, 128, 0, 0, 0, 42, 1, 1)) == cq.ERR_ARG  # value side
    assert copy(cq.Side(cq.MXFP4, 0, 64, 8, 128, 0, 0, 0, 42, 1, 1)) == cq.ERR_ARG
    assert copy(cq.Side(cq.MXFP4, 0, 128, 4, 128, 0, 0, 0, 42, 1, 1)) == cq.ERR_ARG
    assert copy(cq.Side(cq.MXFP4, 0, 128, 8, 128, cq.ROT_HADAMARD, 0, 0, 42, 1, 1)) == cq.ERR_ARG
    big = cq.Side(cq.MXFP4, 0, 128, 8, 128, 0, 0, 0, 42, 1, 1)
    assert copy(big, tokens=65) == cq.ERR_ARG  # more than the source holds
    assert b"capacities" in L.cqkv_last_error()
    assert copy(cq.Side(cq.MXFP4, 0, 128, 8, 32, 0, 0, 0, 42, 1, 1)) == cq.ERR_ARG  # 40 > 32
    assert copy(big, batch=0) == cq.ERR_ARG
    assert copy(big, tokens=0) == cq.OK
    # an unrotated side ignores the seed; a rotated one needs the same seed
    assert copy(cq.Side(cq.MXFP4, 0, 128, 8, 128, 0, 0, 0, 7, 1, 1), tokens=0) == cq.OK
    rsrc = cq.Side(cq.MXFP4, 0, 128, 8, 64, cq.ROT_HADAMARD, 0, 0, 42, 1, 1)
    rdst = cq.Side(cq.MXFP4, 0, 128, 8, 128, cq.ROT_HADAMARD, 0, 0, 7, 1, 1)
    assert L.cqkv_side_copy(ctypes.byref(rdst), ctypes.byref(rsrc), 2, 0, None) == cq.ERR_ARG
    assert b"seed" in L.cqkv_last_error()


def test_grown_capacity_follows_cache_append(cq):
    """Cache::grown_capacity (candle-nn/src/kv_cache.rs:60-66): cap += max(grow_by, cap / 2, 1)
    until the need fits, rounded up to 32 tokens here."""
    assert cq.grown_capacity(64, 16, 64) == 64
    assert cq.grown_capacity(64, 16, 65) == 96       # 64 + max(16, 32)
    assert cq.grown_capacity(64, 100, 65) == 192     # 64 + 100 = 164 -> 192
    assert cq.grown_capacity(32, 8, 100) == 128      # 32 -> 48 -> 72 -> 108 -> 128
    assert cq.grown_capacity(0, 0, 1) == 32          # max(.., 1) makes progress


def test_flash_attn_blocks_argument_errors(cq):
    """cqkv_flash_attn_blocks checks its blocks like the reference's check_blocks
    (candle-nn/src/flash_attn.rs:650-686) before any launch."""
    L = cq.lib()
    qs = (ctypes.c_int64 * 3)(8 * 4 * 128, 4 * 128, 128)
    one = ctypes.c_void_p(256)

    def blk(rows=10, k=256, kr=128, vr=128):
        b = cq.PlainBlock()
        b.k, b.v, b.rows = k, 256, rows
        b.k_strides[:] = [2 * 64 * kr, 64 * kr, kr]
        b.v_strides[:] = [2 * 64 * vr, 64 * vr, vr]
        return b

    def call(*bl, dtype=0, kvd=None, d=128, softcap=0.0, hq=8):
        arr = (cq.PlainBlock * max(len(bl), 1))(*bl)
        kvd = dtype if kvd is None else kvd
        return L.cqkv_flash_attn_blocks(one, qs, arr, len(bl), dtype, kvd, 1, hq, 1, 2, d, 0.1,
                                        -1, 0, softcap, None, 0, one, qs, None, 0, None)
    assert call() == cq.ERR_ARG
    assert b"no blocks" in L.cqkv_last_error()
    assert call(blk(rows=0), blk(rows=0)) == cq.ERR_ARG
    assert b"no keys" in L.cqkv_last_error()
    assert call(blk(rows=-1)) == cq.ERR_ARG
    assert call(blk(), blk(kr=136)) == cq.ERR_ARG
    assert b"row strides" in L.cqkv_last_error()
    assert call(blk(k=264)) == cq.ERR_ARG
    assert b"aligned" in L.cqkv_last_error()
    assert call(blk(), dtype=0, kvd=1) == cq.ERR_ARG
    assert b"dtype" in L.cqkv_last_error()
    assert call(blk(), dtype=1, kvd=2) == cq.ERR_ARG
    assert call(blk(k=260), dtype=2, kvd=1) == cq.ERR_ARG  # 4-element (8-byte) pieces
    assert b"aligned" in L.cqkv_last_error()
    assert call(blk(), d=300) == cq.ERR_ARG
    assert call(blk(), softcap=-1.0) == cq.ERR_ARG
    assert call(blk(), hq=5) == cq.ERR_ARG
    # workspace: the segment table, plus partials once the keys are split
    arr = (cq.PlainBlock * 1)(blk(rows=10))
    small = L.cqkv_flash_attn_blocks_workspace_bytes(arr, 1, 1, 8, 1, 2, 128)
    arr2 = (cq.PlainBlock * 2)(blk(rows=64), blk(rows=64))
    assert 0 < small < L.cqkv_flash_attn_blocks_workspace_bytes(arr2, 2, 1, 8, 1, 2, 128)


def test_turboprod_sides_and_qjl_matrix(cq):
    """TurboProd key sides: plane sizes (nibble codes; norms, |r|, D / 8 sign bytes per token),
    the reference row of 3-bit codes + D sign bits + 2 (formats.rs:226-240), keys only, a QJL
    matrix required; cqkv_qjl_matrix is the oracle's qjl_matrix bit for bit."""
    L = cq.lib()
    assert L.cqkv_codes_plane_bytes(cq.TURBOPROD, 128, 64) == 64 * 64
    assert L.cqkv_scales_plane_bytes(cq.TURBOPROD, 128, 64) == 64 * (8 + 16)
    assert L.cqkv_reference_row_words(cq.TURBOPROD, 0, 128) == 12 + 4 + 2
    assert L.cqkv_reference_row_words(cq.TURBOPROD, 4, 64) == 6 + 2 + 2
    np.testing.assert_array_equal(cq.qjl_matrix(128, 42).numpy(), O.qjl_matrix(128, 42))
    x = (ctypes.c_int64 * 3)(1, 128, 128)
    one = ctypes.c_void_p(256)
    val = cq.Side(cq.TURBOPROD, 1, 128, 2, 64, 0, 0, 0, 44, 256, 256, 256)
    assert L.cqkv_quant_append(ctypes.byref(val), one, 0, x, 1, 4, None, 0, None) == cq.ERR_ARG
    assert b"key format" in L.cqkv_last_error()
    noqjl = cq.Side(cq.TURBOPROD, 0, 128, 2, 64, 0, 0, 0, 42, 256, 256, None)
    assert L.cqkv_quant_append(ctypes.byref(noqjl), one, 0, x, 1, 4, None, 0, None) == cq.ERR_ARG
    assert b"QJL" in L.cqkv_last_error()
