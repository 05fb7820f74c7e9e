"""Writes the golden fixtures of tests/golden/ from the reference's own kernel code.

Run in a checkout where the reference tree is mounted (it is absent on the GPU box):
    make -C oracle ref && python tests/golden/make_vectors.py
The inputs are SplitMix64 normals (candle-core/src/accel/turbo.rs:150-176, the generator of
the reference's own tests); the outputs come from oracle/_ref/accel_host_test, i.e. the
reference's tq_quant / tq_attn / tq_combine kernels run on its host emulator. The reference's
test candle-core/tests/accel_kernels_host.rs:960-1070 asserts that this tq_quant is bit-exact
with the CPU codec RowCodec::quantize_row for the FP8 / MX formats.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests.golden import ref_harness as H  # noqa: E402


def quant_case(name, mode, bits, d, rows, seed):
    l = O.row_layout(mode, bits, d)
    x = O.normal(seed, (rows, d)) * np.float32(2.0)
    x[0, 3] = 0.0
    x[1, :] = 0.0  # an all-zero row
    x[2, 5] = 40.0  # an outlier
    x[3, :32] = 1e-30  # a subnormal-scale block
    if mode == O.TURBO_MSE:
        c, b = O.lloyd_max(d, bits)
        tab = H.tq_tab(c, b)
    else:
        tab = H.tq_tab()
    got = H.tq_quant(x.astype(np.float32), mode, l.code_bits, l.code_words, l.aux_words,
                     l.row_words, tab)
    np.savez_compressed(os.path.join(HERE, f"ref_quant_{name}.npz"), x=x, rows=got,
                        mode=mode, bits=bits, d=d)
    print(name, got.shape)


def attn_case():
    # GQA pack G = 4 FP8 rows (the decode path of BASELINE config 2 at a small size)
    B, Hq, Hkv, D, Lk = 2, 8, 2, 64, 200
    q = O.normal(101, (B, Hq, 1, D))
    k = O.normal(102, (B, Hkv, Lk, D))
    v = O.normal(103, (B, Hkv, Lk, D))
    kd = O.quantize_rows(O.FP8, 0, k)
    vd = O.quantize_rows(O.FP8, 0, v)
    l = O.row_layout(O.FP8, 0, D)
    side = (O.FP8, 8, l.code_words, l.code_words + l.aux_words)
    tab = np.zeros(64, dtype=np.float32)
    out = H.tq_attn(q, kd, vd, side, side, tab, 0.125, splits=4, group=4, fp8=True)
    np.savez_compressed(os.path.join(HERE, "ref_attn_fp8.npz"), q=q, kd=kd, vd=vd, out=out,
                        scale=0.125)
    print("attn", out.shape)


def attn_format_case(name, mode, bits):
    """The reference's fused decode (tq_attn* + tq_combine on its host emulator) over rows of one
    format, GQA group 4, three splits, outlier channels (1 % of the (head, dim) channels x8),
    then the value unrotation of fused_attention_rows (candle-nn/src/turbo_quant.rs:1263) in f32.
    TurboQuant-4 rows are the reference kernel's encoding of the Hadamard-rotated rows (keys seed
    42, values 44), the query is rotated with the key rotation (turbo_quant.rs:1162)."""
    B, Hq, Hkv, D, Lq, Lk = 2, 8, 2, 128, 2, 333
    rng = np.random.default_rng(400 + mode)
    mask = rng.random((Hkv, D)) < 0.01
    mask[0, 5] = mask[1, 77] = True
    q = O.round_bf16(O.normal(401 + mode, (B, Hq, Lq, D)))
    k = O.normal(402 + mode, (B, Hkv, Lk, D))
    v = O.normal(403 + mode, (B, Hkv, Lk, D))
    k = O.round_bf16(np.where(mask[None, :, None, :], k * 8, k)).astype(np.float32)
    v = O.round_bf16(np.where(mask[None, :, None, :], v * 8, v)).astype(np.float32)
    l = O.row_layout(mode, bits, D)
    turbo = mode == O.TURBO_MSE
    if turbo:
        c, b = O.lloyd_max(D, bits)
        tab = H.tq_tab(c, b)
        pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42)
        pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44)
        kx = O.rotate_rows(pk, k.reshape(-1, D))
        vx = O.rotate_rows(pv, v.reshape(-1, D))
        qx = O.rotate_rows(pk, q.reshape(-1, D)).reshape(q.shape)
    else:
        tab = H.tq_tab()
        kx, vx, qx = k.reshape(-1, D), v.reshape(-1, D), q
    enc = lambda x: H.tq_quant(x.astype(np.float32), mode, l.code_bits, l.code_words,
                               l.aux_words, l.row_words, tab).reshape(B, Hkv, Lk, l.row_words)
    kd, vd = enc(kx), enc(vx)
    side = (mode, l.code_bits, l.code_words, l.code_words + l.aux_words)
    tab64 = np.concatenate([tab, tab]).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(D))
    o = H.tq_attn(qx.astype(np.float32), kd, vd, side, side, tab64, float(scale), splits=3,
                  group=4)
    if turbo:
        o = (o.reshape(-1, D) @ pv).reshape(o.shape).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, f"ref_decode_{name}.npz"), q=q.astype(np.float32),
                        kd=kd, vd=vd, out=o, scale=scale, mode=mode, bits=bits)
    print("decode", name, o.shape)


def fa_case():
    # soft-capping, per-(batch, head) ALiBi slopes and a window through the reference's tile
    # kernel, dense and variable-length (the score terms of candle-flash-attn's *_softcap / *_alibi
    # / *_varlen entry points)
    B, Lq, Lk, Hq, Hkv, D = 2, 37, 53, 4, 2, 32
    q = O.normal(301, (B, Lq, Hq, D))
    k = O.normal(302, (B, Lk, Hkv, D))
    v = O.normal(303, (B, Lk, Hkv, D))
    slopes = (0.05 * (1 + np.arange(B * Hq))).astype(np.float32).reshape(B, Hq)
    dense = H.fa(q, k, v, 0.3, softcap=2.5, wl=20, wr=2, alibi=slopes, alibi_bs=Hq)
    cu_q = np.array([0, 9, 9, 40], dtype=np.uint32)  # an empty second sequence
    cu_k = np.array([0, 14, 20, 61], dtype=np.uint32)
    qv = O.normal(304, (int(cu_q[-1]), Hq, D))
    kv = O.normal(305, (int(cu_k[-1]), Hkv, D))
    vv = O.normal(306, (int(cu_k[-1]), Hkv, D))
    var = H.fa(qv, kv, vv, 0.25, softcap=4.0, wr=0, alibi=slopes[0], cu_q=cu_q, cu_k=cu_k,
               max_q=31, max_k=41)
    np.savez_compressed(os.path.join(HERE, "ref_fa_terms.npz"), q=q, k=k, v=v, slopes=slopes,
                        dense=dense, cu_q=cu_q, cu_k=cu_k, qv=qv, kv=kv, vv=vv, var=var)
    print("fa", dense.shape, var.shape)


def prod_rows(y: np.ndarray, s: np.ndarray, bits: int = 4) -> tuple[np.ndarray, np.ndarray]:
    """TurboProd rows of rotated rows y through the reference's GPU pipeline
    (TurboQuantizer::quantize_gpu, candle-nn/src/turbo_quant.rs:214-234): tq_quant (stage one:
    codes and norm), the residual of tq_resid_impl (turbo_quant_impl.h:161-176, elementwise f32:
    u = y * (1 / norm), u - centroid), proj = resid S^T (the reference's matmul; float64 here,
    rounded to f32), tq_signs (signs of proj, rsc1 = |resid|). Returns (rows, proj)."""
    d = y.shape[-1]
    l = O.row_layout(O.TURBO_PROD, bits, d)
    c, b = O.lloyd_max(d, bits - 1)
    tab = H.tq_tab(c, b)
    packed = H.tq_quant(y.astype(np.float32), O.TURBO_PROD, l.code_bits, l.code_words,
                        l.aux_words, l.row_words, tab)
    norm = packed[:, l.code_words + l.aux_words].view(np.float32)
    inv = np.where(norm > 0, np.float32(1.0) / np.where(norm > 0, norm, 1), 0).astype(np.float32)
    u = (y * inv[:, None]).astype(np.float32)
    # 3-bit codes straddle words: read them bit by bit
    codes = np.zeros((y.shape[0], d), dtype=np.int64)
    for j in range(d):
        for bit in range(l.code_bits):
            pos = j * l.code_bits + bit
            codes[:, j] |= ((packed[:, pos // 32] >> (pos % 32)) & 1).astype(np.int64) << bit
    resid = (u - c[codes]).astype(np.float32)
    proj = (resid.astype(np.float64) @ s.astype(np.float64).T).astype(np.float32)
    return H.tq_signs(packed, proj, resid, l.code_words), proj


def prod_case():
    """TurboProd-4 keys (3-bit MSE codes + QJL signs) at D = 128: rows through the reference
    kernels (prod_rows), and its fused decode (tq_attn with [q Pi^T, q Pi^T S^T] queries, then
    the value unrotation) over them with TurboQuant-4 values."""
    B, Hq, Hkv, D, Lq, Lk = 2, 8, 2, 128, 2, 300
    rng = np.random.default_rng(700)
    mask = rng.random((Hkv, D)) < 0.01
    q = O.round_bf16(O.normal(701, (B, Hq, Lq, D)))
    k = O.normal(702, (B, Hkv, Lk, D))
    v = O.normal(703, (B, Hkv, Lk, D))
    k = O.round_bf16(np.where(mask[None, :, None, :], k * 8, k)).astype(np.float32)
    v = O.round_bf16(np.where(mask[None, :, None, :], v * 8, v)).astype(np.float32)
    s = O.qjl_matrix(D, 42)
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42)
    pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44)
    kx = O.rotate_rows(pk, k.reshape(-1, D))
    vx = O.rotate_rows(pv, v.reshape(-1, D))
    kd, proj = prod_rows(kx, s)
    kd = kd.reshape(B, Hkv, Lk, -1)
    lv = O.row_layout(O.TURBO_MSE, 4, D)
    cv, bv = O.lloyd_max(D, 4)
    vd = H.tq_quant(vx.astype(np.float32), O.TURBO_MSE, lv.code_bits, lv.code_words,
                    lv.aux_words, lv.row_words, H.tq_tab(cv, bv)).reshape(B, Hkv, Lk, -1)
    lk_ = O.row_layout(O.TURBO_PROD, 4, D)
    ck, bk = O.lloyd_max(D, 3)
    tab64 = np.concatenate([H.tq_tab(ck, bk), H.tq_tab(cv, bv)]).astype(np.float32)
    qr = O.rotate_rows(pk, q.reshape(-1, D)).reshape(q.shape)
    qs = (qr.reshape(-1, D).astype(np.float64) @ s.astype(np.float64).T).astype(np.float32)
    qx = np.concatenate([qr, qs.reshape(q.shape)], -1).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(D))
    k_side = (O.TURBO_PROD, lk_.code_bits, lk_.code_words, lk_.code_words + lk_.aux_words)
    v_side = (O.TURBO_MSE, lv.code_bits, lv.code_words, lv.code_words + lv.aux_words)
    o = H.tq_attn(qx, kd, vd, k_side, v_side, tab64, float(scale), splits=3)
    o = (o.reshape(-1, D) @ pv).reshape(o.shape).astype(np.float32)
    # the inputs regenerate from the seeds above (prod_inputs in the tests); kept: the rows and
    # the output
    np.savez_compressed(os.path.join(HERE, "ref_prod4.npz"), kd=kd, vd=vd, out=o, scale=scale)
    print("prod", kd.shape, o.shape)


def widths_case():
    """TurboQuant widths other than 4 (QuantFormat::TurboMse{1..3}, TurboProd{2, 3}): rows
    through the reference kernels, and its fused decode over TurboMse{4} keys with TurboMse{3}
    values (TurboKvCache::with_formats(TurboMse{4}, TurboMse{3}, ..), the pairing of the
    reference's turbo_kv_cache_fused_matches_unfused test) and over TurboProd{3} keys with
    TurboMse{2} values."""
    quant_case("turbo3_d128", O.TURBO_MSE, 3, 128, 37, 21)
    quant_case("turbo2_d64", O.TURBO_MSE, 2, 64, 19, 22)
    quant_case("turbo1_d64", O.TURBO_MSE, 1, 64, 19, 23)
    prods = {}
    for bits, d, seed in ((3, 128, 24), (2, 64, 25)):
        y = O.normal(seed, (33, d)) * np.float32(2.0)
        y[1, :] = 0.0
        rows, _ = prod_rows(y, O.qjl_matrix(d, 42), bits)
        prods[f"x{bits}"], prods[f"rows{bits}"] = y, rows
    np.savez_compressed(os.path.join(HERE, "ref_prod_widths.npz"), **prods)
    B, Hq, Hkv, D, Lq, Lk = 2, 8, 2, 128, 2, 300
    q = O.round_bf16(O.normal(801, (B, Hq, Lq, D)))
    k = O.round_bf16(O.normal(802, (B, Hkv, Lk, D))).astype(np.float32)
    v = O.round_bf16(O.normal(803, (B, Hkv, Lk, D))).astype(np.float32)
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42)
    pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44)
    kx = O.rotate_rows(pk, k.reshape(-1, D))
    vx = O.rotate_rows(pv, v.reshape(-1, D))
    qr = O.rotate_rows(pk, q.reshape(-1, D)).reshape(q.shape)
    scale = np.float32(1.0 / np.sqrt(D))
    out = {"scale": scale}
    for name, kmode, kbits, vbits in (("mse4_mse3", O.TURBO_MSE, 4, 3),
                                      ("prod3_mse2", O.TURBO_PROD, 3, 2)):
        lk_ = O.row_layout(kmode, kbits, D)
        lv = O.row_layout(O.TURBO_MSE, vbits, D)
        ck, bk = O.lloyd_max(D, lk_.code_bits)
        cv, bv = O.lloyd_max(D, vbits)
        if kmode == O.TURBO_PROD:
            s = O.qjl_matrix(D, 42)
            kd, _ = prod_rows(kx, s, kbits)
            qs = (qr.reshape(-1, D).astype(np.float64) @ s.astype(np.float64).T).astype(np.float32)
            qx = np.concatenate([qr, qs.reshape(q.shape)], -1).astype(np.float32)
        else:
            kd = H.tq_quant(kx.astype(np.float32), kmode, lk_.code_bits, lk_.code_words,
                            lk_.aux_words, lk_.row_words, H.tq_tab(ck, bk))
            qx = qr.astype(np.float32)
        kd = kd.reshape(B, Hkv, Lk, -1)
        vd = H.tq_quant(vx.astype(np.float32), O.TURBO_MSE, lv.code_bits, lv.code_words,
                        lv.aux_words, lv.row_words, H.tq_tab(cv, bv)).reshape(B, Hkv, Lk, -1)
        tab64 = np.concatenate([H.tq_tab(ck, bk), H.tq_tab(cv, bv)]).astype(np.float32)
        k_side = (kmode, lk_.code_bits, lk_.code_words, lk_.code_words + lk_.aux_words)
        v_side = (O.TURBO_MSE, lv.code_bits, lv.code_words, lv.code_words + lv.aux_words)
        o = H.tq_attn(qx, kd, vd, k_side, v_side, tab64, float(scale), splits=3, group=4)
        o = (o.reshape(-1, D) @ pv).reshape(o.shape).astype(np.float32)
        out[f"kd_{name}"], out[f"vd_{name}"], out[f"out_{name}"] = kd, vd, o
        print("decode", name, o.shape)
    np.savez_compressed(os.path.join(HERE, "ref_decode_widths.npz"), **out)


def prod5_case():
    """TurboProd{5} (4-bit MSE codes plus the QJL sketch, QuantFormat::TurboProd { bits: 5 },
    candle-core/src/accel/formats.rs:26-29): rows through the reference kernels at D 128 and 64,
    and the reference's fused decode over TurboProd{5} keys with TurboMse{4} and TurboMse{3}
    values (the inputs of widths_case)."""
    out = {}
    for d, seed in ((128, 26), (64, 27)):
        y = O.normal(seed, (33, d)) * np.float32(2.0)
        y[1, :] = 0.0
        rows, _ = prod_rows(y, O.qjl_matrix(d, 42), 5)
        out[f"x_d{d}"], out[f"rows_d{d}"] = y, rows
    B, Hq, Hkv, D, Lq, Lk = 2, 8, 2, 128, 2, 300
    q = O.round_bf16(O.normal(801, (B, Hq, Lq, D)))
    k = O.round_bf16(O.normal(802, (B, Hkv, Lk, D))).astype(np.float32)
    v = O.round_bf16(O.normal(803, (B, Hkv, Lk, D))).astype(np.float32)
    pk = O.rotation_matrix(D, O.ROT_HADAMARD, 42)
    pv = O.rotation_matrix(D, O.ROT_HADAMARD, 44)
    kx = O.rotate_rows(pk, k.reshape(-1, D))
    vx = O.rotate_rows(pv, v.reshape(-1, D))
    qr = O.rotate_rows(pk, q.reshape(-1, D)).reshape(q.shape)
    scale = np.float32(1.0 / np.sqrt(D))
    out["scale"] = scale
    s = O.qjl_matrix(D, 42)
    lk_ = O.row_layout(O.TURBO_PROD, 5, D)
    ck, bk = O.lloyd_max(D, lk_.code_bits)
    kd, _ = prod_rows(kx, s, 5)
    qs = (qr.reshape(-1, D).astype(np.float64) @ s.astype(np.float64).T).astype(np.float32)
    qx = np.concatenate([qr, qs.reshape(q.shape)], -1).astype(np.float32)
    kd = kd.reshape(B, Hkv, Lk, -1)
    out["kd"] = kd
    for vbits in (4, 3):
        lv = O.row_layout(O.TURBO_MSE, vbits, D)
        cv, bv = O.lloyd_max(D, vbits)
        vd = H.tq_quant(vx.astype(np.float32), O.TURBO_MSE, lv.code_bits, lv.code_words,
                        lv.aux_words, lv.row_words, H.tq_tab(cv, bv)).reshape(B, Hkv, Lk, -1)
        tab64 = np.concatenate([H.tq_tab(ck, bk), H.tq_tab(cv, bv)]).astype(np.float32)
        k_side = (O.TURBO_PROD, lk_.code_bits, lk_.code_words, lk_.code_words + lk_.aux_words)
        v_side = (O.TURBO_MSE, lv.code_bits, lv.code_words, lv.code_words + lv.aux_words)
        o = H.tq_attn(qx, kd, vd, k_side, v_side, tab64, float(scale), splits=3, group=4)
        o = (o.reshape(-1, D) @ pv).reshape(o.shape).astype(np.float32)
        out[f"vd_mse{vbits}"], out[f"out_mse{vbits}"] = vd, o
        print("decode prod5 mse", vbits, o.shape)
    np.savez_compressed(os.path.join(HERE, "ref_prod5.npz"), **out)


def combine_case():
    splits, rows, d = 5, 7, 32
    po = O.normal(201, (splits, rows, d))
    pl = O.normal(202, (splits, rows)) * np.float32(3.0)
    pl[1, 2] = -np.inf
    pl[:, 4] = -np.inf  # a row without keys
    t = H.combine(po, pl)
    np.savez_compressed(os.path.join(HERE, "ref_combine.npz"), part_o=po, part_lse=pl, o=t)
    print("combine", t.shape)


if __name__ == "__main__":
    if not H.available():
        sys.exit("oracle/_ref/accel_host_test missing: run `make -C oracle ref` first")
    if sys.argv[1:] == ["widths"]:  # only the TurboQuant widths fixtures
        widths_case()
        sys.exit(0)
    if sys.argv[1:] == ["prod5"]:  # only the TurboProd{5} fixture
        prod5_case()
        sys.exit(0)
    quant_case("fp8_d128", O.FP8, 0, 128, 37, 11)
    quant_case("fp8_d80", O.FP8, 0, 80, 19, 12)
    quant_case("mxfp4_d128", O.MXFP4, 0, 128, 37, 13)
    quant_case("mxfp4_d64", O.MXFP4, 0, 64, 19, 14)
    quant_case("turbo4_d128", O.TURBO_MSE, 4, 128, 37, 15)
    quant_case("nvfp4_d128", O.NVFP4, 0, 128, 11, 16)
    quant_case("nvfp4_d64", O.NVFP4, 0, 64, 19, 18)
    quant_case("mxfp8_d128", O.MXFP8, 0, 128, 37, 17)
    quant_case("mxfp8_d64", O.MXFP8, 0, 64, 19, 19)
    fa_case()
    attn_case()
    attn_format_case("turbo4", O.TURBO_MSE, 4)
    attn_format_case("mxfp4", O.MXFP4, 0)
    attn_format_case("nvfp4", O.NVFP4, 0)
    attn_format_case("mxfp8", O.MXFP8, 0)
    prod_case()
    widths_case()
    prod5_case()
    combine_case()
