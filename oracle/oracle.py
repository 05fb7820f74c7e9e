"""ctypes front end of the CPU oracle (oracle.c) plus numpy helpers.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker. The product package never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

TURBO_MSE, TURBO_PROD, MXFP4, NVFP4, MXFP8, FP8 = 0, 1, 2, 3, 4, 5
ROT_NONE, ROT_HADAMARD, ROT_DENSE = 0, 1, 2

_lib = None


def build() -> None:
    """Compiles liboracle.so with the oracle's Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, u64, f32, sz = ctypes.c_int, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t
        L.orc_splitmix_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_splitmix_next.restype = ctypes.c_uint64
        L.orc_fill_normal.argtypes = [u64, P, sz]
        L.orc_f32_to_bf16.argtypes = [f32]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_e4m3_to_f32.restype = f32
        L.orc_f32_to_e4m3.argtypes = [f32]
        L.orc_f32_to_e4m3.restype = ctypes.c_uint8
        L.orc_fp4_to_f32.argtypes = [ctypes.c_uint32]
        L.orc_fp4_to_f32.restype = f32
        L.orc_f32_to_fp4.argtypes = [f32]
        L.orc_f32_to_fp4.restype = ctypes.c_uint32
        L.orc_e8m0_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_e8m0_to_f32.restype = f32
        L.orc_mx_scale_code.argtypes = [f32, i32]
        L.orc_mx_scale_code.restype = ctypes.c_uint8
        L.orc_row_layout.argtypes = [i32, i32, i32, P]
        L.orc_lloyd_max.argtypes = [i32, i32, P, P]
        L.orc_rotation_matrix.argtypes = [i32, i32, u64, P]
        L.orc_rotate_rows.argtypes = [P, i32, P, sz, P]
        L.orc_unrotate_rows.argtypes = [P, i32, P, sz, P]
        L.orc_quantize_rows.argtypes = [i32, i32, i32, sz, P, P, i32]
        L.orc_dequantize_rows.argtypes = [i32, i32, i32, sz, P, P, i32]
        L.orc_key_range.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, i32, i32,
                                    ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
        L.orc_attention_unfused.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, P, f32, f32,
                                            i32, i32, P, P, i32]
        L.orc_cache_attention.argtypes = [P, P, P, i32, i32, i32, i32, P, P, P, i32, i32, i32,
                                          i32, i32, i32, P, i32, f32, i32, i32, f32, P, P, i32]
        L.orc_qjl_matrix.argtypes = [i32, u64, P]
        L.orc_quantize_rows_qjl.argtypes = [i32, i32, sz, P, P, P, i32]
        L.orc_dequantize_rows_qjl.argtypes = [i32, i32, sz, P, P, P, i32]
        L.orc_combine.argtypes = [P, P, P, sz, i32, i32]
        L.orc_e4m3_encode_n.argtypes = [P, P, sz]
        L.orc_fp4_encode_n.argtypes = [P, P, sz]
        L.orc_split_count_grouped.argtypes = [sz, i32, sz, i32, i32]
        L.orc_row_group.argtypes = [i32, i32]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------------------------
# scalar codecs
# --------------------------------------------------------------------------------------------
def e4m3_to_f32(c: int) -> float:
    return lib().orc_e4m3_to_f32(c)


def f32_to_e4m3(x: float) -> int:
    return lib().orc_f32_to_e4m3(x)


def fp4_to_f32(c: int) -> float:
    return lib().orc_fp4_to_f32(c)


def f32_to_fp4(x: float) -> int:
    return lib().orc_f32_to_fp4(x)


def e8m0_to_f32(c: int) -> float:
    return lib().orc_e8m0_to_f32(c)


def mx_scale_code(amax: float, emax: int) -> int:
    return lib().orc_mx_scale_code(amax, emax)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_e4m3_encode_n(_p(x), _p(out), x.size)
    return out


def fp4_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_fp4_encode_n(_p(x), _p(out), x.size)
    return out


def splitmix_u64(seed: int, n: int) -> list[int]:
    s = ctypes.c_uint64(seed)
    return [lib().orc_splitmix_next(ctypes.byref(s)) for _ in range(n)]


def normal(seed: int, shape) -> np.ndarray:
    """`SplitMix64::new(seed).next_normal() as f32`, row-major over `shape`."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(seed, _p(out), n)
    return out.reshape(shape)


# --------------------------------------------------------------------------------------------
# bf16 helpers (vectorised; same rule as orc_f32_to_bf16 / half::bf16::from_f32)
# --------------------------------------------------------------------------------------------
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    up = ((u & 0x8000) != 0) & ((u & 0x17FFF) != 0)
    r = (u >> 16) + up.astype(np.uint32)
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# --------------------------------------------------------------------------------------------
# layouts, codebooks, rotations, row codec
# --------------------------------------------------------------------------------------------
class Layout(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int), ("code_bits", ctypes.c_int), ("code_words", ctypes.c_int),
                ("aux_words", ctypes.c_int), ("row_words", ctypes.c_int)]


def row_layout(mode: int, bits: int, dim: int) -> Layout:
    l = Layout()
    if lib().orc_row_layout(mode, bits, dim, ctypes.byref(l)) != 0:
        raise ValueError(f"invalid format {mode}/{bits} for dim {dim}")
    return l


def lloyd_max(dim: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    k = 1 << bits
    c = np.zeros(16, dtype=np.float32)
    b = np.zeros(16, dtype=np.float32)
    if lib().orc_lloyd_max(dim, bits, _p(c), _p(b)) != 0:
        raise ValueError("bad codebook args")
    return c[:k].copy(), b[: k - 1].copy()


def rotation_matrix(dim: int, kind: int, seed: int) -> np.ndarray:
    m = np.zeros((dim, dim), dtype=np.float32)
    if lib().orc_rotation_matrix(dim, kind, seed, _p(m)) != 0:
        raise ValueError("bad rotation args")
    return m


def rotate_rows(pi: np.ndarray, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = pi.shape[0]
    y = np.empty_like(x)
    lib().orc_rotate_rows(_p(np.ascontiguousarray(pi)), d, _p(x), x.size // d, _p(y))
    return y


def unrotate_rows(pi: np.ndarray, y: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    d = pi.shape[0]
    x = np.empty_like(y)
    lib().orc_unrotate_rows(_p(np.ascontiguousarray(pi)), d, _p(y), y.size // d, _p(x))
    return x


def quantize_rows(mode: int, bits: int, y: np.ndarray, threads: int = 8) -> np.ndarray:
    """Rows (.., dim) f32 (already rotated) -> (.., row_words) u32 reference rows."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    d = y.shape[-1]
    l = row_layout(mode, bits, d)
    rows = y.size // d
    out = np.zeros(rows * l.row_words, dtype=np.uint32)
    if lib().orc_quantize_rows(mode, bits, d, rows, _p(y), _p(out), threads) != 0:
        raise ValueError("quantize_rows failed")
    return out.reshape(y.shape[:-1] + (l.row_words,))


def dequantize_rows(mode: int, bits: int, dim: int, words: np.ndarray, threads: int = 8) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    l = row_layout(mode, bits, dim)
    rows = words.size // l.row_words
    out = np.zeros(rows * dim, dtype=np.float32)
    if lib().orc_dequantize_rows(mode, bits, dim, rows, _p(words), _p(out), threads) != 0:
        raise ValueError("dequantize_rows failed")
    return out.reshape(words.shape[:-1] + (dim,))


def qjl_matrix(dim: int, seed: int) -> np.ndarray:
    """The QJL projection S (dim, dim) f32 of TurboProd (turbo.rs:236-239)."""
    s = np.zeros((dim, dim), dtype=np.float32)
    lib().orc_qjl_matrix(dim, seed, _p(s))
    return s


def quantize_rows_qjl(bits: int, y: np.ndarray, s: np.ndarray, threads: int = 8) -> np.ndarray:
    """TurboProd{bits} rows (RowCodec::quantize_row with the QJL stage, turbo.rs:299-323) of
    rotated rows y (.., dim) with the QJL matrix s."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    s = np.ascontiguousarray(s, dtype=np.float32)
    d = y.shape[-1]
    l = row_layout(TURBO_PROD, bits, d)
    rows = y.size // d
    out = np.zeros(rows * l.row_words, dtype=np.uint32)
    if lib().orc_quantize_rows_qjl(bits, d, rows, _p(y), _p(s), _p(out), threads) != 0:
        raise ValueError("quantize_rows_qjl failed")
    return out.reshape(y.shape[:-1] + (l.row_words,))


def dequantize_rows_qjl(bits: int, dim: int, words: np.ndarray, s: np.ndarray,
                        threads: int = 8) -> np.ndarray:
    """RowCodec::dequantize_row with the QJL correction (turbo.rs:401-424), rotated domain."""
    words = np.ascontiguousarray(words, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.float32)
    l = row_layout(TURBO_PROD, bits, dim)
    rows = words.size // l.row_words
    out = np.zeros(rows * dim, dtype=np.float32)
    if lib().orc_dequantize_rows_qjl(bits, dim, rows, _p(words), _p(s), _p(out), threads) != 0:
        raise ValueError("dequantize_rows_qjl failed")
    return out.reshape(words.shape[:-1] + (dim,))


def key_range(i: int, lq: int, lk: int, wl: int, wr: int) -> tuple[int, int]:
    lo, hi = ctypes.c_int64(), ctypes.c_int64()
    lib().orc_key_range(i, lq, lk, wl, wr, ctypes.byref(lo), ctypes.byref(hi))
    return lo.value, hi.value


# --------------------------------------------------------------------------------------------
# per-tensor FP8 quantization
# --------------------------------------------------------------------------------------------
def fp8_quantize_tensor(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """flash_attn_fp8's K / V quantization (candle-nn/src/flash_attn.rs:882-887): amax = max |x|
    over the f32 tensor, scale = amax / 448 (1 when amax is 0), codes = E4M3 of x / scale, where
    candle's `tensor / f64` is affine(1 / rhs, 0) (candle-core/src/tensor.rs:3124) computed as
    v * f32(mul) + f32(add) (candle-core/src/cpu_backend/mod.rs:313-315): the reciprocal in f64,
    rounded to f32, one f32 multiply, then + 0 (which turns -0 into +0)."""
    x = np.asarray(x, np.float32)
    amax = np.float32(np.abs(x).max()) if x.size else np.float32(0.0)
    scale = np.float32(amax / np.float32(448.0)) if amax > 0 else np.float32(1.0)
    mul = np.float32(1.0 / np.float64(scale))
    q = (x * mul + np.float32(0.0)).astype(np.float32)
    return e4m3_encode(q).astype(np.uint8), scale


# --------------------------------------------------------------------------------------------
# rotary embeddings
# --------------------------------------------------------------------------------------------
ROPE_HALVES, ROPE_INTERLEAVED = 1, 2


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """x (f32) rounded to "bf16" / "f16" (round to nearest even) and back, or left as "f32"."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, kind: int, pos0: int) -> np.ndarray:
    """Rotary embedding of x (..., t, d) f32, token i at table row pos0 + i of cos / sin
    ((rows, d/2) f32); f32 result, before the rounding to the tensor dtype.

    Follows the reference's ROCm kernels rope_impl / rope_i_impl
    (candle-core/kernels/nn.hip:107-148: products rounded to f32 separately, then the difference
    or sum) and its f32 CPU path (candle-nn/src/rotary_emb.rs:47-76, the same expressions):
      halves:      y_i = x_i c_i - x_{i+d/2} s_i,   y_{i+d/2} = x_i s_i + x_{i+d/2} c_i
      interleaved: y_2i = x_2i c_i - x_2i+1 s_i,   y_2i+1 = x_2i s_i + x_2i+1 c_i
    numpy evaluates each product and sum in f32 with one rounding each, as those kernels do."""
    x = np.asarray(x, np.float32)
    t, d = x.shape[-2], x.shape[-1]
    c = np.asarray(cos, np.float32)[pos0:pos0 + t]
    s = np.asarray(sin, np.float32)[pos0:pos0 + t]
    if c.shape[0] != t:
        raise ValueError("rope: positions past the cos / sin table")
    y = np.empty_like(x)
    if kind == ROPE_HALVES:
        a, b = x[..., :d // 2], x[..., d // 2:]
        y[..., :d // 2] = a * c - b * s
        y[..., d // 2:] = a * s + b * c
    elif kind == ROPE_INTERLEAVED:
        a, b = x[..., 0::2], x[..., 1::2]
        y[..., 0::2] = a * c - b * s
        y[..., 1::2] = a * s + b * c
    else:
        raise ValueError(f"rope kind {kind}")
    return y


# --------------------------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------------------------
def attention_unfused(q, k, v, scale, kv_lens=None, softcap=0.0, wl=-1, wr=-1, alibi=None,
                      threads: int = 8) -> np.ndarray:
    """q (b, hq, lq, d), k / v (b, hkv, lk, d) f32 -> (b, hq, lq, d) f32 (CPU unfused path)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    b, hq, lq, d = q.shape
    _, hkv, lk, _ = k.shape
    out = np.zeros_like(q)
    kl = None if kv_lens is None else np.ascontiguousarray(kv_lens, dtype=np.int32)
    al = None if alibi is None else np.ascontiguousarray(alibi, dtype=np.float32)
    rc = lib().orc_attention_unfused(_p(q), _p(k), _p(v), b, hq, hkv, lq, lk, d, _p(kl), scale,
                                     softcap, wl, wr, _p(al), _p(out), threads)
    if rc != 0:
        raise ValueError("attention_unfused failed")
    return out


def cache_attention(q_bf16_bits, k_rows, v_rows, k_fmt, v_fmt, pi_k, pi_v, lk, scale,
                    kv_lens=None, wl=-1, wr=-1, threads: int = 8, qjl_k=None, softcap=0.0,
                    alibi=None) -> np.ndarray:
    """The reference CPU decode path over packed rows. q_bf16_bits (b, hq, lq, d) u16,
    k_rows / v_rows (b, hkv, cap, row_words) u32, formats (mode, bits); qjl_k: the QJL matrix
    of TurboProd keys; softcap and per-head ALiBi slopes as attention_unfused. Output f32."""
    q = np.ascontiguousarray(q_bf16_bits, dtype=np.uint16)
    k_rows = np.ascontiguousarray(k_rows, dtype=np.uint32)
    v_rows = np.ascontiguousarray(v_rows, dtype=np.uint32)
    b, hq, lq, d = q.shape
    _, hkv, cap, _ = k_rows.shape
    out = np.zeros((b, hq, lq, d), dtype=np.float32)
    kl = None if kv_lens is None else np.ascontiguousarray(kv_lens, dtype=np.int32)
    pk = None if pi_k is None else np.ascontiguousarray(pi_k, dtype=np.float32)
    pv = None if pi_v is None else np.ascontiguousarray(pi_v, dtype=np.float32)
    sk = None if qjl_k is None else np.ascontiguousarray(qjl_k, dtype=np.float32)
    al = None if alibi is None else np.ascontiguousarray(alibi, dtype=np.float32)
    rc = lib().orc_cache_attention(_p(q), _p(k_rows), _p(v_rows), k_fmt[0], k_fmt[1], v_fmt[0],
                                   v_fmt[1], _p(pk), _p(pv), _p(sk), b, hq, hkv, lq, cap, d, _p(kl), lk,
                                   scale, wl, wr, softcap, _p(al), _p(out), threads)
    if rc != 0:
        raise ValueError(f"cache_attention failed ({rc})")
    return out


def combine(part_o: np.ndarray, part_lse: np.ndarray) -> np.ndarray:
    part_o = np.ascontiguousarray(part_o, dtype=np.float32)
    part_lse = np.ascontiguousarray(part_lse, dtype=np.float32)
    splits, rows, d = part_o.shape
    o = np.zeros((rows, d), dtype=np.float32)
    lib().orc_combine(_p(part_o), _p(part_lse), _p(o), rows, d, splits)
    return o


def split_count_grouped(rows: int, group: int, lk: int, compute_units: int, fixed: int = 0) -> int:
    return lib().orc_split_count_grouped(rows, group, lk, fixed, compute_units)


def row_group(hq: int, hkv: int) -> int:
    return lib().orc_row_group(hq, hkv)
