"""Driver of the reference's host-emulator kernel harness (oracle/_ref/accel_host_test).

The harness is the reference's own tq_quant / tq_attn / combine kernel code compiled for the
CPU by oracle/Makefile (`make -C oracle ref`) from the reference tree. File protocol
(candle-core/kernels/tests/accel_host_test.cpp:1-5): repeated
[u32 name_len][name][u8 kind][u64 bytes][bytes], kinds 0 f32, 1 u32, 2 u64, 3 i32, 4 bytes.
"""
from __future__ import annotations

import os
import struct
import subprocess
import tempfile

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
BIN = os.path.join(REPO, "oracle", "_ref", "accel_host_test")

_KINDS = {0: np.float32, 1: np.uint32, 2: np.uint64, 3: np.int32}


def available() -> bool:
    return os.path.exists(BIN) and os.access(BIN, os.X_OK)


def _write(path: str, arrays: dict) -> None:
    with open(path, "wb") as f:
        for name, val in arrays.items():
            if isinstance(val, str):
                kind, data = 4, val.encode()
            else:
                a = np.ascontiguousarray(val)
                kind = {np.dtype(np.float32): 0, np.dtype(np.uint32): 1,
                        np.dtype(np.uint64): 2, np.dtype(np.int32): 3}[a.dtype]
                data = a.tobytes()
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<BQ", kind, len(data)) + data)


def _read(path: str) -> dict:
    out = {}
    with open(path, "rb") as f:
        buf = f.read()
    pos = 0
    while pos < len(buf):
        (nl,) = struct.unpack_from("<I", buf, pos)
        pos += 4
        name = buf[pos:pos + nl].decode()
        pos += nl
        kind, nb = struct.unpack_from("<BQ", buf, pos)
        pos += 9
        raw = buf[pos:pos + nb]
        pos += nb
        out[name] = np.frombuffer(raw, dtype=_KINDS[kind]).copy() if kind in _KINDS else raw
    return out


def run(arrays: dict) -> dict:
    with tempfile.TemporaryDirectory() as d:
        pin, pout = os.path.join(d, "in"), os.path.join(d, "out")
        _write(pin, arrays)
        subprocess.run([BIN, pin, pout], check=True, capture_output=True)
        return _read(pout)


def tq_tab(centroids=None, boundaries=None) -> np.ndarray:
    """The 32-float table of the kernels: [centroids; 16][boundaries; 16], unused = +inf
    (candle-core/src/accel/turbo.rs:47-55)."""
    t = np.zeros(32, dtype=np.float32)
    if centroids is not None:
        t[: len(centroids)] = centroids
        t[16: 16 + len(boundaries)] = boundaries
        t[16 + len(boundaries):] = np.inf
    return t


def tq_quant(x: np.ndarray, mode: int, code_bits: int, code_words: int, aux_words: int,
             row_words: int, tab: np.ndarray, gx: int = 5) -> np.ndarray:
    """Reference `tq_quant_f32` over rows x (rows, D) f32 -> (rows, row_words) u32."""
    rows, d = x.shape
    p = np.array([rows, d, mode, code_bits, code_words, aux_words, row_words, gx, 0], dtype=np.uint32)
    out = run({"op": "tq_quant", "x": x.astype(np.float32), "tab": tab, "params": p})
    return out["out"].reshape(rows, row_words)


def tq_signs(packed: np.ndarray, proj: np.ndarray, resid: np.ndarray, code_words: int,
             gx: int = 5) -> np.ndarray:
    """Reference `tq_signs`: packed prod rows (rows, row_words) with proj = S resid and resid
    (rows, D) f32 -> rows with the QJL sign bits and rsc1 = |resid|."""
    rows, rw = packed.shape
    d = resid.shape[1]
    p = np.array([rows, d, code_words, rw, gx], dtype=np.uint32)
    out = run({"op": "tq_signs", "data": packed.astype(np.uint32),
               "proj": proj.astype(np.float32), "resid": resid.astype(np.float32), "params": p})
    return out["out"].reshape(rows, rw)


def tq_attn(q: np.ndarray, kd: np.ndarray, vd: np.ndarray, k_side, v_side, tab64: np.ndarray,
            scale: float, splits: int = 1, wl: int = -1, wr: int = -1, group: int = 1,
            fp8: bool = False) -> np.ndarray:
    """Reference `tq_attn*` + `tq_combine`: q (B, Hq, Lq, W) f32 rotated queries (W = D, or 2 D
    with S q behind them for prod keys), kd / vd (B, Hkv, Lk, words) u32 rows; sides (mode,
    code_bits, code_words, rsc_offset)."""
    B, Hq, Lq, W = q.shape
    D = W // 2 if k_side[0] == 1 else W
    _, Hkv, Lk, kw = kd.shape
    vw = vd.shape[3]
    u = np.array([B, Lq, Lk, Hq, Hkv, D, *k_side, *v_side, splits, 3, 0, int(fp8), group],
                 dtype=np.uint32)
    s = np.array([Hq * Lq * W, Lq * W, W, Hkv * Lk * kw, Lk * kw, kw, Hkv * Lk * vw, Lk * vw, vw],
                 dtype=np.uint64)
    out = run({"op": "tq_attn", "uparams": u, "strides": s,
               "fparams": np.array([scale, 0.0], dtype=np.float32),
               "iparams": np.array([wl, wr], dtype=np.int32), "q": q.astype(np.float32),
               "kd": kd.astype(np.uint32), "vd": vd.astype(np.uint32), "tab": tab64})
    return out["o"].reshape(B, Hq, Lq, D)


def combine(part_o: np.ndarray, part_lse: np.ndarray) -> np.ndarray:
    """Reference `tq_combine` (output `t`)."""
    splits, rows, d = part_o.shape
    out = run({"op": "combine", "part_o": part_o.astype(np.float32),
               "part_lse": part_lse.astype(np.float32),
               "params": np.array([rows, d, splits], dtype=np.uint32)})
    return out["t"].reshape(rows, d)


def fa(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, softcap: float = 0.0,
       wl: int = -1, wr: int = -1, alibi: np.ndarray | None = None, alibi_bs: int = 0,
       cu_q: np.ndarray | None = None, cu_k: np.ndarray | None = None,
       max_q: int = 0, max_k: int = 0) -> np.ndarray:
    """Reference `fa_tile_impl` (FA3 tiles, f32 q / k / v; flash_attn_impl.h:330-443).
    Dense: q (B, Lq, Hq, D), k / v (B, Lk, Hkv, D) -> (B, Lq, Hq, D). Variable length
    (cu_q / cu_k given): q (total_q, Hq, D), k / v (total_k, Hkv, D) -> (total_q, Hq, D), with
    max_q / max_k as Lq / Lk. Slopes alibi[b * alibi_bs + h]."""
    varlen = cu_q is not None
    if varlen:
        total_q, Hq, D = q.shape
        _, Hkv, _ = k.shape
        B, Lq, Lk = len(cu_q) - 1, max_q, max_k
        st = [0, Hq * D, D, 0, Hkv * D, D, 0, Hkv * D, D]
    else:
        B, Lq, Hq, D = q.shape
        _, Lk, Hkv, _ = k.shape
        total_q = B * Lq
        st = [Lq * Hq * D, Hq * D, D, Lk * Hkv * D, Hkv * D, D, Lk * Hkv * D, Hkv * D, D]
    dmax = 64 if D <= 64 else 128
    arrays = {"op": "fa", "dtypes": np.array([0, 0], dtype=np.uint32),
              "dims": np.array([B, Lq, Lk, Hq, Hkv, D, total_q], dtype=np.uint32),
              "strides": np.array(st, dtype=np.uint64),
              "fparams": np.array([scale, softcap, 1.0, 1.0], dtype=np.float32),
              "iparams": np.array([wl, wr], dtype=np.int32),
              "cfg": np.array([1, dmax, 3, 1, int(varlen), 3, alibi_bs], dtype=np.uint32),
              "q": q.astype(np.float32), "k": k.astype(np.float32), "v": v.astype(np.float32)}
    if alibi is not None:
        arrays["alibi"] = np.ascontiguousarray(alibi, dtype=np.float32)
    if varlen:
        arrays["cu_q"] = np.ascontiguousarray(cu_q, dtype=np.uint32)
        arrays["cu_k"] = np.ascontiguousarray(cu_k, dtype=np.uint32)
    return run(arrays)["o"].reshape(q.shape)
