"""ctypes front end of libcqkv.so (the C ABI of include/cqkv.h) over torch device tensors.

torch supplies device memory and the current stream; every computation runs in the HIP kernels
of libcqkv.so. There is no fallback: when the library is missing or the device is not a GPU,
the calls raise.

Names follow the reference's candle-nn API (paths relative to the reference repository root):
TurboKvCache (candle-nn/src/turbo_quant.rs:793-991), flash_attn
(candle-flash-attn/src/lib.rs:149-157).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcqkv.so")

# formats: the reference's kernel mode ids (candle-core/src/accel/formats.rs:41-48)
TURBO4, TURBOPROD, MXFP4, NVFP4, MXFP8, FP8 = 0, 1, 2, 3, 4, 5
FORMAT_NAMES = {"fp8": FP8, "mxfp4": MXFP4, "turbo4": TURBO4, "turboprod": TURBOPROD,
                "nvfp4": NVFP4, "mxfp8": MXFP8}
BF16, F16, F32 = 0, 1, 2
# cache-side rotations (RotationKind, candle-core/src/accel/config.rs:104-139): DEFAULT is AUTO for
# the TurboQuant formats and NONE for the others; AUTO is HADAMARD at power-of-two head dims and
# DENSE otherwise; HADAMARD at other head dims resolves to DENSE
ROT_DEFAULT, ROT_NONE, ROT_HADAMARD, ROT_DENSE, ROT_AUTO = 0, 1, 2, 3, 4
# rotary layouts: rope (halves) and rope_i (interleaved) of candle-nn/src/rotary_emb.rs
ROPE_HALVES, ROPE_INTERLEAVED = 1, 2
_DTYPES = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}

OK, ERR_ARG, ERR_HIP, ERR_WORKSPACE = 0, -1, -2, -3


class CqkvError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"cqkv error {code}: {msg}")
        self.code = code


class Side(ctypes.Structure):
    _fields_ = [("format", ctypes.c_int32), ("is_value", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
                ("capacity", ctypes.c_int32), ("rotation", ctypes.c_int32),
                ("bits", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("seed", ctypes.c_uint64), ("codes", ctypes.c_void_p),
                ("scales", ctypes.c_void_p), ("qjl", ctypes.c_void_p), ("rot", ctypes.c_void_p)]


class PlainBlock(ctypes.Structure):
    """cqkv_plain_block: plain K / V (batch, kv_heads, capacity, D) with {batch, head, row}
    strides and the valid rows at the start of their planes."""
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("k_strides", ctypes.c_int64 * 3), ("v_strides", ctypes.c_int64 * 3),
                ("rows", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class KvBlock(ctypes.Structure):
    """cqkv_kv_block: a key side, a value side and the valid rows at the start of their planes."""
    _fields_ = [("k", ctypes.POINTER(Side)), ("v", ctypes.POINTER(Side)),
                ("rows", ctypes.c_int32), ("reserved", ctypes.c_int32)]


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libcqkv.so (built by __graft_entry__.build() / `make -C <pkg>/csrc`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {HERE}/csrc`")
        L = ctypes.CDLL(LIB_PATH)
        P, i32, sz, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t, ctypes.c_float
        I64P = ctypes.POINTER(ctypes.c_int64)
        SP = ctypes.POINTER(Side)
        L.cqkv_codes_plane_bytes.argtypes = [i32, i32, i32]
        L.cqkv_codes_plane_bytes.restype = sz
        L.cqkv_scales_plane_bytes.argtypes = [i32, i32, i32]
        L.cqkv_scales_plane_bytes.restype = sz
        L.cqkv_quant_append.argtypes = [SP, P, i32, I64P, i32, i32, P, i32, P]
        L.cqkv_rope_quant_append.argtypes = [SP, SP, P, I64P, P, I64P, P, I64P, i32, i32, i32,
                                             i32, P, P, i32, i32, P, i32, P, I64P, P]
        L.cqkv_decode_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
        L.cqkv_decode_workspace_bytes.restype = sz
        L.cqkv_decode_splits.argtypes = [i32, i32, i32, i32, i32, i32]
        L.cqkv_decode_splits.restype = i32
        L.cqkv_decode_attention.argtypes = [P, i32, I64P, SP, SP, i32, i32, i32, P, i32, f32,
                                            i32, i32, f32, P, i32, P, i32, I64P, i32, P, sz, P]
        L.cqkv_decode_attention_noalloc.argtypes = [P, i32, I64P, SP, SP, i32, i32, i32, P, i32,
                                                    f32, i32, i32, f32, P, i32, P, i32, I64P, i32,
                                                    P]
        BP = ctypes.POINTER(KvBlock)
        L.cqkv_decode_paged_workspace_bytes.argtypes = [BP, i32, i32, i32, i32]
        L.cqkv_decode_paged_workspace_bytes.restype = sz
        L.cqkv_decode_attention_paged.argtypes = [P, i32, I64P, BP, i32, i32, i32, i32, f32, i32,
                                                  i32, f32, P, i32, P, i32, I64P, P, sz, P]
        L.cqkv_flash_attn.argtypes = [P, I64P, P, I64P, P, I64P, P, I64P, i32, i32, i32, i32,
                                      i32, i32, i32, f32, i32, i32, SP, SP, i32, P]
        L.cqkv_flash_attn_ext.argtypes = [P, I64P, P, I64P, P, I64P, P, I64P, i32, i32, i32,
                                          i32, i32, i32, i32, i32, f32, i32, i32, f32, P, i32,
                                          P, P, i32, i32, SP, SP, i32, P, sz, P]
        L.cqkv_flash_attn_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32, i32, i32]
        L.cqkv_flash_attn_workspace_bytes.restype = sz
        PBP = ctypes.POINTER(PlainBlock)
        L.cqkv_flash_attn_blocks_workspace_bytes.argtypes = [PBP, i32, i32, i32, i32, i32, i32]
        L.cqkv_flash_attn_blocks_workspace_bytes.restype = sz
        L.cqkv_flash_attn_blocks.argtypes = [P, I64P, PBP, i32, i32, i32, i32, i32, i32, i32,
                                             i32, f32, i32, i32, f32, P, i32, P, I64P, P, sz, P]
        L.cqkv_fp8_quantize_tensor.argtypes = [P, i32, ctypes.c_int64, P, P, P]
        L.cqkv_hadamard_rows.argtypes = [P, i32, ctypes.c_int64, ctypes.c_int64, i32,
                                         ctypes.c_uint64, P, ctypes.c_int64, P]
        L.cqkv_flash_attn_fp8.argtypes = [P, I64P, P, I64P, P, I64P, P, I64P, i32, i32, i32, i32,
                                          i32, i32, i32, f32, i32, i32, f32, f32, P, P, P, sz, P]
        L.cqkv_flash_attn_fp8_workspace_bytes.argtypes = [i32] * 7
        L.cqkv_flash_attn_fp8_workspace_bytes.restype = sz
        L.cqkv_reference_row_words.argtypes = [i32, i32, i32]
        L.cqkv_reference_row_words.restype = i32
        L.cqkv_rows_import.argtypes = [SP, P, i32, i32, i32, P]
        L.cqkv_rows_export.argtypes = [SP, P, i32, i32, i32, P]
        L.cqkv_side_copy.argtypes = [SP, SP, i32, i32, P]
        L.cqkv_turbo_codebook.argtypes = [i32, i32, P, P]
        L.cqkv_turbo_signs.argtypes = [i32, ctypes.c_uint64, P]
        L.cqkv_qjl_matrix.argtypes = [i32, ctypes.c_uint64, P]
        L.cqkv_rotation_matrix.argtypes = [i32, i32, ctypes.c_uint64, P]
        L.cqkv_resolve_rotation.argtypes = [i32, i32, i32]
        L.cqkv_resolve_rotation.restype = i32
        L.cqkv_dequantize_workspace_bytes.argtypes = [SP, i32, i32, i32]
        L.cqkv_dequantize_workspace_bytes.restype = sz
        L.cqkv_dequantize_rows.argtypes = [SP, i32, i32, i32, i32, P, i32, I64P, P, sz, P]
        L.cqkv_last_error.restype = ctypes.c_char_p
        L.cqkv_version.restype = ctypes.c_char_p
        _lib = L
    return _lib


EXPORTED = ["cqkv_codes_plane_bytes", "cqkv_scales_plane_bytes", "cqkv_quant_append",
            "cqkv_rope_quant_append",
            "cqkv_decode_workspace_bytes", "cqkv_decode_splits", "cqkv_decode_attention",
            "cqkv_decode_attention_noalloc",
            "cqkv_decode_paged_workspace_bytes", "cqkv_decode_attention_paged",
            "cqkv_flash_attn", "cqkv_flash_attn_ext", "cqkv_flash_attn_workspace_bytes",
            "cqkv_flash_attn_blocks", "cqkv_flash_attn_blocks_workspace_bytes",
            "cqkv_fp8_quantize_tensor",
            "cqkv_flash_attn_fp8", "cqkv_flash_attn_fp8_workspace_bytes", "cqkv_hadamard_rows", "cqkv_reference_row_words", "cqkv_rows_import",
            "cqkv_rows_export", "cqkv_side_copy", "cqkv_turbo_codebook", "cqkv_turbo_signs",
            "cqkv_qjl_matrix", "cqkv_rotation_matrix", "cqkv_resolve_rotation",
            "cqkv_dequantize_workspace_bytes", "cqkv_dequantize_rows",
            "cqkv_last_error",
            "cqkv_version"]


def _check(rc: int) -> None:
    if rc != OK:
        raise CqkvError(rc, lib().cqkv_last_error().decode())


def _strides3(t: torch.Tensor, dims) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*[t.stride(i) for i in dims])


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise CqkvError(ERR_ARG, f"{what} must be a GPU tensor (got {t.device})")


# ------------------------------------------------------------------------------------------
# cache sides
# ------------------------------------------------------------------------------------------
@dataclass
class CacheSide:
    """One side (keys or values) of a quantized cache: codes + scales planes for
    (batch, kv_heads) at `capacity` tokens each (layout in include/cqkv.h)."""
    fmt: int
    is_value: bool
    batch: int
    kv_heads: int
    head_dim: int
    capacity: int
    codes: torch.Tensor
    scales: torch.Tensor
    seed: int = 0
    rotation: int = ROT_DEFAULT
    qjl: torch.Tensor | None = None  # TURBOPROD: the (D, D) f32 QJL matrix on the device
    # TurboQuant width (TURBO4: TurboMse{bits} 1-4, TURBOPROD: TurboProd{bits} 2-5; 0 = 4)
    bits: int = 0
    rot: torch.Tensor | None = None  # rotating sides: the (D, D) f32 rotation matrix on the device

    @staticmethod
    def empty(fmt: int, is_value: bool, batch: int, kv_heads: int, head_dim: int,
              capacity: int, device, seed: int = 0,
              rotation: int = ROT_DEFAULT, bits: int = 0) -> "CacheSide":
        capacity = (capacity + 31) // 32 * 32
        cb = lib().cqkv_codes_plane_bytes(fmt, head_dim, capacity)
        sb = lib().cqkv_scales_plane_bytes(fmt, head_dim, capacity)
        if cb == 0:
            raise CqkvError(ERR_ARG, f"format {fmt} / head_dim {head_dim} not supported")
        codes = torch.zeros(batch * kv_heads * cb, dtype=torch.uint8, device=device)
        scales = torch.zeros(batch * kv_heads * sb, dtype=torch.uint8, device=device)
        qjl = qjl_matrix(head_dim, seed).to(device) if fmt == TURBOPROD else None
        kind = resolve_rotation(fmt, rotation, head_dim)
        # the rotation matrix, as TurboQuantizer keeps it on the device whenever it rotates
        rot = (rotation_matrix(head_dim, kind, seed).to(device)
               if kind in (ROT_HADAMARD, ROT_DENSE) else None)
        return CacheSide(fmt, is_value, batch, kv_heads, head_dim, capacity, codes, scales, seed,
                         rotation, qjl, bits, rot)

    def rotation_kind(self) -> int:
        """The resolved rotation: ROT_NONE, ROT_HADAMARD or ROT_DENSE."""
        return resolve_rotation(self.fmt, self.rotation, self.head_dim)

    def rotates(self) -> bool:
        """Whether rows are stored rotated (by the seeded Hadamard or Dense matrix)."""
        return self.rotation_kind() in (ROT_HADAMARD, ROT_DENSE)

    def struct(self) -> Side:
        return Side(self.fmt, int(self.is_value), self.head_dim, self.kv_heads, self.capacity,
                    self.rotation, self.bits, 0, self.seed, self.codes.data_ptr(),
                    self.scales.data_ptr(),
                    None if self.qjl is None else self.qjl.data_ptr(),
                    None if self.rot is None else self.rot.data_ptr())

    def nbytes(self) -> int:
        return self.codes.numel() + self.scales.numel()


def quant_append(side: CacheSide, x: torch.Tensor, position: int = 0,
                 positions: torch.Tensor | None = None) -> None:
    """Quantize x (batch, kv_heads, tokens, D) and write it at `position` (or the per-batch
    device int32 `positions`)."""
    _need_gpu(x, "x")
    if x.dim() != 4 or x.stride(3) != 1:
        raise CqkvError(ERR_ARG, "x must be (batch, kv_heads, tokens, D) with contiguous D")
    b, h, t, d = x.shape
    if h != side.kv_heads or d != side.head_dim or b != side.batch:
        raise CqkvError(ERR_ARG, f"x {tuple(x.shape)} does not match the cache side")
    s = side.struct()
    _check(lib().cqkv_quant_append(ctypes.byref(s), _ptr(x), _DTYPES[x.dtype],
                                   _strides3(x, (0, 1, 2)), b, t, _ptr(positions), position,
                                   _stream(x.device)))


def rope_quant_append(k_side: CacheSide, v_side: CacheSide, q: torch.Tensor, k: torch.Tensor,
                      v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                      kind: int = ROPE_HALVES, position: int = 0,
                      positions: torch.Tensor | None = None,
                      q_out: torch.Tensor | None = None) -> torch.Tensor:
    """rope(q), rope(k) and TurboKvCache::append(k, v) in one launch.

    q (batch, q_heads, tokens, D), k / v (batch, kv_heads, tokens, D), any strides with D
    contiguous, one dtype; cos / sin (rows, D/2) contiguous tables of that dtype, row p holding
    position p. Token i of batch b takes position `position` + i (or positions[b] + i). Returns
    the rotated queries (q_out, or a new (batch, q_heads, tokens, D) tensor)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (cos, "cos"), (sin, "sin")):
        _need_gpu(t, n)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or k.shape != v.shape:
        raise CqkvError(ERR_ARG, "q / k / v must be 4-d and k, v of one shape")
    if any(t.stride(3) != 1 for t in (q, k, v)):
        raise CqkvError(ERR_ARG, "q / k / v need a contiguous head dim")
    b, hq, t_, d = q.shape
    if k.shape[0] != b or k.shape[2] != t_ or k.shape[3] != d:
        raise CqkvError(ERR_ARG, f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree")
    if k.shape[1] != k_side.kv_heads or d != k_side.head_dim or b != k_side.batch:
        raise CqkvError(ERR_ARG, f"k {tuple(k.shape)} does not match the cache side")
    if len({q.dtype, k.dtype, v.dtype, cos.dtype, sin.dtype}) != 1 or q.dtype not in _DTYPES:
        raise CqkvError(ERR_ARG, "q, k, v, cos and sin must share one float dtype")
    if (cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] != d // 2
            or not cos.is_contiguous() or not sin.is_contiguous()):
        raise CqkvError(ERR_ARG, f"cos / sin must be contiguous (rows, {d // 2}) tables")
    if q_out is None:
        q_out = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif q_out.shape != q.shape or q_out.dtype != q.dtype or q_out.stride(3) != 1:
        raise CqkvError(ERR_ARG, "q_out must match q in shape and dtype, with a contiguous D")
    ks, vs = k_side.struct(), v_side.struct()
    _check(lib().cqkv_rope_quant_append(
        ctypes.byref(ks), ctypes.byref(vs), _ptr(q), _strides3(q, (0, 1, 2)), _ptr(k),
        _strides3(k, (0, 1, 2)), _ptr(v), _strides3(v, (0, 1, 2)), _DTYPES[q.dtype], b, t_, hq,
        _ptr(cos), _ptr(sin), cos.shape[0], kind, _ptr(positions), position, _ptr(q_out),
        _strides3(q_out, (0, 1, 2)), _stream(q.device)))
    return q_out


def split_qkv(qkv: torch.Tensor, q_heads: int, kv_heads: int):
    """Views q (b, q_heads, t, D), k, v (b, kv_heads, t, D) of a QKV projection output
    (b, t, (q_heads + 2 kv_heads) D), as the models reshape and transpose it."""
    b, t, w = qkv.shape
    d = w // (q_heads + 2 * kv_heads)
    q = qkv[..., :q_heads * d].view(b, t, q_heads, d).transpose(1, 2)
    k = qkv[..., q_heads * d:(q_heads + kv_heads) * d].view(b, t, kv_heads, d).transpose(1, 2)
    v = qkv[..., (q_heads + kv_heads) * d:].view(b, t, kv_heads, d).transpose(1, 2)
    return q, k, v


def decode_workspace_bytes(batch, q_heads, q_len, head_dim, splits) -> int:
    return lib().cqkv_decode_workspace_bytes(batch, q_heads, q_len, head_dim, splits)


def decode_splits(batch, kv_heads, kv_len, fmt: int = FP8, ragged: bool = False,
                  v_fmt: int | None = None) -> int:
    """Key splits decode_attention uses with splits=0 for keys in `fmt` and values in `v_fmt`
    (default: `fmt`); size the workspace with it."""
    return lib().cqkv_decode_splits(fmt, fmt if v_fmt is None else v_fmt, batch, kv_heads,
                                    kv_len, int(ragged))


def decode_attention(q: torch.Tensor, k: CacheSide, v: CacheSide, kv_len: int,
                     softmax_scale: float, kv_lens: torch.Tensor | None = None,
                     window_left: int = -1, window_right: int = -1,
                     out: torch.Tensor | None = None, splits: int = 0,
                     workspace: torch.Tensor | None = None, softcap: float = 0.0,
                     alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
    """q (batch, q_heads, q_len, D) -> out of the same shape (dtype of q unless `out` given);
    softcap / alibi_slopes ((q_heads) or (batch, q_heads) f32) as FlashAttnConfig's."""
    _need_gpu(q, "q")
    b, hq, lq, d = q.shape
    if q.stride(3) != 1:
        raise CqkvError(ERR_ARG, "q must have a contiguous head dim")
    if b != k.batch or b != v.batch or d != k.head_dim:
        raise CqkvError(ERR_ARG, f"q {tuple(q.shape)} does not match the cache sides")
    if kv_lens is not None and (kv_lens.numel() != b or kv_lens.dtype != torch.int32):
        raise CqkvError(ERR_ARG, "kv_lens must be int32 with one length per batch entry")
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape) or out.stride(3) != 1:
        raise CqkvError(ERR_ARG, f"out {tuple(out.shape)} does not match q")
    ks, vs = k.struct(), v.struct()
    al, al_bs = _alibi_arg(alibi_slopes, b, hq)
    _check(lib().cqkv_decode_attention(
        _ptr(q), _DTYPES[q.dtype], _strides3(q, (0, 1, 2)), ctypes.byref(ks), ctypes.byref(vs), b,
        hq, lq, _ptr(kv_lens), kv_len, softmax_scale, window_left, window_right, softcap, al,
        al_bs, _ptr(out), _DTYPES[out.dtype], _strides3(out, (0, 1, 2)), splits, _ptr(workspace),
        0 if workspace is None else workspace.numel() * workspace.element_size(),
        _stream(q.device)))
    return out


DECODE_SCRATCH_BYTES = 32 << 20  # CQKV_DECODE_SCRATCH_BYTES


def decode_attention_noalloc(q: torch.Tensor, k: CacheSide, v: CacheSide, kv_len: int,
                             softmax_scale: float, kv_lens: torch.Tensor | None = None,
                             window_left: int = -1, window_right: int = -1,
                             out: torch.Tensor | None = None, splits: int = 0,
                             softcap: float = 0.0,
                             alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
    """decode_attention through cqkv_decode_attention_noalloc: no device allocation by the
    library (split partials in its per-GPU device scratch array). `out` must be given for a call
    that may not allocate at all (otherwise torch allocates it here)."""
    _need_gpu(q, "q")
    b, hq, lq, d = q.shape
    if q.stride(3) != 1:
        raise CqkvError(ERR_ARG, "q must have a contiguous head dim")
    if b != k.batch or b != v.batch or d != k.head_dim:
        raise CqkvError(ERR_ARG, f"q {tuple(q.shape)} does not match the cache sides")
    if kv_lens is not None and (kv_lens.numel() != b or kv_lens.dtype != torch.int32):
        raise CqkvError(ERR_ARG, "kv_lens must be int32 with one length per batch entry")
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape) or out.stride(3) != 1:
        raise CqkvError(ERR_ARG, f"out {tuple(out.shape)} does not match q")
    ks, vs = k.struct(), v.struct()
    al, al_bs = _alibi_arg(alibi_slopes, b, hq)
    _check(lib().cqkv_decode_attention_noalloc(
        _ptr(q), _DTYPES[q.dtype], _strides3(q, (0, 1, 2)), ctypes.byref(ks), ctypes.byref(vs), b,
        hq, lq, _ptr(kv_lens), kv_len, softmax_scale, window_left, window_right, softcap, al,
        al_bs, _ptr(out), _DTYPES[out.dtype], _strides3(out, (0, 1, 2)), splits,
        _stream(q.device)))
    return out


def _blocks_struct(blocks):
    """[(k_side, v_side, rows), ...] -> (ctypes array of KvBlock, the Side structs it points to)."""
    sides = [(k.struct(), v.struct()) for k, v, _ in blocks]
    arr = (KvBlock * len(blocks))()
    for i, ((ks, vs), (_, _, rows)) in enumerate(zip(sides, blocks)):
        arr[i].k = ctypes.pointer(ks)
        arr[i].v = ctypes.pointer(vs)
        arr[i].rows = rows
    return arr, sides


def decode_paged_workspace_bytes(blocks, batch: int, q_heads: int, q_len: int) -> int:
    arr, _sides = _blocks_struct(blocks)
    return lib().cqkv_decode_paged_workspace_bytes(arr, len(blocks), batch, q_heads, q_len)


def decode_attention_paged(q: torch.Tensor, blocks, softmax_scale: float, window_left: int = -1,
                           window_right: int = -1, out: torch.Tensor | None = None,
                           workspace: torch.Tensor | None = None, softcap: float = 0.0,
                           alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
    """Decode over paged cache blocks [(k_side, v_side, rows), ...]: the keys are the blocks'
    first `rows` tokens concatenated (attention_packed_blocks, candle-nn/src/turbo_quant.rs:
    1082-1114). q (batch, q_heads, q_len, D) -> out of the same shape."""
    _need_gpu(q, "q")
    b, hq, lq, d = q.shape
    if q.stride(3) != 1:
        raise CqkvError(ERR_ARG, "q must have a contiguous head dim")
    if not blocks:
        raise CqkvError(ERR_ARG, "no blocks")
    for k, v, _ in blocks:
        if b != k.batch or b != v.batch or d != k.head_dim:
            raise CqkvError(ERR_ARG, f"q {tuple(q.shape)} does not match a block's sides")
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape) or out.stride(3) != 1:
        raise CqkvError(ERR_ARG, f"out {tuple(out.shape)} does not match q")
    arr, _sides = _blocks_struct(blocks)
    al, al_bs = _alibi_arg(alibi_slopes, b, hq)
    _check(lib().cqkv_decode_attention_paged(
        _ptr(q), _DTYPES[q.dtype], _strides3(q, (0, 1, 2)), arr, len(blocks), b, hq, lq,
        softmax_scale, window_left, window_right, softcap, al, al_bs, _ptr(out), _DTYPES[out.dtype],
        _strides3(out, (0, 1, 2)), _ptr(workspace),
        0 if workspace is None else workspace.numel() * workspace.element_size(),
        _stream(q.device)))
    return out


def _alibi_arg(alibi_slopes, batch: int, q_heads: int):
    """ALiBi slopes (q_heads) or (batch, q_heads) f32 on the device -> (pointer, batch stride)."""
    if alibi_slopes is None:
        return None, 0
    _need_gpu(alibi_slopes, "alibi_slopes")
    if alibi_slopes.dtype != torch.float32 or not alibi_slopes.is_contiguous():
        raise CqkvError(ERR_ARG, "alibi_slopes must be contiguous float32")
    if tuple(alibi_slopes.shape) == (q_heads,):
        return _ptr(alibi_slopes), 0
    if tuple(alibi_slopes.shape) == (batch, q_heads):
        return _ptr(alibi_slopes), q_heads
    raise CqkvError(ERR_ARG, f"alibi slopes must be ({q_heads}) or ({batch}, {q_heads}), "
                             f"got {tuple(alibi_slopes.shape)}")


def _attn_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple[int, int]:
    """The dtype ids of q and of k / v (head dim contiguous on the GPU): one of bf16, f16, f32
    for all three, or f32 q over f16 / bf16 k / v (kv_dtype_supported,
    candle-core/src/accel/attention.rs:569-576)."""
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _need_gpu(t, name)
        if t.stride(-1) != 1:
            raise CqkvError(ERR_ARG, f"{name} needs a contiguous head dim (stride {t.stride()})")
    ok = q.dtype in _DTYPES and k.dtype == v.dtype and (
        k.dtype == q.dtype or (q.dtype == torch.float32 and k.dtype in (torch.bfloat16,
                                                                         torch.float16)))
    if not ok:
        raise CqkvError(ERR_ARG, f"flash-attn: k/v dtype {k.dtype} / {v.dtype} must match q "
                                 f"{q.dtype}, or be f16 / bf16 with f32 queries")
    return _DTYPES[q.dtype], _DTYPES[k.dtype]


def flash_attn_workspace_bytes(dtype: torch.dtype, batch: int, q_len: int, kv_len: int,
                               q_heads: int, kv_heads: int, head_dim: int,
                               varlen: bool = False) -> int:
    return lib().cqkv_flash_attn_workspace_bytes(_DTYPES[dtype], batch, q_len, kv_len, q_heads,
                                                 kv_heads, head_dim, int(varlen))


def flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, softmax_scale: float,
               causal: bool, window_left: int = -1, window_right: int = -1,
               k_cache: CacheSide | None = None, v_cache: CacheSide | None = None,
               position: int = 0, out: torch.Tensor | None = None, softcap: float = 0.0,
               alibi_slopes: torch.Tensor | None = None,
               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """candle_flash_attn::flash_attn layout: q (b, s_q, h_q, d), k / v (b, s_kv, h_kv, d), all
    bf16, f16 or f32, or f32 q over f16 / bf16 k / v; d a multiple of 8 up to 256; out in q's
    dtype. With k_cache / v_cache K / V are also quantized into the cache at `position`.
    softcap / alibi_slopes as flash_attn_alibi_windowed_softcap (candle-flash-attn/src/lib.rs)."""
    dt, kvt = _attn_inputs(q, k, v)
    b, sq, hq, d = q.shape
    _, sk, hkv, _ = k.shape
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise CqkvError(ERR_ARG, "out must match q in shape and dtype, with a contiguous head dim")
    if causal:
        window_right = 0
    kc = None if k_cache is None else ctypes.byref(k_cache.struct())
    vc = None if v_cache is None else ctypes.byref(v_cache.struct())
    al, al_bs = _alibi_arg(alibi_slopes, b, hq)
    ws = None if workspace is None else _ptr(workspace)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().cqkv_flash_attn_ext(
        _ptr(q), _strides3(q, (0, 1, 2)), _ptr(k), _strides3(k, (0, 1, 2)), _ptr(v),
        _strides3(v, (0, 1, 2)), _ptr(out), _strides3(out, (0, 1, 2)), dt, kvt, b, sq, sk, hq, hkv,
        d, softmax_scale, window_left, window_right, softcap, al, al_bs, None, None, 0, 0, kc, vc,
        position, ws, ws_bytes, _stream(q.device)))
    return out


def flash_attn_blocks(q: torch.Tensor, blocks, softmax_scale: float, window_left: int = -1,
                      window_right: int = -1, softcap: float = 0.0,
                      alibi_slopes: torch.Tensor | None = None,
                      out: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None) -> torch.Tensor:
    """flash_attn_blocks (candle-nn/src/flash_attn.rs:719-765): q (batch, q_heads, q_len, d) over
    blocks [(k, v, rows)] of plain K / V (batch, kv_heads, capacity, d) - the valid rows of all
    blocks in order are the keys of every sequence."""
    _need_gpu(q, "q")
    if not blocks:
        raise CqkvError(ERR_ARG, "no blocks")
    dt, kvt = _attn_inputs(q, blocks[0][0], blocks[0][1])
    b, hq, lq, d = q.shape
    hkv = blocks[0][0].shape[1]
    arr = (PlainBlock * len(blocks))()
    for i, (k, v, rows) in enumerate(blocks):
        _attn_inputs(q, k, v)
        if k.dtype != blocks[0][0].dtype:
            raise CqkvError(ERR_ARG, f"block {i}: K / V dtype {k.dtype} differs from block 0's")
        if k.dim() != 4 or v.shape != k.shape or k.shape[0] != b or k.shape[1] != hkv or \
                k.shape[3] != d:
            raise CqkvError(ERR_ARG, f"block {i}: k {tuple(k.shape)} / v {tuple(v.shape)} do not "
                                     f"match (batch {b}, {hkv} kv heads, head dim {d})")
        if rows > k.shape[2]:
            raise CqkvError(ERR_ARG, f"block {i}: {rows} rows above its capacity {k.shape[2]}")
        arr[i].k, arr[i].v, arr[i].rows = _ptr(k), _ptr(v), int(rows)
        arr[i].k_strides[:] = [k.stride(0), k.stride(1), k.stride(2)]
        arr[i].v_strides[:] = [v.stride(0), v.stride(1), v.stride(2)]
    if out is None:
        out = torch.empty((b, hq, lq, d), dtype=q.dtype, device=q.device)
    al, al_bs = _alibi_arg(alibi_slopes, b, hq)
    ws = None if workspace is None else _ptr(workspace)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().cqkv_flash_attn_blocks(
        _ptr(q), _strides3(q, (0, 1, 2)), arr, len(blocks), dt, kvt, b, hq, lq, hkv, d,
        softmax_scale,
        window_left, window_right, softcap, al, al_bs, _ptr(out), _strides3(out, (0, 1, 2)), ws,
        ws_bytes, _stream(q.device)))
    return out


def fp8_quantize_tensor(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The per-tensor FP8 quantization of flash_attn_fp8 (candle-nn/src/flash_attn.rs:882-887):
    E4M3 codes (uint8, the shape of x) and a device f32 tensor whose element 0 is the scale
    amax / 448 (1 for an all-zero tensor); element 1 is scratch."""
    _need_gpu(x, "x")
    if x.dtype not in _DTYPES or not x.is_contiguous():
        raise CqkvError(ERR_ARG, "x must be a contiguous bf16 / f16 / f32 tensor")
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scale = torch.empty(2, dtype=torch.float32, device=x.device)
    _check(lib().cqkv_fp8_quantize_tensor(_ptr(x), _DTYPES[x.dtype], x.numel(), _ptr(codes),
                                          _ptr(scale), _stream(x.device)))
    return codes, scale


def _fp8_codes(t: torch.Tensor, name: str) -> torch.Tensor:
    if getattr(torch, "float8_e4m3fn", None) is not None and t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    if t.dtype != torch.uint8:
        raise CqkvError(ERR_ARG, f"{name} must hold E4M3 codes (uint8 or float8_e4m3fn)")
    return t


def flash_attn_fp8_codes(q: torch.Tensor, k8: torch.Tensor, v8: torch.Tensor,
                         softmax_scale: float, causal: bool, k_descale: float = 1.0,
                         v_descale: float = 1.0, window_left: int = -1, window_right: int = -1,
                         k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
                         out: torch.Tensor | None = None,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """flash_attn_with_config on F8E4M3 K / V with descale factors (FlashAttnConfig::descale,
    candle-nn/src/flash_attn.rs:113-117): q (b, s_q, h_q, d) bf16, f16 or f32, k8 / v8
    (b, s_kv, h_kv, d) E4M3 codes; keys and values are k8 * k_descale * k_scale[0],
    v8 * v_descale * v_scale[0] (the device scales optional). workspace: a device byte tensor
    of flash_attn_fp8_workspace_bytes (None: allocated by the call)."""
    _need_gpu(q, "q")
    if q.dtype not in _DTYPES:
        raise CqkvError(ERR_ARG, f"q must be bfloat16, float16 or float32, got {q.dtype}")
    k8, v8 = _fp8_codes(k8, "k8"), _fp8_codes(v8, "v8")
    b, sq, hq, d = q.shape
    _, sk, hkv, _ = k8.shape
    if out is None:
        out = torch.empty_like(q)
    if causal:
        window_right = 0
    ws, wsb = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel())
    _check(lib().cqkv_flash_attn_fp8(
        _ptr(q), _strides3(q, (0, 1, 2)), _ptr(k8), _strides3(k8, (0, 1, 2)), _ptr(v8),
        _strides3(v8, (0, 1, 2)), _ptr(out), _strides3(out, (0, 1, 2)), _DTYPES[q.dtype], b, sq,
        sk, hq, hkv, d, softmax_scale, window_left, window_right, k_descale, v_descale,
        _ptr(k_scale), _ptr(v_scale), ws, wsb, _stream(q.device)))
    return out


def flash_attn_fp8_workspace_bytes(dtype, batch: int, q_len: int, kv_len: int, q_heads: int,
                                   kv_heads: int, head_dim: int) -> int:
    """Device bytes flash_attn_fp8_codes needs for a call of these sizes."""
    return lib().cqkv_flash_attn_fp8_workspace_bytes(_DTYPES[dtype], batch, q_len, kv_len,
                                                     q_heads, kv_heads, head_dim)


FP8_HADAMARD_SEED = 0x46413346  # flash_attn.rs:869


def hadamard_rows(x: torch.Tensor, seed: int = FP8_HADAMARD_SEED) -> torch.Tensor:
    """x (..., D) times rotation_matrix(D, Hadamard, seed)^T, in f32, rounded to x's dtype."""
    _need_gpu(x, "x")
    x = x.contiguous()
    d = x.shape[-1]
    out = torch.empty_like(x)
    _check(lib().cqkv_hadamard_rows(_ptr(x), _DTYPES[x.dtype], x.numel() // d, d, d, seed,
                                    _ptr(out), d, _stream(x.device)))
    return out


def flash_attn_fp8(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, softmax_scale: float,
                   causal: bool, window_left: int = -1, window_right: int = -1,
                   out: torch.Tensor | None = None, hadamard: bool = False) -> torch.Tensor:
    """candle_nn::flash_attn::flash_attn_fp8 (candle-nn/src/flash_attn.rs:862-892): K and V
    quantized to E4M3 with per-tensor scales, then attention with those scales as descale
    factors. hadamard=True is the reference's CANDLE_FLASH_ATTN_HADAMARD switch: q and k rotated
    by the same Hadamard matrix first (Q K^T unchanged, outliers spread before the FP8 rounding).
    Nothing waits on the host: the scales stay on the device."""
    d = q.shape[-1]
    if hadamard and d > 1 and d & (d - 1) == 0:  # power-of-two head dims, as the reference
        q, k = hadamard_rows(q), hadamard_rows(k)
    k8, ks = fp8_quantize_tensor(k.contiguous())
    v8, vs = fp8_quantize_tensor(v.contiguous())
    return flash_attn_fp8_codes(q, k8, v8, softmax_scale, causal, 1.0, 1.0, window_left,
                                window_right, ks, vs, out)


def flash_attn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                      max_seqlen_k: int, softmax_scale: float, causal: bool,
                      window_left: int = -1, window_right: int = -1, softcap: float = 0.0,
                      alibi_slopes: torch.Tensor | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """candle_flash_attn::flash_attn_varlen layout: q (total_q, h_q, d), k / v (total_k, h_kv,
    d) with the dtypes of flash_attn, cumulative sequence offsets cu_seqlens_q / cu_seqlens_k
    (batch + 1,) int32 on the device (the reference takes u32)."""
    dt, kvt = _attn_inputs(q, k, v)
    total_q, hq, d = q.shape
    total_k, hkv, _ = k.shape
    for name, c in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k)):
        _need_gpu(c, name)
        if c.dtype != torch.int32 or c.dim() != 1 or not c.is_contiguous():
            raise CqkvError(ERR_ARG, f"{name} must be a contiguous 1-D int32 tensor")
    if cu_seqlens_q.shape != cu_seqlens_k.shape or cu_seqlens_q.numel() < 2:
        raise CqkvError(ERR_ARG, "cu_seqlens_q / cu_seqlens_k must both have batch + 1 entries")
    b = cu_seqlens_q.numel() - 1
    if out is None:
        out = torch.empty_like(q)
    if causal:
        window_right = 0
    al, al_bs = _alibi_arg(alibi_slopes, b, hq)
    strides = lambda t: (ctypes.c_int64 * 3)(0, t.stride(0), t.stride(1))
    _check(lib().cqkv_flash_attn_ext(
        _ptr(q), strides(q), _ptr(k), strides(k), _ptr(v), strides(v), _ptr(out), strides(out),
        dt, kvt, b, max_seqlen_q, max_seqlen_k, hq, hkv, d, softmax_scale, window_left,
        window_right,
        softcap, al, al_bs, _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), total_q, total_k, None, None,
        0, None, 0, _stream(q.device)))
    return out


def reference_row_words(fmt: int, head_dim: int, bits: int = 0) -> int:
    """u32 words of one reference row (formats.rs:206-242); `bits` as CacheSide.bits."""
    return lib().cqkv_reference_row_words(fmt, bits, head_dim)


def rows_import(side: CacheSide, rows: torch.Tensor, position: int = 0) -> None:
    """Reference rows (batch, kv_heads, tokens, row_words) u32 (as int32) -> cache."""
    _need_gpu(rows, "rows")
    b, h, t, w = rows.shape
    if (b, h, w) != (side.batch, side.kv_heads,
                     reference_row_words(side.fmt, side.head_dim, side.bits)):
        raise CqkvError(ERR_ARG, f"rows {tuple(rows.shape)} do not match the cache side")
    if rows.dtype not in (torch.int32, torch.uint32):
        raise CqkvError(ERR_ARG, "rows must be 32-bit words")
    s = side.struct()
    _check(lib().cqkv_rows_import(ctypes.byref(s), _ptr(rows.contiguous()), b, t, position,
                                  _stream(rows.device)))


def rows_export(side: CacheSide, tokens: int, position: int = 0) -> torch.Tensor:
    w = reference_row_words(side.fmt, side.head_dim, side.bits)
    rows = torch.zeros((side.batch, side.kv_heads, tokens, w), dtype=torch.int32,
                       device=side.codes.device)
    s = side.struct()
    _check(lib().cqkv_rows_export(ctypes.byref(s), _ptr(rows), side.batch, tokens, position,
                                  _stream(rows.device)))
    return rows


def side_copy(dst: CacheSide, src: CacheSide, tokens: int) -> None:
    """The first `tokens` positions of every plane of src into dst (a side of another capacity)."""
    ds, ss = dst.struct(), src.struct()
    _check(lib().cqkv_side_copy(ctypes.byref(ds), ctypes.byref(ss), src.batch, tokens,
                                _stream(src.codes.device)))


def grown_capacity(capacity: int, grow_by: int, need: int) -> int:
    """Cache::grown_capacity (candle-nn/src/kv_cache.rs:60-66): the capacity plus
    max(grow_by, capacity / 2, 1) until it holds `need`, here rounded up to 32 tokens."""
    cap = capacity
    while cap < need:
        cap += max(grow_by, cap // 2, 1)
    return (cap + 31) // 32 * 32


def turbo_codebook(head_dim: int, bits: int = 4):
    import numpy as np
    c = np.zeros(16, dtype=np.float32)
    bnd = np.zeros(16, dtype=np.float32)
    _check(lib().cqkv_turbo_codebook(head_dim, bits, c.ctypes.data, bnd.ctypes.data))
    k = 1 << bits
    return c[:k].copy(), bnd[:k - 1].copy()


def qjl_matrix(head_dim: int, seed: int) -> torch.Tensor:
    """The QJL projection S (head_dim, head_dim) f32 of TurboProd (cqkv_qjl_matrix), on the host."""
    s = torch.empty((head_dim, head_dim), dtype=torch.float32)
    _check(lib().cqkv_qjl_matrix(head_dim, seed, ctypes.c_void_p(s.data_ptr())))
    return s


def resolve_rotation(fmt: int, rotation: int, head_dim: int) -> int:
    """RotationKind::resolve of a side's rotation (cqkv_resolve_rotation)."""
    r = lib().cqkv_resolve_rotation(fmt, rotation, head_dim)
    if r < 0:
        raise CqkvError(ERR_ARG, f"rotation {rotation} at head_dim {head_dim}")
    return r


def rotation_matrix(head_dim: int, kind: int, seed: int) -> torch.Tensor:
    """rotation_matrix(head_dim, kind, seed) (candle-core/src/accel/turbo.rs:180-233), f32 on the
    host (cqkv_rotation_matrix)."""
    m = torch.empty((head_dim, head_dim), dtype=torch.float32)
    _check(lib().cqkv_rotation_matrix(head_dim, kind, seed, ctypes.c_void_p(m.data_ptr())))
    return m


def dequantize(side: CacheSide, tokens: int, position: int = 0, unrotate: bool = True,
               dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None) -> torch.Tensor:
    """Cache positions [position, position + tokens) as (batch, kv_heads, tokens, D) values of
    `dtype` (cqkv_dequantize_rows): TurboQuantizer::dequantize_rows, unrotated when `unrotate`
    (candle-nn/src/turbo_quant.rs:250-300)."""
    if out is None:
        out = torch.empty((side.batch, side.kv_heads, tokens, side.head_dim), dtype=dtype,
                          device=side.codes.device)
    elif (tuple(out.shape) != (side.batch, side.kv_heads, tokens, side.head_dim)
          or out.stride(3) != 1):
        raise CqkvError(ERR_ARG, f"out {tuple(out.shape)} does not match the cache side")
    s = side.struct()
    _check(lib().cqkv_dequantize_rows(ctypes.byref(s), side.batch, position, tokens, int(unrotate),
                                      _ptr(out), _DTYPES[out.dtype], _strides3(out, (0, 1, 2)),
                                      None, 0, _stream(out.device)))
    return out


def turbo_signs(head_dim: int, seed: int):
    import numpy as np
    s = np.zeros(head_dim, dtype=np.float32)
    _check(lib().cqkv_turbo_signs(head_dim, seed, s.ctypes.data))
    return s


# ------------------------------------------------------------------------------------------
# host-side mirror of candle-nn's TurboKvCache (candle-nn/src/turbo_quant.rs:793-991)
# ------------------------------------------------------------------------------------------
class TurboKvCache:
    """A quantized KV cache for (batch, kv_heads, head_dim), keys in `key_format` (FP8, MXFP4,
    MXFP8, NVFP4, TURBO4 or TURBOPROD) and values in `value_format` (the same but TURBOPROD),
    TurboQuant widths `key_bits` / `value_bits` (0: 4), rotated per `rotation` with seeds `seed`
    (keys) and `seed + 2` (values) as TurboKvCache::with_formats does
    (candle-nn/src/turbo_quant.rs:858-879). It grows past `capacity` as Cache::append does."""

    def __init__(self, key_format: int, value_format: int, batch: int, kv_heads: int,
                 head_dim: int, capacity: int, device="cuda", seed: int = 42,
                 grow_by: int | None = None, rotation: int = ROT_DEFAULT, key_bits: int = 0,
                 value_bits: int = 0):
        if value_format == TURBOPROD:
            raise CqkvError(ERR_ARG, "turbo-quant: values use the MSE codebooks, not the prod "
                                     "(QJL) format")
        self.k = CacheSide.empty(key_format, False, batch, kv_heads, head_dim, capacity, device,
                                 seed, rotation, key_bits)
        self.v = CacheSide.empty(value_format, True, batch, kv_heads, head_dim, capacity, device,
                                 seed + 2, rotation, value_bits)
        self._len = 0
        self.dim = head_dim
        # Cache::new(dim, max_seq_len) grows by max_seq_len (kv_cache.rs:19-27)
        self.grow_by = capacity if grow_by is None else grow_by

    def _reserve(self, need: int) -> None:
        """Grows both sides to hold `need` tokens as Cache::append does: one new buffer at the
        grown capacity and one copy of the tokens so far."""
        if need <= self.k.capacity:
            return
        cap = grown_capacity(self.k.capacity, self.grow_by, need)
        dev = self.k.codes.device
        sides = []
        for old in (self.k, self.v):
            new = CacheSide.empty(old.fmt, old.is_value, old.batch, old.kv_heads, old.head_dim,
                                  cap, dev, old.seed, old.rotation, old.bits)
            new.qjl = old.qjl
            new.rot = old.rot
            if self._len:
                side_copy(new, old, self._len)
            sides.append(new)
        self.k, self.v = sides

    def formats(self):
        return self.k.fmt, self.v.fmt

    def seq_len(self) -> int:
        return self._len

    def reset(self) -> None:
        self._len = 0

    def storage_bytes(self) -> int:
        return self.k.nbytes() + self.v.nbytes()

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: (batch, kv_heads, tokens, head_dim)."""
        if k.shape != v.shape or k.dim() != 4 or k.shape[3] != self.dim:
            raise CqkvError(ERR_ARG, f"turbo-quant cache: k {tuple(k.shape)} / v {tuple(v.shape)}"
                                     f" do not match head dim {self.dim}")
        t = k.shape[2]
        self._reserve(self._len + t)
        quant_append(self.k, k, self._len)
        quant_append(self.v, v, self._len)
        self._len += t

    def rope_append(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, kind: int = ROPE_HALVES) -> torch.Tensor:
        """The model step rope(q), rope(k), append(k, v) in one launch, the new tokens taking
        positions seq_len.. (their rows of cos / sin). Returns the rotated q."""
        t = k.shape[2] if k.dim() == 4 else 0
        self._reserve(self._len + t)
        out = rope_quant_append(self.k, self.v, q, k, v, cos, sin, kind, self._len)
        self._len += t
        return out

    def attention(self, q: torch.Tensor, softmax_scale: float, window_left: int = -1,
                  window_right: int = -1, splits: int = 0, softcap: float = 0.0,
                  alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
        """q (batch, q_heads, q_len, head_dim), bottom-right aligned over the cached tokens."""
        if self._len == 0:
            raise CqkvError(ERR_ARG, "turbo-quant cache: attention on an empty cache")
        return decode_attention(q, self.k, self.v, self._len, softmax_scale,
                                window_left=window_left, window_right=window_right,
                                splits=splits, softcap=softcap, alibi_slopes=alibi_slopes)

    def keys_values(self, dtype: torch.dtype = torch.float32):
        """The cached keys and values (batch, kv_heads, seq_len, head_dim), dequantized and
        unrotated, in `dtype` (TurboKvCache::keys_values, candle-nn/src/turbo_quant.rs:948-966);
        None on an empty cache."""
        if self._len == 0:
            return None
        return (dequantize(self.k, self._len, dtype=dtype),
                dequantize(self.v, self._len, dtype=dtype))
