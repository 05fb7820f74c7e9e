/*
 * cqkv: MI355X (gfx950) quantized-KV fused attention, C ABI.
 *
 * This is the drop-in boundary of the quantized-KV attention path of the candle fork
 * Qntology/candle-rocm-vulkan. Every entry point is a host function taking device pointers,
 * explicit sizes / strides and a hipStream_t (NULL = the legacy stream the reference launches on),
 * and returning CQKV_OK or a negative status; cqkv_last_error() gives the message of the last
 * failure of the calling thread. Device memory is allocated (stream-ordered, hipMallocAsync /
 * hipFreeAsync on the call's stream) only by: cqkv_decode_attention,
 * cqkv_decode_attention_paged, cqkv_flash_attn_ext, cqkv_flash_attn_blocks and
 * cqkv_dequantize_rows when they are given no workspace (each has a *_workspace_bytes query);
 * cqkv_flash_attn (its workspace); cqkv_flash_attn_fp8 given no workspace (the staged K / V and
 * the attention's workspace); cqkv_quant_append, cqkv_rope_quant_append and the cache append of
 * cqkv_flash_attn(_ext) for a side whose rows are staged (a rotation by its matrix, or a head dim
 * below the plane row: an f32 copy of the rows, and a padded QJL matrix for TurboProd), and
 * cqkv_rope_quant_append when it runs as separate launches (plane rows of 256, staged sides: the
 * rotated keys). cqkv_decode_attention_noalloc allocates nothing; its scratch array is a
 * 32 MiB (CQKV_DECODE_SCRATCH_BYTES) static device array that every process loading the library
 * holds on every device it uses, whether or not that entry point is called. Nothing here holds
 * torch or candle types.
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   cqkv_quant_append      RocmStorage::tq_quantize + Cache::append
 *                          (candle-core/src/rocm_backend/accel.rs:269-303,
 *                           candle-nn/src/turbo_quant.rs:916-945, candle-nn/src/kv_cache.rs:68-99)
 *   cqkv_rope_quant_append the model-side sequence rope(q), rope(k), TurboKvCache::append(k, v)
 *                          in one launch: candle_nn::rotary_emb::rope / rope_i
 *                          (candle-nn/src/rotary_emb.rs:275-303, 585-611; ROCm kernels
 *                          candle-core/kernels/nn.hip:107-148) followed by the append above
 *   cqkv_decode_attention  RocmStorage::tq_attention (+ tq_combine)
 *                          (candle-core/src/rocm_backend/accel.rs:425-571,
 *                           candle-nn/src/turbo_quant.rs:1143-1264)
 *   cqkv_decode_attention_paged
 *                          RocmStorage::tq_attention_paged over a PageTable of cache blocks
 *                          (candle-core/src/rocm_backend/accel.rs:425-571,
 *                           candle-core/src/accel/attention.rs:293-366,
 *                           candle-nn/src/turbo_quant.rs:1082-1114 attention_packed_blocks)
 *   cqkv_flash_attn        RocmStorage::flash_attn (candle-core/src/rocm_backend/accel.rs:54-158),
 *                          behind candle_flash_attn::flash_attn (candle-flash-attn/src/lib.rs:149)
 *   cqkv_flash_attn_ext    the same with soft-capping, ALiBi and variable-length batches:
 *                          flash_attn_alibi_windowed_softcap / flash_attn_varlen*
 *                          (candle-flash-attn/src/lib.rs:41-511; FlashAttnParams.softcap,
 *                          FaExtra.alibi, cu_seqlens in candle-core/src/accel/attention.rs)
 *   cqkv_fp8_quantize_tensor / cqkv_flash_attn_fp8 / cqkv_hadamard_rows
 *                          flash_attn_fp8 and the F8E4M3 K / V path of flash_attn_with_config
 *                          with FlashAttnConfig::descale (candle-nn/src/flash_attn.rs:113-117,
 *                          862-892; kernels candle-core/kernels/flash_attn_impl.h:52-63, 381, 434)
 *   cqkv_flash_attn_blocks flash_attn_blocks over blocks of plain K / V, the paged row kernels
 *                          fa_rowp_* (candle-nn/src/flash_attn.rs:705-836,
 *                          candle-core/src/accel/attention.rs:293-366)
 *   cqkv_rows_import /     the reference's packed row layout [codes][aux][rsc0][rsc1]
 *   cqkv_rows_export       (candle-core/src/accel/formats.rs:206-242)
 *   cqkv_side_copy         the grown-buffer copy of Cache::append (candle-nn/src/kv_cache.rs:56-99)
 *   cqkv_dequantize_rows   RocmStorage::tq_dequantize + TurboQuantizer::dequantize_rows
 *                          (candle-core/src/rocm_backend/accel.rs:380-419,
 *                           candle-nn/src/turbo_quant.rs:250-300, 612-689, 948-966)
 *   cqkv_qjl_matrix / cqkv_turbo_codebook / cqkv_turbo_signs / cqkv_rotation_matrix /
 *   cqkv_resolve_rotation  qjl_matrix, Codebook, the Hadamard signs, rotation_matrix
 *                          (candle-core/src/accel/turbo.rs), RotationKind::resolve
 *                          (candle-core/src/accel/config.rs:131-138)
 *
 * Cache layout in HBM (one "plane" per (batch, kv head), planes batch-major, `capacity` tokens):
 *   format        codes plane (bytes)                  scales plane (bytes)
 *   FP8   keys    capacity * D      row-major          capacity * 4   f32 absmax/448 per token
 *   FP8   values  capacity * D      8-token tiles      capacity * 4   f32 per token
 *   MXFP4 keys    capacity * D/2    row-major nibbles  capacity * D/32  E8M0 per 32-element block
 *   MXFP4 values  capacity * D/2    8-token tiles      capacity * D/32  E8M0
 *   TURBO4 keys   capacity * D/2    row-major nibbles  capacity * 4   f32 norm per token
 *   TURBO4 values capacity * D/2    8-token tiles      capacity * 4   f32 norm
 *   MXFP8 keys    capacity * D      row-major          capacity * D/32  E8M0 per 32-element block
 *   MXFP8 values  capacity * D      8-token tiles      capacity * D/32  E8M0
 *   NVFP4 keys    capacity * D/2    row-major nibbles  capacity * D/16  E4M3 per 16-element block,
 *                                                      then capacity * 4  f32 per token
 *   NVFP4 values  capacity * D/2    8-token tiles      the same
 *   TURBOPROD keys capacity * D/2   row-major nibbles  capacity * (8 + D/8): f32 norms, f32 |r|,
 *                  (3-bit codes)                       then D/8 QJL sign-bit bytes per token
 * D in this table is the plane row length D' = 64, 128 or 256, the smallest that holds the head
 * dim (elements past the head dim are zero codes with zero block scales).
 * Row-major: token t's codes at t * row_bytes, element j at byte j (FP8) or nibble j (bits 4(j%2)
 * of byte j/2), i.e. the reference's code stream. 8-token tiles (values): token t, element j at
 * tile t/8, offset j*8 + t%8 bytes (FP8) or bits 4(t%8) of the little-endian u32 j (4-bit). The
 * code values are the reference encoders' codes bit for bit; only their positions differ.
 */
#ifndef CQKV_H
#define CQKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *cqkv_stream_t; /* == hipStream_t */

/* Status codes. */
enum {
    CQKV_OK = 0,
    CQKV_ERR_ARG = -1,      /* invalid argument / unsupported shape (the reference's bail!) */
    CQKV_ERR_HIP = -2,      /* a HIP runtime call failed (the reference's RocmError::Hip) */
    CQKV_ERR_WORKSPACE = -3 /* workspace too small */
};

/* Empty inputs (the reference's accelerated attention, candle-core/src/rocm_backend/accel.rs:87,
 * 197, 481): an attention call with no query rows (batch or q_len 0) returns CQKV_OK after its
 * argument checks and launches nothing but the cache append of cqkv_flash_attn(_ext) when K / V
 * rows are given; q / out (and K / V without rows) may then be null. No keys (kv_len 0) in the
 * dense attention calls give zero output rows (a query with an empty key range, as every masked
 * row). The paged calls still refuse blocks holding no keys (flash_attn.rs:682), and negative
 * sizes are errors everywhere. */

/* Cache formats: the reference's kernel mode ids (candle-core/src/accel/formats.rs:41-48).
 * TURBO4 = TurboQuant MSE, Hadamard rotation (QuantFormat::TurboMse{bits}, cqkv_side.bits 1-4,
 * default 4); TURBOPROD = TurboQuant prod (QuantFormat::TurboProd{bits}, bits 2-5, default 4;
 * keys only): (bits - 1)-bit MSE codes of the rotated unit row, plus the sign bits of S r (r =
 * the residual of the unit row to its centroids, S = cqkv_qjl_matrix(D, seed)) and |r| - an
 * unbiased inner-product estimate (RowCodec::quantize_row, candle-core/src/accel/turbo.rs:
 * 299-323);
 * NVFP4 = E2M1 codes, an E4M3 scale per 16 elements and an f32 scale per token
 * (QuantFormat::Nvfp4); MXFP8 = E4M3 codes with an E8M0 scale per 32 elements
 * (QuantFormat::Mxfp8).
 * Plane layouts (per (batch, kv head), `capacity` tokens): codes are D bytes (8-bit formats) or
 * D/2 bytes (4-bit; TurboQuant codes of every width as nibbles) per token, keys row-major and values in
 * 8-token tiles; scales are the block-scale bytes of every token, then an f32 per token (FP8
 * scale, TurboQuant norm, NVFP4 global scale); TURBOPROD scales: the norms, then |r| (f32 per
 * token), then D/8 sign-bit bytes per token (bit i of word i / 32 = sign of (S r)_i >= 0). */
enum {
    CQKV_FMT_TURBO4 = 0,
    CQKV_FMT_TURBOPROD = 1,
    CQKV_FMT_MXFP4 = 2,
    CQKV_FMT_NVFP4 = 3,
    CQKV_FMT_MXFP8 = 4,
    CQKV_FMT_FP8 = 5
};

/* Element types of q / k / v / outputs. */
enum { CQKV_BF16 = 0, CQKV_F16 = 1, CQKV_F32 = 2 };

/* Rotary embedding layouts: rope (halves, element i pairs with i + D/2) and rope_i (interleaved,
 * element 2i pairs with 2i + 1) of candle-nn/src/rotary_emb.rs. */
enum { CQKV_ROPE_HALVES = 1, CQKV_ROPE_INTERLEAVED = 2 };

/* Rotation of the rows before quantization (RotationKind of candle-core/src/accel/config.rs:
 * 104-139, TurboQuantizer::rotate, candle-nn/src/turbo_quant.rs:182-189). Resolved for the head
 * dim D as RotationKind::resolve (config.rs:131-138):
 *   DEFAULT   the format's own: AUTO for the TurboQuant formats, NONE for the others;
 *   AUTO      HADAMARD when D is a power of two, else DENSE;
 *   HADAMARD  the sign-flipped Sylvester matrix / sqrt(D) of `seed` (rotation_matrix,
 *             candle-core/src/accel/turbo.rs:180-203); DENSE when D is not a power of two;
 *   DENSE     the seeded Gram-Schmidt orthogonal matrix of rotation_matrix (turbo.rs:204-230).
 * The cache stores codes of the rotated rows x Pi^T; decode rotates the queries with the key
 * rotation and unrotates the output with the value rotation. A HADAMARD side at D = 64, 128 or
 * 256 runs the in-register Walsh-Hadamard transform; every other rotating side multiplies by its
 * matrix cqkv_side.rot (f32, sums in index order). */
enum {
    CQKV_ROT_DEFAULT = 0,
    CQKV_ROT_NONE = 1,
    CQKV_ROT_HADAMARD = 2,
    CQKV_ROT_DENSE = 3,
    CQKV_ROT_AUTO = 4
};

/* One side (keys or values) of a quantized cache. */
typedef struct cqkv_side {
    int32_t format;    /* CQKV_FMT_* */
    int32_t is_value;  /* 0 keys (row-major codes), 1 values (8-token tiles) */
    int32_t head_dim;  /* D: 1-256 (the reference's fused attention takes D <= FA_MAX_HEAD_DIM =
                          256, candle-nn/src/turbo_quant.rs:1158); MXFP4 / MXFP8 a multiple of 32
                          and NVFP4 of 16 (QuantFormat::validate, formats.rs:166-187). Planes hold
                          rows of D' = 64, 128 or 256 elements (the smallest that holds D); the
                          elements past D are stored as zeros and never read into a result. */
    int32_t kv_heads;  /* Hkv */
    int32_t capacity;  /* tokens per plane, a multiple of 32 */
    int32_t rotation;  /* CQKV_ROT_* */
    int32_t bits;      /* TurboQuant width: TURBO4 = TurboMse{bits} 1-4, TURBOPROD = TurboProd{bits}
                          2-5 (QuantFormat bits, formats.rs:22-29); 0 = 4. The codes (bits, or
                          bits - 1 for TURBOPROD) are stored as nibbles at every width. 0 for the
                          other formats. */
    int32_t reserved;  /* 0 */
    uint64_t seed;     /* rotation seed (keys 42, values 44 by default); unused without rotation */
    void *codes;       /* device, batch * kv_heads planes of cqkv_codes_plane_bytes() */
    void *scales;      /* device, batch * kv_heads planes of cqkv_scales_plane_bytes() */
    const float *qjl;  /* TURBOPROD: device D x D f32 QJL matrix S (row-major, cqkv_qjl_matrix
                          of the side's seed); NULL for the other formats */
    const float *rot;  /* device D x D f32 rotation matrix Pi of the side (row-major,
                          cqkv_rotation_matrix(D, rotation, seed)): required when the rotation
                          resolves to DENSE, or to HADAMARD at a D other than 64, 128 and 256,
                          and by cqkv_dequantize_rows(unrotate) on any rotating side; may be
                          NULL otherwise (the reference's TurboQuantizer keeps Pi on the device
                          whenever it rotates, turbo_quant.rs:57-68) */
} cqkv_side;

/* The QJL projection S of TurboProd: D x D row-major f32 standard normals from SplitMix64 seeded
 * with (seed + 1) ^ 0x514a4c5f534b4554, Box-Muller in f64 (qjl_matrix,
 * candle-core/src/accel/turbo.rs:236-239). Host memory; upload it for cqkv_side.qjl. */
int cqkv_qjl_matrix(int32_t head_dim, uint64_t seed, float *out);

/* The rotation a side of `format` with rotation `kind` uses at head dim D (CQKV_ROT_NONE,
 * CQKV_ROT_HADAMARD or CQKV_ROT_DENSE; RotationKind::resolve, candle-core/src/accel/config.rs:
 * 131-138, with DEFAULT as the format's own), or -1 for an invalid kind / D. */
int32_t cqkv_resolve_rotation(int32_t format, int32_t kind, int32_t head_dim);

/* The D x D row-major f32 matrix Pi of rotation `kind` (resolved for D, DEFAULT as AUTO) and
 * `seed`: rotation_matrix (candle-core/src/accel/turbo.rs:180-233) - the identity, the seeded
 * sign-flipped Hadamard matrix / sqrt(D), or the Dense matrix: D x D standard normals of
 * SplitMix64(seed ^ 0x524f544154452121) (Box-Muller in f64), orthonormalised by two passes of
 * modified Gram-Schmidt in f64 (sums in index order), rounded to f32. Host memory; upload it for
 * cqkv_side.rot. D 1-1024. */
int cqkv_rotation_matrix(int32_t head_dim, int32_t kind, uint64_t seed, float *out);

/* Bytes of one (batch, head) plane of codes / scales; 0 for an invalid format or D. */
size_t cqkv_codes_plane_bytes(int32_t format, int32_t head_dim, int32_t capacity);
size_t cqkv_scales_plane_bytes(int32_t format, int32_t head_dim, int32_t capacity);

/* Quantize-and-append (RowCodec::quantize_row per (token, head) row, turbo.rs:293-381, then the
 * Cache::append copy): x is (batch, kv_heads, tokens, D) with element strides x_strides[0..2] for
 * batch, head and token (D contiguous), dtype CQKV_BF16 / F16 / F32. Token i of batch b lands at
 * position positions[b] + i (device int32 array of `batch`) or, when positions is NULL, at
 * `position` + i. Positions past the capacity are an error when positions is NULL and are
 * skipped otherwise (the device array is not read on the host). */
int cqkv_quant_append(const cqkv_side *side, const void *x, int32_t x_dtype,
                      const int64_t x_strides[3], int32_t batch, int32_t tokens,
                      const int32_t *positions, int32_t position, cqkv_stream_t stream);

/* Fused RoPE + quantize-append from the QKV projection output. q (batch, q_heads, tokens, D),
 * k / v (batch, kv_heads, tokens, D) with element strides *_strides[0..2] for batch, head, token
 * (D contiguous; q, k and v may be views into one (batch, tokens, (q_heads + 2 kv_heads) D)
 * projection output), all of `dtype`. cos / sin: (cs_rows, D/2) tables of `dtype`, row p = the
 * rotary angles of position p. Token i of batch b sits at position p = positions[b] + i (device
 * int32 array) or `position` + i: q is rotated with row p and written to q_out (strides
 * q_out_strides, `dtype`); k is rotated with row p, rounded to `dtype` as the reference's rope
 * output is, and quantized into k_side at cache position p; v is quantized into v_side as
 * cqkv_quant_append does. The sides must share D, heads and capacity; values of another format
 * than the keys are appended by a second launch on the stream. Positions past the
 * capacity (keys and values) or the tables (all three) are an error when positions is NULL and
 * are skipped otherwise. */
int cqkv_rope_quant_append(const cqkv_side *k_side, const cqkv_side *v_side, const void *q,
                           const int64_t q_strides[3], const void *k, const int64_t k_strides[3],
                           const void *v, const int64_t v_strides[3], int32_t dtype,
                           int32_t batch, int32_t tokens, int32_t q_heads, const void *cos,
                           const void *sin, int32_t cs_rows, int32_t rope_kind,
                           const int32_t *positions, int32_t position, void *q_out,
                           const int64_t q_out_strides[3], cqkv_stream_t stream);

/* Decode attention over a quantized cache (TqAttn + tq_combine, bottom-right aligned masks of
 * candle-core/src/accel/attention.rs:80-92):
 *   q   (batch, q_heads, q_len, D), element strides q_strides[0..2] for batch, head, query;
 *   out same shape, strides out_strides, dtype out_dtype;
 *   keys [0, kv_lens[b]) of plane b are attended (device int32 array; NULL: kv_len for all),
 *   kv_len = the largest length (host), used to size the launch;
 *   window_left / window_right: -1 = unbounded (causal = (-1, 0));
 *   softcap > 0: score = softcap * tanh(score / softcap) (0 disables it); alibi_slopes (device
 *   f32, NULL: none): score -= slope * |pos - key| with slope = alibi_slopes[b *
 *   alibi_batch_stride + head], stride 0 (slopes per head) or q_heads - the reference's
 *   tq_logit (candle-core/kernels/turbo_quant_impl.h:37-41) from FlashAttnConfig's softcap and
 *   alibi_slopes (TqAttnArgs, candle-core/src/accel/turbo.rs:506-530);
 *   q head h reads kv head h / (q_heads / kv_heads); any q_len (chunked prefill or speculative
 *   decode over the cache: the reference's grid (Lq * Hq / G, splits, B),
 *   candle-core/kernels/turbo_quant_impl.h:621-627).
 *   The key and value sides may differ in format; a side that rotates (CQKV_ROT_*) has the
 *   queries rotated with the key rotation and the output unrotated with the value rotation.
 * splits: key splits per (batch, kv head); 0 = automatic. workspace: device scratch of at least
 * cqkv_decode_workspace_bytes() for the split count used (it is used for more than one split,
 * for a rotating value side, for a key side that rotates by its matrix and for TURBOPROD keys
 * below a plane row length; it holds the partials, the rotated queries and the combined rows
 * before their unrotation); NULL = allocated (and freed) by the call. */
size_t cqkv_decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t q_len, int32_t head_dim,
                                   int32_t splits);
/* The key splits cqkv_decode_attention uses with splits = 0 for a cache of key / value formats
 * k_format / v_format, `batch` sequences, `kv_heads` heads and largest length kv_len, with
 * (ragged != 0) or without per-sequence lengths: size the workspace with it. */
int32_t cqkv_decode_splits(int32_t k_format, int32_t v_format, int32_t batch, int32_t kv_heads,
                           int32_t kv_len, int32_t ragged);
int cqkv_decode_attention(const void *q, int32_t q_dtype, const int64_t q_strides[3],
                          const cqkv_side *k, const cqkv_side *v, int32_t batch, int32_t q_heads,
                          int32_t q_len, const int32_t *kv_lens, int32_t kv_len,
                          float softmax_scale, int32_t window_left, int32_t window_right,
                          float softcap, const float *alibi_slopes, int32_t alibi_batch_stride,
                          void *out, int32_t out_dtype, const int64_t out_strides[3],
                          int32_t splits, void *workspace, size_t workspace_bytes,
                          cqkv_stream_t stream);

/* Allocation-free variant of cqkv_decode_attention. It has no counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results as cqkv_decode_attention
 * without the workspace; the split partials live in a library-owned device array of
 * CQKV_DECODE_SCRATCH_BYTES per GPU (held until the process ends; its address is looked up once
 * per device, with that device current). Automatic splits (splits = 0) are lowered until the
 * partials fit that array; an explicit split count whose partials do not fit is refused with
 * CQKV_ERR_WORKSPACE. Nothing is allocated or freed. Every call on one GPU shares that GPU's
 * array, and the array keeps the last call's partials: calls that overlap on one GPU (on
 * concurrent streams) race, so serialize them. */
#define CQKV_DECODE_SCRATCH_BYTES (32u << 20)
int cqkv_decode_attention_noalloc(const void *q, int32_t q_dtype, const int64_t q_strides[3],
                                  const cqkv_side *k, const cqkv_side *v, int32_t batch,
                                  int32_t q_heads, int32_t q_len, const int32_t *kv_lens,
                                  int32_t kv_len, float softmax_scale, int32_t window_left,
                                  int32_t window_right, float softcap, const float *alibi_slopes,
                                  int32_t alibi_batch_stride, void *out, int32_t out_dtype,
                                  const int64_t out_strides[3], int32_t splits,
                                  cqkv_stream_t stream);

/* One block of a paged cache (the reference's KvBlockRef, candle-nn/src/flash_attn.rs:609-613,
 * packed into a PageTable, candle-core/src/accel/attention.rs:307-366): a key side and a value
 * side holding `rows` valid tokens at the start of every (batch, kv head) plane. The keys of a
 * paged call are the blocks' valid rows concatenated in block order; masks are bottom-right
 * aligned over that concatenation. Every block has the formats, head dim, kv heads, rotations,
 * seeds (and TURBOPROD QJL matrix) of block 0; capacities may differ. */
typedef struct cqkv_kv_block {
    const cqkv_side *k;
    const cqkv_side *v;
    int32_t rows;
    int32_t reserved;
} cqkv_kv_block;

/* Device scratch a cqkv_decode_attention_paged call over these blocks needs (its block table and
 * split partials); 0 if the blocks or sizes are invalid. */
size_t cqkv_decode_paged_workspace_bytes(const cqkv_kv_block *blocks, int32_t n_blocks,
                                         int32_t batch, int32_t q_heads, int32_t q_len);
/* cqkv_decode_attention over the concatenated valid rows of n_blocks blocks, without copying
 * them (any number of blocks; the reference's kernel takes at most 128 and concatenates beyond).
 * Every sequence of the batch sees all the rows. Errors as the reference's check_blocks
 * (flash_attn.rs:650-686): no blocks, mismatched blocks, rows above a capacity, no keys. */
int cqkv_decode_attention_paged(const void *q, int32_t q_dtype, const int64_t q_strides[3],
                                const cqkv_kv_block *blocks, int32_t n_blocks, int32_t batch,
                                int32_t q_heads, int32_t q_len, float softmax_scale,
                                int32_t window_left, int32_t window_right, float softcap,
                                const float *alibi_slopes, int32_t alibi_batch_stride, void *out,
                                int32_t out_dtype, const int64_t out_strides[3], void *workspace,
                                size_t workspace_bytes, cqkv_stream_t stream);

/* Dense flash attention (FlashAttnOp / candle_flash_attn::flash_attn):
 *   q (batch, q_len, q_heads, D), k / v (batch, kv_len, kv_heads, D), out like q, all of
 *   `dtype` (CQKV_BF16, CQKV_F16 or CQKV_F32), element strides {batch, token, head} (D
 *   contiguous); head_dim any multiple of 8 up to 256 (the reference's FA_MAX_HEAD_DIM); any
 *   q_heads % kv_heads == 0; bottom-right aligned windows; causal = window (-1, 0).
 *   bf16 / f16 at head_dim 128 with more than 16 queries runs the MFMA prefill kernel; every
 *   other bf16 / f16 call runs the plain-dtype kernels over split-K: up to 16 (query, head)
 *   columns per kv head the row kernel (the reference's fa_row_* / fa_rowg_*,
 *   candle-core/kernels/flash_attn_impl.h:49-328), more the shared-tile kernel (its tile
 *   kernels, :330-443). K / V need 16-byte aligned rows (pointers and strides whole 8-element
 *   chunks). f32 runs the f32 kernels (f32 math on the f32 MFMA, as the reference's
 *   fa_row_f32_* / fa*_f32_*); their K / V need rows aligned to 4 elements (pointers and
 *   strides whole 4-element chunks), row strides below 2^24 elements.
 *   When k_cache / v_cache are non-NULL (a key and a value side of any formats and rotations)
 *   the same call also quantizes and appends k / v at positions [position, position + kv_len)
 *   of the cache: inside the MFMA prefill's pre-pass for unrotated FP8 sides at a position that
 *   is a multiple of 8, else as two cqkv_quant_append launches. Allocates its workspace. */
int cqkv_flash_attn(const void *q, const int64_t q_strides[3], const void *k,
                    const int64_t k_strides[3], const void *v, const int64_t v_strides[3],
                    void *out, const int64_t out_strides[3], int32_t dtype, int32_t batch,
                    int32_t q_len, int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                    int32_t head_dim, float softmax_scale, int32_t window_left,
                    int32_t window_right, const cqkv_side *k_cache, const cqkv_side *v_cache,
                    int32_t position, cqkv_stream_t stream);

/* Device workspace cqkv_flash_attn_ext needs for a call of these sizes (varlen != 0: per-sequence
 * lengths, q_len / kv_len their maxima; dtype is q's, the K / V dtype does not change it): the
 * MFMA prefill's V^T copy, or the plain kernel's split partials (0 when it does not split). */
size_t cqkv_flash_attn_workspace_bytes(int32_t dtype, int32_t batch, int32_t q_len,
                                       int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                                       int32_t head_dim, int32_t varlen);

/* cqkv_flash_attn plus mixed dtypes, the reference's optional score terms and variable-length
 * batches (fa_logit, candle-core/kernels/flash_attn_impl.h:42-47; fa_tile_impl :330-443):
 *   dtype is q's and out's, kv_dtype k's and v's: equal, or f32 queries over CQKV_F16 /
 *     CQKV_BF16 K / V (the reference's kv_dtype_supported, candle-core/src/accel/attention.rs:
 *     569-576; the K / V elements are widened exactly, then f32 math; E4M3 K / V go through
 *     cqkv_flash_attn_fp8). A cache append quantizes k / v from kv_dtype;
 *   softcap > 0: score = softcap * tanh(score / softcap) (0 disables it);
 *   alibi_slopes (device f32, NULL: none): score -= slope * |pos - key| with slope =
 *     alibi_slopes[b * alibi_batch_stride + head], stride 0 (slopes per head) or q_heads;
 *   cu_seqlens_q / cu_seqlens_k (device int32, batch + 1 prefix sums, NULL: dense): q / out are
 *     (total_q, q_heads, D) and k / v (total_k, kv_heads, D) with element strides
 *     {unused, token, head}; sequence b is rows cu[b] .. cu[b + 1] - 1; q_len / kv_len are the
 *     maximum sequence lengths. Offsets are clamped into the totals and lengths to the maxima.
 *     No cache append with variable-length batches.
 *   workspace: at least cqkv_flash_attn_workspace_bytes(); NULL = allocated (stream-ordered) and
 *     freed by the call.
 * Soft-capping precedes ALiBi, and masked keys stay masked, as in the reference. */
int cqkv_flash_attn_ext(const void *q, const int64_t q_strides[3], const void *k,
                        const int64_t k_strides[3], const void *v, const int64_t v_strides[3],
                        void *out, const int64_t out_strides[3], int32_t dtype, int32_t kv_dtype,
                        int32_t batch, int32_t q_len, int32_t kv_len, int32_t q_heads,
                        int32_t kv_heads, int32_t head_dim, float softmax_scale, int32_t window_left,
                        int32_t window_right, float softcap, const float *alibi_slopes,
                        int32_t alibi_batch_stride, const int32_t *cu_seqlens_q,
                        const int32_t *cu_seqlens_k, int32_t total_q, int32_t total_k,
                        const cqkv_side *k_cache, const cqkv_side *v_cache, int32_t position,
                        void *workspace, size_t workspace_bytes, cqkv_stream_t stream);

/* One block of plain K / V for cqkv_flash_attn_blocks (the reference's KvBlockRef over dense
 * tensors, candle-nn/src/flash_attn.rs:609-613): k / v of layout (batch, kv_heads, capacity, D)
 * with element strides {batch, head, row} (D contiguous) and `rows` valid rows. */
typedef struct cqkv_plain_block {
    const void *k, *v;
    int64_t k_strides[3], v_strides[3];
    int32_t rows;
    int32_t reserved;
} cqkv_plain_block;

/* flash_attn_blocks (candle-nn/src/flash_attn.rs:719-765, the paged row kernel fa_rowp_* of
 * RocmStorage::flash_attn_paged): attention of q (batch, q_heads, q_len, D), element strides
 * {batch, head, query}, over the concatenated valid rows of n_blocks blocks without copying them
 * (any number of blocks; the reference's kernel takes at most 128 and concatenates beyond);
 * every sequence sees all the rows; masks, soft-capping and ALiBi bottom-right aligned over
 * them. q / out of `dtype`, K / V of `kv_dtype`, the pairs of cqkv_flash_attn_ext (bf16 / bf16,
 * f16 / f16, f32 / f32, f32 / f16, f32 / bf16), K / V rows aligned as there with one row stride
 * per side across the blocks. out like q (strides {batch, head, query}). Errors as the
 * reference's check_blocks (flash_attn.rs:650-686). The workspace does not depend on the
 * dtypes. */
size_t cqkv_flash_attn_blocks_workspace_bytes(const cqkv_plain_block *blocks, int32_t n_blocks,
                                              int32_t batch, int32_t q_heads, int32_t q_len,
                                              int32_t kv_heads, int32_t head_dim);
int cqkv_flash_attn_blocks(const void *q, const int64_t q_strides[3],
                           const cqkv_plain_block *blocks, int32_t n_blocks, int32_t dtype,
                           int32_t kv_dtype, int32_t batch, int32_t q_heads, int32_t q_len,
                           int32_t kv_heads,
                           int32_t head_dim, float softmax_scale, int32_t window_left,
                           int32_t window_right, float softcap, const float *alibi_slopes,
                           int32_t alibi_batch_stride, void *out, const int64_t out_strides[3],
                           void *workspace, size_t workspace_bytes, cqkv_stream_t stream);

/* Per-tensor FP8 quantization (flash_attn_fp8, candle-nn/src/flash_attn.rs:882-887): over the n
 * elements of x (dtype CQKV_BF16 / F16 / F32, contiguous), amax = max |x|, scale = amax > 0 ?
 * amax / 448 : 1, codes[i] = E4M3(x[i] * f32(1 / f64(scale)) + 0) (candle's `x / scale`).
 * scale: device float[2]; scale[0] receives the scale, scale[1] is scratch. Asynchronous. */
int cqkv_fp8_quantize_tensor(const void *x, int32_t x_dtype, int64_t n, uint8_t *codes,
                             float *scale, cqkv_stream_t stream);

/* Attention over E4M3 K / V with descale factors (flash_attn_with_config on F8E4M3 tensors):
 * shapes, strides, head dims and masks as cqkv_flash_attn (q, out of `dtype`, bf16, f16 or f32;
 * k8 / v8 E4M3 bytes, strides multiples of 8, 8-byte aligned). Keys are e4m3(k8) * k_descale *
 * (k_scale ? *k_scale : 1), values likewise with v_descale / v_scale (device floats, e.g. the
 * scales written by cqkv_fp8_quantize_tensor, read on the device). bf16 / f16: the codes are
 * converted to the dtype (exactly) into the workspace, then the attention runs with the descales
 * folded into the query scale and the output normalisation. f32 (the reference's
 * fa_row_f32_fp8): the f32 kernels read the codes directly, widen them exactly and compute in
 * f32, the descales folded the same way. workspace: at least
 * cqkv_flash_attn_fp8_workspace_bytes(); NULL = allocated (stream-ordered) and freed by the call. */
size_t cqkv_flash_attn_fp8_workspace_bytes(int32_t dtype, int32_t batch, int32_t q_len,
                                           int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                                           int32_t head_dim);
int cqkv_flash_attn_fp8(const void *q, const int64_t q_strides[3], const void *k8,
                        const int64_t k_strides[3], const void *v8, const int64_t v_strides[3],
                        void *out, const int64_t out_strides[3], int32_t dtype, int32_t batch,
                        int32_t q_len, int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, float softmax_scale, int32_t window_left,
                        int32_t window_right, float k_descale, float v_descale,
                        const float *k_scale, const float *v_scale, void *workspace,
                        size_t workspace_bytes, cqkv_stream_t stream);

/* Hadamard rotation of rows (flash_attn_fp8's incoherent processing, candle-nn/src/flash_attn.rs:
 * 868-880): out_r = x_r * rotation_matrix(D, Hadamard, seed)^T for each of `rows` rows of D
 * contiguous elements (row strides in elements), computed in f32 and rounded to `dtype`
 * (CQKV_BF16 / F16 / F32). D a power of two from 2 to 256 (the reference rotates power-of-two
 * head dims only). The matrix is the sign-flipped Sylvester Hadamard matrix / sqrt(D) of
 * candle-core/src/accel/turbo.rs:180-203. */
int cqkv_hadamard_rows(const void *x, int32_t dtype, int64_t rows, int64_t x_row_stride,
                       int32_t head_dim, uint64_t seed, void *out, int64_t out_row_stride,
                       cqkv_stream_t stream);

/* Reference row layout interop (candle-core/src/accel/formats.rs:206-242): rows are
 * (batch, kv_heads, tokens, row_words) u32 on the device, row_words = code + aux + 2 words
 * (TurboQuant codes packed at their width, LSB first). `bits` as cqkv_side.bits (0 for the
 * formats without a width). import: rows -> cache positions [position, position + tokens);
 * export: the reverse. */
int32_t cqkv_reference_row_words(int32_t format, int32_t bits, int32_t head_dim);
int cqkv_rows_import(const cqkv_side *side, const uint32_t *rows, int32_t batch, int32_t tokens,
                     int32_t position, cqkv_stream_t stream);
int cqkv_rows_export(const cqkv_side *side, uint32_t *rows, int32_t batch, int32_t tokens,
                     int32_t position, cqkv_stream_t stream);

/* Dequantization of cache rows (TqDequant + TurboQuantizer::dequantize_rows, the device half of
 * TurboKvCache::keys_values: candle-core/src/rocm_backend/accel.rs:380-419,
 * candle-nn/src/turbo_quant.rs:250-300, 612-689, 948-966): positions [position, position +
 * tokens) of every (batch, kv head) plane are written to out (batch, kv_heads, tokens, D) with
 * element strides out_strides {batch, head, token} (D contiguous) in out_dtype (CQKV_BF16 / F16 /
 * F32, rounded to nearest even from f32). Each element is rsc0 * element_j of
 * RowCodec::dequantize_row (candle-core/src/accel/turbo.rs:398-424) in f32 - the FP8 scale times
 * the E4M3 value, E2M1 times its E8M0 / E4M3 block scale (NVFP4: then times the token's scale),
 * the centroid times the norm - plus, for TURBOPROD keys, the QJL correction
 * sum_i z_i S[i][j] with z_i = +-rsc0 rsc1 sqrt(pi/2) / D (sums in index order). unrotate != 0
 * then multiplies the rows by the side's Pi (y Pi, TurboQuantizer::unrotate, sums in index order;
 * needs cqkv_side.rot when the side rotates), giving the unrotated values keys_values returns
 * before its dtype cast. Positions past the capacity are an error. workspace: device scratch of
 * at least cqkv_dequantize_workspace_bytes() (non-zero only for TURBOPROD or unrotate on a
 * rotating side); NULL = allocated (stream-ordered) and freed by the call. */
size_t cqkv_dequantize_workspace_bytes(const cqkv_side *side, int32_t batch, int32_t tokens,
                                       int32_t unrotate);
int cqkv_dequantize_rows(const cqkv_side *side, int32_t batch, int32_t position, int32_t tokens,
                         int32_t unrotate, void *out, int32_t out_dtype,
                         const int64_t out_strides[3], void *workspace, size_t workspace_bytes,
                         cqkv_stream_t stream);

/* Cache growth (the copy of Cache::append into a grown buffer, candle-nn/src/kv_cache.rs:56-99):
 * the first `tokens` positions of every (batch, kv head) plane of src are copied into dst, a side
 * of the same format, kind, head dim, kv heads and rotation (and seed, when it rotates) whose
 * capacity may differ (at least `tokens`). Value sides copy whole 8-token tiles. Strided device copies on `stream`; no kernel,
 * nothing allocated. The caller allocates dst (e.g. at the reference's grown capacity
 * cap += max(grow_by, cap / 2) until it holds the new length, rounded up to 32). */
int cqkv_side_copy(const cqkv_side *dst, const cqkv_side *src, int32_t batch, int32_t tokens,
                   cqkv_stream_t stream);

/* TurboQuant tables the kernels use (host): the Lloyd-Max codebook of TurboMse{bits} at head
 * dim D (candle-core/src/accel/turbo.rs:58-129; 2^bits centroids, 2^bits - 1 boundaries) and
 * the Hadamard sign vector of `seed` (turbo.rs:188-203; +1 / -1 per column). */
int cqkv_turbo_codebook(int32_t head_dim, int32_t bits, float *centroids, float *boundaries);
int cqkv_turbo_signs(int32_t head_dim, uint64_t seed, float *signs);

/* Message of the last failed call on this thread ("" if none). */
const char *cqkv_last_error(void);
/* Library version string, e.g. "cqkv 0.1 gfx950". */
const char *cqkv_version(void);

#ifdef __cplusplus
}
#endif
#endif
