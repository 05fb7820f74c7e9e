// TurboQuant (TurboMse) append of bf16 / f16 rows with the rotation on MFMA
// (RowCodec::quantize_row, candle-core/src/accel/turbo.rs:299-323, after TurboQuantizer::rotate,
// candle-nn/src/turbo_quant.rs:182-189, then Cache::append, candle-nn/src/kv_cache.rs:68-99).
//
// The row-parallel encoder of append_rows.h spends most of its VALU issue on the sign flip, the
// seven Walsh-Hadamard stages and a three-step codebook search per element. Here:
//  * y = x diag(s) H^T (unscaled) is two MFMA products per 16 rows, one per half of the row
//    (H = H_2 (x) H_{D/2}: y = (u + v, u - v) with u, v the halves' H_{D/2} transforms, added
//    and subtracted in f32 by the lane that holds both): the rows are the A operand as they
//    arrive (16-byte loads of bf16 / f16, no conversion), B is the +-1 matrix
//    B_h[k][c] = s_{h D/2 + k} H_{D/2}[pi(c)][k] (exact in bf16 / f16, so every product is
//    exact), built once per workgroup in LDS and read from there by each product. The output
//    columns are permuted, pi(16 nb + n) = (D / 32) n + nb, so that lane (n, g) ends with D / 32
//    consecutive columns of each half for rows 4 g .. 4 g + 3. (The whole D x D matrix took
//    twice the products: keys 39 -> 36 us, values 51 -> 47 us per config-2-shape call.)
//  * One workgroup of 16 wavefronts per CU shares B and the table: 32 KB of B per wavefront in
//    registers would have allowed two wavefronts per SIMD, and B per 4-wavefront workgroup would
//    have limited the CU to two workgroups by LDS. With B shared the kernel runs four wavefronts
//    per SIMD, each with the next chunk's rows in flight (measured at D = 128, keys: 51 -> 43 us
//    per call against B in registers).
//  * The norm of each row is a 16-lane DPP sum; 1 / sqrt(D) goes into the stored norm only (u is
//    scale-free). The square root and reciprocal are the hardware's (1 ulp), which moves a code
//    only for an element within about an ulp of a boundary, inside the TurboQuant criterion.
//  * The codebook index #{boundaries <= u} (Codebook::index, turbo.rs:40-44) is a table lookup:
//    bin j = trunc(S u) (S a power of two, so S u is exact) holds the count of the boundaries
//    below the bin and the one boundary inside it (S is chosen so that no bin holds two); the
//    index is that count plus one exact compare. The table is replicated per lane of a 32-lane
//    half in LDS, so the lookups do not conflict on banks.
// Rows whose norm or 1 / norm is not finite take the plain count, as in rows_block.
#include <algorithm>
#include <cstring>

#include "append_rows.h"

namespace cqkv {

constexpr int kLutMaxS = 64;
constexpr int kLutN = 2 * kLutMaxS + 1;
constexpr int kLutCopies = 32;

struct TurboMfmaArgs {
    AppendArgs a;
    int32_t lut_s;            // S
    int32_t chunks_per_plane;  // ROWS-token blocks of one (batch, head) plane
    int32_t total_chunks;
    float lut_b[kLutN];     // the boundary inside bin j (index j + S), times S; +inf if none
    uint32_t lut_c[kLutN];  // #{boundaries below bin j}
};

// Sum over the 16 lanes sharing lane / 16 (quad xor 1, quad xor 2, half-row mirror, row mirror).
__device__ inline float sum16(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));
    return v;
}

// A chunk: 16 rows per wavefront (one MFMA row group), loaded while the previous chunk computes.
constexpr int kTqThreads = 1024;  // 16 wavefronts
constexpr int kTqRows = 16 * (kTqThreads / 64);

template <bool F16>
using tq_op_t = typename std::conditional<F16, f16x8, bf16x8>::type;

// The cache position range of one chunk (ROWS tokens from c0 = the first value tile of the
// append + bx ROWS); valid false when the chunk writes nothing.
struct TqChunk {
    int b, h, pos, c0, end;
    bool valid;
};
// pos0: a.position, read once into a register (a select between it and a.positions[b] as
// memory reads became one flat load, waited for before the chunk's row loads could issue).
template <int ROWS, typename Args>
__device__ inline TqChunk tq_chunk(const Args &p, int ck, int pos0) {
    const AppendArgs &a = p.a;
    TqChunk c = {};
    if (ck >= p.total_chunks) return c;  // valid false: past the last chunk
    const int bx = ck % p.chunks_per_plane, plane = ck / p.chunks_per_plane;
    c.h = plane % a.kv_heads;
    c.b = plane / a.kv_heads;
    c.pos = pos0;
    if (a.positions) c.pos = a.positions[c.b];
    c.c0 = c.pos / 8 * 8 + bx * ROWS;
    c.end = min(c.pos + a.tokens, a.capacity);
    if (a.cs_rows > 0) c.end = min(c.end, a.cs_rows);
    c.valid = c.pos >= 0 && c.c0 < c.end;
    return c;
}

// This lane's A operands of 16-row group grp of a chunk: row (group row n), head dims
// 32 ks + 8 g .. + 7; rows outside [pos, end) read zeros. Buffer loads from the chunk's first
// row (its position c0 may precede the first appended row: only rows in [pos, end) are read),
// with dead rows pointed past the range, so that the loads are unconditional: the compiler can
// then count them, and wait for them without also waiting for the stores issued after them.
constexpr uint32_t kTqOOB = 0x80000000u;
template <int D, int ROWS>
__device__ inline void tq_load(const AppendArgs &a, const TqChunk &c, int grp, int n, int g,
                               u32x4 (&av)[D / 32]) {
    const int t = c.c0 + 16 * grp + n;
    const bool live = c.valid && t >= c.pos && t < c.end;
    const uint16_t *base = (const uint16_t *)a.x + (int64_t)c.b * a.sb + (int64_t)c.h * a.sh +
                           (int64_t)(c.c0 - c.pos) * a.st;
    const rsrc_t r = make_rsrc(base, kTqOOB);
    const uint32_t off = live ? (uint32_t)((int64_t)(t - c.c0) * a.st * 2 + 16 * g) : kTqOOB;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) av[ks] = ld128(r, off + 64 * ks);
}

template <int IS_VALUE, int D, bool F16>
__global__ __launch_bounds__(kTqThreads) void turbo_mfma_kernel(TurboMfmaArgs p) {
    constexpr int NW = kTqThreads / 64;
    // NBH column blocks and KSH k-steps per half of the row (the H_2 (x) H_{D/2} split)
    constexpr int NB = D / 16, KS = D / 32, NBH = NB / 2, KSH = KS / 2;
    constexpr int ROWS = kTqRows, GPW = ROWS / (16 * NW);
    constexpr int kRowBytes = D / 2;
    using op_t = tq_op_t<F16>;
    __shared__ __attribute__((aligned(16))) u32x4 sm_b[2 * NBH * KSH * 64];
    __shared__ __attribute__((aligned(16))) u32x2 sm_lut[kLutN * kLutCopies];
    // values: the chunk's codes, double-buffered (chunk parity) so that one barrier per chunk
    // separates their writes from the tile writer's reads
    __shared__ __attribute__((aligned(16))) uint8_t sm_codes_buf[IS_VALUE ? 2 * ROWS * kRowBytes : 16];
    const AppendArgs &a = p.a;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;

    // ---- once per workgroup: B (as [half][nb][ks][lane] operands) and the replicated table;
    // every read of the kernel arguments here has a workgroup-uniform index (scalar loads) ----
    // The Sylvester matrix is H_2 (x) H_{D/2} (the top index bit): with u = H_{D/2} (s x)[first
    // half] and v = H_{D/2} (s x)[second half], y = (u + v, u - v). The products take the two
    // halves' B_h[k][c] = s_{h D/2 + k} H_{D/2}[pi(c)][k], pi(16 nb + n) = NBH n + nb, half the
    // products of the whole matrix; each lane then adds and subtracts its own u and v.
    const uint32_t sgn[4] = {a.sign_bits[0], a.sign_bits[1], a.sign_bits[2], a.sign_bits[3]};
#pragma unroll
    for (int it = 0; it < (2 * NBH * KSH * 64 + kTqThreads - 1) / kTqThreads; ++it) {
        const int i = tid + kTqThreads * it;
        if (i >= 2 * NBH * KSH * 64) break;
        const int l = i & 63, ks = (i >> 6) % KSH, nb = ((i >> 6) / KSH) % NBH;
        const int half = (i >> 6) / (KSH * NBH);
        const int col = NBH * (l & 15) + nb;
        const uint32_t one = F16 ? 0x3C00u : 0x3F80u;
        const int kw = half * KSH + ks;  // sign word of the row's elements 32 kw ..
        const uint32_t sw = kw == 0 ? sgn[0] : kw == 1 ? sgn[1] : kw == 2 ? sgn[2] : sgn[3];
        uint32_t w[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            uint32_t v = 0;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int k = 32 * ks + 8 * (l >> 4) + 2 * e2 + h2;  // index in the half
                const uint32_t par = ((uint32_t)__popc(col & k) + (sw >> (k & 31))) & 1u;
                v |= (one | (par << 15)) << (16 * h2);
            }
            w[e2] = v;
        }
        sm_b[i] = u32x4{w[0], w[1], w[2], w[3]};
    }
    const int S = p.lut_s;
    // wavefront w copies entries 2 w, 2 w + 1, then 2 w + 2 NW, ...: lanes 0..31 write the 32
    // copies of the first, lanes 32..63 those of the second
#pragma unroll 4
    for (int e0 = 2 * wave; e0 <= 2 * S; e0 += 2 * NW) {
        const u32x2 lo = u32x2{__float_as_uint(p.lut_b[e0]), p.lut_c[e0]};
        const u32x2 hi = e0 + 1 <= 2 * S ? u32x2{__float_as_uint(p.lut_b[e0 + 1]), p.lut_c[e0 + 1]}
                                         : u32x2{0u, 0u};
        if (lane < 32) sm_lut[e0 * kLutCopies + lane] = lo;
        else if (e0 + 1 <= 2 * S) sm_lut[(e0 + 1) * kLutCopies + lane - 32] = hi;
    }
    __syncthreads();
    // this lane's copy of the entry of bin 0 (bin j is entry j + S)
    const u32x2 *lut0 = sm_lut + S * kLutCopies + (lane & 31);

    // ---- the chunks of this workgroup; the next chunk's rows load while this one computes ----
    // The rows are loaded in one place only, into nv, and copied to av at the top of the next
    // iteration, before that iteration issues its own loads; the first iteration (ck < 0) only
    // loads. (Loads into av before the loop made the compiler's wait for av at the first product
    // also wait for the prefetch issued in the loop, serialising every load with the compute.)
    // Chunk descriptors are formed one iteration ahead of their loads (nn), so that a per-batch
    // position read is waited for together with the rows, not before them.
    const int pos0 = a.position;
    TqChunk nxt = {}, nn = tq_chunk<ROWS>(p, blockIdx.x, pos0);
    u32x4 av[GPW][KS], nv[GPW][KS] = {};
    for (int ck = (int)blockIdx.x - (int)gridDim.x; ck < p.total_chunks; ck += gridDim.x) {
        const TqChunk cur = nxt;
#pragma unroll
        for (int grp = 0; grp < GPW; ++grp)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) av[grp][ks] = nv[grp][ks];
        nxt = nn;
        nn = tq_chunk<ROWS>(p, ck + 2 * (int)gridDim.x, pos0);
#pragma unroll
        for (int grp = 0; grp < GPW; ++grp) tq_load<D, ROWS>(a, nxt, wave * GPW + grp, n, g, nv[grp]);
        uint8_t *sm_codes = sm_codes_buf + (IS_VALUE ? (((ck - (int)blockIdx.x) / (int)gridDim.x) & 1) * ROWS * kRowBytes : 0);
        // Every iteration computes, also for a chunk that writes nothing (the first iteration,
        // chunks past the end): its rows are dead and its stores dropped. With a branch around
        // the compute, the compiler's wait for nv at the top of the iteration counted on the
        // path without stores and so waited for the stores of the previous chunk as well.
        {
            // B is re-read from LDS by each product: an index the compiler cannot see through
            // keeps it from hoisting the 32 operands out of the loop (and spilling them)
            int bl = lane;
            asm volatile("" : "+v"(bl));
            const u32x4 *bsm = sm_b + bl;
            const int64_t plane = (int64_t)cur.b * a.kv_heads + cur.h;
            uint8_t *codes = a.codes + plane * a.codes_plane;
            // (buffer stores, dead rows past the range: unconditional, as the loads)
            const rsrc_t code_r = make_rsrc(codes, kTqOOB);
            const rsrc_t norm_r = make_rsrc(a.scales + plane * a.scales_plane, kTqOOB);
#pragma unroll
            for (int grp = 0; grp < GPW; ++grp) {
                const int r0 = 16 * (wave * GPW + grp);  // the group's first row in the chunk
                // u (acc[0 .. NBH)) and v (acc[NBH ..)), ks-major: consecutive products update
                // different accumulators
                f32x4 acc[NB];
#pragma unroll
                for (int ks = 0; ks < KSH; ++ks)
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        const int half = j / NBH, nb = j % NBH;
                        acc[j] = mfma16x16x32(
                            __builtin_bit_cast(op_t, av[grp][half * KSH + ks]),
                            __builtin_bit_cast(op_t, bsm[((half * NBH + nb) * KSH + ks) * 64]),
                            ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[j]);
                    }
#pragma unroll
                for (int nb = 0; nb < NBH; ++nb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float uu = acc[nb][i], vv = acc[NBH + nb][i];
                        acc[nb][i] = uu + vv;
                        acc[NBH + nb][i] = uu - vv;
                    }
                // lane (n, g): rows r0 + 4 g + i, columns h D / 2 + NBH n + nb in acc[h NBH + nb]
                // (h the half). Row norms by the hardware square root and reciprocal (1 ulp; the
                // rotation itself already leaves the reference's last bits unpinned).
                float norm[4], inv[4], w[4];
                bool fin = true;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float ss = 0.0f;
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) ss = __builtin_fmaf(acc[nb][i], acc[nb][i], ss);
                    norm[i] = __builtin_amdgcn_sqrtf(sum16(ss));
                    inv[i] = norm[i] > 0.0f ? __builtin_amdgcn_rcpf(norm[i]) : 0.0f;
                    w[i] = (float)S * inv[i];
                    fin = fin && norm[i] <= 3.0e38f && w[i] <= 3.0e38f;
                }
                uint32_t word[4];
                if (__all(fin)) {
                    // |u| <= 1 (+ rounding): S u truncates into [-S, S], the table's range
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        word[i] = 0;
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const float us = acc[nb][i] * w[i];
                            const u32x2 ent = lut0[(int)us * kLutCopies];
                            word[i] |= (ent.y + (us >= __uint_as_float(ent.x) ? 1u : 0u)) << (4 * nb);
                        }
                    }
                } else {  // the plain count (NaN -> 0, infinities)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        word[i] = 0;
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const float u = acc[nb][i] * inv[i];
                            uint32_t k = 0;
#pragma unroll
                            for (int kk = 0; kk < 15; ++kk) k += u >= a.bnd[kk] ? 1u : 0u;
                            word[i] |= k << (4 * nb);
                        }
                    }
                }
                const int rg = r0 + 4 * g, tg = cur.c0 + rg;  // this lane's first row
                {
                    // one store of the group's 16 norms: lane (n < 4, g) writes row 4 g + n's
                    // (every lane of a 16-lane row holds all four of its rows' norms)
                    const float nm = n == 0 ? norm[0] : n == 1 ? norm[1] : n == 2 ? norm[2] : norm[3];
                    const bool live = n < 4 && tg + n >= cur.pos && tg + n < cur.end;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(nm * a.rot_scale), norm_r,
                                                          live ? (uint32_t)(tg + n) * 4u : kTqOOB,
                                                          0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool live = tg + i >= cur.pos && tg + i < cur.end;
                    // the NBH codes of each half: bytes (NBH / 2) n of the first and the second
                    // half of the row's codes
                    const uint32_t lo = word[i] & ((1u << (4 * NBH)) - 1u), hi = word[i] >> (4 * NBH);
                    if constexpr (IS_VALUE != 0) {
                        uint8_t *dst = sm_codes + (rg + i) * kRowBytes + (NBH / 2) * n;
                        if constexpr (NBH == 4) {
                            *(uint16_t *)dst = (uint16_t)lo;
                            *(uint16_t *)(dst + kRowBytes / 2) = (uint16_t)hi;
                        } else {
                            dst[0] = (uint8_t)lo;
                            dst[kRowBytes / 2] = (uint8_t)hi;
                        }
                    } else {
                        const uint32_t off =
                            live ? (uint32_t)(tg + i) * kRowBytes + (NBH / 2) * n : kTqOOB;
                        const uint32_t off2 = live ? off + kRowBytes / 2 : kTqOOB;
                        if constexpr (NBH == 4) {
                            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)lo, code_r, off, 0, 0);
                            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)hi, code_r, off2, 0, 0);
                        } else {
                            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)lo, code_r, off, 0, 0);
                            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)hi, code_r, off2, 0, 0);
                        }
                    }
                }
            }
            if constexpr (IS_VALUE != 0) {
                __syncthreads();
                // (the next chunk writes the other buffer; the one after it this buffer again,
                // behind the next chunk's barrier)
                write_value_tiles<false, D, ROWS, kTqThreads>(codes, sm_codes, cur.c0, cur.pos, cur.end, tid);
            }
        }
    }
}

// The bin table of a sorted boundary list (+inf entries unused) at scale S: bin j (index j + S)
// covers S u in [j, j + 1) for j > 0, (-1, 1) for j = 0 and (j - 1, j] for j < 0 (the
// truncation of S u); count = #{boundaries below the bin}, inner = the boundary inside it.
// False when a bin holds two boundaries.
static bool tq_build_lut(const float bnd[16], int S, TurboMfmaArgs &p) {
    p.lut_s = S;
    for (int j = -S; j <= S; ++j) {
        // below: b <= j (j > 0) or b <= j - 1 (j <= 0); inside: b < j + 1 (j > 0), b < 1 (j = 0),
        // b <= j (j < 0)
        const double lo = j > 0 ? j : j - 1;
        int below = 0, inner = 0;
        float in = __builtin_inff();
        for (int k = 0; k < 15; ++k) {
            if (!(bnd[k] < __builtin_inff())) continue;
            const double b = (double)bnd[k] * S;  // exact: S is a power of two
            const bool inside = j > 0 ? b < j + 1 : j == 0 ? b < 1 : b <= j;
            if (b <= lo) {
                ++below;
            } else if (inside) {
                ++inner;
                in = (float)b;
            }
        }
        if (inner > 1) return false;
        p.lut_b[j + S] = in;
        p.lut_c[j + S] = (uint32_t)below;
    }
    return true;
}

template <int IS_VALUE, int D>
static void tq_launch_d(bool f16, dim3 grid, hipStream_t st, const TurboMfmaArgs &p) {
    if (f16) hipLaunchKernelGGL((turbo_mfma_kernel<IS_VALUE, D, true>), grid, dim3(kTqThreads), 0, st, p);
    else hipLaunchKernelGGL((turbo_mfma_kernel<IS_VALUE, D, false>), grid, dim3(kTqThreads), 0, st, p);
}

// Launches the MFMA form for a TurboMse side appended from 16-byte aligned bf16 / f16 rows with
// the Hadamard rotation; false (nothing launched) for any other case.
bool turbo_mfma_launch(const cqkv_side *s, int32_t tokens, int32_t batch, hipStream_t st,
                       const AppendArgs &a) {
    if (s->format != CQKV_FMT_TURBO4 || !a.rotate) return false;
    if (a.row_loads != kRowBF16 && a.row_loads != kRowF16) return false;
    const int d = s->head_dim;
    if (d != 64 && d != 128) return false;
    // 31-bit buffer offsets: rows of a chunk from its first row, codes and norms of a plane
    if (a.st < 0 || (int64_t)kTqRows * a.st * 2 + 2 * d >= kTqOOB ||
        (int64_t)s->capacity * (d / 2) >= kTqOOB)
        return false;
    TurboMfmaArgs p = {};
    p.a = a;
    bool ok = false;
    for (int S = 8; S <= kLutMaxS && !ok; S *= 2) ok = tq_build_lut(a.bnd, S, p);
    if (!ok) return false;
    // chunks start at the value tile of the first position: with one position for every batch
    // entry its offset in the tile is known here (no chunk that writes nothing)
    const int lead = !a.positions && a.position >= 0 ? a.position % 8 : 7;
    p.chunks_per_plane = (int)(((int64_t)tokens + lead + kTqRows - 1) / kTqRows);
    const int64_t total = (int64_t)p.chunks_per_plane * s->kv_heads * batch;
    if (total <= 0 || total > 0x7fffffff) return false;
    p.total_chunks = (int32_t)total;
    // 256 CUs; at D = 64 (half the registers and LDS) two workgroups fit on a CU
    const dim3 grid((unsigned)std::min<int64_t>(total, d == 64 ? 512 : 256));
    const bool f16 = a.row_loads == kRowF16;
    if (s->is_value) {
        if (d == 128) tq_launch_d<1, 128>(f16, grid, st, p);
        else tq_launch_d<1, 64>(f16, grid, st, p);
    } else {
        if (d == 128) tq_launch_d<0, 128>(f16, grid, st, p);
        else tq_launch_d<0, 64>(f16, grid, st, p);
    }
    return true;
}

// ---------------------------------------------------------------------------------------------
// TurboProd keys (RowCodec::quantize_row, candle-core/src/accel/turbo.rs:299-323): the MSE codes
// of the rotated unit row u = y / |y| in the (bits - 1)-bit codebook, the residual
// r = u - centroid[code], |r|, and the sign bits of p = S r (S the D x D QJL matrix).
//
// The rows enter as the B operand of v_mfma_f32_32x32x16 (32 tokens per wavefront), so the
// products leave each lane with one token:
//  * rotation: U_h^T = A_h X_h^T per half h of the row (the H_2 (x) H_{D/2} split of the
//    turbo_mfma_kernel), A_h[f][k] = s_{h D/2 + k} H_{D/2}[f][k] with the feature rows permuted
//    so that lane (token n, half l) receives features (D/4) l + q, q < D/4, of u and v; then
//    y = (u + v, u - v) gives the lane the features (D/4) l + q and D/2 + (D/4) l + q: two
//    contiguous runs of D/4 codes (one 16- or 8-byte store each);
//  * norm and |r|: lane sums plus the partner lane l ^ 32 (v_permlane32_swap);
//  * codes by the bin table of the TurboMse kernel, centroids from a per-lane LDS copy;
//  * S r: P^T = S' R^T with R^T straight from the registers (B operand of k-step c = the lane's
//    residuals 8 c .. 8 c + 7, in the order of its two runs), S' = S with its columns in that
//    order and its output rows permuted so that lane l receives outputs (D/2) l .. + D/2 - 1
//    (one store of D/2 sign bits). The residual is scaled by 64 (exact) and split into f16
//    hi + lo, S likewise: p = S_hi r_hi + S_hi r_lo + S_lo r_hi on the f16 MFMA (products
//    exact, f32 sums; the dropped S_lo r_lo is 2^-22 of a term), as in the row-parallel form.
// S' (hi and lo) and the rotation operands are built once per workgroup in LDS.
constexpr int kPqThreads = 512;  // 8 wavefronts, two per SIMD (at most 256 VGPRs)
constexpr int kPqTok = 32;       // tokens per chunk: one wavefront's
typedef float pq_f32x16 __attribute__((ext_vector_type(16)));

__device__ inline pq_f32x16 pq_mfma(f16x8 a, f16x8 b, pq_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ inline pq_f32x16 pq_mfma(bf16x8 a, bf16x8 b, pq_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// the 32x32 MFMA output / operand row m = 8 j + 4 hm + i as (j, hm, i)
__device__ inline int pq_perm(int m, int quarter, int blk) {
    // row m of output block blk -> index quarter * hm + 16 blk + 4 j + i
    return quarter * ((m >> 2) & 1) + 16 * blk + 4 * (m >> 3) + (m & 3);
}

template <int D, bool F16>
__global__ __launch_bounds__(kPqThreads) void prod_mfma_kernel(TurboMfmaArgs p) {
    constexpr int NW = kPqThreads / 64;
    constexpr int H = D / 2;           // half row
    constexpr int FB = H / 32;         // 32-feature blocks of a half's transform
    constexpr int KH = H / 16;         // 16-wide k-steps of a half
    constexpr int Q = H / 2;           // features per lane and run
    constexpr int OB = D / 32;         // 32-output blocks of S r
    constexpr int KC = D / 16;         // k-steps of S r
    using op_t = tq_op_t<F16>;
    // rotation operands [half][fb][ks][lane], S' operands [ob][c][hi / lo][lane]
    __shared__ __attribute__((aligned(16))) u32x4 sm_h[2 * FB * KH * 64];
    __shared__ __attribute__((aligned(16))) u32x4 sm_s[OB * KC * 2 * 64];
    // bin table entries with the two centroids a code of the bin can take, times -64:
    // (inner boundary, count below, -64 centroid[count], -64 centroid[count + 1])
    __shared__ __attribute__((aligned(16))) u32x4 sm_lut[kLutN * kLutCopies];
    const AppendArgs &a = p.a;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, l = lane >> 5;

    // ---- once per workgroup ----
    const uint32_t one = F16 ? 0x3C00u : 0x3F80u;
    for (int i = tid; i < 2 * FB * KH * 64; i += kPqThreads) {
        const int ln = i & 63, ks = (i >> 6) % KH, fb = ((i >> 6) / KH) % FB, half = (i >> 6) / (KH * FB);
        const int f = pq_perm(ln & 31, Q, fb);  // feature of operand row ln % 32 (in the half)
        uint32_t w[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            uint32_t v = 0;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int k = 16 * ks + 8 * (ln >> 5) + 2 * e2 + h2;  // index in the half
                const int el = half * H + k;
                const uint32_t par = ((uint32_t)__popc(f & k) + (a.sign_bits[el >> 5] >> (el & 31))) & 1u;
                v |= (one | (par << 15)) << (16 * h2);
            }
            w[e2] = v;
        }
        sm_h[i] = u32x4{w[0], w[1], w[2], w[3]};
    }
    {
        // S' operands: each thread's rows of S (two 16-byte loads per operand lane) are loaded
        // before any is converted
        constexpr int NS = OB * KC * 64, IT = (NS + kPqThreads - 1) / kPqThreads;
        f32x4 sv[IT][2];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int i = tid + it * kPqThreads;
            if (i < NS) {
                const int ln = i & 63, c = (i >> 6) % KC, ob = (i >> 6) / KC;
                const int o = pq_perm(ln & 31, H, ob);  // output row of operand row ln % 32
                // slots 8 hl .. + 7 of k-step c: residuals 8 c' .. 8 c' + 7 of lane half hl's runs
                const int f0 = (c < KC / 2 ? 0 : H) + Q * (ln >> 5) + 8 * (c % (KC / 2));
                const f32x4 *src = (const f32x4 *)(a.qjl + (int64_t)o * D + f0);
                sv[it][0] = src[0];
                sv[it][1] = src[1];
            }
        }
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int i = tid + it * kPqThreads;
            if (i < NS) {
                const int ln = i & 63, c = (i >> 6) % KC, ob = (i >> 6) / KC;
                const float v[8] = {sv[it][0].x, sv[it][0].y, sv[it][0].z, sv[it][0].w,
                                    sv[it][1].x, sv[it][1].y, sv[it][1].z, sv[it][1].w};
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    const float h0 = (float)(_Float16)v[2 * e2], h1 = (float)(_Float16)v[2 * e2 + 1];
                    hi[e2] = pack_f16x2(h0, h1);
                    lo[e2] = pack_f16x2(v[2 * e2] - h0, v[2 * e2 + 1] - h1);
                }
                sm_s[((ob * KC + c) * 2 + 0) * 64 + ln] = u32x4{hi[0], hi[1], hi[2], hi[3]};
                sm_s[((ob * KC + c) * 2 + 1) * 64 + ln] = u32x4{lo[0], lo[1], lo[2], lo[3]};
            }
        }
    }
    // the bin table: one thread per entry writes copy 0 (two dependent argument reads), then
    // every thread fills the other copies from it
    const int S = p.lut_s;
    if (tid <= 2 * S) {
        const int c = p.lut_c[tid];
        sm_lut[tid * kLutCopies] =
            u32x4{__float_as_uint(p.lut_b[tid]), (uint32_t)c, __float_as_uint(-64.0f * a.cent[c]),
                  __float_as_uint(-64.0f * a.cent[min(c + 1, 15)])};
    }
    __syncthreads();
    for (int i = tid; i < (2 * S + 1) * kLutCopies; i += kPqThreads)
        if (i % kLutCopies != 0) sm_lut[i] = sm_lut[i / kLutCopies * kLutCopies];
    __syncthreads();
    const int lut0 = S * kLutCopies + (lane & 31);  // this lane's copy of bin 0's entry

    // ---- chunks of 32 tokens of one plane, one per wavefront at a time (the wavefronts of a
    // workgroup take consecutive chunks); two wavefronts per SIMD, each with the next chunk's rows
    // in flight while it encodes the current one (three per SIMD without the prefetch: 2 % slower) ----
    const int pos0 = a.position;
    const int gw = (int)blockIdx.x * NW + wave, gstride = (int)gridDim.x * NW;
    // lane (n, l): token c0 + n, elements h H + 16 ks + 8 l .. + 7 (past the last chunk: zeros)
    const auto load_rows = [&](const TqChunk &c, u32x4 (&xv)[2][KH]) {
        const int t = c.c0 + n;
        const bool live = c.valid && t >= c.pos && t < c.end;
        const uint16_t *base = (const uint16_t *)a.x + (int64_t)c.b * a.sb +
                               (int64_t)c.h * a.sh + (int64_t)(c.c0 - c.pos) * a.st;
        const rsrc_t r = make_rsrc(base, kTqOOB);
        const uint32_t off = live ? (uint32_t)((int64_t)(t - c.c0) * a.st * 2 + 16 * l) : kTqOOB;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int ks = 0; ks < KH; ++ks) xv[h][ks] = ld128(r, off + 2 * (h * H + 16 * ks));
    };
    TqChunk cur = tq_chunk<kPqTok>(p, gw, pos0);
    u32x4 xv[2][KH];
    load_rows(cur, xv);
    for (int ck = gw; ck < p.total_chunks; ck += gstride) {
        // the next chunk's rows are in flight while this one is encoded
        const TqChunk nxt = tq_chunk<kPqTok>(p, ck + gstride, pos0);
        u32x4 xn[2][KH];
        load_rows(nxt, xn);
        // (every iteration computes; dead tokens read zeros and store nothing)
        int bl = lane;  // keeps the operand reads from being hoisted out of the loop
        asm volatile("" : "+v"(bl));
        const u32x4 *hsm = sm_h + bl;
        const u32x4 *ssm = sm_s + bl;
        // rotation: u in ya[fb], v in yb[fb]
        pq_f32x16 ya[FB], yb[FB];
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) {
            ya[fb] = pq_f32x16{};
            yb[fb] = pq_f32x16{};
        }
#pragma unroll
        for (int ks = 0; ks < KH; ++ks)
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                ya[fb] = pq_mfma(__builtin_bit_cast(op_t, hsm[((0 * FB + fb) * KH + ks) * 64]),
                                 __builtin_bit_cast(op_t, xv[0][ks]), ya[fb]);
                yb[fb] = pq_mfma(__builtin_bit_cast(op_t, hsm[((1 * FB + fb) * KH + ks) * 64]),
                                 __builtin_bit_cast(op_t, xv[1][ks]), yb[fb]);
            }
        // y = (u + v, u - v): lane features Q l + q (ya) and H + Q l + q (yb), q = 16 fb + j
        float ss = 0.0f;
#pragma unroll
        for (int fb = 0; fb < FB; ++fb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float u = ya[fb][j], v = yb[fb][j];
                ya[fb][j] = u + v;
                yb[fb][j] = u - v;
                ss = __builtin_fmaf(ya[fb][j], ya[fb][j], ss);
                ss = __builtin_fmaf(yb[fb][j], yb[fb][j], ss);
            }
        const float norm = __builtin_amdgcn_sqrtf(xor32_sum(ss));
        const float inv = norm > 0.0f ? __builtin_amdgcn_rcpf(norm) : 0.0f;
        const float w = (float)S * inv;
        const bool fin = norm <= 3.0e38f && w <= 3.0e38f;
        // codes (nibble q of run 0, then of run 1) and the residuals r = u - centroid[code],
        // scaled by 64, as f16 hi / lo B operands (k-step c: word c of run 0, then of run 1);
        // where a norm is not finite, the plain count (NaN -> 0, infinities) and the centroid
        // from the kernel arguments
        uint32_t cw[2][Q / 8];
        f16x8 rhi[KC], rlo[KC];
        float rr = 0.0f;
        const float inv64 = 64.0f * inv;
        const bool fast = __all(fin);
#pragma unroll
        for (int run = 0; run < 2; ++run)
#pragma unroll
            for (int wd = 0; wd < Q / 8; ++wd) {
                uint32_t word = 0;
                float rv[8];
                if (fast) {
                    // four lookups at a time in flight together, then their use
#pragma unroll
                    for (int e0 = 0; e0 < 8; e0 += 4) {
                        float us[4];
                        u32x4 ent[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int q = 8 * wd + e0 + e;
                            us[e] = (run == 0 ? ya[q / 16][q % 16] : yb[q / 16][q % 16]) * w;
                            ent[e] = sm_lut[lut0 + (int)us[e] * kLutCopies];
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int q = 8 * wd + e0 + e;
                            const float y = run == 0 ? ya[q / 16][q % 16] : yb[q / 16][q % 16];
                            const bool up = us[e] >= __uint_as_float(ent[e].x);
                            word |= (ent[e].y + (up ? 1u : 0u)) << (4 * (e0 + e));
                            rv[e0 + e] = __builtin_fmaf(y, inv64, __uint_as_float(up ? ent[e].w : ent[e].z));
                        }
                    }
                } else {
                    for (int e = 0; e < 8; ++e) {
                        const int q = 8 * wd + e;
                        const float y = run == 0 ? ya[q / 16][q % 16] : yb[q / 16][q % 16];
                        const float u = y * inv;
                        uint32_t code = 0;
                        for (int kk = 0; kk < 15; ++kk) code += u >= a.bnd[kk] ? 1u : 0u;
                        word |= code << (4 * e);
                        rv[e] = 64.0f * (u - a.cent[code]);
                    }
                }
                // f16 hi (round to nearest) and lo = v - hi rounded once to f16: one
                // v_cvt_pk_f16_f32 per pair, one mixed-precision FMA per element
                u32x4 hw, lw;
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    rr = __builtin_fmaf(rv[2 * e2], rv[2 * e2], rr);
                    rr = __builtin_fmaf(rv[2 * e2 + 1], rv[2 * e2 + 1], rr);
                    const uint32_t h2 = pack_f16x2(rv[2 * e2], rv[2 * e2 + 1]);
                    uint32_t l2;
                    asm("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]"
                        : "=v"(l2) : "v"(rv[2 * e2]), "v"(h2));
                    asm("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
                        : "+v"(l2) : "v"(rv[2 * e2 + 1]), "v"(h2));
                    hw[e2] = h2;
                    lw[e2] = l2;
                }
                const f16x8 hi = __builtin_bit_cast(f16x8, hw), lo = __builtin_bit_cast(f16x8, lw);
                cw[run][wd] = word;
                rhi[run * (KC / 2) + wd] = hi;
                rlo[run * (KC / 2) + wd] = lo;
            }
        const float r1 = __builtin_amdgcn_sqrtf(xor32_sum(rr)) * (1.0f / 64.0f);
        // p = S r for the lane's outputs (D/2) l + 16 ob + j
        // two passes of half the output blocks each (half the accumulators live)
        uint32_t sg[OB / 2];
#pragma unroll
        for (int i = 0; i < OB / 2; ++i) sg[i] = 0;
#pragma unroll
        for (int ph = 0; ph < 2; ++ph) {
            pq_f32x16 pp[OB / 2];
#pragma unroll
            for (int o2 = 0; o2 < OB / 2; ++o2) pp[o2] = pq_f32x16{};
#pragma unroll
            for (int c = 0; c < KC; ++c)
#pragma unroll
                for (int o2 = 0; o2 < OB / 2; ++o2) {
                    const int ob = ph * (OB / 2) + o2;
                    const f16x8 shi = __builtin_bit_cast(f16x8, ssm[((ob * KC + c) * 2 + 0) * 64]);
                    const f16x8 slo = __builtin_bit_cast(f16x8, ssm[((ob * KC + c) * 2 + 1) * 64]);
                    pp[o2] = pq_mfma(shi, rhi[c], pp[o2]);
                    pp[o2] = pq_mfma(shi, rlo[c], pp[o2]);
                    pp[o2] = pq_mfma(slo, rhi[c], pp[o2]);
                }
#pragma unroll
            for (int o2 = 0; o2 < OB / 2; ++o2) {
                const int ob = ph * (OB / 2) + o2;
                // bit j of the block's 16 = (p_j >= 0), shifted in from the top (one add with
                // carry per bit)
                uint32_t g = 0;
#pragma unroll
                for (int j = 15; j >= 0; --j) g = 2u * g + (pp[o2][j] >= 0.0f ? 1u : 0u);
                sg[ob / 2] |= g << (16 * (ob & 1));
            }
        }

        // ---- stores (dead tokens: offsets past the range, dropped); the lane's token and half
        // are recomputed here, so that their store offsets are not held across the loop ----
        int sl = lane;
        asm volatile("" : "+v"(sl));
        const int t = cur.c0 + (sl & 31), l = sl >> 5;
        const bool live = cur.valid && t >= cur.pos && t < cur.end;
        const int64_t plane = (int64_t)cur.b * a.kv_heads + cur.h;
        const rsrc_t code_r = make_rsrc(a.codes + plane * a.codes_plane, kTqOOB);
        const rsrc_t sc_r = make_rsrc(a.scales + plane * a.scales_plane, kTqOOB);
        const uint32_t crow = live ? (uint32_t)t * (D / 2) : kTqOOB;
        // run 0 at byte (D/8) l of the row, run 1 at D/4 + (D/8) l
        if constexpr (Q / 8 == 4) {
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{cw[0][0], cw[0][1], cw[0][2], cw[0][3]}, code_r,
                                                   live ? crow + (D / 8) * l : kTqOOB, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{cw[1][0], cw[1][1], cw[1][2], cw[1][3]}, code_r,
                                                   live ? crow + D / 4 + (D / 8) * l : kTqOOB, 0, 0);
        } else {
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{cw[0][0], cw[0][1]}, code_r,
                                                  live ? crow + (D / 8) * l : kTqOOB, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{cw[1][0], cw[1][1]}, code_r,
                                                  live ? crow + D / 4 + (D / 8) * l : kTqOOB, 0, 0);
        }
        const uint32_t cap = (uint32_t)a.capacity;
        // norm (lane half 0) and |r| (lane half 1) of the token
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l == 0 ? norm * a.rot_scale : r1), sc_r,
                                              live ? (uint32_t)t * 4u + 4u * cap * (uint32_t)l : kTqOOB,
                                              0, 0);
        // sign bits of outputs (D/2) l .. : bytes (D/16) l of the token's D/8
        const uint32_t soff = live ? 8u * cap + (uint32_t)t * (D / 8) + (D / 16) * l : kTqOOB;
        if constexpr (OB == 4) __builtin_amdgcn_raw_buffer_store_b64(u32x2{sg[0], sg[1]}, sc_r, soff, 0, 0);
        else __builtin_amdgcn_raw_buffer_store_b32(sg[0], sc_r, soff, 0, 0);
        cur = nxt;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int ks = 0; ks < KH; ++ks) xv[h][ks] = xn[h][ks];
    }
}

template <int D>
static void pq_launch_d(bool f16, dim3 grid, hipStream_t st, const TurboMfmaArgs &p) {
    if (f16) hipLaunchKernelGGL((prod_mfma_kernel<D, true>), grid, dim3(kPqThreads), 0, st, p);
    else hipLaunchKernelGGL((prod_mfma_kernel<D, false>), grid, dim3(kPqThreads), 0, st, p);
}

// Launches the MFMA form for a TurboProd key side appended from 16-byte aligned bf16 / f16 rows
// with the Hadamard rotation at D = 64 / 128; false (nothing launched) for any other case.
bool prod_mfma_launch(const cqkv_side *s, int32_t tokens, int32_t batch, hipStream_t st,
                      const AppendArgs &a) {
    if (s->format != CQKV_FMT_TURBOPROD || s->is_value || !a.rotate || !a.qjl) return false;
    if (a.row_loads != kRowBF16 && a.row_loads != kRowF16) return false;
    const int d = s->head_dim;
    if ((d != 64 && d != 128) || a.dim != d) return false;
    if (a.st < 0 || (int64_t)kPqTok * a.st * 2 + 2 * d >= kTqOOB ||
        (int64_t)s->capacity * (8 + d / 8) >= kTqOOB || (int64_t)s->capacity * (d / 2) >= kTqOOB)
        return false;
    TurboMfmaArgs p = {};
    p.a = a;
    bool ok = false;
    for (int S = 8; S <= kLutMaxS && !ok; S *= 2) ok = tq_build_lut(a.bnd, S, p);
    if (!ok) return false;
    const int lead = !a.positions && a.position >= 0 ? a.position % 8 : 7;
    p.chunks_per_plane = (int)(((int64_t)tokens + lead + kPqTok - 1) / kPqTok);
    const int64_t total = (int64_t)p.chunks_per_plane * s->kv_heads * batch;
    if (total <= 0 || total > 0x7fffffff) return false;
    p.total_chunks = (int32_t)total;
    // one workgroup per CU (the LDS tables), enough of them for every chunk
    const dim3 grid((unsigned)std::min<int64_t>((total + kPqThreads / 64 - 1) / (kPqThreads / 64), 256));
    const bool f16 = a.row_loads == kRowF16;
    if (d == 128) pq_launch_d<128>(f16, grid, st, p);
    else pq_launch_d<64>(f16, grid, st, p);
    return true;
}

}  // namespace cqkv
