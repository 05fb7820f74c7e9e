// TurboQuant (TurboMse) append of bf16 / f16 rows with the rotation on MFMA
// (RowCodec::quantize_row, candle-core/src/accel/turbo.rs:299-323, after TurboQuantizer::rotate,
// candle-nn/src/turbo_quant.rs:182-189, then Cache::append, candle-nn/src/kv_cache.rs:68-99).
//
// The row-parallel encoder of append_rows.h spends most of its VALU issue on the sign flip, the
// seven Walsh-Hadamard stages and a three-step codebook search per element. Here:
//  * y = x diag(s) H^T (unscaled) is one MFMA product per 16 rows: the rows are the A operand as
//    they arrive (16-byte loads of bf16 / f16, no conversion), B is the +-1 matrix
//    B[k][c] = s_k H[pi(c)][k] (exact in bf16 / f16, so every product is exact), built once per
//    workgroup in LDS and read from there by each product. The output columns are permuted,
//    pi(16 nb + n) = (D / 16) n + nb, so that lane (n, g) ends with D / 16 consecutive columns of
//    rows 4 g .. 4 g + 3.
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
template <int ROWS>
__device__ inline TqChunk tq_chunk(const TurboMfmaArgs &p, int ck) {
    const AppendArgs &a = p.a;
    TqChunk c = {};
    if (ck >= p.total_chunks) return c;  // valid false: past the last chunk
    const int bx = ck % p.chunks_per_plane, plane = ck / p.chunks_per_plane;
    c.h = plane % a.kv_heads;
    c.b = plane / a.kv_heads;
    c.pos = a.positions ? a.positions[c.b] : a.position;
    c.c0 = c.pos / 8 * 8 + bx * ROWS;
    c.end = min(c.pos + a.tokens, a.capacity);
    if (a.cs_rows > 0) c.end = min(c.end, a.cs_rows);
    c.valid = c.pos >= 0 && c.c0 < c.end;
    return c;
}

// This lane's A operands of 16-row group grp of a chunk: row (group row n), head dims
// 32 ks + 8 g .. + 7; rows outside [pos, end) read zeros.
template <int D, int ROWS>
__device__ inline void tq_load(const AppendArgs &a, const TqChunk &c, int grp, int n, int g,
                               u32x4 (&av)[D / 32]) {
    const int t = c.c0 + 16 * grp + n;
    const bool live = c.valid && t >= c.pos && t < c.end;
    const uint16_t *row = (const uint16_t *)a.x + (int64_t)c.b * a.sb + (int64_t)c.h * a.sh +
                          (int64_t)(t - c.pos) * a.st + 8 * g;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
        av[ks] = live ? *(const u32x4 *)(row + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
}

template <int IS_VALUE, int D, bool F16>
__global__ __launch_bounds__(kTqThreads) void turbo_mfma_kernel(TurboMfmaArgs p) {
    constexpr int NW = kTqThreads / 64;
    constexpr int NB = D / 16, KS = D / 32, ROWS = kTqRows, GPW = ROWS / (16 * NW);
    constexpr int kRowBytes = D / 2;
    using op_t = tq_op_t<F16>;
    __shared__ __attribute__((aligned(16))) u32x4 sm_b[NB * KS * 64];
    __shared__ __attribute__((aligned(16))) u32x2 sm_lut[kLutN * kLutCopies];
    __shared__ __attribute__((aligned(16))) uint8_t sm_codes[IS_VALUE ? ROWS * kRowBytes : 16];
    const AppendArgs &a = p.a;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;

    // ---- once per workgroup: B (as [nb][ks][lane] operands) and the replicated table; every
    // read of the kernel arguments here has a workgroup-uniform index (scalar loads) ----
    const uint32_t sgn[4] = {a.sign_bits[0], a.sign_bits[1], a.sign_bits[2], a.sign_bits[3]};
#pragma unroll
    for (int it = 0; it < (NB * KS * 64 + kTqThreads - 1) / kTqThreads; ++it) {
        const int i = tid + kTqThreads * it;
        if (i >= NB * KS * 64) break;
        const int l = i & 63, ks = (i >> 6) % KS, nb = (i >> 6) / KS;
        const int col = NB * (l & 15) + nb;
        const uint32_t one = F16 ? 0x3C00u : 0x3F80u;
        const uint32_t sw = ks == 0 ? sgn[0] : ks == 1 ? sgn[1] : ks == 2 ? sgn[2] : sgn[3];
        uint32_t w[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            uint32_t v = 0;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int k = 32 * ks + 8 * (l >> 4) + 2 * e2 + h2;
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
    const u32x4 *bsm = sm_b + lane;
    // this lane's copy of the entry of bin 0 (bin j is entry j + S)
    const u32x2 *lut0 = sm_lut + S * kLutCopies + (lane & 31);

    // ---- the chunks of this workgroup; the next chunk's rows load while this one computes ----
    int ck = blockIdx.x;
    TqChunk cur = tq_chunk<ROWS>(p, ck);
    u32x4 av[GPW][KS], nv[GPW][KS];
#pragma unroll
    for (int grp = 0; grp < GPW; ++grp) tq_load<D, ROWS>(a, cur, wave * GPW + grp, n, g, av[grp]);
    for (; ck < p.total_chunks; ck += gridDim.x) {
        const TqChunk nxt = tq_chunk<ROWS>(p, ck + (int)gridDim.x);
#pragma unroll
        for (int grp = 0; grp < GPW; ++grp) tq_load<D, ROWS>(a, nxt, wave * GPW + grp, n, g, nv[grp]);
        if (cur.valid) {  // workgroup-uniform
            const int64_t plane = (int64_t)cur.b * a.kv_heads + cur.h;
            uint8_t *codes = a.codes + plane * a.codes_plane;
            float *norms = (float *)(a.scales + plane * a.scales_plane);
#pragma unroll
            for (int grp = 0; grp < GPW; ++grp) {
                const int r0 = 16 * (wave * GPW + grp);  // the group's first row in the chunk
                // MFMAs in ks-major order: consecutive products update different accumulators
                f32x4 acc[NB];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = mfma16x16x32(__builtin_bit_cast(op_t, av[grp][0]),
                                           __builtin_bit_cast(op_t, bsm[(nb * KS) * 64]),
                                           f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int ks = 1; ks < KS; ++ks)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[nb] = mfma16x16x32(__builtin_bit_cast(op_t, av[grp][ks]),
                                               __builtin_bit_cast(op_t, bsm[(nb * KS + ks) * 64]),
                                               acc[nb]);
                // lane (n, g): rows r0 + 4 g + i, columns NB n .. NB n + NB - 1 (column NB n + nb
                // in acc[nb]). Row norms by the hardware square root and reciprocal (1 ulp; the
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
                uint8_t *dst = (IS_VALUE ? sm_codes + rg * kRowBytes
                                         : codes + (int64_t)tg * kRowBytes) + (NB / 2) * n;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool live = tg + i >= cur.pos && tg + i < cur.end;
                    if (live && n == 0) norms[tg + i] = norm[i] * a.rot_scale;
                    if (IS_VALUE || live) {
                        if constexpr (NB == 8) *(uint32_t *)(dst + i * kRowBytes) = word[i];
                        else *(uint16_t *)(dst + i * kRowBytes) = (uint16_t)word[i];
                    }
                }
            }
            if constexpr (IS_VALUE != 0) {
                __syncthreads();
                write_value_tiles<false, D, ROWS, kTqThreads>(codes, sm_codes, cur.c0, cur.pos, cur.end, tid);
                __syncthreads();  // sm_codes is rewritten by the next chunk
            }
        }
        cur = nxt;
#pragma unroll
        for (int grp = 0; grp < GPW; ++grp)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) av[grp][ks] = nv[grp][ks];
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
    TurboMfmaArgs p = {};
    p.a = a;
    bool ok = false;
    for (int S = 8; S <= kLutMaxS && !ok; S *= 2) ok = tq_build_lut(a.bnd, S, p);
    if (!ok) return false;
    p.chunks_per_plane = (int)(((int64_t)tokens + 7 + kTqRows - 1) / kTqRows);
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

}  // namespace cqkv
