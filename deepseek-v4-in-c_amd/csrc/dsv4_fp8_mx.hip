/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_fp8_mx.hip - the block-scaled FP8 GEMV and its batched form (prefill)
 * on gfx950's matrix cores, for FP8 matrices with E8M0 block scales (the
 * reference's format, dsv4.h:199-214).
 *
 * WHAT IT COMPUTES: dsv4_matmul_fp8 / dsv4_matmul_fp8_n (src/core/
 * dsv4_matmul.c:293-318, :378-428): y[t][o] = sum over the row's columns of
 * e4m3(W[o][c]) * 2^(S[o/blk_r][c/blk_c] - 127) * x[t][c], within 1e-5
 * relative of the reference's double accumulation.
 *
 * ONE ARITHMETIC FOR EVERY BATCH SIZE. The reference's batched call must give
 * each (row, token) the bits of the single-token call (the k_mmq_fp8_n
 * contract, dsv4_cuda.cu:161-230; tests/unit/test_cuda.c:194-256). Here both
 * run the same chain of matrix-core instructions per (row, token):
 *   - A (16 rows x 32 K of v_mfma_f32_16x16x32_bf16) is the weights decoded
 *     with their block scale folded in: v_cvt_scalef32_pk_bf16_fp8 turns an
 *     e4m3 code times a power of two into bf16 exactly (3 mantissa bits into
 *     7), so no per-block product remains to be rounded separately;
 *   - B holds x as three bf16 terms hi + mid + lo (all 24 bits of the f32),
 *     one column per (token, term), five tokens per 16-column tile; every
 *     product is exact and the matrix core accumulates in f32;
 *   - per (row, term column): the columns are cut into segments of 1024
 *     (four units of 256); within a segment one accumulator runs through
 *     the segment's K steps in order, starting from zero; the segments'
 *     partials are then added in segment order; y = (hi + mid) + lo.
 *   The K order inside a unit is fixed by how a lane reads the staged unit:
 *   lane (row r, group g) takes the 16 bytes [64 q + 16 g, +16) of quarter
 *   q, the first 8 for step (q, 0) and the last 8 for step (q, 1); B is read
 *   in the same order.
 * The single-token kernel spreads a 16-row tile's segments over up to 8
 * waves (so short matrices still fill the machine); the first of them keeps
 * the running sum in registers and continues it over the others' partials
 * from LDS. The batched kernel walks the segments in order inside one wave;
 * for one or two groups of at most five tokens its k_fp8_mxk form splits them
 * over 2 or 4 waves the same way.
 * Matrix-core columns are computed independently, so where a token sits
 * among the columns does not change its bits; the tests check every case
 * bit for bit.
 *
 * MEMORY: weights stream in units of 16 rows x 256 bytes, loaded as four
 * 4-row x 256-byte requests per wave (fully coalesced), staged through a
 * wave-private LDS buffer into the matrix core's operand order (the layout
 * dsv4_moe_mx.hip measured fastest on MI355X). The single-token kernel is
 * persistent: each wave keeps one segment (16 KB) in flight ahead of the
 * one it computes, across tiles, and its workgroup turns x into terms once.
 * The memory counter is in order, so every kernel issues what it waits for
 * first (x, then the weights in K order) and keeps every load outside
 * branches; register arrays are indexed by compile-time constants only.
 */
#include <type_traits>

#include "dsv4_dev.h"
#include "dsv4_internal.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int XU = 256;                 /* K (bytes) per row per unit      */
constexpr int XSEG_U = 4;               /* units per segment               */
constexpr int XSEG = XU * XSEG_U;       /* K per segment                   */
constexpr int XWP = XU + 16;            /* LDS pitch of a staged unit row  */
constexpr int XUNIT_B = 16 * XWP;       /* one wave's unit buffer          */
constexpr int XNT = 3;                  /* bf16 terms per activation       */
constexpr int XTOK = 5;                 /* tokens per 16-column tile       */
constexpr int XSEG_MAX = 16;            /* segments per row (cols <= 16384) */

__device__ __forceinline__ uint32_t rne_bf16(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

/* v = hi + mid + lo exactly (finite v). */
__device__ __forceinline__ void terms3(float v, uint32_t *t)
{
    t[0] = rne_bf16(v);
    const float r1 = v - __uint_as_float(t[0] << 16);
    t[1] = rne_bf16(r1);
    const float r2 = r1 - __uint_as_float(t[1] << 16);
    t[2] = rne_bf16(r2);
}

/* Eight e4m3 codes (two dwords, element order) times the power of two s,
 * as eight bf16 -- exactly. */
__device__ __forceinline__ v8bf fp8x8_bf16(uint32_t lo, uint32_t hi, float s)
{
    const v2s p0 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, s, false));
    const v2s p1 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, s, true));
    const v2s p2 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, s, false));
    const v2s p3 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, s, true));
    const v8s r = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    return __builtin_bit_cast(v8bf, r);
}

/* The wave's LDS accesses before this point complete before those after it,
 * for every lane: a lane reads what other lanes of its wave staged. */
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* One unit of a 16-row tile in flight: lane l holds row 4 q + l / 16, bytes
 * [16 (l % 16), +16) of the unit, for q = 0..3. With per-lane scales (UNI
 * false) also the E8M0 bytes of the four pieces the lane will decode (row
 * l % 16, columns 64 q + 16 (l / 16) of the unit), loaded with the weights so
 * that they arrive together. With uniform scales (blk_r a multiple of 16 and
 * blk_c of 64: every row of a tile and every lane share each quarter's
 * scale) the scales travel once per segment instead (xs_seg). */
template <bool UNI>
struct XUnit {
    u32x4 w[4];
    uint32_t sb[UNI ? 1 : 4];
};

/* k / blk_c for 0 <= k < 2^16 and 16 <= blk_c <= 2^16, with m = ceil(2^32 /
 * blk_c): m blk_c - 2^32 = e < blk_c, so k m / 2^32 = k / blk_c + k e /
 * (blk_c 2^32), and the added k e / (blk_c 2^32) < 1 / blk_c never carries
 * the quotient past an integer. */
__device__ __forceinline__ int div_bc(int k, uint32_t m)
{
    return (int)__umulhi((uint32_t)k, m);
}

inline uint32_t bc_magic(int blk_c)
{
    return (uint32_t)((((uint64_t)1 << 32) + (uint64_t)blk_c - 1) / (uint64_t)blk_c);
}

/* Unit u of the tile whose row 0 is W + row0 * cols (rows past `rows` read
 * the last row, pieces past `cols` the row's first piece: their results are
 * discarded or zeroed). srow: this lane's scale row offset, (row / blk_r) sc
 * for its A row, row0 + lane % 16 clamped to the last row. STREAM: a
 * non-temporal load, for weights read once (the single-token kernel); the
 * batched kernel's token groups read each unit again, from L2. */
template <bool UNI, bool STREAM = true>
__device__ __forceinline__ void xu_load(XUnit<UNI> &U, const uint8_t *W, const uint8_t *S,
                                        int srow, uint32_t bc_m, int row0, int rows, int cols,
                                        int k0, int lane)
{
    const int c = k0 + 16 * (lane & 15);
    const int cc = c < cols ? c : 0;
    if (!UNI) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = min(k0 + 64 * q + 16 * (lane >> 4), cols - 1);
            U.sb[UNI ? 0 : q] = ldg8(S + srow + div_bc(k, bc_m));
        }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int r = min(row0 + 4 * q + (lane >> 4), rows - 1);
        if (STREAM)
            U.w[q] = ldg16_stream(W + (size_t)r * cols + cc);
        else
            U.w[q] = *(const DSV4_GLOBAL u32x4 *)(W + (size_t)r * cols + cc);
    }
}

/* Uniform scales: the E8M0 bytes of the 16 quarters of the segment at k0
 * (quarter m = 4 unit + q in lane m % 16; srow is the tile's scale row
 * offset). Decoded once per segment, xs_getf reads quarter m's scale back
 * from its lane. */
__device__ __forceinline__ uint32_t xs_seg(const uint8_t *S, int srow, uint32_t bc_m, int k0,
                                           int cols, int lane)
{
    return ldg8(S + srow + div_bc(min(k0 + 64 * (lane & 15), cols - 1), bc_m));
}

/* Quarter m's scale from a register of decoded scales (lane m holds
 * quarter m's 2^(e - 127), decoded once per segment): one readlane per
 * fragment instead of a readlane and a scalar decode. */
__device__ __forceinline__ float xs_getf(float sf, int m)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sf), m));
}

template <bool UNI>
__device__ __forceinline__ void xu_stage(unsigned char *buf, const XUnit<UNI> &U, int lane)
{
#pragma unroll
    for (int q = 0; q < 4; q++)
        *reinterpret_cast<u32x4 *>(buf + (4 * q + (lane >> 4)) * XWP + 16 * (lane & 15)) = U.w[q];
}

/* The A operands of quarter q for this lane: steps (q, 0) and (q, 1). A piece
 * past the row's end is zero (its codes are replaced and its scale is 0: a
 * NaN code times 0 would still be NaN). */
__device__ __forceinline__ void xu_frags(v8bf *a, const unsigned char *buf, int q, uint32_t sb,
                                         bool live, int lane)
{
    const u32x4 v = *reinterpret_cast<const u32x4 *>(buf + (lane & 15) * XWP + 64 * q +
                                                      16 * (lane >> 4));
    const u32x4 z = live ? v : u32x4{0u, 0u, 0u, 0u};
    const float s = live ? dec_e8m0(sb) : 0.0f;
    a[0] = fp8x8_bf16(z.x, z.y, s);
    a[1] = fp8x8_bf16(z.z, z.w, s);
}

/* The same with the quarter's scale already decoded (uniform scales). */
__device__ __forceinline__ void xu_frags_f(v8bf *a, const unsigned char *buf, int q, float sq,
                                           bool live, int lane)
{
    const u32x4 v = *reinterpret_cast<const u32x4 *>(buf + (lane & 15) * XWP + 64 * q +
                                                      16 * (lane >> 4));
    const u32x4 z = live ? v : u32x4{0u, 0u, 0u, 0u};
    const float s = live ? sq : 0.0f;
    a[0] = fp8x8_bf16(z.x, z.y, s);
    a[1] = fp8x8_bf16(z.z, z.w, s);
}

/* ------------------------------------------------------ single token */

/* One segment of a tile for a single token: units j = 0..nu-1 of the
 * segment at column k0, held in P4[j], staged through the wave's buffer and
 * run through the matrix core in order (accumulator from zero). With PF each
 * slot, once staged, is refilled with unit j of the next job (the segment at
 * k0n of the tile at row0n; slots past its nun units repeat its last unit).
 * Returns the segment's accumulator (D layout). */
template <bool UNI, bool PF>
__device__ __forceinline__ v4f mx1_seg(XUnit<UNI> (&P4)[XSEG_U], unsigned char *buf,
                                       const uint16_t *pl, int bplane, const uint8_t *W,
                                       const uint8_t *S, int rows, int cols, uint32_t bc_m,
                                       int k0, int nu, float sfb, int row0n, int srown,
                                       int k0n, int nun, int lane)
{
    const int g = lane >> 4;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < XSEG_U; j++) {
        if (j < nu) {
            wave_lds_sync();                           /* the previous unit's reads */
            xu_stage(buf, P4[j], lane);
        }
        uint32_t sbj[4];
#pragma unroll
        for (int q = 0; q < 4; q++) sbj[q] = UNI ? 0u : P4[j].sb[UNI ? 0 : q];
        if (PF) {
            __builtin_amdgcn_sched_barrier(0);
            xu_load(P4[j], W, S, srown, bc_m, row0n, rows, cols, k0n + XU * min(j, nun - 1),
                    lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (j < nu) {
            wave_lds_sync();
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int k = k0 + XU * j + 64 * q + 16 * g;
                v8bf af[2];
                if (UNI)
                    xu_frags_f(af, buf, q, xs_getf(sfb, 4 * j + q), k < cols, lane);
                else
                    xu_frags(af, buf, q, sbj[q], k < cols, lane);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const u32x4 bw = *reinterpret_cast<const u32x4 *>(
                        pl + bplane + k0 + XU * j + 64 * q + 16 * g + 8 * h);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        af[h], __builtin_bit_cast(v8bf, bw), acc, 0, 0, 0);
                }
            }
        }
    }
    return acc;
}

/* Persistent single-token kernel. A tile's segments are split over P waves
 * (wave p takes segments [p spw, (p + 1) spw)); a workgroup holds TPW tiles
 * of P waves and walks tile groups blockIdx.x, + gridDim.x, ... Each wave
 * streams its segments one segment ahead: while it runs unit j of a segment,
 * units j+1..3 of it and 0..j of its next segment (the next tile's first, at
 * a tile's end) are in flight. The workgroup turns x into bf16 terms in LDS
 * once (three planes of xp bf16, zeros past cols). Wave 0 of a tile (whose
 * segments start at 0) chains its segment partials in registers and, after
 * a barrier, continues the chain over the other waves' partials from LDS in
 * segment order: the arithmetic of every (row, term column) is the segment
 * chain whatever P is. Every register array is indexed by compile-time
 * constants (a run-time index would put it in scratch memory). */
constexpr int X1_XM = 8;                    /* x pieces (f32x4) per thread */

template <bool UNI>
__global__ void __launch_bounds__(512, UNI ? 4 : 2)   /* uniform: two 8-wave groups per CU */
k_fp8_mx1(Dsv4Fp8Mx a)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char x1lds[];
    /* the wave index through readfirstlane: everything per wave (tile, row,
     * segment, scale row) is then scalar and takes no vector registers */
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nw = blockDim.x >> 6;
    const int gi = blockIdx.y;
    const float *x = a.x + (size_t)gi * a.x_stride;
    const uint8_t *W = a.list ? a.wl[gi] : a.w + (size_t)gi * a.w_stride;
    const uint8_t *S = a.list ? a.sl[gi] : a.s + (size_t)gi * a.s_stride;
    float *y = a.list ? a.yl[gi] : a.y + (size_t)gi * a.y_stride;
    const int rows = a.list ? a.rl[gi] : a.rows;
    const int cols = a.cols;
    const int ntiles = (rows + 15) / 16;
    const int ngrp = (ntiles + a.tpw - 1) / a.tpw;
    if ((int)blockIdx.x >= ngrp) return;               /* the whole workgroup */
    const int nseg = (cols + XSEG - 1) / XSEG, nu_all = (cols + XU - 1) / XU;
    const int P = a.wpt, tw = w / P, p = w - tw * P;
    const int sa = p * a.spw, sb = min(nseg, sa + a.spw);
    const int xp = a.xp;
    uint16_t *pl = (uint16_t *)x1lds;                              /* [3][xp] */
    unsigned char *buf = x1lds + (size_t)XNT * xp * 2 + (size_t)w * XUNIT_B;
    /* part: per tile slot, a.npb buffers of the segments past wave 0's
     * ([nseg - spw][16][XNT] floats): two when the workgroup walks more
     * than one tile group (a tile's partials must not overwrite the ones
     * wave 0 is still reading), else one */
    float *part = (float *)(x1lds + (size_t)XNT * xp * 2 + (size_t)nw * XUNIT_B);
    const int part_n = (nseg - a.spw) * 16 * XNT;
    float *mypart = part + (size_t)tw * a.npb * part_n;
    const int g = lane >> 4, col = lane & 15;
    /* B columns 3..15 read plane col % 3 too: those columns of the result
     * are never used, and unconditional reads keep the steps branch-free */
    const int bplane = (col % XNT) * xp;

    /* x first (the memory counter is in order: waiting for x then leaves
     * the weights in flight): piece i = tid + nthreads m of the padded row */
    f32x4 xv[X1_XM];
    const int npc = nu_all * (XU / 4);                 /* pieces incl. padding */
#pragma unroll
    for (int m = 0; m < X1_XM; m++) {
        const int c = 4 * ((int)threadIdx.x + (int)blockDim.x * m);
        xv[m] = *(const DSV4_GLOBAL f32x4 *)(x + (c < cols ? c : 0));
    }
    __builtin_amdgcn_sched_barrier(0);

    /* the first job: tile group blockIdx.x, segment sa */
    int it = blockIdx.x, s = sa;
    int row0 = min(it * a.tpw + tw, ntiles - 1) * 16;
    int srow = ((UNI ? row0 : min(row0 + col, rows - 1)) / a.blk_r) * a.sc;
    uint32_t ssb = UNI ? xs_seg(S, srow, a.bc_m, s * XSEG, cols, lane) : 0u;
    XUnit<UNI> P4[XSEG_U];
    {
        const int nu0 = min(XSEG_U, nu_all - s * XSEG_U);
#pragma unroll
        for (int j = 0; j < XSEG_U; j++)
            xu_load(P4[j], W, S, srow, a.bc_m, row0, rows, cols, s * XSEG + XU * min(j, nu0 - 1),
                    lane);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < X1_XM; m++) {
        const int i = (int)threadIdx.x + (int)blockDim.x * m;
        if (i < npc) {
            const bool in = 4 * i < cols;
            const float e[4] = {in ? xv[m].x : 0.f, in ? xv[m].y : 0.f, in ? xv[m].z : 0.f,
                                in ? xv[m].w : 0.f};
            uint32_t t[4][XNT];
#pragma unroll
            for (int k = 0; k < 4; k++) terms3(e[k], t[k]);
#pragma unroll
            for (int q = 0; q < XNT; q++)
                *reinterpret_cast<uint2 *>(pl + q * xp + 4 * i) =
                    uint2{t[0][q] | (t[1][q] << 16), t[2][q] | (t[3][q] << 16)};
        }
    }
    __syncthreads();

    int pb = 0;                                        /* part buffer of this tile */
    v4f tot = {0.f, 0.f, 0.f, 0.f};
    /* the end of segment s of the current tile: wave 0 of the tile chains
     * it, the others keep it for wave 0; at the tile's end wave 0 continues
     * the chain over theirs and writes y = (hi + mid) + lo */
    auto finish = [&](const v4f &acc, bool tile_end) {
        if (p == 0) {
            tot = s == 0 ? acc : tot + acc;
        } else if (col < XNT) {
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                mypart[(size_t)pb * part_n + ((s - a.spw) * 16 + 4 * g + jj) * XNT + col] = acc[jj];
        }
        if (!tile_end) return;
        if (P > 1) __syncthreads();
        if (p == 0) {
            for (int s2 = sb; s2 < nseg; s2++) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
                    tot[jj] = tot[jj] + mypart[(size_t)pb * part_n +
                                               ((s2 - a.spw) * 16 + 4 * g + jj) * XNT + col % XNT];
            }
            const bool live = it * a.tpw + tw < ntiles;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const float c1 = __shfl(tot[jj], min(lane + 1, 63), 64);
                const float c2 = __shfl(tot[jj], min(lane + 2, 63), 64);
                const int rr = row0 + 4 * g + jj;
                if (live && col == 0 && rr < rows) y[rr] = (tot[jj] + c1) + c2;
            }
        }
        pb = a.npb - 1 - pb;
    };
    /* every job but the wave's last prefetches the next one; the last runs
     * after the loop, without loads (the loop is left before any load of
     * its iteration, so no wait after it has to allow for loads that might
     * not have been issued) */
    for (;;) {
        int itn = it, sn = s + 1;
        if (sn == sb) { sn = sa; itn = it + gridDim.x; }
        if (itn >= ngrp) break;
        const int tilen = min(itn * a.tpw + tw, ntiles - 1);
        const int row0n = tilen * 16;
        const int srown = ((UNI ? row0n : min(row0n + col, rows - 1)) / a.blk_r) * a.sc;
        const int k0n = sn * XSEG, nun = min(XSEG_U, nu_all - sn * XSEG_U);
        const uint32_t ssn = UNI ? xs_seg(S, srown, a.bc_m, k0n, cols, lane) : 0u;
        const v4f acc = mx1_seg<UNI, true>(P4, buf, pl, bplane, W, S, rows, cols, a.bc_m,
                                           s * XSEG, min(XSEG_U, nu_all - s * XSEG_U),
                                           UNI ? dec_e8m0(ssb) : 0.0f,
                                           row0n, srown, k0n, nun, lane);
        finish(acc, sn == sa);
        it = itn; s = sn; row0 = row0n; ssb = ssn;
    }
    const v4f acc = mx1_seg<UNI, false>(P4, buf, pl, bplane, W, S, rows, cols, a.bc_m, s * XSEG,
                                        min(XSEG_U, nu_all - s * XSEG_U), UNI ? dec_e8m0(ssb) : 0.0f, 0, 0, 0, 1, lane);
    finish(acc, true);
}

/* ------------------------------------------------------------ batched */

/* x terms of a group's tokens for one unit's 256 columns, in LDS as term
 * rows: bl[(tok * XNT + term) * BP + k], BP = XU + 8. */
constexpr int BP = XU + 8;
/* MW: waves (16-row tiles) per workgroup, a template parameter of the
 * batched kernel and its helpers (4, or 8 when the batch takes three or more
 * token groups: the x terms are then staged for twice the rows) */

/* f32x4 pieces of x per thread per unit: a group holds at most XTOK * NT
 * tokens of XU / 4 pieces, spread over the workgroup's 64 MW threads. */
template <int NT, int MW>
struct XnDim {
    static constexpr int M = (XTOK * NT * (XU / 4) + 64 * MW - 1) / (64 * MW);
};

/* Request piece i = tid + 64 MW m of the unit at column kc. Pieces past the
 * group's tokens or past cols read the group's first piece (unconditional
 * loads: no branch for the weight requests to wait behind) and become zeros
 * in xn_terms. */
template <int NT, int MW>
__device__ __forceinline__ void xn_load(f32x4 *v, const float *x, int t0, int ntok, int kc,
                                        int cols, int tpg)
{
#pragma unroll
    for (int m = 0; m < XnDim<NT, MW>::M; m++) {
        const int i = (int)threadIdx.x + 64 * MW * m;
        const int tk = i / (XU / 4), c = kc + 4 * (i % (XU / 4));
        const bool in = i < tpg * (XU / 4) && tk < ntok && c < cols;
        v[m] = *(const DSV4_GLOBAL f32x4 *)(x + (in ? (size_t)(t0 + tk) * cols + c
                                                   : (size_t)t0 * cols));
    }
}

template <int NT, int MW>
__device__ __forceinline__ void xn_terms(uint16_t *bl, const f32x4 *v, int ntok, int kc,
                                         int cols, int tpg)
{
#pragma unroll
    for (int m = 0; m < XnDim<NT, MW>::M; m++) {
        const int i = (int)threadIdx.x + 64 * MW * m;
        if (i < tpg * (XU / 4)) {
            const int tk = i / (XU / 4), c4 = i % (XU / 4);
            const bool in = tk < ntok && kc + 4 * c4 < cols;
            const float e[4] = {in ? v[m].x : 0.f, in ? v[m].y : 0.f, in ? v[m].z : 0.f,
                                in ? v[m].w : 0.f};
            uint32_t tt[4][XNT];
#pragma unroll
            for (int j = 0; j < 4; j++) terms3(e[j], tt[j]);
#pragma unroll
            for (int p = 0; p < XNT; p++)
                *reinterpret_cast<uint2 *>(bl + (size_t)(tk * XNT + p) * BP + 4 * c4) =
                    uint2{tt[0][p] | (tt[1][p] << 16), tt[2][p] | (tt[3][p] << 16)};
        }
    }
}

/* The batch's x as bf16 term planes, once per call (k_fp8_xsplit): xt[t][p]
 * is term p of token t's row, padded with zeros to cpad = a whole number of
 * units; the batched kernel then copies a unit's terms into LDS instead of
 * every workgroup forming them again. Same terms3, so the same bits. */
__global__ void __launch_bounds__(256)
k_fp8_xsplit(uint16_t *__restrict__ xt, const float *__restrict__ x, int nt, int cols,
             int cpad)
{
    /* 8 columns per thread: two 16-byte loads (x is 16-byte aligned and cols
     * a multiple of 16 wherever this form runs), three 16-byte stores */
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int per = cpad >> 3;
    if (i >= nt * per) return;
    const int t = i / per, c = 8 * (i - t * per);
    float e[8];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const f32x4 v = c + 4 * h < cols
                            ? *(const DSV4_GLOBAL f32x4 *)(x + (size_t)t * cols + c + 4 * h)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
        e[4 * h] = v.x;
        e[4 * h + 1] = v.y;
        e[4 * h + 2] = v.z;
        e[4 * h + 3] = v.w;
    }
    uint32_t tt[8][XNT];
#pragma unroll
    for (int j = 0; j < 8; j++) terms3(e[j], tt[j]);
#pragma unroll
    for (int p = 0; p < XNT; p++)
        *reinterpret_cast<u32x4 *>(xt + ((size_t)t * XNT + p) * cpad + c) =
            u32x4{tt[0][p] | (tt[1][p] << 16), tt[2][p] | (tt[3][p] << 16),
                  tt[4][p] | (tt[5][p] << 16), tt[6][p] | (tt[7][p] << 16)};
}

/* 16-byte pieces of the term planes per thread per unit: a group's tpg
 * tokens x XNT planes x XU / 8 pieces over the workgroup's 64 MW threads. */
template <int NT, int MW>
struct XpDim {
    static constexpr int M = (XTOK * NT * XNT * (XU / 8) + 64 * MW - 1) / (64 * MW);
};

/* Request piece i = tid + 64 MW m of unit u's term rows (row = token * XNT +
 * plane): rows past the group's tokens read its first row (unconditional
 * loads) and are stored as zeros. */
template <int NT, int MW>
__device__ __forceinline__ void xp_load(u32x4 *v, const uint16_t *xt, int t0, int ntok, int u,
                                        int cpad, int tpg)
{
#pragma unroll
    for (int m = 0; m < XpDim<NT, MW>::M; m++) {
        const int i = (int)threadIdx.x + 64 * MW * m;
        const int row = i / (XU / 8), pc = i % (XU / 8);
        const bool in = row < tpg * XNT && row / XNT < ntok;
        v[m] = *(const DSV4_GLOBAL u32x4 *)(xt + (in ? ((size_t)t0 * XNT + row) * cpad +
                                                         XU * u + 8 * pc
                                                       : (size_t)t0 * XNT * cpad));
    }
}

template <int NT, int MW>
__device__ __forceinline__ void xp_store(uint16_t *bl, const u32x4 *v, int ntok, int tpg)
{
#pragma unroll
    for (int m = 0; m < XpDim<NT, MW>::M; m++) {
        const int i = (int)threadIdx.x + 64 * MW * m;
        const int row = i / (XU / 8), pc = i % (XU / 8);
        if (row < tpg * XNT)
            *reinterpret_cast<u32x4 *>(bl + (size_t)row * BP + 8 * pc) =
                row / XNT < ntok ? v[m] : u32x4{0u, 0u, 0u, 0u};
    }
}

/* Workgroup (blockIdx.x: MW 16-row tiles, one per wave; blockIdx.y: a group
 * of tpg tokens starting at t0). Per unit u: the workgroup turns x(u), which
 * it requested one unit earlier, into terms in B buffer u % 2, each wave
 * stages its weight unit u (requested two units earlier), requests x(u + 1)
 * and weight unit u + 2, and after one barrier runs its tile's 8 steps x NT
 * column tiles. The weights are read with ordinary loads, so that the
 * other token groups read each unit again from L2: their workgroups for the
 * same rows are gridDim.x apart in launch order, so when gridDim.x is a
 * multiple of 8 (7168 rows: 56) they run on one XCD and share its L2 (7168 x
 * 7168 at nt 64: 66.5 -> 63.6 us against non-temporal loads). At each
 * segment's end the segment's accumulators join the running sums in segment
 * order. Every register array is indexed by compile-time constants: the
 * unit loop is unrolled by a segment's 4. */
template <int NT, bool UNI, int MW>
__global__ void __launch_bounds__(64 * MW)
k_fp8_mxn(float *__restrict__ y, const float *__restrict__ x, const uint8_t *__restrict__ W,
          const uint8_t *__restrict__ S, int rows, int cols, int sc, int blk_r, uint32_t bc_m,
          int nt, int tpg, const uint16_t *__restrict__ xt, int cpad)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char xnlds[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const size_t bl_n = (size_t)tpg * XNT * BP;           /* bf16 per B buffer */
    uint16_t *const bl0 = (uint16_t *)xnlds, *const bl1 = bl0 + bl_n;
    unsigned char *buf = xnlds + 4 * bl_n + (size_t)w * XUNIT_B;
    const int row0 = (blockIdx.x * MW + w) * 16;
    const int t0 = blockIdx.y * tpg;
    const int ntok = min(tpg, nt - t0);
    const int g = lane >> 4, col = lane & 15;
    const bool live = row0 < rows;
    const int wrow0 = live ? row0 : 0;
    const int srow = ((UNI ? wrow0 : min(wrow0 + col, rows - 1)) / blk_r) * sc;
    /* this lane's B row per column tile: token 5 n + col / 3, term col % 3;
     * column 15 and columns of tokens past the group read row 0 (their
     * results are never used; unconditional reads keep the steps
     * branch-free) */
    int boff[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int tk = XTOK * n + col / XNT;
        boff[n] = (col < XNT * XTOK && tk < ntok) ? (tk * XNT + col % XNT) * BP : 0;
    }
    v4f acc[NT], tot[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
        tot[n] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    const int nu = (cols + XU - 1) / XU;
    /* x(u): the pre-split term planes when the caller gave them (copied
     * into LDS as they are), else the f32 row (turned into terms here) */
    constexpr int XM = XpDim<NT, MW>::M > XnDim<NT, MW>::M ? XpDim<NT, MW>::M : XnDim<NT, MW>::M;
    u32x4 XR[XM];                       /* x(u + 1) in flight while unit u runs */
    XUnit<UNI> P[2];
    auto xload = [&](u32x4 *v, int u) {
        if (xt)
            xp_load<NT, MW>(v, xt, t0, ntok, u, cpad, tpg);
        else
            xn_load<NT, MW>(reinterpret_cast<f32x4 *>(v), x, t0, ntok, XU * u, cols, tpg);
    };
    auto xstore = [&](uint16_t *bl, const u32x4 *v, int u) {
        if (xt)
            xp_store<NT, MW>(bl, v, ntok, tpg);
        else
            xn_terms<NT, MW>(bl, reinterpret_cast<const f32x4 *>(v), ntok, XU * u, cols, tpg);
    };
    xload(XR, 0);
    /* uniform scales: the current segment's (ssb) and the next one's */
    uint32_t ssb = UNI ? xs_seg(S, srow, bc_m, 0, cols, lane) : 0u, ssn = 0u;
    __builtin_amdgcn_sched_barrier(0);
    xu_load<UNI, false>(P[0], W, S, srow, bc_m, wrow0, rows, cols, 0, lane);
    xu_load<UNI, false>(P[1], W, S, srow, bc_m, wrow0, rows, cols, XU * min(1, nu - 1), lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int s0 = 0; s0 < nu; s0 += XSEG_U) {
        const float sfb = UNI ? dec_e8m0(ssb) : 0.0f;   /* this segment's scales */
#pragma unroll
        for (int j = 0; j < XSEG_U; j++) {
            const int u = s0 + j;
            uint16_t *bl = (j & 1) ? bl1 : bl0;
            if (u < nu) {
                xstore(bl, XR, u);
                xu_stage(buf, P[j & 1], lane);
            }
            uint32_t sb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) sb[q] = UNI ? 0u : P[j & 1].sb[UNI ? 0 : q];
            /* x(u + 1) before weight unit u + 2, both unconditional (past
             * the last unit they repeat it, unused): the wait for x(u + 1)
             * then leaves unit u + 2 in flight, and no load sits in a branch
             * that would make the waits fall back to waiting for all */
            __builtin_amdgcn_sched_barrier(0);
            xload(XR, min(u + 1, nu - 1));
            if (UNI && j == XSEG_U - 2)        /* before the next segment's first unit */
                ssn = xs_seg(S, srow, bc_m, XU * (min(s0 + XSEG_U, nu - 1) & ~(XSEG_U - 1)),
                             cols, lane);
            __builtin_amdgcn_sched_barrier(0);
            xu_load<UNI, false>(P[j & 1], W, S, srow, bc_m, wrow0, rows, cols,
                                XU * min(u + 2, nu - 1), lane);
            __builtin_amdgcn_sched_barrier(0);
            if (u < nu) {
                __syncthreads();          /* B(u) whole; every wave is past B(u - 2)'s reads */
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int k = XU * u + 64 * q + 16 * g;
                    v8bf af[2];
                    if (UNI)
                        xu_frags_f(af, buf, q, xs_getf(sfb, 4 * j + q), k < cols, lane);
                    else
                        xu_frags(af, buf, q, sb[q], k < cols, lane);
#pragma unroll
                    for (int h = 0; h < 2; h++) {
#pragma unroll
                        for (int n = 0; n < NT; n++) {
                            const u32x4 bw = *reinterpret_cast<const u32x4 *>(
                                bl + boff[n] + 64 * q + 16 * g + 8 * h);
                            acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                af[h], __builtin_bit_cast(v8bf, bw), acc[n], 0, 0, 0);
                        }
                    }
                }
            }
        }
        /* a segment ends: its partials join the running sums in order */
#pragma unroll
        for (int n = 0; n < NT; n++) {
            tot[n] = s0 == 0 ? acc[n] : tot[n] + acc[n];
            acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        ssb = ssn;
    }
    if (!live) return;
    /* y = (hi + mid) + lo per (row, token): column 3 s of a tile gathers its
     * token's three columns from the two lanes after it */
#pragma unroll
    for (int n = 0; n < NT; n++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float c0 = tot[n][j];
            const float c1 = __shfl(tot[n][j], min(lane + 1, 63), 64);
            const float c2 = __shfl(tot[n][j], min(lane + 2, 63), 64);
            const int tk = XTOK * n + col / XNT;
            const int rr = row0 + 4 * g + j;
            if (col % XNT == 0 && col < XNT * XTOK && tk < ntok && rr < rows)
                y[(size_t)(t0 + tk) * rows + rr] = (c0 + c1) + c2;
        }
    }
}

/* The batched kernel with its operands staged by direct-to-LDS loads
 * (k_fp8_mxd; uniform scales, pre-split x terms). A workgroup of MW waves
 * owns 16 MW rows (MW tiles) and a group of tokens in one of two layouts:
 *  - up to 20 tokens in 4 column tiles of five (token j in columns 3 j ..
 *    3 j + 2, column 15 unused); wave w takes RT x CT = 2 x 2 tiles, so
 *    each A fragment feeds two column tiles and each B fragment two row
 *    tiles;
 *  - planar (CT = 3): up to 16 tokens, column tile n holding term n of
 *    every token (token = column), so every column is used; wave w takes
 *    its row tile and all three, and a token's terms meet in one lane.
 *
 * The K axis runs in stages of 128 columns (half a unit): the workgroup's
 * weight rows x 128 bytes and its group's term rows (60 or 48) x 128 bf16,
 * copied by
 * global_load_lds_dwordx4 (each lane's 16 bytes land at the instruction's
 * LDS base + 16 lane, so nothing in flight holds a register) into a ring of
 * NS stages, NS - 1 of them in flight while one is read. Each lane fetches
 * the piece that the swizzled layout puts in its slot: weight piece c of
 * row R sits at piece c ^ (R & 7) of its 128-byte row (an in-bounds LDS
 * probe on MI355X: 437-495 GB/s per CU against 146 and 76 with the rows
 * unswizzled; SQ_LDS_BANK_CONFLICT counts none on these reads). Groups of
 * 20 keep term piece c of term row j at c ^ (j & 15) of its 256-byte row,
 * which still costs about 3 conflict cycles per term read. The planar
 * groups keep each term row as two 128-byte half rows, ordered (term, K
 * half, token), with the piece a lane group g reads for MFMA h at slot
 * (4 h + g) ^ (token & 7): a fragment read then takes 16 consecutive half
 * rows and, across its four lane groups, four consecutive slots, as the
 * weight reads do, and counts no conflicts (it counted 4 cycles per read
 * with whole 256-byte rows: 64 tokens 40.6 -> 36.7 us). A wave
 * reads stage s's fragments into one register set while the set read at
 * stage s - 1 runs through the matrix core, so the reads' latency hides
 * behind a stage of MFMAs.
 *
 * On a SIMD the VALU and the scalar unit's work adds to the matrix core's
 * time, so the per-stage path is kept short: the segment's scales are
 * decoded once per segment, each lane's read offsets and load pointers are
 * formed once, and whole segments are unrolled so that a stage's place in
 * its segment is a compile-time constant.
 *
 * Per (row, term column) the chain is k_fp8_mxn's: the same K steps (whole
 * units, zero operands past cols), the same fragments, one accumulator per
 * segment from zero, the segments joined in order and y = (hi + mid) + lo,
 * so the bits are the same. */
constexpr int XD_K = 128;                        /* K (weight bytes) per stage */
constexpr int XD_TR = XTOK * 4 * XNT;            /* term rows per stage (60)   */
constexpr int XP_TOK = 16;                       /* tokens per planar group    */
constexpr int XP_TR = XP_TOK * XNT;              /* its term rows (48)         */

/* MW waves own 16 MW rows; a stage is their weights and the group's TR term
 * rows; NS stages in the ring */
template <int MW, int TR = XD_TR>
struct XdDim {
    static constexpr int R = 16 * MW;                    /* rows per workgroup   */
    static constexpr int WB = R * XD_K;                  /* weight bytes / stage */
    static constexpr int SB = WB + TR * XD_K * 2;        /* bytes per stage      */
    static constexpr int DX = (TR / 4 + MW - 1) / MW;    /* term loads per wave  */
    static constexpr int DPW = 2 + DX;                   /* loads per wave/stage */
};
template <int MW, int NS, int TR = XD_TR>
constexpr size_t xd_lds() { return (size_t)NS * XdDim<MW, TR>::SB; }

typedef __attribute__((address_space(3))) void lds_void;

template <int N>
__device__ __forceinline__ void xd_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/* this wave's loads older than its newest `ahead` stages (DPW loads each)
 * are complete (the loop's only memory requests are the stage loads) */
template <int DPW>
__device__ __forceinline__ void xd_wait(int ahead)
{
    if (ahead >= 3) xd_vm<3 * DPW>();
    else if (ahead == 2) xd_vm<2 * DPW>();
    else if (ahead == 1) xd_vm<DPW>();
    else xd_vm<0>();
}

template <int RT, int CT, int MW, int NS>
__global__ void __launch_bounds__(64 * MW)
k_fp8_mxd(float *__restrict__ y, const uint8_t *__restrict__ W, const uint8_t *__restrict__ S,
          int rows, int cols, int sc, int blk_r, uint32_t bc_m, int nt, int tpg,
          const uint16_t *__restrict__ xt, int cpad)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char xdlds[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    /* PL: the planar group (XP_TOK tokens, column tile n = term n of every
     * token, token = column); else groups of 20 tokens in 4 column tiles of
     * five (token j in columns 3 j .. 3 j + 2) */
    constexpr bool PL = CT == XNT;
    constexpr int TR = PL ? XP_TR : XD_TR;
    static_assert(PL ? RT == 1 : RT * CT == 4,
                  "MW waves x RT x CT = MW row tiles x 4 column tiles (or x 3 terms, one each)");
    static_assert(NS >= 2 && NS <= 5, "stage waits for up to 3 stages ahead");
    using D = XdDim<MW, TR>;
    const int rp = w % (MW / RT), ch = w / (MW / RT);
    const int row0 = blockIdx.x * D::R;
    const int t0 = blockIdx.y * tpg;
    const int ntok = min(tpg, nt - t0);
    if (ntok <= 0) return;                           /* the whole workgroup */
    const int g = lane >> 4, col = lane & 15;
    const int nst = 2 * ((cols + XU - 1) / XU);      /* whole units, as k_fp8_mxn */

    /* the loads: weight instructions 2w, 2w + 1 (rows 8 i .. 8 i + 7 of the
     * workgroup, lane -> row 8 i + lane / 8, slot lane % 8) and term
     * instructions DX w + i, at most TR / 4 - 1 (term rows 4 i .. 4 i + 3, lane ->
     * row 4 i + lane / 16, slot lane % 16); rows past the matrix read its
     * last row, term rows past the group's tokens its first (never used) */
    constexpr int DH = 2, DX = D::DX;                /* loads of each kind    */
    const uint8_t *wsrc[DH], *wrow[DH];
    int wcol[DH], xoff[DX];
    const uint16_t *xsrc[DX];
#pragma unroll
    for (int i = 0; i < DH; i++) {
        const int R = 8 * (DH * w + i) + (lane >> 3);
        wcol[i] = 16 * ((lane & 7) ^ (R & 7));
        wrow[i] = W + (size_t)min(row0 + R, rows - 1) * cols;
        wsrc[i] = wrow[i] + wcol[i];
    }
#pragma unroll
    for (int i = 0; i < DX; i++) {
        const int xi = min(DX * w + i, TR / 4 - 1);
        if constexpr (PL) {
            /* planar: 128-byte half rows r = 16 (2 n + qq) + t (term n, K half
             * qq, token t); piece 2 g + h of a half row (lane group g's piece
             * for MFMA h) at slot (4 h + g) ^ (r & 7), so each fragment read
             * takes four consecutive slots across its lane groups; lane ->
             * half row 8 i + lane / 8, slot lane % 8 */
            const int r = 8 * xi + (lane >> 3);
            const int n = r >> 5, qq = (r >> 4) & 1, t = r & 15;
            const int jj = t < ntok ? XNT * t + n : 0;
            const int q = (lane & 7) ^ (t & 7);
            xsrc[i] = xt + ((size_t)t0 * XNT + jj) * cpad + 8 * (8 * qq + 2 * (q & 3) + (q >> 2));
        } else {
            const int j = 4 * xi + (lane >> 4);
            const int jj = j / XNT < ntok ? j : 0;
            xsrc[i] = xt + ((size_t)t0 * XNT + jj) * cpad + 8 * ((lane & 15) ^ (j & 15));
        }
        xoff[i] = D::WB + 1024 * xi;
    }
    /* FULL: the caller knows the whole stage lies inside the rows */
    auto issue = [&](int s, int slot, auto full) {
        unsigned char *st = xdlds + (size_t)slot * D::SB;
        const int k0 = XD_K * s;
        if (decltype(full)::value || k0 + XD_K <= cols) {
#pragma unroll
            for (int i = 0; i < DH; i++)
                __builtin_amdgcn_global_load_lds((const void *)(wsrc[i] + k0),
                                                 (lds_void *)(st + 1024 * (DH * w + i)), 16, 0,
                                                 0);
        } else {
#pragma unroll
            for (int i = 0; i < DH; i++) {
                const int k = k0 + wcol[i];
                __builtin_amdgcn_global_load_lds((const void *)(wrow[i] + (k < cols ? k : 0)),
                                                 (lds_void *)(st + 1024 * (DH * w + i)), 16, 0,
                                                 0);
            }
        }
#pragma unroll
        for (int i = 0; i < DX; i++)
            __builtin_amdgcn_global_load_lds((const void *)(xsrc[i] + k0),
                                             (lds_void *)(st + xoff[i]), 16, 0, 0);
    };

    /* the fragment reads: A row 16 a + col of tile a = RT rp + i; B term row
     * 15 n + min(col, 14) of column tile n = CT ch + jn (column 15 repeats
     * column 14; its result is never used), or in the planar group half row
     * 16 (2 n + qq) + col (token col, term n) */
    int aoff[RT], asw[RT], boff[CT], bsw[CT];
    bool live[RT];
    int srow[RT];
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const int R = 16 * (RT * rp + i) + col;
        aoff[i] = R * XD_K;
        asw[i] = R & 7;
        const int tr0 = row0 + 16 * (RT * rp + i);
        live[i] = tr0 < rows;
        srow[i] = ((live[i] ? tr0 : 0) / blk_r) * sc;
    }
#pragma unroll
    for (int n = 0; n < CT; n++) {
        const int j = PL ? XNT * col + n : 15 * (CT * ch + n) + min(col, 14);
        boff[n] = D::WB + j * (2 * XD_K);
        bsw[n] = j & 15;
    }
    v4f acc[RT][CT], tot[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int n = 0; n < CT; n++) {
            acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};
            tot[i][n] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < nst) issue(s, s, std::false_type{});
    __builtin_amdgcn_sched_barrier(0);
    /* every segment's scales for the wave's row tiles, requested once behind
     * the first stages (the loop then issues no memory request the compiler
     * waits for, so its only waits on the memory counter are the stage
     * waits): segment z, quarter m is byte z / 4 of sr[i] in lane 16 (z % 4)
     * + m */
    uint32_t sr[RT];
#pragma unroll
    for (int i = 0; i < RT; i++) {
        sr[i] = 0u;
#pragma unroll
        for (int b = 0; b < XSEG_MAX / 4; b++)
            sr[i] |= xs_seg(S, srow[i], bc_m, XSEG * (4 * b + (lane >> 4)), cols, lane) << (8 * b);
    }

    /* Stage s: wait for its loads, one barrier (every wave's loads of s are
     * in LDS, and every wave's reads of s - 1 are complete, so s - 1's slot
     * takes stage s + NS - 1), then read s's fragments into one register
     * set while the other set, read one stage earlier, runs through the
     * matrix core: the fragment reads' latency hides behind a stage of
     * MFMAs. */
    struct Ops {
        u32x4 a[RT][2];                          /* [row tile][quarter]        */
        u32x4 b[2][2][CT];                       /* [quarter][step][col tile]  */
    };
    /* the slot of stage s (s % NS), kept as a running count */
    auto sync = [&](int s, int slot) {
        xd_wait<D::DPW>(min(NS - 2, nst - 1 - s));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (s + NS - 1 < nst) issue(s + NS - 1, slot == 0 ? NS - 1 : slot - 1, std::false_type{});
    };
    /* the same where stage s + NS - 1 exists and lies inside the rows */
    auto sync_deep = [&](int s, int slot) {
        xd_vm<(NS - 2) * D::DPW>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(s + NS - 1, slot == 0 ? NS - 1 : slot - 1, std::true_type{});
    };
    /* each read's lane offset within a stage, formed once */
    int fa[RT][2], fb[2][2][CT];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int qq = 0; qq < 2; qq++) fa[i][qq] = aoff[i] + 16 * ((4 * qq + g) ^ asw[i]);
#pragma unroll
    for (int qq = 0; qq < 2; qq++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int n = 0; n < CT; n++)
                fb[qq][h][n] = PL ? D::WB + (16 * (2 * n + qq) + col) * 128 +
                                        16 * ((4 * h + g) ^ (col & 7))
                                  : boff[n] + 16 * ((8 * qq + 2 * g + h) ^ bsw[n]);
    auto fetch = [&](Ops &o, int slot) {
        const unsigned char *st = xdlds + (size_t)slot * D::SB;
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int qq = 0; qq < 2; qq++)
                o.a[i][qq] = *reinterpret_cast<const u32x4 *>(st + fa[i][qq]);
#pragma unroll
        for (int qq = 0; qq < 2; qq++)
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int n = 0; n < CT; n++)
                    o.b[qq][h][n] = *reinterpret_cast<const u32x4 *>(st + fb[qq][h][n]);
    };
    /* one stage through the matrix core; FULL: every column of the stage
     * is inside the row (no piece to zero) */
    /* the current segment's 16 quarter scales per row tile, decoded: lane 16
     * (z % 4) + m holds quarter m's (set as each segment starts) */
    float sf[RT];
#pragma unroll
    for (int i = 0; i < RT; i++) sf[i] = 0.0f;
    auto mma = [&](const Ops &o, int s, auto full) {
        constexpr bool FULL = decltype(full)::value;
        const int sl = s & 7;                    /* stage within its segment */
        const int z = s >> 3;
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const bool in = FULL || XD_K * s + 64 * qq + 16 * g < cols;
            v8bf af[RT][2];
#pragma unroll
            for (int i = 0; i < RT; i++) {
                const u32x4 zv = in ? o.a[i][qq] : u32x4{0u, 0u, 0u, 0u};
                const float sx = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sf[i]),
                                                     16 * (z & 3) + 2 * sl + qq));
                const float sv = in ? sx : 0.0f;
                af[i][0] = fp8x8_bf16(zv.x, zv.y, sv);
                af[i][1] = fp8x8_bf16(zv.z, zv.w, sv);
            }
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int i = 0; i < RT; i++)
#pragma unroll
                    for (int n = 0; n < CT; n++)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            af[i][h], __builtin_bit_cast(v8bf, o.b[qq][h][n]), acc[i][n], 0, 0,
                            0);
        }
    };
    auto run = [&](const Ops &o, int s) {
        if ((s & 7) == 0) {                      /* a segment starts: its scales */
            asm volatile("" ::: "memory");
            const int z = s >> 3;
#pragma unroll
            for (int i = 0; i < RT; i++) sf[i] = dec_e8m0((sr[i] >> (8 * (z >> 2))) & 0xffu);
        }
        if (XD_K * (s + 1) <= cols)
            mma(o, s, std::true_type{});
        else
            mma(o, s, std::false_type{});
        if ((s & 7) == 7 || s == nst - 1) {      /* a segment ends */
            asm volatile("" ::: "memory");       /* a branch, not selects on every stage */
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int n = 0; n < CT; n++) {
                    tot[i][n] = s < 8 ? acc[i][n] : tot[i][n] + acc[i][n];
                    acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};
                }
        }
    };
    Ops o0, o1;
    sync(0, 0);
    fetch(o0, 0);
    int slot = 1;
    auto next = [&](int q) { return q + 1 == NS ? 0 : q + 1; };
    /* Whole segments first: group z runs stages 8z .. 8z + 7 (every column
     * inside the rows) while stages 8z + 1 .. 8z + 8 are waited for and
     * read, so each step's place in its segment is a compile-time constant
     * and the segment's start and end need no test per stage. */
    auto seg_step = [&](int z, auto jc, auto deep) {
        constexpr int j = decltype(jc)::value;
        const int r = 8 * z + j;                 /* the stage run; r + 1 is read */
        Ops &of = (j & 1) ? o0 : o1;
        const Ops &orun = (j & 1) ? o1 : o0;
        if constexpr (decltype(deep)::value)
            sync_deep(r + 1, slot);
        else
            sync(r + 1, slot);
        fetch(of, slot);
        if constexpr (j == 0) {
#pragma unroll
            for (int i = 0; i < RT; i++) sf[i] = dec_e8m0((sr[i] >> (8 * (z >> 2))) & 0xffu);
        }
        mma(orun, r, std::true_type{});
        if constexpr (j == 7) {
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int n = 0; n < CT; n++) {
                    tot[i][n] = z == 0 ? acc[i][n] : tot[i][n] + acc[i][n];
                    acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};
                }
        }
        slot = next(slot);
    };
    auto segment = [&](int z, auto deep) {
        seg_step(z, std::integral_constant<int, 0>{}, deep);
        seg_step(z, std::integral_constant<int, 1>{}, deep);
        seg_step(z, std::integral_constant<int, 2>{}, deep);
        seg_step(z, std::integral_constant<int, 3>{}, deep);
        seg_step(z, std::integral_constant<int, 4>{}, deep);
        seg_step(z, std::integral_constant<int, 5>{}, deep);
        seg_step(z, std::integral_constant<int, 6>{}, deep);
        seg_step(z, std::integral_constant<int, 7>{}, deep);
    };
    /* deep: every stage the group requests (up to 8z + 8 + NS - 1) exists and
     * lies inside the rows, so its waits and loads need no test */
    int z = 0;
    for (; 8 * z + 8 + NS - 1 < nst && (8 * z + 8 + NS) * XD_K <= cols; z++)
        segment(z, std::true_type{});
    for (; 8 * z + 8 < nst && (8 * z + 8) * XD_K <= cols; z++)
        segment(z, std::false_type{});
    /* the rest stage by stage (nst is even: stages 1, 2 | 3, 4 | ... pair up,
     * and the last is odd) */
    int s = 8 * z + 1;
    for (; s + 1 < nst; s += 2) {
        sync(s, slot);
        fetch(o1, slot);
        run(o0, s - 1);
        slot = next(slot);
        sync(s + 1, slot);
        fetch(o0, slot);
        run(o1, s);
        slot = next(slot);
    }
    sync(s, slot);
    fetch(o1, slot);
    run(o0, s - 1);
    run(o1, s);
    /* y = (hi + mid) + lo per (row, token), as k_fp8_mxn */
    if constexpr (PL) {
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int rr = row0 + 16 * (RT * rp + i) + 4 * g + j;
                if (live[i] && col < ntok && rr < rows)
                    y[(size_t)(t0 + col) * rows + rr] = (tot[i][0][j] + tot[i][1][j]) + tot[i][2][j];
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int n = 0; n < CT; n++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float c0 = tot[i][n][j];
                const float c1 = __shfl(tot[i][n][j], min(lane + 1, 63), 64);
                const float c2 = __shfl(tot[i][n][j], min(lane + 2, 63), 64);
                const int tk = XTOK * (CT * ch + n) + col / XNT;
                const int rr = row0 + 16 * (RT * rp + i) + 4 * g + j;
                if (live[i] && col % XNT == 0 && col < XNT * XTOK && tk < ntok && rr < rows)
                    y[(size_t)(t0 + tk) * rows + rr] = (c0 + c1) + c2;
            }
}

/* The batched kernel for one column tile (at most five tokens) with each
 * tile's segments split over KP waves, as the single-token kernel splits
 * them: a workgroup of 4 waves holds 4 / KP tiles, and wave p of a tile takes
 * units [p up, (p + 1) up), up = spw segments of 4 units. Step i: the
 * workgroup copies the pre-split x terms of unit p up + i of every part p
 * into B buffer i % 2 (part p's rows after part p - 1's), each wave stages
 * its weight unit and requests the next x step and its weight unit i + 2,
 * and after one barrier runs its unit's 8 steps. Part 0 chains its segments
 * in registers; the other parts leave each segment's accumulator in LDS, and
 * part 0 continues its chain over them in segment order after a barrier: the
 * chain of k_fp8_mxn, so the same bits. */
template <int KP, bool XF>
struct XkDim {
    /* 16-byte pieces per thread per step: term-plane pieces, or with XF f32
     * pieces of the token rows */
    static constexpr int M = XF ? (KP * XTOK * (XU / 4) + 255) / 256
                                : (KP * XTOK * XNT * (XU / 8) + 255) / 256;
};

/* XF: x comes as the f32 rows and each workgroup forms the terms of its
 * steps itself (terms3, the bits of k_fp8_xsplit), so no split launch runs
 * before it. */
template <bool UNI, int KP, bool XF>
__global__ void __launch_bounds__(256)
k_fp8_mxk(float *__restrict__ y, const float *__restrict__ x, const uint8_t *__restrict__ W,
          const uint8_t *__restrict__ S, int rows, int cols, int sc, int blk_r, uint32_t bc_m,
          int nt, int tpg, const uint16_t *__restrict__ xt, int cpad, int spw)
{
    constexpr int MW = 4, TT = MW / KP, XM = XkDim<KP, XF>::M;
    extern __shared__ __attribute__((aligned(16))) unsigned char xklds[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int p = w % KP, tl = w / KP;
    const int prows = tpg * XNT;                            /* B rows per part */
    const size_t bl_n = (size_t)KP * prows * BP;            /* bf16 per B buffer */
    uint16_t *const bl0 = (uint16_t *)xklds, *const bl1 = bl0 + bl_n;
    unsigned char *buf = xklds + 4 * bl_n + (size_t)w * XUNIT_B;
    const int nu = (cols + XU - 1) / XU, nseg = (nu + XSEG_U - 1) / XSEG_U;
    const int up = spw * XSEG_U, ub = p * up;
    v4f *part = (v4f *)(xklds + 4 * bl_n + (size_t)MW * XUNIT_B) +
                (size_t)tl * (nseg - spw) * 64;             /* [nseg - spw][64] */
    const int row0 = (blockIdx.x * TT + tl) * 16;
    const int t0 = blockIdx.y * tpg;
    const int ntok = min(tpg, nt - t0);
    const int g = lane >> 4, col = lane & 15;
    const bool live = row0 < rows;
    const int wrow0 = live ? row0 : 0;
    const int srow = ((UNI ? wrow0 : min(wrow0 + col, rows - 1)) / blk_r) * sc;
    const int boff = (col < XNT * XTOK && col / XNT < ntok)
                         ? (p * prows + col) * BP : p * prows * BP;
    /* this thread's x pieces, step-independent except for the unit. Term
     * planes: piece i = tid + 256 m is part i / 32 / prows, B row (i / 32) %
     * prows, 16-byte piece i % 32. XF: part i / 64 / tpg, token (i / 64) %
     * tpg, f32 columns 4 (i % 64) .. + 3 of the unit. Pieces of tokens past
     * the group (and, XF, columns past cols) load the group's first row and
     * store zeros. */
    int xo[XM], xu0[XM], xs[XM], xc[XM];
    bool xin[XM], xok[XM];
#pragma unroll
    for (int m = 0; m < XM; m++) {
        const int i = (int)threadIdx.x + 256 * m;
        if (XF) {
            const int pr = i / (XU / 4), c4 = i % (XU / 4);
            const int pp = pr / tpg, tk = pr - pp * tpg;
            xs[m] = pr < KP * tpg ? (pp * prows + tk * XNT) * BP + 4 * c4 : -1;
            xin[m] = pr < KP * tpg && tk < ntok;
            xo[m] = xin[m] ? (t0 + tk) * cols + 4 * c4 : t0 * cols;
            xu0[m] = xin[m] ? pp * up : 0;
            xc[m] = 4 * c4;
        } else {
            const int prow = i / (XU / 8), pc = i % (XU / 8);
            const int pp = prow / prows, r = prow - pp * prows;
            xs[m] = prow < KP * prows ? prow * BP + 8 * pc : -1;
            xin[m] = prow < KP * prows && r / XNT < ntok;
            xo[m] = xin[m] ? (t0 * XNT + r) * cpad + 8 * pc : t0 * XNT * cpad;
            xu0[m] = xin[m] ? pp * up : 0;
            xc[m] = 0;
        }
        xok[m] = xin[m];
    }
    u32x4 XR[XM];
    auto xload = [&](int i) {
#pragma unroll
        for (int m = 0; m < XM; m++) {
            const int cu = XU * min(xu0[m] + i, nu - 1);
            if (XF) {
                /* the unit's columns past cols: the group's first piece */
                xok[m] = xin[m] && xc[m] + cu < cols;
                XR[m] = __builtin_bit_cast(u32x4, *(const DSV4_GLOBAL f32x4 *)(
                    x + (xok[m] ? xo[m] + cu : t0 * cols)));
            } else {
                XR[m] = *(const DSV4_GLOBAL u32x4 *)(xt + xo[m] + cu);
            }
        }
    };
    auto xstore = [&](uint16_t *bl) {
#pragma unroll
        for (int m = 0; m < XM; m++) {
            if (xs[m] < 0) continue;
            if (XF) {
                const f32x4 v = __builtin_bit_cast(f32x4, XR[m]);
                const float e[4] = {xok[m] ? v.x : 0.f, xok[m] ? v.y : 0.f, xok[m] ? v.z : 0.f,
                                    xok[m] ? v.w : 0.f};
                uint32_t tt[4][XNT];
#pragma unroll
                for (int j = 0; j < 4; j++) terms3(e[j], tt[j]);
#pragma unroll
                for (int p = 0; p < XNT; p++)
                    *reinterpret_cast<uint2 *>(bl + xs[m] + p * BP) =
                        uint2{tt[0][p] | (tt[1][p] << 16), tt[2][p] | (tt[3][p] << 16)};
            } else {
                *reinterpret_cast<u32x4 *>(bl + xs[m]) = xin[m] ? XR[m] : u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    v4f acc = {0.f, 0.f, 0.f, 0.f}, tot = {0.f, 0.f, 0.f, 0.f};
    XUnit<UNI> P[2];
    xload(0);
    uint32_t ssb = UNI ? xs_seg(S, srow, bc_m, XU * min(ub, nu - 1), cols, lane) : 0u, ssn = 0u;
    __builtin_amdgcn_sched_barrier(0);
    xu_load<UNI, false>(P[0], W, S, srow, bc_m, wrow0, rows, cols, XU * min(ub, nu - 1), lane);
    xu_load<UNI, false>(P[1], W, S, srow, bc_m, wrow0, rows, cols, XU * min(ub + 1, nu - 1), lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int s0 = 0; s0 < up; s0 += XSEG_U) {
        /* this segment's scales, decoded once where that measured faster
         * (4 parts: 2 tokens 15.4 -> 14.9 us, 4 tokens 18.2 -> 17.8; with 2
         * parts, 8 tokens, the scalar decode per quarter stays: 24.0 against
         * 24.5) */
        const float sfb = UNI && KP == 4 ? dec_e8m0(ssb) : 0.0f;
#pragma unroll
        for (int j = 0; j < XSEG_U; j++) {
            const int i = s0 + j, u = ub + i;
            uint16_t *bl = (j & 1) ? bl1 : bl0;
            xstore(bl);
            xu_stage(buf, P[j & 1], lane);
            uint32_t sb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) sb[q] = UNI ? 0u : P[j & 1].sb[UNI ? 0 : q];
            __builtin_amdgcn_sched_barrier(0);
            xload(min(i + 1, up - 1));
            if (UNI && j == XSEG_U - 2)        /* before the next segment's first unit */
                ssn = xs_seg(S, srow, bc_m, XU * (min(ub + s0 + XSEG_U, nu - 1) & ~(XSEG_U - 1)),
                             cols, lane);
            __builtin_amdgcn_sched_barrier(0);
            xu_load<UNI, false>(P[j & 1], W, S, srow, bc_m, wrow0, rows, cols,
                                XU * min(u + 2, nu - 1), lane);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();              /* B(i) whole; every wave is past B(i - 2)'s reads */
            if (u < nu) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int k = XU * u + 64 * q + 16 * g;
                    v8bf af[2];
                    if (UNI && KP == 4)
                        xu_frags_f(af, buf, q, xs_getf(sfb, 4 * j + q), k < cols, lane);
                    else
                        xu_frags(af, buf, q,
                                 UNI ? (uint32_t)__builtin_amdgcn_readlane((int)ssb, 4 * j + q)
                                     : sb[q],
                                 k < cols, lane);
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const u32x4 bw = *reinterpret_cast<const u32x4 *>(
                            bl + boff + 64 * q + 16 * g + 8 * h);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            af[h], __builtin_bit_cast(v8bf, bw), acc, 0, 0, 0);
                    }
                }
            }
        }
        /* a segment ends: part 0 chains it, the others leave it in LDS */
        const int sg = p * spw + s0 / XSEG_U;
        if (p == 0)
            tot = s0 == 0 ? acc : tot + acc;
        else if (sg < nseg)
            part[(size_t)(sg - spw) * 64 + lane] = acc;
        acc = v4f{0.f, 0.f, 0.f, 0.f};
        ssb = ssn;
    }
    __syncthreads();                      /* every part's segments in LDS */
    if (p != 0 || !live) return;
    for (int s = spw; s < nseg; s++) tot = tot + part[(size_t)(s - spw) * 64 + lane];
    /* y = (hi + mid) + lo per (row, token), as k_fp8_mxn */
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float c0 = tot[j];
        const float c1 = __shfl(tot[j], min(lane + 1, 63), 64);
        const float c2 = __shfl(tot[j], min(lane + 2, 63), 64);
        const int tk = col / XNT;
        const int rr = row0 + 4 * g + j;
        if (col % XNT == 0 && col < XNT * XTOK && tk < ntok && rr < rows)
            y[(size_t)(t0 + tk) * rows + rr] = (c0 + c1) + c2;
    }
}

/* Every row of a 16-row tile and every lane of a quarter share the quarter's
 * scale: tiles start at multiples of 16 and quarters at multiples of 64. */
bool xs_uniform(int blk_r, int blk_c)
{
    return blk_r % 16 == 0 && blk_c % 64 == 0;
}

/* Opt a kernel in to the device's whole LDS for its dynamic allocation;
 * false (with a message) when the runtime refuses, so that no launch asks
 * for more than the kernel was granted. */
template <typename K>
bool optin(K kernel, const char *name)
{
    return dsv4_lds_optin((const void *)kernel, dsv4_lds_limit(), name);
}

int mx_cu_count()
{
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

int mx_env(const char *name, int dflt)
{
    const char *e = getenv(name);
    return e ? atoi(e) : dflt;
}

/* Launch shape of k_fp8_mx1 for rows x cols (n groups): waves per tile P
 * (rows past 8 segments: 8 waves of two segments; else the smallest of 1,
 * 2, 4 and nseg that gives `target` waves in all, else nseg), segments per
 * wave, tiles per workgroup (8 waves a workgroup, or P when P does not
 * divide 8; halved while that leaves most CUs idle), the x planes' pitch,
 * LDS bytes and the persistent grid (at most
 * what fits on the CUs at once). Measured on MI355X (E8M0, cold weights):
 * 7168 x 7168 is fastest at P 4 x 2 tiles, 24576 x 1536 at P 1 x 8 tiles,
 * 7168 x 16384 at P 8, the LM head at P 1. */
bool mx1_config(int rows, int cols, int n, Dsv4Fp8Mx *b)
{
    const int ntiles = (rows + 15) / 16;
    const int nseg = (cols + XSEG - 1) / XSEG, nu_all = (cols + XU - 1) / XU;
    const int target = mx_env("DSV4_GPU_MX_WAVES", 1536);
    const int cand[4] = {1, 2, 4, nseg};
    int P = nseg > 8 ? 8 : 0;
    for (int i = 0; i < 4 && !P; i++) {
        const int c = cand[i];
        if (c > nseg || c > 8) continue;
        const int spw = (nseg + c - 1) / c;
        if ((long long)ntiles * ((nseg + spw - 1) / spw) * n >= target) P = c;
    }
    if (!P) P = nseg;
    const int force = mx_env("DSV4_GPU_MX_P", 0);
    if (force >= 1 && force <= 8 && force <= nseg) P = force;
    int spw = 0, tpw = 0, nw = 0;
    for (int pass = 0; pass < 2; pass++) {
        spw = (nseg + P - 1) / P;
        P = (nseg + spw - 1) / spw;                    /* no wave without a segment */
        tpw = 8 / P;
        if (tpw < 1) tpw = 1;
        /* fewer tiles per workgroup while the grid would leave more than half
         * the CUs without one (1024 x 4096: 7.95 -> 6.44 us, 8192 x 1024:
         * 7.75 -> 6.3 us; 7168 x 7168, with 224 workgroups of two tiles,
         * keeps them: one tile each measured 13.7 against 12.9 us) */
        while (tpw > 1 && (long long)((ntiles + tpw - 1) / tpw) * n < mx_cu_count() / 2)
            tpw /= 2;
        const int ft = mx_env("DSV4_GPU_MX_TPW", 0);
        if (ft >= 1 && ft * P <= 8) tpw = ft;
        if (tpw > ntiles) tpw = ntiles;
        nw = P * tpw;
        if (nw * 64 * X1_XM >= nu_all * (XU / 4)) break;   /* x staging coverage */
        if (pass) return false;
        P = nseg < 8 ? nseg : 8;                       /* the most waves per tile */
    }
    const int xp = nu_all * XU + 8;
    const int ngrp = (ntiles + tpw - 1) / tpw;
    const size_t base = (size_t)XNT * xp * 2 + (size_t)nw * XUNIT_B;
    const size_t pbuf = (size_t)tpw * (nseg - spw) * 16 * XNT * sizeof(float);
    /* one partials buffer when every tile group gets its own workgroup */
    const size_t cap = dsv4_lds_limit();
    const int per_cu1 = base + pbuf <= cap / 2 ? 2 : 1;
    int npb = 2, gx = 0;
    if ((long long)per_cu1 * mx_cu_count() >= (long long)ngrp * n) {
        npb = 1;
        gx = ngrp;
    }
    const size_t lds = base + npb * pbuf;
    if (lds > cap) return false;
    if (!gx) {
        const int per_cu = lds <= cap / 2 ? 2 : 1;
        gx = (per_cu * mx_cu_count() + n - 1) / n;
        if (gx > ngrp) gx = ngrp;
    }
    b->wpt = P; b->spw = spw; b->tpw = tpw; b->xp = xp; b->gx = gx; b->lds = lds; b->npb = npb;
    return true;
}

} // namespace

bool dsv4_fp8_mx_ok(int sfmt, int cols, int blk_r, int blk_c)
{
    return sfmt == 0 && cols > 0 && (cols % 16) == 0 && cols <= XSEG * XSEG_MAX &&
           blk_r >= 1 && blk_c >= 16 && blk_c <= 65536 && (blk_c % 16) == 0;
}

int dsv4_fp8_mx_launch(const Dsv4Fp8Mx &a, hipStream_t st)
{
    if (!dsv4_fp8_mx_ok(0, a.cols, a.blk_r, a.blk_c) || a.n < 1 || a.n > 65535) {
        DSV4_ERR("fp8 mx: shape not taken (cols %d, blk %dx%d)", a.cols, a.blk_r, a.blk_c);
        return -1;
    }
    int rmax = a.rows;
    if (a.list)
        for (int i = 0; i < a.n; i++) rmax = a.rl[i] > rmax ? a.rl[i] : rmax;
    if (rmax <= 0) return 0;
    Dsv4Fp8Mx b = a;
    if (!mx1_config(rmax, a.cols, a.n, &b)) {
        DSV4_ERR("fp8 mx: no launch shape for %dx%d", rmax, a.cols);
        return -1;
    }
    b.bc_m = bc_magic(a.blk_c);
    /* once per process: 1 granted, -1 refused (launches past 64 KiB of
     * LDS then fail here instead of reaching the runtime) */
    static int opted = 0;
    if (!opted)
        opted = optin(k_fp8_mx1<false>, "fp8 mx") && optin(k_fp8_mx1<true>, "fp8 mx") ? 1 : -1;
    if (opted < 0 && b.lds > 64 * 1024) {
        DSV4_ERR("fp8 mx: %zu bytes of LDS without the opt-in", b.lds);
        return -1;
    }
    const dim3 grid(b.gx, a.n), block(64 * b.wpt * b.tpw);
    if (xs_uniform(a.blk_r, a.blk_c))
        hipLaunchKernelGGL(k_fp8_mx1<true>, grid, block, b.lds, st, b);
    else
        hipLaunchKernelGGL(k_fp8_mx1<false>, grid, block, b.lds, st, b);
    HIP_OK(hipGetLastError(), "fp8 mx launch");
    return 0;
}

size_t dsv4_fp8_mxn_scratch_bytes(int cols, int nt)
{
    const size_t cpad = (size_t)((cols + XU - 1) / XU) * XU;
    return (size_t)nt * XNT * cpad * 2;
}

int dsv4_fp8_mxn_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S, int rows,
                        int cols, int blk_r, int blk_c, int nt, hipStream_t st, void *xscratch)
{
    if (!dsv4_fp8_mx_ok(0, cols, blk_r, blk_c) || rows <= 0 || nt < 1 || nt > DSV4_MAX_BATCH) {
        DSV4_ERR("fp8 mxn: shape not taken (%dx%d, nt %d)", rows, cols, nt);
        return -1;
    }
    const int sc = (cols + blk_c - 1) / blk_c;
    const uint32_t bc_m = bc_magic(blk_c);
    /* tokens per workgroup: at most 4 column tiles of 5 (the accumulators and
     * running sums of 4 tiles stay in registers); more tokens take more
     * workgroups along y, each reading the weights again. Up to 4 tiles of
     * tokens one tile per workgroup, up to 8 two, then four: a workgroup's
     * per-unit work grows with its tiles, and the extra token groups read the
     * weights from L2 (7168 x 7168, us, against four tiles: 8 tokens 26.7 /
     * 33.2, 16 tokens 33.5 / 50.4, 32 tokens 45.5 / 54.0; 64 tokens keep 4) */
    const int ntile = (nt + XTOK - 1) / XTOK;
    int ntmax = mx_env("DSV4_GPU_MXN_NT", ntile <= 4 ? 1 : ntile <= 8 ? 2 : 4);
    ntmax = ntmax < 1 ? 1 : ntmax > 7 ? 7 : ntmax;
    const int ngrp = (ntile + ntmax - 1) / ntmax;      /* fewest weight passes */
    const int NTc = (ntile + ngrp - 1) / ngrp;         /* then the fewest tiles each */
    const int tpg = XTOK * NTc < nt ? XTOK * NTc : nt;
    const int groups = (nt + tpg - 1) / tpg;
    /* 8 waves of rows per workgroup when there are three or more token
     * groups of four tiles (each workgroup then stages a group's x terms for
     * 128 rows; 7168 x 7168 at nt 64: 75.0 -> 67.4 us), else 4 (at nt 16-32 the
     * extra workgroups of 4 waves are faster: 50.5 vs 57.8 us at nt 16) */
    const int mw = (groups >= 3 && NTc == 4) ? 8 : 4;
    const size_t lds = 2 * (size_t)tpg * XNT * BP * 2 + (size_t)mw * XUNIT_B;
    const dim3 grid((rows + 16 * mw - 1) / (16 * mw), groups);
    static int opted = 0;                          /* 1 granted, -1 refused */
    if (!opted) {
        const char *nm = "fp8 mxn";
        bool ok = optin(k_fp8_mxn<1, false, 4>, nm) && optin(k_fp8_mxn<2, false, 4>, nm) &&
                  optin(k_fp8_mxn<3, false, 4>, nm) && optin(k_fp8_mxn<4, false, 4>, nm) &&
                  optin(k_fp8_mxn<5, false, 4>, nm) && optin(k_fp8_mxn<6, false, 4>, nm) &&
                  optin(k_fp8_mxn<7, false, 4>, nm) && optin(k_fp8_mxn<1, true, 4>, nm) &&
                  optin(k_fp8_mxn<2, true, 4>, nm) && optin(k_fp8_mxn<3, true, 4>, nm) &&
                  optin(k_fp8_mxn<4, true, 4>, nm) && optin(k_fp8_mxn<5, true, 4>, nm) &&
                  optin(k_fp8_mxn<6, true, 4>, nm) && optin(k_fp8_mxn<7, true, 4>, nm) &&
                  optin(k_fp8_mxn<4, false, 8>, nm) && optin(k_fp8_mxn<4, true, 8>, nm);
        opted = ok ? 1 : -1;
    }
    if (opted < 0 && lds > 64 * 1024) {
        DSV4_ERR("fp8 mxn: %zu bytes of LDS without the opt-in", lds);
        return -1;
    }
    const bool uni = xs_uniform(blk_r, blk_c);
    const int cpad = ((cols + XU - 1) / XU) * XU;
    const uint16_t *xt = (const uint16_t *)xscratch;
    auto xsplit = [&]() {
        const int n8 = nt * (cpad / 8);
        hipLaunchKernelGGL(k_fp8_xsplit, dim3((n8 + 255) / 256), dim3(256), 0, st,
                           (uint16_t *)xscratch, x, nt, cols, cpad);
        return hipGetLastError();
    };
    /* one column tile per group, one or two groups: the segments of a tile
     * split over KP waves, 4 when two workgroups still fit a CU, else 2
     * (7168 x 7168, us, against one wave per tile: 2 tokens 17.2 / 25.3, 4
     * tokens 18.2 / 25.8, 8 tokens (two groups, KP 2) 24.1 / 26.7; with more
     * groups the one-wave form is faster: 16 tokens 33.5 against 42.6 at KP 2).
     * DSV4_GPU_MXK = 0 keeps one wave per tile, 2 or 4 forces KP. */
    const int nseg = (cpad / XU + XSEG_U - 1) / XSEG_U;
    auto mxk_lds = [&](int k) {
        const int spw = (nseg + k - 1) / k;
        return 4 * (size_t)k * tpg * XNT * BP + 4 * (size_t)XUNIT_B +
               (size_t)(4 / k) * (nseg - spw) * 64 * sizeof(float) * 4;
    };
    int kp = mx_env("DSV4_GPU_MXK", -1);
    if (kp < 0)
        kp = groups > 2 ? 0 : groups == 2 ? 2 : mxk_lds(4) <= dsv4_lds_limit() / 2 ? 4 : 2;
    /* x as f32 rows, each workgroup forming its terms, for one group of at
     * most three tokens: no split launch (2 tokens 15.6 against 17.4 us);
     * from 4 tokens the per-workgroup terms cost more than the launch (4
     * tokens 18.7 / 18.2, 8 tokens 26.6 / 24.1). DSV4_GPU_MXKF = 0 / 1
     * forces the pre-split planes / the f32 rows. */
    const int xfe = mx_env("DSV4_GPU_MXKF", -1);
    const bool xf = xfe < 0 ? (groups == 1 && tpg <= 3) : xfe != 0;
    if ((xf || xt) && NTc == 1 && (kp == 2 || kp == 4) && nseg >= kp) {
        const int spw = (nseg + kp - 1) / kp, tt = 4 / kp;
        const size_t lds_k = mxk_lds(kp);
        if (lds_k <= dsv4_lds_limit()) {
            static int opted_k = 0;                /* 1 granted, -1 refused */
            if (!opted_k) {
                const char *nm = "fp8 mxk";
                const bool ok =
                    optin(k_fp8_mxk<false, 2, false>, nm) && optin(k_fp8_mxk<true, 2, false>, nm) &&
                    optin(k_fp8_mxk<false, 4, false>, nm) && optin(k_fp8_mxk<true, 4, false>, nm) &&
                    optin(k_fp8_mxk<false, 2, true>, nm) && optin(k_fp8_mxk<true, 2, true>, nm) &&
                    optin(k_fp8_mxk<false, 4, true>, nm) && optin(k_fp8_mxk<true, 4, true>, nm);
                opted_k = ok ? 1 : -1;
            }
            if (opted_k < 0 && lds_k > 64 * 1024) {
                DSV4_ERR("fp8 mxk: %zu bytes of LDS without the opt-in", lds_k);
                return -1;
            }
            if (!xf) HIP_OK(xsplit(), "fp8 mxn x split launch");
            const dim3 gk(((rows + 15) / 16 + tt - 1) / tt, groups);
#define XK(U, K, F) hipLaunchKernelGGL((k_fp8_mxk<U, K, F>), gk, dim3(256), lds_k, st, y, x, W, \
                                       S, rows, cols, sc, blk_r, bc_m, nt, tpg, xt, cpad, spw)
#define XKF(U, K) do { if (xf) XK(U, K, true); else XK(U, K, false); } while (0)
            if (kp == 2) { if (uni) XKF(true, 2); else XKF(false, 2); }
            else { if (uni) XKF(true, 4); else XKF(false, 4); }
#undef XKF
#undef XK
            HIP_OK(hipGetLastError(), "fp8 mxk launch");
            return 0;
        }
    }
    /* the DMA-staged kernel (uniform scales, pre-split terms) wherever the
     * segment split above did not take the batch. 7168 x 7168, us, against
     * the register-staged kernel: 64 tokens 43.1-43.5 / 62.4-64.3, 41
     * tokens 40.8-41.2 / 54.5-54.9, 32 tokens 30.4 / 45.2-45.5, 16 tokens
     * 28.0-28.1 / 33.4-33.6, 11 tokens 27.7-27.9 / 32.0 (groups of 20).
     * Planar groups of 16 tokens (3 column tiles, all used) against groups
     * of 20 (4 tiles; 16 tokens fill 48 of their 64 columns): 64 tokens
     * 40.6-40.8 / 42.9-43.4, 60 tokens 40.4-40.9 / 41.6-41.8, 41 tokens
     * 37.4-37.6 / 40.7, 24 tokens 27.8-28.1 / 29.9-30.0, 17 tokens 27.1-27.2
     * / 28.0-28.1, 11 tokens 24.5-24.7 / 27.8-28.0; but 40 tokens 37.5 /
     * 30.2-30.4, where two groups of 20 (8 tiles) beat three of 16 (9), so
     * the groups of 20 run where they take two or more groups and fewer
     * tiles (with the planar term reads free of bank conflicts: 64 tokens
     * 36.5-37.1, 20 tokens 25.7-25.8 / 28.1-28.2, 40 tokens 32.7 /
     * 30.6-30.7, 33 tokens 32.3-32.6 / 30.2-30.5). Workgroups: planar, 4
     * waves over 64 rows (64 tokens 40.3-40.9
     * against 42.6-43.5 with 8 waves over 128; 16 tokens 26.2 against 37.9),
     * 2 waves over 32 when there is one group, so that it still covers the
     * CUs (16 tokens 24.8-25.0 against 26.1-26.2); the 4-wave form with a
     * ring of 4 stages (80 KB, two still fit a CU), which the conflict-free
     * term reads made the faster (64 tokens 36.4-36.8 against 36.8-37.0
     * with 3, 48 tokens 32.4-32.7 / 33.2-33.5, 32 tokens 25.7-25.9 /
     * 26.6-26.7; with conflicting reads 4 stages measured no better, 40.5 /
     * 40.3-40.9 and 29.5 / 28.3-28.4). Groups of 20,
     * 8 waves over 128 rows from three groups on (64 tokens: 43.1-43.5
     * against 45.7 with 4 waves), else 4 waves over 64 rows (32 tokens 30.4
     * against 39.1-39.5 with 8 waves, 16 tokens 28.0 against 37.6).
     * DSV4_GPU_MXD = 0 / 1 forces the kernel off / on where it applies,
     * DSV4_GPU_MXD_PL = 0 / 1 the groups, DSV4_GPU_MXD_MW = 2 (planar only)
     * / 4 / 8 the workgroup size. */
    const int g20 = (nt + XTOK * 4 - 1) / (XTOK * 4), g16 = (nt + XP_TOK - 1) / XP_TOK;
    const int dpl = mx_env("DSV4_GPU_MXD_PL", g20 >= 2 && 4 * g20 < XNT * g16 ? 0 : 1);
    const int gtok = dpl ? XP_TOK : XTOK * 4;      /* tokens per group */
    const int gd = (nt + gtok - 1) / gtok;
    const int dme = mx_env("DSV4_GPU_MXD", -1);
    int dmw = mx_env("DSV4_GPU_MXD_MW", dpl ? (gd == 1 ? 2 : 4) : (gd >= 3 ? 8 : 4));
    if (dmw != 2 && dmw != 8) dmw = 4;
    if (!dpl && dmw == 2) dmw = 4;
    const size_t lds_d = dpl ? (dmw == 2   ? xd_lds<2, 3, XP_TR>()
                                : dmw == 4 ? xd_lds<4, 4, XP_TR>()
                                           : xd_lds<8, 5, XP_TR>())
                             : (dmw == 4 ? xd_lds<4, 3>() : xd_lds<8, 5>());
    if (dme != 0 && uni && xt && lds_d <= dsv4_lds_limit()) {
        static int opted_d = 0;                    /* 1 granted, -1 refused */
        if (!opted_d)
            opted_d = optin(k_fp8_mxd<2, 2, 8, 5>, "fp8 mxd") &&
                              optin(k_fp8_mxd<2, 2, 4, 3>, "fp8 mxd") &&
                              optin(k_fp8_mxd<1, 3, 8, 5>, "fp8 mxd") &&
                              optin(k_fp8_mxd<1, 3, 4, 4>, "fp8 mxd") &&
                              optin(k_fp8_mxd<1, 3, 2, 3>, "fp8 mxd")
                          ? 1
                          : -1;
        if (opted_d > 0) {
            const int td = (nt + gd - 1) / gd;      /* tokens spread evenly */
            HIP_OK(xsplit(), "fp8 mxn x split launch");
#define XD(RT, CT, MWV, NSV) hipLaunchKernelGGL((k_fp8_mxd<RT, CT, MWV, NSV>),                 \
                                                dim3((rows + 16 * MWV - 1) / (16 * MWV), gd),   \
                                                dim3(64 * MWV), lds_d, st, y, W, S, rows, cols,  \
                                                sc, blk_r, bc_m, nt, td, xt, cpad)
            if (dpl) {
                if (dmw == 2) XD(1, 3, 2, 3);
                else if (dmw == 4) XD(1, 3, 4, 4);
                else XD(1, 3, 8, 5);
            } else {
                if (dmw == 4) XD(2, 2, 4, 3);
                else XD(2, 2, 8, 5);
            }
#undef XD
            HIP_OK(hipGetLastError(), "fp8 mxd launch");
            return 0;
        }
    }
    if (xt) HIP_OK(xsplit(), "fp8 mxn x split launch");
#define XN(NTV, MWV) do {                                                                      \
        if (uni)                                                                               \
            hipLaunchKernelGGL((k_fp8_mxn<NTV, true, MWV>), grid, dim3(64 * MWV), lds, st, y, x,  \
                               W, S, rows, cols, sc, blk_r, bc_m, nt, tpg, xt, cpad);           \
        else                                                                                   \
            hipLaunchKernelGGL((k_fp8_mxn<NTV, false, MWV>), grid, dim3(64 * MWV), lds, st, y, x, \
                               W, S, rows, cols, sc, blk_r, bc_m, nt, tpg, xt, cpad);           \
    } while (0)
    if (mw == 8) XN(4, 8);
    else switch (NTc) {
    case 1: XN(1, 4); break;
    case 2: XN(2, 4); break;
    case 3: XN(3, 4); break;
    case 4: XN(4, 4); break;
    case 5: XN(5, 4); break;
    case 6: XN(6, 4); break;
    default: XN(7, 4); break;
    }
#undef XN
    HIP_OK(hipGetLastError(), "fp8 mxn launch");
    return 0;
}
