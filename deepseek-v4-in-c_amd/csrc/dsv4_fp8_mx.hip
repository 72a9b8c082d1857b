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
 * The single-token kernel spreads a 16-row tile's segments over the waves of
 * a workgroup (so short matrices still fill the machine) and adds the
 * segment partials through LDS; the batched kernel walks the segments in
 * order inside one wave and keeps the running sum in registers. Matrix-core
 * columns are computed independently, so where a token sits among the
 * columns does not change its bits; the tests check every case bit for bit.
 *
 * MEMORY: weights stream in units of 16 rows x 256 bytes, loaded as four
 * 4-row x 256-byte requests per wave (fully coalesced), staged through a
 * wave-private LDS buffer into the matrix core's operand order (the layout
 * dsv4_moe_mx.hip measured fastest on MI355X). The single-token kernel
 * requests every weight unit of its segment before it stages x, so the
 * whole matrix is in flight from the first microsecond.
 */
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
constexpr int XPL = XSEG + 8;           /* LDS pitch of a term plane (x1)  */

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
 * [16 (l % 16), +16) of the unit, for q = 0..3. */
struct XUnit {
    u32x4 w[4];
};

/* Unit u of the tile whose row 0 is W + row0 * cols (rows past `rows` read
 * the last row, pieces past `cols` the row's first piece: their results are
 * discarded or zeroed). */
__device__ __forceinline__ void xu_load(XUnit &U, const uint8_t *W, int row0, int rows,
                                        int cols, int k0, int lane)
{
    const int c = k0 + 16 * (lane & 15);
    const int cc = c < cols ? c : 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int r = min(row0 + 4 * q + (lane >> 4), rows - 1);
        U.w[q] = ldg16_stream(W + (size_t)r * cols + cc);
    }
}

__device__ __forceinline__ void xu_stage(unsigned char *buf, const XUnit &U, int lane)
{
#pragma unroll
    for (int q = 0; q < 4; q++)
        *reinterpret_cast<u32x4 *>(buf + (4 * q + (lane >> 4)) * XWP + 16 * (lane & 15)) = U.w[q];
}

/* The block scale of lane (row r, group g)'s piece of quarter q of the unit
 * at column k0, as the f32 2^(b - 127) (0 for a piece past the row's end:
 * its codes are then treated as zeros). */
__device__ __forceinline__ float xu_scale(const uint8_t *S, int sc, int blk_r, int blk_c,
                                          int row, int k, int cols)
{
    if (k >= cols) return 0.0f;
    return dec_e8m0(S[(size_t)(row / blk_r) * sc + k / blk_c]);
}

/* The A operands of quarter q for this lane: steps (q, 0) and (q, 1). A piece
 * past the row's end is zero (its codes are replaced, not scaled: a NaN code
 * times 0 would still be NaN). */
__device__ __forceinline__ void xu_frags(v8bf *a, const unsigned char *buf, int q, float s,
                                         bool live, int lane)
{
    const u32x4 v = *reinterpret_cast<const u32x4 *>(buf + (lane & 15) * XWP + 64 * q +
                                                      16 * (lane >> 4));
    const u32x4 z = live ? v : u32x4{0u, 0u, 0u, 0u};
    a[0] = fp8x8_bf16(z.x, z.y, s);
    a[1] = fp8x8_bf16(z.z, z.w, s);
}

/* ------------------------------------------------------ single token */

/* LDS of one wave of the single-token kernel: its segment's x terms (three
 * planes of XPL bf16), then its unit buffer. */
constexpr int X1_WAVE_B = XNT * XPL * 2 + XUNIT_B;

/* x[k0 .. k0 + XSEG) as three bf16 term planes in the wave's LDS, zeros past
 * cols. Each lane takes 16 consecutive values. */
__device__ __forceinline__ void x1_stage(uint16_t *pl, const float *x, int k0, int cols,
                                         int lane)
{
    f32x4 v[4];
    const int c0 = k0 + 16 * lane;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = c0 + 4 * j;
        v[j] = c < cols ? *(const DSV4_GLOBAL f32x4 *)(x + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        uint32_t t[4][XNT];
#pragma unroll
        for (int i = 0; i < 4; i++) terms3(e[i], t[i]);
#pragma unroll
        for (int p = 0; p < XNT; p++) {
            const uint32_t lo = t[0][p] | (t[1][p] << 16), hi = t[2][p] | (t[3][p] << 16);
            *reinterpret_cast<uint2 *>(pl + p * XPL + 16 * lane + 4 * j) = uint2{lo, hi};
        }
    }
}

/* The segment chain of one 16-row tile for a single token: units in flight
 * D deep in VGPRs, staged through the wave's buffer, 8 matrix-core steps per
 * unit. Returns the accumulator (D layout). */
template <int D>
__device__ __forceinline__ v4f x1_segment(const uint8_t *W, const uint8_t *S, int row0,
                                          int rows, int cols, int sc, int blk_r, int blk_c,
                                          int k0, int nu, const uint16_t *pl,
                                          unsigned char *buf, XUnit *P, int lane)
{
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, g = lane >> 4;
    const int row = min(row0 + r, rows - 1);
    const int col = lane & 15;                          /* B column: term plane */
    for (int u = 0; u < nu; u++) {
        wave_lds_sync();                      /* the previous unit's reads, x's terms */
        xu_stage(buf, P[u % D], lane);
        if (u + D < nu) xu_load(P[u % D], W, row0, rows, cols, k0 + XU * (u + D), lane);
        wave_lds_sync();
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = k0 + XU * u + 64 * q + 16 * g;
            const float s = xu_scale(S, sc, blk_r, blk_c, row, k, cols);
            v8bf a[2];
            xu_frags(a, buf, q, s, k < cols, lane);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                u32x4 bw = {0u, 0u, 0u, 0u};
                if (col < XNT)
                    bw = *reinterpret_cast<const u32x4 *>(pl + col * XPL + XU * u + 64 * q +
                                                          16 * g + 8 * h);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[h], __builtin_bit_cast(v8bf, bw),
                                                              acc, 0, 0, 0);
            }
        }
    }
    return acc;
}

/* One workgroup per 16-row tile (blockIdx.x), one group of the launch per
 * blockIdx.y (lists: several matrices reading the same x; strided groups:
 * wo_a's slices). Wave w takes segments w, w + nw, ...; it requests its
 * segment's weight units first, then stages the segment's x terms, then
 * streams. The segment partials (per row and term column) meet in LDS and
 * are added in segment order. */
template <int D>
__global__ void __launch_bounds__(512)
k_fp8_mx1(Dsv4Fp8Mx a)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char x1lds[];
    __shared__ float part[XSEG_MAX][16][XNT];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int gi = blockIdx.y;
    const float *x = a.x + (size_t)gi * a.x_stride;
    const uint8_t *W = a.list ? a.wl[gi] : a.w + (size_t)gi * a.w_stride;
    const uint8_t *S = a.list ? a.sl[gi] : a.s + (size_t)gi * a.s_stride;
    float *y = a.list ? a.yl[gi] : a.y + (size_t)gi * a.y_stride;
    const int rows = a.list ? a.rl[gi] : a.rows;
    const int cols = a.cols;
    const int row0 = blockIdx.x * 16;
    if (row0 >= rows) return;                          /* the whole workgroup */
    const int nseg = (cols + XSEG - 1) / XSEG;
    uint16_t *pl = (uint16_t *)(x1lds + (size_t)w * X1_WAVE_B);
    unsigned char *buf = x1lds + (size_t)w * X1_WAVE_B + XNT * XPL * 2;
    for (int seg = w; seg < nseg; seg += nw) {
        const int k0 = seg * XSEG;
        const int nu = min(XSEG_U, (cols - k0 + XU - 1) / XU);
        XUnit P[D];
#pragma unroll
        for (int j = 0; j < D; j++)
            xu_load(P[j], W, row0, rows, cols, k0 + XU * min(j, nu - 1), lane);
        x1_stage(pl, x, k0, cols, lane);
        const v4f acc = x1_segment<D>(W, S, row0, rows, cols, a.sc, a.blk_r, a.blk_c, k0, nu,
                                      pl, buf, P, lane);
        const int col = lane & 15;
        if (col < XNT) {
#pragma unroll
            for (int j = 0; j < 4; j++) part[seg][4 * (lane >> 4) + j][col] = acc[j];
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < 16 && row0 + (int)threadIdx.x < rows) {
        float c[XNT];
#pragma unroll
        for (int t = 0; t < XNT; t++) c[t] = part[0][threadIdx.x][t];
        for (int s = 1; s < nseg; s++)
#pragma unroll
            for (int t = 0; t < XNT; t++) c[t] = c[t] + part[s][threadIdx.x][t];
        y[row0 + threadIdx.x] = (c[0] + c[1]) + c[2];
    }
}

/* ------------------------------------------------------------ batched */

/* x[t][kc .. kc + XU) of the group's tokens as term rows in LDS:
 * bl[(tok * XNT + term) * BP + k], BP = XU + 8; zeros past cols and past
 * the group's tokens. The workgroup's threads share the work. */
constexpr int BP = XU + 8;

__device__ __forceinline__ void xn_stage(uint16_t *bl, const float *x, int t0, int ntok, int nt,
                                         int kc, int cols, int tpg)
{
    const int per = XU / 4;                              /* f32x4 pieces per token */
    const int total = tpg * per;
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int tk = i / per, c4 = i - tk * per;
        const int c = kc + 4 * c4;
        const int t = t0 + tk;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (tk < ntok && t < nt && c < cols)
            v = *(const DSV4_GLOBAL f32x4 *)(x + (size_t)t * cols + c);
        const float e[4] = {v.x, v.y, v.z, v.w};
        uint32_t tt[4][XNT];
#pragma unroll
        for (int j = 0; j < 4; j++) terms3(e[j], tt[j]);
#pragma unroll
        for (int p = 0; p < XNT; p++)
            *reinterpret_cast<uint2 *>(bl + (size_t)(tk * XNT + p) * BP + 4 * c4) =
                uint2{tt[0][p] | (tt[1][p] << 16), tt[2][p] | (tt[3][p] << 16)};
    }
}

/* Workgroup (blockIdx.x: MW 16-row tiles, one per wave; blockIdx.y: a group
 * of tpg tokens starting at t0). Per unit: the workgroup stages the group's x
 * terms for the unit's 256 columns, every wave runs its tile's 8 steps x NT
 * column tiles from its own staged unit, and at the end of each segment the
 * segment's accumulators join the running sums in segment order. */
template <int NT, int D>
__global__ void __launch_bounds__(256)
k_fp8_mxn(float *__restrict__ y, const float *__restrict__ x, const uint8_t *__restrict__ W,
          const uint8_t *__restrict__ S, int rows, int cols, int sc, int blk_r, int blk_c,
          int nt, int tpg)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char xnlds[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    uint16_t *bl = (uint16_t *)xnlds;                    /* [tpg * 3][BP] */
    unsigned char *buf = xnlds + (size_t)tpg * XNT * BP * 2 + (size_t)w * XUNIT_B;
    const int row0 = (blockIdx.x * nw + w) * 16;
    const int t0 = blockIdx.y * tpg;
    const int ntok = min(tpg, nt - t0);
    const int r = lane & 15, g = lane >> 4;
    const int row = min(row0 + r, rows - 1);
    const int col = lane & 15;
    /* this lane's B row per column tile: token 5 n + col / 3, term col % 3 */
    int boff[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int tk = XTOK * n + col / XNT;
        boff[n] = (col < XNT * XTOK && tk < ntok) ? (tk * XNT + col % XNT) * BP : -1;
    }
    v4f acc[NT], tot[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
        tot[n] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    const int nu_all = (cols + XU - 1) / XU;
    const bool live = row0 < rows;
    XUnit P[D];
#pragma unroll
    for (int j = 0; j < D; j++)
        xu_load(P[j], W, live ? row0 : 0, rows, cols, XU * min(j, nu_all - 1), lane);
    for (int u = 0; u < nu_all; u++) {
        __syncthreads();                                /* the previous unit's B reads */
        xn_stage(bl, x, t0, ntok, nt, XU * u, cols, tpg);
        xu_stage(buf, P[u % D], lane);
        if (u + D < nu_all)
            xu_load(P[u % D], W, live ? row0 : 0, rows, cols, XU * (u + D), lane);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = XU * u + 64 * q + 16 * g;
            const float s = xu_scale(S, sc, blk_r, blk_c, row, k, cols);
            v8bf a[2];
            xu_frags(a, buf, q, s, k < cols, lane);
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    u32x4 bw = {0u, 0u, 0u, 0u};
                    if (boff[n] >= 0)
                        bw = *reinterpret_cast<const u32x4 *>(bl + boff[n] + 64 * q + 16 * g +
                                                              8 * h);
                    acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        a[h], __builtin_bit_cast(v8bf, bw), acc[n], 0, 0, 0);
                }
            }
        }
        /* a segment ends: its partials join the running sums in order */
        if ((u + 1) % XSEG_U == 0 || u + 1 == nu_all) {
            const bool first = u < XSEG_U;
#pragma unroll
            for (int n = 0; n < NT; n++) {
                tot[n] = first ? acc[n] : tot[n] + acc[n];
                acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
            }
        }
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

template <typename K>
void optin(K kernel)
{
    (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)dsv4_lds_limit());
    (void)hipGetLastError();
}

} // namespace

bool dsv4_fp8_mx_ok(int sfmt, int cols, int blk_r, int blk_c)
{
    return sfmt == 0 && cols > 0 && (cols % 16) == 0 && cols <= XSEG * XSEG_MAX &&
           blk_r >= 1 && blk_c >= 16 && (blk_c % 16) == 0;
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
    const int nseg = (a.cols + XSEG - 1) / XSEG;
    const int nw = nseg < 8 ? nseg : 8;
    const size_t lds = (size_t)nw * X1_WAVE_B;
    static bool opted = false;
    if (!opted) { optin(k_fp8_mx1<4>); opted = true; }
    hipLaunchKernelGGL((k_fp8_mx1<4>), dim3((rmax + 15) / 16, a.n), dim3(64 * nw), lds, st, a);
    HIP_OK(hipGetLastError(), "fp8 mx launch");
    return 0;
}

int dsv4_fp8_mxn_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S, int rows,
                        int cols, int blk_r, int blk_c, int nt, hipStream_t st)
{
    if (!dsv4_fp8_mx_ok(0, cols, blk_r, blk_c) || rows <= 0 || nt < 1 || nt > DSV4_MAX_BATCH) {
        DSV4_ERR("fp8 mxn: shape not taken (%dx%d, nt %d)", rows, cols, nt);
        return -1;
    }
    const int sc = (cols + blk_c - 1) / blk_c;
    /* tokens per workgroup: at most 4 column tiles of 5 (the accumulators and
     * running sums of 4 tiles stay in registers); more tokens take more
     * workgroups along y, each reading the weights again */
    const int ntile = (nt + XTOK - 1) / XTOK;
    const int NTc = ntile >= 4 ? 4 : ntile >= 2 ? (ntile == 3 ? 3 : 2) : 1;
    const int tpg = XTOK * NTc < nt ? XTOK * NTc : nt;
    const int groups = (nt + tpg - 1) / tpg;
    constexpr int MW = 4;
    const size_t lds = (size_t)tpg * XNT * BP * 2 + (size_t)MW * XUNIT_B;
    const dim3 grid((rows + 16 * MW - 1) / (16 * MW), groups);
    static bool opted = false;
    if (!opted) {
        optin(k_fp8_mxn<1, 2>); optin(k_fp8_mxn<2, 2>); optin(k_fp8_mxn<3, 2>);
        optin(k_fp8_mxn<4, 2>);
        opted = true;
    }
#define XN(NTV) hipLaunchKernelGGL((k_fp8_mxn<NTV, 2>), grid, dim3(64 * MW), lds, st, y, x, W, S, \
                                   rows, cols, sc, blk_r, blk_c, nt, tpg)
    switch (NTc) {
    case 1: XN(1); break;
    case 2: XN(2); break;
    case 3: XN(3); break;
    default: XN(4); break;
    }
#undef XN
    HIP_OK(hipGetLastError(), "fp8 mxn launch");
    return 0;
}
