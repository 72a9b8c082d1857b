/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe_mx.hip - the routed-expert MXFP4 matvec with gfx950's matrix cores.
 *
 * Same computation as dsv4_moe.hip -- the routed half of the reference's moe()
 * for one token (src/model/dsv4_layer.c:199-206, :412-476):
 *     acc_k  = w2_k . swiglu(w1_k . x, w3_k . x)
 *     out[i] = ((0 + w0*acc_0[i]) + w1*acc_1[i]) + ...   strictly in k order
 * -- for hidden and inter that are multiples of 128.
 *
 * WHY THE MATRIX CORE. On MI355X the VALU form issues about 60 instructions
 * per 16 weight bytes (16 nibble-pair converts, 32 FMAs, the rest
 * bookkeeping), and at the 2 waves per SIMD its registers allow, that
 * arithmetic does not hide behind the HBM stream. Here the VALU only decodes:
 * v_cvt_scalef32_pk_bf16_fp4 turns two e2m1 nibbles times their E8M0 block
 * scale into two bf16 values, exactly (e2m1 times a power of two is exact in
 * bf16). The multiply-adds go to v_mfma_f32_16x16x32_bf16, which accumulates
 * in fp32.
 *
 * THE ACTIVATION, EXACTLY. The MFMA's other operand is bf16 too, so the f32
 * activation (x, later h) is carried as three bf16 terms,
 *     v = hi + mid + lo,   hi = bf16(v), mid = bf16(v - hi), lo = bf16(v - hi - mid)
 * which holds all 24 bits of v. B's first three columns carry the terms, so
 * row i of the result's columns 0..2 sums to W[i] . v.
 *
 * OPERAND LAYOUT of v_mfma_f32_16x16x32_bf16, measured on gfx950:
 *   A : lane l holds row l%16, K elements [8(l/16), +8) (8 bf16);
 *   B : lane l holds column l%16, K elements [8(l/16), +8);
 *   D : lane l, register j holds row 4(l/16) + j, column l%16.
 * Within a 128-wide K block, lane (row r, group g) loads the 16 bytes (32
 * nibbles) of K [32g, 32g + 32), one E8M0 scale block, and feeds dword m of
 * them to the m-th of four MFMAs; the B lanes read their terms in the same
 * permuted K order. The order of the K sum changes, the set of products does
 * not.
 *
 * KERNELS
 *   k_mc_split    x -> three bf16 term planes (once per call).
 *   k_mc_gate_up  grid (row blocks of 16*OT, expert slot k). The 4 waves of a
 *                 workgroup split the K blocks and meet in LDS. It applies
 *                 SwiGLU and writes h_k as three bf16 term planes.
 *   k_mc_down     grid (row blocks of 16*OT). One wave per expert slot, then
 *                 the k-ordered, separately rounded combine in LDS (this file
 *                 is built with -ffp-contract=off).
 * Every reduction order is fixed, so a result is the same bits on every run.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

#include <stdlib.h>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int MC_NT = 3;          /* bf16 terms per activation value */
constexpr int MC_KMAX = 64;       /* expert slots per call */

size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

/* f32 -> bf16 bits, round to nearest even (finite inputs). */
__device__ __forceinline__ uint32_t bf16_rne(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

/* v = hi + mid + lo, each a bf16; exact for every finite f32 v whose terms
 * stay in bf16's (f32's) exponent range. */
__device__ __forceinline__ void bf16_terms(float v, uint32_t *t)
{
    t[0] = bf16_rne(v);
    const float r1 = v - __uint_as_float(t[0] << 16);
    t[1] = bf16_rne(r1);
    const float r2 = r1 - __uint_as_float(t[1] << 16);
    t[2] = bf16_rne(r2);
}

__device__ __forceinline__ Dsv4ExpertDev mc_expert(const Dsv4ExpertDev *table,
                                                   int n_table, const int *idx, int k)
{
    const int e = idx[k];
    if (e < 0 || e >= n_table)
        return Dsv4ExpertDev{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    return table[e];
}

/* Eight e2m1 nibbles (one dword, element order) times 2^(e-127) -> 8 bf16,
 * exactly. */
__device__ __forceinline__ v8bf fp4x8_bf16(uint32_t v, float scale)
{
    const v2s p0 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 0));
    const v2s p1 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 1));
    const v2s p2 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 2));
    const v2s p3 = __builtin_bit_cast(v2s, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 3));
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s r = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    return __builtin_bit_cast(v8bf, r);
}

/* Sum of columns 0..MC_NT-1 of a 16x16 result tile, per row: the sum of
 * row 4q + j lands in register j of every lane of the 16-lane group q, added
 * in column order. */
__device__ __forceinline__ v4f term_sum(const v4f &d, int lane)
{
    const int base = lane & ~15;
    v4f s;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float a = __shfl(d[j], base + 0, 64);
#pragma unroll
        for (int t = 1; t < MC_NT; t++) a = a + __shfl(d[j], base + t, 64);
        s[j] = a;
    }
    return s;
}

/* x -> three bf16 term planes xt[t][n]. */
__global__ void __launch_bounds__(256)
k_mc_split(uint16_t *__restrict__ xt, const float *__restrict__ x, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t t[MC_NT];
    bf16_terms(x[i], t);
#pragma unroll
    for (int c = 0; c < MC_NT; c++) xt[(size_t)c * n + i] = (uint16_t)t[c];
}

/* One 128-wide K block of weights for NM matrices x OT row tiles: 16 bytes
 * and one scale byte per lane each. */
template <int OT, int NM>
struct McBuf {
    u32x4 a[NM][OT];
    uint32_t sa[NM][OT];
};

template <int OT, int NM>
__device__ __forceinline__ void mc_load(McBuf<OT, NM> &B, const uint8_t *const (*wr)[OT],
                                        const uint8_t *const (*sr)[OT], int kb)
{
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int it = 0; it < OT; it++) {
            B.a[m][it] = ldg16_stream(wr[m][it] + (size_t)kb * 64);
            B.sa[m][it] = ldg8(sr[m][it] + kb * 4);
        }
}

/* acc += W(kb) . terms(kb); this lane's activation-term slice of the K block
 * comes from LDS (bl: the lane's term plane; the rest read a zero plane).
 * live = false adds zero (the weights are decoded with scale 0). */
template <int OT, int NM>
__device__ __forceinline__ void mc_mac(v4f (*acc)[OT], const McBuf<OT, NM> &B,
                                       const uint16_t *bl, int kb, bool live)
{
    v8bf b[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        b[q] = __builtin_bit_cast(v8bf, *reinterpret_cast<const u32x4 *>(bl + kb * 128 + q * 8));
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int it = 0; it < OT; it++) {
            const float sc = live ? dec_e8m0(B.sa[m][it]) : 0.0f;
            const uint32_t d[4] = {B.a[m][it].x, B.a[m][it].y, B.a[m][it].z, B.a[m][it].w};
#pragma unroll
            for (int q = 0; q < 4; q++)
                acc[m][it] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    fp4x8_bf16(d[q], sc), b[q], acc[m][it], 0, 0, 0);
        }
}

/* The K blocks kb0, kb0 + step, ... < nkb with D blocks of weights in flight.
 * mc_prefetch requests the first D blocks (they do not depend on LDS, so the
 * caller issues them before staging the activation terms); mc_run consumes
 * them. The steady state is straight-line code, so the compiler can wait for
 * each block's loads alone (a branch per block would make it wait for all of
 * them): past the last block, a slot reloads the last block and is added
 * with scale 0. */
template <int OT, int NM, int D>
struct McPipe {
    McBuf<OT, NM> buf[D];
    int cnt, last;
};

template <int OT, int NM, int D>
__device__ __forceinline__ void mc_prefetch(McPipe<OT, NM, D> &P,
                                            const uint8_t *const (*wr)[OT],
                                            const uint8_t *const (*sr)[OT], int kb0,
                                            int step, int nkb)
{
    P.cnt = nkb > kb0 ? (nkb - kb0 + step - 1) / step : 0;
    P.last = kb0 + (P.cnt > 0 ? P.cnt - 1 : 0) * step;
    if (P.cnt <= 0) return;
#pragma unroll
    for (int j = 0; j < D; j++) mc_load<OT, NM>(P.buf[j], wr, sr, min(kb0 + j * step, P.last));
}

template <int OT, int NM, int D>
__device__ __forceinline__ void mc_run(v4f (*acc)[OT], McPipe<OT, NM, D> &P,
                                       const uint8_t *const (*wr)[OT],
                                       const uint8_t *const (*sr)[OT],
                                       const uint16_t *bl, int kb0, int step)
{
    const int rounds = (P.cnt + D - 1) / D;
    for (int rd = 0; rd < rounds; rd++) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            const int i = rd * D + j;
            const bool live = i < P.cnt;
            const int kb = kb0 + i * step;
            mc_mac<OT, NM>(acc, P.buf[j], bl, live ? kb : P.last, live);
            mc_load<OT, NM>(P.buf[j], wr, sr, min(kb + D * step, P.last));
        }
    }
}

/* LDS plane pitch in bf16 elements: 16 bytes of skew per plane keeps the
 * lanes of a ds_read_b128 on distinct banks. */
__host__ __device__ __forceinline__ int mc_pitch(int n) { return n + 8; }

/* Copy `planes` bf16 planes of n elements (global pitch n) into LDS (pitch
 * mc_pitch(n)) and zero one more plane after them. Each thread has a batch
 * of loads in flight before it stores any of them. */
__device__ __forceinline__ void mc_stage(uint16_t *lds, const uint16_t *src, int planes,
                                         int n)
{
    constexpr int SB = 8;
    const int pitch = mc_pitch(n);
    const int per = n >> 3;                              /* 16-byte pieces per plane */
    const int total = (planes + 1) * per;
    for (int i0 = threadIdx.x; i0 < total; i0 += SB * blockDim.x) {
        u32x4 v[SB];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = i0 + u * blockDim.x;
            const int p = i / per, c = i - p * per;
            v[u] = (i < total && p < planes) ? ld16(src + (size_t)p * n + c * 8)
                                             : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = i0 + u * blockDim.x;
            if (i < total) {
                const int p = i / per, c = i - p * per;
                *reinterpret_cast<u32x4 *>(lds + p * pitch + c * 8) = v[u];
            }
        }
    }
}

/* Pass A: h-rows [o0, o0 + 16*OT) of expert slot k; 4 waves split the K
 * blocks (wave w takes kb = w, w+4, ...). x's terms are staged in LDS once.
 * SwiGLU, then h as three bf16 term planes ht[k][t][inter]. */
template <int OT, int D>
__global__ void __launch_bounds__(256)
k_mc_gate_up(uint16_t *__restrict__ ht, const uint16_t *__restrict__ xt,
             const Dsv4ExpertDev *__restrict__ table, int n_table,
             const int *__restrict__ idx, int hidden, int inter, float limit)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t xl[];  /* [MC_NT+1][pitch] */
    __shared__ float red[4][2][16 * OT];
    const int k = blockIdx.y;
    const Dsv4ExpertDev E = mc_expert(table, n_table, idx, k);
    if (!E.w1) return;                      /* the down pass reports it (NaN) */
    const int o0 = blockIdx.x * (16 * OT);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int nkb = hidden >> 7, nsb = hidden >> 5;
    const size_t rowb = (size_t)hidden >> 1;

    const uint8_t *wr[2][OT], *sr[2][OT];
#pragma unroll
    for (int it = 0; it < OT; it++) {
        const size_t row = (size_t)(o0 + 16 * it + r);
        wr[0][it] = E.w1 + row * rowb + 16 * g;
        wr[1][it] = E.w3 + row * rowb + 16 * g;
        sr[0][it] = E.s1 + row * nsb + g;
        sr[1][it] = E.s3 + row * nsb + g;
    }
    McPipe<OT, 2, D> pipe;
    mc_prefetch<OT, 2, D>(pipe, wr, sr, w, 4, nkb);
    mc_stage(xl, xt, MC_NT, hidden);
    __syncthreads();
    const uint16_t *bl = xl + (r < MC_NT ? r : MC_NT) * mc_pitch(hidden) + 32 * g;

    v4f acc[2][OT];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int it = 0; it < OT; it++) acc[m][it] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    mc_run<OT, 2, D>(acc, pipe, wr, sr, bl, w, 4);

    /* per wave: the sum of the term columns; then the 4 waves in order */
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int it = 0; it < OT; it++) {
            const v4f s = term_sum(acc[m][it], lane);
            if (r == 0) {
#pragma unroll
                for (int j = 0; j < 4; j++) red[w][m][16 * it + 4 * g + j] = s[j];
            }
        }
    __syncthreads();
    for (int i = tid; i < 16 * OT; i += blockDim.x) {
        const float gs = ((red[0][0][i] + red[1][0][i]) + red[2][0][i]) + red[3][0][i];
        const float us = ((red[0][1][i] + red[1][1][i]) + red[2][1][i]) + red[3][1][i];
        uint32_t t[MC_NT];
        bf16_terms(swiglu1(gs, us, limit), t);
#pragma unroll
        for (int c = 0; c < MC_NT; c++)
            ht[((size_t)k * MC_NT + c) * inter + o0 + i] = (uint16_t)t[c];
    }
}

/* Pass B + combine: output rows [r0, r0 + 16*OT); the h terms of every slot
 * are staged in LDS; wave w handles slots k = w, w + nwaves, ...; acc_k stays
 * in LDS; then the k-ordered combine. */
template <int OT, int D>
__global__ void __launch_bounds__(512)
k_mc_down(float *__restrict__ out, const uint16_t *__restrict__ ht,
          const Dsv4ExpertDev *__restrict__ table, int n_table,
          const int *__restrict__ idx, const float *__restrict__ wts, int topk,
          int hidden, int inter)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t hl[];  /* [topk*MC_NT+1][pitch] */
    __shared__ float accl[MC_KMAX][16 * OT];
    const int r0 = blockIdx.x * (16 * OT);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nw = blockDim.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int nkb = inter >> 7, nsb = inter >> 5;
    const size_t rowb = (size_t)inter >> 1;
    const int pitch = mc_pitch(inter);

    /* the first slot of this wave is requested before the h terms are staged */
    const uint8_t *wr[1][OT], *sr[1][OT];
    McPipe<OT, 1, D> pipe;
    Dsv4ExpertDev E = w < topk ? mc_expert(table, n_table, idx, w)
                               : Dsv4ExpertDev{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    auto bind = [&](const Dsv4ExpertDev &X) {
#pragma unroll
        for (int it = 0; it < OT; it++) {
            const size_t row = (size_t)(r0 + 16 * it + r);
            wr[0][it] = X.w2 + row * rowb + 16 * g;
            sr[0][it] = X.s2 + row * nsb + g;
        }
    };
    if (E.w1) {
        bind(E);
        mc_prefetch<OT, 1, D>(pipe, wr, sr, 0, 1, nkb);
    }
    mc_stage(hl, ht, topk * MC_NT, inter);
    __syncthreads();
    for (int k = w; k < topk; k += nw) {
        if (k != w) {
            E = mc_expert(table, n_table, idx, k);
            if (E.w1) {
                bind(E);
                mc_prefetch<OT, 1, D>(pipe, wr, sr, 0, 1, nkb);
            }
        }
        if (!E.w1) {
            if (lane < 16 * OT) accl[k][lane] = __builtin_nanf("");
            continue;
        }
        const uint16_t *bl = hl + (r < MC_NT ? k * MC_NT + r : topk * MC_NT) * pitch + 32 * g;
        v4f acc[1][OT];
#pragma unroll
        for (int it = 0; it < OT; it++) acc[0][it] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        mc_run<OT, 1, D>(acc, pipe, wr, sr, bl, 0, 1);
#pragma unroll
        for (int it = 0; it < OT; it++) {
            const v4f s = term_sum(acc[0][it], lane);
            if (r == 0) {
#pragma unroll
                for (int j = 0; j < 4; j++) accl[k][16 * it + 4 * g + j] = s[j];
            }
        }
    }
    __syncthreads();
    if (tid < 16 * OT) {
        float o = 0.0f;
        for (int kk = 0; kk < topk; kk++) {
            const float p = wts[kk] * accl[kk][tid];
            o = o + p;
        }
        out[r0 + tid] = o;
    }
}

/* ------------------------------------------------- staged matrix-core form */

/* The MFMA's fragment order reads 16 rows x 64 B per load, which streams at
 * about 4.6 TB/s; loads of 4 rows x 256 B stream at 6.3 TB/s (measured on
 * MI355X over the C3 expert bytes). So here each wave brings a unit of 16
 * rows x 256 B (and the unit's scale bytes) into its own LDS area in that
 * order, and reads the fragments back from LDS. The arithmetic is that of
 * k_mc_gate_up / k_mc_down: lane (row r, group g) takes the 16 bytes of row
 * r at [64 qb + 16 g, +16) of the unit and feeds dword m to the MFMA of
 * chunk (qb, m); B reads the activation terms in the same permuted K order. */
constexpr int M2_UB = 256;                       /* bytes per row per unit */
constexpr int M2_WP = M2_UB + 16;                /* LDS row pitch (bank skew) */
constexpr int M2_SOFF = 16 * M2_WP;              /* scales after the 16 rows */
constexpr int M2_WBUF = M2_SOFF + 16 * 16;       /* one wave's unit buffer */

struct M2Unit {
    u32x4 w[4];                                  /* rows 4q + lane/16, 16 bytes */
    uint32_t s;                                  /* scale bytes of row lane/4 */
};

/* The unit u of the 16-row tile whose row 0 starts at base (scales at sb);
 * always in bounds for u < the row's unit count. */
__device__ __forceinline__ void m2_load(M2Unit &U, const uint8_t *base, size_t rowb,
                                        const uint8_t *sb, int nsb, int u, int lane)
{
#pragma unroll
    for (int q = 0; q < 4; q++)
        U.w[q] = ldg16_stream(base + (size_t)(4 * q + (lane >> 4)) * rowb + M2_UB * u +
                              16 * (lane & 15));
    U.s = *(const DSV4_GLOBAL uint32_t *)(sb + (size_t)(lane >> 2) * nsb + 16 * u +
                                          4 * (lane & 3));
}

__device__ __forceinline__ void m2_stage(unsigned char *buf, const M2Unit &U, int lane)
{
#pragma unroll
    for (int q = 0; q < 4; q++)
        *reinterpret_cast<u32x4 *>(buf + (4 * q + (lane >> 4)) * M2_WP + 16 * (lane & 15)) = U.w[q];
    *reinterpret_cast<uint32_t *>(buf + M2_SOFF + (lane >> 2) * 16 + 4 * (lane & 3)) = U.s;
}

/* acc[qb & 1] += the unit's 16 chunks; bl = this lane's activation-term
 * plane in LDS at the unit's first element (a zero plane for columns >= 3).
 * live = false adds zero (the weights are decoded with scale 0). */
__device__ __forceinline__ void m2_mac(v4f *acc, const unsigned char *buf,
                                       const uint16_t *bl, int lane, bool live)
{
    const int r = lane & 15, g = lane >> 4;
    const u32x4 sv = *reinterpret_cast<const u32x4 *>(buf + M2_SOFF + r * 16);
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int qb = 0; qb < 4; qb++) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(buf + r * M2_WP + 64 * qb + 16 * g);
        const float sc = live ? dec_e8m0((sw[qb] >> (8 * g)) & 0xFFu) : 0.0f; /* segment 4 qb + g */
        const uint32_t d[4] = {a.x, a.y, a.z, a.w};
        /* only the lanes of columns 0..MC_NT-1 carry terms; the others
         * feed zeros without an LDS read */
        u32x4 bw[4] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u},
                       u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
        if (r < MC_NT) {
#pragma unroll
            for (int m = 0; m < 4; m++)
                bw[m] = *reinterpret_cast<const u32x4 *>(bl + 128 * qb + 32 * g + 8 * m);
        }
        v8bf b[4];
#pragma unroll
        for (int m = 0; m < 4; m++) b[m] = __builtin_bit_cast(v8bf, bw[m]);
#pragma unroll
        for (int m = 0; m < 4; m++)
            acc[qb & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(d[m], sc), b[m],
                                                                   acc[qb & 1], 0, 0, 0);
    }
}

/* The first D units of a 16-row tile (past unit nu-1, the last again). */
template <int D>
__device__ __forceinline__ void m2_prologue(M2Unit *P, const uint8_t *base, size_t rowb,
                                            const uint8_t *sb, int nsb, int nu, int lane)
{
#pragma unroll
    for (int j = 0; j < D; j++) m2_load(P[j], base, rowb, sb, nsb, min(j, nu - 1), lane);
}

/* Units 0 .. nu-1 of one 16-row tile, D units in flight in VGPRs; P holds
 * the first D, requested by m2_prologue (a caller can issue them before it
 * stages the activation terms). The LDS buffer is the wave's own (its writes
 * follow its previous reads in order). NU > 0 is the unit count known at
 * compile time: the loop unrolls whole, so each unit's wait counts only its
 * own loads (a loop-carried wait is for all of them). Otherwise the loop is
 * straight-line per D units: past the last unit, a slot reloads the last
 * unit and is added with scale 0. */
template <int D, int NU>
__device__ __forceinline__ v4f m2_tile(M2Unit *P, const uint8_t *base, size_t rowb,
                                       const uint8_t *sb, int nsb, int nu, unsigned char *buf,
                                       const uint16_t *bl0, int lane)
{
    v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    if (NU > 0) nu = NU;
    if (NU > 0) {
        /* the scheduling barriers keep each unit's loads where they are
         * issued: sunk toward their use, they would no longer be in flight
         * D units ahead */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NU; u++) {
            m2_stage(buf, P[u % D], lane);
            if (u + D < NU) m2_load(P[u % D], base, rowb, sb, nsb, u + D, lane);
            __builtin_amdgcn_sched_barrier(0);
            m2_mac(acc, buf, bl0 + 512 * u, lane, true);
        }
    } else {
        for (int u0 = 0; u0 < nu; u0 += D) {
#pragma unroll
            for (int j = 0; j < D; j++) {
                const int u = u0 + j;
                m2_stage(buf, P[j], lane);
                m2_load(P[j], base, rowb, sb, nsb, min(u + D, nu - 1), lane);
                m2_mac(acc, buf, bl0 + 512 * min(u, nu - 1), lane, u < nu);
            }
        }
    }
    return acc[0] + acc[1];
}

/* x staging, in two steps so that a caller can put other loads between
 * them: m2_x_load requests NL 16-byte pieces of x per thread (elements i0 +
 * 4 (j * blockDim + tid) ...; past n it reloads the last piece), m2_x_store
 * writes their MC_NT bf16 terms into the planes at lds (pitch mc_pitch(n)).
 * n is a multiple of 4 and x 16-byte aligned. */
template <int NL>
__device__ __forceinline__ void m2_x_load(f32x4 *xv, const float *x, int n, int i0)
{
#pragma unroll
    for (int j = 0; j < NL; j++) {
        const int i = i0 + 4 * (j * (int)blockDim.x + (int)threadIdx.x);
        xv[j] = *(const DSV4_GLOBAL f32x4 *)(x + min(i, n - 4));
    }
}

template <int NL>
__device__ __forceinline__ void m2_x_store(uint16_t *lds, const f32x4 *xv, int n, int i0)
{
    const int pitch = mc_pitch(n);
#pragma unroll
    for (int j = 0; j < NL; j++) {
        const int i = i0 + 4 * (j * (int)blockDim.x + (int)threadIdx.x);
        if (i < n) {
            const float vv[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t t[MC_NT];
                bf16_terms(vv[e], t);
#pragma unroll
                for (int c = 0; c < MC_NT; c++) lds[c * pitch + i + e] = (uint16_t)t[c];
            }
        }
    }
}

/* Pass A's body for row block bx (16 TILES h-rows) of slot k, 2 TILES
 * waves: wave w runs matrix w & 1 (w1 / w3) over row tile w >> 1. The
 * workgroup splits x into its bf16 terms in LDS; all of x is requested
 * before the first weight units, so the split waits for x alone while those
 * units are in flight. false when slot k's expert is missing (nothing
 * written: the down pass reports it). COHERENT: h leaves as agent-scope
 * stores (written through to the device's coherence point), for a consumer
 * on another XCD in the same launch. */
template <int D, int NU, int TILES, bool COHERENT>
__device__ __forceinline__ bool mc2_gate_up_body(uint16_t *__restrict__ ht,
                                                 const float *__restrict__ x,
                                                 const Dsv4ExpertDev *__restrict__ table,
                                                 int n_table, const int *__restrict__ idx,
                                                 int hidden, int inter, float limit, int bx,
                                                 int k)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char m2lds[];
    uint16_t *xl = (uint16_t *)m2lds;                      /* [MC_NT][pitch] */
    __shared__ float red[TILES][2][16];
    /* hidden = 512 NU: NL 16-byte pieces of x per thread of 2 TILES waves,
     * requested before the expert lookup (x does not depend on it, and it is
     * the last input to arrive before the first product) */
    constexpr int NL = NU > 0 ? (NU * 512 + 4 * 128 * TILES - 1) / (4 * 128 * TILES) : 1;
    f32x4 xv[NL];
    if constexpr (NU > 0) m2_x_load<NL>(xv, x, hidden, 0);
    const Dsv4ExpertDev E = mc_expert(table, n_table, idx, k);
    if (!E.w1) return false;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int mat = w & 1, tile = w >> 1;
    const int o0 = bx * 16 * TILES + 16 * tile;
    const int nsb = hidden >> 5;
    const size_t rowb = (size_t)hidden >> 1;
    const int nu = (int)(rowb / M2_UB);
    const int pitch = mc_pitch(hidden);
    unsigned char *buf = m2lds + (size_t)MC_NT * pitch * 2 + (size_t)w * M2_WBUF;
    const uint8_t *base = (mat ? E.w3 : E.w1) + (size_t)o0 * rowb;
    const uint8_t *sb = (mat ? E.s3 : E.s1) + (size_t)o0 * nsb;

    M2Unit P[D];
    if constexpr (NU > 0) {
        __builtin_amdgcn_sched_barrier(0);
        m2_prologue<D>(P, base, rowb, sb, nsb, NU, lane);
        __builtin_amdgcn_sched_barrier(0);
        m2_x_store<NL>(xl, xv, hidden, 0);
    } else {
        m2_prologue<D>(P, base, rowb, sb, nsb, nu, lane);
        for (int i0 = 0; i0 < hidden; i0 += 8 * 4 * (int)blockDim.x) {
            f32x4 xv[8];
            m2_x_load<8>(xv, x, hidden, i0);
            m2_x_store<8>(xl, xv, hidden, i0);
        }
    }
    __syncthreads();
    const int r = lane & 15, g = lane >> 4;
    const uint16_t *bl = xl + min(r, MC_NT - 1) * pitch;
    const v4f acc = m2_tile<D, NU>(P, base, rowb, sb, nsb, nu, buf, bl, lane);
    const v4f s = term_sum(acc, lane);
    if (r == 0) {
#pragma unroll
        for (int j = 0; j < 4; j++) red[tile][mat][4 * g + j] = s[j];
    }
    __syncthreads();
    if (tid < 16 * TILES) {
        const int t = tid >> 4, i = tid & 15;
        uint32_t tt[MC_NT];
        bf16_terms(swiglu1(red[t][0][i], red[t][1][i], limit), tt);
#pragma unroll
        for (int c = 0; c < MC_NT; c++) {
            uint16_t *dst = ht + ((size_t)k * MC_NT + c) * inter + bx * 16 * TILES + 16 * t + i;
            if (COHERENT)
                __hip_atomic_store(dst, (uint16_t)tt[c], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            else
                *dst = (uint16_t)tt[c];
        }
    }
    return true;
}

/* Pass A: workgroup (32 h-rows of expert slot k); wave w: matrix w & 1 (w1 /
 * w3), row tile w >> 1 (mc2_gate_up_body). */
template <int D, int NU>
__global__ void __launch_bounds__(256)
k_mc2_gate_up(uint16_t *__restrict__ ht, const float *__restrict__ x,
              const Dsv4ExpertDev *__restrict__ table, int n_table,
              const int *__restrict__ idx, int hidden, int inter, float limit)
{
    (void)mc2_gate_up_body<D, NU, 2, false>(ht, x, table, n_table, idx, hidden, inter, limit,
                                            blockIdx.x, blockIdx.y);
}

/* Both 16-row tiles of a 32-row group as one stream of 2 NU units (tile 0's
 * units, then tile 1's), D in flight across the tile boundary; P holds units
 * 0 .. D-1 (D <= NU). res[t] = tile t's sum. */
template <int D, int NU>
__device__ __forceinline__ void m2_tiles2(v4f *res, M2Unit *P, const uint8_t *base,
                                          size_t rowb, const uint8_t *sb, int nsb,
                                          unsigned char *buf, const uint16_t *bl0, int lane)
{
    static_assert(NU > 0 && D <= NU, "units in flight within the first tile");
    v4f acc[2][2] = {{v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}},
                     {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}}};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 2 * NU; u++) {
        const int t = u / NU, uu = u - t * NU;
        m2_stage(buf, P[u % D], lane);
        if (u + D < 2 * NU) {
            const int t2 = (u + D) / NU, u2 = u + D - t2 * NU;
            m2_load(P[u % D], base + (size_t)16 * t2 * rowb, rowb, sb + (size_t)16 * t2 * nsb,
                    nsb, u2, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
        m2_mac(acc[t], buf, bl0 + 512 * uu, lane, true);
    }
    res[0] = acc[0][0] + acc[0][1];
    res[1] = acc[1][0] + acc[1][1];
}

/* LDS of one down-pass wave: its slot's MC_NT h planes, then its unit
 * buffer. */
__host__ __device__ __forceinline__ size_t m2_hplanes_b(int inter)
{
    return (size_t)MC_NT * mc_pitch(inter) * 2;
}
__host__ __device__ __forceinline__ size_t m2_wave_b(int inter)
{
    return m2_hplanes_b(inter) + M2_WBUF;
}
__host__ __device__ __forceinline__ int m2_down_waves(int topk) { return topk < 8 ? topk : 8; }

/* Pass B + combine: workgroup (32 output rows); wave w takes slots w, w + nw,
 * ..., both row tiles of each. A wave stages its own slot's h terms in its
 * own LDS (no workgroup barrier: it requests them before its first weight
 * units and waits for them alone); acc_k meets in LDS for the k-ordered
 * combine. */
template <int D, int NU>
__global__ void __launch_bounds__(512)
k_mc2_down(float *__restrict__ out, const uint16_t *__restrict__ ht,
           const Dsv4ExpertDev *__restrict__ table, int n_table,
           const int *__restrict__ idx, const float *__restrict__ wts, int topk,
           int hidden, int inter)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char m2lds[];
    __shared__ float accl[MC_KMAX][32];
    const int r0 = blockIdx.x * 32;
    /* the wave index uniform, so that the slot's expert lookup is scalar
     * loads, counted apart from the h loads in flight before it */
    const int tid = threadIdx.x, lane = tid & 63,
              w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = blockDim.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int nsb = inter >> 5;
    const size_t rowb = (size_t)inter >> 1;
    const int nu = (int)(rowb / M2_UB);
    const int pitch = mc_pitch(inter);
    unsigned char *region = m2lds + (size_t)w * m2_wave_b(inter);
    uint16_t *hl = (uint16_t *)region;
    unsigned char *buf = region + m2_hplanes_b(inter);
    const uint16_t *bl = hl + min(r, MC_NT - 1) * pitch;

    for (int k = w; k < topk; k += nw) {
        /* slot k's planes are contiguous in ht: MC_NT * inter elements; with
         * NU known they are requested before the expert lookup, which they
         * do not depend on */
        const uint16_t *hk = ht + (size_t)k * MC_NT * inter;
        constexpr int IN = 512 * (NU > 0 ? NU : 1);        /* inter */
        constexpr int NH = MC_NT * IN / 512;               /* 1 KB pieces per wave */
        u32x4 hv[NH];
        if constexpr (NU > 0) {
#pragma unroll
            for (int j = 0; j < NH; j++)
                hv[j] = *(const DSV4_GLOBAL u32x4 *)(hk + 512 * j + 8 * lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        const Dsv4ExpertDev E = mc_expert(table, n_table, idx, k);
        /* (a registered expert has all six pointers, a missing one none: the
         * pass tests the pointer it reads, so one load serves both) */
        if (!E.w2) {
            /* (an empty use of the planes on this path too, so that their
             * loads stay ahead of the lookup's branch) */
            if constexpr (NU > 0) {
#pragma unroll
                for (int j = 0; j < NH; j++) asm volatile("" ::"v"(hv[j]));
            }
            if (lane < 32) accl[k][lane] = __builtin_nanf("");
            continue;
        }
        const uint8_t *base = E.w2 + (size_t)r0 * rowb;
        const uint8_t *sb = E.s2 + (size_t)r0 * nsb;
        v4f res[2];
        if constexpr (NU > 0) {
            __builtin_amdgcn_sched_barrier(0);
            M2Unit P[D];
            m2_prologue<D>(P, base, rowb, sb, nsb, NU, lane);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NH; j++) {
                const int e = 512 * j + 8 * lane, c = e / IN;
                *reinterpret_cast<u32x4 *>(hl + c * pitch + (e - c * IN)) = hv[j];
            }
            m2_tiles2<D, NU>(res, P, base, rowb, sb, nsb, buf, bl, lane);
        } else {
            for (int e = 8 * lane; e < MC_NT * inter; e += 512) {
                const int c = e / inter;
                *reinterpret_cast<u32x4 *>(hl + c * pitch + (e - c * inter)) =
                    *(const DSV4_GLOBAL u32x4 *)(hk + e);
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                M2Unit P[D];
                m2_prologue<D>(P, base + (size_t)16 * t * rowb, rowb, sb + (size_t)16 * t * nsb,
                               nsb, nu, lane);
                res[t] = m2_tile<D, 0>(P, base + (size_t)16 * t * rowb, rowb,
                                       sb + (size_t)16 * t * nsb, nsb, nu, buf, bl, lane);
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v4f s = term_sum(res[t], lane);
            if (r == 0) {
#pragma unroll
                for (int j = 0; j < 4; j++) accl[k][16 * t + 4 * g + j] = s[j];
            }
        }
    }
    __syncthreads();
    if (tid < 32) {
        float o = 0.0f;
        for (int kk = 0; kk < topk; kk++) {
            const float p = wts[kk] * accl[kk][tid];
            o = o + p;
        }
        out[r0 + tid] = o;
    }
}

/* ------------------------------------------------------------ one launch
 *
 * Pass A and pass B in one launch of 8-wave workgroups. Workgroups [0, ga)
 * run pass A over 64 h-rows (mc2_gate_up_body with four row tiles;
 * workgroup b is row block b % nx of slot b / nx, nx = inter / 64), the
 * others pass B over 32 output rows, wave w taking slots w, w + 8, ... as
 * k_mc2_down does. For each slot a pass-B wave requests its first weight
 * units (they do not depend on h), then waits until all nx pass-A
 * workgroups of the slot have published h_k, then stages h_k and runs both
 * row tiles with k_mc2_down's arithmetic; the k-ordered combine is
 * k_mc2_down's, so the output has the two-launch form's bits.
 *
 * THE HAND-OFF, ACROSS XCDs. Each XCD has its own L2, and a release or
 * acquire fence at agent scope writes back or invalidates that whole L2 --
 * measured, a fence per workgroup (and per slot of a pass-B wave) took the
 * launch from 39 to 87 us. So the data crossing XCDs never lives in a
 * non-coherent line instead: pass A stores h with agent-scope atomic
 * stores (written through to the device's coherence point), waits for them
 * to complete (s_waitcnt), then counts itself in with an atomic add on the
 * slot's counter in `sync`; pass B polls the counter and reads h with
 * agent-scope atomic loads (served from the coherence point, never from a
 * stale line).
 *
 * ENDING. The workgroups of one XCD are dispatched in increasing id, so
 * every pass-A workgroup is running or done before a pass-B workgroup can
 * take a CU, and pass A waits on nothing: the waits end. A wait that still
 * exceeds MC_SPIN polls gives up, marks sync[MC_KMAX + 1] and leaves NaN in
 * the rows. The last pass-B workgroup to finish (sync[MC_KMAX] counts them)
 * returns the counters to zero, so the next call starts from zeros without
 * a memset (and a captured graph replays). */
constexpr int MC_SYNC_WORDS = MC_KMAX + 2;
static_assert(MC_SYNC_WORDS == DSV4_MOE_SYNC_WORDS, "the counters' size");
constexpr int MC_SPIN = 1 << 22;

/* Wave-uniform: true once *cnt reaches need (lane 0 polls). */
__device__ __forceinline__ bool slot_wait(uint32_t *cnt, uint32_t need)
{
    uint32_t v = 0;
    if ((threadIdx.x & 63) == 0) {
        for (int it = 0; it < MC_SPIN; it++) {
            v = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (v >= need) break;
            __builtin_amdgcn_s_sleep(2);
        }
    }
    return __shfl(v, 0, 64) >= need;
}

/* Slot k's h planes into a pass-B wave's LDS (pitch mc_pitch(inter)) with
 * agent-scope atomic loads, 16 bytes per lane per piece. */
template <int NUB>
__device__ __forceinline__ void mc2_h_coherent(uint16_t *hl, const uint16_t *hk, int inter,
                                               int lane)
{
    const int pitch = mc_pitch(inter);
    if constexpr (NUB > 0) {
        constexpr int IN = 512 * NUB;                      /* inter */
        constexpr int NH = MC_NT * IN / 512;               /* 1 KB pieces per wave */
        uint64_t hv[2 * NH];
#pragma unroll
        for (int j = 0; j < NH; j++) {
            const uint64_t *q = (const uint64_t *)(hk + 512 * j + 8 * lane);
            hv[2 * j] = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            hv[2 * j + 1] = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int j = 0; j < NH; j++) {
            const int e = 512 * j + 8 * lane, c = e / IN;
            uint64_t *d = reinterpret_cast<uint64_t *>(hl + c * pitch + (e - c * IN));
            d[0] = hv[2 * j];
            d[1] = hv[2 * j + 1];
        }
    } else {
        for (int e = 8 * lane; e < MC_NT * inter; e += 512) {
            const int c = e / inter;
            const uint64_t *q = (const uint64_t *)(hk + e);
            uint64_t *d = reinterpret_cast<uint64_t *>(hl + c * pitch + (e - c * inter));
            d[0] = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            d[1] = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

/* LDS of the one-launch form: pass A's (x planes, eight unit buffers) or
 * pass B's (eight waves' h planes and unit buffers). */
__host__ __device__ __forceinline__ size_t m2_lds_fused(int hidden, int inter)
{
    const size_t a = (size_t)MC_NT * mc_pitch(hidden) * 2 + 8 * M2_WBUF;
    const size_t b = 8 * m2_wave_b(inter);
    return a > b ? a : b;
}

template <int DA, int NUA, int DB, int NUB>
__global__ void __launch_bounds__(512)
k_mc2_fused(float *__restrict__ out, uint16_t *__restrict__ ht, const float *__restrict__ x,
            const Dsv4ExpertDev *__restrict__ table, int n_table, const int *__restrict__ idx,
            const float *__restrict__ wts, int topk, int hidden, int inter, float limit,
            uint32_t *__restrict__ sync, int ga)
{
    const int nx = inter >> 6;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if ((int)blockIdx.x < ga) {
        const int k = (int)blockIdx.x / nx;
        (void)mc2_gate_up_body<DA, NUA, 4, true>(ht, x, table, n_table, idx, hidden, inter,
                                                 limit, (int)blockIdx.x - k * nx, k);
        /* h_k's rows of this workgroup are wave 0's stores (or none, for a
         * missing expert): wait until they are complete, then count in */
        if (w == 0) {
            __builtin_amdgcn_s_waitcnt(0);
            if (lane == 0)
                __hip_atomic_fetch_add(sync + k, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    extern __shared__ __attribute__((aligned(16))) unsigned char m2lds[];
    __shared__ float accl[MC_KMAX][32];
    const int r0 = ((int)blockIdx.x - ga) * 32;
    const int r = lane & 15, g = lane >> 4;
    const int nsb = inter >> 5;
    const size_t rowb = (size_t)inter >> 1;
    const int nu = (int)(rowb / M2_UB);
    const int pitch = mc_pitch(inter);
    unsigned char *region = m2lds + (size_t)w * m2_wave_b(inter);
    uint16_t *hl = (uint16_t *)region;
    unsigned char *buf = region + m2_hplanes_b(inter);
    const uint16_t *bl = hl + min(r, MC_NT - 1) * pitch;
    for (int k = w; k < topk; k += 8) {
        const Dsv4ExpertDev E = mc_expert(table, n_table, idx, k);
        if (!E.w1) {
            if (lane < 32) accl[k][lane] = __builtin_nanf("");
            continue;
        }
        /* slot k's planes are contiguous in ht: MC_NT * inter elements */
        const uint16_t *hk = ht + (size_t)k * MC_NT * inter;
        const uint8_t *base = E.w2 + (size_t)r0 * rowb;
        const uint8_t *sb = E.s2 + (size_t)r0 * nsb;
        v4f res[2];
        bool ok;
        if constexpr (NUB > 0) {
            M2Unit P[DB];
            m2_prologue<DB>(P, base, rowb, sb, nsb, NUB, lane);
            ok = slot_wait(sync + k, (uint32_t)nx);
            mc2_h_coherent<NUB>(hl, hk, inter, lane);
            m2_tiles2<DB, NUB>(res, P, base, rowb, sb, nsb, buf, bl, lane);
        } else {
            ok = slot_wait(sync + k, (uint32_t)nx);
            mc2_h_coherent<0>(hl, hk, inter, lane);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                M2Unit P[DB];
                m2_prologue<DB>(P, base + (size_t)16 * t * rowb, rowb, sb + (size_t)16 * t * nsb,
                                nsb, nu, lane);
                res[t] = m2_tile<DB, 0>(P, base + (size_t)16 * t * rowb, rowb,
                                        sb + (size_t)16 * t * nsb, nsb, nu, buf, bl, lane);
            }
        }
        if (!ok && lane == 0)
            __hip_atomic_store(sync + MC_KMAX + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v4f sm = term_sum(res[t], lane);
            if (r == 0) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    accl[k][16 * t + 4 * g + j] = ok ? sm[j] : __builtin_nanf("");
            }
        }
    }
    __syncthreads();
    if (tid < 32) {
        float o = 0.0f;
        for (int kk = 0; kk < topk; kk++) {
            const float p = wts[kk] * accl[kk][tid];
            o = o + p;
        }
        out[r0 + tid] = o;
    }
    /* every wave of this workgroup is past its waits: count it out; the
     * last one zeroes the counters for the next call */
    if (tid == 0) {
        const uint32_t gb = gridDim.x - (uint32_t)ga;
        if (__hip_atomic_fetch_add(sync + MC_KMAX, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == gb - 1) {
            for (int kk = 0; kk < topk; kk++)
                __hip_atomic_store(sync + kk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sync + MC_KMAX, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

/* ------------------------------------------------------- batched (prefill)
 *
 * The routed half of the reference's moe_n (dsv4_layer.c:714-855) for nt
 * tokens. The batch's (token, k) pairs ask for the distinct experts in
 * first-request order; each distinct expert streams its weights once, for
 * every pair routed to it (the reference's union, :728-739, and
 * run_expert_n, :681-703). Per pair the products are the staged form's
 * (k_mc2_gate_up / k_mc2_down), column for column: the matrix core computes
 * each result column from its own B column, so a pair sitting in columns
 * 3j..3j+2 of a 16-column tile gets the bits it gets in columns 0..2 alone.
 * The unit order, the two alternating accumulators, the term sum and the
 * k-ordered combine are the single-token ones, so every token's output row
 * is bit-identical to the single-token call on that token.
 *
 * LAUNCHES: k_mn_split (x -> bf16 term planes, every token), k_mn_route (one
 * workgroup: slots, per-slot pair lists), k_mn_pass<GATE> (h of every pair),
 * k_mn_pass<DOWN> (acc_k of every pair), k_mn_combine (the k-ordered sum). */
constexpr int MN_TOK = 5;                          /* pairs per 16-column B tile  */
constexpr int MN_BROWS = MN_TOK * MC_NT;           /* B term rows per tile (15)   */
constexpr int MN_BP = 512 + 8;                     /* LDS pitch of a term row     */
constexpr int MN_BBUF = MN_BROWS * MN_BP;          /* bf16 per B buffer           */
constexpr int MN_NL = (16 * 64) / 256;             /* 16-byte B pieces per thread */
constexpr int MN_PMAX = 4096;                      /* pairs per call              */

/* Slot s: expert eid[s] (-1 for ids outside the table: its pairs give NaN,
 * as the single-token call does), its pairs plist[off[s] .. off[s] + cnt[s])
 * in pair order (pair p = token * topk + k). */
struct MnRoute {
    int n_uniq, n_pairs, pad[62];
    int eid[MN_PMAX], off[MN_PMAX], cnt[MN_PMAX], plist[MN_PMAX];
};

__global__ void __launch_bounds__(256)
k_mn_split(uint16_t *__restrict__ xt, const float *__restrict__ x, int nt, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nt * n) return;
    const int t = i / n, c = i - t * n;
    uint32_t tt[MC_NT];
    bf16_terms(x[i], tt);
#pragma unroll
    for (int q = 0; q < MC_NT; q++) xt[((size_t)t * MC_NT + q) * n + c] = (uint16_t)tt[q];
}

/* One workgroup of 1024. Pair p's key is its expert id (-1 outside the
 * table); its rank is the number of earlier pairs with the same key; rank 0
 * marks the key's first request, and the firsts in pair order number the
 * slots. A pair's place in plist is (pairs of earlier slots) + its rank. */
__global__ void __launch_bounds__(1024)
k_mn_route(MnRoute *__restrict__ rt, const int *__restrict__ idx, int np, int n_table)
{
    constexpr int RND = MN_PMAX / 1024;
    __shared__ int key[MN_PMAX];
    __shared__ int slot[MN_PMAX];
    __shared__ int wcnt[RND * 16];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int r = 0; r < RND; r++) {
        const int p = r * 1024 + tid;
        if (p < np) {
            const int e = idx[p];
            key[p] = (e >= 0 && e < n_table) ? e : -1;
        }
    }
    __syncthreads();
    int q0[RND], rk[RND];
    unsigned long long bal[RND];
#pragma unroll
    for (int r = 0; r < RND; r++) {
        const int p = r * 1024 + tid;
        int f = p, c = 0;
        if (p < np) {
            const int kp = key[p];
            for (int q = 0; q < p; q++)
                if (key[q] == kp) {
                    if (c == 0) f = q;
                    c++;
                }
        }
        q0[r] = f;
        rk[r] = c;
        bal[r] = __ballot(p < np && c == 0);
        if (lane == 0) wcnt[r * 16 + w] = __popcll(bal[r]);
    }
    __syncthreads();
    int nu = 0;
    for (int i = 0; i < RND * 16; i++) nu += wcnt[i];
#pragma unroll
    for (int r = 0; r < RND; r++) {
        const int p = r * 1024 + tid;
        if (p < np && rk[r] == 0) {
            int base = 0;
            for (int i = 0; i < r * 16 + w; i++) base += wcnt[i];
            slot[p] = base + __popcll(bal[r] & ((1ull << lane) - 1ull));
        }
    }
    __syncthreads();
    int sl[RND];
#pragma unroll
    for (int r = 0; r < RND; r++) {
        const int p = r * 1024 + tid;
        sl[r] = p < np ? slot[q0[r]] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RND; r++) {
        const int p = r * 1024 + tid;
        if (p < np) slot[p] = sl[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RND; r++) {
        const int p = r * 1024 + tid;
        if (p >= np) continue;
        const int sp = sl[r];
        int less = 0, same = 0;
        for (int q = 0; q < np; q++) {
            const int sq = slot[q];
            less += sq < sp;
            same += sq == sp;
        }
        rt->plist[less + rk[r]] = p;
        if (rk[r] == 0) {
            rt->off[sp] = less;
            rt->cnt[sp] = same;
            rt->eid[sp] = key[p];
        }
    }
    if (tid == 0) {
        rt->n_uniq = nu;
        rt->n_pairs = np;
    }
}

/* The B terms of unit u for a pass's nb pairs: term row (j MC_NT + c) is
 * plane c of source row prow[j] (src [row][MC_NT][K]), 512 elements from
 * 512 u. Requested by every thread (rows past the pass read prow[0], rows
 * past the tile too: no branch before the loads), stored as zeros past nb. */
__device__ __forceinline__ void mn_bload(u32x4 *v, const uint16_t *src, const int *prow,
                                         int nb, int K, int u)
{
#pragma unroll
    for (int m = 0; m < MN_NL; m++) {
        const int i = (int)threadIdx.x + 256 * m;
        const int row = i >> 6, piece = i & 63;
        const int j = row / MC_NT, c = row - j * MC_NT;
        const int pr = j < nb ? prow[j] : prow[0];
        v[m] = *(const DSV4_GLOBAL u32x4 *)(src + ((size_t)pr * MC_NT + c) * K + 512 * u +
                                            8 * piece);
    }
}

__device__ __forceinline__ void mn_bstore(uint16_t *bb, const u32x4 *v, int nb)
{
#pragma unroll
    for (int m = 0; m < MN_NL; m++) {
        const int i = (int)threadIdx.x + 256 * m;
        const int row = i >> 6, piece = i & 63;
        if (row < MN_BROWS)
            *reinterpret_cast<u32x4 *>(bb + row * MN_BP + 8 * piece) =
                row / MC_NT < nb ? v[m] : u32x4{0u, 0u, 0u, 0u};
    }
}

/* m2_mac with the B tile of a pass: column r reads term row r (15 rows; the
 * unused column 15 repeats row 14). Same steps, same accumulators. */
__device__ __forceinline__ void mn_mac(v4f *acc, const unsigned char *buf, const uint16_t *bb,
                                       int lane, bool live)
{
    const int r = lane & 15, g = lane >> 4;
    const u32x4 sv = *reinterpret_cast<const u32x4 *>(buf + M2_SOFF + r * 16);
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    const uint16_t *bl = bb + min(r, MN_BROWS - 1) * MN_BP;
#pragma unroll
    for (int qb = 0; qb < 4; qb++) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(buf + r * M2_WP + 64 * qb + 16 * g);
        const float sc = live ? dec_e8m0((sw[qb] >> (8 * g)) & 0xFFu) : 0.0f;
        const uint32_t d[4] = {a.x, a.y, a.z, a.w};
        v8bf b[4];
#pragma unroll
        for (int m = 0; m < 4; m++)
            b[m] = __builtin_bit_cast(v8bf, *reinterpret_cast<const u32x4 *>(
                                                bl + 128 * qb + 32 * g + 8 * m));
#pragma unroll
        for (int m = 0; m < 4; m++)
            acc[qb & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(d[m], sc), b[m],
                                                                   acc[qb & 1], 0, 0, 0);
    }
}

/* Columns c0..c0+MC_NT-1 of a result tile summed in column order, per row
 * (term_sum for the pair at columns c0..). */
__device__ __forceinline__ v4f term_sum_at(const v4f &d, int lane, int c0)
{
    const int base = (lane & ~15) + c0;
    v4f s;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float a = __shfl(d[j], base + 0, 64);
#pragma unroll
        for (int t = 1; t < MC_NT; t++) a = a + __shfl(d[j], base + t, 64);
        s[j] = a;
    }
    return s;
}

__device__ __forceinline__ void mn_wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* One pass kernel for both halves; workgroup (row block, slot), 4 waves, a
 * 16-row tile each:
 *   GATE: rows blockIdx.x * 32 + 16 (w >> 1) of w1 (w even) / w3 (w odd),
 *         B = the pairs' tokens' x terms (src = xt [nt][MC_NT][hidden]);
 *         SwiGLU, h terms into dst = ht [pair][MC_NT][inter];
 *   DOWN: rows blockIdx.x * 64 + 16 w of w2, B = the pairs' h terms (src =
 *         ht); acc_k into dst = accp [pair][hidden].
 * The slot's pairs run in passes of MN_TOK. Per unit: each wave stages its
 * weight unit (requested D units earlier) in its own buffer, requests the
 * next unit's B and the weight unit D ahead (B first: the end-of-unit wait
 * for B then leaves that weight unit in flight), runs the unit, stores the
 * next B into the other buffer, and the workgroup meets at one barrier. NU >
 * 0: the unit count, every unit live (k_mc2_*'s NU > 0 forms); NU == 0: a
 * run-time count padded to a multiple of D with dead units, as m2_tile's
 * run-time form pads (D must then equal the single-token form's, 3). */
template <int D, int NU, bool GATE>
__global__ void __launch_bounds__(256)
k_mn_pass(void *__restrict__ dst, const uint16_t *__restrict__ src,
          const MnRoute *__restrict__ rt, const Dsv4ExpertDev *__restrict__ table,
          int topk, int hidden, int inter, float limit)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char mnlds[];
    __shared__ float red[2][2][MN_TOK][16];             /* GATE: [tile][mat][pair][row] */
    __shared__ int prow[MN_TOK], pidx[MN_TOK];
    const int sl = blockIdx.y;
    if (sl >= rt->n_uniq) return;                       /* the whole workgroup */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int e = rt->eid[sl], cnt = rt->cnt[sl], off = rt->off[sl];
    const Dsv4ExpertDev E = e >= 0 ? table[e]
                                   : Dsv4ExpertDev{nullptr, nullptr, nullptr, nullptr, nullptr,
                                                   nullptr};
    if (!E.w1) {
        if (!GATE) {                                    /* as k_mc2_down: NaN results */
            float *accp = (float *)dst;
            for (int i = tid; i < cnt * 64; i += blockDim.x)
                accp[(size_t)rt->plist[off + i / 64] * hidden + blockIdx.x * 64 + (i & 63)] =
                    __builtin_nanf("");
        }
        return;
    }
    const int K = GATE ? hidden : inter;
    const int nsb = K >> 5;
    const size_t rowb = (size_t)K >> 1;
    const int nu = NU > 0 ? NU : (int)(rowb / M2_UB);
    const int nup = NU > 0 ? NU : ((nu + D - 1) / D) * D;   /* units run, dead included */
    const int mat = GATE ? (w & 1) : 0, tile = GATE ? (w >> 1) : w;
    const int o0 = GATE ? blockIdx.x * 32 + 16 * tile : blockIdx.x * 64 + 16 * w;
    const uint8_t *base = (GATE ? (mat ? E.w3 : E.w1) : E.w2) + (size_t)o0 * rowb;
    const uint8_t *sb = (GATE ? (mat ? E.s3 : E.s1) : E.s2) + (size_t)o0 * nsb;
    uint16_t *bbuf = (uint16_t *)mnlds;                             /* [2][MN_BBUF] */
    unsigned char *buf = mnlds + (size_t)2 * MN_BBUF * 2 + (size_t)w * M2_WBUF;
    const int r = lane & 15, g = lane >> 4;

    for (int p0 = 0; p0 < cnt; p0 += MN_TOK) {
        const int nb = min(MN_TOK, cnt - p0);
        __syncthreads();                                /* the last pass's epilogue */
        if (tid < MN_TOK) {
            const int p = rt->plist[off + p0 + min(tid, nb - 1)];
            pidx[tid] = p;
            prow[tid] = GATE ? p / topk : p;
        }
        __syncthreads();
        u32x4 bv[MN_NL];
        M2Unit P[D];
        mn_bload(bv, src, prow, nb, K, 0);
        __builtin_amdgcn_sched_barrier(0);
        m2_prologue<D>(P, base, rowb, sb, nsb, nu, lane);
        __builtin_amdgcn_sched_barrier(0);
        mn_bstore(bbuf, bv, nb);
        __syncthreads();
        v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
        auto unit = [&](int u, M2Unit &slot) {
            m2_stage(buf, slot, lane);
            mn_bload(bv, src, prow, nb, K, min(u + 1, nu - 1));
            __builtin_amdgcn_sched_barrier(0);
            if (NU == 0 || u + D < nup)
                m2_load(slot, base, rowb, sb, nsb, min(u + D, nu - 1), lane);
            __builtin_amdgcn_sched_barrier(0);
            mn_wave_sync();
            mn_mac(acc, buf, bbuf + (u & 1) * MN_BBUF, lane, u < nu);
            mn_bstore(bbuf + ((u + 1) & 1) * MN_BBUF, bv, nb);
            __syncthreads();
        };
        if constexpr (NU > 0) {
#pragma unroll
            for (int u = 0; u < NU; u++) unit(u, P[u % D]);
        } else {
            for (int u0 = 0; u0 < nup; u0 += D) {
#pragma unroll
                for (int j = 0; j < D; j++) unit(u0 + j, P[j]);
            }
        }
        const v4f res = acc[0] + acc[1];
        for (int j = 0; j < nb; j++) {
            const v4f sj = term_sum_at(res, lane, MC_NT * j);
            if (r == 0) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if (GATE)
                        red[tile][mat][j][4 * g + jj] = sj[jj];
                    else
                        ((float *)dst)[(size_t)pidx[j] * hidden + o0 + 4 * g + jj] = sj[jj];
                }
            }
        }
        if (GATE) {
            __syncthreads();
            uint16_t *ht = (uint16_t *)dst;
            for (int q = tid; q < 2 * nb * 16; q += blockDim.x) {
                const int t = q / (nb * 16), rem = q - t * nb * 16;
                const int j = rem >> 4, i = rem & 15;
                uint32_t tt[MC_NT];
                bf16_terms(swiglu1(red[t][0][j][i], red[t][1][j][i], limit), tt);
#pragma unroll
                for (int c = 0; c < MC_NT; c++)
                    ht[((size_t)pidx[j] * MC_NT + c) * inter + blockIdx.x * 32 + 16 * t + i] =
                        (uint16_t)tt[c];
            }
        }
    }
}

/* out[t][i] = ((0 + w_0 acc_0[i]) + w_1 acc_1[i]) + ...: k_mc2_down's
 * combine, per token (the reference's k-ordered sum, dsv4_layer.c:829-839). */
__global__ void __launch_bounds__(256)
k_mn_combine(float *__restrict__ out, const float *__restrict__ accp,
             const float *__restrict__ wts, int topk, int hidden)
{
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    float o = 0.0f;
    for (int k = 0; k < topk; k++) {
        const float p = wts[(size_t)t * topk + k] * accp[((size_t)t * topk + k) * hidden + i];
        o = o + p;
    }
    out[(size_t)t * hidden + i] = o;
}

size_t mn_lds() { return (size_t)2 * MN_BBUF * 2 + 4 * M2_WBUF; }

size_t m2_lds_a(int hidden) { return (size_t)MC_NT * mc_pitch(hidden) * 2 + 4 * M2_WBUF; }
size_t m2_lds_b(int topk, int inter) { return (size_t)m2_down_waves(topk) * m2_wave_b(inter); }

bool m2_shape_ok(int topk, int hidden, int inter)
{
    if (topk <= 0 || topk > MC_KMAX || hidden <= 0 || inter <= 0 ||
        (hidden % 512) || (inter % 512) || (inter % 32) || (hidden % 32))
        return false;
    const size_t cap = dsv4_lds_limit() - 8 * 1024;      /* static LDS of the kernels */
    return m2_lds_a(hidden) <= cap && m2_lds_b(topk, inter) <= cap;
}

size_t mc_lds_a(int hidden) { return (size_t)(MC_NT + 1) * mc_pitch(hidden) * 2; }
size_t mc_lds_b(int topk, int inter) { return (size_t)(topk * MC_NT + 1) * mc_pitch(inter) * 2; }

int mc_env(const char *name, int dflt)
{
    const char *e = getenv(name);
    return e ? atoi(e) : dflt;
}

bool mc_shape_ok(int topk, int hidden, int inter)
{
    if (topk <= 0 || topk > MC_KMAX || hidden <= 0 || inter <= 0 ||
        (hidden & 127) || (inter & 127))
        return false;
    const size_t cap = dsv4_lds_limit() - 16 * 1024;     /* static LDS of the kernels */
    return mc_lds_a(hidden) <= cap && mc_lds_b(topk, inter) <= cap;
}

template <typename K>
void mc_lds_optin(K kernel)
{
    (void)dsv4_lds_optin((const void *)kernel, dsv4_lds_limit() - 16 * 1024, "routed experts");
}

size_t mc_scratch_bytes(int topk, int hidden, int inter)
{
    return a256((size_t)MC_NT * hidden * 2) + a256((size_t)topk * MC_NT * inter * 2);
}

} // namespace

size_t dsv4_moe_scratch_bytes(int topk, int hidden, int inter)
{
    if (topk <= 0 || hidden <= 0 || inter <= 0) return 0;
    const size_t valu = a256((size_t)topk * inter * sizeof(float));
    const size_t mc = (mc_shape_ok(topk, hidden, inter) || m2_shape_ok(topk, hidden, inter))
                    ? mc_scratch_bytes(topk, hidden, inter) : 0;
    return valu > mc ? valu : mc;
}

int dsv4_moe_fp4_launch(float *d_out, const float *d_x,
                        const Dsv4ExpertDev *d_table, int n_table,
                        const int *d_idx, const float *d_w, int topk,
                        int hidden, int inter, float limit, void *scratch,
                        hipStream_t st)
{
    /* Forms (DSV4_GPU_MOE_MC): 2, the default, is the staged matrix-core
     * form -- weights stream in 4-row x 256-byte loads (about 6.3 TB/s from
     * HBM on MI355X) and reach the MFMA fragment order through wave-private
     * LDS; 1 is the fragment-order form, whose 16-row x 64-byte loads stream
     * at about 4.7 TB/s; 0 is the VALU form, also the fallback for shapes and
     * alignments the matrix-core forms do not take. They differ only in the
     * f32 summation order inside a row, and each gives the same bits on
     * every run. */
    const int form = mc_env("DSV4_GPU_MOE_MC", 2);
    const bool m2 = form == 2 && m2_shape_ok(topk, hidden, inter)
                 && ((uintptr_t)d_x & 15u) == 0;
    if (!m2 && (form != 1 || !mc_shape_ok(topk, hidden, inter)))
        return dsv4_moe_fp4_valu_launch(d_out, d_x, d_table, n_table, d_idx, d_w, topk,
                                        hidden, inter, limit, (float *)scratch, st);
    uint16_t *xt = (uint16_t *)scratch;
    uint16_t *ht = (uint16_t *)((char *)scratch + a256((size_t)MC_NT * hidden * 2));
    if (!m2) {
        hipLaunchKernelGGL(k_mc_split, dim3((hidden + 255) / 256), dim3(256), 0, st, xt, d_x,
                           hidden);
        HIP_OK(hipGetLastError(), "moe split launch");
    }
    uint32_t *sync = dsv4_moe_sync();
    const size_t lf = m2_lds_fused(hidden, inter);
    /* DSV4_GPU_MOE_FUSE=1: one launch, where a workgroup fits a CU's LDS
     * with the static arrays and inter is a multiple of 64 rows. Not the
     * default: at C3 it measured 40.7 us against 38.8 us for the two
     * launches. Every expert's h completes at about the same time (pass A's
     * workgroups all run at once), so pass B's per-slot waits end together
     * and the launch only trades the kernel boundary for its own hand-off;
     * the same bits either way. */
    if (m2 && sync && mc_env("DSV4_GPU_MOE_FUSE", 0) != 0 && inter % 64 == 0 &&
        lf + 16 * 1024 <= dsv4_lds_limit()) {
        static bool optedf = false;
        if (!optedf) {
            mc_lds_optin(k_mc2_fused<2, 14, 2, 4>); mc_lds_optin(k_mc2_fused<2, 14, 3, 0>);
            mc_lds_optin(k_mc2_fused<3, 0, 2, 4>); mc_lds_optin(k_mc2_fused<3, 0, 3, 0>);
            optedf = true;
        }
        const int ga = (inter / 64) * topk, gb = hidden / 32;
        const int nua = hidden / 512, nub = inter / 512;
#define M2_F(DA, NUA, DB, NUB) hipLaunchKernelGGL((k_mc2_fused<DA, NUA, DB, NUB>), dim3(ga + gb), \
            dim3(512), lf, st, d_out, ht, d_x, d_table, n_table, d_idx, d_w, topk, hidden, inter, \
            limit, sync, ga)
        if (nua == 14) { if (nub == 4) M2_F(2, 14, 2, 4); else M2_F(2, 14, 3, 0); }
        else { if (nub == 4) M2_F(3, 0, 2, 4); else M2_F(3, 0, 3, 0); }
#undef M2_F
        HIP_OK(hipGetLastError(), "moe one-launch");
        return 0;
    }
    if (m2) {
        /* The staged form: two units in flight per wave (three or four
         * measured slower at C3: more bytes in flight per CU only lengthen
         * the memory queues). */
        static bool opted2 = false;
        if (!opted2) {
            mc_lds_optin(k_mc2_gate_up<2, 14>); mc_lds_optin(k_mc2_gate_up<3, 0>);
            mc_lds_optin(k_mc2_down<2, 4>); mc_lds_optin(k_mc2_down<3, 0>);
            opted2 = true;
        }
        const size_t la = m2_lds_a(hidden), lb = m2_lds_b(topk, inter);
        const int nwb = m2_down_waves(topk);
        const dim3 ga(inter / 32, topk), gb(hidden / 32);
        const int nua = hidden / 512, nub = inter / 512;   /* units per row */
#define M2_A(D, NU) hipLaunchKernelGGL((k_mc2_gate_up<D, NU>), ga, dim3(256), la, st, ht, d_x, d_table, n_table, d_idx, hidden, inter, limit)
#define M2_B(D, NU) hipLaunchKernelGGL((k_mc2_down<D, NU>), gb, dim3(64 * nwb), lb, st, d_out, ht, d_table, n_table, d_idx, d_w, topk, hidden, inter)
        if (nua == 14) M2_A(2, 14); else M2_A(3, 0);
        HIP_OK(hipGetLastError(), "moe gate/up launch");
        if (nub == 4) M2_B(2, 4); else M2_B(3, 0);
        HIP_OK(hipGetLastError(), "moe down launch");
#undef M2_A
#undef M2_B
        return 0;
    }
    /* Fragment-order form: one row tile per gate/up workgroup with four
     * weight blocks in flight; two row tiles per down workgroup of eight
     * waves with eight blocks in flight (the best of a sweep; none changes
     * the arithmetic of a row). */
    static bool opted = false;
    if (!opted) {
        mc_lds_optin(k_mc_gate_up<1, 4>);
        mc_lds_optin(k_mc_down<2, 8>);
        opted = true;
    }
    const size_t la = mc_lds_a(hidden);
    hipLaunchKernelGGL((k_mc_gate_up<1, 4>), dim3(inter / 16, topk), dim3(256), la, st, ht, xt,
                       d_table, n_table, d_idx, hidden, inter, limit);
    HIP_OK(hipGetLastError(), "moe gate/up launch");
    const size_t lb = mc_lds_b(topk, inter);
    hipLaunchKernelGGL((k_mc_down<2, 8>), dim3(hidden / 32), dim3(512), lb, st, d_out, ht,
                       d_table, n_table, d_idx, d_w, topk, hidden, inter);
    HIP_OK(hipGetLastError(), "moe down launch");
    return 0;
}

size_t dsv4_moe_n_scratch_bytes(int nt, int topk, int hidden, int inter)
{
    if (nt <= 0 || topk <= 0 || hidden <= 0 || inter <= 0) return 0;
    const size_t single = dsv4_moe_scratch_bytes(topk, hidden, inter);
    if (nt == 1) return single;
    const size_t np = (size_t)nt * topk;
    const size_t batched = a256(sizeof(MnRoute)) + a256((size_t)nt * MC_NT * hidden * 2) +
                           a256(np * MC_NT * inter * 2) + a256(np * hidden * sizeof(float));
    return batched > single ? batched : single;
}

int dsv4_moe_fp4_n_launch(float *d_out, const float *d_x, const Dsv4ExpertDev *d_table,
                          int n_table, const int *d_idx, const float *d_w, int nt, int topk,
                          int hidden, int inter, float limit, void *scratch, hipStream_t st)
{
    if (nt < 1 || topk < 1) return -1;
    const int form = mc_env("DSV4_GPU_MOE_MC", 2);
    const bool batched = nt > 1 && form == 2 && m2_shape_ok(topk, hidden, inter) &&
                         ((uintptr_t)d_x & 15u) == 0 && (size_t)nt * topk <= MN_PMAX &&
                         mn_lds() + 8 * 1024 <= dsv4_lds_limit();
    if (!batched) {
        /* token by token: each token's own call, so its bits by construction */
        for (int t = 0; t < nt; t++)
            if (dsv4_moe_fp4_launch(d_out + (size_t)t * hidden, d_x + (size_t)t * hidden,
                                    d_table, n_table, d_idx + (size_t)t * topk,
                                    d_w + (size_t)t * topk, topk, hidden, inter, limit,
                                    scratch, st) != 0)
                return -1;
        return 0;
    }
    const int np = nt * topk;
    char *p = (char *)scratch;
    MnRoute *rt = (MnRoute *)p;                         p += a256(sizeof(MnRoute));
    uint16_t *xt = (uint16_t *)p;                       p += a256((size_t)nt * MC_NT * hidden * 2);
    uint16_t *ht = (uint16_t *)p;                       p += a256((size_t)np * MC_NT * inter * 2);
    float *accp = (float *)p;
    const int slots = np < n_table + 1 ? np : n_table + 1;
    static bool opted = false;
    if (!opted) {
        mc_lds_optin(k_mn_pass<2, 14, true>); mc_lds_optin(k_mn_pass<3, 0, true>);
        mc_lds_optin(k_mn_pass<2, 4, false>); mc_lds_optin(k_mn_pass<3, 0, false>);
        opted = true;
    }
    const size_t lds = mn_lds();
    hipLaunchKernelGGL(k_mn_split, dim3((nt * hidden + 255) / 256), dim3(256), 0, st, xt, d_x,
                       nt, hidden);
    hipLaunchKernelGGL(k_mn_route, dim3(1), dim3(1024), 0, st, rt, d_idx, np, n_table);
    HIP_OK(hipGetLastError(), "moe_n route launch");
    const dim3 ga(inter / 32, slots), gb(hidden / 64, slots);
    if (hidden / 512 == 14)
        hipLaunchKernelGGL((k_mn_pass<2, 14, true>), ga, dim3(256), lds, st, (void *)ht, xt, rt,
                           d_table, topk, hidden, inter, limit);
    else
        hipLaunchKernelGGL((k_mn_pass<3, 0, true>), ga, dim3(256), lds, st, (void *)ht, xt, rt,
                           d_table, topk, hidden, inter, limit);
    HIP_OK(hipGetLastError(), "moe_n gate/up launch");
    if (inter / 512 == 4)
        hipLaunchKernelGGL((k_mn_pass<2, 4, false>), gb, dim3(256), lds, st, (void *)accp, ht,
                           rt, d_table, topk, hidden, inter, limit);
    else
        hipLaunchKernelGGL((k_mn_pass<3, 0, false>), gb, dim3(256), lds, st, (void *)accp, ht,
                           rt, d_table, topk, hidden, inter, limit);
    HIP_OK(hipGetLastError(), "moe_n down launch");
    hipLaunchKernelGGL(k_mn_combine, dim3((hidden + 255) / 256, nt), dim3(256), 0, st, d_out,
                       accp, d_w, topk, hidden);
    HIP_OK(hipGetLastError(), "moe_n combine launch");
    return 0;
}
