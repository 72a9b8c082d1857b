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
    (void)hipFuncSetAttribute((const void *)kernel,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)dsv4_lds_limit() - 16 * 1024);
    (void)hipGetLastError();
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
    const size_t mc = mc_shape_ok(topk, hidden, inter) ? mc_scratch_bytes(topk, hidden, inter) : 0;
    return valu > mc ? valu : mc;
}

int dsv4_moe_fp4_launch(float *d_out, const float *d_x,
                        const Dsv4ExpertDev *d_table, int n_table,
                        const int *d_idx, const float *d_w, int topk,
                        int hidden, int inter, float limit, void *scratch,
                        hipStream_t st)
{
    /* The VALU form is the default: on MI355X it is faster at the C3 shape
     * (49.9 vs 77 us), because the MFMA fragment order reads each weight row
     * in 64-byte pieces spread over 16 rows per load, which streams from HBM
     * at about 4.7 TB/s against 6.5 TB/s for 1 KB contiguous loads.
     * DSV4_GPU_MOE_MC=1 selects this matrix-core form. */
    if (!mc_shape_ok(topk, hidden, inter) || !mc_env("DSV4_GPU_MOE_MC", 0))
        return dsv4_moe_fp4_valu_launch(d_out, d_x, d_table, n_table, d_idx, d_w, topk,
                                        hidden, inter, limit, (float *)scratch, st);
    uint16_t *xt = (uint16_t *)scratch;
    uint16_t *ht = (uint16_t *)((char *)scratch + a256((size_t)MC_NT * hidden * 2));
    hipLaunchKernelGGL(k_mc_split, dim3((hidden + 255) / 256), dim3(256), 0, st, xt, d_x,
                       hidden);
    HIP_OK(hipGetLastError(), "moe split launch");
    /* Row tiles per workgroup, waves per down workgroup and weight blocks in
     * flight (none changes the arithmetic of a row). */
    static bool opted = false;
    if (!opted) {
        mc_lds_optin(k_mc_gate_up<1, 4>); mc_lds_optin(k_mc_gate_up<2, 4>);
        mc_lds_optin(k_mc_gate_up<1, 8>); mc_lds_optin(k_mc_gate_up<2, 8>);
        mc_lds_optin(k_mc_down<1, 8>); mc_lds_optin(k_mc_down<2, 8>);
        mc_lds_optin(k_mc_down<1, 4>); mc_lds_optin(k_mc_down<2, 4>);
        opted = true;
    }
    const int ota = mc_env("DSV4_GPU_MOE_OTA", 1) >= 2 ? 2 : 1;
    const int da = mc_env("DSV4_GPU_MOE_DA", 4) >= 8 ? 8 : 4;
    const size_t la = mc_lds_a(hidden);
    const dim3 ga(inter / (16 * ota), topk);
#define MC_A(OT, D) hipLaunchKernelGGL((k_mc_gate_up<OT, D>), ga, dim3(256), la, st, ht, xt, d_table, n_table, d_idx, hidden, inter, limit)
    if (ota == 2) { if (da == 8) MC_A(2, 8); else MC_A(2, 4); }
    else          { if (da == 8) MC_A(1, 8); else MC_A(1, 4); }
#undef MC_A
    HIP_OK(hipGetLastError(), "moe gate/up launch");
    const int otb = mc_env("DSV4_GPU_MOE_OTB", 2) >= 2 ? 2 : 1;
    const int db = mc_env("DSV4_GPU_MOE_DB", 8) >= 8 ? 8 : 4;
    const int wv = mc_env("DSV4_GPU_MOE_WAVES", 8);
    const int nthr = 64 * (wv >= 8 ? 8 : wv >= 4 ? 4 : wv >= 2 ? 2 : 1);
    const size_t lb = mc_lds_b(topk, inter);
    const dim3 gb(hidden / (16 * otb));
#define MC_B(OT, D) hipLaunchKernelGGL((k_mc_down<OT, D>), gb, dim3(nthr), lb, st, d_out, ht, d_table, n_table, d_idx, d_w, topk, hidden, inter)
    if (otb == 2) { if (db == 8) MC_B(2, 8); else MC_B(2, 4); }
    else          { if (db == 8) MC_B(1, 8); else MC_B(1, 4); }
#undef MC_B
    HIP_OK(hipGetLastError(), "moe down launch");
    return 0;
}
