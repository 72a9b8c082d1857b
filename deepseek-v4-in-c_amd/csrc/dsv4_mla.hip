/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_mla.hip - sparse-MLA decode on gfx950: the CSA indexer score, its
 * top-k, and softmax attention over the gathered latent-KV rows.
 *
 * INDEXER SCORE (dsv4_indexer.c:64-85), bit-exact. For each key row t and
 * head h: dot = fma-chain over c ascending of (double)q[h][c] *
 * (double)k[t][c]; then, in head order, `if (dot > 0) total += dot * w[h]`
 * with the multiply and the add rounded separately (this file is built with
 * -ffp-contract=off); out[t] = (float)total * scale, the scale computed by
 * the caller in float as the reference does. Lane = key row: a wave runs
 * the chains of 8 heads for 64 rows, q reaching every lane through a DPP
 * row broadcast fused into the fma (k_iscore). With a top-k to follow, the
 * kernel also builds its level-1 histogram.
 *
 * TOP-K (dsv4_indexer.c:92-106), bit-exact: the k largest, ordered by score
 * descending, ties to the lower index. Scores map to order-preserving 32-bit
 * keys (-0.0 folded into +0.0, since the reference's `>` treats them as
 * equal). The histogram of the key's bits 31..21 gives B, the bin of the
 * k-th largest; every element above B is taken, and each is placed by
 * counting the composites (key << 32 | ~index: score descending, ties to
 * the lower index) ahead of it; an element of B likewise among B's, taken
 * when it ranks below the k-th's place in B. Past 4096 elements in B, a
 * radix select over bits 20..10 and 9..0 first finds T, the key of the k-th
 * largest, and how many elements equal to T are taken (k_tk_part,
 * k_tk_final).
 * Up to 4096 scores, one launch ranks every element directly (k_tk_small).
 * NaN scores follow the reference's scan too: it takes a NaN exactly when
 * that NaN is the lowest index not yet taken, and otherwise the first
 * maximum of the untaken finite scores. NaNs key below every finite score;
 * when any is present, one workgroup sorts the selection and inserts the
 * NaNs where the scan takes them (nan_finish).
 *
 * SPARSE ATTENTION (dsv4_attn.c:60-108): split over the selected rows and a
 * log-sum-exp combine. Partial pass: per split of selected rows, the scores,
 * the split's max m_s, e_j = expf(s_j - m_s), l_s = sum e_j and o_s = sum_j
 * e_j * v_j -- on the matrix cores for bf16 KV (k_attn_mc), on the VALU
 * otherwise (k_attn_partial). Combine: M = max m_s, denom = sum l_s
 * expf(m_s - M) (+ expf(sink - M) when a sink is given: denominator only,
 * not in the max), o = (sum o_s expf(m_s - M)) * (float)(1/denom). Masked
 * (-1) rows take no part. Agrees with the reference within 1e-5 relative.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

#include <stdlib.h>

namespace {

__device__ __forceinline__ float bf16_to_f32(uint16_t b)
{
    return __uint_as_float((uint32_t)b << 16);
}

template <int KF>
__device__ __forceinline__ float key_at(const void *keys, const float *ks,
                                        size_t row, int key_stride, int c)
{
    if (KF == DSV4_GPU_KV_F32)
        return ((const float *)keys)[row * key_stride + c];
    if (KF == DSV4_GPU_KV_BF16)
        return bf16_to_f32(((const uint16_t *)keys)[row * key_stride + c]);
    return dec_e4m3(((const uint8_t *)keys)[row * key_stride + c]) * ks[row];
}

/* ------------------------------------------------------- indexer score */

/* Score kernel geometry: lane = key row, a wave runs the chains of IS_HB
 * heads for its 64 rows; a workgroup of up to IS_MAXW waves covers all the
 * heads of one or more 64-row blocks (its waves loop over head groups when
 * there are more groups than waves). */
constexpr int IS_HB = 8;                        /* heads per wave */
constexpr int IS_MAXW = 4;                      /* waves per workgroup */

/* Top-k constants the score kernel shares: its histogram is the first level
 * of the selection. */
constexpr int TK_KMAX = 4096;
constexpr int TK_BINS = 2048;                   /* top 11 bits of the key */
constexpr int TK_SLICES = 4;                    /* spread of the global atomics */

/* meta words in the scratch */
constexpr int MT_BIN = 2;                       /* B */
constexpr int MT_KREM = 3;                      /* rank of the k-th inside B */
constexpr int MT_NAN = 4;                       /* nonzero: a score is NaN */
constexpr int MT_CNT = 6;                       /* words 6-7: one 64-bit append counter,
                                                 * cand[] in the low word, bsel[] high */

/* Restart the top-k's append counter and NaN flag (one thread). */
__device__ __forceinline__ void meta_restart(uint32_t *meta)
{
    *reinterpret_cast<unsigned long long *>(meta + MT_CNT) = 0ull;
    meta[MT_NAN] = 0u;
}


/* Order-preserving 32-bit key of a score: a > b as floats iff fkey(a) >
 * fkey(b) as integers; -0.0 folds into +0.0 since the reference's `>`
 * treats them as equal. Every NaN keys to 0, below every other score (the
 * smallest, -inf, keys to 0x007FFFFF), so the key's top 11 bits put NaNs
 * alone in bin 0. */
__device__ __forceinline__ uint32_t fkey(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
    if ((u & 0x7FFFFFFFu) == 0u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* One 16-byte piece of a key row, as floats (16 / element-size of them);
 * for FP8 the reference's float product e4m3(code) * row_scale. */
template <int KF>
__device__ __forceinline__ void key_piece(u32x4 v, float rs, float *k)
{
    if (KF == DSV4_GPU_KV_FP8) {
        dec_e4m3x4(v.x, k + 0);
        dec_e4m3x4(v.y, k + 4);
        dec_e4m3x4(v.z, k + 8);
        dec_e4m3x4(v.w, k + 12);
#pragma unroll
        for (int e = 0; e < 16; e++) k[e] = k[e] * rs;
    } else if (KF == DSV4_GPU_KV_BF16) {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            k[2 * e] = __uint_as_float(w4[e] << 16);
            k[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
        }
    } else {
        k[0] = __uint_as_float(v.x); k[1] = __uint_as_float(v.y);
        k[2] = __uint_as_float(v.z); k[3] = __uint_as_float(v.w);
    }
}

/* q of the wave's IS_HB heads for columns c0 .. c0 + 15, one column per
 * lane of each 16-lane row (every row holds the same values): lane l gets
 * q[h0 + j][c0 + l % 16]. Heads past H read head H-1, columns past D the
 * last column. q is the workgroup's LDS copy (an L2 round trip per 16
 * columns would leave the chains waiting whenever there are few rows to
 * overlap them). */
__device__ __forceinline__ void q_cols(float *dst, const float *q, int h0, int H,
                                       int D, int c0, int lane)
{
    const int c = min(c0 + (lane & 15), D - 1);
    /* unconditional loads (clamped head; chain_16 zeroes heads past H): a
     * load under a branch would make the next wait cover every load in
     * flight */
#pragma unroll
    for (int j = 0; j < IS_HB; j++) dst[j] = q[(size_t)min(h0 + j, H - 1) * D + c];
}

/* acc += q(lane R of this 16-lane row) * kd: the broadcast is the DPP
 * row_newbcast form of the fma's first operand (one instruction). q must
 * not have been written by a VALU instruction in the two issue slots before
 * (DPP source hazard); chain_16 separates them with an s_nop, since the
 * compiler does not look inside this asm for hazards. */
template <int R>
__device__ __forceinline__ void fma_bcast(double &acc, double q, double kd)
{
    asm("v_fmac_f64_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
        : "+v"(acc) : "v"(q), "v"(kd), "n"(R));
}

/* Chain steps for column c0 + R of every head of the group: q[.][c0 + R]
 * reaches all lanes by the row broadcast of lane R. */
template <int R>
__device__ __forceinline__ void chain_col(double *acc, const double *qv, float kf)
{
    const double kd = (double)kf;
#pragma unroll
    for (int j = 0; j < IS_HB; j++) fma_bcast<R>(acc[j], qv[j], kd);
}

/* Sixteen columns c0 .. c0 + 15 of the chains (FULL), or the first n of
 * them at the end of a row; k holds the row's elements of those columns and
 * nh the number of the group's heads below H (q of the others is zero). */
template <bool FULL>
__device__ __forceinline__ void chain_16(double *acc, const float *qf, const float *k, int n,
                                         int nh)
{
    double qv[IS_HB];
#pragma unroll
    for (int j = 0; j < IS_HB; j++) qv[j] = j < nh ? (double)qf[j] : 0.0;
    /* two wait states between the conversions above and the broadcasts */
    asm volatile("s_nop 1"
                 : "+v"(qv[0]), "+v"(qv[1]), "+v"(qv[2]), "+v"(qv[3]),
                   "+v"(qv[4]), "+v"(qv[5]), "+v"(qv[6]), "+v"(qv[7]));
#define DSV4_COL(R) if (FULL || R < n) chain_col<R>(acc, qv, k[R]);
    DSV4_COL(0) DSV4_COL(1) DSV4_COL(2) DSV4_COL(3) DSV4_COL(4) DSV4_COL(5)
    DSV4_COL(6) DSV4_COL(7) DSV4_COL(8) DSV4_COL(9) DSV4_COL(10) DSV4_COL(11)
    DSV4_COL(12) DSV4_COL(13) DSV4_COL(14) DSV4_COL(15)
#undef DSV4_COL
}

/* RoPE of the last rd elements of a vector (dsv4_rope.c:105-119), applied by
 * a kernel to its own copy of an input: rd == 0 is none. */
struct Dsv4Rope {
    const float *cs = nullptr, *sn = nullptr;
    int pos = 0, half = 0, rd = 0, inverse = 0;
};

__device__ __forceinline__ void rope_pair_cs(float &a, float &b, float c, float s0, int inverse)
{
    const float s = inverse ? -s0 : s0;
    const float re = a, im = b;
    a = re * c - im * s;
    b = re * s + im * c;
}

/* A kernel's RoPE row at pos in LDS: thread p < rd/2 loads its pair's cos
 * and sin with rope_row_load (issued before the kernel's other loads, so the
 * latencies overlap) and stores them with rope_row_store before the
 * kernel's next barrier. */
constexpr int RP_MAX = 128;                      /* rd <= 2 RP_MAX */
struct RopeRow {
    float c = 0.0f, s = 0.0f;
};

__device__ __forceinline__ RopeRow rope_row_load(const Dsv4Rope &r)
{
    RopeRow v;
    if (r.rd && (int)threadIdx.x < r.rd / 2) {
        v.c = r.cs[(size_t)r.pos * r.half + threadIdx.x];
        v.s = r.sn[(size_t)r.pos * r.half + threadIdx.x];
    }
    return v;
}

__device__ __forceinline__ void rope_row_store(const Dsv4Rope &r, const RopeRow &v, float *rc,
                                               float *rs)
{
    if (r.rd && (int)threadIdx.x < r.rd / 2) {
        rc[threadIdx.x] = v.c;
        rs[threadIdx.x] = v.s;
    }
}

template <int KF, int VEC, int HIST, int MW>
__global__ void __launch_bounds__(MW * 64)
k_iscore(float *__restrict__ out, uint32_t *__restrict__ hist,
         uint32_t *__restrict__ meta, const float *__restrict__ q, const float *__restrict__ w,
         int H, int HP, int D, const void *__restrict__ keys,
         const float *__restrict__ ks, int key_stride, int n, float scale, int ng,
         Dsv4Rope qr)
{
    extern __shared__ double dots[];            /* [kb * 64][HP + 1], w[HP], q[H][D], then
                                                 * (HIST) the workgroup's histogram [TK_BINS] */
    constexpr int ES = KF == DSV4_GPU_KV_F32 ? 4 : KF == DSV4_GPU_KV_BF16 ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kb = (blockDim.x >> 6) / ng;      /* key blocks of 64 rows */
    const int b = wv / ng, hw = wv - b * ng;    /* this wave's block, head wave */
    const int t = (blockIdx.x * kb + b) * 64 + lane;
    const int tr = t < n ? t : n - 1;           /* rows past n compute row n-1 */
    const int pitch = HP + 1;
    double *wd = dots + (size_t)kb * 64 * pitch;
    float *qs = (float *)(wd + HP);
    uint32_t *lh = (uint32_t *)(qs + H * D);
    __shared__ float rcs[RP_MAX], rsn[RP_MAX];
    const RopeRow rrow = rope_row_load(qr);
    for (int i = threadIdx.x; i < H; i += blockDim.x) wd[i] = (double)w[i];
    if (HIST)
        for (int i = threadIdx.x; i < TK_BINS; i += blockDim.x) lh[i] = 0u;
    /* q into LDS (the launcher checks that it fits): batches of loads in
     * flight before any store, one memory latency per batch of 8 per thread */
    for (int i0 = 0; i0 < H * D; i0 += 8 * (int)blockDim.x) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = q[min(i0 + u * (int)blockDim.x + (int)threadIdx.x, H * D - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * (int)blockDim.x + (int)threadIdx.x;
            if (i < H * D) qs[i] = v[u];
        }
    }
    rope_row_store(qr, rrow, rcs, rsn);
    __syncthreads();
    if (qr.rd) {
        /* the indexer's q RoPE'd at pos, head by head (dsv4_layer.c:282-284) */
        const int hp = qr.rd / 2;
        for (int i = threadIdx.x; i < H * hp; i += blockDim.x) {
            const int hh = i / hp, p = i - hh * hp;
            float *t = qs + (size_t)hh * D + (D - qr.rd) + 2 * p;
            rope_pair_cs(t[0], t[1], rcs[p], rsn[p], qr.inverse);
        }
        __syncthreads();
    }
    const float rs = KF == DSV4_GPU_KV_FP8 ? ks[tr] : 1.0f;
    const unsigned char *row = (const unsigned char *)keys + (size_t)tr * key_stride * ES;
    double *drow = dots + (size_t)(b * 64 + lane) * pitch;

    for (int g = hw; g * IS_HB < HP; g += ng) {
        const int h0 = g * IS_HB;
        const int nh = min(IS_HB, H - h0);
        double acc[IS_HB];
#pragma unroll
        for (int j = 0; j < IS_HB; j++) acc[j] = 0.0;
        /* q for the next 16 columns is loaded while the current 16 compute */
        float qf[IS_HB], qn[IS_HB];
        q_cols(qf, qs, h0, H, D, 0, lane);
        if (VEC) {
            constexpr int CPP = 16 / ES;        /* columns per 16-byte piece */
            constexpr int BLK = 8 * CPP;        /* columns per batch of loads */
            constexpr int PPG = 16 / CPP;       /* pieces per 16 columns */
            for (int c0 = 0; c0 < D; c0 += BLK) {
                const int np = min(8, (D - c0) / CPP);
                u32x4 v[8];
#pragma unroll
                for (int u = 0; u < 8; u++)
                    v[u] = *(const DSV4_GLOBAL u32x4 *)(row + (size_t)(c0 + CPP * min(u, np - 1)) * ES);
                /* a rolled loop over the groups of 16 columns, the batch
                 * shifting down one group per trip: unrolled, the chains
                 * are tens of KB of straight-line code that every wave
                 * streams through the instruction cache once */
#pragma unroll 1
                for (int cc = c0; cc < min(c0 + BLK, D); cc += 16) {
                    float k[16];
#pragma unroll
                    for (int pc = 0; pc < PPG; pc++) key_piece<KF>(v[pc], rs, k + pc * CPP);
#pragma unroll
                    for (int u = 0; u + PPG < 8; u++) v[u] = v[u + PPG];
                    q_cols(qn, qs, h0, H, D, cc + 16, lane);
                    if (cc + 16 <= D) chain_16<true>(acc, qf, k, 16, nh);
                    else              chain_16<false>(acc, qf, k, D - cc, nh);
#pragma unroll
                    for (int j = 0; j < IS_HB; j++) qf[j] = qn[j];
                }
            }
        } else {
            for (int c0 = 0; c0 < D; c0 += 16) {
                float k[16];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int c = min(c0 + e, D - 1);
                    if (KF == DSV4_GPU_KV_FP8)
                        k[e] = dec_e4m3(row[c]) * rs;
                    else if (KF == DSV4_GPU_KV_BF16)
                        k[e] = bf16_to_f32(((const uint16_t *)row)[c]);
                    else
                        k[e] = ((const float *)row)[c];
                }
                q_cols(qn, qs, h0, H, D, c0 + 16, lane);
                if (c0 + 16 <= D) chain_16<true>(acc, qf, k, 16, nh);
                else              chain_16<false>(acc, qf, k, D - c0, nh);
#pragma unroll
                for (int j = 0; j < IS_HB; j++) qf[j] = qn[j];
            }
        }
#pragma unroll
        for (int j = 0; j < IS_HB; j++) drow[g * IS_HB + j] = acc[j];
    }
    __syncthreads();
    if (hw == 0) {
        /* the reference's `if (dot > 0) total += dot * w`, as a select */
        double total = 0.0;
        for (int hh = 0; hh < H; hh++) {
            const double d = drow[hh];
            const double prod = d * wd[hh];
            total = d > 0.0 ? total + prod : total;
        }
        const float tf = (float)total;
        const float sc = tf * scale;
        if (t < n) out[t] = sc;
        if (HIST && blockIdx.x == 0 && lane == 0) meta_restart(meta);
        if (HIST && t < n) atomicAdd(&lh[fkey(sc) >> 21], 1u);
    }
    if (HIST) {
        /* the workgroup's bins into the global histogram, one atomic per
         * bin it holds: scores crowd into few bins, and device-scope
         * atomics on one address serialise (per-wave merging left up to
         * ~32 per hot address and cost 4.7 us at C4, this 1.1) */
        __syncthreads();
        uint32_t *hs = hist + (blockIdx.x % TK_SLICES) * TK_BINS;
        for (int i = threadIdx.x; i < TK_BINS; i += blockDim.x) {
            const uint32_t c = lh[i];
            if (c) atomicAdd(&hs[i], c);
        }
    }
}

/* Matrix-core form of the score (D <= MF_DMAX, D % 4 == 0, H <= 64): the
 * fp64 chains on v_mfma_f64_16x16x4f64. That instruction computes each of
 * its outputs as a sequential fma chain over its four k in order (checked
 * bit for bit on the GPU against a CPU fma chain over 512000 outputs, f32
 * and full-precision operands; k in reverse or pairwise sums differ in
 * about 30% of them), so the instructions chained over columns 0, 4, 8, ...
 * are the reference's chain over c ascending. One instruction advances the
 * chains of 16 key rows x 16 heads by 4 columns. Operand layout: lane l
 * holds A[l % 16][l / 16] = key row l % 16 at column 4 m + l / 16,
 * B[l / 16][l % 16] = q of head l % 16 at that column, and D[l / 16 + 4 r]
 * [l % 16], r = 0 .. 3 (row, head). A key element is decoded once for 16
 * heads, and q comes from LDS (f32, RoPE'd, pitch D + 4: the 16 heads x 4
 * columns of a read hit distinct banks; heads padded to 16 HT with zeros).
 * A workgroup is MF_WAVES waves of MF_RT row tiles; each lane's key elements
 * are loaded before q is staged (PIECE: the 16-byte pieces of an FP8 row,
 * four needed bytes in each; else the elements one by one). The dots meet
 * in LDS and a thread per row folds the heads as the VALU form does. */
constexpr int MF_RT = 2;                         /* row tiles of 16 per wave */
constexpr int MF_WAVES = 4;
constexpr int MF_ROWS = 16 * MF_RT * MF_WAVES;   /* rows per workgroup */
constexpr int MF_DMAX = 128;
typedef double mf_v4d __attribute__((ext_vector_type(4)));

__host__ __device__ __forceinline__ size_t mf_lds_bytes(int H, int HT, int D, int hist)
{
    return sizeof(double) * ((size_t)MF_ROWS * (16 * HT + 1) + H) +
           sizeof(float) * (size_t)16 * HT * (D + 4) + (hist ? sizeof(uint32_t) * TK_BINS : 0);
}

template <int KF, int PIECE, int HIST, int HT>
__global__ void __launch_bounds__(MF_WAVES * 64)
k_iscore_mf(float *__restrict__ out, uint32_t *__restrict__ hist, uint32_t *__restrict__ meta,
            const float *__restrict__ q, const float *__restrict__ w, int H, int D,
            const void *__restrict__ keys, const float *__restrict__ ks, int key_stride, int n,
            float scale, Dsv4Rope qr)
{
    /* drow [MF_ROWS][16 HT + 1] f64, w [H] f64, q [16 HT][D + 4] f32, then
     * (HIST) the workgroup's histogram [TK_BINS] */
    extern __shared__ double mfl[];
    constexpr int ES = KF == DSV4_GPU_KV_F32 ? 4 : KF == DSV4_GPU_KV_BF16 ? 2 : 1;
    constexpr int NP = MF_DMAX / 16, NE = MF_DMAX / 4;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int HP = 16 * HT, pitch = HP + 1, QP = D + 4;
    double *drow = mfl;
    double *wd = drow + (size_t)MF_ROWS * pitch;
    float *qs = (float *)(wd + H);
    uint32_t *lh = (uint32_t *)(qs + (size_t)HP * QP);
    __shared__ float rcs[RP_MAX], rsn[RP_MAX];

    /* ---- q into LDS (rows of pitch QP, heads H .. HP-1 zero), w ---- */
    const RopeRow rrow = rope_row_load(qr);
    for (int i = H * QP + tid; i < HP * QP; i += MF_WAVES * 64) qs[i] = 0.0f;
    if (HIST)
        for (int i = tid; i < TK_BINS; i += MF_WAVES * 64) lh[i] = 0u;
    /* w's and q's first loads, then the keys', then their stores (the
     * memory counter returns in order: the stores wait for w and q only) */
    const float wf = w[min(tid, H - 1)];                 /* H <= 64 < MF_WAVES * 64 */
    float qv0[8];
#pragma unroll
    for (int u = 0; u < 8; u++) qv0[u] = q[min(u * MF_WAVES * 64 + tid, H * D - 1)];
    /* ---- this lane's key elements (row tile rt: row l % 16 of the tile,
     *      columns 4 m + g), in flight while q is staged ---- */
    const int r0 = blockIdx.x * MF_ROWS + wv * 16 * MF_RT;
    const int nm = D / 4;
    u32x4 kpc[MF_RT][PIECE ? NP : 1];
    uint32_t kel[MF_RT][PIECE ? 1 : NE];
    float rs[MF_RT];
#pragma unroll
    for (int rt = 0; rt < MF_RT; rt++) {
        const int row = min(r0 + 16 * rt + l16, n - 1);
        const unsigned char *rp = (const unsigned char *)keys + (size_t)row * key_stride * ES;
        rs[rt] = KF == DSV4_GPU_KV_FP8 ? ks[row] : 1.0f;
        if (PIECE) {
#pragma unroll
            for (int a = 0; a < NP; a++)
                kpc[rt][a] = *(const DSV4_GLOBAL u32x4 *)(rp + 16 * min(a, nm / 4 - 1));
        } else {
#pragma unroll
            for (int m = 0; m < NE; m++) {
                const int c = 4 * min(m, nm - 1) + g;
                kel[rt][m] = KF == DSV4_GPU_KV_F32 ? ((const uint32_t *)rp)[c]
                           : KF == DSV4_GPU_KV_BF16 ? (uint32_t)((const uint16_t *)rp)[c]
                           : (uint32_t)rp[c];
            }
        }
    }

    /* every load above is issued before any store below */
    __builtin_amdgcn_sched_barrier(0);
    /* unconditional (threads past H rewrite w[H-1]'s own value): a store
     * under `tid < H` let the compiler sink the load past the keys', and the
     * wait before it then covered them all */
    wd[min(tid, H - 1)] = (double)wf;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int i = min(u * MF_WAVES * 64 + tid, H * D - 1);     /* likewise */
        qs[(i / D) * QP + i % D] = qv0[u];
    }
    for (int i0 = 8 * MF_WAVES * 64; i0 < H * D; i0 += 8 * MF_WAVES * 64) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = q[min(i0 + u * MF_WAVES * 64 + tid, H * D - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = min(i0 + u * MF_WAVES * 64 + tid, H * D - 1);
            qs[(i / D) * QP + i % D] = v[u];
        }
    }
    rope_row_store(qr, rrow, rcs, rsn);
    __syncthreads();
    if (qr.rd) {
        /* the indexer's q RoPE'd at pos, head by head (dsv4_layer.c:282-284) */
        const int hp = qr.rd / 2;
        for (int i = tid; i < H * hp; i += MF_WAVES * 64) {
            const int hh = i / hp, p = i - hh * hp;
            float *t = qs + (size_t)hh * QP + (D - qr.rd) + 2 * p;
            rope_pair_cs(t[0], t[1], rcs[p], rsn[p], qr.inverse);
        }
        __syncthreads();
    }

    /* ---- the chains: step m takes columns 4 m .. 4 m + 3 ---- */
    mf_v4d acc[MF_RT][HT];
#pragma unroll
    for (int rt = 0; rt < MF_RT; rt++)
#pragma unroll
        for (int ht = 0; ht < HT; ht++) acc[rt][ht] = mf_v4d{0.0, 0.0, 0.0, 0.0};
    /* every step runs (no branch in the chain: the accumulators stay in
     * place); steps past D take zero operands, which leave a chain
     * unchanged bit for bit (it is never -0.0: it starts at +0.0 and an exact
     * cancellation rounds to +0.0) */
    const float *qcol = qs + (size_t)l16 * QP + g;
#pragma unroll
    for (int m = 0; m < NE; m++) {
        const bool live = m < nm;
        double qv[HT];
#pragma unroll
        for (int ht = 0; ht < HT; ht++) {
            const double x = (double)qcol[(size_t)ht * 16 * QP + 4 * min(m, nm - 1)];
            qv[ht] = live ? x : 0.0;
        }
#pragma unroll
        for (int rt = 0; rt < MF_RT; rt++) {
            float kf;
            if (PIECE) {
                const u32x4 pc = kpc[rt][m / 4];
                const uint32_t wd4 = (m & 3) == 0 ? pc.x : (m & 3) == 1 ? pc.y
                                   : (m & 3) == 2 ? pc.z : pc.w;
                kf = dec_e4m3((uint8_t)(wd4 >> (8 * g))) * rs[rt];
            } else if (KF == DSV4_GPU_KV_FP8) {
                kf = dec_e4m3((uint8_t)kel[rt][m]) * rs[rt];
            } else if (KF == DSV4_GPU_KV_BF16) {
                kf = __uint_as_float(kel[rt][m] << 16);
            } else {
                kf = __uint_as_float(kel[rt][m]);
            }
            const double kd = live ? (double)kf : 0.0;
#pragma unroll
            for (int ht = 0; ht < HT; ht++)
                acc[rt][ht] = __builtin_amdgcn_mfma_f64_16x16x4f64(kd, qv[ht], acc[rt][ht],
                                                                  0, 0, 0);
        }
    }
#pragma unroll
    for (int rt = 0; rt < MF_RT; rt++)
#pragma unroll
        for (int ht = 0; ht < HT; ht++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                drow[(size_t)(wv * 16 * MF_RT + 16 * rt + g + 4 * r) * pitch + 16 * ht + l16] =
                    acc[rt][ht][r];
    __syncthreads();

    /* ---- a thread per row: the reference's `if (dot > 0) total += dot * w`,
     *      as a select, in head order ---- */
    if (tid < MF_ROWS) {
        const int t = blockIdx.x * MF_ROWS + tid;
        double total = 0.0;
        for (int hh = 0; hh < H; hh++) {
            const double d = drow[(size_t)tid * pitch + hh];
            const double prod = d * wd[hh];
            total = d > 0.0 ? total + prod : total;
        }
        const float sc = (float)total * scale;
        if (t < n) out[t] = sc;
        if (HIST && t == 0) meta_restart(meta);
        if (HIST && t < n) atomicAdd(&lh[fkey(sc) >> 21], 1u);
    }
    if (HIST) {
        __syncthreads();
        uint32_t *hs = hist + (blockIdx.x % TK_SLICES) * TK_BINS;
        for (int i = tid; i < TK_BINS; i += MF_WAVES * 64) {
            const uint32_t c = lh[i];
            if (c) atomicAdd(&hs[i], c);
        }
    }
}

/* Few f32 keys (the attention block's compressed rows, n <= SK_NMAX): one
 * thread per (key, head) runs that pair's fp64 fma chain over c ascending,
 * with q (RoPE'd when asked) and the workgroup's key rows staged in LDS; a
 * thread per key then folds the heads in order from LDS. The same
 * arithmetic, step for step, as the reference and as k_iscore, with a
 * workgroup of SK_THREADS / HP keys. Written for every key format, but
 * launched for short f32 score vectors with no top-k histogram to build,
 * where it is the faster form. */
constexpr int SK_NMAX = 4096;
constexpr int SK_THREADS = 256;

template <int KF>
__global__ void __launch_bounds__(SK_THREADS)
k_iscore_kh(float *__restrict__ out, const float *__restrict__ q, const float *__restrict__ w, int H, int HP, int D,
            const void *__restrict__ keys, const float *__restrict__ ks, int key_stride, int n,
            float scale, Dsv4Rope qr)
{
    extern __shared__ double skl[];   /* dots[kpw][HP], w[H], q[H][D + 1], then keys[kpw][D] */
    const int kpw = SK_THREADS / HP;
    const int qp = D + 1;                       /* odd pitch: the heads of a wave hit distinct banks */
    double *dots = skl;
    double *wd = dots + (size_t)kpw * HP;
    float *qs = (float *)(wd + H);
    float *ksl = qs + (size_t)H * qp;
    __shared__ float rcs[RP_MAX], rsn[RP_MAX];
    const RopeRow rrow = rope_row_load(qr);
    /* Staging: w, the workgroup's key rows and q. When each fits one batch
     * (as at the attention block's shapes), every load is issued before any
     * store: one memory latency instead of three. */
    const int t0k = blockIdx.x * kpw;
    const int nq4 = (H * D) >> 2;
    if (kpw * D <= 8 * SK_THREADS && nq4 <= 8 * SK_THREADS) {
        const double wv = (int)threadIdx.x < H ? (double)w[threadIdx.x] : 0.0;
        float kv8[8];
        f32x4 qv8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = min(u * SK_THREADS + (int)threadIdx.x, kpw * D - 1);
            const int kk = i / D, c = i - kk * D;
            kv8[u] = key_at<KF>(keys, ks, (size_t)min(t0k + kk, n - 1), key_stride, c);
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            qv8[u] = ldf4(q + 4 * min(u * SK_THREADS + (int)threadIdx.x, nq4 - 1));
        if ((int)threadIdx.x < H) wd[threadIdx.x] = wv;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = u * SK_THREADS + (int)threadIdx.x;
            if (i < kpw * D) ksl[i] = kv8[u];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = u * SK_THREADS + (int)threadIdx.x;
            if (i < nq4) {
                const int e = 4 * i, hh = e / D, c = e - hh * D;   /* D % 4 == 0 */
                float *d = qs + (size_t)hh * qp + c;
                d[0] = qv8[u].x; d[1] = qv8[u].y; d[2] = qv8[u].z; d[3] = qv8[u].w;
            }
        }
    } else {
        for (int i = threadIdx.x; i < H; i += SK_THREADS) wd[i] = (double)w[i];
        constexpr int KB = 8;
        for (int i0 = 0; i0 < kpw * D; i0 += KB * SK_THREADS) {
            float v[KB];
#pragma unroll
            for (int u = 0; u < KB; u++) {
                const int i = min(i0 + u * SK_THREADS + (int)threadIdx.x, kpw * D - 1);
                const int kk = i / D, c = i - kk * D;
                v[u] = key_at<KF>(keys, ks, (size_t)min(t0k + kk, n - 1), key_stride, c);
            }
#pragma unroll
            for (int u = 0; u < KB; u++) {
                const int i = i0 + u * SK_THREADS + (int)threadIdx.x;
                if (i < kpw * D) ksl[i] = v[u];
            }
        }
        for (int i0 = 0; i0 < nq4; i0 += 8 * SK_THREADS) {
            f32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                v[u] = ldf4(q + 4 * min(i0 + u * SK_THREADS + (int)threadIdx.x, nq4 - 1));
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * SK_THREADS + (int)threadIdx.x;
                if (i < nq4) {
                    const int e = 4 * i, hh = e / D, c = e - hh * D;
                    float *d = qs + (size_t)hh * qp + c;
                    d[0] = v[u].x; d[1] = v[u].y; d[2] = v[u].z; d[3] = v[u].w;
                }
            }
        }
    }
    rope_row_store(qr, rrow, rcs, rsn);
    __syncthreads();
    if (qr.rd) {
        const int hp = qr.rd / 2;
        for (int i = threadIdx.x; i < H * hp; i += SK_THREADS) {
            const int hh = i / hp, p = i - hh * hp;
            float *t = qs + (size_t)hh * qp + (D - qr.rd) + 2 * p;
            rope_pair_cs(t[0], t[1], rcs[p], rsn[p], qr.inverse);
        }
        __syncthreads();
    }
    const int kl = threadIdx.x / HP, h = threadIdx.x - kl * HP;
    const int t = blockIdx.x * kpw + kl;
    if (h < H && t < n) {
        const float *kr = ksl + (size_t)kl * D;
        const float *qh = qs + (size_t)h * qp;
        double dot = 0.0;
#pragma unroll 16
        for (int c = 0; c < D; c++) dot = fma((double)qh[c], (double)kr[c], dot);
        dots[kl * HP + h] = dot;
    }
    __syncthreads();
    const int tt = blockIdx.x * kpw + (int)threadIdx.x;
    if ((int)threadIdx.x < kpw && tt < n) {
        double total = 0.0;
        for (int hh = 0; hh < H; hh++) {
            const double d = dots[threadIdx.x * HP + hh];
            const double prod = d * wd[hh];
            total = d > 0.0 ? total + prod : total;
        }
        out[tt] = (float)total * scale;
    }
}

template <int KF, int HIST, int MW>
void launch_iscore(bool vec, int grid, int thr, size_t lds, hipStream_t st,
                   float *d_out, uint32_t *hist, uint32_t *meta, const float *d_q,
                   const float *d_w,
                   int H, int HP, int D, const void *d_keys, const float *d_ks,
                   int key_stride, int n, float scale, int ng, const Dsv4Rope &qr)
{
    if (vec)
        hipLaunchKernelGGL((k_iscore<KF, 1, HIST, MW>), dim3(grid), dim3(thr), lds, st, d_out,
                           hist, meta, d_q, d_w, H, HP, D, d_keys, d_ks, key_stride, n, scale,
                           ng, qr);
    else
        hipLaunchKernelGGL((k_iscore<KF, 0, HIST, MW>), dim3(grid), dim3(thr), lds, st, d_out,
                           hist, meta, d_q, d_w, H, HP, D, d_keys, d_ks, key_stride, n, scale,
                           ng, qr);
}

/* --------------------------------------------------------------- top-k */

/* Top-k in two passes after the level-1 histogram (built by the score
 * kernel, or by k_tk_hist for stand-alone scores):
 *   k_tk_part   many workgroups: the bin B of the k-th largest from the
 *               histogram; elements of higher bins go to cand[], those of B
 *               to bsel[] (any order, as composites), and also to a
 *               per-workgroup list in index order;
 *   k_tk_final  many workgroups, each placing a share of the elements: from
 *               cand[] and bsel[] directly when B holds at most RF_LIST
 *               elements, else after a refinement of B's list (levels 2 and
 *               3 give T, the exact key of the k-th largest) that every
 *               workgroup repeats; the first need_eq elements == T then
 *               follow the candidates > T in index order. */

constexpr int PT_THREADS = 256;                 /* partition workgroup */
constexpr int PT_EPT = 4;                       /* elements per thread */
constexpr int PT_ELEMS = PT_THREADS * PT_EPT;   /* elements per workgroup */
constexpr int RF_LIST = 4096;                   /* B's list kept in LDS */
constexpr int RF_GMAX = 4096;                   /* partition workgroups */
constexpr int TK_NMAX = RF_GMAX * PT_ELEMS;     /* scores per top-k */

__device__ __forceinline__ unsigned long long lanemask_lt(int lane)
{
    return lane ? (~0ull >> (64 - lane)) : 0ull;
}

/* Level-1 histogram for a stand-alone top-k (the fused path gets it from the
 * score kernel): top 11 key bits of every score, TH_EPT per thread merged in
 * the workgroup's LDS histogram first, then one atomic per bin it holds.
 * Also restarts the append counter. */
constexpr int TH_EPT = 4;

__global__ void __launch_bounds__(256)
k_tk_hist(uint32_t *__restrict__ hist, uint32_t *__restrict__ meta,
          const float *__restrict__ scores, int n)
{
    __shared__ uint32_t lh[TK_BINS];
    const int tid = threadIdx.x, e0 = blockIdx.x * 256 * TH_EPT + tid;
    float v[TH_EPT];
#pragma unroll
    for (int m = 0; m < TH_EPT; m++) v[m] = scores[min(e0 + 256 * m, n - 1)];
    for (int i = tid; i < TK_BINS; i += 256) lh[i] = 0u;
    if (blockIdx.x == 0 && tid == 0) meta_restart(meta);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < TH_EPT; m++)
        if (e0 + 256 * m < n) atomicAdd(&lh[fkey(v[m]) >> 21], 1u);
    __syncthreads();
    uint32_t *hs = hist + (blockIdx.x % TK_SLICES) * TK_BINS;
    for (int i = tid; i < TK_BINS; i += 256) {
        const uint32_t c = lh[i];
        if (c) atomicAdd(&hs[i], c);
    }
}

/* Descending search over TK_BINS bins, BPT per thread of NT: thread t holds
 * c[j] = count of bin TK_BINS - 1 - BPT t - j. Finds the bin holding the
 * krem-th largest element (krem >= 1, at most the total count) and the rank
 * it has among that bin's elements: res[0] = bin, res[1] = rank (a safe
 * bin 0 / rank 1 when none fits). Ends on a barrier; callers read res and
 * pass a barrier before the next call. */
template <int NT, int BPT>
__device__ __forceinline__ void tk_find(const uint32_t *c, uint32_t krem,
                                        uint32_t *wsum, uint32_t *res)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    if (tid == 0) { res[0] = 0u; res[1] = 1u; }
    uint32_t s = 0u;
#pragma unroll
    for (int j = 0; j < BPT; j++) s += c[j];
    uint32_t inc = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
    }
    if (lane == 63) wsum[wid] = inc;
    __syncthreads();
    uint32_t base = 0u;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) base += w < wid ? wsum[w] : 0u;
    inc += base;
    const uint32_t exc = inc - s;
    if (exc < krem && inc >= krem) {
        uint32_t run = exc;
#pragma unroll
        for (int j = 0; j < BPT; j++) {
            if (run + c[j] >= krem) {
                res[0] = (uint32_t)(TK_BINS - 1 - BPT * tid - j);
                res[1] = krem - run;
                break;
            }
            run += c[j];
        }
    }
    __syncthreads();
}

/* Exclusive prefix over the threads of an NT-thread workgroup (thread
 * order); *total gets the sum. Ends on a barrier. */
template <int NT>
__device__ __forceinline__ uint32_t tk_scan(uint32_t v, uint32_t *wsum, uint32_t *total)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) wsum[wid] = inc;
    __syncthreads();
    uint32_t before = 0u, all = 0u;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) {
        const uint32_t x = wsum[w];
        before += w < wid ? x : 0u;
        all += x;
    }
    *total = all;
    __syncthreads();
    return before + inc - v;
}

/* Exclusive prefix maximum over the threads of an NT-thread workgroup
 * (thread order; 0 for thread 0). Ends on a barrier. */
template <int NT>
__device__ __forceinline__ uint32_t tk_scan_max(uint32_t v, uint32_t *wsum)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (lane >= o) inc = max(inc, t);
    }
    uint32_t exc = __shfl_up(inc, 1, 64);
    if (lane == 0) exc = 0u;
    if (lane == 63) wsum[wid] = inc;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NT / 64; w++) exc = w < wid ? max(exc, wsum[w]) : exc;
    __syncthreads();
    return exc;
}

/* Bitonic sort of a[0 .. np), np a power of two, into descending order by
 * the NT threads of the workgroup. Starts and ends on a barrier. */
template <int NT>
__device__ __forceinline__ void lds_sort_desc(unsigned long long *a, uint32_t np)
{
    __syncthreads();
    for (uint32_t size = 2; size <= np; size <<= 1)
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = threadIdx.x; t < np / 2; t += NT) {
                const uint32_t i = 2 * t - (t & (stride - 1)), j = i + stride;
                const unsigned long long x = a[i], y = a[j];
                /* blocks with (i & size) == 0 run descending, the others
                 * ascending; the last merge (size == np) is all descending */
                if ((x < y) == ((i & size) == 0u)) { a[i] = y; a[j] = x; }
            }
            __syncthreads();
        }
}

__device__ __forceinline__ uint32_t pow2_at_least(uint32_t x)
{
    uint32_t p = 1u;
    while (p < x) p <<= 1;
    return p;
}

/* The reference's selection when scores hold NaNs (dsv4_indexer.c:92-106).
 * Each pick of its scan starts at the lowest index not yet taken and moves
 * only on `scores[c] > scores[best]`, so a NaN is taken exactly when it is
 * that lowest index; otherwise the pick is the first maximum of the untaken
 * finite scores. Its output is therefore the finite scores in (score desc,
 * index asc) order with each NaN i inserted after P(i) of them, where P(i)
 * is the largest 1-based place in that order of a finite index below i
 * (0 when there is none): NaN i lands at (NaNs below i) + P(i). Since
 * P(i) >= (finite indices below i), that position is at least i, so only
 * NaNs below k can be taken, and only scores[0 .. k) are read.
 *
 * srt[0 .. k): the k largest composites in descending order with NaNs
 * keyed 0 (so any NaN among them comes after every finite score, and a
 * finite index missing from srt has a place >= k, which keeps every NaN
 * above it out). aux: k words of LDS apart from srt's first k words. The
 * NaNs' places are marked in aux; the other places take the finite
 * entries in order. Called by every thread of the workgroup; writes
 * idxs[0 .. k). */
template <int NT>
__device__ __forceinline__ void nan_finish(int *__restrict__ idxs, unsigned long long *srt, uint32_t *aux,
                           const float *__restrict__ scores, int k, uint32_t *wsum)
{
    constexpr int CM = TK_KMAX / NT;                 /* entries per thread, at most */
    constexpr uint32_t FAR = 0x3FFFFFFFu;            /* a place past any k */
    const int tid = threadIdx.x;
    const int C = (k + NT - 1) / NT, c0 = tid * C;
    uint32_t *L = reinterpret_cast<uint32_t *>(srt);

    float sv[CM];
    uint32_t lw[CM];
#pragma unroll
    for (int c = 0; c < CM; c++) {
        const int r = c0 + c;
        const bool live = c < C && r < k;
        sv[c] = scores[live ? r : 0];
        const unsigned long long e = srt[live ? r : 0];
        /* the index, bit 31 set for a NaN */
        lw[c] = (0xFFFFFFFFu - (uint32_t)e) | ((e >> 32) == 0ull ? 0x80000000u : 0u);
    }
    __syncthreads();                                  /* srt read: reuse as L */
#pragma unroll
    for (int c = 0; c < CM; c++)
        if (c < C && c0 + c < k) L[c0 + c] = lw[c];
    for (int i = tid; i < k; i += NT) aux[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CM; c++)                      /* place in L of finite indices < k */
        if (c < C && c0 + c < k && lw[c] < (uint32_t)k) aux[lw[c]] = (uint32_t)(c0 + c) + 1u;
    __syncthreads();

    /* thread t: indices [c0, c0 + C). pe = 0 for a NaN, the place in L of a
     * finite index, FAR for a finite index missing from L */
    bool isn[CM];
    uint32_t pe[CM], cnt = 0u, mx = 0u;
#pragma unroll
    for (int c = 0; c < CM; c++) {
        const int i = c0 + c;
        const bool live = c < C && i < k;
        isn[c] = live && __builtin_isnan(sv[c]);
        const uint32_t a = live ? aux[i] : 0u;
        pe[c] = isn[c] ? 0u : (a ? a : FAR);
        cnt += isn[c] ? 1u : 0u;
        mx = live ? max(mx, pe[c]) : mx;
    }
    uint32_t tot;
    const uint32_t j0 = tk_scan<NT>(cnt, wsum, &tot);
    const uint32_t p0 = tk_scan_max<NT>(mx, wsum);
    for (int i = tid; i < k; i += NT) aux[i] = 0xFFFFFFFFu;
    __syncthreads();
    {
        uint32_t j = j0, P = p0;
#pragma unroll
        for (int c = 0; c < CM; c++) {
            const int i = c0 + c;
            if (!(c < C && i < k)) continue;
            if (isn[c]) {
                const uint32_t pos = j + P;
                if (pos < (uint32_t)k) aux[pos] = (uint32_t)i;
                j++;
            } else {
                P = max(P, pe[c]);
            }
        }
    }
    __syncthreads();

    /* places [c0, c0 + C): a NaN's, or the next finite entry of L */
    uint32_t o[CM], nf = 0u;
#pragma unroll
    for (int c = 0; c < CM; c++) {
        const int p = c0 + c;
        const bool live = c < C && p < k;
        o[c] = live ? aux[p] : 0u;
        nf += live && o[c] == 0xFFFFFFFFu ? 1u : 0u;
    }
    uint32_t f = tk_scan<NT>(nf, wsum, &tot);
#pragma unroll
    for (int c = 0; c < CM; c++) {
        const int p = c0 + c;
        if (!(c < C && p < k)) continue;
        if (o[c] != 0xFFFFFFFFu) {
            idxs[p] = (int)o[c];
        } else {
            idxs[p] = (int)(L[min(f, (uint32_t)k - 1u)] & 0x7FFFFFFFu);
            f++;
        }
    }
}

/* Partition: workgroup g owns elements [g PT_ELEMS, (g + 1) PT_ELEMS); slot
 * m of thread t is element g PT_ELEMS + m PT_THREADS + t (coalesced loads,
 * index order = (slot, wave, lane)). Every workgroup reads the whole sliced
 * histogram and finds the same B. */
__global__ void __launch_bounds__(PT_THREADS)
k_tk_part(unsigned long long *__restrict__ cand, unsigned long long *__restrict__ bsel,
          uint32_t *__restrict__ meta, uint32_t *__restrict__ bcnt,
          unsigned long long *__restrict__ blist,
          const uint32_t *__restrict__ hist_g, const float *__restrict__ scores,
          int n, int k)
{
    constexpr int NW = PT_THREADS / 64;
    constexpr int BPT = TK_BINS / PT_THREADS;      /* 8 bins per thread */
    __shared__ uint32_t wsum[NW], res[2];
    __shared__ uint32_t scnt[PT_EPT][NW];
    __shared__ unsigned long long wcnt[NW], wbase;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int e0 = blockIdx.x * PT_ELEMS + tid;     /* slot m: e0 + m PT_THREADS */
    const unsigned long long lt = lanemask_lt(lane);

    uint32_t key[PT_EPT];
#pragma unroll
    for (int m = 0; m < PT_EPT; m++)
        key[m] = __float_as_uint(scores[min(e0 + m * PT_THREADS, n - 1)]);
    const int blo = TK_BINS - BPT * (tid + 1);      /* bins [blo, blo + BPT) */
    u32x4 hv[TK_SLICES][BPT / 4];
#pragma unroll
    for (int s = 0; s < TK_SLICES; s++)
#pragma unroll
        for (int q = 0; q < BPT / 4; q++)
            hv[s][q] = *reinterpret_cast<const u32x4 *>(hist_g + s * TK_BINS + blo + 4 * q);
    bool nan = false;
#pragma unroll
    for (int m = 0; m < PT_EPT; m++) {
        const bool in = e0 + m * PT_THREADS < n;
        nan = nan || (in && __builtin_isnan(__uint_as_float(key[m])));
        key[m] = in ? fkey(__uint_as_float(key[m])) : 0u;
    }
    /* a NaN anywhere: the final pass applies the reference's NaN rule
     * (its order then depends on positions, not only on the keys) */
    if (__ballot(nan) != 0ull && lane == 0) atomicOr(&meta[MT_NAN], 1u);

    uint32_t c[BPT];                                /* c[j]: bin blo + BPT-1-j */
#pragma unroll
    for (int j = 0; j < BPT; j++) c[j] = 0u;
#pragma unroll
    for (int s = 0; s < TK_SLICES; s++)
#pragma unroll
        for (int q = 0; q < BPT / 4; q++) {
            c[BPT - 1 - 4 * q] += hv[s][q].x;
            c[BPT - 2 - 4 * q] += hv[s][q].y;
            c[BPT - 3 - 4 * q] += hv[s][q].z;
            c[BPT - 4 - 4 * q] += hv[s][q].w;
        }
    tk_find<PT_THREADS, BPT>(c, (uint32_t)k, wsum, res);
    const uint32_t B = res[0];
    if (blockIdx.x == 0 && tid == 0) { meta[MT_BIN] = B; meta[MT_KREM] = res[1]; }

    /* elements of higher bins and of B, as composites (key << 32 | ~index),
     * appended in any order to cand[] and bsel[]: one 64-bit atomic per
     * workgroup takes both places (cand[] count in the low word, bsel[]
     * high; one per wave had 128 returning atomics queue on one address, 2 us
     * at C4). B's elements also go to this workgroup's list in index order
     * (read by the final pass only when B holds more than RF_LIST elements),
     * written while the atomic is in flight. */
    unsigned long long ma[PT_EPT], mb[PT_EPT];
    uint32_t na = 0u, nbw = 0u;
#pragma unroll
    for (int m = 0; m < PT_EPT; m++) {
        const bool in = e0 + m * PT_THREADS < n;
        ma[m] = __ballot(in && (key[m] >> 21) > B);
        mb[m] = __ballot(in && (key[m] >> 21) == B);
        na += (uint32_t)__popcll(ma[m]);
        nbw += (uint32_t)__popcll(mb[m]);
        if (lane == 0) scnt[m][wid] = (uint32_t)__popcll(mb[m]);
    }
    if (lane == 0) wcnt[wid] = (unsigned long long)na | ((unsigned long long)nbw << 32);
    __syncthreads();
    if (tid == 0) {
        unsigned long long all = 0ull;
#pragma unroll
        for (int w = 0; w < NW; w++) all += wcnt[w];
        wbase = all ? atomicAdd(reinterpret_cast<unsigned long long *>(meta + MT_CNT), all) : 0ull;
    }
    uint32_t off[PT_EPT], tot = 0u;
#pragma unroll
    for (int m = 0; m < PT_EPT; m++)
#pragma unroll
        for (int w = 0; w < NW; w++) {
            if (w == wid) off[m] = tot;
            tot += scnt[m][w];
        }
    unsigned long long *mine = blist + (size_t)blockIdx.x * PT_ELEMS;
#pragma unroll
    for (int m = 0; m < PT_EPT; m++)
        if ((mb[m] >> lane) & 1ull)
            mine[off[m] + (uint32_t)__popcll(mb[m] & lt)] =
                ((unsigned long long)key[m] << 32) | (uint32_t)(e0 + m * PT_THREADS);
    if (tid == 0) bcnt[blockIdx.x] = tot;
    __syncthreads();
    unsigned long long at = wbase;
#pragma unroll
    for (int w = 0; w < NW; w++) at += w < wid ? wcnt[w] : 0ull;
    uint32_t pa = (uint32_t)at, pb = (uint32_t)(at >> 32);
#pragma unroll
    for (int m = 0; m < PT_EPT; m++) {
        const uint32_t i = (uint32_t)(e0 + m * PT_THREADS);
        const unsigned long long comp = ((unsigned long long)key[m] << 32) | (0xFFFFFFFFull - i);
        if ((ma[m] >> lane) & 1ull) {
            const uint32_t pos = pa + (uint32_t)__popcll(ma[m] & lt);
            if (pos < (uint32_t)TK_KMAX) cand[pos] = comp;
        } else if ((mb[m] >> lane) & 1ull) {
            const uint32_t pos = pb + (uint32_t)__popcll(mb[m] & lt);
            if (pos < (uint32_t)RF_LIST) bsel[pos] = comp;
        }
        pa += (uint32_t)__popcll(ma[m]);
        pb += (uint32_t)__popcll(mb[m]);
    }
}

/* Final pass. The composites (key << 32 | ~index) order the scores as the
 * output does, score descending with ties to the lower index, and they are
 * distinct: an element's place is the number of composites ahead of it.
 *
 * Direct form (B holds at most RF_LIST elements, the usual case): the
 * elements above B (cand[], all selected) and those of B (bsel[]) make one
 * array u of c_above + nb composites, cand[] first, and workgroup b places
 * the elements [RK_EPW b, RK_EPW (b + 1)) of u. An element above B is ahead
 * of every element of B, so it counts only the cand[] composites ahead of it
 * and lands there; an element of B counts only B's, r of them, and is
 * selected when r < krem (the k-th largest is the krem-th of B), landing at
 * c_above + r. A workgroup stages only the part(s) of u its elements are in,
 * in one batch of loads issued right after the meta words.
 *
 * Refinement form (B larger than RF_LIST): B's elements, in index order,
 * are the lists of the G partition workgroups one after another (entry j of
 * the whole list lies in the list of the workgroup w with pfx[w] <= j <
 * pfx[w + 1]), read from global memory. Levels 2 and 3 of the radix select
 * over that list give T, the exact key of the k-th largest, and need_eq;
 * the candidates -- cand[] plus the list's elements > T, in list order --
 * are the same array in every workgroup, each workgroup places RK_EPW of
 * them by counting, and workgroup 0 writes the first need_eq elements == T
 * after them, in index order.
 *
 * Every workgroup clears its share of the level-1 histogram. */
constexpr int FN_THREADS = 512;
constexpr int FN_WAVES = FN_THREADS / 64;
constexpr int RK_TPE = 32;                              /* threads per element */
constexpr int RK_EPW = FN_THREADS / RK_TPE;             /* elements per workgroup */

/* Number of composites list[f] > mine over f = f0, f0 + TPE, ... < f1,
 * summed over the TPE lanes of an element (called by every lane): the
 * lanes of an element read consecutive words, the elements of a wave the
 * same ones, and sixteen reads are in flight per trip (the loop is
 * LDS-latency bound). */
template <int TPE = RK_TPE>
__device__ __forceinline__ uint32_t rank_count(const unsigned long long *list, uint32_t f0,
                                               uint32_t f1, unsigned long long mine)
{
    constexpr int RU = 16;
    uint32_t r = 0u, f = f0;
    for (; f + (RU - 1) * TPE < f1; f += RU * TPE) {
        unsigned long long x[RU];
#pragma unroll
        for (int u = 0; u < RU; u++) x[u] = list[f + u * TPE];
#pragma unroll
        for (int u = 0; u < RU; u++) r += x[u] > mine ? 1u : 0u;
    }
    for (; f < f1; f += TPE) r += list[f] > mine ? 1u : 0u;
#pragma unroll
    for (int o = 1; o < TPE; o <<= 1) r += __shfl_xor(r, o, 64);
    return r;
}

__global__ void __launch_bounds__(FN_THREADS)
k_tk_final(int *__restrict__ idxs, const unsigned long long *__restrict__ cand,
           const unsigned long long *__restrict__ bsel, const uint32_t *__restrict__ meta,
           const uint32_t *__restrict__ bcnt, const unsigned long long *__restrict__ blist,
           uint32_t *__restrict__ hist_g, const float *__restrict__ scores, int G, int k)
{
    constexpr int BPT = TK_BINS / FN_THREADS;           /* bins per thread */
    constexpr int GPT = RF_GMAX / FN_THREADS;           /* list lengths per thread */
    /* direct form: u; refinement form: the candidates in the first TK_KMAX
     * words, the level-2/3 histogram and the list prefix after them */
    __shared__ unsigned long long sh[TK_KMAX + RF_LIST];
    __shared__ uint32_t wsum[FN_WAVES], res[2];
    static_assert(sizeof(uint32_t) * (TK_BINS + RF_GMAX + 1) <=
                  sizeof(unsigned long long) * RF_LIST, "refinement LDS");

    const int tid = threadIdx.x;

    for (int i = blockIdx.x * FN_THREADS + tid; i < TK_SLICES * TK_BINS / 4;
         i += gridDim.x * FN_THREADS)
        reinterpret_cast<u32x4 *>(hist_g)[i] = u32x4{0u, 0u, 0u, 0u};
    /* NaN scores (uniform per launch): workgroup 0 alone sorts the
     * selection and applies the reference's NaN rule (nan_finish) */
    const bool nanm = meta[MT_NAN] != 0u;
    if (nanm && blockIdx.x != 0) return;
    const uint32_t B = meta[MT_BIN], krem1 = meta[MT_KREM];
    const unsigned long long cnt = *reinterpret_cast<const unsigned long long *>(meta + MT_CNT);
    const uint32_t c_above = min((uint32_t)cnt, (uint32_t)TK_KMAX);
    const uint32_t nbs = (uint32_t)(cnt >> 32);

    if (nbs <= (uint32_t)RF_LIST) {
        /* ---- direct form ---- */
        const uint32_t u = c_above + nbs, e0 = blockIdx.x * RK_EPW;
        if (nanm) {
            /* all of u (at most TK_KMAX + RF_LIST composites), padded with
             * zeros to a power of two, sorted; its first k are the k largest */
            const uint32_t np = pow2_at_least(max(u, (uint32_t)k));
            for (uint32_t j = tid; j < np; j += FN_THREADS)
                sh[j] = j < c_above ? cand[j] : j < u ? bsel[j - c_above] : 0ull;
            lds_sort_desc<FN_THREADS>(sh, np);
            nan_finish<FN_THREADS>(idxs, sh, reinterpret_cast<uint32_t *>(sh + TK_KMAX),
                                   scores, k, wsum);
            return;
        }
        if (e0 >= u) return;                                /* the whole workgroup */
        const uint32_t ja = e0 < c_above ? 0u : c_above;
        const uint32_t jb = e0 + RK_EPW > c_above ? u : c_above;
        constexpr int SB = 16;
        for (uint32_t j0 = ja; j0 < jb; j0 += SB * FN_THREADS) {
            unsigned long long v[SB];
#pragma unroll
            for (int q = 0; q < SB; q++) {
                const uint32_t j = min(j0 + q * FN_THREADS + tid, jb - 1);
                const unsigned long long *src = j < c_above ? cand + j : bsel + (j - c_above);
                v[q] = *src;
            }
#pragma unroll
            for (int q = 0; q < SB; q++) {
                const uint32_t j = j0 + q * FN_THREADS + tid;
                if (j < jb) sh[j] = v[q];
            }
        }
        __syncthreads();
        const uint32_t e = e0 + tid / RK_TPE, sub = tid % RK_TPE;
        const bool live = e < u, inb = e >= c_above;
        const unsigned long long mine = live ? sh[e] : ~0ull;
        const uint32_t f0 = live ? (inb ? c_above : 0u) : 0u;
        const uint32_t f1 = live ? (inb ? u : c_above) : 0u;
        const uint32_t r = rank_count(sh, f0 + sub, f1, mine);
        if (sub == 0 && live) {
            const uint32_t pos = inb ? c_above + r : r;
            if ((!inb || r < krem1) && pos < (uint32_t)k)
                idxs[pos] = (int)(0xFFFFFFFFu - (uint32_t)mine);
        }
        return;
    }

    /* ---- refinement form ---- */
    unsigned long long *cs = sh;
    uint32_t *hist = reinterpret_cast<uint32_t *>(sh + TK_KMAX);
    uint32_t *pfx = hist + TK_BINS;

    /* list lengths (prefix below): thread t takes entries GPT t .. GPT t + GPT-1;
     * their loads are issued before the candidates' */
    uint32_t v[GPT];
#pragma unroll
    for (int q = 0; q < GPT; q++) v[q] = bcnt[min(GPT * tid + q, G - 1)];
    /* candidates above B: into LDS */
    for (uint32_t i0 = 0; i0 < c_above; i0 += 8 * FN_THREADS) {
        unsigned long long cv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) cv[u] = cand[min(i0 + u * FN_THREADS + tid, c_above - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + u * FN_THREADS + tid < c_above) cs[i0 + u * FN_THREADS + tid] = cv[u];
    }

    uint32_t sg = 0u;
#pragma unroll
    for (int q = 0; q < GPT; q++) {
        v[q] = GPT * tid + q < G ? v[q] : 0u;
        sg += v[q];
    }
    uint32_t nb;
    uint32_t run = tk_scan<FN_THREADS>(sg, wsum, &nb);
#pragma unroll
    for (int q = 0; q < GPT; q++) {
        if (GPT * tid + q < G) pfx[GPT * tid + q] = run;
        run += v[q];
    }
    if (tid == 0) pfx[G] = nb;
#pragma unroll
    for (int q = 0; q < BPT; q++) hist[BPT * tid + q] = 0u;
    __syncthreads();

    auto ent = [&](uint32_t j) -> unsigned long long {   /* entry j of B's list */
        int lo = 0, hi = G - 1;                           /* last w with pfx[w] <= j */
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pfx[mid] <= j) lo = mid; else hi = mid - 1;
        }
        return blist[(uint32_t)lo * PT_ELEMS + (j - pfx[lo])];
    };

    /* ---- level 2: bits 20..10 ---- */
    for (uint32_t j = tid; j < nb; j += FN_THREADS)
        atomicAdd(&hist[(uint32_t)(ent(j) >> 42) & 2047u], 1u);
    __syncthreads();
    uint32_t c[BPT];
#pragma unroll
    for (int q = 0; q < BPT; q++) c[q] = hist[TK_BINS - 1 - BPT * tid - q];
    tk_find<FN_THREADS, BPT>(c, krem1, wsum, res);
    const uint32_t P22 = (B << 11) | res[0], krem2 = res[1];

    /* ---- level 3: bits 9..0 ---- */
#pragma unroll
    for (int q = 0; q < BPT; q++) hist[BPT * tid + q] = 0u;
    __syncthreads();
    for (uint32_t j = tid; j < nb; j += FN_THREADS) {
        const uint32_t key = (uint32_t)(ent(j) >> 32);
        if ((key >> 10) == P22) atomicAdd(&hist[key & 1023u], 1u);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < BPT; q++) c[q] = hist[TK_BINS - 1 - BPT * tid - q];
    tk_find<FN_THREADS, BPT>(c, krem2, wsum, res);
    const uint32_t T = (P22 << 10) | res[0];
    /* need_eq is in [1, k] for a histogram that matches the scores; the
     * clamp keeps every write below in bounds whatever the histogram held. */
    const uint32_t need_eq = min(max(res[1], 1u), (uint32_t)k);
    const uint32_t c_gt = (uint32_t)k - need_eq;

    /* ---- B's elements > T join the candidates (list order); the first
     *      need_eq == T, in index order, are output by workgroup 0. Thread
     *      t takes list entries [per t, per (t + 1)): one scan of the
     *      per-thread counts places them. ---- */
    {
        const uint32_t per = (nb + FN_THREADS - 1) / FN_THREADS;
        const uint32_t j0 = min(per * tid, nb), j1 = min(j0 + per, nb);
        uint32_t ng = 0u, ne = 0u;
        for (uint32_t j = j0; j < j1; j++) {
            const uint32_t key = (uint32_t)(ent(j) >> 32);
            ng += key > T ? 1u : 0u;
            ne += key == T ? 1u : 0u;
        }
        uint32_t all, pg, pe;
        if (nb <= 0xFFFFu) {                    /* both counts in one word */
            const uint32_t pre = tk_scan<FN_THREADS>(ng | (ne << 16), wsum, &all);
            pg = c_above + (pre & 0xFFFFu);
            pe = pre >> 16;
        } else {
            pg = c_above + tk_scan<FN_THREADS>(ng, wsum, &all);
            pe = tk_scan<FN_THREADS>(ne, wsum, &all);
        }
        if (ng | ne) {
            for (uint32_t j = j0; j < j1; j++) {
                const unsigned long long e = ent(j);
                const uint32_t key = (uint32_t)(e >> 32), idx = (uint32_t)e;
                if (key > T) {
                    if (pg < c_gt) cs[pg] = ((unsigned long long)key << 32) | (0xFFFFFFFFull - idx);
                    pg++;
                } else if (key == T) {
                    /* with NaNs, into the sorted selection instead */
                    if (pe < need_eq && nanm)
                        cs[c_gt + pe] = ((unsigned long long)key << 32) | (0xFFFFFFFFull - idx);
                    else if (pe < need_eq && blockIdx.x == 0)
                        idxs[c_gt + pe] = (int)idx;
                    pe++;
                }
            }
        }
    }
    __syncthreads();
    if (nanm) {
        /* cs[0 .. k): the candidates > T, then need_eq == T (below every
         * candidate, in index order as composites); zeros pad to a power
         * of two within cs, and the level-2/3 words after cs are free */
        const uint32_t np = pow2_at_least((uint32_t)k);
        for (uint32_t j = (uint32_t)k + tid; j < np; j += FN_THREADS) cs[j] = 0ull;
        lds_sort_desc<FN_THREADS>(cs, np);
        nan_finish<FN_THREADS>(idxs, cs, reinterpret_cast<uint32_t *>(sh + TK_KMAX), scores,
                               k, wsum);
        return;
    }

    /* ---- place this workgroup's candidates ---- */
    const uint32_t e = blockIdx.x * RK_EPW + tid / RK_TPE, sub = tid % RK_TPE;
    if (blockIdx.x * RK_EPW >= c_gt) return;            /* the whole workgroup */
    const unsigned long long mine = e < c_gt ? cs[e] : ~0ull;
    const uint32_t r = rank_count(cs, sub, c_gt, mine);
    if (sub == 0 && e < c_gt) idxs[r] = (int)(0xFFFFFFFFu - (uint32_t)mine);
}

/* Top-k of a short score vector (n <= TS_NMAX) in one launch: every
 * element's 64-bit composite (order key << 32 | ~index: descending composite
 * order is score descending, ties to the lower index) is ranked by counting
 * the composites above it -- the composites are distinct, so the ranks are
 * a permutation -- and the elements ranked below k land at idxs[rank]. A
 * workgroup stages all n composites in LDS (every score load issued before
 * any store) and ranks TS_EPW elements, TS_TPE threads per element: thread q
 * counts composites q, q + TS_TPE, ..., so the lanes of an element read
 * consecutive words (no bank conflicts) and the elements of a wave read the
 * same ones (broadcast); the count loop keeps 8 LDS reads in flight. */
constexpr int TS_NMAX = 4096;
constexpr int TS_TPE = 16;
constexpr int TS_EPW = 256 / TS_TPE;

__global__ void __launch_bounds__(256)
k_tk_small(int *__restrict__ idxs, const float *__restrict__ scores, int n, int k)
{
    __shared__ unsigned long long comp[TS_NMAX];
    bool nan = false;
    {
        constexpr int PT = TS_NMAX / 256;
        float v[PT];
#pragma unroll
        for (int u = 0; u < PT; u++) {
            const int i = u * 256 + (int)threadIdx.x;
            v[u] = i < n ? scores[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < PT; u++) {
            const int i = u * 256 + (int)threadIdx.x;
            if (i < n)
                comp[i] = ((unsigned long long)fkey(v[u]) << 32) | (0xFFFFFFFFu - (uint32_t)i);
            nan = nan || (i < n && __builtin_isnan(v[u]));
        }
    }
    const int anynan = __syncthreads_or(nan ? 1 : 0);
    const int e = blockIdx.x * TS_EPW + (int)(threadIdx.x / TS_TPE);
    const int q = threadIdx.x % TS_TPE;
    if (anynan) {
        /* every workgroup saw every score and takes this branch; workgroup
         * 0 sorts all n composites (NaNs keyed 0, zeros padding to a power
         * of two) and applies the reference's NaN rule (nan_finish) */
        __shared__ uint32_t wsum[256 / 64];
        if (blockIdx.x != 0) return;
        const uint32_t np = pow2_at_least((uint32_t)n);
        for (uint32_t j = (uint32_t)n + threadIdx.x; j < np; j += 256) comp[j] = 0ull;
        lds_sort_desc<256>(comp, np);
        nan_finish<256>(idxs, comp, reinterpret_cast<uint32_t *>(comp) + TS_NMAX, scores, k,
                        wsum);
        return;
    }
    const unsigned long long me = comp[min(e, n - 1)];
    int cnt = 0;
#pragma unroll 8
    for (int j = q; j < n; j += TS_TPE) cnt += comp[j] > me ? 1 : 0;
#pragma unroll
    for (int o = TS_TPE / 2; o >= 1; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
    if (q == 0 && e < n && cnt < k) idxs[cnt] = e;
}

/* ----------------------------------------------------- sparse attention */

constexpr int AT_THREADS = 256;
constexpr int AT_HB = 8;       /* heads per workgroup */

template <int KVF>
__device__ __forceinline__ float kv_at(const void *kv, size_t row, int stride, int c)
{
    if (KVF == DSV4_GPU_KV_BF16)
        return bf16_to_f32(((const uint16_t *)kv)[row * stride + c]);
    return ((const float *)kv)[row * stride + c];
}

/* Eight consecutive elements of a staged row, as floats. */
template <int KVF>
__device__ __forceinline__ void row8(const unsigned char *p, float *o)
{
    if (KVF == DSV4_GPU_KV_BF16) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(p);
        o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xFFFF0000u);
        o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xFFFF0000u);
        o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xFFFF0000u);
        o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xFFFF0000u);
    } else {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(p + 16);
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
}

template <int KVF>
__device__ __forceinline__ float row1(const unsigned char *p, int c)
{
    if (KVF == DSV4_GPU_KV_BF16) return bf16_to_f32(((const uint16_t *)p)[c]);
    return ((const float *)p)[c];
}

/* Selected row j of the attention: idxs[j], or with rw.on the attention
 * block's list built in place -- the window's ring slots newest first
 * (dsv4_attn.c:118-128), then the compressed rows offset past the window
 * (dsv4_indexer.c:113-117): all of them (mode 1) or the top-k's selection in
 * idxs[0 ...] (mode 2, negative entries kept). */
__device__ __forceinline__ int sel_row(const int *__restrict__ idxs, const Dsv4Rows &rw, int j)
{
    if (!rw.on) return idxs[j];
    if (j < rw.n_win) return (rw.pos - j) % rw.win;
    const int k = j - rw.n_win;
    if (rw.mode == 1) return rw.offset + k;
    const int v = idxs[k];
    return v >= 0 ? v + rw.offset : v;
}

/* One split of SR selected rows x one group of AT_HB heads.
 *   stage : the SR rows are gathered into LDS (every thread's loads in
 *           flight at once), with q of the group's heads;
 *   scores: thread (head, row) dots over d_qk from LDS;
 *   split softmax: per head m_s, e_j = expf(s_j - m_s), l_s;
 *   values: thread per column pair accumulates e_j * v_j over the rows for
 *           all heads of the group. */
template <int KVF>
__global__ void __launch_bounds__(AT_THREADS)
k_attn_partial(float *__restrict__ pm, float *__restrict__ pl,
               float *__restrict__ po, const float *__restrict__ q,
               const void *__restrict__ kv, int kv_stride,
               const int *__restrict__ idxs, int kv_rows, int h, int d_qk,
               int d_v, int topk, float scale, int SR, int rowb, int vec, int qnorm,
               float qeps, Dsv4Rope qrp, Dsv4Rows rw)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_b[];
    constexpr int ES = KVF == DSV4_GPU_KV_BF16 ? 2 : 4;
    const int ldq = d_qk + 4;
    float *qs = (float *)lds_b;                                  /* [HB][ldq]  */
    unsigned char *kvs = lds_b + (size_t)AT_HB * ldq * 4;        /* [SR][rowb] */
    float *ps = (float *)(kvs + (size_t)SR * rowb);              /* [SR][HB]   */
    int *sidx = (int *)(ps + (size_t)SR * AT_HB);                /* [SR]       */

    const int split = blockIdx.x, hg = blockIdx.y;
    const int nsplit = gridDim.x;
    const int h0 = hg * AT_HB;
    const int nh = min(AT_HB, h - h0);
    const int j0 = split * SR;
    const int nj = min(SR, topk - j0);
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int dmax = d_qk > d_v ? d_qk : d_v;

    __shared__ float rcs[RP_MAX], rsn[RP_MAX];
    const RopeRow rrow = rope_row_load(qrp);
    /* the split's row indices: loaded first, stored with q (so their wait is
     * q's) */
    int ridx = -1;
    if (tid < SR && tid < nj) ridx = sel_row(idxs, rw, j0 + tid);
    /* Staging issues a whole batch of loads before storing any of them: one
     * memory latency per batch rather than per element. */
    constexpr int SB = 8;
    if ((d_qk & 3) == 0 && (((uintptr_t)q & 15) == 0)) {
        /* 16-byte pieces: up to 8 x 1024 floats of q in one batch */
        const int nq4 = (AT_HB * d_qk) >> 2;
        for (int i0 = 0; i0 < nq4; i0 += SB * AT_THREADS) {
            f32x4 v[SB];
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const int i = i0 + u * AT_THREADS + tid;
                const int e = 4 * min(i, nq4 - 1), hh = e / d_qk, c = e - hh * d_qk;
                v[u] = (i < nq4 && hh < nh) ? ldf4(q + (size_t)(h0 + hh) * d_qk + c)
                                            : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const int i = i0 + u * AT_THREADS + tid;
                if (i < nq4) {
                    const int e = 4 * i, hh = e / d_qk, c = e - hh * d_qk;
                    *reinterpret_cast<f32x4 *>(qs + hh * ldq + c) = v[u];
                }
            }
        }
    } else {
        for (int i0 = 0; i0 < AT_HB * d_qk; i0 += SB * AT_THREADS) {
            float v[SB];
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const int i = i0 + u * AT_THREADS + tid;
                const int hh = i / d_qk, c = i - hh * d_qk;
                v[u] = (i < AT_HB * d_qk && hh < nh) ? q[(size_t)(h0 + hh) * d_qk + c] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const int i = i0 + u * AT_THREADS + tid;
                if (i < AT_HB * d_qk) {
                    const int hh = i / d_qk, c = i - hh * d_qk;
                    qs[hh * ldq + c] = v[u];
                }
            }
        }
    }
    if (tid < SR) sidx[tid] = (ridx >= 0 && ridx < kv_rows) ? ridx : -1;   /* never a wild read */
    rope_row_store(qrp, rrow, rcs, rsn);
    __syncthreads();
    /* the attention block's q: each head scaled by 1/sqrt(mean square +
     * eps) and RoPE'd at pos (dsv4_layer.c:223-231). All heads at once: QL
     * lanes per head (a half wave for AT_HB = 8). It touches only q's LDS
     * copy, so it runs while the row loads below are in flight. */
    auto q_transform = [&]() {
        constexpr int QL = AT_THREADS / AT_HB;
        const int t0 = d_qk - qrp.rd;
        const int hh = tid / QL, ql = tid - hh * QL;
        float *qh = qs + hh * ldq;
        float inv = 1.0f;
        if (qnorm) {
            double sq = 0.0;
            for (int c = ql; c < d_qk; c += QL) {
                const double v = (double)qh[c];
                sq += v * v;
            }
#pragma unroll
            for (int o = QL / 2; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
            inv = (float)(1.0 / sqrt(sq / (double)d_qk + (double)qeps));
            for (int c = ql; c < t0; c += QL) qh[c] = qh[c] * inv;
        }
        for (int p = ql; p < qrp.rd / 2; p += QL) {
            float a = qh[t0 + 2 * p], b = qh[t0 + 2 * p + 1];
            if (qnorm) { a = a * inv; b = b * inv; }
            rope_pair_cs(a, b, rcs[p], rsn[p], qrp.inverse);
            qh[t0 + 2 * p] = a;
            qh[t0 + 2 * p + 1] = b;
        }
    };
    const bool qx = qnorm || qrp.rd;
    /* stage the rows (q's transform between the first batch's loads and its
     * stores) */
    if (vec) {
        const int nc = dmax * ES / 16;                           /* 16-B chunks per row */
        for (int e0 = 0; e0 < SR * nc; e0 += SB * AT_THREADS) {
            u32x4 v[SB];
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const int e = e0 + u * AT_THREADS + tid;
                const int r = e / nc, c = e - r * nc;
                const int row = e < SR * nc ? sidx[r] : -1;
                v[u] = row >= 0
                    ? ld16((const unsigned char *)kv + ((size_t)row * kv_stride) * ES + (size_t)c * 16)
                    : u32x4{0, 0, 0, 0};
            }
            if (e0 == 0 && qx) q_transform();
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const int e = e0 + u * AT_THREADS + tid;
                if (e < SR * nc) {
                    const int r = e / nc, c = e - r * nc;
                    *reinterpret_cast<u32x4 *>(kvs + (size_t)r * rowb + (size_t)c * 16) = v[u];
                }
            }
        }
    } else {
        for (int e = tid; e < SR * dmax; e += AT_THREADS) {
            const int r = e / dmax, c = e - r * dmax;
            const int row = sidx[r];
            const float v = row >= 0 ? kv_at<KVF>(kv, (size_t)row, kv_stride, c) : 0.0f;
            if (KVF == DSV4_GPU_KV_BF16)
                ((uint16_t *)(kvs + (size_t)r * rowb))[c] = (uint16_t)(__float_as_uint(v) >> 16);
            else
                ((float *)(kvs + (size_t)r * rowb))[c] = v;
        }
        if (qx) q_transform();
    }
    __syncthreads();

    /* scores: the AT_HB x SR (head, row) pairs over every lane. A pair's dot
     * is split over LPP lanes that sit 64 / LPP apart in the wave (each takes
     * every LPP-th 8-column piece), so the 16-lane groups that read the LDS
     * together hold 16 different rows (the row pitch's 16-byte skew keeps
     * them on different banks) and the lanes of one head read q as a
     * broadcast. */
    if (KVF == DSV4_GPU_KV_F32 && SR == 16 && vec && (d_qk & 15) == 0 &&
        AT_HB * ldq >= 4 * 16 * 16) {
        /* f32 rows in 16-row splits: the scores as one 16 x 16 tile on the
         * matrix core (v_mfma_f32_16x16x4f32; rows x heads, heads past AT_HB
         * zero), each wave over a quarter of d_qk: every q and row element
         * is read from LDS once per wave instead of once per (head, row)
         * pair. The quarters' tiles meet in LDS (in q's region, which the
         * scores no longer need and which holds them), added in wave order. */
        static_assert(AT_HB <= 16 && AT_THREADS == 256, "one 16 x 16 tile, four waves");
        typedef float v4f_t __attribute__((ext_vector_type(4)));
        const int r16 = lane & 15, kq = lane >> 4;
        const float *krow = (const float *)(kvs + (size_t)r16 * rowb);
        const float *qrow = qs + (size_t)min(r16, AT_HB - 1) * ldq;
        const bool hv = r16 < AT_HB;
        const int kw = d_qk >> 2, kb = wid * kw;      /* a multiple of 4 */
        /* four independent chains over the quarter's steps (step s feeds
         * chain s % 4), each batch's LDS reads issued before its products */
        v4f_t acc[4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f},
                        {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        int k0 = kb;
        for (; k0 + 16 <= kb + kw; k0 += 16) {
            float a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                a[u] = krow[k0 + 4 * u + kq];
                b[u] = hv ? qrow[k0 + 4 * u + kq] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc[u], 0, 0, 0);
        }
        for (int u = 0; k0 < kb + kw; k0 += 4, u++) {
            const float a = krow[k0 + kq];
            const float b = hv ? qrow[k0 + kq] : 0.0f;
            if (u == 0) acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[0], 0, 0, 0);
            else if (u == 1) acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[1], 0, 0, 0);
            else acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[2], 0, 0, 0);
        }
        acc[0] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        __syncthreads();                       /* every wave is done with qs */
        float *red = qs;                       /* [4 waves][16 rows][16 heads] */
#pragma unroll
        for (int r = 0; r < 4; r++) red[(wid * 16 + 4 * kq + r) * 16 + r16] = acc[0][r];
        __syncthreads();
        if (tid < AT_HB * SR) {
            const int jj = tid / AT_HB, hh = tid - jj * AT_HB;
            const float v = ((red[jj * 16 + hh] + red[(16 + jj) * 16 + hh]) +
                             red[(32 + jj) * 16 + hh]) + red[(48 + jj) * 16 + hh];
            ps[jj * AT_HB + hh] = sidx[jj] >= 0 ? v * scale : -INFINITY;
        }
    } else {
        const int pairs = AT_HB * SR;
        const int LPP = pairs >= AT_THREADS ? 1 : (pairs * 2 >= AT_THREADS ? 2 : 4);
        const int span = 64 / LPP;                         /* pairs per wave per pass */
        const int part = lane / span, pl = lane - part * span;
        for (int pr0 = wid * span; pr0 < pairs; pr0 += (AT_THREADS / 64) * span) {
            const int pr = pr0 + pl;
            const bool live = pr < pairs;
            const int hh = live ? pr / SR : 0, jj = live ? pr - (pr / SR) * SR : 0;
            const float *qr = qs + hh * ldq;
            const unsigned char *kr = kvs + (size_t)jj * rowb;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            if (vec) {
#pragma unroll 4
                for (int c = 8 * part; c + 8 <= d_qk; c += 8 * LPP) {
                    float kk[8];
                    row8<KVF>(kr + (size_t)c * ES, kk);
                    const f32x4 qa = *reinterpret_cast<const f32x4 *>(qr + c);
                    const f32x4 qb = *reinterpret_cast<const f32x4 *>(qr + c + 4);
                    a0 = fmaf(qa.x, kk[0], a0); a1 = fmaf(qa.y, kk[1], a1);
                    a2 = fmaf(qa.z, kk[2], a2); a3 = fmaf(qa.w, kk[3], a3);
                    a0 = fmaf(qb.x, kk[4], a0); a1 = fmaf(qb.y, kk[5], a1);
                    a2 = fmaf(qb.z, kk[6], a2); a3 = fmaf(qb.w, kk[7], a3);
                }
                for (int c = (d_qk & ~7) + part; c < d_qk; c += LPP)
                    a0 = fmaf(qr[c], row1<KVF>(kr, c), a0);
            } else {
                for (int c = part; c < d_qk; c += LPP) a0 = fmaf(qr[c], row1<KVF>(kr, c), a0);
            }
            float v = (a0 + a1) + (a2 + a3);
            for (int o = span; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
            if (live && part == 0) ps[jj * AT_HB + hh] = sidx[jj] >= 0 ? v * scale : -INFINITY;
        }
    }
    __syncthreads();

    /* split softmax: G = SR lanes per head (SR is a power of two), 64 / G
     * heads per wave side by side */
    {
        const int G = SR < 64 ? SR : 64;
        const int hpw = 64 / G;
        const int gi = lane / G, gl = lane - gi * G;
        for (int hb = wid * hpw; hb < AT_HB; hb += (AT_THREADS / 64) * hpw) {
            const int hh = hb + gi;
            const bool hv = hh < AT_HB;
            float mx = -INFINITY;
            for (int j = gl; j < SR; j += G)
                if (hv) mx = fmaxf(mx, ps[j * AT_HB + hh]);
            for (int o = G / 2; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            float l = 0.0f;
            for (int j = gl; j < SR; j += G) {
                if (!hv) continue;
                const float sv = ps[j * AT_HB + hh];
                const float e = (mx == -INFINITY || sv == -INFINITY) ? 0.0f : expf(sv - mx);
                ps[j * AT_HB + hh] = e;
                l += e;
            }
            for (int o = G / 2; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
            if (gl == 0 && hv && hh < nh) {
                pm[(size_t)(h0 + hh) * nsplit + split] = mx;
                pl[(size_t)(h0 + hh) * nsplit + split] = l;
            }
        }
    }
    __syncthreads();

    /* values: thread per column pair, all heads of the group */
    for (int c = 2 * tid; c < d_v; c += 2 * AT_THREADS) {
        const bool two = c + 1 < d_v;
        float acc0[AT_HB], acc1[AT_HB];
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++) { acc0[hh] = 0.0f; acc1[hh] = 0.0f; }
#pragma unroll 4
        for (int jj = 0; jj < SR; jj++) {
            const unsigned char *kr = kvs + (size_t)jj * rowb;
            float v0, v1;
            if (KVF == DSV4_GPU_KV_F32 && two) {
                const float2 v = *reinterpret_cast<const float2 *>(kr + (size_t)c * 4);
                v0 = v.x; v1 = v.y;
            } else {
                v0 = row1<KVF>(kr, c);
                v1 = two ? row1<KVF>(kr, c + 1) : 0.0f;
            }
            const f32x4 pa = *reinterpret_cast<const f32x4 *>(ps + jj * AT_HB);
            const f32x4 pb = *reinterpret_cast<const f32x4 *>(ps + jj * AT_HB + 4);
            const float pp[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
            for (int hh = 0; hh < AT_HB; hh++) {
                acc0[hh] = fmaf(pp[hh], v0, acc0[hh]);
                acc1[hh] = fmaf(pp[hh], v1, acc1[hh]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++) {
            if (hh < nh) {
                float *dst = po + ((size_t)(h0 + hh) * nsplit + split) * d_v + c;
                if (two && (d_v & 1) == 0) {
                    *reinterpret_cast<float2 *>(dst) = make_float2(acc0[hh], acc1[hh]);
                } else {
                    dst[0] = acc0[hh];
                    if (two) dst[1] = acc1[hh];
                }
            }
        }
    }
}

/* Combine: workgroup (head, slice of CB_COLS columns); every workgroup of a
 * head derives the same split weights and denominator. */
constexpr int CB_COLS = 128;
constexpr int CB_SPLITS = 1024;

/* Head hh, columns [CB_COLS cy, CB_COLS (cy + 1)); fs and lp hold
 * CB_SPLITS floats each (lp: l_s * e^(m_s - M), rounded to float). */
__device__ __forceinline__ void cb_body(float *__restrict__ o, const float *__restrict__ pm,
                                        const float *__restrict__ pl, const float *__restrict__ po,
                                        const float *__restrict__ sink, int nsplit, int d_v,
                                        const Dsv4Rope &orp, int hh, int cy, float *fs, float *lp,
                                        float *sh_inv_p)
{
    float &sh_inv = *sh_inv_p;
    const int tid = threadIdx.x;
    if (tid < 64) {
        const float sk = sink ? sink[hh] : 0.0f;
        float M = -INFINITY;
        for (int s = tid; s < nsplit; s += 64) M = fmaxf(M, pm[(size_t)hh * nsplit + s]);
        M = wave_max(M);
        /* the lanes form the denominator's terms in parallel; lane 0 then
         * adds them in split order from LDS */
        for (int s = tid; s < nsplit; s += 64) {
            const float ms = pm[(size_t)hh * nsplit + s];
            const float ls = pl[(size_t)hh * nsplit + s];
            const float f = (ms == -INFINITY) ? 0.0f : expf(ms - M);
            fs[s] = f;
            lp[s] = ls * f;
        }
        /* lane 0 reads the other lanes' terms: order the wave's LDS writes
         * before its reads (a wave-scope release / acquire around the wave
         * barrier, so the compiler cannot hoist the reads either) */
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (tid == 0) {
            double denom = 0.0;
#pragma unroll 8
            for (int s = 0; s < nsplit; s++) denom += (double)lp[s];
            if (sink) denom += (double)expf(sk - M);
            sh_inv = (float)(1.0 / denom);
        }
    }
    const int c = cy * CB_COLS + tid;
    const bool live = c < d_v;
    const int cc = live ? c : d_v - 1;
    /* this column's de-rotation pair's cos / sin, loaded with the partials */
    const int rt0 = d_v - orp.rd;
    float rcv = 1.0f, rsv = 0.0f;
    if (orp.rd && live && c >= rt0) {
        rcv = orp.cs[(size_t)orp.pos * orp.half + ((c - rt0) >> 1)];
        rsv = orp.sn[(size_t)orp.pos * orp.half + ((c - rt0) >> 1)];
    }
    /* the partials' loads do not wait for the weights */
    constexpr int B = 32;
    float v[B];
    int s0 = 0;
#pragma unroll
    for (int u = 0; u < B; u++)
        v[u] = po[((size_t)hh * nsplit + min(u, nsplit - 1)) * d_v + cc];
    __syncthreads();
    const float inv = sh_inv;
    float acc = 0.0f;
    for (;;) {
#pragma unroll
        for (int u = 0; u < B; u++)
            if (s0 + u < nsplit) acc = fmaf(v[u], fs[s0 + u], acc);
        s0 += B;
        if (s0 >= nsplit) break;
#pragma unroll
        for (int u = 0; u < B; u++)
            v[u] = po[((size_t)hh * nsplit + min(s0 + u, nsplit - 1)) * d_v + cc];
    }
    float val = acc * inv;
    if (orp.rd) {
        /* the output's de-rotation (dsv4_layer.c:304-305): column pairs
         * (t0 + 2p, t0 + 2p + 1) sit in neighbouring lanes */
        const float other = __shfl_xor(val, 1, 64);
        if (c >= rt0 && live) {
            const bool odd = (c - rt0) & 1;
            float a = odd ? other : val, b = odd ? val : other;
            rope_pair_cs(a, b, rcv, rsv, orp.inverse);
            val = odd ? b : a;
        }
    }
    if (live) o[(size_t)hh * d_v + c] = val;
}

__global__ void __launch_bounds__(CB_COLS)
k_attn_combine(float *__restrict__ o, const float *__restrict__ pm,
               const float *__restrict__ pl, const float *__restrict__ po,
               const float *__restrict__ sink, int nsplit, int d_v, Dsv4Rope orp)
{
    __shared__ float fs[CB_SPLITS], lp[CB_SPLITS], sh_inv;
    cb_body(o, pm, pl, po, sink, nsplit, d_v, orp, blockIdx.x, blockIdx.y, fs, lp, &sh_inv);
}

/* ------------------------------------------ sparse attention, matrix core */

/* The same split softmax on v_mfma_f32_16x16x32_bf16 for bf16 KV, d_qk a
 * multiple of 32, d_v of 16 and h of 16 (h <= 128). Operand layout of the
 * MFMA (measured on gfx950): A lane l holds row l%16, K elements [8(l/16),
 * +8); B lane l holds column l%16, the same K elements; D lane l, register
 * j holds row 4(l/16) + j, column l%16.
 *
 * q and the softmax weights are f32: each is carried as three bf16 terms
 * hi + mid + lo, which hold all 24 bits, against the exact bf16 KV, so every
 * product is exact and the sums accumulate in f32 (in another order than
 * the reference's; within 1e-5 relative).
 *
 * One workgroup of AM_WAVES waves per split of AM_SR selected rows:
 *   stage : the rows, gathered once: row-major for the scores' B operand
 *           (K rows), transposed (columns x rows) for the values' B operand;
 *   scores: S = q . K^T, (head tile, half of the rows) per wave;
 *   softmax: per head m_s, e_j = expf(s_j - m_s), l_s (rows in lanes);
 *   values: O_s = P . V, (head tile, columns) per wave;
 * then k_attn_combine as for the VALU form. */
typedef float am_v4f __attribute__((ext_vector_type(4)));
typedef __bf16 am_v8bf __attribute__((ext_vector_type(8)));
typedef short am_v8s __attribute__((ext_vector_type(8)));

constexpr int AM_SR = 64;                        /* rows per split */
constexpr int AM_WAVES = 8;
constexpr int AM_THREADS = AM_WAVES * 64;
constexpr int AM_PP = AM_SR + 4;                 /* weights pitch (f32) */
constexpr int AM_KCMAX = 20;                     /* d_qk <= 32 AM_KCMAX */

typedef __bf16 am_v2bf __attribute__((ext_vector_type(2)));
typedef float am_v2f __attribute__((ext_vector_type(2)));

/* Two f32 values -> two bf16 (round to nearest even, v_cvt_pk_bf16_f32). */
__device__ __forceinline__ uint32_t am_cvt2(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(am_v2f{a, b}, am_v2bf));
}

/* Eight f32 values -> their three bf16 term vectors (v = t0 + t1 + t2,
 * exactly: each residual is exact in f32). */
__device__ __forceinline__ void am_terms8(const float *v, am_v8bf *t)
{
    u32x4 w[3];
    uint32_t *w0 = (uint32_t *)&w[0], *w1 = (uint32_t *)&w[1], *w2 = (uint32_t *)&w[2];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = v[2 * i], b = v[2 * i + 1];
        const uint32_t hi = am_cvt2(a, b);
        const float ra = a - __uint_as_float(hi << 16), rb = b - __uint_as_float(hi & 0xFFFF0000u);
        const uint32_t mi = am_cvt2(ra, rb);
        const float sa = ra - __uint_as_float(mi << 16), sb = rb - __uint_as_float(mi & 0xFFFF0000u);
        w0[i] = hi;
        w1[i] = mi;
        w2[i] = am_cvt2(sa, sb);
    }
    t[0] = __builtin_bit_cast(am_v8bf, w[0]);
    t[1] = __builtin_bit_cast(am_v8bf, w[1]);
    t[2] = __builtin_bit_cast(am_v8bf, w[2]);
}

/* LDS layout in bytes for a shape and nw waves: the rows [AM_SR][kp],
 * row-major, then the score partials [nw][16][AM_PP] f32, which the weights
 * [16][AM_PP] reuse. */
__host__ __device__ __forceinline__ int am_kpitch(int d_qk) { return 2 * d_qk + 16; }
__host__ __device__ __forceinline__ size_t am_lds_bytes(int d_qk, int nw)
{
    return (size_t)AM_SR * am_kpitch(d_qk) + sizeof(float) * nw * 16 * AM_PP;
}

typedef short am_v4s __attribute__((ext_vector_type(4)));
typedef short am_v8s __attribute__((ext_vector_type(8)));

/* The values' B operand for rows r0 .. r0 + 31 of a chunk and columns
 * cb .. cb + 15, read transposed from the row-major rows: lane l gets
 * V[r0 + 8 (l / 16) + e][cb + l % 16], e = 0 .. 7. ds_read_b64_tr_b16 gives
 * lane i of each 16-lane group element (i % 4) of the four 16-bit values
 * that lane 4 j + i / 4 addressed, as its element j (checked on the GPU);
 * so lane 4 j + q addresses row r0 + 8 (l / 16) + j, columns cb + 4 q ..
 * cb + 4 q + 3, and a second read four rows further gives e = 4 .. 7. */
__device__ __forceinline__ am_v8bf am_vfrag(const unsigned char *kr, int kp, int r0, int cb,
                                             int l16, int g)
{
    const unsigned char *a =
        kr + (size_t)(r0 + 8 * g + (l16 >> 2)) * kp + 2 * (cb + 4 * (l16 & 3));
    typedef __attribute__((address_space(3))) am_v4s lds_v4s;
    const am_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s *)a);
    const am_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s *)(a + 4 * kp));
    const am_v8s both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(am_v8bf, both);
}

/* The attention of one workgroup, NW waves: (split of AM_SR rows, tile of
 * 16 heads), the split's rows in sidx (set by the caller before the call,
 * -1 masked):
 *   stage : the rows gathered once into LDS, row-major, consecutive lanes
 *           on consecutive 16-byte pieces of a row (each cache line fetched
 *           once, every load issued before any store); meanwhile each wave
 *           loads q for its K chunks w, w + NW, ...;
 *   scores: each wave the partial S over its K chunks for all row tiles,
 *           summed across the waves in LDS in wave order;
 *   softmax: per head m_s, e_j = expf(s_j - m_s), l_s (lane = row), 16 / NW
 *           heads per wave;
 *   values: O_s = P . V, each wave every NW-th column tile. */
template <int NW>
__device__ __forceinline__ void am_body(float *__restrict__ pm, float *__restrict__ pl,
                                        float *__restrict__ po, const float *__restrict__ q,
                                        const uint16_t *__restrict__ kv, int kv_stride,
                                        int d_qk, int d_v, float scale, int split, int nsplit,
                                        int ht, const int *sidx, unsigned char *am_lds)
{
    constexpr int NT = 64 * NW;
    constexpr int KCW = (AM_KCMAX + NW - 1) / NW;      /* K chunks per wave */
    constexpr int HPW = 16 / NW;                       /* softmax heads per wave */
    constexpr int VT = 32 / NW;                        /* value column tiles per pass */
    const int kp = am_kpitch(d_qk);
    unsigned char *kr = am_lds;                                  /* [AM_SR][kp] */
    float *red = (float *)(am_lds + (size_t)AM_SR * kp);         /* [NW][16][AM_PP] */
    float *pw = red;                                             /* [16][AM_PP] */
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int KC = d_qk / 32;

    /* q of the head tile for this wave's K chunks (A operand rows l%16, K
     * [8(l/16), +8) of each chunk), in flight with the staging loads */
    float qv[KCW][8];
    {
        const float *qr = q + (size_t)(ht * 16 + l16) * d_qk + 8 * g;
#pragma unroll
        for (int i = 0; i < KCW; i++) {
            const int kc = min(wv + NW * i, KC - 1);
            const f32x4 a0 = ldf4(qr + 32 * kc), a1 = ldf4(qr + 32 * kc + 4);
            qv[i][0] = a0.x; qv[i][1] = a0.y; qv[i][2] = a0.z; qv[i][3] = a0.w;
            qv[i][4] = a1.x; qv[i][5] = a1.y; qv[i][6] = a1.z; qv[i][7] = a1.w;
        }
    }
    __syncthreads();                                   /* sidx visible */

    /* ---- stage: piece p = u NT + tid of the split is row p / ck, 16-byte
     *      piece p % ck (stepped without a division per piece); a masked
     *      row loads row 0 and stores zeros ---- */
    {
        const int ck = d_qk / 8;                                 /* pieces per row */
        const int np = AM_SR * ck;
        constexpr int NB = (AM_SR * 4 * AM_KCMAX + NT - 1) / NT; /* pieces per thread, at most */
        const int dr = NT / ck, dp = NT - dr * ck;
        int rr = tid / ck, pc = tid - rr * ck;
        u32x4 v[NB];
        bool z[NB];
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int r = min(rr, AM_SR - 1), row = sidx[r];
            const int pcc = u * NT + tid < np ? pc : ck - 1;
            v[u] = *(const DSV4_GLOBAL u32x4 *)(kv + (size_t)max(row, 0) * kv_stride + 8 * pcc);
            z[u] = row < 0;
            rr += dr;
            pc += dp;
            if (pc >= ck) { pc -= ck; rr++; }
        }
        rr = tid / ck;
        pc = tid - rr * ck;
#pragma unroll
        for (int u = 0; u < NB; u++) {
            if (u * NT + tid < np)
                *reinterpret_cast<u32x4 *>(kr + (size_t)rr * kp + 16 * pc) =
                    z[u] ? u32x4{0u, 0u, 0u, 0u} : v[u];
            rr += dr;
            pc += dp;
            if (pc >= ck) { pc -= ck; rr++; }
        }
    }
    __syncthreads();

    /* ---- scores: this wave's K chunks for all four row tiles; one
     *      accumulator per (row tile, term) ---- */
    am_v4f acc[4][3];
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
#pragma unroll
        for (int t = 0; t < 3; t++) acc[rt][t] = am_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KCW; i++) {
        const int kc = wv + NW * i;
        if (kc < KC) {
            am_v8bf bk[4];
#pragma unroll
            for (int rt = 0; rt < 4; rt++)
                bk[rt] = __builtin_bit_cast(am_v8bf, *reinterpret_cast<const u32x4 *>(
                    kr + (size_t)(rt * 16 + l16) * kp + 2 * (32 * kc + 8 * g)));
            am_v8bf at[3];
            am_terms8(qv[i], at);
#pragma unroll
            for (int t = 0; t < 3; t++)
#pragma unroll
                for (int rt = 0; rt < 4; rt++)
                    acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at[t], bk[rt],
                                                                        acc[rt][t], 0, 0, 0);
        }
    }
#pragma unroll
    for (int rt = 0; rt < 4; rt++) {
        const am_v4f sv = (acc[rt][0] + acc[rt][1]) + acc[rt][2];
#pragma unroll
        for (int j = 0; j < 4; j++)
            red[(wv * 16 + 4 * g + j) * AM_PP + rt * 16 + l16] = sv[j];
    }
    __syncthreads();

    /* ---- split softmax: wave w takes heads HPW w .. HPW w + HPW - 1,
     *      lane = row; the partials summed in wave order ---- */
    {
        const bool live = sidx[lane] >= 0;
        float sv[HPW], m[HPW], e[HPW], l[HPW];
#pragma unroll
        for (int i = 0; i < HPW; i++) {
            const int hh = HPW * wv + i;
            float a = red[hh * AM_PP + lane];
#pragma unroll
            for (int w = 1; w < NW; w++) a = a + red[(w * 16 + hh) * AM_PP + lane];
            sv[i] = live ? a * scale : -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < HPW; i++) m[i] = wave_max(sv[i]);
#pragma unroll
        for (int i = 0; i < HPW; i++)
            e[i] = (m[i] == -INFINITY || sv[i] == -INFINITY) ? 0.0f : expf(sv[i] - m[i]);
#pragma unroll
        for (int i = 0; i < HPW; i++) l[i] = wave_sum(e[i]);
        __syncthreads();                /* every partial read before pw overwrites */
#pragma unroll
        for (int i = 0; i < HPW; i++) pw[(HPW * wv + i) * AM_PP + lane] = e[i];
        if (lane < HPW) {
            float mi = m[0], li = l[0];
#pragma unroll
            for (int i = 1; i < HPW; i++) if (lane == i) { mi = m[i]; li = l[i]; }
            const int hh = ht * 16 + HPW * wv + lane;
            pm[(size_t)hh * nsplit + split] = mi;
            pl[(size_t)hh * nsplit + split] = li;
        }
    }
    __syncthreads();

    /* ---- values: column tiles wv, wv + NW, ... ---- */
    const int CT = d_v / 16;
    for (int c0 = wv; c0 < CT; c0 += VT * NW) {
        am_v4f o[VT];
#pragma unroll
        for (int ct = 0; ct < VT; ct++) o[ct] = am_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < AM_SR / 32; kc++) {
            const float *pr = pw + l16 * AM_PP + 32 * kc + 8 * g;
            const f32x4 a0 = *reinterpret_cast<const f32x4 *>(pr);
            const f32x4 a1 = *reinterpret_cast<const f32x4 *>(pr + 4);
            const float pv[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            am_v8bf at[3];
            am_terms8(pv, at);
            am_v8bf bv[VT];
#pragma unroll
            for (int ct = 0; ct < VT; ct++)
                bv[ct] = am_vfrag(kr, kp, 32 * kc, min(c0 + NW * ct, CT - 1) * 16, l16, g);
#pragma unroll
            for (int t = 0; t < 3; t++)
#pragma unroll
                for (int ct = 0; ct < VT; ct++)
                    o[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at[t], bv[ct], o[ct], 0, 0, 0);
        }
#pragma unroll
        for (int ct = 0; ct < VT; ct++) {
            const int cti = c0 + NW * ct;
            if (cti < CT) {
                const int c = cti * 16 + l16;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int hh = ht * 16 + 4 * g + j;
                    po[((size_t)hh * nsplit + split) * d_v + c] = o[ct][j];
                }
            }
        }
    }
}

/* Workgroup (split of AM_SR rows, tile of 16 heads), AM_WAVES waves: the
 * split's rows are idxs[AM_SR split ...]. */
__global__ void __launch_bounds__(AM_THREADS)
k_attn_mc(float *__restrict__ pm, float *__restrict__ pl, float *__restrict__ po,
          const float *__restrict__ q, const uint16_t *__restrict__ kv, int kv_stride,
          const int *__restrict__ idxs, int kv_rows, int d_qk, int d_v, int topk, float scale)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char am_lds[];
    __shared__ int sidx[AM_SR];
    const int j0 = blockIdx.x * AM_SR;
    if (threadIdx.x < AM_SR) {
        const int r = j0 + (int)threadIdx.x < topk ? idxs[j0 + threadIdx.x] : -1;
        sidx[threadIdx.x] = (r >= 0 && r < kv_rows) ? r : -1;    /* never a wild read */
    }
    am_body<AM_WAVES>(pm, pl, po, q, kv, kv_stride, d_qk, d_v, scale, blockIdx.x, gridDim.x,
                      blockIdx.y, sidx, am_lds);
}

/* LDS bytes of k_attn_mc for a shape, 0 when the shape is not one it takes. */
size_t attn_mc_lds(int kv_fmt, int h, int d_qk, int d_v, int kv_stride)
{
    if (kv_fmt != DSV4_GPU_KV_BF16 || h % 16 || d_qk % 32 || d_qk > 32 * AM_KCMAX ||
        d_v % 16 || d_v > d_qk || kv_stride % 8)
        return 0;
    const size_t lds = am_lds_bytes(d_qk, AM_WAVES);
    return lds + AM_SR * sizeof(int) <= dsv4_lds_limit() ? lds : 0;
}

/* Rows per split: the staged rows, q and the scores must fit the LDS a
 * workgroup may use. */
size_t attn_partial_lds(int sr, int d_qk, int rowb)
{
    return (size_t)AT_HB * (d_qk + 4) * 4 + (size_t)sr * rowb + (size_t)sr * AT_HB * 4 +
           (size_t)sr * 4;
}

/* Rows per split of the VALU form: the most that fit the LDS (at most 64),
 * halved while the grid would leave most CUs idle (splits x head groups
 * below two per CU), down to AT_SR_MIN -- the staged rows' LDS traffic of a
 * split grows with its rows, so short selections spread over more CUs. With
 * topk < 0 only the LDS bound applies. */
constexpr int AT_SR_MIN = 16;

int attn_split_rows(int kv_fmt, int d_qk, int d_v, int *rowb_out, size_t *lds_out,
                    int h = 0, int topk = -1)
{
    const size_t cap = dsv4_lds_limit();
    const int es = kv_fmt == DSV4_GPU_KV_BF16 ? 2 : 4;
    const int dmax = d_qk > d_v ? d_qk : d_v;
    const int rowb = ((dmax * es + 15) / 16) * 16 + 16;          /* +16 B: bank skew */
    int sr = 64;
    /* (the kernel's static LDS, the RoPE row, comes on top) */
    while (sr >= 1 && attn_partial_lds(sr, d_qk, rowb) + 2 * RP_MAX * sizeof(float) > cap)
        sr >>= 1;
    if (sr < 1) return 0;
    if (topk > 0) {
        static int cus = 0;
        if (!cus) {
            int dev = 0, v = 0;
            cus = (hipGetDevice(&dev) == hipSuccess &&
                   hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                       hipSuccess && v > 0) ? v : 256;
        }
        const int hg = (h + AT_HB - 1) / AT_HB;
        while (sr > AT_SR_MIN && ((topk + sr - 1) / sr) * hg < 2 * cus) sr >>= 1;
    }
    *rowb_out = rowb;
    *lds_out = attn_partial_lds(sr, d_qk, rowb);
    return sr;
}

} // namespace

/* Index scratch: [hist: TK_SLICES x TK_BINS u32][meta: 256 B]
 * [cand: TK_KMAX u64][bsel: RF_LIST u64][bcnt: RF_GMAX u32]
 * [blist: G x PT_ELEMS u64]. The histogram and the append counter must be
 * zero when a top-k starts from them; every top-k leaves the histogram
 * zero, and the score kernel (or k_tk_hist) restarts the counter. */
static const size_t IX_HIST = 0;
static const size_t IX_META = IX_HIST + sizeof(uint32_t) * TK_SLICES * TK_BINS;
static const size_t IX_CAND = IX_META + 256;
static const size_t IX_BSEL = IX_CAND + sizeof(unsigned long long) * TK_KMAX;
static const size_t IX_BCNT = IX_BSEL + sizeof(unsigned long long) * RF_LIST;
static const size_t IX_BLIST = IX_BCNT + sizeof(uint32_t) * RF_GMAX;

static int ix_heads_padded(int H) { return (H + IS_HB - 1) / IS_HB * IS_HB; }

size_t dsv4_index_scratch_bytes(int n)
{
    const size_t g = n > 0 ? ((size_t)n + PT_ELEMS - 1) / PT_ELEMS : 1;
    return IX_BLIST + sizeof(unsigned long long) * PT_ELEMS * g;
}

int dsv4_topk_kmax(void) { return TK_KMAX; }

int dsv4_attn_max_rows(int kv_fmt, int d_qk, int d_v)
{
    int rowb;
    size_t lds;
    const int sr = attn_split_rows(kv_fmt, d_qk, d_v, &rowb, &lds);
    /* the launch halves the split width only while the splits are fewer
     * than two per CU (< 1024), so the base width bounds the rows */
    return sr > 0 ? 1024 * sr : 0;
}

int dsv4_topk_takes_hist(int n, int k)
{
    return k > 0 && n >= k && n > TS_NMAX && n <= TK_NMAX && k <= TK_KMAX;
}

int dsv4_indexer_score_rope_launch(float *d_out, const float *d_q, const float *d_w,
                                   int H, int D, const void *d_keys,
                                   const float *d_key_scales, int key_fmt,
                                   int key_stride, int n, float scale, void *scratch,
                                   int with_hist, const float *rope_cs,
                                   const float *rope_sn, int rope_pos, int rope_half,
                                   int rope_dim, hipStream_t st)
{
    if (H <= 0 || D <= 0 || n < 0 || key_stride < D || H > 256 || rope_dim < 0 ||
        (rope_dim & 1) || rope_dim > D || rope_dim > 2 * RP_MAX ||
        (rope_dim && (!rope_cs || !rope_sn))) {
        DSV4_ERR("indexer score: bad shape H %d D %d n %d stride %d rope %d",
                 H, D, n, key_stride, rope_dim);
        return -1;
    }
    if (key_fmt == DSV4_GPU_KV_FP8 && !d_key_scales) {
        DSV4_ERR("indexer score: FP8 keys need row scales");
        return -1;
    }
    if (key_fmt != DSV4_GPU_KV_FP8 && key_fmt != DSV4_GPU_KV_BF16 &&
        key_fmt != DSV4_GPU_KV_F32) {
        DSV4_ERR("indexer score: unknown key format %d", key_fmt);
        return -1;
    }
    if (n == 0) return 0;
    /* few f32 keys: a thread per (key, head) (at C4's 32768 FP8 keys the
     * same kernel measured slower than the lane-per-row one, 20.5 vs 13.8
     * us, so it stays for short score vectors) */
    if (key_fmt == DSV4_GPU_KV_F32 && !with_hist && n <= SK_NMAX && (D & 3) == 0 &&
        ((uintptr_t)d_q & 15) == 0) {
        int hp = 1;
        while (hp < H) hp <<= 1;                   /* H <= 256: a power of two divides 256 */
        const size_t lds = sizeof(double) * ((size_t)(SK_THREADS / hp) * hp + H) +
                           sizeof(float) * ((size_t)H * (D + 1) + (size_t)(SK_THREADS / hp) * D);
        if (lds <= dsv4_lds_limit()) {
            static bool kh_opted = false;
            if (!kh_opted) {
                (void)dsv4_lds_optin((const void *)k_iscore_kh<DSV4_GPU_KV_F32>,
                                     dsv4_lds_limit(), "indexer score");
                kh_opted = true;
            }

            Dsv4Rope qr;
            if (rope_dim) {
                qr.cs = rope_cs; qr.sn = rope_sn; qr.pos = rope_pos; qr.half = rope_half;
                qr.rd = rope_dim;
            }
            const int kpw = SK_THREADS / hp;
            hipLaunchKernelGGL((k_iscore_kh<DSV4_GPU_KV_F32>), dim3((n + kpw - 1) / kpw),
                               dim3(SK_THREADS), lds, st, d_out, d_q, d_w, H,
                               hp, D, d_keys, d_key_scales, key_stride, n, scale, qr);
            HIP_OK(hipGetLastError(), "indexer score (few keys) launch");
            return 0;
        }
    }
    uint32_t *hist = with_hist ? (uint32_t *)((char *)scratch + IX_HIST) : nullptr;
    uint32_t *meta = with_hist ? (uint32_t *)((char *)scratch + IX_META) : nullptr;
    Dsv4Rope qr;
    if (rope_dim) {
        qr.cs = rope_cs; qr.sn = rope_sn; qr.pos = rope_pos; qr.half = rope_half;
        qr.rd = rope_dim;
    }
    const int es = key_fmt == DSV4_GPU_KV_F32 ? 4 : key_fmt == DSV4_GPU_KV_BF16 ? 2 : 1;

    /* the matrix-core form where the shape allows (DSV4_GPU_SCORE_MC=0 keeps
     * the VALU form) */
    const char *mc_env = getenv("DSV4_GPU_SCORE_MC");
    if (D % 4 == 0 && D <= MF_DMAX && H <= 64 && !(mc_env && atoi(mc_env) == 0)) {
        const int HT = H <= 16 ? 1 : H <= 32 ? 2 : 4;
        const size_t lds = mf_lds_bytes(H, HT, D, with_hist);
        if (lds <= dsv4_lds_limit()) {
            static bool mf_opted = false;
            if (!mf_opted) {
                const size_t cap = dsv4_lds_limit();
#define DSV4_MF_OPT(KF, P)                                                                  \
    do {                                                                                    \
        const void *f_[] = {(const void *)k_iscore_mf<KF, P, 0, 1>,                         \
                            (const void *)k_iscore_mf<KF, P, 0, 2>,                         \
                            (const void *)k_iscore_mf<KF, P, 0, 4>,                         \
                            (const void *)k_iscore_mf<KF, P, 1, 1>,                         \
                            (const void *)k_iscore_mf<KF, P, 1, 2>,                         \
                            (const void *)k_iscore_mf<KF, P, 1, 4>};                        \
        for (const void *f : f_) (void)dsv4_lds_optin(f, cap, "indexer score");            \
    } while (0)
                DSV4_MF_OPT(DSV4_GPU_KV_FP8, 1);
                DSV4_MF_OPT(DSV4_GPU_KV_FP8, 0);
                DSV4_MF_OPT(DSV4_GPU_KV_BF16, 0);
                DSV4_MF_OPT(DSV4_GPU_KV_F32, 0);
#undef DSV4_MF_OPT
                mf_opted = true;
            }
            const bool piece = key_fmt == DSV4_GPU_KV_FP8 && D % 16 == 0 &&
                               key_stride % 16 == 0 && ((uintptr_t)d_keys & 15) == 0;
            const int grid = (n + MF_ROWS - 1) / MF_ROWS;
#define DSV4_MF_GO(KF, P, HS, HTV)                                                          \
    hipLaunchKernelGGL((k_iscore_mf<KF, P, HS, HTV>), dim3(grid), dim3(MF_WAVES * 64), lds, st,  \
                       d_out, hist, meta, d_q, d_w, H, D, d_keys, d_key_scales, key_stride, n,  \
                       scale, qr)
#define DSV4_MF_HT(KF, P, HS)                                                               \
    do {                                                                                    \
        if (HT == 1) DSV4_MF_GO(KF, P, HS, 1);                                              \
        else if (HT == 2) DSV4_MF_GO(KF, P, HS, 2);                                         \
        else DSV4_MF_GO(KF, P, HS, 4);                                                      \
    } while (0)
#define DSV4_MF_KF(KF, P)                                                                   \
    do {                                                                                    \
        if (with_hist) DSV4_MF_HT(KF, P, 1); else DSV4_MF_HT(KF, P, 0);                     \
    } while (0)
            if (piece) DSV4_MF_KF(DSV4_GPU_KV_FP8, 1);
            else if (key_fmt == DSV4_GPU_KV_FP8) DSV4_MF_KF(DSV4_GPU_KV_FP8, 0);
            else if (key_fmt == DSV4_GPU_KV_BF16) DSV4_MF_KF(DSV4_GPU_KV_BF16, 0);
            else DSV4_MF_KF(DSV4_GPU_KV_F32, 0);
#undef DSV4_MF_KF
#undef DSV4_MF_HT
#undef DSV4_MF_GO
            HIP_OK(hipGetLastError(), "indexer score (matrix cores) launch");
            return 0;
        }
    }

    const int HP = ix_heads_padded(H);
    /* four waves per workgroup where the heads allow it: one wave per SIMD
     * of a CU (up to 4 head waves per block of 64 rows, blocks filling the
     * rest); f32 keys (the attention block's compressed rows: few rows, many
     * heads) take up to 8 head waves, two per SIMD */
    const int groups = HP / IS_HB;
    const bool mw8 = key_fmt == DSV4_GPU_KV_F32 && groups >= 8;
    const int mw = mw8 ? 8 : IS_MAXW;
    const int ng = groups < mw ? groups : mw;
    const int kb = mw / ng;
    const size_t lds = sizeof(double) * ((size_t)64 * kb * (HP + 1) + HP) +
                       sizeof(float) * (size_t)H * D +
                       (with_hist ? sizeof(uint32_t) * TK_BINS : 0);
    if (lds > dsv4_lds_limit()) {
        DSV4_ERR("indexer score: %d heads do not fit in LDS", H);
        return -1;
    }
    static bool lds_opted = false;
    if (!lds_opted) {
        const size_t cap = dsv4_lds_limit();
        const void *fns[] = {
            (const void *)k_iscore<DSV4_GPU_KV_FP8, 1, 0, 4>, (const void *)k_iscore<DSV4_GPU_KV_FP8, 1, 1, 4>,
            (const void *)k_iscore<DSV4_GPU_KV_FP8, 0, 0, 4>, (const void *)k_iscore<DSV4_GPU_KV_FP8, 0, 1, 4>,
            (const void *)k_iscore<DSV4_GPU_KV_BF16, 1, 0, 4>, (const void *)k_iscore<DSV4_GPU_KV_BF16, 1, 1, 4>,
            (const void *)k_iscore<DSV4_GPU_KV_BF16, 0, 0, 4>, (const void *)k_iscore<DSV4_GPU_KV_BF16, 0, 1, 4>,
            (const void *)k_iscore<DSV4_GPU_KV_F32, 1, 0, 4>, (const void *)k_iscore<DSV4_GPU_KV_F32, 1, 1, 4>,
            (const void *)k_iscore<DSV4_GPU_KV_F32, 0, 0, 4>, (const void *)k_iscore<DSV4_GPU_KV_F32, 0, 1, 4>,
            (const void *)k_iscore<DSV4_GPU_KV_F32, 1, 0, 8>, (const void *)k_iscore<DSV4_GPU_KV_F32, 1, 1, 8>,
            (const void *)k_iscore<DSV4_GPU_KV_F32, 0, 0, 8>, (const void *)k_iscore<DSV4_GPU_KV_F32, 0, 1, 8>};
        for (const void *f : fns) (void)dsv4_lds_optin(f, cap, "indexer score");
        lds_opted = true;
    }
    const bool vec = ((size_t)D * es) % 16 == 0 && ((size_t)key_stride * es) % 16 == 0 &&
                     ((uintptr_t)d_keys & 15) == 0;
    const int grid = (n + 64 * kb - 1) / (64 * kb);
    const int thr = 64 * ng * kb;
#define DSV4_ISCORE(KF, MW)                                                             \
    do {                                                                                \
        if (with_hist)                                                                  \
            launch_iscore<KF, 1, MW>(vec, grid, thr, lds, st, d_out, hist, meta, d_q, d_w, H, \
                                     HP, D, d_keys, d_key_scales, key_stride, n, scale, ng, qr); \
        else                                                                            \
            launch_iscore<KF, 0, MW>(vec, grid, thr, lds, st, d_out, hist, meta, d_q, d_w, H, \
                                     HP, D, d_keys, d_key_scales, key_stride, n, scale, ng, qr); \
    } while (0)
    if (key_fmt == DSV4_GPU_KV_FP8) DSV4_ISCORE(DSV4_GPU_KV_FP8, 4);
    else if (key_fmt == DSV4_GPU_KV_BF16) DSV4_ISCORE(DSV4_GPU_KV_BF16, 4);
    else if (mw8) DSV4_ISCORE(DSV4_GPU_KV_F32, 8);
    else DSV4_ISCORE(DSV4_GPU_KV_F32, 4);
#undef DSV4_ISCORE
    HIP_OK(hipGetLastError(), "indexer score launch");
    return 0;
}

int dsv4_indexer_score_launch(float *d_out, const float *d_q, const float *d_w,
                              int H, int D, const void *d_keys,
                              const float *d_key_scales, int key_fmt,
                              int key_stride, int n, float scale, void *scratch,
                              int with_hist, hipStream_t st)
{
    return dsv4_indexer_score_rope_launch(d_out, d_q, d_w, H, D, d_keys, d_key_scales, key_fmt,
                                          key_stride, n, scale, scratch, with_hist, nullptr,
                                          nullptr, 0, 0, 0, st);
}

int dsv4_topk_launch(int *d_idxs, const float *d_scores, int n, int k,
                     void *scratch, int hist_ready, hipStream_t st)
{
    if (k > n) k = n;
    if (k <= 0) return 0;
    if (k > TK_KMAX || n > TK_NMAX) {
        DSV4_ERR("topk: k %d of n %d exceeds the supported %d of %d", k, n,
                 TK_KMAX, TK_NMAX);
        return -1;
    }
    if (hist_ready && !dsv4_topk_takes_hist(n, k)) {
        DSV4_ERR("topk: a level-1 histogram was built for n %d k %d", n, k);
        return -1;
    }
    if (n <= TS_NMAX) {
        hipLaunchKernelGGL(k_tk_small, dim3((n + TS_EPW - 1) / TS_EPW), dim3(256), 0, st,
                           d_idxs, d_scores, n, k);
        HIP_OK(hipGetLastError(), "topk (short) launch");
        return 0;
    }
    char *sb = (char *)scratch;
    uint32_t *hist = (uint32_t *)(sb + IX_HIST);
    uint32_t *meta = (uint32_t *)(sb + IX_META);
    unsigned long long *cand = (unsigned long long *)(sb + IX_CAND);
    unsigned long long *bsel = (unsigned long long *)(sb + IX_BSEL);
    uint32_t *bcnt = (uint32_t *)(sb + IX_BCNT);
    unsigned long long *blist = (unsigned long long *)(sb + IX_BLIST);
    const int G = (n + PT_ELEMS - 1) / PT_ELEMS;
    if (!hist_ready) {
        hipLaunchKernelGGL(k_tk_hist, dim3((n + 256 * TH_EPT - 1) / (256 * TH_EPT)), dim3(256), 0,
                           st, hist, meta, d_scores, n);
        HIP_OK(hipGetLastError(), "topk histogram launch");
    }
    hipLaunchKernelGGL(k_tk_part, dim3(G), dim3(PT_THREADS), 0, st, cand, bsel, meta, bcnt,
                       blist, hist, d_scores, n, k);
    HIP_OK(hipGetLastError(), "topk partition launch");
    /* the direct form places up to k - 1 + RF_LIST elements, the refinement
     * form k */
    hipLaunchKernelGGL(k_tk_final, dim3((k + RF_LIST + RK_EPW - 1) / RK_EPW), dim3(FN_THREADS),
                       0, st, d_idxs, cand, bsel, meta, bcnt, blist, hist, d_scores, G, k);
    HIP_OK(hipGetLastError(), "topk final launch");
    return 0;
}

size_t dsv4_attn_scratch_bytes(int h, int d_qk, int d_v, int topk, int kv_fmt)
{
    int rowb;
    size_t lds;
    int sr = attn_split_rows(kv_fmt, d_qk, d_v, &rowb, &lds);
    if (sr <= 0) return 0;
    if (sr > AT_SR_MIN) sr = AT_SR_MIN;      /* any smaller topk may split this finely */
    const size_t nsplit = (size_t)(topk > 0 ? (topk + sr - 1) / sr : 1);
    return sizeof(float) * (size_t)h * nsplit * (2 + (size_t)d_v);
}

int dsv4_attn_block_launch(float *d_o, const float *d_q, const void *d_kv,
                           int kv_fmt, int kv_stride, int kv_rows,
                           const float *d_sink, const int *d_idxs, int h, int d_qk,
                           int d_v, int topk, float scale, void *scratch, int q_norm,
                           float q_eps, const float *rope_cs, const float *rope_sn,
                           int rope_pos, int rope_half, int rope_dim, hipStream_t st,
                           const Dsv4Rows *rows)
{
    const Dsv4Rows rw = rows ? *rows : Dsv4Rows{};
    if (rw.on && (rw.win <= 0 || rw.n_win < 0 || rw.n_win > rw.win || rw.n_win > topk ||
                  rw.pos < 0 || (rw.mode != 1 && rw.mode != 2))) {
        DSV4_ERR("sparse attn: bad row list (win %d n_win %d mode %d)", rw.win, rw.n_win,
                 rw.mode);
        return -1;
    }
    if (rope_dim < 0 || (rope_dim & 1) || rope_dim > d_qk || rope_dim > d_v ||
        rope_dim > 2 * RP_MAX || (rope_dim && ((d_v & 1) || !rope_cs || !rope_sn))) {
        DSV4_ERR("sparse attn: bad RoPE (dim %d, d_qk %d, d_v %d)", rope_dim, d_qk, d_v);
        return -1;
    }
    Dsv4Rope qrp, orp;
    if (rope_dim) {
        qrp.cs = orp.cs = rope_cs;
        qrp.sn = orp.sn = rope_sn;
        qrp.pos = orp.pos = rope_pos;
        qrp.half = orp.half = rope_half;
        qrp.rd = orp.rd = rope_dim;
        orp.inverse = 1;
    }
    const bool qx = q_norm || rope_dim;
    if (h <= 0 || d_qk <= 0 || d_v <= 0 || topk < 0 || kv_stride < d_qk ||
        kv_stride < d_v) {
        DSV4_ERR("sparse attn: bad shape h %d d_qk %d d_v %d stride %d",
                 h, d_qk, d_v, kv_stride);
        return -1;
    }
    if (kv_fmt != DSV4_GPU_KV_BF16 && kv_fmt != DSV4_GPU_KV_F32) {
        DSV4_ERR("sparse attn: KV format %d not supported", kv_fmt);
        return -1;
    }
    int rowb;
    size_t lds;
    const int sr = attn_split_rows(kv_fmt, d_qk, d_v, &rowb, &lds, h, topk);
    if (sr <= 0) {
        DSV4_ERR("sparse attn: d_qk %d / d_v %d too wide", d_qk, d_v);
        return -1;
    }
    const int nsplit = topk > 0 ? (topk + sr - 1) / sr : 1;
    if (nsplit > 1024) {
        DSV4_ERR("sparse attn: topk %d exceeds %d", topk, 1024 * sr);
        return -1;
    }
    const int es = kv_fmt == DSV4_GPU_KV_BF16 ? 2 : 4;
    const int dmax = d_qk > d_v ? d_qk : d_v;
    const int vec = ((dmax * es) % 16 == 0) && ((d_qk % 4) == 0) &&
                    (((size_t)kv_stride * es) % 16 == 0) && (((uintptr_t)d_kv & 15) == 0);
    float *pm = (float *)scratch;
    float *pl = pm + (size_t)h * nsplit;
    float *po = pl + (size_t)h * nsplit;
    dim3 grid(nsplit, (h + AT_HB - 1) / AT_HB);
    static bool lds_opted = false;
    if (!lds_opted) {
        const size_t cap = dsv4_lds_limit();
        (void)dsv4_lds_optin((const void *)k_attn_partial<DSV4_GPU_KV_BF16>, cap,
                             "sparse attention");
        (void)dsv4_lds_optin((const void *)k_attn_partial<DSV4_GPU_KV_F32>, cap,
                             "sparse attention");
        (void)dsv4_lds_optin((const void *)k_attn_mc, cap, "sparse attention");
        lds_opted = true;
    }
    /* the matrix-core form where the shape allows (DSV4_GPU_ATTN_MC=0 keeps
     * the VALU form) */
    const size_t mc_lds = attn_mc_lds(kv_fmt, h, d_qk, d_v, kv_stride);
    const char *mc_env = getenv("DSV4_GPU_ATTN_MC");
    if (mc_lds && !qx && !rw.on && topk > 0 && ((uintptr_t)d_kv & 15) == 0 &&
        !(mc_env && atoi(mc_env) == 0)) {
        const int ns = (topk + AM_SR - 1) / AM_SR;          /* <= nsplit: sr <= AM_SR */
        pl = pm + (size_t)h * ns;
        po = pl + (size_t)h * ns;
        hipLaunchKernelGGL(k_attn_mc, dim3(ns, h / 16), dim3(AM_THREADS), mc_lds, st, pm, pl, po,
                           d_q, (const uint16_t *)d_kv, kv_stride, d_idxs, kv_rows,
                           d_qk, d_v, topk, scale);
        HIP_OK(hipGetLastError(), "attn mc launch");
        hipLaunchKernelGGL(k_attn_combine, dim3(h, (d_v + CB_COLS - 1) / CB_COLS),
                           dim3(CB_COLS), 0, st, d_o, pm, pl, po, d_sink, ns, d_v, orp);
        HIP_OK(hipGetLastError(), "attn combine launch");
        return 0;
    }
    if (kv_fmt == DSV4_GPU_KV_BF16)
        hipLaunchKernelGGL((k_attn_partial<DSV4_GPU_KV_BF16>), grid, dim3(AT_THREADS), lds, st,
                           pm, pl, po, d_q, d_kv, kv_stride, d_idxs, kv_rows, h,
                           d_qk, d_v, topk, scale, sr, rowb, vec, q_norm, q_eps, qrp, rw);
    else
        hipLaunchKernelGGL((k_attn_partial<DSV4_GPU_KV_F32>), grid, dim3(AT_THREADS), lds, st,
                           pm, pl, po, d_q, d_kv, kv_stride, d_idxs, kv_rows, h,
                           d_qk, d_v, topk, scale, sr, rowb, vec, q_norm, q_eps, qrp, rw);
    HIP_OK(hipGetLastError(), "attn partial launch");
    hipLaunchKernelGGL(k_attn_combine, dim3(h, (d_v + CB_COLS - 1) / CB_COLS),
                       dim3(CB_COLS), 0, st, d_o, pm, pl, po, d_sink, nsplit, d_v, orp);
    HIP_OK(hipGetLastError(), "attn combine launch");
    return 0;
}

int dsv4_attn_launch(float *d_o, const float *d_q, const void *d_kv,
                     int kv_fmt, int kv_stride, int kv_rows,
                     const float *d_sink, const int *d_idxs, int h, int d_qk,
                     int d_v, int topk, float scale, void *scratch,
                     hipStream_t st)
{
    return dsv4_attn_block_launch(d_o, d_q, d_kv, kv_fmt, kv_stride, kv_rows, d_sink, d_idxs,
                                  h, d_qk, d_v, topk, scale, scratch, 0, 0.0f, nullptr,
                                  nullptr, 0, 0, 0, st);
}
