/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_mla.hip - sparse-MLA decode on gfx950: the CSA indexer score, its
 * top-k, and softmax attention over the gathered latent-KV rows.
 *
 * INDEXER SCORE (dsv4_indexer.c:64-85), bit-exact. For each key row t and
 * head h: dot = fma-chain over c ascending of (double)q[h][c] *
 * (double)k[t][c]; then, in head order, `if (dot > 0) total += dot * w[h]`
 * with the multiply and the add rounded separately (this file is built with
 * -ffp-contract=off); out[t] = (float)total * scale, the scale computed by
 * the caller in float as the reference does. One thread per (t, h) runs the
 * 128-step fp64 chain; a thread per t then folds the heads in order. q and
 * the workgroup's key rows are staged in LDS as f32 (FP8 keys dequantised
 * exactly: e4m3(code) * row_scale) and widened exactly to double per use.
 *
 * TOP-K (dsv4_indexer.c:92-106), bit-exact: the k largest, ordered by score
 * descending, ties to the lower index. One workgroup of 1024 threads:
 *   - scores map to order-preserving 32-bit keys (-0.0 folded into +0.0,
 *     since the reference's `>` treats them as equal);
 *   - four 8-bit radix passes find T, the exact key of the k-th largest, and
 *     how many of the elements equal to T are needed;
 *   - a block scan over contiguous index ranges compacts the elements > T
 *     and the first needed elements == T in index order;
 *   - the > T elements are bitonic-sorted in LDS by (key desc, index asc);
 *     the == T ones already follow in index order.
 *
 * SPARSE ATTENTION (dsv4_attn.c:60-108): split over the selected rows and a
 * log-sum-exp combine. Partial pass: per (split of SR rows, group of HB
 * heads) a workgroup computes scores (fp32 dots, one wave per row), the
 * split's max m_s, e_j = expf(s_j - m_s), l_s = sum e_j and o_s = sum_j e_j *
 * v_j. Combine: M = max m_s, denom = sum l_s expf(m_s - M) (+ expf(sink - M)
 * when a sink is given: denominator only, not in the max),
 * o = (sum o_s expf(m_s - M)) * (float)(1/denom). Masked (-1) rows take no
 * part. Agrees with the reference within 1e-5 relative.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

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

/* Workgroup: P = TL * IS_CH key rows for all H heads, H * TL threads.
 * Thread (h, tl) runs the fma chains of head h for rows tl, tl + TL,
 * tl + 2 TL, tl + 3 TL: four independent chains keep the fp64 pipe busy.
 * The rows are widened to double once, into LDS; q too when it fits (QD),
 * else q stays f32 there and is widened per use (exact either way). */
constexpr int IS_CH = 4;                        /* chains per thread */

template <int KF, int QD>
__global__ void __launch_bounds__(256)
k_indexer_score(float *__restrict__ out, const float *__restrict__ q,
                const float *__restrict__ w, int H, int D,
                const void *__restrict__ keys, const float *__restrict__ ks,
                int key_stride, int n, float scale, int TL)
{
    extern __shared__ double lds_d[];
    const int P = TL * IS_CH;                   /* rows per workgroup */
    const int ld = D + 1;                       /* padded pitch */
    double *dots = lds_d;                       /* [P][H]   */
    double *kd = dots + (size_t)P * H;          /* [P][D+1] */
    double *qd = kd + (size_t)P * ld;           /* [H][D+1] (QD) */
    float *qf = (float *)qd;                    /* [H][D+1] (!QD) */

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int t0 = blockIdx.x * P;

    /* Staging issues every load of a batch before using any of them, so the
     * workgroup waits one memory latency per batch, not one per element. */
    constexpr int SB = 8;
    for (int i0 = 0; i0 < H * D; i0 += SB * nthr) {
        float v[SB];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = i0 + u * nthr + tid;
            v[u] = i < H * D ? q[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = i0 + u * nthr + tid;
            if (i < H * D) {
                const int hh = i / D, c = i - hh * D;
                if (QD) qd[hh * ld + c] = (double)v[u];
                else    qf[hh * ld + c] = v[u];
            }
        }
    }
    for (int i0 = 0; i0 < P * D; i0 += SB * nthr) {
        float v[SB];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = i0 + u * nthr + tid;
            const int p = i / D, c = i - p * D;
            const int t = t0 + p;
            v[u] = (i < P * D && t < n) ? key_at<KF>(keys, ks, (size_t)t, key_stride, c) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = i0 + u * nthr + tid;
            if (i < P * D) {
                const int p = i / D, c = i - p * D;
                kd[p * ld + c] = (double)v[u];
            }
        }
    }
    __syncthreads();

    if (tid < H * TL) {
        const int hh = tid % H, tl = tid / H;
        const double *k0 = kd + (size_t)(tl + 0 * TL) * ld;
        const double *k1 = kd + (size_t)(tl + 1 * TL) * ld;
        const double *k2 = kd + (size_t)(tl + 2 * TL) * ld;
        const double *k3 = kd + (size_t)(tl + 3 * TL) * ld;
        double d0 = 0.0, d1 = 0.0, d2 = 0.0, d3 = 0.0;
#pragma unroll 4
        for (int c = 0; c < D; c++) {
            const double qc = QD ? qd[hh * ld + c] : (double)qf[hh * ld + c];
            d0 = fma(qc, k0[c], d0);
            d1 = fma(qc, k1[c], d1);
            d2 = fma(qc, k2[c], d2);
            d3 = fma(qc, k3[c], d3);
        }
        dots[(tl + 0 * TL) * H + hh] = d0;
        dots[(tl + 1 * TL) * H + hh] = d1;
        dots[(tl + 2 * TL) * H + hh] = d2;
        dots[(tl + 3 * TL) * H + hh] = d3;
    }
    __syncthreads();

    for (int p = tid; p < P; p += nthr) {
        const int t = t0 + p;
        if (t < n) {
            double total = 0.0;
            for (int hh = 0; hh < H; hh++) {
                const double d = dots[p * H + hh];
                if (d > 0.0) {
                    const double prod = d * (double)w[hh];
                    total = total + prod;
                }
            }
            const float tf = (float)total;
            out[t] = tf * scale;
        }
    }
}

template <int KF>
void launch_score(bool qd, int grid, int thr, size_t lds, hipStream_t st,
                  float *d_out, const float *d_q, const float *d_w, int H, int D,
                  const void *d_keys, const float *d_key_scales, int key_stride,
                  int n, float scale, int TL)
{
    if (qd)
        hipLaunchKernelGGL((k_indexer_score<KF, 1>), dim3(grid), dim3(thr), lds, st,
                           d_out, d_q, d_w, H, D, d_keys, d_key_scales, key_stride,
                           n, scale, TL);
    else
        hipLaunchKernelGGL((k_indexer_score<KF, 0>), dim3(grid), dim3(thr), lds, st,
                           d_out, d_q, d_w, H, D, d_keys, d_key_scales, key_stride,
                           n, scale, TL);
}

/* --------------------------------------------------------------- top-k */

constexpr int TK_THREADS = 1024;
constexpr int TK_WAVES = TK_THREADS / 64;
constexpr int TK_KMAX = 4096;

__device__ __forceinline__ uint32_t fkey(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) == 0u) u = 0u;        /* -0.0 ties with +0.0 */
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long lanemask_lt(int lane)
{
    return lane ? (~0ull >> (64 - lane)) : 0ull;
}

/* Histogram bump for one key per lane (want = this lane's key counts). A few
 * rounds give the leading lane's digit a single aggregated add -- the top
 * digits of similar scores coincide and would otherwise serialise on one
 * LDS bank -- and whatever is left is added lane by lane. */
__device__ __forceinline__ void hist_add(uint32_t *hist, bool want, uint32_t d,
                                         int lane)
{
    bool todo = want;
#pragma unroll
    for (int it = 0; it < 3; ++it) {
        const unsigned long long pend = __ballot(todo);
        if (pend == 0ull) return;
        const int leader = __ffsll((long long)pend) - 1;
        const uint32_t dl = (uint32_t)__builtin_amdgcn_readlane((int)d, leader);
        const bool mine = todo && d == dl;
        const unsigned long long same = __ballot(mine);
        if (lane == leader) atomicAdd(&hist[dl], (uint32_t)__popcll(same));
        if (mine) todo = false;
    }
    if (todo) atomicAdd(&hist[d], 1u);
}

/* Top-k for n <= TK_THREADS * KPT: thread t holds the keys of elements
 * t, t + 1024, ... in registers (slot m = element / 1024). */
template <int KPT>
__global__ void __launch_bounds__(TK_THREADS)
k_topk(int *__restrict__ idxs, const float *__restrict__ scores, int n, int k)
{
    __shared__ uint32_t hist[256];
    __shared__ uint32_t cnt[2][KPT][TK_WAVES];      /* per (slot, wave) counts */
    __shared__ uint32_t sh_prefix, sh_krem;
    __shared__ unsigned long long sel[TK_KMAX];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;

    uint32_t key[KPT];
#pragma unroll
    for (int m = 0; m < KPT; m++) {
        const int i = m * TK_THREADS + tid;
        key[m] = i < n ? fkey(scores[i]) : 0u;
    }

    /* ---- radix select: T = key of the k-th largest, krem = how many of
     *      the elements equal to T are taken ---- */
    uint32_t prefix = 0u, mask = 0u, krem = (uint32_t)k;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < KPT; m++) {
            const int i = m * TK_THREADS + tid;
            const bool want = i < n && (key[m] & mask) == prefix;
            hist_add(hist, want, (key[m] >> shift) & 255u, lane);
        }
        __syncthreads();
        if (tid < 64) {
            uint32_t c4[4], sum = 0u;
#pragma unroll
            for (int q = 0; q < 4; q++) { c4[q] = hist[255 - (lane * 4 + q)]; sum += c4[q]; }
            uint32_t inc = sum;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(inc, o, 64);
                if (lane >= o) inc += t;
            }
            const uint32_t exc = inc - sum;
            if (exc < krem && inc >= krem) {
                uint32_t run = exc;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (run + c4[q] >= krem) {
                        const uint32_t digit = 255u - (uint32_t)(lane * 4 + q);
                        sh_prefix = prefix | (digit << shift);
                        sh_krem = krem - run;
                        break;
                    }
                    run += c4[q];
                }
            }
        }
        __syncthreads();
        prefix = sh_prefix;
        krem = sh_krem;
        mask |= 255u << shift;
    }
    const uint32_t T = prefix;
    const uint32_t need_eq = krem;                 /* >= 1 */
    const uint32_t c_gt = (uint32_t)k - need_eq;

    /* ---- compaction in index order: element index order is (slot, wave,
     *      lane), so per-(slot, wave) counts scanned in that order give each
     *      element its position ---- */
    unsigned long long mgt[KPT], meq[KPT];
#pragma unroll
    for (int m = 0; m < KPT; m++) {
        const int i = m * TK_THREADS + tid;
        mgt[m] = __ballot(i < n && key[m] > T);
        meq[m] = __ballot(i < n && key[m] == T);
        if (lane == 0) {
            cnt[0][m][wid] = (uint32_t)__popcll(mgt[m]);
            cnt[1][m][wid] = (uint32_t)__popcll(meq[m]);
        }
    }
    __syncthreads();
    if (wid < 2) {                                  /* wave 0: gt, wave 1: eq */
        uint32_t *c = &cnt[wid][0][0];
        constexpr int NE = KPT * TK_WAVES;          /* entries, slot-major */
        constexpr int PER = (NE + 63) / 64;
        uint32_t v[PER], sum = 0u;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = lane * PER + q;
            v[q] = e < NE ? c[e] : 0u;
            sum += v[q];
        }
        uint32_t inc = sum;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(inc, o, 64);
            if (lane >= o) inc += t;
        }
        uint32_t run = inc - sum;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = lane * PER + q;
            if (e < NE) c[e] = run;
            run += v[q];
        }
    }
    __syncthreads();
    const unsigned long long lt = lanemask_lt(lane);
#pragma unroll
    for (int m = 0; m < KPT; m++) {
        const int i = m * TK_THREADS + tid;
        if ((mgt[m] >> lane) & 1ull) {
            const uint32_t pos = cnt[0][m][wid] + (uint32_t)__popcll(mgt[m] & lt);
            if (pos < (uint32_t)TK_KMAX)
                sel[pos] = ((unsigned long long)key[m] << 32)
                         | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
        } else if ((meq[m] >> lane) & 1ull) {
            const uint32_t pos = cnt[1][m][wid] + (uint32_t)__popcll(meq[m] & lt);
            if (pos < need_eq) idxs[c_gt + pos] = i;
        }
    }
    uint32_t p2 = 1u;
    while (p2 < c_gt) p2 <<= 1;
    for (uint32_t i = c_gt + tid; i < p2; i += TK_THREADS) sel[i] = 0ull;
    __syncthreads();

    /* ---- bitonic sort of sel[0, p2), descending (key desc, index asc) ---- */
    if (p2 <= 2u * TK_THREADS) {
        /* Thread t owns elements a = 128*wave + lane and b = a + 64 of its
         * wave's 128-element block: strides < 64 are lane shuffles, stride
         * 64 is a register swap, strides >= 128 go through LDS. */
        const uint32_t ea = 128u * wid + lane, eb = ea + 64u;
        const bool act = ea < p2;
        unsigned long long a = act ? sel[ea] : 0ull;
        unsigned long long b = (eb < p2) ? sel[eb] : 0ull;
        for (uint32_t size = 2; size <= p2; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                if (stride >= 128) {
                    if (act) sel[ea] = a;
                    if (eb < p2) sel[eb] = b;
                    __syncthreads();
                    for (uint32_t t = tid; t < p2 / 2; t += TK_THREADS) {
                        const uint32_t lo = 2 * t - (t & (stride - 1));
                        const uint32_t hi = lo + stride;
                        const bool desc = ((lo & size) == 0);
                        const unsigned long long x = sel[lo], y = sel[hi];
                        if (desc ? (x < y) : (x > y)) { sel[lo] = y; sel[hi] = x; }
                    }
                    __syncthreads();
                    a = act ? sel[ea] : 0ull;
                    b = (eb < p2) ? sel[eb] : 0ull;
                } else if (stride == 64) {
                    const bool desc = ((ea & size) == 0);
                    if (desc ? (a < b) : (a > b)) { const unsigned long long t = a; a = b; b = t; }
                } else {
                    /* partner = element ^ stride, same register, lane ^ stride */
                    const unsigned long long pa =
                        ((unsigned long long)(uint32_t)__shfl_xor((int)(a >> 32), (int)stride, 64) << 32)
                        | (uint32_t)__shfl_xor((int)(uint32_t)a, (int)stride, 64);
                    const unsigned long long pb =
                        ((unsigned long long)(uint32_t)__shfl_xor((int)(b >> 32), (int)stride, 64) << 32)
                        | (uint32_t)__shfl_xor((int)(uint32_t)b, (int)stride, 64);
                    const bool lower = (lane & stride) == 0;
                    {
                        const uint32_t lo = lower ? ea : (ea ^ stride);
                        const bool desc = ((lo & size) == 0);
                        /* the lower element keeps the larger when descending */
                        const bool keep_big = (lower == desc);
                        a = keep_big ? (a > pa ? a : pa) : (a < pa ? a : pa);
                    }
                    {
                        const uint32_t lo = lower ? eb : (eb ^ stride);
                        const bool desc = ((lo & size) == 0);
                        const bool keep_big = (lower == desc);
                        b = keep_big ? (b > pb ? b : pb) : (b < pb ? b : pb);
                    }
                }
            }
        }
        if (act) sel[ea] = a;
        if (eb < p2) sel[eb] = b;
        __syncthreads();
    } else {
        for (uint32_t size = 2; size <= p2; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t t = tid; t < p2 / 2; t += TK_THREADS) {
                    const uint32_t lo = 2 * t - (t & (stride - 1));
                    const uint32_t hi = lo + stride;
                    const bool desc = ((lo & size) == 0);
                    const unsigned long long x = sel[lo], y = sel[hi];
                    if (desc ? (x < y) : (x > y)) { sel[lo] = y; sel[hi] = x; }
                }
                __syncthreads();
            }
        }
    }
    for (uint32_t i = tid; i < c_gt; i += TK_THREADS)
        idxs[i] = (int)(0xFFFFFFFFu - (uint32_t)(sel[i] & 0xFFFFFFFFull));
}

/* Any n: the same selection reading the scores from global memory on every
 * pass (coalesced), compaction by slot with a count array in dynamic LDS. */
__global__ void __launch_bounds__(TK_THREADS)
k_topk_big(int *__restrict__ idxs, const float *__restrict__ scores, int n, int k)
{
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sh_prefix, sh_krem, sh_base[2];
    __shared__ uint32_t wcnt[2][TK_WAVES];
    __shared__ unsigned long long sel[TK_KMAX];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int slots = (n + TK_THREADS - 1) / TK_THREADS;

    uint32_t prefix = 0u, mask = 0u, krem = (uint32_t)k;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
        for (int m = 0; m < slots; m++) {
            const int i = m * TK_THREADS + tid;
            const uint32_t key = i < n ? fkey(scores[i]) : 0u;
            const bool want = i < n && (key & mask) == prefix;
            hist_add(hist, want, (key >> shift) & 255u, lane);
        }
        __syncthreads();
        if (tid < 64) {
            uint32_t c4[4], sum = 0u;
            for (int q = 0; q < 4; q++) { c4[q] = hist[255 - (lane * 4 + q)]; sum += c4[q]; }
            uint32_t inc = sum;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(inc, o, 64);
                if (lane >= o) inc += t;
            }
            const uint32_t exc = inc - sum;
            if (exc < krem && inc >= krem) {
                uint32_t run = exc;
                for (int q = 0; q < 4; q++) {
                    if (run + c4[q] >= krem) {
                        sh_prefix = prefix | ((255u - (uint32_t)(lane * 4 + q)) << shift);
                        sh_krem = krem - run;
                        break;
                    }
                    run += c4[q];
                }
            }
        }
        __syncthreads();
        prefix = sh_prefix;
        krem = sh_krem;
        mask |= 255u << shift;
    }
    const uint32_t T = prefix, need_eq = krem, c_gt = (uint32_t)k - need_eq;
    if (tid == 0) { sh_base[0] = 0u; sh_base[1] = 0u; }
    __syncthreads();
    const unsigned long long lt = lanemask_lt(lane);
    for (int m = 0; m < slots; m++) {
        const int i = m * TK_THREADS + tid;
        const uint32_t key = i < n ? fkey(scores[i]) : 0u;
        const unsigned long long g = __ballot(i < n && key > T);
        const unsigned long long e = __ballot(i < n && key == T);
        if (lane == 0) { wcnt[0][wid] = (uint32_t)__popcll(g); wcnt[1][wid] = (uint32_t)__popcll(e); }
        __syncthreads();
        uint32_t og = sh_base[0], oe = sh_base[1];
        for (int w = 0; w < wid; w++) { og += wcnt[0][w]; oe += wcnt[1][w]; }
        if ((g >> lane) & 1ull) {
            const uint32_t pos = og + (uint32_t)__popcll(g & lt);
            if (pos < (uint32_t)TK_KMAX)
                sel[pos] = ((unsigned long long)key << 32)
                         | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
        } else if ((e >> lane) & 1ull) {
            const uint32_t pos = oe + (uint32_t)__popcll(e & lt);
            if (pos < need_eq) idxs[c_gt + pos] = i;
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t sg = 0u, se = 0u;
            for (int w = 0; w < TK_WAVES; w++) { sg += wcnt[0][w]; se += wcnt[1][w]; }
            sh_base[0] += sg;
            sh_base[1] += se;
        }
        __syncthreads();
    }
    uint32_t p2 = 1u;
    while (p2 < c_gt) p2 <<= 1;
    for (uint32_t i = c_gt + tid; i < p2; i += TK_THREADS) sel[i] = 0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= p2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = tid; t < p2 / 2; t += TK_THREADS) {
                const uint32_t lo = 2 * t - (t & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const unsigned long long x = sel[lo], y = sel[hi];
                if (desc ? (x < y) : (x > y)) { sel[lo] = y; sel[hi] = x; }
            }
            __syncthreads();
        }
    }
    for (uint32_t i = tid; i < c_gt; i += TK_THREADS)
        idxs[i] = (int)(0xFFFFFFFFu - (uint32_t)(sel[i] & 0xFFFFFFFFull));
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
               int d_v, int topk, float scale, int SR, int rowb, int vec)
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

    if (tid < SR) {
        const int r = tid < nj ? idxs[j0 + tid] : -1;
        sidx[tid] = (r >= 0 && r < kv_rows) ? r : -1;            /* never a wild read */
    }
    /* Staging issues a whole batch of loads before storing any of them: one
     * memory latency per batch rather than per element. */
    constexpr int SB = 8;
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
    __syncthreads();

    /* stage the rows */
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
    }
    __syncthreads();

    /* scores: thread (hh, lt) takes rows lt, lt + 32, ... */
    {
        const int hh = tid >> 5, lt = tid & 31;
        const float *qr = qs + hh * ldq;
        for (int jj = lt; jj < SR; jj += 32) {
            const unsigned char *kr = kvs + (size_t)jj * rowb;
            float a0 = 0.0f, a1 = 0.0f;
            int c = 0;
            if (vec) {
                for (; c + 8 <= d_qk; c += 8) {
                    float kk[8];
                    row8<KVF>(kr + (size_t)c * ES, kk);
                    const f32x4 qa = *reinterpret_cast<const f32x4 *>(qr + c);
                    const f32x4 qb = *reinterpret_cast<const f32x4 *>(qr + c + 4);
                    a0 = fmaf(qa.x, kk[0], a0); a1 = fmaf(qa.y, kk[1], a1);
                    a0 = fmaf(qa.z, kk[2], a0); a1 = fmaf(qa.w, kk[3], a1);
                    a0 = fmaf(qb.x, kk[4], a0); a1 = fmaf(qb.y, kk[5], a1);
                    a0 = fmaf(qb.z, kk[6], a0); a1 = fmaf(qb.w, kk[7], a1);
                }
            }
            for (; c < d_qk; c++) a0 = fmaf(qr[c], row1<KVF>(kr, c), a0);
            const float sc = (a0 + a1) * scale;
            ps[jj * AT_HB + hh] = sidx[jj] >= 0 ? sc : -INFINITY;
        }
    }
    __syncthreads();

    /* split softmax: wave per head, lane per row */
    for (int hh = wid; hh < AT_HB; hh += AT_THREADS / 64) {
        const float sv = lane < SR ? ps[lane * AT_HB + hh] : -INFINITY;
        const float m = wave_max(sv);
        const float e = (m == -INFINITY || sv == -INFINITY) ? 0.0f : expf(sv - m);
        if (lane < SR) ps[lane * AT_HB + hh] = e;
        const float l = wave_sum(e);
        if (lane == 0 && hh < nh) {
            pm[(size_t)(h0 + hh) * nsplit + split] = m;
            pl[(size_t)(h0 + hh) * nsplit + split] = l;
        }
    }
    __syncthreads();

    /* values: thread per column pair, all heads of the group */
    for (int c = 2 * tid; c < d_v; c += 2 * AT_THREADS) {
        const bool two = c + 1 < d_v;
        float acc0[AT_HB], acc1[AT_HB];
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++) { acc0[hh] = 0.0f; acc1[hh] = 0.0f; }
        for (int jj = 0; jj < SR; jj++) {
            const unsigned char *kr = kvs + (size_t)jj * rowb;
            const float v0 = row1<KVF>(kr, c);
            const float v1 = two ? row1<KVF>(kr, c + 1) : 0.0f;
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
                dst[0] = acc0[hh];
                if (two) dst[1] = acc1[hh];
            }
        }
    }
}

__global__ void __launch_bounds__(AT_THREADS)
k_attn_combine(float *__restrict__ o, const float *__restrict__ pm,
               const float *__restrict__ pl, const float *__restrict__ po,
               const float *__restrict__ sink, int nsplit, int d_v)
{
    const int hh = blockIdx.x;
    __shared__ float fs[1024];
    __shared__ float sh_inv;
    const int tid = threadIdx.x;
    if (tid < 64) {
        float M = -INFINITY;
        for (int s = tid; s < nsplit; s += 64) M = fmaxf(M, pm[(size_t)hh * nsplit + s]);
        M = wave_max(M);
        for (int s = tid; s < nsplit; s += 64) {
            const float ms = pm[(size_t)hh * nsplit + s];
            fs[s] = (ms == -INFINITY) ? 0.0f : expf(ms - M);
        }
        if (tid == 0) {
            double denom = 0.0;
            for (int s = 0; s < nsplit; s++)
                denom += (double)(pl[(size_t)hh * nsplit + s] * fs[s]);
            if (sink) denom += (double)expf(sink[hh] - M);
            sh_inv = (float)(1.0 / denom);
        }
    }
    __syncthreads();
    const float inv = sh_inv;
    for (int c = tid; c < d_v; c += AT_THREADS) {
        float acc = 0.0f;
        int s = 0;
        for (; s + 8 <= nsplit; s += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = po[((size_t)hh * nsplit + s + u) * d_v + c];
#pragma unroll
            for (int u = 0; u < 8; u++) acc = fmaf(v[u], fs[s + u], acc);
        }
        for (; s < nsplit; s++)
            acc = fmaf(po[((size_t)hh * nsplit + s) * d_v + c], fs[s], acc);
        o[(size_t)hh * d_v + c] = acc * inv;
    }
}

/* Rows per split: the staged rows, q and the scores must fit the LDS a
 * workgroup may use. */
int attn_split_rows(int kv_fmt, int d_qk, int d_v, int *rowb_out, size_t *lds_out)
{
    const size_t cap = dsv4_lds_limit();
    const int es = kv_fmt == DSV4_GPU_KV_BF16 ? 2 : 4;
    const int dmax = d_qk > d_v ? d_qk : d_v;
    const int rowb = ((dmax * es + 15) / 16) * 16 + 16;          /* +16 B: bank skew */
    for (int sr = 64; sr >= 1; sr >>= 1) {
        const size_t lds = (size_t)AT_HB * (d_qk + 4) * 4 + (size_t)sr * rowb +
                           (size_t)sr * AT_HB * 4 + (size_t)sr * 4;
        if (lds <= cap) {
            *rowb_out = rowb;
            *lds_out = lds;
            return sr;
        }
    }
    return 0;
}

} // namespace

int dsv4_indexer_score_launch(float *d_out, const float *d_q, const float *d_w,
                              int H, int D, const void *d_keys,
                              const float *d_key_scales, int key_fmt,
                              int key_stride, int n, float scale,
                              hipStream_t st)
{
    if (H <= 0 || D <= 0 || n < 0 || key_stride < D || H > 256) {
        DSV4_ERR("indexer score: bad shape H %d D %d n %d stride %d",
                 H, D, n, key_stride);
        return -1;
    }
    if (key_fmt == DSV4_GPU_KV_FP8 && !d_key_scales) {
        DSV4_ERR("indexer score: FP8 keys need row scales");
        return -1;
    }
    if (n == 0) return 0;
    /* About 128 threads per workgroup; q widened in LDS when it fits. */
    int TL = 128 / H > 0 ? 128 / H : 1;
    size_t lds = 0;
    bool qd = true;
    for (;; TL = TL > 1 ? TL / 2 : 0) {
        if (TL == 0) {
            DSV4_ERR("indexer score: H %d x D %d does not fit in LDS", H, D);
            return -1;
        }
        const size_t P = (size_t)TL * IS_CH;
        const size_t base = 8 * (P * H + P * (D + 1));
        if (base + 8 * (size_t)H * (D + 1) <= 64 * 1024) { qd = true; lds = base + 8 * (size_t)H * (D + 1); break; }
        if (base + 4 * (size_t)H * (D + 1) <= 64 * 1024) { qd = false; lds = base + 4 * (size_t)H * (D + 1); break; }
    }
    const int P = TL * IS_CH;
    const int thr = ((H * TL + 63) / 64) * 64;
    const int grid = (n + P - 1) / P;
    switch (key_fmt) {
    case DSV4_GPU_KV_F32:
        launch_score<DSV4_GPU_KV_F32>(qd, grid, thr, lds, st, d_out, d_q, d_w, H, D,
                                      d_keys, d_key_scales, key_stride, n, scale, TL);
        break;
    case DSV4_GPU_KV_BF16:
        launch_score<DSV4_GPU_KV_BF16>(qd, grid, thr, lds, st, d_out, d_q, d_w, H, D,
                                       d_keys, d_key_scales, key_stride, n, scale, TL);
        break;
    case DSV4_GPU_KV_FP8:
        launch_score<DSV4_GPU_KV_FP8>(qd, grid, thr, lds, st, d_out, d_q, d_w, H, D,
                                      d_keys, d_key_scales, key_stride, n, scale, TL);
        break;
    default:
        DSV4_ERR("indexer score: unknown key format %d", key_fmt);
        return -1;
    }
    HIP_OK(hipGetLastError(), "indexer score launch");
    return 0;
}

int dsv4_topk_launch(int *d_idxs, const float *d_scores, int n, int k,
                     hipStream_t st)
{
    if (k > n) k = n;
    if (k <= 0) return 0;
    if (k > TK_KMAX) {
        DSV4_ERR("topk: k %d exceeds the supported %d", k, TK_KMAX);
        return -1;
    }
    if (n <= 8 * TK_THREADS)
        hipLaunchKernelGGL((k_topk<8>), dim3(1), dim3(TK_THREADS), 0, st, d_idxs,
                           d_scores, n, k);
    else if (n <= 32 * TK_THREADS)
        hipLaunchKernelGGL((k_topk<32>), dim3(1), dim3(TK_THREADS), 0, st, d_idxs,
                           d_scores, n, k);
    else
        hipLaunchKernelGGL(k_topk_big, dim3(1), dim3(TK_THREADS), 0, st, d_idxs,
                           d_scores, n, k);
    HIP_OK(hipGetLastError(), "topk launch");
    return 0;
}

size_t dsv4_attn_scratch_bytes(int h, int d_qk, int d_v, int topk, int kv_fmt)
{
    int rowb;
    size_t lds;
    const int sr = attn_split_rows(kv_fmt, d_qk, d_v, &rowb, &lds);
    if (sr <= 0) return 0;
    const size_t nsplit = (size_t)(topk > 0 ? (topk + sr - 1) / sr : 1);
    return sizeof(float) * (size_t)h * nsplit * (2 + (size_t)d_v);
}

int dsv4_attn_launch(float *d_o, const float *d_q, const void *d_kv,
                     int kv_fmt, int kv_stride, int kv_rows,
                     const float *d_sink, const int *d_idxs, int h, int d_qk,
                     int d_v, int topk, float scale, void *scratch,
                     hipStream_t st)
{
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
    const int sr = attn_split_rows(kv_fmt, d_qk, d_v, &rowb, &lds);
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
        const int cap = (int)dsv4_lds_limit();
        (void)hipFuncSetAttribute((const void *)k_attn_partial<DSV4_GPU_KV_BF16>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, cap);
        (void)hipFuncSetAttribute((const void *)k_attn_partial<DSV4_GPU_KV_F32>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, cap);
        (void)hipGetLastError();
        lds_opted = true;
    }
    if (kv_fmt == DSV4_GPU_KV_BF16)
        hipLaunchKernelGGL((k_attn_partial<DSV4_GPU_KV_BF16>), grid, dim3(AT_THREADS), lds, st,
                           pm, pl, po, d_q, d_kv, kv_stride, d_idxs, kv_rows, h,
                           d_qk, d_v, topk, scale, sr, rowb, vec);
    else
        hipLaunchKernelGGL((k_attn_partial<DSV4_GPU_KV_F32>), grid, dim3(AT_THREADS), lds, st,
                           pm, pl, po, d_q, d_kv, kv_stride, d_idxs, kv_rows, h,
                           d_qk, d_v, topk, scale, sr, rowb, vec);
    HIP_OK(hipGetLastError(), "attn partial launch");
    hipLaunchKernelGGL(k_attn_combine, dim3(h), dim3(AT_THREADS), 0, st, d_o,
                       pm, pl, po, d_sink, nsplit, d_v);
    HIP_OK(hipGetLastError(), "attn combine launch");
    return 0;
}
