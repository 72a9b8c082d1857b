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

template <int KF>
__global__ void __launch_bounds__(256)
k_indexer_score(float *__restrict__ out, const float *__restrict__ q,
                const float *__restrict__ w, int H, int D,
                const void *__restrict__ keys, const float *__restrict__ ks,
                int key_stride, int n, float scale, int P)
{
    extern __shared__ double lds_d[];
    const int ldq = D + 1;                      /* padded row pitch */
    double *dots = lds_d;                       /* [P][H]    */
    float *qs = (float *)(dots + (size_t)P * H);/* [H][D+1]  */
    float *kl = qs + (size_t)H * ldq;           /* [P][D+1]  */

    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * P;

    for (int i = tid; i < H * D; i += blockDim.x) {
        const int hh = i / D, c = i - hh * D;
        qs[hh * ldq + c] = q[i];
    }
    for (int i = tid; i < P * D; i += blockDim.x) {
        const int p = i / D, c = i - p * D;
        const int t = t0 + p;
        kl[p * ldq + c] = t < n ? key_at<KF>(keys, ks, (size_t)t, key_stride, c)
                                : 0.0f;
    }
    __syncthreads();

    if (tid < P * H) {
        const int p = tid / H, hh = tid - p * H;
        const float *qr = qs + hh * ldq;
        const float *kr = kl + p * ldq;
        double dot = 0.0;
        for (int c = 0; c < D; c++) dot = fma((double)qr[c], (double)kr[c], dot);
        dots[p * H + hh] = dot;
    }
    __syncthreads();

    if (tid < P) {
        const int t = t0 + tid;
        if (t < n) {
            double total = 0.0;
            for (int hh = 0; hh < H; hh++) {
                const double d = dots[tid * H + hh];
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

/* --------------------------------------------------------------- top-k */

constexpr int TK_THREADS = 1024;
constexpr int TK_KMAX = 4096;

__device__ __forceinline__ uint32_t fkey(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) == 0u) u = 0u;        /* -0.0 ties with +0.0 */
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* Block-wide exclusive scan of one value per thread (TK_THREADS threads);
 * returns the exclusive prefix, and the total in *tot. */
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *tot)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint32_t inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) wsum[wid] = inc;
    __syncthreads();
    if (wid == 0) {
        const int nw = TK_THREADS / 64;
        uint32_t s = lane < nw ? wsum[lane] : 0u;
        uint32_t si = s;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(si, o, 64);
            if (lane >= o) si += t;
        }
        if (lane < nw) wsum[lane] = si - s;      /* exclusive per wave */
        if (lane == nw - 1) wsum[TK_THREADS / 64] = si;
    }
    __syncthreads();
    const uint32_t r = wsum[wid] + inc - v;
    *tot = wsum[TK_THREADS / 64];
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(TK_THREADS)
k_topk(int *__restrict__ idxs, const float *__restrict__ scores, int n, int k)
{
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wsum[TK_THREADS / 64 + 1];
    __shared__ uint32_t sh_prefix, sh_krem;
    __shared__ unsigned long long sel[TK_KMAX];

    const int tid = threadIdx.x, lane = tid & 63;
    const int per = (n + TK_THREADS - 1) / TK_THREADS;
    const int base = tid * per;
    const int end = min(n, base + per);

    uint32_t prefix = 0u, mask = 0u;
    uint32_t krem = (uint32_t)k;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < 256; i += TK_THREADS) hist[i] = 0u;
        __syncthreads();
        for (int m = 0; m < per; m++) {
            const int i = base + m;
            bool want = false;
            uint32_t d = 0u;
            if (i < end) {
                const uint32_t key = fkey(scores[i]);
                want = (key & mask) == prefix;
                d = (key >> shift) & 255u;
            }
            const unsigned long long pend = __ballot(want);
            if (pend == 0ull) continue;
            const int leader = __ffsll((long long)pend) - 1;
            const uint32_t dl = (uint32_t)__shfl((int)d, leader, 64);
            const unsigned long long diff = __ballot(want && d != dl);
            if (diff == 0ull) {
                if (lane == leader) atomicAdd(&hist[dl], (uint32_t)__popcll(pend));
            } else if (want) {
                atomicAdd(&hist[d], 1u);
            }
        }
        __syncthreads();
        /* Wave 0 finds the digit holding the krem-th largest. */
        if (tid < 64) {
            uint32_t c4[4], s = 0u;
#pragma unroll
            for (int q = 0; q < 4; q++) { c4[q] = hist[255 - (lane * 4 + q)]; s += c4[q]; }
            uint32_t inc = s;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(inc, o, 64);
                if (lane >= o) inc += t;
            }
            const uint32_t exc = inc - s;
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
        __syncthreads();
    }
    const uint32_t T = prefix;
    const uint32_t need_eq = krem;                 /* >= 1 */
    const uint32_t c_gt = (uint32_t)k - need_eq;

    uint32_t ngt = 0u, neq = 0u;
    for (int i = base; i < end; i++) {
        const uint32_t key = fkey(scores[i]);
        ngt += key > T;
        neq += key == T;
    }
    uint32_t tot;
    uint32_t pgt = block_excl_scan(ngt, wsum, &tot);
    uint32_t peq = block_excl_scan(neq, wsum, &tot);

    for (int i = base; i < end; i++) {
        const uint32_t key = fkey(scores[i]);
        if (key > T) {
            if (pgt < (uint32_t)TK_KMAX)
                sel[pgt] = ((unsigned long long)key << 32)
                         | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
            pgt++;
        } else if (key == T) {
            if (peq < need_eq) idxs[c_gt + peq] = i;
            peq++;
        }
    }
    /* Pad the > T part to a power of two with entries that sort last. */
    uint32_t p2 = 1u;
    while (p2 < c_gt) p2 <<= 1;
    for (uint32_t i = c_gt + tid; i < p2; i += TK_THREADS) sel[i] = 0ull;
    __syncthreads();

    /* Bitonic sort, descending. */
    for (uint32_t size = 2; size <= p2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = tid; t < p2 / 2; t += TK_THREADS) {
                const uint32_t lo = 2 * t - (t & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const unsigned long long a = sel[lo], b = sel[hi];
                if (desc ? (a < b) : (a > b)) { sel[lo] = b; sel[hi] = a; }
            }
            __syncthreads();
        }
    }
    for (uint32_t i = tid; i < c_gt; i += TK_THREADS)
        idxs[i] = (int)(0xFFFFFFFFu - (uint32_t)(sel[i] & 0xFFFFFFFFull));
}

/* ----------------------------------------------------- sparse attention */

constexpr int AT_THREADS = 256;
constexpr int AT_HB = 8;       /* heads per workgroup        */
constexpr int AT_SR = 64;      /* selected rows per split    */

template <int KVF>
__device__ __forceinline__ float kv_at(const void *kv, size_t row, int stride, int c)
{
    if (KVF == DSV4_GPU_KV_BF16)
        return bf16_to_f32(((const uint16_t *)kv)[row * stride + c]);
    return ((const float *)kv)[row * stride + c];
}

template <int KVF>
__global__ void __launch_bounds__(AT_THREADS)
k_attn_partial(float *__restrict__ pm, float *__restrict__ pl,
               float *__restrict__ po, const float *__restrict__ q,
               const void *__restrict__ kv, int kv_stride,
               const int *__restrict__ idxs, int kv_rows, int h, int d_qk,
               int d_v, int topk, float scale)
{
    extern __shared__ float lds_f[];
    const int ldq = d_qk + 1;
    float *qs = lds_f;                               /* [HB][d_qk+1] */
    float *ps = qs + AT_HB * ldq;                     /* [HB][SR]     */
    __shared__ int sidx[AT_SR];

    const int split = blockIdx.x, hg = blockIdx.y;
    const int nsplit = gridDim.x;
    const int h0 = hg * AT_HB;
    const int nh = min(AT_HB, h - h0);
    const int j0 = split * AT_SR;
    const int nj = min(AT_SR, topk - j0);
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;

    for (int i = tid; i < AT_HB * d_qk; i += AT_THREADS) {
        const int hh = i / d_qk, c = i - hh * d_qk;
        qs[hh * ldq + c] = hh < nh ? q[(size_t)(h0 + hh) * d_qk + c] : 0.0f;
    }
    if (tid < AT_SR) {
        const int r = tid < nj ? idxs[j0 + tid] : -1;
        sidx[tid] = (r >= 0 && r < kv_rows) ? r : -1;   /* never a wild read */
    }
    __syncthreads();

    /* Scores: one wave per selected row. */
    for (int jj = wid; jj < AT_SR; jj += AT_THREADS / 64) {
        const int row = sidx[jj];
        float part[AT_HB];
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++) part[hh] = 0.0f;
        if (row >= 0) {
            for (int c = lane; c < d_qk; c += 64) {
                const float v = kv_at<KVF>(kv, (size_t)row, kv_stride, c);
#pragma unroll
                for (int hh = 0; hh < AT_HB; hh++)
                    part[hh] = fmaf(qs[hh * ldq + c], v, part[hh]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++) {
            const float s = wave_sum(part[hh]);
            if (lane == 0)
                ps[hh * AT_SR + jj] = row >= 0 ? s * scale : -INFINITY;
        }
    }
    __syncthreads();

    /* Per head: split max, exponentials, split sum. One wave per head. */
    for (int hh = wid; hh < AT_HB; hh += AT_THREADS / 64) {
        const float s = ps[hh * AT_SR + lane];       /* AT_SR == 64 */
        const float m = wave_max(s);
        const float e = (m == -INFINITY || s == -INFINITY) ? 0.0f : expf(s - m);
        ps[hh * AT_SR + lane] = e;
        const float l = wave_sum(e);
        if (lane == 0 && hh < nh) {
            pm[(size_t)(h0 + hh) * nsplit + split] = m;
            pl[(size_t)(h0 + hh) * nsplit + split] = l;
        }
    }
    __syncthreads();

    /* Weighted values: thread per column, all heads of the group. */
    for (int c = tid; c < d_v; c += AT_THREADS) {
        float acc[AT_HB];
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++) acc[hh] = 0.0f;
        for (int jj = 0; jj < nj; jj++) {
            const int row = sidx[jj];
            if (row < 0) continue;
            const float v = kv_at<KVF>(kv, (size_t)row, kv_stride, c);
#pragma unroll
            for (int hh = 0; hh < AT_HB; hh++)
                acc[hh] = fmaf(ps[hh * AT_SR + jj], v, acc[hh]);
        }
#pragma unroll
        for (int hh = 0; hh < AT_HB; hh++)
            if (hh < nh)
                po[((size_t)(h0 + hh) * nsplit + split) * d_v + c] = acc[hh];
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
    if (tid == 0) {
        float M = -INFINITY;
        for (int s = 0; s < nsplit; s++) M = fmaxf(M, pm[(size_t)hh * nsplit + s]);
        double denom = 0.0;
        for (int s = 0; s < nsplit; s++) {
            const float ms = pm[(size_t)hh * nsplit + s];
            const float f = (ms == -INFINITY) ? 0.0f : expf(ms - M);
            fs[s] = f;
            denom += (double)(pl[(size_t)hh * nsplit + s] * f);
        }
        if (sink) denom += (double)expf(sink[hh] - M);
        sh_inv = (float)(1.0 / denom);
    }
    __syncthreads();
    const float inv = sh_inv;
    for (int c = tid; c < d_v; c += AT_THREADS) {
        float acc = 0.0f;
        for (int s = 0; s < nsplit; s++)
            acc = fmaf(po[((size_t)hh * nsplit + s) * d_v + c], fs[s], acc);
        o[(size_t)hh * d_v + c] = acc * inv;
    }
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
    const int P = 256 / H;
    const size_t lds = sizeof(double) * (size_t)P * H
                     + sizeof(float) * (size_t)(H + P) * (D + 1);
    if (lds > 64 * 1024) {
        DSV4_ERR("indexer score: H %d x D %d needs %zu B of LDS", H, D, lds);
        return -1;
    }
    const int grid = (n + P - 1) / P;
    switch (key_fmt) {
    case DSV4_GPU_KV_F32:
        hipLaunchKernelGGL((k_indexer_score<DSV4_GPU_KV_F32>), dim3(grid), dim3(256), lds, st,
                           d_out, d_q, d_w, H, D, d_keys, d_key_scales, key_stride, n, scale, P);
        break;
    case DSV4_GPU_KV_BF16:
        hipLaunchKernelGGL((k_indexer_score<DSV4_GPU_KV_BF16>), dim3(grid), dim3(256), lds, st,
                           d_out, d_q, d_w, H, D, d_keys, d_key_scales, key_stride, n, scale, P);
        break;
    case DSV4_GPU_KV_FP8:
        hipLaunchKernelGGL((k_indexer_score<DSV4_GPU_KV_FP8>), dim3(grid), dim3(256), lds, st,
                           d_out, d_q, d_w, H, D, d_keys, d_key_scales, key_stride, n, scale, P);
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
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(TK_THREADS), 0, st, d_idxs,
                       d_scores, n, k);
    HIP_OK(hipGetLastError(), "topk launch");
    return 0;
}

size_t dsv4_attn_scratch_bytes(int h, int d_v, int topk)
{
    const size_t nsplit = (size_t)((topk + AT_SR - 1) / AT_SR);
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
    const int nsplit = topk > 0 ? (topk + AT_SR - 1) / AT_SR : 1;
    if (nsplit > 1024) {
        DSV4_ERR("sparse attn: topk %d exceeds %d", topk, 1024 * AT_SR);
        return -1;
    }
    float *pm = (float *)scratch;
    float *pl = pm + (size_t)h * nsplit;
    float *po = pl + (size_t)h * nsplit;
    const size_t lds = sizeof(float) * ((size_t)AT_HB * (d_qk + 1) + (size_t)AT_HB * AT_SR);
    if (lds > 64 * 1024) {
        DSV4_ERR("sparse attn: d_qk %d too large", d_qk);
        return -1;
    }
    dim3 grid(nsplit, (h + AT_HB - 1) / AT_HB);
    if (kv_fmt == DSV4_GPU_KV_BF16)
        hipLaunchKernelGGL((k_attn_partial<DSV4_GPU_KV_BF16>), grid, dim3(AT_THREADS), lds, st,
                           pm, pl, po, d_q, d_kv, kv_stride, d_idxs, kv_rows, h,
                           d_qk, d_v, topk, scale);
    else if (kv_fmt == DSV4_GPU_KV_F32)
        hipLaunchKernelGGL((k_attn_partial<DSV4_GPU_KV_F32>), grid, dim3(AT_THREADS), lds, st,
                           pm, pl, po, d_q, d_kv, kv_stride, d_idxs, kv_rows, h,
                           d_qk, d_v, topk, scale);
    else {
        DSV4_ERR("sparse attn: KV format %d not supported", kv_fmt);
        return -1;
    }
    HIP_OK(hipGetLastError(), "attn partial launch");
    hipLaunchKernelGGL(k_attn_combine, dim3(h), dim3(AT_THREADS), 0, st, d_o,
                       pm, pl, po, d_sink, nsplit, d_v);
    HIP_OK(hipGetLastError(), "attn combine launch");
    return 0;
}
