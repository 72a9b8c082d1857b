/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_head.hip - the decode loop's head on the device: greedy argmax over
 * the logits and the embedding-row gather.
 *
 * argmax is the reference's own scan (src/cli/dsv4_run.c:471-472):
 *   best = 0; for v in 1..n-1: if (logits[v] > logits[best]) best = v;
 * i.e. the first index of the maximum, NaNs never chosen except at index 0
 * (nothing compares greater than a NaN at best = 0, so it stays). On the
 * device every element becomes a 64-bit composite (order-preserving key of
 * the value << 32 | ~index, -0.0 folded into +0.0 since `>` treats them as
 * equal, NaN the smallest composite), and the maximum composite is the
 * reference's answer; two passes (per-workgroup maxima, then one workgroup)
 * keep it deterministic without atomics.
 *
 * embed_row is dsv4_embed_row (include/dsv4/dsv4.h:300-314): a BF16 row
 * widened exactly (the 16 bits are the top half of the float) or an f32 row
 * copied.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

#include <math.h>

namespace {

constexpr int AM_THREADS = 256;
constexpr int AM_GRID = 256;

__device__ __forceinline__ unsigned long long am_key(float v, int i)
{
    if (v != v) return 0ull;                          /* NaN: never the maximum */
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7FFFFFFFu) == 0u) u = 0u;              /* -0.0 == +0.0 */
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long t = __shfl_xor(v, o, 64);
        v = t > v ? t : v;
    }
    return v;
}

/* The maximum composite of a workgroup's threads, in every lane of wave 0. */
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v)
{
    __shared__ unsigned long long wm[AM_THREADS / 64];
    v = wave_max_u64(v);
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long m = wm[0];
#pragma unroll
    for (int w = 1; w < AM_THREADS / 64; w++) m = wm[w] > m ? wm[w] : m;
    return m;
}

__global__ void __launch_bounds__(AM_THREADS)
k_argmax_part(unsigned long long *__restrict__ part, const float *__restrict__ v, int n)
{
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * AM_THREADS + threadIdx.x; i < n; i += gridDim.x * AM_THREADS) {
        const unsigned long long k = am_key(v[i], i);
        best = k > best ? k : best;
    }
    best = block_max_u64(best);
    if (threadIdx.x == 0) part[blockIdx.x] = best;
}

__global__ void __launch_bounds__(AM_THREADS)
k_argmax_final(int *__restrict__ out, const unsigned long long *__restrict__ part, int g,
               const float *__restrict__ v)
{
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < g; i += AM_THREADS) best = part[i] > best ? part[i] : best;
    best = block_max_u64(best);
    if (threadIdx.x == 0) {
        const float v0 = v[0];
        /* a NaN at index 0 is never displaced; no maximum at all (every
         * element NaN) leaves the scan at 0 too */
        out[0] = (v0 != v0 || best == 0ull) ? 0 : (int)(0xFFFFFFFFu - (uint32_t)best);
    }
}

__global__ void __launch_bounds__(256)
k_embed_row(float *__restrict__ dst, const void *__restrict__ table, int wdt, long long row,
            int hidden)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < hidden; i += gridDim.x * 256) {
        if (wdt == DSV4_WBF16) {
            const uint16_t h = ((const uint16_t *)table)[(size_t)row * hidden + i];
            dst[i] = __uint_as_float((uint32_t)h << 16);
        } else {
            dst[i] = ((const float *)table)[(size_t)row * hidden + i];
        }
    }
}

} // namespace

size_t dsv4_argmax_scratch_bytes(void) { return AM_GRID * sizeof(unsigned long long); }

int dsv4_argmax_launch(int *d_out, const float *d_v, int n, void *scratch, hipStream_t st)
{
    if (n <= 0 || !d_out || !d_v || !scratch) {
        DSV4_ERR("argmax: bad arguments (n %d)", n);
        return -1;
    }
    const int g = (n + AM_THREADS - 1) / AM_THREADS < AM_GRID ? (n + AM_THREADS - 1) / AM_THREADS
                                                             : AM_GRID;
    unsigned long long *part = (unsigned long long *)scratch;
    hipLaunchKernelGGL(k_argmax_part, dim3(g), dim3(AM_THREADS), 0, st, part, d_v, n);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(AM_THREADS), 0, st, d_out, part, g, d_v);
    HIP_OK(hipGetLastError(), "argmax launch");
    return 0;
}

int dsv4_embed_row_launch(float *d_dst, const void *d_table, int wdt, long long row,
                          int hidden, hipStream_t st)
{
    if (!d_dst || !d_table || hidden <= 0 || row < 0 ||
        (wdt != DSV4_WBF16 && wdt != DSV4_WF32)) {
        DSV4_ERR("embed_row: bad arguments (wdt %d, row %lld, hidden %d)", wdt, row, hidden);
        return -1;
    }
    const int g = (hidden + 255) / 256 < 64 ? (hidden + 255) / 256 : 64;
    hipLaunchKernelGGL(k_embed_row, dim3(g), dim3(256), 0, st, d_dst, d_table, wdt, row,
                       hidden);
    HIP_OK(hipGetLastError(), "embed_row launch");
    return 0;
}
