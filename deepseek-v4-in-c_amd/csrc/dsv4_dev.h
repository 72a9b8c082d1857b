/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_dev.h - device helpers shared by the gfx950 kernels.
 *
 * Decoders: the three numeric formats of dsv4_quant.h (E4M3FN weights, E8M0
 * scales, E2M1 nibbles) decoded exactly. E4M3 and E2M1 use gfx950's
 * hardware conversions (v_cvt_pk_f32_fp8 is OCP e4m3fn on gfx950;
 * v_cvt_scalef32_pk_f32_fp4 with scale 1.0); E8M0 is bit assembly. The
 * decoder gates dump these exact functions for all 256/256/16 codes and
 * compare them bit for bit with the reference decoders.
 *
 * Reductions: wave64 sums built from DPP moves in one fixed order, so every
 * result is the same bits on every run and for every launch shape.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DSV4_WAVE 64

/* ------------------------------------------------------------- decoders */

/* Four E4M3FN bytes of one dword -> four floats, element order = byte order.
 * Exact: every e4m3 value is representable in f32; 0x7F / 0xFF give NaN. */
__device__ __forceinline__ void dec_e4m3x4(uint32_t v, float *o)
{
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, true);
    o[0] = lo[0]; o[1] = lo[1]; o[2] = hi[0]; o[3] = hi[1];
}

__device__ __forceinline__ float dec_e4m3(uint8_t b)
{
    float o[4];
    dec_e4m3x4((uint32_t)b, o);
    return o[0];
}

/* E4M3FN byte b times the power of two s, as bf16 widened to f32: the
 * matrix-core FP8 form's decode (v_cvt_scalef32_pk_bf16_fp8), exact while
 * the product stays in bf16's range. */
__device__ __forceinline__ float dec_e4m3_bf16(uint8_t b, float s)
{
    typedef short v2s_ __attribute__((ext_vector_type(2)));
    const v2s_ p = __builtin_bit_cast(v2s_, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                                (uint32_t)b, s, false));
    return __uint_as_float((uint32_t)(uint16_t)p.x << 16);
}

/* 2^(b-127); b == 0 is the subnormal 2^-127, b == 255 is NaN
 * (dsv4_quant.h:74-88). */
__device__ __forceinline__ float dec_e8m0(uint32_t b)
{
    const uint32_t u = (b == 0xFFu) ? 0x7FC00000u
                     : (b == 0u)    ? 0x00400000u
                                    : (b << 23);
    return __uint_as_float(u);
}

/* The two E2M1 elements packed in byte `sel` of v: [0] = low nibble (the
 * even element), [1] = high nibble (dsv4_quant.h:155-164). */
template <int SEL>
__device__ __forceinline__ void dec_fp4x2(uint32_t v, float *o)
{
    const auto p = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, SEL);
    o[0] = p[0]; o[1] = p[1];
}

/* Eight E2M1 elements of one dword, in element order. */
__device__ __forceinline__ void dec_fp4x8(uint32_t v, float *o)
{
    dec_fp4x2<0>(v, o + 0);
    dec_fp4x2<1>(v, o + 2);
    dec_fp4x2<2>(v, o + 4);
    dec_fp4x2<3>(v, o + 6);
}

/* ------------------------------------------------------------- SwiGLU */

/* dsv4_swiglu for one element (dsv4_ops.c:60-78): up clamped to [-L, L],
 * gate clamped above only, silu(g) = g / (1 + expf(-g)). */
__device__ __forceinline__ float swiglu1(float g, float u, float limit)
{
    if (limit > 0.0f) {
        if (u > limit) u = limit;
        if (u < -limit) u = -limit;
        if (g > limit) g = limit;
        const float s = g / (1.0f + expf(-g));
        return s * u;
    }
    return (g / (1.0f + expf(-g))) * u;
}

/* ----------------------------------------------------------- reductions */

/* DPP control codes (GCN/CDNA "dpp_ctrl"). */
#define DPP_QUAD_XOR1   0xB1   /* quad_perm [1,0,3,2] */
#define DPP_QUAD_XOR2   0x4E   /* quad_perm [2,3,0,1] */
#define DPP_ROW_HMIRROR 0x141  /* lane i <- 7-i within 8  */
#define DPP_ROW_MIRROR  0x140  /* lane i <- 15-i within 16 */
#define DPP_ROW_BCAST15 0x142  /* row r <- lane 15 of row r-1 */
#define DPP_ROW_BCAST31 0x143  /* rows 2,3 <- lane 31 */

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

/* Sum over aligned segments of SEG lanes (SEG a power of two, 1..64). The
 * full segment sum lands in the segment's LAST lane (lane SEG-1 of it); other
 * lanes hold partial sums. The addition order is fixed by the steps below. */
template <int SEG>
__device__ __forceinline__ float seg_sum(float v)
{
    if (SEG >= 2)  v += dpp_f<DPP_QUAD_XOR1, 0xF>(v);
    if (SEG >= 4)  v += dpp_f<DPP_QUAD_XOR2, 0xF>(v);
    if (SEG >= 8)  v += dpp_f<DPP_ROW_HMIRROR, 0xF>(v);
    if (SEG >= 16) v += dpp_f<DPP_ROW_MIRROR, 0xF>(v);
    if (SEG >= 32) v += dpp_f<DPP_ROW_BCAST15, 0xA>(v);
    if (SEG >= 64) v += dpp_f<DPP_ROW_BCAST31, 0xC>(v);
    return v;
}

/* Runtime segment width (power of two). */
__device__ __forceinline__ float seg_sum_rt(float v, int seg)
{
    if (seg >= 2)  v += dpp_f<DPP_QUAD_XOR1, 0xF>(v);
    if (seg >= 4)  v += dpp_f<DPP_QUAD_XOR2, 0xF>(v);
    if (seg >= 8)  v += dpp_f<DPP_ROW_HMIRROR, 0xF>(v);
    if (seg >= 16) v += dpp_f<DPP_ROW_MIRROR, 0xF>(v);
    if (seg >= 32) v += dpp_f<DPP_ROW_BCAST15, 0xA>(v);
    if (seg >= 64) v += dpp_f<DPP_ROW_BCAST31, 0xC>(v);
    return v;
}

/* Whole-wave sum, broadcast to every lane (from lane 63). */
__device__ __forceinline__ float wave_sum(float v)
{
    v = seg_sum<64>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* Whole-wave max, broadcast to every lane. */
__device__ __forceinline__ float wave_max(float v)
{
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const void *p)
{
    return *reinterpret_cast<const u32x4 *>(p);
}

/* Streaming 16-byte load: the weights are read exactly once per call, so keep
 * them from displacing reused lines (x, scales) in the caches. */
__device__ __forceinline__ u32x4 ld16_stream(const void *p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

/* The same loads through a global-address-space pointer. Pointers read from
 * memory (an expert table) are generic to the compiler, which would emit
 * flat loads; those also count against lgkmcnt, so any LDS wait in the loop
 * would wait for every weight load in flight. */
#define DSV4_GLOBAL __attribute__((address_space(1)))

__device__ __forceinline__ u32x4 ldg16_stream(const void *p)
{
    return __builtin_nontemporal_load((const DSV4_GLOBAL u32x4 *)p);
}

__device__ __forceinline__ uint32_t ldg8(const uint8_t *p)
{
    return *(const DSV4_GLOBAL uint8_t *)p;
}

__device__ __forceinline__ f32x4 ldf4(const float *p)
{
    return *reinterpret_cast<const f32x4 *>(p);
}
