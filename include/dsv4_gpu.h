/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_gpu.h - MI355X (gfx950) decode backend for deepseek-v4-in-c, C ABI.
 *
 * A drop-in for the reference's GPU co-processor header
 * (include/dsv4/dsv4_cuda.h:65-99) and its CPU stub
 * (src/cuda/dsv4_cuda_stub.c): the same entry points under the dsv4_gpu_
 * prefix, the same argument meaning and the same error behaviour, plus the
 * three hot-path families the reference leaves on the CPU:
 *
 *   1. block-scaled FP8 e4m3 GEMV        (replaces k_mmq_fp8, dsv4_cuda.cu:93)
 *   2. fused MXFP4 routed-expert matvec  (dsv4_layer.c:199-206, :412-476)
 *   3. sparse-MLA indexer score, top-k and gather attention
 *                                         (dsv4_indexer.c:64-106,
 *                                          dsv4_attn.c:60-108)
 *
 * CONVENTIONS (as dsv4_cuda.h / dsv4_cuda.cu:16-24):
 *   - Plain C, plain pointers and sizes. Host-buffer entry points take and
 *     return host memory and are synchronous; the *_d entry points take
 *     device pointers and a hipStream_t passed as void* (NULL = the default
 *     stream) and are stream-ordered.
 *   - int 0 on success, -1 on a recoverable failure, with a message prefixed
 *     "dsv4_gpu:" on stderr. A contract violation (mmq on a matrix that is not
 *     resident) calls abort(), as dsv4_cuda_mmq does (dsv4_cuda.cu:390-394).
 *   - The caller owns every host buffer. The backend owns device copies made
 *     by upload calls until dsv4_gpu_shutdown. Matrices are keyed by their host
 *     weight pointer, which must stay stable (dsv4_cuda.cu:232-236).
 *   - Single-threaded: call from one host thread (the reference contract,
 *     dsv4_cuda.cu:243-249). Calls that overlap on one device race on the
 *     backend's staging and scratch buffers.
 *
 * Built with hipcc for gfx950 as libdsv4_gpu.so; a CPU-only build links
 * dsv4_gpu_stub.c instead, which defines every symbol below and reports no
 * device.
 */
#ifndef DSV4_GPU_H
#define DSV4_GPU_H

#include <stddef.h>
#include <stdint.h>

/* The operand types come from the reference's include/dsv4/dsv4.h. When that
 * header is not in the include path, a layout-identical copy of the three
 * pieces this ABI uses is declared here (dsv4.h:83, :92, :208-214,
 * :252-255), so the same binary serves both. */
#ifndef DSV4_H
#define DSV4_MAX_BATCH 64
enum { DSV4_WF32 = 0, DSV4_WBF16 = 1, DSV4_WFP8 = 2, DSV4_WFP4 = 3 };
typedef struct {
    const void *w;          /* packed weight bytes                     */
    const void *s;          /* block scales (E8M0 bytes, or fp32)      */
    int wdt;                /* DSV4_W*                                 */
    int rows, cols;         /* LOGICAL element dims                    */
    int blk_r, blk_c;       /* scale block: 128x128 (FP8), 1x32 (FP4)  */
} DSV4QMat;
typedef struct {
    DSV4QMat w1, w3;        /* FP4 [inter, hidden]                     */
    DSV4QMat w2;            /* FP4 [hidden, inter]                     */
} DSV4ExpertW;
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ======================================================== device bring-up */

/* 1 when built with HIP and a usable device is present; the stub returns 0.
 * Replaces dsv4_cuda_available (dsv4_cuda.h:65, dsv4_cuda.cu:251). */
int dsv4_gpu_available(void);

/* Make the calling thread block instead of spin while waiting on the device.
 * Must precede dsv4_gpu_init. Replaces dsv4_cuda_set_blocking_sync
 * (dsv4_cuda.cu:264). */
int dsv4_gpu_set_blocking_sync(void);

/* Bring up device 0; prints name, arch and free/total HBM. 0 / -1.
 * Replaces dsv4_cuda_init (dsv4_cuda.h:70, dsv4_cuda.cu:271). */
int dsv4_gpu_init(void);

/* Bytes of HBM still free (0 before init). Replaces dsv4_cuda_free_vram
 * (dsv4_cuda.h:97). */
size_t dsv4_gpu_free_vram(void);

/* Free every device copy, staging and scratch buffer; reset state.
 * Replaces dsv4_cuda_shutdown (dsv4_cuda.h:99, dsv4_cuda.cu:436). */
void dsv4_gpu_shutdown(void);

/* ================================================= FP8 / FP4 dense matrices */

/* Copy one FP8 matrix (E8M0 block scales, the reference's format), one
 * MXFP4 matrix (e2m1 nibbles, E8M0 scale per blk_r x blk_c block; cols a
 * multiple of 32 up to 16384, blk_c a multiple of 32) or one BF16 matrix
 * (m->s unused; cols a multiple of 8 up to 16384) into HBM, keyed by m->w.
 * 0 ok; -1 recoverable (another format or shape, no room with 256 MiB of
 * headroom, copy failed) -- the matrix then stays on the CPU. Idempotent per
 * key. Replaces dsv4_cuda_upload (dsv4_cuda.h:80, dsv4_cuda.cu:307), which
 * took FP8 only; FP4 and BF16 residency let the reference's dispatch
 * (dsv4_matmul.c:525-546) run the experts' matrices, the router gate and the
 * LM head on the device too. */
int dsv4_gpu_upload(const DSV4QMat *m);

/* The same for an FP8 matrix whose block scales are fp32 (m->s is a float
 * grid ceil(rows/blk_r) x ceil(cols/blk_c)). No reference counterpart: the
 * benchmark configurations specify fp32 block scales. */
int dsv4_gpu_upload_f32s(const DSV4QMat *m);

/* Is m resident? True for an uploaded matrix and for a ROW-RANGE VIEW of one:
 * m->w points inside a resident weight block at a whole-row offset, with the
 * same cols/wdt/blocking and m->s at the matching scale-grid row (how
 * attention() slices wo_a per group, dsv4_layer.c:321-334). A view then runs
 * only its own rows -- the reference keyed only exact pointers, so group 0's
 * slice ran the whole wo_a (dsv4_cuda.cu:296-305). Replaces dsv4_cuda_has
 * (dsv4_cuda.h:83). */
int dsv4_gpu_has(const DSV4QMat *m);

/* y[rows] = dequant(m) . x[cols], host buffers, synchronous. abort() if m is
 * not resident. FP8 as dsv4_matmul_fp8, FP4 as dsv4_matmul_fp4, BF16 as
 * dsv4_matmul_bf16 (dsv4_matmul.c:275-345). Replaces dsv4_cuda_mmq
 * (dsv4_cuda.h:88, dsv4_cuda.cu:387). */
void dsv4_gpu_mmq(float *y, const float *x, const DSV4QMat *m);

/* y[nt][rows] for x[nt][cols]: one pass over the weights for the batch. Per
 * (row, token) bit-identical to dsv4_gpu_mmq; nt == 1 forwards to it;
 * nt > DSV4_MAX_BATCH aborts. Replaces dsv4_cuda_mmq_n (dsv4_cuda.h:94,
 * dsv4_cuda.cu:410). */
void dsv4_gpu_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt);

/* Device-resident GEMV on raw device buffers, stream-ordered:
 * d_y[rows] = dequant(d_w, d_s) . d_x[cols], 128x128 blocks. scale_fmt 0 =
 * E8M0 bytes, 1 = fp32. What dsv4_gpu_mmq runs after staging. d_x and d_w
 * must be 16-byte aligned wherever cols is a multiple of 16 (the chunked
 * kernels read 16-byte pieces); an unaligned pointer is refused (-1), never
 * sent to other arithmetic, so a matrix's bits do not depend on where the
 * caller's buffers lie. The arithmetic follows from the scale format and the
 * shape alone (and the process's DSV4_GPU_FP8_MX). */
int dsv4_gpu_fp8_gemv_d(float *d_y, const float *d_x, const uint8_t *d_w,
                        const void *d_s, int scale_fmt, int rows, int cols,
                        void *stream);

/* The batched form (prefill, the k_mmq_fp8_n contract of dsv4_cuda.cu:161-
 * 230): d_y[nt][rows] for d_x[nt][cols], each (row, token) bit-identical to
 * dsv4_gpu_fp8_gemv_d on that token. nt <= DSV4_MAX_BATCH. What
 * dsv4_gpu_mmq_n runs after staging. The same alignment rule; its scratch
 * (x's term planes or part sums) is the library's, grown on demand. */
int dsv4_gpu_fp8_gemv_n_d(float *d_y, const float *d_x, const uint8_t *d_w,
                          const void *d_s, int scale_fmt, int rows, int cols, int nt,
                          void *stream);

/* The MXFP4 GEMV on raw device buffers, stream-ordered: d_y[rows] =
 * dsv4_matmul_fp4 (dsv4_matmul.c:320-345) of d_w (e2m1 nibbles [rows][cols/2],
 * 16-byte aligned) with E8M0 scales d_s [ceil(rows/blk_r)][ceil(cols/blk_c)]
 * and d_x (16-byte aligned). What dsv4_gpu_mmq runs for a resident FP4 matrix.
 * 0 / -1 (shape not taken: cols a multiple of 32 up to 16384, blk_c a
 * multiple of 32). */
int dsv4_gpu_fp4_gemv_d(float *d_y, const float *d_x, const uint8_t *d_w,
                        const uint8_t *d_s, int rows, int cols, int blk_r, int blk_c,
                        void *stream);

/* The BF16 GEMV on raw device buffers, stream-ordered: d_y[rows] =
 * dsv4_matmul_bf16 (dsv4_matmul.c:275-291) of d_w (bf16 [rows][cols]) and
 * d_x, both 16-byte aligned. What dsv4_gpu_mmq runs for a resident BF16
 * matrix. 0 / -1 (cols not a multiple of 8 up to 16384). */
int dsv4_gpu_bf16_gemv_d(float *d_y, const float *d_x, const uint16_t *d_w, int rows,
                         int cols, void *stream);

/* The batched FP4 and BF16 forms (prefill: the weights are read once for the
 * whole batch, as dsv4_mmq_n does for every format, dsv4_matmul.c:560-591):
 * d_y[nt][rows] for d_x[nt][cols], each (row, token) bit-identical to the
 * single-token call above on that token. nt <= DSV4_MAX_BATCH. What
 * dsv4_gpu_mmq_n runs after staging for a resident FP4 / BF16 matrix. */
int dsv4_gpu_fp4_gemv_n_d(float *d_y, const float *d_x, const uint8_t *d_w,
                          const uint8_t *d_s, int rows, int cols, int blk_r, int blk_c, int nt,
                          void *stream);
int dsv4_gpu_bf16_gemv_n_d(float *d_y, const float *d_x, const uint16_t *d_w, int rows,
                           int cols, int nt, void *stream);

/* ================================================================ the head */

/* The decode loop's head in one call (dsv4_run.c:467-472): logits =
 * head . x with head a resident matrix (BF16 as the reference's, or FP8/FP4),
 * then the greedy argmax over them -- the first index of the maximum, as the
 * reference's scan `if (logits[v] > logits[best]) best = v` gives it (a NaN
 * is never chosen unless it sits at index 0). x host f32[head->cols].
 * Returns the token id, or -1 (head not resident, launch failure). Only the
 * id crosses back to the host, not the vocab-wide logits. No reference
 * counterpart (the reference runs the head on the CPU). */
int dsv4_gpu_head_argmax(const float *x, const DSV4QMat *head);

/* The same argmax on a device vector, stream-ordered: d_out[0] = argmax of
 * d_v[n]. Uses library scratch (calls on one device do not overlap). 0 / -1.
 * No reference counterpart. */
int dsv4_gpu_argmax_d(int *d_out, const float *d_v, int n, void *stream);

/* dsv4_embed_row (include/dsv4/dsv4.h:300-314) on device buffers: d_dst[hidden]
 * = row `row` of the device table d_table (DSV4_WBF16, widened exactly, or
 * DSV4_WF32), stream-ordered. 0 / -1. */
int dsv4_gpu_embed_row_d(float *d_dst, const void *d_table, int wdt, long long row,
                         int hidden, void *stream);

/* ============================================ a checkpoint straight into HBM
 * The reference streams its checkpoint through host memory (a pinned trunk,
 * an NVMe expert cache: src/io/dsv4_st.c, src/io/dsv4_trunk.c,
 * src/cache/dsv4_cache.c). On an MI355X the whole Flash checkpoint fits in
 * HBM, so these calls read the safetensors shards (the container of
 * src/io/dsv4_st.c:377-537, the same dtype table and consistency checks) into
 * device memory once, through pinned staging, with no host copy of a matrix.
 * What they load is resident under its DEVICE address: the DSV4QMat /
 * DSV4ExpertW they fill carry device pointers, which the caller's dispatch
 * passes back to dsv4_gpu_has / dsv4_gpu_mmq (and slices into row-range
 * views, as attention() does with wo_a); the host must never dereference
 * them. Freed by dsv4_gpu_shutdown. No counterpart in the reference. */
typedef struct dsv4_gpu_ckpt dsv4_gpu_ckpt;

/* Index every *.safetensors file of dir (initialising the device if
 * needed). NULL on failure, with a message. */
dsv4_gpu_ckpt *dsv4_gpu_ckpt_open(const char *dir);
void dsv4_gpu_ckpt_close(dsv4_gpu_ckpt *c);
/* 1 when the checkpoint holds a tensor of that name. */
int dsv4_gpu_ckpt_has(const dsv4_gpu_ckpt *c, const char *name);

/* The matrix <base>.weight (+ <base>.scale) in the binder's stored form
 * (src/model/dsv4_bind.c:86-131): DSV4_WFP8 F8_E4M3 [rows][cols] with E8M0
 * 128x128 scales, DSV4_WFP4 packed I8 [rows][cols/2] with E8M0 1x32 scales,
 * DSV4_WBF16 [rows][cols]. *out receives the resident matrix. 0 / -1 (absent,
 * stored otherwise, no room). */
int dsv4_gpu_ckpt_load_qmat(dsv4_gpu_ckpt *c, const char *base, int wdt, int rows,
                            int cols, DSV4QMat *out);

/* Routed expert (layer, expert): layers.L.ffn.experts.E.w{1,3,2} (FP4, w1/w3
 * [inter][hidden], w2 [hidden][inter]) into one HBM block, registered for
 * dsv4_gpu_moe_fp4[_d] as dsv4_gpu_upload_expert does and its three
 * matrices resident. *out (may be NULL) receives them. 0 / -1. */
int dsv4_gpu_ckpt_load_expert(dsv4_gpu_ckpt *c, int layer, int expert, int hidden,
                              int inter, DSV4ExpertW *out);

/* The shapes a layer's tensors take (from DSV4Cfg, dsv4.h:94-156). */
typedef struct {
    int hidden, q_lora, n_heads, head_dim, o_groups, o_lora;
    int moe_inter, n_shared, n_experts;
    int index_n_heads, index_head_dim;
    int compress_ratio;        /* the layer's (0: no compressor)            */
    int has_indexer;           /* 1 where the layer has the CSA indexer     */
} dsv4_gpu_ckpt_dims;

/* Every matrix of one decoder layer, resident (device pointers). */
typedef struct {
    DSV4QMat wq_a, wq_b, wkv, wo_a, wo_b;                /* FP8            */
    DSV4QMat shared_w1, shared_w2, shared_w3;            /* FP8            */
    DSV4QMat gate;                                       /* BF16 router    */
    DSV4QMat comp_wkv, comp_wgate;                       /* BF16, ratio>0  */
    DSV4QMat idx_wq_b;                                   /* FP8, indexer   */
    DSV4QMat idx_wproj, idx_comp_wkv, idx_comp_wgate;    /* BF16, indexer  */
} dsv4_gpu_layer_mats;

/* Layer `layer` under the binder's names (src/model/dsv4_bind.c:152-243):
 * the attention's wq_a, wq_b, wkv, wo_a, wo_b, the shared expert, the
 * router gate, the compressor and indexer projections where the layer has
 * them, and all d->n_experts routed experts (experts[e] filled when experts
 * is not NULL). The layer's f32 vectors (norms, sinks, RoPE-free weights)
 * are not loaded: they are small host-side inputs. 0 / -1; on -1 nothing
 * this call loaded stays resident or registered (its HBM is freed), so the
 * same layer can be loaded again. */
int dsv4_gpu_ckpt_load_layer(dsv4_gpu_ckpt *c, const dsv4_gpu_ckpt_dims *d, int layer,
                             dsv4_gpu_layer_mats *out, DSV4ExpertW *experts);

typedef struct {
    int shards;
    long long tensors;                 /* indexed                              */
    long long matrices, experts;       /* loaded                               */
    long long bytes;                   /* read into HBM                        */
    double seconds;                    /* spent in the loads                   */
} dsv4_gpu_ckpt_stats;
int dsv4_gpu_ckpt_stats_get(const dsv4_gpu_ckpt *c, dsv4_gpu_ckpt_stats *out);

/* ========================================================== decoder gates */

/* Device decode of all 256 E4M3FN codes / 256 E8M0 codes / 16 E2M1 codes with
 * the exact decoders the kernels use, for bit-equality gates against
 * dsv4_quant.h:74-164. dump_e4m3 replaces dsv4_cuda_dump_e4m3
 * (dsv4_cuda.cu:460); the other two have no reference counterpart. */
int dsv4_gpu_dump_e4m3(float *host256);
int dsv4_gpu_dump_e8m0(float *host256);
int dsv4_gpu_dump_e2m1(float *host16);

/* Device decode of all 256 E4M3FN codes times the E8M0 scale 2^(e8m0 - 127)
 * the way the matrix-core FP8 form decodes them (into bf16 with the scale
 * folded in, widened back to f32), for a bit-equality gate against
 * dsv4_quant.h:74-130: exact while the product stays in bf16's range. No
 * reference counterpart. */
int dsv4_gpu_dump_e4m3_scaled(float *host256, int e8m0);

/* Device decode of every packed FP4 byte b = 0..255 into its two elements,
 * out[2b] = even (low nibble), out[2b+1] = odd (high nibble), the order
 * dsv4_fp4_at defines (dsv4_quant.h:155-164). No reference counterpart. */
int dsv4_gpu_dump_fp4_bytes(float *host512);

/* ================================================= MXFP4 routed experts */

/* Copy one routed expert (w1/w3 FP4 [inter, hidden], w2 FP4 [hidden, inter],
 * E8M0 scales per 1x32) into HBM, keyed by (layer, expert) -- not by
 * pointer, since the reference's expert slots are reused (dsv4_cuda.cu:
 * 232-236). 0 / -1 as dsv4_gpu_upload. No reference counterpart (the
 * reference runs experts on the CPU, dsv4_cuda.h:19-21). */
int dsv4_gpu_upload_expert(int layer, int expert, const DSV4ExpertW *e);

/* Register an expert whose tensors already live in HBM (e->*.w / .s are
 * device pointers owned by the caller, e.g. a checkpoint loaded straight into
 * device memory). Same keying and use as dsv4_gpu_upload_expert. The weight
 * pointers must be 16-byte and the scale pointers 4-byte aligned (-1 if
 * not). */
int dsv4_gpu_bind_expert_d(int layer, int expert, const DSV4ExpertW *e);

int dsv4_gpu_has_expert(int layer, int expert);

/* The routed half of moe() (dsv4_layer.c:380, :412-476) on the device:
 *   out[i] = sum_k w[k] * (w2_k . swiglu(w1_k . x, w3_k . x, limit))[i]
 * with the sum taken strictly in k order, multiply and add rounded
 * separately, as dsv4_layer.c:471-475; SwiGLU as dsv4_ops.c:60-78 (limit <=
 * 0 disables the clamp). Host buffers: out/x [hidden], idx/w [topk].
 * 0 / -1 (an expert not resident, or a shape that does not match). */
int dsv4_gpu_moe_fp4(float *out, const float *x, int layer, const int *idx,
                     const float *w, int topk, int hidden, int inter,
                     float swiglu_limit);

/* Stream-ordered form on device buffers; d_idx/d_w live in HBM so routing
 * computed on the device needs no host round trip. */
int dsv4_gpu_moe_fp4_d(float *d_out, const float *d_x, int layer,
                       const int *d_idx, const float *d_w, int topk,
                       int hidden, int inter, float swiglu_limit,
                       void *stream);

/* The routed half of moe_n (dsv4_layer.c:714-855, the batched prefill
 * path) on the device: out[t] = dsv4_gpu_moe_fp4 of token t, for nt <=
 * DSV4_MAX_BATCH tokens (x/out [nt][hidden], idx/w [nt][topk], host
 * buffers). As in the reference, the distinct experts the batch asks for are
 * found first (in first-request order) and each one's weights are read once
 * for every (token, k) routed to it; each token's row is bit-identical to
 * dsv4_gpu_moe_fp4 on that token. 0 / -1 (an expert not resident, a shape
 * that does not match, nt out of range). */
int dsv4_gpu_moe_fp4_n(float *out, const float *x, int layer, const int *idx,
                       const float *w, int nt, int topk, int hidden, int inter,
                       float swiglu_limit);

/* Stream-ordered form on device buffers (the routing stays on the device:
 * an id outside the layer's table, or an expert not registered, gives that
 * token a NaN row, as dsv4_gpu_moe_fp4_d does). */
int dsv4_gpu_moe_fp4_n_d(float *d_out, const float *d_x, int layer, const int *d_idx,
                         const float *d_w, int nt, int topk, int hidden, int inter,
                         float swiglu_limit, void *stream);

/* dsv4_gpu_moe_fp4_d without any allocation: the same kernels and the same
 * bits, with their scratch (x's and h's bf16 term planes, or h in f32) in a
 * fixed 1 MiB array in each device's global memory instead of a buffer the
 * library grows with hipMalloc. No counterpart in the reference: it is for
 * callers that cannot allocate -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. It calls no hipMalloc,
 * hipFree or allocating library routine. The experts must be registered
 * (dsv4_gpu_upload_expert / dsv4_gpu_bind_expert_d) before; -1 with a
 * message when the call needs more scratch than the array holds (the staged
 * matrix-core form takes hidden x 6 + topk x inter x 6 bytes, the VALU form
 * topk x inter x 4: topk 64 at inter 2048 and hidden 16384 fit). Every call
 * on one device shares that device's array: calls that overlap on one
 * device (two streams, or two host threads) race. */
int dsv4_gpu_moe_fp4_noalloc_d(float *d_out, const float *d_x, int layer,
                               const int *d_idx, const float *d_w, int topk,
                               int hidden, int inter, float swiglu_limit,
                               void *stream);

/* ============================================================ sparse MLA */

/* A device-resident row store for the latent KV cache or the indexer's key
 * cache, with an append API (dsv4_gpu_kv_create / dsv4_gpu_kv_write_row).
 * fmt: DSV4_GPU_KV_F32 (the reference's f32 cache), DSV4_GPU_KV_BF16, or
 * DSV4_GPU_KV_FP8 (e4m3 bytes with one fp32 scale per row; a row dequantises
 * to e4m3(code) * scale, exact in f32). */
enum { DSV4_GPU_KV_F32 = 0, DSV4_GPU_KV_BF16 = 1, DSV4_GPU_KV_FP8 = 2 };
typedef struct dsv4_gpu_kv dsv4_gpu_kv;

dsv4_gpu_kv *dsv4_gpu_kv_create(int n_rows, int row_dim, int fmt);
/* Write rows [row0, row0+n) from host memory laid out [n][row_dim] in the
 * store's format; row_scales[n] for FP8 (ignored otherwise). */
int dsv4_gpu_kv_write_rows(dsv4_gpu_kv *kv, int row0, int n, const void *rows,
                           const float *row_scales);
/* Device base pointers, for stream-ordered calls and for writing rows from
 * device code: data [n_rows][row_dim], scales [n_rows] (FP8 only, else
 * NULL). */
void *dsv4_gpu_kv_data(const dsv4_gpu_kv *kv);
float *dsv4_gpu_kv_scales(const dsv4_gpu_kv *kv);
void dsv4_gpu_kv_free(dsv4_gpu_kv *kv);

/* dsv4_indexer_score (dsv4_indexer.c:64-85), bit-exact: out[t] for the n
 * rows of `keys` starting at row0, each read as D values with a row pitch of
 * key_stride elements (the reference call passes rows of width D,
 * dsv4_layer.c:286-289). q [H][D], w [H] host f32. 0 / -1. */
int dsv4_gpu_indexer_score(float *out, const float *q, const float *w, int H,
                           int D, const dsv4_gpu_kv *keys, int row0,
                           int key_stride, int n);

/* dsv4_topk (dsv4_indexer.c:92-106), bit-exact: the k largest scores,
 * ordered by score descending with ties to the lower index; k is clamped to
 * n; returns the count written, or -1. NaN scores are placed as the
 * reference's scan (`scores[c] > scores[best]`, best starting at the lowest
 * index not yet taken) places them: a NaN is taken exactly when it is the
 * lowest untaken index, otherwise the pick is the first maximum of the
 * untaken finite scores. */
int dsv4_gpu_topk(int *idxs, const float *scores, int n, int k);

/* Score then top-k in one call, the CSA selection of dsv4_layer.c:280-291.
 * Returns the count written, or -1. */
int dsv4_gpu_indexer_topk(int *idxs, const float *q, const float *w, int H,
                          int D, const dsv4_gpu_kv *keys, int row0,
                          int key_stride, int n, int k);

/* dsv4_sparse_attn (dsv4_attn.c:60-108): o[h][d_v] = softmax over the
 * gathered rows idxs[topk] (entries of -1 are masked) of q . kv[:, :d_qk] *
 * scale, applied to kv[:, :d_v]; sink[h] enters the denominator only, or is
 * absent when NULL. q [h][d_qk] host f32. Within 1e-5 relative of the
 * reference. 0 / -1. */
int dsv4_gpu_sparse_attn(float *o, const float *q, const dsv4_gpu_kv *kv,
                         const float *sink, const int *idxs, int h, int d_qk,
                         int d_v, int topk, float scale);

/* Stream-ordered forms on device buffers. Keys/KV are raw device arrays in
 * the DSV4_GPU_KV_* formats (d_key_scales for FP8 keys, else NULL).
 * dsv4_gpu_indexer_score_d takes the score scale precomputed as the
 * reference does in float: (1/sqrtf(D)) * (1/sqrtf(H)). */
int dsv4_gpu_indexer_score_d(float *d_out, const float *d_q, const float *d_w,
                             int H, int D, const void *d_keys,
                             const float *d_key_scales, int key_fmt,
                             int key_stride, int n, float scale, void *stream);
/* dsv4_gpu_topk_d (and the top-k inside dsv4_gpu_mla_decode_d and the
 * attention block) selects exactly as dsv4_gpu_topk does, NaN scores
 * included. */
int dsv4_gpu_topk_d(int *d_idxs, const float *d_scores, int n, int k,
                    void *stream);
/* Selected rows outside [0, kv_rows) are treated as masked and never read
 * (the host-buffer form rejects them instead). */
int dsv4_gpu_sparse_attn_d(float *d_o, const float *d_q, const void *d_kv,
                           int kv_fmt, int kv_stride, int kv_rows,
                           const float *d_sink, const int *d_idxs, int h,
                           int d_qk, int d_v, int topk, float scale,
                           void *stream);

/* One sparse-MLA decode step on device buffers: indexer score over n keys,
 * top-k, then attention over the selected KV rows (indices are positions in
 * the KV store, no window offset). Writes the selection to d_idxs[k]. */
int dsv4_gpu_mla_decode_d(float *d_o, int *d_idxs,
                          const float *d_q_idx, const float *d_w_idx, int H,
                          int D, const void *d_keys, const float *d_key_scales,
                          int key_fmt, int key_stride, int n, int k,
                          const float *d_q, const void *d_kv, int kv_fmt,
                          int kv_stride, int kv_rows, const float *d_sink,
                          int h, int d_qk, int d_v, float attn_scale,
                          void *stream);

/* ------------------------------------------------- the attention block ---
 * attention() of the reference (src/model/dsv4_layer.c:213-336) for one
 * token, entirely on the device: q (wq_a, q_norm, wq_b, the per-head norm
 * and RoPE), kv (wkv, kv_norm, RoPE, into the sliding ring), the compressor
 * (comp wkv / wgate, the slot update and, when a window closes, the pool,
 * comp norm and RoPE at the window's first position into the next
 * compressed row), the CSA selection (indexer wq_b, RoPE, weights_proj,
 * score over the compressed rows at index_head_dim stride, top-k) or all
 * compressed rows, the sparse attention over [ring | selection] with the
 * sinks, the output de-rotation, the wo_a group slices and wo_b. The
 * reference crosses the host-device boundary once per matmul here (about
 * nine times per layer); this is one call. No counterpart in the
 * reference's GPU header: the caller's binding is one test at the top of
 * attention() that calls dsv4_gpu_attn_step when dsv4_gpu_attn_ready(layer).
 *
 * The block keeps the layer's state (the ring, the compressed rows, the
 * compressor's slots) on the device. Positions must come in order from 0,
 * as the reference's decode does; dsv4_gpu_attn_reset starts over. Within
 * 1e-5-scale relative error of the reference per step (its GEMVs accumulate
 * in fp32 where the reference uses double); the selection is the
 * reference's wherever the scores it ranks agree. */
typedef struct {
    int hidden, q_lora, n_heads, head_dim, rope_dim;   /* DSV4Cfg (qk_rope)  */
    int window;                /* sliding_window                            */
    int ratio;                 /* the layer's compress ratio (0: none)      */
    int idx_heads, idx_dim, idx_topk;  /* the indexer; idx_heads 0 if none  */
    int o_groups, o_lora;
    int max_pos;               /* positions 0 .. max_pos-1                  */
    float rms_eps;
} dsv4_gpu_attn_cfg;

typedef struct {
    DSV4QMat wq_a, wq_b, wkv, wo_a, wo_b;     /* resident (dsv4_gpu_upload);
                                                wo_a FP8                   */
    DSV4QMat comp_wkv, comp_wgate;            /* ratio > 0, resident        */
    DSV4QMat idx_wq_b, idx_wproj;             /* idx_heads > 0, resident    */
    const float *q_norm, *kv_norm;            /* [q_lora], [head_dim]       */
    const float *sink;                        /* [n_heads], or NULL         */
    const float *comp_norm, *comp_ape;        /* [head_dim],
                                                [ratio][coff*head_dim]     */
    const float *rope_cos, *rope_sin;         /* the layer's RoPE table,
                                                [max_pos][rope_dim/2]      */
} dsv4_gpu_attn_w;

/* Copies the vectors and the RoPE table, resolves the matrices (which must
 * be resident already) and allocates the layer's state; rebinding a layer
 * replaces it. 0 / -1. */
int dsv4_gpu_attn_bind(int layer, const dsv4_gpu_attn_cfg *c, const dsv4_gpu_attn_w *w);
/* 1 if the layer is bound. */
int dsv4_gpu_attn_ready(int layer);
/* The layer's state back to position 0. 0 / -1. */
int dsv4_gpu_attn_reset(int layer);
/* out[hidden] = attention(x[hidden]) at pos; host buffers, synchronous. */
int dsv4_gpu_attn_step(float *out, const float *x, int layer, int pos);
/* The same on device buffers (16-byte aligned), stream-ordered. */
int dsv4_gpu_attn_step_d(float *d_out, const float *d_x, int layer, int pos, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_GPU_H */
