/* SPDX-License-Identifier: Apache-2.0 */
/* e2e_decode.c - end-to-end greedy decode of a tiny deepseek_v4 checkpoint
 * through the reference's OWN C99 model code, CPU path against GPU trunk.
 *
 * TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles
 * this driver together with the reference's sources, where they lie under
 * /root/reference, into oracle/_ref/dsv4_e2e:
 *   - src/core: matmul, ops, hc, rope, compress, indexer, attn;
 *   - src/model: layer, bind;
 *   - src/io: st.
 * Its matmul dispatch (dsv4_matmul.c:525,572) is compiled with dsv4_cuda_has /
 * dsv4_cuda_mmq / dsv4_cuda_mmq_n renamed to dsv4_gpu_*, and it links
 * deepseek-v4-in-c_amd/lib/libdsv4_gpu.so. That is the drop-in binding of
 * the matmul dispatch (the three dsv4_cuda_* calls replaced by their
 * dsv4_gpu_* counterparts), made with the preprocessor instead of an edit.
 *
 * The decode loop restates the reference's own (dsv4_run.c:444-483,
 * tests/unit/test_model_oracle.c:196-245):
 *   embedding row -> hc_mult copies -> every layer's dsv4_layer_forward
 *   -> the head's hc reduction -> final RMSNorm -> head matmul -> argmax.
 * The run goes twice over the same teacher-forced tokens, from fresh layer
 * state each time:
 *   - pass 1: nothing resident, so every matmul runs on the reference CPU
 *     path;
 *   - pass 2: the checkpoint read straight into HBM by the backend's
 *     loader (dsv4_gpu_ckpt_load_layer / _load_qmat: every FP8 trunk
 *     matrix, every BF16 matrix -- router gates, compressors, indexer
 *     weights, the LM head -- and every routed expert), and the binder's
 *     matrices swapped for the resident ones, so every FP8 matmul (including
 *     the wo_a group slices), the experts' matmuls of expert_forward
 *     (dsv4_layer.c:199-206) and the rest run on the MI355X through the
 *     reference's dispatch; and the CSA calls of attention()
 *     (dsv4_layer.c:286-301) go to the device. oracle/Makefile compiles
 *     dsv4_layer.c with dsv4_indexer_score / dsv4_topk / dsv4_sparse_attn
 *     renamed to the e2e_* wrappers below, which call dsv4_gpu_indexer_score
 *     / dsv4_gpu_topk / dsv4_gpu_sparse_attn in pass 2 and the reference's
 *     own functions otherwise -- the CSA call sites of attention()
 *     (dsv4_layer.c:286-301) bound to the device, made with the
 *     preprocessor instead of an edit.
 *   - pass 3 (GPU runs): the same, with every layer's attention() taken
 *     from the device attention block (dsv4_gpu_attn_step, one call per
 *     layer and position) and its routed experts' k-ordered sum from the
 *     fused pass (dsv4_gpu_moe_fp4), through the matmul hooks described at
 *     e2e_mmq.
 *   - pass 4: the reference's batched prefill protocol
 *     (tests/unit/test_model_oracle.c:295-378): dsv4_layer_forward_n over
 *     chunks of 1, 2, 3 and all the tokens, from fresh layer state each
 *     time, with pass 2's residency and device CSA calls, so moe_n's
 *     batched matmuls (dsv4_layer.c:714-855: the router gate, every routed
 *     expert of the batch's union, the shared expert) run as
 *     dsv4_gpu_mmq_n. Every position's logits must equal pass 2's bit for
 *     bit. With --cpu-only it runs on the CPU against the CPU pass.
 *   - pass 5 (GPU runs): the same chunks with pass 3's device attention
 *     block, and moe_n's routed sum from the device's batched pass
 *     (dsv4_gpu_moe_fp4_n, hooked at e2e_mmq_n); every position's logits
 *     must equal pass 3's bit for bit.
 * Routed experts come from memory (all resident).
 *
 * usage: dsv4_e2e CKPT_DIR TOKENS_FILE [--cpu-only]
 * Prints one line per position and a summary; exit 0 when every argmax
 * agrees, 1 when one differs or a step fails, 2 when no GPU is available
 * (unless --cpu-only).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dsv4_cfg.h"
#include "dsv4_st.h"
#include "dsv4_bind.h"
#include "dsv4_layer.h"
#include "dsv4_gpu.h"

void dsv4_rmsnorm(float *y, const float *x, const float *w, int n, float eps);
void dsv4_mmq(float *y, const float *x, const DSV4QMat *m);
void dsv4_rope_table(float *cs, float *sn, int rd, int maxpos, int orig_ctx,
                     double theta, double factor, double beta_fast, double beta_slow);

/* ------------------------------------------------- CSA on the device ---- */
/* The reference's own functions (dsv4_layer.c:58-66 declares them). */
void dsv4_sparse_attn(float *, const float *, const float *, const float *,
                      const int *, int, int, int, float, float *);
void dsv4_indexer_score(float *, const float *, const float *, const float *,
                        int, int, int);
int dsv4_topk(int *, const float *, int, int);

static int g_gpu_csa;                       /* pass 2: CSA calls on the device */
static long g_n_score, g_n_topk, g_n_attn, g_n_head, g_n_head_ok;

static void csa_fail(const char *what)
{
    fprintf(stderr, "e2e: %s on the device failed\n", what);
    abort();
}

/* dsv4_indexer_score (dsv4_indexer.c:64-85): the n key rows of width D
 * starting at kv, as the caller passes them (dsv4_layer.c:286-289). */
void e2e_indexer_score(float *out, const float *q, const float *kv, const float *w,
                       int H, int D, int n)
{
    if (!g_gpu_csa || n <= 0) {
        dsv4_indexer_score(out, q, kv, w, H, D, n);
        return;
    }
    dsv4_gpu_kv *keys = dsv4_gpu_kv_create(n, D, DSV4_GPU_KV_F32);
    if (!keys || dsv4_gpu_kv_write_rows(keys, 0, n, kv, NULL) != 0 ||
        dsv4_gpu_indexer_score(out, q, w, H, D, keys, 0, D, n) != 0)
        csa_fail("indexer score");
    dsv4_gpu_kv_free(keys);
    g_n_score++;
}

/* dsv4_topk (dsv4_indexer.c:92-106). */
int e2e_topk(int *idxs, const float *scores, int n, int k)
{
    if (!g_gpu_csa || n <= 0 || k <= 0) return dsv4_topk(idxs, scores, n, k);
    const int r = dsv4_gpu_topk(idxs, scores, n, k);
    if (r < 0) csa_fail("top-k");
    g_n_topk++;
    return r;
}

/* dsv4_sparse_attn (dsv4_attn.c:60-108) over the rows of the layer's KV ring
 * that idxs names (-1 entries masked). */
void e2e_sparse_attn(float *o, const float *q, const float *kv, const float *sink,
                     const int *idxs, int h, int d, int topk, float scale, float *scratch)
{
    int rows = 0;
    for (int i = 0; i < topk; i++)
        if (idxs[i] + 1 > rows) rows = idxs[i] + 1;
    if (!g_gpu_csa || rows == 0) {
        dsv4_sparse_attn(o, q, kv, sink, idxs, h, d, topk, scale, scratch);
        return;
    }
    dsv4_gpu_kv *cache = dsv4_gpu_kv_create(rows, d, DSV4_GPU_KV_F32);
    if (!cache || dsv4_gpu_kv_write_rows(cache, 0, rows, kv, NULL) != 0 ||
        dsv4_gpu_sparse_attn(o, q, cache, sink, idxs, h, d, d, topk, scale) != 0)
        csa_fail("sparse attention");
    dsv4_gpu_kv_free(cache);
    g_n_attn++;
}

/* ------------------------------------------- the attention block ---- */
/* Pass 3: dsv4_layer.c is also compiled with dsv4_mmq renamed to e2e_mmq.
 * attention()'s first matmul (wq_a, dsv4_layer.c:220) then also runs the
 * whole block on the device, dsv4_gpu_attn_step, from the same x; its last
 * (wo_b, :335) returns the block's output instead of computing its own. So
 * the layer carries on from the device block's result, while the body in
 * between still runs on its own (its results unused). The routed experts'
 * sum is replaced the same way by dsv4_gpu_moe_fp4 (below). Every other
 * matmul passes through to the reference's dispatch. */
void dsv4_mmq(float *y, const float *x, const DSV4QMat *m);

static int g_attn_block, g_attn_nl, g_attn_pending = -1;
static int g_lpos[DSV4_MAX_LAYERS];         /* the next position of each layer's block */
static const DSV4LayerBind *g_attn_lb;
static const DSV4Cfg *g_cfg;
static DSV4Scratch *g_scr;
static DSV4Batch *g_bat;                    /* the batch of a prefill pass */
static float *g_attn_out;
static long g_n_block, g_n_moe, g_n_moe_n;

void e2e_mmq(float *y, const float *x, const DSV4QMat *m)
{
    if (g_attn_block) {
        for (int L = 0; L < g_attn_nl; L++) {
            /* moe() (dsv4_layer.c:369-484) has summed the routed experts in k
             * order into its output, s->qr (:518), when the shared expert's
             * first matmul (:480) arrives with the same x: replace that sum
             * with the fused routed-expert pass, from the router's own
             * selection and weights (s->topk_idx, s->topk_w) */
            if (m == &g_attn_lb[L].w.moe.shared.w1) {
                const DSV4Cfg *c = g_cfg;
                if (dsv4_gpu_moe_fp4(g_attn_out, x, L, g_scr->topk_idx, g_scr->topk_w, c->topk,
                                     c->hidden, c->moe_inter, c->swiglu_limit) != 0)
                    csa_fail("routed experts");
                memcpy(g_scr->qr, g_attn_out, (size_t)c->hidden * sizeof(float));
                g_n_moe++;
                break;
            }
            if (m == &g_attn_lb[L].w.attn.wq_a) {
                /* a layer's attention() runs once per position, in position
                 * order, in decode and in prefill (dsv4_layer.c:865-894) */
                if (dsv4_gpu_attn_step(g_attn_out, x, L, g_lpos[L]++) != 0)
                    csa_fail("attention block");
                g_attn_pending = L;
                g_n_block++;
                break;
            }
            if (m == &g_attn_lb[L].w.attn.wo_b && g_attn_pending == L) {
                memcpy(y, g_attn_out, (size_t)m->rows * sizeof(float));
                g_attn_pending = -1;
                return;
            }
        }
    }
    dsv4_mmq(y, x, m);
}

/* dsv4_layer.c is also compiled with dsv4_mmq_n renamed to e2e_mmq_n. In
 * pass 5, moe_n (dsv4_layer.c:714-855) has summed the batch's routed experts
 * in k order into its output, the batch's blk_out (:912), when the shared
 * expert's first batched matmul (:843) arrives with the same x: replace
 * that sum with the device's batched routed-expert pass, from the router's
 * own selection and weights (b->topk_idx, b->topk_w). Every batched matmul
 * then goes to the reference's dispatch, dsv4_mmq_n (dsv4_matmul.c:562). */
void dsv4_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt);

void e2e_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt)
{
    if (g_attn_block && g_bat) {
        for (int L = 0; L < g_attn_nl; L++)
            if (m == &g_attn_lb[L].w.moe.shared.w1) {
                const DSV4Cfg *c = g_cfg;
                if (dsv4_gpu_moe_fp4_n(g_bat->blk_out, x, L, g_bat->topk_idx, g_bat->topk_w, nt,
                                       c->topk, c->hidden, c->moe_inter, c->swiglu_limit) != 0)
                    csa_fail("batched routed experts");
                g_n_moe_n++;
                break;
            }
    }
    dsv4_mmq_n(y, x, m, nt);
}

/* ---------------------------------------------------- routed experts ---- */
typedef struct {
    DSV4ExpertW *w;          /* [n_layers][n_experts] */
    void **blocks;
    int n_layers, n_experts, nblocks;
} Experts;

static void *read_tensor(const DSV4St *st, const char *name, int64_t *nbytes)
{
    const DSV4Tensor *t = dsv4_st_find(st, name);
    if (!t) { fprintf(stderr, "e2e: %s missing\n", name); return NULL; }
    void *buf = malloc((size_t)t->nbytes);
    if (!buf || dsv4_st_read(st, t, buf) != t->nbytes) {
        fprintf(stderr, "e2e: reading %s failed\n", name);
        free(buf);
        return NULL;
    }
    if (nbytes) *nbytes = t->nbytes;
    return buf;
}

/* Every routed expert, read once into memory and described as the expert
 * cache describes a slot (dsv4_cache.c:51-66: FP4, 1x32 blocks). */
static int load_experts(Experts *E, const DSV4St *st, const DSV4Cfg *c)
{
    E->n_layers = c->n_layers;
    E->n_experts = c->n_experts;
    E->w = calloc((size_t)c->n_layers * c->n_experts, sizeof *E->w);
    E->blocks = calloc((size_t)c->n_layers * c->n_experts * 6, sizeof(void *));
    E->nblocks = 0;
    if (!E->w || !E->blocks) return -1;
    for (int L = 0; L < c->n_layers; L++)
        for (int e = 0; e < c->n_experts; e++) {
            DSV4ExpertW *x = &E->w[(size_t)L * c->n_experts + e];
            DSV4QMat *m[3] = {&x->w1, &x->w2, &x->w3};
            const int rows[3] = {c->moe_inter, c->hidden, c->moe_inter};
            const int cols[3] = {c->hidden, c->moe_inter, c->hidden};
            for (int i = 0; i < 3; i++) {
                char nm[128];
                snprintf(nm, sizeof nm, "layers.%d.ffn.experts.%d.w%d.weight", L, e, i + 1);
                void *wb = read_tensor(st, nm, NULL);
                snprintf(nm, sizeof nm, "layers.%d.ffn.experts.%d.w%d.scale", L, e, i + 1);
                void *sb = read_tensor(st, nm, NULL);
                if (!wb || !sb) return -1;
                E->blocks[E->nblocks++] = wb;
                E->blocks[E->nblocks++] = sb;
                m[i]->w = wb;
                m[i]->s = sb;
                m[i]->wdt = DSV4_WFP4;
                m[i]->rows = rows[i];
                m[i]->cols = cols[i];
                m[i]->blk_r = 1;
                m[i]->blk_c = 32;
            }
        }
    return 0;
}

static const DSV4ExpertW *expert_get(void *ctx, int layer, int expert)
{
    const Experts *E = ctx;
    if (layer < 0 || layer >= E->n_layers || expert < 0 || expert >= E->n_experts)
        return NULL;
    return &E->w[(size_t)layer * E->n_experts + expert];
}

/* --------------------------------------------------------------- head ---- */
/* The head's own hc reduction (dsv4_run.c:94-116): a sigmoid gate per
 * stream from one RMS-scaled dot, no Sinkhorn, one scalar scale. */
static void head_hc(float *y, const float *x, const DSV4HcW *w, int hc, int hidden,
                    float norm_eps, float hc_eps)
{
    const int n = hc * hidden;
    double sq = 0.0;
    for (int i = 0; i < n; i++) sq += (double)x[i] * x[i];
    const float rs = (float)(1.0 / sqrt(sq / (double)n + (double)norm_eps));
    float gate[DSV4_MAX_HC_MULT];
    for (int j = 0; j < hc; j++) {
        double dot = 0.0;
        for (int i = 0; i < n; i++)
            dot = fma((double)w->fn[(size_t)j * n + i], (double)x[i], dot);
        const float m = (float)dot * rs;
        gate[j] = 1.0f / (1.0f + expf(-(m * w->scale[0] + w->base[j]))) + hc_eps;
    }
    for (int d = 0; d < hidden; d++) {
        double acc = 0.0;
        for (int j = 0; j < hc; j++)
            acc += (double)gate[j] * (double)x[(size_t)j * hidden + d];
        y[d] = (float)acc;
    }
}

/* The reference sizes s->idxs for window + index_topk entries
 * (dsv4_layer.c:128, :185), but a compressed layer without the indexer
 * attends to every compressed row (:293): past index_topk of them it writes
 * beyond that buffer, and its per-head attention scratch (:143 vs :175)
 * past its carve. The drivers give both room for every position; what is
 * computed does not change. */
static int widen_scratch(DSV4Scratch *s, const DSV4Cfg *c, int maxpos)
{
    const size_t rows = (size_t)c->sliding_window + (size_t)maxpos + 1;
    int *ix = calloc(rows, sizeof(int));
    float *sc = calloc((size_t)c->n_heads * rows, sizeof(float));
    if (!ix || !sc) { free(ix); free(sc); return -1; }
    free(s->idxs);
    s->idxs = ix;
    s->attn_scratch = sc;      /* lives until the process ends */
    return 0;
}

/* --------------------------------------------------------------- main ---- */
static int read_tokens(const char *path, int **out)
{
    FILE *f = fopen(path, "r");
    if (!f) { perror(path); return -1; }
    int cap = 64, n = 0;
    int *t = malloc(sizeof(int) * cap);
    long v;
    while (t && fscanf(f, "%ld", &v) == 1) {
        if (n == cap) { cap *= 2; t = realloc(t, sizeof(int) * cap); if (!t) break; }
        t[n++] = (int)v;
    }
    fclose(f);
    *out = t;
    return t ? n : -1;
}

typedef struct {
    const DSV4Cfg *c;
    DSV4LayerBind *lb;
    DSV4ModelBind *mb;
    DSV4ExpertSrc *src;
    DSV4Scratch *s;
    float *cs_d, *sn_d, *cs_c, *sn_c;
    int maxpos;
    DSV4QMat head;           /* the LM head: host bytes, or loaded into HBM */
} Model;

/* The reference's greedy pick (dsv4_run.c:471-472). */
static int first_max(const float *v, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* One greedy pass over the tokens from fresh layer state; logits[pos][vocab].
 * In the GPU pass the head also runs as dsv4_gpu_head_argmax (the GEMV and
 * the argmax on the device, only the token id back), which must pick what
 * the reference's scan picks from the logits. */
static int run_pass(const Model *M, const int *tok, int n, float *logits)
{
    const DSV4Cfg *c = M->c;
    const int hc = c->hc_mult, d = c->hidden;
    DSV4LayerState *ls = calloc((size_t)c->n_layers, sizeof *ls);
    float *h = calloc((size_t)hc * d, sizeof(float));
    float *y = calloc((size_t)d, sizeof(float));
    if (!ls || !h || !y) return -1;
    for (int L = 0; L < c->n_layers; L++)
        if (dsv4_state_init(&ls[L], c, L, M->maxpos) != 0) return -1;
    const DSV4QMat head = M->head;
    for (int pos = 0; pos < n; pos++) {
        dsv4_embed_row(y, M->mb->w.embed, M->mb->w.wdt, tok[pos], d);
        for (int j = 0; j < hc; j++) memcpy(h + (size_t)j * d, y, (size_t)d * sizeof(float));
        for (int L = 0; L < c->n_layers; L++) {
            const int comp = dsv4_compress_ratio(c, L) != 0;
            dsv4_layer_forward(h, &M->lb[L].w, c, M->s, M->src, &ls[L],
                               comp ? M->cs_c : M->cs_d, comp ? M->sn_c : M->sn_d,
                               pos, tok[pos]);
        }
        head_hc(y, h, &M->mb->w.hc_head, hc, d, c->rms_eps, c->hc_eps);
        dsv4_rmsnorm(y, y, M->mb->w.norm, d, c->rms_eps);
        dsv4_mmq(logits + (size_t)pos * c->vocab, y, &head);
        if (g_gpu_csa) {
            const int t = dsv4_gpu_head_argmax(y, &head);
            g_n_head++;
            g_n_head_ok += t == first_max(logits + (size_t)pos * c->vocab, c->vocab);
        }
    }
    for (int L = 0; L < c->n_layers; L++) dsv4_state_free(&ls[L]);
    free(ls); free(h); free(y);
    return 0;
}

/* The reference's batched prefill (tests/unit/test_model_oracle.c:303-372):
 * chunks of `chunk` tokens through dsv4_layer_forward_n from fresh layer
 * state, then each token's head as in run_pass; logits[pos][vocab]. */
static int run_prefill(const Model *M, const int *tok, int n, int chunk, float *logits)
{
    const DSV4Cfg *c = M->c;
    const int hc = c->hc_mult, d = c->hidden;
    DSV4LayerState *ls = calloc((size_t)c->n_layers, sizeof *ls);
    float *hb = calloc((size_t)chunk * hc * d, sizeof(float));
    float *y = calloc((size_t)d, sizeof(float));
    int32_t *tid = calloc((size_t)chunk, sizeof(int32_t));
    DSV4Batch bat;
    if (!ls || !hb || !y || !tid || dsv4_batch_init(&bat, c, chunk) != 0) return -1;
    for (int L = 0; L < c->n_layers; L++)
        if (dsv4_state_init(&ls[L], c, L, M->maxpos) != 0) return -1;
    const DSV4QMat head = M->head;
    g_bat = &bat;
    for (int p0 = 0; p0 < n; p0 += chunk) {
        const int nt = n - p0 < chunk ? n - p0 : chunk;
        for (int t = 0; t < nt; t++) {
            tid[t] = (int32_t)tok[p0 + t];
            dsv4_embed_row(y, M->mb->w.embed, M->mb->w.wdt, tok[p0 + t], d);
            for (int j = 0; j < hc; j++)
                memcpy(hb + ((size_t)t * hc + j) * d, y, (size_t)d * sizeof(float));
        }
        for (int L = 0; L < c->n_layers; L++) {
            const int comp = dsv4_compress_ratio(c, L) != 0;
            dsv4_layer_forward_n(hb, &M->lb[L].w, c, M->s, &bat, M->src, &ls[L],
                                 comp ? M->cs_c : M->cs_d, comp ? M->sn_c : M->sn_d,
                                 p0, tid, nt);
        }
        for (int t = 0; t < nt; t++) {
            head_hc(y, hb + (size_t)t * hc * d, &M->mb->w.hc_head, hc, d, c->rms_eps,
                    c->hc_eps);
            dsv4_rmsnorm(y, y, M->mb->w.norm, d, c->rms_eps);
            dsv4_mmq(logits + (size_t)(p0 + t) * c->vocab, y, &head);
        }
    }
    g_bat = NULL;
    for (int L = 0; L < c->n_layers; L++) dsv4_state_free(&ls[L]);
    dsv4_batch_free(&bat);
    free(ls); free(hb); free(y); free(tid);
    return 0;
}

/* Positions whose logits equal want's bit for bit, and whose argmax equals
 * ref's. */
static void compare_bits(const float *got, const float *want, const float *ref, int n,
                         int vocab, int *same, int *agree);

static int argmax(const float *v, int n, float *margin)
{
    int a = 0;
    for (int i = 1; i < n; i++) if (v[i] > v[a]) a = i;
    float second = -INFINITY;
    for (int i = 0; i < n; i++) if (i != a && v[i] > second) second = v[i];
    if (margin) *margin = v[a] - second;
    return a;
}

static void compare_bits(const float *got, const float *want, const float *ref, int n,
                         int vocab, int *same, int *agree)
{
    *same = *agree = 0;
    for (int p = 0; p < n; p++) {
        const size_t o = (size_t)p * vocab;
        *same += memcmp(got + o, want + o, (size_t)vocab * sizeof(float)) == 0;
        *agree += argmax(got + o, vocab, NULL) == argmax(ref + o, vocab, NULL);
    }
}

/* The block's per-layer device state and position counters, restarted
 * before a pass that runs the device attention block from position 0. */
static int restart_blocks(int n_layers)
{
    for (int L = 0; L < n_layers; L++) {
        g_lpos[L] = 0;
        if (dsv4_gpu_attn_reset(L) != 0) return -1;
    }
    return 0;
}

/* Vector-scaled relative error (tests/unit/test_cuda.c:160-167). */
static double vec_rel(const float *got, const float *ref, int n)
{
    double sq = 0.0;
    for (int i = 0; i < n; i++) sq += (double)ref[i] * ref[i];
    const double rms = sqrt(sq / n);
    double worst = 0.0;
    for (int i = 0; i < n; i++) {
        double s = fabs((double)ref[i]);
        if (fabs((double)got[i]) > s) s = fabs((double)got[i]);
        if (rms > s) s = rms;
        const double r = s > 0 ? fabs((double)got[i] - ref[i]) / s : 0.0;
        if (r > worst) worst = r;
    }
    return worst;
}

int main(int argc, char **argv)
{
    if (argc < 3) {
        fprintf(stderr, "usage: %s CKPT_DIR TOKENS_FILE [--cpu-only]\n", argv[0]);
        return 1;
    }
    const int cpu_only = argc > 3 && !strcmp(argv[3], "--cpu-only");
    char path[1024];
    DSV4Cfg c;
    int cr[DSV4_MAX_LAYERS];
    snprintf(path, sizeof path, "%s/config.json", argv[1]);
    if (!dsv4_cfg_load_file(&c, cr, DSV4_MAX_LAYERS, path)) return 1;
    DSV4St st;
    if (dsv4_st_open(&st, argv[1]) != 0) return 1;
    int *tok = NULL;
    const int n = read_tokens(argv[2], &tok);
    if (n <= 0) return 1;
    for (int i = 0; i < n; i++)
        if (tok[i] < 0 || tok[i] >= c.vocab) {
            fprintf(stderr, "e2e: token %d out of range\n", tok[i]);
            return 1;
        }

    DSV4LayerBind *lb = calloc((size_t)c.n_layers, sizeof *lb);
    for (int L = 0; L < c.n_layers; L++)
        if (dsv4_bind_layer(&st, &c, L, &lb[L]) != 0) return 1;
    DSV4ModelBind mb;
    if (dsv4_bind_model(&st, &c, 1, &mb) != 0) return 1;
    Experts E;
    if (load_experts(&E, &st, &c) != 0) return 1;
    DSV4ExpertSrc src = {.get = expert_get, .ctx = &E};

    Model M = {.c = &c, .lb = lb, .mb = &mb, .src = &src, .maxpos = n + 16};
    M.head = (DSV4QMat){mb.w.head, NULL, DSV4_WBF16, c.vocab, c.hidden, 0, 0};
    const int half = c.qk_rope / 2;
    M.cs_d = malloc((size_t)M.maxpos * half * 4); M.sn_d = malloc((size_t)M.maxpos * half * 4);
    M.cs_c = malloc((size_t)M.maxpos * half * 4); M.sn_c = malloc((size_t)M.maxpos * half * 4);
    dsv4_rope_table(M.cs_d, M.sn_d, c.qk_rope, M.maxpos, 0, c.rope_theta,
                    c.yarn_factor, c.yarn_beta_fast, c.yarn_beta_slow);
    dsv4_rope_table(M.cs_c, M.sn_c, c.qk_rope, M.maxpos, c.yarn_orig_ctx,
                    c.compress_rope_theta, c.yarn_factor, c.yarn_beta_fast,
                    c.yarn_beta_slow);
    DSV4Scratch s;
    if (dsv4_scratch_init(&s, &c, M.maxpos) != 0 || widen_scratch(&s, &c, M.maxpos) != 0)
        return 1;
    M.s = &s;
    printf("e2e: hidden %d, %d layers, vocab %d, %d experts (top-%d), index_topk %d, "
           "%d positions\n", c.hidden, c.n_layers, c.vocab, c.n_experts, c.topk,
           c.index_topk, n);

    float *ref = malloc((size_t)n * c.vocab * sizeof(float));
    float *got = malloc((size_t)n * c.vocab * sizeof(float));
    if (!ref || !got || run_pass(&M, tok, n, ref) != 0) return 1;

    int gpu_mats = 0, fp4_mats = 0, bf16_mats = 0;
    if (cpu_only) {
        if (run_pass(&M, tok, n, got) != 0) return 1;
    } else {
        if (!dsv4_gpu_available() || dsv4_gpu_init() != 0) {
            fprintf(stderr, "e2e: no GPU\n");
            return 2;
        }
        /* the checkpoint straight into HBM: every matrix and routed expert
         * read from the shards by the backend's loader (no copy of the
         * host's), then the binder's matrices swapped for the resident
         * ones, which carry device addresses */
        dsv4_gpu_ckpt *ck = dsv4_gpu_ckpt_open(argv[1]);
        if (!ck) return 1;
        for (int L = 0; L < c.n_layers; L++) {
            DSV4LayerW *w = &lb[L].w;
            const dsv4_gpu_ckpt_dims dm = {
                .hidden = c.hidden, .q_lora = c.q_lora, .n_heads = c.n_heads,
                .head_dim = c.head_dim, .o_groups = c.o_groups, .o_lora = c.o_lora,
                .moe_inter = c.moe_inter, .n_shared = c.n_shared, .n_experts = c.n_experts,
                .index_n_heads = c.index_n_heads, .index_head_dim = c.index_head_dim,
                .compress_ratio = dsv4_compress_ratio(&c, L), .has_indexer = w->has_idx};
            dsv4_gpu_layer_mats lm;
            if (dsv4_gpu_ckpt_load_layer(ck, &dm, L, &lm, &E.w[(size_t)L * c.n_experts]) != 0) {
                fprintf(stderr, "e2e: loading layer %d into HBM failed\n", L);
                return 1;
            }
            DSV4AttnW *a = &w->attn;
            a->wq_a = lm.wq_a; a->wq_b = lm.wq_b; a->wkv = lm.wkv;
            a->wo_a = lm.wo_a; a->wo_b = lm.wo_b;
            w->moe.shared.w1 = lm.shared_w1; w->moe.shared.w2 = lm.shared_w2;
            w->moe.shared.w3 = lm.shared_w3; w->moe.gate = lm.gate;
            gpu_mats += 8;
            bf16_mats += 1;
            if (a->has_comp) { a->comp.wkv = lm.comp_wkv; a->comp.wgate = lm.comp_wgate; bf16_mats += 2; }
            if (a->has_idx) {
                a->idx.wq_b = lm.idx_wq_b; a->idx.weights_proj = lm.idx_wproj;
                a->idx.comp.wkv = lm.idx_comp_wkv; a->idx.comp.wgate = lm.idx_comp_wgate;
                gpu_mats += 1;
                bf16_mats += 3;
            }
            fp4_mats += 3 * c.n_experts;
        }
        /* the LM head, the QMat run_pass uses (dsv4_run.c:467-474) */
        if (dsv4_gpu_ckpt_load_qmat(ck, "head", DSV4_WBF16, c.vocab, c.hidden, &M.head) != 0)
            return 1;
        bf16_mats++;
        dsv4_gpu_ckpt_stats cs;
        dsv4_gpu_ckpt_stats_get(ck, &cs);
        printf("load: %d shards, %lld tensors indexed; %lld matrices and %lld experts read "
               "into HBM, %lld bytes in %.3f s (%.2f GB/s), no host upload\n", cs.shards,
               cs.tensors, cs.matrices, cs.experts, cs.bytes, cs.seconds,
               cs.seconds > 0 ? (double)cs.bytes / cs.seconds / 1e9 : 0.0);
        dsv4_gpu_ckpt_close(ck);
        printf("gpu: %d FP8, %d FP4 and %d BF16 matrices resident, CSA on the device\n",
               gpu_mats, fp4_mats, bf16_mats);
        g_gpu_csa = 1;
        if (gpu_mats == 0 || run_pass(&M, tok, n, got) != 0) return 1;
        g_gpu_csa = 0;
    }

    /* pass 3: every layer's attention() from the device block */
    int agree3 = 0;
    double worst3 = 0.0;
    float *got3 = NULL;
    if (!cpu_only) {
        for (int L = 0; L < c.n_layers; L++) {
            const DSV4AttnW *a = &lb[L].w.attn;
            const int ratio = dsv4_compress_ratio(&c, L);
            dsv4_gpu_attn_cfg ac = {
                .hidden = c.hidden, .q_lora = c.q_lora, .n_heads = c.n_heads,
                .head_dim = c.head_dim, .rope_dim = c.qk_rope, .window = c.sliding_window,
                .ratio = ratio, .idx_heads = a->has_idx ? c.index_n_heads : 0,
                .idx_dim = c.index_head_dim, .idx_topk = c.index_topk, .o_groups = c.o_groups,
                .o_lora = c.o_lora, .max_pos = M.maxpos, .rms_eps = c.rms_eps};
            dsv4_gpu_attn_w aw = {
                .wq_a = a->wq_a, .wq_b = a->wq_b, .wkv = a->wkv, .wo_a = a->wo_a,
                .wo_b = a->wo_b, .q_norm = a->q_norm, .kv_norm = a->kv_norm, .sink = a->sink,
                .rope_cos = ratio ? M.cs_c : M.cs_d, .rope_sin = ratio ? M.sn_c : M.sn_d};
            if (a->has_comp) {
                aw.comp_wkv = a->comp.wkv; aw.comp_wgate = a->comp.wgate;
                aw.comp_norm = a->comp.norm; aw.comp_ape = a->comp.ape;
            }
            if (a->has_idx) { aw.idx_wq_b = a->idx.wq_b; aw.idx_wproj = a->idx.weights_proj; }
            if (dsv4_gpu_attn_bind(L, &ac, &aw) != 0) return 1;
        }
        /* the routed experts were registered for the fused pass when the
         * loader read them */
        g_attn_lb = lb;
        g_attn_nl = c.n_layers;
        g_cfg = &c;
        g_scr = &s;
        g_attn_out = malloc((size_t)c.hidden * sizeof(float));
        got3 = malloc((size_t)n * c.vocab * sizeof(float));
        if (!g_attn_out || !got3) return 1;
        g_attn_block = 1;
        if (restart_blocks(c.n_layers) != 0 || run_pass(&M, tok, n, got3) != 0) return 1;
        g_attn_block = 0;
        for (int p = 0; p < n; p++) {
            const int ar = argmax(ref + (size_t)p * c.vocab, c.vocab, NULL);
            const int ag = argmax(got3 + (size_t)p * c.vocab, c.vocab, NULL);
            const double r = vec_rel(got3 + (size_t)p * c.vocab, ref + (size_t)p * c.vocab,
                                     c.vocab);
            if (r > worst3) worst3 = r;
            agree3 += ar == ag;
        }
    }

    /* passes 4 and 5: the reference's batched prefill at chunks 1, 2, 3 and
     * all the tokens (test_model_oracle.c:303), each position's logits bit
     * for bit against the per-token GPU pass with the same device parts */
    /* the per-token passes' device call counts, before the prefill passes
     * add theirs */
    const long n_score2 = g_n_score, n_topk2 = g_n_topk, n_attn2 = g_n_attn;
    const long n_block3 = g_n_block, n_moe3 = g_n_moe;
    int pf_runs = 0, pf_same[2] = {0, 0}, pf_agree[2] = {0, 0}, pf_pos = 0;
    char pf_list[64] = "";
    {
        const int chunks[4] = {1, 2, 3, n};
        float *got4 = malloc((size_t)n * c.vocab * sizeof(float));
        if (!got4) return 1;
        for (int ci = 0; ci < 4; ci++) {
            const int ch = chunks[ci];
            if (ch < 1 || ch > DSV4_MAX_BATCH || (ci > 0 && ch == chunks[ci - 1])) continue;
            for (int v = 0; v < (cpu_only ? 1 : 2); v++) {
                int same, agree_c;
                if (v == 0) {                /* pass 4: dispatch + device CSA
                                              * (all on the CPU with --cpu-only) */
                    g_gpu_csa = !cpu_only;
                    if (run_prefill(&M, tok, n, ch, got4) != 0) return 1;
                    g_gpu_csa = 0;
                    compare_bits(got4, got, ref, n, c.vocab, &same, &agree_c);
                } else {                     /* pass 5: device block + moe_n */
                    g_attn_block = 1;
                    if (restart_blocks(c.n_layers) != 0 ||
                        run_prefill(&M, tok, n, ch, got4) != 0)
                        return 1;
                    g_attn_block = 0;
                    compare_bits(got4, got3, ref, n, c.vocab, &same, &agree_c);
                }
                printf("prefill pass %d chunk %d: %d of %d positions bit-identical to pass %d, "
                       "argmax equal to the CPU path at %d\n", 4 + v, ch, same, n, 2 + v,
                       agree_c);
                pf_same[v] += same;
                pf_agree[v] += agree_c;
            }
            pf_pos += n;
            pf_runs++;
            snprintf(pf_list + strlen(pf_list), sizeof pf_list - strlen(pf_list), "%s%d",
                     pf_runs > 1 ? "," : "", ch);
        }
        free(got4);
    }

    int agree = 0;
    double worst = 0.0;
    for (int p = 0; p < n; p++) {
        float mr, mg;
        const int ar = argmax(ref + (size_t)p * c.vocab, c.vocab, &mr);
        const int ag = argmax(got + (size_t)p * c.vocab, c.vocab, &mg);
        const double r = vec_rel(got + (size_t)p * c.vocab, ref + (size_t)p * c.vocab, c.vocab);
        if (r > worst) worst = r;
        agree += ar == ag;
        printf("pos %d tok %d cpu %d %s %d margin %.6g rel %.3g\n", p, tok[p], ar,
               cpu_only ? "cpu2" : "gpu", ag, (double)mr, r);
    }
    printf("summary: positions %d argmax_equal %d worst_rel %.3g gpu_mats %d "
           "fp4_mats %d gpu_score %ld gpu_topk %ld gpu_attn %ld bf16_mats %d "
           "head_ok %ld/%ld\n", n, agree, worst, gpu_mats, fp4_mats, n_score2, n_topk2,
           n_attn2, bf16_mats, g_n_head_ok, g_n_head);
    printf("summary45: prefill chunks %s positions %d pass4_bit_identical %d "
           "pass4_argmax_equal %d pass5_bit_identical %d pass5_argmax_equal %d "
           "moe_n_calls %ld\n", pf_list, pf_pos, pf_same[0], pf_agree[0], pf_same[1],
           pf_agree[1], g_n_moe_n);
    if (!cpu_only) {
        printf("summary3: attention blocks on the device: steps %ld argmax_equal %d "
               "worst_rel %.3g fused_moe %ld\n", n_block3, agree3, worst3, n_moe3);
        dsv4_gpu_shutdown();
    }
    const int pf_ok = pf_same[0] == pf_pos && pf_agree[0] == pf_pos &&
                      (cpu_only || (pf_same[1] == pf_pos && pf_agree[1] == pf_pos));
    return (agree == n && (cpu_only || agree3 == n) && pf_ok) ? 0 : 1;
}
