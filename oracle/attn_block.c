/* SPDX-License-Identifier: Apache-2.0 */
/* attn_block.c - the device attention block against the reference's own
 * attention(), layer by layer, on the tiny checkpoint.
 *
 * TEST INFRASTRUCTURE ONLY. attention() is static in the reference
 * (src/model/dsv4_layer.c:213-336), so this driver #includes that file as it
 * lies under /root/reference and calls it directly; oracle/Makefile compiles
 * it with the reference's other model sources into oracle/_ref/dsv4_attn.
 * Nothing of the reference is copied.
 *
 * For every layer of the checkpoint (compress ratios 0, 4 with the indexer,
 * and 8), fresh layer state, positions 0 .. n-1, one seeded N(0,1) input per
 * position:
 *   pass 1: the reference's attention() with every matmul on its CPU path
 *           (nothing resident yet);
 *   pass 2: the layer's matrices made resident, dsv4_gpu_attn_bind, then
 *           dsv4_gpu_attn_step per position -- the whole block on the device.
 * Prints the vector-scaled relative error per layer and position and a
 * summary; exit 0 when every step is within --tol (default 1e-4), 1
 * otherwise, 2 when no GPU is available.
 *
 * A second mode runs the same comparison at the DeepSeek-V4-Flash shapes
 * (tests/fixtures/cfg/dsv4_flash_config.json: hidden 4096, 64 heads x 512,
 * RoPE 64, q_lora 1024, wo_a 8 groups x 1024, window 128, indexer 64 x 128
 * top 512) with synthetic random-init weights of those shapes (FP8 with
 * E8M0 128x128 scales, BF16 compressor and indexer weights), one layer of
 * the given compress ratio, and times the reference's attention() on the
 * host cores (its matmuls run OpenMP + AVX2 as built) beside the device
 * block's host-buffer call.
 *
 * usage: dsv4_attn CKPT_DIR [N_POSITIONS] [--tol T]
 *        dsv4_attn --flash N_POSITIONS RATIO [--tol T] [--topk K] [--cpu-only]
 * --cpu-only times the reference's attention() on the host cores and stops
 * before the device pass (the CPU baseline of bench.py).
 */
#include "dsv4_layer.c"

#include <omp.h>
#include <time.h>

#include "dsv4_cfg.h"
#include "dsv4_gpu.h"
#include "dsv4_st.h"

void dsv4_rope_table(float *cs, float *sn, int rd, int maxpos, int orig_ctx, double theta,
                     double factor, double beta_fast, double beta_slow);

/* splitmix64 -> Box-Muller: the inputs, reproducible per (layer, pos). */
static uint64_t sm64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void normal_vec(float *v, int n, uint64_t seed)
{
    uint64_t s = seed;
    for (int i = 0; i < n; i += 2) {
        const double u1 = ((sm64(&s) >> 11) + 1.0) / 9007199254740993.0;
        const double u2 = (sm64(&s) >> 11) / 9007199254740992.0;
        const double r = sqrt(-2.0 * log(u1));
        v[i] = (float)(r * cos(2.0 * M_PI * u2));
        if (i + 1 < n) v[i + 1] = (float)(r * sin(2.0 * M_PI * u2));
    }
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

static double now_s(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

/* A synthetic FP8 matrix: codes uniform over the 254 finite e4m3 codes,
 * E8M0 scales 2^e, e in -8..-4, per 128x128 block. */
static DSV4QMat syn_fp8(uint64_t *s, int rows, int cols)
{
    const int sr = (rows + 127) / 128, sc = (cols + 127) / 128;
    uint8_t *w = malloc((size_t)rows * cols), *sb = malloc((size_t)sr * sc);
    for (size_t i = 0; i < (size_t)rows * cols; i++) {
        uint8_t v = (uint8_t)(sm64(s) % 254u);
        w[i] = (uint8_t)(v + (v >= 127));
    }
    for (int i = 0; i < sr * sc; i++) sb[i] = (uint8_t)(127 - 4 - (int)(sm64(s) % 5u));
    DSV4QMat m = {w, sb, DSV4_WFP8, rows, cols, 128, 128};
    return m;
}

/* A synthetic BF16 matrix: N(0,1) * scale rounded to nearest even. */
static DSV4QMat syn_bf16(uint64_t seed, int rows, int cols, float scale)
{
    const size_t n = (size_t)rows * cols;
    float *f = malloc(n * sizeof(float));
    uint16_t *w = malloc(n * 2);
    normal_vec(f, (int)n, seed);
    for (size_t i = 0; i < n; i++) {
        union { float f; uint32_t u; } v = {f[i] * scale};
        w[i] = (uint16_t)((v.u + 0x7FFFu + ((v.u >> 16) & 1u)) >> 16);
    }
    free(f);
    DSV4QMat m = {w, NULL, DSV4_WBF16, rows, cols, 0, 0};
    return m;
}

static float *syn_vec(uint64_t seed, int n, float scale, float add)
{
    float *v = malloc((size_t)n * sizeof(float));
    normal_vec(v, n, seed);
    for (int i = 0; i < n; i++) v[i] = v[i] * scale + add;
    return v;
}

static int upload(const DSV4QMat *m);

static int flash_mode(int n, int ratio, double tol, int idx_topk, int cpu_only)
{
    static int cr[1];
    cr[0] = ratio;
    DSV4Cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = 4096; c.n_layers = 1; c.vocab = 129280; c.rms_eps = 1e-6f;
    c.max_pos = n + 16; c.n_heads = 64; c.n_kv_heads = 1; c.head_dim = 512;
    c.q_lora = 1024; c.o_lora = 1024; c.o_groups = 8; c.qk_rope = 64;
    c.sliding_window = 128; c.index_n_heads = 64; c.index_head_dim = 128;
    c.index_topk = idx_topk; c.n_compress = 1; c.compress_ratios = cr;
    c.compress_rope_theta = 160000.0f; c.hc_mult = 4; c.n_experts = 256; c.topk = 6;
    c.n_shared = 1; c.moe_inter = 2048; c.rope_theta = 10000.0f; c.yarn_factor = 16.0f;
    c.yarn_beta_fast = 32.0f; c.yarn_beta_slow = 1.0f; c.yarn_orig_ctx = 65536;
    c.wblock_m = c.wblock_n = 128;
    const int hd = c.head_dim, H = c.n_heads, coff = ratio == 4 ? 2 : 1;
    uint64_t sd = 0xF1A5Full;
    DSV4LayerW w;
    memset(&w, 0, sizeof w);
    w.layer = 0;
    w.compress_ratio = ratio;
    w.has_comp = ratio != 0;
    w.has_idx = ratio == 4;
    DSV4AttnW *a = &w.attn;
    a->wq_a = syn_fp8(&sd, c.q_lora, c.hidden);
    a->wq_b = syn_fp8(&sd, H * hd, c.q_lora);
    a->wkv = syn_fp8(&sd, hd, c.hidden);
    a->wo_a = syn_fp8(&sd, c.o_groups * c.o_lora, H * hd / c.o_groups);
    a->wo_b = syn_fp8(&sd, c.hidden, c.o_groups * c.o_lora);
    a->q_norm = syn_vec(11, c.q_lora, 0.1f, 1.0f);
    a->kv_norm = syn_vec(12, hd, 0.1f, 1.0f);
    a->sink = syn_vec(13, H, 1.0f, 0.0f);
    a->has_comp = w.has_comp;
    a->has_idx = w.has_idx;
    if (w.has_comp) {
        a->comp.ratio = ratio;
        a->comp.coff = coff;
        a->comp.ape = syn_vec(14, ratio * coff * hd, 0.5f, 0.0f);
        a->comp.norm = syn_vec(15, hd, 0.1f, 1.0f);
        a->comp.wkv = syn_bf16(16, coff * hd, c.hidden, 0.02f);
        a->comp.wgate = syn_bf16(17, coff * hd, c.hidden, 0.02f);
    }
    if (w.has_idx) {
        a->idx.wq_b = syn_fp8(&sd, c.index_n_heads * c.index_head_dim, c.q_lora);
        a->idx.weights_proj = syn_bf16(18, c.index_n_heads, c.hidden, 0.02f);
    }
    const int maxpos = c.max_pos, half = c.qk_rope / 2;
    float *cs = malloc((size_t)maxpos * half * 4), *sn = malloc((size_t)maxpos * half * 4);
    if (ratio)
        dsv4_rope_table(cs, sn, c.qk_rope, maxpos, c.yarn_orig_ctx, c.compress_rope_theta,
                        c.yarn_factor, c.yarn_beta_fast, c.yarn_beta_slow);
    else
        dsv4_rope_table(cs, sn, c.qk_rope, maxpos, 0, c.rope_theta, c.yarn_factor,
                        c.yarn_beta_fast, c.yarn_beta_slow);
    DSV4Scratch s;
    DSV4LayerState ls;
    if (dsv4_scratch_init(&s, &c, maxpos) != 0 || widen_scratch(&s, &c, maxpos) != 0 ||
        dsv4_state_init(&ls, &c, 0, maxpos) != 0)
        return 1;
    float *x = malloc((size_t)n * c.hidden * sizeof(float));
    float *ref = malloc((size_t)n * c.hidden * sizeof(float));
    float *got = malloc((size_t)c.hidden * sizeof(float));
    for (int p = 0; p < n; p++) normal_vec(x + (size_t)p * c.hidden, c.hidden, 0xF1A5ull * 7919 + p);
    /* the reference on the host: every matmul on its CPU path */
    double t_cpu = 0.0;
    int n_cpu = 0;
    for (int p = 0; p < n; p++) {
        const int n_idx = dsv4_window_idxs(s.idxs, p, c.sliding_window);
        const double t0 = now_s();
        attention(ref + (size_t)p * c.hidden, x + (size_t)p * c.hidden, &w, &c, &s, &ls, cs,
                  sn, p, n_idx);
        const double t1 = now_s();
        if (p >= 4) { t_cpu += t1 - t0; n_cpu++; }
    }
    if (cpu_only) {
        printf("flash: ratio %d positions %d cpu_ms_per_position %.3f threads %d\n", ratio, n,
               n_cpu ? 1e3 * t_cpu / n_cpu : 0.0, omp_get_max_threads());
        return 0;
    }
    if (!dsv4_gpu_available() || dsv4_gpu_init() != 0) {
        fprintf(stderr, "attn: no GPU\n");
        printf("flash: ratio %d positions %d cpu_ms_per_position %.3f threads %d\n", ratio, n,
               n_cpu ? 1e3 * t_cpu / n_cpu : 0.0, omp_get_max_threads());
        return 2;
    }
    const DSV4QMat *m[9] = {&a->wq_a, &a->wq_b, &a->wkv, &a->wo_a, &a->wo_b,
                            w.has_comp ? &a->comp.wkv : NULL, w.has_comp ? &a->comp.wgate : NULL,
                            w.has_idx ? &a->idx.wq_b : NULL,
                            w.has_idx ? &a->idx.weights_proj : NULL};
    for (int k = 0; k < 9; k++)
        if (upload(m[k]) < 0) { fprintf(stderr, "attn: flash upload %d\n", k); return 1; }
    dsv4_gpu_attn_cfg ac = {
        .hidden = c.hidden, .q_lora = c.q_lora, .n_heads = H, .head_dim = hd,
        .rope_dim = c.qk_rope, .window = c.sliding_window, .ratio = ratio,
        .idx_heads = w.has_idx ? c.index_n_heads : 0, .idx_dim = c.index_head_dim,
        .idx_topk = c.index_topk, .o_groups = c.o_groups, .o_lora = c.o_lora,
        .max_pos = maxpos, .rms_eps = c.rms_eps};
    dsv4_gpu_attn_w aw = {
        .wq_a = a->wq_a, .wq_b = a->wq_b, .wkv = a->wkv, .wo_a = a->wo_a, .wo_b = a->wo_b,
        .q_norm = a->q_norm, .kv_norm = a->kv_norm, .sink = a->sink, .rope_cos = cs,
        .rope_sin = sn};
    if (w.has_comp) {
        aw.comp_wkv = a->comp.wkv; aw.comp_wgate = a->comp.wgate;
        aw.comp_norm = a->comp.norm; aw.comp_ape = a->comp.ape;
    }
    if (w.has_idx) { aw.idx_wq_b = a->idx.wq_b; aw.idx_wproj = a->idx.weights_proj; }
    if (dsv4_gpu_attn_bind(0, &ac, &aw) != 0) { fprintf(stderr, "attn: flash bind\n"); return 1; }
    double worst = 0.0, t_gpu = 0.0;
    int bad = 0, n_gpu = 0;
    for (int p = 0; p < n; p++) {
        const double t0 = now_s();
        if (dsv4_gpu_attn_step(got, x + (size_t)p * c.hidden, 0, p) != 0) {
            fprintf(stderr, "attn: flash step %d failed\n", p);
            return 1;
        }
        const double t1 = now_s();
        if (p >= 4) { t_gpu += t1 - t0; n_gpu++; }
        const double r = vec_rel(got, ref + (size_t)p * c.hidden, c.hidden);
        printf("flash pos %d rel %.3g\n", p, r);
        if (r > worst) worst = r;
        bad += !(r <= tol);
    }
    printf("flash: ratio %d positions %d worst_rel %.3g over_tol %d tol %.3g "
           "cpu_ms_per_position %.3f threads %d gpu_host_call_us %.1f\n", ratio, n, worst, bad,
           tol, n_cpu ? 1e3 * t_cpu / n_cpu : 0.0, omp_get_max_threads(),
           n_gpu ? 1e6 * t_gpu / n_gpu : 0.0);
    dsv4_gpu_shutdown();
    return bad == 0 ? 0 : 1;
}

static int upload(const DSV4QMat *m)
{
    if (!m || !m->w) return 0;
    return dsv4_gpu_upload(m) == 0 ? 1 : -1;
}

int main(int argc, char **argv)
{
    if (argc < 2) {
        fprintf(stderr, "usage: %s CKPT_DIR [N_POSITIONS] [--tol T]\n"
                        "       %s --flash N_POSITIONS RATIO [--tol T] [--topk K] "
                        "[--cpu-only]\n",
                argv[0], argv[0]);
        return 1;
    }
    int n = 40;
    double tol = 1e-4;
    if (!strcmp(argv[1], "--flash")) {
        if (argc < 4) return 1;
        int idx_topk = 512;                     /* DeepSeek-V4-Flash's index_topk */
        int cpu_only = 0;
        for (int i = 4; i < argc; i++) {
            if (!strcmp(argv[i], "--cpu-only")) cpu_only = 1;
            else if (!strcmp(argv[i], "--tol") && i + 1 < argc) tol = atof(argv[++i]);
            else if (!strcmp(argv[i], "--topk") && i + 1 < argc) idx_topk = atoi(argv[++i]);
        }
        if (idx_topk <= 0) return 1;
        return flash_mode(atoi(argv[2]), atoi(argv[3]), tol, idx_topk, cpu_only);
    }
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--tol") && i + 1 < argc) tol = atof(argv[++i]);
        else n = atoi(argv[i]);
    }
    char path[1024];
    DSV4Cfg c;
    int cr[DSV4_MAX_LAYERS];
    snprintf(path, sizeof path, "%s/config.json", argv[1]);
    if (!dsv4_cfg_load_file(&c, cr, DSV4_MAX_LAYERS, path)) return 1;
    DSV4St st;
    if (dsv4_st_open(&st, argv[1]) != 0) return 1;
    DSV4LayerBind *lb = calloc((size_t)c.n_layers, sizeof *lb);
    for (int L = 0; L < c.n_layers; L++)
        if (dsv4_bind_layer(&st, &c, L, &lb[L]) != 0) return 1;

    const int maxpos = n + 16, half = c.qk_rope / 2, hd = c.head_dim;
    float *cs_d = malloc((size_t)maxpos * half * 4), *sn_d = malloc((size_t)maxpos * half * 4);
    float *cs_c = malloc((size_t)maxpos * half * 4), *sn_c = malloc((size_t)maxpos * half * 4);
    dsv4_rope_table(cs_d, sn_d, c.qk_rope, maxpos, 0, c.rope_theta, c.yarn_factor,
                    c.yarn_beta_fast, c.yarn_beta_slow);
    dsv4_rope_table(cs_c, sn_c, c.qk_rope, maxpos, c.yarn_orig_ctx, c.compress_rope_theta,
                    c.yarn_factor, c.yarn_beta_fast, c.yarn_beta_slow);
    DSV4Scratch s;
    if (dsv4_scratch_init(&s, &c, maxpos) != 0 || widen_scratch(&s, &c, maxpos) != 0) return 1;

    const size_t per = (size_t)n * c.hidden;
    float *x = malloc(per * c.n_layers * sizeof(float));
    float *ref = malloc(per * c.n_layers * sizeof(float));
    float *got = malloc(per * sizeof(float));
    if (!x || !ref || !got) return 1;
    for (int L = 0; L < c.n_layers; L++)
        for (int p = 0; p < n; p++)
            normal_vec(x + (size_t)L * per + (size_t)p * c.hidden, c.hidden,
                       0x5EEDull * 1000003ull + (uint64_t)L * 4096 + (uint64_t)p);

    /* pass 1: the reference, every matmul on the CPU */
    for (int L = 0; L < c.n_layers; L++) {
        const int comp = dsv4_compress_ratio(&c, L) != 0;
        DSV4LayerState ls;
        if (dsv4_state_init(&ls, &c, L, maxpos) != 0) return 1;
        for (int p = 0; p < n; p++) {
            const int n_idx = dsv4_window_idxs(s.idxs, p, c.sliding_window);
            attention(ref + (size_t)L * per + (size_t)p * c.hidden,
                      x + (size_t)L * per + (size_t)p * c.hidden, &lb[L].w, &c, &s, &ls,
                      comp ? cs_c : cs_d, comp ? sn_c : sn_d, p, n_idx);
        }
        dsv4_state_free(&ls);
    }

    /* pass 2: the block on the device */
    if (!dsv4_gpu_available() || dsv4_gpu_init() != 0) {
        fprintf(stderr, "attn: no GPU\n");
        return 2;
    }
    double worst_all = 0.0;
    int bad = 0, steps = 0;
    for (int L = 0; L < c.n_layers; L++) {
        const DSV4AttnW *a = &lb[L].w.attn;
        const int ratio = dsv4_compress_ratio(&c, L), comp = ratio != 0;
        const DSV4QMat *m[9] = {&a->wq_a, &a->wq_b, &a->wkv, &a->wo_a, &a->wo_b,
                                a->has_comp ? &a->comp.wkv : NULL,
                                a->has_comp ? &a->comp.wgate : NULL,
                                a->has_idx ? &a->idx.wq_b : NULL,
                                a->has_idx ? &a->idx.weights_proj : NULL};
        for (int k = 0; k < 9; k++)
            if (upload(m[k]) < 0) { fprintf(stderr, "attn: upload %d of layer %d\n", k, L); return 1; }
        dsv4_gpu_attn_cfg ac = {
            .hidden = c.hidden, .q_lora = c.q_lora, .n_heads = c.n_heads, .head_dim = hd,
            .rope_dim = c.qk_rope, .window = c.sliding_window, .ratio = ratio,
            .idx_heads = a->has_idx ? c.index_n_heads : 0, .idx_dim = c.index_head_dim,
            .idx_topk = c.index_topk, .o_groups = c.o_groups, .o_lora = c.o_lora,
            .max_pos = maxpos, .rms_eps = c.rms_eps};
        dsv4_gpu_attn_w aw = {
            .wq_a = a->wq_a, .wq_b = a->wq_b, .wkv = a->wkv, .wo_a = a->wo_a, .wo_b = a->wo_b,
            .q_norm = a->q_norm, .kv_norm = a->kv_norm, .sink = a->sink,
            .rope_cos = comp ? cs_c : cs_d, .rope_sin = comp ? sn_c : sn_d};
        if (a->has_comp) {
            aw.comp_wkv = a->comp.wkv; aw.comp_wgate = a->comp.wgate;
            aw.comp_norm = a->comp.norm; aw.comp_ape = a->comp.ape;
        }
        if (a->has_idx) { aw.idx_wq_b = a->idx.wq_b; aw.idx_wproj = a->idx.weights_proj; }
        if (dsv4_gpu_attn_bind(L, &ac, &aw) != 0) { fprintf(stderr, "attn: bind %d\n", L); return 1; }
        double worst = 0.0;
        for (int p = 0; p < n; p++) {
            if (dsv4_gpu_attn_step(got + (size_t)p * c.hidden,
                                   x + (size_t)L * per + (size_t)p * c.hidden, L, p) != 0) {
                fprintf(stderr, "attn: step layer %d pos %d failed\n", L, p);
                return 1;
            }
            const double r = vec_rel(got + (size_t)p * c.hidden,
                                     ref + (size_t)L * per + (size_t)p * c.hidden, c.hidden);
            printf("layer %d ratio %d pos %d rel %.3g\n", L, ratio, p, r);
            if (r > worst) worst = r;
            bad += !(r <= tol);
            steps++;
        }
        printf("layer %d ratio %d indexer %d: worst_rel %.3g over %d positions\n", L, ratio,
               a->has_idx, worst, n);
        if (worst > worst_all) worst_all = worst;
    }
    printf("summary: layers %d steps %d worst_rel %.3g over_tol %d tol %.3g\n", c.n_layers,
           steps, worst_all, bad, tol);
    dsv4_gpu_shutdown();
    return bad == 0 ? 0 : 1;
}
