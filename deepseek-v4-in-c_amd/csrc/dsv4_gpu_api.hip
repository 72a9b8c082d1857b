/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_gpu_api.hip - the C ABI of include/dsv4_gpu.h: device bring-up,
 * residency, staging, scratch and the entry points.
 *
 * Mirrors the reference backend's contract (src/cuda/dsv4_cuda.cu:232-469):
 * matrices resident in HBM keyed by their host weight pointer, activations
 * crossing through pinned host staging allocated once and reused (the
 * reference measured pageable copies cost CPU-side throughput 32x,
 * dsv4_cuda.cu:357-369), 0 / -1 for recoverable failures and abort() on a
 * contract violation. What differs is MI355X-first:
 *   - all work goes to one library stream at default priority; host-buffer
 *     calls are one H2D copy, the kernels, one D2H copy and a stream sync;
 *   - every input of a call shares one staging arena, so a call with several
 *     inputs still makes one H2D transfer;
 *   - the residency table resolves row-range views of a resident matrix;
 *   - routed experts and KV stores are resident too, keyed by (layer,
 *     expert) and by handle.
 */
#include "dsv4_internal.h"
#include "dsv4_dev.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <vector>

/* Scratch of dsv4_gpu_moe_fp4_noalloc_d: a fixed array in every device's
 * global memory, so that entry point allocates nothing. Host code never uses
 * the array's name as an address (on the host it is only a stand-in for the
 * symbol): dsv4_gpu_init looks up its device address once per device with
 * hipGetSymbolAddress and keeps it in g_static_scratch. */
#define DSV4_STATIC_SCRATCH_MAX (1u << 20)
#define DSV4_MAX_DEVICES 64
static __device__ __align__(256) unsigned char scratch[DSV4_STATIC_SCRATCH_MAX];
static void *g_static_scratch[DSV4_MAX_DEVICES];
/* The routed-expert pass's arrival counters (the one-launch form of
 * dsv4_moe_mx.hip): zero when the module loads, zero again after every
 * call, on every device; their device address is looked up once per
 * device, as for `scratch`. */
static __device__ __align__(256) uint32_t moe_sync[DSV4_MOE_SYNC_WORDS];
static void *g_moe_sync[DSV4_MAX_DEVICES];

namespace {

/* ------------------------------------------------------------- residency */
struct Res {
    const uint8_t *key, *key_end;   /* the caller's weight bytes [key, key_end):
                                       host memory for an upload, the device
                                       copy itself for a matrix loaded into
                                       HBM directly                          */
    const uint8_t *skey;            /* the caller's scale grid               */
    uint8_t *dw, *ds;
    void *own_w, *own_s;            /* device blocks freed at shutdown (or
                                       nullptr: owned elsewhere)             */
    int wdt;                        /* DSV4_WFP8, DSV4_WFP4 or DSV4_WBF16  */
    int rows, cols, blk_r, blk_c, sc, sfmt;
    size_t row_bytes() const
    {
        return wdt == DSV4_WFP4 ? (size_t)cols / 2
             : wdt == DSV4_WBF16 ? (size_t)cols * 2 : (size_t)cols;
    }
};

struct LayerExperts {
    std::vector<Dsv4ExpertDev> host;        /* by expert id              */
    std::vector<void *> owned;              /* device blocks we allocated */
    Dsv4ExpertDev *dev = nullptr;           /* device copy of `host`      */
    size_t dev_cap = 0;
    bool dirty = false;
    int hidden = 0, inter = 0;
};

struct Arena {
    char *h = nullptr, *d = nullptr;
    char *hd = nullptr;                 /* the device's address of h (mapped) */
    size_t cap = 0;
};

struct Scratch {
    void *p = nullptr;
    size_t cap = 0;
};

bool g_ready = false;
hipStream_t g_stream = nullptr;
/* Resident matrices by the start of their key range. Ranges never overlap
 * (registration refuses that), so the one that can hold a pointer p is the
 * last starting at or below p: an O(log n) lookup, which matters once every
 * routed expert matrix of a checkpoint is resident (Flash: 43 x 256 x 3). */
std::map<uintptr_t, Res> g_res;

/* The resident matrix whose key range holds p, or nullptr. */
const Res *res_at(const void *p)
{
    auto it = g_res.upper_bound((uintptr_t)p);
    if (it == g_res.begin()) return nullptr;
    --it;
    return (const uint8_t *)p < it->second.key_end ? &it->second : nullptr;
}

/* Add r unless its key range overlaps a resident one. */
int res_insert(const Res &r)
{
    const uintptr_t a = (uintptr_t)r.key, b = (uintptr_t)r.key_end;
    auto it = g_res.lower_bound(a);
    if (it != g_res.end() && it->first < b) return -1;
    if (it != g_res.begin()) {
        --it;
        if ((uintptr_t)it->second.key_end > a) return -1;
    }
    g_res.emplace(a, r);
    return 0;
}
std::vector<LayerExperts> g_layers;
Arena g_ar;
Scratch g_moe, g_attn, g_scores, g_index, g_amax, g_xsplit;

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

void attn_blocks_free();

int arena_reserve(size_t bytes)
{
    if (bytes <= g_ar.cap) return 0;
    size_t cap = g_ar.cap ? g_ar.cap : (1u << 20);
    while (cap < bytes) cap *= 2;
    HIP_OK(hipStreamSynchronize(g_stream), "sync before staging growth");
    if (g_ar.h) (void)hipHostFree(g_ar.h);
    if (g_ar.d) (void)hipFree(g_ar.d);
    g_ar.h = g_ar.d = nullptr;
    g_ar.cap = 0;
    /* coherent and mapped: kernels write outputs straight into it */
    HIP_OK(hipHostMalloc((void **)&g_ar.h, cap, hipHostMallocMapped | hipHostMallocCoherent),
           "hipHostMalloc staging");
    HIP_OK(hipHostGetDevicePointer((void **)&g_ar.hd, g_ar.h, 0), "staging device address");
    HIP_OK(hipMalloc((void **)&g_ar.d, cap), "hipMalloc staging");
    g_ar.cap = cap;
    return 0;
}

int scratch_reserve(Scratch &s, size_t bytes)
{
    if (bytes <= s.cap) return 0;
    /* A buffer may still be in use by stream-ordered work on any stream. */
    HIP_OK(hipDeviceSynchronize(), "sync before scratch growth");
    if (s.p) (void)hipFree(s.p);
    s.p = nullptr;
    s.cap = 0;
    HIP_OK(hipMalloc(&s.p, bytes), "hipMalloc scratch");
    /* Kernels that keep arrival counters in their scratch expect zeros on
     * first use (and leave zeros behind). */
    HIP_OK(hipMemset(s.p, 0, bytes), "hipMemset scratch");
    s.cap = bytes;
    return 0;
}

/* A staged host-buffer call: inputs are packed into the pinned arena and
 * moved to the device in one step; outputs come back in one step.
 *
 * By default the staging is zero-copy: one small kernel pulls the packed
 * inputs to the device through the arena's device mapping, and the call's
 * last kernel writes its outputs (plain stores, each written once, never
 * read back on the device) straight into the mapped arena, so no DMA
 * transfer is set up in either direction. Intermediate buffers stay in
 * device memory. DSV4_GPU_HOST_ZC=0 stages through two DMA copies instead
 * (hipMemcpyAsync H2D and D2H). */
struct Stage {
    size_t used = 0;
    struct In { const void *src; size_t off, bytes; };
    std::vector<In> ins;
    size_t add(size_t bytes) { const size_t o = used; used = align256(used + bytes); return o; }
    size_t in(const void *src, size_t bytes)
    {
        const size_t o = add(bytes);
        ins.push_back({src, o, bytes});
        return o;
    }
};

__global__ void __launch_bounds__(256) k_pull(u32x4 *__restrict__ dst,
                                              const u32x4 *__restrict__ src, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

/* read at each call, as the other switches are */
bool host_zc()
{
    const char *e = getenv("DSV4_GPU_HOST_ZC");
    return !(e && atoi(e) == 0);
}

/* where the call's last kernel writes an output at arena offset off */
char *out_at(size_t off) { return (host_zc() ? g_ar.hd : g_ar.d) + off; }

int stage_push(Stage &s, size_t *in_end)
{
    if (arena_reserve(s.used ? s.used : 256) != 0) return -1;
    size_t end = 0;
    for (const auto &i : s.ins) {
        memcpy(g_ar.h + i.off, i.src, i.bytes);
        end = i.off + i.bytes;
    }
    if (end && host_zc()) {
        const int n = (int)((end + 15) / 16);
        hipLaunchKernelGGL(k_pull, dim3((n + 255) / 256), dim3(256), 0, g_stream,
                           (u32x4 *)g_ar.d, (const u32x4 *)g_ar.hd, n);
        HIP_OK(hipGetLastError(), "staging pull");
    } else if (end) {
        HIP_OK(hipMemcpyAsync(g_ar.d, g_ar.h, end, hipMemcpyHostToDevice, g_stream),
               "H2D staging");
    }
    *in_end = end;
    return 0;
}

/* the output at arena offset off (written through out_at) into dst */
int stage_pull(size_t off, size_t bytes, void *dst)
{
    if (bytes && !host_zc())
        HIP_OK(hipMemcpyAsync(g_ar.h + off, g_ar.d + off, bytes,
                              hipMemcpyDeviceToHost, g_stream), "D2H staging");
    HIP_OK(hipStreamSynchronize(g_stream), "stream sync");
    if (bytes) memcpy(dst, g_ar.h + off, bytes);
    return 0;
}

/* A DSV4QMat resolved on the device: the resident matrix it lies in, and the
 * device addresses of its own first weight row and first scale-grid row. */
struct View {
    const Res *r = nullptr;
    const uint8_t *w = nullptr, *s = nullptr;
};

/* Resolve m: its weight pointer at a whole-row offset inside a resident
 * matrix of the same format, width and blocking, its rows inside that
 * matrix, and (FP8 / FP4) its scale pointer at a whole row of that matrix's
 * scale grid with its ceil(rows / blk_r) scale rows inside the grid. The
 * device then computes exactly what the reference's CPU kernel computes for
 * m: row r of m against scale row r / blk_r counted from m->s (dsv4_matmul.c:
 * 293-345). That covers attention()'s wo_a group slices whatever o_lora is
 * (dsv4_layer.c:321-334 offsets the scale pointer by g * (o_lora / blk_r)
 * grid rows). false if m resolves to nothing. */
bool find_view(const DSV4QMat *m, View *v)
{
    if (!m || !m->w || m->rows <= 0) return false;
    const uint8_t *p = (const uint8_t *)m->w;
    const Res *rp = res_at(p);
    if (!rp) return false;
    const Res &r = *rp;
    if (m->wdt != r.wdt || m->cols != r.cols) return false;
    const size_t off = (size_t)(p - r.key);
    if (off % r.row_bytes()) return false;
    const int row0 = (int)(off / r.row_bytes());
    if (row0 + m->rows > r.rows) return false;
    v->r = &r;
    v->w = r.dw + off;
    v->s = nullptr;
    if (r.wdt == DSV4_WBF16) return true;               /* no scales, no blocking */
    if (m->blk_r != r.blk_r || m->blk_c != r.blk_c || !m->s) return false;
    const size_t srow = (size_t)r.sc * (r.sfmt ? 4 : 1);  /* bytes per grid row */
    const uint8_t *sp = (const uint8_t *)m->s;
    if (sp < r.skey) return false;
    const size_t soff = (size_t)(sp - r.skey);
    if (soff % srow) return false;
    const size_t srow0 = soff / srow;
    const size_t grid_rows = (size_t)(r.rows + r.blk_r - 1) / r.blk_r;
    if (srow0 + (size_t)(m->rows + r.blk_r - 1) / r.blk_r > grid_rows) return false;
    v->s = r.ds + soff;
    return true;
}

/* Register m (the caller's key pointers m->w / m->s and logical shape) as
 * resident, its bytes at dw / ds in HBM; own_w / own_s are freed at
 * shutdown. -1 when its key range overlaps a resident one. */
int res_add(const DSV4QMat *m, int sfmt, uint8_t *dw, uint8_t *ds, void *own_w,
            void *own_s)
{
    Res r;
    const size_t wb = m->wdt == DSV4_WFP4 ? (size_t)m->rows * (size_t)m->cols / 2
                    : m->wdt == DSV4_WBF16 ? (size_t)m->rows * (size_t)m->cols * 2
                                          : (size_t)m->rows * (size_t)m->cols;
    r.key = (const uint8_t *)m->w;
    r.key_end = r.key + wb;
    r.skey = (const uint8_t *)m->s;
    r.dw = dw; r.ds = ds;
    r.own_w = own_w; r.own_s = own_s;
    r.wdt = m->wdt;
    r.rows = m->rows; r.cols = m->cols;
    r.blk_r = m->blk_r; r.blk_c = m->blk_c;
    r.sc = m->wdt == DSV4_WBF16 ? 0 : (m->cols + m->blk_c - 1) / m->blk_c;
    r.sfmt = sfmt;
    if (res_insert(r) != 0) {
        DSV4_ERR("a %dx%d matrix at %p overlaps a resident one", m->rows, m->cols, m->w);
        return -1;
    }
    return 0;
}

/* The shapes the device kernels take, per format. */
bool qmat_shape_ok(const DSV4QMat *m, int sfmt)
{
    if (!m || !m->w || m->rows <= 0 || m->cols <= 0) return false;
    if (m->wdt == DSV4_WBF16) return sfmt == 0 && dsv4_bf16_gemv_ok(m->rows, m->cols);
    if (!m->s || m->blk_r <= 0 || m->blk_c <= 0) return false;
    if (m->wdt == DSV4_WFP4)
        return sfmt == 0 && dsv4_fp4_gemv_ok(m->rows, m->cols, m->blk_r, m->blk_c);
    return m->wdt == DSV4_WFP8;
}

/* FP8 (sfmt 0: E8M0 scale bytes, 1: fp32), FP4 (E8M0 bytes) or BF16 (no
 * scales) matrices, copied from host memory. */
int upload_qmat(const DSV4QMat *m, int sfmt)
{
    if (!g_ready || !qmat_shape_ok(m, sfmt)) return -1;
    View v;
    if (find_view(m, &v)) return 0;             /* resident already (or a view of one) */
    const bool bf = m->wdt == DSV4_WBF16;
    const size_t wb = bf ? (size_t)m->rows * (size_t)m->cols * 2
                    : (size_t)m->rows * (size_t)m->cols / (m->wdt == DSV4_WFP4 ? 2 : 1);
    const int sc = bf ? 0 : (m->cols + m->blk_c - 1) / m->blk_c;
    const size_t sb = bf ? 0 : (size_t)((m->rows + m->blk_r - 1) / m->blk_r) * sc *
                               (sfmt ? 4u : 1u);
    if (wb + sb + (256u << 20) > dsv4_gpu_free_vram()) return -1;
    uint8_t *dw = nullptr, *ds = nullptr;
    if (hipMalloc((void **)&dw, wb) != hipSuccess) return -1;
    if (sb && hipMalloc((void **)&ds, sb) != hipSuccess) { (void)hipFree(dw); return -1; }
    if (hipMemcpy(dw, m->w, wb, hipMemcpyHostToDevice) != hipSuccess ||
        (sb && hipMemcpy(ds, m->s, sb, hipMemcpyHostToDevice) != hipSuccess) ||
        res_add(m, sfmt, dw, ds, dw, ds) != 0) {
        (void)hipFree(dw);
        if (ds) (void)hipFree(ds);
        return -1;
    }
    return 0;
}

/* y[rows] = the view's rows . x (x and y device pointers), on stream st.
 * A null st is the default stream, as in every stream-ordered entry point:
 * it is never replaced by the library's own stream, which is non-blocking
 * and so not ordered against the default stream. */
int res_gemv(const View &v, int rows, float *d_y, const float *d_x, hipStream_t st,
             bool valu = false)
{
    const Res &r = *v.r;
    if (r.wdt == DSV4_WBF16)
        return dsv4_bf16_gemv_launch(d_y, d_x, (const uint16_t *)v.w, rows, r.cols, st);
    if (r.wdt == DSV4_WFP4)
        return dsv4_fp4_gemv_launch(d_y, d_x, v.w, v.s, rows, r.cols, r.blk_r, r.blk_c, st);
    return dsv4_fp8_gemv_launch(d_y, d_x, v.w, v.s, r.sfmt, rows, r.cols, r.blk_r, r.blk_c,
                                st, valu);
}

/* --------------------------------------------------------------- experts */
bool expert_shape_ok(const DSV4ExpertW *e, int *hidden, int *inter)
{
    const DSV4QMat &a = e->w1, &b = e->w3, &c = e->w2;
    if (a.wdt != DSV4_WFP4 || b.wdt != DSV4_WFP4 || c.wdt != DSV4_WFP4) return false;
    if (!a.w || !a.s || !b.w || !b.s || !c.w || !c.s) return false;
    if (a.rows != b.rows || a.cols != b.cols) return false;
    if (c.rows != a.cols || c.cols != a.rows) return false;
    if (a.blk_r != 1 || a.blk_c != 32 || b.blk_r != 1 || b.blk_c != 32 ||
        c.blk_r != 1 || c.blk_c != 32)
        return false;
    if ((a.cols & 31) || (a.rows & 31)) return false;
    *hidden = a.cols;
    *inter = a.rows;
    return true;
}

LayerExperts *layer_slot(int layer, int expert)
{
    if (layer < 0 || expert < 0 || layer > 4096 || expert > (1 << 20)) return nullptr;
    if ((size_t)layer >= g_layers.size()) g_layers.resize(layer + 1);
    LayerExperts &L = g_layers[layer];
    if ((size_t)expert >= L.host.size()) L.host.resize(expert + 1, Dsv4ExpertDev{});
    return &L;
}

int layer_sync(LayerExperts &L)
{
    if (!L.dirty) return 0;
    const size_t bytes = L.host.size() * sizeof(Dsv4ExpertDev);
    if (bytes > L.dev_cap) {
        HIP_OK(hipDeviceSynchronize(), "sync before expert table growth");
        if (L.dev) (void)hipFree(L.dev);
        L.dev = nullptr;
        L.dev_cap = 0;
        HIP_OK(hipMalloc((void **)&L.dev, bytes * 2), "hipMalloc expert table");
        L.dev_cap = bytes * 2;
    }
    HIP_OK(hipMemcpy(L.dev, L.host.data(), bytes, hipMemcpyHostToDevice),
           "expert table copy");
    L.dirty = false;
    return 0;
}

int register_expert(int layer, int expert, const Dsv4ExpertDev &d, int hidden,
                    int inter, void *owned)
{
    LayerExperts *L = layer_slot(layer, expert);
    if (!L) return -1;
    /* the kernels read weights in 16-byte and scales in 4-byte pieces */
    if ((((uintptr_t)d.w1 | (uintptr_t)d.w3 | (uintptr_t)d.w2) & 15) ||
        (((uintptr_t)d.s1 | (uintptr_t)d.s3 | (uintptr_t)d.s2) & 3)) {
        DSV4_ERR("layer %d expert %d: weights must be 16-byte and scales 4-byte aligned",
                 layer, expert);
        return -1;
    }
    if ((L->hidden || L->inter) && (L->hidden != hidden || L->inter != inter)) {
        DSV4_ERR("layer %d expert %d is %dx%d but the layer's experts are %dx%d",
                 layer, expert, inter, hidden, L->inter, L->hidden);
        return -1;
    }
    L->hidden = hidden;
    L->inter = inter;
    L->host[expert] = d;
    if (owned) L->owned.push_back(owned);
    L->dirty = true;
    /* the device table follows every registration, so a MoE call never has
     * to copy (or grow) it -- the no-allocation entry point relies on that */
    return layer_sync(*L);
}

hipStream_t as_stream(void *s) { return (hipStream_t)s; }

/* ----------------------------------------------------------- decoder dumps */
__global__ void k_dump(float *out, int which, int e8m0)
{
    const int i = threadIdx.x;
    if (which == 4) out[i] = dec_e4m3_bf16((uint8_t)i, dec_e8m0((uint32_t)e8m0));
    else if (which == 0) out[i] = dec_e4m3((uint8_t)i);
    else if (which == 1) out[i] = dec_e8m0((uint32_t)i);
    else if (which == 2) {
        if (i < 16) {
            float o[2];
            dec_fp4x2<0>((uint32_t)i, o);               /* code i in the low nibble */
            out[i] = o[0];
        }
    } else {
        float o[8];
        dec_fp4x8((uint32_t)i, o);                      /* byte i in byte lane 0 */
        out[2 * i] = o[0];
        out[2 * i + 1] = o[1];
    }
}

int dump(float *host, int which, int count, int e8m0 = 127)
{
    if (!g_ready && dsv4_gpu_init() != 0) return -1;
    float *d = nullptr;
    HIP_OK(hipMalloc((void **)&d, 512 * sizeof(float)), "hipMalloc dump");
    hipLaunchKernelGGL(k_dump, dim3(1), dim3(256), 0, g_stream, d, which, e8m0);
    const hipError_t e = hipGetLastError();
    hipError_t c = hipSuccess;
    if (e == hipSuccess)
        c = hipMemcpyAsync(host, d, (size_t)count * sizeof(float),
                           hipMemcpyDeviceToHost, g_stream);
    const hipError_t s = hipStreamSynchronize(g_stream);
    (void)hipFree(d);
    if (e != hipSuccess || c != hipSuccess || s != hipSuccess) {
        DSV4_ERR("decoder dump failed");
        return -1;
    }
    return 0;
}

} // namespace

size_t dsv4_lds_limit(void)
{
    static size_t cached = 0;
    if (!cached) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
            v >= 64 * 1024)
            cached = (size_t)v;
        else
            cached = 64 * 1024;
    }
    return cached;
}

bool dsv4_lds_optin(const void *kernel, size_t bytes, const char *what)
{
    /* the dynamic allocation shares the workgroup's LDS with the kernel's
     * static arrays: ask for at most what they leave */
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, kernel) == hipSuccess) {
        const size_t lim = dsv4_lds_limit(), st = fa.sharedSizeBytes;
        if (bytes > (st < lim ? lim - st : 0)) bytes = st < lim ? lim - st : 0;
    } else {
        (void)hipGetLastError();
    }
    const hipError_t e =
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) return true;
    (void)hipGetLastError();
    DSV4_ERR("%s: dynamic LDS opt-in to %zu bytes refused: %s", what, bytes,
             hipGetErrorString(e));
    return false;
}

/* ===================================================================== ABI */
extern "C" {

int dsv4_gpu_available(void)
{
    int n = 0;
    return (hipGetDeviceCount(&n) == hipSuccess && n > 0) ? 1 : 0;
}

int dsv4_gpu_set_blocking_sync(void)
{
    HIP_OK(hipSetDeviceFlags(hipDeviceScheduleBlockingSync), "hipSetDeviceFlags");
    return 0;
}

int dsv4_gpu_init(void)
{
    if (g_ready) return 0;
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (n < 1) { DSV4_ERR("no device"); return -1; }
    HIP_OK(hipSetDevice(0), "hipSetDevice");
    hipDeviceProp_t p;
    HIP_OK(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
    size_t freeb = 0, totb = 0;
    HIP_OK(hipMemGetInfo(&freeb, &totb), "hipMemGetInfo");
    HIP_OK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking),
           "hipStreamCreate");
    /* the static scratch's address on this device (device 0 is current) */
    int dev = 0;
    HIP_OK(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= DSV4_MAX_DEVICES) { DSV4_ERR("device %d out of range", dev); return -1; }
    if (!g_static_scratch[dev]) {
        void *ptr = nullptr;
        HIP_OK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress scratch");
        g_static_scratch[dev] = ptr;
    }
    if (!g_moe_sync[dev]) {
        void *ptr = nullptr;
        HIP_OK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(moe_sync)), "hipGetSymbolAddress moe_sync");
        g_moe_sync[dev] = ptr;
    }
    printf("hip: %s (%s), %d CUs, %.2f GB free of %.2f GB\n", p.name,
           p.gcnArchName, p.multiProcessorCount, (double)freeb / 1073741824.0,
           (double)totb / 1073741824.0);
    fflush(stdout);
    g_ready = true;
    return 0;
}

size_t dsv4_gpu_free_vram(void)
{
    size_t freeb = 0, totb = 0;
    if (!g_ready || hipMemGetInfo(&freeb, &totb) != hipSuccess) return 0;
    return freeb;
}

void dsv4_gpu_shutdown(void)
{
    if (!g_ready) return;
    (void)hipDeviceSynchronize();
    for (auto &kv : g_res) {
        if (kv.second.own_w) (void)hipFree(kv.second.own_w);
        if (kv.second.own_s) (void)hipFree(kv.second.own_s);
    }
    g_res.clear();
    for (LayerExperts &L : g_layers) {
        for (void *p : L.owned) (void)hipFree(p);
        if (L.dev) (void)hipFree(L.dev);
    }
    g_layers.clear();
    attn_blocks_free();
    for (Scratch *s : {&g_moe, &g_attn, &g_scores, &g_index, &g_amax, &g_xsplit}) {
        if (s->p) (void)hipFree(s->p);
        s->p = nullptr;
        s->cap = 0;
    }
    if (g_ar.h) (void)hipHostFree(g_ar.h);
    if (g_ar.d) (void)hipFree(g_ar.d);
    g_ar = Arena{};
    if (g_stream) (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
    g_ready = false;
}

/* ------------------------------------------------------------------- FP8 */
int dsv4_gpu_upload(const DSV4QMat *m) { return upload_qmat(m, 0); }
int dsv4_gpu_upload_f32s(const DSV4QMat *m) { return upload_qmat(m, 1); }

int dsv4_gpu_has(const DSV4QMat *m)
{
    View v;
    return (g_ready && find_view(m, &v)) ? 1 : 0;
}

void dsv4_gpu_mmq(float *y, const float *x, const DSV4QMat *m)
{
    View v;
    const Res *r = (g_ready && find_view(m, &v)) ? v.r : nullptr;
    if (!r) {
        DSV4_ERR("mmq called for a matrix that is not resident");
        abort();
    }
    Stage s;
    const size_t xo = s.in(x, (size_t)r->cols * sizeof(float));
    const size_t yo = s.add((size_t)m->rows * sizeof(float));
    size_t end;
    if (stage_push(s, &end) != 0) abort();
    const int rc = res_gemv(v, m->rows, (float *)out_at(yo), (const float *)(g_ar.d + xo),
                            g_stream);
    if (rc != 0 || stage_pull(yo, (size_t)m->rows * sizeof(float), y) != 0) {
        DSV4_ERR("mmq failed");
        abort();
    }
}

void dsv4_gpu_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt)
{
    if (nt <= 1) { dsv4_gpu_mmq(y, x, m); return; }
    View v;
    const Res *r = (g_ready && find_view(m, &v)) ? v.r : nullptr;
    if (!r || nt > DSV4_MAX_BATCH) {
        DSV4_ERR("mmq_n called for a matrix that is not resident, or a batch "
                 "of %d above %d", nt, DSV4_MAX_BATCH);
        abort();
    }
    Stage s;
    const size_t xo = s.in(x, (size_t)nt * r->cols * sizeof(float));
    const size_t yo = s.add((size_t)nt * m->rows * sizeof(float));
    const bool fp8 = r->wdt != DSV4_WFP4 && r->wdt != DSV4_WBF16;
    const size_t to = fp8 ? s.add(dsv4_fp8_n_scratch_bytes(m->rows, r->cols, nt)) : 0;
    size_t end;
    if (stage_push(s, &end) != 0) abort();
    int rc = 0;
    /* one pass over the weights for the whole batch; per (row, token) the
     * single-token GEMV's own arithmetic */
    if (r->wdt == DSV4_WFP4) {
        rc = dsv4_fp4_gemv_n_launch((float *)out_at(yo), (const float *)(g_ar.d + xo),
                                    v.w, v.s, m->rows, r->cols, r->blk_r, r->blk_c, nt,
                                    g_stream);
    } else if (r->wdt == DSV4_WBF16) {
        rc = dsv4_bf16_gemv_n_launch((float *)out_at(yo), (const float *)(g_ar.d + xo),
                                     (const uint16_t *)v.w, m->rows, r->cols, nt, g_stream);
    } else {
        rc = dsv4_fp8_gemv_n_launch(
            (float *)out_at(yo), (const float *)(g_ar.d + xo),
            v.w, v.s, r->sfmt, m->rows, r->cols, r->blk_r, r->blk_c, nt, g_stream,
            g_ar.d + to);
    }
    if (rc != 0 ||
        stage_pull(yo, (size_t)nt * m->rows * sizeof(float), y) != 0) {
        DSV4_ERR("mmq_n failed");
        abort();
    }
}

int dsv4_gpu_fp8_gemv_d(float *d_y, const float *d_x, const uint8_t *d_w,
                        const void *d_s, int scale_fmt, int rows, int cols,
                        void *stream)
{
    if (!d_y || !d_x || !d_w || !d_s || (scale_fmt != 0 && scale_fmt != 1)) {
        DSV4_ERR("fp8_gemv_d: bad arguments");
        return -1;
    }
    return dsv4_fp8_gemv_launch(d_y, d_x, d_w, d_s, scale_fmt, rows, cols, 128,
                                128, as_stream(stream));
}

int dsv4_gpu_fp8_gemv_n_d(float *d_y, const float *d_x, const uint8_t *d_w,
                          const void *d_s, int scale_fmt, int rows, int cols, int nt,
                          void *stream)
{
    if (!d_y || !d_x || !d_w || !d_s || (scale_fmt != 0 && scale_fmt != 1) || nt < 1 ||
        nt > DSV4_MAX_BATCH) {
        DSV4_ERR("fp8_gemv_n_d: bad arguments (nt %d)", nt);
        return -1;
    }
    if (scratch_reserve(g_xsplit, dsv4_fp8_n_scratch_bytes(rows, cols, nt)) != 0) return -1;
    return dsv4_fp8_gemv_n_launch(d_y, d_x, d_w, d_s, scale_fmt, rows, cols, 128, 128, nt,
                                  as_stream(stream), g_xsplit.p);
}

int dsv4_gpu_fp4_gemv_d(float *d_y, const float *d_x, const uint8_t *d_w,
                        const uint8_t *d_s, int rows, int cols, int blk_r, int blk_c,
                        void *stream)
{
    if (!d_y || !d_x || !d_w || !d_s) {
        DSV4_ERR("fp4_gemv_d: bad arguments");
        return -1;
    }
    return dsv4_fp4_gemv_launch(d_y, d_x, d_w, d_s, rows, cols, blk_r, blk_c,
                                as_stream(stream));
}

int dsv4_gpu_fp4_gemv_n_d(float *d_y, const float *d_x, const uint8_t *d_w,
                          const uint8_t *d_s, int rows, int cols, int blk_r, int blk_c, int nt,
                          void *stream)
{
    if (!d_y || !d_x || !d_w || !d_s || nt < 1 || nt > DSV4_MAX_BATCH) {
        DSV4_ERR("fp4_gemv_n_d: bad arguments (nt %d)", nt);
        return -1;
    }
    return dsv4_fp4_gemv_n_launch(d_y, d_x, d_w, d_s, rows, cols, blk_r, blk_c, nt,
                                  as_stream(stream));
}

int dsv4_gpu_bf16_gemv_n_d(float *d_y, const float *d_x, const uint16_t *d_w, int rows,
                           int cols, int nt, void *stream)
{
    if (!d_y || !d_x || !d_w || nt < 1 || nt > DSV4_MAX_BATCH) {
        DSV4_ERR("bf16_gemv_n_d: bad arguments (nt %d)", nt);
        return -1;
    }
    return dsv4_bf16_gemv_n_launch(d_y, d_x, d_w, rows, cols, nt, as_stream(stream));
}

int dsv4_gpu_bf16_gemv_d(float *d_y, const float *d_x, const uint16_t *d_w, int rows,
                         int cols, void *stream)
{
    if (!d_y || !d_x || !d_w) {
        DSV4_ERR("bf16_gemv_d: bad arguments");
        return -1;
    }
    return dsv4_bf16_gemv_launch(d_y, d_x, d_w, rows, cols, as_stream(stream));
}

/* ----------------------------------------------------------------- head */
int dsv4_gpu_head_argmax(const float *x, const DSV4QMat *head)
{
    View v;
    const Res *r = (g_ready && find_view(head, &v)) ? v.r : nullptr;
    if (!r || !x) {
        DSV4_ERR("head_argmax: the head matrix is not resident");
        return -1;
    }
    if (scratch_reserve(g_amax, dsv4_argmax_scratch_bytes()) != 0) return -1;
    Stage s;
    const size_t xo = s.in(x, (size_t)r->cols * sizeof(float));
    const size_t lo = s.add((size_t)head->rows * sizeof(float));
    const size_t to = s.add(sizeof(int));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    if (res_gemv(v, head->rows, (float *)(g_ar.d + lo), (const float *)(g_ar.d + xo),
                 g_stream) != 0 ||
        dsv4_argmax_launch((int *)out_at(to), (const float *)(g_ar.d + lo), head->rows,
                           g_amax.p, g_stream) != 0)
        return -1;
    int tok = -1;
    if (stage_pull(to, sizeof(int), &tok) != 0) return -1;
    return tok;
}

int dsv4_gpu_argmax_d(int *d_out, const float *d_v, int n, void *stream)
{
    if (!g_ready || scratch_reserve(g_amax, dsv4_argmax_scratch_bytes()) != 0) return -1;
    return dsv4_argmax_launch(d_out, d_v, n, g_amax.p, as_stream(stream));
}

int dsv4_gpu_embed_row_d(float *d_dst, const void *d_table, int wdt, long long row,
                         int hidden, void *stream)
{
    return dsv4_embed_row_launch(d_dst, d_table, wdt, row, hidden, as_stream(stream));
}

/* ---------------------------------------------------------------- dumps */
int dsv4_gpu_dump_e4m3(float *host256) { return dump(host256, 0, 256); }
int dsv4_gpu_dump_e8m0(float *host256) { return dump(host256, 1, 256); }
int dsv4_gpu_dump_e2m1(float *host16) { return dump(host16, 2, 16); }
int dsv4_gpu_dump_fp4_bytes(float *host512) { return dump(host512, 3, 512); }
int dsv4_gpu_dump_e4m3_scaled(float *host256, int e8m0)
{
    if (e8m0 < 0 || e8m0 > 255) return -1;
    return dump(host256, 4, 256, e8m0);
}

/* -------------------------------------------------------------- experts */
int dsv4_gpu_upload_expert(int layer, int expert, const DSV4ExpertW *e)
{
    int hidden, inter;
    if (!g_ready || !e || !expert_shape_ok(e, &hidden, &inter)) return -1;
    const size_t wb13 = (size_t)inter * hidden / 2, sb13 = (size_t)inter * hidden / 32;
    const size_t wb2 = (size_t)hidden * inter / 2, sb2 = (size_t)hidden * inter / 32;
    const size_t o1 = 0, os1 = align256(o1 + wb13), o3 = align256(os1 + sb13),
                 os3 = align256(o3 + wb13), o2 = align256(os3 + sb13),
                 os2 = align256(o2 + wb2), total = align256(os2 + sb2);
    if (total + (256u << 20) > dsv4_gpu_free_vram()) return -1;
    uint8_t *blk = nullptr;
    if (hipMalloc((void **)&blk, total) != hipSuccess) return -1;
    const struct { size_t off; const void *src; size_t n; } parts[6] = {
        {o1, e->w1.w, wb13}, {os1, e->w1.s, sb13}, {o3, e->w3.w, wb13},
        {os3, e->w3.s, sb13}, {o2, e->w2.w, wb2}, {os2, e->w2.s, sb2}};
    for (const auto &pp : parts)
        if (hipMemcpy(blk + pp.off, pp.src, pp.n, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(blk);
            return -1;
        }
    LayerExperts *L = layer_slot(layer, expert);
    if (L && L->host[expert].w1) {
        /* Re-upload of the same key: keep the first copy (idempotent). */
        (void)hipFree(blk);
        return 0;
    }
    Dsv4ExpertDev d{blk + o1, blk + os1, blk + o3, blk + os3, blk + o2, blk + os2};
    if (register_expert(layer, expert, d, hidden, inter, blk) != 0) {
        (void)hipFree(blk);
        return -1;
    }
    return 0;
}

int dsv4_gpu_bind_expert_d(int layer, int expert, const DSV4ExpertW *e)
{
    int hidden, inter;
    if (!g_ready || !e || !expert_shape_ok(e, &hidden, &inter)) return -1;
    Dsv4ExpertDev d{(const uint8_t *)e->w1.w, (const uint8_t *)e->w1.s,
                    (const uint8_t *)e->w3.w, (const uint8_t *)e->w3.s,
                    (const uint8_t *)e->w2.w, (const uint8_t *)e->w2.s};
    return register_expert(layer, expert, d, hidden, inter, nullptr);
}

/* ------------------------------------------- matrices loaded into HBM */
} /* extern "C" */

int dsv4_res_adopt(const DSV4QMat *m, void *owned)
{
    if (!g_ready || !qmat_shape_ok(m, 0)) {
        DSV4_ERR("adopt: a %dx%d matrix of format %d is not one the kernels take",
                 m ? m->rows : 0, m ? m->cols : 0, m ? m->wdt : -1);
        return -1;
    }
    return res_add(m, 0, (uint8_t *)m->w, (uint8_t *)m->s, owned, nullptr);
}

int dsv4_expert_adopt(int layer, int expert, const DSV4ExpertW *e, void *owned)
{
    int hidden, inter;
    if (!g_ready || !e || !expert_shape_ok(e, &hidden, &inter)) return -1;
    if (dsv4_gpu_has_expert(layer, expert)) {
        DSV4_ERR("adopt: layer %d expert %d is registered already", layer, expert);
        return -1;
    }
    /* its three matrices resident too (keyed by their device addresses), so
     * the reference's dispatch reaches them one by one as expert_forward
     * does, besides the fused pass */
    int added = 0;
    const DSV4QMat *ms[3] = {&e->w1, &e->w3, &e->w2};
    for (; added < 3; added++)
        if (!qmat_shape_ok(ms[added], 0) ||
            res_add(ms[added], 0, (uint8_t *)ms[added]->w, (uint8_t *)ms[added]->s, nullptr,
                    nullptr) != 0)
            break;
    const Dsv4ExpertDev d{(const uint8_t *)e->w1.w, (const uint8_t *)e->w1.s,
                          (const uint8_t *)e->w3.w, (const uint8_t *)e->w3.s,
                          (const uint8_t *)e->w2.w, (const uint8_t *)e->w2.s};
    if (added == 3 && register_expert(layer, expert, d, hidden, inter, owned) == 0) return 0;
    for (int i = 0; i < added; i++) g_res.erase((uintptr_t)ms[i]->w);   /* roll back */
    return -1;
}

uint32_t *dsv4_moe_sync(void)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= DSV4_MAX_DEVICES) return nullptr;
    return (uint32_t *)g_moe_sync[dev];
}

/* Undo dsv4_res_adopt: the matrix keyed at `key` leaves the residency
 * table and its owned device blocks are freed (after the device drains, so
 * no kernel still reads them). 0, or -1 when nothing is resident there. */
int dsv4_res_release(const void *key)
{
    auto it = g_res.find((uintptr_t)key);
    if (!g_ready || it == g_res.end()) return -1;
    (void)hipDeviceSynchronize();
    if (it->second.own_w) (void)hipFree(it->second.own_w);
    if (it->second.own_s && it->second.own_s != it->second.own_w) (void)hipFree(it->second.own_s);
    g_res.erase(it);
    return 0;
}

/* Undo dsv4_expert_adopt: the expert's three matrices leave the residency
 * table, the layer's table forgets the expert, and the block it owned (the
 * one that starts at its w1, as the loader lays it out) is freed. */
int dsv4_expert_release(int layer, int expert)
{
    if (!dsv4_gpu_has_expert(layer, expert)) return -1;
    (void)hipDeviceSynchronize();
    LayerExperts &L = g_layers[layer];
    const Dsv4ExpertDev d = L.host[expert];
    for (const uint8_t *w : {d.w1, d.w3, d.w2}) g_res.erase((uintptr_t)w);
    for (size_t i = 0; i < L.owned.size(); i++)
        if (L.owned[i] == (const void *)d.w1) {
            (void)hipFree(L.owned[i]);
            L.owned.erase(L.owned.begin() + (long)i);
            break;
        }
    L.host[expert] = Dsv4ExpertDev{};
    L.dirty = true;
    return layer_sync(L);
}

extern "C" {

int dsv4_gpu_has_expert(int layer, int expert)
{
    if (!g_ready || layer < 0 || expert < 0 || (size_t)layer >= g_layers.size())
        return 0;
    const LayerExperts &L = g_layers[layer];
    return ((size_t)expert < L.host.size() && L.host[expert].w1) ? 1 : 0;
}

static int moe_prepare(int layer, int topk, int hidden, int inter,
                       LayerExperts **out)
{
    if (!g_ready || layer < 0 || (size_t)layer >= g_layers.size() || topk <= 0) {
        DSV4_ERR("moe: layer %d has no resident experts", layer);
        return -1;
    }
    LayerExperts &L = g_layers[layer];
    if (L.hidden != hidden || L.inter != inter) {
        DSV4_ERR("moe: layer %d experts are %dx%d, call asks %dx%d", layer,
                 L.inter, L.hidden, inter, hidden);
        return -1;
    }
    if (layer_sync(L) != 0) return -1;
    if (scratch_reserve(g_moe, dsv4_moe_scratch_bytes(topk, hidden, inter)) != 0)
        return -1;
    *out = &L;
    return 0;
}

int dsv4_gpu_moe_fp4(float *out, const float *x, int layer, const int *idx,
                     const float *w, int topk, int hidden, int inter,
                     float swiglu_limit)
{
    LayerExperts *L;
    if (moe_prepare(layer, topk, hidden, inter, &L) != 0) return -1;
    for (int k = 0; k < topk; k++)
        if (!dsv4_gpu_has_expert(layer, idx[k])) {
            DSV4_ERR("moe: layer %d expert %d (k = %d) is not resident", layer,
                     idx[k], k);
            return -1;
        }
    Stage s;
    const size_t xo = s.in(x, (size_t)hidden * sizeof(float));
    const size_t io = s.in(idx, (size_t)topk * sizeof(int));
    const size_t wo = s.in(w, (size_t)topk * sizeof(float));
    const size_t oo = s.add((size_t)hidden * sizeof(float));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    if (dsv4_moe_fp4_launch((float *)out_at(oo), (const float *)(g_ar.d + xo),
                            L->dev, (int)L->host.size(),
                            (const int *)(g_ar.d + io), (const float *)(g_ar.d + wo),
                            topk, hidden, inter, swiglu_limit, g_moe.p,
                            g_stream) != 0)
        return -1;
    return stage_pull(oo, (size_t)hidden * sizeof(float), out);
}

int dsv4_gpu_moe_fp4_d(float *d_out, const float *d_x, int layer,
                       const int *d_idx, const float *d_w, int topk,
                       int hidden, int inter, float swiglu_limit, void *stream)
{
    LayerExperts *L;
    if (moe_prepare(layer, topk, hidden, inter, &L) != 0) return -1;
    return dsv4_moe_fp4_launch(d_out, d_x, L->dev, (int)L->host.size(), d_idx,
                               d_w, topk, hidden, inter, swiglu_limit,
                               g_moe.p, as_stream(stream));
}

static int moen_tokenwise_env(void)
{
    const char *e = getenv("DSV4_GPU_MOEN_TOKENWISE");
    return e ? (atoi(e) != 0) : -1;
}

int dsv4_gpu_moe_fp4_n(float *out, const float *x, int layer, const int *idx,
                       const float *w, int nt, int topk, int hidden, int inter,
                       float swiglu_limit)
{
    LayerExperts *L;
    if (nt < 1 || nt > DSV4_MAX_BATCH || !out || !x || !idx || !w) {
        DSV4_ERR("moe_n: bad arguments (nt %d)", nt);
        return -1;
    }
    if (moe_prepare(layer, topk, hidden, inter, &L) != 0) return -1;
    for (int i = 0; i < nt * topk; i++)
        if (!dsv4_gpu_has_expert(layer, idx[i])) {
            DSV4_ERR("moe_n: layer %d expert %d (token %d, k = %d) is not resident", layer,
                     idx[i], i / topk, i % topk);
            return -1;
        }
    if (scratch_reserve(g_moe, dsv4_moe_n_scratch_bytes(nt, topk, hidden, inter)) != 0)
        return -1;
    Stage s;
    const size_t xo = s.in(x, (size_t)nt * hidden * sizeof(float));
    const size_t io = s.in(idx, (size_t)nt * topk * sizeof(int));
    const size_t wo = s.in(w, (size_t)nt * topk * sizeof(float));
    const size_t oo = s.add((size_t)nt * hidden * sizeof(float));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    /* With the routing in hand: when the batch's (token, k) pairs barely
     * share experts (distinct experts above 9 in 10 pairs), reading each
     * expert once saves next to nothing and the batched passes' per-unit
     * staging costs more (4 tokens, 31.1 of 32 pairs distinct: 167.1 us
     * batched against 152.5 us token by token), so the tokens go one by one
     * through the single-token kernels. Both give every token the same bits.
     * DSV4_GPU_MOEN_TOKENWISE: 1 always token by token, 0 never. */
    int tokenwise = moen_tokenwise_env();
    if (tokenwise < 0) {
        std::vector<int> seen(idx, idx + (size_t)nt * topk);
        std::sort(seen.begin(), seen.end());
        const size_t distinct = std::unique(seen.begin(), seen.end()) - seen.begin();
        tokenwise = nt > 1 && 10 * distinct > 9 * (size_t)nt * topk;
    }
    if (tokenwise) {
        for (int t = 0; t < nt; t++)
            if (dsv4_moe_fp4_launch((float *)out_at(oo) + (size_t)t * hidden,
                                    (const float *)(g_ar.d + xo) + (size_t)t * hidden, L->dev,
                                    (int)L->host.size(), (const int *)(g_ar.d + io) + t * topk,
                                    (const float *)(g_ar.d + wo) + t * topk, topk, hidden,
                                    inter, swiglu_limit, g_moe.p, g_stream) != 0)
                return -1;
    } else if (dsv4_moe_fp4_n_launch((float *)out_at(oo), (const float *)(g_ar.d + xo),
                                     L->dev, (int)L->host.size(), (const int *)(g_ar.d + io),
                                     (const float *)(g_ar.d + wo), nt, topk, hidden, inter,
                                     swiglu_limit, g_moe.p, g_stream) != 0) {
        return -1;
    }
    return stage_pull(oo, (size_t)nt * hidden * sizeof(float), out);
}

int dsv4_gpu_moe_fp4_n_d(float *d_out, const float *d_x, int layer, const int *d_idx,
                         const float *d_w, int nt, int topk, int hidden, int inter,
                         float swiglu_limit, void *stream)
{
    LayerExperts *L;
    if (nt < 1 || nt > DSV4_MAX_BATCH || !d_out || !d_x || !d_idx || !d_w) {
        DSV4_ERR("moe_n_d: bad arguments (nt %d)", nt);
        return -1;
    }
    if (moe_prepare(layer, topk, hidden, inter, &L) != 0) return -1;
    if (scratch_reserve(g_moe, dsv4_moe_n_scratch_bytes(nt, topk, hidden, inter)) != 0)
        return -1;
    return dsv4_moe_fp4_n_launch(d_out, d_x, L->dev, (int)L->host.size(), d_idx, d_w, nt,
                                 topk, hidden, inter, swiglu_limit, g_moe.p,
                                 as_stream(stream));
}

int dsv4_gpu_moe_fp4_noalloc_d(float *d_out, const float *d_x, int layer,
                               const int *d_idx, const float *d_w, int topk,
                               int hidden, int inter, float swiglu_limit,
                               void *stream)
{
    if (!g_ready || layer < 0 || (size_t)layer >= g_layers.size() || topk <= 0 ||
        !d_out || !d_x || !d_idx || !d_w) {
        DSV4_ERR("moe_noalloc: layer %d has no resident experts, or bad arguments", layer);
        return -1;
    }
    const LayerExperts &L = g_layers[layer];
    if (L.hidden != hidden || L.inter != inter) {
        DSV4_ERR("moe_noalloc: layer %d experts are %dx%d, call asks %dx%d", layer,
                 L.inter, L.hidden, inter, hidden);
        return -1;
    }
    if (L.dirty || !L.dev) {
        /* registration keeps the table current; only a failed copy leaves it stale */
        DSV4_ERR("moe_noalloc: layer %d's expert table is not on the device", layer);
        return -1;
    }
    const size_t need = dsv4_moe_scratch_bytes(topk, hidden, inter);
    if (need == 0 || need > DSV4_STATIC_SCRATCH_MAX) {
        DSV4_ERR("moe_noalloc: topk %d x %d x %d needs %zu bytes of scratch; the static "
                 "scratch holds %u", topk, inter, hidden, need, DSV4_STATIC_SCRATCH_MAX);
        return -1;
    }
    int dev = 0;
    HIP_OK(hipGetDevice(&dev), "hipGetDevice");
    void *ptr = (dev >= 0 && dev < DSV4_MAX_DEVICES) ? g_static_scratch[dev] : nullptr;
    if (!ptr) {
        DSV4_ERR("moe_noalloc: no static scratch on device %d (dsv4_gpu_init runs on "
                 "device 0)", dev);
        return -1;
    }
    /* the kernels overwrite every scratch byte they read (x's and h's term
     * planes) before reading it, so the previous call's contents need no
     * clearing */
    return dsv4_moe_fp4_launch(d_out, d_x, L.dev, (int)L.host.size(), d_idx, d_w, topk,
                               hidden, inter, swiglu_limit, ptr, as_stream(stream));
}

/* ------------------------------------------------------------ KV stores */
struct dsv4_gpu_kv {
    void *data;
    float *scales;
    int n_rows, row_dim, fmt;
    size_t esize;
};

dsv4_gpu_kv *dsv4_gpu_kv_create(int n_rows, int row_dim, int fmt)
{
    if (!g_ready || n_rows <= 0 || row_dim <= 0) return nullptr;
    size_t es;
    switch (fmt) {
    case DSV4_GPU_KV_F32: es = 4; break;
    case DSV4_GPU_KV_BF16: es = 2; break;
    case DSV4_GPU_KV_FP8: es = 1; break;
    default: DSV4_ERR("kv_create: unknown format %d", fmt); return nullptr;
    }
    dsv4_gpu_kv *kv = (dsv4_gpu_kv *)calloc(1, sizeof *kv);
    if (!kv) return nullptr;
    kv->n_rows = n_rows; kv->row_dim = row_dim; kv->fmt = fmt; kv->esize = es;
    if (hipMalloc(&kv->data, (size_t)n_rows * row_dim * es) != hipSuccess) {
        free(kv);
        return nullptr;
    }
    if (fmt == DSV4_GPU_KV_FP8 &&
        hipMalloc((void **)&kv->scales, (size_t)n_rows * sizeof(float)) != hipSuccess) {
        (void)hipFree(kv->data);
        free(kv);
        return nullptr;
    }
    return kv;
}

int dsv4_gpu_kv_write_rows(dsv4_gpu_kv *kv, int row0, int n, const void *rows,
                           const float *row_scales)
{
    if (!kv || row0 < 0 || n < 0 || row0 + n > kv->n_rows || (n && !rows)) return -1;
    if (kv->fmt == DSV4_GPU_KV_FP8 && n && !row_scales) return -1;
    const size_t rb = (size_t)kv->row_dim * kv->esize;
    HIP_OK(hipMemcpy((char *)kv->data + (size_t)row0 * rb, rows, (size_t)n * rb,
                     hipMemcpyHostToDevice), "kv write");
    if (kv->fmt == DSV4_GPU_KV_FP8 && n)
        HIP_OK(hipMemcpy(kv->scales + row0, row_scales, (size_t)n * sizeof(float),
                         hipMemcpyHostToDevice), "kv scale write");
    return 0;
}

void *dsv4_gpu_kv_data(const dsv4_gpu_kv *kv) { return kv ? kv->data : nullptr; }
float *dsv4_gpu_kv_scales(const dsv4_gpu_kv *kv) { return kv ? kv->scales : nullptr; }

void dsv4_gpu_kv_free(dsv4_gpu_kv *kv)
{
    if (!kv) return;
    (void)hipDeviceSynchronize();
    (void)hipFree(kv->data);
    if (kv->scales) (void)hipFree(kv->scales);
    free(kv);
}

/* Key rows [row0 + t] read at element offset row0*row_dim + t*key_stride. */
static int key_view(const dsv4_gpu_kv *keys, int row0, int key_stride, int D,
                    int n, const void **base, const float **sc)
{
    if (!keys || row0 < 0 || n < 0 || D <= 0 || key_stride < D) return -1;
    if (keys->fmt == DSV4_GPU_KV_FP8 && key_stride != keys->row_dim) {
        DSV4_ERR("indexer: FP8 keys carry one scale per stored row; the key "
                 "stride must equal the row width");
        return -1;
    }
    const size_t start = (size_t)row0 * keys->row_dim;
    const size_t need = n ? start + (size_t)(n - 1) * key_stride + D : start;
    if (need > (size_t)keys->n_rows * keys->row_dim) {
        DSV4_ERR("indexer: %d keys at stride %d from row %d overrun the store",
                 n, key_stride, row0);
        return -1;
    }
    *base = (const char *)keys->data + start * keys->esize;
    *sc = keys->scales ? keys->scales + row0 : nullptr;
    return 0;
}

static float indexer_scale(int D, int H)
{
    return (1.0f / sqrtf((float)D)) * (1.0f / sqrtf((float)H));
}

int dsv4_gpu_indexer_score(float *out, const float *q, const float *w, int H,
                           int D, const dsv4_gpu_kv *keys, int row0,
                           int key_stride, int n)
{
    const void *kb;
    const float *ks;
    if (!g_ready || key_view(keys, row0, key_stride, D, n, &kb, &ks) != 0) return -1;
    if (n == 0) return 0;
    Stage s;
    const size_t qo = s.in(q, (size_t)H * D * sizeof(float));
    const size_t wo = s.in(w, (size_t)H * sizeof(float));
    const size_t oo = s.add((size_t)n * sizeof(float));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    if (dsv4_indexer_score_launch((float *)out_at(oo), (const float *)(g_ar.d + qo),
                                  (const float *)(g_ar.d + wo), H, D, kb, ks,
                                  keys->fmt, key_stride, n, indexer_scale(D, H),
                                  nullptr, 0, g_stream) != 0)
        return -1;
    return stage_pull(oo, (size_t)n * sizeof(float), out);
}

int dsv4_gpu_topk(int *idxs, const float *scores, int n, int k)
{
    if (!g_ready || n < 0) return -1;
    if (k > n) k = n;
    if (k <= 0) return k < 0 ? -1 : 0;
    if (scratch_reserve(g_index, dsv4_index_scratch_bytes(n)) != 0) return -1;
    Stage s;
    const size_t so = s.in(scores, (size_t)n * sizeof(float));
    const size_t io = s.add((size_t)k * sizeof(int));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    if (dsv4_topk_launch((int *)out_at(io), (const float *)(g_ar.d + so), n, k,
                         g_index.p, 0, g_stream) != 0)
        return -1;
    if (stage_pull(io, (size_t)k * sizeof(int), idxs) != 0) return -1;
    return k;
}

int dsv4_gpu_indexer_topk(int *idxs, const float *q, const float *w, int H,
                          int D, const dsv4_gpu_kv *keys, int row0,
                          int key_stride, int n, int k)
{
    const void *kb;
    const float *ks;
    if (!g_ready || key_view(keys, row0, key_stride, D, n, &kb, &ks) != 0) return -1;
    if (k > n) k = n;
    if (k <= 0) return k < 0 ? -1 : 0;
    if (scratch_reserve(g_index, dsv4_index_scratch_bytes(n)) != 0) return -1;
    const int hist = dsv4_topk_takes_hist(n, k);
    Stage s;
    const size_t qo = s.in(q, (size_t)H * D * sizeof(float));
    const size_t wo = s.in(w, (size_t)H * sizeof(float));
    const size_t so = s.add((size_t)n * sizeof(float));
    const size_t io = s.add((size_t)k * sizeof(int));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    if (dsv4_indexer_score_launch((float *)(g_ar.d + so), (const float *)(g_ar.d + qo),
                                  (const float *)(g_ar.d + wo), H, D, kb, ks,
                                  keys->fmt, key_stride, n, indexer_scale(D, H),
                                  g_index.p, hist, g_stream) != 0 ||
        dsv4_topk_launch((int *)out_at(io), (const float *)(g_ar.d + so), n, k,
                         g_index.p, hist, g_stream) != 0)
        return -1;
    if (stage_pull(io, (size_t)k * sizeof(int), idxs) != 0) return -1;
    return k;
}

int dsv4_gpu_sparse_attn(float *o, const float *q, const dsv4_gpu_kv *kv,
                         const float *sink, const int *idxs, int h, int d_qk,
                         int d_v, int topk, float scale)
{
    if (!g_ready || !kv || h <= 0 || topk < 0 || d_qk > kv->row_dim ||
        d_v > kv->row_dim || kv->fmt == DSV4_GPU_KV_FP8)
        return -1;
    for (int j = 0; j < topk; j++)
        if (idxs[j] >= kv->n_rows) {
            DSV4_ERR("sparse attn: slot %d selects row %d of %d", j, idxs[j],
                     kv->n_rows);
            return -1;
        }
    if (scratch_reserve(g_attn, dsv4_attn_scratch_bytes(h, d_qk, d_v, topk, kv->fmt) + 4) != 0)
        return -1;
    Stage s;
    const size_t qo = s.in(q, (size_t)h * d_qk * sizeof(float));
    const size_t so = sink ? s.in(sink, (size_t)h * sizeof(float)) : 0;
    const size_t io = topk ? s.in(idxs, (size_t)topk * sizeof(int)) : s.add(sizeof(int));
    const size_t oo = s.add((size_t)h * d_v * sizeof(float));
    size_t end;
    if (stage_push(s, &end) != 0) return -1;
    if (dsv4_attn_launch((float *)out_at(oo), (const float *)(g_ar.d + qo),
                         kv->data, kv->fmt, kv->row_dim, kv->n_rows,
                         sink ? (const float *)(g_ar.d + so) : nullptr,
                         (const int *)(g_ar.d + io), h, d_qk, d_v, topk, scale,
                         g_attn.p, g_stream) != 0)
        return -1;
    return stage_pull(oo, (size_t)h * d_v * sizeof(float), o);
}

int dsv4_gpu_indexer_score_d(float *d_out, const float *d_q, const float *d_w,
                             int H, int D, const void *d_keys,
                             const float *d_key_scales, int key_fmt,
                             int key_stride, int n, float scale, void *stream)
{
    if (!g_ready) return -1;
    return dsv4_indexer_score_launch(d_out, d_q, d_w, H, D, d_keys, d_key_scales,
                                     key_fmt, key_stride, n, scale, nullptr, 0,
                                     as_stream(stream));
}

int dsv4_gpu_topk_d(int *d_idxs, const float *d_scores, int n, int k,
                    void *stream)
{
    if (!g_ready || scratch_reserve(g_index, dsv4_index_scratch_bytes(n)) != 0)
        return -1;
    return dsv4_topk_launch(d_idxs, d_scores, n, k, g_index.p, 0, as_stream(stream));
}

int dsv4_gpu_sparse_attn_d(float *d_o, const float *d_q, const void *d_kv,
                           int kv_fmt, int kv_stride, int kv_rows,
                           const float *d_sink, const int *d_idxs, int h,
                           int d_qk, int d_v, int topk, float scale,
                           void *stream)
{
    if (!g_ready) return -1;
    if (scratch_reserve(g_attn, dsv4_attn_scratch_bytes(h, d_qk, d_v, topk, kv_fmt) + 4) != 0)
        return -1;
    return dsv4_attn_launch(d_o, d_q, d_kv, kv_fmt, kv_stride, kv_rows, d_sink,
                            d_idxs, h, d_qk, d_v, topk, scale, g_attn.p,
                            as_stream(stream));
}

int dsv4_gpu_mla_decode_d(float *d_o, int *d_idxs,
                          const float *d_q_idx, const float *d_w_idx, int H,
                          int D, const void *d_keys, const float *d_key_scales,
                          int key_fmt, int key_stride, int n, int k,
                          const float *d_q, const void *d_kv, int kv_fmt,
                          int kv_stride, int kv_rows, const float *d_sink,
                          int h, int d_qk, int d_v, float attn_scale,
                          void *stream)
{
    if (!g_ready) return -1;
    if (k > n) k = n;
    if (k < 0) return -1;
    hipStream_t st = as_stream(stream);
    if (H <= 0 || D <= 0 ||
        scratch_reserve(g_scores, (size_t)(n > 0 ? n : 1) * sizeof(float)) != 0 ||
        scratch_reserve(g_index, dsv4_index_scratch_bytes(n)) != 0 ||
        scratch_reserve(g_attn, dsv4_attn_scratch_bytes(h, d_qk, d_v, k, kv_fmt) + 4) != 0)
        return -1;
    const int hist = dsv4_topk_takes_hist(n, k);
    if (n > 0 &&
        (dsv4_indexer_score_launch((float *)g_scores.p, d_q_idx, d_w_idx, H, D,
                                   d_keys, d_key_scales, key_fmt, key_stride, n,
                                   indexer_scale(D, H), g_index.p, hist, st) != 0 ||
         dsv4_topk_launch(d_idxs, (const float *)g_scores.p, n, k, g_index.p, hist,
                          st) != 0))
        return -1;
    return dsv4_attn_launch(d_o, d_q, d_kv, kv_fmt, kv_stride, kv_rows, d_sink,
                            d_idxs, h, d_qk, d_v, k, attn_scale, g_attn.p, st);
}

} /* extern "C" */

/* ===================================================== attention blocks */
namespace {

/* A resident matrix (or a row range of one) as a block reads it. */
struct MatRef {
    Res r{};
    const uint8_t *w = nullptr, *s = nullptr;   /* device: its first row / scale row */
    View view() const
    {
        View v;
        v.r = &r;
        v.w = w;
        v.s = s;
        return v;
    }
};

int mat_ref(const DSV4QMat *m, int rows, int cols, MatRef *out, const char *what)
{
    View v;
    if (!m || !find_view(m, &v) || m->rows != rows || m->cols != cols) {
        DSV4_ERR("attn_bind: %s (%dx%d) is not a resident %dx%d matrix", what,
                 m ? m->rows : 0, m ? m->cols : 0, rows, cols);
        return -1;
    }
    out->r = *v.r;
    out->w = v.w;
    out->s = v.s;
    return 0;
}

/* One layer's attention on the device: its cfg, its resident matrices, and
 * one device allocation holding the small weights, the RoPE table, the
 * state (KV cache = window ring then compressed rows; the compressor's
 * slots) and the step's buffers. */
struct AttnBlock {
    bool bound = false;
    dsv4_gpu_attn_cfg c{};
    MatRef wq_a, wq_b, wkv, wo_a, wo_b, cwkv, cwgate, iwq_b, iwproj;
    char *mem = nullptr;
    float *q_norm = nullptr, *kv_norm = nullptr, *sink = nullptr, *comp_norm = nullptr;
    float *ape = nullptr, *cs = nullptr, *sn = nullptr;
    float *kv_cache = nullptr, *comp_kv = nullptr, *comp_score = nullptr;
    float *x = nullptr, *qr = nullptr, *q = nullptr, *kv = nullptr, *ckv = nullptr;
    float *csc = nullptr, *idx_q = nullptr, *idx_w = nullptr;
    float *scores = nullptr, *o = nullptr, *ogrp = nullptr, *out = nullptr;
    int *idxs = nullptr;
    void *iscr = nullptr, *ascr = nullptr;
    int max_comp = 0, width = 0, nslot = 0, n_comp = 0, next_pos = 0;
};
std::vector<AttnBlock> g_blocks;

void block_free(AttnBlock &b)
{
    if (b.mem) (void)hipFree(b.mem);
    b = AttnBlock{};
}

/* Back to position 0: an empty ring, no compressed rows, score slots at
 * -inf (dsv4_compress.c:75). */
int block_reset(AttnBlock &b)
{
    /* the state may still be in use on any stream a caller stepped it on */
    HIP_OK(hipDeviceSynchronize(), "attn reset sync");
    const size_t kvb = (size_t)(b.c.window + b.max_comp) * b.c.head_dim * sizeof(float);
    HIP_OK(hipMemset(b.kv_cache, 0, kvb), "attn reset");
    if (b.nslot) {
        const size_t n = (size_t)b.nslot * b.width;
        std::vector<float> ninf(n, -INFINITY);
        HIP_OK(hipMemset(b.comp_kv, 0, n * sizeof(float)), "attn reset");
        HIP_OK(hipMemcpy(b.comp_score, ninf.data(), n * sizeof(float), hipMemcpyHostToDevice),
               "attn reset");
    }
    b.n_comp = 0;
    b.next_pos = 0;
    return 0;
}

int block_bind(int layer, const dsv4_gpu_attn_cfg *cp, const dsv4_gpu_attn_w *w)
{
    if (!g_ready || !cp || !w || layer < 0 || layer >= 4096) return -1;
    const dsv4_gpu_attn_cfg c = *cp;
    const int H = c.n_heads, hd = c.head_dim, rd = c.rope_dim;
    const bool comp = c.ratio > 0, idx = c.idx_heads > 0;
    if (c.hidden <= 0 || c.q_lora <= 0 || H <= 0 || hd <= 0 || rd < 0 || rd > hd ||
        (rd & 1) || c.window <= 0 || c.ratio < 0 || c.max_pos <= 0 || c.o_groups <= 0 ||
        c.o_lora <= 0 || (H * hd) % c.o_groups ||
        (idx && (!comp || c.idx_dim < rd || c.idx_dim > hd || c.idx_topk <= 0)) ||
        !w->q_norm || !w->kv_norm || !w->rope_cos || !w->rope_sin ||
        (comp && (!w->comp_norm || !w->comp_ape))) {
        DSV4_ERR("attn_bind: layer %d: inconsistent configuration or missing vectors", layer);
        return -1;
    }
    AttnBlock b;
    b.c = c;
    const int gw = H * hd / c.o_groups, coff = c.ratio == 4 ? 2 : 1;
    if (mat_ref(&w->wq_a, c.q_lora, c.hidden, &b.wq_a, "wq_a") ||
        mat_ref(&w->wq_b, H * hd, c.q_lora, &b.wq_b, "wq_b") ||
        mat_ref(&w->wkv, hd, c.hidden, &b.wkv, "wkv") ||
        mat_ref(&w->wo_a, c.o_groups * c.o_lora, gw, &b.wo_a, "wo_a") ||
        mat_ref(&w->wo_b, c.hidden, c.o_groups * c.o_lora, &b.wo_b, "wo_b") ||
        (comp && (mat_ref(&w->comp_wkv, coff * hd, c.hidden, &b.cwkv, "comp wkv") ||
                  mat_ref(&w->comp_wgate, coff * hd, c.hidden, &b.cwgate, "comp wgate"))) ||
        (idx && (mat_ref(&w->idx_wq_b, c.idx_heads * c.idx_dim, c.q_lora, &b.iwq_b, "idx wq_b") ||
                 mat_ref(&w->idx_wproj, c.idx_heads, c.hidden, &b.iwproj, "idx weights_proj"))))
        return -1;
    if (b.wo_a.r.wdt != DSV4_WFP8) {
        DSV4_ERR("attn_bind: wo_a must be FP8 (its group slices)");
        return -1;
    }
    b.max_comp = comp ? c.max_pos / c.ratio + 1 : 0;
    b.width = comp ? coff * hd : 0;
    b.nslot = comp ? coff * c.ratio : 0;
    const int half = rd / 2, rows = c.window + b.max_comp;
    const size_t ascr = dsv4_attn_scratch_bytes(H, hd, hd, rows, DSV4_GPU_KV_F32);
    if (!ascr) {
        DSV4_ERR("attn_bind: head_dim %d not supported by the sparse attention", hd);
        return -1;
    }
    /* Refuse here what a step could not run: a step changes the layer's
     * state (ring slot, compressor slots, compressed rows) before its last
     * launches, so a refusal part way through would leave the state ahead of
     * the position. */
    if (idx && c.idx_topk > dsv4_topk_kmax()) {
        DSV4_ERR("attn_bind: index_topk %d above the device top-k's %d", c.idx_topk,
                 dsv4_topk_kmax());
        return -1;
    }
    if (rows > dsv4_attn_max_rows(DSV4_GPU_KV_F32, hd, hd)) {
        DSV4_ERR("attn_bind: window + max_pos / ratio + 1 = %d rows above the sparse "
                 "attention's %d", rows, dsv4_attn_max_rows(DSV4_GPU_KV_F32, hd, hd));
        return -1;
    }
    if (comp && hd > 1024) {
        DSV4_ERR("attn_bind: head_dim %d: the compressor's close takes at most 1024 "
                 "channels", hd);
        return -1;
    }
    const size_t F = sizeof(float);
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(bytes ? bytes : 4); return o; };
    const size_t o_qn = take(c.q_lora * F), o_kn = take(hd * F), o_sink = take(H * F);
    const size_t o_cn = take(comp ? hd * F : 0), o_ape = take((size_t)c.ratio * b.width * F);
    const size_t o_cs = take((size_t)c.max_pos * half * F), o_sn = take((size_t)c.max_pos * half * F);
    const size_t o_kv = take((size_t)rows * hd * F);
    const size_t o_ckv = take((size_t)b.nslot * b.width * F), o_csc = take((size_t)b.nslot * b.width * F);
    const size_t o_x = take(c.hidden * F), o_qr = take(c.q_lora * F), o_q = take((size_t)H * hd * F);
    const size_t o_k = take(hd * F), o_ki = take(b.width * F), o_si = take(b.width * F);
    const size_t o_iq = take((size_t)c.idx_heads * c.idx_dim * F);
    const size_t o_iw = take(c.idx_heads * F), o_sc = take((size_t)b.max_comp * F);
    const size_t o_o = take((size_t)H * hd * F), o_og = take((size_t)c.o_groups * c.o_lora * F);
    const size_t o_out = take(c.hidden * F), o_ix = take((size_t)rows * sizeof(int));
    const size_t o_is = take(idx ? dsv4_index_scratch_bytes(b.max_comp) : 0);
    const size_t o_as = take(ascr + 4);
    if (off + (64u << 20) > dsv4_gpu_free_vram() ||
        hipMalloc((void **)&b.mem, off) != hipSuccess) {
        DSV4_ERR("attn_bind: layer %d: no room for %zu bytes", layer, off);
        return -1;
    }
    char *m = b.mem;
    b.q_norm = (float *)(m + o_qn); b.kv_norm = (float *)(m + o_kn); b.sink = (float *)(m + o_sink);
    b.comp_norm = (float *)(m + o_cn); b.ape = (float *)(m + o_ape);
    b.cs = (float *)(m + o_cs); b.sn = (float *)(m + o_sn);
    b.kv_cache = (float *)(m + o_kv); b.comp_kv = (float *)(m + o_ckv); b.comp_score = (float *)(m + o_csc);
    b.x = (float *)(m + o_x); b.qr = (float *)(m + o_qr); b.q = (float *)(m + o_q);
    b.kv = (float *)(m + o_k); b.ckv = (float *)(m + o_ki); b.csc = (float *)(m + o_si);
    b.idx_q = (float *)(m + o_iq); b.idx_w = (float *)(m + o_iw);
    b.scores = (float *)(m + o_sc); b.o = (float *)(m + o_o); b.ogrp = (float *)(m + o_og);
    b.out = (float *)(m + o_out); b.idxs = (int *)(m + o_ix);
    b.iscr = m + o_is; b.ascr = m + o_as;
    /* the top-k's histogram and counters expect zeros on first use (and
     * leave zeros behind) */
    if (hipMemset(b.mem, 0, off) != hipSuccess) {
        DSV4_ERR("attn_bind: layer %d: clearing the block failed", layer);
        block_free(b);
        return -1;
    }
    bool ok = hipMemcpy(b.q_norm, w->q_norm, c.q_lora * F, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(b.kv_norm, w->kv_norm, hd * F, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(b.cs, w->rope_cos, (size_t)c.max_pos * half * F, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(b.sn, w->rope_sin, (size_t)c.max_pos * half * F, hipMemcpyHostToDevice) == hipSuccess;
    if (ok && w->sink)
        ok = hipMemcpy(b.sink, w->sink, H * F, hipMemcpyHostToDevice) == hipSuccess;
    if (ok && comp)
        ok = hipMemcpy(b.comp_norm, w->comp_norm, hd * F, hipMemcpyHostToDevice) == hipSuccess &&
             hipMemcpy(b.ape, w->comp_ape, (size_t)c.ratio * b.width * F, hipMemcpyHostToDevice) == hipSuccess;
    if (!w->sink) b.sink = nullptr;
    if (!ok || block_reset(b) != 0) {
        DSV4_ERR("attn_bind: layer %d: copying the vectors failed", layer);
        block_free(b);
        return -1;
    }
    b.bound = true;
    if ((int)g_blocks.size() <= layer) g_blocks.resize(layer + 1);
    block_free(g_blocks[layer]);
    g_blocks[layer] = b;
    return 0;
}

/* GEMVs that read the same x: FP8 matrices of one width, scale format and
 * blocking go in one launch, BF16 matrices of one width in another (each
 * row keeps the bits of its own launch); anything else goes alone. */
struct XJob {
    const MatRef *m;
    float *y;
    int rows;
};

int x_gemvs(const XJob *jobs, int n, const float *d_x, hipStream_t st, bool valu = false)
{
    bool done[8] = {};
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        const Res &r = jobs[i].m->r;
        if (r.wdt != DSV4_WFP8 && r.wdt != DSV4_WBF16) {
            if (res_gemv(jobs[i].m->view(), jobs[i].rows, jobs[i].y, d_x, st, valu) != 0)
                return -1;
            done[i] = true;
            continue;
        }
        const uint8_t *W[4];
        const void *S[4];
        float *Y[4];
        int R[4], k = 0;
        for (int j = i; j < n && k < 4; j++) {
            const Res &q = jobs[j].m->r;
            if (done[j] || q.wdt != r.wdt || q.cols != r.cols ||
                (r.wdt == DSV4_WFP8 &&
                 (q.sfmt != r.sfmt || q.blk_r != r.blk_r || q.blk_c != r.blk_c)))
                continue;
            W[k] = jobs[j].m->w;
            S[k] = jobs[j].m->s;
            Y[k] = jobs[j].y;
            R[k] = jobs[j].rows;
            done[j] = true;
            k++;
        }
        const int rc = r.wdt == DSV4_WFP8
                           ? dsv4_fp8_gemv_list_launch(d_x, r.cols, r.sfmt, r.blk_r, r.blk_c, k,
                                                       W, S, Y, R, st, valu)
                           : dsv4_bf16_gemv_list_launch(d_x, r.cols, k,
                                                        (const uint16_t *const *)W, Y, R, st);
        if (rc != 0) return -1;
    }
    return 0;
}

/* The x projections of a block step: its FP8 matrices and its BF16 ones
 * read the same x, so they share one launch when every FP8 one has the
 * same scale format and blocking and all have the same width (the VALU
 * form for the FP8 ones); otherwise listed launches as x_gemvs makes. */
int x_proj(const XJob *jobs, int n, const float *d_x, hipStream_t st)
{
    const uint8_t *Wf[4];
    const void *Sf[4];
    float *Yf[4], *Yb[4];
    const uint16_t *Wb[4];
    int Rf[4], Rb[4], nf = 0, nb = 0;
    const Res *f0 = nullptr;
    bool ok = n > 0;
    for (int i = 0; i < n && ok; i++) {
        const Res &r = jobs[i].m->r;
        ok = r.cols == jobs[0].m->r.cols;
        if (r.wdt == DSV4_WFP8) {
            if (!f0) f0 = &r;
            ok = ok && nf < 4 && r.sfmt == f0->sfmt && r.blk_r == f0->blk_r &&
                 r.blk_c == f0->blk_c;
            if (ok) {
                Wf[nf] = jobs[i].m->w; Sf[nf] = jobs[i].m->s;
                Yf[nf] = jobs[i].y; Rf[nf] = jobs[i].rows; nf++;
            }
        } else if (r.wdt == DSV4_WBF16) {
            ok = ok && nb < 4;
            if (ok) {
                Wb[nb] = (const uint16_t *)jobs[i].m->w;
                Yb[nb] = jobs[i].y; Rb[nb] = jobs[i].rows; nb++;
            }
        } else {
            ok = false;
        }
    }
    if (!ok || nf == 0 || nb == 0) return x_gemvs(jobs, n, d_x, st, true);
    return dsv4_xproj_launch(d_x, jobs[0].m->r.cols, f0->sfmt, f0->blk_r, f0->blk_c, nf, Wf, Sf,
                             Yf, Rf, nb, Wb, Yb, Rb, st);
}

/* attention() of dsv4_layer.c:213-336 for the token at pos, on stream st;
 * x and out are device buffers of hidden floats. */
int block_step(AttnBlock &b, float *d_out, const float *d_x, int pos, hipStream_t st)
{
    const dsv4_gpu_attn_cfg &c = b.c;
    const int H = c.n_heads, hd = c.head_dim, rd = c.rope_dim, half = rd / 2;
    if (pos != b.next_pos || pos >= c.max_pos) {
        DSV4_ERR("attn_step: position %d out of order (next %d, max %d); "
                 "dsv4_gpu_attn_reset starts over", pos, b.next_pos, c.max_pos);
        return -1;
    }
#define OK(e) do { if ((e) != 0) return -1; } while (0)
    /* The block's FP8 projections take the VALU form whatever their scale
     * format: nothing batched has to share their bits, and at batch 1 it is
     * the faster form (Flash shapes: 86.5 -> 84.4 us per CSA step, 61.8 ->
     * 58.5 us per HCA step against the matrix-core form) */
    constexpr bool VALU = true;
    const bool closes = c.ratio > 0 && (pos + 1) % c.ratio == 0;
    /* The indexer runs only when it has a choice to make. With no more
     * compressed rows than index_topk the reference's score and top-k take
     * every row (dsv4_layer.c:278-290, take = avail), only in score order;
     * attention over the same rows in index order differs by the float
     * summation order alone, so those steps take mode 1 and skip the
     * indexer's projections, score and top-k. */
    const bool use_idx = c.ratio > 0 && c.idx_heads > 0 &&
                         b.n_comp + (closes ? 1 : 0) > c.idx_topk;
    /* the projections of x: wq_a, wkv, the compressor's wkv / wgate and the
     * indexer's weights_proj (when it runs this step) */
    XJob xj[5] = {{&b.wq_a, b.qr, c.q_lora}, {&b.wkv, b.kv, hd}};
    int nx = 2;
    if (c.ratio > 0) {
        xj[nx++] = XJob{&b.cwkv, b.ckv, b.width};
        xj[nx++] = XJob{&b.cwgate, b.csc, b.width};
    }
    if (use_idx) xj[nx++] = XJob{&b.iwproj, b.idx_w, c.idx_heads};
    OK(x_proj(xj, nx, d_x, st));
    /* What needs only the projections: q's learned norm, kv_norm + RoPE
     * into the ring slot, and the compressor's token into its slot
     * (dsv4_layer.c:222, 235-238, and the slot write of the compress step
     * called at :250); then q: wq_b (each head's norm and RoPE happen inside
     * the attention, on its copy), and the indexer's wq_b when the indexer
     * runs. Both GEMVs read the normed qr, so they share one launch, whose
     * workgroups norm their own copy of qr while the ring and compressor
     * jobs run beside them (dsv4_qproj_launch); matrices of another form
     * take the prep launch and then listed launches. */
    Dsv4Prep pp{};
    pp.job[0] = Dsv4NormJob{b.kv_cache + (size_t)(pos % c.window) * hd, b.kv, b.kv_norm, hd, rd};
    pp.nj = 1;
    pp.eps = c.rms_eps;
    pp.cs = b.cs; pp.sn = b.sn; pp.pos = pos; pp.half = half;
    if (c.ratio > 0) {
        const int ph = pos % c.ratio, slot = c.ratio == 4 ? c.ratio + ph : ph;
        pp.kvs = b.comp_kv + (size_t)slot * b.width;
        pp.scs = b.comp_score + (size_t)slot * b.width;
        pp.kv_in = b.ckv; pp.sc_in = b.csc; pp.apr = b.ape + (size_t)ph * b.width;
        pp.width = b.width;
    }
    XJob qj[2] = {{&b.wq_b, b.q, H * hd}, {&b.iwq_b, b.idx_q, c.idx_heads * c.idx_dim}};
    const int nq = use_idx ? 2 : 1;
    const Res &r0 = b.wq_b.r;
    bool qfp8 = r0.wdt == DSV4_WFP8;
    for (int i = 1; i < nq; i++) {
        const Res &ri = qj[i].m->r;
        qfp8 = qfp8 && ri.wdt == DSV4_WFP8 && ri.cols == r0.cols && ri.sfmt == r0.sfmt &&
               ri.blk_r == r0.blk_r && ri.blk_c == r0.blk_c;
    }
    if (qfp8) {
        const uint8_t *W[2];
        const void *S[2];
        float *Y[2];
        int R[2];
        for (int i = 0; i < nq; i++) {
            W[i] = qj[i].m->w; S[i] = qj[i].m->s; Y[i] = qj[i].y; R[i] = qj[i].rows;
        }
        OK(dsv4_qproj_launch(b.qr, c.q_lora, b.q_norm, c.rms_eps, r0.sfmt, r0.blk_r, r0.blk_c,
                             nq, W, S, Y, R, &pp, st));
    } else {
        pp.job[1] = pp.job[0];
        pp.job[0] = Dsv4NormJob{b.qr, b.qr, b.q_norm, c.q_lora, 0};
        pp.nj = 2;
        OK(dsv4_block_prep_launch(&pp, st));
        OK(x_gemvs(qj, nq, b.qr, st, VALU));
    }
    const int n_win = pos + 1 < c.window ? pos + 1 : c.window;
    int take = 0, mode = 1;
    if (c.ratio > 0) {
        /* the compressor's pool when the window closes (dsv4_layer.c:250-261) */
        if (closes) {
            if (b.n_comp >= b.max_comp) {
                DSV4_ERR("attn_step: compressed rows exceed max_pos / ratio + 1");
                return -1;
            }
            float *crow = b.kv_cache + (size_t)(c.window + b.n_comp) * hd;
            /* pool, comp.norm and RoPE at the window's first position in one
             * launch (bind took head_dim <= 1024) */
            OK(dsv4_comp_close_launch(crow, b.comp_kv, b.comp_score, c.ratio, hd,
                                      b.comp_norm, c.rms_eps, rd, b.cs, b.sn,
                                      pos + 1 - c.ratio, half, st));
            b.n_comp++;
        }
        /* which compressed rows attention sees (dsv4_layer.c:267-297) */
        const int avail = b.n_comp;
        if (use_idx) {
            const int ih = c.idx_heads, idd = c.idx_dim;
            take = avail < c.idx_topk ? avail : c.idx_topk;
            const int hist = dsv4_topk_takes_hist(avail, take);
            /* the keys are the compressed region read at index_head_dim
             * stride, as the reference's call does (dsv4_layer.c:286-289) */
            /* (the indexer's q is RoPE'd at pos inside the score kernel) */
            OK(dsv4_indexer_score_rope_launch(b.scores, b.idx_q, b.idx_w, ih, idd,
                                              b.kv_cache + (size_t)c.window * hd, nullptr,
                                              DSV4_GPU_KV_F32, idd, avail,
                                              indexer_scale(idd, ih), b.iscr, hist, b.cs,
                                              b.sn, pos, half, rd, st));
            OK(dsv4_topk_launch(b.idxs + n_win, b.scores, avail, take, b.iscr, hist, st));
            mode = 2;
        } else {
            take = avail;
        }
    }
    /* the attention with its row list (window, then compressed rows), q's
     * per-head norm and RoPE, and the output's de-rotation, folded in */
    Dsv4Rows rw;
    rw.on = 1;
    rw.win = c.window; rw.n_win = n_win; rw.pos = pos; rw.mode = mode; rw.offset = c.window;
    OK(dsv4_attn_block_launch(b.o, b.q, b.kv_cache, DSV4_GPU_KV_F32, hd,
                              c.window + b.max_comp, b.sink, b.idxs + n_win, H, hd, hd,
                              n_win + take, 1.0f / sqrtf((float)hd), b.ascr, 1, c.rms_eps,
                              b.cs, b.sn, pos, half, rd, st, &rw));
    /* wo_a's groups in one launch (the FP8 slices of dsv4_layer.c:321-334:
     * group g's rows from g * o_lora, its scale rows from g * (o_lora /
     * blk_r), its input o + g * (H * hd / o_groups)), then wo_b */
    const Res &wa = b.wo_a.r;
    const int gw = H * hd / c.o_groups, gr = c.o_lora;
    const long long ssz = wa.sfmt ? 4 : 1;
    OK(dsv4_fp8_gemv_groups_launch(
        b.ogrp, b.o, b.wo_a.w, b.wo_a.s, wa.sfmt, gr, gw, wa.blk_r,
        wa.blk_c, c.o_groups, gr, gw, (long long)gr * wa.cols,
        (long long)(gr / wa.blk_r) * wa.sc * ssz, st, VALU));
    OK(res_gemv(b.wo_b.view(), c.hidden, d_out, b.ogrp, st, VALU));
#undef OK
    b.next_pos = pos + 1;
    return 0;
}

AttnBlock *block_of(int layer)
{
    if (!g_ready || layer < 0 || layer >= (int)g_blocks.size() || !g_blocks[layer].bound)
        return nullptr;
    return &g_blocks[layer];
}

void attn_blocks_free()
{
    for (AttnBlock &b : g_blocks) block_free(b);
    g_blocks.clear();
}

} // namespace

extern "C" {

int dsv4_gpu_attn_bind(int layer, const dsv4_gpu_attn_cfg *c, const dsv4_gpu_attn_w *w)
{
    return block_bind(layer, c, w);
}

int dsv4_gpu_attn_ready(int layer) { return block_of(layer) ? 1 : 0; }

int dsv4_gpu_attn_reset(int layer)
{
    AttnBlock *b = block_of(layer);
    return b ? block_reset(*b) : -1;
}

int dsv4_gpu_attn_step(float *out, const float *x, int layer, int pos)
{
    AttnBlock *b = block_of(layer);
    if (!b || !out || !x) return -1;
    const size_t bytes = (size_t)b->c.hidden * sizeof(float);
    HIP_OK(hipMemcpyAsync(b->x, x, bytes, hipMemcpyHostToDevice, g_stream), "attn x");
    if (block_step(*b, b->out, b->x, pos, g_stream) != 0) {
        (void)hipStreamSynchronize(g_stream);
        return -1;
    }
    HIP_OK(hipMemcpyAsync(out, b->out, bytes, hipMemcpyDeviceToHost, g_stream), "attn out");
    HIP_OK(hipStreamSynchronize(g_stream), "attn sync");
    return 0;
}

int dsv4_gpu_attn_step_d(float *d_out, const float *d_x, int layer, int pos, void *stream)
{
    AttnBlock *b = block_of(layer);
    if (!b || !d_out || !d_x) return -1;
    if (((uintptr_t)d_x | (uintptr_t)d_out) & 15) {
        DSV4_ERR("attn_step: x and out must be 16-byte aligned");
        return -1;
    }
    return block_step(*b, d_out, d_x, pos, as_stream(stream));
}

} /* extern "C" */
