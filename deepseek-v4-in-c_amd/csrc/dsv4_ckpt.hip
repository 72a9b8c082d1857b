/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_ckpt.hip - a DeepSeek-V4 checkpoint read straight into HBM.
 *
 * The reference streams its checkpoint from NVMe through host memory: a
 * pinned trunk plus an LRU cache of routed experts (src/io/dsv4_st.c,
 * src/io/dsv4_trunk.c, src/cache/dsv4_cache.c), because a 160 GB Flash
 * checkpoint does not fit its GPU. An MI355X holds 288 GB, so here every
 * matrix and every routed expert is read once, from the safetensors shards
 * into device memory, and stays resident; nothing is kept in host memory.
 *
 * CONTAINER (the reference's reader, src/io/dsv4_st.c:377-537): every
 * *.safetensors file of the directory, in name order; each is an 8-byte
 * little-endian header length N, N bytes of JSON {name: {dtype, shape,
 * data_offsets: [start, end]}}, then the data, offsets relative to the end of
 * the header. The dtype spellings are the released checkpoint's (U8, I8 --
 * packed FP4, two values per byte --, F16, F32, I64, BF16, F8_E4M3, F8_E8M0);
 * a tensor whose byte span is not its element count times its element size,
 * or that ends past the end of its file, is refused, as there.
 *
 * SCHEMA (src/model/dsv4_bind.c:86-243): a quantised matrix is the pair
 * <base>.weight / <base>.scale -- F8_E4M3 [rows][cols] with E8M0 scales per
 * 128x128, or packed FP4 (I8) [rows][cols/2] with E8M0 scales per 1x32 --
 * and a BF16 matrix is <base>.weight alone. dsv4_gpu_ckpt_load_layer loads
 * every matrix of a layer under the binder's names, and its routed experts
 * layers.L.ffn.experts.E.w{1,2,3}.
 *
 * DATA PATH: pread into pinned staging buffers, hipMemcpyAsync on the
 * loader's own copy stream, an event per buffer so a buffer is refilled only
 * once its copy is done; a reader thread fills the next buffers while
 * earlier ones are copying. A load call returns once its bytes are in HBM.
 * The loaded matrices are registered as resident under their DEVICE
 * addresses (dsv4_res_adopt): a DSV4QMat filled by the loader is what the
 * caller's dispatch passes back to dsv4_gpu_has / dsv4_gpu_mmq, and row-range
 * views of it (attention()'s wo_a group slices) resolve as usual. The host
 * never dereferences those pointers: every matmul on them runs on the device.
 */
#include "dsv4_internal.h"

#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

enum Dtype { DT_U8, DT_I8, DT_F16, DT_F32, DT_I64, DT_BF16, DT_E4M3, DT_E8M0, DT_BAD };

struct Spelling {
    const char *name;
    Dtype dt;
    int bytes;                       /* per stored element (I8: per packed byte) */
};
const Spelling kDtypes[] = {{"U8", DT_U8, 1},       {"I8", DT_I8, 1},
                            {"F16", DT_F16, 2},     {"F32", DT_F32, 4},
                            {"I64", DT_I64, 8},     {"BF16", DT_BF16, 2},
                            {"F8_E4M3", DT_E4M3, 1}, {"F8_E8M0", DT_E8M0, 1}};

struct Tensor {
    int shard = -1;
    Dtype dt = DT_BAD;
    int ndim = 0;
    int64_t shape[4] = {0, 0, 0, 0};
    int64_t off = 0, nbytes = 0;     /* absolute file offset, byte span */
};

/* A cursor over the JSON header: only what a safetensors header holds
 * (objects, arrays, strings, integers; other values are skipped). */
struct Json {
    const char *p, *end;
    void ws() { while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++; }
    bool take(char c) { ws(); if (p < end && *p == c) { p++; return true; } return false; }
    bool peek(char c) { ws(); return p < end && *p == c; }
    bool str(std::string &out)
    {
        if (!take('"')) return false;
        out.clear();
        while (p < end && *p != '"') {
            if (*p == '\\') {                       /* names carry no escapes in practice */
                if (++p >= end) return false;
                switch (*p) {
                case 'n': out += '\n'; break;
                case 't': out += '\t'; break;
                case 'u':                           /* keep \uXXXX verbatim */
                    out += "\\u";
                    break;
                default: out += *p; break;
                }
                p++;
                continue;
            }
            out += *p++;
        }
        return take('"');
    }
    bool integer(int64_t &v)
    {
        ws();
        bool neg = false;
        if (p < end && *p == '-') { neg = true; p++; }
        if (p >= end || *p < '0' || *p > '9') return false;
        int64_t x = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            if (x > (INT64_MAX - 9) / 10) return false;
            x = x * 10 + (*p++ - '0');
        }
        v = neg ? -x : x;
        return true;
    }
    bool skip()
    {
        ws();
        if (p >= end) return false;
        if (*p == '"') { std::string s; return str(s); }
        if (*p == '{' || *p == '[') {
            const char open = *p, close = open == '{' ? '}' : ']';
            p++;
            if (take(close)) return true;
            do {
                if (open == '{') {
                    std::string k;
                    if (!str(k) || !take(':')) return false;
                }
                if (!skip()) return false;
            } while (take(','));
            return take(close);
        }
        while (p < end && *p != ',' && *p != '}' && *p != ']') p++;   /* number / literal */
        return true;
    }
};

int64_t numel(const Tensor &t)
{
    int64_t n = 1;
    for (int i = 0; i < t.ndim; i++) n *= t.shape[i];
    return n;
}

struct Shard {
    std::string path;
    int fd = -1;
    int64_t size = 0;
};

constexpr int NSTAGE = 4;
constexpr size_t STAGE_BYTES = 32u << 20;

double now_s()
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

} // namespace

struct dsv4_gpu_ckpt {
    std::vector<Shard> shards;
    std::unordered_map<std::string, Tensor> index;
    hipStream_t cs = nullptr;
    char *stage[NSTAGE] = {};
    hipEvent_t done[NSTAGE] = {};
    bool pending[NSTAGE] = {};
    int next = 0;
    dsv4_gpu_ckpt_stats st{};
    /* One reader thread for the handle's life: stream_in hands it one chunk
     * at a time (job) and waits until it has taken it back to nullptr. */
    pthread_t reader{};
    bool reader_on = false, quit = false;
    pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
    pthread_cond_t cv = PTHREAD_COND_INITIALIZER;
    void *job = nullptr;
};

namespace {

int scan_shard(dsv4_gpu_ckpt *c, int si)
{
    Shard &sh = c->shards[si];
    sh.fd = open(sh.path.c_str(), O_RDONLY);
    if (sh.fd < 0) { DSV4_ERR("ckpt: cannot open %s", sh.path.c_str()); return -1; }
    struct stat sb;
    if (fstat(sh.fd, &sb) != 0) return -1;
    sh.size = (int64_t)sb.st_size;
    unsigned char lb[8];
    if (pread(sh.fd, lb, 8, 0) != 8) { DSV4_ERR("ckpt: %s has no header", sh.path.c_str()); return -1; }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | lb[i];
    if (hlen == 0 || hlen > (uint64_t)sh.size - 8) {
        DSV4_ERR("ckpt: %s: header length %llu does not fit the file", sh.path.c_str(),
                 (unsigned long long)hlen);
        return -1;
    }
    std::string js(hlen, '\0');
    size_t got = 0;
    while (got < hlen) {
        const ssize_t r = pread(sh.fd, &js[got], hlen - got, (off_t)(8 + got));
        if (r <= 0) { DSV4_ERR("ckpt: %s: short header read", sh.path.c_str()); return -1; }
        got += (size_t)r;
    }
    const int64_t base = 8 + (int64_t)hlen;
    Json j{js.data(), js.data() + js.size()};
    if (!j.take('{')) { DSV4_ERR("ckpt: %s: header is not an object", sh.path.c_str()); return -1; }
    if (j.take('}')) return 0;
    do {
        std::string name;
        if (!j.str(name) || !j.take(':')) goto bad;
        if (name == "__metadata__") { if (!j.skip()) goto bad; continue; }
        {
            Tensor t;
            t.shard = si;
            bool have_dt = false, have_off = false;
            int64_t o0 = 0, o1 = 0;
            if (!j.take('{')) goto bad;
            if (!j.peek('}')) {
                do {
                    std::string key;
                    if (!j.str(key) || !j.take(':')) goto bad;
                    if (key == "dtype") {
                        std::string v;
                        if (!j.str(v)) goto bad;
                        for (const Spelling &s : kDtypes)
                            if (v == s.name) t.dt = s.dt;
                        if (t.dt == DT_BAD) {
                            DSV4_ERR("ckpt: %s: dtype '%s' of %s is not one this checkpoint "
                                     "uses", sh.path.c_str(), v.c_str(), name.c_str());
                            return -1;
                        }
                        have_dt = true;
                    } else if (key == "shape") {
                        if (!j.take('[')) goto bad;
                        if (!j.take(']')) {
                            do {
                                int64_t d;
                                if (!j.integer(d) || d < 0 || t.ndim >= 4) goto bad;
                                t.shape[t.ndim++] = d;
                            } while (j.take(','));
                            if (!j.take(']')) goto bad;
                        }
                    } else if (key == "data_offsets") {
                        if (!j.take('[') || !j.integer(o0) || !j.take(',') || !j.integer(o1) ||
                            !j.take(']'))
                            goto bad;
                        have_off = true;
                    } else if (!j.skip()) {
                        goto bad;
                    }
                } while (j.take(','));
            }
            if (!j.take('}')) goto bad;
            if (!have_dt || !have_off || o1 < o0) {
                DSV4_ERR("ckpt: %s: %s lacks dtype or data_offsets", sh.path.c_str(), name.c_str());
                return -1;
            }
            int eb = 1;
            for (const Spelling &s : kDtypes)
                if (s.dt == t.dt) eb = s.bytes;
            t.off = base + o0;
            t.nbytes = o1 - o0;
            if (t.nbytes != numel(t) * eb) {
                DSV4_ERR("ckpt: %s: %s spans %lld bytes, its shape %lld", sh.path.c_str(),
                         name.c_str(), (long long)t.nbytes, (long long)(numel(t) * eb));
                return -1;
            }
            if (t.off + t.nbytes > sh.size) {
                DSV4_ERR("ckpt: %s: %s ends past the end of the file", sh.path.c_str(),
                         name.c_str());
                return -1;
            }
            if (!c->index.emplace(name, t).second) {
                DSV4_ERR("ckpt: %s: %s appears twice", sh.path.c_str(), name.c_str());
                return -1;
            }
        }
    } while (j.take(','));
    if (!j.take('}')) goto bad;
    return 0;
bad:
    DSV4_ERR("ckpt: %s: malformed header near byte %ld", sh.path.c_str(),
             (long)(j.p - js.data()));
    return -1;
}

/* The reader thread of one copy: fills a staging buffer with [off, off+len)
 * of a shard while the copy stream drains the others. */
struct ReadJob {
    int fd;
    char *buf;
    int64_t off, len;
    int err;
};

void *read_job(void *a)
{
    ReadJob *r = (ReadJob *)a;
    int64_t got = 0;
    r->err = 0;
    while (got < r->len) {
        const ssize_t n = pread(r->fd, r->buf + got, (size_t)(r->len - got), (off_t)(r->off + got));
        if (n <= 0) {
            if (n < 0 && errno == EINTR) continue;
            r->err = 1;
            break;
        }
        got += n;
    }
    return nullptr;
}

/* The reader thread: reads each job handed over, then clears the slot. */
void *reader_main(void *a)
{
    dsv4_gpu_ckpt *c = (dsv4_gpu_ckpt *)a;
    pthread_mutex_lock(&c->mu);
    for (;;) {
        while (!c->job && !c->quit) pthread_cond_wait(&c->cv, &c->mu);
        if (!c->job) break;                             /* quit, nothing pending */
        ReadJob *j = (ReadJob *)c->job;
        pthread_mutex_unlock(&c->mu);
        read_job(j);
        pthread_mutex_lock(&c->mu);
        c->job = nullptr;
        pthread_cond_broadcast(&c->cv);
    }
    pthread_mutex_unlock(&c->mu);
    return nullptr;
}

void reader_submit(dsv4_gpu_ckpt *c, ReadJob *j)
{
    pthread_mutex_lock(&c->mu);
    c->job = j;
    pthread_cond_broadcast(&c->cv);
    pthread_mutex_unlock(&c->mu);
}

void reader_wait(dsv4_gpu_ckpt *c)
{
    pthread_mutex_lock(&c->mu);
    while (c->job) pthread_cond_wait(&c->cv, &c->mu);
    pthread_mutex_unlock(&c->mu);
}

/* Copy `len` bytes of shard `fd` from file offset `off` to device address
 * dst: chunks through the staging ring, the reader thread's read of chunk
 * i + 1 overlapping the copy of chunk i (without a reader thread every read
 * is inline). Stream-ordered on the loader's copy stream. */
int stream_in(dsv4_gpu_ckpt *c, int fd, int64_t off, int64_t len, uint8_t *dst)
{
    ReadJob job{}, nxt{};
    bool running = false;
    int64_t done = 0;
    int b = -1;
    while (done < len || running) {
        if (running) {                                  /* the chunk in flight */
            reader_wait(c);
            running = false;
            if (job.err) { DSV4_ERR("ckpt: read failed at offset %lld", (long long)job.off); return -1; }
            HIP_OK(hipMemcpyAsync(dst + (job.off - off), job.buf, (size_t)job.len,
                                  hipMemcpyHostToDevice, c->cs), "ckpt copy");
            HIP_OK(hipEventRecord(c->done[b], c->cs), "ckpt event");
            c->pending[b] = true;
        }
        if (done < len) {                               /* start the next read */
            b = c->next;
            c->next = (c->next + 1) % NSTAGE;
            if (c->pending[b]) {
                HIP_OK(hipEventSynchronize(c->done[b]), "ckpt buffer wait");
                c->pending[b] = false;
            }
            nxt.fd = fd;
            nxt.buf = c->stage[b];
            nxt.off = off + done;
            nxt.len = std::min<int64_t>((int64_t)STAGE_BYTES, len - done);
            job = nxt;
            if (c->reader_on) {
                reader_submit(c, &job);
                running = true;
            } else {
                read_job(&job);                         /* no thread: read inline */
                if (job.err) { DSV4_ERR("ckpt: read failed"); return -1; }
                HIP_OK(hipMemcpyAsync(dst + (job.off - off), job.buf, (size_t)job.len,
                                      hipMemcpyHostToDevice, c->cs), "ckpt copy");
                HIP_OK(hipEventRecord(c->done[b], c->cs), "ckpt event");
                c->pending[b] = true;
            }
            done += nxt.len;
        }
    }
    return 0;
}

const Tensor *find(const dsv4_gpu_ckpt *c, const std::string &name)
{
    auto it = c->index.find(name);
    if (it == c->index.end()) {
        DSV4_ERR("ckpt: tensor %s is not in the checkpoint", name.c_str());
        return nullptr;
    }
    return &it->second;
}

size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

/* One part of a device block: a tensor read to block + at. */
struct Part {
    const Tensor *t;
    size_t at;
};

/* Read every part into one new device block of `total` bytes; the block on
 * success (synchronised), nullptr on failure. */
uint8_t *load_parts(dsv4_gpu_ckpt *c, const Part *parts, int n, size_t total)
{
    if (total + (256u << 20) > dsv4_gpu_free_vram()) {
        DSV4_ERR("ckpt: no room in HBM for %zu more bytes", total);
        return nullptr;
    }
    uint8_t *blk = nullptr;
    if (hipMalloc((void **)&blk, total) != hipSuccess) return nullptr;
    const double t0 = now_s();
    int rc = 0;
    for (int i = 0; i < n && rc == 0; i++)
        rc = stream_in(c, c->shards[parts[i].t->shard].fd, parts[i].t->off, parts[i].t->nbytes,
                       blk + parts[i].at);
    if (rc == 0 && hipStreamSynchronize(c->cs) != hipSuccess) rc = -1;
    for (int b = 0; b < NSTAGE; b++) c->pending[b] = false;
    if (rc != 0) {
        (void)hipStreamSynchronize(c->cs);
        (void)hipFree(blk);
        return nullptr;
    }
    for (int i = 0; i < n; i++) c->st.bytes += parts[i].t->nbytes;
    c->st.seconds += now_s() - t0;
    return blk;
}

/* The stored form the schema expects for a matrix of this format. */
bool check_pair(const Tensor *w, const Tensor *s, int wdt, int rows, int cols,
                const std::string &base)
{
    const int64_t R = rows, C = cols;
    bool ok = false;
    if (wdt == DSV4_WFP8)
        ok = w->dt == DT_E4M3 && w->nbytes == R * C && s && s->dt == DT_E8M0 &&
             s->nbytes == ((R + 127) / 128) * ((C + 127) / 128);
    else if (wdt == DSV4_WFP4)
        ok = w->dt == DT_I8 && (C % 2) == 0 && w->nbytes == R * (C / 2) && s &&
             s->dt == DT_E8M0 && (C % 32) == 0 && s->nbytes == R * (C / 32);
    else if (wdt == DSV4_WBF16)
        ok = w->dt == DT_BF16 && w->nbytes == R * C * 2;
    if (!ok)
        DSV4_ERR("ckpt: %s is not a %dx%d matrix of format %d as stored", base.c_str(), rows,
                 cols, wdt);
    return ok;
}

void qmat_init(DSV4QMat *m, int wdt, int rows, int cols)
{
    m->wdt = wdt;
    m->rows = rows;
    m->cols = cols;
    m->blk_r = wdt == DSV4_WFP8 ? 128 : wdt == DSV4_WFP4 ? 1 : 0;
    m->blk_c = wdt == DSV4_WFP8 ? 128 : wdt == DSV4_WFP4 ? 32 : 0;
}

} // namespace

extern "C" {

dsv4_gpu_ckpt *dsv4_gpu_ckpt_open(const char *dir)
{
    if (!dir || dsv4_gpu_init() != 0) return nullptr;
    DIR *d = opendir(dir);
    if (!d) { DSV4_ERR("ckpt: cannot open directory %s", dir); return nullptr; }
    std::vector<std::string> files;
    while (struct dirent *e = readdir(d)) {
        const size_t n = strlen(e->d_name);
        if (n > 12 && !strcmp(e->d_name + n - 12, ".safetensors"))
            files.push_back(std::string(dir) + "/" + e->d_name);
    }
    closedir(d);
    if (files.empty()) { DSV4_ERR("ckpt: no .safetensors files in %s", dir); return nullptr; }
    std::sort(files.begin(), files.end());        /* stable shard order */
    dsv4_gpu_ckpt *c = new dsv4_gpu_ckpt;
    for (const std::string &f : files) {
        c->shards.push_back(Shard{});
        c->shards.back().path = f;
    }
    bool ok = true;
    for (int i = 0; i < (int)c->shards.size() && ok; i++) ok = scan_shard(c, i) == 0;
    if (ok) ok = hipStreamCreateWithFlags(&c->cs, hipStreamNonBlocking) == hipSuccess;
    for (int b = 0; b < NSTAGE && ok; b++)
        ok = hipHostMalloc((void **)&c->stage[b], STAGE_BYTES, hipHostMallocDefault) ==
                 hipSuccess &&
             hipEventCreateWithFlags(&c->done[b], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        dsv4_gpu_ckpt_close(c);
        return nullptr;
    }
    /* without the thread every read is made inline, just slower */
    c->reader_on = pthread_create(&c->reader, nullptr, reader_main, c) == 0;
    c->st.tensors = (long long)c->index.size();
    c->st.shards = (int)c->shards.size();
    return c;
}

void dsv4_gpu_ckpt_close(dsv4_gpu_ckpt *c)
{
    if (!c) return;
    if (c->reader_on) {
        pthread_mutex_lock(&c->mu);
        c->quit = true;
        pthread_cond_broadcast(&c->cv);
        pthread_mutex_unlock(&c->mu);
        pthread_join(c->reader, nullptr);
        c->reader_on = false;
    }
    if (c->cs) (void)hipStreamSynchronize(c->cs);
    for (int b = 0; b < NSTAGE; b++) {
        if (c->stage[b]) (void)hipHostFree(c->stage[b]);
        if (c->done[b]) (void)hipEventDestroy(c->done[b]);
    }
    if (c->cs) (void)hipStreamDestroy(c->cs);
    for (Shard &s : c->shards)
        if (s.fd >= 0) close(s.fd);
    delete c;
}

int dsv4_gpu_ckpt_has(const dsv4_gpu_ckpt *c, const char *name)
{
    return (c && name && c->index.count(name)) ? 1 : 0;
}

int dsv4_gpu_ckpt_load_qmat(dsv4_gpu_ckpt *c, const char *base, int wdt, int rows, int cols,
                            DSV4QMat *out)
{
    if (!c || !base || !out || rows <= 0 || cols <= 0) return -1;
    const std::string b(base);
    const Tensor *w = find(c, b + ".weight");
    const Tensor *s = wdt == DSV4_WBF16 ? nullptr : find(c, b + ".scale");
    if (!w || (wdt != DSV4_WBF16 && !s) || !check_pair(w, s, wdt, rows, cols, b)) return -1;
    const size_t wat = 0, sat = a256((size_t)w->nbytes);
    Part parts[2] = {{w, wat}, {s, sat}};
    const size_t total = s ? sat + (size_t)s->nbytes : (size_t)w->nbytes;
    uint8_t *blk = load_parts(c, parts, s ? 2 : 1, total);
    if (!blk) return -1;
    DSV4QMat m;
    qmat_init(&m, wdt, rows, cols);
    m.w = blk + wat;
    m.s = s ? blk + sat : nullptr;
    if (dsv4_res_adopt(&m, blk) != 0) {
        (void)hipFree(blk);
        return -1;
    }
    *out = m;
    c->st.matrices++;
    return 0;
}

int dsv4_gpu_ckpt_load_expert(dsv4_gpu_ckpt *c, int layer, int expert, int hidden, int inter,
                              DSV4ExpertW *out)
{
    if (!c || layer < 0 || expert < 0 || hidden <= 0 || inter <= 0) return -1;
    /* one block: w1, s1, w3, s3, w2, s2 (the layout dsv4_gpu_upload_expert
     * makes), each part 256-byte aligned */
    const int rows[3] = {inter, inter, hidden}, cols[3] = {hidden, hidden, inter};
    const int which[3] = {1, 3, 2};
    Part parts[6];
    size_t at = 0;
    for (int i = 0; i < 3; i++) {
        char nm[128];
        snprintf(nm, sizeof nm, "layers.%d.ffn.experts.%d.w%d", layer, expert, which[i]);
        const std::string b(nm);
        const Tensor *w = find(c, b + ".weight"), *s = find(c, b + ".scale");
        if (!w || !s || !check_pair(w, s, DSV4_WFP4, rows[i], cols[i], b)) return -1;
        parts[2 * i] = Part{w, at};
        at = a256(at + (size_t)w->nbytes);
        parts[2 * i + 1] = Part{s, at};
        at = a256(at + (size_t)s->nbytes);
    }
    uint8_t *blk = load_parts(c, parts, 6, at);
    if (!blk) return -1;
    DSV4ExpertW e;
    DSV4QMat *ms[3] = {&e.w1, &e.w3, &e.w2};
    for (int i = 0; i < 3; i++) {
        qmat_init(ms[i], DSV4_WFP4, rows[i], cols[i]);
        ms[i]->w = blk + parts[2 * i].at;
        ms[i]->s = blk + parts[2 * i + 1].at;
    }
    if (dsv4_expert_adopt(layer, expert, &e, blk) != 0) {
        (void)hipFree(blk);
        return -1;
    }
    if (out) *out = e;
    c->st.experts++;
    return 0;
}

int dsv4_gpu_ckpt_load_layer(dsv4_gpu_ckpt *c, const dsv4_gpu_ckpt_dims *d, int layer,
                             dsv4_gpu_layer_mats *out, DSV4ExpertW *experts)
{
    if (!c || !d || !out || layer < 0) return -1;
    memset(out, 0, sizeof *out);
    const int H = d->n_heads, hd = d->head_dim;
    const int gw = d->o_groups > 0 ? H * hd / d->o_groups : 0;
    const int coff = d->compress_ratio == 4 ? 2 : 1;
    const int inter_s = d->moe_inter * d->n_shared;
    char nm[160];
    auto load = [&](DSV4QMat *m, int wdt, int rows, int cols, const char *fmt) {
        snprintf(nm, sizeof nm, fmt, layer);
        return dsv4_gpu_ckpt_load_qmat(c, nm, wdt, rows, cols, m);
    };
    /* dsv4_bind.c:177-199 (attention), :233-242 (the shared expert), :220
     * (the router gate), :142-149 and :203-214 (compressors, the indexer) */
    int rc = load(&out->wq_a, DSV4_WFP8, d->q_lora, d->hidden, "layers.%d.attn.wq_a") ||
             load(&out->wq_b, DSV4_WFP8, H * hd, d->q_lora, "layers.%d.attn.wq_b") ||
             load(&out->wkv, DSV4_WFP8, hd, d->hidden, "layers.%d.attn.wkv") ||
             load(&out->wo_a, DSV4_WFP8, d->o_lora * d->o_groups, gw, "layers.%d.attn.wo_a") ||
             load(&out->wo_b, DSV4_WFP8, d->hidden, d->o_lora * d->o_groups,
                  "layers.%d.attn.wo_b") ||
             load(&out->shared_w1, DSV4_WFP8, inter_s, d->hidden,
                  "layers.%d.ffn.shared_experts.w1") ||
             load(&out->shared_w2, DSV4_WFP8, d->hidden, inter_s,
                  "layers.%d.ffn.shared_experts.w2") ||
             load(&out->shared_w3, DSV4_WFP8, inter_s, d->hidden,
                  "layers.%d.ffn.shared_experts.w3") ||
             load(&out->gate, DSV4_WBF16, d->n_experts, d->hidden, "layers.%d.ffn.gate");
    if (!rc && d->compress_ratio > 0)
        rc = load(&out->comp_wkv, DSV4_WBF16, coff * hd, d->hidden,
                  "layers.%d.attn.compressor.wkv") ||
             load(&out->comp_wgate, DSV4_WBF16, coff * hd, d->hidden,
                  "layers.%d.attn.compressor.wgate");
    if (!rc && d->has_indexer)
        rc = load(&out->idx_wq_b, DSV4_WFP8, d->index_n_heads * d->index_head_dim, d->q_lora,
                  "layers.%d.attn.indexer.wq_b") ||
             load(&out->idx_wproj, DSV4_WBF16, d->index_n_heads, d->hidden,
                  "layers.%d.attn.indexer.weights_proj") ||
             load(&out->idx_comp_wkv, DSV4_WBF16, coff * d->index_head_dim, d->hidden,
                  "layers.%d.attn.indexer.compressor.wkv") ||
             load(&out->idx_comp_wgate, DSV4_WBF16, coff * d->index_head_dim, d->hidden,
                  "layers.%d.attn.indexer.compressor.wgate");
    int loaded = 0;                                 /* experts registered by this call */
    for (int e = 0; !rc && e < d->n_experts; e++) {
        rc = dsv4_gpu_ckpt_load_expert(c, layer, e, d->hidden, d->moe_inter,
                                       experts ? &experts[e] : nullptr);
        loaded += rc == 0;
    }
    if (!rc) return 0;
    /* roll back what this call made resident, so that HBM is returned and
     * a retry of the layer starts from nothing */
    for (int e = 0; e < loaded; e++) (void)dsv4_expert_release(layer, e);
    const DSV4QMat *ms[] = {&out->wq_a, &out->wq_b, &out->wkv, &out->wo_a, &out->wo_b,
                            &out->shared_w1, &out->shared_w2, &out->shared_w3, &out->gate,
                            &out->comp_wkv, &out->comp_wgate, &out->idx_wq_b, &out->idx_wproj,
                            &out->idx_comp_wkv, &out->idx_comp_wgate};
    for (const DSV4QMat *m : ms)
        if (m->w) (void)dsv4_res_release(m->w);
    memset(out, 0, sizeof *out);
    if (experts)
        for (int e = 0; e < loaded; e++) memset(&experts[e], 0, sizeof experts[e]);
    c->st.experts -= loaded;
    return -1;
}

int dsv4_gpu_ckpt_stats_get(const dsv4_gpu_ckpt *c, dsv4_gpu_ckpt_stats *out)
{
    if (!c || !out) return -1;
    *out = c->st;
    return 0;
}

} /* extern "C" */
