/* k3gc_load.c - routed experts from safetensors checkpoint shards into the HBM cache's
 * host bank (C99).
 *
 * The engine indexes every tensor of every *.safetensors file of a directory
 * (src/io/k3_st.c:364-452: shards sorted by name, the JSON header's dtype, shape and
 * data_offsets per tensor, the byte span checked against the shape) and resolves one
 * routed expert as six U8 tensors named
 *   language_model.model.layers.L.block_sparse_moe.experts.E.{w1,w2,w3}.{weight_packed,
 *   weight_scale}
 * whose geometry it validates and which, in the checkpoint, tile one contiguous run in
 * the order w1.packed w1.scale w2.packed w2.scale w3.packed w3.scale
 * (src/io/k3_load.c:15-100, src/io/k3_load.h:3-9). Here the run goes straight into the
 * bank: one read when contiguous (six reads in the run order otherwise, :123-135), into
 * the bank's pinned memory for the checkpoint layout, or through a buffer and the host
 * tiler for the tiled layout the matrix cores stream.
 *
 * A contiguous run is read with O_DIRECT where the filesystem takes it, as the engine's
 * k3_expert_load_direct does (src/io/k3_st.c:457-497, K3_ST_ALIGN 4096): the read is
 * widened to the enclosing 4096-byte window of the file, lands in a 4096-aligned buffer,
 * and the run is copied out of it. Several hundred GB of experts then do not pass through
 * (and evict everything else from) the page cache. Shards whose filesystem refuses
 * O_DIRECT, and scattered runs, use ordinary reads. */
#define _GNU_SOURCE            /* O_DIRECT */
#include "k3gc_cache.h"
#include "k3g_kernels.h"

#include <dirent.h>
#include <fcntl.h>
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

typedef struct {
    char *name;
    int shard, dtype_u8, ndim;
    int64_t shape[4];
    int64_t off, nbytes;          /* absolute file offset, bytes */
} StTensor;

#define ST_ALIGN 4096
#define ST_READ_MAX ((int64_t)1 << 30)

struct K3gcSt {
    int nshard;
    char **path;
    int *fd;
    int *dfd;                     /* O_DIRECT descriptor of each shard, or -1 */
    StTensor *t;                  /* sorted by name */
    int nt, capt;
    int borrowed;                 /* descriptors belong to the engine's K3St */
};

/* ------------------------------------------------------------ a JSON scanner ---- */
typedef struct {
    const char *p, *end;
} Js;

static void js_ws(Js *s)
{
    while (s->p < s->end && (*s->p == ' ' || *s->p == '\n' || *s->p == '\r' || *s->p == '\t'))
        s->p++;
}

static int js_lit(Js *s, char c)
{
    js_ws(s);
    if (s->p < s->end && *s->p == c) { s->p++; return 1; }
    return 0;
}

/* a string into out (escapes kept as the character they name; \u above 0x7f refused) */
static int js_str(Js *s, char *out, size_t cap)
{
    if (!js_lit(s, '"')) return 0;
    size_t n = 0;
    while (s->p < s->end && *s->p != '"') {
        char c = *s->p++;
        if (c == '\\') {
            if (s->p >= s->end) return 0;
            c = *s->p++;
            if (c == 'u') {
                if (s->end - s->p < 4) return 0;
                unsigned v = 0;
                for (int i = 0; i < 4; i++) {
                    const char h = *s->p++;
                    v = v * 16 + (unsigned)(h >= '0' && h <= '9' ? h - '0'
                                          : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                          : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
                }
                if (v > 0x7f) return 0;
                c = (char)v;
            } else if (c == 'n') c = '\n';
            else if (c == 't') c = '\t';
            else if (c == 'r') c = '\r';
            else if (c == 'b') c = '\b';
            else if (c == 'f') c = '\f';
        }
        if (n + 1 >= cap) return 0;
        out[n++] = c;
    }
    if (s->p >= s->end) return 0;
    s->p++;
    out[n] = 0;
    return 1;
}

static int js_i64(Js *s, int64_t *v)
{
    js_ws(s);
    int neg = 0;
    if (s->p < s->end && *s->p == '-') { neg = 1; s->p++; }
    if (s->p >= s->end || *s->p < '0' || *s->p > '9') return 0;
    int64_t x = 0;
    while (s->p < s->end && *s->p >= '0' && *s->p <= '9') {
        if (x > (INT64_MAX - 9) / 10) return 0;
        x = x * 10 + (*s->p++ - '0');
    }
    *v = neg ? -x : x;
    return 1;
}

/* skip any value (object, array, string, number, true/false/null) */
static int js_skip(Js *s, int depth)
{
    if (depth > 64) return 0;
    js_ws(s);
    if (s->p >= s->end) return 0;
    const char c = *s->p;
    if (c == '"') {
        char tmp[1024];
        return js_str(s, tmp, sizeof tmp);
    }
    if (c == '{' || c == '[') {
        const char close = c == '{' ? '}' : ']';
        s->p++;
        if (js_lit(s, close)) return 1;
        for (;;) {
            if (c == '{') {
                char key[1024];
                if (!js_str(s, key, sizeof key) || !js_lit(s, ':')) return 0;
            }
            if (!js_skip(s, depth + 1)) return 0;
            if (js_lit(s, ',')) continue;
            return js_lit(s, close);
        }
    }
    while (s->p < s->end && *s->p != ',' && *s->p != '}' && *s->p != ']' && *s->p != ' ' &&
           *s->p != '\n')
        s->p++;
    return 1;
}

/* ---------------------------------------------------------------- the index ---- */
static int push_tensor(K3gcSt *st, const StTensor *t)
{
    if (st->nt == st->capt) {
        const int nc = st->capt ? 2 * st->capt : 256;
        StTensor *n = (StTensor *)realloc(st->t, (size_t)nc * sizeof *n);
        if (!n) return -1;
        st->t = n;
        st->capt = nc;
    }
    st->t[st->nt++] = *t;
    return 0;
}

/* One shard's header (src/io/k3_st.c:195-350): little-endian u64 length, JSON object of
 * name -> {dtype, shape, data_offsets}, offsets relative to the end of the header. */
static int scan_shard(K3gcSt *st, int shard, const char *path)
{
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { fprintf(stderr, "k3gc: cannot open %s\n", path); return -1; }
    st->fd[shard] = fd;
    unsigned char lb[8];
    if (pread(fd, lb, 8, 0) != 8) { fprintf(stderr, "k3gc: %s: no header length\n", path); return -1; }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | lb[i];
    struct stat sb;
    if (fstat(fd, &sb) != 0 || hlen == 0 || sb.st_size < 8 ||
        hlen > (uint64_t)sb.st_size - 8) {
        fprintf(stderr, "k3gc: %s: impossible header length %llu\n", path, (unsigned long long)hlen);
        return -1;
    }
    char *json = (char *)malloc(hlen + 1);
    if (!json) return -1;
    if ((uint64_t)pread(fd, json, hlen, 8) != hlen) {
        fprintf(stderr, "k3gc: %s: short header\n", path);
        free(json);
        return -1;
    }
    json[hlen] = 0;
    const int64_t base = (int64_t)(8 + hlen);
    Js s = {json, json + hlen};
    int rc = -1;
    if (!js_lit(&s, '{')) goto done;
    if (js_lit(&s, '}')) { rc = 0; goto done; }
    for (;;) {
        char name[512];
        if (!js_str(&s, name, sizeof name) || !js_lit(&s, ':')) goto done;
        if (!strcmp(name, "__metadata__")) {
            if (!js_skip(&s, 0)) goto done;
        } else {
            StTensor t;
            memset(&t, 0, sizeof t);
            t.shard = shard;
            int have_dt = 0, have_off = 0;
            int64_t o0 = 0, o1 = 0, elem = 0;
            if (!js_lit(&s, '{')) goto done;
            if (!js_lit(&s, '}')) for (;;) {
                char key[64];
                if (!js_str(&s, key, sizeof key) || !js_lit(&s, ':')) goto done;
                if (!strcmp(key, "dtype")) {
                    char dv[32];
                    if (!js_str(&s, dv, sizeof dv)) goto done;
                    have_dt = 1;
                    t.dtype_u8 = !strcmp(dv, "U8");
                    elem = !strcmp(dv, "U8") || !strcmp(dv, "I8") || !strcmp(dv, "BOOL") ? 1
                         : !strcmp(dv, "BF16") || !strcmp(dv, "F16") || !strcmp(dv, "I16") ? 2
                         : !strcmp(dv, "F32") || !strcmp(dv, "I32") || !strcmp(dv, "U32") ? 4
                         : !strcmp(dv, "F64") || !strcmp(dv, "I64") ? 8
                         : !strcmp(dv, "F8_E4M3") || !strcmp(dv, "F8_E5M2") ? 1 : 0;
                    if (!elem) { fprintf(stderr, "k3gc: %s: dtype %s of %s\n", path, dv, name); goto done; }
                } else if (!strcmp(key, "shape")) {
                    if (!js_lit(&s, '[')) goto done;
                    if (!js_lit(&s, ']')) for (;;) {
                        int64_t dim;
                        /* the expert API takes dimensions as int */
                        if (!js_i64(&s, &dim) || dim < 0 || dim > INT_MAX) goto done;
                        if (t.ndim >= 4) { fprintf(stderr, "k3gc: %s: rank > 4\n", name); goto done; }
                        t.shape[t.ndim++] = dim;
                        if (js_lit(&s, ',')) continue;
                        if (js_lit(&s, ']')) break;
                        goto done;
                    }
                } else if (!strcmp(key, "data_offsets")) {
                    if (!js_lit(&s, '[') || !js_i64(&s, &o0) || !js_lit(&s, ',') ||
                        !js_i64(&s, &o1) || !js_lit(&s, ']'))
                        goto done;
                    have_off = 1;
                } else if (!js_skip(&s, 0)) {
                    goto done;
                }
                if (js_lit(&s, ',')) continue;
                if (js_lit(&s, '}')) break;
                goto done;
            }
            if (!have_dt || !have_off || o0 < 0 || o1 < o0) {
                fprintf(stderr, "k3gc: %s: %s lacks dtype or valid data_offsets\n", path, name);
                goto done;
            }
            /* elements x element size and the span's end, with every product and sum
             * checked (an untrusted header must not overflow them) */
            int64_t numel = 1, span = 0, end = 0;
            for (int i = 0; i < t.ndim; i++)
                if (__builtin_mul_overflow(numel, t.shape[i], &numel)) goto overflow;
            if (__builtin_mul_overflow(numel, elem, &span) ||
                __builtin_add_overflow(base, o1, &end))
                goto overflow;
            t.off = base + o0;
            t.nbytes = o1 - o0;
            /* the span must equal elements x element size, and lie inside the file */
            if (t.nbytes != span || end > (int64_t)sb.st_size) {
                fprintf(stderr, "k3gc: %s: %s spans %lld bytes, its shape %lld\n", path, name,
                        (long long)t.nbytes, (long long)span);
                goto done;
            }
            t.name = strdup(name);
            if (!t.name || push_tensor(st, &t) != 0) goto done;
        }
        if (js_lit(&s, ',')) continue;
        if (js_lit(&s, '}')) break;
        goto done;
    }
    rc = 0;
    goto done;
overflow:
    fprintf(stderr, "k3gc: %s: a tensor's size overflows\n", path);
done:
    if (rc) fprintf(stderr, "k3gc: %s: malformed header near byte %ld\n", path, (long)(s.p - json));
    free(json);
    return rc;
}

static int cmp_name(const void *a, const void *b)
{
    return strcmp(((const StTensor *)a)->name, ((const StTensor *)b)->name);
}

static int cmp_path(const void *a, const void *b)
{
    return strcmp(*(char *const *)a, *(char *const *)b);
}

static int sort_and_check(K3gcSt *st);

void k3gc_st_close(K3gcSt *st)
{
    if (!st) return;
    for (int i = 0; i < st->nshard; i++) {
        if (!st->borrowed && st->fd && st->fd[i] >= 0) close(st->fd[i]);
        if (!st->borrowed && st->dfd && st->dfd[i] >= 0) close(st->dfd[i]);
        if (st->path) free(st->path[i]);
    }
    for (int i = 0; i < st->nt; i++) free(st->t[i].name);
    free(st->fd);
    free(st->dfd);
    free(st->path);
    free(st->t);
    free(st);
}

int k3gc_st_open(K3gcSt **out, const char *dir)
{
    *out = NULL;
    DIR *d = opendir(dir);
    if (!d) { fprintf(stderr, "k3gc: cannot open directory %s\n", dir); return -1; }
    K3gcSt *st = (K3gcSt *)calloc(1, sizeof *st);
    if (!st) { closedir(d); return -1; }
    int cap = 0;
    struct dirent *e;
    while ((e = readdir(d))) {
        const size_t n = strlen(e->d_name);
        if (n < 12 || strcmp(e->d_name + n - 12, ".safetensors")) continue;
        if (st->nshard == cap) {
            cap = cap ? 2 * cap : 16;
            char **np = (char **)realloc(st->path, (size_t)cap * sizeof *np);
            if (!np) { closedir(d); k3gc_st_close(st); return -1; }
            st->path = np;
        }
        const size_t len = strlen(dir) + n + 2;
        st->path[st->nshard] = (char *)malloc(len);
        if (!st->path[st->nshard]) { closedir(d); k3gc_st_close(st); return -1; }
        snprintf(st->path[st->nshard], len, "%s/%s", dir, e->d_name);
        st->nshard++;
    }
    closedir(d);
    if (!st->nshard) {
        fprintf(stderr, "k3gc: no .safetensors files in %s\n", dir);
        k3gc_st_close(st);
        return -1;
    }
    /* shard numbers stable across machines: sorted by name, not readdir order */
    qsort(st->path, (size_t)st->nshard, sizeof *st->path, cmp_path);
    st->fd = (int *)malloc((size_t)st->nshard * sizeof(int));
    st->dfd = (int *)malloc((size_t)st->nshard * sizeof(int));
    if (!st->fd || !st->dfd) { k3gc_st_close(st); return -1; }
    for (int i = 0; i < st->nshard; i++) st->fd[i] = st->dfd[i] = -1;
    /* K3GC_NO_DIRECT set: ordinary reads only (one binary, both read paths) */
    const int direct = getenv("K3GC_NO_DIRECT") == NULL;
    for (int i = 0; i < st->nshard && direct; i++)
        st->dfd[i] = open(st->path[i], O_RDONLY | O_DIRECT);   /* -1: not supported */
    for (int i = 0; i < st->nshard; i++)
        if (scan_shard(st, i, st->path[i]) != 0) { k3gc_st_close(st); return -1; }
    if (sort_and_check(st) != 0) { k3gc_st_close(st); return -1; }
    *out = st;
    return 0;
}

int k3gc_st_count(const K3gcSt *st) { return st ? st->nt : 0; }

static int sort_and_check(K3gcSt *st)
{
    qsort(st->t, (size_t)st->nt, sizeof *st->t, cmp_name);
    for (int i = 1; i < st->nt; i++)
        if (!strcmp(st->t[i].name, st->t[i - 1].name)) {
            fprintf(stderr, "k3gc: duplicate tensor %s\n", st->t[i].name);
            return -1;
        }
    return 0;
}

/* The engine's own index (a K3St its k3_st_open filled, src/io/k3_st.h:56-70): every
 * tensor's name, shard and span copied into this index, the shards' descriptors borrowed
 * (the engine's k3_st_close closes them, after the cache is freed). */
int k3gc_st_from_engine(K3gcSt **out, const K3St *es)
{
    *out = NULL;
    if (!es || es->nshard < 1 || !es->fd || es->nt < 0 || (es->nt > 0 && !es->t)) return -1;
    K3gcSt *st = (K3gcSt *)calloc(1, sizeof *st);
    if (!st) return -1;
    st->borrowed = 1;
    st->nshard = es->nshard;
    st->fd = (int *)malloc((size_t)st->nshard * sizeof(int));
    st->dfd = (int *)malloc((size_t)st->nshard * sizeof(int));
    if (!st->fd || !st->dfd) { k3gc_st_close(st); return -1; }
    for (int i = 0; i < st->nshard; i++) {
        st->fd[i] = es->fd[i];
        st->dfd[i] = es->dfd ? es->dfd[i] : -1;
    }
    for (int i = 0; i < es->nt; i++) {
        const K3Tensor *et = &es->t[i];
        if (!et->name || et->shard < 0 || et->shard >= es->nshard || et->off < 0 ||
            et->nbytes < 0 || et->ndim < 0 || et->ndim > 4) {
            fprintf(stderr, "k3gc: the engine's index holds a malformed tensor entry %d\n", i);
            k3gc_st_close(st);
            return -1;
        }
        StTensor t;
        memset(&t, 0, sizeof t);
        t.name = strdup(et->name);
        t.shard = et->shard;
        t.dtype_u8 = et->dtype == K3_DT_U8;
        t.ndim = et->ndim;
        for (int k = 0; k < et->ndim; k++) t.shape[k] = et->shape[k];
        t.off = et->off;
        t.nbytes = et->nbytes;
        if (!t.name || push_tensor(st, &t) != 0) {
            free(t.name);
            k3gc_st_close(st);
            return -1;
        }
    }
    if (sort_and_check(st) != 0) { k3gc_st_close(st); return -1; }
    *out = st;
    return 0;
}

static const StTensor *st_find(const K3gcSt *st, const char *name)
{
    int lo = 0, hi = st->nt - 1;
    while (lo <= hi) {
        const int mid = (lo + hi) / 2;
        const int c = strcmp(st->t[mid].name, name);
        if (!c) return &st->t[mid];
        if (c < 0) lo = mid + 1; else hi = mid - 1;
    }
    return NULL;
}

/* ------------------------------------------------------------ expert runs ---- */
int k3gc_st_expert(const K3gcSt *st, int layer, int expert, K3gcExpertRun *r)
{
    static const char *W[3] = {"w1", "w2", "w3"};
    memset(r, 0, sizeof *r);
    if (!st) return -1;
    const StTensor *pk[3], *sc[3];
    for (int i = 0; i < 3; i++) {
        char name[256];
        snprintf(name, sizeof name,
                 "language_model.model.layers.%d.block_sparse_moe.experts.%d.%s.weight_packed",
                 layer, expert, W[i]);
        pk[i] = st_find(st, name);
        snprintf(name, sizeof name,
                 "language_model.model.layers.%d.block_sparse_moe.experts.%d.%s.weight_scale",
                 layer, expert, W[i]);
        sc[i] = st_find(st, name);
        if (!pk[i] || !sc[i]) {
            fprintf(stderr, "k3gc: layer %d expert %d: %s missing\n", layer, expert, W[i]);
            return -1;
        }
        /* src/io/k3_load.c:33-66: U8, 2-D, rows agree, one scale per 32 elements, one shard */
        if (!pk[i]->dtype_u8 || !sc[i]->dtype_u8 || pk[i]->ndim != 2 || sc[i]->ndim != 2 ||
            pk[i]->shape[0] != sc[i]->shape[0] || sc[i]->shape[1] * 32 != 2 * pk[i]->shape[1] ||
            pk[i]->shard != sc[i]->shard || pk[i]->shard != pk[0]->shard) {
            fprintf(stderr, "k3gc: layer %d expert %d: %s is not a 2-D U8 MXFP4 pair with "
                            "group 32 in one shard\n", layer, expert, W[i]);
            return -1;
        }
        r->rows[i] = (int)pk[i]->shape[0];
        r->pcols[i] = (int)pk[i]->shape[1];
        r->p_bytes[i] = pk[i]->nbytes;
        r->s_bytes[i] = sc[i]->nbytes;
        r->p_file[i] = pk[i]->off;
        r->s_file[i] = sc[i]->off;
    }
    r->shard = pk[0]->shard;
    /* one contiguous run when the six spans tile [lowest, highest) exactly and come in
     * the checkpoint order */
    int64_t lo = pk[0]->off, hi = 0, own = 0;
    const StTensor *all[6] = {pk[0], sc[0], pk[1], sc[1], pk[2], sc[2]};
    int ordered = 1;
    for (int i = 0; i < 6; i++) {
        if (all[i]->off < lo) lo = all[i]->off;
        if (all[i]->off + all[i]->nbytes > hi) hi = all[i]->off + all[i]->nbytes;
        own += all[i]->nbytes;
        if (i && all[i]->off != all[i - 1]->off + all[i - 1]->nbytes) ordered = 0;
    }
    r->off = lo;
    r->nbytes = own;
    r->contiguous = hi - lo == own && ordered;
    return 0;
}

static int read_full(int fd, unsigned char *dst, int64_t n, int64_t off)
{
    int64_t got = 0;
    while (got < n) {
        const int64_t want = n - got < ((int64_t)1 << 30) ? n - got : ((int64_t)1 << 30);
        const ssize_t r = pread(fd, dst + got, (size_t)want, (off_t)(off + got));
        if (r <= 0) return -1;
        got += r;
    }
    return 0;
}

/* The 4096-byte-aligned window around [off, off + n) with O_DIRECT into an aligned
 * buffer, then the span into dst. Returns 0, or -1 (the caller then reads buffered). The
 * last window of a shard may run past its end: a short read is fine once the span is in. */
static int read_direct(int dfd, unsigned char *dst, int64_t n, int64_t off)
{
    const int64_t lo = off & ~(int64_t)(ST_ALIGN - 1);
    const int64_t hi = (off + n + ST_ALIGN - 1) & ~(int64_t)(ST_ALIGN - 1);
    const int64_t len = hi - lo, pad = off - lo;
    void *buf = NULL;
    if (posix_memalign(&buf, ST_ALIGN, (size_t)len) != 0) return -1;
    int64_t got = 0;
    while (got < len) {
        const int64_t want = len - got < ST_READ_MAX ? len - got : ST_READ_MAX;
        const ssize_t r = pread(dfd, (char *)buf + got, (size_t)want, (off_t)(lo + got));
        if (r <= 0) break;
        got += r;
    }
    const int ok = got >= pad + n;
    if (ok) memcpy(dst, (char *)buf + pad, (size_t)n);
    free(buf);
    return ok ? 0 : -1;
}

int k3gc_st_direct(const K3gcSt *st)
{
    int n = 0;
    for (int i = 0; st && st->dfd && i < st->nshard; i++) n += st->dfd[i] >= 0;
    return n;
}

/* The run's bytes in the checkpoint order into dst: one read when contiguous (O_DIRECT
 * where the shard has it), six otherwise (src/io/k3_load.c:105-136). */
int k3gc_st_read_run(const K3gcSt *st, const K3gcExpertRun *r, unsigned char *dst)
{
    const int fd = st->fd[r->shard];
    if (r->contiguous) {
        const int dfd = st->dfd ? st->dfd[r->shard] : -1;
        if (dfd >= 0 && read_direct(dfd, dst, r->nbytes, r->off) == 0) return 0;
        return read_full(fd, dst, r->nbytes, r->off);
    }
    int64_t o = 0;
    for (int i = 0; i < 3; i++) {
        if (read_full(fd, dst + o, r->p_bytes[i], r->p_file[i]) != 0) return -1;
        o += r->p_bytes[i];
        if (read_full(fd, dst + o, r->s_bytes[i], r->s_file[i]) != 0) return -1;
        o += r->s_bytes[i];
    }
    return 0;
}

/* The run's bytes into buf (capacity cap): a contiguous run with O_DIRECT straight into
 * buf when buf is 4096-aligned and holds the enclosing 4096-byte window (the run then
 * starts at buf + *pad, as the engine's k3_expert_load_direct leaves it, src/io/k3_st.c:
 * 457-497), otherwise ordinary reads into buf (*pad = 0). Returns 0, or -1 on a short
 * read. */
int k3gc_st_read_run_into(const K3gcSt *st, const K3gcExpertRun *r, unsigned char *buf,
                          int64_t cap, int64_t *pad)
{
    *pad = 0;
    if (r->nbytes > cap) return -1;
    if (r->contiguous) {
        const int dfd = st->dfd ? st->dfd[r->shard] : -1;
        const int64_t lo = r->off & ~(int64_t)(ST_ALIGN - 1);
        const int64_t hi = (r->off + r->nbytes + ST_ALIGN - 1) & ~(int64_t)(ST_ALIGN - 1);
        if (dfd >= 0 && ((uintptr_t)buf & (ST_ALIGN - 1)) == 0 && hi - lo <= cap) {
            int64_t got = 0;
            while (got < hi - lo) {
                const int64_t want = hi - lo - got < ST_READ_MAX ? hi - lo - got : ST_READ_MAX;
                const ssize_t n = pread(dfd, buf + got, (size_t)want, (off_t)(lo + got));
                if (n <= 0) break;
                got += n;
            }
            if (got >= r->off - lo + r->nbytes) {
                *pad = r->off - lo;
                return 0;
            }
        }
        return read_full(st->fd[r->shard], buf, r->nbytes, r->off);
    }
    return k3gc_st_read_run(st, r, buf);
}

/* ------------------------------------------------------------- host tiling ---- */
/* The tiled MXFP4 layout of k3g_tile.hip, written on the host: quad tile (row block rb,
 * 512-column quad Q) at (rb * nQ + Q) * 4352; chunk j's lane L (16 bytes at 1024 j + 16 L)
 * holds row 16 rb + L % 16, block 16 Q + 4 j + L / 16; lane L's scale dword at 4096 + 4 L;
 * scale-255 and padding blocks as zero nibbles with scale 127. */
int k3gc_tile_mxfp4_host(unsigned char *dst, const unsigned char *packed,
                         const unsigned char *scales, int rows, int cols)
{
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 32) return -1;
    const int nq = (cols + 511) / 512, nb = cols / 32;
    for (int rb = 0; rb < rows / 16; rb++)
        for (int Q = 0; Q < nq; Q++) {
            unsigned char *t = dst + ((size_t)rb * nq + Q) * 4352;
            for (int L = 0; L < 64; L++) {
                const int row = 16 * rb + (L & 15);
                for (int j = 0; j < 4; j++) {
                    const int b = 16 * Q + 4 * j + (L >> 4);
                    unsigned char *o = t + 1024 * j + 16 * L;
                    const int live = b < nb && scales[(size_t)row * nb + b] != 255;
                    if (live) memcpy(o, packed + (size_t)row * (cols / 2) + 16 * (size_t)b, 16);
                    else memset(o, 0, 16);
                    t[4096 + 4 * L + j] = live ? scales[(size_t)row * nb + b] : 127;
                }
            }
        }
    return 0;
}

/* ------------------------------------------------------------ into the bank ---- */
int k3gc_bank_load(K3gcBank *b, const K3gcSt *st, int ck_layer0, int bank_layer0, int n_layers)
{
    if (!b || !st || !b->layer_host || n_layers < 1 || bank_layer0 < 0 ||
        bank_layer0 + n_layers > b->n_layers || ck_layer0 < 0)
        return -1;
    const int tiled = b->layout == K3G_EXPERT_MXFP4_TILED;
    unsigned char *buf = NULL;
    int64_t bufcap = 0;
    for (int l = 0; l < n_layers; l++)
        for (int e = 0; e < b->n_experts; e++) {
            K3gcExpertRun r;
            if (k3gc_st_expert(st, ck_layer0 + l, e, &r) != 0) { free(buf); return -1; }
            /* a bank with a layer shape takes experts of that shape only: w1/w3 [inter]
             * [hidden/2], w2 [hidden][inter/2] */
            if (b->hidden > 0 &&
                (r.rows[0] != b->inter || 2 * r.pcols[0] != b->hidden || r.rows[2] != b->inter ||
                 2 * r.pcols[2] != b->hidden || r.rows[1] != b->hidden ||
                 2 * r.pcols[1] != b->inter)) {
                fprintf(stderr, "k3gc_bank_load: layer %d expert %d is not a hidden %d x inter "
                                "%d expert\n", ck_layer0 + l, e, b->hidden, b->inter);
                free(buf);
                return -1;
            }
            unsigned char *dst = (unsigned char *)k3gc_bank_expert(b, bank_layer0 + l, e);
            if (b->hidden == 0) {
                /* a bank without a layer shape keeps the runs' matrix offsets: every run
                 * must share them */
                int64_t o[6], at = 0;
                for (int i = 0; i < 3; i++) {
                    o[2 * i] = at;
                    at += r.p_bytes[i];
                    o[2 * i + 1] = at;
                    at += r.s_bytes[i];
                }
                if (!b->raw_geometry) {
                    memcpy(b->raw_off, o, sizeof o);
                    b->raw_geometry = 1;
                } else if (memcmp(b->raw_off, o, sizeof o) != 0) {
                    fprintf(stderr, "k3gc_bank_load: layer %d expert %d: matrix sizes differ "
                                    "from the bank's other runs\n", ck_layer0 + l, e);
                    return -1;
                }
            }
            if (!tiled) {
                if (r.nbytes != b->expert_bytes) {
                    fprintf(stderr, "k3gc_bank_load: run of %lld bytes for %lld-byte slots\n",
                            (long long)r.nbytes, (long long)b->expert_bytes);
                    return -1;
                }
                if (k3gc_st_read_run(st, &r, dst) != 0) {
                    fprintf(stderr, "k3gc_bank_load: short read, layer %d expert %d\n",
                            ck_layer0 + l, e);
                    return -1;
                }
                continue;
            }
            if (r.nbytes > bufcap) {
                unsigned char *nb = (unsigned char *)realloc(buf, (size_t)r.nbytes);
                if (!nb) { free(buf); return -1; }
                buf = nb;
                bufcap = r.nbytes;
            }
            if (k3gc_st_read_run(st, &r, buf) != 0) { free(buf); return -1; }
            /* w1, w3, w2 tiled back to back, as the tiled bank holds them */
            const K3gExpertLayout g = k3g_expert_layout(b->hidden, b->inter);
            const size_t t13 = k3k_tiled_mxfp4_bytes(b->inter, b->hidden);
            if (k3gc_tile_mxfp4_host(dst, buf + g.p1_off, buf + g.s1_off, b->inter, b->hidden) ||
                k3gc_tile_mxfp4_host(dst + t13, buf + g.p3_off, buf + g.s3_off, b->inter,
                                     b->hidden) ||
                k3gc_tile_mxfp4_host(dst + 2 * t13, buf + g.p2_off, buf + g.s2_off, b->hidden,
                                     b->inter)) {
                free(buf);
                return -1;
            }
        }
    free(buf);
    return 0;
}
