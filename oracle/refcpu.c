/*
 * refcpu.c -- CPU oracle for llama.go's sparse-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates the reference's Go CPU code
 * (AndersHsueh/llama.go) in C so that the HIP path can be checked against it
 * on the same inputs.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it, and only as the reference result or the timed CPU
 * baseline; the product library never links or calls it.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math), so
 * that float arithmetic is IEEE single with no FMA contraction, like Go's
 * gc compiler on amd64.
 *
 * Pinning: every function here is checked by tests/test_oracle.py against
 * known-answer vectors, float64 brute force, closed forms or invariants
 * (the header of that file lists which check pins which function).
 */
#define _POSIX_C_SOURCE 200809L /* pread, strdup */
#include "refcpu.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---- gguf/types.go:70-102 ------------------------------------------------ */
static int type_info(int t, int *block, int *tsize) {
    switch (t) {
    case REFCPU_F32: *block = 1; *tsize = 4; return 0;   /* types.go:71 */
    case REFCPU_F16: *block = 1; *tsize = 2; return 0;   /* types.go:72 */
    case REFCPU_Q4_0: *block = 32; *tsize = 18; return 0; /* types.go:73 */
    case REFCPU_Q8_0: *block = 32; *tsize = 34; return 0; /* types.go:77 */
    default: return -1;
    }
}

int64_t refcpu_byte_size(int t, int64_t n) {
    int bs, ts;
    if (type_info(t, &bs, &ts) != 0) return -1;          /* types.go:93-96 */
    if (n % bs != 0) return -1;                          /* types.go:98-100 */
    return (n / bs) * (int64_t)ts;                       /* types.go:101 */
}

/* ---- tensor/dtype.go:417-443 -------------------------------------------- */
static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float refcpu_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (uint32_t)((h >> 10) & 0x1F);
    uint32_t mant = (uint32_t)(h & 0x3FF);
    switch (exp) {
    case 0:
        if (mant == 0) return bits_f32(sign);
        /* subnormal: normalise (dtype.go:427-434) */
        exp = 1;
        while ((mant & 0x400) == 0) {
            mant <<= 1;
            exp--; /* uint32 wrap, exactly as Go's uint32 arithmetic */
        }
        mant &= ~(uint32_t)0x400;
        return bits_f32(sign | ((exp + 127 - 15) << 23) | (mant << 13));
    case 31:
        if (mant == 0) return bits_f32(sign | 0x7F800000u); /* +-Inf */
        return bits_f32(sign | 0x7FC00000u);                /* NaN, payload dropped */
    default:
        return bits_f32(sign | ((exp + 127 - 15) << 23) | (mant << 13));
    }
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- tensor/dtype.go:12-82, 249-268 ------------------------------------- */
int64_t refcpu_dequantize(const uint8_t *raw, int64_t nbytes, int t, float *out) {
    switch (t) {
    case REFCPU_F32: { /* dtype.go:26-38 */
        if (nbytes % 4) return -1;
        int64_t n = nbytes / 4;
        for (int64_t i = 0; i < n; i++) {
            uint32_t u = (uint32_t)raw[4 * i] | ((uint32_t)raw[4 * i + 1] << 8) |
                         ((uint32_t)raw[4 * i + 2] << 16) | ((uint32_t)raw[4 * i + 3] << 24);
            out[i] = bits_f32(u);
        }
        return n;
    }
    case REFCPU_F16: { /* dtype.go:12-24 */
        if (nbytes % 2) return -1;
        int64_t n = nbytes / 2;
        for (int64_t i = 0; i < n; i++) out[i] = refcpu_f16_to_f32(le16(raw + 2 * i));
        return n;
    }
    case REFCPU_Q8_0: { /* dtype.go:41-58 */
        if (nbytes % 34) return -1;
        int64_t nb = nbytes / 34;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = raw + b * 34;
            float scale = refcpu_f16_to_f32(le16(base));
            for (int i = 0; i < 32; i++) {
                int8_t q = (int8_t)base[2 + i];
                out[b * 32 + i] = (float)q * scale;
            }
        }
        return nb * 32;
    }
    case REFCPU_Q4_0: { /* dtype.go:62-82 -- interleaved nibble order */
        if (nbytes % 18) return -1;
        int64_t nb = nbytes / 18;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = raw + b * 18;
            float scale = refcpu_f16_to_f32(le16(base));
            for (int i = 0; i < 16; i++) {
                uint8_t packed = base[2 + i];
                int8_t lo = (int8_t)((uint8_t)(packed & 0x0F) - 8);
                int8_t hi = (int8_t)((uint8_t)(packed >> 4) - 8);
                out[b * 32 + i * 2] = (float)lo * scale;
                out[b * 32 + i * 2 + 1] = (float)hi * scale;
            }
        }
        return nb * 32;
    }
    default:
        return -1; /* dtype.go:266 */
    }
}

/* ---- tensor/ops.go ------------------------------------------------------ */
/* Threads that refcpu_matmulvec splits its rows over (1: the reference's one
 * goroutine).  Each row's sum keeps its sequential order on whichever thread
 * computes it, so the results are bit-identical for every setting; more
 * threads only shorten the tests that run long sequences through the oracle. */
static int g_threads = 1;

void refcpu_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }

/* [0, n) split into g_threads contiguous ranges, one per thread (this thread
 * takes the first); with fewer than min_each items per thread fewer threads
 * are used.  Every caller gives each item its own outputs, computed in the
 * reference's order, so the split changes no result. */
typedef void (*range_fn)(void *ctx, int i0, int i1);
typedef struct {
    range_fn fn;
    void *ctx;
    int i0, i1;
} range_part;

static void *range_worker(void *arg) {
    range_part *p = (range_part *)arg;
    p->fn(p->ctx, p->i0, p->i1);
    return NULL;
}

static void par_for(int n, int min_each, range_fn fn, void *ctx) {
    int nt = g_threads;
    if (min_each < 1) min_each = 1;
    if (nt > n / min_each) nt = n / min_each;
    if (nt <= 1) {
        fn(ctx, 0, n);
        return;
    }
    range_part parts[64];
    pthread_t th[64];
    int started[64];
    for (int k = 0; k < nt; k++) {
        parts[k] = (range_part){fn, ctx, (int)((int64_t)n * k / nt), (int)((int64_t)n * (k + 1) / nt)};
        started[k] = k > 0 && pthread_create(&th[k], NULL, range_worker, &parts[k]) == 0;
    }
    range_worker(&parts[0]);
    for (int k = 1; k < nt; k++) {
        if (started[k]) pthread_join(th[k], NULL);
        else range_worker(&parts[k]); /* no thread: this one takes that range */
    }
}

typedef struct {
    const float *w, *x;
    float *y;
    int in_dim;
} mv_ctx;

static void matmulvec_rows(void *arg, int r0, int r1) {
    const mv_ctx *c = (const mv_ctx *)arg;
    for (int i = r0; i < r1; i++) { /* ops.go:51-58 */
        float sum = 0.0f;
        const float *row = c->w + (size_t)i * c->in_dim;
        for (int j = 0; j < c->in_dim; j++) sum += row[j] * c->x[j];
        c->y[i] = sum;
    }
}

void refcpu_matmulvec(const float *w, int out_dim, int in_dim, const float *x, float *y) {
    mv_ctx c = {w, x, y, in_dim};
    if ((int64_t)out_dim * in_dim < (1 << 20)) { /* small: not worth a thread */
        matmulvec_rows(&c, 0, out_dim);
        return;
    }
    par_for(out_dim, 1, matmulvec_rows, &c);
}

void refcpu_relu(float *x, int n) { /* ops.go:168-174: NaN and -0.0 pass through */
    for (int i = 0; i < n; i++)
        if (x[i] < 0) x[i] = 0;
}

void refcpu_silu(float *x, int n) { /* ops.go:177-181 */
    for (int i = 0; i < n; i++) {
        float v = x[i];
        x[i] = v / (1.0f + (float)exp((double)(-v)));
    }
}

void refcpu_gelu(float *x, int n) { /* ops.go:184-189, untyped consts become float32 */
    const float c = (float)0.7978845608028654;
    const float k = (float)0.044715;
    for (int i = 0; i < n; i++) {
        float v = x[i];
        float inner = c * (v + k * v * v * v);
        x[i] = 0.5f * v * (1.0f + (float)tanh((double)inner));
    }
}

void refcpu_activation(int act, float *x, int n) { /* ffn_flash.go:303-312 */
    if (act == REFCPU_ACT_SILU)
        refcpu_silu(x, n);
    else if (act == REFCPU_ACT_GELU)
        refcpu_gelu(x, n);
    else
        refcpu_relu(x, n);
}

void refcpu_rmsnorm(const float *x, const float *w, float *out, int n, float eps) {
    float sum_sq = 0.0f; /* ops.go:124-127 */
    for (int i = 0; i < n; i++) sum_sq += x[i] * x[i];
    float rms = (float)sqrt((double)(sum_sq / (float)n) + (double)eps);
    float scale = 1.0f / rms;
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

void refcpu_layernorm(const float *x, const float *w, const float *b, float *out, int n,
                      float eps) {
    float mean = 0.0f; /* ops.go:148-162 */
    for (int i = 0; i < n; i++) mean += x[i];
    mean /= (float)n;
    float var = 0.0f;
    for (int i = 0; i < n; i++) {
        float d = x[i] - mean;
        var += d * d;
    }
    var /= (float)n;
    float sd = (float)sqrt((double)var + (double)eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] - mean) / sd * w[i] + b[i];
}

/* ---- inference/forward.go:463-479 --------------------------------------- */
void refcpu_softmax_inplace(float *v, int n) {
    float maxv = v[0];
    for (int i = 0; i < n; i++)
        if (v[i] > maxv) maxv = v[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        float e = (float)exp((double)(v[i] - maxv));
        v[i] = e;
        sum += e;
    }
    for (int i = 0; i < n; i++) v[i] /= sum;
}

/* ---- inference/predictor.go --------------------------------------------- */
int refcpu_select(const float *logits, int ff, float thr, int32_t *active) {
    int n = 0; /* predictor.go:76-82 */
    for (int i = 0; i < ff; i++)
        if (logits[i] > thr) active[n++] = i;
    return n;
}

int refcpu_predict(const float *wup, const float *wout, const float *bias, int h, int rank,
                   int ff, const float *a, float thr, int32_t *active, float *logits_out) {
    if (!wup || !wout) return -1; /* predictor.go:52-54 */
    float *hidden = (float *)malloc(sizeof(float) * (size_t)rank);
    float *logits = logits_out ? logits_out : (float *)malloc(sizeof(float) * (size_t)ff);
    refcpu_matmulvec(wup, rank, h, a, hidden); /* :57 */
    refcpu_relu(hidden, rank);                 /* :61 */
    refcpu_matmulvec(wout, ff, rank, hidden, logits); /* :64 */
    if (bias)                                  /* :69-73, tensor.Add ops.go:87-95 */
        for (int i = 0; i < ff; i++) logits[i] += bias[i];
    int n = refcpu_select(logits, ff, thr, active);
    free(hidden);
    if (!logits_out) free(logits);
    return n;
}

/* ---- flash/storage.go:246-319 ------------------------------------------- */
typedef struct {
    const uint8_t *raw;
    int64_t rb;
    int t, in_dim, out_dim;
    const int32_t *rows;
    float *out;
    int *errs;
} rr_ctx;

static void read_rows_range(void *arg, int i0, int i1) {
    rr_ctx *c = (rr_ctx *)arg;
    for (int i = i0; i < i1; i++) {
        int32_t r = c->rows[i];
        if (r < 0 || r >= c->out_dim) { /* :292-294 */
            c->errs[i] = -2;
            continue;
        }
        int64_t off = (int64_t)r * c->rb; /* :296 */
        if (refcpu_dequantize(c->raw + off, c->rb, c->t, c->out + (size_t)i * c->in_dim) < 0)
            c->errs[i] = -1;
    }
}

int refcpu_read_rows(const uint8_t *raw, int t, int in_dim, int out_dim, const int32_t *rows,
                     int n_rows, float *out) {
    int64_t rb = refcpu_byte_size(t, in_dim); /* :253 */
    if (rb < 0) return -1;
    if (n_rows <= 0) return 0;
    rr_ctx c = {raw, rb, t, in_dim, out_dim, rows, out, (int *)calloc((size_t)n_rows, sizeof(int))};
    par_for(n_rows, 64, read_rows_range, &c);
    int rc = 0;
    for (int i = 0; i < n_rows && rc == 0; i++) rc = c.errs[i]; /* the first failing row */
    free(c.errs);
    return rc;
}

/* ---- flash/storage.go:246-319 ReadRowsParallel --------------------------- */
typedef struct {
    const char *path;
    int64_t offset, rb;
    int t, in_dim, out_dim, n_rows;
    const int32_t *rows;
    float *out;
    int *errs;          /* per destination row, :259 */
    atomic_int next;    /* the job queue, :265-270 */
} rows_job;

static void *rows_worker(void *arg) { /* :278-312 */
    rows_job *j = (rows_job *)arg;
    int fd = open(j->path, O_RDONLY); /* its own descriptor, :281 */
    uint8_t *buf = NULL;
    for (;;) {
        int i = atomic_fetch_add(&j->next, 1);
        if (i >= j->n_rows) break;
        if (fd < 0) { j->errs[i] = -3; continue; } /* :282-287 */
        int32_t r = j->rows[i];
        if (r < 0 || r >= j->out_dim) { j->errs[i] = -2; continue; } /* :291-294 */
        buf = (uint8_t *)malloc((size_t)j->rb); /* :296-297, a buffer per row */
        int64_t done = 0, off = j->offset + (int64_t)r * j->rb;
        while (done < j->rb) {
            ssize_t n = pread(fd, buf + done, (size_t)(j->rb - done), (off_t)(off + done));
            if (n <= 0) break;
            done += n;
        }
        if (done < j->rb) j->errs[i] = -4; /* :298-300 */
        else if (refcpu_dequantize(buf, j->rb, j->t, j->out + (size_t)i * j->in_dim) < 0)
            j->errs[i] = -1; /* :302-305 */
        free(buf);
    }
    if (fd >= 0) close(fd);
    return NULL;
}

int refcpu_read_rows_file(const char *path, int64_t tensor_offset, int t, int in_dim,
                          int out_dim, const int32_t *rows, int n_rows, int nthreads,
                          float *out) {
    int64_t rb = refcpu_byte_size(t, in_dim); /* :253 */
    if (rb < 0) return -1;
    if (n_rows <= 0) return 0;
    if (nthreads <= 0) nthreads = 32; /* :272-274 */
    rows_job j;
    j.path = path;
    j.offset = tensor_offset;
    j.rb = rb;
    j.t = t;
    j.in_dim = in_dim;
    j.out_dim = out_dim;
    j.n_rows = n_rows;
    j.rows = rows;
    j.out = out;
    j.errs = (int *)calloc((size_t)n_rows, sizeof(int));
    atomic_init(&j.next, 0);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    int started = 0;
    for (int i = 0; i < nthreads; i++)
        if (pthread_create(&th[i], NULL, rows_worker, &j) == 0) started++;
        else break;
    if (started == 0) rows_worker(&j); /* no thread could start: read on this one */
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL); /* :315 */
    int rc = 0;
    for (int i = 0; i < n_rows && rc == 0; i++) rc = j.errs[i]; /* :317-321 */
    free(th);
    free(j.errs);
    return rc;
}

/* ---- inference/ffn_flash.go:254-299 ------------------------------------- */
/* :272-298 on rows already read and dequantized.  The up dots split over
 * neurons and the down sums over output elements; every output element still
 * adds the neurons in ascending order, so the split changes no result. */
typedef struct {
    const float *up_rows, *down_rows, *x;
    float *inter, *out;
    int h, n_active;
} sc_ctx;

static void sparse_up_range(void *arg, int j0, int j1) {
    sc_ctx *c = (sc_ctx *)arg;
    for (int j = j0; j < j1; j++) { /* :273-281 */
        const float *row = c->up_rows + (size_t)j * c->h;
        float dot = 0.0f;
        for (int d = 0; d < c->h; d++) dot += row[d] * c->x[d];
        c->inter[j] = dot;
    }
}

static void sparse_down_range(void *arg, int d0, int d1) {
    sc_ctx *c = (sc_ctx *)arg;
    for (int j = 0; j < c->n_active; j++) { /* :288-298 */
        if (c->inter[j] == 0) continue;
        const float *row = c->down_rows + (size_t)j * c->h;
        float scale = c->inter[j];
        for (int d = d0; d < d1; d++) c->out[d] += scale * row[d];
    }
}

static void sparse_compute(const float *up_rows, const float *down_rows, int h, const float *x,
                           int n_active, int act, float *out) {
    float *inter = (float *)malloc(sizeof(float) * (size_t)n_active);
    sc_ctx c = {up_rows, down_rows, x, inter, out, h, n_active};
    par_for(n_active, 64, sparse_up_range, &c);
    refcpu_activation(act, inter, n_active); /* :284-285 */
    par_for(h, 256, sparse_down_range, &c);
    free(inter);
}

int refcpu_ffn_sparse_load(const uint8_t *up_raw, const uint8_t *down_t_raw, int t, int h,
                           int ff, const float *x, const int32_t *active, int n_active,
                           int act, float *out) {
    memset(out, 0, sizeof(float) * (size_t)h);
    if (n_active == 0) return 0; /* :255-257 */
    float *up_rows = (float *)malloc(sizeof(float) * (size_t)n_active * h);
    float *down_rows = (float *)malloc(sizeof(float) * (size_t)n_active * h);
    int rc = refcpu_read_rows(up_raw, t, h, ff, active, n_active, up_rows); /* :262 */
    if (rc == 0) rc = refcpu_read_rows(down_t_raw, t, h, ff, active, n_active, down_rows);
    if (rc == 0) sparse_compute(up_rows, down_rows, h, x, n_active, act, out);
    free(up_rows);
    free(down_rows);
    return rc;
}

int refcpu_ffn_sparse_load_file(const char *path, int64_t up_offset, int64_t down_t_offset,
                                int t, int h, int ff, const float *x, const int32_t *active,
                                int n_active, int act, int nthreads, float *out) {
    memset(out, 0, sizeof(float) * (size_t)h);
    if (n_active == 0) return 0; /* :255-257 */
    float *up_rows = (float *)malloc(sizeof(float) * (size_t)n_active * h);
    float *down_rows = (float *)malloc(sizeof(float) * (size_t)n_active * h);
    int rc = refcpu_read_rows_file(path, up_offset, t, h, ff, active, n_active, nthreads,
                                   up_rows); /* :262-265 */
    if (rc == 0)
        rc = refcpu_read_rows_file(path, down_t_offset, t, h, ff, active, n_active, nthreads,
                                   down_rows); /* :267-270 */
    if (rc == 0) sparse_compute(up_rows, down_rows, h, x, n_active, act, out);
    free(up_rows);
    free(down_rows);
    return rc;
}

/* ---- inference/forward.go:318-353, 428-445 ------------------------------ */
int refcpu_ffn_dense(const uint8_t *up_raw, const uint8_t *down_raw, int t, int h, int ff,
                     const float *x, int act, float *out) {
    int64_t nu = (int64_t)h * ff;
    int64_t bu = refcpu_byte_size(t, nu);
    if (bu < 0 || refcpu_byte_size(t, h) < 0 || refcpu_byte_size(t, ff) < 0) return -1;
    float *up = (float *)malloc(sizeof(float) * (size_t)nu);   /* ReadTensor, storage.go:111-128 */
    float *down = (float *)malloc(sizeof(float) * (size_t)nu);
    float *hid = (float *)malloc(sizeof(float) * (size_t)ff);
    refcpu_dequantize(up_raw, bu, t, up);
    refcpu_dequantize(down_raw, bu, t, down);
    refcpu_matmulvec(up, ff, h, x, hid);   /* forward.go:343: FFNUp shape [F, h] */
    refcpu_activation(act, hid, ff);       /* forward.go:347 (ReLU) / 361 (GELU) */
    refcpu_matmulvec(down, h, ff, hid, out); /* forward.go:348: FFNDown shape [h, F] */
    free(up);
    free(down);
    free(hid);
    return 0;
}

/* ffnSwiGLU, inference/forward.go:368-389 (the SiLU model's dense FFN,
 * forward.go:328-329): gate = MatMulVec(FFNGate, x); SiLU(gate) (ops.go:177-181);
 * up = MatMulVec(FFNUp, x); Mul(gate, up) (ops.go:223-231, gate[i] *= up[i]);
 * out = MatMulVec(FFNDown, gate). */
int refcpu_ffn_swiglu(const uint8_t *gate_raw, const uint8_t *up_raw, const uint8_t *down_raw,
                      int t, int h, int ff, const float *x, float *out) {
    int64_t nu = (int64_t)h * ff;
    int64_t bu = refcpu_byte_size(t, nu);
    if (bu < 0 || refcpu_byte_size(t, h) < 0 || refcpu_byte_size(t, ff) < 0) return -1;
    float *w = (float *)malloc(sizeof(float) * (size_t)nu);
    float *gate = (float *)malloc(sizeof(float) * (size_t)ff);
    float *up = (float *)malloc(sizeof(float) * (size_t)ff);
    refcpu_dequantize(gate_raw, bu, t, w);
    refcpu_matmulvec(w, ff, h, x, gate);
    refcpu_silu(gate, ff);
    refcpu_dequantize(up_raw, bu, t, w);
    refcpu_matmulvec(w, ff, h, x, up);
    for (int i = 0; i < ff; i++) gate[i] *= up[i];
    refcpu_dequantize(down_raw, bu, t, w);
    refcpu_matmulvec(w, h, ff, gate, out);
    free(w);
    free(gate);
    free(up);
    return 0;
}

/* ---- inference/window.go ------------------------------------------------ */
struct refcpu_neuron_cache {
    float *matrix;       /* [max_neurons, 2*hidden] bundled up|down, window.go:23 */
    int *pointers;       /* matrix row -> neuron, :25 */
    int *in_cache;       /* neuron -> matrix row or -1 (the Go map), :27 */
    int32_t **last_k;    /* ring of active sets, :30 */
    int *last_k_len;
    int *last_k_set;     /* non-nil flag for each ring slot */
    int window_head;     /* :31 */
    int num_used, max_neurons, hidden, window, ff;
    const uint8_t *up_raw, *down_raw;
    int type;
    char *path; /* file-backed rows when set */
    int64_t up_off, down_off;
    int nthreads;
};

refcpu_neuron_cache *refcpu_nc_new(int max_neurons, int hidden, int window, int ff,
                                   const uint8_t *up_raw, const uint8_t *down_raw, int t) {
    refcpu_neuron_cache *c = (refcpu_neuron_cache *)calloc(1, sizeof(*c)); /* window.go:48-63 */
    c->matrix = (float *)calloc((size_t)max_neurons * 2 * hidden, sizeof(float));
    c->pointers = (int *)calloc((size_t)max_neurons, sizeof(int));
    c->in_cache = (int *)malloc(sizeof(int) * (size_t)ff);
    for (int i = 0; i < ff; i++) c->in_cache[i] = -1;
    c->last_k = (int32_t **)calloc((size_t)window, sizeof(int32_t *));
    c->last_k_len = (int *)calloc((size_t)window, sizeof(int));
    c->last_k_set = (int *)calloc((size_t)window, sizeof(int));
    c->max_neurons = max_neurons;
    c->hidden = hidden;
    c->window = window;
    c->ff = ff;
    c->up_raw = up_raw;
    c->down_raw = down_raw;
    c->type = t;
    return c;
}

refcpu_neuron_cache *refcpu_nc_new_file(int max_neurons, int hidden, int window, int ff,
                                        const char *path, int64_t up_offset,
                                        int64_t down_t_offset, int t, int nthreads) {
    refcpu_neuron_cache *c = refcpu_nc_new(max_neurons, hidden, window, ff, NULL, NULL, t);
    c->path = strdup(path);
    c->up_off = up_offset;
    c->down_off = down_t_offset;
    c->nthreads = nthreads;
    return c;
}

void refcpu_nc_free(refcpu_neuron_cache *c) {
    if (!c) return;
    free(c->path);
    for (int i = 0; i < c->window; i++) free(c->last_k[i]);
    free(c->last_k);
    free(c->last_k_len);
    free(c->last_k_set);
    free(c->matrix);
    free(c->pointers);
    free(c->in_cache);
    free(c);
}

static void nc_evict(refcpu_neuron_cache *c, int n) { /* window.go:188-204 */
    int row = c->in_cache[n];
    if (row < 0) return;
    int last = c->num_used - 1;
    size_t w = (size_t)2 * c->hidden;
    if (row != last) {
        memcpy(c->matrix + (size_t)row * w, c->matrix + (size_t)last * w, w * sizeof(float));
        c->pointers[row] = c->pointers[last];
        c->in_cache[c->pointers[row]] = row;
    }
    c->in_cache[n] = -1;
    c->num_used--;
}

static int nc_load_rows(refcpu_neuron_cache *c, const int32_t *neurons, int n) {
    int h = c->hidden; /* window.go:207-245 */
    float *up = (float *)malloc(sizeof(float) * (size_t)n * h);
    float *down = (float *)malloc(sizeof(float) * (size_t)n * h);
    int rc;
    if (c->path) { /* :211, :216 */
        rc = refcpu_read_rows_file(c->path, c->up_off, c->type, h, c->ff, neurons, n,
                                   c->nthreads, up);
        if (rc == 0)
            rc = refcpu_read_rows_file(c->path, c->down_off, c->type, h, c->ff, neurons, n,
                                       c->nthreads, down);
    } else {
        rc = refcpu_read_rows(c->up_raw, c->type, h, c->ff, neurons, n, up); /* :211 */
        if (rc == 0) rc = refcpu_read_rows(c->down_raw, c->type, h, c->ff, neurons, n, down);
    }
    if (rc == 0) {
        for (int j = 0; j < n; j++) {
            if (c->num_used >= c->max_neurons) { /* grow by 10%: :222-232 */
                int new_cap = c->max_neurons + c->max_neurons / 10 + 1;
                c->matrix = (float *)realloc(c->matrix, sizeof(float) * (size_t)new_cap * 2 * h);
                c->pointers = (int *)realloc(c->pointers, sizeof(int) * (size_t)new_cap);
                c->max_neurons = new_cap;
            }
            int row = c->num_used;
            c->pointers[row] = neurons[j];
            c->in_cache[neurons[j]] = row;
            float *dest = c->matrix + (size_t)row * 2 * h; /* :238-240 */
            memcpy(dest, up + (size_t)j * h, sizeof(float) * (size_t)h);
            memcpy(dest + h, down + (size_t)j * h, sizeof(float) * (size_t)h);
            c->num_used++;
        }
    }
    free(up);
    free(down);
    return rc;
}

int refcpu_nc_update(refcpu_neuron_cache *c, const int32_t *active, int n_active,
                     int *n_loaded_out, int32_t *load_list_out) {
    int head = c->window_head;
    if (c->last_k_set[head]) { /* window.go:73-95 */
        char *still = (char *)calloc((size_t)c->ff, 1);
        for (int i = 0; i < c->window; i++) {
            if (i == head || !c->last_k_set[i]) continue;
            for (int j = 0; j < c->last_k_len[i]; j++) still[c->last_k[i][j]] = 1;
        }
        for (int j = 0; j < n_active; j++) still[active[j]] = 1;
        for (int j = 0; j < c->last_k_len[head]; j++) {
            int n = c->last_k[head][j];
            if (!still[n]) nc_evict(c, n);
        }
        free(still);
    }
    int32_t *to_load = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_active ? n_active : 1));
    int nl = 0; /* :98-103 */
    for (int j = 0; j < n_active; j++)
        if (c->in_cache[active[j]] < 0) to_load[nl++] = active[j];
    int rc = 0;
    if (nl > 0) rc = nc_load_rows(c, to_load, nl); /* :106-110 */
    if (n_loaded_out) *n_loaded_out = nl;
    if (load_list_out) memcpy(load_list_out, to_load, sizeof(int32_t) * (size_t)nl);
    free(to_load);
    if (rc != 0) return rc;
    /* :113-114 record the active set (a private copy) and advance the head */
    free(c->last_k[head]);
    c->last_k[head] = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_active ? n_active : 1));
    memcpy(c->last_k[head], active, sizeof(int32_t) * (size_t)n_active);
    c->last_k_len[head] = n_active;
    c->last_k_set[head] = 1;
    c->window_head = (head + 1) % c->window;
    return 0;
}

int refcpu_nc_ffn_forward(refcpu_neuron_cache *c, const float *x, const int32_t *active,
                          int n_active, int act, float *out) {
    int h = c->hidden; /* window.go:143-180 */
    float *inter = (float *)calloc((size_t)(n_active ? n_active : 1), sizeof(float));
    for (int j = 0; j < n_active; j++) {
        int row = c->in_cache[active[j]];
        if (row < 0) continue; /* :150-152 */
        const float *up = c->matrix + (size_t)row * 2 * h;
        float dot = 0.0f;
        for (int d = 0; d < h; d++) dot += up[d] * x[d];
        inter[j] = dot;
    }
    refcpu_activation(act, inter, n_active);
    memset(out, 0, sizeof(float) * (size_t)h);
    for (int j = 0; j < n_active; j++) {
        if (inter[j] == 0) continue; /* :167-169 */
        int row = c->in_cache[active[j]];
        if (row < 0) continue;
        const float *down = c->matrix + (size_t)row * 2 * h + h;
        float scale = inter[j];
        for (int d = 0; d < h; d++) out[d] += scale * down[d];
    }
    free(inter);
    return 0;
}

int refcpu_nc_num_cached(const refcpu_neuron_cache *c) { return c->num_used; } /* :183 */

int refcpu_nc_is_cached(const refcpu_neuron_cache *c, int n) {
    return (n >= 0 && n < c->ff && c->in_cache[n] >= 0) ? 1 : 0;
}

/* ---- inference/moe_forward.go:32-150 ------------------------------------ */
int refcpu_moe_route(const float *logits_in, int n_exp, int k, int32_t *ids_out, float *w_out) {
    if (k <= 0 || n_exp <= 0 || k > n_exp) return -1;
    float *p = (float *)malloc(sizeof(float) * (size_t)n_exp);
    int *idx = (int *)malloc(sizeof(int) * (size_t)n_exp);
    memcpy(p, logits_in, sizeof(float) * (size_t)n_exp);
    refcpu_softmax_inplace(p, n_exp); /* :47 */
    for (int i = 0; i < n_exp; i++) idx[i] = i;
    /* :58 sort.Slice descending.  Go's pdqsort runs insertion sort for n <= 12,
     * which keeps equal scores in index order; a stable insertion sort restates it. */
    for (int i = 1; i < n_exp; i++) {
        int cur = idx[i];
        int j = i;
        while (j > 0 && p[cur] > p[idx[j - 1]]) {
            idx[j] = idx[j - 1];
            j--;
        }
        idx[j] = cur;
    }
    float wsum = 0.0f; /* :62-68 */
    for (int i = 0; i < k; i++) wsum += p[idx[i]];
    if (wsum < 1e-9f) wsum = 1.0f;
    for (int i = 0; i < k; i++) {
        ids_out[i] = idx[i];
        w_out[i] = p[idx[i]] / wsum; /* :73 e.score/wsum */
    }
    free(p);
    free(idx);
    return 0;
}

int refcpu_moe_ffn(const float *router, const uint8_t *gate_raw, const uint8_t *up_raw,
                   const uint8_t *down_raw, int t, int hidden, int eff, int n_exp, int k,
                   const float *x, float *out, int32_t *ids_out, float *w_out) {
    if (k <= 0 || n_exp <= 0 || eff <= 0) return -1; /* :38-40 */
    if (k > n_exp) return -1;
    int64_t rb_h = refcpu_byte_size(t, hidden);
    int64_t rb_f = refcpu_byte_size(t, eff);
    if (rb_h < 0 || rb_f < 0) return -1;
    float *logits = (float *)malloc(sizeof(float) * (size_t)n_exp);
    refcpu_matmulvec(router, n_exp, hidden, x, logits); /* :43 */
    int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
    float *ws = (float *)malloc(sizeof(float) * (size_t)k);
    refcpu_moe_route(logits, n_exp, k, ids, ws);
    float *gu = (float *)malloc(sizeof(float) * (size_t)eff * hidden); /* ExpertScratch */
    float *dn = (float *)malloc(sizeof(float) * (size_t)hidden * eff);
    float *gate = (float *)malloc(sizeof(float) * (size_t)eff);
    float *up = (float *)malloc(sizeof(float) * (size_t)eff);
    float *hv = (float *)malloc(sizeof(float) * (size_t)eff);
    memset(out, 0, sizeof(float) * (size_t)hidden); /* :71 */
    for (int s = 0; s < k; s++) {                   /* :72-77 */
        int e = ids[s];
        float w = ws[s];
        /* :96 ReadContiguousRows(gate, e*eff, eff) -- storage.go:72-94 */
        refcpu_dequantize(gate_raw + (int64_t)e * eff * rb_h, rb_h * eff, t, gu);
        for (int j = 0; j < eff; j++) { /* :102-109 */
            const float *row = gu + (size_t)j * hidden;
            float dot = 0.0f;
            for (int d = 0; d < hidden; d++) dot += row[d] * x[d];
            gate[j] = dot;
        }
        refcpu_dequantize(up_raw + (int64_t)e * eff * rb_h, rb_h * eff, t, gu); /* :112 */
        for (int j = 0; j < eff; j++) { /* :118-125 */
            const float *row = gu + (size_t)j * hidden;
            float dot = 0.0f;
            for (int d = 0; d < hidden; d++) dot += row[d] * x[d];
            up[j] = dot;
        }
        for (int j = 0; j < eff; j++) { /* :128-132 */
            float g = gate[j];
            float silu = g / (1.0f + (float)exp(-(double)g));
            hv[j] = silu * up[j];
        }
        refcpu_dequantize(down_raw + (int64_t)e * hidden * rb_f, rb_f * hidden, t, dn); /* :135 */
        for (int d = 0; d < hidden; d++) { /* :141-148 */
            const float *row = dn + (size_t)d * eff;
            float dot = 0.0f;
            for (int j = 0; j < eff; j++) dot += row[j] * hv[j];
            out[d] += w * dot;
        }
    }
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * (size_t)k);
    if (w_out) memcpy(w_out, ws, sizeof(float) * (size_t)k);
    free(logits);
    free(ids);
    free(ws);
    free(gu);
    free(dn);
    free(gate);
    free(up);
    free(hv);
    return 0;
}

/* ---- Falcon decode on the sparse FFN path ------------------------------- */
struct refcpu_falcon {
    refcpu_falcon_params p;
    float *embed, *wq, *wk, *wv, *wo, *lm; /* dequantized at load (loader/ReadTensor) */
    float *kcache, *vcache;                 /* [n_layers][max_seq][kv_dim] (kvcache.go:25-37) */
    int seq_len;                            /* KVCache.SeqLen */
    /* FFN rows read from a GGUF file by ReadRowsParallel (ffn_flash.go:262-270)
     * instead of from p.up / p.down_t when ffn_path is set */
    char *ffn_path;
    int64_t *ffn_up_off, *ffn_down_off; /* [n_layers] tensor offsets in the file */
    int ffn_threads;
};

static float *dequant_rows(const uint8_t *raw, int t, int64_t rows, int cols) {
    const int64_t rb = refcpu_byte_size(t, cols);
    float *out = (float *)malloc(sizeof(float) * (size_t)(rows * cols));
    if (!out || rb < 0) {
        free(out);
        return NULL;
    }
    refcpu_dequantize(raw, rb * rows, t, out);
    return out;
}

refcpu_falcon *refcpu_falcon_new(const refcpu_falcon_params *p) {
    refcpu_falcon *m = (refcpu_falcon *)calloc(1, sizeof(refcpu_falcon));
    if (!m) return NULL;
    m->p = *p;
    const int L = p->n_layers, h = p->hidden, hd = p->head_dim;
    const int qd = p->n_heads * hd, kvd = p->n_kv * hd;
    m->embed = dequant_rows(p->embed, p->t, p->vocab, h);
    m->wq = dequant_rows(p->wq, p->t, (int64_t)L * qd, h);
    m->wk = dequant_rows(p->wk, p->t, (int64_t)L * kvd, h);
    m->wv = dequant_rows(p->wv, p->t, (int64_t)L * kvd, h);
    m->wo = dequant_rows(p->wo, p->t, (int64_t)L * h, qd);
    m->lm = dequant_rows(p->lm_head, p->t, p->vocab, h);
    m->kcache = (float *)calloc((size_t)L * p->max_seq * kvd, sizeof(float));
    m->vcache = (float *)calloc((size_t)L * p->max_seq * kvd, sizeof(float));
    if (!m->embed || !m->wq || !m->wk || !m->wv || !m->wo || !m->lm || !m->kcache ||
        !m->vcache) {
        refcpu_falcon_free(m);
        return NULL;
    }
    return m;
}

void refcpu_falcon_free(refcpu_falcon *m) {
    if (!m) return;
    free(m->ffn_path);
    free(m->ffn_up_off);
    free(m->ffn_down_off);
    free(m->embed);
    free(m->wq);
    free(m->wk);
    free(m->wv);
    free(m->wo);
    free(m->lm);
    free(m->kcache);
    free(m->vcache);
    free(m);
}

void refcpu_falcon_commit(refcpu_falcon *m) { m->seq_len++; }

int refcpu_falcon_ffn_file(refcpu_falcon *m, const char *path, const int64_t *up_off,
                           const int64_t *down_off, int nthreads) {
    free(m->ffn_path);
    free(m->ffn_up_off);
    free(m->ffn_down_off);
    m->ffn_path = NULL;
    m->ffn_up_off = m->ffn_down_off = NULL;
    if (!path) return 0;
    const size_t L = (size_t)m->p.n_layers;
    m->ffn_path = strdup(path);
    m->ffn_up_off = (int64_t *)malloc(sizeof(int64_t) * L);
    m->ffn_down_off = (int64_t *)malloc(sizeof(int64_t) * L);
    if (!m->ffn_path || !m->ffn_up_off || !m->ffn_down_off) {
        refcpu_falcon_ffn_file(m, NULL, NULL, NULL, 0);
        return -1;
    }
    memcpy(m->ffn_up_off, up_off, sizeof(int64_t) * L);
    memcpy(m->ffn_down_off, down_off, sizeof(int64_t) * L);
    m->ffn_threads = nthreads;
    return 0;
}

/* forward.go:263-301 for query heads [h0, h1) of one layer; each head has its
 * own score row, so heads split over threads change no result */
typedef struct {
    const float *q, *kc, *vc;
    float *att, *scores;
    int n_heads, n_kv, hd, kvd, seq;
    float scale;
} attn_ctx;

static void attn_heads(void *arg, int h0, int h1) {
    const attn_ctx *c = (const attn_ctx *)arg;
    for (int hh = h0; hh < h1; hh++) {
        const float *qh = c->q + (size_t)hh * c->hd;
        const int kvh = hh * c->n_kv / c->n_heads;
        float *scores = c->scores + (size_t)hh * c->seq;
        for (int t = 0; t < c->seq; t++) {
            const float *kh = c->kc + (size_t)t * c->kvd + (size_t)kvh * c->hd;
            float dot = 0.0f;
            for (int d = 0; d < c->hd; d++) dot += qh[d] * kh[d];
            scores[t] = dot * c->scale;
        }
        refcpu_softmax_inplace(scores, c->seq);
        float *oh = c->att + (size_t)hh * c->hd;
        for (int t = 0; t < c->seq; t++) {
            const float *vh = c->vc + (size_t)t * c->kvd + (size_t)kvh * c->hd;
            for (int d = 0; d < c->hd; d++) oh[d] += scores[t] * vh[d];
        }
    }
}

/* inference/forward.go:483-497 */
static void rope_inplace(float *vec, int n_heads, int head_dim, int pos, float base) {
    const int half = head_dim / 2;
    for (int hh = 0; hh < n_heads; hh++) {
        float *head = vec + (size_t)hh * head_dim;
        for (int i = 0; i < half; i++) {
            const double freq = (double)pos / pow((double)base, (double)(2 * i) / (double)head_dim);
            const float c = (float)cos(freq), s = (float)sin(freq);
            const float x0 = head[i], x1 = head[i + half];
            head[i] = x0 * c - x1 * s;
            head[i + half] = x0 * s + x1 * c;
        }
    }
}

int refcpu_falcon_forward(refcpu_falcon *m, int32_t token, int pos, float *logits,
                          int32_t *n_active_out) {
    return refcpu_falcon_forward_ex(m, token, pos, logits, n_active_out, NULL);
}

int refcpu_falcon_forward_ex(refcpu_falcon *m, int32_t token, int pos, float *logits,
                             int32_t *n_active_out, float *pred_logits_out) {
    const refcpu_falcon_params *p = &m->p;
    const int h = p->hidden, hd = p->head_dim, qd = p->n_heads * hd, kvd = p->n_kv * hd;
    if (token < 0 || token >= p->vocab || m->seq_len >= p->max_seq) return -1;
    const int64_t rb_h = refcpu_byte_size(p->t, h);
    float *x = (float *)malloc(sizeof(float) * (size_t)h);
    float *normed = (float *)malloc(sizeof(float) * (size_t)h);
    float *q = (float *)malloc(sizeof(float) * (size_t)qd);
    float *k = (float *)malloc(sizeof(float) * (size_t)kvd);
    float *v = (float *)malloc(sizeof(float) * (size_t)kvd);
    float *att = (float *)malloc(sizeof(float) * (size_t)qd);
    float *attn_out = (float *)malloc(sizeof(float) * (size_t)h);
    float *ffn_out = (float *)malloc(sizeof(float) * (size_t)h);
    float *scores = (float *)malloc(sizeof(float) * (size_t)p->n_heads * (m->seq_len + 1));
    int32_t *active = (int32_t *)malloc(sizeof(int32_t) * (size_t)p->ff);
    memcpy(x, m->embed + (size_t)token * h, sizeof(float) * (size_t)h); /* forward.go:449-454 */
    const int seq = m->seq_len + 1;                                     /* forward.go:249 */
    const float scale = (float)(1.0 / sqrt((double)hd));                /* forward.go:255 */
    for (int l = 0; l < p->n_layers; l++) {
        /* ffn_flash.go:142-146: the one LayerNorm of Falcon's parallel block */
        refcpu_layernorm(x, p->norm_w + (size_t)l * h, p->norm_b + (size_t)l * h, normed, h,
                         p->eps);
        /* forward.go:211-222 */
        refcpu_matmulvec(m->wq + (size_t)l * qd * h, qd, h, normed, q);
        refcpu_matmulvec(m->wk + (size_t)l * kvd * h, kvd, h, normed, k);
        refcpu_matmulvec(m->wv + (size_t)l * kvd * h, kvd, h, normed, v);
        if (p->rope_base > 0) { /* forward.go:249-252: no RoPE without a positive base */
            rope_inplace(q, p->n_heads, hd, pos, p->rope_base);
            rope_inplace(k, p->n_kv, hd, pos, p->rope_base);
        }
        float *kc = m->kcache + (size_t)l * p->max_seq * kvd;
        float *vc = m->vcache + (size_t)l * p->max_seq * kvd;
        memcpy(kc + (size_t)m->seq_len * kvd, k, sizeof(float) * (size_t)kvd); /* :245-246 */
        memcpy(vc + (size_t)m->seq_len * kvd, v, sizeof(float) * (size_t)kvd);
        memset(att, 0, sizeof(float) * (size_t)qd);
        attn_ctx ac = {q, kc, vc, att, scores, p->n_heads, p->n_kv, hd, kvd, seq, scale};
        par_for(p->n_heads, 1, attn_heads, &ac); /* forward.go:263-301 */
        refcpu_matmulvec(m->wo + (size_t)l * h * qd, h, qd, att, attn_out); /* :305 */
        /* ffnFlash path 2: predictor on the attention output (ffn_flash.go:157,
         * 225-231), sparse FFN on the normed input */
        const int n_act = refcpu_predict(p->pwup + (size_t)l * p->rank * h,
                                         p->pwout + (size_t)l * p->ff * p->rank, NULL, h, p->rank,
                                         p->ff, attn_out, p->thr[l], active,
                                         pred_logits_out ? pred_logits_out + (size_t)l * p->ff
                                                         : NULL);
        if (n_active_out) n_active_out[l] = n_act;
        int frc;
        if (m->ffn_path) /* the rows from the file by the row-read pool */
            frc = refcpu_ffn_sparse_load_file(m->ffn_path, m->ffn_up_off[l], m->ffn_down_off[l],
                                              p->t, h, p->ff, normed, active, n_act, p->act,
                                              m->ffn_threads, ffn_out);
        else
            frc = refcpu_ffn_sparse_load(p->up + (size_t)l * p->ff * rb_h,
                                         p->down_t + (size_t)l * p->ff * rb_h, p->t, h, p->ff,
                                         normed, active, n_act, p->act, ffn_out);
        if (frc) { /* a row the file could not give (ffn_flash.go:263-270 returns the error) */
            free(x);
            free(normed);
            free(q);
            free(k);
            free(v);
            free(att);
            free(attn_out);
            free(ffn_out);
            free(scores);
            free(active);
            return -2;
        }
        for (int i = 0; i < h; i++) x[i] += attn_out[i]; /* ffn_flash.go:161-166 */
        for (int i = 0; i < h; i++) x[i] += ffn_out[i];
    }
    refcpu_layernorm(x, p->out_w, p->out_b, normed, h, p->eps); /* ffn_flash.go:126 */
    refcpu_matmulvec(m->lm, p->vocab, h, normed, logits);       /* ffn_flash.go:130 */
    free(x);
    free(normed);
    free(q);
    free(k);
    free(v);
    free(att);
    free(attn_out);
    free(ffn_out);
    free(scores);
    free(active);
    return 0;
}

int refcpu_argmax(const float *v, int n) { /* cmd/generate.go:197-205 */
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}
