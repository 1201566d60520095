/*
 * g4_oracle.c -- CPU restatement of gemma4-rs's attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP backend, never part of it.
 * Citations are file:line in the gemma4-rs repository.  Build flags matter:
 * -ffp-contract=off keeps every a*b+c as two rounded operations, as rustc
 * emits them; the libm calls (expf, sinf, cosf, powf, sqrtf) are the
 * platform's, which is what Rust's f32 methods call on Linux.
 */
#define _GNU_SOURCE
#include "g4_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

static _Thread_local char last_error[256];

static int fail(int code, const char *msg) {
    snprintf(last_error, sizeof last_error, "%s", msg);
    return code;
}

const char *or_last_error(void) { return last_error; }

int or_fail(int code, const char *msg) { return fail(code, msg); }

/* Rust's `Iterator::sum` for floats folds from -0.0 (neutral element of +). */
#define SUM_START (-0.0f)

/* ops.rs:65-76 -- 16 lane accumulators over 16-wide chunks, lanes summed in
 * order, then the remainder summed sequentially and added last. */
float or_dot_f32(const float *a, const float *b, size_t n) {
    enum { LANES = 16 };
    float lanes[LANES] = {0};
    size_t full = n / LANES * LANES;
    float tail = SUM_START;
    for (size_t i = full; i < n; ++i) tail += a[i] * b[i];
    for (size_t c = 0; c < full; c += LANES)
        for (size_t l = 0; l < LANES; ++l) lanes[l] += a[c + l] * b[c + l];
    float s = SUM_START;
    for (size_t l = 0; l < LANES; ++l) s += lanes[l];
    return s + tail;
}

/* Rust's f32::total_cmp order: -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN. */
static int32_t total_key(float x) {
    int32_t bits;
    memcpy(&bits, &x, 4);
    return bits ^ (int32_t)(((uint32_t)(bits >> 31)) >> 1);
}

/* ops.rs:105-127 -- max by total_cmp (the last maximal element, as
 * Iterator::max_by returns), exp(x - max), sequential sum, error if the sum
 * is not finite or zero, then divide. */
int or_softmax_f32(const float *x, size_t n, float *out) {
    if (n == 0) return fail(OR_ERR_COMPUTE, "softmax requires a non-empty buffer");
    float max = x[0];
    for (size_t i = 1; i < n; ++i)
        if (total_key(x[i]) >= total_key(max)) max = x[i];
#ifdef G4_PLANT_SOFTMAX_NO_MAX /* planted mistake, test_oracle.py only */
    max = 0.0f;
#endif
    for (size_t i = 0; i < n; ++i) out[i] = expf(x[i] - max);
    float sum = SUM_START;
    for (size_t i = 0; i < n; ++i) sum += out[i];
    if (!isfinite(sum) || sum == 0.0f) return fail(OR_ERR_COMPUTE, "softmax input is not finite");
    for (size_t i = 0; i < n; ++i) out[i] = out[i] / sum;
    return OR_OK;
}

/* ops.rs:45-56 -- mean of squares accumulated in f64 (each square rounded
 * in f32 first), mean cast to f32, scale = 1 / sqrt(mean + eps), x*scale*w. */
int or_rms_norm(const float *x, size_t n, const float *weight, size_t weight_len, float eps,
                float *out) {
    if (n == 0 || eps < 0.0f || (weight && weight_len != n))
        return fail(OR_ERR_COMPUTE, "invalid RMS norm inputs");
    double sum = -0.0;
    for (size_t i = 0; i < n; ++i) {
        float sq = x[i] * x[i];
        sum += (double)sq;
    }
    float mean = (float)(sum / (double)n);
    float scale = 1.0f / sqrtf(mean + eps);
    if (weight)
#ifdef G4_PLANT_RMS_WEIGHT_SHIFT /* planted mistake: Gemma's (1 + w) convention */
        for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * (1.0f + weight[i]);
#else
        for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * weight[i];
#endif
    else
        for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale;
    return OR_OK;
}

/* ops.rs:134-162 -- NEOX pairs (x[i], x[i+half]); theta starts at the
 * position and is multiplied by base^(-2/n_rot) after every pair; the angle
 * is theta / freq_factors[i]. */
int or_rope_neox(float *x, size_t len, size_t position, float base, size_t n_rot,
                 const float *freq_factors, size_t n_factors) {
    size_t half = n_rot / 2;
    if (n_rot == 0 || n_rot % 2 != 0 || n_rot > len || base <= 0.0f ||
        (freq_factors && n_factors < half))
        return fail(OR_ERR_COMPUTE, "invalid RoPE inputs");
    float theta_scale = powf(base, -2.0f / (float)n_rot);
    float theta = (float)position;
    for (size_t i = 0; i < half; ++i) {
        float factor = freq_factors ? freq_factors[i] : 1.0f;
        float angle = theta / factor;
        float s = sinf(angle), c = cosf(angle);
        float a = x[i], b = x[i + half];
#ifdef G4_PLANT_ROPE_SIGN /* planted mistake */
        x[i] = a * c + b * s;
#else
        x[i] = a * c - b * s;
#endif
        x[i + half] = a * s + b * c;
        theta *= theta_scale;
    }
    return OR_OK;
}

/* model.rs:326-343 */
int or_attend_head(const float *q, const float *keys, const float *values, size_t T,
                   size_t kv_width, size_t head_dim, size_t n_heads, size_t n_kv_heads,
                   float scale, size_t head, float *out) {
    const float *qh = q + head * head_dim;
#ifdef G4_PLANT_GQA_MAP /* planted mistake: interleaved head map */
    size_t kv_head = head % n_kv_heads;
#else
    size_t kv_head = head * n_kv_heads / n_heads;
#endif
    size_t kv = kv_head * head_dim;
    float *scores = (float *)malloc((T ? T : 1) * sizeof(float));
    float *probs = (float *)malloc((T ? T : 1) * sizeof(float));
    for (size_t t = 0; t < T; ++t) scores[t] = or_dot_f32(qh, keys + t * kv_width + kv, head_dim) * scale;
    int rc = or_softmax_f32(scores, T, probs);
    if (rc == OR_OK) {
        for (size_t i = 0; i < head_dim; ++i) out[i] = 0.0f;
        for (size_t t = 0; t < T; ++t) {
#ifdef G4_PLANT_PV_STRIDE /* planted mistake: rows read at head_dim stride */
            const float *v = values + t * head_dim + kv;
#else
            const float *v = values + t * kv_width + kv;
#endif
            float p = probs[t];
            for (size_t i = 0; i < head_dim; ++i) out[i] += p * v[i];
        }
    }
    free(scores);
    free(probs);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Persistent worker pool with the split map_items uses (pool.rs:145-197):   */
/* chunk_len = ceil(count / (threads*4)), chunks claimed through an atomic   */
/* counter by the caller and the workers; below `parallel_min_work` the     */
/* caller runs everything itself.  Workers spin ~200 us before sleeping.     */
/* ------------------------------------------------------------------------ */
typedef void (*or_chunk_fn)(void *ctx, size_t begin, size_t end);

typedef struct {
    size_t count, chunk_len, chunks;
    atomic_size_t next, remaining;
    or_chunk_fn fn;
    void *ctx;
} or_task;

static struct {
    pthread_once_t once;
    size_t threads;
    atomic_ulong gen; /* odd while the caller rewrites `task` */
    atomic_int active;
    pthread_mutex_t m, call_lock;
    pthread_cond_t cv;
    or_task task;
} pool = {PTHREAD_ONCE_INIT, 0, 0, 0, PTHREAD_MUTEX_INITIALIZER, PTHREAD_MUTEX_INITIALIZER,
          PTHREAD_COND_INITIALIZER, {0}};

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void task_work(or_task *t) {
    for (;;) {
        size_t chunk = atomic_fetch_add(&t->next, 1);
        if (chunk >= t->chunks) return;
        size_t begin = chunk * t->chunk_len;
        size_t end = begin + t->chunk_len < t->count ? begin + t->chunk_len : t->count;
        t->fn(t->ctx, begin, end);
        atomic_fetch_sub(&t->remaining, 1);
    }
}

static void *worker_main(void *arg) {
    (void)arg;
    unsigned long seen = atomic_load(&pool.gen);
    for (;;) {
        unsigned long g;
        double t0 = now_s();
        while (((g = atomic_load(&pool.gen)) == seen || (g & 1)) && now_s() - t0 < 200e-6) sched_yield();
        if (g == seen || (g & 1)) {
            pthread_mutex_lock(&pool.m);
            while ((g = atomic_load(&pool.gen)) == seen || (g & 1)) pthread_cond_wait(&pool.cv, &pool.m);
            pthread_mutex_unlock(&pool.m);
        }
        atomic_fetch_add(&pool.active, 1);
        if (atomic_load(&pool.gen) != g) { /* the caller started rewriting the task */
            atomic_fetch_sub(&pool.active, 1);
            continue;
        }
        seen = g;
        task_work(&pool.task);
        atomic_fetch_sub(&pool.active, 1);
    }
    return NULL;
}

static void pool_init(void) {
    size_t threads = 0;
    const char *env = getenv("LLM_THREADS");
    if (env) {
        long v = strtol(env, NULL, 10);
        if (v > 0) threads = (size_t)v;
    }
    if (!threads) {
        long n = sysconf(_SC_NPROCESSORS_ONLN);
        threads = n > 0 ? (size_t)n : 1;
    }
    pool.threads = threads;
    for (size_t i = 1; i < threads; ++i) {
        pthread_t th;
        pthread_create(&th, NULL, worker_main, NULL);
        pthread_detach(th);
    }
}

size_t or_pool_threads(void) {
    pthread_once(&pool.once, pool_init);
    return pool.threads;
}

static void run_chunks(size_t count, size_t work_per_item, size_t parallel_min_work, or_chunk_fn fn,
                       void *ctx) {
    size_t threads = or_pool_threads();
    if (threads <= 1 || count * work_per_item < parallel_min_work) {
        fn(ctx, 0, count);
        return;
    }
    pthread_mutex_lock(&pool.call_lock);
    atomic_fetch_add(&pool.gen, 1); /* odd: workers may not enter */
    while (atomic_load(&pool.active) != 0) sched_yield();
    size_t chunk_len = (count + threads * 4 - 1) / (threads * 4);
    if (chunk_len == 0) chunk_len = 1;
    pool.task.count = count;
    pool.task.chunk_len = chunk_len;
    pool.task.chunks = (count + chunk_len - 1) / chunk_len;
    atomic_store(&pool.task.next, 0);
    atomic_store(&pool.task.remaining, pool.task.chunks);
    pool.task.fn = fn;
    pool.task.ctx = ctx;
    pthread_mutex_lock(&pool.m);
    atomic_fetch_add(&pool.gen, 1); /* even: published */
    pthread_cond_broadcast(&pool.cv);
    pthread_mutex_unlock(&pool.m);
    task_work(&pool.task);
    while (atomic_load(&pool.task.remaining) != 0) sched_yield();
    pthread_mutex_unlock(&pool.call_lock);
}

/* model.rs:308 */
#define ATTENTION_PARALLEL_MIN_WORK ((size_t)1 << 18)

typedef struct {
    const float *q, *keys, *values;
    size_t T, kv_width, head_dim, n_heads, n_kv_heads;
    float scale;
    float *out;
    atomic_int failed;
} attend_ctx;

static void attend_chunk(void *vctx, size_t begin, size_t end) {
    attend_ctx *c = (attend_ctx *)vctx;
    for (size_t h = begin; h < end; ++h)
        if (or_attend_head(c->q, c->keys, c->values, c->T, c->kv_width, c->head_dim, c->n_heads,
                           c->n_kv_heads, c->scale, h, c->out + h * c->head_dim) != OR_OK)
            atomic_store(&c->failed, 1);
}

static int attend_image(const float *q, size_t q_len, const float *keys, const float *values,
                        size_t T, size_t n_heads, size_t n_kv_heads, float scale, int pooled,
                        float *out) {
    size_t head_dim = q_len / n_heads;
    attend_ctx c = {q, keys, values, T, n_kv_heads * head_dim, head_dim, n_heads, n_kv_heads,
                    scale, out, 0};
    size_t work_per_head = 2 * T * head_dim;
    if (pooled)
        run_chunks(n_heads, work_per_head, ATTENTION_PARALLEL_MIN_WORK, attend_chunk, &c);
    else
        attend_chunk(&c, 0, n_heads);
    /* model.rs:362-364: a failed head returns no values, and a q longer than
     * n_heads * head_dim leaves the concatenation shorter than q; either way
     * attended.len() != q.len(). */
    if (atomic_load(&c.failed) || n_heads * head_dim != q_len)
        return fail(OR_ERR_COMPUTE, "softmax input is not finite");
    return OR_OK;
}

/* model.rs:348-366 without the pool (heads run in order on this thread). */
int or_attend(const float *q, size_t q_len, const float *keys, const float *values, size_t T,
              size_t n_heads, size_t n_kv_heads, float scale, float *out) {
    return attend_image(q, q_len, keys, values, T, n_heads, n_kv_heads, scale, 0, out);
}

/* model.rs:348-366 with the `concat` copy and, for threads != 1, the pool. */
int or_attend_rows(const float *q, size_t q_len, const float *const *key_rows,
                   const float *const *value_rows, size_t T, size_t n_heads, size_t n_kv_heads,
                   float scale, size_t threads, float *out) {
    size_t head_dim = q_len / n_heads;
    size_t width = n_kv_heads * head_dim;
    float *qc = (float *)malloc(q_len * sizeof(float));
    float *kc = (float *)malloc((T ? T : 1) * width * sizeof(float));
    float *vc = (float *)malloc((T ? T : 1) * width * sizeof(float));
    memcpy(qc, q, q_len * sizeof(float));
    for (size_t t = 0; t < T; ++t) {
        memcpy(kc + t * width, key_rows[t], width * sizeof(float));
        memcpy(vc + t * width, value_rows[t], width * sizeof(float));
    }
    int rc = attend_image(qc, q_len, kc, vc, T, n_heads, n_kv_heads, scale, threads != 1, out);
    free(qc);
    free(kc);
    free(vc);
    return rc;
}

typedef struct {
    const float *q, *keys, *values;
    size_t q_len, N, pos0, window, n_heads, n_kv_heads, threads, width;
    float scale;
    int *status;
    float *out;
    atomic_int failed;
    size_t index; /* this worker's first query (first query group when blocked) */
    int blocked;  /* or_attend_prefill_blocked: groups of PF_GROUP queries */
    const size_t *positions; /* blocked: query i's position, or NULL for pos0 + i */
} prefill_ctx;

/* Query groups of the blocked checker: PF_GROUP consecutive queries walk
 * their keys together, PF_CHUNK rows at a time, so that a key or value row
 * is fetched from memory once per group rather than once per query and
 * head. */
enum { PF_GROUP = 16, PF_CHUNK = 64 };

/* One group of queries [i0, i1) with or_attend's arithmetic: per query and
 * head the scores are or_dot_f32 * scale in key order, the weights are
 * or_softmax_f32 over the query's whole range, and out[d] += p_t * v_t[d]
 * runs over the keys in order; only the loop nest differs from attend_image
 * (keys outermost, then queries, then heads), which changes no operation or
 * its order.  A query with a failing head gets that head's output untouched
 * and the error, as attend_image leaves it. */
static void prefill_group(prefill_ctx *w, size_t i0, size_t i1) {
    const size_t nh = w->n_heads, hd = w->q_len / nh, G = i1 - i0;
    size_t b[PF_GROUP], e[PF_GROUP], off[PF_GROUP];
    size_t lo = (size_t)-1, hi = 0, total = 0;
    for (size_t j = 0; j < G; ++j) {
        const size_t i = i0 + j, pos = w->positions ? w->positions[i] : w->pos0 + i;
        if (w->window)
            or_windowed_len(pos + 1, w->window, &b[j], &e[j]);
        else
            b[j] = 0, e[j] = pos + 1;
        off[j] = total;
        total += (e[j] - b[j]) * nh;
        if (b[j] < lo) lo = b[j];
        if (e[j] > hi) hi = e[j];
    }
    float *s = (float *)malloc((total ? total : 1) * sizeof(float));
    int ok[PF_GROUP * 64]; /* per (query, head); run_prefill admits at most 64 heads */
    for (size_t t0 = lo; t0 < hi; t0 += PF_CHUNK) {
        const size_t t1 = t0 + PF_CHUNK < hi ? t0 + PF_CHUNK : hi;
        for (size_t j = 0; j < G; ++j) {
            const size_t tb = t0 > b[j] ? t0 : b[j], te = t1 < e[j] ? t1 : e[j], T = e[j] - b[j];
            for (size_t h = 0; h < nh && tb < te; ++h) {
                const float *qh = w->q + (i0 + j) * w->q_len + h * hd;
                const size_t kv = (h * w->n_kv_heads / nh) * hd;
                float *sc = s + off[j] + h * T;
                for (size_t t = tb; t < te; ++t)
                    sc[t - b[j]] = or_dot_f32(qh, w->keys + t * w->width + kv, hd) * w->scale;
            }
        }
    }
    for (size_t j = 0; j < G; ++j) {
        const size_t T = e[j] - b[j];
        for (size_t h = 0; h < nh; ++h) {
            float *sc = s + off[j] + h * T;
            ok[j * 64 + h] = or_softmax_f32(sc, T, sc) == OR_OK; /* in place: element i is read before written */
            if (ok[j * 64 + h]) memset(w->out + (i0 + j) * w->q_len + h * hd, 0, hd * sizeof(float));
        }
    }
    for (size_t t0 = lo; t0 < hi; t0 += PF_CHUNK) {
        const size_t t1 = t0 + PF_CHUNK < hi ? t0 + PF_CHUNK : hi;
        for (size_t j = 0; j < G; ++j) {
            const size_t tb = t0 > b[j] ? t0 : b[j], te = t1 < e[j] ? t1 : e[j], T = e[j] - b[j];
            for (size_t h = 0; h < nh && tb < te; ++h) {
                if (!ok[j * 64 + h]) continue;
                const size_t kv = (h * w->n_kv_heads / nh) * hd;
                const float *pr = s + off[j] + h * T;
                float *o = w->out + (i0 + j) * w->q_len + h * hd;
                for (size_t t = tb; t < te; ++t) {
                    const float p = pr[t - b[j]];
                    const float *v = w->values + t * w->width + kv;
                    for (size_t d = 0; d < hd; ++d) o[d] += p * v[d];
                }
            }
        }
    }
    for (size_t j = 0; j < G; ++j) {
        int failed = nh * hd != w->q_len;
        for (size_t h = 0; h < nh; ++h) failed |= !ok[j * 64 + h];
        const int rc = failed ? fail(OR_ERR_COMPUTE, "softmax input is not finite") : OR_OK;
        if (w->status) w->status[i0 + j] = rc;
        if (failed) atomic_store(&w->failed, 1);
    }
    free(s);
}

static void *prefill_worker(void *arg) {
    prefill_ctx *w = (prefill_ctx *)arg;
    if (w->blocked) {
        for (size_t i0 = w->index * PF_GROUP; i0 < w->N; i0 += w->threads * PF_GROUP)
            prefill_group(w, i0, i0 + PF_GROUP < w->N ? i0 + PF_GROUP : w->N);
        return NULL;
    }
    for (size_t i = w->index; i < w->N; i += w->threads) {
        size_t begin, end;
        /* generate.rs:37-41: token i runs as a decode at position pos0 + i. */
        if (w->window)
            or_windowed_len(w->pos0 + i + 1, w->window, &begin, &end);
        else
            begin = 0, end = w->pos0 + i + 1;
        int rc = attend_image(w->q + i * w->q_len, w->q_len, w->keys + begin * w->width,
                              w->values + begin * w->width, end - begin, w->n_heads, w->n_kv_heads,
                              w->scale, 0, w->out + i * w->q_len);
        if (w->status) w->status[i] = rc;
        if (rc != OR_OK) atomic_store(&w->failed, 1);
    }
    return NULL;
}

static int run_prefill(const float *q, size_t q_len, size_t N, const float *keys, const float *values,
                       size_t pos0, size_t window, size_t n_heads, size_t n_kv_heads, float scale,
                       size_t threads, int *status, float *out, int blocked, const size_t *positions) {
    if (n_heads == 0 || threads == 0) return fail(OR_ERR_COMPUTE, "attend_prefill: zero heads or threads");
    if (blocked && n_heads > 64) return fail(OR_ERR_COMPUTE, "attend_prefill_blocked: more than 64 heads");
    if (threads > 256) threads = 256;
    prefill_ctx base = {q, keys, values, q_len, N, pos0, window, n_heads, n_kv_heads, threads,
                        n_kv_heads * (q_len / n_heads), scale, status, out, 0, 0, blocked, positions};
    prefill_ctx w[256];
    pthread_t th[256];
    for (size_t t = 0; t < threads; ++t) {
        w[t] = base;
        w[t].index = t;
    }
    size_t started = 1;
    for (size_t t = 1; t < threads; ++t, ++started)
        if (pthread_create(&th[t], NULL, prefill_worker, &w[t]) != 0) break;
    /* Queries of threads that could not start run here. */
    for (size_t t = started; t < threads; ++t) prefill_worker(&w[t]);
    prefill_worker(&w[0]);
    int failed = atomic_load(&w[0].failed);
    for (size_t t = 1; t < started; ++t) {
        pthread_join(th[t], NULL);
        failed |= atomic_load(&w[t].failed);
    }
    for (size_t t = started; t < threads; ++t) failed |= atomic_load(&w[t].failed);
    return failed ? fail(OR_ERR_COMPUTE, "softmax input is not finite") : OR_OK;
}

int or_attend_prefill(const float *q, size_t q_len, size_t N, const float *keys, const float *values,
                      size_t pos0, size_t window, size_t n_heads, size_t n_kv_heads, float scale,
                      size_t threads, int *status, float *out) {
    return run_prefill(q, q_len, N, keys, values, pos0, window, n_heads, n_kv_heads, scale, threads, status,
                       out, 0, NULL);
}

int or_attend_prefill_blocked(const float *q, size_t q_len, size_t N, const size_t *positions,
                              const float *keys, const float *values, size_t pos0, size_t window,
                              size_t n_heads, size_t n_kv_heads, float scale, size_t threads, int *status,
                              float *out) {
    return run_prefill(q, q_len, N, keys, values, pos0, window, n_heads, n_kv_heads, scale, threads, status,
                       out, 1, positions);
}

/* f64 twin: same structure, double throughout (plain sequential sums). */
int or_attend_f64(const float *q, size_t q_len, const float *keys, const float *values, size_t T,
                  size_t n_heads, size_t n_kv_heads, double scale, double *out) {
    size_t head_dim = q_len / n_heads, width = n_kv_heads * head_dim;
    if (T == 0) return fail(OR_ERR_COMPUTE, "softmax input is not finite");
    double *s = (double *)malloc(T * sizeof(double));
    int rc = OR_OK;
    for (size_t h = 0; h < n_heads && rc == OR_OK; ++h) {
        const float *qh = q + h * head_dim;
        size_t kv = (h * n_kv_heads / n_heads) * head_dim;
        double mx = -INFINITY;
        int has_nan = 0;
        for (size_t t = 0; t < T; ++t) {
            double acc = 0.0;
            for (size_t i = 0; i < head_dim; ++i) acc += (double)qh[i] * (double)keys[t * width + kv + i];
            s[t] = acc * scale;
            if (isnan(s[t])) has_nan = 1;
            else if (s[t] > mx) mx = s[t];
        }
        if (has_nan) mx = NAN;
        double sum = 0.0;
        for (size_t t = 0; t < T; ++t) {
            s[t] = exp(s[t] - mx);
            sum += s[t];
        }
        if (!isfinite(sum) || sum == 0.0) {
            rc = fail(OR_ERR_COMPUTE, "softmax input is not finite");
            break;
        }
        double *o = out + h * head_dim;
        for (size_t i = 0; i < head_dim; ++i) o[i] = 0.0;
        for (size_t t = 0; t < T; ++t) {
            double p = s[t] / sum;
            for (size_t i = 0; i < head_dim; ++i) o[i] += p * (double)values[t * width + kv + i];
        }
    }
    free(s);
    return rc;
}

/* model.rs:283-290 */
int or_norm_heads(float *x, size_t len, size_t head_dim, const float *weight, float eps) {
    float *tmp = (float *)malloc(head_dim * sizeof(float));
    for (size_t h = 0; h + head_dim <= len; h += head_dim) {
        int rc = or_rms_norm(x + h, head_dim, weight, weight ? head_dim : 0, eps, tmp);
        if (rc != OR_OK) {
            free(tmp);
            return rc;
        }
        memcpy(x + h, tmp, head_dim * sizeof(float));
    }
    free(tmp);
    return OR_OK;
}

/* model.rs:295-304 (n_rot = head_dim: whole heads rotate). */
int or_rope_heads(float *x, size_t len, size_t head_dim, size_t position, float base,
                  const float *freq_factors, size_t n_factors) {
    for (size_t h = 0; h + head_dim <= len; h += head_dim) {
        int rc = or_rope_neox(x + h, head_dim, position, base, head_dim, freq_factors, n_factors);
        if (rc != OR_OK) return rc;
    }
    return OR_OK;
}

/* idea/mod.rs:148-156 */
int or_layer_attention_kind(size_t n_layers, size_t layer) {
    return (layer + 1 == n_layers || layer % 5 == 4) ? 1 : 0;
}

/* idea/mod.rs:140-145 */
size_t or_head_dim(size_t n_layers, size_t layer, size_t head_dim_local, size_t head_dim_global) {
    return or_layer_attention_kind(n_layers, layer) ? head_dim_global : head_dim_local;
}

/* idea/mod.rs:162-165 -- `(head_dim as f32 * p / 2.0) as usize` pairs turn. */
void or_proportional_rope_freq_factors(size_t head_dim, float p, float *out) {
    float r = (float)head_dim * p / 2.0f;
    size_t rotated = r > 0.0f ? (size_t)r : 0;
    for (size_t pair = 0; pair < head_dim / 2; ++pair) out[pair] = pair < rotated ? 1.0f : 1e30f;
}

/* eng/mod.rs:10-12 */
void or_windowed_len(size_t seq_len, size_t window, size_t *begin, size_t *end) {
#ifdef G4_PLANT_WINDOW /* planted mistake: window excludes one row too many */
    *begin = seq_len > window ? seq_len - window + 1 : 0;
#else
    *begin = seq_len > window ? seq_len - window : 0;
#endif
    *end = seq_len;
}

/* eng/mod.rs:71-90 */
int or_kv_source_layer(size_t n_layers, size_t shared_kv_layers, size_t layer, size_t *source) {
    char msg[160];
    if (layer >= n_layers) {
        snprintf(msg, sizeof msg, "layer %zu must be within n_layers %zu", layer, n_layers);
        return fail(OR_ERR_KV_LAYER_OUT_OF_RANGE, msg);
    }
    if (shared_kv_layers >= n_layers) {
        snprintf(msg, sizeof msg, "%zu KV-shared layers leave no layer of %zu to own a cache",
                 shared_kv_layers, n_layers);
        return fail(OR_ERR_KV_TOO_MANY_SHARED, msg);
    }
    size_t first_shared = n_layers - shared_kv_layers;
    if (layer < first_shared) {
        *source = layer;
        return OR_OK;
    }
    int kind = or_layer_attention_kind(n_layers, layer);
#ifdef G4_PLANT_KV_SOURCE /* planted mistake: first instead of last earlier layer */
    for (size_t e = 0; e < first_shared; ++e) {
#else
    for (size_t e = first_shared; e-- > 0;) {
#endif
        if (or_layer_attention_kind(n_layers, e) == kind) {
            *source = e;
            return OR_OK;
        }
    }
    snprintf(msg, sizeof msg, "KV-shared layer %zu has no earlier layer of the same attention kind",
             layer);
    return fail(OR_ERR_KV_NO_EARLIER_SAME_KIND, msg);
}

/* context_memory.rs:21-86: one growable row store per layer. */
typedef struct {
    size_t width, rows, cap;
    float *k, *v;
} or_kv_layer;

struct or_kv_cache {
    size_t n_layers;
    or_kv_layer *layers;
};

or_kv_cache *or_kv_new(void) { return (or_kv_cache *)calloc(1, sizeof(or_kv_cache)); }

void or_kv_clear(or_kv_cache *c) {
    for (size_t i = 0; i < c->n_layers; ++i) {
        free(c->layers[i].k);
        free(c->layers[i].v);
    }
    free(c->layers);
    c->layers = NULL;
    c->n_layers = 0;
}

void or_kv_free(or_kv_cache *c) {
    if (!c) return;
    or_kv_clear(c);
    free(c);
}

/* context_memory.rs:44-51 -- grows the layer list up to `layer`, pushes a row. */
int or_kv_append(or_kv_cache *c, size_t layer, const float *k, const float *v, size_t width) {
    if (c->n_layers <= layer) {
        c->layers = (or_kv_layer *)realloc(c->layers, (layer + 1) * sizeof(or_kv_layer));
        memset(c->layers + c->n_layers, 0, (layer + 1 - c->n_layers) * sizeof(or_kv_layer));
        c->n_layers = layer + 1;
    }
    or_kv_layer *L = &c->layers[layer];
    if (L->rows == 0 && L->cap == 0) L->width = width;
    if (width != L->width) return fail(OR_ERR_COMPUTE, "K/V row width differs from the layer's");
    if (L->rows == L->cap) {
        L->cap = L->cap ? 2 * L->cap : 64;
        L->k = (float *)realloc(L->k, L->cap * width * sizeof(float));
        L->v = (float *)realloc(L->v, L->cap * width * sizeof(float));
    }
    memcpy(L->k + L->rows * width, k, width * sizeof(float));
    memcpy(L->v + L->rows * width, v, width * sizeof(float));
    L->rows++;
    return OR_OK;
}

/* context_memory.rs:53-69 */
int or_kv_view(const or_kv_cache *c, size_t layer, size_t len, const float **keys,
               const float **values, size_t *width) {
    char msg[128];
    if (layer >= c->n_layers) {
        if (len == 0) {
            *keys = *values = NULL;
            *width = 0;
            return OR_OK;
        }
        snprintf(msg, sizeof msg, "layer %zu has no cached K/V", layer);
        return fail(OR_ERR_MISSING_LAYER, msg);
    }
    const or_kv_layer *L = &c->layers[layer];
    if (len > L->rows) {
        snprintf(msg, sizeof msg, "context length %zu exceeds configured max %zu", len, L->rows);
        return fail(OR_ERR_CONTEXT_TOO_LONG, msg);
    }
    *keys = L->k;
    *values = L->v;
    *width = L->width;
    return OR_OK;
}

/* model.rs:386-411, attention segment (projections are the caller's). */
int or_layer_attention(or_kv_cache *c, const or_hparams *hp, size_t layer, size_t position,
                       float *q, float *k, float *v, const float *q_norm_w,
                       const float *k_norm_w, const float *rope_freqs, size_t n_freqs,
                       float *out, size_t *source_layer, size_t *kv_begin, size_t *kv_end) {
    int global = or_layer_attention_kind(hp->n_layers, layer);
    size_t head_dim = global ? hp->head_dim_global : hp->head_dim_local;
    float base = global ? hp->global_rope_base : hp->local_rope_base;
    const float *factors = global ? rope_freqs : NULL;
    size_t q_len = hp->n_heads * head_dim, kv_len = hp->n_kv_heads * head_dim;
    int rc = or_norm_heads(q, q_len, head_dim, q_norm_w, hp->rms_norm_eps);
    if (rc == OR_OK) rc = or_rope_heads(q, q_len, head_dim, position, base, factors, n_freqs);
    size_t source = 0;
    if (rc == OR_OK) rc = or_kv_source_layer(hp->n_layers, hp->shared_kv_layers, layer, &source);
    if (rc != OR_OK) { /* model.rs:398 maps KvShareError to EngError::Compute(e.to_string()) */
        char msg[sizeof last_error];
        memcpy(msg, last_error, sizeof msg);
        return fail(OR_ERR_COMPUTE, msg);
    }
    if (source == layer) {
        rc = or_norm_heads(k, kv_len, head_dim, k_norm_w, hp->rms_norm_eps);
        if (rc == OR_OK) rc = or_norm_heads(v, kv_len, head_dim, NULL, hp->rms_norm_eps);
        if (rc == OR_OK) rc = or_rope_heads(k, kv_len, head_dim, position, base, factors, n_freqs);
        if (rc == OR_OK) rc = or_kv_append(c, layer, k, v, kv_len);
        if (rc != OR_OK) return rc;
    }
    const float *keys, *values;
    size_t width;
    rc = or_kv_view(c, source, position + 1, &keys, &values, &width);
    if (rc != OR_OK) return rc;
    size_t begin = 0, end = position + 1;
    if (!global) or_windowed_len(position + 1, hp->sliding_window, &begin, &end);
    *source_layer = source;
    *kv_begin = begin;
    *kv_end = end;
    return or_attend(q, q_len, keys + begin * width, values + begin * width, end - begin,
                     hp->n_heads, hp->n_kv_heads, 1.0f, out);
}

int or_prepare_rows(float *x, size_t n_rows, size_t row_width, size_t head_dim,
                    const float *weight, float eps, size_t pos0, float base,
                    const float *freq_factors, size_t n_factors) {
    for (size_t r = 0; r < n_rows; ++r) {
        float *row = x + r * row_width;
        int rc = or_norm_heads(row, row_width, head_dim, weight, eps);
        if (rc == OR_OK && base > 0.0f)
            rc = or_rope_heads(row, row_width, head_dim, pos0 + r, base, freq_factors, n_factors);
        if (rc != OR_OK) return rc;
    }
    return OR_OK;
}
