/* CPU baseline harness (benchmark infrastructure, not product code).
 *
 * Times a pyrite_matvec-compatible function -- the reference's own
 * pyrite/kernels/native.c:518-555 built into oracle/_ref, or the oracle's
 * restatement when that build is absent -- over a list of matrix-vector calls,
 * with no Python in the timed region:
 *
 *   one untimed warm-up pass, then `runs` timed runs of `passes` passes each;
 *   run_s[k] receives run k's wall time (CLOCK_MONOTONIC).
 *
 * With nthreads > 1, thread i runs every call on its own contiguous i-th share
 * of each matrix's rows (the reference function is reentrant and rows are
 * independent), so the threads never wait for each other inside a run.
 */
#define _POSIX_C_SOURCE 200809L
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <time.h>

typedef int (*matvec_fn)(int, const uint8_t *, size_t, const double *, double *, size_t, size_t);

typedef struct {
    matvec_fn fn;
    int ncalls;
    const int *types;
    const uint8_t *const *w;
    const size_t *rows, *cols, *row_bytes;
    const double *const *x;
    int tid, nthreads, passes;
    double *out; /* max rows doubles */
    int rc;
} job_t;

static void *worker(void *p) {
    job_t *j = (job_t *)p;
    for (int pass = 0; pass < j->passes && j->rc == 0; ++pass) {
        for (int c = 0; c < j->ncalls; ++c) {
            const size_t rows = j->rows[c], rb = j->row_bytes[c];
            const size_t r0 = rows * (size_t)j->tid / (size_t)j->nthreads;
            const size_t r1 = rows * (size_t)(j->tid + 1) / (size_t)j->nthreads;
            if (r1 <= r0) continue;
            const int rc = j->fn(j->types[c], j->w[c] + r0 * rb, (r1 - r0) * rb, j->x[c], j->out, r1 - r0, j->cols[c]);
            if (rc != 0) {
                j->rc = rc;
                break;
            }
        }
    }
    return NULL;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* One round of `passes` passes on nthreads threads; returns its wall seconds,
 * or a negative value on error (*rc set). */
static double round_s(job_t *jobs, pthread_t *th, int nthreads, int passes, int *rc) {
    for (int i = 0; i < nthreads; ++i) jobs[i].passes = passes;
    const double t0 = now_s();
    if (nthreads == 1) {
        worker(&jobs[0]);
    } else {
        for (int i = 0; i < nthreads; ++i)
            if (pthread_create(&th[i], NULL, worker, &jobs[i]) != 0) {
                for (int k = 0; k < i; ++k) pthread_join(th[k], NULL);
                *rc = -5;
                return -1.0;
            }
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    }
    const double dt = now_s() - t0;
    for (int i = 0; i < nthreads; ++i)
        if (jobs[i].rc != 0) {
            *rc = jobs[i].rc;
            return -1.0;
        }
    return dt;
}

/* Returns 0, the matvec's error code, -5 (thread creation) or -6 (memory). */
int cpu_bench_run(void *fn, int ncalls, const int *types, const uint8_t *const *w, const size_t *rows,
                  const size_t *cols, const size_t *row_bytes, const double *const *x, int nthreads, int runs,
                  int passes, double *run_s) {
    if (!fn || ncalls < 1 || nthreads < 1 || runs < 1 || passes < 1) return -3;
    size_t max_rows = 0;
    for (int c = 0; c < ncalls; ++c)
        if (rows[c] > max_rows) max_rows = rows[c];
    job_t *jobs = calloc((size_t)nthreads, sizeof(job_t));
    pthread_t *th = calloc((size_t)nthreads, sizeof(pthread_t));
    int rc = (jobs && th) ? 0 : -6;
    for (int i = 0; i < nthreads && rc == 0; ++i) {
        jobs[i] = (job_t){(matvec_fn)fn, ncalls, types, w, rows, cols, row_bytes, x, i, nthreads, 1, NULL, 0};
        jobs[i].out = malloc(max_rows * sizeof(double));
        if (!jobs[i].out) rc = -6;
    }
    if (rc == 0) round_s(jobs, th, nthreads, 1, &rc); /* warm-up */
    for (int k = 0; k < runs && rc == 0; ++k) run_s[k] = round_s(jobs, th, nthreads, passes, &rc);
    if (jobs)
        for (int i = 0; i < nthreads; ++i) free(jobs[i].out);
    free(jobs);
    free(th);
    return rc;
}
