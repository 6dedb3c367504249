/* ora_internal.h -- helpers shared by the oracle's C files (test infrastructure). */
#ifndef ULSPEC_ORA_INTERNAL_H
#define ULSPEC_ORA_INTERNAL_H

#include "oracle.h"

#include <pthread.h>
#include <stdlib.h>

void ora_normals_range(uint64_t seed, uint64_t stream, uint64_t i0, size_t n, double mean, double std, float* out);
void ora_q4k_scale_min(const uint8_t* scales, int j, int* sc, int* m);

typedef void (*ora_range_fn)(void* arg, int64_t lo, int64_t hi);

typedef struct {
    ora_range_fn fn;
    void* arg;
    int64_t lo, hi;
} ora_task;

static void* ora_task_main(void* p)
{
    ora_task* t = (ora_task*)p;
    if (t->lo < t->hi) t->fn(t->arg, t->lo, t->hi);
    return NULL;
}

/* Split [0, n) in nthreads contiguous ranges; the caller's thread runs the first. */
static inline void ora_parallel_for(int nthreads, int64_t n, ora_range_fn fn, void* arg)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t)nthreads > n) nthreads = n > 0 ? (int)n : 1;
    if (nthreads == 1) {
        if (n > 0) fn(arg, 0, n);
        return;
    }
    pthread_t th[256];
    ora_task tasks[256];
    for (int i = 0; i < nthreads; ++i) {
        tasks[i].fn = fn;
        tasks[i].arg = arg;
        tasks[i].lo = n * i / nthreads;
        tasks[i].hi = n * (i + 1) / nthreads;
    }
    for (int i = 1; i < nthreads; ++i) pthread_create(&th[i], NULL, ora_task_main, &tasks[i]);
    ora_task_main(&tasks[0]);
    for (int i = 1; i < nthreads; ++i) pthread_join(th[i], NULL);
}

#endif
