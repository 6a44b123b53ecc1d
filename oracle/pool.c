/* pool.c — the CPU baseline's persistent thread pool.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Behaviour of src/threads.c:27-149: workers persist between regions; a
 * region is n tasks claimed one index at a time from a shared counter; the
 * calling thread claims tasks too; the caller returns only when every task
 * has FINISHED (a count of tasks left, decremented after each task returns),
 * never when workers have merely shown up. Default size: all online cores.
 *
 * SPDX-License-Identifier: MIT */
#define _GNU_SOURCE
#include "oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <unistd.h>

static pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t wake = PTHREAD_COND_INITIALIZER;
static pthread_cond_t finished = PTHREAD_COND_INITIALIZER;
static pthread_t *workers;
static int nthreads = 1;
static int stopping;
static unsigned generation;

static void (*task_fn)(void *, int);
static void *task_ctx;
static int task_n, task_next, task_left;

static void drain(void) {
    for (;;) {
        pthread_mutex_lock(&mu);
        if (task_next >= task_n) { pthread_mutex_unlock(&mu); return; }
        const int i = task_next++;
        void (*fn)(void *, int) = task_fn;
        void *ctx = task_ctx;
        pthread_mutex_unlock(&mu);

        fn(ctx, i);

        pthread_mutex_lock(&mu);
        if (--task_left == 0) pthread_cond_broadcast(&finished);
        pthread_mutex_unlock(&mu);
    }
}

static void *worker_main(void *arg) {
    (void)arg;
    unsigned seen = 0;
    for (;;) {
        pthread_mutex_lock(&mu);
        while (!stopping && generation == seen) pthread_cond_wait(&wake, &mu);
        if (stopping) { pthread_mutex_unlock(&mu); return NULL; }
        seen = generation;
        pthread_mutex_unlock(&mu);
        drain();
    }
}

void orc_threads_shutdown(void) {
    if (nthreads > 1) {
        pthread_mutex_lock(&mu);
        stopping = 1;
        pthread_cond_broadcast(&wake);
        pthread_mutex_unlock(&mu);
        for (int i = 0; i < nthreads - 1; i++) pthread_join(workers[i], NULL);
    }
    free(workers);
    workers = NULL;
    nthreads = 1;
}

int orc_threads_init(int n) {
    if (n <= 0) {
        const long online = sysconf(_SC_NPROCESSORS_ONLN);
        n = online > 0 ? (int)online : 1;
    }
    if (n == nthreads) return nthreads;
    orc_threads_shutdown();
    if (n <= 1) return nthreads;
    workers = (pthread_t *)calloc((size_t)(n - 1), sizeof *workers);
    if (workers == NULL) return nthreads;
    stopping = 0;
    generation = 0;
    int spawned = 0;
    for (int i = 0; i < n - 1; i++)
        if (pthread_create(&workers[spawned], NULL, worker_main, NULL) == 0) spawned++;
    nthreads = spawned + 1;
    return nthreads;
}

int orc_threads_count(void) { return nthreads; }

void orc_pool_run(int n, void (*fn)(void *, int), void *ctx) {
    if (n <= 0) return;
    if (n == 1 || nthreads <= 1) {
        for (int i = 0; i < n; i++) fn(ctx, i);
        return;
    }
    pthread_mutex_lock(&mu);
    task_fn = fn;
    task_ctx = ctx;
    task_n = n;
    task_next = 0;
    task_left = n;
    generation++;
    pthread_cond_broadcast(&wake);
    pthread_mutex_unlock(&mu);

    drain();

    pthread_mutex_lock(&mu);
    while (task_left > 0) pthread_cond_wait(&finished, &mu);
    pthread_mutex_unlock(&mu);
}
