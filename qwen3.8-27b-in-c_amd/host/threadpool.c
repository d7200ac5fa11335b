/*
 * threadpool.c -- host thread pool with the reference's interface
 * (include/threadpool.h).  Workers wait on a generation counter; pool_run
 * publishes a job, runs slice 0 on the caller and waits for the others.
 */
#define _GNU_SOURCE
#include "threadpool.h"
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>

struct pool {
    int n;
    pthread_t *th;
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    unsigned long gen;
    int pending, quit;
    pool_fn_t fn;
    void *arg;
};

typedef struct { pool_t *p; int tid; } wctx;

static void *worker(void *a)
{
    wctx *w = a;
    pool_t *p = w->p;
    const int tid = w->tid;
    free(w);
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (p->gen == seen && !p->quit) pthread_cond_wait(&p->go, &p->mu);
        if (p->quit) { pthread_mutex_unlock(&p->mu); return NULL; }
        seen = p->gen;
        pool_fn_t fn = p->fn;
        void *arg = p->arg;
        pthread_mutex_unlock(&p->mu);
        fn(arg, tid, p->n);
        pthread_mutex_lock(&p->mu);
        if (--p->pending == 0) pthread_cond_signal(&p->done);
        pthread_mutex_unlock(&p->mu);
    }
}

pool_t *pool_create(int n_threads, int pin)
{
    if (n_threads < 1) n_threads = 1;
    pool_t *p = calloc(1, sizeof *p);
    if (!p) return NULL;
    p->n = n_threads;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->go, NULL);
    pthread_cond_init(&p->done, NULL);
    p->th = calloc((size_t)n_threads, sizeof *p->th);
    for (int k = 1; k < n_threads; k++) {
        wctx *w = malloc(sizeof *w);
        w->p = p;
        w->tid = k;
        if (pthread_create(&p->th[k], NULL, worker, w)) { free(w); p->n = k; break; }
        if (pin) {
            cpu_set_t s;
            CPU_ZERO(&s);
            CPU_SET(k - 1, &s);
            pthread_setaffinity_np(p->th[k], sizeof s, &s);
        }
    }
    return p;
}

void pool_run(pool_t *p, pool_fn_t fn, void *arg)
{
    if (!p || p->n == 1) { fn(arg, 0, 1); return; }
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->arg = arg;
    p->pending = p->n - 1;
    p->gen++;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    fn(arg, 0, p->n);
    pthread_mutex_lock(&p->mu);
    while (p->pending) pthread_cond_wait(&p->done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

void pool_destroy(pool_t *p)
{
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    for (int k = 1; k < p->n; k++) pthread_join(p->th[k], NULL);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->go);
    pthread_cond_destroy(&p->done);
    free(p->th);
    free(p);
}
