/*
 * threadpool.h -- the reference's persistent host thread pool interface
 * (reference include/threadpool.h:1-17).  The GPU path does not need host
 * threads; the pool is kept so reference callers compile and link unchanged,
 * and pool_run still runs fn on n_threads host threads for host-side work.
 */
#if !defined(QWEN_THREADPOOL_H) && !defined(THREADPOOL_H)   /* either header, whichever came first */
#define QWEN_THREADPOOL_H
/* the reference header of the same name is superseded by this one when both
   are on the include path (reference drivers compiled against this library) */
#define THREADPOOL_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pool pool_t;
typedef void (*pool_fn_t)(void *arg, int tid, int ntotal);

pool_t *pool_create(int n_threads, int pin);
void    pool_destroy(pool_t *p);
void    pool_run(pool_t *p, pool_fn_t fn, void *arg);

#ifdef __cplusplus
}
#endif
#endif
