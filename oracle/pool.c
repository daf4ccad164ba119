/* pool.c — persistent fork/join worker pool for the CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle and timed CPU baseline).
 *
 * Plays the role of redukt's par_pool (src/domain/par_pool.rs:50-83): it decides
 * which thread runs a block, never how the block computes, so every output is
 * bit-identical for any thread count.  Blocks are claimed with an atomic counter.
 */
#include <pthread.h>
#include <stdlib.h>
#include <unistd.h>

#include "pool.h"

#define MAX_THREADS 256

static struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    int threads;          /* total threads including the caller */
    int started;          /* worker threads running */
    unsigned long gen;    /* job generation */
    int active;           /* workers still inside the current job */
    int nblocks;
    int next;             /* next block to claim (atomic) */
    void (*fn)(void*, int);
    void* ctx;
    pthread_t tid[MAX_THREADS];
} P = { PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER,
        0, 0, 0, 0, 0, 0, NULL, NULL, {0} };

static void run_blocks(void) {
    for (;;) {
        int b = __atomic_fetch_add(&P.next, 1, __ATOMIC_RELAXED);
        if (b >= P.nblocks) break;
        P.fn(P.ctx, b);
    }
}

static void* worker(void* arg) {
    int idx = (int)(long)arg;
    unsigned long seen = 0;
    pthread_mutex_lock(&P.mu);
    for (;;) {
        while (P.gen == seen) pthread_cond_wait(&P.go, &P.mu);
        seen = P.gen;
        int participate = idx < P.threads - 1;  /* a shrunk pool idles the extra workers */
        pthread_mutex_unlock(&P.mu);
        if (participate) run_blocks();
        pthread_mutex_lock(&P.mu);
        if (--P.active == 0) pthread_cond_signal(&P.done);
    }
    return NULL;
}

static void ensure_started(void) {
    if (P.threads == 0) {
        long n = sysconf(_SC_NPROCESSORS_ONLN);
        const char* env = getenv("ORACLE_THREADS");
        if (env && atoi(env) > 0) n = atoi(env);
        if (n < 1) n = 1;
        if (n > MAX_THREADS) n = MAX_THREADS;
        P.threads = (int)n;
    }
    while (P.started < P.threads - 1) {
        if (pthread_create(&P.tid[P.started], NULL, worker, (void*)(long)P.started) != 0) {
            P.threads = P.started + 1;
            break;
        }
        pthread_detach(P.tid[P.started]);
        P.started++;
    }
}

void orc_set_threads(int n) {
    pthread_mutex_lock(&P.mu);
    if (n < 1) n = 1;
    if (n > MAX_THREADS) n = MAX_THREADS;
    P.threads = n;
    pthread_mutex_unlock(&P.mu);
}

int orc_get_threads(void) {
    pthread_mutex_lock(&P.mu);
    ensure_started();
    int t = P.threads;
    pthread_mutex_unlock(&P.mu);
    return t;
}

void pool_run(int nblocks, void (*fn)(void*, int), void* ctx) {
    if (nblocks <= 0) return;
    pthread_mutex_lock(&P.mu);
    ensure_started();
    int workers = P.threads - 1;
    if (workers > P.started) workers = P.started;
    if (workers <= 0 || nblocks == 1) {
        pthread_mutex_unlock(&P.mu);
        for (int b = 0; b < nblocks; b++) fn(ctx, b);
        return;
    }
    /* Every started worker wakes and acknowledges; only the first P.threads-1 claim blocks. */
    P.fn = fn;
    P.ctx = ctx;
    P.nblocks = nblocks;
    __atomic_store_n(&P.next, 0, __ATOMIC_RELAXED);
    P.active = P.started;
    P.gen++;
    pthread_cond_broadcast(&P.go);
    pthread_mutex_unlock(&P.mu);
    run_blocks();
    pthread_mutex_lock(&P.mu);
    while (P.active > 0) pthread_cond_wait(&P.done, &P.mu);
    pthread_mutex_unlock(&P.mu);
}
