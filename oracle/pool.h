/* pool.h — fork/join worker pool of the CPU oracle (test infrastructure only). */
#ifndef REDUKT_ORACLE_POOL_H
#define REDUKT_ORACLE_POOL_H

/* Run fn(ctx, b) for b in [0, nblocks) on the pool; returns when all are done. */
void pool_run(int nblocks, void (*fn)(void*, int), void* ctx);

#endif
