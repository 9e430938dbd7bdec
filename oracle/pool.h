/*
 * pool.h -- the oracle's worker split (restates native-engine pool.rs:118-168:
 * ranges in multiples of `grain`, at most `max` long, taken by threads as
 * they finish; a range never splits one output's reduction).
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#ifndef IEN_ORACLE_POOL_H
#define IEN_ORACLE_POOL_H
#include <stddef.h>
typedef void (*or_task)(void *ctx, size_t start, size_t end);
void or_parallel(int threads, size_t items, size_t grain, size_t max,
                 or_task task, void *ctx);
#endif
