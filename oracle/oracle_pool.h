/*
 * oracle_pool.h — the oracle's worker pool, shared by its source files
 * (internal; not part of the oracle's API). parallel_for of the reference's
 * ThreadPool (src/backends/cpu_backend.cpp:62-95): indices [0, n) handed out
 * one per atomic fetch to the workers and the calling thread.
 */
#ifndef IKV_ORACLE_POOL_H
#define IKV_ORACLE_POOL_H

#include <stdint.h>

void oracle_pool_for(int64_t n, void (*fn)(int64_t i, void *ctx), void *ctx);

#endif
