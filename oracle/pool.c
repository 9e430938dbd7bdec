/*
 * pool.c -- pthread restatement of native-engine pool.rs's split_by
 * (pool.rs:127-168).  TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Pin: every task runs once (tests/test_oracle_gemm.py compares threaded and
 * single-threaded products bit for bit).
 */
#include "pool.h"

#include <pthread.h>
#include <stdatomic.h>

typedef struct {
  atomic_size_t next;
  size_t items, chunk;
  or_task task;
  void *ctx;
} pool_state;

static void *worker(void *arg) {
  pool_state *s = (pool_state *)arg;
  for (;;) {
    size_t start = atomic_fetch_add(&s->next, s->chunk);
    if (start >= s->items) break;
    size_t end = start + s->chunk < s->items ? start + s->chunk : s->items;
    s->task(s->ctx, start, end);
  }
  return 0;
}

void or_parallel(int threads, size_t items, size_t grain, size_t max,
                 or_task task, void *ctx) {
  if (items == 0) return;
  if (grain == 0) grain = 1;
  size_t chunk = (max / grain) * grain;
  if (chunk == 0) chunk = grain;
  size_t tasks = (items + chunk - 1) / chunk;
  if (threads < 1) threads = 1;
  /* Share what is left: smaller ranges when there are more threads than
   * ranges of `max` (pool.rs sizes each range to the work left). */
  if ((size_t)threads > tasks && chunk > grain) {
    size_t per = (items + (size_t)threads - 1) / (size_t)threads;
    per = (per + grain - 1) / grain * grain;
    if (per < chunk) chunk = per;
    tasks = (items + chunk - 1) / chunk;
  }
  pool_state s;
  atomic_init(&s.next, 0);
  s.items = items;
  s.chunk = chunk;
  s.task = task;
  s.ctx = ctx;
  int n = threads < (int)tasks ? threads : (int)tasks;
  if (n <= 1) {
    worker(&s);
    return;
  }
  pthread_t tid[256];
  if (n > 256) n = 256;
  for (int i = 1; i < n; i++) pthread_create(&tid[i], 0, worker, &s);
  worker(&s);
  for (int i = 1; i < n; i++) pthread_join(tid[i], 0);
}
