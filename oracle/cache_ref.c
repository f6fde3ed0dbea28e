/*
 * cache_ref.c -- TEST INFRASTRUCTURE: restatement of the expert-cache
 * bookkeeping in src/engine/expert_cache.zig (Lru 39-148, ExpertCache.get
 * 230-249, Stats 18-36) and src/core/stats.zig:135-160 hottestWithinBudget.
 * Only the slot bookkeeping is restated; the byte movement is the product's.
 */
#include "loom_oracle.h"

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define NIL SIZE_MAX

struct lo_lru {
    size_t capacity, free_top;
    size_t head, tail; /* head = most recently used */
    size_t *ids, *prev, *next;
    size_t *map; /* id -> slot, NIL when absent; grown on demand */
    size_t map_len;
};

lo_lru *lo_lru_create(size_t capacity) {
    lo_lru *l = (lo_lru *)calloc(1, sizeof(lo_lru));
    l->capacity = capacity;
    l->head = l->tail = NIL;
    l->ids = (size_t *)malloc((capacity + 1) * sizeof(size_t));
    l->prev = (size_t *)malloc((capacity + 1) * sizeof(size_t));
    l->next = (size_t *)malloc((capacity + 1) * sizeof(size_t));
    return l;
}

void lo_lru_destroy(lo_lru *l) {
    if (!l)
        return;
    free(l->ids);
    free(l->prev);
    free(l->next);
    free(l->map);
    free(l);
}

static size_t map_get(const lo_lru *l, size_t id) { return id < l->map_len ? l->map[id] : NIL; }

static void map_put(lo_lru *l, size_t id, size_t slot) {
    if (id >= l->map_len) {
        size_t n = l->map_len ? l->map_len : 64;
        while (n <= id)
            n *= 2;
        l->map = (size_t *)realloc(l->map, n * sizeof(size_t));
        for (size_t i = l->map_len; i < n; i++)
            l->map[i] = NIL;
        l->map_len = n;
    }
    l->map[id] = slot;
}

static void unlink_slot(lo_lru *l, size_t s) {
    size_t p = l->prev[s], n = l->next[s];
    if (p != NIL)
        l->next[p] = n;
    else
        l->head = n;
    if (n != NIL)
        l->prev[n] = p;
    else
        l->tail = p;
}

static void push_front(lo_lru *l, size_t s) {
    l->prev[s] = NIL;
    l->next[s] = l->head;
    if (l->head != NIL)
        l->prev[l->head] = s;
    l->head = s;
    if (l->tail == NIL)
        l->tail = s;
}

/* expert_cache.zig:97-103 find: hit marks the slot most recently used. */
long lo_lru_find(lo_lru *l, size_t id) {
    size_t s = map_get(l, id);
    if (s == NIL)
        return -1;
    if (l->head != s) {
        unlink_slot(l, s);
        push_front(l, s);
    }
    return (long)s;
}

/* expert_cache.zig:107-123 reserve: fill never-used slots first, then evict
 * the least recently used tail. */
long lo_lru_reserve(lo_lru *l, size_t id, size_t *evicted) {
    if (evicted)
        *evicted = NIL;
    if (l->capacity == 0)
        return -1;
    size_t s;
    if (l->free_top < l->capacity) {
        s = l->free_top++;
    } else {
        s = l->tail;
        unlink_slot(l, s);
        if (evicted)
            *evicted = l->ids[s];
        map_put(l, l->ids[s], NIL);
    }
    l->ids[s] = id;
    map_put(l, id, s);
    push_front(l, s);
    return (long)s;
}

/* expert_cache.zig:138-147 abort: unpublish a failed fill. */
void lo_lru_abort(lo_lru *l, size_t id) {
    size_t s = map_get(l, id);
    if (s == NIL)
        return;
    map_put(l, id, NIL);
    unlink_slot(l, s);
    if (s + 1 == l->free_top)
        l->free_top--;
}

/* expert_cache.zig:128-133 clear */
void lo_lru_clear(lo_lru *l) {
    for (size_t i = 0; i < l->map_len; i++)
        l->map[i] = NIL;
    l->head = l->tail = NIL;
    l->free_top = 0;
}

/* expert_cache.zig:230-249 ExpertCache.get order over a trace. */
void lo_cache_replay(size_t capacity, const uint8_t *pinned, size_t n_ids, const uint32_t *trace,
                     size_t n_trace, uint64_t *counts, uint8_t *hit_mask) {
    lo_lru *l = lo_lru_create(capacity);
    counts[0] = counts[1] = counts[2] = 0;
    for (size_t i = 0; i < n_trace; i++) {
        uint32_t id = trace[i];
        uint8_t h;
        if (pinned && id < n_ids && pinned[id]) {
            counts[0]++;
            h = 1;
        } else if (lo_lru_find(l, id) >= 0) {
            counts[1]++;
            h = 2;
        } else {
            lo_lru_reserve(l, id, NULL);
            counts[2]++;
            h = 0;
        }
        if (hit_mask)
            hit_mask[i] = h;
    }
    lo_lru_destroy(l);
}

/* stats.zig:135-160: stable sort by count descending (ties keep ascending
 * id), take while within capacity and the count is non-zero. */
typedef struct {
    size_t id;
    uint64_t count;
} pair_t;

static int cmp_pair(const void *a, const void *b) {
    const pair_t *x = (const pair_t *)a, *y = (const pair_t *)b;
    if (x->count != y->count)
        return x->count > y->count ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

size_t lo_hottest_within_budget(const uint64_t *access_count, size_t n, size_t expert_bytes,
                                uint64_t budget, size_t *out_ids) {
    pair_t *p = (pair_t *)malloc((n ? n : 1) * sizeof(pair_t));
    for (size_t i = 0; i < n; i++) {
        p[i].id = i;
        p[i].count = access_count[i];
    }
    qsort(p, n, sizeof(pair_t), cmp_pair);
    size_t cap = expert_bytes == 0 ? 0 : (size_t)(budget / expert_bytes);
    size_t m = 0;
    for (size_t i = 0; i < n && i < cap; i++) {
        if (p[i].count == 0)
            break;
        out_ids[m++] = p[i].id;
    }
    free(p);
    return m;
}
