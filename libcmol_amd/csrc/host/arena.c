/*
 * arena.c — bump allocator over the single host allocation made by
 * cmol_load; zero-fills on allocation (reference src/arena.c:9-29).
 */
#include "internal.h"

#include <string.h>

void cmol_arena_init(cmol_arena_t *a, void *buf, size_t size)
{
    a->base = (uint8_t *)buf;
    a->size = size;
    a->used = 0;
}

void *cmol_arena_alloc(cmol_arena_t *a, size_t size, size_t align)
{
    size_t start = (a->used + align - 1u) & ~(align - 1u);
    if (start > a->size || size > a->size - start) return NULL;
    void *p = a->base + start;
    a->used = start + size;
    memset(p, 0, size);
    return p;
}

void *cmol_arena_alloc_n(cmol_arena_t *a, size_t count, size_t elem_size)
{
    if (count && elem_size > (size_t)-1 / count) return NULL;
    return cmol_arena_alloc(a, count * elem_size, elem_size < 8 ? (elem_size ? elem_size : 1) : 8);
}
