/*
 * platform.c — read-only file mapping (reference src/platform.c:47-77).
 * The CPU-feature probe of the reference has no counterpart here: the
 * compute backend is the gfx950 device (cmol_hip.h).
 */
#ifndef _DEFAULT_SOURCE
#define _DEFAULT_SOURCE
#endif
#include "internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

cmol_err_t cmol_mmap_open(const char *path, cmol_mmap_t *out)
{
    if (!path || !out) return CMOL_ERR_ARGS;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return CMOL_ERR_IO;
    struct stat st;
    if (fstat(fd, &st) < 0 || st.st_size <= 0) {
        close(fd);
        return CMOL_ERR_IO;
    }
    void *p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return CMOL_ERR_IO;
#ifdef MADV_SEQUENTIAL
    madvise(p, (size_t)st.st_size, MADV_SEQUENTIAL);
#endif
    out->data = p;
    out->size = (size_t)st.st_size;
    return CMOL_OK;
}

void cmol_mmap_close(cmol_mmap_t *m)
{
    if (!m || !m->data) return;
    munmap(m->data, m->size);
    m->data = NULL;
    m->size = 0;
}
