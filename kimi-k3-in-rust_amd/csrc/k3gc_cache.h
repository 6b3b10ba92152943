/* k3gc_cache.h - HBM expert cache (private declarations shared with the drop-in). */
#ifndef K3GC_CACHE_H
#define K3GC_CACHE_H

#include "../../include/k3moe.h"

/* 1 when src is an HBM expert cache, whose get() hands out device pointers. */
int k3gc_is_device_src(const K3ExpertSrc *src);

#endif
