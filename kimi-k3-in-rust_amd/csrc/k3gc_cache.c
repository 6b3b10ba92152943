/* k3gc_cache.c - HBM-resident expert cache. */
#include "k3gc_cache.h"

int k3gc_is_device_src(const K3ExpertSrc *src)
{
    (void)src;
    return 0;
}
